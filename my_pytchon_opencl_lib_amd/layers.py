"""The Python reference's Linear layer on the HIP kernels.

core/layers.py:7-33 keeps the weight as [out_channels, in_features] and, in forward, first
materialises its transpose with permute([1, 0]) (a tensor_permute launch and a copy of the
weight) and then runs bmm(x, W^T) (:27-29). Here forward runs the same product as ONE NT GEMM
(B stored [N, K]: migemm_bmm_permute_tiled with transB and a broadcast weight), so no
transposed copy of the weight is ever made.

Like the reference's forward, this one returns x @ W^T and does not add the bias (layers.py:
21-33 never reads self.bias, which starts at zero, :16); LinearForward (the C# host's
NnClGlob.LinearForward) is the bias-epilogue form.
"""
import numpy as np
import torch

from .nncl_glob import NnClGlob, _require


class Linear:
    """Linear(in_features, out_channels, nnclglob) as core/layers.py:7-33."""

    def __init__(self, in_features, out_channels, nnclglob=None, weight=None, seed=None):
        self.nnclglob = nnclglob if nnclglob is not None else NnClGlob()
        self.in_features = int(in_features)
        self.out_channels = int(out_channels)
        dev = self.nnclglob.device
        if weight is None:
            # U(-1/sqrt(in), 1/sqrt(in)) of shape [out, in] (layers.py:14-15)
            bound = 1.0 / np.sqrt(self.in_features)
            rng = np.random.default_rng(seed)
            weight = rng.uniform(-bound, bound, size=(self.out_channels, self.in_features))
        w = torch.as_tensor(np.asarray(weight, dtype=np.float32)) if not isinstance(
            weight, torch.Tensor) else weight.to(torch.float32)
        _require(list(w.shape) == [self.out_channels, self.in_features],
                 f"weight must be [{self.out_channels}, {self.in_features}]")
        self.weight = w.to(dev).contiguous()
        self.bias = torch.zeros(self.out_channels, dtype=torch.float32, device=dev)  # :16

    def forward(self, x):
        """y[..., out] = x[..., in] @ weight^T, as one NT GEMM over all rows of x."""
        _require(x.shape[-1] == self.in_features,
                 f"x must end in {self.in_features} features (got {list(x.shape)})")
        x3 = x.reshape(1, -1, self.in_features).contiguous()  # layers.py:23-24
        y = self.nnclglob.BmmPermute(x3, self.weight.unsqueeze(0), transA=False, transB=True)
        return y.reshape(list(x.shape[:-1]) + [self.out_channels])  # :31-33

    __call__ = forward

    def parameters(self):
        return [self.weight, self.bias]
