"""Gradient nodes of the matmul path on the HIP kernels.

Mirrors the reference's autograd nodes ("cs/" = csharp/cstorchcl/cstorchcl/):
  BmmOp.Backward    cs/core/BmmOp.cs:27-68     dA = dC @ B^T (NT), dB = A^T @ dC (TN)
  LinearOp.Backward cs/core/LinearOp.cs:16-49  dX = dY @ W^T (NT), dW = sum_b X_b^T dY_b,
                                               db = column sum of dY
and exposes the same mathematics as torch.autograd.Function objects (bmm, linear) so a
PyTorch caller gets the NT/TN gradient kernels from loss.backward().

Where the reference forms a gradient by materialising a transpose (Permute + Bmm,
BmmOp.cs:44-60) or a [B,K,N] per-batch product followed by Sum (LinearOp.cs:37-38), these
nodes run the NT / TN kernels directly; a broadcast operand (batch 1) receives the batch
sum of its gradient, which the reference's BmmOp leaves unsummed.
"""
import torch

from .nncl_glob import NnClGlob

_glob = None


def _g():
    global _glob
    if _glob is None:
        _glob = NnClGlob()
    return _glob


class BmmOp:
    """Graph node of C = Bmm(A, B) (cs/core/BmmOp.cs:10-69)."""

    def __init__(self, a, b, output, nnclglob=None):
        self.Inputs = [a, b]
        self.Output = output
        self._nncl = nnclglob or _g()

    def Backward(self, gradOutput, a_requires_grad=True, b_requires_grad=True):
        a, b = self.Inputs
        grad_a = grad_b = None
        if a_requires_grad:
            grad_a = self._nncl.BmmPermute(gradOutput, b, transA=False, transB=True)
        if b_requires_grad:
            if b.shape[0] == 1 and a.shape[0] > 1:
                grad_b = self._nncl.linear_weight_grad(a.contiguous(), gradOutput.contiguous())
            else:
                grad_b = self._nncl.BmmPermute(a, gradOutput, transA=True, transB=False)
        return [grad_a, grad_b]


class LinearOp:
    """Graph node of Y = LinearForward(X, W, bias) (cs/core/LinearOp.cs:4-50)."""

    def __init__(self, x, w, bias, output, nnclglob=None):
        self.Inputs = [x, w, bias]
        self.Output = output
        self._nncl = nnclglob or _g()

    def Backward(self, gradOutput, x_requires_grad=True, w_requires_grad=True,
                 bias_requires_grad=True):
        x, w, bias = self.Inputs
        k, n = w.shape[-2], w.shape[-1]
        grad_x = grad_w = grad_b = None
        if x_requires_grad:
            grad_x = self._nncl.BmmPermute(gradOutput, w.reshape(1, k, n), transA=False,
                                           transB=True)
        if w_requires_grad:
            grad_w = self._nncl.linear_weight_grad(x, gradOutput).reshape(w.shape)
        if bias_requires_grad:
            grad_b = self._nncl.LinearBiasBackward(gradOutput, list(bias.shape))
        return [grad_x, grad_w, grad_b]


class _BmmFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, a, b):
        a = a.contiguous()
        b = b.contiguous()
        ctx.save_for_backward(a, b)
        return _g().BmmPermute(a, b)

    @staticmethod
    def backward(ctx, grad):
        a, b = ctx.saved_tensors
        node = BmmOp(a, b, None)
        ga, gb = node.Backward(grad.contiguous(), ctx.needs_input_grad[0],
                               ctx.needs_input_grad[1])
        return ga, gb


class _LinearFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, w, bias):
        x = x.contiguous()
        w = w.contiguous()
        bias = bias.contiguous()
        ctx.save_for_backward(x, w, bias)
        return _g().LinearForward(x, w, bias)

    @staticmethod
    def backward(ctx, grad):
        x, w, bias = ctx.saved_tensors
        node = LinearOp(x, w, bias, None)
        return tuple(node.Backward(grad.contiguous(), *ctx.needs_input_grad))


def bmm(a, b):
    """Differentiable a[B,M,K] @ b[B|1,K,N] on the HIP kernels."""
    return _BmmFunction.apply(a, b)


def linear(x, w, bias):
    """Differentiable x[B,M,K] @ w[1,K,N] + bias[N] on the HIP kernels."""
    return _LinearFunction.apply(x, w, bias)
