"""Host-side operator API of the matmul path, mirroring the reference's NnClGlob.

Reference interfaces mirrored (paths relative to the reference repository;
"cs/" = csharp/cstorchcl/cstorchcl/):
  C# NnClGlob (cs/compiler/NnClGlob.cs)        this module
  ------------------------------------------   ---------------------------------------
  Tensor Bmm(Tensor a, Tensor b)      :441     NnClGlob.Bmm(a, b)
  Tensor BmmPermute(a, b, transA, transB):1702 NnClGlob.BmmPermute(a, b, transA, transB)
  Tensor Permute(Tensor x, int[] axes) :382    NnClGlob.Permute(x, axes)
  Tensor LinearForward(x, w, bias)    :1493    NnClGlob.LinearForward(x, w, bias)
  Tensor LinearBiasBackward(g, shape) :1557    NnClGlob.LinearBiasBackward(g, shape)
  Tensor Sum(x, axis, keepDims)       :1595    NnClGlob.Sum(x, axis, keepDims)
  LstmWithWithState gate loop        :1067    NnClGlob.LstmHidGates(x, w, u, bias, hPrev,
                                                                   hOut, workspace, t)
  Python NnClGlob (compiler/nncl_glob.py)
  bmm(A, B)                           :110     NnClGlob.bmm(A, B)
  permute(x, axes)                    :148     NnClGlob.permute(x, axes)
  bmm_backward(grad_output, A, B)     :283     NnClGlob.bmm_backward(grad_output, A, B)

Tensors are torch float32 tensors resident on the GPU (torch is only the device-memory and
stream plumbing); every operator enqueues a HIP kernel of libmigemm.so on the current torch
stream through the C ABI. There is no CPU fallback: a CPU tensor or a missing library raises.

Deliberate differences from the reference, each an aliasing or safety fix:
  * every call returns a fresh output tensor; the reference's name-keyed buffer pool makes
    every Bmm output the same "bmm_c" buffer (NnClGlob.cs:460, OpenCLBufferManager.cs:29-40);
  * bmm_backward / BmmOp.Backward use the NT / TN kernels directly instead of
    Permute + Bmm (BmmOp.cs:44-60, nncl_glob.py:300-310) -- same mathematics, no transposed
    copies, and grad_A is no longer overwritten by grad_B;
  * BmmPermute and LinearForward also validate batch / inner sizes, which the reference
    leaves unchecked (an out-of-bounds read there).
"""
import ctypes

import torch

from . import _native


class ShapeError(ValueError, AssertionError):
    """Shape / rank / broadcast error raised before any launch. It is an AssertionError for
    callers of the Python reference (which asserts, nncl_glob.py:116-118) and a ValueError
    (the ArgumentException of NnClGlob.cs:443-452) for everyone else."""


def _require(cond, msg):
    if not cond:
        raise ShapeError(msg)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


_INT_RANGES = {ctypes.c_int: (-2 ** 31, 2 ** 31 - 1), ctypes.c_int64: (-2 ** 63, 2 ** 63 - 1)}


def _launch(name, tensors, *args):
    """Calls C-ABI entry `name` on the current stream of the tensors' device, with that
    device current (the library launches on the current HIP device). All tensors of one
    call must live on one device. Integer arguments are range-checked against the C types
    first: ctypes would silently wrap a size or stride of 2^31 or more into a valid-looking
    int32 (the reference's kernels take int sizes and strides, matmul.cl:8-14, 78-87)."""
    argtypes = _native.SIGNATURES[name][0][1:]
    for i, (t, v) in enumerate(zip(argtypes, args)):
        if t in _INT_RANGES and isinstance(v, int):
            lo, hi = _INT_RANGES[t]
            _require(lo <= v <= hi, f"{name}: argument {i + 1} = {v} does not fit the C "
                                    f"ABI's {'int32' if t is ctypes.c_int else 'int64'}")
    devices = {t.device for t in tensors}
    _require(len(devices) == 1,
             f"all operands must be on one device (got {sorted(map(str, devices))})")
    dev = tensors[0].device
    with torch.cuda.device(dev):
        _native.call(name, _stream(tensors[0]), *args)


def _check_tensor(name, t):
    _require(isinstance(t, torch.Tensor), f"{name} must be a torch.Tensor")
    _require(t.dtype == torch.float32, f"{name} must be float32 (got {t.dtype})")
    _require(t.is_cuda, f"{name} must live on the GPU: the matmul path has no CPU fallback")
    _require(t.is_contiguous(), f"{name} must be contiguous (row-major, as Tensor.cs:283-295)")


class NnClGlob:
    """Operator dispatcher of the matmul path (the drop-in for NnClGlob's GEMM ops)."""

    def __init__(self, device=None):
        _native.load()
        self.device = torch.device(device) if device is not None else torch.device("cuda", 0)

    # ------------------------------------------------------------------ C# names
    def Bmm(self, a, b):
        """C[B,M,N] = a[B,M,K] @ b[B|1,K,N]; b with batch 1 is broadcast (stride 0).
        Synchronous, like the reference's Finish() (NnClGlob.cs:498)."""
        _check_tensor("a", a)
        _check_tensor("b", b)
        _require(a.dim() == 3 and b.dim() == 3, "Bmm expects 3-D tensors [Batch, M, K]")
        _require(a.shape[0] == b.shape[0] or b.shape[0] == 1,
                 f"batch mismatch: {a.shape[0]} and {b.shape[0]}")
        _require(a.shape[2] == b.shape[1],
                 f"inner dimensions differ: K={a.shape[2]} != {b.shape[1]}")
        batch, m, k = a.shape
        n = b.shape[2]
        c = torch.empty((batch, m, n), dtype=torch.float32, device=a.device)
        sB = 0 if b.shape[0] == 1 else k * n
        _launch("migemm_bmm_tiled", (a, b, c), _ptr(a), _ptr(b), _ptr(c), m, k, n, m * k, sB,
                m * n, batch)
        torch.cuda.current_stream(a.device).synchronize()
        return c

    def BmmPermute(self, a, b, transA=False, transB=False):
        """C = op(a) @ op(b) with op = transpose of the last two axes when requested
        (NnClGlob.cs:1702-1751). Batch = a.shape[0]; an operand with batch 1 is broadcast.
        Asynchronous on the current stream, like the reference."""
        _check_tensor("a", a)
        _check_tensor("b", b)
        _require(a.dim() == 3 and b.dim() == 3, "BmmPermute expects 3-D tensors")
        batch = a.shape[0]
        m = a.shape[2] if transA else a.shape[1]
        kA = a.shape[1] if transA else a.shape[2]
        kB = b.shape[2] if transB else b.shape[1]
        n = b.shape[1] if transB else b.shape[2]
        _require(kA == kB, f"inner dimensions differ: {kA} != {kB}")
        _require(b.shape[0] in (batch, 1), f"batch mismatch: {batch} and {b.shape[0]}")
        c = torch.empty((batch, m, n), dtype=torch.float32, device=a.device)
        sA = 0 if a.shape[0] == 1 else a.shape[1] * a.shape[2]
        sB = 0 if b.shape[0] == 1 else b.shape[1] * b.shape[2]
        _launch("migemm_bmm_permute_tiled", (a, b, c), _ptr(a), _ptr(b), _ptr(c), m, kA, n, sA,
                sB, m * n, int(bool(transA)), int(bool(transB)), batch)
        return c

    def Permute(self, x, axes):
        """y = x.permute(axes) materialised (NnClGlob.cs:382-424), up to 10-D."""
        _check_tensor("x", x)
        axes = [int(v) for v in axes]
        _require(len(axes) == x.dim(), "the number of axes must equal the tensor rank")
        _require(sorted(axes) == list(range(x.dim())), f"axes {axes} is not a permutation")
        y = torch.empty([x.shape[i] for i in axes], dtype=torch.float32, device=x.device)
        dims = (ctypes.c_int * x.dim())(*x.shape)
        ax = (ctypes.c_int * x.dim())(*axes)
        _launch("migemm_tensor_permute", (x, y), _ptr(x), _ptr(y), dims, ax, x.dim())
        return y

    def LinearForward(self, x, w, bias):
        """Y[B,M,N] = x[B,M,K] @ w[1,K,N] + bias[N], bias added after the k loop
        (NnClGlob.cs:1493-1551, linear.cl:107-143)."""
        _check_tensor("x", x)
        _check_tensor("w", w)
        _check_tensor("bias", bias)
        _require(x.dim() == 3, "LinearForward expects x [Batch, M, K]")
        batch, m, k = x.shape
        n = w.shape[-1]
        _require(w.numel() == k * n and w.shape[-2] == k,
                 f"w must be [1, {k}, N] (got {list(w.shape)})")
        _require(bias.numel() == n, f"bias must have {n} elements (got {bias.numel()})")
        y = torch.empty((batch, m, n), dtype=torch.float32, device=x.device)
        _launch("migemm_linear_forward", (x, w, bias, y), _ptr(x), _ptr(w), _ptr(bias), _ptr(y),
                m, k, n, m * k, m * n, batch)
        return y

    def LinearBiasBackward(self, gradOutput, biasShape):
        """grad_bias[n] = sum over batch and rows of gradOutput (NnClGlob.cs:1557-1584)."""
        _check_tensor("gradOutput", gradOutput)
        n = gradOutput.shape[-1]
        rows = gradOutput.numel() // n
        gb = torch.empty(list(biasShape), dtype=torch.float32, device=gradOutput.device)
        _require(gb.numel() == n, f"bias shape {list(biasShape)} does not hold {n} values")
        _launch("migemm_linear_bias_backward", (gradOutput, gb), _ptr(gradOutput), _ptr(gb),
                rows, n)
        return gb

    # ---- LSTM GEMM stages (NnClGlob.Lstm / LstmBackward, cs/compiler/NnClGlob.cs:850-1061).
    # The recurrent kernels between them (lstm_recurrent_forward / _backward) are not part
    # of the matmul path; these are the three GEMM launches of those two methods.
    def LstmGemmXW(self, x, w, bias):
        """XW[T, 4H] = x[B, S, F] (as [T, F]) @ w[F, 4H] + bias[4H]: stage 1 of NnClGlob.Lstm
        (NnClGlob.cs:877-899, lstm_gemm_xw lstm.cl:273-367)."""
        _check_tensor("x", x)
        _check_tensor("w", w)
        _check_tensor("bias", bias)
        f = x.shape[-1]
        t = x.numel() // f
        _require(w.dim() == 2 and w.shape[0] == f,
                 f"w must be [{f}, 4*hidden] (got {list(w.shape)})")
        g = w.shape[1]
        _require(bias.numel() == g, f"bias must have {g} elements (got {bias.numel()})")
        xw = torch.empty((t, g), dtype=torch.float32, device=x.device)
        _launch("migemm_lstm_gemm_xw", (x, w, bias, xw), _ptr(x), _ptr(w), _ptr(bias), _ptr(xw),
                t, f, g)
        return xw

    def LstmRecurrentGates(self, xw, hOut, u, t):
        """The recurrent product of step t inside lstm_recurrent_forward (lstm.cl:80-101,
        enqueued by NnClGlob.Lstm, NnClGlob.cs:912-928), in place on xw [B, S, 4H]:
        xw[:, t] += hOut[:, t-1] @ u (u [H, 4H]); xw[:, t] then holds the step's raw gates
        (the reference's workspace[t, b, :4H], lstm.cl:103-106). A no-op at t = 0."""
        _check_tensor("xw", xw)
        _check_tensor("hOut", hOut)
        _check_tensor("u", u)
        _require(xw.dim() == 3 and hOut.dim() == 3, "xw and hOut must be [Batch, Seq, *]")
        b, s_, g = xw.shape
        h = hOut.shape[2]
        _require(g == 4 * h, f"xw must end in 4*hidden = {4 * h} gates (got {g})")
        _require(hOut.shape[0] == b and hOut.shape[1] == s_, "xw and hOut batch/seq differ")
        _require(list(u.shape) == [h, g], f"u must be [{h}, {g}] (got {list(u.shape)})")
        _require(0 <= t < s_, f"step {t} is outside [0, {s_})")
        _launch("migemm_lstm_recurrent_gates", (xw, hOut, u), _ptr(xw), _ptr(hOut), _ptr(u), b,
                s_, h, int(t))
        return xw

    def LstmHidGates(self, x, w, u, bias, hPrev, hOut, workspace, t):
        """The gate product of step t of lstm_hid_forward (lstm.cl:788-870, gate loop
        :832-844), enqueued by NnClGlob.LstmWithWithState (NnClGlob.cs:1067-1100), in place
        on workspace [S, B, 4H]: workspace[t] = bias + x[:, t] @ w + h_{t-1} @ u, with
        h_{t-1} = hPrev [B, H] at t = 0 and hOut[:, t-1] ([B, S, H]) after. x is [B, S, F],
        w [F, 4H], u [H, 4H], bias [4H]. One launch over the four separate buffers; the
        activations and cell update that follow in the reference kernel are the caller's."""
        for name, v in (("x", x), ("w", w), ("u", u), ("bias", bias), ("hPrev", hPrev),
                        ("hOut", hOut), ("workspace", workspace)):
            _check_tensor(name, v)
        _require(x.dim() == 3, f"x must be [Batch, Seq, In] (got {list(x.shape)})")
        b, s_, f = x.shape
        _require(u.dim() == 2 and u.shape[1] == 4 * u.shape[0],
                 f"u must be [hidden, 4*hidden] (got {list(u.shape)})")
        h = u.shape[0]
        g = 4 * h
        _require(list(w.shape) == [f, g], f"w must be [{f}, {g}] (got {list(w.shape)})")
        _require(bias.numel() == g, f"bias must have {g} elements (got {bias.numel()})")
        _require(list(hPrev.shape) == [b, h], f"hPrev must be [{b}, {h}] (got {list(hPrev.shape)})")
        _require(list(hOut.shape) == [b, s_, h],
                 f"hOut must be [{b}, {s_}, {h}] (got {list(hOut.shape)})")
        _require(list(workspace.shape) == [s_, b, g],
                 f"workspace must be [{s_}, {b}, {g}] (got {list(workspace.shape)})")
        _require(0 <= t < s_, f"step {t} is outside [0, {s_})")
        _launch("migemm_lstm_hid_gates", (x, w, u, bias, hPrev, hOut, workspace), _ptr(x),
                _ptr(w), _ptr(u), _ptr(bias), _ptr(hPrev), _ptr(hOut), _ptr(workspace), b, s_,
                f, h, int(t))
        return workspace

    def LstmGemmGradX(self, allGradGates, w, xShape):
        """grad_X (shape xShape) = allGradGates[T, 4H] @ w[F, 4H]^T: stage 2 of
        NnClGlob.LstmBackward (NnClGlob.cs:967-994, lstm_gemm_grad_x lstm.cl:372-457)."""
        _check_tensor("allGradGates", allGradGates)
        _check_tensor("w", w)
        _require(w.dim() == 2, f"w must be [in_features, 4*hidden] (got {list(w.shape)})")
        f, g = w.shape
        _require(allGradGates.shape[-1] == g,
                 f"allGradGates must end in {g} gates (got {list(allGradGates.shape)})")
        t = allGradGates.numel() // g
        gx = torch.empty(list(xShape), dtype=torch.float32, device=w.device)
        _require(gx.numel() == t * f, f"xShape {list(xShape)} does not hold [{t}, {f}]")
        _launch("migemm_lstm_gemm_grad_x", (w, allGradGates, gx), _ptr(allGradGates), _ptr(w),
                _ptr(gx), t, f, g)
        return gx

    def LstmGemmGradWeights(self, x, hOut, allGradGates, gradW, gradU, gradBias):
        """Stage 3 of NnClGlob.LstmBackward (NnClGlob.cs:996-1024, lstm_gemm_grad_weights
        lstm.cl:459-636), accumulating in place like w.Grad / u.Grad / bias.Grad there:
        gradW += X^T G, gradU += H_prev^T G (h_{t-1} of the same sequence, 0 at its first
        step), gradBias += sum over tokens of G. x is [B, S, F], hOut [B, S, H]."""
        for name, t in (("x", x), ("hOut", hOut), ("allGradGates", allGradGates),
                        ("gradW", gradW), ("gradU", gradU), ("gradBias", gradBias)):
            _check_tensor(name, t)
        _require(x.dim() == 3 and hOut.dim() == 3, "x and hOut must be [Batch, Seq, *]")
        b, s_, f = x.shape
        h = hOut.shape[2]
        _require(hOut.shape[0] == b and hOut.shape[1] == s_, "x and hOut batch/seq differ")
        _require(allGradGates.numel() == b * s_ * 4 * h, "allGradGates must be [B*S, 4*hidden]")
        _require(gradW.numel() == f * 4 * h, f"gradW must hold [{f}, {4 * h}]")
        _require(gradU.numel() == h * 4 * h, f"gradU must hold [{h}, {4 * h}]")
        _require(gradBias.numel() == 4 * h, f"gradBias must hold {4 * h} values")
        _launch("migemm_lstm_gemm_grad_weights", (x, hOut, allGradGates, gradW, gradU, gradBias),
                _ptr(x), _ptr(hOut), _ptr(allGradGates), _ptr(gradW), _ptr(gradU),
                _ptr(gradBias), b, s_, f, h)
        return gradW, gradU, gradBias

    def Sum(self, x, axis, keepDims=False):
        """Sum over one axis, ascending order (NnClGlob.cs:1595-1664)."""
        _check_tensor("x", x)
        ax = axis + x.dim() if axis < 0 else axis
        if ax < 0 or ax >= x.dim():
            raise IndexError(f"axis {axis} is out of range for a {x.dim()}-D tensor")
        outer = 1
        for s in x.shape[:ax]:
            outer *= s
        inner = 1
        for s in x.shape[ax + 1:]:
            inner *= s
        if keepDims:
            shape = list(x.shape)
            shape[ax] = 1
        elif x.dim() == 1:
            shape = [1]
        else:
            shape = [s for i, s in enumerate(x.shape) if i != ax]
        y = torch.empty(shape, dtype=torch.float32, device=x.device)
        _launch("migemm_reduce_sum_axis", (x, y), _ptr(x), _ptr(y), outer, x.shape[ax], inner)
        return y

    # -------------------------------------------------------------- Python names
    def bmm(self, A, B):
        """Python reference bmm (nncl_glob.py:110-147): equal batches required."""
        _check_tensor("A", A)
        _check_tensor("B", B)
        _require(A.dim() == 3 and B.dim() == 3,
                 "BMM expects 3-D tensors [Batch, M/K, K/N]")
        _require(A.shape[0] == B.shape[0], "the Batch dimension of A and B must match")
        return self.Bmm(A, B)

    def permute(self, x, axes):
        """Python reference permute (nncl_glob.py:148-174); synchronous like it."""
        y = self.Permute(x, axes)
        torch.cuda.current_stream(x.device).synchronize()
        return y

    def bmm_backward(self, grad_output, A, B):
        """(grad_A, grad_B) = (dC @ B^T, A^T @ dC) (nncl_glob.py:283-312), computed with
        the NT and TN kernels instead of permute + bmm."""
        grad_A = self.BmmPermute(grad_output, B, transA=False, transB=True)
        grad_B = self.BmmPermute(A, grad_output, transA=True, transB=False)
        torch.cuda.current_stream(A.device).synchronize()
        return grad_A, grad_B

    # ------------------------------------------------------------- extra forms
    def linear_weight_grad(self, x, grad_output):
        """dW[1,K,N] = sum_b x_b^T @ dY_b in one TN GEMM over batch*M rows (the
        BmmPermute(transA) + Sum(axis 0) pair of LinearOp.cs:37-38)."""
        _check_tensor("x", x)
        _check_tensor("grad_output", grad_output)
        _require(x.dim() == 3 and grad_output.dim() == 3, "expects 3-D tensors")
        batch, m, k = x.shape
        _require(grad_output.shape[0] == batch and grad_output.shape[1] == m,
                 "x and grad_output must share [Batch, M]")
        n = grad_output.shape[2]
        dw = torch.empty((1, k, n), dtype=torch.float32, device=x.device)
        _launch("migemm_linear_weight_grad", (x, grad_output, dw), _ptr(x), _ptr(grad_output),
                _ptr(dw), m, k, n, batch)
        return dw

    @staticmethod
    def reserve_workspace(stream, nbytes):
        """Sizes the library workspace of `stream` (a torch.cuda.Stream) to at least nbytes
        per buffer before it is captured into a HIP graph: a capture allocates nothing, and a
        split GEMM captured on a stream whose workspace is too small fails with
        MIGEMM_ERR_WORKSPACE (migemm_workspace_reserve)."""
        _native.call("migemm_workspace_reserve", ctypes.c_void_p(stream.cuda_stream),
                     int(nbytes))

    def gemm(self, a, b, transA=False, transB=False, bias=None, out=None):
        """General 2-D / batched entry point: out = op(a) @ op(b) (+ bias)."""
        _check_tensor("a", a)
        _check_tensor("b", b)
        squeeze = a.dim() == 2 and b.dim() == 2
        a3 = a.unsqueeze(0) if a.dim() == 2 else a
        b3 = b.unsqueeze(0) if b.dim() == 2 else b
        _require(a3.dim() == 3 and b3.dim() == 3, "gemm expects 2-D or 3-D tensors")
        batch = max(a3.shape[0], b3.shape[0])
        _require(a3.shape[0] in (batch, 1) and b3.shape[0] in (batch, 1), "batch mismatch")
        m, k = (a3.shape[2], a3.shape[1]) if transA else (a3.shape[1], a3.shape[2])
        kb, n = (b3.shape[2], b3.shape[1]) if transB else (b3.shape[1], b3.shape[2])
        _require(k == kb, f"inner dimensions differ: {k} != {kb}")
        if bias is not None:
            _check_tensor("bias", bias)
            _require(bias.numel() == n, f"bias must have {n} elements")
        if out is None:
            out = torch.empty((batch, m, n), dtype=torch.float32, device=a.device)
        else:
            _check_tensor("out", out)
            _require(out.numel() == batch * m * n, "out has the wrong size")
        sA = 0 if a3.shape[0] == 1 else a3.shape[1] * a3.shape[2]
        sB = 0 if b3.shape[0] == 1 else b3.shape[1] * b3.shape[2]
        _launch("migemm_gemm_strided_batched", (a, b, out) + ((bias,) if bias is not None else ()),
                int(transA), int(transB), m, n, k, _ptr(a3), a3.shape[2], sA, _ptr(b3),
                b3.shape[2], sB, _ptr(bias) if bias is not None else None, _ptr(out), n, m * n,
                batch)
        return out.view(m, n) if squeeze else out
