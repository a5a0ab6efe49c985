"""Parity helpers shared by the GPU tests: run a GEMM form through the C ABI on the GPU and
check it against the oracle (fp64 evaluation + the restated reference arithmetic).

Bar (stated by the matmul path's north star): relative error <= 1e-5 * sqrt(K) against fp64,
both normwise ||C - C64||_F / ||C64||_F and componentwise max |C - C64| / (|A||B|)."""
import numpy as np
import torch

import oracle


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def sample_rows(M, count=24, seed=0):
    """Rows that cover every tile edge class: first/last rows, 32/64/128 boundaries, random."""
    rows = {0, M - 1}
    for b in (31, 32, 63, 64, 127, 128, 255, 256):
        if b < M:
            rows.add(b)
    rng = np.random.default_rng(seed)
    rows.update(int(r) for r in rng.integers(0, M, size=count))
    return sorted(rows)


def check_gemm(C, A, B, transA, transB, bias=None, M=None, N=None, K=None, lda=None, ldb=None,
               sA=0, sB=0, batch=1, rows=None, ref=None):
    """Compare GPU output C (numpy [batch, M, N]) with fp64 on the selected rows.
    Returns (normwise, componentwise, vs_ref) where vs_ref is the componentwise distance to
    the restated reference arithmetic `ref` (if given)."""
    C = np.asarray(C).reshape(batch, M, N)
    rows = list(range(M)) if rows is None else rows
    tol = oracle.tolerance(K)
    worst_nw = worst_cw = 0.0
    vs_ref = 0.0
    # contiguous runs of rows keep the fp64 calls few
    runs = []
    for r in rows:
        if runs and runs[-1][1] == r:
            runs[-1][1] = r + 1
        else:
            runs.append([r, r + 1])
    c64_parts, ap_parts, c_parts, ref_parts = [], [], [], []
    for r0, r1 in runs:
        kw = dict(M=M, N=N, K=K, lda=lda, ldb=ldb, sA=sA, sB=sB, batch=batch, rows=(r0, r1))
        c64_parts.append(oracle.gemm_f64(A, B, transA, transB, bias, **kw))
        ap_parts.append(oracle.gemm_absprod(A, B, transA, transB, bias, **kw))
        c_parts.append(C[:, r0:r1, :])
        if ref is not None:
            ref_parts.append(np.asarray(ref).reshape(batch, M, N)[:, r0:r1, :])
    c64 = np.concatenate(c64_parts, axis=1)
    ap = np.concatenate(ap_parts, axis=1)
    cg = np.concatenate(c_parts, axis=1)
    worst_nw, worst_cw = oracle.errors(cg, c64, ap)
    if ref is not None:
        rr = np.concatenate(ref_parts, axis=1).astype(np.float64)
        with np.errstate(divide="ignore", invalid="ignore"):
            d = np.abs(cg.astype(np.float64) - rr)
            vs_ref = float(np.max(np.where(ap > 0, d / ap, np.where(d > 0, np.inf, 0.0))))
    assert np.all(np.isfinite(cg)), "non-finite output"
    assert worst_nw <= tol, f"normwise error {worst_nw:.3e} > {tol:.3e}"
    assert worst_cw <= tol, f"componentwise error {worst_cw:.3e} > {tol:.3e}"
    if ref is not None:
        assert vs_ref <= 2 * tol, f"distance to the reference arithmetic {vs_ref:.3e}"
    return worst_nw, worst_cw, vs_ref


class Tuner:
    """Sets dispatcher tuning overrides through the C ABI (migemm_set_tuning: tile=,
    splitk=, direct=, small_tiles=, small_splitk=; None = the dispatcher's choice) and
    restores the values it replaced."""

    def __init__(self):
        self.saved = {}

    def set(self, **kv):
        from my_pytchon_opencl_lib_amd import _native
        for k, v in kv.items():
            if k == "tile" and v == "128x256":
                v = _native.MIGEMM_TILE_128x256
            prev = _native.set_tuning(k, 0 if v is None else int(v))
            self.saved.setdefault(k, prev)

    def restore(self):
        from my_pytchon_opencl_lib_amd import _native
        for k, v in self.saved.items():
            _native.set_tuning(k, v)
        self.saved = {}


def check_full(C, A, B, transA, transB, bias=None, ref=None):
    """Whole-output check of a single 2-D GEMM C = op(A) op(B) (+ bias) against fp64: C64
    and |op(A)| |op(B)| (+ |bias|) by numpy's float64 matmul over every element, both error
    bounds of oracle.errors, and (if given) the componentwise distance of every element to
    the reference kernel's output `ref`. Returns (normwise, componentwise, vs_ref)."""
    a = np.asarray(A, np.float64)
    b = np.asarray(B, np.float64)
    a = a.T if transA else a
    b = b.T if transB else b
    K = a.shape[1]
    c64 = a @ b
    ap = np.abs(a) @ np.abs(b)
    if bias is not None:
        c64 += np.asarray(bias, np.float64)
        ap += np.abs(np.asarray(bias, np.float64))
    C = np.asarray(C).reshape(c64.shape)
    assert np.all(np.isfinite(C)), "non-finite output"
    tol = oracle.tolerance(K)
    nw, cw = oracle.errors(C, c64, ap)
    assert nw <= tol, f"normwise error {nw:.3e} > {tol:.3e}"
    assert cw <= tol, f"componentwise error {cw:.3e} > {tol:.3e}"
    vs_ref = 0.0
    if ref is not None:
        d = np.abs(C.astype(np.float64) - np.asarray(ref, np.float64).reshape(c64.shape))
        with np.errstate(divide="ignore", invalid="ignore"):
            vs_ref = float(np.max(np.where(ap > 0, d / ap, np.where(d > 0, np.inf, 0.0))))
        assert vs_ref <= 2 * tol, f"distance to the reference kernel {vs_ref:.3e}"
    return nw, cw, vs_ref
