"""The stateful LSTM gate product on the GPU: migemm_lstm_hid_gates, the per-step
workspace[t] = bias + x_t W + h_{t-1} U of kernel lstm_hid_forward (cs/cl_kernels/lstm.cl:
788-870, gate loop :832-844; enqueued by NnClGlob.LstmWithWithState, cs/compiler/NnClGlob.cs:
1067-1100), with x, h, W and U as four separate buffers. The reference kernel itself is run
in tests/test_reference_gpu.py; here the HIP path is checked against exact small-integer
answers on every kernel family and against fp64 at BASELINE config 3's sizes."""
import ctypes

import numpy as np
import pytest
import torch

import oracle
from parity import dev, host

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)


def small_ints(shape, seed, lo=-3, hi=3):
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=shape).astype(np.float32)


def hp_of(Hp, Ho, t):
    """h_{t-1} of every sequence: the incoming state at t = 0, else the previous output."""
    return Hp if t == 0 else Ho[:, t - 1]


# (batch, seq, in_features, hidden): config 3's LSTM (input 512, hidden 1024, 64 sequences);
# panel-eligible shapes with few and many rows; ragged ones that run as two GEMMs
SHAPES = [(64, 3, 512, 1024), (40, 2, 96, 64), (5, 3, 64, 32), (3, 4, 10, 12),
          (33, 2, 30, 17), (1, 2, 7, 5), (17, 2, 64, 31)]


@pytest.mark.parametrize("B,S,F,H", SHAPES)
def test_hid_gates_exact(nncl, policy, B, S, F, H):
    """Small-integer operands make every partial sum exact, so each step's gates equal the
    integer answer bias + x_t W + h_{t-1} U bit for bit whatever the summation order, under
    every kernel family. Only workspace[t] is written (NaN canaries elsewhere)."""
    say("hid_gates exact", policy, B, S, F, H)
    G = 4 * H
    X = small_ints((B, S, F), B + F)
    W = small_ints((F, G), F + G)
    U = small_ints((H, G), H + G + 1)
    bias = small_ints((G,), G, -20, 20)
    Hp = small_ints((B, H), B + H + 2)
    Ho = small_ints((B, S, H), B + S + H)
    x, w, u, b, hp, ho = dev(X), dev(W), dev(U), dev(bias), dev(Hp), dev(Ho)
    ws = torch.full((S, B, G), float("nan"), device="cuda:0")
    for t in range(S):
        nncl.LstmHidGates(x, w, u, b, hp, ho, ws, t)
        got = host(ws)
        expect = (bias.astype(np.int64) + X[:, t].astype(np.int64) @ W.astype(np.int64) +
                  hp_of(Hp, Ho, t).astype(np.int64) @ U.astype(np.int64))
        assert np.array_equal(got[t], expect.astype(np.float32)), t
        assert np.all(np.isnan(got[t + 1:])), "a later step's gates were written"


def test_hid_gates_one_launch_at_config3(nncl):
    """At config 3's sizes the product is one panel launch over both operand pairs (48
    k-groups: 16 of x W, 32 of h U), not a concatenation plus a GEMM."""
    from my_pytchon_opencl_lib_amd import _native
    B, S, F, H = 64, 2, 512, 1024
    z = lambda *s: torch.zeros(*s, device="cuda:0")
    nncl.LstmHidGates(z(B, S, F), z(F, 4 * H), z(H, 4 * H), z(4 * H), z(B, H), z(B, S, H),
                      z(S, B, 4 * H), 1)
    plan = _native.last_plan()
    assert plan.startswith("panel-pair ") and " K=1536 " in plan, plan


def test_hid_gates_config3_fp64(nncl):
    """BASELINE config 3 in the reference's stateful form: 64 sequences, input 512, hidden
    1024, W and U ~ U(-1/32, 1/32), bias likewise, x ~ N(0, 1), h in (-1, 1); every step
    within 1e-5*sqrt(1536) of fp64, normwise and componentwise, and equal to the same product
    through the general GEMM entry on the concatenated [x_t || h_{t-1}] and [W; U] within
    that bound."""
    B, S, F, H = 64, 4, 512, 1024
    G = 4 * H
    X = oracle.normal((B, S, F), 2, 10)
    W = oracle.uniform((F, G), 2, 11, -1 / 32, 1 / 32)
    U = oracle.uniform((H, G), 2, 12, -1 / 32, 1 / 32)
    bias = oracle.uniform((G,), 2, 13, -1 / 32, 1 / 32)
    Hp = oracle.uniform((B, H), 2, 14, -1.0, 1.0)
    Ho = oracle.uniform((B, S, H), 2, 15, -1.0, 1.0)
    x, w, u, b, hp, ho = dev(X), dev(W), dev(U), dev(bias), dev(Hp), dev(Ho)
    ws = torch.empty((S, B, G), device="cuda:0")
    WU = np.concatenate([W, U]).astype(np.float64)
    tol = oracle.tolerance(F + H)
    for t in range(S):
        nncl.LstmHidGates(x, w, u, b, hp, ho, ws, t)
        got = host(ws)[t]
        xh = np.concatenate([X[:, t], hp_of(Hp, Ho, t)], axis=1).astype(np.float64)
        c64 = xh @ WU + bias
        ap = np.abs(xh) @ np.abs(WU) + np.abs(bias)
        nw, cw = oracle.errors(got, c64, ap)
        say("step", t, "normwise", nw, "componentwise", cw)
        assert nw <= tol and cw <= tol, (t, nw, cw)
        cat = nncl.gemm(dev(xh.astype(np.float32)), dev(WU.astype(np.float32)), bias=b)
        d = np.max(np.abs(host(cat).astype(np.float64) - got) / ap)
        assert d <= 2 * tol, (t, d)


def test_hid_gates_validation(nncl):
    """Argument errors are reported before any launch, as ValueError (the reference's
    ArgumentException): wrong shapes, a step outside the sequence, a null state at the step
    that reads it, and gates that overlap an input."""
    from my_pytchon_opencl_lib_amd import _native
    B, S, F, H = 4, 3, 32, 8
    z = lambda *s: torch.zeros(*s, device="cuda:0")
    x, w, u, b = z(B, S, F), z(F, 4 * H), z(H, 4 * H), z(4 * H)
    hp, ho, ws = z(B, H), z(B, S, H), z(S, B, 4 * H)
    with pytest.raises(ValueError):
        nncl.LstmHidGates(x, w, u, b, hp, ho, ws, S)
    with pytest.raises(ValueError):
        nncl.LstmHidGates(x, z(F + 1, 4 * H), u, b, hp, ho, ws, 0)
    with pytest.raises(ValueError):
        nncl.LstmHidGates(x, w, u, b, z(B, H + 1), ho, ws, 0)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    L = _native.load()
    # H_prev may be NULL after step 0, H_out at step 0; not the other way round
    assert L.migemm_lstm_hid_gates(stream, p(x), p(w), p(u), p(b), None, p(ho), p(ws), B, S, F,
                                   H, 1) == _native.MIGEMM_OK
    assert L.migemm_lstm_hid_gates(stream, p(x), p(w), p(u), p(b), p(hp), None, p(ws), B, S, F,
                                   H, 0) == _native.MIGEMM_OK
    assert L.migemm_lstm_hid_gates(stream, p(x), p(w), p(u), p(b), None, p(ho), p(ws), B, S, F,
                                   H, 0) == _native.MIGEMM_ERR_INVALID_ARG
    assert L.migemm_lstm_hid_gates(stream, p(x), p(w), p(u), p(b), p(hp), None, p(ws), B, S, F,
                                   H, 2) == _native.MIGEMM_ERR_INVALID_ARG
    # the step's gates on top of h_{t-1}
    big = z(S * B * 4 * H + B * S * H)
    ws_alias = big[:S * B * 4 * H]
    ho_alias = big[S * B * 4 * H - B * 4 * H:][:B * S * H]
    assert L.migemm_lstm_hid_gates(stream, p(x), p(w), p(u), p(b), p(hp), p(ho_alias),
                                   p(ws_alias), B, S, F, H, S - 1) == _native.MIGEMM_ERR_ALIAS
    torch.cuda.synchronize()
