"""GEMM shapes whose kernel choice is pinned, shared by the CPU plan test
(tests/test_plans.py, through the dry-run entry migemm_gemm_plan) and the GPU tests (which
run them and compare the plan a real call records).

  BASELINE  every BASELINE.json config and the forms the bench times;
  CALLERS   the path's callers at the reference's sizes: Linear(500 -> 6565) on [8, 1500, 500]
            (TestLSTMRealTrain/EncoderDecoder.cs:29,75) forward, dX, dW; the LSTM of config 3
            (64 sequences x 100 steps, input 512, hidden 1024): lstm_gemm_xw, lstm_gemm_grad_x,
            the two accumulating weight-gradient GEMMs and one recurrent step;
  AUTO_REGIMES  shapes at the edges of the dispatcher's regimes.
Each entry is (name, arguments of migemm_gemm_strided_batched_ex as a dict, expected plan).
Addresses are fixed multiples of 2^32 (the real tests' tensors are at least 512-byte
aligned, so alignment-dependent choices agree); `off*` shift an operand by elements, as the
recurrent step's views of H_out and XW do."""

BASES = {"A": 1 << 32, "B": 2 << 32, "bias": 3 << 32, "C": 4 << 32}


def args(M, N, K, ta=0, tb=0, batch=1, bias=False, acc=False, lda=None, ldb=None, ldc=None,
         sA=None, sB=None, sC=None, offA=0, offC=0):
    """Positional arguments of migemm_gemm_plan / _ex (without the stream)."""
    lda = lda if lda is not None else (M if ta else K)
    ldb = ldb if ldb is not None else (K if tb else N)
    ldc = ldc if ldc is not None else N
    sA = sA if sA is not None else (M * K if batch > 1 else 0)
    sB = sB if sB is not None else (K * N if batch > 1 else 0)
    sC = sC if sC is not None else (M * N if batch > 1 else 0)
    return (ta, tb, M, N, K, BASES["A"] + 4 * offA, lda, sA, BASES["B"], ldb, sB,
            BASES["bias"] if bias else None, BASES["C"] + 4 * offC, ldc, sC, batch,
            1 if acc else 0)


BASELINE = [
    ("cfg1 NN 256^3", dict(M=256, N=256, K=256),
     "tiny tile=16x16 splits=4 load_bytes=0 M=256 N=256 K=256 batch=1 NN"),
    ("cfg2a Q K^T batch 32", dict(M=128, N=128, K=64, batch=32),
     "tiny tile=16x16 splits=1 load_bytes=0 M=128 N=128 K=64 batch=32 NN"),
    ("cfg2b P V batch 32", dict(M=128, N=64, K=128, batch=32),
     "tiny tile=16x16 splits=4 load_bytes=0 M=128 N=64 K=128 batch=32 NN"),
    ("cfg3 LSTM gate step + bias", dict(M=64, N=4096, K=1536, bias=True),
     "panel tile=32x32 splits=1 load_bytes=16 M=64 N=4096 K=1536 batch=1 NN"),
    ("cfg4 NN", dict(M=4096, N=4096, K=4096),
     "tiled-direct tile=256x256 splits=1 load_bytes=16 M=4096 N=4096 K=4096 batch=1 NN"),
    ("cfg4 NT dA", dict(M=4096, N=4096, K=4096, tb=1),
     "tiled-direct tile=256x256 splits=1 load_bytes=16 M=4096 N=4096 K=4096 batch=1 NT"),
    ("cfg4 TN dB", dict(M=4096, N=4096, K=4096, ta=1),
     "tiled-direct tile=256x256 splits=1 load_bytes=16 M=4096 N=4096 K=4096 batch=1 TN"),
    ("cfg5a ragged", dict(M=1000, N=3000, K=777),
     "tiled-direct tile=64x64 splits=1 load_bytes=4 M=1000 N=3000 K=777 batch=1 NN"),
    ("cfg5b GEMV", dict(M=1, N=11008, K=4096),
     "skinny tile=0x256 splits=16 load_bytes=0 M=1 N=11008 K=4096 batch=1 NN"),
]

CALLERS = [
    ("Linear forward (C#: W [1, 500, 6565] + bias)",
     dict(M=1500, N=6565, K=500, batch=8, sB=0, bias=True),
     "tiled-direct tile=128x128 splits=1 load_bytes=4 M=12000 N=6565 K=500 batch=1 NN"),
    ("Linear forward (Python: W [6565, 500], NT)", dict(M=12000, N=6565, K=500, tb=1),
     "tiled-direct tile=128x256 splits=1 load_bytes=16 M=12000 N=6565 K=500 batch=1 NT"),
    ("Linear dX = dY W^T", dict(M=1500, N=500, K=6565, batch=8, tb=1, sB=0),
     "tiled-direct tile=128x128 splits=4 load_bytes=4 M=12000 N=500 K=6565 batch=1 NT"),
    ("Linear dW = X^T dY over 12000 rows", dict(M=500, N=6565, K=12000, ta=1),
     "tiled-direct tile=128x128 splits=6 load_bytes=4 M=500 N=6565 K=12000 batch=1 TN"),
    ("lstm_gemm_xw", dict(M=6400, N=4096, K=512, bias=True),
     "tiled-direct tile=64x64 splits=1 load_bytes=16 M=6400 N=4096 K=512 batch=1 NN"),
    ("lstm_gemm_grad_x", dict(M=6400, N=512, K=4096, tb=1),
     "tiled-direct tile=64x64 splits=3 load_bytes=16 M=6400 N=512 K=4096 batch=1 NT"),
    ("lstm grad_W += X^T G", dict(M=512, N=4096, K=6400, ta=1, acc=True),
     "tiled-direct tile=64x64 splits=1 load_bytes=16 M=512 N=4096 K=6400 batch=1 TN"),
    ("lstm grad_U += H_prev^T G", dict(M=1024, N=4096, K=6400, ta=1, acc=True),
     "tiled-direct tile=256x256 splits=4 load_bytes=16 M=1024 N=4096 K=6400 batch=1 TN"),
    ("lstm recurrent step t=50", dict(M=64, N=4096, K=1024, acc=True, lda=100 * 1024,
                                      ldc=100 * 4096, offA=49 * 1024, offC=50 * 4096),
     "panel tile=32x32 splits=1 load_bytes=16 M=64 N=4096 K=1024 batch=1 NN"),
]

# (spec, expected plan prefix) -- the regime table of the GPU test test_auto_regimes
AUTO_REGIMES = [
    # 5-16 rows over >= 256 MB of B: 32x32 tiles, k split to ~1536 work-groups
    (dict(batch=16, M=8, K=6000, N=1024, ta=0, tb=0), "tiled-staged tile=32x32 splits=3"),
    # operands not loadable 16 bytes per lane, short K, large output: 64x64 tiles
    (dict(batch=1, M=2047, K=61, N=2051, ta=1, tb=1), "tiled-direct tile=64x64"),
    # 16 or fewer rows: the small kernel, or the short-K kernel for K <= 80
    (dict(batch=32, M=8, K=195, N=1000, ta=0, tb=0), "small"),
    (dict(batch=8, M=10, K=75, N=2166, ta=0, tb=0), "tiny"),
    (dict(batch=32, M=2, K=35, N=7626, ta=1, tb=0), "tiny"),
    # few 64x64 tiles and K < 256: the small kernel
    (dict(batch=1, M=1000, K=100, N=700, ta=0, tb=0), "small"),
    # a weight stored [N, K] at M = 1: rows streamed whole
    (dict(batch=1, M=1, K=4096, N=2048, ta=0, tb=1), "skinny-rows"),
    # a tiny output over a huge K (dot products): the small kernel in 256 k ranges
    (dict(batch=1, M=1, K=1000000, N=1, ta=0, tb=0), "small tile=16x16 splits=256"),
    (dict(batch=1, M=7, K=300000, N=9, ta=0, tb=1), "small tile=16x16 splits=254"),
    # outputs of >= 64 MB over K <= 16 with C rows on 128-byte lines: 128x128 tiles
    (dict(batch=1, M=8192, K=4, N=8192, ta=0, tb=0), "tiled-direct tile=128x128"),
    # the same with rows off the lines: the short-K kernel
    (dict(batch=1, M=7008, K=6, N=6220, ta=0, tb=0), "tiny"),
    # short K, C rows off 64-byte boundaries: 64x64 tiles; on them (operands loaded 4 bytes
    # per lane, >= 6 rounds of tiles): 128x128
    (dict(batch=1, M=8192, K=64, N=8180, ta=0, tb=0), "tiled-direct tile=64x64"),
    (dict(batch=1, M=12592, K=47, N=2304, ta=0, tb=0), "tiled-direct tile=128x128"),
    # long K over few tiles: 64x64 tiles in k ranges (the LSTM gate gradient)
    (dict(batch=1, M=6400, K=4096, N=512, ta=0, tb=1), "tiled-direct tile=64x64 splits=3"),
    # one row of C, B stored [N, K], few rows: the rows GEMV; 3 rows over a batch whose
    # entries hold small B: the small kernel
    (dict(batch=1, M=1, K=1301, N=440, ta=0, tb=1), "skinny-rows"),
    (dict(batch=8, M=3, K=6278, N=362, ta=0, tb=0), "small"),
    # 3-4 rows over a batch with N % 4 != 0: from 96 MB of B over the batch, the skinny
    # kernel (below it, the small kernel)
    (dict(batch=4, M=4, K=11887, N=529, ta=0, tb=0), "skinny tile=0x256"),
    (dict(batch=8, M=3, K=3350, N=866, ta=0, tb=0), "small"),
    # a narrow output over long K with 16 MB or more of operands: 1.5x the k ranges
    (dict(batch=1, M=1846, K=4713, N=17, ta=0, tb=0), "small tile=32x32 splits=8"),
]


def regime_args(spec):
    return args(spec["M"], spec["N"], spec["K"], ta=spec["ta"], tb=spec["tb"],
                batch=spec["batch"])
