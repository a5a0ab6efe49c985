"""The dispatcher's kernel choices, pinned on the CPU through the dry-run entry point
migemm_gemm_plan (validates and plans exactly as migemm_gemm_strided_batched_ex, launches
nothing, makes no HIP call): every BASELINE config, every caller shape of the path and the
regime table (tests/dispatch_cases.py). A change to the dispatcher shows up here as a
changed plan string; the GPU suite checks that real calls record the same plans
(tests/test_gemm_gpu.py::test_dry_run_plans_match_real_calls)."""
import pytest

import dispatch_cases as dc
from my_pytchon_opencl_lib_amd import _native


@pytest.fixture(autouse=True)
def auto_policy():
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_AUTO)
    yield
    _native.set_gemm_policy(prev)


@pytest.mark.parametrize("name,spec,plan", dc.BASELINE + dc.CALLERS,
                         ids=[c[0] for c in dc.BASELINE + dc.CALLERS])
def test_plan_of_baseline_and_callers(name, spec, plan):
    assert _native.gemm_plan(*dc.args(**spec)) == plan


@pytest.mark.parametrize("spec,plan", dc.AUTO_REGIMES)
def test_plan_of_regime_table(spec, plan):
    assert _native.gemm_plan(*dc.regime_args(spec)).startswith(plan)


def test_plan_validates_like_the_gemm_entry():
    a = dc.args(64, 64, 64)
    with pytest.raises(_native.MigemmArgumentError, match="sizes must be >= 1"):
        _native.gemm_plan(*dc.args(0, 64, 64))
    # C on top of A
    bad = list(a)
    bad[12] = bad[5]
    with pytest.raises(_native.MigemmArgumentError, match="overlaps"):
        _native.gemm_plan(*bad)
    with pytest.raises(_native.MigemmArgumentError, match="unknown flags"):
        _native.gemm_plan(*a[:-1], 2)


def test_plan_follows_policy_and_tuning():
    """The dry run sees the process-wide policy and tuning overrides as a real call does."""
    a = dc.args(4096, 4096, 4096)
    prev = _native.set_gemm_policy(_native.MIGEMM_POLICY_SMALL)
    try:
        assert _native.gemm_plan(*a).startswith("small ")
    finally:
        _native.set_gemm_policy(prev)
    with _native.tuned(tile=128, splitk=2):
        assert _native.gemm_plan(*a).startswith("tiled-direct tile=128x128 splits=2 ")
    assert _native.gemm_plan(*a).startswith("tiled-direct tile=256x256 splits=1 ")
