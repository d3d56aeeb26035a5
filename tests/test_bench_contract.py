"""CPU checks of bench.py's contract: one GPU only, and the algorithmic byte
and flop constants the roofline fractions are computed from."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import bench  # noqa: E402
from oracle import ref_moe as R  # noqa: E402


def test_more_than_one_gpu_exits_with_message():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2", "--no-pmc"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "one GPU" in r.stderr and r.stdout == ""


def test_algorithmic_constants():
    # per active expert: weights + block scales (the published 1.41 GB for all 32 experts)
    assert bench.W1_EXPERT_BYTES == 29_367_296 and bench.W2_EXPERT_BYTES == 14_683_648
    assert 32 * (bench.W1_EXPERT_BYTES + bench.W2_EXPERT_BYTES) == 1_409_630_208
    # the whole-call formula agrees with the oracle's restatement of it
    for T, a_e in ((1, 0), (64, 20), (8192, 28)):
        assert bench.call_bytes(T, a_e) == R.algorithmic_bytes(T, a_e)
    assert bench.GEMM1_FLOPS_PER_SLOT + bench.GEMM2_FLOPS_PER_SLOT == R.algorithmic_flops(1)
    # per-launch GEMM bytes: weights once per active expert, one row in and out per slot
    assert bench.gemm1_bytes(105, 20) == 20 * 29_367_296 + 105 * (7168 + 224 + 4096)
    assert bench.gemm2_bytes(105, 20) == 20 * 14_683_648 + 105 * (4096 + 14336)


def test_counter_passes_never_start_under_a_profiler(monkeypatch):
    """Run under rocprofv3 (its tool library preloaded), bench.py must not
    start its own rocprofv3 children: the profiler has already initialised
    the GPU in this process. pmc_counters returns None without spawning."""
    started = []
    monkeypatch.setattr(bench.subprocess, "run", lambda *a, **k: started.append(a) or None)
    monkeypatch.setattr(bench.shutil, "which", lambda name: "/opt/rocm/bin/" + name)
    for env in ({"LD_PRELOAD": "/opt/rocm/lib/rocprofiler-sdk/librocprofiler-sdk-tool.so"},
                {"ROCP_TOOL_LIBRARIES": "/opt/rocm/lib/rocprofiler-sdk/librocprofiler-sdk-tool.so"},
                {"LD_PRELOAD": "/x/libharness.so:/opt/rocm/lib/librocprofiler-sdk.so"}):
        for k in ("LD_PRELOAD", "ROCP_TOOL_LIBRARIES", "HSA_TOOLS_LIB"):
            monkeypatch.delenv(k, raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        assert bench.profiler_inherited()
        assert bench.pmc_counters("c3_t8192", "gemm1_tile") is None
    assert started == []
    # an unrelated preload is not a profiler
    assert not bench.profiler_inherited({"LD_PRELOAD": "/usr/lib/libharness.so"})
    assert not bench.profiler_inherited({})
