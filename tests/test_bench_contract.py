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


def test_parity_block_pass_and_planted_error():
    """The parity fields the bench prints per workload: the oracle's own bf16
    output passes with zero routing mismatches; a planted error in one
    element (made on the CPU) is counted outside the bar."""
    import torch
    from flashinfer_amd import workloads as W
    wl = W.make_workload("tiny", T=40, seed=21, H=256, I=128, weight_seed=99)
    tok = bench.parity_tokens(wl.T)
    assert torch.equal(tok, torch.arange(40))
    ref = R.moe_forward(*wl.args())
    chk = {"tokens": tok, "out": ref.output.clone(), "ids": ref.route.ids.clone()}
    p = bench.parity_block(wl, chk)
    assert p["pass"] and p["routing_set_mismatches"] == 0 and p["frac_outside"] == 0.0
    assert p["tokens_checked"] == 40 and p["of_tokens"] == 40
    assert p["normwise_rel"] < 5e-3  # the bf16 rounding of the output alone
    bad = dict(chk, out=chk["out"].clone())
    r, c = divmod(int(ref.acc.abs().argmax()), 256)
    bad["out"][r, c] = -bad["out"][r, c]
    q = bench.parity_block(wl, bad)
    assert not q["pass"] and q["frac_outside"] > 0 and q["max_rel_err"] >= 1.9
    ids = chk["ids"].clone()
    a0, a1 = int(ids[3, 0]), int(ids[3, 1])
    ids[3, 0], ids[3, 1] = a1, a0  # order within a set does not count
    assert bench.parity_block(wl, dict(chk, ids=ids))["routing_set_mismatches"] == 0
    ids[5, 0] = (int(ids[5, 0]) + 1) % 256 if int(ids[5, 0]) + 1 not in ids[5].tolist() else 255
    assert bench.parity_block(wl, dict(chk, ids=ids))["routing_set_mismatches"] == 1


def test_parity_subset_spreads_over_large_t():
    tok = bench.parity_tokens(14000)
    assert tok[0] == 0 and tok[-1] == 13999 and len(tok) == bench.PARITY_SUBSET
    assert torch_sorted(tok)


def torch_sorted(t):
    return bool((t[1:] > t[:-1]).all())


def test_compact_sweep_entry_is_small():
    import json
    res = {"workload": "c3_t8192", "T": 8192, "slots": 11559, "active_experts": 28,
           "us_per_call": 870.1, "us_per_call_cold": 900.2, "us_per_call_graph": 880.3,
           "gbps": 1600.1, "tflops": 1150.2, "roofline_frac": 0.23, "mixed_roofline_frac": 0.31,
           "phase_us": {"route": 12.34, "sort": 16.5, "gemm1_swiglu": 407.21, "gemm2": 380.4,
                        "combine": 52.2},
           "roofline": {"kernel": "gemm1_swiglu", "bound": "mfma", "achieved": 1666.9,
                        "unit": "TFLOP/s", "frac": 0.3334, "avg_launch_us": 407.2, "mfma_dtype": "fp8",
                        "algorithmic_bytes_per_launch": 1, "gbps": 2.0},
           "kernels": {"gemm1_swiglu": {"x": 1}, "gemm2": {"y": 2}}, "trials_us": [1.0] * 5,
           "parity": {"pass": True}, "cpu_baseline": {"value": 1.0}}
    c = bench.compact(res)
    assert "kernels" not in c and "trials_us" not in c and c["parity"] == {"pass": True}
    assert set(c["roofline"]) == {"kernel", "bound", "achieved", "unit", "frac", "avg_launch_us"}
    assert len(json.dumps(c)) < 900
