"""Env-gated phase timing of ``run`` (the reference's FIB_PROFILE_PHASES /
FIB_PHASE_TIMING_OUTPUT switch, solution/triton/kernel.py:10-55, :631-672):
one JSON file on the first call, the same top-level keys, the same output."""
import json

import pytest
import torch

from _helpers import log, run_gpu

from flashinfer_amd import kernel
from flashinfer_amd import workloads as W

pytestmark = pytest.mark.gpu


def test_phase_timing_json_written_once(tmp_path, monkeypatch):
    from oracle import ref_moe as R
    log("test_phase_timing_json_written_once")
    wl = W.standard("c1_t64")
    plain = run_gpu(wl)
    out_path = tmp_path / "phases" / "t64.json"
    monkeypatch.setenv("FIB_PROFILE_PHASES", "1")
    monkeypatch.setenv("FIB_PHASE_TIMING_OUTPUT", str(out_path))
    monkeypatch.setattr(kernel, "_PHASE_JSON_WRITTEN", False)
    timed = run_gpu(wl)
    assert torch.equal(timed.view(torch.int16).cpu(), plain.view(torch.int16).cpu())
    d = json.loads(out_path.read_text())
    assert set(d) >= {"total_tokens", "phase_ms", "ratio_percent", "total_ms"}
    r = R.route(wl.tensors["routing_logits"], wl.tensors["routing_bias"], wl.routed_scaling_factor)
    slots = R.local_assignment(r.ids, r.weights, wl.local_expert_offset, 32)
    assert d["total_tokens"] == sum(len(tk) for tk, _ in slots)
    assert set(d["phase_ms"]) == {"phase1_route_permute", "phase3_gemm1", "phase5_gemm2",
                                  "phase6_scatter"}
    assert all(v > 0 for v in d["phase_ms"].values())
    assert d["total_ms"] == pytest.approx(sum(d["phase_ms"].values()))
    assert sum(d["ratio_percent"].values()) == pytest.approx(100.0)
    assert set(d["phase_ms_native"]) == {"route", "sort", "gemm1_swiglu", "gemm2", "combine"}
    # once per process, as the reference: a second call writes nothing
    out_path.unlink()
    run_gpu(wl)
    assert not out_path.exists()


def test_profiler_range(monkeypatch):
    """With FIB_PROFILE_PHASES=1 each call sits in a record_function range
    (the reference's _profile_region, kernel.py:10-24) that torch.profiler
    sees; without it there is none. The output is unchanged."""
    log("test_profiler_range")
    wl = W.standard("c1_t16")
    plain = run_gpu(wl)
    monkeypatch.delenv("FIB_PHASE_TIMING_OUTPUT", raising=False)
    for flag, expect in (("1", True), ("0", False)):
        monkeypatch.setenv("FIB_PROFILE_PHASES", flag)
        with torch.profiler.profile(activities=[torch.profiler.ProfilerActivity.CPU]) as prof:
            out = run_gpu(wl)
        names = {e.key for e in prof.key_averages()}
        assert ("mi_moe_run" in names) == expect, sorted(names)[:20]
        assert torch.equal(out.view(torch.int16), plain.view(torch.int16))
