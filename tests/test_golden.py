"""Golden fixtures (tests/golden/, written by tests/golden/make_golden.py).

CPU: the seeded generator still produces the same inputs (SHA-256), and the
oracle still produces the stored routing and output. GPU: the operator's
output and routing match the stored answer without running the oracle."""
import json
import os

import numpy as np
import pytest
import torch

from flashinfer_amd import workloads as W
from oracle import ref_moe as R

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TENSORS = ["routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
           "gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale"]


def _c0_meta():
    with open(os.path.join(GOLDEN, "c0_t16.json")) as f:
        return json.load(f)


def _c0_arrays():
    return np.load(os.path.join(GOLDEN, "c0_t16.npz"))


def _golden_output(z):
    return torch.from_numpy(z["output_bf16_bits"].copy()).view(torch.bfloat16).float()


def test_c0_inputs_match_golden_hashes():
    meta = _c0_meta()
    wl = W.standard(meta["workload"])
    assert (wl.T, wl.seed, wl.local_expert_offset) == (meta["T"], meta["seed"],
                                                       meta["local_expert_offset"])
    assert W.WEIGHT_SEED == meta["weight_seed"]
    assert wl.routed_scaling_factor == meta["routed_scaling_factor"]
    for n in TENSORS:
        assert W.sha256(wl.tensors[n]) == meta["sha256"][n], n


def test_oracle_reproduces_c0_golden():
    z = _c0_arrays()
    wl = W.standard("c0_t16")
    res = R.moe_forward(*wl.args())
    assert torch.equal(res.route.ids.to(torch.int32), torch.from_numpy(z["ids"]))
    assert torch.allclose(res.route.weights, torch.from_numpy(z["weights"]), rtol=1e-6, atol=0)
    # The fp32 oracle may differ by a bf16 ulp across BLAS builds; the stored
    # output must agree to far inside the operator tolerance.
    rep = R.tolerance_report(res.output.float(), _golden_output(z), rtol=4e-3, atol_rel=1e-3)
    assert rep["n_bad"] == 0, rep
    assert rep["normwise_rel"] < 1e-3, rep


def test_oracle_reproduces_tiny_golden():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", os.path.join(GOLDEN, "make_golden.py"))
    mg = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mg)
    z = np.load(os.path.join(GOLDEN, "tiny_t24.npz"))
    wl = mg.tiny_workload()
    res = R.moe_forward(*wl.args(), acc_dtype=torch.float64)
    assert torch.equal(res.route.ids.to(torch.int32), torch.from_numpy(z["ids"]))
    assert torch.allclose(res.route.weights, torch.from_numpy(z["weights"]), rtol=1e-6, atol=0)
    want = torch.from_numpy(z["acc"])
    assert torch.allclose(res.acc, want, rtol=1e-9, atol=1e-12 * float(want.abs().max()))
    # the tiny case must route to some local experts and some non-local ones
    local = (res.route.ids >= wl.local_expert_offset) & (res.route.ids < wl.local_expert_offset + 32)
    assert 0 < int(local.sum()) < res.route.ids.numel()


@pytest.mark.gpu
def test_gpu_matches_c0_golden():
    from _helpers import log, run_gpu
    from flashinfer_amd import kernel
    log("test_gpu_matches_c0_golden")
    z = _c0_arrays()
    wl = W.standard("c0_t16")
    out = run_gpu(wl, fill=float("nan")).float().cpu()
    rep = R.tolerance_report(out, _golden_output(z))
    log(f"golden c0_t16: {rep}")
    assert torch.isfinite(out).all()
    assert rep["n_bad"] == 0, rep
    t = wl.tensors
    ids, w = kernel.route(t["routing_logits"].cuda(), t["routing_bias"].cuda(),
                          wl.routed_scaling_factor)
    assert torch.equal(ids.cpu().to(torch.int32), torch.from_numpy(z["ids"]))
    assert torch.allclose(w.cpu(), torch.from_numpy(z["weights"]), rtol=1e-6, atol=0)
