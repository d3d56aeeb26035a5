"""mi_moe_run_noalloc (no workspace, no allocation: intermediates in the
library's static per-GPU scratch) against mi_moe_run with a caller workspace,
through the C ABI: the same kernels run, so outputs must be equal bit for bit
(stricter than the 1e-2 output bar). Calls in a row, each with fewer tokens
than the one before (the scratch keeps the previous call's contents), and the
Python mirror ``kernel.run_noalloc``."""
import ctypes

import pytest
import torch

from _helpers import gpu_args, log

from flashinfer_amd import _lib, kernel
from flashinfer_amd import workloads as W

pytestmark = pytest.mark.gpu
H = 7168


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _c_args(args, out, workspace=None):
    t = args[:8]
    ws, nbytes = (None, 0) if workspace is None else (workspace.data_ptr(), workspace.numel())
    return _lib.MiMoeArgs(
        routing_logits=t[0].data_ptr(), routing_bias=t[1].data_ptr(),
        hidden_states=t[2].data_ptr(), hidden_states_scale=t[3].data_ptr(),
        gemm1_weights=t[4].data_ptr(), gemm1_weights_scale=t[5].data_ptr(),
        gemm2_weights=t[6].data_ptr(), gemm2_weights_scale=t[7].data_ptr(),
        local_expert_offset=int(args[8]), routed_scaling_factor=float(args[9]),
        output=out.data_ptr(), num_tokens=int(t[0].shape[0]), bias_dtype=_lib.MI_MOE_DTYPE_BF16,
        reserved=0, workspace=ws, workspace_bytes=nbytes)


def _both(wl):
    """(output of mi_moe_run with a workspace, output of mi_moe_run_noalloc)."""
    L = _lib.lib()
    args = gpu_args(wl)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ref = torch.full((wl.T, H), float("nan"), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(_lib.workspace_size(wl.T), dtype=torch.uint8, device="cuda")
    a = _c_args(args, ref, ws)
    _lib.check(L.mi_moe_run(ctypes.byref(a), stream))
    got = torch.full_like(ref, float("nan"))
    b = _c_args(args, got)
    _lib.check(L.mi_moe_run_noalloc(ctypes.byref(b), stream))
    torch.cuda.synchronize()
    return ref, got


@pytest.mark.parametrize("names", [("t256", "c1_t64"), ("c1_t64", "c1_t16", "c1_t4", "c1_t1")])
def test_noalloc_matches_run_on_calls_in_a_row(names):
    for name in names:
        wl = W.standard(name)
        log(f"test_noalloc_matches_run_on_calls_in_a_row[{name}: T={wl.T}]")
        ref, got = _both(wl)
        assert torch.isfinite(got.float()).all()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), name


def test_noalloc_skewed_shard_and_python_mirror():
    """A skewed shard at the largest accepted T (every token on the same 8
    local experts, 256 rows each), then the Python mirror at T = 16."""
    wl = W.make_workload("noalloc_skew", 256, 77, skew=True, local_expert_offset=32)
    log("test_noalloc_skewed_shard_and_python_mirror: T=256 skew")
    ref, got = _both(wl)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
    wl = W.standard("c0_t16")
    args = gpu_args(wl)
    ref = torch.empty(wl.T, H, dtype=torch.bfloat16, device="cuda")
    kernel.run(*args, ref)
    got = torch.full_like(ref, float("nan"))
    kernel.run_noalloc(*args, got)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))


def test_noalloc_refuses_oversize_without_launch():
    L = _lib.lib()
    wl = W.make_workload("noalloc_big", _lib.MI_MOE_NOALLOC_MAX_TOKENS + 1, 78)
    args = gpu_args(wl)
    out = torch.full((wl.T, H), 7.0, dtype=torch.bfloat16, device="cuda")
    b = _c_args(args, out)
    rc = L.mi_moe_run_noalloc(ctypes.byref(b), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == _lib.MI_MOE_ERR_INVALID
    assert b"MI_MOE_NOALLOC_MAX_TOKENS" in L.mi_moe_last_error()
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())  # nothing was enqueued


_CAPTURE_FIRST_CALL = r"""
import ctypes, sys
sys.path.insert(0, {root!r})
sys.path.insert(0, {tests!r})
import torch
from _helpers import gpu_args
from flashinfer_amd import _lib, kernel
from flashinfer_amd import workloads as W
wl = W.standard("c1_t64")
args = gpu_args(wl)
ref = torch.empty(wl.T, 7168, dtype=torch.bfloat16, device="cuda")
kernel.run(*args, ref)  # loads the library and its kernels (mi_moe_run)
out = torch.full_like(ref, float("nan"))
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    kernel.run_noalloc(*args, out)  # the first mi_moe_run_noalloc call of the process
torch.cuda.synchronize()
ok = []
for rep in range(3):
    out.fill_(float("nan"))
    g.replay()
    torch.cuda.synchronize()
    ok.append(bool(torch.equal(out.view(torch.int16), ref.view(torch.int16))))
    junk = torch.empty_like(ref)
    kernel.run(*args, junk)  # eager work of the program between replays
    torch.cuda.synchronize()
print("REPLAYS", ok, flush=True)
"""


def test_noalloc_first_call_inside_graph_capture():
    """In a fresh process, the first mi_moe_run_noalloc call (which looks up
    the scratch's device address) is made inside a HIP graph capture; every
    replay equals an eager mi_moe_run bit for bit."""
    import os
    import subprocess
    import sys
    log("test_noalloc_first_call_inside_graph_capture (child process)")
    tests = os.path.dirname(os.path.abspath(__file__))
    code = _CAPTURE_FIRST_CALL.format(root=os.path.dirname(tests), tests=tests)
    r = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    assert "REPLAYS [True, True, True]" in r.stdout, (r.stdout, r.stderr[-2000:])
