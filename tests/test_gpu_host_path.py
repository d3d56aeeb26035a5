"""The native host path of ``run`` (the _mi_moe_host extension: checks,
workspace and argument block in C++) against the general Python path: the
same output bit for bit, the same workspace, the same errors, and the cases
it leaves to the general path (a tensor offset, a non-contiguous output,
another stream) still correct."""
import pytest
import torch

from _helpers import gpu_args, log

from flashinfer_amd import _lib, kernel, shapes
from flashinfer_amd import workloads as W

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    if not kernel.host_path_loaded():
        pytest.fail("the native host path (_mi_moe_host) is not built")


def _general_only(*a, **k):
    raise AssertionError("the general path ran")


def _outputs(args, T, H=W.H_DEF):
    return torch.full((T, H), float("nan"), dtype=torch.bfloat16, device="cuda")


@pytest.mark.parametrize("name", ["c1_t1", "c1_t16", "t256"])
def test_native_path_matches_general_path(name, monkeypatch):
    log(f"test_native_path_matches_general_path[{name}]")
    wl = W.standard(name)
    args = gpu_args(wl)
    ref = _outputs(args, wl.T)
    with monkeypatch.context() as m:
        m.setattr(kernel, "_HOST", None)
        kernel.run(*args, ref)
    kernel.run(*args, _outputs(args, wl.T))  # registers the definition
    out = _outputs(args, wl.T)
    with monkeypatch.context() as m:
        m.setattr(kernel, "_call", _general_only)
        kernel.run(*args, out)
        out2 = _outputs(args, wl.T)
        kernel.run(*args, out2)  # the cached workspace
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(out2.view(torch.int16), ref.view(torch.int16))
    ws = kernel.last_workspace()
    assert ws.numel() >= _lib.workspace_size(wl.T)


def test_native_path_leaves_other_cases_to_general_path():
    log("test_native_path_leaves_other_cases_to_general_path")
    wl = W.standard("c1_t16")
    args = gpu_args(wl)
    ref = _outputs(args, wl.T)
    kernel.run(*args, ref)
    # a 0-d tensor offset and scaling factor
    out = _outputs(args, wl.T)
    a = list(args)
    a[8] = torch.tensor(wl.local_expert_offset)
    a[9] = torch.tensor(wl.routed_scaling_factor)
    kernel.run(*a, out)
    # a non-contiguous output and a non-contiguous hidden_states_scale
    big = torch.full((wl.T, 2 * W.H_DEF), float("nan"), dtype=torch.bfloat16, device="cuda")
    a = list(args)
    a[3] = args[3].t().contiguous().t()
    kernel.run(*a, big[:, ::2])
    # another stream
    s = torch.cuda.Stream()
    out3 = _outputs(args, wl.T)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        kernel.run(*args, out3)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for o in (out, big[:, ::2], out3):
        assert torch.equal(o.contiguous().view(torch.int16), ref.view(torch.int16))


def test_native_path_errors_unchanged():
    log("test_native_path_errors_unchanged")
    wl = W.standard("c1_t4")
    args = gpu_args(wl)
    out = _outputs(args, wl.T)
    kernel.run(*args, out)
    bad = list(args)
    bad[0] = args[0].double()
    with pytest.raises(TypeError, match="routing_logits"):
        kernel.run(*bad, out)
    bad = list(args)
    bad[3] = args[3].t()
    with pytest.raises(ValueError, match="hidden_states_scale"):
        kernel.run(*bad, out)
    with pytest.raises(ValueError, match="output"):
        kernel.run(*args, out[:, :1024])
    with pytest.raises(ValueError, match="same device"):
        a = list(args)
        a[1] = args[1].cpu()
        kernel.run(*a, out)


def test_native_path_reports_library_errors():
    """A call the library refuses (routing_logits not 16-byte aligned) raises
    the library's message from the native path too, before any launch."""
    log("test_native_path_reports_library_errors")
    wl = W.standard("c1_t4")
    args = gpu_args(wl)
    out = _outputs(args, wl.T)
    kernel.run(*args, out)
    buf = torch.empty(args[0].numel() + 1, dtype=torch.float32, device="cuda")
    lg = buf[1:].view_as(args[0])
    lg.copy_(args[0])
    a = list(args)
    a[0] = lg
    assert kernel._HOST.run(*a, out) not in (0, kernel._NOT_FAST)
    with pytest.raises(_lib.MiMoeError, match="aligned"):
        kernel.run(*a, out)


@pytest.mark.parametrize("defn", [d for d in shapes.DEFINITIONS if d != shapes.DEFAULT],
                         ids=lambda d: d.tag)
def test_native_path_other_definitions_and_fp32_bias(defn, monkeypatch):
    """Each definition's library is registered for its own shapes; fp32
    routing bias takes the native path too; outputs equal the Python path's."""
    log(f"test_native_path_other_definitions_and_fp32_bias[{defn.tag}]")
    wl = W.make_for(defn, f"{defn.tag}_host", 24, 7300, local_expert_offset=0)
    args = gpu_args(wl)
    args[1] = args[1].float()
    ref = _outputs(args, wl.T, defn.H)
    with monkeypatch.context() as m:
        m.setattr(kernel, "_HOST", None)
        kernel.run(*args, ref)
    kernel.run(*args, _outputs(args, wl.T, defn.H))  # registers the definition
    out = _outputs(args, wl.T, defn.H)
    with monkeypatch.context() as m:
        m.setattr(kernel, "_call", _general_only)
        kernel.run(*args, out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
