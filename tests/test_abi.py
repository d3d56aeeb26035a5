"""CPU tests of the C ABI: the library loads, exports every function that
include/mi_moe.h declares, and rejects bad calls before any launch."""
import ctypes
import os
import re

import pytest
import torch

from flashinfer_amd import _lib, kernel

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

# Tests that hand made-up device addresses to real entry points rely on every
# such call being rejected before a launch. They run only where no GPU is
# visible, so a check that a later change relaxes cannot launch a kernel on an
# unmapped address.
cpu_only = pytest.mark.skipif(torch.cuda.is_available(),
                              reason="passes fake device pointers; CPU-only session")


def _declared_functions(header="mi_moe.h", prefix="mi_moe_"):
    src = open(os.path.join(ROOT, "include", header)).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(" + prefix + r"[a-z0-9_]+)\s*\(", src)))


def test_library_exports_every_declared_symbol():
    L = _lib.lib()
    decl = _declared_functions()
    assert decl, "no declarations parsed"
    for name in decl:
        assert hasattr(L, name), f"{name} declared in mi_moe.h but not exported"
    assert set(decl) == set(_lib.EXPORTED)


@cpu_only
def test_peaks_library_exports_every_declared_symbol():
    L = ctypes.CDLL(os.path.join(ROOT, "flashinfer_amd", "libmi_peaks.so"))
    decl = _declared_functions("mi_peaks.h", "mi_peak_")
    assert decl == ["mi_peak_copy", "mi_peak_mfma", "mi_peak_mfma_flops", "mi_peak_read"]
    for name in decl:
        assert hasattr(L, name), f"{name} declared in mi_peaks.h but not exported"
    # argument checks return before any launch
    L.mi_peak_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int32, ctypes.c_void_p,
                               ctypes.c_void_p]
    assert L.mi_peak_read(None, 16, 1024, None, None) == 1
    assert L.mi_peak_read(1 << 20, 15, 1024, 1 << 21, None) == 1
    L.mi_peak_mfma.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
                               ctypes.c_void_p]
    assert L.mi_peak_mfma(2, 10, 512, 1 << 20, None) == 1
    L.mi_peak_mfma_flops.argtypes = [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32]
    L.mi_peak_mfma_flops.restype = ctypes.c_double
    assert L.mi_peak_mfma_flops(0, 10, 512) == 2 * 16 * 16 * 128 * 8 * 4 * 512 * 10


def test_version():
    assert b"gfx950" in _lib.lib().mi_moe_version()


def test_workspace_layout_monotone_and_aligned():
    prev = 0
    for T in (1, 2, 16, 64, 1024, 8192, 14000):
        L = _lib.workspace_layout(T)
        offs = [L.topk_ids, L.topk_w, L.expert_off, L.sorted_tok, L.sorted_w, L.tok_slot,
                L.chunk_cnt, L.act, L.part]
        assert offs == sorted(offs)
        assert all(o % 256 == 0 for o in offs)
        assert L.total == _lib.workspace_size(T) and L.total > prev
        assert L.total - L.part >= 8 * T * 7168 * 2
        prev = L.total


def test_workspace_reserves_fp32_rows_to_1024_and_act_lo_to_256():
    """fp32 partial rows (4 bytes per element) up to T = 1024, bf16 above;
    act_lo (the split activation) only up to T = 256."""
    def sizes(T):
        L = _lib.workspace_layout(T)
        return L.act_lo - L.part, L.total - L.act_lo
    slots = lambda T: 8 * T  # noqa: E731
    for T, part_bytes, lo_bytes in ((256, 4, 2), (257, 4, 0), (1024, 4, 0), (1025, 2, 0)):
        part, lo = sizes(T)
        assert slots(T) * 7168 * part_bytes <= part < slots(T) * 7168 * part_bytes + 256, T
        assert slots(T) * 2048 * lo_bytes <= lo < slots(T) * 2048 * lo_bytes + 256, T


def _args(**over):
    a = _lib.MiMoeArgs()
    ptr = 1 << 20  # 256-byte aligned fake addresses: never dereferenced on these paths
    for f, _ in _lib.MiMoeArgs._fields_:
        if f in ("local_expert_offset", "num_tokens", "bias_dtype", "reserved", "workspace_bytes"):
            continue
        if f == "routed_scaling_factor":
            continue
        setattr(a, f, ptr)
        ptr += 1 << 20
    a.num_tokens = 16
    a.routed_scaling_factor = 2.5
    a.workspace_bytes = 0
    for k, v in over.items():
        setattr(a, k, v)
    return a


def _call(a):
    return _lib.lib().mi_moe_run(ctypes.byref(a), None)


@cpu_only
def test_run_rejects_before_launch():
    L = _lib.lib()
    assert L.mi_moe_run(None, None) == _lib.MI_MOE_ERR_INVALID
    assert _call(_args(num_tokens=-1)) == _lib.MI_MOE_ERR_INVALID
    assert b"num_tokens" in L.mi_moe_last_error()
    assert _call(_args(bias_dtype=7)) == _lib.MI_MOE_ERR_INVALID
    assert _call(_args(reserved=1)) == _lib.MI_MOE_ERR_INVALID
    assert _call(_args(routed_scaling_factor=float("nan"))) == _lib.MI_MOE_ERR_INVALID
    assert _call(_args(gemm2_weights=None)) == _lib.MI_MOE_ERR_INVALID
    assert b"gemm2_weights is NULL" in L.mi_moe_last_error()
    assert _call(_args(hidden_states=(1 << 20) + 4)) == _lib.MI_MOE_ERR_INVALID
    assert b"aligned" in L.mi_moe_last_error()
    assert _call(_args(workspace_bytes=100)) == _lib.MI_MOE_ERR_WORKSPACE
    assert b"workspace" in L.mi_moe_last_error()
    # the largest T whose gathered-row offsets fit the tile GEMMs' 32 bits
    big = _lib.MI_MOE_MAX_TOKENS
    assert _call(_args(num_tokens=big + 1)) == _lib.MI_MOE_ERR_INVALID
    assert b"out of range" in L.mi_moe_last_error()
    lay = _lib.MiMoeLayout()
    assert L.mi_moe_workspace_layout(big, ctypes.byref(lay)) == _lib.MI_MOE_OK
    assert L.mi_moe_workspace_layout(big + 1, ctypes.byref(lay)) == _lib.MI_MOE_ERR_INVALID
    # T == 0 is a valid no-op
    assert _call(_args(num_tokens=0)) == _lib.MI_MOE_OK
    assert L.mi_moe_last_error() == b""


@cpu_only
def test_route_rejects_before_launch():
    L = _lib.lib()
    assert L.mi_moe_route(None, None, 0, -1, 2.5, None, None, None) == _lib.MI_MOE_ERR_INVALID
    assert L.mi_moe_route(None, None, 0, 4, 2.5, None, None, None) == _lib.MI_MOE_ERR_INVALID
    assert L.mi_moe_route(None, None, 5, 4, 2.5, None, None, None) == _lib.MI_MOE_ERR_INVALID
    assert L.mi_moe_route(None, None, 0, 0, 2.5, None, None, None) == _lib.MI_MOE_OK


@cpu_only
def test_run_bf16_rejects_before_launch():
    L = _lib.lib()
    a = _args()
    assert L.mi_moe_run_bf16(ctypes.byref(a), None, None) == _lib.MI_MOE_ERR_INVALID
    assert b"hidden_bf16" in L.mi_moe_last_error()
    assert L.mi_moe_run_bf16(ctypes.byref(a), ctypes.c_void_p((1 << 30) + 8), None) \
        == _lib.MI_MOE_ERR_INVALID
    assert b"aligned" in L.mi_moe_last_error()
    # the checks of mi_moe_run apply as well (workspace_bytes is 0 here)
    assert L.mi_moe_run_bf16(ctypes.byref(a), ctypes.c_void_p(1 << 30), None) \
        == _lib.MI_MOE_ERR_WORKSPACE


@cpu_only
def test_sort_rejects_before_launch():
    L = _lib.lib()
    fake = 1 << 20  # never dereferenced: every check runs before a launch
    ws = _lib.workspace_size(16)
    assert L.mi_moe_sort(None, None, -1, 0, None, 0, None) == _lib.MI_MOE_ERR_INVALID
    assert L.mi_moe_sort(None, None, 1 << 23, 0, None, 0, None) == _lib.MI_MOE_ERR_INVALID
    assert L.mi_moe_sort(None, None, 16, 0, fake, ws, None) == _lib.MI_MOE_ERR_INVALID
    assert L.mi_moe_sort(fake + 4, fake, 16, 0, fake, ws, None) == _lib.MI_MOE_ERR_INVALID
    assert L.mi_moe_sort(fake, fake, 16, 0, fake + 16, ws, None) == _lib.MI_MOE_ERR_INVALID
    assert L.mi_moe_sort(fake, fake, 16, 0, fake, ws - 1, None) == _lib.MI_MOE_ERR_WORKSPACE
    assert "workspace" in L.mi_moe_last_error().decode()
    assert L.mi_moe_sort(None, None, 0, 0, None, 0, None) == _lib.MI_MOE_OK


@cpu_only
def test_quantize_rejects_before_launch():
    L = _lib.lib()
    assert L.mi_moe_quantize_fp8(None, -1, None, None, None) == _lib.MI_MOE_ERR_INVALID
    assert L.mi_moe_quantize_fp8(None, 0, None, None, None) == _lib.MI_MOE_OK
    assert L.mi_moe_quantize_fp8(None, 4, None, None, None) == _lib.MI_MOE_ERR_INVALID
    assert L.mi_moe_quantize_fp8((1 << 20) + 8, 4, 1 << 21, 1 << 22, None) == _lib.MI_MOE_ERR_INVALID
    assert b"misaligned" in L.mi_moe_last_error()


def test_python_wrapper_validates_shapes_and_device():
    T = 4
    good = dict(
        routing_logits=torch.zeros(T, 256), routing_bias=torch.zeros(256, dtype=torch.bfloat16),
        hidden_states=torch.zeros(T, 7168).to(torch.float8_e4m3fn),
        hidden_states_scale=torch.zeros(56, T),
        gemm1_weights=torch.empty(32, 4096, 7168, dtype=torch.float8_e4m3fn),
        gemm1_weights_scale=torch.zeros(32, 32, 56),
        gemm2_weights=torch.empty(32, 7168, 2048, dtype=torch.float8_e4m3fn),
        gemm2_weights_scale=torch.zeros(32, 56, 16),
        local_expert_offset=0, routed_scaling_factor=2.5,
        output=torch.zeros(T, 7168, dtype=torch.bfloat16))
    bad = dict(good, hidden_states_scale=torch.zeros(T, 56))
    with pytest.raises(ValueError, match="hidden_states_scale"):
        kernel.run(**bad)
    bad = dict(good, routing_logits=torch.zeros(T, 256, dtype=torch.float64))
    with pytest.raises(TypeError, match="routing_logits"):
        kernel.run(**bad)
    with pytest.raises(ValueError, match="GPU"):
        kernel.run(**good)


def test_phase_timing_switch(monkeypatch):
    """Timing is on only with FIB_PROFILE_PHASES=1 and an output path, and only
    until the first file is written (kernel.py:30-35 of the reference)."""
    monkeypatch.setattr(kernel, "_PHASE_JSON_WRITTEN", False)
    monkeypatch.delenv("FIB_PROFILE_PHASES", raising=False)
    monkeypatch.delenv("FIB_PHASE_TIMING_OUTPUT", raising=False)
    assert not kernel._phase_json_wanted()
    monkeypatch.setenv("FIB_PROFILE_PHASES", "1")
    assert not kernel._phase_json_wanted()
    monkeypatch.setenv("FIB_PHASE_TIMING_OUTPUT", "/tmp/x.json")
    assert kernel._phase_json_wanted()
    monkeypatch.setenv("FIB_PROFILE_PHASES", "0")
    assert not kernel._phase_json_wanted()
    monkeypatch.setenv("FIB_PROFILE_PHASES", "1")
    monkeypatch.setattr(kernel, "_PHASE_JSON_WRITTEN", True)
    assert not kernel._phase_json_wanted()


@pytest.mark.parametrize("shape", [(7168, 2048), (4096, 1536)])
def test_each_shape_library_reports_shape_and_exports(shape):
    """Every built (H, I) library loads next to the default one, says which
    shape it is, exports the whole declared ABI and sizes its workspace by it."""
    from flashinfer_amd import shapes
    assert shape in shapes.SHAPES and shapes.supported(*shape)
    L = _lib.lib(shape)
    h, i = ctypes.c_int32(), ctypes.c_int32()
    assert L.mi_moe_shape(ctypes.byref(h), ctypes.byref(i)) == _lib.MI_MOE_OK
    assert (h.value, i.value) == shape
    assert f"h{shape[0]} i{shape[1]}" in L.mi_moe_version().decode()
    for name in _declared_functions():
        assert hasattr(L, name), name
    lay = _lib.workspace_layout(100, shape)
    assert lay.part - lay.act >= 800 * shape[1] * 2  # act rows of I bf16 for 8T slots
    assert lay.total - lay.part >= 800 * shape[0] * 2


@pytest.mark.parametrize("defn", __import__("flashinfer_amd.shapes", fromlist=["x"]).DEFINITIONS,
                         ids=lambda d: d.tag)
def test_each_definition_library(defn):
    """Every definition's library reports that definition, exports the whole
    declared ABI, and sizes its workspace by top_k slots per token and its
    local experts."""
    from flashinfer_amd import shapes
    assert shapes.definition_supported(defn)
    L = _lib.lib(defn)
    got = _lib.MiMoeDefinition()
    assert L.mi_moe_get_definition(ctypes.byref(got)) == _lib.MI_MOE_OK
    assert (got.hidden_size, got.intermediate_size, got.num_local_experts, got.num_experts,
            got.n_group, got.topk_group, got.top_k) == (defn.H, defn.I, defn.EL, defn.EG, defn.NG,
                                                        defn.KG, defn.TOPK)
    assert f"e{defn.EL} g{defn.EG} ng{defn.NG} kg{defn.KG} k{defn.TOPK}" in L.mi_moe_version().decode()
    for name in _declared_functions():
        assert hasattr(L, name), name
    T = 100
    lay = _lib.workspace_layout(T, defn)
    assert lay.part - lay.act >= T * defn.TOPK * defn.I * 2      # act rows for top_k*T slots
    assert lay.total - lay.part >= T * defn.TOPK * defn.H * 2
    assert lay.tok_slot - lay.sorted_w >= T * defn.TOPK * 4
    assert lay.expert_off - lay.topk_w >= T * 8 * 4              # top-k rows are 8 wide
    assert lay.sorted_tok - lay.expert_off >= 3 * _lib.meta_stride(defn) * 4
    assert _lib.meta_stride(defn) >= defn.EL + 1
    assert _lib.definition_for(defn.H, defn.I, defn.EL, defn.EG) == defn


def test_definition_registry_rejects_unsupported():
    from flashinfer_amd import shapes
    D = shapes.Definition
    assert not shapes.definition_supported(D(7168, 2048, EL=48))
    assert not shapes.definition_supported(D(7168, 2048, EG=160, NG=8))     # not 64-lane whole
    assert not shapes.definition_supported(D(7168, 2048, EG=256, NG=2))     # 32 lanes per group
    assert shapes.definition_supported(D(7168, 2048, EG=256, NG=4))         # 16 lanes per group
    assert not shapes.definition_supported(D(7168, 2048, TOPK=9))
    assert not shapes.definition_supported(D(7168, 2048, KG=9))
    assert shapes.definition_supported(D(7168, 2048, EG=64, NG=8, KG=2, TOPK=4, EL=16))
    # the shard's gemm1_weights must stay under 2^31 bytes (32-bit signed
    # weight-row offsets in the LDS-tiled GEMMs): 64 x 4096 x 7168 fits,
    # 64 x 2 x 4096 x 8192 does not
    assert shapes.definition_supported(D(7168, 2048, EL=64))
    assert not shapes.definition_supported(D(8192, 4096, EL=64))
    with pytest.raises(ValueError, match="no library"):
        _lib.definition_for(7168, 2048, 16, 64)


def test_unbuilt_shape_is_refused():
    with pytest.raises(ValueError, match="no library"):
        _lib.lib((2048, 768))
    with pytest.raises(ValueError, match="H % 1024"):
        _lib.lib((7000, 2048))


def test_header_constants_match_bindings():
    """The Python mirror's constants are the header's #defines."""
    hdr = open(os.path.join(os.path.dirname(__file__), "..", "include", "mi_moe.h")).read()
    defs = dict(re.findall(r"#define (MI_MOE_[A-Z0-9_]+) (\d+)", hdr))
    for name in ("MI_MOE_OK", "MI_MOE_ERR_INVALID", "MI_MOE_ERR_WORKSPACE", "MI_MOE_ERR_HIP",
                 "MI_MOE_DTYPE_BF16", "MI_MOE_DTYPE_F32", "MI_MOE_MAX_TOKENS",
                 "MI_MOE_NOALLOC_MAX_TOKENS"):
        assert int(defs[name]) == getattr(_lib, name), name


@cpu_only
def test_run_noalloc_rejects_before_launch():
    """The no-allocation entry point refuses a caller workspace and T above its
    static scratch before looking anything up on a device."""
    L = _lib.lib()
    assert L.mi_moe_run_noalloc(None, None) == _lib.MI_MOE_ERR_INVALID
    a = _args(workspace=1 << 30, workspace_bytes=0)
    assert L.mi_moe_run_noalloc(ctypes.byref(a), None) == _lib.MI_MOE_ERR_INVALID
    assert b"workspace must be NULL" in L.mi_moe_last_error()
    a = _args(workspace=None, workspace_bytes=0, num_tokens=_lib.MI_MOE_NOALLOC_MAX_TOKENS + 1)
    assert L.mi_moe_run_noalloc(ctypes.byref(a), None) == _lib.MI_MOE_ERR_INVALID
    assert b"MI_MOE_NOALLOC_MAX_TOKENS" in L.mi_moe_last_error()


def test_native_host_path_module():
    """The native host path is built and loaded, and leaves every case it does
    not handle (here: tensors not on a GPU) to the general path."""
    assert kernel.host_path_loaded()
    H = kernel._HOST
    for name in ("run", "register_definition", "workspace", "cached_workspace"):
        assert callable(getattr(H, name)), name
    assert H.NOT_FAST == -1
    T = 2
    args = [torch.zeros(T, 256), torch.zeros(256, dtype=torch.bfloat16),
            torch.zeros(T, 7168).to(torch.float8_e4m3fn), torch.zeros(56, T),
            torch.empty(32, 4096, 7168, dtype=torch.float8_e4m3fn), torch.zeros(32, 32, 56),
            torch.empty(32, 7168, 2048, dtype=torch.float8_e4m3fn), torch.zeros(32, 56, 16),
            0, 2.5, torch.zeros(T, 7168, dtype=torch.bfloat16)]
    assert H.run(*args) == H.NOT_FAST
    assert H.run(*(["not a tensor"] * 8 + [0, 2.5, "x"])) == H.NOT_FAST


def test_native_host_registration():
    """Registering a definition's library twice is a no-op; another library
    for the same shapes is refused."""
    L = _lib.lib()
    kernel._register_host(_lib.DEFAULT, L)
    kernel._register_host(_lib.DEFAULT, L)
    d = _lib.DEFAULT
    run_addr = ctypes.cast(L.mi_moe_run, ctypes.c_void_p).value
    size_addr = ctypes.cast(L.mi_moe_workspace_size, ctypes.c_void_p).value
    kernel._HOST.register_definition(d.EL, 2 * d.I, d.H, d.EG, run_addr, size_addr)
    with pytest.raises(RuntimeError, match="another library"):
        kernel._HOST.register_definition(d.EL, 2 * d.I, d.H, d.EG, size_addr, size_addr)


def test_oversize_t_raises_before_any_workspace(monkeypatch):
    """T past MI_MOE_MAX_TOKENS is refused by the Python path before a
    workspace is sized or allocated (the native host path hands such calls
    to it): torch.empty tensors of the right shapes, never read."""
    allocated = []
    monkeypatch.setattr(kernel, "_workspace", lambda *a: allocated.append(a))
    T = _lib.MI_MOE_MAX_TOKENS + 1
    e = torch.empty
    args = [e(T, 256), e(256, dtype=torch.bfloat16), e(T, 7168, dtype=torch.float8_e4m3fn),
            e(56, T), e(32, 4096, 7168, dtype=torch.float8_e4m3fn), e(32, 32, 56),
            e(32, 7168, 2048, dtype=torch.float8_e4m3fn), e(32, 56, 16), 0, 2.5,
            e(T, 7168, dtype=torch.bfloat16)]
    with pytest.raises(ValueError, match="MI_MOE_MAX_TOKENS"):
        kernel.run(*args)
    assert allocated == []
