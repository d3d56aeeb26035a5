"""ctypes binding of libmi_moe.so (the C ABI in include/mi_moe.h), and of
the libraries built for other layer definitions (``shapes.py``: hidden and
intermediate size, local experts, routing parameters), one per definition.

The library is loaded after ``import torch`` so that its ``libamdhip64.so.7``
dependency binds to the HIP runtime torch already loaded (same SONAME):
stream handles and device pointers from torch are then valid inside it.
There is no fallback: if the library is missing the import of the operator
raises with the command that builds it.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

from . import shapes

HERE = os.path.dirname(os.path.abspath(__file__))
DEFAULT_SHAPE = shapes.DEFAULT_SHAPE
DEFAULT = shapes.DEFAULT

MI_MOE_OK = 0
MI_MOE_ERR_INVALID = 1
MI_MOE_ERR_WORKSPACE = 2
MI_MOE_ERR_HIP = 3
MI_MOE_DTYPE_BF16 = 0
MI_MOE_DTYPE_F32 = 1
MI_MOE_MAX_TOKENS = 131072  # largest num_tokens the library accepts
MI_MOE_NOALLOC_MAX_TOKENS = 256  # largest num_tokens of mi_moe_run_noalloc

EXPORTED = ("mi_moe_workspace_size", "mi_moe_workspace_layout", "mi_moe_run",
            "mi_moe_run_profiled", "mi_moe_run_bf16", "mi_moe_run_noalloc", "mi_moe_route",
            "mi_moe_sort", "mi_moe_quantize_fp8", "mi_moe_shape", "mi_moe_get_definition",
            "mi_moe_last_error", "mi_moe_version")
NUM_PHASES = 5
PHASES = ("route", "sort", "gemm1_swiglu", "gemm2", "combine")


class MiMoeArgs(ctypes.Structure):
    _fields_ = [
        ("routing_logits", ctypes.c_void_p),
        ("routing_bias", ctypes.c_void_p),
        ("hidden_states", ctypes.c_void_p),
        ("hidden_states_scale", ctypes.c_void_p),
        ("gemm1_weights", ctypes.c_void_p),
        ("gemm1_weights_scale", ctypes.c_void_p),
        ("gemm2_weights", ctypes.c_void_p),
        ("gemm2_weights_scale", ctypes.c_void_p),
        ("local_expert_offset", ctypes.c_int64),
        ("routed_scaling_factor", ctypes.c_float),
        ("output", ctypes.c_void_p),
        ("num_tokens", ctypes.c_int64),
        ("bias_dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
    ]


class MiMoeDefinition(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("hidden_size", "intermediate_size", "num_local_experts", "num_experts", "n_group",
                 "topk_group", "top_k")]


class MiMoeLayout(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in
                ("topk_ids", "topk_w", "expert_off", "sorted_tok", "sorted_w", "tok_slot",
                 "chunk_cnt", "act", "part", "act_lo", "total")]


_libs: dict = {}
_lock = threading.Lock()


class MiMoeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"mi_moe error {code}: {msg}")
        self.code = code


def _bind(L: ctypes.CDLL) -> None:
    L.mi_moe_workspace_size.argtypes = [ctypes.c_int64]
    L.mi_moe_workspace_size.restype = ctypes.c_size_t
    L.mi_moe_workspace_layout.argtypes = [ctypes.c_int64, ctypes.POINTER(MiMoeLayout)]
    L.mi_moe_workspace_layout.restype = ctypes.c_int
    L.mi_moe_run.argtypes = [ctypes.POINTER(MiMoeArgs), ctypes.c_void_p]
    L.mi_moe_run.restype = ctypes.c_int
    L.mi_moe_run_noalloc.argtypes = [ctypes.POINTER(MiMoeArgs), ctypes.c_void_p]
    L.mi_moe_run_noalloc.restype = ctypes.c_int
    L.mi_moe_run_bf16.argtypes = [ctypes.POINTER(MiMoeArgs), ctypes.c_void_p, ctypes.c_void_p]
    L.mi_moe_run_bf16.restype = ctypes.c_int
    L.mi_moe_run_profiled.argtypes = [ctypes.POINTER(MiMoeArgs), ctypes.c_void_p,
                                      ctypes.POINTER(ctypes.c_void_p), ctypes.c_int32]
    L.mi_moe_run_profiled.restype = ctypes.c_int
    L.mi_moe_route.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                               ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    L.mi_moe_route.restype = ctypes.c_int
    L.mi_moe_sort.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64,
                              ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    L.mi_moe_sort.restype = ctypes.c_int
    L.mi_moe_quantize_fp8.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p]
    L.mi_moe_quantize_fp8.restype = ctypes.c_int
    L.mi_moe_last_error.argtypes = []
    L.mi_moe_last_error.restype = ctypes.c_char_p
    L.mi_moe_version.argtypes = []
    L.mi_moe_version.restype = ctypes.c_char_p
    L.mi_moe_shape.argtypes = [ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]
    L.mi_moe_shape.restype = ctypes.c_int
    L.mi_moe_get_definition.argtypes = [ctypes.POINTER(MiMoeDefinition)]
    L.mi_moe_get_definition.restype = ctypes.c_int


def lib_path(defn=DEFAULT) -> str:
    d = shapes.as_definition(defn)
    return os.path.join(HERE, shapes.lib_name_of(d))


def built_definitions() -> list:
    """Every definition whose library is present next to this file."""
    return [d for d in shapes.DEFINITIONS if os.path.exists(lib_path(d))]


def built_shapes() -> list:
    """(H, I) of every library present with the default routing and 32 local experts."""
    return [(d.H, d.I) for d in built_definitions() if d.default_routing]


_DEF_FOR: dict = {}


def definition_for(H: int, I: int, EL: int, EG: int):
    """The built definition with hidden size H, intermediate size I, EL local
    and EG global experts (tensor shapes fix these; the routing parameters
    follow from the definition). Looked up once per key: the call path of
    ``run`` stats no files."""
    key = (H, I, EL, EG)
    d = _DEF_FOR.get(key)
    if d is not None:
        return d
    found = [d for d in built_definitions() if (d.H, d.I, d.EL, d.EG) == key]
    if len(found) == 1:
        _DEF_FOR[key] = found[0]
        return found[0]
    if not found:
        d = shapes.Definition(H, I, EL, EG)
        hint = ("add it to DEFINITIONS in flashinfer_amd/shapes.py and rebuild"
                if shapes.supported(H, I) else "supported shapes have H % 1024 == 0 and I % 256 == 0")
        raise ValueError(f"no library for hidden size {H}, intermediate size {I}, {EL} local of "
                         f"{EG} experts (built: {[x.name for x in built_definitions()]}); {hint}"
                         if d not in shapes.DEFINITIONS else
                         f"{lib_path(d)} is missing: build it with `python -m flashinfer_amd.build`")
    raise ValueError(f"several built definitions match H={H}, I={I}, {EL} of {EG} experts: "
                     f"{[x.name for x in found]}")


def lib(defn=DEFAULT) -> ctypes.CDLL:
    """The library compiled for ``defn`` (a shapes.Definition, or an (H, I)
    pair meaning the default routing), loaded once."""
    d = shapes.as_definition(defn)
    L = _libs.get(d)
    if L is not None:
        return L
    with _lock:
        if d in _libs:
            return _libs[d]
        path = lib_path(d)
        if not os.path.exists(path):
            if d == DEFAULT:
                raise RuntimeError(
                    f"{path} is missing: build it with `python -m flashinfer_amd.build` "
                    "(hipcc, gfx950). There is no non-native fallback.")
            if d in shapes.DEFINITIONS:
                raise ValueError(f"{path} is missing: build it with `python -m flashinfer_amd.build`")
            hint = ("add it to DEFINITIONS in flashinfer_amd/shapes.py and rebuild"
                    if shapes.supported(d.H, d.I) else
                    "supported shapes have H % 1024 == 0 and I % 256 == 0")
            raise ValueError(f"no library for hidden size {d.H} and intermediate size {d.I} "
                             f"(built: {built_shapes()}); {hint}")
        L = ctypes.CDLL(path)
        _bind(L)
        got = MiMoeDefinition()
        if L.mi_moe_get_definition(ctypes.byref(got)) != MI_MOE_OK:
            raise RuntimeError(f"{path}: mi_moe_get_definition failed")
        have = shapes.Definition(got.hidden_size, got.intermediate_size, got.num_local_experts,
                                 got.num_experts, got.n_group, got.topk_group, got.top_k)
        if have != d:
            raise RuntimeError(f"{path} reports {have}, expected {d}")
        _libs[d] = L
        return L


def check(code: int, L: ctypes.CDLL | None = None) -> None:
    """Raise with the library's message (each library keeps its own) on error."""
    if code != MI_MOE_OK:
        msg = (L or lib()).mi_moe_last_error().decode("utf-8", "replace")
        raise MiMoeError(code, msg)


def workspace_size(num_tokens: int, defn=DEFAULT) -> int:
    return int(lib(defn).mi_moe_workspace_size(int(num_tokens)))


def workspace_layout(num_tokens: int, defn=DEFAULT) -> MiMoeLayout:
    out = MiMoeLayout()
    L = lib(defn)
    check(L.mi_moe_workspace_layout(int(num_tokens), ctypes.byref(out)), L)
    return out


def meta_stride(defn=DEFAULT) -> int:
    """Int offset between the expert-offset table and each row-tile prefix
    table at the start of the workspace's meta region."""
    return 64 if shapes.as_definition(defn).EL < 64 else 128
