"""The operator at a second (H, I): hidden size 4096, expert intermediate size
1536 (the hidden and MoE-intermediate sizes of a large public MoE model),
from its own library (libmi_moe_h4096_i1536.so). Routing and the 32 local
experts are those of the ds-routing definition family; every kernel family
and the quantiser are checked against the oracle, which takes its shapes from
the tensors."""
import pytest
import torch

from _helpers import log, run_gpu, spread_tokens

from flashinfer_amd import _lib, kernel
from flashinfer_amd import workloads as W

pytestmark = pytest.mark.gpu
SHAPE = (4096, 1536)


def _wl(T, seed, offset=0, skew=False):
    return W.make_workload(f"h4096_i1536_t{T}", T=T, seed=seed, local_expert_offset=offset,
                           skew=skew, H=SHAPE[0], I=SHAPE[1])


def _check(wl, out, tokens):
    from oracle import ref_moe as R
    from _helpers import oracle_subset
    ref = oracle_subset(wl, tokens)
    got = out[tokens.to(out.device)].float().cpu()
    rep = R.tolerance_report(got, ref.acc)
    log(f"output {wl.name}: tokens={len(tokens)} {rep}")
    assert torch.isfinite(got).all()
    assert rep["n_bad"] == 0, rep


def test_library_reports_its_shape():
    h, i = kernel.ctypes.c_int32(), kernel.ctypes.c_int32()
    assert _lib.lib(SHAPE).mi_moe_shape(kernel.ctypes.byref(h), kernel.ctypes.byref(i)) == 0
    assert (h.value, i.value) == SHAPE


# default kernels by T: fused front end, one-wave / workgroup / chunked sort,
# K-split stream (up to T = 256 at this shape, with a sort launch above 64),
# wide and LDS-tiled GEMMs
@pytest.mark.parametrize("T,offset", [(1, 0), (4, 32), (16, 0), (64, 96), (65, 0), (200, 0),
                                      (256, 160), (257, 0), (512, 224), (1024, 64), (2049, 0)])
def test_default_kernels_second_shape(T, offset):
    log(f"test_default_kernels_second_shape[T={T}]")
    wl = _wl(T, 500 + T, offset)
    out = run_gpu(wl, fill=float("nan"))
    _check(wl, out, spread_tokens(T, 64))


# every kernel family forced, including GEMM2 rings deeper than I/128 = 12
# k-blocks allow (variants 8 and 11 fall back to 2 deep)
@pytest.mark.parametrize("variant", ["0", "1", "2", "3", "4", "5,10", "6,6", "7,7", "8,8", "11,11",
                                     "12,12", "9,13", "16,14", "15", "15,3", "19,20", "19,21"])
def test_every_variant_second_shape(variant, monkeypatch):
    log(f"test_every_variant_second_shape[{variant}]")
    monkeypatch.setenv("MI_MOE_VARIANT", variant)
    wl = _wl(96, 777)
    out = run_gpu(wl, fill=float("nan"))
    _check(wl, out, spread_tokens(96, 48))


def test_skew_second_shape():
    """Every token on the same 8 local experts: thousands of rows per expert."""
    log("test_skew_second_shape")
    wl = _wl(3000, 901, skew=True)
    out = run_gpu(wl, fill=float("nan"))
    _check(wl, out, spread_tokens(3000, 24))


def test_quantiser_second_shape():
    from oracle import ref_moe as R
    log("test_quantiser_second_shape")
    g = torch.Generator().manual_seed(3)
    x = (torch.randn(300, SHAPE[0], generator=g) * 3).to(torch.bfloat16)
    q, s = kernel.quantize_activations(x.cuda())
    want_q, want_s = R.quantize_fp8_blocks(x)
    assert s.shape == (SHAPE[0] // 128, 300)
    assert torch.equal(q.view(torch.uint8).cpu(), want_q.view(torch.uint8))
    assert torch.equal(s.cpu(), want_s)
