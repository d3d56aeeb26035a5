"""GPU parity of the FP8 activation quantiser (mi_moe_quantize_fp8) against
the oracle: fp8 bytes and fp32 scales bit-exact, including ties, subnormal
results, all-zero blocks, signed zeros and huge magnitudes."""
import pytest
import torch

from _helpers import log

from flashinfer_amd import workloads as W
from oracle import ref_moe as R

pytestmark = pytest.mark.gpu
H = 7168


def _random_hidden(T, seed):
    g = torch.Generator().manual_seed(seed)
    # per-block magnitudes spread over 12 decades so every exponent range is hit
    mag = torch.logspace(-6, 6, H // 128)[torch.randperm(H // 128, generator=g)]
    x = torch.randn(T, H, generator=g) * mag.repeat_interleave(128)
    return x.to(torch.bfloat16)


def _check(x):
    from flashinfer_amd import kernel
    q, s = kernel.quantize_activations(x.cuda())
    torch.cuda.synchronize()
    q_ref, s_ref = R.quantize_fp8_blocks(x)
    qb, qr = q.cpu().view(torch.uint8), q_ref.view(torch.uint8)
    sb, sr = s.cpu().view(torch.int32), s_ref.view(torch.int32)
    n_q = int((qb != qr).sum())
    n_s = int((sb != sr).sum())
    log(f"quant T={x.shape[0]}: fp8 byte mismatches {n_q}, scale mismatches {n_s}")
    if n_q:
        i = (qb != qr).nonzero()[0].tolist()
        log(f"  first at {i}: x={float(x[i[0], i[1]])} gpu={int(qb[i[0], i[1]]):#04x} "
            f"ref={int(qr[i[0], i[1]]):#04x} scale={float(s_ref[i[1] // 128, i[0]])}")
    assert n_s == 0 and n_q == 0


@pytest.mark.parametrize("T,seed", [(1, 1), (3, 2), (64, 3), (1000, 4), (8192, 5)])
def test_quantize_bit_exact(T, seed):
    log(f"test_quantize_bit_exact[T={T}]")
    _check(_random_hidden(T, seed))


def test_quantize_edge_blocks():
    log("test_quantize_edge_blocks")
    T = 6
    x = torch.zeros(T, H)
    # token 0: exact midpoints between e4m3 neighbours once divided by the scale
    # (block max 448 -> scale 1): 0.5*(a+b) for a run of codes, both signs
    codes = torch.arange(0, 126, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    mids = 0.5 * (codes[:-1] + codes[1:])
    x[0, :125] = mids
    x[0, 125:250] = -mids
    x[0, 127] = 448.0  # block 0 max
    x[0, 255] = -448.0  # block 1 max
    # token 1: all-zero row apart from one tiny block; token 2: signed zeros
    x[1, 300] = 1e-30
    x[2, :] = -0.0
    # token 3: huge magnitudes near the bf16 range limit
    x[3] = torch.linspace(-3e38, 3e38, H, dtype=torch.float64).float()  # fp32 step would overflow
    # token 4: values whose quotient lands in the fp8 subnormal range
    x[4, :128] = torch.linspace(0, 1, 128) * 2 ** -8
    x[4, 0] = 448.0
    # token 5: a random row
    x[5] = torch.randn(H, generator=torch.Generator().manual_seed(9))
    _check(x.to(torch.bfloat16))


def test_quantize_then_run_matches_oracle():
    """End to end: bf16 activations -> quantiser -> fused MoE, against the
    oracle fed by its own quantisation of the same activations."""
    from _helpers import device_weights
    from flashinfer_amd import kernel
    log("test_quantize_then_run_matches_oracle")
    wl = W.standard("c0_t16")
    T = wl.T
    x = _random_hidden(T, 11)
    q, s = kernel.quantize_activations(x.cuda())
    dw = device_weights()
    t = wl.tensors
    out = torch.empty(T, H, dtype=torch.bfloat16, device="cuda")
    kernel.run(t["routing_logits"].cuda(), t["routing_bias"].cuda(), q, s, dw["gemm1_weights"],
               dw["gemm1_weights_scale"], dw["gemm2_weights"], dw["gemm2_weights_scale"],
               wl.local_expert_offset, wl.routed_scaling_factor, out)
    torch.cuda.synchronize()
    q_ref, s_ref = R.quantize_fp8_blocks(x)
    ref = R.moe_forward(t["routing_logits"], t["routing_bias"], q_ref, s_ref, t["gemm1_weights"],
                        t["gemm1_weights_scale"], t["gemm2_weights"], t["gemm2_weights_scale"],
                        wl.local_expert_offset, wl.routed_scaling_factor)
    rep = R.tolerance_report(out.float().cpu(), ref.acc)
    log(f"quantise+run T={T}: {rep}")
    assert rep["n_bad"] == 0, rep


def test_quantize_rejects_bad_arguments():
    from flashinfer_amd import kernel
    with pytest.raises(TypeError):
        kernel.quantize_activations(torch.zeros(2, H, device="cuda"))  # fp32, not bf16
    with pytest.raises(ValueError):
        kernel.quantize_activations(torch.zeros(2, 100, dtype=torch.bfloat16, device="cuda"))
    q, s = kernel.quantize_activations(torch.zeros(0, H, dtype=torch.bfloat16, device="cuda"))
    assert q.shape == (0, H) and s.shape == (H // 128, 0)


@pytest.mark.parametrize("T", [1, 4, 16, 64, 100, 200, 300, 1500])
def test_run_bf16_matches_quantize_then_run(T):
    """run_bf16 (quantiser and routing in one launch, then the layer) writes
    the fp8 pair of quantize_activations and the output of run on it, bit for
    bit, through each front end (T=1..64 sort in the stream GEMM1, 100 and
    200 in the wide GEMM1, 300 sort kernel, 1500 chunked sort)."""
    from flashinfer_amd import kernel
    from _helpers import gpu_args
    log(f"test_run_bf16_matches_quantize_then_run[T={T}]")
    wl = W.make_workload("run_bf16", T, 700 + T, local_expert_offset=32 * (T % 3))
    g = torch.Generator().manual_seed(T)
    x = (torch.randn(T, H, generator=g) * 0.5).to(torch.bfloat16).cuda()
    args = gpu_args(wl)
    q, s = kernel.quantize_activations(x)
    args[2], args[3] = q, s
    ref = torch.full((T, H), float("nan"), dtype=torch.bfloat16, device="cuda")
    kernel.run(*args, ref)
    out = torch.full_like(ref, float("nan"))
    rest = args[:2] + args[4:]
    q2, s2 = kernel.run_bf16(rest[0], rest[1], x, *rest[2:], out)
    torch.cuda.synchronize()
    assert torch.equal(q2.view(torch.uint8), q.view(torch.uint8))
    assert torch.equal(s2, s)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
