"""Pins the CPU oracle (oracle/ref_moe.py) against known answers, invariants
and brute force, so that a plausible mistake in it fails here."""
import math

import pytest
import torch

from oracle import ref_moe as R
from flashinfer_amd import workloads as W

E, G, KG, K = 256, 8, 4, 8


def _route(logits, bias, rsf=2.5):
    return R.route(logits, bias, rsf, G, KG, K)


def test_route_group_score_is_top2_sum_not_top1():
    # Group 7 holds the single best expert, but groups 0-3 each hold two good
    # experts: top1+top2 must prefer groups 0-3; a top-1 group score would pick 7.
    logits = torch.full((1, E), -10.0)
    logits[0, 7 * 32 + 5] = 10.0
    good = []
    for g in range(4):
        for j in (3, 17):
            logits[0, g * 32 + j] = 3.0
            good.append(g * 32 + j)
    for g in (4, 5, 6):
        for j in (1, 2):
            logits[0, g * 32 + j] = 2.0
    r = _route(logits, torch.zeros(E))
    assert sorted(r.ids[0].tolist()) == sorted(good)
    assert 7 * 32 + 5 not in r.ids[0].tolist()


def test_route_bias_selects_but_does_not_weight():
    logits = torch.full((1, E), -5.0)
    logits[0, :8] = torch.arange(8) * 0.1
    bias = torch.zeros(E)
    bias[:8] = 1.0
    rsf = 2.5
    r = _route(logits, bias, rsf)
    assert sorted(r.ids[0].tolist()) == list(range(8))
    s = torch.sigmoid(logits[0, :8].double())
    want = (s * rsf / s.sum()).float()
    got = torch.zeros(8)
    for k in range(8):
        got[r.ids[0, k]] = r.weights[0, k]
    assert torch.allclose(got, want, rtol=1e-6, atol=0)
    # a weight computed from s+bias would be (s+1)*rsf/sum(s+1): clearly different
    wrong = ((s + 1) * rsf / (s + 1).sum()).float()
    assert not torch.allclose(got, wrong, rtol=1e-3)


def test_route_order_and_lowest_index_tie_break():
    # Equal scores everywhere: groups 0-3 and experts 0..7 of group 0 (lowest ids).
    logits = torch.zeros(1, E)
    r = _route(logits, torch.zeros(E))
    assert r.ids[0].tolist() == list(range(8))
    assert torch.allclose(r.weights[0], torch.full((8,), 2.5 / 8))


def test_route_skew_known_answer():
    tok = W.make_tokens(64, seed=7, skew=True, local_expert_offset=96)
    r = _route(tok["routing_logits"], tok["routing_bias"])
    for t in range(64):
        assert sorted(r.ids[t].tolist()) == list(range(96, 104))
    s = r.scores.gather(1, r.ids).double()
    want = s * 2.5 / s.sum(1, keepdim=True)
    assert torch.allclose(r.weights.double(), want, rtol=1e-6)


def _brute_route(logits, bias, rsf, n_group=None, topk_group=None, top_k=None):
    """Pure-Python selection on the same fp32 sigmoid values."""
    n_group, topk_group, top_k = n_group or G, topk_group or KG, top_k or K
    n_exp = logits.shape[1]
    gsize = n_exp // n_group
    s = torch.sigmoid(logits.float())
    sb = (s + bias.float()[None, :])
    out_ids, out_w = [], []
    for t in range(logits.shape[0]):
        row = sb[t].tolist()
        gscore = []
        for g in range(n_group):
            vals = sorted(row[g * gsize:(g + 1) * gsize], reverse=True)
            gscore.append(torch.tensor(vals[0], dtype=torch.float32) + torch.tensor(vals[1], dtype=torch.float32))
        groups = sorted(range(n_group), key=lambda g: (-float(gscore[g]), g))[:topk_group]
        cand = [e for e in range(n_exp) if e // gsize in groups]
        ids = sorted(cand, key=lambda e: (-row[e], e))[:top_k]
        out_ids.append(ids)
    return out_ids


@pytest.mark.parametrize("n_exp,n_group,topk_group,top_k", [(128, 8, 3, 6), (256, 4, 2, 8),
                                                            (64, 8, 4, 4)])
def test_route_other_definitions_brute_force(n_exp, n_group, topk_group, top_k):
    """The routing restatement for other definitions of the family (the
    reference's constexpr E_GLOBAL / N_GROUP / TOPK_GROUP / TOP_K,
    kernel.py:371-389) against the pure-Python selection, plus its
    invariants: top_k distinct ids from at most topk_group groups, weights
    summing to the scaling factor."""
    tok = W.make_tokens(80, seed=11, E_global=n_exp)
    logits, bias = tok["routing_logits"], tok["routing_bias"]
    r = R.route(logits, bias, 2.5, n_group, topk_group, top_k)
    brute = _brute_route(logits, bias, 2.5, n_group, topk_group, top_k)
    assert [sorted(x) for x in r.ids.tolist()] == [sorted(x) for x in brute]
    gsize = n_exp // n_group
    for t in range(80):
        ids = r.ids[t].tolist()
        assert len(set(ids)) == top_k
        assert len({i // gsize for i in ids}) <= topk_group
        assert abs(float(r.weights[t].sum()) - 2.5) < 1e-5


def test_route_brute_force_and_invariants():
    tok = W.make_tokens(96, seed=3)
    logits, bias = tok["routing_logits"], tok["routing_bias"]
    r = _route(logits, bias, 2.5)
    brute = _brute_route(logits, bias, 2.5)
    assert [sorted(x) for x in r.ids.tolist()] == [sorted(x) for x in brute]
    sb = r.scores + bias.float()[None, :]
    for t in range(96):
        ids = r.ids[t].tolist()
        assert len(set(ids)) == 8
        groups = {i // 32 for i in ids}
        assert len(groups) <= 4
        assert abs(float(r.weights[t].sum()) - 2.5) < 1e-5
        # selection order: descending s+bias
        v = sb[t, r.ids[t]]
        assert bool((v[:-1] >= v[1:]).all())


def test_dequant_layouts_one_hot():
    # hidden_states_scale is [H/128, T] (block-major); weights scale [R/128, C/128].
    T, H = 3, 384
    hs = torch.ones(T, H).to(W.FP8)
    sc = torch.ones(H // 128, T)
    sc[1, 0] = 7.0
    a = R.dequant_activations(hs, sc)
    assert torch.all(a[0, 128:256] == 7.0) and torch.all(a[0, :128] == 1.0)
    assert torch.all(a[1:] == 1.0)
    w = torch.ones(256, 384).to(W.FP8)
    ws = torch.ones(2, 3)
    ws[1, 2] = 5.0  # rows 128..255, cols 256..383
    wf = R.dequant_blocks(w, ws)
    assert torch.all(wf[128:, 256:] == 5.0)
    assert float(wf.sum()) == 256 * 384 + 4.0 * 128 * 128


def test_dequant_elementwise_brute_force():
    g = torch.Generator().manual_seed(1)
    T, H = 2, 256
    hs = torch.randn(T, H, generator=g).to(W.FP8)
    sc = torch.rand(H // 128, T, generator=g) + 0.5
    a = R.dequant_activations(hs, sc, torch.float64)
    for t in range(T):
        for k in range(0, H, 37):
            assert a[t, k] == float(hs[t, k].float()) * float(sc[k // 128, t])


def test_swiglu_halves():
    g = torch.tensor([[2.0, 2.0, 3.0, 3.0]])
    out = R.swiglu(g)
    want = 3.0 / (1 + math.exp(-3.0)) * 2.0
    assert torch.allclose(out, torch.full((1, 2), want))
    swapped = 2.0 / (1 + math.exp(-2.0)) * 3.0
    assert abs(want - swapped) > 0.1


def _tiny_expert(gen, H=256, I=128):
    w1 = torch.randn(2 * I, H, generator=gen).to(W.FP8)
    w1s = torch.rand(2 * I // 128, H // 128, generator=gen) * 0.01 + 0.001
    w2 = torch.randn(H, I, generator=gen).to(W.FP8)
    w2s = torch.rand(H // 128, I // 128, generator=gen) * 0.01 + 0.001
    return w1, w1s, w2, w2s


def test_expert_forward_brute_force_fp64():
    gen = torch.Generator().manual_seed(5)
    H, I, M = 256, 128, 2
    w1, w1s, w2, w2s = _tiny_expert(gen, H, I)
    a = torch.randn(M, H, generator=gen, dtype=torch.float64)
    out = R.expert_forward(a, w1, w1s, w2, w2s, torch.float64)
    w1f = w1.double().tolist()
    w2f = w2.double().tolist()
    for m in range(M):
        g = []
        for n in range(2 * I):
            acc = 0.0
            for k in range(H):
                acc += float(a[m, k]) * w1f[n][k] * float(w1s[n // 128, k // 128])
            g.append(acc)
        x = [g[I + j] / (1 + math.exp(-g[I + j])) * g[j] for j in range(I)]
        for n in range(0, H, 11):
            acc = 0.0
            for k in range(I):
                acc += x[k] * w2f[n][k] * float(w2s[n // 128, k // 128])
            assert abs(acc - float(out[m, n])) <= 1e-9 * (abs(acc) + 1e-12) + 1e-15


def _tiny_workload(T=24, seed=11, off=0, skew=False):
    return W.make_workload("tiny", T=T, seed=seed, local_expert_offset=off, skew=skew,
                           H=256, I=128, weight_seed=99)


def test_moe_combine_per_token_brute_force():
    wl = _tiny_workload(T=24, seed=11, off=64)
    args = wl.args()
    res = R.moe_forward(*args, acc_dtype=torch.float64)
    t = wl.tensors
    a = R.dequant_activations(t["hidden_states"], t["hidden_states_scale"], torch.float64)
    r = res.route
    for tok in range(24):
        acc = torch.zeros(256, dtype=torch.float64)
        for k in range(8):
            e = int(r.ids[tok, k]) - 64
            if 0 <= e < 32:
                o = R.expert_forward(a[tok:tok + 1], t["gemm1_weights"][e], t["gemm1_weights_scale"][e],
                                     t["gemm2_weights"][e], t["gemm2_weights_scale"][e], torch.float64)
                acc += float(r.weights[tok, k]) * o[0]
        assert torch.allclose(acc, res.acc[tok], rtol=1e-9, atol=1e-15)
    # at least some tokens routed locally and some not, so both branches ran
    n_local = sum(len(tk) for tk, _ in res.slots)
    assert n_local > 0


def test_moe_linearity():
    wl = _tiny_workload(T=16, seed=12)
    args = wl.args()
    base = R.moe_forward(*args, acc_dtype=torch.float64).acc
    args2 = list(args)
    args2[9] = 2 * args[9]
    assert torch.allclose(R.moe_forward(*args2, acc_dtype=torch.float64).acc, 2 * base, rtol=1e-12, atol=0)
    args3 = list(args)
    args3[7] = args[7] * 2
    assert torch.allclose(R.moe_forward(*args3, acc_dtype=torch.float64).acc, 2 * base, rtol=1e-12, atol=0)


def test_moe_dequant_all_experts_schedule_same_result():
    """The definition-style schedule (every expert's weights dequantised
    before routing, as the bench's full-dequant CPU baseline runs it) gives
    the same output; the per-token brute force above pins both."""
    wl = _tiny_workload(T=24, seed=15, off=0)
    a = R.moe_forward(*wl.args(), acc_dtype=torch.float64)
    b = R.moe_forward(*wl.args(), acc_dtype=torch.float64, dequant_all_experts=True)
    assert sum(len(tk) for tk, _ in a.slots) > 0
    assert torch.allclose(a.acc, b.acc, rtol=1e-12, atol=1e-18)
    assert torch.equal(a.output, b.output)


def test_moe_empty_routing_is_zero():
    wl = _tiny_workload(T=8, seed=13, off=256)  # no expert is local
    res = R.moe_forward(*wl.args())
    assert res.output.dtype == torch.bfloat16
    assert torch.count_nonzero(res.output) == 0


def test_skew_all_slots_on_biased_experts():
    wl = _tiny_workload(T=32, seed=14, off=0, skew=True)
    res = R.moe_forward(*wl.args())
    counts = [len(tk) for tk, _ in res.slots]
    assert counts[:8] == [32] * 8 and sum(counts[8:]) == 0


def test_tolerance_report_flags_planted_error():
    ref = torch.randn(4, 64, generator=torch.Generator().manual_seed(0))
    out = ref.clone()
    assert R.tolerance_report(out, ref)["n_bad"] == 0
    out[1, 3] += 0.5 * float(ref.abs().max())
    assert R.tolerance_report(out, ref)["n_bad"] == 1


def test_algorithmic_counts():
    assert R.algorithmic_bytes(0, 32) - 512 == 1_409_630_208
    assert R.algorithmic_flops(1) == 88_080_384


# ---------------------------------------------------------------- quantiser


def _e4m3fn_value(code: int) -> float:
    """Decode one e4m3fn byte (bias 7, subnormals, no infinities)."""
    sign = -1.0 if code & 0x80 else 1.0
    exp, man = (code >> 3) & 15, code & 7
    if exp == 15 and man == 7:
        return math.nan
    if exp == 0:
        return sign * man * 2.0 ** -9
    return sign * (1 + man / 8) * 2.0 ** (exp - 7)


def _e4m3fn_rne(v: float) -> int:
    """Nearest finite e4m3fn code to v, ties to the even code (|v| <= 448)."""
    best = None
    for code in range(256):
        c = _e4m3fn_value(code)
        if math.isnan(c) or (code == 0x80 and v >= 0) or (code == 0 and v < 0 and math.copysign(1, v) < 0):
            continue
        d = abs(v - c)
        key = (d, code & 1)
        if best is None or key < best[0]:
            best = (key, code)
    return best[1]


def test_e4m3fn_rounding_matches_brute_force():
    # every adjacent pair's midpoint (exact ties), points just off the
    # midpoints, and random values across the whole range
    vals = [_e4m3fn_value(c) for c in range(0x7F)]  # non-negative finite codes, ascending
    pts = []
    for a, b in zip(vals, vals[1:]):
        m = (a + b) / 2
        pts += [m, -m, m * (1 + 2 ** -20), m * (1 - 2 ** -20), a, -b]
    g = torch.Generator().manual_seed(5)
    pts += (torch.randn(2000, generator=g) * 40).clamp(-448, 448).tolist()
    pts += (torch.rand(500, generator=g) * 2 ** -6).tolist()  # subnormal range
    x = torch.tensor(pts, dtype=torch.float32)
    got = x.to(torch.float8_e4m3fn).view(torch.uint8).tolist()
    for v, code in zip(x.tolist(), got):
        assert code == _e4m3fn_rne(v), (v, hex(code), hex(_e4m3fn_rne(v)))


def test_quantize_block_max_hits_448_and_layout():
    T, H = 3, 512
    g = torch.Generator().manual_seed(6)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    # block (t=2, b=1) gets a much larger magnitude: its scale must land at [1, 2]
    x[2, 128:256] *= 1000
    x[1, 256:384] = 0  # an all-zero block
    q, s = R.quantize_fp8_blocks(x)
    assert q.dtype == torch.float8_e4m3fn and q.shape == (T, H)
    assert s.dtype == torch.float32 and s.shape == (H // 128, T)
    xf = x.float().view(T, H // 128, 128)
    amax = xf.abs().amax(2)
    assert torch.equal(s[1, 2], torch.max(amax[2, 1], torch.tensor(1e-10)) / 448)
    assert s[1, 2] > 100 * s[0, 2] and s[1, 2] > 100 * s[1, 0]
    qf = q.float().view(T, H // 128, 128)
    for t in range(T):
        for b in range(H // 128):
            if amax[t, b] == 0:
                assert torch.count_nonzero(qf[t, b]) == 0
                assert s[b, t] == torch.tensor(1e-10, dtype=torch.float32) / 448
                continue
            i = int(xf[t, b].abs().argmax())
            assert abs(float(qf[t, b, i])) == 448.0
            assert math.copysign(1, float(qf[t, b, i])) == math.copysign(1, float(xf[t, b, i]))


def test_quantize_round_trip_error_bound():
    T, H = 4, 1024
    g = torch.Generator().manual_seed(8)
    x = (torch.randn(T, H, generator=g) * torch.logspace(-3, 3, H // 128).repeat_interleave(128)).to(torch.bfloat16)
    q, s = R.quantize_fp8_blocks(x)
    deq = R.dequant_activations(q, s, torch.float64)
    xd = x.double()
    sd = s.double().t().repeat_interleave(128, 1)
    y = xd / sd  # value in fp8 units
    normal = y.abs() >= 2 ** -6
    # 3 mantissa bits: half an ulp is 2^-4 relative (normal) or 2^-10 absolute (subnormal)
    assert ((deq - xd).abs() <= 2 ** -4 * xd.abs() * (1 + 1e-6))[normal].all()
    assert ((deq - xd).abs() <= 2 ** -10 * sd * (1 + 1e-6))[~normal].all()
    # a value that is already an fp8 multiple of its block's scale survives exactly
    z = torch.zeros(1, 128)
    z[0, 0], z[0, 1], z[0, 2] = 448.0, -3.5, 0.013671875  # 7 * 2^-9 is subnormal
    q2, s2 = R.quantize_fp8_blocks(z.to(torch.bfloat16))
    assert float(s2[0, 0]) == 1.0
    assert torch.equal(q2.float()[0, :3], z[0, :3])
