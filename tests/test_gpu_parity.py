"""GPU parity of the fused MoE against the CPU oracle, through the C ABI.

Bars (written in each test):
* routing: top-8 id SETS bit-exact per token (order is unspecified);
  weights within 1e-6 relative (same formula, fp32, different sum order);
* slot order, expert offsets, per-token slot lists: bit-exact;
* output: |out - ref| <= 1e-2 * |ref| + 1e-2 * max|ref| elementwise against the
  oracle's fp32 accumulator, no element outside;
* determinism: two calls are bit-identical.
"""
import pytest
import torch

from flashinfer_amd import workloads as W

from _helpers import log, oracle_subset, run_gpu, spread_tokens, gpu_args

pytestmark = pytest.mark.gpu

RTOL, ATOL_REL = 1e-2, 1e-2


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from flashinfer_amd import _lib
    _lib.lib()


def _route_check(wl):
    from flashinfer_amd import kernel
    from oracle import ref_moe as R
    t = wl.tensors
    ids, w = kernel.route(t["routing_logits"].cuda(), t["routing_bias"].cuda(), wl.routed_scaling_factor)
    ids, w = ids.cpu(), w.cpu()
    ref = R.route(t["routing_logits"], t["routing_bias"], wl.routed_scaling_factor)
    mism = R.routing_set_mismatch(ids, ref.ids)
    ties = R.near_tie_tokens(t["routing_logits"], t["routing_bias"])
    log(f"route {wl.name}: T={wl.T} set mismatches={mism} near-tie tokens={ties}")
    assert mism == 0
    # same selection order, so weights line up position by position
    assert torch.equal(ids.long(), ref.ids)
    assert torch.allclose(w, ref.weights, rtol=1e-6, atol=0)


@pytest.mark.parametrize("name", ["c1_t1", "c1_t4", "c0_t16", "c1_t64", "c2_t1024_o0", "c3_t8192",
                                  "c4_t14000_skew"])
def test_route_parity(name):
    log(f"test_route_parity[{name}]")
    wl = W.standard_tokens(name)
    _route_check(wl)


def _check_output(wl, out, tokens):
    from oracle import ref_moe as R
    ref = oracle_subset(wl, tokens)
    got = out[tokens.to(out.device)].float().cpu()
    rep = R.tolerance_report(got, ref.acc)
    n_slots = sum(len(tk) for tk, _ in ref.slots)
    log(f"output {wl.name}: tokens={len(tokens)} slots={n_slots} {rep}")
    assert torch.isfinite(got).all()
    assert rep["n_bad"] == 0, rep
    return rep


@pytest.mark.parametrize("name", ["c1_t1", "c1_t4", "c0_t16", "c1_t16", "c1_t64", "t256"])
def test_output_parity_decode(name):
    log(f"test_output_parity_decode[{name}]")
    wl = W.standard(name)
    out = run_gpu(wl, fill=float("nan"))
    _check_output(wl, out, torch.arange(wl.T))


@pytest.mark.parametrize("name", ["c2_t1024_o0", "c2_t1024_o64", "c2_t1024_o128", "c2_t1024_o224"])
def test_output_parity_mid(name):
    """T=1024 at each of the four shard offsets: every token."""
    log(f"test_output_parity_mid[{name}]")
    wl = W.standard(name)
    out = run_gpu(wl, fill=float("nan"))
    _check_output(wl, out, torch.arange(wl.T))


def test_output_parity_prefill_every_token():
    """T=8192: every token against the oracle (11,559 slots over 28 experts,
    each expert spanning several 256-row tiles with a partial last one), so a
    mis-indexed row tile or tile order shows up wherever it lands."""
    log("test_output_parity_prefill_every_token[c3_t8192]")
    wl = W.standard("c3_t8192")
    out = run_gpu(wl, fill=float("nan"))
    assert torch.isfinite(out.float()).all()
    _check_output(wl, out, torch.arange(wl.T))


def test_output_parity_skew_every_token():
    """T=14000 with every token on the same 8 local experts (14,000 rows each,
    token-ascending, so every 256-row tile of all 8 experts is checked,
    including the partial last one of 176 rows): every token."""
    log("test_output_parity_skew_every_token[c4_t14000_skew]")
    wl = W.standard("c4_t14000_skew")
    out = run_gpu(wl, fill=float("nan"))
    assert torch.isfinite(out.float()).all()
    _check_output(wl, out, torch.arange(wl.T))


@pytest.mark.parametrize("name,fuse", [("c1_t1", "0"), ("c1_t4", "1"), ("c1_t16", "1"), ("c1_t16", "0"),
                                       ("c1_t64", "0"), ("c1_t64", "1"), ("t256", "1"), ("t256", "0"),
                                       ("c2_t1024_o64", "0"), ("c3_t8192", "0")])
def test_sort_stage_bit_exact(name, fuse, monkeypatch):
    """Expert offsets, slot order (token-ascending per expert) and per-token
    slot lists from the workspace equal the oracle's local assignment, for the
    one-wave sort (T <= 64), the one-workgroup sort, the fused routing + sort
    and the chunked sort."""
    from flashinfer_amd import _lib, kernel
    from oracle import ref_moe as R
    log(f"test_sort_stage_bit_exact[{name}-{fuse}]")
    monkeypatch.setenv("MI_MOE_FUSE_FRONT", fuse)
    wl = W.standard(name)
    run_gpu(wl)
    L = _lib.workspace_layout(wl.T)
    ws = kernel.last_workspace().cpu()
    T = wl.T
    eoff = ws[L.expert_off:L.expert_off + 33 * 4].view(torch.int32)
    r = R.route(wl.tensors["routing_logits"], wl.tensors["routing_bias"], wl.routed_scaling_factor)
    slots = R.local_assignment(r.ids, r.weights, wl.local_expert_offset, 32)
    counts = torch.tensor([len(tk) for tk, _ in slots])
    want_off = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    assert torch.equal(eoff.long(), want_off)
    S = int(want_off[-1])
    stok = ws[L.sorted_tok:L.sorted_tok + S * 4].view(torch.int32).long()
    sw = ws[L.sorted_w:L.sorted_w + S * 4].view(torch.float32)
    assert torch.equal(stok, torch.cat([tk for tk, _ in slots]))
    assert torch.allclose(sw, torch.cat([w for _, w in slots]), rtol=1e-6, atol=0)
    tslot = ws[L.tok_slot:L.tok_slot + T * 8 * 4].view(torch.int32).view(T, 8).long()
    for t in range(0, T, max(1, T // 150)):
        mine = [int(s) for s in tslot[t] if s >= 0]
        assert all(int(stok[s]) == t for s in mine)
        exp = [int(want_off[e]) + int((slots[e][0] == t).nonzero()[0]) for e in range(32)
               if bool((slots[e][0] == t).any())]
        assert mine == exp
        assert all(int(s) == -1 for s in tslot[t][len(mine):])


def test_gemm1_stage_against_oracle(monkeypatch):
    """SwiGLU(GEMM1) rows in the workspace against the oracle's fp32 values:
    act (bf16) within the output bar, and act + act_lo (written with
    MI_MOE_SPLIT_ACT=1, 16 mantissa bits) within 5e-5 normwise (measured
    2.1e-5: the fp32 accumulation of the fp8 MFMAs and their block-scale
    FMAs, and the SiLU), 80x below the bf16 rounding of act alone (1.7e-3)."""
    from flashinfer_amd import _lib, kernel
    from oracle import ref_moe as R
    log("test_gemm1_stage_against_oracle")
    monkeypatch.setenv("MI_MOE_SPLIT_ACT", "1")
    wl = W.standard("c1_t64")
    run_gpu(wl)
    L = _lib.workspace_layout(wl.T)
    ws = kernel.last_workspace()
    t = wl.tensors
    r = R.route(t["routing_logits"], t["routing_bias"], wl.routed_scaling_factor)
    slots = R.local_assignment(r.ids, r.weights, wl.local_expert_offset, 32)
    a = R.dequant_activations(t["hidden_states"], t["hidden_states_scale"])
    S = sum(len(tk) for tk, _ in slots)
    act = ws[L.act:L.act + S * 2048 * 2].view(torch.bfloat16).view(S, 2048).float().cpu()
    lo = ws[L.act_lo:L.act_lo + S * 2048 * 2].view(torch.bfloat16).view(S, 2048).float().cpu()
    row = 0
    worst = worst_split = 0.0
    for e, (tk, _) in enumerate(slots):
        if len(tk) == 0:
            continue
        g = a[tk] @ R.dequant_blocks(t["gemm1_weights"][e], t["gemm1_weights_scale"][e]).t()
        x = R.swiglu(g)
        got = act[row:row + len(tk)]
        rep = R.tolerance_report(got, x)
        worst = max(worst, rep["normwise_rel"])
        assert rep["n_bad"] == 0, (e, rep)
        # act_lo is the rounding remainder: at most half a bf16 ulp of act
        assert bool((lo[row:row + len(tk)].abs() <= got.abs() * 2.0 ** -8).all())
        rep2 = R.tolerance_report(got + lo[row:row + len(tk)], x)
        worst_split = max(worst_split, rep2["normwise_rel"])
        row += len(tk)
    log(f"gemm1 stage worst normwise rel: act {worst:.2e}, act + act_lo {worst_split:.2e}")
    assert worst_split <= 5e-5


@pytest.mark.parametrize("name", ["c1_t1_local", "c1_t4", "c1_t16", "c1_t64", "t256"])
def test_gemm2_precision_modes(name, monkeypatch):
    """The three GEMM2 paths at decode sizes against the oracle on every
    token: bf16 partial rows (MI_MOE_F32_PARTIALS=0), fp32 partial rows (the
    default up to T = 1024) and the split activation act + act_lo with fp32
    rows (MI_MOE_SPLIT_ACT=1). All inside the output bar; each step no less
    precise than the one before; the split path within 10% of the floor
    that the bf16 rounding of the output alone leaves (CPU model of the
    three paths on c1_t64: 2.86e-3, 2.35e-3, 1.67e-3 against a 1.67e-3
    floor). At T <= 4 GEMM2 sums in fp32 itself (fused combine), so the
    first two paths coincide there."""
    from oracle import ref_moe as R
    log(f"test_gemm2_precision_modes[{name}]")
    wl = W.standard(name)
    tokens = torch.arange(wl.T)
    ref = oracle_subset(wl, tokens)
    reps = {}
    for mode, env in (("bf16", {"MI_MOE_F32_PARTIALS": "0"}), ("f32", {}),
                      ("split", {"MI_MOE_SPLIT_ACT": "1"})):
        monkeypatch.delenv("MI_MOE_F32_PARTIALS", raising=False)
        monkeypatch.delenv("MI_MOE_SPLIT_ACT", raising=False)
        for k, v in env.items():
            monkeypatch.setenv(k, v)
        out = run_gpu(wl, fill=float("nan"))
        reps[mode] = R.tolerance_report(out.float().cpu(), ref.acc)
        assert reps[mode]["n_bad"] == 0, (mode, reps[mode])
    floor = R.tolerance_report(ref.acc.to(torch.bfloat16).float(), ref.acc)["normwise_rel"]
    e = {k: v["normwise_rel"] for k, v in reps.items()}
    log(f"  normwise: bf16 rows {e['bf16']:.3e}, fp32 rows {e['f32']:.3e}, split "
        f"{e['split']:.3e}, bf16 output floor {floor:.3e}")
    if sum(len(tk) for tk, _ in ref.slots) > 0:
        assert e["f32"] <= e["bf16"] * 1.0001
        assert e["split"] < e["f32"]
        assert e["split"] <= 1.1 * floor


@pytest.mark.parametrize("name", ["c2_t1024_o0", "c3_t8192"])
def test_gemm2_precision_modes_prefill(name, monkeypatch):
    """GEMM2's partial rows at T = 1024 and 8192 (the LDS-tiled GEMM2),
    against the oracle. T = 1024 (every token): fp32 rows, the default up to
    T = 1024, at least 10% below bf16 rows (MI_MOE_F32_PARTIALS=0) in
    normwise error (measured on MI355X: 2.35e-3 against 2.89e-3). T = 8192
    (256 tokens spread over the batch): the workspace holds 2-byte partials
    above T = 1024, so rows are bf16 whatever the environment asks, and the
    error stays at the bf16-row level (measured 2.86e-3; fp32 rows would cost
    4% of the call there)."""
    from oracle import ref_moe as R
    log(f"test_gemm2_precision_modes_prefill[{name}]")
    wl = W.standard(name)
    tokens = torch.arange(wl.T) if wl.T <= 1024 else spread_tokens(wl.T, 256)
    ref = oracle_subset(wl, tokens)
    outs, e = {}, {}
    for mode, flag in (("default", None), ("bf16", "0"), ("f32", "1")):
        monkeypatch.delenv("MI_MOE_F32_PARTIALS", raising=False)
        if flag is not None:
            monkeypatch.setenv("MI_MOE_F32_PARTIALS", flag)
        outs[mode] = run_gpu(wl, fill=float("nan"))
        rep = R.tolerance_report(outs[mode][tokens.cuda()].float().cpu(), ref.acc)
        assert rep["n_bad"] == 0, (mode, rep)
        e[mode] = rep["normwise_rel"]
    log(f"  normwise: default {e['default']:.3e}, bf16 rows {e['bf16']:.3e}, "
        f"fp32 asked {e['f32']:.3e}")
    if wl.T <= 1024:
        assert torch.equal(outs["default"].view(torch.int16), outs["f32"].view(torch.int16))
        assert e["default"] <= 0.9 * e["bf16"]
    else:
        for mode in ("bf16", "f32"):
            assert torch.equal(outs["default"].view(torch.int16), outs[mode].view(torch.int16))
        assert e["default"] <= 3.2e-3


@pytest.mark.parametrize("T", [2, 3, 4])
def test_decode_row_loop_many_tiles(T, monkeypatch):
    """At T <= 4 the GEMM1 front kernel has 8 workgroup rows, each looping
    over row tiles y, y + 8, .... Logits that send token t to local experts
    8t .. 8t+7 (zero bias) put every slot on its own expert: 8T one-row tiles,
    so the rows loop from T = 2. Every token matches the oracle, 8T experts
    hold a slot, and the output has the bits of the separate routing and sort
    launches (whose GEMM1 takes one tile per workgroup row)."""
    from flashinfer_amd import _lib, kernel
    from oracle import ref_moe as R
    log(f"test_decode_row_loop_many_tiles[T={T}]")
    wl = W.make_workload("row_loop", T, 500 + T, local_expert_offset=0)
    t = wl.tensors
    t["routing_bias"].zero_()
    lg = t["routing_logits"]
    lg.mul_(0.1)
    for tok in range(T):
        lg[tok, 8 * tok:8 * tok + 8] = 6.0 + 0.1 * torch.arange(8, dtype=lg.dtype)
    for k in ("MI_MOE_FUSE_FRONT", "MI_MOE_ROUTE_IN_GEMM1", "MI_MOE_SORT_IN_GEMM1"):
        monkeypatch.delenv(k, raising=False)
    out = run_gpu(wl, fill=float("nan")).clone()
    L = _lib.workspace_layout(T)
    eoff = kernel.last_workspace()[L.expert_off:L.expert_off + 33 * 4].view(torch.int32).cpu()
    assert int((eoff[1:] > eoff[:-1]).sum()) == 8 * T and int(eoff[32]) == 8 * T
    _check_output(wl, out, torch.arange(T))
    for k in ("MI_MOE_FUSE_FRONT", "MI_MOE_ROUTE_IN_GEMM1", "MI_MOE_SORT_IN_GEMM1"):
        monkeypatch.setenv(k, "0")
    ref = run_gpu(wl, fill=float("nan"))
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def test_deterministic_bitwise():
    log("test_deterministic_bitwise")
    wl = W.standard("c2_t1024_o0")
    a = run_gpu(wl)
    b = run_gpu(wl, fill=1.0)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_empty_routing_zero_fill():
    log("test_empty_routing_zero_fill")
    wl = W.standard("c1_t64", local_expert_offset=256)
    out = run_gpu(wl, fill=float("nan"))
    assert torch.count_nonzero(out.float().nan_to_num(1.0)) == 0


def test_skew_all_rows_on_biased_experts():
    """Full-size property at T=14000: every token routes to exactly the 8
    biased local experts, so S = 8T and experts 8..31 are empty."""
    from flashinfer_amd import _lib, kernel
    log("test_skew_all_rows_on_biased_experts")
    wl = W.standard("c4_t14000_skew")
    run_gpu(wl)
    L = _lib.workspace_layout(wl.T)
    eoff = kernel.last_workspace()[L.expert_off:L.expert_off + 33 * 4].view(torch.int32).cpu()
    want = torch.tensor([min(e, 8) * wl.T for e in range(33)], dtype=torch.int32)
    assert torch.equal(eoff, want)


@pytest.mark.parametrize("T", [16, 64, 256])
def test_skewed_decode_parity(T):
    """Every token on the same 8 local experts at decode sizes: each expert
    holds T rows, so the stream kernels (T = 16, 64) and the wide ones (256)
    run several row tiles per expert, re-reading its weights, with the load
    policy of a random batch of that size. Every token against the oracle."""
    log(f"test_skewed_decode_parity[T={T}]")
    wl = W.make_workload(f"skew_decode_t{T}", T, 900 + T, local_expert_offset=0, skew=True)
    _route_check(wl)
    out = run_gpu(wl, fill=float("nan"))
    _check_output(wl, out, torch.arange(T))


def test_max_tokens_every_slot_local():
    """The largest accepted batch with every token routed to the same 8 local
    experts: S = 8T = 2^20 slots, so the last slots' gathered-row offsets are
    the largest the tile GEMMs form (just under 2^32 bytes). Expert offsets
    are exact, and the first and last tokens (the extreme slots of each
    expert) and a spread between them match the oracle."""
    from flashinfer_amd import _lib, kernel
    T = _lib.MI_MOE_MAX_TOKENS
    log(f"test_max_tokens_every_slot_local[T={T}]: generating inputs")
    wl = W.make_workload("max_tokens_skew", T, 113, skew=True)
    log("test_max_tokens_every_slot_local: running")
    out = run_gpu(wl, fill=float("nan"))
    L = _lib.workspace_layout(T)
    eoff = kernel.last_workspace()[L.expert_off:L.expert_off + 33 * 4].view(torch.int32).cpu()
    want = torch.tensor([min(e, 8) * T for e in range(33)], dtype=torch.int32)
    assert torch.equal(eoff, want)
    tokens = torch.cat([torch.tensor([0, 1, T - 2, T - 1]), spread_tokens(T, 12)]).unique()
    _check_output(wl, out, tokens)


def _random_workloads(n=20, seed=2026):
    """Seeded (T, offset, skew, routed_scaling_factor) draws: ragged T from 1
    to ~1100 (weighted to decode sizes), shard offsets that are negative,
    unaligned or near the end of the 256 experts."""
    g = torch.Generator().manual_seed(seed)
    pick = lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))]
    out = []
    for i in range(n):
        band = pick([(1, 8), (9, 64), (9, 64), (65, 300), (1000, 1100)])
        T = int(torch.randint(band[0], band[1] + 1, (1,), generator=g))
        offset = pick([-40, -8, 0, 5, 32, 100, 200, 224, 250])
        skew = offset >= 0 and offset <= 248 and bool(torch.rand(1, generator=g) < 0.25)
        out.append((i, T, offset, skew, pick([1.0, 2.5])))
    return out


@pytest.mark.parametrize("i,T,offset,skew,rsf", _random_workloads())
def test_random_workloads(i, T, offset, skew, rsf):
    """Output against the oracle on seeded random shapes and shard offsets
    through the default kernel choice for each T."""
    log(f"test_random_workloads[{i}: T={T} off={offset} skew={skew} rsf={rsf}]")
    wl = W.make_workload(f"random_{i}", T, 5000 + i, local_expert_offset=offset, skew=skew,
                         routed_scaling_factor=rsf)
    _route_check(wl)
    out = run_gpu(wl, fill=float("nan"))
    assert torch.isfinite(out.float()).all()
    _check_output(wl, out, spread_tokens(T, 40))


# Both sides of every T at which the default kernels change: fused GEMM2+combine
# (T <= 4), routing inside GEMM1 (T = 1), sort inside GEMM1 (T <= 64), GEMM2 stream
# shapes (16 / 17; 8 / 9 in smaller layers), wide GEMM1 with the sort folded in
# (65..256), GEMM2 stream shapes and the stream kernels' weight load policy (128 /
# 129), wide GEMM2 (177..256), tiled GEMM2 (> 256), the wide GEMM1's load policy
# (512 / 513), chunked two-kernel sort (> 1024), LDS-tiled GEMM1 (> 1536).
@pytest.mark.parametrize("T", [1, 2, 4, 5, 8, 9, 16, 17, 32, 33, 64, 65, 128, 129, 176, 177, 192,
                               193, 256, 257, 512, 513, 1024, 1025, 1536, 1537, 2049])
def test_variant_boundaries(T):
    log(f"test_variant_boundaries[T={T}]")
    wl = W.make_workload(f"boundary_t{T}", T=T, seed=1000 + T, local_expert_offset=32 * (T % 8))
    _route_check(wl)
    out = run_gpu(wl, fill=float("nan"))
    assert torch.isfinite(out.float()).all()
    _check_output(wl, out, spread_tokens(wl.T, 96))


def test_strided_inputs_and_output():
    """Non-contiguous views (kernel.py:545-546, :733-737 pass explicit strides) give the
    same bits as contiguous tensors: hidden_states_scale as the transpose of a [T, 56]
    tensor, routing_logits as a column slice, output as a strided view."""
    from flashinfer_amd import kernel
    log("test_strided_inputs_and_output")
    wl = W.standard("c1_t64")
    a = run_gpu(wl)
    args = gpu_args(wl)
    T = wl.T
    wide = torch.zeros(T, 512, device="cuda")
    wide[:, 100:356] = args[0]
    args[0] = wide[:, 100:356]
    args[3] = args[3].t().contiguous().t()  # [56, T] view with strides (1, 56)
    assert not args[0].is_contiguous() and not args[3].is_contiguous()
    buf = torch.full((T, 2 * 7168), float("nan"), dtype=torch.bfloat16, device="cuda")
    out = buf[:, ::2]
    assert not out.is_contiguous()
    kernel.run(*args, out)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), out.contiguous().view(torch.int16))


def test_scalar_tensor_arguments():
    """Scalars given as 0-d tensors behave like Python numbers (kernel.py:547-548)."""
    from flashinfer_amd import kernel
    log("test_scalar_tensor_arguments")
    wl = W.standard("c1_t16")
    a = run_gpu(wl)
    args = gpu_args(wl)
    args[8] = torch.tensor(wl.local_expert_offset)
    args[9] = torch.tensor(wl.routed_scaling_factor)
    out = torch.empty_like(a)
    kernel.run(*args, out)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), out.view(torch.int16))


# Every GEMM1 id (0-9, 11, 12, 15, 16, 18, 19) and every GEMM2 id (0-18, 20, 21) appears at least once.
@pytest.mark.parametrize("variant", ["0", "1", "2", "3", "4", "0,3", "3,0", "5,10", "6,6", "7,1",
                                     "8,2", "9,10", "1,10", "11,11", "12,12", "5,13", "5,14",
                                     "2,9", "9,5", "5,7", "5,8", "15", "15,3", "5,15", "16", "16,14",
                                     "16,17", "18", "18,5", "16,16", "16,9", "19,3", "19,14",
                                     "15,20", "19,20", "15,21", "19,21"])
@pytest.mark.parametrize("name", ["c1_t64", "t256", "c2_t1024_o128"])
def test_every_gemm_variant_matches_oracle(name, variant, monkeypatch):
    """Each GEMM kernel family (weight-streaming with 16/32/64-row tiles, LDS
    tiles of two sizes, and mixes) gives the same answer within the bar."""
    log(f"test_every_gemm_variant_matches_oracle[{name}-{variant}]")
    monkeypatch.setenv("MI_MOE_VARIANT", variant)
    wl = W.standard(name)
    out = run_gpu(wl, fill=float("nan"))
    _check_output(wl, out, spread_tokens(wl.T, 96))


@pytest.mark.parametrize("variant", ["15", "15,3", "3,3", "18,3", "19,3", "19,20", "19,21"])
@pytest.mark.parametrize("name", ["c3_t8192", "c4_t14000_skew"])
def test_wide_variants_large(name, variant, monkeypatch):
    """The wide kernels and the LDS tiles (GEMM1 variant 3, 18 with swapped
    operands, 19 with register-held weight fragments; GEMM2 variant 3, its
    pipelined form 20 and that form run by one workgroup per CU, 21) at prefill sizes: many row tiles per expert (T=8192)
    and 14,000 rows on each of 8 experts."""
    log(f"test_wide_variants_large[{name}-{variant}]")
    monkeypatch.setenv("MI_MOE_VARIANT", variant)
    wl = W.standard(name)
    out = run_gpu(wl, fill=float("nan"))
    assert torch.isfinite(out.float()).all()
    _check_output(wl, out, spread_tokens(wl.T, 48))


@pytest.mark.parametrize("name,T,variant", [
    ("c1_t1_local", 1, "16,17"), ("c1_t4", 4, "16,17"), ("c1_t16", 16, "16,16"),
    ("c1_t64", 64, "16,14"), ("t256", 128, "15,14"), ("t256", 176, "15,13"), ("t256", 256, "15,15"),
    ("c2_t1024_o0", 512, "15,15"), ("c2_t1024_o64", 1024, "15,21"), ("c3_t8192", 2048, "19,21")])
def test_default_variants_by_T(name, T, variant, monkeypatch):
    """The kernels picked from T (no MI_MOE_VARIANT) are the ones of the
    selection table: the default call is bitwise the call with that variant
    pair forced (a forced pair gives other bits: the GEMM2 families sum their
    k chunks in different orders)."""
    log(f"test_default_variants_by_T[{name}:{T}-{variant}]")
    monkeypatch.delenv("MI_MOE_VARIANT", raising=False)
    wl = W.standard(name, T=T)
    out = run_gpu(wl, fill=float("nan")).clone()
    monkeypatch.setenv("MI_MOE_VARIANT", variant)
    forced = run_gpu(wl, fill=float("nan"))
    assert torch.equal(out.view(torch.int16), forced.view(torch.int16))


@pytest.mark.parametrize("name,T,extra", [("c2_t1024_o0", 1024, {}), ("c2_t1024_o64", 1024, {}),
                                          ("c2_t1024_o0", 768, {}), ("c2_t1024_o64", 1280, {}),
                                          ("c2_t1024_o224", 1280, {}), ("c2_t1024_o128", 1536, {}),
                                          ("c2_t1024_o0", 640, {}),
                                          ("c2_t1024_o0", 1024, {"local_expert_offset": 256}),
                                          ("c2_t1024_o0", 1024, {"skew": True})])
def test_gemm1_device_choice(name, T, extra, monkeypatch):
    """From T = 640 to 1536 the sort chooses the GEMM1 kernel from the expert
    counts: the LDS tile (variant 19) when the 64-row tiling has at least 11
    more row tiles than active experts, else the wide kernel (15). The chosen
    kernel's row-tile table holds the tiles and the other one's holds none;
    the output is bitwise the one either variant gives when forced (both
    apply the same per-block products in the same fp32 order, so the choice
    changes only the time), and within the bar of the oracle."""
    from oracle import ref_moe as R
    from flashinfer_amd import _lib, kernel
    log(f"test_gemm1_device_choice[{name}:{T}:{extra}]")
    wl = W.standard(name, T=T, **extra)  # extra: no local token (offset 256), or all on 8 experts
    r = R.route(wl.tensors["routing_logits"], wl.tensors["routing_bias"], wl.routed_scaling_factor)
    ids = r.ids.flatten() - wl.local_expert_offset
    cnt = torch.bincount(ids[(ids >= 0) & (ids < 32)], minlength=32)
    want = int(((cnt + 63) // 64).sum()) - int((cnt > 0).sum()) >= 11
    out = run_gpu(wl, fill=float("nan")).clone()
    L = _lib.workspace_layout(T)
    meta = kernel.last_workspace()[L.expert_off:L.expert_off + 320 * 4].view(torch.int32).cpu()
    assert int(meta[256]) == int(want)
    tiles64, tiles256 = int(((cnt + 63) // 64).sum()), int(((cnt + 255) // 256).sum())
    assert int(meta[64 + 32]) == (0 if want else tiles64)
    assert int(meta[192 + 32]) == (tiles256 if want else 0)
    g2 = "15" if T <= 640 else "21"  # the default GEMM2 of this T
    monkeypatch.setenv("MI_MOE_VARIANT", ("19," if want else "15,") + g2)
    forced = run_gpu(wl, fill=float("nan"))
    assert torch.equal(out.view(torch.int16), forced.view(torch.int16))
    monkeypatch.setenv("MI_MOE_VARIANT", ("15," if want else "19,") + g2)
    other = run_gpu(wl, fill=float("nan"))
    assert torch.equal(out.view(torch.int16), other.view(torch.int16))
    _check_output(wl, out, spread_tokens(T, 64))


@pytest.mark.parametrize("fuse", ["0", "1"])
@pytest.mark.parametrize("name", ["c1_t1", "c0_t16", "c1_t64", "t256"])
def test_front_end_fused_and_split_agree(name, fuse, monkeypatch):
    """Routing + sort as one launch or as two gives the oracle's answer."""
    log(f"test_front_end_fused_and_split_agree[{name}-{fuse}]")
    monkeypatch.setenv("MI_MOE_FUSE_FRONT", fuse)
    wl = W.standard(name)
    out = run_gpu(wl, fill=float("nan"))
    _check_output(wl, out, spread_tokens(wl.T, 64))


def _sort_tables(T):
    """Copies of the sort's tables in the workspace of the last call."""
    from flashinfer_amd import _lib, kernel
    L = _lib.workspace_layout(T)
    ws = kernel.last_workspace()
    meta = ws[L.expert_off:L.expert_off + 192 * 4].view(torch.int32)
    S = int(meta[32])
    return {"expert_off": meta[0:33].clone(), "mtile1": meta[64:97].clone(),
            "mtile2": meta[128:161].clone(),
            "sorted_tok": ws[L.sorted_tok:L.sorted_tok + S * 4].view(torch.int32).clone(),
            "sorted_w": ws[L.sorted_w:L.sorted_w + S * 4].view(torch.int32).clone(),
            "tok_slot": ws[L.tok_slot:L.tok_slot + T * 32].view(torch.int32).clone()}


@pytest.mark.parametrize("T,offset,skew,variant", [
    (1, 0, False, ""), (1, 0, False, "5,17"), (3, 32, True, "5,17"), (3, 32, True, ""),
    (4, 0, False, ""), (9, 0, False, ""), (16, 96, False, ""), (33, 224, False, ""),
    (64, 0, False, ""), (64, 32, True, ""), (48, 256, False, ""), (65, 0, False, ""),
    (100, 32, True, ""), (128, 224, False, ""), (129, 0, False, ""), (200, 96, False, ""),
    (256, 32, True, ""), (160, 256, False, ""), (257, 0, False, ""), (300, 64, False, ""),
    (449, 0, True, ""), (512, 160, False, ""), (511, 32, False, ""), (512, 224, True, ""),
    (480, 256, False, "")])
def test_sort_in_gemm1_matches_sort_launch(T, offset, skew, variant, monkeypatch):
    """GEMM1 finding its row tiles from the top-k ids (and writing the sort's
    tables itself) gives bit-identical output and tables to the separate sort
    launch, for every GEMM1 kernel that can do it (K split up to 64, single-
    wave workgroups when asked for, the wide 64-row tiles from 65 to 512, up to
    8 chunks of 64 tokens): ragged T, other shard offsets, several row tiles
    per expert (skew) and no local token at all (offset 256)."""
    from flashinfer_amd import _lib, kernel
    log(f"test_sort_in_gemm1_matches_sort_launch[T={T}-off={offset}-skew={skew}-v={variant}]")
    wl = W.make_workload("sort_in_gemm1", T, 300 + T, local_expert_offset=offset, skew=skew)
    if variant:
        monkeypatch.setenv("MI_MOE_VARIANT", variant)
    monkeypatch.setenv("MI_MOE_FUSE_FRONT", "0")
    monkeypatch.setenv("MI_MOE_ROUTE_IN_GEMM1", "0")
    monkeypatch.setenv("MI_MOE_SORT_IN_GEMM1", "0")
    monkeypatch.setenv("MI_MOE_G1_SELECT", "0")  # the plain 64-row table at T = 640
    ref = run_gpu(wl, fill=float("nan")).clone()
    want = _sort_tables(T)
    # scribble over the tables so the second call must rewrite them
    L = _lib.workspace_layout(T)
    ws = kernel.last_workspace()
    ws[L.expert_off:L.tok_slot + T * 32].fill_(0x5A)
    monkeypatch.setenv("MI_MOE_SORT_IN_GEMM1", "1")
    out = run_gpu(wl, fill=float("nan"))
    got = _sort_tables(T)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    for k in want:
        assert torch.equal(got[k], want[k]), k
    if offset == 256:
        assert int(want["expert_off"][32]) == 0 and bool((out == 0).all())
    if skew and T > 16:  # some expert spans several 16-row tiles
        assert int(want["mtile1"][32]) > int((want["expert_off"][1:] > want["expert_off"][:-1]).sum())


@pytest.mark.parametrize("T,offset,skew,force,variant", [
    (1, 0, False, False, ""), (1, 0, False, False, "5,17"), (2, 32, True, False, ""),
    (4, 96, False, False, ""), (7, 0, False, False, ""), (16, 224, False, False, ""),
    (16, 32, True, False, ""), (12, 256, False, False, ""), (33, 0, False, True, ""),
    (64, 32, True, True, ""), (3, 32, True, True, "5,17"), (64, 0, False, True, "5,17")])
def test_route_in_gemm1_matches_separate_launches(T, offset, skew, force, variant, monkeypatch):
    """GEMM1 routing every token itself (each workgroup, into LDS), sorting,
    and writing the top-k and the sort tables gives bit-identical output,
    top-k and tables to the routing and sort kernels: both GEMM1 shapes
    (K split by default, single-wave workgroups when asked for), T up to 64
    when forced on, other shard offsets, skewed routing and no local token."""
    from flashinfer_amd import _lib, kernel
    log(f"test_route_in_gemm1_matches_separate_launches[T={T}-off={offset}-skew={skew}-v={variant}]")
    wl = W.make_workload("route_in_gemm1", T, 400 + T, local_expert_offset=offset, skew=skew)
    if variant:
        monkeypatch.setenv("MI_MOE_VARIANT", variant)
    for k in ("MI_MOE_FUSE_FRONT", "MI_MOE_ROUTE_IN_GEMM1", "MI_MOE_SORT_IN_GEMM1"):
        monkeypatch.setenv(k, "0")
    ref = run_gpu(wl, fill=float("nan")).clone()
    want = _sort_tables(T)
    L = _lib.workspace_layout(T)
    ws = kernel.last_workspace()
    topk_want = ws[L.topk_ids:L.expert_off].clone()
    ws[L.topk_ids:L.tok_slot + T * 32].fill_(0x5A)
    if force:
        monkeypatch.setenv("MI_MOE_ROUTE_IN_GEMM1", "1")
    else:
        for k in ("MI_MOE_FUSE_FRONT", "MI_MOE_ROUTE_IN_GEMM1", "MI_MOE_SORT_IN_GEMM1"):
            monkeypatch.delenv(k)
    out = run_gpu(wl, fill=float("nan"))
    got = _sort_tables(T)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert torch.equal(ws[L.topk_ids:L.topk_ids + T * 32], topk_want[:T * 32])
    assert torch.equal(ws[L.topk_w:L.topk_w + T * 32], topk_want[L.topk_w - L.topk_ids:][:T * 32])
    for k in want:
        assert torch.equal(got[k], want[k]), k


@pytest.mark.parametrize("T,fuse", [(1, ""), (4, ""), (64, ""), (300, ""), (1500, ""), (4, "1"),
                                    (100, "1")])
def test_fp32_bias_matches_bf16_bias(T, fuse, monkeypatch):
    """routing_bias as fp32 holding the bf16 bias's values (exact) gives the
    bf16 call's output bit for bit, through each front end: routing in GEMM1
    (T=1), the sort in GEMM1 (T=4, 64), routing and sort kernels (T=300),
    the chunked sort (T=1500) and the fused routing + sort kernel."""
    from flashinfer_amd import kernel
    log(f"test_fp32_bias_matches_bf16_bias[T={T}-fuse={fuse or 'default'}]")
    if fuse:
        monkeypatch.setenv("MI_MOE_FUSE_FRONT", fuse)
    wl = W.make_workload("fp32_bias", T, 600 + T, local_expert_offset=32 * (T % 3))
    ref = run_gpu(wl, fill=float("nan")).clone()
    args = gpu_args(wl)
    args[1] = args[1].float()
    out = torch.full_like(ref, float("nan"))
    kernel.run(*args, out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))


def _check_sort_tables(ids, w, offset, got):
    """The sort entry point's tables against the oracle's local assignment."""
    from oracle import ref_moe as R
    eoff, stok, sw, slots = [x.cpu() for x in got]
    T = ids.shape[0]
    want = R.local_assignment(ids.long(), w, offset, 32)
    counts = torch.tensor([len(tk) for tk, _ in want])
    want_off = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    assert torch.equal(eoff.long(), want_off)
    assert torch.equal(stok.long(), torch.cat([tk for tk, _ in want]))
    assert torch.equal(sw, torch.cat([x for _, x in want]).float())
    # token -> slots: ascending local expert, then -1
    expect = torch.full((T, 8), -1, dtype=torch.long)
    fill = torch.zeros(T, dtype=torch.long)
    for e, (tk, _) in enumerate(want):
        pos = int(want_off[e]) + torch.arange(len(tk))
        expect[tk, fill[tk]] = pos
        fill[tk] += 1
    assert torch.equal(slots.long(), expect)


@pytest.mark.parametrize("name", ["c1_t4", "c1_t64", "c2_t1024_o128", "c3_t8192"])
def test_sort_entry_from_oracle_routing(name):
    """mi_moe_sort fed with the oracle's routing (not the GPU's) builds exactly
    the oracle's local assignment: one-wave, one-workgroup and chunked sorts."""
    from flashinfer_amd import kernel
    from oracle import ref_moe as R
    log(f"test_sort_entry_from_oracle_routing[{name}]")
    wl = W.standard(name)
    r = R.route(wl.tensors["routing_logits"], wl.tensors["routing_bias"], wl.routed_scaling_factor)
    ids = r.ids.to(torch.int32)
    w = r.weights.to(torch.float32)
    got = kernel.sort(ids.cuda(), w.cuda(), wl.local_expert_offset)
    _check_sort_tables(ids, w, wl.local_expert_offset, got)


@pytest.mark.parametrize("T,offset,mode", [(2049, 0, "same8"), (3000, 96, "random"), (64, 224, "none"),
                                           (1, 0, "same8"), (1024, 32, "random")])
def test_sort_entry_adversarial(T, offset, mode):
    """Every token on the same 8 local experts (one expert holds T slots, across
    sort chunks), random distinct ids over all 256 experts, and no local id."""
    from flashinfer_amd import kernel
    log(f"test_sort_entry_adversarial[T={T}-{mode}]")
    g = torch.Generator().manual_seed(T + offset)
    if mode == "same8":
        ids = (offset + torch.tensor([3, 0, 7, 1, 30, 12, 5, 31])).repeat(T, 1)
    elif mode == "random":
        ids = torch.stack([torch.randperm(256, generator=g)[:8] for _ in range(T)])
    else:
        ids = torch.randint(0, offset, (T, 8), generator=g)
    ids = ids.to(torch.int32)
    w = torch.rand(T, 8, generator=g)
    got = kernel.sort(ids.cuda(), w.cuda(), offset)
    _check_sort_tables(ids, w, offset, got)
