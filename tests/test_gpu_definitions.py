"""The operator for other layer definitions, each from its own library:

* the default layer with 64 local experts (its 256 experts sharded over 4
  GPUs instead of 8);
* another routing family: 128 experts in 8 groups of 16, top-3 groups,
  top-6 experts, 16 local experts, H=4096, I=1536.

The reference's routing kernel takes these as constexpr parameters
(kernel.py:371-389); here each is a library build. Bars, as for the default
definition: routing sets bit-exact (and the same order), weights within 1e-6;
sort tables bit-exact; output |out-ref| <= 1e-2*|ref| + 1e-2*max|ref| against
the oracle run with the definition's parameters, at T = 1, 64, 170, 171, 1024,
8192 and a skewed batch.
"""
import pytest
import torch

from _helpers import gpu_args, log, oracle_subset, run_gpu, spread_tokens

from flashinfer_amd import _lib, kernel, shapes
from flashinfer_amd import workloads as W

pytestmark = pytest.mark.gpu

DEFS = [d for d in shapes.DEFINITIONS if not d.default_routing]


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _route_ref(wl, defn):
    from oracle import ref_moe as R
    t = wl.tensors
    return R.route(t["routing_logits"], t["routing_bias"], wl.routed_scaling_factor,
                   defn.NG, defn.KG, defn.TOPK)


def _offset_with_local(defn, T, seed):
    """A shard offset holding one of token 0's experts (so T = 1 has a local slot)."""
    wl = W.make_tokens(T, seed, defn.H, defn.EG)
    from oracle import ref_moe as R
    r = R.route(wl["routing_logits"], wl["routing_bias"], 2.5, defn.NG, defn.KG, defn.TOPK)
    return (int(r.ids[0, 0]) // defn.EL) * defn.EL


def _check_route(wl, defn):
    from oracle import ref_moe as R
    t = wl.tensors
    ids, w = kernel.route(t["routing_logits"].cuda(), t["routing_bias"].cuda(),
                          wl.routed_scaling_factor, definition=defn)
    ids, w = ids.cpu(), w.cpu()
    ref = _route_ref(wl, defn)
    assert ids.shape == (wl.T, defn.TOPK)
    mism = R.routing_set_mismatch(ids, ref.ids)
    log(f"route {defn.name} T={wl.T}: set mismatches={mism}")
    assert mism == 0
    assert torch.equal(ids.long(), ref.ids)
    assert torch.allclose(w, ref.weights, rtol=1e-6, atol=0)
    return ref


def _check_tables(wl, defn, ref):
    """Expert offsets, slots and per-token slot lists of the call's sort."""
    from oracle import ref_moe as R
    L = _lib.workspace_layout(wl.T, defn)
    ws = kernel.last_workspace().cpu()
    EL = defn.EL
    eoff = ws[L.expert_off:L.expert_off + (EL + 1) * 4].view(torch.int32).long()
    slots = R.local_assignment(ref.ids, ref.weights, wl.local_expert_offset, EL)
    counts = torch.tensor([len(tk) for tk, _ in slots])
    want = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)])
    assert torch.equal(eoff, want)
    S = int(want[-1])
    stok = ws[L.sorted_tok:L.sorted_tok + S * 4].view(torch.int32).long()
    assert torch.equal(stok, torch.cat([tk for tk, _ in slots]))
    tslot = ws[L.tok_slot:L.tok_slot + wl.T * 32].view(torch.int32).view(wl.T, 8).long()
    for t in range(0, wl.T, max(1, wl.T // 100)):
        mine = [int(s) for s in tslot[t] if s >= 0]
        exp = [int(want[e]) + int((slots[e][0] == t).nonzero()[0]) for e in range(EL)
               if bool((slots[e][0] == t).any())]
        assert mine == exp
    return S


def _check_output(wl, out, tokens):
    from oracle import ref_moe as R
    ref = oracle_subset(wl, tokens)
    got = out[tokens.to(out.device)].float().cpu()
    rep = R.tolerance_report(got, ref.acc)
    log(f"output {wl.name}: tokens={len(tokens)} {rep}")
    assert torch.isfinite(got).all()
    assert rep["n_bad"] == 0, rep


# 170 / 171: the 128-expert top-6 build's switch from the stream to the wide
# kernels (T * top_k <= 8 * global experts)
@pytest.mark.parametrize("T", [1, 64, 170, 171, 1024, 8192])
@pytest.mark.parametrize("defn", DEFS, ids=lambda d: d.tag)
def test_definition_parity(defn, T):
    log(f"test_definition_parity[{defn.name}-T={T}]")
    seed = 7000 + T
    offset = _offset_with_local(defn, T, seed) if T <= 64 else (defn.EL * (T % 3)) % defn.EG
    wl = W.make_for(defn, f"{defn.tag}_t{T}", T, seed, local_expert_offset=offset)
    ref = _check_route(wl, defn)
    out = run_gpu(wl, fill=float("nan"))
    S = _check_tables(wl, defn, ref)
    log(f"  offset {offset}: {S} local slots")
    if T <= 64:
        assert S >= 1  # the shard holds token 0's first expert
    tokens = torch.arange(T) if T <= 1024 else spread_tokens(T, 1024)
    _check_output(wl, out, tokens)


@pytest.mark.parametrize("T,offset,want", [(768, 0, 0), (768, 128, 1), (1024, 128, 1)])
def test_ep4_gemm1_device_choice(T, offset, want, monkeypatch):
    """The default layer with 64 local experts: from T = 640 to 1536 the sort
    chooses the GEMM1 kernel from the expert counts, as in the 32-expert
    build (the LDS tile when the 64-row tiling has at least 11 more row tiles
    than active experts). The choice and both tables are as the oracle's
    counts give, and the output is bitwise either kernel's forced output and
    within the bar."""
    from oracle import ref_moe as R
    defn = [d for d in DEFS if d.EL == 64][0]
    log(f"test_ep4_gemm1_device_choice[T={T}-off={offset}]")
    wl = W.make_for(defn, f"{defn.tag}_choice", T, 900 + T + offset, local_expert_offset=offset)
    ref = _route_ref(wl, defn)
    ids = ref.ids.flatten() - offset
    cnt = torch.bincount(ids[(ids >= 0) & (ids < defn.EL)], minlength=defn.EL)
    extra = int(((cnt + 63) // 64).sum()) - int((cnt > 0).sum())
    assert int(extra >= 11) == want  # the batches were picked for each branch
    out = run_gpu(wl, fill=float("nan")).clone()
    L = _lib.workspace_layout(T, defn)
    meta = kernel.last_workspace()[L.expert_off:L.expert_off + 576 * 4].view(torch.int32).cpu()
    assert int(meta[512]) == want  # stride 128: prefixes at 128 (64-row), 384 (256-row)
    assert int(meta[128 + 64]) == (0 if want else int(((cnt + 63) // 64).sum()))
    assert int(meta[384 + 64]) == (int(((cnt + 255) // 256).sum()) if want else 0)
    for forced in ("15,21", "19,21"):
        monkeypatch.setenv("MI_MOE_VARIANT", forced)
        f = run_gpu(wl, fill=float("nan"))
        assert torch.equal(out.view(torch.int16), f.view(torch.int16)), forced
    _check_output(wl, out, spread_tokens(T, 48))


@pytest.mark.parametrize("defn", DEFS, ids=lambda d: d.tag)
def test_definition_skewed_batch(defn):
    """Every token's bias makes it pick local experts offset..: each of the top_k
    biased experts holds T rows (several tiles, the chunked sort above 1024)."""
    T = 2049
    log(f"test_definition_skewed_batch[{defn.name}]")
    wl = W.make_for(defn, f"{defn.tag}_skew", T, 7777, local_expert_offset=defn.EL, skew=True)
    ref = _check_route(wl, defn)
    out = run_gpu(wl, fill=float("nan"))
    S = _check_tables(wl, defn, ref)
    assert S == T * min(defn.TOPK, 8)
    tokens = torch.cat([torch.arange(8), torch.arange(T - 8, T), spread_tokens(T, 48)]).unique()
    _check_output(wl, out, tokens)


@pytest.mark.parametrize("defn", DEFS, ids=lambda d: d.tag)
def test_definition_sort_entry(defn):
    """mi_moe_sort fed the oracle's [T, top_k] routing (repacked to the
    workspace's 8-wide rows when top_k < 8) builds the oracle's assignment."""
    from oracle import ref_moe as R
    T = 1500
    log(f"test_definition_sort_entry[{defn.name}]")
    wl = W.make_for(defn, f"{defn.tag}_sort", T, 7100, local_expert_offset=defn.EL)
    ref = _route_ref(wl, defn)
    eoff, stok, sw, slots = kernel.sort(ref.ids.to(torch.int32).cuda(),
                                        ref.weights.to(torch.float32).cuda(), wl.local_expert_offset,
                                        definition=defn)
    want = R.local_assignment(ref.ids, ref.weights, wl.local_expert_offset, defn.EL)
    counts = torch.tensor([len(tk) for tk, _ in want])
    assert torch.equal(eoff.cpu().long(), torch.cat([torch.zeros(1, dtype=torch.long),
                                                     counts.cumsum(0)]))
    assert torch.equal(stok.cpu().long(), torch.cat([tk for tk, _ in want]))
    assert torch.equal(sw.cpu(), torch.cat([x for _, x in want]).float())
    assert bool((slots.cpu()[:, defn.TOPK:] == -1).all())


@pytest.mark.parametrize("defn", DEFS, ids=lambda d: d.tag)
def test_definition_run_bf16_and_graph(defn):
    """The bf16 front end (quantiser + routing in one launch) and a captured
    graph replay give the plain call's output bit for bit."""
    T = 48
    log(f"test_definition_run_bf16_and_graph[{defn.name}]")
    wl = W.make_for(defn, f"{defn.tag}_bf16", T, 7200, local_expert_offset=0)
    g = torch.Generator().manual_seed(5)
    x = torch.randn(T, defn.H, generator=g).to(torch.bfloat16).cuda()
    args = gpu_args(wl)
    hs, sc = kernel.quantize_activations(x)
    args[2], args[3] = hs, sc
    ref = torch.empty(T, defn.H, dtype=torch.bfloat16, device="cuda")
    kernel.run(*args, ref)
    out = torch.full_like(ref, float("nan"))
    kernel.run_bf16(args[0], args[1], x, *args[4:10], out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    graph = torch.cuda.CUDAGraph()
    out2 = torch.full_like(ref, float("nan"))
    with torch.cuda.graph(graph):
        kernel.run(*args, out2)
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out2.view(torch.int16), ref.view(torch.int16))
