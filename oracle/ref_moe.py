"""CPU restatement of the FP8 block-scaled DeepSeek-routed fused MoE.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, as the answer GPU results are compared
with (or the timed CPU baseline). Never on the product path.

It restates the definition ``moe_fp8_block_scale_ds_routing_topk8_ng8_kg4_e32_h7168_i2048``
(config.toml:3) as the Triton solution in ``solution/triton/kernel.py``
computes it, in plain fp32 (or fp64 with ``acc_dtype=torch.float64``) torch
on the CPU. Shapes are taken from the tensors, so tiny instantiations
(H=256, I=128, ...) run in milliseconds for brute-force tests.

Pinning status (each function's checks live in ``tests/test_oracle.py``):

* ``route``           pinned: hand-built known-answer cases (group top-2 sum
                      vs top-1, bias ordering, skewed bias, out-of-range
                      offset), invariants, and a pure-Python brute force.
* ``dequant_blocks``  pinned: element-by-element fp64 loop + one-hot scale
                      probes that fail on a transposed scale layout.
* ``swiglu``          pinned: halves known-answer (SiLU on the second half).
* ``expert_forward``  pinned: brute-force fp64 loops at a tiny shape.
* ``moe_forward``     pinned: combine known-answer (two experts, one-hot
                      weights), linearity in the routed scaling factor and
                      in the GEMM2 scales, zero output for empty routing.
* ``quantize_fp8_blocks`` (the activation quantiser that produces
                      hidden_states / hidden_states_scale; no reference
                      code exists for it) pinned: a pure-Python e4m3fn
                      round-to-nearest-even over all 256 codes, the block
                      maximum landing exactly on +-448, the rounding-error
                      bound, zero blocks and a scale-layout probe.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch

BLOCK = 128  # scale block along every quantised axis (kernel.py:622)


@dataclass
class RouteResult:
    ids: torch.Tensor  # int64 [T, top_k] global expert ids, selection order
    weights: torch.Tensor  # fp32 [T, top_k] normalised, scaled weights
    scores: torch.Tensor  # fp32 [T, E] sigmoid(logits) (no bias)


def route(
    routing_logits: torch.Tensor,
    routing_bias: torch.Tensor,
    routed_scaling_factor: float,
    n_group: int = 8,
    topk_group: int = 4,
    top_k: int = 8,
) -> RouteResult:
    """DeepSeek no-aux routing (kernel.py:400-452).

    s = sigmoid(logit); sb = s + bias; group score = top1 + top2 of sb in each
    group (kernel.py:406-416); keep the ``topk_group`` best groups
    (kernel.py:418-426); pick ``top_k`` experts by sb among them
    (kernel.py:428-438); weight = s * rsf / (sum of the top_k s + 1e-20)
    (kernel.py:440, :450). Ties go to the lowest index (``tl.argmax``'s
    left-most rule), reproduced here with a stable descending sort.
    """
    logits = routing_logits.to(torch.float32)
    T, E = logits.shape
    gsize = E // n_group
    s = torch.sigmoid(logits)
    sb = s + routing_bias.to(torch.float32)[None, :]

    grouped = sb.view(T, n_group, gsize)
    top2 = torch.sort(grouped, dim=-1, descending=True, stable=True).values[..., :2]
    group_scores = top2[..., 0] + top2[..., 1]
    gsel = torch.sort(group_scores, dim=-1, descending=True, stable=True).indices[:, :topk_group]
    gmask = torch.zeros(T, n_group, dtype=torch.bool)
    gmask.scatter_(1, gsel, True)
    emask = gmask[:, :, None].expand(T, n_group, gsize).reshape(T, E)
    pruned = torch.where(emask, sb, torch.full_like(sb, float("-inf")))
    ids = torch.sort(pruned, dim=-1, descending=True, stable=True).indices[:, :top_k]

    topk_s = torch.gather(s, 1, ids)
    denom = topk_s.sum(dim=-1, keepdim=True)
    weights = topk_s * routed_scaling_factor / (denom + 1e-20)
    return RouteResult(ids=ids, weights=weights.to(torch.float32), scores=s)


def local_assignment(ids: torch.Tensor, weights: torch.Tensor, local_expert_offset: int, e_local: int):
    """Per local expert (ascending), its tokens (ascending) and their weights.

    Mirrors the local filter of kernel.py:442-452 (non-local -> dropped) and
    the per-expert grouping of kernel.py:460-505, with a deterministic
    token-ascending order inside each expert.
    """
    out = []
    for e in range(e_local):
        hit = ids == (local_expert_offset + e)  # [T, k]; at most one True per row
        tok = torch.nonzero(hit.any(dim=1), as_tuple=False).flatten()
        w = (weights * hit.to(weights.dtype)).sum(dim=1)[tok]
        out.append((tok, w))
    return out


def dequant_blocks(x8: torch.Tensor, scale: torch.Tensor, acc_dtype=torch.float32) -> torch.Tensor:
    """Dequantise a 2-D fp8 tensor with one scale per 128x128 block.

    ``scale`` has shape [ceil(R/128), ceil(C/128)] (rows-block major), the
    layout of gemm{1,2}_weights_scale[e] (kernel.py:170, :275).
    """
    R, C = x8.shape
    full = scale.to(acc_dtype).repeat_interleave(BLOCK, 0)[:R].repeat_interleave(BLOCK, 1)[:, :C]
    return x8.to(acc_dtype) * full


def dequant_activations(hs8: torch.Tensor, hs_scale: torch.Tensor, acc_dtype=torch.float32) -> torch.Tensor:
    """hidden_states [T, H] fp8 with hidden_states_scale [H/128, T] (K-block major,
    kernel.py:169 reads ``A_scale_ptr + kb*stride_as_kb + t*stride_as_t``)."""
    T, H = hs8.shape
    full = hs_scale.to(acc_dtype).t().repeat_interleave(BLOCK, 1)[:, :H]
    return hs8.to(acc_dtype) * full


FP8_MAX = 448.0  # largest finite e4m3fn value
QUANT_EPS = 1e-10  # floor of a block's amax, so an all-zero block gets a finite scale


def quantize_fp8_blocks(x: torch.Tensor, eps: float = QUANT_EPS):
    """Per-token, per-128-element-block fp8 e4m3fn quantisation of activations.

    Produces the ``hidden_states`` / ``hidden_states_scale`` pair that
    ``run`` consumes (kernel.py:600-613), with the scale in the block-major
    [H/128, T] layout kernel.py:169 reads. In fp32: s = max(amax, eps) / 448,
    q = e4m3fn(clamp(x / s, -448, 448)) rounded to nearest even.
    Returns (q [T, H] float8_e4m3fn, s [H/128, T] fp32). Finite inputs only.
    """
    T, H = x.shape
    xf = x.to(torch.float32).reshape(T, H // BLOCK, BLOCK)
    amax = xf.abs().amax(dim=2)
    s = torch.clamp(amax, min=eps) / FP8_MAX
    q = torch.clamp(xf / s[..., None], -FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q.reshape(T, H), s.t().contiguous()


def swiglu(g: torch.Tensor) -> torch.Tensor:
    """silu(second half) * first half (kernel.py:297-298, :318-326)."""
    inter = g.shape[-1] // 2
    gate = g[..., :inter]
    up = g[..., inter:]
    return up * torch.sigmoid(up) * gate


def expert_forward(a: torch.Tensor, w1: torch.Tensor, w1s: torch.Tensor, w2: torch.Tensor,
                   w2s: torch.Tensor, acc_dtype=torch.float32, act_round=None) -> torch.Tensor:
    """One expert: dequantised GEMM1 -> SwiGLU -> dequantised GEMM2.

    ``a`` is the already dequantised activation block [M, H] in ``acc_dtype``.
    ``act_round`` optionally rounds the SwiGLU output (e.g. ``torch.bfloat16``)
    before GEMM2, to model an implementation's intermediate precision.
    """
    w1f = dequant_blocks(w1, w1s, acc_dtype)  # [2I, H]
    g = a @ w1f.t()
    x = swiglu(g)
    if act_round is not None:
        x = x.to(act_round).to(acc_dtype)
    w2f = dequant_blocks(w2, w2s, acc_dtype)  # [H, I]
    return x @ w2f.t()


@dataclass
class MoEResult:
    output: torch.Tensor  # bf16 [T, H]
    route: RouteResult
    acc: torch.Tensor  # [T, H] accumulator before the bf16 cast
    slots: list  # per local expert (tokens, weights)


def moe_forward(
    routing_logits, routing_bias, hidden_states, hidden_states_scale,
    gemm1_weights, gemm1_weights_scale, gemm2_weights, gemm2_weights_scale,
    local_expert_offset, routed_scaling_factor,
    *, n_group=8, topk_group=4, top_k=8, acc_dtype=torch.float32, act_round=None,
    dequant_all_experts=False,
) -> MoEResult:
    """The whole layer for one expert-parallel shard (kernel.py:600-825).

    Non-local experts contribute nothing; tokens with no local expert get a
    zero row (kernel.py:692-695, :801). Contributions are summed per token in
    ascending local-expert order, then cast to bf16 (kernel.py:822).

    ``dequant_all_experts=True`` dequantises every local expert's weights
    before routing, as a definition-style reference that materialises the
    dequantised weight tensors does on every call; the result is the same,
    only the work (and its CPU time) differs.
    """
    local_expert_offset = int(local_expert_offset)
    routed_scaling_factor = float(routed_scaling_factor)
    T, H = hidden_states.shape
    e_local = gemm1_weights.shape[0]
    full = None
    if dequant_all_experts:
        full = [(dequant_blocks(gemm1_weights[e], gemm1_weights_scale[e], acc_dtype),
                 dequant_blocks(gemm2_weights[e], gemm2_weights_scale[e], acc_dtype))
                for e in range(e_local)]
    r = route(routing_logits, routing_bias, routed_scaling_factor, n_group, topk_group, top_k)
    slots = local_assignment(r.ids, r.weights, local_expert_offset, e_local)
    acc = torch.zeros(T, H, dtype=acc_dtype)
    if T > 0 and any(len(t) for t, _ in slots):
        a = dequant_activations(hidden_states, hidden_states_scale, acc_dtype)
        for e, (tok, w) in enumerate(slots):
            if len(tok) == 0:
                continue
            if full is None:
                o = expert_forward(a[tok], gemm1_weights[e], gemm1_weights_scale[e],
                                   gemm2_weights[e], gemm2_weights_scale[e], acc_dtype, act_round)
            else:
                x = swiglu(a[tok] @ full[e][0].t())
                if act_round is not None:
                    x = x.to(act_round).to(acc_dtype)
                o = x @ full[e][1].t()
            acc.index_add_(0, tok, o * w.to(acc_dtype)[:, None])
    return MoEResult(output=acc.to(torch.bfloat16), route=r, acc=acc, slots=slots)


def algorithmic_bytes(T: int, active_experts: int, H=7168, I=2048, E=256) -> int:
    """HBM bytes a call must move at minimum: logits, bias, hs, hs_scale, the
    bf16 output, and the weights + scales of every active local expert."""
    per_tok = E * 4 + H + (H // BLOCK) * 4 + H * 2
    per_expert = 2 * I * H + H * I + (2 * I // BLOCK) * (H // BLOCK) * 4 + (H // BLOCK) * (I // BLOCK) * 4
    return per_tok * T + E * 2 + active_experts * per_expert


def algorithmic_flops(slots: int, H=7168, I=2048) -> int:
    """GEMM1 (2*2I*H) + GEMM2 (2*H*I) flops per local slot."""
    return slots * (2 * 2 * I * H + 2 * H * I)


def tolerance_report(out: torch.Tensor, ref: torch.Tensor, rtol=1e-2, atol_rel=1e-2) -> dict:
    """Elementwise check |out-ref| <= rtol*|ref| + atol_rel*max|ref|, plus
    normwise error. ``atol`` is relative to the output magnitude because the
    output's scale (~1e-4) makes an absolute 1e-2 vacuous."""
    o = out.to(torch.float64)
    r = ref.to(torch.float64)
    d = (o - r).abs()
    maxref = float(r.abs().max()) if r.numel() else 0.0
    bound = rtol * r.abs() + atol_rel * maxref
    bad = int((d > bound).sum())
    nrm = float(r.norm())
    return {
        "max_abs_err": float(d.max()) if d.numel() else 0.0,
        "max_ref": maxref,
        "normwise_rel": float((o - r).norm() / nrm) if nrm > 0 else float(d.max() if d.numel() else 0.0),
        "n_bad": bad,
        "frac_bad": bad / max(1, d.numel()),
    }


def routing_set_mismatch(ids_a: torch.Tensor, ids_b: torch.Tensor) -> int:
    """Number of tokens whose top-k id SETS differ (order is unspecified)."""
    a = torch.sort(ids_a.to(torch.int64), dim=1).values
    b = torch.sort(ids_b.to(torch.int64), dim=1).values
    return int((a != b).any(dim=1).sum())


def near_tie_tokens(routing_logits, routing_bias, n_group=8, topk_group=4, top_k=8, ulps=4) -> int:
    """Tokens whose expert-(k/k+1) or group-(kg/kg+1) boundary is within
    ``ulps`` float32 ulps: where a 1-ulp sigmoid difference could flip the set."""
    logits = routing_logits.to(torch.float32)
    T, E = logits.shape
    s = torch.sigmoid(logits)
    sb = s + routing_bias.to(torch.float32)[None, :]
    grouped = sb.view(T, n_group, E // n_group)
    top2 = torch.sort(grouped, dim=-1, descending=True).values[..., :2]
    gs = torch.sort(top2.sum(-1), dim=-1, descending=True).values
    eps = torch.finfo(torch.float32).eps
    g_gap = (gs[:, topk_group - 1] - gs[:, topk_group]).abs() <= ulps * eps * gs[:, topk_group - 1].abs()
    r = route(routing_logits, routing_bias, 1.0, n_group, topk_group, top_k)
    gsize = E // n_group
    gsel = torch.zeros(T, n_group, dtype=torch.bool)
    sel_groups = (r.ids // gsize)
    gsel.scatter_(1, sel_groups, True)
    pruned = torch.where(gsel[:, :, None].expand(T, n_group, gsize).reshape(T, E), sb,
                         torch.full_like(sb, float("-inf")))
    vals = torch.sort(pruned, dim=-1, descending=True).values
    e_gap = (vals[:, top_k - 1] - vals[:, top_k]).abs() <= ulps * eps * vals[:, top_k - 1].abs()
    return int((g_gap | e_gap).sum())
