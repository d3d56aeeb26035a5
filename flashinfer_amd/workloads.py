"""Seeded synthetic workloads for the fused-MoE operator.

Every tensor is generated on the CPU with ``torch.Generator`` so that the GPU
path and the CPU oracle see identical bytes (the GPU copy is made with
``.to(device)``). Two generators are used:

* a weight generator (``WEIGHT_SEED``) draws, in order, gemm1_weights (expert
  by expert), gemm1_weights_scale, gemm2_weights (expert by expert) and
  gemm2_weights_scale, so every workload shares the same 1.4 GB of weights;
* a per-workload generator (``seed``) draws, in order, routing_logits,
  routing_bias, hidden_states and hidden_states_scale.

Distributions: logits N(0,1) fp32 [T,256]; bias N(0,0.1) -> bf16 [256];
hidden_states N(0,1) clipped to +-448 -> fp8 e4m3fn [T,H]; hidden_states_scale
U(0.01,0.1) fp32 [H/128,T]; weights N(0,1) -> fp8 e4m3fn; weight scales
U(0.001,0.01) fp32. ``skew=True`` sets the bias of local experts 0-7 to +3.0.
"""
from __future__ import annotations

import hashlib
from dataclasses import dataclass, field

import torch

WEIGHT_SEED = 20260101
H_DEF, I_DEF, E_GLOBAL_DEF, E_LOCAL_DEF = 7168, 2048, 256, 32
BLOCK = 128
FP8 = torch.float8_e4m3fn

_WEIGHT_CACHE: dict = {}


@dataclass
class Workload:
    name: str
    T: int
    seed: int
    local_expert_offset: int = 0
    skew: bool = False
    routed_scaling_factor: float = 2.5
    tensors: dict = field(default_factory=dict)
    # routing of the definition (n_group, topk_group, top_k), for the oracle
    routing: tuple = (8, 4, 8)

    def args(self, device=None):
        """Positional arguments of ``run`` (minus ``output``) in reference order."""
        t = self.tensors
        names = ["routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
                 "gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale"]
        vals = [t[n] if device is None else t[n].to(device) for n in names]
        return vals + [self.local_expert_offset, self.routed_scaling_factor]


def _randn_fp8(shape, gen):
    return torch.randn(shape, generator=gen).clamp_(-448.0, 448.0).to(FP8)


def make_weights(H=H_DEF, I=I_DEF, E_local=E_LOCAL_DEF, seed=WEIGHT_SEED, cache=True):
    key = (H, I, E_local, seed)
    if cache and key in _WEIGHT_CACHE:
        return _WEIGHT_CACHE[key]
    g = torch.Generator().manual_seed(seed)
    w1 = torch.empty(E_local, 2 * I, H, dtype=FP8)
    for e in range(E_local):
        w1[e] = _randn_fp8((2 * I, H), g)
    w1s = torch.empty(E_local, 2 * I // BLOCK, H // BLOCK).uniform_(0.001, 0.01, generator=g)
    w2 = torch.empty(E_local, H, I, dtype=FP8)
    for e in range(E_local):
        w2[e] = _randn_fp8((H, I), g)
    w2s = torch.empty(E_local, H // BLOCK, I // BLOCK).uniform_(0.001, 0.01, generator=g)
    out = {"gemm1_weights": w1, "gemm1_weights_scale": w1s,
           "gemm2_weights": w2, "gemm2_weights_scale": w2s}
    if cache:
        _WEIGHT_CACHE[key] = out
    return out


def make_tokens(T, seed, H=H_DEF, E_global=E_GLOBAL_DEF, skew=False, local_expert_offset=0):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(T, E_global, generator=g)
    bias = (torch.randn(E_global, generator=g) * 0.1)
    if skew:
        bias[local_expert_offset:local_expert_offset + 8] = 3.0
    bias = bias.to(torch.bfloat16)
    hs = _randn_fp8((T, H), g)
    hs_scale = torch.empty(H // BLOCK, T).uniform_(0.01, 0.1, generator=g)
    return {"routing_logits": logits, "routing_bias": bias,
            "hidden_states": hs, "hidden_states_scale": hs_scale}


def make_workload(name, T, seed, local_expert_offset=0, skew=False, H=H_DEF, I=I_DEF,
                  E_global=E_GLOBAL_DEF, E_local=E_LOCAL_DEF, weight_seed=WEIGHT_SEED,
                  routed_scaling_factor=2.5, routing=(8, 4, 8)) -> Workload:
    tens = make_tokens(T, seed, H, E_global, skew, local_expert_offset)
    tens.update(make_weights(H, I, E_local, weight_seed))
    return Workload(name=name, T=T, seed=seed, local_expert_offset=local_expert_offset,
                    skew=skew, routed_scaling_factor=routed_scaling_factor, tensors=tens,
                    routing=tuple(routing))


def make_for(defn, name, T, seed, **kw) -> Workload:
    """A workload for a shapes.Definition: its H, I, local and global expert
    counts and routing parameters."""
    return make_workload(name, T, seed, H=defn.H, I=defn.I, E_global=defn.EG, E_local=defn.EL,
                         routing=(defn.NG, defn.KG, defn.TOPK), **kw)


# The five workload families of the benchmark definition (T, offsets, skew).
STANDARD = {
    "c0_t16": dict(T=16, seed=100, local_expert_offset=0),
    "c1_t1": dict(T=1, seed=101, local_expert_offset=0),
    # one token with two local slots (experts 10 and 23): single-token decode
    # that streams two experts' weights (seed 101 routes its token elsewhere)
    "c1_t1_local": dict(T=1, seed=121, local_expert_offset=0),
    "c1_t4": dict(T=4, seed=102, local_expert_offset=0),
    "c1_t16": dict(T=16, seed=103, local_expert_offset=0),
    "c1_t64": dict(T=64, seed=104, local_expert_offset=0),
    "t256": dict(T=256, seed=111, local_expert_offset=0),
    "c2_t1024_o0": dict(T=1024, seed=105, local_expert_offset=0),
    "c2_t1024_o64": dict(T=1024, seed=106, local_expert_offset=64),
    "c2_t1024_o128": dict(T=1024, seed=107, local_expert_offset=128),
    "c2_t1024_o224": dict(T=1024, seed=108, local_expert_offset=224),
    "c3_t8192": dict(T=8192, seed=109, local_expert_offset=0),
    "c4_t14000_skew": dict(T=14000, seed=110, local_expert_offset=0, skew=True),
}


def standard(name, **over) -> Workload:
    kw = dict(STANDARD[name])
    kw.update(over)
    return make_workload(name, **kw)


def standard_tokens(name, **over) -> Workload:
    """A standard workload's per-token tensors only (no weights)."""
    kw = dict(STANDARD[name])
    kw.update(over)
    T, seed = kw["T"], kw["seed"]
    off, skew = kw.get("local_expert_offset", 0), kw.get("skew", False)
    return Workload(name=name, T=T, seed=seed, local_expert_offset=off, skew=skew,
                    tensors=make_tokens(T, seed, skew=skew, local_expert_offset=off))


def sha256(t: torch.Tensor) -> str:
    """SHA-256 of a CPU tensor's raw bytes."""
    t = t.contiguous().reshape(-1)
    return hashlib.sha256(t.view(torch.uint8).numpy().tobytes()).hexdigest()
