"""Shared helpers for the GPU parity tests: cached device weights, a GPU call
of the operator, and the oracle on a subset of tokens (tokens are
independent, so slicing every per-token input gives the same rows)."""
from __future__ import annotations

import sys
import time

import torch

from flashinfer_amd import workloads as W

_DEV_WEIGHTS = {}


def log(msg: str) -> None:
    print(f"[{time.strftime('%H:%M:%S')}] {msg}", file=sys.stderr, flush=True)


def device_weights(device="cuda", H=W.H_DEF, I=W.I_DEF, E_local=W.E_LOCAL_DEF):
    """Device copies of the seeded weights of shape (H, I) for E_local experts,
    one set per device; another shape evicts the previous one."""
    key = (device, H, I, E_local)
    if key not in _DEV_WEIGHTS:
        for k in [k for k in _DEV_WEIGHTS if k[0] == device]:
            del _DEV_WEIGHTS[k]
        t0 = time.time()
        w = W.make_weights(H, I, E_local)
        _DEV_WEIGHTS[key] = {k: v.to(device) for k, v in w.items()}
        log(f"weights (H={H}, I={I}, {E_local} experts) generated and copied in "
            f"{time.time() - t0:.1f}s")
    return _DEV_WEIGHTS[key]


def gpu_args(wl: W.Workload, device="cuda"):
    t = wl.tensors
    w1 = t["gemm1_weights"]
    dw = device_weights(device, int(w1.shape[2]), int(w1.shape[1]) // 2, int(w1.shape[0]))
    return [t["routing_logits"].to(device), t["routing_bias"].to(device),
            t["hidden_states"].to(device), t["hidden_states_scale"].to(device),
            dw["gemm1_weights"], dw["gemm1_weights_scale"], dw["gemm2_weights"],
            dw["gemm2_weights_scale"], wl.local_expert_offset, wl.routed_scaling_factor]


def run_gpu(wl: W.Workload, device="cuda", fill=None):
    from flashinfer_amd import kernel
    args = gpu_args(wl, device)
    out = torch.empty(wl.T, wl.tensors["gemm1_weights"].shape[2], dtype=torch.bfloat16, device=device)
    if fill is not None:
        out.fill_(fill)
    kernel.run(*args, out)
    torch.cuda.synchronize()
    return out


def subset_args(wl: W.Workload, tokens: torch.Tensor):
    t = wl.tensors
    return [t["routing_logits"][tokens], t["routing_bias"], t["hidden_states"][tokens],
            t["hidden_states_scale"][:, tokens].contiguous(), t["gemm1_weights"],
            t["gemm1_weights_scale"], t["gemm2_weights"], t["gemm2_weights_scale"],
            wl.local_expert_offset, wl.routed_scaling_factor]


def oracle_subset(wl: W.Workload, tokens: torch.Tensor):
    from oracle import ref_moe as R
    ng, kg, k = wl.routing
    return R.moe_forward(*subset_args(wl, tokens), n_group=ng, topk_group=kg, top_k=k)


def spread_tokens(T: int, n: int) -> torch.Tensor:
    """n token indices spread over [0, T), always including the first and last."""
    if T <= n:
        return torch.arange(T)
    idx = torch.linspace(0, T - 1, n).round().long()
    return torch.unique(idx)
