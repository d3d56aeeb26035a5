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


def device_weights(device="cuda"):
    if device not in _DEV_WEIGHTS:
        t0 = time.time()
        w = W.make_weights()
        _DEV_WEIGHTS[device] = {k: v.to(device) for k, v in w.items()}
        log(f"weights generated and copied in {time.time() - t0:.1f}s")
    return _DEV_WEIGHTS[device]


def gpu_args(wl: W.Workload, device="cuda"):
    dw = device_weights(device)
    t = wl.tensors
    return [t["routing_logits"].to(device), t["routing_bias"].to(device),
            t["hidden_states"].to(device), t["hidden_states_scale"].to(device),
            dw["gemm1_weights"], dw["gemm1_weights_scale"], dw["gemm2_weights"],
            dw["gemm2_weights_scale"], wl.local_expert_offset, wl.routed_scaling_factor]


def run_gpu(wl: W.Workload, device="cuda", fill=None):
    from flashinfer_amd import kernel
    args = gpu_args(wl, device)
    out = torch.empty(wl.T, W.H_DEF, dtype=torch.bfloat16, device=device)
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
    return R.moe_forward(*subset_args(wl, tokens))


def spread_tokens(T: int, n: int) -> torch.Tensor:
    """n token indices spread over [0, T), always including the first and last."""
    if T <= n:
        return torch.arange(T)
    idx = torch.linspace(0, T - 1, n).round().long()
    return torch.unique(idx)
