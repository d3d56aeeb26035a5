"""Writes the golden fixtures under tests/golden/ (run from the repo root):

    python tests/golden/make_golden.py

* tiny_t24.npz: a tiny-shape workload (H=256, I=128, 32 local experts of
  256, T=24, offset 64, seeds 11 / weight seed 99): the oracle's fp64
  accumulator and routing. Inputs are regenerated from the seeds.
* c0_t16.npz + c0_t16.json: the real-shape decode workload c0_t16 (T=16,
  H=7168, I=2048): SHA-256 of every generated input tensor, the oracle's
  routing (ids in selection order, weights) and its bf16 output as uint16.

The reference ships no fixtures of its own; these pin the seeded generator
and the oracle across machines, and give the GPU tests a stored answer.
"""
import json
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from flashinfer_amd import workloads as W  # noqa: E402
from oracle import ref_moe as R  # noqa: E402

TENSORS = ["routing_logits", "routing_bias", "hidden_states", "hidden_states_scale",
           "gemm1_weights", "gemm1_weights_scale", "gemm2_weights", "gemm2_weights_scale"]


def tiny_workload():
    return W.make_workload("tiny", T=24, seed=11, local_expert_offset=64, H=256, I=128,
                           weight_seed=99)


def main():
    wl = tiny_workload()
    res = R.moe_forward(*wl.args(), acc_dtype=torch.float64)
    np.savez(os.path.join(HERE, "tiny_t24.npz"), acc=res.acc.numpy(),
             ids=res.route.ids.numpy().astype(np.int32), weights=res.route.weights.numpy())

    wl = W.standard("c0_t16")
    hashes = {n: W.sha256(wl.tensors[n]) for n in TENSORS}
    res = R.moe_forward(*wl.args())
    np.savez(os.path.join(HERE, "c0_t16.npz"),
             output_bf16_bits=res.output.view(torch.int16).numpy(),
             ids=res.route.ids.numpy().astype(np.int32), weights=res.route.weights.numpy())
    with open(os.path.join(HERE, "c0_t16.json"), "w") as f:
        json.dump({"workload": "c0_t16", "T": wl.T, "seed": wl.seed,
                   "weight_seed": W.WEIGHT_SEED, "local_expert_offset": wl.local_expert_offset,
                   "routed_scaling_factor": wl.routed_scaling_factor, "sha256": hashes}, f, indent=1)
    print("wrote", os.listdir(HERE))


if __name__ == "__main__":
    main()
