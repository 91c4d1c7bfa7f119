"""Calibrates the router-logit temperature tau of configuration C4 so that the
busiest 10% of experts (13 of 128) receive 50% +- 2% of the 16384 top-8
assignments at T=2048 (logits = N(0,1) + tau * log p, p ~ rank^-1.1).
Prints the realised share for a few tau; the chosen value is committed as
ZIPF_TAU_C4 in vllm_xpu_kernels/workloads.py."""
import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "vllm-xpu-kernels_amd"))

from oracle import moe_oracle as O  # noqa: E402
from vllm_xpu_kernels import workloads as W  # noqa: E402


def share(tau, T=2048, E=128, k=8, seed=2):
    cfg = W.MoeConfig("c4", 4096, 1536, E, k, "fp8block", "softmax", zipf_tau=tau)
    logits = W.make_router_logits(cfg, T, "cpu", seed)
    _, ids, _ = O.topk_softmax(logits, k, True)
    cnt = torch.bincount(ids.flatten().long(), minlength=E).sort(descending=True).values
    return float(cnt[:13].sum()) / (T * k)


if __name__ == "__main__":
    for tau in [0.5, 0.52, 0.535, 0.55, 0.6]:
        print(f"tau={tau:.2f} top10%-share={share(tau):.4f}")
