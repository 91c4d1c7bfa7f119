"""Calibrates the router-logit temperature tau of configuration C4 so that the
busiest 10% of experts (13 of 128) receive 50% +- 2% of the 16384 top-8
assignments at T=2048 (logits = N(0,1) + tau * log p, p ~ rank^-1.1).
Prints the realised share for a few tau; the chosen value is committed as
ZIPF_TAU_C4 in vllm_xpu_kernels/workloads.py.  The logits come from the
generator of the device the bench and tests draw them on (argument: device,
default cuda when present), so the calibration holds for those draws."""
import os
import sys

import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "vllm-xpu-kernels_amd"))

from oracle import moe_oracle as O  # noqa: E402
from vllm_xpu_kernels import workloads as W  # noqa: E402


def share(tau, device, T=2048, E=128, k=8, seed=2):
    cfg = W.MoeConfig("c4", 4096, 1536, E, k, "fp8block", "softmax", zipf_tau=tau)
    logits = W.make_router_logits(cfg, T, device, seed).cpu()
    _, ids, _ = O.topk_softmax(logits, k, True)
    cnt = torch.bincount(ids.flatten().long(), minlength=E).sort(descending=True).values
    return float(cnt[:13].sum()) / (T * k)


if __name__ == "__main__":
    dev = sys.argv[1] if len(sys.argv) > 1 else ("cuda" if torch.cuda.is_available() else "cpu")
    for i in range(21):
        tau = 0.45 + 0.01 * i
        print(f"{dev} tau={tau:.3f} top10%-share={share(tau, dev):.4f}", flush=True)
