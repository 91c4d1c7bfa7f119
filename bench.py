#!/usr/bin/env python3
"""Fused-MoE layer benchmark on one MI355X.

A step is one MoE layer call over one batch of T synthetic tokens already
resident in HBM: routing (softmax top-k or grouped sigmoid top-k) followed by
XpuFusedMoe.apply (alignment, w13 grouped GEMM + fused activation, w2 grouped
GEMM, weighted top-k reduction).  The headline line is configuration C3
(DeepSeek-V3 shape, fp8 e4m3 weights with 128x128 block scales, T=8192), the
largest single-GPU configuration; the other BASELINE configurations are
reported in the same JSON line under "sweep".

Timed region: W eager warm-up steps, then K steps captured in one HIP graph
and replayed once between two events (torch.cuda.synchronize on both sides).
When one step's weights and activations are smaller than 512 MB (decode
points), consecutive steps rotate over several copies of the expert weights
(each an XpuFusedMoe of its own), so that the weights come from HBM rather
than from the 256 MB last-level cache.  Stage durations for the roofline come
from a second, eager pass (rotating the same way) in which the library records
HIP events around each of its launches on the same stream
(mi355moe_fused_moe_timed).

Only the cpu_baseline leg imports the CPU oracle (oracle/), and only to time
it as the reported baseline.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "vllm-xpu-kernels_amd"))
sys.path.insert(0, ROOT)

import torch  # noqa: E402


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemm_work(cfg, T, active, which):
    """Algorithmic (bytes, flops) of one grouped-GEMM launch."""
    H, I, k = cfg.hidden, cfg.inter, cfg.topk
    slots = T * k
    if cfg.recipe == "bf16":
        bw, sc, bx, sx = 2.0, 0.0, 2.0, 0.0
    elif cfg.recipe == "fp8block":
        bw, sc, bx, sx = 1.0, 4.0 / (128 * 128), 1.0, 4.0 / 128
    elif cfg.recipe == "mxfp8":
        bw, sc, bx, sx = 1.0, 1.0 / 32, 1.0, 1.0 / 32
    elif cfg.recipe == "fp8":    # per-expert e4m3 weights, 16-bit activations
        bw, sc, bx, sx = 1.0, 0.0, 2.0, 0.0
    elif cfg.recipe == "int4":   # u4 + a 16-bit scale per 128 along K
        bw, sc, bx, sx = 0.5, 2.0 / 128, 2.0, 0.0
    elif cfg.prequant:   # e2m1 x e2m1
        bw, sc, bx, sx = 0.5, 1.0 / 32, 0.5, 1.0 / 32
    else:
        bw, sc, bx, sx = 0.5, 1.0 / 32, 2.0, 0.0
    if which == "gemm_w13":
        n = 2 * I * H
        b = active * (n * (bw + sc) + (2 * 2 * I if cfg.bias else 0))
        b += T * H * (bx + sx) + slots * I * (bx + sx)
        f = 2.0 * slots * n
    else:
        n = H * I
        b = active * (n * (bw + sc) + (2 * H if cfg.bias else 0))
        b += slots * I * (bx + sx) + slots * H * 2
        f = 2.0 * slots * n
    return b, f


def _oracle_inputs(cfg, w, x, tw, ti):
    """CPU copies of only the experts the given tokens route to, ids remapped
    to that compact set (nk layouts)."""
    ti_c = ti.cpu().long()
    used = torch.unique(ti_c)
    remap = torch.full((cfg.experts,), -1, dtype=torch.long)
    remap[used] = torch.arange(used.numel())
    ids = remap[ti_c]
    u = used.to(w.w13.device)
    if cfg.recipe in ("bf16", "fp8"):   # reference layout [E, K, N]
        w13 = w.w13.index_select(0, u).transpose(1, 2).contiguous().cpu()
        w2 = w.w2.index_select(0, u).transpose(1, 2).contiguous().cpu()
    else:
        w13 = w.w13.view(torch.uint8).index_select(0, u).cpu()
        w2 = w.w2.view(torch.uint8).index_select(0, u).cpu()
        if cfg.recipe == "fp8block":
            w13, w2 = w13.view(torch.float8_e4m3fn), w2.view(torch.float8_e4m3fn)
    pick = lambda t: t.index_select(0, u).cpu() if t is not None else None  # noqa: E731
    return (x.cpu(), w13, pick(w.w13_scale), pick(w.w13_bias), w2,
            pick(w.w2_scale), pick(w.w2_bias), tw.cpu(), ids)


def host_cpu():
    """(model name, physical cores, logical CPUs) of this host from
    /proc/cpuinfo, and the CPUs this process may run on."""
    model, cores, logical = "unknown", set(), 0
    try:
        phys = core = None
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "processor":
                    logical += 1
                elif k == "model name":
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                    cores.add((phys, core))
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count()
    return model, len(cores) or None, logical or os.cpu_count(), usable


def cpu_baseline(cfg, w, x, tw, ti, n_tok, budget_s=20.0, warmup=True):
    """Times the CPU oracle (torch on the host cores) on the first n_tok
    tokens of the workload (all of them: the whole timed batch): an optional
    warm-up run, then the median of up to 5 runs within the budget (at least
    one)."""
    from oracle import moe_oracle as O
    T = x.shape[0]
    args = _oracle_inputs(cfg, w, x[:n_tok], tw[:n_tok], ti[:n_tok])
    if warmup:
        O.fused_moe(cfg.recipe, *args, activation=cfg.activation)
    times = []
    t_start = time.time()
    while len(times) < 5 and (not times or (time.time() - t_start) < budget_s):
        t0 = time.perf_counter()
        O.fused_moe(cfg.recipe, *args, activation=cfg.activation)
        times.append(time.perf_counter() - t0)
        log(f"cpu baseline: {n_tok} tokens in {times[-1]:.2f} s")
    med = statistics.median(times)
    model, phys, logical, usable = host_cpu()
    which = (f"all T={T} tokens of the timed batch" if n_tok == T
             else f"the first {n_tok} of the timed batch's T={T} tokens")
    return {"value": n_tok / med, "unit": "tokens/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{cfg.name} ({cfg.recipe}) {which} (their {int(args[-1].max()) + 1} "
                      f"experts, weights dequantised per expert inside the loop), "
                      f"oracle/moe_oracle.py fused_moe, median of {len(times)} run(s)"
                      f"{' after a warm-up run' if warmup else ' (weights already in host memory)'}"
                      f", {med * 1e3:.1f} ms per run; host CPU {model}, {phys} physical cores / "
                      f"{logical} logical CPUs, {usable} usable by this process, torch "
                      f"threads {torch.get_num_threads()}"}


ROTATE_BYTES = 512e6   # 2x the MI355X last-level cache (256 MB MALL)
MAX_COPIES = 8


class Point:
    def __init__(self, cfg, T, dev, weights=None, rotate_bytes=ROTATE_BYTES):
        from vllm_xpu_kernels import workloads as W
        from vllm_xpu_kernels.fused_moe_interface import XpuFusedMoe
        self.cfg, self.T, self.dev = cfg, T, dev
        self.w = weights if weights is not None else W.make_weights(cfg, dev)
        self.x = W.make_activations(cfg, T, dev)
        self.logits = W.make_router_logits(cfg, T, dev)
        self.bias = (W.make_correction_bias(cfg, dev)
                     if cfg.routing == "grouped_sigmoid" else None)
        w = self.w
        self.out = torch.empty_like(self.x)
        self.tw, self.ti = W.route(cfg, self.logits, self.bias)
        self.active = int(torch.unique(self.ti).numel())
        # steps rotate over enough layers, each on its own copy of the weights
        # (prepared in place), that one pass over them exceeds rotate_bytes;
        # self.w keeps the reference layouts for the CPU baseline
        per_step = W.algorithmic_bytes(cfg, T, self.active)
        self.copies = int(min(MAX_COPIES, max(1, math.ceil(rotate_bytes / per_step))))
        self.moes = [XpuFusedMoe(*w.layer_args(copy=True), cfg.topk, cfg.activation,
                                 cfg.experts)
                     for _ in range(self.copies)]
        self.moe = self.moes[0]
        self.i = 0
        # pre-quantised mxfp4 input (w4a4): e2m1 bytes [T, H/2] + e8m0 [T, H/32]
        self.xq = self.xs8 = None
        if cfg.prequant:
            from vllm_xpu_kernels import ops
            q, sc = ops.per_token_group_quant_mxfp4(self.x, 32)
            self.xq = q.view(torch.uint8)
            self.xs8 = (torch.log2(sc).round().to(torch.int32) + 127).to(torch.uint8)

    def step(self):
        from vllm_xpu_kernels import workloads as W
        tw, ti = W.route(self.cfg, self.logits, self.bias)
        moe = self.moes[self.i % self.copies]
        if self.xq is not None:
            moe.apply(self.out, self.xq.view(torch.float4_e2m1fn_x2), tw, ti,
                      a1q_scale=self.xs8.view(torch.float8_e8m0fnu))
        else:
            moe.apply(self.out, self.x, tw, ti)
        self.i += 1

    def time_steps(self, steps, warmup, graph=True):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(warmup):
                self.step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        if graph:
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                for _ in range(steps):
                    self.step()
            g.replay()
            torch.cuda.synchronize()
            e0.record()
            g.replay()
            e1.record()
            torch.cuda.synchronize()
            del g
        else:
            e0.record()
            for _ in range(steps):
                self.step()
            e1.record()
            torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    def stage_times(self, steps):
        from vllm_xpu_kernels import capi
        x = self.xq if self.xq is not None else self.x
        args = [capi.fused_args(m, self.out, x, self.tw, self.ti, hidden_scale=self.xs8)
                for m in self.moes]
        ws = capi.workspace_for(args[0], self.dev)
        timer = capi.StageTimer(steps)
        try:
            torch.cuda.synchronize()
            try:   # give the host a head start so no stage waits for a launch
                torch.cuda._sleep(int(5e6))
            except Exception:
                pass
            for i in range(steps):
                timer.run(args[i % len(args)], ws, i)
            torch.cuda.synchronize()
            per = [timer.stage_ms(i) for i in range(steps)]
        finally:
            timer.close()
        return [statistics.mean(p[j] for p in per) for j in range(capi.FUSED_STAGES)]


def summarize(pt, ms, stages):
    from vllm_xpu_kernels import capi
    from vllm_xpu_kernels import workloads as W
    cfg, T = pt.cfg, pt.T
    t_h, t_m = W.roofline_time_s(cfg, T, pt.active)
    t = ms * 1e-3
    d = {"config": cfg.name, "recipe": cfg.recipe + (" (pre-quantised mxfp4 input)"
                                                     if cfg.prequant else ""),
         "tokens": T, "active_experts": pt.active,
         "us_per_layer": round(ms * 1e3, 2), "tokens_per_s": round(T / t, 1),
         "hbm_GBps": round(W.algorithmic_bytes(cfg, T, pt.active) / t / 1e9, 1),
         "TFLOPs": round(W.algorithmic_flops(cfg, T) / t / 1e12, 2),
         "roofline_frac": round(max(t_h, t_m) / t, 4),
         "bound": "hbm" if t_h >= t_m else "mfma",
         "weight_copies": pt.copies,
         "stage_us": {n: round(v * 1e3, 2) for n, v in zip(capi.STAGE_NAMES, stages)}}
    return d


def measured_traffic(key, stage):
    """HBM bytes per launch of a GEMM stage from the committed rocprofv3
    summaries (profiles/*.txt lines "traffic[<config> T=<tokens> <stage>] = N":
    FETCH_SIZE and WRITE_SIZE of separate --pmc runs, each scaled by what the
    counter reads for a plain copy of known size); None when no summary covers
    this workload."""
    import glob
    import re
    pat = re.compile(r"^traffic\[" + re.escape(f"{key} {stage}") + r"\] = (\d+)")
    for path in sorted(glob.glob(os.path.join(ROOT, "profiles", "*.txt"))):
        with open(path) as fh:
            for line in fh:
                m = pat.match(line)
                if m:
                    return int(m.group(1))
    return None


def kernel_roofline(pt, stages, key):
    from vllm_xpu_kernels import capi
    from vllm_xpu_kernels import workloads as W
    names = capi.STAGE_NAMES
    gi = max((2, 3), key=lambda i: stages[i])
    name = names[gi]
    ms = stages[gi]
    traffic = measured_traffic(key, name)
    b, f = gemm_work(pt.cfg, pt.T, pt.active, name)
    peak_tf = W.PEAK_TFLOPS_FP4 if pt.cfg.prequant else W.PEAK_TFLOPS[pt.cfg.recipe]
    t_h, t_m = b / 8e12, f / (peak_tf * 1e12)
    if t_h >= t_m:
        ach = b / (ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(ach, 1), "peak": 8000.0, "unit": "GB/s",
                "frac": round(ach / 8000.0, 4), "traffic": traffic, "kernel": name,
                "bytes_per_launch": int(b), "flops_per_launch": int(f),
                "ms_per_launch": round(ms, 5)}
    ach = f / (ms * 1e-3) / 1e12
    return {"bound": "mfma", "achieved": round(ach, 2), "peak": peak_tf, "unit": "TFLOP/s",
            "frac": round(ach / peak_tf, 4), "traffic": traffic, "kernel": name,
            "bytes_per_launch": int(b), "flops_per_launch": int(f),
            "ms_per_launch": round(ms, 5)}


SWEEP = [("C1", 64), ("C2", 1), ("C2", 16), ("C2", 64), ("C2", 256), ("C2", 4096),
         ("C3", 1), ("C3", 64), ("C3", 8192), ("C4", 2048), ("C5", 1), ("C5", 128),
         ("C5", 4096),
         # recipe variants on the same shapes: mxfp8 weights, w4a4 (e2m1 x e2m1),
         # per-expert fp8 (the e4m3 weights read as such), int4 (w4a16)
         ("C3-mxfp8", 8192), ("C5-w4a4", 4096), ("C3-fp8", 1), ("C2-int4", 4096)]


def op_bandwidth(dev, steps):
    """Standalone ops of the path at the shapes they see inside the layers
    (C3 DeepSeek-V3 T=8192: 65536 slots, I=2048, H=7168; C5 gpt-oss-20b
    T=4096: 16384 slots, I=2880; C2 Qwen3-30B-A3B T=4096: 32768 slots,
    I=768): algorithmic bytes (inputs read once, outputs written once) over
    the mean time of `steps` launches between HIP events on torch's current
    stream, which the ops launch on."""
    from vllm_xpu_kernels import ops
    g = torch.Generator(device=dev).manual_seed(3)

    def rnd(*shape):
        return torch.randn(*shape, generator=g, device=dev).bfloat16()

    cases = [
        ("silu_and_mul_per_block_quant e4m3 g128", (65536, 2048),
         lambda x: ops.silu_and_mul_per_block_quant(x, 128, torch.float8_e4m3fn),
         lambda T, H: T * 2 * H * 2 + T * H + T * (H // 128) * 4),
        ("silu_and_mul_mxfp4_quant", (16384, 2880),
         lambda x: ops.silu_and_mul_mxfp4_quant(x),
         lambda T, H: T * 2 * H * 2 + T * H // 2 + T * (H // 32) * 4),
        ("silu_and_mul", (32768, 768), lambda x: ops.silu_and_mul(x),
         lambda T, H: T * 2 * H * 2 + T * H * 2),
        ("per_token_group_fp8_quant g128", (8192, 7168 // 2),
         lambda x: ops.per_token_group_fp8_quant(x, 128),
         lambda T, H: T * 2 * H * 2 + T * 2 * H + T * (2 * H // 128) * 4),
    ]
    out = []
    for name, (T, H), fn, nbytes in cases:
        x = rnd(T, 2 * H)
        for _ in range(3):
            fn(x)
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(steps):
            fn(x)
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / steps
        gbps = nbytes(T, H) / us / 1e3
        out.append({"op": name, "input": [T, 2 * H], "bytes": nbytes(T, H),
                    "us": round(us, 2), "GBps": round(gbps, 1),
                    "hbm_frac": round(gbps / 8000.0, 3)})
        del x
    out += prologue_bandwidth(dev, steps, g)
    out += index_op_latency(dev, steps, g)
    return out


def index_op_latency(dev, steps, g):
    """Latency of the index-only ops (bytes are small; "bytes" counts the
    index arrays read and written once): moe_lora_align_block_size at the
    reference test's largest case (T=4096, k=6, E=512, 32 adapters) and
    topk_softplus_sqrt at C3's routing shape (T=8192, E=256, k=8)."""
    from vllm_xpu_kernels import ops
    out = []
    T, k, E, L, bs = 4096, 6, 512, 32, 16
    ids = torch.stack([torch.randperm(E, device=dev, generator=g)[:k] for _ in range(T)]).int()
    tok = torch.randint(0, L, (T,), generator=g, device=dev, dtype=torch.int32)
    mx = (ids.numel() + E * (bs - 1) + bs - 1) // bs * bs
    nb = mx // bs
    srt = torch.empty(L * mx, dtype=torch.int32, device=dev)
    eid = torch.empty(L * nb, dtype=torch.int32, device=dev)
    ntp = torch.empty(L, dtype=torch.int32, device=dev)
    en = torch.ones(L + 1, dtype=torch.int32, device=dev)
    lids = torch.arange(L + 1, dtype=torch.int32, device=dev)
    logits = torch.randn(8192, 256, generator=g, device=dev)
    cases = [("moe_lora_align_block_size T=4096 k=6 E=512 32 adapters", [T, k, E, L],
              lambda: ops.moe_lora_align_block_size(ids, tok, E, bs, L, mx, nb, srt, eid, ntp,
                                                    en, lids),
              ids.numel() * 4 + T * 4 + (srt.numel() + eid.numel()) * 4),
             ("topk_softplus_sqrt T=8192 E=256 k=8", [8192, 256, 8],
              lambda: ops.topk_softplus_sqrt(logits, 8, True, 2.5),
              logits.numel() * 4 + 8192 * 8 * 8)]
    for name, shape, fn, nbytes in cases:
        for _ in range(3):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / steps
        out.append({"op": name, "input": shape, "bytes": nbytes, "us": round(us, 2),
                    "GBps": round(nbytes / us / 1e3, 1),
                    "hbm_frac": round(nbytes / us / 1e3 / 8000.0, 3)})
    return out


def prologue_bandwidth(dev, steps, g):
    """fused_moe_prologue at C3's T=8192 (fp8 block-scaled activations,
    H=7168, k=8 of 256 experts) and at the reference test's largest case
    (bf16, T=8192, H=8192, k=2 of 16).  Algorithmic bytes: every input row
    and scale row read once, every routed row written once, the ids and
    token scales read, the four per-row index/scale entries written."""
    from vllm_xpu_kernels import capi, ops
    out = []
    for name, T, H, k, E, fp8 in (("fused_moe_prologue fp8block C3", 8192, 7168, 8, 256, True),
                                  ("fused_moe_prologue bf16 ref-test", 8192, 8192, 2, 16, False)):
        x = torch.randn(T, H, generator=g, device=dev)
        x = x.to(torch.float8_e4m3fn) if fp8 else x.bfloat16()
        sc = torch.rand(T, H // 128, generator=g, device=dev) if fp8 else None
        ids = torch.stack([torch.randperm(E, device=dev, generator=g)[:k] for _ in range(T)])
        fs = torch.rand(T, k, generator=g, device=dev)
        eb, sb, bk = (1, 4, 128) if fp8 else (2, 0, 1)
        total, _ = capi.prologue_layout(T, k, H, eb, bk, sb, E)
        ws = torch.empty(total, dtype=torch.uint8, device=dev)

        def fn():
            ops.fused_moe_prologue(x, sc, ids, fs, ws, H, 2048, bk, 0, 1, E)
        for _ in range(3):
            fn()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        for _ in range(steps):
            fn()
        b.record()
        torch.cuda.synchronize()
        us = a.elapsed_time(b) * 1e3 / steps
        N = T * k
        row = H * eb + (H // bk) * sb
        nbytes = T * row + N * row + N * (8 + 4) + N * 16 + (E + 1) * 8
        gbps = nbytes / us / 1e3
        out.append({"op": name, "input": [T, H, k, E], "bytes": nbytes,
                    "us": round(us, 2), "GBps": round(gbps, 1),
                    "hbm_frac": round(gbps / 8000.0, 3)})
        del x, ws
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="C3")
    ap.add_argument("--tokens", type=int, default=8192)
    ap.add_argument("--cpu-tokens", type=int, default=0,
                    help="tokens of the CPU baseline (0: the whole batch); a 16-token "
                         "sample is reported beside it")
    ap.add_argument("--sweep", default="default",
                    help="'none', 'default' or a list like C3:1,C3:8192")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-ops", action="store_true",
                    help="skip the standalone-op bandwidth table")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB 5 times (the "
                         "known-size kernel that scales rocprofv3 FETCH_SIZE / "
                         "WRITE_SIZE readings)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build runs the MoE layer on a "
              "single MI355X (no collectives); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        n = args.copy_calibration << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n,
                          "launches": 5}), flush=True)
        return

    from vllm_xpu_kernels import workloads as W
    graph = not args.no_graph
    cfg = W.config(args.config)
    log(f"bench: {args.config} ({cfg.name}) T={args.tokens} steps={args.steps} "
        f"warmup={args.warmup} graph={graph} on {torch.cuda.get_device_name(0)}")

    pt = Point(cfg, args.tokens, dev)
    ms = pt.time_steps(args.steps, args.warmup, graph)
    stages = pt.stage_times(args.steps)
    head = summarize(pt, ms, stages)
    log("headline:", json.dumps(head))
    roof = kernel_roofline(pt, stages, f"{args.config} T={args.tokens}")
    head["kernel_roofline"] = roof
    cpu = None
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        n_cpu = min(args.cpu_tokens or args.tokens, args.tokens)
        # the whole batch once (about 20 s of host work at C3 T=8192), and a
        # 16-token sample, median of up to 5 runs
        cpu = cpu_baseline(cfg, pt.w, pt.x, pt.tw, pt.ti, n_tok=n_cpu, budget_s=0.0,
                           warmup=False)
        if n_cpu > 16:
            small = cpu_baseline(cfg, pt.w, pt.x, pt.tw, pt.ti, n_tok=16)
            cpu["small_sample"] = {"value": small["value"], "unit": small["unit"],
                                   "sample": small["sample"]}
        log("cpu baseline:", json.dumps(cpu))

    op_table = None
    if not args.no_ops:
        op_table = op_bandwidth(dev, max(args.steps, 10))
        for d in op_table:
            log("op:", json.dumps(d))

    sweep = []
    if args.sweep != "none":
        pts = SWEEP if args.sweep == "default" else [
            (s.split(":")[0], int(s.split(":")[1])) for s in args.sweep.split(",")]
        cache = {args.config: pt.w}
        for name, T in pts:
            if name == args.config and T == args.tokens:
                sweep.append(head)
                continue
            c = W.config(name)
            if name not in cache:
                for k in list(cache):
                    if k != name:
                        del cache[k]
                torch.cuda.empty_cache()
                cache[name] = W.make_weights(c, dev)
            p = Point(c, T, dev, weights=cache[name])
            m = p.time_steps(args.steps, args.warmup, graph)
            st = p.stage_times(args.steps)
            d = summarize(p, m, st)
            d["kernel_roofline"] = kernel_roofline(p, st, f"{name} T={T}")
            log("sweep:", json.dumps(d))
            sweep.append(d)
            del p

    line = {
        "metric": "fused-MoE layer tokens/s",
        "value": head["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": ("mxfp4xmxfp4" if cfg.prequant else
                  {"bf16": "bf16", "fp8block": "fp8e4m3", "mxfp4": "mxfp4xbf16",
                   "mxfp8": "mxfp8e4m3", "fp8": "e4m3xbf16", "int4": "int4xbf16"}[cfg.recipe]),
        "data": "synthetic (seeded N(0,1) activations/logits, N(0,0.02) weights; random init)",
        "config": {"workload": f"{args.config} {cfg.name} fused MoE layer, T={args.tokens}",
                   "tokens": args.tokens, "hidden": cfg.hidden, "inter": cfg.inter,
                   "experts": cfg.experts, "active_experts": head["active_experts"],
                   "topk": cfg.topk, "recipe": cfg.recipe,
                   "routing": cfg.routing, "graph": graph, "parallelism": "none (1 GPU)"},
        "layer_roofline_frac": head["roofline_frac"],
        "hbm_GBps": head["hbm_GBps"],
        "TFLOPs": head["TFLOPs"],
        "stage_us": head["stage_us"],
        "roofline": roof,
        "cpu_baseline": cpu,
        "ops": op_table,
        "sweep": sweep,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
