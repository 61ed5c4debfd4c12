#!/usr/bin/env python3
"""Benchmark of the TQ4 quantised-KV hot path on one MI355X.

Workload (the metric's "@ctx4096"): single-sequence
TQ4 paged decode, batch 1, 32 q heads : 8 kv heads, head_dim 128, ctx 4096,
page 16, random block table from a 4096-page pool, scale 1/sqrt(128); the
cache is prefilled through the GPU reshape_and_cache from N(0,1) BF16 K/V.
A step is one fused decode launch (partials + last-workgroup LSE combine +
inverse rotation + BF16 store). Cold cache by default: a 1 GiB buffer is
rewritten between steps (outside the timed events) so the 256 MiB Infinity
Cache holds nothing of the working set; each decode is bracketed by HIP
events on the launch stream and value = algorithmic bytes / mean decode time.

Also reported: reshape_and_cache tokens/s on BASELINE config 2 (1024 BF16
tokens, 4096-page pool, permuted pages), and the CPU baseline -- the C
oracle's decode of the same workload on the host cores (kind "port").

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--cache cold|warm]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published

B, HQ, HKV, D, S, CTX, POOL = 1, 32, 8, 128, 16, 4096, 4096


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_algorithmic_bytes(ctx_lens, hq, hkv, d, s):
    """Bytes the contract forces across HBM for one decode step: K+V nibbles
    and both FP32 scales of every live token, the block-table entries, the
    context lengths, q and out (BF16)."""
    per_token = hkv * (d + 8)  # d/2 key + d/2 value bytes + 2 x 4-byte scales per kv head
    kv = sum(ctx_lens) * per_token
    tables = sum((c + s - 1) // s for c in ctx_lens) * 4
    qo = 2 * len(ctx_lens) * hq * d * 2
    return kv + tables + qo + 4 * len(ctx_lens)


def writer_algorithmic_bytes(tokens, hkv, d, in_bytes):
    """Inputs read + packed nibbles + scales written + slot mapping read."""
    return tokens * (2 * hkv * d * in_bytes + hkv * d + 2 * hkv * 4 + 4)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cache", choices=("cold", "warm"), default="cold")
    ap.add_argument("--splits", type=int, default=0, help="0 = auto")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the TQ4 path is "
              "single-GPU in this build and no multi-GPU figure is produced.", file=sys.stderr)
        sys.exit(2)

    import torch

    import __graft_entry__
    tq4 = __graft_entry__.package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    rng = np.random.default_rng(0x71340003)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x71340003)

    # ---- cache: prefill ctx tokens of N(0,1) K/V through the GPU writer
    signs_np = np.array([-1.0 if ((c * c + 3 * c + 1) % 7) < 3 else 1.0 for c in range(D)],
                        np.float32)
    signs = torch.from_numpy(signs_np).to(dev)
    isl = 1.0 / math.sqrt(D)
    scale = 1.0 / math.sqrt(D)
    nbytes = POOL * HKV * S * D // 2
    kc = torch.zeros(nbytes, dtype=torch.int8, device=dev)
    vc = torch.zeros(nbytes, dtype=torch.int8, device=dev)
    sc = torch.zeros(2 * POOL * HKV * S, dtype=torch.float32, device=dev)
    pages = torch.from_numpy(rng.permutation(POOL)[: CTX // S].astype(np.int32)).to(dev)
    slots = (pages[:, None] * S + torch.arange(S, device=dev, dtype=torch.int32)[None, :]).reshape(-1)
    k_in = torch.randn((CTX, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
    v_in = torch.randn((CTX, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
    tq4.reshape_and_cache_bf16(k_in, v_in, kc, vc, sc, slots.contiguous(), pi_signs=signs,
                               num_blocks=POOL, block_size=S, inv_sqrt_len=isl)
    tables = pages[None, :].contiguous()
    ctx = torch.tensor([CTX], dtype=torch.int32, device=dev)
    q = torch.randn((B, HQ, D), generator=gen, device=dev).to(torch.bfloat16)
    out = torch.empty_like(q)
    splits = args.splits or tq4.auto_splits(B, HKV, tables.shape[1], S)
    ws = tq4.decode_workspace(B, HQ, HKV, D, splits)
    flush = torch.empty(1 << 30, dtype=torch.uint8, device=dev) if args.cache == "cold" else None
    torch.cuda.synchronize()

    def decode():
        tq4.paged_decode(q, kc, vc, sc, tables, ctx, signs, HKV, S, POOL, out=out, workspace=ws,
                         num_splits=splits, scale=scale, inv_sqrt_len=isl)

    def timed_steps(fn, steps, warmup):
        for _ in range(warmup):
            if flush is not None:
                flush.zero_()
            fn()
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(steps)]
        t0 = time.perf_counter()
        for e0, e1 in ev:
            if flush is not None:
                flush.zero_()
            e0.record()
            fn()
            e1.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms = np.array([e0.elapsed_time(e1) for e0, e1 in ev])
        return ms, wall

    log(f"decode: B={B} Hq={HQ} Hkv={HKV} d={D} ctx={CTX} splits={splits} cache={args.cache}")
    ms, wall = timed_steps(decode, args.steps, args.warmup)
    dec_bytes = decode_algorithmic_bytes([CTX], HQ, HKV, D, S)
    mean_ms = float(ms.mean())
    gbs = dec_bytes / (mean_ms * 1e-3) / 1e9
    log(f"decode: mean {mean_ms * 1e3:.2f} us  median {np.median(ms) * 1e3:.2f} us  "
        f"min {ms.min() * 1e3:.2f} us  p99 {np.percentile(ms, 99) * 1e3:.2f} us  "
        f"-> {gbs:.1f} GB/s ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak)")

    # ---- reshape_and_cache rate, BASELINE config 2 (1024 BF16 tokens, permuted pages)
    wt = 1024
    w_pages = torch.from_numpy(rng.permutation(POOL)[: wt // S].astype(np.int32)).to(dev)
    w_slots = (w_pages[:, None] * S + torch.arange(S, device=dev, dtype=torch.int32)[None, :]).reshape(-1).contiguous()
    wk = torch.randn((wt, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
    wv = torch.randn((wt, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
    wkc, wvc, wsc = torch.zeros_like(kc), torch.zeros_like(vc), torch.zeros_like(sc)

    def write():
        tq4.reshape_and_cache_bf16(wk, wv, wkc, wvc, wsc, w_slots, pi_signs=signs,
                                   num_blocks=POOL, block_size=S, inv_sqrt_len=isl)

    wms, _ = timed_steps(write, max(20, args.steps // 4), 5)
    w_mean = float(wms.mean())
    w_tps = wt / (w_mean * 1e-3)
    w_gbs = writer_algorithmic_bytes(wt, HKV, D, 2) / (w_mean * 1e-3) / 1e9
    log(f"reshape_and_cache: {wt} tokens mean {w_mean * 1e3:.2f} us -> {w_tps / 1e6:.1f} M tokens/s "
        f"({w_gbs:.1f} GB/s)")

    # ---- CPU baseline: the C oracle's decode of the same workload on host cores
    cpu = None
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(REPO, "tests"))
        from oracle_bindings import Oracle
        o = Oracle()
        threads = min(16, os.cpu_count() or 1)
        h_q = q.view(torch.int16).cpu().numpy().view(np.uint16)
        h_kc, h_vc, h_sc = kc.cpu().numpy(), vc.cpu().numpy(), sc.cpu().numpy()
        h_tab, h_ctx = tables.cpu().numpy(), ctx.cpu().numpy()
        iters, t0 = 0, time.perf_counter()
        while True:
            o.paged_decode(h_q, h_kc, h_vc, h_sc, h_tab, h_ctx, signs_np, None, HQ, HKV, D, S,
                           POOL, splits, np.float32(scale), np.float32(isl), 1, threads=threads)
            iters += 1
            el = time.perf_counter() - t0
            if el >= args.cpu_seconds:
                break
        cpu_gbs = dec_bytes * iters / el / 1e9
        cpu = {"value": round(cpu_gbs, 4), "unit": "GB/s", "cores": threads, "kind": "port",
               "sample": f"{iters} config-3 decodes (B=1, 32q:8kv, d128, ctx4096, {splits} splits) "
                         f"by oracle/tq4_oracle.c, {el:.1f} s, {threads} threads",
               "us_per_decode": round(el / iters * 1e6, 1)}
        log(f"cpu baseline: {cpu}")

    result = {
        "metric": "TQ4 paged decode µs + HBM GB/s (% peak) @ctx4096; reshape_and_cache tokens/s",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(mean_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4-cache/fp16-mfma/fp32-softmax",
        "data": "synthetic: N(0,1) BF16 K/V quantised by the GPU writer, N(0,1) BF16 q, seeded",
        "config": {"workload": "config3 single-sequence TQ4 paged decode",
                   "batch": B, "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "ctx": CTX,
                   "page_size": S, "pool_pages": POOL, "splits": splits,
                   "cache": args.cache, "parallelism": "single GPU"},
        "decode_us": {"mean": round(mean_ms * 1e3, 3), "median": round(float(np.median(ms)) * 1e3, 3),
                      "min": round(float(ms.min()) * 1e3, 3),
                      "p99": round(float(np.percentile(ms, 99)) * 1e3, 3)},
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "reshape_and_cache": {"tokens": wt, "us": round(w_mean * 1e3, 3),
                              "tokens_per_s": round(w_tps, 1), "GBps": round(w_gbs, 2)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "decode_kernel<128,1> (fused)",
                     "algorithmic_bytes": dec_bytes},
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
