#!/usr/bin/env python3
"""Benchmark of the TQ4 quantised-KV hot path on one MI355X.

Headline workload (the metric's "@ctx4096"):
single-sequence TQ4 paged decode -- batch 1, 32 q heads : 8 kv heads,
head_dim 128, ctx 4096, page 16, random block table, scale 1/sqrt(128). A
step is one fused decode launch (split-K partials + last-workgroup LSE
combine + inverse rotation + BF16 store). The cache is prefilled through the
GPU reshape_and_cache from N(0,1) BF16 K/V.

Cold reads without a flush kernel: SLICES independent config-3 sequences
(each its own 256 random pages of one shared pool, its own q) are decoded in
turn, so a sequence's 4.47 MB is read again only after SLICES-1 others
(572 MB, more than the 256 MiB Infinity Cache) have been. The timed steps are
captured once in a HIP graph and replayed back to back; HIP events on the
launch stream bracket the replays, so ms_per_step is the average launch
duration including the dispatch gap between consecutive kernels.

Also reported: reshape_and_cache tokens/s on BASELINE configs[1] (1024 BF16
tokens into a 4096-page pool, seeded page permutation; and the same tokens at
token-granular slots through the scatter writer), the configs[0] A8 strip,
the configs[3] split sweep (ctx 4096 / 16384 / 32768 x 2..16 splits, ragged
4103), the batched decode step of configs[4] (64 sequences, ctx ~U[512,
8192]), and the CPU baseline: the C oracle's decode of the same sequence on
the host cores (kind "port"), on all of them and on one.

Usage:
  python bench.py [--gpus 1] [--steps K] [--warmup W]
  python bench.py --pmc-run            # workload for rocprofv3 --pmc passes
  python bench.py --summarize-pmc FETCH_DB WRITE_DB   # -> profiles/*traffic*
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
METRIC = "TQ4 paged decode µs + HBM GB/s (% peak) @ctx4096; reshape_and_cache tokens/s"

B, HQ, HKV, D, S, CTX = 1, 32, 8, 128, 16, 4096
PAGES = CTX // S
SLICES = 128
SEED = 0x71340003
CALIB_BYTES = 64 << 20  # plain copy (x * 2) of known size for the PMC scale factors
TRAFFIC_FILE = os.path.join(REPO, "profiles", "decode_config3_traffic.json")
DECODE_KERNEL = "decode_kernel<128, 1>"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def decode_algorithmic_bytes(ctx_lens, hq, hkv, d, s):
    """Bytes the contract forces across HBM for one decode: K+V nibbles and
    both FP32 scales of every live token, the block-table entries, the
    context lengths, q and out (BF16)."""
    per_token = hkv * (d + 8)  # d/2 key + d/2 value bytes + 2 x 4-byte scales per kv head
    kv = sum(ctx_lens) * per_token
    tables = sum((c + s - 1) // s for c in ctx_lens) * 4
    qo = 2 * len(ctx_lens) * hq * d * 2
    return kv + tables + qo + 4 * len(ctx_lens)


def writer_algorithmic_bytes(tokens, hkv, d, in_bytes):
    """Inputs read + packed nibbles + scales written + slot mapping read."""
    return tokens * (2 * hkv * d * in_bytes + hkv * d + 2 * hkv * 4 + 4)


# ---------------------------------------------------------------- PMC summary
def _pmc_per_dispatch(db, counter):
    """Mean value of `counter` per dispatch, by kernel name (rocprofv3 db)."""
    import sqlite3
    con = sqlite3.connect(db)
    cols = {r[1] for r in con.execute("pragma table_info(counters_collection)")}
    name_col = "kernel_name" if "kernel_name" in cols else "name"
    q = (f"select {name_col}, avg(value) , count(*) from counters_collection "
         f"where counter_name = ? group by {name_col}")
    rows = list(con.execute(q, (counter,)))
    con.close()
    return {r[0]: (float(r[1]), int(r[2])) for r in rows}


def summarize_pmc(fetch_db, write_db):
    """FETCH_SIZE / WRITE_SIZE (KiB per dispatch) of the decode kernel, each
    scaled by what the counter reads for a plain copy of CALIB_BYTES."""
    fetch = _pmc_per_dispatch(fetch_db, "FETCH_SIZE")
    write = _pmc_per_dispatch(write_db, "WRITE_SIZE")

    def pick(tab, key):
        hits = [(k, v) for k, v in tab.items() if key in k]
        if not hits:
            raise SystemExit(f"no kernel matching {key!r} in {sorted(tab)}")
        return hits[0]

    dn, (dec_f, nf) = pick(fetch, "decode_kernel")
    _, (dec_w, nw) = pick(write, "decode_kernel")
    cn, (cp_f, _) = pick(fetch, "MulFunctor")
    _, (cp_w, _) = pick(write, "MulFunctor")
    f_scale = CALIB_BYTES / (cp_f * 1024.0)
    w_scale = CALIB_BYTES / (cp_w * 1024.0)
    fetch_b = dec_f * 1024.0 * f_scale
    write_b = dec_w * 1024.0 * w_scale
    out = {"kernel": dn, "dispatches": [nf, nw], "fetch_kib_raw": dec_f, "write_kib_raw": dec_w,
           "calib_kernel": cn, "calib_bytes": CALIB_BYTES, "fetch_scale": f_scale,
           "write_scale": w_scale, "fetch_bytes": fetch_b, "write_bytes": write_b,
           "traffic_bytes": fetch_b + write_b,
           "algorithmic_bytes": decode_algorithmic_bytes([CTX], HQ, HKV, D, S)}
    os.makedirs(os.path.dirname(TRAFFIC_FILE), exist_ok=True)
    with open(TRAFFIC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print(json.dumps(out))


def read_traffic():
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


# -------------------------------------------------------------------- workload
class Workload:
    """SLICES config-3 sequences in one page pool, prefilled on the GPU."""

    def __init__(self, tq4, torch, dev, slices):
        self.tq4, self.torch = tq4, torch
        rng = np.random.default_rng(SEED)
        gen = torch.Generator(device=dev)
        gen.manual_seed(SEED)
        self.slices = slices
        self.pool = slices * PAGES
        pool = self.pool
        self.signs_np = np.where(rng.random(D) < 0.5, -1.0, 1.0).astype(np.float32)
        self.signs = torch.from_numpy(self.signs_np).to(dev)
        self.isl = 1.0 / math.sqrt(D)
        self.scale = 1.0 / math.sqrt(D)
        nbytes = pool * HKV * S * D // 2
        self.kc = torch.zeros(nbytes, dtype=torch.int8, device=dev)
        self.vc = torch.zeros(nbytes, dtype=torch.int8, device=dev)
        self.sc = torch.zeros(2 * pool * HKV * S, dtype=torch.float32, device=dev)
        perm = rng.permutation(pool).astype(np.int32).reshape(slices, PAGES)
        self.tables = [torch.from_numpy(perm[i][None, :].copy()).to(dev) for i in range(slices)]
        ar = torch.arange(S, device=dev, dtype=torch.int32)
        for i in range(slices):
            slots = (self.tables[i][0][:, None] * S + ar[None, :]).reshape(-1).contiguous()
            k = torch.randn((CTX, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
            v = torch.randn((CTX, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
            tq4.reshape_and_cache_bf16(k, v, self.kc, self.vc, self.sc, slots,
                                       pi_signs=self.signs, num_blocks=pool, block_size=S,
                                       inv_sqrt_len=self.isl)
        self.ctx = torch.tensor([CTX], dtype=torch.int32, device=dev)
        self.q = [torch.randn((B, HQ, D), generator=gen, device=dev).to(torch.bfloat16)
                  for _ in range(slices)]
        self.out = torch.empty((B, HQ, D), dtype=torch.bfloat16, device=dev)
        self.splits = tq4.auto_splits(B, HKV, PAGES, S)
        self.ws = tq4.decode_workspace(B, HQ, HKV, D, self.splits)

    def decode(self, i, out=None):
        tq4 = self.tq4
        tq4.paged_decode(self.q[i], self.kc, self.vc, self.sc, self.tables[i], self.ctx,
                         self.signs, HKV, S, self.pool, out=self.out if out is None else out,
                         workspace=self.ws, num_splits=self.splits, scale=self.scale,
                         inv_sqrt_len=self.isl)


def graph_time(torch, fns, steps, warmup):
    """Capture fns (a list of launch closures) once in a HIP graph, replay it
    until `steps` launches have run, and time the replays with events on the
    launch stream. Returns (ms per launch, wall seconds of the timed region)."""
    n = len(fns)
    reps = max(1, steps // n)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(max(1, warmup // n)):
            for f in fns:
                f()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for f in fns:
            f()
    g.replay()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return e0.elapsed_time(e1) / (reps * n), wall, reps * n


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline decode only")
    ap.add_argument("--pmc-run", action="store_true",
                    help="a few cold decodes plus a plain copy of known size, for rocprofv3 --pmc")
    ap.add_argument("--summarize-pmc", nargs=2, metavar=("FETCH_DB", "WRITE_DB"))
    args = ap.parse_args()

    if args.summarize_pmc:
        summarize_pmc(*args.summarize_pmc)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): the TQ4 path is "
              "built and measured on a single MI355X; no multi-GPU figure is produced.",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import __graft_entry__
    tq4 = __graft_entry__.package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.pmc_run:
        w = Workload(tq4, torch, dev, 32)
        torch.cuda.synchronize()
        for i in range(32):
            w.decode(i)
        src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(4):
            torch.mul(src, 2.0, out=dst)  # the calibration copy: reads and writes CALIB_BYTES
        torch.cuda.synchronize()
        log("pmc workload done")
        return

    log(f"prefilling {SLICES} config-3 sequences ({SLICES * PAGES} pages)")
    w = Workload(tq4, torch, dev, SLICES)
    torch.cuda.synchronize()

    # correctness gates: finite output, and the last graph replay (slice
    # SLICES-1) bit-identical to an eager decode of the same slice
    ref = torch.empty_like(w.out)
    w.decode(SLICES - 1, out=ref)
    torch.cuda.synchronize()
    assert torch.isfinite(ref.float()).all(), "decode produced non-finite values"

    cold_ms, wall, nsteps = graph_time(torch, [lambda i=i: w.decode(i) for i in range(SLICES)],
                                       args.steps, args.warmup)
    torch.cuda.synchronize()
    assert torch.equal(w.out.view(torch.int16), ref.view(torch.int16)), \
        "graph replays changed the decode result"
    warm_ms, _, _ = graph_time(torch, [lambda: w.decode(0)] * 64, 512, 64)
    dec_bytes = decode_algorithmic_bytes([CTX], HQ, HKV, D, S)
    gbs = dec_bytes / (cold_ms * 1e-3) / 1e9
    log(f"decode cold: {cold_ms * 1e3:.2f} us/step -> {gbs:.1f} GB/s "
        f"({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak); warm {warm_ms * 1e3:.2f} us; "
        f"splits={w.splits}")

    extra = {}
    if not args.no_extra:
        extra = extra_workloads(tq4, torch, dev, w, cpu=not args.no_cpu)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, w, dec_bytes, args.cpu_seconds)
        log(f"cpu baseline: {cpu}")

    traffic = read_traffic()
    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": nsteps,
        "warmup": args.warmup,
        "ms_per_step": round(cold_ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int4 cache, fp16 MFMA operands, fp32 softmax/accumulate",
        "data": "synthetic: N(0,1) BF16 K/V quantised by the GPU writer, N(0,1) BF16 q, seeded",
        "config": {"workload": "configs[2] single-sequence TQ4 paged decode", "batch": B,
                   "q_heads": HQ, "kv_heads": HKV, "head_dim": D, "ctx": CTX, "page_size": S,
                   "splits": w.splits, "cache": f"cold ({SLICES} rotated sequences)",
                   "parallelism": "single GPU"},
        "decode_us": {"cold": round(cold_ms * 1e3, 3), "warm": round(warm_ms * 1e3, 3)},
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "traffic": round(traffic["traffic_bytes"]) if traffic else None,
                     "kernel": DECODE_KERNEL, "algorithmic_bytes": dec_bytes},
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
    }
    result.update(extra)
    print(json.dumps(result), flush=True)


def extra_workloads(tq4, torch, dev, w, cpu=True):
    """reshape_and_cache tokens/s (configs[1], and its scatter variant), the A8
    strip, the split sweep, the batched step
    (configs[4]), the codebook leaves and the KV4/FP8 decode."""
    out = {}
    rng = np.random.default_rng(0x71340002)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x71340002)
    # --- 1024 BF16 tokens, 4096-page pool, permuted pages; 32 input sets rotated
    wt, pool, nin = 1024, 4096, 32
    wkc = torch.zeros(pool * HKV * S * D // 2, dtype=torch.int8, device=dev)
    wvc, wsc = torch.zeros_like(wkc), torch.zeros(2 * pool * HKV * S, device=dev)
    ar = torch.arange(S, device=dev, dtype=torch.int32)
    ins = []
    for _ in range(nin):
        pages = torch.from_numpy(rng.permutation(pool)[: wt // S].astype(np.int32)).to(dev)
        slots = (pages[:, None] * S + ar[None, :]).reshape(-1).contiguous()
        k = torch.randn((wt, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
        v = torch.randn((wt, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
        ins.append((k, v, slots))

    def write(i):
        k, v, slots = ins[i]
        tq4.reshape_and_cache_bf16(k, v, wkc, wvc, wsc, slots, pi_signs=w.signs,
                                   num_blocks=pool, block_size=S, inv_sqrt_len=w.isl)

    wms, _, _ = graph_time(torch, [lambda i=i: write(i) for i in range(nin)], 512, 64)
    wbytes = writer_algorithmic_bytes(wt, HKV, D, 2)
    out["reshape_and_cache"] = {"workload": "configs[1] BF16 1024 tokens", "us": round(wms * 1e3, 3),
                                "tokens_per_s": round(wt / (wms * 1e-3), 1),
                                "GBps": round(wbytes / (wms * 1e-3) / 1e9, 2),
                                "algorithmic_bytes": wbytes}
    log(f"reshape_and_cache: {wms * 1e3:.2f} us -> {wt / (wms * 1e-3) / 1e6:.1f} M tokens/s")

    # --- configs[1], secondary: the same 1024 tokens at token-granular slots
    # through the scatter writer, which merges each token into its value
    # strip (RMW). The writer's contract gives a strip one owner per launch,
    # so the slots are a random token position in each of 1024 distinct
    # strips (of the pool's 4096).
    sins = []
    for i in range(nin):
        k, v, _ = ins[i]
        strips = rng.permutation(pool * S // 16)[:wt]
        sl = torch.from_numpy((strips * 16 + rng.integers(0, 16, wt)).astype(np.int32)).to(dev)
        sins.append((k, v, sl))

    def scatter(i):
        k, v, sl = sins[i]
        tq4.reshape_scatter(k, v, wkc, wvc, wsc, sl, w.signs, num_blocks=pool, block_size=S,
                            inv_sqrt_len=w.isl)

    sms_, _, _ = graph_time(torch, [lambda i=i: scatter(i) for i in range(nin)], 512, 64)
    sbytes_ = wbytes + wt * HKV * 2 * (D * S // 2)  # + the value-strip read and write-back
    out["reshape_scatter"] = {"workload": "configs[1] secondary: 1024 BF16 tokens, one per "
                                          "strip at random positions (value-strip RMW)", "us": round(sms_ * 1e3, 3),
                              "tokens_per_s": round(wt / (sms_ * 1e-3), 1),
                              "GBps": round(sbytes_ / (sms_ * 1e-3) / 1e9, 2),
                              "algorithmic_bytes": sbytes_}
    log(f"reshape_scatter: {sms_ * 1e3:.2f} us -> {wt / (sms_ * 1e-3) / 1e6:.1f} M tokens/s")

    # --- one 16-token A8 strip, uniform ints in [-127, 127], slot = identity
    # into page 0 (latency-bound: one strip x 8 heads)
    a8 = [(torch.randint(-127, 128, (S, HKV, D), dtype=torch.int8, device=dev, generator=gen),
           torch.randint(-127, 128, (S, HKV, D), dtype=torch.int8, device=dev, generator=gen))
          for _ in range(8)]
    ident = torch.arange(S, dtype=torch.int32, device=dev)

    def write_a8(i):
        k, v = a8[i]
        tq4.reshape_and_cache_a8(k, v, wkc, wvc, wsc, ident, pi_signs=w.signs, num_blocks=pool,
                                 block_size=S, inv_sqrt_len=w.isl)

    ams, _, _ = graph_time(torch, [lambda i=i: write_a8(i) for i in range(8)], 512, 64)
    abytes = writer_algorithmic_bytes(S, HKV, D, 1)
    out["reshape_and_cache_a8"] = {"workload": "configs[0] A8, one 16-token strip",
                                   "us": round(ams * 1e3, 3),
                                   "tokens_per_s": round(S / (ams * 1e-3), 1),
                                   "algorithmic_bytes": abytes}
    log(f"reshape_and_cache A8 strip: {ams * 1e3:.2f} us")

    # --- split sweep. Sequences at ctx 4096 / 16384 / 32768 (and
    # the ragged 4096 + 7) over random pages of the headline pool; each time
    # rotates over enough sequences that >= 512 MB are read between re-reads.
    out["split_sweep"] = split_sweep(tq4, torch, dev, w)

    # --- batched decode step, 64 sequences, ctx ~U[512, 8192]
    r = np.random.default_rng(0x71340005)
    ctxs = [int(x) for x in r.integers(512, 8193, 64)]
    bsz = len(ctxs)
    npages = [(c + 1 + S - 1) // S for c in ctxs]  # room for the step's new token
    pool5 = int(sum(npages) * 1.1) + 16
    maxb = max(npages)
    perm = r.permutation(pool5).astype(np.int32)
    tab = np.zeros((bsz, maxb), np.int32)
    at = 0
    for b, n in enumerate(npages):
        tab[b, :n] = perm[at:at + n]
        at += n
    tables = torch.from_numpy(tab).to(dev)
    kc5 = torch.randint(-128, 127, (pool5 * HKV * S * D // 2,), dtype=torch.int8, device=dev,
                        generator=gen)
    vc5 = torch.randint(-128, 127, kc5.shape, dtype=torch.int8, device=dev, generator=gen)
    sc5 = torch.rand(2 * pool5 * HKV * S, device=dev, generator=gen) * 0.05 + 0.01
    ctx_now = torch.tensor([c + 1 for c in ctxs], dtype=torch.int32, device=dev)
    slot_np = np.array([tab[b, c // S] * S + c % S for b, c in enumerate(ctxs)], np.int32)
    slots5 = torch.from_numpy(slot_np).to(dev)
    q5 = torch.randn((bsz, HQ, D), generator=gen, device=dev).to(torch.bfloat16)
    kn = torch.randn((bsz, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
    vn = torch.randn((bsz, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
    out5 = torch.empty_like(q5)
    # configs[4] asks for a split-K decode. tq4_decode_auto_splits picks one
    # split here (its rule knows the batch's longest context, not the spread);
    # three splits, with the persistent kernel ordering the last splits
    # longest first, measured best for this batch (K = 1..8 sweep).
    k5 = 3
    ws5 = tq4.decode_workspace(bsz, HQ, HKV, D, k5)

    def step():
        tq4.reshape_scatter(kn, vn, kc5, vc5, sc5, slots5, w.signs, num_blocks=pool5,
                            block_size=S, inv_sqrt_len=w.isl)
        tq4.paged_decode(q5, kc5, vc5, sc5, tables, ctx_now, w.signs, HKV, S, pool5, out=out5,
                         workspace=ws5, num_splits=k5, scale=w.scale, inv_sqrt_len=w.isl)

    sms, _, _ = graph_time(torch, [step] * 8, 64, 16)
    sbytes = decode_algorithmic_bytes([c + 1 for c in ctxs], HQ, HKV, D, S) + bsz * (
        2 * HKV * D * 2 + HKV * D // 2 + 2 * HKV * 4 + 4) + bsz * HKV * 1024  # + value-strip RMW
    out["batched_step"] = {"workload": "configs[4] 64 seqs ctx~U[512,8192]: scatter 64 tokens + "
                                       "split-K decode", "us": round(sms * 1e3, 3),
                           "tokens_per_s": round(bsz / (sms * 1e-3), 1),
                           "GBps": round(sbytes / (sms * 1e-3) / 1e9, 2),
                           "pct_hbm_peak": round(100 * sbytes / (sms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
                           "splits": k5, "algorithmic_bytes": sbytes, "cache": "warm (one step)"}
    log(f"batched step: {sms * 1e3:.2f} us -> {sbytes / (sms * 1e-3) / 1e9:.0f} GB/s")

    # --- codebook leaves (HBM streams): Lloyd-Max 4-bit over 32M FP32 values
    # (in + centroids + codes), ICDF over 64M FP16 values (in + codes)
    nl = 1 << 25
    xl = torch.randn(nl, generator=gen, device=dev)
    rl = torch.empty_like(xl)
    cl = torch.empty(nl // 2, dtype=torch.uint8, device=dev)
    lms, _, _ = graph_time(torch, [lambda: tq4.lloydmax_quantize(xl, 4, 0, dst=rl, codes=cl)],
                           20, 4)
    lbytes = nl * (4 + 4) + nl // 2
    xi = torch.randn(2 * nl, generator=gen, device=dev).to(torch.float16)
    ci = torch.empty(nl, dtype=torch.uint8, device=dev)
    ims, _, _ = graph_time(torch, [lambda: tq4.icdf_quantize(xi, out=ci)], 20, 4)
    ibytes = 2 * nl * 2 + nl
    out["codebook"] = {
        "lloydmax4_32M_fp32": {"us": round(lms * 1e3, 2), "GBps": round(lbytes / (lms * 1e-3) / 1e9, 1),
                               "algorithmic_bytes": lbytes},
        "icdf_64M_fp16": {"us": round(ims * 1e3, 2), "GBps": round(ibytes / (ims * 1e-3) / 1e9, 1),
                          "algorithmic_bytes": ibytes}}
    log(f"codebook: Lloyd-Max {lbytes / (lms * 1e-3) / 1e9:.0f} GB/s, "
        f"ICDF {ibytes / (ims * 1e-3) / 1e9:.0f} GB/s")
    out["kv4fp8_decode"] = kv4fp8_workloads(tq4, torch, dev, cpu)
    return out


def kv4fp8_cache_bytes(tokens, ctx, kv_heads):
    """Live KV4/FP8 cache bytes, as the reference's benchmark counts them
    (Fixture::cache_bytes: 256 packed bytes per row and KV head for K and V,
    plus the row's 32-byte scale slot)."""
    return tokens * ctx * (kv_heads * 256 + 32)


def kv4fp8_workloads(tq4, torch, dev, cpu=True):
    """The KV4/FP8 NZ-tiled decode: the reference benchmark's shape
    (bench_turboquant_decode_splitk --impl fused-opt: 1 request, 16 q heads over
    one KV head, D=256, 128-row pages, FP32 pre-rotated query, FP16 output) at
    ctx 4096, and a batched case beyond the 256 MiB Infinity Cache."""
    res = {}
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x4B5F8)
    gain = 2.9832882881
    for name, (T, H, G, S, ctx) in (("ref_shape_1x16q1kv_ctx4096", (1, 1, 16, 128, 4096)),
                                     ("batched_32x64q4kv_ctx8192", (32, 4, 16, 128, 8192))):
        pages = (ctx + S - 1) // S
        P = T * pages
        key = torch.randint(0, 256, (P * S * H * 128,), dtype=torch.uint8, device=dev,
                            generator=gen)
        val = torch.randint(0, 256, key.shape, dtype=torch.uint8, device=dev, generator=gen)
        sc = (torch.rand(P * S * 8, device=dev, generator=gen) * 1.5 + 0.5) * gain
        tb = torch.randperm(P, device=dev, generator=gen).to(torch.int32).view(T, pages)
        ln = torch.full((T,), ctx, dtype=torch.int32, device=dev)
        q = torch.randn((T, H * G, 256), device=dev, generator=gen)
        o = torch.empty((T, H * G, 256), dtype=torch.float16, device=dev)
        L = tq4.fused_decode_opt_launch(T, H * G, H, S, pages, num_blocks=P)
        ws = torch.zeros(tq4.kv4fp8_workspace_bytes(L), dtype=torch.uint8, device=dev)
        run = lambda: tq4.kv4fp8_decode(q, key, val, sc, tb, ln, H, S, P, out=o,  # noqa: E731
                                        workspace=ws)
        run()
        torch.cuda.synchronize()
        assert torch.isfinite(o.float()).all(), "kv4fp8 decode produced non-finite values"
        ms, _, _ = graph_time(torch, [run] * 16, 256 if T == 1 else 64, 32 if T == 1 else 8)
        nbytes = kv4fp8_cache_bytes(T, ctx, H) + T * H * G * 256 * (4 + 2) + T * pages * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        res[name] = {"us": round(ms * 1e3, 3), "GBps": round(gbs, 1),
                     "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                     "tokens": T, "q_heads": H * G, "kv_heads": H, "head_dim": 256,
                     "ctx": ctx, "page_size": S, "algorithmic_bytes": nbytes,
                     "cache": "warm" if nbytes < (256 << 20) else "beyond the Infinity Cache"}
        log(f"kv4fp8 {name}: {ms * 1e3:.2f} us -> {gbs:.0f} GB/s")
        if cpu and T == 1:
            # the C oracle (oracle/kv4fp8_oracle.c) on the same inputs, bounded at ~2 s
            sys.path.insert(0, os.path.join(REPO, "tests"))
            from oracle_bindings import Oracle
            orc = Oracle()
            threads = min(16, os.cpu_count() or 1)
            h = [x.cpu().numpy() for x in (q, key, val, sc, tb, ln)]
            iters, t0 = 0, time.perf_counter()
            while time.perf_counter() - t0 < 2.0:
                orc.kv4fp8_decode(*h, heads=H * G, kv_heads=H, block_size=S, max_blocks=pages,
                                  num_blocks=P, threads=threads)
                iters += 1
            el = time.perf_counter() - t0
            res[name]["cpu_baseline"] = {
                "value": round(nbytes * iters / el / 1e9, 4), "unit": "GB/s",
                "cores": min(threads, T * H),
                "kind": "port", "us_per_decode": round(el / iters * 1e6, 1),
                "sample": f"{iters} decodes of this shape by oracle/kv4fp8_oracle.c in "
                          f"{el:.1f} s (FP64 products; one task per (token, kv head), so "
                          f"{min(threads, T * H)} thread(s) busy)"}
    return res


def split_sweep(tq4, torch, dev, w):
    """the fused decode at ctx {4096, 16384, 32768} x K {2, 4, 8,
    16, auto}, plus the ragged ctx 4103 at auto."""
    rng = np.random.default_rng(0x71340004)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x71340004)
    rows = []
    for ctx, ks in ((4096, (2, 4, 8, 16, 0)), (16384, (2, 4, 8, 16, 0)),
                    (32768, (2, 4, 8, 16, 0)), (4103, (0,))):
        pages = (ctx + S - 1) // S
        nseq = max(4, (512 << 20) // (ctx * HKV * (D + 8)))
        tabs = [torch.from_numpy(rng.permutation(w.pool)[:pages].astype(np.int32)[None, :]).to(dev)
                for _ in range(nseq)]
        qs = [torch.randn((1, HQ, D), generator=gen, device=dev).to(torch.bfloat16)
              for _ in range(nseq)]
        ctx_t = torch.tensor([ctx], dtype=torch.int32, device=dev)
        out = torch.empty((1, HQ, D), dtype=torch.bfloat16, device=dev)
        nbytes = decode_algorithmic_bytes([ctx], HQ, HKV, D, S)
        for k in ks:
            kk = k or tq4.auto_splits(1, HKV, pages, S)
            ws = tq4.decode_workspace(1, HQ, HKV, D, kk)

            def dec(i, kk=kk, ws=ws):
                tq4.paged_decode(qs[i], w.kc, w.vc, w.sc, tabs[i], ctx_t, w.signs, HKV, S, w.pool,
                                 out=out, workspace=ws, num_splits=kk, scale=w.scale,
                                 inv_sqrt_len=w.isl)

            ms, _, _ = graph_time(torch, [lambda i=i: dec(i) for i in range(nseq)],
                                  max(256, nseq), max(32, nseq))
            gbs = nbytes / (ms * 1e-3) / 1e9
            rows.append({"ctx": ctx, "splits": kk, "auto": k == 0, "us": round(ms * 1e3, 2),
                         "GBps": round(gbs, 1),
                         "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                         "algorithmic_bytes": nbytes})
            log(f"split sweep ctx {ctx} K {kk}{' (auto)' if k == 0 else ''}: "
                f"{ms * 1e3:.2f} us -> {gbs:.0f} GB/s")
    return {"workload": "configs[3] single-sequence decode, 32q:8kv, d128, page 16, cold "
                        "(rotated sequences)", "rows": rows}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_baseline(torch, w, dec_bytes, seconds):
    """The C oracle's decode of slice 0 on the host cores, bounded in time."""
    sys.path.insert(0, os.path.join(REPO, "tests"))
    from oracle_bindings import Oracle
    o = Oracle()
    threads = min(16, os.cpu_count() or 1)
    h_q = w.q[0].view(torch.int16).cpu().numpy().view(np.uint16)
    h_kc, h_vc, h_sc = w.kc.cpu().numpy(), w.vc.cpu().numpy(), w.sc.cpu().numpy()
    h_tab, h_ctx = w.tables[0].cpu().numpy(), w.ctx.cpu().numpy()

    def timed(nthreads, budget):
        iters, t0 = 0, time.perf_counter()
        while True:
            o.paged_decode(h_q, h_kc, h_vc, h_sc, h_tab, h_ctx, w.signs_np, None, HQ, HKV, D, S,
                           w.pool, w.splits, np.float32(w.scale), np.float32(w.isl), 1,
                           threads=nthreads)
            iters += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return iters, el

    iters1, el1 = timed(1, seconds / 2)
    iters, el = timed(threads, seconds)
    try:
        nproc = len(os.sched_getaffinity(0))
    except AttributeError:
        nproc = os.cpu_count()
    return {"value": round(dec_bytes * iters / el / 1e9, 4), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"{iters} configs[2] decodes (B=1, 32q:8kv, d128, ctx4096, {w.splits} "
                      f"splits) by oracle/tq4_oracle.c in {el:.1f} s on {threads} threads",
            "us_per_decode": round(el / iters * 1e6, 1),
            "single_thread": {"value": round(dec_bytes * iters1 / el1 / 1e9, 4), "unit": "GB/s",
                              "us_per_decode": round(el1 / iters1 * 1e6, 1),
                              "sample": f"{iters1} decodes in {el1:.1f} s on 1 thread"},
            "nproc": nproc, "cpu_model": cpu_model()}


if __name__ == "__main__":
    main()
