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
(568 MB, more than the 256 MiB Infinity Cache) have been.

Timing (every row, `time_launches`): the W warmup launches and then exactly
the K timed launches are captured as two HIP graphs and replayed back to
back; HIP events on the replay stream bracket the timed graph, so
ms_per_step is the average launch duration including the dispatch gap
between consecutive kernels. The spread (min / median / p99) comes from
further replays of graphs of `chunk` launches, each bracketed by events: one
sample is the per-launch time of one replay.

Also reported: reshape_and_cache tokens/s on BASELINE configs[1] (1024 BF16
tokens into a 4096-page pool; and the same tokens at token-granular slots
through the scatter writer), the RMS codec writer on the same tokens, the
configs[0] A8 strip, the configs[3] split sweep, the configs[4] batched step
(64 sequences, ctx ~U[512, 8192], two batches rotated so each is read cold),
the codebook leaves and the KV4/FP8 decode; and per row the CPU baseline:
the C oracle (oracle/*.c, kind "port") on one thread and on every core this
process may run on, each on a bounded sample of the row's workload.

Usage:
  python bench.py [--gpus 1] [--steps K] [--warmup W]
  python bench.py --pmc-run              # workload for rocprofv3 --pmc passes
  python bench.py --summarize-pmc DIR [--pmc-merge]  # DIR/<row>/<pass>/run_counter_collection.csv
  python bench.py --pmc-table            # the committed summary as markdown
  python bench.py --summarize-trace DIR  # a rocprofv3 --kernel-trace csv run
  python bench.py --phases               # configs[2] phase timeline and the configs[4]
                                         # per-item timeline (libtq4_stamps.so)
  python bench.py --floor                # compute-free floors (libtq4_floor.so)
"""
from __future__ import annotations

import argparse
import csv
import glob
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
STRIP = 16  # tokens per cache strip: the aligned writer's unit
SLICES = 128
SEED = 0x71340003
CALIB_BYTES = 64 << 20  # plain copy (x * 2) of known size for the PMC scale factors
PMC_FILE = os.path.join(REPO, "profiles", "pmc_summary.json")
CALIB_KERNEL = "MulFunctor<float"
SWEEP = ((4096, (2, 4, 8, 16, 0)), (16384, (2, 4, 8, 16, 0)), (32768, (2, 4, 8, 16, 0)),
         (65536, (8, 16, 0)), (4103, (0,)))


def sweep_row(ctx, k):
    """PMC row name of a split-sweep row (k = the split count, auto resolved)."""
    return f"sweep_ctx{ctx}_K{k}"


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


def decode_overhead_bytes(ctx_lens, hq, hkv, d, s, splits, max_blocks):
    """Workspace traffic of one fused decode, kept out of the algorithmic
    bytes: for each (seq, kv head) with more than one live split, the split
    records [m, l, 0, 0, acc[d]] of its q heads, stored by every live split
    but the combiner and loaded and zeroed by the combiner:
    (3 k_live - 1) x G x (d + 4) x 4 bytes."""
    if splits <= 1:
        return 0
    g = hq // hkv
    width = -(-max_blocks // splits)
    total = 0
    for c in ctx_lens:
        k_live = -(-(-(-c // s)) // width)
        if k_live > 1:
            total += hkv * (3 * k_live - 1) * g * (d + 4) * 4
    return total


def writer_algorithmic_bytes(tokens, hkv, d, in_bytes):
    """Inputs read + packed nibbles + scales written + slot mapping read."""
    return tokens * (2 * hkv * d * in_bytes + hkv * d + 2 * hkv * 4 + 4)


def rms_writer_algorithmic_bytes(tokens, hkv, d, in_bytes):
    """Inputs read + packed codes + the slot's scale record written + slot read."""
    return tokens * (2 * hkv * d * in_bytes + hkv * d + 4 * ((2 * hkv + 7) // 8 * 8) + 4)


# ---------------------------------------------------------------- timing
def _graph(torch, stream, fns):
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for f in fns:
            f()
    return g


def _pct(v, q):
    return float(np.percentile(np.asarray(v), q))


def time_launches(torch, fns, steps, warmup, samples=32, chunk=32, after_timed=None,
                  warm_replays=0):
    """Throughput and spread of launches over a rotation of input sets.

    fns[i] launches one step on input set i; launch j takes set j % len(fns),
    so a set is read again only after len(fns) - 1 others. Launch 0 runs
    eagerly (any first-call set-up stays outside capture); launches 1 ..
    warmup-1 form the warmup graph and launches warmup .. warmup+steps-1 the
    timed graph, replayed right after it; HIP events on the replay stream
    bracket the timed replay. Then `samples` replays of graphs of `chunk`
    launches (continuing the rotation), each bracketed by events, give the
    spread of the per-launch time. after_timed() runs once the timed replay
    has finished, before the spread's launches. warm_replays > 0: the warmup
    is launch 0 and that many replays of the timed graph itself (warmup =
    1 + warm_replays * steps launches, one input set), for a row whose first
    milliseconds after an idle GPU run slower than its steady state."""
    n = len(fns)
    warmup = max(1, warmup)
    rot = lambda a, b: [fns[i % n] for i in range(a, b)]  # noqa: E731
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fns[0]()
    torch.cuda.synchronize()
    if warm_replays:
        assert n == 1, "the timed graph's own replays warm up one input set"
        warmup = 1 + warm_replays * steps  # launch 0 and the warm replays
        gw = None
        gt = _graph(torch, stream, rot(1, 1 + steps))
    else:
        gw = _graph(torch, stream, rot(1, warmup)) if warmup > 1 else None
        gt = _graph(torch, stream, rot(warmup, warmup + steps))
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        if gw is not None:
            gw.replay()
        for _ in range(warm_replays):
            gt.replay()
        e0.record(stream)
        gt.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / steps
    del gw, gt
    if after_timed is not None:
        after_timed()
    # spread: graphs of `chunk` consecutive launches, covering the rotation
    start = warmup + steps
    ngraphs = max(1, math.ceil(n / chunk))
    graphs = [_graph(torch, stream, rot(start + k * chunk, start + (k + 1) * chunk))
              for k in range(ngraphs)]
    torch.cuda.synchronize()
    evs = []
    with torch.cuda.stream(stream):
        for s_ in range(samples):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            graphs[s_ % ngraphs].replay()
            b.record(stream)
            evs.append((a, b))
    torch.cuda.synchronize()
    per = [a.elapsed_time(b) * 1e3 / chunk for a, b in evs]
    spread = {"min_us": round(min(per), 3), "median_us": round(float(np.median(per)), 3),
              "p99_us": round(_pct(per, 99), 3), "samples": samples, "launches_per_sample": chunk}
    return {"ms": ms, "wall_s": wall, "steps": steps, "warmup": warmup, "spread": spread}


def row_times(res):
    return {"us": round(res["ms"] * 1e3, 3), "steps": res["steps"], "warmup": res["warmup"],
            "spread_us": res["spread"]}


# ---------------------------------------------------------------- PMC
def read_pmc():
    try:
        with open(PMC_FILE) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def roofline(nbytes, ms, kernel, pmc=None):
    """The roofline object of a row: algorithmic bytes over the measured
    launch time against the HBM peak; traffic from the committed PMC summary
    (FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by a plain copy)."""
    gbs = nbytes / (ms * 1e-3) / 1e9
    t = (pmc or {}).get(kernel, {})
    return {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": round(t["traffic_bytes"]) if "traffic_bytes" in t else None,
            "kernel": kernel, "algorithmic_bytes": nbytes,
            "traffic_ratio": round(t["traffic_bytes"] / nbytes, 3) if "traffic_bytes" in t else None,
            "traffic_source": "profiles/pmc_summary.json" if "traffic_bytes" in t else None}


def summarize_pmc(root, merge=False):
    """Mean counter value per dispatch of each profiled row: root/<row>/<pass>/
    run_counter_collection.csv (rocprofv3 --output-format csv) over the passes
    of `bench.py --pmc-run <row>`; the row's dispatches are those of its
    kernel and grid (pmc_kernel_of), FETCH_SIZE / WRITE_SIZE scaled to bytes
    by what they read for the row run's own plain copy of CALIB_BYTES."""
    out = {}
    for rdir in sorted(glob.glob(os.path.join(root, "*"))):
        row = os.path.basename(rdir)
        if not os.path.isdir(rdir) or row not in pmc_row_names():
            continue
        frag, grid_wg = pmc_kernel_of(row)
        vals, cals, meta = {}, {}, None
        for f in sorted(glob.glob(os.path.join(rdir, "*", "run_counter_collection.csv"))):
            with open(f) as fh:
                for r in csv.DictReader(fh):
                    name = r.get("Kernel_Name", "")
                    grid, wg = int(r["Grid_Size"]), int(r["Workgroup_Size"])
                    nwg = grid // max(1, wg)
                    if CALIB_KERNEL in name:  # the copy is the largest such multiply
                        cals.setdefault(grid, {}).setdefault(r["Counter_Name"], []).append(
                            float(r["Counter_Value"]))
                        continue
                    if frag not in name or (grid_wg is not None and nwg != grid_wg):
                        continue
                    vals.setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
                    short = name.replace("(anonymous namespace)::", "").replace("void ", "")
                    meta = meta or {"kernel": short.split("(")[0].replace("tq4::", ""),
                                    "workgroups": nwg, "workgroup_size": wg,
                                    "vgprs": int(r["VGPR_Count"]),
                                    "agprs": int(r["Accum_VGPR_Count"]),
                                    "sgprs": int(r["SGPR_Count"]),
                                    "lds_bytes": int(r["LDS_Block_Size"]),
                                    "scratch_bytes": int(r["Scratch_Size"])}
        if not vals:
            continue
        cal = cals[max(cals)] if cals else {}
        e = {**meta, "dispatches": max(len(v) for v in vals.values()),
             "counters": {c: float(np.mean(v)) for c, v in vals.items()}}
        if "FETCH_SIZE" in vals and "WRITE_SIZE" in vals and "FETCH_SIZE" in cal \
                and "WRITE_SIZE" in cal:
            fs = CALIB_BYTES / (float(np.mean(cal["FETCH_SIZE"])) * 1024.0)
            ws = CALIB_BYTES / (float(np.mean(cal["WRITE_SIZE"])) * 1024.0)
            e["fetch_bytes"] = e["counters"]["FETCH_SIZE"] * 1024.0 * fs
            e["write_bytes"] = e["counters"]["WRITE_SIZE"] * 1024.0 * ws
            e["traffic_bytes"] = e["fetch_bytes"] + e["write_bytes"]
            e["calibration"] = {"fetch_kib_raw": float(np.mean(cal["FETCH_SIZE"])),
                                "write_kib_raw": float(np.mean(cal["WRITE_SIZE"])),
                                "fetch_scale": fs, "write_scale": ws}
        out[row] = e
    if not out:
        raise SystemExit(f"no profiled rows under {root}")
    if os.path.exists(PMC_FILE):
        with open(PMC_FILE) as f:
            old = json.load(f)
        if merge:  # a re-run of some rows: the others keep their committed figures
            out = {**old, **out}
        elif set(old) - set(out):
            raise SystemExit(f"{PMC_FILE} holds rows this run does not ({', '.join(sorted(set(old) - set(out)))}): "
                             "pass --pmc-merge to keep them, or remove the file to replace it")
    os.makedirs(os.path.dirname(PMC_FILE), exist_ok=True)
    with open(PMC_FILE, "w") as f:
        json.dump(out, f, indent=1)
    print_pmc_table(out)


def print_pmc_table(out):
    """Markdown view of the PMC summary: HBM traffic for every row, then the
    LDS, occupancy and instruction counters of the rows that have them (one
    line per bench row, per-dispatch means)."""
    keys = sorted(out)
    cals = [out[k]["calibration"] for k in keys if "calibration" in out[k]]
    if cals:
        fs = [c["fetch_scale"] for c in cals]
        ws = [c["write_scale"] for c in cals]
        print(f"Calibration (each row's run has its own plain copy of {CALIB_BYTES >> 20} MiB "
              f"read and written): FETCH_SIZE scale {min(fs):.3f} .. {max(fs):.3f}, WRITE_SIZE "
              f"scale {min(ws):.3f} .. {max(ws):.3f}.\n")

    def c(e, n):
        return e["counters"].get(n, float("nan"))

    print("| row | kernel | workgroups | dispatches | FETCH_SIZE KiB | WRITE_SIZE KiB | "
          "HBM bytes (scaled) |")
    print("|---|---|---|---|---|---|---|")
    for k in keys:
        e = out[k]
        print(f"| {k} | `{e['kernel']}` | {e['workgroups']} | {e['dispatches']} | "
              f"{c(e, 'FETCH_SIZE'):.1f} | {c(e, 'WRITE_SIZE'):.1f} | "
              f"{e.get('traffic_bytes', 0):.0f} |")
    detail = [k for k in keys if not math.isnan(c(out[k], "SQ_WAVES"))]
    if not detail:
        return
    print("\n| row | LDS bank-conflict cycles / LDS-active cycles | SQ_INSTS_LDS | "
          "MeanOccupancyPerActiveCU | SQ_WAVES | SQ_INSTS_VALU | SQ_INSTS_MFMA | "
          "SQ_INSTS_VMEM_RD | SQ_BUSY_CU_CYCLES / GRBM_GUI_ACTIVE |")
    print("|---|---|---|---|---|---|---|---|---|")
    for k in detail:
        e = out[k]
        bc, act = c(e, "SQ_LDS_BANK_CONFLICT"), c(e, "SQ_LDS_IDX_ACTIVE")
        share = f"{bc / act:.3f}" if act > 0 else "no LDS"
        print(f"| {k} | {share} ({bc:.0f} / {act:.0f}) | {c(e, 'SQ_INSTS_LDS'):.0f} | "
              f"{c(e, 'MeanOccupancyPerActiveCU'):.3f} | {c(e, 'SQ_WAVES'):.0f} | "
              f"{c(e, 'SQ_INSTS_VALU'):.0f} | {c(e, 'SQ_INSTS_MFMA'):.0f} | "
              f"{c(e, 'SQ_INSTS_VMEM_RD'):.0f} | "
              f"{c(e, 'SQ_BUSY_CU_CYCLES'):.0f} / {c(e, 'GRBM_GUI_ACTIVE'):.0f} |")


def summarize_trace(root, limit=0):
    """Per (kernel, grid) launch statistics of a rocprofv3 --kernel-trace run
    (--output-format csv) under root: calls, mean, median, p99, min, max (us).
    limit > 0: only the first `limit` dispatches of each (kernel, grid), in
    dispatch order."""
    rows = {}
    for f in sorted(glob.glob(os.path.join(root, "**", "*kernel_trace.csv"), recursive=True)):
        with open(f) as fh:
            for r in csv.DictReader(fh):
                try:
                    blocks = 1
                    for ax in "XYZ":
                        blocks *= int(r[f"Grid_Size_{ax}"]) // max(1, int(r[f"Workgroup_Size_{ax}"]))
                except (KeyError, ValueError):
                    blocks = r.get("Grid_Size", "?")
                us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) * 1e-3
                rows.setdefault((r["Kernel_Name"], blocks), []).append(
                    (int(r.get("Dispatch_Id") or 0), us))
    print("| kernel | workgroups | calls | mean us | median us | p99 us | min us | max us |")
    print("|---|---|---|---|---|---|---|---|")
    for key in rows:
        v = [us for _, us in sorted(rows[key])]
        rows[key] = v[:limit] if limit > 0 else v
    for (name, blocks), v in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
        if len(v) < 4:
            continue
        short = name.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]
        print(f"| `{short}` | {blocks} | {len(v)} | {np.mean(v):.2f} | {np.median(v):.2f} | "
              f"{_pct(v, 99):.2f} | {min(v):.2f} | {max(v):.2f} |")


# ---------------------------------------------------------------- CPU leg
def cpu_threads():
    """Cores this process may run on (its affinity mask)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_host():
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            quota = f.read().strip()
    except OSError:
        pass
    return {"affinity_cores": cpu_threads(), "os_cpu_count": os.cpu_count(),
            "cpu_model": cpu_model(), "cgroup_cpu_max": quota}


def cpu_run(fn, budget):
    """Call fn until `budget` seconds have passed (at least once)."""
    it, t0 = 0, time.perf_counter()
    while True:
        fn()
        it += 1
        el = time.perf_counter() - t0
        if el >= budget:
            return it, el


def cpu_leg(fn_threads, amount, unit, sample, budget, max_tasks):
    """The oracle on one thread and on every core (capped at its number of
    independent tasks); `amount` is the row's measure per call (bytes for
    GB/s, tokens for tokens/s)."""
    scale = 1e-9 if unit == "GB/s" else 1.0
    it1, el1 = cpu_run(lambda: fn_threads(1), budget / 2)
    n = max(1, min(cpu_threads(), max_tasks))
    itn, eln = cpu_run(lambda: fn_threads(n), budget / 2)
    return {"value": round(amount * itn / eln * scale, 4), "unit": unit, "cores": n,
            "kind": "port", "us_per_call": round(eln / itn * 1e6, 1),
            "sample": f"{sample}: {itn} calls in {eln:.2f} s on {n} threads",
            "single_thread": {"value": round(amount * it1 / el1 * scale, 4), "unit": unit,
                              "us_per_call": round(el1 / it1 * 1e6, 1),
                              "sample": f"{it1} calls in {el1:.2f} s on 1 thread"},
            **cpu_host()}


def oracle():
    sys.path.insert(0, os.path.join(REPO, "tests"))
    from oracle_bindings import Oracle
    return Oracle()


# ---------------------------------------------------------------- workloads
class Workload:
    """SLICES config-3 sequences in one page pool, prefilled on the GPU."""

    def __init__(self, tq4, torch, dev, slices, touch=True):
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
        # Decode every slice once: the first read of a slice's pages after
        # the prefill pays address-translation misses (a fresh 20-step run
        # measured 9.3 us/step without this pass, 8.5 with it). The data
        # stays cold for the timed steps: at least 96 other slices (> 400 MB,
        # more than the 256 MiB Infinity Cache) are read between this pass
        # and any slice's next use.
        for i in range(slices if touch else 0):
            self.decode(i)

    def decode(self, i, out=None):
        self.tq4.paged_decode(self.q[i], self.kc, self.vc, self.sc, self.tables[i], self.ctx,
                              self.signs, HKV, S, self.pool,
                              out=self.out if out is None else out, workspace=self.ws,
                              num_splits=self.splits, scale=self.scale, inv_sqrt_len=self.isl)


class Batch:
    """One configs[4] batch: 64 sequences, ctx ~U[512, 8192] (seeded), their
    own page pool, prefilled through the GPU writers from N(0,1) BF16 K/V the
    way tests/test_gpu_scatter.py builds its cache (whole strips by the
    aligned writer, each partial tail by the scatter writer), so the timed
    decode sees the data the parity test checks; one new token per sequence
    for the step's scatter. Decoded at the split count of the length-aware
    auto rule (tq4_decode_auto_splits_lens)."""

    def __init__(self, tq4, torch, dev, seed, signs):
        S_ = S
        self.tq4 = tq4
        r = np.random.default_rng(0x71340005)
        self.ctxs = [int(x) for x in r.integers(512, 8193, 64)]  # the shape is the config's
        rb = np.random.default_rng(seed)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        bsz = len(self.ctxs)
        npages = [(c + 1 + S_ - 1) // S_ for c in self.ctxs]  # room for the step's token
        self.pool = int(sum(npages) * 1.1) + 16
        perm = rb.permutation(self.pool).astype(np.int32)
        tab = np.zeros((bsz, max(npages)), np.int32)
        at = 0
        for b, n in enumerate(npages):
            tab[b, :n] = perm[at:at + n]
            at += n
        self.tab_np = tab
        self.tables = torch.from_numpy(tab).to(dev)
        nb = self.pool * HKV * S_ * D // 2
        self.kc = torch.zeros(nb, dtype=torch.int8, device=dev)
        self.vc = torch.zeros(nb, dtype=torch.int8, device=dev)
        self.sc = torch.zeros(2 * self.pool * HKV * S_, dtype=torch.float32, device=dev)
        self.signs = signs
        self.isl = 1.0 / math.sqrt(D)
        for b, c in enumerate(self.ctxs):
            full = c // STRIP * STRIP
            tok = np.arange(c)
            sl = torch.from_numpy((tab[b, tok // S_] * S_ + tok % S_).astype(np.int32)).to(dev)
            k = torch.randn((c, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
            v = torch.randn((c, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
            if full:
                tq4.reshape_and_cache_bf16(k[:full].contiguous(), v[:full].contiguous(), self.kc,
                                           self.vc, self.sc, sl[:full].contiguous(),
                                           pi_signs=signs, num_blocks=self.pool, block_size=S_,
                                           inv_sqrt_len=self.isl)
            if c > full:
                tq4.reshape_scatter(k[full:].contiguous(), v[full:].contiguous(), self.kc,
                                    self.vc, self.sc, sl[full:].contiguous(), signs,
                                    cu_seqlens=torch.tensor([0, c - full], dtype=torch.int32,
                                                            device=dev),
                                    num_requests=1, num_blocks=self.pool, block_size=S_,
                                    inv_sqrt_len=self.isl)
        self.ctx_now = torch.tensor([c + 1 for c in self.ctxs], dtype=torch.int32, device=dev)
        self.slots = torch.from_numpy(np.array(
            [tab[b, c // S_] * S_ + c % S_ for b, c in enumerate(self.ctxs)], np.int32)).to(dev)
        self.q = torch.randn((bsz, HQ, D), generator=gen, device=dev).to(torch.bfloat16)
        self.kn = torch.randn((bsz, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
        self.vn = torch.randn((bsz, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
        self.out = torch.empty_like(self.q)
        # the host holds the lengths: the length-aware split rule
        self.K = tq4.auto_splits(bsz, HKV, tab.shape[1], S_, context_lens=[c + 1 for c in self.ctxs])
        self.ws = tq4.decode_workspace(bsz, HQ, HKV, D, self.K) if self.K > 1 else None

    def scatter(self):
        self.tq4.reshape_scatter(self.kn, self.vn, self.kc, self.vc, self.sc, self.slots,
                                 self.signs, num_blocks=self.pool, block_size=S,
                                 inv_sqrt_len=self.isl)

    def decode(self):
        self.tq4.paged_decode(self.q, self.kc, self.vc, self.sc, self.tables, self.ctx_now,
                              self.signs, HKV, S, self.pool, out=self.out, workspace=self.ws,
                              num_splits=self.K, scale=self.isl, inv_sqrt_len=self.isl)

    def step(self):
        self.scatter()
        self.decode()

    def decode_bytes(self):
        return decode_algorithmic_bytes([c + 1 for c in self.ctxs], HQ, HKV, D, S)

    def step_bytes(self):
        bsz = len(self.ctxs)
        # + the scatter: inputs, nibbles, scales, slots, and the value-strip RMW
        return self.decode_bytes() + bsz * (2 * HKV * D * 2 + HKV * D // 2 + 2 * HKV * 4 + 4) \
            + bsz * HKV * 1024


# ---------------------------------------------------------------- main
def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1024)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--cpu-seconds", type=float, default=4.0,
                    help="CPU-leg budget of the headline row (other rows use less)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true", help="headline decode only")
    ap.add_argument("--pmc-run", metavar="ROW",
                    help="one bench row's workload (8 or more launches of its kernel) plus a "
                         "plain copy of known size, for rocprofv3 --pmc; --pmc-rows lists them")
    ap.add_argument("--pmc-rows", action="store_true", help="the rows --pmc-run knows")
    ap.add_argument("--phases", action="store_true",
                    help="configs[2] per-phase timeline from the measurement build's in-kernel "
                         "stamps (libtq4_stamps.so), the split tail delta, the host enqueue "
                         "cost of one decode call, and the configs[4] persistent decode's "
                         "per-item timeline")
    ap.add_argument("--floor", action="store_true",
                    help="compute-free copies of the configs[2] decode chain and the configs[1] "
                         "writer traffic (libtq4_floor.so) beside the real kernels")
    ap.add_argument("--summarize-pmc", metavar="DIR")
    ap.add_argument("--pmc-merge", action="store_true",
                    help="with --summarize-pmc: keep the committed rows not under DIR "
                         "(without it, a run that lacks committed rows is refused)")
    ap.add_argument("--pmc-table", action="store_true",
                    help="print the committed PMC summary as markdown")
    ap.add_argument("--summarize-trace", metavar="DIR")
    ap.add_argument("--trace-limit", type=int, default=0,
                    help="with --summarize-trace: the first N dispatches of each kernel and grid")
    args = ap.parse_args()

    if args.summarize_pmc:
        summarize_pmc(args.summarize_pmc, merge=args.pmc_merge)
        return
    if args.pmc_table:
        with open(PMC_FILE) as f:
            print_pmc_table(json.load(f))
        return
    if args.summarize_trace:
        summarize_trace(args.summarize_trace, args.trace_limit)
        return
    if args.pmc_rows:
        print(" ".join(pmc_row_names()))
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}): the TQ4 path is "
              "built and measured on a single MI355X; no multi-GPU figure is produced.",
              file=sys.stderr)
        sys.exit(2)
    if args.steps < 1:
        raise SystemExit("--steps must be at least 1")

    if args.phases:
        os.environ["TQ4_LIBRARY"] = "libtq4_stamps.so"  # before the library is first loaded
    import torch

    import __graft_entry__
    tq4 = __graft_entry__.package()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.pmc_run:
        pmc_workload(tq4, torch, dev, args.pmc_run)
        return
    if args.phases:
        phases(tq4, torch, dev)
        return
    if args.floor:
        floor(tq4, torch, dev)
        return

    log(f"prefilling {SLICES} config-3 sequences ({SLICES * PAGES} pages)")
    w = Workload(tq4, torch, dev, SLICES)
    torch.cuda.synchronize()

    # correctness gate: the last timed launch (slice (W + K - 1) % SLICES)
    # must equal an eager decode of that slice, bit for bit (made after the
    # timed replay, so that no slice is read just before it)
    warm_n = max(1, args.warmup)
    last = (warm_n + args.steps - 1) % SLICES
    ref = torch.empty_like(w.out)

    def gate():
        w.decode(last, out=ref)
        torch.cuda.synchronize()
        assert torch.isfinite(ref.float()).all(), "decode produced non-finite values"
        assert torch.equal(w.out.view(torch.int16), ref.view(torch.int16)), \
            "graph replays changed the decode result"

    res = time_launches(torch, [lambda i=i: w.decode(i) for i in range(SLICES)], args.steps,
                        args.warmup, samples=48, chunk=32, after_timed=gate)
    timeouts = tq4.decode_poll_timeouts(w.ws, B, HKV)
    cold_ms = res["ms"]
    warm = time_launches(torch, [lambda: w.decode(0)], 256, 16, samples=16, chunk=64)
    timeouts += tq4.decode_poll_timeouts(w.ws, B, HKV)
    dec_bytes = decode_algorithmic_bytes([CTX], HQ, HKV, D, S)
    gbs = dec_bytes / (cold_ms * 1e-3) / 1e9
    log(f"decode cold: {cold_ms * 1e3:.2f} us/step ({res['steps']} steps) -> {gbs:.1f} GB/s "
        f"({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak); spread {res['spread']}; "
        f"warm {warm['ms'] * 1e3:.2f} us; splits={w.splits}")

    pmc = read_pmc()
    extra = {}
    if not args.no_extra:
        extra = extra_workloads(tq4, torch, dev, w, pmc, cpu=not args.no_cpu)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_decode_leg(torch, w, dec_bytes, args.cpu_seconds)
        log(f"cpu baseline: {cpu}")

    result = {
        "metric": METRIC,
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": res["steps"],
        "warmup": res["warmup"],
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
        "valid": timeouts == 0,
        "poll_timeouts": timeouts,
        "decode_us": {"cold": round(cold_ms * 1e3, 3), "cold_spread": res["spread"],
                      "warm": round(warm["ms"] * 1e3, 3), "warm_spread": warm["spread"]},
        "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "roofline": roofline(dec_bytes, cold_ms, "configs2_decode", pmc),
        "overhead_bytes": decode_overhead_bytes([CTX], HQ, HKV, D, S, w.splits, PAGES),
        "launch_floor_note": "a back-to-back graph launch of an empty kernel of 128 workgroups "
                             "costs about 1.7 us; one launch moving 4.47 MB therefore tops "
                             "out near 33 % of peak",
        "cpu_baseline": cpu,
        "wall_s_timed": round(res["wall_s"], 3),
    }
    if timeouts:
        result["INVALID"] = f"{timeouts} combine rows gave up their bounded poll"
    result.update(extra)
    print(json.dumps(result), flush=True)


PHASES = ["start", "phase-0 loads retired", "first strip pairs issued", "q operands built",
          "wave 0 strip loop done", "waves merged", "record exported (non-combining split)",
          "first row combined (poll + merge)", "egress done (combiner)"]


def phases(tq4, torch, dev, samples=64):
    """The configs[2] decode's phase timeline from the measurement build:
    after each replay of a graph of 32 cold back-to-back launches, the stamps
    of its last launch (128 workgroups) are read; per phase the median over
    workgroups of (stamp - the launch's first start), then the median over
    samples. The split tail delta is the slowest split's export minus the
    median split's. Host enqueue: wall time of eager tq4.paged_decode calls
    (Python + ctypes + C ABI + launch), no synchronisation inside. Then the
    configs[4] per-item timeline (batched_timeline)."""
    import ctypes as C
    lib_path = sys.modules[tq4.__name__ + ".tq4"].LIB_PATH
    assert lib_path.endswith("libtq4_stamps.so"), lib_path
    w = Workload(tq4, torch, dev, SLICES)
    torch.cuda.synchronize()
    nblk = B * HKV * w.splits
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    gs = [_graph(torch, stream, [lambda i=i: w.decode((32 * k + i) % SLICES) for i in range(32)])
          for k in range(4)]
    buf = np.zeros((4096, 16), np.uint64)
    rows = []
    for k in range(samples):
        with torch.cuda.stream(stream):
            gs[k % 4].replay()
        torch.cuda.synchronize()
        assert tq4.lib().tq4_decode_stamps(buf.ctypes.data_as(C.c_void_p), buf.nbytes) == 0
        st = buf[:nblk].astype(np.int64)
        t0 = st[:, 0].min()
        rel = np.where(st > 0, (st - t0) * 0.01, np.nan)  # 100 MHz counter -> us
        rows.append(rel)
    rel = np.stack(rows)  # [sample][workgroup][slot]
    out = {}
    for i, name in enumerate(PHASES):
        per = np.nanmedian(rel[:, :, i], axis=1) if np.isfinite(rel[:, :, i]).any() else None
        if per is not None:
            out[name] = round(float(np.nanmedian(per)), 3)
    exp = rel[:, :, 6]
    tail = np.nanmax(exp, axis=1) - np.nanmedian(exp, axis=1)
    out["split export spread (max - median)"] = round(float(np.nanmedian(tail)), 3)
    out["launch end (last combiner's egress)"] = round(float(np.nanmedian(np.nanmax(rel[:, :, 8], axis=1))), 3)
    out["workgroup start spread (max)"] = round(float(np.nanmedian(np.nanmax(rel[:, :, 0], axis=1))), 3)
    # host enqueue cost of one call (the GPU drains afterwards)
    torch.cuda.synchronize()
    n = 2000
    t = time.perf_counter()
    for i in range(n):
        w.decode(i % SLICES)
    host_us = (time.perf_counter() - t) / n * 1e6
    torch.cuda.synchronize()
    res = {"phases_us": out, "host_enqueue_us_per_call": round(host_us, 2),
           "workload": "configs[2] single-sequence decode, cold, graphs of 32 back-to-back "
                       "launches; stamps of the last launch (thread 0 of each workgroup)",
           "samples": samples, "workgroups": int(nblk), "library": "libtq4_stamps.so",
           "clock": "s_memrealtime, 100 MHz"}
    res["configs4_timeline"] = batched_timeline(tq4, torch, dev, w.signs)
    print(json.dumps(res), flush=True)


def batched_timeline(tq4, torch, dev, signs, samples=24, bin_us=2.0):
    """The configs[4] persistent decode per queue item, from the measurement
    build: graphs of 8 launches alternating the bench's two batches (each
    read cold); after each replay the last launch's per-item stamps. Per
    phase the median and 90th percentile over items; a least-squares fit of
    item duration (start to end) = fixed + per_page * pages; and, per
    `bin_us` bin from the launch's first item start, the items in flight and
    the cache bytes streamed, each item's strips (pages x 2176 B) spread
    evenly over its strip loop (first strip pairs issued to wave 0's loop
    done) -- an attribution, not a counter. Medians over samples."""
    import ctypes as C
    bats = [Batch(tq4, torch, dev, 0x71340050 + k, signs) for k in range(2)]
    K = bats[0].K
    assert all(b.ctxs == bats[0].ctxs and b.K == K for b in bats)
    pages_seq = np.array([(c + 1 + S - 1) // S for c in bats[0].ctxs])
    width = -(-bats[0].tab_np.shape[1] // K)
    n_items = int(HKV * (np.maximum(1, -(-pages_seq // width)) - 1).sum() + len(pages_seq) * HKV)
    assert n_items <= 4096, n_items
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    g = _graph(torch, stream, [bats[i % 2].decode for i in range(8)])
    buf = np.zeros((4096, 16), np.uint64)
    names = (("queue item -> phase-0 loads retired", 10, 1),
             ("phase-0 loads retired -> first strip pairs issued", 1, 2),
             ("first strip pairs issued -> q operands built", 2, 3),
             ("q operands built -> wave 0 strip loop done", 3, 4),
             ("strip loop done -> waves merged", 4, 5), ("waves merged -> item end", 5, 11))
    edges = np.arange(0.0, 200.0 + bin_us, bin_us)
    fits, ends, last_start, bws, acts, phs = [], [], [], [], [], []
    for k in range(samples + 2):
        with torch.cuda.stream(stream):
            g.replay()
        torch.cuda.synchronize()
        assert tq4.lib().tq4_decode_stamps(buf.ctypes.data_as(C.c_void_p), buf.nbytes) == 0
        if k < 2:
            continue  # the first replays warm the graph
        st = buf[:n_items].astype(np.int64)
        rel = (st - st[:, 10].min()) * 0.01  # 100 MHz counter -> us
        pg = np.minimum(width, pages_seq[st[:, 12]] - st[:, 13] * width).astype(float)
        start, end = rel[:, 10], rel[:, 11]
        coef = np.linalg.lstsq(np.stack([np.ones_like(pg), pg], 1), end - start, rcond=None)[0]
        fits.append(coef)
        ends.append(end.max())
        last_start.append(start.max())
        phs.append([np.median(rel[:, b] - rel[:, a]) for _, a, b in names] +
                   [np.percentile(rel[:, b] - rel[:, a], 90) for _, a, b in names])
        bw = np.zeros(len(edges) - 1)
        act = np.zeros(len(edges) - 1)
        for a, b, nbytes, s0, s1 in zip(rel[:, 2], rel[:, 4], pg * (2 * S * D // 2 + 2 * S * 4),
                                        start, end):
            if b > a:
                bw += nbytes * (np.clip(edges[1:], a, b) - np.clip(edges[:-1], a, b)) / (b - a)
            act += (np.clip(edges[1:], s0, s1) - np.clip(edges[:-1], s0, s1)) / bin_us
        bws.append(bw / (bin_us * 1e-6) / 1e12)
        acts.append(act)
    ph = np.median(np.array(phs), 0)
    nb = int(np.ceil(np.median(ends) / bin_us))
    fit = np.median(np.array(fits), 0)
    return {
        "splits": K, "items": n_items, "width_pages": int(width),
        "phase_us_median_p90": {n: [round(float(ph[i]), 2), round(float(ph[i + len(names)]), 2)]
                                for i, (n, _, _) in enumerate(names)},
        "item_us_fit": {"fixed": round(float(fit[0]), 2), "per_page": round(float(fit[1]), 4)},
        "last_item_start_us": round(float(np.median(last_start)), 2),
        "launch_end_us": round(float(np.median(ends)), 2),
        "bin_us": bin_us,
        "items_in_flight": [round(float(x), 1) for x in np.median(np.array(acts), 0)[:nb]],
        "attributed_TBps": [round(float(x), 2) for x in np.median(np.array(bws), 0)[:nb]],
        "workload": "configs[4] decode (the bench's two batches alternating, K = the "
                    "length-aware auto count), per-item stamps of the persistent kernel"}


def floor(tq4, torch, dev, rounds=2):
    """Compute-free copies beside the real kernels (libtq4_floor.so, built by
    `make -C ascend-micro-harness_amd/csrc floor`): the configs[2] decode's
    chain by cumulative stage (0: launch and output words; 1: + phase 0;
    2: + the strip loads of two pairs per wave and the merge barrier; 3: +
    tickets, device-coherent record export, the last ticket's poll and
    zeroing) on the headline's own cold workload and grid; the configs[1]
    writer's traffic (0: stores only; 1: loads and stores) on its own inputs;
    the same two stages for the token scatter (configs[1]'s secondary row:
    slot, rows and the dependent value-strip read, strip written back whole);
    and the configs[4] decode's cache strips read once each, at 2, 4 and 8
    workgroups per CU, beside the real batched decode; and the strips of one
    ctx-65536 sequence (rotated, cold) at 1 and 4 workgroups per CU, the
    former the decode's K = 32 grid size. Every case is timed as
    the bench rows are (graph replays), `rounds` times alternating, in one
    process."""
    import ctypes

    class FloorDecode(ctypes.Structure):
        _fields_ = [(n, ctypes.c_void_p) for n in (
            "q", "key_cache", "value_cache", "scale_cache", "block_tables", "context_lens",
            "pi_signs", "records", "tickets", "out")] + \
            [(n, ctypes.c_uint32) for n in ("B", "Hq", "Hkv", "G", "S", "P", "max_blocks", "K",
                                            "mode")]

    class FloorWriter(ctypes.Structure):
        _fields_ = [(n, ctypes.c_void_p) for n in (
            "key", "value", "slots", "key_cache", "value_cache", "scale_cache")] + \
            [(n, ctypes.c_uint32) for n in ("H", "D", "S", "P", "tokens", "mode")]

    class FloorScatter(ctypes.Structure):
        _fields_ = [(n, ctypes.c_void_p) for n in (
            "key", "value", "slots", "key_cache", "value_cache", "scale_cache")] + \
            [(n, ctypes.c_uint32) for n in ("H", "D", "S", "P", "tokens", "mode")]

    class FloorGather(ctypes.Structure):
        _fields_ = [(n, ctypes.c_void_p) for n in (
            "key_cache", "value_cache", "scale_cache", "rows", "out")] + \
            [(n, ctypes.c_uint32) for n in ("n_rows", "P", "Hkv")]

    import __graft_entry__
    lib = ctypes.CDLL(os.path.join(__graft_entry__.PKG_DIR, "libtq4_floor.so"))
    for fn in (lib.tq4_floor_decode_launch, lib.tq4_floor_writer_launch,
               lib.tq4_floor_scatter_launch):
        fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        fn.restype = ctypes.c_int
    lib.tq4_floor_gather_launch.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32]
    lib.tq4_floor_gather_launch.restype = ctypes.c_int
    log(f"prefilling {SLICES} config-3 sequences ({SLICES * PAGES} pages)")
    w = Workload(tq4, torch, dev, SLICES)
    if w.splits != 16:
        raise SystemExit(f"the decode floor copies the 16-split chain; auto splits gave {w.splits}")
    records = torch.zeros(B * HQ * 16 * (D + 4), dtype=torch.float32, device=dev)
    tickets = torch.zeros(B * HKV * 32, dtype=torch.int32, device=dev)
    out = torch.empty((B, HQ, D), dtype=torch.bfloat16, device=dev)

    def decode_case(mode):
        ps = []
        for i in range(SLICES):
            fp = FloorDecode(w.q[i].data_ptr(), w.kc.data_ptr(), w.vc.data_ptr(),
                             w.sc.data_ptr(), w.tables[i].data_ptr(), w.ctx.data_ptr(),
                             w.signs.data_ptr(), records.data_ptr(), tickets.data_ptr(),
                             out.data_ptr(), B, HQ, HKV, HQ // HKV, S, w.pool, PAGES, 16, mode)
            ps.append(fp)

        def launch(fp):
            rc = lib.tq4_floor_decode_launch(torch.cuda.current_stream().cuda_stream,
                                             ctypes.addressof(fp))
            if rc != 0:
                raise RuntimeError(f"tq4_floor_decode_launch returned {rc}")
        return [lambda fp=fp: launch(fp) for fp in ps]

    wr = WriterInputs(tq4, torch, dev, w, 32, 1024)

    def writer_case(mode):
        ps = []
        for k, v, slots in wr.ins:
            ps.append(FloorWriter(k.data_ptr(), v.data_ptr(), slots.data_ptr(), wr.kc.data_ptr(),
                                  wr.vc.data_ptr(), wr.sc.data_ptr(), HKV, D, S, wr.pool,
                                  wr.tokens, mode))

        def launch(fp):
            rc = lib.tq4_floor_writer_launch(torch.cuda.current_stream().cuda_stream,
                                             ctypes.addressof(fp))
            if rc != 0:
                raise RuntimeError(f"tq4_floor_writer_launch returned {rc}")
        return [lambda fp=fp: launch(fp) for fp in ps]

    # configs[1] secondary: the scatter row's own inputs (one token in each of
    # 1024 distinct strips, random positions), built as extra_workloads does
    srng = np.random.default_rng(0x71340012)
    sins = []
    for k, v, _ in wr.ins:
        strips = srng.permutation(wr.pool * S // 16)[:wr.tokens]
        sins.append((k, v, torch.from_numpy(
            (strips * 16 + srng.integers(0, 16, wr.tokens)).astype(np.int32)).to(dev)))

    def scatter_case(mode):
        ps = [FloorScatter(k.data_ptr(), v.data_ptr(), sl.data_ptr(), wr.kc.data_ptr(),
                           wr.vc.data_ptr(), wr.sc.data_ptr(), HKV, D, S, wr.pool, wr.tokens,
                           mode) for k, v, sl in sins]

        def launch(fp):
            rc = lib.tq4_floor_scatter_launch(torch.cuda.current_stream().cuda_stream,
                                              ctypes.addressof(fp))
            if rc != 0:
                raise RuntimeError(f"tq4_floor_scatter_launch returned {rc}")
        return [lambda fp=fp: launch(fp) for fp in ps]

    def real_scatter(i):
        k, v, sl = sins[i]
        tq4.reshape_scatter(k, v, wr.kc, wr.vc, wr.sc, sl, w.signs, num_blocks=wr.pool,
                            block_size=S, inv_sqrt_len=w.isl)

    # the two batches the bench rotates, as strip lists
    log("prefilling two configs[4] batches")
    bats = [Batch(tq4, torch, dev, 0x71340050 + k, w.signs) for k in range(2)]
    gbufs, gbytes = [], []
    for b in bats:
        rows = []
        for i, c in enumerate(b.ctxs):
            pages = (c + 1 + S - 1) // S  # the step's context: c + 1 tokens
            phys = b.tab_np[i, :pages].astype(np.int64)
            rows.append(((phys[:, None] * HKV + np.arange(HKV)[None, :]) * S).reshape(-1))
        rows = np.concatenate(rows).astype(np.uint32)
        gbufs.append((b, torch.from_numpy(rows.view(np.int32)).to(dev)))
        gbytes.append(int(rows.size) * (S * D + 2 * S * 4))
    gout = torch.zeros(65536, dtype=torch.int32, device=dev)
    cus = torch.cuda.get_device_properties(dev).multi_processor_count

    def gather_case(per_cu):
        ps = [FloorGather(b.kc.data_ptr(), b.vc.data_ptr(), b.sc.data_ptr(), rows.data_ptr(),
                          gout.data_ptr(), rows.numel(), b.pool, HKV) for b, rows in gbufs]

        def launch(fp):
            rc = lib.tq4_floor_gather_launch(torch.cuda.current_stream().cuda_stream,
                                             ctypes.addressof(fp), cus * per_cu)
            if rc != 0:
                raise RuntimeError(f"tq4_floor_gather_launch returned {rc}")
        return [lambda fp=fp: launch(fp) for fp in ps]

    # configs[3] ctx 65536: single sequences of random pool pages, rotated
    # over enough of them that each is read cold (as the split sweep does)
    lctx = 65536
    lpages = lctx // S
    nseq = max(4, (512 << 20) // (lctx * HKV * (D + 8)))
    lrng = np.random.default_rng(0x71340004)
    lrows = []
    for _ in range(nseq):
        phys = lrng.permutation(w.pool)[:lpages].astype(np.int64)
        r = ((phys[:, None] * HKV + np.arange(HKV)[None, :]) * S).reshape(-1).astype(np.uint32)
        lrows.append(torch.from_numpy(r.view(np.int32)).to(dev))
    lbytes = lpages * HKV * (S * D + 2 * S * 4)

    def long_case(per_cu):
        ps = [FloorGather(w.kc.data_ptr(), w.vc.data_ptr(), w.sc.data_ptr(), rows.data_ptr(),
                          gout.data_ptr(), rows.numel(), w.pool, HKV) for rows in lrows]

        def launch(fp):
            rc = lib.tq4_floor_gather_launch(torch.cuda.current_stream().cuda_stream,
                                             ctypes.addressof(fp), cus * per_cu)
            if rc != 0:
                raise RuntimeError(f"tq4_floor_gather_launch returned {rc}")
        return [lambda fp=fp: launch(fp) for fp in ps]

    cases = [("decode_stage0", decode_case(0)), ("decode_stage1", decode_case(1)),
             ("decode_stage2", decode_case(2)), ("decode_stage3", decode_case(3)),
             ("decode", [lambda i=i: w.decode(i) for i in range(SLICES)]),
             ("writer_stores", writer_case(0)), ("writer_loads_stores", writer_case(1)),
             ("writer", [lambda i=i: wr.write(i) for i in range(len(wr.ins))]),
             ("scatter_stores", scatter_case(0)), ("scatter_loads_stores", scatter_case(1)),
             ("scatter", [lambda i=i: real_scatter(i) for i in range(len(sins))]),
             ("gather_2_per_cu", gather_case(2)), ("gather_4_per_cu", gather_case(4)),
             ("gather_8_per_cu", gather_case(8)),
             ("batched_decode", [b.decode for b in bats]),
             ("ctx65536_gather_1_per_cu", long_case(1)), ("ctx65536_gather_4_per_cu", long_case(4))]
    res = {name: [] for name, _ in cases}
    for _ in range(rounds):
        for name, fns in cases:
            big = name.startswith(("gather", "batched", "ctx65536"))
            r = time_launches(torch, fns, 32 if big else 1024, 4 if big else 128)
            res[name].append(round(r["ms"] * 1e3, 3))
            log(f"{name}: {res[name][-1]} us")
    torch.cuda.synchronize()
    if int(tickets.abs().sum().item()) != 0:
        raise RuntimeError("the decode floor left a ticket counter set")
    cache_bytes = sum(gbytes) / len(gbytes)
    tbs = {name: [round(cache_bytes / (us * 1e-6) / 1e12, 2) for us in res[name]]
           for name in res if name.startswith(("gather", "batched"))}
    ltbs = {name: [round(lbytes / (us * 1e-6) / 1e12, 2) for us in res[name]]
            for name in res if name.startswith("ctx65536")}
    print(json.dumps({
        "floor_us": res,
        "configs4_cache_bytes": int(cache_bytes),
        "configs4_cache_TBps": tbs,
        "ctx65536_cache_bytes": int(lbytes),
        "ctx65536_cache_TBps": ltbs,
        "workload": "configs[2] cold (the headline's sequences, grid and buffers), configs[1] "
                    "(1024 BF16 tokens, 32 input sets; the strip writer and the token scatter "
                    "at one token per strip) and configs[4] (its two batches rotated; cache "
                    "strips only); compute-free copies beside the real kernels, graphs of 1024 "
                    "(32 for configs[4]) launches, alternating",
        "library": "libtq4_floor.so"}), flush=True)


def pmc_row_names():
    names = ["configs2_decode", "configs4_decode", "configs4_step_scatter", "configs1_writer",
             "configs1_scatter", "rms_writer", "configs0_a8", "kv4_ref_shape", "kv4_batched",
             "codebook_lloyd", "codebook_icdf"]
    for ctx, ks in SWEEP:
        names += [sweep_row(ctx, k) for k in ks if k]
        names.append(sweep_row(ctx, "auto"))
    return names


def pmc_kernel_of(row):
    """(kernel-name fragment, workgroups or None) of a PMC row's dispatches."""
    fixed = {"configs2_decode": ("decode_kernel<128, 1>", B * HKV * 16),
             "configs4_step_scatter": ("scatter_token_writer<128>", None),
             "configs1_writer": ("strip_writer<128, unsigned short>", 512),
             "configs1_scatter": ("scatter_token_writer<128>", None),
             "rms_writer": ("rms_writer<128, 1>", None),
             "configs0_a8": ("strip_writer<128, signed char>", None),
             "kv4_ref_shape": ("kv4_decode_kernel", None), "kv4_batched": ("kv4_decode_kernel", None),
             "codebook_lloyd": ("quantize_kernel", None), "codebook_icdf": ("icdf_kernel", None)}
    if row in fixed:
        return fixed[row]
    if row == "configs4_decode":
        return ("decode_", None)  # the kernel the auto split count selects
    if row.startswith("sweep_"):
        return ("decode_kernel<128, 1>", None)
    raise SystemExit(f"unknown PMC row {row}")


def pmc_workload(tq4, torch, dev, row):
    """One bench row's workload on the bench's own input shapes (at least 8
    launches of its kernel, cold where the bench is cold), then a plain copy
    of CALIB_BYTES (the row run's calibration)."""
    if row not in pmc_row_names():
        raise SystemExit(f"unknown PMC row {row}; known: {' '.join(pmc_row_names())}")
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x71340007)
    if row == "configs2_decode" or row.startswith("sweep_"):
        # no set-up pass: a sweep row's kernel may share the headline's grid
        w = Workload(tq4, torch, dev, 32, touch=row == "configs2_decode")
        if row == "configs2_decode":
            for i in range(32):
                w.decode(i)
        else:
            ctx = int(row.split("_")[1][3:])
            kk = row.split("_")[2][1:]
            pages = (ctx + S - 1) // S
            k = tq4.auto_splits(1, HKV, pages, S) if kk == "auto" else int(kk)
            rng = np.random.default_rng(0x71340004)
            ws = tq4.decode_workspace(1, HQ, HKV, D, k)
            ctx_t = torch.tensor([ctx], dtype=torch.int32, device=dev)
            out = torch.empty((1, HQ, D), dtype=torch.bfloat16, device=dev)
            for _ in range(8):
                tab = torch.from_numpy(rng.permutation(w.pool)[:pages].astype(np.int32)[None, :]).to(dev)
                q = torch.randn((1, HQ, D), generator=gen, device=dev).to(torch.bfloat16)
                tq4.paged_decode(q, w.kc, w.vc, w.sc, tab, ctx_t, w.signs, HKV, S, w.pool,
                                 out=out, workspace=ws, num_splits=k, scale=w.scale,
                                 inv_sqrt_len=w.isl)
    elif row in ("configs4_decode", "configs4_step_scatter"):
        signs = torch.ones(D, device=dev)
        bats = [Batch(tq4, torch, dev, 0x71340050 + k, signs) for k in range(2)]
        for _ in range(4):
            for b in bats:
                b.decode() if row == "configs4_decode" else b.scatter()
    elif row in ("configs1_writer", "configs1_scatter", "rms_writer", "configs0_a8"):
        w = Workload(tq4, torch, dev, 1, touch=False)
        wr = WriterInputs(tq4, torch, dev, w, 8)
        if row == "configs1_writer":
            for i in range(8):
                wr.write(i)
        elif row == "configs1_scatter":
            rng = np.random.default_rng(0x71340008)
            for i in range(8):
                k, v, _ = wr.ins[i]
                strips = rng.permutation(wr.pool * S // 16)[:1024]
                sl = torch.from_numpy((strips * 16 + rng.integers(0, 16, 1024)).astype(np.int32)).to(dev)
                tq4.reshape_scatter(k, v, wr.kc, wr.vc, wr.sc, sl, w.signs, num_blocks=wr.pool,
                                    block_size=S, inv_sqrt_len=w.isl)
        elif row == "rms_writer":
            rpool = wr.pool * S
            rkc = torch.zeros(rpool * HKV * D // 2, dtype=torch.int8, device=dev)
            rvc = torch.zeros_like(rkc)
            rsc = torch.zeros(rpool * tq4.rms_scale_slot_floats(HKV), device=dev)
            for i in range(8):
                k, v, slots = wr.ins[i]
                tq4.rms_reshape_and_cache(k, v, rkc, rvc, rsc, slots, w.signs, num_blocks=wr.pool,
                                          block_size=S, inv_sqrt_len=w.isl)
        else:
            ident = torch.arange(S, dtype=torch.int32, device=dev)
            for _ in range(8):
                k = torch.randint(-127, 128, (S, HKV, D), dtype=torch.int8, device=dev, generator=gen)
                v = torch.randint(-127, 128, (S, HKV, D), dtype=torch.int8, device=dev, generator=gen)
                tq4.reshape_and_cache_a8(k, v, wr.kc, wr.vc, wr.sc, ident, pi_signs=w.signs,
                                         num_blocks=wr.pool, block_size=S, inv_sqrt_len=w.isl)
    elif row.startswith("kv4_"):
        kv4fp8_workloads(tq4, torch, dev, None, only=row, launches=8)
    elif row == "codebook_lloyd":
        x = torch.randn(1 << 25, generator=gen, device=dev)
        r_, c_ = torch.empty_like(x), torch.empty((1 << 24), dtype=torch.uint8, device=dev)
        for _ in range(8):
            tq4.lloydmax_quantize(x, 4, 0, dst=r_, codes=c_)
    elif row == "codebook_icdf":
        x = torch.randn(1 << 26, generator=gen, device=dev).to(torch.float16)
        c_ = torch.empty((1 << 25), dtype=torch.uint8, device=dev)
        for _ in range(8):
            tq4.icdf_quantize(x, out=c_)
    torch.cuda.synchronize()
    src = torch.ones(CALIB_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(4):
        torch.mul(src, 2.0, out=dst)  # the calibration copy: reads and writes CALIB_BYTES
    torch.cuda.synchronize()
    log(f"pmc workload {row} done")


class WriterInputs:
    """1024 BF16 tokens per launch into a 4096-page pool at the
    pages of a seeded permutation; `n` input sets rotated."""

    def __init__(self, tq4, torch, dev, w, n, tokens=1024, pool=4096):
        self.tq4, self.w, self.tokens, self.pool = tq4, w, tokens, pool
        rng = np.random.default_rng(0x71340002)
        gen = torch.Generator(device=dev)
        gen.manual_seed(0x71340002)
        self.kc = torch.zeros(pool * HKV * S * D // 2, dtype=torch.int8, device=dev)
        self.vc = torch.zeros_like(self.kc)
        self.sc = torch.zeros(2 * pool * HKV * S, device=dev)
        ar = torch.arange(S, device=dev, dtype=torch.int32)
        self.ins = []
        for _ in range(n):
            pages = torch.from_numpy(rng.permutation(pool)[: tokens // S].astype(np.int32)).to(dev)
            slots = (pages[:, None] * S + ar[None, :]).reshape(-1).contiguous()
            k = torch.randn((tokens, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
            v = torch.randn((tokens, HKV, D), generator=gen, device=dev).to(torch.bfloat16)
            self.ins.append((k, v, slots))
        self.rng = rng

    def write(self, i):
        k, v, slots = self.ins[i]
        self.tq4.reshape_and_cache_bf16(k, v, self.kc, self.vc, self.sc, slots,
                                        pi_signs=self.w.signs, num_blocks=self.pool,
                                        block_size=S, inv_sqrt_len=self.w.isl)


def extra_workloads(tq4, torch, dev, w, pmc, cpu=True):
    """Every other BASELINE row, each with its spread and CPU leg."""
    out = {}
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x71340006)
    orc = oracle() if cpu else None
    # --- 1024 BF16 tokens, 4096-page pool, permuted pages; 32 input sets rotated
    wt, nin = 1024, 32
    wr = WriterInputs(tq4, torch, dev, w, nin, wt)
    res = time_launches(torch, [lambda i=i: wr.write(i) for i in range(nin)], 512, 64)
    wbytes = writer_algorithmic_bytes(wt, HKV, D, 2)
    row = {"workload": "configs[1] BF16 1024 tokens -> 4096-page pool", **row_times(res),
           "tokens_per_s": round(wt / (res["ms"] * 1e-3), 1),
           "GBps": round(wbytes / (res["ms"] * 1e-3) / 1e9, 2), "algorithmic_bytes": wbytes,
           "roofline": roofline(wbytes, res["ms"], "configs1_writer", pmc)}
    if cpu:
        from oracle_bindings import IN_BF16
        k, v, slots = (t.cpu() for t in wr.ins[0])
        hk = k.view(torch.int16).numpy().view(np.uint16)
        hv = v.view(torch.int16).numpy().view(np.uint16)
        hs = slots.numpy()
        nbytes = wr.pool * HKV * S * D // 2
        ck, cv = np.zeros(nbytes, np.int8), np.zeros(nbytes, np.int8)
        cs = np.zeros(2 * wr.pool * HKV * S, np.float32)
        row["cpu_baseline"] = cpu_leg(
            lambda t: orc.reshape_and_cache(IN_BF16, hk, hv, ck, cv, cs, hs, w.signs_np, HKV, D, S,
                                            wr.pool, np.float32(w.isl), threads=t),
            wt, "tokens/s", "oracle/tq4_oracle.c writer, the same 1024 tokens", 2.0, wt // 16)
    out["reshape_and_cache"] = row
    log(f"reshape_and_cache: {res['ms'] * 1e3:.2f} us -> {wt / (res['ms'] * 1e-3) / 1e6:.1f} "
        f"M tokens/s")

    # --- configs[1], secondary: the same tokens at token-granular slots
    # through the scatter writer, which merges each token into its value
    # strip (RMW). The writer's contract gives a strip one owner per launch,
    # so the slots are a random token position in each of 1024 distinct
    # strips (of the pool's 4096).
    rng = wr.rng
    sins = []
    for i in range(nin):
        k, v, _ = wr.ins[i]
        strips = rng.permutation(wr.pool * S // 16)[:wt]
        sl = torch.from_numpy((strips * 16 + rng.integers(0, 16, wt)).astype(np.int32)).to(dev)
        sins.append((k, v, sl))

    def scatter(i):
        k, v, sl = sins[i]
        tq4.reshape_scatter(k, v, wr.kc, wr.vc, wr.sc, sl, w.signs, num_blocks=wr.pool,
                            block_size=S, inv_sqrt_len=w.isl)

    res = time_launches(torch, [lambda i=i: scatter(i) for i in range(nin)], 512, 64)
    sbytes = wbytes + wt * HKV * 2 * (D * S // 2)  # + the value-strip read and write-back
    row = {"workload": "configs[1] secondary: 1024 BF16 tokens, one per strip at random "
                       "positions (value-strip RMW)", **row_times(res),
           "tokens_per_s": round(wt / (res["ms"] * 1e-3), 1),
           "GBps": round(sbytes / (res["ms"] * 1e-3) / 1e9, 2), "algorithmic_bytes": sbytes,
           "roofline": roofline(sbytes, res["ms"], "configs1_scatter", pmc)}
    if cpu:
        k, v, sl = (t.cpu() for t in sins[0])
        hk = k.view(torch.int16).numpy().view(np.uint16)
        hv = v.view(torch.int16).numpy().view(np.uint16)
        hs = sl.numpy()
        cu = np.array([0, wt], np.int32)
        row["cpu_baseline"] = cpu_leg(
            lambda t: orc.reshape_scatter(hk, hv, ck, cv, cs, hs, w.signs_np, cu, 1, HKV, D, S,
                                          wr.pool, 0, HKV, np.float32(w.isl)),
            wt, "tokens/s", "oracle/tq4_oracle.c scatter writer (single-threaded; the "
            "'all cores' run is the same call), the same 1024 tokens", 1.0, 1)
    out["reshape_scatter"] = row
    log(f"reshape_scatter: {res['ms'] * 1e3:.2f} us")

    # --- N2: the vllm-ascend RMS codec writer on the same 1024 BF16 tokens
    # (rows at slot * kv_heads, the slot's 8-float scale record)
    rpool = wr.pool * S
    rkc = torch.zeros(rpool * HKV * D // 2, dtype=torch.int8, device=dev)
    rvc = torch.zeros_like(rkc)
    rsc = torch.zeros(rpool * tq4.rms_scale_slot_floats(HKV), device=dev)

    def rms(i):
        k, v, slots = wr.ins[i]
        tq4.rms_reshape_and_cache(k, v, rkc, rvc, rsc, slots, w.signs, num_blocks=wr.pool,
                                  block_size=S, inv_sqrt_len=w.isl)

    res = time_launches(torch, [lambda i=i: rms(i) for i in range(nin)], 512, 64)
    rbytes = rms_writer_algorithmic_bytes(wt, HKV, D, 2)
    row = {"workload": "N2 RMS + threshold codec writer, 1024 BF16 tokens (the reference "
                       "bench's baseline writer)", **row_times(res),
           "tokens_per_s": round(wt / (res["ms"] * 1e-3), 1),
           "GBps": round(rbytes / (res["ms"] * 1e-3) / 1e9, 2), "algorithmic_bytes": rbytes,
           "roofline": roofline(rbytes, res["ms"], "rms_writer", pmc)}
    if cpu:
        k, v, slots = (t.cpu() for t in wr.ins[0])
        hk = k.view(torch.int16).numpy().view(np.uint16)
        hv = v.view(torch.int16).numpy().view(np.uint16)
        hs = slots.numpy()
        ok = np.zeros(rpool * HKV * D // 2, np.int8)
        ov = np.zeros_like(ok)
        os_ = np.zeros(rpool * tq4.rms_scale_slot_floats(HKV), np.float32)
        row["cpu_baseline"] = cpu_leg(
            lambda t: orc.rms_reshape_and_cache(1, hk, hv, ok, ov, os_, hs, w.signs_np, HKV, D,
                                                S, wr.pool, wt, np.float32(w.isl)),
            wt, "tokens/s", "oracle/tq4_oracle.c RMS codec writer (single-threaded; the "
            "'all cores' run is the same call), the same 1024 tokens", 1.0, 1)
    out["rms_reshape_and_cache"] = row
    log(f"rms writer: {res['ms'] * 1e3:.2f} us")

    # --- one 16-token A8 strip, uniform ints in [-127, 127], slot = identity
    # into page 0 (latency-bound: one strip x 8 heads)
    a8 = [(torch.randint(-127, 128, (S, HKV, D), dtype=torch.int8, device=dev, generator=gen),
           torch.randint(-127, 128, (S, HKV, D), dtype=torch.int8, device=dev, generator=gen))
          for _ in range(8)]
    ident = torch.arange(S, dtype=torch.int32, device=dev)

    def write_a8(i):
        k, v = a8[i]
        tq4.reshape_and_cache_a8(k, v, wr.kc, wr.vc, wr.sc, ident, pi_signs=w.signs,
                                 num_blocks=wr.pool, block_size=S, inv_sqrt_len=w.isl)

    res = time_launches(torch, [lambda i=i: write_a8(i) for i in range(8)], 512, 64,
                        chunk=64)
    abytes = writer_algorithmic_bytes(S, HKV, D, 1)
    row = {"workload": "configs[0] A8, one 16-token strip", **row_times(res),
           "tokens_per_s": round(S / (res["ms"] * 1e-3), 1), "algorithmic_bytes": abytes,
           "roofline": roofline(abytes, res["ms"], "configs0_a8", pmc)}
    if cpu:
        from oracle_bindings import IN_INT8
        hk, hv = a8[0][0].cpu().numpy(), a8[0][1].cpu().numpy()
        hs = ident.cpu().numpy()
        row["cpu_baseline"] = cpu_leg(
            lambda t: orc.reshape_and_cache(IN_INT8, hk, hv, ck, cv, cs, hs, w.signs_np, HKV, D,
                                            S, wr.pool, np.float32(w.isl), threads=t),
            S, "tokens/s", "oracle/tq4_oracle.c writer, the same A8 strip (one task: the "
            "'all cores' run uses one thread)", 1.0, 1)
    out["reshape_and_cache_a8"] = row
    log(f"reshape_and_cache A8 strip: {res['ms'] * 1e3:.2f} us")

    # --- split sweep over the headline pool
    out["split_sweep"] = split_sweep(tq4, torch, dev, w, orc, pmc)

    # --- the batched step, two batches rotated (each 0.3 GB,
    # more than the Infinity Cache, so each step reads its batch cold)
    bats = [Batch(tq4, torch, dev, 0x71340050 + k, w.signs) for k in range(2)]
    res = time_launches(torch, [b.step for b in bats], 32, 4, samples=16, chunk=8)
    t_step = sum(tq4.decode_poll_timeouts(b.ws, 64, HKV) for b in bats if b.ws is not None)
    resd = time_launches(torch, [b.decode for b in bats], 32, 4, samples=16, chunk=8)
    t_step += sum(tq4.decode_poll_timeouts(b.ws, 64, HKV) for b in bats if b.ws is not None)
    sbytes, dbytes = bats[0].step_bytes(), bats[0].decode_bytes()
    bsz = len(bats[0].ctxs)
    row = {"workload": "configs[4] 64 seqs ctx~U[512,8192]: scatter 64 tokens + split-K decode",
           **row_times(res), "tokens_per_s": round(bsz / (res["ms"] * 1e-3), 1),
           "GBps": round(sbytes / (res["ms"] * 1e-3) / 1e9, 2),
           "pct_hbm_peak": round(100 * sbytes / (res["ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 2),
           "splits": bats[0].K, "auto_splits": True, "algorithmic_bytes": sbytes,
           "cache": "cold (2 batches of 0.3 GB rotated)",
           "decode_only": {**row_times(resd), "GBps": round(dbytes / (resd["ms"] * 1e-3) / 1e9, 2),
                           "algorithmic_bytes": dbytes,
                           "overhead_bytes": decode_overhead_bytes(
                               [c + 1 for c in bats[0].ctxs], HQ, HKV, D, S, bats[0].K,
                               bats[0].tables.shape[1])},
           "roofline": roofline(dbytes, resd["ms"], "configs4_decode", pmc),
           "poll_timeouts": t_step}
    if t_step:
        row["INVALID"] = f"{t_step} combine rows gave up their bounded poll"
    if cpu:
        # a bounded sample: the first 8 sequences of batch 0 (decode + their scatter)
        b0 = bats[0]
        nseq = 8
        hq = b0.q[:nseq].cpu().view(torch.int16).numpy().view(np.uint16)
        hk, hv, hs = b0.kc.cpu().numpy(), b0.vc.cpu().numpy(), b0.sc.cpu().numpy()
        htab = np.ascontiguousarray(b0.tab_np[:nseq])
        hctx = b0.ctx_now[:nseq].cpu().numpy()
        sample_bytes = decode_algorithmic_bytes([c + 1 for c in b0.ctxs[:nseq]], HQ, HKV, D, S)
        row["cpu_baseline"] = cpu_leg(
            lambda t: orc.paged_decode(hq, hk, hv, hs, htab, hctx, w.signs_np, None, HQ, HKV, D,
                                       S, b0.pool, b0.K, np.float32(b0.isl),
                                       np.float32(b0.isl), 1, threads=t),
            sample_bytes, "GB/s", f"oracle/tq4_oracle.c decode of sequences 0..{nseq - 1} of the "
            f"batch (ctx sum {sum(b0.ctxs[:nseq]) + nseq}, {b0.K} splits)", 3.0,
            nseq * HKV * b0.K)
    out["batched_step"] = row
    log(f"batched step: {res['ms'] * 1e3:.2f} us -> {sbytes / (res['ms'] * 1e-3) / 1e9:.0f} GB/s; "
        f"decode only {resd['ms'] * 1e3:.2f} us")
    del bats

    # --- codebook leaves (HBM streams): Lloyd-Max 4-bit over 32M FP32 values
    # (in + centroids + codes), ICDF over 64M FP16 values (in + codes)
    nl = 1 << 25
    xl = torch.randn(nl, generator=gen, device=dev)
    rl = torch.empty_like(xl)
    cl = torch.empty(nl // 2, dtype=torch.uint8, device=dev)
    res_l = time_launches(torch, [lambda: tq4.lloydmax_quantize(xl, 4, 0, dst=rl, codes=cl)],
                          20, 4, samples=8, chunk=4)
    lbytes = nl * (4 + 4) + nl // 2
    xi = torch.randn(2 * nl, generator=gen, device=dev).to(torch.float16)
    ci = torch.empty(nl, dtype=torch.uint8, device=dev)
    res_i = time_launches(torch, [lambda: tq4.icdf_quantize(xi, out=ci)], 20, 4, samples=8,
                          chunk=4)
    ibytes = 2 * nl * 2 + nl
    out["codebook"] = {
        "lloydmax4_32M_fp32": {**row_times(res_l),
                               "GBps": round(lbytes / (res_l["ms"] * 1e-3) / 1e9, 1),
                               "algorithmic_bytes": lbytes,
                               "roofline": roofline(lbytes, res_l["ms"], "codebook_lloyd", pmc)},
        "icdf_64M_fp16": {**row_times(res_i), "GBps": round(ibytes / (res_i["ms"] * 1e-3) / 1e9, 1),
                          "algorithmic_bytes": ibytes,
                          "roofline": roofline(ibytes, res_i["ms"], "codebook_icdf", pmc)}}
    log(f"codebook: Lloyd-Max {lbytes / (res_l['ms'] * 1e-3) / 1e9:.0f} GB/s, "
        f"ICDF {ibytes / (res_i['ms'] * 1e-3) / 1e9:.0f} GB/s")
    out["kv4fp8_decode"] = kv4fp8_workloads(tq4, torch, dev, orc, pmc=pmc)

    # --- the practical streaming ceiling on this box: a plain device copy of
    # 512 MiB (1 GiB read + written per launch), two buffer pairs rotated
    n = (512 << 20) // 4
    bufs = [(torch.ones(n, device=dev), torch.empty(n, device=dev)) for _ in range(2)]
    res_c = time_launches(torch, [lambda i=i: bufs[i][1].copy_(bufs[i][0]) for i in range(2)],
                          16, 4, samples=8, chunk=4)
    cbytes = 2 * n * 4
    out["device_copy"] = {"workload": "torch copy_ of 512 MiB float32 (read + write 1 GiB)",
                          **row_times(res_c),
                          "GBps": round(cbytes / (res_c["ms"] * 1e-3) / 1e9, 1),
                          "pct_hbm_peak": round(100 * cbytes / (res_c["ms"] * 1e-3) / 1e9
                                                / HBM_PEAK_GBS, 2),
                          "algorithmic_bytes": cbytes}
    log(f"device copy: {cbytes / (res_c['ms'] * 1e-3) / 1e9:.0f} GB/s")
    del bufs
    return out


def kv4fp8_cache_bytes(tokens, ctx, kv_heads):
    """Live KV4/FP8 cache bytes, as the reference's benchmark counts them
    (Fixture::cache_bytes: 256 packed bytes per row and KV head for K and V,
    plus the row's 32-byte scale slot)."""
    return tokens * ctx * (kv_heads * 256 + 32)


def kv4fp8_workloads(tq4, torch, dev, orc=None, pmc=None, only=None, launches=0):
    """The KV4/FP8 NZ-tiled decode: the reference benchmark's shape
    (bench_turboquant_decode_splitk --impl fused-opt: 1 request, 16 q heads over
    one KV head, D=256, 128-row pages, FP32 pre-rotated query, FP16 output) at
    ctx 4096, and a batched case beyond the 256 MiB Infinity Cache."""
    res = {}
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x4B5F8)
    gain = 2.9832882881
    for name, (T, H, G, S_, ctx) in (("ref_shape_1x16q1kv_ctx4096", (1, 1, 16, 128, 4096)),
                                      ("batched_32x64q4kv_ctx8192", (32, 4, 16, 128, 8192))):
        row_name = "kv4_ref_shape" if T == 1 else "kv4_batched"
        if only is not None and only != row_name:
            continue
        pages = (ctx + S_ - 1) // S_
        P = T * pages
        key = torch.randint(0, 256, (P * S_ * H * 128,), dtype=torch.uint8, device=dev,
                            generator=gen)
        val = torch.randint(0, 256, key.shape, dtype=torch.uint8, device=dev, generator=gen)
        sc = (torch.rand(P * S_ * 8, device=dev, generator=gen) * 1.5 + 0.5) * gain
        tb = torch.randperm(P, device=dev, generator=gen).to(torch.int32).view(T, pages)
        ln = torch.full((T,), ctx, dtype=torch.int32, device=dev)
        q = torch.randn((T, H * G, 256), device=dev, generator=gen)
        o = torch.empty((T, H * G, 256), dtype=torch.float16, device=dev)
        L = tq4.fused_decode_opt_launch(T, H * G, H, S_, pages, num_blocks=P)
        ws = torch.zeros(tq4.kv4fp8_workspace_bytes(L), dtype=torch.uint8, device=dev)
        run = lambda: tq4.kv4fp8_decode(q, key, val, sc, tb, ln, H, S_, P, out=o,  # noqa: E731
                                        workspace=ws)
        run()
        torch.cuda.synchronize()
        assert torch.isfinite(o.float()).all(), "kv4fp8 decode produced non-finite values"
        if only is not None:  # the PMC workload: plain launches, no timing
            for _ in range(launches):
                run()
            continue
        # The batched case follows the reference shape's CPU baseline (the GPU
        # idle for about a second); its first ~8 ms of launches then run at
        # 64-66 us and later ones at 57-58 us, so it warms up for three
        # replays of its timed graph (about 11 ms)
        r = time_launches(torch, [run], 256 if T == 1 else 64, 32,
                          samples=16, chunk=16, warm_replays=0 if T == 1 else 3)
        timeouts = tq4.kv4fp8_poll_timeouts(ws, T, H * G, H, S_, pages, P)
        nbytes = kv4fp8_cache_bytes(T, ctx, H) + T * H * G * 256 * (4 + 2) + T * pages * 4
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        res[name] = {**row_times(r), "GBps": round(gbs, 1),
                     "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                     "tokens": T, "q_heads": H * G, "kv_heads": H, "head_dim": 256,
                     "ctx": ctx, "page_size": S_, "algorithmic_bytes": nbytes,
                     "cache": "warm" if nbytes < (256 << 20) else "beyond the Infinity Cache",
                     "poll_timeouts": timeouts,
                     "roofline": roofline(nbytes, r["ms"], row_name, pmc)}
        if timeouts:
            res[name]["INVALID"] = f"{timeouts} combine rows gave up their bounded poll"
        log(f"kv4fp8 {name}: {r['ms'] * 1e3:.2f} us -> {gbs:.0f} GB/s")
        if orc is not None and T == 1:
            h = [x.cpu().numpy() for x in (q, key, val, sc, tb, ln)]
            res[name]["cpu_baseline"] = cpu_leg(
                lambda t: orc.kv4fp8_decode(*h, heads=H * G, kv_heads=H, block_size=S_,
                                            max_blocks=pages, num_blocks=P, threads=t),
                nbytes, "GB/s", "oracle/kv4fp8_oracle.c decode of this shape (FP64 products; "
                "one task per (token, kv head))", 2.0, T * H)
    return res


def split_sweep(tq4, torch, dev, w, orc=None, pmc=None):
    """the fused decode at ctx {4096, 16384, 32768, 65536} x K
    {2, 4, 8, 16, auto}, plus the ragged ctx 4103 at auto; cold (each time
    rotates over enough sequences that >= 512 MB are read between re-reads).
    The CPU leg runs the auto-K row of each context."""
    rng = np.random.default_rng(0x71340004)
    gen = torch.Generator(device=dev)
    gen.manual_seed(0x71340004)
    rows = []
    for ctx, ks in SWEEP:
        pages = (ctx + S - 1) // S
        if pages > w.pool:
            continue
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

            r = time_launches(torch, [lambda i=i: dec(i) for i in range(nseq)], max(128, nseq),
                              max(16, nseq // 4), samples=16, chunk=max(8, min(32, nseq)))
            timeouts = tq4.decode_poll_timeouts(ws, 1, HKV)
            gbs = nbytes / (r["ms"] * 1e-3) / 1e9
            row = {"ctx": ctx, "splits": kk, "auto": k == 0, **row_times(r),
                   "GBps": round(gbs, 1), "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
                   "algorithmic_bytes": nbytes,
                   "overhead_bytes": decode_overhead_bytes([ctx], HQ, HKV, D, S, kk, pages),
                   "poll_timeouts": timeouts,
                   "roofline": roofline(nbytes, r["ms"], sweep_row(ctx, k or "auto"), pmc)}
            if timeouts:
                row["INVALID"] = f"{timeouts} combine rows gave up their bounded poll"
            if orc is not None and k == 0:
                hq = qs[0].cpu().view(torch.int16).numpy().view(np.uint16)
                htab = tabs[0].cpu().numpy()
                hctx = ctx_t.cpu().numpy()
                hk, hv, hs = w.host_cache()
                row["cpu_baseline"] = cpu_leg(
                    lambda t: orc.paged_decode(hq, hk, hv, hs, htab, hctx, w.signs_np, None, HQ,
                                               HKV, D, S, w.pool, kk, np.float32(w.scale),
                                               np.float32(w.isl), 1, threads=t),
                    nbytes, "GB/s", f"oracle/tq4_oracle.c decode, ctx {ctx}, {kk} splits",
                    2.0, HKV * kk)
            rows.append(row)
            log(f"split sweep ctx {ctx} K {kk}{' (auto)' if k == 0 else ''}: "
                f"{r['ms'] * 1e3:.2f} us -> {gbs:.0f} GB/s")
    return {"workload": "configs[3] single-sequence decode, 32q:8kv, d128, page 16, cold "
                        "(rotated sequences)", "rows": rows}


def _host_cache(self):
    if not hasattr(self, "_host"):
        self._host = (self.kc.cpu().numpy(), self.vc.cpu().numpy(), self.sc.cpu().numpy())
    return self._host


Workload.host_cache = _host_cache


def cpu_decode_leg(torch, w, dec_bytes, seconds):
    """The C oracle's decode of slice 0 on the host cores, bounded in time."""
    o = oracle()
    h_q = w.q[0].view(torch.int16).cpu().numpy().view(np.uint16)
    h_kc, h_vc, h_sc = w.host_cache()
    h_tab, h_ctx = w.tables[0].cpu().numpy(), w.ctx.cpu().numpy()
    return cpu_leg(
        lambda t: o.paged_decode(h_q, h_kc, h_vc, h_sc, h_tab, h_ctx, w.signs_np, None, HQ, HKV,
                                 D, S, w.pool, w.splits, np.float32(w.scale), np.float32(w.isl),
                                 1, threads=t),
        dec_bytes, "GB/s", f"oracle/tq4_oracle.c decode of one configs[2] sequence (B=1, "
        f"32q:8kv, d128, ctx4096, {w.splits} splits)", seconds, HKV * w.splits)


if __name__ == "__main__":
    main()
