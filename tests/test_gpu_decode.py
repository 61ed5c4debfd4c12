"""GPU parity of the paged split-K decode against the C oracle.

Tolerances (BF16 output, the north_star's): max-abs <= 2e-2 and mean-rel <=
1e-3 against the FP32 oracle rounded to BF16 (the same final rounding the
device applies); also reported against the FP64 reference. Partial records
are checked against the oracle's FP32 records with budgets 1e-3*max(1,|m|)
for m, 2e-3*max(1,l) for l and 2e-3*max|acc| + 1e-5*l + 1e-6 for acc, and
the empty-split neutral element exactly. The reference rig's budgets
(tests/npu/turboquant_splitk_rigs.hpp:144-158: m 2e-6, l 1e-4, acc 2e-4)
assume its exact BF16 score panel; the MFMA kernel feeds the rotated query
in fp16 and P * value scale in fp16, so a score carries a relative error up
to ~2^-11 and m moves by that much. TQ4_DECODE_PRECISE (FP32 recurrence,
BF16 q_rot) is held to the rig's budgets.
"""
import math

import numpy as np
import pytest

from gpu_helpers import bf16_out_error, canary_bytes, canary_floats, dev, host, record_margin
from oracle_bindings import (FLAG_PRECISE, FLAG_QROT_BF16, FLAG_QUERY_ROTATED, IN_BF16, bf16_to_f32,
                             f32_to_bf16)

pytestmark = pytest.mark.gpu

MAX_ABS = 2e-2
MEAN_REL = 1e-3


def build_cache(oracle, rng, ctx_lens, H, d, S, P, tail_canary=True):
    """Quantise N(0,1) K/V for every sequence through the oracle writer into a
    shuffled page pool; dead slots of partial pages keep the NaN canary."""
    B = len(ctx_lens)
    pages_per = [(c + S - 1) // S for c in ctx_lens]
    assert sum(pages_per) <= P
    perm = rng.permutation(P)
    max_blocks = max(max(pages_per), 1)
    tables = np.zeros((B, max_blocks), np.int32)
    nbytes = P * H * S * d // 2
    kc, vc, sc = canary_bytes(nbytes), canary_bytes(nbytes), canary_floats(2 * P * H * S)
    if not tail_canary:
        kc[:] = 0
        vc[:] = 0
        sc[:] = 0
    at = 0
    isl = np.float32(1.0 / math.sqrt(d))
    signs = oracle.canonical_signs(d)
    for b, c in enumerate(ctx_lens):
        n = pages_per[b]
        tables[b, :n] = perm[at:at + n]
        at += n
        tok = np.arange(c)
        slots = (tables[b, tok // S] * S + tok % S).astype(np.int32)
        # whole strips through the aligned writer, the tail through the scatter writer
        full = (c // 16) * 16
        if full:
            k = f32_to_bf16(rng.standard_normal((full, H, d)).astype(np.float32))
            v = f32_to_bf16(rng.standard_normal((full, H, d)).astype(np.float32))
            assert oracle.reshape_and_cache(IN_BF16, k, v, kc, vc, sc, slots[:full], signs, H, d,
                                            S, P, isl) == 0
        if c > full:
            t = c - full
            k = f32_to_bf16(rng.standard_normal((t, H, d)).astype(np.float32))
            v = f32_to_bf16(rng.standard_normal((t, H, d)).astype(np.float32))
            cu = np.array([0, t], np.int32)
            oracle.reshape_scatter(k, v, kc, vc, sc, slots[full:], signs, cu, 1, H, d, S, P, 0,
                                   H, isl)
    return kc, vc, sc, tables, signs, isl


def run_decode(tq4, oracle, rng, ctx_lens, Hq, H, d, S, P, K, stage=1, gate=None):
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx_lens, H, d, S, P)
    B = len(ctx_lens)
    ctx = np.array(ctx_lens, np.int32)
    q = f32_to_bf16(rng.standard_normal((B, Hq, d)).astype(np.float32))
    scale = np.float32(1.0 / math.sqrt(d))
    want16, want = oracle.paged_decode(q, kc, vc, sc, tables, ctx, signs, gate, Hq, H, d, S, P,
                                       K, scale, isl, stage, threads=8)
    out = tq4.paged_decode(dev(q), dev(kc), dev(vc), dev(sc), dev(tables), dev(ctx), dev(signs),
                           H, S, P, gate=dev(gate) if gate is not None else None, num_splits=K,
                           scale=float(scale), inv_sqrt_len=float(isl), output_stage=stage)
    return host(out), want, (q, kc, vc, sc, tables, ctx, signs, isl, scale)


def check_out(got, want, label="", max_abs=MAX_ABS, mean_rel=MEAN_REL):
    mx, mr = bf16_out_error(got, want)
    record_margin(label, mx, mr, max_abs, mean_rel)
    assert np.all(np.isfinite(bf16_to_f32(got))), f"{label}: non-finite output"
    assert mx <= max_abs and mr <= mean_rel, f"{label}: max-abs {mx:.3g} mean-rel {mr:.3g}"
    return mx, mr


def test_config3_single_sequence_ctx4096(tq4, oracle):
    """batch 1, 32q:8kv, d 128, ctx 4096, page 16."""
    rng = np.random.default_rng(0x71340003)
    got, want, _ = run_decode(tq4, oracle, rng, [4096], 32, 8, 128, 16, 4096, 32)
    check_out(got, want, "config3")


@pytest.mark.parametrize("ctx", [4096, 16384, 4103])
@pytest.mark.parametrize("K", [2, 4, 8, 16, 0])
def test_config4_split_sweep(tq4, oracle, ctx, K):
    """split-K sweep incl. ragged ctx 4103 (NaN canaries
    in the tail); K = 0 is the auto count the bench times."""
    rng = np.random.default_rng(0x71340004 + ctx + K)
    kk = K or tq4.auto_splits(1, 8, (ctx + 15) // 16, 16)
    got, want, _ = run_decode(tq4, oracle, rng, [ctx], 32, 8, 128, 16, (ctx + 15) // 16 + 8, kk)
    check_out(got, want, f"ctx {ctx} K {kk}{' (auto)' if K == 0 else ''}")


@pytest.mark.parametrize("K", [24, 40, 64])
def test_multi_chunk_combine_one_launch(tq4, oracle, K):
    """More than 16 live splits in the one-launch kernel: the combiner polls
    16 records per round trip, its own record (kept in registers) may sit in
    any chunk, and earlier chunks are zeroed after the last poll. Three calls
    on one workspace with different queries must each match the oracle (a
    record left unzeroed would be taken by the next call's poll)."""
    import torch
    rng = np.random.default_rng(0x5E20 + K)
    ctx = [4096 + 7]
    P = (ctx[0] + 15) // 16 + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx, 8, 128, 16, P)
    scale = np.float32(1 / math.sqrt(128))
    ws = tq4.decode_workspace(1, 32, 8, 128, K)
    args = [dev(kc), dev(vc), dev(sc), dev(tables), dev(np.array(ctx, np.int32)), dev(signs)]
    for call in range(3):
        q = f32_to_bf16(rng.standard_normal((1, 32, 128)).astype(np.float32))
        _, want = oracle.paged_decode(q, kc, vc, sc, tables, np.array(ctx, np.int32), signs,
                                      None, 32, 8, 128, 16, P, K, scale, isl, 1, threads=8)
        out = tq4.paged_decode(dev(q), *args, 8, 16, P, workspace=ws, num_splits=K,
                               scale=float(scale), inv_sqrt_len=float(isl))
        check_out(host(out), want, f"K {K} call {call}")


def multi_call_case(tq4, oracle, rng, ctx, Hq, H, d, K, calls, label):
    """`calls` decodes of one cache with fresh queries on one workspace, each
    against the oracle (a consumed record left unzeroed would be taken by
    the next call's poll)."""
    import torch
    P = sum((c + 15) // 16 for c in ctx) + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx, H, d, 16, P)
    scale = np.float32(1 / math.sqrt(d))
    ctx_a = np.array(ctx, np.int32)
    ws = tq4.decode_workspace(len(ctx), Hq, H, d, K)
    args = [dev(kc), dev(vc), dev(sc), dev(tables), dev(ctx_a), dev(signs)]
    for call in range(calls):
        q = f32_to_bf16(rng.standard_normal((len(ctx), Hq, d)).astype(np.float32))
        _, want = oracle.paged_decode(q, kc, vc, sc, tables, ctx_a, signs, None, Hq, H, d, 16,
                                      P, K, scale, isl, 1, threads=8)
        out = tq4.paged_decode(dev(q), *args, H, 16, P, workspace=ws, num_splits=K,
                               scale=float(scale), inv_sqrt_len=float(isl))
        check_out(host(out), want, f"{label} call {call}")


@pytest.mark.parametrize("d,K", [(64, 40), (256, 24)])
def test_multi_chunk_combine_head_sizes(tq4, oracle, d, K):
    """More than 16 live splits in the one-launch kernel at d = 64 (K = 40,
    three poll chunks) and d = 256 (K = 24, two; 8 x 24 workgroups stay
    within its 256 resident slots): the combiner's record loads, own-slot
    substitution and zeroing in their two- and eight-word lane layouts."""
    rng = np.random.default_rng(0x5E50 + d)
    multi_call_case(tq4, oracle, rng, [4096 + 7], 32, 8, d, K, 2, f"d {d} K {K}")


@pytest.mark.parametrize("d,K", [(128, 24), (128, 40), (256, 40)])
def test_persistent_multi_chunk_combine(tq4, oracle, d, K):
    """The persistent form with more than 16 live splits per (seq, kv head):
    its combiner stores its own record and polls it with the others, chunk
    by chunk (6 x 8 x K items exceed the resident workgroups: 512 at
    d = 128, 256 at d = 256); ragged lengths with an empty and a one-page
    sequence."""
    rng = np.random.default_rng(0x5E60 + K + d)
    multi_call_case(tq4, oracle, rng, [4103, 3001, 0, 17, 2500, 4096], 32, 8, d, K, 2,
                    f"persistent d {d} K {K}")


@pytest.fixture(scope="module")
def long_context(oracle):
    """One ctx-32768 sequence (configs[3]'s longest), cache built once."""
    rng = np.random.default_rng(0x71340004)
    P = 2048 + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, [32768], 8, 128, 16, P)
    q = f32_to_bf16(rng.standard_normal((1, 32, 128)).astype(np.float32))
    return P, q, kc, vc, sc, tables, signs, isl


@pytest.mark.parametrize("K", [2, 4, 8, 16, 32, 0])
def test_config4_ctx32768(tq4, oracle, long_context, K):
    """configs[3] at ctx 32768, every split count of the sweep and the auto
    count the bench times there (0 = tq4_decode_auto_splits)."""
    P, q, kc, vc, sc, tables, signs, isl = long_context
    ctx = np.array([32768], np.int32)
    kk = K or tq4.auto_splits(1, 8, tables.shape[1], 16)
    scale = np.float32(1.0 / math.sqrt(128))
    _, want = oracle.paged_decode(q, kc, vc, sc, tables, ctx, signs, None, 32, 8, 128, 16, P,
                                  kk, scale, isl, 1, threads=16)
    out = tq4.paged_decode(dev(q), dev(kc), dev(vc), dev(sc), dev(tables), dev(ctx), dev(signs),
                           8, 16, P, num_splits=K, scale=float(scale), inv_sqrt_len=float(isl))
    check_out(host(out), want, f"ctx 32768 K {kk}{' (auto)' if K == 0 else ''}")


@pytest.fixture(scope="module")
def longest_context(oracle):
    """One ctx-65536 sequence (the split sweep's longest row), cache built once."""
    rng = np.random.default_rng(0x71340014)
    P = 4096 + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, [65536], 8, 128, 16, P)
    q = f32_to_bf16(rng.standard_normal((1, 32, 128)).astype(np.float32))
    return P, q, kc, vc, sc, tables, signs, isl


@pytest.mark.parametrize("K", [8, 16, 32, 0])
def test_sweep_ctx65536(tq4, oracle, longest_context, K):
    """The split sweep's ctx 65536 rows (K 8, 16, 32 and the auto count the
    bench times): the longest single sequence timed, where the combine's
    mean-relative error grows most with context."""
    P, q, kc, vc, sc, tables, signs, isl = longest_context
    ctx = np.array([65536], np.int32)
    kk = K or tq4.auto_splits(1, 8, tables.shape[1], 16)
    scale = np.float32(1.0 / math.sqrt(128))
    _, want = oracle.paged_decode(q, kc, vc, sc, tables, ctx, signs, None, 32, 8, 128, 16, P,
                                  kk, scale, isl, 1, threads=16)
    print(f"ctx 65536 K {kk}", flush=True)
    out = tq4.paged_decode(dev(q), dev(kc), dev(vc), dev(sc), dev(tables), dev(ctx), dev(signs),
                           8, 16, P, num_splits=K, scale=float(scale), inv_sqrt_len=float(isl))
    check_out(host(out), want, f"ctx 65536 K {kk}{' (auto)' if K == 0 else ''}")


@pytest.mark.parametrize("G", [1, 4, 6, 16])
@pytest.mark.parametrize("d", [64, 128, 256])
def test_gqa_and_head_size(tq4, oracle, G, d):
    rng = np.random.default_rng(G * 1000 + d)
    H = 2
    got, want, _ = run_decode(tq4, oracle, rng, [333, 77], G * H, H, d, 32, 40, 3)
    check_out(got, want, f"G {G} d {d}")


@pytest.mark.parametrize("stage", [0, 2])
def test_output_stages(tq4, oracle, stage):
    rng = np.random.default_rng(50 + stage)
    gate = rng.standard_normal((2, 16, 128)).astype(np.float32) if stage == 2 else None
    got, want, _ = run_decode(tq4, oracle, rng, [500, 1000], 16, 4, 128, 16, 120, 4, stage, gate)
    check_out(got, want, f"stage {stage}")


def test_single_split_and_empty_splits(tq4, oracle):
    """K=1 finalises in-workgroup; K > pages leaves empty splits (neutral element)."""
    rng = np.random.default_rng(99)
    for K in (1, 40):
        got, want, _ = run_decode(tq4, oracle, rng, [5, 200, 17], 8, 2, 128, 16, 40, K)
        check_out(got, want, f"K {K}")


@pytest.mark.parametrize("case", ["k1", "k4", "persistent"])
def test_invalid_live_pages_are_skipped(tq4, oracle, case):
    """Table entries of live pages that name no page (negative or >= the
    pool) send their window through the masked path, which drops those
    pages' tokens. Softmax attention does not depend on token order, so the
    result must equal the oracle's over the same table with those pages
    removed and the context shortened by theirs. Invalid entries past the
    context change nothing. K = 1 puts an invalid page past the first 256
    entries of a window; "persistent" runs the work-queue form."""
    rng = np.random.default_rng({"k1": 0xBAD1, "k4": 0xBAD4, "persistent": 0xBAD8}[case])
    S, H, Hq, d = 16, 8, 32, 128
    if case == "persistent":
        ctx_lens, K = [int(x) for x in rng.integers(40, 1500, 80)], 8
    else:
        ctx_lens, K = [1000, 4200, 300], (1 if case == "k1" else 4)
    pages = [(c + S - 1) // S for c in ctx_lens]
    P = sum(pages) + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx_lens, H, d, S, P)
    bad = tables.copy()
    comp = np.zeros_like(tables)
    comp_ctx = []
    for b, c in enumerate(ctx_lens):
        full = c // S  # whole live pages (the partial last page stays)
        drop = set(int(i) for i in rng.choice(full, size=min(2, full // 2), replace=False))
        if case != "persistent" and b == 1:
            drop.add(260)  # past the first 256 entries of the K = 1 window
        for j, i in enumerate(sorted(drop)):
            bad[b, i] = -1 if j % 2 == 0 else P + 3
        keep = [tables[b, i] for i in range(pages[b]) if i not in drop]
        comp[b, :len(keep)] = keep
        comp_ctx.append(c - S * len(drop))
        if b == 2:
            bad[b, pages[b]:] = -1  # dead entries: no effect
    q = f32_to_bf16(rng.standard_normal((len(ctx_lens), Hq, d)).astype(np.float32))
    scale = np.float32(1.0 / math.sqrt(d))
    _, want = oracle.paged_decode(q, kc, vc, sc, comp, np.array(comp_ctx, np.int32), signs, None,
                                  Hq, H, d, S, P, K, scale, isl, 1, threads=8)
    got = tq4.paged_decode(dev(q), dev(kc), dev(vc), dev(sc), dev(bad),
                           dev(np.array(ctx_lens, np.int32)), dev(signs), H, S, P, num_splits=K,
                           scale=float(scale), inv_sqrt_len=float(isl), output_stage=1)
    check_out(host(got), want, f"invalid pages {case}")


def test_partials_match_oracle(tq4, oracle):
    """Partial records (m, l, acc) per split, incl. exact neutral records."""
    rng = np.random.default_rng(123)
    H, Hq, d, S, P, K = 2, 8, 128, 16, 64, 8
    ctx_lens = [100, 37]
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx_lens, H, d, S, P)
    ctx = np.array(ctx_lens, np.int32)
    q = f32_to_bf16(rng.standard_normal((2, Hq, d)).astype(np.float32))
    scale = np.float32(1.0 / math.sqrt(d))
    want = oracle.decode_partials(q, kc, vc, sc, tables, ctx, signs, Hq, H, d, S, P, K, scale, isl)
    ws = tq4.paged_decode_partials(dev(q), dev(kc), dev(vc), dev(sc), dev(tables), dev(ctx),
                                   dev(signs), H, S, P, K, scale=float(scale),
                                   inv_sqrt_len=float(isl))
    got = host(ws)
    m_g, l_g, a_g = got[..., 0], got[..., 1], got[..., 4:]
    m_w, l_w, a_w = want[..., 0], want[..., 1], want[..., 4:]
    empty = l_w == 0
    assert np.all(m_g[empty] == np.float32(-3e38)) and np.all(l_g[empty] == 0)
    assert np.all(a_g[empty] == 0)
    live = ~empty
    assert np.all(np.abs(m_g - m_w)[live] <= 1e-3 * np.maximum(1, np.abs(m_w[live])))
    assert np.all(np.abs(l_g - l_w)[live] <= 2e-3 * np.maximum(1, l_w[live]))
    amax = np.abs(a_w).max(axis=-1, keepdims=True)
    tol = 2e-3 * amax + 1e-5 * l_w[..., None] + 1e-6
    assert np.all(np.abs(a_g - a_w) <= tol)
    # and the separate combine kernel agrees with the oracle's combine
    out = tq4.splitk_combine(ws, dev(signs), 2, Hq, d, K, inv_sqrt_len=float(isl))
    _, want_out = oracle.combine(want, signs, None, Hq, d, K, isl, 1)
    check_out(host(out), want_out, "combine")


@pytest.mark.parametrize("d,G", [(128, 4), (64, 16), (256, 6)])
def test_precise_partials_rig_budgets(tq4, oracle, d, G):
    """TQ4_DECODE_PRECISE on an unrotated query: the kernel rotates q in FP32
    and rounds Pi q to BF16 (the reference device's score operand), the
    oracle does the same (FLAG_QROT_BF16); the records meet the reference
    rig's budgets (m 2e-6, l 1e-4, acc 2e-4: turboquant_splitk_rigs.hpp:144-158)
    for several split counts, a ragged tail whose dead slots hold NaN
    canaries, a short sequence with empty splits, and G up to 16 rows."""
    from test_gpu_golden import RIG, check_records
    rng = np.random.default_rng(0x7E5 + d + G)
    H, S = 2, 16
    Hq = H * G
    ctx_lens = [1000 + 7, 37]
    P = sum((c + S - 1) // S for c in ctx_lens) + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx_lens, H, d, S, P)
    ctx = np.array(ctx_lens, np.int32)
    q = f32_to_bf16(rng.standard_normal((2, Hq, d)).astype(np.float32))
    scale = np.float32(1.0 / math.sqrt(d))
    worst = [0.0, 0.0, 0.0]
    for K in (1, 3, 8):
        want = oracle.decode_partials(q, kc, vc, sc, tables, ctx, signs, Hq, H, d, S, P, K, scale,
                                      isl, flags=FLAG_QROT_BF16)
        ws = tq4.paged_decode_partials(dev(q), dev(kc), dev(vc), dev(sc), dev(tables), dev(ctx),
                                       dev(signs), H, S, P, K, scale=float(scale),
                                       inv_sqrt_len=float(isl), flags=FLAG_PRECISE)
        got = host(ws).astype(np.float64)
        for b in range(2):
            for h in range(Hq):
                for k in range(K):
                    rec = got[b, h, k][None]
                    w = want[b, h, k].astype(np.float64)
                    fr = check_records(rec, w[None, 0], w[None, 1], w[None, 4:], RIG,
                                       f"d {d} G {G} K {K} b {b} h {h} split {k}")
                    worst = [max(x, y) for x, y in zip(worst, fr)]
    print(f"precise partials d {d} G {G}: worst m/l/acc fraction of the rig budget "
          f"{worst[0]:.3f} / {worst[1]:.3f} / {worst[2]:.3f}")


def test_combine_uniform_closed_form(tq4, oracle):
    """Uniform records (all m equal): the combine is an exact sum, acc/l = c + 1."""
    K, d = 8, 128
    recs = np.zeros((1, 2, K, d + 4), np.float32)
    for k in range(K):
        recs[:, :, k, 0] = -4.0
        recs[:, :, k, 1] = 2.0 ** k
        recs[:, :, k, 4:] = (2.0 ** k) * (np.arange(d) + 1)
    out = tq4.splitk_combine(dev(recs), dev(oracle.canonical_signs(d)), 1, 2, d, K,
                             output_stage=0)
    got = host(out)
    want = f32_to_bf16((np.arange(d) + 1).astype(np.float32))
    assert np.array_equal(got[0, 0], want) and np.array_equal(got[0, 1], want)


def test_fused_repeated_calls_reset_counters(tq4, oracle):
    """The fused entry leaves its arrival counters at zero: calls in a row agree."""
    rng = np.random.default_rng(5)
    _, want, args = run_decode(tq4, oracle, rng, [700, 300], 16, 4, 128, 16, 80, 6)
    q, kc, vc, sc, tables, ctx, signs, isl, scale = args
    ws = tq4.decode_workspace(2, 16, 4, 128, 6)
    outs = []
    for _ in range(3):
        out = tq4.paged_decode(dev(q), dev(kc), dev(vc), dev(sc), dev(tables), dev(ctx),
                               dev(signs), 4, 16, 80, workspace=ws, num_splits=6,
                               scale=float(scale), inv_sqrt_len=float(isl))
        outs.append(host(out))
    for o in outs:
        check_out(o, want, "repeat")
        assert np.array_equal(o, outs[0])


def test_persistent_ragged_batch(tq4, oracle):
    """More (seq, kv head, split) items than resident workgroups: the fused
    entry runs its persistent form (live items only, a work queue). Ragged
    lengths incl. empty and one-token contexts."""
    rng = np.random.default_rng(0x5E11)
    ctx = [0, 1, 17, 4103, 2000, 15, 16, 33] + [int(x) for x in rng.integers(1, 3000, 56)]
    got, want, _ = run_decode(tq4, oracle, rng, ctx, 16, 4, 128, 16,
                              sum((c + 15) // 16 for c in ctx) + 8, 16)
    check_out(got, want, "persistent ragged")


@pytest.mark.parametrize("d", [64, 256])
def test_persistent_head_sizes_and_pages(tq4, oracle, d):
    """The persistent form at d = 64 and d = 256 (its other instantiations),
    32-token pages, GQA 3, ragged lengths with an empty sequence."""
    rng = np.random.default_rng(0x5E30 + d)
    ctx = [0, 5, 31, 32, 33] + [int(x) for x in rng.integers(1, 700, 75)]
    got, want, _ = run_decode(tq4, oracle, rng, ctx, 12, 4, d, 32,
                              sum((c + 31) // 32 for c in ctx) + 8, 8)
    check_out(got, want, f"persistent d {d}")


@pytest.mark.parametrize("S", [48, 64, 128])
@pytest.mark.parametrize("K", [1, 5, 0])
def test_large_pages(tq4, oracle, S, K):
    """Pages of 3, 4 and 8 strips: a split boundary falls inside a page's
    strip run only in whole pages, ragged tails end mid-page (NaN canaries
    in the dead slots); K = 0 takes the auto count."""
    rng = np.random.default_rng(0x5E40 + S + K)
    ctx = [1, S - 1, S, S + 1, 3 * S + 7, 2100]
    P = sum((c + S - 1) // S for c in ctx) + 4
    kk = K or tq4.auto_splits(len(ctx), 4, (max(ctx) + S - 1) // S, S)
    got, want, _ = run_decode(tq4, oracle, rng, ctx, 16, 4, 128, S, P, kk)
    check_out(got, want, f"S {S} K {kk}")


@pytest.mark.parametrize("B", [1000, 1100])
def test_persistent_large_batch(tq4, oracle, B):
    """Up to 1024 sequences the persistent kernel ranks the last splits by
    length (four ranks per thread at 1000, many ties); past that they run
    in sequence order."""
    rng = np.random.default_rng(0x5E14 + B)
    ctx = [int(x) for x in rng.integers(0, 160, B)]
    got, want, _ = run_decode(tq4, oracle, rng, ctx, 4, 1, 128, 16,
                              sum((c + 15) // 16 for c in ctx) + 8, 2)
    check_out(got, want, f"persistent B={B}")


@pytest.mark.parametrize("B", [1000, 64])
def test_short_splits_repeatable(tq4, oracle, B):
    """Splits of one to three 32-token pairs leave waves without pairs; those
    park their merge rows while the other waves may still be reading the
    staged q rows, so the two LDS areas must not overlap. Six calls on one
    workspace (the persistent kernel at B = 1000, the one-launch kernel at
    B = 64) must each match the oracle and be bit-identical to the first."""
    import torch
    rng = np.random.default_rng(0x5E30 + B)
    # page 16, 10 pages per table, K = 2: the last split (pages 5..) holds
    # 1..80 tokens, mostly one to three pairs
    ctx = [int(x) for x in rng.integers(81, 160, B)]
    P = sum((c + 15) // 16 for c in ctx) + 8
    Hq, H, d, S, K = 4, 1, 128, 16, 2
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx, H, d, S, P)
    ctx_a = np.array(ctx, np.int32)
    q = f32_to_bf16(rng.standard_normal((B, Hq, d)).astype(np.float32))
    scale = np.float32(1.0 / math.sqrt(d))
    _, want = oracle.paged_decode(q, kc, vc, sc, tables, ctx_a, signs, None, Hq, H, d, S, P, K,
                                  scale, isl, 1, threads=8)
    ws = tq4.decode_workspace(B, Hq, H, d, K)
    args = [dev(q), dev(kc), dev(vc), dev(sc), dev(tables), dev(ctx_a), dev(signs)]
    first = None
    for call in range(6):
        out = tq4.paged_decode(*args, H, S, P, workspace=ws, num_splits=K, scale=float(scale),
                               inv_sqrt_len=float(isl))
        torch.cuda.synchronize()
        got = host(out)
        check_out(got, want, f"short splits B={B} call {call}")
        if first is None:
            first = got
        else:
            assert np.array_equal(got, first), f"call {call} differs from call 0"
    assert tq4.decode_poll_timeouts(ws, B, H) == 0


@pytest.mark.parametrize("case", [
    # (ctx lengths, Hq, H, d, page, K): configs[2]; ragged with 40 splits
    # (three record chunks); GQA 16 at d = 256; short splits at d = 64
    ([4096], 32, 8, 128, 16, 16),
    ([4103], 32, 8, 128, 16, 40),
    ([700, 1500], 32, 2, 256, 32, 6),
    ([90, 33, 160, 7], 8, 4, 64, 16, 8),
])
def test_one_launch_repeat_bit_identical(tq4, oracle, case):
    """The one-launch fused decode, four calls on one workspace: every call
    matches the oracle and has the first call's bits (the output may not
    depend on which split takes the last ticket or on wave timing)."""
    import torch
    ctx, Hq, H, d, S, K = case
    rng = np.random.default_rng(0x5E40 + d + K)
    P = sum((c + S - 1) // S for c in ctx) + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx, H, d, S, P)
    ctx_a = np.array(ctx, np.int32)
    q = f32_to_bf16(rng.standard_normal((len(ctx), Hq, d)).astype(np.float32))
    scale = np.float32(1.0 / math.sqrt(d))
    _, want = oracle.paged_decode(q, kc, vc, sc, tables, ctx_a, signs, None, Hq, H, d, S, P, K,
                                  scale, isl, 1, threads=8)
    ws = tq4.decode_workspace(len(ctx), Hq, H, d, K)
    args = [dev(q), dev(kc), dev(vc), dev(sc), dev(tables), dev(ctx_a), dev(signs)]
    first = None
    for call in range(4):
        out = tq4.paged_decode(*args, H, S, P, workspace=ws, num_splits=K, scale=float(scale),
                               inv_sqrt_len=float(isl))
        torch.cuda.synchronize()
        got = host(out)
        check_out(got, want, f"repeat {ctx} K {K} call {call}")
        if first is None:
            first = got
        else:
            assert np.array_equal(got, first), f"call {call} differs from call 0"
    assert tq4.decode_poll_timeouts(ws, len(ctx), H) == 0


def test_persistent_fewer_live_items_than_slots(tq4, oracle):
    """A large split grid whose live items are fewer than the resident
    workgroups: the surplus workgroups leave at once, nobody fetches."""
    rng = np.random.default_rng(0x5E12)
    ctx = [int(x) for x in rng.integers(0, 40, 48)] + [900]
    got, want, _ = run_decode(tq4, oracle, rng, ctx, 8, 8, 128, 16,
                              sum((c + 15) // 16 for c in ctx) + 8, 64)
    check_out(got, want, "persistent sparse")


def test_persistent_repeat_and_graph(tq4, oracle):
    """The queue counter resets itself: calls in a row and HIP-graph replays
    on one workspace all give the first call's bits."""
    import torch
    rng = np.random.default_rng(0x5E13)
    ctx = [int(x) for x in rng.integers(200, 2500, 40)]
    P = sum((c + 15) // 16 for c in ctx) + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx, 4, 128, 16, P)
    q = f32_to_bf16(rng.standard_normal((len(ctx), 16, 128)).astype(np.float32))
    scale = np.float32(1 / math.sqrt(128))
    want16, want = oracle.paged_decode(q, kc, vc, sc, tables, np.array(ctx, np.int32), signs,
                                       None, 16, 4, 128, 16, P, 12, scale, isl, 1, threads=8)
    args = [dev(q), dev(kc), dev(vc), dev(sc), dev(tables), dev(np.array(ctx, np.int32)),
            dev(signs)]
    ws = tq4.decode_workspace(len(ctx), 16, 4, 128, 12)
    out = torch.empty_like(args[0])
    call = lambda: tq4.paged_decode(*args, 4, 16, P, out=out, workspace=ws, num_splits=12,
                                    scale=float(scale), inv_sqrt_len=float(isl))
    call()
    first = host(out).copy()
    check_out(first, want, "persistent first")
    for _ in range(3):
        call()
        assert np.array_equal(host(out), first)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        call()
    for _ in range(3):
        g.replay()
        assert np.array_equal(host(out), first)
        call()
        assert np.array_equal(host(out), first)
