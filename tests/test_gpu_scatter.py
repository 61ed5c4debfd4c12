"""GPU parity of reshape_scatter (arbitrary slots) against the C oracle, and
a batched decode step (64 sequences, ctx ~U[512, 8192],
write the new tokens at slot ctx_b, then split-K decode with ctx_b + 1).

Bit-exact cache images (the value strip's unowned nibbles preserved, canary
everywhere nothing was written); decode per sequence within the north_star's
BF16 tolerance (max-abs 2e-2, mean-rel 1e-3 vs the FP32 oracle rounded to BF16).
"""
import math

import numpy as np
import pytest
import torch

from gpu_helpers import bf16_out_error, canary_bytes, canary_floats, dev, host, record_margin
from oracle_bindings import f32_to_bf16

pytestmark = pytest.mark.gpu


def scatter_pair(tq4, oracle, key, val, slots, cu, R, H, d, S, P, prior=None, item_begin=0,
                 item_count=None, block_dim=0, probe=None):
    nb = P * H * S * d // 2
    if prior is None:
        prior = (canary_bytes(nb), canary_bytes(nb), canary_floats(2 * P * H * S))
    o = [x.copy() for x in prior]
    g = [dev(x) for x in prior]
    isl = np.float32(1 / math.sqrt(d))
    signs = oracle.canonical_signs(d)
    count = R * H if item_count is None else item_count
    oracle.reshape_scatter(key, val, *o, slots, signs, cu, R, H, d, S, P, item_begin, count, isl)
    tq4.reshape_scatter(dev(key), dev(val), *g, dev(slots), dev(signs),
                        cu_seqlens=dev(cu) if cu is not None else None, launch_probe=probe,
                        num_requests=R, num_blocks=P, block_size=S, item_begin=item_begin,
                        item_count=count, block_dim=block_dim, inv_sqrt_len=float(isl))
    return [host(x) for x in g], o


def strip_disjoint_slots(rng, R, P, S):
    """R slots in R distinct strips: the writer's contract gives each strip one
    owner per launch (pages belong to one sequence), so two requests never
    share a value strip's read-modify-write."""
    strips = rng.choice(P * S // 16, R, replace=False)
    return (strips * 16 + rng.integers(0, 16, R)).astype(np.int32)


def assert_same(got, want):
    for a, b in zip(got, want):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), np.count_nonzero(a.view(np.uint8) != b.view(np.uint8))


@pytest.mark.parametrize("d", [64, 128, 256])
def test_decode_step_single_tokens(tq4, oracle, d):
    """One token per request (cu_seqlens NULL) at random slots, one owner per strip."""
    rng = np.random.default_rng(d)
    R, H, S, P = 64, 8, 16, 512
    slots = strip_disjoint_slots(rng, R, P, S)
    key = f32_to_bf16(rng.standard_normal((R, H, d)).astype(np.float32))
    val = f32_to_bf16(rng.standard_normal((R, H, d)).astype(np.float32))
    got, want = scatter_pair(tq4, oracle, key, val, slots, None, R, H, d, S, P)
    assert_same(got, want)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_single_tokens_zero_pad_wide_rows(tq4, oracle, d):
    """The one-token writer (cu_seqlens NULL) on random prior bytes: an
    all-zero key and value row (codes 0, scale 1.0), slot -1 pads, a slot past
    the pool, and rows scaled by 2^k, k in [-60, 60] (the exact policy's
    exponent far below the prefill floor)."""
    rng = np.random.default_rng(0x5CA7 + d)
    R, H, S, P = 48, 4, 32, 64
    slots = strip_disjoint_slots(rng, R, P, S)
    slots[5] = -1
    slots[17] = -1
    slots[30] = P * S + 3  # past the pool
    k = rng.integers(-60, 61, (2, R, H, 1)).astype(np.float64)
    x = rng.standard_normal((2, R, H, d)) * np.exp2(k)
    key, val = (f32_to_bf16(x[i].astype(np.float32)) for i in range(2))
    key[9] = 0
    val[9] = 0
    nb = P * H * S * d // 2
    prior = (rng.integers(-128, 128, nb, dtype=np.int8), rng.integers(-128, 128, nb, dtype=np.int8),
             rng.standard_normal(2 * P * H * S).astype(np.float32))
    got, want = scatter_pair(tq4, oracle, key, val, slots, None, R, H, d, S, P, prior=prior)
    assert_same(got, want)


def test_single_tokens_item_window_past_2_32(tq4, oracle):
    """An item window reaching past 2^32 (the writer's 64-bit item loop):
    every item there belongs to no request, so nothing is written."""
    R, H, d, S, P = 8, 4, 128, 16, 16
    rng = np.random.default_rng(32)
    slots = strip_disjoint_slots(rng, R, P, S)
    key = f32_to_bf16(rng.standard_normal((R, H, d)).astype(np.float32))
    val = f32_to_bf16(rng.standard_normal((R, H, d)).astype(np.float32))
    got, want = scatter_pair(tq4, oracle, key, val, slots, None, R, H, d, S, P,
                             item_begin=0xFFFFFF00, item_count=0x200)
    assert_same(got, want)
    nb = P * H * S * d // 2
    assert np.array_equal(got[0].view(np.uint8), canary_bytes(nb).view(np.uint8))


def test_runs_pads_zero_rows_and_preservation(tq4, oracle):
    """Runs that cross strips, slot -1 pads, an all-zero row, random prior bytes."""
    rng = np.random.default_rng(9)
    H, d, S, P = 4, 128, 32, 16
    cu = np.array([0, 7, 8, 20, 20, 23], np.int32)
    R = len(cu) - 1
    slots = np.concatenate([np.arange(13, 20), [100], np.arange(40, 52), [-1, 200, 201]]).astype(np.int32)
    slots[10] = -1
    key = f32_to_bf16(rng.standard_normal((cu[-1], H, d)).astype(np.float32) * 4)
    val = f32_to_bf16(rng.standard_normal((cu[-1], H, d)).astype(np.float32) * 4)
    key[3] = 0
    val[3] = 0
    nb = P * H * S * d // 2
    prior = (rng.integers(-128, 128, nb, dtype=np.int8), rng.integers(-128, 128, nb, dtype=np.int8),
             rng.standard_normal(2 * P * H * S).astype(np.float32))
    got, want = scatter_pair(tq4, oracle, key, val, slots, cu, R, H, d, S, P, prior=prior)
    assert_same(got, want)


def test_item_window_grid_stride_and_probe(tq4, oracle):
    """A sub-range of items on a small grid (items strided by the grid size)
    and the launch probe fields."""
    rng = np.random.default_rng(4)
    R, H, d, S, P = 40, 4, 128, 16, 64
    slots = strip_disjoint_slots(rng, R, P, S)
    key = f32_to_bf16(rng.standard_normal((R, H, d)).astype(np.float32))
    val = f32_to_bf16(rng.standard_normal((R, H, d)).astype(np.float32))
    probe = torch.full((32,), -7, dtype=torch.int32, device="cuda")
    got, want = scatter_pair(tq4, oracle, key, val, slots, None, R, H, d, S, P, item_begin=10,
                             item_count=100, block_dim=7, probe=probe)
    assert_same(got, want)
    pr = host(probe)
    assert list(pr[0:8]) == [0] * 8 and list(pr[8:16]) == [7] * 8
    assert list(pr[16:24]) == [1] * 8 and list(pr[24:32]) == [100] * 8


def test_config5_batched_decode_step(tq4, oracle):
    """64 sequences, ctx ~U[512, 8192] (seeded), 32q:8kv,
    d 128, page 16, shuffled tables from a shared pool. The prefix is written by
    the aligned writer, the new token of each sequence by the scatter writer;
    then split-K decode over ctx_b + 1."""
    rng = np.random.default_rng(0x71340005)
    B, Hq, H, d, S = 64, 32, 8, 128, 16
    ctx = rng.integers(512, 8193, B).astype(np.int32)
    pages_per = (ctx + 1 + S - 1) // S
    P = int(pages_per.sum() * 1.1) + 8
    perm = rng.permutation(P)
    maxb = int(pages_per.max())
    tables = np.zeros((B, maxb), np.int32)
    at = 0
    for b in range(B):
        tables[b, :pages_per[b]] = perm[at:at + pages_per[b]]
        at += pages_per[b]
    nb = P * H * S * d // 2
    kc, vc, sc = dev(canary_bytes(nb)), dev(canary_bytes(nb)), dev(canary_floats(2 * P * H * S))
    signs = oracle.canonical_signs(d)
    isl = 1.0 / math.sqrt(d)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    for b in range(B):  # prefix: whole strips (aligned writer) + the partial tail (scatter)
        c = int(ctx[b])
        full = c // 16 * 16
        tok = np.arange(c)
        sl = (tables[b, tok // S] * S + tok % S).astype(np.int32)
        k = torch.randn((c, H, d), generator=gen, device="cuda").to(torch.bfloat16)
        v = torch.randn((c, H, d), generator=gen, device="cuda").to(torch.bfloat16)
        if full:
            tq4.reshape_and_cache_bf16(k[:full].contiguous(), v[:full].contiguous(), kc, vc, sc,
                                       dev(sl[:full]), pi_signs=dev(signs), num_blocks=P,
                                       block_size=S, inv_sqrt_len=isl)
        if c > full:
            tq4.reshape_scatter(k[full:].contiguous(), v[full:].contiguous(), kc, vc, sc,
                                dev(sl[full:]), dev(signs), cu_seqlens=dev(np.array([0, c - full], np.int32)),
                                num_requests=1, num_blocks=P, block_size=S, inv_sqrt_len=isl)
    # the decode step: one new token per sequence at slot ctx_b (scatter), checked bit-exact
    new_slots = (tables[np.arange(B), ctx // S] * S + ctx % S).astype(np.int32)
    nk = f32_to_bf16(rng.standard_normal((B, H, d)).astype(np.float32))
    nv = f32_to_bf16(rng.standard_normal((B, H, d)).astype(np.float32))
    before = [host(kc), host(vc), host(sc)]
    o = [x.copy() for x in before]
    oracle.reshape_scatter(nk, nv, *o, new_slots, signs, None, B, H, d, S, P, 0, B * H, np.float32(isl))
    tq4.reshape_scatter(dev(nk), dev(nv), kc, vc, sc, dev(new_slots), dev(signs), num_requests=B,
                        num_blocks=P, block_size=S, inv_sqrt_len=isl)
    after = [host(kc), host(vc), host(sc)]
    assert_same(after, o)
    # split-K decode over ctx + 1, against the oracle on the same cache image:
    # the length-blind auto split count (K = 2 for this 513-page table), and
    # the length-aware one that bench.py times for this batch (K = 3: the
    # persistent work-queue kernel, 64 x 8 x 3 items > the resident workgroup
    # slots) on a fresh workspace
    q = f32_to_bf16(rng.standard_normal((B, Hq, d)).astype(np.float32))
    ctx1 = (ctx + 1).astype(np.int32)
    scale = np.float32(1 / math.sqrt(d))
    _, want = oracle.paged_decode(q, after[0], after[1], after[2], tables, ctx1, signs, None, Hq,
                                  H, d, S, P, 1, scale, np.float32(isl), 1, threads=16)
    k_lens = tq4.auto_splits(B, H, maxb, S, context_lens=ctx1)
    assert k_lens == 3, k_lens  # the ragged batch the rule is for
    for K in (0, k_lens):
        ws = tq4.decode_workspace(B, Hq, H, d, K) if K else None
        print(f"configs[4] decode K={K or 'auto'}", flush=True)
        out = tq4.paged_decode(dev(q), kc, vc, sc, dev(tables), dev(ctx1), dev(signs), H, S, P,
                               workspace=ws, num_splits=K, scale=float(scale), inv_sqrt_len=isl)
        got = host(out)
        for b in range(B):
            mx, mr = bf16_out_error(got[b], want[b])
            record_margin(f"configs[4] K={K or 'auto'} seq {b}", mx, mr, 2e-2, 1e-3)
            assert mx <= 2e-2 and mr <= 1e-3, (K, b, mx, mr)
        if K:
            # the work queue deals items to workgroups in a different order
            # on every call; the output must not depend on it
            for call in range(3):
                again = tq4.paged_decode(dev(q), kc, vc, sc, dev(tables), dev(ctx1), dev(signs),
                                         H, S, P, workspace=ws, num_splits=K,
                                         scale=float(scale), inv_sqrt_len=isl)
                assert np.array_equal(host(again), got), f"K={K} call {call + 1} differs"
            assert tq4.decode_poll_timeouts(ws, B, H) == 0
