"""The bounded waits of both fused decodes report a give-up to the host.

A combiner polls the other parts' records at most a bounded number of times;
if records are still missing it combines what arrived and adds one to a
sticky count in the workspace (tq4_decode_poll_timeouts,
tq4_kv4fp8_poll_timeouts), the way the reference's watchdog publishes a
timeout (kernels/ops/turboquant/turboquant_splitk_reduce.cpp:34-45).

The give-up is forced from the host with the test hooks (never set in use):
a 16-attempt poll bound, and the part holding ticket 0 of every group
skipping its record, so the combiners that need it give up. Every workgroup
still exits. Then the workspace is zeroed again and a normal call on it must
match the oracle and report no timeout.
"""
import math

import numpy as np
import pytest
import torch

from gpu_helpers import dev, host
from test_gpu_decode import build_cache, check_out
from oracle_bindings import f32_to_bf16

pytestmark = pytest.mark.gpu


def decode_case(oracle, rng, ctx_lens, H, d, S):
    P = sum((c + S - 1) // S for c in ctx_lens) + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx_lens, H, d, S, P)
    return P, [dev(kc), dev(vc), dev(sc), dev(tables), dev(np.array(ctx_lens, np.int32)),
               dev(signs)], (kc, vc, sc, tables, signs, isl)


@pytest.mark.parametrize("B,K,persistent", [(1, 4, False), (64, 4, True)])
def test_tq4_forced_poll_timeout_is_counted(tq4, oracle, B, K, persistent):
    rng = np.random.default_rng(0x7130 + B)
    Hq, H, d, S = 32, 8, 128, 16
    ctx_lens = [int(x) for x in rng.integers(600, 2049, B)] if B > 1 else [2048]
    P, args, (kc, vc, sc, tables, signs, isl) = decode_case(oracle, rng, ctx_lens, H, d, S)
    if persistent:  # more (seq, kv head, split) items than workgroup slots
        assert B * H * K > 2 * 256
    scale = 1.0 / math.sqrt(d)
    ws = tq4.decode_workspace(B, Hq, H, d, K)
    q = f32_to_bf16(rng.standard_normal((B, Hq, d)).astype(np.float32))
    hooks = tq4.TQ4_DECODE_TEST_POLL_BOUND | tq4.TQ4_DECODE_TEST_WITHHOLD
    print(f"forced give-up: B={B} K={K}", flush=True)
    tq4.paged_decode(dev(q), *args, H, S, P, workspace=ws, num_splits=K, scale=scale,
                     inv_sqrt_len=float(isl), flags=hooks)
    # every (seq, kv head) with two or more live splits: its G rows gave up
    maxb = tables.shape[1]
    width = -(-maxb // K)
    live = [-(-(-(-c // S)) // width) for c in ctx_lens]
    expected = sum(Hq for k in live if k >= 2)
    assert expected > 0
    got = tq4.decode_poll_timeouts(ws, B, H)
    assert got == expected, (got, expected)
    # zeroed again, a normal call is exact and reports nothing
    tq4.decode_workspace_init(ws)
    _, want = oracle.paged_decode(q, kc, vc, sc, tables, np.array(ctx_lens, np.int32), signs,
                                  None, Hq, H, d, S, P, K, np.float32(scale), isl, 1, threads=16)
    out = tq4.paged_decode(dev(q), *args, H, S, P, workspace=ws, num_splits=K, scale=scale,
                           inv_sqrt_len=float(isl))
    got_out = host(out)
    for b in range(B):
        check_out(got_out[b], want[b], f"seq {b} after re-init")
    assert tq4.decode_poll_timeouts(ws, B, H) == 0


def test_tq4_hook_flags_are_checked(tq4):
    """The withhold hook is refused without its poll bound (a wait of 2^20
    polls per row), and unknown flag bits are refused."""
    q = torch.zeros(1, 8, 128, dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros(4 * 2 * 16 * 64, dtype=torch.int8, device="cuda")
    sc = torch.zeros(2 * 4 * 2 * 16, device="cuda")
    tb = torch.zeros(1, 4, dtype=torch.int32, device="cuda")
    ln = torch.full((1,), 64, dtype=torch.int32, device="cuda")
    sg = torch.ones(128, device="cuda")
    for flags in (tq4.TQ4_DECODE_TEST_WITHHOLD, 1 << 5):
        with pytest.raises(ValueError, match="flag"):
            tq4.paged_decode(q, kc, kc, sc, tb, ln, sg, 2, 16, 4, num_splits=2, flags=flags)


def test_kv4fp8_forced_poll_timeout_is_counted(tq4, oracle):
    from test_gpu_kv4fp8 import bits, compare, random_case
    rng = np.random.default_rng(0x7131)
    T, H, G, S, ctx = 2, 2, 16, 128, [2048, 1500]
    P = sum((c + S - 1) // S for c in ctx) + 3
    q, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, ctx, key_scale=(0.5, 2.0))
    pages = tb.shape[1]
    L = tq4.fused_decode_opt_launch(T, H * G, H, S, pages, num_blocks=P)
    ws = torch.zeros(tq4.kv4fp8_workspace_bytes(L), dtype=torch.uint8, device="cuda")
    args = (dev(q), dev(key), dev(val), dev(sc), dev(tb), dev(ln), H, S, P)
    print("kv4fp8 forced give-up", flush=True)
    tq4.kv4fp8_decode(*args, workspace=ws,
                      test_flags=tq4.TQ4_KV4FP8_TEST_POLL_BOUND | tq4.TQ4_KV4FP8_TEST_WITHHOLD)
    got = tq4.kv4fp8_poll_timeouts(ws, T, H * G, H, S, pages, P)
    assert 0 < got <= T * H * G, got
    with pytest.raises(ValueError, match="flag"):
        tq4.kv4fp8_decode(*args, workspace=ws, test_flags=tq4.TQ4_KV4FP8_TEST_WITHHOLD)
    tq4.kv4fp8_workspace_init(ws)
    _, want = oracle.kv4fp8_decode(q, key, val, sc, tb, ln, heads=H * G, kv_heads=H,
                                   block_size=S, max_blocks=pages, num_blocks=P)
    out = tq4.kv4fp8_decode(*args, workspace=ws)
    mx, mr = compare(bits(out), want, 0)
    assert mx <= 2e-2 and mr <= 1e-3, (mx, mr)
    assert tq4.kv4fp8_poll_timeouts(ws, T, H * G, H, S, pages, P) == 0
