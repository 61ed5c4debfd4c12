"""Calls on different streams with their own buffers run at the same time and
give the bits they give alone (include/tq4.h: calls on different streams
with different buffers are independent).

Each persistent launch sizes its grid to every workgroup slot of the GPU, so
two of them running together leave part of each grid waiting for a free
slot. A combiner that waited on a part that had not started would stall
there; its wait is bounded, so such a fault would show as differing bits and
a nonzero give-up count, never as a hang. Every kernel here is deterministic
(fixed split order), so a concurrent result must equal the serial one bit
for bit.
"""
import math

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, dev, host
from oracle_bindings import f32_to_bf16
from test_gpu_decode import build_cache, check_out
from test_oracle_kv4fp8 import random_case

pytestmark = pytest.mark.gpu


def tq4_case(tq4, oracle, rng, ctx, Hq, H, d, K, label):
    """A fused TQ4 decode with its own cache, workspace and output; the
    first call is checked against the oracle."""
    S = 16
    P = sum((c + S - 1) // S for c in ctx) + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx, H, d, S, P)
    q = f32_to_bf16(rng.standard_normal((len(ctx), Hq, d)).astype(np.float32))
    ctx_a = np.array(ctx, np.int32)
    scale = np.float32(1.0 / math.sqrt(d))
    args = [dev(q), dev(kc), dev(vc), dev(sc), dev(tables), dev(ctx_a), dev(signs)]
    ws = tq4.decode_workspace(len(ctx), Hq, H, d, K)
    out = torch.empty_like(args[0])

    def call():
        tq4.paged_decode(*args, H, S, P, out=out, workspace=ws, num_splits=K,
                         scale=float(scale), inv_sqrt_len=float(isl))

    call()
    first = host(out).copy()
    _, want = oracle.paged_decode(q, kc, vc, sc, tables, ctx_a, signs, None, Hq, H, d, S, P, K,
                                  scale, isl, 1, threads=8)
    check_out(first, want, label)
    return call, out, ws, first


def concurrent(calls, reps=4):
    """Each call twice on its own stream, all streams at once, `reps` times."""
    streams = [torch.cuda.Stream() for _ in calls]
    for _ in range(reps):
        for s, c in zip(streams, calls):
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                c()
                c()
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        yield


def test_two_persistent_decodes_on_two_streams(tq4, oracle):
    """Two ragged batches, each with more (seq, kv head, split) items than
    the GPU's workgroup slots (48 x 8 x 4 and 40 x 8 x 3 against 512)."""
    rng = np.random.default_rng(0xC0C1)
    print("concurrency: two persistent TQ4 decodes", flush=True)
    a_call, a_out, a_ws, a0 = tq4_case(tq4, oracle, rng,
                                       [int(x) for x in rng.integers(500, 4000, 48)], 32, 8,
                                       128, 4, "stream A alone")
    b_call, b_out, b_ws, b0 = tq4_case(tq4, oracle, rng,
                                       [int(x) for x in rng.integers(300, 3000, 40)], 32, 8,
                                       128, 3, "stream B alone")
    for _ in concurrent([a_call, b_call]):
        assert np.array_equal(host(a_out), a0)
        assert np.array_equal(host(b_out), b0)
    assert tq4.decode_poll_timeouts(a_ws, 48, 8) == 0
    assert tq4.decode_poll_timeouts(b_ws, 40, 8) == 0


def test_kv4fp8_and_tq4_decodes_on_two_streams(tq4, oracle):
    """The KV4/FP8 decode over about 2000 workgroups (up to eight parts per
    group, four combiners) beside a persistent TQ4 decode."""
    rng = np.random.default_rng(0xC0C2)
    print("concurrency: KV4/FP8 decode beside a persistent TQ4 decode", flush=True)
    t_call, t_out, t_ws, t0 = tq4_case(tq4, oracle, rng,
                                       [int(x) for x in rng.integers(500, 4000, 48)], 32, 8,
                                       128, 4, "TQ4 alone")
    T, H, G, S = 96, 4, 16, 64
    ctx = [int(c) for c in rng.integers(2000, 8192, T)]
    P = sum((c + S - 1) // S for c in ctx) + 4
    q, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, ctx, key_scale=(0.5, 2.0))
    L = tq4.fused_decode_opt_launch(T, H * G, H, S, tb.shape[1], num_blocks=P)
    ws = tq4.kv4fp8_workspace_init(
        torch.empty(tq4.kv4fp8_workspace_bytes(L), dtype=torch.uint8, device=DEV))
    args = (dev(q), dev(key), dev(val), dev(sc), dev(tb), dev(ln), H, S, P)
    k_out = tq4.kv4fp8_decode(*args, workspace=ws)
    k0 = host(k_out).copy()

    def k_call():
        tq4.kv4fp8_decode(*args, workspace=ws, out=k_out)

    for _ in concurrent([k_call, t_call]):
        assert np.array_equal(host(k_out), k0)
        assert np.array_equal(host(t_out), t0)
    assert tq4.decode_poll_timeouts(t_ws, 48, 8) == 0
    assert not torch.any(ws)  # the KV4 tickets and records are zero again
