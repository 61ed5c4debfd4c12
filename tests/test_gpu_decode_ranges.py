"""Decode numerics at the edges of the kernel's range logic, against the C
oracle (FP32, the reference's score / recurrence order,
tests/common/single_token_decode_oracle.hpp:257-310).

The kernel runs its softmax in the exp2 domain with a lazy maximum: a q
row's running maximum moves only when a score exceeds it by 2^8 (log2
units). The P.V MFMA takes P times the value scale in fp16, normalised per
row by a power of two chosen at each rescale so that the largest product of
that pair lands in [1, 2); a rescale also happens when a product could reach
2^15. These cases drive each branch:

* one dominant token under a large |q| (scores hundreds of nats above the
  rest), placed first, mid-stream and in the partial last strip, so the
  running maximum jumps and every accumulator rescales, and the other
  splits' records carry maxima far below the combined one;
* value scales spread over 2^-20 .. 2^20 from token to token;
* both at once, with the dominant token carrying the smallest value scale,
  so tokens of huge value scale sit under probabilities that underflow.

Budgets: the north_star's max-abs 2e-2 and mean-rel 1e-3 (BF16 output
against the FP32 oracle rounded to BF16). Where the value scales make the
output itself large or tiny, the max-abs budget is taken relative to the
largest output magnitude (2e-2 * max|out|); the mean-rel budget is unchanged.
"""
import math

import numpy as np
import pytest

from gpu_helpers import dev, host
from oracle_bindings import IN_BF16, f32_to_bf16, bf16_to_f32
from test_gpu_decode import check_out

pytestmark = pytest.mark.gpu

HQ, H, D, S = 32, 8, 128, 16
G = HQ // H


def cache_from(oracle, rng, k, v, P, exact=False):
    """Quantise given K/V [ctx][H][D] (FP32, rounded to BF16) through the
    oracle writer into a shuffled pool; returns the cache image and table.
    exact: every token through the scatter writer, whose quantiser takes the
    exact row absmax (the prefill writer floors it at 1.0, so values far
    below 1 would all quantise to 0)."""
    ctx = k.shape[0]
    pages = (ctx + S - 1) // S
    table = rng.permutation(P)[:pages].astype(np.int32)[None, :]
    nbytes = P * H * S * D // 2
    kc, vc = np.zeros(nbytes, np.int8), np.zeros(nbytes, np.int8)
    sc = np.zeros(2 * P * H * S, np.float32)
    isl = np.float32(1.0 / math.sqrt(D))
    signs = oracle.canonical_signs(D)
    tok = np.arange(ctx)
    slots = (table[0, tok // S] * S + tok % S).astype(np.int32)
    kb, vb = f32_to_bf16(k.astype(np.float32)), f32_to_bf16(v.astype(np.float32))
    full = 0 if exact else ctx // 16 * 16
    if full:
        assert oracle.reshape_and_cache(IN_BF16, kb[:full], vb[:full], kc, vc, sc, slots[:full],
                                        signs, H, D, S, P, isl) == 0
    if ctx > full:
        oracle.reshape_scatter(kb[full:], vb[full:], kc, vc, sc, slots[full:], signs,
                               np.array([0, ctx - full], np.int32), 1, H, D, S, P, 0, H, isl)
    return kc, vc, sc, table, signs, isl


def run(tq4, oracle, q, kc, vc, sc, table, signs, isl, ctx, P, K, label, relative):
    scale = np.float32(1.0 / math.sqrt(D))
    ctx_a = np.array([ctx], np.int32)
    _, want = oracle.paged_decode(q, kc, vc, sc, table, ctx_a, signs, None, HQ, H, D, S, P, K,
                                  scale, isl, 1, threads=16)
    print(f"range case {label}", flush=True)
    out = tq4.paged_decode(dev(q), dev(kc), dev(vc), dev(sc), dev(table), dev(ctx_a),
                           dev(signs), H, S, P, num_splits=K, scale=float(scale),
                           inv_sqrt_len=float(isl))
    got = host(out)
    assert np.all(np.isfinite(want))
    budget = 2e-2 * max(1.0, float(np.abs(want).max())) if relative else 2e-2
    check_out(got, want, label, max_abs=budget)
    return bf16_to_f32(got), want


def dominant_keys(rng, q, ctx, pos, strength):
    """N(0,1) keys, except token `pos`, whose key for KV head h is
    `strength` times the sum of its group's query rows."""
    k = rng.standard_normal((ctx, H, D)).astype(np.float32)
    qf = bf16_to_f32(q).reshape(H, G, D)
    k[pos] = strength * qf.sum(axis=1)
    return k


@pytest.mark.parametrize("where", ["first", "middle", "tail"])
@pytest.mark.parametrize("qmul", [8.0, 64.0])
def test_dominant_token(tq4, oracle, where, qmul):
    """Scores of one token far above the rest: the output is (nearly) that
    token's value; the running maximum jumps when the stream meets it."""
    rng = np.random.default_rng({"first": 1, "middle": 2, "tail": 3}[where] + int(qmul))
    ctx = 4096 + 9
    P = (ctx + S - 1) // S + 16
    pos = {"first": 0, "middle": 2500, "tail": ctx - 3}[where]
    q = f32_to_bf16((rng.standard_normal((1, HQ, D)) * qmul).astype(np.float32))
    k = dominant_keys(rng, q, ctx, pos, 0.2)
    v = rng.standard_normal((ctx, H, D)).astype(np.float32)
    kc, vc, sc, table, signs, isl = cache_from(oracle, rng, k, v, P)
    for K in (1, 16):
        run(tq4, oracle, q, kc, vc, sc, table, signs, isl, ctx, P, K,
            f"dominant {where} q*{qmul:g} K {K}", relative=False)


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("K", [1, 8])
def test_value_scales_over_many_binades(tq4, oracle, K, exact):
    """Each token's values scaled by 2^e, e uniform in [-20, 20]: the value
    scales (powers of two) span 30 to 40 binades (the prefill writer's floor
    cuts the lower end), so products keep outgrowing the fp16 headroom and
    the rows re-normalise for them."""
    rng = np.random.default_rng(40 + K + 2 * exact)
    ctx = 2048 + 5
    P = (ctx + S - 1) // S + 16
    q = f32_to_bf16(rng.standard_normal((1, HQ, D)).astype(np.float32))
    k = rng.standard_normal((ctx, H, D)).astype(np.float32)
    e = rng.integers(-20, 21, ctx).astype(np.float32)
    v = rng.standard_normal((ctx, H, D)).astype(np.float32) * np.exp2(e)[:, None, None]
    kc, vc, sc, table, signs, isl = cache_from(oracle, rng, k, v, P, exact)
    vs = sc[P * H * S:].reshape(P, H, S)[table[0]].reshape(-1)[: ctx * H]
    spread = np.log2(vs.max() / vs[vs > 0].min())
    assert spread >= (38 if exact else 23), spread  # the stored scales do span the range
    run(tq4, oracle, q, kc, vc, sc, table, signs, isl, ctx, P, K,
        f"value binades K {K}{' exact' if exact else ''}", relative=True)


@pytest.mark.parametrize("K", [1, 4, 16])
def test_dominant_token_with_tiny_value_among_huge(tq4, oracle, K):
    """The dominant token's values are scaled by 2^-20, the rest's by up to
    2^20 (every token quantised with its exact absmax, so the tiny values
    survive): tokens of huge value scale sit under probabilities of about
    e^-90, and the output is the dominant token's tiny value. A row
    normalised by the largest value scale instead of the largest product
    would flush that token's fp16 operand to zero."""
    rng = np.random.default_rng(70 + K)
    ctx = 3000
    P = (ctx + S - 1) // S + 16
    pos = 1777
    q = f32_to_bf16((rng.standard_normal((1, HQ, D)) * 16).astype(np.float32))
    k = dominant_keys(rng, q, ctx, pos, 0.05)
    e = rng.integers(0, 21, ctx).astype(np.float32)
    e[pos] = -20
    v = rng.standard_normal((ctx, H, D)).astype(np.float32) * np.exp2(e)[:, None, None]
    kc, vc, sc, table, signs, isl = cache_from(oracle, rng, k, v, P, exact=True)
    got, want = run(tq4, oracle, q, kc, vc, sc, table, signs, isl, ctx, P, K,
                    f"tiny dominant among huge K {K}", relative=True)
    assert 1e-8 < np.abs(want).max() < 1e-4  # one-hot on the 2^-20 token
