"""The reference AIC decode's page-window ladder, through the mapping a
reference-side caller uses (tq4_paged_decode_partials over a window of the
block table).

The reference validation (tests/npu/validation/
test_turboquant_decode_splitk_aic_validation.cpp:55-150) launches its split
decode over pages [page_begin, page_begin + page_count) of a sequence of
`pages` 128-token pages with seq_len live tokens, for pages {1,4,8,3,5,7} x
K {1,2,4,8} x page_begin {0,1}, and for tail rungs whose last `dead` tokens
of the capacity are not live ({1,1}, {1,15}, {1,127}, {4,1}, {4,15}, {4,129},
{5,273}); geometry: 2 requests, 2 heads, 16 query rows per head, 256 channels.
The window maps onto this library as
    block_tables = table + page_begin (rows of page_count entries),
    max_blocks_per_seq = page_count,
    context_lens = clamp(seq_len - page_begin * 128, 0, page_count * 128),
so Partition(page_count, K, split) is the reference's own partition of the
window. Checked per rung: every split's record against the oracle on the
same window (TQ4_DECODE_PRECISE within the reference rig's budgets, the MFMA
path within its own), the exact neutral record of every split with no live
token, and the split records' combine (the MFMA path's against the FP64
direct softmax over the window's live tokens, the precise mode's against the
oracle's combine of the same BF16-q_rot records).
"""
import math

import numpy as np
import pytest

from gpu_helpers import bf16_out_error, dev, host
from oracle_bindings import FLAG_PRECISE, FLAG_QROT_BF16, f32_to_bf16
from test_gpu_decode import MAX_ABS, MEAN_REL, build_cache
from test_gpu_golden import MFMA, RIG, check_records

pytestmark = pytest.mark.gpu

B, H, G, D, S = 2, 2, 16, 256, 128
HQ = H * G
LADDER = [(1, 0), (4, 0), (8, 0), (3, 0), (5, 0), (7, 0),
          (1, 1), (1, 15), (1, 127), (4, 1), (4, 15), (4, 129), (5, 273)]  # (pages, dead)


@pytest.mark.parametrize("pages,dead", LADDER)
def test_page_window_ladder(tq4, oracle, pages, dead):
    rng = np.random.default_rng(0x1ADD + 31 * pages + dead)
    capacity = pages * S
    live = capacity - dead
    P = B * pages + 3
    # every capacity token written (the dead ones hold data that must stay
    # masked), the sequence live up to `live`
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, [capacity] * B, H, D, S, P)
    q = f32_to_bf16(rng.standard_normal((B, HQ, D)).astype(np.float32))
    scale = np.float32(1.0 / math.sqrt(D))
    dk = [dev(x) for x in (kc, vc, sc, signs)]
    worst = [0.0, 0.0, 0.0]
    for begin in ((0, 1) if pages > 1 else (0,)):
        count = pages - begin
        win = np.ascontiguousarray(tables[:, begin:begin + count])
        ctx = np.full(B, min(max(live - begin * S, 0), count * S), np.int32)
        ref64 = oracle.decode_reference_f64(q, kc, vc, sc, win, ctx, signs, None, HQ, H, D, S, P,
                                           scale, isl, 1)
        for K in (1, 2, 4, 8):
            for precise in (True, False):
                # the precise mode's score operand is Pi q rounded to BF16
                # (the reference device's), the MFMA path's FP16 (the oracle
                # keeps FP32 there)
                want = oracle.decode_partials(q, kc, vc, sc, win, ctx, signs, HQ, H, D, S, P, K,
                                              scale, isl, flags=FLAG_QROT_BF16 if precise else 0)
                label = f"pages {pages} dead {dead} begin {begin} K {K}"
                print(f"window ladder: {label} {'precise' if precise else 'mfma'}", flush=True)
                ws = tq4.paged_decode_partials(dev(q), dk[0], dk[1], dk[2], dev(win), dev(ctx),
                                               dk[3], H, S, P, K, scale=float(scale),
                                               inv_sqrt_len=float(isl),
                                               flags=FLAG_PRECISE if precise else 0)
                got = host(ws).astype(np.float64)
                for b in range(B):
                    for h in range(HQ):
                        for k in range(K):
                            wk = want[b, h, k].astype(np.float64)
                            fr = check_records(got[b, h, k][None], wk[None, 0], wk[None, 1],
                                               wk[None, 4:], RIG if precise else MFMA,
                                               f"{label} {'precise' if precise else 'mfma'} b {b} h {h} split {k}")
                            if precise:
                                worst = [max(x, y) for x, y in zip(worst, fr)]
                            pb = k * ((count + K - 1) // K)
                            if pb >= count or pb * S >= ctx[b]:  # the window holds no live token here
                                assert got[b, h, k, 1] == 0 and np.float32(got[b, h, k, 0]) == \
                                    np.float32(-3e38), f"{label}: split {k} not neutral"
                # the splits' combine: the MFMA path against the direct FP64
                # softmax over the window; the precise mode against the
                # oracle's combine of its BF16-q_rot records (BF16 q_rot is
                # coarser than the exact query: it reproduces the reference's
                # operand, not a closer answer)
                out = tq4.splitk_combine(ws, dk[3], B, HQ, D, K, inv_sqrt_len=float(isl))
                ref = oracle.combine(want, signs, None, HQ, D, K, isl, 1)[1] if precise else \
                    ref64.astype(np.float32)
                mx, mr = bf16_out_error(host(out), ref)
                assert mx <= MAX_ABS and mr <= MEAN_REL, (label, precise, mx, mr)
    print(f"window ladder pages {pages} dead {dead}: precise worst m/l/acc fraction "
          f"{worst[0]:.3f} / {worst[1]:.3f} / {worst[2]:.3f}")
