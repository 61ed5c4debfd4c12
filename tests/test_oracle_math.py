"""Closed-form pins of the C oracle that hold at any head size.

The golden vectors pin d = 256 (and d = 128 for the writer); these checks pin
what mathematics fixes, at d in {64, 128, 256}: the rotation is orthogonal up
to d, the butterfly cascade equals the dense matrix exactly on integers, the
quantiser rounds half to even with the +7 clamp, the index maps are
bijections, the uniform combine is an exact sum, and the decode is invariant
under the split count and agrees with an FP64 direct softmax.
"""
import math

import numpy as np
import pytest

from oracle_bindings import IN_BF16, IN_INT8, POLICY_EXACT, POLICY_PREFILL, f32_to_bf16, ptr


@pytest.mark.parametrize("d", [64, 128, 256])
def test_rotation_is_orthogonal_up_to_d(oracle, d):
    """M M^T = d I, from the dense definition (rotate_butterfly_oracle.hpp:84-92)."""
    s = oracle.canonical_signs(d)
    M = np.stack([oracle.rotate_dense(np.eye(d, dtype=np.float32)[i], s) for i in range(d)], axis=1)
    assert np.array_equal(M @ M.T, d * np.eye(d))
    assert set(np.unique(M)) == {-1.0, 1.0}


@pytest.mark.parametrize("d", [64, 128, 256])
def test_butterfly_equals_dense_on_integers(oracle, d):
    """The staged cascade is the dense M exactly (integer data is exact in FP32),
    and egress(ingress(x)) = d x."""
    rng = np.random.default_rng(d)
    s = np.where(rng.random(d) < 0.5, -1.0, 1.0).astype(np.float32)
    for _ in range(8):
        x = rng.integers(-128, 128, d).astype(np.float32)
        y = oracle.rotate_ingress(x, s)
        assert np.array_equal(y.astype(np.float64), oracle.rotate_dense(x, s))
        assert np.array_equal(oracle.rotate_egress(x, s).astype(np.float64),
                              oracle.rotate_dense(x, s, transpose=True))
        assert np.array_equal(oracle.rotate_egress(y, s), d * x)


def test_quantiser_closed_form(oracle):
    """q = min(rint_even(y * 2^(2-e)), 7), scale = 2^(e-2) * isl: ties go to
    even, the clamp is at +7 only, and |y - q 2^(e-2)| <= 2^(e-3) except where
    clamped (turboquant_oracle.hpp:412-448)."""
    d, isl = 128, np.float32(1 / math.sqrt(128))
    # absmax 16 -> e = 4, step 4: ties at odd multiples of 2
    y = np.zeros(d, np.float32)
    y[:8] = [16, 2, 6, -2, -6, 10, -16, 15]
    q, sc = oracle.quantise_row(y, isl, POLICY_PREFILL)
    assert sc == np.float32(4.0) * isl
    assert list(q[:8]) == [4, 0, 2, 0, -2, 2, -4, 4]
    # +8 clamps to +7, -8 is kept
    y2 = np.zeros(d, np.float32)
    y2[0], y2[1] = 31, -31  # e = 4: 31/4 = 7.75 -> 8 -> 7 ; -7.75 -> -8
    q2, _ = oracle.quantise_row(y2, isl, POLICY_PREFILL)
    assert q2[0] == 7 and q2[1] == -8
    # half-step bound on random rows
    rng = np.random.default_rng(3)
    for _ in range(50):
        y = rng.standard_normal(d).astype(np.float32) * rng.uniform(0.5, 500)
        q, sc = oracle.quantise_row(y, isl, POLICY_EXACT)
        step = np.float64(sc) / np.float64(isl)
        err = np.abs(y.astype(np.float64) - q.astype(np.float64) * step)
        clamped = q == 7
        assert np.all(err[~clamped] <= step / 2 + 1e-12)
    # zero row: prefill floors absmax at 1 (e = 0), exact gives scale 1.0
    z = np.zeros(d, np.float32)
    qz, sz = oracle.quantise_row(z, isl, POLICY_PREFILL)
    assert np.all(qz == 0) and sz == np.float32(0.25) * isl
    qz, sz = oracle.quantise_row(z, isl, POLICY_EXACT)
    assert np.all(qz == 0) and sz == 1.0


def test_index_maps_are_bijections(oracle):
    """Every (page, head, token, channel) owns one nibble of each plane and one
    scale slot (turboquant_scatter_oracle.hpp:110-132)."""
    H, S, d, P = 3, 32, 64, 5
    L = oracle.lib
    keys, vals, scs = set(), set(), set()
    for page in range(P):
        for h in range(H):
            for t in range(S):
                for c in range(d):
                    keys.add(L.tq4o_key_nibble(H, S, d, page, h, t, c))
                    vals.add(L.tq4o_value_nibble(H, S, d, page, h, t, c))
                for plane in range(2):
                    scs.add(L.tq4o_scale_index(P, H, S, plane, page, h, t))
    n = P * H * S * d
    assert keys == set(range(n)) and vals == set(range(n)) and scs == set(range(2 * P * H * S))


def test_combine_uniform_closed_form(oracle):
    """Equal m for every split: the combine is an exact sum, acc = (2^K - 1)(c + 1)
    (l2_atomic_oracle.hpp:178-195)."""
    d = 128
    for K in range(1, 9):
        m = np.array([-3e38], np.float32)
        l = np.zeros(1, np.float32)
        acc = np.zeros(d, np.float32)
        for k in range(K):
            t = ((2.0 ** k) * (np.arange(d) + 1)).astype(np.float32)
            oracle.lib.tq4o_combine_step(ptr(m), ptr(l), ptr(acc), -4.0, float(2 ** k), ptr(t), d)
        assert np.array_equal(acc, ((2 ** K - 1) * (np.arange(d) + 1)).astype(np.float32))
        assert l[0] == 2 ** K - 1 and m[0] == -4.0


def make_cache(oracle, rng, ctx_lens, H, d, S, P):
    pages_per = [(c + S - 1) // S for c in ctx_lens]
    perm = rng.permutation(P)
    tables = np.zeros((len(ctx_lens), max(pages_per)), np.int32)
    nb = P * H * S * d // 2
    kc, vc, sc = np.zeros(nb, np.int8), np.zeros(nb, np.int8), np.zeros(2 * P * H * S, np.float32)
    at = 0
    isl = np.float32(1 / math.sqrt(d))
    signs = oracle.canonical_signs(d)
    for b, c in enumerate(ctx_lens):
        tables[b, :pages_per[b]] = perm[at:at + pages_per[b]]
        at += pages_per[b]
        full = (c + 15) // 16 * 16
        tok = np.arange(full)
        slots = (tables[b, tok // S] * S + tok % S).astype(np.int32)
        k = f32_to_bf16(rng.standard_normal((full, H, d)).astype(np.float32))
        v = f32_to_bf16(rng.standard_normal((full, H, d)).astype(np.float32))
        assert oracle.reshape_and_cache(IN_BF16, k, v, kc, vc, sc, slots, signs, H, d, S, P, isl) == 0
    return kc, vc, sc, tables, signs, isl


@pytest.mark.parametrize("d", [64, 128, 256])
def test_decode_split_invariance_and_fp64(oracle, d):
    """The FP32 split-K decode equals itself at any split count to rounding, and
    the FP64 direct softmax to ~1e-5 relative (splitk_decode_fixture.hpp:193-248)."""
    rng = np.random.default_rng(d + 7)
    H, Hq, S, P = 2, 8, 32, 64
    ctx = np.array([300, 33, 512], np.int32)
    kc, vc, sc, tables, signs, isl = make_cache(oracle, rng, list(ctx), H, d, S, P)
    q = f32_to_bf16(rng.standard_normal((3, Hq, d)).astype(np.float32))
    scale = np.float32(1 / math.sqrt(d))
    outs = [oracle.paged_decode(q, kc, vc, sc, tables, ctx, signs, None, Hq, H, d, S, P, K, scale,
                                isl, 1)[1] for K in (1, 2, 5, 16)]
    ref = oracle.decode_reference_f64(q, kc, vc, sc, tables, ctx, signs, None, Hq, H, d, S, P,
                                      scale, isl, 1)
    mag = np.abs(ref).max()
    for o in outs:
        assert np.abs(o - outs[0]).max() <= 2e-6 * mag
        assert np.abs(o - ref).max() <= 2e-5 * mag


def test_decode_empty_splits_are_neutral(oracle):
    rng = np.random.default_rng(1)
    H, Hq, d, S, P = 1, 4, 128, 16, 8
    ctx = np.array([20], np.int32)
    kc, vc, sc, tables, signs, isl = make_cache(oracle, rng, list(ctx), H, d, S, P)
    ws = oracle.decode_partials(q=f32_to_bf16(rng.standard_normal((1, Hq, d)).astype(np.float32)),
                                kc=kc, vc=vc, sc=sc, tables=tables, ctx=ctx, signs=signs,
                                num_heads=Hq, num_kv_heads=H, head_size=d, block_size=S,
                                num_blocks=P, num_splits=5, scale=np.float32(0.1),
                                inv_sqrt_len=isl)
    # 2 pages over 5 splits: splits 2.. own no page
    assert np.all(ws[0, :, 2:, 0] == np.float32(-3e38))
    assert np.all(ws[0, :, 2:, 1:] == 0)
    assert np.all(ws[0, :, :2, 1] > 0)


def test_writer_int8_equals_bf16_integers(oracle):
    """The BF16 path on integer values is byte-identical to the A8 path."""
    rng = np.random.default_rng(2)
    H, d, S, P, T = 4, 128, 16, 8, 64
    ints = rng.integers(-64, 65, (2, T, H, d), dtype=np.int8)
    slots = ((np.arange(T // 16) * 2 + 1)[:, None] * 16 + np.arange(16)).reshape(-1).astype(np.int32)
    s = oracle.canonical_signs(d)
    isl = np.float32(1 / math.sqrt(d))
    imgs = []
    for dt, k, v in ((IN_INT8, ints[0], ints[1]),
                     (IN_BF16, f32_to_bf16(ints[0].astype(np.float32)), f32_to_bf16(ints[1].astype(np.float32)))):
        kc, vc, sc = np.zeros(P * H * S * d // 2, np.int8), np.zeros(P * H * S * d // 2, np.int8), np.zeros(2 * P * H * S, np.float32)
        oracle.reshape_and_cache(dt, k, v, kc, vc, sc, slots, s, H, d, S, P, isl)
        imgs.append((kc, vc, sc.view(np.uint32)))
    for a, b in zip(*imgs):
        assert np.array_equal(a, b)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_rotation_tables_compose_to_M(oracle, d):
    """The INT8 rotation tables (T[s][g][c0][i], turboquant_oracle.hpp:157-195)
    rebuild the dense rotation the way the reference's Cube applies them:
    M[c1*32 + c0][g*32 + i] = T[parity(c1 & g)][g][c0][i] (the outer H_{d/32}
    picks the table's sign); compared column by column with the dense M
    from the butterfly definition. The signs come back out of the tables."""
    rng = np.random.default_rng(d)
    signs = np.where(rng.random(d) < 0.5, -1.0, 1.0).astype(np.float32)
    groups = d // 32
    tables = np.zeros(2 * groups * 32 * 32, np.int8)
    oracle.lib.tq4o_build_tables_i8(d, signs.ctypes.data, tables.ctypes.data)
    T = tables.reshape(2, groups, 32, 32).astype(np.int64)
    M = np.zeros((d, d), np.int64)
    for c1 in range(groups):
        for g in range(groups):
            par = bin(c1 & g).count("1") & 1
            M[c1 * 32:(c1 + 1) * 32, g * 32:(g + 1) * 32] = T[par, g]
    dense = np.stack([oracle.rotate_dense(np.eye(d, dtype=np.float32)[j], signs)
                      for j in range(d)], axis=1)
    assert np.array_equal(dense, M.astype(np.float64))
    back = np.zeros(d, np.float32)
    assert oracle.lib.tq4o_signs_from_tables_i8(d, tables.ctypes.data, back.ctypes.data) == 0
    assert np.array_equal(back, signs)
    tables[5] = -tables[5]  # a corrupted block is detected
    assert oracle.lib.tq4o_signs_from_tables_i8(d, tables.ctypes.data, back.ctypes.data) == -1


@pytest.mark.parametrize("d", [128, 256])
def test_rotation_tables_match_reference(oracle, ref, d):
    """Byte for byte against tq_oracle::build_tables on the canonical signs
    (tests/common/turboquant_oracle.hpp:157-171), where oracle/_ref is built."""
    signs = oracle.canonical_signs(d)
    ours = np.zeros(2 * (d // 32) * 1024, np.int8)
    oracle.lib.tq4o_build_tables_i8(d, signs.ctypes.data, ours.ctypes.data)
    theirs = np.zeros_like(ours)
    ref.lib.ref_tq_build_tables(d, theirs.ctypes.data)
    assert np.array_equal(ours, theirs)
