"""The RMS + threshold codec oracle (vllm-ascend TurboQuantCodec<4>,
kernels/ops/turboquant/baseline/common/turboquant_codec_950.h) pinned on the
CPU. The reference holds no fixture for this codec, so it is pinned by what
the mathematics fixes:

* ApplyPi equals the KV4/FP8 oracle's ApplyPi bit for bit (that one is
  pinned to the reference's own fixture: its raw query rotates to the
  fixture's pre-rotated query exactly), and equals diag(s) H diag(s)/sqrt(n)
  in FP64 to rounding;
* the scale equals sqrt(sum y^2)/sqrt(n) + 1e-20 in FP64 to a few ulp (the
  FP32 summation order is this library's), and a zero vector gives 1e-20;
* the thresholds and centroids are the Lloyd-Max 4-bit codebook pinned by the
  reference's fixture (tests/golden/cb_lloyd_b4.npz), bit for bit, and each
  centroid lies inside its own cell;
* levels match a brute-force strict count at every threshold, its float
  neighbours, +-0, +-inf and NaN;
* a numpy FP32 restatement in the same operation order reproduces the C
  oracle bit for bit, and each plausible slip planted in it -- the second
  sign multiply dropped, >= instead of >, the nibbles swapped, the 128 bias
  dropped, no epsilon -- makes it disagree on the same data.
"""
import numpy as np
import pytest

T = np.array([-2.4008033987632817, -1.8435318062766393, -1.4371387916845330,
              -1.0992858269170722, -0.7995497875097155, -0.5224037090113789,
              -0.2582216646707196, 0.0, 0.2582216646707196, 0.5224037090113789,
              0.7995497875097155, 1.0992858269170722, 1.4371387916845330,
              1.8435318062766393, 2.4008033987632817], np.float32)


def hadamard(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


@pytest.mark.parametrize("n", [64, 128, 256])
def test_apply_pi_equals_pinned_kv4_apply_pi(oracle, n):
    rng = np.random.default_rng(n)
    signs = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    isl = np.float32(1 / np.sqrt(n))
    for _ in range(20):
        x = (rng.standard_normal(n) * rng.choice([1e-3, 1.0, 300.0])).astype(np.float32)
        got = oracle.rms_apply_pi(x, signs, isl)
        kv4 = x.copy()
        oracle.lib.tq4o_kv4fp8_apply_pi(kv4.ctypes.data, signs.ctypes.data, isl, n)
        assert np.array_equal(got.view(np.uint32), kv4.view(np.uint32))
        dense = np.diag(signs.astype(np.float64)) @ hadamard(n) @ np.diag(signs.astype(np.float64))
        want = dense @ x.astype(np.float64) / np.sqrt(n)
        assert np.abs(got - want).max() <= 1e-5 * np.abs(x).max() * np.sqrt(n)


@pytest.mark.parametrize("n", [64, 128, 256])
def test_scale_closed_form_and_zero_row(oracle, n):
    rng = np.random.default_rng(100 + n)
    isl = np.float32(1 / np.sqrt(n))
    for mag in (1e-30, 1e-3, 1.0, 1e4, 1e18):
        y = (rng.standard_normal(n) * mag).astype(np.float32)
        s = oracle.lib.tq4o_rms_scale(y.ctypes.data, n, isl)
        want = np.sqrt(np.sum(y.astype(np.float64) ** 2)) * float(isl) + 1e-20
        assert abs(s - want) <= 4 * np.spacing(np.float32(want)), (mag, s, want)
    z = np.zeros(n, np.float32)
    assert np.float32(oracle.lib.tq4o_rms_scale(z.ctypes.data, n, isl)) == np.float32(1e-20)


@pytest.mark.parametrize("n", [64, 256])
def test_scale_exact_sums_pin_the_bits_in_any_order(oracle, n):
    """Rows whose rotation has entries +-a/8 or +-(a +- b)/8 (one- and two-hot
    x, inv_sqrt_len = 1/8): every square and partial sum is exact in FP32 and
    sqrt is exact (n a perfect square), so the scale's bits are fixed whatever
    the summation order -- the reference's ReduceSum order included."""
    rng = np.random.default_rng(7 + n)
    h = hadamard(n)
    for trial in range(200):
        x = np.zeros(n)
        a = rng.choice([1.0, 1.5, 3.0, 0.25, 96.0, 2.0 ** -10])
        j = rng.integers(n)
        x[j] = a
        if trial % 2:
            x[(j + 1 + rng.integers(n - 1)) % n] = rng.choice([0.5, 2.0, 5.0]) * a * rng.choice([-1, 1])
        s = np.where(rng.random(n) < 0.5, -1.0, 1.0)
        y = (s * (h @ (s * x)) * 0.125).astype(np.float32)
        ss = float(np.sum(y.astype(np.float64) ** 2))
        assert ss == float(np.float32(ss))
        got = np.float32(oracle.lib.tq4o_rms_scale(y.ctypes.data, n, np.float32(0.125)))
        want = np.float32(np.float32(np.sqrt(ss)) * np.float32(0.125)) + np.float32(1e-20)
        assert got == want, (trial, got, want)
        # and a shuffled order of the same squares gives the same sum
        assert float(np.sum(rng.permutation(y.astype(np.float64) ** 2))) == ss


def test_tables_are_the_pinned_lloydmax_codebook(oracle):
    from test_oracle_codebook import load
    f = load("cb_lloyd_b4")  # the reference's lloyd:: fixture
    for i in range(15):
        a = np.float32(oracle.lib.tq4o_rms_threshold(i))
        assert a == T[i]
        assert a.view(np.uint32) == f["thresholds_lm"][i].view(np.uint32)
    for q in range(16):
        c = np.float32(oracle.lib.tq4o_rms_centroid(q))
        assert c.view(np.uint32) == f["centroids_lm"][q].view(np.uint32)
        # the centroid lies inside its own cell: re-quantising it gives q
        assert oracle.lib.tq4o_rms_level(float(c), 1.0) == q


def test_levels_brute_force_at_the_boundaries(oracle):
    vals = [0.0, -0.0, np.inf, -np.inf, 1e-30, -1e-30]
    for t in T:
        vals += [float(t), float(np.nextafter(t, np.float32(9))), float(np.nextafter(t, np.float32(-9)))]
    vals += list(np.random.default_rng(7).standard_normal(2000) * 2)
    for v in vals:
        z = np.float32(v)
        want = int(np.sum(T < z))
        assert oracle.lib.tq4o_rms_level(float(z), 1.0) == want, v
    assert oracle.lib.tq4o_rms_level(float("nan"), 1.0) == 0


def numpy_row(x, signs, isl, slip=None):
    """FP32 restatement of one vector in the oracle's operation order."""
    f = np.float32
    y = (x * signs).astype(f)
    n = y.size
    s = 1
    while s < n:
        y2 = y.copy()
        for i in range(n):
            if not i & s:
                y2[i], y2[i | s] = f(y[i] + y[i | s]), f(y[i] - y[i | s])
        y = y2
        s <<= 1
    y = (y * isl).astype(f)
    if slip != "one_sign":
        y = (y * signs).astype(f)
    per = n // 16
    part = []
    for lane in range(16):
        acc = f(y[lane * per] * y[lane * per])
        for j in range(1, per):
            acc = f(acc + f(y[lane * per + j] * y[lane * per + j]))
        part.append(acc)
    m = 1
    while m < 16:
        part = [f(part[i] + part[i ^ m]) for i in range(16)]
        m <<= 1
    scale = f(f(np.sqrt(part[0]) * isl) + (f(0) if slip == "no_eps" else f(1e-20)))
    with np.errstate(divide="ignore", invalid="ignore"):  # the no-eps slip on a zero row
        r = f(f(1) / scale)
        z = (y * r).astype(f)
    if slip == "ge":
        lv = np.array([np.sum(T <= v) for v in z], np.uint32)
    else:
        lv = np.array([np.sum(T < v) for v in z], np.uint32)
    lo, hi = lv[0::2], lv[1::2]
    if slip == "swap":
        lo, hi = hi, lo
    byte = lo | (hi << 4)
    if slip != "no_bias":
        byte = byte ^ 0x80
    return byte.astype(np.uint8).view(np.int8), scale


@pytest.mark.parametrize("slip", [None, "one_sign", "ge", "swap", "no_bias", "no_eps"])
def test_numpy_restatement_and_planted_slips(oracle, slip):
    rng = np.random.default_rng(11)
    n = 64
    signs = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    isl = np.float32(1 / np.sqrt(n))
    rows = [rng.standard_normal(n).astype(np.float32) for _ in range(6)]
    rows.append(np.zeros(n, np.float32))
    # a row whose rotated, scaled values land exactly on thresholds: the
    # inverse rotation of the thresholds times a power of two
    tgt = np.tile(np.concatenate([T, [T[3]]]), n // 16).astype(np.float32)
    rows.append(oracle.rms_apply_pi(tgt, signs, isl))
    same = True
    for x in rows:
        _, pk, sc = oracle.rms_quantize_row(x, signs, isl)
        npk, nsc = numpy_row(x, signs, isl, slip)
        same &= bool(np.array_equal(npk, pk)) and np.float32(sc).view(np.uint32) == nsc.view(np.uint32)
    assert same == (slip is None), slip


def test_writer_layout_slots_and_padding(oracle):
    """Rows land at slot*H*(d/2) + h*(d/2); the scale record holds K scales,
    then V scales, then zeros to a multiple of 8; tokens past token_limit
    and slots outside the pool write nothing; dequantize gives centroids."""
    from oracle_bindings import f32_to_bf16
    rng = np.random.default_rng(5)
    T_, H, d, S, P = 6, 3, 128, 16, 4
    key = f32_to_bf16(rng.standard_normal((T_, H, d)).astype(np.float32))
    val = f32_to_bf16(rng.standard_normal((T_, H, d)).astype(np.float32))
    slots = np.array([5, -1, 63, 64, 0, 17], np.int32)
    nb = P * S * H * d // 2
    ssf = oracle.lib.tq4o_rms_scale_slot_floats(H)
    assert ssf == 8
    kc = np.full(nb, 0x55, np.int8)
    vc = np.full(nb, 0x55, np.int8)
    sc = np.full(P * S * ssf, np.nan, np.float32)
    signs = oracle.canonical_signs(d)
    isl = np.float32(1 / np.sqrt(d))
    n = oracle.rms_reshape_and_cache(1, key, val, kc, vc, sc, slots, signs, H, d, S, P, 5, isl)
    assert n == 3 * 2 * H  # tokens 0, 2, 4 (1: pad, 3: outside the pool, 5: past the limit)
    from oracle_bindings import bf16_to_f32
    for t in (0, 2, 4):
        s = slots[t]
        for h in range(H):
            for plane, src, cache in ((0, key, kc), (1, val, vc)):
                _, pk, scale = oracle.rms_quantize_row(bf16_to_f32(src[t, h]), signs, isl)
                row = cache[(s * H + h) * (d // 2):(s * H + h + 1) * (d // 2)]
                assert np.array_equal(row, pk)
                assert sc[s * ssf + plane * H + h] == scale
        assert np.all(sc[s * ssf + 2 * H:(s + 1) * ssf] == 0)
    untouched = [s for s in range(P * S) if s not in (5, 63, 0)]
    assert np.all(np.isnan(sc.reshape(P * S, ssf)[untouched]))
    assert np.all(kc.reshape(P * S, -1)[untouched] == 0x55)
    rec = oracle.rms_dequantize(kc[5 * H * (d // 2):5 * H * (d // 2) + d // 2])
    lv, _, _ = oracle.rms_quantize_row(bf16_to_f32(key[0, 0]), signs, isl)
    assert np.array_equal(rec, np.array([oracle.lib.tq4o_rms_centroid(int(q)) for q in lv],
                                        np.float32))
