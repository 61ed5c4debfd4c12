"""The codebook quantiser leaves of the C oracle (no GPU), pinned three ways:

* the reference's own fixtures and oracles (tests/golden/cb_*, written by
  tests/golden/gen_golden.py through oracle/_ref): the ICDF fixture's packed
  bytes (tests/cpu/icdf_fixture.hpp), lloyd::code / centroid / pack
  (tests/common/lloydmax_oracle.hpp) on lloyd::fixture inputs incl. every
  threshold's neighbours, +-0 and +-100;
* closed forms computed here independently with scipy: a Lloyd-Max centroid
  is the N(0,1) conditional mean of its cell, a threshold the midpoint of its
  centroids, a Gaussian-CDF centroid the normal quantile (i + 1/2) / 2^b, and
  the ICDF code is RNE(14 sigmoid(x) - 7);
* planted mistakes (a negated input, an off-by-one threshold count, ties to
  the lower bin) must fail against the fixtures.
"""
import os

import numpy as np
import pytest
from scipy.stats import norm

from oracle_bindings import f32_to_bf16

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
LM, CDF = 0, 1


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("tag,bf16", [("fp16", 0), ("bf16", 1)])
def test_icdf_matches_reference_fixture(oracle, tag, bf16):
    f = load(f"cb_icdf_{tag}")
    got = oracle.icdf_quantize(f["in_bits"], bf16)
    assert np.array_equal(got, f["packed"])


def _icdf_numpy(x):
    y = 14.0 / (1.0 + np.exp(-x.astype(np.float64))) - 7.0
    return np.clip(np.rint(y), -8, 7).astype(np.int64)  # np.rint is RNE


@pytest.mark.parametrize("tag,bf16", [("fp16", 0), ("bf16", 1)])
def test_icdf_closed_form_and_planted_errors(oracle, tag, bf16):
    f = load(f"cb_icdf_{tag}")
    bits = f["in_bits"]
    if bf16:
        x = (bits.astype(np.uint32) << 16).view(np.float32)
    else:
        x = bits.view(np.float16).astype(np.float32)
    q = _icdf_numpy(x)
    packed = ((q[1::2] & 0xF) << 4 | (q[0::2] & 0xF)).astype(np.uint8)
    assert np.array_equal(packed, f["packed"])
    # a negated input or swapped nibble order must not pass the fixture
    qn = _icdf_numpy(-x)
    assert not np.array_equal(((qn[1::2] & 0xF) << 4 | (qn[0::2] & 0xF)).astype(np.uint8),
                              f["packed"])
    assert not np.array_equal(((q[0::2] & 0xF) << 4 | (q[1::2] & 0xF)).astype(np.uint8),
                              f["packed"])


def test_icdf_special_values(oracle):
    lib = oracle.lib
    assert lib.tq4o_icdf_code(0.0) == 0 and lib.tq4o_icdf_code(-0.0) == 0
    assert lib.tq4o_icdf_code(100.0) == 7 and lib.tq4o_icdf_code(-100.0) == -7
    assert lib.tq4o_icdf_code(float("inf")) == 7 and lib.tq4o_icdf_code(float("-inf")) == -7
    assert lib.tq4o_icdf_code(float("nan")) == 0
    # y(x) = k + 1/2 exactly: ties to even
    for k in range(-7, 7):
        p = (k + 0.5 + 7.0) / 14.0
        x = np.log(p / (1 - p))
        assert lib.tq4o_icdf_code(float(x)) in (k, k + 1)


@pytest.mark.parametrize("bits", [2, 4])
def test_lloyd_tables_match_reference(oracle, bits):
    f = load(f"cb_lloyd_b{bits}")
    n = 1 << bits
    for book, key in ((LM, "centroids_lm"), (CDF, "centroids_cdf")):
        mine = np.array([oracle.lib.tq4o_codebook_centroid(book, bits, i) for i in range(n)],
                        np.float32)
        assert np.array_equal(mine.view(np.uint32), f[key].view(np.uint32))
    th = np.array([oracle.lib.tq4o_lloydmax_threshold(bits, i) for i in range(n - 1)], np.float32)
    assert np.array_equal(th.view(np.uint32), f["thresholds_lm"].view(np.uint32))


@pytest.mark.parametrize("bits", [2, 4])
def test_lloyd_tables_closed_form(bits):
    f = load(f"cb_lloyd_b{bits}")
    c = f["centroids_lm"].astype(np.float64)
    t = f["thresholds_lm"].astype(np.float64)
    edges = np.concatenate([[-np.inf], t, [np.inf]])
    # conditional mean of N(0,1) over each cell: (phi(a) - phi(b)) / (Phi(b) - Phi(a))
    mean = (norm.pdf(edges[:-1]) - norm.pdf(edges[1:])) / (norm.cdf(edges[1:]) - norm.cdf(edges[:-1]))
    assert np.max(np.abs(c - mean)) < (2e-5 if bits == 2 else 5e-7)
    assert np.max(np.abs(t - (c[:-1] + c[1:]) / 2)) < 2e-7
    q = norm.ppf((np.arange(1 << bits) + 0.5) / (1 << bits))
    assert np.max(np.abs(f["centroids_cdf"].astype(np.float64) - q)) < 1e-7
    assert np.allclose(c, -c[::-1]) and np.allclose(t, -t[::-1])


@pytest.mark.parametrize("bits", [2, 4])
def test_lloyd_codes_and_packing_match_reference(oracle, bits):
    f = load(f"cb_lloyd_b{bits}")
    keys = [k[2:] for k in f if k.startswith("x_")]
    assert len(keys) == 3
    for key in keys:
        x = f[f"x_{key}"]
        for book, tag in ((LM, "lm"), (CDF, "cdf")):
            codes = oracle.codebook_codes(book, bits, x)
            assert np.array_equal(codes, f[f"codes_{tag}_{key}"]), (tag, key)
            recon, packed = oracle.codebook_quantize(book, bits, x)
            assert np.array_equal(packed, f[f"packed_{tag}_{key}"]), (tag, key)
            want = f[f"centroids_{tag}"][codes]
            assert np.array_equal(recon.view(np.uint32), want.view(np.uint32))
            back = oracle.codebook_dequantize(book, bits, packed, x.size)
            assert np.array_equal(back.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [2, 4])
def test_lloyd_planted_errors_fail(oracle, bits):
    """Ties to the lower bin, or a count off by one, disagree with the fixture
    (its boundary rows hold every threshold and both neighbours)."""
    f = load(f"cb_lloyd_b{bits}")
    x = f["x_n128_r1_b1"].astype(np.float32)
    t = f["thresholds_lm"]
    want = f["codes_lm_n128_r1_b1"]
    assert np.array_equal((x[:, None] >= t[None, :]).sum(1), want)
    assert not np.array_equal((x[:, None] > t[None, :]).sum(1), want)
    assert not np.array_equal(np.minimum((x[:, None] >= t[None, :]).sum(1) + (x > 2.0), 15), want)


@pytest.mark.parametrize("bits", [2, 4])
def test_lloyd_nearest_centroid(oracle, bits):
    """The Lloyd-Max code is the nearest centroid (to FP32 threshold rounding)."""
    rng = np.random.default_rng(bits)
    x = np.concatenate([rng.standard_normal(20000), rng.uniform(-4, 4, 5000)]).astype(np.float32)
    f = load(f"cb_lloyd_b{bits}")
    c = f["centroids_lm"].astype(np.float64)
    codes = oracle.codebook_codes(LM, bits, x)
    d_code = np.abs(x.astype(np.float64) - c[codes])
    d_best = np.abs(x.astype(np.float64)[:, None] - c[None, :]).min(1)
    assert np.all(d_code <= d_best + 3e-7)


def test_codes_live_reference(oracle, ref):
    """Against the compiled reference directly, on values the fixtures do not
    hold: NaN, +-inf, subnormals, and a dense sweep."""
    xs = np.concatenate([
        np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -1e-40, 1e30, -1e30], np.float32),
        np.linspace(-6, 6, 4001, dtype=np.float32),
    ])
    for bits in (2, 4):
        for book in (LM, CDF):
            mine = oracle.codebook_codes(book, bits, xs)
            theirs = np.array([ref.lib.ref_lloyd_code(bits, float(v), book) for v in xs], np.uint32)
            assert np.array_equal(mine, theirs), (bits, book)


def test_bf16_helper_roundtrip():
    x = np.array([1.0, -2.5, 3.140625], np.float32)
    assert np.array_equal((f32_to_bf16(x).astype(np.uint32) << 16).view(np.float32), x)
