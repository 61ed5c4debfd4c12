"""GPU parity of reshape_and_cache (aligned strips) against the C oracle.

Bit-exact: packed key/value nibbles and FP32 scale bits, plus every unowned
byte of the canary-filled pools left untouched. Cases follow the reference's
writer validation (tests/npu/validation/test_turboquant_{a8,bf16}_validation.cpp)
and BASELINE configs 1-2.
"""
import math

import numpy as np
import pytest
import torch

from gpu_helpers import canary_bytes, canary_floats, dev, host
from oracle_bindings import IN_BF16, IN_INT8, f32_to_bf16

pytestmark = pytest.mark.gpu


def run_pair(tq4, oracle, in_dtype, key, val, slots, H, d, S, P, signs=None, tables=None,
             isl=None):
    """Run the GPU writer and the oracle on canary pools; return both images."""
    isl = np.float32(1.0 / math.sqrt(d)) if isl is None else np.float32(isl)
    nbytes = P * H * S * d // 2
    kc, vc, sc = canary_bytes(nbytes), canary_bytes(nbytes), canary_floats(2 * P * H * S)
    o_kc, o_vc, o_sc = kc.copy(), vc.copy(), sc.copy()
    o_signs = signs if signs is not None else oracle.canonical_signs(d)
    skipped = oracle.reshape_and_cache(in_dtype, key, val, o_kc, o_vc, o_sc, slots, o_signs, H,
                                       d, S, P, isl)
    g_kc, g_vc, g_sc = dev(kc), dev(vc), dev(sc)
    fn = tq4.reshape_and_cache_bf16 if in_dtype == IN_BF16 else tq4.reshape_and_cache_a8
    fn(dev(key), dev(val), g_kc, g_vc, g_sc, dev(slots),
       pi_signs=dev(signs) if signs is not None else None,
       tables=dev(tables) if tables is not None else None, num_blocks=P, block_size=S,
       inv_sqrt_len=float(isl))
    return (host(g_kc), host(g_vc), host(g_sc)), (o_kc, o_vc, o_sc), skipped


def assert_images_equal(got, want):
    g_kc, g_vc, g_sc = got
    o_kc, o_vc, o_sc = want
    assert np.array_equal(g_kc, o_kc), f"key cache: {np.count_nonzero(g_kc != o_kc)} bytes differ"
    assert np.array_equal(g_vc, o_vc), f"value cache: {np.count_nonzero(g_vc != o_vc)} bytes differ"
    assert np.array_equal(g_sc.view(np.uint32), o_sc.view(np.uint32)), (
        f"scales: {np.count_nonzero(g_sc.view(np.uint32) != o_sc.view(np.uint32))} differ")


def test_config1_a8_one_strip(tq4, oracle):
    """int8 uniform [-127,127], 8 heads x 128, slots -> page 0."""
    rng = np.random.default_rng(0x71340001)
    H, d, S, P = 8, 128, 16, 4
    key = rng.integers(-127, 128, (16, H, d), dtype=np.int8)
    val = rng.integers(-127, 128, (16, H, d), dtype=np.int8)
    slots = np.arange(16, dtype=np.int32)
    got, want, skipped = run_pair(tq4, oracle, IN_INT8, key, val, slots, H, d, S, P,
                                  signs=oracle.canonical_signs(d))
    assert skipped == 0
    assert_images_equal(got, want)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_bf16_integer_equals_a8(tq4, oracle, d):
    """BF16 with integer values in [-64,64] must equal the A8 run byte for byte."""
    rng = np.random.default_rng(0x71340002 + d)
    H, S, P, T = 8, 16, 256, 256
    ints = rng.integers(-64, 65, (2, T, H, d), dtype=np.int8)
    slots = (rng.permutation(P)[: T // 16, None] * 16 + np.arange(16)).reshape(-1).astype(np.int32)
    signs = oracle.canonical_signs(d)
    a8, want, _ = run_pair(tq4, oracle, IN_INT8, ints[0], ints[1], slots, H, d, S, P, signs=signs)
    bf, _, _ = run_pair(tq4, oracle, IN_BF16, f32_to_bf16(ints[0].astype(np.float32)),
                        f32_to_bf16(ints[1].astype(np.float32)), slots, H, d, S, P, signs=signs)
    assert_images_equal(a8, want)
    assert_images_equal(bf, a8)


def test_config2_bf16_integer_1024(tq4, oracle):
    """BASELINE config 2 (integer run): 1024 BF16 tokens with integer values
    in [-64, 64] into the 4096-page pool at permuted pages must equal the A8
    writer on the same integers byte for byte, and the oracle."""
    rng = np.random.default_rng(0x71340012)
    H, d, S, P, T = 8, 128, 16, 4096, 1024
    ints = rng.integers(-64, 65, (2, T, H, d), dtype=np.int8)
    pages = rng.permutation(P)[: T // 16]
    slots = (pages[:, None] * 16 + np.arange(16)).reshape(-1).astype(np.int32)
    signs = oracle.canonical_signs(d)
    a8, want, skipped = run_pair(tq4, oracle, IN_INT8, ints[0], ints[1], slots, H, d, S, P,
                                 signs=signs)
    assert skipped == 0
    bf, want_bf, _ = run_pair(tq4, oracle, IN_BF16, f32_to_bf16(ints[0].astype(np.float32)),
                              f32_to_bf16(ints[1].astype(np.float32)), slots, H, d, S, P,
                              signs=signs)
    assert_images_equal(a8, want)
    assert_images_equal(bf, want_bf)
    assert_images_equal(bf, a8)


def test_config2_bf16_normal_1024(tq4, oracle):
    """BASELINE config 2 (N(0,1) run): 1024 tokens, 4096-page pool, permuted pages."""
    rng = np.random.default_rng(0x71340002)
    H, d, S, P, T = 8, 128, 16, 4096, 1024
    key = f32_to_bf16(rng.standard_normal((T, H, d)).astype(np.float32))
    val = f32_to_bf16(rng.standard_normal((T, H, d)).astype(np.float32))
    pages = rng.permutation(P)[: T // 16]
    slots = (pages[:, None] * 16 + np.arange(16)).reshape(-1).astype(np.int32)
    got, want, skipped = run_pair(tq4, oracle, IN_BF16, key, val, slots, H, d, S, P,
                                  signs=oracle.canonical_signs(d))
    assert skipped == 0
    assert_images_equal(got, want)


@pytest.mark.parametrize("d", [64, 128, 256])
def test_wide_range_rows(tq4, oracle, d):
    """Rows scaled by 2^k, k in [-40, 100] per (token, head, plane): the
    quantiser's exponent runs from the prefill floor (e = 0) to e ~ 110, and
    rows of one strip differ by up to 2^140; bit-exact against the oracle."""
    rng = np.random.default_rng(0x7134000D + d)
    H, S, P, T = 4, 16, 128, 256
    k = rng.integers(-40, 101, (2, T, H, 1)).astype(np.float64)
    x = rng.standard_normal((2, T, H, d)) * np.exp2(k)
    key, val = (f32_to_bf16(x[i].astype(np.float32)) for i in range(2))
    slots = (rng.permutation(P)[: T // 16, None] * 16 + np.arange(16)).reshape(-1).astype(np.int32)
    got, want, skipped = run_pair(tq4, oracle, IN_BF16, key, val, slots, H, d, S, P,
                                  signs=oracle.canonical_signs(d))
    assert skipped == 0
    assert_images_equal(got, want)


@pytest.mark.parametrize("S", [32, 64])
def test_multi_strip_pages(tq4, oracle, S):
    """block_size > 16: strips land at their strip-in-page, strip-blocked value layout."""
    rng = np.random.default_rng(S)
    H, d, P, T = 4, 128, 64, 192
    key = f32_to_bf16(rng.standard_normal((T, H, d)).astype(np.float32) * 3)
    val = f32_to_bf16(rng.standard_normal((T, H, d)).astype(np.float32) * 3)
    strips = rng.permutation(P * S // 16)[: T // 16]
    slots = (strips[:, None] * 16 + np.arange(16)).reshape(-1).astype(np.int32)
    got, want, _ = run_pair(tq4, oracle, IN_BF16, key, val, slots, H, d, S, P,
                            signs=oracle.canonical_signs(d))
    assert_images_equal(got, want)


def test_tables_only_rotation(tq4, oracle):
    """pi_signs NULL: the signs come from the reference's INT8 tables."""
    rng = np.random.default_rng(7)
    H, d, S, P, T = 4, 256, 16, 10, 64
    key = rng.integers(-128, 128, (T, H, d), dtype=np.int8)
    val = rng.integers(-128, 128, (T, H, d), dtype=np.int8)
    signs = np.where(rng.random(d) < 0.5, -1.0, 1.0).astype(np.float32)
    tables = np.zeros(2 * (d // 32) * 32 * 32, np.int8)
    oracle.lib.tq4o_build_tables_i8(d, signs.ctypes.data, tables.ctypes.data)
    slots = ((2 * np.arange(T // 16) + 1)[:, None] * 16 + np.arange(16)).reshape(-1).astype(np.int32)
    nbytes = P * H * S * d // 2
    o_kc, o_vc, o_sc = canary_bytes(nbytes), canary_bytes(nbytes), canary_floats(2 * P * H * S)
    g = [dev(o_kc.copy()), dev(o_vc.copy()), dev(o_sc.copy())]
    oracle.reshape_and_cache(IN_INT8, key, val, o_kc, o_vc, o_sc, slots, signs, H, d, S, P,
                             np.float32(1 / 16))
    tq4.reshape_and_cache_a8(dev(key), dev(val), *g, dev(slots), pi_signs=None,
                             tables=dev(tables.view(np.int8)), num_blocks=P, block_size=S,
                             inv_sqrt_len=1 / 16)
    assert_images_equal([host(x) for x in g], (o_kc, o_vc, o_sc))


def test_bad_slot_strip_writes_nothing(tq4, oracle):
    """A strip whose slots break the contract is skipped (oracle's bad_slot_strip)."""
    rng = np.random.default_rng(11)
    H, d, S, P, T = 2, 128, 16, 8, 48
    key = rng.integers(-100, 100, (T, H, d), dtype=np.int8)
    val = rng.integers(-100, 100, (T, H, d), dtype=np.int8)
    slots = np.concatenate([np.arange(16) + 16 * 1, np.arange(16) + 16 * 3 + 1,
                            np.arange(16) + 16 * 5]).astype(np.int32)  # middle strip misaligned
    slots[40] = 7  # third strip non-consecutive
    got, want, skipped = run_pair(tq4, oracle, IN_INT8, key, val, slots, H, d, S, P,
                                  signs=oracle.canonical_signs(d))
    assert skipped == 2
    assert_images_equal(got, want)


def test_refusals(tq4):
    """Geometry the launcher refuses: nothing runs, ValueError names the status."""
    z8 = torch.zeros(16 * 2 * 128, dtype=torch.int8, device="cuda")
    k = torch.zeros((17, 2, 128), dtype=torch.int8, device="cuda")
    slots = torch.zeros(17, dtype=torch.int32, device="cuda")
    sc = torch.zeros(64, dtype=torch.float32, device="cuda")
    signs = torch.ones(128, dtype=torch.float32, device="cuda")
    with pytest.raises(ValueError, match="whole number"):
        tq4.reshape_and_cache_a8(k, k, z8, z8, sc, slots, pi_signs=signs, num_blocks=1)
    k2 = torch.zeros((16, 2, 96), dtype=torch.int8, device="cuda")
    with pytest.raises(ValueError, match="head_size"):
        tq4.reshape_and_cache_a8(k2, k2, z8, z8, sc, slots[:16], pi_signs=signs, num_blocks=1)
    k3 = torch.zeros((16, 2, 128), dtype=torch.int8, device="cuda")
    with pytest.raises(ValueError, match="pi_signs nor tables"):
        tq4.reshape_and_cache_a8(k3, k3, z8, z8, sc, slots[:16], num_blocks=1)
