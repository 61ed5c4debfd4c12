"""GPU parity of the vllm-ascend RMS + threshold codec writer
(tq4_rms_reshape_and_cache) and its decode (tq4_rms_dequantize) against the
C oracle (oracle/tq4_oracle.c, tq4o_rms_*), bit for bit: packed bytes, FP32
scale bits, the zero padding of the scale record, and every byte the launch
does not own left at its canary. Inputs: N(0,1) rows at several magnitudes
(down to where the sum of squares is subnormal), all-zero rows, FP16 and
BF16, head sizes 64/128/256 (the reference bench's H = 4, d = 256 included),
pad and out-of-pool slots, and the block_dim * tokens_per_core coverage.
"""
import math

import numpy as np
import pytest
import torch

from gpu_helpers import canary_bytes, canary_floats, dev, host
from oracle_bindings import f32_to_bf16

pytestmark = pytest.mark.gpu


def to_elem(x, bf16):
    if bf16:
        return f32_to_bf16(x.astype(np.float32))
    return x.astype(np.float16).view(np.uint16)


def run_case(tq4, oracle, T, H, d, S, P, bf16, seed, block_dim=0, tpc=0):
    rng = np.random.default_rng(seed)
    mags = rng.choice([1e-18, 1e-3, 1.0, 30.0, 1e4 if bf16 else 100.0], size=(T, H, 1))
    key = to_elem(rng.standard_normal((T, H, d)) * mags, bf16)
    val = to_elem(rng.standard_normal((T, H, d)) * mags[::-1], bf16)
    key[0] = 0  # an all-zero token: scale 1e-20, every level 7
    slots = rng.permutation(P * S)[:T].astype(np.int32)
    slots[1] = -1
    if T > 3:
        slots[3] = P * S + 5  # past the pool
    ssf = tq4.rms_scale_slot_floats(H)
    nb = P * S * H * d // 2
    kc, vc, sc = canary_bytes(nb), canary_bytes(nb), canary_floats(P * S * ssf)
    o = [kc.copy(), vc.copy(), sc.copy()]
    isl = np.float32(1 / math.sqrt(d))
    signs = np.where(rng.random(d) < 0.5, -1.0, 1.0).astype(np.float32)
    limit = min(T, block_dim * tpc) if block_dim else T
    oracle.rms_reshape_and_cache(1 if bf16 else 0, key, val, o[0], o[1], o[2], slots, signs, H,
                                 d, S, P, limit, isl)
    g = [dev(kc), dev(vc), dev(sc)]
    dt = torch.bfloat16 if bf16 else torch.float16
    kt = torch.from_numpy(key.view(np.int16)).cuda().view(dt)
    vt = torch.from_numpy(val.view(np.int16)).cuda().view(dt)
    print(f"rms writer T={T} H={H} d={d} bf16={bf16}", flush=True)
    tq4.rms_reshape_and_cache(kt, vt, *g, dev(slots), dev(signs), num_blocks=P, block_size=S,
                              inv_sqrt_len=float(isl), block_dim=block_dim, tokens_per_core=tpc)
    got = [host(x) for x in g]
    for a, b, name in zip(got, o, ("key", "value", "scale")):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (
            name, np.count_nonzero(a.view(np.uint8) != b.view(np.uint8)))
    return got


@pytest.mark.parametrize("H,d", [(8, 128), (4, 256), (2, 64), (3, 128)])
@pytest.mark.parametrize("bf16", [True, False])
def test_writer_bit_exact(tq4, oracle, H, d, bf16):
    run_case(tq4, oracle, 300, H, d, 16, 64, bf16, seed=H * 1000 + d + bf16)


def test_writer_coverage_of_the_reference_grid(tq4, oracle):
    """block_dim * tokens_per_core < num_tokens: only those tokens are written."""
    run_case(tq4, oracle, 100, 4, 256, 16, 16, True, seed=77, block_dim=7, tpc=9)


def test_writer_configs1_shape(tq4, oracle):
    """1024 BF16 tokens x 8 KV heads x 128 into a 4096-page pool (configs[1]'s
    shape), 2M codes, bit for bit."""
    run_case(tq4, oracle, 1024, 8, 128, 16, 4096, True, seed=0x71340002)


@pytest.mark.parametrize("n", [2, 6, 4096 * 2 + 6])
def test_dequantize_matches_oracle(tq4, oracle, n):
    rng = np.random.default_rng(n)
    packed = rng.integers(-128, 128, n // 2, dtype=np.int8)
    want = oracle.rms_dequantize(packed)
    got = host(tq4.rms_dequantize(dev(packed)))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_written_rows_decode_to_their_centroids(tq4, oracle):
    """Writer then decode on the GPU: re-quantising the decoded centroids
    (times the row's scale) reproduces the row's levels."""
    got = run_case(tq4, oracle, 64, 4, 128, 16, 8, True, seed=3)
    rows = got[0].reshape(-1, 64)
    dec = host(tq4.rms_dequantize(dev(rows.reshape(-1)))).reshape(-1, 128)
    lv = (rows.view(np.uint8) ^ 0x80)
    want = np.stack([lv & 15, lv >> 4], axis=-1).reshape(-1, 128)
    cents = np.array([oracle.lib.tq4o_rms_centroid(q) for q in range(16)], np.float32)
    assert np.array_equal(dec, cents[want])


@pytest.mark.parametrize("d", [64, 256])
def test_scale_closed_form_in_any_summation_order(tq4, oracle, d):
    """The reference sums the squares with AscendC ReduceSum, in an order this
    writer does not restate; for general data the scale's last bits depend on
    it, so its parity with the reference is unpinned there. Here every sum is
    exact in any order, which pins the scale bits independently of it: rows
    a*e_j and a*e_j + b*e_k (one- and two-hot, BF16), inv_sqrt_len = 1/8.
    Pi x = s . H (s . x) / 8 then has entries +-a/8 (or +-(a +- b)/8), whose
    squares and every partial sum of them are exact in FP32, and d is a
    perfect square, so sqrt is exact too: scale = sqrt(sum y^2) / 8 + 1e-20
    with a single rounding, for both planes, on the GPU and in the oracle."""
    rng = np.random.default_rng(0x5C + d)
    H, S, P = 2, 16, 4
    T = 24
    key = np.zeros((T, H, d), np.float32)
    val = np.zeros((T, H, d), np.float32)
    for t in range(T):
        for h in range(H):
            for x in (key, val):
                a = float(rng.choice([1.0, 1.5, 3.0, 0.25, 96.0, 2.0 ** -10]))
                j = rng.integers(d)
                x[t, h, j] = a * rng.choice([-1, 1])
                if t % 2:  # two-hot
                    k = (j + 1 + rng.integers(d - 1)) % d
                    x[t, h, k] = float(rng.choice([0.5, 2.0, 5.0])) * a * rng.choice([-1, 1])
    kb, vb = f32_to_bf16(key), f32_to_bf16(val)
    signs = np.where(rng.random(d) < 0.5, -1.0, 1.0).astype(np.float32)
    isl = np.float32(0.125)
    slots = rng.permutation(P * S)[:T].astype(np.int32)
    ssf = tq4.rms_scale_slot_floats(H)
    nb = P * S * H * d // 2
    kc, vc, sc = canary_bytes(nb), canary_bytes(nb), canary_floats(P * S * ssf)
    o = [kc.copy(), vc.copy(), sc.copy()]
    oracle.rms_reshape_and_cache(1, kb, vb, o[0], o[1], o[2], slots, signs, H, d, S, P, T, isl)
    g = [dev(kc), dev(vc), dev(sc)]
    kt = torch.from_numpy(kb.view(np.int16)).cuda().view(torch.bfloat16)
    vt = torch.from_numpy(vb.view(np.int16)).cuda().view(torch.bfloat16)
    tq4.rms_reshape_and_cache(kt, vt, *g, dev(slots), dev(signs), num_blocks=P, block_size=S,
                              inv_sqrt_len=float(isl))
    got = [host(x) for x in g]
    for a, b, name in zip(got, o, ("key", "value", "scale")):
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), name
    hd = hadamard(d)
    for t in range(T):
        rec = got[2][slots[t] * ssf: slots[t] * ssf + 2 * H]
        for plane in range(2 * H):
            x = (kb if plane < H else vb)[t, plane % H].astype(np.uint32) << 16
            x = x.view(np.float32).astype(np.float64)
            y = signs * (hd @ (signs * x)) * 0.125
            ss = float(np.sum(y * y))
            assert ss == float(np.float32(ss)), "the sum of squares is exact in FP32"
            want = np.float32(np.float32(np.sqrt(ss)) * np.float32(0.125)) + np.float32(1e-20)
            assert rec[plane].view(np.uint32) == np.float32(want).view(np.uint32), (t, plane)


def hadamard(n):
    h = np.array([[1.0]])
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h
