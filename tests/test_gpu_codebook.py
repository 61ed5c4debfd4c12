"""GPU parity of the codebook quantiser leaves against the C oracle and the
reference's fixtures (tests/golden/cb_*):

* ICDF (FP16/BF16 -> signed INT4): the reference fixture's packed bytes, bit
  for bit (its inputs keep 1/16 from every rounding boundary, so any
  evaluation within that of the exact sigmoid must agree);
* Lloyd-Max (2/4-bit): codes, packing and FP32 centroids bit for bit, on the
  fixture (every threshold and its neighbours, +-0, +-100) and on 1M random
  values incl. NaN and +-inf; decode of every code at every word position;
* Gaussian-CDF compander: codes equal to the oracle's wherever the compander
  value is not within 1e-5 of an integer (the device's expf may differ from
  libm's by an ulp there), and there by at most one; centroids of the
  device's codes bit for bit;
* at 16M elements, size-independent properties: quantise(centroids) returns
  the same codes, decode(codes) returns the centroids.
"""
import os

import numpy as np
import pytest
import torch

from gpu_helpers import DEV, host

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def dev16(bits, dtype):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(DEV).view(dtype)


@pytest.mark.parametrize("tag,dtype", [("fp16", torch.float16), ("bf16", torch.bfloat16)])
def test_icdf_reference_fixture(tq4, tag, dtype):
    f = load(f"cb_icdf_{tag}")
    out = tq4.icdf_quantize(dev16(f["in_bits"], dtype))
    assert np.array_equal(host(out), f["packed"])
    if tag == "fp16":  # the same leaf through the Lloyd-Max entry, mode 3
        _, codes = tq4.lloydmax_quantize(dev16(f["in_bits"], dtype), bits=4, mode=3)
        assert np.array_equal(host(codes), f["packed"])


@pytest.mark.parametrize("tag,dtype,bf16", [("fp16", torch.float16, 0), ("bf16", torch.bfloat16, 1)])
def test_icdf_every_16bit_input(tq4, oracle, tag, dtype, bf16):
    """Every one of the 65536 input bit patterns (zeros, subnormals, both
    infinities, every NaN) against the C oracle's double evaluation: the
    codes agree bit for bit everywhere, not only on the fixture's inputs."""
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    out = host(tq4.icdf_quantize(dev16(h, dtype)))
    want = oracle.icdf_quantize(h, bf16)
    bad = np.nonzero(out != want)[0]
    assert bad.size == 0, f"{tag}: {bad.size} bytes differ, first pairs at {bad[:8] * 2}"


def test_icdf_specials(tq4, oracle):
    x = np.array([0.0, -0.0, 100.0, -100.0, np.inf, -np.inf, np.nan, 60000.0] * 128, np.float32)
    h = x.astype(np.float16).view(np.uint16)
    out = host(tq4.icdf_quantize(dev16(h, torch.float16)))
    assert np.array_equal(out, oracle.icdf_quantize(h, 0))


@pytest.mark.parametrize("bits", [2, 4])
def test_lloydmax_reference_fixture(tq4, bits):
    f = load(f"cb_lloyd_b{bits}")
    for key in [k[2:] for k in f if k.startswith("x_")]:
        x = torch.from_numpy(f[f"x_{key}"]).to(DEV)
        recon, codes = tq4.lloydmax_quantize(x, bits=bits, mode=0)
        assert np.array_equal(host(codes), f[f"packed_lm_{key}"]), key
        want = f["centroids_lm"][f[f"codes_lm_{key}"]]
        assert np.array_equal(host(recon).view(np.uint32), want.view(np.uint32)), key


@pytest.mark.parametrize("bits", [2, 4])
def test_lloydmax_random_and_specials(tq4, oracle, bits):
    rng = np.random.default_rng(100 + bits)
    x = np.concatenate([
        rng.standard_normal(1 << 20).astype(np.float32),
        np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 1e-40, -1e-40, 3e38], np.float32),
    ])
    x = x[: x.size // 8 * 8]
    recon, codes = tq4.lloydmax_quantize(torch.from_numpy(x).to(DEV), bits=bits, mode=1)
    w_recon, w_codes = oracle.codebook_quantize(0, bits, x)
    assert np.array_equal(host(codes), w_codes)
    assert np.array_equal(host(recon).view(np.uint32), w_recon.view(np.uint32))


@pytest.mark.parametrize("bits", [2, 4])
def test_gaussian_cdf_compander(tq4, oracle, bits):
    rng = np.random.default_rng(200 + bits)
    f = load(f"cb_lloyd_b{bits}")
    x = np.concatenate([f["x_n256_r8_b1"], rng.standard_normal(1 << 18).astype(np.float32),
                        np.array([np.nan, np.inf, -np.inf, 0.0, -0.0, 50.0, -50.0, 1.0],
                                 np.float32)])
    x = x[: x.size // 8 * 8]
    recon, packed = tq4.lloydmax_quantize(torch.from_numpy(x).to(DEV), bits=bits, mode=2)
    got = host(packed)
    # unpack the device's codes
    q = np.zeros(x.size, np.uint32)
    for i in range(8 // bits):
        q[i::8 // bits] = (got >> (bits * i)) & ((1 << bits) - 1)
    want = oracle.codebook_codes(1, bits, x)
    with np.errstate(all="ignore"):
        xd = x.astype(np.float64)
        v = (1 << bits) / (1.0 + np.exp(-(1.5976 + 0.070565 * xd * xd) * xd))
    near = np.abs(v - np.rint(v)) < 1e-5
    diff = q != want
    assert not np.any(diff & ~near), np.nonzero(diff & ~near)[0][:10]
    assert np.all(np.abs(q.astype(np.int64) - want.astype(np.int64))[diff] <= 1)
    assert diff.sum() <= 4
    c = f["centroids_cdf"]
    assert np.array_equal(host(recon).view(np.uint32), c[q].view(np.uint32))
    # the reference fixture alone (its boundary rows included) agrees exactly
    n_fx = f["x_n256_r8_b1"].size
    assert np.array_equal(q[:n_fx], f["codes_cdf_n256_r8_b1"])


@pytest.mark.parametrize("bits", [2, 4])
def test_decode_every_code_every_position(tq4, oracle, bits):
    n = 2048
    q = (np.arange(n) % (1 << bits)).astype(np.uint32)
    packed = np.zeros(n * bits // 8, np.uint8)
    oracle.lib.tq4o_codebook_pack(q.ctypes.data, n, bits, packed.ctypes.data)
    for mode in (4, 5):
        recon, _ = tq4.lloydmax_quantize(torch.from_numpy(packed).to(DEV), bits=bits, mode=mode)
        want = oracle.codebook_dequantize(0, bits, packed, n)
        assert np.array_equal(host(recon).view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("bits", [2, 4])
def test_large_round_trip_properties(tq4, bits):
    """16M elements: each centroid lies inside its own cell, so quantising the
    reconstruction reproduces the codes; decoding the codes reproduces it."""
    n = 1 << 24
    g = torch.Generator(device=DEV)
    g.manual_seed(7 + bits)
    x = torch.randn(n, device=DEV, generator=g)
    recon, codes = tq4.lloydmax_quantize(x, bits=bits, mode=0)
    recon2, codes2 = tq4.lloydmax_quantize(recon, bits=bits, mode=0)
    dec, _ = tq4.lloydmax_quantize(codes, bits=bits, mode=4)
    torch.cuda.synchronize()
    assert torch.equal(codes, codes2)
    assert torch.equal(recon.view(torch.int32), recon2.view(torch.int32))
    assert torch.equal(dec.view(torch.int32), recon.view(torch.int32))
    # reconstruction error of N(0,1) input: the Lloyd-Max distortion
    mse = torch.mean((x - recon) ** 2).item()
    assert mse < (0.1175 * 1.02 if bits == 2 else 0.00950 * 1.02), mse
