"""The C oracle of the KV4/FP8 fused decode (oracle/kv4fp8_oracle.c), no GPU.

Pinned against:
* the reference's own fixture (tests/golden/fd_*, written by gen_golden.py from
  tests/common/fused_decode_opt_fixture.hpp through oracle/_ref): FP16 and BF16
  outputs bit for bit on every rung of the reference's NPU validation ladder
  that is stored here, at every split count the ladder uses (its ULP budget
  is 0); the raw-query prologue reproduces the fixture's pre-rotated query
  bit for bit; output stages 1 and 2 against the fixture's expected rows;
* the reference's NzTiledPackedByte on a grid of (slot, kv head, column);
* brute force: the FP8 e4m3 encoder picks the nearest grid value, ties to
  even, over every finite code and the midpoints between them;
* closed forms: a one-tile, two-level case whose answer is a two-term
  expression; an FP64 softmax attention on random caches, which the oracle
  must follow to within the FP8 operand rounding (3-4 % mean relative), and
  which planted mistakes (unsigned nibbles, swapped value planes, swapped
  K/V scale lanes) miss by 40x more;
* the split count changes only the partition, never the answer.
"""
import os

import numpy as np
import pytest

from oracle_bindings import Kv4Geom  # noqa: F401  (struct layout used by the binding)

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GAIN = np.float32(2.9832882881)
FIXTURES = ["fd_n79_b1_h1_g16_p64", "fd_n257_b1_h1_g16_p64", "fd_n1055_b1_h4_g16_p64",
            "fd_n512_b1_h4_g16_p64", "fd_n192_b2_h2_g3_p64", "fd_n128_b1_h1_g1_p128"]
LADDER_SPLITS = {79: [1, 2, 3], 257: [1, 2, 3, 5], 1055: [1, 3, 5, 7], 512: [1, 2, 4, 8],
                 192: [1, 2], 128: [1, 2]}


def load(name):
    with np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def run_fixture(oracle, f, splits, element, stage=0, query=None):
    n, b, h, g, block, pages, phys = (int(x) for x in f["geometry"])
    q = f["query"] if query is None else query
    tag = "bf16" if element else "fp16"
    return oracle.kv4fp8_decode(
        q, f["key"], f["value"], f["scales"], f["block_table"], f["context_lens"],
        heads=h * g, kv_heads=h, block_size=block, max_blocks=pages, num_blocks=phys,
        splits=splits, fused_context_limit=0, element_type=element, output_stage=stage,
        pi_signs=f["pi_signs"], gate=f[f"gate_{tag}"] if stage == 2 else None)


@pytest.mark.parametrize("name", FIXTURES)
@pytest.mark.parametrize("element", [0, 1])
def test_fixture_bit_exact(oracle, name, element):
    f = load(name)
    n = int(f["geometry"][0])
    for k in LADDER_SPLITS[n]:
        out, _ = run_fixture(oracle, f, k, element)
        want = f["expected_bits_bf16" if element else "expected_bits_fp16"]
        assert np.array_equal(out.reshape(-1), want), (name, element, k)


def test_fixture_fused_limit_is_partition_only(oracle):
    """A context under the fused limit runs as one worker: same bits."""
    f = load("fd_n1055_b1_h4_g16_p64")
    n, b, h, g, block, pages, phys = (int(x) for x in f["geometry"])
    out, _ = oracle.kv4fp8_decode(
        f["query"], f["key"], f["value"], f["scales"], f["block_table"], f["context_lens"],
        heads=h * g, kv_heads=h, block_size=block, max_blocks=pages, num_blocks=phys, splits=7,
        fused_context_limit=4096)
    assert np.array_equal(out.reshape(-1), f["expected_bits_fp16"])


@pytest.mark.parametrize("element", [0, 1])
def test_raw_query_prologue_reproduces_fixture_query(oracle, element):
    f = load("fd_n79_b1_h1_g16_p64")
    tag = "bf16" if element else "fp16"
    rot = oracle.kv4fp8_rotate_query(f[f"raw_query_{tag}"].reshape(-1, 256), f["pi_signs"],
                                     0.0625, element)
    assert np.array_equal(rot.reshape(-1).view(np.uint32), f["query"].view(np.uint32))


@pytest.mark.parametrize("stage", [1, 2])
@pytest.mark.parametrize("element", [0, 1])
def test_output_stages_against_fixture(oracle, stage, element):
    for name in ("fd_n79_b1_h1_g16_p64", "fd_n192_b2_h2_g3_p64"):
        f = load(name)
        out, of = run_fixture(oracle, f, 2, element, stage=stage)
        want = f[f"expected_stage{stage}"]
        # FP32 butterflies against the fixture's FP64 ones: a few FP32 ulps
        assert np.allclose(of.reshape(-1), want, rtol=1e-5, atol=2e-6), (name, stage)
        wb = np.array([oracle.lib.tq4o_f32_to_elem(element, float(x)) for x in want], np.uint16)
        ulp = np.abs(out.reshape(-1).astype(np.int64) - wb.astype(np.int64))
        assert ulp.max() <= 1 and (ulp > 0).mean() < 0.01, (name, stage, ulp.max())
        # planted mistake: the stage skipped -> far from the expected rows
        if stage == 1:
            assert not np.allclose(f["expected"], want, rtol=1e-2, atol=1e-3)


def test_nz_layout_matches_reference(oracle):
    f = load("fd_nz_layout")
    got = np.array([oracle.lib.tq4o_nz_byte(int(s), int(k), int(c), int(h), 128)
                    for s, k, c, h in f["args"]], np.uint64)
    assert np.array_equal(got, f["byte"])
    for H in (1, 2, 4):  # a bijection onto one 64-row tile of every head
        seen = {oracle.lib.tq4o_nz_byte(r, k, c, H, 128)
                for r in range(64) for k in range(H) for c in range(128)}
        assert seen == set(range(64 * H * 128))


def _fp8_grid():
    codes = np.arange(256, dtype=np.uint8)
    e = (codes >> 3) & 15
    m = codes & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1 + m / 8.0) * 2.0 ** (e.astype(np.int64) - 7))
    val = np.where(codes & 0x80, -mag, mag)
    finite = ~((e == 15) & (m == 7))
    return codes[finite], val[finite]


def test_fp8_encoder_brute_force(oracle):
    codes, vals = _fp8_grid()
    pos = np.unique(vals[vals >= 0])
    mids = (pos[:-1] + pos[1:]) / 2
    rng = np.random.default_rng(1)
    xs = np.concatenate([pos, mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
                         np.nextafter(mids.astype(np.float32), np.float32(1e9)),
                         rng.uniform(0, 448, 20000), 2.0 ** rng.uniform(-12, 8.8, 20000)])
    xs = np.concatenate([xs, -xs]).astype(np.float32)
    for x in xs:
        b = oracle.lib.tq4o_fp8_e4m3_encode(float(x))
        got = oracle.lib.tq4o_fp8_e4m3_decode(b)
        d = np.abs(vals - np.float64(x))
        best = d.min()
        cand = codes[d == best]
        if cand.size > 1:  # a tie: the even mantissa
            cand = cand[(cand & 1) == 0]
        want = vals[codes == cand[0]][0]
        assert got == want or (got == 0 and want == 0), (x, got, want)


def test_two_level_tile_closed_form(oracle):
    """One tile, q = e0 (so q quantises to 448 e0 exactly), keys at two levels
    on channel 0, constant scales. The answer is the two-term expression
    (sum_t fp8(448 p_t / p_max) v_t) * (p_max / 448) / sum_t p_t: it pins where
    the probability operand is normalised and rounded."""
    H, G, S, P = 1, 1, 64, 2
    key = np.zeros(P * S * H * 128, np.uint8)
    val = np.zeros_like(key)
    lo, hi = 3, 1  # channel 0 levels 3.5 (rows 0..31) and 1.5 (rows 32..63)
    for r in range(64):
        key[oracle.lib.tq4o_nz_byte(r, 0, 0, H, 128)] = lo if r < 32 else hi
        for c in range(128):
            vb = (r * 7 + c) % 16 | (((r + 3 * c) % 16) << 4)
            val[oracle.lib.tq4o_nz_byte(r, 0, c, H, 128)] = vb
    scales = np.zeros(P * S * 8, np.float32)
    scales[0::8] = GAIN * 4.0
    scales[1::8] = GAIN
    q = np.zeros((1, 1, 256), np.float32)
    q[0, 0, 0] = 1.0
    table = np.array([[0]], np.int32)
    scale = np.float32(0.37)
    _, of = oracle.kv4fp8_decode(q, key, val, scales, table, np.array([64], np.int32), heads=1,
                                 kv_heads=1, block_size=S, max_blocks=1, num_blocks=P,
                                 scale=float(scale))
    # the logits in FP32, as the reference rounds them
    ks = np.float32(GAIN * np.float32(4.0)) * np.float32(scale / GAIN)
    qinv = np.float32(1) / np.float32(np.float32(448) / np.float32(1 + 1e-20))
    s = np.array([np.float32(np.float32(np.float32(448 * (lv + 0.5)) * ks) * qinv)
                  for lv in (lo, hi)], np.float64)
    p = np.exp(s - s.max())               # [1, e^-d]
    pop = np.array([448.0, oracle.fp8_round(np.float32(448.0 * p[1]))[0]])
    lev = lambda b, h: ((b >> 4) if h else (b & 15)) - 16 * (((b >> 4) if h else (b & 15)) >= 8) + 0.5
    want = np.zeros(256)
    for r in range(64):
        w = pop[0] if r < 32 else pop[1]
        for c in range(128):
            vb = (r * 7 + c) % 16 | (((r + 3 * c) % 16) << 4)
            want[c] += w * lev(vb, 0)
            want[c + 128] += w * lev(vb, 1)
    want = want / 448.0 / (32 * p[0] + 32 * p[1])  # v scale / gain = 1
    assert np.allclose(of[0, 0], want, rtol=1e-5, atol=1e-6)
    # planted mistake: rounding p * v_scale without the 448 normalisation
    bad = np.array([oracle.fp8_round(np.float32(x))[0] for x in p])
    assert abs(bad[1] / bad[0] - pop[1] / pop[0]) > 1e-3


# ------------------------------------------------------------ random caches
def _nz_tile_index(h):
    r = np.arange(64)[:, None]
    c = np.arange(128)[None, :]
    return h * 64 * 128 + ((c // 32) * 64 + r) * 32 + c % 32


def _levels(b, hi, signed=True):
    n = ((b >> 4) if hi else (b & 15)).astype(np.int64)
    return (np.where(n >= 8, n - 16, n) if signed else n) + 0.5


def random_case(rng, T, H, G, S, P, ctx, key_scale=(0.02, 0.3)):
    """Random NZ caches; key_scale sets the logit spread (the default gives
    logits of standard deviation ~0.5, (0.5, 2.0) about 5: a peaked softmax)."""
    key = rng.integers(0, 256, P * S * H * 128, dtype=np.uint8)
    val = rng.integers(0, 256, P * S * H * 128, dtype=np.uint8)
    scales = np.full(P * S * 8, np.nan, np.float32)
    for h in range(H):
        scales[h::8] = rng.uniform(*key_scale, P * S).astype(np.float32) * GAIN
        scales[H + h::8] = rng.uniform(0.5, 2.0, P * S).astype(np.float32) * GAIN
    maxb = max((c + S - 1) // S for c in ctx)
    table = np.full((T, maxb), -1, np.int32)
    perm = rng.permutation(P)
    k = 0
    for t in range(T):
        nb = (ctx[t] + S - 1) // S
        table[t, :nb] = perm[k:k + nb]
        k += nb
    q = rng.standard_normal((T, H * G, 256)).astype(np.float32)
    return q, key, val, scales, table, np.array(ctx, np.int32)


def fp64_attention(q, key, val, scales, table, ctx, H, G, S, scale, signed=True, swap_v=False,
                   lane_swap=False, keep=None):
    T = len(ctx)
    out = np.zeros((T, H * G, 256))
    for t in range(T):
        n = int(ctx[t])
        for h in range(H):
            K = np.zeros((n, 256))
            V = np.zeros((n, 256))
            ks = np.zeros(n)
            vs = np.zeros(n)
            for r0 in range(0, n, 64):
                phys = table[t, r0 // S]
                idx = phys * S * H * 128 + (r0 % S) * H * 128 + _nz_tile_index(h)
                m = min(64, n - r0)
                kb, vb = key[idx][:m], val[idx][:m]
                K[r0:r0 + m, :128], K[r0:r0 + m, 128:] = _levels(kb, 0, signed), _levels(kb, 1, signed)
                a, b = (1, 0) if swap_v else (0, 1)
                V[r0:r0 + m, :128], V[r0:r0 + m, 128:] = _levels(vb, a, signed), _levels(vb, b, signed)
                sl = (phys * S + r0 % S + np.arange(m)) * 8
                kl, vl = (H + h, h) if lane_swap else (h, H + h)
                ks[r0:r0 + m], vs[r0:r0 + m] = scales[sl + kl], scales[sl + vl]
            K *= (ks / GAIN)[:, None]
            V *= (vs / GAIN)[:, None]
            for g in range(G):
                s = scale * (K @ q[t, h * G + g].astype(np.float64))
                if keep is not None:
                    s = np.where(keep[:n], s, -np.inf)
                p = np.exp(s - s.max())
                out[t, h * G + g] = (p / p.sum()) @ V
    return out


def test_random_against_fp64_attention_and_split_invariance(oracle):
    rng = np.random.default_rng(5)
    T, H, G, S, P = 3, 2, 8, 64, 80
    q, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, [1000, 77, 2049])
    kw = dict(heads=H * G, kv_heads=H, block_size=S, max_blocks=tb.shape[1], num_blocks=P)
    outs = [oracle.kv4fp8_decode(q, key, val, sc, tb, ln, splits=k, **kw)[1] for k in (1, 3, 8)]
    for o in outs[1:]:
        assert np.allclose(o, outs[0], rtol=2e-5, atol=2e-6)
    ref = fp64_attention(q, key, val, sc, tb, ln, H, G, S, 0.0625)
    err = np.abs(outs[0] - ref)
    mag = np.abs(ref).mean()
    # the FP8 rounding of the query and probability operands
    assert err.mean() / mag < 0.05 and err.max() < 0.3, (err.mean() / mag, err.max())
    for kwargs in (dict(signed=False), dict(swap_v=True), dict(lane_swap=True)):
        bad = fp64_attention(q, key, val, sc, tb, ln, H, G, S, 0.0625, **kwargs)
        assert np.abs(outs[0] - bad).mean() > 20 * err.mean(), kwargs


def test_unmapped_pages_are_dropped_and_geometry_refused(oracle):
    rng = np.random.default_rng(6)
    T, H, G, S, P = 1, 1, 4, 64, 12
    q, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, [400])
    kw = dict(heads=H * G, kv_heads=H, block_size=S, num_blocks=P)
    tb2 = tb.copy()
    tb2[0, 2] = -1  # rows 128..191 dropped
    _, a = oracle.kv4fp8_decode(q, key, val, sc, tb2, ln, max_blocks=tb.shape[1], **kw)
    keep = np.ones(400, bool)
    keep[128:192] = False
    ref = fp64_attention(q, key, val, sc, tb, ln, H, G, S, 0.0625, keep=keep)
    full = fp64_attention(q, key, val, sc, tb, ln, H, G, S, 0.0625)
    err = np.abs(a - ref).mean()
    assert err / np.abs(ref).mean() < 0.05
    assert np.abs(a - full).mean() > 2 * err  # the dropped rows mattered
    with pytest.raises(ValueError):
        oracle.kv4fp8_decode(q, key, val, sc, tb, ln, max_blocks=tb.shape[1], splits=9, **kw)
    with pytest.raises(ValueError):
        oracle.kv4fp8_decode(q, key, val, sc, tb, ln, max_blocks=tb.shape[1], heads=4,
                             kv_heads=1, block_size=96, num_blocks=P)
