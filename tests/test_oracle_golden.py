"""The C oracle (oracle/tq4_oracle.c) against the reference's golden vectors.

Fixtures in tests/golden/ were produced by tests/golden/gen_golden.py from the
reference's own header-only oracles (see its docstring for the functions).
Writer images are compared bit for bit; decode outputs within the reference
rigs' budgets. Each golden set also carries a planted-mistake control: the
same comparison on a deliberately wrong oracle input must fail, so a test that
passes is not passing vacuously.
"""
import json
import math
import os

import numpy as np
import pytest

from oracle_bindings import FLAG_QUERY_ROTATED, IN_BF16, IN_INT8, POLICY_EXACT, ptr

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name + ".npz"), allow_pickle=False)


def test_manifest_hashes():
    import hashlib
    man = json.load(open(os.path.join(GOLD, "manifest.json")))
    for name, meta in man.items():
        if name.startswith("_"):
            continue
        data = open(os.path.join(GOLD, meta["file"]), "rb").read()
        assert hashlib.sha256(data).hexdigest() == meta["sha256"], name


# ------------------------------------------------------------------ writer
def run_writer(oracle, f, signs=None):
    T, H, d, S, P = (int(x) for x in f["shape"])
    kc = np.zeros_like(f["key_cache"])
    vc = np.zeros_like(f["value_cache"])
    sc = np.zeros_like(f["scale_cache"])
    sg = oracle.canonical_signs(d) if signs is None else signs
    skipped = oracle.reshape_and_cache(IN_INT8, f["key"], f["value"], kc, vc, sc, f["slots"], sg,
                                       H, d, S, P, np.float32(1.0 / math.sqrt(d)))
    return kc, vc, sc, skipped


@pytest.mark.parametrize("name", ["w1_ref_d256_h4", "w1_ref_d128_h8", "w1_config1_d128_h8"])
def test_writer_matches_tq_oracle(oracle, name):
    """tq_oracle::compute_oracle_reference, bit for bit (turboquant_oracle.hpp:476-513)."""
    f = load(name)
    assert int(f["audit_ok"][0]) == 1 or name.startswith("w1_config1")
    assert int(f["bad_slot_strip"][0]) == -1
    kc, vc, sc, skipped = run_writer(oracle, f)
    assert skipped == 0
    assert np.array_equal(kc, f["key_cache"])
    assert np.array_equal(vc, f["value_cache"])
    assert np.array_equal(sc.view(np.uint32), f["scale_cache"].view(np.uint32))


def test_writer_planted_sign_mistake_is_caught(oracle):
    f = load("w1_ref_d128_h8")
    signs = oracle.canonical_signs(128)
    signs[37] = -signs[37]
    kc, vc, sc, _ = run_writer(oracle, f, signs)
    assert not np.array_equal(kc, f["key_cache"])


def test_scatter_matches_tq_scatter(oracle):
    """tq_scatter::compute_reference incl. the zero row and preserved lanes
    (turboquant_scatter_oracle.hpp:291-342)."""
    f = load("w2_scatter_d256")
    R, H, d, S, P = (int(x) for x in f["shape"])
    kc = f["prior_key_cache"].copy()
    vc = f["prior_value_cache"].copy()
    sc = f["prior_scale_cache"].copy()
    n = oracle.reshape_scatter(f["key"], f["value"], kc, vc, sc, f["slots"], f["signs"],
                               f["cu_seqlens"], R, H, d, S, P, 0, R * H,
                               np.float32(1.0 / math.sqrt(d)))
    assert n > 0 and int(f["zero_rows"][0]) > 0
    assert np.array_equal(kc, f["key_cache"])
    assert np.array_equal(vc, f["value_cache"])
    assert np.array_equal(sc.view(np.uint32), f["scale_cache"].view(np.uint32))


# ------------------------------------------------------------------ decode
def decode_fixture_out(oracle, f, K, stage=2, table=None):
    n, batch, heads, rows, page, seq_len, fill, pg = (int(x) for x in f["params"])
    ctx = np.full(batch, seq_len, np.int32)
    P = batch * pg
    q = f["q"].reshape(batch, heads * rows, 256)
    tb = f["table"] if table is None else table
    _, out = oracle.paged_decode(q, f["key_cache"].view(np.int8), f["value_cache"].view(np.int8),
                                 f["scale_cache"], tb, ctx, f["signs"], f["gate"], heads * rows,
                                 heads, 256, page, P, K, np.float32(1.0), np.float32(1.0 / 16),
                                 stage, flags=FLAG_QUERY_ROTATED)
    return out.reshape(-1)


@pytest.mark.parametrize("name", ["d1_splitk_384", "d1_splitk_48_b2_g16", "d1_splitk_400_tail_nan"])
@pytest.mark.parametrize("K", [1, 3, 8])
def test_decode_matches_fp64_fixture(oracle, name, K):
    """Split-K decode + LSE combine + egress + gate vs the reference's FP64
    full-context Fixture::Reference (splitk_decode_fixture.hpp:193-248)."""
    f = load(name)
    out = decode_fixture_out(oracle, f, K)
    exp = f["expected"]
    assert np.all(np.isfinite(out))
    scale = np.abs(exp).max()
    assert np.abs(out - exp).max() <= 2e-5 * scale


def test_decode_planted_cyclic_pages_is_caught(oracle):
    """A decode that re-reads one page for every logical page must fail (the
    reference's cyclic-page negative control, test_splitk_decode_probe.cpp:76-90).
    A mere permutation of the table would not do: softmax over the whole
    context is invariant under reordering its pages."""
    f = load("d1_splitk_384")
    wrong = np.full(f["table"].shape, f["table"].reshape(-1)[0], dtype=np.int32)
    out = decode_fixture_out(oracle, f, 1, table=wrong)
    exp = f["expected"]
    assert np.abs(out - exp).max() > 1e-2 * np.abs(exp).max()


@pytest.mark.parametrize("name,Ks", [("d2_aic_partials_48", (1, 2, 4)), ("d2_aic_partials_tail", (1, 4))])
def test_partials_match_aic_reference(oracle, name, Ks):
    """Per-split (m, l, acc) vs ReferenceAicPartial (FP64), with the device rig's
    budgets (tests/npu/turboquant_splitk_rigs.hpp:144-158); empty or dead splits
    carry the exact neutral element."""
    f = load(name)
    n, batch, heads, rows, page, seq_len, fill, pg = (int(x) for x in f["params"])
    ctx = np.full(batch, seq_len, np.int32)
    q = f["q"].reshape(batch, heads * rows, 256)
    for K in Ks:
        ws = oracle.decode_partials(q, f["key_cache"].view(np.int8), f["value_cache"].view(np.int8),
                                    f["scale_cache"], f["table"], ctx, f["signs"], heads * rows,
                                    heads, 256, page, batch * pg, K, np.float32(1.0),
                                    np.float32(1.0 / 16), FLAG_QUERY_ROTATED)
        # ws [B][Hq][K][260] with Hq = heads*16 -> [B][heads][16][K]
        ws = ws.reshape(batch, heads, 16, K, 260)
        m_ref, l_ref, a_ref = f[f"m_K{K}"], f[f"l_K{K}"], f[f"acc_K{K}"]  # [B][heads][K][16(...)]
        for b in range(batch):
            for h in range(heads):
                for s in range(K):
                    m = ws[b, h, :, s, 0].astype(np.float64)
                    l = ws[b, h, :, s, 1].astype(np.float64)
                    a = ws[b, h, :, s, 4:].astype(np.float64)
                    mr, lr, ar = m_ref[b, h, s], l_ref[b, h, s], a_ref[b, h, s]
                    dead = lr == 0
                    assert np.all(m[dead] == np.float32(-3e38)) and np.all(l[dead] == 0)
                    assert np.all(a[dead] == 0)
                    live = ~dead
                    assert np.all(np.abs(m - mr)[live] <= 2e-6 * np.maximum(1, np.abs(mr[live])))
                    assert np.all(np.abs(l - lr)[live] <= 1e-4 * np.maximum(1, lr[live]))
                    amax = np.abs(ar).max(axis=1, keepdims=True)
                    tol = 2e-4 * amax + 1e-5 * lr[:, None] + 1e-6
                    assert np.all(np.abs(a - ar) <= tol)


# ------------------------------------------------------------ combine/egress
@pytest.mark.parametrize("tag", ["uniform", "staggered"])
@pytest.mark.parametrize("K", [2, 4, 8])
def test_combine_and_egress_match_l2_oracle(oracle, tag, K):
    """combine_step in split order and the tail egress, bit for bit
    (l2_atomic_oracle.hpp:156-176,247-260)."""
    f = load("c1_l2_combine")
    tiles = f[f"{tag}_K{K}_tiles"]
    m = np.array([-3e38], np.float32)
    l = np.zeros(1, np.float32)
    acc = np.zeros(256, np.float32)
    for s in range(K):
        t = np.ascontiguousarray(tiles[s, 2:])
        oracle.lib.tq4o_combine_step(ptr(m), ptr(l), ptr(acc), float(tiles[s, 0]),
                                     float(tiles[s, 1]), ptr(t), 256)
    comb = f[f"{tag}_K{K}_combined"]
    assert m[0] == comb[0] and l[0] == comb[1]
    assert np.array_equal(acc.view(np.uint32), comb[2:].view(np.uint32))
    # egress through the oracle's combine entry (records [m, l, 0, 0, acc])
    rec = np.zeros((1, 1, K, 260), np.float32)
    rec[0, 0, :, 0] = tiles[:, 0]
    rec[0, 0, :, 1] = tiles[:, 1]
    rec[0, 0, :, 4:] = tiles[:, 2:]
    _, out = oracle.combine(rec, f["signs"], f["gate"][None, :].copy(), 1, 256, K,
                            np.float32(1.0 / 16), 2)
    assert np.array_equal(out.reshape(-1).view(np.uint32), f[f"{tag}_K{K}_egress"].view(np.uint32))
    if tag == "uniform":
        u = f[f"uniform_expected_K{K}"]
        assert np.array_equal(acc, u[2:]) and l[0] == u[1]


# ---------------------------------------------------------------- rotation
@pytest.mark.parametrize("tag", ["canon", "alt"])
def test_rotation_stage_order_bit_exact(oracle, tag):
    """rot_oracle::staged in both directions, bit for bit, and the dense
    definition to FP32 rounding (rotate_butterfly_oracle.hpp:84-142)."""
    f = load("rot_d256")
    signs = f["signs"] if tag == "canon" else f["signs_alt"]
    for i, x in enumerate(f["x"]):
        y = oracle.rotate_ingress(x, signs)
        assert np.array_equal(y.view(np.uint32), f[f"ingress_{tag}"][i].view(np.uint32))
        z = oracle.rotate_egress(x, signs)
        assert np.array_equal(z.view(np.uint32), f[f"egress_{tag}"][i].view(np.uint32))
        yd = oracle.rotate_dense(x, signs)
        assert np.allclose(yd, f[f"dense_left_{tag}"][i], rtol=1e-6, atol=1e-3)
        zd = oracle.rotate_dense(x, signs, transpose=True)
        assert np.allclose(zd, f[f"dense_right_{tag}"][i], rtol=1e-6, atol=1e-3)


# ----------------------------------------------------------- partition/tail
def test_partition_matches_contract(oracle):
    """Partition (turboquant_splitk_contract.hpp:123-130), pages 1..128 x K 1..16."""
    part = load("tail_partition")["partition"]
    for pages in range(1, 129):
        for K in range(1, 17):
            owned = np.zeros(pages, np.int32)
            for s in range(K):
                b, c = oracle.partition(pages, K, s)
                assert (b, c) == tuple(part[pages - 1, K - 1, s])
                owned[b:b + c] += 1
            assert np.all(owned == 1)


def test_active_in_strip_matches_tail(oracle):
    f = load("tail_partition")
    for i, base in enumerate(f["bases"]):
        for j, s in enumerate(f["seq_lens"]):
            assert oracle.lib.tq4o_active_in_strip(int(base), int(s)) == f["active"][i, j]
