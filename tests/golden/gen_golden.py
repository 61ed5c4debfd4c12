#!/usr/bin/env python3
"""Write the golden fixtures under tests/golden/ from the reference's own oracles.

Runs only where the reference checkout is mounted and oracle/_ref/libtq4_ref.so
was built from it (``make -C oracle ref``). Every vector comes from calling the
reference's header-only CPU oracles through that shim; nothing of the
reference's source is stored -- only inputs and expected outputs, as .npz data
(load with numpy.load, allow_pickle=False) plus manifest.json with sha256 and
provenance. Reference functions used (paths relative to the reference checkout):

  w1_*   tq_oracle::compute_oracle_reference, build_activations,
         build_slot_mapping, audit_reference    tests/common/turboquant_oracle.hpp
  w2_*   tq_scatter::compute_reference, activation
                                                tests/common/turboquant_scatter_oracle.hpp
  d1_*   splitk_decode_test::Fixture (FP64 expected context)
                                                tests/common/splitk_decode_fixture.hpp
  d2_*   splitk_decode_test::ReferenceAicPartial
                                                tests/common/aic_splitk_decode_fixture.hpp
  c1_*   l2_probe_oracle::tile_state, combine_sequence, uniform_expected,
         egress_reference, gate_vector          tests/common/l2_atomic_oracle.hpp
  rot_*  rot_oracle::staged, dense_left, dense_right
                                                tests/common/rotate_butterfly_oracle.hpp
  cb_*   icdf::make_fixture (inputs + packed bytes of the ICDF leaf's oracle)
                                                tests/cpu/icdf_fixture.hpp
         lloyd::fixture, lloyd::code, lloyd::centroid, lloyd::pack, thresholds
                                                tests/common/lloydmax_oracle.hpp,
                                                include/routines/routine_vector_lloydmax_quantize.hpp
  fd_*   fused_decode_opt_test::Fixture (KV4/FP8 NZ cache, inputs and FP64
         expected rows in both element formats), RawQueryBasis, raw_query,
         gate_logits, expected_row (output stages 1, 2)
                                                tests/common/fused_decode_opt_fixture.hpp
  tail_* turboquant_splitk::Partition, turboquant_decode_tail::ActiveInStrip,
         LiveStripsInWindow                     include/turboquant_splitk_contract.hpp,
                                                kernels/ops/turboquant/turboquant_decode_tail.hpp
"""
import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
from oracle_bindings import Ref, ptr  # noqa: E402


def save(name, **arrays):
    path = os.path.join(HERE, name + ".npz")
    np.savez_compressed(path, **arrays)
    return path


def tq_fixture(r, T, H, d, S, P, key=None, value=None, slots=None):
    if key is None:
        key = np.zeros((T, H, d), np.int8)
        value = np.zeros((T, H, d), np.int8)
        r.lib.ref_tq_build_activations(T, H, d, S, P, ptr(key), ptr(value))
    if slots is None:
        slots = np.zeros(T, np.int32)
        r.lib.ref_tq_build_slot_mapping(T, H, d, S, P, ptr(slots))
    nbytes = P * H * S * d // 2
    kc = np.zeros(nbytes, np.int8)
    vc = np.zeros(nbytes, np.int8)
    sc = np.zeros(2 * P * H * S, np.float32)
    pw = np.zeros(P, np.int8)
    ok = np.zeros(1, np.int32)
    bad = r.lib.ref_tq_compute_reference(T, H, d, S, P, ptr(key), ptr(value), ptr(slots), ptr(kc),
                                         ptr(vc), ptr(sc), ptr(pw), ptr(ok))
    return dict(key=key, value=value, slots=slots, key_cache=kc, value_cache=vc, scale_cache=sc,
                page_written=pw, audit_ok=ok, bad_slot_strip=np.array([bad], np.int32),
                shape=np.array([T, H, d, S, P], np.int32))


def main():
    if not Ref.available():
        sys.exit("oracle/_ref/libtq4_ref.so missing: run make -C oracle ref (needs the reference)")
    r = Ref()
    files = {}

    # ---- W1: the aligned writer
    files["w1_ref_d256_h4"] = save("w1_ref_d256_h4", **tq_fixture(r, 64, 4, 256, 16, 10))
    files["w1_ref_d128_h8"] = save("w1_ref_d128_h8", **tq_fixture(r, 64, 8, 128, 16, 10))
    rng = np.random.default_rng(0x71340001)
    k = rng.integers(-127, 128, (16, 8, 128), dtype=np.int8)
    v = rng.integers(-127, 128, (16, 8, 128), dtype=np.int8)
    files["w1_config1_d128_h8"] = save(
        "w1_config1_d128_h8", **tq_fixture(r, 16, 8, 128, 16, 4, k, v, np.arange(16, dtype=np.int32)))

    # ---- W2: the arbitrary-slot writer (d = 256 only in the reference)
    H, S, P, d = 4, 32, 8, 256
    cu = np.array([0, 5, 6, 10], np.int32)
    slots = np.array([45, 46, 47, 48, 49,      # request 0: crosses the strip boundary at 48
                      100,                     # request 1: one token
                      200, -1, 130, 131], np.int32)  # request 2: a pad and a jump
    zero_token = 2
    key = np.zeros((cu[-1], H, d), np.uint16)
    value = np.zeros_like(key)
    from oracle_bindings import f32_to_bf16
    for req in range(len(cu) - 1):
        for t in range(cu[req], cu[req + 1]):
            for h in range(H):
                for plane, arr in ((0, key), (1, value)):
                    row = [r.lib.ref_scatter_activation(req, plane, h, t, c, zero_token) for c in range(d)]
                    arr[t, h] = f32_to_bf16(np.array(row, np.float32))
    signs = np.array([float(r.lib.ref_tq_pi_sign(c)) for c in range(d)], np.float32)
    prng = np.random.default_rng(0x51ED)
    prior_k = prng.integers(-128, 128, P * H * S * d // 2, dtype=np.int8)
    prior_v = prng.integers(-128, 128, P * H * S * d // 2, dtype=np.int8)
    prior_s = prng.standard_normal(2 * P * H * S).astype(np.float32)
    kc, vc, sc = prior_k.copy(), prior_v.copy(), prior_s.copy()
    zr = np.zeros(1, np.int32)
    cr = np.zeros(1, np.int32)
    rc = r.lib.ref_scatter_compute_reference(len(cu) - 1, H, S, P, ptr(cu), ptr(slots), ptr(signs),
                                             zero_token, ptr(kc), ptr(vc), ptr(sc), ptr(zr), ptr(cr))
    assert rc == 0, rc
    files["w2_scatter_d256"] = save(
        "w2_scatter_d256", key=key, value=value, slots=slots, cu_seqlens=cu, signs=signs,
        prior_key_cache=prior_k, prior_value_cache=prior_v, prior_scale_cache=prior_s,
        key_cache=kc, value_cache=vc, scale_cache=sc, zero_rows=zr, clamped_rows=cr,
        shape=np.array([len(cu) - 1, H, d, S, P], np.int32))

    # ---- D1: the split-K decode fixture and its FP64 expected context
    def splitk(n, batch, heads, rows, page, live, fill):
        pages = np.zeros(1, np.int32)
        tokens = np.zeros(1, np.int32)
        r.lib.ref_splitk_fixture_dims(n, page, ptr(pages), ptr(tokens))
        pg = int(pages[0])
        q = np.zeros(batch * heads * rows * 256, np.uint16)
        kk = np.zeros(batch * pg * heads * page * 128, np.uint8)
        vv = np.zeros_like(kk)
        ss = np.zeros(batch * pg * heads * page * 2, np.float32)
        gate = np.zeros(q.size, np.float32)
        sg = np.zeros(256, np.float32)
        table = np.zeros(batch * pg, np.uint32)
        exp = np.zeros(q.size, np.float32)
        assert r.lib.ref_splitk_fixture(n, batch, heads, rows, page, live, fill, ptr(q), ptr(kk),
                                        ptr(vv), ptr(ss), ptr(gate), ptr(sg), ptr(table),
                                        ptr(exp)) == 0
        seq_len = n if live < 0 else live
        return dict(q=q, key_cache=kk, value_cache=vv, scale_cache=ss, gate=gate, signs=sg,
                    table=table.reshape(batch, pg).astype(np.int32), expected=exp,
                    params=np.array([n, batch, heads, rows, page, seq_len, fill, pg], np.int32))

    files["d1_splitk_384"] = save("d1_splitk_384", **splitk(384, 1, 4, 6, 128, -1, 1))
    files["d1_splitk_48_b2_g16"] = save("d1_splitk_48_b2_g16", **splitk(48, 2, 2, 16, 16, -1, 1))
    files["d1_splitk_400_tail_nan"] = save("d1_splitk_400_tail_nan", **splitk(400, 1, 4, 6, 128, 389, 2))

    # ---- D2: partial records of the AIC split-K decode (FP64), fixture (48, 2, 2, 16, 16)
    # and a ragged NaN-tailed one (40 tokens of capacity 48, 37 live)
    def partials(n, batch, heads, page, live, fill, Ks):
        pages = (n + page - 1) // page
        out = {}
        for K in Ks:
            m = np.zeros((batch, heads, K, 16), np.float64)
            l = np.zeros_like(m)
            acc = np.zeros((batch, heads, K, 16, 256), np.float64)
            for b in range(batch):
                for h in range(heads):
                    for s in range(K):
                        beg = np.zeros(1, np.uint32)
                        cnt = np.zeros(1, np.uint32)
                        r.lib.ref_partition(pages, K, s, ptr(beg), ptr(cnt))
                        mm = np.zeros(16, np.float64)
                        ll = np.zeros(16, np.float64)
                        aa = np.zeros(16 * 256, np.float64)
                        assert r.lib.ref_aic_partial(n, batch, heads, page, live, fill, b, h,
                                                     int(beg[0]), int(cnt[0]), ptr(mm), ptr(ll),
                                                     ptr(aa)) == 0
                        m[b, h, s], l[b, h, s], acc[b, h, s] = mm, ll, aa.reshape(16, 256)
            out[f"m_K{K}"], out[f"l_K{K}"], out[f"acc_K{K}"] = m, l, acc
        return out

    fx = splitk(48, 2, 2, 16, 16, -1, 1)
    files["d2_aic_partials_48"] = save("d2_aic_partials_48", **fx,
                                       **partials(48, 2, 2, 16, -1, 1, (1, 2, 4)))
    fx = splitk(48, 1, 2, 16, 16, 37, 2)
    files["d2_aic_partials_tail"] = save("d2_aic_partials_tail", **fx,
                                         **partials(48, 1, 2, 16, 37, 2, (1, 4)))

    # ---- C1: the LSE combine and the tail egress
    c1 = {}
    for fixture, tag in ((0, "uniform"), (1, "staggered")):
        for K in (2, 4, 8):
            tiles = np.zeros((K, 258), np.float32)
            for s in range(K):
                r.lib.ref_l2_tile_state(fixture, s, ptr(tiles[s]))
            comb = np.zeros(258, np.float32)
            egr = np.zeros(256, np.float32)
            r.lib.ref_l2_combine_and_egress(fixture, K, ptr(comb), ptr(egr))
            c1[f"{tag}_K{K}_tiles"] = tiles
            c1[f"{tag}_K{K}_combined"] = comb
            c1[f"{tag}_K{K}_egress"] = egr
    for K in range(1, 9):
        u = np.zeros(258, np.float32)
        assert r.lib.ref_l2_uniform_expected(K, 1, ptr(u)) == 0
        c1[f"uniform_expected_K{K}"] = u
    gate = np.zeros(256, np.float32)
    r.lib.ref_l2_gate_vector(ptr(gate))
    c1["gate"] = gate
    c1["signs"] = np.array([float(r.lib.ref_tq_pi_sign(c)) for c in range(256)], np.float32)
    files["c1_l2_combine"] = save("c1_l2_combine", **c1)

    # ---- rotation at d = 256
    rrng = np.random.default_rng(0xB0771E)
    xs = np.concatenate([rrng.integers(-128, 128, (4, 256)).astype(np.float32),
                         rrng.standard_normal((4, 256)).astype(np.float32)])
    sg = np.array([float(r.lib.ref_tq_pi_sign(c)) for c in range(256)], np.float32)
    alt = np.where(rrng.random(256) < 0.5, -1.0, 1.0).astype(np.float32)
    rot = {"x": xs, "signs": sg, "signs_alt": alt}
    for tag, s in (("canon", sg), ("alt", alt)):
        for name, fn in (("ingress", 1), ("egress", 0)):
            out = np.zeros_like(xs)
            for i in range(len(xs)):
                r.lib.ref_rot_staged(fn, ptr(xs[i]), ptr(s), 1.0, ptr(out[i]))
            rot[f"{name}_{tag}"] = out
        dl = np.zeros_like(xs)
        dr = np.zeros_like(xs)
        for i in range(len(xs)):
            r.lib.ref_rot_dense_left(ptr(xs[i]), ptr(s), ptr(dl[i]))
            r.lib.ref_rot_dense_right(ptr(xs[i]), ptr(s), ptr(dr[i]))
        rot[f"dense_left_{tag}"] = dl
        rot[f"dense_right_{tag}"] = dr
    files["rot_d256"] = save("rot_d256", **rot)

    # ---- split partition and tail arithmetic
    part = np.zeros((128, 16, 16, 2), np.int32)
    for pages in range(1, 129):
        for K in range(1, 17):
            for s in range(K):
                beg = np.zeros(1, np.uint32)
                cnt = np.zeros(1, np.uint32)
                r.lib.ref_partition(pages, K, s, ptr(beg), ptr(cnt))
                part[pages - 1, K - 1, s] = (beg[0], cnt[0])
    bases = np.arange(0, 300, 3, dtype=np.uint64)
    seqs = np.array([0, 1, 15, 16, 17, 127, 129, 273], np.uint32)
    active = np.array([[r.lib.ref_active_in_strip(int(b), int(s)) for s in seqs] for b in bases],
                      np.int32)
    live_cases = np.array([[sl, pb, sp, bs, sb, st] for sl in (0, 1, 15, 16, 17, 100, 4103)
                           for (pb, sp, bs, sb, st) in ((0, 4, 16, 0, 1), (1, 3, 32, 0, 2),
                                                        (0, 300, 16, 0, 1))], np.uint32)
    live = np.array([r.lib.ref_live_strips_in_window(*map(int, c)) for c in live_cases], np.int32)
    files["tail_partition"] = save("tail_partition", partition=part, bases=bases, seq_lens=seqs,
                                   active=active, live_cases=live_cases, live=live)

    # ---- codebook leaves: ICDF (FP16/BF16 fixtures with the oracle's bytes),
    # Lloyd-Max and the Gaussian-CDF compander (codes, centroids, packing)
    for bf16, tag in ((0, "fp16"), (1, "bf16")):
        tiles = 4
        in_bits = np.zeros(tiles * 1024, np.uint16)
        packed = np.zeros(tiles * 512, np.uint8)
        assert r.lib.ref_icdf_fixture(bf16, tiles, ptr(in_bits), ptr(packed)) == 0
        files[f"cb_icdf_{tag}"] = save(f"cb_icdf_{tag}", in_bits=in_bits, packed=packed)
    for bits in (2, 4):
        cb = {}
        for n, rows, bnd in ((128, 1, 1), (256, 8, 1), (256, 8, 0)):
            x = np.zeros(n * rows, np.float32)
            r.lib.ref_lloyd_fixture(n, rows, bnd, bits, ptr(x))
            key = f"n{n}_r{rows}_b{bnd}"
            cb[f"x_{key}"] = x
            for sig, book in ((0, "lm"), (1, "cdf")):
                q = np.array([r.lib.ref_lloyd_code(bits, float(v), sig) for v in x], np.uint32)
                pk = np.zeros(x.size * bits // 8, np.uint8)
                r.lib.ref_lloyd_pack(ptr(q), q.size, bits, ptr(pk))
                cb[f"codes_{book}_{key}"] = q
                cb[f"packed_{book}_{key}"] = pk
        cb["centroids_lm"] = np.array([r.lib.ref_lloyd_centroid(bits, i, 0) for i in range(1 << bits)],
                                      np.float32)
        cb["centroids_cdf"] = np.array([r.lib.ref_lloyd_centroid(bits, i, 1) for i in range(1 << bits)],
                                       np.float32)
        cb["thresholds_lm"] = np.array([r.lib.ref_lloyd_threshold(bits, i)
                                        for i in range((1 << bits) - 1)], np.float32)
        files[f"cb_lloyd_b{bits}"] = save(f"cb_lloyd_b{bits}", **cb)

    # ---- FD: the KV4/FP8 fused decode fixture (the reference's NPU ladder rungs)
    for (n, b, h, g, block) in [(79, 1, 1, 16, 64), (257, 1, 1, 16, 64), (1055, 1, 4, 16, 64),
                                (512, 1, 4, 16, 64), (192, 2, 2, 3, 64), (128, 1, 1, 1, 128)]:
        sz = np.zeros(6, np.int64)
        pages = r.lib.ref_fdo_dims(n, b, h, g, block, ptr(sz))
        assert pages > 0
        fd = {"geometry": np.array([n, b, h, g, block, pages, sz[5]], np.int32)}
        for el, tag in ((0, "fp16"), (1, "bf16")):
            q = np.zeros(sz[0], np.float32)
            kk = np.zeros(sz[1], np.uint8)
            vv = np.zeros(sz[1], np.uint8)
            sc = np.zeros(sz[2], np.float32)
            tb = np.zeros(sz[3], np.int32)
            ln = np.zeros(sz[4], np.int32)
            ex = np.zeros(sz[0], np.float32)
            eb = np.zeros(sz[0], np.uint16)
            assert r.lib.ref_fdo_fixture(n, b, h, g, block, el, *[ptr(x) for x in
                                         (q, kk, vv, sc, tb, ln, ex, eb)]) == 0
            if el == 0:
                fd.update(query=q, key=kk, value=vv, scales=sc, block_table=tb,
                          context_lens=ln[:b], expected=ex)
            else:  # the element changes no input and no FP32 expected value
                assert np.array_equal(q, fd["query"]) and np.array_equal(ex, fd["expected"])
            fd[f"expected_bits_{tag}"] = eb
            raw = np.zeros(sz[0], np.uint16)
            gate = np.zeros(sz[0], np.uint16)
            signs = np.zeros(256, np.float32)
            for stage in (1, 2):
                er = np.zeros(sz[0], np.float32)
                assert r.lib.ref_fdo_raw(n, b, h, g, block, el, stage, ptr(raw), ptr(gate),
                                         ptr(signs), ptr(er)) == 0
                fd[f"expected_stage{stage}"] = er  # identical for both elements
            fd[f"raw_query_{tag}"] = raw
            fd[f"gate_{tag}"] = gate
            fd["pi_signs"] = signs
        fd["gain"] = np.array([r.lib.ref_fdo_gain()], np.float32)
        name = f"fd_n{n}_b{b}_h{h}_g{g}_p{block}"
        files[name] = save(name, **fd)
    nz = np.array([[s_, k_, c_, hh] for hh in (1, 3, 4) for s_ in (0, 1, 63, 64, 65, 127, 200)
                   for k_ in range(hh) for c_ in (0, 1, 31, 32, 63, 64, 127)], np.uint64)
    nz_bytes = np.array([r.lib.ref_nz_byte(int(a), int(b_), int(c), int(hh), 128)
                         for a, b_, c, hh in nz], np.uint64)
    files["fd_nz_layout"] = save("fd_nz_layout", args=nz, byte=nz_bytes)

    manifest = {}
    for name, path in files.items():
        data = open(path, "rb").read()
        manifest[name] = {"file": os.path.basename(path), "bytes": len(data),
                          "sha256": hashlib.sha256(data).hexdigest()}
    manifest["_provenance"] = (
        "generated by tests/golden/gen_golden.py from the reference's header-only CPU oracles "
        "compiled in place into oracle/_ref (tests/common/*.hpp, include/turboquant_splitk_contract.hpp, "
        "kernels/ops/turboquant/turboquant_decode_tail.hpp, "
        "kernels/ops/turboquant/vllm_integration_layer/op_kernel/common/turboquant_layout.h)")
    with open(os.path.join(HERE, "manifest.json"), "w") as f:
        json.dump(manifest, f, indent=1, sort_keys=True)
    for name, meta in sorted(manifest.items()):
        if not name.startswith("_"):
            print(f"{meta['file']:34s} {meta['bytes']:8d} B")


if __name__ == "__main__":
    main()
