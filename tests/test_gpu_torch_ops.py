"""torch.ops.tq4 on the GPU: each operator's result equals the direct C-ABI
binding's bit for bit (same kernels), the writers equal the C oracle's cache
image, the decode is within the north_star's BF16 tolerance of the FP32
oracle, and a HIP graph of the decode operator replays to the eager result
every time (several replays, eager work and synchronisations in between)."""
import math

import numpy as np
import pytest
import torch

from gpu_helpers import bf16_out_error, canary_bytes, canary_floats, dev, host
from oracle_bindings import IN_BF16, f32_to_bf16

pytestmark = pytest.mark.gpu


def cache_shapes(P, H, S, d):
    return (P, H, S, d // 2), (2, P, H, S)


def written_cache(oracle, rng, P, H, S, d, T):
    key = f32_to_bf16(rng.standard_normal((T, H, d)).astype(np.float32))
    val = f32_to_bf16(rng.standard_normal((T, H, d)).astype(np.float32))
    pages = rng.permutation(P)[: T // S].astype(np.int32)
    slots = (pages[:, None] * S + np.arange(S, dtype=np.int32)[None, :]).reshape(-1)
    return key, val, pages, slots


def test_reshape_and_cache_op_matches_oracle(tq4, oracle):
    rng = np.random.default_rng(11)
    P, H, S, d, T = 32, 8, 16, 128, 64
    key, val, _, slots = written_cache(oracle, rng, P, H, S, d, T)
    signs = oracle.canonical_signs(d)
    isl = np.float32(1 / math.sqrt(d))
    kc, vc, sc = canary_bytes(P * H * S * d // 2), canary_bytes(P * H * S * d // 2), \
        canary_floats(2 * P * H * S)
    want = [x.copy() for x in (kc, vc, sc)]
    assert oracle.reshape_and_cache(IN_BF16, key, val, *want, slots, signs, H, d, S, P, isl) == 0
    ks, ss = cache_shapes(P, H, S, d)
    g_kc, g_vc, g_sc = dev(kc).view(ks), dev(vc).view(ks), dev(sc).view(ss)
    torch.ops.tq4.reshape_and_cache(dev(key), dev(val), g_kc, g_vc, g_sc, dev(slots), dev(signs),
                                    None, S, float(isl))
    assert np.array_equal(host(g_kc).reshape(-1), want[0])
    assert np.array_equal(host(g_vc).reshape(-1), want[1])
    assert np.array_equal(host(g_sc).reshape(-1).view(np.uint32), want[2].view(np.uint32))


def test_reshape_and_cache_op_int8(tq4, oracle):
    """INT8 input dispatches to the A8 writer: same bytes as the direct binding."""
    rng = np.random.default_rng(12)
    P, H, S, d, T = 16, 4, 16, 64, 32
    key = rng.integers(-127, 128, (T, H, d), dtype=np.int8)
    val = rng.integers(-127, 128, (T, H, d), dtype=np.int8)
    slots = (np.arange(T) + 3 * S).astype(np.int32)
    signs = oracle.canonical_signs(d)
    ks, ss = cache_shapes(P, H, S, d)
    a = [torch.zeros(ks, dtype=torch.int8, device="cuda"), torch.zeros(ks, dtype=torch.int8,
         device="cuda"), torch.zeros(ss, device="cuda")]
    b = [x.clone() for x in a]
    torch.ops.tq4.reshape_and_cache(dev(key), dev(val), *a, dev(slots), dev(signs), None, S, 0.0)
    tq4.reshape_and_cache_a8(dev(key), dev(val), *b, dev(slots), pi_signs=dev(signs),
                             num_blocks=P, block_size=S)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_reshape_scatter_op_matches_binding(tq4, oracle):
    rng = np.random.default_rng(13)
    P, H, S, d, R = 24, 4, 16, 128, 20
    key = f32_to_bf16(rng.standard_normal((R, H, d)).astype(np.float32))
    val = f32_to_bf16(rng.standard_normal((R, H, d)).astype(np.float32))
    strips = rng.permutation(P)[:R]
    slots = (strips * S + rng.integers(0, S, R)).astype(np.int32)
    slots[3] = -1  # padding token
    signs = dev(oracle.canonical_signs(d))
    ks, ss = cache_shapes(P, H, S, d)
    a = [dev(canary_bytes(P * H * S * d // 2)).view(ks), dev(canary_bytes(P * H * S * d // 2)).view(ks),
         dev(canary_floats(2 * P * H * S)).view(ss)]
    b = [x.clone() for x in a]
    torch.ops.tq4.reshape_scatter(dev(key), dev(val), *a, dev(slots), signs, None, S, 0.0)
    tq4.reshape_scatter(dev(key), dev(val), *b, dev(slots), signs, num_blocks=P, block_size=S)
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.int32), y.view(torch.int32))


def decode_inputs(oracle, rng, ctx_lens, Hq, H, d, S, P):
    from test_gpu_decode import build_cache
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx_lens, H, d, S, P)
    q = f32_to_bf16(rng.standard_normal((len(ctx_lens), Hq, d)).astype(np.float32))
    return q, kc, vc, sc, tables, np.array(ctx_lens, np.int32), signs, isl


def test_paged_attention_op_matches_binding_and_oracle(tq4, oracle):
    rng = np.random.default_rng(14)
    Hq, H, d, S, P = 16, 4, 128, 16, 220
    q, kc, vc, sc, tables, ctx, signs, isl = decode_inputs(oracle, rng, [900, 333, 2000], Hq, H,
                                                           d, S, P)
    scale = np.float32(1 / math.sqrt(d))
    want16, want = oracle.paged_decode(q, kc, vc, sc, tables, ctx, signs, None, Hq, H, d, S, P,
                                       6, scale, isl, 1, threads=8)
    ks, ss = cache_shapes(P, H, S, d)
    args = (dev(q), dev(kc).view(ks), dev(vc).view(ks), dev(sc).view(ss), dev(tables), dev(ctx),
            dev(signs))
    ws = tq4.torch_ops.workspace_for(args[0], H, args[4], S, 6)
    out = torch.ops.tq4.paged_attention(*args, ws, None, H, S, 6, float(scale), float(isl), 1, False)
    direct = tq4.paged_decode(*args, H, S, P, num_splits=6, scale=float(scale),
                              inv_sqrt_len=float(isl))
    assert torch.equal(out.view(torch.int16), direct.view(torch.int16))
    mx, mr = bf16_out_error(host(out), want)
    assert mx <= 2e-2 and mr <= 1e-3, (mx, mr)


def test_paged_attention_op_in_hip_graph(tq4, oracle):
    """Graph replays of the operator (workspace left zeroed by each call) match
    the eager output, with eager launches and synchronisations in between."""
    rng = np.random.default_rng(15)
    Hq, H, d, S, P = 32, 8, 128, 16, 340
    q, kc, vc, sc, tables, ctx, signs, isl = decode_inputs(oracle, rng, [4096, 1000], Hq, H, d,
                                                           S, P)
    ks, ss = cache_shapes(P, H, S, d)
    args = (dev(q), dev(kc).view(ks), dev(vc).view(ks), dev(sc).view(ss), dev(tables), dev(ctx),
            dev(signs))
    ws = tq4.torch_ops.workspace_for(args[0], H, args[4], S, 16)
    call = lambda: torch.ops.tq4.paged_attention(*args, ws, None, H, S, 16, 0.0, 0.0, 1, False)
    eager = call().clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_out = call()
    for i in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_out.view(torch.int16), eager.view(torch.int16)), f"replay {i}"
        assert torch.equal(call().view(torch.int16), eager.view(torch.int16)), f"eager {i}"


def test_fused_decode_opt_ops_match_bindings(tq4):
    """torch.ops.tq4.fused_decode_opt(_raw_query): the direct bindings' bits."""
    from test_oracle_kv4fp8 import random_case
    rng = np.random.default_rng(16)
    T, H, G, S = 2, 2, 16, 64
    ctx = [700, 1500]
    P = sum((c + S - 1) // S for c in ctx) + 2
    q, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, ctx, key_scale=(0.5, 2.0))
    d = [dev(x) for x in (q, key, val, sc, tb, ln)]
    ws = tq4.torch_ops.kv4fp8_workspace_for(d[0], H, d[4], S, P)
    for bf16 in (False, True):
        a = torch.ops.tq4.fused_decode_opt(d[0], d[1], d[2], d[3], d[4], d[5], ws, H, S, 3, 16,
                                           4096, 0.0, 0.0, bf16)
        b = tq4.kv4fp8_decode(*d, H, S, P, out_dtype=torch.bfloat16 if bf16 else torch.float16)
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    signs = dev(np.where(rng.random(256) < 0.5, -1.0, 1.0).astype(np.float32))
    raw = torch.from_numpy(q).to("cuda").to(torch.bfloat16)
    gate = torch.from_numpy(rng.standard_normal(q.shape).astype(np.float32)).to("cuda").to(torch.bfloat16)
    qr1, qr2 = torch.empty_like(d[0]), torch.empty_like(d[0])
    a = torch.ops.tq4.fused_decode_opt_raw_query(raw, signs, gate, qr1, d[1], d[2], d[3], d[4],
                                                 d[5], ws, H, S, 3, 16, 2, 4096, 0.0, 0.0)
    b = tq4.kv4fp8_decode_raw_query(raw, signs, d[1], d[2], d[3], d[4], d[5], H, S, P, gate=gate,
                                    output_stage=2, query_out=qr2)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert torch.equal(qr1.view(torch.int32), qr2.view(torch.int32))
