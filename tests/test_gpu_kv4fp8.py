"""GPU parity of the KV4/FP8 NZ-tiled decode (include/tq4_kv4fp8.h).

* the FP8 e4m3 operand rounding the kernel uses equals the oracle's
  round-to-nearest-even encoder bit for bit (grid values, midpoints and their
  neighbours, subnormals, random values);
* the reference's fixture: FP16 and BF16 outputs bit for bit on the stored
  rungs of its NPU ladder (its ULP budget is 0), every split count the ladder
  uses; the raw-query entry reproduces the fixture's rotated query bit for
  bit and its stage 0/1/2 outputs match the oracle's;
* random caches (ragged contexts, 1..4 KV heads, 1..32 q heads per KV head,
  64/128/256-row pages, several tokens): against the C oracle within
  max-abs 2e-2 (beyond one element ULP) and mean-rel 1e-3 of the
  element-rounded oracle output
  (both compute the reference's FP8 operands; they differ in FP32 summation
  order and the exp implementation);
* unmapped pages and NaN-poisoned tail rows;
* at a bench-sized context, size-independent properties: a shuffled page
  pool with the same logical content gives the same bits, and the result
  does not depend on the reference's split count.
"""
import numpy as np
import pytest
import torch

from gpu_helpers import DEV, dev
from test_oracle_kv4fp8 import FIXTURES, LADDER_SPLITS, load, random_case

pytestmark = pytest.mark.gpu


def bits(t):
    torch.cuda.synchronize()
    return t.view(torch.int16).cpu().numpy().view(np.uint16)


def elem_dtype(element):
    return torch.bfloat16 if element else torch.float16


def elem_to_f32(b, element):
    b = np.asarray(b, np.uint16)
    if element:
        return (b.astype(np.uint32) << 16).view(np.float32)
    return b.view(np.float16).astype(np.float32)


def test_fp8_rounding_matches_oracle(tq4, oracle):
    from test_oracle_kv4fp8 import _fp8_grid
    _, vals = _fp8_grid()
    pos = np.unique(vals[vals >= 0])
    mids = (pos[:-1] + pos[1:]) / 2
    rng = np.random.default_rng(3)
    x = np.concatenate([pos, mids, np.nextafter(mids.astype(np.float32), np.float32(0)),
                        np.nextafter(mids.astype(np.float32), np.float32(1e9)),
                        rng.uniform(0, 448, 50000), 2.0 ** rng.uniform(-14, 8.8, 50000),
                        [448.00003, 447.99997, 1e-30, 0.0]]).astype(np.float32)
    x = np.concatenate([x, -x])
    x = x[: x.size // 2 * 2]
    got = bits(tq4.fp8_e4m3_round(dev(x))).view(np.float16).astype(np.float32)
    want = oracle.fp8_round(x)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, [(x[i], got[i], want[i]) for i in bad[:8]]


def table_of(f):
    """The fixture's block table is padded to 32 bytes: [tokens][pages]."""
    b, pages = int(f["geometry"][1]), int(f["geometry"][5])
    return np.ascontiguousarray(f["block_table"][: b * pages].reshape(b, pages))


def run_fixture(tq4, f, splits, element):
    n, b, h, g, block, pages, phys = (int(v) for v in f["geometry"])
    out = tq4.kv4fp8_decode(dev(f["query"].reshape(b, h * g, 256)), dev(f["key"]),
                            dev(f["value"]), dev(f["scales"]), dev(table_of(f)),
                            dev(f["context_lens"]), h, block, phys, splits=splits,
                            out_dtype=elem_dtype(element), fused_context_limit=0)
    return bits(out).reshape(-1)


@pytest.mark.parametrize("name", FIXTURES)
@pytest.mark.parametrize("element", [0, 1])
def test_fixture_bit_exact(tq4, name, element):
    f = load(name)
    want = f["expected_bits_bf16" if element else "expected_bits_fp16"]
    for k in LADDER_SPLITS[int(f["geometry"][0])]:
        got = run_fixture(tq4, f, k, element)
        ulp = np.abs(got.astype(np.int64) - want.astype(np.int64))
        assert ulp.max() == 0, (name, element, k, int(ulp.max()), int((ulp > 0).sum()))


@pytest.mark.parametrize("element", [0, 1])
def test_raw_query_fixture_and_stages(tq4, oracle, element):
    tag = "bf16" if element else "fp16"
    for name in ("fd_n79_b1_h1_g16_p64", "fd_n192_b2_h2_g3_p64", "fd_n1055_b1_h4_g16_p64"):
        f = load(name)
        n, b, h, g, block, pages, phys = (int(v) for v in f["geometry"])
        shape = (b, h * g, 256)
        raw = dev(f[f"raw_query_{tag}"].reshape(shape).view(np.int16)).view(elem_dtype(element))
        gate = dev(f[f"gate_{tag}"].reshape(shape).view(np.int16)).view(elem_dtype(element))
        for stage in (0, 1, 2):
            qout = torch.full(shape, float("nan"), device=DEV)
            out = tq4.kv4fp8_decode_raw_query(
                raw, dev(f["pi_signs"]), dev(f["key"]), dev(f["value"]), dev(f["scales"]),
                dev(table_of(f)), dev(f["context_lens"]), h, block, phys,
                gate=gate if stage == 2 else None, output_stage=stage, query_out=qout,
                splits=3)
            got = bits(out).reshape(-1)
            assert np.array_equal(qout.cpu().numpy().reshape(-1).view(np.uint32),
                                  f["query"].view(np.uint32)), (name, stage)
            if stage == 0:
                want = f[f"expected_bits_{tag}"]
                assert np.array_equal(got, want), (name, stage)
            else:
                want, _ = oracle.kv4fp8_decode(
                    f["query"], f["key"], f["value"], f["scales"], f["block_table"],
                    f["context_lens"], heads=h * g, kv_heads=h, block_size=block,
                    max_blocks=pages, num_blocks=phys, splits=3, element_type=element,
                    output_stage=stage, pi_signs=f["pi_signs"],
                    gate=f[f"gate_{tag}"] if stage == 2 else None)
                ulp = np.abs(got.astype(np.int64) - want.reshape(-1).astype(np.int64))
                assert ulp.max() <= 1 and (ulp > 0).mean() < 0.01, (name, stage, ulp.max())


def compare(got_bits, want_f32, element):
    """(max-abs beyond one element ULP, mean-rel) of the device output against
    the oracle's FP32 rows rounded to the element format. One ULP of the
    element is allowed on top of the absolute bound: a BF16 output of
    magnitude 8..16 has a ULP of 0.0625, and an FP32-level difference can
    move the rounding by one."""
    got = elem_to_f32(got_bits, element).astype(np.float64)
    from oracle_bindings import f32_to_bf16
    if element:
        want = elem_to_f32(f32_to_bf16(want_f32), 1).astype(np.float64)
    else:
        want = want_f32.astype(np.float16).astype(np.float64)
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(want), 1e-30))) - (7 if element else 10))
    diff = np.abs(got - want)
    return float(np.max(np.maximum(diff - ulp, 0.0))), float(diff.sum() / max(np.abs(want).sum(), 1e-30))


CASES = [  # (tokens, kv heads, q heads per kv head, page rows, contexts)
    (1, 1, 16, 64, [1055]),
    (3, 2, 8, 64, [1000, 77, 2049]),
    (2, 4, 16, 128, [4096 + 7, 63]),
    (2, 1, 32, 256, [3000, 1]),
    (4, 3, 5, 64, [0, 64, 65, 500]),
]


@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("element", [0, 1])
def test_random_against_oracle(tq4, oracle, case, element):
    T, H, G, S, ctx = case
    rng = np.random.default_rng(hash((T, H, G, S)) & 0xFFFF)
    P = sum((c + S - 1) // S for c in ctx) + 5
    q, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, ctx, key_scale=(0.5, 2.0))
    kw = dict(heads=H * G, kv_heads=H, block_size=S, max_blocks=tb.shape[1], num_blocks=P,
              element_type=element)
    _, want = oracle.kv4fp8_decode(q, key, val, sc, tb, ln, **kw)
    out = tq4.kv4fp8_decode(dev(q), dev(key), dev(val), dev(sc), dev(tb), dev(ln), H, S, P,
                            out_dtype=elem_dtype(element))
    mx, mr = compare(bits(out), want, element)
    assert mx <= 2e-2 and mr <= 1e-3, (case, element, mx, mr)
    # the data discriminates: a plausible slip (adjacent query channels
    # swapped) moves the oracle's own output far outside that bound
    qs = q.copy()
    qs[..., 0::2], qs[..., 1::2] = q[..., 1::2], q[..., 0::2]
    _, slip = oracle.kv4fp8_decode(qs, key, val, sc, tb, ln, **kw)
    live = ln > 0
    if live.any():
        d = np.abs(slip[live] - want[live])
        assert d.sum() / np.abs(want[live]).sum() > 20e-3, (case, d.max())
    zero_rows = np.nonzero(ln == 0)[0]
    assert np.all(bits(out)[zero_rows] == 0)


@pytest.mark.parametrize("element", [0, 1])
def test_raw_query_zero_context_and_gate(tq4, oracle, element):
    """Raw-query entry, output stage 2, with tokens of zero context between
    live ones: part 0 writes the rotated query and the rows' gated zero
    output; the live tokens match the oracle on the same rotated query."""
    rng = np.random.default_rng(41 + element)
    T, H, G, S = 4, 2, 16, 64
    ctx = [0, 700, 0, 65]
    P = sum((c + S - 1) // S for c in ctx) + 3
    _, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, ctx, key_scale=(0.5, 2.0))
    from oracle_bindings import f32_to_bf16
    raw_f = rng.standard_normal((T, H * G, 256)).astype(np.float32)
    gate_f = rng.standard_normal((T, H * G, 256)).astype(np.float32) * 3
    if element:
        raw_b, gate_b = f32_to_bf16(raw_f), f32_to_bf16(gate_f)
    else:
        raw_b, gate_b = raw_f.astype(np.float16).view(np.uint16), gate_f.astype(np.float16).view(np.uint16)
    signs = np.where(rng.random(256) < 0.5, -1.0, 1.0).astype(np.float32)
    isl = np.float32(1 / 16)
    q_rot = oracle.kv4fp8_rotate_query(raw_b, signs, isl, element)
    want, want_f32 = oracle.kv4fp8_decode(q_rot, key, val, sc, tb, ln, heads=H * G,
                                          kv_heads=H, block_size=S, max_blocks=tb.shape[1],
                                          num_blocks=P, element_type=element, output_stage=2,
                                          pi_signs=signs, gate=gate_b)
    shape = (T, H * G, 256)
    raw = dev(raw_b.view(np.int16)).view(elem_dtype(element))
    gate = dev(gate_b.view(np.int16)).view(elem_dtype(element))
    qout = torch.full(shape, float("nan"), device=DEV)
    out = tq4.kv4fp8_decode_raw_query(raw, dev(signs), dev(key), dev(val), dev(sc), dev(tb),
                                      dev(ln), H, S, P, gate=gate, output_stage=2,
                                      query_out=qout)
    assert np.array_equal(qout.cpu().numpy().view(np.uint32), q_rot.view(np.uint32))
    got = bits(out)
    assert np.all(elem_to_f32(got[[0, 2]], element) == 0)  # +-0: the zero rows' signs follow Pi
    assert np.array_equal(got[[0, 2]], want[[0, 2]])
    # live rows: the decode's tolerance (the parts merge in another FP32 order)
    mx, mr = compare(got[[1, 3]], want_f32[[1, 3]], element)
    assert mx <= 2e-2 and mr <= 1e-3, (mx, mr)


@pytest.mark.parametrize("case", ["two_parts", "many_parts"])
def test_grid_beyond_resident_workgroups(tq4, oracle, case):
    """Grids beyond the resident workgroups: 75 tokens x 4 KV heads x 2 parts
    (600 workgroups), and 96 tokens x 4 KV heads with up to 8 live parts
    (about 2000 workgroups), so groups have four combiners and an early
    combiner can finish before its group's last ticket holder has started:
    it then hands its rows to the last ticket, and no combiner waits on a
    part that has not started. Two calls on one workspace agree bit for bit
    and leave the whole workspace zero."""
    rng = np.random.default_rng(31 if case == "two_parts" else 32)
    T, H, G, S = (75, 4, 16, 64) if case == "two_parts" else (96, 4, 16, 64)
    lo, hi = (300, 1500) if case == "two_parts" else (2000, 8192)
    ctx = [int(c) for c in rng.integers(lo, hi, T)]
    P = sum((c + S - 1) // S for c in ctx) + 4
    q, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, ctx, key_scale=(0.5, 2.0))
    kw = dict(heads=H * G, kv_heads=H, block_size=S, max_blocks=tb.shape[1], num_blocks=P)
    _, want = oracle.kv4fp8_decode(q, key, val, sc, tb, ln, **kw)
    L = tq4.fused_decode_opt_launch(T, H * G, H, S, tb.shape[1], num_blocks=P)
    ws = tq4.kv4fp8_workspace_init(
        torch.empty(tq4.kv4fp8_workspace_bytes(L), dtype=torch.uint8, device=DEV))
    args = (dev(q), dev(key), dev(val), dev(sc), dev(tb), dev(ln), H, S, P)
    first = bits(tq4.kv4fp8_decode(*args, workspace=ws)).copy()
    mx, mr = compare(first, want, 0)
    assert mx <= 2e-2 and mr <= 1e-3, (mx, mr)
    assert np.array_equal(bits(tq4.kv4fp8_decode(*args, workspace=ws)), first)
    assert not torch.any(ws)  # tickets and records are zero again


def test_unmapped_pages_and_poisoned_tail_rows(tq4, oracle):
    rng = np.random.default_rng(9)
    T, H, G, S = 2, 2, 8, 64
    ctx = [700, 301]
    P = 20
    q, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, ctx)
    tb[0, 3] = -1
    tb[1, 1] = P + 100  # out of the pool: skipped like an unmapped page
    # rows past each context inside its last tile: NaN scales
    for t, c in enumerate(ctx):
        page = tb[t, (c - 1) // S]
        for r in range(c % S, S):
            sc[(page * S + r) * 8:(page * S + r) * 8 + 8] = np.nan
    out = tq4.kv4fp8_decode(dev(q), dev(key), dev(val), dev(sc), dev(tb), dev(ln), H, S, P)
    tb_o = tb.copy()
    tb_o[1, 1] = -1
    _, want = oracle.kv4fp8_decode(q, key, val, np.nan_to_num(sc, nan=1.0), tb_o, ln,
                                   heads=H * G, kv_heads=H, block_size=S,
                                   max_blocks=tb.shape[1], num_blocks=P)
    got = bits(out)
    assert np.all(np.isfinite(elem_to_f32(got, 0)))
    mx, mr = compare(got, want, 0)
    assert mx <= 2e-2 and mr <= 1e-3, (mx, mr)


def test_bench_size_properties(tq4):
    """ctx 16384, 4 KV heads x 16: a shuffled pool with the same logical
    content gives the same bits; the reference's split count and fused limit
    (partition only) do not change the bits."""
    rng = np.random.default_rng(11)
    T, H, G, S, ctx = 1, 4, 16, 128, 16384
    P = ctx // S
    q, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, [ctx])
    args = lambda k, v, s, t: (dev(q), dev(k), dev(v), dev(s), dev(t), dev(ln), H, S, P)
    a = bits(tq4.kv4fp8_decode(*args(key, val, sc, tb), splits=1))
    b = bits(tq4.kv4fp8_decode(*args(key, val, sc, tb), splits=8, fused_context_limit=0))
    assert np.array_equal(a, b)
    perm = rng.permutation(P)  # physical page p moves to perm[p]
    page_bytes = S * H * 128
    key2 = np.empty_like(key)
    val2 = np.empty_like(val)
    sc2 = np.empty_like(sc)
    for p in range(P):
        key2[perm[p] * page_bytes:(perm[p] + 1) * page_bytes] = key[p * page_bytes:(p + 1) * page_bytes]
        val2[perm[p] * page_bytes:(perm[p] + 1) * page_bytes] = val[p * page_bytes:(p + 1) * page_bytes]
        sc2[perm[p] * S * 8:(perm[p] + 1) * S * 8] = sc[p * S * 8:(p + 1) * S * 8]
    tb2 = perm[tb].astype(np.int32)
    c = bits(tq4.kv4fp8_decode(*args(key2, val2, sc2, tb2)))
    assert np.array_equal(a, c)


def test_workspace_reuse_and_graph_replays(tq4):
    """The part tickets and records return to zero after every call: one
    workspace serves repeated eager calls and HIP graph replays (eager work
    and synchronisations in between), every result bit-identical; a second
    geometry on the same workspace too."""
    rng = np.random.default_rng(21)
    T, H, G, S = 3, 2, 16, 64
    ctx = [900, 1, 2000]
    P = sum((c + S - 1) // S for c in ctx) + 3
    q, key, val, sc, tb, ln = random_case(rng, T, H, G, S, P, ctx, key_scale=(0.5, 2.0))
    L = tq4.fused_decode_opt_launch(T, H * G, H, S, tb.shape[1], num_blocks=P)
    ws = torch.zeros(tq4.kv4fp8_workspace_bytes(L) + 4096, dtype=torch.uint8, device=DEV)
    args = (dev(q), dev(key), dev(val), dev(sc), dev(tb), dev(ln), H, S, P)
    out = torch.empty((T, H * G, 256), dtype=torch.float16, device=DEV)
    call = lambda: tq4.kv4fp8_decode(*args, out=out, workspace=ws)  # noqa: E731
    first = bits(call()).copy()
    for _ in range(3):
        assert np.array_equal(bits(call()), first)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for i in range(4):
        out.zero_()
        g.replay()
        assert np.array_equal(bits(out), first), f"replay {i}"
        assert np.array_equal(bits(call()), first), f"eager {i}"
    # another geometry on the same (still zero-ticketed) workspace
    q2, k2, v2, s2, t2, l2 = random_case(rng, 1, 1, 16, 128, 40, [3000])
    a = bits(tq4.kv4fp8_decode(dev(q2), dev(k2), dev(v2), dev(s2), dev(t2), dev(l2), 1, 128, 40,
                               workspace=ws))
    b = bits(tq4.kv4fp8_decode(dev(q2), dev(k2), dev(v2), dev(s2), dev(t2), dev(l2), 1, 128, 40))
    assert np.array_equal(a, b)
    assert np.array_equal(bits(call()), first)
    assert not torch.any(ws)  # tickets and records are zero again
