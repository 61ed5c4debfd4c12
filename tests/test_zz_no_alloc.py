"""tq4_paged_decode_noalloc: the fused decode on the library's static scratch.

Called through the C ABI (ctypes), it must give the bits of tq4_paged_decode
on a workspace of its own (same kernels, same split count) and the oracle's
result within the decode budget -- on calls in a row whose geometry shrinks
(the scratch keeps the previous call's contents: every word the decode uses
must be back at zero), including the persistent work-queue form, and under
HIP-graph replay. A call too large for the scratch is refused.
"""
import math

import numpy as np
import pytest
import torch

from gpu_helpers import dev, host
from oracle_bindings import f32_to_bf16
from test_gpu_decode import build_cache, check_out

pytestmark = pytest.mark.gpu

HQ, H, D, S = 32, 8, 128, 16


def make_case(oracle, seed, ctx_lens):
    rng = np.random.default_rng(seed)
    P = sum((c + S - 1) // S for c in ctx_lens) + 8
    kc, vc, sc, tables, signs, isl = build_cache(oracle, rng, ctx_lens, H, D, S, P)
    q = f32_to_bf16(rng.standard_normal((len(ctx_lens), HQ, D)).astype(np.float32))
    ctx = np.array(ctx_lens, np.int32)
    return dict(P=P, q=q, kc=kc, vc=vc, sc=sc, tables=tables, signs=signs, isl=isl, ctx=ctx,
                d=[dev(x) for x in (q, kc, vc, sc, tables, ctx, signs)])


def run_both(tq4, oracle, case, K, label):
    q, kc, vc, sc, tables, ctx, signs = case["d"]
    B = case["q"].shape[0]
    scale = 1.0 / math.sqrt(D)
    ws = tq4.decode_workspace(B, HQ, H, D, K)
    ref = tq4.paged_decode(q, kc, vc, sc, tables, ctx, signs, H, S, case["P"], workspace=ws,
                           num_splits=K, scale=scale, inv_sqrt_len=float(case["isl"]))
    out = torch.empty_like(q)
    print(f"noalloc call: {label} B={B} K={K}", flush=True)
    tq4.paged_decode_noalloc(q, kc, vc, sc, tables, ctx, signs, H, S, case["P"], out,
                             num_splits=K, scale=scale, inv_sqrt_len=float(case["isl"]))
    got = host(out)
    assert np.array_equal(got, host(ref)), f"{label}: differs from tq4_paged_decode"
    _, want = oracle.paged_decode(case["q"], case["kc"], case["vc"], case["sc"], case["tables"],
                                  case["ctx"], case["signs"], None, HQ, H, D, S, case["P"], K,
                                  np.float32(scale), case["isl"], 1, threads=16)
    for b in range(B):
        check_out(got[b], want[b], f"noalloc {label} seq {b}")
    return got


def test_noalloc_first_call_under_graph_capture(tq4, oracle):
    """The process's first no-allocation call is made while a HIP graph is
    being captured: it launches nothing of its own (no set-up fill enters the
    graph), and every replay matches the workspace entry bit for bit, with
    eager no-allocation calls and synchronisations between the replays. The
    scratch's timeout count stays zero; a reset, then a call, still agrees."""
    case = make_case(oracle, 4, [2048 + 5, 700])
    q, kc, vc, sc, tables, ctx, signs = case["d"]
    kw = dict(num_splits=8, inv_sqrt_len=float(case["isl"]))
    ws = tq4.decode_workspace(2, HQ, H, D, 8)
    ref = host(tq4.paged_decode(q, kc, vc, sc, tables, ctx, signs, H, S, case["P"], workspace=ws,
                                **kw)).copy()
    out = torch.empty_like(q)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    print("noalloc: first call inside a graph capture", flush=True)
    with torch.cuda.graph(g):
        tq4.paged_decode_noalloc(q, kc, vc, sc, tables, ctx, signs, H, S, case["P"], out, **kw)
    for i in range(3):
        out.zero_()
        g.replay()
        assert np.array_equal(host(out), ref), f"replay {i}"
        tq4.paged_decode_noalloc(q, kc, vc, sc, tables, ctx, signs, H, S, case["P"], out, **kw)
        assert np.array_equal(host(out), ref), f"eager call {i}"
    assert tq4.paged_decode_noalloc_poll_timeouts(2, H) == 0
    tq4.paged_decode_noalloc_reset()
    out.zero_()
    tq4.paged_decode_noalloc(q, kc, vc, sc, tables, ctx, signs, H, S, case["P"], out, **kw)
    assert np.array_equal(host(out), ref), "after a reset"


def test_noalloc_matches_workspace_entry_on_shrinking_calls(tq4, oracle):
    rng = np.random.default_rng(0xA110C)
    big = make_case(oracle, 1, [int(x) for x in rng.integers(200, 1500, 64)])
    small = make_case(oracle, 2, [900])
    # the persistent form (64 x 8 x 3 items > the resident slots), then a
    # smaller one-launch call, then the first again
    first = run_both(tq4, oracle, big, 3, "persistent")
    run_both(tq4, oracle, small, 4, "smaller")
    again = run_both(tq4, oracle, big, 3, "persistent again")
    assert np.array_equal(first, again)


def test_noalloc_in_hip_graph(tq4, oracle):
    case = make_case(oracle, 3, [4096, 1000])
    q, kc, vc, sc, tables, ctx, signs = case["d"]
    out = torch.empty_like(q)
    call = lambda: tq4.paged_decode_noalloc(q, kc, vc, sc, tables, ctx, signs, H, S,  # noqa: E731
                                            case["P"], out, num_splits=16,
                                            inv_sqrt_len=float(case["isl"]))
    call()
    eager = host(out).copy()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        call()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        call()
    for _ in range(3):
        out.zero_()
        g.replay()
        assert np.array_equal(host(out), eager)
        call()
        assert np.array_equal(host(out), eager)


def test_noalloc_refuses_beyond_scratch(tq4):
    """64 sequences x 32 q heads x 16 splits need about 17.3 MB of workspace:
    refused before any launch."""
    B = 64
    q = torch.zeros(B, HQ, D, dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros(8 * H * S * D // 2, dtype=torch.int8, device="cuda")
    sc = torch.zeros(2 * 8 * H * S, device="cuda")
    tb = torch.zeros(B, 512, dtype=torch.int32, device="cuda")
    ln = torch.zeros(B, dtype=torch.int32, device="cuda")
    sg = torch.ones(D, device="cuda")
    with pytest.raises(ValueError, match="static scratch"):
        tq4.paged_decode_noalloc(q, kc, kc, sc, tb, ln, sg, H, S, 8, torch.empty_like(q),
                                 num_splits=16)
