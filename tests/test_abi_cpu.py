"""The C ABI without a GPU: libtq4.so loads, exports every symbol include/*.h
declares, and refuses bad geometry before touching the HIP runtime (no compute
call is made here)."""
import ctypes as C
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(REPO, "include", h) for h in ("tq4.h", "tq4_kv4fp8.h")]
LIB = os.path.join(REPO, "ascend-micro-harness_amd", "libtq4.so")


def declared_functions():
    names = set()
    for h in HEADERS:
        text = re.sub(r"/\*.*?\*/", "", open(h).read(), flags=re.S)
        names |= set(re.findall(r"\b(tq4_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


@pytest.fixture(scope="module")
def lib(tq4):
    return tq4.lib()


def test_library_exports_every_declared_symbol(lib):
    names = declared_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/ but not exported"


def test_status_strings_and_version(lib):
    assert lib.tq4_status_string(0) == b"ok"
    for st in range(-12, 0):
        assert lib.tq4_status_string(st) != b"unknown status"
    assert lib.tq4_version() >> 16 == 1


def test_writer_refusals(lib):
    f = lib.tq4_reshape_and_cache_a8
    dummy = C.c_void_p(16)  # never dereferenced: every call below is refused first
    args = lambda T, H, d, S, P, tpc, signs=dummy: (None, dummy, dummy, dummy, dummy, dummy, dummy,  # noqa: E731
                                                    signs, None, T, H, d, S, P, tpc, 0.1, True)
    assert f(*args(16, 2, 96, 16, 4, 16)) == -2          # head_size
    assert f(*args(16, 0, 128, 16, 4, 16)) == -3         # no heads
    assert f(*args(16, 2, 128, 24, 4, 16)) == -3         # block_size % 16
    assert f(*args(17, 2, 128, 16, 4, 16)) == -4         # partial strip
    assert f(*args(32, 2, 128, 16, 4, 24)) == -4         # tokens_per_core % 16
    assert f(*args(16, 2, 128, 16, 4, 16, None)) == -8   # no rotation operand
    assert f(*args(0, 2, 128, 16, 4, 16)) == 0           # nothing to do
    assert f(*args(16, 65536, 128, 16, 4, 16)) == -10    # more heads than the grid's y
    g = lib.tq4_reshape_and_cache_bf16
    assert g(None, None, dummy, dummy, dummy, dummy, dummy, dummy, None, 16, 2, 128, 16, 4, 16,
             0.1, True) == -1                            # NULL key


def test_decode_refusals_and_sizes(lib):
    d = C.c_void_p(16)
    dec = lib.tq4_paged_decode

    def call(Hq=32, Hkv=8, hd=128, S=16, K=4, ws=None, wsb=0, stage=1, gate=None, maxb=256):
        return dec(None, d, d, d, d, d, d, d, gate, ws, wsb, d, 1, Hq, Hkv, hd, S, 4096, maxb, K,
                   0.1, 0.1, stage, 0)

    assert call(hd=96) == -2
    assert call(Hq=34) == -3                 # GQA group not integral
    assert call(Hq=8 * 17) == -3             # GQA group > 16
    assert call(S=8) == -3
    assert call(K=300) == -5
    assert call(K=1, maxb=4096) == -5        # a split may walk at most 2048 strips
    assert call(K=4) == -6                   # no workspace
    assert call(K=4, ws=d, wsb=100) == -6    # too small
    assert call(K=1, stage=3) == -7
    assert call(K=1, stage=2) == -7          # stage 2 needs a gate
    need = lib.tq4_decode_workspace_bytes(1, 32, 8, 128, 4)
    assert need >= 1 * 32 * 4 * (128 + 4) * 4 + 8 * 4
    k = lib.tq4_decode_auto_splits(1, 8, 256, 16)
    assert 1 <= k <= 256 and (256 + k - 1) // k <= 2048
    assert lib.tq4_decode_auto_splits(1, 1, 8192, 16) >= 4   # 8192 strips need >= 4 splits
    comb = lib.tq4_splitk_combine
    assert comb(None, d, d, None, d, 1, 32, 128, 0, 0.1, 1) == -5
    assert comb(None, d, d, None, d, 1, 32, 128, 4, 0.1, 2) == -7


def test_auto_splits_operating_points(lib):
    """The split counts the rule was measured at (32q:8kv, d 128, page 16):
    one sequence K = 16 up to ctx 8192 and 32 from 12288 (one workgroup per
    CU once each split keeps 20 strips past one 16-split record chunk); two
    and four sequences one workgroup per CU (16 strips per split suffice
    within one chunk); a 64-sequence batch one split per (seq, kv head)."""
    f = lib.tq4_decode_auto_splits
    pages = lambda ctx: (ctx + 15) // 16
    want = {(1, 2048): 8, (1, 4096): 16, (1, 4103): 16, (1, 8192): 16, (1, 12288): 32,
            (1, 16384): 32, (1, 32768): 32, (1, 65536): 32, (2, 4096): 16, (2, 8192): 16,
            (4, 4096): 8, (4, 8192): 8, (64, 8192): 1}
    got = {k: f(k[0], 8, pages(k[1]), 16) for k in want}
    assert got == want
    # the grid of one launch stays within one workgroup per CU at these points
    for (b, ctx), k in want.items():
        if b <= 4:
            assert b * 8 * k <= 256


def test_scatter_refusals(lib):
    d = C.c_void_p(16)
    f = lib.tq4_reshape_scatter
    assert f(None, 0, d, d, d, d, d, d, d, None, None, 1, 2, 48, 16, 4, 0, 2, 0.1) == -2
    assert f(None, 0, d, d, d, d, d, d, None, None, None, 1, 2, 128, 16, 4, 0, 2, 0.1) == -1
    assert f(None, 0, d, d, d, d, d, d, d, None, None, 1, 2, 128, 16, 4, 0, 0, 0.1) == 0


def test_codebook_refusals(lib):
    d = C.c_void_p(16)
    f = lib.tq4_lloydmax_quantize
    f.argtypes = [C.c_void_p] * 5 + [C.c_uint32] * 4
    assert f(None, d, d, d, None, 3, 0, 128, 1) == -11   # bits
    assert f(None, d, d, d, None, 4, 6, 128, 1) == -11   # mode
    assert f(None, d, d, d, None, 4, 0, 12, 1) == -11    # not a multiple of 8
    assert f(None, d, d, d, None, 2, 3, 128, 1) == -11   # ICDF is 4-bit only
    assert f(None, None, d, d, None, 4, 0, 128, 1) == -1
    assert f(None, d, d, None, None, 4, 2, 128, 1) == -1  # codes needed
    assert f(None, d, None, d, None, 4, 4, 128, 1) == -1  # decode needs dst
    assert f(None, d, d, d, None, 4, 0, 0, 1) == 0        # nothing to do
    g = lib.tq4_icdf_quantize
    g.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_void_p, C.c_uint32]
    assert g(None, 0, None, d, 1) == -1
    assert g(None, 1, d, d, 0) == 0



def test_kv4fp8_refusals_and_workspace(tq4, lib):
    """The KV4/FP8 entry points: valid_launch's refusals (before any HIP call)
    and the workspace size."""
    d = C.c_void_p(4096)
    L = lambda **kw: tq4.fused_decode_opt_launch(**{**dict(  # noqa: E731
        tokens=1, heads=16, kv_heads=1, block_size=64, max_blocks=17, splits=3,
        num_blocks=36), **kw})
    ok = L()
    need = tq4.kv4fp8_workspace_bytes(ok)
    assert need > 0 and need % 256 == 0
    bufs = tq4.Kv4Fp8Buffers(d, d, d, d, d, d, None, d, d, None)
    dec = lambda launch, b=bufs: lib.tq4_kv4fp8_decode(None, C.byref(launch), C.byref(b))  # noqa: E731
    ok.workspace_bytes = need - 256
    assert dec(ok) == -6                                   # workspace too small
    bad = L()
    bad.head_size = 128
    assert dec(bad) == -2                                  # D = 256 only
    for kw in (dict(kv_heads=5, heads=20), dict(heads=18, kv_heads=4), dict(block_size=96),
               dict(block_size=192), dict(max_blocks=0), dict(num_blocks=0)):
        x = L(**kw)
        x.workspace_bytes = 1 << 30
        assert dec(x) == -3, kw
        assert tq4.kv4fp8_workspace_bytes(x) == 0
    for k in (0, 9):
        x = L(splits=k)
        x.workspace_bytes = 1 << 30
        assert dec(x) == -5
    x = L()
    x.workspace_bytes = 1 << 30
    x.grid = 1
    x.tasks_per_block = 1                                  # tasks not covered
    assert dec(x) == -3
    x = L()
    x.workspace_bytes = 1 << 30
    x.element_type = 2
    assert dec(x) == -3
    nb = tq4.Kv4Fp8Buffers(None, d, d, d, d, d, None, d, d, None)
    x = L()
    x.workspace_bytes = 1 << 30
    assert dec(x, nb) == -1                                # no query
    raw = lambda launch, g=d: lib.tq4_kv4fp8_decode_raw_query(  # noqa: E731
        None, C.byref(launch), C.byref(tq4.Kv4Fp8RawQueryBuffers(d, d, None, None, g, bufs)))
    x = tq4.fused_decode_opt_launch(1, 16, 1, 64, 17, 3, num_blocks=36, raw_query=True,
                                    output_stage=3)
    x.workspace_bytes = 1 << 30
    assert raw(x) == -7                                    # stage
    x.output_stage = 2
    assert raw(x, None) == -7                              # gated without a gate
    x.output_stage = 1
    x.prologue_cube_chunk_vectors = 8
    assert raw(x) == -3                                    # Cube chunk 0 or 16
    x.prologue_cube_chunk_vectors = 16
    x.prologue_vectors_per_block = 0
    assert raw(x) == -3                                    # prologue share
    assert lib.tq4_fp8_e4m3_round(None, d, d, 3) == -10   # odd count


def test_flag_and_timeout_refusals(lib):
    """Unknown decode flags, the withhold hook without its poll bound, and a
    timeout read of a missing or too small workspace are refused before any
    HIP call."""
    d = C.c_void_p(16)
    dec = lib.tq4_paged_decode
    ws = 1 << 20

    def call(flags):
        return dec(None, d, d, d, d, d, d, d, None, d, ws, d, 1, 8, 2, 128, 16, 64, 4, 2,
                   C.c_float(0.1), C.c_float(0.1), 1, flags)
    assert call(1 << 5) == -12
    assert call(1 << 31) == -12                      # withhold without the bound
    assert call(2) == -12                            # TQ4_DECODE_PRECISE: partials only
    part = lib.tq4_paged_decode_partials
    assert part(None, d, d, d, d, d, d, d, d, ws, 1, 8, 2, 128, 16, 64, 4, 2, C.c_float(0.1),
                C.c_float(0.1), 1 << 30) == -12       # partials: no poll, no hook
    cnt = C.c_uint32(0)
    to = lib.tq4_decode_poll_timeouts
    assert to(None, None, ws, 1, 2, C.byref(cnt)) == -1
    assert to(None, d, ws, 1, 2, None) == -1
    assert to(None, d, 100, 1, 2, C.byref(cnt)) == -6  # smaller than the tail
    assert to(None, d, ws, 0, 2, C.byref(cnt)) == -6


def test_noalloc_refusals_before_any_hip_call(lib):
    """The no-allocation entry refuses a call beyond its static scratch, and
    the test hooks, before touching the device."""
    d = C.c_void_p(16)
    na = lib.tq4_paged_decode_noalloc

    def call(B, K, flags=0):
        return na(None, d, d, d, d, d, d, d, None, d, B, 32, 8, 128, 16, 4096, 512, K,
                  C.c_float(0.1), C.c_float(0.1), 1, flags)
    assert call(64, 16) == -13                       # 17.3 MB of workspace > 16 MiB
    assert call(1, 4, 1 << 30) == -12                # no test hooks
    assert call(1, 4, 2) == -12                      # nor the partials' precise mode
    assert call(1, 300) == -5                        # splits
    assert lib.tq4_status_string(-13) != b"unknown status"
    cnt = C.c_uint32(0)
    to = lib.tq4_paged_decode_noalloc_poll_timeouts
    assert to(None, 1, 8, None) == -1                   # no count pointer
    assert to(None, 0, 8, C.byref(cnt)) == -3           # no sequences
    assert to(None, 1 << 20, 8, C.byref(cnt)) == -13    # a tail beyond the scratch


def test_auto_splits_lens_rule(lib):
    """The length-aware split rule is a host function: NULL lengths give the
    plain rule; a ragged batch (longest >= 1.6 x mean) of 256..768 (seq, kv
    head) items takes at least 3 splits; uniform, mildly ragged and larger
    batches keep the plain rule."""
    import numpy as np
    f = lib.tq4_decode_auto_splits_lens
    f.restype = C.c_uint32
    f.argtypes = [C.c_uint32] * 4 + [C.c_void_p]
    plain = lib.tq4_decode_auto_splits
    plain.restype = C.c_uint32

    def lens(a):
        a = np.ascontiguousarray(np.asarray(a, np.int32))
        return a, a.ctypes.data
    r = np.random.default_rng(0x71340005)
    ragged, p = lens(r.integers(512, 8193, 64) + 1)
    assert f(64, 8, 513, 16, None) == plain(64, 8, 513, 16) == 2
    assert f(64, 8, 513, 16, p) == 3                       # configs[4]
    uni, pu = lens([8192] * 64)
    assert f(64, 8, 512, 16, pu) == plain(64, 8, 512, 16)  # uniform
    mild, pm = lens(np.random.default_rng(7).integers(2048, 8193, 64))
    assert f(64, 8, 513, 16, pm) == plain(64, 8, 513, 16)  # max/mean 1.53
    big, pb = lens(np.random.default_rng(7).integers(512, 8193, 128))
    assert f(128, 8, 513, 16, pb) == plain(128, 8, 513, 16)  # 1024 items
    small, ps = lens([4096] + [16] * 15)
    assert f(16, 8, 256, 16, ps) == plain(16, 8, 256, 16)  # 128 items
    wide, pw = lens(np.random.default_rng(3).integers(1, 32769, 64))
    assert f(64, 8, 2048, 16, pw) == max(3, plain(64, 8, 2048, 16)) == 4


def test_floor_library_refuses_other_geometry():
    """libtq4_floor.so (bench.py --floor's compute-free copies) loads, exports
    its launchers, and refuses any geometry but the measured rows' before it
    launches anything."""
    path = os.path.join(REPO, "ascend-micro-harness_amd", "libtq4_floor.so")
    if not os.path.exists(path):
        pytest.skip("libtq4_floor.so is not built (make -C ascend-micro-harness_amd/csrc floor)")
    fl = C.CDLL(path)
    for fn in (fl.tq4_floor_decode_launch, fl.tq4_floor_writer_launch,
               fl.tq4_floor_scatter_launch):
        fn.argtypes = [C.c_void_p, C.c_void_p]
        fn.restype = C.c_int

    class FloorDecode(C.Structure):
        _fields_ = [(f"p{i}", C.c_void_p) for i in range(10)] + \
            [(n, C.c_uint32) for n in ("B", "Hq", "Hkv", "G", "S", "P", "max_blocks", "K", "mode")]

    class FloorWriter(C.Structure):
        _fields_ = [(f"p{i}", C.c_void_p) for i in range(6)] + \
            [(n, C.c_uint32) for n in ("H", "D", "S", "P", "tokens", "mode")]

    assert fl.tq4_floor_decode_launch(None, None) == -1
    d = FloorDecode(B=1, Hq=32, Hkv=8, G=4, S=16, P=32768, max_blocks=256, K=16, mode=0)
    for field, bad in (("G", 8), ("S", 32), ("K", 8), ("max_blocks", 128), ("mode", 4),
                       ("Hq", 16)):
        e = FloorDecode.from_buffer_copy(d)
        setattr(e, field, bad)
        assert fl.tq4_floor_decode_launch(None, C.addressof(e)) == -1, field
    wp = FloorWriter(H=8, D=128, S=16, P=4096, tokens=1024, mode=0)
    for field, bad in (("D", 64), ("S", 32), ("tokens", 1000), ("mode", 2)):
        e = FloorWriter.from_buffer_copy(wp)
        setattr(e, field, bad)
        assert fl.tq4_floor_writer_launch(None, C.addressof(e)) == -1, field
    # the token scatter's copy shares the writer's argument block
    sp = FloorWriter(H=8, D=128, S=16, P=4096, tokens=1024, mode=0)
    for field, bad in (("D", 256), ("S", 64), ("tokens", 0), ("mode", 2)):
        e = FloorWriter.from_buffer_copy(sp)
        setattr(e, field, bad)
        assert fl.tq4_floor_scatter_launch(None, C.addressof(e)) == -1, field
    assert fl.tq4_floor_scatter_launch(None, None) == -1
