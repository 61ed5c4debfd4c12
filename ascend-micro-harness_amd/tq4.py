"""Host-side mirror of the reference's TQ4 operator interface over libtq4.so.

The functions keep the reference launchers' names, argument meaning and error
behaviour (a refused geometry raises ``ValueError``, the analogue of the
reference's ``std::invalid_argument``), and call straight through the C ABI in
include/tq4.h. PyTorch supplies device memory and the current HIP stream;
every byte of compute runs in the HIP kernels. There is no CPU fallback: if
libtq4.so is missing the first call raises.

Reference launchers mirrored (paths relative to the reference checkout):
  reshape_and_cache_a8    kernels/ops/turboquant/turboquant_reshape_and_cache_a8.cpp:1578-1627
  reshape_and_cache_bf16  kernels/ops/turboquant/turboquant_reshape_and_cache_bf16.cpp:1993-2059
  reshape_scatter         kernels/ops/turboquant/turboquant_reshape_scatter_aiv.cpp:760-773
  paged_decode_partials   kernels/ops/turboquant/turboquant_paged_decode_attention.cpp:1727-1766
  paged_decode            kernels/ops/turboquant/baseline/turboquant_paged_attention.cpp:773-793
  splitk_combine          tests/common/l2_atomic_oracle.hpp:156-176 (host merge in the reference)
  icdf_quantize           kernels/camodel/icdf_quantize.cpp:161-172
  lloydmax_quantize       kernels/camodel/lloydmax_quantize.cpp:96-99
  kv4fp8_decode           include/turboquant_fused_decode_opt.hpp:186-188 (launch_fused_decode_opt)
  kv4fp8_decode_raw_query include/turboquant_fused_decode_opt.hpp:192-194
  fused_decode_opt_launch tests/common/fused_decode_opt_fixture.hpp (Fixture::launch, launch_raw)
"""
from __future__ import annotations

import ctypes as C
import math
import os

import torch  # noqa: F401  (loads torch's HIP runtime first; libtq4 binds to it)

_HERE = os.path.dirname(os.path.abspath(__file__))
# TQ4_LIBRARY=libtq4_stamps.so selects the measurement build (bench.py --phases)
LIB_PATH = os.path.join(_HERE, os.environ.get("TQ4_LIBRARY", "libtq4.so"))

TQ4_DECODE_QUERY_ROTATED = 1
TQ4_DECODE_PRECISE = 2  # partials only: FP32 recurrence, BF16 q_rot (reference rig budgets)
TQ4_DECODE_TEST_POLL_BOUND = 1 << 30  # test hooks of the bounded wait (include/tq4.h)
TQ4_DECODE_TEST_WITHHOLD = 1 << 31
TQ4_KV4FP8_TEST_POLL_BOUND = 1 << 30
TQ4_KV4FP8_TEST_WITHHOLD = 1 << 31
TQ4_MAX_SPLITS = 256

_P = C.c_void_p
_U32 = C.c_uint32
_F32 = C.c_float
_I32 = C.c_int
_SZ = C.c_size_t

_lib = None


class TQ4Error(ValueError):
    """A refused launch: the C ABI returned a negative tq4_status."""

    def __init__(self, status, what):
        self.status = status
        super().__init__(f"{what}: {status_string(status)} (status {status})")


def lib():
    """The loaded libtq4.so; raises if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"libtq4.so not found at {LIB_PATH}: run __graft_entry__.build() "
            "(make -C ascend-micro-harness_amd/csrc)")
    L = C.CDLL(LIB_PATH)
    L.tq4_status_string.restype = C.c_char_p
    L.tq4_status_string.argtypes = [_I32]
    L.tq4_version.restype = _U32
    L.tq4_reshape_and_cache_a8.restype = _I32
    L.tq4_reshape_and_cache_a8.argtypes = [_P] * 9 + [_U32] * 6 + [_F32, C.c_bool]
    L.tq4_reshape_and_cache_bf16.restype = _I32
    L.tq4_reshape_and_cache_bf16.argtypes = [_P] * 9 + [_U32] * 6 + [_F32, C.c_bool]
    L.tq4_reshape_scatter.restype = _I32
    L.tq4_reshape_scatter.argtypes = [_P, _U32] + [_P] * 9 + [_U32] * 7 + [_F32]
    L.tq4_decode_workspace_bytes.restype = _SZ
    L.tq4_decode_workspace_bytes.argtypes = [_U32] * 5
    L.tq4_decode_auto_splits.restype = _U32
    L.tq4_decode_auto_splits.argtypes = [_U32] * 4
    L.tq4_decode_auto_splits_lens.restype = _U32
    L.tq4_decode_auto_splits_lens.argtypes = [_U32] * 4 + [_P]
    L.tq4_decode_workspace_init.restype = _I32
    L.tq4_decode_workspace_init.argtypes = [_P, _P, _SZ]
    L.tq4_decode_poll_timeouts.restype = _I32
    L.tq4_decode_poll_timeouts.argtypes = [_P, _P, _SZ, _U32, _U32, _P]
    L.tq4_kv4fp8_poll_timeouts.restype = _I32
    L.tq4_kv4fp8_poll_timeouts.argtypes = [_P, _P, _P, _P]
    L.tq4_paged_decode.restype = _I32
    L.tq4_paged_decode.argtypes = [_P] * 10 + [_SZ, _P] + [_U32] * 8 + [_F32, _F32, _U32, _U32]
    L.tq4_paged_decode_noalloc.restype = _I32
    L.tq4_paged_decode_noalloc.argtypes = [_P] * 10 + [_U32] * 8 + [_F32, _F32, _U32, _U32]
    L.tq4_paged_decode_noalloc_poll_timeouts.restype = _I32
    L.tq4_paged_decode_noalloc_poll_timeouts.argtypes = [_P, _U32, _U32, _P]
    L.tq4_paged_decode_noalloc_reset.restype = _I32
    L.tq4_paged_decode_noalloc_reset.argtypes = [_P]
    L.tq4_paged_decode_partials.restype = _I32
    L.tq4_paged_decode_partials.argtypes = [_P] * 9 + [_SZ] + [_U32] * 8 + [_F32, _F32, _U32]
    L.tq4_splitk_combine.restype = _I32
    L.tq4_splitk_combine.argtypes = [_P] * 5 + [_U32] * 4 + [_F32, _U32]
    L.tq4_rms_reshape_and_cache.restype = _I32
    L.tq4_rms_reshape_and_cache.argtypes = [_P, _I32, _U32] + [_P] * 8 + [_U32] * 6 + [_F32]
    L.tq4_rms_dequantize.restype = _I32
    L.tq4_rms_dequantize.argtypes = [_P, _P, _P, C.c_uint64]
    L.tq4_icdf_quantize.restype = _I32
    L.tq4_icdf_quantize.argtypes = [_P, _I32, _P, _P, _U32]
    L.tq4_lloydmax_quantize.restype = _I32
    L.tq4_lloydmax_quantize.argtypes = [_P] * 5 + [_U32] * 4
    L.tq4_kv4fp8_workspace_bytes.restype = C.c_uint64
    L.tq4_kv4fp8_workspace_bytes.argtypes = [_P]
    L.tq4_kv4fp8_decode.restype = _I32
    L.tq4_kv4fp8_decode.argtypes = [_P, _P, _P]
    L.tq4_kv4fp8_decode_raw_query.restype = _I32
    L.tq4_kv4fp8_decode_raw_query.argtypes = [_P, _P, _P]
    L.tq4_kv4fp8_workspace_init.restype = _I32
    L.tq4_kv4fp8_workspace_init.argtypes = [_P, _P, C.c_uint64]
    L.tq4_fp8_e4m3_round.restype = _I32
    L.tq4_fp8_e4m3_round.argtypes = [_P, _P, _P, C.c_uint64]
    _lib = L
    return L


def status_string(status):
    return lib().tq4_status_string(int(status)).decode()


def _ptr(t):
    if t is None:
        return None
    if not t.is_contiguous():
        raise ValueError("tensors handed to libtq4 must be contiguous")
    return _P(t.data_ptr())


def _stream(stream=None):
    s = torch.cuda.current_stream() if stream is None else stream
    return _P(s.cuda_stream)


def _check(status, what):
    if status != 0:
        raise TQ4Error(status, what)


def _dev(t, name):
    if t is not None and not t.is_cuda:
        raise ValueError(f"{name} must be a device tensor")


_CACHE_BYTES = (torch.int8, torch.uint8)


def _need(what, name, t, dtypes, numel=None, min_numel=None, ndim=None, optional=False):
    """Refuse (ValueError) a tensor whose dtype or size the kernels would
    misread: they take raw pointers, so a wrong element type or a short
    buffer is otherwise an out-of-bounds or garbage read."""
    if t is None:
        if optional:
            return
        raise ValueError(f"{what}: {name} is required")
    if t.dtype not in dtypes:
        names = " or ".join(str(d).replace("torch.", "") for d in dtypes)
        raise ValueError(f"{what}: {name} must be {names}, got {str(t.dtype).replace('torch.', '')}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"{what}: {name} must have {ndim} dimensions, got shape {tuple(t.shape)}")
    if numel is not None and t.numel() != numel:
        raise ValueError(f"{what}: {name} must hold {numel} elements, got {t.numel()}")
    if min_numel is not None and t.numel() < min_numel:
        raise ValueError(f"{what}: {name} must hold at least {min_numel} elements, "
                         f"got {t.numel()}")


def _check_cache(what, key_cache, value_cache, scale_cache, num_blocks, num_kv_heads,
                 block_size, head_size):
    rows = num_blocks * num_kv_heads * block_size
    _need(what, "key_cache", key_cache, _CACHE_BYTES, min_numel=rows * head_size // 2)
    _need(what, "value_cache", value_cache, _CACHE_BYTES, min_numel=rows * head_size // 2)
    _need(what, "scale_cache", scale_cache, (torch.float32,), min_numel=2 * rows)


# --------------------------------------------------------------- writers
def reshape_and_cache_a8(key, value, key_cache, value_cache, scale_cache, slot_mapping,
                         pi_signs=None, tables=None, num_blocks=None, block_size=16,
                         tokens_per_core=16, inv_sqrt_len=None, reuse_mode4_flags=True,
                         stream=None):
    """INT8 K/V [num_tokens][num_kv_heads][head_size] -> TQ4 cache, whole strips."""
    return _reshape_and_cache(lib().tq4_reshape_and_cache_a8, "reshape_and_cache_a8", torch.int8,
                              key, value, key_cache, value_cache, scale_cache, slot_mapping,
                              pi_signs, tables, num_blocks, block_size, tokens_per_core,
                              inv_sqrt_len, reuse_mode4_flags, stream)


def reshape_and_cache_bf16(key, value, key_cache, value_cache, scale_cache, slot_mapping,
                           pi_signs=None, tables=None, num_blocks=None, block_size=16,
                           tokens_per_core=16, inv_sqrt_len=None, reuse_mode4_flags=True,
                           stream=None):
    """BF16 K/V [num_tokens][num_kv_heads][head_size] -> TQ4 cache, whole strips."""
    return _reshape_and_cache(lib().tq4_reshape_and_cache_bf16, "reshape_and_cache_bf16",
                              torch.bfloat16, key, value, key_cache, value_cache, scale_cache,
                              slot_mapping, pi_signs, tables, num_blocks, block_size,
                              tokens_per_core, inv_sqrt_len, reuse_mode4_flags, stream)


def _reshape_and_cache(fn, what, dtype, key, value, key_cache, value_cache, scale_cache,
                       slot_mapping, pi_signs, tables, num_blocks, block_size, tokens_per_core,
                       inv_sqrt_len, reuse_mode4_flags, stream):
    if key.dtype != dtype or value.dtype != dtype:
        raise ValueError(f"{what}: key/value must be {dtype}")
    _need(what, "key", key, (dtype,), ndim=3)
    _need(what, "value", value, (dtype,), numel=key.numel())
    num_tokens, num_kv_heads, head_size = key.shape
    if num_blocks is None:
        num_blocks = key_cache.numel() * 2 // (num_kv_heads * block_size * head_size)
    _check_cache(what, key_cache, value_cache, scale_cache, num_blocks, num_kv_heads,
                 block_size, head_size)
    _need(what, "slot_mapping", slot_mapping, (torch.int32,), min_numel=num_tokens)
    _need(what, "pi_signs", pi_signs, (torch.float32,), min_numel=head_size, optional=True)
    # the rotation tables' first column: entry c*32 for channel c, INT8 for
    # the A8 writer, BF16 (+-1 bit patterns) for the BF16 writer
    tdt = (torch.int8, torch.uint8) if dtype == torch.int8 else (torch.bfloat16, torch.int16)
    _need(what, "tables", tables, tdt, min_numel=32 * head_size, optional=True)
    for name, t in (("key", key), ("value", value), ("key_cache", key_cache),
                    ("value_cache", value_cache), ("scale_cache", scale_cache),
                    ("slot_mapping", slot_mapping), ("pi_signs", pi_signs), ("tables", tables)):
        _dev(t, name)
    if inv_sqrt_len is None:
        inv_sqrt_len = 1.0 / math.sqrt(head_size)
    st = fn(_stream(stream), _ptr(key), _ptr(value), _ptr(key_cache), _ptr(value_cache),
            _ptr(scale_cache), _ptr(slot_mapping), _ptr(pi_signs), _ptr(tables), num_tokens,
            num_kv_heads, head_size, block_size, num_blocks, tokens_per_core, inv_sqrt_len,
            bool(reuse_mode4_flags))
    _check(st, what)


def reshape_scatter(key, value, key_cache, value_cache, scale_cache, slot_mapping, pi_signs,
                    cu_seqlens=None, launch_probe=None, num_requests=None, num_blocks=None,
                    block_size=16, item_begin=0, item_count=None, block_dim=0,
                    inv_sqrt_len=None, stream=None):
    """BF16 tokens at arbitrary slots; items are (request, kv_head)."""
    what = "reshape_scatter"
    _need(what, "key", key, (torch.bfloat16,), ndim=3)
    _need(what, "value", value, (torch.bfloat16,), numel=key.numel())
    num_tokens, num_kv_heads, head_size = key.shape
    if num_requests is None:
        num_requests = (cu_seqlens.numel() - 1) if cu_seqlens is not None else num_tokens
    if num_blocks is None:
        num_blocks = key_cache.numel() * 2 // (num_kv_heads * block_size * head_size)
    _check_cache(what, key_cache, value_cache, scale_cache, num_blocks, num_kv_heads,
                 block_size, head_size)
    _need(what, "slot_mapping", slot_mapping, (torch.int32,), min_numel=num_tokens)
    _need(what, "pi_signs", pi_signs, (torch.float32,), min_numel=head_size)
    _need(what, "cu_seqlens", cu_seqlens, (torch.int32,), min_numel=num_requests + 1,
          optional=True)
    if cu_seqlens is None and num_requests > num_tokens:
        raise ValueError(f"{what}: {num_requests} requests of one token each need "
                         f"{num_requests} tokens, got {num_tokens}")
    _need(what, "launch_probe", launch_probe, (torch.int32,), min_numel=32, optional=True)
    for name, t in (("key", key), ("value", value), ("key_cache", key_cache),
                    ("value_cache", value_cache), ("scale_cache", scale_cache),
                    ("slot_mapping", slot_mapping), ("pi_signs", pi_signs),
                    ("cu_seqlens", cu_seqlens), ("launch_probe", launch_probe)):
        _dev(t, name)
    if item_count is None:
        item_count = num_requests * num_kv_heads
    if inv_sqrt_len is None:
        inv_sqrt_len = 1.0 / math.sqrt(head_size)
    st = lib().tq4_reshape_scatter(
        _stream(stream), block_dim, _ptr(key), _ptr(value), _ptr(key_cache), _ptr(value_cache),
        _ptr(scale_cache), _ptr(slot_mapping), _ptr(pi_signs), _ptr(cu_seqlens),
        _ptr(launch_probe), num_requests, num_kv_heads, head_size, block_size, num_blocks,
        item_begin, item_count, inv_sqrt_len)
    _check(st, "reshape_scatter")


# ---------------------------------------------------------------- decode
def decode_workspace_bytes(num_seqs, num_heads, num_kv_heads, head_size, num_splits):
    return int(lib().tq4_decode_workspace_bytes(num_seqs, num_heads, num_kv_heads, head_size,
                                                num_splits))


def auto_splits(num_seqs, num_kv_heads, max_blocks_per_seq, block_size, context_lens=None):
    """The decode's split count (tq4_decode_auto_splits); with the context
    lengths on the host (a sequence of ints, not a device tensor), the
    length-aware rule (tq4_decode_auto_splits_lens)."""
    if context_lens is None:
        return int(lib().tq4_decode_auto_splits(num_seqs, num_kv_heads, max_blocks_per_seq,
                                                block_size))
    import numpy as np
    lens = np.ascontiguousarray(np.asarray(context_lens, dtype=np.int32))
    if lens.size != num_seqs:
        raise ValueError(f"auto_splits: {lens.size} context lengths for {num_seqs} sequences")
    return int(lib().tq4_decode_auto_splits_lens(num_seqs, num_kv_heads, max_blocks_per_seq,
                                                 block_size, lens.ctypes.data))


def decode_workspace_init(workspace, stream=None):
    """Zero a fused-decode workspace in stream order (tq4_decode_workspace_init):
    before its first use, and again after a reported poll timeout."""
    _dev(workspace, "workspace")
    _check(lib().tq4_decode_workspace_init(_stream(stream), _ptr(workspace),
                                           workspace.numel() * workspace.element_size()),
           "decode_workspace_init")
    return workspace


def decode_workspace(num_seqs, num_heads, num_kv_heads, head_size, num_splits=0, device="cuda",
                     stream=None):
    """A zero-initialised workspace (counters at zero) for tq4_paged_decode."""
    nbytes = decode_workspace_bytes(num_seqs, num_heads, num_kv_heads, head_size, num_splits)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    _check(lib().tq4_decode_workspace_init(_stream(stream), _ptr(ws), nbytes),
           "decode_workspace_init")
    return ws


def _check_decode_inputs(what, q, key_cache, value_cache, scale_cache, block_tables,
                         context_lens, pi_signs, num_kv_heads, block_size, num_blocks,
                         pi_needed=True):
    """The decode's operand contract (include/tq4.h): q BF16 [B][Hq][d];
    block_tables int32 [B][max_blocks]; context_lens int32 [B]; the caches as
    the writer leaves them; pi_signs FP32 [d]."""
    _need(what, "q", q, (torch.bfloat16,), ndim=3)
    B, Hq, d = q.shape
    _check_cache(what, key_cache, value_cache, scale_cache, num_blocks, num_kv_heads,
                 block_size, d)
    _need(what, "block_tables", block_tables, (torch.int32,), ndim=2)
    if block_tables.shape[0] != B:
        raise ValueError(f"{what}: block_tables must have {B} rows (one per sequence), "
                         f"got shape {tuple(block_tables.shape)}")
    _need(what, "context_lens", context_lens, (torch.int32,), numel=B)
    _need(what, "pi_signs", pi_signs, (torch.float32,), min_numel=d, optional=not pi_needed)


def _read_count(fn, what, stream):
    """Copy a 32-bit device count to pinned host memory in stream order, wait
    for the stream, return it."""
    host = torch.zeros(1, dtype=torch.int32, pin_memory=True)
    _check(fn(_P(host.data_ptr())), what)
    s = torch.cuda.current_stream() if stream is None else stream
    s.synchronize()
    return int(host[0]) & 0xFFFFFFFF


def decode_poll_timeouts(workspace, num_seqs, num_kv_heads, stream=None):
    """Rows whose fused-decode combiner gave up its bounded poll since the
    workspace was last zeroed (tq4_decode_poll_timeouts). Nonzero: those
    outputs are invalid and the workspace must be zeroed again. Synchronises
    the stream."""
    _dev(workspace, "workspace")
    nbytes = workspace.numel() * workspace.element_size()
    return _read_count(lambda dst: lib().tq4_decode_poll_timeouts(
        _stream(stream), _ptr(workspace), nbytes, num_seqs, num_kv_heads, dst),
        "decode_poll_timeouts", stream)


def paged_decode(q, key_cache, value_cache, scale_cache, block_tables, context_lens, pi_signs,
                 num_kv_heads, block_size, num_blocks, out=None, workspace=None, gate=None,
                 num_splits=0, scale=None, inv_sqrt_len=None, output_stage=1, flags=0,
                 stream=None):
    """Fused split-K decode: q [B][Hq][d] bf16 -> out [B][Hq][d] bf16."""
    _check_decode_inputs("paged_decode", q, key_cache, value_cache, scale_cache, block_tables,
                         context_lens, pi_signs, num_kv_heads, block_size, num_blocks,
                         pi_needed=output_stage >= 1 or not (flags & TQ4_DECODE_QUERY_ROTATED))
    _need("paged_decode", "gate", gate, (torch.float32,), numel=q.numel(), optional=True)
    _need("paged_decode", "out", out, (torch.bfloat16,), numel=q.numel(), optional=True)
    for name, t in (("q", q), ("key_cache", key_cache), ("value_cache", value_cache),
                    ("scale_cache", scale_cache), ("block_tables", block_tables),
                    ("context_lens", context_lens), ("pi_signs", pi_signs), ("gate", gate),
                    ("workspace", workspace), ("out", out)):
        _dev(t, name)
    B, Hq, d = q.shape
    if out is None:
        out = torch.empty_like(q)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if inv_sqrt_len is None:
        inv_sqrt_len = 1.0 / math.sqrt(d)
    max_blocks = block_tables.shape[1]
    if num_splits == 0:
        num_splits = auto_splits(B, num_kv_heads, max_blocks, block_size)
    if workspace is None and num_splits > 1:
        workspace = decode_workspace(B, Hq, num_kv_heads, d, num_splits, q.device, stream)
    ws_bytes = workspace.numel() * workspace.element_size() if workspace is not None else 0
    st = lib().tq4_paged_decode(
        _stream(stream), _ptr(q), _ptr(key_cache), _ptr(value_cache), _ptr(scale_cache),
        _ptr(block_tables), _ptr(context_lens), _ptr(pi_signs), _ptr(gate), _ptr(workspace),
        ws_bytes, _ptr(out), B, Hq, num_kv_heads, d, block_size, num_blocks, max_blocks,
        num_splits, scale, inv_sqrt_len, output_stage, flags)
    _check(st, "paged_decode")
    return out


def paged_decode_noalloc(q, key_cache, value_cache, scale_cache, block_tables, context_lens,
                         pi_signs, num_kv_heads, block_size, num_blocks, out, gate=None,
                         num_splits=0, scale=None, inv_sqrt_len=None, output_stage=1, flags=0,
                         stream=None):
    """paged_decode on the library's static 16 MiB scratch
    (tq4_paged_decode_noalloc): no workspace, nothing allocated -- `out` is
    required. Calls that overlap on one GPU race."""
    _check_decode_inputs("paged_decode_noalloc", q, key_cache, value_cache, scale_cache,
                         block_tables, context_lens, pi_signs, num_kv_heads, block_size,
                         num_blocks,
                         pi_needed=output_stage >= 1 or not (flags & TQ4_DECODE_QUERY_ROTATED))
    _need("paged_decode_noalloc", "gate", gate, (torch.float32,), numel=q.numel(), optional=True)
    _need("paged_decode_noalloc", "out", out, (torch.bfloat16,), numel=q.numel())
    for name, t in (("q", q), ("key_cache", key_cache), ("value_cache", value_cache),
                    ("scale_cache", scale_cache), ("block_tables", block_tables),
                    ("context_lens", context_lens), ("pi_signs", pi_signs), ("gate", gate),
                    ("out", out)):
        _dev(t, name)
    B, Hq, d = q.shape
    st = lib().tq4_paged_decode_noalloc(
        _stream(stream), _ptr(q), _ptr(key_cache), _ptr(value_cache), _ptr(scale_cache),
        _ptr(block_tables), _ptr(context_lens), _ptr(pi_signs), _ptr(gate), _ptr(out), B, Hq,
        num_kv_heads, d, block_size, num_blocks, block_tables.shape[1], num_splits,
        1.0 / math.sqrt(d) if scale is None else scale,
        1.0 / math.sqrt(d) if inv_sqrt_len is None else inv_sqrt_len, output_stage, flags)
    _check(st, "paged_decode_noalloc")
    return out


def paged_decode_noalloc_poll_timeouts(num_seqs, num_kv_heads, stream=None):
    """The no-allocation decode's sticky poll-timeout count for the geometry
    of its last call (tq4_paged_decode_noalloc_poll_timeouts). Nonzero: call
    paged_decode_noalloc_reset before the next no-allocation call.
    Synchronises the stream."""
    return _read_count(lambda dst: lib().tq4_paged_decode_noalloc_poll_timeouts(
        _stream(stream), num_seqs, num_kv_heads, dst), "paged_decode_noalloc_poll_timeouts",
        stream)


def paged_decode_noalloc_reset(stream=None):
    """Zero the no-allocation decode's static scratch on this device
    (tq4_paged_decode_noalloc_reset: one fill kernel, nothing allocated)."""
    _check(lib().tq4_paged_decode_noalloc_reset(_stream(stream)), "paged_decode_noalloc_reset")


def paged_decode_partials(q, key_cache, value_cache, scale_cache, block_tables, context_lens,
                          pi_signs, num_kv_heads, block_size, num_blocks, num_splits,
                          workspace=None, scale=None, inv_sqrt_len=None, flags=0, stream=None):
    """Partial records [B][Hq][K][d+4] = (m, l, 0, 0, acc[d]) per split."""
    _check_decode_inputs("paged_decode_partials", q, key_cache, value_cache, scale_cache,
                         block_tables, context_lens, pi_signs, num_kv_heads, block_size,
                         num_blocks, pi_needed=not (flags & TQ4_DECODE_QUERY_ROTATED))
    B, Hq, d = q.shape
    _need("paged_decode_partials", "workspace", workspace, (torch.float32,),
          min_numel=B * Hq * num_splits * (d + 4), optional=True)
    for name, t in (("q", q), ("key_cache", key_cache), ("value_cache", value_cache),
                    ("scale_cache", scale_cache), ("block_tables", block_tables),
                    ("context_lens", context_lens), ("pi_signs", pi_signs),
                    ("workspace", workspace)):
        _dev(t, name)
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    if inv_sqrt_len is None:
        inv_sqrt_len = 1.0 / math.sqrt(d)
    if workspace is None:
        workspace = torch.empty((B, Hq, num_splits, d + 4), dtype=torch.float32, device=q.device)
    ws_bytes = workspace.numel() * workspace.element_size()
    st = lib().tq4_paged_decode_partials(
        _stream(stream), _ptr(q), _ptr(key_cache), _ptr(value_cache), _ptr(scale_cache),
        _ptr(block_tables), _ptr(context_lens), _ptr(pi_signs), _ptr(workspace), ws_bytes, B,
        Hq, num_kv_heads, d, block_size, num_blocks, block_tables.shape[1], num_splits, scale,
        inv_sqrt_len, flags)
    _check(st, "paged_decode_partials")
    return workspace


def splitk_combine(workspace, pi_signs, num_seqs, num_heads, head_size, num_splits, out=None,
                   gate=None, inv_sqrt_len=None, output_stage=1, stream=None):
    """LSE combine + egress of partial records into BF16 [B][Hq][d]."""
    what = "splitk_combine"
    rows = num_seqs * num_heads
    _need(what, "workspace", workspace, (torch.float32,),
          min_numel=rows * num_splits * (head_size + 4))
    _need(what, "pi_signs", pi_signs, (torch.float32,), min_numel=head_size,
          optional=output_stage == 0)
    _need(what, "gate", gate, (torch.float32,), numel=rows * head_size, optional=True)
    _need(what, "out", out, (torch.bfloat16,), numel=rows * head_size, optional=True)
    for name, t in (("workspace", workspace), ("pi_signs", pi_signs), ("gate", gate),
                    ("out", out)):
        _dev(t, name)
    if out is None:
        out = torch.empty((num_seqs, num_heads, head_size), dtype=torch.bfloat16,
                          device=workspace.device)
    if inv_sqrt_len is None:
        inv_sqrt_len = 1.0 / math.sqrt(head_size)
    st = lib().tq4_splitk_combine(_stream(stream), _ptr(workspace), _ptr(pi_signs), _ptr(gate),
                                  _ptr(out), num_seqs, num_heads, head_size, num_splits,
                                  inv_sqrt_len, output_stage)
    _check(st, "splitk_combine")
    return out


# ------------------------------------------------------------ RMS codec
def rms_scale_slot_floats(num_kv_heads):
    """Floats per slot of the baseline cache's scale record: 2H rounded up to 8."""
    return (2 * num_kv_heads + 7) // 8 * 8


def rms_reshape_and_cache(key, value, key_cache, value_cache, scale_cache, slot_mapping,
                          pi_signs, num_blocks=None, block_size=16, inv_sqrt_len=None,
                          block_dim=0, tokens_per_core=0, tables=None, stream=None):
    """The vllm-ascend baseline writer (turboquant_reshape_and_cache_impl):
    FP16/BF16 K/V [tokens][kv_heads][head_size] -> int8 rows [slot][kv_heads]
    [head_size/2] and the scale record [slot][ceil(2 kv_heads / 8) * 8]."""
    what = "rms_reshape_and_cache"
    _need(what, "key", key, (torch.float16, torch.bfloat16), ndim=3)
    _need(what, "value", value, (key.dtype,), numel=key.numel())
    T, H, d = key.shape
    if num_blocks is None:
        num_blocks = key_cache.numel() // (block_size * H * (d // 2))
    slots = num_blocks * block_size
    _need(what, "key_cache", key_cache, _CACHE_BYTES, min_numel=slots * H * d // 2)
    _need(what, "value_cache", value_cache, _CACHE_BYTES, min_numel=slots * H * d // 2)
    _need(what, "scale_cache", scale_cache, (torch.float32,),
          min_numel=slots * rms_scale_slot_floats(H))
    _need(what, "slot_mapping", slot_mapping, (torch.int32,), min_numel=T)
    _need(what, "pi_signs", pi_signs, (torch.float32,), min_numel=d)
    for name, t in (("key", key), ("value", value), ("key_cache", key_cache),
                    ("value_cache", value_cache), ("scale_cache", scale_cache),
                    ("slot_mapping", slot_mapping), ("pi_signs", pi_signs), ("tables", tables)):
        _dev(t, name)
    if inv_sqrt_len is None:
        inv_sqrt_len = 1.0 / math.sqrt(d)
    st = lib().tq4_rms_reshape_and_cache(
        _stream(stream), 1 if key.dtype == torch.bfloat16 else 0, block_dim, _ptr(key),
        _ptr(value), _ptr(key_cache), _ptr(value_cache), _ptr(scale_cache), _ptr(slot_mapping),
        _ptr(pi_signs), _ptr(tables), T, H, d, block_size, num_blocks, tokens_per_core,
        inv_sqrt_len)
    _check(st, what)


def rms_dequantize(packed, out=None, stream=None):
    """Packed codes (int8, two per byte) -> their centroids (float32)."""
    _need("rms_dequantize", "packed", packed, _CACHE_BYTES)
    n = 2 * packed.numel()
    _need("rms_dequantize", "out", out, (torch.float32,), numel=n, optional=True)
    _dev(packed, "packed")
    _dev(out, "out")
    if out is None:
        out = torch.empty(n, dtype=torch.float32, device=packed.device)
    _check(lib().tq4_rms_dequantize(_stream(stream), _ptr(packed), _ptr(out), n),
           "rms_dequantize")
    return out


# ------------------------------------------------------------ codebooks
def icdf_quantize(x, out=None, stream=None):
    """FP16 or BF16 values (a multiple of 1024) -> packed signed INT4 codes of
    RNE(14 sigmoid(x) - 7), element 2j in the low nibble of byte j."""
    _dev(x, "x")
    if x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("icdf_quantize: x must be float16 or bfloat16")
    if x.numel() % 1024:
        raise ValueError("icdf_quantize: the element count must be a multiple of 1024")
    if out is None:
        out = torch.empty(x.numel() // 2, dtype=torch.uint8, device=x.device)
    st = lib().tq4_icdf_quantize(_stream(stream), 1 if x.dtype == torch.bfloat16 else 0,
                                 _ptr(x), _ptr(out), x.numel() // 1024)
    _check(st, "icdf_quantize")
    return out


def lloydmax_quantize(src, bits=4, mode=0, dst=None, codes=None, stream=None):
    """The Lloyd-Max leaf and its companions (mode as tq4_lloydmax_quantize):
    0/1 Lloyd-Max, 2 Gaussian-CDF compander, 3 ICDF (FP16 src), 4/5 decode of
    packed codes. Returns (dst, codes)."""
    _dev(src, "src")
    if mode >= 4:
        n = src.numel() * 8 // bits
    else:
        n = src.numel()
    if mode <= 2 and codes is None:
        codes = torch.empty(n * bits // 8, dtype=torch.uint8, device=src.device)
    if mode == 3 and codes is None:
        codes = torch.empty(n // 2, dtype=torch.uint8, device=src.device)
    if mode != 3 and dst is None:
        dst = torch.empty(n, dtype=torch.float32, device=src.device)
    st = lib().tq4_lloydmax_quantize(_stream(stream), _ptr(src), _ptr(dst), _ptr(codes), None,
                                     bits, mode, n, 1)
    _check(st, "lloydmax_quantize")
    return dst, codes


__all__ = [
    "TQ4Error", "lib", "status_string", "reshape_and_cache_a8", "reshape_and_cache_bf16",
    "reshape_scatter", "decode_workspace_bytes", "auto_splits", "decode_workspace",
    "paged_decode", "paged_decode_partials", "splitk_combine", "icdf_quantize",
    "decode_workspace_init", "paged_decode_noalloc", "paged_decode_noalloc_poll_timeouts",
    "paged_decode_noalloc_reset", "rms_reshape_and_cache", "rms_dequantize",
    "rms_scale_slot_floats",
    "lloydmax_quantize", "TQ4_DECODE_QUERY_ROTATED", "TQ4_MAX_SPLITS",
    "Kv4Fp8Launch", "Kv4Fp8Buffers", "Kv4Fp8RawQueryBuffers", "fused_decode_opt_launch",
    "kv4fp8_workspace_bytes", "kv4fp8_workspace_init", "kv4fp8_decode", "kv4fp8_decode_raw_query",
    "fp8_e4m3_round", "decode_poll_timeouts", "kv4fp8_poll_timeouts", "TQ4_DECODE_TEST_POLL_BOUND",
    "TQ4_DECODE_TEST_WITHHOLD", "TQ4_KV4FP8_TEST_POLL_BOUND", "TQ4_KV4FP8_TEST_WITHHOLD",
]


# ------------------------------------------------- KV4/FP8 NZ-tiled decode
class Kv4Fp8Launch(C.Structure):
    """tq4_kv4fp8_launch (include/tq4_kv4fp8.h): the reference's Launch fields
    (include/turboquant_fused_decode_opt.hpp:98-124) plus num_blocks and
    workspace_bytes."""
    _fields_ = [(n, _U32) for n in (
        "grid", "tokens", "heads", "kv_heads", "head_size", "block_size", "max_blocks", "splits",
        "heads_per_task", "tasks_per_block", "reduce_tasks_per_block", "fused_context_limit")] + \
        [("scale", _F32), ("inv_sqrt_len", _F32)] + \
        [(n, _U32) for n in ("prologue_vectors_per_block", "prologue_cube_chunk_vectors",
                             "output_stage", "element_type", "probe_page", "probe_tile",
                             "num_blocks")] + [("workspace_bytes", C.c_uint64),
                                               ("test_flags", _U32)]


class Kv4Fp8Buffers(C.Structure):
    _fields_ = [(n, _P) for n in ("query", "key", "value", "scales", "block_table",
                                  "context_lengths", "mode_tables", "workspace", "output",
                                  "tiling")]


class Kv4Fp8RawQueryBuffers(C.Structure):
    _fields_ = [(n, _P) for n in ("raw_query", "pi_signs", "rot_tables", "h16", "gate")] + \
        [("decode", Kv4Fp8Buffers)]


def fused_decode_opt_launch(tokens, heads, kv_heads, block_size, max_blocks, splits=1,
                            heads_per_task=16, fused_context_limit=4096, scale=0.0625,
                            inv_sqrt_len=0.0625, output_stage=0, element_type=0,
                            raw_query=False, num_blocks=0):
    """The Launch the reference's fixture builds (Fixture::launch / launch_raw):
    tasks spread over at most 32 blocks."""
    group = heads // kv_heads if kv_heads else 0
    chunk = min(heads_per_task, group) if group else 1
    tasks = tokens * kv_heads * splits * ((group + chunk - 1) // chunk if chunk else 0)
    tpb = max(1, (tasks + 31) // 32)
    grid = max(1, (tasks + tpb - 1) // tpb)
    L = Kv4Fp8Launch()
    L.grid, L.tokens, L.heads, L.kv_heads = grid, tokens, heads, kv_heads
    L.head_size, L.block_size, L.max_blocks, L.splits = 256, block_size, max_blocks, splits
    L.heads_per_task, L.tasks_per_block = heads_per_task, tpb
    L.reduce_tasks_per_block = max(1, (tokens * heads + grid - 1) // grid)
    L.fused_context_limit, L.scale, L.inv_sqrt_len = fused_context_limit, scale, inv_sqrt_len
    if raw_query:
        L.prologue_vectors_per_block = (tokens * heads + grid - 1) // grid
    L.output_stage, L.element_type = output_stage, element_type
    L.probe_page, L.probe_tile = 0xFFFFFFFF, 0
    L.num_blocks = num_blocks
    return L


def kv4fp8_workspace_bytes(launch):
    return int(lib().tq4_kv4fp8_workspace_bytes(C.byref(launch)))


def kv4fp8_poll_timeouts(workspace, tokens, heads, kv_heads, block_size, max_blocks,
                         num_blocks, stream=None):
    """Rows whose KV4/FP8 combiner gave up its bounded poll since the
    workspace was last zeroed (tq4_kv4fp8_poll_timeouts), for a workspace
    sized for this geometry. Synchronises the stream."""
    _dev(workspace, "workspace")
    L = fused_decode_opt_launch(tokens, heads, kv_heads, block_size, max_blocks,
                                num_blocks=num_blocks)
    L.workspace_bytes = workspace.numel() * workspace.element_size()
    return _read_count(lambda dst: lib().tq4_kv4fp8_poll_timeouts(
        _stream(stream), C.byref(L), _ptr(workspace), dst), "kv4fp8_poll_timeouts", stream)


def kv4fp8_workspace_init(workspace, stream=None):
    """Zero a KV4/FP8 decode workspace (tq4_kv4fp8_workspace_init): needed
    once before its first call; every call leaves it zero again."""
    _dev(workspace, "workspace")
    _check(lib().tq4_kv4fp8_workspace_init(_stream(stream), _ptr(workspace),
                                           workspace.numel() * workspace.element_size()),
           "kv4fp8_workspace_init")
    return workspace


def _kv4_check(what, q, key_cache, value_cache, scales, block_table, context_lens, kv_heads,
               block_size, num_blocks):
    """The KV4/FP8 operand contract (include/tq4_kv4fp8.h): NZ byte pools of
    num_blocks * block_size * kv_heads * 128 bytes, an eight-lane FP32 scale
    slot per row, int32 tables [T][max_blocks] and lengths [T]."""
    T = q.shape[0]
    rows = num_blocks * block_size
    _need(what, "key_cache", key_cache, _CACHE_BYTES, min_numel=rows * kv_heads * 128)
    _need(what, "value_cache", value_cache, _CACHE_BYTES, min_numel=rows * kv_heads * 128)
    _need(what, "scales", scales, (torch.float32,), min_numel=rows * 8)
    _need(what, "block_table", block_table, (torch.int32,), ndim=2)
    if block_table.shape[0] != T:
        raise ValueError(f"{what}: block_table must have {T} rows, got shape "
                         f"{tuple(block_table.shape)}")
    _need(what, "context_lens", context_lens, (torch.int32,), numel=T)


def _kv4_prepare(launch, tensors, workspace, device, stream):
    for name, t in tensors:
        _dev(t, name)
    need = kv4fp8_workspace_bytes(launch)
    if need == 0:
        raise ValueError("kv4fp8 decode: unsupported geometry")
    if workspace is None:  # a zeroed one for this call
        workspace = torch.zeros(need, dtype=torch.uint8, device=device)
    launch.workspace_bytes = workspace.numel() * workspace.element_size()
    return workspace


def kv4fp8_decode(query, key_cache, value_cache, scales, block_table, context_lens, kv_heads,
                  block_size, num_blocks, out=None, workspace=None, out_dtype=torch.float16,
                  splits=1, heads_per_task=16, fused_context_limit=4096, scale=None,
                  inv_sqrt_len=None, test_flags=0, stream=None):
    """The pre-rotated entry: query FP32 [T][Hq][256] -> out [T][Hq][256] (FP16/BF16).
    test_flags: the bounded wait's test hooks (TQ4_KV4FP8_TEST_*), 0 in use."""
    what = "kv4fp8_decode"
    _need(what, "query", query, (torch.float32,), ndim=3)
    _kv4_check(what, query, key_cache, value_cache, scales, block_table, context_lens,
               kv_heads, block_size, num_blocks)
    _need(what, "out", out, (torch.float16, torch.bfloat16), numel=query.numel(), optional=True)
    T, Hq, d = query.shape
    element = 1 if (out.dtype if out is not None else out_dtype) == torch.bfloat16 else 0
    if out is None:
        out = torch.empty((T, Hq, d), dtype=out_dtype, device=query.device)
    L = fused_decode_opt_launch(T, Hq, kv_heads, block_size, block_table.shape[1], splits,
                                heads_per_task, fused_context_limit,
                                1.0 / math.sqrt(d) if scale is None else scale,
                                1.0 / math.sqrt(d) if inv_sqrt_len is None else inv_sqrt_len,
                                0, element, False, num_blocks)
    L.test_flags = test_flags
    workspace = _kv4_prepare(L, (("query", query), ("key_cache", key_cache),
                                 ("value_cache", value_cache), ("scales", scales),
                                 ("block_table", block_table), ("context_lens", context_lens),
                                 ("out", out)), workspace, query.device, stream)
    B = Kv4Fp8Buffers(_ptr(query), _ptr(key_cache), _ptr(value_cache), _ptr(scales),
                      _ptr(block_table), _ptr(context_lens), None, _ptr(workspace), _ptr(out),
                      None)
    _check(lib().tq4_kv4fp8_decode(_stream(stream), C.byref(L), C.byref(B)), "kv4fp8_decode")
    return out


def kv4fp8_decode_raw_query(raw_query, pi_signs, key_cache, value_cache, scales, block_table,
                            context_lens, kv_heads, block_size, num_blocks, gate=None,
                            output_stage=1, query_out=None, out=None, workspace=None,
                            splits=1, heads_per_task=16, fused_context_limit=4096, scale=None,
                            inv_sqrt_len=None, stream=None):
    """The raw-query entry: raw_query FP16/BF16 [T][Hq][256] in the original
    basis -> out (same element type); query_out receives the rotated FP32 query."""
    what = "kv4fp8_decode_raw_query"
    _need(what, "raw_query", raw_query, (torch.float16, torch.bfloat16), ndim=3)
    _kv4_check(what, raw_query, key_cache, value_cache, scales, block_table, context_lens,
               kv_heads, block_size, num_blocks)
    _need(what, "pi_signs", pi_signs, (torch.float32,), min_numel=raw_query.shape[2])
    # the gate and the output share the raw query's element type
    _need(what, "gate", gate, (raw_query.dtype,), numel=raw_query.numel(), optional=True)
    _need(what, "out", out, (raw_query.dtype,), numel=raw_query.numel(), optional=True)
    _need(what, "query_out", query_out, (torch.float32,), numel=raw_query.numel(),
          optional=True)
    T, Hq, d = raw_query.shape
    element = 1 if raw_query.dtype == torch.bfloat16 else 0
    if out is None:
        out = torch.empty_like(raw_query)
    L = fused_decode_opt_launch(T, Hq, kv_heads, block_size, block_table.shape[1], splits,
                                heads_per_task, fused_context_limit,
                                1.0 / math.sqrt(d) if scale is None else scale,
                                1.0 / math.sqrt(d) if inv_sqrt_len is None else inv_sqrt_len,
                                output_stage, element, True, num_blocks)
    workspace = _kv4_prepare(L, (("raw_query", raw_query), ("pi_signs", pi_signs),
                                 ("key_cache", key_cache), ("value_cache", value_cache),
                                 ("scales", scales), ("block_table", block_table),
                                 ("context_lens", context_lens), ("gate", gate),
                                 ("query_out", query_out), ("out", out)),
                             workspace, raw_query.device, stream)
    D = Kv4Fp8Buffers(_ptr(query_out), _ptr(key_cache), _ptr(value_cache), _ptr(scales),
                      _ptr(block_table), _ptr(context_lens), None, _ptr(workspace), _ptr(out),
                      None)
    R = Kv4Fp8RawQueryBuffers(_ptr(raw_query), _ptr(pi_signs), None, None, _ptr(gate), D)
    _check(lib().tq4_kv4fp8_decode_raw_query(_stream(stream), C.byref(L), C.byref(R)),
           "kv4fp8_decode_raw_query")
    return out


def fp8_e4m3_round(x, stream=None):
    """FP32 -> the FP8 e4m3 operand grid (RNE), as FP16 values."""
    _dev(x, "x")
    out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    _check(lib().tq4_fp8_e4m3_round(_stream(stream), _ptr(x), _ptr(out), x.numel()),
           "fp8_e4m3_round")
    return out
