"""ctypes bindings of the test-infrastructure oracles.

``Oracle`` wraps oracle/libtq4_oracle.so (the C restatement of the reference's
CPU path). ``Ref`` wraps oracle/_ref/libtq4_ref.so, the reference's own
header-only oracles compiled in place, when it was built (it needs the
reference checkout, so it exists only where that is mounted).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module; the product path never does.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(REPO, "oracle", "libtq4_oracle.so")
REF_SO = os.path.join(REPO, "oracle", "_ref", "libtq4_ref.so")

P = C.c_void_p
U32 = C.c_uint32
I32 = C.c_int
F32 = C.c_float
I64 = C.c_int64
U64 = C.c_uint64

IN_INT8 = 0
IN_BF16 = 1
POLICY_PREFILL = 0
POLICY_EXACT = 1
FLAG_QUERY_ROTATED = 1
FLAG_QROT_BF16 = 2  # oracle: round Pi q to BF16 before the score (the reference device operand)
FLAG_PRECISE = 2  # device partials: TQ4_DECODE_PRECISE


def ptr(a):
    """Data pointer of a contiguous numpy array (None passes NULL)."""
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays handed to C must be contiguous"
    return C.c_void_p(a.ctypes.data)


def f32_to_bf16(x):
    """RNE float32 -> bfloat16 bits (numpy), quiet NaN kept, as tq4o_f32_to_bf16."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = ((b & 0x7F800000) == 0x7F800000) & ((b & 0x7FFFFF) != 0)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)
    r = np.where(nan, ((b >> 16) | 0x40).astype(np.uint16), r)
    return r.astype(np.uint16)


def bf16_to_f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


class Kv4Geom(C.Structure):
    """tq4o_kv4fp8_geom (oracle/kv4fp8_oracle.h)."""
    _fields_ = [(n, U32) for n in ("tokens", "heads", "kv_heads", "head_size", "block_size",
                                   "max_blocks", "num_blocks", "splits", "fused_context_limit")] + \
        [("scale", F32), ("inv_sqrt_len", F32), ("output_stage", U32), ("element_type", U32)]


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise RuntimeError(f"oracle library missing: {path} (run make -C oracle)")
        L = self.lib = C.CDLL(path)
        L.tq4o_key_nibble.restype = U64
        L.tq4o_key_nibble.argtypes = [U32] * 7
        L.tq4o_value_nibble.restype = U64
        L.tq4o_value_nibble.argtypes = [U32] * 7
        L.tq4o_scale_index.restype = U64
        L.tq4o_scale_index.argtypes = [U32] * 7
        L.tq4o_pi_sign.restype = I32
        L.tq4o_pi_sign.argtypes = [I32]
        L.tq4o_canonical_signs.argtypes = [U32, P]
        L.tq4o_build_tables_i8.argtypes = [U32, P, P]
        L.tq4o_signs_from_tables_i8.restype = I32
        L.tq4o_signs_from_tables_i8.argtypes = [U32, P, P]
        L.tq4o_rotate_ingress.argtypes = [P, P, U32, P]
        L.tq4o_rotate_egress.argtypes = [P, P, U32, P]
        L.tq4o_rotate_dense.argtypes = [P, P, U32, I32, P]
        L.tq4o_quantise_row.argtypes = [P, U32, F32, I32, P, P]
        L.tq4o_reshape_and_cache.restype = I64
        L.tq4o_reshape_and_cache.argtypes = [I32, P, P, P, P, P, P, P, U32, U32, U32, U32, U32, F32, I32]
        L.tq4o_reshape_and_cache_mt.restype = I64
        L.tq4o_reshape_and_cache_mt.argtypes = [I32, P, P, P, P, P, P, P, U32, U32, U32, U32, U32, F32, I32, U32]
        L.tq4o_reshape_scatter.restype = I64
        L.tq4o_reshape_scatter.argtypes = [P, P, P, P, P, P, P, P, U32, U32, U32, U32, U32, U32, U32, F32]
        L.tq4o_partition.argtypes = [U32, U32, U32, P, P]
        L.tq4o_active_in_strip.restype = U32
        L.tq4o_active_in_strip.argtypes = [U64, U32]
        L.tq4o_rotate_query.argtypes = [P, P, U32, F32, F32, P]
        L.tq4o_combine_step.argtypes = [P, P, P, F32, F32, P, U32]
        L.tq4o_decode_partials.restype = I32
        L.tq4o_decode_partials.argtypes = [P] * 8 + [U32] * 8 + [F32, F32, U32]
        L.tq4o_combine.restype = I32
        L.tq4o_combine.argtypes = [P, P, P, P, P, U32, U32, U32, U32, F32, U32]
        L.tq4o_paged_decode.restype = I32
        L.tq4o_paged_decode.argtypes = [P] * 10 + [U32] * 8 + [F32, F32, U32, U32, U32]
        L.tq4o_decode_reference_f64.restype = I32
        L.tq4o_decode_reference_f64.argtypes = [P] * 9 + [U32] * 7 + [F32, F32, U32, U32]
        L.tq4o_record_floats.restype = U32
        L.tq4o_record_floats.argtypes = [U32]
        L.tq4o_f32_to_bf16.restype = C.c_uint16
        L.tq4o_f32_to_bf16.argtypes = [F32]
        L.tq4o_codebook_centroid.restype = F32
        L.tq4o_codebook_centroid.argtypes = [U32, U32, U32]
        L.tq4o_lloydmax_threshold.restype = F32
        L.tq4o_lloydmax_threshold.argtypes = [U32, U32]
        L.tq4o_lloydmax_code.restype = U32
        L.tq4o_lloydmax_code.argtypes = [U32, F32]
        L.tq4o_gaussian_cdf_code.restype = U32
        L.tq4o_gaussian_cdf_code.argtypes = [U32, F32]
        L.tq4o_codebook_pack.argtypes = [P, U64, U32, P]
        L.tq4o_codebook_quantize.restype = I32
        L.tq4o_codebook_quantize.argtypes = [U32, U32, P, U64, P, P]
        L.tq4o_codebook_dequantize.restype = I32
        L.tq4o_codebook_dequantize.argtypes = [U32, U32, P, U64, P]
        L.tq4o_f16_to_f32.restype = F32
        L.tq4o_f16_to_f32.argtypes = [C.c_uint16]
        L.tq4o_icdf_code.restype = I32
        L.tq4o_icdf_code.argtypes = [C.c_double]
        L.tq4o_icdf_quantize.restype = I32
        L.tq4o_icdf_quantize.argtypes = [I32, P, U64, P]
        L.tq4o_nz_byte.restype = U64
        L.tq4o_nz_byte.argtypes = [U64] * 5
        L.tq4o_fp8_e4m3_encode.restype = C.c_uint8
        L.tq4o_fp8_e4m3_encode.argtypes = [F32]
        L.tq4o_fp8_e4m3_decode.restype = F32
        L.tq4o_fp8_e4m3_decode.argtypes = [C.c_uint8]
        L.tq4o_f32_to_f16.restype = C.c_uint16
        L.tq4o_f32_to_f16.argtypes = [F32]
        L.tq4o_elem_to_f32.restype = F32
        L.tq4o_elem_to_f32.argtypes = [U32, C.c_uint16]
        L.tq4o_f32_to_elem.restype = C.c_uint16
        L.tq4o_f32_to_elem.argtypes = [U32, F32]
        L.tq4o_kv4fp8_apply_pi.argtypes = [P, P, F32, U32]
        L.tq4o_rms_threshold.restype = F32
        L.tq4o_rms_threshold.argtypes = [U32]
        L.tq4o_rms_centroid.restype = F32
        L.tq4o_rms_centroid.argtypes = [U32]
        L.tq4o_rms_apply_pi.argtypes = [P, P, F32, U32]
        L.tq4o_rms_scale.restype = F32
        L.tq4o_rms_scale.argtypes = [P, U32, F32]
        L.tq4o_rms_level.restype = U32
        L.tq4o_rms_level.argtypes = [F32, F32]
        L.tq4o_rms_quantize_row.argtypes = [P, P, U32, F32, P, P, P]
        L.tq4o_rms_scale_slot_floats.restype = U32
        L.tq4o_rms_scale_slot_floats.argtypes = [U32]
        L.tq4o_rms_reshape_and_cache.restype = C.c_int64
        L.tq4o_rms_reshape_and_cache.argtypes = [I32] + [P] * 7 + [U32] * 6 + [F32]
        L.tq4o_rms_dequantize.argtypes = [P, U64, P]
        L.tq4o_kv4fp8_rotate_query.argtypes = [U32, P, P, F32, U64, U32, P]
        L.tq4o_kv4fp8_partial_floats.restype = U32
        L.tq4o_kv4fp8_partial_floats.argtypes = [U32]
        L.tq4o_kv4fp8_decode.restype = I32
        L.tq4o_kv4fp8_decode.argtypes = [P] * 12 + [I32]

    # ------------------------------------------------------------ KV4/FP8
    def kv4fp8_decode(self, query, key, value, scales, table, lengths, *, heads, kv_heads,
                      block_size, max_blocks, num_blocks, splits=1, fused_context_limit=0,
                      scale=0.0625, inv_sqrt_len=0.0625, output_stage=0, element_type=0,
                      pi_signs=None, gate=None, want_partials=False, threads=8):
        """Output element bits [tokens, heads, 256], the FP32 rows before the
        cast, and (want_partials) the split partials [tokens, heads, splits, 272]."""
        tokens = int(np.asarray(lengths).size)
        g = Kv4Geom(tokens, heads, kv_heads, 256, block_size, max_blocks, num_blocks, splits,
                    fused_context_limit, scale, inv_sqrt_len, output_stage, element_type)
        out = np.zeros((tokens, heads, 256), np.uint16)
        out_f32 = np.zeros((tokens, heads, 256), np.float32)
        ws = np.zeros((tokens, heads, splits, 272), np.float32) if want_partials else None
        a = [np.ascontiguousarray(x) if x is not None else None
             for x in (query, key, value, scales, table, lengths, pi_signs, gate)]
        st = self.lib.tq4o_kv4fp8_decode(C.byref(g), *[ptr(x) for x in a], ptr(ws), ptr(out),
                                         ptr(out_f32), threads)
        if st != 0:
            raise ValueError(f"tq4o_kv4fp8_decode refused: {st}")
        return (out, out_f32, ws) if want_partials else (out, out_f32)

    def kv4fp8_rotate_query(self, raw_bits, signs, inv_sqrt_len, element_type):
        raw = np.ascontiguousarray(raw_bits, np.uint16)
        out = np.zeros(raw.shape, np.float32)
        n = raw.shape[-1]
        self.lib.tq4o_kv4fp8_rotate_query(element_type, ptr(raw),
                                          ptr(np.ascontiguousarray(signs, np.float32)),
                                          inv_sqrt_len, raw.size // n, n, ptr(out))
        return out

    def fp8_round(self, x):
        x = np.asarray(x, np.float32).reshape(-1)
        return np.array([self.lib.tq4o_fp8_e4m3_decode(self.lib.tq4o_fp8_e4m3_encode(float(v)))
                         for v in x], np.float32)

    # ------------------------------------------------------------ codebooks
    def codebook_quantize(self, book, bits, x):
        """(recon float32[n], packed uint8[n*bits/8]) of the Lloyd-Max (book 0)
        or Gaussian-CDF (book 1) leaf."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        recon = np.zeros_like(x)
        packed = np.zeros(x.size * bits // 8, np.uint8)
        assert self.lib.tq4o_codebook_quantize(book, bits, ptr(x), x.size, ptr(recon),
                                               ptr(packed)) == 0
        return recon, packed

    def codebook_codes(self, book, bits, x):
        fn = self.lib.tq4o_lloydmax_code if book == 0 else self.lib.tq4o_gaussian_cdf_code
        return np.array([fn(bits, float(v)) for v in np.asarray(x, np.float32).reshape(-1)],
                        np.uint32)

    def codebook_dequantize(self, book, bits, packed, n):
        packed = np.ascontiguousarray(packed, np.uint8)
        recon = np.zeros(n, np.float32)
        assert self.lib.tq4o_codebook_dequantize(book, bits, ptr(packed), n, ptr(recon)) == 0
        return recon

    def icdf_quantize(self, in_bits, bf16):
        in_bits = np.ascontiguousarray(in_bits, np.uint16).reshape(-1)
        out = np.zeros(in_bits.size // 2, np.uint8)
        assert self.lib.tq4o_icdf_quantize(int(bf16), ptr(in_bits), in_bits.size, ptr(out)) == 0
        return out

    # ------------------------------------------------------------ RMS codec
    def rms_apply_pi(self, x, signs, inv_sqrt_len):
        y = np.ascontiguousarray(x, np.float32).copy()
        self.lib.tq4o_rms_apply_pi(ptr(y), ptr(np.ascontiguousarray(signs, np.float32)),
                                   inv_sqrt_len, y.size)
        return y

    def rms_quantize_row(self, x, signs, inv_sqrt_len):
        """(levels uint8[n], packed int8[n/2], scale float32) of one vector."""
        x = np.ascontiguousarray(x, np.float32)
        lv = np.zeros(x.size, np.uint8)
        pk = np.zeros(x.size // 2, np.int8)
        sc = np.zeros(1, np.float32)
        self.lib.tq4o_rms_quantize_row(ptr(x), ptr(np.ascontiguousarray(signs, np.float32)),
                                       x.size, inv_sqrt_len, ptr(lv), ptr(pk), ptr(sc))
        return lv, pk, sc[0]

    def rms_reshape_and_cache(self, in_dtype, key, value, key_cache, value_cache, scale_cache,
                              slots, signs, H, d, S, P, token_limit, inv_sqrt_len):
        """In place on the cache arrays; returns the rows written."""
        a = [np.ascontiguousarray(x) for x in (key, value)]
        n = self.lib.tq4o_rms_reshape_and_cache(
            in_dtype, ptr(a[0]), ptr(a[1]), ptr(key_cache), ptr(value_cache), ptr(scale_cache),
            ptr(np.ascontiguousarray(slots, np.int32)), ptr(np.ascontiguousarray(signs, np.float32)),
            a[0].shape[0], H, d, S, P, token_limit, inv_sqrt_len)
        assert n >= 0
        return n

    def rms_dequantize(self, packed):
        packed = np.ascontiguousarray(packed, np.int8).reshape(-1)
        out = np.zeros(2 * packed.size, np.float32)
        self.lib.tq4o_rms_dequantize(ptr(packed), out.size, ptr(out))
        return out

    # ------------------------------------------------------------ rotation
    def canonical_signs(self, d):
        s = np.zeros(d, np.float32)
        self.lib.tq4o_canonical_signs(d, ptr(s))
        return s

    def rotate_ingress(self, x, signs):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros_like(x)
        self.lib.tq4o_rotate_ingress(ptr(x), ptr(signs), x.size, ptr(y))
        return y

    def rotate_egress(self, x, signs):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros_like(x)
        self.lib.tq4o_rotate_egress(ptr(x), ptr(signs), x.size, ptr(y))
        return y

    def rotate_dense(self, x, signs, transpose=False):
        x = np.ascontiguousarray(x, np.float32)
        y = np.zeros(x.size, np.float64)
        self.lib.tq4o_rotate_dense(ptr(x), ptr(signs), x.size, int(transpose), ptr(y))
        return y

    def quantise_row(self, y, inv_sqrt_len, policy):
        y = np.ascontiguousarray(y, np.float32)
        q = np.zeros(y.size, np.int8)
        s = np.zeros(1, np.float32)
        self.lib.tq4o_quantise_row(ptr(y), y.size, inv_sqrt_len, policy, ptr(q), ptr(s))
        return q, s[0]

    # ------------------------------------------------------------- writers
    def reshape_and_cache(self, in_dtype, key, value, key_cache, value_cache, scale_cache, slots,
                          signs, num_kv_heads, head_size, block_size, num_blocks, inv_sqrt_len,
                          policy=POLICY_PREFILL, threads=1):
        num_tokens = slots.size
        return self.lib.tq4o_reshape_and_cache_mt(
            in_dtype, ptr(key), ptr(value), ptr(key_cache), ptr(value_cache), ptr(scale_cache),
            ptr(slots), ptr(signs), num_tokens, num_kv_heads, head_size, block_size, num_blocks,
            inv_sqrt_len, policy, threads)

    def reshape_scatter(self, key, value, key_cache, value_cache, scale_cache, slots, signs,
                        cu_seqlens, num_requests, num_kv_heads, head_size, block_size, num_blocks,
                        item_begin, item_count, inv_sqrt_len):
        return self.lib.tq4o_reshape_scatter(
            ptr(key), ptr(value), ptr(key_cache), ptr(value_cache), ptr(scale_cache), ptr(slots),
            ptr(signs), ptr(cu_seqlens), num_requests, num_kv_heads, head_size, block_size,
            num_blocks, item_begin, item_count, inv_sqrt_len)

    # -------------------------------------------------------------- decode
    def partition(self, pages, splits, split):
        b = U32()
        c = U32()
        self.lib.tq4o_partition(pages, splits, split, C.byref(b), C.byref(c))
        return b.value, c.value

    def record_floats(self, d):
        return self.lib.tq4o_record_floats(d)

    def decode_partials(self, q, kc, vc, sc, tables, ctx, signs, num_heads, num_kv_heads,
                        head_size, block_size, num_blocks, num_splits, scale, inv_sqrt_len,
                        flags=0):
        B = ctx.size
        ws = np.zeros((B, num_heads, num_splits, self.record_floats(head_size)), np.float32)
        rc = self.lib.tq4o_decode_partials(
            ptr(q), ptr(kc), ptr(vc), ptr(sc), ptr(tables), ptr(ctx), ptr(signs), ptr(ws), B,
            num_heads, num_kv_heads, head_size, block_size, num_blocks, tables.shape[1],
            num_splits, scale, inv_sqrt_len, flags)
        assert rc == 0, rc
        return ws

    def combine(self, ws, signs, gate, num_heads, head_size, num_splits, inv_sqrt_len, stage):
        B = ws.shape[0]
        out = np.zeros((B, num_heads, head_size), np.uint16)
        outf = np.zeros((B, num_heads, head_size), np.float32)
        rc = self.lib.tq4o_combine(ptr(ws), ptr(signs), ptr(gate), ptr(out), ptr(outf), B,
                                   num_heads, head_size, num_splits, inv_sqrt_len, stage)
        assert rc == 0, rc
        return out, outf

    def paged_decode(self, q, kc, vc, sc, tables, ctx, signs, gate, num_heads, num_kv_heads,
                     head_size, block_size, num_blocks, num_splits, scale, inv_sqrt_len, stage,
                     flags=0, threads=1):
        B = ctx.size
        out = np.zeros((B, num_heads, head_size), np.uint16)
        outf = np.zeros((B, num_heads, head_size), np.float32)
        rc = self.lib.tq4o_paged_decode(
            ptr(q), ptr(kc), ptr(vc), ptr(sc), ptr(tables), ptr(ctx), ptr(signs), ptr(gate),
            ptr(out), ptr(outf), B, num_heads, num_kv_heads, head_size, block_size, num_blocks,
            tables.shape[1], num_splits, scale, inv_sqrt_len, stage, flags, threads)
        assert rc == 0, rc
        return out, outf

    def decode_reference_f64(self, q, kc, vc, sc, tables, ctx, signs, gate, num_heads,
                             num_kv_heads, head_size, block_size, num_blocks, scale,
                             inv_sqrt_len, stage, flags=0):
        B = ctx.size
        out = np.zeros((B, num_heads, head_size), np.float64)
        rc = self.lib.tq4o_decode_reference_f64(
            ptr(q), ptr(kc), ptr(vc), ptr(sc), ptr(tables), ptr(ctx), ptr(signs), ptr(gate),
            ptr(out), B, num_heads, num_kv_heads, head_size, block_size, num_blocks,
            tables.shape[1], scale, inv_sqrt_len, stage, flags)
        assert rc == 0, rc
        return out


class Ref:
    """The reference's own oracles (oracle/_ref), present only where built."""

    @staticmethod
    def available():
        return os.path.exists(REF_SO)

    def __init__(self, path=REF_SO):
        L = self.lib = C.CDLL(path)
        L.ref_tq_compute_reference.restype = I32
        L.ref_tq_compute_reference.argtypes = [I32] * 5 + [P] * 8
        L.ref_tq_build_activations.argtypes = [I32] * 5 + [P, P]
        L.ref_tq_build_slot_mapping.argtypes = [I32] * 5 + [P]
        L.ref_tq_build_tables.argtypes = [I32, P]
        L.ref_tq_audit_tables.restype = C.c_longlong
        L.ref_tq_audit_tables.argtypes = [I32, P]
        L.ref_tq_rint_even_shift.restype = C.c_longlong
        L.ref_tq_rint_even_shift.argtypes = [C.c_longlong, I32]
        L.ref_tq_pi_sign.restype = I32
        L.ref_tq_pi_sign.argtypes = [I32]
        L.ref_rot_staged.argtypes = [I32, P, P, F32, P]
        L.ref_rot_dense_left.argtypes = [P, P, P]
        L.ref_rot_dense_right.argtypes = [P, P, P]
        L.ref_scatter_activation.restype = F32
        L.ref_scatter_activation.argtypes = [I32] * 6
        L.ref_scatter_compute_reference.restype = I32
        L.ref_scatter_compute_reference.argtypes = [I32] * 4 + [P, P, P, I32, P, P, P, P, P]
        for n in ("ref_scatter_value_nibble", "ref_scatter_key_nibble"):
            getattr(L, n).restype = C.c_ulonglong
            getattr(L, n).argtypes = [I32] * 8
        L.ref_scatter_scale_index.restype = C.c_ulonglong
        L.ref_scatter_scale_index.argtypes = [I32] * 7
        L.ref_partition.argtypes = [U32, U32, U32, P, P]
        L.ref_active_in_strip.restype = U32
        L.ref_active_in_strip.argtypes = [C.c_ulonglong, U32]
        L.ref_live_strips_in_window.restype = U32
        L.ref_live_strips_in_window.argtypes = [U32] * 6
        L.ref_l2_combine_step.argtypes = [P, P, P]
        L.ref_l2_tile_state.argtypes = [I32, U32, P]
        L.ref_l2_uniform_expected.restype = I32
        L.ref_l2_uniform_expected.argtypes = [U32, U32, P]
        L.ref_l2_combine_and_egress.argtypes = [I32, U32, P, P]
        L.ref_l2_gate_vector.argtypes = [P]
        L.ref_splitk_fixture_dims.argtypes = [I32, I32, P, P]
        L.ref_splitk_fixture.restype = I32
        L.ref_splitk_fixture.argtypes = [I32] * 7 + [P] * 8
        L.ref_aic_partial.restype = I32
        L.ref_aic_partial.argtypes = [I32] * 8 + [U32, U32, P, P, P]
        L.ref_icdf_fixture.restype = I32
        L.ref_icdf_fixture.argtypes = [I32, U32, P, P]
        L.ref_lloyd_fixture.argtypes = [U32, U32, I32, U32, P]
        L.ref_lloyd_code.restype = U32
        L.ref_lloyd_code.argtypes = [U32, F32, I32]
        L.ref_lloyd_centroid.restype = F32
        L.ref_lloyd_centroid.argtypes = [U32, U32, I32]
        L.ref_lloyd_threshold.restype = F32
        L.ref_lloyd_threshold.argtypes = [U32, U32]
        L.ref_lloyd_pack.argtypes = [P, U32, U32, P]
        L.ref_fdo_dims.restype = I32
        L.ref_fdo_dims.argtypes = [I32] * 5 + [P]
        L.ref_fdo_fixture.restype = I32
        L.ref_fdo_fixture.argtypes = [I32] * 6 + [P] * 8
        L.ref_fdo_raw.restype = I32
        L.ref_fdo_raw.argtypes = [I32] * 6 + [U32, P, P, P, P]
        L.ref_fdo_gain.restype = F32
        L.ref_nz_byte.restype = C.c_ulonglong
        L.ref_nz_byte.argtypes = [C.c_ulonglong] * 5
