"""PyTorch operator registrations of the TQ4 path over libtq4.so.

The reference declares a vLLM-facing schema inventory and defers the
registrations (kernels/ops/turboquant/vllm_integration_layer/op_adapter/
turboquant_torch_ops.h:3-11, turboquant_torch_adpt.h:1-47). The operator
argument lists follow the reference's vLLM-style entry points
(kernels/ops/turboquant/baseline/turboquant_paged_attention.cpp:754-793):

  tq4::reshape_and_cache   turboquant_reshape_and_cache_impl   (A8 or BF16 K/V)
  tq4::reshape_scatter     launch_turboquant_reshape_scatter_aiv
  tq4::paged_attention     turboquant_paged_attention_impl     (fused split-K decode)
  tq4::fused_decode_opt    turboquant_mm_fused_decode_opt_impl (KV4/FP8 NZ cache,
                           vllm_integration_layer/include/turboquant_fused_decode_opt.hpp:198-207)
  tq4::fused_decode_opt_raw_query
                           turboquant_mm_fused_decode_opt_raw_query_impl, the decode
                           symbol of the reference's schema inventory
                           (op_adapter/turboquant_torch_adpt.h:12-22,
                           turboquant_torch_ops.h:6-7)

Sizes that the reference passes as integers (num_tokens, num_kv_heads,
head_size, num_heads, max_blocks_per_seq, num_blocks) come from tensor shapes
here. Caches are the TQ4 byte pools: key_cache and value_cache int8
[num_blocks, num_kv_heads, block_size, head_size // 2], scale_cache float32
[2, num_blocks, num_kv_heads, block_size] (any contiguous shape with those
element counts is accepted; num_blocks is taken from dim 0 of a 4-D key
cache, else from its size).

The device implementations are the ctypes calls of the `tq4` module, on
torch's current stream; there is no CPU implementation (a CPU tensor raises).
Each operator also has a fake implementation, so FakeTensor / meta tracing
(torch.compile, shape propagation) sees the right outputs without a GPU.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from . import tq4 as _tq4

NAMESPACE = "tq4"


def _num_blocks(key_cache: torch.Tensor, num_kv_heads: int, block_size: int,
                head_size: int) -> int:
    if key_cache.dim() == 4:
        return int(key_cache.shape[0])
    return key_cache.numel() * 2 // (num_kv_heads * block_size * head_size)


def _isl(inv_sqrt_len: float, head_size: int) -> float:
    return inv_sqrt_len if inv_sqrt_len > 0.0 else 1.0 / math.sqrt(head_size)


@torch.library.custom_op(f"{NAMESPACE}::reshape_and_cache",
                         mutates_args=("key_cache", "value_cache", "scale_cache"),
                         device_types="cuda")
def reshape_and_cache(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                      value_cache: torch.Tensor, scale_cache: torch.Tensor,
                      slot_mapping: torch.Tensor, pi_signs: Optional[torch.Tensor],
                      tables: Optional[torch.Tensor], block_size: int,
                      inv_sqrt_len: float) -> None:
    """Whole 16-token strips of INT8 or BF16 K/V [tokens][kv_heads][head_size]
    into the cache (slot contract: consecutive, strip-aligned slots).
    inv_sqrt_len <= 0 means 1/sqrt(head_size)."""
    num_tokens, num_kv_heads, head_size = key.shape
    P = _num_blocks(key_cache, num_kv_heads, block_size, head_size)
    isl = _isl(inv_sqrt_len, head_size)
    if key.dtype == torch.int8:
        fn = _tq4.reshape_and_cache_a8
    elif key.dtype == torch.bfloat16:
        fn = _tq4.reshape_and_cache_bf16
    else:
        raise ValueError(f"tq4::reshape_and_cache: key/value must be int8 or bfloat16, "
                         f"got {key.dtype}")
    fn(key, value, key_cache, value_cache, scale_cache, slot_mapping, pi_signs=pi_signs,
       tables=tables, num_blocks=P, block_size=block_size, inv_sqrt_len=isl)


@reshape_and_cache.register_fake
def _(key, value, key_cache, value_cache, scale_cache, slot_mapping, pi_signs, tables,
      block_size, inv_sqrt_len):
    return None


@torch.library.custom_op(f"{NAMESPACE}::reshape_scatter",
                         mutates_args=("key_cache", "value_cache", "scale_cache"),
                         device_types="cuda")
def reshape_scatter(key: torch.Tensor, value: torch.Tensor, key_cache: torch.Tensor,
                    value_cache: torch.Tensor, scale_cache: torch.Tensor,
                    slot_mapping: torch.Tensor, pi_signs: torch.Tensor,
                    cu_seqlens: Optional[torch.Tensor], block_size: int,
                    inv_sqrt_len: float) -> None:
    """BF16 tokens at arbitrary slots (negative slot = padding); requests are
    cu_seqlens segments, or one token each when cu_seqlens is None."""
    num_tokens, num_kv_heads, head_size = key.shape
    P = _num_blocks(key_cache, num_kv_heads, block_size, head_size)
    _tq4.reshape_scatter(key, value, key_cache, value_cache, scale_cache, slot_mapping,
                         pi_signs, cu_seqlens=cu_seqlens, num_blocks=P, block_size=block_size,
                         inv_sqrt_len=_isl(inv_sqrt_len, head_size))


@reshape_scatter.register_fake
def _(key, value, key_cache, value_cache, scale_cache, slot_mapping, pi_signs, cu_seqlens,
      block_size, inv_sqrt_len):
    return None


@torch.library.custom_op(f"{NAMESPACE}::paged_attention", mutates_args=("workspace",),
                         device_types="cuda")
def paged_attention(query: torch.Tensor, key_cache: torch.Tensor, value_cache: torch.Tensor,
                    scale_cache: torch.Tensor, block_tables: torch.Tensor,
                    context_lens: torch.Tensor, pi_signs: torch.Tensor,
                    workspace: torch.Tensor, gate: Optional[torch.Tensor], num_kv_heads: int,
                    block_size: int, num_splits: int, scale: float, inv_sqrt_len: float,
                    output_stage: int, query_rotated: bool) -> torch.Tensor:
    """Fused split-K decode: query [B][num_heads][head_size] BF16 ->
    output [B][num_heads][head_size] BF16. The workspace comes from
    `workspace_for` (zeroed once; the operator leaves it zeroed). num_splits 0
    = auto; scale / inv_sqrt_len <= 0 mean 1/sqrt(head_size)."""
    B, Hq, d = query.shape
    P = _num_blocks(key_cache, num_kv_heads, block_size, d)
    return _tq4.paged_decode(
        query, key_cache, value_cache, scale_cache, block_tables, context_lens, pi_signs,
        num_kv_heads, block_size, P, workspace=workspace, gate=gate, num_splits=num_splits,
        scale=scale if scale > 0.0 else 1.0 / math.sqrt(d), inv_sqrt_len=_isl(inv_sqrt_len, d),
        output_stage=output_stage,
        flags=_tq4.TQ4_DECODE_QUERY_ROTATED if query_rotated else 0)


@paged_attention.register_fake
def _(query, key_cache, value_cache, scale_cache, block_tables, context_lens, pi_signs,
      workspace, gate, num_kv_heads, block_size, num_splits, scale, inv_sqrt_len, output_stage,
      query_rotated):
    return torch.empty_like(query)


def _kv4_blocks(key_cache: torch.Tensor, num_kv_heads: int, block_size: int) -> int:
    if key_cache.dim() >= 2 and key_cache.numel() // key_cache.shape[0] == \
            block_size * num_kv_heads * 128:
        return int(key_cache.shape[0])
    return key_cache.numel() // (block_size * num_kv_heads * 128)


@torch.library.custom_op(f"{NAMESPACE}::fused_decode_opt", mutates_args=("workspace",),
                         device_types="cuda")
def fused_decode_opt(query_rot: torch.Tensor, key_cache: torch.Tensor,
                     value_cache: torch.Tensor, scale_cache: torch.Tensor,
                     block_tables: torch.Tensor, context_lens: torch.Tensor,
                     workspace: torch.Tensor, num_kv_heads: int, block_size: int,
                     num_splits: int, heads_per_task: int, fused_context_limit: int,
                     scale: float, inv_sqrt_len: float, bf16_output: bool) -> torch.Tensor:
    """KV4/FP8 NZ-tiled decode, pre-rotated entry: query_rot FP32
    [T][num_heads][256] -> output [T][num_heads][256] FP16 (BF16 when
    bf16_output). key_cache / value_cache uint8 (any shape of num_blocks *
    block_size * num_kv_heads * 128 bytes), scale_cache FP32 [..][8]. The
    workspace comes from `kv4fp8_workspace_for`."""
    T, Hq, d = query_rot.shape
    P = _kv4_blocks(key_cache, num_kv_heads, block_size)
    return _tq4.kv4fp8_decode(
        query_rot, key_cache, value_cache, scale_cache, block_tables, context_lens,
        num_kv_heads, block_size, P, workspace=workspace,
        out_dtype=torch.bfloat16 if bf16_output else torch.float16, splits=num_splits,
        heads_per_task=heads_per_task, fused_context_limit=fused_context_limit,
        scale=scale if scale > 0.0 else 1.0 / math.sqrt(d), inv_sqrt_len=_isl(inv_sqrt_len, d))


@fused_decode_opt.register_fake
def _(query_rot, key_cache, value_cache, scale_cache, block_tables, context_lens, workspace,
      num_kv_heads, block_size, num_splits, heads_per_task, fused_context_limit, scale,
      inv_sqrt_len, bf16_output):
    return torch.empty(query_rot.shape, dtype=torch.bfloat16 if bf16_output else torch.float16,
                       device=query_rot.device)


@torch.library.custom_op(f"{NAMESPACE}::fused_decode_opt_raw_query",
                         mutates_args=("query_rot", "workspace"), device_types="cuda")
def fused_decode_opt_raw_query(query: torch.Tensor, pi_signs: torch.Tensor,
                               gate: Optional[torch.Tensor], query_rot: torch.Tensor,
                               key_cache: torch.Tensor, value_cache: torch.Tensor,
                               scale_cache: torch.Tensor, block_tables: torch.Tensor,
                               context_lens: torch.Tensor, workspace: torch.Tensor,
                               num_kv_heads: int, block_size: int, num_splits: int,
                               heads_per_task: int, output_stage: int,
                               fused_context_limit: int, scale: float,
                               inv_sqrt_len: float) -> torch.Tensor:
    """KV4/FP8 NZ-tiled decode, raw-query entry: query FP16 or BF16
    [T][num_heads][256] in the original basis -> output of the same element
    type; query_rot (FP32, same shape) receives the rotated query. Output
    stage 0 keeps the rotated basis, 1 rotates back, 2 also divides by
    1 + exp(-gate)."""
    T, Hq, d = query.shape
    P = _kv4_blocks(key_cache, num_kv_heads, block_size)
    return _tq4.kv4fp8_decode_raw_query(
        query, pi_signs, key_cache, value_cache, scale_cache, block_tables, context_lens,
        num_kv_heads, block_size, P, gate=gate, output_stage=output_stage, query_out=query_rot,
        workspace=workspace, splits=num_splits, heads_per_task=heads_per_task,
        fused_context_limit=fused_context_limit,
        scale=scale if scale > 0.0 else 1.0 / math.sqrt(d), inv_sqrt_len=_isl(inv_sqrt_len, d))


@fused_decode_opt_raw_query.register_fake
def _(query, pi_signs, gate, query_rot, key_cache, value_cache, scale_cache, block_tables,
      context_lens, workspace, num_kv_heads, block_size, num_splits, heads_per_task,
      output_stage, fused_context_limit, scale, inv_sqrt_len):
    return torch.empty_like(query)


def kv4fp8_workspace_for(query: torch.Tensor, num_kv_heads: int, block_tables: torch.Tensor,
                         block_size: int, num_blocks: int = 1) -> torch.Tensor:
    """A zeroed workspace for tq4::fused_decode_opt(_raw_query) at this
    geometry (every call leaves it zero again, so it can be reused)."""
    T, Hq, d = query.shape
    L = _tq4.fused_decode_opt_launch(T, Hq, num_kv_heads, block_size, block_tables.shape[1],
                                     num_blocks=max(1, num_blocks))
    n = _tq4.kv4fp8_workspace_bytes(L)
    if n == 0:
        raise ValueError("kv4fp8_workspace_for: unsupported geometry")
    return torch.zeros(n, dtype=torch.uint8, device=query.device)


def workspace_for(query: torch.Tensor, num_kv_heads: int, block_tables: torch.Tensor,
                  block_size: int = 16, num_splits: int = 0) -> torch.Tensor:
    """A zeroed workspace for tq4::paged_attention at this geometry (the
    split count the operator will use when num_splits is 0)."""
    B, Hq, d = query.shape
    if num_splits == 0:
        num_splits = _tq4.auto_splits(B, num_kv_heads, block_tables.shape[1], block_size)
    return _tq4.decode_workspace(B, Hq, num_kv_heads, d, num_splits, query.device)


__all__ = ["NAMESPACE", "reshape_and_cache", "reshape_scatter", "paged_attention",
           "workspace_for", "fused_decode_opt", "fused_decode_opt_raw_query",
           "kv4fp8_workspace_for"]
