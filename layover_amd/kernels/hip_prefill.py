"""Paged causal prefill attention as a gfx950 HIP kernel (lk_paged_prefill).

Drop-in for the reference's layover/model.py:69-98 prefill_attention(q, k, v, cache, layer,
chunk, groups): the same arguments and result ([query_heads, tokens, head_dim] in q's dtype),
but K and V of the whole history are read in place from the pool through chunk.block_ids
instead of being gathered out of it every layer. As in the reference's model
(model.py:131-135), the chunk's own K/V must be in the pool first (PagedKVCache.write_at), so
k and v are not read again here. The pool may be the cache's BF16 pool or an FP8-resident
Fp8KVPool of the same blocks.
"""

from __future__ import annotations

import math

import torch

from layover_amd.kernels import _lib
from layover_amd.kernels.hip_decode import Fp8KVPool, _is_fp8


def validate(q, pool, layer: int, block_ids: torch.Tensor, start: int, kv_groups: int) -> None:
    """Everything the kernel relies on, from tensor metadata alone (no device reads)."""
    if q.dim() != 3:
        raise ValueError(f"q must be [query_heads, tokens, head_dim], got {tuple(q.shape)}")
    if q.dtype != torch.bfloat16 or not q.is_contiguous():
        raise ValueError("q must be contiguous BF16")
    if pool.dim() != 6 or pool.shape[1] != 2:
        raise ValueError(f"pool must be [blocks, 2, layers, kv_heads, slots, head_dim], got {tuple(pool.shape)}")
    blocks, _, layers, kv_heads, slots, head_dim = pool.shape
    query_heads, tokens, dim = q.shape
    if not _is_fp8(pool) and pool.dtype != torch.bfloat16:
        raise ValueError(f"the paged prefill kernel reads BF16 or FP8-record pools, not {pool.dtype}")
    if not pool.is_contiguous():
        raise ValueError("the pool must be contiguous")
    if (slots, head_dim, dim) != (16, 128, 128):
        raise ValueError(f"the paged prefill kernel needs 16-slot blocks of 128 dims, got {slots} x {head_dim}")
    if query_heads != kv_heads * kv_groups:
        raise ValueError(f"{query_heads} query heads do not match {kv_heads} KV heads x {kv_groups}")
    if not 0 <= layer < layers:
        raise ValueError(f"layer {layer} out of range for {layers} layers")
    if tokens < 1 or start < 0:
        raise ValueError(f"a chunk needs tokens >= 1 and start >= 0, got {tokens} and {start}")
    if block_ids.dtype != torch.int32 or block_ids.dim() != 1 or not block_ids.is_contiguous():
        raise ValueError("block_ids must be a contiguous 1-D int32 tensor")
    if block_ids.shape[0] * slots < start + tokens:
        raise ValueError(f"{block_ids.shape[0]} blocks cannot hold tokens up to {start + tokens}")
    devices = {q.device, pool.device, block_ids.device}
    if len(devices) != 1 or q.device.type != "cuda":
        raise ValueError(f"q, pool and block ids must be on one GPU, got {devices}")


def run_kernel(q, pool, layer: int, block_ids: torch.Tensor, start: int, kv_groups: int, out: torch.Tensor) -> None:
    """Launch on the current stream into `out` (q's shape and dtype). Block ids are not read
    on the host: the caller has checked them against the pool (as chunk_locations' table
    does). A chunk whose tiles would leave CUs idle splits its keys (split-K) into a workspace
    taken from torch's allocator on this stream, then merges them."""
    query_heads, tokens, head_dim = q.shape
    _, _, layers, kv_heads, slots, _ = pool.shape
    kv_format = _lib.LK_FP8_RECORD if _is_fp8(pool) else _lib.LK_BF16
    shape = _lib.PrefillShape(tokens, start, query_heads, kv_heads, head_dim, layers, slots, layer, _lib.LK_BF16, kv_format,
                              1.0 / math.sqrt(head_dim))
    storage = pool.records if isinstance(pool, Fp8KVPool) else pool
    lib = _lib.load()
    need = int(lib.lk_paged_prefill_workspace(shape))
    workspace = torch.empty(need, dtype=torch.uint8, device=q.device) if need else None
    _lib.check(
        lib.lk_paged_prefill_split(shape, q.data_ptr(), storage.data_ptr(), block_ids.data_ptr(), block_ids.shape[0], out.data_ptr(),
                                   workspace.data_ptr() if need else None, need, _lib.current_stream(q.device))
    )


def paged_prefill_attention_hip(q, pool, layer: int, block_ids: torch.Tensor, start: int, kv_groups: int) -> torch.Tensor:
    """Causal attention of the chunk's tokens [start, start + tokens) over keys [0, start + t]."""
    validate(q, pool, layer, block_ids, start, kv_groups)
    out = torch.empty_like(q)
    run_kernel(q, pool, layer, block_ids, start, kv_groups, out)
    return out


def prefill_attention(q, k, v, cache, layer: int, chunk, groups: int, pool=None) -> torch.Tensor:
    """The reference's prefill_attention signature (model.py:69): q [heads, tokens, dim]; k and
    v are the chunk's own, already written to the cache; returns [heads, tokens, dim]."""
    if k.shape[1] != chunk.tokens or v.shape[1] != chunk.tokens or q.shape[1] != chunk.tokens:
        raise ValueError("q, k and v must hold the chunk's tokens")
    return paged_prefill_attention_hip(q.contiguous(), cache.pool if pool is None else pool, layer, chunk.block_ids, chunk.start, groups)
