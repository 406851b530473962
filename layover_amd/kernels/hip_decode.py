"""Paged GQA decode attention as a gfx950 HIP kernel.

Drop-in for the reference's layover/kernels/triton_decode.py call sites:
paged_decode_attention_hip / paged_decode_attention_hip_trusted take the arguments of
paged_decode_attention_triton / _trusted (triton_decode.py:235-261) and refuse the same bad
inputs before anything is launched (validate_shapes / validate, triton_decode.py:182-232).
The kernel reads K and V through the block table straight from the pool, with an online
softmax in FP32, split-K over the context and a combine pass (layover_amd/csrc/
decode_attention.h), through liblayover_kernels.so.

Pools: BF16 or FP32 tensors shaped [block, 2, layers, kv_heads, slots, dim]
(paged_cache.py:40-49), or an Fp8KVPool of FP8 records in the format of
layover_amd.kernels.fp8 (the reference has no FP8 decode; its record format is reused).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch

from layover_amd.kernels import _lib
from layover_amd.kernels.fp8 import Fp8Layout

KV_KINDS = 2
KV_DTYPES = (torch.bfloat16, torch.float32)
_FORMATS = {torch.bfloat16: _lib.LK_BF16, torch.float32: _lib.LK_F32}


@dataclass
class Fp8KVPool:
    """A KV pool held as FP8 records: `records` is uint8 [blocks, record_bytes], each row the
    record lk_fp8_quantize writes for one block of a [2, layers, kv_heads, slots, head_dim]
    BF16 block."""

    records: torch.Tensor
    layers: int
    kv_heads: int
    slots: int
    head_dim: int

    @property
    def layout(self) -> Fp8Layout:
        return Fp8Layout(self.slots * self.head_dim, KV_KINDS * self.layers * self.kv_heads)

    @property
    def shape(self) -> tuple[int, ...]:
        return (self.records.shape[0], KV_KINDS, self.layers, self.kv_heads, self.slots, self.head_dim)

    @property
    def device(self) -> torch.device:
        return self.records.device

    def dim(self) -> int:
        return 6

    def is_contiguous(self) -> bool:
        return self.records.is_contiguous()

    def write(self, write_blocks: torch.Tensor, write_slots: torch.Tensor, layer: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Write one token per row into layer `layer`, the FP8 counterpart of the reference's
        decode-time pool assignment (model.py:139-140): k and v are BF16 [batch, kv_heads,
        head_dim]; row b goes to slot write_slots[b] of block write_blocks[b]. Each group it
        touches is re-encoded at a new shift (a new value may raise the group's largest
        exponent), from the old values decoded at the old shift for earlier slots, the new
        value at the write slot, and zero for the later slots, which no length covers yet.
        write_blocks and write_slots are int32 on the pool's device, 1-D with one stride
        between rows (columns of PagedKVCache.decode_rows are accepted as they are). Ids are
        not checked against the pool: the caller has (as decode_rows does). Rows must name
        distinct (block, layer) groups; two rows writing one group race. Enqueued on the
        current stream."""
        batch = _check_token_write(self.records.device, self.layers, self.kv_heads, self.head_dim, write_blocks, write_slots, layer, k, v)
        if batch == 0:
            return
        _lib.check(
            _lib.load().lk_fp8_append(self.records.data_ptr(), write_blocks.data_ptr(), write_slots.data_ptr(), write_blocks.stride(0),
                                      batch, k.data_ptr(), v.data_ptr(), layer, self.layers, self.kv_heads, self.slots,
                                      self.head_dim, _lib.current_stream(self.records.device))
        )

    @classmethod
    def empty(cls, blocks: int, layers: int, kv_heads: int, slots: int, head_dim: int, device) -> "Fp8KVPool":
        layout = Fp8Layout(slots * head_dim, KV_KINDS * layers * kv_heads)
        return cls(torch.zeros(blocks, layout.record_bytes, dtype=torch.uint8, device=device), layers, kv_heads, slots, head_dim)


def _check_token_write(device, layers, kv_heads, head_dim, write_blocks, write_slots, layer, k, v) -> int:
    """Arguments of a decode-time token write, from tensor metadata alone; returns the rows."""
    if not 0 <= layer < layers:
        raise ValueError(f"layer {layer} out of range for {layers} layers")
    batch = write_blocks.shape[0]
    for name, rows in (("write_blocks", write_blocks), ("write_slots", write_slots)):
        if rows.dtype != torch.int32 or rows.dim() != 1 or rows.shape[0] != batch:
            raise ValueError(f"{name} must be 1-D int32 with one entry per row")
    if batch and write_blocks.stride(0) != write_slots.stride(0):
        raise ValueError("write_blocks and write_slots must share one row stride")
    expected = (batch, kv_heads, head_dim)
    for name, t in (("k", k), ("v", v)):
        if t.dtype != torch.bfloat16 or tuple(t.shape) != expected or not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous BF16 shaped {expected}")
    devices = {device, write_blocks.device, write_slots.device, k.device, v.device}
    if len(devices) != 1 or device.type != "cuda":
        raise ValueError("the pool, rows, k and v must be on one GPU")
    return batch


def write_tokens(pool: torch.Tensor, write_blocks: torch.Tensor, write_slots: torch.Tensor, layer: int, k: torch.Tensor,
                 v: torch.Tensor) -> None:
    """The decode-time write of one token per row into a BF16 pool [blocks, 2, layers,
    kv_heads, slots, head_dim], as one kernel: the same result as the reference's
    pool[write_blocks, 0, layer, :, write_slots] = k and likewise for v (model.py:139-140).
    Rows as for Fp8KVPool.write (int32, one shared stride, e.g. columns of decode_rows); ids
    and slots are not checked against the pool. Enqueued on the current stream."""
    if pool.dtype != torch.bfloat16 or pool.dim() != 6 or pool.shape[1] != KV_KINDS or not pool.is_contiguous():
        raise ValueError("the pool must be a contiguous BF16 [blocks, 2, layers, kv_heads, slots, head_dim] tensor")
    _, _, layers, kv_heads, slots, head_dim = pool.shape
    batch = _check_token_write(pool.device, layers, kv_heads, head_dim, write_blocks, write_slots, layer, k, v)
    if batch == 0:
        return
    _lib.check(
        _lib.load().lk_kv_write(pool.data_ptr(), write_blocks.data_ptr(), write_slots.data_ptr(), write_blocks.stride(0), batch,
                                k.data_ptr(), v.data_ptr(), layer, layers, kv_heads, slots, head_dim, _lib.current_stream(pool.device))
    )


def _is_fp8(pool) -> bool:
    return isinstance(pool, Fp8KVPool)


def validate_shapes(q, pool, layer, block_table, lengths, kv_groups) -> None:
    """Everything that can be checked without reading the GPU (triton_decode.py:182-215)."""
    if q.dim() != 3 or pool.dim() != 6 or block_table.dim() != 2 or lengths.dim() != 1:
        raise ValueError(f"bad ranks: q {tuple(q.shape)}, pool {tuple(pool.shape)}, table {tuple(block_table.shape)}, lengths {tuple(lengths.shape)}")
    if not pool.is_contiguous():
        raise ValueError("the pool must be contiguous: its strides are derived from its shape")
    if _is_fp8(pool):
        if pool.records.dtype != torch.uint8 or pool.records.dim() != 2 or pool.records.shape[1] != pool.layout.record_bytes:
            raise ValueError("an FP8 pool is uint8 [blocks, record_bytes]")
    elif pool.dtype not in KV_DTYPES:
        raise ValueError(f"the pool is {pool.dtype}; the kernel takes {KV_DTYPES} or an Fp8KVPool")
    if q.dtype not in KV_DTYPES:
        raise ValueError(f"q is {q.dtype}; the kernel takes {KV_DTYPES}")
    batch, query_heads, head_dim = q.shape
    blocks, kinds, layers, kv_heads, slots, pool_dim = pool.shape
    if kinds != KV_KINDS:
        raise ValueError(f"pool has {kinds} kinds, expected K and V")
    if head_dim != pool_dim:
        raise ValueError(f"q head_dim {head_dim} differs from the pool's {pool_dim}")
    if kv_groups < 1 or query_heads != kv_heads * kv_groups:
        raise ValueError(f"{query_heads} query heads cannot share {kv_heads} KV heads in groups of {kv_groups}")
    if not 0 <= layer < layers:
        raise ValueError(f"layer {layer} out of range for {layers} layers")
    if block_table.shape[0] != batch or lengths.shape[0] != batch:
        raise ValueError(f"batch {batch} disagrees with table {tuple(block_table.shape)} and lengths {tuple(lengths.shape)}")
    if block_table.shape[1] < 1:
        raise ValueError("the block table has no columns")
    devices = {q.device, pool.device, block_table.device, lengths.device}
    if len(devices) != 1:
        raise ValueError(f"tensors span devices {devices}")
    if q.device.type != "cuda":
        raise ValueError(f"tensors are on {q.device}: the HIP kernel runs on the GPU only")
    if q.device.index != torch.cuda.current_device():
        raise ValueError(f"tensors are on {q.device}, the current device is {torch.cuda.current_device()}")
    if block_table.is_floating_point() or lengths.is_floating_point():
        raise TypeError("the block table and lengths must be integers")
    if head_dim > 256 and not (slots == 16 and head_dim == 128):
        raise ValueError(f"head_dim {head_dim} is not supported (at most 256)")


def validate(q, pool, layer, block_table, lengths, kv_groups) -> int:
    """validate_shapes plus the bounds a kernel cannot check for itself, at the cost of one
    device read (triton_decode.py:218-232). Returns the number of table entries the lengths
    cover (blocks the launch reads, counted once per row), taken in the same read."""
    validate_shapes(q, pool, layer, block_table, lengths, kv_groups)
    slots, blocks = pool.shape[4], pool.shape[0]
    wide = lengths.long()
    listed = torch.div(wide + slots - 1, slots, rounding_mode="floor").sum()
    bounds = torch.stack([*torch.aminmax(wide), *torch.aminmax(block_table.long()), listed])
    shortest, longest, lowest, highest, listed = bounds.tolist()
    if shortest < 1 or longest > block_table.shape[1] * slots:
        raise ValueError(f"lengths in [{shortest}, {longest}] do not fit a table of {block_table.shape[1]} blocks")
    if lowest < 0 or highest >= blocks:
        raise ValueError(f"block ids in [{lowest}, {highest}] are outside a pool of {blocks} blocks")
    return listed


def decode_shape(q, pool, layer, block_table, kv_groups, lengths=None, shared_blocks: bool = False) -> _lib.DecodeShape:
    """The launch's shape; the table's row stride and the lengths' stride are taken from the
    tensors, so columns of a packed row block (PagedKVCache.decode_rows) pass without a copy,
    as the reference's launcher passes strides (triton_decode.py:131-179). shared_blocks sets
    LK_DECODE_SHARED_BLOCKS: rows read some of the same blocks, so the kernel keeps tiles in
    the caches instead of streaming them (the same results, a different speed)."""
    batch, query_heads, head_dim = q.shape
    _, _, layers, kv_heads, slots, _ = pool.shape
    kv_format = _lib.LK_FP8_RECORD if _is_fp8(pool) else _FORMATS[pool.dtype]
    table_stride = block_table.stride(0) if block_table.dim() == 2 else block_table.shape[-1]
    lengths_stride = lengths.stride(0) if lengths is not None and lengths.dim() == 1 else 1
    return _lib.DecodeShape(batch, query_heads, kv_heads, head_dim, layers, slots, layer, block_table.shape[1],
                            _FORMATS[q.dtype], kv_format, 1.0 / math.sqrt(head_dim), table_stride, lengths_stride,
                            _lib.LK_DECODE_SHARED_BLOCKS if shared_blocks else 0)


def _check_layout(q, block_table, lengths, out) -> None:
    """What the kernel assumes of memory layout, checked from tensor metadata alone (no device
    reads): a wrong stride would make it read the wrong rows, or past the table."""
    if not (q.is_contiguous() and out.is_contiguous() and out.shape == q.shape and out.dtype == q.dtype):
        raise ValueError("q and out must be contiguous tensors of one shape and dtype")
    if block_table.dtype != torch.int32 or lengths.dtype != torch.int32:
        raise ValueError("the block table and lengths must be int32 for the kernel")
    if block_table.dim() != 2 or lengths.dim() != 1 or not lengths.shape[0] == block_table.shape[0] == q.shape[0]:
        raise ValueError("the block table must be [batch, width] and lengths [batch]")
    if block_table.shape[1] > 1 and block_table.stride(1) != 1:
        raise ValueError("block table rows must be contiguous (any row stride)")
    if block_table.stride(0) < block_table.shape[1] or lengths.stride(0) < 1:
        raise ValueError("the block table's rows must not overlap")


def workspace_bytes(shape: _lib.DecodeShape) -> int:
    return int(_lib.load().lk_paged_decode_workspace(shape))


def run_kernel(q, pool, layer, block_table, lengths, kv_groups, out, workspace=None, shared_blocks: bool = False) -> None:
    """Launch without validating values, on the current stream. q and out contiguous; table
    int32 [batch, width] with contiguous rows at any row stride; lengths int32 [batch] at any
    stride. A workspace passed in must not be in use by another launch at the same time.
    shared_blocks as for decode_shape."""
    _check_layout(q, block_table, lengths, out)
    lib = _lib.load()
    shape = decode_shape(q, pool, layer, block_table, kv_groups, lengths, shared_blocks)
    need = int(lib.lk_paged_decode_workspace(shape))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=q.device)
    storage = pool.records if _is_fp8(pool) else pool
    _lib.check(
        lib.lk_paged_decode(shape, q.data_ptr(), storage.data_ptr(), block_table.data_ptr(), lengths.data_ptr(), out.data_ptr(),
                            workspace.data_ptr(), workspace.numel(), _lib.current_stream(q.device))
    )


def run_kernel_append(q, pool, layer, block_table, lengths, kv_groups, write_blocks, write_slots, k, v, out, workspace=None,
                      shared_blocks: bool = False) -> None:
    """write_tokens (BF16 pool) or Fp8KVPool.write (FP8 records) of each row's new token into
    `layer`, then run_kernel of that layer, as one decode launch where the shape allows
    (lk_paged_decode_append). The write position must be the row's last token, as the first
    two columns of PagedKVCache.decode_rows give it; that is not checked. Rows must name
    distinct blocks, and a row's token is written only if 1 <= its length <= the table's
    width x slots (decode_rows guarantees both). Enqueued on the current stream. shared_blocks
    as for decode_shape."""
    _check_layout(q, block_table, lengths, out)
    if _is_fp8(pool):
        storage, layers, kv_heads, head_dim = pool.records, pool.layers, pool.kv_heads, pool.head_dim
    else:
        if pool.dtype != torch.bfloat16:
            raise ValueError("a fused write needs a BF16 or FP8-record pool")
        storage, layers, kv_heads, head_dim = pool, pool.shape[2], pool.shape[3], pool.shape[5]
    batch = _check_token_write(storage.device, layers, kv_heads, head_dim, write_blocks, write_slots, layer, k, v)
    if batch != q.shape[0]:
        raise ValueError("one written token per decode row")
    lib = _lib.load()
    shape = decode_shape(q, pool, layer, block_table, kv_groups, lengths, shared_blocks)
    need = int(lib.lk_paged_decode_workspace(shape))
    if workspace is None or workspace.numel() < need:
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=q.device)
    _lib.check(
        lib.lk_paged_decode_append(shape, q.data_ptr(), storage.data_ptr(), block_table.data_ptr(), lengths.data_ptr(),
                                   write_blocks.data_ptr(), write_slots.data_ptr(), write_blocks.stride(0), k.data_ptr(), v.data_ptr(),
                                   out.data_ptr(), workspace.data_ptr(), workspace.numel(), _lib.current_stream(q.device))
    )


def _launch(q, pool, layer, block_table, lengths, kv_groups, shared_blocks: bool) -> torch.Tensor:
    q = q.contiguous()
    block_table = block_table.to(torch.int32).contiguous()
    lengths = lengths.to(torch.int32).contiguous()
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    run_kernel(q, pool, layer, block_table, lengths, kv_groups, out, shared_blocks=shared_blocks)
    return out


def paged_decode_attention_hip(q, pool, layer, block_table, lengths, kv_groups, shared_blocks: bool | None = None) -> torch.Tensor:
    """Drop-in for paged_decode_attention_triton: validated, result in q's dtype and device.
    shared_blocks (see decode_shape) left as None is decided from the validation's read-back:
    rows listing more blocks than the pool holds must share some of them."""
    listed = validate(q, pool, layer, block_table, lengths, kv_groups)
    if shared_blocks is None:
        shared_blocks = listed > pool.shape[0]
    return _launch(q, pool, layer, block_table, lengths, kv_groups, shared_blocks)


def paged_decode_attention_hip_trusted(q, pool, layer, block_table, lengths, kv_groups, shared_blocks: bool = False) -> torch.Tensor:
    """For tables whose lengths and ids the caller checked on the host (as
    PagedKVCache.decode_batch does): reads nothing back from the GPU. shared_blocks as for
    decode_shape; the caller knows whether its rows share blocks (forked prefixes)."""
    validate_shapes(q, pool, layer, block_table, lengths, kv_groups)
    return _launch(q, pool, layer, block_table, lengths, kv_groups, shared_blocks)
