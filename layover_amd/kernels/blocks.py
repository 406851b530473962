"""Block gather and scatter between a paged pool and contiguous staging on the GPU
(lk_gather_blocks / lk_scatter_blocks, include/layover_kernels.h): the BF16 swap's kernels,
the counterpart of the reference's gather_kernel / scatter_kernel (native/transfer_cuda.cu:
20-28), for callers that stage blocks themselves. Enqueued on torch's current stream."""

from __future__ import annotations

import torch

from layover_amd.kernels import _lib


def _block_args(pool: torch.Tensor, ids: torch.Tensor, staging: torch.Tensor) -> tuple[int, int]:
    if not (pool.is_cuda and ids.is_cuda and staging.is_cuda):
        raise ValueError("pool, ids and staging must be on the GPU")
    if not (pool.is_contiguous() and ids.is_contiguous() and staging.is_contiguous()):
        raise ValueError("pool, ids and staging must be contiguous")
    if ids.dtype not in (torch.int32, torch.uint32) or ids.dim() != 1:
        raise ValueError("ids must be a 1-D int32 tensor")
    block_bytes = pool[0].numel() * pool.element_size()
    count = ids.shape[0]
    if staging.numel() * staging.element_size() < count * block_bytes:
        raise ValueError(f"staging holds {staging.numel() * staging.element_size()} bytes, {count} blocks need {count * block_bytes}")
    return count, block_bytes


def gather_blocks(pool: torch.Tensor, ids: torch.Tensor, staging: torch.Tensor) -> None:
    """staging[i] = pool[ids[i]] as bytes, for every i."""
    count, block_bytes = _block_args(pool, ids, staging)
    _lib.check(_lib.load().lk_gather_blocks(pool.data_ptr(), ids.data_ptr(), count, block_bytes, staging.data_ptr(),
                                            _lib.current_stream(pool.device)))


def scatter_blocks(staging: torch.Tensor, ids: torch.Tensor, pool: torch.Tensor) -> None:
    """pool[ids[i]] = staging[i] as bytes, for every i."""
    count, block_bytes = _block_args(pool, ids, staging)
    _lib.check(_lib.load().lk_scatter_blocks(pool.data_ptr(), ids.data_ptr(), count, block_bytes, staging.data_ptr(),
                                             _lib.current_stream(pool.device)))
