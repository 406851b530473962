// Block gather and scatter between a paged pool and a contiguous staging buffer: the kernels
// of the BF16 swap (the reference's native/transfer_cuda.cu:20-28 and pack.h:41-68), shared
// by the transfer library (transfer_hip.hip, behind lt_out_gather / lt_in_scatter) and the
// kernel library (kernels.hip, lk_gather_blocks / lk_scatter_blocks).
//
// One workgroup of one wave moves one chunk of one block: 64 words, 1 KiB with 16-byte words
// (one load and one store per lane), 512 bytes with 8-byte words. grid.x = chunks per block x
// blocks, flattened. 16-byte words when pool, staging and block_bytes allow it, else 8-byte
// words (the ABI only promises 8-byte alignment). Loads and stores are non-temporal: every
// byte is moved once. Measured on MI355X, 56 random blocks of 2.36 MB of a 12 GiB pool per
// launch, back to back, with the staging side rotated over 1 GiB so that no launch finds it in
// the Infinity Cache: gather 40.7 us and scatter 41.1 us per launch (0.81 / 0.80 of 8 TB/s),
// against 50.3 / 53.4 us with 256-lane workgroups moving 64 KiB chunks (non-temporal loads,
// plain stores) and 44-47 us for 2-4 KiB or 64 KiB per workgroup with non-temporal stores.
#ifndef LAYOVER_AMD_BLOCK_COPY_H
#define LAYOVER_AMD_BLOCK_COPY_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace blockcopy {

constexpr uint32_t kLanes = 64;  // one wave per workgroup
typedef uint32_t Word16 __attribute__((ext_vector_type(4)));
typedef uint32_t Word8 __attribute__((ext_vector_type(2)));

template <class Word>
constexpr uint64_t chunk_bytes() {
    return uint64_t(kLanes) * sizeof(Word);
}

// This workgroup's chunk: lane l moves word l of it, if the block has that word.
template <class Word>
__device__ __forceinline__ void copy_word(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint64_t offset, uint64_t block_bytes) {
    const uint64_t at = offset + uint64_t(threadIdx.x) * sizeof(Word);
    if (at < block_bytes) __builtin_nontemporal_store(__builtin_nontemporal_load(reinterpret_cast<const Word*>(src + at)), reinterpret_cast<Word*>(dst + at));
}

template <class Word>
__global__ __launch_bounds__(kLanes) void gather_blocks(const uint8_t* __restrict__ pool, const uint32_t* __restrict__ ids,
                                                         uint8_t* __restrict__ staging, uint64_t block_bytes, uint32_t chunks_per_block) {
    const uint32_t index = blockIdx.x / chunks_per_block;
    const uint64_t offset = uint64_t(blockIdx.x % chunks_per_block) * chunk_bytes<Word>();
    copy_word<Word>(pool + uint64_t(ids[index]) * block_bytes, staging + uint64_t(index) * block_bytes, offset, block_bytes);
}

template <class Word>
__global__ __launch_bounds__(kLanes) void scatter_blocks(uint8_t* __restrict__ pool, const uint32_t* __restrict__ ids,
                                                          const uint8_t* __restrict__ staging, uint64_t block_bytes, uint32_t chunks_per_block) {
    const uint32_t index = blockIdx.x / chunks_per_block;
    const uint64_t offset = uint64_t(blockIdx.x % chunks_per_block) * chunk_bytes<Word>();
    copy_word<Word>(staging + uint64_t(index) * block_bytes, pool + uint64_t(ids[index]) * block_bytes, offset, block_bytes);
}

inline bool wide(const void* a, const void* b, uint64_t block_bytes) {
    return ((reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) | block_bytes) & 15) == 0;
}

// Chunks per block for the word size the launch will use; the 8-byte count bounds both.
inline uint64_t chunks_for(uint64_t block_bytes, bool wide_words) {
    const uint64_t chunk = wide_words ? chunk_bytes<Word16>() : chunk_bytes<Word8>();
    return (block_bytes + chunk - 1) / chunk;
}

// A launch moves at most this many chunks: a dispatch holds fewer than 2^32 work-items, one
// 64-lane workgroup per chunk.
constexpr uint64_t kMaxChunks = 0xFFFFFFFFull / kLanes;

// Whether `blocks` blocks of `block_bytes` fit one launch with either word size (the 8-byte
// count bounds both).
inline bool launch_fits(uint64_t block_bytes, uint64_t blocks) {
    const uint64_t chunks = chunks_for(block_bytes, false);
    return blocks == 0 || (chunks <= kMaxChunks && chunks * blocks <= kMaxChunks);
}

// Launch helpers: `blocks` blocks of `block_bytes` (a multiple of 8; pool and staging 8-byte
// aligned), ids[i] naming the pool block of staging slot i. The caller checks the arguments
// (launch_fits among them); a grid beyond one dispatch is refused here too.
inline hipError_t launch_gather(hipStream_t stream, const uint8_t* pool, const uint32_t* ids, uint8_t* staging, uint64_t block_bytes,
                                uint32_t blocks) {
    const bool w16 = wide(pool, staging, block_bytes);
    if (!launch_fits(block_bytes, blocks)) return hipErrorInvalidValue;
    const uint32_t chunks = uint32_t(chunks_for(block_bytes, w16));
    const dim3 grid(uint32_t(uint64_t(chunks) * blocks));
    if (w16)
        hipLaunchKernelGGL(gather_blocks<Word16>, grid, dim3(kLanes), 0, stream, pool, ids, staging, block_bytes, chunks);
    else
        hipLaunchKernelGGL(gather_blocks<Word8>, grid, dim3(kLanes), 0, stream, pool, ids, staging, block_bytes, chunks);
    return hipGetLastError();
}

inline hipError_t launch_scatter(hipStream_t stream, uint8_t* pool, const uint32_t* ids, const uint8_t* staging, uint64_t block_bytes,
                                 uint32_t blocks) {
    const bool w16 = wide(pool, staging, block_bytes);
    if (!launch_fits(block_bytes, blocks)) return hipErrorInvalidValue;
    const uint32_t chunks = uint32_t(chunks_for(block_bytes, w16));
    const dim3 grid(uint32_t(uint64_t(chunks) * blocks));
    if (w16)
        hipLaunchKernelGGL(scatter_blocks<Word16>, grid, dim3(kLanes), 0, stream, pool, ids, staging, block_bytes, chunks);
    else
        hipLaunchKernelGGL(scatter_blocks<Word8>, grid, dim3(kLanes), 0, stream, pool, ids, staging, block_bytes, chunks);
    return hipGetLastError();
}

}  // namespace blockcopy

#endif
