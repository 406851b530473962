// Paged GQA decode attention on gfx950: one query token per sequence against its block table,
// K/V read straight from the pool (BF16, FP32 or FP8 records), split-K over the context with a
// combine kernel. Replaces the reference's Triton kernel (layover/kernels/triton_decode.py:
// 39-119) and adds the FP8-record KV format.
//
// The math is the reference's online softmax (FlashAttention-2 style decode): running max m,
// running weight sum l and running weighted sum of V, in FP32, with slots at or past the
// sequence length excluded from the scores and their V zeroed (NaN-safe,
// triton_decode.py:97-109). Scores are kept in base 2 (scale * log2 e folded into one
// multiply) so the exponentials are single v_exp_f32 instructions.
//
// Fast path (16 slots x 128 dims, the Qwen3 shape; G = 1, 2, 4 or 8 query heads per KV head):
//   workgroup = (sequence, KV head, split of `bps` blocks), 4 waves taking the split's blocks
//   round-robin. Each K or V tile of a block (16 x 128) is read once for all G query heads:
//   no GQA re-reads, so HBM traffic is the "unique" bytes of bench/decode_bandwidth.py:
//   129-139. Lane l of a wave owns slots l/8 and l/8 + 8 and 16 of the 128 dims (c = l % 8):
//   for BF16, dims c*8..c*8+7 and 64+c*8..64+c*8+7, which makes each 16-byte load
//   instruction of the wave cover 8 whole 128-byte lines; for FP8, dims c*16..c*16+15.
//   A score is a dot product over the lane's 16 dims (v_dot2_f32_bf16 for BF16 q and K)
//   reduced over the 8 lanes of its slot with three DPP adds. Each lane keeps its own
//   online-softmax state per head (m, l, 16 accumulators) over the slots it sees, so no
//   per-tile cross-lane max is needed; the states of the 64 lanes and 4 waves are merged
//   once at the end of the split. The running max is only raised (with a rescale of the
//   accumulators) when a score exceeds it by more than 2^8, a wave-uniform branch that is
//   almost never taken after the first tile; weights are then at most 2^8, harmless in FP32.
//   FP8 tiles are dequantized in registers: codes -> FP32 by the hardware convert (exact),
//   the group's power of two folded into the score (K) and the weights (V). Groups whose
//   shift could leave BF16's normal range use the exact integer decode of fp8.py instead.
// Generic path (any slots <= 64 and head_dim <= 256, any G): one wave per (sequence, query
//   head, split), lane d owning dims d, d+64, ...; used for shapes other than Qwen3's.
// Combine: one wave per (sequence, query head) merges the split partials (m, l, acc) and
//   writes the output rounded to nearest even.
#ifndef LAYOVER_AMD_DECODE_ATTENTION_H
#define LAYOVER_AMD_DECODE_ATTENTION_H

#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "fp8_codec.h"
#include "layover_kernels.h"

namespace lk {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kRescaleThreshold = 8.0f;  // log2 units
constexpr uint32_t kDecodeWaves = 4;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xFFFF0000u); }

// Round to nearest even, NaN kept as the canonical quiet NaN.
__device__ __forceinline__ uint16_t to_bf16(float value) {
    const uint32_t bits = __float_as_uint(value);
    if ((bits & 0x7FFFFFFFu) > 0x7F800000u) return 0x7FC0;
    return uint16_t((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

template <int Ctrl>
__device__ __forceinline__ float dpp(float value) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(value), Ctrl, 0xF, 0xF, false));
}

// Sum over the 8 lanes l with equal l / 8: quad swaps, then mirror within the half-row.
__device__ __forceinline__ float sum8(float v) {
    v += dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp<0x141>(v);  // row_half_mirror
    return v;
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

// Weight of a partial state with running max m against the merged max top; an empty state
// (m = -inf) weighs nothing, even when every state is empty.
__device__ __forceinline__ float merge_weight(float m, float top) { return m == -INFINITY ? 0.0f : exp2_fast(m - top); }

struct DecodeArgs {
    const void* q;
    const uint8_t* pool;
    const int32_t* table;
    const int32_t* lengths;
    float* partial_acc;    // [batch, query_heads, splits, head_dim]
    float* partial_ml;     // [batch, query_heads, splits, 2]
    uint32_t batch, query_heads, kv_heads, head_dim, layers, slots, layer, table_width;
    uint32_t groups;       // query heads per KV head
    uint32_t splits;       // splits per sequence (grid)
    uint32_t bps;          // blocks per split
    uint64_t block_bytes;  // bytes from one pool block to the next
    float scale_log2;      // softmax scale * log2(e)
};

__device__ __forceinline__ uint32_t blocks_of(int32_t length, uint32_t slots) { return (uint32_t(length) + slots - 1) / slots; }

// ---------------------------------------------------------------------------------------
// Fast path: 16 slots x 128 dims.

constexpr uint32_t kSlots = 16;
constexpr uint32_t kDim = 128;

// The lane's 16 dims: index j of lane c -> head dim.
template <int KV>
__device__ __forceinline__ uint32_t lane_dim(uint32_t c, uint32_t j) {
    if (KV == LK_FP8_RECORD) return c * 16 + j;
    return j < 8 ? c * 8 + j : 64 + c * 8 + (j - 8);
}

// One slot's 16 values for this lane, raw: BF16 as 8 packed pairs, FP8 as 16 bytes, FP32 as
// 16 floats (bit patterns). `row` points at the slot's first element.
template <int KV>
struct SlotRaw;
template <>
struct SlotRaw<LK_BF16> {
    uint32_t w[8];
};
template <>
struct SlotRaw<LK_FP8_RECORD> {
    uint32_t w[4];
};
template <>
struct SlotRaw<LK_F32> {
    uint32_t w[16];
};

template <int KV>
__device__ __forceinline__ void load_slot(SlotRaw<KV>& raw, const uint8_t* row, uint32_t c) {
    if constexpr (KV == LK_BF16) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(row + c * 16);
        const u32x4 b = *reinterpret_cast<const u32x4*>(row + 128 + c * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            raw.w[i] = a[i];
            raw.w[4 + i] = b[i];
        }
    } else if constexpr (KV == LK_FP8_RECORD) {
        const u32x4 a = *reinterpret_cast<const u32x4*>(row + c * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) raw.w[i] = a[i];
    } else {
#pragma unroll
        for (int half = 0; half < 2; ++half)
#pragma unroll
            for (int quarter = 0; quarter < 2; ++quarter) {
                const u32x4 a = *reinterpret_cast<const u32x4*>(row + (half * 64 + c * 8 + quarter * 4) * 4);
#pragma unroll
                for (int i = 0; i < 4; ++i) raw.w[half * 8 + quarter * 4 + i] = a[i];
            }
    }
}

// The lane's 16 values of one slot as FP32 (FP8 codes unscaled: the group's power of two is
// applied by the caller, or `exact_shift` selects the exact integer decode for groups whose
// shift can leave BF16's normal range).
template <int KV>
__device__ __forceinline__ void unpack_slot(const SlotRaw<KV>& raw, float (&out)[16], bool exact, int32_t shift) {
    if constexpr (KV == LK_BF16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            out[2 * i] = bf16_lo(raw.w[i]);
            out[2 * i + 1] = bf16_hi(raw.w[i]);
        }
    } else if constexpr (KV == LK_FP8_RECORD) {
        if (!exact) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                out[4 * i + 0] = __builtin_amdgcn_cvt_f32_fp8(int(raw.w[i]), 0);
                out[4 * i + 1] = __builtin_amdgcn_cvt_f32_fp8(int(raw.w[i]), 1);
                out[4 * i + 2] = __builtin_amdgcn_cvt_f32_fp8(int(raw.w[i]), 2);
                out[4 * i + 3] = __builtin_amdgcn_cvt_f32_fp8(int(raw.w[i]), 3);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int b = 0; b < 4; ++b) out[4 * i + b] = __uint_as_float(decode_e4m3((raw.w[i] >> (8 * b)) & 0xFFu, shift) << 16);
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) out[i] = __uint_as_float(raw.w[i]);
    }
}

// A shift for which every E4M3 code times 2**shift is zero, NaN or a BF16 normal below
// 0x7F7F, so code * 2**shift in FP32 equals the reference's decode exactly.
__device__ __forceinline__ bool shift_is_exact_in_fp32(int32_t shift) { return shift >= -117 && shift <= 119; }

__device__ __forceinline__ float pow2(int32_t e) { return __uint_as_float(uint32_t(e + 127) << 23); }

// One (block, KV head) unit of a wave: the lane's share of the K and V tiles and, for FP8,
// the two group shifts.
template <int KV>
struct Tile {
    SlotRaw<KV> k[2];
    SlotRaw<KV> v[2];
    static constexpr int32_t k_shift = 0, v_shift = 0;
};
template <>
struct Tile<LK_FP8_RECORD> {
    SlotRaw<LK_FP8_RECORD> k[2];
    SlotRaw<LK_FP8_RECORD> v[2];
    int32_t k_shift, v_shift;
};

// BF16 pairs of a lane's 16 K values: BF16 tiles as loaded; FP8 codes by the exact hardware
// convert (every E4M3 value is a BF16 value), or, for groups whose shift can leave BF16's
// normal range, by the reference's integer decode with the shift applied.
template <int KV>
__device__ __forceinline__ void slot_bf16_pairs(const SlotRaw<KV>& raw, uint32_t (&pairs)[8], bool exact, int32_t shift) {
    if constexpr (KV == LK_BF16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) pairs[i] = raw.w[i];
    } else if constexpr (KV == LK_FP8_RECORD) {
        if (!exact) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pairs[2 * i] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw.w[i], 1.0f, false));
                pairs[2 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(raw.w[i], 1.0f, true));
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint32_t word = raw.w[i] >> (16 * h);
                    pairs[2 * i + h] = decode_e4m3(word & 0xFFu, shift) | (decode_e4m3((word >> 8) & 0xFFu, shift) << 16);
                }
            }
        }
    }
}

// Register buffers per wave (see the main loop of decode_split_fast).
#ifndef LK_DECODE_RING_BF16
#define LK_DECODE_RING_BF16 2
#endif
template <int KV>
struct RingDepth {
    static constexpr int value = KV == LK_BF16 ? LK_DECODE_RING_BF16 : 3;
};
#ifdef LK_DECODE_TWO_WAVES
#define LK_DECODE_OCCUPANCY __attribute__((amdgpu_waves_per_eu(2)))
#else
#define LK_DECODE_OCCUPANCY
#endif

template <int KV, int QF, int G>
__global__ __launch_bounds__(kWave* kDecodeWaves) LK_DECODE_OCCUPANCY void decode_split_fast(DecodeArgs a) {
    const uint32_t lane = threadIdx.x % kWave;
    // Wave-uniform by construction; readfirstlane tells the compiler, so everything derived
    // from it (block ids, tile addresses' uniform part) goes through scalar loads and
    // registers. A vector load of a block id would otherwise have to wait for every tile
    // load in flight before it (loads retire in order), draining the pipeline each unit.
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t c = lane % 8;       // dim group
    const uint32_t row = lane / 8;     // slots row and row + 8
    const uint32_t split = blockIdx.x % a.splits;
    const uint32_t pair = blockIdx.x / a.splits;
    const uint32_t kv_head = pair % a.kv_heads;
    const uint32_t seq = pair / a.kv_heads;

    const int32_t length = a.lengths[seq];
    const uint32_t nblocks = blocks_of(length, kSlots);
    const uint32_t first = split * a.bps;
    if (first >= nblocks) return;
    const uint32_t count = min(a.bps, nblocks - first);

    // q for the G heads of this KV head, this lane's 16 dims, in FP32; BF16 q also packed.
    // The lane's dims are runs of 8 (BF16 tiles) or 16 (FP8) consecutive ones: 16-byte loads.
    float qf[G][16];
    uint32_t qp[G][8];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        const uint64_t row_at = (uint64_t(seq) * a.query_heads + kv_head * G + h) * kDim;
#pragma unroll
        for (int run = 0; run < 2; ++run) {
            const uint32_t d0 = lane_dim<KV>(c, 8 * run);
            if constexpr (QF == LK_BF16) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.q) + row_at + d0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    qp[h][4 * run + i] = w[i];
                    qf[h][8 * run + 2 * i] = bf16_lo(w[i]);
                    qf[h][8 * run + 2 * i + 1] = bf16_hi(w[i]);
                }
            } else {
                const float* src = reinterpret_cast<const float*>(a.q) + row_at + d0;
#pragma unroll
                for (int quarter = 0; quarter < 2; ++quarter) {
                    const u32x4 w = *reinterpret_cast<const u32x4*>(src + 4 * quarter);
#pragma unroll
                    for (int i = 0; i < 4; ++i) qf[h][8 * run + 4 * quarter + i] = __uint_as_float(w[i]);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    qp[h][4 * run + i] = (__float_as_uint(qf[h][8 * run + 2 * i]) >> 16) | (__float_as_uint(qf[h][8 * run + 2 * i + 1]) & 0xFFFF0000u);
            }
        }
    }

    constexpr uint32_t kElem = KV == LK_FP8_RECORD ? 1 : (KV == LK_F32 ? 4 : 2);
    const uint64_t tile_bytes = uint64_t(kSlots) * kDim * kElem;
    const uint64_t head_tile = uint64_t(a.layer) * a.kv_heads + kv_head;  // group index of K
    const uint64_t k_offset = head_tile * tile_bytes + uint64_t(row) * kDim * kElem;
    const uint64_t v_offset = (uint64_t(a.layers) * a.kv_heads + head_tile) * tile_bytes + uint64_t(row) * kDim * kElem;
    const uint64_t half_offset = 8ull * kDim * kElem;                            // slot row + 8
    const uint64_t block_elems = uint64_t(2) * a.layers * a.kv_heads * kSlots * kDim;  // FP8: shifts follow the data
    const int32_t* row_ids = a.table + uint64_t(seq) * a.table_width + first;

    float m[G], l[G], acc[G][16];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        m[h] = -INFINITY;
        l[h] = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[h][j] = 0.0f;
    }

    // The block ids of this wave's units, one per lane (a wave has at most 64 units:
    // blocks per split <= 256), loaded once before any tile and read back with v_readlane.
    const uint32_t mine = count > wave ? (count - wave + kDecodeWaves - 1) / kDecodeWaves : 0;
    const int32_t my_block = lane < mine ? row_ids[wave + lane * kDecodeWaves] : 0;
    // FP8: the unit's two group shifts, likewise one unit per lane, so no load in the main
    // loop has to be waited for before the tile loads issued ahead of it.
    int32_t my_k_shift = 0, my_v_shift = 0;
    if constexpr (KV == LK_FP8_RECORD) {
        if (lane < mine) {
            const int16_t* shifts = reinterpret_cast<const int16_t*>(a.pool + uint64_t(uint32_t(my_block)) * a.block_bytes + block_elems);
            my_k_shift = shifts[head_tile];
            my_v_shift = shifts[uint64_t(a.layers) * a.kv_heads + head_tile];
        }
    }

    auto fetch = [&](Tile<KV>& tile, uint32_t i) {
        const int32_t block = __builtin_amdgcn_readlane(my_block, i);
        const uint8_t* base = a.pool + uint64_t(uint32_t(block)) * a.block_bytes;
        load_slot<KV>(tile.k[0], base + k_offset, c);
        load_slot<KV>(tile.k[1], base + k_offset + half_offset, c);
        load_slot<KV>(tile.v[0], base + v_offset, c);
        load_slot<KV>(tile.v[1], base + v_offset + half_offset, c);
        if constexpr (KV == LK_FP8_RECORD) {
            tile.k_shift = __builtin_amdgcn_readlane(my_k_shift, i);
            tile.v_shift = __builtin_amdgcn_readlane(my_v_shift, i);
        }
    };

    // The unit of tile t: scores, online-softmax update, weighted V.
    auto consume = [&](const Tile<KV>& tile, uint32_t t) {
        const uint32_t token0 = (first + t) * kSlots;
        const bool partial = token0 + kSlots > uint32_t(length);
        const bool visible[2] = {token0 + row < uint32_t(length), token0 + row + 8 < uint32_t(length)};

        float score[G][2];
        bool k_exact = false;
        float k_factor = a.scale_log2;
        if constexpr (KV == LK_FP8_RECORD) {
            k_exact = !shift_is_exact_in_fp32(tile.k_shift);
            if (!k_exact) k_factor *= pow2(tile.k_shift);
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float dot[G];
            if constexpr (KV != LK_F32 && QF == LK_BF16) {
                uint32_t pairs[8];
                slot_bf16_pairs<KV>(tile.k[half], pairs, k_exact, tile.k_shift);
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    float s = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pairs[i]), __builtin_bit_cast(bf16x2, qp[h][i]), s, false);
                    dot[h] = s;
                }
            } else {
                float kv[16];
                unpack_slot<KV>(tile.k[half], kv, k_exact, tile.k_shift);
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    float s = 0.0f;
#pragma unroll
                    for (int j = 0; j < 16; ++j) s = fmaf(qf[h][j], kv[j], s);
                    dot[h] = s;
                }
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float s = sum8(dot[h]) * k_factor;
                score[h][half] = visible[half] ? s : -INFINITY;
            }
        }

        // Raise the running max only when a score passes it by more than 2^8.
        bool raise = false;
#pragma unroll
        for (int h = 0; h < G; ++h) raise |= fmaxf(score[h][0], score[h][1]) > m[h] + kRescaleThreshold;
        if (__builtin_expect(__any(raise), 0)) {
            // Kept as a branch: flattened, its multiplies would run on every unit.
            asm volatile("" ::: "memory");
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float top = fmaxf(score[h][0], score[h][1]);
                const float next = top > m[h] + kRescaleThreshold ? top : m[h];
                const float alpha = merge_weight(m[h], next);
                m[h] = next;
                l[h] *= alpha;
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[h][j] *= alpha;
            }
        }

        bool v_exact = false;
        float v_factor = 1.0f;
        if constexpr (KV == LK_FP8_RECORD) {
            v_exact = !shift_is_exact_in_fp32(tile.v_shift);
            if (!v_exact) v_factor = pow2(tile.v_shift);
        }
#pragma unroll
        for (int half = 0; half < 2; ++half) {
            float vv[16];
            unpack_slot<KV>(tile.v[half], vv, v_exact, tile.v_shift);
            if (partial && !visible[half]) {
#pragma unroll
                for (int j = 0; j < 16; ++j) vv[j] = 0.0f;
            }
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float p = score[h][half] == -INFINITY ? 0.0f : exp2_fast(score[h][half] - m[h]);
                l[h] += p;
                const float pv = p * v_factor;
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[h][j] = fmaf(pv, vv[j], acc[h][j]);
            }
        }
    };

    // This wave's units are t = wave, wave + 4, ...: a ring of kRing register buffers, each
    // refilled as soon as it is consumed, keeps kRing - 1 units' loads in flight while one
    // computes.
    constexpr int kRing = RingDepth<KV>::value;
    Tile<KV> ring[kRing];
    auto unit = [&](uint32_t i) { return wave + i * kDecodeWaves; };
    // Refills are unconditional: past the wave's last unit they re-read that unit (an L2 hit),
    // because a conditional load would make every later wait assume it might not have been
    // issued, i.e. wait for all loads in flight.
    if (mine > 0) {
        const uint32_t last = mine - 1;
#pragma unroll
        for (int d = 0; d < kRing; ++d) fetch(ring[d], min(uint32_t(d), last));
        for (uint32_t i = 0; i < mine; i += kRing) {
#pragma unroll
            for (int d = 0; d < kRing; ++d) {
                if (i + d < mine) consume(ring[d], unit(i + d));
                fetch(ring[d], min(i + d + kRing, last));
            }
        }
    }

    // Merge the 8 rows of lanes (slots) of this wave: lanes with equal c.
    __shared__ float s_acc[kDecodeWaves][G][kDim];
    __shared__ float s_m[kDecodeWaves][G];
    __shared__ float s_l[kDecodeWaves][G];
#pragma unroll
    for (int h = 0; h < G; ++h) {
        float top = m[h];
#pragma unroll
        for (int mask = 8; mask <= 32; mask <<= 1) top = fmaxf(top, __shfl_xor(top, mask, kWave));
        const float w = merge_weight(m[h], top);
        float lsum = l[h] * w;
#pragma unroll
        for (int mask = 8; mask <= 32; mask <<= 1) lsum += __shfl_xor(lsum, mask, kWave);
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            float v = acc[h][j] * w;
#pragma unroll
            for (int mask = 8; mask <= 32; mask <<= 1) v += __shfl_xor(v, mask, kWave);
            acc[h][j] = v;
        }
        if (row == 0) {
#pragma unroll
            for (int j = 0; j < 16; ++j) s_acc[wave][h][lane_dim<KV>(c, j)] = acc[h][j];
        }
        if (lane == 0) {
            s_m[wave][h] = top;
            s_l[wave][h] = lsum;
        }
    }
    __syncthreads();

    // Merge the waves and write this split's partial state for each query head.
    for (uint32_t e = threadIdx.x; e < G * kDim; e += kWave * kDecodeWaves) {
        const uint32_t h = e / kDim, d = e % kDim;
        float top = -INFINITY;
#pragma unroll
        for (int w = 0; w < int(kDecodeWaves); ++w) top = fmaxf(top, s_m[w][h]);
        float sum = 0.0f, lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < int(kDecodeWaves); ++w) {
            const float weight = merge_weight(s_m[w][h], top);
            sum += s_acc[w][h][d] * weight;
            lsum += s_l[w][h] * weight;
        }
        const uint64_t slot = (uint64_t(seq) * a.query_heads + kv_head * G + h) * a.splits + split;
        a.partial_acc[slot * kDim + d] = sum;
        if (d == 0) {
            a.partial_ml[2 * slot] = top;
            a.partial_ml[2 * slot + 1] = lsum;
        }
    }
}

// ---------------------------------------------------------------------------------------
// Generic path: one wave per (sequence, query head, split), lane d owns dims d, d + 64, ...

template <int KV>
__device__ __forceinline__ float kv_element(const uint8_t* tile, uint32_t index, int32_t shift) {
    if constexpr (KV == LK_BF16) return __uint_as_float(uint32_t(reinterpret_cast<const uint16_t*>(tile)[index]) << 16);
    else if constexpr (KV == LK_F32) return reinterpret_cast<const float*>(tile)[index];
    else return __uint_as_float(decode_e4m3(tile[index], shift) << 16);
}

constexpr uint32_t kMaxGenericDim = 256;

template <int KV, int QF>
__global__ __launch_bounds__(kWave) void decode_split_generic(DecodeArgs a) {
    const uint32_t lane = threadIdx.x;
    const uint32_t split = blockIdx.x % a.splits;
    const uint32_t pair = blockIdx.x / a.splits;
    const uint32_t qh = pair % a.query_heads;
    const uint32_t seq = pair / a.query_heads;
    const uint32_t kv_head = qh / a.groups;
    const int32_t length = a.lengths[seq];
    const uint32_t nblocks = blocks_of(length, a.slots);
    const uint32_t first = split * a.bps;
    if (first >= nblocks) return;
    const uint32_t last = min(nblocks, first + a.bps);

    constexpr uint32_t kElem = KV == LK_FP8_RECORD ? 1 : (KV == LK_F32 ? 4 : 2);
    constexpr uint32_t kPer = kMaxGenericDim / kWave;
    float q[kPer], acc[kPer];
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
        const uint32_t d = lane + i * kWave;
        acc[i] = 0.0f;
        q[i] = 0.0f;
        if (d < a.head_dim) {
            const uint64_t at = (uint64_t(seq) * a.query_heads + qh) * a.head_dim + d;
            q[i] = QF == LK_BF16 ? __uint_as_float(uint32_t(reinterpret_cast<const uint16_t*>(a.q)[at]) << 16)
                                 : reinterpret_cast<const float*>(a.q)[at];
        }
    }
    const uint64_t tile_elems = uint64_t(a.slots) * a.head_dim;
    const uint64_t head_tile = uint64_t(a.layer) * a.kv_heads + kv_head;
    const uint64_t v_group = uint64_t(a.layers) * a.kv_heads + head_tile;
    const uint64_t block_elems = 2ull * a.layers * a.kv_heads * tile_elems;

    float m = -INFINITY, l = 0.0f;
    for (uint32_t b = first; b < last; ++b) {
        const uint8_t* base = a.pool + uint64_t(a.table[uint64_t(seq) * a.table_width + b]) * a.block_bytes;
        const uint8_t* k_tile = base + head_tile * tile_elems * kElem;
        const uint8_t* v_tile = base + v_group * tile_elems * kElem;
        int32_t ks = 0, vs = 0;
        if constexpr (KV == LK_FP8_RECORD) {
            const uint8_t* shifts = base + block_elems;
            ks = int16_t(uint16_t(shifts[2 * head_tile]) | uint16_t(shifts[2 * head_tile + 1] << 8));
            vs = int16_t(uint16_t(shifts[2 * v_group]) | uint16_t(shifts[2 * v_group + 1] << 8));
        }
        const uint32_t visible = min(a.slots, uint32_t(length) - b * a.slots);
        for (uint32_t s = 0; s < visible; ++s) {
            float dot = 0.0f;
#pragma unroll
            for (uint32_t i = 0; i < kPer; ++i) {
                const uint32_t d = lane + i * kWave;
                if (d < a.head_dim) dot = fmaf(q[i], kv_element<KV>(k_tile, s * a.head_dim + d, ks), dot);
            }
#pragma unroll
            for (int mask = 32; mask >= 1; mask >>= 1) dot += __shfl_xor(dot, mask, kWave);
            const float score = dot * a.scale_log2;
            const float next = fmaxf(m, score);
            const float alpha = merge_weight(m, next);
            const float p = exp2_fast(score - next);
            l = l * alpha + p;
#pragma unroll
            for (uint32_t i = 0; i < kPer; ++i) {
                const uint32_t d = lane + i * kWave;
                const float v = d < a.head_dim ? kv_element<KV>(v_tile, s * a.head_dim + d, vs) : 0.0f;
                acc[i] = fmaf(p, v, acc[i] * alpha);
            }
            m = next;
        }
    }
    const uint64_t slot = (uint64_t(seq) * a.query_heads + qh) * a.splits + split;
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
        const uint32_t d = lane + i * kWave;
        if (d < a.head_dim) a.partial_acc[slot * a.head_dim + d] = acc[i];
    }
    if (lane == 0) {
        a.partial_ml[2 * slot] = m;
        a.partial_ml[2 * slot + 1] = l;
    }
}

// ---------------------------------------------------------------------------------------
// Combine: out[seq, qh] = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).

template <int QF>
__global__ __launch_bounds__(kWave) void decode_combine(DecodeArgs a, void* out) {
    const uint32_t lane = threadIdx.x;
    const uint32_t qh = blockIdx.x % a.query_heads;
    const uint32_t seq = blockIdx.x / a.query_heads;
    const uint32_t used = (blocks_of(a.lengths[seq], a.slots) + a.bps - 1) / a.bps;
    const uint64_t base = (uint64_t(seq) * a.query_heads + qh) * a.splits;
    const float* ml = a.partial_ml + 2 * base;

    // Lanes across splits: the largest running max, then the total weight.
    float top = -INFINITY;
    for (uint32_t s = lane; s < used; s += kWave) top = fmaxf(top, ml[2 * s]);
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) top = fmaxf(top, __shfl_xor(top, mask, kWave));
    float total = 0.0f;
    for (uint32_t s = lane; s < used; s += kWave) total += ml[2 * s + 1] * merge_weight(ml[2 * s], top);
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) total += __shfl_xor(total, mask, kWave);
    const float inverse = 1.0f / total;

    // Lanes across dims: sum the splits' accumulators, 64 splits' weights at a time, each
    // broadcast from the lane that computed it.
    constexpr uint32_t kPer = kMaxGenericDim / kWave;
    float sum[kPer];
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) sum[i] = 0.0f;
    const float* acc = a.partial_acc + base * a.head_dim;
    for (uint32_t chunk = 0; chunk < used; chunk += kWave) {
        const uint32_t s = chunk + lane;
        const float weight = s < used ? merge_weight(ml[2 * s], top) : 0.0f;
        const uint32_t n = min(kWave, used - chunk);
        for (uint32_t j = 0; j < n; ++j) {
            const float w = __shfl(weight, j, kWave);
            const float* row = acc + uint64_t(chunk + j) * a.head_dim;
#pragma unroll
            for (uint32_t i = 0; i < kPer; ++i) {
                const uint32_t d = lane + i * kWave;
                if (d < a.head_dim) sum[i] = fmaf(w, row[d], sum[i]);
            }
        }
    }
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) {
        const uint32_t d = lane + i * kWave;
        if (d >= a.head_dim) continue;
        const float value = sum[i] * inverse;
        const uint64_t at = (uint64_t(seq) * a.query_heads + qh) * a.head_dim + d;
        if constexpr (QF == LK_BF16) reinterpret_cast<uint16_t*>(out)[at] = to_bf16(value);
        else reinterpret_cast<float*>(out)[at] = value;
    }
}

}  // namespace lk

#endif  // LAYOVER_AMD_DECODE_ATTENTION_H
