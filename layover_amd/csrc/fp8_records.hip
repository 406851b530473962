// Fused gather+quantize and dequantize+scatter of Qwen3-shaped FP8 records (2048-value
// groups, 16-byte aligned records), the kernels of lk_fp8_quantize / lk_fp8_dequantize.
//
// This translation unit is compiled with FP32 denormals flushed to zero (Makefile), which
// the fast path relies on. Each wave takes one group:
//
// quantize: one pass over the group's 32 values per lane computes, on BF16 pairs packed in
//   32-bit words, the masked exponent plus one step (so infinity/NaN wrap to 0 and set bit
//   15 of their half, flagging the group) and a packed 16-bit max; a wave max gives the
//   shift (fp8.py:86-92). Then, when the group has no infinity/NaN and shift >= -126:
//     code = cvt_fp8_e4m3_rne(float(bf16) * 2^-shift)     (v_cvt_pk_fp8_f32)
//   float(bf16) * 2^-shift is exact (a BF16 value times a power of two), so the one
//   rounding is the convert's round-to-nearest-even, as in fp8.py:103-109; BF16
//   subnormals are flushed to signed zero by the multiply (denormals off), as fp8.py:114
//   requires; and the computed shift keeps every value below 2^8, far from E4M3's 448, so
//   nothing saturates. Other groups run the reference's integer codec (encode_e4m3).
// dequantize: with no NaN code in the group (a SWAR byte test) and a shift in [-117, 119],
//     bf16 = high half of float(e4m3) * 2^shift              (v_cvt_pk_f32_fp8, v_perm)
//   is exact: every E4M3 value times such a power of two is a BF16 normal (or zero) below
//   0x7F7F, so fp8.py:133-134's saturation and flush never apply. Otherwise decode_e4m3.
// Both fast paths are checked bit for bit against the integer codec on every BF16 pattern
// at every shift the computed scale can take (tests/test_gpu_kernels.py).
// Loads and stores are non-temporal: each byte is touched once, and the outputs (records for
// the copy engine, restored blocks) are not read again soon. Measured on MI355X at the
// bench's 113-block launches, non-temporal stores gained quantize about 1 and dequantize
// about 4 points of the 8 TB/s peak (with the rest of today's kernels they run at 0.78 and
// 0.74-0.75 of it, 0.91 and 0.89 of a plain stream with the same read/write mix).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fp8_codec.h"

namespace lk {

typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float power_of_two(int32_t e) { return __uint_as_float(uint32_t(e + 127) << 23); }

// This wave's contiguous run of groups [first, stop) out of `total`: consecutive groups of a
// block share its id, and a wave's next group is the next 4 KiB of the same block.
__device__ __forceinline__ bool wave_range(uint64_t total, uint64_t& first, uint64_t& stop) {
    const uint64_t waves = uint64_t(gridDim.x) * kRecordWaves;
    // readfirstlane: the wave index is uniform, so group indices and block-id reads stay in
    // scalar registers and scalar loads, whose waits do not wait on the vector loads in flight.
    const uint64_t wave = uint64_t(blockIdx.x) * kRecordWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint64_t per = (total + waves - 1) / waves;
    first = wave * per;
    stop = first + per < total ? first + per : total;
    return first < stop;
}

struct QuantizeLoad {
    u32x4 words[4];
    uint64_t group;
};

// The loads of one group: its 4 KiB of BF16, 4 x 16 bytes per lane.
__device__ __forceinline__ void quantize_load(const uint16_t* __restrict__ pool, const int32_t* __restrict__ ids, uint32_t groups_per_block,
                                              uint64_t group, uint32_t lane, QuantizeLoad& in) {
    const uint32_t index = uint32_t(group / groups_per_block);
    const uint32_t g = uint32_t(group % groups_per_block);
    const uint64_t block_elems = uint64_t(kFastGroup) * groups_per_block;
    const u32x4* source = reinterpret_cast<const u32x4*>(pool + uint64_t(ids[index]) * block_elems + uint64_t(g) * kFastGroup);
#pragma unroll
    for (int j = 0; j < 4; ++j) in.words[j] = __builtin_nontemporal_load(source + j * kWave + lane);
    in.group = group;
}

// Shift, codes and their stores for a loaded group.
__device__ __forceinline__ void quantize_finish(uint8_t* __restrict__ stage, uint32_t groups_per_block, uint32_t lane, const QuantizeLoad& in) {
    const uint64_t group = in.group;
    const uint32_t index = uint32_t(group / groups_per_block);
    const uint32_t g = uint32_t(group % groups_per_block);
    const uint64_t block_elems = uint64_t(kFastGroup) * groups_per_block;
    const uint64_t record = block_elems + 2ull * groups_per_block;
    const u32x4* words = in.words;

    u16x2 keys = {0, 0};
    uint32_t flags = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t stepped = (words[j][w] & 0x7F807F80u) + 0x00800080u;
            flags |= stepped;
            keys = __builtin_elementwise_max(keys, __builtin_bit_cast(u16x2, stepped & 0x7FFF7FFFu));
        }
    const uint32_t lane_key = uint32_t(keys.x > keys.y ? keys.x : keys.y) >> 7;
    const int32_t shift = shift_from_key(wave_max(lane_key));
    const bool nonfinite = __any((flags & 0x80008000u) != 0);

    uint8_t* out = stage + uint64_t(index) * record;
    u32x2* codes = reinterpret_cast<u32x2*>(out + uint64_t(g) * kFastGroup);
    if (!nonfinite && shift >= -126) {
        const float scale = power_of_two(-shift);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t packed[2];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const uint32_t a = words[j][2 * half], b = words[j][2 * half + 1];
                int p = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(a << 16) * scale, __uint_as_float(a & 0xFFFF0000u) * scale, 0, false);
                p = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(b << 16) * scale, __uint_as_float(b & 0xFFFF0000u) * scale, p, true);
                packed[half] = uint32_t(p);
            }
            __builtin_nontemporal_store(u32x2{packed[0], packed[1]}, codes + j * kWave + lane);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t packed[2];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const uint32_t a = words[j][2 * half], b = words[j][2 * half + 1];
                packed[half] = encode_e4m3(a & 0xFFFFu, shift) | (encode_e4m3(a >> 16, shift) << 8) |
                               (encode_e4m3(b & 0xFFFFu, shift) << 16) | (encode_e4m3(b >> 16, shift) << 24);
            }
            __builtin_nontemporal_store(u32x2{packed[0], packed[1]}, codes + j * kWave + lane);
        }
    }
    if (lane == 0) *reinterpret_cast<int16_t*>(out + block_elems + 2ull * g) = int16_t(shift);
}

__global__ __launch_bounds__(kWave* kRecordWaves) void quantize_groups_2048(const uint16_t* __restrict__ pool,
                                                                         const int32_t* __restrict__ ids, uint8_t* __restrict__ stage,
                                                                         uint32_t count, uint32_t groups_per_block) {
    const uint32_t lane = threadIdx.x % kWave;
    uint64_t group, stop;
    if (!wave_range(uint64_t(count) * groups_per_block, group, stop)) return;
    // Software-pipelined over two buffers that swap roles (no register copies, which would
    // wait for the prefetched data): the next group's loads are in flight while one converts.
    QuantizeLoad even, odd;
    quantize_load(pool, ids, groups_per_block, group, lane, even);
    while (true) {
        if (group + 1 >= stop) {
            quantize_finish(stage, groups_per_block, lane, even);
            return;
        }
        quantize_load(pool, ids, groups_per_block, group + 1, lane, odd);
        quantize_finish(stage, groups_per_block, lane, even);
        if (++group + 1 >= stop) {
            quantize_finish(stage, groups_per_block, lane, odd);
            return;
        }
        quantize_load(pool, ids, groups_per_block, group + 1, lane, even);
        quantize_finish(stage, groups_per_block, lane, odd);
        ++group;
    }
}

struct DequantizeLoad {
    u32x2 bytes[4];
    int32_t shift;
    int32_t block;
    uint64_t group;
};

// The loads of one record group: 2 KiB of codes (4 x 8 bytes per lane), its shift, its block.
__device__ __forceinline__ void dequantize_load(const uint8_t* __restrict__ stage, const int32_t* __restrict__ ids, uint32_t groups_per_block,
                                                uint64_t group, uint32_t lane, DequantizeLoad& in) {
    const uint32_t index = uint32_t(group / groups_per_block);
    const uint32_t g = uint32_t(group % groups_per_block);
    const uint64_t block_elems = uint64_t(kFastGroup) * groups_per_block;
    const uint64_t record = block_elems + 2ull * groups_per_block;
    const uint8_t* base = stage + uint64_t(index) * record;
    const u32x2* codes = reinterpret_cast<const u32x2*>(base + uint64_t(g) * kFastGroup);
#pragma unroll
    for (int j = 0; j < 4; ++j) in.bytes[j] = __builtin_nontemporal_load(codes + j * kWave + lane);
    in.shift = *reinterpret_cast<const int16_t*>(base + block_elems + 2ull * g);
    in.block = ids[index];
    in.group = group;
}

// One group's codes (lane's 4 x 8 bytes) at `shift` to BF16, stored as 4 x 16 bytes per lane
// at `target` (2,048 values); non-temporal stores unless the values are read again soon.
template <bool kNontemporal = true>
__device__ __forceinline__ void store_bf16(u32x4* target, u32x4 value) {
    if constexpr (kNontemporal) __builtin_nontemporal_store(value, target);
    else *target = value;
}

template <bool kNontemporal = true>
__device__ __forceinline__ void decode_group_to(u32x4* __restrict__ target, int32_t shift, const u32x2* bytes, uint32_t lane) {
    // A byte 0x7F or 0xFF (NaN) becomes 0x80 after masking off its sign and adding one.
    uint32_t flags = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) flags |= ((bytes[j][0] & 0x7F7F7F7Fu) + 0x01010101u) | ((bytes[j][1] & 0x7F7F7F7Fu) + 0x01010101u);
    const bool any_nan = __any((flags & 0x80808080u) != 0);

    if (!any_nan && shift >= -117 && shift <= 119) {
        // Two codes to a BF16 pair in one scaled convert (v_cvt_scalef32_pk_bf16_fp8): the
        // scale is an exact power of two and every product is a BF16 normal or zero, so the
        // result is exact, as the float path it replaces (two converts to FP32, four
        // multiplies, two permutes per four codes) was.
        const float scale = power_of_two(shift);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            u32x4 out;
#pragma unroll
            for (int w = 0; w < 2; ++w) {
                const uint32_t word = bytes[j][w];
                out[2 * w] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, scale, false));
                out[2 * w + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, scale, true));
            }
            store_bf16<kNontemporal>(target + j * kWave + lane, out);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            u32x4 out;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t word = bytes[j][w / 2] >> (16 * (w % 2));
                out[w] = decode_e4m3(word & 0xFFu, shift) | (decode_e4m3((word >> 8) & 0xFFu, shift) << 16);
            }
            store_bf16<kNontemporal>(target + j * kWave + lane, out);
        }
    }
}

__device__ __forceinline__ void dequantize_finish(uint16_t* __restrict__ pool, uint32_t groups_per_block, uint32_t lane, const DequantizeLoad& in) {
    const uint32_t g = uint32_t(in.group % groups_per_block);
    const uint64_t block_elems = uint64_t(kFastGroup) * groups_per_block;
    decode_group_to(reinterpret_cast<u32x4*>(pool + uint64_t(uint32_t(in.block)) * block_elems + uint64_t(g) * kFastGroup), in.shift, in.bytes,
                    lane);
}

__global__ __launch_bounds__(kWave* kRecordWaves) void dequantize_groups_2048(const uint8_t* __restrict__ stage,
                                                                           const int32_t* __restrict__ ids, uint16_t* __restrict__ pool,
                                                                           uint32_t count, uint32_t groups_per_block) {
    const uint32_t lane = threadIdx.x % kWave;
    uint64_t group, stop;
    if (!wave_range(uint64_t(count) * groups_per_block, group, stop)) return;
    DequantizeLoad even, odd;
    dequantize_load(stage, ids, groups_per_block, group, lane, even);
    while (true) {
        if (group + 1 >= stop) {
            dequantize_finish(pool, groups_per_block, lane, even);
            return;
        }
        dequantize_load(stage, ids, groups_per_block, group + 1, lane, odd);
        dequantize_finish(pool, groups_per_block, lane, even);
        if (++group + 1 >= stop) {
            dequantize_finish(pool, groups_per_block, lane, odd);
            return;
        }
        dequantize_load(stage, ids, groups_per_block, group + 1, lane, even);
        dequantize_finish(pool, groups_per_block, lane, odd);
        ++group;
    }
}

// One layer of a sequence's history, FP8 records to BF16 for the paged prefill: wave w takes
// group (block b, kind, KV head) = (w / (2 kv_heads), w / kv_heads % 2, w % kv_heads) of
// block ids[b], and writes it to stage[b][kind][head] (16 x 128 BF16, a one-layer pool block);
// the first wave of each block also writes index[b] = b. Same decode, bit for bit, as
// dequantize_groups_2048. kWide: the records are 8-byte aligned and the codes are read 8 bytes
// a lane; otherwise (records of a layout whose size is not a multiple of 8, always even) the
// same bytes are read 2 at a time.
template <bool kWide>
__global__ __launch_bounds__(kWave* kCodecWaves) void stage_history_2048(const uint8_t* __restrict__ records,
                                                                       const int32_t* __restrict__ ids, uint64_t record_bytes,
                                                                       uint32_t groups_per_block, uint32_t layer, uint32_t layers,
                                                                       uint32_t kv_heads, uint32_t blocks, uint16_t* __restrict__ stage,
                                                                       int32_t* __restrict__ index) {
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t unit = uint64_t(blockIdx.x) * kCodecWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (unit >= uint64_t(blocks) * 2 * kv_heads) return;
    const uint32_t b = uint32_t(unit / (2 * kv_heads));
    const uint32_t kind = uint32_t(unit / kv_heads % 2), head = uint32_t(unit % kv_heads);
    const uint8_t* record = records + uint64_t(uint32_t(ids[b])) * record_bytes;
    const uint64_t group = (uint64_t(kind) * layers + layer) * kv_heads + head;
    u32x2 bytes[4];
    if constexpr (kWide) {
        const u32x2* codes = reinterpret_cast<const u32x2*>(record + group * kFastGroup);
#pragma unroll
        for (int j = 0; j < 4; ++j) bytes[j] = __builtin_nontemporal_load(codes + j * kWave + lane);
    } else {
        const uint16_t* codes = reinterpret_cast<const uint16_t*>(record + group * kFastGroup);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint16_t* word = codes + 4 * (j * kWave + lane);
            bytes[j] = u32x2{uint32_t(word[0]) | uint32_t(word[1]) << 16, uint32_t(word[2]) | uint32_t(word[3]) << 16};
        }
    }
    const int32_t shift = reinterpret_cast<const int16_t*>(record + uint64_t(kFastGroup) * groups_per_block)[group];
    decode_group_to<false>(reinterpret_cast<u32x4*>(stage + unit * kFastGroup), shift, bytes, lane);
    if (unit % (2 * kv_heads) == 0 && lane == 0) index[b] = int32_t(b);
}

// One token per row written into Qwen3-shaped records (lk_fp8_append): one wave per (row,
// kind, KV head) group, running append_group_2048. The new token's loads need only the row
// and go out with the write position's; the old codes and shift follow.
__global__ __launch_bounds__(kWave* kCodecWaves) void append_groups_2048(uint8_t* __restrict__ records, const int32_t* __restrict__ write_block,
                                                                       const int32_t* __restrict__ write_slot, uint32_t row_stride,
                                                                       uint32_t batch, const uint16_t* __restrict__ k,
                                                                       const uint16_t* __restrict__ v, uint32_t layer, uint32_t layers,
                                                                       uint32_t kv_heads) {
    constexpr uint32_t kDims = 128;
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t unit = uint64_t(blockIdx.x) * kCodecWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    if (unit >= uint64_t(batch) * 2 * kv_heads) return;
    const uint32_t head = uint32_t(unit % kv_heads);
    const uint32_t kind = uint32_t(unit / kv_heads % 2);
    const uint32_t row = uint32_t(unit / (2ull * kv_heads));

    const u32x4* fresh_at = reinterpret_cast<const u32x4*>((kind == 0 ? k : v) + (uint64_t(row) * kv_heads + head) * kDims + 32 * (lane % 4));
    u32x4 fresh[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) fresh[j] = fresh_at[j];
    const uint32_t block = uint32_t(write_block[uint64_t(row) * row_stride]);
    const uint32_t write = uint32_t(write_slot[uint64_t(row) * row_stride]);

    const uint32_t groups_per_block = 2 * layers * kv_heads;
    const uint64_t block_elems = uint64_t(kFastGroup) * groups_per_block;
    const uint64_t record = block_elems + 2ull * groups_per_block;
    const uint32_t g = (kind * layers + layer) * kv_heads + head;
    uint8_t* base = records + uint64_t(block) * record;
    append_group_2048(base + uint64_t(g) * kFastGroup, reinterpret_cast<int16_t*>(base + block_elems + 2ull * g), write, fresh, lane);
}

void launch_append_2048(uint8_t* records, const int32_t* write_block, const int32_t* write_slot, uint32_t row_stride, uint32_t batch,
                        const uint16_t* k, const uint16_t* v, uint32_t layer, uint32_t layers, uint32_t kv_heads, uint32_t grid,
                        hipStream_t stream) {
    hipLaunchKernelGGL(append_groups_2048, dim3(grid), dim3(kWave * kCodecWaves), 0, stream, records, write_block, write_slot, row_stride, batch, k,
                       v, layer, layers, kv_heads);
}

void launch_stage_history_2048(const uint8_t* records, const int32_t* ids, uint64_t record_bytes, uint32_t groups_per_block, uint32_t layer,
                               uint32_t layers, uint32_t kv_heads, uint32_t blocks, uint16_t* stage, int32_t* index, hipStream_t stream) {
    const uint64_t waves = uint64_t(blocks) * 2 * kv_heads;
    const uint32_t grid = uint32_t((waves + kCodecWaves - 1) / kCodecWaves);
    if (((reinterpret_cast<uintptr_t>(records) | record_bytes) & 7) == 0)
        hipLaunchKernelGGL(stage_history_2048<true>, dim3(grid), dim3(kWave * kCodecWaves), 0, stream, records, ids, record_bytes, groups_per_block,
                           layer, layers, kv_heads, blocks, stage, index);
    else
        hipLaunchKernelGGL(stage_history_2048<false>, dim3(grid), dim3(kWave * kCodecWaves), 0, stream, records, ids, record_bytes, groups_per_block,
                           layer, layers, kv_heads, blocks, stage, index);
}

void launch_quantize_2048(const uint16_t* pool, const int32_t* ids, uint8_t* stage, uint32_t count, uint32_t groups_per_block,
                          uint32_t grid, hipStream_t stream) {
    hipLaunchKernelGGL(quantize_groups_2048, dim3(grid), dim3(kWave * kRecordWaves), 0, stream, pool, ids, stage, count, groups_per_block);
}

// The dequantize launch reserves LDS it does not use, 8 KiB per single-wave workgroup, which
// caps it at 20 waves per CU (160 KiB of LDS): fewer of its reads and writes are in flight at
// once, and HBM serves its 1:2 read/write mix faster. Measured on MI355X at the swap's
// 113-record launches back to back, staging rotated over 1 GiB (A/B in one process): 62.9 us
// uncapped, 61.0 us with 8 KiB. With the staging in two slots (partly cached): 62.3-62.6
// uncapped, 60.6-60.8 with 8 KiB, 60.9 with 6.5 KiB (25 per CU), 61.8-61.9 with 9.4-10.9 KiB
// (15-17 per CU). The same caps only slow the quantize (58.2 -> 59.5-75 us).
constexpr uint32_t kDequantizeOccupancyLds = 8192;

void launch_dequantize_2048(const uint8_t* stage, const int32_t* ids, uint16_t* pool, uint32_t count, uint32_t groups_per_block,
                            uint32_t grid, hipStream_t stream) {
    hipLaunchKernelGGL(dequantize_groups_2048, dim3(grid), dim3(kWave * kRecordWaves), kDequantizeOccupancyLds, stream, stage, ids, pool, count,
                       groups_per_block);
}

}  // namespace lk
