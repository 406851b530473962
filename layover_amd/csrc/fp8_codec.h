// FP8 E4M3 records of KV blocks on gfx950: the fused gather+quantize and dequantize+scatter
// kernels behind lk_fp8_quantize / lk_fp8_dequantize, and the elementwise codec.
//
// Arithmetic: the reference's integer codec on BF16 bit patterns (layover/kernels/fp8.py:
// 86-137), so every byte and every restored BF16 pattern is identical to its output by
// construction, including the cases a hardware float convert treats differently (BF16
// subnormals -> signed zero, infinity and overflow -> sign|0x7F, decode saturating at
// 0x7F7F and flushing below BF16's smallest normal). The Qwen3-shaped kernels of
// fp8_records.hip use the hardware E4M3 converts instead, only for groups where those are
// proven to give the same bytes, and this integer codec for every other group.
//
// Layout of work: one wave64 per group. A Qwen3-4B group (16 slots x 128 dims = 2048 values,
// 4 KiB of BF16) is 4 loads of 16 bytes per lane, each wave instruction reading 1 KiB
// contiguous; the shift is a wave max-reduction of the masked exponents; the 2 KiB of codes
// go out as 4 stores of 8 bytes per lane (512 bytes contiguous per instruction). Other group
// sizes take a strided element loop. The kernels are HBM-bound: per Qwen3-4B block, quantize
// reads 2,359,296 bytes and writes 1,180,800; dequantize the reverse.
#ifndef LAYOVER_AMD_FP8_CODEC_H
#define LAYOVER_AMD_FP8_CODEC_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace lk {

constexpr uint32_t kWave = 64;
constexpr uint32_t kCodecWaves = 4;  // waves per workgroup
// Waves per workgroup of the Qwen-shaped record kernels (quantize_groups_2048,
// dequantize_groups_2048), which give each wave one 2,048-value group. One: measured on MI355X
// at the swap's 113-block launches, quantize 57.7-57.8 us per launch against 58.6-58.7 us with
// four waves (59.3-59.8 with two); dequantize the same either way (62.1-62.4 us).
#ifndef LK_RECORD_WAVES
#define LK_RECORD_WAVES 1
#endif
constexpr uint32_t kRecordWaves = LK_RECORD_WAVES;

// fp8.py:95-116: BF16 bits / 2**shift -> E4M3 byte, rounding the significand to nearest even.
__device__ __forceinline__ uint32_t encode_e4m3(uint32_t bits, int32_t shift) {
    const uint32_t sign = (bits >> 15) & 1u;
    const int32_t raw = int32_t((bits >> 7) & 0xFFu);
    const int32_t biased = raw - 127 - shift + 7;
    const uint32_t significand = (bits & 0x7Fu) | 0x80u;
    int32_t right = 4 + (biased < 1 ? 1 - biased : 0);
    right = right > 15 ? 15 : right;
    uint32_t kept = significand >> right;
    const uint32_t remainder = significand & ((1u << right) - 1u);
    const uint32_t half = 1u << (right - 1);
    kept += (remainder > half || (remainder == half && (kept & 1u))) ? 1u : 0u;
    int32_t magnitude = biased > 0 ? ((biased - 1) << 3) + int32_t(kept) : int32_t(kept);
    magnitude = magnitude > 0x7E ? 0x7F : magnitude;
    magnitude = raw == 0 ? 0 : magnitude;
    magnitude = raw == 0xFF ? 0x7F : magnitude;
    return (sign << 7) | uint32_t(magnitude);
}

// fp8.py:119-137: E4M3 byte * 2**shift -> BF16 bits.
__device__ __forceinline__ uint32_t decode_e4m3(uint32_t code, int32_t shift) {
    const uint32_t sign = (code >> 7) & 1u;
    const uint32_t magnitude = code & 0x7Fu;
    const int32_t raw = int32_t(magnitude >> 3);
    uint32_t fraction = magnitude & 7u;
    const int32_t top = fraction >= 4 ? 2 : (fraction >= 2 ? 1 : 0);
    const int32_t exponent = raw > 0 ? raw - 7 : top - 9;
    fraction = raw > 0 ? fraction : ((fraction << (3 - top)) & 7u);
    const int32_t biased = exponent + shift + 127;
    uint32_t out = (uint32_t(biased) << 7) | (fraction << 4);
    out = biased >= 0xFF ? 0x7F7Fu : out;
    out = biased <= 0 ? 0u : out;
    out = magnitude == 0 ? 0u : out;
    out |= sign << 15;
    return magnitude == 0x7F ? 0x7FC0u : out;
}

// Exponent field shifted up one step, with infinity/NaN mapped to 0, so a plain unsigned max
// over a group finds the largest finite exponent (+1; zero and subnormals give 1).
__device__ __forceinline__ uint32_t exponent_key(uint32_t bits) {
    return (((bits & 0x7F80u) + 0x80u) & 0x7FFFu) >> 7;
}

__device__ __forceinline__ int32_t shift_from_key(uint32_t largest_key) {
    const int32_t largest = int32_t(largest_key) - 1;  // back to the raw exponent
    return largest > 0 ? largest - 127 - 7 : 0;
}

__device__ __forceinline__ uint32_t wave_max(uint32_t value) {
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) {
        const uint32_t other = __shfl_xor(value, mask, kWave);
        value = other > value ? other : value;
    }
    return value;
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float codec_f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float codec_pow2(int32_t e) { return __uint_as_float(uint32_t(e + 127) << 23); }

// Both halves of a BF16 pair with subnormals replaced by signed zero (fp8.py:114), so the
// hardware convert below gives the reference's bytes whatever the FP32 denormal mode.
__device__ __forceinline__ uint32_t flush_bf16_pair(uint32_t pair) {
    pair = (pair & 0x7F80u) == 0 ? (pair & 0xFFFF8000u) : pair;
    return (pair & 0x7F800000u) == 0 ? (pair & 0x8000FFFFu) : pair;
}

// One token written into a Qwen3-shaped group of FP8 records (16 slots x 128 dims, 2,048
// codes at `group`, its shift at `shift_at`), by one wave: lane l holds bytes 32l .. 32l+31
// (slot l/4, dims 32(l%4) .. +31), so the group is read once and written once. Element e
// becomes the old value decoded at the old shift for slots before `write`, the new BF16 value
// (`fresh`: the lane's 32 values of the new token's row, dims 32(l%4) .. +31) at it, and zero
// after it; the group is re-encoded at the shift of those values (fp8.py:86-137). Decode and
// encode take the hardware converts where they are exact (as the record kernels do), else the
// reference's integer codec.
//
// append_group_2048_loaded takes the lane's old codes and the old shift from the caller (who
// can then load several groups at once), stores the group and returns its new codes in `out`
// and its new shift.
__device__ __forceinline__ int32_t append_group_2048_loaded(uint8_t* group, int16_t* shift_at, uint32_t write, const u32x4 (&fresh)[4],
                                                            uint32_t lane, const u32x4 (&old)[2], int32_t old_shift, u32x4 (&out)[2]) {
    u32x4* codes = reinterpret_cast<u32x4*>(group) + 2 * lane;
    const uint32_t slot = lane / 4;

    // The old values (lanes before the write slot): a NaN code anywhere among them, or a shift
    // whose products could leave BF16's normal range, sends the wave to the integer decode.
    uint32_t nan_flags = 0;
#pragma unroll
    for (int w = 0; w < 8; ++w) nan_flags |= (old[w / 4][w % 4] & 0x7F7F7F7Fu) + 0x01010101u;
    const bool exact_decode = __any(slot < write && (nan_flags & 0x80808080u) != 0) || old_shift < -117 || old_shift > 119;
    uint32_t pairs[16];  // the lane's 32 new BF16 values, two per word
    if (slot < write) {
        if (!exact_decode) {
            const float scale = codec_pow2(old_shift);
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const int word = int(old[w / 4][w % 4]);
                const codec_f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(word, false);
                const codec_f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8(word, true);
                pairs[2 * w] = __builtin_amdgcn_perm(__float_as_uint(lo.y * scale), __float_as_uint(lo.x * scale), 0x07060302u);
                pairs[2 * w + 1] = __builtin_amdgcn_perm(__float_as_uint(hi.y * scale), __float_as_uint(hi.x * scale), 0x07060302u);
            }
        } else {
#pragma unroll
            for (int w = 0; w < 8; ++w) {
                const uint32_t word = old[w / 4][w % 4];
                pairs[2 * w] = decode_e4m3(word & 0xFFu, old_shift) | (decode_e4m3((word >> 8) & 0xFFu, old_shift) << 16);
                pairs[2 * w + 1] = decode_e4m3((word >> 16) & 0xFFu, old_shift) | (decode_e4m3(word >> 24, old_shift) << 16);
            }
        }
    } else if (slot == write) {
#pragma unroll
        for (int x = 0; x < 16; ++x) pairs[x] = fresh[x / 4][x % 4];
    } else {
#pragma unroll
        for (int x = 0; x < 16; ++x) pairs[x] = 0u;
    }

    // Shift of the new values, and whether any is infinite or NaN (exponent field all ones).
    uint32_t key = 0, flags = 0;
#pragma unroll
    for (int x = 0; x < 16; ++x) {
        const uint32_t lo = exponent_key(pairs[x] & 0xFFFFu), hi = exponent_key(pairs[x] >> 16);
        key = lo > key ? lo : key;
        key = hi > key ? hi : key;
        flags |= (pairs[x] & 0x7F807F80u) + 0x00800080u;
    }
    const int32_t shift = shift_from_key(wave_max(key));
    const bool nonfinite = __any((flags & 0x80008000u) != 0);
    if (!nonfinite && shift >= -126) {
        // value * 2^-shift is exact for a normal BF16 value and stays below 2^8; the convert
        // rounds to nearest even. Subnormal inputs are flushed first; products below FP32's
        // normal range round to zero codes either way.
        const float scale = codec_pow2(-shift);
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t a = flush_bf16_pair(pairs[2 * w]), b = flush_bf16_pair(pairs[2 * w + 1]);
            int p = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(a << 16) * scale, __uint_as_float(a & 0xFFFF0000u) * scale, 0, false);
            p = __builtin_amdgcn_cvt_pk_fp8_f32(__uint_as_float(b << 16) * scale, __uint_as_float(b & 0xFFFF0000u) * scale, p, true);
            out[w / 4][w % 4] = uint32_t(p);
        }
    } else {
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const uint32_t a = pairs[2 * w], b = pairs[2 * w + 1];
            out[w / 4][w % 4] = encode_e4m3(a & 0xFFFFu, shift) | (encode_e4m3(a >> 16, shift) << 8) |
                                (encode_e4m3(b & 0xFFFFu, shift) << 16) | (encode_e4m3(b >> 16, shift) << 24);
        }
    }
    codes[0] = out[0];
    codes[1] = out[1];
    if (lane == 0) *shift_at = int16_t(shift);
    return shift;
}

__device__ __forceinline__ void append_group_2048(uint8_t* group, int16_t* shift_at, uint32_t write, const u32x4 (&fresh)[4], uint32_t lane) {
    const u32x4* codes = reinterpret_cast<const u32x4*>(group) + 2 * lane;
    const u32x4 old[2] = {codes[0], codes[1]};
    u32x4 out[2];
    append_group_2048_loaded(group, shift_at, write, fresh, lane, old, *shift_at, out);
}

// Qwen3-shaped groups (2048 values, 16-byte aligned records) run the kernels of
// fp8_records.hip; these launch them on `stream`.
constexpr uint32_t kFastGroup = 2048;
void launch_quantize_2048(const uint16_t* pool, const int32_t* ids, uint8_t* stage, uint32_t count, uint32_t groups_per_block,
                          uint32_t grid, hipStream_t stream);
void launch_dequantize_2048(const uint8_t* stage, const int32_t* ids, uint16_t* pool, uint32_t count, uint32_t groups_per_block,
                            uint32_t grid, hipStream_t stream);
// One token per row written into Qwen3-shaped FP8 records (16 slots x 128 dims, 16-byte
// aligned records, k and v), the fast form of lk_fp8_append.
void launch_append_2048(uint8_t* records, const int32_t* write_block, const int32_t* write_slot, uint32_t row_stride, uint32_t batch,
                        const uint16_t* k, const uint16_t* v, uint32_t layer, uint32_t layers, uint32_t kv_heads, uint32_t grid,
                        hipStream_t stream);
// One layer of the FP8 records of blocks ids[0 .. blocks) decoded into a compact one-layer BF16
// pool `stage` [blocks][2][kv_heads][16 x 128], with index[b] = b (the paged prefill's
// FP8 path). Groups of 2,048 values; the records' shifts follow their codes. records and
// record_bytes need only be even.
void launch_stage_history_2048(const uint8_t* records, const int32_t* ids, uint64_t record_bytes, uint32_t groups_per_block, uint32_t layer,
                               uint32_t layers, uint32_t kv_heads, uint32_t blocks, uint16_t* stage, int32_t* index, hipStream_t stream);

// Kernels below have internal linkage: this header is included by more than one translation
// unit of the library.
namespace {

// Any group size and alignment: element-strided loops, one wave per group.
__global__ __launch_bounds__(kWave* kCodecWaves) void quantize_groups_any(const uint16_t* __restrict__ pool, const int32_t* __restrict__ ids,
                                                                        uint8_t* __restrict__ stage, uint32_t count,
                                                                        uint64_t group_elems, uint32_t groups_per_block) {
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t group = uint64_t(blockIdx.x) * kCodecWaves + threadIdx.x / kWave;
    if (group >= uint64_t(count) * groups_per_block) return;
    const uint32_t index = uint32_t(group / groups_per_block);
    const uint32_t g = uint32_t(group % groups_per_block);
    const uint64_t block_elems = group_elems * groups_per_block;
    const uint64_t record = block_elems + 2ull * groups_per_block;
    const uint16_t* source = pool + uint64_t(ids[index]) * block_elems + uint64_t(g) * group_elems;
    uint32_t key = 0;
    for (uint64_t e = lane; e < group_elems; e += kWave) {
        const uint32_t k = exponent_key(source[e]);
        key = k > key ? k : key;
    }
    const int32_t shift = shift_from_key(wave_max(key));
    uint8_t* out = stage + uint64_t(index) * record;
    for (uint64_t e = lane; e < group_elems; e += kWave) out[uint64_t(g) * group_elems + e] = uint8_t(encode_e4m3(source[e], shift));
    if (lane == 0) {
        const uint16_t stored = uint16_t(int16_t(shift));
        out[block_elems + 2ull * g] = uint8_t(stored & 0xFFu);
        out[block_elems + 2ull * g + 1] = uint8_t(stored >> 8);
    }
}

__global__ __launch_bounds__(kWave* kCodecWaves) void dequantize_groups_any(const uint8_t* __restrict__ stage,
                                                                          const int32_t* __restrict__ ids, uint16_t* __restrict__ pool,
                                                                          uint32_t count, uint64_t group_elems, uint32_t groups_per_block) {
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t group = uint64_t(blockIdx.x) * kCodecWaves + threadIdx.x / kWave;
    if (group >= uint64_t(count) * groups_per_block) return;
    const uint32_t index = uint32_t(group / groups_per_block);
    const uint32_t g = uint32_t(group % groups_per_block);
    const uint64_t block_elems = group_elems * groups_per_block;
    const uint64_t record = block_elems + 2ull * groups_per_block;
    const uint8_t* in = stage + uint64_t(index) * record;
    const int32_t shift = int16_t(uint16_t(in[block_elems + 2ull * g]) | uint16_t(in[block_elems + 2ull * g + 1] << 8));
    uint16_t* target = pool + uint64_t(ids[index]) * block_elems + uint64_t(g) * group_elems;
    for (uint64_t e = lane; e < group_elems; e += kWave) target[e] = uint16_t(decode_e4m3(in[uint64_t(g) * group_elems + e], shift));
}

__global__ void encode_elements(const uint16_t* __restrict__ bits, uint8_t* __restrict__ out, uint64_t n, int32_t shift) {
    const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = uint8_t(encode_e4m3(bits[i], shift));
}

__global__ void decode_elements(const uint8_t* __restrict__ codes, uint16_t* __restrict__ out, uint64_t n, int32_t shift) {
    const uint64_t i = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = uint16_t(decode_e4m3(codes[i], shift));
}

}  // namespace

}  // namespace lk

#endif  // LAYOVER_AMD_FP8_CODEC_H
