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
// Fast path (16 slots x 128 dims, the Qwen3 shape; up to 16 query heads per KV head), on the
//   matrix cores (details above decode_split_mfma): workgroup = (sequence, split of `bps`
//   blocks, KV head), 4 waves taking the split's blocks round-robin, one (block, KV head) unit
//   at a time. Each K or V tile (16 x 128) is read once for all G query heads: no GQA
//   re-reads, so HBM traffic is the "unique" bytes of bench/decode_bandwidth.py:129-139.
//   QK^T is four v_mfma_f32_16x16x32_bf16 (slots x heads); the online softmax runs per lane
//   on the MFMA result (head n, four slots); PV is v_mfma_f32_16x16x16_bf16 with the weights
//   as BF16 hi + lo parts, so they keep FP32-like precision. The running max is only raised
//   (with a rescale of the accumulators) when a score exceeds it by more than 2^8, a
//   wave-uniform branch almost never taken after the first tile; weights are then at most
//   2^8, harmless in FP32. Tiles stream through a ring of register buffers refilled as they
//   are consumed; block ids (and FP8 shifts) are loaded one per lane up front and read with
//   v_readlane. FP8 tiles are dequantized in registers: codes -> BF16 by the hardware
//   convert (exact), the group's power of two folded into the score (K) and the weights (V).
//   Groups whose shift could leave BF16's normal range use the exact integer decode of
//   fp8.py instead, so results equal attention over the reference's decode_bits output.
// Generic path (any slots <= 64 and head_dim <= 256, any G): one wave per (sequence, query
//   head, split), lane d owning dims d, d+64, ...; used for shapes other than Qwen3's.
// Combine: one wave per (sequence, query head) merges the split partials (m, l, acc) and
//   writes the output rounded to nearest even. A table of one split needs no merge: the
//   split kernel (8-wave form) writes the output itself. (Merging inside the split kernel,
//   in the last split to arrive, was slower both ways it was built: behind a device-scope
//   release, which on MI355X writes back the XCD's L2, and with agent-scope partials and an
//   agent-scope arrival count, whose chain outlasts the separate merge launch.)
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

// Max of a value over lanes n, n + 16, n + 32 and n + 48 (the four lane groups of an MFMA
// result column), with gfx950's row-swapping permlanes instead of LDS-routed shuffles: given
// the same register twice, permlane16_swap returns rows (0, 0, 2, 2) and (1, 1, 3, 3) of it,
// and permlane32_swap rows (0, 1, 0, 1) and (2, 3, 2, 3).
__device__ __forceinline__ float max_over_lane_groups(float value) {
    const uint32_t bits = __float_as_uint(value);
    const auto rows16 = __builtin_amdgcn_permlane16_swap(bits, bits, false, false);
    const float half = fmaxf(__uint_as_float(rows16[0]), __uint_as_float(rows16[1]));
    const uint32_t half_bits = __float_as_uint(half);
    const auto rows32 = __builtin_amdgcn_permlane32_swap(half_bits, half_bits, false, false);
    return fmaxf(__uint_as_float(rows32[0]), __uint_as_float(rows32[1]));
}

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
    uint32_t table_stride;   // int32 elements from one table row to the next (>= table_width)
    uint32_t lengths_stride; // int32 elements from one length to the next
    uint32_t groups;       // query heads per KV head
    uint32_t splits;       // splits per sequence (grid)
    uint32_t bps;          // blocks per split
    uint32_t order;        // workgroup order, see decode_unit_of
    uint32_t vector_combine;  // workspace and out aligned for combine_dim128's vector accesses
    uint32_t shared_blocks;   // LK_DECODE_SHARED_BLOCKS: the cached form of the tile loads
    uint64_t block_bytes;  // bytes from one pool block to the next
    float scale_log2;      // softmax scale * log2(e)
    // Fused decode-time write (lk_paged_decode_append; null write_block: none): row b's new
    // token, k_new/v_new [batch, kv_heads, head_dim] BF16, goes to slot write_slot[b] of block
    // write_block[b] (rows write_stride int32 apart), which must hold the row's last token.
    const int32_t* write_block;
    const int32_t* write_slot;
    uint32_t write_stride;
    const uint16_t* k_new;
    const uint16_t* v_new;
    // Non-null when every row fits one split (splits == 1, matrix-core kernel with 8 waves):
    // that split's state is the answer, so the split kernel writes the output here and no
    // combine runs.
    void* out;
};

__device__ __forceinline__ uint32_t blocks_of(int32_t length, uint32_t slots) { return (uint32_t(length) + slots - 1) / slots; }

// ---------------------------------------------------------------------------------------
// Fast path: 16 slots x 128 dims on the matrix cores.
//
// A wave takes one (block, KV head) unit at a time; lane l is (g, n) = (l / 16, l % 16).
//   QK:  S^T[slot][head] = sum_d K[slot][d] q[head][d] with v_mfma_f32_16x16x32_bf16, four
//        steps over the 128 dims. A = K: lane (g, n) holds slot n and, for step j, 8 dims
//        chosen per format so the loads stay contiguous (MfmaTile) (BF16; FP8 codes
//        are converted to BF16 exactly in registers). B = q^T, the same dims of query head n
//        (zero for n >= G): up to 16 query heads per KV head cost nothing extra.
//        The result lands as lane (g, n) = head n, slots 4g .. 4g+3.
//   PV:  O[head][dim] = sum_slot P[head][slot] V[slot][dim] with v_mfma_f32_16x16x16_bf16.
//        A = P: lane (g, n) needs head n, slots 4g .. 4g+3 -- exactly the QK result, after
//        the online softmax, as BF16 hi + lo parts (two MFMAs, so the weights keep FP32-like
//        precision). B = V: lane (g, n) loads slots 4g .. 4g+3, dims 8n .. 8n+7 (16 bytes each,
//        every load instruction reading 4 whole 256-byte slot rows) and v_perm builds, for each
//        e < 8, the four slots' values at dim 8n + e; MFMA e then produces dims 8n' + e for
//        n' = 0..15. Eight MFMAs (x2 for hi/lo) cover the 128 dims; O stays in 32 registers.
//   Softmax per lane: head n, its 4 slots; the tile max of a head is reduced over the four
//        lane groups, so every lane holding that head uses the same running max.
//   Launch order: workgroups run (sequence, split, KV head) with the KV head fastest, so the
//        eight heads' tiles of a block -- adjacent 4 KiB pieces of one 32 KiB run per kind and
//        layer -- are read at about the same time. Measured on MI355X (Qwen3-4B, batch 32,
//        mixed contexts): 306 us per layer against 419 us with the head slowest.

constexpr uint32_t kSlots = 16;
constexpr uint32_t kDim = 128;
constexpr uint32_t kMaxHeads = 16;  // query heads per KV head the MFMA tile holds

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

template <int KV>
struct MfmaTile;
// Lane group g of K holds, for QK step j, the dims kGroupDims * g + kStepDims * j .. +8 of
// slot n (q's B operand uses the same dims). BF16: 8g + 32j, so each of the four K load
// instructions reads 64 contiguous bytes of every slot row (whole 64-byte halves of its
// 128-byte lines). FP8: 32g + 8j, one 32-byte run of codes per lane.
template <>
struct MfmaTile<LK_BF16> {
    uint32_t k[16];     // slot n, dims 8g + 32j .. +8 for j = 0..3 (BF16 pairs)
    uint32_t v[4][4];   // slot 4g + r, dims 8n .. 8n+7 (BF16 pairs)
    static constexpr int32_t k_shift = 0, v_shift = 0;
    static constexpr uint32_t kGroupDims = 8, kStepDims = 32;
};
template <>
struct MfmaTile<LK_FP8_RECORD> {
    uint32_t k[8];      // slot n, dims 32g .. 32g+31 (E4M3 codes)
    uint32_t v[4][2];   // slot 4g + r, dims 8n .. 8n+7 (E4M3 codes)
    int32_t k_shift, v_shift;
    static constexpr uint32_t kGroupDims = 32, kStepDims = 8;
};

// A shift for which every E4M3 code times 2**shift is zero, NaN or a BF16 normal below
// 0x7F7F, so code * 2**shift equals the reference's decode exactly.
__device__ __forceinline__ bool shift_is_exact_in_fp32(int32_t shift) { return shift >= -117 && shift <= 119; }

__device__ __forceinline__ float pow2(int32_t e) { return __uint_as_float(uint32_t(e + 127) << 23); }

// Two E4M3 codes (the low or high half of `word`) to a BF16 pair: the exact hardware convert,
// or for groups whose shift can leave BF16's normal range the reference's integer decode with
// the shift applied.
__device__ __forceinline__ uint32_t fp8_pair(uint32_t word, bool high, bool exact, int32_t shift) {
    if (!exact) {
        return high ? __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, 1.0f, true))
                    : __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(word, 1.0f, false));
    }
    const uint32_t half = high ? word >> 16 : word & 0xFFFFu;
    return decode_e4m3(half & 0xFFu, shift) | (decode_e4m3(half >> 8, shift) << 16);
}

__device__ __forceinline__ bf16x8 as_bf16x8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(bf16x8, u32x4{a, b, c, d});
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// Register buffers per wave (see the main loop of decode_split_mfma). Two for both formats,
// measured on MI355X per layer (Qwen3-4B): BF16 batch 32 mixed contexts on distinct blocks
// 389 -> 377-383 us with three, batch 1 @ 32,768 34.1 -> 32.4 us; FP8 batch 64 @ 4,096
// 86.1 -> 82.7 us and batch 1 23.5 -> 22.3 us against four. More buffers in flight per wave
// do not buy bandwidth here, and cost registers and issue slots.
#ifndef LK_DECODE_RING_BF16
#define LK_DECODE_RING_BF16 2
#endif
#ifndef LK_DECODE_RING_FP8
#define LK_DECODE_RING_FP8 2
#endif
// Tile loads go through a buffer resource that spans one pool block (base and size in
// scalar registers, offsets per lane). A resource of size 0 turns every load into zeros that
// touch no memory: the ring's refills past a wave's last unit cost nothing, yet every load is
// still issued unconditionally, so the compiler's wait counts stay exact. The streaming form
// (see decode_split_mfma) sets the non-temporal bit.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t block_resource(const uint8_t* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), short(0), int(bytes), 0x00020000);
}
template <bool kNT>
__device__ __forceinline__ u32x4 tile_load16(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, kNT ? 2 : 0));
}
template <bool kNT>
__device__ __forceinline__ u32x2 tile_load8(__amdgpu_buffer_rsrc_t r, uint32_t offset) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, offset, 0, kNT ? 2 : 0));
}

// Workgroup -> (sequence, split, KV head). Order 1 (the default): KV head fastest, so the
// eight heads' tiles of a block (adjacent 4 KiB pieces) are read close together in time, by
// workgroups that the round-robin dealing puts on different XCDs. Order 0: KV head slowest.
// Measured on MI355X, batch 32 mixed contexts, per layer: order 1 294 us, order 0 419 us, and
// keeping a block's heads on one XCD instead (so they share its L2) 370 us.
__device__ __forceinline__ bool decode_unit_of(const DecodeArgs& a, uint32_t w, uint32_t* seq, uint32_t* split, uint32_t* kv_head) {
    if (a.order == 0) {
        *split = w % a.splits;
        *kv_head = (w / a.splits) % a.kv_heads;
        *seq = w / (a.splits * a.kv_heads);
    } else {
        *kv_head = w % a.kv_heads;
        *split = (w / a.kv_heads) % a.splits;
        *seq = w / (a.kv_heads * a.splits);
    }
    return *seq < a.batch;
}

// kWaves waves per workgroup take the split's blocks round-robin: 4 for full grids; 8 when
// the grid gives each CU at most one workgroup (small batches), so each CU has more waves
// streaming tiles and each wave a shorter chain of dependent loads. The LDS merge keeps
// kWaves * kHeads * kDim floats, 32 KiB either way: 8 waves hold at most 8 query heads per
// KV head, 4 waves 16.
// FP8 pools ask the compiler for at least two waves per SIMD (amdgpu_waves_per_eu): its
// register allocation then comes out at 166 rather than 204, so three waves fit per SIMD, and
// the FP8 kernel went from 170 to 152 us per layer at batch 32 (0.79 -> 0.89 of 8 TB/s) and
// from 84.5 to 76 us at batch 64 @ 4,096 (measured on MI355X, A/B in one process). For BF16
// pools the same request, or three or four waves with a one-tile ring, measured no faster.
template <int KV, int QF, int kWaves, bool kStream, bool kAppend>
__global__ __launch_bounds__(kWave* kWaves) __attribute__((amdgpu_waves_per_eu(KV == LK_FP8_RECORD ? 2 : 1))) void decode_split_mfma(
    DecodeArgs a) {
    constexpr uint32_t kDecodeWaves = kWaves;
    constexpr uint32_t kHeads = kMaxHeads * 4 / kWaves;
    const uint32_t lane = threadIdx.x % kWave;
    // Wave-uniform by construction; readfirstlane tells the compiler, so values derived from
    // it stay in scalar registers.
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t g = lane / 16;
    const uint32_t n = lane % 16;
    uint32_t split, kv_head, seq;
    if (!decode_unit_of(a, blockIdx.x, &seq, &split, &kv_head)) return;
    const uint32_t groups = a.groups;

    // The split's block ids are loaded (one per lane, this wave's units) before the length
    // is known, bounded by the table width alone, so the two loads overlap; the length then
    // decides how many are used.
    const uint32_t first = split * a.bps;
    const int32_t* row_ids = a.table + uint64_t(seq) * a.table_stride + first;
    const uint32_t width_here = min(a.bps, a.table_width - first);
    const uint32_t listed = width_here > wave ? (width_here - wave + kDecodeWaves - 1) / kDecodeWaves : 0;
    // Unconditional (lanes past the listed ones re-read the split's first id, which exists),
    // so no branch stands between this load and the waits that follow it.
    const int32_t listed_block = row_ids[lane < listed ? wave + lane * kDecodeWaves : 0];
    const int32_t length = a.lengths[uint64_t(seq) * a.lengths_stride];

    // B operands of QK: query head n (zero past the group), the dims kDimsOf(g, j) .. +8 that
    // lane group g of K holds for step j. An FP32 q is split into BF16 hi + lo parts, one MFMA
    // each.
    constexpr int kQParts = QF == LK_BF16 ? 1 : 2;
    uint32_t qt[kQParts][16];
#pragma unroll
    for (int part = 0; part < kQParts; ++part)
#pragma unroll
        for (int i = 0; i < 16; ++i) qt[part][i] = 0;
    if (n < groups) {
        const uint64_t row_at = (uint64_t(seq) * a.query_heads + kv_head * groups + n) * kDim + MfmaTile<KV>::kGroupDims * g;
        constexpr uint32_t kStepDims = MfmaTile<KV>::kStepDims;
        if constexpr (QF == LK_BF16) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.q) + row_at + j * kStepDims);
#pragma unroll
                for (int i = 0; i < 4; ++i) qt[0][4 * j + i] = w[i];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(a.q) + row_at + (j / 2) * kStepDims + 4 * (j % 2));
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const float x0 = __uint_as_float(w[2 * i]), x1 = __uint_as_float(w[2 * i + 1]);
                    const uint32_t hi = pack_bf16(x0, x1);
                    qt[0][2 * j + i] = hi;
                    qt[kQParts - 1][2 * j + i] = pack_bf16(x0 - bf16_lo(hi), x1 - bf16_hi(hi));
                }
            }
        }
    }

    // q, the ids and the length are in flight together; only now is the length needed. With
    // the output written here (one split; 8-wave kernels only, which small grids run), a row
    // of no tokens still writes it (NaN, as the combine would).
    const uint32_t nblocks = blocks_of(length, kSlots);
    constexpr bool kMayWriteOut = kWaves >= 8;
    const bool writes_out = kMayWriteOut && a.out != nullptr;
    if (first >= nblocks && !writes_out) return;
    const uint32_t count = min(a.bps, nblocks - first);

    constexpr uint32_t kElem = KV == LK_FP8_RECORD ? 1 : 2;
    const uint64_t tile_bytes = uint64_t(kSlots) * kDim * kElem;
    const uint64_t head_tile = uint64_t(a.layer) * a.kv_heads + kv_head;  // group index of K
    const uint64_t k_offset = head_tile * tile_bytes + (uint64_t(n) * kDim + MfmaTile<KV>::kGroupDims * g) * kElem;
    const uint64_t v_offset = (uint64_t(a.layers) * a.kv_heads + head_tile) * tile_bytes + (uint64_t(4 * g) * kDim + 8 * n) * kElem;
    const uint64_t block_elems = uint64_t(2) * a.layers * a.kv_heads * kSlots * kDim;  // FP8: shifts follow the data

    // Fused decode-time write. The token is the row's last, so no other split reads its block,
    // and in this split only the last unit does. The wave that owns that unit (round-robin)
    // writes the token of its KV head at the start and takes the written values from its own
    // registers when it consumes the unit, so no wave waits for the write: BF16 tiles are
    // fetched as usual and the written slot's rows replaced by the new token (which is what
    // memory holds once the write lands); FP8 groups are re-encoded whole, and the new codes go
    // to LDS, where the same wave reads them back in the tile's layout, with the new shifts.
    const bool writes = kAppend && a.write_block != nullptr && count > 0 && first + count == nblocks;
    const uint32_t writer = writes ? (count - 1) % kDecodeWaves : kDecodeWaves;
    constexpr bool kBf16 = KV == LK_BF16;
    uint32_t patch_k[kBf16 ? 16 : 1] = {}, patch_v[kBf16 ? 4 : 1] = {};
    uint32_t write_slot = 0;
    int32_t new_k_shift = 0, new_v_shift = 0;
    __shared__ __align__(16) uint8_t s_written[kBf16 ? 16 : 2 * kFastGroup];
    uint8_t* write_base = nullptr;
    u32x4 old_k[2], old_v[2], row_k[kBf16 ? 1 : 4], row_v[kBf16 ? 1 : 4];
    int32_t old_k_shift = 0, old_v_shift = 0;
    // With 8 waves (small grids) the writer issues its first tile loads before re-encoding, so
    // the two sets of loads are in flight together; the 4-wave kernel re-encodes at once, which
    // keeps the loaded values out of its main loop's registers (three waves per SIMD for FP8).
    constexpr bool kLateEncode = !kBf16 && kWaves >= 8;
    // FP8: the two re-encodes, their codes also to LDS for the written unit's consume.
    auto reencode = [&]() __attribute__((always_inline)) {
        if constexpr (!kBf16) {
            const uint64_t k_group = head_tile, v_group = uint64_t(a.layers) * a.kv_heads + head_tile;
            int16_t* shifts = reinterpret_cast<int16_t*>(write_base + block_elems);
            u32x4 out[2];
            new_k_shift = append_group_2048_loaded(write_base + k_group * kFastGroup, shifts + k_group, write_slot, row_k, lane, old_k, old_k_shift, out);
            reinterpret_cast<u32x4*>(s_written)[2 * lane] = out[0];
            reinterpret_cast<u32x4*>(s_written)[2 * lane + 1] = out[1];
            new_v_shift = append_group_2048_loaded(write_base + v_group * kFastGroup, shifts + v_group, write_slot, row_v, lane, old_v, old_v_shift, out);
            reinterpret_cast<u32x4*>(s_written + kFastGroup)[2 * lane] = out[0];
            reinterpret_cast<u32x4*>(s_written + kFastGroup)[2 * lane + 1] = out[1];
        }
    };
    if (wave == writer) {
        const uint32_t block = uint32_t(a.write_block[uint64_t(seq) * a.write_stride]);
        write_slot = uint32_t(a.write_slot[uint64_t(seq) * a.write_stride]);
        const uint16_t* k_row = a.k_new + (uint64_t(seq) * a.kv_heads + kv_head) * kDim;
        const uint16_t* v_row = a.v_new + (uint64_t(seq) * a.kv_heads + kv_head) * kDim;
        uint8_t* base = const_cast<uint8_t*>(a.pool) + uint64_t(block) * a.block_bytes;  // the pool is written only here
        const uint64_t k_group = head_tile, v_group = uint64_t(a.layers) * a.kv_heads + head_tile;
        if constexpr (kBf16) {
            if (lane < 32) {
                const u32x4 w = reinterpret_cast<const u32x4*>(lane < 16 ? k_row : v_row)[lane % 16];
                reinterpret_cast<u32x4*>(base + ((lane < 16 ? k_group : v_group) * kSlots + write_slot) * kDim * kElem)[lane % 16] = w;
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(k_row + MfmaTile<KV>::kGroupDims * g + j * MfmaTile<KV>::kStepDims);
#pragma unroll
                for (int x = 0; x < 4; ++x) patch_k[4 * j + x] = w[x];
            }
            const u32x4 w = *reinterpret_cast<const u32x4*>(v_row + 8 * n);
#pragma unroll
            for (int x = 0; x < 4; ++x) patch_v[x] = w[x];
        } else {
            // Both groups' old codes, shifts and new rows are loaded before either re-encode.
            write_base = base;
            const u32x4* old_k_at = reinterpret_cast<const u32x4*>(base + k_group * kFastGroup) + 2 * lane;
            const u32x4* old_v_at = reinterpret_cast<const u32x4*>(base + v_group * kFastGroup) + 2 * lane;
            old_k[0] = old_k_at[0];
            old_k[1] = old_k_at[1];
            old_v[0] = old_v_at[0];
            old_v[1] = old_v_at[1];
            const int16_t* shifts = reinterpret_cast<const int16_t*>(base + block_elems);
            old_k_shift = shifts[k_group];
            old_v_shift = shifts[v_group];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                row_k[j] = reinterpret_cast<const u32x4*>(k_row + 32 * (lane % 4))[j];
                row_v[j] = reinterpret_cast<const u32x4*>(v_row + 32 * (lane % 4))[j];
            }
            if constexpr (!kLateEncode) reencode();
        }
    }
    // The written unit's tile as memory holds it after the write (see above).
    auto written = [&](MfmaTile<KV>& tile) __attribute__((always_inline)) {
        if constexpr (kBf16) {
#pragma unroll
            for (int x = 0; x < 16; ++x) tile.k[x] = n == write_slot ? patch_k[x] : tile.k[x];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int x = 0; x < 4; ++x) tile.v[r][x] = 4 * g + r == write_slot ? patch_v[x] : tile.v[r][x];
        } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const u32x4 w = reinterpret_cast<const u32x4*>(s_written + n * kDim + MfmaTile<KV>::kGroupDims * g)[j];
#pragma unroll
                for (int x = 0; x < 4; ++x) tile.k[4 * j + x] = w[x];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const u32x2 w = *reinterpret_cast<const u32x2*>(s_written + kFastGroup + (4 * g + r) * kDim + 8 * n);
                tile.v[r][0] = w[0];
                tile.v[r][1] = w[1];
            }
            tile.k_shift = new_k_shift;
            tile.v_shift = new_v_shift;
        }
    };

    // The block ids (and FP8 shifts) of this wave's units, one unit per lane (at most 64:
    // blocks per split <= 256), held before any tile is loaded and read back with v_readlane,
    // so no load inside the main loop has to wait for the tile loads issued ahead of it. The
    // shifts are loaded by every lane (block 0's past the wave's units) and read only when a
    // unit is consumed, so the first tiles' loads go out without waiting for them: ids, then
    // tiles and shifts together, two trips to memory before the first unit rather than three.
    const uint32_t mine = count > wave ? (count - wave + kDecodeWaves - 1) / kDecodeWaves : 0;
    const int32_t my_block = lane < mine ? listed_block : 0;
    int32_t my_k_shift = 0, my_v_shift = 0;
    if constexpr (KV == LK_FP8_RECORD) {
        const int16_t* shifts = reinterpret_cast<const int16_t*>(a.pool + uint64_t(uint32_t(my_block)) * a.block_bytes + block_elems);
        my_k_shift = shifts[head_tile];
        my_v_shift = shifts[uint64_t(a.layers) * a.kv_heads + head_tile];
    }

    // Two forms of the tile loads (kStream, chosen by the caller's LK_DECODE_SHARED_BLOCKS):
    // - Streaming (rows read distinct blocks, the usual case): K comes in whole lines -- load
    //   i, lane l reads bytes 1024 i + 16 l of the K tile -- and relayout() moves the pieces
    //   through this wave's LDS buffer into the matrix-core layout; V loads already cover
    //   whole lines (four slot rows each). V, and for FP8 K too, carry the non-temporal hint,
    //   which keeps the tiles, read once, from allocating in the caches on their way in.
    //   The hint needs whole lines per load: on the direct K layout (every load instruction
    //   touching half of each of 16 lines) it made the kernel slower, lines evicted between
    //   the two halves. Measured per layer on MI355X, Qwen3-4B batch 32 mixed contexts on
    //   distinct blocks, against the cached form: FP8 207.7 -> 190.1 us (tile probe 180),
    //   BF16 376.5 -> 357.1 us; FP8 batch 1 @ 32,768 20.4 -> 19.2 us; FP8 batch 64 @ 4,096
    //   105.3 -> 98.7 us. BF16 K keeps plain loads (non-temporal K measured no faster there).
    // - Cached (rows share blocks, e.g. forked prefixes or tables drawn from a pool smaller
    //   than the blocks they list): direct loads in the matrix-core layout, no hint, so a
    //   block that another row read lately is found in the Infinity Cache. On the 12 GiB pool
    //   at batch 32: FP8 153.1 against 181.0 us streaming, BF16 290.3 against 294.6 us.
    // In LDS each slot row's 16-byte pieces are stored at piece ^ (row % pieces per row), so
    // the reads of 16 lanes, one row each, spread over the banks.
    constexpr bool kNTK = kStream && KV == LK_FP8_RECORD, kNTV = kStream;
    constexpr uint32_t kKTile = kSlots * kDim * kElem;
    constexpr uint32_t kKLoads = kKTile / 1024;               // whole-line K loads per tile
    constexpr uint32_t kRowPieces = kDim * kElem / 16;        // 16-byte pieces per slot row
    __shared__ __align__(16) uint8_t s_ktile[kStream ? kDecodeWaves : 1][kStream ? kKTile : 16];
    const uint64_t k_line_offset = head_tile * tile_bytes + 16 * lane;
    auto relayout = [&](MfmaTile<KV>& tile) __attribute__((always_inline)) {
        if constexpr (kStream) {
            uint8_t* buffer = s_ktile[wave];
#pragma unroll
            for (uint32_t i = 0; i < kKLoads; ++i) {
                const uint32_t row = (1024 * i + 16 * lane) / (kRowPieces * 16), piece = lane % kRowPieces;
                *reinterpret_cast<u32x4*>(buffer + (row * kRowPieces + (piece ^ (row % kRowPieces))) * 16) =
                    u32x4{tile.k[4 * i], tile.k[4 * i + 1], tile.k[4 * i + 2], tile.k[4 * i + 3]};
            }
            // Lane (g, n) takes the pieces of slot n that the direct loads give it: dims
            // kGroupDims * g + kStepDims * j for BF16 (piece g + 4j), 32g .. 32g + 31 for FP8
            // (pieces 2g, 2g + 1).
#pragma unroll
            for (uint32_t j = 0; j < kKLoads; ++j) {
                const uint32_t piece = KV == LK_BF16 ? g + 4 * j : 2 * g + j;
                const u32x4 w = *reinterpret_cast<const u32x4*>(buffer + (n * kRowPieces + (piece ^ (n % kRowPieces))) * 16);
#pragma unroll
                for (int x = 0; x < 4; ++x) tile.k[4 * j + x] = w[x];
            }
        }
    };
    // Unit i of this wave into a ring buffer; i at or past the wave's units (the ring's
    // refills after its last unit) loads zeros from an empty resource.
    const uint32_t k_first = uint32_t(kStream ? k_line_offset : k_offset), v_first = uint32_t(v_offset);
    auto fetch = [&](MfmaTile<KV>& tile, uint32_t i) __attribute__((always_inline)) {
        const uint32_t block = uint32_t(__builtin_amdgcn_readlane(my_block, min(i, mine - 1)));
        const __amdgpu_buffer_rsrc_t r = block_resource(a.pool + uint64_t(block) * a.block_bytes, i < mine ? uint32_t(a.block_bytes) : 0u);
        if constexpr (kStream) {
#pragma unroll
            for (uint32_t x = 0; x < kKLoads; ++x) {
                const u32x4 w = tile_load16<kNTK>(r, k_first + 1024 * x);
#pragma unroll
                for (int y = 0; y < 4; ++y) tile.k[4 * x + y] = w[y];
            }
        } else {
            constexpr uint32_t kStep = KV == LK_BF16 ? MfmaTile<KV>::kStepDims * kElem : 16;
#pragma unroll
            for (uint32_t x = 0; x < kKLoads; ++x) {
                const u32x4 w = tile_load16<false>(r, k_first + kStep * x);
#pragma unroll
                for (int y = 0; y < 4; ++y) tile.k[4 * x + y] = w[y];
            }
        }
#pragma unroll
        for (uint32_t row = 0; row < 4; ++row) {
            if constexpr (KV == LK_BF16) {
                const u32x4 w = tile_load16<kNTV>(r, v_first + row * kDim * kElem);
#pragma unroll
                for (int y = 0; y < 4; ++y) tile.v[row][y] = w[y];
            } else {
                const u32x2 w = tile_load8<kNTV>(r, v_first + row * kDim * kElem);
                tile.v[row][0] = w[0];
                tile.v[row][1] = w[1];
            }
        }
    };
    // The shifts of the wave's unit i, taken when the unit is consumed.
    auto shifts_of = [&](MfmaTile<KV>& tile, uint32_t i) __attribute__((always_inline)) {
        if constexpr (KV == LK_FP8_RECORD) {
            tile.k_shift = __builtin_amdgcn_readlane(my_k_shift, i);
            tile.v_shift = __builtin_amdgcn_readlane(my_v_shift, i);
        }
    };

    // Online-softmax state: lane (g, n) tracks head n over slots 4g..4g+3 of every unit (the
    // running max is shared by the four lanes of a head); o[e] holds heads 4g + r, dims 8n + e.
    float m = -INFINITY, l = 0.0f;
    f32x4 o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto consume = [&](MfmaTile<KV>& tile, uint32_t t) {
        const uint32_t token0 = (first + t) * kSlots;
        bool k_exact = false, v_exact = false;
        float k_factor = a.scale_log2, v_factor = 1.0f;
        if constexpr (KV == LK_FP8_RECORD) {
            k_exact = !shift_is_exact_in_fp32(tile.k_shift);
            v_exact = !shift_is_exact_in_fp32(tile.v_shift);
            if (!k_exact) k_factor *= pow2(tile.k_shift);
            if (!v_exact) v_factor = pow2(tile.v_shift);
        }

        // K and V of the unit as BF16 pairs. For FP8 the exact integer decode is a separate,
        // wave-uniform branch (groups whose shift can leave BF16's normal range), kept apart so
        // the common path does not compute it.
        uint32_t kb[16];
        uint32_t v[4][4];
        if constexpr (KV == LK_BF16) {
#pragma unroll
            for (int x = 0; x < 16; ++x) kb[x] = tile.k[x];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int x = 0; x < 4; ++x) v[r][x] = tile.v[r][x];
        } else {
            if (__builtin_expect(k_exact || v_exact, 0)) {
                asm volatile("" ::: "memory");
#pragma unroll
                for (int x = 0; x < 8; ++x) {
                    kb[2 * x] = fp8_pair(tile.k[x], false, k_exact, tile.k_shift);
                    kb[2 * x + 1] = fp8_pair(tile.k[x], true, k_exact, tile.k_shift);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int x = 0; x < 2; ++x) {
                        v[r][2 * x] = fp8_pair(tile.v[r][x], false, v_exact, tile.v_shift);
                        v[r][2 * x + 1] = fp8_pair(tile.v[r][x], true, v_exact, tile.v_shift);
                    }
            } else {
#pragma unroll
                for (int x = 0; x < 8; ++x) {
                    kb[2 * x] = fp8_pair(tile.k[x], false, false, 0);
                    kb[2 * x + 1] = fp8_pair(tile.k[x], true, false, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int x = 0; x < 2; ++x) {
                        v[r][2 * x] = fp8_pair(tile.v[r][x], false, false, 0);
                        v[r][2 * x + 1] = fp8_pair(tile.v[r][x], true, false, 0);
                    }
            }
        }

        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bf16x8 kk = as_bf16x8(kb[4 * j], kb[4 * j + 1], kb[4 * j + 2], kb[4 * j + 3]);
#pragma unroll
            for (int part = 0; part < kQParts; ++part)
                s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    kk, as_bf16x8(qt[part][4 * j], qt[part][4 * j + 1], qt[part][4 * j + 2], qt[part][4 * j + 3]), s, 0, 0, 0);
        }

        float score[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) score[r] = token0 + 4 * g + r < uint32_t(length) ? s[r] * k_factor : -INFINITY;
        const float top = max_over_lane_groups(fmaxf(fmaxf(score[0], score[1]), fmaxf(score[2], score[3])));
        // Raise the running max only when a score passes it by more than 2^8.
        if (__builtin_expect(__any(top > m + kRescaleThreshold), 0)) {
            // Kept as a branch: flattened, its multiplies would run on every unit.
            asm volatile("" ::: "memory");
            const float next = top > m + kRescaleThreshold ? top : m;
            const float alpha = merge_weight(m, next);
            m = next;
            l *= alpha;
            // o's rows are heads 4g + r: their factors live in lanes 4g + r (heads < 16).
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float factor = __shfl(alpha, int(4 * g + r), kWave);
#pragma unroll
                for (int e = 0; e < 8; ++e) o[e][r] *= factor;
            }
        }
        float p[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            p[r] = score[r] == -INFINITY ? 0.0f : exp2_fast(score[r] - m);
            l += p[r];
            p[r] *= v_factor;
        }
        const uint32_t hi01 = pack_bf16(p[0], p[1]), hi23 = pack_bf16(p[2], p[3]);
        const uint32_t lo01 = pack_bf16(p[0] - bf16_lo(hi01), p[1] - bf16_hi(hi01));
        const uint32_t lo23 = pack_bf16(p[2] - bf16_lo(hi23), p[3] - bf16_hi(hi23));
        const s16x4 p_hi = __builtin_bit_cast(s16x4, u32x2{hi01, hi23});
        const s16x4 p_lo = __builtin_bit_cast(s16x4, u32x2{lo01, lo23});

        // V (slot 4g + r, dims 8n + 2x, 8n + 2x + 1): slots at or past the length are zeroed,
        // since a zero weight times NaN would still be NaN.
        if (token0 + kSlots > uint32_t(length)) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool visible = token0 + 4 * g + r < uint32_t(length);
#pragma unroll
                for (int x = 0; x < 4; ++x) v[r][x] = visible ? v[r][x] : 0u;
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t select = (e & 1) ? 0x07060302u : 0x05040100u;
            const uint32_t b01 = __builtin_amdgcn_perm(v[1][e / 2], v[0][e / 2], select);
            const uint32_t b23 = __builtin_amdgcn_perm(v[3][e / 2], v[2][e / 2], select);
            const s16x4 vb = __builtin_bit_cast(s16x4, u32x2{b01, b23});
            o[e] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(p_hi, vb, o[e], 0, 0, 0);
            // The low half carries the weights' bits below BF16; FP8 values (3 significand
            // bits) do without it, and the FP8 kernel is not HBM-bound without it.
            if constexpr (KV == LK_BF16) o[e] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(p_lo, vb, o[e], 0, 0, 0);
        }
    };

    // A ring of kRing register buffers, each refilled as soon as it is consumed. Refills are
    // unconditional (past the wave's last unit, from an empty resource: zeros, no memory
    // access), because a conditional load would make every later wait assume it might not
    // have been issued, i.e. wait for all loads in flight.
#ifndef LK_DECODE_RING8_BF16
#define LK_DECODE_RING8_BF16 LK_DECODE_RING_BF16
#endif
#ifndef LK_DECODE_RING8_FP8
#define LK_DECODE_RING8_FP8 LK_DECODE_RING_FP8
#endif
    constexpr int kRing = kWaves >= 8 ? (KV == LK_BF16 ? LK_DECODE_RING8_BF16 : LK_DECODE_RING8_FP8)
                                      : (KV == LK_BF16 ? LK_DECODE_RING_BF16 : LK_DECODE_RING_FP8);
    MfmaTile<KV> ring[kRing];
    if (mine > 0) {
#pragma unroll
        for (int d = 0; d < kRing; ++d) fetch(ring[d], uint32_t(d));
        if (kLateEncode && wave == writer) reencode();
        for (uint32_t i = 0; i < mine; i += kRing) {
#pragma unroll
            for (int d = 0; d < kRing; ++d) {
                if (i + d < mine) {
                    const uint32_t t = wave + (i + d) * kDecodeWaves;
                    shifts_of(ring[d], i + d);
                    relayout(ring[d]);
                    if (t == count - 1 && wave == writer) written(ring[d]);
                    consume(ring[d], t);
                }
                fetch(ring[d], i + d + kRing);
            }
        }
    }

    // This wave's state per head: l summed over the four lane groups; o to LDS by head, dim.
    __shared__ float s_acc[kDecodeWaves][kHeads][kDim];
    __shared__ float s_m[kDecodeWaves][kHeads];
    __shared__ float s_l[kDecodeWaves][kHeads];
    l += __shfl_xor(l, 16, kWave);
    l += __shfl_xor(l, 32, kWave);
    if (g == 0 && n < groups) {
        s_m[wave][n] = m;
        s_l[wave][n] = l;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        if (4 * g + r < groups) {
#pragma unroll
            for (int e = 0; e < 8; ++e) s_acc[wave][4 * g + r][8 * n + e] = o[e][r];
        }
    }
    __syncthreads();

    // Merge the waves and write this split's partial state for each query head.
    for (uint32_t idx = threadIdx.x; idx < groups * kDim; idx += kWave * kDecodeWaves) {
        const uint32_t h = idx / kDim, d = idx % kDim;
        float best = -INFINITY;
#pragma unroll
        for (int w = 0; w < int(kDecodeWaves); ++w) best = fmaxf(best, s_m[w][h]);
        float sum = 0.0f, lsum = 0.0f;
#pragma unroll
        for (int w = 0; w < int(kDecodeWaves); ++w) {
            const float weight = merge_weight(s_m[w][h], best);
            sum += s_acc[w][h][d] * weight;
            lsum += s_l[w][h] * weight;
        }
        if (writes_out) {
            // The row's only split: the combine's arithmetic for one split (weight 1, its sum
            // starting from +0, so a -0 becomes +0 there too), times the reciprocal of l, so
            // results equal the two-launch form bit for bit.
            const uint64_t at = (uint64_t(seq) * a.query_heads + kv_head * groups + h) * kDim + d;
            const float inverse = 1.0f / lsum;
            const float merged = sum + 0.0f;
            if constexpr (QF == LK_BF16) reinterpret_cast<uint16_t*>(a.out)[at] = to_bf16(merged * inverse);
            else reinterpret_cast<float*>(a.out)[at] = merged * inverse;
            continue;
        }
        const uint64_t slot = (uint64_t(seq) * a.query_heads + kv_head * groups + h) * a.splits + split;
        a.partial_acc[slot * kDim + d] = sum;
        if (d == 0) {
            a.partial_ml[2 * slot] = best;
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
    const int32_t length = a.lengths[uint64_t(seq) * a.lengths_stride];
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
        const uint8_t* base = a.pool + uint64_t(a.table[uint64_t(seq) * a.table_stride + b]) * a.block_bytes;
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

// Combine for 128-dim heads and at most 128 splits (batch 1 at 32,768 tokens has 32): lane l
// takes dims 4 (l % 32) .. +3 of the splits of parity l / 32. Every row load of the first 64
// splits goes out at once with the length and the (m, l) pairs, so up to 64 splits nothing
// waits on more than one round trip to memory; splits 64-127 are a second batch of loads. The
// two halves' sums meet in one cross-half shuffle.
constexpr uint32_t kVectorSplits = 2 * kWave;
template <int QF, bool kTwoPages>
__device__ __forceinline__ void combine_dim128(const DecodeArgs& a, void* out, uint32_t seq, uint32_t qh) {
    constexpr uint32_t kPages = kTwoPages ? 2 : 1;
    const uint32_t lane = threadIdx.x;
    const uint32_t quad = lane % 32, half = lane / 32;
    const int32_t length = a.lengths[uint64_t(seq) * a.lengths_stride];
    const uint64_t base = (uint64_t(seq) * a.query_heads + qh) * a.splits;
    const float* ml = a.partial_ml + 2 * base;
    const f32x4* acc = reinterpret_cast<const f32x4*>(a.partial_acc + base * kDim);
    // Lane l holds the (m, l) of splits l and 64 + l.
    float lane_m[kPages], lane_l[kPages];
#pragma unroll
    for (uint32_t page = 0; page < kPages; ++page) {
        lane_m[page] = -INFINITY;
        lane_l[page] = 0.0f;
        if (page * kWave + lane < a.splits) {
            lane_m[page] = ml[2 * (page * kWave + lane)];
            lane_l[page] = ml[2 * (page * kWave + lane) + 1];
        }
    }
    f32x4 rows[kWave / 2];
    auto load_page = [&](uint32_t page) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t j = 0; j < kWave / 2; ++j) {
            const uint32_t s = page * kWave + 2 * j;
            if (s < a.splits) rows[j] = acc[uint64_t(min(s + half, a.splits - 1)) * (kDim / 4) + quad];
        }
    };
    load_page(0);
    const uint32_t used = (blocks_of(length, a.slots) + a.bps - 1) / a.bps;
    float top = -INFINITY;
#pragma unroll
    for (uint32_t page = 0; page < kPages; ++page) top = page * kWave + lane < used ? fmaxf(top, lane_m[page]) : top;
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) top = fmaxf(top, __shfl_xor(top, mask, kWave));
    float weight[kPages], total = 0.0f;
#pragma unroll
    for (uint32_t page = 0; page < kPages; ++page) {
        weight[page] = page * kWave + lane < used ? merge_weight(lane_m[page], top) : 0.0f;
        total += page * kWave + lane < used ? lane_l[page] * weight[page] : 0.0f;
    }
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) total += __shfl_xor(total, mask, kWave);
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
    auto add_page = [&](uint32_t page) __attribute__((always_inline)) {
#pragma unroll
        for (uint32_t j = 0; j < kWave / 2; ++j) {
            const uint32_t s = page * kWave + 2 * j + half;
            if (page * kWave + 2 * j >= a.splits) break;
            const float w = __shfl(weight[page], int(2 * j + half), kWave);
            // Splits past the used ones hold anything: selected away, never multiplied by zero.
#pragma unroll
            for (int i = 0; i < 4; ++i) sum[i] = s < used ? fmaf(w, rows[j][i], sum[i]) : sum[i];
        }
    };
    add_page(0);
    if constexpr (kTwoPages) {
        load_page(1);
        add_page(1);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) sum[i] += __shfl_xor(sum[i], 32, kWave);
    if (half != 0) return;
    const float inverse = 1.0f / total;
    const uint64_t at = (uint64_t(seq) * a.query_heads + qh) * kDim + 4 * quad;
    if constexpr (QF == LK_BF16) {
        const uint32_t lo = uint32_t(to_bf16(sum[0] * inverse)) | (uint32_t(to_bf16(sum[1] * inverse)) << 16);
        const uint32_t hi = uint32_t(to_bf16(sum[2] * inverse)) | (uint32_t(to_bf16(sum[3] * inverse)) << 16);
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(out) + at) = u32x2{lo, hi};
    } else {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + at) = f32x4{sum[0] * inverse, sum[1] * inverse, sum[2] * inverse, sum[3] * inverse};
    }
}

// The vector combine as its own kernel per page count, so each keeps its own register count.
template <int QF, bool kTwoPages>
__global__ __launch_bounds__(kWave) void decode_combine_vector(DecodeArgs a, void* out) {
    combine_dim128<QF, kTwoPages>(a, out, blockIdx.x / a.query_heads, blockIdx.x % a.query_heads);
}

// Combine for 128-dim heads spread over four workgroups per (sequence, query head), one per
// quarter of the dims: lane l takes dims 32 q + 4 (l % 8) .. +3 of splits l / 8, l / 8 + 8, ...
// A lane loads a quarter of the rows combine_dim128 does (4 rather than 32 at 32 splits), so
// the one round trip to memory that the merge costs ends sooner.
template <int QF, bool kTwoPages>
__global__ __launch_bounds__(kWave) void decode_combine_quarter(DecodeArgs a, void* out) {
    constexpr uint32_t kPages = kTwoPages ? 2 : 1;
    constexpr uint32_t kGroups = 8, kRows = kPages * kWave / kGroups;
    const uint32_t lane = threadIdx.x, col = lane % kGroups, grp = lane / kGroups;
    const uint32_t quarter = blockIdx.x % 4, pair = blockIdx.x / 4;
    const uint32_t seq = pair / a.query_heads, qh = pair % a.query_heads;
    const int32_t length = a.lengths[uint64_t(seq) * a.lengths_stride];
    const uint64_t base = (uint64_t(seq) * a.query_heads + qh) * a.splits;
    const float* ml = a.partial_ml + 2 * base;
    const f32x4* acc = reinterpret_cast<const f32x4*>(a.partial_acc + base * kDim) + quarter * 8 + col;
    float lane_m[kPages], lane_l[kPages];
#pragma unroll
    for (uint32_t page = 0; page < kPages; ++page) {
        lane_m[page] = -INFINITY;
        lane_l[page] = 0.0f;
        if (page * kWave + lane < a.splits) {
            lane_m[page] = ml[2 * (page * kWave + lane)];
            lane_l[page] = ml[2 * (page * kWave + lane) + 1];
        }
    }
    f32x4 rows[kRows];
#pragma unroll
    for (uint32_t j = 0; j < kRows; ++j) {
        const uint32_t s = grp + kGroups * j;
        if (s < a.splits) rows[j] = acc[uint64_t(s) * (kDim / 4)];
    }
    const uint32_t used = (blocks_of(length, a.slots) + a.bps - 1) / a.bps;
    float top = -INFINITY;
#pragma unroll
    for (uint32_t page = 0; page < kPages; ++page) top = page * kWave + lane < used ? fmaxf(top, lane_m[page]) : top;
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) top = fmaxf(top, __shfl_xor(top, mask, kWave));
    float weight[kPages], total = 0.0f;
#pragma unroll
    for (uint32_t page = 0; page < kPages; ++page) {
        weight[page] = page * kWave + lane < used ? merge_weight(lane_m[page], top) : 0.0f;
        total += page * kWave + lane < used ? lane_l[page] * weight[page] : 0.0f;
    }
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) total += __shfl_xor(total, mask, kWave);
    f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (uint32_t j = 0; j < kRows; ++j) {
        const uint32_t s = grp + kGroups * j;
        const float w = __shfl(weight[j * kGroups / kWave], int(s % kWave), kWave);
        // Splits past the used ones hold anything: selected away, never multiplied by zero.
#pragma unroll
        for (int i = 0; i < 4; ++i) sum[i] = s < used ? fmaf(w, rows[j][i], sum[i]) : sum[i];
    }
#pragma unroll
    for (int mask = kGroups; mask < int(kWave); mask <<= 1)
#pragma unroll
        for (int i = 0; i < 4; ++i) sum[i] += __shfl_xor(sum[i], mask, kWave);
    if (grp != 0) return;
    const float inverse = 1.0f / total;
    const uint64_t at = (uint64_t(seq) * a.query_heads + qh) * kDim + 32 * quarter + 4 * col;
    if constexpr (QF == LK_BF16) {
        const uint32_t lo = uint32_t(to_bf16(sum[0] * inverse)) | (uint32_t(to_bf16(sum[1] * inverse)) << 16);
        const uint32_t hi = uint32_t(to_bf16(sum[2] * inverse)) | (uint32_t(to_bf16(sum[3] * inverse)) << 16);
        *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(out) + at) = u32x2{lo, hi};
    } else {
        *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(out) + at) = f32x4{sum[0] * inverse, sum[1] * inverse, sum[2] * inverse, sum[3] * inverse};
    }
}

__host__ inline bool vector_combine_fits(const DecodeArgs& a) { return a.vector_combine && a.head_dim == kDim && a.splits <= kVectorSplits; }

template <int QF>
__global__ __launch_bounds__(kWave) void decode_combine(DecodeArgs a, void* out) {

    // Latency-bound at small batch (one wave per (sequence, query head), a few KiB each): every
    // load that does not depend on another is issued at once. The sequence's length, the splits'
    // (m, l) pairs and the first kChunk splits' rows all go out together; splits past the ones
    // the sequence uses hold anything (the workspace is not initialized), so they are masked
    // by selects, never multiplied by zero.
    const uint32_t lane = threadIdx.x;
    const uint32_t qh = blockIdx.x % a.query_heads;
    const uint32_t seq = blockIdx.x / a.query_heads;
    const int32_t length = a.lengths[uint64_t(seq) * a.lengths_stride];
    const uint64_t base = (uint64_t(seq) * a.query_heads + qh) * a.splits;
    const float* ml = a.partial_ml + 2 * base;
    const float* acc = a.partial_acc + base * a.head_dim;
    constexpr uint32_t kPer = kMaxGenericDim / kWave;
    constexpr uint32_t kChunk = 16;
    // Lane s holds split s's (m, l) for the first kWave splits (more only beyond 64 splits).
    float lane_m = -INFINITY, lane_l = 0.0f;
    if (lane < a.splits) {
        lane_m = ml[2 * lane];
        lane_l = ml[2 * lane + 1];
    }
    auto load_rows = [&](uint32_t chunk, float (&rows)[kChunk][kPer]) {
#pragma unroll
        for (uint32_t u = 0; u < kChunk; ++u) {
            const float* row = acc + uint64_t(min(chunk + u, a.splits - 1)) * a.head_dim;
#pragma unroll
            for (uint32_t i = 0; i < kPer; ++i) {
                const uint32_t d = lane + i * kWave;
                rows[u][i] = d < a.head_dim ? row[d] : 0.0f;
            }
        }
    };
    float rows[kChunk][kPer];
    load_rows(0, rows);

    const uint32_t used = (blocks_of(length, a.slots) + a.bps - 1) / a.bps;
    // The largest running max over the used splits, then the total weight.
    float top = lane < used ? lane_m : -INFINITY;
    for (uint32_t s = lane + kWave; s < used; s += kWave) top = fmaxf(top, ml[2 * s]);
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) top = fmaxf(top, __shfl_xor(top, mask, kWave));
    float total = lane < used ? lane_l * merge_weight(lane_m, top) : 0.0f;
    for (uint32_t s = lane + kWave; s < used; s += kWave) total += ml[2 * s + 1] * merge_weight(ml[2 * s], top);
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) total += __shfl_xor(total, mask, kWave);
    const float inverse = 1.0f / total;

    // Lanes across dims: sum the used splits' accumulators, each split's weight broadcast from
    // the lane that holds its (m, l); the next chunk's rows are loaded before this one is summed.
    float sum[kPer];
#pragma unroll
    for (uint32_t i = 0; i < kPer; ++i) sum[i] = 0.0f;
    for (uint32_t chunk = 0; chunk < used; chunk += kChunk) {
        float next[kChunk][kPer];
        const bool more = chunk + kChunk < used;
        if (more) load_rows(chunk + kChunk, next);
        const uint32_t window = chunk & ~(kWave - 1);  // the 64 splits whose (m, l) lanes hold
        const float weight_lane = window == 0 ? (lane < used ? merge_weight(lane_m, top) : 0.0f)
                                              : (window + lane < used ? merge_weight(ml[2 * (window + lane)], top) : 0.0f);
#pragma unroll
        for (uint32_t u = 0; u < kChunk; ++u) {
            const uint32_t s = chunk + u;
            const float w = __shfl(weight_lane, int((s - window) % kWave), kWave);
#pragma unroll
            for (uint32_t i = 0; i < kPer; ++i) sum[i] = s < used ? fmaf(w, rows[u][i], sum[i]) : sum[i];
        }
        if (more) {
#pragma unroll
            for (uint32_t u = 0; u < kChunk; ++u)
#pragma unroll
                for (uint32_t i = 0; i < kPer; ++i) rows[u][i] = next[u][i];
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
