// Paged causal prefill attention on gfx950: a chunk of query tokens [start, start + tokens) of
// one sequence attends to every key [0, start + t] through the sequence's block ids, read in
// place from the pool (BF16 or FP8 records). The reference gathers the history out of the
// pool once per layer and runs FlashAttention with a bottom-right causal mask
// (layover/model.py:69-98; "reading it in place needs a paged prefill kernel"); the math here
// is the same causal softmax attention, with FP32 accumulation.
//
// Work: query rows are (token, query head) pairs of one KV head, head fastest, so the G heads
// sharing a KV head sit in adjacent rows. A wave owns 16 rows and walks the key blocks (16
// slots each) up to its last row's causal limit, on the matrix cores exactly as the decode
// kernel does for one block (decode_attention.h): S^T = K Q^T with v_mfma_f32_16x16x32_bf16
// (lane (g, n): keys 4g..4g+3 of row n), an online softmax per row with the lazy 2^8 rescale,
// and O += P V with v_mfma_f32_16x16x16_bf16 (lane (g, n): rows 4g..4g+3, dims 8n + e of
// MFMA e). P enters the MFMA as one BF16 (not the decode kernel's hi + lo pair): relative
// error at most 2^-8 per weight, against the north-star tolerance of 1e-2. Keys past a row's
// limit score -inf; V of slots at or past the chunk's end is zeroed, since those slots can
// hold anything (0 * NaN is NaN).
// Workgroups: 4 waves = 64 rows. Launch order: KV head fastest, and the heaviest row tiles
// (latest tokens, most keys) first. With 8 KV heads the round-robin dealing of workgroups
// onto the 8 XCDs then keeps each KV head's workgroups on one XCD, whose L2 holds that
// head's K/V for all of them.
#ifndef LAYOVER_AMD_PREFILL_ATTENTION_H
#define LAYOVER_AMD_PREFILL_ATTENTION_H

#include "decode_attention.h"

namespace lk {

constexpr uint32_t kPrefillWaves = 4;
constexpr uint32_t kPrefillRows = 16;  // rows per wave

struct PrefillArgs {
    const uint16_t* q;         // BF16 [query_heads, tokens, 128]
    const uint8_t* pool;
    const int32_t* block_ids;  // the sequence's blocks, at least ceil((start + tokens) / 16)
    uint16_t* out;             // BF16 [query_heads, tokens, 128]
    uint32_t tokens, start, query_heads, kv_heads, groups, layers, layer;
    uint32_t row_tiles;        // workgroups per KV head
    uint64_t block_bytes;
    float scale_log2;
    // Split-K (the LDS kernel only): workgroup (KV head, row tile, split) takes key steps
    // [split * split_steps, (split + 1) * split_steps) of its tile and, with key_splits > 1,
    // writes unnormalized partials [kv_heads, rows, key_splits] of (acc[128]) and (m, l)
    // instead of out; prefill_merge then combines them.
    uint32_t key_splits;       // 1: no split, results straight to out
    uint32_t split_steps;
    // Tile order of the LDS kernel. 0: heaviest first (causal tiles grow with their index), for
    // grids that run in several rounds. 1: the grid is resident at once (at most two
    // workgroups per CU): the first half of the order heaviest first, the second half lightest
    // first, so that the two workgroups that share a CU (w and w + half the grid, dealt
    // alike) carry about equal work together.
    uint32_t paired;
    float* partial_acc;
    float* partial_ml;
    // Paired key halves (paired grids without key splits, given a workspace). A CU pair is a
    // heavy tile's workgroup (order < half) and its partner (order + half), which takes the
    // light tile. When the heavy tile has more steps than half the pair's work, the heavy
    // workgroup stops at about that half and the partner takes the heavy tile's remaining
    // steps, then its own light tile. Each side writes its unnormalized state to
    // pair_state[(kv head, pair, side)] and swaps pair_tag | side into
    // pair_tags[(kv head, pair)] (pair: the light tile's index); the side that finds its
    // partner's tag of this launch there merges both, in side order, and writes out. Only the
    // first side stores its state, then publishes its tag in pair_ready[(kv head, pair)].
    // pair_tag is unique per launch, so neither word needs clearing. pair_bias (steps) moves the split
    // point toward the heavy side, for the partner's second prologue and epilogue.
    uint32_t pair_halves;
    int32_t pair_bias;
    uint64_t pair_tag;
    uint32_t* pair_state;
    uint64_t* pair_tags;
    uint64_t* pair_ready;
};

// Polls of a partner's ready word (each a memory round trip after a short sleep) before the
// merging side gives up and writes NaN: a few seconds, far beyond the microseconds a resident
// partner needs.
constexpr uint32_t kPairWaitBound = 1u << 22;
// A pair's words after its merge: odd with every bit set, never tag | side for an even tag
// below 2^64 - 2.
constexpr uint64_t kPairCleared = ~0ull;

// Floats of one workgroup's state in the pair merge: per thread, 64 accumulators of its rows
// and dims, then the 8 rows' maxima and 8 weight totals, in 16-byte pieces, thread-fastest.
constexpr uint32_t kPairStateFloats = 80;

// The running maximum of a row that has seen no key yet: finite, so that a weight taken
// against it is exp2(-inf) = 0 even when every score of the step is masked (a split can hold
// no visible key for some of its rows), and its merge weight exp2(kNoMax - m) underflows to 0.
constexpr float kNoMax = -1e30f;

template <int KV>
__global__ __launch_bounds__(kWave* kPrefillWaves) void prefill_mfma(PrefillArgs a) {
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t g = lane / 16;
    const uint32_t n = lane % 16;
    const uint32_t kv_head = blockIdx.x % a.kv_heads;
    const uint32_t tile = a.row_tiles - 1 - blockIdx.x / a.kv_heads;
    const uint32_t total_rows = a.tokens * a.groups;
    const uint32_t row0 = (tile * kPrefillWaves + wave) * kPrefillRows;
    if (row0 >= total_rows) return;

    // This lane's row n: its token, query head, and causal limit (last key position it sees).
    const uint32_t row = row0 + n;
    const bool live = row < total_rows;
    const uint32_t token = live ? row / a.groups : 0;
    const uint32_t head = kv_head * a.groups + (live ? row % a.groups : 0);
    const int64_t limit = live ? int64_t(a.start) + token : -1;
    const uint32_t last_row = min(row0 + kPrefillRows, total_rows) - 1;
    const uint32_t end = a.start + a.tokens;
    const uint32_t key_blocks = (a.start + last_row / a.groups) / kSlots + 1;

    // B operand of QK: row n, dims 32g .. 32g+31 (step j takes dims 32g + 8j .. +8).
    uint32_t qt[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) qt[i] = 0;
    if (live) {
        const u32x4* src = reinterpret_cast<const u32x4*>(a.q + (uint64_t(head) * a.tokens + token) * kDim + 32 * g);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4 w = src[j];
#pragma unroll
            for (int i = 0; i < 4; ++i) qt[4 * j + i] = w[i];
        }
    }

    constexpr uint32_t kElem = KV == LK_FP8_RECORD ? 1 : 2;
    const uint64_t tile_bytes = uint64_t(kSlots) * kDim * kElem;
    const uint64_t head_tile = uint64_t(a.layer) * a.kv_heads + kv_head;
    const uint64_t k_offset = head_tile * tile_bytes + (uint64_t(n) * kDim + 32 * g) * kElem;
    const uint64_t v_offset = (uint64_t(a.layers) * a.kv_heads + head_tile) * tile_bytes + (uint64_t(4 * g) * kDim + 8 * n) * kElem;
    const uint64_t block_elems = uint64_t(2) * a.layers * a.kv_heads * kSlots * kDim;

    auto fetch = [&](MfmaTile<KV>& t, uint32_t kb) {
        const int32_t block = a.block_ids[kb];  // uniform: a scalar load
        const uint8_t* base = a.pool + uint64_t(uint32_t(block)) * a.block_bytes;
        if constexpr (KV == LK_BF16) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const u32x4 w = reinterpret_cast<const u32x4*>(base + k_offset)[j];
#pragma unroll
                for (int x = 0; x < 4; ++x) t.k[4 * j + x] = w[x];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(base + v_offset + uint64_t(r) * kDim * kElem);
#pragma unroll
                for (int x = 0; x < 4; ++x) t.v[r][x] = w[x];
            }
        } else {
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const u32x4 w = reinterpret_cast<const u32x4*>(base + k_offset)[j];
#pragma unroll
                for (int x = 0; x < 4; ++x) t.k[4 * j + x] = w[x];
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const u32x2 w = *reinterpret_cast<const u32x2*>(base + v_offset + uint64_t(r) * kDim * kElem);
                t.v[r][0] = w[0];
                t.v[r][1] = w[1];
            }
            const int16_t* shifts = reinterpret_cast<const int16_t*>(base + block_elems);
            t.k_shift = shifts[head_tile];
            t.v_shift = shifts[uint64_t(a.layers) * a.kv_heads + head_tile];
        }
    };

    float m = -INFINITY, l = 0.0f;
    f32x4 o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) o[e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    auto consume = [&](MfmaTile<KV>& t, uint32_t kb) {
        const uint32_t key0 = kb * kSlots;
        bool k_exact = false, v_exact = false;
        float k_factor = a.scale_log2, v_factor = 1.0f;
        if constexpr (KV == LK_FP8_RECORD) {
            k_exact = !shift_is_exact_in_fp32(t.k_shift);
            v_exact = !shift_is_exact_in_fp32(t.v_shift);
            if (!k_exact) k_factor *= pow2(t.k_shift);
            if (!v_exact) v_factor = pow2(t.v_shift);
        }
        uint32_t kb_[16];
        uint32_t v[4][4];
        if constexpr (KV == LK_BF16) {
#pragma unroll
            for (int x = 0; x < 16; ++x) kb_[x] = t.k[x];
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int x = 0; x < 4; ++x) v[r][x] = t.v[r][x];
        } else {
            if (__builtin_expect(k_exact || v_exact, 0)) {
                asm volatile("" ::: "memory");
#pragma unroll
                for (int x = 0; x < 8; ++x) {
                    kb_[2 * x] = fp8_pair(t.k[x], false, k_exact, t.k_shift);
                    kb_[2 * x + 1] = fp8_pair(t.k[x], true, k_exact, t.k_shift);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int x = 0; x < 2; ++x) {
                        v[r][2 * x] = fp8_pair(t.v[r][x], false, v_exact, t.v_shift);
                        v[r][2 * x + 1] = fp8_pair(t.v[r][x], true, v_exact, t.v_shift);
                    }
            } else {
#pragma unroll
                for (int x = 0; x < 8; ++x) {
                    kb_[2 * x] = fp8_pair(t.k[x], false, false, 0);
                    kb_[2 * x + 1] = fp8_pair(t.k[x], true, false, 0);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int x = 0; x < 2; ++x) {
                        v[r][2 * x] = fp8_pair(t.v[r][x], false, false, 0);
                        v[r][2 * x + 1] = fp8_pair(t.v[r][x], true, false, 0);
                    }
            }
        }

        f32x4 s = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < 4; ++j)
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(kb_[4 * j], kb_[4 * j + 1], kb_[4 * j + 2], kb_[4 * j + 3]),
                                                        as_bf16x8(qt[4 * j], qt[4 * j + 1], qt[4 * j + 2], qt[4 * j + 3]), s, 0, 0, 0);

        float score[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) score[r] = int64_t(key0 + 4 * g + r) <= limit ? s[r] * k_factor : -INFINITY;
        const float top = max_over_lane_groups(fmaxf(fmaxf(score[0], score[1]), fmaxf(score[2], score[3])));
        if (__builtin_expect(__any(top > m + kRescaleThreshold), 0)) {
            asm volatile("" ::: "memory");
            const float next = top > m + kRescaleThreshold ? top : m;
            const float alpha = merge_weight(m, next);
            m = next;
            l *= alpha;
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
        const s16x4 pb = __builtin_bit_cast(s16x4, u32x2{pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3])});

        if (key0 + kSlots > end) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool written = key0 + 4 * g + r < end;
#pragma unroll
                for (int x = 0; x < 4; ++x) v[r][x] = written ? v[r][x] : 0u;
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint32_t select = (e & 1) ? 0x07060302u : 0x05040100u;
            const uint32_t b01 = __builtin_amdgcn_perm(v[1][e / 2], v[0][e / 2], select);
            const uint32_t b23 = __builtin_amdgcn_perm(v[3][e / 2], v[2][e / 2], select);
            o[e] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(pb, __builtin_bit_cast(s16x4, u32x2{b01, b23}), o[e], 0, 0, 0);
        }
    };

    // Register ring, refilled unconditionally (see decode_split_mfma).
    constexpr int kRing = KV == LK_BF16 ? LK_DECODE_RING_BF16 : LK_DECODE_RING_FP8;
    MfmaTile<KV> ring[kRing];
    const uint32_t last = key_blocks - 1;
#pragma unroll
    for (int d = 0; d < kRing; ++d) fetch(ring[d], min(uint32_t(d), last));
    for (uint32_t i = 0; i < key_blocks; i += kRing) {
#pragma unroll
        for (int d = 0; d < kRing; ++d) {
            if (i + d < key_blocks) consume(ring[d], i + d);
            fetch(ring[d], min(i + d + kRing, last));
        }
    }

    // Row n's weight sum over the four lane groups, then O rows 4g + r scaled by 1 / l of
    // their row (held by lane 4g + r) and written as BF16, 16 bytes (dims 8n .. 8n+7) a row.
    l += __shfl_xor(l, 16, kWave);
    l += __shfl_xor(l, 32, kWave);
    const float inverse = 1.0f / l;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float factor = __shfl(inverse, int(4 * g + r), kWave);
        const uint32_t out_row = row0 + 4 * g + r;
        if (out_row < total_rows) {
            const uint32_t out_token = out_row / a.groups;
            const uint32_t out_head = kv_head * a.groups + out_row % a.groups;
            u32x4 packed;
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const uint32_t lo = to_bf16(o[2 * x][r] * factor), hi = to_bf16(o[2 * x + 1][r] * factor);
                packed[x] = lo | (hi << 16);
            }
            *reinterpret_cast<u32x4*>(a.out + (uint64_t(out_head) * a.tokens + out_token) * kDim + 8 * n) = packed;
        }
    }
}

// ---------------------------------------------------------------------------------------
// K/V shared through LDS. A workgroup of 4 waves owns 128 rows (32 per wave, as two sets of
// 16) and walks the keys in steps of 32 (two blocks). Each step's K and V tiles (4 x 4 KiB)
// are loaded once per workgroup: for BF16 pools by direct-to-LDS copies into four buffers,
// steps going in pairs (the next pair's copies issued when a pair starts, one barrier per
// pair), for FP8 pools through registers one step ahead (the codes become BF16 on the way)
// into one of two. Per wave and step:
//   QK   for each block and set, four v_mfma_f32_16x16x32_bf16 on K read from LDS (lane
//        (g, n): key n, dims 32g + 8j .. +8), reused by both sets;
//   P    8 scores per lane (keys 4g..4g+3 of each block) of row n;
//   PV   v_mfma_f32_16x16x32_bf16 over the step's 32 keys for output dims 16e .. 16e+15: the
//        MFMA's k index 8g + i stands for key 4g + i of block 0 (i < 4) or of block 1
//        (i >= 4), in both P (the lane's own 8 weights, as BF16) and V. V stays row-major in
//        LDS (a key per row) and reaches the B operand through the transposing read
//        ds_read_b64_tr_b16: within a 16-lane group, lane i receives element i % 4 of the
//        8-byte rows fetched by lanes i / 4 + 4t (t = 0..3). Lane 4t + q of group g fetches
//        key 4g + t, dims 16e + 4q .. +3, so lane n receives keys 4g..4g+3 of dim 16e + n,
//        which is its B operand half for that block, with no register shuffles.
//   sum  BF16 pools: the weight sums come from one more MFMA of P against a B of ones, so
//        they land in the layout of O (lane (g, n): rows 4g + r) and use the same rounded
//        weights as the numerator. FP8 pools weight P by the V block's 2^shift, so their
//        sums stay per-lane VALU adds of the unscaled weights.
// Causal masking runs only in steps that reach past the wave's first row's limit (the later
// rows of a wave only see more keys). The tiles' LDS layout (k_slot, v_slot below) has no row
// padding, which direct-to-LDS copies cannot write, and is swizzled instead so that the K reads
// hit distinct banks and the V reads stay within one region.
// Registers are held to 256 per lane (amdgpu_waves_per_eu(2)), so two workgroups share a CU
// and one computes while the other waits at its step barrier. Measured on MI355X at a
// 2,048-token chunk ending a 32,768-token context: 2.97 ms per layer at one wave per SIMD and
// 1.61 ms at two; 1.39 ms with conflict-free LDS stores, one FMA per weight's exponent, 32-bit
// causal compares and permlane-swapped row maxima, with V regrouped by 32 v_perm per step;
// 1.18 ms with the transposing V reads, per-set stretches, masks only where needed and the
// sums on the matrix cores; 1.13 ms with the lane-local rescale check; 1.10 ms with the
// direct-to-LDS copies two steps ahead into the swizzled layout. Steps in pairs with one
// barrier per pair (four buffers) against a barrier per step (three): 1.064-1.077 -> 1.059-1.067
// ms there (on a slower box), and 0.060-0.062 -> 0.058 ms for a 2,048-token chunk at position 0.
// O leaves through LDS: its rows are spread over lanes by dim (16e + n), so each wave writes
// its 32 rows there and reads them back as 16-byte pieces of whole rows.
constexpr uint32_t kLdsWaves = 4;
constexpr uint32_t kLdsRows = 32;                        // rows per wave
constexpr uint32_t kLdsRowBytes = kDim * 2 + 16;         // 272: rows of the output staging
// A step's tiles (K0, K1, V0, V1: 16 keys x 256 bytes each) are laid out without row padding,
// each as four 1 KiB regions 16 bytes apart; a region is what one 16-byte-per-lane copy of a
// wave fills. K region x holds keys 4x .. 4x+3, their 16-byte chunks XOR-swizzled by
// 4 * (key % 4), so the 16 lanes reading one chunk of 16 keys hit 16 different bank quads.
// V region x holds chunks 4x .. 4x+3 (dims 32x .. 32x+31) of all 16 keys, 64 bytes a key, so
// the transposing reads (keys 4g .. 4g+3, 8 bytes each, of one dim group) stay in one region.
constexpr uint32_t kRegionStride = 1024 + 16;
constexpr uint32_t kLdsTile = 4 * kRegionStride;         // one block's K or V
constexpr uint32_t kLdsStep = 4 * kLdsTile;              // K0, K1, V0, V1
constexpr uint32_t kLdsAllocated = 4;  // step buffers allocated (FP8 rotates through two)
static_assert(kLdsWaves * kLdsRows * kLdsRowBytes <= 3 * kLdsStep, "the output staging must fit three step buffers");

// Byte offset of key `key`'s 16-byte chunk `chunk` (dims 8 chunk .. +8) inside a K or V tile.
__device__ __forceinline__ uint32_t k_slot(uint32_t key, uint32_t chunk) {
    return (key / 4) * kRegionStride + (key % 4) * 256 + 16 * (chunk ^ (4 * (key % 4)));
}
__device__ __forceinline__ uint32_t v_slot(uint32_t key, uint32_t chunk) {
    return (chunk / 4) * kRegionStride + key * 64 + 16 * (chunk % 4);
}

// BF16 pools copy each pair of steps straight into LDS one pair ahead (four buffers); FP8
// pools convert their codes on the way, through registers, one step ahead (two buffers).
template <int KV>
constexpr uint32_t lds_buffers() {
    return KV == LK_BF16 ? 4 : 2;
}
constexpr uint32_t kCopiesPerStep = 4;  // 16-byte-per-lane copies per wave and step (BF16)

typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// FP8-record pools: each thread converts its 32 codes to BF16 as it stages them (the exact
// hardware convert), and each block's 2^shift is applied to that block's scores (K) and
// weights (V), one factor per block and step kept beside the tiles in LDS. A block whose shift
// could leave BF16's normal range is decoded exactly with the shift included (the reference's
// decode_bits) and gets factor 1.
struct PrefillStaged {
    // BF16: 64 bytes; FP8: w0 and w1 hold 32 codes. Named registers, not an array, so that the
    // compiler keeps them in VGPRs (an indexed array here ended up in scratch memory).
    u32x4 w0, w1, w2, w3;
    int32_t shift;
};

template <int KV>
__global__ __launch_bounds__(kWave* kLdsWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_mfma_lds(PrefillArgs a) {
    constexpr uint32_t kLdsBuffers = lds_buffers<KV>();
    static_assert(kLdsBuffers <= kLdsAllocated, "more step buffers than allocated");
    __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsBuffers > 3 ? kLdsBuffers : 3][kLdsStep];
    __shared__ int32_t lds_shift[kLdsBuffers][4];  // FP8: per buffer, the shift of K0, K1, V0, V1
    __shared__ uint32_t pair_merges;               // this workgroup merges its pair's states
    __shared__ uint32_t pair_lost;                 // ... but its partner's state never came
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t g = lane / 16;
    const uint32_t n = lane % 16;
    // KV head fastest (a head's workgroups stay on one XCD), then the splits of a tile, then
    // the tiles, heaviest first, or paired (see PrefillArgs::paired). Measured on MI355X,
    // 2,048-token chunk at position 0 (512 workgroups, two per CU): 62.7 -> 57.4 us per layer
    // paired; chunks of 1,024 and 4,096 tokens unchanged.
    const uint32_t kv_head = blockIdx.x % a.kv_heads;
    const uint32_t split = (blockIdx.x / a.kv_heads) % a.key_splits;
    const uint32_t order = blockIdx.x / (a.kv_heads * a.key_splits);
    const uint32_t half = (a.row_tiles + 1) / 2;
    const uint32_t total_rows = a.tokens * a.groups;
    const uint32_t end = a.start + a.tokens;
    const uint32_t last_block = (end + kSlots - 1) / kSlots - 1;
    // Key steps of a tile: up to its last row's limit, in steps of two blocks.
    auto steps_of = [&](uint32_t t) __attribute__((always_inline)) {
        const uint32_t last_row = min((t + 1) * kLdsWaves * kLdsRows, total_rows) - 1;
        const uint32_t key_blocks = (a.start + last_row / a.groups) / kSlots + 1;
        return (key_blocks + 1) / 2;
    };

    // Jobs: (tile, steps [first, last), pair part 0 none / 1 heavy side / 2 partner side).
    uint32_t jobs = 1;
    uint32_t job_tile[2], job_first[2], job_last[2], job_part[2];
    {
        const uint32_t tile = a.paired && order >= half ? order - half : a.row_tiles - 1 - order;
        const uint32_t tile_steps = steps_of(tile);
        job_tile[0] = tile;
        job_first[0] = min(split * a.split_steps, tile_steps);
        job_last[0] = min(job_first[0] + a.split_steps, tile_steps);
        job_part[0] = 0;
        if (a.pair_halves) {
            // The heavy tile of this CU pair and where its steps divide: about equal work on
            // both sides; no division when the light tile already carries as much.
            const uint32_t light = order < half ? order : order - half;
            const bool partnered = light + half < a.row_tiles;
            const uint32_t heavy = a.row_tiles - 1 - light;
            const uint32_t heavy_steps = steps_of(heavy);
            const int64_t share = (int64_t(heavy_steps) + steps_of(light) + a.pair_bias + 1) / 2;
            const uint32_t cut = uint32_t(share < 1 ? 1 : share);
            // Only when the moved steps are worth a merge: at least an eighth of the tile (long
            // histories, where paired tiles differ by a few percent, stay whole).
            if (partnered && cut < heavy_steps && (heavy_steps - cut) * 8 >= heavy_steps) {
                if (order < half) {
                    job_last[0] = cut;
                    job_part[0] = 1;
                } else {
                    // The heavy tile's remaining steps first, its own light tile after: its
                    // state is then out early and the heavy side, which finishes later,
                    // merges. Measured on MI355X (2,048 tokens at position 0): 0.049 ms per
                    // layer against 0.051-0.052 with the light tile first (each at its best
                    // pair_bias).
                    jobs = 2;
                    job_tile[1] = job_tile[0];
                    job_first[1] = job_first[0];
                    job_last[1] = job_last[0];
                    job_part[1] = 0;
                    job_tile[0] = heavy;
                    job_first[0] = cut;
                    job_last[0] = heavy_steps;
                    job_part[0] = 2;
                }
            }
        }
    }

    // Per set: row n's token, head and causal limit; Q as the QK B operand. A job's Q is
    // loaded before its loop (the first job) or, in the BF16 kernel, as the previous job's loop
    // ends, so that the round trip overlaps that job's epilogue.
    int32_t limit[2];
    uint32_t qt[2][16];
    auto load_q = [&](uint32_t tile) __attribute__((always_inline)) {
#pragma unroll
        for (int set = 0; set < 2; ++set) {
            const uint32_t row = tile * kLdsWaves * kLdsRows + wave * kLdsRows + 16 * set + n;
            const bool live = row < total_rows;
            const uint32_t token = live ? row / a.groups : 0;
            const uint32_t head = kv_head * a.groups + (live ? row % a.groups : 0);
            limit[set] = live ? int32_t(a.start + token) : -1;
#pragma unroll
            for (int i = 0; i < 16; ++i) qt[set][i] = 0;
            if (live) {
                const u32x4* src = reinterpret_cast<const u32x4*>(a.q + (uint64_t(head) * a.tokens + token) * kDim + 32 * g);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const u32x4 w = src[j];
#pragma unroll
                    for (int i = 0; i < 4; ++i) qt[set][4 * j + i] = w[i];
                }
            }
        }
    };
    if constexpr (KV == LK_BF16) load_q(job_tile[0]);

    for (uint32_t job = 0; job < jobs; ++job) {
    const uint32_t tile = job_tile[job];
    if constexpr (KV != LK_BF16) load_q(tile);
    const uint32_t wg_row0 = tile * kLdsWaves * kLdsRows;
    const uint32_t row0 = wg_row0 + wave * kLdsRows;
    // This job's steps [first_step, steps); a split past the tile's keys does none.
    const uint32_t first_step = job_first[job];
    const uint32_t steps = job_last[job];
    // The wave's first row's limit (later rows only see more keys); -1 for a wave past the end.
    const int64_t first_limit = row0 < total_rows ? int64_t(a.start) + row0 / a.groups : -1;

    // Cooperative step loads: wave w brings tile w (K0, K1, V0, V1). Chunk x of lane t is
    // values 512x + 8t .. +8 of the tile (16 bytes of BF16, or 8 FP8 codes that become 16
    // bytes of BF16), so each wave-wide load reads 1 KiB (or 512 bytes) contiguous, and each
    // LDS store fills whole 256-byte rows, 16 lanes a row.
    constexpr uint32_t kElem = KV == LK_FP8_RECORD ? 1 : 2;
    const uint32_t part = threadIdx.x / kWave;          // which tile
    const uint32_t piece = threadIdx.x % kWave;         // which 8 values of each 512
    const uint64_t tile_bytes = uint64_t(kSlots) * kDim * kElem;
    const uint64_t head_tile = uint64_t(a.layer) * a.kv_heads + kv_head;
    const uint64_t group = part < 2 ? head_tile : uint64_t(a.layers) * a.kv_heads + head_tile;
    const uint64_t part_offset = group * tile_bytes + uint64_t(piece) * 8 * kElem;
    const uint64_t block_elems = uint64_t(2) * a.layers * a.kv_heads * kSlots * kDim;
    // Value 512x + 8t of a tile is key 4x + t / 16, chunk t % 16; where it goes in LDS:
    const uint32_t tile_lds = part * kLdsTile;
    auto slot_of = [&](uint32_t x) __attribute__((always_inline)) {
        const uint32_t key = 4 * x + piece / 16, chunk = piece % 16;
        return tile_lds + (part < 2 ? k_slot(key, chunk) : v_slot(key, chunk));
    };
    auto load_step = [&](uint32_t step, PrefillStaged& r) __attribute__((always_inline)) {
        const uint32_t block_index = min(2 * step + (part & 1), last_block);
        const int32_t block = a.block_ids[block_index];
        const uint8_t* base = a.pool + uint64_t(uint32_t(block)) * a.block_bytes + part_offset;
        const u32x2 c0 = *reinterpret_cast<const u32x2*>(base), c1 = *reinterpret_cast<const u32x2*>(base + 512);
        const u32x2 c2 = *reinterpret_cast<const u32x2*>(base + 1024), c3 = *reinterpret_cast<const u32x2*>(base + 1536);
        r.w0 = u32x4{c0[0], c0[1], c1[0], c1[1]};
        r.w1 = u32x4{c2[0], c2[1], c3[0], c3[1]};
        r.shift = reinterpret_cast<const int16_t*>(a.pool + uint64_t(uint32_t(block)) * a.block_bytes + block_elems)[group];
    };
    auto store_step = [&](uint32_t buffer, const PrefillStaged& r) __attribute__((always_inline)) {
        uint8_t* dst = lds[buffer];
        // Chunk x's 8 codes are words (2x, 2x + 1) of w0, w1.
        const bool exact = !shift_is_exact_in_fp32(r.shift);
        auto convert = [&](uint32_t lo, uint32_t hi) __attribute__((always_inline)) {
            return u32x4{fp8_pair(lo, false, exact, r.shift), fp8_pair(lo, true, exact, r.shift), fp8_pair(hi, false, exact, r.shift),
                         fp8_pair(hi, true, exact, r.shift)};
        };
        *reinterpret_cast<u32x4*>(dst + slot_of(0)) = convert(r.w0[0], r.w0[1]);
        *reinterpret_cast<u32x4*>(dst + slot_of(1)) = convert(r.w0[2], r.w0[3]);
        *reinterpret_cast<u32x4*>(dst + slot_of(2)) = convert(r.w1[0], r.w1[1]);
        *reinterpret_cast<u32x4*>(dst + slot_of(3)) = convert(r.w1[2], r.w1[3]);
        if (piece == 0) lds_shift[buffer][part] = r.shift;
    };

    // BF16 pools: wave w copies tile w of a step straight into its LDS buffer, one 1 KiB region
    // per instruction (lane t writes bytes 16t .. 16t+15 of the region), so lane t fetches the
    // chunk the layout puts there: for K key 4x + t/16, chunk (t % 16) ^ 4(t/16); for V key
    // t/4, chunk 4x + t % 4. The copies are issued as inline assembly, which the compiler's wait
    // counting does not see (it would otherwise wait for them before any LDS read it cannot
    // prove disjoint); they are waited for only at the barrier before their step is read (the
    // pair's step_barrier, which waits for all of this wave's vector-memory operations; block ids are
    // scalar loads).
    const auto* scalar_ids = (const __attribute__((address_space(4))) int32_t*)a.block_ids;
    const uint32_t wave_part = __builtin_amdgcn_readfirstlane(part);
    const uint32_t copy_src = wave_part < 2 ? (piece / 16) * 256 + 16 * ((piece % 16) ^ (4 * (piece / 16))) : (piece / 4) * 256 + 16 * (piece % 4);
    const uint32_t copy_step = wave_part < 2 ? 1024 : 64;  // source bytes between regions
    const uint64_t copy_tile = group * tile_bytes;
    auto copy_step_tiles = [&](uint32_t step) __attribute__((always_inline)) {
        const uint32_t block_index = min(2 * step + (wave_part & 1), last_block);
        const uint32_t block = uint32_t(scalar_ids[block_index]);
        const uint8_t* src = a.pool + uint64_t(block) * a.block_bytes + copy_tile + copy_src;
        const uint32_t dst = uint32_t(uintptr_t((__attribute__((address_space(3))) uint8_t*)(lds[step % kLdsBuffers] + tile_lds)));
        // An LDS-DMA load reads its LDS address from M0, and a scalar write of M0 needs one wait
        // state before such a load (the compiler inserts it for its own code but cannot see
        // into this asm): without the s_nop a copy could take the previous copy's M0 and land
        // in the wrong region, depending on how other waves' instructions interleave.
#pragma unroll
        for (uint32_t x = 0; x < kCopiesPerStep; ++x)
            asm volatile("s_mov_b32 m0, %1\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src + copy_step * x),
                         "s"(__builtin_amdgcn_readfirstlane(dst + kRegionStride * x))
                         : "memory", "m0");
    };
    // The end of a BF16 pair of steps: this wave's copies of the next pair must have landed,
    // and every LDS read of this pair must be done before any wave refills its buffers.
    auto step_barrier = [&]() __attribute__((always_inline)) {
        asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    };

    // Running maximum per row (lane (g, n): row n of each set); output and, for BF16 pools,
    // weight sums in the MFMA output layout (lane (g, n): rows 4g + r, dims 16e + n).
    float m[2] = {kNoMax, kNoMax}, l[2] = {0.0f, 0.0f};
    f32x4 o[2][8], sums[2];
#pragma unroll
    for (int set = 0; set < 2; ++set) {
        sums[set] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < 8; ++e) o[set][e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    }
    const bf16x8 ones = as_bf16x8(0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u);

    // Transposing V reads: lane 4t + q of group g fetches key 4g + t, dims 16e + 4q .. +3,
    // i.e. bytes 8q .. 8q+7 of chunks 2e, 2e + 1 (region e / 2, offset 32 (e % 2)).
    const uint32_t v_read = 2 * kLdsTile + (4 * g + n / 4) * 64 + (n % 4) * 8;
    // K reads: lane (g, n) reads key n's chunks 4g .. 4g+3, stored at 4(g ^ (n % 4)) + j.
    const uint32_t k_read = (n / 4) * kRegionStride + (n % 4) * 256 + 64 * (g ^ (n % 4));

    // Per step: the scale of each block's scores (log2 units) and of its weights.
    struct Factors {
        float k[2];
        float v[2];
    };
    auto factors = [&](uint32_t step) __attribute__((always_inline)) {
        Factors f{{a.scale_log2, a.scale_log2}, {1.0f, 1.0f}};
        if constexpr (KV == LK_FP8_RECORD) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int32_t ks = lds_shift[step % kLdsBuffers][b], vs = lds_shift[step % kLdsBuffers][2 + b];
                if (shift_is_exact_in_fp32(ks)) f.k[b] *= pow2(ks);
                if (shift_is_exact_in_fp32(vs)) f.v[b] = pow2(vs);
            }
        }
        return f;
    };

    // K of a step as A operands (lane (g, n): key n, dims 32g + 8j .. +8), then one set's scores
    // S^T = K Q^T for both blocks.
    auto read_k = [&](uint32_t step, bf16x8 (&kk)[2][4]) __attribute__((always_inline)) {
        const uint8_t* buf = lds[step % kLdsBuffers];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const uint8_t* k_row = buf + b * kLdsTile + k_read;
#pragma unroll
            for (int j = 0; j < 4; ++j) kk[b][j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(k_row + 16 * j));
        }
    };
    auto scores = [&](int set, const bf16x8 (&kk)[2][4], f32x4 (&s)[2]) __attribute__((always_inline)) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                    kk[b][j], as_bf16x8(qt[set][4 * j], qt[set][4 * j + 1], qt[set][4 * j + 2], qt[set][4 * j + 3]), acc, 0, 0, 0);
            s[b] = acc;
        }
    };

    // V of a step as B operands, one per 16 output dims: keys 4g..4g+3 of block 0, then of
    // block 1, for dim 16e + n, as four BF16 pairs.
    auto values = [&](uint32_t step, u32x4 (&vb)[8]) __attribute__((always_inline)) {
        const auto* buf = (const __attribute__((address_space(3))) uint8_t*)(lds[step % kLdsBuffers]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const auto* at = buf + v_read + (e / 2) * kRegionStride + 32 * (e % 2);
            const i16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(at));
            const i16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(at + kLdsTile));
            const u32x2 w0 = __builtin_bit_cast(u32x2, v0), w1 = __builtin_bit_cast(u32x2, v1);
            vb[e] = u32x4{w0[0], w0[1], w1[0], w1[1]};
        }
    };

    // Keys past a row's limit become -inf, for the maximum and the weight alike (exp2(-inf)
    // = 0: every live row sees key 0 in the first step, so m is finite).
    auto mask = [&](uint32_t step, int set, f32x4 (&s)[2]) __attribute__((always_inline)) {
        const uint32_t key0 = step * 2 * kSlots;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (int32_t(key0 + b * kSlots + 4 * g + r) > limit[set]) s[b][r] = -INFINITY;
    };

    // Rescaling. The state of a row is rescaled only when a score exceeds its running maximum
    // by more than kRescaleThreshold (log2 units), which is rare after the first steps. The
    // common path therefore only compares each lane's own maximum with a precomputed limit:
    // for BF16 pools on the raw scores against (m + threshold) / scale, for FP8 pools on the
    // scaled scores of each block. Only when some lane exceeds it are the row maxima reduced
    // over the lane groups (row n lives in lanes n, n + 16, n + 32, n + 48) and the state
    // rescaled. A lane that misses the limit by rounding at most lets a weight reach 2^8 times
    // an ulp more, which the threshold exists to bound anyway.
    float raw_limit[2] = {-INFINITY, -INFINITY};  // BF16: (m + threshold) / scale per set
    auto lane_max = [&](const f32x4 (&s)[2], const Factors& f) __attribute__((always_inline)) {
        if constexpr (KV == LK_BF16) {
            return fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])), fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
        } else {
            float top_b[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) top_b[b] = fmaxf(fmaxf(fmaxf(s[b][0], s[b][1]), s[b][2]), s[b][3]) * f.k[b];
            return fmaxf(top_b[0], top_b[1]);
        }
    };
    auto exceeds = [&](int set, float lane_top) __attribute__((always_inline)) {
        if constexpr (KV == LK_BF16) return lane_top > raw_limit[set];
        else return lane_top > m[set] + kRescaleThreshold;
    };
    auto rescale = [&](const float (&lane_top)[2]) __attribute__((always_inline)) {
        if (__builtin_expect(__any(exceeds(0, lane_top[0]) || exceeds(1, lane_top[1])), 0)) {
            asm volatile("" ::: "memory");
#pragma unroll
            for (int set = 0; set < 2; ++set) {
                float top = max_over_lane_groups(lane_top[set]);
                if constexpr (KV == LK_BF16) top *= a.scale_log2;
                const float next = top > m[set] + kRescaleThreshold ? top : m[set];
                const float alpha = merge_weight(m[set], next);
                m[set] = next;
                if constexpr (KV == LK_BF16) raw_limit[set] = (next + kRescaleThreshold) / a.scale_log2;
                l[set] *= alpha;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float factor = __shfl(alpha, int(4 * g + r), kWave);
                    sums[set][r] *= factor;
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[set][e][r] *= factor;
                }
            }
        }
    };

    // One set's weights as a BF16 A operand (each exponent one FMA); FP8 pools weight each
    // block by its V factor and keep the unscaled sums per lane.
    auto weights = [&](int set, const f32x4 (&s)[2], const Factors& f) __attribute__((always_inline)) {
        float p[8];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float w = exp2_fast(fmaf(s[b][r], f.k[b], -m[set]));
                if constexpr (KV == LK_BF16) {
                    p[4 * b + r] = w;
                } else {
                    l[set] += w;
                    p[4 * b + r] = w * f.v[b];
                }
            }
        return as_bf16x8(pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]), pack_bf16(p[4], p[5]), pack_bf16(p[6], p[7]));
    };

    // One set's PV (and, for BF16 pools, its weight sums).
    auto accumulate = [&](int set, const bf16x8& pb, const u32x4 (&vb)[8]) __attribute__((always_inline)) {
        if constexpr (KV == LK_BF16) sums[set] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pb, ones, sums[set], 0, 0, 0);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            o[set][e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pb, __builtin_bit_cast(bf16x8, vb[e]), o[set][e], 0, 0, 0);
    };

    PrefillStaged staged;
    // One step, per set: scores, mask and maximum, then (after a rare rescale of both sets)
    // weights and PV, in two straight stretches that the scheduler fills from both sets. Then
    // the next step's tiles go into the other buffer and the one after into registers. Steps
    // that need the causal mask (and the chunk-end V mask, which only the last step can need)
    // run in a second copy of the loop. Forcing an MFMA/VALU interleave with scheduling
    // barriers measured 4% slower: the two waves on each SIMD already overlap each other.
    auto run_step = [&](uint32_t step, auto masked_tag) __attribute__((always_inline)) {
        constexpr bool kMasked = decltype(masked_tag)::value;
        if constexpr (KV == LK_BF16) {
            // Steps go in pairs (first_step + 2i, + 2i + 1): the next pair's copies go out
            // when a pair starts, and only the pair's last step ends at the barrier.
            if ((step - first_step) % 2 == 0) {
                if (step + 2 < steps) copy_step_tiles(step + 2);
                if (step + 3 < steps) copy_step_tiles(step + 3);
            }
        }
        const Factors f = factors(step);
        bf16x8 kk[2][4];
        read_k(step, kk);
        u32x4 vb[8];
        values(step, vb);
        f32x4 s[2][2];
        scores(0, kk, s[0]);
        scores(1, kk, s[1]);
        if constexpr (kMasked) mask(step, 0, s[0]);
        float top[2];
        // The softmax stretch (row maxima, rescale, exponentials, with set 0's PV in between)
        // runs at raised wave priority: the SIMD's other wave is then mostly in its matrix-core
        // stretch, whose MFMAs keep running while this wave's dependent VALU chain is issued
        // first. Measured on MI355X (2,048 tokens ending a 32,768 context): 1.094 -> 1.023 ms
        // per layer; raising it for the QK MFMAs instead, or dropping it around set 0's PV, was
        // 1.08-1.11 and 1.07 ms. With the steps paired it still gains 1-2% there (1.059-1.067
        // against 1.079-1.081 ms on one box), and under the max-ilp scheduling the prefill kernels
        // build with (0.991-1.001 against 1.003-1.010 ms).
        __builtin_amdgcn_s_setprio(1);
        top[0] = lane_max(s[0], f);
        if constexpr (kMasked) {
            mask(step, 1, s[1]);
            // Keys at or past the chunk's end hold anything: zero their V (0 * NaN is NaN).
            const uint32_t key0 = step * 2 * kSlots;
            if (key0 + 2 * kSlots > end) {
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const int32_t first = int32_t(key0 + b * kSlots + 4 * g);
                    const int32_t valid = min(max(int32_t(end) - first, 0), 4);
                    const uint32_t lo = valid >= 2 ? 0xFFFFFFFFu : valid == 1 ? 0x0000FFFFu : 0u;
                    const uint32_t hi = valid >= 4 ? 0xFFFFFFFFu : valid == 3 ? 0x0000FFFFu : 0u;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        vb[e][2 * b] &= lo;
                        vb[e][2 * b + 1] &= hi;
                    }
                }
            }
        }
        top[1] = lane_max(s[1], f);
        rescale(top);
        const bf16x8 p0 = weights(0, s[0], f);
        accumulate(0, p0, vb);
        const bf16x8 p1 = weights(1, s[1], f);
        __builtin_amdgcn_s_setprio(0);
        accumulate(1, p1, vb);
        if constexpr (KV == LK_BF16) {
            if ((step - first_step) % 2 == 1 || step + 1 == steps) step_barrier();
        } else {
            if (step + 1 < steps) {
                store_step((step + 1) % kLdsBuffers, staged);
                if (step + 2 < steps) load_step(step + 2, staged);
            }
            __syncthreads();
        }
    };

    if (first_step < steps) {
        if constexpr (KV == LK_BF16) {
            // Q's loads must be complete (and known to be) before the first copy: a wait for
            // them inside the loop would count the copies issued after them.
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            copy_step_tiles(first_step);
            if (first_step + 1 < steps) copy_step_tiles(first_step + 1);
            step_barrier();  // the first pair's tiles are in
        } else {
            load_step(first_step, staged);
            store_step(first_step % kLdsBuffers, staged);
            if (first_step + 1 < steps) load_step(first_step + 1, staged);
            __syncthreads();
        }
        // Steps whose 32 keys all lie at or below the wave's first row's limit need no mask.
        const uint32_t unmasked = first_limit < 0 ? 0u : min(steps, uint32_t((first_limit + 1) / (2 * kSlots)));
        uint32_t step = first_step;
        for (; step < unmasked; ++step) run_step(step, std::false_type{});
        for (; step < steps; ++step) run_step(step, std::true_type{});
    }
    // This job's Q and limits are done with. (The FP8 kernel loads the next job's Q at its
    // start instead: held across this epilogue it would spill.)
    if constexpr (KV == LK_BF16) {
        if (job + 1 < jobs) load_q(job_tile[job + 1]);
    }

    if (a.key_splits > 1) {
        // Unnormalized partials of this split: lane (g, n) holds rows 4g + r of each set (dims
        // 16e + n); the row's running maximum lives in lane 4g + r (row n of the score layout).
#pragma unroll
        for (int set = 0; set < 2; ++set) {
            float row_l;
            if constexpr (KV == LK_BF16) {
                row_l = 0.0f;
            } else {
                row_l = l[set];
                row_l += __shfl_xor(row_l, 16, kWave);
                row_l += __shfl_xor(row_l, 32, kWave);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float row_m = __shfl(m[set], int(4 * g + r), kWave);
                const float total = KV == LK_BF16 ? sums[set][r] : __shfl(row_l, int(4 * g + r), kWave);
                const uint32_t row = row0 + 16 * set + 4 * g + r;
                if (row >= total_rows) continue;
                const uint64_t slot = (uint64_t(kv_head) * total_rows + row) * a.key_splits + split;
#pragma unroll
                for (int e = 0; e < 8; ++e) a.partial_acc[slot * kDim + 16 * e + n] = o[set][e][r];
                if (n == 0) {
                    a.partial_ml[2 * slot] = row_m;
                    a.partial_ml[2 * slot + 1] = total;
                }
            }
        }
        return;
    }

    // Row totals in the layout of O: lane (g, n) needs rows 4g + r. FP8 pools summed per lane
    // (row n, a quarter of the keys each): reduce over the lane groups, then fetch row 4g + r.
    float row_total[2][4];
#pragma unroll
    for (int set = 0; set < 2; ++set) {
        if constexpr (KV == LK_BF16) {
#pragma unroll
            for (int r = 0; r < 4; ++r) row_total[set][r] = sums[set][r];
        } else {
            float total = l[set];
            total += __shfl_xor(total, 16, kWave);
            total += __shfl_xor(total, 32, kWave);
#pragma unroll
            for (int r = 0; r < 4; ++r) row_total[set][r] = __shfl(total, int(4 * g + r), kWave);
        }
    }

    if (job_part[job] != 0) {
        // One side of a divided heavy tile. Both sides have the same rows in the same lanes, so
        // thread t's state meets thread t's. A side announces itself by swapping its tag into
        // the pair's word. The first to arrive stores its state with agent-scope stores (past
        // the XCD's own L2, which other XCDs do not see), waits for every store, and then
        // publishes its tag in the pair's ready word. The second finds the first's tag in the
        // pair's word; the first is then resident and has nothing left to wait for, so the
        // second waits for the ready word (with a bound of a few seconds that turns a lost
        // partner into NaN output, not a hang), reads the state with agent-scope loads and merges. The merge
        // takes side 1's state first whichever side runs it, so the output bits do not depend
        // on which side arrived last.
        const uint32_t self = job_part[job] - 1;
        const uint64_t pair_index = uint64_t(kv_head) * half + (a.row_tiles - 1 - tile);  // the pair's light tile
        constexpr uint32_t kSideBytes = kPairStateFloats * 4 * kWave * kLdsWaves;
        const auto side = [&](uint32_t which) __attribute__((always_inline)) {
            return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<uint8_t*>(a.pair_state) + (pair_index * 2 + which) * kSideBytes, short(0),
                                                     int(kSideBytes), 0x00020000);
        };
        const __amdgpu_buffer_rsrc_t own = side(self), other = side(1 - self);
        // Thread t's 16-byte piece c sits at (256 c + t) x 16: pieces 0-15 the accumulators
        // o[set][e] (rows 4g + r), 16-17 the rows' maxima, 18-19 their weight totals.
        constexpr int kAgent = 16;  // cache policy: coherent at agent scope (past the XCD's L2)
        // The thread's byte offset in a vector register (an opaque copy, so that it is formed
        // here and not held through the step loop), the piece's in the scalar offset operand.
        uint32_t thread_at = threadIdx.x * 16;
        asm volatile("" : "+v"(thread_at));
        const auto piece_at = [](uint32_t piece) { return int(piece * kWave * kLdsWaves * 16); };
        f32x4 row_m[2], totals[2];
#pragma unroll
        for (int set = 0; set < 2; ++set)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                row_m[set][r] = __shfl(m[set], int(4 * g + r), kWave);
                totals[set][r] = row_total[set][r];
            }
        if (threadIdx.x == 0) {
            const uint64_t found = __hip_atomic_exchange(a.pair_tags + pair_index, a.pair_tag | self, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            pair_merges = found == (a.pair_tag | (1 - self)) ? 1u : 0u;
        }
        __syncthreads();
        if (!pair_merges) {
#pragma unroll
            for (int set = 0; set < 2; ++set) {
#pragma unroll
                for (int e = 0; e < 8; ++e) __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, o[set][e]), own, thread_at, piece_at(set * 8 + e), kAgent);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, row_m[set]), own, thread_at, piece_at(16 + set), kAgent);
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, totals[set]), own, thread_at, piece_at(18 + set), kAgent);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (threadIdx.x == 0) __hip_atomic_store(a.pair_ready + pair_index, a.pair_tag | self, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            continue;  // the partner merges (a later job, if any, starts clean)
        }
        if (threadIdx.x == 0) {
            uint32_t tries = 0;
            while (__hip_atomic_load(a.pair_ready + pair_index, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != (a.pair_tag | (1 - self)) &&
                   ++tries < kPairWaitBound)
                __builtin_amdgcn_s_sleep(2);
            pair_lost = tries < kPairWaitBound ? 0u : 1u;
        }
        __syncthreads();
        const bool lost = pair_lost != 0;
        asm volatile("" ::: "memory");
        // Both words are done with (the partner swapped and published before this side got
        // here); clearing them lets a launch that repeats this tag, such as a replay of a
        // captured graph, start clean.
        if (threadIdx.x == 0) {
            __hip_atomic_store(a.pair_tags + pair_index, kPairCleared, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(a.pair_ready + pair_index, kPairCleared, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
#pragma unroll
        for (int set = 0; set < 2; ++set) {
            const f32x4 m_in = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(other, thread_at, piece_at(16 + set), kAgent));
            const f32x4 total_in = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(other, thread_at, piece_at(18 + set), kAgent));
            f32x4 o_in[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o_in[e] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(other, thread_at, piece_at(set * 8 + e), kAgent));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float m0 = self == 0 ? row_m[set][r] : m_in[r], m1 = self == 0 ? m_in[r] : row_m[set][r];
                const float t0 = self == 0 ? totals[set][r] : total_in[r], t1 = self == 0 ? total_in[r] : totals[set][r];
                const float top = fmaxf(m0, m1);
                const float w0 = exp2_fast(m0 - top), w1 = exp2_fast(m1 - top);  // kNoMax sides: 0
                row_total[set][r] = fmaf(t0, w0, t1 * w1);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float o0 = self == 0 ? o[set][e][r] : o_in[e][r], o1 = self == 0 ? o_in[e][r] : o[set][e][r];
                    o[set][e][r] = fmaf(o0, w0, o1 * w1);
                }
                if (lost) row_total[set][r] = __builtin_nanf("");
            }
        }
    }

    float inverse[2][4];
#pragma unroll
    for (int set = 0; set < 2; ++set)
#pragma unroll
        for (int r = 0; r < 4; ++r) inverse[set][r] = 1.0f / row_total[set][r];

    // O through LDS (the loop's last barrier has released the buffers): row 16 set + 4g + r,
    // dim 16e + n of this wave's 32 rows, then whole rows out in 16-byte pieces.
    uint8_t* staging = &lds[0][0] + wave * kLdsRows * kLdsRowBytes;
#pragma unroll
    for (int set = 0; set < 2; ++set)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int e = 0; e < 8; ++e)
                *reinterpret_cast<uint16_t*>(staging + (16 * set + 4 * g + r) * kLdsRowBytes + (16 * e + n) * 2) =
                    to_bf16(o[set][e][r] * inverse[set][r]);
    __syncthreads();
#pragma unroll
    for (int x = 0; x < 8; ++x) {
        const uint32_t piece_index = lane + kWave * x;  // 16 pieces of 8 dims per row
        const uint32_t local_row = piece_index / 16;
        const uint32_t out_row = row0 + local_row;
        if (out_row < total_rows) {
            const uint32_t out_token = out_row / a.groups;
            const uint32_t out_head = kv_head * a.groups + out_row % a.groups;
            *reinterpret_cast<u32x4*>(a.out + (uint64_t(out_head) * a.tokens + out_token) * kDim + 8 * (piece_index % 16)) =
                *reinterpret_cast<const u32x4*>(staging + local_row * kLdsRowBytes + 16 * (piece_index % 16));
        }
    }
    if (job + 1 < jobs) __syncthreads();  // the staging rows are the next job's step buffers
    }
}


// Split-K merge: one wave per (KV head, row), 4 rows a workgroup; lane s holds split s's
// (m, l) (at most 64 splits), lanes across dims sum the splits' accumulators in split order.
constexpr uint32_t kMaxKeySplits = 64;

__global__ __launch_bounds__(kWave * 4) void prefill_merge(PrefillArgs a) {
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t total_rows = a.tokens * a.groups;
    const uint64_t unit = uint64_t(blockIdx.x) * 4 + threadIdx.x / kWave;  // kv_head * rows + row
    if (unit >= uint64_t(a.kv_heads) * total_rows) return;
    const uint32_t kv_head = uint32_t(unit / total_rows), row = uint32_t(unit % total_rows);
    const uint64_t base = unit * a.key_splits;
    // The first kEarly splits' accumulators are loaded before (m, l) is combined, so that both
    // loads are one round trip.
    constexpr uint32_t kEarly = 8;
    float early[kEarly][2];
#pragma unroll
    for (uint32_t s = 0; s < kEarly; ++s)
#pragma unroll
        for (int i = 0; i < 2; ++i) early[s][i] = s < a.key_splits ? a.partial_acc[(base + s) * kDim + lane + kWave * i] : 0.0f;
    const float lane_m = lane < a.key_splits ? a.partial_ml[2 * (base + lane)] : kNoMax;
    const float lane_l = lane < a.key_splits ? a.partial_ml[2 * (base + lane) + 1] : 0.0f;
    float top = lane_m;
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) top = fmaxf(top, __shfl_xor(top, mask, kWave));
    const float weight = exp2_fast(lane_m - top);  // kNoMax splits: exp2(-1e30) = 0
    float total = lane_l * weight;
#pragma unroll
    for (int mask = 32; mask >= 1; mask >>= 1) total += __shfl_xor(total, mask, kWave);
    const float inverse = 1.0f / total;
    float sum[2] = {0.0f, 0.0f};
#pragma unroll
    for (uint32_t s = 0; s < kEarly; ++s) {
        const float w = __shfl(weight, int(s), kWave);
#pragma unroll
        for (int i = 0; i < 2; ++i) sum[i] = s < a.key_splits ? fmaf(w, early[s][i], sum[i]) : sum[i];
    }
    for (uint32_t s = kEarly; s < a.key_splits; ++s) {
        const float w = __shfl(weight, int(s), kWave);
        const float* acc = a.partial_acc + (base + s) * kDim;
#pragma unroll
        for (int i = 0; i < 2; ++i) sum[i] = fmaf(w, acc[lane + kWave * i], sum[i]);
    }
    const uint32_t token = row / a.groups, head = kv_head * a.groups + row % a.groups;
    uint16_t* out = a.out + (uint64_t(head) * a.tokens + token) * kDim;
#pragma unroll
    for (int i = 0; i < 2; ++i) out[lane + kWave * i] = to_bf16(sum[i] * inverse);
}

}  // namespace lk

#endif  // LAYOVER_AMD_PREFILL_ATTENTION_H
