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
// error about 2^-9 per weight, against the north-star tolerance of 1e-2. Keys past a row's
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
};

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
// BF16 pools: K/V shared through LDS. A workgroup of 4 waves owns 128 rows (32 per wave, as
// two sets of 16) and walks the keys in steps of 32 (two blocks). Each step's K and V tiles
// (4 x 4 KiB) are loaded once per workgroup, every thread bringing 64 contiguous bytes, into
// one of two LDS buffers while the other is read; the next step's bytes are already in
// registers, loaded one step ahead. Per wave and step:
//   QK   for each block and set, four v_mfma_f32_16x16x32_bf16 on K read from LDS (lane
//        (g, n): key n, dims 32g + 8j .. +8), reused by both sets;
//   P    8 scores per lane (keys 4g..4g+3 of each block) of row n;
//   PV   v_mfma_f32_16x16x32_bf16 over the step's 32 keys: the MFMA's k index 8g + i stands
//        for key 4g + i of block 0 (i < 4) or of block 1 (i >= 4), in both P (the lane's
//        own 8 weights, as BF16) and V (read from LDS as 16-byte rows of 8 dims, regrouped by
//        v_perm per output dim), reused by both sets.
// LDS rows are padded to 272 bytes so the 16 lanes reading one column of 16 rows hit
// distinct banks. Registers are held to 256 per lane (amdgpu_waves_per_eu(2)), so two
// workgroups share a CU and one computes while the other waits at its step barrier: measured
// on MI355X at a 2,048-token chunk ending a 32,768-token context, 2.97 ms per layer at one
// wave per SIMD (268 registers) and 1.61 ms at two; 1.51 ms with conflict-free LDS stores and
// one FMA per weight's exponent; 1.39 ms with 32-bit causal compares, one mask per score and
// the row maxima exchanged by permlane swaps instead of LDS-routed shuffles.
constexpr uint32_t kLdsWaves = 4;
constexpr uint32_t kLdsRows = 32;                   // rows per wave
constexpr uint32_t kLdsRowBytes = kDim * 2 + 16;    // 272
constexpr uint32_t kLdsTile = kSlots * kLdsRowBytes; // one block's K or V
constexpr uint32_t kLdsStep = 4 * kLdsTile;          // K0, K1, V0, V1

// FP8-record pools: each thread converts its 32 codes to BF16 as it stages them (the exact
// hardware convert), and each block's 2^shift is applied to that block's scores (K) and
// weights (V), one factor per block and step kept beside the tiles in LDS. A block whose shift
// could leave BF16's normal range is decoded exactly with the shift included (the reference's
// decode_bits) and gets factor 1.
struct PrefillStaged {
    u32x4 w[4];  // BF16: 64 bytes; FP8: the first two hold 32 codes
    int32_t shift;
};

template <int KV>
__global__ __launch_bounds__(kWave* kLdsWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void prefill_mfma_lds(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t lds[2][kLdsStep];
    __shared__ int32_t lds_shift[2][4];  // FP8: per buffer, the shift of K0, K1, V0, V1
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const uint32_t g = lane / 16;
    const uint32_t n = lane % 16;
    const uint32_t kv_head = blockIdx.x % a.kv_heads;
    const uint32_t tile = a.row_tiles - 1 - blockIdx.x / a.kv_heads;
    const uint32_t total_rows = a.tokens * a.groups;
    const uint32_t wg_row0 = tile * kLdsWaves * kLdsRows;
    const uint32_t row0 = wg_row0 + wave * kLdsRows;
    const uint32_t end = a.start + a.tokens;

    // Keys the workgroup needs: up to its last row's limit; in steps of two blocks.
    const uint32_t wg_last = min(wg_row0 + kLdsWaves * kLdsRows, total_rows) - 1;
    const uint32_t key_blocks = (a.start + wg_last / a.groups) / kSlots + 1;
    const uint32_t steps = (key_blocks + 1) / 2;
    const uint32_t last_block = (end + kSlots - 1) / kSlots - 1;

    // Per set: row n's token, head and causal limit; Q as the QK B operand.
    int32_t limit[2];
    uint32_t qt[2][16];
#pragma unroll
    for (int set = 0; set < 2; ++set) {
        const uint32_t row = row0 + 16 * set + n;
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

    // Cooperative step loads: wave w brings tile w (K0, K1, V0, V1). Chunk x of lane t is
    // values 512x + 8t .. +8 of the tile (16 bytes of BF16, or 8 FP8 codes that become 16
    // bytes of BF16), so each wave-wide load reads 1 KiB (or 512 bytes) contiguous, and each
    // LDS store fills whole 256-byte rows, 16 lanes a row: every bank once per 8 lanes.
    constexpr uint32_t kElem = KV == LK_FP8_RECORD ? 1 : 2;
    const uint32_t part = threadIdx.x / kWave;          // which tile
    const uint32_t piece = threadIdx.x % kWave;         // which 8 values of each 512
    const uint64_t tile_bytes = uint64_t(kSlots) * kDim * kElem;
    const uint64_t head_tile = uint64_t(a.layer) * a.kv_heads + kv_head;
    const uint64_t group = part < 2 ? head_tile : uint64_t(a.layers) * a.kv_heads + head_tile;
    const uint64_t part_offset = group * tile_bytes + uint64_t(piece) * 8 * kElem;
    const uint64_t block_elems = uint64_t(2) * a.layers * a.kv_heads * kSlots * kDim;
    // Value 512x + 8t sits in slot 4x + t / 16, dims 8 (t % 16) .. +8.
    const uint32_t lds_offset = part * kLdsTile + (piece / 16) * kLdsRowBytes + (piece % 16) * 16;
    auto load_step = [&](uint32_t step, PrefillStaged& r) {
        const uint32_t block_index = min(2 * step + (part & 1), last_block);
        const int32_t block = a.block_ids[block_index];
        const uint8_t* base = a.pool + uint64_t(uint32_t(block)) * a.block_bytes + part_offset;
        if constexpr (KV == LK_BF16) {
#pragma unroll
            for (int x = 0; x < 4; ++x) r.w[x] = *reinterpret_cast<const u32x4*>(base + 1024 * x);
        } else {
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const u32x2 codes = *reinterpret_cast<const u32x2*>(base + 512 * x);
                r.w[x / 2][2 * (x % 2)] = codes[0];
                r.w[x / 2][2 * (x % 2) + 1] = codes[1];
            }
            r.shift = reinterpret_cast<const int16_t*>(a.pool + uint64_t(uint32_t(block)) * a.block_bytes + block_elems)[group];
        }
    };
    auto store_step = [&](uint32_t buffer, const PrefillStaged& r) {
        uint8_t* dst = lds[buffer] + lds_offset;
        if constexpr (KV == LK_BF16) {
#pragma unroll
            for (int x = 0; x < 4; ++x) *reinterpret_cast<u32x4*>(dst + 4 * kLdsRowBytes * x) = r.w[x];
        } else {
            const bool exact = !shift_is_exact_in_fp32(r.shift);
#pragma unroll
            for (int x = 0; x < 4; ++x) {
                const uint32_t lo = r.w[x / 2][2 * (x % 2)], hi = r.w[x / 2][2 * (x % 2) + 1];
                *reinterpret_cast<u32x4*>(dst + 4 * kLdsRowBytes * x) =
                    u32x4{fp8_pair(lo, false, exact, r.shift), fp8_pair(lo, true, exact, r.shift), fp8_pair(hi, false, exact, r.shift),
                          fp8_pair(hi, true, exact, r.shift)};
            }
            if (piece == 0) lds_shift[buffer][part] = r.shift;
        }
    };

    float m[2] = {-INFINITY, -INFINITY}, l[2] = {0.0f, 0.0f};
    f32x4 o[2][8];
#pragma unroll
    for (int set = 0; set < 2; ++set)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[set][e] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    PrefillStaged staged;
    load_step(0, staged);
    store_step(0, staged);
    if (steps > 1) load_step(1, staged);
    __syncthreads();

    for (uint32_t step = 0; step < steps; ++step) {
        const uint8_t* buf = lds[step & 1];
        const uint32_t key0 = step * 2 * kSlots;
        float k_factor[2] = {a.scale_log2, a.scale_log2}, v_factor[2] = {1.0f, 1.0f};
        if constexpr (KV == LK_FP8_RECORD) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                const int32_t ks = lds_shift[step & 1][b], vs = lds_shift[step & 1][2 + b];
                if (shift_is_exact_in_fp32(ks)) k_factor[b] *= pow2(ks);
                if (shift_is_exact_in_fp32(vs)) v_factor[b] = pow2(vs);
            }
        }

        // Scores S^T = K Q^T for both blocks and both sets.
        f32x4 s[2][2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const uint8_t* k_row = buf + b * kLdsTile + n * kLdsRowBytes + 64 * g;
            bf16x8 kk[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) kk[j] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(k_row + 16 * j));
#pragma unroll
            for (int set = 0; set < 2; ++set) {
                f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        kk[j], as_bf16x8(qt[set][4 * j], qt[set][4 * j + 1], qt[set][4 * j + 2], qt[set][4 * j + 3]), acc, 0, 0, 0);
                s[set][b] = acc;
            }
        }

        // V of the step as B operands: for output dim 8n + e, the values of keys
        // (4g + r of block 0, then of block 1), as four BF16 pairs.
        u32x4 rows[2][4];
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                rows[b][r] = *reinterpret_cast<const u32x4*>(buf + (2 + b) * kLdsTile + (4 * g + r) * kLdsRowBytes + 16 * n);
        // Keys at or past the chunk's end hold anything: zero their V (0 * NaN is NaN).
        if (key0 + 2 * kSlots > end) {
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (key0 + b * kSlots + 4 * g + r >= end) rows[b][r] = u32x4{0u, 0u, 0u, 0u};
        }

        // Softmax and PV for one row set. Row maxima are taken on the raw scores of each block
        // and then scaled (the factors are positive), and each weight's exponent is one FMA.
        // (A separate unmasked path for steps below every limit made the register allocator
        // spill.) The V operand for output dim 8n + e is keys 4g..4g+3 of block 0 then of
        // block 1, as four BF16 pairs.
        auto attend = [&](int set) {
            // Keys past the row's limit become -inf once, for the maximum and the weight alike
            // (exp2(-inf) = 0: every live row sees key 0 in the first step, so m is finite).
            float raw[2][4];
            float top_b[2];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
                float t = -INFINITY;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    raw[b][r] = int32_t(key0 + b * kSlots + 4 * g + r) <= limit[set] ? s[set][b][r] : -INFINITY;
                    t = fmaxf(t, raw[b][r]);
                }
                top_b[b] = t * k_factor[b];
            }
            const float top = max_over_lane_groups(fmaxf(top_b[0], top_b[1]));
            if (__builtin_expect(__any(top > m[set] + kRescaleThreshold), 0)) {
                asm volatile("" ::: "memory");
                const float next = top > m[set] + kRescaleThreshold ? top : m[set];
                const float alpha = merge_weight(m[set], next);
                m[set] = next;
                l[set] *= alpha;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float factor = __shfl(alpha, int(4 * g + r), kWave);
#pragma unroll
                    for (int e = 0; e < 8; ++e) o[set][e][r] *= factor;
                }
            }
            float p[8];
#pragma unroll
            for (int b = 0; b < 2; ++b)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float w = exp2_fast(fmaf(raw[b][r], k_factor[b], -m[set]));
                    l[set] += w;
                    p[4 * b + r] = w * v_factor[b];
                }
            const bf16x8 pb = as_bf16x8(pack_bf16(p[0], p[1]), pack_bf16(p[2], p[3]), pack_bf16(p[4], p[5]), pack_bf16(p[6], p[7]));
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const uint32_t select = (e & 1) ? 0x07060302u : 0x05040100u;
                const uint32_t w = e / 2;
                const bf16x8 vb = as_bf16x8(__builtin_amdgcn_perm(rows[0][1][w], rows[0][0][w], select),
                                            __builtin_amdgcn_perm(rows[0][3][w], rows[0][2][w], select),
                                            __builtin_amdgcn_perm(rows[1][1][w], rows[1][0][w], select),
                                            __builtin_amdgcn_perm(rows[1][3][w], rows[1][2][w], select));
                o[set][e] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pb, vb, o[set][e], 0, 0, 0);
            }
        };
        // A step wholly at or below the first live row's limit, and inside the chunk, needs no
        // mask for any row of this wave (later rows only see more keys).
        attend(0);
        attend(1);

        // The next step's tiles into the other buffer; then the one after into registers.
        if (step + 1 < steps) {
            store_step((step + 1) & 1, staged);
            if (step + 2 < steps) load_step(step + 2, staged);
        }
        __syncthreads();
    }

#pragma unroll
    for (int set = 0; set < 2; ++set) {
        float total = l[set];
        total += __shfl_xor(total, 16, kWave);
        total += __shfl_xor(total, 32, kWave);
        const float inverse = 1.0f / total;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float factor = __shfl(inverse, int(4 * g + r), kWave);
            const uint32_t out_row = row0 + 16 * set + 4 * g + r;
            if (out_row < total_rows) {
                const uint32_t out_token = out_row / a.groups;
                const uint32_t out_head = kv_head * a.groups + out_row % a.groups;
                u32x4 packed;
#pragma unroll
                for (int x = 0; x < 4; ++x)
                    packed[x] = uint32_t(to_bf16(o[set][2 * x][r] * factor)) | (uint32_t(to_bf16(o[set][2 * x + 1][r] * factor)) << 16);
                *reinterpret_cast<u32x4*>(a.out + (uint64_t(out_head) * a.tokens + out_token) * kDim + 8 * n) = packed;
            }
        }
    }
}

}  // namespace lk

#endif  // LAYOVER_AMD_PREFILL_ATTENTION_H
