// The C ABI's paged prefill (lk_paged_prefill, lk_paged_prefill_workspace,
// lk_paged_prefill_split): the launch plan (split keys, paired key halves, FP8 staging), the
// workspace layout and the launches of prefill_attention.h's kernels. A translation unit of its
// own so that its kernels build with their own scheduling options (see the Makefile).
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <string>

#include "fp8_codec.h"
#include "host_common.h"
#include "layover_kernels.h"
#include "prefill_attention.h"

#define LK_EXPORT extern "C" __attribute__((visibility("default")))

namespace lk {

// Split-K plan for the LDS prefill kernel. Workgroups are (KV head, 128-row tile); a chunk
// whose tiles do not give every CU two of them (short chunks against long histories) also
// splits each tile's keys, at least 4 steps (128 keys) per split and at most kMaxKeySplits
// splits, and merges the partials in prefill_merge. LAYOVER_PREFILL_SPLITS=n forces n
// splits (tests), read per launch.
//
// FP8-record pools, given a workspace (lk_paged_prefill_split): the chunk's history is first
// decoded, one layer, into a compact BF16 pool in the workspace (stage_history_2048: each
// record byte read once, 2 bytes written), and the BF16 kernel runs on that. The FP8 form of
// the LDS kernel converts every K/V tile in every workgroup that reads it instead, once per
// 128-row tile. LAYOVER_PREFILL_FP8=direct keeps the direct FP8 kernel (tests), read per
// launch; lk_paged_prefill, which has no workspace, always runs it.
struct PrefillPlan {
    uint64_t row_tiles;
    uint32_t key_splits;
    uint32_t split_steps;
    bool shared;      // the LDS kernel (the register-only one never splits)
    bool stage_fp8;   // FP8 pool decoded into the workspace first
    bool paired;      // the grid is resident at once, two workgroups per CU
    bool pair_halves; // paired, unsplit, and some CU pair's heavy tile divides its steps
    int32_t pair_bias;
};

// Steps moved toward the heavy side of a divided tile (the partner side pays a second
// prologue and epilogue); LAYOVER_PREFILL_PAIR_BIAS overrides it, read per launch. Measured on
// MI355X, 2,048 tokens at position 0 (partner on the heavy remainder first): 0.049-0.051 ms per
// layer at 8, 0.049 at 10, 0.050-0.051 at 12, 0.050-0.052 at 14-16 (two runs each, one box).
constexpr int32_t kPairBias = 10;

// Key steps of a 128-row tile of the LDS kernel, and whether a CU pair divides its heavy
// tile: the same arithmetic as prefill_mfma_lds's job plan.
uint32_t lds_tile_steps(uint64_t start, uint64_t rows, uint32_t groups, uint64_t tile) {
    const uint64_t tile_rows = uint64_t(kLdsRows) * kLdsWaves;
    const uint64_t last_row = ((tile + 1) * tile_rows < rows ? (tile + 1) * tile_rows : rows) - 1;
    return uint32_t(((start + last_row / groups) / kSlots + 2) / 2);
}
bool any_pair_divides(const lk_prefill_shape& s, uint64_t row_tiles, int32_t bias) {
    const uint32_t groups = s.query_heads / s.kv_heads;
    const uint64_t rows = uint64_t(s.tokens) * groups, half = (row_tiles + 1) / 2;
    for (uint64_t light = 0; light + half < row_tiles; ++light) {
        const uint32_t heavy_steps = lds_tile_steps(s.start, rows, groups, row_tiles - 1 - light);
        const int64_t share = (int64_t(heavy_steps) + lds_tile_steps(s.start, rows, groups, light) + bias + 1) / 2;
        const uint32_t cut = uint32_t(share < 1 ? 1 : share);
        if (cut < heavy_steps && uint64_t(heavy_steps - cut) * 8 >= heavy_steps) return true;
    }
    return false;
}

PrefillPlan prefill_plan(const lk_prefill_shape& s) {
    PrefillPlan p{};
    const uint32_t groups = s.query_heads / s.kv_heads;
    const uint64_t rows = uint64_t(s.tokens) * groups;
    // The LDS-shared kernel (128 rows a workgroup) unless LAYOVER_PREFILL_KERNEL=1 asks for the
    // register-only one (64 rows a workgroup, each wave streaming its own tiles).
    // FP8 records that are not 16-byte aligned (2 x layers x kv_heads groups of 2,050 bytes:
    // layers x kv_heads not a multiple of 4) are always staged as BF16 for the LDS kernel,
    // the only path that does not read the records in place.
    const bool unaligned_records = s.kv_format == LK_FP8_RECORD && (uint64_t(2) * s.layers * s.kv_heads * (kDim * kSlots + 2)) % 16 != 0;
    const char* choice = getenv("LAYOVER_PREFILL_KERNEL");
    p.shared = unaligned_records || !(choice && strtoul(choice, nullptr, 10) == 1);
    const uint64_t tile_rows = p.shared ? uint64_t(kLdsRows) * kLdsWaves : uint64_t(kPrefillRows) * kPrefillWaves;
    p.row_tiles = (rows + tile_rows - 1) / tile_rows;
    const uint64_t end = uint64_t(s.start) + s.tokens;
    const uint32_t max_steps = uint32_t((((end + kSlots - 1) / kSlots) + 1) / 2);
    p.key_splits = 1;
    p.split_steps = max_steps;
    if (!p.shared) return p;
    const char* fp8_choice = getenv("LAYOVER_PREFILL_FP8");
    p.stage_fp8 = unaligned_records || (s.kv_format == LK_FP8_RECORD && !(fp8_choice && strcmp(fp8_choice, "direct") == 0));
    uint32_t wanted = 0;
    if (const char* forced = getenv("LAYOVER_PREFILL_SPLITS")) {
        wanted = uint32_t(strtoul(forced, nullptr, 10));
    } else {
        const uint64_t workgroups = p.row_tiles * s.kv_heads, target = 2ull * compute_units();
        if (workgroups < target) {
            const uint64_t fill = (target + workgroups - 1) / workgroups, cap = max_steps / 4;
            wanted = uint32_t(fill < cap ? fill : cap);
        }
    }
    const uint32_t most = kMaxKeySplits < max_steps ? kMaxKeySplits : max_steps;
    wanted = wanted < 1 ? 1 : (wanted > most ? most : wanted);
    if (wanted > 1) {
        p.split_steps = (max_steps + wanted - 1) / wanted;
        p.key_splits = (max_steps + p.split_steps - 1) / p.split_steps;
    }
    p.paired = p.row_tiles * s.kv_heads * p.key_splits <= 2ull * compute_units();
    // Paired, unsplit chunks divide their heavy tiles' keys within each CU pair where that pays
    // (LAYOVER_PREFILL_PAIR_HALVES=0 turns it off, read per launch).
    const char* halves = getenv("LAYOVER_PREFILL_PAIR_HALVES");
    const char* bias = getenv("LAYOVER_PREFILL_PAIR_BIAS");
    p.pair_bias = bias ? int32_t(strtol(bias, nullptr, 10)) : kPairBias;
    p.pair_halves = p.paired && p.key_splits == 1 && !(halves && strcmp(halves, "0") == 0) && any_pair_divides(s, p.row_tiles, p.pair_bias);
    return p;
}

// Workspace layout: [staged BF16 history | staged block index | split partials | pair states |
// pair tags and ready words], each part 256-byte aligned; parts the plan does not use are absent.
struct PrefillWorkspace {
    uint64_t stage_bytes, index_bytes, partial_bytes, pair_state_bytes, pair_tag_bytes;
    uint64_t total() const { return stage_bytes + index_bytes + partial_bytes + pair_state_bytes + pair_tag_bytes; }
};

uint64_t round_up_256(uint64_t bytes) { return (bytes + 255) / 256 * 256; }

// Pair tags: even, distinct for every launch of the process, and with a start drawn from the
// clock and an address, so that tags left in a reused workspace by another process do not
// repeat either. A side swaps tag | side into its tile's word.
uint64_t next_pair_tag() {
    static const int anchor = 0;
    static std::atomic<uint64_t> counter{[] {
        uint64_t x = uint64_t(std::chrono::steady_clock::now().time_since_epoch().count()) ^ uint64_t(uintptr_t(&anchor));
        x += 0x9E3779B97F4A7C15ull;  // splitmix64 finalizer
        x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
        x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
        return x ^ (x >> 31);
    }()};
    return counter.fetch_add(1, std::memory_order_relaxed) << 1;
}

uint64_t staged_block_bytes(const lk_prefill_shape& s) { return uint64_t(2) * s.kv_heads * kSlots * kDim * 2; }

PrefillWorkspace prefill_workspace_parts(const lk_prefill_shape& s, const PrefillPlan& p) {
    PrefillWorkspace w{};
    if (p.stage_fp8) {
        const uint64_t blocks = (uint64_t(s.start) + s.tokens + kSlots - 1) / kSlots;
        w.stage_bytes = round_up_256(blocks * staged_block_bytes(s));
        w.index_bytes = round_up_256(blocks * sizeof(int32_t));
    }
    if (p.key_splits > 1) {
        const uint64_t rows = uint64_t(s.tokens) * (s.query_heads / s.kv_heads);
        w.partial_bytes = uint64_t(s.kv_heads) * rows * p.key_splits * (kDim + 2) * sizeof(float);
    }
    if (p.pair_halves) {
        const uint64_t tiles = uint64_t(s.kv_heads) * ((p.row_tiles + 1) / 2);  // CU pairs
        w.pair_state_bytes = round_up_256(tiles * 2 * kPairStateFloats * kWave * kLdsWaves * sizeof(float));
        w.pair_tag_bytes = round_up_256(tiles * 2 * sizeof(uint64_t));  // tags, then ready words
    }
    return w;
}

uint64_t prefill_workspace(const lk_prefill_shape& s, const PrefillPlan& p) { return prefill_workspace_parts(s, p).total(); }

void check_prefill(const lk_prefill_shape& s) {
    require(s.tokens > 0 && s.query_heads > 0 && s.kv_heads > 0 && s.layers > 0, "every prefill dimension must be positive");
    require(s.query_heads % s.kv_heads == 0, "query heads must be a multiple of KV heads");
    require(s.layer < s.layers, "layer out of range");
    require(s.slots == kSlots && s.head_dim == kDim, "paged prefill supports 16-slot blocks of 128 dims");
    require(s.q_format == LK_BF16, "paged prefill takes BF16 q");
    require(s.kv_format == LK_BF16 || s.kv_format == LK_FP8_RECORD, "paged prefill reads BF16 or FP8-record pools");
    require(uint64_t(s.start) + s.tokens <= 0x7FFFFFFFull, "a chunk must end below 2^31 tokens");
}

void run_prefill(const lk_prefill_shape& s, const void* q, const void* pool, const int32_t* block_ids, uint32_t num_block_ids, void* out,
                 void* workspace, uint64_t workspace_bytes, bool may_split, hipStream_t st) {
    require(q && pool && block_ids && out, "null q, pool, block ids or out");
    check_prefill(s);
    const uint64_t end = uint64_t(s.start) + s.tokens;
    require(uint64_t(num_block_ids) * s.slots >= end, "fewer block ids than the chunk's end needs");
    lk_decode_shape d{};
    d.layers = s.layers;
    d.kv_heads = s.kv_heads;
    d.slots = s.slots;
    d.head_dim = s.head_dim;
    d.kv_format = s.kv_format;
    const uint64_t block_bytes = pool_block_bytes(d);
    PrefillPlan p = prefill_plan(s);
    if (!may_split) {
        p.key_splits = 1;
        p.split_steps = uint32_t((((end + kSlots - 1) / kSlots) + 1) / 2);
        p.stage_fp8 = false;
        p.paired = p.row_tiles * s.kv_heads <= 2ull * compute_units();
        p.pair_halves = false;
    }
    // Staged records are read 2 bytes at a time and need only be even; everything read in
    // place, and q and out, must be 16-byte aligned.
    require(aligned(q, 16) && aligned(out, 16), "q and out must be 16-byte aligned");
    require(p.stage_fp8 ? aligned(pool, 2) : aligned(pool, 16) && block_bytes % 16 == 0,
            p.stage_fp8 ? "FP8 records must be 2-byte aligned" : "pool blocks must be 16-byte aligned");
    const PrefillWorkspace parts = prefill_workspace_parts(s, p);
    const uint64_t need = parts.total();
    require(need == 0 || (workspace != nullptr && workspace_bytes >= need && aligned(workspace, 16)),
            "workspace smaller than lk_paged_prefill_workspace");
    const uint32_t groups = s.query_heads / s.kv_heads;
    const uint64_t rows = uint64_t(s.tokens) * groups;
    const uint64_t grid = p.row_tiles * s.kv_heads * p.key_splits;
    require(rows <= 0xFFFFFFFFull && grid <= 0x7FFFFFFFull, "prefill chunk too large for one launch");
    PrefillArgs a{};
    a.q = static_cast<const uint16_t*>(q);
    a.pool = static_cast<const uint8_t*>(pool);
    a.block_ids = block_ids;
    a.out = static_cast<uint16_t*>(out);
    a.tokens = s.tokens;
    a.start = s.start;
    a.query_heads = s.query_heads;
    a.kv_heads = s.kv_heads;
    a.groups = groups;
    a.layers = s.layers;
    a.layer = s.layer;
    a.row_tiles = uint32_t(p.row_tiles);
    a.block_bytes = block_bytes;
    a.scale_log2 = s.scale * kLog2e;
    a.key_splits = p.key_splits;
    a.split_steps = p.split_steps;
    a.paired = p.paired ? 1u : 0u;
    uint8_t* const space = static_cast<uint8_t*>(workspace);
    a.partial_acc = p.key_splits > 1 ? reinterpret_cast<float*>(space + parts.stage_bytes + parts.index_bytes) : nullptr;
    a.partial_ml = p.key_splits > 1 ? a.partial_acc + uint64_t(s.kv_heads) * rows * p.key_splits * kDim : nullptr;
    if (p.pair_halves) {
        uint8_t* const pair_space = space + parts.stage_bytes + parts.index_bytes + parts.partial_bytes;
        a.pair_halves = 1;
        a.pair_state = reinterpret_cast<uint32_t*>(pair_space);
        a.pair_tags = reinterpret_cast<uint64_t*>(pair_space + parts.pair_state_bytes);
        a.pair_ready = a.pair_tags + uint64_t(s.kv_heads) * ((p.row_tiles + 1) / 2);
        a.pair_tag = next_pair_tag();
        a.pair_bias = p.pair_bias;
    }
    if (p.stage_fp8) {
        // The history's blocks, this layer only, as a one-layer BF16 pool; the BF16 kernel then
        // reads block b of it through index[b] = b.
        const uint32_t blocks = uint32_t((end + kSlots - 1) / kSlots);
        uint16_t* stage = reinterpret_cast<uint16_t*>(space);
        int32_t* index = reinterpret_cast<int32_t*>(space + parts.stage_bytes);
        const uint32_t groups_per_block = 2 * s.layers * s.kv_heads;
        launch_stage_history_2048(static_cast<const uint8_t*>(pool), block_ids, block_bytes, groups_per_block, s.layer, s.layers, s.kv_heads,
                                  blocks, stage, index, st);
        a.pool = space;
        a.block_ids = index;
        a.layers = 1;
        a.layer = 0;
        a.block_bytes = staged_block_bytes(s);
        hipLaunchKernelGGL(prefill_mfma_lds<LK_BF16>, dim3(uint32_t(grid)), dim3(kWave * kLdsWaves), 0, st, a);
    } else if (p.shared && s.kv_format == LK_BF16)
        hipLaunchKernelGGL(prefill_mfma_lds<LK_BF16>, dim3(uint32_t(grid)), dim3(kWave * kLdsWaves), 0, st, a);
    else if (p.shared)
        hipLaunchKernelGGL(prefill_mfma_lds<LK_FP8_RECORD>, dim3(uint32_t(grid)), dim3(kWave * kLdsWaves), 0, st, a);
    else if (s.kv_format == LK_BF16)
        hipLaunchKernelGGL(prefill_mfma<LK_BF16>, dim3(uint32_t(grid)), dim3(kWave * kPrefillWaves), 0, st, a);
    else
        hipLaunchKernelGGL(prefill_mfma<LK_FP8_RECORD>, dim3(uint32_t(grid)), dim3(kWave * kPrefillWaves), 0, st, a);
    if (p.key_splits > 1) {
        const uint64_t units = uint64_t(s.kv_heads) * rows;
        hipLaunchKernelGGL(prefill_merge, dim3(uint32_t((units + 3) / 4)), dim3(kWave * 4), 0, st, a);
    }
}

}  // namespace lk

LK_EXPORT int lk_paged_prefill(const lk_prefill_shape* shape, const void* q, const void* pool, const int32_t* block_ids,
                               uint32_t num_block_ids, void* out, void* stream) {
    return lk::guarded([&] {
        lk::require(shape != nullptr, "null shape");
        lk::run_prefill(*shape, q, pool, block_ids, num_block_ids, out, nullptr, 0, false, static_cast<hipStream_t>(stream));
    });
}

LK_EXPORT uint64_t lk_paged_prefill_workspace(const lk_prefill_shape* shape) {
    // No launch here, so no HIP error check either (without a device every HIP call reports
    // one; the plan then assumes 256 CUs).
    if (shape == nullptr) return 0;
    try {
        lk::check_prefill(*shape);
        return lk::prefill_workspace(*shape, lk::prefill_plan(*shape));
    } catch (const std::exception& error) {
        lk::last_error = error.what();
        return 0;
    }
}

LK_EXPORT int lk_paged_prefill_split(const lk_prefill_shape* shape, const void* q, const void* pool, const int32_t* block_ids,
                                     uint32_t num_block_ids, void* out, void* workspace, uint64_t workspace_bytes, void* stream) {
    return lk::guarded([&] {
        lk::require(shape != nullptr, "null shape");
        lk::run_prefill(*shape, q, pool, block_ids, num_block_ids, out, workspace, workspace_bytes, true, static_cast<hipStream_t>(stream));
    });
}
