// The C ABI of include/layover_kernels.h: host-side argument checks, launch geometry and
// template dispatch for the FP8 record kernels (fp8_codec.h) and paged decode attention
// (decode_attention.h). Every entry point only enqueues; nothing here reads device memory.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <chrono>
#include <mutex>
#include <stdexcept>
#include <string>

#include "block_copy.h"
#include "decode_attention.h"
#include "fp8_codec.h"
#include "layover_kernels.h"
#include "host_common.h"

namespace lk {

thread_local std::string last_error;

inline uint32_t grid_for_groups(uint64_t groups) {
    const uint64_t workgroups = (groups + kCodecWaves - 1) / kCodecWaves;
    require(workgroups <= 0x7FFFFFFFull, "too many groups for one launch");
    return uint32_t(workgroups);
}

// Grid of the Qwen-shaped codec kernels. By default one wave per group. LAYOVER_CODEC_WG_PER_CU
// caps the grid at that many workgroups per CU instead, each wave then looping over a
// contiguous run of groups with the next group's loads in flight. Measured on MI355X at the
// bench's 113-block launches: alone, 63 us per launch uncapped against 66 us at 2-8 per CU;
// a 2,048-block swap-out during batch-32 decode takes about 79 ms either way.
uint32_t codec_grid(uint64_t groups) {
    static const uint32_t per_cu = [] {
        const char* text = getenv("LAYOVER_CODEC_WG_PER_CU");
        return text ? uint32_t(strtoul(text, nullptr, 10)) : 0u;
    }();
    const uint64_t workgroups = (groups + kRecordWaves - 1) / kRecordWaves;
    require(workgroups <= 0x7FFFFFFFull, "too many groups for one launch");
    const uint32_t full = uint32_t(workgroups);
    if (per_cu == 0) return full;
    static int units[64] = {};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) return full;
    if (units[device] == 0) {
        int count = 0;
        if (hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || count <= 0) return full;
        units[device] = count;
    }
    const uint64_t resident = uint64_t(units[device]) * per_cu;
    return full < resident ? full : uint32_t(resident);
}

void check_records(const void* pool, const int32_t* ids, uint32_t count, const void* stage, uint64_t group_elems,
                   uint32_t groups_per_block) {
    require(count == 0 || (pool != nullptr && stage != nullptr && ids != nullptr), "null pool, ids or stage");
    require(group_elems > 0 && groups_per_block > 0, "group_elems and groups_per_block must be positive");
    require(aligned(pool, 2), "the BF16 pool must be 2-byte aligned");
}

bool fast_records(const void* pool, const void* stage, uint64_t group_elems, uint32_t groups_per_block) {
    const uint64_t record = group_elems * groups_per_block + 2ull * groups_per_block;
    return group_elems == kFastGroup && aligned(pool, 16) && aligned(stage, 16) && record % 16 == 0;
}

// Decode launch geometry: blocks per split (bps) and splits per sequence, from the shape only.
// About 16 workgroups per CU if every row used the whole table width (so about 8 at the
// typical half-full width of mixed lengths), with splits of 64 to 256 blocks: shorter splits
// spend more on each workgroup's q load and state merge and on the combine pass than they
// gain in balance (measured on MI355X: batch 1 at 32k tokens, 16-block splits 92 us per
// layer, 64-block splits 38 us).
struct Geometry {
    uint32_t bps;
    uint32_t splits;
    bool fast;
};

uint32_t env_order() {
    static const uint32_t value = [] {
        const char* text = getenv("LAYOVER_DECODE_ORDER");
        return text && strtoul(text, nullptr, 10) == 0 ? 0u : 1u;
    }();
    return value;
}

// Read at every launch (a getenv is far cheaper than a launch), so tests can compare both forms.
uint32_t env_combine() { return getenv("LAYOVER_DECODE_COMBINE") != nullptr ? 1u : 0u; }

uint32_t env_waves() {
    static const uint32_t value = [] {
        const char* text = getenv("LAYOVER_DECODE_WAVES");
        return text ? uint32_t(strtoul(text, nullptr, 10)) : 0u;
    }();
    return value;
}

uint32_t env_bps() {
    static const uint32_t value = [] {
        const char* text = getenv("LAYOVER_DECODE_BPS");
        return text ? uint32_t(strtoul(text, nullptr, 10)) : 0u;
    }();
    return value;
}

// CUs of the current device, cached per device; 256 (MI355X) when no device answers, with the
// failed query's error cleared so that it is not reported by a later check.
uint32_t compute_units() {
    static int units[64] = {};
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= 64) {
        (void)hipGetLastError();
        return 256;
    }
    if (units[device] == 0) {
        int count = 0;
        if (hipDeviceGetAttribute(&count, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || count <= 0) {
            (void)hipGetLastError();
            return 256;
        }
        units[device] = count;
    }
    return uint32_t(units[device]);
}

uint64_t pool_block_bytes(const lk_decode_shape& s) {
    const uint64_t elems = 2ull * s.layers * s.kv_heads * s.slots * s.head_dim;
    if (s.kv_format == LK_FP8_RECORD) return elems + 2ull * 2 * s.layers * s.kv_heads;
    return elems * (s.kv_format == LK_F32 ? 4 : 2);
}

// The matrix-core kernel needs the Qwen3 tile shape (16 slots x 128 dims), at most 16 query
// heads per KV head, a BF16 or FP8-record pool, 16-byte aligned tiles (pool base and block
// stride) and blocks below 2 GiB (its loads address a block through a buffer resource of 32-bit
// size); anything else runs the generic kernel.
bool fast_decode(const lk_decode_shape& s, const void* pool) {
    const uint32_t groups = s.query_heads / s.kv_heads;
    return s.slots == kSlots && s.head_dim == kDim && groups <= kMaxHeads && s.kv_format != LK_F32 && aligned(pool, 16) &&
           pool_block_bytes(s) % 16 == 0 && pool_block_bytes(s) <= 0x7FFFFFFFull;
}

uint32_t compute_units();

Geometry geometry(const lk_decode_shape& s, const void* pool = nullptr) {
    Geometry g{};
    g.fast = pool != nullptr && fast_decode(s, pool);
    // Work units counted per KV head for both kernels, so the split count (and with it the
    // workspace size) does not depend on which kernel runs.
    const uint64_t units = uint64_t(s.batch) * s.kv_heads;
    // At most 256 blocks per split: the fast kernel's waves hold their block ids one per lane.
    //
    // Blocks per split, a power of two in [8, 256]. Large batches aim at about 4,096
    // workgroups (at least 64 blocks each); FP8 records, whose tiles are half the bytes, at
    // about 8,192: batch 32 at 1,024-32,768 tokens on distinct blocks 189.7 -> 186 us per layer,
    // on shared blocks 153 -> 151.5 us, with 64 blocks a split instead of 128 (the same change
    // slowed the BF16 decode, 288 -> 291.6 us on shared blocks). A grid that would leave CUs idle instead takes
    // about one workgroup per CU: measured per layer at batch 1, 4,096 tokens 19.9 -> 12.8 us
    // (BF16) with 16 splits instead of 4, and at 16,384 tokens 22.3 -> 20.3 us. An FP8-record
    // table of at most 64 blocks stays one split, which writes the output itself with no merge
    // launch (10.8 against 12.2 us at 1,024 tokens); BF16 tiles, twice the bytes, gain more from
    // spreading (13.3 -> 11.8 us).
    uint32_t bps = env_bps() > 256 ? 256 : env_bps();
    if (bps == 0) {
        const uint64_t work = units * s.table_width;
        const uint64_t target = s.kv_format == LK_FP8_RECORD ? 8192 : 4096;
        const uint64_t large = (work + target - 1) / target;
        const uint64_t fill = (work + compute_units() - 1) / compute_units();
        const uint64_t wanted = s.kv_format == LK_FP8_RECORD && s.table_width <= 64 ? 64 : std::max(large, std::min<uint64_t>(fill, 64));
        bps = 8;
        while (bps < wanted && bps < 256) bps *= 2;
    }
    g.bps = bps;
    g.splits = (s.table_width + bps - 1) / bps;
    return g;
}

void check_shape(const lk_decode_shape& s) {
    require(s.batch > 0 && s.query_heads > 0 && s.kv_heads > 0 && s.head_dim > 0 && s.layers > 0 && s.slots > 0 &&
                s.table_width > 0,
            "every decode dimension must be positive");
    require(s.query_heads % s.kv_heads == 0, "query heads must be a multiple of KV heads");
    require(s.layer < s.layers, "layer out of range");
    require(s.q_format == LK_BF16 || s.q_format == LK_F32, "q must be LK_BF16 or LK_F32");
    require(s.kv_format == LK_BF16 || s.kv_format == LK_F32 || s.kv_format == LK_FP8_RECORD, "unknown KV format");
    require(s.head_dim <= kMaxGenericDim || (s.slots == kSlots && s.head_dim == kDim), "head_dim above 256 is not supported");
    require(s.slots <= 1024, "more than 1024 slots per block is not supported");
    require((s.flags & ~uint32_t(LK_DECODE_SHARED_BLOCKS)) == 0, "unknown decode flags");
}

// Workspace: split partials, acc [batch, query_heads, splits, head_dim] then (m, l) pairs.
uint64_t workspace_bytes(const lk_decode_shape& s) {
    const Geometry g = geometry(s);
    return uint64_t(s.batch) * s.query_heads * g.splits * (uint64_t(s.head_dim) + 2) * sizeof(float);
}

// Waves per workgroup of the matrix-core kernel: 4 when the grid gives the CUs two or more
// workgroups each; otherwise 8 (at most 8 query heads per KV head), so the few workgroups
// still put two waves on each SIMD. (16 waves would leave each 128 registers, and the kernel
// needs more.) LAYOVER_DECODE_WAVES=4|8 forces a count the head group allows.
uint32_t decode_waves(const DecodeArgs& a, uint64_t grid) {
    const uint32_t forced = env_waves();
    if (forced == 4 || (forced == 8 && a.groups <= 8)) return forced;
    if (grid >= 2ull * compute_units()) return 4;
    return a.groups <= 8 ? 8 : 4;
}

template <int KV, int QF, bool kAppend>
void launch_split_mfma_as(const DecodeArgs& a, uint32_t waves, uint32_t grid, hipStream_t stream) {
    const dim3 block(kWave * waves);
    if (a.shared_blocks) {
        if (waves == 8) hipLaunchKernelGGL((decode_split_mfma<KV, QF, 8, false, kAppend>), dim3(grid), block, 0, stream, a);
        else hipLaunchKernelGGL((decode_split_mfma<KV, QF, 4, false, kAppend>), dim3(grid), block, 0, stream, a);
    } else {
        if (waves == 8) hipLaunchKernelGGL((decode_split_mfma<KV, QF, 8, true, kAppend>), dim3(grid), block, 0, stream, a);
        else hipLaunchKernelGGL((decode_split_mfma<KV, QF, 4, true, kAppend>), dim3(grid), block, 0, stream, a);
    }
}

// Kernels with the fused token write (lk_paged_decode_append) are separate instances, so the
// plain decode does not reserve the write's registers.
template <int KV, int QF>
void launch_split_mfma(const DecodeArgs& a, uint32_t grid, hipStream_t stream) {
    const uint32_t waves = decode_waves(a, grid);
    if (a.write_block != nullptr) launch_split_mfma_as<KV, QF, true>(a, waves, grid, stream);
    else launch_split_mfma_as<KV, QF, false>(a, waves, grid, stream);
}

// Above this many splits the merge runs as four workgroups per (sequence, query head), one per
// quarter of the dims (decode_combine_quarter). Measured on MI355X, FP8 records, per layer:
// batch 1 @ 32,768 (32 splits) 18.9 -> 18.15 us, BF16 28.3 -> 27.55 us; batch 8 @ 4,096 (4
// splits) 18.2 -> 18.35 us, so few splits keep one workgroup.
constexpr uint32_t kQuarterSplits = 8;

template <int QF>
void launch_decode(const DecodeArgs& a, const Geometry& g, int kv, void* out, hipStream_t stream) {
    if (g.fast) {
        const uint64_t grid = uint64_t(a.batch) * g.splits * a.kv_heads;
        require(grid <= 0x7FFFFFFFull, "decode grid too large");
        if (kv == LK_BF16) launch_split_mfma<LK_BF16, QF>(a, uint32_t(grid), stream);
        else launch_split_mfma<LK_FP8_RECORD, QF>(a, uint32_t(grid), stream);
    } else {
        const uint64_t grid = uint64_t(a.batch) * a.query_heads * g.splits;
        require(grid <= 0x7FFFFFFFull, "decode grid too large");
        if (kv == LK_BF16) hipLaunchKernelGGL((decode_split_generic<LK_BF16, QF>), dim3(uint32_t(grid)), dim3(kWave), 0, stream, a);
        else if (kv == LK_F32) hipLaunchKernelGGL((decode_split_generic<LK_F32, QF>), dim3(uint32_t(grid)), dim3(kWave), 0, stream, a);
        else hipLaunchKernelGGL((decode_split_generic<LK_FP8_RECORD, QF>), dim3(uint32_t(grid)), dim3(kWave), 0, stream, a);
    }
    if (a.out != nullptr) return;  // the split kernel wrote the output
    const dim3 grid(a.batch * a.query_heads);
    if (!vector_combine_fits(a)) hipLaunchKernelGGL((decode_combine<QF>), grid, dim3(kWave), 0, stream, a, out);
    else if (a.splits > kQuarterSplits) {
        const dim3 quarters(a.batch * a.query_heads * 4);
        if (a.splits <= kWave) hipLaunchKernelGGL((decode_combine_quarter<QF, false>), quarters, dim3(kWave), 0, stream, a, out);
        else hipLaunchKernelGGL((decode_combine_quarter<QF, true>), quarters, dim3(kWave), 0, stream, a, out);
    } else if (a.splits <= kWave) hipLaunchKernelGGL((decode_combine_vector<QF, false>), grid, dim3(kWave), 0, stream, a, out);
    else hipLaunchKernelGGL((decode_combine_vector<QF, true>), grid, dim3(kWave), 0, stream, a, out);
}

// Streaming probes. Each wave moves one chunk, once: kRead 16-byte words per lane from `src`
// (a contiguous kRead KiB) and, when kWrite > 0, kWrite words per lane to `dst`, all
// non-temporal. With no write the loaded words are hashed into `sink` only if they hash to a
// value chosen never to occur. Measured on MI355X over 8 GiB, these one-shot 4 KiB chunks read
// at 7.1 TB/s, against 6.3-6.5 TB/s for a grid-stride loop with four loads per lane in flight.
// `words` bounds the reads (the last chunk may be partial); writes stop at the same chunk.
template <int kRead, int kWrite>
__global__ __launch_bounds__(256) void stream_probe(const u32x4* __restrict__ src, u32x4* __restrict__ dst, uint64_t words,
                                                    uint32_t* __restrict__ sink) {
    const uint64_t chunk = uint64_t(blockIdx.x) * 4 + threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t first = chunk * kRead * kWave;
    if (first >= words) return;
    u32x4 w[kRead];
    const bool whole = first + kRead * kWave <= words;
#pragma unroll
    for (int k = 0; k < kRead; ++k) {
        const uint64_t i = first + k * kWave + lane;
        w[k] = whole || i < words ? __builtin_nontemporal_load(src + i) : u32x4{0, 0, 0, 0};
    }
    if constexpr (kWrite == 0) {
        uint32_t hash = 0;
#pragma unroll
        for (int k = 0; k < kRead; ++k) hash ^= w[k][0] ^ w[k][1] ^ w[k][2] ^ w[k][3];
        if (hash == 0x9E3779B9u) *sink = hash;
    } else {
        // Output chunk `chunk` of kWrite words per lane, built from the loaded words.
        const uint64_t out_first = chunk * kWrite * kWave;
        const uint64_t out_words = kRead == kWrite ? words : (words / kRead) * kWrite;
#pragma unroll
        for (int k = 0; k < kWrite; ++k) {
            const u32x4 value = kRead >= kWrite ? (kRead == kWrite ? w[k] : w[2 * k] ^ w[2 * k + 1]) : w[k / 2];
            const uint64_t i = out_first + k * kWave + lane;
            if (whole || i < out_words) __builtin_nontemporal_store(value, dst + i);
        }
    }
}

// Streaming probes of one wave per workgroup: lane l of workgroup w reads input word
// 64 w + l (16 or 8 bytes) and writes output word 64 w + l (16 or 8 bytes), non-temporally.
// For mixed traffic this shape measured faster on MI355X than whole 4 KiB chunks per wave
// (copy 6.7 against 6.1 TB/s, the 2:1 mix 6.9 against 6.2, the 1:2 mix 6.8 against 5.9).
// kIn / kOut: bytes per word read / written; 16 / 8 XORs the input's halves, 8 / 16 repeats
// the input word.
template <int kIn, int kOut>
__global__ __launch_bounds__(kWave) void wave_stream_probe(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, uint64_t words) {
    const uint64_t word = uint64_t(blockIdx.x) * kWave + threadIdx.x;
    if (word >= words) return;
    if constexpr (kIn == 16) {
        const u32x4 in = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + word);
        if constexpr (kOut == 16) __builtin_nontemporal_store(in, reinterpret_cast<u32x4*>(dst) + word);
        else __builtin_nontemporal_store(u32x2{in[0] ^ in[2], in[1] ^ in[3]}, reinterpret_cast<u32x2*>(dst) + word);
    } else {
        const u32x2 in = __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(src) + word);
        __builtin_nontemporal_store(u32x4{in[0], in[1], in[0], in[1]}, reinterpret_cast<u32x4*>(dst) + word);
    }
}

// Tile probe: reads exactly the K and V tiles a decode launch of this shape reads from a BF16
// pool (16 x 128 tiles, 4 KiB each) or an FP8-record pool (2 KiB tiles and the two groups'
// shifts), in the decode kernel's order (KV head fastest, then the row's blocks, then the
// rows), one wave per (row, block, KV head), and does nothing with them: the read rate of the
// decode's access pattern on this pool, with no compute. Like the decode, each wave first
// loads its row's length and block id.
template <int KV>
__global__ __launch_bounds__(256) void tile_probe(const uint8_t* __restrict__ pool, uint64_t block_bytes, const int32_t* __restrict__ table,
                                                  uint32_t table_stride, const int32_t* __restrict__ lengths, uint32_t lengths_stride,
                                                  uint32_t batch, uint32_t width, uint32_t kv_heads, uint32_t layers, uint32_t layer,
                                                  uint32_t* __restrict__ sink) {
    const uint64_t unit = uint64_t(blockIdx.x) * 4 + threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint32_t kv = uint32_t(unit % kv_heads);
    const uint32_t j = uint32_t((unit / kv_heads) % width);
    const uint64_t seq = unit / (uint64_t(kv_heads) * width);
    if (seq >= batch) return;
    const uint32_t nblocks = blocks_of(lengths[seq * lengths_stride], kSlots);
    if (j >= nblocks) return;
    const uint8_t* base = pool + uint64_t(uint32_t(table[seq * table_stride + j])) * block_bytes;
    constexpr uint64_t kTile = uint64_t(kSlots) * kDim * (KV == LK_FP8_RECORD ? 1 : 2);
    constexpr int kWords = int(kTile / (16 * kWave));  // 16-byte words per lane and tile
    const uint64_t k_group = uint64_t(layer) * kv_heads + kv, v_group = (uint64_t(layers) + layer) * kv_heads + kv;
    const u32x4* k = reinterpret_cast<const u32x4*>(base + k_group * kTile);
    const u32x4* v = reinterpret_cast<const u32x4*>(base + v_group * kTile);
    u32x4 w = {0, 0, 0, 0};
#pragma unroll
#ifdef LK_PROBE_PLAIN
    for (int i = 0; i < kWords; ++i) w ^= k[i * kWave + lane] ^ v[i * kWave + lane];
#else
    for (int i = 0; i < kWords; ++i) w ^= __builtin_nontemporal_load(k + i * kWave + lane) ^ __builtin_nontemporal_load(v + i * kWave + lane);
#endif
    if constexpr (KV == LK_FP8_RECORD) {
        // The two groups' shifts, as the decode loads them (after the record's codes).
        const int16_t* shifts = reinterpret_cast<const int16_t*>(base + 2 * layers * kv_heads * kTile);
        if (lane == 0) w[0] ^= uint32_t(shifts[k_group]) ^ (uint32_t(shifts[v_group]) << 16);
    }
    if ((w[0] ^ w[1] ^ w[2] ^ w[3]) == 0x9E3779B9u) *sink = 1;
}

// One token per sequence written into an FP8-record pool (lk_fp8_append). One wave per
// (row, kind, KV head) group: element e of the group (slot e / head_dim) becomes the old
// value decoded at the old shift for slots before the write slot, the new BF16 value at the
// write slot, and zero after it; the group is then re-encoded at the shift of those values,
// with the reference's integer codec (fp8.py:86-137). Each lane reads and writes only its
// own elements, and the old shift is read before the wave max that precedes its overwrite.
__global__ __launch_bounds__(kWave* kCodecWaves) void append_groups(uint8_t* __restrict__ records, const int32_t* __restrict__ write_block,
                                                                  const int32_t* __restrict__ write_slot, uint32_t row_stride,
                                                                  uint32_t batch, const uint16_t* __restrict__ k,
                                                                  const uint16_t* __restrict__ v, uint32_t layer, uint32_t layers,
                                                                  uint32_t kv_heads, uint32_t slots, uint32_t head_dim) {
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t unit = uint64_t(blockIdx.x) * kCodecWaves + threadIdx.x / kWave;
    if (unit >= uint64_t(batch) * 2 * kv_heads) return;
    const uint32_t head = uint32_t(unit % kv_heads);
    const uint32_t kind = uint32_t(unit / kv_heads % 2);
    const uint32_t row = uint32_t(unit / (2ull * kv_heads));
    const uint64_t group_elems = uint64_t(slots) * head_dim;
    const uint32_t groups_per_block = 2 * layers * kv_heads;
    const uint64_t block_elems = group_elems * groups_per_block;
    const uint64_t record = block_elems + 2ull * groups_per_block;
    const uint32_t g = (kind * layers + layer) * kv_heads + head;
    uint8_t* base = records + uint64_t(uint32_t(write_block[uint64_t(row) * row_stride])) * record;
    uint8_t* codes = base + uint64_t(g) * group_elems;
    uint8_t* shift_at = base + block_elems + 2ull * g;
    const uint32_t slot = uint32_t(write_slot[uint64_t(row) * row_stride]);
    const uint16_t* fresh = (kind == 0 ? k : v) + (uint64_t(row) * kv_heads + head) * head_dim;
    const int32_t old_shift = int16_t(uint16_t(shift_at[0]) | uint16_t(shift_at[1] << 8));

    auto value = [&](uint64_t e) -> uint32_t {
        const uint64_t s = e / head_dim;
        if (s < slot) return decode_e4m3(codes[e], old_shift);
        if (s == slot) return fresh[e - s * head_dim];
        return 0u;
    };
    uint32_t key = 0;
    for (uint64_t e = lane; e < group_elems; e += kWave) {
        const uint32_t k_ = exponent_key(value(e));
        key = k_ > key ? k_ : key;
    }
    const int32_t shift = shift_from_key(wave_max(key));
    for (uint64_t e = lane; e < group_elems; e += kWave) codes[e] = uint8_t(encode_e4m3(value(e), shift));
    if (lane == 0) {
        const uint16_t stored = uint16_t(int16_t(shift));
        shift_at[0] = uint8_t(stored & 0xFFu);
        shift_at[1] = uint8_t(stored >> 8);
    }
}


// One token per sequence written into a BF16 pool (lk_kv_write): the reference's decode-time
// pool assignment (model.py:139-140) as one launch. Thread t of a row copies 16 bytes: K for
// the first kv_heads * head_dim / 8 threads, V for the rest.
__global__ void write_tokens_bf16(uint16_t* __restrict__ pool, const int32_t* __restrict__ write_block,
                                  const int32_t* __restrict__ write_slot, uint32_t row_stride, uint32_t batch,
                                  const uint16_t* __restrict__ k, const uint16_t* __restrict__ v, uint32_t layer, uint32_t layers,
                                  uint32_t kv_heads, uint32_t slots, uint32_t head_dim) {
    const uint32_t per_kind = kv_heads * head_dim / 8;  // 16-byte pieces of one kind
    const uint64_t index = uint64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (index >= uint64_t(batch) * 2 * per_kind) return;
    const uint32_t row = uint32_t(index / (2 * per_kind));
    const uint32_t within = uint32_t(index % (2 * per_kind));
    const uint32_t kind = within / per_kind;
    const uint32_t piece = within % per_kind;
    const uint32_t head = piece * 8 / head_dim;
    const uint32_t dim = piece * 8 % head_dim;
    const uint64_t block = uint32_t(write_block[uint64_t(row) * row_stride]);
    const uint64_t slot = uint32_t(write_slot[uint64_t(row) * row_stride]);
    const uint64_t tile = ((uint64_t(kind) * layers + layer) * kv_heads + head) * slots + slot;
    const uint64_t block_elems = 2ull * layers * kv_heads * slots * head_dim;
    const u32x4 value = *reinterpret_cast<const u32x4*>((kind == 0 ? k : v) + (uint64_t(row) * kv_heads + head) * head_dim + dim);
    *reinterpret_cast<u32x4*>(pool + block * block_elems + tile * head_dim + dim) = value;
}

}  // namespace lk

#define LK_EXPORT extern "C" __attribute__((visibility("default")))

LK_EXPORT int lk_abi_version(void) { return LK_ABI_VERSION; }
LK_EXPORT const char* lk_last_error(void) { return lk::last_error.c_str(); }

LK_EXPORT int lk_fp8_quantize(const void* pool, const int32_t* ids, uint32_t count, void* stage, uint64_t group_elems,
                              uint32_t groups_per_block, void* stream) {
    return lk::guarded([&] {
        lk::check_records(pool, ids, count, stage, group_elems, groups_per_block);
        if (count == 0) return;
        const uint64_t groups = uint64_t(count) * groups_per_block;
        const uint32_t grid = lk::grid_for_groups(groups);
        const dim3 block(lk::kWave * lk::kCodecWaves);
        auto s = static_cast<hipStream_t>(stream);
        if (lk::fast_records(pool, stage, group_elems, groups_per_block))
            lk::launch_quantize_2048(static_cast<const uint16_t*>(pool), ids, static_cast<uint8_t*>(stage), count, groups_per_block,
                                     lk::codec_grid(groups), s);
        else
            hipLaunchKernelGGL(lk::quantize_groups_any, dim3(grid), block, 0, s, static_cast<const uint16_t*>(pool), ids,
                               static_cast<uint8_t*>(stage), count, group_elems, groups_per_block);
    });
}

LK_EXPORT int lk_fp8_dequantize(const void* stage, const int32_t* ids, uint32_t count, void* pool, uint64_t group_elems,
                                uint32_t groups_per_block, void* stream) {
    return lk::guarded([&] {
        lk::check_records(pool, ids, count, stage, group_elems, groups_per_block);
        if (count == 0) return;
        const uint64_t groups = uint64_t(count) * groups_per_block;
        const uint32_t grid = lk::grid_for_groups(groups);
        const dim3 block(lk::kWave * lk::kCodecWaves);
        auto s = static_cast<hipStream_t>(stream);
        if (lk::fast_records(pool, stage, group_elems, groups_per_block))
            lk::launch_dequantize_2048(static_cast<const uint8_t*>(stage), ids, static_cast<uint16_t*>(pool), count, groups_per_block,
                                       lk::codec_grid(groups), s);
        else
            hipLaunchKernelGGL(lk::dequantize_groups_any, dim3(grid), block, 0, s, static_cast<const uint8_t*>(stage), ids,
                               static_cast<uint16_t*>(pool), count, group_elems, groups_per_block);
    });
}

LK_EXPORT int lk_fp8_encode(const uint16_t* bits, uint8_t* out, uint64_t n, int32_t shift, void* stream) {
    return lk::guarded([&] {
        lk::require(bits != nullptr && out != nullptr, "null input or output");
        if (n == 0) return;
        const uint64_t grid = (n + 255) / 256;
        lk::require(grid <= 0x7FFFFFFFull, "too many elements for one launch");
        hipLaunchKernelGGL(lk::encode_elements, dim3(uint32_t(grid)), dim3(256), 0, static_cast<hipStream_t>(stream), bits, out, n, shift);
    });
}

LK_EXPORT int lk_fp8_decode(const uint8_t* codes, uint16_t* out, uint64_t n, int32_t shift, void* stream) {
    return lk::guarded([&] {
        lk::require(codes != nullptr && out != nullptr, "null input or output");
        if (n == 0) return;
        const uint64_t grid = (n + 255) / 256;
        lk::require(grid <= 0x7FFFFFFFull, "too many elements for one launch");
        hipLaunchKernelGGL(lk::decode_elements, dim3(uint32_t(grid)), dim3(256), 0, static_cast<hipStream_t>(stream), codes, out, n, shift);
    });
}

LK_EXPORT int lk_kv_write(void* pool, const int32_t* write_block, const int32_t* write_slot, uint32_t row_stride, uint32_t batch,
                          const void* k, const void* v, uint32_t layer, uint32_t layers, uint32_t kv_heads, uint32_t slots,
                          uint32_t head_dim, void* stream) {
    return lk::guarded([&] {
        lk::require(pool && write_block && write_slot && k && v, "null pool, write rows, k or v");
        lk::require(layers > 0 && kv_heads > 0 && slots > 0 && head_dim > 0, "every pool dimension must be positive");
        lk::require(layer < layers, "layer out of range");
        lk::require(row_stride > 0, "row_stride must be positive");
        lk::require(head_dim % 8 == 0 && lk::aligned(pool, 16) && lk::aligned(k, 16) && lk::aligned(v, 16),
                    "head_dim must be a multiple of 8 and pool, k and v 16-byte aligned");
        if (batch == 0) return;
        const uint64_t threads = uint64_t(batch) * 2 * kv_heads * head_dim / 8;
        const uint64_t grid = (threads + 255) / 256;
        lk::require(grid <= 0x7FFFFFFFull, "too many rows for one launch");
        hipLaunchKernelGGL(lk::write_tokens_bf16, dim3(uint32_t(grid)), dim3(256), 0, static_cast<hipStream_t>(stream),
                           static_cast<uint16_t*>(pool), write_block, write_slot, row_stride, batch, static_cast<const uint16_t*>(k),
                           static_cast<const uint16_t*>(v), layer, layers, kv_heads, slots, head_dim);
    });
}

LK_EXPORT int lk_fp8_append(void* records, const int32_t* write_block, const int32_t* write_slot, uint32_t row_stride,
                            uint32_t batch, const void* k, const void* v, uint32_t layer, uint32_t layers, uint32_t kv_heads,
                            uint32_t slots, uint32_t head_dim, void* stream) {
    return lk::guarded([&] {
        lk::require(records && write_block && write_slot && k && v, "null records, write rows, k or v");
        lk::require(layers > 0 && kv_heads > 0 && slots > 0 && head_dim > 0, "every record dimension must be positive");
        lk::require(layer < layers, "layer out of range");
        lk::require(row_stride > 0, "row_stride must be positive");
        if (batch == 0) return;
        const uint64_t waves = uint64_t(batch) * 2 * kv_heads;
        const uint32_t grid = lk::grid_for_groups(waves);
        const uint64_t record = uint64_t(slots) * head_dim * 2 * layers * kv_heads + 4ull * layers * kv_heads;
        if (slots * head_dim == lk::kFastGroup && head_dim == 128 && record % 16 == 0 && lk::aligned(records, 16) && lk::aligned(k, 16) &&
            lk::aligned(v, 16)) {
            lk::launch_append_2048(static_cast<uint8_t*>(records), write_block, write_slot, row_stride, batch, static_cast<const uint16_t*>(k),
                                   static_cast<const uint16_t*>(v), layer, layers, kv_heads, grid, static_cast<hipStream_t>(stream));
            return;
        }
        hipLaunchKernelGGL(lk::append_groups, dim3(grid), dim3(lk::kWave * lk::kCodecWaves), 0, static_cast<hipStream_t>(stream),
                           static_cast<uint8_t*>(records), write_block, write_slot, row_stride, batch, static_cast<const uint16_t*>(k),
                           static_cast<const uint16_t*>(v), layer, layers, kv_heads, slots, head_dim);
    });
}

LK_EXPORT uint64_t lk_paged_decode_workspace(const lk_decode_shape* shape) {
    if (shape == nullptr) return 0;
    try {
        lk::check_shape(*shape);
    } catch (const std::exception&) {
        return 0;
    }
    return lk::workspace_bytes(*shape);
}

namespace lk {

struct TokenWrite {
    const int32_t* write_block;
    const int32_t* write_slot;
    uint32_t stride;
    const void* k;
    const void* v;
};

void run_decode(const lk_decode_shape& s, const void* q, const void* pool, const int32_t* table, const int32_t* lengths, void* out,
                void* workspace, uint64_t workspace_bytes, const TokenWrite* write, hipStream_t st) {
    check_shape(s);
    require(q && pool && table && lengths && out && workspace, "null q, pool, table, lengths, out or workspace");
    require(workspace_bytes >= ::lk::workspace_bytes(s), "workspace smaller than lk_paged_decode_workspace");
    require(aligned(workspace, 4), "workspace must be 4-byte aligned");
    const Geometry g = geometry(s, pool);
    DecodeArgs a{};
    a.q = q;
    a.pool = static_cast<const uint8_t*>(pool);
    a.table = table;
    a.lengths = lengths;
    a.partial_acc = static_cast<float*>(workspace);
    a.partial_ml = a.partial_acc + uint64_t(s.batch) * s.query_heads * g.splits * s.head_dim;
    a.batch = s.batch;
    a.query_heads = s.query_heads;
    a.kv_heads = s.kv_heads;
    a.head_dim = s.head_dim;
    a.layers = s.layers;
    a.slots = s.slots;
    a.layer = s.layer;
    a.table_width = s.table_width;
    a.table_stride = s.table_stride != 0 ? s.table_stride : s.table_width;
    a.lengths_stride = s.lengths_stride != 0 ? s.lengths_stride : 1;
    require(a.table_stride >= s.table_width, "table_stride is smaller than table_width");
    a.groups = s.query_heads / s.kv_heads;
    a.splits = g.splits;
    a.bps = g.bps;
    a.order = env_order();
    a.shared_blocks = (s.flags & LK_DECODE_SHARED_BLOCKS) != 0;
    a.vector_combine = aligned(workspace, 16) && aligned(out, s.q_format == LK_BF16 ? 8 : 16);
    a.block_bytes = pool_block_bytes(s);
    a.scale_log2 = s.scale * kLog2e;
    // One split per row (tables of at most `bps` blocks) on a grid small enough for 8-wave
    // workgroups: the split kernel writes the output. (The 4-wave kernel has no such branch,
    // which measurably costs the large-batch loop.) LAYOVER_DECODE_COMBINE keeps the combine
    // launch (for comparisons).
    if (g.fast && g.splits == 1 && env_combine() == 0 && decode_waves(a, uint64_t(s.batch) * s.kv_heads) == 8) a.out = out;
    require(aligned(pool, s.kv_format == LK_F32 ? 4 : (s.kv_format == LK_BF16 ? 2 : 1)), "misaligned pool");
    if (write != nullptr) {
        require(write->write_block && write->write_slot && write->k && write->v, "null write rows, k or v");
        require(write->stride > 0, "write_stride must be positive");
        require(s.kv_format == LK_BF16 || s.kv_format == LK_FP8_RECORD, "a fused write needs a BF16 or FP8-record pool");
        require(aligned(write->k, 16) && aligned(write->v, 16), "k and v must be 16-byte aligned");
        if (g.fast) {
            a.write_block = write->write_block;
            a.write_slot = write->write_slot;
            a.write_stride = write->stride;
            a.k_new = static_cast<const uint16_t*>(write->k);
            a.v_new = static_cast<const uint16_t*>(write->v);
        } else {
            // Shapes the matrix-core kernel does not take: the write as its own launch first.
            const int status = s.kv_format == LK_BF16
                                   ? lk_kv_write(const_cast<void*>(pool), write->write_block, write->write_slot, write->stride, s.batch, write->k,
                                                 write->v, s.layer, s.layers, s.kv_heads, s.slots, s.head_dim, st)
                                   : lk_fp8_append(const_cast<void*>(pool), write->write_block, write->write_slot, write->stride, s.batch,
                                                   write->k, write->v, s.layer, s.layers, s.kv_heads, s.slots, s.head_dim, st);
            if (status == LK_ERR_INVALID) throw Invalid(last_error);
            if (status != LK_OK) throw std::runtime_error(last_error);
        }
    }
    if (s.q_format == LK_BF16) launch_decode<LK_BF16>(a, g, s.kv_format, out, st);
    else launch_decode<LK_F32>(a, g, s.kv_format, out, st);
}

}  // namespace lk

LK_EXPORT int lk_paged_decode(const lk_decode_shape* shape, const void* q, const void* pool, const int32_t* table,
                              const int32_t* lengths, void* out, void* workspace, uint64_t workspace_bytes, void* stream) {
    return lk::guarded([&] {
        lk::require(shape != nullptr, "null shape");
        lk::run_decode(*shape, q, pool, table, lengths, out, workspace, workspace_bytes, nullptr, static_cast<hipStream_t>(stream));
    });
}

LK_EXPORT int lk_paged_decode_append(const lk_decode_shape* shape, const void* q, void* pool, const int32_t* table, const int32_t* lengths,
                                     const int32_t* write_block, const int32_t* write_slot, uint32_t write_stride, const void* k,
                                     const void* v, void* out, void* workspace, uint64_t workspace_bytes, void* stream) {
    return lk::guarded([&] {
        lk::require(shape != nullptr, "null shape");
        const lk::TokenWrite write{write_block, write_slot, write_stride, k, v};
        lk::run_decode(*shape, q, pool, table, lengths, out, workspace, workspace_bytes, &write, static_cast<hipStream_t>(stream));
    });
}

// lk_paged_decode_static: lk_paged_decode with its split partials in a file-scope device array
// instead of a caller's workspace, for callers that cannot allocate. The array's address is
// looked up once per device (hipGetSymbolAddress, with that device current) and kept; the
// host-side name `decode_scratch` is only a stand-in and never reaches a kernel. Nothing in it
// needs clearing between calls (the merge reads only the splits a row's length covers, all
// written by the same launch).
//
// Calls on one device share the array, so they are ordered: each call records an event on its
// stream after its launches, and a call on another stream first makes its stream wait for that
// event, so a launch never overwrites partials that another stream's merge has yet to read.
// Under HIP graph capture (either call's stream capturing) events are left alone: a captured
// call's order is the graph's, and replays on different streams must not overlap (the
// caller's rule). The stream must belong to the current device, whose array is used.
namespace lk {

constexpr uint64_t kStaticScratchBytes = 32ull << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) uint8_t decode_scratch[kStaticScratchBytes];

struct StaticScratch {
    void* address = nullptr;
    hipEvent_t done = nullptr;       // recorded after the last uncaptured call's launches
    hipStream_t stream = nullptr;    // that call's stream
    bool recorded = false;
};
std::mutex scratch_lock;  // held from the lookup to the event record, so calls from two threads are ordered too
StaticScratch scratch_state[kMaxDevices];

void run_decode_static(const lk_decode_shape& s, const void* q, const void* pool, const int32_t* table, const int32_t* lengths, void* out,
                       hipStream_t stream) {
    int device = -1;
    require(hipGetDevice(&device) == hipSuccess && device >= 0 && device < kMaxDevices, "no usable current HIP device");
    int stream_device = device;
    if (stream != nullptr) require(hipStreamGetDevice(stream, &stream_device) == hipSuccess, "hipStreamGetDevice failed on the stream");
    if (stream_device != device)
        throw Invalid("the stream belongs to device " + std::to_string(stream_device) + ", the current device is " + std::to_string(device) +
                      ": make the stream's device current");
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    require(hipStreamIsCapturing(stream, &capture) == hipSuccess, "hipStreamIsCapturing failed");
    const bool captured = capture != hipStreamCaptureStatusNone;
    std::lock_guard<std::mutex> hold(scratch_lock);
    StaticScratch& state = scratch_state[device];
    if (state.address == nullptr) {
        void* address = nullptr;
        const hipError_t status = hipGetSymbolAddress(&address, HIP_SYMBOL(decode_scratch));
        if (status != hipSuccess || address == nullptr)
            throw std::runtime_error(std::string("hipGetSymbolAddress(decode_scratch): ") + hipGetErrorString(status));
        state.address = address;
    }
    if (state.done == nullptr) require(hipEventCreateWithFlags(&state.done, hipEventDisableTiming) == hipSuccess, "hipEventCreate failed");
    if (!captured && state.recorded && state.stream != stream)
        require(hipStreamWaitEvent(stream, state.done, 0) == hipSuccess, "hipStreamWaitEvent on the previous static call failed");
    run_decode(s, q, pool, table, lengths, out, state.address, kStaticScratchBytes, nullptr, stream);
    if (!captured) {
        require(hipEventRecord(state.done, stream) == hipSuccess, "hipEventRecord after the static call failed");
        state.stream = stream;
        state.recorded = true;
    }
}

}  // namespace lk

LK_EXPORT int lk_paged_decode_static(const lk_decode_shape* shape, const void* q, const void* pool, const int32_t* table,
                                     const int32_t* lengths, void* out, void* stream) {
    return lk::guarded([&] {
        lk::require(shape != nullptr, "null shape");
        lk::check_shape(*shape);
        const uint64_t need = lk::workspace_bytes(*shape);
        if (need > lk::kStaticScratchBytes)
            throw lk::Invalid("lk_paged_decode_static: this shape needs " + std::to_string(need) + " bytes of split partials, above the " +
                              std::to_string(lk::kStaticScratchBytes) + "-byte static scratch; use lk_paged_decode with a workspace");
        lk::run_decode_static(*shape, q, pool, table, lengths, out, static_cast<hipStream_t>(stream));
    });
}


namespace lk {

// The arguments lt_out_gather / lt_in_scatter accept, checked the same way.
void check_block_copy(const void* pool, const uint32_t* ids, uint32_t count, uint64_t block_bytes, const void* staging) {
    require(count == 0 || (pool != nullptr && staging != nullptr && ids != nullptr), "null pool, ids or staging");
    require(block_bytes > 0 && block_bytes % 8 == 0 && aligned(pool, 8) && aligned(staging, 8),
            "pool and staging must be 8-byte aligned and block_bytes a positive multiple of 8");
    require(blockcopy::launch_fits(block_bytes, count), "too many chunks for one launch (at most 2^32 / 64 chunks of 512 bytes)");
}

}  // namespace lk

LK_EXPORT int lk_gather_blocks(const void* pool, const uint32_t* ids, uint32_t count, uint64_t block_bytes, void* staging, void* stream) {
    return lk::guarded([&] {
        lk::check_block_copy(pool, ids, count, block_bytes, staging);
        if (count == 0) return;
        const hipError_t status = blockcopy::launch_gather(static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(pool), ids,
                                                           static_cast<uint8_t*>(staging), block_bytes, count);
        if (status != hipSuccess) throw std::runtime_error(std::string("gather_blocks launch failed: ") + hipGetErrorString(status));
    });
}

LK_EXPORT int lk_scatter_blocks(void* pool, const uint32_t* ids, uint32_t count, uint64_t block_bytes, const void* staging, void* stream) {
    return lk::guarded([&] {
        lk::check_block_copy(pool, ids, count, block_bytes, staging);
        if (count == 0) return;
        const hipError_t status = blockcopy::launch_scatter(static_cast<hipStream_t>(stream), static_cast<uint8_t*>(pool), ids,
                                                            static_cast<const uint8_t*>(staging), block_bytes, count);
        if (status != hipSuccess) throw std::runtime_error(std::string("scatter_blocks launch failed: ") + hipGetErrorString(status));
    });
}

LK_EXPORT int lk_stream_probe(const void* src, void* dst, uint64_t bytes, uint32_t* sink, void* stream) {
    return lk::guarded([&] {
        lk::require(src != nullptr && sink != nullptr, "null src or sink");
        lk::require(bytes % 16 == 0 && lk::aligned(src, 16) && (dst == nullptr || lk::aligned(dst, 16)), "16-byte granularity required");
        if (bytes == 0) return;
        const uint64_t grid = (bytes + 16 * 1024 - 1) / (16 * 1024);  // four 4 KiB chunks per workgroup
        lk::require(grid <= 0x7FFFFFFFull, "probe too large");
        const auto s = static_cast<hipStream_t>(stream);
        const auto in = static_cast<const lk::u32x4*>(src);
        if (dst == nullptr) {
            hipLaunchKernelGGL((lk::stream_probe<4, 0>), dim3(uint32_t(grid)), dim3(256), 0, s, in, nullptr, bytes / 16, sink);
        } else {
            const uint64_t words = bytes / 16, waves = (words + lk::kWave - 1) / lk::kWave;
            lk::require(waves <= 0x7FFFFFFFull, "probe too large");
            hipLaunchKernelGGL((lk::wave_stream_probe<16, 16>), dim3(uint32_t(waves)), dim3(lk::kWave), 0, s, static_cast<const uint8_t*>(src),
                               static_cast<uint8_t*>(dst), words);
        }
    });
}

LK_EXPORT int lk_tile_probe(const lk_decode_shape* shape, const void* pool, const int32_t* table, const int32_t* lengths, void* sink,
                            void* stream) {
    return lk::guarded([&] {
        lk::require(shape != nullptr && pool != nullptr && table != nullptr && lengths != nullptr && sink != nullptr,
                    "null shape, pool, table, lengths or sink");
        const lk_decode_shape& s = *shape;
        lk::check_shape(s);
        lk::require((s.kv_format == LK_BF16 || s.kv_format == LK_FP8_RECORD) && s.slots == lk::kSlots && s.head_dim == lk::kDim,
                    "the tile probe reads BF16 or FP8-record 16 x 128 tiles");
        const uint32_t table_stride = s.table_stride != 0 ? s.table_stride : s.table_width;
        const uint32_t lengths_stride = s.lengths_stride != 0 ? s.lengths_stride : 1;
        const uint64_t waves = uint64_t(s.batch) * s.table_width * s.kv_heads;
        const uint64_t grid = (waves + 3) / 4;
        lk::require(grid <= 0x7FFFFFFFull, "too many tiles for one launch");
        const auto kernel = s.kv_format == LK_BF16 ? lk::tile_probe<LK_BF16> : lk::tile_probe<LK_FP8_RECORD>;
        hipLaunchKernelGGL(kernel, dim3(uint32_t(grid)), dim3(256), 0, static_cast<hipStream_t>(stream), static_cast<const uint8_t*>(pool),
                           lk::pool_block_bytes(s), table, table_stride, lengths, lengths_stride, s.batch, s.table_width, s.kv_heads, s.layers,
                           s.layer, static_cast<uint32_t*>(sink));
        lk::require(hipGetLastError() == hipSuccess, "tile_probe launch failed");
    });
}

LK_EXPORT int lk_stream_probe_mix(const void* src, uint64_t src_bytes, void* dst, uint64_t dst_bytes, void* stream) {
    return lk::guarded([&] {
        lk::require(src != nullptr && dst != nullptr, "null src or dst");
        lk::require(lk::aligned(src, 16) && lk::aligned(dst, 16), "16-byte alignment required");
        const bool two_to_one = src_bytes == 2 * dst_bytes, one_to_two = dst_bytes == 2 * src_bytes;
        lk::require(two_to_one || one_to_two, "src_bytes and dst_bytes must be in the ratio 2:1 or 1:2");
        const uint64_t in_word = two_to_one ? 16 : 8;
        lk::require(src_bytes % in_word == 0, "src_bytes must be a multiple of 16 (2:1) or 8 (1:2)");
        if (src_bytes == 0) return;
        const uint64_t words = src_bytes / in_word, waves = (words + lk::kWave - 1) / lk::kWave;
        lk::require(waves <= 0x7FFFFFFFull, "probe too large");
        const auto s = static_cast<hipStream_t>(stream);
        const auto in = static_cast<const uint8_t*>(src);
        const auto out = static_cast<uint8_t*>(dst);
        if (two_to_one) hipLaunchKernelGGL((lk::wave_stream_probe<16, 8>), dim3(uint32_t(waves)), dim3(lk::kWave), 0, s, in, out, words);
        else hipLaunchKernelGGL((lk::wave_stream_probe<8, 16>), dim3(uint32_t(waves)), dim3(lk::kWave), 0, s, in, out, words);
    });
}
