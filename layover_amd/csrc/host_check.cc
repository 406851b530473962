// Checks of the host flavour built with the address and undefined-behaviour sanitizers
// (make check). Each case drives the C ABI only and exits non-zero on the first failure:
//   - swaps of random blocks out and back into other ids, for block sizes on and off the
//     16-byte word, through staging that forces many segments, and an id ring small enough
//     to wrap within every swap;
//   - two swaps in flight at once on one engine, finishing in either order;
//   - the FP8-style caller path: a caller "kernel" on the host stream fills a slot, the engine
//     copies it out, and the reverse;
//   - teardown with work queued and with every stream paused.
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <numeric>
#include <random>
#include <vector>

#include "layover_transfer.h"

namespace {

int failures = 0;

void expect(bool ok, const char* what) {
    if (!ok) {
        fprintf(stderr, "host_check: %s (%s)\n", what, lt_last_error());
        ++failures;
        exit(1);
    }
}

void ok(int status, const char* what) { expect(status == LT_OK, what); }

struct Pool {
    uint64_t block_bytes;
    std::vector<uint8_t> bytes;
    Pool(uint64_t block, uint32_t blocks, uint64_t seed) : block_bytes(block), bytes(block * blocks) {
        std::mt19937 draw{uint32_t(seed)};
        for (uint8_t& b : bytes) b = uint8_t(draw());
    }
    uint8_t* block(uint32_t id) { return bytes.data() + uint64_t(id) * block_bytes; }
};

std::vector<uint32_t> shuffled(uint32_t n, uint64_t seed) {
    std::vector<uint32_t> ids(n);
    std::iota(ids.begin(), ids.end(), 0u);
    std::shuffle(ids.begin(), ids.end(), std::mt19937(uint32_t(seed)));
    return ids;
}

void finish(lt_engine* engine, lt_transfer* transfer) {
    ok(lt_wait(engine, transfer), "wait");
    ok(lt_release(engine, transfer), "release");
}

// Out from `from`, back into `into` (disjoint), then compare block by block.
void swap_case(uint64_t block_bytes, uint32_t blocks, uint32_t moved, uint32_t staging_blocks, uint32_t ring, uint64_t seed) {
    Pool pool(block_bytes, blocks, seed);
    const std::vector<uint32_t> order = shuffled(blocks, seed + 1);
    std::vector<uint32_t> from(order.begin(), order.begin() + moved);
    std::vector<uint32_t> into(order.begin() + moved, order.begin() + 2 * moved);
    lt_engine* engine = nullptr;
    ok(lt_create(0, staging_blocks * block_bytes, 2, ring, 64ull << 20, &engine), "create");
    for (int repeat = 0; repeat < 3; ++repeat) {
        void* host = nullptr;
        ok(lt_host_alloc(engine, moved * block_bytes, &host), "host_alloc");
        lt_transfer* out = nullptr;
        ok(lt_out_gather(engine, pool.bytes.data(), block_bytes, from.data(), moved, host, &out), "out_gather");
        finish(engine, out);
        for (uint32_t i = 0; i < moved; ++i)
            expect(memcmp(static_cast<uint8_t*>(host) + i * block_bytes, pool.block(from[i]), block_bytes) == 0, "gathered record differs");
        const Pool untouched = pool;
        lt_transfer* in = nullptr;
        ok(lt_in_scatter(engine, pool.bytes.data(), block_bytes, into.data(), moved, host, &in), "in_scatter");
        finish(engine, in);
        std::vector<bool> target(blocks, false);
        for (uint32_t i = 0; i < moved; ++i) {
            target[into[i]] = true;
            expect(memcmp(pool.block(into[i]), static_cast<uint8_t*>(host) + i * block_bytes, block_bytes) == 0, "scattered block differs");
        }
        for (uint32_t id = 0; id < blocks; ++id)
            if (!target[id]) expect(memcmp(pool.block(id), untouched.bytes.data() + uint64_t(id) * block_bytes, block_bytes) == 0, "a block outside the targets changed");
        ok(lt_host_free(engine, host), "host_free");
        std::swap(from, into);
    }
    lt_stats stats{};
    ok(lt_get_stats(engine, &stats), "stats");
    const uint64_t per_swap = (moved + staging_blocks - 1) / staging_blocks;
    expect(stats.kernels == 2 * 3 * per_swap, "one kernel per segment");
    expect(stats.ids_uploads == 2 * 3, "one id upload per transfer");
    ok(lt_destroy(engine), "destroy");
}

void overlapping_case() {
    const uint64_t block = 4096;
    Pool pool(block, 40, 7);
    lt_engine* engine = nullptr;
    ok(lt_create(0, 3 * block, 2, 16, 1 << 24, &engine), "create");
    ok(lt_host_set_copy_delay_us(engine, 300), "delay");
    std::vector<uint32_t> a = {3, 17, 9, 30, 1, 22, 5}, b = {11, 2, 38, 14, 27, 8, 19};
    void *ha = nullptr, *hb = nullptr;
    ok(lt_host_alloc(engine, a.size() * block, &ha), "alloc a");
    ok(lt_host_alloc(engine, b.size() * block, &hb), "alloc b");
    lt_transfer *ta = nullptr, *tb = nullptr;
    ok(lt_out_gather(engine, pool.bytes.data(), block, a.data(), uint32_t(a.size()), ha, &ta), "out a");
    ok(lt_out_gather(engine, pool.bytes.data(), block, b.data(), uint32_t(b.size()), hb, &tb), "out b");
    int done = 0;
    ok(lt_poll(engine, tb, &done), "poll b");
    finish(engine, tb);  // the later one first
    finish(engine, ta);
    for (size_t i = 0; i < a.size(); ++i) expect(memcmp(static_cast<uint8_t*>(ha) + i * block, pool.block(a[i]), block) == 0, "a");
    for (size_t i = 0; i < b.size(); ++i) expect(memcmp(static_cast<uint8_t*>(hb) + i * block, pool.block(b[i]), block) == 0, "b");
    ok(lt_destroy(engine), "destroy");
}

struct Fill {
    uint8_t* staging;
    uint64_t bytes;
    uint8_t value;
};

int fill_kernel(void* context) {
    Fill* fill = static_cast<Fill*>(context);
    memset(fill->staging, fill->value, fill->bytes);
    return 0;
}

// The "dequantize" side: the slot must hold the segment's bytes when the kernel runs.
int check_kernel(void* context) {
    const Fill* fill = static_cast<const Fill*>(context);
    for (uint64_t i = 0; i < fill->bytes; ++i)
        if (fill->staging[i] != fill->value) return 1;
    return 0;
}

void caller_path_case() {
    lt_engine* engine = nullptr;
    ok(lt_create(0, 1 << 16, 2, 8, 1 << 24, &engine), "create");
    void* stream = nullptr;
    ok(lt_host_stream(engine, &stream), "host_stream");
    std::vector<uint8_t> staging[2] = {std::vector<uint8_t>(1 << 16), std::vector<uint8_t>(1 << 16)};
    void* host = nullptr;
    ok(lt_host_alloc(engine, 6 << 16, &host), "alloc");
    Fill fills[6];
    for (uint32_t segment = 0; segment < 6; ++segment) {
        const uint32_t slot = segment % 2;
        fills[segment] = {staging[slot].data(), 1 << 16, uint8_t(0x30 + segment)};
        ok(lt_ext_wait(engine, stream, slot, LT_SLOT_RELEASED), "ext_wait");
        ok(lt_host_call(engine, stream, fill_kernel, &fills[segment]), "host_call");
        ok(lt_ext_record(engine, stream, slot, LT_SLOT_FILLED), "ext_record");
        ok(lt_ext_copy_out(engine, staging[slot].data(), static_cast<uint8_t*>(host) + (uint64_t(segment) << 16), 1 << 16, slot), "copy_out");
    }
    lt_transfer* out = nullptr;
    ok(lt_ext_finish(engine, nullptr, &out), "finish");
    finish(engine, out);
    for (uint32_t segment = 0; segment < 6; ++segment) {
        const uint8_t* record = static_cast<uint8_t*>(host) + (uint64_t(segment) << 16);
        expect(record[0] == 0x30 + segment && record[(1 << 16) - 1] == 0x30 + segment, "segment overwritten before its copy");
    }
    for (uint32_t segment = 0; segment < 6; ++segment) {
        const uint32_t slot = segment % 2;
        ok(lt_ext_copy_in(engine, staging[slot].data(), static_cast<uint8_t*>(host) + (uint64_t(segment) << 16), 1 << 16, slot), "copy_in");
        ok(lt_ext_wait(engine, stream, slot, LT_SLOT_FILLED), "ext_wait");
        ok(lt_host_call(engine, stream, check_kernel, &fills[segment]), "host_call");
        ok(lt_ext_record(engine, stream, slot, LT_SLOT_RELEASED), "ext_record");
    }
    lt_transfer* in = nullptr;
    ok(lt_ext_finish(engine, stream, &in), "finish");
    finish(engine, in);  // a check kernel that saw the wrong bytes fails the engine here
    expect(lt_ext_wait(engine, nullptr, 0, LT_SLOT_FILLED) == LT_ERR_INVALID, "null stream refused");
    expect(lt_ext_wait(engine, stream, 2, LT_SLOT_FILLED) == LT_ERR_INVALID, "slot past num_staging refused");
    ok(lt_host_free(engine, host), "free");
    ok(lt_destroy(engine), "destroy");
}

void teardown_case(bool paused) {
    const uint64_t block = 8192;
    Pool pool(block, 24, 11);
    lt_engine* engine = nullptr;
    ok(lt_create(0, 2 * block, 2, 32, 1 << 24, &engine), "create");
    void* host = nullptr;
    ok(lt_host_alloc(engine, 20 * block, &host), "alloc");
    if (paused) ok(lt_host_set_paused(engine, 1), "pause");
    const std::vector<uint32_t> ids = shuffled(24, 3);
    lt_transfer* out = nullptr;
    ok(lt_out_gather(engine, pool.bytes.data(), block, ids.data(), 20, host, &out), "out");
    int done = 1;
    ok(lt_poll(engine, out, &done), "poll");
    if (paused) expect(done == 0, "a paused engine finished a transfer");
    ok(lt_destroy(engine), "destroy with work queued");
}

}  // namespace

int main() {
    swap_case(4096, 40, 13, 2, 20, 1);         // 7 segments; a 20-id ring wraps on every other transfer
    swap_case(8, 64, 20, 3, 64, 2);             // one 8-byte word per block
    swap_case(65536 + 24, 10, 5, 5, 8, 3);      // 8-byte words only, one segment
    swap_case(1 << 20, 8, 4, 1, 4, 4);          // one block per segment
    swap_case(2359296 / 8, 12, 6, 4, 6, 5);     // a Qwen3-4B layer pair
    overlapping_case();
    caller_path_case();
    teardown_case(false);
    teardown_case(true);
    printf("host_check: ok\n");
    return failures;
}
