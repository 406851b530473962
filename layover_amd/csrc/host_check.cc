// C++ checks of the host flavour, run under the address and undefined-behaviour sanitizers by
// `make check`: scattered round trips, many segments, an id ring that wraps, a block of
// exactly the staging size, partial last chunks, and teardown with work still queued. Exits
// non-zero on the first failure.
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <numeric>
#include <random>
#include <vector>

#include "layover_transfer.h"

static void must(int status, const char* what) {
    if (status != LT_OK) {
        fprintf(stderr, "%s failed: %s\n", what, lt_last_error());
        exit(1);
    }
}

static void finish(lt_engine* engine, lt_transfer* transfer) {
    must(lt_wait(engine, transfer), "wait");
    must(lt_release(engine, transfer), "release");
}

static void case_round_trips(uint64_t block_bytes, uint32_t pool_blocks, uint32_t count, uint64_t staging, uint32_t ring, uint32_t seed) {
    std::mt19937 random(seed);
    std::vector<uint8_t> pool(block_bytes * pool_blocks);
    for (auto& byte : pool) byte = uint8_t(random());
    const std::vector<uint8_t> original = pool;
    std::vector<uint32_t> ids(pool_blocks);
    std::iota(ids.begin(), ids.end(), 0u);
    std::shuffle(ids.begin(), ids.end(), random);
    ids.resize(count);

    lt_engine* engine = nullptr;
    must(lt_create(0, staging, 2, ring, 1 << 24, &engine), "create");
    for (int round = 0; round < 4; ++round) {
        void* host = nullptr;
        must(lt_host_alloc(engine, block_bytes * count, &host), "host_alloc");
        lt_transfer* transfer = nullptr;
        must(lt_out_gather(engine, pool.data(), block_bytes, ids.data(), count, host, &transfer), "out_gather");
        finish(engine, transfer);
        for (uint32_t id : ids) memset(pool.data() + uint64_t(id) * block_bytes, 0, block_bytes);
        must(lt_in_scatter(engine, pool.data(), block_bytes, ids.data(), count, host, &transfer), "in_scatter");
        finish(engine, transfer);
        if (pool != original) {
            fprintf(stderr, "round trip of %u blocks of %llu bytes changed the pool\n", count, (unsigned long long)block_bytes);
            exit(1);
        }
        must(lt_host_free(engine, host), "host_free");
    }
    void* host = nullptr;
    must(lt_host_alloc(engine, block_bytes * count, &host), "host_alloc");
    lt_transfer* transfer = nullptr;
    must(lt_out_gather(engine, pool.data(), block_bytes, ids.data(), count, host, &transfer), "out_gather");
    must(lt_destroy(engine), "destroy with work queued");
}

int main() {
    case_round_trips(4096, 16, 9, 8192, 12, 1);
    case_round_trips(6144, 8, 8, 6144, 8, 2);
    case_round_trips(1 << 20, 6, 5, 3 << 20, 16, 3);
    case_round_trips((1 << 18) + 8, 6, 6, 1 << 21, 8, 4);
    printf("host_check: ok\n");
    return 0;
}
