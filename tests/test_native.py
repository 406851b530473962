"""The transfer library's host flavour: the behaviour of the reference's tests/test_native.py,
run against this repo's library and, where oracle/_ref holds it, against the reference's own
host build compiled from its sources, so every behavioural claim is checked on both.

Byte-exactness uses CRC32 and byte comparison (reference test_native.py:48-63)."""

import ctypes
import mmap
import random
import subprocess
import time
import zlib

import numpy as np
import pytest
import torch

from layover_amd import CSRC_DIR
from layover_amd.kv import native
from layover_amd.kv.native import Engine, HostMemoryError, NativeError, NativeUnavailable, build_host, library_path, load_library
from oracle import oracle

BLOCK = 8192
MIB = 1 << 20
IMPLEMENTATIONS = ["ours"] + (["reference"] if oracle.REFERENCE_LIBRARY.exists() else [])


@pytest.fixture(scope="module", autouse=True)
def built():
    build_host()


@pytest.fixture(params=IMPLEMENTATIONS)
def make_engine(request):
    library = None if request.param == "ours" else oracle.REFERENCE_LIBRARY
    created = []

    def make(**options):
        engine = Engine("host", library=library, **options)
        created.append(engine)
        return engine

    make.implementation = request.param
    yield make
    for engine in created:
        try:
            engine.destroy()
        except NativeError:
            pass


@pytest.fixture
def engine(make_engine):
    return make_engine(staging_bytes=2 * BLOCK, ids_capacity=64, host_cache_bytes=1 << 24)


def filled_pool(blocks, block_bytes=BLOCK, seed=0):
    return torch.randint(0, 256, (blocks * block_bytes,), dtype=torch.uint8, generator=torch.Generator().manual_seed(seed))


def host_bytes(pointer, nbytes):
    return bytes((ctypes.c_uint8 * nbytes).from_address(pointer))


def blocks_of(pool, ids, block_bytes=BLOCK):
    return b"".join(pool[i * block_bytes : (i + 1) * block_bytes].numpy().tobytes() for i in ids)


def finish(engine, transfer):
    engine.wait(transfer)
    engine.release(transfer)


def round_trip(engine, pool, ids, out=None, into=None, block_bytes=BLOCK):
    out = out or engine.out_gather
    into = into or engine.in_scatter
    before = zlib.crc32(blocks_of(pool, ids, block_bytes))
    host = engine.host_alloc(len(ids) * block_bytes)
    finish(engine, out(pool.data_ptr(), block_bytes, ids, host))
    assert zlib.crc32(host_bytes(host, len(ids) * block_bytes)) == before
    # The oracle's gather is the same bytes (pack.h:56-61).
    assert host_bytes(host, len(ids) * block_bytes) == oracle.gather(pool.numpy(), block_bytes, ids).tobytes()
    for i in ids:
        pool[i * block_bytes : (i + 1) * block_bytes] = 0
    finish(engine, into(pool.data_ptr(), block_bytes, ids, host))
    assert zlib.crc32(blocks_of(pool, ids, block_bytes)) == before
    engine.host_free(host)


def test_library_exports_every_declared_symbol():
    lib = load_library("host")
    header = (CSRC_DIR.parent.parent / "include" / "layover_transfer.h").read_text()
    declared = {line.split("(")[0].split()[-1].lstrip("*") for line in header.splitlines() if line.startswith(("int lt_", "const char* lt_"))}
    assert len(declared) == 26
    for name in declared:
        assert hasattr(lib, name), name
    assert lib.lt_flavor() == b"host"
    assert lib.lt_abi_version() == 2


def test_flavor_and_abi_are_checked():
    with pytest.raises(NativeUnavailable):
        load_library("no-such-flavor")
    with pytest.raises(NativeUnavailable, match="flavor"):
        load_library("hip", library_path("host"))


def test_build_is_keyed_by_platform_and_flavor():
    path = library_path("host")
    assert path.exists() and path.parent.name.startswith("host-")
    assert library_path("hip").parent.name.startswith("hip-")


@pytest.mark.parametrize("ids", [[0], [7, 2, 5], [3, 0, 7, 1, 6, 2, 5, 4]], ids=["one", "few", "all_shuffled"])
def test_gather_and_scatter_round_trip_scattered_blocks(engine, ids):
    round_trip(engine, filled_pool(8), ids)


def test_host_order_follows_the_id_list_and_other_blocks_stay_put(engine):
    pool = filled_pool(8)
    original = pool.clone()
    ids = [6, 1, 4]
    host = engine.host_alloc(3 * BLOCK)
    finish(engine, engine.out_gather(pool.data_ptr(), BLOCK, ids, host))
    assert host_bytes(host, 3 * BLOCK) == blocks_of(original, ids)
    pool[:] = 0
    finish(engine, engine.in_scatter(pool.data_ptr(), BLOCK, [2, 5, 0], host))
    assert blocks_of(pool, [2, 5, 0]) == blocks_of(original, ids)
    assert blocks_of(pool, [1, 3, 4, 6, 7]) == b"\0" * (5 * BLOCK)


@pytest.mark.parametrize("block_bytes", [64, 8, 2048, 65536, 65536 + 8, 262144, 2_359_296 // 16], ids=lambda b: f"{b}B")
def test_block_sizes_around_chunk_and_lane_boundaries(make_engine, block_bytes):
    engine = make_engine(staging_bytes=4 * block_bytes, ids_capacity=8)
    round_trip(engine, filled_pool(5, block_bytes), [3, 0, 4], block_bytes=block_bytes)


def test_transfer_larger_than_staging_splits_into_segments(engine):
    pool = filled_pool(16)
    before = engine.stats()
    round_trip(engine, pool, [15, 3, 8, 0, 12, 1, 9, 6, 2])
    after = engine.stats()
    delta = {key: after[key] - before[key] for key in ("kernels", "memcpys", "ids_uploads", "bytes_to_host", "bytes_to_device")}
    assert delta == {"kernels": 10, "memcpys": 10, "ids_uploads": 2, "bytes_to_host": 9 * BLOCK, "bytes_to_device": 9 * BLOCK}


def test_one_dma_per_segment_and_not_per_block(make_engine):
    wide = make_engine(staging_bytes=64 * BLOCK, ids_capacity=64)
    round_trip(wide, filled_pool(64), list(range(64)))
    stats = wide.stats()
    assert stats["memcpys"] == 2 and stats["kernels"] == 2


def test_per_block_baseline_copies_once_per_block_and_is_correct(engine):
    round_trip(engine, filled_pool(8), [7, 2, 5, 0], engine.out_per_block, engine.in_per_block)
    stats = engine.stats()
    assert stats["memcpys"] == 8 and stats["kernels"] == 0 and stats["ids_uploads"] == 0


def test_slow_copies_do_not_let_a_later_gather_overwrite_staging(engine):
    engine.set_copy_delay_us(2000)
    round_trip(engine, filled_pool(16), [15, 3, 8, 0, 12, 1, 9, 6, 2, 10, 4, 14])


def test_two_overlapping_transfers_finish_correct(engine):
    pool = filled_pool(16)
    original = pool.clone()
    engine.set_paused(True)
    first_ids, second_ids = [1, 9, 3, 11, 5], [14, 0, 7]
    first_host, second_host = engine.host_alloc(5 * BLOCK), engine.host_alloc(3 * BLOCK)
    first = engine.out_gather(pool.data_ptr(), BLOCK, first_ids, first_host)
    second = engine.out_gather(pool.data_ptr(), BLOCK, second_ids, second_host)
    assert not engine.poll(first) and not engine.poll(second)
    engine.set_paused(False)
    engine.wait(second)
    engine.wait(first)
    assert host_bytes(first_host, 5 * BLOCK) == blocks_of(original, first_ids)
    assert host_bytes(second_host, 3 * BLOCK) == blocks_of(original, second_ids)


def test_poll_does_not_block_and_turns_true_on_completion(engine):
    pool = filled_pool(4)
    engine.set_paused(True)
    host = engine.host_alloc(4 * BLOCK)
    transfer = engine.out_gather(pool.data_ptr(), BLOCK, [0, 1, 2, 3], host)
    start = time.perf_counter()
    assert engine.poll(transfer) is False
    assert time.perf_counter() - start < 0.5
    with pytest.raises(NativeError, match="in flight"):
        engine.release(transfer)
    engine.set_paused(False)
    deadline = time.monotonic() + 30
    while not engine.poll(transfer):
        assert time.monotonic() < deadline
    engine.release(transfer)
    with pytest.raises(NativeError, match="not a live transfer"):
        engine.poll(transfer)


def test_destroy_mid_flight_waits_and_frees_everything(make_engine):
    engine = make_engine(staging_bytes=2 * BLOCK, ids_capacity=64)
    pool = filled_pool(8)
    engine.set_copy_delay_us(5000)
    host = engine.host_alloc(8 * BLOCK)
    transfer = engine.out_gather(pool.data_ptr(), BLOCK, list(range(8)), host)
    assert not engine.poll(transfer)
    engine.destroy()
    assert engine.closed
    engine.destroy()
    with pytest.raises(NativeError, match="closed"):
        engine.stats()


def test_destroy_while_paused_does_not_hang(make_engine):
    engine = make_engine(staging_bytes=2 * BLOCK, ids_capacity=64)
    pool = filled_pool(4)
    engine.set_paused(True)
    host = engine.host_alloc(4 * BLOCK)
    engine.out_gather(pool.data_ptr(), BLOCK, [0, 1, 2, 3], host)
    engine.destroy()


def test_id_ring_wraps_and_reclaims_across_many_transfers(make_engine):
    engine = make_engine(staging_bytes=8 * BLOCK, ids_capacity=8)
    pool = filled_pool(8)
    for index in range(40):
        ids = np.random.default_rng(index).permutation(8)[: 1 + index % 8]
        round_trip(engine, pool, [int(i) for i in ids])


def test_full_id_ring_applies_backpressure_instead_of_failing(make_engine):
    engine = make_engine(staging_bytes=8 * BLOCK, ids_capacity=8)
    pool = filled_pool(8)
    original = pool.clone()
    engine.set_copy_delay_us(1000)
    hosts = [engine.host_alloc(6 * BLOCK) for _ in range(5)]
    rows = [[(i + j) % 8 for j in range(6)] for i in range(5)]
    transfers = [engine.out_gather(pool.data_ptr(), BLOCK, row, host) for row, host in zip(rows, hosts)]
    for transfer in transfers:
        engine.wait(transfer)
    for row, host in zip(rows, hosts):
        assert host_bytes(host, 6 * BLOCK) == blocks_of(original, row)


def test_transfers_address_the_pool_with_64_bits(make_engine):
    block = 2_359_296
    pool_blocks, source, target = 2400, 2399, 2100
    assert source * block > 1 << 32
    mapped = mmap.mmap(-1, pool_blocks * block, flags=mmap.MAP_PRIVATE | getattr(mmap, "MAP_NORESERVE", 0))
    pointer = ctypes.addressof(ctypes.c_char.from_buffer(mapped))
    pattern = bytes(random.Random(0).getrandbits(8) for _ in range(4096)) * (block // 4096)
    mapped[source * block : (source + 1) * block] = pattern
    engine = make_engine(staging_bytes=2 * block, ids_capacity=8)
    host = engine.host_alloc(block)
    finish(engine, engine.out_gather(pointer, block, [source], host))
    assert host_bytes(host, block) == pattern
    finish(engine, engine.in_scatter(pointer, block, [target], host))
    assert mapped[target * block : (target + 1) * block] == pattern
    wrapped = (target * block) % (1 << 32)
    assert mapped[wrapped : wrapped + 4096] == bytes(4096)
    engine.destroy()


def test_segments_are_capped_like_the_reference(make_engine):
    engine = make_engine(staging_bytes=1 << 20, ids_capacity=1 << 18)
    count = 70_000
    pool = torch.arange(count, dtype=torch.int64)
    host = engine.host_alloc(8 * count)
    finish(engine, engine.out_gather(pool.data_ptr(), 8, list(range(count)), host))
    assert host_bytes(host, 8 * count) == pool.numpy().tobytes()
    stats = engine.stats()
    assert stats["kernels"] == 2 and stats["memcpys"] == 2


@pytest.mark.parametrize(
    "request_bytes,pinned",
    [(1, MIB), (MIB, MIB), (MIB + 1, 5 << 18), (40 * MIB, 40 * MIB), (40 * MIB + 1, 48 * MIB), (3 * MIB, 3 * MIB), (2 * MIB + 1, 5 * MIB // 2)],
    ids=["tiny", "smallest_class", "just_over", "on_a_class", "just_over_a_class", "three_mib", "two_mib_plus"],
)
def test_pinned_allocations_waste_at_most_a_quarter(make_engine, request_bytes, pinned):
    engine = make_engine(staging_bytes=MIB, ids_capacity=8)
    pointer = engine.host_alloc(request_bytes)
    assert engine.stats()["host_bytes_live"] == pinned
    assert pinned <= max(MIB, request_bytes * 5 // 4)
    engine.host_free(pointer)


def test_host_buffers_are_reused_and_accounted(engine):
    first = engine.host_alloc(1000)
    held = engine.stats()["host_bytes_held"]
    engine.host_free(first)
    assert engine.stats()["host_bytes_live"] == 0
    assert engine.host_alloc(2000) == first
    assert engine.stats()["host_bytes_held"] == held
    with pytest.raises(NativeError, match="not a live host buffer"):
        engine.host_free(12345)


def test_cache_limit_returns_memory_to_the_system(make_engine):
    engine = make_engine(staging_bytes=BLOCK, ids_capacity=8, host_cache_bytes=0)
    engine.host_free(engine.host_alloc(1000))
    assert engine.stats()["host_bytes_held"] == 0


@pytest.mark.parametrize(
    "call,match",
    [
        (lambda e, p, h: e.out_gather(p, 16 * BLOCK, [0], h), "larger than a staging"),
        (lambda e, p, h: e.out_gather(p + 1, BLOCK, [0], h), "8-byte aligned"),
        (lambda e, p, h: e.out_gather(p, BLOCK - 4, [0], h), "multiple of 8"),
        (lambda e, p, h: e.out_gather(p, BLOCK, list(range(65)), h), "ids_capacity"),
        (lambda e, p, h: e.in_scatter(None, BLOCK, [0], h), "null pool"),
        (lambda e, p, h: e.ext_copy_out(p, h, BLOCK, 99), "bad slot"),
    ],
    ids=["block_too_big", "misaligned_pool", "odd_block", "too_many_ids", "null_pool", "bad_slot"],
)
def test_misuse_raises_with_the_reason_and_engine_stays_usable(engine, call, match):
    pool = filled_pool(2)
    host = engine.host_alloc(2 * BLOCK)
    with pytest.raises(NativeError, match=match):
        call(engine, pool.data_ptr(), host)
    round_trip(engine, filled_pool(4), [1, 3])


def test_bad_construction_is_refused(make_engine):
    with pytest.raises(NativeError):
        make_engine(staging_bytes=0)


def test_failed_kernel_is_surfaced_and_stops_further_work(make_engine):
    engine = make_engine(staging_bytes=BLOCK, ids_capacity=8)
    stream = engine.host_stream()

    def kernel():
        raise ValueError("boom")

    keep = engine.host_call(stream, kernel)
    transfer = engine.ext_finish(stream)
    with pytest.raises(NativeError, match="boom"):
        for _ in range(100_000):
            engine.poll(transfer)
    with pytest.raises(NativeError):
        engine.host_alloc(16)
    with pytest.raises(NativeError, match="host kernel failed"):
        engine.destroy()
    assert engine.closed
    del keep


def test_a_null_stream_is_refused_instead_of_meaning_the_legacy_default(engine):
    with pytest.raises(NativeError, match="null stream"):
        engine.ext_wait(None, 0, 0)
    with pytest.raises(NativeError, match="null stream"):
        engine.ext_record(None, 0, 0)


def test_ext_pipeline_orders_caller_kernels_against_the_copy_stream(engine):
    """The FP8 path's protocol (layover_transfer.h:84-96) on host streams: a caller kernel
    fills a stage, the copy stream drains it, and a slow copy never sees a later fill."""
    stream = engine.host_stream()
    stage = torch.zeros(BLOCK, dtype=torch.uint8)
    host = engine.host_alloc(4 * BLOCK)
    engine.set_copy_delay_us(3000)
    keep = []
    for index in range(4):
        engine.ext_wait(stream, index % 2, native.SLOT_RELEASED)
        keep.append(engine.host_call(stream, lambda index=index: stage.fill_(index + 1)))
        engine.ext_record(stream, index % 2, native.SLOT_FILLED)
        engine.ext_copy_out(stage.data_ptr(), host + index * BLOCK, BLOCK, index % 2)
    finish(engine, engine.ext_finish(None))
    # One stage shared by both slots is a caller bug the slot events cannot fix; what they do
    # guarantee is that every copy saw a completed fill.
    data = host_bytes(host, 4 * BLOCK)
    for index in range(4):
        chunk = data[index * BLOCK : (index + 1) * BLOCK]
        assert len(set(chunk)) == 1 and chunk[0] in range(1, 5)


def test_c_checks_pass_under_address_and_undefined_sanitizers():
    done = subprocess.run(["make", "-C", str(CSRC_DIR), "check"], capture_output=True, text=True, timeout=600)
    assert done.returncode == 0, done.stderr[-3000:] + done.stdout[-3000:]
    assert "host_check: ok" in done.stdout


def test_a_full_host_cache_gives_up_what_it_has_held_longest(engine):
    old, kept = engine.host_alloc(4 * MIB), engine.host_alloc(5 * MIB)
    engine.host_free(old)
    engine.host_free(kept)
    large = engine.host_alloc(10 * MIB)
    engine.host_free(large)
    pins = engine.stats()["host_pins"]
    assert engine.host_alloc(10 * MIB) == large
    assert engine.host_alloc(5 * MIB) == kept
    assert engine.stats()["host_pins"] == pins
    engine.host_alloc(4 * MIB)
    assert engine.stats()["host_pins"] == pins + 1


def test_a_buffer_larger_than_the_cache_is_not_kept(engine):
    engine.host_free(engine.host_alloc(20 * MIB))
    assert engine.stats()["host_bytes_held"] == 0


def test_pins_are_counted_and_timed_and_a_cached_buffer_is_not_a_pin(engine):
    pointer = engine.host_alloc(MIB)
    stats = engine.stats()
    assert stats["host_pins"] == 1 and stats["host_pin_bytes"] == MIB
    assert stats["host_pin_ns"] > 0 and stats["host_pin_max_ns"] == stats["host_pin_ns"]
    engine.host_free(pointer)
    engine.host_alloc(MIB)
    assert engine.stats()["host_pins"] == 1


def test_a_failed_pin_is_its_own_error_and_leaves_the_engine_working(engine):
    engine.set_pin_limit(MIB)
    with pytest.raises(HostMemoryError):
        engine.host_alloc(2 * MIB)
    assert engine.stats()["host_pin_failures"] == 1
    assert engine.stats()["host_bytes_held"] == 0
    engine.set_pin_limit(1 << 40)
    original = filled_pool(4)
    host = engine.host_alloc(2 * BLOCK)
    finish(engine, engine.out_gather(original.data_ptr(), BLOCK, [2, 0], host))
    assert host_bytes(host, 2 * BLOCK) == blocks_of(original, [2, 0])


def test_a_failed_pin_gives_back_cached_memory_before_giving_up(engine):
    engine.set_pin_limit(5 * MIB)
    engine.host_free(engine.host_alloc(4 * MIB))
    engine.host_alloc(3 * MIB)
    stats = engine.stats()
    assert stats["host_pin_failures"] == 0 and stats["host_bytes_held"] == 3 * MIB


def test_a_bad_request_is_not_mistaken_for_a_failed_pin(engine):
    with pytest.raises(NativeError) as raised:
        engine.host_alloc(0)
    assert not isinstance(raised.value, HostMemoryError)
