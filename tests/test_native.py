"""The swap library's host flavour through its C ABI, run on two builds: this package's
(layover_amd/csrc, host_streams.h + swap_engine.h) and, where oracle/_ref holds it, the
reference's own host library compiled from its sources. Each behaviour the ABI promises is
asserted on both, so a difference between them fails here.

What is covered: byte-exact round trips of scattered blocks (a seeded sweep over block
sizes, staging sizes, id-ring sizes and id orders, checked against the oracle's gather and
scatter, pack.h:56-68), the counters of a staged transfer (the reference's own known answer,
its tests/test_native.py:114-124), the segment cap, 64-bit pool offsets, the pinned cache
(size classes, reuse, oldest-first eviction, limits, failed pins), overlap under slow and
paused streams, the caller-staging path (lt_ext_*), misuse and device-failure codes, and
teardown with work in flight.
"""

import ctypes
import mmap
import subprocess

import numpy as np
import pytest

from layover_amd import CSRC_DIR
from layover_amd.kv.native import (LT_ERR_DEVICE, LT_ERR_INVALID, SLOT_FILLED, SLOT_RELEASED, Engine, HostMemoryError, NativeError,
                                   NativeUnavailable, build_host, load_library)
from oracle import oracle

MIB = 1 << 20
BUILDS = ["package"] + (["reference"] if oracle.REFERENCE_LIBRARY.exists() else [])


@pytest.fixture(scope="module", autouse=True)
def host_library():
    build_host()


@pytest.fixture(params=BUILDS)
def new_engine(request):
    """Makes engines on one build and destroys them after the test."""
    path = oracle.REFERENCE_LIBRARY if request.param == "reference" else None
    made = []

    def make(staging_bytes=4 * 4096, num_staging=2, ids_capacity=64, host_cache_bytes=64 * MIB):
        engine = Engine("host", 0, staging_bytes, num_staging, ids_capacity, host_cache_bytes, library=path)
        made.append(engine)
        return engine

    yield make
    for engine in made:
        try:
            engine.destroy()
        except NativeError:
            pass


class Pool:
    """A byte pool in a numpy array; block i is bytes [i*B, (i+1)*B)."""

    def __init__(self, blocks, block_bytes, seed):
        self.block_bytes = block_bytes
        self.bytes = np.random.default_rng(seed).integers(0, 256, blocks * block_bytes, dtype=np.uint8)

    @property
    def address(self):
        return self.bytes.ctypes.data

    def block(self, i):
        return self.bytes[i * self.block_bytes : (i + 1) * self.block_bytes]


def host_view(pointer, nbytes):
    return np.ctypeslib.as_array((ctypes.c_uint8 * nbytes).from_address(pointer))


def done(engine, transfer):
    engine.wait(transfer)
    engine.release(transfer)


def swap(engine, pool, out_ids, in_ids):
    """Out from out_ids, back into in_ids; checks both legs against the oracle."""
    b = pool.block_bytes
    host = engine.host_alloc(len(out_ids) * b)
    done(engine, engine.out_gather(pool.address, b, out_ids, host))
    records = host_view(host, len(out_ids) * b)
    assert np.array_equal(records, oracle.gather(pool.bytes, b, out_ids))
    expected = pool.bytes.copy()
    oracle.scatter(expected, b, in_ids, records)
    done(engine, engine.in_scatter(pool.address, b, in_ids, host))
    assert np.array_equal(pool.bytes, expected)
    engine.host_free(host)


def sweep(count=24, seed=7):
    rng = np.random.default_rng(seed)
    for _ in range(count):
        block = int(rng.choice([8, 16, 24, 4096, 8200, 65536, 65544, 3 * 65536 + 40]))
        blocks = int(rng.integers(4, 40))
        moved = int(rng.integers(1, blocks // 2 + 1))
        yield dict(block=block, blocks=blocks, moved=moved, staging=int(rng.integers(1, 6)),
                   ring=int(rng.integers(moved, 3 * moved + 1)), seed=int(rng.integers(1 << 30)))


@pytest.mark.parametrize("case", list(sweep()), ids=lambda c: f"B{c['block']}-n{c['moved']}-s{c['staging']}-r{c['ring']}")
def test_scattered_swaps_match_the_oracle(new_engine, case):
    engine = new_engine(staging_bytes=case["staging"] * case["block"], ids_capacity=case["ring"])
    pool = Pool(case["blocks"], case["block"], case["seed"])
    order = np.random.default_rng(case["seed"]).permutation(case["blocks"]).tolist()
    n = case["moved"]
    for _ in range(3):  # the id ring wraps across repeats
        swap(engine, pool, order[:n], order[n : 2 * n] if 2 * n <= len(order) else order[:n][::-1])


def test_counters_of_a_staged_swap(new_engine):
    # Nine 8 KiB blocks through 2-block slots: 5 segments each way, so 10 kernels and 10 DMAs,
    # one id upload per transfer, 9 x 8 KiB each way (the reference's known answer).
    engine = new_engine(staging_bytes=2 * 8192, ids_capacity=64)
    pool = Pool(16, 8192, 1)
    swap(engine, pool, [3, 9, 0, 14, 7, 1, 12, 5, 10], [2, 4, 6, 8, 11, 13, 15, 3, 9])
    stats = engine.stats()
    assert (stats["kernels"], stats["memcpys"], stats["ids_uploads"], stats["transfers"]) == (10, 10, 2, 2)
    assert stats["bytes_to_host"] == stats["bytes_to_device"] == 9 * 8192


def test_per_block_copies_are_one_dma_per_block(new_engine):
    engine = new_engine()
    pool = Pool(12, 4096, 2)
    ids = [11, 0, 5, 6]
    host = engine.host_alloc(4 * 4096)
    done(engine, engine.out_per_block(pool.address, 4096, ids, host))
    assert np.array_equal(host_view(host, 4 * 4096), oracle.gather(pool.bytes, 4096, ids))
    done(engine, engine.in_per_block(pool.address, 4096, [1, 2, 3, 4], host))
    for slot, source in zip([1, 2, 3, 4], ids):
        assert np.array_equal(pool.block(slot), host_view(host, 4 * 4096)[ids.index(source) * 4096 :][:4096])
    stats = engine.stats()
    assert stats["memcpys"] == 8 and stats["kernels"] == 0
    engine.host_free(host)


def test_segments_stop_at_65535_blocks(new_engine):
    # 70,000 blocks of 8 bytes fit one 1 MiB staging slot, but a segment holds at most 65,535.
    engine = new_engine(staging_bytes=MIB, ids_capacity=70000)
    pool = Pool(70000, 8, 3)
    ids = np.random.default_rng(3).permutation(70000).tolist()
    host = engine.host_alloc(70000 * 8)
    done(engine, engine.out_gather(pool.address, 8, ids, host))
    assert np.array_equal(host_view(host, 70000 * 8), oracle.gather(pool.bytes, 8, ids))
    assert engine.stats()["kernels"] == 2
    engine.host_free(host)


def test_pool_offsets_past_4_gib(new_engine):
    block = 64 * 1024
    blocks = (5 << 30) // block
    space = mmap.mmap(-1, blocks * block, flags=mmap.MAP_PRIVATE | mmap.MAP_ANONYMOUS)  # pages appear when touched
    try:
        base = ctypes.addressof(ctypes.c_char.from_buffer(space))
        ids = [blocks - 1, 70000, 3]
        rng = np.random.default_rng(4)
        for i in ids:
            np.ctypeslib.as_array((ctypes.c_uint8 * block).from_address(base + i * block))[:] = rng.integers(0, 256, block, dtype=np.uint8)
        expected = b"".join(space[i * block : (i + 1) * block] for i in ids)
        engine = new_engine(staging_bytes=2 * block)
        host = engine.host_alloc(3 * block)
        done(engine, engine.out_gather(base, block, ids, host))
        assert host_view(host, 3 * block).tobytes() == expected
        done(engine, engine.in_scatter(base, block, [blocks - 2, 5, 65536 * 1 + 17], host))
        assert space[(blocks - 2) * block : (blocks - 1) * block] == expected[:block]
        engine.host_free(host)
        del base
    finally:
        try:
            space.close()
        except BufferError:
            pass


@pytest.mark.parametrize("asked,pinned", [(1, MIB), (MIB, MIB), (MIB + 1, MIB + MIB // 4), (40 * MIB, 40 * MIB), (40 * MIB + 1, 48 * MIB),
                                          (3 * MIB, 3 * MIB), (5 * MIB - 1, 5 * MIB)])
def test_pinned_sizes_round_up_by_at_most_a_quarter(new_engine, asked, pinned):
    engine = new_engine()
    pointer = engine.host_alloc(asked)
    assert engine.stats()["host_bytes_live"] == pinned
    engine.host_free(pointer)


def test_a_returned_buffer_serves_the_next_request_of_its_size(new_engine):
    engine = new_engine(host_cache_bytes=16 * MIB)
    first = engine.host_alloc(3 * MIB)
    engine.host_free(first)
    pins = engine.stats()["host_pins"]
    again = engine.host_alloc(3 * MIB - 100)  # same size class
    stats = engine.stats()
    assert again == first and stats["host_pins"] == pins
    assert stats["host_bytes_live"] == 3 * MIB and stats["host_bytes_held"] == 3 * MIB
    other = engine.host_alloc(2 * MIB)
    assert engine.stats()["host_pins"] == pins + 1 and engine.stats()["host_bytes_held"] == 5 * MIB
    engine.host_free(again)
    engine.host_free(other)
    assert engine.stats()["host_bytes_live"] == 0 and engine.stats()["host_bytes_held"] == 5 * MIB


def test_the_cache_evicts_what_came_back_first(new_engine):
    engine = new_engine(host_cache_bytes=6 * MIB)
    a, b, c = engine.host_alloc(2 * MIB), engine.host_alloc(3 * MIB), engine.host_alloc(MIB)
    for pointer in (a, b, c):
        engine.host_free(pointer)  # 6 MiB idle: at the limit
    d = engine.host_alloc(4 * MIB)  # a miss; 10 MiB held until d comes back
    engine.host_free(d)  # room for 4 MiB: a (2) and b (3) go, the oldest first
    assert engine.stats()["host_bytes_held"] == 5 * MIB
    pins = engine.stats()["host_pins"]
    assert engine.host_alloc(MIB) == c and engine.host_alloc(4 * MIB) == d
    assert engine.stats()["host_pins"] == pins
    engine.host_alloc(2 * MIB)  # a was freed: a new pin
    assert engine.stats()["host_pins"] == pins + 1


def test_a_buffer_above_the_cache_limit_goes_back_to_the_system(new_engine):
    engine = new_engine(host_cache_bytes=2 * MIB)
    big = engine.host_alloc(3 * MIB)
    engine.host_free(big)
    assert engine.stats()["host_bytes_held"] == 0


def test_pins_are_timed_and_failures_counted_and_survived(new_engine):
    engine = new_engine(host_cache_bytes=32 * MIB)
    engine.set_pin_limit(engine.stats()["host_bytes_held"] + 8 * MIB + 4 * 64)  # the id ring is pinned too
    kept = engine.host_alloc(3 * MIB)
    engine.host_free(kept)  # idle, 3 MiB
    live = engine.host_alloc(4 * MIB)
    with pytest.raises(HostMemoryError):
        engine.host_alloc(6 * MIB)  # gives the idle 3 MiB back, then still fails
    stats = engine.stats()
    assert stats["host_pin_failures"] == 1 and stats["host_bytes_held"] == 4 * MIB
    assert stats["host_pins"] >= 3 and stats["host_pin_ns"] >= stats["host_pin_max_ns"] > 0
    small = engine.host_alloc(4 * MIB)  # fits once the idle buffer is gone: the engine still works
    for pointer in (live, small):
        engine.host_free(pointer)
    with pytest.raises(NativeError) as refused:
        engine.host_alloc(0)
    assert not isinstance(refused.value, HostMemoryError) and refused.value.status == LT_ERR_INVALID


def test_slow_copies_never_let_a_later_segment_overwrite_staging(new_engine):
    engine = new_engine(staging_bytes=2 * 4096, ids_capacity=64)
    engine.set_copy_delay_us(1500)
    pool = Pool(24, 4096, 5)
    order = np.random.default_rng(5).permutation(24).tolist()
    swap(engine, pool, order[:11], order[11:22])


def test_transfers_in_flight_together_finish_in_any_order(new_engine):
    engine = new_engine(staging_bytes=3 * 4096)
    engine.set_copy_delay_us(300)
    pool = Pool(30, 4096, 6)
    first, second = [4, 19, 2, 27, 8, 13, 0], [21, 5, 16, 9, 29, 1, 11]
    h1, h2 = engine.host_alloc(7 * 4096), engine.host_alloc(7 * 4096)
    t1 = engine.out_gather(pool.address, 4096, first, h1)
    t2 = engine.out_gather(pool.address, 4096, second, h2)
    done(engine, t2)
    done(engine, t1)
    assert np.array_equal(host_view(h1, 7 * 4096), oracle.gather(pool.bytes, 4096, first))
    assert np.array_equal(host_view(h2, 7 * 4096), oracle.gather(pool.bytes, 4096, second))


def test_poll_never_blocks_and_a_paused_transfer_is_not_done(new_engine):
    engine = new_engine()
    pool = Pool(8, 4096, 7)
    host = engine.host_alloc(5 * 4096)
    engine.set_paused(True)
    transfer = engine.out_gather(pool.address, 4096, [7, 1, 3, 0, 2], host)
    assert not engine.poll(transfer) and not engine.poll(transfer)
    with pytest.raises(NativeError) as early:
        engine.release(transfer)  # still in flight
    assert early.value.status == LT_ERR_INVALID
    engine.set_paused(False)
    engine.wait(transfer)
    assert engine.poll(transfer)
    engine.release(transfer)
    with pytest.raises(NativeError):
        engine.release(transfer)  # no longer a live transfer
    assert np.array_equal(host_view(host, 5 * 4096), oracle.gather(pool.bytes, 4096, [7, 1, 3, 0, 2]))


def test_a_full_id_ring_waits_for_the_oldest_transfer(new_engine):
    engine = new_engine(staging_bytes=2 * 4096, ids_capacity=6)
    engine.set_copy_delay_us(500)
    pool = Pool(20, 4096, 8)
    sets = [[0, 5, 9, 13], [2, 7, 11, 17], [19, 3, 6, 1]]
    hosts = [engine.host_alloc(4 * 4096) for _ in sets]
    transfers = [engine.out_gather(pool.address, 4096, ids, host) for ids, host in zip(sets, hosts)]
    for transfer in transfers:
        done(engine, transfer)
    for ids, host in zip(sets, hosts):
        assert np.array_equal(host_view(host, 4 * 4096), oracle.gather(pool.bytes, 4096, ids))
    assert engine.stats()["ids_uploads"] == 3


def _stream_kernels(engine, stream, fn):
    return engine.host_call(stream, fn)


def test_caller_staging_orders_kernels_against_copies(new_engine):
    """The FP8 path's protocol with a stand-in kernel: each segment's 'quantize' fills a slot
    that the previous-but-one segment's copy may still be reading; the copies see every
    segment's own bytes, and the reverse path's kernels see the bytes copied in."""
    engine = new_engine(staging_bytes=4096, num_staging=2)
    engine.set_copy_delay_us(700)
    stream = engine.host_stream()
    stages = [np.zeros(4096, dtype=np.uint8) for _ in range(2)]
    host = engine.host_alloc(6 * 4096)
    keep = []
    for segment in range(6):
        slot = segment % 2
        engine.ext_wait(stream, slot, SLOT_RELEASED)
        keep.append(_stream_kernels(engine, stream, lambda s=stages[slot], v=segment: s.fill(40 + v)))
        engine.ext_record(stream, slot, SLOT_FILLED)
        engine.ext_copy_out(stages[slot].ctypes.data, host + segment * 4096, 4096, slot)
    done(engine, engine.ext_finish(None))
    assert [int(host_view(host + s * 4096, 4096).min()) for s in range(6)] == [40 + s for s in range(6)]
    assert [int(host_view(host + s * 4096, 4096).max()) for s in range(6)] == [40 + s for s in range(6)]
    seen = []
    for segment in range(6):
        slot = segment % 2
        engine.ext_copy_in(stages[slot].ctypes.data, host + segment * 4096, 4096, slot)
        engine.ext_wait(stream, slot, SLOT_FILLED)
        keep.append(_stream_kernels(engine, stream, lambda s=stages[slot]: seen.append((int(s.min()), int(s.max())))))
        engine.ext_record(stream, slot, SLOT_RELEASED)
    done(engine, engine.ext_finish(stream))
    assert seen == [(40 + s, 40 + s) for s in range(6)]


@pytest.mark.parametrize(
    "misuse",
    ["misaligned_pool", "block_over_staging", "more_ids_than_ring", "zero_block_bytes", "null_stream", "slot_out_of_range",
     "unknown_event", "unknown_transfer", "unknown_host_buffer", "zero_copy"],
)
def test_misuse_is_refused_and_the_engine_keeps_working(new_engine, misuse):
    engine = new_engine(staging_bytes=2 * 4096, ids_capacity=8)
    pool = Pool(10, 4096, 9)
    host = engine.host_alloc(9 * 4096)
    calls = {
        "misaligned_pool": lambda: engine.out_gather(pool.address + 4, 4096, [1], host),
        "block_over_staging": lambda: engine.out_gather(pool.address, 3 * 4096, [0], host),
        "more_ids_than_ring": lambda: engine.out_gather(pool.address, 4096, list(range(9)), host),
        "zero_block_bytes": lambda: engine.out_gather(pool.address, 0, [0], host),
        "null_stream": lambda: engine.ext_wait(None, 0, SLOT_FILLED),
        "slot_out_of_range": lambda: engine.ext_record(engine.host_stream(), 2, SLOT_FILLED),
        "unknown_event": lambda: engine.ext_wait(engine.host_stream(), 0, 7),
        "unknown_transfer": lambda: engine.wait(host),
        "unknown_host_buffer": lambda: engine.host_free(host + 64),
        "zero_copy": lambda: engine.ext_copy_out(host, host, 0, 0),
    }
    with pytest.raises(NativeError) as refused:
        calls[misuse]()
    assert refused.value.status == LT_ERR_INVALID, str(refused.value)
    assert engine.stats()["transfers"] == 0
    swap(engine, pool, [3, 8], [0, 1])


@pytest.mark.parametrize("field", ["staging_bytes", "num_staging", "ids_capacity"])
def test_an_engine_needs_positive_sizes(new_engine, field):
    with pytest.raises(NativeError) as refused:
        new_engine(**{field: 0})
    assert refused.value.status == LT_ERR_INVALID


def test_a_failed_kernel_fails_the_engine_for_good(new_engine):
    engine = new_engine()
    stream = engine.host_stream()

    def broken():
        raise RuntimeError("kernel fault")

    keep = engine.host_call(stream, broken)
    with pytest.raises(NativeError) as failed:
        done(engine, engine.ext_finish(stream))
    assert failed.value.status == LT_ERR_DEVICE
    with pytest.raises(NativeError) as later:
        engine.host_alloc(100)
    assert later.value.status == LT_ERR_DEVICE
    del keep


@pytest.mark.parametrize("paused", [False, True], ids=["running", "paused"])
def test_destroy_waits_for_work_in_flight(new_engine, paused):
    engine = new_engine(staging_bytes=2 * 4096)
    engine.set_copy_delay_us(2000)
    pool = Pool(16, 4096, 10)
    host = engine.host_alloc(12 * 4096)
    if paused:
        engine.set_paused(True)
    engine.out_gather(pool.address, 4096, list(range(12)), host)
    engine.destroy()  # returns (no hang), having waited for or discarded the queued work
    assert engine.closed
    engine.destroy()


def test_loading_checks_flavour_and_existence():
    with pytest.raises(NativeUnavailable, match="does not exist"):
        load_library("no-such-flavour")
    with pytest.raises(NativeUnavailable, match="host build"):
        load_library("hip", path=build_host())


def test_sanitized_checks_of_the_c_abi_pass():
    result = subprocess.run(["make", "-s", "-B", "-C", str(CSRC_DIR), "check"], capture_output=True, text=True, timeout=600)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "host_check: ok" in result.stdout
