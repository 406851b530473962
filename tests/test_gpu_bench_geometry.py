"""GPU parity at the benchmark's own geometries (4 and 5).

The other decode tests run small batches, where the split size is always 64 blocks. Here the
launches are the ones bench.py times:

- config 3: batch 32, 32 query / 8 KV heads, lengths uniform in [1,024, 32,768], a Qwen3-4B
  pool whose block offsets pass 32 bits; 128-block splits. A batch of 64 with 32,768-token
  rows reaches 256-block splits (lanes 16-63 of each wave then hold block ids).
- config 4: the same kernel over FP8 records (576 groups per block, 0.1% outliers at +/-40):
  batch 1 at 32,768, batch 64 at 4,096 and batch 32 mixed, against the oracle run on the
  dequantized pool.
- the fused token write (lk_paged_decode_append) at 64- to 256-block splits and with more
  than 64 splits at 8 KV heads, BF16 and FP8, against the two-launch sequence and the oracle.
- config 5: decode steps computed while 2,048 blocks swap out as FP8 records and back in equal
  the same steps computed alone, bit for bit; every swapped record equals the oracle's quantize
  and every restored block its dequantize.
- config 2: the 512-block FP8 swap of the 12 GiB pool through two 128 MiB slots, every record
  and every restored block against the oracle.
- the paged prefill's three bench chunks (2,048 tokens at 0, where heavy tiles divide within
  CU pairs; 2,048 ending a 32,768 context; 512 at 8,192 with split keys), BF16 and FP8
  pools, against the oracle on sampled tokens.
- a seeded randomized sweep of shapes, lengths, gains and dtypes, after the reference's
  property test (tests/test_triton_decode.py:335-353), and the reference's Qwen3-4B-shape
  case at layers 0, 17 and 35 (tests/test_triton_decode.py:649-684).

Oracle inputs are copied off the GPU one layer at a time; the float64 oracle runs over row
slices in threads (its ctypes calls release the GIL).
"""

import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

LAYERS, KV_HEADS, SLOTS, DIM, QUERY_HEADS = 36, 8, 16, 128, 32
GROUPS = QUERY_HEADS // KV_HEADS
GROUP_ELEMS, GROUPS_PER_BLOCK = SLOTS * DIM, 2 * LAYERS * KV_HEADS
POOL_BLOCKS = 2112  # 4.98 GB of BF16: past 32-bit byte offsets, room for 2,048-block rows
ORACLE_THREADS = 12


def log(message):
    print(message, flush=True)


def bf16_pool(blocks, seed, layers=LAYERS, outliers=0.0, chunk=128):
    """N(0,1) BF16 pool on the GPU, drawn in block slices; a fraction `outliers` of the
    elements set to +/-40 (signs and positions seeded), as bench.py fills config 2."""
    gen = torch.Generator(device="cuda").manual_seed(seed)
    pool = torch.empty(blocks, 2, layers, KV_HEADS, SLOTS, DIM, dtype=torch.bfloat16, device="cuda")
    for at in range(0, blocks, chunk):
        piece = pool[at : at + chunk]
        piece.copy_(torch.randn(piece.shape, generator=gen, device="cuda"))
        if outliers:
            mask = torch.rand(piece.shape, generator=gen, device="cuda") < outliers
            signs = torch.where(torch.rand(piece.shape, generator=gen, device="cuda") < 0.5, -40.0, 40.0)
            piece[mask] = signs[mask].to(torch.bfloat16)
    return pool


def layer_bits(pool, layer):
    """One layer of a BF16 pool as host bits, shaped as a one-layer pool for the oracle."""
    return pool[:, :, layer : layer + 1].contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def oracle_decode(q_bits, pool_layer_bits, table, lengths, groups=GROUPS):
    rows = [r for r in np.array_split(np.arange(len(lengths)), ORACLE_THREADS) if len(r)]
    with ThreadPoolExecutor(len(rows)) as pool:
        parts = pool.map(lambda r: oracle.decode_attention(q_bits[r], pool_layer_bits, 0, table[r], lengths[r], groups), rows)
        return np.concatenate(list(parts))


def weight_rounding(q_bits, pool_layer_bits, table, lengths):
    """The attention-weighted mean |v|: the FP8 kernel feeds the weights to the matrix cores
    as single BF16s (relative error at most 2^-8), so it may err by 2^-8 of this."""
    magnitudes = pool_layer_bits.copy()
    magnitudes[:, 1] &= 0x7FFF
    return oracle_decode(q_bits, magnitudes, table, lengths)


def assert_close(out, expected, what, rounding=None):
    got = out.double().cpu().numpy()
    allowed = np.abs(expected) * 2.0**-8 + 1e-3
    if rounding is not None:
        allowed = allowed + 2.0**-8 * rounding
    error = np.abs(got - expected)
    assert np.isfinite(got).all(), what
    assert (error <= allowed).all(), f"{what}: max error {error.max():.3g} at {np.unravel_index(error.argmax(), error.shape)}"
    assert (error <= 2e-2 + 1e-2 * np.abs(expected)).all(), what


def tables_for(rng, lengths, pool_blocks, reserved_last=None):
    """Rows of random blocks, each row without repeats (rows alias one another, as in the
    bench's 12 GiB pool). reserved_last: ids given to each row's last block, one per row, and
    used nowhere else, so that rows write distinct blocks."""
    width = max(-(-int(n) // SLOTS) for n in lengths)
    table = np.zeros((len(lengths), width), dtype=np.int32)
    body = pool_blocks if reserved_last is None else pool_blocks - len(lengths)
    for b, n in enumerate(lengths):
        need = -(-int(n) // SLOTS)
        table[b, :need] = rng.choice(body, need, replace=False)
        if reserved_last is not None:
            table[b, need - 1] = reserved_last[b]
    return table


def splits_of(hip_decode, q, pool, table, lengths):
    from layover_amd.kernels import _lib

    shape = hip_decode.decode_shape(q, pool, 0, table, GROUPS, lengths)
    need = int(_lib.load().lk_paged_decode_workspace(shape))
    return need // (q.shape[0] * QUERY_HEADS * (DIM + 2) * 4)


def q_for(batch, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(batch, QUERY_HEADS, DIM, generator=gen, device="cuda").to(torch.bfloat16)


def q_host_bits(q):
    return q.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.fixture(scope="module")
def hip_decode():
    from layover_amd.kernels import hip_decode as module

    return module


@pytest.fixture(scope="module")
def pools(hip_decode):
    """The module's pools: BF16 with outliers, its FP8 records, and the records dequantized."""
    from layover_amd.kernels import fp8

    log(f"bench-geometry pools: {POOL_BLOCKS} Qwen3-4B blocks")
    pool = bf16_pool(POOL_BLOCKS, seed=3, outliers=1e-3)
    layout = fp8.Fp8Layout(GROUP_ELEMS, GROUPS_PER_BLOCK)
    ids = torch.arange(POOL_BLOCKS, dtype=torch.int32, device="cuda")
    records = torch.empty(POOL_BLOCKS, layout.record_bytes, dtype=torch.uint8, device="cuda")
    fp8.quantize_blocks(pool, ids, records.view(-1), layout)
    dequantized = torch.empty_like(pool)
    fp8.dequantize_blocks(records.view(-1), ids, dequantized, layout)
    torch.cuda.synchronize()
    # The GPU codec is checked exhaustively elsewhere; here a sample of these very blocks is
    # checked against the oracle's records and dequantization.
    sample = [0, 1, 977, POOL_BLOCKS - 1]
    bits = pool[sample].view(torch.int16).cpu().numpy().view(np.uint16)
    expected = oracle.quantize_records(bits, range(len(sample)), GROUP_ELEMS, GROUPS_PER_BLOCK)
    assert np.array_equal(records[sample].cpu().numpy().reshape(-1), expected)
    restored = np.zeros_like(bits)
    oracle.dequantize_records(expected, range(len(sample)), restored, GROUP_ELEMS, GROUPS_PER_BLOCK)
    assert np.array_equal(dequantized[sample].view(torch.int16).cpu().numpy().view(np.uint16), restored)
    kv = hip_decode.Fp8KVPool(records, LAYERS, KV_HEADS, SLOTS, DIM)
    yield {"bf16": pool, "fp8": kv, "dequantized": dequantized}
    del pool, records, dequantized, kv
    torch.cuda.empty_cache()


def run_case(hip_decode, pools, kind, lengths, seed, layers, expect_splits=None):
    rng = np.random.default_rng(seed)
    table = tables_for(rng, lengths, POOL_BLOCKS)
    lens = np.array(lengths, dtype=np.int32)
    q = q_for(len(lengths), seed)
    table_gpu, lens_gpu = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    target = pools["fp8"] if kind == "fp8" else pools["bf16"]
    values = pools["dequantized"] if kind == "fp8" else pools["bf16"]
    splits = splits_of(hip_decode, q, target, table_gpu, lens_gpu)
    if expect_splits is not None:
        assert splits == expect_splits
    qb = q_host_bits(q)
    for layer in layers:
        log(f"{kind} decode batch {len(lengths)} width {table.shape[1]} splits {splits} layer {layer}")
        out = hip_decode.paged_decode_attention_hip(q, target, layer, table_gpu, lens_gpu, GROUPS)
        host = layer_bits(values, layer)
        expected = oracle_decode(qb, host, table, lens)
        rounding = weight_rounding(qb, host, table, lens) if kind == "fp8" else None
        assert_close(out, expected, f"{kind} batch {len(lengths)} layer {layer}", rounding)


def mixed_lengths(seed, batch):
    return [int(n) for n in np.random.default_rng(seed).integers(1024, 32769, size=batch)]


def test_config3_bf16_batch32_mixed_contexts(hip_decode, pools):
    lengths = mixed_lengths(11, 32)
    lengths[0] = 32768  # the full 2,048-block width, as the bench's draw nearly reaches
    run_case(hip_decode, pools, "bf16", lengths, seed=11, layers=(0, 35), expect_splits=16)


def test_bf16_batch64_long_rows_take_256_block_splits(hip_decode, pools):
    lengths = mixed_lengths(12, 64)
    lengths[5] = 32768
    run_case(hip_decode, pools, "bf16", lengths, seed=12, layers=(17,), expect_splits=8)


@pytest.mark.parametrize(
    "case",
    ["batch1_32768", "batch64_4096", "batch32_mixed"],
)
def test_config4_fp8_records_match_the_oracle_on_the_dequantized_pool(hip_decode, pools, case):
    lengths = {"batch1_32768": [32768], "batch64_4096": [4096] * 64}.get(case)
    if lengths is None:
        lengths = mixed_lengths(13, 32)
        lengths[3] = 32768
    splits = {"batch1_32768": 32, "batch64_4096": 4, "batch32_mixed": 32}[case]
    run_case(hip_decode, pools, "fp8", lengths, seed=len(case), layers=(0, 35), expect_splits=splits)


# (FP8 records?, batch): the split count the plan gives, 2,048 // blocks per split. FP8 records
# aim at twice the workgroups, so their 256-block splits need batch 128.
LONG_SPLITS = {(False, 32): 16, (False, 64): 8, (True, 32): 32, (True, 64): 16, (True, 128): 8}


@pytest.mark.parametrize("fp8,batch", list(LONG_SPLITS), ids=lambda v: str(v))
def test_fused_write_at_long_splits_equals_two_launches_and_the_oracle(hip_decode, pools, fp8, batch):
    """lk_paged_decode_append at long splits: 128- and 256-block splits on the BF16 pool (batch
    32, 64), 64-, 128- and 256-block splits on FP8 records (batch 32, 64, 128). Each row
    writes one new token at its last position, into a block no other row holds. Pool bytes
    and outputs equal write-then-decode launched separately, and outputs match the oracle on
    the written pool."""
    rng = np.random.default_rng(20 + batch)
    # Rows up to the full 2,048-block width, or as long as the pool allows once every row has
    # a last block of its own (batch 128 leaves 1,984 blocks); row 1 the longest.
    cap = min(32768, (POOL_BLOCKS - batch) * SLOTS)
    lengths = [min(n, cap) for n in mixed_lengths(20 + batch, batch)]
    lengths[1] = cap
    last = np.arange(POOL_BLOCKS - batch, POOL_BLOCKS)
    table = tables_for(rng, lengths, POOL_BLOCKS, reserved_last=last)
    lens = np.array(lengths, dtype=np.int32)
    write_blocks = torch.from_numpy(last.astype(np.int32)).cuda()
    write_slots = torch.from_numpy(((lens - 1) % SLOTS).astype(np.int32)).cuda()
    table_gpu, lens_gpu = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    q = q_for(batch, 30 + batch)
    gen = torch.Generator(device="cuda").manual_seed(40 + batch)
    k = (torch.randn(batch, KV_HEADS, DIM, generator=gen, device="cuda") * 3).to(torch.bfloat16)
    v = torch.randn(batch, KV_HEADS, DIM, generator=gen, device="cuda").to(torch.bfloat16)
    layer = 35
    if fp8:
        fused_pool = hip_decode.Fp8KVPool(pools["fp8"].records.clone(), LAYERS, KV_HEADS, SLOTS, DIM)
        split_pool = hip_decode.Fp8KVPool(pools["fp8"].records.clone(), LAYERS, KV_HEADS, SLOTS, DIM)
    else:
        fused_pool, split_pool = pools["bf16"].clone(), pools["bf16"].clone()
    splits = splits_of(hip_decode, q, fused_pool, table_gpu, lens_gpu)
    assert splits == LONG_SPLITS[(fp8, batch)]
    log(f"fused write+decode fp8={fp8} batch {batch} splits {splits}")
    fused, separate = torch.empty_like(q), torch.empty_like(q)
    hip_decode.run_kernel_append(q, fused_pool, layer, table_gpu, lens_gpu, GROUPS, write_blocks, write_slots, k, v, fused)
    if fp8:
        split_pool.write(write_blocks, write_slots, layer, k, v)
    else:
        hip_decode.write_tokens(split_pool, write_blocks, write_slots, layer, k, v)
    hip_decode.run_kernel(q, split_pool, layer, table_gpu, lens_gpu, GROUPS, separate)
    torch.cuda.synchronize()
    if fp8:
        assert torch.equal(fused_pool.records, split_pool.records)
        from layover_amd.kernels import fp8 as codec

        layout = codec.Fp8Layout(GROUP_ELEMS, GROUPS_PER_BLOCK)
        values = torch.empty_like(pools["bf16"])
        codec.dequantize_blocks(fused_pool.records.view(-1), torch.arange(POOL_BLOCKS, dtype=torch.int32, device="cuda"), values, layout)
        del split_pool
    else:
        assert torch.equal(fused_pool.view(torch.int16), split_pool.view(torch.int16))
        values = fused_pool
        del split_pool
    assert torch.equal(fused.view(torch.int16), separate.view(torch.int16))
    qb = q_host_bits(q)
    host = layer_bits(values, layer)
    expected = oracle_decode(qb, host, table, lens)
    rounding = weight_rounding(qb, host, table, lens) if fp8 else None
    assert_close(fused, expected, f"fused fp8={fp8} batch {batch}", rounding)
    del fused_pool, values
    torch.cuda.empty_cache()


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16_pool", "fp8_pool"])
def test_fused_write_with_65_to_128_splits_at_8_kv_heads(hip_decode, fp8):
    """A 66,560-token row at 8 KV heads: 65 splits of 64 blocks, so the merge takes its second
    batch of row loads, with the fused write in the last split."""
    from layover_amd.kernels import fp8 as codec

    layers, blocks = 2, 4400
    pool = bf16_pool(blocks, seed=50, layers=layers)
    rng = np.random.default_rng(50)
    lengths = [66560, 3000, 17]
    width = -(-lengths[0] // SLOTS)
    table = np.zeros((3, width), dtype=np.int32)
    ids = rng.permutation(blocks)
    at = 0
    for b, n in enumerate(lengths):
        need = -(-n // SLOTS)
        table[b, :need] = ids[at : at + need]
        at += need
    lens = np.array(lengths, dtype=np.int32)
    last = np.array([table[b, -(-n // SLOTS) - 1] for b, n in enumerate(lengths)], dtype=np.int32)
    q = q_for(3, 51)
    gen = torch.Generator(device="cuda").manual_seed(52)
    k = torch.randn(3, KV_HEADS, DIM, generator=gen, device="cuda").to(torch.bfloat16)
    v = torch.randn(3, KV_HEADS, DIM, generator=gen, device="cuda").to(torch.bfloat16)
    table_gpu, lens_gpu = torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda()
    write_blocks = torch.from_numpy(last).cuda()
    write_slots = torch.from_numpy(((lens - 1) % SLOTS).astype(np.int32)).cuda()
    if fp8:
        layout = codec.Fp8Layout(GROUP_ELEMS, 2 * layers * KV_HEADS)
        records = torch.empty(blocks, layout.record_bytes, dtype=torch.uint8, device="cuda")
        codec.quantize_blocks(pool, torch.arange(blocks, dtype=torch.int32, device="cuda"), records.view(-1), layout)
        fused_pool = hip_decode.Fp8KVPool(records, layers, KV_HEADS, SLOTS, DIM)
        split_pool = hip_decode.Fp8KVPool(records.clone(), layers, KV_HEADS, SLOTS, DIM)
    else:
        fused_pool, split_pool = pool, pool.clone()
    assert splits_of(hip_decode, q, fused_pool, table_gpu, lens_gpu) == 65
    log(f"fused write+decode 65 splits fp8={fp8}")
    fused, separate = torch.empty_like(q), torch.empty_like(q)
    hip_decode.run_kernel_append(q, fused_pool, 1, table_gpu, lens_gpu, GROUPS, write_blocks, write_slots, k, v, fused)
    if fp8:
        split_pool.write(write_blocks, write_slots, 1, k, v)
    else:
        hip_decode.write_tokens(split_pool, write_blocks, write_slots, 1, k, v)
    hip_decode.run_kernel(q, split_pool, 1, table_gpu, lens_gpu, GROUPS, separate)
    torch.cuda.synchronize()
    if fp8:
        assert torch.equal(fused_pool.records, split_pool.records)
        values = torch.empty_like(pool)
        codec.dequantize_blocks(fused_pool.records.view(-1), torch.arange(blocks, dtype=torch.int32, device="cuda"), values, layout)
    else:
        assert torch.equal(fused_pool.view(torch.int16), split_pool.view(torch.int16))
        values = fused_pool
    assert torch.equal(fused.view(torch.int16), separate.view(torch.int16))
    qb = q_host_bits(q)
    host = layer_bits(values, 1)
    expected = oracle_decode(qb, host, table, lens)
    rounding = weight_rounding(qb, host, table, lens) if fp8 else None
    assert_close(fused, expected, f"65 splits fp8={fp8}", rounding)


def assert_swap_matches_the_oracle(pool, src, dst, payload, layout, chunk=128):
    """Every record of a swap-out payload (host bytes, records in src order) against the
    oracle's quantize of the source blocks, and every restored block (pool[dst]) against the
    oracle's dequantize of those records, chunk by chunk, the oracle split over threads."""
    record = layout.record_bytes
    for start in range(0, len(src), chunk):
        ids = src[start : start + chunk]
        bits = pool[ids].view(torch.int16).cpu().numpy().view(np.uint16)
        parts = [part for part in np.array_split(np.arange(len(ids)), ORACLE_THREADS) if len(part)]

        def leg(part):
            local = np.ascontiguousarray(bits[part])
            local_ids = np.arange(len(part), dtype=np.int32)
            records = oracle.quantize_records(local, local_ids, layout.group_elems, layout.groups_per_block)
            restored = np.zeros_like(local)
            oracle.dequantize_records(records, local_ids, restored, layout.group_elems, layout.groups_per_block)
            return records, restored

        with ThreadPoolExecutor(len(parts)) as workers:
            legs = list(workers.map(leg, parts))
        records = np.concatenate([r for r, _ in legs])
        restored = np.concatenate([b for _, b in legs])
        got = payload[start * record : (start + len(ids)) * record]
        if not np.array_equal(got, records):
            bad = np.flatnonzero(got != records)[0]
            raise AssertionError(f"record {start + bad // record} (block {ids[bad // record]}) differs from the oracle at byte {bad % record}")
        back = pool[dst[start : start + len(ids)]].view(torch.int16).cpu().numpy().view(np.uint16)
        assert np.array_equal(back, restored), f"restored blocks {start}..{start + len(ids)} differ from the oracle's dequantize"


def test_config2_swap_of_512_blocks_equals_the_oracle_record_for_record():
    """BASELINE config 2 exactly: a 12 GiB Qwen3-4B pool (5,461 blocks) of N(0,1) BF16 with
    0.1% of the elements at +/-40, 512 random non-contiguous blocks swapped out as FP8 records
    through two 128 MiB staging slots (113 records each, so 5 segments) into pinned host
    memory, then swapped in to 512 fresh random ids. All 512 records equal the oracle's
    quantize of the source blocks, all 512 restored blocks equal the oracle's dequantize, and
    every other block of the pool is unchanged (reference tests/test_fp8.py:264-278,
    tests/test_transfer.py:546-569)."""
    from layover_amd.config import ModelConfig
    from layover_amd.kernels import fp8 as codec
    from layover_amd.kv.paged_cache import PagedKVCache
    from layover_amd.kv.transfer import NativeBackend

    config = ModelConfig.qwen3_4b()
    block_bytes = 2 * LAYERS * KV_HEADS * SLOTS * DIM * 2
    blocks = (12 << 30) // block_bytes
    assert blocks == 5461
    cache = PagedKVCache(config, blocks, device="cuda", fill=False)
    cache.pool.copy_(bf16_pool(blocks, seed=0, outliers=1e-3))
    before = cache.pool.clone()
    rng = np.random.default_rng(20)
    picked = rng.permutation(blocks)
    src, dst = [int(i) for i in picked[:512]], [int(i) for i in picked[512:1024]]
    layout = codec.Fp8Layout(GROUP_ELEMS, GROUPS_PER_BLOCK)
    backend = NativeBackend("cuda", staging_bytes=128 << 20, num_staging=2, ids_capacity=1 << 20)
    try:
        log("config 2: 512-block FP8 swap-out")
        out_ticket = backend.start_out(cache, src, fp8=True)
        out_ticket.wait()
        payload = out_ticket.payload
        host = payload.memory.numpy()[: 512 * layout.record_bytes].copy()
        log("config 2: swap-in to 512 fresh ids")
        backend.start_in(cache, dst, payload).wait()
        torch.cuda.synchronize()
        backend.free(payload)
    finally:
        backend.close()
    log("config 2: all records and restored blocks against the oracle")
    assert_swap_matches_the_oracle(cache.pool, src, dst, host, layout)
    untouched = torch.ones(blocks, dtype=torch.bool, device="cuda")
    untouched[torch.tensor(dst, device="cuda")] = False
    assert torch.equal(cache.pool[untouched].view(torch.int16), before[untouched].view(torch.int16))
    del cache, before
    torch.cuda.empty_cache()


def test_config5_decode_during_a_2048_block_fp8_swap_equals_decode_alone(hip_decode):
    """Config 5's overlap: batch-32 decode steps (36 layers each, mixed 1k-32k contexts) on
    torch's stream while 2,048 blocks swap out to pinned host memory as FP8 records on the
    backend's streams, then back in to fresh ids. Every overlapped step's outputs equal the
    solo step's bit for bit; the payload equals a quiet quantize of the same blocks and, all
    2,048 records, the oracle's quantize; the restored blocks equal a quiet dequantize and the
    oracle's dequantize; and no block outside the targets changes."""
    from layover_amd.config import ModelConfig
    from layover_amd.kernels import fp8 as codec
    from layover_amd.kv.paged_cache import PagedKVCache
    from layover_amd.kv.transfer import NativeBackend

    swap_blocks, decode_region = 2048, 2112
    blocks = decode_region + swap_blocks
    cache = PagedKVCache(ModelConfig.qwen3_4b(), blocks, device="cuda", fill=False)
    cache.pool.copy_(bf16_pool(blocks, seed=60, outliers=1e-3))
    rng = np.random.default_rng(60)
    lengths = mixed_lengths(60, 32)
    table = torch.from_numpy(tables_for(rng, lengths, decode_region)).cuda()
    lens = torch.tensor(lengths, dtype=torch.int32, device="cuda")
    q = q_for(32, 61)
    outs = torch.empty(LAYERS, *q.shape, dtype=q.dtype, device="cuda")

    def step():
        for layer in range(LAYERS):
            hip_decode.run_kernel(q, cache.pool, layer, table, lens, GROUPS, outs[layer])
        return outs.clone()

    solo = step()
    torch.cuda.synchronize()
    src = [int(i) for i in rng.choice(decode_region, swap_blocks, replace=False)]
    dst = list(range(decode_region, blocks))
    layout = codec.Fp8Layout(GROUP_ELEMS, GROUPS_PER_BLOCK)
    quiet = torch.empty(swap_blocks * layout.record_bytes, dtype=torch.uint8, device="cuda")
    codec.quantize_blocks(cache.pool, torch.tensor(src, dtype=torch.int32, device="cuda"), quiet, layout)
    expected_pool = cache.pool.clone()
    codec.dequantize_blocks(quiet, torch.tensor(dst, dtype=torch.int32, device="cuda"), expected_pool, layout)
    torch.cuda.synchronize()

    backend = NativeBackend("cuda", staging_bytes=128 << 20, num_staging=2, ids_capacity=1 << 20)
    try:
        backend.prepare(cache, fp8=True)
        overlapped = []

        def during(start):
            """Keep two decode steps queued while the transfer runs (at least one step)."""
            ticket = start()
            pending = []
            while not ticket.done() or not pending:
                pending = [e for e in pending if not e.query()]
                if len(pending) < 2 and len(overlapped) < 400:
                    overlapped.append(step())
                    event = torch.cuda.Event()
                    event.record()
                    pending.append(event)
                else:
                    time.sleep(0.0002)
            ticket.wait()
            return ticket

        log("config 5: swap-out with decode steps beside it")
        out_ticket = during(lambda: backend.start_out(cache, src, fp8=True))
        payload = out_ticket.payload
        host = payload.memory.numpy()[: swap_blocks * layout.record_bytes]
        log("config 5: swap-in with decode steps beside it")
        in_ticket = during(lambda: backend.start_in(cache, dst, payload))
        torch.cuda.synchronize()
        log(f"config 5: {len(overlapped)} decode steps overlapped the swap")
        assert np.array_equal(host, quiet.cpu().numpy())
        assert torch.equal(cache.pool.view(torch.int16), expected_pool.view(torch.int16))
        log("config 5: all 2,048 swapped records and restored blocks against the oracle")
        assert_swap_matches_the_oracle(cache.pool, src, dst, host, layout)
        for i, got in enumerate(overlapped):
            assert torch.equal(got.view(torch.int16), solo.view(torch.int16)), f"overlapped step {i} differs from the solo step"
        assert in_ticket.done()
        backend.free(payload)
    finally:
        backend.close()
    # The solo step itself against the oracle, at one layer.
    qb = q_host_bits(q)
    expected = oracle_decode(qb, layer_bits(cache.pool, 20), table.cpu().numpy(), lens.cpu().numpy())
    assert_close(solo[20], expected, "config 5 solo step, layer 20")
    del cache, expected_pool, quiet
    torch.cuda.empty_cache()


def test_qwen3_4b_shape_at_layers_0_17_35(hip_decode):
    """The reference's Qwen3-4B-shape case: 2,048 blocks (offsets past 32 bits), each sequence
    on its own blocks with the pool's last block among them, short rows padded with block 0."""
    pool = bf16_pool(2048, seed=70)
    assert pool.numel() > 2**31
    lengths = [1, 16, 17, 255, 256, 1024, 4000, 8192]
    need = [-(-n // SLOTS) for n in lengths]
    rng = np.random.default_rng(70)
    ids = rng.permutation(2047)[: sum(need)]
    ids[0] = 2047
    table = np.zeros((len(lengths), max(need)), dtype=np.int32)
    at = 0
    for b, n in enumerate(need):
        table[b, :n] = ids[at : at + n]
        at += n
    lens = np.array(lengths, dtype=np.int32)
    q = q_for(len(lengths), 71)
    qb = q_host_bits(q)
    for layer in (0, 17, 35):
        out = hip_decode.paged_decode_attention_hip(q, pool, layer, torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), GROUPS)
        assert out.dtype == q.dtype and out.device == q.device
        assert_close(out, oracle_decode(qb, layer_bits(pool, layer), table, lens), f"qwen3-4b layer {layer}")
    del pool
    torch.cuda.empty_cache()


def sweep_cases(count=60, seed=2024):
    """Seeded draws over the reference property test's space (test_triton_decode.py:337-347),
    plus the Qwen tile shape (head_dim 128, 16 slots) that takes the matrix-core kernel."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(count):
        qwen_tile = i % 3 == 0
        cases.append(
            dict(
                seed=int(rng.integers(0, 2**16)),
                kv_heads=int(rng.choice([1, 2, 3])),
                groups=int(rng.choice([1, 2, 4])),
                head_dim=128 if qwen_tile else int(rng.choice([8, 16, 24, 31, 32])),
                slots=16 if qwen_tile else int(rng.choice([4, 7, 16])),
                layer=int(rng.integers(0, 3)),
                gain=float(rng.choice([0.1, 1.0, 8.0])),
                dtype=str(rng.choice(["float32", "bfloat16"])),
                lengths=[int(n) for n in rng.integers(1, 71, size=int(rng.integers(1, 5)))],
            )
        )
    return cases


@pytest.mark.parametrize("case", sweep_cases(), ids=lambda c: f"s{c['seed']}")
def test_randomized_shapes_match_the_oracle(hip_decode, case):
    rng = np.random.default_rng(case["seed"])
    kv_heads, groups, dim, slots = case["kv_heads"], case["groups"], case["head_dim"], case["slots"]
    lengths = case["lengths"]
    width = max(-(-n // slots) for n in lengths)
    blocks = len(lengths) * width + 2
    pool = oracle.bf16_bits(rng.standard_normal((blocks, 2, 3, kv_heads, slots, dim), dtype=np.float32))
    table = rng.permutation(blocks)[: len(lengths) * width].reshape(len(lengths), width).astype(np.int32)
    q = oracle.bf16_bits((case["gain"] * rng.standard_normal((len(lengths), kv_heads * groups, dim))).astype(np.float32))
    lens = np.array(lengths, dtype=np.int32)
    dtype = getattr(torch, case["dtype"])
    q_gpu = torch.from_numpy(q.view(np.int16)).cuda().view(torch.bfloat16).to(dtype)
    pool_gpu = torch.from_numpy(pool.view(np.int16)).cuda().view(torch.bfloat16).to(dtype)
    out = hip_decode.paged_decode_attention_hip(q_gpu, pool_gpu, case["layer"], torch.from_numpy(table).cuda(), torch.from_numpy(lens).cuda(), groups)
    assert out.dtype == dtype and torch.isfinite(out.float()).all()
    expected = oracle.decode_attention(q, pool, case["layer"], table, lens, groups)
    if dtype == torch.float32:
        error = np.abs(out.double().cpu().numpy() - expected)
        assert error.max() < 1e-4 * max(1.0, np.abs(expected).max()), (case, error.max())
    else:
        assert_close(out, expected, str(case))


PREFILL_SAMPLES = {
    # (start, tokens): sampled tokens. At position 0 tiles of 32 tokens (128 rows) pair up on
    # a CU, and tiles 44-63 (tokens 1,408-2,047) divide their key steps with their partners.
    (0, 2048): [0, 1, 15, 16, 31, 32, 33, 500, 1023, 1024, 1407, 1408, 1439, 1600, 1800, 2000, 2015, 2016, 2046, 2047],
    (30720, 2048): [0, 1, 127, 128, 1000, 2047],
    (8192, 512): [0, 1, 255, 256, 511],
}


@pytest.mark.parametrize("kind", ["bf16", "fp8"])
@pytest.mark.parametrize("start,tokens", list(PREFILL_SAMPLES), ids=lambda v: str(v))
def test_prefill_at_the_bench_geometry_matches_the_oracle_on_sampled_tokens(hip_decode, pools, kind, start, tokens):
    """bench.py's three prefill chunks (2,048 tokens at 0 and ending a 32,768 context, 512 at
    8,192 with its keys split) over the 36-layer Qwen3-4B pool with 0.1% outliers, BF16 and
    FP8 records (staged as BF16, against the oracle on the dequantized pool): sampled tokens,
    each one decode row of the float64 oracle (query t sees start + t + 1 keys)."""
    from layover_amd.kernels.hip_prefill import paged_prefill_attention_hip

    layer = 17
    end = start + tokens
    used = -(-end // SLOTS)
    rng = np.random.default_rng(start + tokens)
    block_ids = rng.choice(POOL_BLOCKS, used, replace=False).astype(np.int32)
    gen = torch.Generator(device="cuda").manual_seed(tokens)
    q = torch.randn(QUERY_HEADS, tokens, DIM, generator=gen, device="cuda").to(torch.bfloat16)
    log(f"bench-geometry prefill {kind} start={start} tokens={tokens}")
    pool = pools["bf16"] if kind == "bf16" else pools["fp8"]
    out = paged_prefill_attention_hip(q, pool, layer, torch.from_numpy(block_ids).cuda(), start, GROUPS)
    torch.cuda.synchronize()
    sample = PREFILL_SAMPLES[(start, tokens)]
    q_bits = q[:, sample].permute(1, 0, 2).contiguous().view(torch.int16).cpu().numpy().view(np.uint16)
    reference_pool = layer_bits(pools["bf16" if kind == "bf16" else "dequantized"], layer)
    table = np.repeat(block_ids[None], len(sample), axis=0)
    lengths = np.array([start + t + 1 for t in sample], dtype=np.int32)
    expected = oracle_decode(q_bits, reference_pool, table, lengths)
    rounding = weight_rounding(q_bits, reference_pool, table, lengths)
    assert_close(out[:, sample].permute(1, 0, 2), expected, f"prefill {kind} {start}+{tokens}", rounding=np.abs(rounding))
