"""CPU side of the decode-step data path: the oracle's FP8 append (pinned against the record
quantizer, which test_oracle.py pins against the reference's codec) and the bookkeeping of
DecodeAttentionGraphs (reference layover/decode_graphs.py: sizes, padding rows on a reserved
scratch block, fixed table width). Replays themselves run in tests/test_gpu_graphs.py."""

import math

import numpy as np
import pytest
import torch

from layover_amd.config import ModelConfig
from layover_amd.kv.decode_graphs import DecodeAttentionGraphs
from layover_amd.kv.paged_cache import BlockTable, PagedKVCache
from oracle import oracle

LAYERS, HEADS, SLOTS, DIM = 2, 2, 16, 24
GROUP, GROUPS = SLOTS * DIM, 2 * LAYERS * HEADS


def quantized_blocks(blocks, seed):
    bits = oracle.bf16_bits(np.random.default_rng(seed).standard_normal((blocks, 2, LAYERS, HEADS, SLOTS, DIM), dtype=np.float32))
    return bits, oracle.quantize_records(bits, list(range(blocks)), GROUP, GROUPS).reshape(blocks, -1)


def tokens(rows, seed, scale=1.0):
    return oracle.bf16_bits(np.random.default_rng(seed).standard_normal((rows, HEADS, DIM), dtype=np.float32) * scale)


def test_append_into_an_empty_block_quantizes_just_that_token():
    records = np.zeros((1, GROUP * GROUPS + 2 * GROUPS), dtype=np.uint8)
    k, v = tokens(1, 1, 9.0), tokens(1, 2, 0.01)
    got = oracle.append_tokens(records, LAYERS, HEADS, SLOTS, DIM, [0], [0], 1, k, v)
    block = np.zeros((1, 2, LAYERS, HEADS, SLOTS, DIM), dtype=np.uint16)
    block[0, 0, 1, :, 0], block[0, 1, 1, :, 0] = k[0], v[0]
    assert np.array_equal(got[0], oracle.quantize_records(block, [0], GROUP, GROUPS))


def test_append_that_keeps_every_shift_leaves_earlier_codes_and_other_layers_alone():
    _, records = quantized_blocks(3, 3)
    k, v = tokens(1, 4, 0.5), tokens(1, 5, 0.5)  # small: cannot raise a group's largest exponent
    got = oracle.append_tokens(records, LAYERS, HEADS, SLOTS, DIM, [2], [9], 0, k, v)
    assert np.array_equal(got[:2], records[:2])
    block_elems = GROUP * GROUPS
    for kind in (0, 1):
        for head in range(HEADS):
            g = (kind * LAYERS + 0) * HEADS + head
            codes, old = got[2, g * GROUP : (g + 1) * GROUP], records[2, g * GROUP : (g + 1) * GROUP]
            assert np.array_equal(codes[: 9 * DIM], old[: 9 * DIM])  # earlier slots: same codes
            assert not codes[10 * DIM :].any()  # later slots: zero
            assert np.array_equal(got[2, block_elems + 2 * g : block_elems + 2 * g + 2], records[2, block_elems + 2 * g : block_elems + 2 * g + 2])
    untouched = [g for g in range(GROUPS) if (g // HEADS) % LAYERS != 0]
    for g in untouched:
        assert np.array_equal(got[2, g * GROUP : (g + 1) * GROUP], records[2, g * GROUP : (g + 1) * GROUP])


def test_append_that_raises_the_largest_exponent_requantizes_the_group():
    bits, records = quantized_blocks(1, 6)
    k = tokens(1, 7, 1000.0)
    got = oracle.append_tokens(records, LAYERS, HEADS, SLOTS, DIM, [0], [15], 1, k, tokens(1, 8))
    block_elems = GROUP * GROUPS
    g = (0 * LAYERS + 1) * HEADS + 0
    shift = got[0, block_elems + 2 * g : block_elems + 2 * g + 2].view(np.int16)[0]
    restored = np.zeros((1, GROUP), dtype=np.uint16)
    restored[0, : 15 * DIM] = oracle.decode(records[0, g * GROUP : g * GROUP + 15 * DIM],
                                            int(records[0, block_elems + 2 * g : block_elems + 2 * g + 2].view(np.int16)[0]))
    restored[0, 15 * DIM :] = k[0, 0]
    assert shift == oracle.group_shifts(restored)[0] > records[0, block_elems + 2 * g : block_elems + 2 * g + 2].view(np.int16)[0]
    assert np.array_equal(got[0, g * GROUP : (g + 1) * GROUP], oracle.encode(restored[0], int(shift)))


def stub_capture(step, pool=None):
    from layover_amd.kv.decode_graphs import Replay

    return Replay(lambda: None, None, pool)


def test_graph_bookkeeping_reserves_a_scratch_block_and_pads_with_it():
    cache = PagedKVCache(ModelConfig.micro(), 12, fill=False)
    graphs = DecodeAttentionGraphs(cache, 4, sizes=(4, 1, 2), max_tokens=100, capture=stub_capture)
    assert graphs.sizes == (1, 2, 4) and graphs.width == 7
    scratch = graphs.scratch_blocks
    assert len(set(scratch)) == 4 and all(cache.allocator.refcount(b) == 1 for b in scratch)
    assert [graphs.size_for(n) for n in (1, 2, 3, 4, 5)] == [1, 2, 4, 4, None]
    padding = graphs._padding(2)
    assert padding.tolist() == [[b, 0, 1, b, 0, 0, 0, 0, 0, 0] for b in scratch[:2]]
    assert graphs.packed.shape == (4, 10) and torch.equal(graphs.packed, graphs._padding(4))
    graphs.release()
    assert cache.allocator.num_used == 0
    assert graphs.q.shape == (2, 4, 4, 24) and graphs.k_new.shape == (2, 4, 2, 24)
    assert graphs.widths == [7] and set(graphs._workspaces) == {(1, 7), (2, 7), (4, 7)}


def test_graphs_decline_batches_and_tables_they_were_not_captured_for():
    cache = PagedKVCache(ModelConfig.micro(), 12, fill=False)
    graphs = DecodeAttentionGraphs(cache, 4, sizes=(1, 2), max_tokens=32, capture=stub_capture)
    q, kv = torch.zeros(2, 3, 4, 24), torch.zeros(2, 3, 2, 24)
    assert graphs.run([BlockTable([1], 3)] * 3, q, kv, kv) is None
    assert graphs.run([BlockTable([1, 2, 3], 40)], q[:, :1], kv[:, :1], kv[:, :1]) is None


def test_graphs_refuse_a_head_count_that_does_not_divide():
    with pytest.raises(ValueError, match="divide"):
        DecodeAttentionGraphs(PagedKVCache(ModelConfig.micro(), 4, fill=False), 3, capture=stub_capture)


def test_decode_launch_layout_takes_packed_columns_and_refuses_what_it_cannot_describe():
    from layover_amd.kernels import hip_decode

    cache = PagedKVCache(ModelConfig.micro(), 12, fill=False)
    packed = cache.decode_rows([BlockTable([3, 7], 20), BlockTable([5], 1), BlockTable([1, 2, 9], 48)])
    table, lengths = packed[:, 3:], packed[:, 2]
    q = torch.zeros(3, 4, 24, dtype=torch.bfloat16)
    hip_decode._check_layout(q, table, lengths, q.clone())
    shape = hip_decode.decode_shape(q, cache.pool, 1, table, 2, lengths)
    assert (shape.table_width, shape.table_stride, shape.lengths_stride) == (3, 6, 6)
    with pytest.raises(ValueError, match="rows must be contiguous"):
        hip_decode._check_layout(q, packed.t().contiguous().t()[:, 3:], lengths, q.clone())
    with pytest.raises(ValueError, match="int32"):
        hip_decode._check_layout(q, table.long(), lengths, q.clone())
    with pytest.raises(ValueError, match="batch"):
        hip_decode._check_layout(q, table, lengths[:2], q.clone())
    with pytest.raises(ValueError, match="contiguous tensors"):
        hip_decode._check_layout(q, table, lengths, q.transpose(0, 1).contiguous().transpose(0, 1))


def test_token_write_and_prefill_arguments_are_checked_without_a_gpu():
    """The metadata checks run before any launch, so they refuse CPU tensors and bad shapes
    on any machine."""
    from layover_amd.kernels import hip_decode, hip_prefill

    rows = torch.zeros(2, dtype=torch.int32)
    k = torch.zeros(2, 8, 128, dtype=torch.bfloat16)
    pool = torch.zeros(4, 2, 3, 8, 16, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="one GPU"):
        hip_decode.write_tokens(pool, rows, rows, 0, k, k)
    with pytest.raises(ValueError, match="layer"):
        hip_decode.write_tokens(pool, rows, rows, 3, k, k)
    with pytest.raises(ValueError, match="int32"):
        hip_decode.write_tokens(pool, rows.long(), rows, 0, k, k)
    with pytest.raises(ValueError, match="row stride"):
        packed = torch.zeros(2, 5, dtype=torch.int32)
        hip_decode.write_tokens(pool, packed[:, 0], torch.zeros(2, dtype=torch.int32), 0, k, k)
    with pytest.raises(ValueError, match="BF16"):
        hip_decode.write_tokens(pool, rows, rows, 0, k.float(), k)
    with pytest.raises(ValueError, match="contiguous BF16"):
        hip_decode.write_tokens(pool.float(), rows, rows, 0, k, k)

    q = torch.zeros(32, 10, 128, dtype=torch.bfloat16)
    ids = torch.arange(4, dtype=torch.int32)
    with pytest.raises(ValueError, match="one GPU"):
        hip_prefill.paged_prefill_attention_hip(q, pool, 0, ids, 0, 4)
    with pytest.raises(ValueError, match="16-slot blocks of 128"):
        hip_prefill.paged_prefill_attention_hip(q[..., :64].contiguous(), pool[..., :64].contiguous(), 0, ids, 0, 4)
    with pytest.raises(ValueError, match="cannot hold"):
        hip_prefill.paged_prefill_attention_hip(q, pool, 0, ids[:1], 10, 4)


def test_fused_write_and_decode_arguments_are_checked_without_a_gpu():
    """run_kernel_append checks the decode layout and the token write from metadata alone,
    before any launch, so it refuses CPU tensors, an FP32 pool and a row count mismatch here."""
    from layover_amd.kernels import hip_decode

    cache = PagedKVCache(ModelConfig.micro(), 12, fill=False)
    packed = cache.decode_rows([BlockTable([3, 7], 20), BlockTable([5], 1)])
    table, lengths, blocks, slots = packed[:, 3:], packed[:, 2], packed[:, 0], packed[:, 1]
    q = torch.zeros(2, 4, 24, dtype=torch.bfloat16)
    k = torch.zeros(2, 2, 24, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="one GPU"):
        hip_decode.run_kernel_append(q, cache.pool, 1, table, lengths, 2, blocks, slots, k, k, q.clone())
    with pytest.raises(ValueError, match="BF16 or FP8-record pool"):
        hip_decode.run_kernel_append(q, cache.pool.float(), 1, table, lengths, 2, blocks, slots, k, k, q.clone())
    with pytest.raises(ValueError, match="int32"):
        hip_decode.run_kernel_append(q, cache.pool, 1, table, lengths, 2, blocks.long(), slots, k, k, q.clone())
    with pytest.raises(ValueError, match="layer"):
        hip_decode.run_kernel_append(q, cache.pool, 2, table, lengths, 2, blocks, slots, k, k, q.clone())


def test_prefill_split_plan_sizes_its_workspace(monkeypatch):
    """Short chunks against long histories split their keys; full-GPU chunks do not. The plan
    assumes 256 CUs when no device answers (as here)."""
    from layover_amd.kernels import _lib

    lib = _lib.load()
    long_chunk = _lib.PrefillShape(2048, 30720, 32, 8, 128, 36, 16, 0, _lib.LK_BF16, _lib.LK_BF16, 128**-0.5)
    assert lib.lk_paged_prefill_workspace(long_chunk) == 0  # 16 x 8 x 4 = 512 workgroups fill 256 CUs twice
    short = _lib.PrefillShape(512, 8192, 32, 8, 128, 36, 16, 0, _lib.LK_BF16, _lib.LK_BF16, 128**-0.5)
    # 128 workgroups: 4 splits of 68 of the 272 key steps; partials [8, 2048 rows, 4] x (128 + 2) floats.
    assert lib.lk_paged_prefill_workspace(short) == 8 * 2048 * 4 * 130 * 4
    monkeypatch.setenv("LAYOVER_PREFILL_SPLITS", "1")
    assert lib.lk_paged_prefill_workspace(short) == 0
    monkeypatch.setenv("LAYOVER_PREFILL_SPLITS", "1000")  # capped at 64: 5 steps each, so 55 splits
    assert lib.lk_paged_prefill_workspace(short) == 8 * 2048 * 55 * 130 * 4
    bad = _lib.PrefillShape(512, 8192, 30, 8, 128, 36, 16, 0, _lib.LK_BF16, _lib.LK_BF16, 1.0)
    assert lib.lk_paged_prefill_workspace(bad) == 0


def test_prefill_pair_halves_size_their_workspace(monkeypatch):
    """A 2,048-token chunk at position 0 (512 resident workgroups, causal tiles of 1 to 64 key
    steps) divides its heavy tiles within CU pairs: per (KV head, pair) two sides' states of
    256 threads x 80 floats, then a tag and a ready word, each part 256-byte aligned. A chunk
    ending a 32,768 context divides nothing (its paired tiles differ by a few percent) and
    needs no workspace; LAYOVER_PREFILL_PAIR_HALVES=0 turns the division off, and a bias that
    leaves the heavy tiles whole does too."""
    from layover_amd.kernels import _lib

    lib = _lib.load()
    at_zero = _lib.PrefillShape(2048, 0, 32, 8, 128, 36, 16, 0, _lib.LK_BF16, _lib.LK_BF16, 128**-0.5)
    pairs = 8 * 32
    assert lib.lk_paged_prefill_workspace(at_zero) == pairs * 2 * 256 * 80 * 4 + pairs * 2 * 8
    long_chunk = _lib.PrefillShape(2048, 30720, 32, 8, 128, 36, 16, 0, _lib.LK_BF16, _lib.LK_BF16, 128**-0.5)
    assert lib.lk_paged_prefill_workspace(long_chunk) == 0
    monkeypatch.setenv("LAYOVER_PREFILL_PAIR_BIAS", "64")  # every cut at or past the heavy tile's end
    assert lib.lk_paged_prefill_workspace(at_zero) == 0
    monkeypatch.setenv("LAYOVER_PREFILL_PAIR_BIAS", "12")
    monkeypatch.setenv("LAYOVER_PREFILL_PAIR_HALVES", "0")
    assert lib.lk_paged_prefill_workspace(at_zero) == 0


def test_fp8_prefill_workspace_holds_the_staged_history(monkeypatch):
    """An FP8-record pool's history is staged as a one-layer BF16 pool (64 KiB a block at
    Qwen3-4B's 8 KV heads) plus an int32 index, each part 256-byte aligned, ahead of any split
    partials; LAYOVER_PREFILL_FP8=direct leaves only the partials."""
    from layover_amd.kernels import _lib

    lib = _lib.load()
    fp8 = _lib.LK_FP8_RECORD
    long_chunk = _lib.PrefillShape(2048, 30720, 32, 8, 128, 36, 16, 0, _lib.LK_BF16, fp8, 128**-0.5)
    blocks = 32768 // 16
    assert lib.lk_paged_prefill_workspace(long_chunk) == blocks * 65536 + blocks * 4
    short = _lib.PrefillShape(512, 8192 + 5, 32, 8, 128, 36, 16, 0, _lib.LK_BF16, fp8, 128**-0.5)
    blocks = -(-(8192 + 5 + 512) // 16)  # 545
    index = -(-blocks * 4 // 256) * 256
    monkeypatch.setenv("LAYOVER_PREFILL_SPLITS", "4")
    assert lib.lk_paged_prefill_workspace(short) == blocks * 65536 + index + 8 * 2048 * 4 * 130 * 4
    monkeypatch.setenv("LAYOVER_PREFILL_FP8", "direct")
    assert lib.lk_paged_prefill_workspace(short) == 8 * 2048 * 4 * 130 * 4
    monkeypatch.delenv("LAYOVER_PREFILL_SPLITS")
    assert lib.lk_paged_prefill_workspace(long_chunk) == 0


def test_decode_split_plan_fills_the_gpu_at_small_batch():
    """The decode workspace follows the split plan: about 4,096 workgroups of at least 64
    blocks at large batch, about one workgroup per CU (256 without a GPU) when that would
    leave CUs idle, and one split for FP8-record tables of at most 64 blocks. Workspace =
    batch x query heads x splits x (128 + 2) x 4 bytes."""
    from layover_amd.kernels import _lib

    lib = _lib.load()

    def splits(batch, width, kv_format=_lib.LK_BF16):
        shape = _lib.DecodeShape(batch, 32, 8, 128, 36, 16, 0, width, _lib.LK_BF16, kv_format, 1.0 / math.sqrt(128), 0, 0)
        return lib.lk_paged_decode_workspace(shape) // (batch * 32 * 130 * 4)

    assert splits(32, 2048) == 16  # 128-block splits: 32 x 8 x 16 = 4,096 workgroups
    assert splits(64, 256) == 4 and splits(1, 2048) == 32  # 64-block splits
    assert splits(1, 256) == 32 and splits(1, 1024) == 32 and splits(2, 256) == 16  # 8, 32, 16 blocks: 256 workgroups
    assert splits(4, 256) == 8 and splits(8, 256) == 4
    assert splits(1, 64) == 8 and splits(1, 64, _lib.LK_FP8_RECORD) == 1 and splits(1, 65, _lib.LK_FP8_RECORD) == 9
