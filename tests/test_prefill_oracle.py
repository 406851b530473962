"""The prefill oracle (a composition of the decode oracle, one query token at a time) against
causal softmax attention written out directly in float64 numpy on tiny inputs: GQA head
mapping, the bottom-right causal offset of a chunk that starts mid-block, and block-table
indirection."""

import numpy as np
import pytest

from oracle import oracle


def brute_force(q, pool_bits, layer, block_ids, start, groups):
    values = oracle.bf16_to_float(pool_bits).astype(np.float64)
    slots = pool_bits.shape[4]
    heads, tokens, dim = q.shape
    end = start + tokens
    keys = np.stack([values[block_ids[p // slots], 0, layer, :, p % slots] for p in range(end)], axis=1)  # [kv, end, dim]
    vals = np.stack([values[block_ids[p // slots], 1, layer, :, p % slots] for p in range(end)], axis=1)
    out = np.zeros((heads, tokens, dim))
    for h in range(heads):
        for t in range(tokens):
            visible = start + t + 1
            scores = keys[h // groups, :visible] @ q[h, t] / np.sqrt(dim)
            weights = np.exp(scores - scores.max())
            out[h, t] = weights @ vals[h // groups, :visible] / weights.sum()
    return out


@pytest.mark.parametrize("start,tokens,groups", [(0, 5, 2), (7, 9, 1), (16, 3, 3), (21, 12, 2)])
def test_prefill_oracle_is_causal_softmax_attention(start, tokens, groups):
    rng = np.random.default_rng(start + tokens)
    blocks, layers, kv_heads, slots, dim = 6, 2, 2, 8, 12
    pool = oracle.bf16_bits(rng.standard_normal((blocks, 2, layers, kv_heads, slots, dim), dtype=np.float32))
    block_ids = rng.permutation(blocks)[: -(-(start + tokens) // slots)].astype(np.int32)
    q = rng.standard_normal((kv_heads * groups, tokens, dim))
    got = oracle.prefill_attention(q, pool, 1, block_ids, start, groups)
    assert np.abs(got - brute_force(q, pool, 1, block_ids, start, groups)).max() < 1e-12
