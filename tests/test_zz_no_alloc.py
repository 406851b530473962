"""lk_paged_decode_static, the decode entry point that allocates nothing (its split partials
live in a file-scope device array), against lk_paged_decode with a caller's workspace: the
same kernels, so the outputs must be identical bit for bit. Two calls in a row, the second
smaller, so the second reads an array that still holds the first call's partials."""

import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu


def case(batch, max_len, seed, fp8=False):
    from layover_amd.kernels import fp8 as codec
    from layover_amd.kernels import hip_decode

    rng = np.random.default_rng(seed)
    layers, kv_heads, slots, dim = 4, 8, 16, 128
    lengths = rng.integers(1, max_len + 1, size=batch).astype(np.int32)
    lengths[0] = max_len
    width = -(-max_len // slots)
    blocks = width + 8
    gen = torch.Generator(device="cuda").manual_seed(seed)
    pool = torch.randn(blocks, 2, layers, kv_heads, slots, dim, generator=gen, device="cuda").to(torch.bfloat16)
    table = np.stack([rng.choice(blocks, width, replace=False) for _ in range(batch)]).astype(np.int32)
    q = torch.randn(batch, 32, dim, generator=gen, device="cuda").to(torch.bfloat16)
    target = pool
    if fp8:
        layout = codec.Fp8Layout(slots * dim, 2 * layers * kv_heads)
        records = torch.empty(blocks, layout.record_bytes, dtype=torch.uint8, device="cuda")
        codec.quantize_blocks(pool, torch.arange(blocks, dtype=torch.int32, device="cuda"), records.view(-1), layout)
        target = hip_decode.Fp8KVPool(records, layers, kv_heads, slots, dim)
    return q, target, pool, torch.from_numpy(table).cuda(), torch.from_numpy(lengths).cuda()


def run_both(q, target, table, lengths, layer):
    from layover_amd.kernels import _lib, hip_decode

    lib = _lib.load()
    shape = hip_decode.decode_shape(q, target, layer, table, 4, lengths)
    storage = target.records if isinstance(target, hip_decode.Fp8KVPool) else target
    stream = _lib.current_stream(q.device)
    with_workspace = torch.empty_like(q)
    need = int(lib.lk_paged_decode_workspace(shape))
    workspace = torch.empty(need, dtype=torch.uint8, device="cuda")
    _lib.check(lib.lk_paged_decode(shape, q.data_ptr(), storage.data_ptr(), table.data_ptr(), lengths.data_ptr(),
                                   with_workspace.data_ptr(), workspace.data_ptr(), need, stream))
    static = torch.full_like(q, float("nan"))
    _lib.check(lib.lk_paged_decode_static(shape, q.data_ptr(), storage.data_ptr(), table.data_ptr(), lengths.data_ptr(),
                                          static.data_ptr(), stream))
    torch.cuda.synchronize()
    return with_workspace, static


@pytest.mark.parametrize("fp8", [False, True], ids=["bf16_pool", "fp8_pool"])
def test_static_scratch_decode_equals_the_workspace_decode_on_two_calls(fp8):
    print(f"no-alloc decode fp8={fp8}: batch 32 at up to 32,768 tokens, then batch 3 at up to 700", flush=True)
    first = case(32, 32768, seed=1, fp8=fp8)
    a, b = run_both(first[0], first[1], first[3], first[4], layer=3)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    second = case(3, 700, seed=2, fp8=fp8)
    a, b = run_both(second[0], second[1], second[3], second[4], layer=1)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    if not fp8:
        q, _, pool, table, lengths = second
        bits = pool.view(torch.int16).cpu().numpy().view(np.uint16)
        expected = oracle.decode_attention(q.view(torch.int16).cpu().numpy().view(np.uint16), bits, 1, table.cpu().numpy(),
                                           lengths.cpu().numpy(), 4)
        error = np.abs(b.double().cpu().numpy() - expected)
        assert (error <= 2e-2 + 1e-2 * np.abs(expected)).all()


def test_a_shape_beyond_the_static_scratch_is_refused_before_launch():
    from layover_amd.kernels import _lib

    lib = _lib.load()
    shape = _lib.DecodeShape(512, 32, 8, 128, 36, 16, 0, 4096, _lib.LK_BF16, _lib.LK_BF16, 128**-0.5)
    assert lib.lk_paged_decode_workspace(shape) > 32 << 20
    dummy = torch.zeros(16, dtype=torch.uint8, device="cuda")
    status = lib.lk_paged_decode_static(shape, dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(), dummy.data_ptr(),
                                        dummy.data_ptr(), _lib.current_stream(dummy.device))
    assert status == _lib.LK_ERR_INVALID
    assert b"static scratch" in lib.lk_last_error()


def test_static_calls_on_two_streams_are_ordered_and_equal_the_workspace_decode():
    """Calls alternating between two streams share the one array; each call's stream waits for
    the previous call, so every output equals its workspace decode bit for bit, the case with
    the most splits (batch 32 up to 32,768 tokens) followed by a small one on the other stream,
    in a row with no synchronization between them."""
    from layover_amd.kernels import _lib, hip_decode

    lib = _lib.load()
    print("no-alloc decode on two streams", flush=True)
    cases = [case(32, 32768, seed=5), case(3, 700, seed=6), case(16, 8000, seed=7)]
    expected = [run_both(c[0], c[1], c[3], c[4], layer=2)[0] for c in cases]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.full_like(c[0], float("nan")) for c in cases]
    torch.cuda.synchronize()
    for round_ in range(3):
        for i, (q, target, _, table, lengths) in enumerate(cases):
            stream = streams[(i + round_) % 2]
            shape = hip_decode.decode_shape(q, target, 2, table, 4, lengths)
            _lib.check(lib.lk_paged_decode_static(shape, q.data_ptr(), target.data_ptr(), table.data_ptr(), lengths.data_ptr(),
                                                  outs[i].data_ptr(), stream.cuda_stream))
        torch.cuda.synchronize()
        for i in range(len(cases)):
            assert torch.equal(outs[i].view(torch.int16), expected[i].view(torch.int16)), f"round {round_}, case {i}"
            outs[i].fill_(float("nan"))


def test_static_decode_captured_in_a_graph_replays_like_the_eager_call():
    """The entry point under HIP graph capture (the callers it is for): replays, with eager work
    and synchronizations between them, each equal the workspace decode bit for bit."""
    from layover_amd.kernels import _lib, hip_decode

    lib = _lib.load()
    print("no-alloc decode under graph capture", flush=True)
    q, target, _, table, lengths = case(8, 4096, seed=8)
    expected = run_both(q, target, table, lengths, layer=0)[0]
    shape = hip_decode.decode_shape(q, target, 0, table, 4, lengths)
    out = torch.full_like(q, float("nan"))
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            _lib.check(lib.lk_paged_decode_static(shape, q.data_ptr(), target.data_ptr(), table.data_ptr(), lengths.data_ptr(),
                                                  out.data_ptr(), side.cuda_stream))
    torch.cuda.synchronize()
    other = case(3, 700, seed=9)
    for replay in range(3):
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), expected.view(torch.int16)), f"replay {replay}"
        run_both(other[0], other[1], other[3], other[4], layer=1)  # eager static call between replays
