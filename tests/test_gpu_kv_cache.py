"""GPU slot writes and gathers are bit-exact against the oracle (``oracle/paged_kv.py``)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import paged_kv

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _as_np(t: torch.Tensor) -> np.ndarray:
    t = t.cpu()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy()
    return t.numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("table_dtype", [torch.int32, torch.int64])
def test_append_matches_oracle_bit_exact(dtype, table_dtype) -> None:
    import hip_ops

    gen = torch.Generator().manual_seed(21)
    batch, kv_heads, dim, bs, pool_blocks, max_blocks = 3, 2, 256, 16, 30, 8
    key_pool = torch.randn(pool_blocks, kv_heads, bs, dim, generator=gen).to(dtype)
    value_pool = torch.randn(pool_blocks, kv_heads, bs, dim, generator=gen).to(dtype)
    perm = torch.randperm(pool_blocks, generator=gen)[: batch * max_blocks].reshape(batch, max_blocks)
    starts = [0, 7, 31]
    seq = 20
    counts = [20, 9, 20]
    new_k = torch.randn(batch, kv_heads, seq, dim, generator=gen).to(dtype)
    new_v = torch.randn(batch, kv_heads, seq, dim, generator=gen).to(dtype)
    # oracle on numpy copies
    ok, ov = _as_np(key_pool).copy(), _as_np(value_pool).copy()
    for b in range(batch):
        paged_kv.append_tokens(ok, perm[b].numpy(), starts[b], _as_np(new_k[b, :, : counts[b]]), block_size=bs, pool_layout="phbd")
        paged_kv.append_tokens(ov, perm[b].numpy(), starts[b], _as_np(new_v[b, :, : counts[b]]), block_size=bs, pool_layout="phbd")
    kp, vp = key_pool.to(DEV), value_pool.to(DEV)
    hip_ops.paged_kv_append(
        new_k.to(DEV), new_v.to(DEV), kp, vp, perm.to(DEV, table_dtype), torch.tensor(starts, device=DEV), bs,
        counts=torch.tensor(counts, device=DEV, dtype=torch.int32),
    )
    np.testing.assert_array_equal(_as_np(kp), ok)
    np.testing.assert_array_equal(_as_np(vp), ov)


def test_append_reference_layout_scalar_start_matches_oracle() -> None:
    import hip_ops

    gen = torch.Generator().manual_seed(22)
    heads, dim, bs, blocks = 4, 8, 2, 6
    pool_k = torch.randn(1, heads, blocks, bs, dim, generator=gen)
    pool_v = torch.randn(1, heads, blocks, bs, dim, generator=gen)
    table = torch.tensor([3, 1, 4, 0])
    new_k = torch.randn(1, heads, 5, dim, generator=gen)
    new_v = torch.randn(1, heads, 5, dim, generator=gen)
    ok, ov = pool_k[0].numpy().copy(), pool_v[0].numpy().copy()
    paged_kv.append_tokens(ok, table.numpy(), 2, new_k[0].numpy(), block_size=bs, pool_layout="hpbd")
    paged_kv.append_tokens(ov, table.numpy(), 2, new_v[0].numpy(), block_size=bs, pool_layout="hpbd")
    kp, vp = pool_k.to(DEV), pool_v.to(DEV)
    hip_ops.paged_kv_append(new_k.to(DEV), new_v.to(DEV), kp, vp, table.to(DEV), 2, bs)
    np.testing.assert_array_equal(kp[0].cpu().numpy(), ok)
    np.testing.assert_array_equal(vp[0].cpu().numpy(), ov)


def test_gather_matches_oracle_and_zero_fills_invalid() -> None:
    import hip_ops

    gen = torch.Generator().manual_seed(23)
    kv_heads, dim, bs, blocks = 2, 256, 16, 12
    kp = torch.randn(blocks, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    vp = torch.randn(blocks, kv_heads, bs, dim, generator=gen).to(torch.bfloat16)
    tables = torch.tensor([[5, 2, 9, -1], [0, 11, 3, 7]])
    valid = 50
    k_out, v_out = hip_ops.paged_kv_gather(kp.to(DEV), vp.to(DEV), tables.to(DEV), valid, bs)
    for b in range(2):
        expect_k = paged_kv.gather_tokens_bruteforce(_as_np(kp), [max(x, 0) for x in tables[b].tolist()], valid, block_size=bs, pool_layout="phbd")
        got = _as_np(k_out[b])
        if b == 0:
            np.testing.assert_array_equal(got[:, :48], expect_k[:, :48])
            assert (got[:, 48:] == 0).all()
        else:
            np.testing.assert_array_equal(got, expect_k)
    expect_v = paged_kv.gather_tokens(_as_np(vp), tables[1].tolist(), valid, block_size=bs, pool_layout="phbd")
    np.testing.assert_array_equal(_as_np(v_out[1]), expect_v)


def test_append_then_decode_equals_dense_reference() -> None:
    """Round trip: appended tokens are exactly what decode and gather read back."""
    import hip_ops
    from oracle import attention

    gen = torch.Generator().manual_seed(24)
    heads, kv_heads, dim, bs = 16, 2, 256, 16
    lens = [33, 64]
    pool_blocks = 16
    kp = torch.zeros(pool_blocks, kv_heads, bs, dim, dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros_like(kp)
    tables = torch.tensor([[7, 1, 12, -1], [3, 14, 0, 9]], device=DEV)
    dense_k = torch.randn(2, kv_heads, 64, dim, generator=gen).to(torch.bfloat16)
    dense_v = torch.randn(2, kv_heads, 64, dim, generator=gen).to(torch.bfloat16)
    hip_ops.paged_kv_append(dense_k.to(DEV), dense_v.to(DEV), kp, vp, tables, 0, bs, counts=torch.tensor(lens, device=DEV))
    k_back, _ = hip_ops.paged_kv_gather(kp, vp, tables, 33, bs)
    assert torch.equal(k_back[0].cpu(), dense_k[0, :, :33])
    q = torch.randn(2, heads, 1, dim, generator=gen).to(torch.bfloat16)
    out = hip_ops.paged_attention_decode_batched(q.to(DEV), tables, kp, vp, torch.tensor(lens, device=DEV), bs)
    for b in range(2):
        ref = attention.dense_attention(q[b : b + 1], dense_k[b : b + 1, :, : lens[b]], dense_v[b : b + 1, :, : lens[b]], position_offset=lens[b] - 1)
        torch.testing.assert_close(out[b : b + 1].cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("table_dtype,batch", [(torch.int32, 5), (torch.int64, 3000)])
def test_device_reserve_matches_oracle_bit_exact(table_dtype, batch) -> None:
    import hip_ops

    rng = np.random.default_rng(31 + batch)
    bs, max_blocks, capacity = 16, 24, 40000
    lengths = rng.integers(0, 300, batch)
    counts = rng.integers(0, 60, batch)
    counts[::7] = 0
    free = sorted(rng.permutation(capacity)[: capacity - 1000].tolist())
    tables = np.full((batch, max_blocks), -1, dtype=np.int64)
    status, want_t, want_pos, want_len, want_free = paged_kv.reserve_step(tables, lengths, counts, free, bs)
    assert status == 0
    print(f"device reserve: batch {batch}, table {table_dtype}, {len(free) - len(want_free)} blocks", flush=True)
    free_list = torch.full((capacity,), -1, dtype=torch.int32, device=DEV)
    free_list[: len(free)] = torch.tensor(free, dtype=torch.int32, device=DEV)
    free_state = torch.tensor([0, len(free)], dtype=torch.int32, device=DEV)
    st = torch.full((1,), 99, dtype=torch.int32, device=DEV)
    t = torch.from_numpy(tables).to(DEV, table_dtype)
    lens = torch.from_numpy(lengths).to(DEV, torch.int32)
    pos = torch.full((batch,), -5, dtype=torch.int64, device=DEV)
    hip_ops.paged_kv_reserve(t, lens, free_list, free_state, st, bs, counts=torch.from_numpy(counts).to(DEV), positions=pos)
    assert int(st.item()) == 0
    np.testing.assert_array_equal(t.cpu().numpy().astype(np.int64), want_t)
    np.testing.assert_array_equal(pos.cpu().numpy(), want_pos)
    np.testing.assert_array_equal(lens.cpu().numpy(), want_len)
    head, count = free_state.tolist()
    assert free_list[head : head + count].tolist() == want_free


def test_device_reserve_failure_writes_nothing() -> None:
    import hip_ops

    bs = 16
    free_list = torch.arange(3, dtype=torch.int32, device=DEV)
    free_state = torch.tensor([0, 3], dtype=torch.int32, device=DEV)
    st = torch.zeros(1, dtype=torch.int32, device=DEV)
    tables = torch.full((2, 4), -1, dtype=torch.int32, device=DEV)
    lens = torch.tensor([0, 0], dtype=torch.int64, device=DEV)
    # 40 + 20 tokens need 3 + 2 blocks, 3 are free
    hip_ops.paged_kv_reserve(tables, lens, free_list, free_state, st, bs, counts=torch.tensor([40, 20], device=DEV))
    assert int(st.item()) == 1
    # 70 tokens need 5 blocks of a 4-wide row
    hip_ops.paged_kv_reserve(tables, lens, free_list, free_state, st, bs, counts=torch.tensor([70, 0], device=DEV))
    assert int(st.item()) == 2
    assert (tables == -1).all().item() and lens.tolist() == [0, 0] and free_state.tolist() == [0, 3]
    # then a fitting request succeeds from the untouched state
    hip_ops.paged_kv_reserve(tables, lens, free_list, free_state, st, bs, counts=torch.tensor([17, 16], device=DEV))
    assert int(st.item()) == 0 and tables.tolist() == [[0, 1, -1, -1], [2, -1, -1, -1]] and free_state.tolist() == [3, 0]


def test_device_allocator_release_resorts_and_reuses() -> None:
    from decode_state import DeviceBlockAllocator

    alloc = DeviceBlockAllocator(8, device=DEV)
    tables = torch.full((2, 4), -1, dtype=torch.int32, device=DEV)
    lens = torch.tensor([0, 0], dtype=torch.int32, device=DEV)
    alloc.reserve(tables, lens, 4, counts=torch.tensor([9, 6], dtype=torch.int32, device=DEV))
    alloc.check()
    assert tables.tolist() == [[0, 1, 2, -1], [3, 4, -1, -1]] and alloc.free_blocks() == [5, 6, 7]
    alloc.release([3, 1])
    assert alloc.free_blocks() == [1, 3, 5, 6, 7] and alloc.free_count == 5
    tables2 = torch.full((1, 4), -1, dtype=torch.int32, device=DEV)
    alloc.reserve(tables2, torch.zeros(1, dtype=torch.int32, device=DEV), 4, counts=5)
    alloc.check()
    assert tables2.tolist() == [[1, 3, -1, -1]]
    alloc.reserve(tables2, torch.zeros(1, dtype=torch.int32, device=DEV), 4, counts=16)  # 4 blocks, 3 free
    with pytest.raises(RuntimeError, match="exhausted"):
        alloc.check()
    alloc.reserve(tables2, torch.zeros(1, dtype=torch.int32, device=DEV), 4, counts=17)  # 5 blocks of a 4-wide row
    with pytest.raises(RuntimeError, match="table too short"):
        alloc.check()
    assert tables2.tolist() == [[1, 3, -1, -1]] and alloc.free_blocks() == [5, 6, 7]


def test_reserve_after_shared_pool_hand_off_reuses_released_cache_blocks() -> None:
    """A cache on a shared pool releases its blocks after the pool's free list went to the device:
    the next device reservation takes those ids first (lowest free id)."""
    from decode_state import FullAttentionCache, SharedKVBlockPool

    pool = SharedKVBlockPool(6, kv_heads=1, head_dim=8, block_size=4, dtype=torch.bfloat16, device=DEV)
    cache = FullAttentionCache(block_size=4, shared_pool=pool)
    cache.append_blocks(torch.ones(1, 1, 7, 8, dtype=torch.bfloat16, device=DEV), torch.ones(1, 1, 7, 8, dtype=torch.bfloat16, device=DEV))
    assert cache.block_table == [0, 1]
    alloc = pool.device_allocator()
    tables = torch.full((1, 4), -1, dtype=torch.int32, device=DEV)
    lens = torch.zeros(1, dtype=torch.int32, device=DEV)
    alloc.reserve(tables, lens, 4, counts=4)
    alloc.check()
    assert tables.tolist() == [[2, -1, -1, -1]]
    cache.release()
    alloc.reserve(tables, lens, 4, counts=8)
    alloc.check()
    assert tables.tolist() == [[2, 0, 1, -1]] and lens.tolist() == [12] and alloc.free_blocks() == [3, 4, 5]


def test_graph_captured_decode_step_matches_eager_and_oracle() -> None:
    """reserve -> K/V append -> batched decode captured once and replayed step after
    step; every replay equals the same step run eagerly on a twin state, and the last
    one matches the oracle's attention over the gathered cache."""
    import hip_ops
    from decode_state import DeviceBlockAllocator
    from oracle import attention as oracle_attn

    gen = torch.Generator().manual_seed(41)
    batch, heads, kv_heads, dim, bs, pool_blocks, max_blocks, steps = 6, 16, 2, 256, 16, 96, 12, 5
    init = torch.tensor([1, 15, 16, 33, 0, 47], dtype=torch.int32)

    def make_state():
        pool_k = torch.zeros(pool_blocks, kv_heads, bs, dim, dtype=torch.bfloat16, device=DEV)
        pool_v = torch.zeros_like(pool_k)
        alloc = DeviceBlockAllocator(pool_blocks, device=DEV)
        tables = torch.full((batch, max_blocks), -1, dtype=torch.int32, device=DEV)
        lens = torch.zeros(batch, dtype=torch.int32, device=DEV)
        pos = torch.zeros(batch, dtype=torch.int64, device=DEV)
        return dict(pool_k=pool_k, pool_v=pool_v, alloc=alloc, tables=tables, lens=lens, pos=pos)

    prefill_k = torch.randn(batch, kv_heads, 64, dim, generator=gen).to(torch.bfloat16).to(DEV)
    prefill_v = torch.randn(batch, kv_heads, 64, dim, generator=gen).to(torch.bfloat16).to(DEV)

    def prefill(s):
        s["alloc"].reserve(s["tables"], s["lens"], bs, counts=init.to(DEV), positions=s["pos"])
        hip_ops.paged_kv_append(prefill_k, prefill_v, s["pool_k"], s["pool_v"], s["tables"], s["pos"], bs, counts=init.to(DEV))

    def step(s, q, k, v):
        s["alloc"].reserve(s["tables"], s["lens"], bs, counts=1, positions=s["pos"])
        hip_ops.paged_kv_append(k, v, s["pool_k"], s["pool_v"], s["tables"], s["pos"], bs)
        return hip_ops.paged_attention_decode_batched(q, s["tables"], s["pool_k"], s["pool_v"], s["lens"], bs)

    eager, graphed, scratch = make_state(), make_state(), make_state()
    for s in (eager, graphed, scratch):
        prefill(s)
    q_static = torch.zeros(batch, heads, 1, dim, dtype=torch.bfloat16, device=DEV)
    k_static = torch.zeros(batch, kv_heads, 1, dim, dtype=torch.bfloat16, device=DEV)
    v_static = torch.zeros_like(k_static)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(scratch, q_static, k_static, v_static)  # first-call set-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_static = step(graphed, q_static, k_static, v_static)
    print("graph captured", flush=True)
    for i in range(steps):
        q = torch.randn(batch, heads, 1, dim, generator=gen).to(torch.bfloat16).to(DEV)
        k = torch.randn(batch, kv_heads, 1, dim, generator=gen).to(torch.bfloat16).to(DEV)
        v = torch.randn(batch, kv_heads, 1, dim, generator=gen).to(torch.bfloat16).to(DEV)
        q_static.copy_(q)
        k_static.copy_(k)
        v_static.copy_(v)
        graph.replay()
        out_eager = step(eager, q, k, v)
        torch.cuda.synchronize()
        eager["alloc"].check()
        graphed["alloc"].check()
        assert torch.equal(out_static, out_eager), f"replay {i}"
        for name in ("tables", "lens", "pos", "pool_k", "pool_v"):
            assert torch.equal(graphed[name], eager[name]), f"replay {i}: {name}"
        assert torch.equal(graphed["alloc"].free_state, eager["alloc"].free_state)
    lens = eager["lens"].tolist()
    assert lens == [int(n) + steps for n in init]
    tables = eager["tables"].cpu().tolist()
    ref = oracle_attn.paged_decode(
        q.cpu(), [eager["pool_k"].cpu()] * batch, [eager["pool_v"].cpu()] * batch, tables, lens, block_size=bs, pool_layout="phbd"
    )
    torch.testing.assert_close(out_static.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)
    # ids were handed out lowest first in row order: the prefill's blocks, then one per
    # row whose next token opens a block
    status, want_t, _p, want_len, _f = paged_kv.reserve_step(
        np.full((batch, max_blocks), -1, dtype=np.int64), np.zeros(batch, dtype=np.int64), init.numpy(), list(range(pool_blocks)), bs
    )
    cur = want_len
    for _ in range(steps):
        status, want_t, _p, cur, _f = paged_kv.reserve_step(want_t, cur, 1, sorted(set(range(pool_blocks)) - set(want_t[want_t >= 0].tolist())), bs)
        assert status == 0
    np.testing.assert_array_equal(np.asarray(tables, dtype=np.int64), want_t)
