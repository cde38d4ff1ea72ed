"""Runtime-level hot path on the GPU: caches + dispatch + kernels against the oracle."""

from __future__ import annotations

import pytest
import torch

import attention_runtime as ar
from decode_state import FullAttentionCache, LinearStatePool, SharedKVBlockPool
from oracle import attention as oracle_attn
from oracle import gated_delta as gd

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _enabled(heads=2, kv_heads=2, dim=4) -> ar.AttentionConfig:
    text = {
        "linear_num_key_heads": 2, "linear_num_value_heads": 4, "linear_key_head_dim": 128, "linear_value_head_dim": 128,
        "linear_conv_kernel_dim": 4, "num_attention_heads": heads, "num_key_value_heads": kv_heads, "head_dim": dim,
        "attn_output_gate": True, "native_paged_attention": True,
    }
    return ar.parse_attention_config({"text_config": text})


@pytest.mark.parametrize("seed,seqs", [(0, (3, 5)), (7, (1, 9, 4))])
def test_batched_native_matches_dense_without_dense_views(seed, seqs) -> None:
    # tests/unit/test_tp_runtime.py:760-822 (fp32 per-request pools, atol 1e-4)
    torch.manual_seed(seed)
    caches, keys, values = [], [], []
    for row, seq in enumerate(seqs):
        cache = FullAttentionCache(block_size=2)
        key = torch.randn((1, 2, seq, 4), device=DEV) + row
        value = torch.randn((1, 2, seq, 4), device=DEV) - row
        cache.append_blocks(key, value)
        caches.append(cache)
        keys.append(key)
        values.append(value)
    query = torch.randn((len(seqs), 2, 1, 4), device=DEV)
    runtime = ar.HotPathRuntime()
    heads = ar.full_attention_paged_batch(query, None, caches, _enabled(), runtime)
    assert heads is not None and runtime.paged_attention_stats.native_hits == 1
    expected = torch.cat(
        [oracle_attn.dense_attention(query[r : r + 1].cpu(), keys[r].cpu(), values[r].cpu(), position_offset=seqs[r] - 1, cast_probs=False) for r in range(len(seqs))]
    )
    torch.testing.assert_close(heads.cpu(), expected, rtol=1e-4, atol=1e-4)
    assert all(c.stats().contiguous_view_calls == 0 and c.stats().gather_view_calls == 0 for c in caches)


def test_shared_pool_decode_loop_with_gate_matches_oracle() -> None:
    """Engine-like loop: prefill appends, then decode steps append one token and attend (bf16, GQA 16/2, D=256)."""
    gen = torch.Generator().manual_seed(61)
    heads, kv_heads, dim = 16, 2, 256
    config = _enabled(heads, kv_heads, dim)
    pool = SharedKVBlockPool(64, kv_heads, dim, block_size=16, device=DEV)
    prompt = [37, 5, 80]
    caches = [FullAttentionCache(capacity_hint=p + 4, block_size=16, shared_pool=pool) for p in prompt]
    dense_k = [torch.randn(1, kv_heads, p + 3, dim, generator=gen).to(torch.bfloat16) for p in prompt]
    dense_v = [torch.randn(1, kv_heads, p + 3, dim, generator=gen).to(torch.bfloat16) for p in prompt]
    for cache, k, v, p in zip(caches, dense_k, dense_v, prompt):
        cache.append_blocks(k[:, :, :p].to(DEV), v[:, :, :p].to(DEV))
    runtime = ar.HotPathRuntime()
    for step in range(3):
        for r, cache in enumerate(caches):
            pos = prompt[r] + step
            cache.append_blocks(dense_k[r][:, :, pos : pos + 1].to(DEV), dense_v[r][:, :, pos : pos + 1].to(DEV))
        q = torch.randn(3, heads, 1, dim, generator=gen).to(torch.bfloat16)
        gate = torch.randn(3, 1, heads * dim, generator=gen).to(torch.bfloat16)
        out = ar.full_attention_paged_batch(q.to(DEV), gate.to(DEV), caches, config, runtime)
        for r in range(3):
            n = prompt[r] + step + 1
            ref = oracle_attn.dense_attention(q[r : r + 1], dense_k[r][:, :, :n], dense_v[r][:, :, :n], position_offset=n - 1, gate=gate[r : r + 1])
            torch.testing.assert_close(out[r : r + 1].cpu().float(), ref.transpose(1, 2).reshape(1, 1, heads * dim).float(), atol=2e-2, rtol=2e-2)
    assert runtime.paged_attention_stats.native_hits == 3
    for cache in caches:
        cache.release()
    assert len(pool.free_blocks) == 64


def test_linear_attention_decode_batch_on_slot_pool_matches_oracle() -> None:
    config = _enabled()
    lin = config.linear_attention
    shape = gd.LinearShape(lin.key_heads, lin.value_heads, lin.key_head_dim, lin.value_head_dim, lin.conv_kernel_dim)
    gen = torch.Generator().manual_seed(62)
    batch, steps = 3, 4
    mixed = torch.randn(batch, steps, shape.qkv_dim, generator=gen).to(torch.bfloat16)
    a = torch.randn(batch, steps, shape.value_heads, generator=gen)
    b = torch.randn(batch, steps, shape.value_heads, generator=gen)
    a_log = torch.randn(shape.value_heads, generator=gen) * 0.3
    dt_bias = torch.zeros(shape.value_heads)
    w = torch.randn(shape.qkv_dim, 1, 4, generator=gen) * 0.5
    ref, ref_state, _ = gd.linear_attention_core(mixed.float(), a, b, a_log, dt_bias, w, shape)
    pool = LinearStatePool(6, shape.value_heads, 128, 128, shape.qkv_dim, 4, device=DEV)
    slots = torch.tensor([pool.acquire() for _ in range(batch)], device=DEV)
    outs = []
    for t in range(steps):
        outs.append(
            ar.linear_attention_decode_batch(
                mixed[:, t].contiguous().to(DEV), a[:, t].contiguous().to(DEV), b[:, t].contiguous().to(DEV), a_log.to(DEV), dt_bias.to(DEV), w.to(DEV),
                pool, slots, config, out_dtype=torch.float32,
            ).cpu()
        )
    torch.testing.assert_close(torch.stack(outs, dim=1), ref, atol=2e-3, rtol=2e-3)
    err = (pool.state[slots].cpu().double() - ref_state.double()).norm() / ref_state.double().norm()
    assert float(err) < 1e-3


def test_recurrent_wrapper_matches_oracle_and_keeps_dtype() -> None:
    gen = torch.Generator().manual_seed(63)
    q = torch.randn(2, 6, 3, 16, generator=gen)
    k = torch.randn(2, 6, 3, 16, generator=gen)
    v = torch.randn(2, 6, 3, 8, generator=gen)
    g = -torch.rand(2, 6, 3, generator=gen)
    beta = torch.rand(2, 6, 3, generator=gen)
    s0 = torch.randn(2, 3, 16, 8, generator=gen) * 0.1
    out, state = ar.recurrent_gated_delta_rule(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), beta.to(DEV), initial_state=s0.to(DEV), return_state=True)
    ref_out, ref_state = gd.recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=s0)
    assert out.dtype == q.dtype and out.shape == (2, 6, 3, 8) and state.dtype == torch.float32
    torch.testing.assert_close(out.cpu(), ref_out, atol=2e-5, rtol=2e-5)
    torch.testing.assert_close(state.cpu(), ref_state, atol=2e-5, rtol=2e-5)


def test_device_page_tables_running_batch_two_layers_matches_oracle_and_replays_as_a_graph() -> None:
    """A running batch on device-resident page tables shared by two full-attention layers: prompts
    admitted, decode steps (one reservation per step for both layers, the step's K/V appended, then
    attention), a request released and a new one reusing its blocks and row, then the whole step
    captured in a HIP graph (no-alloc attention) and replayed three times -- every step and every
    replay against the oracle's dense attention over the tokens written so far (bf16, 2e-2)."""
    import hip_ops
    from decode_state import DeviceBatchPageTables

    gen = torch.Generator().manual_seed(64)
    heads, kv_heads, dim, bs, layers = 16, 2, 256, 16, 2
    config = _enabled(heads, kv_heads, dim)
    pools = [SharedKVBlockPool(40, kv_heads, dim, block_size=bs, device=DEV) for _ in range(layers)]
    tables = DeviceBatchPageTables(pools[0], rows=4, max_blocks=12)
    runtime = ar.HotPathRuntime()
    total = 160
    # dense K/V of every (layer, request) the test may write, in token order
    dense = {}

    def tokens(layer, req):
        if (layer, req) not in dense:
            dense[(layer, req)] = (torch.randn(1, kv_heads, total, dim, generator=gen).to(torch.bfloat16),
                                   torch.randn(1, kv_heads, total, dim, generator=gen).to(torch.bfloat16))
        return dense[(layer, req)]

    length = {}
    row_of = {}

    def admit(req, prompt):
        row = tables.add_request(prompt)
        row_of[req] = row
        length[req] = prompt
        for layer, pool in enumerate(pools):
            k, v = tokens(layer, req)
            hip_ops.paged_kv_append(k[:, :, :prompt].to(DEV), v[:, :, :prompt].to(DEV), pool.key_blocks, pool.value_blocks,
                                    tables.block_tables[row : row + 1], tables.positions[row : row + 1], bs)

    def step_inputs(layer):
        k_new = torch.zeros(tables.rows, kv_heads, 1, dim, dtype=torch.bfloat16)
        v_new = torch.zeros_like(k_new)
        for req, row in row_of.items():
            k, v = tokens(layer, req)
            k_new[row] = k[0, :, length[req] : length[req] + 1]
            v_new[row] = v[0, :, length[req] : length[req] + 1]
        return k_new.to(DEV), v_new.to(DEV)

    def check(outs, q, gate, written):
        for layer in range(layers):
            for req, row in row_of.items():
                k, v = tokens(layer, req)
                n = written[req]
                ref = oracle_attn.dense_attention(q[row : row + 1].cpu(), k[:, :, :n], v[:, :, :n], position_offset=n - 1, gate=gate[row : row + 1].cpu())
                got = outs[layer][row : row + 1].cpu().float()
                torch.testing.assert_close(got, ref.transpose(1, 2).reshape(1, 1, heads * dim).float(), atol=2e-2, rtol=2e-2)
            free_rows = [r for r in range(tables.rows) if not tables.active[r]]
            for r in free_rows:
                assert torch.count_nonzero(outs[layer][r]) == 0

    for req, prompt in enumerate([37, 5, 80]):
        admit(req, prompt)
    for step in range(3):
        q = torch.randn(tables.rows, heads, 1, dim, generator=gen).to(torch.bfloat16).to(DEV)
        gate = torch.randn(tables.rows, 1, heads * dim, generator=gen).to(torch.bfloat16).to(DEV)
        tables.reserve_step()
        outs = []
        for layer, pool in enumerate(pools):
            k_new, v_new = step_inputs(layer)
            outs.append(ar.full_attention_decode_device(q, gate, k_new, v_new, pool.key_blocks, pool.value_blocks, tables, config, runtime))
        tables.check()
        for req in row_of:
            length[req] += 1
        check(outs, q, gate, length)
        if step == 1:
            released = tables.release_request(row_of.pop(1))
            assert len(released) == 1
            admit(3, 20)  # the freed row and the lowest free block ids
            assert row_of[3] == 1 and int(tables.block_tables[1, 0]) == min(released + tables.allocator.free_blocks() + [int(tables.block_tables[1, 0])])
    assert runtime.paged_attention_stats.native_hits == 3 * layers
    # the whole step in a HIP graph: fixed inputs, each replay appends them at the next position
    q = torch.randn(tables.rows, heads, 1, dim, generator=gen).to(torch.bfloat16).to(DEV)
    gate = torch.randn(tables.rows, 1, heads * dim, generator=gen).to(torch.bfloat16).to(DEV)
    fixed = [step_inputs(layer) for layer in range(layers)]
    for layer in range(layers):  # the reference tokens of the replays: the same K/V at every new position
        for req in row_of:
            k, v = tokens(layer, req)
            for r in range(3):
                k[0, :, length[req] + r] = fixed[layer][0][row_of[req], :, 0].cpu()
                v[0, :, length[req] + r] = fixed[layer][1][row_of[req], :, 0].cpu()

    def step():
        tables.reserve_step()
        return [ar.full_attention_decode_device(q, gate, fixed[layer][0], fixed[layer][1], pool.key_blocks, pool.value_blocks, tables, config,
                                                runtime, no_alloc=True) for layer, pool in enumerate(pools)]

    # first-call set-up of the no-alloc path (its scratch address) outside the capture: a read-only call
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        hip_ops.paged_attention_decode_batched_noalloc(q, tables.block_tables, pools[0].key_blocks, pools[0].value_blocks, tables.sequence_lengths, bs)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        graph_outs = step()
    print("graph captured", flush=True)
    for r in range(3):
        graph.replay()
        torch.cuda.synchronize()
        tables.check()
        for req in row_of:
            length[req] += 1
        check(graph_outs, q, gate, length)
