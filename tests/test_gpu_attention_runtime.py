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
                                    tables.block_tables[row : row + 1], torch.zeros(1, dtype=torch.int32, device=DEV), bs)

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


THETA, FACTOR, EPS = 10_000_000.0, 0.25, 1e-6


def test_prefill_and_decode_from_projection_outputs_match_oracle() -> None:
    """The full-attention layer from its projection outputs through the runtime: two chunked
    prefill steps of a ragged batch (prefixes 0 and not block multiples, rows out of order, a row
    left empty), then decode steps from projection outputs -- q/k RMSNorm (1 + w) + partial RoPE +
    append in one launch, attention over the cache, the output gate read in place from q_proj --
    each against the oracle's norm/rope and dense causal attention over the tokens written so far
    (bf16 outputs, 2e-2).  GQA 16/2, D = 256, block size 16."""
    from decode_state import DeviceBatchPageTables
    from oracle import rope

    gen = torch.Generator().manual_seed(65)
    heads, kv_heads, dim, bs = 16, 2, 256, 16
    config = _enabled(heads, kv_heads, dim)
    rope_cfg = ar.RopeConfig(rms_norm_eps=EPS, rope_theta=THETA, partial_rotary_factor=FACTOR)
    pool = SharedKVBlockPool(48, kv_heads, dim, block_size=bs, device=DEV)
    tables = DeviceBatchPageTables(pool, rows=4, max_blocks=12)
    runtime = ar.HotPathRuntime()
    qw = (torch.randn(dim, generator=gen) * 0.1).to(torch.bfloat16)
    kw = (torch.randn(dim, generator=gen) * 0.1).to(torch.bfloat16)
    hist_k = {r: torch.zeros(0, kv_heads, dim, dtype=torch.bfloat16) for r in range(3)}
    hist_v = {r: torch.zeros(0, kv_heads, dim, dtype=torch.bfloat16) for r in range(3)}
    for _ in range(3):
        tables.add_request(0)

    def projections(tokens):
        q_proj = torch.randn(tokens, heads * 2 * dim, generator=gen).to(torch.bfloat16)
        k_proj = torch.randn(tokens, kv_heads * dim, generator=gen).to(torch.bfloat16)
        v_proj = torch.randn(tokens, kv_heads * dim, generator=gen).to(torch.bfloat16)
        return q_proj, k_proj, v_proj

    def expected(q_proj, k_proj, v_proj, rows, counts):
        """Per row: the oracle's q/k after norm and rope at the row's positions, the K/V history
        extended by the step, and dense causal attention with the gate."""
        outs, off = [], 0
        q3 = q_proj.view(-1, heads, 2 * dim)
        for row, n in zip(rows, counts):
            prefix = hist_k[row].shape[0]
            positions = torch.arange(prefix, prefix + n)
            q, k = rope.qk_norm_rope(q3[off : off + n, :, :dim], k_proj[off : off + n].view(n, kv_heads, dim), qw, kw, positions,
                                     eps=EPS, rope_theta=THETA, partial_rotary_factor=FACTOR)
            hist_k[row] = torch.cat([hist_k[row], k])
            hist_v[row] = torch.cat([hist_v[row], v_proj[off : off + n].view(n, kv_heads, dim)])
            gate = q3[off : off + n, :, dim:].reshape(1, n, heads * dim)
            ref = oracle_attn.dense_attention(q.transpose(0, 1).unsqueeze(0), hist_k[row].transpose(0, 1).unsqueeze(0),
                                              hist_v[row].transpose(0, 1).unsqueeze(0), position_offset=prefix, gate=gate)
            outs.append(ref[0].transpose(0, 1).reshape(n, heads * dim))
            off += n
        return torch.cat(outs)

    for rows, counts in (([0, 1, 2], [37, 5, 80]), ([2, 0], [19, 16])):
        step = tables.reserve_prefill(rows, counts)
        assert step.starts.cpu().tolist() == [hist_k[r].shape[0] for r in rows]
        q_proj, k_proj, v_proj = projections(sum(counts))
        out = ar.full_attention_prefill_device(q_proj.to(DEV), k_proj.to(DEV), v_proj.to(DEV), qw.to(DEV), kw.to(DEV), pool.key_blocks,
                                               pool.value_blocks, step, config, runtime, rope_cfg)
        assert out is not None and out.shape == (sum(counts), heads * dim)
        ref = expected(q_proj, k_proj, v_proj, rows, counts)
        torch.testing.assert_close(out.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)
    assert tables.sequence_lengths.cpu().tolist() == [53, 5, 99, 0]
    for _ in range(2):
        tables.reserve_step()
        q_proj, k_proj, v_proj = projections(tables.rows)
        out = ar.full_attention_decode_step_device(q_proj.to(DEV), k_proj.to(DEV), v_proj.to(DEV), qw.to(DEV), kw.to(DEV), pool.key_blocks,
                                                   pool.value_blocks, tables, config, runtime, rope_cfg)
        tables.check()
        assert out is not None and out.shape == (tables.rows, 1, heads * dim)
        ref = expected(q_proj[:3], k_proj[:3], v_proj[:3], [0, 1, 2], [1, 1, 1])
        torch.testing.assert_close(out[:3, 0].cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)
        assert torch.count_nonzero(out[3]) == 0  # the row without a request
    stats = runtime.paged_attention_stats
    assert (stats.native_prefill_hits, stats.native_hits, stats.dense_fallbacks, stats.calls) == (2, 2, 0, 4)


def test_prefill_on_reference_layout_pools_keeps_the_dense_path() -> None:
    """The native prefill needs the shared GQA pool: a per-request (reference-layout) pool is
    counted as the reference's ``prefill_or_multitoken`` and nothing is written."""
    from decode_state import DeviceBatchPageTables

    heads, kv_heads, dim = 16, 2, 256
    config = _enabled(heads, kv_heads, dim)
    pool = SharedKVBlockPool(8, kv_heads, dim, block_size=16, device=DEV)
    tables = DeviceBatchPageTables(pool, rows=1, max_blocks=4)
    tables.add_request(0)
    step = tables.reserve_prefill([0], [3])
    ref_pool = torch.zeros(1, heads, 4, 16, dim, dtype=torch.bfloat16, device=DEV)
    runtime = ar.HotPathRuntime()
    q_proj = torch.randn(3, heads * 2 * dim, device=DEV).to(torch.bfloat16)
    kv = torch.randn(3, kv_heads * dim, device=DEV).to(torch.bfloat16)
    w = torch.zeros(dim, dtype=torch.bfloat16, device=DEV)
    assert ar.full_attention_prefill_device(q_proj, kv, kv, w, w, ref_pool, ref_pool, step, config, runtime) is None
    stats = runtime.paged_attention_stats
    assert (stats.fallback_prefill_or_multitoken, stats.dense_fallbacks, stats.native_prefill_hits) == (1, 1, 0)
    assert torch.count_nonzero(ref_pool) == 0


def test_admission_between_reserve_and_append_keeps_step_positions() -> None:
    from decode_state import DeviceBatchPageTables

    pool = SharedKVBlockPool(16, 2, 256, block_size=16, device=DEV)
    tables = DeviceBatchPageTables(pool, rows=3, max_blocks=4)
    tables.add_request(20)
    tables.reserve_step()
    before = tables.positions.cpu().tolist()
    tables.add_request(7)
    assert tables.positions.cpu().tolist() == before
    assert tables.sequence_lengths.cpu().tolist() == [21, 7, 0]


def test_linear_prefill_with_output_stage_matches_oracle() -> None:
    """``linear_attention_prefill`` with ``z`` and ``norm_weight`` applies the layer's gated
    RMSNorm + SiLU(z) to the chunked core (bf16 output, 2e-2)."""
    from oracle import gated_norm

    config = _enabled()
    lin = config.linear_attention
    shape = gd.LinearShape(lin.key_heads, lin.value_heads, lin.key_head_dim, lin.value_head_dim, lin.conv_kernel_dim)
    gen = torch.Generator().manual_seed(66)
    batch, seq = 2, 150
    mixed = torch.randn(batch, seq, shape.qkv_dim, generator=gen).to(torch.bfloat16)
    a = torch.randn(batch, seq, shape.value_heads, generator=gen)
    b = torch.randn(batch, seq, shape.value_heads, generator=gen)
    a_log = torch.randn(shape.value_heads, generator=gen) * 0.3
    dt_bias = torch.zeros(shape.value_heads)
    w = torch.randn(shape.qkv_dim, 1, 4, generator=gen) * 0.5
    z = torch.randn(batch, seq, shape.value_heads * 128, generator=gen).to(torch.bfloat16)
    norm_w = (1.0 + 0.1 * torch.randn(128, generator=gen)).to(torch.bfloat16)
    out, state, _ = ar.linear_attention_prefill(mixed.to(DEV), a.to(DEV), b.to(DEV), a_log.to(DEV), dt_bias.to(DEV), w.to(DEV), config,
                                                z=z.to(DEV), norm_weight=norm_w.to(DEV), eps=EPS)
    core, ref_state, _ = gd.linear_attention_core(mixed.float(), a, b, a_log, dt_bias, w, shape)
    ref = gated_norm.linear_attention_output(core.to(torch.bfloat16), z, norm_w, EPS)
    assert out.shape == (batch, seq, shape.value_heads * 128) and out.dtype == torch.bfloat16
    torch.testing.assert_close(out.cpu().float(), ref.reshape(batch, seq, -1).float(), atol=2e-2, rtol=2e-2)
    err = (state.cpu().double() - ref_state.double()).norm() / ref_state.double().norm()
    assert float(err) < 1e-3
