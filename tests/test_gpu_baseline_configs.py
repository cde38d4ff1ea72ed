"""The HIP path at BASELINE configs 2-5's own workloads (the seeded builders of ``bench.py``).

Configs 2-5 are what the benchmark times; these tests run the same launches on the same inputs
and check them against the oracle (``oracle/``):

* config 2 -- all 64 rows of the batched decode (1,024-wave balanced schedule, 74,100-block
  shuffled pool) against ``oracle.attention.paged_decode``;
* config 3 -- the whole 8 x 4096-token prefill in 512-token query chunks (K/V appended chunk by
  chunk, as the benchmark's step does), bit for bit equal to one launch over all 4096 tokens, and
  the first and last position of every chunk of every sequence, all heads, against the oracle's
  dense attention over the gathered prefix;
* config 4 -- the full B=4, T=8192, 16/32-head chunked delta rule: every row against the oracle
  layer core (128 chunks of state carry), and all rows against the fp32 token-serial HIP core on
  the same prepared inputs; plus a weak-decay T=8192 case whose state integrates across chunks;
* config 5 -- one 48-layer hybrid decode step: sampled rows of the first and last layer of each
  kind against the oracle.

Tolerances (north_star): bf16 outputs within 2e-2 absolute/relative, fp32 states within 1e-3
relative (Frobenius, per head), gathers bit-exact.  Each case prints its name and shape before
launching.
"""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

from oracle import attention as oracle_attn
from oracle import gated_delta as gd

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(autouse=True)
def _release_device_memory():
    """These workloads hold up to ~140 GB of device memory: hand it back after each test."""
    yield
    import gc

    gc.collect()
    torch.cuda.empty_cache()


def _say(msg: str) -> None:
    print(msg, flush=True)


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _gather_row(pool: torch.Tensor, table_row: torch.Tensor, tokens: int) -> torch.Tensor:
    """Dense ``(1, H_kv, tokens, D)`` K or V of one row of a shared ``(P, H_kv, bs, D)`` pool (on the device)."""
    bs = pool.shape[2]
    nb = (tokens + bs - 1) // bs
    blocks = pool.index_select(0, table_row[:nb].long())  # (nb, H_kv, bs, D)
    return blocks.transpose(0, 1).reshape(pool.shape[1], nb * bs, pool.shape[3])[:, :tokens].unsqueeze(0)


# ----------------------------------------------------------------------------- config 2


def test_config2_all_rows_match_oracle() -> None:
    import bench
    import hip_ops

    _say("config 2: building workload (64 rows, ctx U[1024, 32768], 74,100-block pool)")
    w = bench.decode_workload(DEV)
    out = hip_ops.paged_attention_decode_batched(w["query"], w["tables"], w["key_pool"], w["value_pool"], w["lens"], w["bs"])
    torch.cuda.synchronize()
    _say("config 2: decode done, checking 64 rows against oracle.attention.paged_decode")
    bs = w["bs"]
    ctx = [int(c) for c in w["ctx"]]
    tables = [w["tables_cpu"][b, : (c + bs - 1) // bs].tolist() for b, c in enumerate(ctx)]
    kp, vp = w["key_pool"].cpu(), w["value_pool"].cpu()
    ref = oracle_attn.paged_decode(w["query"].cpu(), [kp] * 64, [vp] * 64, tables, ctx, block_size=bs, pool_layout="phbd")
    torch.testing.assert_close(out.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)


# ----------------------------------------------------------------------------- config 3


def test_config3_chunked_prefill_matches_one_shot_and_oracle_samples() -> None:
    import bench
    import hip_ops

    _say("config 3: building workload (8 x 4096 new tokens, prefix U[0, 8192], chunk 512)")
    w = bench.prefill_workload(DEV)
    batch, new, chunk, bs = w["batch"], w["new"], w["chunk"], w["bs"]
    prefixes = [int(p) for p in w["prefixes"]]
    heads, dim = w["q"].shape[1], w["q"].shape[2]
    chunked = torch.empty_like(w["q"])
    for c0 in range(0, new, chunk):
        n = min(chunk, new - c0)
        starts = (w["prefixes"] + c0).to(device=DEV, dtype=torch.int32)
        cu = torch.arange(0, batch + 1, device=DEV, dtype=torch.int32) * n
        rows = torch.cat([torch.arange(b * new + c0, b * new + c0 + n) for b in range(batch)]).to(DEV)
        hip_ops.paged_kv_append(w["new_k"][:, :, c0 : c0 + n], w["new_v"][:, :, c0 : c0 + n], w["key_pool"], w["value_pool"], w["tables"],
                                starts, bs)
        out = hip_ops.paged_attention_prefill(w["q"].index_select(0, rows), cu, starts, w["key_pool"], w["value_pool"], w["tables"], bs,
                                              max_new=n, gate=w["gate"].index_select(0, rows))
        chunked.index_copy_(0, rows, out)
    _say("config 3: chunked run done; one launch over all 4096 new tokens")
    cu_all = torch.arange(0, batch + 1, device=DEV, dtype=torch.int32) * new
    one_shot = hip_ops.paged_attention_prefill(w["q"], cu_all, w["prefixes"].to(device=DEV, dtype=torch.int32), w["key_pool"], w["value_pool"],
                                               w["tables"], bs, max_new=new, gate=w["gate"])
    torch.cuda.synchronize()
    assert torch.equal(chunked, one_shot)
    _say("config 3: chunked == one-shot bit for bit; sampled rows against the oracle")
    for b in range(batch):
        total = prefixes[b] + new
        k = _gather_row(w["key_pool"], w["tables"][b], total).cpu()
        v = _gather_row(w["value_pool"], w["tables"][b], total).cpu()
        # the appended tokens are exactly the workload's new K/V, bit for bit
        assert torch.equal(k[0, :, prefixes[b] :], w["new_k"][b].cpu()) and torch.equal(v[0, :, prefixes[b] :], w["new_v"][b].cpu())
        for c0 in range(0, new, chunk):
            for n in (c0, min(new, c0 + chunk) - 1):
                row = b * new + n
                q = w["q"][row].cpu().reshape(1, heads, 1, dim)
                gate = w["gate"][row].cpu().reshape(1, 1, heads * dim)
                ref = oracle_attn.dense_attention(q, k, v, position_offset=prefixes[b] + n, gate=gate)
                torch.testing.assert_close(chunked[row].cpu().float(), ref[0, :, 0].float(), atol=2e-2, rtol=2e-2)


# ----------------------------------------------------------------------------- config 4


def _prepared_inputs_on_device(mixed, a, b, a_log, dt_bias, conv_w, shape: gd.LinearShape):
    """The recurrence's inputs for rows of a linear-attention layer, on the device: the reference
    layer's conv + SiLU, split, gating, head repeat, L2 norm, q scale and head-major transpose
    (``src/reference_ops.py:240-283``, ``src/tp_runtime.py:2790-2805``) as torch operations, to feed
    the fp32 token-serial HIP core."""
    batch, seq, channels = mixed.shape
    taps = shape.conv_kernel_dim
    x = F.pad(mixed.float(), (0, 0, taps - 1, 0))  # (B, taps - 1 + T, C): zero history
    w = conv_w.float().reshape(channels, taps)
    # depthwise causal conv as a sum of shifted products (no MIOpen kernel build on the device)
    acc = torch.zeros(batch, seq, channels, device=mixed.device)
    for i in range(taps):
        acc += w[:, i] * x[:, i : i + seq]
    conv = F.silu(acc)
    q, k, v = torch.split(conv, [shape.key_dim, shape.key_dim, shape.value_state_dim], dim=-1)
    rep = shape.value_heads // shape.key_heads
    q = q.reshape(batch, seq, shape.key_heads, 128).repeat_interleave(rep, dim=2)
    k = k.reshape(batch, seq, shape.key_heads, 128).repeat_interleave(rep, dim=2)
    v = v.reshape(batch, seq, shape.value_heads, 128)
    g = -a_log.float().exp() * F.softplus(a.float() + dt_bias.float())
    beta = torch.sigmoid(b.float())

    def l2(t):
        return t * (t * t).sum(dim=-1, keepdim=True).add(1e-6).rsqrt()

    pq = (l2(q) * 128**-0.5).transpose(1, 2).contiguous()
    pk = l2(k).transpose(1, 2).contiguous()
    pv = v.transpose(1, 2).contiguous()
    state = torch.zeros(batch, shape.value_heads, 128, 128, device=mixed.device)
    return pq, pk, pv, g.transpose(1, 2).contiguous(), beta.transpose(1, 2).contiguous(), state


def _per_head_state_rel(got: torch.Tensor, want: torch.Tensor) -> float:
    got = got.detach().double().cpu().flatten(2)
    want = want.detach().double().cpu().flatten(2)
    return float(((got - want).norm(dim=-1) / want.norm(dim=-1).clamp_min(1e-30)).max())


@pytest.fixture(scope="module")
def config4_run():
    """One config-4 launch (the benchmark's seeded workload); its outputs, the inputs the oracle
    needs and the final states, on the host.  The HIP token-serial core check runs here too, on
    all four rows, while the workload is on the device."""
    import bench
    import hip_ops

    _say("config 4: building workload (B=4, T=8192, 16 key / 32 value heads)")
    w = bench.delta_workload(DEV)
    shape = gd.LinearShape(w["key_heads"], w["value_heads"], 128, 128, 4)
    out, state, tail = hip_ops.chunk_gated_delta_rule(w["mixed"], w["a"], w["b"], w["a_log"], w["dt_bias"], w["conv_w"], key_heads=w["key_heads"],
                                                      value_heads=w["value_heads"])
    torch.cuda.synchronize()
    _say("config 4: chunked prefill done; all rows against the fp32 token-serial HIP core")
    prep = _prepared_inputs_on_device(w["mixed"], w["a"], w["b"], w["a_log"], w["dt_bias"], w["conv_w"], shape)
    rec_out, rec_state = hip_ops.linear_attention_recurrent_core(*prep)
    torch.testing.assert_close(out.float(), rec_out.transpose(1, 2), atol=2e-2, rtol=2e-2)
    assert _per_head_state_rel(state, rec_state) < 1e-3
    del prep, rec_out, rec_state
    inputs = {k: w[k].cpu() for k in ("mixed", "a", "b", "a_log", "dt_bias", "conv_w")}
    result = {"shape": shape, "out": out.cpu(), "state": state.cpu(), "tail": tail.cpu(), **inputs}
    del w, out, state, tail
    return result


@pytest.mark.parametrize("row", [0, 1, 2, 3])
def test_config4_full_chunked_prefill_row_matches_oracle(config4_run, row) -> None:
    """Each row of the full config-4 launch against the oracle layer core (8192-token loop, 128
    chunks of state carry): bf16 core within 2e-2, fp32 state within 1e-3 per head, conv tail
    bit-exact."""
    r = config4_run
    _say(f"config 4: row {row} against the oracle layer core (8192-token loop)")
    sl = slice(row, row + 1)
    ref_core, ref_state, ref_tail = gd.linear_attention_core(r["mixed"][sl].float(), r["a"][sl].float(), r["b"][sl].float(), r["a_log"],
                                                             r["dt_bias"], r["conv_w"], r["shape"])
    torch.testing.assert_close(r["out"][sl].float(), ref_core.float(), atol=2e-2, rtol=2e-2)
    assert _per_head_state_rel(r["state"][sl], ref_state) < 1e-3
    torch.testing.assert_close(r["tail"][sl], ref_tail, atol=0, rtol=0)


def test_long_weak_decay_state_carry_matches_recurrent_core() -> None:
    """T = 8192 with A_log = -5 (g ~ -0.005 per token, the state integrates ~200 tokens, so the
    chunk-to-chunk carry of the state dominates): chunked prefill vs the fp32 token-serial core."""
    import hip_ops

    shape = gd.LinearShape(key_heads=1, value_heads=2, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    seq = 8192
    _say(f"weak decay: B=1, T={seq}, 1 key / 2 value heads")
    gen = torch.Generator(device=DEV).manual_seed(47)
    mixed = torch.randn(1, seq, shape.qkv_dim, generator=gen, device=DEV).to(torch.bfloat16)
    a = torch.randn(1, seq, 2, generator=gen, device=DEV)
    b = torch.randn(1, seq, 2, generator=gen, device=DEV)
    a_log = torch.full((2,), -5.0, device=DEV)
    dt_bias = torch.zeros(2, device=DEV)
    conv_w = torch.randn(shape.qkv_dim, 4, generator=gen, device=DEV) * 0.5
    out, state, _ = hip_ops.chunk_gated_delta_rule(mixed, a, b, a_log, dt_bias, conv_w, key_heads=1, value_heads=2, out_dtype=torch.float32)
    prep = _prepared_inputs_on_device(mixed, a, b, a_log, dt_bias, conv_w, shape)
    rec_out, rec_state = hip_ops.linear_attention_recurrent_core(*prep)
    assert _per_head_state_rel(state, rec_state) < 1e-3
    assert _rel(out.transpose(1, 2), rec_out) < 5e-3
    torch.testing.assert_close(out.transpose(1, 2), rec_out, atol=2e-2, rtol=2e-2)


# ----------------------------------------------------------------------------- config 5


def test_config5_hybrid_step_sampled_rows_match_oracle() -> None:
    import bench
    import hip_ops

    _say("config 5: building workload (48 layers, B=128, ctx U[256, 65536]; ~137 GB)")
    w = bench.hybrid_workload(DEV)
    x = w["inputs"]
    bs, groups = w["bs"], w["groups"]
    shape = gd.LinearShape(w["key_heads"], x["a"].shape[1], 128, 128, 4)
    rows = [0, 1, 37, 64, 101, 127]
    lin_check = {0: None, 3 * groups - 1: None}
    full_check = {0: None, groups - 1: None}
    # the sampled rows' linear state and conv tail before the step (the step updates them in place)
    before = {i: (w["linear"][i]["state"][rows].cpu(), w["linear"][i]["conv"][rows].cpu()) for i in lin_check}
    for g in range(groups):
        for j in range(3):
            i = 3 * g + j
            lin = w["linear"][i]
            o = hip_ops.gated_delta_step_conv(x["mixed"], lin["conv"], lin["conv_w"], x["a"], x["b"], lin["a_log"], lin["dt_bias"], lin["state"],
                                              key_heads=w["key_heads"])
            if i in lin_check:
                lin_check[i] = o
        full = w["full"][g]
        hip_ops.paged_kv_append(x["new_k"], x["new_v"], full["key_pool"], full["value_pool"], full["tables"], x["positions"], bs)
        o = hip_ops.paged_attention_decode_batched(x["query"], full["tables"], full["key_pool"], full["value_pool"], x["lens"], bs)
        if g in full_check:
            full_check[g] = o
    torch.cuda.synchronize()
    _say("config 5: step done; sampled rows of layers against the oracle")
    lens = x["lens"].cpu()
    for g, o in full_check.items():
        full = w["full"][g]
        for r in rows:
            n = int(lens[r])
            k = _gather_row(full["key_pool"], full["tables"][r], n).cpu()
            v = _gather_row(full["value_pool"], full["tables"][r], n).cpu()
            assert torch.equal(k[0, :, -1], x["new_k"][r, :, 0].cpu()) and torch.equal(v[0, :, -1], x["new_v"][r, :, 0].cpu())
            ref = oracle_attn.dense_attention(x["query"][r : r + 1].cpu(), k, v, position_offset=n - 1)
            torch.testing.assert_close(o[r : r + 1].cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)
    for i, o in lin_check.items():
        lin = w["linear"][i]
        state0, tail0 = before[i]
        ref_core, ref_state, ref_tail = gd.linear_attention_core(
            x["mixed"][rows].float().cpu().unsqueeze(1), x["a"][rows].float().cpu().unsqueeze(1), x["b"][rows].float().cpu().unsqueeze(1),
            lin["a_log"].cpu(), lin["dt_bias"].cpu(), lin["conv_w"].cpu(), shape, conv_tail=tail0, initial_state=state0,
        )
        torch.testing.assert_close(o[rows].cpu().float(), ref_core[:, 0].float(), atol=2e-2, rtol=2e-2)
        assert _per_head_state_rel(lin["state"][rows], ref_state) < 1e-3
        torch.testing.assert_close(lin["conv"][rows].cpu(), ref_tail, atol=0, rtol=0)
