"""Seeded randomized parity of the hot-path kernels against the CPU oracle.

Each case draws its own shapes from a fixed seed, so a failure names a reproducible case:
batch sizes, context and prefix lengths around the 16-token block and 64-token chunk
boundaries, both head dims, GQA groups 1..16, int32 and int64 index arrays, table entries
that are -1 or past the pool inside a row, rows with no tokens, and the chunked delta rule
with and without carried states.  Tolerances as in the per-kernel tests: bf16 outputs within
2e-2 absolute/relative, fp32 states within 1e-3 relative (Frobenius), conv tails bit-exact.
"""

from __future__ import annotations

import random

import pytest
import torch

from oracle import attention as oracle_attn
from oracle import gated_delta as gd

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
BS = 16


def _ops():
    import hip_ops

    return hip_ops


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def _length(rng: random.Random, hi: int) -> int:
    # favour the block boundaries: 0, 1, 16k - 1, 16k, 16k + 1
    if rng.random() < 0.5:
        k = rng.randint(0, max(1, hi // BS))
        return max(0, min(hi, BS * k + rng.choice((-1, 0, 1))))
    return rng.randint(0, hi)


@pytest.mark.parametrize("seed", range(8))
def test_randomized_batched_decode_matches_oracle(seed) -> None:
    ops = _ops()
    rng = random.Random(1000 + seed)
    gen = torch.Generator().manual_seed(1000 + seed)
    dim = rng.choice((128, 256))
    kv_heads = rng.choice((1, 2, 4))
    group = rng.choice((1, 2, 4, 8, 16) if kv_heads <= 2 else (1, 2, 4))
    heads = kv_heads * group
    batch = rng.randint(1, 9)
    lens = [_length(rng, 1200) for _ in range(batch)]
    need = [(n + BS - 1) // BS for n in lens]
    pool_blocks = sum(need) + 8
    max_blocks = max(need + [1]) + rng.randint(0, 3)
    table_dtype = rng.choice((torch.int32, torch.int64))
    lens_dtype = rng.choice((torch.int32, torch.int64))
    kp = torch.randn(pool_blocks, kv_heads, BS, dim, generator=gen).to(torch.bfloat16)
    vp = torch.randn(pool_blocks, kv_heads, BS, dim, generator=gen).to(torch.bfloat16)
    q = torch.randn(batch, heads, 1, dim, generator=gen).to(torch.bfloat16)
    perm = torch.randperm(pool_blocks, generator=gen).tolist()
    tables = torch.full((batch, max_blocks), -1, dtype=torch.long)
    kept_tables, kept_lens, cursor = [], [], 0
    for row, n in enumerate(lens):
        t = perm[cursor : cursor + need[row]]
        cursor += need[row]
        tables[row, : len(t)] = torch.tensor(t, dtype=torch.long)
        keep, kept_len = list(t), n
        # a full block inside the row replaced by -1 or by an id past the pool: that block is skipped
        if len(t) >= 3 and n % BS == 0 and rng.random() < 0.5:
            j = rng.randrange(len(t) - 1)
            tables[row, j] = rng.choice((-1, pool_blocks + rng.randint(0, 50)))
            del keep[j]
            kept_len -= BS
        kept_tables.append(keep)
        kept_lens.append(kept_len)
    ref = oracle_attn.paged_decode(q, [kp] * batch, [vp] * batch, kept_tables, kept_lens, block_size=BS, pool_layout="phbd", cast_probs=False)
    out = ops.paged_attention_decode_batched(q.to(DEV), tables.to(DEV, table_dtype), kp.to(DEV), vp.to(DEV),
                                             torch.tensor(lens, device=DEV, dtype=lens_dtype), BS)
    for row, n in enumerate(kept_lens):
        if n == 0:
            assert torch.count_nonzero(out[row]) == 0, f"case {seed}: row {row} has no tokens"
    torch.testing.assert_close(out.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2, msg=lambda m: f"case {seed} (D={dim}, G={group}, lens={lens}): {m}")


@pytest.mark.parametrize("seed", range(6))
def test_randomized_paged_prefill_matches_oracle(seed) -> None:
    ops = _ops()
    rng = random.Random(2000 + seed)
    gen = torch.Generator().manual_seed(2000 + seed)
    dim = rng.choice((128, 256))
    kv_heads = rng.choice((1, 2))
    group = rng.choice((1, 2, 4, 8))
    heads = kv_heads * group
    batch = rng.randint(1, 4)
    prefixes = [_length(rng, 300) for _ in range(batch)]
    news = [max(1, _length(rng, 90)) for _ in range(batch)]
    totals = [p + n for p, n in zip(prefixes, news)]
    need = [(t + BS - 1) // BS for t in totals]
    pool_blocks = sum(need) + 4
    perm = torch.randperm(pool_blocks, generator=gen).tolist()
    idx_dtype = rng.choice((torch.int32, torch.int64))
    table_dtype = rng.choice((torch.int32, torch.int64))
    tables, cursor = [], 0
    table_t = torch.full((batch, max(need)), -1, dtype=torch.long)
    for row, n in enumerate(need):
        tables.append(perm[cursor : cursor + n])
        table_t[row, :n] = torch.tensor(tables[-1], dtype=torch.long)
        cursor += n
    kp = torch.randn(pool_blocks, kv_heads, BS, dim, generator=gen).to(torch.bfloat16)
    vp = torch.randn(pool_blocks, kv_heads, BS, dim, generator=gen).to(torch.bfloat16)
    q = torch.randn(sum(news), heads, dim, generator=gen).to(torch.bfloat16)
    gate = torch.randn(sum(news), heads * dim, generator=gen).to(torch.bfloat16) if rng.random() < 0.5 else None
    cu = [0]
    for n in news:
        cu.append(cu[-1] + n)
    out = ops.paged_attention_prefill(q.to(DEV), torch.tensor(cu, device=DEV, dtype=idx_dtype), torch.tensor(prefixes, device=DEV, dtype=idx_dtype),
                                      kp.to(DEV), vp.to(DEV), table_t.to(DEV, table_dtype), BS, max_new=max(news),
                                      gate=None if gate is None else gate.to(DEV))
    refs = oracle_attn.paged_prefill(q, kp, vp, tables, prefixes, news, block_size=BS, gate=gate)
    torch.testing.assert_close(out.cpu().float(), torch.cat(refs).float(), atol=2e-2, rtol=2e-2,
                               msg=lambda m: f"case {seed} (D={dim}, G={group}, prefixes={prefixes}, news={news}): {m}")


@pytest.mark.parametrize("seed", range(4))
def test_randomized_chunked_delta_rule_matches_oracle(seed) -> None:
    ops = _ops()
    rng = random.Random(3000 + seed)
    gen = torch.Generator().manual_seed(3000 + seed)
    key_heads = rng.choice((1, 2))
    value_heads = key_heads * rng.choice((1, 2))
    shape = gd.LinearShape(key_heads=key_heads, value_heads=value_heads, key_head_dim=128, value_head_dim=128, conv_kernel_dim=4)
    batch = rng.randint(1, 2)
    seq = rng.choice((1, 63, 64, 65, 129, rng.randint(2, 260)))
    mixed = torch.randn(batch, seq, shape.qkv_dim, generator=gen).to(torch.bfloat16)
    a = torch.randn(batch, seq, value_heads, generator=gen)
    b = torch.randn(batch, seq, value_heads, generator=gen)
    a_log = torch.randn(value_heads, generator=gen) * 0.5
    dt_bias = torch.randn(value_heads, generator=gen) * 0.5
    w = torch.randn(shape.qkv_dim, 1, 4, generator=gen) * 0.5
    carried = rng.random() < 0.5
    state0 = torch.randn(batch, value_heads, 128, 128, generator=gen) * 0.05 if carried else None
    tail0 = torch.randn(batch, shape.qkv_dim, 3, generator=gen) if carried else None
    ref_core, ref_state, ref_tail = gd.linear_attention_core(mixed.float(), a, b, a_log, dt_bias, w, shape, conv_tail=tail0, initial_state=state0)
    out, state, tail = ops.chunk_gated_delta_rule(
        mixed.to(DEV), a.to(DEV), b.to(DEV), a_log.to(DEV), dt_bias.to(DEV), w.to(DEV), key_heads=key_heads, value_heads=value_heads,
        conv_state=None if tail0 is None else tail0.to(DEV), initial_state=None if state0 is None else state0.to(DEV),
    )
    case = f"case {seed} (B={batch}, T={seq}, heads {key_heads}/{value_heads}, carried={carried})"
    torch.testing.assert_close(out.cpu().float(), ref_core.float(), atol=2e-2, rtol=2e-2, msg=lambda m: f"{case}: {m}")
    assert _rel(state, ref_state) < 1e-3, case
    torch.testing.assert_close(tail.cpu(), ref_tail, atol=0, rtol=0, msg=lambda m: f"{case}: {m}")
