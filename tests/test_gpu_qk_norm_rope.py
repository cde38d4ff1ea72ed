"""``hip_ops.qk_norm_rope_kv_append`` (q/k RMSNorm (1 + w) + partial rotary + K/V append) on the
GPU against ``oracle/rope.py`` and against vectors the reference's ``full_attention`` wrote.

Tolerances: q and k are bf16 outputs, within 2e-2 absolute and relative; in practice they
differ from the oracle by at most one bf16 ulp where libm's cos/sin or the order of the
mean-of-squares sum rounds differently, so the test also requires 99% of the elements to be
bit-identical.  Slot placement and the v copy are bit-exact, and every slot that is not
written keeps its sentinel.
"""

from __future__ import annotations

import pytest
import torch

from golden_io import bf16, load
from oracle import attention as oa
from oracle import rope

pytestmark = pytest.mark.gpu

DEV = "cuda:0"
THETA = 10_000_000.0
FACTOR = 0.25
EPS = 1e-6


def _build(seed: int, prefixes: list[int], news: list[int], heads: int, kv_heads: int, dim: int, bs: int = 16, idx=torch.int32):
    gen = torch.Generator().manual_seed(seed)
    batch = len(news)
    tokens = sum(news)
    need = [(p + n + bs - 1) // bs for p, n in zip(prefixes, news)]
    pool_blocks = sum(need) + 3
    perm = torch.randperm(pool_blocks, generator=gen)
    tables = torch.full((batch, max(need)), -1, dtype=idx)
    cur = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[cur : cur + n].to(idx)
        cur += n
    q_proj = torch.randn(tokens, heads, 2 * dim, generator=gen).to(torch.bfloat16)
    k_proj = torch.randn(tokens, kv_heads, dim, generator=gen).to(torch.bfloat16)
    v_proj = torch.randn(tokens, kv_heads, dim, generator=gen).to(torch.bfloat16)
    qw = (torch.randn(dim, generator=gen) * 0.1).to(torch.bfloat16)
    kw = (torch.randn(dim, generator=gen) * 0.1).to(torch.bfloat16)
    cu = torch.tensor([0] + list(torch.tensor(news).cumsum(0)), dtype=idx)
    starts = torch.tensor(prefixes, dtype=idx)
    sentinel = torch.full((pool_blocks, kv_heads, bs, dim), 7.0, dtype=torch.bfloat16)
    return dict(q_proj=q_proj, k_proj=k_proj, v_proj=v_proj, qw=qw, kw=kw, cu=cu, starts=starts, tables=tables, pool=sentinel, bs=bs,
                news=news, prefixes=prefixes, dim=dim)


def _positions(case) -> torch.Tensor:
    return torch.cat([torch.arange(p, p + n) for p, n in zip(case["prefixes"], case["news"])])


def _run(case, table_positions: int = 131072):
    import hip_ops

    kp = case["pool"].clone().to(DEV)
    vp = case["pool"].clone().to(DEV)
    q, gate = hip_ops.qk_norm_rope_kv_append(
        case["q_proj"].to(DEV), case["k_proj"].to(DEV), case["v_proj"].to(DEV), case["qw"].to(DEV), case["kw"].to(DEV), kp, vp,
        case["tables"].to(DEV), case["cu"].to(DEV), case["starts"].to(DEV), case["bs"], max_new=max(case["news"]), eps=EPS,
        rope_theta=THETA, partial_rotary_factor=FACTOR, table_positions=table_positions,
    )
    torch.cuda.synchronize()
    return q.cpu(), gate.cpu(), kp.cpu(), vp.cpu()


def _mostly_bit_exact(out: torch.Tensor, ref: torch.Tensor) -> None:
    torch.testing.assert_close(out.float(), ref.float(), atol=2e-2, rtol=2e-2)
    same = (out.view(torch.int16) == ref.view(torch.int16)).float().mean().item()
    assert same >= 0.99, f"only {same:.4f} of the elements are bit-identical"


@pytest.mark.parametrize("idx", [torch.int32, torch.int64])
def test_ragged_prefill_rows_match_oracle_and_land_in_their_slots(idx) -> None:
    case = _build(11, prefixes=[0, 5, 37, 300], news=[19, 1, 64, 33], heads=16, kv_heads=2, dim=256, idx=idx)
    q, gate, kp, vp = _run(case)
    dim = case["dim"]
    pos = _positions(case)
    q_ref, k_ref = rope.qk_norm_rope(case["q_proj"][..., :dim], case["k_proj"], case["qw"], case["kw"], pos, eps=EPS, rope_theta=THETA,
                                     partial_rotary_factor=FACTOR)
    _mostly_bit_exact(q, q_ref)
    assert torch.equal(gate, case["q_proj"][..., dim:])
    # k and v in their slots; every other slot keeps the sentinel
    expect_k = case["pool"].clone()
    expect_v = case["pool"].clone()
    n0 = 0
    for b, (p, n) in enumerate(zip(case["prefixes"], case["news"])):
        for t in range(n):
            blk, off = case["tables"][b, (p + t) // case["bs"]].item(), (p + t) % case["bs"]
            expect_k[blk, :, off] = k_ref[n0 + t]
            expect_v[blk, :, off] = case["v_proj"][n0 + t]
        n0 += n
    assert torch.equal(vp, expect_v)
    _mostly_bit_exact(kp, expect_k)
    untouched = (expect_k == case["pool"]).all(dim=-1)
    assert torch.equal(kp[untouched], case["pool"][untouched])


@pytest.mark.parametrize("table_positions", [131072, 8])  # 8: most positions past the cos/sin table
def test_one_token_per_row_decode_form_and_head_dim_128(table_positions) -> None:
    case = _build(12, prefixes=[0, 1, 15, 16, 1000], news=[1, 1, 1, 1, 1], heads=8, kv_heads=2, dim=128)
    q, _, kp, vp = _run(case, table_positions)
    q_ref, k_ref = rope.qk_norm_rope(case["q_proj"][..., :128], case["k_proj"], case["qw"], case["kw"], _positions(case), eps=EPS,
                                     rope_theta=THETA, partial_rotary_factor=FACTOR)
    _mostly_bit_exact(q, q_ref)
    for b, p in enumerate(case["prefixes"]):
        blk, off = case["tables"][b, p // 16].item(), p % 16
        _mostly_bit_exact(kp[blk, :, off], k_ref[b])
        assert torch.equal(vp[blk, :, off], case["v_proj"][b])


@pytest.mark.parametrize("name", ["full_attention_prefill", "full_attention_rope_d256"])
def test_matches_vectors_written_by_the_reference(name) -> None:
    import hip_ops

    v = load(name)
    batch, seq, heads, kv_heads, dim = (int(x) for x in v["shape"])
    theta, factor, eps, offset = (float(x) for x in v["rope"])
    bs = 16
    total = int(offset) + seq
    nblk = (total + bs - 1) // bs
    table = torch.arange(nblk, dtype=torch.int32).flip(0).view(1, -1)
    kp = torch.zeros(nblk, kv_heads, bs, dim, dtype=torch.bfloat16, device=DEV)
    vp = torch.zeros_like(kp)
    q_proj = bf16(v["q_proj_bf16"]).reshape(seq, heads, 2 * dim).to(DEV)
    k_proj = bf16(v["k_proj_bf16"]).reshape(seq, kv_heads, dim).to(DEV)
    v_proj = bf16(v["v_bf16"]).reshape(seq, kv_heads, dim).to(DEV)
    q, gate = hip_ops.qk_norm_rope_kv_append(
        q_proj, k_proj, v_proj, bf16(v["q_norm_bf16"]).to(DEV), bf16(v["k_norm_bf16"]).to(DEV), kp, vp, table.to(DEV),
        torch.tensor([0, seq], dtype=torch.int32, device=DEV), torch.tensor([int(offset)], dtype=torch.int32, device=DEV), bs, max_new=seq,
        eps=eps, rope_theta=theta, partial_rotary_factor=factor,
    )
    q_ref = bf16(v["q_bf16"])[0].transpose(0, 1)  # (S, H, D)
    k_ref = bf16(v["k_bf16"])[0].transpose(0, 1)  # (S, H_kv, D)
    _mostly_bit_exact(q.cpu(), q_ref)
    kp_c = kp.cpu()
    for t in range(seq):
        p = int(offset) + t
        _mostly_bit_exact(kp_c[table[0, p // bs].item(), :, p % bs], k_ref[t])
    if offset == 0:
        # the whole layer core: prologue, then paged prefill with the gate read in place from q_proj
        out = hip_ops.paged_attention_prefill(q, torch.tensor([0, seq], dtype=torch.int32, device=DEV),
                                              torch.tensor([0], dtype=torch.int32, device=DEV), kp, vp, table.to(DEV), bs, max_new=seq,
                                              gate=gate)
        torch.testing.assert_close(out.cpu().float(), bf16(v["out_bf16"])[0].float(), atol=2e-2, rtol=2e-2)


def test_rotary_dim_must_split_into_lane_groups() -> None:
    import hip_ops

    case = _build(13, prefixes=[0], news=[4], heads=2, kv_heads=1, dim=256)
    with pytest.raises(RuntimeError, match="rotary_dim"):
        hip_ops.qk_norm_rope_kv_append(
            case["q_proj"].to(DEV), case["k_proj"].to(DEV), case["v_proj"].to(DEV), case["qw"].to(DEV), case["kw"].to(DEV),
            case["pool"].to(DEV), case["pool"].clone().to(DEV), case["tables"].to(DEV), case["cu"].to(DEV), case["starts"].to(DEV), 16,
            max_new=4, eps=EPS, rope_theta=THETA, partial_rotary_factor=6 / 256,
        )


def test_prologue_then_prefill_equals_dense_oracle_on_a_ragged_batch() -> None:
    import hip_ops

    case = _build(14, prefixes=[0, 40], news=[48, 24], heads=16, kv_heads=2, dim=256)
    dim = case["dim"]
    # prefixes already in the pool: write them with the same prologue first
    pre = _build(15, prefixes=[0], news=[40], heads=16, kv_heads=2, dim=256)
    kp = case["pool"].clone().to(DEV)
    vp = case["pool"].clone().to(DEV)
    tables = case["tables"].to(DEV)
    pre_q = pre["q_proj"].to(DEV)
    hip_ops.qk_norm_rope_kv_append(pre_q, pre["k_proj"].to(DEV), pre["v_proj"].to(DEV), case["qw"].to(DEV), case["kw"].to(DEV), kp, vp,
                                   tables, torch.tensor([0, 0, 40], dtype=torch.int32, device=DEV),
                                   torch.tensor([0, 0], dtype=torch.int32, device=DEV), 16, max_new=40, eps=EPS, rope_theta=THETA,
                                   partial_rotary_factor=FACTOR)
    q, gate = hip_ops.qk_norm_rope_kv_append(
        case["q_proj"].to(DEV), case["k_proj"].to(DEV), case["v_proj"].to(DEV), case["qw"].to(DEV), case["kw"].to(DEV), kp, vp, tables,
        case["cu"].to(DEV), case["starts"].to(DEV), 16, max_new=48, eps=EPS, rope_theta=THETA, partial_rotary_factor=FACTOR,
    )
    out = hip_ops.paged_attention_prefill(q, case["cu"].to(DEV), case["starts"].to(DEV), kp, vp, tables, 16, max_new=48, gate=gate)
    # oracle: row 1's keys are its 40 prefix tokens then its 24 new ones, all normed and rotated
    q_ref, k_ref = rope.qk_norm_rope(case["q_proj"][..., :dim], case["k_proj"], case["qw"], case["kw"], _positions(case), eps=EPS,
                                     rope_theta=THETA, partial_rotary_factor=FACTOR)
    _, k_pre = rope.qk_norm_rope(pre["q_proj"][:, :, :dim], pre["k_proj"], case["qw"], case["kw"], torch.arange(40), eps=EPS,
                                 rope_theta=THETA, partial_rotary_factor=FACTOR)
    rows = [(0, 48, None, None), (48, 24, k_pre, pre["v_proj"])]
    for n0, n, kprev, vprev in rows:
        qb = q_ref[n0 : n0 + n].transpose(0, 1).unsqueeze(0)          # (1, H, n, D)
        kb = k_ref[n0 : n0 + n]
        vb = case["v_proj"][n0 : n0 + n]
        if kprev is not None:
            kb = torch.cat([kprev, kb])
            vb = torch.cat([vprev, vb])
        prefix = 0 if kprev is None else kprev.shape[0]
        ref = oa.dense_attention(qb, kb.transpose(0, 1).unsqueeze(0), vb.transpose(0, 1).unsqueeze(0), position_offset=prefix,
                                 gate=case["q_proj"][n0 : n0 + n, :, dim:].reshape(1, n, -1))
        torch.testing.assert_close(out[n0 : n0 + n].cpu().float(), ref[0].transpose(0, 1).float(), atol=2e-2, rtol=2e-2)
