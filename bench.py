"""Benchmark of the MI355X attention hot path (one GPU).

Default workload: paged GQA decode, batch 64, 16 query
heads, 2 KV heads, head_dim 256, contexts uniform in [1024, 32768] (seed 0),
block size 16, bf16 Q/K/V from N(0, 1), physical blocks shuffled over a pool
of ceil(sum(ctx)/16 * 1.25) blocks, one query token per sequence.

A step is one ``paged_attention_decode_batched`` call over that batch, inputs
resident in HBM.  ``value`` is the algorithmic HBM rate of a step:
    bytes = sum_b ctx_b*H_kv*D*2(K,V)*2B + 2*B*H*D*2B (q, out) + sum_b ceil(ctx_b/16)*4B (table)
divided by the measured step time.  The JSON line also carries the roofline
of the dominant kernel, the CPU baseline (this repository's restatement of
the reference CPU path, on a bounded sample) and a secondary measurement of
the gated delta-rule chunked prefill when available.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

REPO_ROOT = Path(__file__).resolve().parent
PACKAGE_DIR = REPO_ROOT / "qwen3.6-2080ti_amd"
for _p in (REPO_ROOT, PACKAGE_DIR):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, GB/s
# HBM bytes per launch of the decode kernel from rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
# (profiles/decode_partial_mfma_config2.md, profiles/chunk_gated_delta_config4.md, profiles/gated_rms_norm_config4.md,
# profiles/paged_prefill_config3.md, profiles/qk_norm_rope_config3.md): FETCH_SIZE scaled by 2.0 and WRITE_SIZE by 1.0, the factors
# a plain 1 GiB device copy reads back in the same runs. Counters need rocprofv3, so the figures
# are the committed profile's, not measured live.
TRAFFIC_DECODE = 1959210677
TRAFFIC_DELTA = 831048182  # chunk_kernel alone; the step (with prep_kernel) moves 1,416,829,956
TRAFFIC_PREFILL = 888476672  # average over the eight per-chunk launches
TRAFFIC_PROLOGUE = 675674420
TRAFFIC_OUTPUT_NORM = 805417779
TRAFFIC_FP8_LINEAR = 29648896  # x-resident kernel (one launch), from profiles/fp8_linear_config5_batch.md
TRAFFIC_HYBRID = 122302416625  # config 5's 48-layer step: 12 x (kv append + paged decode + combine) + 36 delta steps
SECONDARY_WARM_MS = 100.0  # wall time of untimed steps before each secondary (config 3, 4, 5) measurement
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16/fp16 MFMA, TFLOP/s


def _log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def kernel_times(step, repeats: int, labels: tuple[str, ...]) -> dict[str, dict[str, float]]:
    """Average duration of each labelled kernel over ``repeats`` steps, from HIP events
    the library records on the launch stream around each launch (``qa_set_kernel_timing``)."""
    import torch

    import hip_loader

    torch.cuda.synchronize()
    # two untimed steps keep the GPU busy up to the first timed launch: started from an idle
    # GPU, the first launch reads several percent slow and skews a short average
    for _ in range(2):
        step()
    with hip_loader.KernelTiming() as timing:
        for _ in range(repeats):
            step()
        torch.cuda.synchronize()
        out = {}
        for label in labels:
            total_ms, launches = timing.read(label)
            if launches:
                out[label] = {"avg_ms": total_ms / launches, "launches_per_step": launches / repeats, "total_ms_per_step": total_ms / repeats}
    return out


# ----------------------------------------------------------------------------- config 2


def decode_workload(device: str, *, seed: int = 0, batch: int = 64, heads: int = 16, kv_heads: int = 2, dim: int = 256, bs: int = 16, lo: int = 1024, hi: int = 32768):
    import torch

    gen = torch.Generator().manual_seed(seed)
    ctx = torch.randint(lo, hi + 1, (batch,), generator=gen)
    need = [(int(c) + bs - 1) // bs for c in ctx]
    pool_blocks = math.ceil(int(ctx.sum()) / bs * 1.25)
    perm = torch.randperm(pool_blocks, generator=gen)
    max_blocks = max(need)
    tables = torch.full((batch, max_blocks), -1, dtype=torch.int32)
    cursor = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[cursor : cursor + n].to(torch.int32)
        cursor += n
    dgen = torch.Generator(device=device).manual_seed(seed)
    key_pool = torch.randn((pool_blocks, kv_heads, bs, dim), generator=dgen, device=device, dtype=torch.bfloat16)
    value_pool = torch.randn((pool_blocks, kv_heads, bs, dim), generator=dgen, device=device, dtype=torch.bfloat16)
    query = torch.randn((batch, heads, 1, dim), generator=dgen, device=device, dtype=torch.bfloat16)
    lens = ctx.to(device=device, dtype=torch.int32)
    algo_bytes = int(ctx.sum()) * kv_heads * dim * 2 * 2 + 2 * batch * heads * dim * 2 + sum(need) * 4
    return {
        "query": query,
        "tables": tables.to(device),
        "tables_cpu": tables,
        "key_pool": key_pool,
        "value_pool": value_pool,
        "lens": lens,
        "ctx": ctx,
        "bs": bs,
        "algo_bytes": algo_bytes,
        "pool_blocks": pool_blocks,
    }


def time_decode(w, steps: int, warmup: int):
    import torch

    import hip_ops

    def step():
        return hip_ops.paged_attention_decode_batched(w["query"], w["tables"], w["key_pool"], w["value_pool"], w["lens"], w["bs"])

    return _timed(step, steps, warmup, ("decode_partial_mfma", "decode_combine"))


def time_serving_step(w, steps: int, warmup: int) -> dict:
    """Config 2 as a serving decode step through the runtime's device-table path
    (``attention_runtime.full_attention_decode_device`` on ``decode_state.DeviceBatchPageTables``):
    one block reservation for the step (one new token per row), the new token's K/V appended,
    then the batched attention -- eager, and replayed from one captured HIP graph.  Appends land
    past the cached lengths (and in free blocks), so the primary measurement's cache is not
    disturbed.  Returns ms per step for both and per-kernel times."""
    import torch

    import attention_runtime as ar
    from decode_state import DeviceBatchPageTables, SharedKVBlockPool

    batch, bs = w["tables"].shape[0], w["bs"]
    extra = 16  # table columns for up to 256 new tokens per row
    kv_heads, dim = w["key_pool"].shape[1], w["key_pool"].shape[3]
    heads = w["query"].shape[1]
    used = set(int(v) for v in w["tables_cpu"][w["tables_cpu"] >= 0].tolist())
    pool = SharedKVBlockPool.from_tensors(w["key_pool"], w["value_pool"], free_blocks=[b for b in range(w["pool_blocks"]) if b not in used])
    tables = DeviceBatchPageTables(pool, rows=batch, max_blocks=w["tables"].shape[1] + extra)
    tables.adopt_rows(w["tables"], w["lens"])
    config = ar.parse_attention_config({"text_config": {
        "num_attention_heads": heads, "num_key_value_heads": kv_heads, "head_dim": dim, "attn_output_gate": False,
        "native_paged_attention": True, "linear_num_key_heads": 16, "linear_num_value_heads": 32, "linear_key_head_dim": 128,
        "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4}})
    runtime = ar.HotPathRuntime()
    gen = torch.Generator(device=w["tables"].device).manual_seed(5)
    k_new = torch.randn((batch, kv_heads, 1, dim), generator=gen, device=w["tables"].device, dtype=torch.bfloat16)
    v_new = torch.randn((batch, kv_heads, 1, dim), generator=gen, device=w["tables"].device, dtype=torch.bfloat16)

    def step():
        tables.reserve_step()
        return ar.full_attention_decode_device(w["query"], None, k_new, v_new, pool.key_blocks, pool.value_blocks, tables, config, runtime)

    eager_ms, kern = _timed(step, steps, warmup, ("kv_reserve", "decode_partial_mfma", "decode_combine"), timing_repeats=3)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(warmup):
        graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        graph.replay()
    end.record()
    torch.cuda.synchronize()
    tables.check()
    if runtime.paged_attention_stats.native_hits == 0:
        raise RuntimeError("serving step: the device decode path did not run")
    graph_ms = start.elapsed_time(end) / steps
    tokens_added = int((tables.sequence_lengths - w["lens"]).max().item())
    return {"eager_ms": eager_ms, "graph_ms": graph_ms, "kernels": kern, "tokens_added": tokens_added}


def reference_layout_workload(w: dict, device: str, *, seed: int = 11) -> dict:
    """Config 2's contexts in the reference engine's own cache layout: one pool per request,
    ``(1, heads, P_b, bs, D)`` fp32 with the KV heads repeated to the 16 query heads
    (``src/decode_state.py:37-44``, ``src/tp_runtime.py:518-525``), blocks shuffled inside each
    pool, handed to ``paged_attention_decode_batched`` as the reference's list of pools
    (``src/tp_runtime.py:626-643``).  ~31 GB of fp32 K/V."""
    import torch

    gen = torch.Generator().manual_seed(seed)
    dgen = torch.Generator(device=device).manual_seed(seed)
    heads, dim, bs = w["query"].shape[1], w["query"].shape[3], w["bs"]
    ctx = [int(c) for c in w["ctx"]]
    need = [(c + bs - 1) // bs for c in ctx]
    tables = torch.full((len(ctx), max(need)), -1, dtype=torch.int64)
    keys, values = [], []
    for b, n in enumerate(need):
        tables[b, :n] = torch.randperm(n, generator=gen)
        keys.append(torch.randn((1, heads, n, bs, dim), generator=dgen, device=device))
        values.append(torch.randn((1, heads, n, bs, dim), generator=dgen, device=device))
    query = w["query"].float()
    layout_bytes = sum(ctx) * heads * dim * 4 * 2 + 2 * len(ctx) * heads * dim * 4 + sum(need) * 8
    return {"query": query, "tables": tables.to(device), "keys": keys, "values": values, "lens": w["lens"].long(), "bs": bs,
            "layout_bytes": layout_bytes, "gqa_bytes": w["algo_bytes"]}


def time_reference_layout(rw: dict, steps: int, warmup: int):
    import hip_ops

    def step():
        return hip_ops.paged_attention_decode_batched(rw["query"], rw["tables"], rw["keys"], rw["values"], rw["lens"], rw["bs"])

    return _timed(step, steps, warmup, ("decode_partial_generic", "decode_combine"))


def _timed(step, steps: int, warmup: int, labels: tuple[str, ...], warm_ms: float = 0.0, timing_repeats: int = 5):
    """(ms per step over ``steps`` timed steps, per-kernel averages from a separate instrumented pass).

    ``warmup`` untimed steps run first, and more until ``warm_ms`` of wall time has passed: after
    the memory-bound decode measurement the GPU takes some tens of milliseconds of compute-heavy
    work to reach its steady clock, and a sub-millisecond step timed before that reads up to 15%
    slow."""
    import time

    import torch

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t_start = time.perf_counter()
    while (time.perf_counter() - t_start) * 1e3 < warm_ms:
        step()
        torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for _ in range(steps):
        step()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    return ms, kernel_times(step, max(1, min(steps, timing_repeats)), labels)


def cpu_baseline_decode(w, budget_s: float = 12.0):
    """Reference CPU decode (repeated heads, gather, dense fp32 softmax) on a sample of rows.

    Runs the restatement of the reference path (``oracle.attention.reference_layout_decode_cpu``)
    one sequence at a time until ``budget_s`` has elapsed; reports the
    algorithmic GB/s of the rows completed.
    """
    import torch

    from oracle import attention

    threads = torch.get_num_threads()
    bs = w["bs"]
    kv_heads = w["key_pool"].shape[1]
    dim = w["key_pool"].shape[3]
    heads = w["query"].shape[1]
    done_bytes = 0
    done_rows = 0
    elapsed = 0.0
    tables = w["tables_cpu"]
    for b in range(w["query"].shape[0]):
        n = int(w["ctx"][b])
        need = (n + bs - 1) // bs
        ids = tables[b, :need].long().to(w["key_pool"].device)
        # the reference cache holds fp32 post-repeat heads in its own pool (src/tp_runtime.py:518-525)
        k = w["key_pool"].index_select(0, ids).float().cpu().permute(1, 0, 2, 3)  # (H_kv, need, bs, D)
        v = w["value_pool"].index_select(0, ids).float().cpu().permute(1, 0, 2, 3)
        k = k.repeat_interleave(heads // kv_heads, dim=0).unsqueeze(0).contiguous()
        v = v.repeat_interleave(heads // kv_heads, dim=0).unsqueeze(0).contiguous()
        order = torch.randperm(need, generator=torch.Generator().manual_seed(b))
        pool_k = torch.empty_like(k)
        pool_v = torch.empty_like(v)
        pool_k[:, :, order] = k
        pool_v[:, :, order] = v
        q = w["query"][b : b + 1].float().cpu()
        t0 = time.perf_counter()
        attention.reference_layout_decode_cpu(q, [pool_k[0]], [pool_v[0]], [order.tolist()], [n], block_size=bs)
        elapsed += time.perf_counter() - t0
        done_rows += 1
        done_bytes += n * kv_heads * dim * 4 + 2 * heads * dim * 2 + need * 4
        del k, v, pool_k, pool_v
        if elapsed >= budget_s:
            break
    return {
        "value": round(done_bytes / elapsed / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{done_rows} of 64 config-2 sequences ({sum(int(w['ctx'][i]) for i in range(done_rows))} cached tokens), "
        f"reference fp32 repeated-head layout, shuffled table, index_select gather + dense fp32 softmax; "
        f"torch CPU threads={threads}, os.cpu_count()={os.cpu_count()}",
    }


def config1_inputs() -> dict:
    """BASELINE config 1's inputs, drawn once for every user (``cpu_baseline_config1`` and the GPU
    parity test ``tests/test_gpu_paged_decode.py``): batch 4, 16 q heads, 2 KV heads, D 256, 512
    cached tokens per row, block size 16, bf16 N(0, 1) Q/K/V, one ``torch.Generator`` seeded 0
    drawing the block permutation, then q, then the K and V pools.  The pool holds 128 physical
    blocks ``(128, H_kv, bs, D)``; row ``b``'s table is blocks ``perm[32 b : 32 b + 32]``."""
    import torch

    batch, heads, kv_heads, dim, ctx, bs, blocks = 4, 16, 2, 256, 512, 16, 128
    gen = torch.Generator().manual_seed(0)
    perm = torch.randperm(blocks, generator=gen)
    q = torch.randn((batch, heads, 1, dim), generator=gen).to(torch.bfloat16)
    key_pool = torch.randn((blocks, kv_heads, bs, dim), generator=gen).to(torch.bfloat16)
    value_pool = torch.randn((blocks, kv_heads, bs, dim), generator=gen).to(torch.bfloat16)
    return {"query": q, "key_pool": key_pool, "value_pool": value_pool, "tables": perm.reshape(batch, ctx // bs),
            "lens": [ctx] * batch, "bs": bs, "heads": heads, "kv_heads": kv_heads, "dim": dim, "ctx": ctx, "batch": batch}


def cpu_baseline_config1(device: str) -> dict:
    """BASELINE config 1 in full on the host (``config1_inputs``: the GPU parity test's inputs)
    through the reference's CPU decode as the engine runs it (fp32, repeated heads,
    ``index_select`` gather, dense softmax; ``oracle.attention.reference_layout_decode_cpu``).
    Reports the algorithmic GB/s of the config-2 formula (bf16 K/V bytes)."""
    import torch

    from oracle import attention

    c1 = config1_inputs()
    batch, heads, kv_heads, dim, ctx, bs = c1["batch"], c1["heads"], c1["kv_heads"], c1["dim"], c1["ctx"], c1["bs"]
    tables = c1["tables"].tolist()
    q = c1["query"].float()
    # each request's reference pool (heads after _repeat_kv, P, bs, D) in fp32 (src/decode_state.py:37-44,
    # src/tp_runtime.py:518-525); every row's table indexes the one 128-block pool, so one tensor serves all rows
    pool_k = c1["key_pool"].float().permute(1, 0, 2, 3).repeat_interleave(heads // kv_heads, dim=0).contiguous()
    pool_v = c1["value_pool"].float().permute(1, 0, 2, 3).repeat_interleave(heads // kv_heads, dim=0).contiguous()
    pools_k, pools_v = [pool_k] * batch, [pool_v] * batch
    attention.reference_layout_decode_cpu(q, pools_k, pools_v, tables, [ctx] * batch, block_size=bs)  # warm
    reps = 0
    t0 = time.perf_counter()
    while True:
        attention.reference_layout_decode_cpu(q, pools_k, pools_v, tables, [ctx] * batch, block_size=bs)
        reps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= 2.0:
            break
    algo = batch * ctx * kv_heads * dim * 2 * 2 + 2 * batch * heads * dim * 2 + batch * (ctx // bs) * 4
    return {"value": round(algo * reps / elapsed / 1e9, 4), "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "ms_per_step": round(elapsed / reps * 1e3, 3),
            "sample": f"config 1 in full (4 rows x 512 tokens, 128 shuffled blocks, seed 0), {reps} steps; reference fp32 repeated-head "
                      f"layout, index_select gather + dense fp32 softmax; torch CPU threads={torch.get_num_threads()}"}


def cpu_baseline_delta(dw: dict, budget_s: float = 30.0, piece: int = 256) -> dict:
    """BASELINE config 4 on the host through the reference's CPU layer core
    (``oracle.gated_delta.linear_attention_core``: fp32 conv1d + SiLU, gating, L2 norm, and the
    per-token ``recurrent_gated_delta_rule`` loop of ``src/reference_ops.py:291-322``) on the same
    seeded inputs as the GPU run, streamed ``piece`` tokens at a time with the conv tail and state
    carried (identical results to one call); stops at ``budget_s`` and reports tokens/s over the
    tokens done (all 4 x 8192 when the budget allows)."""
    import torch

    from oracle import gated_delta as gd

    shape = gd.LinearShape(dw["key_heads"], dw["value_heads"], 128, 128, 4)
    batch, seq = dw["batch"], dw["seq"]
    a_log, dt_bias = dw["a_log"].cpu(), dw["dt_bias"].cpu()
    conv_w = dw["conv_w"].cpu()
    tail = state = None
    done = 0
    elapsed = 0.0
    while done < seq and elapsed < budget_s:
        n = min(piece, seq - done)
        mixed = dw["mixed"][:, done : done + n].float().cpu()
        a = dw["a"][:, done : done + n].float().cpu()
        b = dw["b"][:, done : done + n].float().cpu()
        t0 = time.perf_counter()
        _core, state, tail = gd.linear_attention_core(mixed, a, b, a_log, dt_bias, conv_w, shape, conv_tail=tail, initial_state=state)
        elapsed += time.perf_counter() - t0
        done += n
    return {"value": round(batch * done / elapsed, 1), "unit": "tokens/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"config 4, {done} of {seq} tokens of all {batch} rows x {dw['value_heads']} value heads (same seeded inputs as the GPU "
                      f"run), reference layer core with the per-token recurrence loop, fp32; torch CPU threads={torch.get_num_threads()}, "
                      f"os.cpu_count()={os.cpu_count()}"}


# ----------------------------------------------------------------------------- config 4


def delta_flops(batch: int, seq: int, value_heads: int, chunk: int = 64, dk: int = 128, dv: int = 128) -> float:
    """Algorithmic FLOP of the chunked prefill (BASELINE config-4 formula).

    Per (chunk, value head): 2C^2(3dk + 2dv) + 6 C dk dv + C^3/3.
    """
    per = 2 * chunk * chunk * (3 * dk + 2 * dv) + 6 * chunk * dk * dv + chunk**3 / 3
    return per * batch * value_heads * (seq / chunk)


def delta_workload(device: str, *, seed: int = 0, batch: int = 4, seq: int = 8192, key_heads: int = 16, value_heads: int = 32):
    import torch

    channels = 2 * key_heads * 128 + value_heads * 128
    gen = torch.Generator(device=device).manual_seed(seed)
    mixed = torch.randn((batch, seq, channels), generator=gen, device=device, dtype=torch.bfloat16)
    a = torch.randn((batch, seq, value_heads), generator=gen, device=device, dtype=torch.bfloat16)
    b = torch.randn((batch, seq, value_heads), generator=gen, device=device, dtype=torch.bfloat16)
    # config 4: beta = sigmoid(N(0,1)), alpha = exp(-softplus(N(0,1))) -> A_log = 0, dt_bias = 0
    a_log = torch.zeros(value_heads, device=device)
    dt_bias = torch.zeros(value_heads, device=device)
    conv_w = torch.randn((channels, 4), generator=gen, device=device) * 0.5
    algo_bytes = mixed.numel() * 2 + 2 * a.numel() * 2 + batch * seq * value_heads * 128 * 2 + batch * value_heads * 128 * 128 * 4
    return {"mixed": mixed, "a": a, "b": b, "a_log": a_log, "dt_bias": dt_bias, "conv_w": conv_w, "key_heads": key_heads,
            "value_heads": value_heads, "batch": batch, "seq": seq, "flops": delta_flops(batch, seq, value_heads), "algo_bytes": algo_bytes}


def time_delta(w, steps: int, warmup: int) -> float:
    import torch

    import hip_ops

    def step():
        return hip_ops.chunk_gated_delta_rule(w["mixed"], w["a"], w["b"], w["a_log"], w["dt_bias"], w["conv_w"], key_heads=w["key_heads"],
                                              value_heads=w["value_heads"], keep_conv_state=False)

    return _timed(step, steps, warmup, ("chunk_prep", "chunk_gated_delta"), warm_ms=SECONDARY_WARM_MS)


# ----------------------------------------------------------------------------- config 3


def prefill_workload(device: str, *, seed: int = 0, batch: int = 8, new: int = 4096, heads: int = 16, kv_heads: int = 2, dim: int = 256,
                     bs: int = 16, max_prefix: int = 8192, chunk: int = 512):
    import torch

    gen = torch.Generator().manual_seed(seed)
    prefixes = torch.randint(0, max_prefix + 1, (batch,), generator=gen)
    totals = prefixes + new
    need = [(int(t) + bs - 1) // bs for t in totals]
    pool_blocks = math.ceil(sum(need) * 1.25)
    perm = torch.randperm(pool_blocks, generator=gen)
    tables = torch.full((batch, max(need)), -1, dtype=torch.int32)
    cursor = 0
    for b, n in enumerate(need):
        tables[b, :n] = perm[cursor : cursor + n].to(torch.int32)
        cursor += n
    dgen = torch.Generator(device=device).manual_seed(seed)
    key_pool = torch.randn((pool_blocks, kv_heads, bs, dim), generator=dgen, device=device, dtype=torch.bfloat16)
    value_pool = torch.randn((pool_blocks, kv_heads, bs, dim), generator=dgen, device=device, dtype=torch.bfloat16)
    q = torch.randn((batch * new, heads, dim), generator=dgen, device=device, dtype=torch.bfloat16)
    gate = torch.randn((batch * new, heads * dim), generator=dgen, device=device, dtype=torch.bfloat16)
    new_k = torch.randn((batch, kv_heads, new, dim), generator=dgen, device=device, dtype=torch.bfloat16)
    new_v = torch.randn((batch, kv_heads, new, dim), generator=dgen, device=device, dtype=torch.bfloat16)
    flops = sum(4 * heads * dim * (new * int(p) + new * (new + 1) / 2) for p in prefixes)
    # algorithmic bytes of one step: per launch (a query chunk of n tokens at c0) and row, the K/V of
    # the visible keys read once (prefix + c0 + n keys of 2 * kv_heads * dim bf16 each) with their
    # table entries, and the chunk's q, gate and output rows (bf16)
    algo_bytes = 0
    launches = 0
    for c0 in range(0, new, chunk):
        n = min(chunk, new - c0)
        launches += 1
        for p in prefixes:
            keys = int(p) + c0 + n
            algo_bytes += keys * 2 * kv_heads * dim * 2 + (keys + bs - 1) // bs * 4 + 3 * n * heads * dim * 2
    return {"q": q, "gate": gate, "new_k": new_k, "new_v": new_v, "key_pool": key_pool, "value_pool": value_pool, "tables": tables.to(device),
            "prefixes": prefixes, "batch": batch, "new": new, "chunk": chunk, "bs": bs, "flops": flops, "pool_blocks": pool_blocks,
            "algo_bytes": algo_bytes, "launches": launches}


def time_prefill(w, steps: int, warmup: int) -> float:
    """One step = the whole prefill batch in query chunks: append the chunk's K/V, then attend."""
    import torch

    import hip_ops

    device = w["q"].device
    batch, new, chunk = w["batch"], w["new"], w["chunk"]
    plan = []
    for c0 in range(0, new, chunk):
        n = min(chunk, new - c0)
        starts = (w["prefixes"] + c0).to(device=device, dtype=torch.int32)
        cu = torch.arange(0, batch + 1, device=device, dtype=torch.int32) * n
        rows = torch.cat([torch.arange(b * new + c0, b * new + c0 + n) for b in range(batch)]).to(device)
        plan.append((c0, n, starts, cu, w["q"].index_select(0, rows).contiguous(), w["gate"].index_select(0, rows).contiguous()))

    def step():
        for c0, n, starts, cu, q, gate in plan:
            hip_ops.paged_kv_append(w["new_k"][:, :, c0 : c0 + n], w["new_v"][:, :, c0 : c0 + n], w["key_pool"], w["value_pool"], w["tables"],
                                    starts, w["bs"])
            hip_ops.paged_attention_prefill(q, cu, starts, w["key_pool"], w["value_pool"], w["tables"], w["bs"], max_new=n, gate=gate)

    return _timed(step, steps, warmup, ("paged_prefill",), warm_ms=SECONDARY_WARM_MS)


def prologue_workload(pw: dict, device: str, *, seed: int = 1) -> dict:
    """The full-attention prologue (q/k RMSNorm + partial rotary + K/V append) over all of
    config 3's new tokens in one launch: q_proj (tokens, H, 2D), k/v_proj (tokens, H_kv, D)
    bf16, appended at positions prefix_b + n into config 3's pool and tables."""
    import torch

    batch, new, heads, dim = pw["batch"], pw["new"], pw["q"].shape[1], pw["q"].shape[2]
    kv_heads = pw["key_pool"].shape[1]
    tokens = batch * new
    dgen = torch.Generator(device=device).manual_seed(seed)
    q_proj = torch.randn((tokens, heads, 2 * dim), generator=dgen, device=device, dtype=torch.bfloat16)
    k_proj = torch.randn((tokens, kv_heads, dim), generator=dgen, device=device, dtype=torch.bfloat16)
    v_proj = torch.randn((tokens, kv_heads, dim), generator=dgen, device=device, dtype=torch.bfloat16)
    qw = (torch.randn((dim,), generator=dgen, device=device) * 0.1).to(torch.bfloat16)
    kw = (torch.randn((dim,), generator=dgen, device=device) * 0.1).to(torch.bfloat16)
    cu = torch.arange(0, batch + 1, device=device, dtype=torch.int32) * new
    starts = pw["prefixes"].to(device=device, dtype=torch.int32)
    # bytes: the q half of q_proj, k and v read; q, k and v written (2 bytes each)
    algo = 2 * tokens * dim * (heads + 2 * kv_heads) * 2
    return {"q_proj": q_proj, "k_proj": k_proj, "v_proj": v_proj, "qw": qw, "kw": kw, "cu": cu, "starts": starts, "new": new,
            "algo_bytes": algo, "tokens": tokens}


def time_prologue(w: dict, pw: dict, steps: int, warmup: int):
    import hip_ops

    def step():
        hip_ops.qk_norm_rope_kv_append(w["q_proj"], w["k_proj"], w["v_proj"], w["qw"], w["kw"], pw["key_pool"], pw["value_pool"], pw["tables"],
                                       w["cu"], w["starts"], pw["bs"], max_new=w["new"], eps=1e-6, rope_theta=10_000_000.0,
                                       partial_rotary_factor=0.25)

    return _timed(step, steps, warmup, ("qk_norm_rope",), warm_ms=SECONDARY_WARM_MS)


def output_norm_workload(device: str, *, seed: int = 2, batch: int = 4, seq: int = 8192, value_heads: int = 32, dim: int = 128) -> dict:
    """The linear-attention output stage (gated RMSNorm + SiLU(z)) over config 4's tokens: the bf16
    core the chunked prefill writes, the bf16 in_proj_z output and a bf16 norm weight, bf16 out."""
    import torch

    gen = torch.Generator(device=device).manual_seed(seed)
    core = torch.randn((batch, seq, value_heads, dim), generator=gen, device=device, dtype=torch.bfloat16)
    z = torch.randn((batch, seq, value_heads * dim), generator=gen, device=device, dtype=torch.bfloat16)
    w = (1.0 + 0.2 * torch.randn((dim,), generator=gen, device=device)).to(torch.bfloat16)
    # bytes: core and z read, out written (2 bytes each)
    algo = 3 * batch * seq * value_heads * dim * 2
    return {"core": core, "z": z, "w": w, "algo_bytes": algo, "rows": batch * seq * value_heads}


def time_output_norm(w: dict, steps: int, warmup: int):
    import hip_ops

    def step():
        hip_ops.gated_rms_norm(w["core"], w["z"], w["w"], 1e-6)

    # a 0.16 ms launch: average the per-kernel events over 20 launches rather than 5
    return _timed(step, steps, warmup, ("gated_rms_norm",), warm_ms=SECONDARY_WARM_MS, timing_repeats=20)


def fp8_linear_workload(device: str, *, seed: int = 3, rows: int = 128, out_features: int = 8192, in_features: int = 2048) -> dict:
    """An fp8 E4M3 block-scaled projection at config 5's decode batch: rows = 128 tokens, out =
    16 heads x 2 x 256 (q_proj with its gate half), in = a 2048 hidden size; fp32 input as the
    reference passes it (``hidden_states.float()``), fp32 output; the weight is packed once by
    ``fp8_pack_weight`` as a serving stack would at load time."""
    import torch

    import hip_ops

    gen = torch.Generator(device=device).manual_seed(seed)
    w = (0.5 * torch.randn((out_features, in_features), generator=gen, device=device)).to(torch.float8_e4m3fn)
    s = (0.05 + torch.rand((out_features // 128, in_features // 128), generator=gen, device=device)).to(torch.bfloat16)
    x = torch.randn((rows, in_features), generator=gen, device=device)
    # bytes: weight codes + scales + x read, y written
    algo = out_features * in_features + s.numel() * 2 + rows * in_features * 4 + rows * out_features * 4
    w = hip_ops.fp8_pack_weight(w)  # once, as at weight-load time
    return {"w": w, "s": s, "x": x, "algo_bytes": algo, "flops": 2.0 * rows * out_features * in_features,
            "rows": rows, "out": out_features, "in": in_features}


def time_fp8_linear(w: dict, steps: int, warmup: int):
    import hip_ops

    def step():
        hip_ops.fp8_e4m3_bf16_linear(w["x"], w["w"], w["s"])

    return _timed(step, steps, warmup, ("fp8_linear_cast", "fp8_linear", "fp8_linear_reduce"), warm_ms=SECONDARY_WARM_MS, timing_repeats=20)


# ----------------------------------------------------------------------------- config 5


def hybrid_workload(device: str, *, seed: int = 0, batch: int = 128, groups: int = 12, lo: int = 256, hi: int = 65536, heads: int = 16,
                    kv_heads: int = 2, dim: int = 256, bs: int = 16, key_heads: int = 16, value_heads: int = 32):
    """48 layers = 12 x (3 gated-delta linear layers + 1 paged GQA layer), one decode token per sequence."""
    import torch

    gen = torch.Generator().manual_seed(seed)
    ctx = torch.randint(lo, hi + 1, (batch,), generator=gen)
    dgen = torch.Generator(device=device).manual_seed(seed)
    need = [(int(c) + 1 + bs - 1) // bs for c in ctx]  # room for the appended token
    pool_blocks = math.ceil(sum(need) * 1.25)
    full_layers = []
    for _ in range(groups):
        perm = torch.randperm(pool_blocks, generator=gen)
        tables = torch.full((batch, max(need)), -1, dtype=torch.int32)
        cursor = 0
        for b, n in enumerate(need):
            tables[b, :n] = perm[cursor : cursor + n].to(torch.int32)
            cursor += n
        full_layers.append({
            "key_pool": torch.randn((pool_blocks, kv_heads, bs, dim), generator=dgen, device=device, dtype=torch.bfloat16),
            "value_pool": torch.randn((pool_blocks, kv_heads, bs, dim), generator=dgen, device=device, dtype=torch.bfloat16),
            "tables": tables.to(device),
        })
    channels = 2 * key_heads * 128 + value_heads * 128
    linear_layers = []
    for _ in range(3 * groups):
        linear_layers.append({
            "state": torch.randn((batch, value_heads, 128, 128), generator=dgen, device=device) * 0.05,
            "conv": torch.randn((batch, channels, 3), generator=dgen, device=device),
            "conv_w": torch.randn((channels, 4), generator=dgen, device=device) * 0.5,
            "a_log": torch.zeros(value_heads, device=device),
            "dt_bias": torch.zeros(value_heads, device=device),
        })
    step_inputs = {
        "query": torch.randn((batch, heads, 1, dim), generator=dgen, device=device, dtype=torch.bfloat16),
        "new_k": torch.randn((batch, kv_heads, 1, dim), generator=dgen, device=device, dtype=torch.bfloat16),
        "new_v": torch.randn((batch, kv_heads, 1, dim), generator=dgen, device=device, dtype=torch.bfloat16),
        "mixed": torch.randn((batch, channels), generator=dgen, device=device, dtype=torch.bfloat16),
        "a": torch.randn((batch, value_heads), generator=dgen, device=device, dtype=torch.bfloat16),
        "b": torch.randn((batch, value_heads), generator=dgen, device=device, dtype=torch.bfloat16),
        "positions": ctx.to(device=device, dtype=torch.int32),
        "lens": (ctx + 1).to(device=device, dtype=torch.int32),
    }
    sum_ctx = int(ctx.sum())
    full_bytes = (sum_ctx + batch) * kv_heads * dim * 2 * 2 + 2 * batch * heads * dim * 2 + sum(need) * 4 + batch * kv_heads * dim * 2 * 2
    linear_bytes = batch * (2 * value_heads * 128 * 128 * 4 + 2 * channels * 3 * 4 + channels * 2 + value_heads * 128 * 2)
    return {"full": full_layers, "linear": linear_layers, "inputs": step_inputs, "groups": groups, "bs": bs, "key_heads": key_heads,
            "algo_bytes": groups * full_bytes + 3 * groups * linear_bytes, "sum_ctx": sum_ctx, "pool_blocks": pool_blocks}


def time_hybrid(w, steps: int, warmup: int) -> float:
    """One step = every layer's attention for one decode token of all sequences (KV append + paged decode, or the delta step with its conv update fused in)."""
    import torch

    import hip_ops

    x = w["inputs"]

    def step():
        for g in range(w["groups"]):
            for lin in w["linear"][3 * g : 3 * g + 3]:
                hip_ops.gated_delta_step_conv(x["mixed"], lin["conv"], lin["conv_w"], x["a"], x["b"], lin["a_log"], lin["dt_bias"], lin["state"],
                                              key_heads=w["key_heads"])
            full = w["full"][g]
            hip_ops.paged_kv_append(x["new_k"], x["new_v"], full["key_pool"], full["value_pool"], full["tables"], x["positions"], w["bs"])
            hip_ops.paged_attention_decode_batched(x["query"], full["tables"], full["key_pool"], full["value_pool"], x["lens"], w["bs"])

    return _timed(step, steps, warmup, ("decode_partial_mfma", "decode_combine", "gated_delta_step", "causal_conv1d"), warm_ms=SECONDARY_WARM_MS)


# ----------------------------------------------------------------------------- main


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=20)
    parser.add_argument("--warmup", type=int, default=5)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-delta", action="store_true", help="skip the config-4 secondary measurement")
    parser.add_argument("--no-prefill", action="store_true", help="skip the config-3 secondary measurement")
    parser.add_argument("--no-hybrid", action="store_true", help="skip the config-5 secondary measurement")
    parser.add_argument("--no-prologue", action="store_true", help="skip the full-attention prologue measurement (config 3 shapes)")
    parser.add_argument("--no-output-norm", action="store_true", help="skip the linear-attention output stage measurement (config 4 shapes)")
    parser.add_argument("--no-fp8-linear", action="store_true", help="skip the fp8 block-scaled projection measurement (config 5 batch)")
    parser.add_argument("--no-serving", action="store_true", help="skip the graph-replayed serving decode step (config 2)")
    parser.add_argument("--no-reference-layout", action="store_true", help="skip the decode over the reference's per-request fp32 pools")
    parser.add_argument("--copy-probe-mib", type=int, default=0,
                        help="first run one plain device copy of this many MiB (reference point for HBM byte counters)")
    parser.add_argument("--cpu-budget", type=float, default=12.0)
    parser.add_argument("--cpu-budget-delta", type=float, default=30.0)
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the hot path is not sharded in this build", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    device = "cuda:0"
    if args.copy_probe_mib > 0:
        src = torch.ones(args.copy_probe_mib << 20, dtype=torch.uint8, device=device)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        _log(f"bench: copy probe of {args.copy_probe_mib} MiB done")
        del src, dst
    _log("bench: building config-2 workload")
    w = decode_workload(device)
    _log(f"bench: pool {w['pool_blocks']} blocks, sum ctx {int(w['ctx'].sum())}, algo bytes {w['algo_bytes']/1e9:.3f} GB")
    ms, kern = time_decode(w, args.steps, args.warmup)
    wc = {k: w[k] for k in ("query", "tables_cpu", "key_pool", "value_pool", "ctx", "bs")}
    gbs = w["algo_bytes"] / (ms * 1e-3) / 1e9
    k_ms = kern["decode_partial_mfma"]["avg_ms"]
    k_gbs = w["algo_bytes"] / (k_ms * 1e-3) / 1e9
    _log(f"bench: decode {ms:.4f} ms/step, {gbs:.1f} GB/s ({gbs / HBM_PEAK_GBS:.1%} of HBM peak); "
         f"main kernel {k_ms * 1e3:.1f} us = {k_gbs:.1f} GB/s ({k_gbs / HBM_PEAK_GBS:.1%})")
    record = {
        "metric": "paged decode attn HBM GB/s (% of 8 TB/s) + gated-delta prefill tokens/s",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16 Q/K/V, seeded shuffled block tables)",
        "config": {
            "workload": "paged GQA decode (BASELINE config 2)",
            "batch": 64,
            "q_heads": 16,
            "kv_heads": 2,
            "head_dim": 256,
            "block_size": 16,
            "context": "U[1024, 32768] seed 0",
            "sum_context": int(w["ctx"].sum()),
            "pool_blocks": w["pool_blocks"],
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(k_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(k_gbs / HBM_PEAK_GBS, 4),
            "traffic": TRAFFIC_DECODE,
            "kernel": "qa::decode_partial_mfma<256> (split-K partials); the step adds qa::decode_combine",
            "kernel_avg_us": round(k_ms * 1e3, 2),
            "algo_bytes_per_launch": w["algo_bytes"],
            "kernels": kern,
        },
    }
    if not args.no_serving:
        sv = time_serving_step(w, args.steps, args.warmup)
        # bytes: the primary decode's algorithmic bytes (plus one more token per row, within 0.02%),
        # the appended K/V token per row, and the reserve's lengths/positions
        sv_bytes = w["algo_bytes"] + 64 * 2 * 256 * 2 * 2 + 64 * (4 + 4 + 8)
        sv_gbs = sv_bytes / (sv["graph_ms"] * 1e-3) / 1e9
        _log(f"bench: serving decode step (reserve + append + attention) eager {sv['eager_ms']:.4f} ms, graph replay {sv['graph_ms']:.4f} ms = "
             f"{sv_gbs:.1f} GB/s ({sv_gbs / HBM_PEAK_GBS:.1%} of HBM peak)")
        record["secondary_serving_step"] = {
            "metric": "graph-replayed decode step through the runtime's device page tables (block reservation + K/V append + paged attention) HBM GB/s",
            "value": round(sv_gbs, 2),
            "unit": "GB/s",
            "ms_per_step": round(sv["graph_ms"], 5),
            "eager_ms_per_step": round(sv["eager_ms"], 5),
            "config": {"workload": "config 2 (64 rows, contexts U[1024, 32768] seed 0), one new token per row per step",
                       "tokens_added_per_row": sv["tokens_added"]},
            "roofline": {"bound": "hbm", "achieved": round(sv_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(sv_gbs / HBM_PEAK_GBS, 4),
                         "traffic": None, "algo_bytes_per_step": sv_bytes, "kernel": "kv_reserve_kernel + kv_append_kernel + decode_partial_mfma + decode_combine",
                         "kernels": sv["kernels"]},
        }
    if not args.no_reference_layout:
        _log("bench: building the reference-layout workload (per-request fp32 pools, repeated heads)")
        rw = reference_layout_workload(w, device)
        rms, rkern = time_reference_layout(rw, max(3, args.steps // 4), 1)
        r_gbs = rw["layout_bytes"] / (rms * 1e-3) / 1e9
        r_eq = rw["gqa_bytes"] / (rms * 1e-3) / 1e9
        _log(f"bench: reference layout decode {rms:.3f} ms/step, {r_gbs:.1f} GB/s of its own fp32 bytes ({r_gbs / HBM_PEAK_GBS:.1%} of HBM peak); "
             f"{r_eq:.1f} GB/s GQA-bf16 equivalent")
        record["secondary_reference_layout"] = {
            "metric": "paged decode over the reference's per-request fp32 repeated-head pools, HBM GB/s of that layout",
            "value": round(r_gbs, 2),
            "unit": "GB/s",
            "ms_per_step": round(rms, 4),
            "gqa_bf16_equivalent_gbs": round(r_eq, 2),
            "config": {"workload": "config 2 contexts (64 rows, U[1024, 32768] seed 0) in the reference engine's layout: one (1, 16, P_b, 16, 256) fp32 "
                                   "pool per request, KV heads repeated 8x, shuffled blocks, list of pools", "layout_bytes": rw["layout_bytes"]},
            "roofline": {"bound": "hbm", "achieved": round(r_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(r_gbs / HBM_PEAK_GBS, 4),
                         "traffic": None, "algo_bytes_per_step": rw["layout_bytes"], "kernel": "qa::decode_partial_generic<float, float, 1, 4> + decode_combine",
                         "kernels": rkern},
        }
        del rw
        torch.cuda.empty_cache()
    del w
    torch.cuda.empty_cache()
    cpu_delta = None
    if not args.no_delta:
        _log("bench: building config-4 workload (gated delta-rule chunked prefill)")
        dw = delta_workload(device)
        dms, dkern = time_delta(dw, max(20, args.steps), max(1, args.warmup))
        if not args.no_cpu_baseline:
            _log("bench: CPU baseline of config 4 (reference layer core, per-token loop)")
            cpu_delta = cpu_baseline_delta(dw, args.cpu_budget_delta)
        tflops = dw["flops"] / (dkern["chunk_gated_delta"]["avg_ms"] * 1e-3) / 1e12
        tok_s = dw["batch"] * dw["seq"] / (dms * 1e-3)
        _log(f"bench: delta prefill {dms:.3f} ms, {tok_s:,.0f} tokens/s, {tflops:.1f} TFLOP/s ({tflops / MFMA_BF16_PEAK_TFLOPS:.1%} of MFMA peak)")
        record["secondary"] = {
            "metric": "gated-delta chunked prefill tokens/s (BASELINE config 4)",
            "value": round(tok_s, 1),
            "unit": "tokens/s",
            "ms_per_step": round(dms, 4),
            "config": {"workload": "gated delta-rule chunked prefill (BASELINE config 4)", "batch": 4, "seq_len": 8192, "key_heads": 16,
                       "value_heads": 32, "head_dim": 128, "chunk": 64, "conv_kernel": 4},
            "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": TRAFFIC_DELTA, "algo_flop_per_launch": dw["flops"],
                         "algo_bytes_per_launch": dw["algo_bytes"], "kernel": "qa::cgd::chunk_kernel (fp16 MFMA, fp32 accumulate); the step adds prep_kernel (conv, norms and gating in one grid)",
                         "kernel_avg_us": round(dkern["chunk_gated_delta"]["avg_ms"] * 1e3, 2), "kernels": dkern},
        }
        del dw
        torch.cuda.empty_cache()
        if not args.no_output_norm:
            nw = output_norm_workload(device)
            nms, nkern = time_output_norm(nw, max(20, args.steps), max(1, args.warmup))
            n_ms = nkern["gated_rms_norm"]["avg_ms"]
            ngbs = nw["algo_bytes"] / (n_ms * 1e-3) / 1e9
            _log(f"bench: output norm {n_ms * 1e3:.1f} us for {nw['rows']} rows, {ngbs:.1f} GB/s ({ngbs / HBM_PEAK_GBS:.1%} of HBM peak)")
            record["secondary_output_norm"] = {
                "metric": "linear-attention output stage (gated RMSNorm + SiLU(z)) HBM GB/s",
                "value": round(ngbs, 2),
                "unit": "GB/s",
                "ms_per_step": round(nms, 4),
                "config": {"workload": "config 4's 4 x 8192 tokens x 32 value heads of 128 (bf16 core and z in, bf16 out)", "eps": 1e-6},
                "roofline": {"bound": "hbm", "achieved": round(ngbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ngbs / HBM_PEAK_GBS, 4),
                             "traffic": TRAFFIC_OUTPUT_NORM, "algo_bytes_per_launch": nw["algo_bytes"],
                             "kernel": "qa::gnorm::gated_rms_norm_kernel<128, true>", "kernel_avg_us": round(n_ms * 1e3, 2), "kernels": nkern},
            }
            del nw
            torch.cuda.empty_cache()
    if not args.no_prefill:
        _log("bench: building config-3 workload (chunked paged prefill with gate)")
        pw = prefill_workload(device)
        pms, pkern = time_prefill(pw, max(4, args.steps // 2), 1)
        ptf = pw["flops"] / (pkern["paged_prefill"]["total_ms_per_step"] * 1e-3) / 1e12
        _log(f"bench: paged prefill {pms:.3f} ms, {ptf:.1f} TFLOP/s ({ptf / MFMA_BF16_PEAK_TFLOPS:.1%} of MFMA peak)")
        record["secondary_prefill"] = {
            "metric": "chunked paged prefill TFLOP/s (BASELINE config 3)",
            "value": round(ptf, 2),
            "unit": "TFLOP/s",
            "ms_per_step": round(pms, 4),
            "config": {"workload": "chunked causal paged prefill with sigmoid gate (BASELINE config 3)", "batch": 8, "new_tokens": 4096,
                       "prefix": "U[0, 8192] seed 0", "q_heads": 16, "kv_heads": 2, "head_dim": 256, "block_size": 16, "query_chunk": 512},
            "roofline": {"bound": "mfma", "achieved": round(ptf, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(ptf / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": TRAFFIC_PREFILL, "algo_flop_per_step": pw["flops"],
                         "algo_bytes_per_launch": round(pw["algo_bytes"] / pw["launches"]), "launches_per_step": pw["launches"],
                         "kernel": "qa::pfx::prefill_kernel<256, 1>, one launch per 512-token query chunk (kv_append between)",
                         "kernel_ms_per_step": round(pkern["paged_prefill"]["total_ms_per_step"], 4), "kernels": pkern},
        }
        if not args.no_prologue:
            ow = prologue_workload(pw, device)
            oms, okern = time_prologue(ow, pw, max(10, args.steps), max(1, args.warmup))
            k_ms = okern["qk_norm_rope"]["avg_ms"]
            ogbs = ow["algo_bytes"] / (k_ms * 1e-3) / 1e9
            _log(f"bench: attention prologue {oms * 1e3:.1f} us for {ow['tokens']} tokens, {ogbs:.1f} GB/s ({ogbs / HBM_PEAK_GBS:.1%} of HBM peak)")
            record["secondary_prologue"] = {
                "metric": "full-attention prologue (q/k RMSNorm + partial RoPE + paged K/V append) HBM GB/s",
                "value": round(ogbs, 2),
                "unit": "GB/s",
                "ms_per_step": round(oms, 4),
                "config": {"workload": "config 3's 32768 new tokens (8 x 4096, prefix U[0, 8192] seed 0) in one launch", "q_heads": 16,
                           "kv_heads": 2, "head_dim": 256, "rotary_dim": 64, "rope_theta": 1e7, "block_size": 16},
                "roofline": {"bound": "hbm", "achieved": round(ogbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(ogbs / HBM_PEAK_GBS, 4),
                             "traffic": TRAFFIC_PROLOGUE, "algo_bytes_per_launch": ow["algo_bytes"], "kernel": "qa::qkr::qk_norm_rope_kernel<4, 1>",
                             "kernel_avg_us": round(k_ms * 1e3, 2), "kernels": okern},
            }
            del ow
        del pw
        torch.cuda.empty_cache()
    if not args.no_hybrid:
        _log("bench: building config-5 workload (48-layer hybrid decode step, attention only)")
        hw = hybrid_workload(device)
        hms, hkern = time_hybrid(hw, 3, 1)
        hgbs = hw["algo_bytes"] / (hms * 1e-3) / 1e9
        _log(f"bench: hybrid step {hms:.3f} ms, {hgbs:.1f} GB/s ({hgbs / HBM_PEAK_GBS:.1%} of HBM peak)")
        record["secondary_hybrid"] = {
            "metric": "hybrid decode step HBM GB/s (BASELINE config 5)",
            "value": round(hgbs, 2),
            "unit": "GB/s",
            "ms_per_step": round(hms, 4),
            "config": {"workload": "48-layer hybrid decode step, attention only (BASELINE config 5)", "batch": 128, "layers": "12 x (3 linear + 1 full)",
                       "context": "U[256, 65536] seed 0", "sum_context": hw["sum_ctx"], "pool_blocks_per_layer": hw["pool_blocks"]},
            "roofline": {"bound": "hbm", "achieved": round(hgbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(hgbs / HBM_PEAK_GBS, 4),
                         "traffic": TRAFFIC_HYBRID, "algo_bytes_per_step": hw["algo_bytes"], "kernel": "whole step (12 paged-decode + 36 delta-step layers with the conv update fused in)",
                         "kernels": hkern},
        }
        del hw
        torch.cuda.empty_cache()
    if not args.no_fp8_linear:
        fw = fp8_linear_workload(device)
        fms, fkern = time_fp8_linear(fw, max(20, args.steps), max(1, args.warmup))
        f_ms = sum(fkern.get(k, {}).get("avg_ms", 0.0) for k in ("fp8_linear_cast", "fp8_linear", "fp8_linear_reduce"))
        fgbs = fw["algo_bytes"] / (f_ms * 1e-3) / 1e9
        _log(f"bench: fp8 linear {f_ms * 1e3:.2f} us ({fw['rows']} x {fw['out']} x {fw['in']}), {fgbs:.1f} GB/s ({fgbs / HBM_PEAK_GBS:.1%} of HBM peak)")
        record["secondary_fp8_linear"] = {
            "metric": "fp8 E4M3 block-scaled projection HBM GB/s",
            "value": round(fgbs, 2),
            "unit": "GB/s",
            "ms_per_step": round(fms, 4),
            "config": {"workload": "128 tokens (config 5's decode batch) x q_proj-shaped fp8 weight (8192 x 2048, 128x128 bf16 scales, packed once), fp32 in/out",
                       "rows": fw["rows"], "out_features": fw["out"], "in_features": fw["in"]},
            "roofline": {"bound": "hbm", "achieved": round(fgbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(fgbs / HBM_PEAK_GBS, 4),
                         "traffic": TRAFFIC_FP8_LINEAR, "algo_bytes_per_launch": fw["algo_bytes"], "algo_flop_per_launch": fw["flops"],
                         "kernel": "qa::f8l::fp8_linear_xres_kernel<X_F16, true> (fp32 x rounded to fp16 as it is staged, x resident in LDS, packed weight streamed into registers, one launch)",
                         "kernel_avg_us": round(f_ms * 1e3, 2), "kernels": fkern},
        }
        del fw
        torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        _log("bench: CPU baseline (reference path restatement)")
        record["cpu_baseline"] = cpu_baseline_decode(wc, args.cpu_budget)
        record["cpu_baseline"]["config1"] = cpu_baseline_config1(device)
        if cpu_delta is not None:
            record["cpu_baseline"]["delta"] = cpu_delta
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
