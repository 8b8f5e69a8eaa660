#!/usr/bin/env python3
"""Decode benchmark for the Qwen3 forward-pass hot path on one MI355X.

Default workload (the north-star configuration): Qwen3-8B shape, bf16
weights ~N(0, 0.02) generated on the device, batch-32 paged decode, per-
sequence context lengths uniform in [512, 8192] (seeded) of random KV
(bf16 ~N(0, 1)) in 16-token pages drawn from a shuffled 16384-page pool,
greedy decode. A step is one fh_execute_batch over the 32 rows: tokens in,
greedy choices out, KV appended; the chosen tokens feed the next step.

Prints one JSON line: value = whole-job decode tokens/s over the timed steps
(HIP graph replays, as served; --eager times plain launches instead);
roofline = the dominant kernel's algorithmic HBM bytes per launch / its
average launch time, from HIP events recorded on the runner's stream around
every launch of --profile-steps further eager steps; cpu_baseline = the CPU
oracle timed on a bounded sample of the same step.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_HBM_GBS = 8000.0


def metric_name(model_key, batch):
    """The headline metric's wording for a decode workload's model and batch."""
    model = "Qwen3-8B" if model_key == "8b" else "Qwen3-0.6B"
    return f"decode tokens/s, {model} bf16 batch {batch} (1 GPU); achieved HBM GB/s % peak"

WORKLOADS = {
    # name: (model, batch, (ctx_lo, ctx_hi), physical pages, decode headroom, description)
    "qwen3-8b-b32": ("8b", 32, (512, 8192), 16384, 128,
                     "Qwen3-8B shape, batch-32 paged decode, ctx U[512,8192], 16-token pages permuted over a "
                     "16384-page pool, greedy"),
    "qwen3-8b-b1": ("8b", 1, (4096, 4096), 300, 128,
                    "Qwen3-8B shape, batch-1 decode, ctx 4096 of random KV in 16-token pages, greedy"),
    "qwen3-0.6b-b32": ("0.6b", 32, (128, 2048), 4608, 64,
                       "Qwen3-0.6B shape, batch-32 paged decode, ctx U[128,2048], shuffled page pool, greedy"),
}
# Prefill chunks: (model, sequences, prompt tokens, description)
PREFILL_WORKLOADS = {
    "qwen3-8b-prefill": ("8b", 32, 256, "Qwen3-8B shape, one chunked-prefill batch of 32 prompts x 256 random ids "
                                        "from position 0 into a shuffled 16-token page pool; greedy first token"),
}
# One request end to end: (model, prompt tokens, decode steps, description)
REQUEST_WORKLOADS = {
    "qwen3-0.6b-b1-prompt": ("0.6b", 16, 8, "Qwen3-0.6B shape, batch 1: a 16-token prompt (ids U[0,151936)) as one "
                                            "16-row batch, then 8 greedy decode steps, 16-token pages"),
}
SPEC_WORKLOADS = {
    "qwen3-8b-speculative": (32, 256, 4, "Qwen3-8B target + Qwen3-0.6B draft (random init), 32 prompts x 256 "
                                         "random ids prefilled into both, then greedy speculative rounds with K=4"),
}
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=64)
    p.add_argument("--warmup", type=int, default=4)
    p.add_argument("--workload", default="qwen3-8b-b32",
                   choices=sorted(WORKLOADS) + sorted(PREFILL_WORKLOADS) + sorted(REQUEST_WORKLOADS)
                   + sorted(SPEC_WORKLOADS))
    p.add_argument("--seed", type=int, default=1)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-spec-prompt", type=int, default=16, help="speculative CPU baseline: prompt tokens")
    p.add_argument("--cpu-spec-rounds", type=int, default=12, help="speculative CPU baseline: rounds")
    p.add_argument("--cpu-steps", type=int, default=2, help="decode steps the CPU oracle sample runs")
    p.add_argument("--cpu-prefill-tokens", type=int, default=256,
                   help="prompt tokens of the one sequence the prefill workload's CPU oracle sample prefills")
    p.add_argument("--eager", action="store_true", help="time eager launches instead of HIP graph replays")
    p.add_argument("--profile-steps", type=int, default=16,
                   help="eager steps with per-launch HIP events after the timed steps (per-kernel times, roofline)")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="only run 4 device-to-device copies of this many MiB (calibrates HBM byte counters) and exit")
    return p.parse_args()


def copy_probe(mib):
    """Four plain copies of a known size: under a hardware-counter profiler
    their FETCH_SIZE / WRITE_SIZE per dispatch give the counters' scale."""
    import torch

    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_bytes_read": n, "copy_probe_bytes_written": n, "copies": 4}), flush=True)


def attn_partition_tokens(rows, query_heads):
    """Tokens per decode attention partition: 32 pages of 16, or 16 pages
    when the launch has at most 64 (row, query head) pairs (the library's
    attn_split_pages)."""
    return 256 if rows * query_heads <= 64 else 512


def kernel_bytes(cfg, rows, positions, stride):
    """Algorithmic HBM bytes per launch of each kernel class, for one step."""
    H, QH, KVH, I, V = cfg["hidden"], cfg["query_heads"], cfg["kv_heads"], cfg["intermediate"], cfg["vocabulary"]
    Q, KV = QH * 128, KVH * 128
    nqkv = Q + 2 * KV
    ctx = np.asarray(positions, np.int64) + 1
    kv_read = int(np.sum(ctx)) * KV * 2 * 2  # K and V rows, bf16
    # Rows longer than one partition leave one FP32 record (max, denominator,
    # 128 numerators) per query head and partition.
    tokens = attn_partition_tokens(rows, QH)
    parts = (ctx + tokens - 1) // tokens
    merge_read = int(np.sum(np.where(parts > 1, parts, 0))) * QH * 130 * 4
    merged_rows = int(np.sum(parts > 1))
    norm = rows * H * 2 * 2 + H * 2  # residual row in and out, norm weight
    # One-row steps run each norm inside the projection that consumes it
    # (QKV, gate/up, LM head), which then reads the residual row and norm
    # weight and writes the folded row instead of reading a normalized one.
    in_proj = norm - rows * H * 2 if rows == 1 else 0
    return {
        "attention": kv_read + rows * Q * 2,
        "qkv_gemm": nqkv * H * 2 + rows * H * 2 + rows * nqkv * 2 + in_proj,
        "o_gemm": H * Q * 2 + rows * Q * 2 + rows * H * 2 * 2,
        "gate_up_gemm": 2 * I * H * 2 + rows * H * 2 + rows * I * 2 + in_proj,
        "down_gemm": H * I * 2 + rows * I * 2 + rows * H * 2 * 2,
        "head_gemm": V * H * 2 + rows * H * 2 + rows * V * 4 + in_proj,
        "rmsnorm": 0 if rows == 1 else norm,
        "qknorm_rope_kv": rows * nqkv * 2 + rows * Q * 2 + rows * 2 * KV * 2,
        "attention_merge": merge_read + merged_rows * Q * 2,
        "argmax": rows * V * 4,
        "embedding": rows * H * 2 * 2,
    }


def step_bytes(cfg, rows, positions):
    """Algorithmic bytes of one decode step: weights streamed once, embedding
    rows, KV read over each context (incl. the new token), the new KV rows,
    FP32 logits."""
    H, QH, KVH, I, V, L = (cfg["hidden"], cfg["query_heads"], cfg["kv_heads"], cfg["intermediate"],
                           cfg["vocabulary"], cfg["layers"])
    Q, KV = QH * 128, KVH * 128
    per_layer = ((Q + 2 * KV) * H + H * Q + 3 * I * H) * 2 + (2 * H + 256) * 2
    head = V * H * 2  # the LM head, or the tied embedding table it reads
    weights = L * per_layer + head + H * 2
    kvb = L * 2 * KV * 2
    ctx = np.asarray(positions, np.int64) + 1
    return int(weights + rows * 2 * H + int(np.sum(ctx)) * kvb + rows * kvb + rows * V * 4)


def cpu_baseline(cfg, contexts, args, seed):
    """Times the CPU oracle (all layers, same weights-generator, contexts and
    KV shapes) on args.cpu_steps consecutive decode steps of the workload."""
    from oracle import oracle as orc

    rows = len(contexts)
    steps = args.cpu_steps
    need = [(c + steps + 15) // 16 for c in contexts]
    stride = max(need) + 1
    pages = sum(need) + rows
    m = orc.Model(cfg, pages)
    try:
        t0 = time.perf_counter()
        m.synthesize(seed, 0.02)
        tables = np.full((rows, stride), 0xFFFFFFFF, np.uint32)
        nxt = 0
        for i, n in enumerate(need):
            tables[i, :n] = np.arange(nxt, nxt + n, dtype=np.uint32)
            nxt += n
        m.kv_fill(seed, 1.0, tables, stride, contexts, list(range(1, rows + 1)), 1 << 20)
        setup_s = time.perf_counter() - t0
        toks = np.random.default_rng(seed).integers(0, cfg["vocabulary"], rows)
        positions = np.asarray(contexts, np.int64)
        elapsed = 0.0
        for _ in range(steps):
            counts = np.asarray([(p + 1 + 15) // 16 for p in positions], np.uint32)
            t1 = time.perf_counter()
            out = m.forward(toks, positions, tables, counts, stride, want_logits=False)
            elapsed += time.perf_counter() - t1
            toks = out["choices"]
            positions = positions + 1
        return {
            "value": rows * steps / elapsed,
            "unit": "tokens/s",
            "cores": orc.threads(),
            "kind": "port",
            "sample": (f"{steps} full decode steps ({cfg['layers']} layers, embedding, final norm, FP32 head, "
                       f"argmax) at batch {rows} over the same contexts: {elapsed:.2f} s "
                       f"(weights + KV prefix generation {setup_s:.1f} s untimed)"),
        }
    finally:
        m.close()


def prefill_flops(cfg, seqs, tokens):
    """Algorithmic FLOPs of one prefill chunk: every projection for every
    token, causal attention (QK^T and PV over keys 0..t), and the FP32 head
    for each prompt's last token."""
    H, QH, KVH, I, V, L = (cfg["hidden"], cfg["query_heads"], cfg["kv_heads"], cfg["intermediate"],
                           cfg["vocabulary"], cfg["layers"])
    Q, KV = QH * 128, KVH * 128
    linear = ((Q + 2 * KV) * H + H * Q + 3 * I * H) * 2  # per token per layer
    keys = tokens * (tokens + 1) // 2  # causal key count per sequence
    attn = keys * QH * 128 * 2 * 2  # QK^T + PV per sequence per layer
    return L * (seqs * tokens * linear + seqs * attn) + seqs * V * H * 2


def prefill_bench(args, name):
    import torch

    import ferric_amd
    from ferric_amd import PagedLimits, PagePool, TpBatchRunner

    model_key, seqs, tokens, desc = PREFILL_WORKLOADS[name]
    cfg = dict(ferric_amd.QWEN3_8B if model_key == "8b" else ferric_amd.QWEN3_0_6B)
    rows = seqs * tokens
    context_tokens = (tokens + 15) // 16 * 16
    pages_per_seq = context_tokens // 16
    limits = PagedLimits(context_tokens=context_tokens, physical_page_count=seqs * pages_per_seq * 2,
                         page_table_stride=pages_per_seq)
    runner = TpBatchRunner(cfg, limits, row_capacity=32, use_graphs=False, prefill_rows=rows)
    runner.synthesize_weights(args.seed, 0.02)
    pool = PagePool(limits, seed=args.seed)
    rng = np.random.default_rng(args.seed)
    prompts = rng.integers(0, cfg["vocabulary"], (seqs, tokens))
    outs = [(i + 1) * tokens - 1 for i in range(seqs)]

    def step():
        sids = [pool.admit(0) for _ in range(seqs)]
        b = pool.prepare([(s, int(t)) for s, p in zip(sids, prompts) for t in p])
        out = runner.execute_batch(b, outs)
        for s in sids:
            pool.release(s)
        return out.choices

    for _ in range(args.warmup):
        step()
    steps = max(1, min(args.steps, 8))
    device_ms = 0.0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
        device_ms += runner.last_step_ms()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    runner.set_profiling(True)
    class_ms, class_launches = {}, {}
    for _ in range(2):
        step()
        for k, (ms, n) in runner.kernel_class_ms().items():
            class_ms[k] = class_ms.get(k, 0.0) + ms / 2
            class_launches[k] = class_launches.get(k, 0) + n / 2
    runner.set_profiling(False)
    flops = prefill_flops(cfg, seqs, tokens)
    tflops = flops / (elapsed / steps) / 1e12
    H, QH, KVH, I = cfg["hidden"], cfg["query_heads"], cfg["kv_heads"], cfg["intermediate"]
    gemm_flops = {"qkv_gemm": rows * (QH + 2 * KVH) * 128 * H * 2, "o_gemm": rows * H * QH * 128 * 2,
                  "gate_up_gemm": rows * 2 * I * H * 2, "down_gemm": rows * H * I * 2}
    dominant = max(gemm_flops, key=lambda k: class_ms.get(k, 0.0))
    avg_ms = class_ms[dominant] / max(class_launches[dominant], 1)
    achieved = gemm_flops[dominant] / (avg_ms * 1e-3) / 1e12
    result = {
        "metric": f"prefill tokens/s and MFMA TFLOP/s, {desc}",
        "value": round(rows * steps / elapsed, 1),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / steps, 3),
        "device_ms_per_step": round(device_ms / steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": desc, "sequences": seqs, "prompt_tokens": tokens, "rows_per_chunk": rows},
        "step_tflops": {"achieved": round(tflops, 1), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(tflops / PEAK_BF16_TFLOPS, 4), "flops_per_step": int(flops)},
        "roofline": {"kernel": dominant, "bound": "mfma", "achieved": round(achieved, 1), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4), "traffic": None,
                     "avg_launch_us": round(avg_ms * 1e3, 2), "algorithmic_flops_per_launch": gemm_flops[dominant]},
        "kernels": {k: {"ms_per_step": round(v, 3)} for k, v in sorted(class_ms.items(), key=lambda kv: -kv[1])},
    }
    runner.close()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = prefill_cpu_baseline(cfg, min(args.cpu_prefill_tokens, tokens), args.seed)
    print(json.dumps(result), flush=True)


def prefill_cpu_baseline(cfg, tokens, seed):
    """Times the CPU oracle prefilling one sequence's prompt of `tokens` ids
    from position 0 (one forward over all its rows, every layer, FP32 head
    and argmax for the last row)."""
    from oracle import oracle as orc

    stride = (tokens + 15) // 16
    m = orc.Model(cfg, stride)
    try:
        t0 = time.perf_counter()
        m.synthesize(seed, 0.02)
        setup_s = time.perf_counter() - t0
        ids = np.random.default_rng(seed).integers(0, cfg["vocabulary"], tokens)
        table = np.full((tokens, stride), 0xFFFFFFFF, np.uint32)
        table[:, :] = np.arange(stride, dtype=np.uint32)
        counts = np.full(tokens, stride, np.uint32)
        t1 = time.perf_counter()
        m.forward(ids, np.arange(tokens), table, counts, stride, want_logits=False)
        elapsed = time.perf_counter() - t1
        return {
            "value": round(tokens / elapsed, 2),
            "unit": "tokens/s",
            "cores": orc.threads(),
            "kind": "port",
            "sample": (f"one sequence's {tokens}-token prompt prefilled from position 0 ({cfg['layers']} layers, "
                       f"every row's K/V written, FP32 head and argmax for every row) in {elapsed:.2f} s, "
                       f"tokens/s of that sample (the GPU leg prefills 32 such prompts in one chunk); weight "
                       f"generation {setup_s:.1f} s untimed"),
        }
    finally:
        m.close()


def request_bench(args, name):
    """One request end to end, repeated: a prompt batch, then greedy decode
    steps on the same sequence (a fresh sequence per request)."""
    import torch

    import ferric_amd
    from ferric_amd import PagedLimits, PagePool, TpBatchRunner

    model_key, prompt_len, decode_steps, desc = REQUEST_WORKLOADS[name]
    cfg = dict(ferric_amd.QWEN3_8B if model_key == "8b" else ferric_amd.QWEN3_0_6B)
    ctx = (prompt_len + decode_steps + 15) // 16 * 16
    limits = PagedLimits(context_tokens=ctx, physical_page_count=4 * (ctx // 16), page_table_stride=ctx // 16)
    runner = TpBatchRunner(cfg, limits, row_capacity=prompt_len, use_graphs=not args.eager)
    runner.synthesize_weights(args.seed, 0.02)
    pool = PagePool(limits, seed=args.seed)
    prompt = [int(t) for t in np.random.default_rng(args.seed).integers(0, cfg["vocabulary"], prompt_len)]

    def request():
        sid = pool.admit(0)
        b = pool.prepare([(sid, t) for t in prompt])
        tok = runner.execute_batch(b, [prompt_len - 1]).choices[0]
        pool.commit(b)
        out = []
        for _ in range(decode_steps):
            b = pool.prepare([(sid, tok)])
            tok = runner.execute_batch(b, [0]).choices[0]
            pool.commit(b)
            out.append(tok)
        pool.release(sid)
        return out

    for _ in range(args.warmup):
        request()
    reqs = max(1, args.steps)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(reqs):
        tokens = request()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    result = {
        "metric": f"decode tokens/s per request, {desc}",
        "value": round(decode_steps * reqs / elapsed, 2),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": reqs, "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / reqs, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": desc, "prompt_tokens": prompt_len, "decode_steps": decode_steps,
                   "step": "one request: the prompt batch plus the decode steps", "graphs": not args.eager,
                   "last_request_tokens": [int(t) for t in tokens]},
    }
    runner.close()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = request_cpu_baseline(cfg, prompt, decode_steps, args.seed)
    print(json.dumps(result), flush=True)


def request_cpu_baseline(cfg, prompt, decode_steps, seed):
    """The CPU oracle running the same request end to end (prompt forward,
    then the decode steps, each feeding its greedy choice to the next)."""
    from oracle import oracle as orc

    ctx = (len(prompt) + decode_steps + 15) // 16 * 16
    stride = ctx // 16
    m = orc.Model(cfg, stride)
    try:
        t0 = time.perf_counter()
        m.synthesize(seed, 0.02)
        setup_s = time.perf_counter() - t0
        table = np.full((len(prompt), stride), 0xFFFFFFFF, np.uint32)
        table[:, :] = np.arange(stride, dtype=np.uint32)
        t1 = time.perf_counter()
        n = len(prompt)
        out = m.forward(prompt, np.arange(n), table, np.full(n, stride, np.uint32), stride, want_logits=False)
        tok = int(out["choices"][-1])
        for i in range(decode_steps):
            out = m.forward([tok], [n + i], table[:1], np.full(1, stride, np.uint32), stride, want_logits=False)
            tok = int(out["choices"][0])
        elapsed = time.perf_counter() - t1
        return {
            "value": round(decode_steps / elapsed, 2),
            "unit": "tokens/s",
            "cores": orc.threads(),
            "kind": "port",
            "sample": (f"the same request end to end ({len(prompt)}-token prompt forward, then {decode_steps} "
                       f"decode steps, {cfg['layers']} layers, FP32 head, argmax): {elapsed:.2f} s; weight "
                       f"generation {setup_s:.1f} s untimed"),
        }
    finally:
        m.close()


def speculative_bench(args, name):
    import torch

    import ferric_amd
    from ferric_amd import PagedLimits, PagePool, TpBatchRunner
    from ferric_amd.speculative import SpeculativeDecoder

    seqs, tokens, k, desc = SPEC_WORKLOADS[name]
    rounds = max(1, args.steps)
    context_tokens = (tokens + (rounds + args.warmup + 2) * (k + 1) + 15) // 16 * 16
    stride = context_tokens // 16
    limits = PagedLimits(context_tokens=context_tokens, physical_page_count=seqs * stride + 64,
                         page_table_stride=stride)
    target = TpBatchRunner(ferric_amd.QWEN3_8B, limits, row_capacity=32, use_graphs=True, prefill_rows=seqs * tokens)
    draft = TpBatchRunner(ferric_amd.QWEN3_0_6B, limits, row_capacity=32, use_graphs=True,
                          prefill_rows=seqs * tokens)
    target.synthesize_weights(args.seed, 0.02)
    draft.synthesize_weights(args.seed + 1, 0.02)
    dec = SpeculativeDecoder(target, PagePool(limits, seed=args.seed), draft, PagePool(limits, seed=args.seed + 1), k=k)
    rng = np.random.default_rng(args.seed)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    dec.prefill([list(rng.integers(0, ferric_amd.QWEN3_8B["vocabulary"], tokens)) for _ in range(seqs)])
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    for _ in range(args.warmup):
        dec.round()
    emitted = accepted = 0
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(rounds):
        st = dec.round()
        emitted += sum(len(e) for e in st.emitted)
        accepted += sum(st.accepted)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    result = {
        "metric": f"speculative decode tokens/s, {desc}",
        "value": round(emitted / elapsed, 2),
        "unit": "tokens/s",
        "n_gpus": 1, "steps": rounds, "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1e3 / rounds, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16", "data": "synthetic",
        "config": {"workload": desc, "sequences": seqs, "prompt_tokens": tokens, "k": k,
                   "prefill_both_models_s": round(prefill_s, 3),
                   "acceptance": round(accepted / (rounds * seqs * k), 4),
                   "emitted_per_round": round(emitted / rounds, 2)},
    }
    target.close()
    draft.close()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = speculative_cpu_baseline(ferric_amd.QWEN3_8B, ferric_amd.QWEN3_0_6B, k,
                                                          args.cpu_spec_prompt, args.cpu_spec_rounds, args.seed)
    print(json.dumps(result), flush=True)


def speculative_cpu_baseline(cfg_t, cfg_d, k, prompt_len, rounds, seed):
    """The CPU oracle running greedy speculation for one sequence: the
    prompt through both models, then `rounds` rounds of k draft decode steps
    (one row each) and a (k + 1)-row target verify, the accepted prefix and
    the target's next token emitted, positions advanced by what was emitted
    (a full accept adds the draft's catch-up step)."""
    from oracle import oracle as orc

    ctx = (prompt_len + (rounds + 1) * (k + 1) + 15) // 16 * 16
    stride = ctx // 16
    mt, md = orc.Model(cfg_t, stride), orc.Model(cfg_d, stride)
    try:
        t0 = time.perf_counter()
        mt.synthesize(seed, 0.02)
        md.synthesize(seed + 1, 0.02)
        setup_s = time.perf_counter() - t0
        rows = max(prompt_len, k + 1)
        table = np.tile(np.arange(stride, dtype=np.uint32), (rows, 1))
        counts = np.full(rows, stride, np.uint32)
        prompt = [int(t) for t in np.random.default_rng(seed).integers(0, cfg_t["vocabulary"], prompt_len)]
        t1 = time.perf_counter()
        n = prompt_len
        anchor = int(mt.forward(prompt, np.arange(n), table[:n], counts[:n], stride, want_logits=False)["choices"][-1])
        md.forward(prompt, np.arange(n), table[:n], counts[:n], stride, want_logits=False)
        pos, emitted, accepted = n, 0, 0
        for _ in range(rounds):
            drafts, tok = [], anchor
            for i in range(k):
                tok = int(md.forward([tok], [pos + i], table[:1], counts[:1], stride, want_logits=False)["choices"][0])
                drafts.append(tok)
            ids = [anchor] + drafts
            c = [int(x) for x in mt.forward(ids, np.arange(pos, pos + k + 1), table[:k + 1], counts[:k + 1], stride,
                                            want_logits=False)["choices"]]
            acc = 0
            while acc < k and drafts[acc] == c[acc]:
                acc += 1
            if acc == k:  # the draft never saw its last token
                md.forward([drafts[-1]], [pos + k], table[:1], counts[:1], stride, want_logits=False)
            emitted += acc + 1
            accepted += acc
            anchor = c[acc]
            pos += acc + 1
        elapsed = time.perf_counter() - t1
        return {
            "value": round(emitted / elapsed, 2),
            "unit": "tokens/s",
            "cores": orc.threads(),
            "kind": "port",
            "sample": (f"one sequence: a {prompt_len}-token prompt through both models, then {rounds} rounds of "
                       f"{k} draft steps ({cfg_d['layers']} layers) and a {k + 1}-row verify ({cfg_t['layers']} "
                       f"layers), {emitted} tokens emitted ({accepted} drafts accepted) in {elapsed:.2f} s, tokens/s "
                       f"of that sample (the GPU leg runs 32 sequences); weight generation {setup_s:.1f} s untimed"),
        }
    finally:
        mt.close()
        md.close()


TRAFFIC_PROFILE = "profiles/attention_decode_qwen3_8b_b32_hbm_counters.md"


def measured_traffic(workload):
    """HBM bytes per attention launch of the default workload, as measured by the
    FETCH_SIZE / WRITE_SIZE passes summarised in TRAFFIC_PROFILE (None if absent)."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), TRAFFIC_PROFILE)
    if workload != "qwen3-8b-b32" or not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("| `attn_partition_kernel"):
            cells = [c.strip() for c in line.strip().strip("|").split("|")]
            return int(float(cells[3]) * 1e6)
    return None


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box in this build has one MI355X, so --gpus {args.gpus} is not "
              f"supported (the batch shards by sequence across GPUs; see the sharding notes)", file=sys.stderr)
        sys.exit(2)
    if args.copy_probe_mib:
        copy_probe(args.copy_probe_mib)
        return

    if args.workload in PREFILL_WORKLOADS:
        prefill_bench(args, args.workload)
        return
    if args.workload in SPEC_WORKLOADS:
        speculative_bench(args, args.workload)
        return
    if args.workload in REQUEST_WORKLOADS:
        request_bench(args, args.workload)
        return

    import torch

    import ferric_amd
    from ferric_amd import PagedLimits, PagePool, TpBatchRunner

    name = args.workload
    model_key, batch, (ctx_lo, ctx_hi), phys_pages, headroom, desc = WORKLOADS[name]
    cfg = dict(ferric_amd.QWEN3_8B if model_key == "8b" else ferric_amd.QWEN3_0_6B)
    context_tokens = ctx_hi + headroom + args.warmup + args.steps + args.profile_steps
    context_tokens = (context_tokens + 15) // 16 * 16
    limits = PagedLimits(context_tokens=context_tokens, physical_page_count=phys_pages,
                         page_table_stride=context_tokens // 16)
    rng = np.random.default_rng(args.seed)
    contexts = [int(c) for c in rng.integers(ctx_lo, ctx_hi + 1, batch)]

    t_setup = time.perf_counter()
    runner = TpBatchRunner(cfg, limits, row_capacity=32, use_graphs=not args.eager)
    runner.synthesize_weights(args.seed, 0.02)
    pool = PagePool(limits, seed=args.seed)
    sids = [pool.admit(c) for c in contexts]
    fill = [ferric_amd.PreparedRow(s, 0, c, tuple(pool.sequences[s].pages), pool.sequences[s].pages[-1])
            for s, c in zip(sids, contexts)]
    runner.kv_fill_synthetic(args.seed, 1.0, fill, sids, context_tokens)
    tokens = [int(t) for t in rng.integers(0, cfg["vocabulary"], batch)]
    setup_s = time.perf_counter() - t_setup
    print(f"# setup {setup_s:.1f} s: {name}, contexts mean {np.mean(contexts):.0f}", file=sys.stderr, flush=True)

    outputs = list(range(batch))

    def step(toks):
        b = pool.prepare(list(zip(sids, toks)))
        out = runner.execute_batch(b, outputs)
        pool.commit(b)
        return out.choices, b.rows.position  # the pool's prepared rows carry their columns

    for _ in range(args.warmup):
        tokens, _ = step(tokens)

    step_positions = []
    device_ms = 0.0
    step_device_ms = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        tokens, positions = step(tokens)
        step_device_ms.append(runner.last_step_ms())
        device_ms += step_device_ms[-1]
        step_positions.append(positions)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    step_byte_total = sum(step_bytes(cfg, batch, p) for p in step_positions)

    # Per-kernel times: eager steps with an event pair around every launch.
    class_ms, class_launches, class_bytes = {}, {}, {}
    runner.set_profiling(args.profile_steps > 0)
    for _ in range(args.profile_steps):
        tokens, positions = step(tokens)
        for k, (ms, n) in runner.kernel_class_ms().items():
            class_ms[k] = class_ms.get(k, 0.0) + ms
            class_launches[k] = class_launches.get(k, 0) + n
        for k, b in kernel_bytes(cfg, batch, positions, limits.page_table_stride).items():
            per_layer = cfg["layers"] if k not in ("head_gemm", "argmax", "embedding") else 1
            if k == "rmsnorm":
                per_layer = 2 * cfg["layers"] + 1
            class_bytes[k] = class_bytes.get(k, 0) + b * per_layer
    runner.set_profiling(False)
    # A second figure for the attention launch duration, without an event
    # pair around each launch: the last step's attention re-launched back to
    # back (same inputs, so it rewrites the same outputs).
    relaunch_ms = runner.time_attention(20) if args.profile_steps > 0 else None

    ms_per_step = elapsed * 1e3 / args.steps
    value = batch * args.steps / elapsed
    step_gbs = step_byte_total / elapsed / 1e9

    result = {
        "metric": metric_name(model_key, batch),
        "value": round(value, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (device-generated weights ~N(0,0.02), random KV prefixes ~N(0,1), seeded)",
        "config": {"workload": desc, "batch": batch, "contexts_mean": round(float(np.mean(contexts)), 1),
                   "decode_steps_timed": args.steps, "page_tokens": 16, "physical_pages": phys_pages,
                   "graphs": not args.eager, "profile_steps": args.profile_steps},
        "device_ms_per_step": round(device_ms / args.steps, 4),  # HIP events around each step on the stream
        "device_ms_median": round(float(np.median(step_device_ms)), 4),
        "step_hbm": {"achieved": round(step_gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(step_gbs / PEAK_HBM_GBS, 4),
                     "bytes_per_step": int(step_byte_total / args.steps)},
    }
    if class_ms:
        # The dominant kernel class, timed inside the step: an event pair on the
        # runner's stream around each of its launches in the profiled eager
        # steps; algorithmic bytes per launch from the same steps' contexts.
        dominant = max(class_ms, key=lambda k: class_ms[k])
        avg_ms = class_ms[dominant] / max(class_launches[dominant], 1)
        bytes_per_launch = class_bytes.get(dominant, 0) / max(class_launches[dominant], 1)
        achieved = bytes_per_launch / (avg_ms * 1e-3) / 1e9
        traffic = measured_traffic(name) if dominant == "attention" else None
        result["roofline"] = {"kernel": dominant, "bound": "hbm", "achieved": round(achieved, 1),
                              "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(achieved / PEAK_HBM_GBS, 4),
                              "traffic": traffic, "avg_launch_us": round(avg_ms * 1e3, 2),
                              "algorithmic_bytes_per_launch": int(bytes_per_launch),
                              "launches": class_launches[dominant],
                              "timing": f"HIP events around each of the {class_launches[dominant]} {dominant} launches "
                                        f"of {args.profile_steps} eager steps"}
        if dominant == "attention" and relaunch_ms:
            last = kernel_bytes(cfg, batch, positions, limits.page_table_stride)["attention"]
            result["roofline"]["relaunch"] = {
                "avg_launch_us": round(relaunch_ms * 1e3, 2), "algorithmic_bytes_per_launch": int(last),
                "achieved": round(last / (relaunch_ms * 1e-3) / 1e9, 1),
                "timing": "last layer's attention launch of the last step, re-run 20 times back to back"}
        if traffic:
            result["roofline"]["traffic_source"] = TRAFFIC_PROFILE
        result["kernels"] = {
            k: {"ms_per_step": round(class_ms[k] / args.profile_steps, 4),
                "gbs": round(class_bytes.get(k, 0) / (class_ms[k] * 1e-3) / 1e9, 1) if class_ms[k] > 0 else None}
            for k in sorted(class_ms, key=lambda k: -class_ms[k])}
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, contexts, args, args.seed)
    runner.close()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
