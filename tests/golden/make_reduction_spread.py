#!/usr/bin/env python3
"""Writes tests/golden/reduction_spread.json: for each model-level decode
workload of the GPU parity tests, the CPU oracle run in the reference's two
legal reduction orders (serial v1 sums; wave-order profiles) and in the wave
order with a planted mistake (gate/up narrowed by truncation), on the same
seeded weights, KV prefixes and tokens (teacher-forced on the serial run's
choices), and the end-to-end differences against the serial run.

The GPU tests recompute the serial-vs-wave spread live and check it against
this file (the oracle is deterministic at any thread count), then hold the
GPU's end-to-end drift to spread.SPREAD_FACTOR times it. The planted-mistake
rows show why that end-to-end bound alone cannot catch a small bias: 36
layers amplify any perturbation, legal or not, to about the same level. The
planted mistake is caught by each layer's own RMS error instead
(tests/test_reduction_spread.py).

Usage: python tests/golden/make_reduction_spread.py [case ...]
(default: every case; the 8B batch-32 case needs ~40 GB of host memory and
several minutes on 8 cores).
"""

from __future__ import annotations

import hashlib
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as orc  # noqa: E402
from tests import spread as sp  # noqa: E402

OUT = Path(__file__).resolve().parent / "reduction_spread.json"
STEPS = {"qwen3-8b-b32": 1, "qwen3-8b-b1": 3, "qwen3-0.6b-b32": 3}
# Cases that also run the planted mistake (a multi-step case holds one model
# per order, each with its own KV history; three 8B models exceed the host).
PLANTED = {"qwen3-8b-b32": True, "qwen3-8b-b1": False, "qwen3-0.6b-b32": True}


def pool_tables(case):
    """The page lists PagePool(seed=pool_seed) gives the case's sequences,
    reproduced without the GPU library: a seeded shuffled free list, pages
    handed out per sequence in admission order (ferric_amd/pool.py)."""
    import random

    free = list(range(case["pages"]))
    random.Random(case["pool_seed"]).shuffle(free)
    # admission: each sequence's prefix pages, in order
    tables = [[free.pop() for _ in range((L + 15) // 16)] for L in case["lengths"]]
    # each decode step reserves the page of a row's write slot, in row order
    for step in range(STEPS[case["name"]]):
        for i, L in enumerate(case["lengths"]):
            while (L + step) // 16 >= len(tables[i]):
                tables[i].append(free.pop())
    return tables


def run_case(name):
    case = sp.decode_case(name)
    cfg, stride = case["cfg"], case["stride"]
    steps = STEPS[name]
    rows = len(case["lengths"])
    tables = pool_tables(case)
    t = np.full((rows, stride), 0xFFFFFFFF, np.uint32)
    for i, pg in enumerate(tables):
        t[i, : len(pg)] = pg
    keys = list(range(1, rows + 1))  # sequence ids PagePool assigns in admission order
    models = {}
    t0 = time.time()
    orders = (0, 1, 2) if PLANTED[name] else (0, 1)
    for order in (orders if steps > 1 else (0,)):
        m = orc.Model(cfg, case["pages"])
        m.synthesize(case["seed"], 0.02)
        m.kv_fill(case["kv_seed"], 1.0, t, stride, case["lengths"], keys, case["context_tokens"])
        models[order] = m
    print(f"{name}: models ready in {time.time() - t0:.0f} s", flush=True)
    toks = list(case["tokens"])
    positions = np.asarray(case["lengths"], np.int64)
    result = {"case": name, "steps": []}
    for step in range(steps):
        counts = np.asarray([(p + 16) // 16 for p in positions], np.uint32)
        t1 = time.time()
        if steps == 1:
            # every run rewrites this step's KV slots before attention reads them
            m = models[0]
            runs = {o: m.forward(toks, positions, t, counts, stride, want_hidden=True, order=o)
                    for o in orders[:0:-1]}
            runs[0] = m.forward(toks, positions, t, counts, stride, want_hidden=True)
        else:
            runs = {o: models[o].forward(toks, positions, t, counts, stride, want_hidden=True, order=o)
                    for o in orders}
        ref = runs[0]
        wave = sp.compare(runs[1], ref)
        planted = sp.compare(runs[2], ref) if 2 in runs else None
        entry = {
            "step": step,
            "serial_logits_sha256": hashlib.sha256(np.ascontiguousarray(ref["logits"]).tobytes()).hexdigest(),
            "serial_choices": [int(c) for c in ref["choices"]],
            "serial_gaps": [float(g) for g in ref["gaps"]],
            "wave_vs_serial": {k: wave[k] for k in ("logit_max", "logit_rms", "drift_max", "drift", "flips",
                                                    "row_logit_max")},
        }
        if planted is not None:
            entry["planted_vs_serial"] = {k: planted[k] for k in ("logit_max", "logit_rms", "drift_max", "flips")}
        result["steps"].append(entry)
        print(f"{name} step {step} ({time.time() - t1:.0f} s): wave logit max {wave['logit_max']:.3e} "
              f"rms {wave['logit_rms']:.3e} drift {wave['drift_max']:.3e} flips "
              f"{[(f['row'], round(f['gap'], 4)) for f in wave['flips']]}" +
              (f"; planted logit max {planted['logit_max']:.3e} drift {planted['drift_max']:.3e} flips "
               f"{len(planted['flips'])}" if planted else ""), flush=True)
        toks = [int(c) for c in ref["choices"]]
        positions = positions + 1
    for m in models.values():
        m.close()
    return result


def main():
    names = sys.argv[1:] or list(STEPS)
    data = json.loads(OUT.read_text()) if OUT.exists() else {}
    for name in names:
        data[name] = run_case(name)
        OUT.write_text(json.dumps(data, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main()
