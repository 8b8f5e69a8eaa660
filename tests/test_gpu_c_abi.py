"""The C ABI driven from plain C (tests/c/abi_decode.c, built by build()):
greedy decode with caller-owned page lists, a rejected row that leaves the
context usable, and a prefill batch. The same scenario through the Python
runner must give the same choices, step by step."""

import subprocess
from pathlib import Path

import numpy as np
import pytest

import ferric_amd
from ferric_amd import PagedLimits, PreparedBatch, PreparedRow, TpBatchRunner

pytestmark = pytest.mark.gpu

BIN = Path(__file__).resolve().parent / "c" / "abi_decode"
SEQS, STEPS, STRIDE, POOL, PREFILL = 4, 6, 16, 96, 20


def _pages():
    # The C program's permutation: LCG-driven Fisher-Yates over the pool.
    perm = list(range(POOL))
    lcg = 0x9E3779B97F4A7C15
    for i in range(POOL - 1, 0, -1):
        lcg = (lcg * 6364136223846793005 + 1442695040888963407) % (1 << 64)
        j = (lcg >> 33) % (i + 1)
        perm[i], perm[j] = perm[j], perm[i]
    return [np.array(perm[s * STRIDE:(s + 1) * STRIDE], np.uint32) for s in range(SEQS + 1)]


def _python_scenario():
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=2)
    limits = PagedLimits(context_tokens=STRIDE * 16, physical_page_count=POOL, page_table_stride=STRIDE)
    runner = TpBatchRunner(cfg, limits, row_capacity=8, use_graphs=True, prefill_rows=64)
    pages = _pages()
    prefix = [5, 17, 40, 100]
    lines = [f"row_capacity {runner.row_capacity()}"]
    try:
        runner.synthesize_weights(7, 0.02)
        fill = [PreparedRow(s + 1, 0, prefix[s], pages[s], int(pages[s][prefix[s] // 16])) for s in range(SEQS)]
        runner.kv_fill_synthetic(5, 1.0, fill, [11, 12, 13, 14], STRIDE * 16)
        tokens = [1000, 2000, 3000, 4000]
        batch = 1
        for step in range(STEPS):
            rows = [PreparedRow(s + 1, tokens[s], prefix[s] + step, pages[s], int(pages[s][(prefix[s] + step) // 16]))
                    for s in range(SEQS)]
            out = runner.execute_batch(PreparedBatch(batch, rows, limits), list(range(SEQS)))
            batch += 1
            tokens = list(out.choices)
            lines.append(f"decode {step}: " + " ".join(str(c) for c in tokens))
        batch += 1  # the C program's rejected batch used this id
        prompt = [PreparedRow(SEQS + 1, 100 + 37 * i, i, pages[SEQS], int(pages[SEQS][i // 16]))
                  for i in range(PREFILL)]
        first = runner.execute_batch(PreparedBatch(batch, prompt, limits), [PREFILL - 1]).choices[0]
        batch += 1
        lines.append(f"prefill: {first}")
        row = PreparedRow(SEQS + 1, first, PREFILL, pages[SEQS], int(pages[SEQS][PREFILL // 16]))
        nxt = runner.execute_batch(PreparedBatch(batch, [row], limits), [0]).choices[0]
        lines.append(f"after prefill: {nxt}")
    finally:
        runner.close()
    return lines


def test_c_host_matches_python_runner():
    if not BIN.exists():
        pytest.fail(f"{BIN} is not built (run ferric_amd/build.py)")
    print(f"running {BIN.name}", flush=True)
    proc = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    got = proc.stdout.strip().splitlines()
    assert got[-1] == "done"
    assert any(line.startswith("invalid row: status 3, message set") for line in got), got  # FH_ERR_INVALID_ROW
    assert any(line.startswith("dispatches ") for line in got)
    expected = _python_scenario()
    compared = [line for line in got if line.split(":")[0].split(" ")[0] in ("row_capacity", "decode", "prefill", "after")]
    assert compared == expected
