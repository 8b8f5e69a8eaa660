"""Workload cases of the model-level parity tests and the reduction-order
spread that bounds their end-to-end drift (torch-free: also used on the CPU
by tests/golden/make_reduction_spread.py).

Why a spread. The reference computes the same Qwen3 step with several legal
FP32 summation orders: its serial v1 kernel roots and its wave-order resident
profiles (device/qwen3-tp-batch32-kernels-v5/src/projection.rs:15,
device/qwen3-tp-wave-rmsnorm-kernels-v15/src/rmsnorm.rs:20,
device/qwen3-tp-wave-query-hoist-kernels-v14/src/attention.rs:11). Each bf16
narrowing turns a last-bit FP32 difference into a one-ulp bf16 difference now
and then, and 28-36 layers amplify those. The oracle runs both orders on the
same inputs; their end-to-end difference is the intrinsic spread of the
reference's own arithmetic. A third legal order (the GPU's MFMA tiles,
split-K slabs and wave reductions) must stay within a small multiple of it,
and may only flip greedy choices whose top-2 gap that spread can explain.
End to end, deep models amplify every perturbation to a similar level, so
the discriminating bar is per layer: each layer's own RMS error (on the same
input and KV history) against the wave order's. A 1-ulp-biased rounding in
one projection (oracle order 2, a planted mistake) lands 4-13x the wave
order there, on every layer.
"""

from __future__ import annotations

import numpy as np

# A layer's own error (the run's layer output against the serial oracle's
# layer on the same input and KV history) is measured as a relative RMS over
# the whole residual stream, and its mean over the layer outputs a test checks
# may be at most LAYER_FACTOR times the wave-order oracle's on the same inputs. The maximum element error
# does not separate a legal reassociation from a bug (both saturate at a bf16
# ulp or two of the row maximum); the RMS counts how many elements move.
# Measured on the CPU (Qwen3-0.6B shape, 28 layers, batch 32): wave-vs-serial
# 2.6e-4 .. 2.0e-3 per layer; gate/up narrowed by truncation (oracle order 2)
# 2.4e-3 .. 8.1e-3, 4-13x the wave order on every layer.
LAYER_FACTOR = 2.0
LAYER_RMS_FLOOR = 1e-4  # a fully bit-equal layer pair measures 0; ~1 flip per 1e4 elements
# End-to-end drift allowed for a third order, as a multiple of the
# oracle-vs-oracle spread (maximum |logit| difference and maximum per-layer
# hidden drift against the serial run), plus a floor for shallow models whose
# spread is a few bf16 flips (deep models amplify every order's rounding
# differences to a common, much larger level).
SPREAD_FACTOR = 1.5
LOGIT_FLOOR = 1e-2
DRIFT_FLOOR = 4e-3  # about one bf16 ulp of a row's largest element
NEAR_TIE = 1e-3

QWEN3_8B = dict(layers=36, hidden=4096, query_heads=32, kv_heads=8, head_dim=128, intermediate=12288,
                vocabulary=151936, tied_embedding=0, rope_theta=1_000_000, rms_epsilon=1e-6)
QWEN3_0_6B = dict(layers=28, hidden=1024, query_heads=16, kv_heads=8, head_dim=128, intermediate=3072,
                  vocabulary=151936, tied_embedding=1, rope_theta=1_000_000, rms_epsilon=1e-6)


def decode_case(name: str) -> dict:
    """The seeded inputs of one decode workload: model shape, per-sequence KV
    prefix lengths, pool geometry, first input tokens, weight/pool seeds."""
    if name == "qwen3-8b-b32":  # the decode benchmark: 32 rows, contexts U[512, 8192]
        rng = np.random.default_rng(2024)
        lengths = [int(c) for c in rng.integers(512, 8193, 32)]
        cfg, seed, ctx, stride = dict(QWEN3_8B), 33, 8208, 513
    elif name == "qwen3-8b-b1":  # batch 1 at a 4096-token context
        rng = np.random.default_rng(2025)
        lengths = [4096]
        cfg, seed, ctx, stride = dict(QWEN3_8B), 35, 4112 + 16, 258
    elif name == "qwen3-0.6b-b32":  # 32 rows, contexts U[128, 2048]
        rng = np.random.default_rng(2026)
        lengths = [int(c) for c in rng.integers(128, 2049, 32)]
        cfg, seed, ctx, stride = dict(QWEN3_0_6B), 37, 2064 + 16, 130
    else:
        raise KeyError(name)
    tokens = [int(t) for t in rng.integers(0, cfg["vocabulary"], len(lengths))]
    pages = sum(L // 16 + 2 for L in lengths) + 64
    return dict(name=name, cfg=cfg, lengths=lengths, tokens=tokens, seed=seed, kv_seed=99, context_tokens=ctx,
                stride=stride, pages=pages, pool_seed=seed + 1)


def bf16_f64(bits) -> np.ndarray:
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def row_rel_err(a_bits, b_bits) -> float:
    """max over rows of max|a - b| / max|b| (bf16 rows [rows][width])."""
    a, b = bf16_f64(a_bits), bf16_f64(b_bits)
    a, b = a.reshape(a.shape[0], -1), b.reshape(b.shape[0], -1)
    den = np.maximum(np.max(np.abs(b), axis=1), 1e-30)
    return float(np.max(np.max(np.abs(a - b), axis=1) / den))


def rms_rel(a_bits, b_bits) -> float:
    """sqrt(mean((a - b)^2)) / sqrt(mean(b^2)) over bf16 (uint16) or float arrays."""
    if np.asarray(a_bits).dtype == np.uint16:
        a, b = bf16_f64(a_bits), bf16_f64(b_bits)
    else:
        a, b = np.asarray(a_bits, np.float64), np.asarray(b_bits, np.float64)
    den = np.sqrt(np.mean(b * b))
    return float(np.sqrt(np.mean((a - b) ** 2)) / max(den, 1e-30))


def check_layer_errors(rms_run, rms_wave, label: str, factor: float = LAYER_FACTOR,
                       floor: float = LAYER_RMS_FLOOR) -> None:
    """Mean over layers of the run's own per-layer RMS error within factor
    times the wave-order oracle's (each against the serial oracle on the same
    layer input)."""
    got, lim = float(np.mean(rms_run)), factor * max(float(np.mean(rms_wave)), floor)
    assert got <= lim, (f"{label}: mean per-layer RMS error {got:.3e} beyond {factor} x the oracle orders' "
                        f"{float(np.mean(rms_wave)):.3e}")


def compare(run: dict, ref: dict) -> dict:
    """How far `run` (logits [rows][V], hidden [layers][rows][H] bf16,
    choices) is from `ref` (an oracle run with gaps)."""
    d = np.abs(np.asarray(run["logits"], np.float64) - np.asarray(ref["logits"], np.float64))
    drift = [row_rel_err(run["hidden"][l], ref["hidden"][l]) for l in range(len(ref["hidden"]))]
    flips = [dict(row=i, got=int(c), ref=int(ref["choices"][i]), gap=float(ref["gaps"][i]))
             for i, c in enumerate(run["choices"]) if int(c) != int(ref["choices"][i])]
    return dict(logit_max=float(np.max(d)), logit_rms=float(np.sqrt(np.mean(d * d))),
                row_logit_max=[float(x) for x in np.max(d, axis=1)], drift=drift, drift_max=max(drift),
                flips=flips)


def check_within_spread(gpu: dict, spread: dict, label: str) -> None:
    """The end-to-end bound: the run's logit difference and per-layer drift
    (against the serial oracle) stay within SPREAD_FACTOR times the two oracle
    orders' own (plus the shallow-model floors), and every greedy flip either
    happens in the wave-order oracle too or has a top-2 gap below the wave
    order's own largest logit difference on that row (or the 1e-3 near-tie):
    a legal reassociation moved that row's logits by more than the gap."""
    lim = SPREAD_FACTOR * spread["logit_max"] + LOGIT_FLOOR
    assert gpu["logit_max"] <= lim, (
        f"{label}: end-to-end logits differ by {gpu['logit_max']:.3e}, beyond {lim:.3e} (oracle orders "
        f"{spread['logit_max']:.3e})")
    lim = SPREAD_FACTOR * spread["drift_max"] + DRIFT_FLOOR
    assert gpu["drift_max"] <= lim, (
        f"{label}: hidden drift {gpu['drift_max']:.3e}, beyond {lim:.3e} (oracle orders "
        f"{spread['drift_max']:.3e})")
    wave_rows = {f["row"] for f in spread["flips"]}
    for f in gpu["flips"]:
        row_spread = spread["row_logit_max"][f["row"]]
        print(f"{label}: flip on row {f['row']} at gap {f['gap']:.3e}; the wave order's largest logit difference on "
              f"that row {row_spread:.3e}{' (the wave order flips it too)' if f['row'] in wave_rows else ''}")
        assert f["row"] in wave_rows or f["gap"] < max(NEAR_TIE, row_spread), (
            f"{label}: row {f['row']} chose {f['got']} against {f['ref']} at gap {f['gap']:.3e}, which the "
            f"oracle orders' spread on that row ({row_spread:.3e}) does not explain")
