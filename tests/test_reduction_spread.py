"""The reduction-order yardstick on the CPU (tests/spread.py): the two legal
orders of the reference's arithmetic (serial v1 sums, wave-order profiles)
stay within the per-layer bar of each other, and a planted mistake (the
gate/up projections narrowed by truncation: oracle order 2) fails the same
per-layer check the GPU parity tests apply, although end to end it looks like
any other order. Also pins the committed spread fixture's shape."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as orc
from tests import spread as sp

GOLDEN = Path(__file__).resolve().parent / "golden" / "reduction_spread.json"


def _small_case():
    cfg = dict(sp.QWEN3_0_6B, layers=4, vocabulary=4096)
    rng = np.random.default_rng(9)
    lengths = [int(x) for x in rng.integers(16, 300, 12)]
    pages = sum(L // 16 + 2 for L in lengths)
    stride = max(L // 16 + 2 for L in lengths)
    t = np.full((len(lengths), stride), 0xFFFFFFFF, np.uint32)
    nxt = 0
    for i, L in enumerate(lengths):
        n = L // 16 + 1
        t[i, :n] = np.arange(nxt, nxt + n)
        nxt += n
    m = orc.Model(cfg, pages)
    m.synthesize(3, 0.02)
    m.kv_fill(4, 1.0, t, stride, lengths, list(range(1, len(lengths) + 1)), 512)
    toks = [int(x) for x in rng.integers(0, cfg["vocabulary"], len(lengths))]
    counts = np.asarray([(L + 16) // 16 for L in lengths], np.uint32)
    return cfg, m, toks, lengths, t, counts, stride


def test_planted_mistake_fails_the_per_layer_bar_that_a_legal_order_passes():
    cfg, m, toks, pos, t, counts, stride = _small_case()
    try:
        ref = m.forward(toks, pos, t, counts, stride, want_hidden=True)
        H, V = cfg["hidden"], cfg["vocabulary"]
        inp = orc.embedding(np.array(toks, np.uint32), m.weight(1, 0xFFFFFFFF, V * H), H, V).reshape(-1, H)
        rms = {1: [], 2: []}
        for layer in range(cfg["layers"]):
            iso = m.layer_isolated(layer, inp, pos, t, counts, stride)
            for order in (1, 2):
                rms[order].append(sp.rms_rel(m.layer_isolated(layer, inp, pos, t, counts, stride, order=order), iso))
            inp = ref["hidden"][layer]
        print("wave", [f"{x:.1e}" for x in rms[1]], "planted", [f"{x:.1e}" for x in rms[2]])
        assert all(p > 3 * w for p, w in zip(rms[2], rms[1])), "the planted mistake moves every layer more"
        sp.check_layer_errors(rms[1], rms[1], "wave order against itself")
        with pytest.raises(AssertionError):
            sp.check_layer_errors(rms[2], rms[1], "planted mistake")
    finally:
        m.close()


def test_spread_fixture_shape():
    if not GOLDEN.exists():
        pytest.skip("spread fixture not generated")
    data = json.loads(GOLDEN.read_text())
    for name, case in data.items():
        spec = sp.decode_case(name)
        for st in case["steps"]:
            w = st["wave_vs_serial"]
            assert len(st["serial_choices"]) == len(spec["lengths"]) == len(st["serial_gaps"])
            assert w["logit_max"] > 0 and w["drift_max"] > 0
            assert len(w["drift"]) == spec["cfg"]["layers"]
            for f in w["flips"]:  # the wave order flips only where the serial top-2 gap is small
                assert f["gap"] == st["serial_gaps"][f["row"]] and f["gap"] < w["logit_max"]
