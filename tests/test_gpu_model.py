"""Model-level parity: fh_execute_batch on the GPU against the oracle's
whole-model forward step, on identical seeded weights, KV prefixes and token
inputs (teacher-forced: both sides consume the oracle's greedy choices).

Each step is also run by the oracle in the reference's second legal
reduction order (its wave-order profiles, oracle order 1): the two oracle
orders' difference is the intrinsic spread of the reference's own arithmetic,
the yardstick for the GPU's (a third order). Bars (tests/spread.py):
  * each layer's own error (the oracle's layer l run on the GPU's layer l-1
    output and KV history, against the GPU's layer l): max|gpu - ref| /
    max|ref| <= 2e-2 per row (north star), and the mean of its relative RMS
    over every layer output of the test at most LAYER_FACTOR x the wave
    order's on the same inputs;
  * the head's own error (oracle final norm + FP32 head on the GPU's final
    residual stream): max abs <= 5e-2 (north star), RMS within LAYER_FACTOR x
    the wave order's head;
  * end to end against the serial oracle: logits and per-layer drift within
    SPREAD_FACTOR x the oracle orders' spread (plus a shallow-model floor);
    greedy choices identical except where the wave order flips too or the
    top-2 gap is below that spread (or the 1e-3 near-tie);
  * the GPU's choice is the lowest-id argmax of its own logits;
  * KV page indexing bit-exact: every slot a step writes is the row's
    (pages[pos // 16], pos % 16); every other slot keeps its bits.
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
import ferric_amd  # noqa: E402
from ferric_amd import FerricError, PagedLimits, PagePool, PreparedBatch, PreparedRow, TpBatchRunner  # noqa: E402
from tests import devutil as du  # noqa: E402
from tests import spread as sp  # noqa: E402

HIDDEN_REL = 2e-2
LOGIT_ABS = 5e-2
NEAR_TIE = sp.NEAR_TIE
HEAD_RMS_FLOOR = 1e-6  # FP32 logits: a head whose two orders agree to the last bit measures 0


def tables_of(batch, stride):
    t = np.full((len(batch.rows), stride), 0xFFFFFFFF, np.uint32)
    c = np.zeros(len(batch.rows), np.uint32)
    for i, r in enumerate(batch.rows):
        t[i, : len(r.physical_pages)] = r.physical_pages
        c[i] = len(r.physical_pages)
    return t, c


class Pair:
    """A GPU runner and the CPU oracle model with identical contents."""

    def __init__(self, cfg, limits, seed=7, capture=True, graphs=False, rows=32, prefill_rows=0, pool_seed=None,
                 wave_model=True):
        """wave_model: keep a second oracle model in wave order with its own
        KV history (needed from the second step on, and for the KV check);
        without it the wave-order run of a step reuses the serial model (valid
        only while both share the synthetic KV prefix, i.e. on a first step)."""
        self.cfg, self.limits = cfg, limits
        self.gpu = TpBatchRunner(cfg, limits, row_capacity=rows, use_graphs=graphs, capture_hidden=capture,
                                 prefill_rows=prefill_rows)
        self.gpu.synthesize_weights(seed, 0.02)
        print(f"oracle: {cfg['layers']} layers, hidden {cfg['hidden']}, {limits.physical_page_count} pages", flush=True)
        self.cpu = orc.Model(cfg, limits.physical_page_count)
        self.cpu.synthesize(seed, 0.02)
        self.cpu_wave = None
        if wave_model:
            self.cpu_wave = orc.Model(cfg, limits.physical_page_count)
            self.cpu_wave.synthesize(seed, 0.02)
            self.cpu_wave.set_order(1)
        self.pool = PagePool(limits, seed=seed + 1 if pool_seed is None else pool_seed)
        self.steps = 0
        self.written = {}
        self.rms_gpu, self.rms_wave = [], []  # every layer output checked so far (all steps)

    @classmethod
    def for_case(cls, case, graphs=True, rows=32, wave_model=True):
        """The seeded decode workload `case` (tests/spread.py decode_case)."""
        limits = PagedLimits(context_tokens=case["context_tokens"], physical_page_count=case["pages"],
                             page_table_stride=case["stride"])
        pair = cls(case["cfg"], limits, seed=case["seed"], graphs=graphs, rows=rows, pool_seed=case["pool_seed"],
                   wave_model=wave_model)
        sids = pair.admit_with_prefix(case["lengths"], kv_seed=case["kv_seed"])
        return pair, sids

    def admit_with_prefix(self, lengths, kv_seed=99):
        sids = [self.pool.admit(L) for L in lengths]
        rows = [PreparedRow(s, 0, L, tuple(self.pool.sequences[s].pages),
                            self.pool.sequences[s].pages[L // 16] if L // 16 < len(self.pool.sequences[s].pages)
                            else 0)
                for s, L in zip(sids, lengths)]
        fill = [r for r in rows if r.position > 0]
        if fill:
            keys = [r.sequence for r in fill]
            # pages must cover the prefix; the writable page is irrelevant for the fill
            self.gpu.kv_fill_synthetic(kv_seed, 1.0, fill, keys, self.limits.context_tokens)
            t = np.full((len(fill), self.limits.page_table_stride), 0xFFFFFFFF, np.uint32)
            for i, r in enumerate(fill):
                t[i, : len(r.physical_pages)] = r.physical_pages
            print(f"oracle: KV prefixes of {len(fill)} sequences", flush=True)
            for m in (self.cpu, self.cpu_wave):
                if m is not None:
                    m.kv_fill(kv_seed, 1.0, t, self.limits.page_table_stride, [r.position for r in fill], keys,
                              self.limits.context_tokens)
        return sids

    def step(self, rows, outs=None):
        """One step; `outs` selects the output rows (default: every row). The
        oracle runs the step in wave order (its own model, or first on the
        serial model, whose KV pool the serial run then rewrites) and in
        serial order; logits, choices and gaps are narrowed to the output rows."""
        batch = self.pool.prepare(rows)
        outs = list(range(len(rows))) if outs is None else list(outs)
        out = self.gpu.execute_batch(batch, outs)
        stride = self.limits.page_table_stride
        t, c = tables_of(batch, stride)
        toks, pos = [r.token for r in batch.rows], [r.position for r in batch.rows]
        if self.cpu_wave is not None:
            wave = self.cpu_wave.forward(toks, pos, t, c, stride, want_logits=True, want_hidden=True)
        else:
            assert self.steps == 0, "a later step needs the wave-order model's own KV history"
            wave = self.cpu.forward(toks, pos, t, c, stride, want_logits=True, want_hidden=True, order=1)
        ref = self.cpu.forward(toks, pos, t, c, stride, want_logits=True, want_hidden=True)
        self.steps += 1
        for r in batch.rows:
            self.written[(int(r.writable_physical_page), int(r.position) % 16)] = True
        for run in (ref, wave):
            for key in ("logits", "choices", "gaps"):
                run[key] = run[key][outs]
        ref["tables"], ref["counts"], ref["outs"], ref["wave"] = t, c, outs, wave
        self.pool.commit(batch)
        return batch, out, ref

    def check(self, batch, out, ref, label):
        """Applies every bar of the module docstring to one step; returns
        (worst per-layer max rel err, head max abs err)."""
        logits = self.gpu.read_logits()
        outs = ref["outs"]
        # the GPU's greedy choice is the lowest-id argmax of its own logits
        for i, c in enumerate(out.choices):
            row = logits[i]
            assert c == int(np.flatnonzero(row == row.max())[0]), (label, i)
        L = self.cfg["layers"]
        hidden = [self.gpu.read_hidden(layer) for layer in range(L)]
        positions = [r.position for r in batch.rows]
        V, H = self.cfg["vocabulary"], self.cfg["hidden"]
        table = self.cpu.weight(1, 0xFFFFFFFF, V * H)
        inp = orc.embedding(np.array([r.token for r in batch.rows], np.uint32), table, H, V).reshape(-1, H)
        per_layer, rms_gpu, rms_wave = [], [], []
        stride = self.limits.page_table_stride
        # After the first step the GPU's KV history differs from the oracle's by
        # the end-to-end drift: the isolated layers then attend over the GPU's.
        gpu_kv = self.steps > 1
        for layer in range(L):
            g = hidden[layer]
            kv = (self.gpu.read_kv_cache(layer, 0), self.gpu.read_kv_cache(layer, 1)) if gpu_kv else None
            iso = self.cpu.layer_isolated(layer, inp, positions, ref["tables"], ref["counts"], stride, kv=kv)
            iso_w = self.cpu.layer_isolated(layer, inp, positions, ref["tables"], ref["counts"], stride, order=1,
                                            kv=kv)
            per_layer.append(sp.row_rel_err(g, iso))
            rms_gpu.append(sp.rms_rel(g, iso))
            rms_wave.append(sp.rms_rel(iso_w, iso))
            inp = g
        print(f"{label}: per-layer max rel err " + " ".join(f"{e:.1e}" for e in per_layer))
        print(f"{label}: per-layer RMS gpu  " + " ".join(f"{e:.1e}" for e in rms_gpu))
        print(f"{label}: per-layer RMS wave " + " ".join(f"{e:.1e}" for e in rms_wave))
        print(f"{label}: mean per-layer RMS gpu {np.mean(rms_gpu):.3e}, wave {np.mean(rms_wave):.3e} "
              f"(ratio {np.mean(rms_gpu) / max(np.mean(rms_wave), 1e-30):.2f})")
        if np.mean(rms_gpu) > 1.5 * max(np.mean(rms_wave), sp.LAYER_RMS_FLOOR):
            self._row_report(label, hidden, batch, ref, gpu_kv)
        assert max(per_layer) <= HIDDEN_REL, f"{label}: hidden rel err {max(per_layer)}"
        # The bar is on the mean over every layer output the test has checked
        # (all its steps): a step of a few rows holds only a handful of the
        # rare early one-ulp divergences that either order makes now and then.
        self.rms_gpu += rms_gpu
        self.rms_wave += rms_wave
        print(f"{label}: mean over the test's {len(self.rms_gpu)} layer outputs: gpu {np.mean(self.rms_gpu):.3e}, "
              f"wave {np.mean(self.rms_wave):.3e}")
        sp.check_layer_errors(self.rms_gpu, self.rms_wave, label)
        # The head's own error, on the GPU's final residual stream of the output rows.
        # The spread is the larger of two legal orders' differences from the
        # serial head: the wave order's, and the exactly summed final norm's
        # (order 3). One row's final norm can flip a few dozen elements by an
        # ulp between orders (repeated mantissas sit on the same rounding
        # boundary) while the serial and wave sums happen to agree.
        final = hidden[-1][outs]
        iso = self.cpu.head(final)
        iso_w = self.cpu.head(final, order=1)
        iso_x = self.cpu.head(final, order=3)
        lerr = float(np.max(np.abs(logits - iso["logits"])))
        head_gpu, head_wave = sp.rms_rel(logits, iso["logits"]), sp.rms_rel(iso_w["logits"], iso["logits"])
        head_exact = sp.rms_rel(iso_x["logits"], iso["logits"])
        print(f"{label}: head max abs err {lerr:.2e}, RMS gpu {head_gpu:.3e} wave {head_wave:.3e} "
              f"exact-sum norm {head_exact:.3e}")
        assert lerr <= LOGIT_ABS, f"{label}: logits abs err {lerr}"
        sp.check_layer_errors([head_gpu], [max(head_wave, head_exact)], label + " (head)", floor=HEAD_RMS_FLOOR)
        # End to end against the serial run, within the oracle orders' spread.
        run = {"logits": logits, "hidden": hidden, "choices": out.choices}
        e2e, spread = sp.compare(run, ref), sp.compare(ref["wave"], ref)
        print(f"{label}: end-to-end logits gpu {e2e['logit_max']:.3e} wave {spread['logit_max']:.3e}; drift gpu "
              f"{e2e['drift_max']:.3e} wave {spread['drift_max']:.3e}; flips gpu "
              f"{[(f['row'], round(f['gap'], 4)) for f in e2e['flips']]} wave "
              f"{[(f['row'], round(f['gap'], 4)) for f in spread['flips']]}")
        sp.check_within_spread(e2e, spread, label)
        return max(per_layer), lerr

    def _row_report(self, label, hidden, batch, ref, gpu_kv):
        """Per-row detail of the layers' own errors (printed when the mean is
        well above the wave order's): which rows and layers carry it."""
        positions = [r.position for r in batch.rows]
        V, H = self.cfg["vocabulary"], self.cfg["hidden"]
        table = self.cpu.weight(1, 0xFFFFFFFF, V * H)
        inp = orc.embedding(np.array([r.token for r in batch.rows], np.uint32), table, H, V).reshape(-1, H)
        stride = self.limits.page_table_stride
        for layer in range(self.cfg["layers"]):
            kv = (self.gpu.read_kv_cache(layer, 0), self.gpu.read_kv_cache(layer, 1)) if gpu_kv else None
            iso = self.cpu.layer_isolated(layer, inp, positions, ref["tables"], ref["counts"], stride, kv=kv)
            iso_w = self.cpu.layer_isolated(layer, inp, positions, ref["tables"], ref["counts"], stride, order=1,
                                            kv=kv)
            g = hidden[layer]
            for i in range(g.shape[0]):
                print(f"{label}: layer {layer} row {i} pos {positions[i]} seq {batch.rows[i].sequence}: RMS gpu "
                      f"{sp.rms_rel(g[i], iso[i]):.2e} wave {sp.rms_rel(iso_w[i], iso[i]):.2e}, differing "
                      f"{int(np.sum(g[i] != iso[i]))} / {int(np.sum(iso_w[i] != iso[i]))} of {g.shape[1]}")
            inp = g

    def check_kv(self, layer_list=None):
        """KV pools after the steps: every slot no step wrote is bit-equal to
        the oracle's (indexing is bit-exact), and the written slots differ from
        the serial oracle's by at most SPREAD_FACTOR x what the wave-order
        oracle's own written slots do (plus a bf16-ulp floor)."""
        assert self.cpu_wave is not None, "the KV check compares against the wave-order model's own KV"
        layers = layer_list if layer_list is not None else range(self.cfg["layers"])
        P = self.limits.physical_page_count
        slot_mask = np.zeros((P, 16), bool)
        for page, slot in self.written:
            slot_mask[page, slot] = True
        worst_gpu = worst_wave = 0.0
        for layer in layers:
            for which in (0, 1):
                got = self.gpu.read_kv_cache(layer, which).reshape(P, 16, -1)
                ref = self.cpu.kv(layer, which).reshape(P, 16, -1)
                wav = self.cpu_wave.kv(layer, which).reshape(P, 16, -1)
                differ = np.any(got != ref, axis=2)
                bad = np.argwhere(differ & ~slot_mask)
                assert len(bad) == 0, f"layer {layer} kv {which}: unwritten slots changed, e.g. {bad[:4].tolist()}"
                if slot_mask.any():
                    g, r, w = (sp.bf16_f64(a[slot_mask]) for a in (got, ref, wav))
                    den = np.maximum(np.max(np.abs(r), axis=1), 1e-30)
                    worst_gpu = max(worst_gpu, float(np.max(np.max(np.abs(g - r), axis=1) / den)))
                    worst_wave = max(worst_wave, float(np.max(np.max(np.abs(w - r), axis=1) / den)))
        lim = sp.SPREAD_FACTOR * worst_wave + sp.DRIFT_FLOOR
        print(f"KV written slots: worst rel err gpu {worst_gpu:.3e}, wave order {worst_wave:.3e}")
        assert worst_gpu <= lim, f"written KV slots differ by {worst_gpu:.3e}, beyond {lim:.3e}"

    def close(self):
        self.gpu.close()
        self.cpu.close()
        if self.cpu_wave is not None:
            self.cpu_wave.close()


def _mark_written(pair, batch):
    """Slots a batch run outside Pair.step writes (Pair.step records its own)."""
    for r in batch.rows:
        pair.written[(int(r.writable_physical_page), int(r.position) % 16)] = True


def test_small_qwen3_decode_matches_oracle():
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=2)
    limits = PagedLimits(context_tokens=1536, physical_page_count=320, page_table_stride=96)
    pair = Pair(cfg, limits, seed=11)
    try:
        rng = np.random.default_rng(5)
        lengths = [0, 1, 15, 16, 300, 1000]
        sids = pair.admit_with_prefix(lengths)
        toks = rng.integers(0, cfg["vocabulary"], len(sids))
        worst = (0.0, 0.0)
        for step in range(3):
            rows = list(zip(sids, [int(t) for t in toks]))
            batch, out, ref = pair.step(rows)
            _mark_written(pair, batch)
            h, l = pair.check(batch, out, ref, f"step {step}")
            worst = (max(worst[0], h), max(worst[1], l))
            toks = ref["choices"]
        # a multi-row batch of one sequence (prefill-style rows, positions 0..15) beside decode rows
        new = pair.pool.admit(0)
        prompt = rng.integers(0, cfg["vocabulary"], 16)
        rows = [(new, int(t)) for t in prompt] + [(sids[4], int(toks[4])), (sids[5], int(toks[5]))]
        batch, out, ref = pair.step(rows)
        _mark_written(pair, batch)
        pair.check(batch, out, ref, "prefill rows")
        pair.check_kv()
        print(f"worst hidden rel err {worst[0]:.3e}, worst logits abs err {worst[1]:.3e}")
    finally:
        pair.close()


def test_qwen3_8b_layer_shapes_match_oracle():
    # 8B layer geometry (hidden 4096, 32 q heads on 8 KV heads, FFN 12288, untied head), one layer.
    cfg = dict(ferric_amd.QWEN3_8B, layers=1)
    limits = PagedLimits(context_tokens=4096, physical_page_count=640, page_table_stride=256)
    pair = Pair(cfg, limits, seed=21, rows=8)
    try:
        rng = np.random.default_rng(9)
        lengths = [3, 64, 257, 1023, 2500, 4000]
        sids = pair.admit_with_prefix(lengths)
        toks = rng.integers(0, cfg["vocabulary"], len(sids))
        for step in range(2):
            batch, out, ref = pair.step(list(zip(sids, [int(t) for t in toks])))
            _mark_written(pair, batch)
            pair.check(batch, out, ref, f"8b step {step}")
            toks = ref["choices"]
        pair.check_kv()
    finally:
        pair.close()


def test_small_batches_merge_attention_partitions_in_kernel():
    # Launches of at most 1024 partition workgroups merge their attention
    # partitions in the partition kernel (the last partition of each (row, KV
    # head) to finish). A 2-layer 8B-shaped model, two steps each, graph path,
    # against the oracle: one row at a 30000-token context (16-page
    # partitions, 118 of them: more than one 64-lane chunk of partition
    # weights in the merge), and four rows at up to 8000 tokens (32-page
    # partitions, several rows per launch).
    cfg = dict(ferric_amd.QWEN3_8B, layers=2)
    cases = [([30000], PagedLimits(context_tokens=30080, physical_page_count=2000, page_table_stride=1880)),
             ([8000, 5003, 700, 3001], PagedLimits(context_tokens=8192, physical_page_count=1200, page_table_stride=512))]
    for lengths, limits in cases:
        pair = Pair(cfg, limits, seed=23, rows=len(lengths), graphs=True)
        try:
            sids = pair.admit_with_prefix(lengths)
            toks = [int(t) for t in np.random.default_rng(len(lengths)).integers(0, cfg["vocabulary"], len(sids))]
            for step in range(2):
                batch, out, ref = pair.step(list(zip(sids, toks)))
                _mark_written(pair, batch)
                pair.check(batch, out, ref, f"{len(lengths)} rows step {step}")
                toks = [int(c) for c in ref["choices"]]
            pair.check_kv()
        finally:
            pair.close()


def test_short_context_capacity_takes_one_partition():
    # A context capacity of 257..512 tokens takes one 32-page partition per
    # row whatever the batch (no partition records, no merge; the speculative
    # draft's form). Against the oracle, two steps each through the graph
    # path: the 0.6B shape at 7 rows (16-page partitions otherwise) with the
    # QK-norm inside the partitions, and the 8B shape at 2 rows (2 x 32 query
    # heads, also 16-page otherwise).
    cases = [(dict(ferric_amd.QWEN3_0_6B, layers=2), [0, 15, 100, 257, 300, 480, 500]),
             (dict(ferric_amd.QWEN3_8B, layers=2), [301, 497])]
    limits = PagedLimits(context_tokens=512, physical_page_count=256, page_table_stride=32)
    for cfg, lengths in cases:
        pair = Pair(cfg, limits, seed=29, rows=len(lengths), graphs=True)
        try:
            sids = pair.admit_with_prefix(lengths)
            toks = [int(t) for t in np.random.default_rng(len(lengths)).integers(0, cfg["vocabulary"], len(sids))]
            for step in range(2):
                batch, out, ref = pair.step(list(zip(sids, toks)))
                _mark_written(pair, batch)
                pair.check(batch, out, ref, f"{cfg['hidden']} x {len(lengths)} rows at capacity 512, step {step}")
                toks = [int(c) for c in ref["choices"]]
            pair.check_kv()
        finally:
            pair.close()


GOLDEN_SPREAD = Path(__file__).resolve().parent / "golden" / "reduction_spread.json"


def _check_against_golden(case_name, step, ref):
    """The oracle is deterministic at any thread count: its serial logits and
    its two orders' spread must equal what tests/golden/make_reduction_spread.py
    measured for the same case in the build container."""
    golden = json.loads(GOLDEN_SPREAD.read_text()).get(case_name) if GOLDEN_SPREAD.exists() else None
    if golden is None or step >= len(golden["steps"]):
        return
    g = golden["steps"][step]
    sha = hashlib.sha256(np.ascontiguousarray(ref["logits"]).tobytes()).hexdigest()
    assert sha == g["serial_logits_sha256"], f"{case_name} step {step}: serial oracle logits differ from the fixture"
    spread = sp.compare(ref["wave"], ref)
    assert spread["logit_max"] == g["wave_vs_serial"]["logit_max"], (spread["logit_max"], g["wave_vs_serial"])


def _decode_steps(case_name, steps, rows=32, wave_model=True):
    """`steps` teacher-forced decode steps of a seeded decode workload through
    the HIP-graph path, every bar checked at every step."""
    case = sp.decode_case(case_name)
    pair, sids = Pair.for_case(case, graphs=True, rows=rows, wave_model=wave_model)
    try:
        toks = case["tokens"]
        for step in range(steps):
            print(f"{case_name} step {step}", flush=True)
            batch, out, ref = pair.step(list(zip(sids, toks)))
            _mark_written(pair, batch)
            pair.check(batch, out, ref, f"{case_name} step {step}")
            _check_against_golden(case_name, step, ref)
            toks = [int(c) for c in ref["choices"]]
        return pair
    except BaseException:
        pair.close()
        raise


@pytest.mark.timeout(900)
def test_qwen3_8b_full_depth_batch32_decode_steps():
    # The decode benchmark's shape at full size (the north-star workload):
    # Qwen3-8B with all 36 layers, batch 32, contexts U[512, 8192] on 16-token
    # pages, through the HIP-graph path: 3 teacher-forced steps, so KV that one
    # step writes is read by the next, every bar at every step, and the
    # written KV slots of the first, middle and last layer checked afterwards.
    pair = _decode_steps("qwen3-8b-b32", 3)
    try:
        pair.check_kv(layer_list=[0, 17, 35])
    finally:
        pair.close()


def test_qwen3_8b_batch1_context4096_decode_steps():
    # Batch-1 decode of the 8B shape at a 4096-token context, 3 steps (36
    # layers, graph path, single-row projections and attention).
    pair = _decode_steps("qwen3-8b-b1", 3, rows=1)
    pair.close()


def test_qwen3_0_6b_batch32_decode_steps():
    # The 0.6B shape (28 layers, tied head), batch 32, contexts U[128, 2048]
    # on a shuffled pool, 3 steps; every written KV slot checked afterwards.
    pair = _decode_steps("qwen3-0.6b-b32", 3)
    try:
        pair.check_kv(layer_list=[0, 13, 27])
    finally:
        pair.close()


def test_one_row_steps_with_norms_in_the_projections():
    # One-row steps run every residual + RMSNorm inside the projection after
    # it, the residual stream alternating between two buffers: 4 steps of one
    # row (positions 0 and 700 on), eager and replayed from the graph, must
    # give bit-identical captured layers and logits, each step within the
    # oracle bars, and the written KV slots checked afterwards.
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=3)
    limits = PagedLimits(context_tokens=1024, physical_page_count=128, page_table_stride=64)
    runs = []
    for graphs in (False, True):
        pair = Pair(cfg, limits, seed=13, graphs=graphs, rows=4)
        try:
            sids = pair.admit_with_prefix([0, 700])
            tok, logits, hidden = [17, 4242], [], []
            for step in range(4):
                row = step % 2
                batch, out, ref = pair.step([(sids[row], tok[row])])
                _mark_written(pair, batch)
                pair.check(batch, out, ref, f"one row, graphs {graphs}, step {step}")
                tok[row] = int(ref["choices"][0])
                logits.append(pair.gpu.read_logits().copy())
                hidden.append(np.stack([pair.gpu.read_hidden(l) for l in range(cfg["layers"])]))
            pair.check_kv()
            runs.append((np.stack(logits), np.stack(hidden)))
        finally:
            pair.close()
    assert np.array_equal(runs[0][0].view(np.uint32), runs[1][0].view(np.uint32))
    assert np.array_equal(runs[0][1], runs[1][1])


def test_graph_replay_is_bit_identical_to_eager():
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=2)
    limits = PagedLimits(context_tokens=512, physical_page_count=64, page_table_stride=32)
    results = []
    for graphs in (False, True):
        r = TpBatchRunner(cfg, limits, row_capacity=8, use_graphs=graphs)
        try:
            r.synthesize_weights(3, 0.02)
            pool = PagePool(limits, seed=1)
            s = [pool.admit(0) for _ in range(3)]
            logits = []
            toks = [1, 2, 3]
            for _ in range(4):
                b = pool.prepare(list(zip(s, toks)))
                toks = r.execute_batch(b, [0, 1, 2]).choices
                pool.commit(b)
                logits.append(r.read_logits().copy())
            results.append((toks, np.stack(logits)))
        finally:
            r.close()
    assert results[0][0] == results[1][0]
    assert np.array_equal(results[0][1].view(np.uint32), results[1][1].view(np.uint32))


def test_batch_validation_mirrors_the_reference():
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=1)
    limits = PagedLimits(context_tokens=256, physical_page_count=32, page_table_stride=16)
    r = TpBatchRunner(cfg, limits, row_capacity=4, use_graphs=False)
    try:
        r.synthesize_weights(1, 0.02)

        def run(rows, outs=None, bid=[100]):
            bid[0] += 1
            return r.execute_batch(PreparedBatch(bid[0], rows, limits), outs if outs is not None else [0])

        ok = PreparedRow(1, 5, 3, (4, 9), 4)
        assert len(run([ok]).choices) == 1
        cases = [
            ([], None, 2),                                                     # empty batch
            ([ok] * 5, None, 2),                                               # over row capacity
            ([PreparedRow(1, cfg["vocabulary"], 3, (4,), 4)], None, 3),        # token out of vocabulary
            ([PreparedRow(1, 5, 256, (4,) * 1, 4)], None, 3),                  # position beyond context
            ([PreparedRow(1, 5, 16, (4,), 4)], None, 3),                       # logical page missing
            ([PreparedRow(1, 5, 3, (4, 4), 4)], None, 3),                      # duplicate page in one row
            ([PreparedRow(1, 5, 3, (40,), 40)], None, 3),                      # page outside the pool
            ([PreparedRow(1, 5, 3, (4,), 9)], None, 3),                        # writable page mismatch
            ([ok, PreparedRow(1, 6, 3, (4, 9), 4)], None, 3),                  # aliased write slot
            ([ok, PreparedRow(2, 6, 20, (7, 4), 4)], None, 4),                 # write page shared with another sequence
            ([ok, PreparedRow(1, 6, 4, (4, 9), 4)], [1, 0], 5),                # output rows not ascending
            ([ok], [3], 5),                                                    # output row outside the batch
        ]
        for rows, outs, status in cases:
            with pytest.raises(FerricError) as e:
                run(rows, outs)
            assert e.value.status == status, (rows, e.value)
        # a stale batch id is refused
        with pytest.raises(FerricError) as e:
            r.execute_batch(PreparedBatch(1, [ok], limits), [0])
        assert e.value.status == 2
        # validation failures happen before submission and do not poison the runner
        assert len(run([PreparedRow(1, 7, 4, (4, 9), 4)]).choices) == 1
    finally:
        r.close()


@pytest.mark.parametrize("graphs", [True, False])
def test_device_error_of_a_decode_step_reaches_the_host(graphs):
    # A decode step's error word and choices come back through pinned host
    # memory that the step's last launch writes. A NaN planted in the final
    # norm makes every logit nonfinite: the step (a replay of the graph the
    # good steps captured, or eager launches) must fail with
    # FH_ERR_NONFINITE, and the runner then refuses further steps.
    from ferric_amd import _lib
    from ferric_amd.checkpoint import NO_LAYER

    cfg = dict(ferric_amd.QWEN3_0_6B, layers=1)
    limits = PagedLimits(context_tokens=256, physical_page_count=32, page_table_stride=16)
    r = TpBatchRunner(cfg, limits, row_capacity=4, use_graphs=graphs)
    try:
        r.synthesize_weights(3, 0.02)
        pool = PagePool(limits, seed=3)
        sids = [pool.admit(0), pool.admit(0)]
        toks = [11, 12]
        for _ in range(3):
            b = pool.prepare(list(zip(sids, toks)))
            toks = r.execute_batch(b, [0, 1]).choices
            pool.commit(b)
            assert all(0 <= t < cfg["vocabulary"] for t in toks)
        norm = r.download_weight(_lib.FINAL_NORM, NO_LAYER, cfg["hidden"])
        norm[17] = 0x7FC0
        r.upload_weight(_lib.FINAL_NORM, NO_LAYER, norm)
        b = pool.prepare(list(zip(sids, toks)))
        with pytest.raises(FerricError) as e:
            r.execute_batch(b, [0, 1])
        assert e.value.status == 6, e.value
        with pytest.raises(FerricError) as e:
            r.execute_batch(pool.prepare(list(zip(sids, toks))), [0, 1])
        assert e.value.status == 8, e.value
    finally:
        r.close()


@pytest.mark.parametrize("private", [True, False])
def test_device_error_of_a_prefill_chunk_reaches_the_host(private):
    # A 42-row prefill chunk (the split-K panel path) with a NaN planted in
    # layer 0's query norm weight: the QK-norm's nonfinite check must fail the
    # chunk with FH_ERR_NONFINITE, whether the QK-norm runs inside the block
    # attention (three prompts, one block each) or in its own launch (one
    # prompt in three blocks, the later ones reading the earlier ones' pages).
    from ferric_amd import _lib

    cfg = dict(ferric_amd.QWEN3_8B, layers=1)
    limits = PagedLimits(context_tokens=256, physical_page_count=32, page_table_stride=16)
    r = TpBatchRunner(cfg, limits, row_capacity=8, use_graphs=False, prefill_rows=64)
    try:
        r.synthesize_weights(9, 0.02)
        qn = r.download_weight(_lib.QUERY_NORM, 0, 128)
        qn[5] = 0x7FC0
        r.upload_weight(_lib.QUERY_NORM, 0, qn)
        pool = PagePool(limits, seed=9)
        if private:
            sids = [pool.admit(0) for _ in range(3)]
            rows = [(s, 7 + t) for s in sids for t in range(14)]
        else:
            s = pool.admit(0)
            rows = [(s, 7 + t) for t in range(42)]
        batch = pool.prepare(rows)
        (pre,) = r.expected_dispatch_counts_for_selection(batch, [41])
        assert pre == 2 + 1 + (7 if private else 8) * cfg["layers"] + 5, pre
        with pytest.raises(FerricError) as e:
            r.execute_batch(batch, [41])
        assert e.value.status == 6, e.value
    finally:
        r.close()


def test_full_small_model_prompt_then_greedy_decode():
    # Qwen3-0.6B shape, all 28 layers, batch 1: a 16-token prompt as one
    # 16-row batch, then 8 greedy decode steps (teacher-forced).
    cfg = dict(ferric_amd.QWEN3_0_6B)
    limits = PagedLimits(context_tokens=64, physical_page_count=16, page_table_stride=4)
    pair = Pair(cfg, limits, seed=42, capture=True, rows=16)
    try:
        rng = np.random.default_rng(2024)
        sid = pair.pool.admit(0)
        prompt = [int(t) for t in rng.integers(0, cfg["vocabulary"], 16)]
        batch, out, ref = pair.step([(sid, t) for t in prompt])
        _mark_written(pair, batch)
        pair.check(batch, out, ref, "prompt")
        tok = int(ref["choices"][-1])
        matches = 0
        for step in range(8):
            batch, out, ref = pair.step([(sid, tok)])
            _mark_written(pair, batch)
            pair.check(batch, out, ref, f"decode {step}")
            matches += int(out.choices[0] == ref["choices"][0])
            tok = int(ref["choices"][0])
        print(f"greedy tokens identical at {matches}/8 decode steps")
        assert matches == 8
        pair.check_kv(layer_list=[0, 27])
    finally:
        pair.close()


def _prefill_case(cfg, limits, prompts, decode_lengths, prefill_rows, seed, label):
    """Prompts (from position 0) plus decode rows of sequences with a KV
    prefix, as one batch larger than row_capacity: the prefill path. The
    output rows are each prompt's last token and every decode row."""
    pair = Pair(cfg, limits, seed=seed, rows=8, prefill_rows=prefill_rows)
    try:
        rng = np.random.default_rng(seed)
        dec = pair.admit_with_prefix(decode_lengths) if decode_lengths else []
        rows, outs = [], []
        for n in prompts:
            sid = pair.pool.admit(0)
            rows += [(sid, int(t)) for t in rng.integers(0, cfg["vocabulary"], n)]
            outs.append(len(rows) - 1)
        for sid in dec:
            rows.append((sid, int(rng.integers(0, cfg["vocabulary"]))))
            outs.append(len(rows) - 1)
        assert len(rows) > 8
        batch, out, ref = pair.step(rows, outs)
        _mark_written(pair, batch)
        pair.check(batch, out, ref, label)
        pair.check_kv()
        # the next step decodes every sequence through the 8-row decode path
        seqs = sorted({r.sequence for r in batch.rows})[:8]
        last = {r.sequence: i for i, r in enumerate(batch.rows)}
        toks = {s: int(out.choices[outs.index(last[s])]) for s in seqs}
        batch, out, ref = pair.step([(s, toks[s]) for s in seqs])
        _mark_written(pair, batch)
        pair.check(batch, out, ref, label + " then decode")
    finally:
        pair.close()


def test_prefill_chunk_matches_oracle():
    # 0.6B shape, 2 layers: 280 rows (two 130-token prompts + 20 decode rows),
    # two attention row blocks and a padded 384-row tile buffer.
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=2)
    limits = PagedLimits(context_tokens=2048, physical_page_count=800, page_table_stride=128)
    _prefill_case(cfg, limits, [130, 130], [5, 16, 17, 600, 1500] * 4, 512, 31, "prefill 0.6b")


def test_prefill_chunk_8b_layer_shapes():
    # 8B layer geometry, one layer: a 40-row prompt beside two decode rows.
    cfg = dict(ferric_amd.QWEN3_8B, layers=1)
    limits = PagedLimits(context_tokens=4096, physical_page_count=300, page_table_stride=256)
    _prefill_case(cfg, limits, [40], [100, 3000], 64, 37, "prefill 8b")


def test_prefill_chunk_of_at_most_32_rows():
    # 0.6B shape, 2 layers, row capacity 8: a 15-row chunk (a 12-token prompt
    # beside three decode rows) takes the prefill path with the decode GEMM's
    # split-K partials (32-row slabs) folded by the norms.
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=2)
    limits = PagedLimits(context_tokens=1024, physical_page_count=160, page_table_stride=64)
    _prefill_case(cfg, limits, [12], [50, 300, 7], 32, 53, "prefill 15 rows")


def test_prefill_chunk_8b_fused_qkv_epilogue():
    # 8B layer geometry, one layer, 292 rows: above 256 rows the QKV
    # projection runs the 256 x 256-block kernel with QK-norm, RoPE and the KV
    # append in its epilogue (32 query + 16 key/value heads, 24 column blocks).
    cfg = dict(ferric_amd.QWEN3_8B, layers=1)
    limits = PagedLimits(context_tokens=4096, physical_page_count=320, page_table_stride=256)
    _prefill_case(cfg, limits, [150, 140], [100, 3000], 512, 43, "prefill 8b fused qkv")


def test_prefill_qknorm_inside_block_attention_is_bit_identical():
    # A chunk of up to 256 rows whose attention blocks write no slot another
    # block reads runs the QK-norm, RoPE and KV append inside the attention
    # workgroups. Three 14-token prompts alone take that form; the same three
    # prompts next to a 20-token prompt of a fourth sequence (two blocks, the
    # second reading the first's page) keep the separate QK-norm launch. A
    # row's projections do not depend on the other rows of a 33-256-row
    # chunk, so the three sequences' K/V slots and output logits must be equal
    # bit for bit between the two runs.
    cfg = dict(ferric_amd.QWEN3_8B, layers=2)
    limits = PagedLimits(context_tokens=256, physical_page_count=64, page_table_stride=16)
    rng = np.random.default_rng(71)
    prompts = [rng.integers(0, cfg["vocabulary"], 14) for _ in range(3)]
    extra = rng.integers(0, cfg["vocabulary"], 20)
    got = []
    for with_extra in (False, True):
        runner = TpBatchRunner(cfg, limits, row_capacity=32, use_graphs=False, prefill_rows=256)
        try:
            runner.synthesize_weights(71, 0.02)
            pool = PagePool(limits, seed=72)
            sids = [pool.admit(0) for _ in range(3)]
            rows = [(s, int(t)) for s, p in zip(sids, prompts) for t in p]
            outs = [13, 27, 41]
            if with_extra:
                e = pool.admit(0)
                rows += [(e, int(t)) for t in extra]
            batch = pool.prepare(rows)
            (pre,) = runner.expected_dispatch_counts_for_selection(batch, outs)
            (before,) = runner.dispatch_counts()
            choices = runner.execute_batch(batch, outs).choices
            (after,) = runner.dispatch_counts()
            assert after - before == pre
            logits = runner.read_logits()[: len(outs)].copy()
            # keyed by (layer, K or V, sequence, logical page): the two pools
            # need not place the sequences on the same physical pages
            kv = {(layer, which, i, lp): runner.read_kv_page(layer, which, int(pg))
                  for layer in range(cfg["layers"]) for which in (0, 1)
                  for i, s in enumerate(sids) for lp, pg in enumerate(pool.sequences[s].pages)}
            got.append((pre, choices, logits, kv))
        finally:
            runner.close()
    (pre_a, ch_a, lg_a, kv_a), (pre_b, ch_b, lg_b, kv_b) = got
    # One launch per layer fewer in the fused form.
    assert pre_b - pre_a == cfg["layers"], (pre_a, pre_b)
    assert list(ch_a) == list(ch_b)
    assert np.array_equal(lg_a.view(np.uint32), lg_b.view(np.uint32)), "output logits"
    assert kv_a.keys() == kv_b.keys()
    for key in kv_a:
        assert np.array_equal(kv_a[key], kv_b[key]), key


@pytest.mark.parametrize("nseq", [40, 80])
def test_prefill_chunk_of_single_row_blocks_with_the_qknorm_inside(nseq):
    # nseq sequences with prefixes of 0..600 tokens, one new row each, as one
    # prefill chunk: nseq one-row attention blocks x 8 KV heads (320
    # workgroups: two page phases; 640: one), none reading another's written
    # slot, so the QK-norm, RoPE and KV append run inside the block
    # attention. Against the oracle, then the written slots.
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=2)
    limits = PagedLimits(context_tokens=1024, physical_page_count=3200, page_table_stride=64)
    pair = Pair(cfg, limits, seed=37, rows=32, prefill_rows=128)
    try:
        rng = np.random.default_rng(37 + nseq)
        lengths = [int(x) for x in rng.integers(0, 601, nseq)]
        sids = pair.admit_with_prefix(lengths)
        rows = [(s, int(t)) for s, t in zip(sids, rng.integers(0, cfg["vocabulary"], len(sids)))]
        outs = [0, 17, nseq // 2, nseq - 1]
        batch, out, ref = pair.step(rows, outs)
        _mark_written(pair, batch)
        pair.check(batch, out, ref, f"{nseq} one-row blocks")
        pair.check_kv()
    finally:
        pair.close()


def test_prefill_continuation_and_interleaved_rows():
    # 0.6B shape, 2 layers. Prefill attention groups runs of rows of one
    # sequence at consecutive positions into blocks: a 70-row continuation of
    # a 300-token sequence (blocks starting mid-page, a long prefix in every
    # block), then three sequences' rows interleaved one by one (every block
    # a single row), one of them a new prompt from position 0.
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=2)
    limits = PagedLimits(context_tokens=2048, physical_page_count=400, page_table_stride=128)
    pair = Pair(cfg, limits, seed=41, rows=8, prefill_rows=256)
    try:
        rng = np.random.default_rng(41)
        a, b = pair.admit_with_prefix([300, 37])
        c = pair.pool.admit(0)
        rows = [(a, int(t)) for t in rng.integers(0, cfg["vocabulary"], 70)]
        for _ in range(12):
            for sid in (b, c, a):
                rows.append((sid, int(rng.integers(0, cfg["vocabulary"]))))
        outs = [0, 33, 69, 70, 71, 72, len(rows) - 3, len(rows) - 2, len(rows) - 1]
        batch, out, ref = pair.step(rows, outs)
        _mark_written(pair, batch)
        pair.check(batch, out, ref, "continuation + interleaved prefill")
        pair.check_kv()
    finally:
        pair.close()


def test_prefill_ignores_unwritten_slots_of_the_last_page():
    # A prefill chunk continuing a 37-token sequence to position 76: slots
    # 13..15 of the page holding position 76 are never written by the
    # sequence and hold NaN and infinity patterns here (as a reused page
    # might). The reference never reads past a row's position, so neither
    # the outputs nor the error word may notice them.
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=2)
    limits = PagedLimits(context_tokens=1024, physical_page_count=64, page_table_stride=64)
    pair = Pair(cfg, limits, seed=51, rows=8, prefill_rows=64)
    try:
        (a,) = pair.admit_with_prefix([37])
        st = pair.pool.sequences[a]
        pair.pool._ensure(st, 77)  # reserve the pages the chunk will write
        page = int(st.pages[76 // 16])
        for layer in range(cfg["layers"]):
            for which in (0, 1):
                got = pair.gpu.read_kv_page(layer, which, page).reshape(16, -1)
                ref = pair.cpu.kv(layer, which).reshape(limits.physical_page_count, 16, -1)
                for slot, bits in ((13, 0x7FC0), (14, 0x7F80), (15, 0xFFC1)):
                    got[slot] = bits
                    ref[page, slot] = bits
                pair.gpu.write_kv_page(layer, which, page, got.reshape(-1))
        rng = np.random.default_rng(51)
        rows = [(a, int(t)) for t in rng.integers(0, cfg["vocabulary"], 40)]
        batch, out, ref = pair.step(rows, [0, 20, 39])
        assert batch.rows[len(rows) - 1].position == 76
        _mark_written(pair, batch)
        pair.check(batch, out, ref, "prefill beside unwritten NaN slots")
        pair.check_kv()
    finally:
        pair.close()


class ParityRunner:
    """A TpBatchRunner stand-in for the speculative decoder that runs every
    batch on the GPU and on the oracle (same prepared rows and page tables,
    the oracle in its wave-order and serial models), checks the GPU's choices and
    logits against the serial run within the two orders' spread, and hands the
    GPU's choices on (so both sides always see identical inputs)."""

    def __init__(self, pair: "Pair", label: str):
        self.pair, self.label = pair, label
        self.limits = pair.limits
        self.batches = 0
        self.worst_logit = 0.0
        self.flips = []
        self.last_ref = None

    def execute_batch(self, batch, outs):
        pair = self.pair
        out = pair.gpu.execute_batch(batch, outs)
        stride = pair.limits.page_table_stride
        t, c = tables_of(batch, stride)
        toks, pos = [r.token for r in batch.rows], [r.position for r in batch.rows]
        wave = pair.cpu_wave.forward(toks, pos, t, c, stride, want_logits=True)
        ref = pair.cpu.forward(toks, pos, t, c, stride, want_logits=True)
        _mark_written(pair, batch)
        self.batches += 1
        if outs:
            outs = list(outs)
            logits = pair.gpu.read_logits()
            if len(batch.rows) <= pair.gpu.row_capacity():
                logits = logits[outs]  # a decode batch keeps every row's logits, in row order
            ref_l, wave_l = ref["logits"][outs], wave["logits"][outs]
            e2e = float(np.max(np.abs(logits - ref_l)))
            spread = float(np.max(np.abs(wave_l - ref_l)))
            self.worst_logit = max(self.worst_logit, e2e)
            label = f"{self.label} batch {self.batches}"
            assert e2e <= sp.SPREAD_FACTOR * spread + sp.LOGIT_FLOOR, (label, e2e, spread)
            wave_c = wave["choices"][outs]
            for i, ch in enumerate(out.choices):
                want, gap = int(ref["choices"][outs[i]]), float(ref["gaps"][outs[i]])
                if ch != want:
                    # explained by the wave order's own logit difference on this row
                    row_spread = float(np.max(np.abs(wave_l[i] - ref_l[i])))
                    print(f"{label}: flip on output row {i} at gap {gap:.3e}; wave order's difference on the row "
                          f"{row_spread:.3e}")
                    assert int(wave_c[i]) != want or gap < max(sp.NEAR_TIE, row_spread), (label, i, ch, want, gap)
                    self.flips.append((label, i, gap))
            self.last_ref = {"choices": [int(x) for x in ref["choices"][outs]]}
        return out


SPEC_SHAPES = {
    # name: (target config, draft config, same weights, sequences, rounds)
    "0.6b-same-draft": (dict(ferric_amd.QWEN3_0_6B, layers=2), dict(ferric_amd.QWEN3_0_6B, layers=2), True, 8, 4),
    "0.6b-other-draft": (dict(ferric_amd.QWEN3_0_6B, layers=2), dict(ferric_amd.QWEN3_0_6B, layers=2), False, 8, 4),
    # the speculative benchmark's geometry with 2 layers each: an 8B-shaped
    # target (untied head) and a 0.6B-shaped draft (tied head), 32
    # sequences, so every verify is a 160-row batch
    "8b-target-0.6b-draft": (dict(ferric_amd.QWEN3_8B, layers=2), dict(ferric_amd.QWEN3_0_6B, layers=2), False, 32, 2),
    # the same pair at full depth (36 + 28 layers): 4 sequences, so every
    # verify is a 20-row chunk of the prefill path, every batch of both models
    # against the oracle
    "8b-0.6b-full-depth": (dict(ferric_amd.QWEN3_8B), dict(ferric_amd.QWEN3_0_6B), False, 4, 2),
}


@pytest.mark.timeout(900)
@pytest.mark.parametrize("shape", list(SPEC_SHAPES))
def test_speculative_rounds_match_the_oracle(shape):
    # Greedy speculation (K = 4), every draft step, catch-up and verify batch
    # run on the GPU and on the oracle in lockstep. With identical weights the
    # draft is mostly accepted (every full acceptance exercises the draft
    # catch-up); with other weights mostly rejected. Then: each round's
    # 120-byte completion records equal the oracle's records built from the
    # same round's choices, and both models' KV pools hold, in every slot the
    # rounds wrote (accepted and rejected suffixes alike), the oracle's K/V;
    # nothing else changed.
    from ferric_amd.speculative import SpeculativeDecoder

    cfg_t, cfg_d, same_draft, nseq, rounds = SPEC_SHAPES[shape]
    K = 4
    limits = PagedLimits(context_tokens=256, physical_page_count=160, page_table_stride=16)
    rng = np.random.default_rng(77)
    lengths = (3, 9, 16, 5, 7, 12, 2, 20) if nseq == 8 else tuple(int(n) for n in rng.integers(1, 5, nseq))
    prompts = [list(rng.integers(0, cfg_t["vocabulary"], n)) for n in lengths]
    rows = 32 if nseq > 16 else 16
    prefill = max(sum(lengths), nseq * (K + 1))  # the prompt batch and every verify batch
    tp = Pair(cfg_t, limits, seed=5, capture=False, rows=rows, prefill_rows=prefill)
    dp = Pair(cfg_d, limits, seed=5 if same_draft else 6, capture=False, rows=rows, prefill_rows=prefill)
    try:
        target, draft = ParityRunner(tp, "target"), ParityRunner(dp, "draft")
        dec = SpeculativeDecoder(target, tp.pool, draft, dp.pool, k=K)
        dec.prefill(prompts)  # the prefill path for both models
        accepted = 0
        for rnd in range(rounds):
            draft_steps_before = draft.batches
            st = dec.round()  # verify batch of nseq x (K + 1) rows: the prefill path
            assert st.target_rows == nseq * (K + 1)
            accepted += sum(st.accepted)
            assert draft.batches - draft_steps_before in (K, K + 1)  # K steps, plus a catch-up after a full accept
            # the GPU's verify choices are the oracle's (checked in ParityRunner, up to near-ties)
            gpu_choices = np.asarray(st.target_choices, np.uint32)
            if not target.flips:
                assert gpu_choices.reshape(-1).tolist() == target.last_ref["choices"]
            # each record is the oracle's restatement of the reference's record for the round's choices
            for j, rec in enumerate(st.records):
                want, _ = orc.compact_record(gpu_choices, st.draft, K + 1, j, 1, rnd, dec.plan, len(prompts), j,
                                             K + 1, dec.k)
                assert rec == want, (rnd, j)
                assert rec[48] == st.accepted[j] and rec[49] == len(st.emitted[j])
        print(f"accepted {accepted} of {rounds * K * len(prompts)} draft tokens; flips target {target.flips} "
              f"draft {draft.flips}; worst logit err target {target.worst_logit:.2e} draft {draft.worst_logit:.2e}")
        if same_draft:
            assert accepted >= rounds * K * len(prompts) // 2
        tp.check_kv()
        dp.check_kv()
    finally:
        tp.close()
        dp.close()


def _golden_spread(case_name="qwen3-8b-b32"):
    """The oracle orders' largest logit difference and drift measured for a
    full-depth case (tests/golden/reduction_spread.json)."""
    g = json.loads(GOLDEN_SPREAD.read_text())[case_name]["steps"][0]["wave_vs_serial"]
    return g["logit_max"], g["drift_max"]


def _golden_row_spread(case_name="qwen3-8b-b32"):
    """A typical row's share of that spread: the median over the case's rows
    of the wave order's largest logit difference on the row (the per-row bar
    for comparisons that have no oracle run of their own rows)."""
    g = json.loads(GOLDEN_SPREAD.read_text())[case_name]["steps"][0]["wave_vs_serial"]
    return float(np.median(g["row_logit_max"]))


def test_prefill_8b_full_depth_two_prompts_match_oracle():
    # The prefill path at full depth: Qwen3-8B, all 36 layers, two 160-token
    # prompts as one 320-row chunk (above 256 rows: the 256 x 256-block
    # projections with QK-norm, RoPE and the KV append in the QKV epilogue,
    # and the block attention), every bar of the module docstring applied,
    # then one decode step on the prefilled cache.
    cfg = dict(ferric_amd.QWEN3_8B)
    limits = PagedLimits(context_tokens=192, physical_page_count=64, page_table_stride=12)
    pair = Pair(cfg, limits, seed=63, rows=8, prefill_rows=320)
    try:
        rng = np.random.default_rng(63)
        a, b = pair.pool.admit(0), pair.pool.admit(0)
        rows = [(a, int(t)) for t in rng.integers(0, cfg["vocabulary"], 160)]
        rows += [(b, int(t)) for t in rng.integers(0, cfg["vocabulary"], 160)]
        print("8b prefill 2 x 160: step", flush=True)
        batch, out, ref = pair.step(rows, [0, 159, 160, 319])
        _mark_written(pair, batch)
        pair.check(batch, out, ref, "8b prefill 2 x 160")
        pair.check_kv(layer_list=[0, 18, 35])
        batch, out, ref = pair.step([(a, int(ref["choices"][1])), (b, int(ref["choices"][3]))])
        _mark_written(pair, batch)
        pair.check(batch, out, ref, "8b prefill 2 x 160 then decode")
    finally:
        pair.close()


def test_prefill_32x256_full_size_kv_indexing_and_first_tokens():
    # The speculative workload's prefill at full size: Qwen3-8B, 36 layers, 32
    # prompts x 256 random ids as one 8192-row chunk. Checked by properties
    # the CPU oracle cannot afford at this size:
    #  * KV indexing bit-exact: in layers 0, 17 and 35 every K and V slot is
    #    written exactly when some row's (pages[pos // 16], pos % 16) names it
    #    (the pool starts zeroed; a written slot holds 1024 nonzero-ish values);
    #  * the same prompts decoded token by token through the decode path (a
    #    second runner, 256 steps of 32 rows) give the same first token, except
    #    where the top-2 gap is below the oracle orders' end-to-end spread, and
    #    the same K/V (layer 0 to a bf16 ulp or 1e-3 of the slot's largest
    #    value, deeper layers within that spread's drift, doubled since both
    #    runs drift).
    cfg = dict(ferric_amd.QWEN3_8B)
    S, T = 32, 256
    limits = PagedLimits(context_tokens=T + 16, physical_page_count=S * 17 + 64, page_table_stride=17)
    pre = TpBatchRunner(cfg, limits, row_capacity=32, use_graphs=False, prefill_rows=S * T)
    dec = TpBatchRunner(cfg, limits, row_capacity=32, use_graphs=True)
    try:
        pre.synthesize_weights(61, 0.02)
        dec.synthesize_weights(61, 0.02)
        rng = np.random.default_rng(61)
        prompts = rng.integers(0, cfg["vocabulary"], (S, T))
        pool_p, pool_d = PagePool(limits, seed=62), PagePool(limits, seed=63)
        sp_ = [pool_p.admit(0) for _ in range(S)]
        batch = pool_p.prepare([(s, int(t)) for s, p in zip(sp_, prompts) for t in p])
        outs = [(i + 1) * T - 1 for i in range(S)]
        print("prefill 32 x 256", flush=True)
        first_pre = pre.execute_batch(batch, outs).choices
        logits_pre = pre.read_logits()
        pool_p.commit(batch)
        expected = {(int(r.writable_physical_page), int(r.position) % 16) for r in batch.rows}
        assert len(expected) == S * T
        for layer in (0, 17, 35):
            for which in (0, 1):
                for page in range(limits.physical_page_count):
                    got = pre.read_kv_page(layer, which, page).reshape(16, -1)
                    for slot in range(16):
                        written = bool(np.any(got[slot] != 0))
                        assert written == ((page, slot) in expected), (layer, which, page, slot)
        print("decode 256 steps", flush=True)
        sd = [pool_d.admit(0) for _ in range(S)]
        for t in range(T):
            b = pool_d.prepare([(s, int(p[t])) for s, p in zip(sd, prompts)])
            first_dec = dec.execute_batch(b, list(range(S))).choices
            pool_d.commit(b)
        logits_dec = dec.read_logits()
        spread_logit, spread_drift = _golden_spread()
        for i in range(S):
            if first_pre[i] != first_dec[i]:
                row = np.sort(logits_dec[i])
                gap = float(row[-1] - row[-2])
                assert gap < max(sp.NEAR_TIE, _golden_row_spread()), (i, first_pre[i], first_dec[i], gap)
                print(f"sequence {i}: near-tie between the paths (gap {gap:.2e})")
        e2e = float(np.max(np.abs(logits_pre - logits_dec)))
        print(f"prefill vs decode: logits max diff {e2e:.3e} (oracle orders' spread {spread_logit:.3e})")
        assert e2e <= 2 * (sp.SPREAD_FACTOR * spread_logit + sp.LOGIT_FLOOR)
        for layer, bound in ((0, None), (35, 2 * (sp.SPREAD_FACTOR * spread_drift + sp.DRIFT_FLOOR))):
            for which in (0, 1):
                for s_p, s_d in list(zip(sp_, sd))[:4]:
                    for pos in (0, 17, 255):
                        pg_p = int(pool_p.sequences[s_p].pages[pos // 16])
                        pg_d = int(pool_d.sequences[s_d].pages[pos // 16])
                        gp = pre.read_kv_page(layer, which, pg_p).reshape(16, -1)[pos % 16]
                        gd = dec.read_kv_page(layer, which, pg_d).reshape(16, -1)[pos % 16]
                        if bound is None:  # one rounding of two orders of the same sums
                            assert du.bf16_close(gp, gd, ulps=1), (layer, which, pos)
                        else:
                            assert du.bf16_rel_err(gp, gd) <= bound, (layer, which, pos)
    finally:
        pre.close()
        dec.close()


def test_speculative_config5_shapes_emit_the_target_greedy_stream():
    # The speculative workload's shapes: a Qwen3-8B target (36 layers,
    # untied head) verifying a Qwen3-0.6B draft (28 layers, tied head),
    # K = 4, 32 sequences, so every verify is a 160-row batch through the
    # prefill path. The emitted streams equal the target's own greedy decode
    # (a third runner with the target's weights, prompt prefill then decode
    # steps), except where a top-2 gap of that decode is below the oracle
    # orders' end-to-end spread at the 8B shape.
    from ferric_amd.speculative import SpeculativeDecoder

    S, P, K = 32, 16, 4
    limits = PagedLimits(context_tokens=128, physical_page_count=S * 8 + 64, page_table_stride=8)
    target = TpBatchRunner(ferric_amd.QWEN3_8B, limits, row_capacity=32, use_graphs=True, prefill_rows=S * P)
    draft = TpBatchRunner(ferric_amd.QWEN3_0_6B, limits, row_capacity=32, use_graphs=True, prefill_rows=S * P)
    plain = TpBatchRunner(ferric_amd.QWEN3_8B, limits, row_capacity=32, use_graphs=True, prefill_rows=S * P)
    try:
        target.synthesize_weights(8, 0.02)
        plain.synthesize_weights(8, 0.02)
        draft.synthesize_weights(9, 0.02)
        rng = np.random.default_rng(88)
        prompts = [list(rng.integers(0, ferric_amd.QWEN3_8B["vocabulary"], P)) for _ in range(S)]
        dec = SpeculativeDecoder(target, PagePool(limits, seed=1), draft, PagePool(limits, seed=2), k=K)
        dec.prefill(prompts)
        for rnd in range(3):
            st = dec.round()
            assert st.target_rows == S * (K + 1) and len(st.records) == S
            print(f"round {rnd}: accepted {sum(st.accepted)}", flush=True)
        pool = PagePool(limits, seed=3)
        sids = [pool.admit(0) for _ in range(S)]
        b = pool.prepare([(s, int(t)) for s, p in zip(sids, prompts) for t in p])
        ref = [[c] for c in plain.execute_batch(b, [(i + 1) * P - 1 for i in range(S)]).choices]
        pool.commit(b)
        gaps = [[float(np.diff(np.sort(row)[-2:])[0])] for row in plain.read_logits()]
        need = max(len(s.emitted) for s in dec.seqs)
        while len(ref[0]) < need:
            b = pool.prepare([(s, r[-1]) for s, r in zip(sids, ref)])
            out = plain.execute_batch(b, list(range(S))).choices
            pool.commit(b)
            lg = plain.read_logits()
            for i in range(S):
                ref[i].append(out[i])
                gaps[i].append(float(np.diff(np.sort(lg[i])[-2:])[0]))
        row_spread = _golden_row_spread()
        for j, s in enumerate(dec.seqs):
            for i, (got, want) in enumerate(zip(s.emitted, ref[j])):
                if got != want:
                    print(f"sequence {j}: differs at token {i} at gap {gaps[j][i]:.2e} (a typical row's oracle-order "
                          f"spread {row_spread:.2e}); compared up to there")
                    assert gaps[j][i] < max(sp.NEAR_TIE, row_spread), (j, i, got, want, gaps[j][i])
                    break
    finally:
        for r in (target, draft, plain):
            r.close()
