"""Real-checkpoint path on the GPU: oracle-synthesized weights written as
two Hugging Face-named safetensors shards, admitted with SHA-256 pins and
uploaded by ferric_amd.checkpoint, read back bit-exactly, then one decode
step checked against the CPU oracle holding the same weights."""

import numpy as np
import pytest

import ferric_amd
from ferric_amd import PagedLimits, PagePool, TpBatchRunner
from ferric_amd.checkpoint import expected_shape, file_sha256, load_safetensors, required_tensors
from oracle import oracle as orc

from test_checkpoint import tensor_name, write_two_shards

pytestmark = pytest.mark.gpu


def test_safetensors_checkpoint_decode_matches_oracle(tmp_path):
    # 0.6B layer geometry, 2 layers, untied 4096-token vocabulary (an lm_head tensor).
    cfg = dict(ferric_amd.QWEN3_0_6B, layers=2, vocabulary=4096, tied_embedding=0)
    limits = PagedLimits(context_tokens=512, physical_page_count=64, page_table_stride=32)
    model = orc.Model(cfg, limits.physical_page_count)
    runner = TpBatchRunner(cfg, limits, row_capacity=8, use_graphs=False)
    try:
        model.synthesize(11, 0.02)
        tensors = {}
        for kind, layer in sorted(required_tensors(cfg)):
            shape = expected_shape(cfg, kind)
            tensors[tensor_name(kind, layer)] = np.array(model.weight(kind, layer, int(np.prod(shape)))).reshape(shape)
        paths = write_two_shards(tmp_path, tensors)
        info = load_safetensors(runner, paths, sha256={p.split("/")[-1]: file_sha256(p) for p in paths})
        assert info["tensors"] == 3 + 11 * cfg["layers"]
        for kind, layer in sorted(required_tensors(cfg)):
            want = tensors[tensor_name(kind, layer)].reshape(-1)
            assert np.array_equal(runner.download_weight(kind, layer, want.size), want), (kind, layer)

        pool = PagePool(limits, seed=3)
        seqs = [pool.admit(0) for _ in range(2)]
        rows = [(seqs[0], 11), (seqs[0], 12), (seqs[0], 13), (seqs[1], 4095)]
        batch = pool.prepare(rows)
        out = runner.execute_batch(batch, list(range(len(rows))))
        logits = runner.read_logits()
        stride = limits.page_table_stride
        tables = np.full((len(rows), stride), 0xFFFFFFFF, np.uint32)
        counts = np.zeros(len(rows), np.uint32)
        for i, r in enumerate(batch.rows):
            tables[i, : len(r.physical_pages)] = r.physical_pages
            counts[i] = len(r.physical_pages)
        ref = model.forward([r.token for r in batch.rows], [r.position for r in batch.rows], tables, counts, stride)
        err = float(np.max(np.abs(logits - ref["logits"])))
        print(f"checkpoint decode: max |logit - oracle| = {err:.3g}")
        assert err <= 5e-2
        for i, c in enumerate(out.choices):
            assert c == ref["choices"][i] or ref["gaps"][i] < 1e-3
    finally:
        runner.close()
        model.close()
