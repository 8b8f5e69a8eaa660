"""Writes hf_qwen3_composition.npz: a model-composition fixture for the oracle.

The reference's own Python oracle (tools/draft_reference.py:317-338) runs
Hugging Face `Qwen3ForCausalLM` in bf16 with SDPA attention and compares
Ferric against it to tolerance. This script does the same for a small
Qwen3 (0.6B layer geometry, 3 layers, tied 4096-token vocabulary) whose
weights come from the oracle's own deterministic generator (seed below), so
the test can rebuild them without storing them. transformers is the
installed library (5.x), not reference code.

Stored: the prompt, HF's per-layer residual stream (outputs of layers 0..L-2;
HF's last hidden state is post-norm) for every 3rd position, and HF's logits
at 256 fixed vocabulary ids for every position plus the full last-row logits.

Run from the repo root: python tests/golden/make_hf_composition.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import oracle as orc  # noqa: E402

SEED, SIGMA = 2027, 0.02
CFG = dict(layers=3, hidden=1024, query_heads=16, kv_heads=8, head_dim=128, intermediate=3072, vocabulary=4096,
           tied_embedding=1, rope_theta=1_000_000, rms_epsilon=1e-6)
T = 24
OUT = Path(__file__).resolve().parent / "hf_qwen3_composition.npz"

KINDS = {0: "lm_head.weight", 1: "model.embed_tokens.weight", 2: "model.norm.weight"}
LAYER_KINDS = {3: "input_layernorm.weight", 4: "post_attention_layernorm.weight", 5: "self_attn.q_norm.weight",
               6: "self_attn.k_norm.weight", 7: "self_attn.q_proj.weight", 8: "self_attn.k_proj.weight",
               9: "self_attn.v_proj.weight", 10: "self_attn.o_proj.weight", 11: "mlp.gate_proj.weight",
               12: "mlp.up_proj.weight", 13: "mlp.down_proj.weight"}


def shape_of(kind):
    c = CFG
    return {1: (c["vocabulary"], c["hidden"]), 2: (c["hidden"],), 3: (c["hidden"],), 4: (c["hidden"],), 5: (128,),
            6: (128,), 7: (c["query_heads"] * 128, c["hidden"]), 8: (c["kv_heads"] * 128, c["hidden"]),
            9: (c["kv_heads"] * 128, c["hidden"]), 10: (c["hidden"], c["query_heads"] * 128),
            11: (c["intermediate"], c["hidden"]), 12: (c["intermediate"], c["hidden"]),
            13: (c["hidden"], c["intermediate"])}[kind]


def bf16_tensor(bits):
    return torch.from_numpy(np.ascontiguousarray(bits, np.uint16).view(np.int16).copy()).view(torch.bfloat16)


def main():
    from transformers import Qwen3Config, Qwen3ForCausalLM

    model = orc.Model(CFG, 64)
    model.synthesize(SEED, SIGMA)
    state = {}
    for kind, name in KINDS.items():
        if kind == 0:
            continue  # tied
        shp = shape_of(kind)
        state[name] = bf16_tensor(model.weight(kind, 0, int(np.prod(shp))).reshape(shp))
    for layer in range(CFG["layers"]):
        for kind, name in LAYER_KINDS.items():
            shp = shape_of(kind)
            state[f"model.layers.{layer}.{name}"] = bf16_tensor(model.weight(kind, layer, int(np.prod(shp))).reshape(shp))
    config = Qwen3Config(vocab_size=CFG["vocabulary"], hidden_size=CFG["hidden"], intermediate_size=CFG["intermediate"],
                         num_hidden_layers=CFG["layers"], num_attention_heads=CFG["query_heads"],
                         num_key_value_heads=CFG["kv_heads"], head_dim=128, rms_norm_eps=CFG["rms_epsilon"],
                         rope_theta=float(CFG["rope_theta"]), max_position_embeddings=4096, tie_word_embeddings=True,
                         attention_bias=False, hidden_act="silu")
    config._attn_implementation = "sdpa"
    hf = Qwen3ForCausalLM(config).to(torch.bfloat16).eval()
    missing, unexpected = hf.load_state_dict(state, strict=False)
    assert not unexpected and all(m == "lm_head.weight" for m in missing), (missing, unexpected)
    hf.tie_weights()
    rng = np.random.default_rng(SEED)
    tokens = rng.integers(0, CFG["vocabulary"], T).astype(np.int64)
    with torch.no_grad():
        out = hf(torch.from_numpy(tokens)[None], output_hidden_states=True)
    logits = out.logits[0].float().numpy()
    hs = [h[0].float().numpy() for h in out.hidden_states]  # embeddings, layer 0 .. L-2 outputs, final norm
    rows = np.arange(0, T, 3)
    ids = np.sort(rng.choice(CFG["vocabulary"], 256, replace=False))
    np.savez_compressed(
        OUT, seed=np.int64(SEED), sigma=np.float32(SIGMA), tokens=tokens.astype(np.uint32), rows=rows,
        hidden=np.stack([hs[1 + l][rows] for l in range(CFG["layers"] - 1)]).astype(np.float32),
        ids=ids.astype(np.int64), logits_ids=logits[:, ids].astype(np.float32), logits_last=logits[-1].astype(np.float32),
        argmax=logits.argmax(axis=1).astype(np.int64),
        gap=np.sort(logits, axis=1)[:, -1] - np.sort(logits, axis=1)[:, -2],
        transformers_version=np.array(__import__("transformers").__version__))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
