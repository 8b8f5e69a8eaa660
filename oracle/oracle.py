"""Test infrastructure only: ctypes view of the CPU oracle (liboracle.so).

Imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
to check the HIP library. The oracle restates the reference's serial scalar
semantics; see oracle.cpp for the per-function citations.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "liboracle.so"

_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_f32p = ctypes.POINTER(ctypes.c_float)
_c_u32 = ctypes.c_uint32
_c_u64 = ctypes.c_uint64


def build() -> Path:
    """Compiles liboracle.so from oracle.cpp with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIBRARY


def _ptr(a, ctype):
    if a is None:
        return None
    return a.ctypes.data_as(ctype)


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        L = ctypes.CDLL(str(LIBRARY))
        L.orc_bf16_from_f32.argtypes = [ctypes.c_float]
        L.orc_bf16_from_f32.restype = ctypes.c_uint16
        L.orc_square_sum.argtypes = [_u16p, _c_u32]
        L.orc_square_sum.restype = ctypes.c_float
        L.orc_norm_weight.argtypes = [ctypes.c_float, ctypes.c_uint16]
        L.orc_norm_weight.restype = _c_u32
        L.orc_rmsnorm.argtypes = [_u16p, _u16p, _u16p, _c_u32, _c_u32, ctypes.c_float, _c_u32, _u16p, _u16p]
        L.orc_rmsnorm.restype = ctypes.c_int
        L.orc_gemm.argtypes = [_u16p, _u16p, _u16p, _c_u32, _c_u32, _c_u32, _c_u32, _u16p, _f32p]
        L.orc_gemm.restype = None
        L.orc_gemm_a4.argtypes = [_u16p, _u16p, _u16p, _c_u32, _c_u32, _c_u32, _c_u32, _u16p]
        L.orc_embedding.argtypes = [_u32p, _u16p, _c_u32, _c_u32, _c_u32, _u16p]
        L.orc_embedding.restype = _c_u32
        L.orc_rope_table.argtypes = [_c_u32, _c_u32, _f32p, _f32p]
        L.orc_rope_pair.argtypes = [ctypes.c_uint16, ctypes.c_uint16, ctypes.c_float, ctypes.c_float, _u16p]
        L.orc_cache_index.argtypes = [_c_u32] * 5
        L.orc_cache_index.restype = _c_u64
        L.orc_attention_head.argtypes = [_u16p, _u16p, _u16p, _u32p, _c_u32, _c_u32, _c_u32, _c_u32, _c_u32, _u16p]
        L.orc_attention_head.restype = ctypes.c_int
        L.orc_swiglu.argtypes = [_u16p, _u16p, _c_u64, _u16p]
        L.orc_swiglu.restype = ctypes.c_int
        L.orc_residual.argtypes = [_f32p, _u16p, _c_u64, _u16p, ctypes.POINTER(ctypes.c_uint8)]
        L.orc_residual.restype = _c_u64
        L.orc_argmax_f32.argtypes = [_f32p, _c_u32, _f32p]
        L.orc_argmax_f32.restype = _c_u32
        L.orc_argmax_bf16.argtypes = [_u16p, _c_u32]
        L.orc_argmax_bf16.restype = _c_u32
        L.orc_token_assembly.argtypes = [_u32p, _u32p, _c_u32, _c_u32, _u32p]
        L.orc_verify_greedy.argtypes = [_u32p, _c_u32, _u32p, _c_u32, _u32p, _u32p, _u32p]
        L.orc_verify_greedy.restype = ctypes.c_int
        L.orc_compact_record.argtypes = [_u32p, _c_u64, _u32p, _c_u64, _c_u32, _c_u32, _c_u32, _c_u64,
                                         ctypes.POINTER(ctypes.c_uint8), _c_u32, _c_u32, _c_u32, _c_u32,
                                         ctypes.POINTER(ctypes.c_uint8), _u64p, _u32p]
        L.orc_compact_record.restype = ctypes.c_int
        L.orc_synth_fill.argtypes = [_u16p, _c_u64, _c_u64, ctypes.c_float]
        L.orc_splitmix64.argtypes = [_c_u64]
        L.orc_splitmix64.restype = _c_u64
        L.orc_synth_tensor_seed.argtypes = [_c_u64, _c_u32, _c_u32]
        L.orc_synth_tensor_seed.restype = _c_u64
        L.orc_synth_scale.argtypes = [ctypes.c_double]
        L.orc_synth_scale.restype = ctypes.c_float
        L.orc_threads.argtypes = []
        L.orc_threads.restype = ctypes.c_int
        L.orc_gemm_wave.argtypes = [_u16p, _u16p, _c_u32, _c_u32, _c_u32, _u16p, _f32p]
        L.orc_gemm_wave.restype = None
        L.orc_square_sum_wave.argtypes = [_u16p, _c_u32]
        L.orc_square_sum_wave.restype = ctypes.c_float
        L.orc_rmsnorm_wave.argtypes = [_u16p, _u16p, _c_u32, _c_u32, ctypes.c_float, _u16p]
        L.orc_rmsnorm_wave.restype = ctypes.c_int
        L.orc_rmsnorm_exact.argtypes = [_u16p, _u16p, _c_u32, _c_u32, ctypes.c_float, _u16p]
        L.orc_rmsnorm_exact.restype = ctypes.c_int
        L.orc_attention_head_wave.argtypes = [_u16p, _u16p, _u16p, _u32p, _c_u32, _c_u32, _c_u32, _c_u32, _c_u32,
                                              _u16p]
        L.orc_attention_head_wave.restype = ctypes.c_int
        L.orc_model_set_order.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.orc_model_set_order.restype = None
        L.orc_model_create.argtypes = [_c_u32] * 8 + [ctypes.c_float, _c_u32]
        L.orc_model_create.restype = ctypes.c_void_p
        L.orc_model_destroy.argtypes = [ctypes.c_void_p]
        L.orc_model_weight.argtypes = [ctypes.c_void_p, _c_u32, _c_u32, _c_u64]
        L.orc_model_weight.restype = _u16p
        L.orc_model_synthesize.argtypes = [ctypes.c_void_p, _c_u64, ctypes.c_float]
        L.orc_model_kv.argtypes = [ctypes.c_void_p, _c_u32, _c_u32]
        L.orc_model_kv.restype = _u16p
        L.orc_model_kv_fill.argtypes = [ctypes.c_void_p, _c_u64, ctypes.c_float, _u32p, _c_u32, _u32p, _u64p, _c_u32,
                                        _c_u32]
        L.orc_model_forward.argtypes = [ctypes.c_void_p, _u32p, _u32p, _u32p, _u32p, _c_u32, _c_u32, _u32p, _f32p,
                                        _u16p, _f32p, ctypes.POINTER(ctypes.c_double)]
        L.orc_model_forward.restype = ctypes.c_int
        L.orc_model_layer_isolated.argtypes = [ctypes.c_void_p, _c_u32, _u16p, _u32p, _u32p, _u32p, _c_u32, _c_u32,
                                               _u16p, _u16p, _u16p]
        L.orc_model_layer_isolated.restype = ctypes.c_int
        L.orc_model_head.argtypes = [ctypes.c_void_p, _u16p, _c_u32, _f32p, _u32p, _f32p]
        L.orc_model_head.restype = ctypes.c_int
        _lib = L
    return _lib


# ---- bf16 helpers (numpy) ------------------------------------------------------

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(values: np.ndarray) -> np.ndarray:
    """Vectorised copy of the reference's RNE narrowing (NaN quieted |0x40)."""
    b = np.asarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    nan = ((b & 0x7F800000) == 0x7F800000) & ((b & 0x007FFFFF) != 0)
    out = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) & 0xFFFF
    out = np.where(nan, ((b >> 16) | 0x40) & 0xFFFF, out)
    return out.astype(np.uint16)


def bf16_from_f32_scalar(v: float) -> int:
    return int(lib().orc_bf16_from_f32(v))


# ---- kernel-level oracles ------------------------------------------------------

def square_sum(x):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    return float(np.float32(lib().orc_square_sum(_ptr(x, _u16p), len(x))))


def square_sum_wave(x):
    """Sum of squares in the wave profile's order (lane l: x[l + 64 c]^2, then
    the 64-lane butterfly)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    return float(np.float32(lib().orc_square_sum_wave(_ptr(x, _u16p), len(x))))


def rmsnorm_wave(x, weight, rows, width, eps=1e-6):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    weight = np.ascontiguousarray(weight, dtype=np.uint16)
    out = np.zeros(rows * width, dtype=np.uint16)
    st = lib().orc_rmsnorm_wave(_ptr(x, _u16p), _ptr(weight, _u16p), rows, width, eps, _ptr(out, _u16p))
    return None if st else out


def rmsnorm_exact(x, weight, rows, width, eps=1e-6):
    """RMSNorm with the sum of squares taken exactly (float64, one rounding)."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    weight = np.ascontiguousarray(weight, dtype=np.uint16)
    out = np.zeros(rows * width, dtype=np.uint16)
    st = lib().orc_rmsnorm_exact(_ptr(x, _u16p), _ptr(weight, _u16p), rows, width, eps, _ptr(out, _u16p))
    return None if st else out


def gemm_wave(a, b, m, n, k, f32_out=False):
    """A W^T in the wave-GEMV order (k % 64 == 0)."""
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    if f32_out:
        out = np.zeros(m * n, np.float32)
        lib().orc_gemm_wave(_ptr(a, _u16p), _ptr(b, _u16p), m, n, k, None, _ptr(out, _f32p))
    else:
        out = np.zeros(m * n, np.uint16)
        lib().orc_gemm_wave(_ptr(a, _u16p), _ptr(b, _u16p), m, n, k, _ptr(out, _u16p), None)
    return out


def attention_head_wave(q, kc, vc, pages, physical_pages, position, kv_heads, kv_head):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    pages = np.ascontiguousarray(pages, dtype=np.uint32)
    out = np.zeros(128, np.uint16)
    st = lib().orc_attention_head_wave(_ptr(q, _u16p), _ptr(kc, _u16p), _ptr(vc, _u16p), _ptr(pages, _u32p),
                                       len(pages), physical_pages, position, kv_heads, kv_head, _ptr(out, _u16p))
    return None if st else out


def square_sum_bits(x) -> int:
    return int(np.array([square_sum(x)], np.float32).view(np.uint32)[0])


def norm_weight(normalized: float, weight_bits: int):
    r = lib().orc_norm_weight(normalized, weight_bits)
    return None if r == 0xFFFFFFFF else int(r)


def rmsnorm(x, weight, rows, width, eps=1e-6, residual=None):
    x = np.ascontiguousarray(x, dtype=np.uint16)
    weight = np.ascontiguousarray(weight, dtype=np.uint16)
    out = np.zeros(rows * width, dtype=np.uint16)
    fused = np.zeros(rows * width, dtype=np.uint16) if residual is not None else None
    res = np.ascontiguousarray(residual, dtype=np.uint16) if residual is not None else None
    st = lib().orc_rmsnorm(_ptr(x, _u16p), _ptr(res, _u16p), _ptr(weight, _u16p), rows, width, eps,
                           1 if residual is not None else 0, _ptr(fused, _u16p), _ptr(out, _u16p))
    if st != 0:
        return None
    return (fused, out) if residual is not None else out


def gemm(a, b, m, n, k, prior=None, f32_out=False):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    prior_arr = np.ascontiguousarray(prior, dtype=np.uint16) if prior is not None else None
    if f32_out:
        out = np.zeros(m * n, dtype=np.float32)
        lib().orc_gemm(_ptr(a, _u16p), _ptr(b, _u16p), None, m, n, k, 0, None, _ptr(out, _f32p))
        return out
    out = np.zeros(m * n, dtype=np.uint16)
    lib().orc_gemm(_ptr(a, _u16p), _ptr(b, _u16p), _ptr(prior_arr, _u16p), m, n, k, 1 if prior is not None else 0,
                   _ptr(out, _u16p), None)
    return out


def gemm_a4(a, b, m, n, k, prior=None):
    a = np.ascontiguousarray(a, dtype=np.uint16)
    b = np.ascontiguousarray(b, dtype=np.uint16)
    prior_arr = np.ascontiguousarray(prior, dtype=np.uint16) if prior is not None else np.zeros(m * n, np.uint16)
    out = np.zeros(m * n, dtype=np.uint16)
    lib().orc_gemm_a4(_ptr(a, _u16p), _ptr(b, _u16p), _ptr(prior_arr, _u16p), m, n, k, 1 if prior is not None else 0,
                      _ptr(out, _u16p))
    return out


def embedding(tokens, weight, hidden, vocab):
    tokens = np.ascontiguousarray(tokens, dtype=np.uint32)
    weight = np.ascontiguousarray(weight, dtype=np.uint16)
    out = np.zeros(len(tokens) * hidden, dtype=np.uint16)
    bad = lib().orc_embedding(_ptr(tokens, _u32p), _ptr(weight, _u16p), len(tokens), hidden, vocab, _ptr(out, _u16p))
    if bad:
        return ("invalid", int(bad) - 1, int(tokens[bad - 1]))
    return out


def rope_table(position, theta=1_000_000):
    c = np.zeros(64, np.float32)
    s = np.zeros(64, np.float32)
    lib().orc_rope_table(position, theta, _ptr(c, _f32p), _ptr(s, _f32p))
    return c, s


def rope_pair(first, second, cos, sin):
    out = np.zeros(2, np.uint16)
    lib().orc_rope_pair(first, second, cos, sin, _ptr(out, _u16p))
    return [int(out[0]), int(out[1])]


def cache_index(page, slot, kv_heads, kv_head, feature):
    return int(lib().orc_cache_index(page, slot, kv_heads, kv_head, feature))


def attention_head(q, k_cache, v_cache, pages, physical_pages, position, kv_heads, kv_head):
    q = np.ascontiguousarray(q, dtype=np.uint16)
    pages = np.ascontiguousarray(pages, dtype=np.uint32)
    out = np.zeros(128, np.uint16)
    st = lib().orc_attention_head(_ptr(q, _u16p), _ptr(k_cache, _u16p), _ptr(v_cache, _u16p), _ptr(pages, _u32p),
                                  len(pages), physical_pages, position, kv_heads, kv_head, _ptr(out, _u16p))
    return None if st else out


def swiglu(gate, up):
    gate = np.ascontiguousarray(gate, dtype=np.uint16)
    up = np.ascontiguousarray(up, dtype=np.uint16)
    out = np.zeros(len(gate), np.uint16)
    st = lib().orc_swiglu(_ptr(gate, _u16p), _ptr(up, _u16p), len(gate), _ptr(out, _u16p))
    return None if st else out


def residual(partial, res, with_rejections=False):
    """bf16((0 + partial) + res); with_rejections also returns the per-element
    flags of the reference's rejections (nonfinite operands, sums or rounding)."""
    partial = np.ascontiguousarray(partial, dtype=np.float32)
    res = np.ascontiguousarray(res, dtype=np.uint16)
    out = np.zeros(len(res), np.uint16)
    rej = np.zeros(len(res), np.uint8)
    lib().orc_residual(_ptr(partial, _f32p), _ptr(res, _u16p), len(res), _ptr(out, _u16p),
                       rej.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
    return (out, rej.astype(bool)) if with_rejections else out


def argmax_f32(logits):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    gap = np.zeros(1, np.float32)
    c = lib().orc_argmax_f32(_ptr(logits, _f32p), len(logits), _ptr(gap, _f32p))
    return (None if c == 0xFFFFFFFF else int(c)), float(gap[0])


def argmax_bf16(logits):
    logits = np.ascontiguousarray(logits, dtype=np.uint16)
    c = lib().orc_argmax_bf16(_ptr(logits, _u16p), len(logits))
    return None if c == 0xFFFFFFFF else int(c)


def token_assembly(anchors, draft, sequences, k):
    anchors = np.ascontiguousarray(anchors, dtype=np.uint32)
    draft = np.ascontiguousarray(draft, dtype=np.uint32)
    out = np.zeros(sequences * (k + 1), np.uint32)
    lib().orc_token_assembly(_ptr(anchors, _u32p), _ptr(draft, _u32p), sequences, k, _ptr(out, _u32p))
    return out


def verify_greedy(draft, target):
    draft = np.ascontiguousarray(draft, dtype=np.uint32)
    target = np.ascontiguousarray(target, dtype=np.uint32)
    acc = np.zeros(1, np.uint32)
    emitted = np.zeros(len(draft) + 1, np.uint32)
    cnt = np.zeros(1, np.uint32)
    st = lib().orc_verify_greedy(_ptr(draft, _u32p), len(draft), _ptr(target, _u32p), len(target), _ptr(acc, _u32p),
                                 _ptr(emitted, _u32p), _ptr(cnt, _u32p))
    if st:
        return st
    return int(acc[0]), [int(x) for x in emitted[: int(cnt[0])]]


def synth(count, tensor_seed, scale):
    out = np.zeros(count, np.uint16)
    lib().orc_synth_fill(_ptr(out, _u16p), count, tensor_seed, scale)
    return out


def synth_tensor_seed(seed, kind, layer):
    return int(lib().orc_synth_tensor_seed(seed, kind, layer))


def synth_scale(sigma):
    return float(lib().orc_synth_scale(sigma))


def threads() -> int:
    return int(lib().orc_threads())


# ---- whole model ------------------------------------------------------------

class Model:
    """CPU Qwen3 with the reference's serial semantics and a paged KV pool."""

    def __init__(self, desc: dict, pages: int):
        self.desc = dict(desc)
        d = self.desc
        self.h = lib().orc_model_create(d["layers"], d["hidden"], d["query_heads"], d["kv_heads"], d["intermediate"],
                                        d["vocabulary"], d["tied_embedding"], d["rope_theta"], d["rms_epsilon"], pages)
        self.pages = pages

    def close(self):
        if self.h:
            lib().orc_model_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def synthesize(self, seed: int, sigma: float):
        lib().orc_model_synthesize(self.h, seed, sigma)

    def weight(self, kind: int, layer: int, elements: int) -> np.ndarray:
        p = lib().orc_model_weight(self.h, kind, layer, elements)
        return np.ctypeslib.as_array(p, shape=(elements,))

    def kv(self, layer: int, which: int) -> np.ndarray:
        d = self.desc
        n = self.pages * 16 * d["kv_heads"] * 128
        return np.ctypeslib.as_array(lib().orc_model_kv(self.h, layer, which), shape=(n,))

    def kv_fill(self, seed, sigma, tables, stride, lengths, keys, context_stride):
        tables = np.ascontiguousarray(tables, np.uint32)
        lengths = np.ascontiguousarray(lengths, np.uint32)
        keys = np.ascontiguousarray(keys, np.uint64)
        lib().orc_model_kv_fill(self.h, seed, sigma, _ptr(tables, _u32p), stride, _ptr(lengths, _u32p),
                                _ptr(keys, _u64p), len(lengths), context_stride)

    def set_order(self, order: int):
        """Reduction order of later calls: 0 = the reference's serial (v1)
        sums, 1 = its wave-order profiles (v5 GEMV, v15 RMSNorm, v14 attention),
        2 = order 1 with a planted mistake (gate/up narrowed by truncation), for
        tests that show a drift bound catches a 1-ulp-biased rounding, 3 =
        order 1 with every RMSNorm's sum of squares taken exactly (the most
        accurate reassociation of the reference's sum)."""
        lib().orc_model_set_order(self.h, int(order))

    def layer_isolated(self, layer, hidden_in, positions, tables, page_counts, stride, order=None, kv=None):
        """One layer from a given input residual stream (on a scratch copy of
        the layer's KV pool, or of kv = (K pool, V pool) when given); order:
        reduction order for this call only."""
        if order is not None:
            self.set_order(order)
            try:
                return self.layer_isolated(layer, hidden_in, positions, tables, page_counts, stride, kv=kv)
            finally:
                self.set_order(0)
        kin = vin = None
        if kv is not None:
            n = self.pages * 16 * self.desc["kv_heads"] * 128
            kin, vin = (np.ascontiguousarray(a, np.uint16) for a in kv)
            assert kin.size == n and vin.size == n
        hidden_in = np.ascontiguousarray(hidden_in, np.uint16).reshape(-1)
        positions = np.ascontiguousarray(positions, np.uint32)
        tables = np.ascontiguousarray(tables, np.uint32)
        page_counts = np.ascontiguousarray(page_counts, np.uint32)
        out = np.zeros_like(hidden_in)
        st = lib().orc_model_layer_isolated(self.h, layer, _ptr(hidden_in, _u16p), _ptr(positions, _u32p),
                                            _ptr(tables, _u32p), _ptr(page_counts, _u32p), stride, len(positions),
                                            _ptr(kin, _u16p), _ptr(vin, _u16p), _ptr(out, _u16p))
        if st:
            raise RuntimeError("oracle layer trapped")
        return out.reshape(len(positions), -1)

    def head(self, hidden_in, order=None):
        """Final RMSNorm + FP32 head + argmax on a given residual stream."""
        if order is not None:
            self.set_order(order)
            try:
                return self.head(hidden_in)
            finally:
                self.set_order(0)
        hidden_in = np.ascontiguousarray(hidden_in, np.uint16)
        rows = hidden_in.size // self.desc["hidden"]
        logits = np.zeros(rows * self.desc["vocabulary"], np.float32)
        choices = np.zeros(rows, np.uint32)
        gaps = np.zeros(rows, np.float32)
        st = lib().orc_model_head(self.h, _ptr(hidden_in.reshape(-1), _u16p), rows, _ptr(logits, _f32p),
                                  _ptr(choices, _u32p), _ptr(gaps, _f32p))
        if st:
            raise RuntimeError("oracle head trapped")
        return {"logits": logits.reshape(rows, -1), "choices": choices, "gaps": gaps}

    def forward(self, tokens, positions, tables, page_counts, stride, want_logits=True, want_hidden=False,
                order=None):
        """One step (KV rows appended in place). order: reduction order for this
        call only (default: the model's current one)."""
        if order is not None:
            self.set_order(order)
            try:
                return self.forward(tokens, positions, tables, page_counts, stride, want_logits, want_hidden)
            finally:
                self.set_order(0)
        d = self.desc
        rows = len(tokens)
        tokens = np.ascontiguousarray(tokens, np.uint32)
        positions = np.ascontiguousarray(positions, np.uint32)
        tables = np.ascontiguousarray(tables, np.uint32)
        page_counts = np.ascontiguousarray(page_counts, np.uint32)
        choices = np.zeros(rows, np.uint32)
        gaps = np.zeros(rows, np.float32)
        logits = np.zeros(rows * d["vocabulary"], np.float32) if want_logits else None
        hidden = np.zeros(d["layers"] * rows * d["hidden"], np.uint16) if want_hidden else None
        seconds = np.zeros(2, np.float64)
        st = lib().orc_model_forward(self.h, _ptr(tokens, _u32p), _ptr(positions, _u32p), _ptr(tables, _u32p),
                                     _ptr(page_counts, _u32p), stride, rows, _ptr(choices, _u32p),
                                     _ptr(logits, _f32p), _ptr(hidden, _u16p), _ptr(gaps, _f32p),
                                     seconds.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
        if st:
            raise RuntimeError(f"oracle forward trapped (code {st})")
        out = {"choices": choices, "gaps": gaps, "seconds_layers": float(seconds[0]),
               "seconds_rest": float(seconds[1])}
        if want_logits:
            out["logits"] = logits.reshape(rows, d["vocabulary"])
        if want_hidden:
            out["hidden"] = hidden.reshape(d["layers"], rows, d["hidden"])
        return out


def compact_record(choices, draft, live, slot, generation, epoch, plan, sequences, sequence, active_tokens, k):
    """(record bytes or None, [("draft"|"choice", index) reads]) of one sequence,
    as the reference's compact_record_with_trace."""
    c = np.ascontiguousarray(np.asarray(choices, dtype=np.uint32).reshape(-1))
    d = np.ascontiguousarray(np.asarray(draft, dtype=np.uint32).reshape(-1))
    plan = np.frombuffer(bytes(plan), dtype=np.uint8).copy()
    assert plan.size == 32
    rec = np.zeros(120, np.uint8)
    reads = np.zeros(2 * k + 2, np.uint64)
    nr = np.zeros(1, np.uint32)
    u8 = ctypes.POINTER(ctypes.c_uint8)
    st = lib().orc_compact_record(_ptr(c, _u32p) if c.size else None, c.size, _ptr(d, _u32p) if d.size else None,
                                  d.size, live, slot, generation, epoch, plan.ctypes.data_as(u8), sequences, sequence,
                                  active_tokens, k, rec.ctypes.data_as(u8), _ptr(reads, _u64p), _ptr(nr, _u32p))
    trace = [("choice" if int(r) & 1 else "draft", int(r) >> 1) for r in reads[: int(nr[0])]]
    return (None if st else bytes(rec)), trace
