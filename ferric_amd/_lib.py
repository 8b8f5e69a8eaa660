"""ctypes binding of libferric_hip.so (the C ABI in include/ferric_hip.h).

There is no fallback: if the library is missing or cannot be loaded, import
fails with the reason. Build it with `python ferric_amd/build.py` (or
__graft_entry__.build()).
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIBRARY = Path(__file__).resolve().parent / "libferric_hip.so"

FH_OK = 0
STATUS_NAMES = {
    0: "FH_OK",
    1: "FH_ERR_INVALID_ARGUMENT",
    2: "FH_ERR_INVALID_BATCH",
    3: "FH_ERR_INVALID_ROW",
    4: "FH_ERR_SHARED_PAGE",
    5: "FH_ERR_OUTPUT_ROWS",
    6: "FH_ERR_NONFINITE",
    7: "FH_ERR_DEVICE",
    8: "FH_ERR_POISONED",
    9: "FH_ERR_OUT_OF_MEMORY",
    10: "FH_ERR_STATE",
}

# Tensor kinds (ferric_hip.h, crates/ferric-spec/src/qwen3.rs:20-35 order).
LANGUAGE_MODEL_HEAD = 0
TOKEN_EMBEDDING = 1
FINAL_NORM = 2
INPUT_LAYER_NORM = 3
POST_ATTENTION_LAYER_NORM = 4
QUERY_NORM = 5
KEY_NORM = 6
QUERY_PROJECTION = 7
KEY_PROJECTION = 8
VALUE_PROJECTION = 9
OUTPUT_PROJECTION = 10
GATE_PROJECTION = 11
UP_PROJECTION = 12
DOWN_PROJECTION = 13

EPI_BF16, EPI_RESIDUAL, EPI_SWIGLU, EPI_F32, EPI_PARTIAL = 0, 1, 2, 3, 4

KERNEL_CLASSES = ["embedding", "rmsnorm", "qkv_gemm", "qknorm_rope_kv", "attention", "attention_merge", "o_gemm",
                  "gate_up_gemm", "down_gemm", "head_gemm", "argmax"]


class ModelDesc(ctypes.Structure):
    _fields_ = [
        ("layers", ctypes.c_uint32),
        ("hidden", ctypes.c_uint32),
        ("query_heads", ctypes.c_uint32),
        ("kv_heads", ctypes.c_uint32),
        ("head_dim", ctypes.c_uint32),
        ("intermediate", ctypes.c_uint32),
        ("vocabulary", ctypes.c_uint32),
        ("tied_embedding", ctypes.c_uint32),
        ("rope_theta", ctypes.c_uint32),
        ("rms_epsilon", ctypes.c_float),
    ]


class CtxOptions(ctypes.Structure):
    _fields_ = [
        ("row_capacity", ctypes.c_uint32),
        ("physical_pages", ctypes.c_uint32),
        ("page_table_stride", ctypes.c_uint32),
        ("context_tokens", ctypes.c_uint32),
        ("use_graphs", ctypes.c_uint32),
        ("capture_hidden", ctypes.c_uint32),
        ("device", ctypes.c_int32),
        ("prefill_rows", ctypes.c_uint32),
    ]


class Row(ctypes.Structure):
    _fields_ = [
        ("sequence", ctypes.c_uint64),
        ("token", ctypes.c_uint32),
        ("position", ctypes.c_uint32),
        ("pages", ctypes.POINTER(ctypes.c_uint32)),
        ("page_count", ctypes.c_uint32),
        ("writable_page", ctypes.c_uint32),
    ]


_u16p = ctypes.POINTER(ctypes.c_uint16)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_u64p = ctypes.POINTER(ctypes.c_uint64)
_f32p = ctypes.POINTER(ctypes.c_float)
_vp = ctypes.c_void_p
_u32 = ctypes.c_uint32
_u64 = ctypes.c_uint64
_st = ctypes.c_int

# (name, restype, argtypes) for every symbol declared in include/ferric_hip.h.
SIGNATURES = [
    ("fh_create", _st, [ctypes.POINTER(ModelDesc), ctypes.POINTER(CtxOptions), ctypes.POINTER(_vp)]),
    ("fh_destroy", None, [_vp]),
    ("fh_last_error", ctypes.c_char_p, [_vp]),
    ("fh_upload_weight", _st, [_vp, _u32, _u32, _u16p, _u64]),
    ("fh_synthesize_weights", _st, [_vp, _u64, ctypes.c_float]),
    ("fh_download_weight", _st, [_vp, _u32, _u32, _u16p, _u64]),
    ("fh_kv_fill_synthetic", _st, [_vp, _u64, ctypes.c_float, ctypes.POINTER(Row), _u64p, _u32, _u32]),
    ("fh_read_kv_page", _st, [_vp, _u32, _u32, _u32, _u16p, _u64]),
    ("fh_write_kv_page", _st, [_vp, _u32, _u32, _u32, _u16p, _u64]),
    ("fh_read_kv_cache", _st, [_vp, _u32, _u32, _u16p, _u64]),
    ("fh_execute_batch", _st, [_vp, _u64, ctypes.POINTER(Row), _u32, _u32p, _u32, _u32p]),
    ("fh_read_logits", _st, [_vp, _f32p, _u64]),
    ("fh_read_hidden", _st, [_vp, _u32, _u16p, _u64]),
    ("fh_row_capacity", _u32, [_vp]),
    ("fh_dispatch_count", _u64, [_vp]),
    ("fh_expected_dispatch_count", _st, [_vp, _u64, ctypes.POINTER(Row), _u32, _u32p, _u32, _u64p]),
    ("fh_last_step_ms", ctypes.c_float, [_vp]),
    ("fh_set_profiling", _st, [_vp, _u32]),
    ("fh_kernel_class_ms", _st, [_vp, _u32, _f32p, _u32p]),
    ("fh_time_attention", _st, [_vp, _u32, _f32p]),
    ("fh_op_tile_weight", _st, [_vp, _vp, _u32, _u32, _vp]),
    ("fh_op_tile_gate_up", _st, [_vp, _vp, _vp, _u32, _u32, _vp]),
    ("fh_op_untile_weight", _st, [_vp, _vp, _u32, _u32, _vp]),
    ("fh_op_embedding", _st, [_vp, _vp, _vp, _u32, _u32, _u32, _vp, _vp]),
    ("fh_op_rmsnorm", _st, [_vp, _vp, _vp, _u32, _u32, ctypes.c_float, _vp, _vp]),
    ("fh_op_gemm", _st, [_vp, _vp, _u32, _u32, _u32, _u32, _u32, _vp, _vp, _u32, _vp, _vp]),
    ("fh_gemm_default_splits", _u32, [_u32, _u32]),
    ("fh_activation_rows", _u32, [_u32]),
    ("fh_partial_slab_rows", _u32, [_u32]),
    ("fh_op_tile_activation", _st, [_vp, _vp, _u32, _u32, _vp]),
    ("fh_op_untile_activation", _st, [_vp, _vp, _u32, _u32, _vp]),
    ("fh_op_residual_rmsnorm", _st, [_vp, _vp, _u32, _vp, _vp, _u32, _u32, _u32, ctypes.c_float, _vp, _vp]),
    ("fh_op_gemm_rmsnorm", _st,
     [_vp, _vp, _vp, _u32, _vp, ctypes.c_float, _vp, _u32, _u32, _u32, _u32, _vp, _u32, _vp, _vp]),
    ("fh_gemm_rmsnorm_supported", _u32, [_u32, _u32, _u32, _u32, _u32]),
    ("fh_op_qknorm_rope_kv", _st, [_vp, _u32] + [_vp] * 9 + [_u32] * 6 + [ctypes.c_float, _vp, _vp]),
    ("fh_attention_scratch_bytes", _u64, [_u32, _u32, _u32]),
    ("fh_op_paged_attention", _st, [_vp] * 6 + [_u32, _vp] + [_u32] * 6 + [_vp, _vp]),
    ("fh_op_qknorm_paged_attention", _st,
     [_vp, _u32] + [_vp] * 9 + [_u32, _vp] + [_u32] * 6 + [ctypes.c_float, _vp, _vp]),
    ("fh_op_paged_attention_noalloc", _st, [_vp] * 6 + [_u32] * 7 + [_vp, _vp]),
    ("fh_op_swiglu", _st, [_vp, _vp, _vp, _u64, _vp, _vp]),
    ("fh_argmax_scratch_bytes", _u64, [_u32]),
    ("fh_op_argmax", _st, [_vp, _u32, _u32, _vp, _vp, _vp, _vp]),
    ("fh_op_synth_fill", _st, [_vp, _u64, _u64, ctypes.c_float, _vp]),
    ("fh_speculative_token_assembly", _st, [_u32p, _u32p, _u32, _u32, _u32p]),
    ("fh_verify_greedy_round", _st, [_u32p, _u32, _u32p, _u32, _u32p, _u32p, _u32p]),
    ("fh_verify_greedy_batch", _st, [_u32p, _u32p, _u32, _u32, _u32p, _u32p]),
    ("fh_compact_completion", _st, [_u32p, _u32p, _u32p, _u32p, _u32p, _u64p, ctypes.POINTER(ctypes.c_uint8), _u32,
                                    _u32, _u32, ctypes.POINTER(ctypes.c_uint8)]),
]

_lib = None


def load() -> ctypes.CDLL:
    """Loads libferric_hip.so and binds every C ABI symbol; raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY.exists():
        raise ImportError(f"{LIBRARY} is not built; run `python ferric_amd/build.py` (hipcc, gfx950)")
    # PyTorch ships its own libamdhip64 under the same soname. Loading torch
    # first makes this library bind to that copy; the other order maps two
    # HIP runtimes into the process, and the second one to touch the device
    # reports that there is none. Without torch the system runtime is used.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(str(LIBRARY))
    for name, restype, argtypes in SIGNATURES:
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


class FerricError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {message}")
        self.status = status
        self.message = message


def check(status: int, ctx=None, what: str = ""):
    if status != FH_OK:
        lib = load()
        msg = lib.fh_last_error(ctx)
        raise FerricError(status, (msg.decode() if msg else "") or what)
