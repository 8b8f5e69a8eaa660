"""Device-memory plumbing for the GPU parity tests (torch owns the buffers;
libferric_hip.so is called through its C ABI on raw pointers)."""

from __future__ import annotations

import numpy as np
import torch

_TORCH = {np.uint16: torch.int16, np.uint32: torch.int32, np.float32: torch.float32, np.uint64: torch.int64}
_SIGNED = {np.uint16: np.int16, np.uint32: np.int32, np.float32: np.float32, np.uint64: np.int64}


def to_dev(a: np.ndarray) -> torch.Tensor:
    a = np.ascontiguousarray(a)
    t = torch.from_numpy(a.view(_SIGNED[a.dtype.type]).copy())
    return t.to("cuda")


def empty(n: int, dtype) -> torch.Tensor:
    return torch.zeros(n, dtype=_TORCH[np.dtype(dtype).type], device="cuda")


def to_host(t: torch.Tensor, dtype) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy().view(np.dtype(dtype))


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def stream():
    return torch.cuda.current_stream().cuda_stream


def sync():
    torch.cuda.synchronize()


def bf16_rel_err(got_bits: np.ndarray, ref_bits: np.ndarray) -> float:
    """max |got - ref| / max |ref| over bf16 arrays."""
    g = (got_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    r = (ref_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    denom = max(np.max(np.abs(r)), 1e-30)
    return float(np.max(np.abs(g - r)) / denom)


def bf16_close(got_bits: np.ndarray, ref_bits: np.ndarray, ulps: int = 1, floor_rel: float = 1e-3) -> bool:
    """Every element within `ulps` bf16 ulps of the reference, or within
    floor_rel * max|ref| absolutely (elements that cancel to near zero carry
    the absolute error of their inputs, not a relative one)."""
    g = (got_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    r = (ref_bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    mag = np.maximum(np.abs(r), 1e-38)
    ulp = 2.0 ** (np.floor(np.log2(mag)) - 7)
    ok = (np.abs(g - r) <= ulps * ulp) | (np.abs(g - r) <= floor_rel * np.max(np.abs(r)))
    return bool(np.all(ok))


def bf16_ulp_diff(got_bits: np.ndarray, ref_bits: np.ndarray) -> int:
    """Largest distance in bf16 ulps (sign-magnitude ordered)."""

    def ordered(b):
        b = b.astype(np.int64)
        return np.where(b & 0x8000, -(b & 0x7FFF), b & 0x7FFF)

    return int(np.max(np.abs(ordered(got_bits) - ordered(ref_bits)))) if got_bits.size else 0
