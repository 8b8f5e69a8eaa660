"""fh_op_paged_attention_noalloc (no workspace argument; its partition records
live in the library's static device array) against fh_op_paged_attention on
the same inputs: bit-identical outputs and error word, on two calls in a row
(the second smaller), plus the size limit. Runs after the other tests."""

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from tests import devutil as du  # noqa: E402
import ferric_amd  # noqa: E402
from ferric_amd import _lib  # noqa: E402

LIB = ferric_amd.load()


def _case(r, rows, pages, stride, context, qh=32, kvh=8):
    positions = r.integers(0, context, rows).astype(np.uint32)
    positions[0] = context - 1  # the longest context of the launch
    kc = orc.f32_to_bf16(r.standard_normal(pages * 16 * kvh * 128).astype(np.float32))
    vc = orc.f32_to_bf16(r.standard_normal(pages * 16 * kvh * 128).astype(np.float32))
    q = orc.f32_to_bf16(r.standard_normal(rows * qh * 128).astype(np.float32))
    table = np.stack([r.permutation(pages)[:stride] for _ in range(rows)]).astype(np.uint32)
    return [du.to_dev(a) for a in (q, kc, vc, positions, table)]


def _both(dev, rows, qh, kvh, stride, pages, context, tiled):
    n = (int(LIB.fh_activation_rows(rows)) if tiled else rows) * qh * 128
    out_a, out_b = du.empty(n, np.uint16), du.empty(n, np.uint16)
    err_a, err_b = du.empty(1, np.uint32), du.empty(1, np.uint32)
    ws = torch.zeros(LIB.fh_attention_scratch_bytes(rows, qh, context) // 4, dtype=torch.float32, device="cuda")
    args = [du.ptr(t) for t in dev]
    _lib.check(LIB.fh_op_paged_attention(*args, du.ptr(out_a), tiled, du.ptr(ws), rows, qh, kvh, stride, pages, context,
                                         du.ptr(err_a), du.stream()))
    _lib.check(LIB.fh_op_paged_attention_noalloc(*args, du.ptr(out_b), tiled, rows, qh, kvh, stride, pages, context,
                                                 du.ptr(err_b), du.stream()))
    return (du.to_host(out_a, np.uint16), du.to_host(err_a, np.uint32)), (du.to_host(out_b, np.uint16),
                                                                           du.to_host(err_b, np.uint32))


def test_noalloc_attention_equals_the_workspace_entry_point():
    r = np.random.default_rng(123)
    # first call: 32 rows at contexts up to 8192 (16 partitions of 512 tokens
    # per row: 32 x 32 x 16 = the full 16384 records), tiled output
    big = dict(rows=32, qh=32, kvh=8, stride=520, pages=600, context=8192, tiled=1)
    dev = _case(r, big["rows"], big["pages"], big["stride"], big["context"])
    (a, ea), (b, eb) = _both(dev, **big)
    assert ea[0] == 0 and eb[0] == 0
    assert np.array_equal(a, b)
    # second call: fewer rows, shorter contexts, row-major output; the static
    # array still holds the first call's records, which must not leak in
    small = dict(rows=5, qh=16, kvh=8, stride=130, pages=200, context=2000, tiled=0)
    dev = _case(r, small["rows"], small["pages"], small["stride"], small["context"], qh=16)
    (a, ea), (b, eb) = _both(dev, **small)
    assert ea[0] == 0 and eb[0] == 0
    assert np.array_equal(a, b)


def test_noalloc_attention_rejects_launches_beyond_its_scratch():
    r = np.random.default_rng(5)
    dev = _case(r, 33, 600, 520, 8192)
    out, err = du.empty(33 * 32 * 128, np.uint16), du.empty(1, np.uint32)
    st = LIB.fh_op_paged_attention_noalloc(*[du.ptr(t) for t in dev], du.ptr(out), 0, 33, 32, 8, 520, 600, 8192,
                                           du.ptr(err), du.stream())
    assert st == 1  # 33 x 32 x 16 records > 16384
    assert b"16384" in LIB.fh_last_error(None)
