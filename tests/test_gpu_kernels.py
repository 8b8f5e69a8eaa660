"""Kernel-level parity: each fh_op_* root on the GPU against the CPU oracle.

Bars (stated per test): bit-exact for integer/byte work and wherever the
GPU keeps the reference's operation order (synthetic fill, tiling, embedding,
QK-norm + RoPE + KV slot, argmax); within bf16/fp32-accumulate tolerance where
the GPU reassociates FP32 sums (RMSNorm width 1024/4096, projections,
attention).
"""

import numpy as np
import pytest

from oracle import oracle as orc

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
from tests import devutil as du  # noqa: E402
import ferric_amd  # noqa: E402
from ferric_amd import _lib  # noqa: E402

LIB = ferric_amd.load()


def rng(seed):
    return np.random.default_rng(seed)


def rand_bf16(r, n, scale=1.0):
    return orc.f32_to_bf16(r.standard_normal(n).astype(np.float32) * np.float32(scale))


def tile_host(w, n, k):
    """Numpy statement of the tiled layout: lane = row%16 + 16*((col%32)//8)."""
    w = w.reshape(n, k)
    t = w.reshape(n // 16, 16, k // 32, 4, 8)  # nb, r, kb, g, e
    t = t.transpose(0, 2, 3, 1, 4)  # nb, kb, g, r, e  -> lane = g*16 + r
    return np.ascontiguousarray(t).reshape(-1)


def test_synth_fill_matches_oracle_bits():
    for count, seed in [(1, 3), (4099, 11), (1 << 16, 12345)]:
        ts = orc.synth_tensor_seed(seed, 7, 2)
        scale = orc.synth_scale(0.02)
        d = du.empty(count, np.uint16)
        _lib.check(LIB.fh_op_synth_fill(du.ptr(d), count, ts, scale, du.stream()))
        got = du.to_host(d, np.uint16)
        assert np.array_equal(got, orc.synth(count, ts, scale)), (count, seed)


def test_tile_untile_round_trip_and_layout():
    r = rng(1)
    for n, k in [(16, 32), (48, 96), (4096, 64)]:
        w = r.integers(0, 65536, n * k, dtype=np.uint64).astype(np.uint16)
        dw = du.to_dev(w)
        dt = du.empty(n * k, np.uint16)
        _lib.check(LIB.fh_op_tile_weight(du.ptr(dw), du.ptr(dt), n, k, du.stream()))
        tiled = du.to_host(dt, np.uint16)
        assert np.array_equal(tiled, tile_host(w, n, k))
        back = du.empty(n * k, np.uint16)
        _lib.check(LIB.fh_op_untile_weight(du.ptr(dt), du.ptr(back), n, k, du.stream()))
        assert np.array_equal(du.to_host(back, np.uint16), w)


def test_embedding_bit_copy_from_tiled_table():
    r = rng(2)
    vocab, hidden = 160, 256
    w = r.integers(0, 65536, vocab * hidden, dtype=np.uint64).astype(np.uint16)
    w[:8] = [0x0000, 0x8000, 0x7F80, 0x7FC1, 0x3F80, 0xBF80, 0x0001, 0x7F7F]  # specials survive a bit copy
    toks = np.array([0, 159, 17, 17, 64, 3], np.uint32)
    dw = du.to_dev(w)
    dt = du.empty(vocab * hidden, np.uint16)
    _lib.check(LIB.fh_op_tile_weight(du.ptr(dw), du.ptr(dt), vocab, hidden, du.stream()))
    out = du.empty(len(toks) * hidden, np.uint16)
    err = du.empty(1, np.uint32)
    dtok = du.to_dev(toks)
    _lib.check(LIB.fh_op_embedding(du.ptr(dtok), du.ptr(dt), du.ptr(out), len(toks), hidden, vocab, du.ptr(err),
                                   du.stream()))
    assert du.to_host(err, np.uint32)[0] == 0
    assert np.array_equal(du.to_host(out, np.uint16), orc.embedding(toks, w, hidden, vocab))
    bad = du.to_dev(np.array([5, vocab], np.uint32))  # kept alive by the name
    _lib.check(LIB.fh_op_embedding(du.ptr(bad), du.ptr(dt), du.ptr(out), 2, hidden, vocab, du.ptr(err), du.stream()))
    assert du.to_host(err, np.uint32)[0] != 0  # the reference traps on token >= vocab


@pytest.mark.parametrize("width", [1024, 4096])
@pytest.mark.parametrize("rows", [1, 5, 32])
def test_rmsnorm_within_tolerance(width, rows):
    r = rng(width + rows)
    x = rand_bf16(r, rows * width, 3.0)
    w = rand_bf16(r, width, 1.0)
    dx, dw_, dy, err = du.to_dev(x), du.to_dev(w), du.empty(rows * width, np.uint16), du.empty(1, np.uint32)
    _lib.check(LIB.fh_op_rmsnorm(du.ptr(dx), du.ptr(dw_), du.ptr(dy), rows, width, 1e-6, du.ptr(err), du.stream()))
    got = du.to_host(dy, np.uint16)
    ref = orc.rmsnorm(x, w, rows, width)
    assert du.to_host(err, np.uint32)[0] == 0
    # Reassociated sum of squares: the inverse RMS may differ in its last f32
    # bits, which can flip the first bf16 rounding (x * inv) by one ulp; the
    # second rounding (* weight) can carry that to two output ulps.
    assert du.bf16_ulp_diff(got, ref) <= 2
    assert du.bf16_rel_err(got, ref) <= 2e-2
    assert np.mean(got == ref) > 0.99


def test_rmsnorm_known_answers():
    for width in [1024, 4096]:
        ones = np.full(width, 0x3F80, np.uint16)
        zeros = np.zeros(2 * width, np.uint16)
        for x, expect in [(ones, ones), (zeros, zeros)]:
            rows = len(x) // width
            dx, dw_, dy, err = du.to_dev(x), du.to_dev(ones), du.empty(len(x), np.uint16), du.empty(1, np.uint32)
            _lib.check(LIB.fh_op_rmsnorm(du.ptr(dx), du.ptr(dw_), du.ptr(dy), rows, width, 1e-6, du.ptr(err),
                                         du.stream()))
            assert np.array_equal(du.to_host(dy, np.uint16), expect)
        bad = ones.copy()
        bad[17] = 0x7F80
        dx, dy, err = du.to_dev(bad), du.empty(width, np.uint16), du.empty(1, np.uint32)
        dw_ = du.to_dev(ones)
        _lib.check(LIB.fh_op_rmsnorm(du.ptr(dx), du.ptr(dw_), du.ptr(dy), 1, width, 1e-6, du.ptr(err), du.stream()))
        assert du.to_host(err, np.uint32)[0] != 0


def tiled_rows(m):
    """Rows of a tiled activation buffer: 32 up to 32 rows, else m rounded up to 256."""
    return 32 if m <= 32 else -(-m // 256) * 256


def act_tile_host(x, m, k):
    """Numpy statement of the activation tile order for x[m][k]:
    tile (kb, mt) = rows 16 mt.., cols 32 kb..; lane = row % 16 + 16 * ((col % 32) // 8)."""
    rows = tiled_rows(m)
    full = np.zeros((rows, k), np.uint16)
    full[:m] = x.reshape(m, k)
    t = full.reshape(rows // 16, 16, k // 32, 4, 8)  # mt, r, kb, g, e
    t = t.transpose(2, 0, 3, 1, 4)  # kb, mt, g, r, e -> lane = g*16 + r
    return np.ascontiguousarray(t).reshape(-1)


def to_tiled_act(x, m, k):
    dx = du.to_dev(x)
    assert LIB.fh_activation_rows(m) == tiled_rows(m)
    dxt = du.empty(tiled_rows(m) * k, np.uint16)
    _lib.check(LIB.fh_op_tile_activation(du.ptr(dx), du.ptr(dxt), m, k, du.stream()))
    return dxt


def test_activation_tile_order_round_trip():
    r = rng(8)
    for m, k in [(1, 32), (7, 64), (16, 1024), (17, 96), (32, 4096), (33, 64), (130, 96), (300, 32)]:
        x = r.integers(0, 65536, m * k, dtype=np.uint64).astype(np.uint16)
        dxt = to_tiled_act(x, m, k)  # rows >= m stay zero (never written)
        assert np.array_equal(du.to_host(dxt, np.uint16), act_tile_host(x, m, k)), (m, k)
        back = du.empty(m * k, np.uint16)
        _lib.check(LIB.fh_op_untile_activation(du.ptr(dxt), du.ptr(back), m, k, du.stream()))
        assert np.array_equal(du.to_host(back, np.uint16), x)


def _gemm_case(m, n, k, epi, seed, splits=1, poison_row=None):
    """One fh_op_gemm launch against the oracle. poison_row: a NaN is planted
    in that activation row (the SwiGLU epilogue must then raise the error word;
    returns the error word instead of the outputs)."""
    r = rng(seed)
    x = rand_bf16(r, m * k, 1.0)
    if poison_row is not None:
        x[poison_row * k + 5] = 0x7FC0
    w = rand_bf16(r, n * k, 0.02)
    dxt = to_tiled_act(x, m, k)
    dw_ = du.to_dev(w)
    dt = du.empty(n * k, np.uint16)
    err = du.empty(1, np.uint32)
    if epi == _lib.EPI_SWIGLU:
        i = n // 2
        gate, up = w[: i * k], w[i * k:]
        dg, du_ = du.to_dev(gate), du.to_dev(up)
        _lib.check(LIB.fh_op_tile_gate_up(du.ptr(dg), du.ptr(du_), du.ptr(dt), i, k, du.stream()))
        out_t = du.empty(tiled_rows(m) * i, np.uint16)  # activation tile order (the down projection's input)
        _lib.check(LIB.fh_op_gemm(du.ptr(dxt), du.ptr(dt), m, n, k, epi, 1, None, du.ptr(out_t), i, du.ptr(err),
                                  du.stream()))
        if poison_row is not None:
            return int(du.to_host(err, np.uint32)[0])
        assert du.to_host(err, np.uint32)[0] == 0
        out = du.empty(m * i, np.uint16)
        _lib.check(LIB.fh_op_untile_activation(du.ptr(out_t), du.ptr(out), m, i, du.stream()))
        got = du.to_host(out, np.uint16)
        g = orc.gemm(x, gate, m, i, k)
        u = orc.gemm(x, up, m, i, k)
        return got, orc.swiglu(g, u)
    _lib.check(LIB.fh_op_tile_weight(du.ptr(dw_), du.ptr(dt), n, k, du.stream()))
    if epi == _lib.EPI_PARTIAL:
        slab_rows = int(LIB.fh_partial_slab_rows(m))
        out = du.to_dev(np.full(splits * slab_rows * n, np.nan, np.float32))  # every slab row < m is written
        _lib.check(LIB.fh_op_gemm(du.ptr(dxt), du.ptr(dt), m, n, k, epi, splits, None, du.ptr(out), n, None, du.stream()))
        slabs = du.to_host(out, np.float32).reshape(splits, slab_rows, n)[:, :m]
        total = slabs[0].copy()
        for sp in range(1, splits):
            total = (total + slabs[sp]).astype(np.float32)
        return total.reshape(-1), orc.gemm(x, w, m, n, k, f32_out=True)
    if epi == _lib.EPI_F32:
        out = du.empty(m * n, np.float32)
        _lib.check(LIB.fh_op_gemm(du.ptr(dxt), du.ptr(dt), m, n, k, epi, 1, None, du.ptr(out), n, None, du.stream()))
        return du.to_host(out, np.float32), orc.gemm(x, w, m, n, k, f32_out=True)
    if epi == _lib.EPI_RESIDUAL:
        res = rand_bf16(r, m * n, 1.0)
        out = du.to_dev(res)  # in place
        _lib.check(LIB.fh_op_gemm(du.ptr(dxt), du.ptr(dt), m, n, k, epi, 1, du.ptr(out), du.ptr(out), n, None, du.stream()))
        part = orc.gemm(x, w, m, n, k, f32_out=True)
        return du.to_host(out, np.uint16), orc.residual(part, res)
    out = du.empty(m * n, np.uint16)
    _lib.check(LIB.fh_op_gemm(du.ptr(dxt), du.ptr(dt), m, n, k, epi, 1, None, du.ptr(out), n, None, du.stream()))
    return du.to_host(out, np.uint16), orc.gemm(x, w, m, n, k)


F32_BOUND = 1.6e-4  # FP32 reassociation of <= 12288 products of |x| ~ 1, |w| ~ 0.02


@pytest.mark.parametrize("m", [1, 7, 16, 17, 32])
@pytest.mark.parametrize("n,k", [(64, 64), (256, 1024), (1024, 4096), (512, 12288), (48, 128)])
def test_gemm_bf16_and_f32_epilogues(m, n, k):
    got, ref = _gemm_case(m, n, k, _lib.EPI_F32, m * 7 + n)
    assert np.max(np.abs(got - ref)) <= F32_BOUND
    got, ref = _gemm_case(m, n, k, _lib.EPI_BF16, m * 7 + n + 1)
    assert du.bf16_close(got, ref, ulps=1)
    assert np.mean(got == ref) > 0.99


@pytest.mark.parametrize("m,n,k,splits", [(32, 6144, 4096, 6), (32, 4096, 12288, 8), (5, 1024, 1024, 2),
                                          (17, 256, 4096, 3), (32, 64, 128, 4),
                                          (32, 6144, 4096, 2), (9, 6144, 1024, 2)])  # 3 n-tiles per wave
def test_gemm_split_k_partials(m, n, k, splits):
    got, ref = _gemm_case(m, n, k, _lib.EPI_PARTIAL, 31 * m + splits, splits=splits)
    assert np.max(np.abs(got - ref)) <= F32_BOUND


# 33-256 rows: the panel kernel, one instance per even m-tile count (4 .. 16
# tiles), slabs of 256 rows; (48, 128, 256, 5): 8 k-blocks in splits of 2, so
# the fifth split is past the end of k and must write zeros. (42, 4096,
# 12288, 8) is the 8B down projection at 42 rows, where a wait counting both
# load kinds together let MFMAs read weight registers and activation tiles
# before they arrived (tens of thousands of wrong outputs per launch).
@pytest.mark.parametrize("m,n,k,splits", [(33, 128, 1024, 2), (80, 384, 2048, 3), (100, 6144, 1024, 5),
                                          (160, 1024, 4096, 8), (176, 256, 4096, 4), (200, 256, 2048, 3),
                                          (256, 128, 1024, 4), (48, 128, 256, 5), (130, 512, 512, 1),
                                          (42, 4096, 12288, 8)])
def test_gemm_wide_split_k_partials(m, n, k, splits):
    got, ref = _gemm_case(m, n, k, _lib.EPI_PARTIAL, 37 * m + splits + n, splits=splits)
    assert np.max(np.abs(got - ref)) <= F32_BOUND


@pytest.mark.parametrize("m", [3, 32])
def test_gemm_residual_and_swiglu_epilogues(m):
    got, ref = _gemm_case(m, 512, 4096, _lib.EPI_RESIDUAL, 99 + m)
    assert du.bf16_close(got, ref, ulps=1)
    assert np.mean(got == ref) > 0.99
    for n in (1024, 6144):
        got, ref = _gemm_case(m, n, 1024, _lib.EPI_SWIGLU, 199 + m + n)
        assert ref is not None
        # gate and up are each one bf16 rounding of a reassociated sum (<= 1 ulp),
        # and SwiGLU multiplies them: <= 2 ulps of the product, plus exp's last ulp.
        assert du.bf16_close(got, ref, ulps=3)
        assert np.mean(got == ref) > 0.97


@pytest.mark.parametrize("m", [3, 40, 300])  # decode kernel, 32-row chunks, 256 x 256 blocks
def test_gemm_swiglu_epilogue_reports_nonfinite(m):
    # A NaN in one activation row makes that row's gate and up NaN: the fused
    # SwiGLU epilogue (decode and prefill kernels) raises the error word where
    # qwen3_swiglu_bf16_f32_v1 traps (swiglu.rs:62-101).
    assert _gemm_case(m, 256, 1024, _lib.EPI_SWIGLU, 5 + m, poison_row=m - 1) & 1


@pytest.mark.parametrize("m", [33, 130, 257])
@pytest.mark.parametrize("n,k", [(128, 64), (256, 1024), (384, 4096)])
def test_gemm_large_m_bf16_and_f32_epilogues(m, n, k):
    # 33-256 rows: the panel kernel (FP32) and the decode kernel over row
    # chunks (bf16); 257 rows: the compute-bound kernel (128 x 128 blocks,
    # no split-K).
    got, ref = _gemm_case(m, n, k, _lib.EPI_F32, m * 5 + n)
    assert np.max(np.abs(got - ref)) <= F32_BOUND
    got, ref = _gemm_case(m, n, k, _lib.EPI_BF16, m * 5 + n + 1)
    assert du.bf16_close(got, ref, ulps=1)
    assert np.mean(got == ref) > 0.99


@pytest.mark.parametrize("m,n,k,epi", [(160, 6144, 1024, "bf16"), (160, 6144, 1024, "f32"), (100, 24576, 256, "swiglu"),
                                       (70, 4096, 2048, "residual")])
def test_gemm_wide_batches(m, n, k, epi):
    # 33-256 rows: bf16 and residual outputs run the decode kernel over row
    # chunks (64-row chunks, or 32-row ones where an 8-wave launch of 64-row
    # chunks would need more than one round of the CUs: n = 6144 at 160
    # rows); FP32 and the fused gate/up run the panel kernel.
    code = {"bf16": _lib.EPI_BF16, "f32": _lib.EPI_F32, "swiglu": _lib.EPI_SWIGLU, "residual": _lib.EPI_RESIDUAL}[epi]
    got, ref = _gemm_case(m, n, k, code, 31 * m + n + k)
    if epi == "f32":
        assert np.max(np.abs(got - ref)) <= F32_BOUND
    else:
        assert du.bf16_close(got, ref, ulps=3 if epi == "swiglu" else 1)
        assert np.mean(got == ref) > 0.97


@pytest.mark.parametrize("m", [40, 200])
def test_gemm_large_m_residual_and_swiglu_epilogues(m):
    got, ref = _gemm_case(m, 512, 4096, _lib.EPI_RESIDUAL, 77 + m)
    assert du.bf16_close(got, ref, ulps=1)
    assert np.mean(got == ref) > 0.99
    for n in (256, 1024):
        got, ref = _gemm_case(m, n, 1024, _lib.EPI_SWIGLU, 177 + m + n)
        assert du.bf16_close(got, ref, ulps=3)
        assert np.mean(got == ref) > 0.97


@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("rows,width", [(1, 1024), (32, 4096), (9, 4096), (100, 1024), (256, 4096), (300, 1024)])
def test_residual_rmsnorm(splits, rows, width):
    if splits and rows > 256:
        pytest.skip("split-K partial slabs hold at most 256 rows")
    r = rng(splits * 100 + rows)
    hidden = rand_bf16(r, rows * width, 2.0)
    w = rand_bf16(r, width, 1.0)
    slab_rows = int(LIB.fh_partial_slab_rows(rows))  # 32 up to 32 rows, else 256
    slabs = (r.standard_normal((max(splits, 1), slab_rows, width)) * 0.5).astype(np.float32)
    dh, dw_, dp = du.to_dev(hidden), du.to_dev(w), du.to_dev(slabs.reshape(-1))
    dy = du.empty(tiled_rows(rows) * width, np.uint16)
    err = du.empty(1, np.uint32)
    _lib.check(LIB.fh_op_residual_rmsnorm(du.ptr(dh), du.ptr(dp) if splits else None, splits, du.ptr(dw_), du.ptr(dy),
                                          1, rows, width, 1e-6, du.ptr(err), du.stream()))
    assert du.to_host(err, np.uint32)[0] == 0
    new_h = du.to_host(dh, np.uint16)
    if splits:
        total = slabs[0, :rows].copy()
        for sp in range(1, splits):
            total = (total + slabs[sp, :rows]).astype(np.float32)
        exp_h = orc.residual(total.reshape(-1), hidden)  # bf16((0 + P) + h): bit-exact
    else:
        exp_h = hidden
    assert np.array_equal(new_h, exp_h)
    y = du.empty(rows * width, np.uint16)
    _lib.check(LIB.fh_op_untile_activation(du.ptr(dy), du.ptr(y), rows, width, du.stream()))
    got = du.to_host(y, np.uint16)
    ref = orc.rmsnorm(exp_h, w, rows, width)
    assert du.bf16_ulp_diff(got, ref) <= 2
    assert np.mean(got == ref) > 0.99


def test_residual_narrowing_is_the_reference_rounding():
    # hidden = bf16((0 + P) + 0) narrows arbitrary FP32 partials: ties to
    # even, carries into the exponent, subnormals, overflow to infinity and
    # NaN payloads (quieted, upper bits kept) must come out bit-exact
    # (gemm reference.rs:112-135 vectors among them). Nonfinite outputs set
    # the error word; the narrowed values are written either way.
    special = [0x3f808000, 0x3f818000, 0x3f807fff, 0x3f808001, 0x3f7fffff, 0x7f7fffff, 0x7f7f7fff,
               0x00008000, 0x00018000, 0x80008000, 0x807fffff, 0x7f800000, 0xff800000, 0x7fc00000,
               0x7fa10001, 0xffa10001, 0x7f800001, 0x00000000, 0x80000000, 0x477fe000, 0xc77fe000]
    width = 1024
    bits = np.concatenate([np.array(special, np.uint32),
                           rng(7).integers(0, 2**32, width - len(special), dtype=np.uint64).astype(np.uint32)])
    slab = np.zeros((32, width), np.float32)
    slab[0] = bits.view(np.float32)
    hidden = np.zeros(width, np.uint16)
    dh, dp = du.to_dev(hidden), du.to_dev(slab.reshape(-1))
    dw_ = du.to_dev(np.full(width, 0x3f80, np.uint16))
    dy = du.empty(tiled_rows(1) * width, np.uint16)
    err = du.empty(1, np.uint32)
    _lib.check(LIB.fh_op_residual_rmsnorm(du.ptr(dh), du.ptr(dp), 1, du.ptr(dw_), du.ptr(dy), 1, 1, width, 1e-6,
                                          du.ptr(err), du.stream()))
    got = du.to_host(dh, np.uint16)
    exp, rejected = orc.residual(slab[0].copy(), hidden, with_rejections=True)
    assert np.array_equal(got, exp), [(hex(b), hex(g), hex(e)) for b, g, e in zip(bits, got, exp) if g != e][:8]
    assert exp[0] == 0x3f80 and exp[1] == 0x3f82 and exp[14] == 0x7fe1  # the vectors' known answers
    assert rejected.any()
    assert du.to_host(err, np.uint32)[0] != 0  # infinities and NaNs were seen, as the reference rejects


# One-row projections with the residual + RMSNorm in their prologue
# (fh_op_gemm_rmsnorm) on the tile shapes the Qwen3-8B and Qwen3-0.6B one-row
# steps launch: (n, k, epilogue, splits, norm slabs). The LM head (151936
# rows) is stood in by 16384 rows, which take the same tiles.
ROWNORM_CASES = [
    (6144, 4096, _lib.EPI_PARTIAL, 2, 0), (6144, 4096, _lib.EPI_PARTIAL, 2, 4),  # 8B QKV, layer 0 and after
    (24576, 4096, _lib.EPI_SWIGLU, 1, 4), (16384, 4096, _lib.EPI_F32, 1, 4),  # 8B gate/up, head
    (4096, 1024, _lib.EPI_PARTIAL, 2, 0), (4096, 1024, _lib.EPI_PARTIAL, 2, 6),  # 0.6B QKV
    (6144, 1024, _lib.EPI_SWIGLU, 1, 4), (16384, 1024, _lib.EPI_F32, 1, 6),  # 0.6B gate/up (8 waves), head
]


def _rownorm_pair(n, k, epi, splits, ns, poison=None):
    """The same row through fh_op_residual_rmsnorm + fh_op_gemm and through
    fh_op_gemm_rmsnorm: (outputs, folded rows, error words) of each."""
    r = rng(n + k + ns)
    hidden = rand_bf16(r, k, 2.0)
    if poison is not None:
        hidden[poison] = 0x7FC0
    w_norm = rand_bf16(r, k, 1.0)
    slabs = (r.standard_normal((max(ns, 1), 32, k)) * 0.5).astype(np.float32)
    dt = du.empty(n * k, np.uint16)  # the tiled weight, filled directly (both paths read the same tiles)
    _lib.check(LIB.fh_op_synth_fill(du.ptr(dt), n * k, orc.synth_tensor_seed(n + k, 3, 1), orc.synth_scale(0.02),
                                    du.stream()))
    dp, dwn = du.to_dev(slabs.reshape(-1)), du.to_dev(w_norm)
    if epi == _lib.EPI_SWIGLU:
        fill, ldo = np.full(tiled_rows(1) * (n // 2), 0xFFFF, np.uint16), n // 2
    else:
        words = splits * 32 * n if epi == _lib.EPI_PARTIAL else n
        fill, ldo = np.full(words, np.nan, np.float32), n
    # two launches
    dh, dy = du.to_dev(hidden), du.empty(tiled_rows(1) * k, np.uint16)
    out_a, err_a = du.to_dev(fill), du.to_dev(np.zeros(1, np.uint32))
    _lib.check(LIB.fh_op_residual_rmsnorm(du.ptr(dh), du.ptr(dp) if ns else None, ns, du.ptr(dwn), du.ptr(dy), 1, 1,
                                          k, 1e-6, du.ptr(err_a), du.stream()))
    _lib.check(LIB.fh_op_gemm(du.ptr(dy), du.ptr(dt), 1, n, k, epi, splits, None, du.ptr(out_a), ldo, du.ptr(err_a),
                              du.stream()))
    # one launch
    dh_in, dh_out = du.to_dev(hidden), du.to_dev(np.full(k, 0xFFFF, np.uint16))
    out_b, err_b = du.to_dev(fill), du.to_dev(np.zeros(1, np.uint32))
    _lib.check(LIB.fh_op_gemm_rmsnorm(du.ptr(dh_in), du.ptr(dh_out), du.ptr(dp) if ns else None, ns, du.ptr(dwn),
                                      1e-6, du.ptr(dt), n, k, epi, splits, du.ptr(out_b), ldo, du.ptr(err_b),
                                      du.stream()))
    dtype = np.uint16 if epi == _lib.EPI_SWIGLU else np.uint32
    assert np.array_equal(du.to_host(dh_in, np.uint16), hidden)  # the input row is never written
    return ((du.to_host(out_a, dtype), du.to_host(dh, np.uint16), int(du.to_host(err_a, np.uint32)[0])),
            (du.to_host(out_b, dtype), du.to_host(dh_out, np.uint16), int(du.to_host(err_b, np.uint32)[0])))


@pytest.mark.parametrize("n,k,epi,splits,ns", ROWNORM_CASES)
def test_gemm_rmsnorm_equals_the_two_launches(n, k, epi, splits, ns):
    # Bar: bit-equal outputs (every slab, bf16 tile or FP32 logit, untouched
    # words included), folded residual row and error word: the fused launch
    # keeps both kernels' arithmetic and summation order.
    assert LIB.fh_gemm_rmsnorm_supported(n, k, epi, splits, ns) == 1
    (out_a, h_a, err_a), (out_b, h_b, err_b) = _rownorm_pair(n, k, epi, splits, ns)
    assert err_a == 0 and err_b == 0
    diff = np.flatnonzero(out_a != out_b)
    assert diff.size == 0, (diff.size, diff[:8])
    if ns:
        assert np.array_equal(h_b, h_a)
    else:
        assert np.all(h_b == 0xFFFF)  # no slabs: nothing folded, nothing written


@pytest.mark.parametrize("n,k,epi,splits,ns", [ROWNORM_CASES[1], ROWNORM_CASES[6]])
def test_gemm_rmsnorm_reports_nonfinite_rows(n, k, epi, splits, ns):
    # A NaN in the residual row: both paths raise the nonfinite bit.
    (_, _, err_a), (_, _, err_b) = _rownorm_pair(n, k, epi, splits, ns, poison=5)
    assert err_a != 0 and err_b == err_a


@pytest.mark.parametrize("n,k,epi,ns", [(151936, 4096, _lib.EPI_F32, 4), (151936, 1024, _lib.EPI_F32, 6),
                                        (24576, 4096, _lib.EPI_SWIGLU, 4), (6144, 4096, _lib.EPI_PARTIAL, 4)])
def test_one_row_projections_at_full_width_match_oracle(n, k, epi, ns):
    # The one-row projections at the full Qwen3 widths (the LM head's 151936
    # rows at both model widths, the 8B gate/up and QKV) against the oracle:
    # the fused norm + projection and the two launches. Weights are
    # synthesized on the device untiled and tiled there; the oracle
    # regenerates them. Bars: FP32 outputs within F32_BOUND, SwiGLU within 3
    # bf16 ulps (as the GEMM tests above), the folded row bit-exact.
    r = rng(n + ns)
    splits = int(LIB.fh_gemm_default_splits(n, k)) if epi == _lib.EPI_PARTIAL else 1
    ts, scale = orc.synth_tensor_seed(n + k, 9, 1), orc.synth_scale(0.02)
    dw, dt = du.empty(n * k, np.uint16), du.empty(n * k, np.uint16)
    _lib.check(LIB.fh_op_synth_fill(du.ptr(dw), n * k, ts, scale, du.stream()))
    if epi == _lib.EPI_SWIGLU:
        _lib.check(LIB.fh_op_tile_gate_up(du.ptr(dw), du.ptr(dw) + (n // 2) * k * 2, du.ptr(dt), n // 2, k, du.stream()))
    else:
        _lib.check(LIB.fh_op_tile_weight(du.ptr(dw), du.ptr(dt), n, k, du.stream()))
    del dw
    w = orc.synth(n * k, ts, scale)
    hidden, w_norm = rand_bf16(r, k, 2.0), rand_bf16(r, k, 1.0)
    slabs = (r.standard_normal((ns, 32, k)) * 0.5).astype(np.float32)
    total = slabs[0, 0].copy()
    for sp in range(1, ns):
        total = (total + slabs[sp, 0]).astype(np.float32)
    h_exp = orc.residual(total, hidden)
    x = orc.rmsnorm(h_exp, w_norm, 1, k)
    if epi == _lib.EPI_SWIGLU:
        i = n // 2
        ref = orc.swiglu(orc.gemm(x, w[: i * k], 1, i, k), orc.gemm(x, w[i * k:], 1, i, k))
        fill, ldo = np.full(tiled_rows(1) * i, 0xFFFF, np.uint16), i
    else:
        ref = orc.gemm(x, w, 1, n, k, f32_out=True)
        fill, ldo = np.full(splits * 32 * n if epi == _lib.EPI_PARTIAL else n, np.nan, np.float32), n
    del w
    dp, dwn = du.to_dev(slabs.reshape(-1)), du.to_dev(w_norm)

    def outputs(out):
        if epi == _lib.EPI_SWIGLU:
            o = du.empty(n // 2, np.uint16)
            _lib.check(LIB.fh_op_untile_activation(du.ptr(out), du.ptr(o), 1, n // 2, du.stream()))
            return du.to_host(o, np.uint16)
        got = du.to_host(out, np.float32)
        if epi == _lib.EPI_PARTIAL:
            s = got.reshape(splits, 32, n)[:, 0]
            acc = s[0].copy()
            for sp in range(1, splits):
                acc = (acc + s[sp]).astype(np.float32)
            return acc
        return got

    def check(got, label):
        if epi == _lib.EPI_SWIGLU:
            assert du.bf16_close(got, ref, ulps=3), label
        else:
            err = np.abs(got.astype(np.float64) - ref)
            assert np.max(err) <= F32_BOUND, (label, float(np.max(err)), int(np.argmax(err)))

    dh_in, dh_out, out, err = du.to_dev(hidden), du.empty(k, np.uint16), du.to_dev(fill), du.empty(1, np.uint32)
    _lib.check(LIB.fh_op_gemm_rmsnorm(du.ptr(dh_in), du.ptr(dh_out), du.ptr(dp), ns, du.ptr(dwn), 1e-6, du.ptr(dt), n,
                                      k, epi, splits, du.ptr(out), ldo, du.ptr(err), du.stream()))
    assert du.to_host(err, np.uint32)[0] == 0
    assert np.array_equal(du.to_host(dh_out, np.uint16), h_exp)
    check(outputs(out), "fused")
    dh, dy, out2 = du.to_dev(hidden), du.empty(tiled_rows(1) * k, np.uint16), du.to_dev(fill)
    _lib.check(LIB.fh_op_residual_rmsnorm(du.ptr(dh), du.ptr(dp), ns, du.ptr(dwn), du.ptr(dy), 1, 1, k, 1e-6, None,
                                          du.stream()))
    _lib.check(LIB.fh_op_gemm(du.ptr(dy), du.ptr(dt), 1, n, k, epi, splits, None, du.ptr(out2), ldo, None, du.stream()))
    check(outputs(out2), "two launches")


def _paged_pool(r, pages, kvh, scale=1.0):
    n = pages * 16 * kvh * 128
    return rand_bf16(r, n, scale), rand_bf16(r, n, scale)


def test_sqrt_rn_is_correctly_rounded_for_every_normal_float():
    # Every RMSNorm's inverse RMS takes a correctly rounded square root, as
    # the reference does (rmsnorm.rs:440-456). The hardware root is only
    # within 1 ulp (it made a QK-norm output differ from the oracle by one
    # bf16 ulp where x * inv fell next to a rounding boundary), so the device
    # corrects it; tests/hip/sqrt_rn_check checks that against the midpoint
    # definition over all 2,130,706,432 positive normal floats.
    import subprocess
    from pathlib import Path

    binary = Path(__file__).parent / "hip" / "sqrt_rn_check"
    assert binary.exists(), "build() compiles tests/hip/sqrt_rn_check"
    proc = subprocess.run([str(binary)], capture_output=True, text=True, timeout=120)
    print(proc.stdout.strip())
    assert proc.returncode == 0 and "failures 0" in proc.stdout, proc.stdout + proc.stderr


# rows = 260: bf16 rows beyond 256 take the lane-per-(row, head) kernel;
# rows = 160 with 5 splits: the wide batches' 256-row partial slabs.
@pytest.mark.parametrize("qh,kvh,splits,rows", [(32, 8, 0, 9), (16, 8, 0, 9), (32, 8, 1, 9), (32, 8, 3, 9),
                                                (32, 8, 0, 260), (32, 8, 5, 160)])
def test_qknorm_rope_kv_bit_exact(qh, kvh, splits, rows):
    r = rng(qh + splits + rows)
    pages, stride, context = 64, 64, 1024
    ld = (qh + 2 * kvh) * 128
    qkv = rand_bf16(r, rows * ld, 2.0)
    qn = rand_bf16(r, 128, 1.0)
    kn = rand_bf16(r, 128, 1.0)
    if rows == 9:
        positions = np.array([0, 1, 15, 16, 17, 255, 256, 511, 1023], np.uint32)
    else:
        positions = (np.arange(rows, dtype=np.uint32) * 3) % context  # distinct slots
    perm = r.permutation(pages).astype(np.uint32)
    table = np.tile(perm[:stride], (rows, 1)).astype(np.uint32)
    # distinct slots: each row writes its own position of the shared list
    cos = np.zeros(context * 64, np.float32)
    sin = np.zeros(context * 64, np.float32)
    for p in range(context):
        c, s = orc.rope_table(p)
        cos[p * 64:(p + 1) * 64], sin[p * 64:(p + 1) * 64] = c, s
    kc0, vc0 = _paged_pool(r, pages, kvh)
    dkc, dvc = du.to_dev(kc0), du.to_dev(vc0)
    dq = du.empty(rows * qh * 128, np.uint16)
    err = du.empty(1, np.uint32)
    if splits == 0:
        src = du.to_dev(qkv)
    else:
        # split-K slabs whose ordered f32 sum is exactly the bf16 value:
        # slab 0 = 2 v, slab 1 = -v (2v - v is exact), rest 0.
        vals = orc.bf16_to_f32(qkv).reshape(rows, ld)
        slabs = np.zeros((splits, int(LIB.fh_partial_slab_rows(rows)), ld), np.float32)
        if splits == 1:
            slabs[0, :rows] = vals
        else:
            slabs[0, :rows] = vals * np.float32(2.0)
            slabs[1, :rows] = -vals
        assert np.array_equal(((slabs[0, :rows] + (slabs[1, :rows] if splits > 1 else 0))).astype(np.float32), vals)
        src = du.to_dev(slabs.reshape(-1))
    keep = [du.to_dev(a) for a in (qn, kn, cos, sin, positions, table)]
    _lib.check(LIB.fh_op_qknorm_rope_kv(du.ptr(src), splits, *[du.ptr(t) for t in keep], du.ptr(dq), du.ptr(dkc),
                                        du.ptr(dvc), rows, qh, kvh, stride, pages, context, 1e-6, du.ptr(err),
                                        du.stream()))
    assert du.to_host(err, np.uint32)[0] == 0
    got_q = du.to_host(dq, np.uint16).reshape(rows, qh * 128)
    got_k = du.to_host(dkc, np.uint16)
    got_v = du.to_host(dvc, np.uint16)
    exp_k, exp_v = kc0.copy(), vc0.copy()
    for i in range(rows):
        row = qkv[i * ld:(i + 1) * ld]
        q = orc.rmsnorm(row[: qh * 128], qn, qh, 128)
        k = orc.rmsnorm(row[qh * 128:(qh + kvh) * 128], kn, kvh, 128)
        v = row[(qh + kvh) * 128:]
        c, s = orc.rope_table(int(positions[i]))
        qr = np.zeros_like(q)
        kr = np.zeros_like(k)
        for srcv, dst, heads in [(q, qr, qh), (k, kr, kvh)]:
            for h in range(heads):
                for j in range(64):
                    a, b = orc.rope_pair(int(srcv[h * 128 + j]), int(srcv[h * 128 + j + 64]), float(c[j]),
                                         float(s[j]))
                    dst[h * 128 + j], dst[h * 128 + j + 64] = a, b
        assert np.array_equal(got_q[i], qr), f"row {i} rotated q"
        pos = int(positions[i])
        page = int(table[i, pos // 16])
        base = orc.cache_index(page, pos % 16, kvh, 0, 0)
        exp_k[base:base + kvh * 128] = kr
        exp_v[base:base + kvh * 128] = v
    assert np.array_equal(got_k, exp_k), "K cache (rotated K at exactly the row slots, nothing else)"
    assert np.array_equal(got_v, exp_v), "V cache (raw V at exactly the row slots, nothing else)"


@pytest.mark.parametrize("qh,kvh", [(32, 8), (16, 8)])
@pytest.mark.parametrize("tiled,many", [(0, False), (1, False), (1, True), (0, None), (1, "short")])
def test_paged_attention_within_tolerance(qh, kvh, tiled, many):
    # Partition sizes follow the (rows x query heads) policy: 14 rows take
    # 32-page (qh 32) or 16-page (qh 16) partitions, 40 rows 32-page ones, and
    # 2 rows 16-page ones (up to 33 partitions per row). A 512-token context
    # ("short") takes one 32-page partition for every shape: each row ends in
    # its partition, with no records and no merge.
    r = rng(1000 + qh + 7 * bool(many) + 13 * (many is None) + 29 * (many == "short"))
    pages, stride, context = 600, 520, 8320
    if many == "short":
        context = 512
        positions = np.array([0, 15, 16, 255, 256, 257, 300, 400, 500, 511, 100, 7, 480, 290], np.uint32)
    elif many:
        # a prefill-size batch: 40 rows, tiled output of fh_activation_rows(40) rows
        positions = r.integers(0, 2000, 40).astype(np.uint32)
    elif many is None:
        positions = np.array([8319, 127], np.uint32)
    else:
        # one partition (<= 512 tokens), several partitions, page-boundary and partial-page cases
        positions = np.array([0, 15, 16, 255, 256, 511, 512, 513, 1000, 4095, 8319, 77, 8190, 6000], np.uint32)
    rows = len(positions)
    kc, vc = _paged_pool(r, pages, kvh)
    q = rand_bf16(r, rows * qh * 128, 1.0)
    table = np.stack([r.permutation(pages)[:stride] for _ in range(rows)]).astype(np.uint32)
    scratch = torch.zeros(LIB.fh_attention_scratch_bytes(rows, qh, context) // 4, dtype=torch.float32, device="cuda")
    out = du.empty((tiled_rows(rows) if tiled else rows) * qh * 128, np.uint16)
    err = du.empty(1, np.uint32)
    dkc, dvc = du.to_dev(kc), du.to_dev(vc)
    dq, dpos, dtab = du.to_dev(q), du.to_dev(positions), du.to_dev(table)
    _lib.check(LIB.fh_op_paged_attention(du.ptr(dq), du.ptr(dkc), du.ptr(dvc), du.ptr(dpos), du.ptr(dtab),
                                         du.ptr(out), tiled, du.ptr(scratch), rows, qh, kvh, stride, pages, context,
                                         du.ptr(err), du.stream()))
    assert du.to_host(err, np.uint32)[0] == 0
    if tiled:
        flat = du.empty(rows * qh * 128, np.uint16)
        _lib.check(LIB.fh_op_untile_activation(du.ptr(out), du.ptr(flat), rows, qh * 128, du.stream()))
        out = flat
    got = du.to_host(out, np.uint16).reshape(rows, qh, 128)
    g = qh // kvh
    worst = 0.0
    for i in range(rows):
        for h in range(qh):
            ref = orc.attention_head(q[(i * qh + h) * 128:(i * qh + h + 1) * 128], kc, vc, table[i], pages,
                                     int(positions[i]), kvh, h // g)
            assert ref is not None
            worst = max(worst, du.bf16_rel_err(got[i, h], ref))
            if positions[i] == 0:
                # one key: softmax weight 1, output = V row bits exactly
                assert np.array_equal(got[i, h], ref)
    assert worst <= 1e-2, worst


# (qh, kvh, positions): 32-page partitions with the separate merge (14 rows of
# the 8B shape, one to 17 partitions), 16-page partitions (one 8B row at a
# 4095-token context; 0.6B rows), pages of one and of several tokens, a
# batch of 32 rows.
@pytest.mark.parametrize("qh,kvh,positions,context", [
    (32, 8, [0, 15, 16, 255, 256, 511, 512, 513, 1000, 4095, 4190, 77, 3000, 2047], 4224),
    (32, 8, [4095], 4224),
    (16, 8, [0, 17, 300, 2047, 1500, 999, 16, 4000], 4224),
    (32, 8, "b32", 4224),
    (16, 8, "b32", 4224),
    (16, 8, "b32", 512),
    (32, 8, [0, 300, 511, 256, 257], 512),
])
def test_qknorm_paged_attention_equals_the_two_launches(qh, kvh, positions, context):
    # The decode step's fused form (QK-norm + RoPE + KV append inside the
    # attention partitions) against fh_op_qknorm_rope_kv then
    # fh_op_paged_attention on the same split-K slabs: attention output, K and
    # V caches and the error word bit for bit. Each row writes a page no
    # other row lists (the fused form's contract).
    r = rng(4242 + qh + (len(positions) if isinstance(positions, list) else 99) + (context if context != 4224 else 0))
    pages, stride = 4096, 264
    if positions == "b32":
        positions = r.integers(0, min(2048, context), 32)
    positions = np.asarray(positions, np.uint32)
    rows = len(positions)
    per_row = pages // rows
    perm = r.permutation(pages).astype(np.uint32)
    table = np.full((rows, stride), 0xFFFFFFFF, np.uint32)
    for i in range(rows):
        n = min(stride, per_row)
        table[i, :n] = perm[i * per_row:i * per_row + n]
        assert int(positions[i]) // 16 < n
    ld = (qh + 2 * kvh) * 128
    slab_rows = int(LIB.fh_partial_slab_rows(rows))
    # Two slabs of random FP32 partial sums (their ordered sum is rounded to bf16).
    slabs = (r.standard_normal((2, slab_rows, ld)) * 0.7).astype(np.float32)
    qn = rand_bf16(r, 128, 1.0)
    kn = rand_bf16(r, 128, 1.0)
    cos = np.zeros(context * 64, np.float32)
    sin = np.zeros(context * 64, np.float32)
    for p in np.unique(positions):
        c, s = orc.rope_table(int(p))
        cos[p * 64:(p + 1) * 64], sin[p * 64:(p + 1) * 64] = c, s
    kc0, vc0 = _paged_pool(r, pages, kvh)
    keep = [du.to_dev(a) for a in (slabs.reshape(-1), qn, kn, cos, sin, positions, table)]
    dslab, dqn, dkn, dcos, dsin, dpos, dtab = keep
    scratch = torch.zeros(LIB.fh_attention_scratch_bytes(rows, qh, context) // 4, dtype=torch.float32, device="cuda")
    out_n = tiled_rows(rows) * qh * 128

    # two launches
    kca, vca = du.to_dev(kc0), du.to_dev(vc0)
    q = du.empty(rows * qh * 128, np.uint16)
    outa = du.empty(out_n, np.uint16)
    erra = du.empty(1, np.uint32)
    _lib.check(LIB.fh_op_qknorm_rope_kv(du.ptr(dslab), 2, du.ptr(dqn), du.ptr(dkn), du.ptr(dcos), du.ptr(dsin),
                                        du.ptr(dpos), du.ptr(dtab), du.ptr(q), du.ptr(kca), du.ptr(vca), rows, qh,
                                        kvh, stride, pages, context, 1e-6, du.ptr(erra), du.stream()))
    _lib.check(LIB.fh_op_paged_attention(du.ptr(q), du.ptr(kca), du.ptr(vca), du.ptr(dpos), du.ptr(dtab),
                                         du.ptr(outa), 1, du.ptr(scratch), rows, qh, kvh, stride, pages, context,
                                         du.ptr(erra), du.stream()))
    # fused
    kcb, vcb = du.to_dev(kc0), du.to_dev(vc0)
    outb = du.empty(out_n, np.uint16)
    errb = du.empty(1, np.uint32)
    scratch.zero_()
    _lib.check(LIB.fh_op_qknorm_paged_attention(du.ptr(dslab), 2, du.ptr(dqn), du.ptr(dkn), du.ptr(dcos),
                                                du.ptr(dsin), du.ptr(dpos), du.ptr(dtab), du.ptr(kcb), du.ptr(vcb),
                                                du.ptr(outb), 1, du.ptr(scratch), rows, qh, kvh, stride, pages,
                                                context, 1e-6, du.ptr(errb), du.stream()))
    ea, eb = du.to_host(erra, np.uint32)[0], du.to_host(errb, np.uint32)[0]
    assert ea == 0 and eb == 0, (ea, eb)
    assert np.array_equal(du.to_host(kca, np.uint16), du.to_host(kcb, np.uint16)), "K cache"
    assert np.array_equal(du.to_host(vca, np.uint16), du.to_host(vcb, np.uint16)), "V cache"
    ga, gb = du.to_host(outa, np.uint16), du.to_host(outb, np.uint16)
    assert np.array_equal(ga, gb), f"attention output: {int(np.sum(ga != gb))} of {ga.size} words differ"
    # The appended slots hold the new token (not the pool's old contents).
    assert not np.array_equal(du.to_host(kcb, np.uint16), kc0)


def test_qknorm_paged_attention_errors_match_the_two_launches():
    # A row whose written page is outside the pool, and one whose position is
    # outside the context: the same error bits as the two-launch form
    # (page fault; position and page fault), and no slot written for them.
    r = rng(31)
    qh, kvh, pages, stride, context = 32, 8, 256, 64, 1024
    positions = np.array([100, 40, 1024, 7], np.uint32)
    rows = len(positions)
    table = np.full((rows, stride), 0xFFFFFFFF, np.uint32)
    perm = r.permutation(pages).astype(np.uint32)
    for i in range(rows):
        table[i] = perm[i * stride:(i + 1) * stride]
    table[1, 40 // 16] = pages + 3
    ld = (qh + 2 * kvh) * 128
    slabs = (r.standard_normal((2, int(LIB.fh_partial_slab_rows(rows)), ld)) * 0.7).astype(np.float32)
    qn, kn = rand_bf16(r, 128, 1.0), rand_bf16(r, 128, 1.0)
    cos = np.zeros(context * 64, np.float32)
    sin = np.zeros(context * 64, np.float32)
    kc0, vc0 = _paged_pool(r, pages, kvh)
    keep = [du.to_dev(a) for a in (slabs.reshape(-1), qn, kn, cos, sin, positions, table)]
    dslab, dqn, dkn, dcos, dsin, dpos, dtab = keep
    scratch = torch.zeros(LIB.fh_attention_scratch_bytes(rows, qh, context) // 4, dtype=torch.float32, device="cuda")
    res = []
    for fused in (False, True):
        kc, vc = du.to_dev(kc0), du.to_dev(vc0)
        out = du.empty(tiled_rows(rows) * qh * 128, np.uint16)
        err = du.empty(1, np.uint32)
        if fused:
            _lib.check(LIB.fh_op_qknorm_paged_attention(du.ptr(dslab), 2, du.ptr(dqn), du.ptr(dkn), du.ptr(dcos),
                                                        du.ptr(dsin), du.ptr(dpos), du.ptr(dtab), du.ptr(kc),
                                                        du.ptr(vc), du.ptr(out), 1, du.ptr(scratch), rows, qh, kvh,
                                                        stride, pages, context, 1e-6, du.ptr(err), du.stream()))
        else:
            q = du.empty(rows * qh * 128, np.uint16)
            _lib.check(LIB.fh_op_qknorm_rope_kv(du.ptr(dslab), 2, du.ptr(dqn), du.ptr(dkn), du.ptr(dcos),
                                                du.ptr(dsin), du.ptr(dpos), du.ptr(dtab), du.ptr(q), du.ptr(kc),
                                                du.ptr(vc), rows, qh, kvh, stride, pages, context, 1e-6,
                                                du.ptr(err), du.stream()))
            _lib.check(LIB.fh_op_paged_attention(du.ptr(q), du.ptr(kc), du.ptr(vc), du.ptr(dpos), du.ptr(dtab),
                                                 du.ptr(out), 1, du.ptr(scratch), rows, qh, kvh, stride, pages,
                                                 context, du.ptr(err), du.stream()))
        res.append((du.to_host(err, np.uint32)[0], du.to_host(kc, np.uint16), du.to_host(vc, np.uint16)))
    assert res[0][0] == res[1][0] == 4 | 8, (res[0][0], res[1][0])
    assert np.array_equal(res[0][1], res[1][1]) and np.array_equal(res[0][2], res[1][2])


def test_paged_attention_out_of_pool_page_is_a_page_error():
    # A page-table entry past the pool is an index fault (the reference traps
    # on it, paged_decode.rs:440-470): the error word carries the page bit, not
    # the nonfinite bit, and the kernel reads nothing outside the pool.
    r = rng(77)
    qh, kvh, pages, stride, context = 32, 8, 64, 64, 1024
    positions = np.array([700, 40, 5], np.uint32)
    kc, vc = _paged_pool(r, pages, kvh)
    q = rand_bf16(r, len(positions) * qh * 128, 1.0)
    table = np.stack([r.permutation(pages)[:stride] for _ in positions]).astype(np.uint32)
    table[0, 3] = pages + 5  # row 0 reads logical page 3
    scratch = torch.zeros(LIB.fh_attention_scratch_bytes(3, qh, context) // 4, dtype=torch.float32, device="cuda")
    out = du.empty(3 * qh * 128, np.uint16)
    err = du.empty(1, np.uint32)
    keep = [du.to_dev(a) for a in (q, kc, vc, positions, table)]
    _lib.check(LIB.fh_op_paged_attention(*[du.ptr(t) for t in keep], du.ptr(out), 0, du.ptr(scratch), 3, qh, kvh,
                                         stride, pages, context, du.ptr(err), du.stream()))
    assert du.to_host(err, np.uint32)[0] == 8  # ERR_PAGE only


def test_paged_attention_long_context():
    # 40960-token context: up to 80 partitions per row, more than one 64-lane
    # chunk of partition weights in the merge; a page table of 2560 entries.
    r = rng(4242)
    qh, kvh = 32, 8
    pages, stride, context = 2600, 2560, 40960
    positions = np.array([40959, 32767, 32768, 16384, 511, 512, 0, 40000], np.uint32)
    rows = len(positions)
    kc, vc = _paged_pool(r, pages, kvh)
    q = rand_bf16(r, rows * qh * 128, 1.0)
    table = np.stack([r.permutation(pages)[:stride] for _ in range(rows)]).astype(np.uint32)
    scratch = torch.zeros(LIB.fh_attention_scratch_bytes(rows, qh, context) // 4, dtype=torch.float32, device="cuda")
    out = du.empty(rows * qh * 128, np.uint16)
    err = du.empty(1, np.uint32)
    dkc, dvc = du.to_dev(kc), du.to_dev(vc)
    dq, dpos, dtab = du.to_dev(q), du.to_dev(positions), du.to_dev(table)
    _lib.check(LIB.fh_op_paged_attention(du.ptr(dq), du.ptr(dkc), du.ptr(dvc), du.ptr(dpos), du.ptr(dtab),
                                         du.ptr(out), 0, du.ptr(scratch), rows, qh, kvh, stride, pages, context,
                                         du.ptr(err), du.stream()))
    assert du.to_host(err, np.uint32)[0] == 0
    got = du.to_host(out, np.uint16).reshape(rows, qh, 128)
    worst = 0.0
    for i in range(rows):
        for h in range(0, qh, 5):  # a spread of query heads over every KV head
            ref = orc.attention_head(q[(i * qh + h) * 128:(i * qh + h + 1) * 128], kc, vc, table[i], pages,
                                     int(positions[i]), kvh, h // (qh // kvh))
            worst = max(worst, du.bf16_rel_err(got[i, h], ref))
    assert worst <= 1e-2, worst


def test_swiglu_standalone():
    r = rng(5)
    n = 1 << 15
    gate = rand_bf16(r, n, 4.0)
    up = rand_bf16(r, n, 1.0)
    gate[:6] = [0x0000, 0x8000, 0x3F80, 0xBF80, 0x42C8, 0xC2C8]
    up[:6] = [0x4000, 0x4000, 0x3F80, 0x3F80, 0x3F00, 0x3F00]
    out = du.empty(n, np.uint16)
    err = du.empty(1, np.uint32)
    dg, dup = du.to_dev(gate), du.to_dev(up)
    _lib.check(LIB.fh_op_swiglu(du.ptr(dg), du.ptr(dup), du.ptr(out), n, du.ptr(err), du.stream()))
    got = du.to_host(out, np.uint16)
    ref = orc.swiglu(gate, up)
    assert du.to_host(err, np.uint32)[0] == 0
    assert got[0] == 0x0000 and got[1] == 0x8000  # signed zeros (swiglu reference.rs:64-88)
    assert du.bf16_ulp_diff(got, ref) <= 1  # device exp vs host libm exp: last-ulp differences only
    assert np.mean(got == ref) > 0.999


def test_argmax_lowest_id_ties_and_nonfinite():
    r = rng(6)
    rows, vocab = 7, 151936
    logits = r.standard_normal(rows * vocab).astype(np.float32).reshape(rows, vocab)
    logits[1, 5] = logits[1, 90000] = 50.0  # exact tie: lowest id wins
    logits[2, :] = 0.0
    logits[2, 3] = -0.0  # +0/-0 tie: id 0 wins
    logits[3, 151935] = 99.0  # last id
    logits[4, 2374 * 5 - 1] = logits[4, 2374 * 5] = 7.0  # tie across a shard boundary
    scratch = torch.zeros(LIB.fh_argmax_scratch_bytes(rows) // 4, dtype=torch.int32, device="cuda")
    ch = du.empty(rows, np.uint32)
    err = du.empty(1, np.uint32)
    dl = du.to_dev(logits.reshape(-1))
    _lib.check(LIB.fh_op_argmax(du.ptr(dl), rows, vocab, du.ptr(scratch), du.ptr(ch), du.ptr(err), du.stream()))
    got = du.to_host(ch, np.uint32)
    assert du.to_host(err, np.uint32)[0] == 0
    for i in range(rows):
        assert got[i] == orc.argmax_f32(logits[i])[0], i
    assert got[1] == 5 and got[2] == 0 and got[3] == 151935 and got[4] == 2374 * 5 - 1
    logits[6, 1234] = np.nan
    dl = du.to_dev(logits.reshape(-1))
    _lib.check(LIB.fh_op_argmax(du.ptr(dl), rows, vocab, du.ptr(scratch), du.ptr(ch), du.ptr(err), du.stream()))
    assert du.to_host(err, np.uint32)[0] != 0
