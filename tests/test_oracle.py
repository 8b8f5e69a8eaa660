"""The oracle pinned against the reference's own known-answer vectors and
against closed forms, before it is trusted as the GPU's checker.

Each test names the reference file:line whose vector it reproduces. Where
the reference has no vector, the check is a closed form or a brute-force
restatement chosen so that a plausible slip (a dropped term, a wrong sign or
index, a transposed operand, a different reduction order) fails it.
"""

import math

import numpy as np
import pytest

from oracle import oracle as orc


def f32_bits(x: float) -> int:
    return int(np.array([x], np.float32).view(np.uint32)[0])


def f32_from_bits(b: int) -> float:
    return float(np.array([b], np.uint32).view(np.float32)[0])


def bf16(vals):
    return orc.f32_to_bf16(np.asarray(vals, np.float32))


# ---- bf16 narrowing: device/qwen3-gemm-v1/tests/reference.rs:112-135,
#      device/qwen3-rmsnorm-v1/tests/reference.rs:255-262 ----
@pytest.mark.parametrize("bits,expected", [
    (0x00000000, 0x0000), (0x80000000, 0x8000), (0x3F800000, 0x3F80), (0x3F808000, 0x3F80),
    (0x3F818000, 0x3F82), (0x7F800000, 0x7F80), (0xFF800000, 0xFF80), (0x7F800001, 0x7FC0),
    (0xFF800001, 0xFFC0), (0x7FA10001, 0x7FE1), (0x3F807FFF, 0x3F80), (0x3F808001, 0x3F81),
])
def test_bf16_rne_and_nan_quieting(bits, expected):
    assert orc.bf16_from_f32_scalar(f32_from_bits(bits)) == expected
    assert int(orc.f32_to_bf16(np.array([bits], np.uint32).view(np.float32))[0]) == expected


# ---- GEMM: device/qwen3-gemm-v1/tests/reference.rs:137-206 ----
def test_gemm_known_answers():
    a = bf16([1.0, 2.0, 3.0, 4.0, -1.0, 0.5, 2.0, -2.0])
    b = bf16([1.0, 0.5, -1.0, 2.0, 0.0, 2.0, 1.0, -0.5, -1.0, 1.0, 0.25, 0.0])
    prior = np.full(6, 0x3F80, np.uint16)
    assert list(orc.gemm(a, b, 2, 3, 4)) == [0x40E0, 0x40A0, 0x3FE0, 0xC0D8, 0x4080, 0x4000]
    assert list(orc.gemm(a, b, 2, 3, 4, prior=prior)) == [0x4100, 0x40C0, 0x4030, 0xC0B8, 0x40A0, 0x4040]


def test_gemm_reference_equals_a4_on_rounding_sensitive_tails():
    palette = [-3.5, -1.25, -0.5, -0.01171875, 0.0, 0.00390625, 0.75, 1.0, 1.5, 2.25]
    m, n, k = 3, 5, 8
    a = bf16([palette[(i * 7 + 3) % 10] for i in range(m * k)])
    b = bf16([palette[(i * 3 + 1) % 10] for i in range(k * n)])
    prior = bf16([palette[(i * 9 + 2) % 10] for i in range(m * n)])
    for beta in (None, prior):
        assert np.array_equal(orc.gemm_a4(a, b, m, n, k, prior=beta), orc.gemm(a, b, m, n, k, prior=beta))


def test_gemm_beta_zero_ignores_nan_prior_and_beta_one_ties_to_even():
    a = bf16([1.0, 0.0, 0.0, 0.0])
    b = bf16([1.0, 0.0, 0.0, 0.0, 1.0, 0.0, 0.0, 0.0])
    assert list(orc.gemm(a, b, 1, 2, 4)) == [0x3F80, 0x3F80]
    assert list(orc.gemm(a, b, 1, 2, 4, prior=np.array([0x3B80, 0x3C40], np.uint16))) == [0x3F80, 0x3F82]


def test_gemm_is_the_serial_ascending_sum():
    # Brute force in numpy with the same operation order; a transposed operand
    # or a tree-ordered sum changes the bits of this cancellation-heavy case.
    r = np.random.default_rng(0)
    m, n, k = 5, 7, 257
    a = bf16(r.standard_normal(m * k) * 3)
    b = bf16(r.standard_normal(n * k) * 3)
    af = orc.bf16_to_f32(a).reshape(m, k)
    bf = orc.bf16_to_f32(b).reshape(n, k)
    exp = np.zeros((m, n), np.float32)
    for i in range(m):
        for j in range(n):
            acc = np.float32(0)
            for t in range(k):
                acc = np.float32(acc + np.float32(af[i, t] * bf[j, t]))
            exp[i, j] = acc
    assert np.array_equal(orc.gemm(a, b, m, n, k, f32_out=True).reshape(m, n).view(np.uint32), exp.view(np.uint32))
    assert np.array_equal(orc.gemm(a, b, m, n, k), orc.f32_to_bf16(exp).reshape(-1))


# ---- embedding: device/qwen3-gemm-v1/tests/reference.rs:208-225 ----
def test_embedding_bit_copy_and_oob():
    w = np.array([0x0000, 0x8000, 0x7F80, 0x7FC1, 0x3F80, 0xBF80, 0x0001, 0x7F7F, 0x4040, 0xC040, 0x3B80, 0xFFFF],
                 np.uint16)
    assert list(orc.embedding([2, 0, 1], w, 4, 3)) == [0x4040, 0xC040, 0x3B80, 0xFFFF, 0x0000, 0x8000, 0x7F80,
                                                       0x7FC1, 0x3F80, 0xBF80, 0x0001, 0x7F7F]
    assert orc.embedding([1, 3], w, 4, 3) == ("invalid", 1, 3)


# ---- RMSNorm: device/qwen3-rmsnorm-v1/tests/reference.rs ----
KAT_ROW = [
    16295, 16734, 15610, 16917, 16782, 17267, 16001, 15365, 17397, 15627, 16562, 15898, 15809, 16186, 17041, 16392,
    16277, 16725, 15587, 16964, 16853, 17263, 16043, 15361, 17318, 15708, 16557, 15923, 15850, 16176, 17133, 16399,
    16327, 16704, 15535, 16903, 16800, 17182, 16120, 15441, 17306, 15648, 16523, 15968, 15767, 16218, 17132, 16489,
    16317, 16670, 15584, 16991, 16879, 17154, 16106, 15478, 17362, 15705, 16590, 15906, 15816, 16184, 17040, 16407,
    16375, 16753, 15605, 16970, 16834, 17178, 16127, 15470, 17358, 15622, 16628, 15991, 15869, 16201, 17112, 16410,
    16373, 16696, 15597, 16969, 16793, 17254, 16057, 15418, 17294, 15655, 16639, 15968, 15798, 16143, 17091, 16496,
    16311, 16755, 15562, 16989, 16884, 17254, 16022, 15451, 17298, 15676, 16621, 15966, 15860, 16137, 17107, 16410,
    16317, 16674, 15498, 16900, 16852, 17177, 16024, 15439, 17370, 15685, 16576, 15983, 15797, 16183, 17030, 16408,
]


def test_rmsnorm_serial_square_sum_pins_the_order():
    # reference.rs:66-91: serial order -> 0x49be1c17; the XOR-tree order gives 0x49be1c1a.
    row = np.array(KAT_ROW, np.uint16)
    assert orc.square_sum_bits(row) == 0x49BE1C17
    lanes = np.zeros(64, np.float32)
    vals = orc.bf16_to_f32(row)
    for lane in range(64):
        for comp in range(64):
            c = lane + comp * 64
            if c < 128:
                lanes[lane] = np.float32(lanes[lane] + np.float32(vals[c] * vals[c]))
    off = 32
    while off:
        lanes = np.array([np.float32(lanes[i] + lanes[i ^ off]) for i in range(64)], np.float32)
        off >>= 1
    assert int(lanes[:1].view(np.uint32)[0]) == 0x49BE1C1A  # the order the oracle must not use


def test_rmsnorm_known_answers():
    for width in (128, 1024, 4096):
        ones = np.full(width, 0x3F80, np.uint16)
        assert np.array_equal(orc.rmsnorm(ones, ones, 1, width), ones)  # reference.rs:204-221
        zeros = np.zeros(2 * width, np.uint16)
        assert np.array_equal(orc.rmsnorm(zeros, ones, 2, width), zeros)  # reference.rs:185-202
    # normalize-then-round witness (reference.rs:264-274)
    w = bf16([0.546875])[0]
    out = orc.norm_weight(-1.5510881, int(w))
    assert orc.bf16_to_f32(np.array([out], np.uint16))[0] == np.float32(-0.8515625)
    # signed zero and even ties (reference.rs:276-290)
    for nb, exp in [(0x00000000, 0x0000), (0x80000000, 0x8000), (0x3F808000, 0x3F80), (0x3F818000, 0x3F82),
                    (0xBF808000, 0xBF80), (0xBF818000, 0xBF82)]:
        assert orc.norm_weight(f32_from_bits(nb), 0x3F80) == exp
    # overflow rejected even with a small weight (reference.rs:292-298)
    assert orc.norm_weight(float(np.finfo(np.float32).max), int(bf16([0.5])[0])) is None


def test_rmsnorm_fused_mode_and_rejections():
    for width in (1024, 4096):
        x = np.array([0x3F80 if i % 2 == 0 else 0xBF00 for i in range(width)], np.uint16)
        res = np.array([0x3E80 if i % 3 == 0 else 0x3F00 for i in range(width)], np.uint16)
        w = np.array([0x4000 if i % 5 == 0 else 0x3F80 for i in range(width)], np.uint16)
        fused, normed = orc.rmsnorm(x, w, 1, width, residual=res)
        assert np.array_equal(fused, orc.f32_to_bf16(orc.bf16_to_f32(x) + orc.bf16_to_f32(res)))
        assert len(set(normed.tolist())) > 1
    ones = np.full(128, 0x3F80, np.uint16)
    bad = ones.copy()
    bad[17] = 0x7F80
    assert orc.rmsnorm(bad, ones, 1, 128) is None
    badw = ones.copy()
    badw[31] = 0x7FC1
    assert orc.rmsnorm(ones, badw, 1, 128) is None
    assert orc.rmsnorm(np.full(128, 0x7F7F, np.uint16), ones, 1, 128) is None


def test_rmsnorm_closed_form():
    # a row of one repeated value v: sum = 128 v^2 exactly for small integers,
    # inverse = 1 / sqrt(v^2 + eps), output = bf16(bf16(v * inv) * w).
    for v in (0.5, 2.0, 3.0):
        x = bf16([v] * 128)
        w = bf16([1.5] * 128)
        inv = np.float32(1.0) / np.sqrt(np.float32(np.float32(v * v * 128) / np.float32(128) + np.float32(1e-6)))
        expect = orc.f32_to_bf16(orc.bf16_to_f32(orc.f32_to_bf16(np.float32(v) * inv)) * np.float32(1.5))
        assert np.all(orc.rmsnorm(x, w, 1, 128) == expect)


# ---- RoPE: device/qwen3-rope-kv-v1/tests/reference.rs:159-175; host table tp_execution.rs:1440-1450 ----
def test_rope_pair_known_answers():
    assert orc.rope_pair(0x3F80, 0x4000, 1.0, 0.0) == [0x3F80, 0x4000]
    assert orc.rope_pair(0x3F80, 0x4000, 0.0, 1.0) == [0xC000, 0x3F80]
    assert orc.rope_pair(0x3F80, 0x4000, 0.5, 0.25) == [0x0000, 0x3FA0]


def test_rope_table_closed_form():
    c, s = orc.rope_table(0)
    assert np.all(c == 1.0) and np.all(s == 0.0)
    for pos in (1, 17, 4095, 8191):
        c, s = orc.rope_table(pos)
        for pair in (0, 1, 31, 63):
            angle = pos * (1_000_000.0 ** (-pair / 64.0))
            assert c[pair] == np.float32(math.cos(angle)) and s[pair] == np.float32(math.sin(angle)), (pos, pair)


# ---- paged KV indexing: device/qwen3-rope-kv-v1/tests/reference.rs:177-283 ----
def test_cache_index_layout():
    assert orc.cache_index(7, 15, 8, 0, 0) == (7 * 16 + 15) * 1024
    assert orc.cache_index(3, 0, 8, 0, 0) == 3 * 16 * 1024
    assert orc.cache_index(16383, 15, 8, 7, 127) == 268_435_456 - 1
    for page, slot, head, feat in [(0, 0, 0, 0), (5, 9, 3, 77), (16383, 15, 7, 127)]:
        idx = orc.cache_index(page, slot, 8, head, feat)
        assert idx // 16384 == page and (idx % 16384) // 1024 == slot and (idx % 1024) == head * 128 + feat


# ---- paged decode: device/qwen3-paged-decode-v1/tests/reference.rs:200-351 ----
def _cache(pages):
    return np.zeros(pages * 16 * 8 * 128, np.uint16)


def test_attention_zero_scores_give_the_mean_value():
    q = np.zeros(128, np.uint16)
    k, v = _cache(2), _cache(2)
    v[:] = 0x3F00
    pages = np.zeros(512, np.uint32)
    pages[1] = 1
    for committed, active, qt in [(0, 1, 0), (13, 4, 3), (16, 1, 0)]:
        out = orc.attention_head(q, k, v, pages, 2, committed + qt, 8, 7)
        assert np.all(out[126:128] == 0x3F00)


def test_attention_page_table_indirection():
    q = np.zeros(128, np.uint16)
    k, v = _cache(2), _cache(2)
    idx = orc.cache_index(1, 0, 8, 3, 10)
    v[idx], v[idx + 1] = 0x3F80, 0xC000
    pages = np.zeros(2 * 512, np.uint32)
    pages[512] = 1
    out = orc.attention_head(q, k, v, pages[512:], 2, 0, 8, 3)
    assert list(out[10:12]) == [0x3F80, 0xC000]


def test_attention_online_recurrence_equals_batch_softmax():
    q = np.zeros(128, np.uint16)
    q[0] = 0x3F80
    k, v = _cache(1), _cache(1)
    kb = [0xBF80, 0x0000, 0x4000]
    vb = [[0x3F80, 0xC000], [0x4040, 0x4080], [0xC0A0, 0x40C0]]
    for t in range(3):
        k[orc.cache_index(0, t, 8, 0, 0)] = kb[t]
        v[orc.cache_index(0, t, 8, 0, 20)] = vb[t][0]
        v[orc.cache_index(0, t, 8, 0, 21)] = vb[t][1]
    out = orc.attention_head(q, k, v, np.zeros(512, np.uint32), 1, 2, 8, 0)
    scale = np.float32(f32_from_bits(0x3DB504F3))
    scores = np.array([-scale, 0.0, 2.0 * scale], np.float32)
    wts = np.exp(scores - scores.max()).astype(np.float32)
    den = np.float32(wts[0] + wts[1] + wts[2])
    e0 = orc.f32_to_bf16(np.float32((1.0 * wts[0] + 3.0 * wts[1] - 5.0 * wts[2]) / den))
    e1 = orc.f32_to_bf16(np.float32((-2.0 * wts[0] + 4.0 * wts[1] + 6.0 * wts[2]) / den))
    assert list(out[20:22]) == [int(e0), int(e1)]


def test_attention_causal_masking_and_rejections():
    q = np.full(128, 0x3F80, np.uint16)
    k, v = _cache(1), _cache(1)
    for t in range(16):
        for f in range(128):
            k[orc.cache_index(0, t, 8, 0, f)] = 0x3C00 if t <= 2 else 0x42C8
            v[orc.cache_index(0, t, 8, 0, f)] = 0x3F00 if t <= 2 else 0xC2C8
    pages = np.zeros(512, np.uint32)
    base = orc.attention_head(q, k, v, pages, 1, 2, 8, 0)
    for t in range(3, 16):
        for f in range(128):
            k[orc.cache_index(0, t, 8, 0, f)] = 0x7F7F
            v[orc.cache_index(0, t, 8, 0, f)] = 0x7F7F
    assert np.array_equal(orc.attention_head(q, k, v, pages, 1, 2, 8, 0), base)
    pages2 = np.zeros(512, np.uint32)
    pages2[0] = 16384
    assert orc.attention_head(np.zeros(128, np.uint16), _cache(1), _cache(1), pages2, 16384, 0, 8, 0) is None
    qn = np.zeros(128, np.uint16)
    qn[17] = 0x7F80
    assert orc.attention_head(qn, _cache(1), _cache(1), pages, 1, 0, 8, 0) is None


# ---- SwiGLU: device/qwen3-swiglu-v1/tests/reference.rs:56-88 ----
def test_swiglu_known_answers_and_closed_form():
    finite = [(0x0000, 0x4000), (0x8000, 0x4000), (0x3F80, 0x3F80), (0xBF80, 0x3F80), (0x42C8, 0x3F00),
              (0xC2C8, 0x3F00), (0x0001, 0x3F80), (0x7F7F, 0x0000)]
    g = np.array([a for a, _ in finite], np.uint16)
    u = np.array([b for _, b in finite], np.uint16)
    out = orc.swiglu(g, u)
    assert out is not None and out[0] == 0x0000 and out[1] == 0x8000
    for gb, ub in [(0x7F80, 0x3F80), (0x3F80, 0xFF80), (0x7FC1, 0x3F80)]:
        assert orc.swiglu(np.array([gb], np.uint16), np.array([ub], np.uint16)) is None
    # closed form: silu(1) * 1 = 1 / (1 + e^-1)
    assert orc.swiglu(bf16([1.0]), bf16([1.0]))[0] == orc.f32_to_bf16(np.float32(1.0 / (1.0 + math.exp(-1.0))))
    assert orc.swiglu(bf16([-2.0]), bf16([3.0]))[0] == orc.f32_to_bf16(
        np.float32(np.float32(-2.0 * np.float32(math.exp(-2.0) / (1 + math.exp(-2.0)))) * 3.0))


# ---- residual: device/qwen3-tp-batch32-kernels-v5/src/collective.rs:62-116 ----
def test_residual_one_rounding_and_zero_partial():
    for res in (0x0000, 0x8000, 0x3F80, 0xBF80, 0x0080, 0x7F00, 0xFF00):
        for part in (0.0, -0.0, 1.0, -1.0, 0.00390625, 0.01171875, float(np.finfo(np.float32).tiny)):
            s = np.float32(np.float32(0.0) + np.float32(part))
            exp = orc.f32_to_bf16(np.float32(s + orc.bf16_to_f32(np.array([res], np.uint16))[0]))
            assert orc.residual(np.array([part], np.float32), np.array([res], np.uint16))[0] == exp
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    fin = allb[(allb & 0x7F80) != 0x7F80]
    got = orc.residual(np.zeros(len(fin), np.float32), fin)
    exp = orc.f32_to_bf16(np.float32(0.0) + orc.bf16_to_f32(fin))
    assert np.array_equal(got, exp)


def test_residual_rejections():
    # The reference rejects a nonfinite partial ("nonfinite row-parallel
    # partial"), a nonfinite residual or sum ("nonfinite residual sum") and a
    # finite sum whose bf16 rounding overflows ("BF16 residual sum overflow"):
    # adapters/m1-engineering-execution-v1/src/tp_execution/collective.rs:44-66,
    # v5 collective.rs:5-20. Finite cases next to them pass.
    f32 = lambda b: np.array([b], np.uint32).view(np.float32)[0]  # noqa: E731
    cases = [
        (float("inf"), 0x3F80, True),          # nonfinite partial
        (float("nan"), 0x0000, True),
        (1.0, 0x7F80, True),                   # nonfinite residual
        (1.0, 0x7FC0, True),
        (f32(0x7F7FFFFF), 0x7F7F, True),       # sum overflows FP32
        (f32(0x7F7FFFFF), 0x0000, True),       # finite sum, bf16 rounding overflows to inf
        (f32(0x7F7F7FFF), 0x0000, False),      # largest sum that still rounds to a finite bf16
        (-f32(0x7F7F7FFF), 0x8000, False),
        (1.0, 0xBF80, False),                  # 1 + (-1) = 0
    ]
    parts = np.array([c[0] for c in cases], np.float32)
    res = np.array([c[1] for c in cases], np.uint16)
    out, rej = orc.residual(parts, res, with_rejections=True)
    assert rej.tolist() == [c[2] for c in cases]
    assert out[6] == 0x7F7F and out[7] == 0xFF7F and out[8] == 0x0000
    assert out[5] == 0x7F80  # still narrowed (RNE carries into the infinity)


# ---- argmax: device/qwen3-logits-v1/tests/reference.rs; v11 README.md:26-32 ----
def test_argmax_lowest_id_rule():
    x = np.zeros(151936, np.float32)
    x[[5, 9, 100]] = 2.0
    assert orc.argmax_f32(x)[0] == 5
    y = np.zeros(10, np.float32)
    y[0], y[3] = -0.0, 0.0
    assert orc.argmax_f32(y)[0] == 0  # +0/-0 tie: lowest id
    z = np.full(151936, -1.0, np.float32)
    z[-1] = 1.0
    assert orc.argmax_f32(z) == (151935, 2.0)
    z[7] = np.inf
    assert orc.argmax_f32(z)[0] is None
    assert orc.argmax_bf16(np.array([0x3F80, 0x4000, 0x4000, 0x3F80], np.uint16)) == 1
    assert orc.argmax_bf16(np.array([0x3F80, 0x7FC0], np.uint16)) is None


# ---- speculative helpers: crates/ferric-spec/src/speculation.rs:211-243; logits.rs:587 ----
def test_greedy_verification_vectors():
    assert orc.verify_greedy([3, 4, 5], [9, 4, 5, 6]) == (0, [9])
    assert orc.verify_greedy([3, 4, 5], [3, 4, 9, 6]) == (2, [3, 4, 9])
    assert orc.verify_greedy([3, 4, 5], [3, 4, 5, 6]) == (3, [3, 4, 5, 6])
    assert orc.verify_greedy([3, 4], [3, 4]) == 2  # IncorrectTargetChoiceCount
    assert orc.verify_greedy([], []) == 1  # MissingTargetBonus


def test_token_assembly_is_anchor_then_iteration_major_draft():
    anchors = [10, 20]
    draft = [1, 2, 3, 4, 5, 6]  # [k=3][s=2]
    assert list(orc.token_assembly(anchors, draft, 2, 3)) == [10, 1, 3, 5, 20, 2, 4, 6]


# ---- synthetic-input generator (include/ferric_synth.h) ----
def _py_splitmix64(x):
    M = (1 << 64) - 1
    x = (x + 0x9E3779B97F4A7C15) & M
    z = x
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
    return z ^ (z >> 31)


def test_synth_generator_pins():
    # SplitMix64's published output sequence from state 0 pins the mixer.
    assert orc.lib().orc_splitmix64(0) == 0xE220A8397B1DCDAF
    assert orc.lib().orc_splitmix64(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4
    # the whole sample path restated in Python integers
    seed, kind, layer = 77, 11, 3
    ts = _py_splitmix64(seed ^ _py_splitmix64((kind << 32) + layer + 1))
    assert orc.synth_tensor_seed(seed, kind, layer) == ts
    scale = orc.synth_scale(0.02)
    got = orc.synth(4096, ts, scale)
    for i in (0, 1, 17, 4095):
        h = _py_splitmix64((ts + i) & ((1 << 64) - 1))
        s = sum((h >> sh) & 0xFFFF for sh in (0, 16, 32, 48)) - 131070
        assert got[i] == orc.f32_to_bf16(np.float32(s) * np.float32(scale)), i
    vals = orc.bf16_to_f32(orc.synth(1 << 18, 12345, orc.synth_scale(0.02))).astype(np.float64)
    assert abs(vals.mean()) < 2e-4
    assert abs(vals.std() - 0.02) < 4e-4
    assert np.max(np.abs(vals)) <= 0.02 * 3.47
    assert orc.synth_scale(1.0) == np.float32(1.0 / 37837.2306413553)


# ---- the wave-order profiles (a second legal reduction order) ----------------
# device/qwen3-tp-batch32-kernels-v5/src/projection.rs:15-137 (GEMV lanes
# k = 64 s + l), device/qwen3-tp-wave-rmsnorm-kernels-v15/src/rmsnorm.rs:60-75
# (lane l: x[l + 64 c]^2), device/qwen3-tp-wave-query-hoist-kernels-v14/src/
# attention.rs:174-217 (lane l: q[l] k[l] + q[l+64] k[l+64]); the 64-lane
# reduction is the xor butterfly (fe2o3's own tree is not in the reference).
# Cancellation at 2^24 (where +1 is absorbed) makes each order visible.

def test_wave_gemm_known_answers():
    k = 128
    a = np.full(k, 0x3F80, np.uint16)  # ones
    w = np.zeros(k, np.uint16)
    w[0], w[64], w[1] = 0x4B80, 0xCB80, 0x3F80  # 2^24 and -2^24 in lane 0 (steps 0, 1), 1 in lane 1
    assert orc.gemm(a, w, 1, 1, k, f32_out=True)[0] == 0.0  # serial: 2^24 + 1 absorbs the 1
    assert orc.gemm_wave(a, w, 1, 1, k, f32_out=True)[0] == 1.0  # lane 0 cancels before lane 1 joins
    w = np.zeros(k, np.uint16)
    w[0], w[32], w[1] = 0x4B80, 0xCB80, 0x3F80  # lanes 0 and 32 meet first in the butterfly
    assert orc.gemm_wave(a, w, 1, 1, k, f32_out=True)[0] == 1.0
    w = np.zeros(k, np.uint16)
    w[0], w[1], w[2] = 0x4B80, 0xCB80, 0x3F80  # lanes 0 and 1 meet last: 2^24 + 1 absorbs first
    assert orc.gemm_wave(a, w, 1, 1, k, f32_out=True)[0] == 0.0
    # exact sums agree with the serial order bit for bit: the 2x3x4 KAT
    # (gemm reference.rs:137-153) zero-padded to k = 64
    A = np.zeros((2, 64), np.uint16)
    B = np.zeros((3, 64), np.uint16)
    A[:, :4] = [[0x3F80, 0x4000, 0x4040, 0x4080], [0xBF80, 0x3F00, 0x4000, 0xC000]]
    B[:, :4] = [[0x3F80, 0x0000, 0x3F80, 0x0000], [0x0000, 0x3F80, 0x0000, 0x3F80], [0x3F00, 0x3F00, 0x3F00, 0x3F00]]
    got = orc.gemm_wave(A.reshape(-1), B.reshape(-1), 2, 3, 64)
    assert got.tolist() == orc.gemm(A.reshape(-1), B.reshape(-1), 2, 3, 64).tolist()


def test_wave_square_sum_known_answer():
    # 4096^2 = 2^24 in lane 0 plus 127 ones: the serial sum absorbs every one
    # (2^24 + 1 rounds to even); in wave order lanes 1..63 first build 2, 4, ...
    # so the butterfly adds 2 + 4 + 8 + 16 + 32 + 64 = 126 exactly.
    x = np.full(128, 0x3F80, np.uint16)
    x[0] = 0x4580
    assert orc.square_sum(x) == 2.0 ** 24
    assert orc.square_sum_wave(x) == 2.0 ** 24 + 126
    # the normalize-and-weight step is the serial one: equal bits on a row
    # whose sum is exact in either order
    r = np.random.default_rng(3).integers(-8, 9, 1024).astype(np.float32)
    xb = orc.f32_to_bf16(r)
    w = np.full(1024, 0x3F80, np.uint16)
    assert np.array_equal(orc.rmsnorm_wave(xb, w, 1, 1024), orc.rmsnorm(xb, w, 1, 1024))


def test_exact_square_sum_norm_known_answer_and_closed_form():
    # The same row: serial order absorbs all 127 ones into 2^24 (sum 2^24),
    # wave order keeps 126 of them, the exact sum keeps 127 and rounds once
    # (2^24 + 127 is odd: FP32 keeps 2^24 + 128 by round-to-even of the ulp-2
    # grid). Each sum gives its own inverse RMS, so the three outputs differ.
    x = np.full(128, 0x3F80, np.uint16)
    x[0] = 0x4580
    w = np.full(128, 0x3F80, np.uint16)
    inv = {}
    for name, s in (("serial", 2.0 ** 24), ("wave", 2.0 ** 24 + 126), ("exact", 2.0 ** 24 + 128)):
        ms = np.float32(np.float32(s) / np.float32(128))
        inv[name] = np.float32(1.0) / np.float32(np.sqrt(np.float64(np.float32(ms + np.float32(1e-6)))))
    want = {k: orc.f32_to_bf16((np.float32(4096.0) * v).astype(np.float32)) for k, v in inv.items()}
    assert orc.rmsnorm_exact(x, w, 1, 128)[0] == want["exact"]
    assert orc.rmsnorm(x, w, 1, 128)[0] == want["serial"]
    assert orc.rmsnorm_wave(x, w, 1, 128)[0] == want["wave"]
    # Closed form on random rows: the FP32 squares summed with math.fsum and
    # rounded once, then the serial inverse and normalize-and-weight steps.
    r = np.random.default_rng(11)
    for width in (1024, 4096):
        xb = orc.f32_to_bf16((r.standard_normal(width) * 30).astype(np.float32))
        wb = orc.f32_to_bf16((r.standard_normal(width) + 1).astype(np.float32))
        f = (xb.astype(np.uint32) << 16).view(np.float32)
        total = np.float32(math.fsum(float(v) for v in (f * f).astype(np.float32)))
        ms = np.float32(total / np.float32(width))
        iv = np.float32(1.0) / np.float32(np.sqrt(np.float64(np.float32(ms + np.float32(1e-6)))))
        xn = orc.f32_to_bf16((f * iv).astype(np.float32))
        wf = (wb.astype(np.uint32) << 16).view(np.float32)
        ref = orc.f32_to_bf16(((xn.astype(np.uint32) << 16).view(np.float32) * wf).astype(np.float32))
        assert np.array_equal(orc.rmsnorm_exact(xb, wb, 1, width), ref), width


def test_wave_attention_score_known_answer():
    # Two keys; key 0's dot is 2^24 + 1 - 2^24 with the terms in dims 0, 1, 64:
    # serial order absorbs the 1 (score 0, the zero-score mean 0x3f00 of
    # paged-decode reference.rs:200-225), wave order cancels dims 0 and 64 in
    # lane 0 first (dot 1, score = f32(0x3db504f3)). V: key 0 ones, key 1 zeros,
    # so the output is 1 / (1 + e^-scale) = 0.5221 -> bf16 0x3f06.
    kvh, pages = 1, 1
    kc = np.zeros(pages * 16 * kvh * 128, np.uint16)
    vc = np.zeros_like(kc)
    q = np.zeros(128, np.uint16)
    q[0], q[1], q[64] = 0x4B80, 0x3F80, 0x4B80
    kc[0], kc[1], kc[64] = 0x3F80, 0x3F80, 0xBF80
    vc[:128] = 0x3F80
    table = np.array([0], np.uint32)
    serial = orc.attention_head(q, kc, vc, table, pages, 1, kvh, 0)
    wave = orc.attention_head_wave(q, kc, vc, table, pages, 1, kvh, 0)
    assert np.all(serial == 0x3F00)
    scale = float(np.array([0x3DB504F3], np.uint32).view(np.float32)[0])
    want = int(orc.f32_to_bf16(np.float32(1.0 / (1.0 + math.exp(-scale)))))
    assert want == 0x3F06 and np.all(wave == want)


def test_model_orders_differ_only_by_reassociation():
    # Two legal orders on a small model: every layer within the per-layer bar
    # of the other, greedy ids equal except at near-ties.
    cfg = dict(layers=2, hidden=256, query_heads=4, kv_heads=2, head_dim=128, intermediate=512, vocabulary=512,
               tied_embedding=1, rope_theta=1_000_000, rms_epsilon=1e-6)
    m = orc.Model(cfg, 16)
    try:
        m.synthesize(5, 0.02)
        toks, pos = [3, 7, 11], [0, 1, 2]
        tables = np.zeros((3, 2), np.uint32)
        counts = np.ones(3, np.uint32)
        a = m.forward(toks, pos, tables, counts, 2, want_hidden=True, order=1)
        b = m.forward(toks, pos, tables, counts, 2, want_hidden=True)
        assert not np.array_equal(a["logits"], b["logits"])  # the orders do differ
        assert float(np.max(np.abs(a["logits"] - b["logits"]))) < 1e-2
        for i, (ca, cb) in enumerate(zip(a["choices"], b["choices"])):
            assert ca == cb or b["gaps"][i] < 1e-2
    finally:
        m.close()


def test_split_context_attention_is_the_softmax():
    # The wave-order attention splits the keys into 8 partitions (v21) and
    # merges their states; both orders must be the softmax-weighted mean of V
    # (float64 closed form) to within a bf16 ulp of the output, for contexts
    # that leave empty, single-key and uneven partitions.
    r = np.random.default_rng(17)
    kvh, pages = 2, 8
    kc = orc.f32_to_bf16(r.standard_normal(pages * 16 * kvh * 128).astype(np.float32))
    vc = orc.f32_to_bf16(r.standard_normal(pages * 16 * kvh * 128).astype(np.float32))
    table = r.permutation(pages).astype(np.uint32)
    scale = float(np.array([0x3DB504F3], np.uint32).view(np.float32)[0])
    differ = 0
    for position in (0, 1, 6, 7, 8, 9, 30, 63, 64, 100, 127):
        for head in range(kvh):
            q = orc.f32_to_bf16((r.standard_normal(128) * 2).astype(np.float32))
            qf = orc.bf16_to_f32(q).astype(np.float64)
            k_rows, v_rows = [], []
            for t in range(position + 1):
                base = orc.cache_index(int(table[t // 16]), t % 16, kvh, head, 0)
                k_rows.append(orc.bf16_to_f32(kc[base:base + 128]).astype(np.float64))
                v_rows.append(orc.bf16_to_f32(vc[base:base + 128]).astype(np.float64))
            s = np.array([qf @ k for k in k_rows]) * scale
            w = np.exp(s - s.max())
            exact = (w[:, None] * np.array(v_rows)).sum(0) / w.sum()
            ulp = 2.0 ** (np.floor(np.log2(np.maximum(np.abs(exact), 1e-30))) - 7)
            serial = orc.attention_head(q, kc, vc, table, pages, position, kvh, head)
            split = orc.attention_head_wave(q, kc, vc, table, pages, position, kvh, head)
            for got in (serial, split):
                assert np.all(np.abs(orc.bf16_to_f32(got) - exact) <= ulp + 1e-6), (position, head)
            differ += int(not np.array_equal(serial, split))
    assert differ > 0  # the two orders are distinct arithmetic
