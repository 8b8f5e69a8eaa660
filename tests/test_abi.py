"""The C ABI boundary on any host: libferric_hip.so loads, exports every
function include/ferric_hip.h declares with the binding's signature, and its
host-only entry points (speculative helpers, scratch sizing, argument
validation) behave like the reference. No GPU calls are made here."""

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

import ferric_amd
from ferric_amd import _lib
from ferric_amd.pool import PagePool
from ferric_amd.runner import PagedLimits
from oracle import oracle as orc

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "ferric_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(fh_[a-z_0-9]+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_every_declared_symbol_is_exported_and_bound():
    lib = ferric_amd.load()
    names = declared_functions()
    assert len(names) >= 30
    bound = {n for n, _, _ in _lib.SIGNATURES}
    for n in names:
        assert hasattr(lib, n), f"{n} not exported by libferric_hip.so"
        assert n in bound, f"{n} has no ctypes signature in ferric_amd/_lib.py"
    assert bound <= set(names), f"binding names a function the header does not declare: {bound - set(names)}"


def test_struct_layouts_match_the_header():
    # Field counts and widths of the boundary structs.
    assert ctypes.sizeof(_lib.ModelDesc) == 10 * 4
    assert ctypes.sizeof(_lib.CtxOptions) == 8 * 4
    assert _lib.Row.pages.offset == 16 and ctypes.sizeof(_lib.Row) == 32
    from ferric_amd.runner import ROW_DTYPE
    assert ROW_DTYPE.itemsize == ctypes.sizeof(_lib.Row)
    for name, _ in _lib.Row._fields_:
        assert ROW_DTYPE.fields[name][1] == getattr(_lib.Row, name).offset, name


def u32(a):
    return (ctypes.c_uint32 * len(a))(*a)


def test_verify_greedy_round_matches_the_reference_vectors():
    lib = ferric_amd.load()
    for draft, target, acc, emitted in [([3, 4, 5], [9, 4, 5, 6], 0, [9]), ([3, 4, 5], [3, 4, 9, 6], 2, [3, 4, 9]),
                                        ([3, 4, 5], [3, 4, 5, 6], 3, [3, 4, 5, 6])]:
        a = ctypes.c_uint32()
        e = (ctypes.c_uint32 * 8)()
        n = ctypes.c_uint32()
        st = lib.fh_verify_greedy_round(u32(draft), len(draft), u32(target), len(target), ctypes.byref(a), e,
                                        ctypes.byref(n))
        assert st == 0 and a.value == acc and list(e[: n.value]) == emitted
        assert (acc, emitted) == orc.verify_greedy(draft, target)
    a, e, n = ctypes.c_uint32(), (ctypes.c_uint32 * 8)(), ctypes.c_uint32()
    assert lib.fh_verify_greedy_round(u32([3, 4]), 2, u32([3, 4]), 2, ctypes.byref(a), e, ctypes.byref(n)) == 1
    assert lib.fh_verify_greedy_round(None, 0, None, 0, ctypes.byref(a), e, ctypes.byref(n)) == 1


def test_verify_greedy_batch_settles_each_sequence_like_the_single_call():
    # Every sequence of a round in one call (draft iteration-major [K][S],
    # target [S][K + 1]) against the oracle's per-sequence verify: random
    # rounds over a 3-token alphabet (every acceptance count occurs), K = 0,
    # and the three reference vectors as one round.
    from ferric_amd.speculative import verify_greedy_batch
    lib = ferric_amd.load()
    r = np.random.default_rng(9)
    cases = [(r.integers(0, 3, (k, s)), r.integers(0, 3, (s, k + 1))) for k, s in [(4, 32), (1, 5), (7, 3), (0, 4)]]
    cases.append((np.array([[3, 3, 3], [4, 4, 4], [5, 5, 5]]), np.array([[9, 4, 5, 6], [3, 4, 9, 6], [3, 4, 5, 6]])))
    for draft, target in cases:
        acc, ems = verify_greedy_batch(draft, target)
        for s in range(target.shape[0]):
            want_a, want_e = orc.verify_greedy([int(x) for x in draft[:, s]], [int(x) for x in target[s]])
            assert int(acc[s]) == want_a and [int(x) for x in ems[s, : want_a + 1]] == want_e, (s, draft, target)
    e, acc = (ctypes.c_uint32 * 8)(), (ctypes.c_uint32 * 2)()
    assert lib.fh_verify_greedy_batch(None, u32([1, 2]), 2, 0, acc, e) == 0  # K = 0: the bonus token only
    assert list(e[:2]) == [1, 2] and list(acc) == [0, 0]
    assert lib.fh_verify_greedy_batch(None, u32([1, 2, 3, 4]), 2, 1, acc, e) == 1  # draft missing
    assert lib.fh_verify_greedy_batch(None, None, 0, 4, None, None) == 0  # no sequences


def test_token_assembly_matches_the_oracle():
    lib = ferric_amd.load()
    r = np.random.default_rng(0)
    for s, k in [(1, 4), (8, 4), (32, 4), (3, 0)]:
        anchors = r.integers(0, 151936, s).tolist()
        draft = r.integers(0, 151936, s * k).tolist()
        out = (ctypes.c_uint32 * (s * (k + 1)))()
        assert lib.fh_speculative_token_assembly(u32(anchors), u32(draft) if k else None, s, k, out) == 0
        assert list(out) == orc.token_assembly(anchors, draft if k else [0], s, k).tolist()


def test_scratch_sizes():
    lib = ferric_amd.load()
    # 32 rows x 32 heads x ceil(8320 / 512) partitions x (2 + 128) f32
    assert lib.fh_attention_scratch_bytes(32, 32, 8320) == 32 * 32 * 17 * 130 * 4
    assert lib.fh_argmax_scratch_bytes(32) == 32 * 64 * 8
    # split-K factors keep about 256 workgroups per projection launch
    assert lib.fh_gemm_default_splits(4096, 4096) == 4  # o
    assert lib.fh_gemm_default_splits(6144, 4096) == 2  # packed qkv
    assert lib.fh_gemm_default_splits(4096, 12288) == 4  # down
    assert lib.fh_gemm_default_splits(24576, 4096) == 1  # gate/up
    assert lib.fh_gemm_default_splits(151936, 4096) == 1  # LM head
    assert lib.fh_gemm_default_splits(1024, 2048) == 4  # capped at 16 k-blocks per split


def test_ops_reject_bad_shapes_before_any_launch():
    lib = ferric_amd.load()
    p = ctypes.c_void_p(16)  # never dereferenced: validation fails first
    assert lib.fh_op_gemm(p, p, 0, 64, 64, 0, 1, None, p, 64, None, None) == 1  # m = 0
    assert lib.fh_op_gemm(p, p, 33, 64, 64, 0, 1, None, p, 64, None, None) == 1  # m > 32 needs n % 128
    assert lib.fh_op_gemm(p, p, 257, 128, 64, 4, 1, None, p, 128, None, None) == 1  # partials above 256 rows
    assert lib.fh_op_gemm(p, p, 33, 128, 64, 4, 1, None, p, 130, None, None) == 1  # partials: 16-byte aligned rows
    assert lib.fh_op_gemm(p, p, 33, 128, 64, 0, 1, None, p, 130, None, None) == 1  # m > 32: 8-byte aligned rows
    assert lib.fh_op_gemm(p, p, 4, 60, 64, 0, 1, None, p, 64, None, None) == 1  # n % 16
    assert lib.fh_op_gemm(p, p, 4, 64, 48, 0, 1, None, p, 64, None, None) == 1  # k % 32
    assert lib.fh_op_gemm(p, p, 4, 64, 64, 1, 1, None, p, 64, None, None) == 1  # residual epilogue without residual
    assert lib.fh_op_gemm(p, p, 4, 64, 64, 9, 1, None, p, 64, None, None) == 1  # unknown epilogue
    assert lib.fh_op_gemm(p, p, 4, 64, 64, 0, 2, None, p, 64, None, None) == 1  # splits on a non-partial epilogue
    assert lib.fh_op_gemm(p, p, 4, 64, 64, 4, 3, None, p, 64, None, None) == 1  # more splits than k-blocks
    assert lib.fh_op_tile_weight(p, p, 17, 32, None) == 1
    assert lib.fh_op_tile_activation(p, p, 33, 48, None) == 1  # k % 32
    assert lib.fh_activation_rows(1) == 32 and lib.fh_activation_rows(32) == 32
    assert lib.fh_activation_rows(33) == 256 and lib.fh_activation_rows(257) == 512
    # split-K partial slabs: 32 rows for decode batches, 256 for wide ones, none beyond
    assert [lib.fh_partial_slab_rows(m) for m in (0, 1, 32, 33, 256, 257)] == [0, 32, 32, 256, 256, 0]
    # one-row projections with the norm in their prologue: the Qwen3 shapes only
    E = ferric_amd._lib
    covered = [(6144, 4096, E.EPI_PARTIAL, 2, 0), (6144, 4096, E.EPI_PARTIAL, 2, 4), (24576, 4096, E.EPI_SWIGLU, 1, 4),
               (151936, 4096, E.EPI_F32, 1, 4), (4096, 1024, E.EPI_PARTIAL, 2, 6), (6144, 1024, E.EPI_SWIGLU, 1, 4),
               (151936, 1024, E.EPI_F32, 1, 6)]
    assert all(lib.fh_gemm_rmsnorm_supported(*c) == 1 for c in covered)
    assert lib.fh_gemm_rmsnorm_supported(6144, 4096, E.EPI_PARTIAL, 2, 3) == 0  # slab count
    assert lib.fh_gemm_rmsnorm_supported(4096, 4096, E.EPI_PARTIAL, 4, 4) == 0  # the O projection's tiles
    assert lib.fh_gemm_rmsnorm_supported(6144, 8192, E.EPI_PARTIAL, 2, 4) == 0  # width
    assert lib.fh_gemm_rmsnorm_supported(6144, 4096, E.EPI_BF16, 1, 4) == 0  # epilogue
    rn = lambda h_in, h_out, part, ns, n=6144, k=4096, epi=E.EPI_PARTIAL, splits=2: lib.fh_op_gemm_rmsnorm(  # noqa: E731
        h_in, h_out, part, ns, p, 1e-6, p, n, k, epi, splits, p, n, None, None)
    q = ctypes.c_void_p(32)
    assert rn(p, p, q, 4) == 1  # the folded row would overwrite the row being read
    assert rn(p, q, None, 4) == 1  # slabs missing
    assert rn(p, None, q, 4) == 1  # no output row
    assert rn(p, q, q, 3) == 1 and rn(p, q, q, 4, n=4096, splits=4) == 1  # not covered
    ms = ctypes.c_float()
    assert lib.fh_time_attention(None, 1, ctypes.byref(ms)) == 1  # no context
    assert lib.fh_op_rmsnorm(p, p, p, 1, 8200, 1e-6, None, None) == 1
    assert lib.fh_op_residual_rmsnorm(p, None, 2, p, p, 1, 4, 4096, 1e-6, None, None) == 1  # partials missing
    assert lib.fh_op_residual_rmsnorm(p, p, 2, p, p, 1, 257, 4096, 1e-6, None, None) == 1  # partials above 256 rows
    assert lib.fh_op_paged_attention(p, p, p, p, p, p, 0, p, 1, 32, 6, 4, 4, 64, None, None) == 1  # 32 % 6
    assert lib.fh_op_paged_attention(p, p, p, p, p, p, 0, p, 1, 32, 8, 4, 4, 65, None, None) == 1  # stride*16 < ctx
    # fused QK-norm + attention: 2 slabs, at most 4 query heads per KV head, at most 32 rows
    qkn = lambda splits, rows, qh: lib.fh_op_qknorm_paged_attention(  # noqa: E731
        p, splits, p, p, p, p, p, p, p, p, p, 1, p, rows, qh, 8, 64, 64, 1024, 1e-6, None, None)
    assert qkn(3, 4, 32) == 1 and qkn(1, 4, 32) == 1  # slab count
    assert qkn(2, 4, 64) == 1  # 8 query heads per KV head
    assert qkn(2, 33, 32) == 1 and qkn(2, 0, 32) == 1  # rows


def test_create_rejects_unsupported_shapes_without_touching_the_device():
    lib = ferric_amd.load()
    desc = _lib.ModelDesc(2, 1024, 16, 8, 64, 3072, 151936, 1, 1_000_000, 1e-6)  # head_dim 64
    opts = _lib.CtxOptions(8, 64, 32, 512, 0, 0, 0, 0)
    ctx = ctypes.c_void_p()
    assert lib.fh_create(ctypes.byref(desc), ctypes.byref(opts), ctypes.byref(ctx)) == 1
    assert b"unsupported model shape" in lib.fh_last_error(None)
    desc = _lib.ModelDesc(2, 1024, 16, 8, 128, 3072, 151936, 1, 1_000_000, 1e-6)
    opts = _lib.CtxOptions(33, 64, 32, 512, 0, 0, 0, 0)  # more rows than the 32-row envelope
    assert lib.fh_create(ctypes.byref(desc), ctypes.byref(opts), ctypes.byref(ctx)) == 1
    opts = _lib.CtxOptions(8, 64, 16, 512, 0, 0, 0, 0)  # stride * 16 < context
    assert lib.fh_create(ctypes.byref(desc), ctypes.byref(opts), ctypes.byref(ctx)) == 1


def test_page_pool_reserves_write_slots_and_consecutive_positions():
    limits = PagedLimits(context_tokens=128, physical_page_count=20, page_table_stride=8)
    pool = PagePool(limits, seed=3)
    a = pool.admit(15)
    b = pool.admit(0)
    batch = pool.prepare([(a, 7), (a, 8), (b, 9)])
    rows = batch.rows
    assert [r.position for r in rows] == [15, 16, 0]
    assert list(rows[0].physical_pages) == list(rows[1].physical_pages) and len(rows[0].physical_pages) == 2
    assert rows[0].writable_physical_page == rows[0].physical_pages[0]
    assert rows[1].writable_physical_page == rows[1].physical_pages[1]
    assert rows[1].writable_token_offset == 0
    pool.commit(batch)
    assert pool.sequences[a].length == 17 and pool.sequences[b].length == 1
    all_pages = [p for s in pool.sequences.values() for p in s.pages]
    assert len(all_pages) == len(set(all_pages))
    with pytest.raises(ValueError):
        pool.prepare([(a, 1)] * 120)


def test_page_pool_large_batch_matches_row_loop():
    # Batches above 256 rows are prepared with array operations; they must
    # give the same positions, page lists, write slots and page-allocation
    # order as the row-by-row path, for interleaved sequences with prefixes.
    from ferric_amd.runner import PreparedRows

    limits = PagedLimits(context_tokens=1024, physical_page_count=400, page_table_stride=64)

    def build():
        pool = PagePool(limits, seed=11)
        sids = [pool.admit(n) for n in (0, 15, 16, 33, 300)]
        rng = np.random.default_rng(5)
        rows = [(sids[i], int(t)) for i, t in zip(rng.integers(0, 5, 600), rng.integers(0, 151936, 600))]
        return pool, rows

    # A decode step (every row a different sequence) takes the per-column path,
    # which reuses the previous decode batch's page-list block while the
    # sequences and their page counts are unchanged: 40 steps in a row (page
    # boundaries crossed, a sequence released and another admitted) against
    # the row loop on a twin pool.
    for pick in ([0, 1, 2, 3, 4], [4, 2, 0, 3, 1]):
        pool_a, _ = build()
        pool_b, _ = build()
        sa, sb = sorted(pool_a.sequences), sorted(pool_b.sequences)
        for step in range(40):
            if step == 20:
                pool_a.release(sa[pick[1]])
                pool_b.release(sb[pick[1]])
                sa[pick[1]], sb[pick[1]] = pool_a.admit(3), pool_b.admit(3)
            ba = pool_a._prepare_decode([(sa[i], 100 + step + i) for i in pick])
            states, sid, token, pos, group = pool_b._prepare_loop([(sb[i], 100 + step + i) for i in pick])
            rows = ba.rows
            np.testing.assert_array_equal(rows.token, token)
            np.testing.assert_array_equal(rows.position, pos)
            for i, r in enumerate(rows):
                np.testing.assert_array_equal(r.physical_pages, states[group[i]].pages)
                assert r.writable_physical_page == r.physical_pages[r.position // 16]
                assert not r.physical_pages.flags.writeable
            assert pool_a.free == pool_b.free
            pool_a.commit(ba)
            for s, p in zip(sid.tolist(), pos.tolist()):
                pool_b.sequences[s].length = p + 1
    pool_a, _ = build()
    assert pool_a._prepare_decode([(1, 5), (2, 6), (1, 7)]) is None  # a repeated sequence
    pool_a, rows = build()
    pool_b, _ = build()
    cols_a = pool_a._prepare_vector(rows)
    cols_b = pool_b._prepare_loop(rows)
    assert [st.sequence for st in cols_a[0]] == [st.sequence for st in cols_b[0]]
    for x, y in zip(cols_a[1:], cols_b[1:]):
        np.testing.assert_array_equal(x, y)
    assert pool_a.free == pool_b.free
    for s in pool_a.sequences:
        np.testing.assert_array_equal(pool_a.sequences[s].pages, pool_b.sequences[s].pages)
    batch = pool_a.prepare(rows[:400])
    assert isinstance(batch.rows, PreparedRows) and len(batch.rows) == 400
    r = batch.rows[-1]
    assert r.writable_physical_page == r.physical_pages[r.position // 16]
    assert not r.physical_pages.flags.writeable
    with pytest.raises(ValueError):
        pool_a.prepare([(rows[0][0], -1)] * 300)


def test_page_pool_small_batches_match_the_general_path():
    # Up to 4 rows are prepared and marshalled on a short path (a batch-1
    # decode step runs it every step); it must give the columns, page lists,
    # allocations and fh_row records of the general path.
    import ctypes

    from ferric_amd.runner import _rows_to_c

    limits = PagedLimits(context_tokens=1024, physical_page_count=200, page_table_stride=64)

    def build():
        pool = PagePool(limits, seed=5)
        return pool, [pool.admit(n) for n in (0, 15, 16, 47, 300)]

    for rows_of in ([(0, 7)], [(1, 9)], [(4, 3), (4, 4)], [(2, 1), (1, 2), (2, 3), (0, 4)], [(3, 8), (3, 9)]):
        pool_a, sa = build()
        pool_b, sb = build()
        rows_a = [(sa[i], t) for i, t in rows_of]
        rows_b = [(sb[i], t) for i, t in rows_of]
        small = pool_a.prepare(rows_a).rows
        states, sid, token, pos, group = pool_b._prepare_loop(rows_b)
        assert pool_a.free == pool_b.free
        for s_a, s_b in zip(sa, sb):
            np.testing.assert_array_equal(pool_a.sequences[s_a].pages, pool_b.sequences[s_b].pages)
        np.testing.assert_array_equal(small.token, token)
        np.testing.assert_array_equal(small.position, pos)
        np.testing.assert_array_equal(small.table_index, group)
        assert small.token.dtype == np.uint32 and small.sequence.dtype == np.uint64
        for i, r in enumerate(small):
            np.testing.assert_array_equal(r.physical_pages, states[group[i]].pages)
            assert r.writable_physical_page == r.physical_pages[r.position // 16]
            assert not r.physical_pages.flags.writeable
        ptr, keep = _rows_to_c(small)
        for i, r in enumerate(small):
            c = ptr[i]
            assert (c.sequence, c.token, c.position, c.page_count, c.writable_page) == (
                r.sequence, r.token, r.position, len(r.physical_pages), r.writable_physical_page)
            assert list(c.pages[: c.page_count]) == list(r.physical_pages)
            assert ctypes.addressof(c.pages.contents) == r.physical_pages.__array_interface__["data"][0]
    pool, s = build()
    with pytest.raises(ValueError):
        pool.prepare([(s[0], -1)])
    with pytest.raises(ValueError):
        pool.prepare([(s[0], 1 << 32)])


def test_library_shares_torch_hip_runtime():
    # Importing the package before torch must still leave one HIP runtime in
    # the process (two copies disagree about which devices exist).
    import subprocess
    import sys

    code = ("import ferric_amd, torch\n"
            "maps = open('/proc/self/maps').read().splitlines()\n"
            "print(len({l.split()[-1] for l in maps if 'libamdhip64' in l}))\n")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, cwd=ROOT, timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.strip() == "1"
