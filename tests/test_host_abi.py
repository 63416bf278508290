"""Host-side entry points of the C-ABI, checked on the CPU against the oracle
and the reference's stated rules: AffineWeights validation (order and
messages, AffineWeights.swift:84-157), rotary frequencies and tables
(DeepSeekV4Attention.swift:28-149, bit-exact) and the V4 index tables
(DeepSeekV4Attention.swift:169-237, bit-exact)."""
import ctypes as C

import numpy as np
import pytest

import minirun_hip as M
import oracle as O


def validate(pdt=M.U32, ps=(1536, 896), sdt=M.BF16, ss=(1536, 112), bdt=None, bs=None, group=64, bits=4):
    bdt = sdt if bdt is None else bdt
    bs = ss if bs is None else bs
    arr = lambda s: (C.c_int64 * len(s))(*s)
    ex, of, inf = C.c_int64(), C.c_int64(), C.c_int64()
    st = M.load().mr_affine_validate(pdt, len(ps), arr(ps), sdt, len(ss), arr(ss), bdt, len(bs), arr(bs), group, bits,
                                     C.byref(ex), C.byref(of), C.byref(inf))
    return st, M.last_error() if st else "", (ex.value, of.value, inf.value)


def test_affine_validate_accepts_config_shapes():
    for out, inp in [(1536, 7168), (24576, 1536), (576, 7168), (7168, 16384), (32768, 512)]:
        st, _, geo = validate(ps=(out, inp // 8), ss=(out, inp // 64))
        assert st == M.OK and geo == (0, out, inp)
    st, _, geo = validate(ps=(8, 64, 32), ss=(8, 64, 4))
    assert st == M.OK and geo == (8, 64, 256)


@pytest.mark.parametrize(
    "kw,status,needle",
    [
        (dict(pdt=M.F32), M.INVALID_DTYPE, "must be .uint32"),
        (dict(sdt=M.I32), M.INVALID_DTYPE, "must be a floating-point type"),
        (dict(sdt=M.BF16, bdt=M.F16), M.INVALID_DTYPE, "scales are bfloat16 but biases are float16"),
        (dict(bs=(1536, 111)), M.INVALID_SHAPE, "must have one shape"),
        (dict(ps=(1536,), ss=(1536,)), M.INVALID_SHAPE, "rank 2 (one matrix) or rank 3"),
        (dict(bits=3), M.INVALID_SHAPE, "bits 3 must divide 32"),
        (dict(group=0), M.INVALID_SHAPE, "group size must be positive"),
        (dict(ps=(4, 1536, 896), ss=(5, 1536, 112)), M.INVALID_SHAPE, "expert count differs: packed has 4, scales has 5"),
        (dict(ss=(1535, 112)), M.INVALID_SHAPE, "row count differs: packed has 1536, scales has 1535"),
        (dict(ps=(1536, 895)), M.INVALID_SHAPE, "inFeatures 7160 is not a multiple of the group size 64"),
        (dict(ss=(1536, 111)), M.INVALID_SHAPE, "group count differs: 7168 input features at group size 64 need 112"),
    ],
)
def test_affine_validate_errors_in_reference_order(kw, status, needle):
    st, msg, _ = validate(**kw)
    assert st == status and needle in msg, (st, msg)
    # the oracle's shape rules agree where they overlap
    if status == M.INVALID_SHAPE and set(kw) == {"ss"} and kw["ss"][0] == 1536:
        ost, _ = O.affine_validate(1536, 896, kw["ss"][1], kw.get("group", 64), kw.get("bits", 4))
        assert ost == O.INVALID_SHAPE


def test_validation_order_dtype_before_shape():
    # both the dtype and the shape are wrong: the dtype error is reported
    st, msg, _ = validate(sdt=M.BF16, bdt=M.F32, bs=(3, 3))
    assert st == M.INVALID_DTYPE


@pytest.mark.parametrize("dim,orig,base,factor", [(64, 0, 10000.0, 1.0), (64, 4096, 10000.0, 40.0),
                                                   (128, 65536, 50000.0, 16.0), (16, 0, 1e6, 1.0)])
def test_rope_frequencies_bit_exact(dim, orig, base, factor):
    a = M.rope_frequencies(dim, base=base, original_len=orig, factor=factor)
    b = O.rope_frequencies(dim, base=base, original_len=orig, factor=factor)
    np.testing.assert_array_equal(a, b)


def test_rope_table_bit_exact_and_errors():
    f = M.rope_frequencies(64)
    pos = np.array([0, 1, 2, 511, 32767, 131071, 1 << 20])
    for inv in (False, True):
        c1, s1 = M.rope_table(pos, f, inverse=inv)
        c2, s2 = O.rope_table(pos, f, inverse=inv)
        np.testing.assert_array_equal(c1, c2)
        np.testing.assert_array_equal(s1, s2)
    with pytest.raises(M.MRError) as e:
        M.rope_table([3, -1], f)
    assert "cannot be negative" in e.value.message
    with pytest.raises(M.MRError) as e:
        M.rope_frequencies(63)
    assert "positive and even" in e.value.message


@pytest.mark.parametrize("window,seq,start", [(4, 1, 5), (4, 1, 3), (4, 1, 2), (3, 5, 0), (128, 1, 130000),
                                              (128, 300, 0), (7, 1, 6), (1, 3, 0)])
def test_window_indices_bit_exact(window, seq, start):
    st, exp = O.window_indices(window, seq, start)
    assert st == O.OK
    np.testing.assert_array_equal(M.attention_indices_window(window, seq, start), exp)


@pytest.mark.parametrize("ratio,seq,start,off", [(4, 1, 9, 100), (4, 1, 2, 100), (2, 5, 0, 7), (128, 1, 131071, 128),
                                                 (4, 333, 0, 128), (1, 4, 0, 0)])
def test_compressed_indices_bit_exact(ratio, seq, start, off):
    st, exp = O.compressed_indices(ratio, seq, start, off)
    assert st == O.OK
    np.testing.assert_array_equal(M.attention_indices_compressed(ratio, seq, start, off), exp)


def test_index_table_errors():
    with pytest.raises(M.MRError) as e:
        M.attention_indices_window(4, 2, 1)
    assert "exactly one token" in e.value.message
    with pytest.raises(M.MRError) as e:
        M.attention_indices_compressed(0, 2, 0, 0)
    assert e.value.status == M.INVALID_SHAPE


@pytest.mark.parametrize("rows,cols,top_k,ratio,start,offset,needle", [
    (0, 4, 2, 1, 0, 0, "invalid lightning-index selection geometry"),
    (2, 4, 2, 0, 0, 0, "invalid lightning-index selection geometry"),
    (2, 4, 2, 1, 3, 0, "exactly one token"),
    (1, 2, 2, 1, 3, 0, "fewer compressed keys"),
    (1, 8, 5000, 1, 7, 0, None),
    (1, 8, 4, 1, 7, 2147483645, "overflows"),
])
def test_topk_geometry_errors(rows, cols, top_k, ratio, start, offset, needle):
    if needle is None:
        assert M.topk_geometry(rows, cols, top_k, ratio, start, offset) == 8
        return
    with pytest.raises(M.MRError) as e:
        M.topk_geometry(rows, cols, top_k, ratio, start, offset)
    assert needle in e.value.message, e.value.message
    # the oracle rejects the reference's own geometry errors alike
    if rows > 0 and "overflows" not in needle:
        st, _ = O.topk_select(np.zeros((rows, cols), np.float32), top_k, ratio, start, offset)
        assert st == O.INVALID_SHAPE


def test_topk_geometry_counts():
    assert M.topk_geometry(1, 32768, 2048, 4, 131071, 0) == 2048
    assert M.topk_geometry(1, 262144, 2048, 4, 1048575, 0) == 2048   # V4 at 1M positions: no key limit
    assert M.topk_geometry(300, 75, 16, 4, 0, 128) == 16
    assert M.topk_geometry(3, 4, 16, 4, 0, 0) == 0   # fewer than ratio tokens: empty rows
    # any top_k, as `selecting` takes any (DeepSeekV4Attention.swift:582-645)
    assert M.topk_geometry(1, 8192, 5000, 1, 8191, 0) == 5000
    assert M.topk_geometry(1, 262144, 100000, 4, 1048575, 0) == 100000


def test_topk_workspace_covers_large_selections():
    # more than 4096 selected keys: slices of 4096 and merge rounds whose
    # lists double up to top_k; the size grows with top_k and covers what
    # the small-k paths need for the same rows and columns
    L = M.load()
    small = L.mr_topk_workspace_size(1, 262144, 4096)
    big = L.mr_topk_workspace_size(1, 262144, 16384)
    assert big > small > 0
    assert L.mr_topk_workspace_size(1, 262144, 16384) <= L.mr_topk_workspace_size(1, 262144, 262144)
    # 64 slices of 4096: the first round holds 64 lists of 4096 composites
    assert big >= 2 * 64 * 4096 * 8
    assert L.mr_topk_workspace_size(5000, 5000, 4500) >= 2 * 5000 * 2 * 4096 * 8


# ---------------------------------------------------------------- lightning-index scores
def _scores_call(seq, heads, dim, n_keys, key_dim, w_rows, w_cols, qdt=M.BF16):
    """Geometry-only calls: every case below returns before any launch."""
    return M.load().mr_indexer_scores(None, qdt, seq, heads, dim, heads * dim, dim, None, M.BF16, n_keys, key_dim,
                                      key_dim, None, M.F32, w_rows, w_cols, w_cols, None, n_keys, None)


@pytest.mark.parametrize("args", [
    (0, 4, 8, 5, 8, 0, 4),     # empty sequence
    (2, 0, 8, 5, 8, 2, 0),     # no heads
    (2, 4, 0, 5, 0, 2, 4),     # zero dimension
    (2, 4, 8, 5, 16, 2, 4),    # key dimension differs from the queries'
    (2, 4, 8, 5, 8, 1, 4),     # weights not [seq, heads]
    (2, 4, 8, 5, 8, 2, 5),
])
def test_indexer_scores_geometry_errors(args):
    """DeepSeekV4Attention.swift:533-541: one error for every geometry
    mismatch, raised before any work."""
    st = _scores_call(*args)
    assert st == O.INVALID_SHAPE
    assert "incompatible geometry" in M.last_error()


def test_indexer_scores_no_keys_and_dtypes():
    # no compressed keys: nothing to compute (:542-544), not an error
    assert _scores_call(2, 4, 8, 0, 8, 2, 4) == 0
    st = _scores_call(2, 4, 8, 0, 8, 2, 4, qdt=M.F16)
    assert st == O.INVALID_DTYPE and "bf16 or f32" in M.last_error()


# ---------------------------------------------------------------- routed experts
def test_affine_gather_preconditions():
    """AffineWeights.swift:290-298: the reference traps on a single matrix and
    on indices that do not match the token count; the ABI returns those
    messages as MR_INVALID_ARGUMENT before any work."""
    w = M.AffineWeightDesc(256, 256, 256, M.BF16, 8, 64, 64, 4)  # dummy aligned pointers: never dereferenced
    st = M.load().mr_affine_gather_matmul(None, M.BF16, 1, 64, C.byref(w), 0, None, 1, None, M.BF16, None)
    assert st == M.INVALID_ARGUMENT and "needs a stacked AffineWeights" in M.last_error()
    st = M.load().mr_affine_gather_matmul(None, M.BF16, 1, 64, C.byref(w), 4, None, 0, None, M.BF16, None)
    assert st == M.INVALID_ARGUMENT and "rhsIndices must be [tokens, expertsPerToken]" in M.last_error()
    # no tokens: nothing to do
    assert M.load().mr_affine_gather_matmul(None, M.BF16, 0, 64, C.byref(w), 4, None, 2, None, M.BF16, None) == 0


# ---------------------------------------------------------------- StorageCore tile hand-off
def test_affine_tile_view_layout_and_errors():
    """QuantizedTileContainer.swift:560-620 (affine, one scale row per row):
    [packed | scales | biases], each a whole number of 16 KiB."""
    base = 1 << 20  # never dereferenced
    d, n = M.affine_tile_view(base, 512, 1024)
    assert (d.packed, d.scales, d.biases) == (base, base + 262144, base + 262144 + 16384)
    assert (d.out_features, d.in_features, d.group, d.bits, n) == (512, 1024, 64, 4, 262144 + 2 * 16384)
    d, n = M.affine_tile_view(base, 256, 1024, scale_dtype=M.F32)  # f32 scales: 16 KiB from 256 rows
    assert d.scales == base + 131072 and n == 131072 + 2 * 16384
    for args, needle in [((512, 1000), "multiple of the group size"),
                         ((16, 1024), "packed bytes per tile (8192) must be a multiple of 16384"),
                         ((256, 1024), "scale bytes per tile (8192) must be a multiple of 16384")]:
        with pytest.raises(M.MRError) as e:
            M.affine_tile_view(base, *args)
        assert needle in e.value.message, e.value.message
    with pytest.raises(M.MRError):
        M.affine_tile_view(base, 512, 1024, scale_dtype=M.U32)
