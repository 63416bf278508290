"""Argument checks of the C-ABI under random arguments (hypothesis), on the
host: the attention entry points, the projections (affine, gathered, dense),
RMSNorm, rotary, cache append, absorption, un-absorption, index checks and
the top-k selection.  With every device buffer NULL no call reaches a GPU
call, so each must come back with a status (never a crash, never MR_OK
with work left undone) and, when refused, with a message; the
workspace-size functions never wrap (0 for widths a call rejects, else a
size below 2^56).  Shapes range over zero, negative and very large values,
scales over non-finite ones.

The host-side tables (window and compressed attention indices, the top-k
selection geometry) are compared with the oracle's restatement of the
reference over random arguments: the same status, and on success the same
table (bit for bit) or the same selected-key count."""
import ctypes as C
import os

import pytest
from hypothesis import HealthCheck, given, settings
from hypothesis import strategies as st

import minirun_hip as M
import numpy as np
import oracle as O

REFUSED = {M.INVALID_SHAPE, M.INVALID_ARGUMENT, M.INVALID_DTYPE, M.WORKSPACE_TOO_SMALL}
# derandomized: the same examples on every run (a longer search:
# MR_FUZZ_EXAMPLES=5000 MR_FUZZ_RANDOM=1)
SETTINGS = settings(max_examples=int(os.environ.get("MR_FUZZ_EXAMPLES", "300")), deadline=None,
                    derandomize=not os.environ.get("MR_FUZZ_RANDOM"),
                    suppress_health_check=[HealthCheck.too_slow])

dim = st.one_of(st.integers(-5, 4200), st.sampled_from([0, 1, 16, 64, 96, 128, 512, 576, 2 ** 31 - 1, -2 ** 31]))
big = st.one_of(st.integers(-3, 300000), st.sampled_from([0, 1, 32768, 131072, 2 ** 31 - 1, -2 ** 31]))
stride = st.one_of(st.integers(-10, 5000), st.sampled_from([0, 576, 2 ** 40, -(2 ** 40)]))
scale = st.one_of(st.floats(allow_nan=True, allow_infinity=True, width=32), st.sampled_from([0.0722, -1.0, 0.0]))


@pytest.fixture(scope="module")
def lib():
    return M.load()


def refused(status):
    assert status in REFUSED, status
    assert M.last_error(), "a refused call leaves a message"


@SETTINGS
@given(batch=dim, heads=dim, n_ctx=big, kv_rank=dim, rope=dim, sc=scale, ls=stride, out_dtype=st.integers(-1, 6),
       n_idx=big, flags=st.integers(0, 15), gathered=st.booleans(), splits=big)
def test_decode_checks(lib, batch, heads, n_ctx, kv_rank, rope, sc, ls, out_dtype, n_idx, flags, gathered, splits):
    a = M.DecodeArgs()
    a.batch, a.heads, a.n_ctx, a.kv_rank, a.rope_dim, a.scale = batch, heads, n_ctx, kv_rank, rope, sc
    a.latent_row_stride = a.rope_row_stride = ls
    a.q_lat_head_stride = a.q_rope_head_stride = a.out_head_stride = ls
    a.out_dtype, a.n_idx, a.flags, a.num_splits = out_dtype, n_idx, flags, splits
    if gathered:
        # a placeholder address: the NULL queries are refused before any
        # pointer is read, and the size functions read none
        a.indices = C.c_void_p(256)
    size = lib.mr_mla_decode_workspace_size(C.byref(a))
    assert 0 <= size < 2 ** 56
    if batch <= 0 or heads <= 0 or n_ctx <= 0 or (gathered and n_idx < 0):
        assert size == 0
    for entry in (lib.mr_mla_decode, lib.mr_mla_decode_noalloc):
        refused(entry(C.byref(a), None))


@SETTINGS
@given(tokens=dim, n_ctx=big, heads=dim, nope=dim, rope=dim, v=dim, kv_rank=dim, sc=scale, qs=stride,
       out_dtype=st.integers(-1, 6))
def test_prefill_checks(lib, tokens, n_ctx, heads, nope, rope, v, kv_rank, sc, qs, out_dtype):
    a = M.PrefillArgs()
    a.tokens, a.n_ctx, a.heads = tokens, n_ctx, heads
    a.qk_nope_dim, a.qk_rope_dim, a.v_head_dim, a.kv_rank = nope, rope, v, kv_rank
    a.scale = sc
    a.q_token_stride = a.q_head_stride = a.latent_row_stride = a.rope_row_stride = qs
    a.kv_b_row_stride = a.out_token_stride = a.out_head_stride = qs
    a.out_dtype = out_dtype
    size = lib.mr_mla_prefill_workspace_size(C.byref(a))
    assert 0 <= size < 2 ** 56
    refused(lib.mr_mla_prefill(C.byref(a), None))


def _block_dims(a, hidden, q_lora, heads, nope, rope, v, kv_rank):
    a.hidden, a.q_lora_rank, a.heads = hidden, q_lora, heads
    a.qk_nope_dim, a.qk_rope_dim, a.v_head_dim, a.kv_rank = nope, rope, v, kv_rank


@SETTINGS
@given(hidden=dim, q_lora=dim, heads=dim, nope=dim, rope=dim, v=dim, kv_rank=dim, position=big, capacity=big,
       eps=scale, nd=st.integers(-1, 6))
def test_decode_block_checks(lib, hidden, q_lora, heads, nope, rope, v, kv_rank, position, capacity, eps, nd):
    a = M.BlockArgs()
    _block_dims(a, hidden, q_lora, heads, nope, rope, v, kv_rank)
    a.eps = eps
    a.position, a.capacity = position, capacity
    a.norm_w_dtype = nd
    size = lib.mr_mla_decode_block_workspace_size(C.byref(a))
    assert 0 <= size < 2 ** 56
    if min(hidden, q_lora, heads, v, kv_rank) <= 0 or min(nope, rope) < 0 or position < 0:
        assert size == 0
    refused(lib.mr_mla_decode_block(C.byref(a), None))


@SETTINGS
@given(tokens=dim, hidden=dim, q_lora=dim, heads=dim, nope=dim, rope=dim, v=dim, kv_rank=dim, position=big,
       capacity=big, eps=scale, xs=stride)
def test_prefill_block_checks(lib, tokens, hidden, q_lora, heads, nope, rope, v, kv_rank, position, capacity, eps, xs):
    a = M.PrefillBlockArgs()
    a.tokens = tokens
    _block_dims(a, hidden, q_lora, heads, nope, rope, v, kv_rank)
    a.eps = eps
    a.position, a.capacity = position, capacity
    a.x_token_stride = a.out_token_stride = a.latent_row_stride = a.rope_row_stride = xs
    size = lib.mr_mla_prefill_block_workspace_size(C.byref(a))
    assert 0 <= size < 2 ** 56
    if min(tokens, hidden, q_lora, heads, v, kv_rank) <= 0 or min(nope, rope) < 0 or position < 0:
        assert size == 0
    refused(lib.mr_mla_prefill_block(C.byref(a), None))


@SETTINGS
@given(batch=dim, n_idx=big, n_rows=big)
def test_validate_indices_checks(lib, batch, n_idx, n_rows):
    size = lib.mr_validate_indices_workspace_size(batch, n_idx)
    assert 0 <= size < 2 ** 56
    if batch <= 0 or n_idx < 0:
        assert size == 0
    tok, pos = C.c_int32(7), C.c_int32(7)
    status = lib.mr_validate_indices(None, batch, n_idx, n_rows, None, 0, C.byref(tok), C.byref(pos), None)
    assert tok.value == -1 and pos.value == -1
    if status != M.OK:  # no entries is the one case with nothing to check
        refused(status)
    else:
        assert n_idx == 0 and batch > 0 and n_rows >= 0


@SETTINGS
@given(rows=dim, cols=big, top_k=big, ratio=st.integers(-2, 300), start=big, offset=big)
def test_topk_geometry(lib, rows, cols, top_k, ratio, start, offset):
    sel = C.c_int32(-7)
    status = lib.mr_topk_geometry(rows, cols, top_k, ratio, start, offset, C.byref(sel))
    if status == M.OK:
        assert 0 <= sel.value <= max(cols, 0)
    else:
        refused(status)
    size = lib.mr_topk_workspace_size(rows, cols, top_k)
    assert 0 <= size < 2 ** 56


def _status_of(call):
    try:
        return M.OK, call()
    except M.MRError as e:
        assert e.message
        return e.status, None


@SETTINGS
@given(window=st.integers(-2, 160), seq=st.one_of(st.just(1), st.integers(-2, 160)),
       start=st.one_of(st.just(0), st.integers(-2, 400), st.integers(2 ** 20, 2 ** 31 - 1)))
def test_window_indices_match_oracle(window, seq, start):
    st_o, exp = O.window_indices(window, seq, start)
    st_m, got = _status_of(lambda: M.attention_indices_window(window, seq, start))
    assert st_m == st_o
    if st_o == O.OK:
        np.testing.assert_array_equal(got, exp)


@SETTINGS
@given(ratio=st.integers(-2, 200), seq=st.one_of(st.just(1), st.integers(-2, 160)),
       start=st.one_of(st.just(0), st.integers(-2, 3000)),
       offset=st.one_of(st.integers(-2, 5000), st.integers(2 ** 31 - 3000, 2 ** 31 - 1)))
def test_compressed_indices_match_oracle(ratio, seq, start, offset):
    st_o, exp = O.compressed_indices(ratio, seq, start, offset)
    st_m, got = _status_of(lambda: M.attention_indices_compressed(ratio, seq, start, offset))
    assert st_m == st_o
    if st_o == O.OK:
        np.testing.assert_array_equal(got, exp)


@SETTINGS
@given(rows=st.one_of(st.just(1), st.integers(-1, 6)), cols=st.integers(-1, 40), top_k=st.integers(-1, 50),
       ratio=st.integers(-1, 9), start=st.one_of(st.just(0), st.integers(-2, 60)), offset=st.integers(-2, 9))
def test_topk_geometry_matches_oracle(lib, rows, cols, top_k, ratio, start, offset):
    # the oracle's selection over zero scores reports the same status and,
    # on success, as many keys per row as the geometry promises; a negative
    # count has no score matrix, and the geometry refuses it
    sel = C.c_int32(-7)
    st_m = lib.mr_topk_geometry(rows, cols, top_k, ratio, start, offset, C.byref(sel))
    if rows < 0 or cols < 0:
        assert st_m == M.INVALID_SHAPE
        return
    scores = np.zeros((max(rows, 1), max(cols, 1)), np.float32)[:rows, :cols]
    st_o, out = O.topk_select(np.ascontiguousarray(scores), top_k, ratio, start, offset)
    assert st_m == st_o
    if st_o == O.OK:
        assert out.shape == (rows, sel.value)


dtype = st.integers(-1, 6)


def _affine(packed_null, out_f, in_f, group, bits, sdt):
    w = M.AffineWeightDesc()
    w.packed = None if packed_null else C.c_void_p(256)
    w.scales = w.biases = None
    w.out_features, w.in_features, w.group, w.bits, w.scale_dtype = out_f, in_f, group, bits, sdt
    return w


def refused_or_empty(status, *counts):
    # a call with nothing to do may return MR_OK; any other call here has a
    # NULL buffer and must be refused
    if status == M.OK:
        assert min(counts) <= 0, counts
    else:
        refused(status)


@SETTINGS
@given(tokens=dim, out_f=big, in_f=big, group=st.sampled_from([0, 16, 32, 64, 128, -64]),
       bits=st.sampled_from([0, 2, 3, 4, 8, 16]), sdt=dtype, xdt=dtype, ydt=dtype, xs=stride, ys=stride,
       experts=st.integers(-2, 300), k=st.integers(-2, 10), pn=st.booleans())
def test_affine_entry_checks(lib, tokens, out_f, in_f, group, bits, sdt, xdt, ydt, xs, ys, experts, k, pn):
    w = _affine(pn, out_f, in_f, group, bits, sdt)
    refused(lib.mr_affine_dequantize(C.byref(w), None, ydt, None))
    refused_or_empty(lib.mr_affine_matmul(None, xdt, tokens, xs, C.byref(w), None, ydt, ys, None), tokens)
    refused_or_empty(lib.mr_affine_gather_matmul(None, xdt, tokens, xs, C.byref(w), experts, None, k, None, ydt,
                                                 None), tokens, k)
    refused(lib.mr_affine_dequantize(None, None, ydt, None))


@SETTINGS
@given(tokens=dim, out_f=big, in_f=big, wdt=dtype, xdt=dtype, ydt=dtype, xs=stride, ys=stride, rs=stride,
       wn=st.booleans())
def test_linear_checks(lib, tokens, out_f, in_f, wdt, xdt, ydt, xs, ys, rs, wn):
    w = M.DenseWeightDesc()
    w.weight = None if wn else C.c_void_p(256)
    w.dtype, w.out_features, w.in_features, w.row_stride = wdt, out_f, in_f, rs
    refused_or_empty(lib.mr_linear(None, xdt, tokens, xs, C.byref(w), None, ydt, ys, None), tokens)
    refused(lib.mr_linear(None, xdt, tokens, xs, None, None, ydt, ys, None))


@SETTINGS
@given(rows=big, d=dim, xdt=dtype, wdt=dtype, odt=dtype, xs=stride, os_=stride, eps=scale, n_pos=big,
       inner=dim, col0=st.integers(-3, 600), kv_rank=dim, rope=dim, tokens=big, heads=dim, nope=dim, v=dim,
       kind=st.integers(-1, 3))
def test_norm_rope_cache_absorb_checks(lib, rows, d, xdt, wdt, odt, xs, os_, eps, n_pos, inner, col0, kv_rank, rope,
                                       tokens, heads, nope, v, kind):
    refused_or_empty(lib.mr_rmsnorm(None, xdt, rows, d, xs, None, wdt, eps, None, odt, os_, None), rows)
    refused_or_empty(lib.mr_rope_apply(None, xdt, n_pos, inner, xs, col0, d, None, None, None), n_pos, inner)
    refused_or_empty(lib.mr_mla_cache_append(None, xdt, xs, tokens, None, wdt, eps, kv_rank, rope, None, None, None,
                                             os_, None, os_, col0, None), tokens)
    p = M.ProjectionDesc()
    p.kind = kind
    p.affine = _affine(False, heads * (nope + v) if heads > 0 and nope + v > 0 else 0, kv_rank, 64, 4, M.BF16)
    refused_or_empty(lib.mr_mla_absorb_query(None, xs, heads, nope, v, C.byref(p), None, os_, None), heads)
    refused_or_empty(lib.mr_mla_unabsorb_values(None, xs, heads, nope, v, C.byref(p), None, odt, None), heads)
    refused(lib.mr_mla_absorb_query(None, xs, heads, nope, v, None, None, os_, None))


@SETTINGS
@given(rows=dim, cols=big, top_k=big, ratio=st.integers(-2, 9), start=big, offset=big, flags=st.integers(0, 15),
       os_=stride, ss=stride, ws=st.sampled_from([0, 1 << 20]))
def test_topk_select_checks(lib, rows, cols, top_k, ratio, start, offset, flags, os_, ss, ws):
    a = M.TopkArgs()
    a.rows, a.cols, a.top_k, a.ratio, a.start_pos, a.offset, a.flags = rows, cols, top_k, ratio, start, offset, flags
    a.score_row_stride, a.out_row_stride, a.workspace_bytes = ss, os_, ws
    refused(lib.mr_topk_select(C.byref(a), None))
    refused(lib.mr_topk_select(None, None))
