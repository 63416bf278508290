"""Pins the oracle's RoPE, RMSNorm, affine and index functions (CPU only).

Each test checks the oracle against something other than its own formula:
closed forms, invariants, hand-written tables from the reference's stated
rules, or an independent numpy computation.
"""
import math

import numpy as np
import pytest

import oracle as O


# ------------------------------------------------------------------ RoPE
# DeepSeekV4Attention.swift:65-165
def test_rope_frequencies_plain_closed_form():
    f = O.rope_frequencies(64, base=10000.0)
    exp = np.array([1 / 10000.0 ** (2 * i / 64) for i in range(32)])
    np.testing.assert_allclose(f, exp, rtol=1e-15)
    assert f[0] == 1.0


def test_rope_frequencies_yarn_ramp_by_hand():
    dim, orig, base, factor = 64, 4096, 10000.0, 40.0
    f = O.rope_frequencies(dim, base=base, original_len=orig, factor=factor, beta_fast=32, beta_slow=1)
    # correction dims by hand
    cd = lambda rot: dim * math.log(orig / (rot * 2 * math.pi)) / (2 * math.log(base))
    low, high = max(math.floor(cd(32)), 0), min(math.ceil(cd(1)), dim - 1)
    assert (low, high) == (10, 23)
    plain = np.array([1 / base ** (2 * i / dim) for i in range(32)])
    assert f[0] == plain[0] and f[low] == plain[low]          # ramp 0 below low
    np.testing.assert_allclose(f[high:], plain[high:] / factor, rtol=1e-15)  # fully scaled
    mid = 16
    ramp = (mid - low) / (high - low)
    np.testing.assert_allclose(f[mid], plain[mid] / factor * ramp + plain[mid] * (1 - ramp), rtol=1e-15)


@pytest.mark.parametrize("args", [(0,), (63,), (64, 0, 1.0), (64, -1, 10000.0)])
def test_rope_frequencies_rejects(args):
    dim = args[0]
    orig = args[1] if len(args) > 1 else 0
    base = args[2] if len(args) > 2 else 10000.0
    with pytest.raises(ValueError):
        O.rope_frequencies(dim, base=base, original_len=orig)


def test_rope_table_kats():
    f = O.rope_frequencies(64)
    pos = np.array([0, 1, 32767, 131071])
    c, s = O.rope_table(pos, f)
    assert (c[0] == 1).all() and (s[0] == 0).all()
    for i, p in enumerate(pos):
        for j in (0, 7, 31):
            ang = float(p) * f[j]
            assert c[i, j] == np.float32(math.cos(ang))
            assert s[i, j] == np.float32(math.sin(ang))
    ci, si = O.rope_table(pos, f, inverse=True)
    np.testing.assert_array_equal(ci, c)
    np.testing.assert_array_equal(si, -s)


def _rotate_f64(x, pos, f):
    y = x.astype(np.float64).copy()
    for i in range(len(f)):
        a = pos * f[i]
        e, o = x[..., 2 * i].astype(np.float64), x[..., 2 * i + 1].astype(np.float64)
        y[..., 2 * i] = e * math.cos(a) - o * math.sin(a)
        y[..., 2 * i + 1] = e * math.sin(a) + o * math.cos(a)
    return y


def test_rope_apply_identity_inverse_norm_relative():
    f = O.rope_frequencies(64)
    x = O.normal_bf16("rope.x", (3, 2, 64))
    pos = np.array([0, 17, 32767])
    c, s = O.rope_table(pos, f)
    y = O.rope_apply_bf16(x, c, s, 0, 64)
    np.testing.assert_array_equal(y[0], x[0])  # position 0 is the identity
    xf, yf = O.bf16_to_f32(x), O.bf16_to_f32(y)
    # pairwise norm preserved up to bf16 rounding
    nx = np.hypot(xf[..., 0::2], xf[..., 1::2])
    ny = np.hypot(yf[..., 0::2], yf[..., 1::2])
    np.testing.assert_allclose(ny, nx, rtol=1e-2, atol=1e-2)
    # matches an fp64 rotation up to one bf16 rounding
    for i, p in enumerate(pos):
        np.testing.assert_allclose(yf[i], _rotate_f64(xf[i], float(p), f), rtol=8e-3, atol=8e-3)
    # inverse undoes forward (up to two bf16 roundings)
    ci, si = O.rope_table(pos, f, inverse=True)
    z = O.bf16_to_f32(O.rope_apply_bf16(y, ci, si, 0, 64))
    np.testing.assert_allclose(z, xf, rtol=2e-2, atol=2e-2)


def test_rope_relative_position_property():
    f = O.rope_frequencies(64)
    q = O.normal_bf16("rel.q", (1, 1, 64))
    k = O.normal_bf16("rel.k", (1, 1, 64))
    def dot(m, n):
        cq, sq = O.rope_table([m], f)
        ck, sk = O.rope_table([n], f)
        a = O.bf16_to_f32(O.rope_apply_bf16(q, cq, sq, 0, 64)).ravel().astype(np.float64)
        b = O.bf16_to_f32(O.rope_apply_bf16(k, ck, sk, 0, 64)).ravel().astype(np.float64)
        return a @ b
    assert abs(dot(10, 3) - dot(1007, 1000)) < 0.05
    assert abs(dot(10, 3) - dot(30010, 30003)) < 0.05


def test_rope_apply_tail_columns_only():
    f = O.rope_frequencies(64)
    row = O.normal_bf16("tail", (2, 1, 576))
    c, s = O.rope_table([5, 9], f)
    y = O.rope_apply_bf16(row, c, s, 512, 64)
    np.testing.assert_array_equal(y[..., :512], row[..., :512])
    assert not np.array_equal(y[..., 512:], row[..., 512:])


# ------------------------------------------------------------------ RMSNorm
# Normalization.swift:15-19
def test_rmsnorm_constant_vector_and_scale_invariance():
    w = 1 + 0.02 * O.bf16_to_f32(O.normal_bf16("w", (512,)))
    x = np.full((1, 512), -3.0, np.float32)
    y = O.rmsnorm(x, w, eps=1e-6)
    np.testing.assert_allclose(y[0], -w * 3.0 / math.sqrt(9.0 + 1e-6), rtol=1e-6)
    x = O.bf16_to_f32(O.normal_bf16("x", (4, 512)))
    a, b = O.rmsnorm(x, w, eps=0.0), O.rmsnorm(7.5 * x, w, eps=0.0)
    np.testing.assert_allclose(a, b, rtol=1e-5)


def test_rmsnorm_eps_inside_sqrt_and_float_path():
    w = np.ones(4, np.float32)
    x = np.array([[1e-3, -1e-3, 1e-3, -1e-3]], np.float32)
    y = O.rmsnorm(x, w, eps=1e-6)
    # eps inside: 1e-3/sqrt(1e-6+1e-6); eps outside would give 1e-3/(1e-3+1e-6)
    np.testing.assert_allclose(abs(y[0, 0]), 1e-3 / math.sqrt(2e-6), rtol=1e-6)
    x = O.bf16_to_f32(O.normal_bf16("x32", (3, 7168)))
    w = 1 + 0.02 * O.bf16_to_f32(O.normal_bf16("w32", (7168,)))
    np.testing.assert_allclose(O.rmsnorm(x, w, acc=0), O.rmsnorm(x, w, acc=1), rtol=2e-5, atol=1e-6)


# ------------------------------------------------------------------ affine
# AffineWeights.swift:65-157,232-342; MXFP4Weights.swift:42-48
def _unit_scales(rows, groups, value=1.0):
    return O.f32_to_bf16(np.full((rows, groups), value, np.float32))


def test_affine_nibble_order_kats():
    packed = np.array([[0x76543210, 0xFEDCBA98] * 4], np.uint32)  # 64 elements, 1 row
    s, b = _unit_scales(1, 1), _unit_scales(1, 1, 0.0)
    w = O.affine_dequantize(packed, s, b, group=64, bits=4)
    np.testing.assert_array_equal(w[0, :16], np.arange(16, dtype=np.float32))
    # bias only
    w0 = O.affine_dequantize(packed, _unit_scales(1, 1, 0.0), _unit_scales(1, 1, -0.5), group=64, bits=4)
    assert (w0 == -0.5).all()


def test_affine_2bit_and_8bit_orders():
    p2 = np.array([[0b11100100] * 2], np.uint32)  # elements 0..3 = 0,1,2,3 then zeros
    w = O.affine_dequantize(p2, _unit_scales(1, 1), _unit_scales(1, 1, 0.0), group=32, bits=2)
    np.testing.assert_array_equal(w[0, :5], [0, 1, 2, 3, 0])
    p8 = np.array([[0x04030201, 0x08070605]], np.uint32)
    w = O.affine_dequantize(p8, _unit_scales(1, 1), _unit_scales(1, 1, 0.0), group=8, bits=8)
    np.testing.assert_array_equal(w[0], np.arange(1, 9))


def test_affine_pack_unpack_round_trip_and_bitwise_closed_form():
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, size=(8, 128)).astype(np.uint32)
    packed = np.zeros((8, 16), np.uint32)
    for j in range(8):
        packed |= q[:, j::8] << (4 * j)
    s = O.abs_normal_bf16("aff.s", (8, 2), std=0.01)
    b = O.normal_bf16("aff.b", (8, 2), std=0.01)
    w = O.affine_dequantize(packed, s, b, group=64, bits=4)
    sf = np.repeat(O.bf16_to_f32(s), 64, axis=1)
    bf = np.repeat(O.bf16_to_f32(b), 64, axis=1)
    # the bf16-scale product is exact, so fp64 (s*q)+b rounded once equals the fp32 result
    exact = (sf.astype(np.float64) * q + bf.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(w.view(np.uint32), exact.view(np.uint32))
    # unpacking recovers q when scale=1, bias=0
    w1 = O.affine_dequantize(packed, _unit_scales(8, 2), _unit_scales(8, 2, 0.0), group=64, bits=4)
    np.testing.assert_array_equal(w1, q.astype(np.float32))


def test_affine_f16_and_f32_scales():
    packed = np.array([[0x76543210] * 8], np.uint32)
    s16 = np.array([[0x3C00]], np.uint16)  # 1.0 in f16
    b16 = np.array([[0xB800]], np.uint16)  # -0.5 in f16
    w = O.affine_dequantize(packed, s16, b16, group=64, bits=4, scale_dtype=O.F16)
    np.testing.assert_array_equal(w[0, :8], np.arange(8) - 0.5)
    s32 = np.array([[0.25]], np.float32)
    b32 = np.array([[1.0]], np.float32)
    w = O.affine_dequantize(packed, s32, b32, group=64, bits=4, scale_dtype=O.F32)
    np.testing.assert_array_equal(w[0, :8], np.arange(8) * 0.25 + 1)


@pytest.mark.parametrize(
    "args,status",
    [
        ((1536, 896, 112, 64, 4), O.OK),
        ((1536, 896, 112, 64, 3), O.INVALID_SHAPE),   # 32 % bits != 0
        ((1536, 896, 112, 0, 4), O.INVALID_SHAPE),    # group <= 0
        ((1536, 895, 112, 64, 4), O.INVALID_SHAPE),   # 7160 % 64 != 0
        ((1536, 896, 111, 64, 4), O.INVALID_SHAPE),   # group count differs
    ],
)
def test_affine_validation(args, status):
    st, inf = O.affine_validate(*args)
    assert st == status
    if status == O.OK:
        assert inf == 7168


def test_affine_matmul_against_dense_float64():
    packed = O.u32("mm.p", (48, 32))
    s = O.abs_normal_bf16("mm.s", (48, 4), std=0.01)
    b = O.normal_bf16("mm.b", (48, 4), std=0.01)
    x = O.bf16_to_f32(O.normal_bf16("mm.x", (3, 256)))
    w = O.affine_dequantize(packed, s, b).astype(np.float64)
    y = O.affine_matmul(x, packed, s, b, acc=1)
    np.testing.assert_allclose(y, x.astype(np.float64) @ w.T, rtol=1e-6, atol=1e-6)
    y32 = O.affine_matmul(x, packed, s, b, acc=0)
    np.testing.assert_allclose(y32, y, rtol=1e-4, atol=1e-4)


# ------------------------------------------------------------------ indices
# DeepSeekV4Attention.swift:170-237
def test_window_tables_by_hand():
    assert O.window_indices(4, 1, 5)[1].tolist() == [[2, 3, 0, 1]]
    assert O.window_indices(4, 1, 3)[1].tolist() == [[0, 1, 2, 3]]
    assert O.window_indices(4, 1, 2)[1].tolist() == [[0, 1, 2, -1]]
    assert O.window_indices(3, 5, 0)[1].tolist() == [
        [0, -1, -1], [0, 1, -1], [0, 1, 2], [1, 2, 3], [2, 3, 4]]
    assert O.window_indices(4, 2, 1)[0] == O.INVALID_SHAPE
    assert O.window_indices(0, 2, 0)[0] == O.INVALID_SHAPE


def test_compressed_tables_by_hand():
    assert O.compressed_indices(4, 1, 9, 100)[1].tolist() == [[100, 101]]
    st, t = O.compressed_indices(4, 1, 2, 100)
    assert st == O.OK and t.shape == (1, 0)
    assert O.compressed_indices(2, 5, 0, 7)[1].tolist() == [
        [-1, -1], [7, -1], [7, -1], [7, 8], [7, 8]]
    assert O.compressed_indices(2, 2, 3, 0)[0] == O.INVALID_SHAPE


# DeepSeekV4Attention.swift:582-645
def _brute_topk(scores, top_k, ratio, start_pos, offset):
    rows, cols = scores.shape
    available = (start_pos + rows) // ratio
    sel = min(top_k, available)
    out = []
    for r in range(rows):
        visible = (r + 1) // ratio if start_pos == 0 else available
        key = lambda k: (-(scores[r, k] if k < visible else -np.inf), k)
        order = sorted(range(available), key=key)
        out.append([offset + k if k < visible else -1 for k in order[:sel]])
    return out


def test_topk_select_brute_force_ties_and_masking():
    rng = np.random.default_rng(3)
    scores = rng.integers(-3, 4, size=(9, 4)).astype(np.float32)  # many ties
    st, got = O.topk_select(scores, top_k=3, ratio=2, start_pos=0, offset=10)
    assert st == O.OK
    assert got.tolist() == _brute_topk(scores, 3, 2, 0, 10)
    assert got[0].tolist() == [-1, -1, -1]  # row 0 sees no compressed key yet
    s1 = rng.standard_normal((1, 64)).astype(np.float32)
    s1[0, 5] = s1[0, 9] = 7.0
    st, got = O.topk_select(s1, top_k=8, ratio=4, start_pos=200, offset=0)
    assert got.tolist() == _brute_topk(s1, 8, 4, 200, 0)
    assert got[0, 0] == 5 and got[0, 1] == 9  # tie -> ascending key id
    # a visible -inf score ties with masked keys (both compare as -inf): key order
    s2 = np.array([[1.0, -np.inf, 2.0, 5.0, 5.0, 5.0]], np.float32)
    st, got = O.topk_select(np.repeat(s2, 6, axis=0), top_k=6, ratio=1, start_pos=0, offset=0)
    assert got.tolist() == _brute_topk(np.repeat(s2, 6, axis=0), 6, 1, 0, 0)
    assert got[2].tolist() == [2, 0, 1, -1, -1, -1] and got[1].tolist() == [0, 1, -1, -1, -1, -1]


def test_topk_select_errors_and_empty():
    s = np.zeros((1, 4), np.float32)
    s[0, 1] = np.nan
    assert O.topk_select(s, 2, 1, 3, 0)[0] == O.NONFINITE
    assert O.topk_select(np.zeros((2, 4), np.float32), 2, 1, 3, 0)[0] == O.INVALID_SHAPE
    assert O.topk_select(np.zeros((1, 2), np.float32), 2, 1, 3, 0)[0] == O.INVALID_SHAPE
    st, got = O.topk_select(np.zeros((1, 4), np.float32), 2, 4, 1, 0)
    assert st == O.OK and got.shape == (1, 0)
    # signed zeros tie
    z = np.array([[0.0, -0.0, 0.0]], np.float32)
    assert O.topk_select(z, 3, 1, 2, 0)[1].tolist() == [[0, 1, 2]]


# ---------------------------------------------------------------- k3Linear and the output gate
def test_linear_identity_one_hot_and_fp64_product():
    # k3Linear (Linear.swift:55-57): y = x . W^T with W output-major
    rng = np.random.default_rng(5)
    x = O.bf16_to_f32(O.f32_to_bf16(rng.standard_normal((3, 64)).astype(np.float32)))
    eye = O.f32_to_bf16(np.eye(64, dtype=np.float32))
    np.testing.assert_array_equal(O.linear(x, eye), x)
    perm = rng.permutation(64)
    sel = O.f32_to_bf16(np.eye(64, dtype=np.float32)[perm])   # row o picks x[perm[o]]
    np.testing.assert_array_equal(O.linear(x, sel), x[:, perm])
    w = O.normal_bf16("lin.w", (40, 64), std=0.1)
    want = x.astype(np.float64) @ O.bf16_to_f32(w).astype(np.float64).T
    np.testing.assert_allclose(O.linear(x, w, acc=1), want, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(O.linear(x, w, acc=0), want, rtol=1e-4, atol=1e-5)
    # f32 weights, and a transposed reading would fail: W is not symmetric
    wf = O.bf16_to_f32(w)
    np.testing.assert_allclose(O.linear(x, wf), want, rtol=1e-6, atol=1e-7)
    assert not np.allclose(O.linear(x[:, :40], O.f32_to_bf16(wf[:, :40].T.copy())), want[:, :40], atol=1e-3)


def test_linear_is_linear():
    rng = np.random.default_rng(6)
    w = O.normal_bf16("lin.l", (17, 96), std=0.1)
    a = rng.standard_normal(96).astype(np.float32)
    b = rng.standard_normal(96).astype(np.float32)
    lhs = O.linear((2 * a + 3 * b)[None], w).astype(np.float64)
    rhs = 2 * O.linear(a[None], w).astype(np.float64) + 3 * O.linear(b[None], w).astype(np.float64)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-5, atol=1e-5)


def test_sigmoid_gate_closed_forms():
    # MLA.swift:209-211: merged * sigmoid(g)
    m = np.array([1.0, -3.0, 7.5, 2.0], np.float32)
    np.testing.assert_array_equal(O.sigmoid_gate(m, np.zeros(4)), m * 0.5)        # sigmoid(0) = 1/2
    np.testing.assert_array_equal(O.sigmoid_gate(m, np.full(4, 100.0)), m)        # saturates to 1
    np.testing.assert_array_equal(O.sigmoid_gate(m, np.full(4, -200.0)), 0 * m)   # and to 0
    g = np.linspace(-6, 6, 25).astype(np.float32)
    s_pos = O.sigmoid_gate(np.ones(25), g).astype(np.float64)
    s_neg = O.sigmoid_gate(np.ones(25), -g).astype(np.float64)
    np.testing.assert_allclose(s_pos + s_neg, 1.0, atol=2e-7)                      # sigmoid(-g) = 1 - sigmoid(g)
    np.testing.assert_allclose(s_pos, 1 / (1 + np.exp(-g.astype(np.float64))), rtol=3e-7)
