"""Pins the oracle's MLA decode, sparse attention and prefill (CPU only).

Reference equations: MLA.swift:174-206 (absorbed decode and eager prefill),
MLA.swift:231-275 (expand, causal mask), DeepSeekV4Attention.swift:861-920
(sparse attention with sinks and the -1 sentinel).
"""
import numpy as np
import pytest

import oracle as O

SCALE = 192 ** -0.5


def f(x):
    return O.bf16_to_f32(x).astype(np.float64)


def numpy_decode(q_lat, q_rope, cache, R=512, dr=64, scale=SCALE, sink=None):
    """Independent fp64 restatement with numpy primitives."""
    c = f(cache)
    s = (f(q_lat) @ c[:, :R].T + (f(q_rope) @ c[:, R:R + dr].T if dr else 0)) * scale
    m = s.max(axis=-1, keepdims=True)
    if sink is not None:
        m = np.maximum(m, sink[:, None])
    e = np.exp(s - m)
    den = e.sum(-1, keepdims=True) + (np.exp(sink[:, None] - m) if sink is not None else 0)
    return (e / den) @ c[:, :R]


def small_inputs(H=4, N=96, R=32, dr=8, seed=11):
    ql = O.normal_bf16("t.ql", (H, R), seed=seed)
    qr = O.normal_bf16("t.qr", (H, dr), seed=seed)
    cache = O.normal_bf16("t.c", (N, R + dr), std=0.5, seed=seed)
    return ql, qr, cache


def test_decode_matches_numpy_fp64_and_fp32_path():
    ql, qr, cache = small_inputs()
    ref = numpy_decode(ql, qr, cache, R=32, dr=8)
    got = O.mla_decode(ql, qr, cache, kv_rank=32, rope_dim=8)[0]
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-7)
    got32 = O.mla_decode(ql, qr, cache, kv_rank=32, rope_dim=8, acc=0)[0]
    np.testing.assert_allclose(got32, ref, rtol=1e-4, atol=1e-5)


def test_decode_16_heads_512_ctx_shape():
    ql = O.normal_bf16("c1.q_lat", (16, 512))
    qr = O.normal_bf16("c1.q_rope", (16, 64))
    cache = O.normal_bf16("c1.cache", (512, 576), std=0.5)
    got = O.mla_decode(ql, qr, cache)[0]
    np.testing.assert_allclose(got, numpy_decode(ql, qr, cache), rtol=1e-6, atol=1e-7)


def test_decode_absorbed_equals_expanded():
    # MLA.swift:100-122: the absorbed expression equals the expanded one.
    H, N, R, dr, dn, dv = 3, 40, 16, 4, 8, 8
    rng = np.random.default_rng(5)
    c = rng.standard_normal((N, R + dr)) * 0.5
    q_nope = rng.standard_normal((H, dn))
    q_rot = rng.standard_normal((H, dr))
    w_uk = rng.standard_normal((H, dn, R)) * 0.3   # kv_b_proj rows for keys, per head
    w_uv = rng.standard_normal((H, dv, R)) * 0.3
    scale = (dn + dr) ** -0.5
    # expanded: K_h = [c W_uk^T | k_rot], V_h = c W_uv^T
    out_exp = np.zeros((H, dv))
    for h in range(H):
        K = np.concatenate([c[:, :R] @ w_uk[h].T, c[:, R:]], axis=1)
        V = c[:, :R] @ w_uv[h].T
        s = np.concatenate([q_nope[h], q_rot[h]]) @ K.T * scale
        p = np.exp(s - s.max()); p /= p.sum()
        out_exp[h] = p @ V
    # absorbed through the oracle: q_lat = q_nope . W_uk, ctx = oracle, out = ctx . W_uv^T
    q_lat = np.einsum("hd,hdr->hr", q_nope, w_uk)
    bf = lambda a: O.f32_to_bf16(a.astype(np.float32))
    # feed exactly-representable bf16 inputs: compare against expanded on the same rounded values
    ql_b, qr_b, c_b = bf(q_lat), bf(q_rot), bf(c)
    ctx = O.mla_decode(ql_b, qr_b, c_b, kv_rank=R, rope_dim=dr, scale=scale)[0]
    out_abs = np.einsum("hr,hvr->hv", ctx.astype(np.float64), w_uv)
    # expanded on the rounded inputs
    cr, qlr, qrr = f(c_b), f(ql_b), f(qr_b)
    out_exp_r = np.zeros((H, dv))
    for h in range(H):
        s = (qlr[h] @ cr[:, :R].T + qrr[h] @ cr[:, R:].T) * scale
        p = np.exp(s - s.max()); p /= p.sum()
        out_exp_r[h] = p @ (cr[:, :R] @ w_uv[h].T)
    np.testing.assert_allclose(out_abs, out_exp_r, rtol=1e-6, atol=1e-8)
    # and the unrounded expanded form agrees to bf16 input precision
    np.testing.assert_allclose(out_abs, out_exp, rtol=5e-2, atol=5e-2)


def test_decode_special_cases():
    ql, qr, cache = small_inputs(N=1)
    got = O.mla_decode(ql, qr, cache, kv_rank=32, rope_dim=8)[0]
    np.testing.assert_array_equal(got, np.broadcast_to(O.bf16_to_f32(cache[0, :32]), got.shape))
    # zero query -> equal scores -> mean of rows
    ql, qr, cache = small_inputs(N=50)
    z = np.zeros_like(ql)
    got = O.mla_decode(z, np.zeros_like(qr), cache, kv_rank=32, rope_dim=8)[0]
    np.testing.assert_allclose(got[0], f(cache)[:, :32].mean(0), rtol=1e-6, atol=1e-7)
    # one dominant score -> that row
    cache2 = cache.copy()
    cache2[17, :32] = O.f32_to_bf16(np.full(32, 8.0, np.float32))
    q = O.f32_to_bf16(np.full((4, 32), 8.0, np.float32))
    got = O.mla_decode(q, np.zeros_like(qr), cache2, kv_rank=32, rope_dim=8, scale=1.0)[0]
    np.testing.assert_allclose(got, np.broadcast_to(f(cache2)[17, :32], got.shape), rtol=1e-9)
    # row permutation leaves the output unchanged
    perm = np.random.default_rng(1).permutation(50)
    a = O.mla_decode(ql, qr, cache, kv_rank=32, rope_dim=8)[0]
    b = O.mla_decode(ql, qr, cache[perm], kv_rank=32, rope_dim=8)[0]
    np.testing.assert_allclose(a, b, rtol=1e-9, atol=1e-12)


# ----------------------------------------------------------------- sparse
def test_sparse_all_indices_equals_dense():
    ql, qr, cache = small_inputs(N=64)
    idx = np.arange(64, dtype=np.int32)[::-1].copy()
    st, got = O.sparse_attention(ql, qr, cache, idx, kv_rank=32, rope_dim=8)
    assert st == O.OK
    np.testing.assert_allclose(got[0], O.mla_decode(ql, qr, cache, kv_rank=32, rope_dim=8)[0], rtol=1e-9, atol=1e-12)


def test_sparse_single_index_sentinel_and_subset():
    ql, qr, cache = small_inputs(N=64)
    st, got = O.sparse_attention(ql, qr, cache, np.array([-1, 9, -1], np.int32), kv_rank=32, rope_dim=8)
    assert st == O.OK
    np.testing.assert_array_equal(got[0], np.broadcast_to(O.bf16_to_f32(cache[9, :32]), got[0].shape))
    sub = np.array([3, 40, 7, 63], np.int32)
    st, got = O.sparse_attention(ql, qr, cache, sub, kv_rank=32, rope_dim=8)
    np.testing.assert_allclose(got[0], numpy_decode(ql, qr, cache[sub], R=32, dr=8), rtol=1e-6, atol=1e-8)


def test_sparse_sink_semantics():
    ql, qr, cache = small_inputs(N=64)
    idx = np.arange(0, 64, 3, dtype=np.int32)
    sinks = np.array([0.5, -2.0, 3.0, 0.0], np.float32)
    st, got = O.sparse_attention(ql, qr, cache, idx, sinks=sinks, kv_rank=32, rope_dim=8)
    ref = numpy_decode(ql, qr, cache[idx], R=32, dr=8, sink=sinks.astype(np.float64))
    np.testing.assert_allclose(got[0], ref, rtol=1e-6, atol=1e-8)
    # a very negative sink is the no-sink result
    st, a = O.sparse_attention(ql, qr, cache, idx, sinks=np.full(4, -1e30, np.float32), kv_rank=32, rope_dim=8)
    st, b = O.sparse_attention(ql, qr, cache, idx, kv_rank=32, rope_dim=8)
    np.testing.assert_allclose(a, b, rtol=1e-12)
    # single row + sink: out = row * e^s / (e^s + e^sink)
    st, one = O.sparse_attention(ql, qr, cache, np.array([5], np.int32), sinks=sinks, kv_rank=32, rope_dim=8)
    s = (f(ql) @ f(cache)[5, :32] + f(qr) @ f(cache)[5, 32:]) * SCALE
    w = 1 / (1 + np.exp(sinks - s))
    np.testing.assert_allclose(one[0], w[:, None] * f(cache)[5, :32][None], rtol=1e-6)


def test_sparse_errors_and_empty():
    ql, qr, cache = small_inputs(N=64)
    st, _ = O.sparse_attention(ql, qr, cache, np.array([1, 64], np.int32), kv_rank=32, rope_dim=8)
    assert st == O.INDEX_OUT_OF_RANGE
    st, _ = O.sparse_attention(ql, qr, cache, np.array([1, -2], np.int32), kv_rank=32, rope_dim=8)
    assert st == O.INDEX_OUT_OF_RANGE
    st, _ = O.sparse_attention(ql, qr, cache, np.array([4, 9, 4], np.int32), kv_rank=32, rope_dim=8)
    assert st == O.DUPLICATE_INDEX
    assert O.validate_indices(np.array([4, 9, -1, 4]), 64) == (O.DUPLICATE_INDEX, 3)
    assert O.validate_indices(np.array([4, 99]), 64) == (O.INDEX_OUT_OF_RANGE, 1)
    # in-order scan: the repeat at 1 stops it before the out-of-range entry at 2
    assert O.validate_indices(np.array([7, 7, 99]), 64) == (O.DUPLICATE_INDEX, 1)
    assert O.validate_indices(np.array([7, 99, 7]), 64) == (O.INDEX_OUT_OF_RANGE, 1)
    assert O.validate_indices(np.array([-1, 3, -1, 3]), 64) == (O.DUPLICATE_INDEX, 3)
    assert O.validate_indices(np.array([-1, -1]), 64) == (O.OK, -1)
    st, got = O.sparse_attention(ql, qr, cache, np.array([-1, -1], np.int32), kv_rank=32, rope_dim=8)
    assert st == O.OK and (got == 0).all()


def test_sparse_v4_form_no_rope():
    # DeepSeek V4 rows: K = V = row (512 wide here 32), sinks present
    H, N, D = 4, 48, 32
    q = O.normal_bf16("v4.q", (H, D))
    rows = O.normal_bf16("v4.rows", (N, D), std=0.5)
    sinks = np.array([0.1, 0.2, -0.3, 1.0], np.float32)
    idx = np.array([0, 5, 47, 20, -1], np.int32)
    st, got = O.sparse_attention(q, None, rows, idx, sinks=sinks, kv_rank=D, rope_dim=0)
    ref = numpy_decode(q, None, rows[idx[idx >= 0]], R=D, dr=0, sink=sinks.astype(np.float64))
    np.testing.assert_allclose(got[0], ref, rtol=1e-6, atol=1e-8)


# ----------------------------------------------------------------- prefill
def numpy_prefill(q, cache, w_uk, w_uv, R, dr, dn, dv, scale):
    T, H, _ = q.shape
    P = cache.shape[0]
    c = f(cache)
    out = np.zeros((T, H, dv))
    for h in range(H):
        K = np.concatenate([c[:, :R] @ f(w_uk)[:, h * dn:(h + 1) * dn], c[:, R:R + dr]], axis=1)
        V = c[:, :R] @ f(w_uv)[:, h * dv:(h + 1) * dv]
        s = f(q[:, h]) @ K.T * scale
        mask = np.arange(P)[None, :] > (np.arange(T)[:, None] + P - T)
        s = np.where(mask, -np.finfo(np.float32).max, s)
        p = np.exp(s - s.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        out[:, h] = p @ V
    return out


def test_prefill_matches_numpy_and_prefix_consistency():
    T, H, R, dr, dn, dv = 12, 3, 16, 4, 8, 8
    scale = (dn + dr) ** -0.5
    q = O.normal_bf16("pf.q", (T, H, dn + dr))
    cache = O.normal_bf16("pf.c", (T, R + dr), std=0.5)
    w_uk = O.normal_bf16("pf.wuk", (R, H * dn), std=0.2)
    w_uv = O.normal_bf16("pf.wuv", (R, H * dv), std=0.2)
    sel_t = np.repeat(np.arange(T), H)
    sel_h = np.tile(np.arange(H), T)
    got = O.mla_prefill_rows(q, cache, w_uk, w_uv, sel_t, sel_h, kv_rank=R, rope_dim=dr, nope_dim=dn,
                             v_dim=dv, scale=scale).reshape(T, H, dv)
    ref = numpy_prefill(q, cache, w_uk, w_uv, R, dr, dn, dv, scale)
    np.testing.assert_allclose(got, ref, rtol=1e-6, atol=1e-8)
    # query 0 sees only key 0: output = V[0]
    np.testing.assert_allclose(got[0, 0], f(cache)[0, :R] @ f(w_uv)[:, :dv], rtol=1e-6)
    # prefix consistency: the first 5 tokens alone give the same first 5 rows
    got5 = O.mla_prefill_rows(q[:5], cache[:5], w_uk, w_uv, sel_t[:5 * H], sel_h[:5 * H], kv_rank=R,
                              rope_dim=dr, nope_dim=dn, v_dim=dv, scale=scale).reshape(5, H, dv)
    np.testing.assert_allclose(got5, got[:5], rtol=1e-12)


def test_prefill_single_query_equals_absorbed_decode():
    P, H, R, dr, dn, dv = 30, 2, 16, 4, 8, 8
    scale = (dn + dr) ** -0.5
    q = O.normal_bf16("pd.q", (1, H, dn + dr))
    cache = O.normal_bf16("pd.c", (P, R + dr), std=0.5)
    w_uk = O.normal_bf16("pd.wuk", (R, H * dn), std=0.2)
    w_uv = O.normal_bf16("pd.wuv", (R, H * dv), std=0.2)
    got = O.mla_prefill_rows(q, cache, w_uk, w_uv, [0, 0], [0, 1], kv_rank=R, rope_dim=dr,
                             nope_dim=dn, v_dim=dv, scale=scale)
    for h in range(H):
        q_lat = f(q[0, h, :dn]) @ f(w_uk)[:, h * dn:(h + 1) * dn].T  # absorb W_UK
        # absorbed decode in fp64 on unrounded q_lat
        c = f(cache)
        s = (q_lat @ c[:, :R].T + f(q[0, h, dn:]) @ c[:, R:].T) * scale
        p = np.exp(s - s.max()); p /= p.sum()
        out = (p @ c[:, :R]) @ f(w_uv)[:, h * dv:(h + 1) * dv]
        np.testing.assert_allclose(got[h], out, rtol=1e-6, atol=1e-8)
