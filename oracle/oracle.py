"""ctypes binding of the CPU oracle (oracle/mr_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by ``__graft_entry__.smoke()``
and by the ``cpu_baseline`` leg of ``bench.py``.  The product path never
imports this module.

Every wrapper mirrors one C function; the C source cites the reference
file:line each follows.  numpy arrays in, numpy arrays out; bf16 tensors are
``np.uint16`` bit patterns.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

OK, INVALID_SHAPE, INVALID_DTYPE, INDEX_OUT_OF_RANGE, DUPLICATE_INDEX, NONFINITE = range(6)
BF16, F16, F32 = 0, 1, 2

MASTER_SEED = 0x4D4C410001  # "MLA" + 0x0001


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = _declare(C.CDLL(LIB_PATH))
    return _lib


def _declare(L):
    u64, i64, i32, f32, f64 = C.c_uint64, C.c_int64, C.c_int32, C.c_float, C.c_double
    P = C.c_void_p
    sig = {
        "mro_splitmix_mix": (u64, [u64]),
        "mro_splitmix_value": (u64, [u64, u64]),
        "mro_splitmix_derive": (u64, [u64, u64]),
        "mro_label": (u64, [C.c_char_p]),
        "mro_f32_to_bf16": (C.c_uint16, [f32]),
        "mro_bf16_to_f32": (f32, [C.c_uint16]),
        "mro_f16_to_f32": (f32, [C.c_uint16]),
        "mro_fill_normal_bf16": (None, [u64, i64, f64, f64, P, C.c_int]),
        "mro_fill_abs_normal_bf16": (None, [u64, i64, f64, P, C.c_int]),
        "mro_fill_u32": (None, [u64, i64, P, C.c_int]),
        "mro_sparse_topk_indices": (C.c_int, [u64, i32, i32, i32, P]),
        "mro_rope_frequencies": (C.c_int, [i32, i32, f64, f64, f64, f64, P]),
        "mro_rope_table": (C.c_int, [P, i64, P, i32, C.c_int, P, P]),
        "mro_rope_apply_bf16": (None, [P, i64, i64, i64, i64, i32, P, P]),
        "mro_rmsnorm": (None, [P, i64, i64, P, f32, C.c_int, P]),
        "mro_mla_decode": (None, [P, P, P, i64, i64, i32, i32, i32, i32, i32, f32, C.c_int, P, C.c_int]),
        "mro_validate_indices": (C.c_int, [P, i32, i32, P]),
        "mro_sparse_attention": (C.c_int, [P, P, P, i64, i64, i32, i32, i32, i32, i32, P, i32, P, f32,
                                           C.c_int, P, C.c_int]),
        "mro_mla_prefill_rows": (None, [P, P, i64, P, P, i32, i32, i32, i32, i32, i32, i32, f32,
                                        C.c_int, P, P, i32, P, C.c_int]),
        "mro_affine_validate": (C.c_int, [i64, i64, i64, i32, i32, P]),
        "mro_affine_dequantize": (C.c_int, [P, P, P, i32, i64, i64, i32, i32, P, C.c_int]),
        "mro_affine_matmul": (C.c_int, [P, i64, P, P, P, i32, i64, i64, i32, i32, C.c_int, P, C.c_int]),
        "mro_linear": (None, [P, i64, P, C.c_int, i64, i64, i64, C.c_int, P, C.c_int]),
        "mro_sigmoid_gate": (None, [P, P, i64, P]),
        "mro_topk_select": (C.c_int, [P, i32, i32, i32, i32, i32, i32, P, P]),
        "mro_indexer_scores": (C.c_int, [P, i32, i32, i32, P, i32, P, P]),
        "mro_window_indices": (C.c_int, [i32, i32, i32, P, P, P]),
        "mro_compressed_indices": (C.c_int, [i32, i32, i32, i32, P, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    return L


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---------------------------------------------------------------- generator
def label(name: str) -> int:
    return lib().mro_label(name.encode())


def stream(name: str, seed: int = MASTER_SEED) -> int:
    return lib().mro_splitmix_derive(seed, label(name))


def normal_bf16(name, shape, mean=0.0, std=1.0, seed=MASTER_SEED, threads=0):
    out = np.empty(int(np.prod(shape)), np.uint16)
    lib().mro_fill_normal_bf16(stream(name, seed), out.size, mean, std, _p(out), threads)
    return out.reshape(shape)


def abs_normal_bf16(name, shape, std=1.0, seed=MASTER_SEED, threads=0):
    out = np.empty(int(np.prod(shape)), np.uint16)
    lib().mro_fill_abs_normal_bf16(stream(name, seed), out.size, std, _p(out), threads)
    return out.reshape(shape)


def u32(name, shape, seed=MASTER_SEED, threads=0):
    out = np.empty(int(np.prod(shape)), np.uint32)
    lib().mro_fill_u32(stream(name, seed), out.size, _p(out), threads)
    return out.reshape(shape)


def sparse_topk_indices(name, n_ctx, k, window, seed=MASTER_SEED):
    out = np.empty(k, np.int32)
    st = lib().mro_sparse_topk_indices(stream(name, seed), n_ctx, k, window, _p(out))
    if st != OK:
        raise ValueError(f"sparse_topk_indices status {st}")
    return out


# ---------------------------------------------------------------- bf16
def bf16_to_f32(a):
    a = np.asarray(a, np.uint16)
    return (a.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(a):
    """Round-to-nearest-even, NaN kept quiet (same rule as mro_f32_to_bf16)."""
    a = np.ascontiguousarray(a, np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


# ---------------------------------------------------------------- rope
def rope_frequencies(dim, base=10000.0, original_len=0, factor=1.0, beta_fast=32.0, beta_slow=1.0):
    out = np.empty(dim // 2, np.float64)
    st = lib().mro_rope_frequencies(dim, original_len, base, factor, beta_fast, beta_slow, _p(out))
    if st != OK:
        raise ValueError(f"rope_frequencies status {st}")
    return out


def rope_table(positions, freqs, inverse=False):
    pos = _c(positions, np.int64)
    half = len(freqs)
    cos = np.empty((pos.size, half), np.float32)
    sin = np.empty((pos.size, half), np.float32)
    st = lib().mro_rope_table(_p(pos), pos.size, _p(_c(freqs, np.float64)), half, int(inverse), _p(cos), _p(sin))
    if st != OK:
        raise ValueError(f"rope_table status {st}")
    return cos, sin


def rope_apply_bf16(x, cos, sin, col0, dim):
    """x: [n_pos, inner, row] uint16 (copied); rotates columns [col0, col0+dim)."""
    x = np.array(x, np.uint16, copy=True, order="C")
    n_pos = x.shape[0]
    inner = int(np.prod(x.shape[1:-1])) if x.ndim > 2 else 1
    lib().mro_rope_apply_bf16(_p(x), n_pos, inner, x.shape[-1], col0, dim,
                              _p(_c(cos, np.float32)), _p(_c(sin, np.float32)))
    return x


# ---------------------------------------------------------------- norm
def rmsnorm(x, weight, eps=1e-6, acc=1):
    x = _c(x, np.float32)
    out = np.empty_like(x)
    rows = x.size // x.shape[-1]
    lib().mro_rmsnorm(_p(x), rows, x.shape[-1], _p(_c(weight, np.float32)), eps, acc, _p(out))
    return out


# ---------------------------------------------------------------- attention
def mla_decode(q_lat, q_rope, cache, kv_rank=512, rope_dim=64, scale=192 ** -0.5, acc=1, threads=0):
    """q_lat [B,H,R] u16, q_rope [B,H,dr] u16, cache [B,N,row] u16 -> [B,H,R] f32."""
    q_lat = _c(q_lat, np.uint16)
    cache = _c(cache, np.uint16)
    if cache.ndim == 2:
        cache = cache[None]
    if q_lat.ndim == 2:
        q_lat = q_lat[None]
    B, H, R = q_lat.shape
    qr = None if rope_dim == 0 else _c(q_rope, np.uint16).reshape(B, H, rope_dim)
    N, row = cache.shape[1], cache.shape[2]
    out = np.empty((B, H, R), np.float32)
    lib().mro_mla_decode(_p(q_lat), _p(qr), _p(cache), row, N * row, B, H, N, kv_rank, rope_dim,
                         scale, acc, _p(out), threads)
    return out


def validate_indices(indices, n_rows):
    idx = _c(indices, np.int32)
    bad = np.array([-1], np.int32)
    st = lib().mro_validate_indices(_p(idx), idx.size, n_rows, _p(bad))
    return st, int(bad[0])


def sparse_attention(q_lat, q_rope, cache, indices, sinks=None, kv_rank=512, rope_dim=64,
                     scale=192 ** -0.5, acc=1, threads=0):
    """Returns (status, out [B,H,R] f32)."""
    q_lat = _c(q_lat, np.uint16)
    cache = _c(cache, np.uint16)
    if cache.ndim == 2:
        cache = cache[None]
    if q_lat.ndim == 2:
        q_lat = q_lat[None]
    B, H, R = q_lat.shape
    qr = None if rope_dim == 0 else _c(q_rope, np.uint16).reshape(B, H, rope_dim)
    idx = _c(indices, np.int32).reshape(B, -1)
    N, row = cache.shape[1], cache.shape[2]
    out = np.zeros((B, H, R), np.float32)
    sk = None if sinks is None else _c(sinks, np.float32)
    st = lib().mro_sparse_attention(_p(q_lat), _p(qr), _p(cache), row, N * row, B, H, N, kv_rank, rope_dim,
                                    _p(idx), idx.shape[1], _p(sk), scale, acc, _p(out), threads)
    return st, out


def mla_prefill_rows(q, cache, w_uk, w_uv, sel_t, sel_h, kv_rank=512, rope_dim=64, nope_dim=128,
                     v_dim=128, scale=192 ** -0.5, round_kv=False, threads=0):
    q = _c(q, np.uint16)
    T, H, _ = q.shape
    cache = _c(cache, np.uint16)
    P, row = cache.shape
    st = _c(sel_t, np.int32)
    sh = _c(sel_h, np.int32)
    out = np.empty((st.size, v_dim), np.float32)
    lib().mro_mla_prefill_rows(_p(q), _p(cache), row, _p(_c(w_uk, np.uint16)), _p(_c(w_uv, np.uint16)),
                               T, P, H, kv_rank, rope_dim, nope_dim, v_dim, scale, int(round_kv),
                               _p(st), _p(sh), st.size, _p(out), threads)
    return out


# ---------------------------------------------------------------- affine
def affine_validate(out_features, packed_cols, scale_cols, group, bits):
    inf = np.zeros(1, np.int64)
    st = lib().mro_affine_validate(out_features, packed_cols, scale_cols, group, bits, _p(inf))
    return st, int(inf[0])


def _scale_buf(a, dtype):
    return _c(a, np.float32 if dtype == F32 else np.uint16)


def affine_dequantize(packed, scales, biases, group=64, bits=4, scale_dtype=BF16, threads=0):
    packed = _c(packed, np.uint32)
    O, words = packed.shape
    I = words * (32 // bits)
    out = np.empty((O, I), np.float32)
    st = lib().mro_affine_dequantize(_p(packed), _p(_scale_buf(scales, scale_dtype)),
                                     _p(_scale_buf(biases, scale_dtype)), scale_dtype, O, I, group,
                                     bits, _p(out), threads)
    if st != OK:
        raise ValueError(f"affine_dequantize status {st}")
    return out


def affine_matmul(x, packed, scales, biases, group=64, bits=4, scale_dtype=BF16, acc=1, threads=0):
    x = _c(x, np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    packed = _c(packed, np.uint32)
    O, words = packed.shape
    I = words * (32 // bits)
    y = np.empty((x2.shape[0], O), np.float32)
    st = lib().mro_affine_matmul(_p(x2), x2.shape[0], _p(packed), _p(_scale_buf(scales, scale_dtype)),
                                 _p(_scale_buf(biases, scale_dtype)), scale_dtype, O, I, group, bits,
                                 acc, _p(y), threads)
    if st != OK:
        raise ValueError(f"affine_matmul status {st}")
    return y.reshape(x.shape[:-1] + (O,))


def linear(x, w, acc=1, threads=0):
    """k3Linear (Linear.swift:55-57): x float [..., in] . W^T, W [out, in]
    as bf16 bits (uint16) or float32."""
    x = _c(x, np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    w_f32 = int(w.dtype == np.float32)
    w = _c(w, np.float32 if w_f32 else np.uint16)
    O, I = w.shape
    y = np.empty((x2.shape[0], O), np.float32)
    lib().mro_linear(_p(x2), x2.shape[0], _p(w), w_f32, O, I, I, acc, _p(y), threads)
    return y.reshape(x.shape[:-1] + (O,))


def sigmoid_gate(merged, g):
    """MLA.swift:209-211: merged * sigmoid(g), fp32."""
    m = _c(merged, np.float32)
    g = _c(g, np.float32)
    out = np.empty_like(m)
    lib().mro_sigmoid_gate(_p(m), _p(g), m.size, _p(out))
    return out


# ---------------------------------------------------------------- indices
def indexer_scores(q, k, w):
    """DeepSeekV4LightningIndexer.scores (DeepSeekV4Attention.swift:530-549):
    q [S, H, D], k [T, D], w [S, H] -> [S, T] fp32."""
    q = _c(q, np.float32)
    k = _c(k, np.float32)
    w = _c(w, np.float32)
    S, H, D = q.shape
    T = k.shape[0]
    out = np.empty((S, T), np.float32)
    st = lib().mro_indexer_scores(_p(q), S, H, D, _p(k), T, _p(w), _p(out))
    if st != OK:
        raise ValueError(f"indexer_scores status {st}")
    return out


def topk_select(scores, top_k, ratio, start_pos, offset):
    s = _c(scores, np.float32)
    rows, cols = s.shape
    out = np.empty(rows * max(min(top_k, (start_pos + rows) // max(ratio, 1)), 1), np.int32)
    cnt = np.zeros(1, np.int32)
    st = lib().mro_topk_select(_p(s), rows, cols, top_k, ratio, start_pos, offset, _p(out), _p(cnt))
    if st != OK:
        return st, None
    return st, out[: rows * int(cnt[0])].reshape(rows, int(cnt[0]))


def window_indices(window, seq_len, start_pos):
    out = np.empty(max(seq_len * min(seq_len, window), window, 1), np.int32)
    r = np.zeros(1, np.int32)
    c = np.zeros(1, np.int32)
    st = lib().mro_window_indices(window, seq_len, start_pos, _p(out), _p(r), _p(c))
    if st != OK:
        return st, None
    return st, out[: int(r[0]) * int(c[0])].reshape(int(r[0]), int(c[0]))


def compressed_indices(ratio, seq_len, start_pos, offset):
    width = max(seq_len // max(ratio, 1), (start_pos + 1) // max(ratio, 1), 1)
    out = np.empty(max(seq_len, 1) * width, np.int32)
    r = np.zeros(1, np.int32)
    c = np.zeros(1, np.int32)
    st = lib().mro_compressed_indices(ratio, seq_len, start_pos, offset, _p(out), _p(r), _p(c))
    if st != OK:
        return st, None
    return st, out[: int(r[0]) * int(c[0])].reshape(int(r[0]), int(c[0]))
