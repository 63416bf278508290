"""Python host binding of the C-ABI in include/minirun_hip.h.

The library is loaded from minirun-app_amd/lib/ (built by build.py); there is
no fallback: if it is missing, every call raises.  torch is used only for
device memory, streams and dtypes; all arithmetic runs in the HIP library.

Names follow the reference operators they stand in for:
  mla_decode            K3MLA absorbed attention core (MLA.swift:174-197)
  sparse_attention      DeepSeekV4SparseAttention.forward (DeepSeekV4Attention.swift:747-770)
  validate_indices      its index checks (DeepSeekV4Attention.swift:884-895)
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libminirun_hip.so")
SELFTEST_PATH = os.path.join(LIB_DIR, "libminirun_selftest.so")

OK, INVALID_SHAPE, INVALID_DTYPE, INDEX_OUT_OF_RANGE, DUPLICATE_INDEX, NONFINITE, HIP_ERROR, \
    INVALID_ARGUMENT, WORKSPACE_TOO_SMALL = range(9)
BF16, F16, F32, U32, I32 = range(5)

DECODE_VALIDATE_INDICES = 1
DECODE_NO_TRANSPOSE_READ = 2


class MRError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[mr_status {status}] {message}")
        self.status = status
        self.message = message


class DecodeArgs(C.Structure):
    _fields_ = [
        ("batch", C.c_int32), ("heads", C.c_int32), ("n_ctx", C.c_int32), ("kv_rank", C.c_int32),
        ("rope_dim", C.c_int32), ("scale", C.c_float),
        ("q_lat", C.c_void_p), ("q_lat_batch_stride", C.c_int64), ("q_lat_head_stride", C.c_int64),
        ("q_rope", C.c_void_p), ("q_rope_batch_stride", C.c_int64), ("q_rope_head_stride", C.c_int64),
        ("latent", C.c_void_p), ("latent_row_stride", C.c_int64), ("latent_batch_stride", C.c_int64),
        ("rope_keys", C.c_void_p), ("rope_row_stride", C.c_int64), ("rope_batch_stride", C.c_int64),
        ("indices", C.c_void_p), ("n_idx", C.c_int32),
        ("sinks", C.c_void_p),
        ("out", C.c_void_p), ("out_dtype", C.c_int), ("out_batch_stride", C.c_int64),
        ("out_head_stride", C.c_int64),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
        ("num_splits", C.c_int32), ("flags", C.c_uint32),
        ("phase_events", C.c_void_p),
    ]


# Every symbol include/minirun_hip.h declares, with its ctypes signature.
SIGNATURES = {
    "mr_version": (C.c_char_p, []),
    "mr_get_last_error": (C.c_char_p, []),
    "mr_mla_decode_workspace_size": (C.c_size_t, [C.POINTER(DecodeArgs)]),
    "mr_mla_decode": (C.c_int, [C.POINTER(DecodeArgs), C.c_void_p]),
    "mr_validate_indices_workspace_size": (C.c_size_t, [C.c_int32, C.c_int32]),
    "mr_validate_indices": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_size_t,
                                      C.POINTER(C.c_int32), C.POINTER(C.c_int32), C.c_void_p]),
}

_lib = None


def load(path: str = LIB_PATH):
    """Load the HIP library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is not built: run `python minirun-app_amd/build.py`")
        lib = C.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def last_error() -> str:
    return load().mr_get_last_error().decode()


def _check(status: int):
    if status != OK:
        raise MRError(status, last_error())


def version() -> str:
    return load().mr_version().decode()


# ------------------------------------------------------------------ torch helpers
def _torch():
    import torch

    return torch


def _stream(stream):
    torch = _torch()
    if stream is None:
        stream = torch.cuda.current_stream()
    return C.c_void_p(stream.cuda_stream)


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def _dtype_code(dt):
    torch = _torch()
    return {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}[dt]


def _need(t, name, dtype=None):
    torch = _torch()
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError(f"{name} must be a CUDA (HIP) tensor")
    if dtype is not None and t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must be contiguous in its last dimension")


def decode_args(q_lat, q_rope, latent, rope_keys, *, scale, indices=None, sinks=None, out=None,
                out_dtype=None, num_splits=0, flags=0, workspace=None):
    """Fill a DecodeArgs from torch tensors.

    q_lat [B,H,512] bf16; q_rope [B,H,64] bf16 or None; latent [B,N,*] or [N,*]
    bf16 rows (first 512 columns used); rope_keys likewise (64 columns) or
    None; indices [B,K] int32 or None; sinks [H] f32 or None.
    """
    torch = _torch()
    _need(q_lat, "q_lat", torch.bfloat16)
    if q_lat.dim() == 2:
        q_lat = q_lat.unsqueeze(0)
    B, H, R = q_lat.shape
    rope_dim = 0 if q_rope is None else q_rope.shape[-1]
    if q_rope is not None:
        _need(q_rope, "q_rope", torch.bfloat16)
        if q_rope.dim() == 2:
            q_rope = q_rope.unsqueeze(0)
    _need(latent, "latent", torch.bfloat16)
    lat3 = latent if latent.dim() == 3 else latent.unsqueeze(0)
    lat_bs = lat3.stride(0) if lat3.shape[0] > 1 else (0 if latent.dim() == 2 else lat3.stride(0))
    rk3 = None
    if rope_keys is not None:
        _need(rope_keys, "rope_keys", torch.bfloat16)
        rk3 = rope_keys if rope_keys.dim() == 3 else rope_keys.unsqueeze(0)
    n_ctx = lat3.shape[1]
    if out is None:
        out = torch.empty((B, H, R), dtype=out_dtype or torch.bfloat16, device=q_lat.device)
    a = DecodeArgs()
    a.batch, a.heads, a.n_ctx, a.kv_rank, a.rope_dim = B, H, n_ctx, R, rope_dim
    a.scale = float(scale)
    a.q_lat, a.q_lat_batch_stride, a.q_lat_head_stride = q_lat.data_ptr(), q_lat.stride(0), q_lat.stride(1)
    if q_rope is not None:
        a.q_rope, a.q_rope_batch_stride, a.q_rope_head_stride = q_rope.data_ptr(), q_rope.stride(0), q_rope.stride(1)
    a.latent, a.latent_row_stride, a.latent_batch_stride = lat3.data_ptr(), lat3.stride(1), lat_bs
    if rk3 is not None:
        rk_bs = rk3.stride(0) if rope_keys.dim() == 3 else 0
        a.rope_keys, a.rope_row_stride, a.rope_batch_stride = rk3.data_ptr(), rk3.stride(1), rk_bs
    if indices is not None:
        _need(indices, "indices", torch.int32)
        idx = indices if indices.dim() == 2 else indices.unsqueeze(0)
        if idx.stride(0) != idx.shape[1] and idx.shape[0] > 1:
            raise ValueError("indices must be a contiguous [B, K] tensor")
        if idx.numel() == 0:  # an empty list is still a (non-NULL) sparse request
            idx = torch.full((idx.shape[0], 1), -1, dtype=torch.int32, device=idx.device)
            a._keep = idx
            a.indices, a.n_idx = idx.data_ptr(), 0
        else:
            a.indices, a.n_idx = idx.data_ptr(), idx.shape[1]
    if sinks is not None:
        _need(sinks, "sinks", torch.float32)
        a.sinks = sinks.data_ptr()
    _need(out, "out")
    a.out, a.out_dtype = out.data_ptr(), _dtype_code(out.dtype)
    o3 = out if out.dim() == 3 else out.unsqueeze(0)
    a.out_batch_stride, a.out_head_stride = o3.stride(0), o3.stride(1)
    a.num_splits, a.flags = int(num_splits), int(flags)
    need = load().mr_mla_decode_workspace_size(C.byref(a))
    if workspace is None:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=q_lat.device)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    return a, out, workspace


def mla_decode(q_lat, q_rope, latent, rope_keys, *, scale, indices=None, sinks=None, out=None,
               out_dtype=None, num_splits=0, flags=0, workspace=None, stream=None):
    """Absorbed MLA decode / sparse decode.  Returns the [B,H,512] context."""
    a, out, ws = decode_args(q_lat, q_rope, latent, rope_keys, scale=scale, indices=indices, sinks=sinks,
                             out=out, out_dtype=out_dtype, num_splits=num_splits, flags=flags, workspace=workspace)
    _check(load().mr_mla_decode(C.byref(a), _stream(stream)))
    return out


def sparse_attention(queries_lat, queries_rope, cache, indices, *, scale, sinks=None, validate=True, **kw):
    """DeepSeekV4SparseAttention.forward over a [B, N, 512+dr] cache (rows
    shared by all heads, K = row[0:512+dr], V = row[0:512])."""
    lat = cache[..., :512]
    rk = cache[..., 512:] if queries_rope is not None else None
    flags = kw.pop("flags", 0) | (DECODE_VALIDATE_INDICES if validate else 0)
    return mla_decode(queries_lat, queries_rope, lat, rk, scale=scale, indices=indices, sinks=sinks,
                      flags=flags, **kw)


def validate_indices(indices, n_rows, stream=None):
    """Returns (status, bad_token, bad_position, message) for an int32 [B, K] tensor."""
    torch = _torch()
    idx = indices if indices.dim() == 2 else indices.unsqueeze(0)
    B, K = idx.shape
    need = load().mr_validate_indices_workspace_size(B, K)
    ws = torch.empty(max(need, 256), dtype=torch.uint8, device=idx.device)
    bt, bp = C.c_int32(-1), C.c_int32(-1)
    st = load().mr_validate_indices(_ptr(idx), B, K, int(n_rows), _ptr(ws), ws.numel(), C.byref(bt), C.byref(bp),
                                    _stream(stream))
    return st, bt.value, bp.value, (last_error() if st != OK else "")
