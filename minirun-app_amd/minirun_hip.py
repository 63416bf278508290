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
import threading
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libminirun_hip.so")
SELFTEST_PATH = os.path.join(LIB_DIR, "libminirun_selftest.so")

OK, INVALID_SHAPE, INVALID_DTYPE, INDEX_OUT_OF_RANGE, DUPLICATE_INDEX, NONFINITE, HIP_ERROR, \
    INVALID_ARGUMENT, WORKSPACE_TOO_SMALL = range(9)
BF16, F16, F32, U32, I32 = range(5)

DECODE_VALIDATE_INDICES = 1
DECODE_SPLIT_ONLY = 4
DECODE_UNCHECKED = 8
DECODE_NOALLOC_SCRATCH_BYTES = 48 * 1024 * 1024


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
        ("index_status", C.c_void_p),
    ]


class AffineWeightDesc(C.Structure):
    _fields_ = [
        ("packed", C.c_void_p), ("scales", C.c_void_p), ("biases", C.c_void_p), ("scale_dtype", C.c_int),
        ("out_features", C.c_int64), ("in_features", C.c_int64), ("group", C.c_int32), ("bits", C.c_int32),
    ]


class DenseWeightDesc(C.Structure):
    _fields_ = [
        ("weight", C.c_void_p), ("dtype", C.c_int), ("out_features", C.c_int64), ("in_features", C.c_int64),
        ("row_stride", C.c_int64),
    ]


PROJ_NONE, PROJ_AFFINE, PROJ_DENSE = 0, 1, 2


class ProjectionDesc(C.Structure):
    _fields_ = [("kind", C.c_int), ("affine", AffineWeightDesc), ("dense", DenseWeightDesc)]


class BlockArgs(C.Structure):
    _fields_ = [
        ("hidden", C.c_int32), ("q_lora_rank", C.c_int32), ("heads", C.c_int32), ("qk_nope_dim", C.c_int32),
        ("qk_rope_dim", C.c_int32), ("v_head_dim", C.c_int32), ("kv_rank", C.c_int32),
        ("eps", C.c_float), ("scale", C.c_float),
        ("x", C.c_void_p), ("input_norm_w", C.c_void_p), ("q_a_norm_w", C.c_void_p), ("kv_a_norm_w", C.c_void_p),
        ("norm_w_dtype", C.c_int),
        ("q_a", ProjectionDesc), ("q_b", ProjectionDesc), ("kv_a", ProjectionDesc), ("kv_b", ProjectionDesc),
        ("o_proj", ProjectionDesc), ("g_proj", ProjectionDesc),
        ("cache_latent", C.c_void_p), ("latent_row_stride", C.c_int64),
        ("cache_rope", C.c_void_p), ("rope_row_stride", C.c_int64),
        ("position", C.c_int32), ("capacity", C.c_int32),
        ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
        ("out", C.c_void_p),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class PrefillArgs(C.Structure):
    _fields_ = [
        ("tokens", C.c_int32), ("n_ctx", C.c_int32), ("heads", C.c_int32),
        ("qk_nope_dim", C.c_int32), ("qk_rope_dim", C.c_int32), ("v_head_dim", C.c_int32), ("kv_rank", C.c_int32),
        ("scale", C.c_float),
        ("q", C.c_void_p), ("q_token_stride", C.c_int64), ("q_head_stride", C.c_int64),
        ("latent", C.c_void_p), ("latent_row_stride", C.c_int64),
        ("rope_keys", C.c_void_p), ("rope_row_stride", C.c_int64),
        ("kv_b", C.c_void_p), ("kv_b_row_stride", C.c_int64),
        ("out", C.c_void_p), ("out_dtype", C.c_int), ("out_token_stride", C.c_int64), ("out_head_stride", C.c_int64),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
        ("phase_events", C.c_void_p),
    ]


class PrefillBlockArgs(C.Structure):
    _fields_ = [
        ("tokens", C.c_int32),
        ("hidden", C.c_int32), ("q_lora_rank", C.c_int32), ("heads", C.c_int32), ("qk_nope_dim", C.c_int32),
        ("qk_rope_dim", C.c_int32), ("v_head_dim", C.c_int32), ("kv_rank", C.c_int32),
        ("eps", C.c_float), ("scale", C.c_float),
        ("x", C.c_void_p), ("x_token_stride", C.c_int64),
        ("input_norm_w", C.c_void_p), ("q_a_norm_w", C.c_void_p), ("kv_a_norm_w", C.c_void_p),
        ("norm_w_dtype", C.c_int),
        ("q_a", ProjectionDesc), ("q_b", ProjectionDesc), ("kv_a", ProjectionDesc), ("kv_b", ProjectionDesc),
        ("o_proj", ProjectionDesc), ("g_proj", ProjectionDesc),
        ("cache_latent", C.c_void_p), ("latent_row_stride", C.c_int64),
        ("cache_rope", C.c_void_p), ("rope_row_stride", C.c_int64),
        ("position", C.c_int32), ("capacity", C.c_int32),
        ("rope_cos", C.c_void_p), ("rope_sin", C.c_void_p),
        ("out", C.c_void_p), ("out_token_stride", C.c_int64),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class TopkArgs(C.Structure):
    _fields_ = [
        ("scores", C.c_void_p), ("score_row_stride", C.c_int64), ("rows", C.c_int32), ("cols", C.c_int32),
        ("top_k", C.c_int32), ("ratio", C.c_int32), ("start_pos", C.c_int32), ("offset", C.c_int32),
        ("out", C.c_void_p), ("out_row_stride", C.c_int64), ("status", C.c_void_p), ("flags", C.c_int32),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


TOPK_CHECK = 1
TOPK_UNCHECKED = 2

_P = C.c_void_p
_I32P = C.POINTER(C.c_int32)
_I64P = C.POINTER(C.c_int64)

# Every symbol include/minirun_hip.h declares, with its ctypes signature.
SIGNATURES = {
    "mr_version": (C.c_char_p, []),
    "mr_get_last_error": (C.c_char_p, []),
    "mr_mla_decode_workspace_size": (C.c_size_t, [C.POINTER(DecodeArgs)]),
    "mr_mla_decode": (C.c_int, [C.POINTER(DecodeArgs), C.c_void_p]),
    "mr_mla_decode_noalloc": (C.c_int, [C.POINTER(DecodeArgs), C.c_void_p]),
    "mr_validate_indices_workspace_size": (C.c_size_t, [C.c_int32, C.c_int32]),
    "mr_validate_indices": (C.c_int, [C.c_void_p, C.c_int32, C.c_int32, C.c_int32, C.c_void_p, C.c_size_t,
                                      C.POINTER(C.c_int32), C.POINTER(C.c_int32), C.c_void_p]),
    "mr_affine_validate": (C.c_int, [C.c_int, C.c_int32, _I64P, C.c_int, C.c_int32, _I64P, C.c_int, C.c_int32, _I64P,
                                     C.c_int32, C.c_int32, _I64P, _I64P, _I64P]),
    "mr_affine_dequantize": (C.c_int, [C.POINTER(AffineWeightDesc), _P, C.c_int, _P]),
    "mr_affine_matmul": (C.c_int, [_P, C.c_int, C.c_int32, C.c_int64, C.POINTER(AffineWeightDesc), _P, C.c_int,
                                   C.c_int64, _P]),
    "mr_affine_tile_view": (C.c_int, [_P, C.c_int64, C.c_int64, C.c_int32, C.c_int32, C.c_int,
                                      C.POINTER(AffineWeightDesc), C.POINTER(C.c_int64)]),
    "mr_tile_upload": (C.c_int, [_P, _P, C.c_int64, _P]),
    "mr_affine_adopt": (C.c_int, [_P, _P, _P, C.c_int, C.c_int64, C.c_int64, C.c_int64, C.c_int32, C.c_int32,
                                  _P, _P, _P, _P, _P, _P, C.POINTER(_P)]),
    "mr_adopted_affine_weight": (C.c_int, [_P, C.POINTER(AffineWeightDesc)]),
    "mr_adopted_affine_retain": (C.c_int, [_P]),
    "mr_adopted_affine_release": (C.c_int, [_P, _P]),
    "mr_adopted_affine_release_now": (C.c_int, [_P]),
    "mr_affine_gather_matmul": (C.c_int, [_P, C.c_int, C.c_int32, C.c_int64, C.POINTER(AffineWeightDesc), C.c_int64,
                                          _P, C.c_int32, _P, C.c_int, _P]),
    "mr_rmsnorm": (C.c_int, [_P, C.c_int, C.c_int64, C.c_int32, C.c_int64, _P, C.c_int, C.c_float, _P, C.c_int,
                             C.c_int64, _P]),
    "mr_rope_frequencies": (C.c_int, [C.c_int32, C.c_int32, C.c_double, C.c_double, C.c_double, C.c_double, _P]),
    "mr_rope_table": (C.c_int, [_P, C.c_int64, _P, C.c_int32, C.c_int32, _P, _P]),
    "mr_rope_apply": (C.c_int, [_P, C.c_int, C.c_int64, C.c_int64, C.c_int64, C.c_int64, C.c_int32, _P, _P, _P]),
    "mr_mla_cache_append": (C.c_int, [_P, C.c_int, C.c_int64, C.c_int64, _P, C.c_int, C.c_float, C.c_int32, C.c_int32,
                                      _P, _P, _P, C.c_int64, _P, C.c_int64, C.c_int64, _P]),
    "mr_mla_absorb_query": (C.c_int, [_P, C.c_int64, C.c_int32, C.c_int32, C.c_int32, C.POINTER(ProjectionDesc), _P,
                                      C.c_int64, _P]),
    "mr_mla_unabsorb_values": (C.c_int, [_P, C.c_int64, C.c_int32, C.c_int32, C.c_int32, C.POINTER(ProjectionDesc),
                                         _P, C.c_int, _P]),
    "mr_linear": (C.c_int, [_P, C.c_int, C.c_int32, C.c_int64, C.POINTER(DenseWeightDesc), _P, C.c_int, C.c_int64,
                            _P]),
    "mr_mla_decode_block_workspace_size": (C.c_size_t, [C.POINTER(BlockArgs)]),
    "mr_mla_decode_block": (C.c_int, [C.POINTER(BlockArgs), _P]),
    "mr_mla_prefill_workspace_size": (C.c_size_t, [C.POINTER(PrefillArgs)]),
    "mr_mla_prefill": (C.c_int, [C.POINTER(PrefillArgs), _P]),
    "mr_mla_prefill_block_workspace_size": (C.c_size_t, [C.POINTER(PrefillBlockArgs)]),
    "mr_mla_prefill_block": (C.c_int, [C.POINTER(PrefillBlockArgs), _P]),
    "mr_topk_geometry": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, C.c_int32, _I32P]),
    "mr_topk_workspace_size": (C.c_size_t, [C.c_int32, C.c_int32, C.c_int32]),
    "mr_topk_select": (C.c_int, [C.POINTER(TopkArgs), _P]),
    "mr_indexer_scores": (C.c_int, [_P, C.c_int, C.c_int32, C.c_int32, C.c_int32, C.c_int64, C.c_int64, _P, C.c_int,
                                    C.c_int32, C.c_int32, C.c_int64, _P, C.c_int, C.c_int32, C.c_int32, C.c_int64,
                                    _P, C.c_int64, _P]),
    "mr_attention_indices_window": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, _P, _I32P, _I32P]),
    "mr_attention_indices_compressed": (C.c_int, [C.c_int32, C.c_int32, C.c_int32, C.c_int32, _P, _I32P, _I32P]),
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
    """A stream argument as the C-ABI takes it: a torch stream, a raw handle
    (int or c_void_p), or None for torch's current stream."""
    if isinstance(stream, C.c_void_p):
        return stream
    if isinstance(stream, int):
        return C.c_void_p(stream)
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
                out_dtype=None, num_splits=0, flags=0, workspace=None, index_status=None):
    """Fill a DecodeArgs from torch tensors.

    q_lat [B,H,R] bf16 (R = kv_rank, 512 for the split kernel, else up to 2048
    on the any-width kernel); q_rope [B,H,dr] bf16 or None; latent [B,N,*] or
    [N,*] bf16 rows (first R columns used); rope_keys likewise (dr columns) or
    None; indices [B,K] int32 or None; sinks [H] f32 or None; index_status
    int32 [B,3] device tensor or None (the device-side index check).
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
    if index_status is not None:
        _need(index_status, "index_status", torch.int32)
        if index_status.numel() < 3 * B or not index_status.is_contiguous():
            raise ValueError("index_status must be a contiguous int32 tensor of at least 3 * batch entries")
        a.index_status = index_status.data_ptr()
    need = load().mr_mla_decode_workspace_size(C.byref(a))
    if workspace is None:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=q_lat.device)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    return a, out, workspace


def mla_decode(q_lat, q_rope, latent, rope_keys, *, scale, indices=None, sinks=None, out=None,
               out_dtype=None, num_splits=0, flags=0, workspace=None, index_status=None, stream=None):
    """Absorbed MLA decode / sparse decode.  Returns the [B,H,512] context.

    With indices, the lists are checked as the reference does: by default
    before the launch (a bad list raises MRError, the call synchronises);
    with an index_status tensor on the device in the same launch (read it
    later: per token (status, position, value)); not at all with
    DECODE_UNCHECKED in flags."""
    a, out, ws = decode_args(q_lat, q_rope, latent, rope_keys, scale=scale, indices=indices, sinks=sinks,
                             out=out, out_dtype=out_dtype, num_splits=num_splits, flags=flags, workspace=workspace,
                             index_status=index_status)
    _check(load().mr_mla_decode(C.byref(a), _stream(stream)))
    return out


def sparse_attention(queries_lat, queries_rope, cache, indices, *, scale, sinks=None, validate=True, **kw):
    """DeepSeekV4SparseAttention.forward over a [B, N, 512+dr] cache (rows
    shared by all heads, K = row[0:512+dr], V = row[0:512]).  validate=False
    skips the index checks (DECODE_UNCHECKED)."""
    lat = cache[..., :512]
    rk = cache[..., 512:] if queries_rope is not None else None
    flags = kw.pop("flags", 0) | (0 if validate else DECODE_UNCHECKED)
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


# ------------------------------------------------------------------ affine weights
class AffineWeights:
    """MLXBridge.AffineWeights (AffineWeights.swift:65-157) over device tensors.

    packed: uint32 (torch.int32 storage) [out, in*bits/32]; scales, biases:
    [out, in/group] bf16 / f16 / f32.  Construction validates through
    mr_affine_validate, so the errors are the reference's.
    """

    def __init__(self, packed, scales, biases, group_size=64, bits=4):
        torch = _torch()
        dt = {torch.bfloat16: BF16, torch.float16: F16, torch.float32: F32}
        sdt = dt.get(scales.dtype, 99)
        bdt = dt.get(biases.dtype, 99)
        pdt = U32 if packed.dtype in (torch.int32, torch.uint32) else (F32 if packed.dtype == torch.float32 else 99)
        ps = (C.c_int64 * packed.dim())(*packed.shape)
        ss = (C.c_int64 * scales.dim())(*scales.shape)
        bs = (C.c_int64 * biases.dim())(*biases.shape)
        ex, of, inf = C.c_int64(), C.c_int64(), C.c_int64()
        _check(load().mr_affine_validate(pdt, packed.dim(), ps, sdt, scales.dim(), ss, bdt, biases.dim(), bs,
                                         group_size, bits, C.byref(ex), C.byref(of), C.byref(inf)))
        for t, n in ((packed, "packed"), (scales, "scales"), (biases, "biases")):
            _need(t, n)
            if not t.is_contiguous():
                raise ValueError(f"{n} must be contiguous")
        self.packed, self.scales, self.biases = packed, scales, biases
        self.group_size, self.bits = group_size, bits
        self.experts = ex.value or None
        self.out_features, self.in_features = of.value, inf.value
        self.scale_dtype = sdt

    def desc(self):
        return AffineWeightDesc(self.packed.data_ptr(), self.scales.data_ptr(), self.biases.data_ptr(),
                                self.scale_dtype, self.out_features, self.in_features, self.group_size, self.bits)


FINALIZER = C.CFUNCTYPE(None, C.c_void_p)

# One C callback for every adopted weight's finalizers, alive as long as the
# module: the library calls it with a context id, which names the Python
# finalizer and its argument in _FINALIZERS.  The library may call it on a
# HIP runtime thread after the AdoptedAffineWeights object is gone, so no
# per-object ctypes thunk is ever handed to it.
_FINALIZERS = {}
_FIN_LOCK = threading.Lock()
_FIN_NEXT = [1]


@FINALIZER
def _finalizer_trampoline(ctx):
    with _FIN_LOCK:
        fn, arg = _FINALIZERS.pop(ctx)
    fn(arg)


def _register_finalizer(fn, arg):
    with _FIN_LOCK:
        key = _FIN_NEXT[0]
        _FIN_NEXT[0] += 1
        _FINALIZERS[key] = (fn, arg)
    return key


class AdoptedAffineWeights:
    """AffineWeights.adopting (AffineWeights.swift:159-198): the three buffers
    (device pointers, or pinned host memory the device reads) pass to the
    library with a finalizer each (Python callables of one argument, the
    context value).  Each finalizer runs exactly once, when the last
    reference is released and the named stream has passed every read; a
    failed adoption runs them before raising.  Shapes: packed [experts?, out,
    in*bits/32], scales/biases [experts?, out, in/group]."""

    def __init__(self, packed_ptr, scales_ptr, biases_ptr, scale_dtype, out_features, in_features, *,
                 experts=0, group_size=64, bits=4, finalizers=(None, None, None), contexts=(None, None, None)):
        cb, ctx = [], []
        for f, c in zip(finalizers, contexts):
            if f is None:
                cb.append(None)
                ctx.append(None)
            else:
                cb.append(C.cast(_finalizer_trampoline, _P))
                ctx.append(_register_finalizer(f, c))
        h = _P()
        _check(load().mr_affine_adopt(packed_ptr, scales_ptr, biases_ptr, scale_dtype, experts, out_features,
                                      in_features, group_size, bits, cb[0], ctx[0], cb[1], ctx[1], cb[2], ctx[2],
                                      C.byref(h)))
        self.handle = h.value
        self.out_features, self.in_features = out_features, in_features

    def desc(self):
        d = AffineWeightDesc()
        _check(load().mr_adopted_affine_weight(self.handle, C.byref(d)))
        return d

    def retain(self):
        _check(load().mr_adopted_affine_retain(self.handle))

    def release(self, stream=None):
        """Drop one reference; the last one runs the finalizers behind the
        work on `stream` (a torch stream or a raw handle; None: torch's
        current stream, as for every other call here)."""
        _check(load().mr_adopted_affine_release(self.handle, _stream(stream)))

    def release_now(self):
        """Drop one reference; the last one runs the finalizers before this
        returns (for a weight no GPU work reads any more)."""
        _check(load().mr_adopted_affine_release_now(self.handle))


class DenseWeights:
    """A dense projection weight for k3Linear (Linear.swift:55-57): output-major
    [out, in] bf16 or f32 on the device."""

    def __init__(self, weight):
        torch = _torch()
        _need(weight, "weight")
        if weight.dim() != 2 or weight.dtype not in (torch.bfloat16, torch.float32):
            raise ValueError("a dense weight is a 2-D bf16 or f32 [out_features, in_features] tensor")
        self.weight = weight
        self.out_features, self.in_features = weight.shape

    def desc(self):
        return DenseWeightDesc(self.weight.data_ptr(), _dtype_code(self.weight.dtype), self.out_features,
                               self.in_features, self.weight.stride(0))


def projection(w):
    """ProjectionDesc of an AffineWeights, a DenseWeights, or None (absent)."""
    p = ProjectionDesc()
    if w is None:
        p.kind = PROJ_NONE
    elif isinstance(w, AffineWeights):
        p.kind, p.affine = PROJ_AFFINE, w.desc()
    elif isinstance(w, DenseWeights):
        p.kind, p.dense = PROJ_DENSE, w.desc()
    else:
        raise TypeError("a projection is AffineWeights, DenseWeights or None")
    return p


def linear(x, w: DenseWeights, out_dtype=None, stream=None):
    """k3Linear (Linear.swift:55-57): x [tokens, in] -> x . W^T [tokens, out]."""
    torch = _torch()
    _need(x, "x")
    x2 = x if x.dim() == 2 else x.reshape(1, -1)
    y = torch.empty(x2.shape[0], w.out_features, dtype=out_dtype or x.dtype, device=x.device)
    _check(load().mr_linear(_ptr(x2), _dtype_code(x2.dtype), x2.shape[0], x2.stride(0), C.byref(w.desc()), _ptr(y),
                            _dtype_code(y.dtype), y.stride(0), _stream(stream)))
    return y if x.dim() == 2 else y.reshape(w.out_features)


def affine_dequantize(w: AffineWeights, dtype=None, stream=None):
    """affineDequantize (AffineWeights.swift:328-342): dense [out, in], f32 by default."""
    torch = _torch()
    out = torch.empty(w.out_features, w.in_features, dtype=dtype or torch.float32, device=w.packed.device)
    _check(load().mr_affine_dequantize(C.byref(w.desc()), _ptr(out), _dtype_code(out.dtype), _stream(stream)))
    return out


def affine_mm(x, w: AffineWeights, out_dtype=None, stream=None):
    """affineMM (AffineWeights.swift:239-254): x [tokens, in] -> [tokens, out]."""
    torch = _torch()
    _need(x, "x")
    x2 = x if x.dim() == 2 else x.reshape(1, -1)
    y = torch.empty(x2.shape[0], w.out_features, dtype=out_dtype or x.dtype, device=x.device)
    _check(load().mr_affine_matmul(_ptr(x2), _dtype_code(x2.dtype), x2.shape[0], x2.stride(0), C.byref(w.desc()),
                                   _ptr(y), _dtype_code(y.dtype), y.stride(0), _stream(stream)))
    return y if x.dim() == 2 else y.reshape(w.out_features)


def affine_tile_view(tile_ptr, rows, cols, group=64, bits=4, scale_dtype=BF16):
    """A StorageCore affine tile [packed | scales | biases] (QuantizedTileContainer
    .swift:219-343) as a weight descriptor over its bytes, and the tile size."""
    d = AffineWeightDesc()
    n = C.c_int64()
    _check(load().mr_affine_tile_view(tile_ptr, rows, cols, group, bits, scale_dtype, C.byref(d), C.byref(n)))
    return d, n.value


def affine_gather_mm(x, w: AffineWeights, rhs_indices, out_dtype=None, stream=None):
    """affineGatherMM (AffineWeights.swift:255-318): x [tokens, in], a
    stacked w (experts != None), rhs_indices int32 [tokens, experts_per_token]
    -> [tokens, experts_per_token, out], row (t, j) = W[rhs[t, j]] . x[t].
    The reference's preconditions raise MRError (INVALID_ARGUMENT)."""
    torch = _torch()
    _need(x, "x")
    experts = w.experts or 0
    if x.dim() != 2:
        raise ValueError("x must be [tokens, inFeatures]; this function inserts the broadcast axes itself")
    if rhs_indices.dim() != 2 or rhs_indices.shape[0] != x.shape[0]:
        _check(load().mr_affine_gather_matmul(None, 0, -1, 0, C.byref(w.desc()), max(experts, 1), None, 0, None, 0,
                                              None))  # raises the reference's message
    if rhs_indices.dtype != torch.int32 or not rhs_indices.is_contiguous():
        raise ValueError("rhs_indices must be contiguous int32")
    T, K = rhs_indices.shape
    y = torch.empty(T, K, w.out_features, dtype=out_dtype or x.dtype, device=x.device)
    _check(load().mr_affine_gather_matmul(_ptr(x), _dtype_code(x.dtype), T, x.stride(0) if T else w.in_features,
                                          C.byref(w.desc()), experts, _ptr(rhs_indices), K, _ptr(y),
                                          _dtype_code(y.dtype), _stream(stream)))
    return y


def rms_norm(x, weight, eps=1e-6, out_dtype=None, stream=None):
    """K3Norm.rms (Normalization.swift:15-19) over the last axis."""
    torch = _torch()
    _need(x, "x")
    _need(weight, "weight")
    x2 = x.reshape(-1, x.shape[-1])
    out = torch.empty(x2.shape, dtype=out_dtype or x.dtype, device=x.device)
    _check(load().mr_rmsnorm(_ptr(x2), _dtype_code(x2.dtype), x2.shape[0], x2.shape[1], x2.stride(0), _ptr(weight),
                             _dtype_code(weight.dtype), eps, _ptr(out), _dtype_code(out.dtype), out.stride(0),
                             _stream(stream)))
    return out.reshape(x.shape)


def rope_frequencies(dim, base=10000.0, original_len=0, factor=1.0, beta_fast=32.0, beta_slow=1.0):
    import numpy as np

    out = np.empty(dim // 2, np.float64)
    _check(load().mr_rope_frequencies(dim, original_len, base, factor, beta_fast, beta_slow,
                                      out.ctypes.data_as(C.c_void_p)))
    return out


def rope_table(positions, freqs, inverse=False):
    import numpy as np

    pos = np.ascontiguousarray(positions, np.int64)
    half = len(freqs)
    cos = np.empty((pos.size, half), np.float32)
    sin = np.empty((pos.size, half), np.float32)
    _check(load().mr_rope_table(pos.ctypes.data_as(C.c_void_p), pos.size,
                                np.ascontiguousarray(freqs, np.float64).ctypes.data_as(C.c_void_p), half, int(inverse),
                                cos.ctypes.data_as(C.c_void_p), sin.ctypes.data_as(C.c_void_p)))
    return cos, sin


def rope_apply_(x, cos_t, sin_t, col0, dim, stream=None):
    """DeepSeekV4Rotary.apply in place on x [n_pos, inner..., row] (device tables)."""
    _need(x, "x")
    n_pos = x.shape[0]
    inner = 1
    for d in x.shape[1:-1]:
        inner *= d
    _check(load().mr_rope_apply(_ptr(x), _dtype_code(x.dtype), n_pos, inner, x.shape[-1], col0, dim, _ptr(cos_t),
                                _ptr(sin_t), _stream(stream)))
    return x


def mla_cache_append(kv, norm_w, eps, cos_t, sin_t, latent, rope, start_row, kv_rank=512, rope_dim=64, stream=None):
    _need(kv, "kv")
    kv2 = kv.reshape(-1, kv.shape[-1])
    _check(load().mr_mla_cache_append(_ptr(kv2), _dtype_code(kv2.dtype), kv2.stride(0), kv2.shape[0], _ptr(norm_w),
                                      _dtype_code(norm_w.dtype), eps, kv_rank, rope_dim, _ptr(cos_t), _ptr(sin_t),
                                      _ptr(latent), latent.stride(0), _ptr(rope), rope.stride(0), start_row,
                                      _stream(stream)))


def mla_absorb_query(q, heads, nope_dim, v_dim, kv_b, stream=None):
    """q_lat = q_nope . W_UK per head (MLA.swift:180-188); kv_b AffineWeights or DenseWeights."""
    torch = _torch()
    q_lat = torch.empty(heads, 512, dtype=torch.bfloat16, device=q.device)
    _check(load().mr_mla_absorb_query(_ptr(q), q.stride(0), heads, nope_dim, v_dim, C.byref(projection(kv_b)),
                                      _ptr(q_lat), 512, _stream(stream)))
    return q_lat


def mla_unabsorb_values(ctx, heads, nope_dim, v_dim, kv_b, out_dtype=None, stream=None):
    """out = ctx . W_UV^T per head (MLA.swift:196-197); kv_b AffineWeights or DenseWeights."""
    torch = _torch()
    out = torch.empty(heads, v_dim, dtype=out_dtype or torch.bfloat16, device=ctx.device)
    _check(load().mr_mla_unabsorb_values(_ptr(ctx), ctx.stride(0), heads, nope_dim, v_dim, C.byref(projection(kv_b)),
                                         _ptr(out), _dtype_code(out.dtype), _stream(stream)))
    return out


def block_args(x, weights, cache, position, rope_cos, rope_sin, out, *, hidden=7168, q_lora_rank=1536, heads=128,
               nope=128, rope=64, v=128, kv_rank=512, eps=1e-6, scale=None, workspace=None):
    """Fill BlockArgs; `weights` is a dict with input_norm (or None), q_a_norm,
    kv_a_norm (tensors) and q_a, q_b, kv_a, kv_b, o_proj, optional g_proj
    (AffineWeights or DenseWeights).  rope_cos = rope_sin = None: NoPE."""
    torch = _torch()
    a = BlockArgs()
    a.hidden, a.q_lora_rank, a.heads, a.qk_nope_dim, a.qk_rope_dim, a.v_head_dim, a.kv_rank = \
        hidden, q_lora_rank, heads, nope, rope, v, kv_rank
    a.eps = eps
    a.scale = scale if scale is not None else (nope + rope) ** -0.5
    a.x = x.data_ptr()
    a.input_norm_w = weights["input_norm"].data_ptr() if weights.get("input_norm") is not None else None
    a.q_a_norm_w = weights["q_a_norm"].data_ptr()
    a.kv_a_norm_w = weights["kv_a_norm"].data_ptr()
    a.norm_w_dtype = _dtype_code(weights["q_a_norm"].dtype)
    for n in ("q_a", "q_b", "kv_a", "kv_b", "o_proj", "g_proj"):
        setattr(a, n, projection(weights.get(n)))
    a.cache_latent, a.latent_row_stride = cache.data_ptr(), cache.stride(0)
    a.cache_rope, a.rope_row_stride = cache[:, kv_rank:].data_ptr(), cache.stride(0)
    a.position, a.capacity = position, cache.shape[0]
    a.rope_cos = rope_cos.data_ptr() if rope_cos is not None else None
    a.rope_sin = rope_sin.data_ptr() if rope_sin is not None else None
    a.out = out.data_ptr()
    need = load().mr_mla_decode_block_workspace_size(C.byref(a))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    return a, workspace


def mla_decode_block(x, weights, cache, position, rope_cos, rope_sin, stream=None, **kw):
    """K3MLA.forwardWithoutTrace for one decode token (affine or dense
    projections, optional gate, rotary or NoPE)."""
    torch = _torch()
    out = torch.empty(kw.get("hidden", 7168), dtype=torch.bfloat16, device=x.device)
    a, ws = block_args(x, weights, cache, position, rope_cos, rope_sin, out, **kw)
    _check(load().mr_mla_decode_block(C.byref(a), _stream(stream)))
    return out


def prefill_args(q, latent, rope_keys, kv_b, *, scale=None, out=None, out_dtype=None, workspace=None):
    """Fill PrefillArgs: q [T,H,nope+rope] bf16; latent [P,>=kv_rank] and
    rope_keys [P,>=rope] bf16 row views (both may be views of one cache);
    kv_b [H*(nope+v), kv_rank] bf16 (kv_b_proj, output-major), which fixes
    kv_rank and v_head.  The widths 128 / 64 / 128 / 512 run on MFMA, others
    on the any-width kernels."""
    torch = _torch()
    for t, n in ((q, "q"), (latent, "latent"), (rope_keys, "rope_keys"), (kv_b, "kv_b")):
        _need(t, n, torch.bfloat16)
    T, H, D = q.shape
    P = latent.shape[0]
    nope = D - rope_keys.shape[1]
    a = PrefillArgs()
    a.tokens, a.n_ctx, a.heads = T, P, H
    a.qk_nope_dim, a.qk_rope_dim = nope, rope_keys.shape[1]
    a.v_head_dim, a.kv_rank = kv_b.shape[0] // H - nope, kv_b.shape[1]
    a.scale = scale if scale is not None else D ** -0.5
    a.q, a.q_token_stride, a.q_head_stride = q.data_ptr(), q.stride(0), q.stride(1)
    a.latent, a.latent_row_stride = latent.data_ptr(), latent.stride(0)
    a.rope_keys, a.rope_row_stride = rope_keys.data_ptr(), rope_keys.stride(0)
    a.kv_b, a.kv_b_row_stride = kv_b.data_ptr(), kv_b.stride(0)
    if out is None:
        out = torch.empty(T, H, a.v_head_dim, dtype=out_dtype or torch.bfloat16, device=q.device)
    a.out, a.out_dtype = out.data_ptr(), _dtype_code(out.dtype)
    a.out_token_stride, a.out_head_stride = out.stride(0), out.stride(1)
    need = load().mr_mla_prefill_workspace_size(C.byref(a))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    a._keep = (q, latent, rope_keys, kv_b, out, workspace)
    return a, out, workspace


def mla_prefill(q, latent, rope_keys, kv_b, *, scale=None, out=None, out_dtype=None, workspace=None, stream=None):
    """K3MLA.forward eager prefill (MLA.swift:159-168,198-206): causal
    attention of the T queries over the P cached rows, per-head keys/values
    up-projected through kv_b."""
    a, out, _ = prefill_args(q, latent, rope_keys, kv_b, scale=scale, out=out, out_dtype=out_dtype,
                             workspace=workspace)
    _check(load().mr_mla_prefill(C.byref(a), _stream(stream)))
    return out


def prefill_block_args(x, weights, cache, position, rope_cos, rope_sin, out, *, q_lora_rank=1536, heads=128,
                       nope=128, rope=64, v=128, kv_rank=512, eps=1e-6, scale=None, workspace=None):
    """Fill PrefillBlockArgs for the T prompt rows of x [T, hidden] (bf16);
    `weights` as for block_args; cache [capacity, kv_rank + rope] bf16, rows
    0 .. position-1 already written; rope_cos / rope_sin [T, rope/2] f32
    tensors (the angles at position .. position+T-1) or None (NoPE)."""
    torch = _torch()
    a = PrefillBlockArgs()
    a.tokens = x.shape[0]
    a.hidden, a.q_lora_rank, a.heads, a.qk_nope_dim, a.qk_rope_dim, a.v_head_dim, a.kv_rank = \
        x.shape[1], q_lora_rank, heads, nope, rope, v, kv_rank
    a.eps = eps
    a.scale = scale if scale is not None else (nope + rope) ** -0.5
    a.x, a.x_token_stride = x.data_ptr(), x.stride(0)
    a.input_norm_w = weights["input_norm"].data_ptr() if weights.get("input_norm") is not None else None
    a.q_a_norm_w = weights["q_a_norm"].data_ptr()
    a.kv_a_norm_w = weights["kv_a_norm"].data_ptr()
    a.norm_w_dtype = _dtype_code(weights["q_a_norm"].dtype)
    for n in ("q_a", "q_b", "kv_a", "kv_b", "o_proj", "g_proj"):
        setattr(a, n, projection(weights.get(n)))
    a.cache_latent, a.latent_row_stride = cache.data_ptr(), cache.stride(0)
    a.cache_rope, a.rope_row_stride = (cache[:, kv_rank:].data_ptr() if rope else None), cache.stride(0)
    a.position, a.capacity = position, cache.shape[0]
    a.rope_cos = rope_cos.data_ptr() if rope_cos is not None else None
    a.rope_sin = rope_sin.data_ptr() if rope_sin is not None else None
    a.out, a.out_token_stride = out.data_ptr(), out.stride(0)
    need = load().mr_mla_prefill_block_workspace_size(C.byref(a))
    if workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=x.device)
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    return a, workspace


def mla_prefill_block(x, weights, cache, position, rope_cos, rope_sin, stream=None, **kw):
    """K3MLA.forward over a prompt (MLA.swift:124-229): the T rows of x
    through the block, appending cache rows position .. position+T-1;
    returns out [T, hidden] bf16."""
    torch = _torch()
    out = torch.empty(x.shape[0], x.shape[1], dtype=torch.bfloat16, device=x.device)
    a, ws = prefill_block_args(x, weights, cache, position, rope_cos, rope_sin, out, **kw)
    _check(load().mr_mla_prefill_block(C.byref(a), _stream(stream)))
    return out


def topk_geometry(rows, cols, top_k, ratio, start_pos, offset):
    """The reference's selection-geometry checks (DeepSeekV4Attention.swift:
    590-612); returns the number of keys each row receives."""
    sel = C.c_int32()
    _check(load().mr_topk_geometry(rows, cols, top_k, ratio, start_pos, offset, C.byref(sel)))
    return sel.value


def lightning_index_scores(queries, compressed_keys, head_weights, *, out=None, stream=None):
    """DeepSeekV4LightningIndexer.scores (DeepSeekV4Attention.swift:530-549):
    queries [S, H, D], compressed_keys [T, D], head_weights [S, H] (bf16 or
    f32, weights already scaled) -> f32 [S, T], sum_h w * max(q . k, 0).
    Geometry errors are the reference's (MRError INVALID_SHAPE)."""
    torch = _torch()
    if queries.dim() != 3 or compressed_keys.dim() != 2 or head_weights.dim() != 2:
        # a zero geometry makes the library raise the reference's error
        _check(load().mr_indexer_scores(None, BF16, 0, 0, 0, 0, 0, None, BF16, 0, 0, 0, None, BF16, 0, 0, 0, None, 0,
                                        None))
    S, H, D = queries.shape
    T, KD = compressed_keys.shape
    WR, WC = head_weights.shape
    codes = {torch.bfloat16: BF16, torch.float32: F32}
    for t, n in ((queries, "queries"), (compressed_keys, "compressed_keys"), (head_weights, "head_weights")):
        if t.dtype not in codes:
            raise ValueError(f"{n} must be bf16 or f32")
        if t.numel() and t.stride(-1) != 1:
            raise ValueError(f"{n} must have a unit last-dimension stride")
    if out is None:
        out = torch.empty(max(S, 0), max(T, 0), dtype=torch.float32, device=queries.device)
    _check(load().mr_indexer_scores(queries.data_ptr(), codes[queries.dtype], S, H, D,
                                    queries.stride(0) if S else 0, queries.stride(1) if H else 0,
                                    compressed_keys.data_ptr(), codes[compressed_keys.dtype], T, KD,
                                    compressed_keys.stride(0) if T else 0, head_weights.data_ptr(),
                                    codes[head_weights.dtype], WR, WC, head_weights.stride(0) if WR else 0,
                                    out.data_ptr(), out.stride(0) if out.numel() else max(T, 0), _stream(stream)))
    return out


def lightning_select(scores, top_k, ratio, start_pos, offset, *, check=True, status=None, stream=None):
    """DeepSeekV4LightningIndexer.select on the device: scores [rows, cols]
    f32 -> int32 [rows, selected] (offset + key, -1 past the visible keys).
    check=True synchronises and raises MRError (NONFINITE) on a NaN score,
    as the reference throws."""
    torch = _torch()
    _need(scores, "scores", torch.float32)
    rows, cols = scores.shape
    sel = topk_geometry(rows, cols, top_k, ratio, start_pos, offset)
    out = torch.empty(rows, max(sel, 1), dtype=torch.int32, device=scores.device)
    ws = torch.empty(max(load().mr_topk_workspace_size(rows, cols, top_k), 1), dtype=torch.uint8,
                     device=scores.device)
    a = TopkArgs()
    a.scores, a.score_row_stride, a.rows, a.cols = scores.data_ptr(), scores.stride(0), rows, cols
    a.top_k, a.ratio, a.start_pos, a.offset = top_k, ratio, start_pos, offset
    a.out, a.out_row_stride = out.data_ptr(), out.stride(0)
    a.status = status.data_ptr() if status is not None else None
    a.flags = TOPK_CHECK if check else (0 if status is not None else TOPK_UNCHECKED)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _check(load().mr_topk_select(C.byref(a), _stream(stream)))
    return out[:, :sel]


def attention_indices_window(window, seq_len, start_pos):
    import numpy as np

    n = max(seq_len * min(seq_len, window), window, 1)
    out = np.empty(n, np.int32)
    r, c = C.c_int32(), C.c_int32()
    _check(load().mr_attention_indices_window(window, seq_len, start_pos, out.ctypes.data_as(C.c_void_p), C.byref(r),
                                              C.byref(c)))
    return out[: r.value * c.value].reshape(r.value, c.value)


def attention_indices_compressed(ratio, seq_len, start_pos, offset):
    import numpy as np

    width = max(seq_len // max(ratio, 1), (start_pos + 1) // max(ratio, 1), 1)
    out = np.empty(max(seq_len, 1) * width, np.int32)
    r, c = C.c_int32(), C.c_int32()
    _check(load().mr_attention_indices_compressed(ratio, seq_len, start_pos, offset, out.ctypes.data_as(C.c_void_p),
                                                  C.byref(r), C.byref(c)))
    return out[: r.value * c.value].reshape(r.value, c.value)
