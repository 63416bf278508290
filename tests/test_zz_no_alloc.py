"""mr_mla_decode_noalloc against mr_mla_decode: the same kernels on the
library's static scratch instead of a caller workspace.  Two calls in a
row, the second on a smaller input, for the dense and the gathered form;
outputs must be bitwise equal to the workspace entry point's (same launch
plan, same kernels) and within the workload bar of the oracle."""
import ctypes as C

import numpy as np
import pytest

import mla_inputs as MI
import oracle as O

pytestmark = pytest.mark.gpu


def dev(a):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    return (t.view(torch.bfloat16) if a.dtype == np.uint16 else t).cuda()


def both(M, ql, qr, cache, idx=None):
    """(workspace output, no-alloc output, index status of the no-alloc call)."""
    import torch

    keep = [dev(ql), dev(qr), dev(cache)]
    kw = {}
    status = None
    if idx is not None:
        keep.append(dev(idx.astype(np.int32)))
        status = torch.full((idx.shape[0], 3), 99, dtype=torch.int32, device="cuda")
        kw = dict(indices=keep[3], index_status=status)
    lib = M.load()
    a, out_ws, ws = M.decode_args(keep[0], keep[1], keep[2][..., :512], keep[2][..., 512:], scale=MI.SCALE, **kw)
    assert lib.mr_mla_decode(C.byref(a), M._stream(None)) == M.OK, M.last_error()
    out_na = torch.full_like(out_ws, float("nan"))
    a.out = out_na.data_ptr()
    a.workspace, a.workspace_bytes = None, 0
    assert lib.mr_mla_decode_noalloc(C.byref(a), M._stream(None)) == M.OK, M.last_error()
    torch.cuda.synchronize()
    return out_ws, out_na, status


def test_noalloc_dense_then_smaller():
    import minirun_hip as M

    import torch

    for H, N, tag in ((128, 32768, "na-big"), (16, 512, "na-small")):
        print(f"no-alloc dense H={H} N={N}", flush=True)
        ql, qr, cache = MI.decode_inputs(H, N, tag=tag)
        out_ws, out_na, _ = both(M, ql, qr, cache)
        assert torch.equal(out_ws.view(torch.int16), out_na.view(torch.int16))
        sub = slice(None) if H <= 16 else slice(0, 128, 37)   # oracle on a head subset of the big case
        ref = O.mla_decode(ql[sub], qr[sub], cache)[0]
        ok, maxerr, scale_err = MI.within_tolerance(out_na.float().cpu().numpy()[0][sub], ref)
        assert ok and scale_err < 1e-2, (maxerr, scale_err)


def test_noalloc_sparse_then_smaller():
    import minirun_hip as M

    import torch

    for B, H, N, K, tag in ((4, 128, 131072, 2048, "nas-big"), (2, 32, 5000, 300, "nas-small")):
        print(f"no-alloc sparse B={B} H={H} N={N} K={K}", flush=True)
        ql, qr, cache, idx = MI.sparse_inputs(B, H, N, K, window=min(128, K // 4), tag=tag)
        out_ws, out_na, status = both(M, ql, qr, cache, idx)
        assert torch.equal(out_ws.view(torch.int16), out_na.view(torch.int16))
        assert (status.cpu().numpy() == np.array([0, -1, -1])).all()
        if B == 2:
            st, ref = O.sparse_attention(ql, qr, cache, idx)
            assert st == O.OK
            ok, maxerr, scale_err = MI.within_tolerance(out_na.float().cpu().numpy(), ref)
            assert ok and scale_err < 1e-2, (maxerr, scale_err)


def test_noalloc_refuses_what_it_cannot_hold():
    # beyond the static scratch: a named error, nothing launched; a
    # synchronous index check is refused too (it would read on the host)
    import minirun_hip as M

    import torch

    lib = M.load()
    q = torch.zeros(16, 128, 512, dtype=torch.bfloat16, device="cuda")
    qr = torch.zeros(16, 128, 64, dtype=torch.bfloat16, device="cuda")
    cache = torch.zeros(1024, 576, dtype=torch.bfloat16, device="cuda")
    a, out, ws = M.decode_args(q, qr, cache[:, :512], cache[:, 512:], scale=MI.SCALE, out_dtype=torch.float32,
                               num_splits=16)
    assert lib.mr_mla_decode_workspace_size(C.byref(a)) > M.DECODE_NOALLOC_SCRATCH_BYTES
    assert lib.mr_mla_decode_noalloc(C.byref(a), M._stream(None)) == M.WORKSPACE_TOO_SMALL
    assert "scratch" in M.last_error()
    idx = torch.arange(64, dtype=torch.int32, device="cuda").reshape(1, 64)
    a, out, ws = M.decode_args(q[:1], qr[:1], cache[:, :512], cache[:, 512:], scale=MI.SCALE, indices=idx)
    assert lib.mr_mla_decode_noalloc(C.byref(a), M._stream(None)) == M.INVALID_ARGUMENT
    assert "index_status" in M.last_error()
