"""Parity of the routed-expert affine matmul (affineGatherMM,
AffineWeights.swift:255-318) with the oracle: row (t, j) of the output is
W[rhs[t, j]] . x[t] for a stack of experts, on the fused 4-bit path and the
generic path, with unsorted and repeated expert ids, several tokens, and an
out-of-range id (a zero row).  Bar: the workload bar plus an output-scale
error below 1e-4, as for the single-matrix GEMV."""
import numpy as np
import pytest

import mla_inputs as MI
import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    import minirun_hip as M

    M.load()
    return M


def stack(tag, E, out_f, in_f, bits=4):
    packed = O.u32(f"gx.{tag}.p", (E, out_f, in_f * bits // 32))
    s = O.abs_normal_bf16(f"gx.{tag}.s", (E, out_f, in_f // 64), std=0.01)
    b = O.normal_bf16(f"gx.{tag}.b", (E, out_f, in_f // 64), std=0.01)
    return packed, s, b


def dev(a):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if a.dtype == np.uint16:
        t = t.view(torch.bfloat16)
    elif a.dtype == np.uint32:
        t = t.view(torch.int32)
    return t.cuda()


def oracle_rows(x, w, rhs, E, bits=4):
    T, K = rhs.shape
    out_f = w[0].shape[1]
    ref = np.zeros((T, K, out_f), np.float32)
    for t in range(T):
        for j in range(K):
            e = int(rhs[t, j])
            if 0 <= e < E:
                ref[t, j] = O.affine_matmul(x[t][None], w[0][e], w[1][e], w[2][e], bits=bits, acc=1)[0]
    return ref


def check(got, ref, tag):
    ok, maxerr, scale_err = MI.within_tolerance(got, ref)
    print(f"{tag}: max|d|={maxerr:.3e} scale_err={scale_err:.3e}", flush=True)
    assert ok, f"{tag}: elementwise tolerance violated (max |d| {maxerr})"
    assert scale_err < 1e-4, f"{tag}: output-scale error {scale_err}"


@pytest.mark.parametrize("T,K,out_f,in_f", [(1, 8, 768, 2048), (3, 4, 200, 512), (2, 3, 64, 1536)])
def test_gather_fused_path(M, T, K, out_f, in_f):
    import torch

    E = 6 if T > 1 else 16
    print(f"gather fused T={T} K={K} E={E} {out_f}x{in_f}", flush=True)
    w = stack(f"f{T}.{K}.{out_f}", E, out_f, in_f)
    W = M.AffineWeights(dev(w[0]), dev(w[1]), dev(w[2]))
    assert W.experts == E
    x = O.normal_bf16(f"gx.x.{T}.{in_f}", (T, in_f))
    rhs = np.random.default_rng(T * 100 + K).integers(0, E, size=(T, K)).astype(np.int32)
    rhs[0, -1] = rhs[0, 0]  # a repeated id
    y = M.affine_gather_mm(dev(x), W, torch.from_numpy(rhs).cuda(), out_dtype=torch.float32)
    torch.cuda.synchronize()
    check(y.cpu().numpy(), oracle_rows(O.bf16_to_f32(x), w, rhs, E), f"gather-fused-{T}x{K}")


def test_gather_generic_path_and_bad_id(M):
    import torch

    print("gather generic: f32 x, 8-bit, an id out of range", flush=True)
    E, out_f, in_f = 5, 96, 256
    w = stack("g", E, out_f, in_f, bits=8)
    W = M.AffineWeights(dev(w[0]), dev(w[1]), dev(w[2]), bits=8)
    x = O.bf16_to_f32(O.normal_bf16("gx.gx", (2, in_f)))
    rhs = np.array([[4, 0, 7], [-1, 2, 2]], np.int32)
    y = M.affine_gather_mm(torch.from_numpy(x).cuda(), W, torch.from_numpy(rhs).cuda(), out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert not got[0, 2].any() and not got[1, 0].any()  # ids 7 and -1: zero rows
    check(got, oracle_rows(x, w, rhs, E, bits=8), "gather-generic")


def test_gather_fused_bad_id_is_zero(M):
    import torch

    print("gather fused: an id out of range gives a zero row", flush=True)
    E, out_f, in_f = 3, 128, 1024
    w = stack("z", E, out_f, in_f)
    W = M.AffineWeights(dev(w[0]), dev(w[1]), dev(w[2]))
    x = O.normal_bf16("gx.zx", (1, in_f))
    rhs = np.array([[1, 3, 0, -5]], np.int32)
    y = M.affine_gather_mm(dev(x), W, torch.from_numpy(rhs).cuda(), out_dtype=torch.float32)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    assert not got[0, 1].any() and not got[0, 3].any()
    check(got, oracle_rows(O.bf16_to_f32(x), w, rhs, E), "gather-fused-bad-id")
