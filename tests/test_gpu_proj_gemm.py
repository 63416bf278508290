"""Token-tiled projections on MFMA: mr_linear (k3Linear, Linear.swift:55-57)
and mr_affine_matmul (affineMM, AffineWeights.swift:239-254) at 64 or more
tokens, against the oracle (fp64 accumulation of the exact fp32 weights).

At T = 4096 the oracle runs on sampled rows (both ends of the first and last
tiles, tile boundaries, a few seeded rows) and every column; the smaller
cases check every output.  Bar: |hip - oracle| <= 1e-2 + 2e-2 |oracle|
elementwise (mla_inputs.within_tolerance), plus the output-scale error.
"""
import numpy as np
import pytest

import mla_inputs as MI
import oracle as O
from test_gpu_block import check, dev, f32, sync

pytestmark = pytest.mark.gpu

T_FULL = 4096


@pytest.fixture(scope="module")
def M():
    import minirun_hip as M

    M.load()
    return M


def sample_rows(t, seed):
    rows = {0, 1, 127, 128, 255, 256, t // 2, t - 2, t - 1}
    rng = np.random.default_rng(seed)
    rows.update(int(r) for r in rng.integers(0, t, 4))
    return np.array(sorted(r for r in rows if r < t))


# K3 (dense bf16, 96 heads) projection shapes: q_a, o_proj, kv_a, q_b
@pytest.mark.parametrize("out_f,in_f", [(1536, 7168), (7168, 12288), (576, 7168), (18432, 1536)])
@pytest.mark.parametrize("ydt", ["f32", "bf16"])
def test_linear_mfma_k3_shapes(M, out_f, in_f, ydt):
    print(f"linear mfma T={T_FULL} [{out_f}, {in_f}] y={ydt}", flush=True)
    import torch

    w = O.normal_bf16(f"pg.lin.{out_f}.{in_f}", (out_f, in_f), std=in_f ** -0.5, threads=16)
    x = O.normal_bf16(f"pg.lin.x.{in_f}", (T_FULL, in_f), threads=16)
    y = M.linear(dev(x), M.DenseWeights(dev(w)), out_dtype=torch.float32 if ydt == "f32" else torch.bfloat16)
    sync()
    rows = sample_rows(T_FULL, out_f)
    ref = O.linear(O.bf16_to_f32(x[rows]), w, acc=1, threads=16)
    check(f32(y)[rows], ref, f"linear-mfma-{out_f}x{in_f}-{ydt}", scale_bar=1e-5 if ydt == "f32" else 1e-2)


# cfg-5 affine 4-bit projection shapes (group 64, bf16 scales): q_a, q_b, kv_a, o_proj
@pytest.mark.parametrize("name,out_f,in_f", [("q_a", 1536, 7168), ("q_b", 24576, 1536), ("kv_a", 576, 7168),
                                             ("o_proj", 7168, 16384)])
@pytest.mark.parametrize("centred", [False, True])
def test_affine_mfma_block_shapes(M, name, out_f, in_f, centred):
    print(f"affine mfma T={T_FULL} {name} [{out_f}, {in_f}] centred={centred}", flush=True)
    import torch

    w = MI.affine_weight(f"pg.{name}", out_f, in_f, centred=centred)
    x = O.normal_bf16(f"pg.{name}.x", (T_FULL, in_f), threads=16)
    wt = M.AffineWeights(dev(w[0]), dev(w[1]), dev(w[2]))
    y = M.affine_mm(dev(x), wt, out_dtype=torch.float32)
    yb = M.affine_mm(dev(x), wt, out_dtype=torch.bfloat16)
    sync()
    rows = sample_rows(T_FULL, in_f)
    ref = O.affine_matmul(O.bf16_to_f32(x[rows]), *w, acc=1, threads=16)
    tag = f"affine-mfma-{name}{'-centred' if centred else ''}"
    check(f32(y)[rows], ref, tag, scale_bar=1e-5)
    check(f32(yb)[rows], ref, tag + "-bf16", scale_bar=1e-2)


def affine_operand(tag, out_f, in_f, group, sdt):
    """4-bit operand with scales / biases in dtype sdt ("bf16", "f16", "f32"),
    as the oracle's arrays and the device tensors."""
    import torch

    packed = O.u32(f"{tag}.p", (out_f, in_f // 8))
    s = O.bf16_to_f32(O.abs_normal_bf16(f"{tag}.s", (out_f, in_f // group), std=0.01))
    b = O.bf16_to_f32(O.normal_bf16(f"{tag}.b", (out_f, in_f // group), std=0.01))
    if sdt == "bf16":
        sa, ba, code = O.f32_to_bf16(s), O.f32_to_bf16(b), O.BF16
        ts, tb = dev(sa), dev(ba)
    elif sdt == "f16":
        sa, ba, code = np.float16(s).view(np.uint16), np.float16(b).view(np.uint16), O.F16
        ts, tb = torch.from_numpy(sa).view(torch.float16).cuda(), torch.from_numpy(ba).view(torch.float16).cuda()
    else:
        sa, ba, code = (s * 1.37).astype(np.float32), (b * 0.71).astype(np.float32), O.F32
        ts, tb = torch.from_numpy(sa).cuda(), torch.from_numpy(ba).cuda()
    return packed, sa, ba, code, ts, tb


@pytest.mark.parametrize("tokens,out_f,in_f,group,sdt,x_pad,ydt", [
    (64, 256, 512, 64, "bf16", 0, "f32"),      # the smallest token count the MFMA path takes
    (100, 200, 512, 32, "f16", 8, "f32"),      # ragged M and N tiles, padded x rows, group 32
    (65, 1000, 832, 64, "bf16", 0, "bf16"),    # one row into a second M tile, 13 groups
    (300, 264, 4096, 128, "f32", 16, "f32"),   # group 128 spans four k-tiles, f32 scales
    (513, 8, 96, 32, "bf16", 0, "bf16"),       # one output chunk, three k-tiles
])
def test_affine_mfma_edges(M, tokens, out_f, in_f, group, sdt, x_pad, ydt):
    print(f"affine mfma edges T={tokens} [{out_f}, {in_f}] g={group} scales={sdt} pad={x_pad} y={ydt}", flush=True)
    import torch

    packed, sa, ba, code, ts, tb = affine_operand(f"pge.{tokens}.{out_f}.{in_f}", out_f, in_f, group, sdt)
    x = O.normal_bf16(f"pge.x.{tokens}.{in_f}", (tokens, in_f + x_pad))
    xt = dev(x)[:, :in_f]
    w = M.AffineWeights(dev(packed), ts, tb, group_size=group)
    y = M.affine_mm(xt, w, out_dtype=torch.float32 if ydt == "f32" else torch.bfloat16)
    sync()
    ref = O.affine_matmul(O.bf16_to_f32(x[:, :in_f]), packed, sa, ba, group=group, scale_dtype=code, acc=1)
    check(f32(y), ref, f"affine-mfma-edge-{tokens}x{out_f}x{in_f}", scale_bar=1e-5 if ydt == "f32" else 1e-2)


@pytest.mark.parametrize("tokens,out_f,in_f,x_pad,ydt", [
    (64, 256, 512, 0, "f32"), (100, 200, 512, 8, "f32"), (65, 1000, 832, 0, "bf16"), (513, 8, 128, 0, "bf16"),
    (257, 264, 1024, 24, "f32"),
])
def test_linear_mfma_edges(M, tokens, out_f, in_f, x_pad, ydt):
    print(f"linear mfma edges T={tokens} [{out_f}, {in_f}] pad={x_pad} y={ydt}", flush=True)
    import torch

    w = O.normal_bf16(f"ple.{out_f}.{in_f}", (out_f, in_f), std=in_f ** -0.5)
    x = O.normal_bf16(f"ple.x.{tokens}.{in_f}", (tokens, in_f + x_pad))
    y = M.linear(dev(x)[:, :in_f], M.DenseWeights(dev(w)), out_dtype=torch.float32 if ydt == "f32" else torch.bfloat16)
    sync()
    ref = O.linear(O.bf16_to_f32(x[:, :in_f]), w, acc=1)
    check(f32(y), ref, f"linear-mfma-edge-{tokens}x{out_f}x{in_f}", scale_bar=1e-5 if ydt == "f32" else 1e-2)


def test_mfma_path_matches_token_tile_path(M):
    """The same rows through the MFMA path (T = 128) and the token-tile GEMV
    (the first 8 rows alone): both inside the bar of the oracle, and within
    fp32 rounding of each other."""
    import torch

    w = MI.affine_weight("pgm.q_a", 1536, 7168)
    x = O.normal_bf16("pgm.x", (128, 7168))
    wt = M.AffineWeights(dev(w[0]), dev(w[1]), dev(w[2]))
    y_big = f32(M.affine_mm(dev(x), wt, out_dtype=torch.float32))
    y_small = f32(M.affine_mm(dev(x[:8]), wt, out_dtype=torch.float32))
    sync()
    ref = O.affine_matmul(O.bf16_to_f32(x[:8]), *w, acc=1)
    check(y_big[:8], ref, "mfma-rows", scale_bar=1e-5)
    check(y_small, ref, "gemv-rows", scale_bar=1e-5)
    np.testing.assert_allclose(y_big[:8], y_small, rtol=1e-4, atol=1e-3)
