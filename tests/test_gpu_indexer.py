"""Parity of the device lightning-index scores (DeepSeekV4LightningIndexer.
scores, DeepSeekV4Attention.swift:530-549) with the oracle: the MFMA kernel
(bf16 inputs, D = 128, 16..64 heads) and the generic kernel (f32 inputs,
other shapes), partial key tiles, several query tokens, strided operands,
NaN propagation, and the selection run on the device scores.

Bar: |hip - oracle| <= 1e-2 + 2e-2 |oracle| elementwise (the workload bar)
and an output-scale error below 1e-5: the products of bf16 inputs are exact
in fp32 and only the order of the fp32 sums differs."""
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


def inputs(tag, S, H, D, T):
    q = O.normal_bf16(f"ix.{tag}.q", (S, H, D))
    k = O.normal_bf16(f"ix.{tag}.k", (T, D))
    w = O.bf16_to_f32(O.normal_bf16(f"ix.{tag}.w", (S, H), std=float((D * H) ** -0.5)))
    return q, k, w


def bf16_dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).view(torch.bfloat16).cuda()


def f32_dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def check(got, ref, tag):
    ok, maxerr, scale_err = MI.within_tolerance(got, ref)
    print(f"{tag}: max|d|={maxerr:.3e} scale_err={scale_err:.3e}", flush=True)
    assert ok, f"{tag}: elementwise tolerance violated (max |d| {maxerr})"
    assert scale_err < 1e-5, f"{tag}: output-scale error {scale_err}"


@pytest.mark.parametrize("S,H,T", [(1, 64, 32768), (1, 64, 1000), (3, 64, 257), (2, 16, 130), (1, 32, 128),
                                   (1, 48, 1)])
def test_mfma_path(M, S, H, T):
    import torch

    print(f"indexer mfma S={S} H={H} D=128 T={T}", flush=True)
    q, k, w = inputs(f"m{S}.{H}.{T}", S, H, 128, T)
    got = M.lightning_index_scores(bf16_dev(q), bf16_dev(k), f32_dev(w))
    torch.cuda.synchronize()
    ref = O.indexer_scores(O.bf16_to_f32(q), O.bf16_to_f32(k), w)
    check(got.cpu().numpy(), ref, f"indexer-mfma-{S}x{H}x{T}")


def test_generic_path_f32_and_odd_shapes(M):
    import torch

    print("indexer generic: f32 q/k, D=96, H=8, bf16 weights", flush=True)
    q, k, w = inputs("g", 2, 8, 96, 77)
    wb = O.f32_to_bf16(w)
    got = M.lightning_index_scores(f32_dev(O.bf16_to_f32(q)), f32_dev(O.bf16_to_f32(k)), bf16_dev(wb))
    torch.cuda.synchronize()
    ref = O.indexer_scores(O.bf16_to_f32(q), O.bf16_to_f32(k), O.bf16_to_f32(wb))
    check(got.cpu().numpy(), ref, "indexer-generic")


def test_strided_operands(M):
    """Queries and keys as views with padded rows (the MFMA path's strides)."""
    import torch

    print("indexer strided: q head stride 136, key stride 144", flush=True)
    q, k, w = inputs("s", 2, 32, 128, 300)
    qp = np.zeros((2, 32, 136), np.uint16)
    qp[:, :, :128] = q
    kp = np.zeros((300, 144), np.uint16)
    kp[:, :128] = k
    out = torch.full((2, 320), float("nan"), dtype=torch.float32, device="cuda")
    M.lightning_index_scores(bf16_dev(qp)[:, :, :128], bf16_dev(kp)[:, :128], f32_dev(w), out=out[:, :300])
    torch.cuda.synchronize()
    ref = O.indexer_scores(O.bf16_to_f32(q), O.bf16_to_f32(k), w)
    o = out.cpu().numpy()
    check(o[:, :300], ref, "indexer-strided")
    assert np.isnan(o[:, 300:]).all()  # nothing written past the keys


def test_nan_propagates_to_the_selection(M):
    import torch

    print("indexer NaN key -> NaN score -> selection error", flush=True)
    q, k, w = inputs("n", 1, 64, 128, 512)
    k = k.copy()
    k[5, 3] = 0x7FC0  # bf16 NaN
    got = M.lightning_index_scores(bf16_dev(q), bf16_dev(k), f32_dev(w))
    torch.cuda.synchronize()
    g = got.cpu().numpy()
    assert np.isnan(g[0, 5]) and np.isfinite(np.delete(g[0], 5)).all()
    with pytest.raises(M.MRError) as e:
        M.lightning_select(got, 64, 4, 2047, 0)
    assert "NaN" in e.value.message


def test_scores_feed_the_selection(M):
    """One decode token's pipeline: scores of 32768 compressed keys, then the
    top-2048 selection on them, bit-exact against the oracle's selection of
    the same device scores."""
    import torch

    print("indexer -> top-2048 of 32768", flush=True)
    q, k, w = inputs("p", 1, 64, 128, 32768)
    got = M.lightning_index_scores(bf16_dev(q), bf16_dev(k), f32_dev(w))
    sel = M.lightning_select(got, 2048, 4, 131071, 7)
    torch.cuda.synchronize()
    st, exp = O.topk_select(got.cpu().numpy(), 2048, 4, 131071, 7)
    assert st == O.OK
    np.testing.assert_array_equal(sel.cpu().numpy(), exp)
