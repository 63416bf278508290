"""The oracle's lightning-index scores (DeepSeekV4Attention.swift:530-549,
scores = sum_h w * max(q . k, 0) in fp32) pinned without the reference's
MLX: an fp64 numpy brute force, and properties a wrong term, sign or index
would break (zero weights, all-negative dots, linearity in the weights,
positive scaling of the keys, NaN propagation, heads swapped with their
weights)."""
import numpy as np
import pytest

import oracle as O


def data(S, H, D, T, seed):
    r = np.random.default_rng(seed)
    q = O.bf16_to_f32(O.f32_to_bf16(r.standard_normal((S, H, D)).astype(np.float32)))
    k = O.bf16_to_f32(O.f32_to_bf16(r.standard_normal((T, D)).astype(np.float32)))
    w = (r.standard_normal((S, H)) / np.sqrt(D * H)).astype(np.float32)
    return q, k, w


def brute(q, k, w):
    d = np.einsum("shd,td->sht", q.astype(np.float64), k.astype(np.float64))
    return (np.maximum(d, 0.0) * w.astype(np.float64)[:, :, None]).sum(axis=1)


@pytest.mark.parametrize("S,H,D,T", [(1, 64, 128, 300), (3, 16, 32, 17), (2, 5, 7, 1)])
def test_matches_fp64_brute_force(S, H, D, T):
    q, k, w = data(S, H, D, T, 11)
    got = O.indexer_scores(q, k, w)
    ref = brute(q, k, w)
    assert got.shape == (S, T)
    assert np.abs(got - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


def test_properties():
    q, k, w = data(2, 8, 16, 40, 12)
    base = O.indexer_scores(q, k, w)
    # zero weights -> zero scores
    assert not O.indexer_scores(q, k, np.zeros_like(w)).any()
    # every dot negative -> the ReLU zeroes every head
    qn = -np.abs(q)
    assert not O.indexer_scores(qn, np.abs(k), w).any()
    # linear in the weights (exact for a power of two)
    assert np.array_equal(O.indexer_scores(q, k, 2 * w), 2 * base)
    # keys scaled by a positive power of two scale the scores alike
    assert np.array_equal(O.indexer_scores(q, 4 * k, w), 4 * base)
    # permuting heads together with their weights leaves the scores (up to order)
    perm = np.random.default_rng(3).permutation(8)
    assert np.allclose(O.indexer_scores(q[:, perm], k, w[:, perm]), base, rtol=1e-6, atol=1e-7)
    # a head's weight alone selects that head's ReLU'd dot
    one = np.zeros_like(w)
    one[1, 3] = 1.0
    d = np.maximum(q[1, 3] @ k.T, 0)
    assert np.allclose(O.indexer_scores(q, k, one)[1], d, rtol=1e-6, atol=1e-6)


def test_nan_propagates():
    q, k, w = data(1, 4, 8, 6, 13)
    k[2, 0] = np.nan
    got = O.indexer_scores(q, k, w)
    assert np.isnan(got[0, 2]) and np.isfinite(np.delete(got[0], 2)).all()
