"""The composed decode block's parity bar, checked on the CPU against the
oracle: it admits the oracle itself under another accumulation order and
rejects plausible mistakes planted in the oracle's block (query rotary
dropped, scale without the rotary dims, W_UK/W_UV swapped, query rotated at
the wrong position, q_a RMSNorm skipped)."""
import numpy as np
import pytest

import mla_inputs as MI
import oracle as O


def _mm_f32(x, w):
    packed, s, b = w
    return O.affine_matmul(np.asarray(x, np.float32)[None], packed, s, b, acc=0)[0]


@pytest.fixture(scope="module", params=[71, 2048])
def case(request):
    d = MI.block_inputs(ctx=request.param, tag=f"bar{request.param}", centred=True)
    ref, _ = MI.block_reference(d)
    return d, ref


def test_bar_admits_reordered_oracle(case, monkeypatch):
    d, ref = case
    monkeypatch.setattr(MI, "_mm", _mm_f32)
    alt, _ = MI.block_reference(d)
    assert not np.array_equal(alt, ref)   # the reordering does change bits
    ok, maxerr, scale_err = MI.within_block_tolerance(alt, ref)
    assert ok, (maxerr, scale_err)


@pytest.mark.parametrize("plant", MI.PLANTS)
def test_bar_rejects_planted_mistakes(case, plant):
    d, ref = case
    bad, _ = MI.block_reference(d, plant=plant)
    ok, maxerr, scale_err = MI.within_block_tolerance(bad, ref)
    assert not ok, (plant, maxerr, scale_err)
    assert scale_err > 5e-2, (plant, scale_err)


def test_workload_weights_hide_common_mode():
    # the block workload's literal weights (biases N(0,0.01)) give outputs
    # dominated by the mean weight; the centred kind does not
    lit, _ = MI.block_reference(MI.block_inputs(ctx=8, tag="cm"))
    cen, _ = MI.block_reference(MI.block_inputs(ctx=8, tag="cm", centred=True))
    assert np.abs(lit).mean() > 100 * np.abs(cen).mean()
