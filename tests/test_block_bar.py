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


# ---------------------------------------------------------------- the prefill block's composition
PB_DIMS = dict(hidden=256, q_lora_rank=64, heads=4, nope=32, rope=16, v=32, kv_rank=64)


@pytest.mark.parametrize("affine,rotary,position", [(False, False, 0), (False, False, 9), (True, True, 13)])
def test_prefill_block_one_token_equals_decode_block(affine, rotary, position):
    # one prompt token through the eager (expanded) composition equals the
    # absorbed decode block's composition at the same position
    # (MLA.swift:174-197 against :198-206): keys and values up-projected
    # per head against W_UK absorbed into the query and W_UV applied after
    d = MI.prefill_block_inputs(1, position, f"pb1.{affine}.{position}", affine=affine, input_norm=affine,
                                rotary=rotary, **PB_DIMS)
    got, rows = MI.prefill_block_reference(d, rotary=rotary, **PB_DIMS)
    dd = dict(d, x=d["x"][0])
    ref, row = MI.block_reference(dd, rotary=rotary, **PB_DIMS)
    assert np.abs(rows[0].astype(np.int32) - row.astype(np.int32)).max() <= 1
    ok, maxerr, scale_err = MI.within_block_tolerance(got[0], ref)
    assert ok, (maxerr, scale_err)


def test_prefill_block_reference_is_causal():
    # token t's output and cache row depend on tokens 0..t only: the first 9
    # tokens alone give the first 9 rows of the 23-token prompt, bit for bit
    d = MI.prefill_block_inputs(23, 0, "pbcz", rotary=True, **PB_DIMS)
    full, rows = MI.prefill_block_reference(d, rotary=True, **PB_DIMS)
    d9 = dict(d, x=d["x"][:9])
    part, rows9 = MI.prefill_block_reference(d9, rotary=True, **PB_DIMS)
    np.testing.assert_array_equal(part, full[:9])
    np.testing.assert_array_equal(rows9, rows[:9])
    # and a later token does see the earlier ones
    d_alt = dict(d, x=d["x"].copy())
    d_alt["x"][3] = d["x"][4]
    alt, _ = MI.prefill_block_reference(d_alt, rotary=True, **PB_DIMS)
    assert np.array_equal(alt[:3], full[:3]) and not np.array_equal(alt[5:], full[5:])


def test_prefill_block_sampled_rows_equal_full_reference():
    # the sampled-row form used at 4096 tokens gives the full composition's
    # rows bit for bit
    d = MI.prefill_block_inputs(30, 0, "pbsr", **PB_DIMS)
    full, rows = MI.prefill_block_reference(d, **PB_DIMS)
    sel = [0, 7, 29]
    part, rows2 = MI.prefill_block_reference_rows(d, sel, **PB_DIMS)
    np.testing.assert_array_equal(rows2, rows)
    np.testing.assert_array_equal(part, full[sel])
