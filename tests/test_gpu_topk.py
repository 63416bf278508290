"""Parity of the device lightning-indexer selection
(DeepSeekV4LightningIndexer.selecting, DeepSeekV4Attention.swift:582-645)
with the oracle: bit-exact indices, including ties (ascending key id),
masked keys (-1), -0 == +0, infinities, NaN reporting and the edge sizes."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    import minirun_hip as M

    M.load()
    return M


def dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def compare(M, scores, top_k, ratio, start_pos, offset, tag):
    print(f"topk {tag}: rows={scores.shape[0]} cols={scores.shape[1]} k={top_k} ratio={ratio} start={start_pos}",
          flush=True)
    st, exp = O.topk_select(scores, top_k, ratio, start_pos, offset)
    assert st == O.OK
    got = M.lightning_select(dev(scores), top_k, ratio, start_pos, offset).cpu().numpy()
    assert got.shape == exp.shape
    np.testing.assert_array_equal(got, exp)


def normal(tag, shape):
    return O.bf16_to_f32(O.normal_bf16(tag, shape)) * np.float32(1.37)


def test_decode_row_top2048_of_32768(M):
    # one decode token at position 131071, ratio 4: 32768 compressed keys
    compare(M, normal("tk.dec", (1, 32768)), 2048, 4, 131071, 0, "decode")


def test_ties_break_by_ascending_key(M):
    s = np.floor(normal("tk.ties", (1, 5000)) * 2).astype(np.float32)  # ~10 distinct values
    compare(M, s, 1000, 1, 4999, 7, "ties")
    s2 = np.zeros((1, 3000), np.float32)  # one value everywhere
    compare(M, s2, 512, 1, 2999, 0, "all-equal")


def test_signed_zero_and_infinities(M):
    s = normal("tk.inf", (1, 4096))
    s[0, ::7] = 0.0
    s[0, 3::7] = -0.0
    s[0, 5::97] = np.inf
    s[0, 6::89] = -np.inf
    compare(M, s, 1024, 1, 4095, 0, "zeros-infs")
    s2 = np.full((1, 600), -np.inf, np.float32)  # visible -inf ties masked keys by key id
    compare(M, s2, 100, 1, 599, 0, "all-minus-inf")


@pytest.mark.parametrize("rows,cols,top_k,ratio,offset", [(300, 75, 16, 4, 128), (64, 64, 64, 1, 0),
                                                          (17, 40, 100, 2, 3), (4096, 1024, 512, 4, 0)])
def test_prefill_rows_with_masking(M, rows, cols, top_k, ratio, offset):
    compare(M, normal(f"tk.pf{rows}", (rows, cols)), top_k, ratio, 0, offset, "prefill")


def test_limits(M):
    compare(M, normal("tk.max", (1, 65535)), 4096, 1, 65534, 0, "two-slices")
    compare(M, normal("tk.one", (1, 1)), 1, 1, 0, 0, "one-key")


def test_v4_full_size_row(M):
    # DeepSeek V4: max_position_embeddings 1048576 at compression ratio 4
    # (Tests/Fixtures/deepseek-v4/current-official-config.json:22) -> 262144
    # compressed keys for the last token: 8 slices of 32768, 3 merge rounds
    compare(M, normal("tk.v4", (1, 262144)), 2048, 4, 1048575, 0, "v4-262144")
    compare(M, normal("tk.v4k", (1, 262144)), 4096, 4, 1048575, 5, "v4-262144-k4096")


def test_slices_ties_odd_counts_and_masking(M):
    # ties across slice boundaries break by ascending key id; three slices
    # (an odd list passes a merge round unmerged); keys past `visible`
    # (-1) when the row has more columns than the position ranks
    s = np.floor(normal("tk.sl", (1, 70000)) * 2).astype(np.float32)   # ~10 distinct values
    compare(M, s, 3000, 1, 69999, 11, "ties-3-slices")
    compare(M, normal("tk.sl2", (1, 100000)), 1000, 1, 80000, 0, "cols-past-available")
    # a short last slice: 32768 + 5 keys, top_k larger than that slice
    compare(M, normal("tk.sl3", (1, 32773)), 2048, 1, 32772, 0, "short-last-slice")
    z = np.zeros((1, 98304), np.float32)   # one value everywhere: the first keys win
    compare(M, z, 4096, 1, 98303, 0, "all-equal-3-slices")


def test_more_than_4096_selected(M):
    # `selecting` takes any topK (DeepSeekV4Attention.swift:582-645): more
    # than 4096 keys run as slices of 4096 that each sort all their keys,
    # then merge rounds whose lists double up to top_k
    compare(M, normal("tk.big1", (1, 70000)), 10000, 1, 69999, 3, "k10000-of-70000")
    compare(M, normal("tk.big2", (1, 262144)), 16384, 4, 1048575, 0, "k16384-of-262144")
    s = np.floor(normal("tk.big3", (1, 20000)) * 2).astype(np.float32)   # ~10 distinct values
    compare(M, s, 8000, 1, 19999, 0, "k8000-ties")
    compare(M, np.zeros((1, 9000), np.float32), 9000, 1, 8999, 0, "all-equal-every-key")
    compare(M, normal("tk.big4", (1, 12000)), 5000, 1, 9000, 0, "k5000-cols-past-available")


def test_more_than_4096_selected_prefill_rows(M):
    # prefill rows (start position 0): row r sees keys 0 .. r, the rest -1
    compare(M, normal("tk.bigpf", (4200, 4200)), 4150, 1, 0, 0, "prefill-k4150")


def test_nan_in_a_late_slice_is_reported(M):
    import torch

    import minirun_hip as MH

    s = normal("tk.nanl", (1, 140000))
    s[0, 139999] = np.nan   # past the last ranked key of a 131072-key row
    with pytest.raises(MH.MRError) as e:
        M.lightning_select(dev(s), 256, 1, 131071, 0)
    assert e.value.status == MH.NONFINITE
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    M.lightning_select(dev(normal("tk.nanok", (1, 140000))), 256, 1, 131071, 0, check=False, status=status)
    assert int(status.item()) == 0
    # the same with more than 4096 selected keys (slices of 4096): a NaN in a
    # middle slice, and one past the ranked keys, through the device status
    for col in (50000, 139999):
        s = normal("tk.nanb", (1, 140000))
        s[0, col] = np.nan
        status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
        M.lightning_select(dev(s), 6000, 1, 131071, 0, check=False, status=status)
        assert int(status.item()) == MH.NONFINITE, col


def test_nan_is_reported(M):
    import torch

    import minirun_hip as MH

    s = normal("tk.nan", (3, 64))
    s[2, 63] = np.nan  # outside the visible keys of every row: still an error
    with pytest.raises(MH.MRError) as e:
        M.lightning_select(dev(s), 8, 1, 0, 0)
    assert e.value.status == MH.NONFINITE and "NaN" in e.value.message
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    M.lightning_select(dev(s), 8, 1, 0, 0, check=False, status=status)
    assert int(status.item()) == MH.NONFINITE
    M.lightning_select(dev(normal("tk.ok", (3, 64))), 8, 1, 0, 0, check=False, status=status)
    assert int(status.item()) == 0


@pytest.mark.parametrize("kind", ["uniform", "quantized", "heavy-tail"])
def test_decode_row_score_distributions(M, kind):
    # 2048 of 32768 keys for score distributions whose selected keys fill
    # the order buckets differently: spread evenly (uniform), many keys per
    # bucket and exact ties (values on a 1/512 grid), and a long tail
    # (exponential magnitudes) where a few buckets hold most keys
    u = O.bf16_to_f32(O.normal_bf16(f"tk.dist.{kind}", (1, 32768))).astype(np.float64)
    if kind == "uniform":
        s = (0.5 * (1.0 + np.tanh(u))).astype(np.float32)
    elif kind == "quantized":
        s = (np.round(u * 512.0) / 512.0).astype(np.float32)
    else:
        s = np.exp(np.abs(u) * 3.0).astype(np.float32)
    compare(M, s, 2048, 4, 131071, 0, f"dist-{kind}")


def test_spread_selection_branches(M):
    # one decode row over many workgroups, through each ordering branch:
    # half of the keys taken with the cut below zero (the taken composites
    # span both signs, buckets fill up and each full one is sorted by a
    # wave), a row whose keys through the cut value exceed the sort buffer
    # (a radix select among the cut value's keys first), and a short last
    # slice
    compare(M, normal("tk.half", (1, 8192)) - np.float32(0.25), 4096, 1, 8191, 0, "half-8192")
    compare(M, normal("tk.half2", (1, 4097)) - np.float32(0.25), 2048, 1, 4096, 3, "half-4097")
    compare(M, normal("tk.sel", (1, 65536)), 4096, 1, 65535, 0, "select-65536-k4096")
    compare(M, normal("tk.short", (1, 6145)), 1000, 1, 6144, 0, "short-last-slice-6145")


def test_spread_nan_among_ranked_keys(M):
    import torch

    import minirun_hip as MH

    s = normal("tk.nanmid", (1, 32768))
    s[0, 12345] = np.nan
    with pytest.raises(MH.MRError) as e:
        M.lightning_select(dev(s), 2048, 4, 131071, 0)
    assert e.value.status == MH.NONFINITE
    status = torch.full((1,), -1, dtype=torch.int32, device="cuda")
    M.lightning_select(dev(s), 2048, 4, 131071, 0, check=False, status=status)
    assert int(status.item()) == MH.NONFINITE


@pytest.mark.parametrize("cols,top_k", [(8192, 4096), (32768, 2048), (16384, 4096)])
def test_spread_heavy_ties(M, cols, top_k):
    # rows where one value holds a large share of the keys: rectified scores
    # (about half the keys exactly 0, and the cut falls among them when half
    # are taken) and a row of one value everywhere (every key ties, so the
    # selection is the first top_k key ids)
    s = np.maximum(normal(f"tk.relu.{cols}", (1, cols)), np.float32(0.0))
    compare(M, s, top_k, 1, cols - 1, 0, f"relu-{cols}-k{top_k}")
    compare(M, np.zeros((1, cols), np.float32), top_k, 1, cols - 1, 0, f"zeros-{cols}-k{top_k}")
    compare(M, np.full((1, cols), np.float32(-2.5)), top_k, 1, cols - 1, 5, f"equal-{cols}-k{top_k}")
    # two adjacent values share the leading keys (one order bucket, and one
    # bucket again over its own span) above a spread tail
    two = normal(f"tk.two.{cols}", (1, cols)) * np.float32(0.1)
    lead = O.bf16_to_f32(O.normal_bf16(f"tk.twosel.{cols}", (1, cols))) > 0.3
    two[lead] = np.where(np.arange(cols)[lead[0]] % 3 == 0, np.float32(1.0), np.nextafter(np.float32(1.0), np.float32(0)))
    compare(M, two, top_k, 1, cols - 1, 0, f"two-values-{cols}-k{top_k}")


def test_spread_ties_full_size(M):
    # rows of the largest spread size (128 slices): rectified scores with
    # the cut among the positives, then with about 500 positive keys, so
    # the cut falls among 260,000 zeros (candidates streamed from the
    # slices, selected by key id)
    big = np.maximum(normal("tk.relu.262144", (1, 262144)), np.float32(0.0))
    compare(M, big, 2048, 1, 262143, 0, "relu-262144")
    big[0, :261000] = 0.0
    compare(M, big, 2048, 1, 262143, 0, "relu-262144-mostly-zero")
    compare(M, np.zeros((1, 262144), np.float32), 4096, 1, 262143, 0, "zeros-262144-k4096")
