"""Pins, on the GPU, the operand layouts the decode kernel is written for:
16x16x32 and 32x32x16 bf16 MFMA and the ds_read_b64_tr_b16 lane mapping.
Inputs are small integers, exact in bf16 and in fp32 accumulation."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def st():
    import minirun_hip as M

    lib = C.CDLL(M.SELFTEST_PATH)
    for n in ("mr_selftest_mfma16", "mr_selftest_mfma32"):
        getattr(lib, n).argtypes = [C.c_void_p] * 4
    lib.mr_selftest_tr16.argtypes = [C.c_void_p] * 4
    return lib


def _bf16(torch, a):
    return torch.tensor(a.astype(np.float32)).to(torch.bfloat16).cuda()


def test_mfma16_layout(st):
    import torch

    print("selftest mfma16", flush=True)
    rng = np.random.default_rng(0)
    A = rng.integers(-4, 5, (16, 32))
    B = rng.integers(-4, 5, (32, 16))
    D = torch.zeros(16, 16, dtype=torch.float32, device="cuda")
    assert st.mr_selftest_mfma16(_bf16(torch, A).data_ptr(), _bf16(torch, B).data_ptr(), D.data_ptr(), None) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(D.cpu().numpy(), (A @ B).astype(np.float32))


def test_mfma32_layout(st):
    import torch

    print("selftest mfma32", flush=True)
    rng = np.random.default_rng(1)
    A = rng.integers(-4, 5, (32, 16))
    B = rng.integers(-4, 5, (16, 32))
    D = torch.zeros(32, 32, dtype=torch.float32, device="cuda")
    assert st.mr_selftest_mfma32(_bf16(torch, A).data_ptr(), _bf16(torch, B).data_ptr(), D.data_ptr(), None) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(D.cpu().numpy(), (A @ B).astype(np.float32))


def test_ds_read_tr16_mapping(st):
    """A 16x64 b16 matrix M[r][c] = 64r + c sits in LDS (row stride 128 B).
    Each 16-lane group g reads the 4x16 block at rows 4g.., cols 16g..: lane j
    addresses row 4g + j/4, cols 16g + 4(j%4).  Expected: lane i of the group
    receives column 16g + i of rows 4g..4g+3."""
    import torch

    print("selftest tr16", flush=True)
    offs = np.zeros(64, np.int32)
    for lane in range(64):
        g, j = lane // 16, lane % 16
        row, col = 4 * g + j // 4, 16 * g + 4 * (j % 4)
        offs[lane] = (row * 64 + col) * 2
    d_offs = torch.tensor(offs, device="cuda")
    out = torch.zeros(64 * 4, dtype=torch.int16, device="cuda")
    assert st.mr_selftest_tr16(offs.ctypes.data, d_offs.data_ptr(), out.data_ptr(), None) == 0
    torch.cuda.synchronize()
    got = out.cpu().numpy().view(np.uint16).reshape(64, 4)
    exp = np.zeros((64, 4), np.uint16)
    for lane in range(64):
        g, i = lane // 16, lane % 16
        for e in range(4):
            exp[lane, e] = (4 * g + e) * 64 + 16 * g + i
    if not np.array_equal(got, exp):
        print("tr16 raw result (lane: 4 values):", file=sys.stderr)
        for lane in range(64):
            print(lane, got[lane].tolist(), file=sys.stderr)
    np.testing.assert_array_equal(got, exp)


def test_permlane32_swap_pairs(st):
    """v_permlane32_swap of two copies of v: lane l gets (v[l], v[l+32]) for
    l < 32 and (v[l-32], v[l]) for l >= 32, the lane-pair exchange the
    decode softmax uses for its max and sum over the two wave halves."""
    import torch

    print("selftest permlane32", flush=True)
    st.mr_selftest_permlane32.argtypes = [C.c_void_p] * 3
    v = np.arange(64, dtype=np.int32) * 7 + 3
    d_in = torch.tensor(v, device="cuda")
    out = torch.zeros(128, dtype=torch.int32, device="cuda")
    assert st.mr_selftest_permlane32(d_in.data_ptr(), out.data_ptr(), None) == 0
    torch.cuda.synchronize()
    r = out.cpu().numpy().reshape(64, 2)
    lanes = np.arange(64)
    lo = np.where(lanes < 32, lanes, lanes - 32)
    np.testing.assert_array_equal(r[:, 0], v[lo])
    np.testing.assert_array_equal(r[:, 1], v[lo + 32])


def test_permlane16_swap_pairs(st):
    """v_permlane16_swap of two copies of v: a lane of row r (16 lanes a row)
    gets (v[l], v[l+16]) for even r and (v[l-16], v[l]) for odd r, the
    exchange the decode softmax uses between lanes l and l ^ 16."""
    import torch

    print("selftest permlane16", flush=True)
    st.mr_selftest_permlane16.argtypes = [C.c_void_p] * 3
    v = np.arange(64, dtype=np.int32) * 5 + 11
    d_in = torch.tensor(v, device="cuda")
    out = torch.zeros(128, dtype=torch.int32, device="cuda")
    assert st.mr_selftest_permlane16(d_in.data_ptr(), out.data_ptr(), None) == 0
    torch.cuda.synchronize()
    r = out.cpu().numpy().reshape(64, 2)
    lanes = np.arange(64)
    lo = np.where((lanes // 16) % 2 == 0, lanes, lanes - 16)
    np.testing.assert_array_equal(r[:, 0], v[lo])
    np.testing.assert_array_equal(r[:, 1], v[lo + 16])


def test_mfma_rate_probe_runs():
    # the bench's on-box MFMA rate probe: plausible rate and clock (wide
    # bounds: a sanity check of the probe, not a performance gate)
    print("selftest mfma rate probe", flush=True)
    import os

    import torch

    import minirun_hip as M

    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench

    r = bench.mfma_probe(torch, M)
    print(r, flush=True)
    assert 100.0 < r["tflops"] < 5000.0, r
    assert 0.5 < r["clock_ghz"] < 3.5, r


def test_permlane16_swap_two_values(st):
    """v_permlane16_swap of two different values a (first operand) and b:
    with rows of 16 lanes, r[0] = (a.row0, b.row0, a.row2, b.row2) and
    r[1] = (a.row1, b.row1, a.row3, b.row3), so max(r[0], r[1]) leaves a's
    pairwise reduction in rows 0 and 2 and b's in rows 1 and 3: the decode
    reduces its two head tiles' maxima and sums in one swap this way."""
    import torch

    print("selftest permlane16 pair", flush=True)
    st.mr_selftest_permlane16_pair.argtypes = [C.c_void_p] * 3
    a = np.arange(64, dtype=np.int32) * 3 + 7
    b = np.arange(64, dtype=np.int32) * 5 + 1000
    d_in = torch.tensor(np.concatenate([a, b]), device="cuda")
    out = torch.zeros(128, dtype=torch.int32, device="cuda")
    assert st.mr_selftest_permlane16_pair(d_in.data_ptr(), out.data_ptr(), None) == 0
    torch.cuda.synchronize()
    r = out.cpu().numpy().reshape(64, 2)
    exp0 = np.empty(64, np.int32)
    exp1 = np.empty(64, np.int32)
    for lane in range(64):
        row, col = lane // 16, lane % 16
        even = 16 * (row & ~1) + col  # the same lane in the pair's even row
        exp0[lane] = a[even] if row % 2 == 0 else b[even]
        exp1[lane] = a[even + 16] if row % 2 == 0 else b[even + 16]
    np.testing.assert_array_equal(r[:, 0], exp0)
    np.testing.assert_array_equal(r[:, 1], exp1)
