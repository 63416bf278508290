"""Parity of the HIP MLA decode / sparse decode against the CPU oracle.

Bar (stated by the workload spec): |hip - oracle| <= 1e-2 + 2e-2 |oracle|
elementwise on bf16 outputs (fp32 accumulation), plus the reference's
output-scale metric max|d| / max|ref| (MacReferenceLogits.swift:29-34),
gated here at 1e-2.  The oracle is fp64 on the same bf16 inputs.
"""
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


def dev(a, dtype=None):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if a.dtype == np.uint16:
        t = t.view(torch.bfloat16)
    return t.cuda() if dtype is None else t.to(dtype).cuda()


def host_f32(t):
    import torch

    return t.float().cpu().numpy()


def check(got, ref, tag, scale_bar=1e-2):
    ok, maxerr, scale_err = MI.within_tolerance(got, ref)
    print(f"{tag}: max|d|={maxerr:.3e} scale_err={scale_err:.3e}", flush=True)
    assert ok, f"{tag}: elementwise tolerance violated (max |d| {maxerr})"
    assert scale_err < scale_bar, f"{tag}: output-scale error {scale_err}"


def run_decode(M, q_lat, q_rope, cache, **kw):
    import torch

    c = dev(cache)
    out = M.mla_decode(dev(q_lat), dev(q_rope), c[..., :512], c[..., 512:], scale=MI.SCALE, **kw)
    torch.cuda.synchronize()
    return out


def test_decode_16_heads_512_ctx(M):
    print("decode H=16 N=512", flush=True)
    ql, qr, cache = MI.decode_inputs(16, 512, tag="c1", rope=False)
    ref = O.mla_decode(ql, qr, cache)[0]
    out = run_decode(M, ql, qr, cache)
    check(host_f32(out)[0], ref, "decode-16x512")


def test_decode_128_heads_32k(M):
    print("decode H=128 N=32768", flush=True)
    ql, qr, cache = MI.decode_inputs(128, 32768, tag="c2")
    ref = O.mla_decode(ql, qr, cache)[0]
    out = run_decode(M, ql, qr, cache)
    check(host_f32(out)[0], ref, "decode-128x32768")
    out32 = run_decode(M, ql, qr, cache, out_dtype=__import__("torch").float32)
    check(host_f32(out32)[0], ref, "decode-128x32768-f32", scale_bar=2e-3)


def test_bf16_output_tracks_f32_output(M):
    # bf16 output combines bf16 split partials (O_s / l_s), f32 output f32
    # ones; the two differ by the partials' rounding (2^-9 of a partial, each
    # a convex combination of rows) plus the final rounding (2^-9 of the
    # output): within 2^-8 |a| + 2^-8 max|a|
    print("decode bf16 vs f32 output", flush=True)
    import torch

    ql, qr, cache = MI.decode_inputs(128, 8192, tag="rne")
    a = host_f32(run_decode(M, ql, qr, cache, out_dtype=torch.float32)).astype(np.float64)
    b = host_f32(run_decode(M, ql, qr, cache)).astype(np.float64)
    err = np.abs(b - a)
    assert (err <= 2.0 ** -8 * (np.abs(a) + np.abs(a).max())).all(), err.max()
    # and one split: the single partial is O / l itself, so the bf16 output
    # is the f32 output's bf16 rounding up to one ulp
    a1 = host_f32(run_decode(M, ql, qr, cache, num_splits=1, out_dtype=torch.float32))
    b1 = run_decode(M, ql, qr, cache, num_splits=1).cpu().view(torch.int16).numpy().view(np.uint16)
    d = np.abs(b1.astype(np.int32) - O.f32_to_bf16(a1).astype(np.int32))
    assert d.max() <= 1, d.max()


@pytest.mark.parametrize("splits", [1, 2, 7, 64])
def test_split_count_invariance(M, splits):
    print(f"decode split invariance splits={splits}", flush=True)
    import torch

    ql, qr, cache = MI.decode_inputs(128, 4096, tag="sp")
    ref = O.mla_decode(ql, qr, cache)[0]
    out = run_decode(M, ql, qr, cache, num_splits=splits, out_dtype=torch.float32)
    check(host_f32(out)[0], ref, f"splits={splits}", scale_bar=2e-3)


# 48, 96 and 144 heads run in head groups of 48 (no padding heads)
@pytest.mark.parametrize("H,N", [(1, 1), (5, 63), (33, 65), (128, 1000), (64, 64), (48, 129), (96, 3000),
                                 (144, 700)])
def test_ragged_shapes(M, H, N):
    print(f"decode ragged H={H} N={N}", flush=True)
    import torch

    ql, qr, cache = MI.decode_inputs(H, N, tag=f"rg{H}_{N}")
    ref = O.mla_decode(ql, qr, cache)[0]
    out = run_decode(M, ql, qr, cache, out_dtype=torch.float32)
    check(host_f32(out)[0], ref, f"H={H},N={N}", scale_bar=2e-3)
    if N == 1:
        np.testing.assert_allclose(host_f32(out)[0], np.broadcast_to(O.bf16_to_f32(cache[0, :512]), (H, 512)),
                                   rtol=1e-6)


def test_separate_latent_and_rope_arrays(M):
    # the reference's State keeps two arrays, [P,512] and [P,64] (MLA.swift:28-36)
    print("decode two-array cache", flush=True)
    import torch

    ql, qr, cache = MI.decode_inputs(32, 777, tag="two")
    lat = dev(np.ascontiguousarray(cache[:, :512]))
    rk = dev(np.ascontiguousarray(cache[:, 512:]))
    out = M.mla_decode(dev(ql), dev(qr), lat, rk, scale=MI.SCALE, out_dtype=torch.float32)
    torch.cuda.synchronize()
    check(host_f32(out)[0], O.mla_decode(ql, qr, cache)[0], "two-array", scale_bar=2e-3)


# ---------------------------------------------------------------- sparse
def run_sparse(M, q_lat, q_rope, cache, idx, sinks=None, **kw):
    import torch

    out = M.sparse_attention(dev(q_lat), dev(q_rope) if q_rope is not None else None, dev(cache),
                             dev(idx), scale=MI.SCALE, sinks=None if sinks is None else dev(sinks), **kw)
    torch.cuda.synchronize()
    return out


def test_sparse_top2048_128k(M):
    print("sparse B=4 H=128 N=131072 K=2048", flush=True)
    ql, qr, cache, idx = MI.sparse_inputs(4, 128, 131072, 2048)
    st, ref = O.sparse_attention(ql, qr, cache, idx)
    assert st == O.OK
    out = run_sparse(M, ql, qr, cache, idx)
    check(host_f32(out), ref, "sparse-4x2048")


def test_sparse_96_heads(M):
    # the K3 layer's head count: two head groups of 48
    print("sparse B=3 H=96 N=9000 K=1024", flush=True)
    ql, qr, cache, idx = MI.sparse_inputs(3, 96, 9000, 1024, tag="s96")
    idx = idx.copy()
    idx[1, 5::11] = -1
    st, ref = O.sparse_attention(ql, qr, cache, idx)
    assert st == O.OK
    out = run_sparse(M, ql, qr, cache, idx)
    check(host_f32(out), ref, "sparse-96")


def test_sparse_sentinels_sinks_and_empty(M):
    print("sparse sentinels/sinks/empty", flush=True)
    import torch

    ql, qr, cache, idx = MI.sparse_inputs(3, 40, 5000, 300, window=16, tag="ss")
    idx = idx.copy()
    idx[0, ::7] = -1          # sentinels skipped
    idx[2, :] = -1            # no valid row -> zeros (DeepSeekV4Attention.swift:896-899)
    sinks = O.bf16_to_f32(O.normal_bf16("ss.sinks", (40,)))
    st, ref = O.sparse_attention(ql, qr, cache, idx, sinks=sinks)
    assert st == O.OK
    out = run_sparse(M, ql, qr, cache, idx, sinks=sinks, out_dtype=torch.float32)
    check(host_f32(out), ref, "sparse-sinks", scale_bar=2e-3)
    assert (host_f32(out)[2] == 0).all()


def test_sparse_all_indices_equals_dense(M):
    print("sparse all == dense", flush=True)
    import torch

    ql, qr, cache = MI.decode_inputs(128, 1024, tag="ad")
    perm = np.random.default_rng(2).permutation(1024).astype(np.int32)
    a = run_sparse(M, ql[None], qr[None], cache[None], perm[None], out_dtype=torch.float32)
    b = run_decode(M, ql, qr, cache, out_dtype=torch.float32)
    ref = O.mla_decode(ql, qr, cache)[0]
    check(host_f32(a)[0], ref, "sparse-all", scale_bar=2e-3)
    check(host_f32(b)[0], ref, "dense", scale_bar=2e-3)
    # P is rounded to bf16 against the running max, which depends on the row
    # order, so the two orders agree to bf16-P precision, not bitwise
    d = np.abs(host_f32(a) - host_f32(b)).max() / np.abs(ref).max()
    assert d < 4e-3, d


@pytest.mark.parametrize("H", [64, 96])
def test_sparse_v4_form_no_rope(M, H):
    print(f"sparse V4 form (512-wide rows, sinks) H={H}", flush=True)
    import torch

    B, N, K = 2, 3000, 640
    q = O.normal_bf16("v4.q", (B, H, 512))
    rows = O.normal_bf16("v4.rows", (N, 512), std=0.5)   # one cache shared by all tokens
    idx = np.stack([O.sparse_topk_indices(f"v4.i{b}", N, K, 128) for b in range(B)])
    sinks = O.bf16_to_f32(O.normal_bf16("v4.s", (H,)))
    st, ref = O.sparse_attention(q, None, np.broadcast_to(rows, (B, N, 512)), idx, sinks=sinks, kv_rank=512,
                                 rope_dim=0)
    r = dev(rows)
    out = M.mla_decode(dev(q), None, r, None, scale=MI.SCALE, indices=dev(idx.astype(np.int32)),
                       sinks=dev(sinks), out_dtype=torch.float32)
    torch.cuda.synchronize()
    check(host_f32(out), ref, "v4-form", scale_bar=2e-3)


@pytest.mark.parametrize(
    "row,status,pos",
    [([1, 5, -1, 9], 0, -1), ([1, 5, 70000, 9], 3, 2), ([1, 5, 1, 9], 4, 2), ([3, -2, 3], 3, 1),
     ([7, 7, 99999], 4, 1)],
)
def test_index_validation(M, row, status, pos):
    print(f"validate {row}", flush=True)
    idx = np.array([[0, 1, 2, 3][: len(row)], row], np.int32)
    st, tok, p, msg = M.validate_indices(dev(idx), 5000)
    ost, opos = O.validate_indices(np.array(row, np.int32), 5000)
    assert st == status == ost
    if status:
        assert (tok, p) == (1, pos) and opos == pos
        assert ("outside the cache" in msg) if status == 3 else ("more than once" in msg)


def raw_sparse(M, ql, qr, cache, idx, **kw):
    """One mr_mla_decode call through ctypes (the C-ABI itself, not the
    Python wrapper's defaults); returns (status, out, index_status)."""
    import ctypes as C

    import torch

    keep = [dev(ql), dev(qr), dev(cache), dev(np.ascontiguousarray(idx, np.int32))]
    status = kw.pop("index_status", None)
    a, out, ws = M.decode_args(keep[0], keep[1], keep[2][..., :512], keep[2][..., 512:], scale=MI.SCALE,
                               indices=keep[3], out_dtype=torch.float32, index_status=status, **kw)
    st = M.load().mr_mla_decode(C.byref(a), M._stream(None))
    torch.cuda.synchronize()
    return st, out, keep, ws


def bad_lists(N, K, seed):
    """Four token lists: valid; a repeat; an out-of-range entry before a
    repeat; a -2 (out of range, not the -1 sentinel)."""
    rng = np.random.default_rng(seed)
    idx = np.stack([rng.permutation(N)[:K] for _ in range(4)]).astype(np.int32)
    idx[0, ::9] = -1
    idx[1, K - 40] = idx[1, 12]
    idx[2, 20] = N
    idx[2, 100] = idx[2, 5]
    idx[3, 3] = -2
    return idx


def test_sparse_device_index_status_matches_oracle(M):
    # the C-ABI default with a status buffer: checked on the device in the
    # same launch, per token (status, position, value) in the reference's
    # order (DeepSeekV4Attention.swift:884-895); valid tokens still attend
    print("sparse device index status", flush=True)
    import torch

    B, H, N, K = 4, 32, 5000, 300
    ql, qr, cache, _ = MI.sparse_inputs(B, H, N, K, window=16, tag="ds")
    idx = bad_lists(N, K, 11)
    status = torch.full((B, 3), 77, dtype=torch.int32, device="cuda")
    st, out, _, _ = raw_sparse(M, ql, qr, cache, idx, index_status=status)
    assert st == M.OK, M.last_error()
    got = status.cpu().numpy()
    for b in range(B):
        ost, opos = O.validate_indices(idx[b], N)
        want = (ost, opos, idx[b, opos] if opos >= 0 else -1)
        print(f"token {b}: device {tuple(got[b])} oracle {want}", flush=True)
        assert tuple(got[b]) == want
    assert [g[0] for g in got] == [M.OK, M.DUPLICATE_INDEX, M.INDEX_OUT_OF_RANGE, M.INDEX_OUT_OF_RANGE]
    st0, ref0 = O.sparse_attention(ql[:1], qr[:1], cache[:1], idx[:1])
    assert st0 == O.OK
    check(host_f32(out)[:1], ref0, "sparse-status-token0", scale_bar=2e-3)
    # the status is rewritten by every call: a valid batch reads all OK
    good = idx.copy()
    good[1:] = good[0]
    st, _, _, _ = raw_sparse(M, ql, qr, cache, good, index_status=status)
    assert st == M.OK and (status.cpu().numpy() == np.array([0, -1, -1])).all()


def test_sparse_default_call_rejects_bad_lists(M):
    # no status buffer and no flag: the call itself returns the reference's
    # error for the first bad token; MR_DECODE_UNCHECKED skips the checks
    print("sparse default call", flush=True)
    B, H, N, K = 4, 32, 5000, 300
    ql, qr, cache, _ = MI.sparse_inputs(B, H, N, K, window=16, tag="dd")
    idx = bad_lists(N, K, 12)
    st, _, _, _ = raw_sparse(M, ql, qr, cache, idx)
    assert st == M.DUPLICATE_INDEX
    assert M.last_error() == f"token 1 names KV row {idx[1, 12]} more than once"
    st, _, _, _ = raw_sparse(M, ql, qr, cache, idx[2:])
    assert st == M.INDEX_OUT_OF_RANGE and M.last_error() == f"token 0 names KV row {N}, outside the cache"
    st, _, _, _ = raw_sparse(M, ql, qr, cache, idx, flags=M.DECODE_UNCHECKED)
    assert st == M.OK


@pytest.mark.parametrize("n_ctx,n_idx,where", [(1 << 20, 8192, 8191), (1 << 20, 8192, None), (262144, 2176, 2000),
                                              (1 << 20, 10176, 10175), (1 << 20, 10177, 10176),
                                              (1 << 22, 300000, 299999), (1 << 22, 300000, None)])
def test_device_index_check_long_lists(M, n_ctx, n_idx, where):
    # V4-sized caches (up to 2^22 positions); the longest list checked in LDS
    # (10176) and the first one past it, and lists far longer, whose hash
    # tables live in the workspace; a repeat at the very end, or none
    print(f"device index check n_ctx={n_ctx} n_idx={n_idx} repeat at {where}", flush=True)
    import ctypes as C

    import torch

    rng = np.random.default_rng(n_idx)
    B = 2
    idx = np.stack([rng.choice(n_ctx, n_idx, replace=False) for _ in range(B)]).astype(np.int32)
    if where is not None:
        idx[1, where] = idx[1, 0]
    lib = M.load()
    ws = torch.zeros(lib.mr_validate_indices_workspace_size(B, n_idx), dtype=torch.uint8, device="cuda")
    bt, bp = C.c_int32(-9), C.c_int32(-9)
    st = M.load().mr_validate_indices(M._ptr(dev(idx)), B, n_idx, n_ctx, M._ptr(ws), ws.numel(), C.byref(bt),
                                      C.byref(bp), M._stream(None))
    for b in range(B):
        print(b, O.validate_indices(idx[b], n_ctx), flush=True)
    want = O.validate_indices(idx[1], n_ctx)
    assert O.validate_indices(idx[0], n_ctx) == (O.OK, -1)
    assert st == want[0]
    if where is not None:
        assert (bt.value, bp.value) == (1, where) == (1, want[1])


def test_sparse_validation_flag_rejects_before_compute(M):
    print("sparse validate flag", flush=True)
    ql, qr, cache, idx = MI.sparse_inputs(2, 32, 1000, 200, window=8, tag="vf")
    idx = idx.copy()
    idx[1, 10] = idx[1, 11]
    with pytest.raises(M.MRError) as e:
        run_sparse(M, ql, qr, cache, idx)
    assert e.value.status == M.DUPLICATE_INDEX and "token 1" in e.value.message


def v4_ratio128_lists(B, start_pos=1048575, window=128, ratio=128):
    """The index list DeepSeekV4CompressedAttention builds for one decode
    token at start_pos with a ratio-128 compressed cache
    (DeepSeekV4CompressedAttention.swift:1156-1166): the window positions,
    then the compressed positions offset by the window, over keys/values
    that are the window cache followed by the compressed cache.  Returns
    (indices [B, 128 + (start_pos + 1) / 128], rows)."""
    st, w = O.window_indices(window, 1, start_pos)
    assert st == O.OK
    st, c = O.compressed_indices(ratio, 1, start_pos, window)
    assert st == O.OK
    row = np.concatenate([w[0], c[0]]).astype(np.int32)
    n_rows = window + (start_pos + 1) // ratio
    return np.repeat(row[None], B, axis=0), n_rows


def test_v4_ratio128_list_at_1m_positions_checked(M):
    # the reference's longest causal sparse list at the V4 context limit
    # (max_position_embeddings 1048576, current-official-config.json:22):
    # 128 + 8192 = 8320 entries, checked on the device by the default call
    # with a status buffer; a planted repeat and a planted out-of-range entry
    # give the oracle's (status, position, value), the valid token's output
    # matches the oracle
    print("v4 ratio-128 list at position 1048575", flush=True)
    import torch

    B, H = 3, 16
    idx, n_rows = v4_ratio128_lists(B)
    K = idx.shape[1]
    assert K == 8320 and n_rows == 8320
    assert sorted(idx[0].tolist()) == list(range(n_rows))
    idx[1, 7000] = idx[1, 300]                  # a repeat
    idx[2, 5000] = n_rows                       # out of range, before
    idx[2, 8000] = idx[2, 10]                   # a later repeat
    ql = O.normal_bf16("v4l.q_lat", (B, H, 512))
    qr = O.normal_bf16("v4l.q_rope", (B, H, 64))
    cache = O.normal_bf16("v4l.cache", (1, n_rows, 576), std=0.5)
    cache_b = np.ascontiguousarray(np.broadcast_to(cache, (B, n_rows, 576)))
    status = torch.full((B, 3), 77, dtype=torch.int32, device="cuda")
    st, out, _, _ = raw_sparse(M, ql, qr, cache_b, idx, index_status=status)
    assert st == M.OK, M.last_error()
    got = status.cpu().numpy()
    for b in range(B):
        ost, opos = O.validate_indices(idx[b], n_rows)
        want = (ost, opos, idx[b, opos] if opos >= 0 else -1)
        print(f"token {b}: device {tuple(got[b])} oracle {want}", flush=True)
        assert tuple(got[b]) == want
    assert [g[0] for g in got] == [M.OK, M.DUPLICATE_INDEX, M.INDEX_OUT_OF_RANGE]
    assert got[1][1] == 7000 and got[2][1] == 5000
    st0, ref0 = O.sparse_attention(ql[:1], qr[:1], cache, idx[:1])
    assert st0 == O.OK
    check(host_f32(out)[:1], ref0, "v4-8320", scale_bar=2e-3)
    # the default call with no status buffer returns the first bad token's error
    st, _, _, _ = raw_sparse(M, ql, qr, cache_b, idx)
    assert st == M.DUPLICATE_INDEX
    assert M.last_error() == f"token 1 names KV row {idx[1, 300]} more than once"


def test_sparse_checked_list_past_lds_capacity(M):
    # a list longer than an LDS table holds: the launch's check workgroups
    # keep their tables in the workspace, the synchronous check too
    print("sparse checked list of 12000 entries", flush=True)
    import torch

    B, H, N, K = 2, 16, 40000, 12000
    ql, qr, cache, idx = MI.sparse_inputs(B, H, N, K, window=64, tag="lc")
    idx = idx.copy()
    idx[1, 11990] = idx[1, 7]
    status = torch.full((B, 3), 77, dtype=torch.int32, device="cuda")
    st, out, _, _ = raw_sparse(M, ql, qr, cache, idx, index_status=status)
    assert st == M.OK, M.last_error()
    got = status.cpu().numpy()
    assert tuple(got[0]) == (M.OK, -1, -1)
    assert tuple(got[1]) == (M.DUPLICATE_INDEX, 11990, idx[1, 7])
    assert O.validate_indices(idx[1], N) == (O.DUPLICATE_INDEX, 11990)
    st0, ref0 = O.sparse_attention(ql[:1], qr[:1], cache[:1], idx[:1])
    check(host_f32(out)[:1], ref0, "sparse-12000", scale_bar=2e-3)
    st, _, _, _ = raw_sparse(M, ql, qr, cache, idx)
    assert st == M.DUPLICATE_INDEX
