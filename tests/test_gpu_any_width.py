"""MLA attention at widths the fixed-width kernels do not take, through the
same entry points (mr_mla_decode, mr_mla_prefill), against the oracle, whose
restatements take any width (MLA.swift:124-275; DeepSeekV4Attention.swift:
861-920).  The reference's synthetic K3 artifact has kv_lora 16, qk_nope 8,
qk_rope 4, v_head 8 and 4 heads (Tests/MinirunRunnersTests/
SyntheticArtifact.swift:48-55); its rows here are packed [latent ++ rope]
with a 20-element stride, which the split kernel would not take.

Bar: |hip - oracle| <= 1e-2 + 2e-2 |oracle| elementwise (mla_inputs.
within_tolerance) plus the output-scale error; the any-width kernels keep P
and the up-projected keys and values in fp32, so the f32 outputs sit far
inside it.  Index checks and empty selections are exact.
"""
import numpy as np
import pytest

import oracle as O
from test_gpu_block import check, dev, f32, sync

pytestmark = pytest.mark.gpu

K3S = dict(heads=4, kv_rank=16, nope=8, rope=4, v=8)  # the synthetic artifact's widths


@pytest.fixture(scope="module")
def M():
    import minirun_hip as M

    M.load()
    return M


def decode_inputs(tag, B, H, N, R, DR):
    q_lat = O.normal_bf16(f"{tag}.ql", (B, H, R))
    q_rope = O.normal_bf16(f"{tag}.qr", (B, H, DR)) if DR else None
    cache = O.normal_bf16(f"{tag}.c", (B, N, R + DR), std=0.5)
    return q_lat, q_rope, cache


def run_decode(M, q_lat, q_rope, cache, R, DR, scale, out_dtype, indices=None, sinks=None, **kw):
    import torch

    c = dev(cache)
    lat = c[:, :, :R]
    rk = c[:, :, R:] if DR else None
    qr = dev(q_rope) if DR else None
    idx = None if indices is None else torch.from_numpy(np.ascontiguousarray(indices, np.int32)).cuda()
    sk = None if sinks is None else torch.from_numpy(np.ascontiguousarray(sinks, np.float32)).cuda()
    a, out, ws = M.decode_args(dev(q_lat), qr, lat, rk, scale=scale, indices=idx, sinks=sk, out_dtype=out_dtype, **kw)
    st = M.load().mr_mla_decode(M.C.byref(a), M._stream(None))
    sync()
    return st, out


@pytest.mark.parametrize("B,N,ydt", [(2, 37, "f32"), (1, 600, "bf16"), (3, 1, "f32")])
def test_decode_synthetic_k3_widths(M, B, N, ydt):
    import torch

    R, DR, H = K3S["kv_rank"], K3S["rope"], K3S["heads"]
    scale = (K3S["nope"] + DR) ** -0.5
    print(f"any-width decode B={B} N={N} H={H} R={R} DR={DR} y={ydt}", flush=True)
    q_lat, q_rope, cache = decode_inputs(f"aw.{B}.{N}", B, H, N, R, DR)
    st, out = run_decode(M, q_lat, q_rope, cache, R, DR, scale, torch.float32 if ydt == "f32" else torch.bfloat16)
    assert st == M.OK, M.last_error()
    ref = np.stack([O.mla_decode(q_lat[b], q_rope[b], cache[b], kv_rank=R, rope_dim=DR, scale=scale, acc=1)[0]
                    for b in range(B)])
    check(f32(out), ref, f"any-decode-{B}x{N}-{ydt}", scale_bar=1e-5 if ydt == "f32" else 1e-2)


@pytest.mark.parametrize("H,N,R,DR", [(8, 3000, 512, 32), (5, 700, 48, 0), (3, 513, 100, 6)])
def test_decode_other_widths(M, H, N, R, DR):
    # kv_rank 512 with a 32-wide rope (a width between the two the split
    # kernel takes), the V4 form (rope 0, K = V = row) at an odd rank, and
    # widths that are not multiples of 8
    import torch

    scale = 0.5 * (R + DR) ** -0.5
    print(f"any-width decode H={H} N={N} R={R} DR={DR}", flush=True)
    q_lat, q_rope, cache = decode_inputs(f"aw2.{H}.{R}.{DR}", 1, H, N, R, DR)
    st, out = run_decode(M, q_lat, q_rope, cache, R, DR, scale, torch.float32)
    assert st == M.OK, M.last_error()
    ref = O.mla_decode(q_lat[0], None if q_rope is None else q_rope[0], cache[0], kv_rank=R, rope_dim=DR, scale=scale,
                       acc=1)
    check(f32(out), ref, f"any-decode-{H}x{N}x{R}x{DR}", scale_bar=1e-5)


def test_sparse_with_sinks_sentinels_and_empty_lists(M):
    import torch

    R, DR, H = K3S["kv_rank"], K3S["rope"], K3S["heads"]
    B, N, K = 3, 50, 12
    scale = (K3S["nope"] + DR) ** -0.5
    q_lat, q_rope, cache = decode_inputs("aws", B, H, N, R, DR)
    rng = np.random.default_rng(7)
    idx = np.stack([rng.permutation(N)[:K] for _ in range(B)]).astype(np.int32)
    idx[0, [2, 5]] = -1          # sentinels are skipped
    idx[2, :] = -1               # an empty selection gives zeros, sinks or not
    sinks = O.bf16_to_f32(O.normal_bf16("aws.sinks", (H,)))
    st, out = run_decode(M, q_lat, q_rope, cache, R, DR, scale, torch.float32, indices=idx, sinks=sinks)
    assert st == M.OK, M.last_error()
    ost, ref = O.sparse_attention(q_lat, q_rope, cache, idx, sinks, kv_rank=R, rope_dim=DR, scale=scale, acc=1)
    assert ost == 0
    got = f32(out)
    assert np.all(got[2] == 0.0)
    check(got, ref, "any-sparse-sinks", scale_bar=1e-5)


def test_sparse_index_checks(M):
    # the reference's in-order scan: the synchronous form returns the first
    # error, the device form writes (status, position, value) per token
    import torch

    R, DR, H = K3S["kv_rank"], K3S["rope"], K3S["heads"]
    B, N, K = 2, 30, 6
    q_lat, q_rope, cache = decode_inputs("awc", B, H, N, R, DR)
    idx = np.array([[1, 2, 3, 4, 5, 6], [7, 8, 7, 9, 40, 1]], np.int32)  # token 1: repeat at 2, range at 4
    st, _ = run_decode(M, q_lat, q_rope, cache, R, DR, 0.3, torch.float32, indices=idx)
    assert st == M.DUPLICATE_INDEX and "more than once" in M.last_error()
    status = torch.full((B, 3), -7, dtype=torch.int32, device="cuda")
    st, _ = run_decode(M, q_lat, q_rope, cache, R, DR, 0.3, torch.float32, indices=idx, index_status=status)
    assert st == M.OK
    got = status.cpu().numpy()
    assert got[0, 0] == M.OK
    assert (got[1, 0], got[1, 1], got[1, 2]) == (M.DUPLICATE_INDEX, 2, 7)
    assert O.validate_indices(idx[1], N)[1] == 2


def prefill_inputs(tag, T, P, H, R, nope, rope, v):
    q = O.normal_bf16(f"{tag}.q", (T, H, nope + rope))
    cache = O.normal_bf16(f"{tag}.c", (P, R + rope), std=0.5)
    w_uk = O.normal_bf16(f"{tag}.wuk", (R, H * nope), std=R ** -0.5)
    w_uv = O.normal_bf16(f"{tag}.wuv", (R, H * v), std=R ** -0.5)
    kv_b = np.empty((H, nope + v, R), np.uint16)
    kv_b[:, :nope, :] = w_uk.reshape(R, H, nope).transpose(1, 2, 0)
    kv_b[:, nope:, :] = w_uv.reshape(R, H, v).transpose(1, 2, 0)
    return q, cache, w_uk, w_uv, kv_b.reshape(H * (nope + v), R)


@pytest.mark.parametrize("T,P,H,R,nope,rope,v,ydt", [
    (5, 9, 4, 16, 8, 4, 8, "f32"),       # the synthetic K3 artifact's widths
    (40, 300, 4, 16, 8, 4, 8, "bf16"),   # more keys than one 256-key chunk
    (7, 7, 3, 64, 24, 8, 40, "f32"),     # v_head unlike qk_nope
    (6, 20, 2, 32, 16, 0, 16, "f32"),    # no rope part
])
def test_prefill_other_widths(M, T, P, H, R, nope, rope, v, ydt):
    import torch

    print(f"any-width prefill T={T} P={P} H={H} R={R} nope={nope} rope={rope} v={v} y={ydt}", flush=True)
    q, cache, w_uk, w_uv, kv_b = prefill_inputs(f"awp.{T}.{P}.{R}.{v}", T, P, H, R, nope, rope, v)
    c = dev(cache)
    rk = c[:, R:] if rope else torch.zeros(P, 0, dtype=torch.bfloat16, device="cuda")
    out = M.mla_prefill(dev(q), c[:, :R], rk, dev(kv_b), scale=(nope + rope) ** -0.5,
                        out_dtype=torch.float32 if ydt == "f32" else torch.bfloat16)
    sync()
    assert tuple(out.shape) == (T, H, v)
    st = np.repeat(np.arange(T, dtype=np.int32), H)
    sh = np.tile(np.arange(H, dtype=np.int32), T)
    ref = O.mla_prefill_rows(q, cache, w_uk, w_uv, st, sh, kv_rank=R, rope_dim=rope, nope_dim=nope, v_dim=v,
                             scale=(nope + rope) ** -0.5, round_kv=False).reshape(T, H, v)
    check(f32(out), ref, f"any-prefill-{T}x{P}x{R}", scale_bar=1e-5 if ydt == "f32" else 1e-2)
