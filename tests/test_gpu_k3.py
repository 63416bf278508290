"""The K3 attention block through the C-ABI: dense projections (k3Linear,
Linear.swift:55-57), NoPE (MLA.swift:5-13), the sigmoid output gate
(MLA.swift:209-211) and 96 heads, against the oracle.

Bars: the workload bar |hip - oracle| <= 1e-2 + 2e-2 |oracle| elementwise
(plus the output-scale error) for single kernels; for the composed block the
count of outputs outside that bar must not exceed the oracle's own count
when its projections accumulate in fp32, and the chain bar of
mla_inputs.within_block_tolerance holds.  Closed forms are bitwise.
"""
import numpy as np
import pytest

import mla_inputs as MI
import oracle as O
from test_gpu_block import bits16, check, check_block, dev, f32, misses, run_block, sync

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    import minirun_hip as M

    M.load()
    return M


@pytest.mark.parametrize(
    "tokens,out_f,in_f,wdt,xdt",
    [(1, 1536, 7168, "bf16", "bf16"), (1, 7168, 12288, "bf16", "bf16"), (3, 576, 7168, "bf16", "bf16"),
     (13, 200, 512, "bf16", "f32"), (2, 64, 20000, "bf16", "bf16"), (1, 100, 1000, "f32", "bf16"),
     (5, 33, 96, "f32", "f32")],
)
def test_linear_matches_oracle(M, tokens, out_f, in_f, wdt, xdt):
    # one weight read per tile of up to 8 tokens; a 20000-wide row takes the
    # unstaged kernel; f32 weights and activations
    print(f"linear {tokens} x [{out_f}, {in_f}] w={wdt} x={xdt}", flush=True)
    import torch

    w = O.normal_bf16(f"lin.{out_f}.{in_f}", (out_f, in_f), std=in_f ** -0.5)
    x = O.normal_bf16(f"lin.x.{tokens}.{in_f}", (tokens, in_f))
    wt = dev(w) if wdt == "bf16" else torch.from_numpy(O.bf16_to_f32(w)).cuda()
    xt = dev(x) if xdt == "bf16" else torch.from_numpy(O.bf16_to_f32(x)).cuda()
    y = M.linear(xt, M.DenseWeights(wt), out_dtype=torch.float32)
    sync()
    ref = O.linear(O.bf16_to_f32(x), w, acc=1)
    check(f32(y), ref, f"linear-{tokens}x{out_f}x{in_f}", scale_bar=1e-5)


def test_linear_rejects_bad_weights(M):
    import torch

    lib = M.load()
    w = torch.zeros(8, 12, dtype=torch.bfloat16, device="cuda")   # 12 is not a whole 16-byte chunk
    d = M.DenseWeights(w).desc()
    x = torch.zeros(1, 12, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros(1, 8, dtype=torch.bfloat16, device="cuda")
    st = lib.mr_linear(M._ptr(x), M.BF16, 1, 12, M.C.byref(d), M._ptr(y), M.BF16, 8, M._stream(None))
    assert st == M.INVALID_SHAPE and "multiple of 8" in M.last_error()
    d.dtype = M.F16
    st = lib.mr_linear(M._ptr(x), M.BF16, 1, 12, M.C.byref(d), M._ptr(y), M.BF16, 8, M._stream(None))
    assert st == M.INVALID_DTYPE
    # f32 weights of 4 inputs pass the chunk rule, but a bf16 activation row
    # of 4 values is 8 bytes: refused (the GEMV reads 16-byte chunks of it)
    w4 = torch.zeros(8, 4, dtype=torch.float32, device="cuda")
    d4 = M.DenseWeights(w4).desc()
    x4 = torch.zeros(1, 4, dtype=torch.bfloat16, device="cuda")
    st = lib.mr_linear(M._ptr(x4), M.BF16, 1, 4, M.C.byref(d4), M._ptr(y), M.BF16, 8, M._stream(None))
    assert st == M.INVALID_SHAPE and "under 16 bytes" in M.last_error()
    x4f = torch.zeros(1, 4, dtype=torch.float32, device="cuda")
    st = lib.mr_linear(M._ptr(x4f), M.F32, 1, 4, M.C.byref(d4), M._ptr(y), M.BF16, 8, M._stream(None))
    assert st == M.OK
    sync()


def test_dense_absorb_and_unabsorb(M):
    # kv_b_proj dense [H*(nope+v), 512] (K3 stores self_attn weights in bf16)
    print("dense absorb / unabsorb, 96 heads", flush=True)
    import torch

    H, dn, dv = 96, 128, 128
    kvb = O.normal_bf16("dab.kvb", (H * (dn + dv), 512), std=512 ** -0.5)
    q = O.normal_bf16("dab.q", (H, 192))
    w = M.DenseWeights(dev(kvb))
    q_lat = M.mla_absorb_query(dev(q), H, dn, dv, w)
    ctx = O.normal_bf16("dab.ctx", (H, 512), std=0.05)
    out = M.mla_unabsorb_values(dev(ctx), H, dn, dv, w, out_dtype=torch.float32)
    sync()
    W = O.bf16_to_f32(kvb).reshape(H, dn + dv, 512).astype(np.float64)
    ref_lat = np.einsum("hd,hdr->hr", O.bf16_to_f32(q[:, :dn]).astype(np.float64), W[:, :dn])
    check(f32(q_lat), ref_lat, "dense-absorb", scale_bar=1e-2)
    ref_out = np.einsum("hr,hvr->hv", O.bf16_to_f32(ctx).astype(np.float64), W[:, dn:])
    check(f32(out), ref_out, "dense-unabsorb", scale_bar=1e-5)


def _lin_f32(x, w):
    return O.linear(np.asarray(x, np.float32)[None], w, acc=0)[0]


def test_k3_flagship_block(M, monkeypatch):
    # the K3 flagship's attention layer (config.json: hidden 7168, 96 heads,
    # q_lora 1536, nope 128 + rope 64 unrotated, v 128, gate on, dense bf16
    # weights, rms eps 1e-5) for one token at position 32767
    dims = dict(MI.K3_DIMS)
    print(f"K3 block {dims} ctx=32768, dense, NoPE, gated", flush=True)
    d = MI.k3_block_inputs()
    out, cache = run_block(M, d, rotary=False, eps=1e-5, hidden=dims["hidden"], q_lora_rank=dims["q_lora_rank"],
                           heads=dims["heads"], nope=dims["nope"], rope=dims["rope"], v=dims["v"])
    ref, row = MI.block_reference(d, heads=96, eps=1e-5, rotary=False)
    got_row = bits16(cache)[d["position"]]
    np.testing.assert_array_equal(got_row[512:], row[512:])   # the shared key slice, stored unrotated
    assert np.abs(got_row[:512].astype(np.int32) - row[:512].astype(np.int32)).max() <= 1
    monkeypatch.setattr(MI, "_lin", _lin_f32)
    ref32, _ = MI.block_reference(d, heads=96, eps=1e-5, rotary=False)
    n_hip, n_f32 = misses(f32(out), ref), misses(ref32, ref)
    print(f"K3 block: outputs outside 1e-2 + 2e-2|ref| of the fp64 oracle: HIP {n_hip}, "
          f"fp32-accumulating oracle {n_f32} (of {ref.size})", flush=True)
    # the per-element workload bar holds for every output whenever the fp32
    # restatement of the same chain meets it; otherwise the HIP chain may
    # miss no more outputs than that restatement does
    if n_f32 == 0:
        assert n_hip == 0, f"HIP misses {n_hip} of {ref.size} outputs; the fp32-accumulating oracle misses none"
    else:
        assert n_hip <= n_f32, f"HIP misses {n_hip} outputs, the fp32-accumulating oracle {n_f32} (of {ref.size})"
    check_block(f32(out), ref, "k3-block")


def test_gate_closed_forms(M):
    # g_proj = 0: sigmoid(0) = 1/2 halves merged exactly, and o_proj is
    # linear, so the gated block is exactly half the ungated one (bf16
    # halving is exact); a gate saturated at 1 leaves the block unchanged
    print("gate closed forms (dense, NoPE, 16 heads, ctx 300)", flush=True)
    dims = dict(hidden=1024, q_lora_rank=256, heads=16, nope=128, rope=64, v=128, kv_rank=512)
    d = MI.k3_block_inputs(ctx=300, tag="gcf", hidden=1024, q_lora_rank=256, heads=16)
    kw = dict(rotary=False, eps=1e-5, hidden=1024, q_lora_rank=256, heads=16)
    ungated = dict(d, g_proj=None)
    base, _ = run_block(M, ungated, **kw)
    half, _ = run_block(M, dict(d, g_proj=np.zeros_like(d["g_proj"])), **kw)
    np.testing.assert_array_equal(f32(half), 0.5 * f32(base))
    # x . g_w = 1e4 on every row: sigmoid saturates to 1 in fp32
    x = O.bf16_to_f32(d["x"]).astype(np.float64)
    g_w = O.f32_to_bf16(np.tile((1e4 * x / (x @ x)).astype(np.float32), (16 * 128, 1)))
    one, _ = run_block(M, dict(d, g_proj=g_w), **kw)
    ref_one, _ = MI.block_reference(dict(d, g_proj=g_w), heads=16, hidden=1024, q_lora_rank=256, eps=1e-5,
                                    rotary=False)
    assert misses(f32(one), ref_one) == 0
    np.testing.assert_array_equal(f32(one), f32(base))
    ref, _ = MI.block_reference(d, heads=16, hidden=1024, q_lora_rank=256, eps=1e-5, rotary=False)
    gated, _ = run_block(M, d, **kw)
    assert misses(f32(gated), ref) == 0
    check_block(f32(gated), ref, "gated-small")


def test_nope_with_affine_weights(M):
    # NoPE on the affine 4-bit block (the cfg-5 shape at a short context):
    # the query rope slice and the cached key are not rotated
    print("NoPE, affine weights, 128 heads, ctx 200", flush=True)
    d = MI.block_inputs(ctx=200, tag="nope", centred=True)
    out, cache = run_block(M, d, rotary=False)
    ref, row = MI.block_reference(d, rotary=False)
    np.testing.assert_array_equal(bits16(cache)[d["position"]][512:], row[512:])
    check_block(f32(out), ref, "nope-affine")
    rot, _ = MI.block_reference(d)
    assert not MI.within_block_tolerance(f32(out), rot)[0]   # the rotated reading is a different block


def test_block_rejects_one_rotary_table(M):
    import torch

    d = MI.k3_block_inputs(ctx=8, tag="rej", hidden=256, q_lora_rank=64, heads=2)
    w = {k: (dev(d[k]) if d.get(k) is not None else None) for k in ("input_norm", "q_a_norm", "kv_a_norm")}
    for k in ("q_a", "q_b", "kv_a", "kv_b", "o_proj", "g_proj"):
        w[k] = M.DenseWeights(dev(d[k]))
    c = torch.zeros(32, dtype=torch.float32, device="cuda")
    with pytest.raises(M.MRError) as e:
        M.mla_decode_block(dev(d["x"]), w, dev(d["cache"]), d["position"], c, None, hidden=256, q_lora_rank=64,
                           heads=2)
    assert e.value.status == M.INVALID_ARGUMENT and "both rotary tables" in e.value.message
