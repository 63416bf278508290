"""The whole prompt through the MLA block in one call (mr_mla_prefill_block,
K3MLA.forward, MLA.swift:124-229) against the oracle's composition of the
same stages (mla_inputs.prefill_block_reference): state == nil (position 0)
and a cached prefix, dense K3 weights with the output gate and NoPE, 4-bit
affine weights with an input norm and rotary keys, the K3 widths and the
reference's synthetic artifact's (SyntheticArtifact.swift:48-55).

Bar: the chain bar of a block of bf16-rounded stages
(mla_inputs.within_block_tolerance: |d| <= 1e-2 max|ref| + 2e-2 |ref|
elementwise, output-scale error <= 1e-2).  Where the outputs stay below 2
(one bf16 ulp of the output scale below the workload bar's absolute 1e-2),
the HIP block also misses the elementwise workload bar (1e-2 + 2e-2 |ref|)
on no more outputs than the oracle accumulating its projections in fp32
does.  Above that scale a one-ulp flip of any bf16 intermediate moves
near-zero outputs by more than 1e-2 whatever the arithmetic (the 128-head
affine case reaches |out| ~ 20), and the HIP attention's bf16 probabilities
(the PV MFMA operand; the reference keeps them fp32) flip more of them than
a reordered fp32 sum does, so there only the chain bar applies.  The new cache rows
match the oracle's to 2^-7 |ref| + 2^-9 of the row's largest element, per
part (latent, rope key); the largest difference in bf16 ulps is printed.
"""
import numpy as np
import pytest

import mla_inputs as MI
import oracle as O
from test_gpu_block import bits16, dev, f32, misses, projection, sync

pytestmark = pytest.mark.gpu

K3 = dict(MI.K3_DIMS)
C5 = dict(MI.BLOCK_DIMS)
SYN = dict(MI.SYNTH_K3_DIMS)


@pytest.fixture(scope="module")
def M():
    import minirun_hip as M

    M.load()
    return M


def run_prefill_block(M, d, dims, rotary):
    import torch

    w = {k: (dev(d[k]) if d.get(k) is not None else None) for k in ("input_norm", "q_a_norm", "kv_a_norm")}
    for k in ("q_a", "q_b", "kv_a", "kv_b", "o_proj", "g_proj"):
        w[k] = projection(M, d.get(k))
    cache = dev(d["cache"])
    T = d["x"].shape[0]
    c = s = None
    if rotary:
        pos = np.arange(d["position"], d["position"] + T)
        c, s = M.rope_table(pos, M.rope_frequencies(dims["rope"]))
        c, s = torch.from_numpy(c).cuda(), torch.from_numpy(s).cuda()
    kw = {k: dims[k] for k in ("q_lora_rank", "heads", "nope", "rope", "v", "kv_rank")}
    out = M.mla_prefill_block(dev(d["x"]), w, cache, d["position"], c, s, **kw)
    sync()
    return out, cache


def check_prefill_block(M, d, dims, rotary, tag):
    out, cache = run_prefill_block(M, d, dims, rotary)
    ref, rows = MI.prefill_block_reference(d, rotary=rotary, **dims)
    pos, T = d["position"], d["x"].shape[0]
    got_cache = bits16(cache)
    np.testing.assert_array_equal(got_cache[:pos], d["cache"][:pos])  # the prefix is left as it was
    R = dims["kv_rank"]
    ulps = np.abs(got_cache[pos:].astype(np.int32) - rows.astype(np.int32)).max()
    for part, cols in (("latents", slice(0, R)), ("rope keys", slice(R, None))):
        # kv_a's outputs are sums with cancellation (an input-norm flip moves
        # one by more than its own ulp) and a rotated key element is a
        # difference of two products: errors scale with the row, not the element
        g, r = O.bf16_to_f32(got_cache[pos:, cols]), O.bf16_to_f32(rows[:, cols])
        if r.size:
            top = np.abs(r).max(axis=1, keepdims=True)
            assert np.all(np.abs(g - r) <= 2 ** -7 * np.abs(r) + 2 ** -9 * top), f"{tag}: cache {part}"
    got = f32(out)
    ok, maxerr, scale_err = MI.within_block_tolerance(got, ref)
    ref32, _ = MI.prefill_block_reference(d, rotary=rotary, acc=0, **dims)
    n_hip, n_f32 = misses(got, ref), misses(ref32, ref)
    top = np.abs(ref).max()
    print(f"{tag}: max|ref|={top:.3e} max|d|={maxerr:.3e} scale_err={scale_err:.3e}; outside the workload bar: "
          f"HIP {n_hip}, fp32-accumulating oracle {n_f32} (of {ref.size}); cache rows within {ulps} ulps", flush=True)
    assert ok, f"{tag}: block bar violated (max |d| {maxerr}, output-scale {scale_err})"
    if top < 2.0:
        # where one bf16 ulp of the output scale is below the bar's 1e-2
        # absolute term, the elementwise bar applies as well
        assert n_hip <= n_f32, (n_hip, n_f32)
    return got


@pytest.mark.parametrize("T,position", [(5, 0), (7, 5), (70, 0), (33, 40)])
def test_synthetic_k3_widths(M, T, position):
    print(f"prefill block synthetic K3 widths T={T} position={position}", flush=True)
    d = MI.prefill_block_inputs(T, position, f"pbs.{T}.{position}", **SYN)
    check_prefill_block(M, d, SYN, False, f"prefill-block-syn-{T}-{position}")


@pytest.mark.parametrize("T,position", [(64, 0), (100, 28)])
def test_k3_dense_gated_nope(M, T, position):
    # K3's attention block: dense bf16 weights, 96 heads, output gate, NoPE;
    # the projections on MFMA tiles, the attention on the fixed-width kernels
    print(f"prefill block K3 T={T} position={position}", flush=True)
    d = MI.prefill_block_inputs(T, position, f"pbk3.{T}.{position}", **K3)
    check_prefill_block(M, d, K3, False, f"prefill-block-k3-{T}-{position}")


def test_k3_4096_tokens_sampled_rows(M):
    # the K3 block over a whole 4096-token prompt (the prefill workload's
    # length): every cache row, and the outputs of sampled token rows (both
    # ends, tile boundaries, a few seeded ones) over all 7168 columns
    T = 4096
    print(f"prefill block K3 T={T} sampled rows", flush=True)
    d = MI.prefill_block_inputs(T, 0, "pbk3full", **K3)
    out, cache = run_prefill_block(M, d, K3, False)
    rng = np.random.default_rng(4096)
    sel = np.array(sorted({0, 1, 63, 64, 127, 128, 255, 256, 2047, 4095} | set(int(r) for r in rng.integers(0, T, 4))))
    ref, rows = MI.prefill_block_reference_rows(d, sel, **K3)
    R = K3["kv_rank"]
    for cols in (slice(0, R), slice(R, None)):  # latents; the shared keys (NoPE: kv_a's outputs as they are)
        g, r = O.bf16_to_f32(bits16(cache)[:, cols]), O.bf16_to_f32(rows[:, cols])
        assert np.all(np.abs(g - r) <= 2 ** -7 * np.abs(r) + 2 ** -9 * np.abs(r).max(axis=1, keepdims=True))
    got = f32(out)[sel]
    ok, maxerr, scale_err = MI.within_block_tolerance(got, ref)
    n_hip = misses(got, ref)
    print(f"prefill-block-k3-4096: max|ref|={np.abs(ref).max():.3e} max|d|={maxerr:.3e} scale_err={scale_err:.3e}; "
          f"outside the workload bar: {n_hip} of {ref.size}", flush=True)
    assert ok, (maxerr, scale_err)
    assert n_hip == 0, n_hip


def test_affine_rotary_input_norm(M):
    # 4-bit affine projections (128 heads), an input norm, rotary query and
    # keys at positions 37..100, no gate
    T, position = 64, 37
    print(f"prefill block affine rotary T={T} position={position}", flush=True)
    d = MI.prefill_block_inputs(T, position, "pba", affine=True, input_norm=True, gated=False, rotary=True, **C5)
    check_prefill_block(M, d, C5, True, "prefill-block-affine-rotary")


def test_affine_any_width_rotary(M):
    dims = dict(hidden=256, q_lora_rank=64, heads=8, nope=24, rope=8, v=40, kv_rank=64)
    print("prefill block affine any-width rotary T=20 position=9", flush=True)
    d = MI.prefill_block_inputs(20, 9, "pbaw", affine=True, input_norm=True, rotary=True, **dims)
    check_prefill_block(M, d, dims, True, "prefill-block-affine-any-width")


def test_prompt_in_one_call_equals_two_chunks(M):
    """Causality: the prompt in one call and the same prompt as two calls (the
    second over the first's cache) give the same cache and outputs, bit for
    bit where the per-token arithmetic is the same, i.e. below 64 tokens per
    call on both sides (one projection kernel)."""
    import torch

    T, split = 40, 17
    d = MI.prefill_block_inputs(T, 0, "pbc", **SYN)
    out_all, cache_all = run_prefill_block(M, d, SYN, False)
    d1 = dict(d, x=d["x"][:split])
    d1["cache"] = d["cache"].copy()
    out1, cache1 = run_prefill_block(M, d1, SYN, False)
    d2 = dict(d, x=d["x"][split:], position=split)
    d2["cache"] = bits16(cache1)
    out2, cache2 = run_prefill_block(M, d2, SYN, False)
    np.testing.assert_array_equal(bits16(cache2), bits16(cache_all))
    np.testing.assert_array_equal(np.concatenate([bits16(out1), bits16(out2)]), bits16(out_all))


def test_one_token_prompt_equals_decode_block(M):
    """A one-token prompt after 4095 cached rows (K3's block: dense, gated,
    NoPE, 96 heads) through the prefill block (expanded keys and values,
    the fixed-width prefill kernels) and through the decode block (absorbed
    queries, the split decode): the two HIP paths of the same K3MLA.forward
    step write the same cache row (within one bf16 ulp: the projections'
    GEMV launches differ) and outputs within the block bar of each other."""
    import torch

    position = 4095
    print(f"one-token prompt vs decode block, K3, position {position}", flush=True)
    d = MI.prefill_block_inputs(1, position, "pb1tok", **K3)
    out_p, cache_p = run_prefill_block(M, d, K3, False)
    w = {k: (dev(d[k]) if d.get(k) is not None else None) for k in ("input_norm", "q_a_norm", "kv_a_norm")}
    for k in ("q_a", "q_b", "kv_a", "kv_b", "o_proj", "g_proj"):
        w[k] = projection(M, d.get(k))
    cache_d = dev(d["cache"])
    kw = {k: K3[k] for k in ("hidden", "q_lora_rank", "heads", "nope", "rope", "v", "kv_rank")}
    out_d = M.mla_decode_block(dev(d["x"][0]), w, cache_d, position, None, None, **kw)
    sync()
    rp, rd = bits16(cache_p)[position].astype(np.int32), bits16(cache_d)[position].astype(np.int32)
    print(f"cache row: largest difference {np.abs(rp - rd).max()} bf16 ulps", flush=True)
    assert np.abs(rp - rd).max() <= 1
    np.testing.assert_array_equal(bits16(cache_p)[:position], bits16(cache_d)[:position])
    got, ref = f32(out_p)[0], f32(out_d)
    ok, maxerr, scale_err = MI.within_block_tolerance(got, ref)
    print(f"prefill vs decode block: max|d|={maxerr:.3e} scale_err={scale_err:.3e}", flush=True)
    assert ok, (maxerr, scale_err)


def test_failed_checks_leave_the_cache(M):
    # a call that fails its checks writes nothing
    import torch

    d = MI.prefill_block_inputs(6, 3, "pbf", **SYN)
    w = {k: dev(d[k]) for k in ("q_a_norm", "kv_a_norm")}
    w["input_norm"] = None
    for k in ("q_a", "q_b", "kv_a", "kv_b", "o_proj", "g_proj"):
        w[k] = projection(M, d.get(k))
    cache = dev(d["cache"])
    before = bits16(cache).copy()
    x = dev(d["x"])
    out = torch.empty(6, SYN["hidden"], dtype=torch.bfloat16, device="cuda")
    kw = {k: SYN[k] for k in ("q_lora_rank", "heads", "nope", "rope", "v", "kv_rank")}
    a, ws = M.prefill_block_args(x, w, cache, 3, None, None, out, **kw)
    a.capacity = 8  # rows 3..8 do not fit
    assert M.load().mr_mla_prefill_block(M.C.byref(a), M._stream(None)) == M.INVALID_SHAPE
    a.capacity = 9
    a.workspace_bytes -= 256
    assert M.load().mr_mla_prefill_block(M.C.byref(a), M._stream(None)) == M.WORKSPACE_TOO_SMALL
    sync()
    np.testing.assert_array_equal(bits16(cache), before)
