"""Seeded inputs for the five MLA workloads, built with the oracle's generator.

Test infrastructure: used by tests/ and by __graft_entry__.smoke().  All
tensors are numpy uint16 (bf16 bits) / int32 / float32 arrays.

Shapes (labels are the SplitMix64 stream names, master seed 0x4D4C410001):
  decode(H, N)     q_lat [H,512] ~N(0,1), q_rope [H,64] ~N(0,1) roped at N-1,
                   cache [N,576] ~N(0,0.5) with columns 512..575 roped at 0..N-1
  sparse(B,H,N,K)  q_lat [B,H,512], q_rope [B,H,64], cache [B,N,576],
                   indices [B,K] = last 128 + (K-128) drawn, sorted
"""
from __future__ import annotations

import numpy as np

import oracle as O

SCALE = 192 ** -0.5
R, DR = 512, 64


def rope_rows(x, positions, col0=512, dim=64, base=10000.0):
    f = O.rope_frequencies(dim, base=base)
    c, s = O.rope_table(np.asarray(positions), f)
    return O.rope_apply_bf16(x, c, s, col0, dim)


def decode_inputs(H, N, tag="c2", rope=True):
    q_lat = O.normal_bf16(f"{tag}.q_lat", (H, R))
    q_rope = O.normal_bf16(f"{tag}.q_rope", (H, DR))
    cache = O.normal_bf16(f"{tag}.cache", (N, R + DR), std=0.5)
    if rope:
        q_rope = rope_rows(q_rope.reshape(1, H, DR), [N - 1], col0=0).reshape(H, DR)
        cache = rope_rows(cache.reshape(N, 1, R + DR), np.arange(N)).reshape(N, R + DR)
    return q_lat, q_rope, cache


def sparse_inputs(B, H, N, K, window=128, tag="c4"):
    q_lat = O.normal_bf16(f"{tag}.q_lat", (B, H, R))
    q_rope = O.normal_bf16(f"{tag}.q_rope", (B, H, DR))
    cache = O.normal_bf16(f"{tag}.cache", (B, N, R + DR), std=0.5)
    idx = np.stack([O.sparse_topk_indices(f"{tag}.idx.{b}", N, K, window) for b in range(B)]).astype(np.int32)
    return q_lat, q_rope, cache, idx


def within_tolerance(got, ref, atol=1e-2, rtol=2e-2):
    """The parity bar on bf16 outputs: |got - ref| <= atol + rtol * |ref|."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    ok = err <= atol + rtol * np.abs(ref)
    scale_err = err.max() / max(np.abs(ref).max(), 1e-30)
    return bool(ok.all()), float(err.max()), float(scale_err)


def within_block_tolerance(got, ref, rtol=2e-2, scale_tol=1e-2):
    """The bar for a chain of bf16-rounded stages (the whole decode block):
    |got - ref| <= scale_tol * max|ref| + rtol * |ref| elementwise, and the
    output-scale error max|d| / max|ref| <= scale_tol (the reference's own
    metric, MacReferenceLogits.swift:28-34).  A one-ulp flip in an
    intermediate bf16 rounding propagates an error proportional to the
    output's scale, not to each element, so the absolute term scales with
    max|ref|; the oracle itself, accumulated in fp32 instead of fp64, misses
    the per-kernel bar on such chains."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    err = np.abs(got - ref)
    top = max(np.abs(ref).max(), 1e-30)
    ok = (err <= scale_tol * top + rtol * np.abs(ref)).all() and err.max() <= scale_tol * top
    return bool(ok), float(err.max()), float(err.max() / top)


# ---------------------------------------------------------------- the decode block workload
def affine_weight(tag, out, inp, group=64, centred=False):
    """MLX affine 4-bit operand, bf16 scales and biases.

    Default (the block workload's definition): nibbles U{0..15}, scales
    |N(0,0.01)|, biases N(0,0.01).  Such weights have mean ~7.5 s, so every
    product carries a large common-mode term.  centred=True lays the operand
    out as MLX's quantizer does for zero-mean weights: biases bf16(-7.5 s +
    N(0,0.002)) (the group minimum ~7.5 scales below zero), so products have
    no common-mode term that would hide errors of the stages before them."""
    packed = O.u32(f"{tag}.packed", (out, inp // 8))
    scales = O.abs_normal_bf16(f"{tag}.scales", (out, inp // group), std=0.01)
    if centred:
        jitter = O.bf16_to_f32(O.normal_bf16(f"{tag}.biases", (out, inp // group), std=0.002))
        biases = O.f32_to_bf16(-7.5 * O.bf16_to_f32(scales) + jitter)
    else:
        biases = O.normal_bf16(f"{tag}.biases", (out, inp // group), std=0.01)
    return packed, scales, biases


BLOCK_DIMS = dict(hidden=7168, q_lora_rank=1536, heads=128, nope=128, rope=64, v=128, kv_rank=512)


def block_inputs(ctx=32768, tag="c5", hidden=7168, q_lora_rank=1536, heads=128, nope=128, rope=64, v=128,
                 kv_rank=512, centred=False):
    """One decode token at position ctx-1 over a cache whose rows 0..ctx-2
    are written (roped at their positions); row ctx-1 is written by the block.
    centred selects zero-mean affine weights (see affine_weight)."""
    norm = lambda name, n: O.f32_to_bf16(1 + 0.02 * O.bf16_to_f32(O.normal_bf16(f"{tag}.{name}", (n,))))
    d = {
        "x": O.normal_bf16(f"{tag}.x", (hidden,)),
        "input_norm": norm("input_norm", hidden),
        "q_a_norm": norm("q_a_norm", q_lora_rank),
        "kv_a_norm": norm("kv_a_norm", kv_rank),
        "q_a": affine_weight(f"{tag}.q_a", q_lora_rank, hidden, centred=centred),
        "q_b": affine_weight(f"{tag}.q_b", heads * (nope + rope), q_lora_rank, centred=centred),
        "kv_a": affine_weight(f"{tag}.kv_a", kv_rank + rope, hidden, centred=centred),
        "kv_b": affine_weight(f"{tag}.kv_b", heads * (nope + v), kv_rank, centred=centred),
        "o_proj": affine_weight(f"{tag}.o_proj", hidden, heads * v, centred=centred),
    }
    cache = O.normal_bf16(f"{tag}.cache", (ctx, kv_rank + rope), std=0.5)
    cache = rope_rows(cache.reshape(ctx, 1, kv_rank + rope), np.arange(ctx)).reshape(ctx, kv_rank + rope)
    cache[ctx - 1] = 0
    d["cache"] = cache
    d["position"] = ctx - 1
    return d


K3_DIMS = dict(hidden=7168, q_lora_rank=1536, heads=96, nope=128, rope=64, v=128, kv_rank=512)


def k3_block_inputs(ctx=32768, tag="k3", hidden=7168, q_lora_rank=1536, heads=96, nope=128, rope=64, v=128,
                    kv_rank=512):
    """The K3 flagship attention block (config.json: hidden 7168, 96 heads,
    q_lora 1536, kv_lora 512, nope 128, rope 64 carried unrotated, v 128,
    mla_use_nope, mla_use_output_gate; self_attn weights dense bf16, not
    quantized): dense weights ~N(0, 1/in) so activations keep unit scale,
    RMSNorm weights ~1+N(0,0.02); x is already through input_layernorm, so
    the block has no input norm.  Cache rows ~N(0,0.5), unrotated (NoPE)."""
    norm = lambda name, n: O.f32_to_bf16(1 + 0.02 * O.bf16_to_f32(O.normal_bf16(f"{tag}.{name}", (n,))))
    dense = lambda name, out, inp: O.normal_bf16(f"{tag}.{name}", (out, inp), std=inp ** -0.5)
    d = {
        "x": O.normal_bf16(f"{tag}.x", (hidden,)),
        "input_norm": None,
        "q_a_norm": norm("q_a_norm", q_lora_rank),
        "kv_a_norm": norm("kv_a_norm", kv_rank),
        "q_a": dense("q_a", q_lora_rank, hidden),
        "q_b": dense("q_b", heads * (nope + rope), q_lora_rank),
        "kv_a": dense("kv_a", kv_rank + rope, hidden),
        "kv_b": dense("kv_b", heads * (nope + v), kv_rank),
        "g_proj": dense("g_proj", heads * v, hidden),
        "o_proj": dense("o_proj", hidden, heads * v),
    }
    cache = O.normal_bf16(f"{tag}.cache", (ctx, kv_rank + rope), std=0.5)
    cache[ctx - 1] = 0
    d["cache"] = cache
    d["position"] = ctx - 1
    return d


def _bf(a):
    return O.bf16_to_f32(O.f32_to_bf16(np.asarray(a, np.float32)))


def _mm(x, w):
    packed, s, b = w
    return O.affine_matmul(np.asarray(x, np.float32)[None], packed, s, b, acc=1)[0]


def _lin(x, w):
    return O.linear(np.asarray(x, np.float32)[None], w, acc=1)[0]


def _proj(x, w):
    """A block projection: affine (packed, scales, biases) or dense [out, in]."""
    return _mm(x, w) if isinstance(w, tuple) else _lin(x, w)


def _dequant_kv_b(w, heads, nope, v, kv_rank):
    dense = O.affine_dequantize(*w) if isinstance(w, tuple) else O.bf16_to_f32(w)
    return dense.reshape(heads, nope + v, kv_rank).astype(np.float64)


PLANTS = ("query_not_rotated", "scale_without_rope_dims", "uk_uv_swapped", "position_off_by_one",
          "q_a_norm_skipped")


def block_reference(d, hidden=7168, q_lora_rank=1536, heads=128, nope=128, rope=64, v=128, kv_rank=512, eps=1e-6,
                    plant=None, rotary=True):
    """The block on the oracle, rounding to bf16 where the HIP path stores
    bf16 (every projection output, the normed activations, the cache row).
    Returns (out [hidden] f32 of bf16 values, the written cache row).

    Projections are affine or dense (d's entries); d["input_norm"] None skips
    the input norm; d["g_proj"], when present, gates merged by
    sigmoid(g_proj(h)) before o_proj (MLA.swift:209-211); rotary=False is
    K3's NoPE (MLA.swift:5-13: the rope slice of the query and the shared
    key are carried through unrotated).

    plant (one of PLANTS) puts a plausible mistake into the oracle's block,
    so a test can show that the parity bar would catch it."""
    assert plant is None or plant in PLANTS, plant
    f = O.bf16_to_f32
    pos = d["position"]
    freqs = O.rope_frequencies(rope)
    cos, sin = O.rope_table([pos], freqs)
    qcos, qsin = O.rope_table([pos + 1], freqs) if plant == "position_off_by_one" else (cos, sin)
    x = f(d["x"])
    h = x if d.get("input_norm") is None else _bf(O.rmsnorm(x[None], f(d["input_norm"]), eps)[0])
    q_lora = _bf(_proj(h, d["q_a"]))
    q_lora_n = q_lora if plant == "q_a_norm_skipped" else _bf(O.rmsnorm(q_lora[None], f(d["q_a_norm"]), eps)[0])
    q = O.f32_to_bf16(_proj(q_lora_n, d["q_b"])).reshape(heads, nope + rope)
    if rotary and plant != "query_not_rotated":
        q = O.rope_apply_bf16(q.reshape(1, heads, nope + rope), qcos, qsin, nope, rope).reshape(heads, nope + rope)
    kvb = _dequant_kv_b(d["kv_b"], heads, nope, v, kv_rank)
    w_uk, w_uv = (kvb[:, nope:], kvb[:, :nope]) if plant == "uk_uv_swapped" else (kvb[:, :nope], kvb[:, nope:])
    q_lat = O.f32_to_bf16(np.einsum("hd,hdr->hr", f(q[:, :nope]).astype(np.float64), w_uk).astype(np.float32))
    kv = O.f32_to_bf16(_proj(h, d["kv_a"]))
    row = np.empty(kv_rank + rope, np.uint16)
    row[:kv_rank] = O.f32_to_bf16(O.rmsnorm(f(kv[:kv_rank])[None], f(d["kv_a_norm"]), eps)[0])
    row[kv_rank:] = (O.rope_apply_bf16(kv[kv_rank:].reshape(1, 1, rope), cos, sin, 0, rope).reshape(rope)
                     if rotary else kv[kv_rank:])
    cache = d["cache"].copy()
    cache[pos] = row
    scale = nope ** -0.5 if plant == "scale_without_rope_dims" else (nope + rope) ** -0.5
    ctx = O.mla_decode(q_lat, q[:, nope:], cache[: pos + 1], kv_rank=kv_rank, rope_dim=rope, scale=scale)[0]
    ctx = _bf(ctx).astype(np.float64)
    attn = _bf(np.einsum("hr,hvr->hv", ctx, w_uv).astype(np.float32)).reshape(-1)
    if d.get("g_proj") is not None:
        g = _bf(_proj(h, d["g_proj"]))
        attn = _bf(O.sigmoid_gate(attn, g))
    out = _bf(_proj(attn, d["o_proj"]))
    return out, row


# ---------------------------------------------------------------- the prefill block
SYNTH_K3_DIMS = dict(hidden=128, q_lora_rank=32, heads=4, nope=8, rope=4, v=8, kv_rank=16)


def prefill_block_inputs(T, position, tag, hidden, q_lora_rank, heads, nope, rope, v, kv_rank, affine=False,
                         input_norm=False, gated=True, rotary=False, centred=True):
    """T prompt tokens after `position` cached rows.  Dense weights ~N(0, 1/in)
    (K3's attention weights are dense bf16) or 4-bit affine ones; the cache
    holds rows 0..position-1 (~N(0,0.5), roped at their positions when
    rotary) and zeros after them."""
    norm = lambda name, n: O.f32_to_bf16(1 + 0.02 * O.bf16_to_f32(O.normal_bf16(f"{tag}.{name}", (n,))))
    if affine:
        mk = lambda name, out, inp: affine_weight(f"{tag}.{name}", out, inp, centred=centred)
    else:
        mk = lambda name, out, inp: O.normal_bf16(f"{tag}.{name}", (out, inp), std=inp ** -0.5, threads=16)
    d = {
        "x": O.normal_bf16(f"{tag}.x", (T, hidden)),
        "input_norm": norm("input_norm", hidden) if input_norm else None,
        "q_a_norm": norm("q_a_norm", q_lora_rank),
        "kv_a_norm": norm("kv_a_norm", kv_rank),
        "q_a": mk("q_a", q_lora_rank, hidden),
        "q_b": mk("q_b", heads * (nope + rope), q_lora_rank),
        "kv_a": mk("kv_a", kv_rank + rope, hidden),
        "kv_b": mk("kv_b", heads * (nope + v), kv_rank),
        "o_proj": mk("o_proj", hidden, heads * v),
    }
    if gated:
        d["g_proj"] = mk("g_proj", heads * v, hidden)
    cache = np.zeros((position + T, kv_rank + rope), np.uint16)
    if position:
        rows = O.normal_bf16(f"{tag}.cache", (position, kv_rank + rope), std=0.5)
        if rotary and rope:
            rows = rope_rows(rows.reshape(position, 1, -1), np.arange(position), col0=kv_rank,
                             dim=rope).reshape(position, -1)
        cache[:position] = rows
    d["cache"] = cache
    d["position"] = position
    return d


def _proj_rows(x, w, acc=1):
    if isinstance(w, tuple):
        return O.affine_matmul(np.asarray(x, np.float32), *w, acc=acc, threads=16)
    return O.linear(np.asarray(x, np.float32), w, acc=acc, threads=16)


def prefill_block_reference(d, hidden, q_lora_rank, heads, nope, rope, v, kv_rank, eps=1e-6, rotary=False, acc=1):
    """K3MLA.forward over the prompt (MLA.swift:124-229) on the oracle,
    rounding to bf16 where the reference's bf16 arrays round (every
    projection output, the normed activations, the cache rows, the
    up-projected keys and values of expand, the attention output and the
    gated product).  Returns (out [T, hidden] f32 of bf16 values, the T new
    cache rows).  acc=0 accumulates the projections in fp32."""
    f = O.bf16_to_f32
    pos = d["position"]
    x = f(d["x"])
    T = x.shape[0]
    h = x if d.get("input_norm") is None else _bf(O.rmsnorm(x, f(d["input_norm"]), eps))
    q_lora = _bf(_proj_rows(h, d["q_a"], acc))
    q_lora_n = _bf(O.rmsnorm(q_lora, f(d["q_a_norm"]), eps))
    q = O.f32_to_bf16(_proj_rows(q_lora_n, d["q_b"], acc)).reshape(T, heads, nope + rope)
    kv = O.f32_to_bf16(_proj_rows(h, d["kv_a"], acc))
    rows = np.empty((T, kv_rank + rope), np.uint16)
    rows[:, :kv_rank] = O.f32_to_bf16(O.rmsnorm(f(kv[:, :kv_rank]), f(d["kv_a_norm"]), eps))
    rows[:, kv_rank:] = kv[:, kv_rank:]
    if rotary and rope:
        cos, sin = O.rope_table(np.arange(pos, pos + T), O.rope_frequencies(rope))
        q = O.rope_apply_bf16(q, cos, sin, nope, rope)
        rows[:, kv_rank:] = O.rope_apply_bf16(kv[:, kv_rank:].reshape(T, 1, rope), cos, sin, 0, rope).reshape(T, rope)
    cache = d["cache"][: pos + T].copy()
    cache[pos:] = rows
    kvb = d["kv_b"]
    if isinstance(kvb, tuple):  # the block reads an affine kv_b dequantized to bf16
        kvb = O.f32_to_bf16(O.affine_dequantize(*kvb))
    kvb = kvb.reshape(heads, nope + v, kv_rank)
    w_uk = np.ascontiguousarray(kvb[:, :nope, :].transpose(2, 0, 1).reshape(kv_rank, heads * nope))
    w_uv = np.ascontiguousarray(kvb[:, nope:, :].transpose(2, 0, 1).reshape(kv_rank, heads * v))
    sel_t = np.repeat(np.arange(T, dtype=np.int32), heads)
    sel_h = np.tile(np.arange(heads, dtype=np.int32), T)
    attn = O.mla_prefill_rows(q, cache, w_uk, w_uv, sel_t, sel_h, kv_rank=kv_rank, rope_dim=rope, nope_dim=nope,
                              v_dim=v, scale=(nope + rope) ** -0.5, round_kv=True, threads=16)
    attn = _bf(attn).reshape(T, heads * v)
    if d.get("g_proj") is not None:
        g = _bf(_proj_rows(h, d["g_proj"], acc))
        attn = _bf(O.sigmoid_gate(attn, g))
    return _bf(_proj_rows(attn, d["o_proj"], acc)), rows


def prefill_block_reference_rows(d, sel, hidden, q_lora_rank, heads, nope, rope, v, kv_rank, eps=1e-6):
    """prefill_block_reference (NoPE) for the token rows `sel` only: every
    token's kv_a row goes into the cache (all of them are keys), but the
    queries, the attention, the gate and o_proj are formed for `sel`.
    Returns (out [len(sel), hidden], the T new cache rows)."""
    f = O.bf16_to_f32
    pos = d["position"]
    x = f(d["x"])
    T = x.shape[0]
    sel = np.asarray(sel)
    h = x if d.get("input_norm") is None else _bf(O.rmsnorm(x, f(d["input_norm"]), eps))
    kv = O.f32_to_bf16(_proj_rows(h, d["kv_a"]))
    rows = np.empty((T, kv_rank + rope), np.uint16)
    rows[:, :kv_rank] = O.f32_to_bf16(O.rmsnorm(f(kv[:, :kv_rank]), f(d["kv_a_norm"]), eps))
    rows[:, kv_rank:] = kv[:, kv_rank:]
    cache = d["cache"][: pos + T].copy()
    cache[pos:] = rows
    hs = h[sel]
    q_lora = _bf(_proj_rows(hs, d["q_a"]))
    q_lora_n = _bf(O.rmsnorm(q_lora, f(d["q_a_norm"]), eps))
    q_sel = O.f32_to_bf16(_proj_rows(q_lora_n, d["q_b"])).reshape(len(sel), heads, nope + rope)
    q = np.zeros((T, heads, nope + rope), np.uint16)  # only the sampled rows are read
    q[sel] = q_sel
    kvb = d["kv_b"]
    if isinstance(kvb, tuple):
        kvb = O.f32_to_bf16(O.affine_dequantize(*kvb))
    kvb = kvb.reshape(heads, nope + v, kv_rank)
    w_uk = np.ascontiguousarray(kvb[:, :nope, :].transpose(2, 0, 1).reshape(kv_rank, heads * nope))
    w_uv = np.ascontiguousarray(kvb[:, nope:, :].transpose(2, 0, 1).reshape(kv_rank, heads * v))
    sel_t = np.repeat(sel.astype(np.int32), heads)
    sel_h = np.tile(np.arange(heads, dtype=np.int32), len(sel))
    attn = O.mla_prefill_rows(q, cache, w_uk, w_uv, sel_t, sel_h, kv_rank=kv_rank, rope_dim=rope, nope_dim=nope,
                              v_dim=v, scale=(nope + rope) ** -0.5, round_kv=True, threads=16)
    attn = _bf(attn).reshape(len(sel), heads * v)
    if d.get("g_proj") is not None:
        g = _bf(_proj_rows(hs, d["g_proj"]))
        attn = _bf(O.sigmoid_gate(attn, g))
    return _bf(_proj_rows(attn, d["o_proj"])), rows
