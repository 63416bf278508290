"""Seeded random sweeps of mr_mla_decode and mr_mla_prefill against the
oracle.  Decode: dense and gathered (sparse) forms over random batch sizes,
head counts (including counts that are not multiples of the head groups),
context lengths, split counts, output dtypes, rope widths (64 and 0, the
split kernel's; 32 and 16 at kv_rank 512, 128 and 256, the any-width
kernel's), index lists (sorted or not, with -1 sentinels, an all-sentinel
token) and attention sinks.  Each case names its draw (seed, index) so a
failure can be rerun alone.

Bar: |hip - oracle| <= 1e-2 + 2e-2 |oracle| elementwise (mla_inputs.
within_tolerance), output-scale error below 1e-2 for bf16 outputs and 2e-3
for f32 outputs (the split kernel's partials are bf16 beyond 4096 records);
a token whose list holds only sentinels gives exact zeros.  Prefill: random
prompt lengths, cached prefixes, head counts, query scales and output dtypes,
sampled (token, head) rows at the prefill bars (elementwise, and a per-row
relative L2 error of at most 1e-2).  Top-k selection: random geometry
(decode tokens at later positions, prompts from position 0, compression
ratios, offsets), scores with ties and -inf masks; indices bit for bit."""
import numpy as np
import pytest

import oracle as O
from test_gpu_any_width import decode_inputs, run_decode
from test_gpu_block import check, f32

pytestmark = pytest.mark.gpu

SEED = 20261202
N_CASES = 24
WIDTHS = [(512, 64), (512, 64), (512, 0), (512, 32), (256, 16), (128, 0)]
HEADS = [1, 3, 16, 17, 32, 40, 48, 64, 96, 100, 128, 160]


def draw(i):
    rng = np.random.default_rng([SEED, i])
    R, DR = WIDTHS[rng.integers(len(WIDTHS))]
    c = dict(
        B=int(rng.integers(1, 4)),
        H=int(HEADS[rng.integers(len(HEADS))]),
        N=int(rng.integers(1, 5000)),
        R=R,
        DR=DR,
        splits=int(rng.integers(1, 80)) if rng.random() < 0.4 else 0,
        f32=bool(rng.random() < 0.35),
        sparse=bool(rng.random() < 0.5),
        sinks=bool(rng.random() < 0.4),
        sorted=bool(rng.random() < 0.5),
    )
    if c["sparse"]:
        c["K"] = int(rng.integers(1, min(c["N"], 2500) + 1))
    return c


def indices(rng, c):
    B, N, K = c["B"], c["N"], c["K"]
    idx = np.stack([rng.choice(N, K, replace=False) for _ in range(B)]).astype(np.int32)
    if c["sorted"]:
        idx.sort(axis=1)
    holes = rng.random(idx.shape) < 0.1
    idx[holes] = -1
    if B > 1:
        idx[B - 1, :] = -1  # one token with no valid row
    return idx


@pytest.mark.parametrize("i", range(N_CASES))
def test_decode_sweep(i):
    import torch

    import minirun_hip as M

    M.load()
    c = draw(i)
    print(f"sweep case ({SEED}, {i}): {c}", flush=True)
    B, H, N, R, DR = c["B"], c["H"], c["N"], c["R"], c["DR"]
    scale = (128 + DR) ** -0.5 if DR else R ** -0.5
    q_lat, q_rope, cache = decode_inputs(f"sw.{i}", B, H, N, R, DR)
    rng = np.random.default_rng([SEED, i, 1])
    idx = indices(rng, c) if c["sparse"] else None
    sinks = O.bf16_to_f32(O.normal_bf16(f"sw.{i}.sinks", (H,))) if c["sinks"] and c["sparse"] else None
    ydt = torch.float32 if c["f32"] else torch.bfloat16
    st, out = run_decode(M, q_lat, q_rope, cache, R, DR, scale, ydt, indices=idx, sinks=sinks,
                         num_splits=c["splits"])
    assert st == M.OK, M.last_error()
    if idx is None:
        ref = np.stack([O.mla_decode(q_lat[b], None if q_rope is None else q_rope[b], cache[b], kv_rank=R,
                                     rope_dim=DR, scale=scale, acc=1)[0] for b in range(B)])
    else:
        ost, ref = O.sparse_attention(q_lat, q_rope, cache, idx, sinks, kv_rank=R, rope_dim=DR, scale=scale, acc=1)
        assert ost == O.OK
    got = f32(out)
    if idx is not None and B > 1:
        assert np.all(got[B - 1] == 0.0), "a token with only sentinels gives zeros"
    check(got, ref, f"sweep-{i}", scale_bar=2e-3 if c["f32"] else 1e-2)


N_PREFILL = 12


def draw_prefill(i):
    rng = np.random.default_rng([SEED, 1000 + i])
    T = int(rng.integers(1, 700))
    return dict(T=T, P=T + (int(rng.integers(0, 900)) if rng.random() < 0.6 else 0), H=int(rng.integers(1, 13)),
                q_std=float(rng.choice([1.0, 4.0])), f32=bool(rng.random() < 0.35),
                rows=int(rng.integers(24, 64)))


@pytest.mark.parametrize("i", range(N_PREFILL))
def test_prefill_sweep(i):
    # causal prefill over a cached prefix of P - T rows (the last T rows are
    # the prompt's own): random sampled (token, head) rows against the oracle
    # with keys and values rounded to bf16 as the HIP path stores them
    import torch

    import minirun_hip as M
    from test_gpu_prefill import check_rows, prefill_inputs, run

    M.load()
    c = draw_prefill(i)
    print(f"prefill sweep case ({SEED}, {1000 + i}): {c}", flush=True)
    T, P, H = c["T"], c["P"], c["H"]
    q, cache, w_uk, w_uv, kv_b = prefill_inputs(T, P, H, f"swp.{i}", c["q_std"])
    got = run(M, q, cache, kv_b, out_dtype=torch.float32 if c["f32"] else None)
    rng = np.random.default_rng([SEED, 1000 + i, 1])
    n = min(c["rows"], T * H)
    flat = rng.choice(T * H, n, replace=False)
    st, sh = (flat // H).astype(np.int32), (flat % H).astype(np.int32)
    st[0], sh[0] = T - 1, H - 1  # the last query sees every row
    ref = O.mla_prefill_rows(q, cache, w_uk, w_uv, st, sh, round_kv=True).reshape(n, 128)
    check_rows(got[st, sh], ref, f"prefill-sweep-{i}")


N_TOPK = 20


def draw_topk(i):
    rng = np.random.default_rng([SEED, 2000 + i])
    ratio = int(rng.integers(1, 9))
    if rng.random() < 0.5:  # one decode token at a later position
        cols = int(rng.integers(1, 40000))
        rows, start = 1, int(rng.integers(0, cols * ratio))
    else:  # a prompt from position 0
        rows = int(rng.integers(1, 65))
        cols = int(rng.integers(max(rows // ratio, 1), 3000))
        start = 0
    return dict(rows=rows, cols=cols, ratio=ratio, start=start, top_k=int(rng.integers(1, 9000)),
                offset=int(rng.integers(0, 1 << 20)), ties=bool(rng.random() < 0.4),
                masked=bool(rng.random() < 0.3))


@pytest.mark.parametrize("i", range(N_TOPK))
def test_topk_sweep(i):
    # bit-exact indices: random geometry, scores with many ties (a few
    # distinct values: ascending key id breaks them) and -inf masked keys
    import minirun_hip as M
    from test_gpu_topk import compare

    M.load()
    c = draw_topk(i)
    print(f"top-k sweep case ({SEED}, {2000 + i}): {c}", flush=True)
    rng = np.random.default_rng([SEED, 2000 + i, 1])
    s = rng.standard_normal((c["rows"], c["cols"])).astype(np.float32)
    if c["ties"]:
        s = np.round(s * 2).astype(np.float32) * np.float32(0.5)
    if c["masked"]:
        s[rng.random(s.shape) < 0.2] = -np.inf
    compare(M, s, c["top_k"], c["ratio"], c["start"], c["offset"], f"sweep-{i}")
