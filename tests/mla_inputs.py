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
