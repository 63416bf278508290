#!/usr/bin/env python3
"""MLA decode benchmark on one MI355X.

Headline (one JSON line on stdout): absorbed-MLA decode, batch 1, 128 heads,
kv_lora 512 + rope 64 (576-wide bf16 latent rows), context 32768, fp32
softmax/accumulation, bf16 output -- microseconds per layer, with the
achieved HBM fraction of the dominant (split) kernel, and the sparse top-2048
decode (batch 4, 128 heads, 128K context) as a second figure.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

A step is one decode layer (split kernel + combine kernel) over inputs
already resident in HBM.  Caches rotate over enough copies that the 256 MB
Infinity Cache cannot hold them, so the traffic is HBM traffic.  Inputs are
synthetic (torch RNG with a fixed seed, the workload's distributions).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "minirun-app_amd"))

HBM_PEAK_GBS = 8000.0
H, N, R, DR = 128, 32768, 512, 64
SCALE = 192 ** -0.5


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def cache_bytes_per_layer():
    # algorithmic bytes of one decode layer: cache rows + q + bf16 out
    return N * (R + DR) * 2 + H * (R + DR) * 2 + H * R * 2


def split_kernel_bytes():
    # the split kernel reads the cache rows and q; the combine writes out
    return N * (R + DR) * 2 + H * (R + DR) * 2


# HBM bytes one launch of the dense split kernel moves (H=128, N=32768):
# FETCH_SIZE x 2.0 + WRITE_SIZE x 1.0 (factors from a streaming kernel of
# known size), from two rocprofv3 --pmc passes over this bench command; the
# passes and the commit they measured are in profiles/mla_decode_hbm_counters.md.
# A recorded value, not measured by this run.  Of it, 16,777,216 B are the
# bf16 split partials written.
SPLIT_TRAFFIC_BYTES = 56408631
SPLIT_TRAFFIC_SOURCE = "recorded: rocprofv3 FETCH_SIZE/WRITE_SIZE passes, profiles/mla_decode_hbm_counters.md"


def sparse_bytes(B=4, K=2048):
    return B * K * (R + DR) * 2 + B * K * 4 + B * H * (R + DR) * 2 + B * H * R * 2


def make_decode_inputs(torch, nbuf):
    g = torch.Generator(device="cuda")
    g.manual_seed(0x4D4C410001)
    q_lat = torch.randn(1, H, R, generator=g, device="cuda").to(torch.bfloat16)
    q_rope = torch.randn(1, H, DR, generator=g, device="cuda").to(torch.bfloat16)
    caches = [(0.5 * torch.randn(N, R + DR, generator=g, device="cuda")).to(torch.bfloat16) for _ in range(nbuf)]
    return q_lat, q_rope, caches


def make_sparse_inputs(torch, ncache, nidx, B=4, NC=131072, K=2048, window=128):
    g = torch.Generator(device="cuda")
    g.manual_seed(0x4D4C410004)
    q_lat = torch.randn(B, H, R, generator=g, device="cuda").to(torch.bfloat16)
    q_rope = torch.randn(B, H, DR, generator=g, device="cuda").to(torch.bfloat16)
    caches = [(0.5 * torch.randn(B, NC, R + DR, generator=g, device="cuda")).to(torch.bfloat16)
              for _ in range(ncache)]
    gc = torch.Generator()
    gc.manual_seed(4)
    sets = []
    for _ in range(nidx):
        rows = []
        for _b in range(B):
            drawn = torch.randperm(NC - window, generator=gc)[: K - window]
            rows.append(torch.sort(torch.cat([drawn, torch.arange(NC - window, NC)])).values)
        sets.append(torch.stack(rows).to(torch.int32).cuda())
    return q_lat, q_rope, caches, sets


BLOCK = dict(hidden=7168, q_lora_rank=1536, heads=128, nope=128, rope=64, v=128, kv_rank=512)
BLOCK_SHAPES = {"q_a": (1536, 7168), "q_b": (128 * 192, 1536), "kv_a": (576, 7168), "kv_b": (128 * 256, 512),
                "o_proj": (7168, 128 * 128)}


def block_bytes():
    """Algorithmic HBM bytes of one decode block: every affine operand once
    (packed nibbles + bf16 scales and biases, kv_b included), the cache rows
    read by the attention, and 264,320 bytes of activations."""
    w = sum(o * i // 2 + 2 * 2 * o * (i // 64) for o, i in BLOCK_SHAPES.values())
    return w + N * (R + DR) * 2 + 264320


def make_block_inputs(torch, M, nset):
    g = torch.Generator(device="cuda")
    g.manual_seed(0x4D4C410005)
    sets = []
    for _ in range(nset):
        w = {}
        for name, (o, i) in BLOCK_SHAPES.items():
            packed = torch.randint(-2 ** 31, 2 ** 31 - 1, (o, i // 8), generator=g, device="cuda", dtype=torch.int32)
            sc = (0.01 * torch.randn(o, i // 64, generator=g, device="cuda")).abs().to(torch.bfloat16)
            bi = (0.01 * torch.randn(o, i // 64, generator=g, device="cuda")).to(torch.bfloat16)
            w[name] = M.AffineWeights(packed, sc, bi)
        for name, n in (("input_norm", 7168), ("q_a_norm", 1536), ("kv_a_norm", 512)):
            w[name] = (1 + 0.02 * torch.randn(n, generator=g, device="cuda")).to(torch.bfloat16)
        cache = (0.5 * torch.randn(N, R + DR, generator=g, device="cuda")).to(torch.bfloat16)
        sets.append((w, cache))
    x = torch.randn(7168, generator=g, device="cuda").to(torch.bfloat16)
    return x, sets


K3_BLOCK = dict(hidden=7168, q_lora_rank=1536, heads=96, nope=128, rope=64, v=128, kv_rank=512)
K3_SHAPES = {"q_a": (1536, 7168), "q_b": (96 * 192, 1536), "kv_a": (576, 7168), "kv_b": (96 * 256, 512),
             "g_proj": (96 * 128, 7168), "o_proj": (7168, 96 * 128)}


def k3_block_bytes():
    """Algorithmic HBM bytes of one K3 attention block for one token: every
    dense bf16 weight once, the cache rows, and the activations (x, the
    projections' outputs, q_lat, ctx, merged, gate, out: 0.4 MB)."""
    w = sum(o * i * 2 for o, i in K3_SHAPES.values())
    act = 2 * (7168 + 1536 * 2 + 96 * 192 + 576 + 96 * 512 * 2 + 96 * 128 * 3 + 7168)
    return w + N * (R + DR) * 2 + act


def time_k3_block(torch, M, steps, warmup, nset=8):
    """The K3 flagship attention layer for one token at position 32767: dense
    bf16 projections (K3 keeps self_attn weights unquantized), NoPE, the
    sigmoid output gate, 96 heads; `nset` weight/cache sets of 502 MB rotate."""
    import ctypes as C

    g = torch.Generator(device="cuda")
    g.manual_seed(0x4D4C41000B)
    sets = []
    for _ in range(nset):
        w = {n: M.DenseWeights((torch.randn(o, i, generator=g, device="cuda") * i ** -0.5).to(torch.bfloat16))
             for n, (o, i) in K3_SHAPES.items()}
        w["input_norm"] = None
        for name, n in (("q_a_norm", 1536), ("kv_a_norm", 512)):
            w[name] = (1 + 0.02 * torch.randn(n, generator=g, device="cuda")).to(torch.bfloat16)
        cache = (0.5 * torch.randn(N, R + DR, generator=g, device="cuda")).to(torch.bfloat16)
        sets.append((w, cache))
    x = torch.randn(7168, generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty(7168, dtype=torch.bfloat16, device="cuda")
    args, ws = [], None
    for w, cache in sets:
        a, ws = M.block_args(x, w, cache, N - 1, None, None, out, workspace=ws, eps=1e-5, **K3_BLOCK)
        args.append(a)
    lib = M.load()
    sp = M._stream(torch.cuda.current_stream())
    for i in range(warmup):
        M._check(lib.mr_mla_decode_block(C.byref(args[i % nset]), sp))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        M._check(lib.mr_mla_decode_block(C.byref(args[i % nset]), sp))
    torch.cuda.synchronize()
    return {"wall_ms": (time.perf_counter() - t0) / steps * 1e3}


def time_decode_96(torch, M, steps, warmup, nbuf=10):
    """Absorbed decode at the K3 flagship's 96 heads over 32768 rows (the
    rows rotate over nbuf caches)."""
    import ctypes as C

    g = torch.Generator(device="cuda")
    g.manual_seed(0x4D4C410096)
    q_lat = torch.randn(1, 96, R, generator=g, device="cuda").to(torch.bfloat16)
    q_rope = torch.randn(1, 96, DR, generator=g, device="cuda").to(torch.bfloat16)
    caches = [(0.5 * torch.randn(N, R + DR, generator=g, device="cuda")).to(torch.bfloat16) for _ in range(nbuf)]
    out = torch.empty(1, 96, R, dtype=torch.bfloat16, device="cuda")
    args, ws = [], None
    for c in caches:
        a, _, ws = M.decode_args(q_lat, q_rope, c[:, :R], c[:, R:], scale=SCALE, out=out, workspace=ws)
        args.append(a)
    lib = M.load()
    sp = M._stream(torch.cuda.current_stream())
    for i in range(warmup):
        M._check(lib.mr_mla_decode(C.byref(args[i % nbuf]), sp))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        M._check(lib.mr_mla_decode(C.byref(args[i % nbuf]), sp))
    torch.cuda.synchronize()
    return {"wall_ms": (time.perf_counter() - t0) / steps * 1e3}


def time_block(torch, M, steps, warmup, nset=8):
    """The decode block (affine 4-bit projections + absorbed attention over a
    32768-row cache) for one token at position 32767; `nset` weight/cache
    sets (143 MB each) rotate so the Infinity Cache cannot hold the operands."""
    import ctypes as C
    import numpy as np

    x, sets = make_block_inputs(torch, M, nset)
    pos = N - 1
    c, s = M.rope_table(np.array([pos]), M.rope_frequencies(DR))
    cos_t, sin_t = torch.from_numpy(c).cuda(), torch.from_numpy(s).cuda()
    out = torch.empty(7168, dtype=torch.bfloat16, device="cuda")
    args, ws = [], None
    for w, cache in sets:
        a, ws = M.block_args(x, w, cache, pos, cos_t, sin_t, out, workspace=ws, **BLOCK)
        args.append(a)
    lib = M.load()
    sp = M._stream(torch.cuda.current_stream())
    for i in range(warmup):
        M._check(lib.mr_mla_decode_block(C.byref(args[i % nset]), sp))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        M._check(lib.mr_mla_decode_block(C.byref(args[i % nset]), sp))
    torch.cuda.synchronize()
    return {"wall_ms": (time.perf_counter() - t0) / steps * 1e3}


MFMA_PEAK_TFLOPS = 2500.0  # dense bf16
PREFILL_T = 4096
# algorithmic work of the causal prefill (T = P = 4096, 128 heads): the
# up-projection 2*T*512*(128*256), QK 2*192 and PV 2*128 flops per visible
# (query, key) pair per head, T(T+1)/2 pairs
UPPROJ_FLOP = 2 * PREFILL_T * 512 * 128 * 256
ATTN_FLOP = (2 * 192 + 2 * 128) * 128 * PREFILL_T * (PREFILL_T + 1) // 2


def time_prefill(torch, M, steps, warmup):
    """Causal prefill, 4096 tokens over a 4096-row latent cache, 128 heads:
    q [4096,128,192] ~N(0,1), latent ~N(0,0.5), kv_b_proj [32768,512] ~N(0,0.02)."""
    import ctypes as C

    g = torch.Generator(device="cuda")
    g.manual_seed(0x4D4C410003)
    T = PREFILL_T
    q = torch.randn(T, H, 192, generator=g, device="cuda").to(torch.bfloat16)
    cache = (0.5 * torch.randn(T, R + DR, generator=g, device="cuda")).to(torch.bfloat16)
    kv_b = (0.02 * torch.randn(H * 256, R, generator=g, device="cuda")).to(torch.bfloat16)
    a, out, ws = M.prefill_args(q, cache[:, :R], cache[:, R:], kv_b)
    lib = M.load()
    sp = M._stream(torch.cuda.current_stream())
    for _ in range(warmup):
        M._check(lib.mr_mla_prefill(C.byref(a), sp))
    torch.cuda.synchronize()
    evs = make_events(torch, steps)
    handles = [(C.c_void_p * 3)(*[e.cuda_event for e in ev]) for ev in evs]
    t0 = time.perf_counter()
    for i in range(steps):
        a.phase_events = C.cast(handles[i], C.c_void_p)
        M._check(lib.mr_mla_prefill(C.byref(a), sp))
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    up_ms = sum(ev[0].elapsed_time(ev[1]) for ev in evs) / steps
    at_ms = sum(ev[1].elapsed_time(ev[2]) for ev in evs) / steps
    return {"wall_ms": wall * 1e3, "upproj_ms": up_ms, "attn_ms": at_ms}


def make_events(torch, n):
    # torch creates the underlying hipEvent lazily: record each once so the
    # handle exists before the library records it
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(n)]
    for ev in evs:
        for e in ev:
            e.record()
    torch.cuda.synchronize()
    return evs


def time_decode(torch, M, steps, warmup):
    nbuf = 10  # 10 x 37.7 MB > 256 MB Infinity Cache
    q_lat, q_rope, caches = make_decode_inputs(torch, nbuf)
    out = torch.empty(1, H, R, dtype=torch.bfloat16, device="cuda")
    args = []
    ws = None
    for c in caches:
        a, _, ws = M.decode_args(q_lat, q_rope, c[:, :R], c[:, R:], scale=SCALE, out=out, workspace=ws)
        args.append(a)
    lib = M.load()
    stream = torch.cuda.current_stream()
    sp = M._stream(stream)
    import ctypes as C

    for i in range(warmup):
        M._check(lib.mr_mla_decode(C.byref(args[i % nbuf]), sp))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        M._check(lib.mr_mla_decode(C.byref(args[i % nbuf]), sp))
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps

    # per-kernel breakdown with the phase-accounting events
    n_ev = min(steps, 200)
    evs = make_events(torch, n_ev)
    handles = [(C.c_void_p * 3)(*[e.cuda_event for e in ev]) for ev in evs]
    for i in range(n_ev):
        a = args[i % nbuf]
        a.phase_events = C.cast(handles[i], C.c_void_p)
        M._check(lib.mr_mla_decode(C.byref(a), sp))
        a.phase_events = None
    torch.cuda.synchronize()
    split_ms = sum(ev[0].elapsed_time(ev[1]) for ev in evs) / n_ev
    layer_ms = sum(ev[0].elapsed_time(ev[2]) for ev in evs) / n_ev
    return {"wall_ms": wall * 1e3, "split_ms": split_ms, "layer_ms": layer_ms,
            "split_kernel_ms": time_split_only(torch, M, args, steps), "splits": None}


def time_split_only(torch, M, args, steps):
    """Average duration of the split kernel alone: `steps` launches with
    MR_DECODE_SPLIT_ONLY between two events on the launch stream, so no
    per-launch event sits between kernels."""
    import ctypes as C

    lib = M.load()
    sp = M._stream(torch.cuda.current_stream())
    for a in args:
        a.flags |= M.DECODE_SPLIT_ONLY
    try:
        for i in range(5):
            M._check(lib.mr_mla_decode(C.byref(args[i % len(args)]), sp))
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            M._check(lib.mr_mla_decode(C.byref(args[i % len(args)]), sp))
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps
    finally:
        for a in args:
            a.flags &= ~M.DECODE_SPLIT_ONLY


def time_sparse(torch, M, steps, warmup, checked=True):
    """Sparse top-2048 decode, B=4, H=128, 128K-row caches.  checked: the
    index lists are checked on the device in the same launch (a status
    buffer, the C-ABI's asynchronous form); else MR_DECODE_UNCHECKED."""
    q_lat, q_rope, caches, sets = make_sparse_inputs(torch, 2, 16)
    out = torch.empty(4, H, R, dtype=torch.bfloat16, device="cuda")
    status = torch.zeros(4, 3, dtype=torch.int32, device="cuda")
    import ctypes as C

    lib = M.load()
    sp = M._stream(torch.cuda.current_stream())
    args, ws = [], None
    for i in range(32):
        c = caches[i % 2]
        a, _, ws = M.decode_args(q_lat, q_rope, c[..., :R], c[..., R:], scale=SCALE, indices=sets[i % 16], out=out,
                                 workspace=ws, index_status=status if checked else None,
                                 flags=0 if checked else M.DECODE_UNCHECKED)
        args.append(a)
    for i in range(warmup):
        M._check(lib.mr_mla_decode(C.byref(args[i % 32]), sp))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        M._check(lib.mr_mla_decode(C.byref(args[i % 32]), sp))
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    n_ev = min(steps, 200)
    evs = make_events(torch, n_ev)
    handles = [(C.c_void_p * 3)(*[e.cuda_event for e in ev]) for ev in evs]
    for i in range(n_ev):
        a = args[i % 32]
        a.phase_events = C.cast(handles[i], C.c_void_p)
        M._check(lib.mr_mla_decode(C.byref(a), sp))
        a.phase_events = None
    torch.cuda.synchronize()
    split_ms = sum(ev[0].elapsed_time(ev[1]) for ev in evs) / n_ev
    layer_ms = sum(ev[0].elapsed_time(ev[2]) for ev in evs) / n_ev
    return {"wall_ms": wall * 1e3, "split_ms": split_ms, "layer_ms": layer_ms,
            "split_kernel_ms": time_split_only(torch, M, args, steps)}


def time_topk(torch, M, steps=200):
    """Lightning-indexer selection of one decode token: 2048 of 32768
    compressed keys (position 131071, ratio 4), scores ~N(0,1) f32; average
    of `steps` launches between two events (no NaN check, no sync)."""
    import ctypes as C

    lib = M.load()
    rows, cols, k, ratio, start = 1, 32768, 2048, 4, 131071
    g = torch.Generator(device="cuda")
    g.manual_seed(0x4D4C410004)
    scores = torch.randn(rows, cols, generator=g, device="cuda")
    sel = M.topk_geometry(rows, cols, k, ratio, start, 0)
    out = torch.empty(rows, sel, dtype=torch.int32, device="cuda")
    ws = torch.empty(max(lib.mr_topk_workspace_size(rows, cols, k), 1), dtype=torch.uint8, device="cuda")
    a = M.TopkArgs()
    a.scores, a.score_row_stride, a.rows, a.cols = scores.data_ptr(), scores.stride(0), rows, cols
    a.top_k, a.ratio, a.start_pos, a.offset = k, ratio, start, 0
    a.out, a.out_row_stride = out.data_ptr(), out.stride(0)
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    a.status, a.flags = status.data_ptr(), 0   # NaN status on the device, no host read
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    sp = M._stream(torch.cuda.current_stream())
    for _ in range(20):
        M._check(lib.mr_topk_select(C.byref(a), sp))
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        M._check(lib.mr_topk_select(C.byref(a), sp))
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_indexer(torch, M, steps=200, nbuf=8):
    """Lightning-index scores of one decode token: 64 index heads of dim 128
    over 32768 compressed keys (bf16, 8 MiB), weights f32; the keys rotate
    over `nbuf` copies so each launch streams them from HBM; average of
    `steps` launches between two events."""
    import ctypes as C

    lib = M.load()
    S, H, D, T = 1, 64, 128, 32768
    g = torch.Generator(device="cuda")
    g.manual_seed(0x4D4C410005)
    q = torch.randn(S, H, D, generator=g, device="cuda").to(torch.bfloat16)
    keys = [torch.randn(T, D, generator=g, device="cuda").to(torch.bfloat16) for _ in range(nbuf)]
    w = torch.randn(S, H, generator=g, device="cuda") * (D * H) ** -0.5
    out = torch.empty(S, T, dtype=torch.float32, device="cuda")
    sp = M._stream(torch.cuda.current_stream())

    def run(i):
        k = keys[i % nbuf]
        M._check(lib.mr_indexer_scores(q.data_ptr(), M.BF16, S, H, D, q.stride(0), q.stride(1), k.data_ptr(), M.BF16,
                                       T, D, k.stride(0), w.data_ptr(), M.F32, S, H, w.stride(0), out.data_ptr(),
                                       out.stride(0), sp))

    for i in range(20):
        run(i)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        run(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def time_gather(torch, M, steps=200, nbuf=4):
    """Routed-expert affine GEMV of one decode token: 8 of 128 experts of a
    4-bit, group-64 [768, 2048] stack (bf16 scales), random distinct ids per
    launch set; stacks rotate over `nbuf` copies; average of `steps` launches
    between two events."""
    import ctypes as C

    lib = M.load()
    E, K, out_f, in_f = 128, 8, 768, 2048
    g = torch.Generator(device="cuda")
    g.manual_seed(0x4D4C410006)
    ws = []
    for _ in range(nbuf):
        packed = torch.randint(-2**31, 2**31 - 1, (E, out_f, in_f // 8), generator=g, dtype=torch.int32, device="cuda")
        scales = (torch.rand(E, out_f, in_f // 64, generator=g, device="cuda") * 0.01).to(torch.bfloat16)
        biases = (torch.randn(E, out_f, in_f // 64, generator=g, device="cuda") * 0.01).to(torch.bfloat16)
        ws.append(M.AffineWeights(packed, scales, biases))
    descs = [w.desc() for w in ws]
    x = torch.randn(1, in_f, generator=g, device="cuda").to(torch.bfloat16)
    ids = [torch.randperm(E, generator=g, device="cuda")[:K].to(torch.int32).reshape(1, K) for _ in range(16)]
    y = torch.empty(1, K, out_f, dtype=torch.bfloat16, device="cuda")
    sp = M._stream(torch.cuda.current_stream())

    def run(i):
        M._check(lib.mr_affine_gather_matmul(x.data_ptr(), M.BF16, 1, x.stride(0), C.byref(descs[i % nbuf]), E,
                                             ids[i % 16].data_ptr(), K, y.data_ptr(), M.BF16, sp))

    for i in range(20):
        run(i)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        run(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def mfma_probe(torch, M):
    """On-box MFMA rate: one 256-thread workgroup per CU, each wave 8
    independent 32x32x16 bf16 MFMA chains for 4000 rounds, no memory traffic
    in the loop.  Returns the dense bf16 rate and the shader clock it ran at
    (s_memtime cycles over 100 MHz wall-clock ticks, mean over workgroups)."""
    import ctypes as C

    lib = C.CDLL(M.SELFTEST_PATH)
    lib.mr_selftest_mfma_rate.argtypes = [C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
    blocks, iters = 256, 4000
    sink = torch.empty(blocks * 256, dtype=torch.float32, device="cuda")
    stamps = torch.zeros(2 * blocks, dtype=torch.int64, device="cuda")
    sp = M._stream(torch.cuda.current_stream())
    for _ in range(2):
        assert lib.mr_selftest_mfma_rate(blocks, iters, sink.data_ptr(), stamps.data_ptr(), sp) == 0
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    assert lib.mr_selftest_mfma_rate(blocks, iters, sink.data_ptr(), stamps.data_ptr(), sp) == 0
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1)
    flop = blocks * 4 * iters * 8 * 2 * 32 * 32 * 16
    st = stamps.view(blocks, 2).double().cpu()
    clock_ghz = float(st[:, 0].mean() / (st[:, 1].mean() * 10.0))
    return {"tflops": round(flop / (ms * 1e-3) / 1e12, 1), "clock_ghz": round(clock_ghz, 3)}


def torch_cpu_decode(torch, threads, budget_s=8.0):
    """The same decode layer as fp32 BLAS products on the host (torch CPU):
    S = (q_lat . c^T + q_rope . k^T) * scale, softmax, O = P . c; median of
    whole layers within the time budget."""
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(0x4D4C410002)
    q_lat = torch.randn(H, R, generator=g)
    q_rope = torch.randn(H, DR, generator=g)
    cache = 0.5 * torch.randn(N, R + DR, generator=g)
    lat, rk = cache[:, :R], cache[:, R:]

    def layer():
        s = (q_lat @ lat.T + q_rope @ rk.T) * SCALE
        return torch.softmax(s, dim=-1) @ lat

    layer()
    times = []
    t_start = time.perf_counter()
    while len(times) < 3 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        layer()
        times.append(time.perf_counter() - t0)
        if len(times) >= 200:
            break
    times.sort()
    return times[len(times) // 2], len(times)


PROJ_T = 4096
# prefill-sized projections (T = 4096 tokens): the 4-bit affine block shapes
# (group 64, bf16 scales) and the K3 dense bf16 ones, [out, in]
PROJ_AFFINE = [("q_a", 1536, 7168), ("q_b", 24576, 1536), ("kv_a", 576, 7168), ("o_proj", 7168, 16384)]
PROJ_DENSE = [("q_a", 1536, 7168), ("q_b", 18432, 1536), ("kv_a", 576, 7168), ("o_proj", 7168, 12288)]


def time_projections(torch, M, reps=20):
    """mr_affine_matmul / mr_linear at T = 4096 on each shape (bf16 x and y,
    random weights): the average duration of `reps` back-to-back launches
    between two events, and the aggregate algorithmic TFLOP/s (2 T out in
    per projection)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(0x50524F4A)
    out = {}
    for kind, shapes in (("affine_4bit", PROJ_AFFINE), ("dense_bf16", PROJ_DENSE)):
        res, flop_total, us_total = {}, 0.0, 0.0
        for name, n, k in shapes:
            x = torch.randn(PROJ_T, k, generator=g, device="cuda").to(torch.bfloat16)
            if kind == "affine_4bit":
                packed = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), generator=g, device="cuda", dtype=torch.int32)
                sc = (torch.rand(n, k // 64, generator=g, device="cuda") * 0.01).to(torch.bfloat16)
                bi = (torch.randn(n, k // 64, generator=g, device="cuda") * 0.01).to(torch.bfloat16)
                w = M.AffineWeights(packed, sc, bi)
                call = lambda: M.affine_mm(x, w)  # noqa: E731
            else:
                w = M.DenseWeights((torch.randn(n, k, generator=g, device="cuda") * k ** -0.5).to(torch.bfloat16))
                call = lambda: M.linear(x, w)  # noqa: E731
            for _ in range(3):
                call()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                call()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / reps * 1e3
            flop = 2.0 * PROJ_T * n * k
            res[f"{name}_us"] = round(us, 1)
            flop_total += flop
            us_total += us
        res["tflops"] = round(flop_total / (us_total * 1e-6) / 1e12, 1)
        res["mfma_fraction"] = round(flop_total / (us_total * 1e-6) / 1e12 / MFMA_PEAK_TFLOPS, 4)
        out[kind] = res
    return out


def time_prefill_block(torch, M, reps=10):
    """The K3 attention block over a 4096-token prompt in one call
    (mr_mla_prefill_block, K3MLA.forward with state == nil): hidden 7168, 96
    heads, q_lora 1536, dense bf16 weights ~N(0, 1/in), gate, NoPE.  The
    average of `reps` back-to-back calls between two events, and the
    projections' share of the flops."""
    import ctypes as C

    g = torch.Generator(device="cuda")
    g.manual_seed(0x4B33504246)
    T, Hk, hid, ql = PROJ_T, 96, 7168, 1536

    def dw(o, i):
        return M.DenseWeights((torch.randn(o, i, generator=g, device="cuda") * i ** -0.5).to(torch.bfloat16))

    w = {"input_norm": None,
         "q_a_norm": (1 + 0.02 * torch.randn(ql, generator=g, device="cuda")).to(torch.bfloat16),
         "kv_a_norm": (1 + 0.02 * torch.randn(R, generator=g, device="cuda")).to(torch.bfloat16),
         "q_a": dw(ql, hid), "q_b": dw(Hk * 192, ql), "kv_a": dw(R + DR, hid), "kv_b": dw(Hk * 256, R),
         "o_proj": dw(hid, Hk * 128), "g_proj": dw(Hk * 128, hid)}
    x = torch.randn(T, hid, generator=g, device="cuda").to(torch.bfloat16)
    cache = torch.zeros(T, R + DR, device="cuda", dtype=torch.bfloat16)
    out = torch.empty(T, hid, device="cuda", dtype=torch.bfloat16)
    a, ws = M.prefill_block_args(x, w, cache, 0, None, None, out, q_lora_rank=ql, heads=Hk, nope=128, rope=DR,
                                 v=128, kv_rank=R)
    lib = M.load()
    sp = M._stream(torch.cuda.current_stream())
    for _ in range(3):
        M._check(lib.mr_mla_prefill_block(C.byref(a), sp))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        M._check(lib.mr_mla_prefill_block(C.byref(a), sp))
    e1.record()
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / reps * 1e3
    proj = 2.0 * T * (ql * hid + (R + DR) * hid + Hk * 128 * hid + Hk * 192 * ql + hid * Hk * 128)
    attn = ATTN_FLOP * Hk / H + UPPROJ_FLOP * Hk / H
    return {"us": round(us, 1), "projection_tflop": round(proj / 1e12, 3), "attention_tflop": round(attn / 1e12, 3),
            "tflops": round((proj + attn) / (us * 1e-6) / 1e12, 1), "workspace_mb": round(ws.numel() / 1e6, 1)}


def cpu_baseline(torch, budget_s=4.0):
    """The decode layer (H=128, N=32768) on this host's cores.  The value is
    the layer as torch-CPU fp32 BLAS products (the fastest CPU form of the
    reference's computation here: a port of the algorithm onto the host's
    BLAS); beside it, the oracle's scalar C loop (OpenMP over heads), timed
    on a bounded sample of at least 2 layers within `budget_s`.  Threads:
    every core of the process's CPU share (OMP_NUM_THREADS when set, else the
    affinity mask)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O

    visible = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    threads = max(1, min(visible, int(os.environ.get("OMP_NUM_THREADS", visible))))
    t_blas, n_blas = torch_cpu_decode(torch, threads)

    ql = O.normal_bf16("c2.q_lat", (H, R), threads=threads)
    qr = O.normal_bf16("c2.q_rope", (H, DR), threads=threads)
    cache = O.normal_bf16("c2.cache", (N, R + DR), std=0.5, threads=threads)
    O.mla_decode(ql, qr, cache, acc=0, threads=threads)  # warm
    times = []
    t_start = time.perf_counter()
    while len(times) < 2 or time.perf_counter() - t_start < budget_s:
        t0 = time.perf_counter()
        O.mla_decode(ql, qr, cache, acc=0, threads=threads)
        times.append(time.perf_counter() - t0)
        if len(times) >= 20:
            break
    times.sort()
    med = times[len(times) // 2]
    try:
        model = [l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo") if l.startswith("model name")][0]
    except Exception:
        model = platform.processor()
    blas = "MKL" if torch.backends.mkl.is_available() else "torch's default CPU BLAS"
    return {"value": round(t_blas * 1e6, 1), "unit": "us/layer", "cores": threads, "kind": "port",
            "path": f"torch CPU fp32 BLAS ({blas})", "host": model,
            "sample": f"{n_blas} full decode layers (H=128, N=32768) as torch CPU fp32 BLAS products "
                      f"(S = q_lat c^T + q_rope k^T, softmax, P c), median; {threads} threads = the process's "
                      f"CPU share ({visible} cores visible)",
            "oracle_scalar": {"value": round(med * 1e6, 1), "unit": "us/layer", "threads": threads,
                              "sample": f"{len(times)} layers of the oracle's scalar C loop (OpenMP over heads), "
                                        "median"}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=400)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain streaming kernel of known size (torch.neg over 64M fp32, 256 MiB read + "
                         "256 MiB written, 3 launches) so HBM counters can be scaled to bytes")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported "
              "(the decode path runs on one GPU; sharding the context across GPUs is a design sketch, not built)",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import minirun_hip as M

    M.load()
    log(f"bench: decode H={H} N={N} steps={args.steps} warmup={args.warmup}")
    d = time_decode(torch, M, args.steps, args.warmup)
    log(f"bench: decode {d}")
    log("bench: sparse B=4 H=128 N=131072 K=2048")
    s = time_sparse(torch, M, args.steps, args.warmup)
    log(f"bench: sparse {s}")
    su = time_sparse(torch, M, args.steps, args.warmup, checked=False)
    log(f"bench: sparse, no index checks {su}")
    log("bench: decode block, hidden 7168, affine 4-bit g64, ctx 32768")
    blk = time_block(torch, M, args.steps, args.warmup)
    log(f"bench: block {blk}")
    log("bench: K3 attention block, dense bf16, 96 heads, NoPE, gated, ctx 32768")
    k3 = time_k3_block(torch, M, args.steps, args.warmup)
    log(f"bench: k3 block {k3}")
    d96 = time_decode_96(torch, M, args.steps, args.warmup)
    log(f"bench: decode 96 heads {d96}")
    log("bench: causal prefill T=4096 H=128")
    pf = time_prefill(torch, M, max(args.steps // 2, 200), max(args.warmup // 2, 20))
    log(f"bench: prefill {pf}")
    tk_ms = time_topk(torch, M)
    log(f"bench: top-k 2048 of 32768 {tk_ms * 1e3:.2f} us")
    log("bench: lightning-index scores, 64 heads x 128, 32768 keys")
    ix_ms = time_indexer(torch, M)
    log(f"bench: indexer scores {ix_ms * 1e3:.2f} us")
    log("bench: routed-expert GEMV, 8 of 128 experts of [768, 2048] 4-bit")
    gx_ms = time_gather(torch, M)
    log(f"bench: gather {gx_ms * 1e3:.2f} us")
    log(f"bench: projections at T={PROJ_T} (4-bit affine and dense bf16, MFMA)")
    pj = time_projections(torch, M)
    log(f"bench: projections {pj}")
    log(f"bench: K3 prefill block, {PROJ_T} tokens in one call")
    pb = time_prefill_block(torch, M)
    log(f"bench: prefill block {pb}")
    mp = mfma_probe(torch, M)
    log(f"bench: mfma probe {mp}")

    layer_us = d["wall_ms"] * 1e3
    split_s = d["split_kernel_ms"] * 1e-3
    achieved = split_kernel_bytes() / split_s / 1e9
    result = {
        "metric": "MLA decode us/layer + % HBM peak (128 heads, 32K ctx); sparse top-2048 us",
        "value": round(layer_us, 3),
        "unit": "us/layer",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(d["wall_ms"], 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (torch RNG, fixed seed; q~N(0,1), cache~N(0,0.5) bf16)",
        "config": {"workload": "mla_absorbed_decode", "batch": 1, "heads": H, "context": N,
                   "kv_lora_rank": R, "rope_dim": DR, "softmax": "fp32", "out": "bf16",
                   "cache_rotation": 10},
        "hbm_fraction_layer": round(cache_bytes_per_layer() / (d["wall_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "layer_us_events": round(d["layer_ms"] * 1e3, 3),
        "split_kernel_us": round(d["split_kernel_ms"] * 1e3, 3),
        "split_us_events": round(d["split_ms"] * 1e3, 3),
        "sparse_top2048_us": round(s["wall_ms"] * 1e3, 3),
        "sparse_split_kernel_us": round(s["split_kernel_ms"] * 1e3, 3),
        "sparse_unchecked_us": round(su["wall_ms"] * 1e3, 3),
        "sparse_hbm_fraction": round(sparse_bytes() / (s["wall_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "block_us": round(blk["wall_ms"] * 1e3, 3),
        "block_hbm_fraction": round(block_bytes() / (blk["wall_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "k3_block_us": round(k3["wall_ms"] * 1e3, 3),
        "k3_block_hbm_fraction": round(k3_block_bytes() / (k3["wall_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "block_weight_cache_sets": 8,
        "decode_96_heads_us": round(d96["wall_ms"] * 1e3, 3),
        "prefill_us": round(pf["wall_ms"] * 1e3, 2),
        "prefill_mfma_fraction": round((UPPROJ_FLOP + ATTN_FLOP) / (pf["wall_ms"] * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
        "prefill_upproj_us": round(pf["upproj_ms"] * 1e3, 2),
        "prefill_attn_us": round(pf["attn_ms"] * 1e3, 2),
        "prefill_attn_mfma_fraction": round(ATTN_FLOP / (pf["attn_ms"] * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4),
        "topk_2048_of_32768_us": round(tk_ms * 1e3, 2),
        "indexer_scores_32768_us": round(ix_ms * 1e3, 2),
        "indexer_hbm_fraction": round(32768 * 128 * 2 / (ix_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "gather_8x768x2048_us": round(gx_ms * 1e3, 2),
        "gather_hbm_fraction": round(8 * 768 * (2048 // 2 + 4 * 2048 // 64) / (gx_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "projections_t4096": pj,
        "k3_prefill_block_t4096": pb,
        "mfma_probe_tflops": mp["tflops"],
        "mfma_probe_clock_ghz": mp["clock_ghz"],
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": SPLIT_TRAFFIC_BYTES,
                     "traffic_source": SPLIT_TRAFFIC_SOURCE,
                     "kernel": "mla_decode_ws", "algorithmic_bytes": split_kernel_bytes(),
                     "layer_frac": round(cache_bytes_per_layer() / (d["wall_ms"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
    }
    if args.copy_calibration:
        src = torch.randn(64 << 20, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.neg(src, out=dst)
        torch.cuda.synchronize()
        log("bench: copy calibration: 3 x neg over 268435456 B read + 268435456 B written")
    if not args.no_cpu_baseline:
        log("bench: cpu baseline (torch CPU BLAS, then the oracle loop)")
        result["cpu_baseline"] = cpu_baseline(torch)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
