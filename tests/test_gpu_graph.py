"""The decode and prefill entry points inside a captured HIP graph (torch.cuda.CUDAGraph), as a
serving loop captures one step and replays it.  The entry points
below enqueue only kernels on the caller's stream (no memset, no host sync,
no allocation), so they can be captured; every replay must equal the eager
call bit for bit, with eager work of the program's own and synchronisations
between the replays.  Cases: the dense decode (H=128, N=32768) on a caller
workspace; the same through mr_mla_decode_noalloc (the library's static
scratch, the form for callers that cannot allocate); the gathered decode
with the device-side index status (B=4, K=2048 of 131072 rows); the K3
decode block (dense projections, output gate, 96 heads); the K3 prefill
block over a 64-token chunk."""
import ctypes as C

import numpy as np
import pytest

import mla_inputs as MI
from test_gpu_block import dev, projection

pytestmark = pytest.mark.gpu

REPLAYS = 3


@pytest.fixture(scope="module")
def M():
    import minirun_hip as M

    M.load()
    return M


def capture(fn):
    """fn run once on a side stream (first-call set-up outside the capture),
    then captured into a graph."""
    import torch

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    torch.cuda.synchronize()
    return g


def other_work(M):
    """Eager work between replays: a small decode on other inputs."""
    import torch

    ql, qr, cache = MI.decode_inputs(16, 512, tag="graph.other")
    c = dev(cache)
    out = M.mla_decode(dev(ql), dev(qr), c[:, :512], c[:, 512:], scale=MI.SCALE)
    torch.cuda.synchronize()
    return out


def replay_and_compare(M, g, out, eager, tag):
    import torch

    for r in range(REPLAYS):
        out.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        other_work(M)
        torch.cuda.synchronize()
        same = torch.equal(out.view(torch.int16), eager.view(torch.int16))
        print(f"{tag}: replay {r} bitwise equal to the eager call: {same}", flush=True)
        assert same, f"{tag}: replay {r} differs from the eager call"


def decode_case(M, noalloc):
    import torch

    H, N = 128, 32768
    ql, qr, cache = MI.decode_inputs(H, N, tag="graph.dense")
    keep = [dev(ql), dev(qr), dev(cache)]
    lib = M.load()
    a, out, ws = M.decode_args(keep[0], keep[1], keep[2][..., :512], keep[2][..., 512:], scale=MI.SCALE)
    if noalloc:
        a.workspace, a.workspace_bytes = None, 0
    entry = lib.mr_mla_decode_noalloc if noalloc else lib.mr_mla_decode

    def call():
        assert entry(C.byref(a), M._stream(None)) == M.OK, M.last_error()

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    g = capture(call)
    replay_and_compare(M, g, out, eager, "noalloc decode" if noalloc else "decode")
    return keep, ws


def test_dense_decode_replays(M):
    print("graph: dense decode H=128 N=32768", flush=True)
    decode_case(M, noalloc=False)


def test_noalloc_decode_replays(M):
    print("graph: no-alloc dense decode H=128 N=32768", flush=True)
    decode_case(M, noalloc=True)


def test_gathered_decode_replays(M):
    import torch

    B, H, N, K = 4, 128, 131072, 2048
    print(f"graph: gathered decode B={B} H={H} N={N} K={K}", flush=True)
    ql, qr, cache, idx = MI.sparse_inputs(B, H, N, K, tag="graph.sparse")
    keep = [dev(ql), dev(qr), dev(cache), dev(idx.astype(np.int32))]
    status = torch.full((B, 3), 99, dtype=torch.int32, device="cuda")
    lib = M.load()
    a, out, ws = M.decode_args(keep[0], keep[1], keep[2][..., :512], keep[2][..., 512:], scale=MI.SCALE,
                               indices=keep[3], index_status=status)

    def call():
        assert lib.mr_mla_decode(C.byref(a), M._stream(None)) == M.OK, M.last_error()

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    assert (status.cpu().numpy() == np.array([0, -1, -1])).all()
    g = capture(call)
    replay_and_compare(M, g, out, eager, "gathered decode")
    assert (status.cpu().numpy() == np.array([0, -1, -1])).all()


def test_k3_block_replays(M):
    # the block appends its key row at `position` on every call: the same
    # row, so replays leave the cache as the eager call did
    import torch

    dims = dict(MI.K3_DIMS)
    print("graph: K3 decode block, 96 heads, ctx 32768", flush=True)
    d = MI.k3_block_inputs(tag="graph.k3")
    w = {k: (dev(d[k]) if d.get(k) is not None else None) for k in ("input_norm", "q_a_norm", "kv_a_norm")}
    for k in ("q_a", "q_b", "kv_a", "kv_b", "o_proj", "g_proj"):
        w[k] = projection(M, d.get(k))
    cache = dev(d["cache"])
    x = dev(d["x"])
    out = torch.empty(dims["hidden"], dtype=torch.bfloat16, device="cuda")
    kw = {k: dims[k] for k in ("hidden", "q_lora_rank", "heads", "nope", "rope", "v", "kv_rank")}
    a, ws = M.block_args(x, w, cache, d["position"], None, None, out, eps=1e-5, **kw)
    lib = M.load()

    def call():
        assert lib.mr_mla_decode_block(C.byref(a), M._stream(None)) == M.OK, M.last_error()

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    row = cache[d["position"]].clone()
    g = capture(call)
    replay_and_compare(M, g, out, eager, "K3 decode block")
    assert torch.equal(cache[d["position"]].view(torch.int16), row.view(torch.int16))


def test_k3_prefill_block_replays(M):
    # a 64-token chunk after 100 cached rows (projections on MFMA tiles,
    # attention with the gate in its stores); the cache rows it appends are
    # the same on every replay
    import torch

    dims = dict(MI.K3_DIMS)
    T, position = 64, 100
    print(f"graph: K3 prefill block, {T} tokens after {position} rows", flush=True)
    d = MI.prefill_block_inputs(T, position, "graph.pb", **dims)
    w = {k: (dev(d[k]) if d.get(k) is not None else None) for k in ("input_norm", "q_a_norm", "kv_a_norm")}
    for k in ("q_a", "q_b", "kv_a", "kv_b", "o_proj", "g_proj"):
        w[k] = projection(M, d.get(k))
    cache = dev(d["cache"])
    x = dev(d["x"])
    out = torch.empty(T, dims["hidden"], dtype=torch.bfloat16, device="cuda")
    kw = {k: dims[k] for k in ("q_lora_rank", "heads", "nope", "rope", "v", "kv_rank")}
    a, ws = M.prefill_block_args(x, w, cache, position, None, None, out, **kw)
    lib = M.load()

    def call():
        assert lib.mr_mla_prefill_block(C.byref(a), M._stream(None)) == M.OK, M.last_error()

    call()
    torch.cuda.synchronize()
    eager = out.clone()
    rows = cache[position:].clone()
    g = capture(call)
    replay_and_compare(M, g, out, eager, "K3 prefill block")
    assert torch.equal(cache[position:].view(torch.int16), rows.view(torch.int16))
