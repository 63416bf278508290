"""Calls from several host threads, each on its own stream: the entry points
keep no shared mutable state beyond the per-thread error string and the
cached CU count, so concurrent decodes on separate streams give what the
same calls give one after another, bit for bit, and a refused call on one
thread reports its own error there while the others succeed."""
import ctypes as C
import threading

import pytest

import mla_inputs as MI
from test_gpu_block import dev

pytestmark = pytest.mark.gpu

THREADS = 4


@pytest.fixture(scope="module")
def M():
    import minirun_hip as M

    M.load()
    return M


def test_concurrent_decodes_match_sequential(M):
    import torch

    print(f"{THREADS} threads x dense decode (H=128, N=32768) on their own streams", flush=True)
    lib = M.load()
    cases = []
    for i in range(THREADS):
        ql, qr, cache = MI.decode_inputs(128, 32768, tag=f"thr.{i}")
        keep = [dev(ql), dev(qr), dev(cache)]
        a, out, ws = M.decode_args(keep[0], keep[1], keep[2][..., :512], keep[2][..., 512:], scale=MI.SCALE)
        cases.append((a, out, ws, keep))
    # one after another on the current stream
    ref = []
    for a, out, _, _ in cases:
        assert lib.mr_mla_decode(C.byref(a), M._stream(None)) == M.OK, M.last_error()
        torch.cuda.synchronize()
        ref.append(out.clone())
        out.fill_(float("nan"))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream() for _ in range(THREADS)]
    errors = []
    start = threading.Barrier(THREADS)

    def work(i):
        try:
            a, out, _, _ = cases[i]
            start.wait()
            for _ in range(5):
                st = lib.mr_mla_decode(C.byref(a), C.c_void_p(streams[i].cuda_stream))
                if st != M.OK:
                    errors.append((i, st, M.last_error()))
            streams[i].synchronize()
        except Exception as e:  # pragma: no cover - reported below
            errors.append((i, repr(e)))

    ts = [threading.Thread(target=work, args=(i,)) for i in range(THREADS)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i, (_, out, _, _) in enumerate(cases):
        assert torch.equal(out.view(torch.int16), ref[i].view(torch.int16)), f"thread {i}"


def test_errors_stay_on_their_thread(M):
    # thread 0 makes a refused call (no workspace) while the others decode;
    # each thread reads back its own status and message
    import torch

    lib = M.load()
    ql, qr, cache = MI.decode_inputs(16, 512, tag="thr.err")
    keep = [dev(ql), dev(qr), dev(cache)]
    results = {}
    start = threading.Barrier(THREADS)

    def work(i):
        a, out, ws = M.decode_args(keep[0], keep[1], keep[2][..., :512], keep[2][..., 512:], scale=MI.SCALE)
        if i == 0:
            a.workspace, a.workspace_bytes = None, 0
        s = torch.cuda.Stream()
        start.wait()
        st = lib.mr_mla_decode(C.byref(a), C.c_void_p(s.cuda_stream))
        msg = M.last_error() if st != M.OK else ""
        s.synchronize()
        results[i] = (st, msg, out)

    ts = [threading.Thread(target=work, args=(i,)) for i in range(THREADS)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    torch.cuda.synchronize()
    assert results[0][0] == M.WORKSPACE_TOO_SMALL and "workspace" in results[0][1], results[0][:2]
    for i in range(1, THREADS):
        assert results[i][0] == M.OK and results[i][1] == "", results[i][:2]
        assert torch.equal(results[i][2].view(torch.int16), results[1][2].view(torch.int16))
