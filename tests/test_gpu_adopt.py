"""Adopted affine weights on the device (AffineWeights.adopting,
MLXBridge/AffineWeights.swift:159-198): a GEMV through the adopted weight's
descriptor equals the one through the same buffers' plain descriptor bit
for bit, and the finalizers run exactly once, only after the stream named
at the last release has passed the read (the stream is held busy by a
bounded spin kernel first, so the release call returns long before it)."""
import threading
import time

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def M():
    import minirun_hip as M

    M.load()
    return M


def dev(a):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(a))
    if a.dtype == np.uint16:
        t = t.view(torch.bfloat16)
    elif a.dtype == np.uint32:
        t = t.view(torch.int32)
    return t.cuda()


def test_adopted_weight_gemv_and_stream_ordered_release(M):
    import torch

    out_f, in_f = 1536, 7168
    print(f"adopt: affine 4-bit [{out_f}, {in_f}], GEMV, release behind a busy stream", flush=True)
    packed = dev(O.u32("ad.p", (out_f, in_f // 8)))
    scales = dev(O.abs_normal_bf16("ad.s", (out_f, in_f // 64), std=0.01))
    biases = dev(O.normal_bf16("ad.b", (out_f, in_f // 64), std=0.01))
    x = dev(O.normal_bf16("ad.x", (1, in_f)))
    ref = M.affine_mm(x, M.AffineWeights(packed, scales, biases))

    calls = []
    lock = threading.Lock()

    def fin(i):
        def f(ctx):
            with lock:
                calls.append((i, ctx, time.perf_counter()))

        return f

    w = M.AdoptedAffineWeights(packed.data_ptr(), scales.data_ptr(), biases.data_ptr(), M.BF16, out_f, in_f,
                               finalizers=(fin(0), fin(1), fin(2)), contexts=(1, 2, 3))
    w.retain()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        torch.cuda._sleep(200_000_000)  # a bounded spin (about 0.1 s) ahead of the read
        y = M.affine_mm(x, w, stream=s)
    done = torch.cuda.Event()
    done.record(s)
    w.release(s)   # one holder left: nothing runs
    w.release(s)   # the last: the finalizers go behind the GEMV
    t_release = time.perf_counter()
    assert calls == [], "finalizers ran before the stream passed the read"
    assert not done.query(), "the stream finished before the check (the spin was too short to tell)"
    s.synchronize()
    for _ in range(100):  # the host function runs on a runtime thread
        if len(calls) == 3:
            break
        time.sleep(0.01)
    assert sorted((i, c) for i, c, _ in calls) == [(0, 1), (1, 2), (2, 3)]
    assert all(t > t_release for _, _, t in calls)
    assert torch.equal(y, ref)


def test_release_with_null_stream_waits_for_the_default_stream(M):
    # stream NULL is the default stream, as in every other entry point: the
    # last release through the raw C-ABI with NULL, behind a GEMV on the
    # default stream held busy by a bounded spin, runs the finalizers only
    # after that GEMV (AffineWeights.swift:159-198: the finalizer never runs
    # before the last GPU use)
    import ctypes as C

    import torch

    out_f, in_f = 1536, 7168
    print("adopt: release(NULL) behind a busy default stream", flush=True)
    packed = dev(O.u32("adn.p", (out_f, in_f // 8)))
    scales = dev(O.abs_normal_bf16("adn.s", (out_f, in_f // 64), std=0.01))
    biases = dev(O.normal_bf16("adn.b", (out_f, in_f // 64), std=0.01))
    x = dev(O.normal_bf16("adn.x", (1, in_f)))
    ref = M.affine_mm(x, M.AffineWeights(packed, scales, biases))
    torch.cuda.synchronize()

    calls = []
    lock = threading.Lock()

    def fin(i):
        def f(ctx):
            with lock:
                calls.append((i, ctx, time.perf_counter()))

        return f

    w = M.AdoptedAffineWeights(packed.data_ptr(), scales.data_ptr(), biases.data_ptr(), M.BF16, out_f, in_f,
                               finalizers=(fin(0), fin(1), fin(2)), contexts=(4, 5, 6))
    default = torch.cuda.default_stream()
    assert default.cuda_stream == 0, "the default stream's handle is the null stream here"
    with torch.cuda.stream(default):
        torch.cuda._sleep(200_000_000)  # a bounded spin (about 0.1 s) ahead of the read
        y = M.affine_mm(x, w, stream=default)
        done = torch.cuda.Event()
        done.record(default)
    h = w.handle
    del w  # the finalizers are reached through the module's one callback
    assert M.load().mr_adopted_affine_release(C.c_void_p(h), None) == M.OK
    t_release = time.perf_counter()
    assert calls == [], "finalizers ran before the default stream passed the read"
    assert not done.query(), "the stream finished before the check (the spin was too short to tell)"
    torch.cuda.synchronize()
    for _ in range(100):
        if len(calls) == 3:
            break
        time.sleep(0.01)
    assert sorted((i, c) for i, c, _ in calls) == [(0, 4), (1, 5), (2, 6)]
    assert all(t > t_release for _, _, t in calls)
    assert torch.equal(y, ref)
