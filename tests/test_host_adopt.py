"""Adopted affine weights (AffineWeights.adopting, MLXBridge/AffineWeights.swift:
159-198): ownership of three buffers passes to the weight, each finalizer
runs exactly once after the last holder releases it (releases may come
from any thread, BufferPool.swift:45-90), and a failed adoption runs them
before its error, since the reference's arrays own the pointers before its
validation.  Host-side checks only: the last holder releases with
release_now (no stream), so nothing runs on a device (the pointers are
never dereferenced)."""
import threading

import pytest

import minirun_hip as M


def recorder():
    calls = []
    lock = threading.Lock()

    def make(i):
        def fin(ctx):
            with lock:
                calls.append((i, ctx))

        return fin

    return calls, [make(i) for i in range(3)]


def adopt(fins, **kw):
    args = dict(experts=0, group_size=64, bits=4, finalizers=fins, contexts=(11, 22, 33))
    args.update(kw)
    return M.AdoptedAffineWeights(0x10000, 0x20000, 0x30000, M.BF16, 1536, 7168, **args)


@pytest.fixture(scope="module", autouse=True)
def lib():
    M.load()


def test_finalizers_run_once_after_the_last_release():
    calls, fins = recorder()
    w = adopt(fins)
    d = w.desc()
    assert (d.packed, d.scales, d.biases) == (0x10000, 0x20000, 0x30000)
    assert (d.out_features, d.in_features, d.group, d.bits, d.scale_dtype) == (1536, 7168, 64, 4, M.BF16)
    w.retain()
    w.retain()
    w.release_now()
    w.release_now()
    assert calls == []
    w.release_now()  # the last holder: the finalizers run now, each once
    assert sorted(calls) == [(0, 11), (1, 22), (2, 33)]


def test_releases_from_other_threads():
    calls, fins = recorder()
    w = adopt(fins)
    for _ in range(8):
        w.retain()
    ts = [threading.Thread(target=w.release_now) for _ in range(8)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert calls == []
    w.release_now()
    assert sorted(calls) == [(0, 11), (1, 22), (2, 33)]


def test_expert_stack_geometry():
    calls, fins = recorder()
    w = M.AdoptedAffineWeights(0x10000, 0x20000, 0x30000, M.F16, 768, 2048, experts=128, finalizers=fins,
                               contexts=(1, 2, 3))
    d = w.desc()
    assert (d.out_features, d.in_features, d.scale_dtype) == (768, 2048, M.F16)
    w.release_now()
    assert sorted(calls) == [(0, 1), (1, 2), (2, 3)]


@pytest.mark.parametrize("kw,status", [(dict(bits=5), M.INVALID_SHAPE), (dict(group_size=0), M.INVALID_SHAPE),
                                       (dict(group_size=100), M.INVALID_SHAPE)])
def test_failed_adoption_runs_the_finalizers(kw, status):
    calls, fins = recorder()
    with pytest.raises(M.MRError) as e:
        adopt(fins, **kw)
    assert e.value.status == status
    assert sorted(calls) == [(0, 11), (1, 22), (2, 33)]


def test_bad_scale_dtype_and_null_buffer():
    calls, fins = recorder()
    with pytest.raises(M.MRError) as e:
        M.AdoptedAffineWeights(0x10000, 0x20000, 0x30000, M.U32, 1536, 7168, finalizers=fins, contexts=(1, 2, 3))
    assert e.value.status == M.INVALID_DTYPE and len(calls) == 3
    calls2, fins2 = recorder()
    with pytest.raises(M.MRError) as e:
        M.AdoptedAffineWeights(0x10000, None, 0x30000, M.BF16, 1536, 7168, finalizers=fins2, contexts=(1, 2, 3))
    assert e.value.status == M.INVALID_ARGUMENT and len(calls2) == 3


def test_missing_finalizers_are_allowed():
    calls, fins = recorder()
    w = M.AdoptedAffineWeights(0x10000, 0x20000, 0x30000, M.BF16, 1536, 7168, finalizers=(fins[0], None, None),
                               contexts=(5, None, None))
    w.release_now()
    assert calls == [(0, 5)]


def test_released_handle_is_rejected():
    # a handle after its last release names nothing: every call with it
    # returns INVALID_ARGUMENT (the library keeps a registry of live handles)
    calls, fins = recorder()
    w = adopt(fins)
    w.release_now()
    assert len(calls) == 3
    for call in (w.retain, w.release_now, w.desc):
        with pytest.raises(M.MRError) as e:
            call()
        assert e.value.status == M.INVALID_ARGUMENT
    assert len(calls) == 3


def test_finalizers_outlive_the_python_object():
    # the Python object is dropped before its last reference is released
    # through the raw handle: the finalizers still run, each once (they are
    # reached through one module-level callback, not per-object thunks)
    import ctypes as C
    import gc

    calls, fins = recorder()
    w = adopt(fins)
    h = w.handle
    del w
    gc.collect()
    assert M.load().mr_adopted_affine_release_now(C.c_void_p(h)) == M.OK
    assert sorted(calls) == [(0, 11), (1, 22), (2, 33)]
    assert not M._FINALIZERS
