"""Pins the oracle's seeded generator and bf16 rounding (CPU only).

SplitMix64 follows StorageCore/Generator/SplitMix64.swift:13-50; the checks
here are the published SplitMix64 test vector, the reference's own
"value(seed, i) equals the i-th next()" identity
(Tests/StorageCoreTests/DeterministicContentTests.swift:6-20), and an
independent Python restatement of the uniform/Box-Muller layer.
"""
import math

import numpy as np
import pytest

import oracle as O

M64 = (1 << 64) - 1


class PySplitMix:
    """Sequential stream written from the published algorithm."""

    def __init__(self, seed):
        self.state = seed & M64

    def next(self):
        self.state = (self.state + 0x9E3779B97F4A7C15) & M64
        z = self.state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
        return z ^ (z >> 31)


def test_published_vector_seed_1234567():
    # The widely published SplitMix64 sequence for seed 1234567.
    expected = [6457827717110365317, 3203168211198807973, 9817491932198370423,
                4593380528125082431, 16408922859458223821]
    got = [O.lib().mro_splitmix_value(1234567, i) for i in range(5)]
    assert got == expected


@pytest.mark.parametrize("seed", [0, 42, 0xDEADBEEF, O.MASTER_SEED])
def test_value_equals_stream(seed):
    s = PySplitMix(seed)
    for i in range(64):
        assert O.lib().mro_splitmix_value(seed, i) == s.next()


def test_derive_separates_streams():
    L = O.lib()
    base = L.mro_splitmix_value(42, 0)
    assert L.mro_splitmix_derive(42, 0) != base
    assert L.mro_splitmix_derive(42, 0) != L.mro_splitmix_derive(42, 1)
    # derive(seed, label) = mix(seed ^ mix(label + 0xD1B54A32D192ED03))
    lab = 7
    inner = L.mro_splitmix_mix((lab + 0xD1B54A32D192ED03) & M64)
    assert L.mro_splitmix_derive(42, lab) == L.mro_splitmix_mix(42 ^ inner)


def test_label_is_fnv1a():
    h = 0xCBF29CE484222325
    for b in b"cache":
        h = ((h ^ b) * 0x100000001B3) & M64
    assert O.label("cache") == h


@pytest.mark.parametrize(
    "value,bits",
    [
        (1.0, 0x3F80),
        (-2.0, 0xC000),
        (1.0 + 2.0 ** -8, 0x3F80),      # exact tie -> even (down)
        (1.0 + 3 * 2.0 ** -8, 0x3F82),  # exact tie -> even (up)
        (1.0 + 2.0 ** -8 + 2.0 ** -20, 0x3F81),
        (-0.0, 0x8000),
        (float("inf"), 0x7F80),
        (3.4028234663852886e38, 0x7F80),  # FLT_MAX rounds up to inf
        (1e-40, 0x0001),  # subnormal keeps its top bits (9.18e-41 -> 0x0001 after RNE)
    ],
)
def test_bf16_rounding_kats(value, bits):
    got = O.lib().mro_f32_to_bf16(value)
    if value == 1e-40:
        # 1e-40 as float32 = 0x000116C2 -> RNE to 0x0001
        assert got == 0x0001
    else:
        assert got == bits
    assert O.f32_to_bf16(np.array([value], np.float32))[0] == got


def test_bf16_nan_stays_nan():
    got = O.lib().mro_f32_to_bf16(float("nan"))
    assert (got & 0x7F80) == 0x7F80 and (got & 0x7F) != 0


def test_normal_matches_python_box_muller():
    n = 64
    st = O.stream("probe")
    got = O.bf16_to_f32(O.normal_bf16("probe", (n,), mean=0.25, std=0.5))
    s = [O.lib().mro_splitmix_value(st, i) for i in range(n)]
    u = [(v >> 11) * (1.0 / 9007199254740992.0) for v in s]
    exp = []
    for j in range(n // 2):
        r = math.sqrt(-2.0 * math.log(1.0 - u[2 * j]))
        a = 2 * math.pi * u[2 * j + 1]
        exp += [0.25 + 0.5 * r * math.cos(a), 0.25 + 0.5 * r * math.sin(a)]
    exp_bf = O.bf16_to_f32(O.f32_to_bf16(np.array(exp, np.float32)))
    np.testing.assert_array_equal(got, exp_bf)


def test_normal_moments():
    x = O.bf16_to_f32(O.normal_bf16("moments", (1 << 20,), std=0.5)).astype(np.float64)
    assert abs(x.mean()) < 3e-3
    assert abs(x.std() - 0.5) < 3e-3
    # roughly Gaussian tails: P(|z|>2) ~ 4.55 %
    frac = np.mean(np.abs(x) > 1.0)
    assert 0.043 < frac < 0.048


def test_abs_normal_and_u32():
    a = O.bf16_to_f32(O.abs_normal_bf16("s", (4096,), std=0.01))
    assert (a >= 0).all() and 0.006 < a.mean() < 0.01
    w = O.u32("w", (1 << 16,))
    nib = (w[:, None] >> (4 * np.arange(8))) & 0xF
    counts = np.bincount(nib.ravel(), minlength=16)
    assert counts.min() > 0.9 * counts.mean()
    # the word is the top half of the stream value
    st = O.stream("w")
    assert int(w[3]) == O.lib().mro_splitmix_value(st, 3) >> 32


def test_sparse_indices_structure_and_fisher_yates():
    n_ctx, k, window = 4096, 256, 32
    idx = O.sparse_topk_indices("idx", n_ctx, k, window)
    assert idx.size == k and (np.diff(idx) > 0).all()
    assert set(range(n_ctx - window, n_ctx)) <= set(idx.tolist())
    assert idx.min() >= 0 and idx.max() < n_ctx
    # restated partial Fisher-Yates
    st = O.stream("idx")
    m = n_ctx - window
    pool = list(range(m))
    for i in range(k - window):
        j = i + O.lib().mro_splitmix_value(st, i) % (m - i)
        pool[i], pool[j] = pool[j], pool[i]
    exp = sorted(pool[: k - window] + list(range(m, n_ctx)))
    assert idx.tolist() == exp


def test_sparse_indices_full_config_shape():
    idx = O.sparse_topk_indices("sparse.idx.0", 131072, 2048, 128)
    assert idx.size == 2048 and (np.diff(idx) > 0).all()
    assert idx[-128:].tolist() == list(range(130944, 131072))
    assert idx[:1920].max() < 130944
