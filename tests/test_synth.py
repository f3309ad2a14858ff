"""The seeded input generators shared by bench.py and the tests
(oxforge.synth): deterministic, in range, with the moments their
distributions fix, and equal to a scalar restatement of SplitMix64 and
Box-Muller on a short stream."""
import math

import numpy as np

from oxforge import synth

MASK = (1 << 64) - 1


def splitmix_scalar(seed, n):
    out, state = [], seed
    for _ in range(n):
        state = (state + 0x9E3779B97F4A7C15) & MASK
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & MASK
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & MASK
        out.append(z ^ (z >> 31))
    return out


def test_splitmix_first_outputs_known_answer():
    # SplitMix64 seeded with 0: the published first outputs of the generator.
    d = splitmix_scalar(0, 3)
    assert d == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]
    assert [int(v) for v in synth._draws(0, 0, 3)] == d


def test_uniform_matches_scalar_restatement():
    d = splitmix_scalar(77, 257)
    ref = np.array([np.float32(-2.0 + 5.0 * ((v >> 40) / 16777216.0)) for v in d], np.float32)
    assert np.array_equal(synth.uniform((257,), 77, -2.0, 3.0), ref)


def test_normal_matches_scalar_restatement():
    d = splitmix_scalar(5, 64)
    ref = []
    for k in range(32):
        u1 = ((d[2 * k] >> 11) + 1.0) / 9007199254740993.0
        u2 = (d[2 * k + 1] >> 11) / 9007199254740992.0
        rad = math.sqrt(-2.0 * math.log(u1))
        ref += [rad * math.cos(2 * math.pi * u2), rad * math.sin(2 * math.pi * u2)]
    got = synth.normal((63,), 5).astype(np.float64)
    assert np.allclose(got, np.array(ref[:63]), rtol=1e-6, atol=1e-7)


def test_generators_deterministic_in_range_and_moments():
    a = synth.uniform((1000,), 5)
    assert np.array_equal(a, synth.uniform((1000,), 5))
    assert not np.array_equal(a, synth.uniform((1000,), 6))
    assert a.min() >= -1 and a.max() < 1 and abs(a.mean()) < 0.1
    n = synth.normal((20001,), 6, 1.0, 0.1)
    assert abs(n.mean() - 1.0) < 0.003 and abs(n.std() - 0.1) < 0.003
    w = synth.xavier(300, 500, 7)
    lim = math.sqrt(6.0 / 800)
    assert w.shape == (300, 500) and np.abs(w).max() <= lim


def test_chunked_draws_equal_one_pass():
    # Arrays longer than one chunk are generated piecewise; the pieces must
    # continue the same stream.
    big = synth.uniform((synth._CHUNK + 5,), 9)
    assert np.array_equal(big[-5:], synth.uniform((synth._CHUNK + 5,), 9)[-5:])
    d = synth._draws(9, synth._CHUNK, 5)
    assert np.array_equal(big[-5:], ((d >> np.uint64(40)).astype(np.float64) * 2.0 ** -24 * 2.0 - 1.0).astype(np.float32))
    nb = synth.normal((synth._CHUNK + 3,), 4)
    d = synth._draws(4, synth._CHUNK, 2)
    u1 = (float(d[0] >> np.uint64(11)) + 1.0) / 9007199254740993.0
    u2 = float(d[1] >> np.uint64(11)) / 9007199254740992.0
    assert np.isclose(nb[synth._CHUNK], math.sqrt(-2 * math.log(u1)) * math.cos(2 * math.pi * u2), rtol=1e-6)
