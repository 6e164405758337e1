"""Attention dropout (attention.py:68, :190): the counter-based keep mask that
include/msa.h defines, restated in the oracle, and pinned here on the CPU.

The reference draws its Bernoulli mask from torch's generator, so parity with
it is statistical only (keep rate 1-p, E[dropout(x)] = x); the kernels and the
oracle share the hash, so the GPU tests compare them exactly.
"""

import numpy as np
import pytest

import screening_oracle as O

# SplitMix64 (Steele, Lea and Flood, OOPSLA 2014) from state 0: its n-th output
# is the finaliser of n * 0x9E3779B97F4A7C15, i.e. keep bits of seed 0, key n.
SPLITMIX64_FROM_ZERO = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F,
                        0xF88BB8A8724C81EC, 0x1B39896A51A8749B]


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def test_hash_is_splitmix64():
    got = O.dropout_keep_bits(0, 0, 0, np.arange(1, 6))
    assert [int(x) for x in got] == [v >> 32 for v in SPLITMIX64_FROM_ZERO]


def test_hash_numpy_matches_integer_restatement():
    rng = np.random.default_rng(0)
    for _ in range(200):
        seed = int(rng.integers(0, 2 ** 63)) * 2 + int(rng.integers(0, 2))
        bh, i, j = int(rng.integers(0, 2 ** 16)), int(rng.integers(0, 2 ** 22)), int(rng.integers(0, 2 ** 22))
        assert int(O.dropout_keep_bits(seed, bh, i, j)) == O._keep_bits_int(seed, bh, i, j)


def test_key_fields_do_not_collide():
    # distinct (bh, i, j) give distinct keys: bh in bits 44.., i in 22..43, j in 0..21
    a = O._keep_bits_int(5, 1, 0, 0)
    b = O._keep_bits_int(5, 0, 1, 0)
    c = O._keep_bits_int(5, 0, 0, 1)
    assert len({a, b, c}) == 3


@pytest.mark.parametrize("p", [0.1, 0.3, 0.5, 0.9])
def test_keep_rate(p):
    f = O.dropout_factor((p, 1234), 2, 4, np.arange(300), np.arange(300))
    kept = float(np.mean(f > 0))
    n = f.size
    assert abs(kept - (1 - p)) < 5 * np.sqrt(p * (1 - p) / n)
    assert set(np.unique(f)) <= {0.0, O.dropout_scale(p)}


def test_threshold_and_scale_edges():
    assert O.dropout_factor((0.0, 7), 1, 1, np.arange(4), np.arange(4)) is None
    assert O.dropout_threshold(0.0) == 0
    assert O.dropout_threshold(np.nextafter(np.float32(1), np.float32(0))) == 4294967295 - 255
    assert O.dropout_scale(0.5) == 2.0


@pytest.mark.parametrize("causal", [True, False])
def test_forward_with_dropout_matches_brute_force(causal):
    B, T, H, D = 2, 9, 2, 5
    q, k, v = rnd((B, T, H, D), 1), rnd((B, T, H, D), 2), rnd((B, T, H, D), 3)
    q[..., 0] += 2.0
    k[..., 0] += 2.0
    r, w = np.array([1.2, 1.6]), np.array([4.5, 30.0])
    drop = (0.35, 987654321)
    got = O.forward(q, k, v, r, w, causal, dropout=drop)
    want = O.brute_force_forward(q, k, v, r, w, causal, dropout=drop)
    assert np.max(np.abs(got - want)) < 1e-12
    # the mask does something, and p = 0 is the identity
    assert np.max(np.abs(got - O.forward(q, k, v, r, w, causal))) > 1e-3
    assert np.array_equal(O.forward(q, k, v, r, w, causal, dropout=(0.0, 5)), O.forward(q, k, v, r, w, causal))


def test_backward_with_dropout_matches_finite_differences():
    B, T, H, D = 1, 7, 2, 6
    q, k, v = rnd((B, T, H, D), 20), rnd((B, T, H, D), 21), rnd((B, T, H, D), 22)
    q[..., 0] += 1.5
    k[..., 0] += 1.5
    dy = rnd((B, T, H, D), 23)
    r, w = np.array([1.15, 1.3]), np.array([3.7, 9.0])
    drop = (0.3, 42)
    dq, dk, dv, dr, dw = O.backward(q, k, v, r, w, dy, True, dropout=drop)
    L = lambda q_, k_, v_, r_, w_: float(np.sum(O.forward(q_, k_, v_, r_, w_, True, dropout=drop) * dy))

    def fd(f, x, idx, h=1e-6):
        xp, xm = x.copy(), x.copy()
        xp[idx] += h
        xm[idx] -= h
        return (f(xp) - f(xm)) / (2 * h)

    for idx in [(0, 3, 1, 2), (0, 6, 0, 0), (0, 5, 1, 4)]:
        assert abs(fd(lambda x: L(x, k, v, r, w), q, idx) - dq[idx]) < 1e-6 * (1 + abs(dq[idx]))
        assert abs(fd(lambda x: L(q, x, v, r, w), k, idx) - dk[idx]) < 1e-6 * (1 + abs(dk[idx]))
        assert abs(fd(lambda x: L(q, k, x, r, w), v, idx) - dv[idx]) < 1e-6 * (1 + abs(dv[idx]))
    for hh in range(H):
        assert abs(fd(lambda x: L(q, k, v, x, w), r, hh) - dr[hh]) < 1e-6 * (1 + abs(dr[hh]))
        assert abs(fd(lambda x: L(q, k, v, r, x), w, hh) - dw[hh]) < 1e-6 * (1 + abs(dw[hh]))


def test_dropout_is_unbiased():
    # E over seeds of the dropped aggregate h equals the undropped h (the
    # property nn.Dropout has); 400 seeds, tolerance 5 standard errors
    B, T, H, D = 1, 12, 1, 4
    q, k, v = rnd((B, T, H, D), 5), rnd((B, T, H, D), 6), rnd((B, T, H, D), 7)
    q[..., 0] += 3.0
    k[..., 0] += 3.0
    r, w = np.array([1.1]), np.array([20.0])
    _, h0 = O.forward(q, k, v, r, w, True, return_h=True)
    hs = np.stack([O.forward(q, k, v, r, w, True, return_h=True, dropout=(0.25, s))[1] for s in range(400)])
    se = hs.std(axis=0) / np.sqrt(len(hs)) + 1e-12
    assert np.all(np.abs(hs.mean(axis=0) - h0) < 5 * se + 1e-9)
