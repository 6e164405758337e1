"""Pins the CPU oracle (oracle/screening_oracle.py) before it is trusted.

Every oracle function is checked against something that does not restate
its own formula: closed-form known answers, a per-pair brute force, central
finite differences, and the golden vectors written from the reference module
(tests/golden/make_golden.py).
"""

import math

import numpy as np
import pytest
import torch

import screening_oracle as O
from helpers import GOLDEN_ATTENTION, golden_inputs, load_golden, rel_err


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


# ---------------------------------------------------------------------------
# forward
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("kpm", [False, True])
def test_forward_matches_brute_force(causal, kpm):
    B, Tq, Tk, H, D = 2, 9, 9 if causal else 13, 3, 8
    q, k, v = rnd((B, Tq, H, D), 1), rnd((B, Tk, H, D), 2), rnd((B, Tk, H, D), 3)
    q[:, :, :, :2] += 2.0
    k[:, :, :, :2] += 2.0        # correlated so that many pairs are live
    r = np.array([1.1, 1.4, 2.0])
    w = np.array([2.0, 4.5, 40.0])
    mask = None
    if kpm:
        mask = np.zeros((B, Tk), dtype=bool)
        mask[0, -3:] = True
        mask[1, 1] = True
    y = O.forward(q, k, v, r, w, causal, key_padding_mask=mask, block=4)
    yb = O.brute_force_forward(q, k, v, r, w, causal, key_padding_mask=mask)
    assert np.max(np.abs(y)) > 1e-2
    np.testing.assert_allclose(y, yb, rtol=0, atol=1e-13)


def test_one_hot_known_answer():
    # q = k = distinct one-hot rows -> s = I, so alpha = I (s=0 < 1-1/r off the
    # diagonal) and h_i = v^_i with |v^_i| = 1 -> y_i = tanh(1) v^_i.
    T, H, D = 6, 1, 8
    e = np.eye(D)[:T][None, :, None, :]
    v = rnd((1, T, H, D), 5)
    y = O.forward(e, e, v, np.array([1.5]), np.array([100.0]), True)
    vn = v / np.linalg.norm(v, axis=-1, keepdims=True)
    np.testing.assert_allclose(y, math.tanh(1.0) * vn, atol=1e-14)


def test_head0_init_window_known_answer():
    # w = exp(0)+1 = 2 (head 0 at init): weights {1, 1/2} at distance {0, 1}, 0 beyond.
    T, D = 7, 4
    q = np.ones((1, T, 1, D))
    v = rnd((1, T, 1, D), 6)
    y, h = O.forward(q, q, v, np.array([2.0]), np.array([2.0]), True, return_h=True)
    vn = v[0, :, 0] / np.linalg.norm(v[0, :, 0], axis=-1, keepdims=True)
    want = vn.copy()
    want[1:] += 0.5 * vn[:-1]
    np.testing.assert_allclose(h[0, 0], want, atol=1e-14)
    m = O.softmask(np.arange(3), np.arange(3), np.array([2.0]), True)[0]
    np.testing.assert_allclose(m, [[1, 0, 0], [0.5, 1, 0], [0, 0.5, 1]], atol=1e-15)


def test_below_threshold_is_exact_zero():
    # orthogonal q/k rows: s = 0 <= 1 - 1/r for every r > 1 -> y == 0 exactly
    T, D = 5, 8
    q = np.zeros((1, T, 1, D))
    k = np.zeros((1, T, 1, D))
    q[..., 0] = 1.0
    k[..., 1] = 1.0
    y = O.forward(q, k, rnd((1, T, 1, D), 7), np.array([1.01]), np.array([1e9]), True)
    assert np.all(y == 0.0)


def test_tanhnorm_properties():
    # mirrors the reference TanhNorm tests (tests/test_attention.py:9-31)
    h = rnd((1, 4, 1, 8), 8) * 100.0
    n = np.linalg.norm(h, axis=-1, keepdims=True)
    y = np.tanh(n) / n * h
    assert np.all(np.linalg.norm(y, axis=-1) <= 1.0 + 1e-12)
    np.testing.assert_allclose(y / np.linalg.norm(y, axis=-1, keepdims=True),
                               h / n, atol=1e-12)


def test_rows_forward_matches_full():
    B, T, H, D = 1, 300, 2, 16
    q, k, v = rnd((B, T, H, D), 9), rnd((B, T, H, D), 10), rnd((B, T, H, D), 11)
    r, w = np.array([1.1, 1.2]), np.array([17.0, 130.5])
    rows = [0, 1, 63, 64, 150, 299]
    y = O.forward(q, k, v, r, w, True)
    np.testing.assert_allclose(O.rows_forward(q, k, v, r, w, rows), y[:, rows], atol=1e-14)


def test_decode_row_is_last_forward_row():
    B, T, H, D = 2, 40, 2, 8
    q, k, v = rnd((B, T, H, D), 12), rnd((B, T, H, D), 13), rnd((B, T, H, D), 14)
    r, w = np.array([1.1, 1.3]), np.array([5.0, 33.0])
    y = O.forward(q, k, v, r, w, True)
    for L in (1, 7, 40):
        np.testing.assert_allclose(O.decode_row(q[:, L - 1], k, v, L, r, w), y[:, L - 1], atol=1e-14)


def test_tile_counts_brute_force():
    B, T, H, D = 1, 150, 2, 8
    q, k = rnd((B, T, H, D), 15), rnd((B, T, H, D), 16)
    r, w = np.array([1.1, 1.5]), np.array([40.0, 100.0])
    nW, nA, act = O.tile_counts(q, k, r, w, True, block=64)
    qn = q / np.linalg.norm(q, axis=-1, keepdims=True)
    kn = k / np.linalg.norm(k, axis=-1, keepdims=True)
    W = A = 0
    for h in range(H):
        for qt in range(3):
            for kt in range(3):
                win = live = False
                for i in range(qt * 64, min(T, qt * 64 + 64)):
                    for j in range(kt * 64, min(T, kt * 64 + 64)):
                        if 0 <= i - j < w[h]:
                            win = True
                            if 1 - r[h] * (1 - qn[0, i, h] @ kn[0, j, h]) > 0:
                                live = True
                W += win
                A += live
    assert (nW, nA) == (W, A)


# ---------------------------------------------------------------------------
# backward: central finite differences of L = sum(y * dy)
# ---------------------------------------------------------------------------
def _fd(f, x, idx, h=1e-6):
    xp, xm = x.copy(), x.copy()
    xp[idx] += h
    xm[idx] -= h
    return (f(xp) - f(xm)) / (2 * h)


@pytest.mark.parametrize("causal,kpm", [(True, False), (True, True), (False, False)])
def test_backward_matches_finite_differences(causal, kpm):
    B, Tq, Tk, H, D = 1, 7, 7 if causal else 10, 2, 6
    q, k, v = rnd((B, Tq, H, D), 20), rnd((B, Tk, H, D), 21), rnd((B, Tk, H, D), 22)
    q[..., 0] += 1.5
    k[..., 0] += 1.5
    dy = rnd((B, Tq, H, D), 23)
    r, w = np.array([1.15, 1.3]), np.array([3.7, 9.0])
    mask = None
    if kpm:
        mask = np.zeros((B, Tk), dtype=bool)
        mask[0, 2] = True
    dq, dk, dv, dr, dw = O.backward(q, k, v, r, w, dy, causal, key_padding_mask=mask)
    L = lambda q_, k_, v_, r_, w_: float(np.sum(O.forward(q_, k_, v_, r_, w_, causal,
                                                            key_padding_mask=mask) * dy))
    rng = np.random.default_rng(0)
    for name, x, g in (("q", q, dq), ("k", k, dk), ("v", v, dv)):
        for _ in range(6):
            idx = tuple(rng.integers(0, s) for s in x.shape)
            f = {"q": lambda t: L(t, k, v, r, w), "k": lambda t: L(q, t, v, r, w),
                 "v": lambda t: L(q, k, t, r, w)}[name]
            assert abs(_fd(f, x, idx) - g[idx]) < 1e-6 * max(1.0, abs(g[idx])), (name, idx)
    for hh in range(H):
        assert abs(_fd(lambda t: L(q, k, v, t, w), r, (hh,)) - dr[hh]) < 1e-6 * max(1, abs(dr[hh]))
        assert abs(_fd(lambda t: L(q, k, v, r, t), w, (hh,)) - dw[hh]) < 1e-6 * max(1, abs(dw[hh]))
    assert np.max(np.abs(dq)) > 1e-3 and abs(dr).max() > 1e-3 and abs(dw).max() > 1e-4


def test_backward_tanhnorm_small_norm_branch():
    # h tiny (|h| ~ 1e-4): the series branch of G must agree with finite differences
    B, T, H, D = 1, 4, 1, 4
    q = np.ones((B, T, H, D))
    v = rnd((B, T, H, D), 30)
    dy = rnd((B, T, H, D), 31)
    # every pair has the same s = c; r = 0.99/(1-c) puts a = 1 - r(1-c) at 0.01
    k = q.copy()
    k[..., 0] += 0.2
    c = float(q[0, 0, 0] @ k[0, 0, 0] / (np.linalg.norm(q[0, 0, 0]) * np.linalg.norm(k[0, 0, 0])))
    r, w = np.array([0.99 / (1.0 - c)]), np.array([3.0])
    dq, dk, dv, dr, dw = O.backward(q, k, v, r, w, dy, True)
    L = lambda v_: float(np.sum(O.forward(q, k, v_, r, w, True) * dy))
    _, h = O.forward(q, k, v, r, w, True, return_h=True)
    assert np.max(np.linalg.norm(h, axis=-1)) < 0.05
    for idx in [(0, 0, 0, 1), (0, 2, 0, 3), (0, 3, 0, 0)]:
        assert abs(_fd(L, v, idx) - dv[idx]) < 1e-7


def test_backward_below_threshold_is_zero():
    T, D = 5, 8
    q = np.zeros((1, T, 1, D))
    k = np.zeros((1, T, 1, D))
    q[..., 0] = 1.0
    k[..., 1] = 1.0
    dq, dk, dv, dr, dw = O.backward(q, k, rnd((1, T, 1, D), 7), np.array([1.5]), np.array([9.0]),
                                    rnd((1, T, 1, D), 8), True)
    for g in (dq, dk, dv, dr, dw):
        assert np.all(g == 0.0)


# ---------------------------------------------------------------------------
# golden vectors from the reference module
# ---------------------------------------------------------------------------
def _weights_from_seed(z):
    torch.manual_seed(int(z["seed"]))
    d = int(z["d_model"])
    lins = [torch.nn.Linear(d, d, bias=False) for _ in range(4)]   # q, k, v, out order
    return [l.weight.detach().double().numpy() for l in lins]


@pytest.mark.parametrize("name", GOLDEN_ATTENTION)
def test_oracle_matches_reference_golden(name):
    z = load_golden(name)
    Wq, Wk, Wv, Wo = _weights_from_seed(z)
    for nm, W in zip("qkvo", (Wq, Wk, Wv, Wo)):
        assert abs(W.sum() - float(z[f"W{nm}_sum"])) < 1e-9 * max(1.0, abs(W).sum())
        np.testing.assert_array_equal(W[:2].astype(np.float32), z[f"W{nm}_head"])
    x, mem, dy, kpm = golden_inputs(z)
    x, mem, dy = (t.double().numpy() for t in (x, mem, dy))
    assert abs(x.sum() - float(z["x_sum"])) < 1e-9 * abs(x).sum()
    H, d = int(z["H"]), int(z["d_model"])
    D = d // H
    B, Tq, Tk = x.shape[0], x.shape[1], mem.shape[1]
    causal = bool(int(z["causal"]))
    r = np.exp(z["s_r"].astype(np.float64)) + 1.0
    w = np.exp(z["s_v"].astype(np.float64)) + 1.0
    kpm_np = None if kpm is None else kpm.numpy()
    q = (x @ Wq.T).reshape(B, Tq, H, D)
    k = (mem @ Wk.T).reshape(B, Tk, H, D)
    v = (mem @ Wv.T).reshape(B, Tk, H, D)
    core = O.forward(q, k, v, r, w, causal, key_padding_mask=kpm_np)
    y = core.reshape(B, Tq, d) @ Wo.T
    assert rel_err(y, z["y"]) < 2e-5 if np.max(np.abs(z["y"])) > 0 else np.all(y == 0)
    dcore = (dy @ Wo).reshape(B, Tq, H, D)
    dq, dk, dv, dr, dw = O.backward(q, k, v, r, w, dcore, causal, key_padding_mask=kpm_np)
    dx = dq.reshape(B, Tq, d) @ Wq
    dmem = dk.reshape(B, Tk, d) @ Wk + dv.reshape(B, Tk, d) @ Wv
    if int(z["same_qkv"]):
        dx = dx + dmem
    else:
        assert rel_err(dmem, z["dmem"]) < 2e-5
    assert rel_err(dx, z["dx"]) < 2e-5
    # s_r, s_v enter through r = exp(s_r)+1, w = exp(s_v)+1
    np.testing.assert_allclose(dr * (r - 1.0), z["ds_r"], rtol=2e-4, atol=1e-7 * max(1, abs(z["ds_r"]).max()))
    np.testing.assert_allclose(dw * (w - 1.0), z["ds_v"], rtol=2e-4, atol=1e-7 * max(1, abs(z["ds_v"]).max()))


# ---------------------------------------------------------------------------
# live-pair form (full-size checks): pinned against the dense functions above
# ---------------------------------------------------------------------------
def _dense_live_set(q, k, r, w, causal, kpm=None):
    qn = q / np.linalg.norm(q, axis=-1, keepdims=True)
    kn = k / np.linalg.norm(k, axis=-1, keepdims=True)
    B, Tq, H, _ = q.shape
    Tk = k.shape[1]
    out = set()
    for b in range(B):
        for h in range(H):
            s = qn[b, :, h] @ kn[b, :, h].T
            for i in range(Tq):
                for j in range(Tk):
                    d = i - j
                    inside = (0 <= d < w[h]) if causal else (abs(d) < w[h])
                    if inside and not (kpm is not None and kpm[b, j]) and 1 - r[h] * (1 - s[i, j]) > 0:
                        out.add((b, h, i, j))
    return out


@pytest.mark.parametrize("causal,Tq,Tk,kpm", [(True, 70, 70, False), (True, 90, 50, True),
                                               (True, 40, 95, False), (False, 60, 110, True)])
def test_live_pairs_equal_dense_set(causal, Tq, Tk, kpm):
    B, H, D = 2, 3, 16
    q, k = rnd((B, Tq, H, D), 40), rnd((B, Tk, H, D), 41)
    q[..., 0] += 1.0
    k[..., 0] += 1.0
    r, w = np.array([1.1, 1.5, 2.0]), np.array([3.5, 20.0, 1e6])
    mask = None
    if kpm:
        mask = np.zeros((B, Tk), dtype=bool)
        mask[0, ::7] = True
        mask[1, -4:] = True
    P = O.live_pairs(q, k, r, w, causal, key_padding_mask=mask, block=32)
    got = set(zip(P["b"].tolist(), P["h"].tolist(), P["i"].tolist(), P["j"].tolist()))
    want = _dense_live_set(q, k, r, w, causal, mask)
    assert len(want) > 100 and got == want
    assert len(got) == len(P["i"])          # no pair listed twice


def test_live_pairs_keep_pairs_just_above_threshold():
    # s a few float32 ulps above 1 - 1/r: the float32 candidate pass must not
    # drop it (SCREEN_MARGIN); s just below must not be listed
    r = 1.7
    thr = 1.0 - 1.0 / r
    D = 64
    q = np.zeros((1, 3, 1, D))
    q[..., 0] = 1.0
    k = np.zeros((1, 3, 1, D))
    for j, c in enumerate((thr + 3e-8, thr - 3e-8, thr + 1e-3)):
        k[0, j, 0, 0] = c
        k[0, j, 0, 1] = math.sqrt(1.0 - c * c)
    P = O.live_pairs(q, k, np.array([r]), np.array([1e9]), True)
    assert sorted(zip(P["i"].tolist(), P["j"].tolist())) == [(0, 0), (1, 0), (2, 0), (2, 2)]


def test_live_pairs_screen_margin_bound():
    # the float32 candidate pass is within a tenth of SCREEN_MARGIN of float64
    for D, seed in ((64, 42), (128, 43), (16, 44)):
        x = rnd((400, D), seed)
        y = rnd((400, D), seed + 100)
        x[:, 0] += 2.0
        y[:, 0] += 2.0
        xn = x / np.linalg.norm(x, axis=-1, keepdims=True)
        yn = y / np.linalg.norm(y, axis=-1, keepdims=True)
        s32 = xn.astype(np.float32) @ yn.astype(np.float32).T
        assert np.max(np.abs(s32.astype(np.float64) - xn @ yn.T)) < 0.1 * O.SCREEN_MARGIN


@pytest.mark.parametrize("causal,Tq,Tk,kpm,drop", [
    (True, 96, 96, False, None), (True, 130, 70, True, None), (True, 50, 120, False, (0.3, 99)),
    (False, 80, 140, True, None), (False, 64, 64, False, (0.5, 7))])
def test_sparse_forward_backward_matches_dense(causal, Tq, Tk, kpm, drop):
    B, H, D = 2, 3, 32
    q, k, v = rnd((B, Tq, H, D), 50), rnd((B, Tk, H, D), 51), rnd((B, Tk, H, D), 52)
    q[..., :2] += 0.8
    k[..., :2] += 0.8
    dy = rnd((B, Tq, H, D), 53)
    r, w = np.array([1.1, 1.3, 1.9]), np.array([7.5, 40.0, 1e5])
    mask = None
    if kpm:
        mask = np.zeros((B, Tk), dtype=bool)
        mask[0, 5:9] = True
        mask[1, -1] = True
    y, grads, P = O.sparse_forward_backward(q, k, v, r, w, dy, causal, key_padding_mask=mask, dropout=drop)
    assert len(P["i"]) > 200
    yd = O.forward(q, k, v, r, w, causal, key_padding_mask=mask, dropout=drop)
    gd = O.backward(q, k, v, r, w, dy, causal, key_padding_mask=mask, dropout=drop)
    assert np.max(np.abs(yd)) > 1e-2
    np.testing.assert_allclose(y, yd, rtol=0, atol=1e-12)
    for name, a, b in zip(("dq", "dk", "dv", "dr", "dw"), grads, gd):
        assert np.max(np.abs(b)) > 1e-4, name
        np.testing.assert_allclose(a, b, rtol=0, atol=1e-11 * max(1.0, np.max(np.abs(b)))), name
