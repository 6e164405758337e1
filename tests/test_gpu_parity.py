"""Parity of the HIP path (libmsa.so, through its C ABI) with the CPU oracle.

Tolerances: <= 1e-5 in fp32 and <= 2e-2 in bf16, for
outputs and all gradients, on each of max|got-ref|/max|ref| per tensor, the
Frobenius ratio ||got-ref||/||ref|| and the per-(b, h) max-relative error
(helpers.rel_err); float16 is held to 5e-3.  The bf16 and fp16 oracle is the
float64 oracle on the same rounded inputs.
"""

import math

import numpy as np
import pytest
import torch

import screening_oracle as O
from helpers import (GOLDEN_ATTENTION, correlated_qkv, golden_inputs, golden_module, load_golden,
                     head_sum_err, np64, qkv, rel_err, rw64)

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 5e-3}
DEV = "cuda"


def _ops():
    from multiscreen import ops
    return ops


def _rw(H, r, w):
    return (torch.tensor(r, dtype=torch.float32, device=DEV),
            torch.tensor(w, dtype=torch.float32, device=DEV))


def _run_fwd(q, k, v, r, w, causal=True, kpm=None):
    ops = _ops()
    rg, wg = _rw(q.shape[2], r, w)
    out = ops.fwd_raw(q.to(DEV), k.to(DEV), v.to(DEV), rg, wg, causal, 1e-8,
                      None if kpm is None else kpm.to(DEV))
    torch.cuda.synchronize()
    return out


def test_mfma_layout_selftest():
    from multiscreen import _native
    L = _native.lib()
    g = torch.Generator().manual_seed(0)
    a16 = torch.randn(32, 16, generator=g).bfloat16().float()
    b16 = torch.randn(16, 32, generator=g).bfloat16().float()
    a2 = torch.randn(32, 2, generator=g)
    b2 = torch.randn(2, 32, generator=g)
    ta, tb, t2a, t2b = (x.to(DEV).contiguous() for x in (a16, b16, a2, b2))
    o16 = torch.zeros(32, 32, device=DEV)
    o2 = torch.zeros(32, 32, device=DEV)
    rc = L.msa_selftest_mfma(ta.data_ptr(), tb.data_ptr(), o16.data_ptr(), t2a.data_ptr(),
                             t2b.data_ptr(), o2.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    np.testing.assert_allclose(o16.cpu().double().numpy(), (a16.double() @ b16.double()).numpy(),
                               rtol=1e-6, atol=1e-5)
    np.testing.assert_allclose(o2.cpu().double().numpy(), (a2.double() @ b2.double()).numpy(),
                               rtol=1e-6, atol=1e-5)


FWD_CASES = [
    # B, Tq, Tk, H, D, causal, r, w, kpm
    (2, 128, 128, 8, 64, True, [1.1] * 8, [16, 32, 64, 96, 128, 160, 200, 256], False),
    (1, 200, 200, 2, 64, True, [1.15, 1.3], [37.5, 1e6], False),          # ragged T
    (2, 130, 130, 4, 16, True, [1.1, 1.2, 1.3, 2.0], [2.0, 5.3, 70.0, 300.0], True),
    (1, 70, 150, 2, 32, False, [1.1, 1.25], [20.0, 400.0], True),          # cross, Tq != Tk
    (1, 96, 96, 2, 128, True, [1.1, 1.2], [50.0, 96.0], False),
    (1, 257, 257, 3, 64, False, [1.12, 1.2, 1.5], [64.5, 129.0, 1e4], False),
    # head_dim 32: the instantiation where an unguarded MFMA source-register
    # hazard once corrupted dq/dk (see the guard in msa_device.h)
    (1, 128, 128, 2, 32, True, [1.1, 1.25], [20.0, 400.0], False),
    # causal with Tq != Tk: both index ranges start at 0 (attention.py:108-118,
    # :171-173), so queries past Tk see the last keys and keys past Tq are seen
    # by no query
    (1, 100, 160, 2, 64, True, [1.1, 1.3], [30.0, 500.0], False),          # Tq < Tk
    (2, 190, 90, 2, 64, True, [1.15, 1.25], [60.0, 1e4], True),            # Tq > Tk, key padding
    (1, 64, 300, 3, 32, True, [1.1, 1.2, 1.4], [2.0, 100.0, 1e6], False),   # one query tile, five key tiles
]


def _case_inputs(case, dtype, seed=0):
    B, Tq, Tk, H, D, causal, r, w, use_kpm = case
    q, k, v = correlated_qkv(B, Tq, Tk, H, D, seed=seed, dtype=dtype, rho=0.35)
    kpm = None
    if use_kpm:
        kpm = torch.zeros(B, Tk, dtype=torch.bool)
        kpm[0, -5:] = True
        kpm[-1, 3] = True
    return q, k, v, kpm


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("case", FWD_CASES, ids=[f"c{i}" for i in range(len(FWD_CASES))])
def test_forward_parity(case, dtype):
    B, Tq, Tk, H, D, causal, r, w, use_kpm = case
    q, k, v, kpm = _case_inputs(case, dtype)
    y, hnorm, bits = _run_fwd(q, k, v, r, w, causal, kpm)
    kpm_np = None if kpm is None else kpm.numpy()
    yref, href = O.forward(np64(q), np64(k), np64(v), rw64(r), rw64(w), causal,
                           key_padding_mask=kpm_np, return_h=True)
    assert np.max(np.abs(yref)) > 1e-3, "vacuous case"
    assert rel_err(np64(y), yref) <= TOL[dtype]
    nref = np.linalg.norm(href, axis=-1)
    assert rel_err(hnorm.cpu().double().numpy(), nref, heads=(0, 1)) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("case", FWD_CASES, ids=[f"c{i}" for i in range(len(FWD_CASES))])
def test_backward_parity(case, dtype):
    B, Tq, Tk, H, D, causal, r, w, use_kpm = case
    q, k, v, kpm = _case_inputs(case, dtype, seed=1)
    g = torch.Generator().manual_seed(7)
    dy = torch.randn(B, Tq, H, D, generator=g).to(dtype)
    ops = _ops()
    rg, wg = _rw(H, r, w)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kpm_d = None if kpm is None else kpm.to(DEV)
    y, hnorm, bits = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, kpm_d)
    dq, dk, dv, dr, dw = ops.bwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, y, hnorm, bits, dy.to(DEV), kpm_d)
    torch.cuda.synchronize()
    kpm_np = None if kpm is None else kpm.numpy()
    # the backward differentiates the kernel's own forward output y, so the
    # oracle is fed the same dy
    ref = O.backward(np64(q), np64(k), np64(v), rw64(r), rw64(w), np64(dy), causal,
                     key_padding_mask=kpm_np)
    tol = TOL[dtype]
    for name, got, want in zip(("dq", "dk", "dv", "dr", "dw"), (dq, dk, dv, dr, dw), ref):
        assert np.max(np.abs(want)) > 0, f"{name} vacuous"
        e = rel_err(np64(got), want)
        assert e <= tol, f"{name}: rel err {e:.3e} > {tol}"
    _check_head_sums(q, k, v, r, w, dy, causal, kpm_np, None, dr, dw, ref, tol)


def _check_head_sums(q, k, v, r, w, dy, causal, kpm_np, drop, dr, dw, ref, tol):
    """dr and dw entry by entry: each head's error against the sum of its
    terms' magnitudes (the live-pair oracle's dr_abs, dw_abs), so a head with
    few or small terms is not hidden behind the largest one."""
    _, _, P = O.sparse_forward_backward(np64(q), np64(k), np64(v), rw64(r), rw64(w), np64(dy), causal,
                                        key_padding_mask=kpm_np, dropout=drop)
    for name, got, want, scale in (("dr", dr, ref[3], P["dr_abs"]), ("dw", dw, ref[4], P["dw_abs"])):
        e = head_sum_err(np64(got), want, scale)
        assert e <= tol, f"{name}: per-head error {e:.3e} > {tol}"


# Attention dropout (attention.py:190): the kernels and the oracle share the
# counter-based keep mask of include/msa.h, so they agree to the usual
# tolerances; cases 1-3 cover ragged T, key padding and Tq != Tk.
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("ci", [0, 1, 2, 3])
def test_dropout_parity(ci, dtype):
    case = FWD_CASES[ci]
    B, Tq, Tk, H, D, causal, r, w, use_kpm = case
    q, k, v, kpm = _case_inputs(case, dtype, seed=4)
    dy = torch.randn(B, Tq, H, D, generator=torch.Generator().manual_seed(9)).to(dtype)
    drop = (0.3, 0x5EED0000ABCD1234 + ci)
    ops = _ops()
    rg, wg = _rw(H, r, w)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    kpm_d = None if kpm is None else kpm.to(DEV)
    y, hnorm, bits = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, kpm_d, *drop)
    grads = ops.bwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, y, hnorm, bits, dy.to(DEV), kpm_d, *drop)
    torch.cuda.synchronize()
    kpm_np = None if kpm is None else kpm.numpy()
    args = (np64(q), np64(k), np64(v), rw64(r), rw64(w))
    yref = O.forward(*args, causal, key_padding_mask=kpm_np, dropout=drop)
    ref = O.backward(*args, np64(dy), causal, key_padding_mask=kpm_np, dropout=drop)
    tol = TOL[dtype]
    assert rel_err(np64(y), yref) <= tol
    # the mask is not the identity on this case
    y0 = O.forward(*args, causal, key_padding_mask=kpm_np)
    assert np.max(np.abs(yref - y0)) > 1e-3 * np.max(np.abs(y0))
    for name, got, want in zip(("dq", "dk", "dv", "dr", "dw"), grads, ref):
        assert np.max(np.abs(want)) > 0, f"{name} vacuous"
        e = rel_err(np64(got), want)
        assert e <= tol, f"{name}: rel err {e:.3e} > {tol}"
    _check_head_sums(q, k, v, r, w, dy, causal, kpm_np, drop, grads[3], grads[4], ref, tol)


def test_dropout_zero_is_identity_and_seed_reproduces():
    case = FWD_CASES[1]
    B, Tq, Tk, H, D, causal, r, w, _ = case
    q, k, v, _ = _case_inputs(case, torch.bfloat16, seed=5)
    ops = _ops()
    rg, wg = _rw(H, r, w)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    base = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, None)[0]
    assert torch.equal(ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, None, 0.0, 12345)[0], base)
    a = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, None, 0.5, 777)[0]
    b = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, None, 0.5, 777)[0]
    c = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, None, 0.5, 778)[0]
    assert torch.equal(a, b) and not torch.equal(a, c)


def test_module_dropout_in_training_mode():
    from multiscreen.attention import ScreeningAttention
    torch.manual_seed(0)
    m = ScreeningAttention(128, 2, dropout=0.25).to(DEV)
    with torch.no_grad():
        m.s_r.fill_(math.log(0.05))  # r = 1.05: most in-window pairs pass the threshold
    x = torch.randn(2, 96, 128, device=DEV)
    m.train()
    torch.manual_seed(11)
    y1 = m(x, x, x)
    torch.manual_seed(11)
    y2 = m(x, x, x)
    y3 = m(x, x, x)
    assert y1.abs().max() > 1e-3
    assert torch.equal(y1, y2) and not torch.equal(y1, y3)
    y1.sum().backward()
    assert m.s_r.grad is not None and torch.isfinite(m.q_proj.weight.grad).all()
    m.eval()
    assert torch.equal(m(x, x, x), m(x, x, x))


def test_backward_deterministic():
    case = FWD_CASES[0]
    q, k, v, kpm = _case_inputs(case, torch.bfloat16, seed=2)
    B, Tq, Tk, H, D, causal, r, w, _ = case
    dy = torch.randn(B, Tq, H, D, generator=torch.Generator().manual_seed(3)).bfloat16().to(DEV)
    ops = _ops()
    rg, wg = _rw(H, r, w)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    outs = []
    for _ in range(2):
        y, hnorm, bits = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, None)
        outs.append((y,) + ops.bwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, y, hnorm, bits, dy))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)


# Screen work distribution: B*H = 4 uses one work queue; 8 uses eight queues
# with heads ranked by window; 72 uses eight queues without ranking; T = 2048
# with wide windows cuts each query group's key range into several parts.
@pytest.mark.parametrize("B,T,H,r,w", [
    (1, 640, 4, [1.1, 1.3, 1.6, 2.0], [100.0, 250.5, 640.0, 1e5]),
    (2, 640, 4, [1.1, 1.3, 1.6, 2.0], [100.0, 250.5, 640.0, 1e5]),
    (9, 192, 8, [1.2] * 8, [30.0, 60.0, 90.0, 120.0, 150.0, 180.0, 1e4, 2.0]),
    (1, 2048, 8, [1.1, 1.2, 1.3, 1.4, 1.5, 1.6, 1.8, 2.0], [1e5, 3000.0, 1700.0, 900.0, 2048.0, 64.0, 1e5, 500.0]),
], ids=["bh4", "bh8", "bh72", "t2048"])
def test_tile_bitmap_matches_oracle_counts(B, T, H, r, w):
    # fp32: the bitmap holds every unit with a live pair, and beyond those only
    # units with a pair within BAND_F32 below the threshold (the vote's slack
    # plus the same bound again for the rounding of the values it votes on)
    D = 64
    q, k, v = correlated_qkv(B, T, T, H, D, seed=4, dtype=torch.float32, rho=0.3)
    y, hnorm, bits = _run_fwd(q, k, v, r, w, True)
    # the bitmap is kept per 32x32 unit: 2*nqt rows of ceil(2*nkt/32) words
    rr = rw64(r)
    nW, nA, act = O.tile_counts(np64(q), np64(k), rr, rw64(w), True, tile=32)
    _, _, band = O.tile_counts(np64(q), np64(k), 1.0 / (1.0 / rr + BAND_F32), rw64(w), True, tile=32)
    _, nA64, act64 = O.tile_counts(np64(q), np64(k), rr, rw64(w), True, tile=64)
    nqu = nku = T // 32
    words = (nku + 31) // 32
    b = bits.cpu().numpy().view(np.uint32).reshape(B, H, nqu, words)
    got = np.zeros((B, H, nqu, nku), dtype=bool)
    for ku in range(nku):
        got[..., ku] = (b[..., ku // 32] >> (ku % 32)) & 1
    assert nA > 0
    assert np.all(got[act]), "a unit with a live pair is not marked"
    assert not np.any(got & ~band), "a marked unit has no pair within the slack"
    # a 64x64 tile is marked iff one of its four units is
    got64 = got.reshape(B, H, nqu // 2, 2, nku // 2, 2).any(axis=(3, 5))
    assert np.all(got64[act64])


# The vote's slack below the threshold 1 - 1/r, in s (kScreenSlack in
# msa_fwd.hip): every type screens on fp16 K^ (unit roundoff 2^-11: 11
# significant bits); fp32 query rows are rounded to fp16 as well (another
# 2^-11), 2-byte ones are exact in fp16; plus fp32 accumulation.
SLACK_F32 = 2.0 ** -10 + 1e-5
BAND_F32 = 2.0 * SLACK_F32
SLACK_16 = 2.0 ** -11 + 1e-5


def _fp16_screen_units(q, k, r, w, causal):
    """The 2-byte screen's vote restated in float64 on its own operands:
    K^ = fp16(1024 k/|k|) as prep_k stores it, each raw query row scaled by
    the power of two c that puts its largest component in [2^10, 2^11) and
    rounded to fp16, s_screen = (q16 . K^) / (1024 c max(|q|, eps)).  Returns
    the units whose best in-window s_screen exceeds 1 - 1/r - SLACK_16, the
    distance of that best value from the vote threshold, and the units with
    an exact live pair (s from the rounded inputs in float64)."""
    q64, k64 = np64(q), np64(k)
    qnorm = np.maximum(np.linalg.norm(q64, axis=-1, keepdims=True), 1e-8)
    mx = np.max(np.abs(q64), axis=-1, keepdims=True)
    ex = np.frexp(np.where(mx > 0, mx, 1.0))[1]
    c = np.where(mx > 0, np.ldexp(1.0, 11 - ex), 1.0)
    q16 = (q64 * c).astype(np.float16).astype(np.float64)
    kf = k.float()
    kh = (1024.0 * kf / kf.norm(dim=-1, keepdim=True).clamp_min(1e-8)).half().double().numpy()
    qn = q64 / qnorm
    kn = k64 / np.maximum(np.linalg.norm(k64, axis=-1, keepdims=True), 1e-8)
    B, T, H, _ = q64.shape
    n = T // 32
    vote = np.zeros((B, H, n, n), dtype=bool)
    exact = np.zeros((B, H, n, n), dtype=bool)
    margin = np.full((B, H, n, n), np.inf)
    i = np.arange(T)[:, None]
    j = np.arange(T)[None, :]
    for h in range(H):
        s_scr = np.einsum("bid,bjd->bij", q16[:, :, h], kh[:, :, h]) / (1024.0 * c[:, :, h] * qnorm[:, :, h])
        s_ex = np.einsum("bid,bjd->bij", qn[:, :, h], kn[:, :, h])
        wc = math.ceil(w[h])
        inside = ((i - j >= 0) & (i - j < wc)) if causal else (np.abs(i - j) < wc)
        thr = 1.0 - 1.0 / r[h]
        d = np.where(inside[None], s_scr - (thr - SLACK_16), -np.inf).reshape(B, n, 32, n, 32)
        best = d.max(axis=(2, 4))
        vote[:, h] = best > 0
        margin[:, h] = np.abs(best)
        e = np.where(inside[None], s_ex - thr, -np.inf).reshape(B, n, 32, n, 32)
        exact[:, h] = e.max(axis=(2, 4)) > 0
    return vote, margin, exact


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "f16"])
@pytest.mark.parametrize("r", [1.9, 2.0, 2.1, 1.5])
def test_2byte_bitmap_matches_exact_test(r, dtype):
    # the 2-byte screen's bitmap is its vote on its own operands (fp16 K^,
    # scaled fp16 q), restated in float64, units within 1e-5 of the vote's
    # threshold excepted (fp32 accumulation); and it holds every unit with
    # an exactly live pair (no pair with alpha > 0 is ever missed)
    B, T, H, D = 2, 1024, 4, 64
    q, k, v = qkv(B, T, T, H, D, seed=11, dtype=dtype)
    rr, ww = [r] * H, [100.0, 400.0, 700.0, 1e5]
    y, hnorm, bits = _run_fwd(q, k, v, rr, ww, True)
    want, margin, exact = _fp16_screen_units(q, k, rr, ww, True)
    n = T // 32
    words = (n + 31) // 32
    b = bits.cpu().numpy().view(np.uint32).reshape(B, H, n, words)
    got = np.zeros((B, H, n, n), dtype=bool)
    for ku in range(n):
        got[..., ku] = (b[..., ku // 32] >> (ku % 32)) & 1
    assert exact.sum() > 0
    assert np.all(got[exact]), int((exact & ~got).sum())
    diff = got != want
    assert np.all(margin[diff] < 1e-5), (int(diff.sum()), float(margin[diff].min()) if diff.any() else 0.0)


def test_window_and_threshold_skip_are_exact():
    # keys outside every query's window, or below threshold, must not change y at all
    B, T, H, D = 1, 512, 2, 64
    q, k, v = correlated_qkv(B, T, T, H, D, seed=5, dtype=torch.bfloat16, rho=0.3)
    r, w = [1.1, 1.2], [40.0, 100.0]
    y0 = _run_fwd(q, k, v, r, w, True)[0]
    # perturb the values of keys no query of tile 7 can see, then compare rows of tile 7
    v2 = v.clone()
    v2[:, :7 * 64 - 101] = torch.randn_like(v2[:, :7 * 64 - 101].float()).bfloat16()
    y1 = _run_fwd(q, k, v2, r, w, True)[0]
    assert torch.equal(y0[:, 7 * 64:8 * 64], y1[:, 7 * 64:8 * 64])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
def test_decode_matches_forward_rows(dtype):
    B, T, H, D = 3, 700, 4, 64
    q, k, v = correlated_qkv(B, T, T, H, D, seed=6, dtype=dtype, rho=0.35)
    r, w = [1.1, 1.2, 1.4, 2.0], [3.0, 77.7, 300.0, 1e6]
    ops = _ops()
    rg, wg = _rw(H, r, w)
    kc, vc = k.to(DEV), v.to(DEV)
    yfull = O.forward(np64(q), np64(k), np64(v), rw64(r), rw64(w), True)
    for L in (1, 2, 64, 257, 700):
        y = ops.decode_step(q[:, L - 1].to(DEV), kc, vc, L, rg, wg)
        torch.cuda.synchronize()
        assert rel_err(np64(y), yfull[:, L - 1], heads=(0, 1)) <= TOL[dtype], L


def test_decode_window_hint_changes_only_the_grid():
    # the hint sizes the launch; too small, exact, too large or absent, the
    # output is bitwise the same and matches the oracle.  H = 72 takes the
    # head scan over more than one wave of lanes.
    B, T, H, D = 2, 5000, 72, 16
    q, k, v = correlated_qkv(B, T, T, H, D, seed=13, dtype=torch.bfloat16, rho=0.35)
    g = torch.Generator().manual_seed(3)
    r = (1.1 + 0.3 * torch.rand(H, generator=g)).tolist()
    w = (2.0 + 6000.0 * torch.rand(H, generator=g) ** 3).tolist()
    ops = _ops()
    rg, wg = _rw(H, r, w)
    kc, vc = k.to(DEV), v.to(DEV)
    for L in (1, 2049, 5000):
        qd = q[:, L - 1].to(DEV)
        base = ops.decode_step(qd, kc, vc, L, rg, wg)
        for hint in (1, 2048, math.ceil(max(w)), 10 ** 6):
            assert torch.equal(ops.decode_step(qd, kc, vc, L, rg, wg, window_hint=hint), base), (L, hint)
        ref = O.decode_row(np64(q[:, L - 1]), np64(k), np64(v), L, rw64(r), rw64(w))
        assert rel_err(np64(base), ref, heads=(0, 1)) <= 2e-2, L


@pytest.mark.parametrize("name", GOLDEN_ATTENTION)
def test_module_matches_reference_golden_fp32(name):
    from multiscreen import ScreeningAttention
    z = load_golden(name)
    m = golden_module(z, ScreeningAttention).to(DEV)
    x, mem, dy, kpm = golden_inputs(z)
    x = x.to(DEV).requires_grad_(True)
    same = bool(int(z["same_qkv"]))
    memd = x if same else mem.to(DEV).requires_grad_(True)
    y = m(x, memd, memd, key_padding_mask=None if kpm is None else kpm.to(DEV))
    (y * dy.to(DEV)).sum().backward()
    torch.cuda.synchronize()
    yref = z["y"]
    if np.max(np.abs(yref)) == 0:
        assert torch.count_nonzero(y) == 0
    else:
        assert rel_err(np64(y), yref) <= 1e-5
        assert rel_err(np64(x.grad), z["dx"]) <= 1e-5
        assert rel_err(np64(m.s_r.grad), z["ds_r"]) <= 1e-5
        assert rel_err(np64(m.s_v.grad), z["ds_v"]) <= 1e-5
        assert rel_err(np64(m.q_proj.weight.grad[:8]), z["dWq_rows"]) <= 1e-5
        assert rel_err(np64(m.out_proj.weight.grad[:8]), z["dWo_rows"]) <= 1e-5
        if not same:
            assert rel_err(np64(memd.grad), z["dmem"]) <= 1e-5


def test_cfg2_full_size_sampled_rows_bf16():
    # BASELINE configs[1] shape: B=4, T=8192, H=8, D=64, bf16, r~U[1.9,2.1], w~U[256,8192]
    B, T, H, D = 4, 8192, 8, 64
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(B, T, H, D, generator=g).bfloat16() for _ in range(3))
    r = (1.9 + 0.2 * torch.rand(H, generator=g)).tolist()
    w = (256 + (8192 - 256) * torch.rand(H, generator=g)).tolist()
    # sharpen some heads so the sampled rows carry live pairs
    r[0], r[1] = 1.15, 1.3
    y = _run_fwd(q, k, v, r, w, True)[0]
    rows = [0, 1, 63, 64, 1000, 4095, 4096, 8191]
    yref = O.rows_forward(np64(q), np64(k), np64(v), rw64(r), rw64(w), rows, True)
    assert np.max(np.abs(yref)) > 1e-3
    assert rel_err(np64(y[:, rows]), yref) <= 2e-2


def test_float16_model_generate():
    # a float16 model (model.half()) decodes through float16 caches; its greedy
    # tokens are those of re-running forward() on the prefix
    from multiscreen import MultiscreenLM
    torch.manual_seed(0)
    lm = MultiscreenLM(vocab_size=50, d_model=64, num_heads=4, num_layers=2, max_seq_len=64)
    for blk in lm.blocks:
        with torch.no_grad():
            blk.attn.s_r.fill_(math.log(0.15))
            blk.attn.s_v.copy_(torch.log(torch.tensor([2.0, 7.0, 20.0, 60.0])))
    lm = lm.half().to(DEV)
    prompt = torch.randint(0, 50, (2, 5), device=DEV)
    got = lm.generate(prompt, max_new_tokens=6, top_k=1)
    assert got.shape == (2, 11)
    ids = prompt
    with torch.no_grad():
        for _ in range(6):
            nxt = lm(ids)["logits"][:, -1].argmax(-1, keepdim=True)
            ids = torch.cat([ids, nxt], 1)
    assert torch.equal(got, ids)


def _rank_permutation(w):
    """Host restatement of the kernels' head ranking (window_rank_key and the
    (key, index) order of msa_device.h): rank of head o among the heads."""
    key = [math.inf if x != x else x for x in w]
    return [sum(1 for p in range(len(w)) if key[p] > key[o] or (key[p] == key[o] and p < o))
            for o in range(len(w))]


def test_nan_window_is_contained():
    # a NaN window (s_v diverged) must not fault or disturb other heads: the
    # head ranking stays a permutation, the NaN head's window is empty (its
    # output is zero where the reference's is NaN), and every other head's
    # output and gradients are bitwise those of a run with a finite window
    assert sorted(_rank_permutation([float("nan"), 3.0, float("nan"), 3.0, math.inf, -math.inf, 0.0, -0.0])) == \
        list(range(8))
    B, T, H, D = 2, 256, 8, 64
    q, k, v = correlated_qkv(B, T, T, H, D, seed=8, dtype=torch.bfloat16, rho=0.35)
    dy = torch.randn(B, T, H, D, generator=torch.Generator().manual_seed(2)).bfloat16().to(DEV)
    r = [1.1, 1.2, 1.15, 1.3, 1.1, 1.25, 1.2, 1.1]
    w_ok = [40.0, 2.0, 100.0, 100.0, 1e5, 7.5, 300.0, 60.0]
    w_nan = list(w_ok)
    w_nan[2] = float("nan")
    ops = _ops()
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    outs = []
    for w in (w_ok, w_nan):
        rg, wg = _rw(H, r, w)
        y, hnorm, bits = ops.fwd_raw(qd, kd, vd, rg, wg, True, 1e-8, None)
        outs.append((y,) + ops.bwd_raw(qd, kd, vd, rg, wg, True, 1e-8, y, hnorm, bits, dy))
    torch.cuda.synchronize()
    keep = [h for h in range(H) if h != 2]
    for a, b in zip(outs[0][:4], outs[1][:4]):          # y, dq, dk, dv
        assert torch.equal(a[:, :, keep], b[:, :, keep])
    assert torch.count_nonzero(outs[1][0][:, :, 2]) == 0
    for a, b in zip(outs[0][4:], outs[1][4:]):          # dr, dw
        assert torch.equal(a[keep], b[keep])
