"""Degenerate parameters and shapes, forward and backward against the oracle.

* r = 1 (threshold 0: every pair with s > 0 is live, the densest case) and
  r just above 1;
* r so large that no pair passes (all outputs and gradients exactly zero);
* one batch with every key masked (its outputs exactly zero);
* w = 1 (each query sees only itself) and w = inf (unbounded window, mask 1);
* a single query (Tq = 1) and a single key (Tk = 1), causal and not.

Tolerances as in test_gpu_parity.py (max|got-ref|/max|ref| <= 1e-5 fp32,
2e-2 bf16); where the reference output is exactly zero, the kernel's must be
exactly zero too.
"""

import math

import numpy as np
import pytest
import torch

import screening_oracle as O
from helpers import correlated_qkv, head_sum_err, np64, rel_err, rw64

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 5e-3}
DEV = "cuda"

# name: B, Tq, Tk, H, D, causal, r, w, kpm rows fully masked
CASES = {
    "r_one": (1, 160, 160, 2, 64, True, [1.0, 1.0 + 1e-7], [60.0, 1e4], []),
    "r_one_noncausal": (1, 96, 130, 2, 32, False, [1.0, 1.05], [40.0, 1e3], []),
    "r_huge": (2, 128, 128, 2, 64, True, [1e6, 5e3], [100.0, 1e4], []),
    "all_keys_masked": (2, 100, 100, 2, 64, True, [1.1, 1.3], [50.0, 1e4], [1]),
    "w_one_and_inf": (1, 130, 130, 2, 64, True, [1.2, 1.3], [1.0, math.inf], []),
    "single_query": (2, 1, 70, 2, 64, False, [1.1, 1.2], [30.0, 1e3], []),
    "single_query_causal": (1, 1, 1, 3, 16, True, [1.0, 1.5, 3.0], [1.0, 2.0, 1e9], []),
    "single_key": (1, 90, 1, 2, 64, False, [1.1, 1.0], [100.0, 1e3], []),
}


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("name", list(CASES))
def test_degenerate_forward_backward(name, dtype):
    from multiscreen import ops
    B, Tq, Tk, H, D, causal, r, w, masked = CASES[name]
    print(f"degenerate {name} {dtype}", flush=True)
    q, k, v = correlated_qkv(B, Tq, Tk, H, D, seed=5, dtype=dtype, rho=0.35)
    dy = torch.randn(B, Tq, H, D, generator=torch.Generator().manual_seed(6)).to(dtype)
    kpm = None
    if masked:
        kpm = torch.zeros(B, Tk, dtype=torch.bool)
        for b in masked:
            kpm[b, :] = True
    rg = torch.tensor(r, dtype=torch.float32, device=DEV)
    wg = torch.tensor(w, dtype=torch.float32, device=DEV)
    qd, kd, vd, dyd = (t.to(DEV) for t in (q, k, v, dy))
    kpm_d = None if kpm is None else kpm.to(DEV)
    y, hnorm, bits = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, kpm_d)
    dq, dk, dv, dr, dw = ops.bwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, y, hnorm, bits, dyd, kpm_d)
    torch.cuda.synchronize()
    kpm_np = None if kpm is None else kpm.numpy()
    rr, ww = rw64(r), rw64(w)
    yref = O.forward(np64(q), np64(k), np64(v), rr, ww, causal, key_padding_mask=kpm_np)
    gref = O.backward(np64(q), np64(k), np64(v), rr, ww, np64(dy), causal, key_padding_mask=kpm_np)
    tol = TOL[dtype]
    for nm, got, want in zip(("y", "dq", "dk", "dv", "dr", "dw"), (y, dq, dk, dv, dr, dw), (yref,) + tuple(gref)):
        g = np64(got)
        assert np.all(np.isfinite(g)), f"{nm} not finite"
        if np.max(np.abs(want)) == 0.0:
            assert np.max(np.abs(g)) == 0.0, f"{nm}: reference is zero, kernel gives {np.max(np.abs(g)):.3e}"
        else:
            e = rel_err(g, want)
            assert e <= tol, f"{nm}: rel err {e:.3e} > {tol}"
    # dr, dw entry by entry, against the sum of each head's |terms| (a head
    # with no terms must be exactly zero)
    _, _, P = O.sparse_forward_backward(np64(q), np64(k), np64(v), rr, ww, np64(dy), causal,
                                        key_padding_mask=kpm_np)
    for nm, got, want, scale in (("dr", dr, gref[3], P["dr_abs"]), ("dw", dw, gref[4], P["dw_abs"])):
        e = head_sum_err(np64(got), want, scale)
        assert e <= tol, f"{nm}: per-head error {e:.3e} > {tol}"
    for b in masked:
        assert torch.count_nonzero(y[b]) == 0
    if name == "r_huge":
        assert torch.count_nonzero(bits) == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
def test_zero_and_tiny_rows(dtype):
    """Rows of q, k and v that are exactly zero (zero-padded inputs) or short
    (|x| about 8e-3, still normal in float16): attention.py:155-158 clamps |x|
    at eps, so a zero row normalises to zero and 1/max(|x|, eps) is 1e8.
    Outputs and gradients must stay finite and match the oracle; in float16 a
    pair weight times that 1e8 would overflow to inf (and inf * 0 = NaN),
    which the fp16 kernels avoid by scaling the rows instead."""
    from multiscreen import ops
    B, T, H, D = 2, 200, 2, 64
    causal, r, w = True, [1.1, 1.3], [60.0, 1e4]
    q, k, v = correlated_qkv(B, T, T, H, D, seed=9, dtype=torch.float32, rho=0.35)
    zero = {"dq": [5, 70], "dk": [3, 40, 41], "dv": [2, 8, 9, 150]}
    for x, zero_rows, tiny_rows in ((q, zero["dq"], [6, 71]), (k, zero["dk"], [4, 99]), (v, zero["dv"], [10, 151])):
        x[:, zero_rows] = 0.0
        x[:, tiny_rows] *= 1e-3
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    dy = torch.randn(B, T, H, D, generator=torch.Generator().manual_seed(4)).to(dtype)
    rg = torch.tensor(r, dtype=torch.float32, device=DEV)
    wg = torch.tensor(w, dtype=torch.float32, device=DEV)
    qd, kd, vd, dyd = (t.to(DEV) for t in (q, k, v, dy))
    y, hnorm, bits = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, None)
    dq, dk, dv, dr, dw = ops.bwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, y, hnorm, bits, dyd)
    torch.cuda.synchronize()
    rr, ww = rw64(r), rw64(w)
    yref = O.forward(np64(q), np64(k), np64(v), rr, ww, causal)
    gref = O.backward(np64(q), np64(k), np64(v), rr, ww, np64(dy), causal)
    for nm, got, want in zip(("y", "dq", "dk", "dv", "dr", "dw"), (y, dq, dk, dv, dr, dw), (yref,) + tuple(gref)):
        g = np64(got)
        assert np.max(np.abs(want)) > 0, f"{nm} vacuous"
        # the gradient of a zero row is dx^/eps (attention.py:155-158 under
        # autograd), 1e8 |dx^|: past the float16 range, where the correctly
        # rounded value is an infinity of the same sign.  Its few entries
        # that stay in range are 1e8 times a sum that cancels to below 6.6e-4,
        # which float16 operands cannot resolve, so in float16 those rows are
        # checked for the overflow only and left out of the comparison.
        over = np.abs(want) > torch.finfo(dtype).max
        if np.any(over):
            assert dtype == torch.float16, nm
            assert np.all(np.isin(np.nonzero(over)[1], zero[nm])), nm
            assert np.all(np.isinf(g[over]) & (np.sign(g[over]) == np.sign(want[over]))), nm
            print(f"zero/tiny rows {dtype} {nm}: {int(over.sum())} values past the float16 range are inf",
                  flush=True)
        if dtype == torch.float16 and nm in zero:
            g, want = g.copy(), want.copy()
            g[:, zero[nm]] = 0.0
            want[:, zero[nm]] = 0.0
        assert np.all(np.isfinite(g)), f"{nm} not finite"
        e = rel_err(g, want)
        print(f"zero/tiny rows {dtype} {nm}: rel err {e:.3e}", flush=True)
        assert e <= TOL[dtype], f"{nm}: rel err {e:.3e} > {TOL[dtype]}"
