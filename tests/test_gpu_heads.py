"""Head-count regimes of the screen planner and the unit kernels' head order.

The planner runs in one of several modes by B*H: one block plans all 32
dispatch lanes (B*H < 32); one block per XCD deals whole heads to XCDs,
widest window first (32 <= B*H <= 512); past 512 heads the ranking is
skipped, and past 8*512 heads a planner block keeps no per-head table.  The
unit kernels rank heads when H <= 64 and H divides the rows.  Each regime is
run forward and backward against the float64 oracle at a short T, with
windows that differ per head (so the ranking matters) and some heads with no
live pair at all.  Tolerances as in test_gpu_parity.py.
"""

import numpy as np
import pytest
import torch

import screening_oracle as O
from helpers import correlated_qkv, np64, rel_err, head_sum_err, rw64

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2}
DEV = "cuda"

# B, T, H, D, causal
REGIMES = [
    (5, 128, 8, 64, True),      # 40 heads: per-XCD planning, XCDs hold 5 or 4 heads
    (3, 96, 11, 32, False),     # 33 heads, H odd, non-causal
    (75, 64, 8, 64, True),      # 600 heads: planner ranking skipped
    (29, 64, 18, 32, True),     # 522 heads, not a multiple of 8: XCDs hold 66 or 65 heads
    (1, 128, 72, 64, True),     # H = 72 > 64: unit kernels keep index order
    (513, 64, 8, 32, True),     # 4104 heads: more than 512 head slots per XCD
]


def _params(H, seed):
    g = torch.Generator().manual_seed(seed)
    r = (1.1 + 0.3 * torch.rand(H, generator=g)).tolist()
    w = (2.0 + 300.0 * torch.rand(H, generator=g) ** 2).tolist()
    r[0] = 40.0  # threshold 0.975: this head has (almost) no live pair
    return r, w


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("regime", REGIMES, ids=[f"B{b}H{h}" for b, _, h, _, _ in REGIMES])
def test_head_regime_forward_backward(regime, dtype):
    from multiscreen import ops
    B, T, H, D, causal = regime
    print(f"heads: B={B} T={T} H={H} D={D} causal={causal} {dtype}", flush=True)
    q, k, v = correlated_qkv(B, T, T, H, D, seed=3, dtype=dtype, rho=0.35)
    dy = torch.randn(B, T, H, D, generator=torch.Generator().manual_seed(5)).to(dtype)
    r, w = _params(H, 17)
    rg = torch.tensor(r, device=DEV)
    wg = torch.tensor(w, device=DEV)
    qd, kd, vd, dyd = (t.to(DEV) for t in (q, k, v, dy))
    y, hnorm, bits = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, None)
    dq, dk, dv, dr, dw = ops.bwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, y, hnorm, bits, dyd)
    torch.cuda.synchronize()
    rr, ww = rw64(r), rw64(w)
    yref = O.forward(np64(q), np64(k), np64(v), rr, ww, causal)
    gref = O.backward(np64(q), np64(k), np64(v), rr, ww, np64(dy), causal)
    tol = TOL[dtype]
    for name, got, want in zip(("y", "dq", "dk", "dv", "dr", "dw"), (y, dq, dk, dv, dr, dw), (yref,) + tuple(gref)):
        assert np.max(np.abs(want)) > 0, f"{name} vacuous"
        e = rel_err(np64(got), want)
        assert e <= tol, f"{name}: rel err {e:.3e} > {tol}"
    # dr, dw entry by entry, against the sum of each head's |terms|
    _, _, P = O.sparse_forward_backward(np64(q), np64(k), np64(v), rr, ww, np64(dy), causal)
    for name, got, want, scale in (("dr", dr, gref[3], P["dr_abs"]), ("dw", dw, gref[4], P["dw_abs"])):
        e = head_sum_err(np64(got), want, scale)
        assert e <= tol, f"{name}: per-head error {e:.3e} > {tol}"
