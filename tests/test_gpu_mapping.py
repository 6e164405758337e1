"""Parity at the sequence lengths that take each branch of the unit kernels'
block -> (head, unit) mapping (msa_device.h xcd_interleave): a unit count
(2*ceil(T/64)) that is a multiple of 32 takes runs of four adjacent units per
XCD, a multiple of 8 only takes every eighth unit, and any other count the
plain order.  T = 1024 (32 units: one run cycle), 1536 (48: every eighth),
1088 (34: plain); the cross case (Tq = 1024, Tk = 1536, not causal) gives the
query-unit passes one branch and the key-unit pass another.  Forward output
and every gradient against the float64 oracle (oracle/screening_oracle.py) at
the bf16 parity tolerance, per tensor and per (b, h), and dr, dw head by head.
"""

import numpy as np
import pytest
import torch

import screening_oracle as O
from helpers import correlated_qkv, head_sum_err, np64, rel_err, rw64

pytestmark = pytest.mark.gpu

TOL = 2e-2  # bf16
DEV = "cuda"
CASES = [
    # Tq, Tk, causal
    (1024, 1024, True),
    (1536, 1536, True),
    (1088, 1088, True),
    (1024, 1536, False),
]


@pytest.mark.parametrize("case", CASES, ids=[f"Tq{c[0]}_Tk{c[1]}" for c in CASES])
def test_mapping_branches(case):
    from multiscreen import ops
    Tq, Tk, causal = case
    B, H, D = 2, 3, 32
    r, w = [1.3, 1.5, 1.8], [100.0, 700.0, 5000.0]
    print(f"mapping case Tq={Tq} Tk={Tk} causal={causal}", flush=True)
    q, k, v = correlated_qkv(B, Tq, Tk, H, D, seed=11, dtype=torch.bfloat16, rho=0.5)
    dy = torch.randn(B, Tq, H, D, generator=torch.Generator().manual_seed(12)).bfloat16()
    rg = torch.tensor(r, dtype=torch.float32, device=DEV)
    wg = torch.tensor(w, dtype=torch.float32, device=DEV)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    y, hnorm, bits = ops.fwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, None)
    dq, dk, dv, dr, dw = ops.bwd_raw(qd, kd, vd, rg, wg, causal, 1e-8, y, hnorm, bits, dy.to(DEV))
    torch.cuda.synchronize()
    args = (np64(q), np64(k), np64(v), rw64(r), rw64(w))
    yref = O.forward(*args, causal)
    ref = O.backward(*args, np64(dy), causal)
    assert np.max(np.abs(yref)) > 1e-3, "vacuous case"
    assert rel_err(np64(y), yref) <= TOL
    for name, got, want in zip(("dq", "dk", "dv"), (dq, dk, dv), ref[:3]):
        e = rel_err(np64(got), want)
        assert e <= TOL, f"{name}: rel err {e:.3e} > {TOL}"
    _, _, P = O.sparse_forward_backward(*args, np64(dy), causal)
    for name, got, want, scale in (("dr", dr, ref[3], P["dr_abs"]), ("dw", dw, ref[4], P["dw_abs"])):
        e = head_sum_err(np64(got), want, scale)
        assert e <= TOL, f"{name}: per-head error {e:.3e} > {TOL}"
