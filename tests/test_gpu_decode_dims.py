"""Decode at every head dimension the kernels instantiate (D = 32, 64, 128;
D = 16 pads to 32) and both input types, through both launch shapes: one
block per head walking its window's 2048-key chunks (window hint at most one
chunk) and the split partial + reduce launch (larger hint).  Each against the
oracle's decode row, and the two launch shapes bitwise equal."""

import numpy as np
import pytest
import torch

import screening_oracle as O
from helpers import correlated_qkv, np64, rel_err, rw64

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 5e-3}
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16], ids=["f32", "bf16", "f16"])
@pytest.mark.parametrize("D", [32, 128])
def test_decode_head_dims(D, dtype):
    from multiscreen import ops
    B, T, H = 2, 4500, 3
    q, k, v = correlated_qkv(B, T, T, H, D, seed=23, dtype=dtype, rho=0.35)
    r, w = [1.15, 1.3, 1.6], [40.0, 2500.0, 1e6]
    rg = torch.tensor(r, device=DEV)
    wg = torch.tensor(w, device=DEV)
    kc, vc = k.to(DEV), v.to(DEV)
    for L in (1, 33, 2049, 4500):
        qd = q[:, L - 1].to(DEV)
        single = ops.decode_step(qd, kc, vc, L, rg, wg, window_hint=64)
        split = ops.decode_step(qd, kc, vc, L, rg, wg, window_hint=10 ** 6)
        torch.cuda.synchronize()
        assert torch.equal(single, split), L
        ref = O.decode_row(np64(q[:, L - 1]), np64(k), np64(v), L, rw64(r), rw64(w))
        assert np.max(np.abs(ref)) > 0
        assert rel_err(np64(split), ref, heads=(0, 1)) <= TOL[dtype], L
