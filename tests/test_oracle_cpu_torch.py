"""Pins the torch-fp32 CPU baseline (oracle/cpu_torch.py) to the float64 oracle,
so the CPU throughput bench.py reports is that of a correct computation."""

import numpy as np
import torch

import cpu_torch
import screening_oracle as O
from helpers import correlated_qkv, np64, rel_err


def test_cpu_torch_baseline_matches_oracle():
    B, T, H, D = 1, 150, 2, 64
    q, k, v = correlated_qkv(B, T, T, H, D, seed=0, rho=0.35)
    r = torch.tensor([1.1, 1.3])
    w = torch.tensor([40.0, 1000.0])
    dy = torch.randn(B, T, H, D, generator=torch.Generator().manual_seed(1))
    y, dq, dk, dv, dr, dw = cpu_torch.fwd_bwd(q, k, v, r, w, dy)
    ref_y = O.forward(np64(q), np64(k), np64(v), r.double().numpy(), w.double().numpy())
    ref = O.backward(np64(q), np64(k), np64(v), r.double().numpy(), w.double().numpy(), np64(dy))
    assert rel_err(np64(y), ref_y) < 1e-5
    for got, want in zip((dq, dk, dv, dr, dw), ref):
        assert rel_err(np64(got), want) < 1e-4
