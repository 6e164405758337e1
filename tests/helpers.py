"""Shared helpers for the tests: seeded inputs, error metrics, golden loading."""

import math
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rel_err(got, ref):
    """max|got-ref| / max|ref|  (per tensor; alpha is mostly zero, so elementwise
    relative error is meaningless)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = np.max(np.abs(ref))
    diff = np.max(np.abs(got - ref)) if got.size else 0.0
    if scale == 0.0:
        return float(diff)
    return float(diff / scale)


def qkv(B, Tq, Tk, H, D, seed=0, dtype=torch.float32):
    """Raw (B,T,H,D) projections drawn N(0,1) on the CPU, rounded to dtype."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, Tq, H, D, generator=g).to(dtype)
    k = torch.randn(B, Tk, H, D, generator=g).to(dtype)
    v = torch.randn(B, Tk, H, D, generator=g).to(dtype)
    return q, k, v


def correlated_qkv(B, Tq, Tk, H, D, seed=0, dtype=torch.float32, rho=0.6):
    """q and k sharing a common component so that many pairs pass a threshold."""
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(B, max(Tq, Tk), H, D, generator=g)
    q = rho * base[:, :Tq] + (1 - rho) * torch.randn(B, Tq, H, D, generator=g)
    k = rho * base[:, :Tk] + (1 - rho) * torch.randn(B, Tk, H, D, generator=g)
    v = torch.randn(B, Tk, H, D, generator=g)
    return q.to(dtype), k.to(dtype), v.to(dtype)


def np64(t):
    return t.detach().cpu().double().numpy()


def load_golden(name):
    return np.load(os.path.join(GOLDEN, f"{name}.npz"))


def golden_inputs(z):
    """Regenerates the reference run's inputs from the fixture's seed."""
    seed, B, Tq, Tk, d = int(z["seed"]), int(z["B"]), int(z["Tq"]), int(z["Tk"]), int(z["d_model"])
    g = torch.Generator().manual_seed(seed + 1)
    x = torch.randn(B, Tq, d, generator=g)
    mem = x if int(z["same_qkv"]) else torch.randn(B, Tk, d, generator=g)
    dy = torch.randn(B, Tq, d, generator=g)
    kpm = torch.from_numpy(z["kpm"]) if "kpm" in z.files else None
    return x, mem, dy, kpm


def golden_module(z, cls):
    """Builds `cls(d_model, H, causal)` under the fixture's seed and r/w values."""
    torch.manual_seed(int(z["seed"]))
    m = cls(int(z["d_model"]), int(z["H"]), causal=bool(int(z["causal"])))
    with torch.no_grad():
        m.s_r.copy_(torch.from_numpy(z["s_r"]))
        m.s_v.copy_(torch.from_numpy(z["s_v"]))
    return m


GOLDEN_ATTENTION = ["cfg1_default", "cfg1_r1p1", "cfg1_r1p135", "cfg1_r1p5", "small_kpm",
                    "small_noncausal_cross"]
