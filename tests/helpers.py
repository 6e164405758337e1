"""Shared helpers for the tests: seeded inputs, error metrics, golden loading."""

import math
import os

import numpy as np
import torch

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


# Slices of a tensor checked at their own scale by rel_err: per (b, h) for
# the (B, T, H, D) layout of q/k/v/y and their gradients; for other tensors
# per index of the axes the caller names (e.g. heads=(0, 1) for (B, H, T) row
# norms or (B, H, D) decode rows).  A slice is measured against
# max(max|ref over the slice|, SLICE_FLOOR * max|ref|): a head whose values
# reach a hundredth of the largest head's is held to the tolerance on its own
# magnitude, and a smaller one at that hundredth.  Below it the comparison
# would divide by values that rounding alone decides: pairs within bf16
# rounding of the threshold (alpha <= (r 2^-9)^2, about 1.6e-5) are voted on
# K^ rounded to bf16, and an fp32 head output that cancels to far below its
# terms carries their rounding.
SLICE_FLOOR = 1e-2


def errors(got, ref, heads=None):
    """Error metrics of got against ref (float64):
      max    max|got-ref| / max|ref| over the whole tensor (alpha is mostly
             zero, so elementwise relative error is meaningless);
      fro    ||got-ref|| / ||ref|| (Frobenius);
      slice  the largest per-slice max|got-ref| / max(max|ref slice|,
             SLICE_FLOOR max|ref|), slices as described above (= max when
             the tensor has no head axes).
    A reference of all zeros gives the absolute error for each."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    d = np.abs(got - ref)
    scale = float(np.max(np.abs(ref))) if ref.size else 0.0
    dmax = float(np.max(d)) if d.size else 0.0
    if scale == 0.0:
        return {"max": dmax, "fro": dmax, "slice": dmax}
    out = {"max": dmax / scale,
           "fro": float(np.sqrt(np.sum(d * d)) / np.sqrt(np.sum(ref * ref)))}
    if heads is None and ref.ndim == 4:
        heads = (0, 2)
    if heads:
        axes = tuple(a for a in range(ref.ndim) if a not in heads)
        sref = np.max(np.abs(ref), axis=axes)
        sd = np.max(d, axis=axes)
        out["slice"] = float(np.max(sd / np.maximum(sref, SLICE_FLOOR * scale)))
    else:
        out["slice"] = out["max"]
    return out


def rel_err(got, ref, heads=None):
    """The largest of errors(got, ref, heads): whole-tensor max-relative,
    Frobenius ratio and per-head max-relative, so an error cannot hide behind
    a larger head of the same tensor."""
    return max(errors(got, ref, heads).values())


def head_sum_err(got, ref, abs_sum, floor=SLICE_FLOOR):
    """Per-entry error of per-head sums (dr, dw): max over heads of
    |got_h - ref_h| / max(S_h, floor * max_h S_h), S_h the sum over the head's
    pairs of |term|.  A sum of terms of both signs can cancel to far below its
    terms, and its rounding error scales with the terms, not with the total;
    for a sum of terms of one sign this is the plain relative error.  As for
    slices, a head whose terms weigh less than `floor` of the heaviest head's
    is held to that level (its few terms sit near the threshold, where a's
    relative error r|ds|/a is large).  Heads with no terms must be exactly
    zero."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    abs_sum = np.asarray(abs_sum, dtype=np.float64)
    d = np.abs(got - ref)
    if np.any((abs_sum == 0) & (d != 0)):
        return float("inf")
    nz = abs_sum > 0
    if not np.any(nz):
        return 0.0
    scale = np.maximum(abs_sum, floor * np.max(abs_sum))
    return float(np.max(d[nz] / scale[nz]))


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


def rw64(x):
    """Per-head r or w as the kernels receive them (fp32 device arrays),
    widened to float64 for the oracle.  Near a window edge the fp32 rounding
    of w matters: at w = 1 + 3e-4, dm/dw of the pair at |i - j| = 1 is
    proportional to w - 1, which fp32(w) shifts by 2e-4 relative."""
    return np.asarray(x, dtype=np.float32).astype(np.float64)


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
