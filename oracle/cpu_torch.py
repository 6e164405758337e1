"""CPU baseline: the reference's dense screening-attention core in torch fp32.

TEST / MEASUREMENT INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg and
tests).  It runs the same sequence of torch ops as the reference's dense path,
/root/reference/multiscreen/attention.py:155-196 and norm.py:23-25
(F.normalize x3, matmul, trim-and-square, cosine soft mask, masked aggregate,
TanhNorm), on CPU tensors with autograd for the backward -- i.e. what the
reference itself executes for this span on a CPU.  Pinned against the float64
oracle in tests/test_oracle_cpu_torch.py.
"""

import math

import torch
import torch.nn.functional as F


def core(q, k, v, r, w, causal=True, eps=1e-8):
    """q,k,v (B,T,H,D) raw projections; r,w (H,).  Returns y (B,Tq,H,D)."""
    q, k, v = (F.normalize(x.transpose(1, 2), dim=-1, eps=eps) for x in (q, k, v))
    H, Tq, Tk = q.shape[1], q.shape[2], k.shape[2]
    sim = torch.matmul(q, k.transpose(-2, -1))
    alpha = F.relu(1.0 - r.view(1, -1, 1, 1) * (1.0 - sim)).pow(2)
    i = torch.arange(Tq).unsqueeze(1)
    j = torch.arange(Tk).unsqueeze(0)
    rel = (j - i).float()
    w3 = w.view(-1, 1, 1)
    cos_mask = 0.5 * (torch.cos(math.pi * rel.unsqueeze(0) / w3) + 1.0)
    if causal:
        inside = (rel.unsqueeze(0) > -w3) & (rel.unsqueeze(0) <= 0)
    else:
        inside = rel.abs().unsqueeze(0) < w3
    alpha = alpha * (cos_mask * inside.float()).unsqueeze(0)
    h = torch.matmul(alpha, v)
    n = h.norm(dim=-1, keepdim=True).clamp(min=eps)
    return ((torch.tanh(n) / n) * h).transpose(1, 2)


def fwd_bwd(q, k, v, r, w, dy, causal=True):
    """One forward + backward; returns (y, dq, dk, dv, dr, dw)."""
    q, k, v, r, w = (t.detach().clone().requires_grad_(True) for t in (q, k, v, r, w))
    y = core(q, k, v, r, w, causal)
    (y * dy).sum().backward()
    return y.detach(), q.grad, k.grad, v.grad, r.grad, w.grad
