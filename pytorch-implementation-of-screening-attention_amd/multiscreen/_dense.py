"""Screening attention core for CPU tensors: explicit (Tq x Tk) matrices.

This is how the module runs when its tensors live on the host (the
reference's own unit tests are CPU-only, tests/test_attention.py).  GPU
tensors never come here: they always take the fused HIP kernels in ops.py.
Same inputs and output as ops.screening_core: raw (B,T,H,D) projections in,
TanhNorm'd (B,Tq,H,D) out, following attention.py:155-196.
"""

import math

import torch
import torch.nn.functional as F


def pair_mask(Tq, Tk, w, causal, device, q_offset=0):
    """(H, Tq, Tk) cosine soft mask with the window cut (attention.py:92-119, :174-183).

    Query row t sits at position q_offset + t (0 in the reference's forward,
    which aligns both index ranges at 0, attention.py:108-110)."""
    i = q_offset + torch.arange(Tq, device=device).view(Tq, 1)
    j = torch.arange(Tk, device=device).view(1, Tk)
    rel = (j - i).to(torch.float32).unsqueeze(0)          # j - i
    w = w.to(torch.float32).view(-1, 1, 1)
    m = 0.5 * (torch.cos(math.pi * rel / w) + 1.0)
    inside = (rel > -w) & (rel <= 0) if causal else (rel.abs() < w)
    return m * inside.to(m.dtype)


def screening_core_dense(q, k, v, r, w, causal=True, eps=1e-8, key_padding_mask=None,
                         dropout=None, q_offset=0):
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    qn = F.normalize(q.transpose(1, 2), dim=-1, eps=eps)
    kn = F.normalize(k.transpose(1, 2), dim=-1, eps=eps)
    vn = F.normalize(v.transpose(1, 2), dim=-1, eps=eps)
    s = qn @ kn.transpose(-2, -1)                            # (B,H,Tq,Tk)
    a = torch.relu(1.0 - r.view(1, H, 1, 1) * (1.0 - s))
    p = a * a * pair_mask(Tq, Tk, w, causal, q.device, q_offset).unsqueeze(0).to(a.dtype)
    if key_padding_mask is not None:
        p = p.masked_fill(key_padding_mask.view(B, 1, 1, Tk), 0.0)
    if dropout is not None:
        p = dropout(p)
    h = p @ vn.to(p.dtype)                                    # (B,H,Tq,D)
    n = torch.linalg.vector_norm(h, dim=-1, keepdim=True).clamp(min=eps)
    y = h * (torch.tanh(n) / n)
    return y.transpose(1, 2)                                  # (B,Tq,H,D)
