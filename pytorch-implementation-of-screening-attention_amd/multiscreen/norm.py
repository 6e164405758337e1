"""TanhNorm: keeps a vector's direction and bounds its length below 1.

    TanhNorm(x) = tanh(|x|) / |x| * x,   |x| clamped below at eps

Same module and argument as the reference (multiscreen/norm.py:8-25).  In the
attention path the same map runs inside the fused HIP forward's epilogue; this
module is the stand-alone form.
"""

import torch
import torch.nn as nn


class TanhNorm(nn.Module):
    def __init__(self, eps: float = 1e-8):
        super().__init__()
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        n = torch.linalg.vector_norm(x, dim=-1, keepdim=True).clamp(min=self.eps)
        return x * (torch.tanh(n) / n)
