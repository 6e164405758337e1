"""Pre-norm Multiscreen blocks (reference: multiscreen/layers.py:15-144).

Same constructors, submodule names and forward signatures as the reference,
so state_dicts are interchangeable:

    MultiscreenBlock(d_model, num_heads, ffn_dim=None, dropout=0.0, causal=True)
        x = x + attn(norm1(x));  x = x + ffn(norm2(x))
    MultiscreenDecoderLayer(d_model, num_heads, ffn_dim=None, dropout=0.0)
        x = x + self_attn(norm1(x));  x = x + cross_attn(norm2(x), memory)
        x = x + ffn(norm3(x))

MultiscreenBlock additionally exposes prefill/decode steps over a KV cache,
used by MultiscreenLM.generate.
"""

import torch
import torch.nn as nn

from .attention import ScreeningAttention


def _ffn(d_model, ffn_dim, dropout):
    return nn.Sequential(
        nn.Linear(d_model, ffn_dim, bias=False),
        nn.GELU(),
        nn.Dropout(dropout),
        nn.Linear(ffn_dim, d_model, bias=False),
        nn.Dropout(dropout),
    )


class MultiscreenBlock(nn.Module):
    def __init__(self, d_model: int, num_heads: int, ffn_dim: int | None = None,
                 dropout: float = 0.0, causal: bool = True):
        super().__init__()
        ffn_dim = ffn_dim or 4 * d_model
        self.norm1 = nn.RMSNorm(d_model)
        self.norm2 = nn.RMSNorm(d_model)
        self.attn = ScreeningAttention(d_model=d_model, num_heads=num_heads, dropout=dropout,
                                       causal=causal)
        self.ffn = _ffn(d_model, ffn_dim, dropout)

    def forward(self, x: torch.Tensor, key_padding_mask: torch.Tensor | None = None) -> torch.Tensor:
        normed = self.norm1(x)
        x = x + self.attn(normed, normed, normed, key_padding_mask=key_padding_mask)
        return x + self.ffn(self.norm2(x))

    def prefill(self, x: torch.Tensor, cache) -> torch.Tensor:
        """forward() over a prompt starting at position 0, storing its raw k/v in `cache`."""
        normed = self.norm1(x)
        x = x + self.attn.prefill(normed, cache)
        return x + self.ffn(self.norm2(x))

    def decode(self, x: torch.Tensor, cache, pos, rw=None) -> torch.Tensor:
        """One token x (B,1,d) at position `pos` (int or device tensor), attending to the cache."""
        normed = self.norm1(x)
        x = x + self.attn.decode(normed, cache, pos, rw)
        return x + self.ffn(self.norm2(x))


class MultiscreenDecoderLayer(nn.Module):
    def __init__(self, d_model: int, num_heads: int, ffn_dim: int | None = None,
                 dropout: float = 0.0):
        super().__init__()
        ffn_dim = ffn_dim or 4 * d_model
        self.norm1 = nn.RMSNorm(d_model)
        self.norm2 = nn.RMSNorm(d_model)
        self.norm3 = nn.RMSNorm(d_model)
        self.self_attn = ScreeningAttention(d_model=d_model, num_heads=num_heads, dropout=dropout,
                                            causal=True)
        self.cross_attn = ScreeningAttention(d_model=d_model, num_heads=num_heads, dropout=dropout,
                                             causal=False)
        self.ffn = _ffn(d_model, ffn_dim, dropout)

    def forward(self, x: torch.Tensor, memory: torch.Tensor,
                tgt_key_padding_mask: torch.Tensor | None = None,
                memory_key_padding_mask: torch.Tensor | None = None) -> torch.Tensor:
        normed = self.norm1(x)
        x = x + self.self_attn(normed, normed, normed, key_padding_mask=tgt_key_padding_mask)
        normed = self.norm2(x)
        x = x + self.cross_attn(normed, memory, memory, key_padding_mask=memory_key_padding_mask)
        return x + self.ffn(self.norm3(x))
