"""Multi-head Screening Attention with the MI355X fused core.

Public interface, parameter names and initialisation are those of the
reference module (multiscreen/attention.py:23-200), so reference state_dicts
load unchanged:

    ScreeningAttention(d_model, num_heads, dropout=0.0, causal=True, eps=1e-8)
    .forward(query, key, value, key_padding_mask=None) -> (B, T_q, d_model)

    q_proj, k_proj, v_proj, out_proj : Linear(d, d, bias=False), created in
                                       that order (attention.py:52-55)
    s_v = linspace(0, ln 255, H)     : w = exp(s_v) + 1   (attention.py:63-64)
    s_r = zeros(H)                   : r = exp(s_r) + 1   (attention.py:65)

The projections and out_proj stay torch GEMMs.  Everything between them --
unit normalisation, similarity, trim-and-square, the cosine window, key
padding, the un-normalised aggregation and TanhNorm (attention.py:155-196) --
is one fused HIP forward and one fused HIP backward (ops.screening_core) for
GPU tensors; CPU tensors use the explicit-matrix form in _dense.py.
"""

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .norm import TanhNorm
from . import ops
from ._dense import screening_core_dense


class ScreeningAttention(nn.Module):
    """Multi-head Screening Attention (reference: attention.py:23-42).

    Args:
        d_model:    Total model dimension.
        num_heads:  Number of attention heads.
        dropout:    Dropout probability on attention weights.
        causal:     If True, apply causal masking (autoregressive decoding).
        eps:        Small value for numerical stability.
    """

    def __init__(self, d_model: int, num_heads: int, dropout: float = 0.0, causal: bool = True,
                 eps: float = 1e-8):
        super().__init__()
        assert d_model % num_heads == 0, "d_model must be divisible by num_heads"
        self.d_model = d_model
        self.num_heads = num_heads
        self.head_dim = d_model // num_heads
        self.causal = causal
        self.eps = eps

        self.q_proj = nn.Linear(d_model, d_model, bias=False)
        self.k_proj = nn.Linear(d_model, d_model, bias=False)
        self.v_proj = nn.Linear(d_model, d_model, bias=False)
        self.out_proj = nn.Linear(d_model, d_model, bias=False)

        # w = exp(s_v) + 1 (window), r = exp(s_r) + 1 (acceptance sharpness)
        self.s_v = nn.Parameter(torch.linspace(0, math.log(255), num_heads))
        self.s_r = nn.Parameter(torch.zeros(num_heads))

        self.attn_dropout = nn.Dropout(dropout)
        # attribute name kept from the reference (attention.py:69)
        self.tahn_norm = TanhNorm(eps=eps)

    def window(self) -> torch.Tensor:
        return torch.exp(self.s_v) + 1.0

    def sharpness(self) -> torch.Tensor:
        return torch.exp(self.s_r) + 1.0

    def project(self, x: torch.Tensor, proj: nn.Linear) -> torch.Tensor:
        """proj(x) viewed as (B, T, H, D) -- no copy (attention.py:150-151)."""
        return proj(x).view(x.shape[0], x.shape[1], self.num_heads, self.head_dim)

    @staticmethod
    def _plain(projs) -> bool:
        """True when every projection is a bias-free nn.Linear with no forward
        hooks (its own or global): only then does one GEMM over the stacked
        weights give exactly what calling the modules gives.  Anything else
        (hooks such as weight_norm or LoRA wrappers, subclasses, a bias) takes
        the per-module calls of attention.py:150-153."""
        from torch.nn.modules import module as _m
        if _m._global_forward_hooks or _m._global_forward_pre_hooks:
            return False
        return all(type(p) is nn.Linear and p.bias is None and not p._forward_hooks
                   and not p._forward_pre_hooks for p in projs)

    def project_qkv(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor):
        """q, k, v projections as (B, T, H, D) views (attention.py:147-153) from
        as few GEMMs as the inputs allow: one over the stacked q/k/v weights
        for self-attention (query is key is value), one for q and one over the
        stacked k/v weights when key is value (cross-attention over a memory),
        else three.  The views' time stride is then 3*d_model (or 2*d_model);
        the fused kernels read them in place.  The stacked weight is formed on
        every call (a copy of 2-3 d x d weights), so weight updates of any kind,
        in place or through .data, are always seen."""
        B, Tq, _ = query.shape
        Tk = key.shape[1]
        H, D, d = self.num_heads, self.head_dim, self.d_model
        if query is key and key is value and self._plain((self.q_proj, self.k_proj, self.v_proj)):
            wqkv = torch.cat((self.q_proj.weight, self.k_proj.weight, self.v_proj.weight))
            q, k, v = F.linear(query, wqkv).split(d, dim=-1)
            return q.view(B, Tq, H, D), k.view(B, Tq, H, D), v.view(B, Tq, H, D)
        q = self.project(query, self.q_proj)
        if key is value and self._plain((self.k_proj, self.v_proj)):
            k, v = F.linear(key, torch.cat((self.k_proj.weight, self.v_proj.weight))).split(d, dim=-1)
            return q, k.view(B, Tk, H, D), v.view(B, Tk, H, D)
        return q, self.project(key, self.k_proj), self.project(value, self.v_proj)

    def core(self, q, k, v, key_padding_mask=None):
        """(B,T,H,D) raw projections -> TanhNorm'd (B,Tq,H,D) head outputs."""
        w, r = self.window(), self.sharpness()
        dropping = self.training and self.attn_dropout.p > 0.0
        if q.is_cuda:
            if dropping:
                # keep mask from a counter-based hash of this seed (drawn from
                # torch's default generator, so torch.manual_seed reproduces it)
                seed = int(torch.randint(0, 2 ** 62, (1,)).item())
                return ops.screening_core(q, k, v, r, w, self.causal, self.eps, key_padding_mask,
                                          self.attn_dropout.p, seed)
            return ops.screening_core(q, k, v, r, w, self.causal, self.eps, key_padding_mask)
        return screening_core_dense(q, k, v, r, w, self.causal, self.eps, key_padding_mask,
                                    self.attn_dropout if dropping else None)

    def forward(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                key_padding_mask: torch.Tensor | None = None) -> torch.Tensor:
        """
        Args:
            query:            (B, T_q, d_model)
            key:              (B, T_k, d_model)
            value:            (B, T_k, d_model)
            key_padding_mask: (B, T_k) bool mask; True = position to ignore.
        Returns:
            out: (B, T_q, d_model)
        """
        B, T_q, _ = query.shape
        q, k, v = self.project_qkv(query, key, value)
        y = self.core(q, k, v, key_padding_mask)
        return self.out_proj(y.reshape(B, T_q, self.d_model))

    # ------------------------------------------------------------------
    # KV-cache inference (no reference counterpart: the reference's
    # MultiscreenLM.generate re-runs forward() on the whole prefix for every
    # token, model.py:111-141).  The cache holds the raw k/v projections
    # (viewed as (B, T_cap, H, D)); decode(pos) computes exactly row `pos` of
    # forward().
    # ------------------------------------------------------------------
    def prefill(self, x: torch.Tensor, cache) -> torch.Tensor:
        """Causal self-attention forward over x (B,T,d) at positions 0..T-1;
        also writes its k/v projections into cache[:, :T]."""
        B, T, _ = x.shape
        q, k, v = self.project_qkv(x, x, x)
        cache.store(k, v, 0)
        y = self.core(q, k, v)
        return self.out_proj(y.reshape(B, T, self.d_model))

    def decode(self, x: torch.Tensor, cache, pos, rw=None) -> torch.Tensor:
        """x (B,1,d) is the token at position `pos`; returns its attention output (B,1,d).

        pos: an int, or (on GPU) a CUDA int64 tensor of one element holding the
        position, so that the step can be captured once and replayed as the
        position advances on the device.  rw: optional (r, w) fp32 tensors
        computed beforehand (exp(s_r)+1, exp(s_v)+1), for callers decoding
        many tokens with fixed parameters."""
        if not self.causal:
            raise RuntimeError("KV-cache decode is defined for causal self-attention only")
        B = x.shape[0]
        q, k, v = self.project_qkv(x, x, x)
        r, w = rw if rw is not None else (self.sharpness(), self.window())
        if torch.is_tensor(pos):
            if not x.is_cuda:
                raise RuntimeError("a device position needs the GPU decode path")
            cache.store_at(k, v, pos)
            y = ops.decode_step_at(q[:, 0].to(cache.k.dtype), cache.k, cache.v, pos, r, w, self.eps,
                                   cache.workspace, cache.window_hint).to(x.dtype)
            return self.out_proj(y.reshape(B, 1, self.d_model))
        cache.store(k, v, pos)
        if x.is_cuda:
            y = ops.decode_step(q[:, 0].to(cache.k.dtype), cache.k, cache.v, pos + 1, r, w, self.eps,
                                cache.workspace, cache.window_hint).to(x.dtype)
        else:
            kc, vc = cache.k[:, :pos + 1], cache.v[:, :pos + 1]
            y = screening_core_dense(q, kc, vc, r, w, True, self.eps, q_offset=pos)[:, 0]
        return self.out_proj(y.reshape(B, 1, self.d_model))


class KVCache:
    """Raw k/v projections of one attention layer.

    Stored head-major, (B, H, capacity, D), so that one head's window is one
    contiguous stream for the decode kernel; `k` and `v` are the (B, capacity,
    H, D) views of that storage, the layout of the projections, in the model's
    dtype (float32, bfloat16 or float16)."""

    def __init__(self, batch, capacity, num_heads, head_dim, dtype, device, window_hint=0):
        # 0, or a bound on ceil(w) over the layer's heads: sizes the decode
        # launch to the windows instead of the cache (results do not depend on it)
        self.window_hint = int(window_hint)
        self._k = torch.zeros((batch, num_heads, capacity, head_dim), dtype=dtype, device=device)
        self._v = torch.zeros_like(self._k)
        self.k = self._k.permute(0, 2, 1, 3)
        self.v = self._v.permute(0, 2, 1, 3)
        self.workspace = None
        if self.k.is_cuda:
            from . import _native
            nbytes = int(_native.lib().msa_decode_workspace_bytes(batch, num_heads, head_dim, capacity))
            self.workspace = torch.empty((max(nbytes, 16),), dtype=torch.uint8, device=device)

    def store(self, k, v, pos):
        T = k.shape[1]
        if pos + T > self.k.shape[1]:
            raise IndexError(f"KV cache capacity {self.k.shape[1]} exceeded at position {pos + T}")
        self.k[:, pos:pos + T] = k.to(self.k.dtype)
        self.v[:, pos:pos + T] = v.to(self.v.dtype)

    def store_at(self, k, v, pos):
        """k, v (B,1,H,D) at the position held by the device int64 tensor pos
        (one element).  The caller keeps pos below the capacity."""
        self._k.index_copy_(2, pos, k.permute(0, 2, 1, 3).to(self._k.dtype))
        self._v.index_copy_(2, pos, v.permute(0, 2, 1, 3).to(self._v.dtype))
