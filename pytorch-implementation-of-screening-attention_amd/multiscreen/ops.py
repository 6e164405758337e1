"""Operator boundary of the fused Screening Attention core on MI355X.

`screening_core(q, k, v, r, w, causal, eps, key_padding_mask)` takes the raw
per-head projections as (B, T, H, D) views -- the `proj(x).view(B,T,H,D)`
tensors of multiscreen/attention.py:150-153, before their transpose -- and
returns TanhNorm(sum_j alpha_ij m_ij v^_j) as a (B, Tq, H, D) tensor, i.e. the
whole span attention.py:155-196 (normalise, similarity, trim-and-square,
softmask, key padding, aggregation, TanhNorm) as one HIP forward and one HIP
backward through libmsa.so.  The backward also returns the gradients of the
per-head r and w that the reference fused path drops
(attention_triton.py:44).

It is the counterpart of the reference's `_ScreeningFunc`
(attention_triton.py:24-48), whose inputs are already normalised and whose
output is pre-TanhNorm; here normalisation and TanhNorm are inside the
kernels, so their backward is too.

GPU tensors only: a CPU tensor, or a missing libmsa.so, raises.
"""

import torch

from . import _native

_DTYPES = {torch.float32: _native.MSA_F32, torch.bfloat16: _native.MSA_BF16, torch.float16: _native.MSA_F16}


def _stream_ptr(device):
    return torch.cuda.current_stream(device).cuda_stream


def _as_bthd(x, name, esize):
    """Returns x (B,T,H,D) with unit D stride and 16-byte-friendly strides."""
    if x.dim() != 4:
        raise ValueError(f"{name} must be 4-D (B, T, H, D), got {tuple(x.shape)}")
    mult = 16 // esize
    ok = (x.stride(3) == 1 and all(s % mult == 0 for s in x.stride()[:3])
          and x.data_ptr() % 16 == 0)
    return x if ok else x.contiguous()


def _args_bthd(x):
    return (x.data_ptr(), x.stride(0), x.stride(1), x.stride(2))


def tile_bits_words(B, H, Tq, Tk):
    return int(_native.lib().msa_tile_bits_words(B, H, Tq, Tk))


def _kpm_u8(key_padding_mask, B, Tk, dev):
    if key_padding_mask is None:
        return None
    if key_padding_mask.shape != (B, Tk):
        raise ValueError(f"key_padding_mask must have shape ({B}, {Tk})")
    return key_padding_mask.to(device=dev, dtype=torch.uint8).contiguous()


def _dropout_args(dropout_p, seed):
    p = float(dropout_p)
    if not 0.0 <= p < 1.0:
        raise ValueError(f"dropout probability must be in [0, 1), got {p}")
    return p, int(seed) & (2 ** 64 - 1)


def fwd_raw(q, k, v, r, w, causal=True, eps=1e-8, key_padding_mask=None, dropout_p=0.0, seed=0):
    """One msa_fwd call.  Returns (y, hnorm, tile_bits).

    q (B,Tq,H,D), k/v (B,Tk,H,D) in float32, bfloat16 or float16 on one GPU; r, w (H,).
    dropout_p / seed: attention dropout with the counter-based keep mask that
    include/msa.h defines (p = 0: none).
    """
    L = _native.lib()
    if not q.is_cuda:
        raise RuntimeError("screening_core runs on the GPU only (got a CPU tensor)")
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"q/k/v must share dtype float32, bfloat16 or float16, got {q.dtype}, {k.dtype}, {v.dtype}")
    dt = _DTYPES[q.dtype]
    es = q.element_size()
    q, k, v = _as_bthd(q, "q", es), _as_bthd(k, "k", es), _as_bthd(v, "v", es)
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    if k.shape != (B, Tk, H, D) or v.shape != k.shape:
        raise ValueError(f"k/v shape {tuple(k.shape)}/{tuple(v.shape)} do not match q {tuple(q.shape)}")
    if r.shape != (H,) or w.shape != (H,):
        raise ValueError(f"r and w must have shape ({H},)")
    dev = q.device
    r32 = r.detach().to(device=dev, dtype=torch.float32).contiguous()
    w32 = w.detach().to(device=dev, dtype=torch.float32).contiguous()
    kpm = _kpm_u8(key_padding_mask, B, Tk, dev)
    p, seed = _dropout_args(dropout_p, seed)
    y = torch.empty((B, Tq, H, D), dtype=q.dtype, device=dev)
    hnorm = torch.empty((B, H, Tq), dtype=torch.float32, device=dev)
    nwords = tile_bits_words(B, H, Tq, Tk)
    bits = torch.empty((max(nwords, 1),), dtype=torch.int32, device=dev)
    wsb = int(L.msa_fwd_workspace_bytes(B, H, Tq, Tk, D, dt))
    ws = torch.empty((max(wsb, 16),), dtype=torch.uint8, device=dev)
    rc = L.msa_fwd(*_args_bthd(q), *_args_bthd(k), *_args_bthd(v),
                   B, H, Tq, Tk, D, dt, r32.data_ptr(), w32.data_ptr(),
                   kpm.data_ptr() if kpm is not None else None, int(bool(causal)), float(eps), p, seed,
                   y.data_ptr(), hnorm.data_ptr(), bits.data_ptr(), nwords,
                   ws.data_ptr(), wsb, _stream_ptr(dev))
    _native.check(rc, "msa_fwd")
    return y, hnorm, bits


def bwd_raw(q, k, v, r, w, causal, eps, y, hnorm, bits, dy, key_padding_mask=None, dropout_p=0.0, seed=0):
    """One msa_bwd call.  Returns (dq, dk, dv, dr, dw); dq/dk/dv in (B,T,H,D).
    dropout_p / seed must be the forward's."""
    L = _native.lib()
    if q.dtype not in _DTYPES or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError(f"q/k/v must share dtype float32, bfloat16 or float16, got {q.dtype}, {k.dtype}, {v.dtype}")
    dt = _DTYPES[q.dtype]
    es = q.element_size()
    q, k, v = _as_bthd(q, "q", es), _as_bthd(k, "k", es), _as_bthd(v, "v", es)
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    dev = q.device
    dq = torch.empty((B, Tq, H, D), dtype=q.dtype, device=dev)
    dk = torch.empty((B, Tk, H, D), dtype=q.dtype, device=dev)
    dv = torch.empty((B, Tk, H, D), dtype=q.dtype, device=dev)
    dr = torch.empty((H,), dtype=torch.float32, device=dev)
    dw = torch.empty((H,), dtype=torch.float32, device=dev)
    if B == 0 or Tq == 0 or Tk == 0:
        return dq.zero_(), dk.zero_(), dv.zero_(), dr.zero_(), dw.zero_()
    dy = dy.to(q.dtype).contiguous()
    r32 = r.detach().to(device=dev, dtype=torch.float32).contiguous()
    w32 = w.detach().to(device=dev, dtype=torch.float32).contiguous()
    kpm = _kpm_u8(key_padding_mask, B, Tk, dev)
    p, seed = _dropout_args(dropout_p, seed)
    wsb = int(L.msa_bwd_workspace_bytes(B, H, Tq, Tk, D, dt))
    ws = torch.empty((max(wsb, 16),), dtype=torch.uint8, device=dev)
    rc = L.msa_bwd(*_args_bthd(q), *_args_bthd(k), *_args_bthd(v),
                   B, H, Tq, Tk, D, dt, r32.data_ptr(), w32.data_ptr(),
                   kpm.data_ptr() if kpm is not None else None, int(bool(causal)), float(eps), p, seed,
                   y.data_ptr(), hnorm.data_ptr(), dy.data_ptr(), bits.data_ptr(),
                   tile_bits_words(B, H, Tq, Tk),
                   dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dr.data_ptr(), dw.data_ptr(),
                   ws.data_ptr(), wsb, _stream_ptr(dev))
    _native.check(rc, "msa_bwd")
    return dq, dk, dv, dr, dw


class ScreeningCoreFunction(torch.autograd.Function):
    """Autograd wrapper: forward = msa_fwd, backward = msa_bwd."""

    @staticmethod
    def forward(ctx, q, k, v, r, w, causal, eps, key_padding_mask, dropout_p=0.0, seed=0):
        y, hnorm, bits = fwd_raw(q, k, v, r, w, causal, eps, key_padding_mask, dropout_p, seed)
        if any(ctx.needs_input_grad[:5]):
            ctx.save_for_backward(q, k, v, r, w, y, hnorm, bits, key_padding_mask)
        ctx.causal = causal
        ctx.eps = eps
        ctx.dropout = (dropout_p, seed)
        return y

    @staticmethod
    def backward(ctx, dy):
        q, k, v, r, w, y, hnorm, bits, kpm = ctx.saved_tensors
        dq, dk, dv, dr, dw = bwd_raw(q, k, v, r, w, ctx.causal, ctx.eps, y, hnorm, bits, dy, kpm, *ctx.dropout)
        return dq, dk, dv, dr.to(r.dtype), dw.to(w.dtype), None, None, None, None, None


def screening_core(q, k, v, r, w, causal=True, eps=1e-8, key_padding_mask=None, dropout_p=0.0, seed=0):
    """Fused screening attention core; see the module docstring.  dropout_p > 0
    applies attention dropout (attention.py:190) with the keep mask of `seed`."""
    return ScreeningCoreFunction.apply(q, k, v, r, w, causal, eps, key_padding_mask, dropout_p, seed)


def _decode_args(q, kcache, vcache, r, w):
    if not q.is_cuda:
        raise RuntimeError("decode_step runs on the GPU only (got a CPU tensor)")
    if q.dtype not in _DTYPES or kcache.dtype != q.dtype or vcache.dtype != q.dtype:
        raise TypeError(f"decode_step needs q and the caches in one of float32 / bfloat16 / float16, got "
                        f"{q.dtype}, {kcache.dtype}, {vcache.dtype}")
    B, H, D = q.shape
    if q.stride(2) != 1:
        q = q.contiguous()
    es = q.element_size()
    kcache, vcache = _as_bthd(kcache, "kcache", es), _as_bthd(vcache, "vcache", es)
    if kcache.shape != vcache.shape or kcache.shape[0] != B or kcache.shape[2:] != (H, D):
        raise ValueError(f"cache shapes {tuple(kcache.shape)}/{tuple(vcache.shape)} do not match q {tuple(q.shape)}")
    dev = q.device
    r32 = r.detach().to(device=dev, dtype=torch.float32).contiguous()
    w32 = w.detach().to(device=dev, dtype=torch.float32).contiguous()
    return q, kcache, vcache, r32, w32


def _decode_workspace(L, workspace, B, H, D, length, dev):
    need = int(L.msa_decode_workspace_bytes(B, H, D, int(length)))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty((max(need, 16),), dtype=torch.uint8, device=dev)
    return workspace


def decode_step(q, kcache, vcache, cache_len, r, w, eps=1e-8, workspace=None, window_hint=0):
    """Screening attention of one new query per (b, h) against a KV cache.

    q (B, H, D); kcache/vcache (B, Tcap, H, D) holding the raw k/v projections
    of positions [0, cache_len), the last being the query's own token.
    window_hint: 0, or a bound on ceil(w) over the heads (sizes the launch only).
    Returns y (B, H, D) = TanhNorm(h) of that token.
    """
    L = _native.lib()
    q, kcache, vcache, r32, w32 = _decode_args(q, kcache, vcache, r, w)
    B, H, D = q.shape
    dev = q.device
    y = torch.empty((B, H, D), dtype=q.dtype, device=dev)
    workspace = _decode_workspace(L, workspace, B, H, D, cache_len, dev)
    rc = L.msa_decode(q.data_ptr(), q.stride(0), q.stride(1),
                      *_args_bthd(kcache), *_args_bthd(vcache),
                      B, H, D, _DTYPES[q.dtype], int(cache_len), int(kcache.shape[1]), int(window_hint),
                      r32.data_ptr(), w32.data_ptr(),
                      float(eps),
                      y.data_ptr(), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                      _stream_ptr(dev))
    _native.check(rc, "msa_decode")
    return y


def decode_step_at(q, kcache, vcache, last_pos, r, w, eps=1e-8, workspace=None, window_hint=0):
    """decode_step with the query's position in device memory: last_pos is a
    CUDA int64 tensor of one element, the position of the newest key, so the
    cache holds positions [0, last_pos] (the length is clamped to the
    capacity).  Launches depend only on the shapes, so a captured call stays
    valid as last_pos advances on the device."""
    L = _native.lib()
    q, kcache, vcache, r32, w32 = _decode_args(q, kcache, vcache, r, w)
    if not (last_pos.is_cuda and last_pos.dtype == torch.int64 and last_pos.numel() == 1):
        raise TypeError("last_pos must be a CUDA int64 tensor of one element")
    B, H, D = q.shape
    dev = q.device
    cap = int(kcache.shape[1])
    y = torch.empty((B, H, D), dtype=q.dtype, device=dev)
    workspace = _decode_workspace(L, workspace, B, H, D, cap, dev)
    rc = L.msa_decode_at(q.data_ptr(), q.stride(0), q.stride(1),
                         *_args_bthd(kcache), *_args_bthd(vcache),
                         B, H, D, _DTYPES[q.dtype], last_pos.data_ptr(), cap, int(window_hint),
                         r32.data_ptr(), w32.data_ptr(),
                         float(eps),
                         y.data_ptr(), workspace.data_ptr(), workspace.numel() * workspace.element_size(),
                         _stream_ptr(dev))
    _native.check(rc, "msa_decode_at")
    return y
