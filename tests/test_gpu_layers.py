"""MultiscreenDecoderLayer on the GPU (reference: multiscreen/layers.py:79-144).

The layer composes causal self-attention over the target (with
tgt_key_padding_mask), non-causal cross-attention from the target to a
memory of another length (with memory_key_padding_mask, layers.py:141) and
the FFN.  Its output and the gradients of x, of memory and of every
parameter (the per-head s_r, s_v of both attentions included) are compared
with a float64 copy of the same layer on the CPU whose attention cores are
the explicit-matrix math of attention.py:155-196.  With attention dropout
p > 0 the copy applies the same keep mask as the kernels (the counter-based
hash of include/msa.h, restated by the oracle) under the seed each core
draws from torch's generator; the FFN's own nn.Dropout is set to 0 in both,
since its mask comes from torch's device generator.

Tolerance: the fp32 bound of the north star, max|got-ref|/max|ref| and the
Frobenius ratio <= 1e-5 per tensor.
"""

import copy
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import screening_oracle as O
from helpers import np64, rel_err

pytestmark = pytest.mark.gpu

DEV = "cuda"
TOL = 1e-5


def _dense_core_f64(attn):
    """attn.core as explicit float64 matrices, with the kernels' dropout mask."""

    def core(q, k, v, key_padding_mask=None):
        B, Tq, H, D = q.shape
        Tk = k.shape[1]
        w, r = attn.window(), attn.sharpness()
        factor = None
        if attn.training and attn.attn_dropout.p > 0.0:
            seed = int(torch.randint(0, 2 ** 62, (1,)).item())   # as ScreeningAttention.core draws it
            f = O.dropout_factor((attn.attn_dropout.p, seed), B, H, np.arange(Tq), np.arange(Tk))
            factor = torch.from_numpy(f)
        qn = F.normalize(q.transpose(1, 2), dim=-1, eps=attn.eps)
        kn = F.normalize(k.transpose(1, 2), dim=-1, eps=attn.eps)
        vn = F.normalize(v.transpose(1, 2), dim=-1, eps=attn.eps)
        s = qn @ kn.transpose(-2, -1)
        a = torch.relu(1.0 - r.view(1, H, 1, 1) * (1.0 - s))
        i = torch.arange(Tq).view(Tq, 1)
        j = torch.arange(Tk).view(1, Tk)
        rel = (j - i).to(torch.float64).unsqueeze(0)
        ww = w.view(-1, 1, 1)
        m = 0.5 * (torch.cos(math.pi * rel / ww) + 1.0)
        inside = (rel > -ww) & (rel <= 0) if attn.causal else (rel.abs() < ww)
        p = a * a * (m * inside).unsqueeze(0)
        if key_padding_mask is not None:
            p = p.masked_fill(key_padding_mask.view(B, 1, 1, Tk), 0.0)
        if factor is not None:
            p = p * factor
        h = p @ vn
        n = torch.linalg.vector_norm(h, dim=-1, keepdim=True).clamp(min=attn.eps)
        return (h * (torch.tanh(n) / n)).transpose(1, 2)
    return core


@pytest.mark.parametrize("dropout", [0.0, 0.25], ids=["p0", "p0.25"])
def test_decoder_layer_self_and_cross_attention(dropout):
    from multiscreen import MultiscreenDecoderLayer
    B, Tq, Tk, d, H = 2, 96, 150, 64, 4
    torch.manual_seed(0)
    layer = MultiscreenDecoderLayer(d, H, dropout=dropout)
    with torch.no_grad():
        # sharpness near 1 and a spread of windows, so that many pairs are live
        layer.self_attn.s_r.copy_(torch.log(torch.tensor([0.1, 0.15, 0.2, 0.3])))
        layer.self_attn.s_v.copy_(torch.log(torch.tensor([3.0, 12.0, 40.0, 200.0])))
        layer.cross_attn.s_r.copy_(torch.log(torch.tensor([0.12, 0.1, 0.25, 0.15])))
        layer.cross_attn.s_v.copy_(torch.log(torch.tensor([20.0, 70.0, 5.0, 1e4])))
    layer.ffn[2].p = 0.0
    layer.ffn[4].p = 0.0
    layer.train()
    ref = copy.deepcopy(layer).double()
    ref.self_attn.core = _dense_core_f64(ref.self_attn)
    ref.cross_attn.core = _dense_core_f64(ref.cross_attn)
    layer = layer.to(DEV)

    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, Tq, d, generator=g)
    mem = torch.randn(B, Tk, d, generator=g)
    dy = torch.randn(B, Tq, d, generator=g)
    tgt_kpm = torch.zeros(B, Tq, dtype=torch.bool)
    tgt_kpm[1, -7:] = True
    tgt_kpm[0, 5] = True
    mem_kpm = torch.zeros(B, Tk, dtype=torch.bool)
    mem_kpm[0, -20:] = True
    mem_kpm[1, :3] = True

    xg, mg = x.to(DEV, copy=True).requires_grad_(), mem.to(DEV, copy=True).requires_grad_()
    torch.manual_seed(123)
    out = layer(xg, mg, tgt_key_padding_mask=tgt_kpm.to(DEV), memory_key_padding_mask=mem_kpm.to(DEV))
    out.backward(dy.to(DEV))
    torch.cuda.synchronize()

    xr, mr = x.double().requires_grad_(), mem.double().requires_grad_()
    torch.manual_seed(123)
    out_r = ref(xr, mr, tgt_key_padding_mask=tgt_kpm, memory_key_padding_mask=mem_kpm)
    out_r.backward(dy.double())

    pairs = {"out": (out, out_r), "dx": (xg.grad, xr.grad), "dmemory": (mg.grad, mr.grad)}
    for (n, p), (_, pr) in zip(layer.named_parameters(), ref.named_parameters()):
        pairs["d" + n] = (p.grad, pr.grad)
    # the attention terms are far from vacuous: the cores move the output
    assert layer.cross_attn.s_r.grad.abs().max() > 1e-4
    assert layer.self_attn.s_v.grad.abs().max() > 1e-6
    assert mg.grad.abs().max() > 1e-3
    for name, (got, want) in pairs.items():
        want = np64(want)
        assert np.max(np.abs(want)) > 0, f"{name} vacuous"
        e = rel_err(np64(got), want)
        print(f"decoder layer p={dropout}: {name} rel err {e:.3e}", flush=True)
        assert e <= TOL, f"{name}: rel err {e:.3e} > {TOL}"
