"""The public API on CPU tensors: the reference's own unit tests
(tests/test_attention.py:8-118) plus golden values from the reference module,
state_dict compatibility and KV-cache generation."""

import math

import numpy as np
import pytest
import torch

from helpers import GOLDEN_ATTENTION, golden_inputs, golden_module, load_golden, np64, rel_err
from multiscreen import MultiscreenBlock, MultiscreenDecoderLayer, MultiscreenLM, ScreeningAttention, TanhNorm


class TestTanhNorm:
    def test_zero_input(self):
        out = TanhNorm()(torch.zeros(2, 4))
        assert out.shape == (2, 4) and torch.allclose(out, torch.zeros_like(out))

    def test_magnitude_bounded(self):
        out = TanhNorm()(torch.randn(8, 16) * 100)
        assert (out.norm(dim=-1) <= 1.0 + 1e-5).all()

    def test_direction_preserved(self):
        x = torch.randn(4, 8)
        out = TanhNorm()(x)
        assert torch.allclose(torch.nn.functional.normalize(x, dim=-1),
                              torch.nn.functional.normalize(out, dim=-1), atol=1e-5)


class TestScreeningAttention:
    def setup_method(self):
        self.B, self.T, self.d = 2, 16, 64
        self.attn = ScreeningAttention(d_model=self.d, num_heads=4)

    def test_output_shape(self):
        x = torch.randn(self.B, self.T, self.d)
        assert self.attn(x, x, x).shape == (self.B, self.T, self.d)

    def test_causal_masking(self):
        attn = ScreeningAttention(d_model=self.d, num_heads=4, causal=True)
        with torch.no_grad():
            attn.s_r.fill_(math.log(0.1))   # r = 1.1 so outputs are non-trivial
        x = torch.randn(1, self.T, self.d)
        x2 = x.clone()
        x2[0, -1] = torch.randn(self.d)
        out1, out2 = attn(x, x, x), attn(x2, x2, x2)
        assert torch.allclose(out1[0, :-1], out2[0, :-1], atol=1e-6)

    def test_key_padding_mask(self):
        x = torch.randn(self.B, self.T, self.d)
        mask = torch.zeros(self.B, self.T, dtype=torch.bool)
        mask[:, -4:] = True
        assert self.attn(x, x, x, key_padding_mask=mask).shape == (self.B, self.T, self.d)

    def test_non_causal(self):
        attn = ScreeningAttention(d_model=self.d, num_heads=4, causal=False)
        x = torch.randn(self.B, self.T, self.d)
        assert attn(x, x, x).shape == (self.B, self.T, self.d)

    def test_different_q_k_lengths(self):
        attn = ScreeningAttention(d_model=self.d, num_heads=4, causal=False)
        q, kv = torch.randn(self.B, 8, self.d), torch.randn(self.B, 20, self.d)
        assert attn(q, kv, kv).shape == (self.B, 8, self.d)

    def test_parameter_names_and_init(self):
        attn = ScreeningAttention(512, 8)
        assert sorted(attn.state_dict()) == sorted(
            ["q_proj.weight", "k_proj.weight", "v_proj.weight", "out_proj.weight", "s_v", "s_r"])
        w = torch.exp(attn.s_v) + 1
        assert abs(float(w[0]) - 2.0) < 1e-6 and abs(float(w[-1]) - 256.0) < 1e-3
        assert torch.all(attn.s_r == 0)
        assert hasattr(attn, "tahn_norm")


class TestMultiscreenBlock:
    def test_output_shape(self):
        block = MultiscreenBlock(d_model=64, num_heads=4)
        x = torch.randn(2, 16, 64)
        assert block(x).shape == x.shape

    def test_residual_gradient_flow(self):
        block = MultiscreenBlock(d_model=64, num_heads=4)
        x = torch.randn(2, 16, 64, requires_grad=True)
        block(x).sum().backward()
        assert x.grad is not None

    def test_decoder_layer(self):
        layer = MultiscreenDecoderLayer(d_model=64, num_heads=4)
        x, mem = torch.randn(2, 10, 64), torch.randn(2, 14, 64)
        assert layer(x, mem).shape == x.shape


class TestMultiscreenLM:
    def setup_method(self):
        self.model = MultiscreenLM(vocab_size=100, d_model=64, num_heads=4, num_layers=2, max_seq_len=64)

    def test_forward_logits_shape(self):
        ids = torch.randint(0, 100, (2, 16))
        assert self.model(ids)["logits"].shape == (2, 16, 100)

    def test_loss_computation(self):
        ids = torch.randint(0, 100, (2, 16))
        labels = ids.clone()
        labels[:, :4] = -100
        out = self.model(ids, labels=labels)
        assert "loss" in out and out["loss"].ndim == 0

    def test_generate(self):
        prompt = torch.randint(0, 100, (1, 4))
        assert self.model.generate(prompt, max_new_tokens=8).shape == (1, 12)

    def test_cached_generate_equals_full_recompute(self):
        # greedy decoding with the KV cache must pick the tokens that re-running
        # forward() on the whole prefix picks (the reference's generate, model.py:130-140)
        torch.manual_seed(0)
        lm = MultiscreenLM(vocab_size=50, d_model=64, num_heads=4, num_layers=2, max_seq_len=64)
        for blk in lm.blocks:
            with torch.no_grad():
                blk.attn.s_r.fill_(math.log(0.15))
                blk.attn.s_v.copy_(torch.log(torch.tensor([2.0, 7.0, 20.0, 60.0])))
        prompt = torch.randint(0, 50, (2, 5))
        got = lm.generate(prompt, max_new_tokens=12, top_k=1)
        ids = prompt
        for _ in range(12):
            nxt = lm(ids)["logits"][:, -1].argmax(-1, keepdim=True)
            ids = torch.cat([ids, nxt], 1)
        assert torch.equal(got, ids)


def test_float16_model_keeps_a_float16_cache():
    # the kernels take float16 directly (MSA_F16): the cache keeps the model's dtype
    from multiscreen.attention import KVCache
    c = KVCache(2, 8, 4, 16, torch.float16, "cpu")
    assert c.k.dtype == torch.float16 and c.v.shape == (2, 8, 4, 16)


def test_lm_matches_reference_golden():
    z = load_golden("lm_tiny")
    torch.manual_seed(0)
    lm = MultiscreenLM(vocab_size=100, d_model=64, num_heads=4, num_layers=2, max_seq_len=64)
    for blk in lm.blocks:
        with torch.no_grad():
            blk.attn.s_r.fill_(math.log(0.2))
            blk.attn.s_v.copy_(torch.log(torch.tensor([3.0, 15.0, 31.0, 63.0])))
    ids = torch.from_numpy(z["ids"])
    out = lm(ids, labels=ids)
    out["loss"].backward()
    sums = dict(zip(z["names"].tolist(), z["values"].tolist()))
    for k, v in lm.state_dict().items():
        assert abs(float(v.double().sum()) - sums[f"sd::{k}"]) <= 1e-6 * max(1.0, abs(sums[f"sd::{k}"])), k
    assert rel_err(np64(out["logits"]), z["logits"]) < 1e-5
    assert abs(float(out["loss"]) - float(z["loss"])) < 1e-5
    for n, p in lm.named_parameters():
        ref = sums[f"grad::{n}"]
        assert abs(float(p.grad.double().abs().sum()) - ref) <= 1e-4 * max(1e-6, ref), n


@pytest.mark.parametrize("name", GOLDEN_ATTENTION)
def test_module_cpu_matches_reference_golden(name):
    z = load_golden(name)
    m = golden_module(z, ScreeningAttention)
    for nm, lin in zip("qkvo", (m.q_proj, m.k_proj, m.v_proj, m.out_proj)):
        np.testing.assert_array_equal(lin.weight[:2].detach().numpy(), z[f"W{nm}_head"])
    x, mem, dy, kpm = golden_inputs(z)
    x.requires_grad_(True)
    same = bool(int(z["same_qkv"]))
    if not same:
        mem.requires_grad_(True)
    y = m(x, x if same else mem, x if same else mem, key_padding_mask=kpm)
    (y * dy).sum().backward()
    yref = z["y"]
    if np.max(np.abs(yref)) == 0:
        assert torch.count_nonzero(y) == 0
        return
    assert rel_err(np64(y), yref) < 1e-5
    assert rel_err(np64(x.grad), z["dx"]) < 1e-5
    assert rel_err(np64(m.s_r.grad), z["ds_r"]) < 1e-5
    assert rel_err(np64(m.s_v.grad), z["ds_v"]) < 1e-5


def test_fused_qkv_projection_matches_separate_linears():
    # one GEMM over the stacked q/k/v weights (self-attention) or k/v weights
    # (cross-attention) gives the three projections; state_dict keys unchanged
    from multiscreen import ScreeningAttention
    torch.manual_seed(0)
    m = ScreeningAttention(64, 4)
    x, mem = torch.randn(2, 9, 64), torch.randn(2, 5, 64)
    sep = [m.project(t, p) for t, p in ((x, m.q_proj), (x, m.k_proj), (x, m.v_proj))]
    for got, want in zip(m.project_qkv(x, x, x), sep):
        assert got.shape == (2, 9, 4, 16)
        torch.testing.assert_close(got, want, rtol=1e-6, atol=1e-6)
    got = m.project_qkv(x, mem, mem)
    for t, p, g in ((x, m.q_proj, got[0]), (mem, m.k_proj, got[1]), (mem, m.v_proj, got[2])):
        torch.testing.assert_close(g, m.project(t, p), rtol=1e-6, atol=1e-6)
    assert sorted(k for k in m.state_dict() if k.endswith("weight")) == \
        ["k_proj.weight", "out_proj.weight", "q_proj.weight", "v_proj.weight"]
    # gradients reach each Linear through the stacked weight
    m.project_qkv(x, x, x)[1].sum().backward()
    assert m.k_proj.weight.grad.abs().sum() > 0
    assert m.q_proj.weight.grad is None or m.q_proj.weight.grad.abs().sum() == 0


def test_stacked_projection_follows_weight_updates_of_every_kind():
    """In place, through .data (no version bump), and by reassignment: the
    next no-grad forward sees the new weights."""
    from multiscreen import ScreeningAttention
    torch.manual_seed(1)
    m = ScreeningAttention(32, 2)
    x = torch.randn(1, 4, 32)
    mem = torch.randn(1, 6, 32)
    with torch.no_grad():
        a = m.project_qkv(x, x, x)[2].clone()
        m.v_proj.weight.mul_(2.0)
        torch.testing.assert_close(m.project_qkv(x, x, x)[2], 2.0 * a, rtol=1e-6, atol=1e-6)
        m.v_proj.weight.data.mul_(3.0)      # .data: the version counter does not move
        torch.testing.assert_close(m.project_qkv(x, x, x)[2], 6.0 * a, rtol=1e-6, atol=1e-6)
        kv0 = m.project_qkv(x, mem, mem)[1].clone()
        m.k_proj.weight.data.copy_(-m.k_proj.weight.data)
        torch.testing.assert_close(m.project_qkv(x, mem, mem)[1], -kv0, rtol=1e-6, atol=1e-6)
        m.s_r.fill_(-3.0)                   # r = 1.05: most pairs are live
        y0 = m(x, x, x)
        assert y0.abs().max() > 0
        m.q_proj.weight.data.add_(torch.randn_like(m.q_proj.weight))
        assert not torch.equal(m(x, x, x), y0)


def test_projection_hooks_are_honoured():
    """A forward hook on a projection (weight_norm, LoRA-style wrappers) takes
    the per-module calls, so the hook runs and its result is used."""
    from multiscreen import ScreeningAttention
    torch.manual_seed(2)
    m = ScreeningAttention(32, 2)
    x = torch.randn(1, 5, 32)
    mem = torch.randn(1, 7, 32)
    calls = []

    def hook(mod, inp, out):
        calls.append(mod)
        return out * 2.0

    want = m.project(x, m.k_proj) * 2.0
    h = m.k_proj.register_forward_hook(hook)
    got = m.project_qkv(x, x, x)[1]
    torch.testing.assert_close(got, want, rtol=1e-6, atol=1e-6)
    got = m.project_qkv(x, mem, mem)[1]
    torch.testing.assert_close(got, m.project(mem, m.k_proj), rtol=1e-6, atol=1e-6)
    assert len(calls) >= 2
    h.remove()
    torch.testing.assert_close(m.project_qkv(x, x, x)[1], want / 2.0, rtol=1e-6, atol=1e-6)
