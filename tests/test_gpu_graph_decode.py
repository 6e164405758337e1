"""Decode with the position in device memory, and the replayed decode graph.

* msa_decode_at (the cache length read on the device) against msa_decode
  with the same length: bitwise equal, for window hints that take the
  one-block-per-head launch and the split launch, and a position past the
  capacity clamped to it.
* GraphDecoder (one greedy decode step captured as a HIP graph, replayed per
  token) against the eager decode loop on its own copy of the caches: every
  replay's logits and token bitwise equal to the eager step's, with eager work
  and synchronisation between the replays.
"""

import math

import numpy as np
import pytest
import torch

import screening_oracle as O
from helpers import correlated_qkv, np64, rel_err, rw64

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _ops():
    from multiscreen import ops
    return ops


def test_decode_at_matches_decode_for_every_launch_shape():
    B, T, H, D = 2, 5000, 24, 64
    q, k, v = correlated_qkv(B, T, T, H, D, seed=21, dtype=torch.bfloat16, rho=0.35)
    g = torch.Generator().manual_seed(4)
    r = (1.1 + 0.3 * torch.rand(H, generator=g)).tolist()
    w = (2.0 + 6000.0 * torch.rand(H, generator=g) ** 3).tolist()
    ops = _ops()
    rg = torch.tensor(r, device=DEV)
    wg = torch.tensor(w, device=DEV)
    kc, vc = k.to(DEV), v.to(DEV)
    for L in (1, 700, 2049, 5000):
        qd = q[:, L - 1].to(DEV)
        base = ops.decode_step(qd, kc, vc, L, rg, wg)
        pos = torch.tensor([L - 1], dtype=torch.int64, device=DEV)
        # 1 and 2048: one block per head (walking several chunks where the
        # hint is too small); 6002 and 0: the split launch
        for hint in (0, 1, 2048, math.ceil(max(w)), 10 ** 6):
            got = ops.decode_step_at(qd, kc, vc, pos, rg, wg, window_hint=hint)
            assert torch.equal(got, base), (L, hint)
            assert torch.equal(ops.decode_step(qd, kc, vc, L, rg, wg, window_hint=hint), base), (L, hint)
        ref = O.decode_row(np64(q[:, L - 1]), np64(k), np64(v), L, rw64(r), rw64(w))
        assert rel_err(np64(base), ref, heads=(0, 1)) <= 2e-2, L
    # a position past the capacity reads as the full cache
    qd = q[:, T - 1].to(DEV)
    far = torch.tensor([T + 100], dtype=torch.int64, device=DEV)
    assert torch.equal(ops.decode_step_at(qd, kc, vc, far, rg, wg, window_hint=64),
                       ops.decode_step(qd, kc, vc, T, rg, wg))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_graph_decoder_matches_eager_steps(dtype):
    from multiscreen import MultiscreenLM
    from multiscreen.model import GraphDecoder
    torch.manual_seed(0)
    B, T, STEPS, VOCAB = 3, 40, 24, 211
    lm = MultiscreenLM(vocab_size=VOCAB, d_model=128, num_heads=4, num_layers=2, max_seq_len=512)
    with torch.no_grad():
        for blk in lm.blocks:  # live pairs at init: r = 1.3, windows 3 .. 300
            blk.attn.s_r.fill_(math.log(0.3))
            blk.attn.s_v.copy_(torch.log(torch.linspace(2.0, 299.0, 4)))
    lm = lm.to(DEV, dtype).eval()
    prompt = torch.randint(0, VOCAB, (B, T), generator=torch.Generator().manual_seed(9)).to(DEV)
    caches_e = lm.new_cache(B, T + STEPS + 1, dtype, DEV)
    caches_g = lm.new_cache(B, T + STEPS + 1, dtype, DEV)
    with torch.no_grad():
        logits_e = lm.prefill(prompt, caches_e)
        logits_g = lm.prefill(prompt, caches_g)
    assert torch.equal(logits_e, logits_g)
    tok = logits_e.argmax(-1, keepdim=True)
    dec = GraphDecoder(lm, caches_g, tok, T, STEPS)
    toks = []
    for s in range(STEPS):
        with torch.no_grad():
            le = lm.decode_step(tok, caches_e, T + s)  # eager work between the replays
        tok = le.argmax(-1, keepdim=True)
        toks.append(tok)
        dec.step()
        torch.cuda.synchronize()
        assert torch.equal(dec.logits, le), s
        assert torch.equal(dec.token, tok), s
    assert torch.equal(dec.tokens, torch.cat(toks, dim=1))
    assert torch.equal(caches_g[0].k[:, :T + STEPS], caches_e[0].k[:, :T + STEPS])
    with pytest.raises(IndexError):
        dec.step()


def test_generate_greedy_matches_eager_argmax_loop():
    from multiscreen import MultiscreenLM
    torch.manual_seed(1)
    B, T, N, VOCAB = 2, 33, 17, 97
    lm = MultiscreenLM(vocab_size=VOCAB, d_model=64, num_heads=2, num_layers=2, max_seq_len=256)
    with torch.no_grad():
        for blk in lm.blocks:
            blk.attn.s_r.fill_(math.log(0.3))
    lm = lm.to(DEV, torch.bfloat16).eval()
    prompt = torch.randint(0, VOCAB, (B, T), generator=torch.Generator().manual_seed(2)).to(DEV)
    got = lm.generate_greedy(prompt, N)
    caches = lm.new_cache(B, T + N, torch.bfloat16, DEV)
    with torch.no_grad():
        tok = lm.prefill(prompt, caches).argmax(-1, keepdim=True)
        out = [prompt, tok]
        for s in range(1, N):
            tok = lm.decode_step(tok, caches, T + s - 1).argmax(-1, keepdim=True)
            out.append(tok)
    assert torch.equal(got, torch.cat(out, dim=1))
