"""MultiscreenLM: causal language model built from Multiscreen blocks.

Reference: multiscreen/model.py:12-141.  Same constructor, submodule names
(token_emb, pos_emb, emb_dropout, blocks, norm, lm_head), tied weights,
initialisation (_init_weights, model.py:64-69), forward() contract (logits and
an un-shifted cross-entropy with ignore_index=-100, model.py:101-106) and
generate() signature and sampling (temperature, optional top-k, multinomial,
model.py:111-141).

generate() differs only in cost: instead of re-running forward() over the
whole prefix for every new token, it prefills a per-layer KV cache once and
then runs one single-query decode step per token (the HIP decode kernel on
GPU), which computes the same last-position logits.
"""

import math

import torch
import torch.nn as nn
import torch.nn.functional as F

from .attention import KVCache
from .layers import MultiscreenBlock


class MultiscreenLM(nn.Module):
    def __init__(self, vocab_size: int, d_model: int = 512, num_heads: int = 8, num_layers: int = 6,
                 ffn_dim: int | None = None, max_seq_len: int = 2048, dropout: float = 0.0,
                 tie_weights: bool = True):
        super().__init__()
        self.d_model = d_model
        self.token_emb = nn.Embedding(vocab_size, d_model)
        self.pos_emb = nn.Embedding(max_seq_len, d_model)
        self.emb_dropout = nn.Dropout(dropout)
        self.blocks = nn.ModuleList([
            MultiscreenBlock(d_model=d_model, num_heads=num_heads, ffn_dim=ffn_dim, dropout=dropout,
                             causal=True)
            for _ in range(num_layers)
        ])
        self.norm = nn.RMSNorm(d_model)
        self.lm_head = nn.Linear(d_model, vocab_size, bias=False)
        if tie_weights:
            self.lm_head.weight = self.token_emb.weight
        self._init_weights()

    def _init_weights(self):
        nn.init.normal_(self.token_emb.weight, std=0.02)
        nn.init.normal_(self.pos_emb.weight, std=0.02)
        for module in self.modules():
            if isinstance(module, nn.Linear):
                nn.init.normal_(module.weight, std=0.02)

    def embed(self, input_ids: torch.Tensor, start=0) -> torch.Tensor:
        """Token + position embeddings from position `start` (an int, or for one
        token a device int64 tensor of one element)."""
        T = input_ids.shape[1]
        if torch.is_tensor(start):
            positions = start.view(1, 1)
        else:
            positions = torch.arange(start, start + T, device=input_ids.device).unsqueeze(0)
        return self.emb_dropout(self.token_emb(input_ids) + self.pos_emb(positions))

    def forward(self, input_ids: torch.Tensor, key_padding_mask: torch.Tensor | None = None,
                labels: torch.Tensor | None = None) -> dict[str, torch.Tensor]:
        """
        Args:
            input_ids:        (B, T) integer token ids.
            key_padding_mask: (B, T) bool -- True = padding position.
            labels:           (B, T) token ids; -100 is ignored.
        Returns:
            {'logits': (B, T, vocab)} plus 'loss' when labels are given.
        """
        x = self.embed(input_ids)
        for block in self.blocks:
            x = block(x, key_padding_mask=key_padding_mask)
        logits = self.lm_head(self.norm(x))
        result = {"logits": logits}
        if labels is not None:
            result["loss"] = F.cross_entropy(logits.view(-1, logits.size(-1)), labels.view(-1),
                                             ignore_index=-100)
        return result

    def new_cache(self, batch: int, capacity: int, dtype: torch.dtype, device) -> list:
        """One KVCache per block.  Each carries its layer's widest window
        (ceil(max_h w_h), read once here) so that decode launches only the
        blocks the windows need."""
        caches = []
        for block in self.blocks:
            attn = block.attn
            with torch.no_grad():
                wmax = float(attn.window().max())
            hint = min(capacity, math.ceil(wmax)) if math.isfinite(wmax) else 0
            caches.append(KVCache(batch, capacity, attn.num_heads, attn.head_dim, dtype, device, hint))
        return caches

    def _head(self, x: torch.Tensor) -> torch.Tensor:
        return self.lm_head(self.norm(x))

    @torch.no_grad()
    def prefill(self, input_ids: torch.Tensor, caches: list) -> torch.Tensor:
        """Runs the prompt once, filling `caches`; returns last-position logits (B, vocab)."""
        x = self.embed(input_ids)
        for block, cache in zip(self.blocks, caches):
            x = block.prefill(x, cache)
        return self._head(x[:, -1:])[:, 0]

    @torch.no_grad()
    def decode_step(self, token: torch.Tensor, caches: list, pos, rws=None) -> torch.Tensor:
        """token (B,1) at position `pos`; returns its logits (B, vocab).

        pos: an int, or on GPU a CUDA int64 tensor of one element (see
        GraphDecoder).  rws: optional per-layer (r, w) fp32 tensors."""
        x = self.embed(token, start=pos)
        for i, (block, cache) in enumerate(zip(self.blocks, caches)):
            x = block.decode(x, cache, pos, None if rws is None else rws[i])
        return self._head(x)[:, 0]

    @torch.no_grad()
    def generate_greedy(self, input_ids: torch.Tensor, max_new_tokens: int = 100) -> torch.Tensor:
        """Greedy decoding (the argmax token; among equal logits the first).

        On GPU the per-token decode step runs as one replayed HIP graph
        (GraphDecoder); on CPU it is the eager loop.  Returns
        (B, T + max_new_tokens) token ids.  generate(top_k=1) samples the same
        distribution but breaks exact ties at random, as the reference does."""
        self.eval()
        B, T = input_ids.shape
        if max_new_tokens <= 0:
            return input_ids
        dtype = self.blocks[0].attn.q_proj.weight.dtype
        caches = self.new_cache(B, T + max_new_tokens, dtype, input_ids.device)
        logits = self.prefill(input_ids, caches)
        first = logits.argmax(-1, keepdim=True)
        if not input_ids.is_cuda or max_new_tokens == 1:
            out, tok = [input_ids, first], first
            for step in range(1, max_new_tokens):
                tok = self.decode_step(tok, caches, T + step - 1).argmax(-1, keepdim=True)
                out.append(tok)
            return torch.cat(out, dim=1)
        dec = GraphDecoder(self, caches, first, T, max_new_tokens - 1)
        for _ in range(max_new_tokens - 1):
            dec.step()
        return torch.cat([input_ids, first, dec.tokens], dim=1)

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int = 100, temperature: float = 1.0,
                 top_k: int | None = None) -> torch.Tensor:
        """Temperature / top-k sampling (top_k=1 is greedy).

        Returns (B, T + max_new_tokens) token ids.
        """
        self.eval()
        B, T = input_ids.shape
        if max_new_tokens <= 0:
            return input_ids
        dtype = self.blocks[0].attn.q_proj.weight.dtype
        if input_ids.is_cuda and torch.is_autocast_enabled("cuda"):
            dtype = torch.get_autocast_dtype("cuda")
        caches = self.new_cache(B, T + max_new_tokens, dtype, input_ids.device)
        logits = self.prefill(input_ids, caches)
        out = [input_ids]
        pos = T
        for step in range(max_new_tokens):
            logits = logits / temperature
            if top_k is not None:
                values, _ = torch.topk(logits, top_k)
                logits[logits < values[:, -1:]] = float("-inf")
            probs = F.softmax(logits, dim=-1)
            next_token = torch.multinomial(probs, num_samples=1)
            out.append(next_token)
            if step + 1 < max_new_tokens:
                logits = self.decode_step(next_token, caches, pos)
                pos += 1
        return torch.cat(out, dim=1)


class GraphDecoder:
    """Greedy decode steps of a MultiscreenLM, captured once as a HIP graph and
    replayed per token.

    One step embeds the token in `token` at the position in `pos` (device
    tensors), runs every layer's cache write and single-query decode
    (msa_decode_at reads the position on the device), the final norm and head,
    writes the argmax into `token` and into `tokens[:, n]` (n a device
    counter) and advances `pos` and n.  Every launch depends only on shapes,
    so the captured graph replays unchanged as the sequence grows; r and w of
    every layer are read once here (the model does not change while it
    decodes).  The first step runs eagerly before the capture: it warms the
    allocator and the kernels up, and the step the capture records overwrites
    its cache writes with the same values.
    """

    def __init__(self, lm, caches, token, pos: int, steps: int):
        if not token.is_cuda:
            raise RuntimeError("GraphDecoder needs the model and caches on the GPU")
        cap = caches[0].k.shape[1]
        if pos + steps > cap:
            raise IndexError(f"KV cache capacity {cap} is below {pos + steps} positions")
        dev = token.device
        self.lm, self.caches, self.steps, self.done = lm, caches, steps, 0
        self.token = token.detach().clone()
        self.pos = torch.tensor([pos], dtype=torch.int64, device=dev)
        self.n = torch.zeros(1, dtype=torch.int64, device=dev)
        self.tokens = torch.zeros((token.shape[0], max(steps, 1)), dtype=token.dtype, device=dev)
        with torch.no_grad():
            self.rws = [(b.attn.sharpness().detach().float().contiguous(),
                         b.attn.window().detach().float().contiguous()) for b in lm.blocks]
        # warm-up: one eager step on a side stream, then the state put back
        tok0, pos0 = self.token.clone(), self.pos.clone()
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            self._body()
        torch.cuda.current_stream(dev).wait_stream(side)
        self.token.copy_(tok0)
        self.pos.copy_(pos0)
        self.n.zero_()
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.logits = self._body()

    @torch.no_grad()
    def _body(self):
        logits = self.lm.decode_step(self.token, self.caches, self.pos, self.rws)
        nxt = logits.argmax(-1, keepdim=True)
        self.token.copy_(nxt)
        self.tokens.index_copy_(1, self.n, nxt)
        self.pos.add_(1)
        self.n.add_(1)
        return logits

    def step(self):
        """Decodes one token; returns the (B, 1) token tensor (overwritten by the
        next step) -- its logits are in self.logits."""
        if self.done >= self.steps:
            raise IndexError("GraphDecoder: all planned steps are done")
        self.graph.replay()
        self.done += 1
        return self.token
