#!/usr/bin/env python3
"""Benchmark of the fused Screening Attention hot path on one MI355X.

Workload: one screening-attention layer core,
forward + backward, bf16, B=4, T=8192, H=8, head_dim=64, causal;
q/k/v ~ N(0,1) in the projection layout (B,T,H,D); r_h ~ U[1.9,2.1];
w_h ~ U[256,8192]; dO ~ N(0,1).  A step is one fused forward (msa_fwd) plus
one fused backward (msa_bwd, incl. dr/dw) over that batch, inputs resident in
HBM.  value = tokens/s = B*T / step time.

Also reported:
  roofline      the dominant kernel (by measured time) against its bound
  cpu_baseline  the reference's dense torch-fp32 math on the host cores, on a
                bounded sample, scaled to the same unit
  decode        the T=100K single-query decode kernel (configs[4] shape) in
                GB/s against HBM peak (decode-stream variant: every key in window)
  cfg3_lm_train_step   configs[2]: one MultiscreenLM training step, tokens/s
                       and the attention kernels' share of it
  cfg4_prefill_100k    configs[3]: the T=100,000 prefill forward, with its
                       algorithmic flop C(|W|+|A|) and bf16-peak fraction
  cfg5_decode_literal  configs[4] as written: ms per generated token, eager
                       and replayed from a captured HIP graph (same tokens)
  cfg2_trained_regime  the configs[1] shape with inputs in the regime its
                       text describes (~5% of in-window alpha non-zero)
  cfg2_f16             the headline workload in float16
  ref_fused_module_fwd the reference's own published fused benchmark
                       (module forward, fp32, T = 512..4096) with peak memory
  peak_memory_mb       device memory of one headline step
The supplementary legs run before the headline's warm-up and timed steps.
Prints ONE JSON line.
"""

import argparse
import json
import math
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "pytorch-implementation-of-screening-attention_amd"))

PEAK_BF16_TFLOPS = 2500.0     # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0         # MI355X HBM3E
TILE_FLOP = 2 * 64 * 64 * 64  # one 64x64 tile product with D=64
TIMER_EVERY = 10              # timed-region launches of the dominant kernel: one in 10 carries events
KERNELS = {1: "prep_k_kernel", 2: "fwd_screen_kernel", 3: "fwd_live_kernel", 4: "dkdv_kernel",
           5: "dq_kernel"}   # msa_kernel_id values (include/msa.h)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    # the GPU reaches its steady clocks after about 50 ms of back-to-back
    # steps (the first steps run up to 8% slower): 300 warmup steps are about 60 ms
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=300)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-decode", action="store_true")
    p.add_argument("--no-configs", action="store_true", help="skip the supplementary legs")
    p.add_argument("--legs", default="", help="comma-separated supplementary legs to run (default: all)")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--calib-copy", action="store_true",
                   help="end with one elementwise pass over 2 GiB (rocprofv3 --pmc byte-counter calibration)")
    return p.parse_args()


def cfg2_inputs(seed=0):
    """BASELINE.json configs[1] inputs, drawn on the CPU so every consumer (this
    bench, the full-shape parity test) sees identical values: q, k, v, dO ~
    N(0,1) of shape (B,T,H,D) = (4,8192,8,64) rounded to bf16, r_h ~ U[1.9,2.1],
    w_h ~ U[256,8192] (lists of H floats), all from torch.Generator(seed)."""
    import torch
    B, T, H, D = 4, 8192, 8, 64
    g = torch.Generator().manual_seed(seed)
    r = (1.9 + 0.2 * torch.rand(H, generator=g)).tolist()
    w = (256.0 + (8192.0 - 256.0) * torch.rand(H, generator=g)).tolist()
    q, k, v, dy = (torch.randn(B, T, H, D, generator=g).bfloat16() for _ in range(4))
    return q, k, v, dy, r, w


def trained_regime_inputs(seed=0, n_clusters=18, rho=0.8, B=4, T=8192):
    """The configs[1] shape, r and w with inputs in the regime its text
    describes ("~95% of alpha at zero", the trained-model figure of the
    reference's README.md:33), which i.i.d. N(0,1) inputs do not reach
    (99.99% zero there).  Each (b, t, h) draws one of n_clusters per-head
    centres c; q = rho c + sqrt(1 - rho^2) n_q and k likewise (own noise),
    v, dO ~ N(0,1).  Same-cluster pairs have s near rho^2 = 0.64, above every
    head's threshold 1 - 1/r in [0.47, 0.53] for most pairs, and other pairs
    rarely pass, so about 0.9/18 = 5% of in-window pairs are live and nearly
    every in-window 32x32 unit holds one."""
    import torch
    H, D = 8, 64
    g = torch.Generator().manual_seed(seed)   # r and w as cfg2_inputs draws them
    r = (1.9 + 0.2 * torch.rand(H, generator=g)).tolist()
    w = (256.0 + (8192.0 - 256.0) * torch.rand(H, generator=g)).tolist()
    g = torch.Generator().manual_seed(seed + 1000)
    centres = torch.randn(H, n_clusters, D, generator=g)
    assign = torch.randint(0, n_clusters, (B, T, H), generator=g)
    base = centres[torch.arange(H).view(1, 1, H), assign]
    sig = math.sqrt(1.0 - rho * rho)
    q = (rho * base + sig * torch.randn(B, T, H, D, generator=g)).bfloat16()
    k = (rho * base + sig * torch.randn(B, T, H, D, generator=g)).bfloat16()
    v, dy = (torch.randn(B, T, H, D, generator=g).bfloat16() for _ in range(2))
    return q, k, v, dy, r, w


def window_tiles(T, w_list, tile=64):
    """|W|: causal 64x64 tiles holding a pair with 0 <= i-j < w, per (b,h) summed over heads."""
    n = 0
    nt = (T + tile - 1) // tile
    for w in w_list:
        wc = min(int(math.ceil(w)), 10 ** 9)
        for qt in range(nt):
            q0 = qt * tile
            qlast = min(q0 + tile - 1, T - 1)
            jlo = max(0, q0 - wc + 1)
            n += qlast // tile - jlo // tile + 1
    return n


def live_counts(bits, B, H, T):
    """(live 32x32 units, live 64x64 tiles) from the live-unit bitmap: per
    (b, h), 2*nqt rows of ceil(2*nkt/32) words; a tile is live iff one of its
    four units is."""
    import torch
    nqt = nkt = (T + 63) // 64
    words = (2 * nkt + 31) // 32
    b = (bits.to(torch.int64) & 0xFFFFFFFF)[:B * H * 2 * nqt * words].view(B * H, 2 * nqt, words, 1)
    sh = torch.arange(32, device=bits.device, dtype=torch.int64)
    u = ((b >> sh) & 1).view(B * H, 2 * nqt, words * 32)[:, :, :2 * nkt].bool()
    tiles = u.view(B * H, nqt, 2, nkt, 2).any(dim=4).any(dim=2)
    return int(u.sum()), int(tiles.sum())


def kernel_times(L, kid, fn, n):
    """Average duration (ms) of kernel `kid` over n calls of fn, via HIP events."""
    import ctypes
    assert L.msa_timer_arm(kid, n) == 0
    for _ in range(n):
        fn()
    buf = (ctypes.c_float * n)()
    got = L.msa_timer_read(kid, buf, n)
    L.msa_timer_arm(0, 0)
    vals = [buf[i] for i in range(got)]
    return sum(vals) / max(1, len(vals)), vals


def profiled_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 byte-counter
    summary (FETCH_SIZE + WRITE_SIZE, scaled by the copy-kernel calibration), or
    None when the summary is absent or lacks the kernel."""
    path = os.path.join(HERE, "profiles", "fwd_bwd_cfg2_pmc_bytes.txt")
    try:
        text = open(path).read()
    except OSError:
        return None
    import re
    m = re.search(r"fetch_factor ([\d.]+) write_factor ([\d.]+)", text)
    k = re.search(r"kernel %s\s+fetch_kib\s+([\d.]+) write_kib\s+([\d.]+)" % re.escape(kernel), text)
    if not m or not k:
        return None
    ff, wf = float(m.group(1)), float(m.group(2))
    return int((float(k.group(1)) / ff + float(k.group(2)) / wf) * 1024)


def cpu_baseline(B, T, H, D, r, w, seed):
    """Dense reference math (torch fp32) fwd+bwd on 1 (b,h) slice of the workload."""
    import torch
    sys.path.insert(0, os.path.join(HERE, "oracle"))
    import cpu_torch
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    Ts = T
    g = torch.Generator().manual_seed(seed + 100)
    q, k, v, dy = (torch.randn(1, Ts, 1, D, generator=g).bfloat16().float() for _ in range(4))
    rr, ww = torch.tensor([r[0]]), torch.tensor([w[0]])
    cpu_torch.fwd_bwd(q[:, :512], k[:, :512], v[:, :512], rr, ww, dy[:, :512])  # warm-up
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        cpu_torch.fwd_bwd(q, k, v, rr, ww, dy)
        times.append(time.perf_counter() - t0)
    t = sorted(times)[1]
    # the full workload is B*H independent slices of this size
    full = t * B * H
    return {"value": B * T / full, "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle/cpu_torch.py dense fp32 fwd+bwd of one (b,h) slice, T={Ts}, D={D}, "
                      f"median of 3 = {t:.3f} s, scaled x{B * H} slices to B={B},H={H}",
            "cpu": _cpu_name()}


def _cpu_name():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def decode_bench(L, ops, torch, steps=20):
    """configs[4] attention shape: B=16, cache 100,000 positions, H=8, D=64, bf16.
    Decode-stream variant: w_h = 1e5 for all heads (the whole cache is in window).
    Timed: the whole decode step (partial-sum kernel + reduce/TanhNorm kernel)."""
    B, Tc, H, D = 16, 100000, 8, 64
    g = torch.Generator(device="cuda").manual_seed(5)
    # head-major storage, as multiscreen.attention.KVCache keeps it, viewed (B, Tc, H, D)
    kc = torch.randn(B, H, Tc, D, device="cuda", generator=g).bfloat16().permute(0, 2, 1, 3)
    vc = torch.randn(B, H, Tc, D, device="cuda", generator=g).bfloat16().permute(0, 2, 1, 3)
    q = torch.randn(B, H, D, device="cuda", generator=g).bfloat16()
    r = torch.full((H,), 2.0, device="cuda")
    w = torch.full((H,), 1e5, device="cuda")
    ws = torch.empty(int(L.msa_decode_workspace_bytes(B, H, D, Tc)), dtype=torch.uint8, device="cuda")
    fn = lambda: ops.decode_step(q, kc, vc, Tc, r, w, 1e-8, ws)
    for _ in range(10):  # untimed warm-up (first touches of the 1.6 GB cache)
        fn()
    torch.cuda.synchronize()
    ms, _ = kernel_times(L, 7, fn, steps)
    torch.cuda.synchronize()
    bytes_k = B * H * Tc * D * 2
    # V rows are read only for live keys; count them exactly on the GPU
    qn = torch.nn.functional.normalize(q.float(), dim=-1)
    kn = torch.nn.functional.normalize(kc.float(), dim=-1)
    live = 0
    for b in range(B):
        s = torch.einsum("hd,thd->th", qn[b], kn[b])
        live += int((1.0 - 2.0 * (1.0 - s) > 0).sum())
    bytes_v = live * D * 2
    gbs = (bytes_k + bytes_v) / (ms * 1e-3) / 1e9
    out = {"workload": "decode B=16, cache 100000, H=8, D=64, bf16, w=1e5 (decode-stream variant)",
           "kernel": "decode_partial_kernel+decode_reduce_kernel", "ms": round(ms, 4), "bytes": bytes_k + bytes_v,
           "live_v_rows": live, "GB/s": round(gbs, 1), "frac": round(gbs / PEAK_HBM_GBS, 4)}
    # V rows are read only for live keys, so the fraction is also stated on the
    # bytes the profiler saw the two kernels move (FETCH_SIZE + WRITE_SIZE)
    moved = [profiled_traffic(k) for k in ("decode_partial_kernel", "decode_reduce_kernel")]
    if all(m is not None for m in moved):
        fgbs = sum(moved) / (ms * 1e-3) / 1e9
        out.update({"bytes_profiled": sum(moved), "GB/s_profiled": round(fgbs, 1),
                    "frac_profiled": round(fgbs / PEAK_HBM_GBS, 4),
                    "bytes_source": "profiles/fwd_bwd_cfg2_pmc_bytes.txt"})
    return out


VOCAB = 50257


def zipf_ids(B, T, s, seed):
    """Token ids drawn from a Zipf(s) distribution over the vocabulary, p(k) ~ (k+1)^-s."""
    import torch
    g = torch.Generator().manual_seed(seed)
    p = torch.arange(1, VOCAB + 1, dtype=torch.float64).pow(-s)
    return torch.multinomial((p / p.sum()).float(), B * T, replacement=True, generator=g).view(B, T)


def _kernel_sum_ms(L, fn, ids=(1, 2, 3, 4, 5), per_call=200):
    """Sum of the durations (ms) of the library's kernels launched by one call of fn."""
    import ctypes
    for kid in ids:
        assert L.msa_timer_arm(kid, per_call) == 0
    fn()
    total = 0.0
    buf = (ctypes.c_float * per_call)()
    for kid in ids:
        n = L.msa_timer_read(kid, buf, per_call)
        total += sum(buf[i] for i in range(max(n, 0)))
    L.msa_timer_arm(0, 0)
    return total


def cfg3_bench(L, torch, steps=5, warmup=2):
    """one training step of MultiscreenLM(50257, 512, 8 heads, 6 layers,
    max_seq_len 2048), random init (seed 0), fp32 master weights under bf16 autocast, on 8 x 2048
    Zipf(1.1) ids with labels = ids: forward + loss, backward, clip_grad_norm_(1.0) and AdamW step
    (train.py:96-104).  Attention share: the library's kernels (6 layers, fwd + bwd) over the step."""
    from multiscreen import MultiscreenLM
    torch.manual_seed(0)
    lm = MultiscreenLM(vocab_size=VOCAB, d_model=512, num_heads=8, num_layers=6, max_seq_len=2048).cuda()
    opt = torch.optim.AdamW(lm.parameters(), lr=3e-4, weight_decay=0.1)
    ids = zipf_ids(8, 2048, 1.1, seed=0).cuda()

    def step():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = lm(ids, labels=ids)["loss"]
        opt.zero_grad(set_to_none=True)
        loss.backward()
        torch.nn.utils.clip_grad_norm_(lm.parameters(), 1.0)
        opt.step()
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(steps):
        loss = step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / steps
    attn_ms = _kernel_sum_ms(L, step)
    torch.cuda.synchronize()
    return {"workload": "configs[2]: MultiscreenLM(50257,512,8,6,2048) training step, 8x2048 Zipf(1.1) ids, "
                        "bf16 autocast, AdamW + clip",
            "ms_per_step": round(ms, 3), "tokens_per_s": round(8 * 2048 / (ms * 1e-3), 1),
            "attention_kernels_ms": round(attn_ms, 3), "attention_share": round(attn_ms / ms, 4),
            "loss": round(float(loss.detach()), 4)}


def cfg4_bench(L, ops, torch, reps=5):
    """long-context prefill forward, B=1, T=100,000, H=8, D=64, bf16,
    causal, r=2, w log-uniform in [512, 1e5] (seed 4); q, k, v ~ N(0,1) drawn on the CPU."""
    B, T, H, D = 1, 100000, 8, 64
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(B, T, H, D, generator=g).bfloat16().cuda() for _ in range(3))
    lo, hi = math.log(512.0), math.log(1e5)
    w = torch.exp(lo + (hi - lo) * torch.rand(H, generator=g)).tolist()
    rg, wg = torch.full((H,), 2.0, device="cuda"), torch.tensor(w, device="cuda")
    fn = lambda: ops.fwd_raw(q, k, v, rg, wg, True, 1e-8, None)
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        y, hn, bits = fn()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    screen_ms, _ = kernel_times(L, 2, fn, 3)
    nW = window_tiles(T, w) * B
    nU, nA = live_counts(bits, B, H, T)
    flop = TILE_FLOP * (nW + nA)
    causal_tiles = B * H * ((T + 63) // 64) * ((T + 63) // 64 + 1) // 2
    return {"workload": "configs[3]: prefill forward B=1 T=100000 H=8 D=64 bf16 causal, r=2, w log-U[512,1e5]",
            "w": [round(x, 1) for x in w], "ms": round(ms, 4), "tokens_per_s": round(B * T / (ms * 1e-3), 1),
            "tiles": {"causal": causal_tiles, "window": nW, "active": nA, "active_units_32": nU},
            "flop_alg": flop, "tflops_alg": round(flop / (ms * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(flop / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 5),
            "screen_kernel_ms": round(screen_ms, 4),
            "screen_frac_bf16_peak": round(TILE_FLOP * nW / (screen_ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 5)}


def cfg5_bench(torch, new_tokens=256):
    """BASELINE.json configs[4] as written: MultiscreenLM(50257, 512, 8 heads, 6 layers,
    max_seq_len 100000) at random init (seed 0, so the init windows 2..256 and r = 2), bf16
    weights and bf16 KV caches of 100,000 positions, batch 16, prompts of 100000-256 uniform
    ids (seed 0), prefill then 256 greedy tokens (MultiscreenLM.generate, top_k=1)."""
    from multiscreen import MultiscreenLM
    B, CAP = 16, 100000
    torch.manual_seed(0)
    lm = MultiscreenLM(vocab_size=VOCAB, d_model=512, num_heads=8, num_layers=6,
                       max_seq_len=CAP).to("cuda", torch.bfloat16).eval()
    g = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, VOCAB, (B, CAP - new_tokens), generator=g).cuda()
    caches = lm.new_cache(B, CAP, torch.bfloat16, "cuda")
    with torch.no_grad():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        logits = lm.prefill(prompt, caches)
        torch.cuda.synchronize()
        t_prefill = time.perf_counter() - t0
        tok = logits.argmax(-1, keepdim=True)
        for s in range(4):  # untimed warm-up of the decode path (positions overwritten below)
            lm.decode_step(tok, caches, CAP - new_tokens + s)
        first = tok
        toks = []
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in range(new_tokens - 1):
            logits = lm.decode_step(tok, caches, CAP - new_tokens + s)
            tok = logits.argmax(-1, keepdim=True)
            toks.append(tok)
        torch.cuda.synchronize()
        t_dec = time.perf_counter() - t0
        # the same 255 steps again, each one replay of a captured HIP graph
        # (GraphDecoder: position and token on the device); same caches, same
        # start, so the same tokens
        from multiscreen.model import GraphDecoder
        dec = GraphDecoder(lm, caches, first, CAP - new_tokens, new_tokens - 1)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for s in range(new_tokens - 1):
            dec.step()
        torch.cuda.synchronize()
        t_graph = time.perf_counter() - t0
        same = bool(torch.equal(dec.tokens, torch.cat(toks, dim=1)))
    return {"workload": "configs[4]: MultiscreenLM 6 layers, B=16, bf16 KV cache 100000, init windows, "
                        "prefill + 256 greedy tokens",
            "prefill_s": round(t_prefill, 4), "ms_per_token": round(t_dec / (new_tokens - 1) * 1e3, 4),
            "tokens_per_s": round(B * (new_tokens - 1) / t_dec, 1),
            "ms_per_token_graph": round(t_graph / (new_tokens - 1) * 1e3, 4),
            "tokens_per_s_graph": round(B * (new_tokens - 1) / t_graph, 1),
            "graph_tokens_equal_eager": same,
            "note": "ms_per_token: eager decode_step per token (launch-bound: about 120 kernel launches); "
                    "ms_per_token_graph: the same steps replayed from one captured HIP graph"}


def live_pair_fraction(q, k, r, w, torch, rows=256, seed=0):
    """Fraction of in-window causal pairs with alpha > 0, on `rows` sampled
    queries per (b, h) of batch row 0 (every key of their windows), in fp32
    from the rounded inputs."""
    B, T, H, D = q.shape
    g = torch.Generator(device=q.device).manual_seed(seed)
    live = tot = 0
    for h in range(H):
        wc = int(math.ceil(w[h]))
        idx = torch.randint(0, T, (rows,), device=q.device, generator=g)
        qn = torch.nn.functional.normalize(q[0, idx, h].float(), dim=-1)
        kn = torch.nn.functional.normalize(k[0, :, h].float(), dim=-1)
        s = qn @ kn.T                                             # (rows, T)
        d = idx.view(-1, 1) - torch.arange(T, device=q.device).view(1, -1)
        inside = (d >= 0) & (d < wc)
        live += int(((s > 1.0 - 1.0 / r[h]) & inside).sum())
        tot += int(inside.sum())
    return live / max(tot, 1)


def step_legs(L, ops, torch, q, k, v, dy, r, w, reps=10):
    """fwd+bwd step time (events, after 3 untimed steps), per-kernel event
    times, tile counts and algorithmic rates of one cfg2-shaped workload."""
    dev = q.device
    rg, wg = torch.tensor(r, device=dev), torch.tensor(w, device=dev)
    B, T, H, D = q.shape

    def step():
        y, hnorm, bits = ops.fwd_raw(q, k, v, rg, wg, True, 1e-8, None)
        ops.bwd_raw(q, k, v, rg, wg, True, 1e-8, y, hnorm, bits, dy)
        return bits
    for _ in range(3):
        bits = step()
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for _ in range(reps):
        bits = step()
    t1.record()
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    per_kernel = {name: round(kernel_times(L, kid, step, 3)[0], 4) for kid, name in KERNELS.items()}
    nW = window_tiles(T, w) * B
    nU, nA = live_counts(bits, B, H, T)
    f_total = TILE_FLOP * (nW + 6 * nA)
    unit_flop = {"fwd_live_kernel": TILE_FLOP * nA, "dq_kernel": TILE_FLOP * nA, "dkdv_kernel": 4 * TILE_FLOP * nA}
    return {"ms_per_step": round(ms, 4), "tokens_per_s": round(B * T / (ms * 1e-3), 1),
            "kernel_ms_event": per_kernel,
            "tiles": {"window": nW, "active": nA, "active_units_32": nU,
                      "active_frac_of_window": round(nA / max(nW, 1), 4)},
            "flop_alg": f_total, "tflops_alg": round(f_total / (ms * 1e-3) / 1e12, 2),
            "frac_bf16_peak": round(f_total / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 5),
            "unit_kernels_frac_bf16_peak": {
                k_: round(f / (per_kernel[k_] * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 5)
                for k_, f in unit_flop.items()}}


def trained_regime_bench(L, ops, torch):
    """configs[1] shape, r, w and dtype with the trained-regime inputs of
    trained_regime_inputs (about 5% of in-window alpha non-zero)."""
    q, k, v, dy, r, w = (t.cuda() if hasattr(t, "cuda") else t for t in trained_regime_inputs(0))
    out = {"workload": "configs[1] shape (B=4 T=8192 H=8 D=64 bf16 causal, its r and w) with clustered q/k "
                       "(18 centres per head, rho 0.8): the regime configs[1] describes, ~5% of in-window "
                       "alpha non-zero",
           "live_pair_frac_of_window": round(live_pair_fraction(q, k, r, w, torch), 4)}
    out.update(step_legs(L, ops, torch, q, k, v, dy, r, w))
    return out


def fp16_bench(L, ops, torch, q, k, v, dy, r, w):
    """The headline workload with the same inputs in float16 (torch.autocast's
    CUDA dtype, the reference's fused dtype, screening_fwd.py:235)."""
    out = {"workload": "configs[1] inputs cast to float16 (v_mfma_f32_32x32x16_f16)"}
    out.update(step_legs(L, ops, torch, *(t.half() for t in (q, k, v, dy)), r, w))
    return out


# The reference's published fused-path numbers (BENCHMARK_REPORT_TRITON.md:61-85,
# RTX 4060 Ti, triton-windows): module forward latency (final column) and peak
# memory, forward only (eval) and forward + backward (training).
REF_TRITON_FWD_MS = {512: 0.681, 1024: 1.389, 2048: 2.825, 4096: 5.858}
REF_TRITON_FWD_MB = {512: 52.6, 1024: 88.2, 2048: 159.5, 4096: 302.1}
REF_TRITON_FWDBWD_MB = {512: 98.2, 1024: 168.8, 2048: 303.8}


def ref_module_bench(torch, reps=20):
    """The reference's own fused-path benchmark (benchmarks/bench_triton.py:19-60):
    ScreeningAttention(512, 8 heads, causal) forward of the whole module in
    fp32 on x ~ N(0,1) of shape (4, T, 512), s_r = -2 (r = 1.135), default
    windows; latency (median of `reps` event-timed calls after warm-up) and
    torch.cuda.max_memory_allocated for the forward (eval, no_grad) and for
    forward + backward (train).  The reference measures in a process of its
    own; here the other legs' tensors are resident, so their bytes (allocated
    before this leg starts) are subtracted from each peak."""
    from multiscreen import ScreeningAttention
    held = torch.cuda.memory_allocated()
    torch.manual_seed(0)
    m = ScreeningAttention(512, num_heads=8, causal=True).cuda()
    with torch.no_grad():
        m.s_r.fill_(-2.0)
    rows = []
    for T in (512, 1024, 2048, 4096):
        x = torch.randn(4, T, 512, device="cuda")
        m.eval()
        with torch.no_grad():
            for _ in range(3):
                m(x, x, x)
            torch.cuda.synchronize()
            times = []
            for _ in range(reps):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                m(x, x, x)
                b.record()
                torch.cuda.synchronize()
                times.append(a.elapsed_time(b))
            torch.cuda.reset_peak_memory_stats()
            m(x, x, x)
            torch.cuda.synchronize()
            mem_fwd = (torch.cuda.max_memory_allocated() - held) / 1e6
        m.train()
        xg = x.clone().requires_grad_()
        torch.cuda.reset_peak_memory_stats()
        m(xg, xg, xg).sum().backward()
        torch.cuda.synchronize()
        mem_fb = (torch.cuda.max_memory_allocated() - held) / 1e6
        m.zero_grad(set_to_none=True)
        ms = sorted(times)[len(times) // 2]
        row = {"T": T, "fwd_ms": round(ms, 4), "fwd_peak_mb": round(mem_fwd, 1), "fwd_bwd_peak_mb": round(mem_fb, 1),
               "ref_triton_fwd_ms": REF_TRITON_FWD_MS.get(T), "ref_triton_fwd_peak_mb": REF_TRITON_FWD_MB.get(T),
               "ref_triton_fwd_bwd_peak_mb": REF_TRITON_FWDBWD_MB.get(T)}
        row["fwd_speedup_vs_ref_published"] = round(REF_TRITON_FWD_MS[T] / ms, 2)
        rows.append(row)
        del x, xg
    torch.cuda.empty_cache()
    return {"workload": "reference benchmarks/bench_triton.py: ScreeningAttention(512, 8, causal) module forward, "
                        "fp32, B=4, s_r=-2 (r=1.135), default windows",
            "ref_hardware": "RTX 4060 Ti (BENCHMARK_REPORT_TRITON.md:61-85; a different GPU)",
            "peak_mb_note": f"max_memory_allocated minus the {held / 1e6:.1f} MB the other legs hold",
            "rows": rows}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (every box here has one); --gpus {args.gpus} "
              "is not supported", file=sys.stderr)
        sys.exit(2)
    import torch
    from multiscreen import _native, ops
    L = _native.lib()
    torch.manual_seed(args.seed)
    dev = torch.device("cuda:0")

    q, k, v, dy, r, w = cfg2_inputs(args.seed)
    B, T, H, D = q.shape
    q, k, v, dy = (t.to(dev) for t in (q, k, v, dy))
    rg = torch.tensor(r, device=dev)
    wg = torch.tensor(w, device=dev)

    def step():
        y, hnorm, bits = ops.fwd_raw(q, k, v, rg, wg, True, 1e-8, None)
        grads = ops.bwd_raw(q, k, v, rg, wg, True, 1e-8, y, hnorm, bits, dy)
        return bits

    # The supplementary legs run first: a few seconds of GPU work, after which
    # the headline below runs at the clocks the GPU holds under sustained
    # work (from a cold start the first ~50 ms of steps run up to 8% slower).
    # The headline's own warm-up is still exactly `warmup` steps.  The
    # HBM-bound decode stream runs after light legs and before the fp16 step
    # leg, so that the headline follows MFMA-heavy work (measured on one box:
    # headline 1.3% faster than after the decode leg, decode unchanged).
    extra = {}
    legs = (("cfg3_lm_train_step", lambda: cfg3_bench(L, torch)),
            ("cfg4_prefill_100k", lambda: cfg4_bench(L, ops, torch)),
            ("cfg5_decode_literal", lambda: cfg5_bench(torch)),
            ("cfg2_trained_regime", lambda: trained_regime_bench(L, ops, torch)),
            ("ref_fused_module_fwd", lambda: ref_module_bench(torch)),
            ("decode", lambda: decode_bench(L, ops, torch)),
            ("cfg2_f16", lambda: fp16_bench(L, ops, torch, q, k, v, dy, r, w)))
    only = set(x for x in args.legs.split(",") if x)
    for key, leg in legs:
        if key == "decode" and args.no_decode:
            continue
        if key != "decode" and (args.no_configs or (only and key not in only)):
            continue
        try:
            extra[key] = leg()
        except Exception as e:  # reported in the line, not hidden
            if key == "decode":
                raise
            extra[key] = {"error": f"{type(e).__name__}: {e}"}
        torch.cuda.empty_cache()

    for _ in range(args.warmup):
        bits = step()
    torch.cuda.synchronize()
    # peak device memory of one step (inputs resident; outputs, workspaces,
    # bitmap and gradients allocated by the step)
    torch.cuda.reset_peak_memory_stats()
    base_mb = torch.cuda.memory_allocated() / 1e6
    step()
    torch.cuda.synchronize()
    peak_mb = torch.cuda.max_memory_allocated() / 1e6

    # per-kernel breakdown (HIP events around each launch, outside the timed
    # region) picks the dominant kernel; its launches are then timed again
    # inside the timed region
    breakdown = {name: kernel_times(L, kid, step, 5)[0] for kid, name in KERNELS.items()}
    torch.cuda.synchronize()
    dom = max(breakdown, key=breakdown.get)
    dom_id = {name: kid for kid, name in KERNELS.items()}[dom]

    # timed region: exactly `steps` steps, synchronised on both sides; the
    # dominant kernel's launches in one step of TIMER_EVERY are bracketed by HIP
    # events on its stream (each event pair adds a few microseconds of stream
    # time, so they are not put on every step)
    import ctypes
    n_timed = (args.steps + TIMER_EVERY - 1) // TIMER_EVERY
    assert L.msa_timer_arm_every(dom_id, n_timed, TIMER_EVERY) == 0
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t0.record()
    for _ in range(args.steps):
        bits = step()
    t1.record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = t0.elapsed_time(t1) / args.steps
    buf = (ctypes.c_float * n_timed)()
    n = L.msa_timer_read(dom_id, buf, n_timed)
    L.msa_timer_arm(0, 0)
    dom_ms = sum(buf[i] for i in range(n)) / max(1, n)

    nW = window_tiles(T, w) * B
    nU, nA = live_counts(bits, B, H, T)
    # canonical algorithmic work on the 64x64 tile grid, C = 2*64*64*D per
    # tile: fwd+bwd = C (|W| + 6 |A|).  Per kernel: the screen Q K^T over W;
    # alpha V over A; the backward's S recompute, dP, dV, dK in dkdv and dQ in
    # dq over A.  (The kernels themselves visit only the live 32x32 units, nU.)
    f_total = TILE_FLOP * (nW + 6 * nA)
    alg_flop = {"fwd_screen_kernel": TILE_FLOP * nW, "fwd_live_kernel": TILE_FLOP * nA,
                "dkdv_kernel": TILE_FLOP * 4 * nA, "dq_kernel": TILE_FLOP * nA}
    dom_flop = alg_flop.get(dom)
    achieved = dom_flop / (dom_ms * 1e-3) / 1e12 if dom_flop else None
    tokens_s = B * T / (ms_step * 1e-3)
    step_tflops = f_total / (ms_step * 1e-3) / 1e12

    out = {
        "metric": "screening-attn fwd+bwd tokens/s at T=8K (% bf16 MFMA peak); T=100K decode GB/s",
        "value": round(tokens_s, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) q/k/v/dO; r~U[1.9,2.1], w~U[256,8192])",
        "config": {"workload": "configs[1]: screening-attention core fwd+bwd, B=4 T=8192 H=8 D=64 causal",
                   "global_batch": B, "seq_len": T, "heads": H, "head_dim": D,
                   "r": [round(x, 4) for x in r], "w": [round(x, 1) for x in w]},
        "roofline": {"bound": "mfma", "kernel": dom, "kernel_ms": round(dom_ms, 4),
                     "kernel_ms_launches": n, "kernel_ms_every": TIMER_EVERY,
                     "achieved": round(achieved, 2) if achieved else None,
                     "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_BF16_TFLOPS, 5) if achieved else None,
                     "traffic": profiled_traffic(dom),
                     "traffic_source": "profiles/fwd_bwd_cfg2_pmc_bytes.txt",
                     "flop_per_launch": dom_flop},
        "tiles": {"causal": B * H * (T // 64) * (T // 64 + 1) // 2, "window": nW, "active": nA,
                  "active_units_32": nU,
                  "window_skip": round(1 - nW / (B * H * (T // 64) * (T // 64 + 1) / 2), 4),
                  "threshold_skip": round(1 - nA / nW, 5)},
        "step_tflops_alg": round(step_tflops, 2),
        "step_frac_bf16_peak": round(step_tflops / PEAK_BF16_TFLOPS, 5),
        "kernel_ms_event": {k_: round(v_, 4) for k_, v_ in breakdown.items()},
        "kernel_ms_note": "HIP events around each launch, outside the timed region: each includes its "
                          "launch gap (about 1-3 us), so they sum past ms_per_step; profiles/ has the "
                          "rocprofv3 durations",
        "wall_s_timed": round(wall, 3),
        "peak_memory_mb": {"step": round(peak_mb, 1), "inputs_resident": round(base_mb, 1),
                           "note": "torch.cuda.max_memory_allocated over one fwd+bwd step; inputs_resident "
                                   "is q, k, v, dO and r, w before it"},
    }
    out.update(extra)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(B, T, H, D, r, w, args.seed)
    if args.calib_copy:
        # one elementwise pass of known traffic (reads and writes 2 GiB of fp32,
        # well past the 256 MB last-level cache), for scaling the byte counters
        src = torch.ones(512 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        out["calib_copy_bytes"] = src.numel() * 4
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
