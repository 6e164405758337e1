"""CPU oracle for the fused Screening Attention path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker (or the timed CPU baseline), never as a
code path of the product.

A float64 numpy restatement of the reference's dense algorithm,
/root/reference/multiscreen/attention.py and norm.py:

  normalize       attention.py:155-158  x / max(|x|, eps)   (F.normalize)
  similarity      attention.py:160-161  s = q^ k^T
  trim-and-square attention.py:75-90    relu(1 - r(1-s))^2
  softmask        attention.py:92-119   causal:  (cos(pi(j-i)/w)+1)/2 on -w<j-i<=0
                  attention.py:174-183  non-causal: same on |j-i| < w
  key padding     attention.py:185-188  alpha[b,:,:,j] = 0 where mask
  dropout         attention.py:190      alpha*m * keep/(1-p), keep from the
                                        counter-based hash of include/msa.h
  aggregate       attention.py:192-193  h = alpha v^   (no normaliser)
  TanhNorm        norm.py:23-25         tanh(n)/n h,  n = max(|h|, eps)
  per-head params attention.py:164-165  w = exp(s_v)+1, r = exp(s_r)+1

plus the analytic backward of the same map (the reference leaves it to torch
autograd; its fused Triton backward states the normalised-operand formulas in
screening_bwd.py:6-18 and drops dr/dw, attention_triton.py:44).

Tensor convention: q (B,Tq,H,D), k/v (B,Tk,H,D) -- the raw projections as the
(B,T,H,D) view of attention.py:150-151 -- and r, w (H,).  Query rows are
processed in blocks so memory stays O(block * Tk) at any length.

Pinning (tests/test_oracle.py): closed-form known answers (one-hot q=k, the
head-0 init window w=2, below-threshold zeros, TanhNorm properties), a
pure-Python per-pair brute force on tiny inputs, central finite differences
for every gradient, torch.autograd of an independent torch restatement, and
the golden vectors written from the reference module (tests/golden/).
"""

import math

import numpy as np

EPS = 1e-8


def normalize(x, eps=EPS):
    """x / max(|x|, eps) over the last axis (F.normalize, attention.py:156-158)."""
    n = np.sqrt(np.sum(x * x, axis=-1, keepdims=True))
    return x / np.maximum(n, eps)


def trim_and_square(s, r):
    """relu(1 - r(1-s))^2 (attention.py:75-90); r broadcasts against s."""
    a = np.maximum(1.0 - r * (1.0 - s), 0.0)
    return a * a


def softmask(qpos, kpos, w, causal):
    """(H, len(qpos), len(kpos)) window-cut cosine mask (attention.py:92-119, :174-183)."""
    rel = (kpos[None, :] - qpos[:, None]).astype(np.float64)[None]   # j - i
    w = np.asarray(w, dtype=np.float64).reshape(-1, 1, 1)
    m = 0.5 * (np.cos(math.pi * rel / w) + 1.0)
    inside = ((rel > -w) & (rel <= 0)) if causal else (np.abs(rel) < w)
    return m * inside


def softmask_dw(qpos, kpos, w, causal):
    """d softmask / d w on in-window pairs (0 elsewhere)."""
    rel = (kpos[None, :] - qpos[:, None]).astype(np.float64)[None]
    w = np.asarray(w, dtype=np.float64).reshape(-1, 1, 1)
    d = 0.5 * np.sin(math.pi * rel / w) * math.pi * rel / (w * w)
    inside = ((rel > -w) & (rel <= 0)) if causal else (np.abs(rel) < w)
    return d * inside


_M64 = (1 << 64) - 1
_PHI, _MIX1, _MIX2 = 0x9E3779B97F4A7C15, 0xBF58476D1CE4E5B9, 0x94D049BB133111EB


def dropout_keep_bits(seed, bh, i, j):
    """Top 32 bits of the SplitMix64 finaliser (Steele, Lea and Flood, OOPSLA
    2014) of seed + key * 0x9E3779B97F4A7C15 mod 2^64, key = bh << 44 | i << 22
    | j -- the counter-based dropout hash that include/msa.h defines.  Array
    arguments broadcast (numpy uint64, wrapping)."""
    bh, i, j = (np.asarray(x, dtype=np.uint64) for x in (bh, i, j))
    with np.errstate(over="ignore"):   # arithmetic mod 2^64 is the definition
        key = (bh << np.uint64(44)) | (i << np.uint64(22)) | j
        z = np.uint64(seed & _M64) + key * np.uint64(_PHI)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(_MIX1)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(_MIX2)
        z = z ^ (z >> np.uint64(31))
    return (z >> np.uint64(32)).astype(np.uint64)


def dropout_threshold(p):
    """Keep threshold min(floor(p * 2^32), 2^32 - 1) of the fp32 probability p."""
    return min(math.floor(float(np.float32(p)) * 4294967296.0), 4294967295)


def dropout_scale(p):
    """1/(1-p) as the kernels form it, in fp32."""
    return float(np.float32(1.0) / (np.float32(1.0) - np.float32(p)))


def dropout_factor(dropout, B, H, qpos, kpos):
    """(B,H,len(qpos),len(kpos)) float64: 0 for dropped pairs, 1/(1-p) for kept
    ones (attention.py:190, nn.Dropout in training mode), for dropout = (p,
    seed); None when dropout is None or p = 0."""
    if dropout is None or float(dropout[0]) == 0.0:
        return None
    p, seed = dropout
    bh = (np.arange(B)[:, None] * H + np.arange(H)[None, :]).reshape(B, H, 1, 1)
    bits = dropout_keep_bits(seed, bh, np.asarray(qpos).reshape(1, 1, -1, 1), np.asarray(kpos).reshape(1, 1, 1, -1))
    return np.where(bits >= np.uint64(dropout_threshold(p)), dropout_scale(p), 0.0)


def _heads(x):
    """(B,T,H,D) -> (B,H,T,D) float64."""
    return np.ascontiguousarray(np.transpose(np.asarray(x, dtype=np.float64), (0, 2, 1, 3)))


def _blocks(T, block):
    for i0 in range(0, T, block):
        yield i0, min(T, i0 + block)


def forward(q, k, v, r, w, causal=True, eps=EPS, key_padding_mask=None, block=256,
            q_offset=0, return_h=False, dropout=None):
    """TanhNorm'd attention output y (B,Tq,H,D); optionally also h (B,H,Tq,D).

    Query row t sits at position q_offset + t (0 in the reference forward).
    dropout = (p, seed): alpha*m times dropout_factor (attention.py:190).
    """
    qn, kn, vn = normalize(_heads(q), eps), normalize(_heads(k), eps), normalize(_heads(v), eps)
    B, H, Tq, D = qn.shape
    Tk = kn.shape[2]
    r = np.asarray(r, dtype=np.float64).reshape(1, H, 1, 1)
    kpos = np.arange(Tk)
    h = np.zeros((B, H, Tq, D))
    for i0, i1 in _blocks(Tq, block):
        s = qn[:, :, i0:i1] @ np.swapaxes(kn, -1, -2)
        p = trim_and_square(s, r) * softmask(np.arange(i0, i1) + q_offset, kpos, w, causal)[None]
        if key_padding_mask is not None:
            p = p * (~np.asarray(key_padding_mask, dtype=bool))[:, None, None, :]
        c = dropout_factor(dropout, B, H, np.arange(i0, i1) + q_offset, kpos)
        if c is not None:
            p = p * c
        h[:, :, i0:i1] = p @ vn
    n = np.sqrt(np.sum(h * h, axis=-1, keepdims=True))
    nc = np.maximum(n, eps)
    y = np.tanh(nc) / nc * h
    y = np.transpose(y, (0, 2, 1, 3))
    return (y, h) if return_h else y


def _tanhnorm_g(n):
    """G(n) = F'(n)/n, F(n) = tanh(n)/n; series where the closed form cancels."""
    n = np.asarray(n, dtype=np.float64)
    small = n < 1e-2
    ns = np.where(small, 1.0, n)
    t = np.tanh(ns)
    closed = ((1.0 - t * t) / ns - t / (ns * ns)) / ns
    n2 = n * n
    series = -2.0 / 3.0 + n2 * (8.0 / 15.0 + n2 * (-34.0 / 105.0 + n2 * (496.0 / 2835.0)))
    return np.where(small, series, closed)


def _normalize_bwd(x, dxn, eps):
    """Gradient of x -> x/max(|x|,eps) (F.normalize) for upstream dxn."""
    n = np.sqrt(np.sum(x * x, axis=-1, keepdims=True))
    xn = x / np.maximum(n, eps)
    proj = np.sum(xn * dxn, axis=-1, keepdims=True)
    big = n > eps
    return np.where(big, (dxn - xn * proj) / np.maximum(n, eps), dxn / eps)


def backward(q, k, v, r, w, dy, causal=True, eps=EPS, key_padding_mask=None, block=256, dropout=None):
    """Gradients (dq, dk, dv, dr, dw) of sum(y * dy) for y = forward(...)."""
    qh, kh, vh = _heads(q), _heads(k), _heads(v)
    qn, kn, vn = normalize(qh, eps), normalize(kh, eps), normalize(vh, eps)
    B, H, Tq, D = qn.shape
    Tk = kn.shape[2]
    r1 = np.asarray(r, dtype=np.float64).reshape(1, H, 1, 1)
    kpos = np.arange(Tk)
    keep = None
    if key_padding_mask is not None:
        keep = (~np.asarray(key_padding_mask, dtype=bool))[:, None, None, :]

    _, h = forward(q, k, v, r, w, causal, eps, key_padding_mask, block, return_h=True, dropout=dropout)
    g = _heads(dy)
    # TanhNorm backward (norm.py:24-25 with the clamp at eps)
    n = np.sqrt(np.sum(h * h, axis=-1, keepdims=True))
    big = n > eps
    nc = np.maximum(n, eps)
    F = np.tanh(nc) / nc
    G = _tanhnorm_g(nc)
    hd = np.sum(h * g, axis=-1, keepdims=True)
    dh = np.where(big, F * g + G * hd * h, (math.tanh(eps) / eps) * g)

    dqn = np.zeros_like(qn)
    dkn = np.zeros_like(kn)
    dvn = np.zeros_like(vn)
    dr = np.zeros(H)
    dw = np.zeros(H)
    for i0, i1 in _blocks(Tq, block):
        qpos = np.arange(i0, i1)
        s = qn[:, :, i0:i1] @ np.swapaxes(kn, -1, -2)
        a = np.maximum(1.0 - r1 * (1.0 - s), 0.0)
        m = softmask(qpos, kpos, w, causal)[None]
        mdw = softmask_dw(qpos, kpos, w, causal)[None]
        if keep is not None:
            m = m * keep
            mdw = mdw * keep
        c = dropout_factor(dropout, B, H, qpos, kpos)
        if c is not None:   # every term is linear in the mask factor
            m = m * c
            mdw = mdw * c
        p = a * a * m
        dP = dh[:, :, i0:i1] @ np.swapaxes(vn, -1, -2)
        dvn += np.swapaxes(p, -1, -2) @ dh[:, :, i0:i1]
        ds = 2.0 * a * r1 * m * dP                     # a = 0 where the relu is off
        dqn[:, :, i0:i1] = ds @ kn
        dkn += np.swapaxes(ds, -1, -2) @ qn[:, :, i0:i1]
        dr += np.sum(-2.0 * a * (1.0 - s) * m * dP, axis=(0, 2, 3))
        dw += np.sum(a * a * mdw * dP, axis=(0, 2, 3))
    dq = _normalize_bwd(qh, dqn, eps)
    dk = _normalize_bwd(kh, dkn, eps)
    dv = _normalize_bwd(vh, dvn, eps)
    t = lambda x: np.transpose(x, (0, 2, 1, 3))
    return t(dq), t(dk), t(dv), dr, dw


def _keep_bits_int(seed, bh, i, j):
    """dropout_keep_bits with Python integers (an independent restatement)."""
    z = (seed + ((bh << 44) | (i << 22) | j) * _PHI) & _M64
    z = ((z ^ (z >> 30)) * _MIX1) & _M64
    z = ((z ^ (z >> 27)) * _MIX2) & _M64
    return (z ^ (z >> 31)) >> 32


def brute_force_forward(q, k, v, r, w, causal=True, eps=EPS, key_padding_mask=None, dropout=None):
    """Pure-Python per-pair loops; tiny inputs only.  Same contract as forward()."""
    q, k, v = (np.asarray(x, dtype=np.float64) for x in (q, k, v))
    B, Tq, H, D = q.shape
    Tk = k.shape[1]
    y = np.zeros((B, Tq, H, D))

    def unit(x):
        n = math.sqrt(sum(float(e) * float(e) for e in x))
        return [float(e) / max(n, eps) for e in x]

    for b in range(B):
        for hh in range(H):
            ks = [unit(k[b, j, hh]) for j in range(Tk)]
            vs = [unit(v[b, j, hh]) for j in range(Tk)]
            for i in range(Tq):
                qi = unit(q[b, i, hh])
                acc = [0.0] * D
                for j in range(Tk):
                    if key_padding_mask is not None and key_padding_mask[b][j]:
                        continue
                    rel = j - i
                    ww = float(w[hh])
                    inside = (-ww < rel <= 0) if causal else (abs(rel) < ww)
                    if not inside:
                        continue
                    s = sum(qi[e] * ks[j][e] for e in range(D))
                    a = max(1.0 - float(r[hh]) * (1.0 - s), 0.0)
                    wt = a * a * 0.5 * (math.cos(math.pi * rel / ww) + 1.0)
                    if dropout is not None and float(dropout[0]) > 0.0:
                        kept = _keep_bits_int(int(dropout[1]), b * H + hh, i, j) >= dropout_threshold(dropout[0])
                        wt *= dropout_scale(dropout[0]) if kept else 0.0
                    for e in range(D):
                        acc[e] += wt * vs[j][e]
                n = max(math.sqrt(sum(e * e for e in acc)), eps)
                f = math.tanh(n) / n
                for e in range(D):
                    y[b, i, hh, e] = f * acc[e]
    return y


def rows_forward(q, k, v, r, w, rows, causal=True, eps=EPS):
    """y at the listed query rows only (B,len(rows),H,D): O(len(rows)*Tk*D).

    For lengths where a full oracle pass is too slow (e.g. T = 100,000)."""
    q = np.asarray(q)[:, rows]
    return _rows(q, k, v, r, w, np.asarray(rows), causal, eps)


def _rows(qsel, k, v, r, w, qpos, causal, eps):
    qn, kn, vn = normalize(_heads(qsel), eps), normalize(_heads(k), eps), normalize(_heads(v), eps)
    B, H, R, D = qn.shape
    Tk = kn.shape[2]
    rr = np.asarray(r, dtype=np.float64).reshape(1, H, 1, 1)
    h = np.zeros((B, H, R, D))
    wmax = float(np.max(w))
    for t, i in enumerate(qpos):
        lo = 0 if not math.isfinite(wmax) else max(0, int(i - math.ceil(wmax)))
        hi = Tk if not causal else min(Tk, int(i) + 1)
        if not causal:
            hi = Tk if not math.isfinite(wmax) else min(Tk, int(i + math.ceil(wmax)) + 1)
        kp = np.arange(lo, hi)
        s = qn[:, :, t:t + 1] @ np.swapaxes(kn[:, :, lo:hi], -1, -2)
        p = trim_and_square(s, rr) * softmask(np.array([i]), kp, w, causal)[None]
        h[:, :, t:t + 1] = p @ vn[:, :, lo:hi]
    n = np.maximum(np.sqrt(np.sum(h * h, axis=-1, keepdims=True)), eps)
    return np.transpose(np.tanh(n) / n * h, (0, 2, 1, 3))


def decode_row(q_new, kcache, vcache, cache_len, r, w, eps=EPS):
    """Decode output (B,H,D) of the token at position cache_len-1 whose query
    projection is q_new (B,H,D), against raw caches (B,T,H,D): row
    cache_len-1 of forward() over the prefix (model.py:133 keeps only it)."""
    q = np.asarray(q_new, dtype=np.float64)[:, None]
    pos = cache_len - 1
    y = _rows(q, np.asarray(kcache)[:, :cache_len], np.asarray(vcache)[:, :cache_len], r, w,
              np.array([pos]), True, eps)
    return y[:, 0]


def tile_counts(q, k, r, w, causal=True, eps=EPS, tile=64, key_padding_mask=None, block=512):
    """(|W|, |A|, active) over all heads: W = tile x tile blocks (64 or 32)
    holding an in-window pair; A = blocks holding an in-window, unmasked pair
    with 1 - r(1-s) > 0.  `active` is the (B,H,nqt,nkt) bool map of A."""
    qn, kn = normalize(_heads(q), eps), normalize(_heads(k), eps)
    B, H, Tq, D = qn.shape
    Tk = kn.shape[2]
    rr = np.asarray(r, dtype=np.float64).reshape(1, H, 1, 1)
    nqt, nkt = -(-Tq // tile), -(-Tk // tile)
    block = max(tile, block // tile * tile)
    win = np.zeros((B, H, nqt, nkt), dtype=bool)
    act = np.zeros((B, H, nqt, nkt), dtype=bool)
    kpos = np.arange(Tk)
    wv = np.asarray(w, dtype=np.float64).reshape(-1, 1, 1)
    for i0, i1 in _blocks(Tq, block):
        s = qn[:, :, i0:i1] @ np.swapaxes(kn, -1, -2)
        rel = (kpos[None, :] - np.arange(i0, i1)[:, None]).astype(np.float64)[None]
        inside = ((rel > -wv) & (rel <= 0)) if causal else (np.abs(rel) < wv)
        live = (1.0 - rr * (1.0 - s) > 0) & inside[None]
        if key_padding_mask is not None:
            live = live & (~np.asarray(key_padding_mask, dtype=bool))[:, None, None, :]
        inside = np.broadcast_to(inside[None], live.shape)
        pq, pk = -(i1 - i0) % tile, nkt * tile - Tk
        def tiles(x):
            x = np.pad(x, ((0, 0), (0, 0), (0, pq), (0, pk)))
            b_, h_, tq, tk = x.shape
            return x.reshape(b_, h_, tq // tile, tile, tk // tile, tile).any(axis=(3, 5))
        q0 = i0 // tile
        win[:, :, q0:q0 + -(-(i1 - i0) // tile)] |= tiles(inside)
        act[:, :, q0:q0 + -(-(i1 - i0) // tile)] |= tiles(live)
    return int(win.sum()), int(act.sum()), act


# ---------------------------------------------------------------------------
# Live-pair form, for full-size checks (e.g. B=4, T=8192 or T=100,000).
#
# alpha_ij = relu(1 - r(1 - s_ij))^2 is zero unless s_ij > 1 - 1/r
# (attention.py:75-90), and at the benchmark shapes almost every pair is
# below that threshold.  live_pairs() lists the pairs that pass, and
# sparse_forward_backward() evaluates forward() and backward() over exactly
# those pairs in float64, so its outputs are those of the dense functions
# (sums in a different order) at a cost linear in the number of live pairs.
# ---------------------------------------------------------------------------

# Candidate margin of the float32 screening pass.  Each unit vector is
# rounded to float32 (relative error 2^-24 per component) and the 64-term
# dot product accumulates in float32, so |s32 - s| <= (D + 2) * 2^-24 *
# sum_d |q^_d k^_d| <= 130 * 6e-8 < 1e-5 for D <= 128 (sum_d |q^_d k^_d| <= 1
# for unit vectors).  A margin of 1e-4 therefore keeps every pair whose exact
# s passes; the exact float64 test then decides.
SCREEN_MARGIN = 1e-4


def live_pairs(q, k, r, w, causal=True, eps=EPS, key_padding_mask=None, block=1024):
    """Every in-window, unmasked pair (b, h, i, j) with 1 - r_h(1 - s_ij) > 0.

    Returns a dict of equal-length arrays: b, h, i, j (int64) and s (float64,
    s_ij = q^_i . k^_j).  Window and padding follow attention.py:111-118,
    :174-183 and :185-188.  Candidates come from a float32 pass over the
    window only (SCREEN_MARGIN bounds its error); the kept pairs are decided
    in float64."""
    qn, kn = normalize(_heads(q), eps), normalize(_heads(k), eps)
    B, H, Tq, D = qn.shape
    Tk = kn.shape[2]
    qn32, kn32 = qn.astype(np.float32), kn.astype(np.float32)
    r = np.asarray(r, dtype=np.float64).reshape(H)
    w = np.asarray(w, dtype=np.float64).reshape(H)
    kpm = None if key_padding_mask is None else np.asarray(key_padding_mask, dtype=bool)
    out = {n: [] for n in ("b", "h", "i", "j", "s")}
    for hh in range(H):
        thr = 1.0 - 1.0 / r[hh]
        wc = math.ceil(w[hh]) if math.isfinite(w[hh]) and w[hh] < 2 ** 40 else 2 ** 40
        for b in range(B):
            for i0, i1 in _blocks(Tq, block):
                lo = max(0, i0 - wc + 1)
                hi = min(Tk, i1 if causal else i1 + wc - 1)
                if hi <= lo:
                    continue
                s32 = qn32[b, hh, i0:i1] @ kn32[b, hh, lo:hi].T
                # flat indices: one pass over a mostly-false mask
                ii, jj = np.divmod(np.flatnonzero(s32 > np.float32(thr - SCREEN_MARGIN)), hi - lo)
                ii = ii.astype(np.int64) + i0
                jj = jj.astype(np.int64) + lo
                rel = ii - jj                       # i - j
                inside = ((rel >= 0) & (rel < w[hh])) if causal else (np.abs(rel) < w[hh])
                if kpm is not None:
                    inside &= ~kpm[b, jj]
                ii, jj = ii[inside], jj[inside]
                s = np.einsum("pd,pd->p", qn[b, hh, ii], kn[b, hh, jj])
                keep = 1.0 - r[hh] * (1.0 - s) > 0.0
                n = int(keep.sum())
                out["b"].append(np.full(n, b, dtype=np.int64))
                out["h"].append(np.full(n, hh, dtype=np.int64))
                out["i"].append(ii[keep])
                out["j"].append(jj[keep])
                out["s"].append(s[keep])
    return {n: (np.concatenate(v) if v else np.zeros(0, dtype=np.float64 if n == "s" else np.int64))
            for n, v in out.items()}


def sparse_forward_backward(q, k, v, r, w, dy=None, causal=True, eps=EPS, key_padding_mask=None,
                            dropout=None, pairs=None):
    """forward() and, when dy is given, backward() evaluated over the live pairs only.

    Returns (y, grads, pairs): y (B,Tq,H,D); grads = (dq, dk, dv, dr, dw) as
    backward() returns them, or None without dy; pairs = live_pairs(...),
    with dy also "dr_abs" and "dw_abs" (H,): the per-head sums of the absolute
    values of the terms that dr and dw sum.
    Same math and conventions as forward()/backward(), float64 throughout."""
    import scipy.sparse as sp
    if pairs is None:
        pairs = live_pairs(q, k, r, w, causal, eps, key_padding_mask)
    qh, kh, vh = _heads(q), _heads(k), _heads(v)
    qn, kn, vn = normalize(qh, eps), normalize(kh, eps), normalize(vh, eps)
    B, H, Tq, D = qn.shape
    Tk = kn.shape[2]
    r = np.asarray(r, dtype=np.float64).reshape(H)
    w = np.asarray(w, dtype=np.float64).reshape(H)
    pb, ph, pi, pj, s = pairs["b"], pairs["h"], pairs["i"], pairs["j"], pairs["s"]
    a = 1.0 - r[ph] * (1.0 - s)                      # > 0 on every listed pair
    rel = (pj - pi).astype(np.float64)               # j - i
    m = 0.5 * (np.cos(math.pi * rel / w[ph]) + 1.0)
    mdw = 0.5 * np.sin(math.pi * rel / w[ph]) * math.pi * rel / (w[ph] * w[ph])
    if dropout is not None and float(dropout[0]) > 0.0:
        p_, seed = dropout
        keep = dropout_keep_bits(seed, pb * H + ph, pi, pj) >= np.uint64(dropout_threshold(p_))
        c = np.where(keep, dropout_scale(p_), 0.0)
        m = m * c
        mdw = mdw * c
    p = a * a * m
    row = (pb * H + ph) * Tq + pi                    # into (B*H*Tq) rows
    col = (pb * H + ph) * Tk + pj                    # into (B*H*Tk) rows
    shape = (B * H * Tq, B * H * Tk)
    P = sp.csr_matrix((p, (row, col)), shape=shape)
    qf, kf, vf = qn.reshape(-1, D), kn.reshape(-1, D), vn.reshape(-1, D)
    h = np.asarray(P @ vf).reshape(B, H, Tq, D)
    n = np.sqrt(np.sum(h * h, axis=-1, keepdims=True))
    nc = np.maximum(n, eps)
    F = np.tanh(nc) / nc
    y = np.transpose(F * h, (0, 2, 1, 3))
    if dy is None:
        return y, None, pairs
    g = _heads(dy)
    G = _tanhnorm_g(nc)
    hd = np.sum(h * g, axis=-1, keepdims=True)
    dh = np.where(n > eps, F * g + G * hd * h, (math.tanh(eps) / eps) * g).reshape(-1, D)
    dP = np.einsum("pd,pd->p", dh[row], vf[col])
    ds = 2.0 * a * r[ph] * m * dP
    DS = sp.csr_matrix((ds, (row, col)), shape=shape)
    dqn = np.asarray(DS @ kf).reshape(B, H, Tq, D)
    dkn = np.asarray(DS.T @ qf).reshape(B, H, Tk, D)
    dvn = np.asarray(P.T @ dh).reshape(B, H, Tk, D)
    tr, tw = -2.0 * a * (1.0 - s) * m * dP, a * a * mdw * dP
    dr = np.bincount(ph, weights=tr, minlength=H)
    dw = np.bincount(ph, weights=tw, minlength=H)
    # per-head sums of |term|: the scale a per-head sum's rounding error has
    pairs["dr_abs"] = np.bincount(ph, weights=np.abs(tr), minlength=H)
    pairs["dw_abs"] = np.bincount(ph, weights=np.abs(tw), minlength=H)
    t = lambda x: np.transpose(x, (0, 2, 1, 3))
    grads = (t(_normalize_bwd(qh, dqn, eps)), t(_normalize_bwd(kh, dkn, eps)),
             t(_normalize_bwd(vh, dvn, eps)), dr, dw)
    return y, grads, pairs
