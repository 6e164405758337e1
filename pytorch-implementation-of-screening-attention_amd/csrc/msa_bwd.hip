// Backward path of fused Screening Attention on gfx950.
//
// Gradients of the dense math in attention.py:142-200 / norm.py:23-25, written
// out for the normalised operands (same derivation as the reference's
// screening_bwd.py:6-18) plus the per-head terms the reference fused path
// drops (attention_triton.py:44):
//   dh_i   = TanhNorm'(h_i)^T dy_i
//   dP_ij  = dh_i . v^_j                        (pair weight p_ij = a_ij^2 m_ij)
//   dv^_j  = sum_i p_ij dh_i
//   ds_ij  = 2 a_ij r m_ij dP_ij  [a_ij > 0]
//   dq^_i  = sum_j ds_ij k^_j,   dk^_j = sum_i ds_ij q^_i
//   dr     = -sum 2 a (1-s) m dP,  dw = sum a^2 dP dm/dw
//   dx     = (dx^ - x^ (x^.dx^)) / |x|   (|x| > eps),  dx^/eps otherwise
// Only the 32x32 units the forward marked live in its bitmap are revisited;
// each wave turns its bitmap row/column into a 64-bit ballot mask and walks
// the set bits.  MFMA operands are the raw q, k, v values (exact in bf16),
// loaded straight from global memory into operand registers, and the 1/|x|
// factors are applied in fp32 to the products, so no normalised copy is
// rounded; dh is formed on the fly from y, dy and |h|.  Operands needed
// transposed come from identity MFMAs on the same registers, per-row scale
// factors reach register order through a small LDS vector.  Key padding
// (attention.py:185-188) enters as a zero 1/|k|, which gives s = 0 and so
// alpha = 0 for those keys.
//
//   dq_kernel   : wave per 32-query unit over its live key units; writes dq
//                 and the unit's (dr, dw) share, and leaves dh and 1/|q| of
//                 its rows for dkdv_kernel.
//   dkdv_kernel : wave per 32-key unit; accumulates dv^, dk^ in MFMA
//                 registers over its live query units and writes dk, dv; one
//                 wave per head also sums the (dr, dw) shares in a fixed
//                 order into dr, dw.
// No atomics anywhere, so every gradient is bitwise reproducible.
#include "msa_device.h"
#include "msa_internal.h"

namespace msa {

// G(n) = F'(n)/n with F(n) = tanh(n)/n.  Series below 0.25 (the closed form
// cancels there): F = 1 - n^2/3 + 2n^4/15 - 17n^6/315 + 62n^8/2835.
__device__ inline float tanhnorm_g(float n, float t) {
  if (n < 0.25f) {
    const float n2 = n * n;
    return -2.0f / 3.0f + n2 * (8.0f / 15.0f + n2 * (-34.0f / 105.0f + n2 * (496.0f / 2835.0f)));
  }
  return ((1.0f - t * t) / n - t / (n * n)) / n;
}

// dh = F dy + G (h.dy) h with h = y/F  ->  dh = c1 dy + c2 (y.dy) y
__device__ inline void tanhnorm_coefs(float n, float eps, float& c1, float& c2) {
  if (n > eps) {
    const float t = tanhf(n);
    c1 = t / n;
    c2 = tanhnorm_g(n, t) / (c1 * c1);
  } else {
    c1 = tanhf(eps) / eps;
    c2 = 0.0f;
  }
}

struct BwdKArgs {
  const void* q; Strides3 qs;
  const void* k; Strides3 ks;
  const void* v; Strides3 vs;
  const uint8_t* kpm;
  const void* y; const void* dy; const float* hnorm;
  const float* r; const float* w;
  const uint32_t* bits;
  void* dq; void* dk; void* dv; float* dr; float* dw;
  float* part;  // workspace: (dr, dw) shares per (b, h, query unit), [2][b*h][2*nqt]
  void* dh; float* iqs;  // workspace: dh [b*h][Tq_pad][DP] (T), 1/|q| [b*h][Tq_pad]
  int B, H, Tq, Tk, D, nqt, nkt, nku_words, causal;
  int64_t Tq_pad;
  float eps;
  Dropout drop;
};

// Query-side rows for row i of head (b,h), in two steps so that other memory
// traffic can be issued between them: load raw q, y, dy and |h|; then finish
// 1/|q| and dh (rounded to T, as the MFMA operand it becomes).  Rows past Tq
// read row 0 and are zeroed.
template <typename T, int DP>
struct QueryRows {
  PRow<T, DP> q, y, dh;
  float hn;
  bool ok;
  __device__ inline void load(const BwdKArgs& a, int b, int h, int bh, int i, int half) {
    ok = i < a.Tq;
    const int ii = ok ? i : 0;
    const int64_t yoff = (((int64_t)b * a.Tq + ii) * a.H + h) * a.D;
    q.load((const T*)a.q + b * a.qs.sb + (int64_t)ii * a.qs.st + h * a.qs.sh, ok, a.D, half);
    y.load((const T*)a.y + yoff, ok, a.D, half);
    dh.load((const T*)a.dy + yoff, ok, a.D, half);
    hn = a.hnorm[(int64_t)bh * a.Tq + ii];
  }
  // returns 1/|q|; dh holds TanhNorm'(h)^T dy afterwards
  __device__ inline float finish(float eps) {
    const float iq = q.inv_norm(eps);
    const float ydot = y.dot(dh);
    float c1, c2;
    tanhnorm_coefs(ok ? hn : 0.0f, eps, c1, c2);
    dh.axpby(c1, c2 * ydot, y);
    return iq;
  }
};

// Key-side rows for key j of head (b,h), load then finish as for the query
// side: raw k with 1/|k| (0 for padded or masked keys), raw v with 1/|v|.
template <typename T, int DP>
struct KeyRows {
  PRow<T, DP> k, v;
  bool ok, masked;
  __device__ inline void load(const BwdKArgs& a, int b, int h, int j, int half) {
    ok = j < a.Tk;
    const int jj = ok ? j : 0;
    k.load((const T*)a.k + b * a.ks.sb + (int64_t)jj * a.ks.st + h * a.ks.sh, ok, a.D, half);
    v.load((const T*)a.v + b * a.vs.sb + (int64_t)jj * a.vs.st + h * a.vs.sh, ok, a.D, half);
    masked = a.kpm != nullptr && a.kpm[(int64_t)b * a.Tk + jj] != 0;
  }
  __device__ inline void finish(float eps, float& ik, float& iv) const {
    ik = (ok && !masked) ? k.inv_norm(eps) : 0.0f;
    iv = v.inv_norm(eps);
  }
};

// Writes dx = normalise-backward(dx^, x) (attention.py:156-158 under
// autograd) for one row: dx^ in C-layout registers acc[dblk] whose rows are
// tcol-ordered columns, x as the lane's raw operand fragments of the same row
// (the operands the kernel already holds, so nothing is re-read).
//   |x| > eps:  dx = (dx^ - x^ (x^ . dx^)) / |x|;   otherwise dx = dx^ / eps.
template <typename T, int DP>
__device__ inline void write_norm_bwd(const f32x16 (&acc)[DP / 32], const typename Mma<T>::frag (&x)[DP / Mma<T>::KS],
                                      bool valid, int D, float eps, int half, T* out) {
  using M = Mma<T>;
  constexpr int NDH = DP / 32, NKS = DP / M::KS;
  float ss = 0.0f;
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) ss = frag_dot(x[ks], x[ks], ss);
  ss = half_sum(ss);
  const float nx = sqrtf(ss);
  const float ix = 1.0f / fmaxf(nx, eps);
  float dot = 0.0f;
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) dot += M::get(x[creg_ks<T>(dblk, r)], creg_e<T>(r)) * ix * acc[dblk][r];
  dot = half_sum(dot);
  const float proj = nx > eps ? dot : 0.0f;
  if (!valid) return;
  store_creg_row<T, NDH>(out, D, half, [&](int dblk, int r) {
    const float xn = M::get(x[creg_ks<T>(dblk, r)], creg_e<T>(r)) * ix;
    return (acc[dblk][r] - xn * proj) * ix;
  });
}

// Waves per SIMD the backward kernels are register-budgeted for: two (256
// registers a lane: the unit's operands, both accumulators and the scaled
// products all stay in registers) where the bf16 working set allows, else one.
template <typename T, int DP>
constexpr int bwd_waves() { return sizeof(T) == 2 && DP <= 64 ? 2 : 1; }

// ---------------------------------------------------------------------------
// dQ (runs first).  One wave (a 64-thread block) per query unit: 32
// consecutive queries of head (b,h), lane -> query i = 32*qu + l%32,
// registers -> keys.  The wave walks its row of the live-unit bitmap; per
// live key unit it loads the 32 raw K and V rows straight into MFMA operand
// registers (A operands, row perm_row(l%32)), forms S^T = K Q^T and
// dP^T = V dH^T, scales them by 1/|k|, 1/|v| (exchanged in register order
// through a 32-float LDS vector), and accumulates dq^T += K^T (ds/|k|)^T with
// K^T from an identity MFMA on the same registers.  Side output for
// dkdv_kernel: dh (rounded to T, as the operand it becomes) and 1/|q| of the
// unit's rows, written by every unit with a live key unit (the only rows
// dkdv_kernel reads).
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 && DP <= 64 ? 3 : 1))) void dq_kernel(BwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  __shared__ __attribute__((aligned(16))) float sk[32];  // 1/|k| (0 if padded or masked) of the unit's key rows
  __shared__ __attribute__((aligned(16))) float sv[32];  // 1/|v|
  __shared__ float mtab[128];  // soft-mask table of the current unit, then its dm/dw table (unit_mask_table)
  __shared__ typename Mma<T>::frag qh[2 * (DP / Mma<T>::KS)][kWave];  // own raw q, dh operand fragments
  const int lane = threadIdx.x, half = lane >> 5, l32 = lane & 31;
  int qu, bh;
  float head_r, head_w;
  xcd_interleave_ranked(a.r, a.w, a.H, qu, bh, head_r, head_w);
  const int b = bh / a.H, h = bh % a.H;
  const bool causal = a.causal != 0;
  const HeadParams hp = head_params_rw(head_r, head_w, causal);
  const int i = qu * kUnit + l32;
  const bool valid = i < a.Tq;
  const int ii = valid ? i : 0;
  T* dqrow = (T*)a.dq + (((int64_t)b * a.Tq + ii) * a.H + h) * a.D;

  int ku_lo, ku_hi;
  {
    const int64_t qa = (int64_t)qu * kUnit, qb = qa + kUnit - 1 < a.Tq - 1 ? qa + kUnit - 1 : a.Tq - 1;
    int64_t jlo = qa - hp.wc + 1;
    int64_t jhi = causal ? qb : qb + hp.wc - 1;
    if (jlo < 0) jlo = 0;
    if (jhi > a.Tk - 1) jhi = a.Tk - 1;
    ku_lo = (int)(jlo / kUnit);
    ku_hi = jhi >= jlo ? (int)(jhi / kUnit) : ku_lo - 1;
  }
  const uint32_t* brow = a.bits + ((int64_t)bh * 2 * a.nqt + qu) * a.nku_words;
  RowWalk walk(brow, ku_lo, ku_hi);
  int cur = walk.next();
  const int64_t nbh = (int64_t)a.B * a.H;
  const int nqu = 2 * a.nqt;
  if (cur < 0) {  // wave-uniform: no live key unit, dq = 0 and no share of dr, dw
    if (valid)
#pragma unroll
      for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * dblk + 8 * g + 4 * half;
          if (d < a.D) store4(dqrow + d, 0.0f, 0.0f, 0.0f, 0.0f);
        }
    if (lane == 0) {
      a.part[(int64_t)bh * nqu + qu] = 0.0f;
      a.part[nbh * nqu + (int64_t)bh * nqu + qu] = 0.0f;
    }
    return;
  }

  // key row of this lane in unit u: 32u + perm_row(l32), read as row Tk-1
  // past Tk (its 1/|k| is then 0, so it contributes nothing); the lane's
  // chunks from a wave-uniform row base plus a 32-bit lane offset
  const int m = perm_row(l32);
  const T* kb0 = (const T*)a.k + b * a.ks.sb + h * a.ks.sh;
  const T* vb0 = (const T*)a.v + b * a.vs.sb + h * a.vs.sh;
  auto load_rows = [&](const T* base, int64_t st, int u, frag (&f)[NKS]) {
    const int r = u * kUnit + m < a.Tk ? m : a.Tk - 1 - u * kUnit;
    const uint32_t off = (uint32_t)(((int64_t)r * st + PER * half) * (int64_t)sizeof(T));
    const char* p = (const char*)(base + (int64_t)u * kUnit * st) + off;
    // chunks past D (D = 16 < DP = 32 only) re-read chunk 0; zero_tail clears them
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int c = DP == 32 && KS * ks >= a.D ? 0 : KS * ks;
      f[ks] = M::load((const T*)(p + c * (int)sizeof(T)));
    }
  };
  auto zero_tail = [&](frag (&f)[NKS]) {
    if constexpr (DP == 32) {
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        if (KS * ks >= a.D) f[ks] = M::zero();
    }
  };
  // 1/|k| is 0 for keys past Tk and for masked keys
  auto key_ok = [&](int u) {
    const int j = u * kUnit + m;
    return j < a.Tk && !(a.kpm != nullptr && a.kpm[(int64_t)b * a.Tk + j] != 0);
  };

  // own queries' rows first, then the first key unit's rows behind them;
  // the raw q and dh operand fragments are kept in LDS (read back per key
  // unit), which leaves registers for three waves per SIMD
  frag kc[NKS], vc[NKS];
  float iql;
  bool kok;
  {
    QueryRows<T, DP> qr;
    qr.load(a, b, h, bh, i, half);
    load_rows(kb0, a.ks.st, cur, kc);
    load_rows(vb0, a.vs.st, cur, vc);
    kok = key_ok(cur);
    iql = qr.finish(a.eps);
    // dh and 1/|q| of this unit's rows for dkdv_kernel (zero past Tq)
    T* dst = (T*)a.dh + ((int64_t)bh * a.Tq_pad + i) * DP;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      qh[ks][lane] = qr.q.f[ks];
      qh[NKS + ks][lane] = qr.dh.f[ks];
      *reinterpret_cast<frag*>(dst + KS * ks + PER * half) = qr.dh.f[ks];
    }
    if (half == 0) a.iqs[(int64_t)bh * a.Tq_pad + i] = valid ? iql : 0.0f;
  }
  const float thq = hp.thr / iql;  // s > thr  <=>  (q . k)/|k| > thr |q|
  float dr_acc = 0.0f, dw_acc = 0.0f;  // this unit's share of dr, dw
  f32x16 adq[NDH];
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) adq[dblk][r] = 0.0f;

  for (;;) {
    const int k0 = cur * kUnit;
    // the unit's mask tables first, while few values are live (the LDS sync
    // after the products below covers these writes too; this iteration's
    // writes follow the previous one's reads in the wave's LDS order)
    unit_mask_table<true>(mtab, mtab + 64, qu * kUnit - k0 - 31, hp, lane);
    const int nxt = walk.next();
    zero_tail(kc);
    zero_tail(vc);
    // register r -> key k0 + rowof(r, half), lane -> query i
    f32x16 s, dp;
    float s2k = 0.0f, s2v = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[r] = 0.0f; dp[r] = 0.0f; }
    {
      frag g[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) g[ks] = qh[ks][lane];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        s = M::mma_ng(kc[ks], g[ks], s);
        s2k = frag_dot(kc[ks], kc[ks], s2k);
      }
      guard_frags(g);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) g[ks] = qh[NKS + ks][lane];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        dp = M::mma_ng(vc[ks], g[ks], dp);
        s2v = frag_dot(vc[ks], vc[ks], s2v);
      }
      guard_frags(g);
    }
    guard_frags(vc);
    s2k = half_sum(s2k);
    s2v = half_sum(s2v);
    const float ikl = kok ? inv_len(s2k, a.eps) : 0.0f;  // this lane's key row m
    {
      const float iv = inv_len(s2v, a.eps);
      wave_lds_sync();
      if (half == 0) { sk[m] = ikl; sv[m] = iv; }
      wave_lds_sync();
    }
    // scaled in place: s = (q . k)/|k|, dp = dH . v^
    {
      float sc[16];
      read_row_scales(sk, half, sc);
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] *= sc[r];
      read_row_scales(sv, half, sc);
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] *= sc[r];
    }
    // every lane forms its pair's terms branch-free (a = 0 below the
    // threshold, the mask and dm/dw, 0 outside the window, from the unit's
    // tables: entry l32 - 8half + 31 - 16(r/8) - r%8 for register r), for
    // every register; with dropout, only for the registers where some lane
    // may pass a conservative gate on the products (s > thr |q|), so the
    // pair hash runs there only
    {
      // entry 23 - (16(r/8) + r%8) of each table: constant offsets from one base
      const float* mrow = mtab + (l32 - 8 * half + 8);
      // (rows past Tq hold q = 0, so s = 0 and a = 1 - r <= 0: no term)
      auto body = [&](int r) {
        const int off = 16 * (r >> 3) + (r & 7);
        const float sv = s[r] * iql;
        const float av = fmaxf(trim(sv, hp.r), 0.0f);
        float g = dp[r];
        if (a.drop.on) g *= dropout_factor(a.drop, bh, i, k0 + 8 * half + off);
        const float t = 2.0f * av * mrow[23 - off] * g;
        dr_acc -= t * (1.0f - sv);
        dw_acc += av * av * g * mrow[64 + 23 - off];
        dp[r] = hp.r * t;
      };
      if (a.drop.on) {  // the pair's hash only where some lane may pass
        const uint32_t pm0 = pass_mask(s, thq);
        for_each_set(pm0, body);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (((pm0 >> r) & 1u) == 0u) dp[r] = 0.0f;
      } else {  // every register: a = 0 gives no term, and no mask or branches
#pragma unroll
        for (int r = 0; r < 16; ++r) body(r);
      }
    }
    // dq^T[d][i] += sum_j K^T[d][j] (ds/|k|)^T[j][i], K^T by identity from
    // the key rows, one 32-column block of d at a time (fp16: K^T takes
    // 1/|k| instead, below)
    if constexpr (!kScaleRowsNotWeights<T>) {
      float ksc[16];
      read_row_scales(sk, half, ksc);
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] *= ksc[r];
    }
    frag db[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) db[c] = M::pack(dp, c * PER);
    frag id[NC];  // identity slices, held (and guarded) as named operands
#pragma unroll
    for (int c = 0; c < NC; ++c) id[c] = ident_frag<T>(c, lane);
#pragma unroll
    for (int dblk = 0; dblk < NDH; ++dblk) {
      frag kt[NC];
      f32x16 tr;
#pragma unroll
      for (int r = 0; r < 16; ++r) tr[r] = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) tr = M::mma_ng(kc[dblk * NC + c], id[c], tr);
      if constexpr (kScaleRowsNotWeights<T>) scale_rows_fp32(tr, sk, half);
#pragma unroll
      for (int c = 0; c < NC; ++c) kt[c] = M::pack(tr, c * PER);
#pragma unroll
      for (int c = 0; c < NC; ++c) adq[dblk] = M::mma_ng(kt[c], db[c], adq[dblk]);
      guard_frags(kt);
    }
    guard_frags(kc);
    guard_frags(db);
    guard_frags(id);
    if (nxt < 0) break;
    cur = nxt;
    load_rows(kb0, a.ks.st, cur, kc);
    load_rows(vb0, a.vs.st, cur, vc);
    kok = key_ok(cur);
  }
  {
    frag x[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) x[ks] = qh[ks][lane];
    write_norm_bwd<T, DP>(adq, x, valid, a.D, a.eps, half, dqrow);
  }
  dr_acc = wave_sum(dr_acc);
  dw_acc = wave_sum(dw_acc);
  if (lane == 0) {
    a.part[(int64_t)bh * nqu + qu] = dr_acc;
    a.part[nbh * nqu + (int64_t)bh * nqu + qu] = dw_acc;
  }
}

// ---------------------------------------------------------------------------
// dK, dV (runs after dq_kernel).  One wave (a 64-thread block) per key unit:
// 32 consecutive keys of head (b,h), lane -> key j = 32*ku + l%32 of the C
// blocks, registers -> queries.  The wave walks its column of the live-unit
// bitmap; per live query unit it loads the raw Q rows and the dh rows and
// 1/|q| that dq_kernel left in the workspace straight into MFMA operand
// registers (A operands, row perm_row(l%32)), forms S = Q K^T and dP = dH V^T
// with its own raw K, V rows as B operands, and accumulates
// dv^T += dH^T P and dk^T += Q^T (ds/|q|) with dH^T, Q^T from identity MFMAs
// on the same registers.  1/|q| reaches register order through a 32-float
// LDS vector.  The wave finishes dk, dv and its (dr, dw) partial.
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(bwd_waves<T, DP>()))) void dkdv_kernel(BwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  __shared__ __attribute__((aligned(16))) float sq[32];  // 1/|q| of the current query unit's rows
  __shared__ float mt[64];  // soft-mask table of the current unit (unit_mask_table)
  __shared__ typename Mma<T>::frag kvs[2 * (DP / Mma<T>::KS)][kWave];  // own raw k, v operand fragments
  const int lane = threadIdx.x, half = lane >> 5, l32 = lane & 31;
  int ku, bh;
  float head_r, head_w;
  xcd_interleave_ranked(a.r, a.w, a.H, ku, bh, head_r, head_w);
  // a key unit's live query units lie after it (its window runs forward), so
  // under a causal mask the lowest key units carry the most work: they go first
  if (a.causal) ku = (int)gridDim.x - 1 - ku;
  const int b = bh / a.H, h = bh % a.H;
  const bool causal = a.causal != 0;
  const HeadParams hp = head_params_rw(head_r, head_w, causal);
  const int k0 = ku * kUnit;
  const int j = k0 + l32;
  const bool jvalid = j < a.Tk;
  const int jj = jvalid ? j : 0;
  const int64_t orow = (((int64_t)b * a.Tk + jj) * a.H + h) * a.D;
  if (ku == 2 * a.nkt - 1 && bh < a.H) {
    // one wave per head: dr, dw from dq_kernel's per-query-unit shares
    // (complete: dq_kernel ran first), summed in a fixed order
    const int64_t nbh = (int64_t)a.B * a.H;
    const int nqu = 2 * a.nqt;
    float ar = 0.0f, aw = 0.0f;
    for (int64_t idx = lane; idx < (int64_t)a.B * nqu; idx += kWave) {
      const int bb = (int)(idx / nqu), u = (int)(idx % nqu);
      const int64_t o = ((int64_t)bb * a.H + bh) * nqu + u;
      ar += a.part[o];
      aw += a.part[nbh * nqu + o];
    }
    ar = wave_sum(ar);
    aw = wave_sum(aw);
    if (lane == 0) {
      a.dr[bh] = ar;
      a.dw[bh] = aw;
    }
  }

  int qu_lo, qu_hi;
  {
    const int64_t klast = k0 + kUnit - 1 < a.Tk - 1 ? k0 + kUnit - 1 : a.Tk - 1;
    int64_t ilo = causal ? (int64_t)k0 : (int64_t)k0 - hp.wc + 1;
    int64_t ihi = klast + hp.wc - 1;
    if (ilo < 0) ilo = 0;
    if (ihi > a.Tq - 1) ihi = a.Tq - 1;
    qu_lo = (int)(ilo / kUnit);
    qu_hi = ihi >= ilo && k0 < a.Tk ? (int)(ihi / kUnit) : qu_lo - 1;
  }
  const uint32_t* bcol = a.bits + (int64_t)bh * 2 * a.nqt * a.nku_words + (ku >> 5);
  ColWalk walk(bcol, a.nku_words, ku & 31, qu_lo, qu_hi);
  int cur = walk.next();
  if (cur < 0) {  // wave-uniform: no live query unit, dk = dv = 0
    if (jvalid)
#pragma unroll
      for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * dblk + 8 * g + 4 * half;
          if (d < a.D) {
            store4((T*)a.dk + orow + d, 0.0f, 0.0f, 0.0f, 0.0f);
            store4((T*)a.dv + orow + d, 0.0f, 0.0f, 0.0f, 0.0f);
          }
        }
    return;
  }

  // query row of this lane in unit u: 32u + perm_row(l32).  Raw q rows past
  // Tq read row Tq-1; their 1/|q| and dh rows (workspace, zero past Tq) are
  // 0, so they contribute nothing.  A wave-uniform row base plus a 32-bit
  // lane offset per operand.
  const int m = perm_row(l32);
  const T* qb0 = (const T*)a.q + b * a.qs.sb + h * a.qs.sh;
  const T* hb0 = (const T*)a.dh + (int64_t)bh * a.Tq_pad * DP;
  const float* iq0 = a.iqs + (int64_t)bh * a.Tq_pad;
  auto load_unit = [&](int u, frag (&qf)[NKS], frag (&hf)[NKS], float& iqv) {
    const int r = u * kUnit + m < a.Tq ? m : a.Tq - 1 - u * kUnit;
    const uint32_t qoff = (uint32_t)(((int64_t)r * a.qs.st + PER * half) * (int64_t)sizeof(T));
    const char* pq = (const char*)(qb0 + (int64_t)u * kUnit * a.qs.st) + qoff;
    const char* ph = (const char*)(hb0 + (int64_t)u * kUnit * DP) + (uint32_t)((m * DP + PER * half) * (int)sizeof(T));
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int c = DP == 32 && KS * ks >= a.D ? 0 : KS * ks;  // chunks past D re-read chunk 0 (cleared at use)
      qf[ks] = M::load((const T*)(pq + c * (int)sizeof(T)));
      hf[ks] = M::load((const T*)(ph + KS * ks * (int)sizeof(T)));
    }
    iqv = iq0[(int64_t)u * kUnit + l32];  // lanes l and l+32 read the same row
  };
  auto zero_tail = [&](frag (&f)[NKS]) {
    if constexpr (DP == 32) {
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        if (KS * ks >= a.D) f[ks] = M::zero();
    }
  };

  // own keys as raw B operands (lane -> key), kept in LDS (read back per
  // query unit; the registers hold the next unit's rows instead), with 1/|k|
  // (0 if padded or masked) and 1/|v|; their loads go first, the first query
  // unit's behind
  frag qf[NKS], hf[NKS];
  float ikl, ivl, iqv;
  {
    KeyRows<T, DP> kr;
    kr.load(a, b, h, j, half);
    load_unit(cur, qf, hf, iqv);
    kr.finish(a.eps, ikl, ivl);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      kvs[ks][lane] = kr.k.f[ks];
      kvs[NKS + ks][lane] = kr.v.f[ks];
    }
  }
  f32x16 acc_k[NDH], acc_v[NDH];
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc_k[dblk][r] = 0.0f; acc_v[dblk][r] = 0.0f; }
  const float thk = hp.thr / ikl;  // s > thr  <=>  (q . k)/|q| > thr |k|  (+inf for masked keys)

  for (;;) {
    const int q0 = cur * kUnit;
    // the next unit's rows load while this one is computed (past the last
    // unit, the current one again, a cache hit: every iteration then waits
    // for the same count)
    const int nxt = walk.next();
    frag qn[NKS], hn[NKS];
    float iqn;
    load_unit(nxt >= 0 ? nxt : cur, qn, hn, iqn);
    zero_tail(qf);
    wave_lds_sync();
    if (half == 0) sq[l32] = iqv;
    unit_mask_table<false>(mt, nullptr, q0 - k0 - 31, hp, lane);
    wave_lds_sync();
    // register r -> query q0 + rowof(r, half), lane -> key j.  Scaled in
    // place: s = (q . k)/|q|, dp = (dh . v)/|v|.
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[r] = 0.0f; dp[r] = 0.0f; }
    {
      frag g[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) g[ks] = kvs[ks][lane];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) s = M::mma_ng(qf[ks], g[ks], s);
      guard_frags(g);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) g[ks] = kvs[NKS + ks][lane];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) dp = M::mma_ng(hf[ks], g[ks], dp);
      guard_frags(g);
    }
    {
      float sc[16];
      read_row_scales(sq, half, sc);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] *= sc[r];
        dp[r] *= ivl;
      }
    }
    // every lane forms its pair's weight and ds branch-free (the mask, 0
    // outside the window, from the unit's table: entry 16(r/8) + r%8 + 8half
    // - l32 + 31 for register r), for every register; with dropout, only for
    // the registers where some lane may pass a conservative gate on the
    // products (s > thr |k|), so the pair hash runs there only
    {
      const float* mrow = mt + (8 * half - l32 + 31);
      auto body = [&](int r) {
        const int off = 16 * (r >> 3) + (r & 7);
        const float av = fmaxf(trim(s[r] * ikl, hp.r), 0.0f);
        float mk = mrow[off];
        if (a.drop.on) mk *= dropout_factor(a.drop, bh, q0 + 8 * half + off, j);
        const float am = av * mk;
        s[r] = av * am;
        dp[r] = 2.0f * hp.r * am * dp[r];
      };
      if (a.drop.on) {  // the pair's hash only where some lane may pass
        const uint32_t pm0 = pass_mask(s, thk);
        for_each_set(pm0, body);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (((pm0 >> r) & 1u) == 0u) { s[r] = 0.0f; dp[r] = 0.0f; }
      } else {  // every register: a = 0 gives no term, and no mask or branches
#pragma unroll
        for (int r = 0; r < 16; ++r) body(r);
      }
    }
    // ds/|q| (fp16: Q^T takes 1/|q| instead, below)
    if constexpr (!kScaleRowsNotWeights<T>) {
      float qsc[16];
      read_row_scales(sq, half, qsc);
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] *= qsc[r];
    }
    // dv^T[d][j] += sum_i dH^T[d][i] P[i][j];  dk^T[d][j] += sum_i Q^T[d][i] (ds/|q|)[i][j]
    // with dH^T, Q^T from identity products on the row registers, one
    // 32-column block of d at a time
    frag pb[NC], db[NC], id[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      pb[c] = M::pack(s, c * PER);
      db[c] = M::pack(dp, c * PER);
      id[c] = ident_frag<T>(c, lane);  // held (and guarded) as named operands
    }
#pragma unroll
    for (int dblk = 0; dblk < NDH; ++dblk) {
#pragma unroll
      for (int op = 0; op < 2; ++op) {  // 0: dH^T P -> dv, 1: Q^T dS -> dk
        frag t[NC];
        f32x16 tr;
#pragma unroll
        for (int r = 0; r < 16; ++r) tr[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
          tr = M::mma_ng(op == 0 ? hf[dblk * NC + c] : qf[dblk * NC + c], id[c], tr);
        if constexpr (kScaleRowsNotWeights<T>)
          if (op == 1) scale_rows_fp32(tr, sq, half);
#pragma unroll
        for (int c = 0; c < NC; ++c) t[c] = M::pack(tr, c * PER);
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          if (op == 0) acc_v[dblk] = M::mma_ng(t[c], pb[c], acc_v[dblk]);
          else acc_k[dblk] = M::mma_ng(t[c], db[c], acc_k[dblk]);
        }
        guard_frags(t);
      }
    }
    guard_frags(qf);
    guard_frags(hf);
    guard_frags(pb);
    guard_frags(db);
    guard_frags(id);
    if (nxt < 0) break;
    cur = nxt;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      qf[ks] = qn[ks];
      hf[ks] = hn[ks];
    }
    iqv = iqn;
  }

  {
    frag x[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) x[ks] = kvs[ks][lane];
    write_norm_bwd<T, DP>(acc_k, x, jvalid, a.D, a.eps, half, (T*)a.dk + orow);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) x[ks] = kvs[NKS + ks][lane];
    write_norm_bwd<T, DP>(acc_v, x, jvalid, a.D, a.eps, half, (T*)a.dv + orow);
  }
}

// Workspace: [dr/dw partials][dh][1/|q|], each 256-byte aligned.
static int64_t bwd_part_bytes(const Geometry& g) { return round_up((int64_t)2 * g.B * g.H * 2 * g.nqt * 4, 256); }
static int64_t bwd_dh_bytes(const Geometry& g) {
  return round_up((int64_t)g.B * g.H * g.Tq_pad * g.DP * (int64_t)g.esize, 256);
}
size_t bwd_ws_bytes(const Geometry& g) {
  return bwd_part_bytes(g) + bwd_dh_bytes(g) + round_up((int64_t)g.B * g.H * g.Tq_pad * 4, 256);
}

template <typename T, int DP>
static hipError_t launch_bwd_t(const BwdCall& c) {
  const Geometry& g = c.g;
  BwdKArgs ka;
  ka.q = c.q; ka.qs = c.qs; ka.k = c.k; ka.ks = c.ks; ka.v = c.v; ka.vs = c.vs; ka.kpm = c.kpm;
  ka.y = c.y; ka.dy = c.dy; ka.hnorm = c.hnorm;
  ka.r = c.r; ka.w = c.w; ka.bits = c.bits;
  ka.dq = c.dq; ka.dk = c.dk; ka.dv = c.dv; ka.dr = c.dr; ka.dw = c.dw;
  char* ws = (char*)c.workspace;
  ka.part = (float*)ws;
  ka.dh = ws + bwd_part_bytes(g);
  ka.iqs = (float*)(ws + bwd_part_bytes(g) + bwd_dh_bytes(g));
  ka.B = g.B; ka.H = g.H; ka.Tq = g.Tq; ka.Tk = g.Tk; ka.D = g.D;
  ka.nqt = g.nqt; ka.nkt = g.nkt; ka.nku_words = g.nku_words; ka.causal = g.causal;
  ka.Tq_pad = g.Tq_pad;
  ka.eps = c.eps;
  ka.drop = c.drop;
  timer_begin(5, c.stream);
  hipLaunchKernelGGL((dq_kernel<T, DP>), dim3((unsigned)(2 * g.nqt), (unsigned)(g.B * g.H)), dim3(64), 0, c.stream,
                     ka);
  timer_end(5, c.stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(4, c.stream);
  hipLaunchKernelGGL((dkdv_kernel<T, DP>), dim3((unsigned)(2 * g.nkt), (unsigned)(g.B * g.H)), dim3(64), 0, c.stream,
                     ka);
  timer_end(4, c.stream);
  return hipGetLastError();
}

hipError_t launch_bwd(const BwdCall& c) {
  const int DP = c.g.DP;
  if (c.g.dtype == 1) {
    if (DP == 32) return launch_bwd_t<bf16, 32>(c);
    if (DP == 64) return launch_bwd_t<bf16, 64>(c);
    return launch_bwd_t<bf16, 128>(c);
  }
  if (c.g.dtype == 2) {
    if (DP == 32) return launch_bwd_t<f16, 32>(c);
    if (DP == 64) return launch_bwd_t<f16, 64>(c);
    return launch_bwd_t<f16, 128>(c);
  }
  if (DP == 32) return launch_bwd_t<float, 32>(c);
  if (DP == 64) return launch_bwd_t<float, 64>(c);
  return launch_bwd_t<float, 128>(c);
}

}  // namespace msa
