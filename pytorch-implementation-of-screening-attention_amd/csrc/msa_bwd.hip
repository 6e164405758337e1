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
// Only the tiles the forward marked live in its bitmap are revisited; each
// wave turns its bitmap row/column into a 64-bit ballot mask and walks the set
// bits.  MFMA operands are the raw q, k, v values (exact in bf16) and the
// 1/|x| factors are applied in fp32 to the products, so no normalised copy is
// rounded; dh is formed on the fly from y, dy and |h|.  Operands needed
// transposed go through a wave-private LDS tile, per-row scale factors
// through a small LDS vector.  Key padding (attention.py:185-188) enters as a
// zero 1/|k|, which gives s = 0 and so alpha = 0 for those keys.
//
//   dkdv_kernel     : wave per 64-key tile; accumulates dv^, dk^ in MFMA
//                     registers over its live query tiles, writes dk, dv and
//                     one (dr, dw) partial.
//   dq_kernel       : wave per 64-query tile over its live key tiles.
//   rw_reduce_kernel: fixed-order sum of the partials -> dr, dw.
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
  void* dq; void* dk; void* dv; float* part;
  int B, H, Tq, Tk, D, nqt, nkt, nkt_words, causal;
  float eps;
};

// Query-side rows for row i of head (b,h): raw q with 1/|q|, and dh.
template <typename T, int DP>
__device__ inline void query_rows(const BwdKArgs& a, int b, int h, int bh, int i, int half, Row<T, DP>& qr,
                                  float& iq, Row<T, DP>& dh) {
  const bool ok = i < a.Tq;
  const int ii = ok ? i : 0;
  qr.load((const T*)a.q + b * a.qs.sb + (int64_t)ii * a.qs.st + h * a.qs.sh, ok, a.D, half);
  iq = qr.inv_norm(a.eps);
  const int64_t yoff = (((int64_t)b * a.Tq + ii) * a.H + h) * a.D;
  Row<T, DP> yr;
  yr.load((const T*)a.y + yoff, ok, a.D, half);
  dh.load((const T*)a.dy + yoff, ok, a.D, half);
  const float ydot = yr.dot(dh);
  float c1, c2;
  tanhnorm_coefs(ok ? a.hnorm[(int64_t)bh * a.Tq + ii] : 0.0f, a.eps, c1, c2);
  const float cy = c2 * ydot;
#pragma unroll
  for (int n = 0; n < Row<T, DP>::N; ++n) dh.x[n] = c1 * dh.x[n] + cy * yr.x[n];
}

// Key-side rows for key j of head (b,h): raw k with 1/|k| (0 for padded or
// masked keys) and raw v with 1/|v|.
template <typename T, int DP>
__device__ inline void key_rows(const BwdKArgs& a, int b, int h, int j, int half, Row<T, DP>& kr, float& ik,
                                Row<T, DP>& vr, float& iv) {
  const bool ok = j < a.Tk;
  const int jj = ok ? j : 0;
  kr.load((const T*)a.k + b * a.ks.sb + (int64_t)jj * a.ks.st + h * a.ks.sh, ok, a.D, half);
  vr.load((const T*)a.v + b * a.vs.sb + (int64_t)jj * a.vs.st + h * a.vs.sh, ok, a.D, half);
  ik = kr.inv_norm(a.eps);
  iv = vr.inv_norm(a.eps);
  if (!ok || (a.kpm != nullptr && a.kpm[(int64_t)b * a.Tk + jj])) ik = 0.0f;
}

// Writes the lane's slots of operand row `m` (rounded to T) into a transposed
// LDS tile t[d][m] of pitch ld.
template <typename T, int DP>
__device__ inline void stash_transposed(T* t, int ld, int m, const Row<T, DP>& row, int half) {
  constexpr int KS = Mma<T>::KS, PER = Mma<T>::PER, NKS = DP / KS;
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
    for (int e = 0; e < PER; ++e) t[(KS * ks + PER * half + e) * ld + m] = from_f<T>(row.x[ks * PER + e]);
}

// Scale factors of the 16 rows a lane's C-block registers cover:
// register r -> row 16*(r/8) + 8*half + r%8 of a 32-row half tile.
__device__ inline void read_row_scales(const float* sc, int half, float (&o)[16]) {
#pragma unroll
  for (int g = 0; g < 2; ++g)
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(sc + 16 * g + 8 * half + 4 * u);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[8 * g + 4 * u + e] = v[e];
    }
}

// Writes dx = normalise-backward(dx^, x) for one row held in C-layout
// registers acc[dh] (rows d = 32*dh + 8*(r/4) + 4*half + r%4) of a lane.
template <typename T, int NDH>
__device__ inline void write_norm_bwd(const f32x16 (&acc)[NDH], const T* xrow, bool valid, int D, float eps,
                                      int half, T* out) {
  f32x4 xv[NDH][4];
  float ss = 0.0f;
#pragma unroll
  for (int dh = 0; dh < NDH; ++dh)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * dh + 8 * g + 4 * half;
      xv[dh][g] = (valid && d < D) ? load4(xrow + d) : f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int e = 0; e < 4; ++e) ss += xv[dh][g][e] * xv[dh][g][e];
    }
  ss += __shfl_xor(ss, 32);
  const float nx = sqrtf(ss);
  const float ix = 1.0f / fmaxf(nx, eps);
  float dot = 0.0f;
#pragma unroll
  for (int dh = 0; dh < NDH; ++dh)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) dot += xv[dh][g][e] * ix * acc[dh][4 * g + e];
  dot += __shfl_xor(dot, 32);
  const float proj = nx > eps ? dot : 0.0f;
  if (!valid) return;
#pragma unroll
  for (int dh = 0; dh < NDH; ++dh)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * dh + 8 * g + 4 * half;
      if (d < D) {
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = (acc[dh][4 * g + e] - xv[dh][g][e] * ix * proj) * ix;
        store4(out + d, o[0], o[1], o[2], o[3]);
      }
    }
}

template <typename T>
struct LdsT {
  static constexpr int LD = 32 + 16 / (int)sizeof(T);  // padded pitch of a transposed half tile
};

// One wave (64-thread block) per 64-key tile of head (b,h); lane -> key
// j = k0 + 32*kh + l32.
template <typename T, int DP>
__global__ __launch_bounds__(64) void dkdv_kernel(BwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  constexpr int LD = LdsT<T>::LD;
  __shared__ __attribute__((aligned(16))) T tq[DP * LD];   // raw q^T [d][i]
  __shared__ __attribute__((aligned(16))) T th[DP * LD];   // dh^T    [d][i]
  __shared__ __attribute__((aligned(16))) float sq[32];    // 1/|q_i|
  const int lane = threadIdx.x, half = lane >> 5, l32 = lane & 31;
  int kt, bh;
  xcd_order(kt, bh);
  const int b = bh / a.H, h = bh % a.H;
  const HeadParams hp = head_params(a.r, a.w, h);
  const bool causal = a.causal != 0;
  const int k0 = kt * kTile;

  // own keys as raw B operands, with their 1/|k| and 1/|v|
  frag kf[2][NKS], vf[2][NKS];
  float ikl[2], ivl[2];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
    Row<T, DP> kr, vr;
    key_rows<T, DP>(a, b, h, k0 + 32 * kh + l32, half, kr, ikl[kh], vr, ivl[kh]);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      kf[kh][ks] = kr.frag(ks, 1.0f);
      vf[kh][ks] = vr.frag(ks, 1.0f);
    }
  }

  f32x16 adv[NDH][2], adk[NDH][2];
#pragma unroll
  for (int dh_ = 0; dh_ < NDH; ++dh_)
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int r = 0; r < 16; ++r) { adv[dh_][kh][r] = 0.0f; adk[dh_][kh][r] = 0.0f; }
  float dr_acc = 0.0f, dw_acc = 0.0f;

  const int64_t klast = k0 + 63 < a.Tk - 1 ? k0 + 63 : a.Tk - 1;
  int64_t ilo = causal ? (int64_t)k0 : (int64_t)k0 - hp.wc + 1;
  int64_t ihi = klast + hp.wc - 1;
  if (ilo < 0) ilo = 0;
  if (ihi > a.Tq - 1) ihi = a.Tq - 1;
  const int qt_lo = (int)(ilo / kTile), qt_hi = ihi >= ilo ? (int)(ihi / kTile) : qt_lo - 1;

  for (int base = qt_lo; base <= qt_hi; base += kWave) {
    const int ql = base + lane;
    bool bit = false;
    if (ql <= qt_hi) bit = (a.bits[((int64_t)bh * a.nqt + ql) * a.nkt_words + (kt >> 5)] >> (kt & 31)) & 1u;
    unsigned long long mask = __ballot(bit);
    while (mask != 0ull) {
      const int qt = base + __builtin_ctzll(mask);
      mask &= mask - 1ull;
      const int q0 = qt * kTile;

      // one 32-row half of the query tile at a time
      for (int qh = 0; qh < 2; ++qh) {
        // rows i = q0 + 32*qh + perm_row(l32) as A operands; transposes and
        // 1/|q| into LDS
        frag qa[NKS], ha[NKS];
        wave_lds_sync();
        {
          const int m = perm_row(l32);
          Row<T, DP> qr, dr;
          float iq;
          query_rows<T, DP>(a, b, h, bh, q0 + 32 * qh + m, half, qr, iq, dr);
#pragma unroll
          for (int ks = 0; ks < NKS; ++ks) {
            qa[ks] = qr.frag(ks, 1.0f);
            ha[ks] = dr.frag(ks, 1.0f);
          }
          stash_transposed<T, DP>(tq, LD, m, qr, half);
          stash_transposed<T, DP>(th, LD, m, dr, half);
          if (half == 0) sq[m] = iq;
        }
        wave_lds_sync();
        float isq[16];
        read_row_scales(sq, half, isq);

        f32x16 s[2], dp[2];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int r = 0; r < 16; ++r) { s[kh][r] = 0.0f; dp[kh][r] = 0.0f; }
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
          for (int kh = 0; kh < 2; ++kh) {
            s[kh] = M::mma(qa[ks], kf[kh][ks], s[kh]);
            dp[kh] = M::mma(ha[ks], vf[kh][ks], dp[kh]);
          }
        // P (into s) and ds/|q| (into dp); register r -> query
        // q0 + 32qh + 16(r/8) + 8half + r%8, lane -> key k0 + 32kh + l32
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const int rel0 = (q0 + 32 * qh + 8 * half) - (k0 + 32 * kh + l32);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dd = rel0 + 16 * (r >> 3) + (r & 7);
            const float sv = s[kh][r] * isq[r] * ikl[kh];
            const float av = trim(sv, hp.r);
            const bool lv = av > 0.0f && in_window(dd, hp.wc, causal);
            float p = 0.0f, ds = 0.0f;
            if (__ballot(lv) != 0) {
              if (lv) {
                const float m = softmask(dd, hp.iw);
                const float g = dp[kh][r] * ivl[kh];
                p = av * av * m;
                ds = 2.0f * av * hp.r * m * g;
                dr_acc -= 2.0f * av * (1.0f - sv) * m * g;
                dw_acc += av * av * g * softmask_dw(dd, hp.iw);
              }
            }
            s[kh][r] = p;
            dp[kh][r] = ds * isq[r];
          }
        }
        // dv^T[d][j] += sum_i dh^T[d][i] P[i][j];  dk^T[d][j] += sum_i q^T[d][i] (ds/|q|)[i][j]
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int r0 = c * PER;
          const int ioff = rowof(r0, half);
#pragma unroll
          for (int dh_ = 0; dh_ < NDH; ++dh_) {
            const frag ht = M::load(&th[(32 * dh_ + l32) * LD + ioff]);
            const frag qT = M::load(&tq[(32 * dh_ + l32) * LD + ioff]);
#pragma unroll
            for (int kh = 0; kh < 2; ++kh) {
              adv[dh_][kh] = M::mma(ht, M::pack(s[kh], r0), adv[dh_][kh]);
              adk[dh_][kh] = M::mma(qT, M::pack(dp[kh], r0), adk[dh_][kh]);
            }
          }
        }
      }
    }
  }

  // Epilogue: dk^ = 1/|k| sum_i (ds/|q|) q and dv^ = 1/|v| ... -> fold the key's
  // own scale, then the normalisation backward; written to (B,Tk,H,D).
#pragma unroll
  for (int kh = 0; kh < 2; ++kh) {
    const int j = k0 + 32 * kh + l32;
    const bool valid = j < a.Tk;
    const int jj = valid ? j : 0;
    f32x16 accs[NDH];
    const int64_t orow = (((int64_t)b * a.Tk + jj) * a.H + h) * a.D;
#pragma unroll
    for (int dh_ = 0; dh_ < NDH; ++dh_) accs[dh_] = adk[dh_][kh];
    write_norm_bwd<T, NDH>(accs, (const T*)a.k + b * a.ks.sb + (int64_t)jj * a.ks.st + h * a.ks.sh, valid, a.D,
                           a.eps, half, (T*)a.dk + orow);
#pragma unroll
    for (int dh_ = 0; dh_ < NDH; ++dh_) accs[dh_] = adv[dh_][kh];
    write_norm_bwd<T, NDH>(accs, (const T*)a.v + b * a.vs.sb + (int64_t)jj * a.vs.st + h * a.vs.sh, valid, a.D,
                           a.eps, half, (T*)a.dv + orow);
  }
  dr_acc = wave_sum(dr_acc);
  dw_acc = wave_sum(dw_acc);
  if (lane == 0) {
    const int64_t nbh = (int64_t)a.B * a.H;
    a.part[(int64_t)bh * a.nkt + kt] = dr_acc;
    a.part[nbh * a.nkt + (int64_t)bh * a.nkt + kt] = dw_acc;
  }
}

// One wave (64-thread block) per 64-query tile of head (b,h); lane -> query
// i = q0 + 32*qh + l32.
template <typename T, int DP>
__global__ __launch_bounds__(64) void dq_kernel(BwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  constexpr int LD = LdsT<T>::LD;
  __shared__ __attribute__((aligned(16))) T tk[DP * LD];   // raw k^T [d][j]
  __shared__ __attribute__((aligned(16))) float sk[32];    // 1/|k_j| (0 if masked)
  __shared__ __attribute__((aligned(16))) float sv[32];    // 1/|v_j|
  const int lane = threadIdx.x, half = lane >> 5, l32 = lane & 31;
  int qt, bh;
  xcd_order(qt, bh);
  const int b = bh / a.H, h = bh % a.H;
  const HeadParams hp = head_params(a.r, a.w, h);
  const bool causal = a.causal != 0;
  const int q0 = qt * kTile;

  frag qb[2][NKS], hb[2][NKS];
  float iql[2];
#pragma unroll
  for (int qh = 0; qh < 2; ++qh) {
    Row<T, DP> qr, dr;
    query_rows<T, DP>(a, b, h, bh, q0 + 32 * qh + l32, half, qr, iql[qh], dr);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      qb[qh][ks] = qr.frag(ks, 1.0f);
      hb[qh][ks] = dr.frag(ks, 1.0f);
    }
  }
  f32x16 adq[NDH][2];
#pragma unroll
  for (int dh_ = 0; dh_ < NDH; ++dh_)
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int r = 0; r < 16; ++r) adq[dh_][qh][r] = 0.0f;

  const int64_t qlast = q0 + 63 < a.Tq - 1 ? q0 + 63 : a.Tq - 1;
  int64_t jlo = (int64_t)q0 - hp.wc + 1;
  int64_t jhi = causal ? qlast : qlast + hp.wc - 1;
  if (jlo < 0) jlo = 0;
  if (jhi > a.Tk - 1) jhi = a.Tk - 1;
  const int kt_lo = (int)(jlo / kTile), kt_hi = jhi >= jlo ? (int)(jhi / kTile) : kt_lo - 1;
  const uint32_t* brow = a.bits + ((int64_t)bh * a.nqt + qt) * a.nkt_words;

  for (int base = kt_lo; base <= kt_hi; base += kWave) {
    const int kl = base + lane;
    const bool bit = kl <= kt_hi && ((brow[kl >> 5] >> (kl & 31)) & 1u);
    unsigned long long mask = __ballot(bit);
    while (mask != 0ull) {
      const int kt = base + __builtin_ctzll(mask);
      mask &= mask - 1ull;
      const int k0 = kt * kTile;

      // one 32-key half of the key tile at a time
      for (int kh = 0; kh < 2; ++kh) {
        // key rows j = k0 + 32*kh + perm_row(l32) as A operands; k^T and the
        // key scales into LDS
        frag ka[NKS], va[NKS];
        wave_lds_sync();
        {
          const int m = perm_row(l32);
          Row<T, DP> kr, vr;
          float ik, iv;
          key_rows<T, DP>(a, b, h, k0 + 32 * kh + m, half, kr, ik, vr, iv);
#pragma unroll
          for (int ks = 0; ks < NKS; ++ks) {
            ka[ks] = kr.frag(ks, 1.0f);
            va[ks] = vr.frag(ks, 1.0f);
          }
          stash_transposed<T, DP>(tk, LD, m, kr, half);
          if (half == 0) { sk[m] = ik; sv[m] = iv; }
        }
        wave_lds_sync();
        float isk[16], isv[16];
        read_row_scales(sk, half, isk);
        read_row_scales(sv, half, isv);

        f32x16 s[2], dp[2];
#pragma unroll
        for (int qh = 0; qh < 2; ++qh)
#pragma unroll
          for (int r = 0; r < 16; ++r) { s[qh][r] = 0.0f; dp[qh][r] = 0.0f; }
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
          for (int qh = 0; qh < 2; ++qh) {
            s[qh] = M::mma(ka[ks], qb[qh][ks], s[qh]);
            dp[qh] = M::mma(va[ks], hb[qh][ks], dp[qh]);
          }
        // (ds/|k|)^T; register r -> key k0 + 32kh + 16(r/8) + 8half + r%8, lane -> query
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
          const int rel0 = (q0 + 32 * qh + l32) - (k0 + 32 * kh + 8 * half);
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int dd = rel0 - (16 * (r >> 3) + (r & 7));
            const float av = trim(s[qh][r] * isk[r] * iql[qh], hp.r);
            const bool lv = av > 0.0f && in_window(dd, hp.wc, causal);
            float ds = 0.0f;
            if (__ballot(lv) != 0) {
              if (lv) ds = 2.0f * av * hp.r * softmask(dd, hp.iw) * dp[qh][r] * isv[r];
            }
            dp[qh][r] = ds * isk[r];
          }
        }
        // dq^T[d][i] += sum_j k^T[d][j] (ds/|k|)^T[j][i]
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int r0 = c * PER;
          const int koff = rowof(r0, half);
#pragma unroll
          for (int dh_ = 0; dh_ < NDH; ++dh_) {
            const frag kT = M::load(&tk[(32 * dh_ + l32) * LD + koff]);
#pragma unroll
            for (int qh = 0; qh < 2; ++qh) adq[dh_][qh] = M::mma(kT, M::pack(dp[qh], r0), adq[dh_][qh]);
          }
        }
      }
    }
  }

#pragma unroll
  for (int qh = 0; qh < 2; ++qh) {
    const int i = q0 + 32 * qh + l32;
    const bool valid = i < a.Tq;
    const int ii = valid ? i : 0;
    f32x16 accs[NDH];
#pragma unroll
    for (int dh_ = 0; dh_ < NDH; ++dh_) accs[dh_] = adq[dh_][qh];
    write_norm_bwd<T, NDH>(accs, (const T*)a.q + b * a.qs.sb + (int64_t)ii * a.qs.st + h * a.qs.sh, valid, a.D,
                           a.eps, half, (T*)a.dq + (((int64_t)b * a.Tq + ii) * a.H + h) * a.D);
  }
}

// dr[h] = sum_{b,kt} part_r[b,h,kt]; dw likewise.  Block per head, fixed order.
__global__ __launch_bounds__(256) void rw_reduce_kernel(const float* part, float* dr, float* dw, int B, int H,
                                                        int nkt) {
  __shared__ float sr[256], sw[256];
  const int h = blockIdx.x;
  const int64_t nbh = (int64_t)B * H;
  float ar = 0.0f, aw = 0.0f;
  for (int64_t idx = threadIdx.x; idx < (int64_t)B * nkt; idx += 256) {
    const int b = (int)(idx / nkt), kt = (int)(idx % nkt);
    const int64_t o = ((int64_t)b * H + h) * nkt + kt;
    ar += part[o];
    aw += part[nbh * nkt + o];
  }
  sr[threadIdx.x] = ar;
  sw[threadIdx.x] = aw;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if ((int)threadIdx.x < s) {
      sr[threadIdx.x] += sr[threadIdx.x + s];
      sw[threadIdx.x] += sw[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) { dr[h] = sr[0]; dw[h] = sw[0]; }
}

size_t bwd_ws_bytes(const Geometry& g) {
  return round_up((int64_t)2 * g.B * g.H * g.nkt * (int64_t)sizeof(float), 256);
}

template <typename T, int DP>
static hipError_t launch_bwd_t(const BwdCall& c) {
  const Geometry& g = c.g;
  BwdKArgs ka;
  ka.q = c.q; ka.qs = c.qs; ka.k = c.k; ka.ks = c.ks; ka.v = c.v; ka.vs = c.vs; ka.kpm = c.kpm;
  ka.y = c.y; ka.dy = c.dy; ka.hnorm = c.hnorm;
  ka.r = c.r; ka.w = c.w; ka.bits = c.bits;
  ka.dq = c.dq; ka.dk = c.dk; ka.dv = c.dv; ka.part = c.part;
  ka.B = g.B; ka.H = g.H; ka.Tq = g.Tq; ka.Tk = g.Tk; ka.D = g.D;
  ka.nqt = g.nqt; ka.nkt = g.nkt; ka.nkt_words = g.nkt_words; ka.causal = g.causal;
  ka.eps = c.eps;
  timer_begin(4, c.stream);
  hipLaunchKernelGGL((dkdv_kernel<T, DP>), dim3((unsigned)g.nkt, (unsigned)(g.B * g.H)), dim3(64), 0, c.stream, ka);
  timer_end(4, c.stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(5, c.stream);
  hipLaunchKernelGGL((dq_kernel<T, DP>), dim3((unsigned)g.nqt, (unsigned)(g.B * g.H)), dim3(64), 0, c.stream, ka);
  timer_end(5, c.stream);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(6, c.stream);
  hipLaunchKernelGGL(rw_reduce_kernel, dim3((unsigned)g.H), dim3(256), 0, c.stream, (const float*)c.part, c.dr, c.dw,
                     g.B, g.H, g.nkt);
  timer_end(6, c.stream);
  return hipGetLastError();
}

hipError_t launch_bwd(const BwdCall& c) {
  const int DP = c.g.DP;
  if (c.g.dtype == 1) {
    if (DP == 32) return launch_bwd_t<bf16, 32>(c);
    if (DP == 64) return launch_bwd_t<bf16, 64>(c);
    return launch_bwd_t<bf16, 128>(c);
  }
  if (DP == 32) return launch_bwd_t<float, 32>(c);
  if (DP == 64) return launch_bwd_t<float, 64>(c);
  return launch_bwd_t<float, 128>(c);
}

}  // namespace msa
