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
// Only tiles the forward marked live in its bitmap are revisited.
//
//   bwd_prep_kernel : per query row: q^ (row + transposed copies) and dh.
//   dkdv_kernel     : wave per 64-key tile, loops over live query tiles;
//                     accumulates dv^, dk^ in MFMA registers, writes dk, dv
//                     and one (dr, dw) partial per wave.
//   dq_kernel       : wave per 64-query tile, loops over live key tiles.
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

struct BwdPrepArgs {
  const void* q; Strides3 qs;
  const void* y; const void* dy; const float* hnorm;
  void* qhat; void* qhatT; void* dh; void* dhT;
  int H, Tq, D;
  int64_t Tq_pad;
  float eps;
};

// One thread per query row; grid (Tq_pad/64, B*H), block 64.
template <typename T, int DP>
__global__ __launch_bounds__(64) void bwd_prep_kernel(BwdPrepArgs a) {
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int64_t i = (int64_t)blockIdx.x * 64 + threadIdx.x;
  const bool valid = i < a.Tq;
  float x[DP];
  {
    const T* src = (const T*)a.q;
    float ss = 0.0f;
#pragma unroll
    for (int d = 0; d < DP; d += 4) {
      f32x4 v4 = {0.f, 0.f, 0.f, 0.f};
      if (valid && d < a.D) v4 = load4(src + b * a.qs.sb + i * a.qs.st + h * a.qs.sh + d);
      x[d] = v4[0]; x[d + 1] = v4[1]; x[d + 2] = v4[2]; x[d + 3] = v4[3];
      ss += v4[0] * v4[0] + v4[1] * v4[1] + v4[2] * v4[2] + v4[3] * v4[3];
    }
    const float inv = valid ? 1.0f / fmaxf(sqrtf(ss), a.eps) : 0.0f;
    T* row = (T*)a.qhat + ((int64_t)bh * a.Tq_pad + i) * DP;
    T* col = (T*)a.qhatT + (int64_t)bh * DP * a.Tq_pad + i;
#pragma unroll
    for (int d = 0; d < DP; d += 4) store4(row + d, x[d] * inv, x[d + 1] * inv, x[d + 2] * inv, x[d + 3] * inv);
#pragma unroll
    for (int d = 0; d < DP; ++d) col[(int64_t)d * a.Tq_pad] = from_f<T>(x[d] * inv);
  }
  {
    const T* yp = (const T*)a.y + (((int64_t)b * a.Tq + (valid ? i : 0)) * a.H + h) * a.D;
    const T* gp = (const T*)a.dy + (((int64_t)b * a.Tq + (valid ? i : 0)) * a.H + h) * a.D;
    float yv[DP];
    float ydot = 0.0f;
#pragma unroll
    for (int d = 0; d < DP; d += 4) {
      f32x4 y4 = {0.f, 0.f, 0.f, 0.f}, g4 = {0.f, 0.f, 0.f, 0.f};
      if (valid && d < a.D) { y4 = load4(yp + d); g4 = load4(gp + d); }
#pragma unroll
      for (int e = 0; e < 4; ++e) { yv[d + e] = y4[e]; x[d + e] = g4[e]; ydot += y4[e] * g4[e]; }
    }
    const float n = valid ? a.hnorm[(int64_t)bh * a.Tq + i] : 0.0f;
    // dh = F dy + G (h.dy) h with h = y/F  ->  dh = F dy + (G/F^2)(y.dy) y
    float c1, c2;
    if (n > a.eps) {
      const float t = tanhf(n);
      c1 = t / n;
      c2 = tanhnorm_g(n, t) / (c1 * c1);
    } else {
      c1 = tanhf(a.eps) / a.eps;
      c2 = 0.0f;
    }
    const float cy = c2 * ydot;
    T* row = (T*)a.dh + ((int64_t)bh * a.Tq_pad + i) * DP;
    T* col = (T*)a.dhT + (int64_t)bh * DP * a.Tq_pad + i;
#pragma unroll
    for (int d = 0; d < DP; ++d) x[d] = c1 * x[d] + cy * yv[d];
#pragma unroll
    for (int d = 0; d < DP; d += 4) store4(row + d, x[d], x[d + 1], x[d + 2], x[d + 3]);
#pragma unroll
    for (int d = 0; d < DP; ++d) col[(int64_t)d * a.Tq_pad] = from_f<T>(x[d]);
  }
}

struct BwdKArgs {
  const void* q; Strides3 qs;
  const void* k; Strides3 ks;
  const void* v; Strides3 vs;
  const float* r; const float* w;
  const uint32_t* bits;
  const void* khat; const void* khatT; const void* vhat;
  const void* qhat; const void* qhatT; const void* dh; const void* dhT;
  void* dq; void* dk; void* dv; float* part;
  int B, H, Tq, Tk, D, nqt, nkt, nkt_words, causal;
  int64_t Tq_pad, Tk_pad;
  float eps;
};

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

// Wave per 64-key tile kt of head (b,h); lane -> key j = k0 + 32*kh + l32.
template <typename T, int DP>
__global__ __launch_bounds__(256) void dkdv_kernel(BwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int kt = blockIdx.x * 4 + wave;
  if (kt >= a.nkt) return;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const HeadParams hp = head_params(a.r, a.w, h);
  const bool causal = a.causal != 0;
  const int k0 = kt * kTile;

  const T* khat = (const T*)a.khat + (int64_t)bh * a.Tk_pad * DP;
  const T* vhat = (const T*)a.vhat + (int64_t)bh * a.Tk_pad * DP;
  const T* qhat = (const T*)a.qhat + (int64_t)bh * a.Tq_pad * DP;
  const T* dh = (const T*)a.dh + (int64_t)bh * a.Tq_pad * DP;
  const T* qhatT = (const T*)a.qhatT + (int64_t)bh * DP * a.Tq_pad;
  const T* dhT = (const T*)a.dhT + (int64_t)bh * DP * a.Tq_pad;

  frag kf[2][NKS], vf[2][NKS];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int64_t off = (int64_t)(k0 + 32 * kh + l32) * DP + KS * ks + PER * half;
      kf[kh][ks] = M::load(khat + off);
      vf[kh][ks] = M::load(vhat + off);
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

  for (int qt = qt_lo; qt <= qt_hi; ++qt) {
    const uint32_t word = a.bits[((int64_t)bh * a.nqt + qt) * a.nkt_words + (kt >> 5)];
    if (((word >> (kt & 31)) & 1u) == 0u) continue;
    const int q0 = qt * kTile;
    f32x16 s[2][2], dp[2][2];
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int r = 0; r < 16; ++r) { s[qh][kh][r] = 0.0f; dp[qh][kh][r] = 0.0f; }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        const int64_t off = (int64_t)(q0 + 32 * qh + perm_row(l32)) * DP + KS * ks + PER * half;
        const frag qa = M::load(qhat + off);
        const frag ha = M::load(dh + off);
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          s[qh][kh] = M::mma(qa, kf[kh][ks], s[qh][kh]);
          dp[qh][kh] = M::mma(ha, vf[kh][ks], dp[qh][kh]);
        }
      }
    // pair weights P (into s) and ds (into dp)
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        const int j = k0 + 32 * kh + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int i = q0 + 32 * qh + rowof(r, half);
          const int64_t dd = (int64_t)i - j;
          const float sv = s[qh][kh][r];
          const float av = trim(sv, hp.r);
          float p = 0.0f, ds = 0.0f;
          if (av > 0.0f && in_window(dd, hp.wc, causal)) {
            const float m = softmask(dd, hp.iw);
            const float g = dp[qh][kh][r];
            p = av * av * m;
            ds = 2.0f * av * hp.r * m * g;
            dr_acc -= 2.0f * av * (1.0f - sv) * m * g;
            dw_acc += av * av * g * softmask_dw(dd, hp.iw);
          }
          s[qh][kh][r] = p;
          dp[qh][kh][r] = ds;
        }
      }
    // dv^T[d][j] += sum_i dh^T[d][i] P[i][j];  dk^T[d][j] += sum_i q^T[d][i] ds[i][j]
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int r0 = c * PER;
        const int ioff = q0 + 32 * qh + rowof(r0, half);
        frag ht[NDH], qT[NDH];
#pragma unroll
        for (int dh_ = 0; dh_ < NDH; ++dh_) {
          ht[dh_] = M::load(dhT + (int64_t)(32 * dh_ + l32) * a.Tq_pad + ioff);
          qT[dh_] = M::load(qhatT + (int64_t)(32 * dh_ + l32) * a.Tq_pad + ioff);
        }
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const frag pb = M::pack(s[qh][kh], r0);
          const frag sb = M::pack(dp[qh][kh], r0);
#pragma unroll
          for (int dh_ = 0; dh_ < NDH; ++dh_) {
            adv[dh_][kh] = M::mma(ht[dh_], pb, adv[dh_][kh]);
            adk[dh_][kh] = M::mma(qT[dh_], sb, adk[dh_][kh]);
          }
        }
      }
  }

  // Epilogue: normalisation backward for k and v, written to (B,Tk,H,D).
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

// Wave per 64-query tile qt of head (b,h); lane -> query i = q0 + 32*qh + l32.
template <typename T, int DP>
__global__ __launch_bounds__(256) void dq_kernel(BwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int qt = blockIdx.x * 4 + wave;
  if (qt >= a.nqt) return;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const HeadParams hp = head_params(a.r, a.w, h);
  const bool causal = a.causal != 0;
  const int q0 = qt * kTile;

  const T* khat = (const T*)a.khat + (int64_t)bh * a.Tk_pad * DP;
  const T* vhat = (const T*)a.vhat + (int64_t)bh * a.Tk_pad * DP;
  const T* khatT = (const T*)a.khatT + (int64_t)bh * DP * a.Tk_pad;
  const T* qhat = (const T*)a.qhat + (int64_t)bh * a.Tq_pad * DP;
  const T* dh = (const T*)a.dh + (int64_t)bh * a.Tq_pad * DP;

  frag qb[2][NKS], hb[2][NKS];
#pragma unroll
  for (int qh = 0; qh < 2; ++qh)
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int64_t off = (int64_t)(q0 + 32 * qh + l32) * DP + KS * ks + PER * half;
      qb[qh][ks] = M::load(qhat + off);
      hb[qh][ks] = M::load(dh + off);
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

  for (int kt = kt_lo; kt <= kt_hi; ++kt) {
    if (((brow[kt >> 5] >> (kt & 31)) & 1u) == 0u) continue;
    const int k0 = kt * kTile;
    f32x16 s[2][2], dp[2][2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int qh = 0; qh < 2; ++qh)
#pragma unroll
        for (int r = 0; r < 16; ++r) { s[kh][qh][r] = 0.0f; dp[kh][qh][r] = 0.0f; }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        const int64_t off = (int64_t)(k0 + 32 * kh + perm_row(l32)) * DP + KS * ks + PER * half;
        const frag ka = M::load(khat + off);
        const frag va = M::load(vhat + off);
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
          s[kh][qh] = M::mma(ka, qb[qh][ks], s[kh][qh]);
          dp[kh][qh] = M::mma(va, hb[qh][ks], dp[kh][qh]);
        }
      }
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        const int i = q0 + 32 * qh + l32;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int j = k0 + 32 * kh + rowof(r, half);
          const int64_t dd = (int64_t)i - j;
          const float av = trim(s[kh][qh][r], hp.r);
          float ds = 0.0f;
          if (av > 0.0f && in_window(dd, hp.wc, causal))
            ds = 2.0f * av * hp.r * softmask(dd, hp.iw) * dp[kh][qh][r];
          dp[kh][qh][r] = ds;
        }
      }
    // dq^T[d][i] += sum_j k^T[d][j] ds^T[j][i]
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int r0 = c * PER;
        const int koff = k0 + 32 * kh + rowof(r0, half);
        frag kT[NDH];
#pragma unroll
        for (int dh_ = 0; dh_ < NDH; ++dh_) kT[dh_] = M::load(khatT + (int64_t)(32 * dh_ + l32) * a.Tk_pad + koff);
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
          const frag sb = M::pack(dp[kh][qh], r0);
#pragma unroll
          for (int dh_ = 0; dh_ < NDH; ++dh_) adq[dh_][qh] = M::mma(kT[dh_], sb, adq[dh_][qh]);
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
  const size_t one = (size_t)g.B * g.H * g.Tq_pad * g.DP * g.esize;
  const size_t part = (size_t)2 * g.B * g.H * g.nkt * sizeof(float);
  return 4 * one + round_up((int64_t)part, 256);
}

BwdWs bwd_ws_carve(const Geometry& g, void* base) {
  const size_t one = (size_t)g.B * g.H * g.Tq_pad * g.DP * g.esize;
  char* p = (char*)base;
  BwdWs ws;
  ws.qhat = p;
  ws.qhatT = p + one;
  ws.dh = p + 2 * one;
  ws.dhT = p + 3 * one;
  ws.part = (float*)(p + 4 * one);
  return ws;
}

template <typename T, int DP>
static hipError_t launch_bwd_t(const BwdCall& c) {
  const Geometry& g = c.g;
  BwdPrepArgs pa;
  pa.q = c.q; pa.qs = c.qs; pa.y = c.y; pa.dy = c.dy; pa.hnorm = c.hnorm;
  pa.qhat = c.bws.qhat; pa.qhatT = c.bws.qhatT; pa.dh = c.bws.dh; pa.dhT = c.bws.dhT;
  pa.H = g.H; pa.Tq = g.Tq; pa.D = g.D; pa.Tq_pad = g.Tq_pad; pa.eps = c.eps;
  timer_begin(3, c.stream);
  hipLaunchKernelGGL((bwd_prep_kernel<T, DP>), dim3((unsigned)(g.Tq_pad / 64), (unsigned)(g.B * g.H)), dim3(64), 0,
                     c.stream, pa);
  timer_end(3, c.stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;

  BwdKArgs ka;
  ka.q = c.q; ka.qs = c.qs; ka.k = c.k; ka.ks = c.ks; ka.v = c.v; ka.vs = c.vs;
  ka.r = c.r; ka.w = c.w; ka.bits = c.bits;
  ka.khat = c.fws.khat; ka.khatT = c.fws.khatT; ka.vhat = c.fws.vhat;
  ka.qhat = c.bws.qhat; ka.qhatT = c.bws.qhatT; ka.dh = c.bws.dh; ka.dhT = c.bws.dhT;
  ka.dq = c.dq; ka.dk = c.dk; ka.dv = c.dv; ka.part = c.bws.part;
  ka.B = g.B; ka.H = g.H; ka.Tq = g.Tq; ka.Tk = g.Tk; ka.D = g.D;
  ka.nqt = g.nqt; ka.nkt = g.nkt; ka.nkt_words = g.nkt_words; ka.causal = g.causal;
  ka.Tq_pad = g.Tq_pad; ka.Tk_pad = g.Tk_pad; ka.eps = c.eps;
  timer_begin(4, c.stream);
  hipLaunchKernelGGL((dkdv_kernel<T, DP>), dim3((unsigned)((g.nkt + 3) / 4), (unsigned)(g.B * g.H)), dim3(256), 0,
                     c.stream, ka);
  timer_end(4, c.stream);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(5, c.stream);
  hipLaunchKernelGGL((dq_kernel<T, DP>), dim3((unsigned)((g.nqt + 3) / 4), (unsigned)(g.B * g.H)), dim3(256), 0,
                     c.stream, ka);
  timer_end(5, c.stream);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(6, c.stream);
  hipLaunchKernelGGL(rw_reduce_kernel, dim3((unsigned)g.H), dim3(256), 0, c.stream, (const float*)c.bws.part, c.dr,
                     c.dw, g.B, g.H, g.nkt);
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
