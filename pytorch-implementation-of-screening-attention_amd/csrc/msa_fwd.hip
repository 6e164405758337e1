// Forward path of fused Screening Attention on gfx950.
//
//   prep_kv_kernel : one pass over the raw k/v projections -> unit-normalised
//                    K^ and V^ in the layouts the MFMA operands read
//                    (attention.py:155-158), key padding folded in as a zero
//                    K^ row (attention.py:185-188: s=0 gives alpha=0 since r>1).
//   fwd_kernel     : one wave per 64-query tile.  For every key tile of the
//                    causal window it forms S^T = K^ Q^T on MFMA (fp32
//                    accumulation), scales by 1/|q_i|, and decides with one
//                    wave ballot whether any in-window pair passes the
//                    trim-and-square threshold (attention.py:75-90).  Only
//                    such tiles compute alpha*m (attention.py:92-119) and
//                    accumulate H^T += V^T P^T on MFMA; the epilogue applies
//                    TanhNorm (norm.py:23-25) and writes y in (B,T,H,D).
//                    The T x T matrices are never materialised.
#include "msa_device.h"
#include "msa_internal.h"

namespace msa {

struct PrepKvArgs {
  const void* k; Strides3 ks;
  const void* v; Strides3 vs;
  const uint8_t* kpm;
  void* khat; void* vhatT; void* khatT; void* vhat;
  int H, Tk, D;
  int64_t Tk_pad;
  float eps;
};

// One thread per key row t of one (b,h); grid (Tk_pad/64, B*H), block 64.
template <typename T, int DP>
__global__ __launch_bounds__(64) void prep_kv_kernel(PrepKvArgs a) {
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int64_t t = (int64_t)blockIdx.x * 64 + threadIdx.x;
  const bool valid = t < a.Tk;
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    const T* src = (const T*)(which == 0 ? a.k : a.v);
    const Strides3 st = which == 0 ? a.ks : a.vs;
    float x[DP];
    float ss = 0.0f;
#pragma unroll
    for (int d = 0; d < DP; d += 4) {
      f32x4 v4 = {0.f, 0.f, 0.f, 0.f};
      if (valid && d < a.D) v4 = load4(src + b * st.sb + t * st.st + h * st.sh + d);
      x[d] = v4[0]; x[d + 1] = v4[1]; x[d + 2] = v4[2]; x[d + 3] = v4[3];
      ss += v4[0] * v4[0] + v4[1] * v4[1] + v4[2] * v4[2] + v4[3] * v4[3];
    }
    float inv = 1.0f / fmaxf(sqrtf(ss), a.eps);
    if (which == 0 && a.kpm != nullptr && valid && a.kpm[(int64_t)b * a.Tk + t]) inv = 0.0f;
    if (!valid) inv = 0.0f;
    T* row = (T*)(which == 0 ? a.khat : a.vhat);
    T* col = (T*)(which == 0 ? a.khatT : a.vhatT);
    if (row != nullptr) {
      T* p = row + ((int64_t)bh * a.Tk_pad + t) * DP;
#pragma unroll
      for (int d = 0; d < DP; d += 4) store4(p + d, x[d] * inv, x[d + 1] * inv, x[d + 2] * inv, x[d + 3] * inv);
    }
    if (col != nullptr) {
      T* p = col + (int64_t)bh * DP * a.Tk_pad + t;
#pragma unroll
      for (int d = 0; d < DP; ++d) p[(int64_t)d * a.Tk_pad] = from_f<T>(x[d] * inv);
    }
  }
}

struct FwdKArgs {
  const void* q; Strides3 qs;
  const void* khat; const void* vhatT;
  const float* r; const float* w;
  void* y; float* hnorm; uint32_t* bits;
  int H, Tq, Tk, D, nqt, nkt_words, causal;
  int64_t Tk_pad;
  float eps;
};

// Four independent waves per block; wave -> 64-query tile qt of head (b,h).
template <typename T, int DP>
__global__ __launch_bounds__(256) void fwd_kernel(FwdKArgs a) {
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

  // Q^T as the B operand: lane -> query q0+32*qh+l32, slots -> d.
  frag qf[2][NKS];
  float iq[2];
  {
    const T* q = (const T*)a.q;
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
      const int i = q0 + 32 * qh + l32;
      const bool ok = i < a.Tq;
      const T* qrow = q + b * a.qs.sb + (int64_t)(ok ? i : 0) * a.qs.st + h * a.qs.sh;
      float ss = 0.0f;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        const int d0 = KS * ks + PER * half;
        qf[qh][ks] = load_or_zero<T>(qrow + d0, ok && d0 < a.D);
#pragma unroll
        for (int e = 0; e < PER; ++e) { float x = M::get(qf[qh][ks], e); ss += x * x; }
      }
      ss += __shfl_xor(ss, 32);
      iq[qh] = 1.0f / fmaxf(sqrtf(ss), a.eps);
    }
  }

  // Key-tile range of the window of this query tile.
  const int64_t qlast = q0 + 63 < a.Tq - 1 ? q0 + 63 : a.Tq - 1;
  int64_t jlo = (int64_t)q0 - hp.wc + 1;
  int64_t jhi = causal ? qlast : qlast + hp.wc - 1;
  if (jlo < 0) jlo = 0;
  if (jhi > a.Tk - 1) jhi = a.Tk - 1;
  const int kt_lo = (int)(jlo / kTile), kt_hi = jhi >= jlo ? (int)(jhi / kTile) : kt_lo - 1;

  uint32_t* brow = a.bits + ((int64_t)bh * a.nqt + qt) * a.nkt_words;
  for (int wi = lane; wi < a.nkt_words; wi += kWave)
    if (kt_hi < kt_lo || wi < (kt_lo >> 5) || wi > (kt_hi >> 5)) brow[wi] = 0u;

  f32x16 o[NDH][2];
#pragma unroll
  for (int dh = 0; dh < NDH; ++dh)
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dh][qh][r] = 0.0f;

  const T* kb = (const T*)a.khat + (int64_t)bh * a.Tk_pad * DP;
  const T* vt = (const T*)a.vhatT + (int64_t)bh * DP * a.Tk_pad;
  uint32_t word = 0u;

  for (int kt = kt_lo; kt <= kt_hi; ++kt) {
    const int k0 = kt * kTile;
    f32x16 acc[2][2];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh)
#pragma unroll
      for (int qh = 0; qh < 2; ++qh)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[kh][qh][r] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        const frag kf = M::load(kb + (int64_t)(k0 + 32 * kh + perm_row(l32)) * DP + KS * ks + PER * half);
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) acc[kh][qh] = M::mma(kf, qf[qh][ks], acc[kh][qh]);
      }
    }

    // Threshold vote.  a(s) is monotone in s and s = acc/|q_i| is monotone in
    // acc, so the tile has a live pair iff the largest in-window acc passes.
    const bool interior = causal ? (k0 + 63 <= q0 && (int64_t)(q0 + 63 - k0) < hp.wc)
                                 : ((int64_t)(q0 + 63 - k0) < hp.wc && (int64_t)(k0 + 63 - q0) < hp.wc);
    bool live = false;
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
      float mx = -INFINITY;
      if (interior) {
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, acc[kh][qh][r]);
      } else {
        const int i = q0 + 32 * qh + l32;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int j = k0 + 32 * kh + rowof(r, half);
            if (in_window((int64_t)i - j, hp.wc, causal)) mx = fmaxf(mx, acc[kh][qh][r]);
          }
      }
      live |= trim(mx * iq[qh], hp.r) > 0.0f;
    }

    if (__ballot(live) != 0) {
      word |= 1u << (kt & 31);
      // P^T[j][i] = alpha_ij * m_ij, in place of S^T.
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
          const int i = q0 + 32 * qh + l32;
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const int j = k0 + 32 * kh + rowof(r, half);
            const int64_t dd = (int64_t)i - j;
            const float av = trim(acc[kh][qh][r] * iq[qh], hp.r);
            float p = 0.0f;
            if (av > 0.0f && in_window(dd, hp.wc, causal)) p = av * av * softmask(dd, hp.iw);
            acc[kh][qh][r] = p;
          }
        }
      // H^T[d][i] += sum_j V^T[d][j] P^T[j][i]
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int r0 = c * PER;
          const int koff = k0 + 32 * kh + rowof(r0, half);
          frag vf[NDH];
#pragma unroll
          for (int dh = 0; dh < NDH; ++dh) vf[dh] = M::load(vt + (int64_t)(32 * dh + l32) * a.Tk_pad + koff);
#pragma unroll
          for (int qh = 0; qh < 2; ++qh) {
            const frag pf = M::pack(acc[kh][qh], r0);
#pragma unroll
            for (int dh = 0; dh < NDH; ++dh) o[dh][qh] = M::mma(vf[dh], pf, o[dh][qh]);
          }
        }
    }
    if ((kt & 31) == 31 || kt == kt_hi) {
      if (lane == 0) brow[kt >> 5] = word;
      word = 0u;
    }
  }

  // Epilogue: TanhNorm per query row, y written in (B,T,H,D).
  T* y = (T*)a.y;
#pragma unroll
  for (int qh = 0; qh < 2; ++qh) {
    float ss = 0.0f;
#pragma unroll
    for (int dh = 0; dh < NDH; ++dh)
#pragma unroll
      for (int r = 0; r < 16; ++r) ss += o[dh][qh][r] * o[dh][qh][r];
    ss += __shfl_xor(ss, 32);
    const float n = sqrtf(ss);
    const float nc = fmaxf(n, a.eps);
    const float f = tanhf(nc) / nc;
    const int i = q0 + 32 * qh + l32;
    if (i < a.Tq) {
      if (half == 0) a.hnorm[(int64_t)bh * a.Tq + i] = n;
      T* yrow = y + (((int64_t)b * a.Tq + i) * a.H + h) * a.D;
#pragma unroll
      for (int dh = 0; dh < NDH; ++dh)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * dh + 8 * g + 4 * half;
          if (d < a.D)
            store4(yrow + d, f * o[dh][qh][4 * g], f * o[dh][qh][4 * g + 1], f * o[dh][qh][4 * g + 2],
                   f * o[dh][qh][4 * g + 3]);
        }
    }
  }
}

size_t fwd_ws_bytes(const Geometry& g, int need_bwd) {
  const size_t one = (size_t)g.B * g.H * g.Tk_pad * g.DP * g.esize;
  return one * (need_bwd ? 4 : 2);
}

FwdWs fwd_ws_carve(const Geometry& g, void* base, int need_bwd) {
  const size_t one = (size_t)g.B * g.H * g.Tk_pad * g.DP * g.esize;
  char* p = (char*)base;
  FwdWs ws;
  ws.khat = p;
  ws.vhatT = p + one;
  ws.khatT = need_bwd ? p + 2 * one : nullptr;
  ws.vhat = need_bwd ? p + 3 * one : nullptr;
  return ws;
}

template <typename T, int DP>
static hipError_t launch_fwd_t(const FwdCall& c) {
  const Geometry& g = c.g;
  PrepKvArgs pa;
  pa.k = c.k; pa.ks = c.ks; pa.v = c.v; pa.vs = c.vs; pa.kpm = c.kpm;
  pa.khat = c.ws.khat; pa.vhatT = c.ws.vhatT; pa.khatT = c.ws.khatT; pa.vhat = c.ws.vhat;
  pa.H = g.H; pa.Tk = g.Tk; pa.D = g.D; pa.Tk_pad = g.Tk_pad; pa.eps = c.eps;
  if (g.Tk_pad > 0) {
    timer_begin(1, c.stream);
    hipLaunchKernelGGL((prep_kv_kernel<T, DP>), dim3((unsigned)(g.Tk_pad / 64), (unsigned)(g.B * g.H)), dim3(64), 0,
                       c.stream, pa);
    timer_end(1, c.stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }

  FwdKArgs fa;
  fa.q = c.q; fa.qs = c.qs; fa.khat = c.ws.khat; fa.vhatT = c.ws.vhatT;
  fa.r = c.r; fa.w = c.w; fa.y = c.y; fa.hnorm = c.hnorm; fa.bits = c.bits;
  fa.H = g.H; fa.Tq = g.Tq; fa.Tk = g.Tk; fa.D = g.D; fa.nqt = g.nqt; fa.nkt_words = g.nkt_words;
  fa.causal = g.causal; fa.Tk_pad = g.Tk_pad; fa.eps = c.eps;
  timer_begin(2, c.stream);
  hipLaunchKernelGGL((fwd_kernel<T, DP>), dim3((unsigned)((g.nqt + 3) / 4), (unsigned)(g.B * g.H)), dim3(256), 0,
                     c.stream, fa);
  timer_end(2, c.stream);
  return hipGetLastError();
}

hipError_t launch_fwd(const FwdCall& c) {
  const int DP = c.g.DP;
  if (c.g.dtype == 1) {
    if (DP == 32) return launch_fwd_t<bf16, 32>(c);
    if (DP == 64) return launch_fwd_t<bf16, 64>(c);
    return launch_fwd_t<bf16, 128>(c);
  }
  if (DP == 32) return launch_fwd_t<float, 32>(c);
  if (DP == 64) return launch_fwd_t<float, 64>(c);
  return launch_fwd_t<float, 128>(c);
}

}  // namespace msa
