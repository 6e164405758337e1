// Forward path of fused Screening Attention on gfx950.
//
//   prep_k_kernel : unit-normalised K^ rows (attention.py:156-157) in a padded
//                   [b*h][Tk_pad][DP] buffer; key padding (attention.py:185-188)
//                   is folded in as a zero row (s = 0 gives alpha = 0: r > 1).
//   fwd_kernel    : 256-thread block = 4 waves, wave -> one 64-query tile of
//                   one head.  Key tiles of the block's window are staged in LDS
//                   (double-buffered, one tile ahead) and shared by the 4 waves.
//                   Each wave forms S^T = K^ Q^T on MFMA (raw bf16 Q, fp32
//                   accumulation, scaled by 1/|q_i|) and votes, with a wave
//                   ballot, whether any in-window pair passes the trim-and-square
//                   threshold (attention.py:75-90).  Only then does the block
//                   stage the normalised V^T tile and the live waves compute
//                   alpha*m (attention.py:92-119) and accumulate H^T += V^T P^T.
//                   The epilogue applies TanhNorm (norm.py:23-25) and writes y
//                   in (B,T,H,D), |h| per row and the live-tile bitmap.
//                   No T x T matrix is ever materialised.
#include "msa_device.h"
#include "msa_internal.h"

namespace msa {

struct PrepKArgs {
  const void* k; Strides3 ks;
  const uint8_t* kpm;
  void* khat;
  int H, Tk, D;
  int64_t Tk_pad;
  float eps;
};

// 16-byte chunk per thread; a key row of DP elements spans CPR threads.
template <typename T, int DP>
__global__ __launch_bounds__(256) void prep_k_kernel(PrepKArgs a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int CPR = DP / VEC;  // chunks per row (power of two, <= 32)
  constexpr int RPB = 256 / CPR;
  const int bh = blockIdx.y, b = bh / a.H, h = bh % a.H;
  const int64_t t = (int64_t)blockIdx.x * RPB + threadIdx.x / CPR;
  const int d0 = (threadIdx.x % CPR) * VEC;
  const bool valid = t < a.Tk && d0 < a.D;
  float x[VEC];
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < VEC; e += 4) {
    f32x4 v4 = {0.f, 0.f, 0.f, 0.f};
    if (valid) v4 = load4((const T*)a.k + b * a.ks.sb + t * a.ks.st + h * a.ks.sh + d0 + e);
    x[e] = v4[0]; x[e + 1] = v4[1]; x[e + 2] = v4[2]; x[e + 3] = v4[3];
    ss += v4[0] * v4[0] + v4[1] * v4[1] + v4[2] * v4[2] + v4[3] * v4[3];
  }
#pragma unroll
  for (int o = 1; o < CPR; o <<= 1) ss += __shfl_xor(ss, o);
  float inv = 1.0f / fmaxf(sqrtf(ss), a.eps);
  if (t >= a.Tk || (a.kpm != nullptr && a.kpm[(int64_t)b * a.Tk + t])) inv = 0.0f;
  if (t < a.Tk_pad) {
    T* p = (T*)a.khat + ((int64_t)bh * a.Tk_pad + t) * DP + d0;
#pragma unroll
    for (int e = 0; e < VEC; e += 4) store4(p + e, x[e] * inv, x[e + 1] * inv, x[e + 2] * inv, x[e + 3] * inv);
  }
}

struct FwdKArgs {
  const void* q; Strides3 qs;
  const void* v; Strides3 vs;
  const void* khat;
  const float* r; const float* w;
  void* y; float* hnorm; uint32_t* bits;
  int H, Tq, Tk, D, nqt, nkt_words, causal;
  int64_t Tk_pad;
  float eps;
};

template <typename T, int DP>
struct FwdTile {
  static constexpr int PAD = 16 / (int)sizeof(T);  // 16-byte row padding
  static constexpr int LDK = DP + PAD;              // K^ tile row pitch (elements)
  static constexpr int LDV = 64 + PAD;              // V^T tile row pitch
  static constexpr int CHUNKS = 64 * DP * (int)sizeof(T) / 16;  // 16-byte chunks per K tile
  static constexpr int CPT = CHUNKS / 256;                      // per thread
  static constexpr int CPR = DP * (int)sizeof(T) / 16;          // per row
};

template <typename T, int DP>
__global__ __launch_bounds__(256, 2) void fwd_kernel(FwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  using G = FwdTile<T, DP>;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
  __shared__ __attribute__((aligned(16))) T kl[2][64 * G::LDK];
  __shared__ __attribute__((aligned(16))) T vl[DP * G::LDV];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  int bx, bh;
  xcd_order(bx, bh);
  const int b = bh / a.H, h = bh % a.H;
  const HeadParams hp = head_params(a.r, a.w, h);
  const bool causal = a.causal != 0;
  const int qt = bx * 4 + wave;
  const bool wave_ok = qt < a.nqt;
  const int q0 = qt * kTile;

  // Q^T as the B operand: lane -> query q0+32*qh+l32, slots -> d (raw values).
  frag qf[2][NKS];
  float iq[2];
#pragma unroll
  for (int qh = 0; qh < 2; ++qh) {
    const int i = q0 + 32 * qh + l32;
    const bool ok = wave_ok && i < a.Tq;
    Row<T, DP> row;
    row.load((const T*)a.q + b * a.qs.sb + (int64_t)(ok ? i : 0) * a.qs.st + h * a.qs.sh, ok, a.D, half);
    iq[qh] = row.inv_norm(a.eps);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qf[qh][ks] = row.frag(ks, 1.0f);
  }

  // Key-tile ranges: this wave's, and the block's union.
  auto krange = [&](int64_t qa, int64_t qb, int& lo, int& hi) {
    int64_t jlo = qa - hp.wc + 1;
    int64_t jhi = causal ? qb : qb + hp.wc - 1;
    if (jlo < 0) jlo = 0;
    if (jhi > a.Tk - 1) jhi = a.Tk - 1;
    lo = (int)(jlo / kTile);
    hi = jhi >= jlo ? (int)(jhi / kTile) : lo - 1;
  };
  int kt_lo, kt_hi, blo, bhi;
  {
    const int64_t qlast = q0 + 63 < a.Tq - 1 ? q0 + 63 : a.Tq - 1;
    krange(q0, qlast, kt_lo, kt_hi);
    if (!wave_ok) { kt_lo = 0; kt_hi = -1; }
    const int64_t bq0 = (int64_t)bx * 4 * kTile;
    const int64_t bq1 = bq0 + 4 * kTile - 1 < a.Tq - 1 ? bq0 + 4 * kTile - 1 : a.Tq - 1;
    krange(bq0, bq1, blo, bhi);
  }

  uint32_t* brow = a.bits + ((int64_t)bh * a.nqt + qt) * a.nkt_words;
  if (wave_ok)
    for (int wi = lane; wi < a.nkt_words; wi += kWave)
      if (kt_hi < kt_lo || wi < (kt_lo >> 5) || wi > (kt_hi >> 5)) brow[wi] = 0u;

  f32x16 o[NDH][2];
#pragma unroll
  for (int dh = 0; dh < NDH; ++dh)
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[dh][qh][r] = 0.0f;

  const T* kg = (const T*)a.khat + (int64_t)bh * a.Tk_pad * DP;
  i32x4 pre[G::CPT];
  auto fetch = [&](int kt) {
#pragma unroll
    for (int u = 0; u < G::CPT; ++u) {
      const int c = tid + 256 * u;
      pre[u] = *reinterpret_cast<const i32x4*>(kg + (int64_t)kt * kTile * DP + (int64_t)c * (16 / sizeof(T)));
    }
  };
  auto stash = [&](int buf) {
#pragma unroll
    for (int u = 0; u < G::CPT; ++u) {
      const int c = tid + 256 * u;
      const int row = c / G::CPR, col = (c % G::CPR) * (16 / (int)sizeof(T));
      *reinterpret_cast<i32x4*>(&kl[buf][row * G::LDK + col]) = pre[u];
    }
  };

  if (bhi >= blo) {
    fetch(blo);
    stash(0);
  }
  __syncthreads();
  uint32_t word = 0u;

  for (int kt = blo; kt <= bhi; ++kt) {
    const int buf = (kt - blo) & 1;
    const int k0 = kt * kTile;
    if (kt < bhi) fetch(kt + 1);
    const bool mine = kt >= kt_lo && kt <= kt_hi;

    f32x16 acc[2][2];
    bool live = false;
    if (mine) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int qh = 0; qh < 2; ++qh)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[kh][qh][r] = 0.0f;
      const T* kb = &kl[buf][0];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const frag kf = M::load(kb + (32 * kh + perm_row(l32)) * G::LDK + KS * ks + PER * half);
#pragma unroll
          for (int qh = 0; qh < 2; ++qh) acc[kh][qh] = M::mma(kf, qf[qh][ks], acc[kh][qh]);
        }
      // Threshold vote: a(s) is monotone in s and s = acc/|q_i| in acc, so a
      // tile has a live pair iff its largest in-window acc passes.
      const bool interior = causal ? (k0 + 63 <= q0 && q0 + 63 - k0 < hp.wc)
                                   : (q0 + 63 - k0 < hp.wc && k0 + 63 - q0 < hp.wc);
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        float mx = -INFINITY;
        if (interior) {
#pragma unroll
          for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, acc[kh][qh][r]);
        } else {
          // register r of block kh holds key k0 + 32kh + 16(r/8) + 8half + r%8
          const int rel0 = (q0 + 32 * qh + l32) - k0 - 8 * half;
#pragma unroll
          for (int kh = 0; kh < 2; ++kh)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int dd = rel0 - (32 * kh + 16 * (r >> 3) + (r & 7));
              if (in_window(dd, hp.wc, causal)) mx = fmaxf(mx, acc[kh][qh][r]);
            }
        }
        live |= trim(mx * iq[qh], hp.r) > 0.0f;
      }
    }
    const bool act = __ballot(live) != 0;
    if (act) word |= 1u << (kt & 31);
    if (mine && ((kt & 31) == 31 || kt == kt_hi)) {
      if (lane == 0) brow[kt >> 5] = word;
      word = 0u;
    }
    if (kt < bhi) stash(buf ^ 1);
    const bool any = __syncthreads_or(act) != 0;

    if (any) {
      // Stage V^T of this key tile: V^[j][d] -> vl[d][j], normalised rows.
      {
        constexpr int VEC = 16 / (int)sizeof(T);
        constexpr int TPR = DP / VEC < 4 ? DP / VEC : 4;   // threads per key row
        constexpr int DPT = DP / TPR;                      // columns per thread
        const int jr = tid / TPR, part = tid % TPR;
        const int64_t j = (int64_t)k0 + jr;
        const bool ok = jr < 64 && j < a.Tk;
        float x[DPT];
        float ss = 0.0f;
#pragma unroll
        for (int e = 0; e < DPT; e += 4) {
          const int d = part * DPT + e;
          f32x4 v4 = {0.f, 0.f, 0.f, 0.f};
          if (ok && d < a.D) v4 = load4((const T*)a.v + b * a.vs.sb + j * a.vs.st + h * a.vs.sh + d);
          x[e] = v4[0]; x[e + 1] = v4[1]; x[e + 2] = v4[2]; x[e + 3] = v4[3];
          ss += v4[0] * v4[0] + v4[1] * v4[1] + v4[2] * v4[2] + v4[3] * v4[3];
        }
#pragma unroll
        for (int o2 = 1; o2 < TPR; o2 <<= 1) ss += __shfl_xor(ss, o2);
        const float iv = 1.0f / fmaxf(sqrtf(ss), a.eps);
        if (jr < 64)
#pragma unroll
          for (int e = 0; e < DPT; ++e) vl[(part * DPT + e) * G::LDV + jr] = from_f<T>(x[e] * iv);
      }
      __syncthreads();
      if (act) {
        // P^T[j][i] = alpha_ij m_ij, in place of S^T; transcendental work only
        // for registers where some lane is live.
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int qh = 0; qh < 2; ++qh) {
            const int rel0 = (q0 + 32 * qh + l32) - k0 - 8 * half;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
              const int dd = rel0 - (32 * kh + 16 * (r >> 3) + (r & 7));
              const float av = trim(acc[kh][qh][r] * iq[qh], hp.r);
              const bool lv = av > 0.0f && in_window(dd, hp.wc, causal);
              float p = 0.0f;
              if (__ballot(lv) != 0) {
                if (lv) p = av * av * softmask(dd, hp.iw);
              }
              acc[kh][qh][r] = p;
            }
          }
        // H^T[d][i] += sum_j V^T[d][j] P^T[j][i]
#pragma unroll
        for (int kh = 0; kh < 2; ++kh)
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            const int r0 = c * PER;
            const int koff = 32 * kh + rowof(r0, half);
#pragma unroll
            for (int qh = 0; qh < 2; ++qh) {
              const frag pf = M::pack(acc[kh][qh], r0);
#pragma unroll
              for (int dh = 0; dh < NDH; ++dh)
                o[dh][qh] = M::mma(M::load(&vl[(32 * dh + l32) * G::LDV + koff]), pf, o[dh][qh]);
            }
          }
      }
    }
  }

  if (!wave_ok) return;
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

size_t fwd_ws_bytes(const Geometry& g) {
  return round_up((int64_t)g.B * g.H * g.Tk_pad * g.DP * (int64_t)g.esize, 256);
}

template <typename T, int DP>
static hipError_t launch_fwd_t(const FwdCall& c) {
  const Geometry& g = c.g;
  if (g.Tk_pad > 0) {
    PrepKArgs pa;
    pa.k = c.k; pa.ks = c.ks; pa.kpm = c.kpm; pa.khat = c.khat;
    pa.H = g.H; pa.Tk = g.Tk; pa.D = g.D; pa.Tk_pad = g.Tk_pad; pa.eps = c.eps;
    constexpr int RPB = 256 / (DP * (int)sizeof(T) / 16);
    timer_begin(1, c.stream);
    hipLaunchKernelGGL((prep_k_kernel<T, DP>), dim3((unsigned)((g.Tk_pad + RPB - 1) / RPB), (unsigned)(g.B * g.H)),
                       dim3(256), 0, c.stream, pa);
    timer_end(1, c.stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  FwdKArgs fa;
  fa.q = c.q; fa.qs = c.qs; fa.v = c.v; fa.vs = c.vs; fa.khat = c.khat;
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
