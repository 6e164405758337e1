// Forward path of fused Screening Attention on gfx950.
//
//   prep_k_kernel : unit-normalised K^ rows (attention.py:156-157) in a padded
//                   [b*h][Tk_pad][DP] buffer; key padding (attention.py:185-188)
//                   is folded in as a zero row (s = 0 gives alpha = 0: r > 1).
//   fwd_screen_kernel : 256-thread block = 4 waves, wave -> one 64-query tile
//                   of one head.  Key tiles of the block's window are copied
//                   global -> LDS by direct DMA into a 4-slot ring (3 tiles in
//                   flight) and shared by the 4 waves.  Each wave forms
//                   S^T = K^ Q^T on MFMA (raw bf16 Q, fp32 accumulation, scaled
//                   by 1/|q_i|) and votes, with a wave ballot, whether any
//                   in-window pair passes the trim-and-square threshold
//                   (attention.py:75-90).  Output: the live-tile bitmap.
//   fwd_live_kernel : 256-thread block per 64-query tile, one 32x32 quadrant
//                   per wave; walks the tile's live bits, recomputes S^T for
//                   those key tiles only, forms alpha*m (attention.py:92-119)
//                   and accumulates H^T += V^T P^T with 1/|v_j| folded into P.
//                   The epilogue applies TanhNorm (norm.py:23-25) and writes y
//                   in (B,T,H,D) and |h| per row.
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

// MFMAs of one 64x64 screen tile: acc[kh][qh] = K^ rows (A, permuted) x Q^T.
// bf16: unguarded MFMAs plus one guard on the K fragments (the Q fragments
// stay live and are guarded once after their last use); fp32: guarded MFMAs.
template <typename T, int DP>
__device__ inline void screen_mma(typename Mma<T>::frag (&kf)[2 * (DP / Mma<T>::KS)],
                                  const typename Mma<T>::frag (&qf)[2 * (DP / Mma<T>::KS)], f32x16 (&acc)[2][2]) {
  using M = Mma<T>;
  constexpr int NKS = DP / M::KS;
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[kh][qh][r] = 0.0f;
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int qh = 0; qh < 2; ++qh)
          acc[kh][qh] = M::mma_ng(kf[kh * NKS + ks], qf[qh * NKS + ks], acc[kh][qh]);
    guard_frags(kf);
  } else {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) acc[kh][qh] = M::mma(kf[kh * NKS + ks], qf[qh * NKS + ks], acc[kh][qh]);
  }
}

// Loads Q^T B-operand fragments (raw values) and 1/|q| for the 64 queries of
// tile qt: lane -> query q0 + 32*qh + l32, slots -> d.
template <typename T, int DP>
__device__ inline void load_q_tile(const FwdKArgs& a, int b, int h, int q0, bool wave_ok, int half, int l32,
                                   typename Mma<T>::frag (&qf)[2 * (DP / Mma<T>::KS)], float (&iq)[2]) {
  constexpr int NKS = DP / Mma<T>::KS;
#pragma unroll
  for (int qh = 0; qh < 2; ++qh) {
    const int i = q0 + 32 * qh + l32;
    const bool ok = wave_ok && i < a.Tq;
    Row<T, DP> row;
    row.load((const T*)a.q + b * a.qs.sb + (int64_t)(ok ? i : 0) * a.qs.st + h * a.qs.sh, ok, a.D, half);
    iq[qh] = row.inv_norm(a.eps);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qf[qh * NKS + ks] = row.frag(ks, 1.0f);
  }
}

// Key-tile range [lo, hi] of the window of queries [qa, qb].
__device__ inline void key_tile_range(const FwdKArgs& a, const HeadParams& hp, bool causal, int64_t qa, int64_t qb,
                                      int& lo, int& hi) {
  int64_t jlo = qa - hp.wc + 1;
  int64_t jhi = causal ? qb : qb + hp.wc - 1;
  if (jlo < 0) jlo = 0;
  if (jhi > a.Tk - 1) jhi = a.Tk - 1;
  lo = (int)(jlo / kTile);
  hi = jhi >= jlo ? (int)(jhi / kTile) : lo - 1;
}

template <typename T, int DP>
struct ScreenTile {
  static constexpr int ROWB = DP * (int)sizeof(T);   // bytes per key row
  static constexpr int CPR = ROWB / 16;              // 16-byte chunks per row (power of two)
  static constexpr int TILEB = 64 * ROWB;            // bytes per staged key tile
  static constexpr int CPT = 64 * CPR / 256;         // DMA chunks per thread per tile
  static constexpr int NST = 4;                      // pipeline stages (3 tiles in flight)
};

template <int N>
__device__ inline void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory"); }

// ---------------------------------------------------------------------------
// Screen: 256-thread block = 4 waves, wave -> one 64-query tile of one head.
// The block's key tiles stream through a 4-stage LDS ring filled by direct
// global->LDS DMA three tiles ahead (no register staging, one raw barrier per
// tile).  Chunks are XOR-swizzled within each key row so the A-operand reads
// of 32 rows spread over the LDS banks.  Each wave forms S^T = K^ Q^T on MFMA
// for the tiles of its own window and votes with a ballot whether any
// in-window pair passes the trim-and-square threshold; the result is the
// live-tile bitmap.
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void fwd_screen_kernel(FwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  using G = ScreenTile<T, DP>;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS;
  __shared__ __attribute__((aligned(16))) char ring[G::NST * G::TILEB];

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

  frag qf[2 * NKS];
  float iq[2];
  load_q_tile<T, DP>(a, b, h, q0, wave_ok, half, l32, qf, iq);

  int kt_lo, kt_hi, blo, bhi;
  key_tile_range(a, hp, causal, q0, q0 + 63 < a.Tq - 1 ? q0 + 63 : a.Tq - 1, kt_lo, kt_hi);
  if (!wave_ok) { kt_lo = 0; kt_hi = -1; }
  {
    const int64_t bq0 = (int64_t)bx * 4 * kTile;
    key_tile_range(a, hp, causal, bq0, bq0 + 4 * kTile - 1 < a.Tq - 1 ? bq0 + 4 * kTile - 1 : a.Tq - 1, blo, bhi);
  }

  uint32_t* brow = a.bits + ((int64_t)bh * a.nqt + qt) * a.nkt_words;
  if (wave_ok)
    for (int wi = lane; wi < a.nkt_words; wi += kWave)
      if (kt_hi < kt_lo || wi < (kt_lo >> 5) || wi > (kt_hi >> 5)) brow[wi] = 0u;

  // DMA of key tile kt into ring slot kt % NST; LDS chunk position p of row r
  // holds global chunk p ^ (r % CPR).
  const char* kg = (const char*)a.khat + (int64_t)bh * a.Tk_pad * G::ROWB;
  auto issue = [&](int kt) {
    char* slot = ring + (kt % G::NST) * G::TILEB;
#pragma unroll
    for (int u = 0; u < G::CPT; ++u) {
      const int c = u * 256 + tid;  // chunk position in the tile
      const int row = c / G::CPR, p = c % G::CPR;
      const char* src = kg + ((int64_t)kt * kTile + row) * G::ROWB + ((p ^ (row & (G::CPR - 1))) << 4);
      __builtin_amdgcn_global_load_lds((const void __attribute__((address_space(1)))*)src,
                                       (void __attribute__((address_space(3)))*)(slot + (u * 256 + wave * 64) * 16),
                                       16, 0, 0);
    }
  };
  for (int kt = blo; kt <= bhi && kt < blo + G::NST - 1; ++kt) issue(kt);

  // element d of row R of the staged tile in ring slot `slot`
  auto lds_elem = [&](const char* slot, int R, int d) -> const T* {
    const int byte = d * (int)sizeof(T);
    return (const T*)(slot + R * G::ROWB + ((((byte >> 4) ^ (R & (G::CPR - 1))) << 4) | (byte & 15)));
  };

  uint32_t word = 0u;
  for (int kt = blo; kt <= bhi; ++kt) {
    // tile kt's DMA (own part) is complete when at most the younger tiles'
    // chunks are outstanding; the barrier then covers all four waves
    const int younger = bhi - kt < G::NST - 2 ? bhi - kt : G::NST - 2;
    if (younger >= 2) wait_vmcnt<2 * G::CPT>();
    else if (younger == 1) wait_vmcnt<G::CPT>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (kt + G::NST - 1 <= bhi) issue(kt + G::NST - 1);

    const bool mine = kt >= kt_lo && kt <= kt_hi;
    bool live = false;
    if (mine) {
      const int k0 = kt * kTile;
      const char* slot = ring + (kt % G::NST) * G::TILEB;
      frag kf[2 * NKS];
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
          kf[kh * NKS + ks] = M::load(lds_elem(slot, 32 * kh + perm_row(l32), KS * ks + PER * half));
      f32x16 acc[2][2];
      screen_mma<T, DP>(kf, qf, acc);
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
    if (__ballot(live) != 0) word |= 1u << (kt & 31);
    if (mine && ((kt & 31) == 31 || kt == kt_hi)) {
      if (lane == 0) brow[kt >> 5] = word;
      word = 0u;
    }
  }
  guard_frags(qf);
}

// ---------------------------------------------------------------------------
// Live tiles.  256-thread block per 64-query tile; wave w works on the
// quadrant (queries 32*qh .. +31, keys 32*kh .. +31) of every key tile the
// screen marked live, qh = w/2, kh = w%2.  Lane -> query i = q0 + 32*qh + l32,
// registers -> keys.  Per tile: S^T from K^ (the screen's operands, so the same
// values), alpha*m (attention.py:92-119) with 1/|v_j| folded in, and
// H^T += V^T P^T with V^T from an identity MFMA on the raw V rows.  The kh = 1
// wave hands its H^T to the kh = 0 wave through LDS, which applies TanhNorm
// (norm.py:23-25) and writes y in (B,T,H,D) and |h| per row.  Rows with no live
// tile get y = 0, |h| = 0.
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 && DP <= 64 ? 2 : 1)))
void fwd_live_kernel(FwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  __shared__ __attribute__((aligned(16))) float sv[4][32];  // per wave: 1/|v_j| of its key rows
  __shared__ __attribute__((aligned(16))) float red[2][NDH][16][kWave];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, kh = w & 1, qh = w >> 1;
  const int half = lane >> 5, l32 = lane & 31;
  int qt, bh;
  xcd_order(qt, bh);
  const int b = bh / a.H, h = bh % a.H;
  const HeadParams hp = head_params(a.r, a.w, h);
  const bool causal = a.causal != 0;
  const int q0 = qt * kTile;
  const int i = q0 + 32 * qh + l32;

  int kt_lo, kt_hi;
  key_tile_range(a, hp, causal, q0, q0 + 63 < a.Tq - 1 ? q0 + 63 : a.Tq - 1, kt_lo, kt_hi);
  const uint32_t* brow = a.bits + ((int64_t)bh * a.nqt + qt) * a.nkt_words;
  bool any = false;
  for (int base = kt_lo; base <= kt_hi && !any; base += kWave) {
    const int kl = base + lane;
    any = __ballot(kl <= kt_hi && ((brow[kl >> 5] >> (kl & 31)) & 1u)) != 0ull;
  }

  f32x16 o[NDH];
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dblk][r] = 0.0f;

  if (any) {
    // own queries as raw B operands (lane -> query) and 1/|q_i|
    frag qf[NKS];
    float iq;
    {
      const bool ok = i < a.Tq;
      PRow<T, DP> qr;
      qr.load((const T*)a.q + b * a.qs.sb + (int64_t)(ok ? i : 0) * a.qs.st + h * a.qs.sh, ok, a.D, half);
      iq = qr.inv_norm(a.eps);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) qf[ks] = qr.f[ks];
    }
    frag id[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) id[c] = ident_frag<T>(c, lane);
    const T* kg = (const T*)a.khat + (int64_t)bh * a.Tk_pad * DP;

    for (int base = kt_lo; base <= kt_hi; base += kWave) {
      const int kl = base + lane;
      unsigned long long mask = __ballot(kl <= kt_hi && ((brow[kl >> 5] >> (kl & 31)) & 1u));
      while (mask != 0ull) {
        const int kt = base + __builtin_ctzll(mask);
        mask &= mask - 1ull;
        const int k0 = kt * kTile;

        // key rows j = k0 + 32*kh + perm_row(l32): K^ (padded rows are zero
        // and inside the buffer) and raw V with 1/|v|
        const int m = perm_row(l32);
        const int j = k0 + 32 * kh + m;
        frag kf[NKS];
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) kf[ks] = M::load(kg + (int64_t)j * DP + KS * ks + PER * half);
        PRow<T, DP> vr;
        const bool vok = j < a.Tk;
        vr.load((const T*)a.v + b * a.vs.sb + (int64_t)(vok ? j : 0) * a.vs.st + h * a.vs.sh, vok, a.D, half);
        float isv[16];
        {
          const float iv = vr.inv_norm(a.eps);
          wave_lds_sync();
          if (half == 0) sv[w][m] = iv;
          wave_lds_sync();
          read_row_scales(sv[w], half, isv);
        }

        f32x16 s;
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) s = M::mma_ng(kf[ks], qf[ks], s);
        guard_frags(kf);

        // P^T[j][i] = alpha_ij m_ij / |v_j|; register r -> key
        // k0 + 32kh + rowof(r, half), lane -> query i
        const int rel0 = i - (k0 + 32 * kh + 8 * half);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int dd = rel0 - (16 * (r >> 3) + (r & 7));
          const float av = trim(s[r] * iq, hp.r);
          const bool pos = av > 0.0f;
          float p = 0.0f;
          if (__ballot(pos) != 0ull) {
            if (pos && in_window(dd, hp.wc, causal)) p = av * av * softmask(dd, hp.iw) * isv[r];
          }
          s[r] = p;
        }
        // H^T[d][i] += sum_j V^T[d][j] P^T[j][i]
        frag pb[NC], ta[NDH * NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) pb[c] = M::pack(s, c * PER);
        {
          f32x16 tr[NDH];
          transpose_rows<T, DP>(vr.f, id, tr);
#pragma unroll
          for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
            for (int c = 0; c < NC; ++c) ta[dblk * NC + c] = M::pack(tr[dblk], c * PER);
        }
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
          for (int dblk = 0; dblk < NDH; ++dblk) o[dblk] = M::mma_ng(ta[dblk * NC + c], pb[c], o[dblk]);
        guard_frags(vr.f);
        guard_frags(ta);
        guard_frags(pb);
      }
    }
    guard_frags(qf);
    guard_frags(id);
  }

  if (kh == 1) {
#pragma unroll
    for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[qh][dblk][r][lane] = o[dblk][r];
  }
  __syncthreads();
  if (kh == 1) return;
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dblk][r] += red[qh][dblk][r][lane];

  // TanhNorm per query row (lane -> query, registers -> d), y in (B,T,H,D)
  float ss = 0.0f;
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) ss += o[dblk][r] * o[dblk][r];
  ss += __shfl_xor(ss, 32);
  const float n = sqrtf(ss);
  const float nc = fmaxf(n, a.eps);
  const float f = tanhf(nc) / nc;
  if (i < a.Tq) {
    if (half == 0) a.hnorm[(int64_t)bh * a.Tq + i] = n;
    T* yrow = (T*)a.y + (((int64_t)b * a.Tq + i) * a.H + h) * a.D;
#pragma unroll
    for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dblk + 8 * g + 4 * half;
        if (d < a.D)
          store4(yrow + d, f * o[dblk][4 * g], f * o[dblk][4 * g + 1], f * o[dblk][4 * g + 2], f * o[dblk][4 * g + 3]);
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
  hipLaunchKernelGGL((fwd_screen_kernel<T, DP>), dim3((unsigned)((g.nqt + 3) / 4), (unsigned)(g.B * g.H)), dim3(256),
                     0, c.stream, fa);
  timer_end(2, c.stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(3, c.stream);
  hipLaunchKernelGGL((fwd_live_kernel<T, DP>), dim3((unsigned)g.nqt, (unsigned)(g.B * g.H)), dim3(256), 0, c.stream,
                     fa);
  timer_end(3, c.stream);
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
