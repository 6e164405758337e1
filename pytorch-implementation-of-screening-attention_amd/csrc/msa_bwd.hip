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
  ss += __shfl_xor(ss, 32);
  const float nx = sqrtf(ss);
  const float ix = 1.0f / fmaxf(nx, eps);
  float dot = 0.0f;
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) dot += M::get(x[creg_ks<T>(dblk, r)], creg_e<T>(r)) * ix * acc[dblk][r];
  dot += __shfl_xor(dot, 32);
  const float proj = nx > eps ? dot : 0.0f;
  if (!valid) return;
  store_creg_row<T, NDH>(out, D, half, [&](int dblk, int r) {
    const float xn = M::get(x[creg_ks<T>(dblk, r)], creg_e<T>(r)) * ix;
    return (acc[dblk][r] - xn * proj) * ix;
  });
}

// Waves per SIMD the backward kernels are register-budgeted for: three (168
// registers a lane; operands are re-read from LDS rather than held) where the
// bf16 working set allows, else one.
template <typename T, int DP>
constexpr int bwd_waves() { return sizeof(T) == 2 && DP <= 64 ? 3 : 1; }

// ---------------------------------------------------------------------------
// dQ (runs first).  256-thread block per 64-query tile of head (b,h); wave w
// works on the quadrant (queries 32*qh .. +31, keys 32*kh .. +31) of every
// live key tile in the query tile's bitmap row, qh = w/2, kh = w%2.  Lane ->
// query i = q0 + 32*qh + l32; registers -> keys.  The live key tiles' raw K
// and V rows are staged into LDS by DMA, double-buffered: tile n+1 streams in
// while tile n is computed.  K^T comes from an identity MFMA.  Side output for
// dkdv_kernel: dh (rounded to T, as the operand it becomes) and 1/|q| of every
// row of a query tile with a live key tile, in the workspace.  The kh = 1
// wave hands its accumulator to the kh = 0 wave through LDS, which finishes dq.
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(bwd_waves<T, DP>()))) void dq_kernel(BwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  using S = StageTile<T, DP>;
  using WS = WaveStage<T, DP>;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  // per wave: DMA ring of its key half of the live key tiles (K rows | V
  // rows), NBUF buffers, NBUF-1 tiles ahead; waves never wait for each other
  // inside the tile loop
  constexpr int NBUF = 1;  // a small LDS footprint leaves room for three blocks per CU
  __shared__ __attribute__((aligned(16))) char stage[4][NBUF][2 * WS::TILEB];
  static_assert(2 * NDH * 16 * kWave * 4 <= 4 * NBUF * 2 * WS::TILEB, "exchange must fit the stage buffers");
  __shared__ __attribute__((aligned(16))) float sk[4][32];                 // per wave: 1/|k| (0 if masked)
  __shared__ __attribute__((aligned(16))) float sv[4][32];              // per wave: 1/|v|
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), kh = w & 1, qh = w >> 1;
  const int half = lane >> 5, l32 = lane & 31;
  int qt, bh;
  xcd_interleave(qt, bh);
  const int b = bh / a.H, h = bh % a.H;
  const bool causal = a.causal != 0;
  const HeadParams hp = head_params(a.r, a.w, h, causal);
  const int q0 = qt * kTile;
  const int i = q0 + 32 * qh + l32;
  const bool valid = i < a.Tq;
  const int ii = valid ? i : 0;
  T* dqrow = (T*)a.dq + (((int64_t)b * a.Tq + ii) * a.H + h) * a.D;

  const int64_t qlast = q0 + 63 < a.Tq - 1 ? q0 + 63 : a.Tq - 1;
  int64_t jlo = (int64_t)q0 - hp.wc + 1;
  int64_t jhi = causal ? qlast : qlast + hp.wc - 1;
  if (jlo < 0) jlo = 0;
  if (jhi > a.Tk - 1) jhi = a.Tk - 1;
  const int kt_lo = (int)(jlo / kTile), kt_hi = jhi >= jlo ? (int)(jhi / kTile) : kt_lo - 1;
  // key tile kl is live for this query tile iff one of its four 32x32 units
  // is: bits 2kl, 2kl+1 of the rows of query units 2qt, 2qt+1
  const uint32_t* brow = a.bits + ((int64_t)bh * 2 * a.nqt + 2 * qt) * a.nku_words;
  const int nw = a.nku_words;
  auto bitf = [brow, nw](int kl) { return (((brow[kl >> 4] | brow[nw + (kl >> 4)]) >> ((2 * kl) & 31)) & 3u) != 0u; };
  BitWalk<decltype(bitf)> walk(bitf, kt_lo, kt_hi);
  int cur = walk.next();
  if (cur < 0) {  // block-uniform: no live key tile, dq = 0
    if (kh == 0 && valid)
#pragma unroll
      for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * dblk + 8 * g + 4 * half;
          if (d < a.D) store4(dqrow + d, 0.0f, 0.0f, 0.0f, 0.0f);
        }
    return;
  }

  const T* krow0 = (const T*)a.k + b * a.ks.sb + h * a.ks.sh;
  const T* vrow0 = (const T*)a.v + b * a.vs.sb + h * a.vs.sh;
  const int m = perm_row(l32);
  // the DMA offsets are formed at each issue from a laundered lane index, so
  // the compiler keeps no per-lane offsets live across the tile loop
  auto stage_tile = [&](int kt, int buf, uint8_t& msk) {
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const auto plk = WS::plan(a.ks.st, a.D, ln), plv = WS::plan(a.vs.st, a.D, ln);
    WS::issue(plk, krow0, a.ks.st, (int64_t)kt * kTile + 32 * kh, a.Tk, a.D, stage[w][buf], ln, 0);
    WS::issue(plv, vrow0, a.vs.st, (int64_t)kt * kTile + 32 * kh, a.Tk, a.D, stage[w][buf] + WS::TILEB, ln, 0);
    const int j = kt * kTile + 32 * kh + m;
    msk = (a.kpm != nullptr && j < a.Tk) ? a.kpm[(int64_t)b * a.Tk + j] : (uint8_t)0;
  };
  // tl[n]: the n-th next live key tile (-1 past the end); mk[n] its key-padding byte
  int tl[3] = {cur, -1, -1};
  uint8_t mk[3] = {0, 0, 0};
  // own queries' rows first, then the first key tiles' DMA behind them
  // (vector memory returns in order, so the rows are not held up by the DMA)
  frag qb[NKS], hb[NKS];
  float iql;
  {
    QueryRows<T, DP> qr;
    qr.load(a, b, h, bh, i, half);
    stage_tile(tl[0], 0, mk[0]);
    tl[1] = walk.next();
    iql = qr.finish(a.eps);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      qb[ks] = qr.q.f[ks];
      hb[ks] = qr.dh.f[ks];
    }
  }
  if (kh == 0) {  // dh and 1/|q| of this tile's rows for dkdv_kernel (zero past Tq)
    T* dst = (T*)a.dh + ((int64_t)bh * a.Tq_pad + i) * DP;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) *reinterpret_cast<frag*>(dst + KS * ks + PER * half) = hb[ks];
    if (half == 0) a.iqs[(int64_t)bh * a.Tq_pad + i] = valid ? iql : 0.0f;
  }
  const float thq = hp.thr / iql;  // s > thr  <=>  (q . k)/|k| > thr |q|
  f32x16 adq[NDH];
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) adq[dblk][r] = 0.0f;

  for (int it = 0; tl[0] >= 0; ++it) {
    // this wave's DMA of tile tl[0] is complete
    wait_vmcnt<0>();
    wave_lds_sync();
    const char* kl = stage[w][0];
    const char* vl = kl + WS::TILEB;
    const int k0 = tl[0] * kTile;
    const uint8_t mk_cur = mk[0];

    // key rows j = k0 + 32*kh + perm_row(l32) as A operands.  S^T = K Q^T and
    // dP^T = V dH^T take one operand set at a time (fragments re-read from
    // LDS when needed again), with the rows' squared norms from the same
    // fragments.
    const int j = k0 + 32 * kh + m;
    const bool jok = j < a.Tk;
    f32x16 s, dp;
    float s2k = 0.0f, s2v = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[r] = 0.0f; dp[r] = 0.0f; }
    {
      frag f[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) f[ks] = WS::frag(kl, m, ks, half, a.D);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        s = M::mma_ng(f[ks], qb[ks], s);
        s2k = frag_dot(f[ks], f[ks], s2k);
      }
      guard_frags(f);
    }
    {
      frag f[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) f[ks] = WS::frag(vl, m, ks, half, a.D);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        dp = M::mma_ng(f[ks], hb[ks], dp);
        s2v = frag_dot(f[ks], f[ks], s2v);
      }
      guard_frags(f);
    }
    s2k += __shfl_xor(s2k, 32);
    s2v += __shfl_xor(s2v, 32);
    {
      const float ik = (jok && mk_cur == 0) ? inv_len(s2k, a.eps) : 0.0f;  // 0 if padded or masked
      const float iv = inv_len(s2v, a.eps);
      wave_lds_sync();
      if (half == 0) { sk[w][m] = ik; sv[w][m] = iv; }
      wave_lds_sync();
    }
    // register r -> key k0 + 32kh + rowof(r, half), lane -> query i.  Scaled
    // in place: s = (q . k)/|k|, dp = dH . v^.
    {
      float sc[16];
      read_row_scales(sk[w], half, sc);
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] *= sc[r];
      read_row_scales(sv[w], half, sc);
#pragma unroll
      for (int r = 0; r < 16; ++r) dp[r] *= sc[r];
    }
    // A conservative gate on the products (s > thr |q|), then the exact test
    // only for registers where some lane passes; only a quadrant with a pair
    // past the threshold contributes to dq.
    bool anyp = false;
#pragma unroll
    for (int r = 0; r < 16; ++r) anyp |= s[r] > thq;
    if (__ballot(anyp) != 0ull) {
      const int rel0 = i - (k0 + 32 * kh + 8 * half);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float ds = 0.0f;
        if (__ballot(s[r] > thq) != 0ull) {
          const int dd = rel0 - (16 * (r >> 3) + (r & 7));
          const float av = trim(s[r] * iql, hp.r);
          if (av > 0.0f && valid && in_window(dd, hp)) {
            ds = 2.0f * av * hp.r * softmask(dd, hp.iw) * dp[r];
            if (a.drop.on) ds *= dropout_factor(a.drop, bh, i, i - dd);
          }
        }
        dp[r] = ds;
        __builtin_amdgcn_sched_barrier(0);  // one register at a time: few live temporaries
      }
      // dq^T[d][i] += sum_j K^T[d][j] (ds/|k|)^T[j][i], K^T by identity from
      // the key rows, one 32-column block of d at a time
      {
        float sc[16];
        read_row_scales(sk[w], half, sc);
#pragma unroll
        for (int r = 0; r < 16; ++r) dp[r] *= sc[r];
      }
      frag db[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) db[c] = M::pack(dp, c * PER);
#pragma unroll
      for (int dblk = 0; dblk < NDH; ++dblk) {
        frag f[NC], kt[NC];
#pragma unroll
        for (int c = 0; c < NC; ++c) f[c] = WS::frag(kl, m, dblk * NC + c, half, a.D);
        f32x16 tr;
#pragma unroll
        for (int r = 0; r < 16; ++r) tr[r] = 0.0f;
#pragma unroll
        for (int c = 0; c < NC; ++c) tr = M::mma_ng(f[c], ident_frag<T>(c, lane), tr);
#pragma unroll
        for (int c = 0; c < NC; ++c) kt[c] = M::pack(tr, c * PER);
        guard_frags(f);
#pragma unroll
        for (int c = 0; c < NC; ++c) adq[dblk] = M::mma_ng(kt[c], db[c], adq[dblk]);
        guard_frags(kt);
      }
      guard_frags(db);
    }

    // every LDS read of this tile is done: its buffer takes the next tile
    wave_lds_sync();
    if (tl[1] >= 0) stage_tile(tl[1], 0, mk[1]);
    tl[0] = tl[1];
    mk[0] = mk[1];
    tl[1] = walk.next();
  }
  guard_frags(qb);
  guard_frags(hb);

  // the kh = 1 wave's accumulator reaches the kh = 0 wave through the
  // (now idle) stage buffers
  __syncthreads();
  float* red = reinterpret_cast<float*>(&stage[0][0][0]);  // [qh][NDH][16][64]
  if (kh == 1) {
#pragma unroll
    for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[((qh * NDH + dblk) * 16 + r) * kWave + lane] = adq[dblk][r];
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
      for (int r = 0; r < 16; ++r) adq[dblk][r] += red[((qh * NDH + dblk) * 16 + r) * kWave + lane];
    write_norm_bwd<T, DP>(adq, qb, valid, a.D, a.eps, half, dqrow);
  }
}

// ---------------------------------------------------------------------------
// dK, dV (runs after dq_kernel).  256-thread block per 64-key tile of head
// (b,h); wave w works on the quadrant (keys 32*kh .. +31, queries
// 32*qh .. +31) of every live query tile in the key tile's bitmap column,
// kh = w%2, qh = w/2, so the two waves of a key half accumulate over
// different query halves.  Lane -> key j = k0 + 32*kh + l32 of the C blocks;
// registers -> queries.  Per live query tile, its raw Q rows, the dh rows and
// 1/|q| that dq_kernel left in the workspace are staged into LDS by DMA,
// double-buffered.  The transposed Q^T and dH^T operands of the dK/dV products
// are formed by identity MFMAs.  At the end the two waves of a key half
// exchange one accumulator through LDS: the qh = 0 wave finishes dk, the
// qh = 1 wave finishes dv.
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(bwd_waves<T, DP>()))) void dkdv_kernel(BwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  using S = StageTile<T, DP>;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  constexpr int SB = 2 * S::TILEB + 1024;  // per buffer: Q tile | dh tile | 1/|q| (64 floats, 1 KB slot)
  constexpr int KVB = 2 * NKS * kWave * (int)sizeof(frag);  // per key half: own K, V fragments
  // DMA ring of staged query tiles: NBUF buffers, NBUF-1 tiles ahead where LDS allows
  // (two buffers for bf16 at D <= 64 keep the block under a third of the LDS,
  // for three blocks per CU)
  constexpr int NBUF = bwd_waves<T, DP>() == 3 ? 2
                       : (3 * SB + 2 * KVB <= 70 * 1024 ? 3 : (2 * SB + 2 * KVB <= 150 * 1024 ? 2 : 1));
  constexpr int PT = 2 * S::CPT;  // DMA operations per thread per tile (wave 0 issues one more)
  static_assert(4 * NDH * 16 * kWave * 4 <= NBUF * SB, "exchange must fit the stage buffers");
  __shared__ __attribute__((aligned(16))) char stage[NBUF][SB];
  __shared__ __attribute__((aligned(16))) char kvs[2][KVB];
  __shared__ float rw[2][4];
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), kh = w & 1, qh = w >> 1;
  const int half = lane >> 5, l32 = lane & 31;
  int kt, bh;
  xcd_interleave(kt, bh);
  // a key tile's live query tiles lie after it (its window runs forward), so
  // under a causal mask the lowest key tiles carry the most work: they go first
  if (a.causal) kt = (int)gridDim.x - 1 - kt;
  const int b = bh / a.H, h = bh % a.H;
  const bool causal = a.causal != 0;
  const HeadParams hp = head_params(a.r, a.w, h, causal);
  const int k0 = kt * kTile;
  const int j = k0 + 32 * kh + l32;
  const bool jvalid = j < a.Tk;
  const int jj = jvalid ? j : 0;
  const int64_t orow = (((int64_t)b * a.Tk + jj) * a.H + h) * a.D;

  const int64_t klast = k0 + 63 < a.Tk - 1 ? k0 + 63 : a.Tk - 1;
  int64_t ilo = causal ? (int64_t)k0 : (int64_t)k0 - hp.wc + 1;
  int64_t ihi = klast + hp.wc - 1;
  if (ilo < 0) ilo = 0;
  if (ihi > a.Tq - 1) ihi = a.Tq - 1;
  const int qt_lo = (int)(ilo / kTile), qt_hi = ihi >= ilo ? (int)(ihi / kTile) : qt_lo - 1;
  // query tile ql is live for this key tile iff one of its four 32x32 units
  // is: bits 2kt, 2kt+1 of the rows of query units 2ql, 2ql+1
  const uint32_t* bcol = a.bits + (int64_t)bh * 2 * a.nqt * a.nku_words + (kt >> 4);
  const int nw = a.nku_words, sh = (2 * kt) & 31;
  auto bitf = [bcol, nw, sh](int ql) {
    return (((bcol[(int64_t)2 * ql * nw] | bcol[(int64_t)(2 * ql + 1) * nw]) >> sh) & 3u) != 0u;
  };
  BitWalk<decltype(bitf)> walk(bitf, qt_lo, qt_hi);
  int cur = walk.next();
  if (cur < 0) {  // block-uniform: no live query tile, dk = dv = 0
    T* out = (T*)(qh == 0 ? a.dk : a.dv) + orow;
    if (jvalid)
#pragma unroll
      for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * dblk + 8 * g + 4 * half;
          if (d < a.D) store4(out + d, 0.0f, 0.0f, 0.0f, 0.0f);
        }
    if (tid == 0) {
      const int64_t nbh = (int64_t)a.B * a.H;
      a.part[(int64_t)bh * a.nkt + kt] = 0.0f;
      a.part[nbh * a.nkt + (int64_t)bh * a.nkt + kt] = 0.0f;
    }
    return;
  }

  const T* qrow0 = (const T*)a.q + b * a.qs.sb + h * a.qs.sh;
  const T* dh0 = (const T*)a.dh + (int64_t)bh * a.Tq_pad * DP;
  const float* iq0 = a.iqs + (int64_t)bh * a.Tq_pad;
  // DMA offsets formed at each issue from a laundered thread index (nothing
  // per-lane kept live across the tile loop)
  auto stage_tile = [&](int qt, int buf) {
    int tx = tid;
    asm volatile("" : "+v"(tx));
    const auto plq = S::plan(a.qs.st, a.D, tx), plh = S::plan(DP, DP, tx);
    S::issue(plq, qrow0, a.qs.st, (int64_t)qt * kTile, a.Tq, a.D, stage[buf], tx, w);
    S::issue(plh, dh0, DP, (int64_t)qt * kTile, a.Tq_pad, DP, stage[buf] + S::TILEB, tx, w);
    if (w == 0)  // 64 floats of 1/|q|: lanes 0-15 carry them, the rest repeat lane 15 into the slot's tail
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(iq0 + (int64_t)qt * kTile + 4 * (lane < 16 ? lane : 15)),
          (void __attribute__((address_space(3)))*)(stage[buf] + 2 * S::TILEB), 16, 0, 0);
  };
  // tl[n]: the n-th next live query tile (-1 past the end)
  int tl[3] = {cur, -1, -1};
  // own keys as raw B operands (lane -> key), kept in LDS (one copy per key
  // half, written by its qh = 0 wave before the loop's first barrier), with
  // 1/|k| (0 if padded or masked) and 1/|v|.  Their loads go first, the first
  // query tile's DMA behind them (vector memory returns in order).
  frag* kvl = reinterpret_cast<frag*>(kvs[kh]);
  float ikl, ivl;
  {
    KeyRows<T, DP> kr;
    kr.load(a, b, h, j, half);
    stage_tile(tl[0], 0);
    for (int n = 1; n < (NBUF > 1 ? NBUF : 2); ++n) tl[n] = walk.next();
    kr.finish(a.eps, ikl, ivl);
    if (qh == 0)
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        kvl[ks * kWave + lane] = kr.k.f[ks];
        kvl[(NKS + ks) * kWave + lane] = kr.v.f[ks];
      }
  }
  f32x16 acc_k[NDH], acc_v[NDH];
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) { acc_k[dblk][r] = 0.0f; acc_v[dblk][r] = 0.0f; }
  float dr_acc = 0.0f, dw_acc = 0.0f;
  const int m = perm_row(l32);
  const float thk = hp.thr / ikl;  // s > thr  <=>  (q . k)/|q| > thr |k|  (+inf for masked keys)

  if (NBUF == 3 && tl[1] >= 0) stage_tile(tl[1], 1);
  for (int it = 0; tl[0] >= 0; ++it) {
    // tile tl[0] is in LDS once this wave's older DMA is done and every wave
    // passed the barrier; the buffer refilled next was read last iteration
    if (NBUF == 3 && tl[1] >= 0) wait_vmcnt<PT>();
    else wait_vmcnt<0>();
    block_sync_lds();
    if (NBUF > 1 && tl[NBUF - 1] >= 0) stage_tile(tl[NBUF - 1], (it + NBUF - 1) % NBUF);
    const char* ql = stage[it % NBUF];
    const char* hl = ql + S::TILEB;
    const float* iql = reinterpret_cast<const float*>(ql + 2 * S::TILEB);
    const int q0 = tl[0] * kTile;

    // query rows i = q0 + 32*qh + perm_row(l32) as A operands: raw q, dh
    // (rows past Tq carry 1/|q| = 0 and dh = 0, so they contribute nothing).
    // S = Q K^T and dP = dH V^T take one operand pair at a time; the
    // fragments are re-read from LDS where needed again.
    f32x16 s, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) { s[r] = 0.0f; dp[r] = 0.0f; }
    {
      frag f[NKS], g[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        f[ks] = S::frag(ql, 32 * qh + m, ks, half, a.D);
        g[ks] = kvl[ks * kWave + lane];
      }
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) s = M::mma_ng(f[ks], g[ks], s);
      guard_frags(f);
      guard_frags(g);
    }
    {
      frag f[NKS], g[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        f[ks] = S::frag(hl, 32 * qh + m, ks, half, DP);
        g[ks] = kvl[(NKS + ks) * kWave + lane];
      }
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) dp = M::mma_ng(f[ks], g[ks], dp);
      guard_frags(f);
      guard_frags(g);
    }
    // register r -> query q0 + 32qh + rowof(r, half), lane -> key j.  Scaled
    // in place: s = (q . k)/|q|, dp = (dh . v)/|v|.
    {
      float sc[16];
      read_row_scales(iql + 32 * qh, half, sc);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] *= sc[r];
        dp[r] *= ivl;
      }
    }

    // A conservative gate on the products (s > thr |k|), then the exact test
    // only for registers where some lane passes; only a quadrant with a pair
    // past the threshold contributes to dk, dv, dr, dw.
    bool anyp = false;
#pragma unroll
    for (int r = 0; r < 16; ++r) anyp |= s[r] > thk;
    if (__ballot(anyp) != 0ull) {
      const int rel0 = (q0 + 32 * qh + 8 * half) - j;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float p = 0.0f, ds = 0.0f;
        if (__ballot(s[r] > thk) != 0ull) {
          const int dd = rel0 + 16 * (r >> 3) + (r & 7);
          const float sv = s[r] * ikl;
          const float av = trim(sv, hp.r);
          if (av > 0.0f && in_window(dd, hp)) {
            const float c = a.drop.on ? dropout_factor(a.drop, bh, j + dd, j) : 1.0f;
            const float mk = softmask(dd, hp.iw) * c;
            const float g = dp[r];
            p = av * av * mk;
            ds = 2.0f * av * hp.r * mk * g;
            dr_acc -= 2.0f * av * (1.0f - sv) * mk * g;
            dw_acc += av * av * g * softmask_dw(dd, hp.iw) * c;
          }
        }
        s[r] = p;
        dp[r] = ds;
        __builtin_amdgcn_sched_barrier(0);  // one register at a time: few live temporaries
      }
      {
        float sc[16];
        read_row_scales(iql + 32 * qh, half, sc);
#pragma unroll
        for (int r = 0; r < 16; ++r) dp[r] *= sc[r];  // ds/|q|
      }
      // dv^T[d][j] += sum_i dH^T[d][i] P[i][j];  dk^T[d][j] += sum_i Q^T[d][i] (ds/|q|)[i][j]
      // with dH^T, Q^T from identity products on re-read rows, one 32-column
      // block of d at a time
      frag pb[NC], db[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        pb[c] = M::pack(s, c * PER);
        db[c] = M::pack(dp, c * PER);
      }
#pragma unroll
      for (int dblk = 0; dblk < NDH; ++dblk) {
#pragma unroll
        for (int op = 0; op < 2; ++op) {  // 0: dH^T P -> dv, 1: Q^T dS -> dk
          frag f[NC], t[NC];
#pragma unroll
          for (int c = 0; c < NC; ++c)
            f[c] = op == 0 ? S::frag(hl, 32 * qh + m, dblk * NC + c, half, DP)
                           : S::frag(ql, 32 * qh + m, dblk * NC + c, half, a.D);
          f32x16 tr;
#pragma unroll
          for (int r = 0; r < 16; ++r) tr[r] = 0.0f;
#pragma unroll
          for (int c = 0; c < NC; ++c) tr = M::mma_ng(f[c], ident_frag<T>(c, lane), tr);
#pragma unroll
          for (int c = 0; c < NC; ++c) t[c] = M::pack(tr, c * PER);
          guard_frags(f);
#pragma unroll
          for (int c = 0; c < NC; ++c) {
            if (op == 0) acc_v[dblk] = M::mma_ng(t[c], pb[c], acc_v[dblk]);
            else acc_k[dblk] = M::mma_ng(t[c], db[c], acc_k[dblk]);
          }
          guard_frags(t);
        }
      }
      guard_frags(pb);
      guard_frags(db);
    }

    if (NBUF == 1 && tl[1] >= 0) {
      block_sync_lds();  // every wave is done with the single buffer
      stage_tile(tl[1], 0);
    }
    tl[0] = tl[1];
    tl[1] = tl[2];
    tl[2] = NBUF == 3 ? walk.next() : -1;
    if (NBUF < 3) tl[1] = walk.next();
  }

  // exchange through the (now idle) stage buffers: the qh = 0 wave of each
  // key half finishes dk, the qh = 1 wave dv
  __syncthreads();
  float* red = reinterpret_cast<float*>(&stage[0][0]);  // [4 waves][NDH][16][64]
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r)
      red[((w * NDH + dblk) * 16 + r) * kWave + lane] = qh == 0 ? acc_v[dblk][r] : acc_k[dblk][r];
  dr_acc = wave_sum(dr_acc);
  dw_acc = wave_sum(dw_acc);
  if (lane == 0) { rw[0][w] = dr_acc; rw[1][w] = dw_acc; }
  __syncthreads();
  f32x16 fin[NDH];
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float other = red[(((w ^ 2) * NDH + dblk) * 16 + r) * kWave + lane];
      fin[dblk][r] = qh == 0 ? acc_k[dblk][r] + other : other + acc_v[dblk][r];
    }
  {
    frag xf[NKS];  // own raw k (qh = 0) or v (qh = 1) rows, from LDS
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) xf[ks] = kvl[(qh * NKS + ks) * kWave + lane];
    write_norm_bwd<T, DP>(fin, xf, jvalid, a.D, a.eps, half, (T*)(qh == 0 ? a.dk : a.dv) + orow);
  }
  if (tid == 0) {
    const int64_t nbh = (int64_t)a.B * a.H;
    a.part[(int64_t)bh * a.nkt + kt] = (rw[0][0] + rw[0][1]) + (rw[0][2] + rw[0][3]);
    a.part[nbh * a.nkt + (int64_t)bh * a.nkt + kt] = (rw[1][0] + rw[1][1]) + (rw[1][2] + rw[1][3]);
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

// Workspace: [dr/dw partials][dh][1/|q|], each 256-byte aligned.
static int64_t bwd_part_bytes(const Geometry& g) { return round_up((int64_t)2 * g.B * g.H * g.nkt * 4, 256); }
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
  ka.dq = c.dq; ka.dk = c.dk; ka.dv = c.dv;
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
  hipLaunchKernelGGL((dq_kernel<T, DP>), dim3((unsigned)g.nqt, (unsigned)(g.B * g.H)), dim3(256), 0, c.stream, ka);
  timer_end(5, c.stream);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(4, c.stream);
  hipLaunchKernelGGL((dkdv_kernel<T, DP>), dim3((unsigned)g.nkt, (unsigned)(g.B * g.H)), dim3(256), 0, c.stream, ka);
  timer_end(4, c.stream);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  timer_begin(6, c.stream);
  hipLaunchKernelGGL(rw_reduce_kernel, dim3((unsigned)g.H), dim3(256), 0, c.stream, (const float*)ka.part, c.dr, c.dw,
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
