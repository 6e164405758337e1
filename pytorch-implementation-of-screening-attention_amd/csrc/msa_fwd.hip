// Forward path of fused Screening Attention on gfx950.
//
//   prep_k_kernel : unit-normalised K^ rows (attention.py:156-157) in a padded
//                   [b*h][Tk_pad][DP] buffer; key padding (attention.py:185-188)
//                   is folded in as a zero row (s = 0 gives alpha = 0: r > 1).
//                   Its first row of blocks plans the screen's work (below).
//   fwd_screen_kernel : 256-thread block = 4 waves, wave -> one 64-query tile
//                   of one head; in step n every wave takes the key tile at
//                   the same tile offset from its query tile, so the waves
//                   reach the window's edges together.  Key tiles stream
//                   global -> LDS by direct DMA into a ring (each tile is read
//                   by the 4 waves in 4 consecutive steps).  Each wave forms
//                   S^T = K^ Q^T on fp16 MFMA (the raw query rows rounded to
//                   fp16, fp32 accumulation, scaled by 1/|q_i|) and votes whether any in-window pair passes the
//                   trim-and-square threshold (attention.py:75-90).  Output:
//                   the live-unit bitmap (32x32 units).
//   fwd_live_kernel : one wave per 32-query unit (S waves for launches with few
//                   units, each taking every S-th live unit); walks the unit's live bits,
//                   recomputes S^T from the raw K rows (exact products, fp32
//                   1/|k|) for those key units only, forms alpha*m
//                   (attention.py:92-119) and accumulates H^T += V^T P^T with
//                   1/|v_j| folded into P.  The epilogue applies TanhNorm
//                   (norm.py:23-25) and writes y in (B,T,H,D) and |h| per row.
//                   No T x T matrix is ever materialised.
#include <type_traits>

#include "msa_device.h"
#include "msa_internal.h"

namespace msa {

// ---------------------------------------------------------------------------
// Screen work plan.  The hardware places the blocks of a launch statically:
// block p runs on XCD p % 8 and, within that XCD, on shader engine
// perm[(p >> 3) % 4] (a fixed permutation per XCD, measured on MI355X with
// per-block hardware-id stamps); only the choice among the engine's 8 CUs is
// dynamic.  So a launch is 32 "lanes" (XCD, engine) of 8 CUs, each taking
// its blocks in order, and the screen's makespan is set by the busiest lane
// and by its longest block.  The plan cuts each 4-query-tile group's range
// of tile offsets (one screen step each) into items of at most `seg` steps,
// near-equal in length,
// sorts items longest first and deals them over lanes in boustrophedon
// order, so every lane gets an equal share and runs its longest items first:
//   per-XCD mode (B*H >= 32): heads are dealt to XCDs widest window first in
//     boustrophedon order and stay there (a head's K^ stays in one L2); each
//     XCD's items are dealt over its 4 engine lanes;
//   group mode (fewer heads, where one XCD per head would leave XCDs idle or
//     overloaded): XCD x takes groups x, x+8, ... of every head, and deals
//     them over its 4 engine lanes.
// Either way each XCD's plan is made by one planner block of its own.
// Screen block p takes entry (p % 8, (p >> 3) % 4, p >> 5) of the table;
// positions past a lane's items hold bh = -1 (the block exits at once).
// Which items run where changes only the time, never the bitmap (live bits
// are ORed).
// ---------------------------------------------------------------------------
constexpr int kScreenBlocksPerLane = 256;
struct ScreenItem {
  int bh, grp, lo, hi;  // head, 4-query-tile group, tile offsets qt - kt in [lo, hi]
  float r, w;           // the head's r_h, w_h (copied, so one load gives the screen all)
  int pad[2];
};
struct ScreenPlan {
  ScreenItem* table;  // [8 XCDs][4 engine lanes][kmax]
  int kmax;           // positions per lane
  int seg;            // steps (tile offsets) per item at most (<= 256)
  int per_xcd;        // 1: per-XCD mode, 0: group mode
};

struct PrepKArgs {
  const void* k; Strides3 ks;
  const uint8_t* kpm;
  void* khat;
  uint32_t* bits;
  int64_t bits_per_bh;  // bitmap words per (b, h)
  int B, H, Tq, Tk, D, nqt, causal;
  int64_t Tk_pad;
  float eps;
  const float* r; const float* w;
  ScreenPlan plan;
};

// Per-XCD mode: the heads of XCD x.  Heads are ranked widest window first
// (NaN keyed as widest, ties by index: a permutation); rank k goes to XCD
// (k/8 odd ? 7 - k%8 : k%8) as its (k/8)-th head.  Above kPlanMaxRanked heads
// the ranking is skipped: slot jh of XCD x is head 8*jh + x.  The count
// follows the same rule as the assignment in each mode, so every slot below
// it holds a head and every head has a slot.
constexpr int kPlanMaxRanked = 512;
constexpr int kPlanMaxHeads = 512;  // head slots a planner block keeps in LDS
__device__ inline int xcd_head_count(int BH, int x) {
  const bool ranked = BH <= kPlanMaxRanked;
  int nh = 0;
  for (int jh = 0; 8 * jh < BH; ++jh) nh += 8 * jh + (ranked && (jh & 1) ? 7 - x : x) < BH ? 1 : 0;
  return nh;
}
// keys[h] (the window ranking key of head h) are in LDS when B*H <= kPlanMaxRanked.
__device__ inline void plan_heads(const PrepKArgs& a, int x, int* heads, const float* keys) {
  const int BH = a.B * a.H;
  if (BH > kPlanMaxRanked) {
    for (int jh = threadIdx.x; 8 * jh < BH && jh < kPlanMaxHeads; jh += blockDim.x)
      if (8 * jh + x < BH) heads[jh] = 8 * jh + x;
    return;
  }
  for (int bh = threadIdx.x; bh < BH; bh += blockDim.x) {
    const float key = keys[bh % a.H];
    int rank = 0;
    for (int o = 0, ho = 0; o < BH; ++o) {
      const float ko = keys[ho];
      rank += (ko > key || (ko == key && o < bh)) ? 1 : 0;
      ho = ho + 1 == a.H ? 0 : ho + 1;
    }
    const int jh = rank >> 3, xr = (jh & 1) ? 7 - (rank & 7) : (rank & 7);
    if (xr == x) heads[jh] = bh;
  }
}

// Integer window as head_params forms it.
__device__ inline int plan_wc(float w) {
  const float c = ceilf(w);
  return !(c > 0.0f) ? 0 : (c > 1073741824.0f ? 1073741824 : (int)c);
}

// Tile offsets o = qt - kt of the key tiles kt in the windows of a group's
// query tiles qt = 4grp .. 4grp+3 (< nqt): the union of each tile's range
// [qt - hi, qt - lo] (its key tiles [lo, hi]); false if no tile has a key.
// Every tile's range is an interval and the intervals overlap, so the union
// is one interval.  wc <= 2^30 and positions < 2^22: no overflow.
__host__ __device__ inline bool group_offsets(int Tq, int Tk, int nqt, int wc, bool causal, int grp, int& olo,
                                              int& ohi) {
  olo = 0x7fffffff;
  ohi = -0x7fffffff;
  for (int w = 0; w < 4; ++w) {
    const int qt = grp * 4 + w;
    if (qt >= nqt) break;
    const int qa = qt * kTile, qb = qa + kTile - 1 < Tq - 1 ? qa + kTile - 1 : Tq - 1;
    int jlo = qa - wc + 1;
    int jhi = causal ? qb : (wc - 1 > Tk ? Tk : qb + wc - 1);
    if (jlo < 0) jlo = 0;
    if (jhi > Tk - 1) jhi = Tk - 1;
    if (jhi < jlo) continue;
    const int a = qt - jhi / kTile, b = qt - jlo / kTile;
    olo = a < olo ? a : olo;
    ohi = b > ohi ? b : ohi;
  }
  return olo <= ohi;
}

// Visits the planned items: fn(bh, grp, olo, ohi) for each (head slot, group)
// pair's near-equal cut of its offset range into ceil(steps / seg) items, over
// groups g0, g0 + gstep, ...  heads[slot] and the integer windows wcs[slot]
// are in LDS for the first kPlanMaxHeads slots; beyond them (per-XCD mode
// without ranking only) slot jh is head 8*jh + x.
template <typename Fn>
__device__ inline void plan_items(const PrepKArgs& a, int x, const int* heads, const int* wcs, int nh, int g0,
                                  int gstep, Fn&& fn) {
  const int ngroups = (a.nqt + 3) / 4;
  const int ng = ngroups > g0 ? (ngroups - g0 + gstep - 1) / gstep : 0;  // groups visited per head
  const bool causal = a.causal != 0;
  const int seg = a.plan.seg;
  for (int idx = threadIdx.x; idx < nh * ng; idx += blockDim.x) {
    const int slot = idx / ng, grp = g0 + (idx - slot * ng) * gstep;
    const bool cached = slot < kPlanMaxHeads;
    const int bh = cached ? heads[slot] : 8 * slot + x;
    const int wc = cached ? wcs[slot] : plan_wc(a.w[bh % a.H]);
    int olo, ohi;
    if (!group_offsets(a.Tq, a.Tk, a.nqt, wc, causal, grp, olo, ohi)) continue;
    const int steps = ohi - olo + 1;
    const int n = (steps + seg - 1) / seg, base = steps / n, rem = steps - base * n;
    // pieces in the order the screen walks offsets (descending)
    for (int i = 0, s1 = ohi; i < n; ++i) {
      const int len = base + (i < rem ? 1 : 0);
      fn(bh, grp, s1 - len + 1, s1);
      s1 -= len;
    }
  }
}

// Boustrophedon deal of sorted position i over nl lanes: (lane, slot).
__device__ inline void plan_deal(int i, int nl, int& e, int& j) {
  j = i / nl;
  const int r = i - j * nl;
  e = (j & 1) ? nl - 1 - r : r;
}

// Planner block x (256 threads) writes the 4 lanes of XCD x: in per-XCD mode
// from the heads dealt to it, in group mode from groups x, x+8, ... of every
// head.
__device__ void screen_plan(const PrepKArgs& a, int x) {
  __shared__ int heads[kPlanMaxHeads], wcs[kPlanMaxHeads];
  __shared__ float keys[kPlanMaxRanked], rh[kPlanMaxRanked], wh[kPlanMaxRanked];
  __shared__ int wch[kPlanMaxRanked];
  __shared__ int hist[257], start[257];
  __shared__ int total;
  const bool per_xcd = a.plan.per_xcd != 0;
  const int t = threadIdx.x, nl = 4, kmax = a.plan.kmax;
  const int g0 = per_xcd ? 0 : x, gstep = per_xcd ? 1 : 8;
  for (int i = t; i < 257; i += blockDim.x) hist[i] = 0;
  const int BH = a.B * a.H;
  const int nh = per_xcd ? xcd_head_count(BH, x) : BH;  // group mode: BH < 32
  // the one global read of the windows (the planner runs beside prep_k's
  // stream, where every dependent memory round trip is slow)
  const bool small_h = a.H <= kPlanMaxRanked;
  if (small_h)
    for (int h = t; h < a.H; h += blockDim.x) {
      const float wf = a.w[h];
      keys[h] = window_rank_key(wf);
      wch[h] = plan_wc(wf);
      rh[h] = a.r[h];
      wh[h] = wf;
    }
  __syncthreads();
  if (per_xcd) {
    plan_heads(a, x, heads, keys);
  } else {
    for (int i = t; i < nh; i += blockDim.x) heads[i] = i;
  }
  __syncthreads();
  for (int i = t; i < nh && i < kPlanMaxHeads; i += blockDim.x) {
    const int h = heads[i] % a.H;
    wcs[i] = small_h ? wch[h] : plan_wc(a.w[h]);
  }
  __syncthreads();
  // items by length (at most seg <= 256), longest first; the order among
  // items of one length is whatever the atomics give (it only moves time)
  plan_items(a, x, heads, wcs, nh, g0, gstep, [&](int, int, int lo, int hi) { atomicAdd(&hist[hi - lo + 1], 1); });
  __syncthreads();
  if (t < 64) {  // exclusive prefix over lengths 256 .. 1: lane t holds 256-4t .. 253-4t
    int v[4], sum = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      v[k] = hist[256 - 4 * t - k];
      sum += v[k];
    }
    int incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int y = __shfl_up(incl, o);
      if (t >= o) incl += y;
    }
    int acc = incl - sum;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      start[256 - 4 * t - k] = acc;
      acc += v[k];
    }
    if (t == 63) total = incl;
  }
  __syncthreads();
  // lane e of this planner -> table lane (XCD x, engine e)
  auto lane_base = [&](int e) -> ScreenItem* { return a.plan.table + (x * 4 + e) * kmax; };
  plan_items(a, x, heads, wcs, nh, g0, gstep, [&](int bh, int grp, int lo, int hi) {
    const int pos = atomicAdd(&start[hi - lo + 1], 1);
    int e, j;
    plan_deal(pos, nl, e, j);
    const int h = bh % a.H;
    const float r = small_h ? rh[h] : a.r[h], w = small_h ? wh[h] : a.w[h];
    if (j < kmax) lane_base(e)[j] = ScreenItem{bh, grp, lo, hi, r, w, {0, 0}};  // j < kmax always (kmax bounds the items)
  });
  // positions past each lane's items: empty
  const int n = total, full = n / nl, r = n - full * nl;
  for (int e = 0; e < nl; ++e) {
    const bool extra = r > 0 && ((full & 1) ? e >= nl - r : e < r);
    ScreenItem* lb = lane_base(e);
    for (int j = full + (extra ? 1 : 0) + t; j < kmax; j += blockDim.x) lb[j] = ScreenItem{-1, 0, 0, -1, 0.0f, 0.0f, {0, 0}};
  }
}

// Plan dimensions from the shape alone (the windows live on the device):
// seg = clamp(ceil(5*nkt/16), 8, 256) steps per item, and kmax bounds a
// lane's items as if every window were unbounded.
void screen_plan_dims(const Geometry& g, int& seg, int& kmax, int& per_xcd) {
  seg = (5 * g.nkt + 15) / 16;
  seg = seg < 8 ? 8 : (seg > 256 ? 256 : seg);
  const int64_t BH = (int64_t)g.B * g.H;
  // group mode for few heads; per-XCD mode keeps at most kPlanMaxHeads per XCD
  per_xcd = BH >= 32 ? 1 : 0;
  const int ngroups = (g.nqt + 3) / 4;
  int64_t per_head = 0, per_class[8] = {0, 0, 0, 0, 0, 0, 0, 0};  // items of groups = x mod 8
  for (int grp = 0; grp < ngroups; ++grp) {
    int olo, ohi;
    if (group_offsets(g.Tq, g.Tk, g.nqt, 1 << 30, g.causal != 0, grp, olo, ohi)) {
      const int64_t n = (ohi - olo + 1 + seg - 1) / seg;
      per_head += n;
      per_class[grp % 8] += n;
    }
  }
  int64_t items = (BH + 7) / 8 * per_head;  // per-XCD mode: the most heads an XCD holds
  if (!per_xcd) {
    items = 0;
    for (int c = 0; c < 8; ++c) items = per_class[c] > items ? per_class[c] : items;
    items *= BH;
  }
  const int64_t k = (items + 3) / 4;
  kmax = (int)(k > 0 ? k : 1);
}
size_t screen_plan_bytes(const Geometry& g) {
  int seg, kmax, per_xcd;
  screen_plan_dims(g, seg, kmax, per_xcd);
  return round_up((int64_t)32 * kmax * (int64_t)sizeof(ScreenItem), 256);
}

// ---------------------------------------------------------------------------
// Screen operands.  Every input type screens on fp16 MFMA operands: K^ =
// k/|k| rounded to fp16, and each raw query row rounded to fp16, so each vote
// sees s up to their rounding: |s_screen - s| <= (u_k + u_q + u_k u_q)
// sum_d |q^_d k^_d| <= u_k + u_q + u_k u_q (unit roundoffs, unit vectors).
// The live-unit bitmap must hold every pair with alpha > 0 (the live and
// backward passes visit nothing else, and a missed pair's gradient terms are
// linear in a = 1 - r(1-s)), so the vote's gate is lowered by that bound.
// The operands are power-of-two scaled into fp16's normal range, which keeps
// their rounding relative: K^ times 2^10 (its components are at most 1, and
// down to 2^-24 stay normal), each raw query row times the 2^e that puts its
// largest component in [2^10, 2^11) (components below 2^-24 of the largest
// become subnormal: an absolute error of at most 2^-35 of |q| each).
//   bf16 and fp16 inputs: the query rows are exact in fp16 (bf16 has 8
//     significant bits, fp16 11), so u_q = 0 and u_k = 2^-11 (fp16 keeps 11
//     significant bits).  fp16, not bf16 (u_k = 2^-8, at the same MFMA rate),
//     because the lowered gate then admits about 2% more 32x32 units than
//     hold a live pair instead of about 18% (counted on the configs[1]
//     inputs).
//   fp32 inputs: u_q = u_k = 2^-11, on the fp16 MFMA (16x the fp32 MFMA rate,
//     a quarter of the operand bytes).
// The vote's gate, in s, is 1 - 1/r - kScreenSlack, the slack covering the
// rounding above, fp32 accumulation of D <= 128 products ((D+3) 2^-24) and
// the fp32 1/|q| and 1/|k|.
// ---------------------------------------------------------------------------
using ScreenOp = f16;              // the screen's MFMA operand type
constexpr float kKhatScale = 1024.0f;  // K^ is stored times 2^10
template <typename T>
constexpr float kScreenSlack = sizeof(T) == 2 ? 4.8828125e-4f + 1e-5f    // 2^-11 + 1e-5
                                              : 9.765625e-4f + 1e-5f;    // 2^-10 + 1e-5

// A query row of fp32 inputs in the 16-bit operand layout (the lane holds
// elements KS*ks + PER*half + e, e < PER, as PRow<bf16, DP>), kept in fp32
// until the screen rounds it to an fp16 operand.
template <int DP>
struct WideQueryRow {
  static constexpr int KS = Mma<f16>::KS, PER = Mma<f16>::PER, NKS = DP / KS;
  float f[NKS][PER];
  __device__ inline void load(const float* p, bool ok, int D, int half) {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d0 = KS * ks + PER * half;
      const bool in = ok && d0 < D;
      const float* s = p + (d0 < D ? d0 : 0);
#pragma unroll
      for (int e = 0; e < PER; e += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(s + e);
#pragma unroll
        for (int j = 0; j < 4; ++j) f[ks][e + j] = in ? v[j] : 0.0f;
      }
    }
  }
  __device__ inline float get(int ks, int e) const { return f[ks][e]; }
  __device__ inline float inv_norm(float eps) const {
    float s = 0.0f;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int e = 0; e < PER; ++e) s += f[ks][e] * f[ks][e];
    return inv_len(half_sum(s), eps);
  }
};
// The screen's view of a raw query row: 2-byte rows as loaded, fp32 rows wide.
template <typename T, int DP>
using ScreenQueryRow = typename std::conditional<sizeof(T) == 2, PRow<T, DP>, WideQueryRow<DP>>::type;

// Power of two p with max|x| * p in [2^10, 2^11) (1 for a zero or non-finite
// max): scales a query row into fp16's normal range exactly.
__device__ inline float row_pow2(float mx) {
  if (!(mx > 0.0f) || !(mx < INFINITY)) return 1.0f;
  int ex;
  (void)frexpf(mx, &ex);  // mx = m 2^ex, m in [0.5, 1)
  int e = 11 - ex;
  e = e > 126 ? 126 : (e < -126 ? -126 : e);
  return ldexpf(1.0f, e);
}

// 16-byte chunk per thread per row; a key row of DP elements spans CPR
// threads, and a thread covers kPrepRows rows RPB apart (all loads first).
constexpr int kPrepRows = 4;
template <typename T, int DP>
__global__ __launch_bounds__(256) void prep_k_kernel(PrepKArgs a) {
  constexpr int VEC = 16 / (int)sizeof(T);
  constexpr int CPR = DP / VEC;  // chunks per row (power of two, <= 32)
  constexpr int RPB = 256 / CPR;
  if (blockIdx.y == 0) {  // the first row plans the screen, one block per XCD
    if (blockIdx.x < 8) screen_plan(a, blockIdx.x);
    return;
  }
  const int bh = blockIdx.y - 1, b = bh / a.H, h = bh % a.H;
  const int d0 = (threadIdx.x % CPR) * VEC;
  float x[kPrepRows][VEC];
#pragma unroll
  for (int u = 0; u < kPrepRows; ++u) {
    const int64_t t = ((int64_t)blockIdx.x * kPrepRows + u) * RPB + threadIdx.x / CPR;
    const bool valid = t < a.Tk && d0 < a.D;
    // one 16-byte load per row chunk (rows past Tk read row 0, then zeroed)
    load_chunk((const T*)a.k + b * a.ks.sb + (valid ? t : 0) * a.ks.st + h * a.ks.sh + (d0 < a.D ? d0 : 0), x[u]);
    if (!valid) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) x[u][e] = 0.0f;
    }
  }
#pragma unroll
  for (int u = 0; u < kPrepRows; ++u) {
    const int64_t t = ((int64_t)blockIdx.x * kPrepRows + u) * RPB + threadIdx.x / CPR;
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < VEC; ++e) ss += x[u][e] * x[u][e];
    ss = group_sum<CPR>(ss);  // the row's CPR lanes
    float inv = kKhatScale / fmaxf(sqrtf(ss), a.eps);
    if (t >= a.Tk || (a.kpm != nullptr && a.kpm[(int64_t)b * a.Tk + t])) inv = 0.0f;
    if (t < a.Tk_pad) {
      ScreenOp* p = (ScreenOp*)a.khat + ((int64_t)bh * a.Tk_pad + t) * DP + d0;
#pragma unroll
      for (int e = 0; e < VEC; e += 4)
        store4(p + e, x[u][e] * inv, x[u][e + 1] * inv, x[u][e + 2] * inv, x[u][e + 3] * inv);
    }
  }
  // clear this head's live-tile bitmap rows; the screen ORs live bits in
  uint32_t* brow = a.bits + (int64_t)bh * a.bits_per_bh;
  for (int64_t wi = (int64_t)blockIdx.x * 256 + threadIdx.x; wi < a.bits_per_bh; wi += (int64_t)gridDim.x * 256)
    brow[wi] = 0u;
}

struct FwdKArgs {
  const void* q; Strides3 qs;
  const void* k; Strides3 ks;
  const void* v; Strides3 vs;
  const uint8_t* kpm;
  const void* khat;
  const float* r; const float* w;
  void* y; float* hnorm; uint32_t* bits;
  Dropout drop;
  int H, Tq, Tk, D, nqt, nku_words, causal;
  int64_t Tk_pad;
  float eps;
  ScreenPlan plan;
};

// Range [lo, hi] of the U-key blocks that hold the window of queries [qa, qb].
template <int U>
__device__ inline void key_range(const FwdKArgs& a, const HeadParams& hp, bool causal, int64_t qa, int64_t qb,
                                 int& lo, int& hi) {
  int64_t jlo = qa - hp.wc + 1;
  int64_t jhi = causal ? qb : qb + hp.wc - 1;
  if (jlo < 0) jlo = 0;
  if (jhi > a.Tk - 1) jhi = a.Tk - 1;
  lo = (int)(jlo / U);
  hi = jhi >= jlo ? (int)(jhi / U) : lo - 1;
}
__device__ inline void key_tile_range(const FwdKArgs& a, const HeadParams& hp, bool causal, int64_t qa, int64_t qb,
                                      int& lo, int& hi) {
  key_range<kTile>(a, hp, causal, qa, qb, lo, hi);
}

template <typename T, int DP>
struct ScreenTile {
  static constexpr int ROWB = DP * (int)sizeof(T);   // bytes per key row
  static constexpr int CPR = ROWB / 16;              // 16-byte chunks per row (power of two)
  static constexpr int TILEB = 64 * ROWB;            // bytes per staged key tile
  static constexpr int CPT = 64 * CPR / 256;         // DMA chunks per thread per tile
  // ring slots: the 4 tiles the waves read in a step plus the tiles in flight
  // (2 for tiles up to 8 KiB: 48 KiB a block, three blocks a CU; 1 above)
  static constexpr int NS = TILEB <= 8192 ? 6 : 5;
  // LDS chunk position of global chunk c of row R: c ^ swz(R), conflict-free
  // for the perm_row operand reads
  __device__ static inline int swz(int R) { return lds_swz<CPR>(R); }
};

// Floor and ceiling of x / kTile for any sign.
__device__ inline int floor_tiles(int x) { return x >= 0 ? x / kTile : -((-x + kTile - 1) / kTile); }
__device__ inline int ceil_tiles(int x) { return -floor_tiles(-x); }

// ---------------------------------------------------------------------------
// Screen: 256-thread block = 4 waves, wave w -> query tile qt = 4grp + w of
// one head.  Each block runs one item of the plan (prep_k_kernel): a group
// and a range [olo, ohi] of tile offsets o = qt - kt.  Step n takes offset
// o = ohi - n for all four waves at once, so wave w reads key tile
// kt = 4grp - ohi + n + w: the waves meet the diagonal and the start of the
// window in the same step, and the steps between are the same straight-line
// code for all of them.  A step's four key tiles are consecutive; each step
// brings in one more tile, which streams global -> LDS by direct DMA into a
// ring of NS slots two steps ahead (one raw barrier per step).  Chunks are
// XOR-swizzled within each key row so the A-operand reads spread over the
// LDS banks.  Each wave forms S^T = K^ Q^T on MFMA for its tile and votes
// whether any in-window pair passes the trim-and-square threshold; live bits
// are ORed into the bitmap (cleared by prep_k_kernel), so items that share a
// bitmap word need no ordering.
// ---------------------------------------------------------------------------
template <typename T, int DP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void fwd_screen_kernel(FwdKArgs a) {
  using S = ScreenOp;  // operand type of the screen's MFMAs
  using M = Mma<S>;
  using frag = typename M::frag;
  using G = ScreenTile<S, DP>;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NS = G::NS;
  __shared__ __attribute__((aligned(16))) char ring[NS * G::TILEB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform values live in SGPRs
  const int half = lane >> 5, l32 = lane & 31;
  const int nkt = (int)(a.Tk_pad / kTile);
  // this block's lane: (XCD p % 8, engine (p >> 3) % 4); it runs the lane's
  // items at positions p >> 5, (p >> 5) + K, ... (K blocks per lane), which
  // are sorted longest first and end with empty entries
  const int p = blockIdx.x;
  const ScreenItem* lane_items = a.plan.table + ((p & 7) * 4 + ((p >> 3) & 3)) * a.plan.kmax;
  const int kstride = (int)(gridDim.x >> 5);
  for (int pos = p >> 5; pos < a.plan.kmax; pos += kstride) {
  // the whole entry in one round trip (the asm keeps the compiler from
  // splitting the loads at the test)
  const int4 item = *(const int4*)(lane_items + pos);
  const float4 irw = *((const float4*)(lane_items + pos) + 1);
  asm volatile("" ::"v"(item.x), "v"(item.y), "v"(item.z), "v"(item.w), "v"(irw.x), "v"(irw.y));
  if (item.x < 0) break;  // block-uniform: past this lane's items
  const int bh = item.x, grp = item.y, olo = item.z, ohi = item.w;
  const int b = bh / a.H, h = bh % a.H;
  const bool causal = a.causal != 0;
  const int qt = grp * 4 + wave;
  const bool wave_ok = qt < a.nqt;
  const int q0 = qt * kTile;

  // The own query rows (raw B operands) and the first key tiles' DMA need
  // only the item: they are issued first, and the head parameters and tile
  // ranges are formed while they are in flight.
  ScreenQueryRow<T, DP> qrow[2];
#pragma unroll
  for (int qh = 0; qh < 2; ++qh) {
    const int i = q0 + 32 * qh + l32;
    const bool ok = wave_ok && i < a.Tq;
    qrow[qh].load((const T*)a.q + b * a.qs.sb + (int64_t)(ok ? i : 0) * a.qs.st + h * a.qs.sh, ok, a.D, half);
  }
  __builtin_amdgcn_sched_barrier(0);  // query loads issue before the DMA
  frag qf[2 * NKS];
  float qthr[2];  // vote threshold on acc for this lane's query of unit qh
  // bitmap rows of the wave's two query units (32 queries each)
  uint32_t* brow = a.bits + ((int64_t)bh * 2 * a.nqt + 2 * (wave_ok ? qt : 0)) * a.nku_words;

  // DMA: chunk c = u*256 + tid of a tile (row c / CPR, LDS position c % CPR)
  // comes from global chunk position ^ swz(row) of that row; the per-lane
  // byte offset inside a tile is fixed, the tile base is uniform.
  const char* kg = (const char*)a.khat + (int64_t)bh * a.Tk_pad * G::ROWB;
  uint32_t goff[G::CPT];
#pragma unroll
  for (int u = 0; u < G::CPT; ++u) {
    const int c = u * 256 + tid;
    const int row = c / G::CPR, pc = c % G::CPR;
    goff[u] = (uint32_t)(row * G::ROWB + ((pc ^ G::swz(row)) << 4));
  }
  // The item's tiles in step order: tile number u is key tile A0 + u (wave w
  // reads number n + w in step n) and sits in ring slot u % NS.  Numbers
  // outside the key tiles any wave reads load a clamped tile instead (their
  // slot is never read), so every step waits for the same count.
  const int nsteps = ohi - olo + 1, A0 = grp * 4 - ohi;
  int tmin = A0 < 0 ? 0 : A0, tmax = A0 + nsteps + 2 < nkt - 1 ? A0 + nsteps + 2 : nkt - 1;
  if (tmin > nkt - 1) tmin = nkt - 1;
  if (tmax < tmin) tmax = tmin;
  auto issue = [&](int u, int slot_idx) {
    int kt = A0 + u;
    kt = kt < tmin ? tmin : (kt > tmax ? tmax : kt);
    const char* tb = kg + (int64_t)kt * G::TILEB;
#pragma unroll
    for (int c = 0; c < G::CPT; ++c)
      __builtin_amdgcn_global_load_lds(
          (const void __attribute__((address_space(1)))*)(tb + goff[c]),
          (void __attribute__((address_space(3)))*)(ring + slot_idx * G::TILEB + (c * 256 + wave * 64) * 16), 16, 0,
          0);
  };
#pragma unroll
  for (int u = 0; u < NS - 1; ++u) issue(u, u);
  __builtin_amdgcn_sched_barrier(0);

  const HeadParams hp = head_params_rw(irw.x, irw.y, causal);
  int kt_lo, kt_hi;
  key_tile_range(a, hp, causal, q0, q0 + 63 < a.Tq - 1 ? q0 + 63 : a.Tq - 1, kt_lo, kt_hi);
  if (!wave_ok) { kt_lo = 0; kt_hi = -1; }

  // A-operand rows of key half kh: row 32kh + perm_row(l32), 16-byte chunk
  // (KS*ks + PER*half)*sizeof(S)/16 = ks*KS*sizeof(S)/16 + half*PER*sizeof(S)/16
  uint32_t aoff[2][NKS];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int R = 32 * kh + perm_row(l32);
      const int byte = (KS * ks + PER * half) * (int)sizeof(S);
      aoff[kh][ks] = (uint32_t)(R * G::ROWB + ((((byte >> 4) ^ G::swz(R)) << 4) | (byte & 15)));
    }

  // MFMAs of key half kh of the staged tile: acc[qh] = K^ rows 32kh + perm x Q^T
  auto half_mma = [&](const char* slot, int kh, f32x16 (&acc)[2]) {
    frag kf[NKS];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) kf[ks] = M::load((const S*)(slot + aoff[kh][ks]));
#pragma unroll
    for (int qh = 0; qh < 2; ++qh)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[qh][r] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) acc[qh] = M::mma_ng(kf[ks], qf[qh * NKS + ks], acc[qh]);
    guard_frags(kf);
  };
  // Threshold vote on key half kh of the tile at k0: a(s) is monotone in s and
  // s = acc/(|q_i| c_i) (c_i: the operands' power-of-two scales), so a 32x32
  // unit has a live pair iff its largest in-window acc exceeds
  // (1 - 1/r)|q_i| c_i.  The vote compares with qthr, that threshold lowered
  // by kScreenSlack, so every unit with a live pair is marked, and a unit
  // whose pairs all lie within the slack below the threshold may be marked
  // too; the live pass's exact test gives those pairs alpha = 0.
  // The compare's lane mask is the wave's vote, so the result is
  // wave-uniform: bit qh set iff unit (qh, kh) has a passing pair.  Register r
  // of the half holds key k0 + 32kh + 16(r/8) + 8half + r%8.  Tiles wholly
  // inside every pair's window skip the per-register window test; in the
  // other tiles each 32x32 unit is classed by its distance range c-31 .. c+31
  // (the window is one interval of distances): wholly inside (plain maximum),
  // wholly outside (no vote) or cut by a window edge (per-register test).
  auto vote_half = [&](const f32x16 (&acc)[2], int k0, int kh, bool interior) -> int {
    int lv = 0;
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
      float mx = -INFINITY;
      const int c = q0 + 32 * qh - k0 - 32 * kh;  // wave-uniform
      if (interior || (in_window(c - 31, hp) && in_window(c + 31, hp))) {
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, acc[qh][r]);
      } else if (c + 31 + hp.wsh >= 0 && c - 31 + hp.wsh < (int)hp.wlim) {
        const int rel0 = (q0 + 32 * qh + l32) - k0 - 32 * kh - 8 * half;
#pragma unroll
        for (int r = 0; r < 16; ++r)
          mx = fmaxf(mx, in_window(rel0 - (16 * (r >> 3) + (r & 7)), hp) ? acc[qh][r] : -INFINITY);
      }
      lv |= (__ballot(mx > qthr[qh]) != 0ull ? 1 : 0) << qh;
    }
    return lv;
  };
  // Live tiles are rare (a few percent of the window): one lane ORs the bits
  // of tile kd's live units into the bitmap (cleared by prep_k_kernel), so
  // items that share a bitmap word need no ordering.  v0, v1: the votes
  // of key halves 0 and 1 (bit qh, wave-uniform).
  auto finish = [&](int kd, int v0, int v1) {
    if ((v0 | v1) != 0 && wave_ok) {
      // row qh, key units 2kd (bit 0) and 2kd + 1 (bit 1): one word
      const uint32_t m0 = (uint32_t)((v0 & 1) | ((v1 & 1) << 1));
      const uint32_t m1 = (uint32_t)(((v0 >> 1) & 1) | (((v1 >> 1) & 1) << 1));
      const int u = 2 * kd;
      if (lane == 0 && m0 != 0u) atomicOr(&brow[u >> 5], m0 << (u & 31));
      if (lane == 0 && m1 != 0u) atomicOr(&brow[a.nku_words + (u >> 5)], m1 << (u & 31));
    }
  };

  // Offsets [fa, fb] at which every wave of the group is valid, holds its tile
  // in its key range, and the tile lies wholly inside every pair's window
  // (distances 64o-63 .. 64o+63 inside [-wsh, wlim-1-wsh]): the straight-line
  // step.  Block-uniform, from the four query tiles' key ranges.
  int fa = olo, fb = ohi;
  {
    const int dl = -hp.wsh, du = (int)hp.wlim - 1 - hp.wsh;
    const int ia = ceil_tiles(dl + 63), ib = floor_tiles(du - 63);
    fa = fa > ia ? fa : ia;
    fb = fb < ib ? fb : ib;
    for (int w = 0; w < 4; ++w) {
      const int qw = grp * 4 + w;
      if (qw >= a.nqt) { fa = 1; fb = 0; break; }
      int lw, hw;
      key_tile_range(a, hp, causal, (int64_t)qw * kTile,
                     (int64_t)qw * kTile + 63 < a.Tq - 1 ? (int64_t)qw * kTile + 63 : a.Tq - 1, lw, hw);
      if (hw < lw) { fa = 1; fb = 0; break; }
      fa = fa > qw - hw ? fa : qw - hw;
      fb = fb < qw - lw ? fb : qw - lw;
    }
  }
  // the first straight-line offset is taken by the general step, so each
  // straight-line step's predecessor is one as well
  const int n_fast0 = fa <= fb - 1 ? ohi - (fb - 1) : nsteps;  // steps [n_fast0, n_fast1)
  const int n_fast1 = fa <= fb - 1 ? ohi - fa + 1 : nsteps;

  // s = acc/(max(|q|, eps) c) passes the lowered gate iff
  // acc > (1 - 1/r - slack) max(|q|, eps) c, with c = kKhatScale times the
  // row's power of two (a negative gate, r within the slack of 1, marks every
  // unit with a pair above it: still a superset of the live units)
  {
    const float vthr = 1.0f - 1.0f / hp.r - kScreenSlack<T>;
#pragma unroll
    for (int qh = 0; qh < 2; ++qh) {
      float mx = 0.0f;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int e = 0; e < PER; ++e) mx = fmaxf(mx, fabsf(qrow[qh].get(ks, e)));
      const float c = row_pow2(half_max(mx));
      qthr[qh] = vthr / qrow[qh].inv_norm(a.eps) * (c * kKhatScale);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {  // the row scaled by c, rounded to fp16
        f32x16 t;
#pragma unroll
        for (int e = 0; e < PER; ++e) t[e] = qrow[qh].get(ks, e) * c;
        qf[qh * NKS + ks] = M::pack(t, 0);
      }
    }
  }

  {
    // Software pipeline over the two 32-key halves of each tile: the vote on
    // one half runs while the MFMAs of the next half are in flight.  Order in
    // step n (this wave's tile kt): MFMA(kt, keys 0-31) -> finish tile kt-1
    // (vote on its keys 32-63) -> MFMA(kt, keys 32-63) -> vote(kt, keys 0-31).
    f32x16 acc0[2], acc1[2];
    bool pend = false, pint = false;  // tile kt-1: keys 32-63 pending in acc1
    int live0 = 0;                    // tile kt-1: vote on keys 0-31
    int pk0 = 0;
    int rslot = wave, dslot = NS - 1;  // this wave's read slot, the DMA slot
    // Step n reads numbers n .. n+3 (landed once at most NS-5 younger tiles
    // are outstanding; the barrier covers all waves) and refills the slot of
    // number n-1, which the previous step read last.
    auto enter = [&](int n) -> const char* {
      wait_vmcnt<(NS - 5) * G::CPT>();
      __builtin_amdgcn_s_barrier();
      issue(n + NS - 1, dslot);
      const char* slot = ring + rslot * G::TILEB;
      rslot = rslot + 1 == NS ? 0 : rslot + 1;
      dslot = dslot + 1 == NS ? 0 : dslot + 1;
      return slot;
    };
    // General step: offsets at the window's edges, or where some wave's tile
    // is outside its key range.
    auto step = [&](int n) {
      const char* slot = enter(n);
      const int o = ohi - n, kt = A0 + n + wave;
      const bool mine = kt >= kt_lo && kt <= kt_hi;
      if (mine) half_mma(slot, 0, acc0);
      if (n > 0 && pend) finish(kt - 1, live0, vote_half(acc1, pk0, 1, pint));
      if (mine) {
        half_mma(slot, 1, acc1);
        pint = in_window(kTile * o + 63, hp) && in_window(kTile * o - 63, hp);
        live0 = vote_half(acc0, kt * kTile, 0, pint);
        pk0 = kt * kTile;
      }
      pend = mine;
    };
    // Straight-line step: every wave's tile is in its range and wholly inside
    // the window, and so was the previous one: plain maxima, no branches but
    // the rare live-tile store.
    auto step_inside = [&](int n) {
      const char* slot = enter(n);
      const int kt = A0 + n + wave;
      half_mma(slot, 0, acc0);
      finish(kt - 1, live0, vote_half(acc1, 0, 1, true));
      half_mma(slot, 1, acc1);
      live0 = vote_half(acc0, 0, 0, true);
      pend = true;
      pint = true;
      pk0 = kt * kTile;
    };
    int n = 0;
    for (; n < n_fast0; ++n) step(n);
    for (; n < n_fast1; ++n) step_inside(n);
    for (; n < nsteps; ++n) step(n);
    if (pend) finish(A0 + nsteps - 1 + wave, live0, vote_half(acc1, pk0, 1, pint));
    // the trailing loads have landed and every wave is done with the ring
    // before the next item refills it
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
  }
  guard_frags(qf);
  }  // item loop
}

// ---------------------------------------------------------------------------
// Live units.  One wave (a 64-thread block) per query unit: 32 consecutive
// queries of one head, lane -> query i = 32*qu + l%32.  The wave walks its
// row of the live-unit bitmap; for each live key unit (32 keys) it loads the
// raw K and V rows straight from global memory as MFMA operands, the next
// unit's loads in flight while the current one is computed: S^T = K Q^T on
// the raw values (exact products, as the backward forms it) scaled by
// 1/|k_j| in fp32, alpha*m (attention.py:92-119) with 1/|v_j| folded in
// (fp16: into the V rows), and H^T += V^T P^T with V^T from an identity MFMA
// on the raw V rows.  The
// epilogue applies TanhNorm (norm.py:23-25) and writes y in (B,T,H,D) and |h|
// per row.  Units with no live key unit get y = 0, |h| = 0.
// S > 1 (launches with at most kLiveSplitWaves / S rows, D <= 64): S waves
// per row in one block, wave w taking the row's live units w, w+S, ...; waves
// 1..S-1 hand their partial H^T to wave 0 through LDS, which adds them in
// wave order (fixed, so results repeat bitwise) and runs the epilogue.
// ---------------------------------------------------------------------------
template <typename T, int DP, int S>
__global__ __launch_bounds__(64 * S)
__attribute__((amdgpu_waves_per_eu(sizeof(T) == 2 && DP <= 64 ? 3 : (S > 1 ? (DP <= 32 ? 3 : 2) : 1))))
void fwd_live_kernel(FwdKArgs a) {
  using M = Mma<T>;
  using frag = typename M::frag;
  using R = PRow<T, DP>;
  constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS, NDH = DP / 32, NC = 32 / KS;
  // per wave:
  __shared__ __attribute__((aligned(16))) float sk_w[S][32];  // 1/|k_j| (0 if padded or masked) of the current unit
  __shared__ __attribute__((aligned(16))) float sv_w[S][32];  // 1/|v_j| of the current unit's key rows
  __shared__ float mt_w[S][64];  // soft-mask table of the current unit (unit_mask_table)
  // own raw q operand fragments; with S > 1 the same bytes then take the
  // wave's partial H^T for wave 0 (after the wave's last read of its q)
  constexpr int kQshBytes = NKS * kWave * (int)sizeof(frag);
  constexpr int kPartBytes = NDH * 16 * kWave * 4;
  constexpr int kWaveBytes = S > 1 && kPartBytes > kQshBytes ? kPartBytes : kQshBytes;
  __shared__ __attribute__((aligned(16))) char wbuf[S][kWaveBytes];
  const int lane = (int)(threadIdx.x & 63), half = lane >> 5, l32 = lane & 31;
  const int wave = S > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;
  float* sk = sk_w[wave];
  float* sv = sv_w[wave];
  float* mt = mt_w[wave];
  frag (&qsh)[NKS][kWave] = *reinterpret_cast<frag(*)[NKS][kWave]>(wbuf[wave]);
  int qu, bh;
  float head_r, head_w;
  xcd_interleave_ranked(a.r, a.w, a.H, qu, bh, head_r, head_w);
  const int b = bh / a.H, h = bh % a.H;
  const bool causal = a.causal != 0;
  const HeadParams hp = head_params_rw(head_r, head_w, causal);
  const int i = qu * kUnit + l32;
  const bool valid = i < a.Tq;
  // output row of query i (formed where it is stored, so nothing holds it
  // across the unit loop)
  auto yrow = [&]() { return (T*)a.y + (((int64_t)b * a.Tq + (valid ? i : 0)) * a.H + h) * a.D; };

  int ku_lo, ku_hi;
  {
    const int qa = qu * kUnit, qb = qa + kUnit - 1 < a.Tq - 1 ? qa + kUnit - 1 : a.Tq - 1;
    key_range<kUnit>(a, hp, causal, qa, qb, ku_lo, ku_hi);
  }
  const uint32_t* brow = a.bits + ((int64_t)bh * 2 * a.nqt + qu) * a.nku_words;
  RowWalk walk(brow, ku_lo, ku_hi);
  int cur = walk.next();
  if (cur < 0) {  // block-uniform: no live key unit, y = 0 and |h| = 0
    if (wave != 0) return;
    if (valid) {
      if (half == 0) a.hnorm[(int64_t)bh * a.Tq + i] = 0.0f;
#pragma unroll
      for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * dblk + 8 * g + 4 * half;
          if (d < a.D) store4(yrow() + d, 0.0f, 0.0f, 0.0f, 0.0f);
        }
    }
    return;
  }

  // key row of this lane in unit u: 32u + perm_row(l32) (A-operand order)
  const int m = perm_row(l32);
  const T* kg = (const T*)a.k + b * a.ks.sb + h * a.ks.sh;
  const T* vg = (const T*)a.v + b * a.vs.sb + h * a.vs.sh;
  // The lane's chunks (elements KS*ks + PER*half) of its raw K or V row of
  // key unit u, from one row address and immediate offsets: a wave-uniform
  // 64-bit unit base plus a 32-bit lane offset.  Rows past Tk read row Tk-1
  // instead; their 1/|k| is 0 (as for masked keys), so they never pass the
  // threshold and their P is exactly 0.  Only D = 16 < DP has chunks past D
  // (they re-read chunk 0; vzero clears them).
  auto load_rows = [&](const T* base, int64_t st, int u, frag (&f)[NKS]) {
    const int r = u * kUnit + m < a.Tk ? m : a.Tk - 1 - u * kUnit;
    const uint32_t off = (uint32_t)(((int64_t)r * st + PER * half) * (int64_t)sizeof(T));
    const char* p = (const char*)(base + (int64_t)u * kUnit * st) + off;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int c = DP == 32 && KS * ks >= a.D ? 0 : KS * ks;
      f[ks] = M::load((const T*)(p + c * (int)sizeof(T)));
    }
  };
  auto load_k = [&](int u, frag (&f)[NKS]) { load_rows(kg, a.ks.st, u, f); };
  auto load_v = [&](int u, frag (&f)[NKS]) { load_rows(vg, a.vs.st, u, f); };
  // 1/|k| is 0 for keys past Tk and for masked keys
  auto key_ok = [&](int u) {
    const int j = u * kUnit + m;
    return j < a.Tk && !(a.kpm != nullptr && a.kpm[(int64_t)b * a.Tk + j] != 0);
  };
  auto vzero = [&](frag (&f)[NKS]) {
    if constexpr (DP == 32) {
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
        if (KS * ks >= a.D) f[ks] = M::zero();
    }
  };
  // S > 1: this wave's first unit is the row's live unit number `wave` (a
  // wave left without one loads the row's first unit's rows and skips the
  // loop)
  const int first = cur;
  for (int w = 0; w < wave && cur >= 0; ++w) cur = walk.next();
  // own queries as raw B operands (lane -> query), kept in LDS and read back
  // per unit (the registers go to the unit rows), and 1/|q_i|; their loads
  // go first, the first unit's behind them
  float iq;
  frag kc[NKS], vc[NKS];
  bool kok;
  {
    R qr;
    qr.load((const T*)a.q + b * a.qs.sb + (int64_t)(valid ? i : 0) * a.qs.st + h * a.qs.sh, valid, a.D, half);
    const int u0 = cur >= 0 ? cur : first;
    load_k(u0, kc);
    load_v(u0, vc);
    kok = key_ok(u0);
    iq = qr.inv_norm(a.eps);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qsh[ks][lane] = qr.f[ks];
  }
  const float thq = hp.thr / iq;  // s > thr  <=>  (k . q)/|k| > thr |q|
  f32x16 o[NDH];
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[dblk][r] = 0.0f;

  while (cur >= 0) {
    const int k0 = cur * kUnit;
    // S^T = K Q^T on the raw rows (exact products of the inputs, fp32
    // accumulation), scaled by 1/|k_j| in fp32 below: register r -> key
    // k0 + rowof(r, half), lane -> query i
    vzero(kc);
    f32x16 s;
    float s2k = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.0f;
    {
      frag qf[NKS];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) qf[ks] = qsh[ks][lane];
      if constexpr (sizeof(T) == 2) {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          s = M::mma_ng(kc[ks], qf[ks], s);
          s2k = frag_dot(kc[ks], kc[ks], s2k);
        }
        guard_frags(kc);
        guard_frags(qf);
      } else {
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          s = M::mma(kc[ks], qf[ks], s);
          s2k = frag_dot(kc[ks], kc[ks], s2k);
        }
      }
    }
    // each operand's registers take the next unit's rows as soon as they are
    // free, so those loads run behind the rest of this unit's work (past the
    // last unit, the current one again, a cache hit: every iteration then
    // waits for the same count)
    int nxt = -1;  // this wave's next unit: S positions on in the row's walk
    for (int w = 0; w < S; ++w) {
      nxt = walk.next();
      if (nxt < 0) break;
    }
    const int nl = nxt >= 0 ? nxt : cur;
    const bool kok_c = kok;
    load_k(nl, kc);
    kok = key_ok(nl);
    // 1/|k_j| and 1/|v_j| of the lane's key row, to LDS (read back in
    // register order), then V^T by identity MFMA
    vzero(vc);
    float ivl;  // this lane's 1/|v| (its row m)
    {
      float s2v = 0.0f;
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) s2v = frag_dot(vc[ks], vc[ks], s2v);
      s2v = half_sum(s2v);
      s2k = half_sum(s2k);
      const float iv = inv_len(s2v, a.eps);
      ivl = iv;
      const float ik = kok_c ? inv_len(s2k, a.eps) : 0.0f;
      wave_lds_sync();
      if (half == 0) {
        sv[m] = iv;
        sk[m] = ik;
      }
      unit_mask_table<false>(mt, nullptr, qu * kUnit - k0 - 31, hp, lane);
      wave_lds_sync();
    }
    {
      float ksc[16];
      read_row_scales(sk, half, ksc);
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] *= ksc[r];
    }
    frag ta[NDH * NC];
    frag id[NC];  // formed per unit: fewer registers held across the loop
#pragma unroll
    for (int c = 0; c < NC; ++c) id[c] = ident_frag<T>(c, lane);
    // fp16: each lane's V row takes its 1/|v| before the transposes (in fp32,
    // rounded once to fp16: the value the transposed row would get), which
    // holds one scale per lane instead of sixteen.  The scheduling barriers
    // keep the conversions in place: hoisted next to the S products they
    // held 32 more values at once and spilled 9 VGPRs (live 42 -> 32 us at
    // configs[1] in fp16 without the spill)
    if constexpr (kScaleRowsNotWeights<T>) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks)
#pragma unroll
        for (int e = 0; e < PER; ++e) vc[ks][e] = (T)((float)vc[ks][e] * ivl);
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int dblk = 0; dblk < NDH; ++dblk) {
      f32x16 tr;
#pragma unroll
      for (int r = 0; r < 16; ++r) tr[r] = 0.0f;
#pragma unroll
      for (int c = 0; c < NC; ++c) tr = M::mma_ng(vc[dblk * NC + c], id[c], tr);
#pragma unroll
      for (int c = 0; c < NC; ++c) ta[dblk * NC + c] = M::pack(tr, c * PER);
    }
    guard_frags(vc);
    guard_frags(id);
    load_v(nl, vc);
    // P^T[j][i] = alpha_ij m_ij / |v_j|: every lane forms its pair's weight
    // branch-free (alpha = 0 below the threshold, the mask, 0 outside the
    // window, from the unit's table: register r holds distance i - k0 - 8half
    // - 16(r/8) - r%8, entry l32 - 8half + 31 - 16(r/8) - r%8), for every
    // register; with dropout, only for the registers where some lane may pass
    // a conservative gate on the products (s > thr), so the pair hash runs
    // there only
    {
      const float* mrow = mt + (l32 - 8 * half + 8);  // entry 23 - (16(r/8) + r%8): a constant offset
      auto body = [&](int r) {
        const int off = 16 * (r >> 3) + (r & 7);
        const float av = fmaxf(trim(s[r] * iq, hp.r), 0.0f);
        float p = av * av * mrow[23 - off];
        if (a.drop.on) p *= dropout_factor(a.drop, bh, i, k0 + 8 * half + off);
        s[r] = p;
      };
      if (a.drop.on) {
        const uint32_t pm0 = pass_mask(s, thq);
        for_each_set(pm0, body);
#pragma unroll
        for (int r = 0; r < 16; ++r)
          if (((pm0 >> r) & 1u) == 0u) s[r] = 0.0f;
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) body(r);
      }
      if constexpr (!kScaleRowsNotWeights<T>) {
        float vsc[16];
        read_row_scales(sv, half, vsc);
#pragma unroll
        for (int r = 0; r < 16; ++r) s[r] *= vsc[r];
      }
    }
    // H^T[d][i] += sum_j V^T[d][j] P^T[j][i]
    frag pb[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) pb[c] = M::pack(s, c * PER);
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
      for (int dblk = 0; dblk < NDH; ++dblk) o[dblk] = M::mma_ng(ta[dblk * NC + c], pb[c], o[dblk]);
    guard_frags(ta);
    guard_frags(pb);
    if (nxt < 0) break;
    cur = nxt;
  }

  if constexpr (S > 1) {
    // waves 1..S-1 hand their H^T to wave 0 (each in its own wbuf row),
    // which adds them in wave order
    auto part = [&](int w) { return reinterpret_cast<float(*)[kWave]>(wbuf[w]); };
    if (wave > 0)
#pragma unroll
      for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
        for (int r = 0; r < 16; ++r) part(wave)[dblk * 16 + r][lane] = o[dblk][r];
    __syncthreads();
    if (wave > 0) return;
    for (int w = 1; w < S; ++w)
#pragma unroll
      for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[dblk][r] += part(w)[dblk * 16 + r][lane];
  }
  // TanhNorm per query row (lane -> query, registers -> d), y in (B,T,H,D)
  float ss = 0.0f;
#pragma unroll
  for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
    for (int r = 0; r < 16; ++r) ss += o[dblk][r] * o[dblk][r];
  ss = half_sum(ss);
  const float n = sqrtf(ss);
  const float nc = fmaxf(n, a.eps);
  const float f = tanhf(nc) / nc;
  if (valid) {
    if (half == 0) a.hnorm[(int64_t)bh * a.Tq + i] = n;
    store_creg_row<T, NDH>(yrow(), a.D, half, [&](int dblk, int r) { return f * o[dblk][r]; });
  }
}

static int64_t khat_bytes(const Geometry& g) {
  return round_up((int64_t)g.B * g.H * g.Tk_pad * g.DP * (int64_t)sizeof(ScreenOp), 256);  // fp16 rows
}
// Rows (32-query units) below which the live pass splits each row's units
// over several waves: about two waves per SIMD of the chip.
constexpr int64_t kLiveSplitWaves = 2048;

// Workspace: [K^][screen plan table]
size_t fwd_ws_bytes(const Geometry& g) { return khat_bytes(g) + screen_plan_bytes(g); }

template <typename T, int DP>
static hipError_t launch_fwd_t(const FwdCall& c) {
  const Geometry& g = c.g;
  ScreenPlan plan;
  screen_plan_dims(g, plan.seg, plan.kmax, plan.per_xcd);
  plan.table = (ScreenItem*)((char*)c.khat + khat_bytes(g));
  FwdKArgs fa;
  fa.q = c.q; fa.qs = c.qs; fa.k = c.k; fa.ks = c.ks; fa.v = c.v; fa.vs = c.vs; fa.kpm = c.kpm;
  fa.khat = c.khat;
  fa.r = c.r; fa.w = c.w; fa.y = c.y; fa.hnorm = c.hnorm; fa.bits = c.bits;
  fa.H = g.H; fa.Tq = g.Tq; fa.Tk = g.Tk; fa.D = g.D; fa.nqt = g.nqt; fa.nku_words = g.nku_words;
  fa.causal = g.causal; fa.Tk_pad = g.Tk_pad; fa.eps = c.eps; fa.drop = c.drop;
  fa.plan = plan;
  if (g.Tk_pad > 0) {  // no keys: no bitmap words and no screen work
    PrepKArgs pa;
    pa.k = c.k; pa.ks = c.ks; pa.kpm = c.kpm; pa.khat = c.khat;
    pa.bits = c.bits; pa.bits_per_bh = (int64_t)2 * g.nqt * g.nku_words;
    pa.B = g.B; pa.H = g.H; pa.Tq = g.Tq; pa.Tk = g.Tk; pa.D = g.D; pa.nqt = g.nqt; pa.causal = g.causal;
    pa.Tk_pad = g.Tk_pad; pa.eps = c.eps;
    pa.r = c.r; pa.w = c.w; pa.plan = plan;
    constexpr int RPB = 256 / (DP * (int)sizeof(T) / 16) * kPrepRows;
    const int64_t nx = (g.Tk_pad + RPB - 1) / RPB;
    // row 0: the screen planner (8 blocks); rows 1..B*H: K^ of head row-1
    timer_begin(1, c.stream);
    hipLaunchKernelGGL((prep_k_kernel<T, DP>), dim3((unsigned)(nx > 8 ? nx : 8), (unsigned)(g.B * g.H + 1)),
                       dim3(256), 0, c.stream, pa);
    timer_end(1, c.stream);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    timer_begin(2, c.stream);
    // at most kScreenBlocksPerLane blocks per lane; blocks beyond the first
    // walk their lane's items with that stride
    const int per_lane = plan.kmax < kScreenBlocksPerLane ? plan.kmax : kScreenBlocksPerLane;
    hipLaunchKernelGGL((fwd_screen_kernel<T, DP>), dim3((unsigned)(32 * per_lane)), dim3(256), 0, c.stream, fa);
    timer_end(2, c.stream);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  // A launch with few rows (under about two waves per SIMD) splits each
  // row's live units over S waves (DP <= 64: the S waves' LDS fits)
  const int64_t rows = (int64_t)2 * g.nqt * g.B * g.H;
  const int S = DP > 64 ? 1 : (rows * 4 <= kLiveSplitWaves ? 4 : (rows * 2 <= kLiveSplitWaves ? 2 : 1));
  const dim3 grid((unsigned)(2 * g.nqt), (unsigned)(g.B * g.H));
  timer_begin(3, c.stream);
  if constexpr (DP <= 64) {
    if (S == 4)
      hipLaunchKernelGGL((fwd_live_kernel<T, DP, 4>), grid, dim3(256), 0, c.stream, fa);
    else if (S == 2)
      hipLaunchKernelGGL((fwd_live_kernel<T, DP, 2>), grid, dim3(128), 0, c.stream, fa);
    else
      hipLaunchKernelGGL((fwd_live_kernel<T, DP, 1>), grid, dim3(64), 0, c.stream, fa);
  } else {
    hipLaunchKernelGGL((fwd_live_kernel<T, DP, 1>), grid, dim3(64), 0, c.stream, fa);
  }
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
  if (c.g.dtype == 2) {
    if (DP == 32) return launch_fwd_t<f16, 32>(c);
    if (DP == 64) return launch_fwd_t<f16, 64>(c);
    return launch_fwd_t<f16, 128>(c);
  }
  if (DP == 32) return launch_fwd_t<float, 32>(c);
  if (DP == 64) return launch_fwd_t<float, 64>(c);
  return launch_fwd_t<float, 128>(c);
}

}  // namespace msa
