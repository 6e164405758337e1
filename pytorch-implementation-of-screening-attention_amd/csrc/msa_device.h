// Device-side building blocks shared by the fused Screening Attention kernels
// for gfx950 (CDNA4): MFMA operand fragments, the tile/lane index maps and the
// per-pair screening math.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace msa {

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef _Float16 f16;
typedef __attribute__((__vector_size__(8 * sizeof(_Float16)))) _Float16 f16x8;
typedef __attribute__((__vector_size__(4 * sizeof(_Float16)))) _Float16 f16x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int kWave = 64;
constexpr int kTile = 64;  // rows of a query tile and of a key tile
constexpr int kUnit = 32;  // rows of a query unit and of a key unit (live-unit bitmap)

// ---------------------------------------------------------------------------
// MFMA fragments.  Both element types use the 32x32 output block; a wave-64
// instruction contracts KS values of k.  Lane l supplies row (A) / column (B)
// l%32 and the PER contraction values of "slot group" l/32.  The mapping of
// (slot group, slot) to the hardware's k index is the same for A and B, so any
// contraction whose A and B slots are filled for the same logical k is exact
// whatever that mapping is.
//   C/D layout: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, col l%32.
//
// Source-operand guard.  This toolchain (ROCm 7.2 clang, gfx950) schedules a
// VALU or LDS write into the A/B source VGPRs of an MFMA as if the MFMA had
// read them at issue.  An MFMA whose accumulator comes from the MFMA before it
// waits for that result and reads A/B later, so it can read the new values.
// The unguarded D=32 bf16 dq kernel shows a v_mov_b64 refilling SrcA one
// instruction after such a chained v_mfma_f32_32x32x16_bf16.  Measured on an
// MI355X: 2 and 4 wait states of padding still corrupted the product, 8 did
// not.  After every MFMA group an s_nop block that takes A and B as read-write
// operands keeps those registers from being reused until 16 wait states have
// passed.  The MFMA pipe is busy far longer than that per instruction, so
// back-to-back MFMA throughput is unchanged.
// ---------------------------------------------------------------------------
template <typename T> struct Mma;

template <typename F>
__device__ inline void guard_mfma_sources(F& a, F& b) {
  asm volatile("s_nop 7\n\ts_nop 7" : "+v"(a), "+v"(b));
}
// Group form: after a run of unguarded MFMAs (mma_ng), one s_nop block that
// takes every A/B fragment of the run as a read-write operand.  The asm must
// follow each MFMA that reads those registers (write-after-read order), so
// none of them can be reused earlier than 16 wait states after the last one.
#define MSA_NOP16 "s_nop 7\n\ts_nop 7"
template <typename F>
__device__ inline void guard_frags(F (&f)[2]) {
  asm volatile(MSA_NOP16 : "+v"(f[0]), "+v"(f[1]));
}
template <typename F>
__device__ inline void guard_frags(F (&f)[4]) {
  asm volatile(MSA_NOP16 : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]));
}
template <typename F>
__device__ inline void guard_frags(F (&f)[8]) {
  asm volatile(MSA_NOP16 : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]),
               "+v"(f[7]));
}
template <typename F, int N>
__device__ inline void guard_frags(F (&f)[N]) {
  static_assert(N % 16 == 0, "guard_frags: unsupported fragment count");
#pragma unroll
  for (int c = 0; c < N; c += 16)
    asm volatile(MSA_NOP16 : "+v"(f[c]), "+v"(f[c + 1]), "+v"(f[c + 2]), "+v"(f[c + 3]), "+v"(f[c + 4]),
                 "+v"(f[c + 5]), "+v"(f[c + 6]), "+v"(f[c + 7]), "+v"(f[c + 8]), "+v"(f[c + 9]), "+v"(f[c + 10]),
                 "+v"(f[c + 11]), "+v"(f[c + 12]), "+v"(f[c + 13]), "+v"(f[c + 14]), "+v"(f[c + 15]));
}
template <typename F>
__device__ inline void guard_frags(F (&f)[16]) {
  asm volatile(MSA_NOP16 : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]),
               "+v"(f[7]), "+v"(f[8]), "+v"(f[9]), "+v"(f[10]), "+v"(f[11]), "+v"(f[12]), "+v"(f[13]),
               "+v"(f[14]), "+v"(f[15]));
}

template <> struct Mma<bf16> {
  static constexpr int KS = 16;
  static constexpr int PER = 8;
  typedef bf16x8 frag;
  __device__ static inline f32x16 mma(frag a, frag b, f32x16 c) {
    const f32x16 d = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    guard_mfma_sources(a, b);
    return d;
  }
  // Unguarded: the caller guards every A/B fragment with guard_frags.
  __device__ static inline f32x16 mma_ng(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  __device__ static inline frag load(const bf16* p) { return *reinterpret_cast<const frag*>(p); }
  __device__ static inline frag zero() { frag z; for (int e = 0; e < 8; ++e) z[e] = (bf16)0.0f; return z; }
  __device__ static inline float get(const frag& f, int e) { return (float)f[e]; }
  // PER fp32 values starting at register r0 of a C block -> operand fragment.
  __device__ static inline frag pack(const f32x16& c, int r0) {
    frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (bf16)c[r0 + e];
    return f;
  }
};

// fp16: the same 32x32x16 operand layout and pass count as bf16
// (v_mfma_f32_32x32x16_f16), so every layout map and the source-operand guard
// apply unchanged.
template <> struct Mma<f16> {
  static constexpr int KS = 16;
  static constexpr int PER = 8;
  typedef f16x8 frag;
  __device__ static inline f32x16 mma(frag a, frag b, f32x16 c) {
    const f32x16 d = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    guard_mfma_sources(a, b);
    return d;
  }
  __device__ static inline f32x16 mma_ng(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  __device__ static inline frag load(const f16* p) { return *reinterpret_cast<const frag*>(p); }
  __device__ static inline frag zero() { frag z; for (int e = 0; e < 8; ++e) z[e] = (f16)0.0f; return z; }
  __device__ static inline float get(const frag& f, int e) { return (float)f[e]; }
  __device__ static inline frag pack(const f32x16& c, int r0) {
    frag f;
#pragma unroll
    for (int e = 0; e < 8; ++e) f[e] = (f16)c[r0 + e];
    return f;
  }
};

// Where a per-row factor 1/|x| enters a product whose other operand is
// packed to the input type.  bf16 (8 exponent bits) folds it into the pair
// weights (alpha*m/|v|, ds/|k|, ds/|q|) and keeps the raw rows exact.  fp16
// has 5 exponent bits: a weight times 1/|x| overflows to inf for rows shorter
// than about 1.5e-5 (a zero row gives 1/eps = 1e8, then inf * 0 = NaN), so
// the fp16 kernels scale the transposed rows instead (x^ = x/|x|, at most 1
// in magnitude) and the weights stay at most 2r|dP|.
template <typename T>
constexpr bool kScaleRowsNotWeights = sizeof(T) == 2 && !__is_same(T, bf16);

template <> struct Mma<float> {
  static constexpr int KS = 2;
  static constexpr int PER = 1;
  typedef float frag;
  __device__ static inline f32x16 mma(frag a, frag b, f32x16 c) {
    const f32x16 d = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
    guard_mfma_sources(a, b);
    return d;
  }
  __device__ static inline f32x16 mma_ng(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
  __device__ static inline frag load(const float* p) { return *p; }
  __device__ static inline frag zero() { return 0.0f; }
  __device__ static inline float get(const frag& f, int) { return f; }
  __device__ static inline frag pack(const f32x16& c, int r0) { return c[r0]; }
};

// Row permutation applied when a lane loads row (l%32) of an A operand whose
// product lands in a C block that is later consumed as the B operand of a
// second product contracting over the same rows.  With it, register r of lane
// l holds source row  rowof(r, l/32) = 16*(r/8) + 8*(l/32) + r%8, so that the
// PER consecutive registers a slot group feeds into one instruction cover
// consecutive source rows (16-byte contiguous loads of the transposed operand).
__device__ inline int perm_row(int m) {
  const int g = m >> 3, hh = (m >> 2) & 1, t = m & 3;
  return 16 * (g >> 1) + 8 * hh + 4 * (g & 1) + t;
}
__device__ inline int rowof(int r, int half) { return 16 * (r >> 3) + 8 * half + (r & 7); }

// Transpose by MFMA.  For 32 rows X held as A fragments x[ks] (lane l%32 ->
// row perm_row(l%32), slots -> columns d = KS*ks + PER*(l/32) + e), the product
// X P with a permutation matrix gives, per 32-column block dblk, a C block with
// lane -> column d = 32*dblk + tcol(l%32) and register r -> X row
// rowof(r, l/32).  Packed PER registers at a time, that is the A operand of a
// second product that contracts over X's rows with a C block over the same
// rows (register index = contraction index on both sides).  Products with 1
// and sums with 0 are exact, so the values come through unchanged.
// The column order tcol makes the second product's C block (rows = X's
// columns) put, in each lane, the columns that lane holds of an operand row
// fragment: register r of block dblk <-> fragment (ks, e) = creg_frag(dblk, r)
// (see below), so a row-wise epilogue can combine the accumulator with the
// operand fragments it already has, and store 16 contiguous bytes per group.
template <typename T>
__device__ inline int tcol(int m) {
  if constexpr (sizeof(T) == 2) return perm_row(m);                 // 16*(m/16) + 8*((m>>2)&1) + ...
  else return 8 * (m >> 3) + 2 * (m & 3) + ((m >> 2) & 1);
}
// Fragment slot (ks, e) that holds, in the same lane, the column that register
// r of C block dblk covers when the block's rows are tcol-ordered columns.
template <typename T>
__device__ constexpr int creg_ks(int dblk, int r) {
  if constexpr (sizeof(T) == 2) return 2 * dblk + (r >> 3);   // column 32*dblk + 16*(r/8) + 8*half + r%8
  else return 16 * dblk + 4 * (r >> 2) + (r & 3);             // column 32*dblk + 8*(r/4) + 2*(r%4) + half
}
template <typename T>
__device__ constexpr int creg_e(int r) {
  if constexpr (sizeof(T) == 2) return r & 7;
  else return 0;
}
// Slice c of the permutation (k-step c of a 32-column block; it does not
// depend on the block): slot e of lane l is 1 iff KS*c + PER*(l/32) + e ==
// tcol(l%32).
template <typename T>
__device__ inline typename Mma<T>::frag ident_frag(int c, int lane) {
  using M = Mma<T>;
  const int l32 = lane & 31, half = lane >> 5;
  const int want = tcol<T>(l32);
  f32x16 t;
#pragma unroll
  for (int e = 0; e < 16; ++e) t[e] = (e < M::PER && M::KS * c + M::PER * half + e == want) ? 1.0f : 0.0f;
  return M::pack(t, 0);
}
// out[dblk] = (X I)[:, 32*dblk .. 32*dblk+31] with unguarded MFMAs: the
// caller guards x and id (guard_frags) before they can be overwritten.
template <typename T, int DP>
__device__ inline void transpose_rows(const typename Mma<T>::frag (&x)[DP / Mma<T>::KS],
                                      const typename Mma<T>::frag (&id)[32 / Mma<T>::KS], f32x16 (&out)[DP / 32]) {
  using M = Mma<T>;
  constexpr int NC = 32 / M::KS;
#pragma unroll
  for (int dblk = 0; dblk < DP / 32; ++dblk) {
#pragma unroll
    for (int r = 0; r < 16; ++r) out[dblk][r] = 0.0f;
#pragma unroll
    for (int c = 0; c < NC; ++c) out[dblk] = M::mma_ng(x[dblk * NC + c], id[c], out[dblk]);
  }
}

// ---------------------------------------------------------------------------
// Screening math for one (query i, key j) pair.
// ---------------------------------------------------------------------------
struct HeadParams {
  float r;     // acceptance sharpness r_h > 1 (may round to 1.0f)
  float w;     // window w_h > 1
  float iw;    // 1/w
  int wc;      // ceil(w) (capped at 2^30): for integer distance d, d < w  <=>  d < wc
  float thr;   // 1 - 1/r - 1e-5: s > thr for every pair with 1 - r(1-s) > 0 when
               // s is formed from exact products with fp32 accumulation and
               // fp32 1/|x| (error below (D+3) 2^-24 <= 8e-6 for D <= 128): a
               // conservative gate; the exact test follows wherever it passes
  int wsh;     // window as one unsigned compare: dd in window  <=>
  unsigned wlim;  // (unsigned)(dd + wsh) < wlim
};

// In-window distances dd = i - j (attention.py:111-118 causal, :176-181
// non-causal): causal 0 <= dd < wc, i.e. shift 0 and limit wc; non-causal
// -wc < dd < wc, i.e. shift wc-1 and limit 2wc-1.  Positions stay below 2^22
// and wc <= 2^30, so dd + wsh never overflows.  A window that is not a number
// (or not positive) is empty: wc = 0, limit 0, so no pair of the head is live
// and its outputs are zero (the reference's dense path gives NaN there).
__device__ inline HeadParams head_params_rw(float r, float w, bool causal) {
  HeadParams p;
  p.r = r;
  p.w = w;
  p.iw = 1.0f / p.w;
  const float c = ceilf(p.w);
  p.wc = !(c > 0.0f) ? 0 : (c > 1073741824.0f ? 1073741824 : (int)c);
  p.thr = 1.0f - 1.0f / p.r - 1e-5f;
  p.wsh = causal ? 0 : p.wc - 1;
  p.wlim = p.wc == 0 ? 0u : (causal ? (unsigned)p.wc : (unsigned)(2 * p.wc - 1));
  return p;
}
__device__ inline HeadParams head_params(const float* r, const float* w, int h, bool causal) {
  return head_params_rw(r[h], w[h], causal);
}

// Wave-uniform mask of the registers r of a C block for which some lane has
// c[r] > th.
__device__ inline uint32_t pass_mask(const f32x16& c, float th) {
  uint32_t m = 0u;
#pragma unroll
  for (int r = 0; r < 16; ++r) m |= __ballot(c[r] > th) != 0ull ? (1u << r) : 0u;
  return m;
}
// Calls fn(r) for each register r whose bit is set in the uniform mask pm:
// a compile-time r and one uniform branch per register, so c[r] inside fn is
// a plain register.  (A loop over the set bits only would make r uniform but
// not constant, and c[r] a register-indexed move, s_set_gpr_idx.  In the fp32
// kernels that form failed the dK parity test: their S/dP accumulation is a
// dependent chain of 16-pass v_mfma_f32_32x32x2_f32 reading B from registers
// that the indexed loop's copies of s and dP reuse 27-32 wait states after
// the chain's last issue, past the 16-wait-state guard.  With the branch-free
// pair math the unrolled form is also the faster one for 2-byte types.)
template <typename Fn>
__device__ inline void for_each_set(uint32_t pm, Fn&& fn) {
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    if ((pm >> r) & 1u) fn(r);
    __builtin_amdgcn_sched_barrier(0);  // one register at a time: few live temporaries
  }
}

// cos(pi x) and sin(pi x) for |x| <= 1 (x clamped there), branch-free and
// without a library call: with y = |x| and t = min(y, 1 - y) in [0, 1/2],
// cos(pi y) = +-cos(pi t) (minus for y > 1/2) and sin(pi y) = sin(pi t); the
// Taylor series of cos(pi t) and sin(pi t) to t^12 and t^13 are within
// 6.4e-9 and 6.7e-10 of them on [0, 1/2] (next terms pi^14 t^14/14! and
// pi^15 t^15/15!), below fp32 rounding.  Coefficients (-1)^k pi^2k/(2k)!
// and (-1)^k pi^(2k+1)/(2k+1)!, evaluated by Horner's rule in t^2.
__device__ inline float cospi_poly(float u) {  // u = t^2
  float c = 0.001929574309403922f;
  c = fmaf(c, u, -0.02580689139001405f);
  c = fmaf(c, u, 0.23533063035889312f);
  c = fmaf(c, u, -1.3352627688545893f);
  c = fmaf(c, u, 4.058712126416768f);
  c = fmaf(c, u, -4.934802200544679f);
  return fmaf(c, u, 1.0f);
}
__device__ inline float sinpi_poly(float t, float u) {  // u = t^2
  float c = 0.00046630280576761234f;
  c = fmaf(c, u, -0.007370430945714348f);
  c = fmaf(c, u, 0.08214588661112819f);
  c = fmaf(c, u, -0.5992645293207919f);
  c = fmaf(c, u, 2.550164039877345f);
  c = fmaf(c, u, -5.167712780049969f);
  c = fmaf(c, u, 3.141592653589793f);
  return c * t;
}
// Soft mask m = (cos(pi dd/w) + 1)/2 (attention.py:114) for an in-window
// distance (|dd| < w, so y = |dd|/w < 1); out of the window the value is
// finite and the caller masks it.  For y <= 1/2, m = 1/2 + cos(pi y)/2 (both
// terms at least 0: no cancellation).  Past 1/2, m falls to 0 at the window's
// edge and that form would cancel, and y = |dd| (1/w) would carry the
// rounding of 1/w into 1 - y; there m = sin^2(pi t/2) with t = 1 - y formed
// as (w - |dd|) / w, whose numerator is exact in fp32 (w/2 <= |dd| <= w:
// Sterbenz), so m keeps a few ulps of relative accuracy down to the last
// in-window distance.  t also gives sin(pi y) = sin(pi t) for dm/dw.
struct MaskArg {
  float y, t;  // |dd|/w, and min(y, 1 - y) with 1 - y = (w - |dd|)/w
  bool far;    // y > 1/2
};
__device__ inline MaskArg mask_arg(int dd, float w, float iw) {
  MaskArg a;
  const float ad = fabsf((float)dd);
  a.y = fminf(ad * iw, 1.0f);
  a.far = a.y > 0.5f;
  a.t = a.far ? fmaxf((w - ad) * iw, 0.0f) : a.y;
  return a;
}
__device__ inline float mask_of(const MaskArg& a) {
  const float z = 0.5f * a.t;  // sin(pi t/2) for the far half
  const float sz = sinpi_poly(z, z * z);
  const float c = cospi_poly(a.t * a.t);
  return a.far ? sz * sz : 0.5f + 0.5f * c;
}
__device__ inline float mask_fast(int dd, float w, float iw) { return mask_of(mask_arg(dd, w, iw)); }
// The same mask and dm/dw = (pi/2) dd sin(pi dd/w) / w^2 (the w-derivative
// of (cos(pi (j-i)/w) + 1)/2, attention.py:114).
__device__ inline void mask_fast_dw(int dd, float w, float iw, float& m, float& dm) {
  const MaskArg a = mask_arg(dd, w, iw);
  m = mask_of(a);
  const float sn = copysignf(sinpi_poly(a.t, a.t * a.t), (float)dd);
  dm = (0.5f * 3.14159265358979f) * (float)dd * sn * iw * iw;
}

// Branch-free in-window test on the integer distance dd = i - j.
__device__ inline bool in_window(int dd, const HeadParams& hp) { return (unsigned)(dd + hp.wsh) < hp.wlim; }

// Soft-mask table of one 32x32 unit (queries q0.., keys k0..): its pairs'
// distances dd = i - j span dmin .. dmin + 62 with dmin = q0 - k0 - 31, so
// lane l (l < 63) evaluates entry l = the mask of distance dmin + l, 0
// outside the window (and, with `dw`, dm/dw in a second table).  A pair
// then reads its mask instead of evaluating it.  Written by one wave for its
// own use: the caller syncs (wave_lds_sync) before reading.
template <bool kDw>
__device__ inline void unit_mask_table(float* mt, float* mdt, int dmin, const HeadParams& hp, int lane) {
  const int dd = dmin + lane;
  const bool in = lane < 63 && in_window(dd, hp);
  if constexpr (kDw) {
    float m, dm;
    mask_fast_dw(dd, hp.w, hp.iw, m, dm);
    mt[lane] = in ? m : 0.0f;
    mdt[lane] = in ? dm : 0.0f;
  } else {
    mt[lane] = in ? mask_fast(dd, hp.w, hp.iw) : 0.0f;
  }
}

// Trim-and-square pre-square value a = 1 - r (1 - s)  (attention.py:90).
__device__ inline float trim(float s, float r) { return 1.0f - r * (1.0f - s); }

// max(x[l], x[l ^ 32]) in every lane (as half_sum, with max).
__device__ inline float half_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return fmaxf(__int_as_float(r[0]), __int_as_float(r[1]));
}

// x[l] + x[l ^ 32] in every lane, with one v_permlane32_swap (no LDS): the
// swap leaves lanes 0..31 of the first result and 32..63 of the second with
// the lane's own value and the others with the partner's, so the two results
// add to the pair sum in every lane.
__device__ inline float half_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(x), __float_as_int(x), false, false);
  return __int_as_float(r[0]) + __int_as_float(r[1]);
}

// Sum over aligned groups of G lanes (G a power of two <= 64), every lane of
// a group getting the group's total: DPP lane swaps within rows of 16 (xor 1,
// xor 2, then the 8- and 16-lane mirrors, which pair each half with the other
// once both halves hold their own sums), lane shuffles beyond.
template <int G>
__device__ inline float group_sum(float x) {
  auto dpp = [](float v, auto ctrl) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), decltype(ctrl)::value, 0xf, 0xf, false));
  };
  if constexpr (G >= 2) x += dpp(x, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  if constexpr (G >= 4) x += dpp(x, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  if constexpr (G >= 8) x += dpp(x, std::integral_constant<int, 0x141>{});  // row_half_mirror
  if constexpr (G >= 16) x += dpp(x, std::integral_constant<int, 0x140>{}); // row_mirror
#pragma unroll
  for (int o = 16; o < G; o <<= 1) x += __shfl_xor(x, o);
  return x;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Loads PER elements of type T from p (16-byte aligned for bf16), or zeros.
template <typename T>
__device__ inline typename Mma<T>::frag load_or_zero(const T* p, bool ok) {
  return ok ? Mma<T>::load(p) : Mma<T>::zero();
}

__device__ inline float to_f(float x) { return x; }
__device__ inline float to_f(bf16 x) { return (float)x; }
__device__ inline float to_f(f16 x) { return (float)x; }
template <typename T> __device__ inline T from_f(float x);
template <> __device__ inline float from_f<float>(float x) { return x; }
template <> __device__ inline bf16 from_f<bf16>(float x) { return (bf16)x; }
template <> __device__ inline f16 from_f<f16>(float x) { return (f16)x; }

// Stores 4 consecutive values.
__device__ inline void store4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<f32x4*>(p) = f32x4{a, b, c, d};
}
__device__ inline void store4(bf16* p, float a, float b, float c, float d) {
  *reinterpret_cast<bf16x4*>(p) = bf16x4{(bf16)a, (bf16)b, (bf16)c, (bf16)d};
}
__device__ inline void store4(f16* p, float a, float b, float c, float d) {
  *reinterpret_cast<f16x4*>(p) = f16x4{(f16)a, (f16)b, (f16)c, (f16)d};
}
// Stores 8 consecutive values (16 bytes for bf16 and fp16).
__device__ inline void store8(bf16* p, const float (&v)[8]) {
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (bf16)v[e];
  *reinterpret_cast<bf16x8*>(p) = o;
}
__device__ inline void store8(f16* p, const float (&v)[8]) {
  f16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = (f16)v[e];
  *reinterpret_cast<f16x8*>(p) = o;
}
__device__ inline void store8(float* p, const float (&v)[8]) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
  *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
}

// Writes one row held in C-layout registers whose rows are tcol-ordered
// columns (a product with a transpose_rows operand): value(dblk, r) -> column
// 32*dblk + (column of register r).  fn(dblk, r) gives the value.
template <typename T, int NDH, typename Fn>
__device__ inline void store_creg_row(T* row, int D, int half, Fn fn) {
  if constexpr (sizeof(T) == 2) {
#pragma unroll
    for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
      for (int g = 0; g < 2; ++g) {
        const int d0 = 32 * dblk + 16 * g + 8 * half;
        if (d0 < D) {
          float v[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) v[e] = fn(dblk, 8 * g + e);
          store8(row + d0, v);
        }
      }
  } else {
#pragma unroll
    for (int dblk = 0; dblk < NDH; ++dblk)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int d = 32 * dblk + 8 * (r >> 2) + 2 * (r & 3) + half;
        if (d < D) row[d] = fn(dblk, r);
      }
  }
}

// Loads one 16-byte chunk (8 bf16/fp16 or 4 fp32 values) as fp32.
__device__ inline void load_chunk(const bf16* p, float (&x)[8]) {
  const bf16x8 v = *reinterpret_cast<const bf16x8*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (float)v[e];
}
__device__ inline void load_chunk(const f16* p, float (&x)[8]) {
  const f16x8 v = *reinterpret_cast<const f16x8*>(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) x[e] = (float)v[e];
}
__device__ inline void load_chunk(const float* p, float (&x)[4]) {
  const f32x4 v = *reinterpret_cast<const f32x4*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = v[e];
}

// 1/max(sqrt(ss), eps) from a squared length, by the hardware reciprocal
// square root (v_rsq_f32, ~1 ulp): min(rsq(ss), 1/eps) is the same clamp
// (rsq(0) = +inf).
__device__ inline float inv_len(float ss, float eps) {
  return fminf(__builtin_amdgcn_rsqf(ss), __builtin_amdgcn_rcpf(eps));
}

// Sum of products of two operand fragments in fp32: v_dot2c_f32_bf16 (two
// exact bf16 products per instruction) for bf16, a plain product for fp32.
__device__ inline float frag_dot(const bf16x8& a, const bf16x8& b, float acc) {
  typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const bf16x2_t x = {a[e], a[e + 1]}, y = {b[e], b[e + 1]};
    acc = __builtin_amdgcn_fdot2_f32_bf16(x, y, acc, false);
  }
  return acc;
}
// fp16: v_dot2_f32_f16, two products per instruction accumulated in fp32.
__device__ inline float frag_dot(const f16x8& a, const f16x8& b, float acc) {
  typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    const f16x2_t x = {a[e], a[e + 1]}, y = {b[e], b[e + 1]};
    acc = __builtin_amdgcn_fdot2(x, y, acc, false);
  }
  return acc;
}
__device__ inline float frag_dot(float a, float b, float acc) { return acc + a * b; }

// An operand row kept in its storage type: the lane's NKS fragments (slots
// d = KS*ks + PER*half + e), converted to fp32 only where arithmetic needs it.
template <typename T, int DP>
struct PRow {
  using M = Mma<T>;
  using frag = typename M::frag;
  static constexpr int KS = M::KS, PER = M::PER, NKS = DP / KS;
  frag f[NKS];

  // `p` must be readable even when !ok: the loads are unconditional and
  // masked afterwards.
  __device__ inline void load(const T* p, bool ok, int D, int half) {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      const int d0 = KS * ks + PER * half;
      f[ks] = M::load(p + (d0 < D ? d0 : 0));
    }
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks)
      if (!(ok && KS * ks + PER * half < D)) f[ks] = M::zero();
  }
  __device__ inline float get(int ks, int e) const { return M::get(f[ks], e); }
  __device__ inline float dot(const PRow& o) const {
    float s = 0.0f;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) s = frag_dot(f[ks], o.f[ks], s);
    return half_sum(s);
  }
  __device__ inline float inv_norm(float eps) const { return inv_len(dot(*this), eps); }
  // this <- a*this + b*o, rounded to T
  __device__ inline void axpby(float a, float b, const PRow& o) {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      f32x16 t;
#pragma unroll
      for (int e = 0; e < PER; ++e) t[e] = a * M::get(f[ks], e) + b * M::get(o.f[ks], e);
      f[ks] = M::pack(t, 0);
    }
  }
};

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

// fp16 row scaling of an identity-MFMA transpose: c holds the raw rows
// exactly in fp32 (products with 1, sums with 0), register r row
// 16*(r/8) + 8*half + r%8, and each register takes its row's factor in fp32;
// the operand pack then rounds once to fp16.  The same value as scaling the
// row registers before the transpose, at one multiply per register instead
// of a convert, multiply and convert per element.
__device__ inline void scale_rows_fp32(f32x16& c, const float* sc, int half) {
  float f[16];
  read_row_scales(sc, half, f);
#pragma unroll
  for (int r = 0; r < 16; ++r) c[r] *= f[r];
}

// Waits until at most N of this wave's vector memory operations (loads,
// stores and global->LDS DMA) are outstanding.
template <int N>
__device__ inline void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"i"(N) : "memory"); }

// Waits for this wave's LDS traffic and keeps the compiler from moving
// memory operations across the point (LDS ops of one wave run in order).
__device__ inline void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// XOR swizzle of the 16-byte chunk positions of LDS row R (rows of CPR
// chunks).  A ds_read_b128 whose lanes read rows perm_row(l%32) at one chunk
// position is conflict-free if the rows a bank window serves land in distinct
// 16-byte bank groups, whether the LDS serves 8 lanes (128 bytes) or 16 lanes
// (256 bytes) a cycle: 8 lanes read rows {0..3, 8..11} (+4, +16), 16 lanes
// rows 0..15 (+16).  With bits b0..b3 of R:
//   CPR 4  (2 rows per 128 B): (b1^b2, b3) is one-to-one on the rows sharing
//          b0 in either set of rows, and on those sharing (b0, b1) in 0..15;
//   CPR 8  (1 row per 128 B) : (b1, b3, b0^b2) is one-to-one on {0..3, 8..11}
//          and on {4..7, 12..15}, and on the even and the odd rows of 0..15;
//   CPR>=16: (b1, b3, b0^b2, b0) is also one-to-one on all of 0..15.
template <int CPR>
__device__ inline int lds_swz(int R) {
  const int b0 = R & 1, b1 = (R >> 1) & 1, b2 = (R >> 2) & 1, b3 = (R >> 3) & 1;
  if constexpr (CPR == 4) return (b1 ^ b2) | (b3 << 1);
  else if constexpr (CPR == 8) return b1 | (b3 << 1) | ((b0 ^ b2) << 2);
  else return b1 | (b3 << 1) | ((b0 ^ b2) << 2) | (b0 << 3);
}

// Set bits lo..hi of one bitmap row (position u = bit u%32 of word u/32),
// visited in increasing order.  Lane l holds word w0 + l, so one load round
// trip brings 2048 positions: a row's walk waits on memory once, not once
// per 64 positions.  The words at the range's ends are masked to it.
struct RowWalk {
  const uint32_t* row;
  uint32_t word;  // this lane's word of the current 64-word window
  int w0, lo, hi;
  __device__ RowWalk(const uint32_t* r, int lo_, int hi_) : row(r), w0(lo_ >> 5), lo(lo_), hi(hi_) { fill(); }
  __device__ inline void fill() {
    const int wi = w0 + (int)(threadIdx.x & 63);
    uint32_t x = lo <= hi && wi <= (hi >> 5) ? row[wi] : 0u;
    if (wi == (lo >> 5)) x &= ~0u << (lo & 31);
    if (wi == (hi >> 5)) x &= ~0u >> (31 - (hi & 31));
    word = x;
  }
  // next set position, or -1
  __device__ inline int next() {
    for (;;) {
      const unsigned long long m = __ballot(word != 0u);
      if (m != 0ull) {
        const int L = (int)__builtin_ctzll(m);
        const uint32_t wv = (uint32_t)__builtin_amdgcn_readlane((int)word, L);
        if ((int)(threadIdx.x & 63) == L) word &= word - 1u;
        return 32 * (w0 + L) + (int)__builtin_ctz(wv);
      }
      w0 += 64;
      if (lo > hi || w0 > (hi >> 5)) return -1;
      fill();
    }
  }
};

// Set bits of one bitmap column: rows lo..hi of bit `sh` in the words
// col[row * stride], visited in increasing order.  One fill issues the loads
// of 256 rows (four per lane) before the first ballot waits, so a column of
// up to 256 rows costs one load round trip.  All state is wave-uniform.
struct ColWalk {
  const uint32_t* col;
  int stride, sh, base, end, hi;
  unsigned long long m0, m1, m2, m3;  // rows base .. base+255, 64 per mask
  __device__ ColWalk(const uint32_t* c, int stride_, int sh_, int lo, int hi_)
      : col(c), stride(stride_), sh(sh_), base(lo), hi(hi_) { fill(); }
  __device__ inline uint32_t word(int p) const { return p <= hi ? col[(int64_t)p * stride] : 0u; }
  __device__ inline void fill() {
    const int p = base + (int)(threadIdx.x & 63);
    const uint32_t x0 = word(p), x1 = word(p + 64), x2 = word(p + 128), x3 = word(p + 192);
    m0 = __ballot(((x0 >> sh) & 1u) != 0u);
    m1 = __ballot(((x1 >> sh) & 1u) != 0u);
    m2 = __ballot(((x2 >> sh) & 1u) != 0u);
    m3 = __ballot(((x3 >> sh) & 1u) != 0u);
    end = base + 256;
  }
  // next set position, or -1
  __device__ inline int next() {
    for (;;) {
      if (m0 != 0ull) {
        const int idx = base + (int)__builtin_ctzll(m0);
        m0 &= m0 - 1ull;
        return idx;
      }
      if ((m1 | m2 | m3) != 0ull) {
        m0 = m1;
        m1 = m2;
        m2 = m3;
        m3 = 0ull;
        base += 64;
        continue;
      }
      base = end;
      if (base > hi) return -1;
      fill();
    }
  }
};

// Balanced XCD mapping for kernels with one block per (tile, head).  Blocks
// are dispatched round-robin over the 8 XCDs in linear order (x fastest).
// With nx % 32 == 0, XCD x receives the runs of four adjacent tiles 4x..4x+3,
// 4x+32.., ... of every head, head after head (with nx % 8 == 0 only, tiles
// x, x+8, ...): each XCD gets an equal share of every head's rows (whose cost
// depends on the head's window and threshold), and the blocks it runs at one
// time cover a few heads.  Adjacent tiles walk nearly the same key rows one
// unit apart, so within a run the rows one block loads are still in the
// XCD's L2 when the next block needs them.  Within a head the highest tiles
// come first.
__device__ inline void xcd_interleave(int& bx, int& by) {
  const int nx = gridDim.x;
  if ((nx & 7) == 0) {
    const int p = blockIdx.x + nx * blockIdx.y;
    const int x = p & 7, s = p >> 3, per = nx >> 3;
    by = s / per;
    const int t = s - by * per;  // the block's place in XCD x's share of the head
    bx = nx - 1 - ((nx & 31) == 0 ? (t >> 2) * 32 + x * 4 + (t & 3) : t * 8 + x);
  } else {
    by = blockIdx.y;
    bx = nx - 1 - blockIdx.x;
  }
}

// xcd_interleave with the heads taken widest window first.  Heads are (b, h)
// b-major and the window depends on h only, so logical head row by = r*B + b
// becomes (b, h of window rank r).  A unit's cost grows with its head's
// window, and blocks run in dispatch order, so the longest units no longer
// start last (the kernel would end with a few of them running alone).  Ties
// keep index order; more than 64 heads per batch keep plain order.  Called by
// every lane of a one-wave block.
//
// Ranks come from a total order, (window key, head index) with a NaN window
// keyed as +inf, so the ranks 0..H-1 are a permutation of the heads whatever
// the windows hold (NaN, infinities, duplicates): every (b, h) gets exactly
// one block row.  The mapping also returns the selected head's r_h and w_h:
// lane o receives r[o] and w[o] from the loads the ranking needs, and the
// head's values come back by readlane (no second dependent load).
__device__ inline float window_rank_key(float w) { return w != w ? INFINITY : w; }
__device__ inline void xcd_interleave_ranked(const float* r, const float* w, int H, int& bx, int& by, float& rh,
                                             float& wh) {
  xcd_interleave(bx, by);
  const int BH = (int)gridDim.y;
  if (H > 64 || BH % H != 0) {
    rh = r[by % H];
    wh = w[by % H];
    return;
  }
  const int lane = threadIdx.x & 63;
  // r and w through uniform (scalar-cache) loads: every wave reads the same
  // few words, and the scalar path does not queue behind the vector loads of
  // the other waves on the CU
  float wraw = 0.0f, rraw = 0.0f;
#pragma unroll 8
  for (int o = 0; o < H; ++o) {
    const float wo = w[o], ro = r[o];
    wraw = lane == o ? wo : wraw;
    rraw = lane == o ? ro : rraw;
  }
  const float wl = window_rank_key(wraw);  // lane o holds head o's key
  const int B = BH / H, rk = by / B, b = by % B;
  int rank = 0;
  for (int o = 0; o < H; ++o) {
    const float wo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wl), o));
    rank += (wo > wl || (wo == wl && o < lane)) ? 1 : 0;
  }
  const unsigned long long sel = __ballot(lane < H && rank == rk);
  const int h = sel != 0ull ? (int)__builtin_ctzll(sel) : rk;  // sel is never empty: ranks are a permutation
  by = b * H + h;
  rh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rraw), h));
  wh = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wraw), h));
}

}  // namespace msa
