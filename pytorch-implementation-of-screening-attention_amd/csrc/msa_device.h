// Device-side building blocks shared by the fused Screening Attention kernels
// for gfx950 (CDNA4): MFMA operand fragments, the tile/lane index maps and the
// per-pair screening math.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace msa {

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int kWave = 64;
constexpr int kTile = 64;  // rows of a query tile and of a key tile

// ---------------------------------------------------------------------------
// MFMA fragments.  Both element types use the 32x32 output block; a wave-64
// instruction contracts KS values of k.  Lane l supplies row (A) / column (B)
// l%32 and the PER contraction values of "slot group" l/32.  The mapping of
// (slot group, slot) to the hardware's k index is the same for A and B, so any
// contraction whose A and B slots are filled for the same logical k is exact
// whatever that mapping is.
//   C/D layout: lane l, register r -> row 8*(r/4) + 4*(l/32) + r%4, col l%32.
// ---------------------------------------------------------------------------
template <typename T> struct Mma;

template <> struct Mma<bf16> {
  static constexpr int KS = 16;
  static constexpr int PER = 8;
  typedef bf16x8 frag;
  __device__ static inline f32x16 mma(frag a, frag b, f32x16 c) {
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

template <> struct Mma<float> {
  static constexpr int KS = 2;
  static constexpr int PER = 1;
  typedef float frag;
  __device__ static inline f32x16 mma(frag a, frag b, f32x16 c) {
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

// ---------------------------------------------------------------------------
// Screening math for one (query i, key j) pair.
// ---------------------------------------------------------------------------
struct HeadParams {
  float r;     // acceptance sharpness r_h > 1 (may round to 1.0f)
  float w;     // window w_h > 1
  float iw;    // 1/w
  int64_t wc;  // ceil(w): for integer distance d, d < w  <=>  d < wc
};

__device__ inline HeadParams head_params(const float* r, const float* w, int h) {
  HeadParams p;
  p.r = r[h];
  p.w = w[h];
  p.iw = 1.0f / p.w;
  float c = ceilf(p.w);
  p.wc = c > 1.0e9f ? (int64_t)1000000000 : (int64_t)c;
  return p;
}

// In-window test on the integer distance dd = i - j (attention.py:111-118 causal,
// :176-181 non-causal).
__device__ inline bool in_window(int64_t dd, int64_t wc, bool causal) {
  return causal ? (dd >= 0 && dd < wc) : (dd < wc && -dd < wc);
}

// Trim-and-square pre-square value a = 1 - r (1 - s)  (attention.py:90).
__device__ inline float trim(float s, float r) { return 1.0f - r * (1.0f - s); }

// Cosine soft mask m = (cos(pi (j-i)/w) + 1)/2 (attention.py:114) and its
// derivative with respect to w, for an in-window distance dd = i - j.
__device__ inline float softmask(int64_t dd, float iw) {
  const float x = (float)(-dd) * iw;
  return 0.5f * (cospif(x) + 1.0f);
}
__device__ inline float softmask_dw(int64_t dd, float iw) {
  // d/dw [ (cos(pi rel/w)+1)/2 ] = sin(pi rel/w) * pi * rel / (2 w^2),  rel = j - i
  const float rel = (float)(-dd);
  const float x = rel * iw;
  return 0.5f * sinpif(x) * 3.14159265358979f * rel * iw * iw;
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
template <typename T> __device__ inline T from_f(float x);
template <> __device__ inline float from_f<float>(float x) { return x; }
template <> __device__ inline bf16 from_f<bf16>(float x) { return (bf16)x; }

// Stores 4 consecutive values.
__device__ inline void store4(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<f32x4*>(p) = f32x4{a, b, c, d};
}
__device__ inline void store4(bf16* p, float a, float b, float c, float d) {
  *reinterpret_cast<bf16x4*>(p) = bf16x4{(bf16)a, (bf16)b, (bf16)c, (bf16)d};
}
// Loads 4 consecutive values as fp32.
__device__ inline f32x4 load4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ inline f32x4 load4(const bf16* p) {
  bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}

__device__ inline int64_t floordiv(int64_t a, int64_t b) {  // b > 0
  return a >= 0 ? a / b : -((-a + b - 1) / b);
}

}  // namespace msa
