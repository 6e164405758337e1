// Host-side internal interface between the C ABI (msa_capi.hip) and the
// kernel translation units.  Everything here is validated before use.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace msa {

// Padded head dimension the kernels are instantiated for.
inline int padded_dim(int D) { return D <= 32 ? 32 : (D <= 64 ? 64 : 128); }
inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }
inline int ntiles(int64_t T) { return (int)((T + 63) / 64); }

struct Geometry {
  int B, H, Tq, Tk, D, DP, dtype, causal;
  int nqt, nkt;
  int nku_words;  // words per row of the live-unit bitmap (2*nkt 32-key units)
  int64_t Tq_pad, Tk_pad;
  size_t esize;  // bytes per element of dtype
};

struct Strides3 { int64_t sb, st, sh; };

// Forward workspace: khat [b*h][Tk_pad][DP], unit-normalised K rows (zero for
// padded and masked keys) that the forward stages through LDS.
size_t fwd_ws_bytes(const Geometry& g);

// Backward workspace: per-query-unit partial sums of dr, dw ([2][b*h][2*nqt]
// fp32), then dh ([b*h][Tq_pad][DP] in the input type) and 1/|q|
// ([b*h][Tq_pad] fp32) that dq_kernel hands to dkdv_kernel.
size_t bwd_ws_bytes(const Geometry& g);

// Attention dropout on alpha*m: pair (b, h, i, j) is kept iff the top 32 bits
// of its hash reach `thresh`, and kept pairs are scaled by `scale` = 1/(1-p).
struct Dropout {
  uint64_t seed;
  uint32_t thresh;
  float scale;
  int on;  // p > 0
};

// Dropout factor of pair (b*H+h, i, j): 0 or d.scale.  The SplitMix64
// finaliser (Steele, Lea and Flood, "Fast splittable pseudorandom number
// generators", OOPSLA 2014) of seed + key * 0x9E3779B97F4A7C15, key =
// bh << 44 | i << 22 | j (bh < 2^16, i, j < 2^22), decides: kept iff its top
// 32 bits reach d.thresh.
__device__ inline float dropout_factor(const Dropout& d, int bh, int i, int j) {
  const uint64_t key = ((uint64_t)(uint32_t)bh << 44) | ((uint64_t)(uint32_t)i << 22) | (uint64_t)(uint32_t)j;
  uint64_t z = d.seed + key * 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  z ^= z >> 31;
  return (uint32_t)(z >> 32) >= d.thresh ? d.scale : 0.0f;
}

struct FwdCall {
  Geometry g;
  const void* q; Strides3 qs;
  const void* k; Strides3 ks;
  const void* v; Strides3 vs;
  const float* r; const float* w; const uint8_t* kpm;
  float eps;
  Dropout drop;
  void* y; float* hnorm; uint32_t* bits;
  void* khat;
  hipStream_t stream;
};
hipError_t launch_fwd(const FwdCall& c);

struct BwdCall {
  Geometry g;
  const void* q; Strides3 qs;
  const void* k; Strides3 ks;
  const void* v; Strides3 vs;
  const float* r; const float* w; const uint8_t* kpm;
  float eps;
  Dropout drop;
  const void* y; const float* hnorm; const void* dy;
  const uint32_t* bits;
  void* workspace;
  void* dq; void* dk; void* dv; float* dr; float* dw;
  hipStream_t stream;
};
hipError_t launch_bwd(const BwdCall& c);

struct DecodeCall {
  int B, H, D, DP, dtype, len;
  const void* q; int64_t q_sb, q_sh;
  const void* kc; Strides3 ks;
  const void* vc; Strides3 vs;
  const float* r; const float* w; float eps;
  void* y; float* part;
  int blocks;  // grid size of the partial-sum kernel (any value >= 1 gives the same result)
  int single;  // 1: one block per head walks its chunks (no partials); same result
  const int64_t* last_pos;  // device position of the newest key, or null (len is the length)
  int cap;                  // cache capacity (bounds the device length)
  hipStream_t stream;
};
int decode_chunk_keys();
// Chunks of a head's window at most, ceil(max_len / chunk): the decode
// workspace holds B*H of them, D floats each.
int decode_max_chunks(int max_len);
hipError_t launch_decode(const DecodeCall& c);

// Optional event pairs around one kernel's launches (msa_timer_arm).
void timer_begin(int kernel, hipStream_t s);
void timer_end(int kernel, hipStream_t s);

hipError_t launch_selftest(const float* a16, const float* b16, float* out16,
                           const float* a2, const float* b2, float* out2,
                           hipStream_t stream);

}  // namespace msa
