// Single-query decode against a KV cache (gfx950).
//
// The query at position pos = len-1 attends to keys j in (pos - w, pos]
// (causal window, attention.py:111-118).  Each head's window is cut into
// chunks of kChunk keys; a work item is one (b, h, chunk), items numbered in
// (b, h, chunk) order, and the number of items is computed on the device from
// the windows themselves, so only windowed keys are ever visited.  For each
// chunk a 256-thread block streams the raw K rows (16-byte loads, D/VEC lanes
// per key), forms s = q.k/(|q||k|) from exact products of the raw values, and
// reads a V row only when its alpha*m is non-zero.  Because screening has no
// softmax normaliser (attention.py:192-193), chunk partials simply add, in a
// fixed order, before TanhNorm (norm.py:23-25).
//
// Two launch shapes, bitwise the same result (same chunk partials, summed in
// the same order):
//   split:  decode_partial_kernel (blocks take items blockIdx.x,
//           blockIdx.x + gridDim.x, ...; partials to the workspace), then
//           decode_reduce_kernel (block per (b, h): sum and TanhNorm);
//   single: decode_single_kernel, block per (b, h) walking its head's chunks
//           (one when the windows fit a chunk: one launch, no workspace
//           traffic).
// The cache length is a host value, or read on the device (the position of
// the newest key plus one, clamped to [1, cap]), so a captured launch stays
// valid as the sequence grows.
#include <type_traits>

#include "msa_device.h"
#include "msa_internal.h"

namespace msa {

constexpr int kChunk = 2048;
constexpr int kDecUnroll = 16;  // K row loads per lane in flight per round

struct DecArgs {
  const void* q; int64_t q_sb, q_sh;
  const void* kc; Strides3 ks;
  const void* vc; Strides3 vs;
  const float* r; const float* w;
  float* part;  // [item][D], items in (b, h, chunk) order
  void* y;
  int B, H, len;
  const int64_t* last_pos;  // device position of the newest key, or null (len holds the length)
  int cap;                  // cache capacity: bounds the device length
  float eps;
};

// The call's arguments with the cache length resolved: the host value, or the
// device one, (*last_pos + 1) clamped to [1, cap].
__device__ inline DecArgs resolve_len(DecArgs a) {
  if (a.last_pos != nullptr) {
    int64_t n = *a.last_pos + 1;
    n = n < 1 ? 1 : (n > a.cap ? a.cap : n);
    a.len = (int)n;
  }
  return a;
}

// 16 bytes of a row in its storage type, and its fp32 dot products.
template <typename T> struct Vec16;
template <> struct Vec16<bf16> {
  typedef bf16x8 type;
  static constexpr int N = 8;
  __device__ static inline float dot(const type& a, const type& b, float acc) { return frag_dot(a, b, acc); }
  __device__ static inline float get(const type& a, int e) { return (float)a[e]; }
};
template <> struct Vec16<f16> {
  typedef f16x8 type;
  static constexpr int N = 8;
  __device__ static inline float dot(const type& a, const type& b, float acc) { return frag_dot(a, b, acc); }
  __device__ static inline float get(const type& a, int e) { return (float)a[e]; }
};
template <> struct Vec16<float> {
  typedef f32x4 type;
  static constexpr int N = 4;
  __device__ static inline float dot(const type& a, const type& b, float acc) {
    return acc + a[0] * b[0] + a[1] * b[1] + a[2] * b[2] + a[3] * b[3];
  }
  __device__ static inline float get(const type& a, int e) { return a[e]; }
};

// First key of head h's window at position pos, and its number of chunks.
__device__ inline int64_t window_lo(const DecArgs& a, int h) {
  const HeadParams hp = head_params(a.r, a.w, h, true);
  const int64_t lo = (int64_t)a.len - hp.wc;  // pos - wc + 1
  return lo < 0 ? 0 : lo;
}
__device__ inline int head_chunks(const DecArgs& a, int h) {
  return (int)(((int64_t)a.len - window_lo(a, h) + kChunk - 1) / kChunk);
}

// Wave-uniform item map (every lane of the wave calls these).  Per batch row
// the items are the heads' chunks in head order.  items_per_b(): the count;
// head_of(rem, h, c0): the head h whose items hold index rem of a batch row,
// and the index c0 of that head's first item.
__device__ inline int lane_inclusive_scan(int x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  return x;
}
__device__ inline int items_per_b(const DecArgs& a) {
  const int lane = threadIdx.x & 63;
  int total = 0;
  for (int h0 = 0; h0 < a.H; h0 += 64) {
    const int c = h0 + lane < a.H ? head_chunks(a, h0 + lane) : 0;
    total += __shfl(lane_inclusive_scan(c), 63);
  }
  return total;
}
__device__ inline void head_of(const DecArgs& a, int rem, int& h, int& c0) {
  const int lane = threadIdx.x & 63;
  int carry = 0;
  for (int h0 = 0; h0 < a.H; h0 += 64) {
    const int c = h0 + lane < a.H ? head_chunks(a, h0 + lane) : 0;
    const int incl = lane_inclusive_scan(c) + carry;
    const unsigned long long sel = __ballot(h0 + lane < a.H && incl > rem);
    if (sel != 0ull) {
      const int l = (int)__builtin_ctzll(sel);
      h = h0 + l;
      c0 = __shfl(incl - c, l);
      return;
    }
    carry = __shfl(incl, 63);
  }
  h = a.H - 1;  // not reached for rem < items_per_b
  c0 = carry;
}

// One chunk (keys [c0, cend)) of head (b, h), by the whole 256-thread block:
// on return red[w][d] holds wave w's sum (the chunk's partial is
// red[0][d] + red[1][d] + red[2][d] + red[3][d]); the caller syncs before
// reading it and again before the next call.
template <typename T, int D>
__device__ inline void chunk_partial(const DecArgs& a, int b, int h, const HeadParams& hp, int64_t c0, int64_t cend,
                                     float (&red)[4][D]) {
  using V = Vec16<T>;
  using vec = typename V::type;
  constexpr int VEC = V::N;                 // elements per 16-byte load
  constexpr int LPK = D / VEC;              // lanes per key row
  constexpr int KPW = kWave / LPK;          // keys per wave per load
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % LPK, kl = lane / LPK;
  const int d0 = sub * VEC;
  const int64_t pos = a.len - 1;
  float acc[VEC];
#pragma unroll
  for (int e = 0; e < VEC; ++e) acc[e] = 0.0f;
  // raw query slice and 1/|q| (each LPK-lane group covers the whole row);
  // s = (q . k) / (|q| |k|) with exact products of the raw values
  const vec qv = *reinterpret_cast<const vec*>((const T*)a.q + b * a.q_sb + h * a.q_sh + d0);
  float qq = V::dot(qv, qv, 0.0f);
#pragma unroll
  for (int o = 1; o < LPK; o <<= 1) qq += __shfl_xor(qq, o);
  const float iq = 1.0f / fmaxf(sqrtf(qq), a.eps);
  const T* kb = (const T*)a.kc + b * a.ks.sb + h * a.ks.sh + d0;
  const T* vb = (const T*)a.vc + b * a.vs.sb + h * a.vs.sh + d0;
  for (int64_t base = c0 + (int64_t)wave * KPW * kDecUnroll; base < cend; base += 4 * KPW * kDecUnroll) {
    vec kv[kDecUnroll];
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      const int64_t j = base + u * KPW + kl;
      // streamed once: non-temporal loads keep the stream from churning the caches
      kv[u] = __builtin_nontemporal_load(reinterpret_cast<const vec*>(kb + (j < cend ? j : c0) * a.ks.st));
    }
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      const float dot = group_sum<LPK>(V::dot(qv, kv[u], 0.0f));
      const float ss = group_sum<LPK>(V::dot(kv[u], kv[u], 0.0f));
      const float s = dot * iq * inv_len(ss, a.eps);
      const float av = trim(s, hp.r);
      const int64_t j = base + u * KPW + kl;
      if (j < cend && av > 0.0f) {
        // every lane of the key's group takes this branch together
        const float m = mask_fast((int)(pos - j), hp.w, hp.iw);
        const vec vv = *reinterpret_cast<const vec*>(vb + j * a.vs.st);
        const float vs2 = group_sum<LPK>(V::dot(vv, vv, 0.0f));
        const float coef = av * av * m * inv_len(vs2, a.eps);
#pragma unroll
        for (int e = 0; e < VEC; ++e) acc[e] += coef * V::get(vv, e);
      }
    }
  }
  // reduce over the key groups of the wave; lane group 0 leaves the wave's sum
#pragma unroll
  for (int o = LPK; o < kWave; o <<= 1)
#pragma unroll
    for (int e = 0; e < VEC; ++e) acc[e] += __shfl_xor(acc[e], o);
  if (kl == 0)
#pragma unroll
    for (int e = 0; e < VEC; ++e) red[wave][d0 + e] = acc[e];
}

// Head (b, h)'s output from its chunk partials, accumulated by thread t
// (group g = t / D of G = 256/D groups, d = t % D) as x0 (chunks g, g+2G,
// ...) and x1 (chunks g+G, g+3G, ...), each in increasing chunk order: the
// groups' sums are added in order, then TanhNorm.  Block-wide.
template <typename T, int D>
__device__ inline void finish_head(const DecArgs& a, int bh, float x0, float x1, float (&red)[256], float (&sq)[D]) {
  constexpr int G = 256 / D;
  const int t = threadIdx.x;
  red[t] = x0 + x1;
  __syncthreads();
  float x = 0.0f;
  if (t < D) {
#pragma unroll
    for (int k = 0; k < G; ++k) x += red[k * D + t];
    sq[t] = x * x;
  }
  __syncthreads();
  for (int s2 = D / 2; s2 > 0; s2 >>= 1) {
    if (t < s2) sq[t] += sq[t + s2];
    __syncthreads();
  }
  const float nc = fmaxf(sqrtf(sq[0]), a.eps);
  const float f = tanhf(nc) / nc;
  if (t < D) ((T*)a.y)[(int64_t)bh * D + t] = from_f<T>(f * x);
}

template <typename T, int D>
__global__ __launch_bounds__(256) void decode_partial_kernel(DecArgs a0) {
  const DecArgs a = resolve_len(a0);
  __shared__ float red[4][D];
  const int per_b = items_per_b(a);
  const int total = a.B * per_b;
  for (int item = blockIdx.x; item < total; item += gridDim.x) {
    const int b = item / per_b;
    int h, c0i;
    head_of(a, item - b * per_b, h, c0i);
    const int chunk = item - b * per_b - c0i;
    const HeadParams hp = head_params(a.r, a.w, h, true);
    const int64_t c0 = window_lo(a, h) + (int64_t)chunk * kChunk;
    const int64_t cend = c0 + kChunk < a.len ? c0 + kChunk : a.len;
    chunk_partial<T, D>(a, b, h, hp, c0, cend, red);
    __syncthreads();
    if (threadIdx.x < D) {
      const int d = threadIdx.x;
      a.part[(int64_t)item * D + d] = red[0][d] + red[1][d] + red[2][d] + red[3][d];
    }
    __syncthreads();  // red is reused by the next item
  }
}

// Sum of head (b, h)'s chunk partials (finish_head's order) and TanhNorm;
// block per (b, h).
template <typename T, int D>
__global__ __launch_bounds__(256) void decode_reduce_kernel(DecArgs a0) {
  const DecArgs a = resolve_len(a0);
  constexpr int G = 256 / D;  // chunk groups
  __shared__ float red[256];
  __shared__ float sq[D];
  __shared__ int map[2];  // first item of head (b, h), its number of items
  const int bh = blockIdx.x, t = threadIdx.x, d = t % D, g = t / D;
  const int b = bh / a.H, hh = bh % a.H;
  if (t < 64) {  // wave 0 maps the items; the block shares the result
    const int per_b = items_per_b(a);
    int carry = 0, first = 0;
    for (int h0 = 0; h0 < a.H; h0 += 64) {
      const int c = h0 + t < a.H ? head_chunks(a, h0 + t) : 0;
      const int incl = lane_inclusive_scan(c) + carry;
      const int excl = __shfl(incl - c, (hh - h0) & 63);  // items of heads before hh
      if (hh >= h0 && hh < h0 + 64) first = excl;
      carry = __shfl(incl, 63);
    }
    if (t == 0) {
      map[0] = b * per_b + first;
      map[1] = head_chunks(a, hh);
    }
  }
  __syncthreads();
  const int used = map[1];
  const float* pp = a.part + d + (int64_t)map[0] * D;
  float x0 = 0.0f, x1 = 0.0f;
  int c = g;
  for (; c + G < used; c += 2 * G) {
    x0 += pp[(int64_t)c * D];
    x1 += pp[(int64_t)(c + G) * D];
  }
  if (c < used) x0 += pp[(int64_t)c * D];
  finish_head<T, D>(a, bh, x0, x1, red, sq);
}

// Block per (b, h): the head's chunks in order, each partial formed exactly as
// decode_partial_kernel forms it and accumulated as decode_reduce_kernel sums
// it, then TanhNorm.  No workspace.
template <typename T, int D>
__global__ __launch_bounds__(256) void decode_single_kernel(DecArgs a0) {
  const DecArgs a = resolve_len(a0);
  constexpr int G = 256 / D;
  __shared__ float part[4][D];
  __shared__ float red[256];
  __shared__ float sq[D];
  const int bh = blockIdx.x, t = threadIdx.x, d = t % D, g = t / D;
  const int b = bh / a.H, h = bh % a.H;
  const HeadParams hp = head_params(a.r, a.w, h, true);
  const int64_t lo = window_lo(a, h);
  const int used = head_chunks(a, h);
  float x0 = 0.0f, x1 = 0.0f;
  for (int c = 0; c < used; ++c) {
    const int64_t c0 = lo + (int64_t)c * kChunk;
    const int64_t cend = c0 + kChunk < a.len ? c0 + kChunk : a.len;
    chunk_partial<T, D>(a, b, h, hp, c0, cend, part);
    __syncthreads();
    if (c % G == g) {
      const float p = part[0][d] + part[1][d] + part[2][d] + part[3][d];
      if (((c / G) & 1) == 0) x0 += p;
      else x1 += p;
    }
    __syncthreads();  // part is reused by the next chunk
  }
  finish_head<T, D>(a, bh, x0, x1, red, sq);
}

int decode_chunk_keys() { return kChunk; }
int decode_max_chunks(int max_len) { return (max_len + kChunk - 1) / kChunk; }

template <typename T, int D>
static hipError_t launch_decode_t(const DecodeCall& c) {
  DecArgs a;
  a.q = c.q; a.q_sb = c.q_sb; a.q_sh = c.q_sh;
  a.kc = c.kc; a.ks = c.ks; a.vc = c.vc; a.vs = c.vs;
  a.r = c.r; a.w = c.w; a.part = c.part; a.y = c.y;
  a.B = c.B; a.H = c.H; a.len = c.len; a.eps = c.eps;
  a.last_pos = c.last_pos; a.cap = c.cap;
  // the decode timer brackets the whole single-query step
  timer_begin(7, c.stream);
  if (c.single) {
    hipLaunchKernelGGL((decode_single_kernel<T, D>), dim3((unsigned)(c.B * c.H)), dim3(256), 0, c.stream, a);
    timer_end(7, c.stream);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((decode_partial_kernel<T, D>), dim3((unsigned)c.blocks), dim3(256), 0, c.stream, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((decode_reduce_kernel<T, D>), dim3((unsigned)(c.B * c.H)), dim3(256), 0, c.stream, a);
  timer_end(7, c.stream);
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeCall& c) {
  if (c.dtype == 1) {
    switch (c.D) {
      case 16: return launch_decode_t<bf16, 16>(c);
      case 32: return launch_decode_t<bf16, 32>(c);
      case 64: return launch_decode_t<bf16, 64>(c);
      default: return launch_decode_t<bf16, 128>(c);
    }
  }
  if (c.dtype == 2) {
    switch (c.D) {
      case 16: return launch_decode_t<f16, 16>(c);
      case 32: return launch_decode_t<f16, 32>(c);
      case 64: return launch_decode_t<f16, 64>(c);
      default: return launch_decode_t<f16, 128>(c);
    }
  }
  switch (c.D) {
    case 16: return launch_decode_t<float, 16>(c);
    case 32: return launch_decode_t<float, 32>(c);
    case 64: return launch_decode_t<float, 64>(c);
    default: return launch_decode_t<float, 128>(c);
  }
}

// ---------------------------------------------------------------------------
// MFMA layout self-test: one wave computes a 32x32 product with each operand
// form, loading operands and storing the result with the lane maps the
// kernels use.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void selftest_kernel(const float* a16, const float* b16, float* out16,
                                                      const float* a2, const float* b2, float* out2) {
  const int lane = threadIdx.x, half = lane >> 5, l32 = lane & 31;
  bf16x8 fa, fb;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    fa[e] = (bf16)a16[l32 * 16 + 8 * half + e];      // A[m=l32][k]
    fb[e] = (bf16)b16[(8 * half + e) * 32 + l32];    // B[k][n=l32]
  }
  f32x16 c = {};
  c = Mma<bf16>::mma(fa, fb, c);
  f32x16 c2 = {};
  c2 = Mma<float>::mma(a2[l32 * 2 + half], b2[half * 32 + l32], c2);
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = 8 * (r / 4) + 4 * half + (r % 4);
    out16[row * 32 + l32] = c[r];
    out2[row * 32 + l32] = c2[r];
  }
}

hipError_t launch_selftest(const float* a16, const float* b16, float* out16, const float* a2, const float* b2,
                           float* out2, hipStream_t stream) {
  hipLaunchKernelGGL(selftest_kernel, dim3(1), dim3(64), 0, stream, a16, b16, out16, a2, b2, out2);
  return hipGetLastError();
}

}  // namespace msa
