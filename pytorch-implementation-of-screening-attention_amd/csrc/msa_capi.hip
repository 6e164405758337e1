// C ABI of libmsa.so (declared in include/msa.h): argument validation on the
// host, workspace carving, then stream-ordered kernel launches.  No device
// memory is allocated here.
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

#include "../../include/msa.h"

#include "msa_internal.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int ok() {
  g_last_error.clear();
  return MSA_OK;
}

constexpr int kMaxT = 1 << 22;  // live-unit bitmap rows are kept to <= 4096 words

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Shared shape validation; fills g on success.
int check_geometry(int B, int H, int Tq, int Tk, int D, int dtype, int causal, msa::Geometry* g) {
  if (dtype != MSA_F32 && dtype != MSA_BF16 && dtype != MSA_F16)
    return fail(MSA_ERR_INVALID, "dtype must be MSA_F32, MSA_BF16 or MSA_F16");
  if (!(D == 16 || D == 32 || D == 64 || D == 128))
    return fail(MSA_ERR_INVALID, "head_dim D=%d unsupported (16, 32, 64 or 128)", D);
  if (B < 0 || H <= 0 || Tq < 0 || Tk < 0) return fail(MSA_ERR_INVALID, "negative or zero size");
  if (Tq > kMaxT || Tk > kMaxT) return fail(MSA_ERR_INVALID, "sequence length above %d", kMaxT);
  if ((int64_t)B * H > 65535) return fail(MSA_ERR_INVALID, "B*H=%lld above 65535", (long long)B * H);
  g->B = B; g->H = H; g->Tq = Tq; g->Tk = Tk; g->D = D; g->DP = msa::padded_dim(D);
  g->dtype = dtype; g->causal = causal ? 1 : 0;
  g->nqt = msa::ntiles(Tq); g->nkt = msa::ntiles(Tk);
  g->nku_words = (2 * g->nkt + 31) / 32;
  g->Tq_pad = (int64_t)g->nqt * 64; g->Tk_pad = (int64_t)g->nkt * 64;
  g->esize = dtype == MSA_F32 ? 4 : 2;
  return MSA_OK;
}

int check_tensor(const char* name, const void* p, int64_t sb, int64_t st, int64_t sh, int dtype) {
  if (p == nullptr) return fail(MSA_ERR_INVALID, "%s is null", name);
  if (!aligned16(p)) return fail(MSA_ERR_INVALID, "%s is not 16-byte aligned", name);
  const int64_t m = dtype == MSA_F32 ? 4 : 8;
  if (sb < 0 || st < 0 || sh < 0 || sb % m || st % m || sh % m)
    return fail(MSA_ERR_INVALID, "%s strides (%lld,%lld,%lld) must be non-negative multiples of %lld elements", name,
                (long long)sb, (long long)st, (long long)sh, (long long)m);
  // kernels address the rows of a 64-row tile by 32-bit byte offsets from the
  // tile's first row
  const int64_t es = dtype == MSA_F32 ? 4 : 2;
  if (st * 64 * es >= (int64_t)1 << 32)
    return fail(MSA_ERR_INVALID, "%s time stride %lld elements is too large (64 rows must span < 4 GiB)", name,
                (long long)st);
  return MSA_OK;
}

int check_out(const char* name, const void* p) {
  if (p == nullptr) return fail(MSA_ERR_INVALID, "%s is null", name);
  if (!aligned16(p)) return fail(MSA_ERR_INVALID, "%s is not 16-byte aligned", name);
  return MSA_OK;
}

int hip_status(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(MSA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
  return ok();
}

// One armed event list per kernel id; several kernels may be armed at once.
struct TimerSlot {
  int next = 0;     // recorded pairs
  int every = 1;    // record launches 0, every, 2*every, ...
  int launch = 0;   // launches seen since arming
  std::vector<hipEvent_t> start, stop;
};
struct TimerState {
  std::mutex mu;
  TimerSlot slot[MSA_K_DECODE + 1];
};
TimerState& timer() {
  static TimerState t;
  return t;
}

void timer_clear(TimerSlot& s) {
  for (hipEvent_t e : s.start) (void)hipEventDestroy(e);
  for (hipEvent_t e : s.stop) (void)hipEventDestroy(e);
  s.start.clear();
  s.stop.clear();
  s.next = 0;
  s.every = 1;
  s.launch = 0;
}

}  // namespace

namespace msa {
void timer_begin(int kernel, hipStream_t s) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> g(t.mu);
  TimerSlot& sl = t.slot[kernel];
  if (sl.next < (int)sl.start.size() && sl.launch % sl.every == 0) (void)hipEventRecord(sl.start[sl.next], s);
}
void timer_end(int kernel, hipStream_t s) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> g(t.mu);
  TimerSlot& sl = t.slot[kernel];
  if (sl.next < (int)sl.stop.size() && sl.launch % sl.every == 0) (void)hipEventRecord(sl.stop[sl.next++], s);
  ++sl.launch;
}
}  // namespace msa

extern "C" {

int msa_timer_arm_every(int kernel, int n, int every) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> g(t.mu);
  if (kernel == 0) {
    for (TimerSlot& sl : t.slot) timer_clear(sl);
    return ok();
  }
  if (kernel < MSA_K_PREP_K || kernel > MSA_K_DECODE) return fail(MSA_ERR_INVALID, "unknown kernel id %d", kernel);
  if (every < 1) return fail(MSA_ERR_INVALID, "every must be >= 1 (got %d)", every);
  TimerSlot& sl = t.slot[kernel];
  timer_clear(sl);
  sl.every = every;
  for (int i = 0; i < n; ++i) {
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess) return fail(MSA_ERR_HIP, "hipEventCreate failed");
    if (hipEventCreate(&b) != hipSuccess) {
      (void)hipEventDestroy(a);
      return fail(MSA_ERR_HIP, "hipEventCreate failed");
    }
    sl.start.push_back(a);
    sl.stop.push_back(b);
  }
  return ok();
}

int msa_timer_arm(int kernel, int n) { return msa_timer_arm_every(kernel, n, 1); }

int msa_timer_read(int kernel, float* ms, int n) {
  TimerState& t = timer();
  std::lock_guard<std::mutex> g(t.mu);
  if (kernel < MSA_K_PREP_K || kernel > MSA_K_DECODE) {
    fail(MSA_ERR_INVALID, "unknown kernel id %d", kernel);
    return -1;
  }
  TimerSlot& sl = t.slot[kernel];
  int cnt = sl.next < n ? sl.next : n;
  for (int i = 0; i < cnt; ++i) {
    if (hipEventSynchronize(sl.stop[i]) != hipSuccess) return -1;
    if (hipEventElapsedTime(&ms[i], sl.start[i], sl.stop[i]) != hipSuccess) return -1;
  }
  return cnt;
}


// 0.1.0: first release; 0.2.0: msa_decode and msa_decode_at take window_hint
// (an argument inserted before r); 0.3.0: MSA_F16.
int msa_version(void) { return (0 << 16) | (3 << 8) | 0; }

const char* msa_last_error(void) { return g_last_error.c_str(); }

size_t msa_fwd_workspace_bytes(int B, int H, int Tq, int Tk, int D, int dtype) {
  // the screen plan's size depends on the mask (a non-causal window reaches
  // both ways, so more items): the larger of the two serves either call
  size_t need = 0;
  for (int causal = 0; causal <= 1; ++causal) {
    msa::Geometry g;
    if (check_geometry(B, H, Tq, Tk, D, dtype, causal, &g) != MSA_OK) return 0;
    const size_t n = msa::fwd_ws_bytes(g);
    need = n > need ? n : need;
  }
  return need;
}

size_t msa_tile_bits_words(int B, int H, int Tq, int Tk) {
  if (B < 0 || H <= 0 || Tq < 0 || Tk < 0) return 0;
  const int64_t nqt = msa::ntiles(Tq), nkt = msa::ntiles(Tk);
  return (size_t)((int64_t)B * H * 2 * nqt * ((2 * nkt + 31) / 32));
}

size_t msa_bwd_workspace_bytes(int B, int H, int Tq, int Tk, int D, int dtype) {
  msa::Geometry g;
  if (check_geometry(B, H, Tq, Tk, D, dtype, 1, &g) != MSA_OK) return 0;
  return msa::bwd_ws_bytes(g);
}

// Keep threshold min(floor(p * 2^32), 2^32-1) and scale 1/(1-p) of dropout p.
static msa::Dropout dropout_of(float p, uint64_t seed) {
  msa::Dropout d;
  d.seed = seed;
  const double t = floor((double)p * 4294967296.0);
  d.thresh = t >= 4294967295.0 ? 0xFFFFFFFFu : (uint32_t)t;
  d.scale = 1.0f / (1.0f - p);
  d.on = p > 0.0f ? 1 : 0;
  return d;
}

int msa_fwd(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, int64_t k_sb, int64_t k_st,
            int64_t k_sh, const void* v, int64_t v_sb, int64_t v_st, int64_t v_sh, int B, int H, int Tq, int Tk,
            int D, int dtype, const float* r, const float* w, const uint8_t* key_padding_mask, int causal, float eps,
            float dropout_p, uint64_t dropout_seed, void* y, float* hnorm, uint32_t* tile_bits, size_t tile_bits_words, void* workspace,
            size_t workspace_bytes, void* stream) {
  msa::Geometry g;
  int rc = check_geometry(B, H, Tq, Tk, D, dtype, causal, &g);
  if (rc != MSA_OK) return rc;
  if (!(eps > 0.0f)) return fail(MSA_ERR_INVALID, "eps must be positive");
  if (!(dropout_p >= 0.0f && dropout_p < 1.0f)) return fail(MSA_ERR_INVALID, "dropout_p must be in [0, 1)");
  if (B == 0 || Tq == 0) return ok();
  if ((rc = check_tensor("q", q, q_sb, q_st, q_sh, dtype)) != MSA_OK) return rc;
  if (Tk > 0) {
    if ((rc = check_tensor("k", k, k_sb, k_st, k_sh, dtype)) != MSA_OK) return rc;
    if ((rc = check_tensor("v", v, v_sb, v_st, v_sh, dtype)) != MSA_OK) return rc;
  }
  if (r == nullptr || w == nullptr) return fail(MSA_ERR_INVALID, "r and w must be device arrays of H floats");
  if ((rc = check_out("y", y)) != MSA_OK) return rc;
  if (hnorm == nullptr) return fail(MSA_ERR_INVALID, "hnorm is null");
  if (tile_bits == nullptr) return fail(MSA_ERR_INVALID, "tile_bits is null");
  if (tile_bits_words < msa_tile_bits_words(B, H, Tq, Tk))
    return fail(MSA_ERR_WORKSPACE, "tile_bits holds %zu words, %zu needed", tile_bits_words,
                msa_tile_bits_words(B, H, Tq, Tk));
  const size_t need = msa::fwd_ws_bytes(g);
  if (workspace_bytes < need || (need > 0 && workspace == nullptr))
    return fail(MSA_ERR_WORKSPACE, "forward workspace holds %zu bytes, %zu needed", workspace_bytes, need);
  if (need > 0 && !aligned16(workspace)) return fail(MSA_ERR_INVALID, "workspace is not 16-byte aligned");

  msa::FwdCall c;
  c.g = g;
  c.q = q; c.qs = {q_sb, q_st, q_sh};
  c.k = k; c.ks = {k_sb, k_st, k_sh};
  c.v = v; c.vs = {v_sb, v_st, v_sh};
  c.r = r; c.w = w; c.kpm = key_padding_mask; c.eps = eps;
  c.drop = dropout_of(dropout_p, dropout_seed);
  c.y = y; c.hnorm = hnorm; c.bits = tile_bits;
  c.khat = workspace;
  c.stream = (hipStream_t)stream;
  return hip_status(msa::launch_fwd(c), "msa_fwd launch");
}

int msa_bwd(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh, const void* k, int64_t k_sb, int64_t k_st,
            int64_t k_sh, const void* v, int64_t v_sb, int64_t v_st, int64_t v_sh, int B, int H, int Tq, int Tk,
            int D, int dtype, const float* r, const float* w, const uint8_t* key_padding_mask, int causal, float eps,
            float dropout_p, uint64_t dropout_seed, const void* y, const float* hnorm, const void* dy, const uint32_t* tile_bits, size_t tile_bits_words,
            void* dq, void* dk, void* dv, float* dr, float* dw, void* workspace, size_t workspace_bytes,
            void* stream) {
  msa::Geometry g;
  int rc = check_geometry(B, H, Tq, Tk, D, dtype, causal, &g);
  if (rc != MSA_OK) return rc;
  if (!(eps > 0.0f)) return fail(MSA_ERR_INVALID, "eps must be positive");
  if (!(dropout_p >= 0.0f && dropout_p < 1.0f)) return fail(MSA_ERR_INVALID, "dropout_p must be in [0, 1)");
  if (dr == nullptr || dw == nullptr) return fail(MSA_ERR_INVALID, "dr and dw must be device arrays of H floats");
  if (B == 0 || Tq == 0 || Tk == 0)
    return fail(MSA_ERR_INVALID, "msa_bwd needs B, Tq, Tk > 0 (the caller zero-fills empty gradients)");
  if ((rc = check_tensor("q", q, q_sb, q_st, q_sh, dtype)) != MSA_OK) return rc;
  if ((rc = check_tensor("k", k, k_sb, k_st, k_sh, dtype)) != MSA_OK) return rc;
  if ((rc = check_tensor("v", v, v_sb, v_st, v_sh, dtype)) != MSA_OK) return rc;
  if (r == nullptr || w == nullptr) return fail(MSA_ERR_INVALID, "r and w must be device arrays of H floats");
  if ((rc = check_out("y", y)) != MSA_OK) return rc;
  if ((rc = check_out("dy", dy)) != MSA_OK) return rc;
  if ((rc = check_out("dq", dq)) != MSA_OK) return rc;
  if ((rc = check_out("dk", dk)) != MSA_OK) return rc;
  if ((rc = check_out("dv", dv)) != MSA_OK) return rc;
  if (hnorm == nullptr || tile_bits == nullptr) return fail(MSA_ERR_INVALID, "hnorm / tile_bits is null");
  if (tile_bits_words < msa_tile_bits_words(B, H, Tq, Tk))
    return fail(MSA_ERR_WORKSPACE, "tile_bits holds %zu words, %zu needed", tile_bits_words,
                msa_tile_bits_words(B, H, Tq, Tk));
  const size_t need = msa::bwd_ws_bytes(g);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(MSA_ERR_WORKSPACE, "backward workspace holds %zu bytes, %zu needed", workspace_bytes, need);
  if (!aligned16(workspace)) return fail(MSA_ERR_INVALID, "workspace is not 16-byte aligned");

  msa::BwdCall c;
  c.g = g;
  c.q = q; c.qs = {q_sb, q_st, q_sh};
  c.k = k; c.ks = {k_sb, k_st, k_sh};
  c.v = v; c.vs = {v_sb, v_st, v_sh};
  c.r = r; c.w = w; c.kpm = key_padding_mask; c.eps = eps;
  c.drop = dropout_of(dropout_p, dropout_seed);
  c.y = y; c.hnorm = hnorm; c.dy = dy; c.bits = tile_bits;
  c.workspace = workspace;
  c.dq = dq; c.dk = dk; c.dv = dv; c.dr = dr; c.dw = dw;
  c.stream = (hipStream_t)stream;
  return hip_status(msa::launch_bwd(c), "msa_bwd launch");
}

size_t msa_decode_workspace_bytes(int B, int H, int D, int max_len) {
  if (B <= 0 || H <= 0 || max_len <= 0 || !(D == 16 || D == 32 || D == 64 || D == 128)) return 0;
  return (size_t)B * H * msa::decode_max_chunks(max_len) * D * sizeof(float);
}

// Validates a decode call and fills c (all but the partial-sum buffer).  The
// cache length is cache_len, or, with last_pos non-null, read on the device
// (*last_pos + 1, clamped to [1, cache_cap]; cache_len is then ignored).
// Returns MSA_OK, an error code, or -1 when B == 0 (nothing to do).
static int decode_setup(const void* q, int64_t q_sb, int64_t q_sh, const void* kcache, int64_t k_sb, int64_t k_st,
                        int64_t k_sh, const void* vcache, int64_t v_sb, int64_t v_st, int64_t v_sh, int B, int H,
                        int D, int dtype, int cache_len, const int64_t* last_pos, int cache_cap, int window_hint,
                        const float* r, const float* w, float eps, void* y, void* stream, msa::DecodeCall* c) {
  msa::Geometry g;
  if (last_pos != nullptr) cache_len = cache_cap;  // the longest the device length can be
  int rc = check_geometry(B, H, 1, cache_len, D, dtype, 1, &g);
  if (rc != MSA_OK) return rc;
  if (B == 0) return -1;
  if (cache_len <= 0) return fail(MSA_ERR_INVALID, "cache_len must be >= 1 (the new token is in the cache)");
  if (cache_len > cache_cap)
    return fail(MSA_ERR_INVALID, "cache_len %d exceeds the cache capacity %d", cache_len, cache_cap);
  if (!(eps > 0.0f)) return fail(MSA_ERR_INVALID, "eps must be positive");
  if ((rc = check_tensor("q", q, q_sb, 0, q_sh, dtype)) != MSA_OK) return rc;
  if ((rc = check_tensor("kcache", kcache, k_sb, k_st, k_sh, dtype)) != MSA_OK) return rc;
  if ((rc = check_tensor("vcache", vcache, v_sb, v_st, v_sh, dtype)) != MSA_OK) return rc;
  if (r == nullptr || w == nullptr) return fail(MSA_ERR_INVALID, "r and w must be device arrays of H floats");
  if ((rc = check_out("y", y)) != MSA_OK) return rc;
  c->B = B; c->H = H; c->D = D; c->DP = g.DP; c->dtype = dtype; c->len = cache_len;
  c->last_pos = last_pos; c->cap = cache_cap;
  c->q = q; c->q_sb = q_sb; c->q_sh = q_sh;
  c->kc = kcache; c->ks = {k_sb, k_st, k_sh};
  c->vc = vcache; c->vs = {v_sb, v_st, v_sh};
  c->r = r; c->w = w; c->eps = eps;
  c->y = y; c->part = nullptr;
  // one block per window chunk of every head when the hint bounds the
  // windows; any grid gives the same result, the hint only sizes it
  const int span = window_hint > 0 && window_hint < cache_len ? window_hint : cache_len;
  c->blocks = B * H * msa::decode_max_chunks(span);
  // windows that fit one chunk: one block per head finishes it (same result)
  c->single = span <= msa::decode_chunk_keys() ? 1 : 0;
  c->stream = (hipStream_t)stream;
  return MSA_OK;
}

int msa_decode(const void* q, int64_t q_sb, int64_t q_sh, const void* kcache, int64_t k_sb, int64_t k_st,
               int64_t k_sh, const void* vcache, int64_t v_sb, int64_t v_st, int64_t v_sh, int B, int H, int D,
               int dtype, int cache_len, int cache_cap, int window_hint, const float* r, const float* w, float eps,
               void* y, void* workspace, size_t workspace_bytes, void* stream) {
  msa::DecodeCall c;
  const int rc = decode_setup(q, q_sb, q_sh, kcache, k_sb, k_st, k_sh, vcache, v_sb, v_st, v_sh, B, H, D, dtype,
                              cache_len, nullptr, cache_cap, window_hint, r, w, eps, y, stream, &c);
  if (rc == -1) return ok();
  if (rc != MSA_OK) return rc;
  const size_t need = msa_decode_workspace_bytes(B, H, D, cache_len);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(MSA_ERR_WORKSPACE, "decode workspace holds %zu bytes, %zu needed", workspace_bytes, need);
  c.part = (float*)workspace;
  return hip_status(msa::launch_decode(c), "msa_decode launch");
}

int msa_decode_at(const void* q, int64_t q_sb, int64_t q_sh, const void* kcache, int64_t k_sb, int64_t k_st,
                  int64_t k_sh, const void* vcache, int64_t v_sb, int64_t v_st, int64_t v_sh, int B, int H, int D,
                  int dtype, const int64_t* last_pos, int cache_cap, int window_hint, const float* r, const float* w,
                  float eps, void* y, void* workspace, size_t workspace_bytes, void* stream) {
  if (last_pos == nullptr) return fail(MSA_ERR_INVALID, "last_pos must be a device int64");
  msa::DecodeCall c;
  const int rc = decode_setup(q, q_sb, q_sh, kcache, k_sb, k_st, k_sh, vcache, v_sb, v_st, v_sh, B, H, D, dtype, 0,
                              last_pos, cache_cap, window_hint, r, w, eps, y, stream, &c);
  if (rc == -1) return ok();
  if (rc != MSA_OK) return rc;
  const size_t need = msa_decode_workspace_bytes(B, H, D, cache_cap);
  if (workspace == nullptr || workspace_bytes < need)
    return fail(MSA_ERR_WORKSPACE, "decode workspace holds %zu bytes, %zu needed", workspace_bytes, need);
  c.part = (float*)workspace;
  return hip_status(msa::launch_decode(c), "msa_decode_at launch");
}

// ---------------------------------------------------------------------------
// Decode without allocation.  The partial sums live in `scratch`, a static
// device array: every GPU the library runs on holds its own copy (16 MiB)
// until the process ends.  Host code never uses the array's name as an
// address: on the first call on each device, with that device current, its
// device address is looked up once and kept per device.  Calls that overlap
// on one GPU share the array and race; nothing in it needs clearing (every
// partial is written before it is read).
// ---------------------------------------------------------------------------
static __device__ __align__(256) float scratch[MSA_DECODE_STATIC_SCRATCH_BYTES / sizeof(float)];

namespace {
struct ScratchTable {
  std::mutex mu;
  std::vector<void*> ptr;  // device address of `scratch`, per device ordinal
};
ScratchTable& scratch_table() {
  static ScratchTable t;
  return t;
}
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(MSA_ERR_HIP, "hipGetDevice: %s", hipGetErrorString(e));
  ScratchTable& t = scratch_table();
  std::lock_guard<std::mutex> g(t.mu);
  if (dev >= (int)t.ptr.size()) t.ptr.resize(dev + 1, nullptr);
  if (t.ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(MSA_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    t.ptr[dev] = p;
  }
  *out = t.ptr[dev];
  return MSA_OK;
}
}  // namespace

int msa_decode_noalloc(const void* q, int64_t q_sb, int64_t q_sh, const void* kcache, int64_t k_sb, int64_t k_st,
                       int64_t k_sh, const void* vcache, int64_t v_sb, int64_t v_st, int64_t v_sh, int B, int H,
                       int D, int dtype, int cache_len, int cache_cap, int window_hint, const float* r,
                       const float* w, float eps, void* y, void* stream) {
  msa::DecodeCall c;
  int rc = decode_setup(q, q_sb, q_sh, kcache, k_sb, k_st, k_sh, vcache, v_sb, v_st, v_sh, B, H, D, dtype,
                        cache_len, nullptr, cache_cap, window_hint, r, w, eps, y, stream, &c);
  if (rc == -1) return ok();
  if (rc != MSA_OK) return rc;
  const size_t need = msa_decode_workspace_bytes(B, H, D, cache_len);
  if (need > (size_t)MSA_DECODE_STATIC_SCRATCH_BYTES)
    return fail(MSA_ERR_WORKSPACE,
                "msa_decode_noalloc: %zu bytes of partial sums needed (B*H*ceil(cache_len/2048)*D*4), the static "
                "scratch holds %zu; use msa_decode with a workspace",
                need, (size_t)MSA_DECODE_STATIC_SCRATCH_BYTES);
  void* p = nullptr;
  if ((rc = scratch_address(&p)) != MSA_OK) return rc;
  c.part = (float*)p;
  return hip_status(msa::launch_decode(c), "msa_decode_noalloc launch");
}

int msa_selftest_mfma(const float* a16, const float* b16, float* out16, const float* a2, const float* b2,
                      float* out2, void* stream) {
  if (!a16 || !b16 || !out16 || !a2 || !b2 || !out2) return fail(MSA_ERR_INVALID, "null pointer");
  return hip_status(msa::launch_selftest(a16, b16, out16, a2, b2, out2, (hipStream_t)stream), "selftest launch");
}

}  // extern "C"
