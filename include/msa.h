/*
 * msa.h -- C ABI of the MI355X (gfx950) fused Screening Attention library
 * (libmsa.so).  Plain pointers, sizes and a hipStream_t passed as void*; no
 * torch or C++ types cross this boundary.
 *
 * The math is that of the reference's dense path
 *   /root/reference/multiscreen/attention.py:142-200 and norm.py:23-25:
 *     q^ = q/max(|q|,eps)   k^, v^ likewise                (attention.py:155-158)
 *     s_ij = q^_i . k^_j                                      (attention.py:160-161)
 *     a_ij = relu(1 - r_h (1 - s_ij)),  alpha_ij = a_ij^2      (attention.py:75-90)
 *     m_ij = (cos(pi (j-i)/w_h) + 1)/2 on -w<j-i<=0 (causal)   (attention.py:92-119)
 *            or on |j-i|<w (non-causal)                        (attention.py:174-183)
 *     alpha_ij = 0 where key_padding_mask[b,j]                 (attention.py:185-188)
 *     h_i = sum_j alpha_ij m_ij v^_j      (no normaliser)      (attention.py:192-193)
 *     y_i = tanh(n_i)/n_i h_i, n_i = max(|h_i|, eps)           (norm.py:23-25)
 *
 * Tensor conventions
 *   q,k,v   : raw projections viewed as (B, T, H, D) with element strides
 *             (sb, st, sh) and unit stride over D -- exactly the
 *             proj(x).view(B,T,H,D) view the reference builds before its
 *             transpose (attention.py:150-153).  Strides and base pointers
 *             must allow 16-byte vector loads (strides multiple of 8 elements
 *             for bf16 and fp16, of 4 for fp32).
 *   y, dy, dq, dk, dv : contiguous (B, T, H, D), i.e. the (B,T,d_model) layout
 *             out_proj consumes (attention.py:198-200).
 *   r, w    : fp32 (H,), r = exp(s_r)+1, w = exp(s_v)+1 (attention.py:164-165).
 *             Precondition r >= 1 (which r = exp(s_r)+1 always meets): padded
 *             and masked keys enter with s = 0, which gives alpha = 0 only
 *             when r >= 1.  A window that is NaN or not positive is treated as
 *             empty (zero output for that head; the reference gives NaN).
 *   key_padding_mask : nullable uint8 (B, Tk), nonzero = ignore key.
 *   dtype   : MSA_F32, MSA_BF16 or MSA_F16 for q,k,v,y,dy,dq,dk,dv (the
 *             reference's fused forward takes float16 or float32 operands,
 *             screening_fwd.py:235; torch.autocast("cuda") gives float16).
 *             bf16 and fp16 run on the 32x32x16 MFMA with fp32 accumulation.
 *   dropout_p, dropout_seed : attention dropout on alpha*m (attention.py:68,
 *             :190, nn.Dropout in training mode), 0 <= p < 1; p = 0 is the
 *             identity.  The keep decision of pair (b, h, i, j) is a
 *             counter-based hash, so forward and backward agree without
 *             storing a mask: with key = (b*H+h) << 44 | i << 22 | j and
 *             z = dropout_seed + key * 0x9E3779B97F4A7C15 (mod 2^64), the
 *             SplitMix64 finaliser
 *               z = (z ^ z>>30) * 0xBF58476D1CE4E5B9
 *               z = (z ^ z>>27) * 0x94D049BB133111EB
 *               z =  z ^ z>>31
 *             keeps the pair iff (z >> 32) >= min(floor(p * 2^32), 2^32-1),
 *             and a kept pair is scaled by 1/(1-p) (fp32).  The reference
 *             draws its mask from torch's generator, so only the statistics
 *             match it (keep rate 1-p, unbiased in expectation).
 *
 * Ownership: the caller allocates every buffer (outputs and workspaces); the
 * library never allocates or frees device memory.  Every call is
 * stream-ordered on `stream` and does not synchronise the host.
 * Errors: a nonzero return code; msa_last_error() gives a thread-local
 * description.  Argument validation runs on the host before any HIP call.
 */
#ifndef MSA_H
#define MSA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum msa_dtype { MSA_F32 = 0, MSA_BF16 = 1, MSA_F16 = 2 };

enum msa_status {
  MSA_OK = 0,
  MSA_ERR_INVALID = 1,   /* bad shape / dtype / stride / pointer / size    */
  MSA_ERR_WORKSPACE = 2, /* workspace or bitmap buffer too small            */
  MSA_ERR_HIP = 3        /* a HIP runtime call or kernel launch failed      */
};

/* Library version, (major<<16)|(minor<<8)|patch.  0.2.0 inserted window_hint
 * before r in msa_decode / msa_decode_at (a binary built against 0.1.0 must
 * be rebuilt); 0.3.0 added MSA_F16. */
int msa_version(void);

/* Thread-local text of the last error raised on this thread ("" if none). */
const char* msa_last_error(void);

/* Bytes of forward workspace: scratch for one unit-normalised copy of K (key
 * padding applied, rows padded to a multiple of 64, head_dim padded to
 * 32/64/128) that the forward stages through LDS, and the screen's work plan.
 * Enough for a causal or a non-causal call of this shape.  Not needed
 * afterwards. */
size_t msa_fwd_workspace_bytes(int B, int H, int Tq, int Tk, int D, int dtype);

/* Number of uint32 words of the live-unit bitmap: one bit per
 * (b, h, 32-query unit, 32-key unit), set for every unit in which some
 * in-window, unmasked pair has alpha > 0, and otherwise only for units with
 * such a pair whose s lies within the screen's slack below the threshold
 * 1 - 1/r (2^-11 + 1e-5 for bf16 and fp16 inputs, 2^-10 + 1e-5 for fp32:
 * the screen votes on fp16 operands); the live and backward passes give
 * those pairs alpha = 0 exactly.  With nqt = ceil(Tq/64), nkt = ceil(Tk/64), the
 * (b, h) block holds 2*nqt rows (query unit qu: queries 32qu .. 32qu+31) of
 * ceil(2*nkt/32) words; key unit ku is bit ku%32 of word ku/32 of the row. */
size_t msa_tile_bits_words(int B, int H, int Tq, int Tk);

/* Bytes of backward workspace: one (dr, dw) partial per (b, h, 32-query
 * unit), summed in a fixed order, plus dh = TanhNorm'(h)^T dy and 1/|q| per
 * query row (padded to 64 rows per tile), which the dQ pass hands to the
 * dK/dV pass. */
size_t msa_bwd_workspace_bytes(int B, int H, int Tq, int Tk, int D, int dtype);

/*
 * Fused forward.  Replaces, as one call, what the reference's fused boundary
 * does across torch and Triton:
 *   F.normalize x3        attention_triton.py:115-117
 *   _ScreeningFunc.forward / screening_attention_fwd
 *                         attention_triton.py:31-36, screening_fwd.py:216-270
 *   TanhNorm + merge      attention_triton.py:135-137
 * and adds key_padding_mask (attention.py:185-188) and attention dropout
 * (attention.py:190), which the Triton path ignores (attention_triton.py:125-132).
 * Outputs: y (B,Tq,H,D) = TanhNorm(h); hnorm (B,H,Tq) fp32 = |h_i| before the
 * eps clamp (needed by msa_bwd); tile_bits (msa_tile_bits_words words).
 */
int msa_fwd(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
            const void* k, int64_t k_sb, int64_t k_st, int64_t k_sh,
            const void* v, int64_t v_sb, int64_t v_st, int64_t v_sh,
            int B, int H, int Tq, int Tk, int D, int dtype,
            const float* r, const float* w, const uint8_t* key_padding_mask,
            int causal, float eps, float dropout_p, uint64_t dropout_seed,
            void* y, float* hnorm, uint32_t* tile_bits, size_t tile_bits_words,
            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Fused backward.  Replaces _ScreeningFunc.backward / screening_attention_bwd
 * (attention_triton.py:38-44, screening_bwd.py:229-287) together with the
 * torch autograd of F.normalize and TanhNorm around it, and -- unlike the
 * reference fused path, which returns None for them (attention_triton.py:44)
 * -- produces the per-head gradients dr, dw (H,) that attention.py's autograd
 * delivers to s_r / s_v through r = exp(s_r)+1, w = exp(s_v)+1.
 * Inputs: the forward's q, k, v, r, w, key_padding_mask, causal, eps,
 * dropout_p, dropout_seed and its outputs y, hnorm, tile_bits; dy (B,Tq,H,D)
 * contiguous.
 * dq (B,Tq,H,D), dk, dv (B,Tk,H,D) are written in full (zeros where no
 * active pair reaches a row).  Deterministic: no atomics.
 */
int msa_bwd(const void* q, int64_t q_sb, int64_t q_st, int64_t q_sh,
            const void* k, int64_t k_sb, int64_t k_st, int64_t k_sh,
            const void* v, int64_t v_sb, int64_t v_st, int64_t v_sh,
            int B, int H, int Tq, int Tk, int D, int dtype,
            const float* r, const float* w, const uint8_t* key_padding_mask,
            int causal, float eps, float dropout_p, uint64_t dropout_seed,
            const void* y, const float* hnorm, const void* dy,
            const uint32_t* tile_bits, size_t tile_bits_words,
            void* dq, void* dk, void* dv, float* dr, float* dw,
            void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of decode workspace (split-key partial sums). */
size_t msa_decode_workspace_bytes(int B, int H, int D, int max_len);

/*
 * Single-query decode against a KV cache.  The reference has no KV cache: its
 * MultiscreenLM.generate re-runs the full forward over the prefix for every
 * token and keeps only the last row (model.py:111-141).  This computes that
 * last row directly: the query at position pos = cache_len-1 attends to the
 * causal window (pos - w, pos] of the cache, which already holds the new
 * token's k and v.
 *   q      : (B, H, D) raw query projection, strides (q_sb, q_sh), unit D.
 *   kcache, vcache : (B, Tcap, H, D) raw k/v projections, strides (sb, st, sh);
 *            cache_cap = Tcap, and 1 <= cache_len <= cache_cap.
 *   window_hint : 0, or a bound on ceil(w_h) over the heads that sizes the
 *            launch (one block per 2048-key chunk of each window; one block
 *            per head and no workspace traffic when the windows fit one
 *            chunk).  Only the windowed keys are visited whatever its value,
 *            and every launch shape gives bitwise the same y: a wrong hint
 *            costs time, never correctness.
 *   y      : (B, H, D) contiguous, TanhNorm(h).
 */
int msa_decode(const void* q, int64_t q_sb, int64_t q_sh,
               const void* kcache, int64_t k_sb, int64_t k_st, int64_t k_sh,
               const void* vcache, int64_t v_sb, int64_t v_st, int64_t v_sh,
               int B, int H, int D, int dtype, int cache_len, int cache_cap, int window_hint,
               const float* r, const float* w, float eps,
               void* y, void* workspace, size_t workspace_bytes, void* stream);

/*
 * msa_decode with the cache length read on the device: last_pos points to
 * the int64 position of the newest key (the query's), so the length is
 * *last_pos + 1, clamped to [1, cache_cap].  No counterpart in the reference
 * (its generate has no cache, model.py:111-141): it is for a decode step
 * captured once in a HIP graph and replayed as the sequence grows, the
 * position advanced on the device.  Workspace: msa_decode_workspace_bytes(B,
 * H, D, cache_cap).  Otherwise the same arguments, checks and results as
 * msa_decode.
 */
int msa_decode_at(const void* q, int64_t q_sb, int64_t q_sh,
                  const void* kcache, int64_t k_sb, int64_t k_st, int64_t k_sh,
                  const void* vcache, int64_t v_sb, int64_t v_st, int64_t v_sh,
                  int B, int H, int D, int dtype, const int64_t* last_pos, int cache_cap, int window_hint,
                  const float* r, const float* w, float eps,
                  void* y, void* workspace, size_t workspace_bytes, void* stream);

/*
 * msa_decode without a workspace argument and without any allocation: the
 * split-key partial sums go to a static device array of
 * MSA_DECODE_STATIC_SCRATCH_BYTES per GPU, held until the process ends.  No
 * counterpart in the reference: it is for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, checks and results as msa_decode; it
 * fails with MSA_ERR_WORKSPACE when msa_decode_workspace_bytes(B, H, D,
 * cache_len) exceeds the array (B*H*ceil(cache_len/2048)*D*4 bytes: e.g.
 * B*H = 128 heads of D = 64 up to cache_len 1,048,576).  Every call on a GPU
 * shares that GPU's array, so calls that overlap on one GPU (several streams
 * or threads) race; calls ordered on one stream do not.
 */
#define MSA_DECODE_STATIC_SCRATCH_BYTES (16u << 20)
int msa_decode_noalloc(const void* q, int64_t q_sb, int64_t q_sh,
                       const void* kcache, int64_t k_sb, int64_t k_st, int64_t k_sh,
                       const void* vcache, int64_t v_sb, int64_t v_st, int64_t v_sh,
                       int B, int H, int D, int dtype, int cache_len, int cache_cap, int window_hint,
                       const float* r, const float* w, float eps, void* y, void* stream);

/* Kernel timing for measurement.  After msa_timer_arm(kernel, n) the next n
 * launches of that kernel (any entry point) each record a HIP event pair on
 * their stream around the launch; several kernels can be armed at once.
 * msa_timer_read(kernel, ...) waits for that kernel's recorded pairs and
 * writes their durations in milliseconds, returning how many were recorded
 * (-1 on error).  msa_timer_arm(0, 0) disarms every kernel.  Process-wide; not
 * for concurrent use from several threads.
 * msa_timer_arm_every(kernel, n, every) records launches 0, every, 2*every, ...
 * of that kernel (n pairs): a timed loop then carries the event markers on
 * one launch in `every` only (each recorded pair adds a few microseconds of
 * stream time).  Measurement helpers: no counterpart in the reference. */
enum msa_kernel_id {
  MSA_K_PREP_K = 1, MSA_K_FWD_SCREEN = 2, MSA_K_FWD_LIVE = 3, MSA_K_DKDV = 4,
  MSA_K_DQ = 5, /* 6: unused (no separate dr/dw reduction launch) */ MSA_K_DECODE = 7
};
int msa_timer_arm(int kernel, int n);
int msa_timer_arm_every(int kernel, int n, int every);
int msa_timer_read(int kernel, float* ms, int n);

/* Device self-test of the MFMA operand layouts the kernels assume: writes the
 * 32x32 products A.B (bf16 32x32x16 and fp32 32x32x2 forms) of the given
 * row-major fp32 inputs a (32xK) and b (Kx32), K=16 and K=2, to out16, out2
 * (each 32x32 fp32, row-major).  Test infrastructure only. */
int msa_selftest_mfma(const float* a16, const float* b16, float* out16,
                      const float* a2, const float* b2, float* out2,
                      void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MSA_H */
