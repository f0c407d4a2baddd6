/*
 * mi_attn.h -- C ABI of the MI355X (gfx950) flash-attention library
 * (libmi_attn.so). This is the drop-in boundary below nanolab's
 * `flash_cuda` Python op: everything above it is Python, everything below it
 * is hand-written HIP for CDNA4.
 *
 * Layout (all contiguous, row-major, no padding):
 *   q, o, dout, dq : [B, S, H,   D]   element type `dtype`
 *   k, v, dk, dv   : [B, S, Hkv, D]   element type `dtype`
 *   lse, dlse      : [B, H, S]        float32, natural-log logsumexp
 *   delta          : float32 backward workspace of mi_attn_bwd_workspace()
 *                    floats, 16-byte aligned. Its head is [2, B, H, S],
 *                    written by mi_attn_bwd_delta: plane 0 is
 *                    Delta = sum_d dout*o - dlse, plane 1 is -lse / scale.
 *                    With float32 sinks, mi_attn_bwd_dkdv keeps per-chunk
 *                    partial sums of the sink keys' dk / dv after the two
 *                    planes; for small 16-bit GQA grids it writes fp32 dk /
 *                    dv partials of one query head each there instead (see
 *                    mi_attn_bwd_workspace).
 * GQA is native: query head h reads KV head h / (H / Hkv); dk/dv are summed
 * over the group inside the dK/dV kernel, or, when the 16-bit dK/dV splits
 * the group across workgroups, by a reduce kernel that adds the heads'
 * partials in head order (no atomics either way -- results are bitwise
 * reproducible run to run).
 *
 * Masking: key j is visible to query i iff j < S and
 *   (causal == 0 || j / L <= i / L) with L = max(block, 1), and
 *   (window <= 0 || j > i - (window - sinks) || j < sinks).
 * block > 1 is the block-causal (semi-autoregressive) mask of
 * nanolab/mixers.py:76-93: bidirectional inside a block of `block` positions,
 * causal across blocks; it needs causal != 0 and window == 0. block <= 1 is
 * plain causal.
 * window > 0 requires causal != 0 (the sliding window is causal-only); it is
 * SWA(window, sinks) of nanolab/mixers.py:96-135: the window - sinks most
 * recent keys (self included) plus the first `sinks` keys (StreamingLLM
 * attention sinks), 0 <= sinks < window; sinks > 0 requires window > 0.
 *
 * Conventions shared by every entry point:
 *   - the caller owns and allocates every buffer (inputs are never written);
 *   - work is enqueued on `stream` and nothing synchronises the host;
 *   - the return value is 0 on success, otherwise an MI_ERR_* code whose text
 *     mi_attn_error_string() returns. Argument checks run before any HIP call,
 *     so an invalid call touches no device state;
 *   - B == 0 or S == 0 or H == 0 is valid and launches nothing.
 *
 * Reference interfaces replaced (paths relative to bharathvbcr/MachineLearning):
 *   mi_attn_fwd       <- nanolab/csrc/flash_attn_cuda.cu:1654-1704  flash_attn_fwd  (pybind `fwd`, cu:1815-1825)
 *   mi_attn_bwd       <- nanolab/csrc/flash_attn_cuda.cu:1743-1813  flash_attn_bwd  (pybind `bwd`)
 *   mi_attn_bwd_delta <- nanolab/csrc/flash_attn_cuda.cu:1231-1262  flash_delta_kernel (first bwd launch, cu:1554-1587)
 *   mi_attn_bwd_dkdv  <- nanolab/csrc/flash_attn_cuda.cu:973-1191   flash_bwd_dkv_mma_kernel launch
 *   mi_attn_bwd_dq    <- nanolab/csrc/flash_attn_cuda.cu:799-971    flash_bwd_dq_mma_kernel launch
 *   mi_mfma_probe     <- nanolab/csrc/flash_attn_cuda.cu:1706-1741  mma_probe (pybind `mma_probe`)
 *   mi_attn_check     <- nanolab/csrc/flash_attn_cuda.cu:1628-1650  check_layout
 *   mi_attn_error_string <- the TORCH_CHECK messages of the same file
 */
#ifndef MI_ATTN_H
#define MI_ATTN_H

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MI_ATTN_ABI_VERSION 10

#if defined(__GNUC__)
#define MI_API __attribute__((visibility("default")))
#else
#define MI_API
#endif

typedef enum {
  MI_F32 = 0,
  MI_F16 = 1,
  MI_BF16 = 2
} mi_dtype;

typedef enum {
  MI_OK = 0,
  MI_ERR_NULL = 1,          /* a required pointer is NULL */
  MI_ERR_SHAPE = 2,         /* negative size, or H not a positive multiple of Hkv */
  MI_ERR_DTYPE = 3,         /* dtype not one of mi_dtype */
  MI_ERR_HEAD_DIM = 4,      /* D not in {32, 64, 128} */
  MI_ERR_WINDOW = 5,        /* bad mask: window < 0, window without causal, not 0 <= sinks < window,
                               block < 0, or block > 1 without causal or with a window */
  MI_ERR_ALIGN = 6,         /* a tensor pointer is not 16-byte aligned */
  MI_ERR_SIZE = 7,          /* an index would overflow the kernels' 32/64-bit math */
  MI_ERR_LAUNCH = 8,        /* hipLaunchKernel / hipGetLastError reported an error */
  MI_ERR_SCALE = 9,         /* scale is not finite, or not > 0 */
  MI_ERR_SCRATCH = 10,      /* mi_attn_bwd_noalloc: the shape needs more than
                               MI_ATTN_NOALLOC_SCRATCH_FLOATS of workspace */
  MI_ERR_HIP = 11,          /* a HIP runtime query failed (current device, scratch address) */
  MI_ERR_RESIDUAL = 12      /* mi_attn_fwd_res / mi_attn_bwd_res: the output residual needs
                               16-bit inputs */
} mi_status;

/* Size in floats of the static device array behind mi_attn_bwd_noalloc (16 MiB
 * per GPU the library runs on, held until the process ends). */
#define MI_ATTN_NOALLOC_SCRATCH_FLOATS (4LL << 20)

typedef struct {
  int B, S, H, Hkv, D;
  int causal;   /* 0 / 1 */
  int window;   /* 0 = no window; > 0 = each query sees at most this many keys (self included) */
  float scale;  /* softmax scale applied to q.k, finite and > 0 (nanolab default 1/sqrt(D)) */
  int dtype;    /* mi_dtype of q/k/v/o/dout/dq/dk/dv */
  int sinks;    /* attention sinks inside the window: 0 <= sinks < window (0 without a window) */
  int block;    /* causal block length: 0 or 1 = plain causal, > 1 = block-causal */
} mi_attn_shape;

/* Validate a shape without launching anything. Replaces check_layout
 * (nanolab/csrc/flash_attn_cuda.cu:1628-1650). */
MI_API int mi_attn_check(const mi_attn_shape* s);

/* Size in floats of the backward workspace `delta` for shape `s`: 2*B*H*S,
 * plus, for float32 with sinks that some query sees beyond its window span,
 * the sink pass's partial sums (16-bit kernels visit the sinks themselves),
 * plus, for a 16-bit GQA shape whose dK/dV grid of (batch, kv head, 128-key block) workgroups
 * fills the GPU less than twice (the current device's CUs x 2 workgroups at
 * D <= 64, x 1 at D = 128), fp32 dK/dV partials of one query head per
 * workgroup (B*H*ceil(S/128)*128*2*D floats, from a 64-float boundary), as
 * long as those partials take at most 16M floats (64 MiB); larger shapes run
 * the unsplit kernel. Query it on the device the backward will run on.
 * No counterpart in the reference, whose backward allocates its Delta buffer
 * inside flash_attn_bwd (nanolab/csrc/flash_attn_cuda.cu:1743-1813); here the
 * caller owns it. */
MI_API int mi_attn_bwd_workspace(const mi_attn_shape* s, long long* floats);

/* Forward: o = softmax(scale * q k^T + mask) v, lse = logsumexp(...) (natural log).
 * Replaces flash_attn_fwd (nanolab/csrc/flash_attn_cuda.cu:1654-1704). */
MI_API int mi_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                const mi_attn_shape* s, hipStream_t stream);

/* Full backward on one stream. 16-bit inputs: dQ (which also fills the
 * workspace's [Delta | -lse/scale] planes), then dK/dV; float32: the delta
 * pass, then dK/dV, then dQ. Either way the workspace ends up as
 * mi_attn_bwd_delta leaves it.
 * `dlse` is the incoming gradient of lse (may be NULL = zero); `delta` is the
 * caller-owned workspace (mi_attn_bwd_workspace() floats, 16-byte aligned).
 * Replaces flash_attn_bwd (nanolab/csrc/flash_attn_cuda.cu:1743-1813). */
MI_API int mi_attn_bwd(const void* q, const void* k, const void* v, const void* o,
                const void* dout, const float* lse, const float* dlse, float* delta,
                void* dq, void* dk, void* dv, const mi_attn_shape* s, hipStream_t stream);

/* mi_attn_fwd that also writes o_res, the rounding residual of o: o_res =
 * (o_exact - o) rounded to `dtype`, in o's layout, so that o + o_res carries
 * the output to about 16 significant bits. 16-bit dtypes only;
 * MI_ERR_RESIDUAL otherwise. o itself is bitwise what mi_attn_fwd writes.
 * Extends flash_attn_fwd (nanolab/csrc/flash_attn_cuda.cu:1654-1704), which
 * returns the rounded output only. */
MI_API int mi_attn_fwd_res(const void* q, const void* k, const void* v, void* o, void* o_res,
                           float* lse, const mi_attn_shape* s, hipStream_t stream);

/* mi_attn_bwd whose delta pass reads o + o_res (o_res from mi_attn_fwd_res)
 * instead of the rounded o alone: Delta = rowsum(dout * O) to about 16 bits.
 * Each row's Delta enters every dS of that row, so with the 8-bit rounding of
 * a bf16 o it bounds the gradients' accuracy on long rows (S = 8192, D = 128:
 * dK off by up to 3e-2). Same conditions as mi_attn_fwd_res.
 * Extends flash_attn_bwd (nanolab/csrc/flash_attn_cuda.cu:1743-1813), whose
 * delta kernel reads the rounded output (cu:1231-1262). */
MI_API int mi_attn_bwd_res(const void* q, const void* k, const void* v, const void* o,
                           const void* o_res, const void* dout, const float* lse,
                           const float* dlse, float* delta, void* dq, void* dk, void* dv,
                           const mi_attn_shape* s, hipStream_t stream);

/* mi_attn_bwd without the caller's workspace, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving and
 * training loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The workspace lives in a static device array of
 * MI_ATTN_NOALLOC_SCRATCH_FLOATS floats per GPU; a shape whose workspace
 * without the GQA dK/dV split partials exceeds it returns MI_ERR_SCRATCH
 * before any launch (the board shape needs 0.39M floats, every BASELINE shape
 * at most 1.05M). A GQA shape whose split partials (counted in
 * mi_attn_bwd_workspace()) do not fit runs the unsplit dK/dV kernel instead.
 * Allocates nothing: no hipMalloc / hipFree, no library allocation. Every call
 * on one GPU shares that GPU's array, which keeps the last call's contents
 * (every entry a call reads is written by the same call first), so calls
 * that overlap on one GPU (other streams, other host threads) race; serialise
 * them. The device current on the calling thread selects the array; its
 * address is looked up once per device (hipGetSymbolAddress) on the first
 * call, which may load the library's code object: make one eager call per
 * device before capturing a graph that contains this entry point (the
 * lookup is not a capturable operation). Results are
 * bitwise those of mi_attn_bwd, except for that unsplit case: dK / dV then
 * sum the GQA group in another float32 order (dQ stays bitwise; dK / dV
 * agree to float32 rounding of the sum). */
MI_API int mi_attn_bwd_noalloc(const void* q, const void* k, const void* v, const void* o,
                               const void* dout, const float* lse, const float* dlse, void* dq,
                               void* dk, void* dv, const mi_attn_shape* s, hipStream_t stream);

/* Gated attention: the output is y = sigmoid(gate) * softmax(...) v per query
 * row, the per-head output gate of nanolab's gated attention
 * (nanolab/mixers.py:340-344, y * sigmoid(gate(x))) applied on O inside the
 * kernel. `gate` holds the gate logits [B, S, H] float32; lse is that of the
 * ungated attention. No counterpart in the reference's extension, whose
 * output is ungated (the mixer applies the gate afterwards). */
MI_API int mi_attn_fwd_gated(const void* q, const void* k, const void* v, const float* gate,
                             void* o, float* lse, const mi_attn_shape* s, hipStream_t stream);

/* Backward of mi_attn_fwd_gated: `o` is its gated output, `dout` the gradient
 * of that output. `dout_attn` is a caller-owned [B,S,H,D] buffer of `dtype`
 * (16-byte aligned) that receives sigmoid(gate) * dout, the attention output's
 * gradient, which the dK/dV and dQ passes read; `dgate` [B,S,H] float32
 * receives the gate logits' gradient (1 - sigmoid) * rowsum(dout * o). */
MI_API int mi_attn_bwd_gated(const void* q, const void* k, const void* v, const float* gate,
                             const void* o, const void* dout, const float* lse,
                             const float* dlse, float* delta, void* dout_attn, void* dq,
                             void* dk, void* dv, float* dgate, const mi_attn_shape* s,
                             hipStream_t stream);

/* Stage 1 of the gated backward: mi_attn_bwd_delta plus dout_attn and dgate
 * (as above). Stages 2 and 3 are then mi_attn_bwd_dkdv / mi_attn_bwd_dq with
 * dout_attn in place of dout. */
MI_API int mi_attn_bwd_delta_gated(const void* o, const void* dout, const float* gate,
                                   const float* lse, const float* dlse, float* delta,
                                   void* dout_attn, float* dgate, const mi_attn_shape* s,
                                   hipStream_t stream);

/* Stage 1 of the backward: fills the [2,B,H,S] head of the workspace `delta`:
 * delta[0][b,h,i] = sum_d dout*o - dlse (dlse may be NULL) and
 * delta[1][b,h,i] = -lse[b,h,i] / scale.
 * Replaces flash_delta_kernel's launch (nanolab/csrc/flash_attn_cuda.cu:1231-1262). */
MI_API int mi_attn_bwd_delta(const void* o, const void* dout, const float* lse, const float* dlse,
                      float* delta, const mi_attn_shape* s, hipStream_t stream);

/* Stage 2: dk, dv over query tiles; `delta` is the workspace
 * mi_attn_bwd_delta filled, mi_attn_bwd_workspace() floats. The stage writes
 * into it beyond the two planes, so it must be writable (it is `const` for
 * the planes only): with float32 sinks, the sink keys' per-chunk partials;
 * for a small 16-bit GQA grid, the split partials of each query head, which a
 * reduce kernel then sums over the group in head order (otherwise the group
 * is summed in-kernel).
 * Replaces flash_bwd_dkv_mma_kernel's launch (nanolab/csrc/flash_attn_cuda.cu:973-1191). */
MI_API int mi_attn_bwd_dkdv(const void* q, const void* k, const void* v, const void* dout,
                     const float* lse, const float* delta, void* dk, void* dv,
                     const mi_attn_shape* s, hipStream_t stream);

/* Stage 3: dq over key tiles; `delta` as for stage 2.
 * Replaces flash_bwd_dq_mma_kernel's launch (nanolab/csrc/flash_attn_cuda.cu:799-971). */
MI_API int mi_attn_bwd_dq(const void* q, const void* k, const void* v, const void* dout,
                   const float* lse, const float* delta, void* dq,
                   const mi_attn_shape* s, hipStream_t stream);

/* One 32x32 MFMA tile through the kernels' own fragment helpers:
 * d[32][32] = a[32][Kp] @ b[Kp][32] (row-major), Kp = 16 for f16/bf16 and 2 for f32.
 * The host compares d with a plain matmul before trusting the layout table.
 * Replaces mma_probe (nanolab/csrc/flash_attn_cuda.cu:1706-1741). */
MI_API int mi_mfma_probe(const void* a, const void* b, float* d, int dtype, hipStream_t stream);

/* ------------------------------------------------------------------------
 * Fused attention prologue: RMSNorm of each head row (QK-norm) then rotary
 * position embedding, the q / k path of nanolab's attention block
 * (nanolab/mixers.py:282-292: q_norm / k_norm = RMSNorm, mixers.py:46-56;
 * apply_rope, mixers.py:68-75). No counterpart in the reference's extension:
 * it replaces that chain of torch ops (and the autocast bridge's cast of its
 * fp32 result) with one pass that writes the attention kernel's input.
 *
 *   x, dx     : [B, T, H, D]  dtype_in
 *   out, dout : [B, T, H, D]  dtype_out
 *   weight    : [D] float32 (used when norm != 0), dweight : [D] float32
 *   cos, sin  : [T, D] float32, row t for sequence position t (rope != 0)
 *   rstd      : [B, T, H] float32, 1/sqrt(mean(x^2) + eps) (written by the
 *               forward when not NULL; read by the backward when norm != 0)
 * ------------------------------------------------------------------------ */
typedef struct {
  int B, T, H, D;  /* D in {32, 64, 128} */
  int dtype_in;    /* mi_dtype of x and dx */
  int dtype_out;   /* mi_dtype of out and dout */
  int norm;        /* 1: RMSNorm with weight, 0: none */
  int rope;        /* 1: rotate by cos / sin, 0: none */
  float eps;       /* RMSNorm epsilon, finite and >= 0 (nanolab: 1e-6) */
} mi_prologue_shape;

/* out = rope(rms_norm(x) * weight). */
MI_API int mi_qk_prologue_fwd(const void* x, const float* weight, const float* cos,
                              const float* sin, void* out, float* rstd,
                              const mi_prologue_shape* s, hipStream_t stream);

/* Floats of the workspace mi_qk_prologue_bwd needs (weight-gradient partials). */
MI_API int mi_qk_prologue_workspace(const mi_prologue_shape* s, long long* floats);

/* dx and dweight (dweight written only when norm != 0, and not at all for an
 * empty input: its gradient is zero) for the incoming gradient dout of out;
 * `workspace` holds mi_qk_prologue_workspace() floats.
 * The weight gradient is summed in a fixed order: bitwise reproducible. */
MI_API int mi_qk_prologue_bwd(const void* dout, const void* x, const float* weight,
                              const float* cos, const float* sin, const float* rstd, void* dx,
                              float* dweight, float* workspace, const mi_prologue_shape* s,
                              hipStream_t stream);

/* ------------------------------------------------------------------------
 * KV-cached attention for incremental decoding: the attention section of
 * nanolab's Attention.forward_cached (nanolab/mixers.py:401-462), where the
 * reference concatenates the cache with the active block's K / V
 * (torch.cat, mixers.py:404-405) and calls SDPA with an explicit mask
 * (mixers.py:407-433, 457-458). No counterpart in the reference's extension.
 * Nothing is concatenated here: the kernels read the cache and the block in
 * place.
 *
 *   q, out           : [B, T, H, D]    the T active queries (dtype)
 *   k_new, v_new     : [B, T, Hkv, D]  the active block's keys / values
 *   k_cache, v_cache : row j of (batch b, kv head h) at element
 *                      b * *_batch_stride + h * *_head_stride + j * D: the
 *                      reference's (B, Hkv, L, D) cache or a view of a larger
 *                      buffer (rows D apart, 16-byte aligned)
 *   cache_pos        : int64 [cached], absolute positions of the cached rows
 *                      (NULL: 0 .. cached-1); read only with a window
 *   gate             : float32 [B, T, H] output gate logits (NULL: none);
 *                      out = softmax(.) V * sigmoid(gate)
 *   lse              : float32 [B, H, T] log-sum-exp of the scaled scores
 *                      (NULL: not written)
 *   workspace        : mi_attn_decode_workspace() floats (NULL when 0)
 * Mask. Query t is at position start + t, and so is key cached + t:
 *   causal = 0: every key (a bidirectional block: block-diffusion drafts);
 *   causal = 1: keys at positions <= the query's (the whole cache, the block
 *               lower-triangular; a self-speculation verify);
 *   window w > 0 (needs causal), sinks s: also position > query - (w - s) or
 *               position < s (mixers.py:423-428). Without a window, positions
 *               are the row indices and `start` is ignored.
 * The cached rows must sit at positions before `start` (the reference's cache
 * holds strictly earlier tokens). GQA: query head h reads kv head h / (H/Hkv).
 * ------------------------------------------------------------------------ */
typedef struct {
  int B, T, H, Hkv, D;  /* D in {32, 64, 128}; H a positive multiple of Hkv */
  int cached;           /* rows in the cache, >= 0 */
  int start;            /* absolute position of active query 0 (window > 0) */
  int causal;           /* 1: causal inside the block; 0: bidirectional */
  int window, sinks;    /* sliding window and its sinks, as in mi_attn_shape */
  float scale;          /* softmax scale, finite and > 0 */
  int dtype;            /* mi_dtype of q, k/v (cache and new) and out */
  long long k_batch_stride, k_head_stride;   /* cache strides in elements */
  long long v_batch_stride, v_head_stride;
} mi_decode_shape;

/* Floats of split-partial workspace mi_attn_decode needs for this shape
 * (0: none; the step then writes its output directly). */
MI_API int mi_attn_decode_workspace(const mi_decode_shape* s, long long* floats);

/* One decode step: out (and lse) for the active queries. Split over the keys
 * and merged in a fixed order: bitwise reproducible. */
MI_API int mi_attn_decode(const void* q, const void* k_new, const void* v_new,
                          const void* k_cache, const void* v_cache, const long long* cache_pos,
                          const float* gate, void* out, float* lse, float* workspace,
                          const mi_decode_shape* s, hipStream_t stream);

/* The K extent mi_mfma_probe expects for `dtype` (16 or 2), or -1. */
MI_API int mi_mfma_probe_k(int dtype);

/* Static text for a status code; never NULL. */
MI_API const char* mi_attn_error_string(int status);

/* MI_ATTN_ABI_VERSION of the loaded library. */
MI_API int mi_attn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* MI_ATTN_H */
