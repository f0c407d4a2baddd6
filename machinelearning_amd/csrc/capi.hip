// extern "C" entry points of libmi_attn.so (declared in include/mi_attn.h):
// argument validation, parameter packing and dispatch to the HIP launchers,
// plus the MFMA layout probe. Validation runs before any HIP call, so an
// invalid call never touches the device.
#include <math.h>
#include <stdint.h>

#include <atomic>
#include <mutex>

#include "../../include/mi_attn.h"
#include "attn_common.h"

namespace mi {
hipError_t launch_fwd(int dtype, int D, const void* q, const void* k, const void* v, void* o,
                      float* lse, const AttnParams& p, hipStream_t st);
hipError_t launch_fwd16(int dtype, int D, const void* q, const void* k, const void* v, void* o,
                        float* lse, const AttnParams& p, hipStream_t st);
hipError_t launch_bwd_delta(int dtype, int D, const void* o, const void* dout, const float* lse,
                            const float* dlse, float* ws, void* doe, float* dz,
                            const AttnParams& p, hipStream_t st);
hipError_t launch_bwd_dkdv(int dtype, int D, const void* q, const void* k, const void* v,
                           const void* dout, const float* lse, const float* delta, void* dk,
                           void* dv, const AttnParams& p, hipStream_t st);
hipError_t launch_bwd_dq(int dtype, int D, const void* q, const void* k, const void* v,
                         const void* dout, const float* lse, const float* delta, void* dq,
                         const AttnParams& p, hipStream_t st);
hipError_t launch_bwd16_dkdv(int dtype, int D, const void* q, const void* k, const void* v,
                             const void* dout, const float* lse, const float* delta, void* dk,
                             void* dv, const AttnParams& p, hipStream_t st);
hipError_t launch_bwd16_dq(int dtype, int D, const void* q, const void* k, const void* v,
                           const void* dout, const float* lse, const float* delta, void* dq,
                           const AttnParams& p, hipStream_t st);
hipError_t launch_sink_fwd(int dtype, int D, const void* q, const void* k, const void* v, void* o,
                           float* lse, const AttnParams& p, hipStream_t st);
hipError_t launch_sink_dq(int dtype, int D, const void* q, const void* k, const void* v,
                          const void* dout, const float* lse, const float* delta, void* dq,
                          const AttnParams& p, hipStream_t st);
hipError_t launch_sink_dkv(int dtype, int D, const void* q, const void* k, const void* v,
                           const void* dout, const float* lse, const float* delta, float* part,
                           void* dk, void* dv, void* dq, const AttnParams& p, hipStream_t st);
bool sink_bwd_fusable(const AttnParams& p);
long long sink_workspace_floats(const AttnParams& p, int D);
int dkdv16_split(const AttnParams& p, int D);
long long dkdv16_split_floats(const AttnParams& p, int D);

void prologue_chunks(ProParams& p, int D, int dtype_in);
hipError_t launch_decode(int dtype, const void* q, const void* kc, const void* vc, const void* kn,
                         const void* vn, void* out, float* lse, float* ws, const DecParams& p,
                         hipStream_t st);
long long decode_workspace_floats(int dtype, const DecParams& p);
hipError_t launch_prologue_fwd(int dtype_in, int dtype_out, int D, const void* x, const float* w,
                               const float* cs, const float* sn, void* out, float* rstd,
                               const ProParams& p, hipStream_t st);
hipError_t launch_prologue_bwd(int dtype_in, int dtype_out, int D, const void* g, const void* x,
                               const float* w, const float* cs, const float* sn,
                               const float* rstd, void* dx, float* dw, float* part,
                               const ProParams& p, hipStream_t st);

// One 32x32 MFMA through the same fragment helpers the attention kernels use:
// A row l32 / B column l32 with k-slots [g*EPL, g*EPL+EPL), accumulator
// register r at row crow(r, g). a: [32][KPI], b: [KPI][32], d: [32][32].
template <typename T>
__global__ void __launch_bounds__(64)
mfma_probe_kernel(const T* __restrict__ a, const T* __restrict__ b, float* __restrict__ d) {
  using M = Mfma32<T>;
  constexpr int EPL = M::EPL, KPI = 2 * EPL;
  const int lane = threadIdx.x, l32 = lane & 31, g = lane >> 5;
  typename M::frag af, bf;
  if constexpr (EPL == 1) {
    af = a[l32 * KPI + g];
    bf = b[g * 32 + l32];
  } else {
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      af[e] = a[l32 * KPI + g * EPL + e];
      bf[e] = b[(g * EPL + e) * 32 + l32];
    }
  }
  const f32x16 acc = M::mma(af, bf, zero16());
#pragma unroll
  for (int r = 0; r < 16; ++r) d[crow(r, g) * 32 + l32] = acc[r];
}
}  // namespace mi

namespace {

int validate(const mi_attn_shape* s) {
  if (!s) return MI_ERR_NULL;
  if (s->B < 0 || s->S < 0 || s->H < 0 || s->Hkv < 0) return MI_ERR_SHAPE;
  if (s->dtype != MI_F32 && s->dtype != MI_F16 && s->dtype != MI_BF16) return MI_ERR_DTYPE;
  if (s->D != 32 && s->D != 64 && s->D != 128) return MI_ERR_HEAD_DIM;
  if (s->Hkv <= 0 || s->H % s->Hkv != 0) {
    // an empty problem may carry H == 0; anything else needs a positive group
    if (!(s->H == 0 && s->Hkv >= 0)) return MI_ERR_SHAPE;
  }
  if (s->window < 0 || (s->window > 0 && !s->causal)) return MI_ERR_WINDOW;
  if (s->sinks < 0 || (s->sinks > 0 && s->sinks >= s->window)) return MI_ERR_WINDOW;
  // Block-causal is causal at block granularity; like the reference, it does not
  // combine with a sliding window (nanolab/mixers.py:300-304).
  if (s->block < 0 || (s->block > 1 && (!s->causal || s->window > 0))) return MI_ERR_WINDOW;
  // The kernels take the running max over raw scores, which is the max of
  // the scaled scores only for scale > 0; the Python layer maps scale <= 0
  // onto this contract exactly (q -> -q, or q -> 0 for scale == 0).
  if (!isfinite(s->scale) || !(s->scale > 0.f)) return MI_ERR_SCALE;
  // Grid sizes and per-(b,h) row indices are 32-bit in the kernels.
  const long long bh = (long long)s->B * (s->H > s->Hkv ? s->H : s->Hkv);
  if (bh * ((s->S + 31) / 32) > 0x7fffffffLL) return MI_ERR_SIZE;
  if ((long long)s->S * s->H * s->D > 0x7fffffffLL) return MI_ERR_SIZE;
  // The sink kernels index workgroups of >= 16 rows of one (b, head) in 32 bits.
  if (s->sinks > 0 && bh * ((s->S + 15) / 16) > 0x7fffffffLL) return MI_ERR_SIZE;
  return MI_OK;
}

bool empty(const mi_attn_shape* s) { return s->B == 0 || s->S == 0 || s->H == 0; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

mi::AttnParams params(const mi_attn_shape* s) {
  mi::AttnParams p;
  p.B = s->B;
  p.S = s->S;
  p.H = s->H;
  p.Hkv = s->Hkv;
  p.group = s->Hkv > 0 ? s->H / s->Hkv : 1;
  p.causal = s->causal ? 1 : 0;
  p.block = s->block > 1 ? s->block : 1;
  // The window kernels take the local span; the sink kernels add the rest.
  p.window = s->window > 0 ? s->window - s->sinks : 0;
  p.sinks = s->window > 0 ? s->sinks : 0;
  // The 16-bit window kernels visit the sinks themselves (their first key
  // tiles, before the window ring); fp32 takes the separate sink kernels,
  // whose chunked partial sums keep a sink key's long dK / dV column inside
  // fp32's bound. A span that covers the whole sequence leaves no sink pair to
  // add: the window kernels then run exactly the causal case. No query sees a
  // sink past key S - span - 1 (query i sees j < i - span + 1 <= S - span),
  // so the folded count stops there.
  const int sink_cap = s->S - p.window;
  p.fold_sinks = (s->dtype != MI_F32 && p.window < s->S) ? (p.sinks < sink_cap ? p.sinks : sink_cap) : 0;
  p.scale = s->scale;
  p.scale_log2 = s->scale * mi::kLog2e;
  p.resc_th = 8.f / p.scale_log2;   // scale > 0 is validated; may be +inf for tiny scales
  p.nblk = 0;
  p.div_h = mi::fast_div((unsigned)p.H);
  p.div_hkv = mi::fast_div((unsigned)p.Hkv);
  p.div_group = mi::fast_div((unsigned)p.group);
  p.div_wi = mi::fast_div(1);   // set by each launcher for its grid
  p.wi_blocks_fastest = 0;
  p.q_rs = (long long)s->H * s->D;
  p.kv_rs = (long long)s->Hkv * s->D;
  p.gate = nullptr;
  p.o = nullptr;
  p.dlse = nullptr;
  p.ws_out = nullptr;
  p.kv_split = 1;
  p.kv_part = nullptr;
  p.o_res = nullptr;
  return p;
}

int status_of(hipError_t e) { return e == hipSuccess ? MI_OK : MI_ERR_LAUNCH; }

// The sink pass keeps its per-chunk partial sums after the workspace's two planes.
float* sink_part(const float* delta, const mi_attn_shape* s) {
  return const_cast<float*>(delta) + 2LL * s->B * s->H * s->S;
}

// Workspace without the split dK/dV partials: the two planes and the sink partials.
long long base_workspace_floats(const mi_attn_shape* s) {
  return 2LL * s->B * s->H * s->S + (empty(s) ? 0 : mi::sink_workspace_floats(params(s), s->D));
}

// The split dK/dV partials (16-bit, GQA, small grids) follow, 256-byte aligned.
long long split_offset(const mi_attn_shape* s) { return (base_workspace_floats(s) + 63) / 64 * 64; }

long long split_floats(const mi_attn_shape* s) {
  if (s->dtype == MI_F32 || empty(s)) return 0;
  return mi::dkdv16_split_floats(params(s), s->D);
}

// Workspace floats of the full backward, with (allow_split) or without the
// split dK/dV partials.
long long workspace_floats(const mi_attn_shape* s, bool allow_split) {
  const long long part = allow_split ? split_floats(s) : 0;
  return part > 0 ? split_offset(s) + part : base_workspace_floats(s);
}

}  // namespace

extern "C" {

int mi_attn_abi_version(void) { return MI_ATTN_ABI_VERSION; }

const char* mi_attn_error_string(int status) {
  switch (status) {
    case MI_OK: return "ok";
    case MI_ERR_NULL: return "mi_attn: a required pointer is NULL";
    case MI_ERR_SHAPE:
      return "mi_attn: invalid shape (sizes must be >= 0 and n_head a positive multiple of n_kv_head)";
    case MI_ERR_DTYPE: return "mi_attn: dtype must be float32, float16 or bfloat16";
    case MI_ERR_HEAD_DIM: return "mi_attn: head_dim must be one of 32, 64, 128";
    case MI_ERR_WINDOW:
      return "mi_attn: window must be >= 0, a window needs causal attention, sinks must "
             "satisfy 0 <= sinks < window (sinks > 0 needs a window), and block > 1 needs "
             "causal attention without a window";
    case MI_ERR_ALIGN: return "mi_attn: every tensor must be 16-byte aligned";
    case MI_ERR_SIZE: return "mi_attn: problem too large for 32-bit grid / row indices";
    case MI_ERR_LAUNCH: return "mi_attn: HIP kernel launch failed";
    case MI_ERR_SCALE: return "mi_attn: scale must be finite and > 0";
    case MI_ERR_SCRATCH:
      return "mi_attn: mi_attn_bwd_noalloc: this shape needs more workspace than the static "
             "scratch array holds (MI_ATTN_NOALLOC_SCRATCH_FLOATS); use mi_attn_bwd with a "
             "caller-owned workspace";
    case MI_ERR_HIP: return "mi_attn: a HIP runtime query failed (current device / scratch address)";
    case MI_ERR_RESIDUAL:
      return "mi_attn: the output residual needs float16 / bfloat16 inputs";
  }
  return "mi_attn: unknown status";
}

int mi_attn_check(const mi_attn_shape* s) { return validate(s); }

int mi_attn_bwd_workspace(const mi_attn_shape* s, long long* floats) {
  if (!floats) return MI_ERR_NULL;
  const int st = validate(s);
  if (st) return st;
  *floats = workspace_floats(s, true);
  return MI_OK;
}

}  // extern "C"

namespace {

// The output residual is written by the 16-bit forward kernel itself (which
// also visits any sinks), so it needs 16-bit inputs.
bool residual_ok(const mi_attn_shape* s) { return s->dtype != MI_F32; }

// Forward with an optional output gate (gate logits [B,S,H] fp32, or nullptr)
// and an optional output residual (o_res, O's layout and dtype, or nullptr).
int run_fwd(const void* q, const void* k, const void* v, const float* gate, void* o, float* lse,
            const mi_attn_shape* s, hipStream_t stream, void* o_res = nullptr) {
  const int st = validate(s);
  if (st) return st;
  if (o_res && !residual_ok(s)) return MI_ERR_RESIDUAL;
  if (empty(s)) return MI_OK;
  if (!q || !k || !v || !o || !lse) return MI_ERR_NULL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) ||
      (o_res && !aligned16(o_res)))
    return MI_ERR_ALIGN;
  mi::AttnParams p = params(s);
  p.gate = gate;
  p.o_res = o_res;
  const hipError_t e = s->dtype == MI_F32
                           ? mi::launch_fwd(s->dtype, s->D, q, k, v, o, lse, p, stream)
                           : mi::launch_fwd16(s->dtype, s->D, q, k, v, o, lse, p, stream);
  if (e != hipSuccess) return MI_ERR_LAUNCH;
  return status_of(mi::launch_sink_fwd(s->dtype, s->D, q, k, v, o, lse, p, stream));
}

// Stage 1 of the backward; with a gate it also writes doe = sigma * dout and
// dgate.
int run_delta(const void* o, const void* dout, const float* gate, const float* lse,
              const float* dlse, float* delta, void* doe, float* dgate, const mi_attn_shape* s,
              hipStream_t stream) {
  const int st = validate(s);
  if (st) return st;
  if (empty(s)) return MI_OK;
  if (!o || !dout || !lse || !delta || (gate && (!doe || !dgate))) return MI_ERR_NULL;
  if (!aligned16(o) || !aligned16(dout) || !aligned16(delta) || (doe && !aligned16(doe)))
    return MI_ERR_ALIGN;
  mi::AttnParams p = params(s);
  p.gate = gate;
  return status_of(mi::launch_bwd_delta(s->dtype, s->D, o, dout, lse, dlse, delta,
                                        gate ? doe : nullptr, gate ? dgate : nullptr, p, stream));
}

}  // namespace

extern "C" {

int mi_attn_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                const mi_attn_shape* s, hipStream_t stream) {
  return run_fwd(q, k, v, nullptr, o, lse, s, stream);
}

int mi_attn_fwd_res(const void* q, const void* k, const void* v, void* o, void* o_res,
                    float* lse, const mi_attn_shape* s, hipStream_t stream) {
  if (!o_res) return MI_ERR_NULL;
  return run_fwd(q, k, v, nullptr, o, lse, s, stream, o_res);
}

int mi_attn_fwd_gated(const void* q, const void* k, const void* v, const float* gate, void* o,
                      float* lse, const mi_attn_shape* s, hipStream_t stream) {
  if (!gate) return MI_ERR_NULL;
  return run_fwd(q, k, v, gate, o, lse, s, stream);
}

int mi_attn_bwd_delta(const void* o, const void* dout, const float* lse, const float* dlse,
                      float* delta, const mi_attn_shape* s, hipStream_t stream) {
  return run_delta(o, dout, nullptr, lse, dlse, delta, nullptr, nullptr, s, stream);
}

int mi_attn_bwd_delta_gated(const void* o, const void* dout, const float* gate, const float* lse,
                            const float* dlse, float* delta, void* dout_attn, float* dgate,
                            const mi_attn_shape* s, hipStream_t stream) {
  if (!gate) return MI_ERR_NULL;
  return run_delta(o, dout, gate, lse, dlse, delta, dout_attn, dgate, s, stream);
}

}  // extern "C"

namespace {

// Which sink passes a backward stage runs: its own (the stage entry points),
// none, or the full backward's fused one (dQ and dK/dV shares in one walk).
enum class SinkPass { kOwn, kNone };

// allow_split: the workspace holds workspace_floats(s, true) floats, so the
// 16-bit dK/dV may split the GQA group (otherwise it runs unsplit).
int run_dkdv(const void* q, const void* k, const void* v, const void* dout, const float* lse,
             const float* delta, void* dk, void* dv, const mi_attn_shape* s,
             hipStream_t stream, SinkPass sp, bool allow_split = true) {
  if (!q || !k || !v || !dout || !lse || !delta || !dk || !dv) return MI_ERR_NULL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dout) || !aligned16(dk) ||
      !aligned16(dv) || !aligned16(delta))
    return MI_ERR_ALIGN;
  mi::AttnParams p = params(s);
  if (allow_split && split_floats(s) > 0) {
    p.kv_split = mi::dkdv16_split(p, s->D);
    p.kv_part = const_cast<float*>(delta) + split_offset(s);
  }
  const hipError_t e =
      s->dtype == MI_F32
          ? mi::launch_bwd_dkdv(s->dtype, s->D, q, k, v, dout, lse, delta, dk, dv, p, stream)
          : mi::launch_bwd16_dkdv(s->dtype, s->D, q, k, v, dout, lse, delta, dk, dv, p, stream);
  if (e != hipSuccess) return MI_ERR_LAUNCH;
  if (sp == SinkPass::kNone) return MI_OK;
  return status_of(mi::launch_sink_dkv(s->dtype, s->D, q, k, v, dout, lse, delta,
                                       sink_part(delta, s), dk, dv, nullptr, p, stream));
}

// With `o` set (16-bit inputs only), the dQ kernel also computes the delta
// pass and writes both workspace planes (`delta`), from o and dlse.
int run_dq(const void* q, const void* k, const void* v, const void* dout, const float* lse,
           const float* delta, void* dq, const mi_attn_shape* s, hipStream_t stream,
           SinkPass sp, const void* o = nullptr, const float* dlse = nullptr,
           const void* o_res = nullptr) {
  if (!q || !k || !v || !dout || !lse || !delta || !dq) return MI_ERR_NULL;
  if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dout) || !aligned16(dq) ||
      (o && !aligned16(o)))
    return MI_ERR_ALIGN;
  mi::AttnParams p = params(s);
  if (o) {
    p.o = o;
    p.dlse = dlse;
    p.ws_out = const_cast<float*>(delta);
    p.o_res = const_cast<void*>(o_res);
  }
  const hipError_t e =
      s->dtype == MI_F32
          ? mi::launch_bwd_dq(s->dtype, s->D, q, k, v, dout, lse, delta, dq, p, stream)
          : mi::launch_bwd16_dq(s->dtype, s->D, q, k, v, dout, lse, delta, dq, p, stream);
  if (e != hipSuccess) return MI_ERR_LAUNCH;
  if (sp == SinkPass::kNone) return MI_OK;
  return status_of(mi::launch_sink_dq(s->dtype, s->D, q, k, v, dout, lse, delta, dq, p, stream));
}

}  // namespace

extern "C" {

int mi_attn_bwd_dkdv(const void* q, const void* k, const void* v, const void* dout,
                     const float* lse, const float* delta, void* dk, void* dv,
                     const mi_attn_shape* s, hipStream_t stream) {
  const int st = validate(s);
  if (st) return st;
  if (empty(s)) return MI_OK;
  return run_dkdv(q, k, v, dout, lse, delta, dk, dv, s, stream, SinkPass::kOwn);
}

int mi_attn_bwd_dq(const void* q, const void* k, const void* v, const void* dout,
                   const float* lse, const float* delta, void* dq, const mi_attn_shape* s,
                   hipStream_t stream) {
  const int st = validate(s);
  if (st) return st;
  if (empty(s)) return MI_OK;
  return run_dq(q, k, v, dout, lse, delta, dq, s, stream, SinkPass::kOwn);
}

}  // extern "C"

namespace {

// The full backward; with a gate, stage 1 writes the gate-scaled output
// gradient into dout_attn and the later passes read that instead of dout.
int run_bwd(const void* q, const void* k, const void* v, const float* gate, const void* o,
            const void* dout, const float* lse, const float* dlse, float* delta, void* dout_attn,
            void* dq, void* dk, void* dv, float* dgate, const mi_attn_shape* s,
            hipStream_t stream, bool allow_split = true, const void* o_res = nullptr) {
  const int st = validate(s);
  if (st) return st;
  if (o_res && (gate || !residual_ok(s))) return MI_ERR_RESIDUAL;
  if (empty(s)) return MI_OK;
  if (o_res && !aligned16(o_res)) return MI_ERR_ALIGN;
  if (!q || !k || !v || !o || !dout || !lse || !delta || !dq || !dk || !dv) return MI_ERR_NULL;
  const mi::AttnParams p = params(s);
  if (!gate && s->dtype != MI_F32) {
    // 16-bit, no gate: the dQ kernel computes the delta pass itself and runs
    // first; dK/dV (and the sink pass) then read the planes it wrote.
    if (!aligned16(o) || !aligned16(delta)) return MI_ERR_ALIGN;
    if (!mi::sink_bwd_fusable(p)) {
      int r = run_dq(q, k, v, dout, lse, delta, dq, s, stream, SinkPass::kOwn, o, dlse, o_res);
      if (r) return r;
      return run_dkdv(q, k, v, dout, lse, delta, dk, dv, s, stream, SinkPass::kOwn, allow_split);
    }
    int r = run_dq(q, k, v, dout, lse, delta, dq, s, stream, SinkPass::kNone, o, dlse, o_res);
    if (r) return r;
    r = run_dkdv(q, k, v, dout, lse, delta, dk, dv, s, stream, SinkPass::kNone, allow_split);
    if (r) return r;
    return status_of(mi::launch_sink_dkv(s->dtype, s->D, q, k, v, dout, lse, delta,
                                         sink_part(delta, s), dk, dv, dq, p, stream));
  }
  int r = run_delta(o, dout, gate, lse, dlse, delta, dout_attn, dgate, s, stream);
  if (r) return r;
  const void* g = gate ? dout_attn : dout;
  if (!mi::sink_bwd_fusable(p)) {
    r = run_dkdv(q, k, v, g, lse, delta, dk, dv, s, stream, SinkPass::kOwn, allow_split);
    if (r) return r;
    return run_dq(q, k, v, g, lse, delta, dq, s, stream, SinkPass::kOwn);
  }
  // Window kernels first, then one pass adds the sinks' share of dQ, dK, dV.
  r = run_dkdv(q, k, v, g, lse, delta, dk, dv, s, stream, SinkPass::kNone, allow_split);
  if (r) return r;
  r = run_dq(q, k, v, g, lse, delta, dq, s, stream, SinkPass::kNone);
  if (r) return r;
  return status_of(mi::launch_sink_dkv(s->dtype, s->D, q, k, v, g, lse, delta,
                                       sink_part(delta, s), dk, dv, dq, p, stream));
}

}  // namespace

extern "C" {

int mi_attn_bwd(const void* q, const void* k, const void* v, const void* o, const void* dout,
                const float* lse, const float* dlse, float* delta, void* dq, void* dk, void* dv,
                const mi_attn_shape* s, hipStream_t stream) {
  return run_bwd(q, k, v, nullptr, o, dout, lse, dlse, delta, nullptr, dq, dk, dv, nullptr, s,
                 stream);
}

int mi_attn_bwd_res(const void* q, const void* k, const void* v, const void* o,
                    const void* o_res, const void* dout, const float* lse, const float* dlse,
                    float* delta, void* dq, void* dk, void* dv, const mi_attn_shape* s,
                    hipStream_t stream) {
  if (!o_res) return MI_ERR_NULL;
  return run_bwd(q, k, v, nullptr, o, dout, lse, dlse, delta, nullptr, dq, dk, dv, nullptr, s,
                 stream, true, o_res);
}

}  // extern "C"

namespace {

// Workspace of mi_attn_bwd_noalloc: one static array per GPU (each device
// holds its own copy of a __device__ variable). Host code never uses the
// array's name as an address: scratch_base() looks up the current device's
// address of the array once (hipGetSymbolAddress, with that device current)
// and every launch gets that pointer.
__device__ __align__(256) float scratch[MI_ATTN_NOALLOC_SCRATCH_FLOATS];

constexpr int kMaxScratchDevices = 64;
std::atomic<float*> g_scratch_base[kMaxScratchDevices];
std::mutex g_scratch_mu;

int scratch_base(float** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxScratchDevices) return MI_ERR_HIP;
  float* base = g_scratch_base[dev].load(std::memory_order_acquire);
  if (!base) {
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    base = g_scratch_base[dev].load(std::memory_order_relaxed);
    if (!base) {
      void* addr = nullptr;
      if (hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch)) != hipSuccess || !addr)
        return MI_ERR_HIP;
      base = static_cast<float*>(addr);
      g_scratch_base[dev].store(base, std::memory_order_release);
    }
  }
  *out = base;
  return MI_OK;
}

}  // namespace

extern "C" {

int mi_attn_bwd_noalloc(const void* q, const void* k, const void* v, const void* o,
                        const void* dout, const float* lse, const float* dlse, void* dq,
                        void* dk, void* dv, const mi_attn_shape* s, hipStream_t stream) {
  const int st = validate(s);
  if (st) return st;
  if (empty(s)) return MI_OK;
  // The split dK/dV partials are used when they fit; the unsplit kernel otherwise.
  const bool split = workspace_floats(s, true) <= MI_ATTN_NOALLOC_SCRATCH_FLOATS;
  if (workspace_floats(s, false) > MI_ATTN_NOALLOC_SCRATCH_FLOATS) return MI_ERR_SCRATCH;
  float* ws = nullptr;
  const int r = scratch_base(&ws);
  if (r) return r;
  return run_bwd(q, k, v, nullptr, o, dout, lse, dlse, ws, nullptr, dq, dk, dv, nullptr, s,
                 stream, split);
}

int mi_attn_bwd_gated(const void* q, const void* k, const void* v, const float* gate,
                      const void* o, const void* dout, const float* lse, const float* dlse,
                      float* delta, void* dout_attn, void* dq, void* dk, void* dv, float* dgate,
                      const mi_attn_shape* s, hipStream_t stream) {
  if (!gate || !dout_attn || !dgate) return MI_ERR_NULL;
  return run_bwd(q, k, v, gate, o, dout, lse, dlse, delta, dout_attn, dq, dk, dv, dgate, s,
                 stream);
}

namespace {

int validate_pro(const mi_prologue_shape* s) {
  if (!s) return MI_ERR_NULL;
  if (s->B < 0 || s->T < 0 || s->H < 0) return MI_ERR_SHAPE;
  for (int dt : {s->dtype_in, s->dtype_out})
    if (dt != MI_F32 && dt != MI_F16 && dt != MI_BF16) return MI_ERR_DTYPE;
  if (s->D != 32 && s->D != 64 && s->D != 128) return MI_ERR_HEAD_DIM;
  if (!isfinite(s->eps) || s->eps < 0.f) return MI_ERR_SCALE;
  if ((long long)s->B * s->T * s->H * s->D > 0x7fffffffLL) return MI_ERR_SIZE;
  return MI_OK;
}

mi::ProParams pro_params(const mi_prologue_shape* s) {
  mi::ProParams p;
  p.rows = s->B * s->T * s->H;
  p.T = s->T;
  p.H = s->H;
  p.norm = s->norm ? 1 : 0;
  p.rope = s->rope ? 1 : 0;
  p.eps = s->eps;
  p.nchunk = 0;
  p.chunk_rows = 0;
  if (p.rows > 0) mi::prologue_chunks(p, s->D, s->dtype_in);
  return p;
}

}  // namespace

int mi_qk_prologue_fwd(const void* x, const float* weight, const float* cos, const float* sin,
                       void* out, float* rstd, const mi_prologue_shape* s, hipStream_t stream) {
  const int st = validate_pro(s);
  if (st) return st;
  if ((long long)s->B * s->T * s->H == 0) return MI_OK;
  if (!x || !out || (s->norm && !weight) || (s->rope && (!cos || !sin))) return MI_ERR_NULL;
  if (!aligned16(x) || !aligned16(out) || (weight && !aligned16(weight)) ||
      (cos && !aligned16(cos)) || (sin && !aligned16(sin)))
    return MI_ERR_ALIGN;
  return status_of(mi::launch_prologue_fwd(s->dtype_in, s->dtype_out, s->D, x, weight, cos, sin,
                                           out, rstd, pro_params(s), stream));
}

int mi_qk_prologue_workspace(const mi_prologue_shape* s, long long* floats) {
  if (!floats) return MI_ERR_NULL;
  const int st = validate_pro(s);
  if (st) return st;
  const mi::ProParams p = pro_params(s);
  *floats = p.rows > 0 && p.norm ? (long long)p.nchunk * s->D : 0;
  return MI_OK;
}

int mi_qk_prologue_bwd(const void* dout, const void* x, const float* weight, const float* cos,
                       const float* sin, const float* rstd, void* dx, float* dweight,
                       float* workspace, const mi_prologue_shape* s, hipStream_t stream) {
  const int st = validate_pro(s);
  if (st) return st;
  if ((long long)s->B * s->T * s->H == 0) return MI_OK;   // nothing written, dweight included
  if (!dout || !dx || (s->rope && (!cos || !sin)) ||
      (s->norm && (!x || !weight || !rstd || !dweight || !workspace)))
    return MI_ERR_NULL;
  if (!aligned16(dout) || !aligned16(dx) || (x && !aligned16(x)) ||
      (weight && !aligned16(weight)) || (cos && !aligned16(cos)) || (sin && !aligned16(sin)))
    return MI_ERR_ALIGN;
  return status_of(mi::launch_prologue_bwd(s->dtype_in, s->dtype_out, s->D, dout, x, weight, cos,
                                           sin, rstd, dx, dweight, workspace, pro_params(s),
                                           stream));
}

namespace {

int validate_dec(const mi_decode_shape* s) {
  if (!s) return MI_ERR_NULL;
  if (s->B < 0 || s->T < 0 || s->H < 0 || s->Hkv < 0 || s->cached < 0) return MI_ERR_SHAPE;
  if (s->dtype != MI_F32 && s->dtype != MI_F16 && s->dtype != MI_BF16) return MI_ERR_DTYPE;
  if (s->D != 32 && s->D != 64 && s->D != 128) return MI_ERR_HEAD_DIM;
  if (s->Hkv <= 0 || s->H % s->Hkv != 0) {
    if (!(s->H == 0 && s->Hkv >= 0)) return MI_ERR_SHAPE;
  }
  if (s->window < 0 || (s->window > 0 && !s->causal)) return MI_ERR_WINDOW;
  if (s->sinks < 0 || (s->sinks > 0 && s->sinks >= s->window)) return MI_ERR_WINDOW;
  if (s->window > 0 && s->start < 0) return MI_ERR_SHAPE;
  if (!isfinite(s->scale) || !(s->scale > 0.f)) return MI_ERR_SCALE;
  // Cache rows must start 16-byte aligned: strides in whole 16-byte chunks.
  const long long chunk = s->dtype == MI_F32 ? 4 : 8;
  for (long long st : {s->k_batch_stride, s->k_head_stride, s->v_batch_stride, s->v_head_stride})
    if (st < 0 || st % chunk != 0) return MI_ERR_ALIGN;
  // Key indices, positions and grid dimensions are 32-bit in the kernels.
  if ((long long)s->cached + s->T > 0x7fffffffLL) return MI_ERR_SIZE;
  if ((long long)s->start + s->T > 0x7fffffffLL) return MI_ERR_SIZE;
  // Workgroups: one per (batch, kv head, tile of >= 8 query rows) and key split.
  if (s->Hkv > 0 &&
      (long long)s->B * s->Hkv * (((long long)s->T * (s->H / s->Hkv) + 7) / 8) > (1LL << 24))
    return MI_ERR_SIZE;
  return MI_OK;
}

mi::DecParams dec_params(const mi_decode_shape* s) {
  mi::DecParams p;
  p.B = s->B;
  p.T = s->T;
  p.H = s->H;
  p.Hkv = s->Hkv;
  p.rep = s->Hkv > 0 ? s->H / s->Hkv : 1;
  p.D = s->D;
  p.Lc = s->cached;
  p.Lk = s->cached + s->T;
  // Without a window the mask only needs row indices: positions = indices.
  p.start = s->window > 0 ? s->start : s->cached;
  p.causal = s->causal ? 1 : 0;
  p.window = s->window;
  p.sinks = s->window > 0 ? s->sinks : 0;
  p.span = s->window > 0 ? s->window - s->sinks : 0;
  p.scale = s->scale;
  p.scale_log2 = s->scale * mi::kLog2e;
  p.k_sb = s->k_batch_stride;
  p.k_sh = s->k_head_stride;
  p.v_sb = s->v_batch_stride;
  p.v_sh = s->v_head_stride;
  p.R = s->T * p.rep;
  p.RT = p.ntiles = p.nsplit = p.bps = 0;   // set by the launcher
  p.pos = nullptr;
  p.gate = nullptr;
  return p;
}

}  // namespace

int mi_attn_decode_workspace(const mi_decode_shape* s, long long* floats) {
  if (!floats) return MI_ERR_NULL;
  const int st = validate_dec(s);
  if (st) return st;
  const long long n = mi::decode_workspace_floats(s->dtype, dec_params(s));
  if (n < 0) return MI_ERR_SHAPE;
  *floats = n;
  return MI_OK;
}

int mi_attn_decode(const void* q, const void* k_new, const void* v_new, const void* k_cache,
                   const void* v_cache, const long long* cache_pos, const float* gate, void* out,
                   float* lse, float* workspace, const mi_decode_shape* s, hipStream_t stream) {
  const int st = validate_dec(s);
  if (st) return st;
  if (s->B == 0 || s->T == 0 || s->H == 0) return MI_OK;
  if (!q || !k_new || !v_new || !out || (s->cached > 0 && (!k_cache || !v_cache)))
    return MI_ERR_NULL;
  mi::DecParams p = dec_params(s);
  const long long ws = mi::decode_workspace_floats(s->dtype, p);
  if (ws > 0 && !workspace) return MI_ERR_NULL;
  if (!aligned16(q) || !aligned16(k_new) || !aligned16(v_new) || !aligned16(out) ||
      (k_cache && !aligned16(k_cache)) || (v_cache && !aligned16(v_cache)) ||
      (workspace && !aligned16(workspace)))
    return MI_ERR_ALIGN;
  if (s->window > 0 && s->cached > 0) p.pos = cache_pos;   // read only for cached rows
  p.gate = gate;
  return status_of(mi::launch_decode(s->dtype, q, k_cache, v_cache, k_new, v_new, out, lse,
                                     workspace, p, stream));
}

int mi_mfma_probe_k(int dtype) {
  switch (dtype) {
    case MI_F32: return 2;
    case MI_F16:
    case MI_BF16: return 16;
  }
  return -1;
}

int mi_mfma_probe(const void* a, const void* b, float* d, int dtype, hipStream_t stream) {
  if (!a || !b || !d) return MI_ERR_NULL;
  switch (dtype) {
    case MI_F32:
      hipLaunchKernelGGL(mi::mfma_probe_kernel<float>, dim3(1), dim3(64), 0, stream,
                         (const float*)a, (const float*)b, d);
      break;
    case MI_F16:
      hipLaunchKernelGGL(mi::mfma_probe_kernel<_Float16>, dim3(1), dim3(64), 0, stream,
                         (const _Float16*)a, (const _Float16*)b, d);
      break;
    case MI_BF16:
      hipLaunchKernelGGL(mi::mfma_probe_kernel<__bf16>, dim3(1), dim3(64), 0, stream,
                         (const __bf16*)a, (const __bf16*)b, d);
      break;
    default:
      return MI_ERR_DTYPE;
  }
  return status_of(hipGetLastError());
}

}  // extern "C"
