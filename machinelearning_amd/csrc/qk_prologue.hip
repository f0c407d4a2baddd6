// Fused attention prologue: RMSNorm over each head row (QK-norm) followed by
// rotary position embedding, the q / k path of nanolab's attention block
// (nanolab/mixers.py:282-292; RMSNorm mixers.py:46-56, apply_rope
// mixers.py:68-75). One pass reads x once and writes the rotated row once, in
// the attention kernel's input dtype, instead of the reference's chain of
// fp32 intermediates (rms_norm, x*cos, cat(-x2, x1), *sin, add, then the
// autocast bridge's cast).
//
//   forward : n = x * rstd, rstd = 1 / sqrt(mean(x^2) + eps)    (norm on)
//             y = n * w
//             out = y * cos[t] + rot(y) * sin[t], rot(y) = cat(-y2, y1)  (rope on)
//   backward: dy = g * cos + rot^T(g * sin), rot^T(u) = cat(u2, -u1)
//             dn = dy * w, dx = rstd * (dn - n * mean(dn * n))
//             dw = sum over rows of dy * n   (per workgroup partials, then a
//             fixed-order reduction: bitwise reproducible)
//
// Memory-bound: LPQ lanes share one row, each holding E consecutive elements
// (one 16-byte load of x); the RoPE partner element d +- D/2 sits LPQ/2 lanes
// away and comes over by a lane swap; row sums are DPP butterflies inside the
// lane group. Statistics and arithmetic are fp32.
#include "attn_common.h"

namespace mi {

namespace {

template <int D, typename Tin>
struct ProGeom {
  static constexpr int E = 16 / (int)sizeof(Tin);   // elements per lane
  static constexpr int LPQ = D / E;                  // lanes per row
  static constexpr int QPW = 64 / LPQ;               // rows per wave
  static constexpr int ROWS = 4 * QPW;               // rows per 256-thread block
};

template <typename T, int N>
__device__ __forceinline__ void pro_ld(float (&r)[N], const T* p) {
  typedef T vN __attribute__((ext_vector_type(N)));
  const vN x = *reinterpret_cast<const vN*>(p);
#pragma unroll
  for (int e = 0; e < N; ++e) r[e] = (float)x[e];
}

template <typename T, int N>
__device__ __forceinline__ void pro_st(T* p, const float (&r)[N]) {
  typedef T vN __attribute__((ext_vector_type(N)));
  vN x;
#pragma unroll
  for (int e = 0; e < N; ++e) x[e] = (T)r[e];
  *reinterpret_cast<vN*>(p) = x;
}

template <int CTRL>
__device__ __forceinline__ float pro_dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of LPQ lanes (quad_perm pairs, row_half_mirror,
// row_mirror: involutions, so both partners add the same two values).
template <int LPQ>
__device__ __forceinline__ float pro_sum(float x) {
  if constexpr (LPQ >= 2) x += pro_dpp<0xB1>(x);
  if constexpr (LPQ >= 4) x += pro_dpp<0x4E>(x);
  if constexpr (LPQ >= 8) x += pro_dpp<0x141>(x);
  if constexpr (LPQ >= 16) x += pro_dpp<0x140>(x);
  if constexpr (LPQ >= 32) x += __shfl_xor(x, 16);
  return x;
}

}  // namespace

// Rows per lane group and loop step, forward and backward: all loads of the
// U rows are issued before any arithmetic, so each lane keeps U x 16 bytes of
// its input (plus the rope rows) in flight. (Measured on the board-shape q:
// forward 10.7 vs 11.1 us with one row per step; the backward within noise.
// Four and eight rows per step, with as many times fewer workgroups, were
// slower: forward 11.8 / 13.4 us, backward 23.2 / 33.5 against 18.5 us.
// One position per lane group, its rope rows loaded once for the H heads,
// was slower: 11.5 us.)
constexpr int kProRows = 2;

template <typename Tin, typename Tout, int D>
__global__ void __launch_bounds__(256)
qk_prologue_fwd_kernel(const Tin* __restrict__ X, const float* __restrict__ W,
                       const float* __restrict__ Cs, const float* __restrict__ Sn,
                       Tout* __restrict__ Out, float* __restrict__ Rstd, ProParams p) {
  using G = ProGeom<D, Tin>;
  constexpr int E = G::E, HALF = G::LPQ / 2, U = kProRows;
  const int lane = threadIdx.x & 63, sub = lane % G::LPQ;
  const int d0 = sub * E;
  const bool lo = sub < HALF;                      // this lane holds d < D/2
  float w[E];
  if (p.norm) pro_ld<float, E>(w, W + d0);
  for (int blk = blockIdx.x; blk * G::ROWS * U < p.rows; blk += gridDim.x) {
    // Row u of this lane group: (blk * U + u) * ROWS + wave * QPW + lane / LPQ.
    int r[U];
    bool valid[U];
    float x[U][E], c[U][E], sn[U][E];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r0 = (blk * U + u) * G::ROWS + (threadIdx.x >> 6) * G::QPW + lane / G::LPQ;
      valid[u] = r0 < p.rows;
      r[u] = valid[u] ? r0 : p.rows - 1;
      pro_ld<Tin, E>(x[u], X + (long long)r[u] * D + d0);
      if (p.rope) {
        const int t = (r[u] / p.H) % p.T;
        pro_ld<float, E>(c[u], Cs + (long long)t * D + d0);
        pro_ld<float, E>(sn[u], Sn + (long long)t * D + d0);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float y[E];
      float rstd = 1.f;
      if (p.norm) {
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) ss = fmaf(x[u][e], x[u][e], ss);
        ss = pro_sum<G::LPQ>(ss);
        rstd = rsqrtf(ss * (1.f / D) + p.eps);
#pragma unroll
        for (int e = 0; e < E; ++e) y[e] = x[u][e] * rstd * w[e];
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) y[e] = x[u][e];
      }
      float o[E];
      if (p.rope) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          // rot(y)[d] = -y[d + D/2] (d < D/2), y[d - D/2] (d >= D/2)
          const float partner = __shfl_xor(y[e], HALF);
          const float ry = lo ? -partner : partner;
          o[e] = fmaf(y[e], c[u][e], ry * sn[u][e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = y[e];
      }
      if (valid[u]) {
        pro_st<Tout, E>(Out + (long long)r[u] * D + d0, o);
        if (sub == 0 && Rstd) Rstd[r[u]] = rstd;
      }
    }
  }
}

template <typename Tin, typename Tout, int D>
__global__ void __launch_bounds__(256)
qk_prologue_bwd_kernel(const Tout* __restrict__ Gr, const Tin* __restrict__ X,
                       const float* __restrict__ W, const float* __restrict__ Cs,
                       const float* __restrict__ Sn, const float* __restrict__ Rstd,
                       Tin* __restrict__ dX, float* __restrict__ part, ProParams p) {
  using G = ProGeom<D, Tin>;
  constexpr int E = G::E, HALF = G::LPQ / 2;
  __shared__ float red[4][D];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPQ, qg = lane / G::LPQ;
  const int d0 = sub * E;
  const bool lo = sub < HALF;
  float w[E];
  if (p.norm) pro_ld<float, E>(w, W + d0);
  const int c = blockIdx.x;                          // one chunk per workgroup
  const int r_lo = c * p.chunk_rows, r_hi = min(p.rows, r_lo + p.chunk_rows);
  float dw[E];
#pragma unroll
  for (int e = 0; e < E; ++e) dw[e] = 0.f;
  // Rows rb + u * ROWS + qg for u < U per step (the same row order as one
  // row per step, so dw sums in the same order), loads of all U rows first.
  constexpr int U = kProRows;
  for (int rb = r_lo + wave * G::QPW; rb < r_hi; rb += G::ROWS * U) {   // wave-uniform
    int r[U];
    bool valid[U];
    float g[U][E], cs[U][E], sn[U][E], xs[U][E], rstd[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int r0 = rb + u * G::ROWS + qg;
      valid[u] = r0 < r_hi;
      r[u] = valid[u] ? r0 : r_hi - 1;
      const long long off = (long long)r[u] * D + d0;
      pro_ld<Tout, E>(g[u], Gr + off);
      if (p.rope) {
        const int t = (r[u] / p.H) % p.T;
        pro_ld<float, E>(cs[u], Cs + (long long)t * D + d0);
        pro_ld<float, E>(sn[u], Sn + (long long)t * D + d0);
      }
      if (p.norm) {
        pro_ld<Tin, E>(xs[u], X + off);
        rstd[u] = Rstd[r[u]];
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float dy[E];
      if (p.rope) {
#pragma unroll
        for (int e = 0; e < E; ++e) {
          // rot^T(v)[d] = v[d + D/2] (d < D/2), -v[d - D/2] (d >= D/2), v = g * sin
          const float partner = __shfl_xor(g[u][e] * sn[u][e], HALF);
          dy[e] = fmaf(g[u][e], cs[u][e], lo ? partner : -partner);
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) dy[e] = g[u][e];
      }
      float dx[E];
      if (p.norm) {
        float n[E], dn[E], dot = 0.f;
#pragma unroll
        for (int e = 0; e < E; ++e) {
          n[e] = xs[u][e] * rstd[u];
          dn[e] = dy[e] * w[e];
          dot = fmaf(dn[e], n[e], dot);
        }
        dot = pro_sum<G::LPQ>(dot) * (1.f / D);
#pragma unroll
        for (int e = 0; e < E; ++e) {
          dx[e] = rstd[u] * (dn[e] - n[e] * dot);
          if (valid[u]) dw[e] = fmaf(dy[e], n[e], dw[e]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; ++e) dx[e] = dy[e];
      }
      if (valid[u]) pro_st<Tin, E>(dX + (long long)r[u] * D + d0, dx);
    }
  }
  if (!p.norm) return;                               // block-uniform
  // dw: sum the wave's row groups (butterfly), then the four waves in order.
#pragma unroll
  for (int off = G::LPQ; off < 64; off <<= 1) {
#pragma unroll
    for (int e = 0; e < E; ++e) dw[e] += __shfl_xor(dw[e], off);
  }
  if (qg == 0) {
#pragma unroll
    for (int e = 0; e < E; ++e) red[wave][d0 + e] = dw[e];
  }
  __syncthreads();
  for (int d = threadIdx.x; d < D; d += 256)
    part[(long long)c * D + d] = ((red[0][d] + red[1][d]) + red[2][d]) + red[3][d];
}

// dweight[d] = sum over chunks of part[c][d]: workgroup d, thread i sums the
// chunks c = i, i + 256, ... in order, then a fixed-shape LDS tree adds the
// 256 subtotals (the same order every run).
template <int D>
__global__ void __launch_bounds__(256)
qk_prologue_dw_kernel(const float* __restrict__ part, float* __restrict__ dW, int nchunk) {
  __shared__ float t[256];
  const int d = blockIdx.x, i = threadIdx.x;
  float s = 0.f;
  for (int c = i; c < nchunk; c += 256) s += part[(long long)c * D + d];
  t[i] = s;
  __syncthreads();
#pragma unroll
  for (int w = 128; w >= 1; w >>= 1) {
    if (i < w) t[i] += t[i + w];
    __syncthreads();
  }
  if (i == 0) dW[d] = t[0];
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
namespace {

constexpr int kProPartBlocks = 1024;   // workgroups of the backward (weight-gradient partials)

template <typename T> struct ProT { using type = T; };

template <typename F>
hipError_t pro_dispatch(int dtype_in, int dtype_out, int D, F&& f) {
  auto by_d = [&](auto ti, auto to) -> hipError_t {
    switch (D) {
      case 32: return f(ti, to, std::integral_constant<int, 32>{});
      case 64: return f(ti, to, std::integral_constant<int, 64>{});
      case 128: return f(ti, to, std::integral_constant<int, 128>{});
    }
    return hipErrorInvalidValue;
  };
  auto by_out = [&](auto ti) -> hipError_t {
    switch (dtype_out) {
      case 0: return by_d(ti, ProT<float>{});
      case 1: return by_d(ti, ProT<_Float16>{});
      case 2: return by_d(ti, ProT<__bf16>{});
    }
    return hipErrorInvalidValue;
  };
  switch (dtype_in) {
    case 0: return by_out(ProT<float>{});
    case 1: return by_out(ProT<_Float16>{});
    case 2: return by_out(ProT<__bf16>{});
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Chunks of the backward: about kProPartBlocks workgroups of whole 256-thread steps.
void prologue_chunks(ProParams& p, int D, int dtype_in) {
  const int E = dtype_in == 0 ? 4 : 8;
  const int step = 4 * (64 / (D / E));
  const int steps = (p.rows + step - 1) / step;
  const int per = (steps + kProPartBlocks - 1) / kProPartBlocks;
  p.chunk_rows = per * step;
  p.nchunk = (p.rows + p.chunk_rows - 1) / p.chunk_rows;
}

hipError_t launch_prologue_fwd(int dtype_in, int dtype_out, int D, const void* x, const float* w,
                               const float* cs, const float* sn, void* out, float* rstd,
                               const ProParams& p, hipStream_t st) {
  return pro_dispatch(dtype_in, dtype_out, D, [&](auto ti, auto to, auto dd) -> hipError_t {
    using Tin = typename decltype(ti)::type;
    using Tout = typename decltype(to)::type;
    constexpr int DD = decltype(dd)::value;
    const int rows_per_blk = ProGeom<DD, Tin>::ROWS * kProRows;
    const int nblk = (p.rows + rows_per_blk - 1) / rows_per_blk;
    const unsigned grid = (unsigned)min(nblk, 1 << 20);
    hipLaunchKernelGGL((qk_prologue_fwd_kernel<Tin, Tout, DD>), dim3(grid), dim3(256), 0, st,
                       (const Tin*)x, w, cs, sn, (Tout*)out, rstd, p);
    return hipGetLastError();
  });
}

// `part` holds p.nchunk * D floats (the caller's workspace).
hipError_t launch_prologue_bwd(int dtype_in, int dtype_out, int D, const void* g, const void* x,
                               const float* w, const float* cs, const float* sn,
                               const float* rstd, void* dx, float* dw, float* part,
                               const ProParams& p, hipStream_t st) {
  return pro_dispatch(dtype_in, dtype_out, D, [&](auto ti, auto to, auto dd) -> hipError_t {
    using Tin = typename decltype(ti)::type;
    using Tout = typename decltype(to)::type;
    constexpr int DD = decltype(dd)::value;
    hipLaunchKernelGGL((qk_prologue_bwd_kernel<Tin, Tout, DD>), dim3((unsigned)p.nchunk),
                       dim3(256), 0, st, (const Tout*)g, (const Tin*)x, w, cs, sn, rstd,
                       (Tin*)dx, part, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !p.norm) return e;
    hipLaunchKernelGGL((qk_prologue_dw_kernel<DD>), dim3(DD), dim3(256), 0, st,
                       (const float*)part, dw, p.nchunk);
    return hipGetLastError();
  });
}

}  // namespace mi
