// StreamingLLM attention sinks for the sliding-window path. SWA(w, s) of
// nanolab/mixers.py:96-135 (and its chunked twin swa_chunked, mixers.py:168-200)
// lets query i see the keys j <= i with j > i - (w - s) -- the local span --
// and, besides, the first s keys of the sequence (the sinks).
//
// The window kernels run with window = span and compute everything the span
// covers. The pairs (i, j) with j < s and j <= i - span (sinks the span does
// not already cover: j < n_i = min(s, i - span + 1)) are added here. Only the
// rows i >= span have such pairs, so every kernel below walks those rows only.
//
//  * forward: attn_sink_fwd_kernel attends query i to its extra sink keys and
//    merges that partial result into the span's (O, LSE) in place by the
//    log-sum-exp combination;
//  * backward: fed the merged LSE and Delta, the window kernels already
//    produce exactly the span pairs' share of every gradient, since P and dS
//    are elementwise in (L, Delta). attn_sink_dq_kernel adds the sink pairs'
//    share of dQ row by row. dK / dV of a sink key sum over all its rows:
//    attn_sink_dkv_part_kernel sums one chunk of rows per workgroup into a
//    partial in the backward workspace, attn_sink_dkv_reduce_kernel adds the
//    partials to dK / dV in a fixed order (no atomics: bitwise reproducible).
//
// This is memory-bound VALU work (a row meets at most s extra keys). LPQ
// lanes share one row, each holding 16 bytes of it (EPL consecutive
// elements, one dwordx4 load), and every lane group carries U rows whose
// loads are all issued before any arithmetic. Dot products are reduced across
// the group's lanes by a butterfly, which leaves the identical sum in every
// lane of the group. A workgroup covers rows of one (b, head) -- or one
// (b, kv head) for dK / dV -- so the sink keys' K and V rows are staged once
// in LDS as fp32 (kSinkStage keys at a time) and read from there.
#include "attn_common.h"

namespace mi {

namespace {

template <typename T, int D>
struct SinkGeom {
  static constexpr int EPL = 16 / (int)sizeof(T);  // elements per lane: 8 (16-bit), 4 (fp32)
  static constexpr int LPQ = D / EPL;               // lanes per row
  static constexpr int QPW = 64 / LPQ;              // rows per wave and step
  static constexpr int U = 2;                       // rows per lane group
  static constexpr int ROWS = 4 * QPW * U;          // rows per 256-thread workgroup
};

constexpr int kSinkChunk = 4;    // sinks per softmax / accumulation pass
constexpr int kSinkStage = 32;   // sink keys staged in LDS at a time

template <typename T, int N>
__device__ __forceinline__ void ldv(float (&r)[N], const T* p) {
  typedef T vN __attribute__((ext_vector_type(N)));
  const vN x = *reinterpret_cast<const vN*>(p);
#pragma unroll
  for (int e = 0; e < N; ++e) r[e] = (float)x[e];
}

template <typename T, int N>
__device__ __forceinline__ void stv(T* p, const float (&r)[N]) {
  typedef T vN __attribute__((ext_vector_type(N)));
  vN x;
#pragma unroll
  for (int e = 0; e < N; ++e) x[e] = (T)r[e];
  *reinterpret_cast<vN*>(p) = x;
}

template <int N>
__device__ __forceinline__ float dotv(const float (&a)[N], const float (&b)[N]) {
  float s = a[0] * b[0];
#pragma unroll
  for (int e = 1; e < N; ++e) s = fmaf(a[e], b[e], s);
  return s;
}

// x from the lane the DPP pattern CTRL names (every lane has a source).
template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// Sum over aligned groups of LPQ lanes, left in every lane of the group. The
// partner patterns are involutions (lane a reads b while b reads a), so both
// compute the same a + b bit for bit. Within a 16-lane row they are DPP moves
// on the VALU: quad_perm [1,0,3,2] and [2,3,0,1], then row_half_mirror
// (lane k <-> 7 - k) and row_mirror (k <-> 15 - k), which pair the quads and
// the 8-lane halves once each holds its own sum.
template <int LPQ>
__device__ __forceinline__ float group_sum(float x) {
  static_assert(LPQ >= 4 && LPQ <= 32, "lane group of 4..32");
  x += dpp<0xB1>(x);
  x += dpp<0x4E>(x);
  if constexpr (LPQ >= 8) x += dpp<0x141>(x);
  if constexpr (LPQ >= 16) x += dpp<0x140>(x);
  if constexpr (LPQ >= 32) x += __shfl_xor(x, 16);
  return x;
}

__device__ __forceinline__ int wave_max(int x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x = max(x, __shfl_xor(x, off));
  return x;
}

// Extra sinks of query i: j in [0, n), n = min(s, i - span + 1) (0 if negative).
__device__ __forceinline__ int extra_sinks(int i, const AttnParams& p) {
  return max(0, min(p.sinks, i - p.window + 1));
}

// Sink keys [j00, j00 + cnt) of the K / V rows at kvrow0, staged in LDS as
// kvs[(jj * 2 + {0: K, 1: V}) * D + d] in fp32 by the whole workgroup: load()
// issues one 16-byte load per chunk (at most PT per thread), store() converts
// and writes them once the caller has made the LDS free.
template <typename T, int D>
struct SinkStage {
  static constexpr int E = 16 / (int)sizeof(T);
  static constexpr int CPR = D / E;                              // 16-byte chunks per row
  static constexpr int PT = (kSinkStage * 2 * CPR + 255) / 256;  // chunks per thread
  typedef T vec __attribute__((ext_vector_type(E)));
  vec buf[PT];

  __device__ __forceinline__ void load(const T* __restrict__ K, const T* __restrict__ V,
                                       long long kvrow0, long long kv_rs, int j00, int cnt) {
#pragma unroll
    for (int k = 0; k < PT; ++k) {
      const int x = threadIdx.x + 256 * k;
      if (x < cnt * 2 * CPR) {
        const int jj = x / (2 * CPR), kv = (x / CPR) & 1, c = x % CPR;
        const long long off = kvrow0 + (long long)(j00 + jj) * kv_rs + c * E;
        buf[k] = *reinterpret_cast<const vec*>((kv ? V : K) + off);
      }
    }
  }

  __device__ __forceinline__ void store(float* kvs, int cnt) const {
#pragma unroll
    for (int k = 0; k < PT; ++k) {
      const int x = threadIdx.x + 256 * k;
      if (x < cnt * 2 * CPR) {
#pragma unroll
        for (int e4 = 0; e4 < E / 4; ++e4) {
          f32x4 y;
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = (float)buf[k][4 * e4 + e];
          reinterpret_cast<f32x4*>(kvs + x * E)[e4] = y;
        }
      }
    }
  }
};

// The lane's EPL-slice of staged key jj (kv 0: K, 1: V).
template <int D, int E>
__device__ __forceinline__ void lds_slice(float (&r)[E], const float* kvs, int jj, int kv,
                                          int sub) {
  const f32x4* src = reinterpret_cast<const f32x4*>(kvs + (jj * 2 + kv) * D + sub * E);
#pragma unroll
  for (int e4 = 0; e4 < E / 4; ++e4) {
    const f32x4 x = src[e4];
#pragma unroll
    for (int e = 0; e < 4; ++e) r[4 * e4 + e] = x[e];
  }
}

}  // namespace

// Forward: merge query i's extra sink keys into (O, LSE), in place. Workgroup
// (b, h, chunk c) takes the ROWS rows i = span + c*ROWS + ...
template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_sink_fwd_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                     T* __restrict__ O, float* __restrict__ LSE, AttnParams p, int nchunk,
                     int nblk) {
  using G = SinkGeom<T, D>;
  constexpr int E = G::EPL, U = G::U, SC = kSinkChunk;
  extern __shared__ f32x4 kvs_raw[];
  float* kvs = reinterpret_cast<float*>(kvs_raw);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPQ, qg = lane / G::LPQ;
  const int ns = min(p.sinks, p.S - p.window);       // sinks any row sees
  for (int blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const int c = blk % nchunk, bh = blk / nchunk;    // 32-bit: sizes are validated
    const int b = bh / p.H, h = bh % p.H;
    int n[U], nm = 0, i_of[U];
    long long qoff[U], li[U];
    float q[U][E], o[U][E], la[U], m[U], l[U], acc[U][E];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ii = p.window + c * G::ROWS + u * 4 * G::QPW + wave * G::QPW + qg;
      n[u] = ii < p.S ? extra_sinks(ii, p) : 0;
      const int i = min(ii, p.S - 1);
      i_of[u] = i;
      qoff[u] = ((long long)b * p.S + i) * p.q_rs + (long long)h * D + sub * E;
      li[u] = (long long)bh * p.S + i;
      ldv<T, E>(q[u], Q + qoff[u]);
      ldv<T, E>(o[u], O + qoff[u]);
      la[u] = LSE[li[u]];                             // finite: key i is in the span
      nm = max(nm, n[u]);
      m[u] = -INFINITY;
      l[u] = 0.f;
#pragma unroll
      for (int e = 0; e < E; ++e) acc[u][e] = 0.f;
    }
    nm = wave_max(nm);
    const long long kvrow0 = (long long)b * p.S * p.kv_rs + (long long)(h / p.group) * D;
    for (int j00 = 0; j00 < ns; j00 += kSinkStage) {
      const int cnt = min(kSinkStage, ns - j00);
      SinkStage<T, D> stage;
      stage.load(K, V, kvrow0, p.kv_rs, j00, cnt);
      __syncthreads();                                // kvs free from the previous pass
      stage.store(kvs, cnt);
      __syncthreads();
      const int jend = min(j00 + cnt, nm);            // wave-uniform
      for (int j0 = j00; j0 < jend; j0 += SC) {
        float s[U][SC], mc[U];
#pragma unroll
        for (int w = 0; w < SC; ++w) {
          float kk[E];
          lds_slice<D, E>(kk, kvs, min(j0 + w, jend - 1) - j00, 0, sub);
#pragma unroll
          for (int u = 0; u < U; ++u) {
            s[u][w] = group_sum<G::LPQ>(dotv<E>(q[u], kk)) * p.scale;
            if (j0 + w >= n[u]) s[u][w] = -INFINITY;
          }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          mc[u] = m[u];
#pragma unroll
          for (int w = 0; w < SC; ++w) mc[u] = fmaxf(mc[u], s[u][w]);
          // A row with no sink yet keeps m = -inf, l = 0, acc = 0: use 0 as
          // its reference so that every factor below is exp(-inf) = 0.
          const float ref = mc[u] == -INFINITY ? 0.f : mc[u];
          const float alpha = __expf(m[u] - ref);
          l[u] *= alpha;
#pragma unroll
          for (int e = 0; e < E; ++e) acc[u][e] *= alpha;
#pragma unroll
          for (int w = 0; w < SC; ++w) {
            s[u][w] = __expf(s[u][w] - ref);
            l[u] += s[u][w];
          }
          m[u] = mc[u];
        }
#pragma unroll
        for (int w = 0; w < SC; ++w) {
          float vv[E];
          lds_slice<D, E>(vv, kvs, min(j0 + w, jend - 1) - j00, 1, sub);
#pragma unroll
          for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int e = 0; e < E; ++e) acc[u][e] = fmaf(s[u][w], vv[e], acc[u][e]);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (n[u] > 0) {
        // Span part (O_a, L_a), sink part (acc / l, L_b = m + log l):
        // L = logaddexp(L_a, L_b), O = e^(L_a - L) O_a + e^(m - L) acc.
        const float lb = m[u] + __logf(l[u]);
        const float mx = fmaxf(la[u], lb);
        const float lt = mx + __logf(__expf(la[u] - mx) + __expf(lb - mx));
        // O_a arrives gated (y_a = sigma * O_a): gate the sink part the same way.
      const float wa = __expf(la[u] - lt);
      const float wb = __expf(m[u] - lt) * gate_sigmoid(p, b, i_of[u], h);
#pragma unroll
        for (int e = 0; e < E; ++e) o[u][e] = fmaf(wa, o[u][e], wb * acc[u][e]);
        stv<T, E>(O + qoff[u], o[u]);
        if (sub == 0) LSE[li[u]] = lt;
      }
    }
  }
}

// dQ_i += scale * sum over query i's extra sinks j of dS_ij K_j,
// dS_ij = P_ij (dO_i . V_j - Delta_i), P_ij = exp(scale q_i . k_j - L_i).
// Same workgroup / row layout as the forward.
template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_sink_dq_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                    const T* __restrict__ dO, const float* __restrict__ LSE,
                    const float* __restrict__ Delta, T* __restrict__ dQ, AttnParams p,
                    int nchunk, int nblk) {
  using G = SinkGeom<T, D>;
  constexpr int E = G::EPL, U = G::U;
  extern __shared__ f32x4 kvs_raw[];
  float* kvs = reinterpret_cast<float*>(kvs_raw);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPQ, qg = lane / G::LPQ;
  const int ns = min(p.sinks, p.S - p.window);
  for (int blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const int c = blk % nchunk, bh = blk / nchunk;    // 32-bit: sizes are validated
    const int b = bh / p.H, h = bh % p.H;
    int n[U], nm = 0;
    long long qoff[U];
    float q[U][E], g[U][E], dq[U][E], acc[U][E], L[U], dl[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int ii = p.window + c * G::ROWS + u * 4 * G::QPW + wave * G::QPW + qg;
      n[u] = ii < p.S ? extra_sinks(ii, p) : 0;
      const int i = min(ii, p.S - 1);
      qoff[u] = ((long long)b * p.S + i) * p.q_rs + (long long)h * D + sub * E;
      ldv<T, E>(q[u], Q + qoff[u]);
      ldv<T, E>(g[u], dO + qoff[u]);
      ldv<T, E>(dq[u], dQ + qoff[u]);
      L[u] = LSE[(long long)bh * p.S + i];
      dl[u] = Delta[(long long)bh * p.S + i];
      nm = max(nm, n[u]);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[u][e] = 0.f;
    }
    nm = wave_max(nm);
    const long long kvrow0 = (long long)b * p.S * p.kv_rs + (long long)(h / p.group) * D;
    for (int j00 = 0; j00 < ns; j00 += kSinkStage) {
      const int cnt = min(kSinkStage, ns - j00);
      SinkStage<T, D> stage;
      stage.load(K, V, kvrow0, p.kv_rs, j00, cnt);
      __syncthreads();                                // kvs free from the previous pass
      stage.store(kvs, cnt);
      __syncthreads();
      const int jend = min(j00 + cnt, nm);
      for (int j = j00; j < jend; ++j) {
        float kk[E], vv[E];
        lds_slice<D, E>(kk, kvs, j - j00, 0, sub);
        lds_slice<D, E>(vv, kvs, j - j00, 1, sub);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const float sc = group_sum<G::LPQ>(dotv<E>(q[u], kk));
          const float dp = group_sum<G::LPQ>(dotv<E>(g[u], vv));
          const float ds = j < n[u] ? __expf(fmaf(sc, p.scale, -L[u])) * (dp - dl[u]) : 0.f;
#pragma unroll
          for (int e = 0; e < E; ++e) acc[u][e] = fmaf(ds, kk[e], acc[u][e]);
        }
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (n[u] > 0) {
#pragma unroll
        for (int e = 0; e < E; ++e) dq[u][e] = fmaf(p.scale, acc[u][e], dq[u][e]);
        stv<T, E>(dQ + qoff[u], dq[u]);
      }
    }
  }
}

// dK_j / dV_j of the sinks, stage 1: workgroup (b, kv head, chunk c) sums
// dS_ij Q_i and P_ij dO_i over its chunk of the (group head, i >= span) rows
// into part[b, kv head, c, j, {dK, dV}, D] (unscaled), kSinkChunk sinks per
// walk over the rows. The walk is software-pipelined: the next U rows of each
// lane group are loaded (as raw 16-byte vectors) while the current ones are
// used. With DQ the same walk also adds the rows' sink share to dQ (the full
// backward's fused sink pass; it needs all sinks in one walk, which the
// launcher guarantees).
template <typename T, int D, bool DQ>
struct SinkRows {
  static constexpr int E = 16 / (int)sizeof(T);
  typedef T vec __attribute__((ext_vector_type(E)));
  vec q[SinkGeom<T, D>::U], g[SinkGeom<T, D>::U], dq[DQ ? SinkGeom<T, D>::U : 1];
  long long qoff[DQ ? SinkGeom<T, D>::U : 1];
  float L[SinkGeom<T, D>::U], dl[SinkGeom<T, D>::U];
  int n[SinkGeom<T, D>::U];

  // Rows tb + u*4*QPW + qg of the chunk [t_lo, t_hi) (clamped; n = 0 past t_hi).
  __device__ __forceinline__ void load(const T* __restrict__ Q, const T* __restrict__ dO,
                                       const T* dQ, const float* __restrict__ LSE,
                                       const float* __restrict__ Delta, const AttnParams& p,
                                       int b, int hkv, int nrow, int tb, int t_hi, int qg,
                                       int sub) {
    using G = SinkGeom<T, D>;
#pragma unroll
    for (int u = 0; u < G::U; ++u) {
      const int t = tb + u * 4 * G::QPW + qg;
      const int tt = min(t, t_hi - 1);
      const int h = hkv * p.group + tt / nrow, i = p.window + tt % nrow;
      const long long off = ((long long)b * p.S + i) * p.q_rs + (long long)h * D + sub * E;
      const long long li = ((long long)b * p.H + h) * p.S + i;
      q[u] = *reinterpret_cast<const vec*>(Q + off);
      g[u] = *reinterpret_cast<const vec*>(dO + off);
      if constexpr (DQ) {
        dq[u] = *reinterpret_cast<const vec*>(dQ + off);
        qoff[u] = off;
      }
      L[u] = LSE[li];
      dl[u] = Delta[li];
      n[u] = t < t_hi ? extra_sinks(i, p) : 0;
    }
  }
};

template <typename T, int D, bool DQ>
__global__ void __launch_bounds__(256)
attn_sink_dkv_part_kernel(const T* __restrict__ Q, const T* __restrict__ K,
                          const T* __restrict__ V, const T* __restrict__ dO,
                          const float* __restrict__ LSE, const float* __restrict__ Delta,
                          T* dQ, float* __restrict__ part, AttnParams p, int nchunk,
                          int chunk_rows, int nblk) {
  using G = SinkGeom<T, D>;
  constexpr int E = G::EPL, U = G::U, SC = kSinkChunk, STEP = 4 * G::QPW * U;
  extern __shared__ f32x4 kvs_raw[];
  float* kvs = reinterpret_cast<float*>(kvs_raw);
  __shared__ float red[4][SC][2][D];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane % G::LPQ, qg = lane / G::LPQ;
  const int nrow = p.S - p.window;
  const int total = nrow * p.group;                   // < 2^31: S * H is validated
  const int ns = min(p.sinks, nrow);
  for (int blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const int c = blk % nchunk, bhk = blk / nchunk;
    const int b = bhk / p.Hkv, hkv = bhk % p.Hkv;
    const int t_lo = c * chunk_rows, t_hi = min(total, t_lo + chunk_rows);
    const int tb0 = t_lo + wave * G::QPW;
    const long long kvrow0 = (long long)b * p.S * p.kv_rs + (long long)hkv * D;
    float* out = part + ((long long)bhk * nchunk + c) * p.sinks * 2 * D;
    for (int j00 = 0; j00 < ns; j00 += kSinkStage) {
      const int cnt = min(kSinkStage, ns - j00);
      SinkRows<T, D, DQ> nxt;
      if (tb0 < t_hi) nxt.load(Q, dO, dQ, LSE, Delta, p, b, hkv, nrow, tb0, t_hi, qg, sub);
      SinkStage<T, D> stage;
      stage.load(K, V, kvrow0, p.kv_rs, j00, cnt);
      __syncthreads();
      stage.store(kvs, cnt);
      __syncthreads();
      for (int j0 = j00; j0 < j00 + cnt; j0 += SC) {
        if (j0 > j00 && tb0 < t_hi)
          nxt.load(Q, dO, dQ, LSE, Delta, p, b, hkv, nrow, tb0, t_hi, qg, sub);
        float dk[SC][E], dv[SC][E];
#pragma unroll
        for (int w = 0; w < SC; ++w) {
#pragma unroll
          for (int e = 0; e < E; ++e) dk[w][e] = dv[w][e] = 0.f;
        }
        // Wave-uniform walk over the chunk's rows, U rows per lane group.
        for (int tb = tb0; tb < t_hi; tb += STEP) {
          const SinkRows<T, D, DQ> cur = nxt;
          if (tb + STEP < t_hi)
            nxt.load(Q, dO, dQ, LSE, Delta, p, b, hkv, nrow, tb + STEP, t_hi, qg, sub);
          float q[U][E], g[U][E], aq[DQ ? U : 1][E];
#pragma unroll
          for (int e = 0; e < E; ++e) {
#pragma unroll
            for (int u = 0; u < (DQ ? U : 1); ++u) aq[u][e] = 0.f;
          }
#pragma unroll
          for (int u = 0; u < U; ++u) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
              q[u][e] = (float)cur.q[u][e];
              g[u][e] = (float)cur.g[u][e];
            }
          }
#pragma unroll
          for (int w = 0; w < SC; ++w) {
            const int jj = min(j0 + w, j00 + cnt - 1) - j00;
            float kk[E], vv[E];
            lds_slice<D, E>(kk, kvs, jj, 0, sub);
            lds_slice<D, E>(vv, kvs, jj, 1, sub);
#pragma unroll
            for (int u = 0; u < U; ++u) {
              const float sc = group_sum<G::LPQ>(dotv<E>(q[u], kk));
              const float dp = group_sum<G::LPQ>(dotv<E>(g[u], vv));
              const float pr = j0 + w < cur.n[u] ? __expf(fmaf(sc, p.scale, -cur.L[u])) : 0.f;
              const float ds = pr * (dp - cur.dl[u]);
#pragma unroll
              for (int e = 0; e < E; ++e) {
                dk[w][e] = fmaf(ds, q[u][e], dk[w][e]);
                dv[w][e] = fmaf(pr, g[u][e], dv[w][e]);
              }
              if constexpr (DQ) {
#pragma unroll
                for (int e = 0; e < E; ++e) aq[u][e] = fmaf(ds, kk[e], aq[u][e]);
              }
            }
          }
          if constexpr (DQ) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
              if (cur.n[u] > 0) {
                float d[E];
#pragma unroll
                for (int e = 0; e < E; ++e) d[e] = fmaf(p.scale, aq[u][e], (float)cur.dq[u][e]);
                stv<T, E>(dQ + cur.qoff[u], d);
              }
            }
          }
        }
        // Sum the wave's row groups, then the four waves, in a fixed order.
#pragma unroll
        for (int off = G::LPQ; off < 64; off <<= 1) {
#pragma unroll
          for (int w = 0; w < SC; ++w) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
              dk[w][e] += __shfl_xor(dk[w][e], off);
              dv[w][e] += __shfl_xor(dv[w][e], off);
            }
          }
        }
        __syncthreads();                              // red[] free from the previous pass
        if (qg == 0) {
#pragma unroll
          for (int w = 0; w < SC; ++w) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
              red[wave][w][0][sub * E + e] = dk[w][e];
              red[wave][w][1][sub * E + e] = dv[w][e];
            }
          }
        }
        __syncthreads();
        for (int x = threadIdx.x; x < SC * 2 * D; x += 256) {
          const int w = x / (2 * D), y = x % (2 * D), kv = y / D, d = y % D;
          if (j0 + w < j00 + cnt) {
            const float sum =
                ((red[0][w][kv][d] + red[1][w][kv][d]) + red[2][w][kv][d]) + red[3][w][kv][d];
            out[(long long)(j0 + w) * 2 * D + y] = sum;
          }
        }
      }
    }
  }
}

// Stage 2: dK_j += scale * sum_c part[.., c, j, 0, :], dV_j += sum_c part[.., c, j, 1, :],
// chunks summed in order (four loads in flight at a time). One workgroup per
// (b, kv head, sink j), grid-strided.
template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_sink_dkv_reduce_kernel(const float* __restrict__ part, T* __restrict__ dK,
                            T* __restrict__ dV, AttnParams p, int nchunk, int nblk) {
  const int ns = min(p.sinks, p.S - p.window);
  const int x = threadIdx.x;
  if (x >= 2 * D) return;
  const long long cs = (long long)p.sinks * 2 * D;   // chunk stride
  for (int blk = blockIdx.x; blk < nblk; blk += gridDim.x) {
    const int j = blk % ns, bhk = blk / ns;
    const int b = bhk / p.Hkv, hkv = bhk % p.Hkv;
    const float* src = part + (long long)bhk * nchunk * cs + (long long)j * 2 * D + x;
    float sum = 0.f;
    int c = 0;
    for (; c + 4 <= nchunk; c += 4) {
      const float a0 = src[c * cs], a1 = src[(c + 1) * cs], a2 = src[(c + 2) * cs],
                  a3 = src[(c + 3) * cs];
      sum = (((sum + a0) + a1) + a2) + a3;
    }
    for (; c < nchunk; ++c) sum += src[c * cs];
    const long long row = ((long long)b * p.S + j) * p.kv_rs + (long long)hkv * D;
    T* dst = x < D ? dK + row + x : dV + row + (x - D);
    *dst = (T)((float)*dst + (x < D ? p.scale * sum : sum));
  }
}

// ---------------------------------------------------------------------------
// launchers and workspace sizing. p.window is the local span; there is
// nothing to add unless some query sees a sink beyond it.
// ---------------------------------------------------------------------------
namespace {

constexpr long long kMaxGrid = 1 << 20;
constexpr int kPartBlocks = 512;     // target workgroups for the dK/dV partial pass
constexpr int kMaxChunks = 64;

// The kernels here have work: sinks beyond the span that the window kernels
// do not visit themselves (p.fold_sinks: float32; 16-bit folds every sink).
bool sinks_active(const AttnParams& p) {
  return p.sinks > 0 && p.fold_sinks == 0 && p.window > 0 && p.window < p.S && p.B > 0 &&
         p.H > 0;
}

unsigned grid_of(long long nblk) { return (unsigned)(nblk < kMaxGrid ? nblk : kMaxGrid); }

// Dynamic LDS of the staged sink keys: min(sinks seen, kSinkStage) x {K, V} x D fp32.
size_t stage_bytes(const AttnParams& p, int D) {
  const int ns = min(p.sinks, p.S - p.window);
  return (size_t)min(ns, kSinkStage) * 2 * D * sizeof(float);
}

template <typename T> struct TypeTag { using type = T; };
template <int D> struct DimTag { static constexpr int value = D; };

// Calls f(TypeTag<T>{}, DimTag<D>{}) for the runtime (dtype, D).
template <typename F>
hipError_t dispatch(int dtype, int D, F&& f) {
  auto by_d = [&](auto tt) -> hipError_t {
    switch (D) {
      case 32: return f(tt, DimTag<32>{});
      case 64: return f(tt, DimTag<64>{});
      case 128: return f(tt, DimTag<128>{});
    }
    return hipErrorInvalidValue;
  };
  switch (dtype) {
    case 0: return by_d(TypeTag<float>{});
    case 1: return by_d(TypeTag<_Float16>{});
    case 2: return by_d(TypeTag<__bf16>{});
  }
  return hipErrorInvalidValue;
}

}  // namespace

// Row chunks per (b, kv head) of the dK/dV partial pass: enough workgroups to
// fill the chip, each with at least 64 rows, at most kMaxChunks.
int sink_chunks(const AttnParams& p, int* chunk_rows) {
  const int total = (p.S - p.window) * p.group;
  const long long units = (long long)p.B * p.Hkv;
  int n = (int)((kPartBlocks + units - 1) / units);
  n = max(1, min(n, min(kMaxChunks, (total + 63) / 64)));
  const int rows = (total + n - 1) / n;
  n = (total + rows - 1) / rows;                    // no empty chunk
  if (chunk_rows) *chunk_rows = rows;
  return n;
}

// Floats of backward workspace the sink pass needs beyond the [2,B,H,S] planes.
long long sink_workspace_floats(const AttnParams& p, int D) {
  if (!sinks_active(p)) return 0;
  return (long long)p.B * p.Hkv * sink_chunks(p, nullptr) * p.sinks * 2 * D;
}

hipError_t launch_sink_fwd(int dtype, int D, const void* q, const void* k, const void* v, void* o,
                           float* lse, const AttnParams& p, hipStream_t st) {
  if (!sinks_active(p)) return hipSuccess;
  return dispatch(dtype, D, [&](auto tt, auto dd) -> hipError_t {
    using T = typename decltype(tt)::type;
    constexpr int DD = decltype(dd)::value;
    const int nchunk = (p.S - p.window + SinkGeom<T, DD>::ROWS - 1) / SinkGeom<T, DD>::ROWS;
    const int nblk = p.B * p.H * nchunk;               // validated to fit
    hipLaunchKernelGGL((attn_sink_fwd_kernel<T, DD>), dim3(grid_of(nblk)), dim3(256),
                       stage_bytes(p, DD), st, (const T*)q, (const T*)k, (const T*)v, (T*)o, lse,
                       p, nchunk, nblk);
    return hipGetLastError();
  });
}

hipError_t launch_sink_dq(int dtype, int D, const void* q, const void* k, const void* v,
                          const void* dout, const float* lse, const float* delta, void* dq,
                          const AttnParams& p, hipStream_t st) {
  if (!sinks_active(p)) return hipSuccess;
  return dispatch(dtype, D, [&](auto tt, auto dd) -> hipError_t {
    using T = typename decltype(tt)::type;
    constexpr int DD = decltype(dd)::value;
    const int nchunk = (p.S - p.window + SinkGeom<T, DD>::ROWS - 1) / SinkGeom<T, DD>::ROWS;
    const int nblk = p.B * p.H * nchunk;
    hipLaunchKernelGGL((attn_sink_dq_kernel<T, DD>), dim3(grid_of(nblk)), dim3(256),
                       stage_bytes(p, DD), st, (const T*)q, (const T*)k, (const T*)v,
                       (const T*)dout, lse, delta, (T*)dq, p, nchunk, nblk);
    return hipGetLastError();
  });
}

// True when the full backward can add the sinks' dQ share in the dK / dV
// pass: every row sees all its sinks within one walk (at most kSinkChunk).
bool sink_bwd_fusable(const AttnParams& p) {
  return sinks_active(p) && min(p.sinks, p.S - p.window) <= kSinkChunk;
}

// `part` is the workspace area after the [2,B,H,S] planes
// (sink_workspace_floats(p, D) floats). With dq != nullptr (only when
// sink_bwd_fusable) the same pass also adds the sinks' share of dQ.
hipError_t launch_sink_dkv(int dtype, int D, const void* q, const void* k, const void* v,
                           const void* dout, const float* lse, const float* delta, float* part,
                           void* dk, void* dv, void* dq, const AttnParams& p, hipStream_t st) {
  if (!sinks_active(p)) return hipSuccess;
  if (dq && !sink_bwd_fusable(p)) return hipErrorInvalidValue;
  int rows = 0;
  const int nchunk = sink_chunks(p, &rows);
  const int ns = min(p.sinks, p.S - p.window);
  return dispatch(dtype, D, [&](auto tt, auto dd) -> hipError_t {
    using T = typename decltype(tt)::type;
    constexpr int DD = decltype(dd)::value;
    const int units = p.B * p.Hkv;
    if (dq)
      hipLaunchKernelGGL((attn_sink_dkv_part_kernel<T, DD, true>), dim3(grid_of(units * nchunk)),
                         dim3(256), stage_bytes(p, DD), st, (const T*)q, (const T*)k,
                         (const T*)v, (const T*)dout, lse, delta, (T*)dq, part, p, nchunk, rows,
                         units * nchunk);
    else
      hipLaunchKernelGGL((attn_sink_dkv_part_kernel<T, DD, false>), dim3(grid_of(units * nchunk)),
                         dim3(256), stage_bytes(p, DD), st, (const T*)q, (const T*)k,
                         (const T*)v, (const T*)dout, lse, delta, (T*)nullptr, part, p, nchunk,
                         rows, units * nchunk);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((attn_sink_dkv_reduce_kernel<T, DD>), dim3(grid_of((long long)units * ns)),
                       dim3(256), 0, st, (const float*)part, (T*)dk, (T*)dv, p, nchunk,
                       units * ns);
    return hipGetLastError();
  });
}

}  // namespace mi
