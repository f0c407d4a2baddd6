// Flash-attention backward for gfx950: three launches on one stream,
//   delta  : Delta[b,h,i] = sum_d dO*O - dLSE, and -LSE/scale       (HBM-bound)
//   dK/dV  : per key block, loop over the GQA group and query tiles  (4 MFMA products)
//   dQ     : per query block, loop over key tiles                    (3 MFMA products)
// No atomics anywhere, so every gradient is bitwise reproducible.
//
// Algebra (nanolab/csrc/flash_attn_cuda.cu:8-14): p = exp(s*scale - L),
// dS = p*(dP - Delta), dQ = scale*dS K, dK = scale*dS^T Q, dV = p^T dO.
// An incoming LSE gradient enters as Delta -= dLSE (dLSE_i/ds_ij = p_ij), so
// the op's second output is differentiable at no extra cost.
//
// Register layouts (one wave, 32x32 MFMA tiles; see attn_common.h):
//  * dK/dV: the wave owns 32 keys held as B operands for the whole kernel.
//    S = Q K^T and dP = dO V^T put one KEY per lane, so P and dS feed
//    dV^T += dO^T P and dK^T += Q^T dS directly from registers; Q and dO are
//    staged twice in LDS: natural (A of S/dP) and transposed with permuted rows
//    (A of dV/dK).
//  * dQ: the wave owns 32 queries held as B operands. S^T = K Q^T and
//    dP^T = V dO^T put one QUERY per lane, so LSE and Delta are lane scalars
//    and dS^T feeds dQ^T += K^T dS^T from registers; K is staged natural (A of
//    S^T) and transposed (A of dQ^T), V natural (A of dP^T).
#include "attn_common.h"

namespace mi {

// ---------------------------------------------------------------------------
// delta: the backward's [2][B][H][S] float workspace.
//   plane 0: Delta[b,h,i] = sum_d dO*O - dLSE      (every backward kernel)
//   plane 1: -LSE[b,h,i] / scale                    (16-bit dK/dV: it seeds the
//            S accumulator, so exp2(scale_log2 * acc) = exp(s*scale - L))
// One workgroup per (b, h, 64 consecutive queries): the O / dO rows are read
// as whole 16-byte chunks (LPR lanes per row), and the 64 outputs of each
// plane are one contiguous run, so the writes are coalesced.
// ---------------------------------------------------------------------------
template <typename T, int D>
struct DeltaGeom {
  static constexpr int EV = 16 / (int)sizeof(T);   // elements per 16-byte chunk
  static constexpr int LPR = D / EV;               // lanes per row
  static constexpr int RPP = 256 / LPR;            // rows per pass of the workgroup
  static constexpr int ROWS = 64;                  // queries per workgroup
};

// With an output gate (p.gate): O is the gated output y = sigma(z) * O_attn
// and dO the gradient of y. Then rowsum(dO * O) is already
// rowsum(dO_attn * O_attn) with dO_attn = sigma * dO, which the kernel also
// writes to dOe for the later passes, and dz = (1 - sigma) * rowsum(dO * O).
template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_bwd_delta_kernel(const T* __restrict__ O, const T* __restrict__ dO,
                      const float* __restrict__ LSE, const float* __restrict__ dlse,
                      float* __restrict__ ws, T* __restrict__ dOe, float* __restrict__ dz,
                      AttnParams p) {
  using G = DeltaGeom<T, D>;
  const int tid = threadIdx.x;
  const int sub = tid % G::LPR, r = tid / G::LPR;
  const int nblk = (p.S + G::ROWS - 1) / G::ROWS;
  const int bh = blockIdx.x / nblk;                    // b * H + h
  const int i0 = (blockIdx.x % nblk) * G::ROWS;
  const int b = bh / p.H, h = bh % p.H;
  const long long plane = (long long)p.B * p.H * p.S;
  const float nls = -1.f / p.scale;
#pragma unroll
  for (int pass = 0; pass < G::ROWS / G::RPP; ++pass) {
    const int i = i0 + pass * G::RPP + r;
    float acc = 0.f;
    const float sg = i < p.S ? gate_sigmoid(p, b, i, h) : 1.f;
    if (i < p.S) {
      const long long off = ((long long)b * p.S + i) * p.q_rs + (long long)h * D + sub * G::EV;
      if constexpr (sizeof(T) == 2) {
        using F8 = typename Mfma32<T>::frag;
        const F8 a = *reinterpret_cast<const F8*>(O + off);
        const F8 d = *reinterpret_cast<const F8*>(dO + off);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc = fmaf((float)a[e], (float)d[e], acc);
        if (p.gate) {
          F8 de;
#pragma unroll
          for (int e = 0; e < 8; ++e) de[e] = (T)((float)d[e] * sg);
          *reinterpret_cast<F8*>(dOe + off) = de;
        }
      } else {
        const f32x4 a = *reinterpret_cast<const f32x4*>(O + off);
        const f32x4 d = *reinterpret_cast<const f32x4*>(dO + off);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = fmaf(a[e], d[e], acc);
        if (p.gate) *reinterpret_cast<f32x4*>(dOe + off) = d * sg;
      }
    }
#pragma unroll
    for (int x = G::LPR / 2; x >= 1; x >>= 1) acc += __shfl_xor(acc, x);
    if (i < p.S && sub == 0) {
      const long long idx = (long long)bh * p.S + i;
      ws[idx] = acc - (dlse ? dlse[idx] : 0.f);
      ws[plane + idx] = LSE[idx] * nls;
      if (p.gate) dz[((long long)b * p.S + i) * p.H + h] = (1.f - sg) * acc;
    }
  }
}

// ---------------------------------------------------------------------------
// dK / dV
// ---------------------------------------------------------------------------
template <typename T, int D, int BQ, bool BLK>
__global__ void __launch_bounds__(256)
attn_bwd_dkdv_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                     const T* __restrict__ dO, const float* __restrict__ LSE,
                     const float* __restrict__ Delta, T* __restrict__ dK, T* __restrict__ dV,
                     AttnParams p) {
  using M = Mfma32<T>;
  using frag = typename M::frag;
  constexpr int EPL = M::EPL, KPI = 2 * EPL;
  constexpr int BK = 128;            // keys per workgroup: 4 waves x 32
  constexpr int DS = D / KPI, DT = D / 32, MQ = BQ / 32;
  using G = TileGeom<T, BQ, D>;
  constexpr int OFF_DOS = G::NAT_BYTES;
  constexpr int OFF_QT = 2 * G::NAT_BYTES;
  constexpr int OFF_DOT = 2 * G::NAT_BYTES + G::TR_BYTES;
  constexpr int OFF_L = 2 * G::NAT_BYTES + 2 * G::TR_BYTES;
  constexpr int OFF_D = OFF_L + BQ * 4;
  constexpr int BUF = OFF_D + BQ * 4;
  constexpr int U = G::UNITS;
  constexpr int UPT = (2 * U + 255) / 256;
  static_assert(2 * BQ <= 256, "vector staging assumes one float per thread");
  __shared__ __attribute__((aligned(16))) char smem[2 * BUF];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int BHk = p.B * p.Hkv;
  const int bhk = blockIdx.x % BHk;
  const int kb = blockIdx.x / BHk;
  const int b = bhk / p.Hkv, hkv = bhk % p.Hkv;
  const int k0 = kb * BK;
  const int kw0 = k0 + wave * 32;
  const int kj = kw0 + l32;

  const T* Kb = K + (long long)b * p.S * p.kv_rs + (long long)hkv * D;
  const T* Vb = V + (long long)b * p.S * p.kv_rs + (long long)hkv * D;
  frag kf[DS], vf[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    const long long off = (long long)kj * p.kv_rs + ds * KPI + g * EPL;
    kf[ds] = (kj < p.S) ? ld_frag<T>(Kb + off) : zero_frag<T>();
    vf[ds] = (kj < p.S) ? ld_frag<T>(Vb + off) : zero_frag<T>();
  }
  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dkacc[dt] = zero16();
    dvacc[dt] = zero16();
  }

  int qbeg = 0, qend = p.S;
  if (p.causal) qbeg = causal_query_begin<BLK>(p, k0);
  if (p.window > 0) qend = min(p.S, k0 + BK - 1 + p.window);
  const int tq_begin = qbeg / BQ;
  const int ntq = max(0, (qend + BQ - 1) / BQ - tq_begin);
  const int niter = p.group * ntq;
  const float c = p.scale_log2;
  // Queries that see key kj: [q_lo, q_hi] (padded queries carry L = +inf, so p = 0).
  const int q_lo = p.causal ? causal_query_begin<BLK>(p, kj) : 0;
  const int wave_q_lo0 = p.causal ? causal_query_begin<BLK>(p, kw0) : 0;
  const int wave_q_lo31 = p.causal ? causal_query_begin<BLK>(p, kw0 + 31) : 0;
  const int q_hi = p.window > 0 ? kj + p.window - 1 : 0x3fffffff;

  Unit pre[UPT];
  float vpre = 0.f;
  auto load_iter = [&](int it) {
    const int gh = it / ntq;
    const int q0 = (tq_begin + it % ntq) * BQ;
    const int h = hkv * p.group + gh;
    const T* Qb = Q + (long long)b * p.S * p.q_rs + (long long)h * D;
    const T* dOb = dO + (long long)b * p.S * p.q_rs + (long long)h * D;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + i * 256;
      if (u < 2 * U) {
        const int tile = u / U, unit = u % U;
        unit_load<T, BQ, D>(pre[i], tile ? dOb : Qb, p.q_rs, q0, p.S, unit);
      }
    }
    if (tid < 2 * BQ) {
      const int qq = q0 + (tid % BQ);
      const long long idx = ((long long)b * p.H + h) * p.S + qq;
      if (tid < BQ) vpre = (qq < p.S) ? LSE[idx] * kLog2e : INFINITY;
      else vpre = (qq < p.S) ? Delta[idx] : 0.f;
    }
  };
  auto store_iter = [&](int buf) {
    char* base = smem + buf * BUF;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + i * 256;
      if (u < 2 * U) {
        const int tile = u / U, unit = u % U;
        unit_store_nat<T, BQ, D>(pre[i], base + (tile ? OFF_DOS : 0), unit);
        unit_store_tr<T, BQ, D>(pre[i], base + (tile ? OFF_DOT : OFF_QT), unit);
      }
    }
    if (tid < 2 * BQ) reinterpret_cast<float*>(base + OFF_L)[tid] = vpre;   // Ls then Ds
  };

  if (niter > 0) {
    load_iter(0);
    store_iter(0);
  }
  __syncthreads();

  for (int it = 0; it < niter; ++it) {
    const int cur = it & 1;
    if (it + 1 < niter) load_iter(it + 1);

    const int q0 = (tq_begin + it % ntq) * BQ;
    bool active = kw0 < p.S;
    if (p.causal) active = active && (q0 + BQ - 1 >= wave_q_lo0);
    if (p.window > 0) active = active && (q0 <= kw0 + 31 + p.window - 1);
    if (active) {
      const char* base = smem + cur * BUF;
      const char* Qs = base;
      const char* dOs = base + OFF_DOS;
      const char* Qt = base + OFF_QT;
      const char* dOt = base + OFF_DOT;
      const float* Ls = reinterpret_cast<const float*>(base + OFF_L);
      const float* Dl = reinterpret_cast<const float*>(base + OFF_D);
      bool need_mask = false;
      if (p.causal) need_mask = (q0 < wave_q_lo31);
      if (p.window > 0) need_mask = need_mask || (q0 + BQ - 1 - p.window >= kw0);

      f32x16 sacc[MQ], dpacc[MQ];
#pragma unroll
      for (int mt = 0; mt < MQ; ++mt) {
        sacc[mt] = zero16();
        dpacc[mt] = zero16();
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          sacc[mt] = M::mma(ld_frag<T>(nat_ptr<T, BQ, D>(Qs, mt * 32 + l32, ds * KPI + g * EPL)),
                            kf[ds], sacc[mt]);
          dpacc[mt] = M::mma(ld_frag<T>(nat_ptr<T, BQ, D>(dOs, mt * 32 + l32, ds * KPI + g * EPL)),
                             vf[ds], dpacc[mt]);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MQ; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 L4 = *reinterpret_cast<const f32x4*>(Ls + mt * 32 + 8 * j + 4 * g);
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            sacc[mt][4 * j + tt] = fast_exp2(fmaf(sacc[mt][4 * j + tt], c, -L4[tt]));
        }
      if (need_mask) {
#pragma unroll
        for (int mt = 0; mt < MQ; ++mt) {
          const int qb = q0 + mt * 32 + 4 * g;
          mask_rows(sacc[mt], q_lo - qb, q_hi - qb, 0.f);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MQ; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const f32x4 D4 = *reinterpret_cast<const f32x4*>(Dl + mt * 32 + 8 * j + 4 * g);
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            dpacc[mt][4 * j + tt] = sacc[mt][4 * j + tt] * (dpacc[mt][4 * j + tt] - D4[tt]);
        }
#pragma unroll
      for (int mt = 0; mt < MQ; ++mt)
#pragma unroll
        for (int s = 0; s < 16 / EPL; ++s) {
          const frag pb = pack_frag<T>(sacc[mt], s * EPL);
          const frag sb = pack_frag<T>(dpacc[mt], s * EPL);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const int pos = mt * 32 + s * KPI + g * EPL;
            dvacc[dt] = M::mma(ld_frag<T>(tr_ptr<T, BQ, D>(dOt, dt * 32 + l32, pos)), pb, dvacc[dt]);
            dkacc[dt] = M::mma(ld_frag<T>(tr_ptr<T, BQ, D>(Qt, dt * 32 + l32, pos)), sb, dkacc[dt]);
          }
        }
    }

    if (it + 1 < niter) store_iter(cur ^ 1);
    __syncthreads();
  }

  if (kj < p.S) {
    const long long off = (long long)b * p.S * p.kv_rs + (long long)kj * p.kv_rs + (long long)hkv * D;
    T* dKr = dK + off;
    T* dVr = dV + off;
    const float sc = p.scale;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = dt * 32 + 8 * j + 4 * g;
        st_quad<T>(dKr + d0, dkacc[dt][4 * j] * sc, dkacc[dt][4 * j + 1] * sc,
                   dkacc[dt][4 * j + 2] * sc, dkacc[dt][4 * j + 3] * sc);
        st_quad<T>(dVr + d0, dvacc[dt][4 * j], dvacc[dt][4 * j + 1], dvacc[dt][4 * j + 2],
                   dvacc[dt][4 * j + 3]);
      }
  }
}

// ---------------------------------------------------------------------------
// dQ
// ---------------------------------------------------------------------------
template <typename T, int D, int BN, bool BLK>
__global__ void __launch_bounds__(256)
attn_bwd_dq_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                   const T* __restrict__ dO, const float* __restrict__ LSE,
                   const float* __restrict__ Delta, T* __restrict__ dQ, AttnParams p) {
  using M = Mfma32<T>;
  using frag = typename M::frag;
  constexpr int EPL = M::EPL, KPI = 2 * EPL;
  constexpr int BM = 128;
  constexpr int DS = D / KPI, DT = D / 32, MK = BN / 32;
  using G = TileGeom<T, BN, D>;
  constexpr int OFF_VS = G::NAT_BYTES;
  constexpr int OFF_KT = 2 * G::NAT_BYTES;
  constexpr int BUF = 2 * G::NAT_BYTES + G::TR_BYTES;
  constexpr int U = G::UNITS;
  constexpr int UPT = (2 * U + 255) / 256;
  __shared__ __attribute__((aligned(16))) char smem[2 * BUF];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  int qb = blockIdx.x / BH;
  if (p.causal) qb = p.nblk - 1 - qb;
  const int b = bh / p.H, h = bh % p.H, hkv = h / p.group;
  const int q0 = qb * BM;
  const int qw0 = q0 + wave * 32;
  const int qi = qw0 + l32;

  const T* Qb = Q + (long long)b * p.S * p.q_rs + (long long)h * D;
  const T* dOb = dO + (long long)b * p.S * p.q_rs + (long long)h * D;
  const T* Kb = K + (long long)b * p.S * p.kv_rs + (long long)hkv * D;
  const T* Vb = V + (long long)b * p.S * p.kv_rs + (long long)hkv * D;

  frag qf[DS], dof[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    const long long off = (long long)qi * p.q_rs + ds * KPI + g * EPL;
    qf[ds] = (qi < p.S) ? ld_frag<T>(Qb + off) : zero_frag<T>();
    dof[ds] = (qi < p.S) ? ld_frag<T>(dOb + off) : zero_frag<T>();
  }
  float L2 = INFINITY, Dq = 0.f;
  if (qi < p.S) {
    const long long idx = ((long long)b * p.H + h) * p.S + qi;
    L2 = LSE[idx] * kLog2e;
    Dq = Delta[idx];
  }

  f32x16 dqacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqacc[dt] = zero16();

  int kbeg = 0, kend = p.S;
  if (p.causal) kend = min(p.S, causal_key_end<BLK>(p, q0 + BM - 1) + 1);
  if (p.window > 0) kbeg = max(0, q0 - p.window + 1);
  const int t_begin = kbeg / BN, t_end = (kend + BN - 1) / BN;
  const float c = p.scale_log2;
  // Visible keys of query qi: [key_lo, key_hi].
  const int key_hi = p.causal ? min(causal_key_end<BLK>(p, qi), p.S - 1) : p.S - 1;
  const int wave_key_lo_end = p.causal ? causal_key_end<BLK>(p, qw0) : p.S;
  const int wave_key_hi_end = p.causal ? causal_key_end<BLK>(p, qw0 + 31) : p.S;
  const int key_lo = p.window > 0 ? qi - p.window + 1 : 0;

  Unit pre[UPT];
  auto load_tile = [&](int t) {
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + i * 256;
      if (u < 2 * U) {
        const int tile = u / U, unit = u % U;
        unit_load<T, BN, D>(pre[i], tile ? Vb : Kb, p.kv_rs, t * BN, p.S, unit);
      }
    }
  };
  auto store_tile = [&](int buf) {
    char* base = smem + buf * BUF;
#pragma unroll
    for (int i = 0; i < UPT; ++i) {
      const int u = tid + i * 256;
      if (u < 2 * U) {
        const int tile = u / U, unit = u % U;
        if (tile == 0) {
          unit_store_nat<T, BN, D>(pre[i], base, unit);
          unit_store_tr<T, BN, D>(pre[i], base + OFF_KT, unit);
        } else {
          unit_store_nat<T, BN, D>(pre[i], base + OFF_VS, unit);
        }
      }
    }
  };

  if (t_begin < t_end) {
    load_tile(t_begin);
    store_tile(0);
  }
  __syncthreads();

  for (int t = t_begin; t < t_end; ++t) {
    const int cur = (t - t_begin) & 1;
    if (t + 1 < t_end) load_tile(t + 1);

    const int k0 = t * BN;
    bool active = qw0 < p.S;
    if (p.causal) active = active && (k0 <= wave_key_hi_end);
    if (p.window > 0) active = active && (k0 + BN - 1 > qw0 - p.window);
    if (active) {
      const char* Ks = smem + cur * BUF;
      const char* Vs = Ks + OFF_VS;
      const char* Kt = Ks + OFF_KT;
      bool need_mask = (k0 + BN > p.S);
      if (p.causal) need_mask = need_mask || (k0 + BN - 1 > wave_key_lo_end);
      if (p.window > 0) need_mask = need_mask || (k0 <= qw0 + 31 - p.window);

      f32x16 sacc[MK], dpacc[MK];
#pragma unroll
      for (int mt = 0; mt < MK; ++mt) {
        sacc[mt] = zero16();
        dpacc[mt] = zero16();
#pragma unroll
        for (int ds = 0; ds < DS; ++ds) {
          sacc[mt] = M::mma(ld_frag<T>(nat_ptr<T, BN, D>(Ks, mt * 32 + l32, ds * KPI + g * EPL)),
                            qf[ds], sacc[mt]);
          dpacc[mt] = M::mma(ld_frag<T>(nat_ptr<T, BN, D>(Vs, mt * 32 + l32, ds * KPI + g * EPL)),
                             dof[ds], dpacc[mt]);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MK; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[mt][r] = fast_exp2(fmaf(sacc[mt][r], c, -L2));
      if (need_mask) {
#pragma unroll
        for (int mt = 0; mt < MK; ++mt) {
          const int kb = k0 + mt * 32 + 4 * g;
          mask_rows(sacc[mt], key_lo - kb, key_hi - kb, 0.f);
        }
      }
#pragma unroll
      for (int mt = 0; mt < MK; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) dpacc[mt][r] = sacc[mt][r] * (dpacc[mt][r] - Dq);
#pragma unroll
      for (int mt = 0; mt < MK; ++mt)
#pragma unroll
        for (int s = 0; s < 16 / EPL; ++s) {
          const frag sb = pack_frag<T>(dpacc[mt], s * EPL);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
            dqacc[dt] = M::mma(ld_frag<T>(tr_ptr<T, BN, D>(Kt, dt * 32 + l32, mt * 32 + s * KPI + g * EPL)),
                               sb, dqacc[dt]);
        }
    }

    if (t + 1 < t_end) store_tile(cur ^ 1);
    __syncthreads();
  }

  if (qi < p.S) {
    T* dQr = dQ + (long long)b * p.S * p.q_rs + (long long)qi * p.q_rs + (long long)h * D;
    const float sc = p.scale;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        st_quad<T>(dQr + dt * 32 + 8 * j + 4 * g, dqacc[dt][4 * j] * sc, dqacc[dt][4 * j + 1] * sc,
                   dqacc[dt][4 * j + 2] * sc, dqacc[dt][4 * j + 3] * sc);
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
// Query tile of dK/dV and key tile of dQ (float32: 32 rows).
constexpr int kDkdvBq = 32, kDqBn = 32;

template <typename T, int D>
static hipError_t launch_delta_t(const void* o, const void* dout, const float* lse,
                                 const float* dlse, float* ws, void* doe, float* dz, AttnParams p,
                                 hipStream_t st) {
  const long long nblocks = (long long)p.B * p.H * ((p.S + DeltaGeom<T, D>::ROWS - 1) / DeltaGeom<T, D>::ROWS);
  hipLaunchKernelGGL((attn_bwd_delta_kernel<T, D>), dim3((unsigned)nblocks), dim3(256), 0, st,
                     (const T*)o, (const T*)dout, lse, dlse, ws, (T*)doe, dz, p);
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_dkdv_t(const void* q, const void* k, const void* v, const void* dout,
                                const float* lse, const float* delta, void* dk, void* dv,
                                AttnParams p, hipStream_t st) {
  constexpr int BK = 128;
  p.nblk = (p.S + BK - 1) / BK;
  const long long nblocks = (long long)p.nblk * p.B * p.Hkv;
  if (p.block > 1) {   // block-causal variant
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, D, kDkdvBq, true>), dim3((unsigned)nblocks), dim3(256),
                       0, st, (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, delta,
                       (T*)dk, (T*)dv, p);
  } else {
    hipLaunchKernelGGL((attn_bwd_dkdv_kernel<T, D, kDkdvBq, false>), dim3((unsigned)nblocks), dim3(256),
                       0, st, (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, delta,
                       (T*)dk, (T*)dv, p);
  }
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_dq_t(const void* q, const void* k, const void* v, const void* dout,
                              const float* lse, const float* delta, void* dq, AttnParams p,
                              hipStream_t st) {
  constexpr int BM = 128;
  p.nblk = (p.S + BM - 1) / BM;
  const long long nblocks = (long long)p.nblk * p.B * p.H;
  if (p.block > 1) {   // block-causal variant
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, D, kDqBn, true>), dim3((unsigned)nblocks), dim3(256), 0,
                       st, (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, delta, (T*)dq, p);
  } else {
    hipLaunchKernelGGL((attn_bwd_dq_kernel<T, D, kDqBn, false>), dim3((unsigned)nblocks), dim3(256), 0,
                       st, (const T*)q, (const T*)k, (const T*)v, (const T*)dout, lse, delta, (T*)dq, p);
  }
  return hipGetLastError();
}

#define MI_DISPATCH(dtype, D, CALL)                                   \
  switch (dtype) {                                                    \
    case 0:                                                           \
      switch (D) {                                                    \
        case 32: { using T = float; constexpr int DD = 32; CALL; }     \
        case 64: { using T = float; constexpr int DD = 64; CALL; }     \
        case 128: { using T = float; constexpr int DD = 128; CALL; }   \
      }                                                               \
      break;                                                          \
    case 1:                                                           \
      switch (D) {                                                    \
        case 32: { using T = _Float16; constexpr int DD = 32; CALL; }  \
        case 64: { using T = _Float16; constexpr int DD = 64; CALL; }  \
        case 128: { using T = _Float16; constexpr int DD = 128; CALL; }\
      }                                                               \
      break;                                                          \
    case 2:                                                           \
      switch (D) {                                                    \
        case 32: { using T = __bf16; constexpr int DD = 32; CALL; }    \
        case 64: { using T = __bf16; constexpr int DD = 64; CALL; }    \
        case 128: { using T = __bf16; constexpr int DD = 128; CALL; }  \
      }                                                               \
      break;                                                          \
  }                                                                   \
  return hipErrorInvalidValue;

// With p.gate set, doe (the gate-scaled output gradient, [B,S,H,D]) and dz
// (the gate logits' gradient, [B,S,H]) are written as well.
hipError_t launch_bwd_delta(int dtype, int D, const void* o, const void* dout, const float* lse,
                            const float* dlse, float* ws, void* doe, float* dz,
                            const AttnParams& p, hipStream_t st) {
  MI_DISPATCH(dtype, D, return (launch_delta_t<T, DD>(o, dout, lse, dlse, ws, doe, dz, p, st)))
}

// dK/dV and dQ: float32 only (the 16-bit types run attn_bwd16.hip's kernels;
// the delta pass above serves every dtype).
hipError_t launch_bwd_dkdv(int dtype, int D, const void* q, const void* k, const void* v,
                           const void* dout, const float* lse, const float* delta, void* dk,
                           void* dv, const AttnParams& p, hipStream_t st) {
  if (dtype != 0) return hipErrorInvalidValue;
  switch (D) {
    case 32: return launch_dkdv_t<float, 32>(q, k, v, dout, lse, delta, dk, dv, p, st);
    case 64: return launch_dkdv_t<float, 64>(q, k, v, dout, lse, delta, dk, dv, p, st);
    case 128: return launch_dkdv_t<float, 128>(q, k, v, dout, lse, delta, dk, dv, p, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_bwd_dq(int dtype, int D, const void* q, const void* k, const void* v,
                         const void* dout, const float* lse, const float* delta, void* dq,
                         const AttnParams& p, hipStream_t st) {
  if (dtype != 0) return hipErrorInvalidValue;
  switch (D) {
    case 32: return launch_dq_t<float, 32>(q, k, v, dout, lse, delta, dq, p, st);
    case 64: return launch_dq_t<float, 64>(q, k, v, dout, lse, delta, dq, p, st);
    case 128: return launch_dq_t<float, 128>(q, k, v, dout, lse, delta, dq, p, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace mi
