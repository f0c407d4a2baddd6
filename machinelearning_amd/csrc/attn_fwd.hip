// Flash-attention forward for gfx950, float32 inputs (v_mfma_f32_32x32x2f32): O = softmax(scale*Q K^T + mask) V and the
// natural-log LSE tape, on [B,S,H,D] / [B,S,Hkv,D] tensors with native GQA.
//
// Algorithm (what the reference's forward computes, nanolab/csrc/flash_attn_cuda.cu:8-14,
// 582-797): an online softmax over key tiles; L = m*scale + ln(l). The design
// here is this file's own:
//
//  * One workgroup = 4 waves = 128 queries of one (batch, head); a wave owns 32
//    queries. Scores are computed TRANSPOSED, S^T = K Q^T, with 32x32 MFMAs:
//    keys are the M dimension (A operand read from LDS), queries the N
//    dimension (B operand, held in registers for the whole kernel). The
//    accumulator then puts ONE query per lane (column l32), so the running max,
//    the running sum and the O rescale are per-lane scalars, and the row
//    reductions need a single cross-half exchange per tile.
//  * P feeds O^T += V^T P^T straight from the accumulator registers (no LDS
//    round trip): V is staged in LDS transposed, with keys permuted by
//    perm_pos() so that each A fragment is one 16-byte read.
//  * exp2-domain softmax: scores stay raw, exp2(s*scale*log2e - m*scale*log2e)
//    is one FMA + one v_exp_f32.
//  * K/V tiles (64 keys) are double-buffered in LDS; the next tile's global
//    loads are issued before the current tile's MFMAs and stored after them,
//    so one barrier per tile suffices.
//  * Causal / sliding-window tile skipping at workgroup granularity (the tile
//    range) and at wave granularity (a wave above the diagonal skips its
//    MFMAs); the per-element mask runs only on tiles that straddle a boundary.
//  * Heaviest causal query blocks are dispatched first, and all blocks of one
//    (batch, head) land on the same XCD (blockIdx % 8 is the XCD and
//    B*H is the fastest-varying part of the block index), so K/V stay in one L2.
#include "attn_common.h"

namespace mi {

template <typename T, int D, bool BLK>
__global__ void __launch_bounds__(256)
attn_fwd_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                T* __restrict__ O, float* __restrict__ LSE, AttnParams p) {
  using M = Mfma32<T>;
  using frag = typename M::frag;
  constexpr int EPL = M::EPL, KPI = 2 * EPL;
  constexpr int BM = 128, BN = 64;
  constexpr int DS = D / KPI;   // k-steps over the head dim
  constexpr int DT = D / 32;    // 32-row output tiles over the head dim
  using G = TileGeom<T, BN, D>;
  constexpr int BUF = G::NAT_BYTES + G::TR_BYTES;
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
  const T* Kb = K + (long long)b * p.S * p.kv_rs + (long long)hkv * D;
  const T* Vb = V + (long long)b * p.S * p.kv_rs + (long long)hkv * D;

  frag qf[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
    qf[ds] = (qi < p.S) ? ld_frag<T>(Qb + (long long)qi * p.q_rs + ds * KPI + g * EPL) : zero_frag<T>();

  int kbeg = 0, kend = p.S;
  if (p.causal) kend = min(p.S, causal_key_end<BLK>(p, q0 + BM - 1) + 1);
  if (p.window > 0) kbeg = max(0, q0 - p.window + 1);
  const int t_begin = kbeg / BN, t_end = (kend + BN - 1) / BN;

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
        if (tile == 0) unit_store_nat<T, BN, D>(pre[i], base, unit);
        else unit_store_tr<T, BN, D>(pre[i], base + G::NAT_BYTES, unit);
      }
    }
  };

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = zero16();
  // Running max of raw scores for query qi. A finite sentinel (not -inf)
  // keeps exp2(s*c - m*c) at exp2(-inf) = 0 for masked scores before the
  // first visible key; every stored row sees at least one key.
  float m_run = -1e30f;
  float l_run = 0.f;         // this lane's share of the running exp-sum
  // Visible keys of query qi: [key_lo, key_hi].
  const int key_hi = p.causal ? min(causal_key_end<BLK>(p, qi), p.S - 1) : p.S - 1;
  const int wave_key_lo_end = p.causal ? causal_key_end<BLK>(p, qw0) : p.S;
  const int wave_key_hi_end = p.causal ? causal_key_end<BLK>(p, qw0 + 31) : p.S;
  const int key_lo = p.window > 0 ? qi - p.window + 1 : 0;
  const float c = p.scale_log2;

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
      const char* Vt = Ks + G::NAT_BYTES;
      bool need_mask = (k0 + BN > p.S);
      if (p.causal) need_mask = need_mask || (k0 + BN - 1 > wave_key_lo_end);
      if (p.window > 0) need_mask = need_mask || (k0 <= qw0 + 31 - p.window);

      f32x16 sacc[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        sacc[mt] = zero16();
#pragma unroll
        for (int ds = 0; ds < DS; ++ds)
          sacc[mt] = M::mma(ld_frag<T>(nat_ptr<T, BN, D>(Ks, mt * 32 + l32, ds * KPI + g * EPL)),
                            qf[ds], sacc[mt]);
      }
      if (need_mask) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
          const int kb = k0 + mt * 32 + 4 * g;
          mask_rows(sacc[mt], key_lo - kb, key_hi - kb, -INFINITY);
        }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[mt][r]);
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      // Lazy rescale: the running max only moves when some query's tile max
      // exceeds it by more than resc_th raw units (2^8 in probability), so
      // p stays <= 256 and the O / l rescale is skipped on most tiles.
      if (wave_any(mx > m_run + p.resc_th)) {
        const float m_new = fmaxf(m_run, mx);
        const float alpha = fast_exp2((m_run - m_new) * c);
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        m_run = m_new;
      }
      const float mc = m_run * c;
      float rs = 0.f;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pv = fast_exp2(fmaf(sacc[mt][r], c, -mc));
          sacc[mt][r] = pv;
          rs += pv;
        }
      l_run += rs;

#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int s = 0; s < 16 / EPL; ++s) {
          const frag pb = pack_frag<T>(sacc[mt], s * EPL);
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
            oacc[dt] = M::mma(ld_frag<T>(tr_ptr<T, BN, D>(Vt, dt * 32 + l32, mt * 32 + s * KPI + g * EPL)),
                              pb, oacc[dt]);
        }
    }

    if (t + 1 < t_end) store_tile(cur ^ 1);
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (qi < p.S) {
    // Normalise, and apply the output gate sigma(z) of this query row when given.
    const float inv = gate_sigmoid(p, b, qi, h) / l_tot;
    T* Ob = O + (long long)b * p.S * p.q_rs + (long long)qi * p.q_rs + (long long)h * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        st_quad<T>(Ob + dt * 32 + 8 * j + 4 * g, oacc[dt][4 * j] * inv, oacc[dt][4 * j + 1] * inv,
                   oacc[dt][4 * j + 2] * inv, oacc[dt][4 * j + 3] * inv);
    if (g == 0) LSE[((long long)b * p.H + h) * p.S + qi] = m_run * p.scale + logf(l_tot);
  }
}

template <typename T, int D>
static hipError_t launch_fwd_t(const void* q, const void* k, const void* v, void* o, float* lse,
                               AttnParams p, hipStream_t st) {
  constexpr int BM = 128;
  p.nblk = (p.S + BM - 1) / BM;
  const long long nblocks = (long long)p.nblk * p.B * p.H;
  if (p.block > 1) {   // block-causal variant
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, true>), dim3((unsigned)nblocks), dim3(256), 0, st,
                       (const T*)q, (const T*)k, (const T*)v, (T*)o, lse, p);
  } else {
    hipLaunchKernelGGL((attn_fwd_kernel<T, D, false>), dim3((unsigned)nblocks), dim3(256), 0, st,
                       (const T*)q, (const T*)k, (const T*)v, (T*)o, lse, p);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_fwd_d(int D, const void* q, const void* k, const void* v, void* o,
                               float* lse, const AttnParams& p, hipStream_t st) {
  switch (D) {
    case 32: return launch_fwd_t<T, 32>(q, k, v, o, lse, p, st);
    case 64: return launch_fwd_t<T, 64>(q, k, v, o, lse, p, st);
    case 128: return launch_fwd_t<T, 128>(q, k, v, o, lse, p, st);
  }
  return hipErrorInvalidValue;
}

// float32 only: the 16-bit types run attn_fwd16_kernel (attn_fwd16.hip).
hipError_t launch_fwd(int dtype, int D, const void* q, const void* k, const void* v, void* o,
                      float* lse, const AttnParams& p, hipStream_t st) {
  if (dtype == 0) return launch_fwd_d<float>(D, q, k, v, o, lse, p, st);
  return hipErrorInvalidValue;
}

}  // namespace mi
