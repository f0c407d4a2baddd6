// Flash-attention forward for 16-bit inputs (bf16 / f16) on gfx950.
//
// Same algorithm as the reference's forward (nanolab/csrc/flash_attn_cuda.cu:8-14,
// 582-797: online softmax over key tiles, L = m*scale + ln(l)); the schedule
// is this file's own:
//
//  * Workgroup = 4 waves = 128 queries of one (batch, head); a wave owns 32
//    queries. Scores are computed transposed, S^T = K Q^T (keys = MFMA rows,
//    read from LDS; queries = MFMA columns, held in registers), so every lane
//    owns one query and the softmax statistics are lane scalars.
//  * K and V tiles (64 keys) stream HBM -> LDS through a ring of NS stages
//    with global_load_lds (no VGPR staging, no LDS store instructions); the
//    loads for tile t+NS-1 are in flight while tile t is computed, and one
//    barrier per tile both publishes tile t and frees the stage refilled next.
//  * P^T feeds O^T += V^T P^T straight from the score registers; the V^T
//    operand comes from the natural V tile through ds_read_b64_tr_b16.
//  * Lazy rescale: the running max moves only when a tile raises some
//    query's max by more than 8 (log2 units), decided by a wave ballot on the
//    lane-local max; the cross-half exchange and the O rescale run only then.
//  * Heaviest causal query blocks first; all blocks of one (batch, head) have
//    equal blockIdx mod 8 when B*H % 8 == 0, so they share one XCD's L2.
#include "attn16.h"

namespace mi {

template <int D>
struct Fwd16 {
  static constexpr int BM = 128, BN = 64;
  static constexpr int NS = D >= 128 ? 2 : 3;      // LDS ring depth
  static constexpr int CH = D / 8;                 // 16-byte chunks per row
  static constexpr int TILE = BN * D * 2;          // bytes of one K (or V) tile
  static constexpr int LPW = CH / 4;               // DMA instructions per wave per tensor
  static constexpr int LPT = 2 * LPW;              // ... per tile (K and V)
  static constexpr int DS = D / 16, DT = D / 32;
};

template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_fwd16_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                  T* __restrict__ O, float* __restrict__ LSE, AttnParams p) {
  using C = Fwd16<D>;
  using M = Mfma32<T>;
  using frag = typename M::frag;
  constexpr int BM = C::BM, BN = C::BN, NS = C::NS, DS = C::DS, DT = C::DT;
  // One LDS array per ring stage and tensor: distinct objects let the
  // compiler's wait-count pass see that a read of stage s cannot alias the
  // DMA still filling another stage (with one shared array it drains every
  // in-flight load before each transposed read).
  __shared__ __attribute__((aligned(1024))) char sK0[C::TILE], sV0[C::TILE];
  __shared__ __attribute__((aligned(1024))) char sK1[C::TILE], sV1[C::TILE];
  __shared__ __attribute__((aligned(1024))) char sK2[NS > 2 ? C::TILE : 16], sV2[NS > 2 ? C::TILE : 16];
  auto kst = [&](int stage) -> char* { return stage == 0 ? sK0 : stage == 1 ? sK1 : sK2; };
  auto vst = [&](int stage) -> char* { return stage == 0 ? sV0 : stage == 1 ? sV1 : sV2; };

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

  // Q fragments (MFMA B operand): query qi, head dims [16*ds + 8*g, +8).
  frag qf[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds)
    qf[ds] = (qi < p.S) ? ld_frag<T>(Qb + (long long)qi * p.q_rs + ds * 16 + g * 8) : zero_frag<T>();

  int kbeg = 0, kend = p.S;
  if (p.causal) kend = min(p.S, q0 + BM);
  if (p.window > 0) kbeg = max(0, q0 - p.window + 1);
  const int t_begin = kbeg / BN, t_end = (kend + BN - 1) / BN;

  // DMA lane map: instruction j of this wave fills LDS slots
  // (4j + wave) * 64 + lane of a tile; slot -> (row, physical chunk), and the
  // lane fetches the logical chunk that the swizzle puts there.
  int drow[C::LPW], dcol[C::LPW];
#pragma unroll
  for (int j = 0; j < C::LPW; ++j) {
    const int slot = (4 * j + wave) * 64 + lane;
    drow[j] = slot / C::CH;
    dcol[j] = ((slot % C::CH) ^ swz<D>(drow[j])) * 8;
  }
  auto issue_tile = [&](int stage, int t) {
    char* bk = kst(stage);
    char* bv = vst(stage);
#pragma unroll
    for (int j = 0; j < C::LPW; ++j) {
      const long long off = (long long)min(t * BN + drow[j], p.S - 1) * p.kv_rs + dcol[j];
      dma16(Kb + off, bk + (4 * j + wave) * 1024);
      dma16(Vb + off, bv + (4 * j + wave) * 1024);
    }
  };

  // Fragment addresses inside a stage (bytes). K rows l32 (+32 for mt = 1),
  // chunk 2*ds + g; V^T reads: see attn16.h (rows 4*(G>>1) + (m>>2) + 32mt +
  // 16s + 8h, columns dt*32 + 16*(G&1) + 4*(m&3)).
  int kaddr[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) kaddr[ds] = tile_off<D>(l32, 2 * ds + g);
  int vaddr[DT];
  {
    const int G = lane >> 4, m = lane & 15;
    const int row = 4 * (G >> 1) + (m >> 2);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int col = dt * 32 + 16 * (G & 1) + 4 * (m & 3);
      vaddr[dt] = tile_off<D>(row, col >> 3) + (col & 7) * 2;
    }
  }

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = zero16();
  // Running max of raw scores (finite sentinel: exp2(s*c - m*c) of a masked
  // score is exp2(-inf) = 0 before the first visible key), lane-local sum.
  float m_run = -1e30f, l_run = 0.f;
  const float c = p.scale_log2;
  const int key_hi = p.causal ? min(qi, p.S - 1) : p.S - 1;
  const int key_lo = p.window > 0 ? qi - p.window + 1 : 0;

  auto compute = [&](int stage, int t) {
    const char* sK = kst(stage);
    const char* sV = vst(stage);
    const int k0 = t * BN;
    bool active = qw0 < p.S;
    if (p.causal) active = active && (k0 <= qw0 + 31);
    if (p.window > 0) active = active && (k0 + BN - 1 > qw0 - p.window);
    if (!active) return;
    bool need_mask = (k0 + BN > p.S);
    if (p.causal) need_mask = need_mask || (k0 + BN - 1 > qw0);
    if (p.window > 0) need_mask = need_mask || (k0 <= qw0 + 31 - p.window);

    f32x16 sacc[2];
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      sacc[mt] = zero16();
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
        sacc[mt] = M::mma(lds_frag<T>(sK + kaddr[ds] + mt * 32 * D * 2), qf[ds], sacc[mt]);
    }
    if (need_mask) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int kb = k0 + mt * 32 + 4 * g;
        mask_rows(sacc[mt], key_lo - kb, key_hi - kb, -INFINITY);
      }
    }
    float mx = fmaxf(sacc[0][0], sacc[1][0]);
#pragma unroll
    for (int r = 1; r < 16; ++r) mx = fmaxf(mx, fmaxf(sacc[0][r], sacc[1][r]));
    if (wave_any(mx > m_run + p.resc_th)) {
      const float m_new = fmaxf(m_run, halves_max(mx));
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
      for (int s = 0; s < 2; ++s) {
        const frag pb = pack_frag<T>(sacc[mt], s * 8);
        const int roff = (32 * mt + 16 * s) * D * 2;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
          oacc[dt] = M::mma(lds_frag_tr<T>(sV + vaddr[dt] + roff, sV + vaddr[dt] + roff + 8 * D * 2),
                            pb, oacc[dt]);
      }
  };

  // One ring step: wait for tile t, publish it, refill the stage freed by
  // tile t-1 with tile t+NS-1, compute tile t.
  auto step = [&](int stage, int t) {
    if (NS == 3 && t + 1 < t_end) wait_vm<C::LPT>();
    else wait_vm<0>();
    lds_barrier();
    if (t + NS - 1 < t_end) issue_tile((stage + NS - 1) % NS, t + NS - 1);
    compute(stage, t);
  };

#pragma unroll
  for (int i = 0; i < NS - 1; ++i)
    if (t_begin + i < t_end) issue_tile(i, t_begin + i);
  // Retire the Q loads (and the prologue) with a wait the compiler's own
  // wait-count pass sees; otherwise it cannot prove the Q registers landed
  // and drains every in-flight tile load before each tile's first MFMA.
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  int t = t_begin;
  for (; t + NS <= t_end; t += NS) {
#pragma unroll
    for (int s = 0; s < NS; ++s) step(s, t + s);
  }
#pragma unroll
  for (int s = 0; s < NS - 1; ++s)
    if (t + s < t_end) step(s, t + s);

  const float l_tot = halves_sum(l_run);
  if (qi < p.S) {
    const float inv = 1.f / l_tot;
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
static hipError_t launch_fwd16_t(const void* q, const void* k, const void* v, void* o, float* lse,
                                 AttnParams p, hipStream_t st) {
  constexpr int BM = Fwd16<D>::BM;
  p.nblk = (p.S + BM - 1) / BM;
  const long long nblocks = (long long)p.nblk * p.B * p.H;
  hipLaunchKernelGGL((attn_fwd16_kernel<T, D>), dim3((unsigned)nblocks), dim3(256), 0, st,
                     (const T*)q, (const T*)k, (const T*)v, (T*)o, lse, p);
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_fwd16_d(int D, const void* q, const void* k, const void* v, void* o,
                                 float* lse, const AttnParams& p, hipStream_t st) {
  switch (D) {
    case 32: return launch_fwd16_t<T, 32>(q, k, v, o, lse, p, st);
    case 64: return launch_fwd16_t<T, 64>(q, k, v, o, lse, p, st);
    case 128: return launch_fwd16_t<T, 128>(q, k, v, o, lse, p, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_fwd16(int dtype, int D, const void* q, const void* k, const void* v, void* o,
                        float* lse, const AttnParams& p, hipStream_t st) {
  switch (dtype) {
    case 1: return launch_fwd16_d<_Float16>(D, q, k, v, o, lse, p, st);
    case 2: return launch_fwd16_d<__bf16>(D, q, k, v, o, lse, p, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace mi
