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
//  * XCD- and L2-aware block order (work_item): each XCD works through its
//    heads in groups whose K/V fit in its L2, heaviest causal blocks first.
#include <type_traits>

#include "attn16.h"

namespace mi {

template <int D>
struct Fwd16 {
  static constexpr int BM = 128, BN = 64;
  // LDS ring depth (units). Two slots against three, A/B in both orders: the
  // board forward within noise (41.6 vs 41.3 us), SWA(256) 1-5% faster, D=32
  // 2.6-4.7% faster; 16 KB less LDS. The unit in flight is one step ahead.
  static constexpr int NS = 2;
  static constexpr int UNROLL = NS == 3 ? 6 : 2;   // lcm(NS, 2): ring slot and score parity fixed
  static constexpr int CH = D / 8;                 // 16-byte chunks per row
  static constexpr int TILE = BN * D * 2;          // bytes of one K (or V) tile
  static constexpr int LPW = CH / 4;               // DMA instructions per wave per tensor
  static constexpr int LPU = 2 * LPW;              // ... per ring unit (K and V)
  static constexpr int DS = D / 16, DT = D / 32;
};

template <int I>
using ic = std::integral_constant<int, I>;

// Wait until at most n ring units (LPU loads each) of this wave are in flight.
template <int LPU>
__device__ __forceinline__ void wait_units(int n) {
  if (n <= 0) wait_vm<0>();
  else if (n == 1) wait_vm<LPU>();
  else wait_vm<2 * LPU>();
}

// Max of the 32 scores a lane holds: two chains of v_maximum3_f32. (The IEEE
// maximum needs no NaN canonicalisation of the MFMA results, unlike fmaxf,
// which doubles the instruction count; scores are finite or -inf.)
__device__ __forceinline__ float max32(const f32x16& a, const f32x16& b) {
  float ma = a[0], mb = b[0];
#pragma unroll
  for (int r = 1; r < 16; ++r) {
    ma = __builtin_elementwise_maximum(ma, a[r]);
    mb = __builtin_elementwise_maximum(mb, b[r]);
  }
  return __builtin_elementwise_maximum(ma, mb);
}

// Scheduling-group masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008, kSchedValu = 0x002, kSchedDsRead = 0x100;

template <typename T, int D, bool BLK>
__global__ void __launch_bounds__(256)
attn_fwd16_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                  T* __restrict__ O, float* __restrict__ LSE, AttnParams p) {
  using C = Fwd16<D>;
  using M = Mfma32<T>;
  using frag = typename M::frag;
  constexpr int BM = C::BM, BN = C::BN, NS = C::NS, DS = C::DS, DT = C::DT;
  // LDS ring: slot s holds the K tile (ring[s][0]) and V tile (ring[s][1]) of one unit.
  __shared__ __attribute__((aligned(1024))) char ring[NS][2][C::TILE];
  // Q of the workgroup's 128 rows (two 64-row tiles), fetched by LDS-DMA and
  // read into registers once (D <= 64; at D = 128 two workgroups per CU leave
  // no room, and Q is loaded directly).
  constexpr bool Q_DMA = D <= 64;
  __shared__ __attribute__((aligned(1024))) char qstage[Q_DMA ? 2 : 1][Q_DMA ? C::TILE : 16];
  auto kst = [&](int slot) __attribute__((always_inline)) -> char* { return ring[slot][0]; };
  auto vst = [&](int slot) __attribute__((always_inline)) -> char* { return ring[slot][1]; };
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const WorkItem wi = work_item(p.nblk, p.B * p.H, p.div_wi, p.causal, p.wi_blocks_fastest);
  const int bh = wi.bh, qb = wi.blk;
  const int b = (int)fdiv((unsigned)bh, p.div_h), h = bh - b * p.H;
  const int hkv = (int)fdiv((unsigned)h, p.div_group);
  const int q0 = qb * BM;
  const int qw0 = q0 + wave * 32;
  const int qi = qw0 + l32;

  const T* Qb = Q + (long long)b * p.S * p.q_rs + (long long)h * D;

  // Q fragments (MFMA B operand): query qi, head dims [16*ds + 8*g, +8).
  frag qf[DS];
  if constexpr (!Q_DMA) {
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
      qf[ds] = (qi < p.S) ? ld_frag<T>(Qb + (long long)qi * p.q_rs + ds * 16 + g * 8) : zero_frag<T>();
  } else {
    // Issued first; read after the prologue's wait and barrier (load_q).
    const RowTiles tQ = row_tiles(Q, b, p.S, p.q_rs, h, D);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      const Rsrc rq = tile_rsrc(tQ, q0 / BN + half);
#pragma unroll
      for (int j = 0; j < C::LPW; ++j) {
        const int slot = (4 * j + wave) * 64 + lane;
        const int row = slot / C::CH;
        const unsigned off = (unsigned)(row * p.q_rs + ((slot % C::CH) ^ swz<D>(row)) * 8) * 2u;
        dma16_buf(rq, off, lds_u32(qstage[half] + wave * 1024) + (unsigned)(4096 * j));
      }
    }
  }
  auto load_q = [&]() __attribute__((always_inline)) {
    if constexpr (Q_DMA) {
      const int qrow = 32 * (wave & 1) + l32;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) qf[ds] = lds_frag<T>(qstage[wave >> 1] + tile_off<D>(qrow, 2 * ds + g));
    }
  };

  // Key tiles of the workgroup [t_begin, t_end) and of this wave [tw_begin, tw_end).
  int kbeg = 0, kend = p.S;
  if (p.causal) kend = min(p.S, causal_key_end<BLK>(p, q0 + BM - 1) + 1);
  if (p.window > 0) kbeg = max(0, q0 - p.window + 1);
  const int t_begin = kbeg / BN, t_end = (kend + BN - 1) / BN;
  int tw_begin = t_begin, tw_end = t_end;
  if (qw0 >= p.S) tw_end = tw_begin;
  if (p.causal) tw_end = min(tw_end, causal_key_end<BLK>(p, qw0 + 31) / BN + 1);
  if (p.window > 0) tw_begin = max(tw_begin, max(0, qw0 - p.window + 1) / BN);

  // DMA lane map: instruction j of this wave fills LDS slots
  // (4j + wave) * 64 + lane of a tile; slot -> (row, physical chunk), and the
  // lane fetches the logical chunk that the swizzle puts there. The byte
  // offset inside a tile is fixed per lane; the tile moves the resource base.
  unsigned dvoff[C::LPW];
#pragma unroll
  for (int j = 0; j < C::LPW; ++j) {
    const int slot = (4 * j + wave) * 64 + lane;
    const int row = slot / C::CH;
    dvoff[j] = (unsigned)(row * p.kv_rs + ((slot % C::CH) ^ swz<D>(row)) * 8) * 2u;
  }
  // Ring unit u = {K tile u+1, V tile u}, kept in slot (u - t_begin + 1) % NS.
  // Each tile is read through a buffer resource whose range ends at row S of
  // this head, so rows past the end read as zeros (masked later) and the
  // unused edge halves (K tile t_end, V tile t_begin - 1, moved to tile 0)
  // still issue their loads: every unit is exactly LPU loads per wave.
  // LDS address of this wave's first DMA chunk of slot 0's K tile; the other
  // targets are constant offsets from it.
  const unsigned m0w = lds_u32(ring[0][0] + wave * 1024);
  const RowTiles tK = row_tiles(K, b, p.S, p.kv_rs, hkv, D);
  const RowTiles tV = row_tiles(V, b, p.S, p.kv_rs, hkv, D);
  auto issue_pair = [&](int slot, int kt, int vt) __attribute__((always_inline)) {
    const Rsrc rk = tile_rsrc(tK, kt);
    const Rsrc rv = tile_rsrc(tV, vt);
#pragma unroll
    for (int j = 0; j < C::LPW; ++j) {
      dma16_buf(rk, dvoff[j], m0w + (unsigned)((2 * slot) * C::TILE + 4096 * j));
      dma16_buf(rv, dvoff[j], m0w + (unsigned)((2 * slot + 1) * C::TILE + 4096 * j));
    }
  };
  auto issue_unit = [&](int slot, int u) __attribute__((always_inline)) {
    issue_pair(slot, u + 1, max(u, 0));
  };

  // Fragment addresses inside a slot (bytes). K rows l32 (+32 for mt = 1),
  // chunk 2*ds + g; V^T reads: rows 4*(G>>1) + (m>>2) + 8h (+ 32mt + 16s as
  // immediates), columns dt*32 + 16*(G&1) + 4*(m&3) (attn16.h's map).
  int kaddr[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) kaddr[ds] = tile_off<D>(l32, 2 * ds + g);
  int vaddr[DT][2];
  {
    const int G = lane >> 4, m = lane & 15;
    const int row = 4 * (G >> 1) + (m >> 2);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int col = dt * 32 + 16 * (G & 1) + 4 * (m & 3);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) vaddr[dt][hh] = tile_off<D>(row + 8 * hh, col >> 3) + (col & 7) * 2;
    }
  }

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = zero16();
  // Scores of two consecutive tiles (ping-pong by tile parity): S^T of the
  // tile being softmaxed and of the next one, whose MFMAs run under it.
  f32x16 sS[2][2];
  // Running max of raw scores (finite sentinel: exp2(s*c - m*c) of a masked
  // score is exp2(-inf) = 0 before the first visible key), lane-local sum.
  float m_run = -1e30f, l_run = 0.f;
  bool sank = false;   // the folded-sink visit already put its share into O and l
  const float c = p.scale_log2;
  const int key_hi = p.causal ? min(causal_key_end<BLK>(p, qi), p.S - 1) : p.S - 1;
  const int wave_key_hi = p.causal ? causal_key_end<BLK>(p, qw0) : p.S;   // smallest key_hi of the wave
  const int key_lo = p.window > 0 ? qi - p.window + 1 : 0;

  auto scores = [&](f32x16 (&sd)[2], const char* sK) {
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      sd[mt] = zero16();
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
        sd[mt] = M::mma(lds_frag<T>(sK + kaddr[ds] + mt * 32 * D * 2), qf[ds], sd[mt]);
    }
  };

  // One ring step for tile t (its scores already in sS[PAR]): wait for unit
  // t, publish it, refill the slot freed by step t-1, then softmax tile t
  // while the MFMAs of tile t+1's scores run, then O^T += V_t^T P_t^T.
  auto step = [&](auto slot_fill_c, auto par_c, int t) __attribute__((always_inline)) {
    constexpr int SF = decltype(slot_fill_c)::value;   // slot refilled now
    constexpr int SR = (SF + 1) % NS;                  // slot holding K_{t+1}, V_t
    constexpr int PAR = decltype(par_c)::value;
    wait_units<C::LPU>(min(NS - 2, t_end - 1 - t));
    lds_barrier();
    if (t + NS - 1 <= t_end - 1) issue_unit(SF, t + NS - 1);
    const char* sK = kst(SR);
    const char* sV = vst(SR);
    const bool cur = t >= tw_begin && t < tw_end;
    const bool nxt = t + 1 >= tw_begin && t + 1 < tw_end;
    f32x16 (&s)[2] = sS[PAR];
    if (cur) {
      const int k0 = t * BN;
      const bool need_hi = (k0 + BN > p.S) || (p.causal && k0 + BN - 1 > wave_key_hi);
      const bool need_lo = p.window > 0 && k0 <= qw0 + 31 - p.window;
      if (need_hi) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) mask_above(s[mt], key_hi - (k0 + mt * 32 + 4 * g), -INFINITY);
      }
      if (need_lo) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) mask_below(s[mt], key_lo - (k0 + mt * 32 + 4 * g), -INFINITY);
      }
      const float mx = max32(s[0], s[1]);
      if (t == tw_begin && !sank) {
        // The wave's first tile, nothing accumulated yet (O = 0, l = 0): set
        // the max, no rescale.
        m_run = fmaxf(m_run, halves_max(mx));
      } else if (wave_any(mx > m_run + p.resc_th)) {
        // Lazy rescale: the running max only moves when some query's tile max
        // exceeds it by more than resc_th raw units (2^8 in probability).
        const float m_new = fmaxf(m_run, halves_max(mx));
        const float alpha = fast_exp2((m_run - m_new) * c);
        l_run *= alpha;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) oacc[dt][r] *= alpha;
        m_run = m_new;
      }
    }
    // Softmax of tile t -> bf16 P fragments, then O^T += V_t^T P_t^T.
    auto softmax_pv = [&]() __attribute__((always_inline)) {
      const float mc = m_run * c;
      float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float pv = fast_exp2(fmaf(s[mt][r], c, -mc));
          s[mt][r] = pv;
          if (mt == 0 && r < 4) rs[r] = pv;   // first term: no add of 0.0 (kept for -0.0)
          else rs[r & 3] += pv;
        }
      l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          const frag pb = pack_frag<T>(s[mt], ks * 8);
          const int roff = (32 * mt + 16 * ks) * D * 2;
#pragma unroll
          for (int dt = 0; dt < DT; ++dt)
            oacc[dt] = M::mma(lds_frag_tr<T>(sV + vaddr[dt][0] + roff, sV + vaddr[dt][1] + roff),
                              pb, oacc[dt]);
        }
    };
    if (cur && nxt) {
      // Steady state as one explicitly scheduled block. Phase A: each of the
      // next tile's score MFMAs is followed by a slice of this tile's
      // exp / sum work, which the wave issues while the matrix core runs
      // the MFMA (8 passes); K fragments are read two MFMAs ahead.
      // Phase B: P fragments -> O^T += V^T P^T, V^T read one MFMA ahead
      // (two at D = 128).
      // sched_barrier(0) pins the slice order against the scheduler, which
      // otherwise issues all MFMAs back to back and the VALU work after.
      constexpr int NM = 2 * DS;          // score MFMAs of the next tile
      constexpr int EPM = 32 / NM;        // exp elements per score MFMA
      f32x16 (&sn)[2] = sS[PAR ^ 1];
      const float mc = m_run * c;
      float rs[4] = {0.f, 0.f, 0.f, 0.f};
      frag kfr[NM];
      auto kread = [&](int i) __attribute__((always_inline)) { return lds_frag<T>(sK + kaddr[i >> 1] + (i & 1) * 32 * D * 2); };
      // LDS read-ahead: K fragments two MFMAs ahead, V^T fragments one (two
      // at D = 128, measured 2.4% faster there; deeper read-ahead measured
      // neutral at D <= 64).
      constexpr int LAK = 2, LAV = D >= 128 ? 2 : 1;
#pragma unroll
      for (int i = 0; i < LAK; ++i) kfr[i] = kread(i);
      sn[0] = zero16();
      sn[1] = zero16();
#pragma unroll
      for (int i = 0; i < NM; ++i) {
        if (i + LAK < NM) kfr[i + LAK] = kread(i + LAK);
        sn[i & 1] = M::mma(kfr[i], qf[i >> 1], sn[i & 1]);
#pragma unroll
        for (int e = 0; e < EPM; ++e) {
          const int idx = i * EPM + e, mt = idx >> 4, r = idx & 15;
          const float pv = fast_exp2(fmaf(s[mt][r], c, -mc));
          s[mt][r] = pv;
          if (idx < 4) rs[idx] = pv;
          else rs[r & 3] += pv;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);
      // Phase B: MFMA j = (mt, ks, dt) in order; V^T fragments LAV ahead.
      constexpr int NP = 4 * DT;
      auto vread = [&](int j) __attribute__((always_inline)) {
        const int mt = j / (2 * DT), ks = (j / DT) & 1, dt = j % DT;
        const int roff = (32 * mt + 16 * ks) * D * 2;
        return lds_frag_tr<T>(sV + vaddr[dt][0] + roff, sV + vaddr[dt][1] + roff);
      };
      frag vfr[NP];
      frag pb[4];
#pragma unroll
      for (int j = 0; j < LAV; ++j) vfr[j] = vread(j);
#pragma unroll
      for (int j = 0; j < NP; ++j) {
        if (j + LAV < NP) vfr[j + LAV] = vread(j + LAV);
        const int mt = j / (2 * DT), ks = (j / DT) & 1, dt = j % DT;
        if (dt == 0) pb[2 * mt + ks] = pack_frag<T>(s[mt], ks * 8);
        oacc[dt] = M::mma(vfr[j], pb[2 * mt + ks], oacc[dt]);
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
      if (nxt) scores(sS[PAR ^ 1], sK);
      if (cur) softmax_pv();
    }
  };

  // Folded sinks: query i >= span also sees keys j < n_i = min(fs, i - span
  // + 1), the sinks its window misses (the ring below covers the window).
  // They lie in the first ceil(fs / 64) key tiles, visited before the ring
  // starts: K and V of each through slot 0, which is then handed to the ring.
  const int fs = p.fold_sinks;
  const bool sink_visit = fs > 0 && q0 + BM - 1 >= p.window;
  if (sink_visit) {
    const bool wave_sinks = qw0 < p.S && qw0 + 31 >= p.window;
    const int n_i = max(0, min(fs, qi - p.window + 1));
    const int nst = (fs + BN - 1) / BN;
    for (int st = 0; st < nst; ++st) {
      issue_pair(0, st, st);
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      lds_barrier();
      if (st == 0) load_q();
      if (wave_sinks) {
        f32x16 (&s)[2] = sS[0];
        scores(s, kst(0));
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) mask_above(s[mt], (n_i - 1) - (st * BN + mt * 32 + 4 * g), -INFINITY);
        const float mx = max32(s[0], s[1]);
        if (st == 0) {
          // The first keys of the row: nothing to rescale yet.
          m_run = fmaxf(m_run, halves_max(mx));
        } else if (wave_any(mx > m_run + p.resc_th)) {
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
        float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int r = 0; r < 16; ++r) {
            const float pv = fast_exp2(fmaf(s[mt][r], c, -mc));
            s[mt][r] = pv;
            if (mt == 0 && r < 4) rs[r] = pv;   // first term: no add of 0.0 (kept for -0.0)
            else rs[r & 3] += pv;
          }
        l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);
        const char* sV = vst(0);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const frag pb = pack_frag<T>(s[mt], ks * 8);
            const int roff = (32 * mt + 16 * ks) * D * 2;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt)
              oacc[dt] = M::mma(lds_frag_tr<T>(sV + vaddr[dt][0] + roff, sV + vaddr[dt][1] + roff),
                                pb, oacc[dt]);
          }
      }
      lds_barrier();   // every wave's reads of slot 0 have returned
    }
    sank = wave_sinks;
  }

  // Prologue: units t_begin-1 .. t_begin+NS-2 into slots 0 .. NS-1, then the
  // scores of tile t_begin from slot 0.
#pragma unroll
  for (int i = 0; i < NS; ++i)
    if (t_begin - 1 + i <= t_end - 1) issue_unit(i, t_begin - 1 + i);
  // Retire the Q loads with a wait the compiler's wait-count pass sees;
  // otherwise it cannot prove the Q registers landed and drains every
  // in-flight unit before each tile's first MFMA.
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  lds_barrier();
  if (!sink_visit) load_q();
  if (tw_begin == t_begin && t_begin < tw_end) scores(sS[0], kst(0));

  for (int t = t_begin; t < t_end; t += C::UNROLL) {
    step(ic<0 % NS>{}, ic<0>{}, t);
    if (t + 1 < t_end) step(ic<1 % NS>{}, ic<1>{}, t + 1);
    if constexpr (C::UNROLL > 2) {
      if (t + 2 < t_end) step(ic<2 % NS>{}, ic<0>{}, t + 2);
      if (t + 3 < t_end) step(ic<3 % NS>{}, ic<1>{}, t + 3);
      if (t + 4 < t_end) step(ic<4 % NS>{}, ic<0>{}, t + 4);
      if (t + 5 < t_end) step(ic<5 % NS>{}, ic<1>{}, t + 5);
    }
  }

  const float l_tot = halves_sum(l_run);
  if (epi_lds_fwd<D>()) {
    // O (and its residual) through LDS in whole rows (store_rows_lds), staged
    // in the ring once every wave has finished reading it; 1 / l (and the
    // gate) per row.
    lds_barrier();
    const float inv = qi < p.S ? gate_sigmoid(p, b, qi, h) / l_tot : 0.f;
    const long long ow = (long long)b * p.S * p.q_rs + (long long)qw0 * p.q_rs + (long long)h * D;
    char* stage = &ring[0][0][0] + wave * (2 * 32 * D * 2);
    if (p.o_res) {
      store_rows_lds<T, D, true>(oacc, inv, stage, O + ow, p.q_rs, p.S - qw0, lane,
                                 reinterpret_cast<T*>(p.o_res) + ow);
    } else {
      store_rows_lds<T, D>(oacc, inv, stage, O + ow, p.q_rs, p.S - qw0, lane);
    }
    if (qi < p.S && g == 0) LSE[((long long)b * p.H + h) * p.S + qi] = m_run * p.scale + logf(l_tot);
  } else if (qi < p.S) {
    // Normalise, and apply the output gate sigma(z) of this query row when given.
    const float inv = gate_sigmoid(p, b, qi, h) / l_tot;
    const long long ooff = (long long)b * p.S * p.q_rs + (long long)qi * p.q_rs + (long long)h * D;
    T* Ob = O + ooff;
    if (p.o_res) {
      // O and its rounding residual (the backward's delta pass reads both).
      T* Rb = reinterpret_cast<T*>(p.o_res) + ooff;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          st_quad_res<T>(Ob + dt * 32 + 8 * j + 4 * g, Rb + dt * 32 + 8 * j + 4 * g,
                         oacc[dt][4 * j] * inv, oacc[dt][4 * j + 1] * inv,
                         oacc[dt][4 * j + 2] * inv, oacc[dt][4 * j + 3] * inv);
    } else {
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          st_quad<T>(Ob + dt * 32 + 8 * j + 4 * g, oacc[dt][4 * j] * inv, oacc[dt][4 * j + 1] * inv,
                     oacc[dt][4 * j + 2] * inv, oacc[dt][4 * j + 3] * inv);
    }
    if (g == 0) LSE[((long long)b * p.H + h) * p.S + qi] = m_run * p.scale + logf(l_tot);
  }
}

template <typename T, int D>
static hipError_t launch_fwd16_t(const void* q, const void* k, const void* v, void* o, float* lse,
                                 AttnParams p, hipStream_t st) {
  constexpr int BM = Fwd16<D>::BM;
  p.nblk = (p.S + BM - 1) / BM;
  const long long nblocks = (long long)p.nblk * p.B * p.H;
  p.wi_blocks_fastest = !p.causal;
  p.div_wi = p.wi_blocks_fastest ? work_item_div_blocks(p.nblk) : work_item_div((long long)p.B * p.H);
  if (p.block > 1) {   // block-causal variant
    hipLaunchKernelGGL((attn_fwd16_kernel<T, D, true>), dim3((unsigned)nblocks), dim3(256), 0, st,
                       (const T*)q, (const T*)k, (const T*)v, (T*)o, lse, p);
  } else {
    hipLaunchKernelGGL((attn_fwd16_kernel<T, D, false>), dim3((unsigned)nblocks), dim3(256), 0, st,
                       (const T*)q, (const T*)k, (const T*)v, (T*)o, lse, p);
  }
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
