// Flash-attention backward for 16-bit inputs (bf16 / f16) on gfx950: the
// dK/dV pass (over query tiles) and the dQ pass (over key tiles). The
// delta pass is shared with float32 (attn_bwd.hip). No atomics: every
// gradient is written once by the workgroup that owns its rows, so the
// results are bitwise reproducible.
//
// Algebra (nanolab/csrc/flash_attn_cuda.cu:8-14): p = exp(s*scale - L),
// dS = p*(dP - Delta), dQ = scale*dS K, dK = scale*dS^T Q, dV = p^T dO.
//
// Both kernels stream their tiles HBM -> LDS with buffer-resource LDS-DMA
// into a ring of NS slots (natural, swizzled layout; attn16.h), one barrier
// per tile (per two tiles in dK/dV at D <= 64), and read transposed operands
// with ds_read_b64_tr_b16:
//  * dQ (per 32-query wave): S^T = K Q^T and dP^T = V dO^T put one query per
//    lane (LSE and Delta are lane scalars); dQ^T += K^T dS^T takes dS^T from
//    registers and K^T from the K tile by transposed reads.
//  * dK/dV (per 32-key wave): S = Q K^T and dP = dO V^T put one key per lane;
//    dV^T += dO^T P and dK^T += Q^T dS take P / dS from registers and dO^T,
//    Q^T from the tiles by transposed reads. The GQA group is summed inside
//    the loop (query tiles of every head of the group).
// Within a tile the MFMAs are interleaved with the softmax-gradient VALU
// work in fixed slices (sched_barrier), so the matrix core runs while the
// wave computes exp / dS.
#include <type_traits>

#include "attn16.h"

namespace mi {

namespace {

template <int D>
struct Bwd16 {
  static constexpr int BW = 128;                 // rows a workgroup owns (4 waves x 32)
  static constexpr int BT = 64;                  // rows per streamed tile
  static constexpr int NS = D >= 128 ? 2 : 3;   // dQ's LDS ring depth
  // dK/dV: 4 slots filled and drained two tiles per barrier (D <= 64).
  static constexpr int NSK = D >= 128 ? 2 : 4;
  static constexpr int CH = D / 8;               // 16-byte chunks per tile row
  static constexpr int TILE = BT * D * 2;        // bytes of one 16-bit tile
  static constexpr int LPW = CH / 4;             // DMA instructions per wave per tile
  static constexpr int DS = D / 16, DT = D / 32;
};

// Per-lane byte offsets of the DMA lane map of a 64-row tile with row
// stride `rs` elements, shared by NW waves: instruction j of wave w fills LDS
// slots (NW j + w)*64 + lane, i.e. row slot / CH, physical chunk slot % CH.
template <int D, int NW = 4>
__device__ __forceinline__ void dma_offsets(unsigned (&voff)[Bwd16<D>::CH / NW], int wave, int lane,
                                            long long rs) {
  using C = Bwd16<D>;
#pragma unroll
  for (int j = 0; j < C::CH / NW; ++j) {
    const int slot = (NW * j + wave) * 64 + lane;
    const int row = slot / C::CH;
    voff[j] = (unsigned)(row * rs + ((slot % C::CH) ^ swz<D>(row)) * 8) * 2u;
  }
}

// Transposed-read base offsets: for output tile dt (32 columns of the tile),
// lane (G = lane >> 4, m = lane & 15) reads rows 4*(G>>1) + (m>>2) + 8h (+ 32mt
// + 16ks as immediates), columns dt*32 + 16*(G&1) + 4*(m&3).
template <int D>
__device__ __forceinline__ void tr_offsets(int (&toff)[Bwd16<D>::DT][2], int lane) {
  const int G = lane >> 4, m = lane & 15;
  const int row = 4 * (G >> 1) + (m >> 2);
#pragma unroll
  for (int dt = 0; dt < Bwd16<D>::DT; ++dt) {
    const int col = dt * 32 + 16 * (G & 1) + 4 * (m & 3);
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) toff[dt][hh] = tile_off<D>(row + 8 * hh, col >> 3) + (col & 7) * 2;
  }
}

template <int N>
__device__ __forceinline__ void wait_ring(int n) {
  if (n <= 0) wait_vm<0>();
  else if (n == 1) wait_vm<N>();
  else wait_vm<2 * N>();
}

template <int I>
using ic = std::integral_constant<int, I>;

// Rows per query head of the split dK/dV partials: S rounded up to 128
// (dkdv16_split_floats sizes them so, whatever the kernel's key block).
__host__ __device__ inline long long split_pitch(int S) { return (S + 127LL) / 128 * 128; }

// The rounding residual of 8 accumulator values (registers base .. base+7)
// against hi, their packed 16-bit fragment: (T)(x - (float)hi) per element.
// bf16: hi back in float32 straight from the packed pairs (a bf16 is the upper
// half of a float32; element 2i in the low half of word i), a shift or a mask
// per element; f16: a conversion. hi + lo carries x to ~16 significant bits.
template <typename T>
__device__ __forceinline__ typename Mfma32<T>::frag lo_frag(const f32x16& acc, int base,
                                                            typename Mfma32<T>::frag hi) {
  typename Mfma32<T>::frag lo;
  const u32x4 hw = __builtin_bit_cast(u32x4, hi);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float h;
    if constexpr (std::is_same_v<T, __bf16>) {
      const unsigned w = hw[e >> 1];
      h = __builtin_bit_cast(float, (e & 1) ? (w & 0xffff0000u) : (w << 16));
    } else {
      h = (float)hi[e];
    }
    lo[e] = (T)(acc[base + e] - h);
  }
  return lo;
}

}  // namespace

// ---------------------------------------------------------------------------
// dQ: per 128-query workgroup, loop over key tiles.
//
// FD (fused delta): the kernel also computes its rows' Delta = rowsum(dO * O)
// - dLSE from the dO fragments it holds and O read alongside, and writes the
// workspace's two planes (Delta, -L/scale) that the dK/dV pass reads; the
// backward then runs dQ before dK/dV and needs no separate delta pass. Each
// query row is owned by exactly one lane pair, so every plane entry is written
// once.
// ---------------------------------------------------------------------------
template <typename T, int D, bool BLK, bool FD>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 3 : 2, 8)))
attn_bwd16_dq_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                     const T* __restrict__ dO, const float* __restrict__ LSE,
                     const float* __restrict__ Delta, T* __restrict__ dQ, AttnParams p) {
  using C = Bwd16<D>;
  using M = Mfma32<T>;
  using frag = typename M::frag;
  constexpr int BM = C::BW, BN = C::BT, NS = C::NS, DS = C::DS, DT = C::DT;
  constexpr int LPU = 2 * C::LPW;
  // LDS ring: slot s holds the K tile (ring[s][0]) and V tile (ring[s][1]).
  __shared__ __attribute__((aligned(1024))) char ring[NS][2][C::TILE];
  auto kst = [&](int s) __attribute__((always_inline)) -> char* { return ring[s][0]; };
  auto vst = [&](int s) __attribute__((always_inline)) -> char* { return ring[s][1]; };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  const WorkItem wi = work_item(p.nblk, p.B * p.H, p.div_wi, p.causal, p.wi_blocks_fastest);
  const int bh = wi.bh;
  const int b = (int)fdiv((unsigned)bh, p.div_h), h = bh - b * p.H;
  const int hkv = (int)fdiv((unsigned)h, p.div_group);
  const int q0 = wi.blk * BM;
  const int qw0 = q0 + wave * 32;
  const int qi = qw0 + l32;

  const T* Qb = Q + (long long)b * p.S * p.q_rs + (long long)h * D;
  const T* dOb = dO + (long long)b * p.S * p.q_rs + (long long)h * D;

  frag qf[DS], dof[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) {
    const long long off = (long long)qi * p.q_rs + ds * 16 + g * 8;
    qf[ds] = (qi < p.S) ? ld_frag<T>(Qb + off) : zero_frag<T>();
    dof[ds] = (qi < p.S) ? ld_frag<T>(dOb + off) : zero_frag<T>();
  }
  float L2 = INFINITY, Dq = 0.f;
  // This row's LSE (and LSE gradient), loaded up front: with O by DMA the
  // delta is finished only after the ring's first wait.
  const long long ridx = ((long long)b * p.H + h) * p.S + qi;
  float Lrow = 0.f, dlrow = 0.f;
  if (FD && qi < p.S) {
    Lrow = LSE[ridx];
    if (p.dlse) dlrow = p.dlse[ridx];
  }
  // Fused delta, given this lane's partial dot product of dO and O (head dims
  // {16 ds + 8 g + e} of row qi; the lane 32 away holds the other half).
  auto finish_delta = [&](float part) __attribute__((always_inline)) {
    Dq = halves_sum(part);
    if (qi < p.S) {
      const long long idx = ridx;
      const float L = Lrow;
      L2 = L * kLog2e;
      Dq -= dlrow;
      if (g == 0) {
        p.ws_out[idx] = Dq;
        p.ws_out[(long long)p.B * p.H * p.S + idx] = L * (-1.f / p.scale);
      }
    }
  };
  // O of the workgroup's 128 rows by LDS-DMA into ring slot NS - 1, which the
  // ring first fills at its first step (three slots, D <= 64; no residual, no
  // sink visit), issued with the ring's first units: coalesced, and its
  // latency overlaps theirs (bitwise identical; backward A/B on one box: board
  // 118.0 -> 116.3 us, SWA(256) 237.7 -> 230.4 us, the E17 GQA shape and recall
  // within 0.5%). Otherwise O is loaded directly here.
  constexpr bool O_DMA_OK = FD && NS == 3;
  const bool o_dma = O_DMA_OK && !p.o_res && p.fold_sinks == 0;
  if constexpr (FD) {
    const long long hoff = (long long)b * p.S * p.q_rs + (long long)h * D;
    const T* Ob = reinterpret_cast<const T*>(p.o) + hoff;
    float part = 0.f;
    if (o_dma) {
      const RowTiles tOr = row_tiles(p.o, b, p.S, p.q_rs, h, D);
      unsigned ooff[C::LPW];
      dma_offsets<D>(ooff, wave, lane, p.q_rs);
      const unsigned m0o = lds_u32(ring[NS - 1][0] + wave * 1024);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const Rsrc ro = tile_rsrc(tOr, q0 / BN + half);
#pragma unroll
        for (int j = 0; j < C::LPW; ++j)
          dma16_buf(ro, ooff[j], m0o + (unsigned)(half * C::TILE + 4096 * j));
      }
    } else if (p.o_res) {
      // O as stored plus its rounding residual: Delta from O to ~16 bits
      // (with O alone, its 8-bit rounding enters every dS of the row).
      const T* Rb = reinterpret_cast<const T*>(p.o_res) + hoff;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const long long off = (long long)qi * p.q_rs + ds * 16 + g * 8;
        const frag of = (qi < p.S) ? ld_frag<T>(Ob + off) : zero_frag<T>();
        const frag orr = (qi < p.S) ? ld_frag<T>(Rb + off) : zero_frag<T>();
#pragma unroll
        for (int e = 0; e < 8; ++e) part = fmaf((float)of[e] + (float)orr[e], (float)dof[ds][e], part);
      }
    } else {
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const frag of = (qi < p.S) ? ld_frag<T>(Ob + (long long)qi * p.q_rs + ds * 16 + g * 8)
                                   : zero_frag<T>();
#pragma unroll
        for (int e = 0; e < 8; ++e) part = fmaf((float)of[e], (float)dof[ds][e], part);
      }
    }
    if (!o_dma) finish_delta(part);
  } else if (qi < p.S) {
    const long long idx = ((long long)b * p.H + h) * p.S + qi;
    L2 = LSE[idx] * kLog2e;
    Dq = Delta[idx];
  }

  int kbeg = 0, kend = p.S;
  if (p.causal) kend = min(p.S, causal_key_end<BLK>(p, q0 + BM - 1) + 1);
  if (p.window > 0) kbeg = max(0, q0 - p.window + 1);
  const int t_begin = kbeg / BN, t_end = (kend + BN - 1) / BN;
  int tw_begin = t_begin, tw_end = t_end;
  if (qw0 >= p.S) tw_end = tw_begin;
  if (p.causal) tw_end = min(tw_end, causal_key_end<BLK>(p, qw0 + 31) / BN + 1);
  if (p.window > 0) tw_begin = max(tw_begin, max(0, qw0 - p.window + 1) / BN);

  unsigned dvoff[C::LPW];
  dma_offsets<D>(dvoff, wave, lane, p.kv_rs);
  const unsigned m0w = lds_u32(ring[0][0] + wave * 1024);   // other DMA targets: constant offsets
  const RowTiles tK = row_tiles(K, b, p.S, p.kv_rs, hkv, D);
  const RowTiles tV = row_tiles(V, b, p.S, p.kv_rs, hkv, D);
  auto issue = [&](int slot, int t) __attribute__((always_inline)) {
    const Rsrc rk = tile_rsrc(tK, t);
    const Rsrc rv = tile_rsrc(tV, t);
#pragma unroll
    for (int j = 0; j < C::LPW; ++j) {
      dma16_buf(rk, dvoff[j], m0w + (unsigned)((2 * slot) * C::TILE + 4096 * j));
      dma16_buf(rv, dvoff[j], m0w + (unsigned)((2 * slot + 1) * C::TILE + 4096 * j));
    }
  };

  int kaddr[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) kaddr[ds] = tile_off<D>(l32, 2 * ds + g);
  int ktoff[DT][2];
  tr_offsets<D>(ktoff, lane);

  f32x16 dqacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqacc[dt] = zero16();
  f32x16 nd16;
#pragma unroll
  for (int r = 0; r < 16; ++r) nd16[r] = -Dq;
  const float c = p.scale_log2;
  const int key_hi = p.causal ? min(causal_key_end<BLK>(p, qi), p.S - 1) : p.S - 1;
  // The wave's smallest and largest key bounds (loop-invariant scalars).
  const int wave_key_lo_end = p.causal ? causal_key_end<BLK>(p, qw0) : p.S;
  const int wave_key_hi_end = p.causal ? causal_key_end<BLK>(p, qw0 + 31) : p.S;
  const int key_lo = p.window > 0 ? qi - p.window + 1 : 0;

  // One key tile in two halves of 32 keys (MFMA rows): each half computes
  // S^T, dP^T, P, dS^T and its dQ^T contribution before the next starts,
  // which keeps half the score registers live (three waves fit per SIMD)
  // and lets a causal diagonal skip a half that no query of the wave sees.
  // SINK: the folded-sink visit of sink tile t (keys j < n_i of query i;
  // halves at or past fs hold no sink) instead of a window step.
  auto compute = [&](const char* sK, const char* sV, int t, auto sink_c) __attribute__((always_inline)) {
    constexpr bool SINK = decltype(sink_c)::value;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt) {
      const int kb = t * BN + mt * 32;
      if (SINK && kb >= p.fold_sinks) continue;                           // no sink there
      if (!SINK && p.causal && kb > wave_key_hi_end) continue;            // above the diagonal
      if (!SINK && p.window > 0 && kb + 31 <= qw0 - p.window) continue;  // left of the window
      const bool need_hi = (kb + 32 > p.S) || (p.causal && kb + 31 > wave_key_lo_end);
      const bool need_lo = p.window > 0 && kb <= qw0 + 31 - p.window;
      const int roff0 = mt * 32 * D * 2;
      // S^T = K Q^T.
      frag kfr[DS], vfr[DS];
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) kfr[ds] = lds_frag<T>(sK + kaddr[ds] + roff0);
      f32x16 sacc = zero16();
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) sacc = M::mma(kfr[ds], qf[ds], sacc);
      // dP^T - Delta = V dO^T + (-Delta), interleaved with p = exp2(s*c - L2).
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) vfr[ds] = lds_frag<T>(sV + kaddr[ds] + roff0);
      f32x16 dpacc = nd16;
      constexpr int EPM = 16 / DS;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        dpacc = M::mma(vfr[ds], dof[ds], dpacc);
#pragma unroll
        for (int e = 0; e < EPM; ++e) sacc[ds * EPM + e] = fast_exp2(fmaf(sacc[ds * EPM + e], c, -L2));
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (SINK) {
        mask_above(sacc, (max(0, min(p.fold_sinks, qi - p.window + 1)) - 1) - (kb + 4 * g), 0.f);
      } else {
        if (need_hi) mask_above(sacc, key_hi - (kb + 4 * g), 0.f);
        if (need_lo) mask_below(sacc, key_lo - (kb + 4 * g), 0.f);
      }
      // dS^T = P * acc -> two fragments; dQ^T += K^T dS^T.
      frag sb[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int e = 0; e < 8; ++e) dpacc[ks * 8 + e] *= sacc[ks * 8 + e];
        sb[ks] = pack_frag<T>(dpacc, ks * 8);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int roff = roff0 + 16 * ks * D * 2;
          dqacc[dt] = M::mma(lds_frag_tr<T>(sK + ktoff[dt][0] + roff, sK + ktoff[dt][1] + roff), sb[ks],
                             dqacc[dt]);
        }
    }
  };

  auto step = [&](auto slot_c, int t) __attribute__((always_inline)) {
    constexpr int SL = decltype(slot_c)::value;
    wait_ring<LPU>(min(NS - 2, t_end - 1 - t));
    lds_barrier();
    if (t + NS - 1 < t_end) issue((SL + NS - 1) % NS, t + NS - 1);
    if (t >= tw_begin && t < tw_end) compute(kst(SL), vst(SL), t, std::false_type{});
  };

  // Folded sinks: query i >= span also sees keys j < n_i = min(fs, i - span
  // + 1), the sinks its window misses, in the first ceil(fs / 64) key tiles:
  // visited before the ring starts, each through slot 0.
  if (p.fold_sinks > 0 && q0 + BM - 1 >= p.window) {
    const int nst = (p.fold_sinks + BN - 1) / BN;
    for (int st = 0; st < nst; ++st) {
      issue(0, st);
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      lds_barrier();
      if (qw0 < p.S && qw0 + 31 >= p.window) compute(kst(0), vst(0), st, std::true_type{});
      lds_barrier();   // every wave's reads of slot 0 have returned
    }
  }

#pragma unroll
  for (int i = 0; i < NS - 1; ++i)
    if (t_begin + i < t_end) issue(i, t_begin + i);
  // Retire the Q / dO / LSE / Delta loads with a wait the compiler's
  // wait-count pass sees (otherwise it drains the ring inside the loop).
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  if constexpr (O_DMA_OK) {
    if (o_dma) {
      lds_barrier();
      const int orow = 32 * (wave & 1) + l32;
      float part = 0.f;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        const frag of = lds_frag<T>(ring[NS - 1][wave >> 1] + tile_off<D>(orow, 2 * ds + g));
#pragma unroll
        for (int e = 0; e < 8; ++e) part = fmaf((float)of[e], (float)dof[ds][e], part);
      }
      finish_delta(part);
#pragma unroll
      for (int r = 0; r < 16; ++r) nd16[r] = -Dq;
    }
  }
  for (int t = t_begin; t < t_end; t += NS) {
    step(ic<0>{}, t);
    if (t + 1 < t_end) step(ic<1>{}, t + 1);
    if constexpr (NS > 2) {
      if (t + 2 < t_end) step(ic<2 % NS>{}, t + 2);
    }
    if constexpr (NS > 3) {
      if (t + 3 < t_end) step(ic<3 % NS>{}, t + 3);
    }
  }

  if constexpr (epi_lds_dq<D>()) {
    lds_barrier();
    T* dQr = dQ + (long long)b * p.S * p.q_rs + (long long)qw0 * p.q_rs + (long long)h * D;
    store_rows_lds<T, D>(dqacc, p.scale, &ring[0][0][0] + wave * (32 * D * 2), dQr, p.q_rs,
                         p.S - qw0, lane);
  } else if (qi < p.S) {
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
// dK / dV: per 128-key workgroup, loop over (group head, query tile).
//
// Both score-like products start from an accumulator seeded out of LDS
// instead of zero, which removes per-element work from the softmax-gradient
// VALU stream:
//   S'  = Q K^T + (-L/scale)          -> p  = exp2(scale_log2 * S')
//   dP' = dO (-V)^T + Delta = Delta - dP  -> dS' = p * dP' = -dS
// (-L/scale and Delta come from the delta workspace; V is negated once in
// registers, exactly.) dK = scale * dS^T Q is then stored as -scale * dS'^T Q.
// ---------------------------------------------------------------------------
template <typename T, int D, bool BLK, bool SSPLIT, int NW>
__global__ void __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(D <= 64 ? 2 : 1, 8)))
attn_bwd16_dkdv_kernel(const T* __restrict__ Q, const T* __restrict__ K, const T* __restrict__ V,
                       const T* __restrict__ dO, const float* __restrict__ WS,
                       T* __restrict__ dK, T* __restrict__ dV, AttnParams p) {
  using C = Bwd16<D>;
  using M = Mfma32<T>;
  using frag = typename M::frag;
  // NW waves of 32 keys each. Four waves (128 keys) share the paired 4-slot
  // ring; two waves (64 keys) a 2-slot ring, at half the LDS per workgroup.
  constexpr int BK = 32 * NW, BQ = C::BT, DS = C::DS, DT = C::DT;
  constexpr int NS = NW == 2 ? 2 : C::NSK;
  constexpr int LPW = C::CH / NW;          // DMA instructions per wave per tile
  constexpr int VPW = 64 / NW;             // vector entries per wave per tile
  constexpr int LPU = 2 * LPW + 2;         // Q, dO tiles + -L/scale, Delta vectors
  // LDS ring: slot s holds the Q tile (ring[s][0]), the dO tile (ring[s][1])
  // and the tile's [-L/scale | Delta] vectors (vecs[s]).
  __shared__ __attribute__((aligned(1024))) char ring[NS][2][C::TILE];
  __shared__ __attribute__((aligned(16))) float vecs_lds[NS][2 * BQ];
  auto qst = [&](int s) __attribute__((always_inline)) -> char* { return ring[s][0]; };
  auto ost = [&](int s) __attribute__((always_inline)) -> char* { return ring[s][1]; };
  auto lst = [&](int s) __attribute__((always_inline)) -> float* { return vecs_lds[s]; };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, g = lane >> 5;
  // Work item (b, kv head, key block) and, when the group is split, the one
  // query head of the group this workgroup walks (otherwise all of them).
  const int nsplit = p.kv_split;
  const WorkItem wi = work_item(p.nblk, p.B * p.Hkv * nsplit, p.div_wi, false, p.wi_blocks_fastest);
  const int bhk = nsplit > 1 ? (int)fdiv((unsigned)wi.bh, p.div_group) : wi.bh;   // nsplit == group
  const int b = (int)fdiv((unsigned)bhk, p.div_hkv), hkv = bhk - b * p.Hkv;
  const int g_first = nsplit > 1 ? wi.bh - bhk * nsplit : 0;    // first group head walked
  const int g_count = nsplit > 1 ? 1 : p.group;           // group heads walked
  const int h_first = hkv * p.group + g_first;
  const int k0 = wi.blk * BK;
  const int kw0 = k0 + wave * 32;
  const int kj = kw0 + l32;

  // K (B operand of S) and -V (B operand of dP') for the wave's 32 keys: with
  // the 4-slot ring (D <= 64) by LDS-DMA through ring slots 2 and 3 before the
  // ring starts (below); otherwise by global loads here, 16 bytes per lane and
  // row, which touch 32 rows per instruction (measured: the DMA path takes
  // dK/dV 4-7% faster, the workgroups' wait for their first operands being
  // ~20% of their time).
  constexpr bool KV_DMA = NS == 4;
  // Two waves: the block's K and V tiles (64 rows each) by LDS-DMA into ring
  // slot 1 before the ring starts; its first step's barrier frees the slot.
  constexpr bool KV_STAGE = NW == 2;
  frag kf[DS], vf[DS];
  if constexpr (!KV_DMA && !KV_STAGE) {
    const T* Kb = K + (long long)b * p.S * p.kv_rs + (long long)hkv * D;
    const T* Vb = V + (long long)b * p.S * p.kv_rs + (long long)hkv * D;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const long long off = (long long)kj * p.kv_rs + ds * 16 + g * 8;
      kf[ds] = (kj < p.S) ? ld_frag<T>(Kb + off) : zero_frag<T>();
      frag vv = (kj < p.S) ? ld_frag<T>(Vb + off) : zero_frag<T>();
      u32x4 bits = __builtin_bit_cast(u32x4, vv);
      bits ^= 0x80008000u;                       // sign of every 16-bit element
      vf[ds] = __builtin_bit_cast(frag, bits);
    }
  }

  // Query tiles of the workgroup and of this wave (wave-uniform scalars).
  // Folded sinks (keys < fs): every query from the key on sees them, so a
  // key block holding any walks the query tiles to the end (work_item starts
  // the low key blocks first) and the sink lanes keep an upper bound of S - 1.
  const int fs = p.fold_sinks;
  int qbeg = 0, qend = p.S;
  if (p.causal) qbeg = causal_query_begin<BLK>(p, k0);
  if (p.window > 0 && k0 >= fs) qend = min(p.S, k0 + BK - 1 + p.window);
  const int tq_begin = qbeg / BQ;
  const int tq_end = max(tq_begin, (qend + BQ - 1) / BQ);
  const int ntq = tq_end - tq_begin;
  const int niter = g_count * ntq;
  int tw_begin = tq_begin, tw_end = tq_end;     // absolute query-tile range of this wave
  if (kw0 >= p.S) tw_end = tw_begin;
  if (p.causal) tw_begin = max(tw_begin, causal_query_begin<BLK>(p, kw0) / BQ);
  if (p.window > 0 && kw0 >= fs) tw_end = min(tw_end, (kw0 + 31 + p.window - 1) / BQ + 1);

  unsigned dvoff[LPW];
  dma_offsets<D, NW>(dvoff, wave, lane, p.q_rs);
  // LDS addresses of this wave's first tile chunk and first vector entry;
  // every other DMA target is a constant offset from one of them.
  const unsigned m0w = lds_u32(ring[0][0] + wave * 1024);
  const unsigned m0v = lds_u32(vecs_lds[0] + wave * VPW);
  const long long plane = (long long)p.B * p.H * p.S;
  // Issue position (group head, query tile), advanced one unit per issue;
  // the head's tile descriptors are rebuilt only when the head changes.
  int is_gh = 0, is_tq = tq_begin;
  RowTiles tQ = row_tiles(Q, b, p.S, p.q_rs, h_first, D);
  RowTiles tO = row_tiles(dO, b, p.S, p.q_rs, h_first, D);
  const float* vecs = WS + ((long long)b * p.H + h_first) * p.S;   // plane 0 of the head
  auto issue = [&](int slot) __attribute__((always_inline)) {
    const Rsrc rq = tile_rsrc(tQ, is_tq);
    const Rsrc ro = tile_rsrc(tO, is_tq);
#pragma unroll
    for (int j = 0; j < LPW; ++j) {
      dma16_buf(rq, dvoff[j], m0w + (unsigned)((2 * slot) * C::TILE + NW * 1024 * j));
      dma16_buf(ro, dvoff[j], m0w + (unsigned)((2 * slot + 1) * C::TILE + NW * 1024 * j));
    }
    // -L/scale and Delta rows of the tile: VPW floats per wave each.
    const int row0 = is_tq * BQ;
    const unsigned vbytes = (unsigned)min(max(0, p.S - row0), BQ) * 4u;
    const Rsrc rl = make_rsrc(vecs + plane + row0, vbytes);
    const Rsrc rd = make_rsrc(vecs + row0, vbytes);
    if (lane < VPW) {
      dma4_buf(rl, (unsigned)(wave * VPW + lane) * 4u, m0v + (unsigned)(slot * 2 * BQ * 4));
      dma4_buf(rd, (unsigned)(wave * VPW + lane) * 4u, m0v + (unsigned)((slot * 2 * BQ + BQ) * 4));
    }
    if (++is_tq == tq_end) {
      is_tq = tq_begin;
      if (++is_gh < g_count) {
        const int h = h_first + is_gh;
        tQ = row_tiles(Q, b, p.S, p.q_rs, h, D);
        tO = row_tiles(dO, b, p.S, p.q_rs, h, D);
        vecs += p.S;
      }
    }
  };

  int qaddr[DS];
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) qaddr[ds] = tile_off<D>(l32, 2 * ds + g);
  int ttoff[DT][2];
  tr_offsets<D>(ttoff, lane);

  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dkacc[dt] = zero16();
    dvacc[dt] = zero16();
  }
  const float c = p.scale_log2;
  // Queries that see key kj: [q_lo, q_hi] (rows past S are zeros: masked).
  const int q_lo = p.causal ? causal_query_begin<BLK>(p, kj) : 0;
  const int wave_q_lo = p.causal ? causal_query_begin<BLK>(p, kw0 + 31) : 0;   // largest q_lo of the wave
  const int q_hi = (p.window > 0 && kj >= fs) ? min(p.S - 1, kj + p.window - 1) : p.S - 1;

  // Accumulator seeded from a per-query LDS vector: register r of lane group g
  // is query row crow(r, g) of the 32-row tile mt, i.e. four consecutive
  // floats per ds_read_b128.
  auto seed = [&](const float* vec, int mt) __attribute__((always_inline)) {
    f32x16 a;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const f32x4 v4 = *reinterpret_cast<const f32x4*>(vec + mt * 32 + 8 * j + 4 * g);
      a[4 * j] = v4[0];
      a[4 * j + 1] = v4[1];
      a[4 * j + 2] = v4[2];
      a[4 * j + 3] = v4[3];
    }
    return a;
  };

  // LDS reads run ahead of the MFMAs that consume them: Q fragments four
  // MFMAs ahead, the first dO fragments and both seeds before the S MFMAs,
  // the first transposed pairs before the dP MFMAs, then two pairs ahead
  // (measured best of the lookaheads tried, within the 256-VGPR budget; D =
  // 128 holds twice the fragments and keeps the shorter 2 / 2 / 1).
  constexpr int LA_S = D <= 64 ? 4 : 2, LA_P = D <= 64 ? 4 : 2, LA_T = D <= 64 ? 2 : 1;
  auto compute = [&](const char* sQ, const char* sO, const float* sLD, int tq) __attribute__((always_inline)) {
    const int q0 = tq * BQ;
    const bool need_lo = p.causal && q0 < wave_q_lo;
    const bool need_hi = (q0 + BQ > p.S) || (p.window > 0 && q0 + BQ - 1 - p.window >= kw0);
    constexpr int NM = 2 * DS;
    f32x16 sacc[2], dpacc[2];
    auto qread = [&](int i) __attribute__((always_inline)) { return lds_frag<T>(sQ + qaddr[i >> 1] + (i & 1) * 32 * D * 2); };
    auto oread = [&](int i) __attribute__((always_inline)) { return lds_frag<T>(sO + qaddr[i >> 1] + (i & 1) * 32 * D * 2); };
    constexpr int NP = 4 * DT;
    auto tread = [&](const char* tile, int j) __attribute__((always_inline)) {
      const int mt = j / (2 * DT), ks = (j / DT) & 1, dt = j % DT;
      const int roff = (32 * mt + 16 * ks) * D * 2;
      return lds_frag_tr<T>(tile + ttoff[dt][0] + roff, tile + ttoff[dt][1] + roff);
    };
    // S' = Q K^T - L/scale (rows = queries).
    frag fr[NM], orr[NM];
#pragma unroll
    for (int i = 0; i < LA_S && i < NM; ++i) fr[i] = qread(i);
    sacc[0] = seed(sLD, 0);
    sacc[1] = seed(sLD, 1);
#pragma unroll
    for (int i = 0; i < LA_P && i < NM; ++i) orr[i] = oread(i);
    dpacc[0] = seed(sLD + BQ, 0);
    dpacc[1] = seed(sLD + BQ, 1);
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      if (i + LA_S < NM) fr[i + LA_S] = qread(i + LA_S);
      sacc[i & 1] = M::mma(fr[i], kf[i >> 1], sacc[i & 1]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // dP' = Delta - dO V^T interleaved with p = exp2(c * S').
    frag to[NP], tqf[NP];
#pragma unroll
    for (int j = 0; j < LA_T && j < NP; ++j) {
      to[j] = tread(sO, j);
      tqf[j] = tread(sQ, j);
    }
    constexpr int EPM = 32 / NM;
#pragma unroll
    for (int i = 0; i < NM; ++i) {
      if (i + LA_P < NM) orr[i + LA_P] = oread(i + LA_P);
      dpacc[i & 1] = M::mma(orr[i], vf[i >> 1], dpacc[i & 1]);
#pragma unroll
      for (int e = 0; e < EPM; ++e) {
        const int idx = i * EPM + e, mt = idx >> 4, r = idx & 15;
        sacc[mt][r] = fast_exp2(sacc[mt][r] * c);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (need_lo) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) mask_below(sacc[mt], q_lo - (q0 + mt * 32 + 4 * g), 0.f);
    }
    if (need_hi) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) mask_above(sacc[mt], q_hi - (q0 + mt * 32 + 4 * g), 0.f);
    }
    // dV^T += dO^T P and dK^T += Q^T dS': MFMA pairs j = (mt, ks, dt), dS'
    // of a fragment computed on first use.
    // SPLIT (D = 128): dS' enters the dK product as two 16-bit terms, its
    // rounding hi and the rounding of the residual dS' - hi, so dK carries
    // dS' to ~16 significant bits instead of 8 (Q is exact in its own type).
    // A dK element sums up to S products whose large terms cancel; with one
    // 16-bit dS' its rounding errors reached 4e-2 on the long config's dK
    // (S 8192, q ~ 2 N(0,1)), twice the 2e-2 bar. The cost is one more MFMA
    // per dK pair and the residual's subtract and pack.
    constexpr bool SPLIT = D >= 128;
    // SSPLIT (folded sinks): the waves holding sink keys (keys < fs) split
    // both P (dV) and dS' (dK) into hi + lo. A sink key's dV and dK
    // sum P dO and dS' Q over every query row from the key on (a whole
    // sequence, not a window span), with P ~ 1/span on each row: one 16-bit
    // rounding per term then accumulates over the rows. With the split the
    // operands carry ~16 bits and what remains is the output's own rounding.
    const bool sw = SSPLIT && kw0 < fs;
    frag pb[4], sb[4], sl[SPLIT || SSPLIT ? 4 : 1], pl[SSPLIT ? 4 : 1];
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      if (j + LA_T < NP) {
        to[j + LA_T] = tread(sO, j + LA_T);
        tqf[j + LA_T] = tread(sQ, j + LA_T);
      }
      const int mt = j / (2 * DT), ks = (j / DT) & 1, dt = j % DT;
      if (dt == 0) {
        const int f = 2 * mt + ks;
        pb[f] = pack_frag<T>(sacc[mt], ks * 8);
#pragma unroll
        for (int e = 0; e < 8; ++e) dpacc[mt][ks * 8 + e] *= sacc[mt][ks * 8 + e];
        sb[f] = pack_frag<T>(dpacc[mt], ks * 8);
        if constexpr (SPLIT) {
          sl[f] = lo_frag<T>(dpacc[mt], ks * 8, sb[f]);
        } else if constexpr (SSPLIT) {
          if (sw) sl[f] = lo_frag<T>(dpacc[mt], ks * 8, sb[f]);
        }
        if constexpr (SSPLIT) {
          if (sw) pl[f] = lo_frag<T>(sacc[mt], ks * 8, pb[f]);
        }
      }
      dvacc[dt] = M::mma(to[j], pb[2 * mt + ks], dvacc[dt]);
      if constexpr (SSPLIT) {
        if (sw) dvacc[dt] = M::mma(to[j], pl[2 * mt + ks], dvacc[dt]);
      }
      dkacc[dt] = M::mma(tqf[j], sb[2 * mt + ks], dkacc[dt]);
      if constexpr (SPLIT) {
        dkacc[dt] = M::mma(tqf[j], sl[2 * mt + ks], dkacc[dt]);
      } else if constexpr (SSPLIT) {
        if (sw) dkacc[dt] = M::mma(tqf[j], sl[2 * mt + ks], dkacc[dt]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Compute position, advanced one unit per step.
  int cp_tq = tq_begin;
  auto step = [&](auto slot_c, int it) __attribute__((always_inline)) {
    constexpr int SL = decltype(slot_c)::value;
    wait_ring<LPU>(min(NS - 2, niter - 1 - it));
    lds_barrier();
    if (it + NS - 1 < niter) issue((SL + NS - 1) % NS);
    if (cp_tq >= tw_begin && cp_tq < tw_end) compute(qst(SL), ost(SL), lst(SL), cp_tq);
    if (++cp_tq == tq_end) cp_tq = tq_begin;
  };

  if constexpr (NS == 4) {
    // Two tiles per barrier: tiles it and it+1 land, the barrier, then tiles
    // it+2 and it+3 go into the slots that tiles it-2 and it-1 held. Half the
    // barriers of one tile per step, so a wave waits for the slowest of the
    // workgroup half as often (measured 2% faster at D <= 64; at D = 128 the
    // four 32 KB slots were slower than two).
    auto pstep = [&](auto slot_c, int it) __attribute__((always_inline)) {
      constexpr int SL = decltype(slot_c)::value;
      wait_vm<0>();
      lds_barrier();
      if (it + 2 < niter) issue((SL + 2) % 4);
      if (it + 3 < niter) issue((SL + 3) % 4);
      if (cp_tq >= tw_begin && cp_tq < tw_end) compute(qst(SL), ost(SL), lst(SL), cp_tq);
      if (++cp_tq == tq_end) cp_tq = tq_begin;
      if (it + 1 < niter) {
        if (cp_tq >= tw_begin && cp_tq < tw_end) compute(qst(SL + 1), ost(SL + 1), lst(SL + 1), cp_tq);
        if (++cp_tq == tq_end) cp_tq = tq_begin;
      }
    };
    if constexpr (KV_DMA) {
      // The block's K and V rows (two 64-row tiles each) by LDS-DMA into ring
      // slots 2 (K) and 3 (V), coalesced like the Q / dO tiles (rows past S
      // read as zeros), read into registers; the first step's barrier then
      // hands slots 2 and 3 back to the ring.
      const RowTiles tK = row_tiles(K, b, p.S, p.kv_rs, hkv, D);
      const RowTiles tV = row_tiles(V, b, p.S, p.kv_rs, hkv, D);
      unsigned kvoff[LPW];
      dma_offsets<D, NW>(kvoff, wave, lane, p.kv_rs);
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const Rsrc rk = tile_rsrc(tK, k0 / BQ + half);
        const Rsrc rv = tile_rsrc(tV, k0 / BQ + half);
#pragma unroll
        for (int j = 0; j < LPW; ++j) {
          dma16_buf(rk, kvoff[j], m0w + (unsigned)((2 * 2 + half) * C::TILE + NW * 1024 * j));
          dma16_buf(rv, kvoff[j], m0w + (unsigned)((2 * 3 + half) * C::TILE + NW * 1024 * j));
        }
      }
    }
    if (0 < niter) issue(0);
    if (1 < niter) issue(1);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    if constexpr (KV_DMA) {
      lds_barrier();
      const int krow = 32 * (wave & 1) + l32;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        kf[ds] = lds_frag<T>(ring[2][wave >> 1] + tile_off<D>(krow, 2 * ds + g));
        frag vv = lds_frag<T>(ring[3][wave >> 1] + tile_off<D>(krow, 2 * ds + g));
        u32x4 bits = __builtin_bit_cast(u32x4, vv);
        bits ^= 0x80008000u;                     // sign of every 16-bit element
        vf[ds] = __builtin_bit_cast(frag, bits);
      }
    }
    for (int it = 0; it < niter; it += 4) {
      pstep(ic<0>{}, it);
      if (it + 2 < niter) pstep(ic<2>{}, it + 2);
    }
  } else {
    if constexpr (KV_STAGE) {
      // K tile k0/64 -> ring[1][0], V tile -> ring[1][1] (rows past S read as zeros).
      const RowTiles tK = row_tiles(K, b, p.S, p.kv_rs, hkv, D);
      const RowTiles tV = row_tiles(V, b, p.S, p.kv_rs, hkv, D);
      unsigned kvoff[LPW];
      dma_offsets<D, NW>(kvoff, wave, lane, p.kv_rs);
      const Rsrc rk = tile_rsrc(tK, k0 / BQ);
      const Rsrc rv = tile_rsrc(tV, k0 / BQ);
#pragma unroll
      for (int j = 0; j < LPW; ++j) {
        dma16_buf(rk, kvoff[j], m0w + (unsigned)(2 * C::TILE + NW * 1024 * j));
        dma16_buf(rv, kvoff[j], m0w + (unsigned)(3 * C::TILE + NW * 1024 * j));
      }
    }
#pragma unroll
    for (int i = 0; i < NS - 1; ++i)
      if (i < niter) issue(i);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    if constexpr (KV_STAGE) {
      lds_barrier();
      const int krow = 32 * wave + l32;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        kf[ds] = lds_frag<T>(ring[1][0] + tile_off<D>(krow, 2 * ds + g));
        frag vv = lds_frag<T>(ring[1][1] + tile_off<D>(krow, 2 * ds + g));
        u32x4 bits = __builtin_bit_cast(u32x4, vv);
        bits ^= 0x80008000u;                     // sign of every 16-bit element
        vf[ds] = __builtin_bit_cast(frag, bits);
      }
    }
    for (int it = 0; it < niter; it += NS) {
      step(ic<0>{}, it);
      if (it + 1 < niter) step(ic<1>{}, it + 1);
      if constexpr (NS > 2) {
        if (it + 2 < niter) step(ic<2 % NS>{}, it + 2);
      }
      if constexpr (NS > 3) {
        if (it + 3 < niter) step(ic<3 % NS>{}, it + 3);
      }
    }
  }

  // The branches on nsplit and epi_lds_dkdv are uniform over the workgroup, so
  // every wave meets the LDS path's barrier or none does.
  if (nsplit > 1) {
    if (kj >= p.S) return;
    // fp32 partials of this query head; the reduce kernel adds the group's.
    float* dst = p.kv_part + ((long long)(b * p.H + h_first) * split_pitch(p.S) + kj) * (2 * D);
    const float sc = -p.scale;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int d0 = dt * 32 + 8 * j + 4 * g;
        f32x4 a, c4;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          a[e] = dkacc[dt][4 * j + e] * sc;
          c4[e] = dvacc[dt][4 * j + e];
        }
        *reinterpret_cast<f32x4*>(dst + d0) = a;
        *reinterpret_cast<f32x4*>(dst + D + d0) = c4;
      }
  } else if (epi_lds_dkdv<D>()) {
    // Whole rows through LDS (store_rows_lds), staged in the ring once every
    // wave has finished reading it.
    lds_barrier();
    char* stage = &ring[0][0][0] + wave * (2 * 32 * D * 2);
    const long long off = (long long)b * p.S * p.kv_rs + (long long)kw0 * p.kv_rs + (long long)hkv * D;
    store_rows_lds<T, D>(dkacc, -p.scale, stage, dK + off, p.kv_rs, p.S - kw0, lane);
    store_rows_lds<T, D>(dvacc, 1.f, stage + 32 * D * 2, dV + off, p.kv_rs, p.S - kw0, lane);
  } else if (kj < p.S) {
    const long long off = (long long)b * p.S * p.kv_rs + (long long)kj * p.kv_rs + (long long)hkv * D;
    T* dKr = dK + off;
    T* dVr = dV + off;
    const float sc = -p.scale;
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
// Sum of the split dK/dV partials over the GQA group, in head order (so the
// result does not depend on which workgroup finished first): one thread per
// 8 consecutive elements of one key row of dK or dV.
// ---------------------------------------------------------------------------
template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_dkdv16_reduce_kernel(const float* __restrict__ part, T* __restrict__ dK, T* __restrict__ dV,
                          AttnParams p, long long total) {
  constexpr int C8 = D / 8;
  const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
  if (t >= total) return;
  const int c8 = (int)(t % C8);
  long long r = t / C8;
  const int which = (int)(r & 1);      // 0: dK, 1: dV
  r >>= 1;
  const int j = (int)(r % p.S);
  r /= p.S;
  const int hkv = (int)(r % p.Hkv), b = (int)(r / p.Hkv);
  const long long rows = split_pitch(p.S);
  const float* src = part + (((long long)b * p.H + hkv * p.group) * rows + j) * (2 * D) + which * D + c8 * 8;
  f32x4 a = *reinterpret_cast<const f32x4*>(src);
  f32x4 c = *reinterpret_cast<const f32x4*>(src + 4);
  for (int h = 1; h < p.group; ++h) {
    src += rows * (2 * D);
    a += *reinterpret_cast<const f32x4*>(src);
    c += *reinterpret_cast<const f32x4*>(src + 4);
  }
  T* dst = (which ? dV : dK) + ((long long)b * p.S + j) * p.kv_rs + (long long)hkv * D + c8 * 8;
  st_quad<T>(dst, a[0], a[1], a[2], a[3]);
  st_quad<T>(dst + 4, c[0], c[1], c[2], c[3]);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
template <typename T, int D>
static hipError_t launch_dq16_t(const void* q, const void* k, const void* v, const void* dout,
                                const float* lse, const float* delta, void* dq, AttnParams p,
                                hipStream_t st) {
  p.nblk = (p.S + Bwd16<D>::BW - 1) / Bwd16<D>::BW;
  const long long nblocks = (long long)p.nblk * p.B * p.H;
  p.wi_blocks_fastest = !p.causal;
  p.div_wi = p.wi_blocks_fastest ? work_item_div_blocks(p.nblk) : work_item_div((long long)p.B * p.H);
  // Variants: block-causal (BLK) x delta fused in (FD, when p.o is set).
  const auto go = [&](auto blk_c, auto fd_c) {
    hipLaunchKernelGGL((attn_bwd16_dq_kernel<T, D, decltype(blk_c)::value, decltype(fd_c)::value>),
                       dim3((unsigned)nblocks), dim3(256), 0, st, (const T*)q, (const T*)k,
                       (const T*)v, (const T*)dout, lse, delta, (T*)dq, p);
  };
  using yes = std::true_type;
  using no = std::false_type;
  if (p.block > 1) {
    if (p.o) go(yes{}, yes{}); else go(yes{}, no{});
  } else {
    if (p.o) go(no{}, yes{}); else go(no{}, no{});
  }
  return hipGetLastError();
}

// Waves per workgroup (32 keys each): four (128 keys, the paired 4-slot ring)
// by default; two (64 keys, a 2-slot ring, twice the resident workgroups) for
// folded sinks at D <= 64, where the key blocks holding sinks walk every query
// tile and a 64-key block halves that walk's wave-tiles. Measured, A/B on
// one box: SWA(64, 4) backward 76.4 -> 73.3 us; the board 119.0 -> 121.0 us,
// SWA(256) 237.7 -> 243.7 us and recall 946 -> 983 us with two waves, which
// lose the paired ring, so they keep four.
template <typename T, int D, int NW>
static hipError_t launch_dkdv16_nw(const void* q, const void* k, const void* v, const void* dout,
                                   const float* delta, void* dk, void* dv, AttnParams p,
                                   hipStream_t st) {
  p.nblk = (p.S + 32 * NW - 1) / (32 * NW);
  const long long nblocks = (long long)p.nblk * p.B * p.Hkv * p.kv_split;
  p.wi_blocks_fastest = !p.causal;
  p.div_wi = p.wi_blocks_fastest ? work_item_div_blocks(p.nblk)
                                 : work_item_div((long long)p.B * p.Hkv * p.kv_split);
  // Variants: block-causal (BLK), folded sinks with split sink-key operands
  // (SSPLIT; sinks need a window, which excludes block-causal masks).
  const auto go = [&](auto blk_c, auto ss_c) {
    hipLaunchKernelGGL((attn_bwd16_dkdv_kernel<T, D, decltype(blk_c)::value, decltype(ss_c)::value, NW>),
                       dim3((unsigned)nblocks), dim3(64 * NW), 0, st, (const T*)q, (const T*)k,
                       (const T*)v, (const T*)dout, delta, (T*)dk, (T*)dv, p);
  };
  if constexpr (NW == 2) {
    go(std::false_type{}, std::true_type{});
  } else {
    if (p.block > 1) go(std::true_type{}, std::false_type{});
    else if (p.fold_sinks > 0) go(std::false_type{}, std::true_type{});
    else go(std::false_type{}, std::false_type{});
  }
  return hipGetLastError();
}

template <typename T, int D>
static hipError_t launch_dkdv16_t(const void* q, const void* k, const void* v, const void* dout,
                                  const float* lse, const float* delta, void* dk, void* dv,
                                  AttnParams p, hipStream_t st) {
  if (p.kv_split < 1 || (p.kv_split > 1 && (p.kv_split != p.group || !p.kv_part)))
    return hipErrorInvalidValue;
  (void)lse;   // the kernels read -L/scale from plane 1 of the delta workspace
  hipError_t e = hipSuccess;
  if constexpr (D <= 64) {
    if (p.fold_sinks > 0) e = launch_dkdv16_nw<T, D, 2>(q, k, v, dout, delta, dk, dv, p, st);
    else e = launch_dkdv16_nw<T, D, 4>(q, k, v, dout, delta, dk, dv, p, st);
  } else {
    e = launch_dkdv16_nw<T, D, 4>(q, k, v, dout, delta, dk, dv, p, st);
  }
  if (e != hipSuccess) return e;
  if (p.kv_split > 1) {
    const long long total = (long long)p.B * p.Hkv * p.S * 2 * (D / 8);
    hipLaunchKernelGGL((attn_dkdv16_reduce_kernel<T, D>), dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, st, p.kv_part, (T*)dk, (T*)dv, p, total);
  }
  return hipGetLastError();
}

#define MI_DISPATCH16(dtype, D, CALL)                                  \
  switch (dtype) {                                                     \
    case 1:                                                            \
      switch (D) {                                                     \
        case 32: { using T = _Float16; constexpr int DD = 32; CALL; }   \
        case 64: { using T = _Float16; constexpr int DD = 64; CALL; }   \
        case 128: { using T = _Float16; constexpr int DD = 128; CALL; } \
      }                                                                \
      break;                                                           \
    case 2:                                                            \
      switch (D) {                                                     \
        case 32: { using T = __bf16; constexpr int DD = 32; CALL; }     \
        case 64: { using T = __bf16; constexpr int DD = 64; CALL; }     \
        case 128: { using T = __bf16; constexpr int DD = 128; CALL; }   \
      }                                                                \
      break;                                                           \
  }                                                                    \
  return hipErrorInvalidValue;

// Compute units of the current device (hipDeviceAttributeMultiprocessorCount),
// cached per device; 256 (MI355X) if the query fails.
static int device_cus() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cache[dev] = n;
  }
  return cache[dev];
}

// Largest split-partial area (fp32 floats) the split may take: 64 MiB. Above it
// (long-context GQA / MQA, where the unsplit grid is small but B*H*S*D is
// large) the unsplit kernel runs and needs no partials.
constexpr long long kSplitCapFloats = 16LL << 20;

// The GQA group is split across workgroups (one query head each, fp32
// partials summed by a reduce kernel) when the unsplit grid of (batch, kv
// head, key block) workgroups fills the chip less than twice at the kernel's
// occupancy (the device's CUs x two workgroups for D <= 64, x one for D =
// 128) and the partials fit kSplitCapFloats: then the longest key block's walk
// over every head of the group sets the kernel time (the E17 shape, B8
// H12/Hkv4 S1024: 256 workgroups on 512 slots, key block 0 walking 48 query
// tiles against 27 on average). The decision depends only on the shape and
// the current device, so mi_attn_bwd_workspace and the launch agree.
int dkdv16_split(const AttnParams& p, int D) {
  if (p.group <= 1) return 1;
  const long long nblk = (p.S + Bwd16<64>::BW - 1) / Bwd16<64>::BW;
  const long long wgs = nblk * p.B * p.Hkv;
  const long long per_cu = D <= 64 ? 2 : 1;
  if (wgs >= 2 * per_cu * device_cus()) return 1;
  if ((long long)p.B * p.H * nblk * Bwd16<64>::BW * 2 * D > kSplitCapFloats) return 1;
  return p.group;
}

long long dkdv16_split_floats(const AttnParams& p, int D) {
  if (dkdv16_split(p, D) <= 1) return 0;
  const long long nblk = (p.S + Bwd16<64>::BW - 1) / Bwd16<64>::BW;
  return (long long)p.B * p.H * nblk * Bwd16<64>::BW * 2 * D;
}

hipError_t launch_bwd16_dkdv(int dtype, int D, const void* q, const void* k, const void* v,
                             const void* dout, const float* lse, const float* delta, void* dk,
                             void* dv, const AttnParams& p, hipStream_t st) {
  MI_DISPATCH16(dtype, D, return (launch_dkdv16_t<T, DD>(q, k, v, dout, lse, delta, dk, dv, p, st)))
}

hipError_t launch_bwd16_dq(int dtype, int D, const void* q, const void* k, const void* v,
                           const void* dout, const float* lse, const float* delta, void* dq,
                           const AttnParams& p, hipStream_t st) {
  MI_DISPATCH16(dtype, D, return (launch_dq16_t<T, DD>(q, k, v, dout, lse, delta, dq, p, st)))
}

}  // namespace mi
