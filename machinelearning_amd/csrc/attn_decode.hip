// KV-cached attention for incremental decoding: the attention section of
// nanolab's Attention.forward_cached (nanolab/mixers.py:372-467).
//
// A step attends T active queries (one block of new tokens, [B, T, H, D]) to
// the keys of a per-layer cache ([B, Hkv, Lc, D] rows, any batch / head
// stride) followed by the block's own keys ([B, T, Hkv, D]); nothing is
// concatenated. Key j < Lc sits at absolute position cache_pos[j] (j when no
// positions are given), key Lc + t at start + t, and query t at start + t.
// Query t sees key j iff
//   * bidirectional block (causal = 0): always (a cache holds only earlier
//     positions);
//   * causal = 1: kpos <= qpos (the cache in full, the block lower-triangular);
//   * window w > 0 (causal only), sinks s: also kpos > qpos - (w - s) or
//     kpos < s (the mask of mixers.py:423-428).
//
// Decoding is HBM-bound: a step reads the whole cache once per kv head, for a
// handful of query rows. The work is split over the keys (flash-decoding):
//   * unit = (batch, kv head, tile of RT query rows), where the rows of a kv
//     head are its T queries x its GQA group of heads (row r = t*rep + head
//     in group), so every K/V byte read serves the whole group;
//   * each workgroup takes one contiguous range of key blocks of one unit,
//     its waves take every W-th block; a wave keeps (max, sum, O) per row;
//   * the waves of a workgroup merge in LDS; with one split per unit the
//     workgroup writes the output, otherwise a partial ((m, l) in fp32, O / l
//     in the input type) that attn_decode_combine_kernel merges in split order, so
//     results are bitwise reproducible.
// Two kernels share that structure:
//  * more than kDecValuRows query rows per kv head, 16-bit inputs (block
//    drafts, verification, GQA groups): MFMA. Per 64-key block, S^T = K Q^T
//    (keys as MFMA rows from LDS, the unit's 32 query rows as columns in
//    registers) and O^T += V^T P^T with V^T read from the natural V tile by
//    ds_read_b64_tr_b16 (the forward kernel's tile layout and fragment
//    maps). Each wave streams its own blocks HBM -> registers -> its private
//    LDS tile, prefetching the next block while it computes, so the loop
//    needs no workgroup barrier;
//  * fp32 inputs, and one-token steps with few query rows per kv head: VALU.
//    A 32-column MFMA would be mostly padding there, and the step is a pure
//    HBM stream. Lane groups over keys, 16 bytes per lane, several keys in
//    flight per group.
#include <type_traits>

#include "attn16.h"

namespace mi {

namespace {

constexpr float kDecNegInit = -1e30f;   // finite running-max sentinel

// Absolute position of key j (cache rows first, then the active block).
// Padding keys (j >= Lk) get INT_MAX, which no causal mask admits.
// Without a window positions are the indices (start == Lc, no pos array).
template <bool SWA>
__device__ __forceinline__ int dec_key_pos(const DecParams& p, int j) {
  if constexpr (!SWA) return j < p.Lk ? j : 0x7fffffff;
  const int cp = p.pos ? (int)p.pos[max(0, min(j, p.Lc - 1))] : j;   // pos set only if Lc >= 1
  return j < p.Lc ? cp : (j < p.Lk ? p.start + (j - p.Lc) : 0x7fffffff);
}

// Element offset of key j's row: cache rows first, then the active block's.
// Indices past the end (padding keys) are clamped to the block's last row,
// so every load is in bounds and none sits behind a branch (a load under
// divergent control flow makes the compiler wait for it at the join); the
// caller zeroes what it loaded for j >= Lk.
struct DecRows {
  const void* kc; const void* vc; const void* kn; const void* vn;
  long long n_rs;        // row stride of the active block (Hkv * D)
};
// Rows of (batch b, kv head kvh): its cache rows and its active-block rows.
template <typename T>
__device__ __forceinline__ DecRows dec_rows(const DecParams& p, const T* Kc, const T* Vc,
                                            const T* Kn, const T* Vn, int b, int kvh) {
  DecRows r;
  r.kc = Kc ? Kc + (long long)b * p.k_sb + (long long)kvh * p.k_sh : nullptr;
  r.vc = Vc ? Vc + (long long)b * p.v_sb + (long long)kvh * p.v_sh : nullptr;
  r.kn = Kn + ((long long)b * p.T * p.Hkv + kvh) * p.D;
  r.vn = Vn + ((long long)b * p.T * p.Hkv + kvh) * p.D;
  r.n_rs = (long long)p.Hkv * p.D;
  return r;
}
template <typename T>
__device__ __forceinline__ void dec_row_ptrs(const DecParams& p, const DecRows& r, int j,
                                             const T*& kp, const T*& vp) {
  if (j < p.Lc) {
    kp = reinterpret_cast<const T*>(r.kc) + (long long)j * p.D;
    vp = reinterpret_cast<const T*>(r.vc) + (long long)j * p.D;
  } else {
    const long long off = (long long)min(j - p.Lc, p.T - 1) * r.n_rs;
    kp = reinterpret_cast<const T*>(r.kn) + off;
    vp = reinterpret_cast<const T*>(r.vn) + off;
  }
}

// Visibility of a key at position kp (index j) for active query t.
template <bool SWA>
__device__ __forceinline__ bool dec_visible(const DecParams& p, int j, int kp, int t) {
  if (j >= p.Lk) return false;
  if (!p.causal) return true;
  const int qp = p.start + t;
  if (kp > qp) return false;
  if constexpr (SWA) return kp > qp - p.span || kp < p.sinks;
  return true;
}

// Output of row r (query t = r / rep, head kvh*rep + r % rep), head dims
// [d0, d0 + 4): O / L (times sigma(gate)); and the row's LSE when d0 == 0.
template <typename T>
__device__ __forceinline__ void dec_emit(const DecParams& p, T* __restrict__ out,
                                         float* __restrict__ lse, int b, int kvh, int r, int d0,
                                         f32x4 o, float M, float L) {
  const int t = r / p.rep, h = kvh * p.rep + r % p.rep;
  float inv = 1.f / L;
  if (p.gate) {
    const float z = p.gate[((long long)b * p.T + t) * p.H + h];
    inv *= 1.f / (1.f + __expf(-z));
  }
  T* dst = out + (((long long)b * p.T + t) * p.H + h) * p.D + d0;
  if constexpr (sizeof(T) == 4) {
    *reinterpret_cast<f32x4*>(dst) = o * inv;
  } else {
    st_quad<T>(dst, o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
  }
  if (lse && d0 == 0) lse[((long long)b * p.H + h) * p.T + t] = M * p.scale + logf(L);
}

// Partial of (unit, split): rows x D of O / l in the input type T, then,
// after those of every unit and split, rows x {m, l} in fp32. O / l is a
// convex combination of V rows, so it lies within V's range (0 where l = 0:
// no visible key in the split); stored in T it moves half the bytes of fp32
// for 16-bit inputs, at one more rounding of the output.
template <typename T>
__device__ __forceinline__ T* dec_part_o(float* ws, const DecParams& p, long long unit, int split) {
  return reinterpret_cast<T*>(ws) + (unit * p.nsplit + split) * (long long)p.RT * p.D;
}
template <typename T>
__device__ __forceinline__ float* dec_part_ml(float* ws, const DecParams& p, long long unit, int split) {
  const long long units = (long long)p.B * p.Hkv * p.ntiles;
  const long long obytes = units * p.nsplit * (long long)p.RT * p.D * (long long)sizeof(T);
  return reinterpret_cast<float*>(reinterpret_cast<char*>(ws) + obytes) +
         (unit * p.nsplit + split) * 2LL * p.RT;
}
// Four consecutive head dims of a partial row, as T in memory and fp32 here.
template <typename T>
__device__ __forceinline__ void dec_part_store(T* dst, f32x4 v) {
  if constexpr (sizeof(T) == 4) *reinterpret_cast<f32x4*>(dst) = v;
  else st_quad<T>(dst, v[0], v[1], v[2], v[3]);
}
template <typename T>
__device__ __forceinline__ f32x4 dec_part_load(const T* src) {
  if constexpr (sizeof(T) == 4) {
    return *reinterpret_cast<const f32x4*>(src);
  } else {
    const typename Mfma32<T>::quad q = *reinterpret_cast<const typename Mfma32<T>::quad*>(src);
    const f32x4 v = {(float)q[0], (float)q[1], (float)q[2], (float)q[3]};
    return v;
  }
}

// Merge NW per-group partials held in LDS (obuf[w][row][D], ml[w][row][2])
// into the unit's output (one split) or its split partial. All NTH threads.
// Group w's partial O starts at obuf + w * wstride floats.
template <typename T, int D, int NW, int RT, int NTH = 256>
__device__ __forceinline__ void dec_merge(const DecParams& p, const float* obuf, int wstride,
                                          const float* ml, T* __restrict__ out,
                                          float* __restrict__ lse, float* __restrict__ ws, int b,
                                          int kvh, int tile, int split) {
  const long long unit = ((long long)b * p.Hkv + kvh) * p.ntiles + tile;
  const float c = p.scale_log2;
  for (int x = threadIdx.x; x < RT * (D / 4); x += NTH) {
    const int row = x / (D / 4), d0 = 4 * (x % (D / 4));
    const int r = tile * RT + row;
    if (r >= p.R) continue;
    float M = ml[2 * row];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, ml[(w * RT + row) * 2]);
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float a = fast_exp2((ml[(w * RT + row) * 2] - M) * c);
      L += a * ml[(w * RT + row) * 2 + 1];
      o += a * *reinterpret_cast<const f32x4*>(obuf + (long long)w * wstride + row * D + d0);
    }
    if (p.nsplit == 1) {
      dec_emit<T>(p, out, lse, b, kvh, r, d0, o, M, L);
    } else {
      dec_part_store<T>(dec_part_o<T>(ws, p, unit, split) + (long long)row * D + d0,
                        o * (L > 0.f ? 1.f / L : 0.f));
      if (d0 == 0) {
        float* pm = dec_part_ml<T>(ws, p, unit, split) + 2 * row;
        pm[0] = M;
        pm[1] = L;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// 16-bit MFMA kernel.
template <int D>
struct Dec16 {
  static constexpr int W = 4;                     // waves per workgroup (shared blocks)
  static constexpr int WS = 8;                    // waves per workgroup (per-wave streaming)
  static constexpr int RT = 32;                   // query rows per unit (MFMA columns)
  static constexpr int BN = D >= 128 ? 32 : 64;   // keys per wave step
  static constexpr int MT = BN / 32;              // 32-key halves per step
  static constexpr int CH = D / 8;                // 16-byte chunks per row
  static constexpr int TILE = BN * D * 2;         // bytes of one K (or V) tile
  static constexpr int LD = TILE / 1024;          // 16-byte loads per lane per tile
  static constexpr int DS = D / 16, DT = D / 32;
};

// One wave's 32 query rows (MFMA columns: lane l32 owns row tile * 32 + l32,
// both halves of the wave) and their running softmax state; `block` folds in
// one BN-key block held in LDS as natural K / V tiles (swizzled chunks, the
// forward kernel's layout and fragment maps) plus, with a window, the keys'
// positions.
template <typename T, int D, bool SWA>
struct Dec16Rows {
  using C = Dec16<D>;
  using M = Mfma32<T>;
  using frag = typename M::frag;
  static constexpr int BN = C::BN, MT = C::MT, DS = C::DS, DT = C::DT;
  frag qf[DS];
  int kaddr[DS];
  int vaddr[DT][2];
  f32x16 oacc[DT];
  float m_run, l_run;
  int t, key_hi, l32, g;

  __device__ __forceinline__ void init(const DecParams& p, const T* __restrict__ Q, int b, int kvh,
                                       int tile, int lane) {
    l32 = lane & 31;
    g = lane >> 5;
    const int r = tile * 32 + l32;
    const bool rvalid = r < p.R;
    t = rvalid ? r / p.rep : 0;                   // padding rows address row 0
    const T* qrow = Q + (((long long)b * p.T + t) * p.H + kvh * p.rep + (rvalid ? r % p.rep : 0)) * D;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) qf[ds] = rvalid ? ld_frag<T>(qrow + ds * 16 + g * 8) : zero_frag<T>();
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) kaddr[ds] = tile_off<D>(l32, 2 * ds + g);
    const int G = lane >> 4, m = lane & 15;
    const int row = 4 * (G >> 1) + (m >> 2);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int col = dt * 32 + 16 * (G & 1) + 4 * (m & 3);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) vaddr[dt][hh] = tile_off<D>(row + 8 * hh, col >> 3) + (col & 7) * 2;
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = zero16();
    m_run = kDecNegInit;
    l_run = 0.f;
    // Highest visible key index of this row without a window (causal: the
    // whole cache and the block up to t; bidirectional: everything).
    key_hi = p.causal ? min(p.Lk - 1, p.Lc + t) : p.Lk - 1;
  }

  // Keys [k0, k0 + BN) from LDS.
  __device__ __forceinline__ void block(const DecParams& p, const char* sK, const char* sV,
                                        const int* sP, int k0) {
    const float c = p.scale_log2;
    f32x16 s[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      s[mt] = zero16();
#pragma unroll
      for (int ds = 0; ds < DS; ++ds)
        s[mt] = M::mma(lds_frag<T>(sK + kaddr[ds] + mt * 32 * D * 2), qf[ds], s[mt]);
    }
    // Masks. Register r of half mt is key k0 + 32 mt + crow(r, g).
    if constexpr (SWA) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int kb = 32 * mt + 8 * jj + 4 * g;
          const int4 kp4 = *reinterpret_cast<const int4*>(sP + kb);
          const int kps[4] = {kp4.x, kp4.y, kp4.z, kp4.w};
#pragma unroll
          for (int i = 0; i < 4; ++i)
            if (!dec_visible<true>(p, k0 + kb + i, kps[i], t)) s[mt][4 * jj + i] = -INFINITY;
        }
    } else if (k0 + BN - 1 > key_hi) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) mask_above(s[mt], key_hi - (k0 + mt * 32 + 4 * g), -INFINITY);
    }
    // Online softmax: the lane owns query row l32 (its keys in both halves
    // of the wave), so the statistics are lane scalars.
    float mx = s[0][0];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx = __builtin_elementwise_maximum(mx, s[mt][i]);
    if (wave_any(mx > m_run)) {
      const float m_new = fmaxf(m_run, halves_max(mx));
      const float alpha = fast_exp2((m_run - m_new) * c);
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int i = 0; i < 16; ++i) oacc[dt][i] *= alpha;
      m_run = m_new;
    }
    const float mc = m_run * c;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float pv = fast_exp2(fmaf(s[mt][i], c, -mc));
        s[mt][i] = pv;
        l_run += pv;
      }
    // O^T += V^T P^T over 16-key chunks.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
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
};

// Block staging in registers: chunk x = NT * i + id of a BN-row tile -> (row
// x / CH, chunk x % CH), for NT threads (a wave, or the workgroup). Loads are
// branch-free (padding keys read a clamped row, zeroed after the load).
template <typename T, int D, int NT>
struct Dec16Stage {
  using C = Dec16<D>;
  static constexpr int BN = C::BN, CH = C::CH;
  static constexpr int LD = C::TILE / (16 * NT);   // 16-byte loads per thread per tile
  typedef T vec8 __attribute__((ext_vector_type(8)));
  static_assert(LD <= 32, "one validity bit per load");
  vec8 kr[LD], vr[LD];
  unsigned valid;   // bit i: load i holds a key row j < Lk (else a clamped row, zeroed on store)
  int kp;

  // Issues the loads only: padding rows are zeroed in store(), since a select
  // on the loaded registers here would make the wave wait for them at once.
  __device__ __forceinline__ void load(const DecParams& p, const DecRows& rows, int blk, int id,
                                       bool swa) {
    valid = 0u;
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int x = NT * i + id, row = x / CH, c = x % CH;
      const int j = blk * BN + row;
      const T *kp_, *vp_;
      dec_row_ptrs<T>(p, rows, j, kp_, vp_);
      kr[i] = *reinterpret_cast<const vec8*>(kp_ + c * 8);
      vr[i] = *reinterpret_cast<const vec8*>(vp_ + c * 8);
      valid |= (j < p.Lk ? 1u : 0u) << i;
    }
    if (swa && id < BN) kp = dec_key_pos<true>(p, blk * BN + id);
  }
  __device__ __forceinline__ void store(char* sK, char* sV, int* sP, int id, bool swa) const {
    const vec8 z = {};
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int x = NT * i + id, row = x / CH, c = x % CH;
      const bool ok = (valid >> i) & 1u;
      *reinterpret_cast<vec8*>(sK + tile_off<D>(row, c)) = ok ? kr[i] : z;
      *reinterpret_cast<vec8*>(sV + tile_off<D>(row, c)) = ok ? vr[i] : z;
    }
    if (swa && id < BN) sP[id] = kp;
  }
};

// At most 32 query rows per kv head: each wave streams its own blocks (every
// WS-th of the split) through its private LDS tile, with no workgroup barrier
// in the loop, and the waves merge at the end.
template <typename T, int D, bool SWA>
__global__ void __launch_bounds__(64 * Dec16<D>::WS)
attn_decode16_kernel(const T* __restrict__ Q, const T* __restrict__ Kc, const T* __restrict__ Vc,
                     const T* __restrict__ Kn, const T* __restrict__ Vn, T* __restrict__ O,
                     float* __restrict__ LSE, float* __restrict__ ws, DecParams p) {
  using C = Dec16<D>;
  constexpr int W = C::WS, RT = C::RT, BN = C::BN, DT = C::DT;
  // Per wave: K tile, V tile, then the keys' positions (SWA). After the loop
  // the same bytes hold the wave's [32 rows][D] fp32 partial O; ml holds
  // every wave's (m, l) per row. (The position area is padded to 256 bytes
  // so every wave's tiles keep the same bank alignment, which the swizzle
  // assumes.)
  __shared__ __attribute__((aligned(1024))) char tiles[W][2 * C::TILE + 256];
  static_assert(BN * 4 <= 256, "positions fit their area");
  __shared__ float ml[W * RT * 2];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ut = blockIdx.x;                        // (b, kvh, tile)
  const int split = blockIdx.y;
  const int tile = ut % p.ntiles, bk = ut / p.ntiles;
  const int b = bk / p.Hkv, kvh = bk % p.Hkv;
  char* sK = tiles[wave];
  char* sV = tiles[wave] + C::TILE;
  int* sP = reinterpret_cast<int*>(tiles[wave] + 2 * C::TILE);

  Dec16Rows<T, D, SWA> st;
  st.init(p, Q, b, kvh, tile, lane);
  const DecRows rows = dec_rows<T>(p, Kc, Vc, Kn, Vn, b, kvh);
  Dec16Stage<T, D, 64> stage;

  const int nblk = (p.Lk + BN - 1) / BN;
  const int blk0 = split * p.bps, blk1 = min(nblk, blk0 + p.bps);
  int blk = blk0 + wave;
  if (blk < blk1) stage.load(p, rows, blk, lane, SWA);
  for (; blk < blk1; blk += W) {
    // The previous block's LDS reads have all returned (their values fed
    // MFMAs), and one wave's LDS operations run in order: overwrite the tile.
    asm volatile("" ::: "memory");
    stage.store(sK, sV, sP, lane, SWA);
    if (blk + W < blk1) stage.load(p, rows, blk + W, lane, SWA);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    st.block(p, sK, sV, sP, blk * BN);
  }

  // Merge the waves. Each wave writes its rows' (m, l) and O into its own
  // LDS (its tile bytes: 32 * D * 4 <= 2 * TILE), then all threads combine.
  const float l_tot = halves_sum(st.l_run);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  float* ob = reinterpret_cast<float*>(tiles[wave]);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const f32x4 v4 = {st.oacc[dt][4 * jj], st.oacc[dt][4 * jj + 1], st.oacc[dt][4 * jj + 2],
                        st.oacc[dt][4 * jj + 3]};
      *reinterpret_cast<f32x4*>(ob + st.l32 * D + dt * 32 + 8 * jj + 4 * st.g) = v4;
    }
  if (st.g == 0) {
    ml[(wave * RT + st.l32) * 2] = st.m_run;
    ml[(wave * RT + st.l32) * 2 + 1] = l_tot;
  }
  __syncthreads();
  constexpr int WSTRIDE = (int)(sizeof(tiles[0]) / sizeof(float));
  static_assert(RT * D * 4 <= 2 * C::TILE, "a wave's partial O fits its tiles");
  dec_merge<T, D, W, RT, 64 * W>(p, reinterpret_cast<const float*>(tiles[0]), WSTRIDE, ml, O, LSE, ws, b,
                         kvh, tile, split);
}

// More than 32 query rows per kv head (block verifies and drafts with GQA):
// the workgroup's four waves own four consecutive 32-row tiles of one
// (batch, kv head) and share every key block, staged once per workgroup
// into a double-buffered LDS tile with one barrier per block. (Per-wave
// streaming would read the keys once per 32-row tile.) Each wave then
// writes its own rows: the output, or its split partial.
template <typename T, int D, bool SWA>
__global__ void __launch_bounds__(256)
attn_decode16_wg_kernel(const T* __restrict__ Q, const T* __restrict__ Kc, const T* __restrict__ Vc,
                        const T* __restrict__ Kn, const T* __restrict__ Vn, T* __restrict__ O,
                        float* __restrict__ LSE, float* __restrict__ ws, DecParams p) {
  using C = Dec16<D>;
  constexpr int W = C::W, BN = C::BN, DT = C::DT;
  __shared__ __attribute__((aligned(1024))) char tiles[2][2 * C::TILE + 256];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int ngrp = (p.ntiles + W - 1) / W;
  const int ut = blockIdx.x;                        // (b, kvh, group of W tiles)
  const int split = blockIdx.y;
  const int grp = ut % ngrp, bk = ut / ngrp;
  const int b = bk / p.Hkv, kvh = bk % p.Hkv;
  const int tile = grp * W + wave;                  // >= ntiles: padding rows only

  Dec16Rows<T, D, SWA> st;
  st.init(p, Q, b, kvh, tile, lane);
  const DecRows rows = dec_rows<T>(p, Kc, Vc, Kn, Vn, b, kvh);
  Dec16Stage<T, D, 256> stage;

  const int nblk = (p.Lk + BN - 1) / BN;
  const int blk0 = split * p.bps, blk1 = min(nblk, blk0 + p.bps);
  if (blk0 < blk1) stage.load(p, rows, blk0, tid, SWA);
  for (int blk = blk0; blk < blk1; ++blk) {
    // Buffer (blk & 1) was last read in block blk - 2; every wave passed the
    // barrier of block blk - 1 after that, so it is free.
    char* buf = tiles[(blk - blk0) & 1];
    stage.store(buf, buf + C::TILE, reinterpret_cast<int*>(buf + 2 * C::TILE), tid, SWA);
    __syncthreads();
    if (blk + 1 < blk1) stage.load(p, rows, blk + 1, tid, SWA);
    st.block(p, buf, buf + C::TILE, reinterpret_cast<const int*>(buf + 2 * C::TILE), blk * BN);
  }

  // Each wave's rows: lane (l32, g) holds head dims dt*32 + 8jj + 4g + 0..3.
  if (tile >= p.ntiles) return;
  const float l_tot = halves_sum(st.l_run);
  const int r = tile * 32 + st.l32;
  if (r >= p.R) return;
  const long long unit = ((long long)b * p.Hkv + kvh) * p.ntiles + tile;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int d0 = dt * 32 + 8 * jj + 4 * st.g;
      const f32x4 o4 = {st.oacc[dt][4 * jj], st.oacc[dt][4 * jj + 1], st.oacc[dt][4 * jj + 2],
                        st.oacc[dt][4 * jj + 3]};
      if (p.nsplit == 1) {
        dec_emit<T>(p, O, LSE, b, kvh, r, d0, o4, st.m_run, l_tot);
      } else {
        dec_part_store<T>(dec_part_o<T>(ws, p, unit, split) + (long long)st.l32 * D + d0,
                          o4 * (l_tot > 0.f ? 1.f / l_tot : 0.f));
      }
    }
  if (p.nsplit > 1 && st.g == 0) {
    float* pm = dec_part_ml<T>(ws, p, unit, split) + 2 * st.l32;
    pm[0] = st.m_run;
    pm[1] = l_tot;
  }
}

// ---------------------------------------------------------------------------
// VALU kernel: fp32 inputs, and 16-bit inputs with at most kDecValuRows query
// rows per kv head (one-token decoding, small GQA groups), where a 32-column
// MFMA would be mostly padding. A lane group of LPK = D / EPL lanes holds one
// key (16 bytes per lane, EPL elements); the workgroup's NG = 256 / LPK
// groups take NB keys each per step, with every load of the step issued
// before any arithmetic. Each lane keeps, for each of the unit's RT query
// rows, its EPL head dims of q and of the output accumulator; a dot product
// is reduced over the group by a DPP butterfly, which leaves the same sum in
// every lane of the group. K and V elements are converted to fp32 once per
// key and shared by the rows.
constexpr int kDecValuRows = 4;

// RT = query rows per unit (a template parameter: a one-token step computes
// one row, with no per-row guards); EPL elements per lane, LPK lanes per key.
template <typename T, int D, int RT>
struct DecV {
  static constexpr int EPL = 16 / (int)sizeof(T);       // elements per lane
  static constexpr int LPK = D / EPL;                   // lanes per key
  static constexpr int NG = 256 / LPK;                  // key groups per workgroup
  static constexpr int NB = RT <= 1 ? 8 : 4;            // keys per group per step
  static constexpr int BN = NG * NB;                    // keys per workgroup step (a block)
};

template <int LPK>
__device__ __forceinline__ float dec_group_sum(float x) {
  auto dpp = [](float v, auto ctrl) __attribute__((always_inline)) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v),
                                                                 decltype(ctrl)::value, 0xF, 0xF, false));
  };
  x += dpp(x, std::integral_constant<int, 0xB1>{});
  x += dpp(x, std::integral_constant<int, 0x4E>{});
  if constexpr (LPK >= 8) x += dpp(x, std::integral_constant<int, 0x141>{});
  if constexpr (LPK >= 16) x += dpp(x, std::integral_constant<int, 0x140>{});
  if constexpr (LPK >= 32) x += __shfl_xor(x, 16);
  return x;
}

template <typename T, int D, int RT, bool SWA>
__global__ void __launch_bounds__(256)
attn_decode_valu_kernel(const T* __restrict__ Q, const T* __restrict__ Kc,
                        const T* __restrict__ Vc, const T* __restrict__ Kn,
                        const T* __restrict__ Vn, T* __restrict__ O, float* __restrict__ LSE,
                        float* __restrict__ ws, DecParams p) {
  using C = DecV<T, D, RT>;
  constexpr int EPL = C::EPL, LPK = C::LPK, NG = C::NG, NB = C::NB, BN = C::BN;
  typedef T vecE __attribute__((ext_vector_type(EPL)));
  __shared__ __attribute__((aligned(16))) float obuf[NG * RT * D];
  __shared__ float ml[NG * RT * 2];

  const int tid = threadIdx.x, gi = tid / LPK, li = tid % LPK;
  const int ut = blockIdx.x;
  const int split = blockIdx.y;
  const int tile = ut % p.ntiles, bk = ut / p.ntiles;
  const int b = bk / p.Hkv, kvh = bk % p.Hkv;

  // Padding rows (r >= R) read row 0's q and are never written back.
  float q[RT][EPL], acc[RT][EPL], m[RT], l[RT];
  int tq[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const int r = tile * RT + i;
    const int rr = r < p.R ? r : 0;
    tq[i] = rr / p.rep;
    const vecE x = *reinterpret_cast<const vecE*>(
        Q + (((long long)b * p.T + rr / p.rep) * p.H + kvh * p.rep + rr % p.rep) * D + EPL * li);
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
      q[i][e] = (float)x[e];
      acc[i][e] = 0.f;
    }
    m[i] = kDecNegInit;
    l[i] = 0.f;
  }

  const DecRows rows = dec_rows<T>(p, Kc, Vc, Kn, Vn, b, kvh);
  const float c = p.scale_log2;
  const vecE zero = {};

  const int nblk = (p.Lk + BN - 1) / BN;
  const int blk0 = split * p.bps, blk1 = min(nblk, blk0 + p.bps);
  for (int blk = blk0; blk < blk1; ++blk) {
    vecE kv[NB], vv[NB];
    int jn[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const int j = blk * BN + n * NG + gi;
      jn[n] = j;
      const T *kp, *vp;
      dec_row_ptrs<T>(p, rows, j, kp, vp);
      kv[n] = *reinterpret_cast<const vecE*>(kp + EPL * li);
      vv[n] = *reinterpret_cast<const vecE*>(vp + EPL * li);
    }
    // Scores of the step's NB keys for every row (K converted once per key).
    float s[RT][NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const int kp = dec_key_pos<SWA>(p, jn[n]);
      float kf[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) kf[e] = (float)kv[n][e];
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        float d = q[i][0] * kf[0];
#pragma unroll
        for (int e = 1; e < EPL; ++e) d = fmaf(q[i][e], kf[e], d);
        d = dec_group_sum<LPK>(d);
        s[i][n] = dec_visible<SWA>(p, jn[n], kp, tq[i]) ? d : -INFINITY;
      }
    }
    // One rescale per row and step, then the probabilities.
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      float mx = s[i][0];
#pragma unroll
      for (int n = 1; n < NB; ++n) mx = fmaxf(mx, s[i][n]);
      if (mx > m[i]) {
        const float alpha = fast_exp2((m[i] - mx) * c);
        l[i] *= alpha;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[i][e] *= alpha;
        m[i] = mx;
      }
      const float mc = m[i] * c;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        s[i][n] = fast_exp2(fmaf(s[i][n], c, -mc));
        l[i] += s[i][n];
      }
    }
    // O += P V; padding keys (j >= Lk) read a clamped row: zero it.
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const vecE vz = jn[n] < p.Lk ? vv[n] : zero;
      float vf[EPL];
#pragma unroll
      for (int e = 0; e < EPL; ++e) vf[e] = (float)vz[e];
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[i][e] = fmaf(s[i][n], vf[e], acc[i][e]);
    }
  }

  // Merge the NG key groups (LDS), then write the output or the split partial.
#pragma unroll
  for (int i = 0; i < RT; ++i) {
#pragma unroll
    for (int e4 = 0; e4 < EPL / 4; ++e4) {
      const f32x4 v4 = {acc[i][4 * e4], acc[i][4 * e4 + 1], acc[i][4 * e4 + 2], acc[i][4 * e4 + 3]};
      *reinterpret_cast<f32x4*>(obuf + (gi * RT + i) * D + EPL * li + 4 * e4) = v4;
    }
    if (li == 0) {
      ml[(gi * RT + i) * 2] = m[i];
      ml[(gi * RT + i) * 2 + 1] = l[i];
    }
  }
  __syncthreads();
  dec_merge<T, D, NG, RT>(p, obuf, RT * D, ml, O, LSE, ws, b, kvh, tile, split);
}

// Fixed-order merge of the split partials. One wave per valid query row;
// lane (split group sg, head dims 4c..4c+3) folds splits sg, sg + SG, ...
// in chunks of NPF with an online max: per chunk one rescale of its running
// (M, L, O) and one weight per split. Each lane loads its splits' O quads
// and (m, l) pairs together, and issues the next chunk's loads before the
// current chunk's math, so the merge waits on one memory round trip per
// chunk at most, with no LDS. The split groups are then combined by a
// butterfly with the same rescale. Every step has a fixed order: bitwise
// reproducible. At most kDecMaxSplits splits.
constexpr int kDecMaxSplits = 1024;

template <int D>
struct DecComb {
  static constexpr int NC = D / 4;          // lanes per row (4 head dims each)
  static constexpr int SG = 64 / NC;        // split groups per wave
  static constexpr int NPF = 4;             // splits per lane per chunk
  static constexpr int CHK = SG * NPF;      // splits per chunk
};

template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_decode_combine_kernel(T* __restrict__ O, float* __restrict__ LSE, const float* __restrict__ ws,
                           DecParams p) {
  using C = DecComb<D>;
  constexpr int NC = C::NC, SG = C::SG, NPF = C::NPF, CHK = C::CHK;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const long long gr = (long long)blockIdx.x * 4 + wave;      // valid row: (b, kvh, r)
  if (gr >= (long long)p.B * p.Hkv * p.R) return;             // whole waves only
  const int r = (int)(gr % p.R);
  const long long bk = gr / p.R;
  const int b = (int)(bk / p.Hkv), kvh = (int)(bk % p.Hkv);
  const long long unit = bk * p.ntiles + r / p.RT;
  const int row = r % p.RT;
  float* wsm = const_cast<float*>(ws);
  const float c = p.scale_log2;
  const int cc = lane % NC, sg = lane / NC;
  // Split s of this row: O quad at po + s * so, (m, l) at pml + s * sml.
  const T* po = dec_part_o<T>(wsm, p, unit, 0) + (long long)row * D + 4 * cc;
  const float* pml = dec_part_ml<T>(wsm, p, unit, 0) + 2 * row;
  const long long so = (long long)p.RT * D, sml = 2LL * p.RT;
  const int last = p.nsplit - 1;

  f32x4 ov[NPF];
  float2 mv[NPF];
  auto load = [&](int s0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      const int s = min(s0 + sg + SG * i, last);              // clamped; extras weigh 0
      ov[i] = dec_part_load<T>(po + s * so);
      mv[i] = *reinterpret_cast<const float2*>(pml + s * sml);
    }
  };
  float M = kDecNegInit, L = 0.f;
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  load(0);
  for (int s0 = 0; s0 < p.nsplit; s0 += CHK) {
    f32x4 cov[NPF];
    float2 cmv[NPF];
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      cov[i] = ov[i];
      cmv[i] = mv[i];
    }
    if (s0 + CHK < p.nsplit) load(s0 + CHK);
    float mc = M;
#pragma unroll
    for (int i = 0; i < NPF; ++i)
      if (s0 + sg + SG * i <= last) mc = fmaxf(mc, cmv[i].x);
    const float a = fast_exp2((M - mc) * c);
    L *= a;
    o *= a;
#pragma unroll
    for (int i = 0; i < NPF; ++i) {
      const float w = s0 + sg + SG * i <= last ? fast_exp2((cmv[i].x - mc) * c) : 0.f;
      L += w * cmv[i].y;
      o += (w * cmv[i].y) * cov[i];                           // the split's O = l * (O / l)
    }
    M = mc;
  }
#pragma unroll
  for (int off = NC; off < 64; off <<= 1) {
    const float Mo = __shfl_xor(M, off), Lo = __shfl_xor(L, off);
    f32x4 oo;
#pragma unroll
    for (int e = 0; e < 4; ++e) oo[e] = __shfl_xor(o[e], off);
    const float Mn = fmaxf(M, Mo);
    const float a = fast_exp2((M - Mn) * c), ao = fast_exp2((Mo - Mn) * c);
    L = L * a + Lo * ao;
    o = o * a + oo * ao;
    M = Mn;
  }
  if (sg == 0) dec_emit<T>(p, O, LSE, b, kvh, r, 4 * cc, o, M, L);
}

// Workgroup target for picking the split count: 4 per CU of the 256.
constexpr int kDecTargetGroups = 1024;
// Bytes of K and V each split streams at least. Measured against 64 and
// 128 KB floors and none (ABBA order): 256 KB takes the one-token board step
// from 5 splits to 1 (14.2 -> 12.8 us) and the 32-token draft from 4 to 1
// (22.5 -> 16.3 us), and leaves the long-cache steps' split counts alone.
constexpr long long kDecMinSplitBytes = 256 * 1024LL;
static_assert(kDecTargetGroups <= kDecMaxSplits, "split count bound");

// Which kernel a step uses, and the VALU kernel's rows per unit (0: MFMA).
// fp32: 1 or 8 rows; 16-bit: 1 or kDecValuRows rows, MFMA above.
template <typename T>
__host__ __forceinline__ int dec_valu_rows(const DecParams& p) {
  if (p.R <= 1) return 1;
  if (sizeof(T) == 4) return 8;
  return p.R <= kDecValuRows ? kDecValuRows : 0;
}

// Workgroups per (batch, kv head) and split: one per 32-row tile, or one
// per four tiles for the shared-block kernel (more than 32 rows, 16-bit).
template <typename T, int D>
__host__ __forceinline__ long long dec_groups(const DecParams& p) {
  if (dec_valu_rows<T>(p) == 0 && p.R > Dec16<D>::RT) return (p.ntiles + Dec16<D>::W - 1) / Dec16<D>::W;
  return p.ntiles;
}

template <typename T, int D>
static void dec_geometry(DecParams& p) {
  const int vr = dec_valu_rows<T>(p);
  int RT, BN, min_blocks;
  long long target = kDecTargetGroups;
  if (vr == 1) {
    RT = 1; BN = DecV<T, D, 1>::BN; min_blocks = 1;
  } else if (vr == 4) {
    RT = 4; BN = DecV<T, D, 4>::BN; min_blocks = 1;
  } else if (vr == 8) {
    RT = 8; BN = DecV<T, D, 8>::BN; min_blocks = 1;
  } else {
    // Per-wave streaming: each split should give every wave at least one
    // block (WS waves). Shared blocks (more than one 32-row tile): at least
    // four blocks per split, and half the workgroup target, since each split
    // writes a partial of four row tiles (as many bytes as ~8 key blocks).
    RT = Dec16<D>::RT; BN = Dec16<D>::BN;
    min_blocks = p.R > Dec16<D>::RT ? 4 : Dec16<D>::WS;
    if (p.R > Dec16<D>::RT) target = kDecTargetGroups / 2;
  }
  p.RT = RT;
  p.ntiles = (p.R + RT - 1) / RT;
  const int nblk = (p.Lk + BN - 1) / BN;
  const long long units = (long long)p.B * p.Hkv * dec_groups<T, D>(p);
  int want = (int)((target + units - 1) / units);
  // Each split should also stream at least kDecMinSplitBytes of K and V, or
  // its fixed costs (the first load's latency, the partial, the merge) are
  // not amortised: short caches take fewer splits than the target asks.
  const long long unit_bytes = 2LL * p.Lk * p.D * (long long)sizeof(T);
  const long long cap = unit_bytes / kDecMinSplitBytes;
  if (want > cap) want = cap > 1 ? (int)cap : 1;
  want = max(1, min(want, nblk / min_blocks));
  p.bps = (nblk + want - 1) / want;
  p.nsplit = (nblk + p.bps - 1) / p.bps;
}

template <typename T, int D, int RT>
static void launch_valu(dim3 grid, bool swa, const T* Q, const T* Kc, const T* Vc, const T* Kn,
                        const T* Vn, T* out, float* lse, float* ws, const DecParams& p,
                        hipStream_t st) {
  if (swa)
    hipLaunchKernelGGL((attn_decode_valu_kernel<T, D, RT, true>), grid, dim3(256), 0, st, Q, Kc, Vc,
                       Kn, Vn, out, lse, ws, p);
  else
    hipLaunchKernelGGL((attn_decode_valu_kernel<T, D, RT, false>), grid, dim3(256), 0, st, Q, Kc,
                       Vc, Kn, Vn, out, lse, ws, p);
}

template <typename T, int D>
static hipError_t launch_decode_t(const void* q, const void* kc, const void* vc, const void* kn,
                                  const void* vn, void* out, float* lse, float* ws, DecParams p,
                                  hipStream_t st) {
  dec_geometry<T, D>(p);
  // Workgroups in x (up to 2^24 of 256 lanes), splits in y.
  const long long units = (long long)p.B * p.Hkv * dec_groups<T, D>(p);
  if (units > (1LL << 24) || p.nsplit > kDecMaxSplits) return hipErrorInvalidValue;
  const dim3 grid((unsigned)units, (unsigned)p.nsplit);
  const bool swa = p.window > 0;
  const T* Q = (const T*)q;
  const T *Kc = (const T*)kc, *Vc = (const T*)vc, *Kn = (const T*)kn, *Vn = (const T*)vn;
  switch (dec_valu_rows<T>(p)) {
    case 1: launch_valu<T, D, 1>(grid, swa, Q, Kc, Vc, Kn, Vn, (T*)out, lse, ws, p, st); break;
    case 8:
      if constexpr (sizeof(T) == 4) launch_valu<T, D, 8>(grid, swa, Q, Kc, Vc, Kn, Vn, (T*)out, lse, ws, p, st);
      break;
    case kDecValuRows:
      if constexpr (sizeof(T) == 2)
        launch_valu<T, D, kDecValuRows>(grid, swa, Q, Kc, Vc, Kn, Vn, (T*)out, lse, ws, p, st);
      break;
    default:
      if constexpr (sizeof(T) == 2) {
        const bool shared = p.R > Dec16<D>::RT;
        if (shared && swa)
          hipLaunchKernelGGL((attn_decode16_wg_kernel<T, D, true>), grid, dim3(256), 0, st, Q, Kc,
                             Vc, Kn, Vn, (T*)out, lse, ws, p);
        else if (shared)
          hipLaunchKernelGGL((attn_decode16_wg_kernel<T, D, false>), grid, dim3(256), 0, st, Q, Kc,
                             Vc, Kn, Vn, (T*)out, lse, ws, p);
        else if (swa)
          hipLaunchKernelGGL((attn_decode16_kernel<T, D, true>), grid, dim3(64 * Dec16<D>::WS), 0, st, Q, Kc, Vc,
                             Kn, Vn, (T*)out, lse, ws, p);
        else
          hipLaunchKernelGGL((attn_decode16_kernel<T, D, false>), grid, dim3(64 * Dec16<D>::WS), 0, st, Q, Kc,
                             Vc, Kn, Vn, (T*)out, lse, ws, p);
      }
  }
  if (p.nsplit > 1) {
    const long long nrows = (long long)p.B * p.Hkv * p.R;
    hipLaunchKernelGGL((attn_decode_combine_kernel<T, D>), dim3((unsigned)((nrows + 3) / 4)),
                       dim3(256), 0, st, (T*)out, lse, ws, p);
  }
  return hipGetLastError();
}

template <typename T>
static hipError_t launch_decode_d(const void* q, const void* kc, const void* vc, const void* kn,
                                  const void* vn, void* out, float* lse, float* ws,
                                  const DecParams& p, hipStream_t st) {
  switch (p.D) {
    case 32: return launch_decode_t<T, 32>(q, kc, vc, kn, vn, out, lse, ws, p, st);
    case 64: return launch_decode_t<T, 64>(q, kc, vc, kn, vn, out, lse, ws, p, st);
    case 128: return launch_decode_t<T, 128>(q, kc, vc, kn, vn, out, lse, ws, p, st);
  }
  return hipErrorInvalidValue;
}

template <typename T>
static long long decode_ws_t(DecParams p) {
  switch (p.D) {
    case 32: dec_geometry<T, 32>(p); break;
    case 64: dec_geometry<T, 64>(p); break;
    case 128: dec_geometry<T, 128>(p); break;
    default: return -1;
  }
  if (p.nsplit <= 1) return 0;
  const long long units = (long long)p.B * p.Hkv * p.ntiles;
  return units * p.nsplit * (long long)p.RT * (p.D * (long long)sizeof(T) / 4 + 2);
}

}  // namespace

// Floats of split-partial workspace a decode step with these parameters needs
// (0: the step writes its output directly).
long long decode_workspace_floats(int dtype, const DecParams& p) {
  if (p.R == 0 || p.B == 0 || p.Lk == 0) return 0;
  switch (dtype) {
    case 0: return decode_ws_t<float>(p);
    case 1: return decode_ws_t<_Float16>(p);
    case 2: return decode_ws_t<__bf16>(p);
  }
  return -1;
}

hipError_t launch_decode(int dtype, const void* q, const void* kc, const void* vc, const void* kn,
                         const void* vn, void* out, float* lse, float* ws, const DecParams& p,
                         hipStream_t st) {
  switch (dtype) {
    case 0: return launch_decode_d<float>(q, kc, vc, kn, vn, out, lse, ws, p, st);
    case 1: return launch_decode_d<_Float16>(q, kc, vc, kn, vn, out, lse, ws, p, st);
    case 2: return launch_decode_d<__bf16>(q, kc, vc, kn, vn, out, lse, ws, p, st);
  }
  return hipErrorInvalidValue;
}

}  // namespace mi
