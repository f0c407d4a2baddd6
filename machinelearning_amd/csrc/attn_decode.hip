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
//     workgroup writes the output, otherwise a partial (m, l, unnormalised
//     O in fp32) that attn_decode_combine_kernel merges in split order, so
//     results are bitwise reproducible.
// 16-bit inputs use MFMA: per 64-key block, S^T = K Q^T (keys as MFMA rows
// from LDS, the unit's 32 query rows as columns in registers) and
// O^T += V^T P^T with V^T read from the natural V tile by ds_read_b64_tr_b16
// (the forward kernel's tile layout and fragment maps). Each wave streams its
// own blocks HBM -> registers -> its private LDS tile, prefetching the next
// block while it computes, so the loop needs no workgroup barrier.
// fp32 inputs use VALU: D/4 lanes share a key (16 bytes each), 64/(D/4) keys
// per wave at a time, 8 query rows per unit; dot products are reduced by a
// DPP butterfly.
#include "attn16.h"

namespace mi {

namespace {

constexpr float kDecNegInit = -1e30f;   // finite running-max sentinel

// Absolute position of key j (cache rows first, then the active block).
// Padding keys (j >= Lk) get INT_MAX, which no causal mask admits.
__device__ __forceinline__ int dec_key_pos(const DecParams& p, int j) {
  if (j < p.Lc) return p.pos ? (int)p.pos[j] : j;
  if (j < p.Lk) return p.start + (j - p.Lc);
  return 0x7fffffff;
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

// Partial of (unit, split): rows x D unnormalised O, then rows x {m, l}.
__device__ __forceinline__ float* dec_part_o(float* ws, const DecParams& p, long long unit, int split) {
  return ws + (unit * p.nsplit + split) * (long long)p.RT * p.D;
}
__device__ __forceinline__ float* dec_part_ml(float* ws, const DecParams& p, long long unit, int split) {
  const long long units = (long long)p.B * p.Hkv * p.ntiles;
  return ws + units * p.nsplit * (long long)p.RT * p.D + (unit * p.nsplit + split) * 2LL * p.RT;
}

// Merge NW per-group partials held in LDS (obuf[w][row][D], ml[w][row][2])
// into the unit's output (one split) or its split partial. All 256 threads.
// Group w's partial O starts at obuf + w * wstride floats.
template <typename T, int D, int NW, int RT>
__device__ __forceinline__ void dec_merge(const DecParams& p, const float* obuf, int wstride,
                                          const float* ml, T* __restrict__ out,
                                          float* __restrict__ lse, float* __restrict__ ws, int b,
                                          int kvh, int tile, int split) {
  const long long unit = ((long long)b * p.Hkv + kvh) * p.ntiles + tile;
  const float c = p.scale_log2;
  for (int x = threadIdx.x; x < RT * (D / 4); x += 256) {
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
      *reinterpret_cast<f32x4*>(dec_part_o(ws, p, unit, split) + (long long)row * D + d0) = o;
      if (d0 == 0) {
        float* pm = dec_part_ml(ws, p, unit, split) + 2 * row;
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
  static constexpr int W = 4;                     // waves per workgroup
  static constexpr int RT = 32;                   // query rows per unit (MFMA columns)
  static constexpr int BN = D >= 128 ? 32 : 64;   // keys per wave step
  static constexpr int MT = BN / 32;              // 32-key halves per step
  static constexpr int CH = D / 8;                // 16-byte chunks per row
  static constexpr int TILE = BN * D * 2;         // bytes of one K (or V) tile
  static constexpr int LD = TILE / 1024;          // 16-byte loads per lane per tile
  static constexpr int DS = D / 16, DT = D / 32;
};

template <typename T, int D, bool SWA>
__global__ void __launch_bounds__(256)
attn_decode16_kernel(const T* __restrict__ Q, const T* __restrict__ Kc, const T* __restrict__ Vc,
                     const T* __restrict__ Kn, const T* __restrict__ Vn, T* __restrict__ O,
                     float* __restrict__ LSE, float* __restrict__ ws, DecParams p) {
  using C = Dec16<D>;
  using M = Mfma32<T>;
  using frag = typename M::frag;
  constexpr int W = C::W, RT = C::RT, BN = C::BN, MT = C::MT, CH = C::CH, LD = C::LD;
  constexpr int DS = C::DS, DT = C::DT;
  typedef T vec8 __attribute__((ext_vector_type(8)));
  // Per wave: K tile, V tile (natural [key][d], swizzled chunks), then the
  // keys' positions (SWA). After the loop the same bytes hold the wave's
  // [32 rows][D] fp32 partial O; ml holds every wave's (m, l) per row.
  // (The position area is padded to 256 bytes so every wave's tiles keep the
  // same bank alignment, which the swizzle assumes.)
  __shared__ __attribute__((aligned(1024))) char tiles[W][2 * C::TILE + 256];
  static_assert(BN * 4 <= 256, "positions fit their area");
  __shared__ float ml[W * RT * 2];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int l32 = lane & 31, g = lane >> 5;
  const int ut = blockIdx.x;                        // (b, kvh, tile)
  const int split = blockIdx.y;
  const int tile = ut % p.ntiles, bk = ut / p.ntiles;
  const int b = bk / p.Hkv, kvh = bk % p.Hkv;
  char* sK = tiles[wave];
  char* sV = tiles[wave] + C::TILE;
  int* sP = reinterpret_cast<int*>(tiles[wave] + 2 * C::TILE);

  // This lane's query row (MFMA column l32).
  const int r = tile * RT + l32;
  const bool rvalid = r < p.R;
  const int t = rvalid ? r / p.rep : 0;           // padding rows address row 0
  frag qf[DS];
  {
    const T* qrow = Q + (((long long)b * p.T + t) * p.H + kvh * p.rep + (rvalid ? r % p.rep : 0)) * D;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) qf[ds] = rvalid ? ld_frag<T>(qrow + ds * 16 + g * 8) : zero_frag<T>();
  }

  // Key blocks of this split; wave w takes blocks blk0 + w, + W, ...
  const int nblk = (p.Lk + BN - 1) / BN;
  const int blk0 = split * p.bps, blk1 = min(nblk, blk0 + p.bps);

  const T* kc = Kc ? Kc + (long long)b * p.k_sb + (long long)kvh * p.k_sh : nullptr;
  const T* vc = Vc ? Vc + (long long)b * p.v_sb + (long long)kvh * p.v_sh : nullptr;
  const long long n_rs = (long long)p.Hkv * D;      // row stride of the active block
  const T* kn = Kn + ((long long)b * p.T * p.Hkv + kvh) * D;
  const T* vn = Vn + ((long long)b * p.T * p.Hkv + kvh) * D;

  // Staging: load i of a tile covers chunk x = 64 i + lane -> (row x / CH, chunk x % CH).
  vec8 kr[LD], vr[LD];
  auto load = [&](int blk) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int x = 64 * i + lane, row = x / CH, c = x % CH;
      const int j = blk * BN + row;
      vec8 kv = {}, vv = {};
      if (j < p.Lc) {
        kv = *reinterpret_cast<const vec8*>(kc + (long long)j * D + c * 8);
        vv = *reinterpret_cast<const vec8*>(vc + (long long)j * D + c * 8);
      } else if (j < p.Lk) {
        kv = *reinterpret_cast<const vec8*>(kn + (long long)(j - p.Lc) * n_rs + c * 8);
        vv = *reinterpret_cast<const vec8*>(vn + (long long)(j - p.Lc) * n_rs + c * 8);
      }
      kr[i] = kv;
      vr[i] = vv;
    }
  };
  int kp_next = 0;
  auto load_pos = [&](int blk) __attribute__((always_inline)) {
    if constexpr (SWA) {
      if (lane < BN) kp_next = dec_key_pos(p, blk * BN + lane);
    }
  };
  auto store = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < LD; ++i) {
      const int x = 64 * i + lane, row = x / CH, c = x % CH;
      *reinterpret_cast<vec8*>(sK + tile_off<D>(row, c)) = kr[i];
      *reinterpret_cast<vec8*>(sV + tile_off<D>(row, c)) = vr[i];
    }
    if constexpr (SWA) {
      if (lane < BN) sP[lane] = kp_next;
    }
  };

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
  float m_run = kDecNegInit, l_run = 0.f;
  const float c = p.scale_log2;
  // Highest visible key index of this row without a window (causal: the
  // whole cache and the block up to t; bidirectional: everything).
  const int key_hi = p.causal ? min(p.Lk - 1, p.Lc + t) : p.Lk - 1;

  int blk = blk0 + wave;
  if (blk < blk1) {
    load(blk);
    load_pos(blk);
  }
  for (; blk < blk1; blk += W) {
    // The previous block's LDS reads have all returned (their values fed
    // MFMAs), and one wave's LDS operations run in order: overwrite the tile.
    asm volatile("" ::: "memory");
    store();
    if (blk + W < blk1) {
      load(blk + W);
      load_pos(blk + W);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const int k0 = blk * BN;
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
    } else if (k0 + BN - 1 > key_hi || k0 + BN > p.Lk) {
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

  // Merge the waves. Each wave writes its rows' (m, l) and O into its own
  // LDS (its tile bytes: 32 * D * 4 <= 2 * TILE), then all threads combine.
  const float l_tot = halves_sum(l_run);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  float* ob = reinterpret_cast<float*>(tiles[wave]);
#pragma unroll
  for (int dt = 0; dt < DT; ++dt)
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      f32x4 v4 = {oacc[dt][4 * jj], oacc[dt][4 * jj + 1], oacc[dt][4 * jj + 2], oacc[dt][4 * jj + 3]};
      *reinterpret_cast<f32x4*>(ob + l32 * D + dt * 32 + 8 * jj + 4 * g) = v4;
    }
  if (g == 0) {
    ml[(wave * RT + l32) * 2] = m_run;
    ml[(wave * RT + l32) * 2 + 1] = l_tot;
  }
  __syncthreads();
  constexpr int WSTRIDE = (int)(sizeof(tiles[0]) / sizeof(float));
  static_assert(RT * D * 4 <= 2 * C::TILE, "a wave's partial O fits its tiles");
  dec_merge<T, D, W, RT>(p, reinterpret_cast<const float*>(tiles[0]), WSTRIDE, ml, O, LSE, ws, b,
                         kvh, tile, split);
}

// ---------------------------------------------------------------------------
// fp32 VALU kernel: a lane group of LPK = D/4 lanes holds one key (16 bytes
// per lane); a workgroup's NG = 256/LPK groups take NB keys each per step.
template <int D>
struct Dec32 {
  static constexpr int LPK = D / 4;
  static constexpr int NG = 256 / LPK;            // key groups per workgroup
  static constexpr int NB = 4;                    // keys per group per step
  static constexpr int RT = 8;                    // query rows per unit
  static constexpr int BN = NG * NB;              // keys per workgroup step (one "block")
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

template <int D, bool SWA>
__global__ void __launch_bounds__(256)
attn_decode32_kernel(const float* __restrict__ Q, const float* __restrict__ Kc,
                     const float* __restrict__ Vc, const float* __restrict__ Kn,
                     const float* __restrict__ Vn, float* __restrict__ O, float* __restrict__ LSE,
                     float* __restrict__ ws, DecParams p) {
  using C = Dec32<D>;
  constexpr int LPK = C::LPK, NG = C::NG, NB = C::NB, RT = C::RT, BN = C::BN;
  __shared__ __attribute__((aligned(16))) float obuf[NG * RT * D];
  __shared__ float ml[NG * RT * 2];

  const int tid = threadIdx.x, gi = tid / LPK, li = tid % LPK;
  const int ut = blockIdx.x;
  const int split = blockIdx.y;
  const int tile = ut % p.ntiles, bk = ut / p.ntiles;
  const int b = bk / p.Hkv, kvh = bk % p.Hkv;

  f32x4 q[RT], acc[RT];
  float m[RT], l[RT];
  int tq[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const int r = tile * RT + i;
    const bool ok = r < p.R;
    const int rr = ok ? r : 0;                    // padding rows address row 0
    tq[i] = rr / p.rep;
    q[i] = ok ? *reinterpret_cast<const f32x4*>(
                    Q + (((long long)b * p.T + rr / p.rep) * p.H + kvh * p.rep + rr % p.rep) * D + 4 * li)
              : f32x4{0.f, 0.f, 0.f, 0.f};
    acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    m[i] = kDecNegInit;
    l[i] = 0.f;
  }
  const int nrows = min(RT, p.R - tile * RT);

  const float* kc = Kc ? Kc + (long long)b * p.k_sb + (long long)kvh * p.k_sh : nullptr;
  const float* vc = Vc ? Vc + (long long)b * p.v_sb + (long long)kvh * p.v_sh : nullptr;
  const long long n_rs = (long long)p.Hkv * D;
  const float* kn = Kn + ((long long)b * p.T * p.Hkv + kvh) * D;
  const float* vn = Vn + ((long long)b * p.T * p.Hkv + kvh) * D;
  const float c = p.scale_log2;

  const int nblk = (p.Lk + BN - 1) / BN;
  const int blk0 = split * p.bps, blk1 = min(nblk, blk0 + p.bps);
  for (int blk = blk0; blk < blk1; ++blk) {
    f32x4 kv[NB], vv[NB];
    int jn[NB], kp[NB];
#pragma unroll
    for (int n = 0; n < NB; ++n) {
      const int j = blk * BN + n * NG + gi;
      jn[n] = j;
      kv[n] = vv[n] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (j < p.Lc) {
        kv[n] = *reinterpret_cast<const f32x4*>(kc + (long long)j * D + 4 * li);
        vv[n] = *reinterpret_cast<const f32x4*>(vc + (long long)j * D + 4 * li);
      } else if (j < p.Lk) {
        kv[n] = *reinterpret_cast<const f32x4*>(kn + (long long)(j - p.Lc) * n_rs + 4 * li);
        vv[n] = *reinterpret_cast<const f32x4*>(vn + (long long)(j - p.Lc) * n_rs + 4 * li);
      }
      kp[n] = dec_key_pos(p, j);
    }
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      if (i >= nrows) break;
      float s[NB];
      float mx = -INFINITY;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        float d = q[i][0] * kv[n][0];
        d = fmaf(q[i][1], kv[n][1], d);
        d = fmaf(q[i][2], kv[n][2], d);
        d = fmaf(q[i][3], kv[n][3], d);
        d = dec_group_sum<LPK>(d);
        s[n] = dec_visible<SWA>(p, jn[n], kp[n], tq[i]) ? d : -INFINITY;
        mx = fmaxf(mx, s[n]);
      }
      if (mx > m[i]) {
        const float alpha = fast_exp2((m[i] - mx) * c);
        l[i] *= alpha;
        acc[i] *= alpha;
        m[i] = mx;
      }
      const float mc = m[i] * c;
#pragma unroll
      for (int n = 0; n < NB; ++n) {
        const float pv = fast_exp2(fmaf(s[n], c, -mc));
        l[i] += pv;
        acc[i] += pv * vv[n];
      }
    }
  }

  // Merge the NG key groups (LDS), then write the output or the split partial.
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    *reinterpret_cast<f32x4*>(obuf + (gi * RT + i) * D + 4 * li) = acc[i];
    if (li == 0) {
      ml[(gi * RT + i) * 2] = m[i];
      ml[(gi * RT + i) * 2 + 1] = l[i];
    }
  }
  __syncthreads();
  dec_merge<float, D, NG, RT>(p, obuf, RT * D, ml, O, LSE, ws, b, kvh, tile, split);
}

// Fixed-order merge of the split partials of every valid row: one thread per
// (unit, row, 4 head dims).
template <typename T, int D>
__global__ void __launch_bounds__(256)
attn_decode_combine_kernel(T* __restrict__ O, float* __restrict__ LSE, const float* __restrict__ ws,
                           DecParams p) {
  const long long x = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long units = (long long)p.B * p.Hkv * p.ntiles;
  if (x >= units * p.RT * (D / 4)) return;
  const int d0 = 4 * (int)(x % (D / 4));
  const long long ur = x / (D / 4);
  const int row = (int)(ur % p.RT);
  const long long unit = ur / p.RT;
  const int tile = (int)(unit % p.ntiles);
  const int bk = (int)(unit / p.ntiles);
  const int b = bk / p.Hkv, kvh = bk % p.Hkv;
  const int r = tile * p.RT + row;
  if (r >= p.R) return;
  float* wsm = const_cast<float*>(ws);
  float M = kDecNegInit;
  for (int s = 0; s < p.nsplit; ++s) M = fmaxf(M, dec_part_ml(wsm, p, unit, s)[2 * row]);
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
  for (int s = 0; s < p.nsplit; ++s) {
    const float* pm = dec_part_ml(wsm, p, unit, s) + 2 * row;
    const float a = fast_exp2((pm[0] - M) * p.scale_log2);
    L += a * pm[1];
    o += a * *reinterpret_cast<const f32x4*>(dec_part_o(wsm, p, unit, s) + (long long)row * D + d0);
  }
  dec_emit<T>(p, O, LSE, b, kvh, r, d0, o, M, L);
}

// Workgroup target for picking the split count: 4 per CU of the 256.
constexpr int kDecTargetGroups = 1024;

template <typename T, int D>
static void dec_geometry(DecParams& p, int RT, int BN) {
  p.RT = RT;
  p.ntiles = (p.R + RT - 1) / RT;
  const int nblk = (p.Lk + BN - 1) / BN;
  const long long units = (long long)p.B * p.Hkv * p.ntiles;
  // Each split should give every wave at least one block (16-bit: 4 waves).
  const int min_blocks = sizeof(T) == 2 ? Dec16<D>::W : 1;
  int want = (int)((kDecTargetGroups + units - 1) / units);
  want = max(1, min(want, nblk / min_blocks));
  p.bps = (nblk + want - 1) / want;
  p.nsplit = (nblk + p.bps - 1) / p.bps;
}

template <typename T, int D>
static hipError_t launch_decode_t(const void* q, const void* kc, const void* vc, const void* kn,
                                  const void* vn, void* out, float* lse, float* ws, DecParams p,
                                  hipStream_t st) {
  if constexpr (sizeof(T) == 2) {
    dec_geometry<T, D>(p, Dec16<D>::RT, Dec16<D>::BN);
  } else {
    dec_geometry<T, D>(p, Dec32<D>::RT, Dec32<D>::BN);
  }
  // Units in x (up to 2^24 workgroups of 256 lanes), splits in y (<= 1024).
  const long long units = (long long)p.B * p.Hkv * p.ntiles;
  if (units > (1LL << 24) || p.nsplit > 65535) return hipErrorInvalidValue;
  const dim3 grid((unsigned)units, (unsigned)p.nsplit);
  const bool swa = p.window > 0;
  if constexpr (sizeof(T) == 2) {
    if (swa)
      hipLaunchKernelGGL((attn_decode16_kernel<T, D, true>), grid, dim3(256), 0, st, (const T*)q,
                         (const T*)kc, (const T*)vc, (const T*)kn, (const T*)vn, (T*)out, lse, ws, p);
    else
      hipLaunchKernelGGL((attn_decode16_kernel<T, D, false>), grid, dim3(256), 0, st, (const T*)q,
                         (const T*)kc, (const T*)vc, (const T*)kn, (const T*)vn, (T*)out, lse, ws, p);
  } else {
    if (swa)
      hipLaunchKernelGGL((attn_decode32_kernel<D, true>), grid, dim3(256), 0, st, (const float*)q,
                         (const float*)kc, (const float*)vc, (const float*)kn, (const float*)vn,
                         (float*)out, lse, ws, p);
    else
      hipLaunchKernelGGL((attn_decode32_kernel<D, false>), grid, dim3(256), 0, st, (const float*)q,
                         (const float*)kc, (const float*)vc, (const float*)kn, (const float*)vn,
                         (float*)out, lse, ws, p);
  }
  if (p.nsplit > 1) {
    const long long n = units * p.RT * (D / 4);
    hipLaunchKernelGGL((attn_decode_combine_kernel<T, D>), dim3((unsigned)((n + 255) / 256)),
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
    case 32:
      if constexpr (sizeof(T) == 2) dec_geometry<T, 32>(p, Dec16<32>::RT, Dec16<32>::BN);
      else dec_geometry<T, 32>(p, Dec32<32>::RT, Dec32<32>::BN);
      break;
    case 64:
      if constexpr (sizeof(T) == 2) dec_geometry<T, 64>(p, Dec16<64>::RT, Dec16<64>::BN);
      else dec_geometry<T, 64>(p, Dec32<64>::RT, Dec32<64>::BN);
      break;
    case 128:
      if constexpr (sizeof(T) == 2) dec_geometry<T, 128>(p, Dec16<128>::RT, Dec16<128>::BN);
      else dec_geometry<T, 128>(p, Dec32<128>::RT, Dec32<128>::BN);
      break;
    default: return -1;
  }
  if (p.nsplit <= 1) return 0;
  const long long units = (long long)p.B * p.Hkv * p.ntiles;
  return units * p.nsplit * (long long)p.RT * (p.D + 2);
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
