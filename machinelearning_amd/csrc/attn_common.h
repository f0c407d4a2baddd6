// Shared device code for the gfx950 attention kernels: MFMA traits, the
// register layout of a 32x32 MFMA tile, the permuted LDS layout that lets an
// accumulator tile feed the next MFMA without any cross-lane movement, and the
// cooperative global->LDS tile stager.
//
// Layout facts used everywhere (one wave = 64 lanes, l32 = lane % 32,
// g = lane / 32):
//   A operand of a 32x32xKPI MFMA: lane holds row l32, k-slots [g*EPL, g*EPL+EPL)
//   B operand:                    lane holds column l32, the same k-slots
//   C/D accumulator (16 floats):  lane holds column l32; register r is row
//                                 crow(r, g) = 8*(r/4) + 4*g + r%4
// (EPL = elements per lane per operand: 8 for f16/bf16, 1 for f32; KPI = 2*EPL.)
// The k-slot order only has to agree between A and B, which it does by
// construction; the row/column/accumulator mapping is checked on the device by
// mi_mfma_probe before any kernel is trusted.
//
// The "transposed" products (P.V, dS.K, P^T.dO, dS^T.Q) contract over the
// dimension an accumulator tile holds in registers. Register r of the lane
// group g is row crow(r, g), so feeding 8 consecutive registers as one B
// fragment means the k-slot (step s, group g, element e) is row crow(s*EPL+e, g).
// The matching A operand is read from an LDS copy whose row order is permuted
// by perm_pos(), which puts exactly those rows next to each other, so one
// 16-byte LDS read fetches a whole fragment.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <utility>

namespace mi {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// Division of a non-negative index n < 2^31 by a divisor fixed per launch,
// without the ~15-instruction integer-division sequence:
//   n / d = (mulhi(n, m) + n) >> s,  s = ceil(log2 d),  m = floor(2^32 (2^s - d) / d) + 1
// (the round-up method of Granlund and Montgomery, "Division by invariant
// integers using multiplication", PLDI 1994; the sum cannot overflow for
// n < 2^31). The host fills (m, s) with fast_div; on wave-uniform operands
// fdiv is three scalar instructions.
struct FastDiv { unsigned m, s; };
inline FastDiv fast_div(unsigned d) {
  if (d < 1) d = 1;
  unsigned s = 0;
  while ((1ull << s) < d) ++s;
  return {(unsigned)((((1ull << 32) * ((1ull << s) - d)) / d) + 1), s};
}
__device__ __forceinline__ unsigned fdiv(unsigned n, FastDiv f) { return (__umulhi(n, f.m) + n) >> f.s; }

struct AttnParams {
  int B, S, H, Hkv, group;
  int causal;
  int block;           // causal granularity: query i sees key j iff j / block <= i / block
                       // (1 = plain causal; > 1 = block-causal / semi-autoregressive)
  int window;          // local span of the sliding window (0 = none)
  int sinks;           // leading keys every query sees besides its span (window > 0)
  int fold_sinks;      // sinks the 16-bit window kernels visit themselves, in their
                       // first key tiles (0: the sink kernels add them; fp32), capped
                       // at S - window (no query sees a sink past it)
  float scale;        // softmax scale
  float scale_log2;   // scale * log2(e): scores enter exp2 in this unit
  float resc_th;      // forward lazy-rescale threshold in raw score units: 8 / scale_log2
  int nblk;           // row blocks per (batch, head) for the launched kernel
  FastDiv div_h, div_hkv, div_group;   // by H, Hkv, H / Hkv
  FastDiv div_wi;     // work_item's divisor for the launched grid (work_item_div)
  int wi_blocks_fastest;   // work_item order with a head's row blocks consecutive
  long long q_rs;     // row stride of q/o/dout/dq in elements (H * D)
  long long kv_rs;    // row stride of k/v/dk/dv in elements (Hkv * D)
  const float* gate;  // per-(b, i, h) output gate logits [B, S, H] (nullptr: no gate)
  // Backward with the delta pass fused into the 16-bit dQ kernel: O, the LSE
  // gradient (or nullptr) and the workspace whose two planes it fills
  // (o == nullptr: the planes were written by the delta kernel).
  const void* o;
  const float* dlse;
  float* ws_out;
  // 16-bit dK/dV with the GQA group split across workgroups: kv_split (1 or
  // group) workgroups per key block, one query head each, each writing fp32
  // partials [B*H][nblk*128 rows][2][D] (dK, dV) to kv_part; a reduce kernel
  // sums them over the group in head order.
  int kv_split;
  float* kv_part;
  // 16-bit outputs only: the rounding residual of O, res = (T)(O - (float)(T)O),
  // in O's layout and dtype. The forward writes it when set; the backward's
  // fused delta pass then reads O + res, O to about 16 significant bits
  // (nullptr: none).
  void* o_res;
};

// Causal bounds at block granularity (the block-causal mask of
// nanolab/mixers.py:76-93: query i sees key j iff j / L <= i / L, L = p.block).
// BLK = false is plain causal (L = 1), compiled without the division; the
// launchers pick BLK = (p.block > 1). Only meaningful when p.causal.
// The last key query i sees:
template <bool BLK>
__device__ __forceinline__ int causal_key_end(const AttnParams& p, int i) {
  if constexpr (BLK) return min(p.S - 1, (i / p.block + 1) * p.block - 1);
  else return i;
}
// The first query that sees key j:
template <bool BLK>
__device__ __forceinline__ int causal_query_begin(const AttnParams& p, int j) {
  if constexpr (BLK) return (j / p.block) * p.block;
  else return j;
}

// sigmoid of the output gate logit of query row (b, i, h); 1 without a gate.
__device__ __forceinline__ float gate_sigmoid(const AttnParams& p, int b, int i, int h) {
  if (!p.gate) return 1.f;
  const float z = p.gate[((long long)b * p.S + i) * p.H + h];
  return 1.f / (1.f + __expf(-z));
}

// Parameters of a KV-cached decode step (attn_decode.hip): T active queries
// against Lc cached keys followed by the T active keys.
struct DecParams {
  int B, T, H, Hkv, rep, D;
  int Lc, Lk;            // cached keys; cached + active keys
  int start;             // absolute position of active query 0 (and of key Lc)
  int causal, window, sinks, span;
  float scale, scale_log2;
  long long k_sb, k_sh, v_sb, v_sh;   // cache strides (elements); rows are D apart
  int R;                 // query rows per kv head: T * rep
  int RT, ntiles;        // rows per unit tile, tiles per kv head
  int nsplit, bps;       // key splits per unit, key blocks per split
  const long long* pos;  // absolute positions of the cached keys (nullptr: 0, 1, ...)
  const float* gate;     // [B, T, H] output gate logits (nullptr: none)
};

// Parameters of the fused q / k prologue (RMSNorm + RoPE, qk_prologue.hip).
struct ProParams {
  int rows;        // B * T * H
  int T, H;        // row r is (b, t, h) with t = (r / H) % T
  int norm, rope;
  float eps;
  int nchunk;      // workgroups of the backward's weight-gradient partials
  int chunk_rows;  // rows per such workgroup
};

// ---------------------------------------------------------------------------
// MFMA traits: one 32x32 f32 accumulator tile per instruction.
// ---------------------------------------------------------------------------
template <typename T> struct Mfma32;

template <> struct Mfma32<__bf16> {
  static constexpr int EPL = 8;
  using frag = bf16x8;
  using quad = bf16x4;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma32<_Float16> {
  static constexpr int EPL = 8;
  using frag = f16x8;
  using quad = f16x4;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma32<float> {
  static constexpr int EPL = 1;
  using frag = float;
  using quad = f32x4;
  static __device__ __forceinline__ f32x16 mma(frag a, frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

__device__ __forceinline__ int crow(int r, int g) { return 8 * (r >> 2) + 4 * g + (r & 3); }

// Position of row `row` (within a tile whose height is a multiple of 32) in the
// permuted LDS order described at the top of this file.
template <int EPL>
__host__ __device__ constexpr int perm_pos(int row) {
  return 32 * (row >> 5) +
         ((4 * ((row & 31) >> 3) + (row & 3)) / EPL) * (2 * EPL) +
         ((row >> 2) & 1) * EPL +
         ((4 * ((row & 31) >> 3) + (row & 3)) % EPL);
}

// Convert EPL consecutive accumulator registers starting at `base` to a fragment.
template <typename T>
__device__ __forceinline__ typename Mfma32<T>::frag pack_frag(const f32x16& acc, int base);

template <>
__device__ __forceinline__ bf16x8 pack_frag<__bf16>(const f32x16& acc, int base) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (__bf16)acc[base + i];
  return r;
}
template <>
__device__ __forceinline__ f16x8 pack_frag<_Float16>(const f32x16& acc, int base) {
  f16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = (_Float16)acc[base + i];
  return r;
}
template <>
__device__ __forceinline__ float pack_frag<float>(const f32x16& acc, int base) {
  return acc[base];
}

template <typename T>
__device__ __forceinline__ typename Mfma32<T>::frag zero_frag() {
  typename Mfma32<T>::frag z;
  if constexpr (Mfma32<T>::EPL == 1) {
    z = 0.f;
  } else {
#pragma unroll
    for (int i = 0; i < Mfma32<T>::EPL; ++i) z[i] = (T)0.f;
  }
  return z;
}

template <typename T>
__device__ __forceinline__ typename Mfma32<T>::frag ld_frag(const T* p) {
  return *reinterpret_cast<const typename Mfma32<T>::frag*>(p);
}

// Store 4 consecutive head-dim values (already scaled) as T.
template <typename T>
__device__ __forceinline__ void st_quad(T* p, float a, float b, float c, float d) {
  typename Mfma32<T>::quad q;
  q[0] = (T)a; q[1] = (T)b; q[2] = (T)c; q[3] = (T)d;
  *reinterpret_cast<typename Mfma32<T>::quad*>(p) = q;
}

// st_quad of the rounded values to p and of their rounding residuals
// (x - (float)(T)x, rounded to T) to r.
template <typename T>
__device__ __forceinline__ void st_quad_res(T* p, T* r, float a, float b, float c, float d) {
  typename Mfma32<T>::quad q, e;
  q[0] = (T)a; q[1] = (T)b; q[2] = (T)c; q[3] = (T)d;
  e[0] = (T)(a - (float)q[0]);
  e[1] = (T)(b - (float)q[1]);
  e[2] = (T)(c - (float)q[2]);
  e[3] = (T)(d - (float)q[3]);
  *reinterpret_cast<typename Mfma32<T>::quad*>(p) = q;
  *reinterpret_cast<typename Mfma32<T>::quad*>(r) = e;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Offset of accumulator register r's row from the lane group's first row
// (crow(r, g) - 4*g): a compile-time constant once r is unrolled.
__device__ __forceinline__ constexpr int crow_off(int r) { return 8 * (r >> 2) + (r & 3); }

// Masks over the 16 accumulator entries of a lane, by a per-lane keep set:
// bit c set keeps the entry at row offset c (offsets 0..27, bits 0..27).
// The caller folds the tile origin, the lane group (4*g) and every mask
// bound into the per-lane integers lo / hi.
__device__ __forceinline__ unsigned keep_upto(int hi) {   // offsets c <= hi
  return ~(~0u << min(max(hi + 1, 0), 28));
}
__device__ __forceinline__ unsigned keep_from(int lo) {   // offsets c >= lo
  return ~0u << min(max(lo, 0), 28);
}

// Entries whose bit is clear in `keep` become `fill`: per entry the bit,
// sign-extended (v_bfe_i32), selects between the two values bitwise (one
// v_bitop3 / v_bfi): two VALU, no lane-mask SGPRs, no branch. Written as a
// compare in C, the select is turned into compares of the lane value against
// the 16 monotone offsets, chained through SGPR masks and exec branches
// (about five VALU per entry). Only the bit extraction is asm, so the
// compiler cannot see that the masks are monotone; its input is VALU
// arithmetic. The select that reads the accumulator stays in C: an MFMA
// result read by VALU needs wait states that the compiler inserts for its
// own instructions only.
template <int R>
__device__ __forceinline__ void mask_entry(f32x16& acc, unsigned keep, unsigned uf) {
  unsigned t;
  asm("v_bfe_i32 %0, %1, %2, 1" : "=v"(t) : "v"(keep), "n"(crow_off(R)));
  const float a = acc[R];
  acc[R] = __builtin_bit_cast(float, (__builtin_bit_cast(unsigned, a) & t) | (uf & ~t));
}
template <int... R>
__device__ __forceinline__ void mask_entries(f32x16& acc, unsigned keep, unsigned uf,
                                             std::integer_sequence<int, R...>) {
  (mask_entry<R>(acc, keep, uf), ...);
}
__device__ __forceinline__ void mask_keep(f32x16& acc, unsigned keep, float fill) {
  mask_entries(acc, keep, __builtin_bit_cast(unsigned, fill), std::make_integer_sequence<int, 16>{});
}

// Entries whose row offset lies outside [lo, hi] become `fill`.
__device__ __forceinline__ void mask_rows(f32x16& acc, int lo, int hi, float fill) {
  mask_keep(acc, keep_from(lo) & keep_upto(hi), fill);
}
// One-sided versions, for tiles that cross only one bound (a causal diagonal
// crosses one; only sliding-window or ragged-edge tiles cross the other).
__device__ __forceinline__ void mask_below(f32x16& acc, int lo, float fill) {
  mask_keep(acc, keep_from(lo), fill);
}
__device__ __forceinline__ void mask_above(f32x16& acc, int hi, float fill) {
  mask_keep(acc, keep_upto(hi), fill);
}

// Work order for a grid of nblk row blocks x BH (batch, head) pairs.
// The dispatcher deals workgroups round-robin over the 8 XCDs (blockIdx % 8),
// each with its own 4 MB L2, and starts them in blockIdx order. XCD x owns
// the heads bh = x (mod 8), every row block of a head lands on one XCD (its
// K / V or Q / dO stay in that L2), and row blocks go level by level over
// the XCD's heads, heaviest level first for causal masks (longest-processing-
// time order, so light blocks fill the tail). (Groups of heads sized to half
// an L2, walked one group at a time, measured slower on the headline shape:
// 46.6 against 43.6 us forward; the lost balance cost more than the L2 hits
// gained.) Falls back to head-fastest order when BH is not a multiple of 8.
// `div` divides by BH / 8 (BH a multiple of 8) or by BH: work_item_div(BH).
//
// With p.wi_blocks_fastest (non-causal masks, whose row blocks all cost the
// same) the row blocks of a head are consecutive instead: XCD x walks its
// heads one after another, so the blocks that read all of a head's K / V (or
// Q / dO) run together and share them in L2 (measured 6-11% faster per
// kernel on the recall shape). Sliding windows keep the level order: each
// tile has only three readers there, and the level order's concurrent blocks
// cover whole [S, H, D] rows (all heads of a row), which measured 8% faster
// for their backward. `div` then divides by nblk (work_item_div_blocks).
struct WorkItem { int bh, blk; };
inline FastDiv work_item_div(long long BH) { return fast_div((unsigned)((BH & 7) == 0 ? BH >> 3 : BH)); }
inline FastDiv work_item_div_blocks(int nblk) { return fast_div((unsigned)nblk); }
__device__ __forceinline__ WorkItem work_item(int nblk, int BH, FastDiv div, bool heavy_last_blocks,
                                             bool blocks_fastest) {
  const int bid = blockIdx.x;
  int bh, blk;
  if (blocks_fastest) {
    if ((BH & 7) == 0) {
      const int x = bid & 7, i = bid >> 3;
      const int hh = (int)fdiv((unsigned)i, div);   // i / nblk
      blk = i - hh * nblk;
      bh = x + 8 * hh;
    } else {
      bh = (int)fdiv((unsigned)bid, div);
      blk = bid - bh * nblk;
    }
    return {bh, blk};
  }
  if ((BH & 7) == 0) {
    const int x = bid & 7, i = bid >> 3;
    blk = (int)fdiv((unsigned)i, div);            // i / (heads of this XCD)
    bh = x + 8 * (i - blk * (BH >> 3));
  } else {
    blk = (int)fdiv((unsigned)bid, div);
    bh = bid - blk * BH;
  }
  if (heavy_last_blocks) blk = nblk - 1 - blk;
  return {bh, blk};
}

// Any lane of the wave (wave-uniform result).
__device__ __forceinline__ bool wave_any(bool x) { return __builtin_amdgcn_ballot_w64(x) != 0; }

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.f;
  return z;
}

// ---------------------------------------------------------------------------
// LDS tile geometry. A tile is ROWS x D elements of T, kept either in natural
// order ([row][d], 16 B of padding per row) or transposed with permuted rows
// ([d][perm_pos(row)], 16 B of padding per d-row). The padding makes the
// 16-byte fragment reads of 16 consecutive lanes (16 different rows) hit 16
// disjoint bank groups.
// ---------------------------------------------------------------------------
template <typename T, int ROWS, int D>
struct TileGeom {
  static constexpr int NAT_STRIDE = D * (int)sizeof(T) + 16;      // bytes per row
  static constexpr int TR_STRIDE = ROWS * (int)sizeof(T) + 16;    // bytes per d-row
  static constexpr int NAT_BYTES = ROWS * NAT_STRIDE;
  static constexpr int TR_BYTES = D * TR_STRIDE;
  static constexpr int CHUNKS = D * (int)sizeof(T) / 16;          // 16-B chunks per row
  static constexpr int QUADS = ROWS / 4;
  static constexpr int UNITS = QUADS * CHUNKS;                   // 4 rows x 16 B each
};

// Fragment address helpers (byte offsets inside a tile).
template <typename T, int ROWS, int D>
__device__ __forceinline__ const T* nat_ptr(const char* base, int row, int col) {
  return reinterpret_cast<const T*>(base + row * TileGeom<T, ROWS, D>::NAT_STRIDE + col * (int)sizeof(T));
}
template <typename T, int ROWS, int D>
__device__ __forceinline__ const T* tr_ptr(const char* base, int d, int pos) {
  return reinterpret_cast<const T*>(base + d * TileGeom<T, ROWS, D>::TR_STRIDE + pos * (int)sizeof(T));
}

// One staging unit: 4 consecutive rows x one 16-byte chunk, held in registers
// between the global load and the LDS store (software pipelining).
struct Unit {
  u32x4 r[4];
};

// Global -> registers. Rows at or beyond `nvalid` read as zero.
template <typename T, int ROWS, int D>
__device__ __forceinline__ void unit_load(Unit& u, const T* gbase, long long row_stride,
                                          int row0, int nvalid, int unit) {
  using G = TileGeom<T, ROWS, D>;
  const int chunk = unit / G::QUADS;
  const int quad = unit % G::QUADS;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = row0 + 4 * quad + i;
    if (row < nvalid) {
      const T* p = gbase + (long long)row * row_stride + chunk * (16 / (int)sizeof(T));
      u.r[i] = *reinterpret_cast<const u32x4*>(p);
    } else {
      u.r[i] = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

template <typename T, int ROWS, int D>
__device__ __forceinline__ void unit_store_nat(const Unit& u, char* lds, int unit) {
  using G = TileGeom<T, ROWS, D>;
  const int chunk = unit / G::QUADS;
  const int quad = unit % G::QUADS;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    *reinterpret_cast<u32x4*>(lds + (4 * quad + i) * G::NAT_STRIDE + chunk * 16) = u.r[i];
}

template <typename T, int ROWS, int D>
__device__ __forceinline__ void unit_store_tr(const Unit& u, char* lds, int unit) {
  using G = TileGeom<T, ROWS, D>;
  const int chunk = unit / G::QUADS;
  const int quad = unit % G::QUADS;
  if constexpr (sizeof(T) == 2) {
    // perm_pos<8> keeps each aligned group of 4 rows contiguous and in order,
    // so one 8-byte store writes the 4 rows of one head-dim column.
    const int pos = perm_pos<8>(4 * quad);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      // v_perm_b32 byte select: bytes 0-3 come from the second operand (row
      // 2i), bytes 4-7 from the first (row 2i+1); even columns are the low
      // halves of a dword, odd columns the high halves.
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
      const int dw = e >> 1;
      u32x2 w;
      w[0] = __builtin_amdgcn_perm(u.r[1][dw], u.r[0][dw], sel);
      w[1] = __builtin_amdgcn_perm(u.r[3][dw], u.r[2][dw], sel);
      const int col = chunk * 8 + e;
      *reinterpret_cast<u32x2*>(lds + col * G::TR_STRIDE + pos * 2) = w;
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int col = chunk * 4 + e;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos = perm_pos<1>(4 * quad + i);
        *reinterpret_cast<uint32_t*>(lds + col * G::TR_STRIDE + pos * 4) = u.r[i][e];
      }
    }
  }
}

}  // namespace mi
