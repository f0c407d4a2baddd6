// Shared device code of the 16-bit (bf16 / f16) attention kernels for gfx950.
//
// Tiles live in LDS in their natural row-major order ([row][d], d contiguous,
// no padding) and are filled straight from HBM by LDS-DMA (buffer_load ...
// lds): each lane of a wave writes the 16 bytes it fetched to LDS slot
// (wave base + 16 * lane), so the lane -> (row, chunk) map is chosen on the
// global side. That map applies an XOR swizzle to the 16-byte chunk index,
//     physical chunk = logical chunk ^ swz(row),
// chosen for gfx950's 64-bank LDS (256 B per cycle: 16 lanes of a
// ds_read_b128, 32 lanes of a ds_read_b64_tr_b16) so that both ways the
// kernels read a tile are free of bank conflicts:
//   * fragment reads (ds_read_b128): lane l32 reads row R0 + l32, chunk C0 + g;
//   * transposed reads (ds_read_b64_tr_b16): within each 16-lane group, lane m
//     points at row K0 + (m >> 2), columns N0 + 4*(m & 3) .. +3; the hardware
//     then hands lane i the four rows K0..K0+3 of column N0 + i. Two such
//     reads (rows +0 and +8) build one MFMA operand whose k-slots run down a
//     column, i.e. the transpose of a natural tile, without ever storing a
//     transposed copy.
// swz() has period 16 in the row, so fragment addresses of rows +16/+32/+48
// are immediate offsets of the row-0 address (rows +8 are not).
// The transposed-read lane map above was confirmed on the device; the MFMA
// register layout itself is checked at load time by mi_mfma_probe.
#pragma once

#include "attn_common.h"

namespace mi {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
typedef __attribute__((address_space(3))) void lds_void;

// Chunk swizzle of row r for a tile with D/8 chunks per row (see above;
// checked against a 64-bank model for both read patterns and every D).
template <int D>
__host__ __device__ constexpr int swz(int r) {
  if constexpr (D >= 128) {
    return ((r & 3) << 2) | ((r >> 2) & 3);        // 16 chunks: one row per 256 B
  } else if constexpr (D == 64) {
    return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); // 8 chunks: two rows per 256 B
  } else {
    return (r >> 2) & 3;                           // 4 chunks: four rows per 256 B
  }
}

// Byte offset of logical 16-byte chunk c of row r.
template <int D>
__host__ __device__ constexpr int tile_off(int r, int c) {
  return r * (D * 2) + ((c ^ swz<D>(r)) << 4);
}

// Buffer resource (V#) over `bytes` bytes from `base`: raw, untyped, stride
// 0, the gfx9 default data format in the last word. Reads past `bytes`
// return zeros instead of touching memory. Every field is wave-uniform and
// lives in SGPRs.
typedef int Rsrc __attribute__((ext_vector_type(4)));
__device__ __forceinline__ Rsrc make_rsrc(const void* base, unsigned bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  Rsrc r;
  r[0] = __builtin_amdgcn_readfirstlane((int)(unsigned)a);
  r[1] = __builtin_amdgcn_readfirstlane((int)((unsigned)(a >> 32) & 0xffffu));
  r[2] = __builtin_amdgcn_readfirstlane((int)bytes);
  r[3] = 0x00020000;
  return r;
}

// 32-bit LDS address of a pointer into a __shared__ array, made
// wave-uniform (it becomes M0 of an LDS-DMA).
__device__ __forceinline__ unsigned lds_u32(const void* p) {
  const unsigned a = (unsigned)reinterpret_cast<unsigned long long>((lds_void*)const_cast<void*>(p));
  return (unsigned)__builtin_amdgcn_readfirstlane((int)a);
}

// 64-row tiles of one head of a [B, S, heads, D] 16-bit tensor, as buffer
// resources: `head` is the byte address of the head's row 0 and `bytes` the
// distance from there to the end of row S - 1 (so rows past S read as zero).
// S * heads * D < 2^31 is validated on the host, so every in-head offset is
// a 32-bit quantity and a tile costs one multiply and one saturating subtract.
struct RowTiles {
  const char* head;
  unsigned bytes;
  unsigned tile_bytes;   // 64 rows
};
__device__ __forceinline__ RowTiles row_tiles(const void* base, int b, int S, long long rs, int h, int D) {
  RowTiles t;
  t.head = reinterpret_cast<const char*>(base) + ((long long)b * S * rs + (long long)h * D) * 2;
  t.bytes = (unsigned)(((long long)S * rs - (long long)h * D) * 2);
  t.tile_bytes = (unsigned)(64 * rs * 2);
  return t;
}
__device__ __forceinline__ Rsrc tile_rsrc(const RowTiles& t, int tile) {
  const unsigned off = (unsigned)tile * t.tile_bytes;
  return make_rsrc(t.head + off, t.bytes > off ? t.bytes - off : 0u);
}

// LDS-DMA through a buffer resource: lane l fetches 16 (or 4) bytes at
// `voff` past the resource base (bounds-checked) into LDS address `m0`
// + 16*l (4*l); `m0` is a wave-uniform 32-bit LDS address (lds_u32).
// Written as inline asm on purpose: the compiler then does not track
// these loads, so it never inserts its own vmcnt waits before LDS reads that
// it cannot prove disjoint from a DMA target (it could not for one ring slot
// of three, which stalled a third of all tiles on a fresh HBM round trip).
// Completion is ordered by the kernels' explicit wait_vm<N>() + lds_barrier()
// instead. M0 is saved and restored around the load (the compiler reserves
// it); the s_nop covers the SALU-writes-M0 -> LDS-DMA hazard and any
// VALU-writes-SGPR -> VMEM-reads hazard on the descriptor.
__device__ __forceinline__ void dma16_buf(Rsrc r, unsigned voff, unsigned m0) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 4\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(r), "s"(m0));
}
__device__ __forceinline__ void dma4_buf(Rsrc r, unsigned voff, unsigned m0) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "s_nop 4\n\t"
      "buffer_load_dword %1, %2, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(r), "s"(m0));
}

// Wait until at most N vector-memory operations of this wave are in flight.
// LDS-DMA loads count here; they complete in issue order.
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// s_waitcnt immediate for vmcnt(0) alone (gfx9 encoding: vmcnt in bits 3:0
// and 15:14, expcnt 6:4, lgkmcnt 11:8; the other counters left at maximum).
constexpr unsigned kWaitVm0 = 0x0F70u;

// Workgroup barrier that also drains this wave's LDS traffic. Written as
// inline asm so the compiler neither adds a vmcnt(0) drain (which would
// serialise the LDS-DMA pipeline) nor moves memory operations across it.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 8 consecutive 16-bit elements of one row (ds_read_b128).
template <typename T>
__device__ __forceinline__ typename Mfma32<T>::frag lds_frag(const char* p) {
  return *reinterpret_cast<const typename Mfma32<T>::frag*>(p);
}

// Two transposed reads -> one 8-element MFMA operand (rows k..k+3 of the
// first read, then rows k+8..k+11 of the second, for the lane's column).
template <typename T>
__device__ __forceinline__ typename Mfma32<T>::frag lds_frag_tr(const char* p0, const char* p1) {
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p0);
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p1);
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(typename Mfma32<T>::frag, ab);
}

// Epilogue stores through LDS. Without it, a wave's 32 x D output rows leave
// the MFMA layout (lane l32 = row, 4 consecutive columns per register quad) as
// D/4 stores per lane of 8 bytes each, every instruction touching 32 rows: 32
// partial-line segments per instruction. Staged as a swizzled row-major
// 32 x D tile in `stage` (32*D*2 bytes of LDS that no other wave uses until
// the caller's next barrier), the rows go out 16 bytes per lane, each
// instruction writing 1024/(2D) whole rows.
// Used where it measured faster and costs no occupancy: the forward and
// dK/dV at D >= 64 (at D = 32 it cost the forward its fourth wave per SIMD and
// dK/dV its third: 120 -> 138 and 158 -> 178 VGPRs), dQ at every D.
#ifndef MI_EPI_LDS
#define MI_EPI_LDS 1
#endif
template <int D> constexpr bool epi_lds_fwd() { return MI_EPI_LDS && D >= 64; }
template <int D> constexpr bool epi_lds_dkdv() { return MI_EPI_LDS && D >= 64; }
template <int D> constexpr bool epi_lds_dq() { return MI_EPI_LDS; }
// acc[dt] register 4j+e is column dt*32 + 8j + 4g + e of row l32; the values
// are multiplied by sc and rounded to T. Rows >= nvalid (relative to row0)
// are not stored. `dst` points at column 0 of row row0; rows are rs elements
// apart.
// RES: also stage the rounding residual of each value, (T)(x - (float)(T)x),
// in a second 32 x D tile at stage + 32*D*2 and store it to res_dst (same
// layout as dst).
template <typename T, int D, bool RES = false>
__device__ __forceinline__ void store_rows_lds(const f32x16 (&acc)[D / 32], float sc, char* stage,
                                               T* dst, long long rs, int nvalid, int lane,
                                               T* res_dst = nullptr) {
  constexpr int CHK = D / 8;                 // 16-byte chunks per row
  constexpr int RPI = 64 / CHK;              // rows per store instruction
  constexpr int TB = 32 * D * 2;             // bytes of one staged tile
  const int l32 = lane & 31, g = lane >> 5;
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      typename Mfma32<T>::quad q, e4;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float x = acc[dt][4 * j + e] * sc;
        q[e] = (T)x;
        if constexpr (RES) e4[e] = (T)(x - (float)q[e]);
      }
      const int c = 4 * dt + j;
      const int off = l32 * (D * 2) + ((c ^ swz<D>(l32)) << 4) + 8 * g;
      *reinterpret_cast<typename Mfma32<T>::quad*>(stage + off) = q;
      if constexpr (RES) *reinterpret_cast<typename Mfma32<T>::quad*>(stage + TB + off) = e4;
    }
  // The rows are read back by other lanes of this wave.
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  const int c = lane % CHK;
#pragma unroll
  for (int i = 0; i < 32 / RPI; ++i) {
    const int r = lane / CHK + i * RPI;
    const int off = r * (D * 2) + ((c ^ swz<D>(r)) << 4);
    const u32x4 w = *reinterpret_cast<const u32x4*>(stage + off);
    if (r < nvalid) *reinterpret_cast<u32x4*>(dst + (long long)r * rs + c * 8) = w;
    if constexpr (RES) {
      const u32x4 wr = *reinterpret_cast<const u32x4*>(stage + TB + off);
      if (r < nvalid) *reinterpret_cast<u32x4*>(res_dst + (long long)r * rs + c * 8) = wr;
    }
  }
}

// Combine a per-lane value with the lane 32 positions away (v_permlane32_swap,
// a VALU op: no LDS round trip). The swap yields r[0] = {lanes 0-31 own,
// lanes 32-63 <- lanes 0-31} and r[1] = {lanes 0-31 <- lanes 32-63, lanes
// 32-63 own}, so r[0] and r[1] hold both copies in every lane.
__device__ __forceinline__ float halves_max(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return fmaxf(__builtin_bit_cast(float, (unsigned)r[0]), __builtin_bit_cast(float, (unsigned)r[1]));
}
__device__ __forceinline__ float halves_sum(float x) {
  const unsigned u = __builtin_bit_cast(unsigned, x);
  const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
  return __builtin_bit_cast(float, (unsigned)r[0]) + __builtin_bit_cast(float, (unsigned)r[1]);
}

}  // namespace mi
