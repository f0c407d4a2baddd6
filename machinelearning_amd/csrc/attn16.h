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
typedef __attribute__((address_space(1))) const void gbl_void;

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

// Issue one 16-byte-per-lane LDS-DMA load: lane l fetches `g` and the data
// lands at `lds_wave` + 16 * l. `lds_wave` must be wave-uniform.
__device__ __forceinline__ void dma16(const void* g, void* lds_wave) {
  __builtin_amdgcn_global_load_lds((gbl_void*)g, (lds_void*)lds_wave, 16, 0, 0);
}

// Buffer resource over `bytes` bytes from `base` (raw, untyped; the
// descriptor's last word is the gfx9 default data format). Reads past
// `bytes` return zeros instead of touching memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// LDS-DMA through a buffer resource: lane l fetches `voff` bytes past the
// resource base (bounds-checked) into `lds_wave` + 16 * l.
__device__ __forceinline__ void dma16_buf(__amdgpu_buffer_rsrc_t r, unsigned voff, void* lds_wave) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void*)lds_wave, 16, voff, 0, 0, 0);
}

// Same with 4 bytes per lane (used for per-row float vectors).
__device__ __forceinline__ void dma4(const void* g, void* lds_wave) {
  __builtin_amdgcn_global_load_lds((gbl_void*)g, (lds_void*)lds_wave, 4, 0, 0);
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
