// Direct global-to-LDS loads and the waits around them (gfx950).
//
// buffer_load_dwordx4 ... lds moves 16 bytes per lane from a buffer straight
// into LDS at M0 + 16 * lane, with no VGPR round trip; a lane whose offset is
// at or past the descriptor's num_records reads zeros.  The loads are counted
// by vmcnt, so a kernel waits for its own with s_waitcnt vmcnt(N) and then
// publishes the tile to the workgroup with a barrier.
#pragma once

#include "common.h"

namespace nmb {

constexpr uint32_t kOOB = 0x80000000u;  // offset past every num_records: the load returns zeros

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef short v4s __attribute__((ext_vector_type(4)));
using lds_v4s = __attribute__((address_space(3))) v4s;

// Buffer descriptor of a raw (untyped) byte range: base, stride 0, num_records
// = bytes, dword 3 = 0x00020000 (32-bit data format on gfx9-class hardware).
__device__ __forceinline__ i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  return i32x4{__builtin_amdgcn_readfirstlane(static_cast<int>(static_cast<uint32_t>(a))),
               __builtin_amdgcn_readfirstlane(static_cast<int>((a >> 32) & 0xffff)),
               __builtin_amdgcn_readfirstlane(static_cast<int>(bytes)), 0x00020000};
}

// Byte offset in LDS of a generic pointer to shared memory: the shared
// aperture keeps the LDS offset in the low 32 bits of a generic address, so a
// truncation gives it (an address-space cast would add a null-pointer select).
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

// 16 bytes per lane from buffer offset voff into LDS at byte address
// lds + 16 * lane (lds is wave-uniform; it goes to M0).  Written as inline asm
// so that the compiler does not treat the LDS written in flight as a pending
// store to every later LDS read (it would wait for all loads before each read);
// the kernel waits for these loads itself with s_waitcnt vmcnt.
__device__ __forceinline__ void load_lds16(const i32x4& r, const bf16* lds, uint32_t voff) {
  // the address is uniform across the wave; readfirstlane makes it scalar
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds));
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(r)
               : "memory");
}

// As load_lds16 with the LDS byte address m0 already wave-uniform (an SGPR
// value) and a wave-uniform byte offset soff added to the lane offsets.
__device__ __forceinline__ void load_lds16s(const i32x4& r, uint32_t m0, uint32_t voff, uint32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(r), "s"(soff)
               : "memory");
}

// 4 bytes per lane from buffer offset voff into LDS at byte address
// lds + 4 * lane (as load_lds16).
__device__ __forceinline__ void load_lds4(const i32x4& r, const void* lds, uint32_t voff) {
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(lds_offset(lds));
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :
               : "s"(m0), "v"(voff), "s"(r)
               : "memory");
}

// s_waitcnt vmcnt(N) (gfx9 encoding: vmcnt bits [3:0] and [15:14]; expcnt and
// lgkmcnt left at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// Workgroup barrier that orders memory accesses for the compiler but adds no
// wait for outstanding loads (each wave waits for its own with wait_vmcnt).
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

// Two ds_read_b64_tr_b16.  In each group of 16 lanes, lane i receives element
// i & 3 of the 8 bytes addressed by lane 4 j + i / 4 (j = 0..3): lanes
// pointing at [r0 + i / 4][c0 + 4 (i & 3)] of a row-major bf16 tile deliver
// column c0 + i, rows r0 .. r0 + 3.  p0 gives elements 0-3, p1 elements 4-7.
__device__ __forceinline__ bf16x8 ld_tr(const bf16* p0, const bf16* p1) {
  const v4s lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(const_cast<bf16*>(p0)));
  const v4s hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4s*)(const_cast<bf16*>(p1)));
  bf16x8 r;
  __builtin_memcpy(&r, &lo, 8);
  __builtin_memcpy(reinterpret_cast<char*>(&r) + 8, &hi, 8);
  return r;
}

}  // namespace nmb
