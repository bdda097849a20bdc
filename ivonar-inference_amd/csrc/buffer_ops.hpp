// Buffer-resource loads issued as inline assembly (gfx950): direct
// buffer-to-LDS loads and plain dword / ushort loads.  The compiler does not
// see these loads, so it inserts no waits for them; every kernel that uses
// them places its own s_waitcnt vmcnt(N) (loads complete in issue order).
#pragma once

#include <hip/hip_runtime.h>

namespace ivo {
namespace {

typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef float f4v __attribute__((ext_vector_type(4)));
typedef float f2v __attribute__((ext_vector_type(2)));

// Buffer resource over `bytes` bytes (raw, no stride): offsets at or past the
// size read zeros.  The launcher keeps every operand below 2 GiB.
__device__ __forceinline__ v4u wide_buffer(const void* base, long long bytes) {
  const unsigned long long address = (unsigned long long)base;
  return v4u{(unsigned)address, (unsigned)(address >> 32) & 0xFFFFu, (unsigned)bytes, 0x00020000u};
}

__device__ __forceinline__ unsigned lds_address(const void* p) {
  return (unsigned)(size_t)(const __attribute__((address_space(3))) void*)p;
}

// Why assembly: the compiler cannot tell which LDS bytes a direct-to-LDS load
// fills, so for its own builtin it waits for every load in flight before the
// first LDS read that follows; these forms leave the waits to the kernel.
//
// One 16-byte piece per lane from a buffer straight into LDS: lane i writes
// lds_base + 16 * i (lds_base is wave-uniform; M0 is restored afterwards).  The
// load reads M0, one wait state after the scalar write of M0.
__device__ __forceinline__ void dma16(v4u buffer, unsigned lds_base, int voffset, int soffset) {
  int saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %2, %3, %4 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds_base), "v"(voffset), "s"(buffer), "s"(soffset)
      : "memory");
}

__device__ __forceinline__ int load_b32(v4u buffer, int voffset, int soffset) {
  int r;
  asm volatile("buffer_load_dword %0, %1, %2, %3 offen" : "=v"(r) : "v"(voffset), "s"(buffer), "s"(soffset) : "memory");
  return r;
}

__device__ __forceinline__ uint2 load_b64(v4u buffer, int voffset, int soffset) {
  uint2 r;
  asm volatile("buffer_load_dwordx2 %0, %1, %2, %3 offen" : "=v"(r) : "v"(voffset), "s"(buffer), "s"(soffset) : "memory");
  return r;
}

__device__ __forceinline__ int load_u16(v4u buffer, int voffset, int soffset) {
  int r;
  asm volatile("buffer_load_ushort %0, %1, %2, %3 offen" : "=v"(r) : "v"(voffset), "s"(buffer), "s"(soffset) : "memory");
  return r;
}

// Token operands in LDS: 16-byte piece p of token t at slot t * 8 +
// (p ^ a_swizzle(t)).  Sixteen lanes reading the same piece of 16 tokens then
// cover all 64 banks once.
__device__ __forceinline__ int a_swizzle(int t) { return (t & 7) ^ ((t >> 3) & 1); }

// Bytes a direct-to-LDS load (dma16) wrote are read only after the issuing
// wave's vmcnt wait has retired that load, lgkmcnt(0), and a workgroup
// barrier that every wave of the block reaches: the sequence AMD's
// composable_kernel places after its direct loads before reading them
// (ck/utility/synchronization.hpp, block_sync_lds_direct_load, as installed
// with ROCm), used here whether the reader is the loading wave or another.
// Kernels that keep later loads in flight across it issue the same three
// instructions with vmcnt(N) (loads retire in issue order).
__device__ __forceinline__ void direct_load_sync() {
  asm volatile("s_waitcnt vmcnt(0)\n\ts_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

}  // namespace
}  // namespace ivo
