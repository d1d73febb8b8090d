// Load-pipeline vocabulary shared by the LDS-staged MFMA kernels (conv_halo, conv_band, conv_pw, conv_stem,
// conv_narrow): buffer resources, direct-to-LDS loads, inline-assembly loads and stores that the kernels count
// themselves, counted waits and the barrier that does not drain prefetches. Private to csrc/kernels.
#pragma once

#include <utility>

#include "device_common.h"

namespace gie_hip {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kBufferWord3 = 0x00020000;
constexpr int kOut = 0x80000000;  // buffer offset past any range: the load returns (writes) zeros
constexpr int kLdsLimit = 160 * 1024;

// s_waitcnt with only the vector-memory counter constrained (gfx9 encoding: vmcnt[3:0], expcnt[6:4],
// lgkmcnt[11:8], vmcnt[5:4] at [15:14])
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// n / d for 0 <= n < 2^22, d > 0, with inv = 1.0f / d: the float estimate is within 1 of the quotient, one
// integer correction makes it exact (the host takes the exact path for larger pixel counts).
__device__ __forceinline__ int fdiv(int n, int d, float inv) {
  int q = int(float(n) * inv);
  const int r = n - int(__umul24(unsigned(q), unsigned(d)));  // q*d < 2^23: the 24-bit multiply is exact
  q += (r >= d ? 1 : 0) - (r < 0 ? 1 : 0);
  return q;
}

// Buffer resource (V#) of a raw byte buffer: base, stride 0, num_records = bytes, word 3 as above. Offsets at or
// past num_records read as zeros.
__device__ __forceinline__ v4i make_vsharp(const void* base, int bytes) {
  const unsigned long long a = reinterpret_cast<unsigned long long>(base);
  return v4i{int(unsigned(a)), int(unsigned(a >> 32) & 0xffffu), bytes, kBufferWord3};
}

// 16 bytes per lane straight into LDS at lds_base + 16 * lane (buffer_load_dwordx4 ... lds; M0 = LDS byte
// address). Issued through inline assembly so the compiler neither waits on it at every later LDS access nor
// reorders it: the kernel counts these loads itself (wait_vmcnt) and fences them with barriers.
__device__ __forceinline__ void dma16(v4i rsrc, unsigned lds_base, int voff) {
  // lds_base is wave-uniform by construction; readfirstlane states it for the compiler (M0 is a scalar)
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(
                   __builtin_amdgcn_readfirstlane(lds_base)),
               "v"(voff), "s"(rsrc)
               : "m0");
}

// The hardware reads the data VGPRs of a store wider than 8 bytes after issue: a VALU write to them in the next
// cycle (the compiler does not look inside inline assembly for this hazard) would change what is stored, so the
// store carries its own wait state.
__device__ __forceinline__ void store16(v4i rsrc, int voff, u32x4 v) {
  asm volatile("buffer_store_dwordx4 %0, %1, %2, 0 offen\n\ts_nop 1" ::"v"(v), "v"(voff), "s"(rsrc) : "memory");
}

// store16 at device scope (sc1): the line is written through this XCD's L2 rather than left dirty in it, so a launch
// that streams its whole output once does not end with the write-back of every dirty L2 line. Whether that pays is
// a property of the kernel's store stream: measured faster for the stem kernel, the pointwise kernel's 128-byte runs
// (slower for its earlier 64-byte runs) and the split slab kernel's staged whole-line output, slower for the slab
// kernels' scattered pixel-pair stores, which keep store16.
__device__ __forceinline__ void store16_wt(v4i rsrc, int voff, u32x4 v) {
  asm volatile("buffer_store_dwordx4 %0, %1, %2, 0 offen sc1\n\ts_nop 1" ::"v"(v), "v"(voff), "s"(rsrc) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Register loads the compiler does not see as loads (so it inserts no waits of its own inside the streaming
// loop): valid only after a counted wait_vm, followed by touch() so every use depends on that wait.
__device__ __forceinline__ u32x4 load16_asm(v4i rsrc, int voff) {
  u32x4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(rsrc));
  return v;
}
__device__ __forceinline__ uint32_t load2_asm(v4i rsrc, int voff) {
  uint32_t v;
  asm volatile("buffer_load_ushort %0, %1, %2, 0 offen" : "=v"(v) : "v"(voff), "s"(rsrc));
  return v;
}
template <typename T>
__device__ __forceinline__ void touch_v(T& v) {
  asm volatile("" : "+v"(v));
}

// Workgroup barrier for the load pipeline. __syncthreads() also emits a release fence, which the compiler
// lowers to s_waitcnt vmcnt(0): that would wait for every prefetch in flight. Here the caller has already waited
// for exactly the loads that must have landed (wait_vmcnt); this barrier only drains this wave's LDS accesses and
// orders the waves. The memory clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt unconstrained
  asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ unsigned lds_addr(const unsigned char* p) {
  return unsigned(reinterpret_cast<size_t>((__attribute__((address_space(3))) const unsigned char*)p));
}

// Raises a kernel's dynamic-LDS limit to the whole 160 KiB once per (function, device) — the largest amount any
// geometry may use, so one attribute call covers them all; launches that need at most 64 KiB skip the call.
inline int set_lds_limit(const void* fn, int bytes) {
  if (bytes <= 64 * 1024) return GIE_HIP_OK;
  return lds_opt_in(fn, kLdsLimit);
}

}  // namespace gie_hip
