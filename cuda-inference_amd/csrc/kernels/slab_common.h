// Device vocabulary of the 3x3 kernels that keep the input rows as padded planes in LDS and shift the tap columns on
// the accumulators (conv_slab, conv_stack): LDS fragment reads (ds_read_b128, the gfx950 transposing
// ds_read_b64_tr_b16), the 144-byte weight-run transpose, DPP lane shifts, direct-to-LDS and register loads with a
// scalar slice offset, range-checked stores, magic-number division and compile-time slot sequences. Private to
// csrc/kernels.
#pragma once

#include <utility>

#include "lds_pipe.h"

namespace gie_hip {

__device__ __forceinline__ int magic_div(int n, unsigned mg, int sh) {
  return int((__umulhi(unsigned(n), mg) + unsigned(n)) >> sh);
}

typedef short v4s __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) u32x4 lds_v4;
typedef __attribute__((address_space(3))) uint16_t lds_h;
__device__ __forceinline__ u32x4 rd16(unsigned a) { return *reinterpret_cast<const lds_v4*>(size_t(a)); }
__device__ __forceinline__ u32x2 rd_tr(unsigned a) {
  const v4s v = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<__attribute__((address_space(3))) v4s*>(size_t(a)));
  return __builtin_bit_cast(u32x2, v);
}

// segment slot swizzle of a channel: the 8 channels one half-wave reads (4 consecutive, and the 4 eight higher)
// land on 8 distinct 32-byte bank groups
__device__ __forceinline__ int seg_swz(int ch) { return (ch & 3) | (((ch >> 3) & 1) << 2); }

// half a of the 144-byte weight run (8 channels x 9 taps) in the low 16 bits, half b in the high 16 bits
__device__ __forceinline__ uint32_t pick2(const uint32_t (&d)[36], int a, int b) {
  const uint32_t lo = (a & 1) ? 0x0302u : 0x0100u;          // bytes of S1 = d[a >> 1]
  const uint32_t hi = (b & 1) ? 0x07060000u : 0x05040000u;  // bytes of S0 = d[b >> 1]
  return __builtin_amdgcn_perm(d[b >> 1], d[a >> 1], lo | hi);
}

// lane i of each 16-lane row takes lane i + k (row_shl) or i - k (row_shr); lanes without a source read 0
template <int CTRL>
__device__ __forceinline__ f32x4 dpp4(const f32x4& v) {
  f32x4 r;
#pragma unroll
  for (int i = 0; i < 4; ++i) r[i] = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v[i]), CTRL, 0xf, 0xf, true));
  return r;
}
constexpr int kShl1 = 0x101, kShl15 = 0x10F, kShr1 = 0x111, kShr15 = 0x11F;

// direct-to-LDS loads whose per-slice advance travels in the scalar offset, so the per-lane offsets are set up once
// (the resource is wave-uniform by construction; readfirstlane states it for the compiler)
__device__ __forceinline__ v4i uniform4(v4i r) {
  return v4i{__builtin_amdgcn_readfirstlane(r.x), __builtin_amdgcn_readfirstlane(r.y),
             __builtin_amdgcn_readfirstlane(r.z), __builtin_amdgcn_readfirstlane(r.w)};
}
__device__ __forceinline__ void dma4s(v4i rsrc, unsigned lds_base, int voff, int soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds" ::"s"(
                   __builtin_amdgcn_readfirstlane(lds_base)),
               "v"(voff), "s"(uniform4(rsrc)), "s"(__builtin_amdgcn_readfirstlane(soff))
               : "m0");
}
__device__ __forceinline__ void dma16s(v4i rsrc, unsigned lds_base, int voff, int soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds" ::"s"(
                   __builtin_amdgcn_readfirstlane(lds_base)),
               "v"(voff), "s"(uniform4(rsrc)), "s"(__builtin_amdgcn_readfirstlane(soff))
               : "m0");
}

// register loads the compiler does not see as loads: valid after a counted wait_vmcnt (then touch_v)
__device__ __forceinline__ uint32_t load2s(v4i rsrc, int voff, int soff) {
  uint32_t v;
  asm volatile("buffer_load_ushort %0, %1, %2, %3 offen"
               : "=v"(v)
               : "v"(voff), "s"(uniform4(rsrc)), "s"(__builtin_amdgcn_readfirstlane(soff)));
  return v;
}

// 16 bytes into registers, not seen by the compiler as a load: valid after a counted wait (then touch_v)
__device__ __forceinline__ u32x4 load16s(v4i rsrc, int voff, int soff) {
  u32x4 v;
  asm volatile("buffer_load_dwordx4 %0, %1, %2, %3 offen"
               : "=v"(v)
               : "v"(voff), "s"(uniform4(rsrc)), "s"(__builtin_amdgcn_readfirstlane(soff)));
  return v;
}
__device__ __forceinline__ void wr16(unsigned a, u32x4 v) { *reinterpret_cast<lds_v4*>(size_t(a)) = v; }

// s_waitcnt vmcnt(n) for a wave-uniform n < 64 known only at run time (prologue bookkeeping)
template <int N>
__device__ __forceinline__ void wait_vm_upto(int n) {
  if constexpr (N > 0) {
    if (n >= N) {
      wait_vm<N>();
      return;
    }
    wait_vm_upto<N - 1>(n);
  } else {
    wait_vm<0>();
  }
}

// 4- and 2-byte buffer stores whose out-of-range offsets (kOut) the hardware drops: the epilogue masks lanes and
// filters through the offset instead of the execution mask
__device__ __forceinline__ void store4(v4i rsrc, int voff, uint32_t v) {
  asm volatile("buffer_store_dword %0, %1, %2, 0 offen" ::"v"(v), "v"(voff), "s"(uniform4(rsrc)) : "memory");
}
// store4 with a wave-uniform byte offset added by the hardware (soffset): per-lane base offsets stay in registers
// across a loop whose steps differ only by a uniform displacement
__device__ __forceinline__ void store4s(v4i rsrc, int voff, int soff, uint32_t v) {
  asm volatile("buffer_store_dword %0, %1, %2, %3 offen" ::"v"(v), "v"(voff), "s"(uniform4(rsrc)),
               "s"(__builtin_amdgcn_readfirstlane(soff))
               : "memory");
}
__device__ __forceinline__ void store2(v4i rsrc, int voff, uint32_t v) {
  asm volatile("buffer_store_short %0, %1, %2, 0 offen" ::"v"(v), "v"(voff), "s"(uniform4(rsrc)) : "memory");
}

template <typename F, int... K>
__device__ __forceinline__ void for_seq(F&& f, std::integer_sequence<int, K...>) {
  (f(std::integral_constant<int, K>{}), ...);
}

}  // namespace gie_hip
