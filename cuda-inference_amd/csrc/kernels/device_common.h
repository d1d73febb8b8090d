// Device-side vocabulary shared by the gfx950 kernels: vector types, the 16-bit storage conversions and the
// fused epilogue. Private to csrc/kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
#include <mutex>
#include <set>
#include <utility>

#include "gie_hip.h"

namespace gie_hip {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Element-type tags; the storage of both is 16-bit, only the decode/encode and the MFMA opcode differ.
struct Fp16 {
  static constexpr int kDtype = GIE_HIP_FP16;
  static __device__ __forceinline__ float to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
  // v_cvt_f16_f32 rounds to nearest even in the default float mode
  static __device__ __forceinline__ uint16_t from_f32(float v) { return __builtin_bit_cast(uint16_t, (_Float16)v); }
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                  0, 0);
  }
  // two values rounded (nearest even) into one word, lo in bits 0-15: one v_cvt_pk_f16_f32 on gfx950
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, h2{(_Float16)lo, (_Float16)hi});
  }
};

struct Bf16 {
  static constexpr int kDtype = GIE_HIP_BF16;
  static __device__ __forceinline__ float to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }
  // IEEE round-to-nearest-even on the upper 16 bits; NaN stays a quiet NaN
  static __device__ __forceinline__ uint16_t from_f32(float v) {
    const uint32_t u = __float_as_uint(v);
    if ((u & 0x7fffffffu) > 0x7f800000u) return uint16_t((u >> 16) | 0x40u);
    return uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
  }
  static __device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  static __device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
  }
  // two values rounded (nearest even, NaN quieted) into one word, lo in bits 0-15: one v_cvt_pk_bf16_f32 on gfx950
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, b2{(__bf16)lo, (__bf16)hi});
  }
};

// Fused output stage: FP32 accumulator + bias, optional ReLU, then the single rounding to storage
// (same order as the reference's apply_epilogue, src/kernels/fused_epilogue.cuh:11-16).
template <typename E>
__device__ __forceinline__ uint16_t epilogue(float acc, const uint16_t* __restrict__ bias, int o, int relu) {
  if (bias != nullptr) acc += E::to_f32(bias[o]);
  if (relu) acc = fmaxf(acc, 0.0f);
  return E::from_f32(acc);
}

inline int ceil_div_i(long long a, long long b) { return int((a + b - 1) / b); }

// Sets a kernel's dynamic-LDS limit to `bytes` once per (function, device). Each host thread remembers the pairs it
// has seen set in a small direct-mapped table, so a launch loop takes no lock and touches no shared state; only a
// thread's first launch of a pair goes through the process-wide set under its mutex.
inline int lds_opt_in(const void* fn, int bytes) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return int(hipErrorInvalidDevice);
  struct Seen {
    const void* fn;
    int dev;
  };
  thread_local Seen seen[16] = {};
  Seen& slot = seen[((reinterpret_cast<uintptr_t>(fn) >> 8) ^ unsigned(dev)) & 15u];
  if (slot.fn == fn && slot.dev == dev) return GIE_HIP_OK;
  static std::mutex mu;
  static std::set<std::pair<const void*, int>> done;
  {
    std::lock_guard<std::mutex> lock(mu);
    if (!done.count({fn, dev})) {
      const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
      if (e != hipSuccess) return int(e);
      done.insert({fn, dev});
    }
  }
  slot = Seen{fn, dev};
  return GIE_HIP_OK;
}

// Compute units of the current device, queried once per device and kept (grid sizing on every launch must not
// pay an attribute query). 256 (MI355X) when the query fails.
inline int current_device_cus() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int cus = cached[dev].load(std::memory_order_relaxed);
  if (cus > 0) return cus;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
  cached[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

}  // namespace gie_hip
