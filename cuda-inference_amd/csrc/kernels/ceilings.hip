// Microbenchmarks behind the cost model's measured ceilings (the role of src/profiling/ceilings.cu:21-58):
// a matrix-core loop (4 independent 16x16x32 f16 MFMA chains per wave, operands in registers), a 16-byte
// vector copy for HBM bandwidth, and an empty kernel for launch cost. Each is a single launch timed by the caller.
#include "device_common.h"

namespace gie_hip {
namespace {

__global__ __launch_bounds__(256) void mfma_loop_kernel(int iters, float* __restrict__ sink) {
  const uint32_t t = threadIdx.x;
  u32x4 a = {t * 0x3c003c00u, t, t ^ 0x1234u, 0x3c00u};
  u32x4 b = {0x3c003c00u, t + 1u, 0x3800u, t};
  f32x4 c0 = {0, 0, 0, 0}, c1 = c0, c2 = c0, c3 = c0;
  for (int i = 0; i < iters; ++i) {
    c0 = Fp16::mfma(a, b, c0);
    c1 = Fp16::mfma(b, a, c1);
    c2 = Fp16::mfma(a, a, c2);
    c3 = Fp16::mfma(b, b, c3);
  }
  const float v = c0[0] + c1[1] + c2[2] + c3[3];
  if (v == 1234.5f) sink[blockIdx.x] = v;  // practically never true; keeps the loop alive
}

__global__ __launch_bounds__(256) void copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst, long long n) {
  for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * blockDim.x)
    dst[i] = src[i];
}

__global__ void empty_kernel() {}
__global__ void empty_kernel_ptr(int* sink) {
  if (threadIdx.x == 4096 && sink) sink[0] = 0;
}

__global__ __launch_bounds__(256) void fill_u16_kernel(uint16_t* __restrict__ dst, long long n, uint16_t v) {
  for (long long i = static_cast<long long>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<long long>(gridDim.x) * blockDim.x)
    dst[i] = v;
}

// Streaming probe: workgroup b reads its own r16 16-byte elements of src and writes its own w16 elements of dst
// (contiguous chunks), 512 elements per step; the reads are spread evenly over the steps. POL: 0 write-back
// stores, 1 device scope (sc1, written through the L2), 2 non-temporal.
template <int POL>
__device__ __forceinline__ void stream_store(u32x4* p, u32x4 v) {
  if constexpr (POL == 0)
    asm volatile("global_store_dwordx4 %0, %1, off\n\ts_nop 1" ::"v"(p), "v"(v) : "memory");
  else if constexpr (POL == 1)
    asm volatile("global_store_dwordx4 %0, %1, off sc1\n\ts_nop 1" ::"v"(p), "v"(v) : "memory");
  else
    asm volatile("global_store_dwordx4 %0, %1, off nt\n\ts_nop 1" ::"v"(p), "v"(v) : "memory");
}
template <int POL>
__global__ __launch_bounds__(512) void stream_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst,
                                                     long long r16, long long w16) {
  const long long rb = static_cast<long long>(blockIdx.x) * r16, wb = static_cast<long long>(blockIdx.x) * w16;
  const int t = threadIdx.x, nt = blockDim.x;
  const long long ws = (w16 + nt - 1) / nt, rs = (r16 + nt - 1) / nt, steps = ws > rs ? ws : rs;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (long long s = 0; s < steps; ++s) {
    const long long k = s * rs / steps;
    if (k != (s + 1) * rs / steps) {  // read step k (each of the rs read steps exactly once)
      const long long i = k * nt + t;
      if (i < r16) acc += src[rb + i];
    }
    if (s < ws) {
      const long long i = s * nt + t;
      if (i < w16) stream_store<POL>(dst + wb + i, u32x4{acc.x, unsigned(s), unsigned(t), 7u});
    }
  }
  if (acc.x == 0x9876543u && acc.y == 17u) dst[0] = acc;  // practically never true: keeps the reads
}

int launched() {
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? GIE_HIP_OK : int(e);
}

}  // namespace
}  // namespace gie_hip

using namespace gie_hip;

extern "C" int gie_hip_ceiling_mfma(int blocks, int iters, float* sink, void* stream) {
  if (blocks <= 0 || iters <= 0 || !sink) return GIE_HIP_EINVAL;
  hipLaunchKernelGGL(mfma_loop_kernel, dim3(unsigned(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream), iters, sink);
  return launched();
}

extern "C" int gie_hip_ceiling_copy(const void* src, void* dst, size_t bytes, void* stream) {
  if (!src || !dst || bytes == 0 || bytes % 16 != 0) return GIE_HIP_EINVAL;
  const long long n = static_cast<long long>(bytes / 16);
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  long long blocks = (n + 255) / 256;
  if (blocks > static_cast<long long>(cus) * 16) blocks = static_cast<long long>(cus) * 16;
  hipLaunchKernelGGL(copy_kernel, dim3(unsigned(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst), n);
  return launched();
}

extern "C" int gie_hip_ceiling_stream(const void* src, size_t read_bytes, void* dst, size_t write_bytes,
                                      int store_policy, int workgroups, void* stream) {
  if (workgroups <= 0 || store_policy < 0 || store_policy > 2 || !dst || (read_bytes > 0 && !src) ||
      (read_bytes == 0 && write_bytes == 0))
    return GIE_HIP_EINVAL;
  const size_t unit = 16 * static_cast<size_t>(workgroups);
  if (read_bytes % unit != 0 || write_bytes % unit != 0) return GIE_HIP_EINVAL;
  using Fn = void (*)(const u32x4*, u32x4*, long long, long long);
  const Fn fns[3] = {&stream_kernel<0>, &stream_kernel<1>, &stream_kernel<2>};
  hipLaunchKernelGGL(fns[store_policy], dim3(unsigned(workgroups)), dim3(512), 0, static_cast<hipStream_t>(stream),
                     static_cast<const u32x4*>(src), static_cast<u32x4*>(dst),
                     static_cast<long long>(read_bytes / unit), static_cast<long long>(write_bytes / unit));
  return launched();
}

extern "C" int gie_hip_ceiling_empty(void* stream) {
  hipLaunchKernelGGL(empty_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream));
  return launched();
}

namespace {
// an argument block of N dwords that the kernel reads (one lane of a lane id no launch has), so nothing is dropped
template <int N>
struct ArgBlock {
  int v[N];
};
template <int N>
__global__ void empty_args_kernel(ArgBlock<N> a, int* sink) {
  if (threadIdx.x == 4096 && sink) sink[0] = a.v[N - 1];
}
}  // namespace

extern "C" int gie_hip_ceiling_empty_args(int arg_bytes, void* stream) {
  const hipStream_t s = static_cast<hipStream_t>(stream);
  switch (arg_bytes) {
    case 8: hipLaunchKernelGGL(empty_kernel_ptr, dim3(1), dim3(64), 0, s, static_cast<int*>(nullptr)); break;
    case 128: hipLaunchKernelGGL(empty_args_kernel<30>, dim3(1), dim3(64), 0, s, ArgBlock<30>{}, nullptr); break;
    case 1024: hipLaunchKernelGGL(empty_args_kernel<254>, dim3(1), dim3(64), 0, s, ArgBlock<254>{}, nullptr); break;
    default: return GIE_HIP_EINVAL;
  }
  return launched();
}

extern "C" int gie_hip_fill_u16(void* dst, int64_t n, uint16_t value, void* stream) {
  if (!dst || n < 0) return GIE_HIP_EINVAL;
  if (n == 0) return GIE_HIP_OK;
  long long blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_u16_kernel, dim3(unsigned(blocks)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<uint16_t*>(dst), static_cast<long long>(n), value);
  return launched();
}
