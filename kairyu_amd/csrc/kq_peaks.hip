// Ceilings of the box that the roofline fractions are read against (no
// counterpart in the reference, whose microbenchmark records only its own
// kernels): a streaming read of a device buffer and a register-only MFMA loop
// for each matrix instruction the GEMMs use.  Nothing else calls them.
#include "kq_common.h"

namespace kq {

constexpr int kPeakThreads = 256;
constexpr int kStreamUnroll = 8;

// Every thread reads kStreamUnroll 16-byte words per step, grid-strided, so a
// wave's loads are whole 1 KB runs and each workgroup keeps 32 KB in flight.
// The words are folded with XOR and stored only when the fold equals `magic`
// (the host passes a value the data does not produce), so the loads stay live
// without a store per thread.
__global__ __launch_bounds__(kPeakThreads) void peak_stream_read_kernel(
    const i32x4* __restrict__ src, int64_t words, uint32_t magic, uint32_t* __restrict__ sink) {
  const int64_t stride = (int64_t)gridDim.x * kPeakThreads;
  int64_t i = (int64_t)blockIdx.x * kPeakThreads + threadIdx.x;
  uint32_t acc = 0;
  for (; i + (kStreamUnroll - 1) * stride < words; i += kStreamUnroll * stride) {
    i32x4 v[kStreamUnroll];
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) v[u] = __builtin_nontemporal_load(&src[i + u * stride]);
#pragma unroll
    for (int u = 0; u < kStreamUnroll; ++u) acc ^= (uint32_t)(v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3]);
  }
  for (; i < words; i += stride) {
    const i32x4 v = src[i];
    acc ^= (uint32_t)(v[0] ^ v[1] ^ v[2] ^ v[3]);
  }
  if (acc == magic) sink[(int64_t)blockIdx.x * kPeakThreads + threadIdx.x] = acc;
}

// KQ_PEAK_MFMA_CHAINS independent accumulators per wave (distinct start
// values, so the compiler cannot merge them), each advanced by one MFMA per
// iteration from operands held in registers: the matrix pipe sees independent
// work every issue slot and no memory traffic.
template <int KIND>
__global__ __launch_bounds__(kPeakThreads) void peak_mfma_kernel(int64_t iterations, uint32_t magic,
                                                                 uint32_t* __restrict__ sink) {
  const int lane = lane_id();
  uint32_t fold = 0;
  if constexpr (KIND == KQ_PEAK_FP16) {
    f16x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a[j] = (_Float16)(0.001f * (float)((lane + j) & 7));
      b[j] = (_Float16)(0.001f * (float)((lane * 3 + j) & 7));
    }
    f32x4 c[KQ_PEAK_MFMA_CHAINS];
#pragma unroll
    for (int q = 0; q < KQ_PEAK_MFMA_CHAINS; ++q) c[q] = f32x4{(float)q, 0.f, 0.f, 0.f};
    for (int64_t it = 0; it < iterations; ++it) {
#pragma unroll
      for (int q = 0; q < KQ_PEAK_MFMA_CHAINS; ++q) c[q] = mfma_f16(a, b, c[q]);
    }
#pragma unroll
    for (int q = 0; q < KQ_PEAK_MFMA_CHAINS; ++q) fold ^= __float_as_uint(c[q][0] + c[q][3]);
  } else if constexpr (KIND == KQ_PEAK_FP8) {
    i32x8 a, b;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      a[j] = 0x30303030 + ((lane + j) & 3);  // small finite e4m3 values
      b[j] = 0x28282828 + ((lane * 5 + j) & 3);
    }
    f32x4 c[KQ_PEAK_MFMA_CHAINS];
#pragma unroll
    for (int q = 0; q < KQ_PEAK_MFMA_CHAINS; ++q) c[q] = f32x4{(float)q, 0.f, 0.f, 0.f};
    for (int64_t it = 0; it < iterations; ++it) {
#pragma unroll
      for (int q = 0; q < KQ_PEAK_MFMA_CHAINS; ++q) c[q] = mfma_fp8(a, b, c[q]);
    }
#pragma unroll
    for (int q = 0; q < KQ_PEAK_MFMA_CHAINS; ++q) fold ^= __float_as_uint(c[q][0] + c[q][3]);
  } else {
    i32x4 a, b;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      a[j] = 0x01010101 * ((lane + j) & 1);
      b[j] = 0x01010101 * ((lane * 7 + j) & 1);
    }
    i32x4 c[KQ_PEAK_MFMA_CHAINS];
#pragma unroll
    for (int q = 0; q < KQ_PEAK_MFMA_CHAINS; ++q) c[q] = i32x4{q, 0, 0, 0};
    for (int64_t it = 0; it < iterations; ++it) {
#pragma unroll
      for (int q = 0; q < KQ_PEAK_MFMA_CHAINS; ++q) c[q] = mfma_i8(a, b, c[q]);
    }
#pragma unroll
    for (int q = 0; q < KQ_PEAK_MFMA_CHAINS; ++q) fold ^= (uint32_t)(c[q][0] + c[q][3]);
  }
  if (fold == magic) sink[(int64_t)blockIdx.x * kPeakThreads + threadIdx.x] = fold;
}

}  // namespace kq

using namespace kq;

extern "C" int kq_peak_stream_read(const void* src, int64_t bytes, int workgroups, void* sink,
                                   void* stream) {
  if (src == nullptr || sink == nullptr || bytes <= 0 || bytes % 16 != 0 ||
      ((uintptr_t)src & 15) != 0 || workgroups < 1 || workgroups > 65536) {
    set_error("kq_peak_stream_read: bad arguments (bytes=%lld, a positive multiple of 16 from a "
              "16-byte aligned address; workgroups=%d in [1, 65536]; a sink)", (long long)bytes,
              workgroups);
    return KQ_EINVAL;
  }
  hipLaunchKernelGGL(peak_stream_read_kernel, dim3((unsigned)workgroups), dim3(kPeakThreads), 0,
                     (hipStream_t)stream, (const i32x4*)src, bytes / 16, 0x9e3779b9u,
                     (uint32_t*)sink);
  return check_launch("kq_peak_stream_read");
}

extern "C" int kq_peak_mfma(int kind, int64_t iterations, int workgroups, void* sink, void* stream) {
  if (sink == nullptr || iterations < 1 || iterations > (1 << 24) || workgroups < 1 ||
      workgroups > 65536) {
    set_error("kq_peak_mfma: bad arguments (iterations=%lld in [1, 2^24], workgroups=%d in "
              "[1, 65536], a sink)", (long long)iterations, workgroups);
    return KQ_EINVAL;
  }
  const dim3 grid((unsigned)workgroups), block(kPeakThreads);
  switch (kind) {
    case KQ_PEAK_FP16:
      hipLaunchKernelGGL(peak_mfma_kernel<KQ_PEAK_FP16>, grid, block, 0, (hipStream_t)stream,
                         iterations, 0x9e3779b9u, (uint32_t*)sink);
      break;
    case KQ_PEAK_FP8:
      hipLaunchKernelGGL(peak_mfma_kernel<KQ_PEAK_FP8>, grid, block, 0, (hipStream_t)stream,
                         iterations, 0x9e3779b9u, (uint32_t*)sink);
      break;
    case KQ_PEAK_INT8:
      hipLaunchKernelGGL(peak_mfma_kernel<KQ_PEAK_INT8>, grid, block, 0, (hipStream_t)stream,
                         iterations, 0x9e3779b9u, (uint32_t*)sink);
      break;
    default:
      set_error("kq_peak_mfma: kind %d is not KQ_PEAK_FP16, KQ_PEAK_FP8 or KQ_PEAK_INT8", kind);
      return KQ_EINVAL;
  }
  return check_launch("kq_peak_mfma");
}
