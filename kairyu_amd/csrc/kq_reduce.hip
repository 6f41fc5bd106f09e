// Second pass of split-K: fixed-order sum of partial accumulators + epilogue.
#include "kq_splitk.h"

namespace kq {

template <int MODE>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(ReduceArgs a) {
  const int64_t total = (int64_t)a.M * a.N;
  const int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  const int64_t plane = total;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int64_t idx = base + e;
    if (idx >= total) return;
    const int m = (int)(idx / a.N), n = (int)(idx % a.N);
    float v;
    if constexpr (MODE == kReduceI8) {
      const int32_t* p = (const int32_t*)a.partials;
      int32_t acc = 0;
      for (int s = 0; s < a.splits; ++s) acc += p[s * plane + idx];
      if (a.acc_out) a.acc_out[idx] = acc;
      v = __fmul_rn((float)acc, a.xscale[m]);
      v = __fmul_rn(v, a.wscale[n]);
    } else {
      const float* p = (const float*)a.partials;
      float acc = 0.0f;
      for (int s = 0; s < a.splits; ++s) acc = __fadd_rn(acc, p[s * plane + idx]);
      if constexpr (MODE == kReduceFp8) {
        v = __fmul_rn(acc, a.xscale[m]);
        v = __fmul_rn(v, a.ws_per_channel ? a.wscale[n] : a.wscale[0]);
      } else {
        v = acc;
      }
    }
    if (a.bias_dtype != KQ_DTYPE_NONE) v = __fadd_rn(v, load_as_f32(a.bias, a.bias_dtype, n));
    ((uint16_t*)a.out)[idx] = f32_to_out(v, a.out_dtype);
  }
}

void launch_splitk_reduce(int mode, const ReduceArgs& a, hipStream_t stream) {
  const int64_t total = (int64_t)a.M * a.N;
  const unsigned blocks = (unsigned)((total + 1023) / 1024);
  if (mode == kReduceI8)
    hipLaunchKernelGGL(splitk_reduce_kernel<kReduceI8>, dim3(blocks), dim3(256), 0, stream, a);
  else if (mode == kReduceFp8)
    hipLaunchKernelGGL(splitk_reduce_kernel<kReduceFp8>, dim3(blocks), dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL(splitk_reduce_kernel<kReduceW4>, dim3(blocks), dim3(256), 0, stream, a);
}

}  // namespace kq
