// Second pass of split-K: fixed-order sum of partial accumulators + epilogue.
#include "kq_splitk.h"

namespace kq {

// Sum of split s = 0..S-1 of element idx, in that order, then the epilogue.
template <int MODE>
KQ_DEV float reduce_epilogue(const ReduceArgs& a, int64_t idx, int m, int n, int64_t plane,
                             float xs, float ws) {
  float v;
  if constexpr (MODE == kReduceI8) {
    const int32_t* p = (const int32_t*)a.partials;
    int32_t acc = 0;
    for (int s = 0; s < a.splits; ++s) acc += p[s * plane + idx];
    if (a.acc_out) a.acc_out[idx] = acc;
    v = __fmul_rn(__fmul_rn((float)acc, xs), ws);
  } else {
    const float* p = (const float*)a.partials;
    float acc = 0.0f;
    for (int s = 0; s < a.splits; ++s) acc = __fadd_rn(acc, p[s * plane + idx]);
    v = MODE == kReduceFp8 ? __fmul_rn(__fmul_rn(acc, xs), ws) : acc;
  }
  if (a.bias_dtype != KQ_DTYPE_NONE) v = __fadd_rn(v, load_as_f32(a.bias, a.bias_dtype, n));
  return v;
}

// Thread = 4 consecutive outputs.  N % 4 == 0 (VEC): they share a row, so
// the partials load as 16-byte vectors and the outputs store as 8 bytes.
template <int MODE, bool VEC>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(ReduceArgs a) {
  const int64_t plane = (int64_t)a.M * a.N;
  const int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (base >= plane) return;
  const int m0 = (int)(base / a.N), n0 = (int)(base - (int64_t)m0 * a.N);
  auto wscale = [&](int n) -> float {
    if constexpr (MODE == kReduceW4) return 1.0f;
    else return (MODE == kReduceI8 || a.ws_per_channel) ? a.wscale[n] : a.wscale[0];
  };
  if constexpr (VEC) {
    const float xs = MODE == kReduceW4 ? 1.0f : a.xscale[m0];
    float v[4];
    if constexpr (MODE == kReduceI8) {
      i32x4 acc = i32x4{0, 0, 0, 0};
      for (int s = 0; s < a.splits; ++s) acc += *(const i32x4*)((const int32_t*)a.partials + s * plane + base);
      if (a.acc_out) *(i32x4*)(a.acc_out + base) = acc;
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = __fmul_rn(__fmul_rn((float)acc[q], xs), wscale(n0 + q));
    } else {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int s = 0; s < a.splits; ++s) {
        const f32x4 p = *(const f32x4*)((const float*)a.partials + s * plane + base);
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[q] = __fadd_rn(acc[q], p[q]);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
        v[q] = MODE == kReduceFp8 ? __fmul_rn(__fmul_rn(acc[q], xs), wscale(n0 + q)) : acc[q];
    }
    uint16_t o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (a.bias_dtype != KQ_DTYPE_NONE) v[q] = __fadd_rn(v[q], load_as_f32(a.bias, a.bias_dtype, n0 + q));
      o[q] = f32_to_out(v[q], a.out_dtype);
    }
    *(u32x2*)((uint16_t*)a.out + base) =
        u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
  } else {
    int m = m0, n = n0;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t idx = base + e;
      if (idx >= plane) return;
      const float xs = MODE == kReduceW4 ? 1.0f : a.xscale[m];
      ((uint16_t*)a.out)[idx] = f32_to_out(reduce_epilogue<MODE>(a, idx, m, n, plane, xs, wscale(n)), a.out_dtype);
      if (++n == a.N) { n = 0; ++m; }
    }
  }
}

void launch_splitk_reduce(int mode, const ReduceArgs& a, hipStream_t stream) {
  const int64_t total = (int64_t)a.M * a.N;
  const unsigned blocks = (unsigned)((total + 1023) / 1024);
  const bool vec = (a.N & 3) == 0 && ((uintptr_t)a.partials & 15) == 0 && ((uintptr_t)a.out & 7) == 0 &&
                   (!a.acc_out || ((uintptr_t)a.acc_out & 15) == 0);
#define KQ_REDUCE(M)                                                                            \
  if (vec) hipLaunchKernelGGL((splitk_reduce_kernel<M, true>), dim3(blocks), dim3(256), 0, stream, a); \
  else hipLaunchKernelGGL((splitk_reduce_kernel<M, false>), dim3(blocks), dim3(256), 0, stream, a);
  if (mode == kReduceI8) { KQ_REDUCE(kReduceI8) }
  else if (mode == kReduceFp8) { KQ_REDUCE(kReduceFp8) }
  else { KQ_REDUCE(kReduceW4) }
#undef KQ_REDUCE
}

}  // namespace kq
