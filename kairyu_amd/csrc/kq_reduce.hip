// Second pass of split-K: fixed-order sum of partial accumulators + epilogue.
#include "kq_splitk.h"

namespace kq {

// The kernels below request a thread's partials of every split (2 to 4,
// compile-time counts) or of kReduceBatch splits at a time (more splits;
// the last batch re-reads the last split for its empty slots) before adding
// them in split order.  (A load per split, waited for before the next, left
// the W4 decode reduce at 4.2 us for a 64 KB plane: four round trips in
// sequence.)
constexpr int kReduceBatch = 4;

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
// (The W8A8 modes with N % 8 == 0 take splitk_reduce8_kernel below.)
template <int MODE, bool VEC, int NS>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(ReduceArgs a) {
  constexpr int B = NS > 0 ? NS : kReduceBatch;  // partial loads in flight per batch
  const int splits = NS > 0 ? NS : a.splits;
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
      for (int s0 = 0; s0 < splits; s0 += B) {
        i32x4 p[B];
#pragma unroll
        for (int u = 0; u < B; ++u)
          p[u] = *(const i32x4*)((const int32_t*)a.partials + min(s0 + u, splits - 1) * plane + base);
#pragma unroll
        for (int u = 0; u < B; ++u)
          if (s0 + u < splits) acc += p[u];
      }
      if (a.acc_out) *(i32x4*)(a.acc_out + base) = acc;
#pragma unroll
      for (int q = 0; q < 4; ++q) v[q] = __fmul_rn(__fmul_rn((float)acc[q], xs), wscale(n0 + q));
    } else {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int s0 = 0; s0 < splits; s0 += B) {
        f32x4 p[B];
#pragma unroll
        for (int u = 0; u < B; ++u)
          p[u] = *(const f32x4*)((const float*)a.partials + min(s0 + u, splits - 1) * plane + base);
#pragma unroll
        for (int u = 0; u < B; ++u)
          if (s0 + u < splits) {
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[q] = __fadd_rn(acc[q], p[u][q]);
          }
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

// W8A8, N % 8 == 0: thread = 8 consecutive outputs of one row; per split two
// 16-byte partial loads (streamed: non-temporal), the weight scales as two
// 16-byte loads, one 16-byte store.  Same sums and roundings as above.
template <int MODE, int NS>
__global__ void __launch_bounds__(256) splitk_reduce8_kernel(ReduceArgs a) {
  constexpr int B = NS > 0 ? NS : kReduceBatch;  // partial loads in flight per batch
  const int splits = NS > 0 ? NS : a.splits;
  const int64_t plane = (int64_t)a.M * a.N;
  const int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (base >= plane) return;
  const int m0 = (int)(base / a.N), n0 = (int)(base - (int64_t)m0 * a.N);
  const float xs = a.xscale[m0];
  float ws[8];
  if (MODE == kReduceI8 || a.ws_per_channel) {
    const f32x4 w0 = *(const f32x4*)(a.wscale + n0), w1 = *(const f32x4*)(a.wscale + n0 + 4);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ws[q] = w0[q];
      ws[4 + q] = w1[q];
    }
  } else {
#pragma unroll
    for (int q = 0; q < 8; ++q) ws[q] = a.wscale[0];
  }
  float v[8];
  if constexpr (MODE == kReduceI8) {
    i32x4 lo = i32x4{0, 0, 0, 0}, hi = i32x4{0, 0, 0, 0};
    for (int s0 = 0; s0 < splits; s0 += B) {
      i32x4 pl[B], ph[B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const i32x4* p = (const i32x4*)((const int32_t*)a.partials + min(s0 + u, splits - 1) * plane + base);
        pl[u] = __builtin_nontemporal_load(p);
        ph[u] = __builtin_nontemporal_load(p + 1);
      }
#pragma unroll
      for (int u = 0; u < B; ++u)
        if (s0 + u < splits) {
          lo += pl[u];
          hi += ph[u];
        }
    }
    if (a.acc_out) {
      *(i32x4*)(a.acc_out + base) = lo;
      *(i32x4*)(a.acc_out + base + 4) = hi;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[q] = __fmul_rn(__fmul_rn((float)lo[q], xs), ws[q]);
      v[4 + q] = __fmul_rn(__fmul_rn((float)hi[q], xs), ws[4 + q]);
    }
  } else {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < splits; s0 += B) {
      f32x4 pl[B], ph[B];
#pragma unroll
      for (int u = 0; u < B; ++u) {
        const f32x4* p = (const f32x4*)((const float*)a.partials + min(s0 + u, splits - 1) * plane + base);
        pl[u] = __builtin_nontemporal_load(p);
        ph[u] = __builtin_nontemporal_load(p + 1);
      }
#pragma unroll
      for (int u = 0; u < B; ++u)
        if (s0 + u < splits) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            acc[q] = __fadd_rn(acc[q], pl[u][q]);
            acc[4 + q] = __fadd_rn(acc[4 + q], ph[u][q]);
          }
        }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) v[q] = __fmul_rn(__fmul_rn(acc[q], xs), ws[q]);
  }
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    float a0 = v[2 * q], a1 = v[2 * q + 1];
    if (a.bias_dtype != KQ_DTYPE_NONE) {
      a0 = __fadd_rn(a0, load_as_f32(a.bias, a.bias_dtype, n0 + 2 * q));
      a1 = __fadd_rn(a1, load_as_f32(a.bias, a.bias_dtype, n0 + 2 * q + 1));
    }
    o[q] = (uint32_t)f32_to_out(a0, a.out_dtype) | ((uint32_t)f32_to_out(a1, a.out_dtype) << 16);
  }
  *(u32x4*)((uint16_t*)a.out + base) = u32x4{o[0], o[1], o[2], o[3]};
}

// With SwiGLU: thread = one output (m, c); gate and up columns of the
// [M][2I] partial plane (swiglu 1: c and I + c, the W8A8 packs; 2: gate and
// up 16-column blocks alternating, (c / 16) * 32 + c % 16 and 16 on, the
// W4A16 interleaved operand), each summed and scaled as above, then
// swiglu_bits: the bits of the epilogue's store followed by the elementwise
// pass.
template <int MODE>
__global__ void __launch_bounds__(256) splitk_reduce_swiglu_kernel(ReduceArgs a) {
  const int I = a.N / 2;
  const int64_t plane = (int64_t)a.M * a.N;
  const int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= (int64_t)a.M * I) return;
  const int m = (int)(o / I), c = (int)(o - (int64_t)m * I);
  const int64_t row = (int64_t)m * a.N;
  const int ng = a.swiglu == 2 ? (c >> 4) * 32 + (c & 15) : c;
  const int nu = a.swiglu == 2 ? ng + 16 : I + c;
  auto wscale = [&](int n) -> float {
    if constexpr (MODE == kReduceW4) return 1.0f;
    else return (MODE == kReduceI8 || a.ws_per_channel) ? a.wscale[n] : a.wscale[0];
  };
  const float xs = MODE == kReduceW4 ? 1.0f : a.xscale[m];
  const float g = reduce_epilogue<MODE>(a, row + ng, m, ng, plane, xs, wscale(ng));
  const float u = reduce_epilogue<MODE>(a, row + nu, m, nu, plane, xs, wscale(nu));
  ((uint16_t*)a.out)[o] = swiglu_bits(g, u, a.out_dtype);
}

void launch_splitk_reduce(int mode, const ReduceArgs& a, hipStream_t stream) {
  const int64_t total = (int64_t)a.M * a.N;
  if (a.swiglu) {
    const dim3 g((unsigned)((total / 2 + 255) / 256)), b(256);
    if (mode == kReduceI8) hipLaunchKernelGGL(splitk_reduce_swiglu_kernel<kReduceI8>, g, b, 0, stream, a);
    else if (mode == kReduceFp8) hipLaunchKernelGGL(splitk_reduce_swiglu_kernel<kReduceFp8>, g, b, 0, stream, a);
    else hipLaunchKernelGGL(splitk_reduce_swiglu_kernel<kReduceW4>, g, b, 0, stream, a);
    return;
  }
  if (mode != kReduceW4 && (a.N & 7) == 0 && ((uintptr_t)a.partials & 15) == 0 &&
      ((uintptr_t)a.out & 15) == 0 && ((uintptr_t)a.wscale & 15) == 0 &&
      (!a.acc_out || ((uintptr_t)a.acc_out & 15) == 0)) {
    const dim3 g((unsigned)((total + 2047) / 2048)), b(256);
#define KQ_REDUCE8(M, NS) hipLaunchKernelGGL((splitk_reduce8_kernel<M, NS>), g, b, 0, stream, a)
#define KQ_REDUCE8_NS(M)                       \
  if (a.splits == 2) KQ_REDUCE8(M, 2);         \
  else if (a.splits == 3) KQ_REDUCE8(M, 3);    \
  else if (a.splits == 4) KQ_REDUCE8(M, 4);    \
  else KQ_REDUCE8(M, 0);
    if (mode == kReduceI8) { KQ_REDUCE8_NS(kReduceI8) }
    else { KQ_REDUCE8_NS(kReduceFp8) }
#undef KQ_REDUCE8_NS
#undef KQ_REDUCE8
    return;
  }
  const unsigned blocks = (unsigned)((total + 1023) / 1024);
  const bool vec = (a.N & 3) == 0 && ((uintptr_t)a.partials & 15) == 0 && ((uintptr_t)a.out & 7) == 0 &&
                   (!a.acc_out || ((uintptr_t)a.acc_out & 15) == 0);
#define KQ_REDUCE_V(M, NS) hipLaunchKernelGGL((splitk_reduce_kernel<M, true, NS>), dim3(blocks), dim3(256), 0, stream, a)
#define KQ_REDUCE(M)                                                                                 \
  if (!vec) hipLaunchKernelGGL((splitk_reduce_kernel<M, false, 0>), dim3(blocks), dim3(256), 0, stream, a); \
  else if (a.splits == 2) KQ_REDUCE_V(M, 2);                                                         \
  else if (a.splits == 3) KQ_REDUCE_V(M, 3);                                                         \
  else if (a.splits == 4) KQ_REDUCE_V(M, 4);                                                         \
  else KQ_REDUCE_V(M, 0);
  if (mode == kReduceI8) { KQ_REDUCE(kReduceI8) }
  else if (mode == kReduceFp8) { KQ_REDUCE(kReduceFp8) }
  else { KQ_REDUCE(kReduceW4) }
#undef KQ_REDUCE
#undef KQ_REDUCE_V
}

}  // namespace kq
