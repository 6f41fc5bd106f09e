// Per-token activation kernels: row amax, INT8 and FP8 quantization.
//
// One workgroup (up to 1024 threads) per row; the row is read once into
// registers (8 elements per chunk, up to 8 chunks per thread: K <= 65536),
// reduced for its amax and quantized from registers.  Arithmetic follows
// the reference's CPU oracle exactly (kairyu/quant/int8.py:25-30,
// kairyu/quant/fp8.py:33-45): fp32 amax, IEEE division for the scale and for
// x/scale, round-half-even for INT8, RNE e4m3 after a +-448 clamp for FP8.
//
// Rows of finite values divide by one correctly rounded reciprocal per row
// plus an fma remainder step (div_by_recip: the IEEE quotient for every
// element that does not quantize to zero) and convert with v_cvt_pk_fp8_f32;
// rows holding inf / NaN, or static scales below 2^-60, take the
// per-element IEEE path.  The row amax is an integer max of |bits|: it
// orders inf and NaN above every finite magnitude, so it is the float amax of
// a finite row, inf for a row with inf, and NaN for a row with NaN (torch's
// amax and clamp propagate NaN into the scale).
#include "kq_common.h"

#include <algorithm>

namespace kq {

// Loads up to 8 consecutive elements of a fp16/bf16 row as fp32; elements at
// or beyond `k` read as 0.
KQ_DEV void load8_f32(const uint16_t* row, int64_t i, int64_t k, int dtype, bool vec_ok,
                      float v[8]) {
  if (vec_ok && i + 8 <= k) {
    u32x4 raw = *(const u32x4*)(row + i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t w = raw[j];
      uint16_t lo = (uint16_t)(w & 0xffffu), hi = (uint16_t)(w >> 16);
      v[2 * j] = dtype == KQ_DTYPE_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
      v[2 * j + 1] = dtype == KQ_DTYPE_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
    }
  } else {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      int64_t c = i + j;
      v[j] = c < k ? (dtype == KQ_DTYPE_BF16 ? bf16_to_f32(row[c]) : f16_to_f32(row[c])) : 0.0f;
    }
  }
}

// Block-wide maximum (every thread gets it).  One call per kernel: `red` is
// not reused afterwards, so no barrier follows the reads.
KQ_DEV uint32_t block_max_u32(uint32_t v, uint32_t* red) {
  v = wave_max_u32_dpp(v);
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  uint32_t r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = max(r, red[w]);
  return r;
}

// max |bits| over the row held in registers (finite rows: the bits of the amax)
template <int NCH>
KQ_DEV uint32_t row_abs_bits(float v[NCH][8]) {
  uint32_t m = 0;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int e = 0; e < 8; ++e) m = max(m, __float_as_uint(v[c][e]) & 0x7fffffffu);
  return m;
}

KQ_DEV float block_max(float v, float* red) {
  v = wave_max(v);
  if (lane_id() == 0) red[wave_id()] = v;
  __syncthreads();
  float r = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); ++w) r = fmaxf(r, red[w]);
  __syncthreads();
  return r;
}

// Single-pass row kernels: each thread holds NCH chunks of 8 elements of the
// row in registers (chunk c = tid + blockDim.x * i), so the row is read from
// HBM once; the amax is reduced across the workgroup and the quantized bytes
// are produced from the registers.
template <int NCH>
KQ_DEV float load_row_regs(const uint16_t* row, int64_t k, int dtype, bool vec_ok,
                           float v[NCH][8]) {
  float m = 0.0f;
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t i = ((int64_t)threadIdx.x + (int64_t)blockDim.x * c) * 8;
    load8_f32(row, i, k, dtype, vec_ok, v[c]);
#pragma unroll
    for (int e = 0; e < 8; ++e) m = fmaxf(m, fabsf(v[c][e]));
  }
  return m;
}

// The same row held as raw 16-bit pairs (4 registers per chunk instead of 8:
// more rows in flight per CU).  Elements at or beyond `k` read as 0.
template <int NCH>
KQ_DEV void load_row_raw(const uint16_t* row, int64_t k, bool vec_ok, u32x4 raw[NCH]) {
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t i = ((int64_t)threadIdx.x + (int64_t)blockDim.x * c) * 8;
    if (vec_ok && i + 8 <= k) {
      raw[c] = *(const u32x4*)(row + i);
    } else {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t lo = i + 2 * j < k ? row[i + 2 * j] : 0u;
        const uint32_t hi = i + 2 * j + 1 < k ? row[i + 2 * j + 1] : 0u;
        w[j] = lo | (hi << 16);
      }
      raw[c] = u32x4{w[0], w[1], w[2], w[3]};
    }
  }
}

// max |bits| of the row as fp32 bits: the 16-bit magnitudes order like their
// values (inf above every finite value, NaN above inf) in fp16 and bf16 alike,
// so the widened maximum magnitude is the fp32 amax of a finite row, inf for a
// row with inf and NaN for a row with NaN
template <int NCH>
KQ_DEV uint32_t row_abs_bits_raw(const u32x4 raw[NCH], int dtype) {
  uint32_t m = 0;
#pragma unroll
  for (int c = 0; c < NCH; ++c)
#pragma unroll
    for (int j = 0; j < 4; ++j) m = max(m, max(raw[c][j] & 0x7fffu, (raw[c][j] >> 16) & 0x7fffu));
  return __float_as_uint(dtype == KQ_DTYPE_BF16 ? bf16_to_f32((uint16_t)m) : f16_to_f32((uint16_t)m));
}

KQ_DEV void widen8(u32x4 raw, int dtype, float v[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint16_t lo = (uint16_t)(raw[j] & 0xffffu), hi = (uint16_t)(raw[j] >> 16);
    v[2 * j] = dtype == KQ_DTYPE_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
    v[2 * j + 1] = dtype == KQ_DTYPE_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
  }
}

template <int NCH>
__global__ void __launch_bounds__(1024)
row_amax_kernel(const uint16_t* __restrict__ x, int dtype, int64_t k, int64_t ldx,
                bool vec_ok, float* __restrict__ out) {
  __shared__ float red[16];
  float v[NCH][8];
  float m = load_row_regs<NCH>(x + (int64_t)blockIdx.x * ldx, k, dtype, vec_ok, v);
  m = block_max(m, red);
  if (threadIdx.x == 0) out[blockIdx.x] = m;
}

KQ_DEV void store8(uint8_t* qrow, int64_t i, int64_t k, uint32_t lo, uint32_t hi) {
  if (i + 8 <= k && (k & 7) == 0) {
    *(u32x2*)(qrow + i) = u32x2{lo, hi};
  } else {
    for (int j = 0; j < 8 && i + j < k; ++j)
      qrow[i + j] = (uint8_t)((((j < 4) ? lo : hi) >> (8 * (j & 3))) & 0xffu);
  }
}

template <int NCH>
__global__ void __launch_bounds__(1024)
act_quant_i8_kernel(const uint16_t* __restrict__ x, int dtype, int64_t k, int64_t ldx,
                    bool vec_ok, int8_t* __restrict__ xq, float* __restrict__ xscale) {
  __shared__ float red[16];
  const int64_t r = blockIdx.x;
  u32x4 raw[NCH];
  load_row_raw<NCH>(x + r * ldx, k, vec_ok, raw);
  const uint32_t abits = block_max_u32(row_abs_bits_raw<NCH>(raw, dtype), (uint32_t*)red);
  const bool fast = abits < 0x7f800000u;
  const float s = __fdiv_rn(max_keep_nan(__uint_as_float(abits), 1e-12f), 127.0f);
  const float rs = __fdiv_rn(1.0f, s);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t i = ((int64_t)threadIdx.x + (int64_t)blockDim.x * c) * 8;
    if (i >= k) break;
    float v[8];
    widen8(raw[c], dtype, v);
    uint32_t packed[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float q = fast ? __builtin_rintf(fminf(fmaxf(div_by_recip(v[e], s, rs), -127.0f), 127.0f))
                           : __builtin_rintf(clamp_keep_nan(__fdiv_rn(v[e], s), 127.0f));
      packed[e >> 2] |= ((uint32_t)(int32_t)q & 0xffu) << (8 * (e & 3));
    }
    store8((uint8_t*)xq + r * k, i, k, packed[0], packed[1]);
  }
  if (threadIdx.x == 0) xscale[r] = s;
}

template <int NCH>
__global__ void __launch_bounds__(1024)
act_quant_fp8_kernel(const uint16_t* __restrict__ x, int dtype, int64_t k, int64_t ldx,
                     bool vec_ok, const float* __restrict__ scale_in, int scale_mode,
                     uint8_t* __restrict__ xq, float* __restrict__ xscale) {
  __shared__ float red[16];
  const int64_t r = blockIdx.x;
  u32x4 raw[NCH];
  load_row_raw<NCH>(x + r * ldx, k, vec_ok, raw);
  const uint32_t abits = block_max_u32(row_abs_bits_raw<NCH>(raw, dtype), (uint32_t*)red);
  bool fast = abits < 0x7f800000u;
  float s;
  if (scale_mode == 0) {
    s = __fdiv_rn(max_keep_nan(__uint_as_float(abits), 1e-12f), 448.0f);
  } else {
    s = scale_mode == 1 ? scale_in[0] : scale_in[r];
    fast = fast && s >= 0x1p-60f && s <= 3.4028235e38f;
  }
  const float rs = __fdiv_rn(1.0f, s);
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int64_t i = ((int64_t)threadIdx.x + (int64_t)blockDim.x * c) * 8;
    if (i >= k) break;
    float v[8];
    widen8(raw[c], dtype, v);
    uint32_t packed[2] = {0u, 0u};
    if (fast) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float q[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) q[e] = fminf(fmaxf(div_by_recip(v[4 * h + e], s, rs), -448.0f), 448.0f);
        packed[h] = pack4_e4m3(q[0], q[1], q[2], q[3]);
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        packed[e >> 2] |= f32_to_e4m3(clamp_keep_nan(__fdiv_rn(v[e], s), 448.0f)) << (8 * (e & 3));
    }
    store8(xq + r * k, i, k, packed[0], packed[1]);
  }
  if (threadIdx.x == 0) xscale[r] = s;
}

// Row geometry: threads (multiple of 64, <= 1024) and chunks per thread.
struct RowPlan {
  int threads, nch;
};

// A row's load -> amax -> quantize -> store chain is latency-bound.  With at
// least one row per CU, about 256 threads per row keep several rows in flight
// on every CU; with fewer rows than CUs (decode batches) each row has a CU to
// itself, so up to 1024 threads per row shorten its serial chain instead.
static RowPlan plan_rows(int64_t rows, int64_t k) {
  const int64_t chunks = (k + 7) / 8;
  const int64_t tmax = rows < 256 ? 1024 : 256;
  RowPlan p{};
  p.nch = chunks <= tmax ? 1 : (chunks <= 2 * tmax ? 2 : (chunks <= 4 * tmax ? 4 : 8));
  const int64_t per = (chunks + p.nch - 1) / p.nch;
  p.threads = (int)std::min<int64_t>(1024, std::max<int64_t>(64, (per + 63) / 64 * 64));
  return p;
}

static int check_rows(const char* what, const void* x, int dtype, int64_t rows, int64_t k,
                      int64_t ldx) {
  if (dtype != KQ_DTYPE_F16 && dtype != KQ_DTYPE_BF16) {
    set_error("%s: activation dtype must be fp16 or bf16 (code %d)", what, dtype);
    return KQ_EUNSUPPORTED;
  }
  if (rows < 0 || k < 1 || ldx < k || rows > 0x7fffffffLL || k > 65536) {
    set_error("%s: bad shape rows=%lld k=%lld ldx=%lld", what, (long long)rows,
              (long long)k, (long long)ldx);
    return KQ_EINVAL;
  }
  if (rows > 0 && x == nullptr) {
    set_error("%s: null activation", what);
    return KQ_EINVAL;
  }
  return KQ_OK;
}

static bool vec_ok(const void* x, int64_t ldx) {
  return ((uintptr_t)x % 16) == 0 && (ldx % 8) == 0;
}

}  // namespace kq

using namespace kq;

extern "C" int kq_row_amax(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                           float* amax, void* stream) {
  int rc = check_rows("kq_row_amax", x, x_dtype, rows, k, ldx);
  if (rc) return rc;
  if (rows == 0) return KQ_OK;
  const RowPlan p = plan_rows(rows, k);
  const bool v = vec_ok(x, ldx);
  const dim3 g((unsigned)rows), b(p.threads);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xs = (const uint16_t*)x;
  switch (p.nch) {
    case 1: hipLaunchKernelGGL(row_amax_kernel<1>, g, b, 0, st, xs, x_dtype, k, ldx, v, amax); break;
    case 2: hipLaunchKernelGGL(row_amax_kernel<2>, g, b, 0, st, xs, x_dtype, k, ldx, v, amax); break;
    case 4: hipLaunchKernelGGL(row_amax_kernel<4>, g, b, 0, st, xs, x_dtype, k, ldx, v, amax); break;
    default: hipLaunchKernelGGL(row_amax_kernel<8>, g, b, 0, st, xs, x_dtype, k, ldx, v, amax); break;
  }
  return check_launch("kq_row_amax");
}

extern "C" int kq_act_quant_i8(const void* x, int x_dtype, int64_t rows, int64_t k,
                               int64_t ldx, int8_t* xq, float* xscale, void* stream) {
  int rc = check_rows("kq_act_quant_i8", x, x_dtype, rows, k, ldx);
  if (rc) return rc;
  if (rows == 0) return KQ_OK;
  const RowPlan p = plan_rows(rows, k);
  const bool v = vec_ok(x, ldx);
  const dim3 g((unsigned)rows), b(p.threads);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xs = (const uint16_t*)x;
  switch (p.nch) {
    case 1: hipLaunchKernelGGL(act_quant_i8_kernel<1>, g, b, 0, st, xs, x_dtype, k, ldx, v, xq, xscale); break;
    case 2: hipLaunchKernelGGL(act_quant_i8_kernel<2>, g, b, 0, st, xs, x_dtype, k, ldx, v, xq, xscale); break;
    case 4: hipLaunchKernelGGL(act_quant_i8_kernel<4>, g, b, 0, st, xs, x_dtype, k, ldx, v, xq, xscale); break;
    default: hipLaunchKernelGGL(act_quant_i8_kernel<8>, g, b, 0, st, xs, x_dtype, k, ldx, v, xq, xscale); break;
  }
  return check_launch("kq_act_quant_i8");
}

extern "C" int kq_act_quant_fp8(const void* x, int x_dtype, int64_t rows, int64_t k,
                                int64_t ldx, const float* scale_in, int scale_mode,
                                uint8_t* xq, float* xscale, void* stream) {
  int rc = check_rows("kq_act_quant_fp8", x, x_dtype, rows, k, ldx);
  if (rc) return rc;
  if (scale_mode < 0 || scale_mode > 2 || (scale_mode != 0 && scale_in == nullptr)) {
    set_error("kq_act_quant_fp8: bad scale_mode %d", scale_mode);
    return KQ_EINVAL;
  }
  if (rows == 0) return KQ_OK;
  const RowPlan p = plan_rows(rows, k);
  const bool v = vec_ok(x, ldx);
  const dim3 g((unsigned)rows), b(p.threads);
  hipStream_t st = (hipStream_t)stream;
  const uint16_t* xs = (const uint16_t*)x;
  switch (p.nch) {
    case 1: hipLaunchKernelGGL(act_quant_fp8_kernel<1>, g, b, 0, st, xs, x_dtype, k, ldx, v, scale_in, scale_mode, xq, xscale); break;
    case 2: hipLaunchKernelGGL(act_quant_fp8_kernel<2>, g, b, 0, st, xs, x_dtype, k, ldx, v, scale_in, scale_mode, xq, xscale); break;
    case 4: hipLaunchKernelGGL(act_quant_fp8_kernel<4>, g, b, 0, st, xs, x_dtype, k, ldx, v, scale_in, scale_mode, xq, xscale); break;
    default: hipLaunchKernelGGL(act_quant_fp8_kernel<8>, g, b, 0, st, xs, x_dtype, k, ldx, v, scale_in, scale_mode, xq, xscale); break;
  }
  return check_launch("kq_act_quant_fp8");
}
