// Shared device/host helpers for the kairyu_amd quantized-linear kernels.
//
// Everything here is written for gfx950 (CDNA4): 64-lane wavefronts, MFMA
// matrix cores, 160 KB LDS per CU.  Numeric helpers mirror the rounding the
// reference's CPU oracle performs with torch on the host:
//   * bf16 <- fp32 : round-to-nearest-even (c10::BFloat16)
//   * fp16 <- fp32 : round-to-nearest-even (v_cvt_f16_f32, default mode)
//   * e4m3fn <- fp32 : round-to-nearest-even after the caller's +-448 clamp
//     (kairyu/quant/fp8.py:29,44 clamps before torch's non-saturating cast)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/kairyu_quant.h"

#define KQ_DEV __device__ __forceinline__

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

namespace kq {

// ---------------------------------------------------------------- host errors
void set_error(const char* fmt, ...);
int check_launch(const char* what);

// ---------------------------------------------------------- scalar converts
KQ_DEV float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

KQ_DEV uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

KQ_DEV float f16_to_f32(uint16_t b) {
  _Float16 h = __builtin_bit_cast(_Float16, b);
  return (float)h;
}

KQ_DEV uint16_t f32_to_f16(float f) {
  _Float16 h = (_Float16)f;
  return __builtin_bit_cast(uint16_t, h);
}

KQ_DEV float load_as_f32(const void* p, int dtype, int64_t i) {
  if (dtype == KQ_DTYPE_F32) return ((const float*)p)[i];
  uint16_t b = ((const uint16_t*)p)[i];
  return dtype == KQ_DTYPE_BF16 ? bf16_to_f32(b) : f16_to_f32(b);
}

KQ_DEV uint16_t f32_to_out(float v, int dtype) {
  return dtype == KQ_DTYPE_BF16 ? f32_to_bf16(v) : f32_to_f16(v);
}

// fp32 -> the activation dtype and back (round to nearest even)
KQ_DEV float round_act(float v, int dtype) {
  if (dtype == KQ_DTYPE_BF16) return (float)(__bf16)v;
  return (float)(_Float16)v;
}

// silu(gate) * up with torch's roundings on fp16 / bf16 tensors
// (kairyu/models/layers.py:243-244): gate and up rounded to the activation
// dtype, silu in fp32 (IEEE division) rounded, the product rounded.
KQ_DEV uint16_t swiglu_bits(float gate, float up, int dtype) {
  const float g = round_act(gate, dtype), u = round_act(up, dtype);
  const float s = round_act(__fdiv_rn(g, __fadd_rn(1.0f, expf(-g))), dtype);
  return f32_to_out(__fmul_rn(s, u), dtype);
}

// W4A16 activation operand: fp16 passes through, bf16 is widened and finite
// values beyond fp16's range saturate to +-65504 while inf/nan stay non-finite
// (reference contract, kairyu/kernels/quant_gemm_gpu.py:296-307).
KQ_DEV _Float16 act_to_f16(uint16_t b, int dtype) {
  if (dtype == KQ_DTYPE_F16) return __builtin_bit_cast(_Float16, b);
  float v = bf16_to_f32(b);
  const float inf = __builtin_inff();
  if (v > 65504.0f && v < inf) v = 65504.0f;
  if (v < -65504.0f && v > -inf) v = -65504.0f;
  return (_Float16)v;
}

// fp32 -> OCP e4m3fn (bias 7, max 448, no inf, nan = 0x7f), round to nearest
// even.  Inputs with |v| >= 448 saturate to +-448; callers clamp beforehand.
KQ_DEV uint32_t f32_to_e4m3(float v) {
  uint32_t u = __float_as_uint(v);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7fu;
  if (a >= 0x43e00000u) return sign | 0x7eu;          // >= 448
  if (a < 0x3c800000u) {                               // < 2^-6: quantum 2^-9
    float q = __builtin_rintf(__uint_as_float(a) * 512.0f);
    return sign | (uint32_t)q;                         // q in [0, 8]
  }
  uint32_t r = a + 0x7ffffu + ((a >> 20) & 1u);        // RNE to 3 mantissa bits
  uint32_t e = (r >> 23) - 120u;                       // rebias 127 -> 7
  uint32_t m = (r >> 20) & 7u;
  return sign | (e << 3) | m;
}

// Four e4m3 bytes of v0..v3 (little-endian) with the hardware converter
// (v_cvt_pk_fp8_f32: round to nearest even, OCP e4m3fn).  Bit-identical to
// f32_to_e4m3 for every |v| <= 448 (checked on gfx950 over all such fp32
// values); callers clamp to +-448 and keep NaN away from it.
KQ_DEV uint32_t pack4_e4m3(float v0, float v1, float v2, float v3) {
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(v0, v1, 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(v2, v3, w, true);
  return (uint32_t)w;
}

// v / s, rounded like IEEE division, from r = RN(1 / s): q0 = RN(v r) is within
// one ulp of v / s, and one fma remainder step rounds it correctly (Markstein's
// theorem) whenever the remainder v - q0 s is a normal float.  With
// s >= 2^-60 that holds for every quotient of magnitude >= 2^-10, i.e. for
// every quotient that does not quantize to zero in e4m3 or int8; copysign
// keeps the sign of a zero dividend (-0 / s = -0).  Checked against IEEE
// division on 2^32 random pairs on gfx950.
KQ_DEV float div_by_recip(float v, float s, float r) {
  const float q0 = v * r;
  const float e = fmaf(-q0, s, v);
  return __builtin_copysignf(fmaf(e, r, q0), v);
}

// max(amax, floor) that keeps a NaN amax (torch.clamp / numpy.maximum)
KQ_DEV float max_keep_nan(float a, float floor) { return a != a ? a : fmaxf(a, floor); }

// Clamp that keeps NaN (torch.clamp semantics).
KQ_DEV float clamp_keep_nan(float v, float lim) {
  return v < -lim ? -lim : (v > lim ? lim : v);
}

KQ_DEV float e4m3_to_f32(uint32_t b) {
  uint32_t s = b & 0x80u, e = (b >> 3) & 0xfu, m = b & 7u;
  float v;
  if (e == 0) v = (float)m * 0.001953125f;             // m * 2^-9
  else if (e == 15 && m == 7) v = __builtin_nanf("");
  else v = __uint_as_float(((e + 120u) << 23) | (m << 20));
  return s ? -v : v;
}

// ---------------------------------------------------------------- MFMA
// D = A * B + C.  Lane layouts (lane l, 64 lanes):
//   A (16 x K): row l%16, K-chunk (l/16); B (K x 16): column l%16, K-chunk (l/16)
//   D (16 x 16): rows 4*(l/16)+r (r=0..3), column l%16
KQ_DEV f32x4 mfma_f16(f16x8 a, f16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
KQ_DEV i32x4 mfma_i8(i32x4 a, i32x4 b, i32x4 c) {
  return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}
// e4m3 x e4m3, 16x16x128; E8M0 scale 127 == 2^0 on both operands.
KQ_DEV f32x4 mfma_fp8(i32x8 a, i32x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

// ------------------------------------------------------------- buffer loads
// Raw buffer loads: a 128-bit resource held in SGPRs (base, byte size, gfx9
// format word) plus a 32-bit per-lane byte offset and a uniform SGPR offset.
// No per-lane 64-bit address arithmetic; offsets at or beyond the resource's
// byte size read as 0.  `aux` bit 1 marks the access non-temporal.
}  // namespace kq
__device__ int32_t kq_rbl_i32(i32x4 rsrc, int32_t voff, int32_t soff, int32_t aux)
    __asm("llvm.amdgcn.raw.buffer.load.i32");
__device__ short kq_rbl_i16(i32x4 rsrc, int32_t voff, int32_t soff, int32_t aux)
    __asm("llvm.amdgcn.raw.buffer.load.i16");
__device__ i32x4 kq_rbl_v4i32(i32x4 rsrc, int32_t voff, int32_t soff, int32_t aux)
    __asm("llvm.amdgcn.raw.buffer.load.v4i32");
__device__ i32x2 kq_rbl_v2i32(i32x4 rsrc, int32_t voff, int32_t soff, int32_t aux)
    __asm("llvm.amdgcn.raw.buffer.load.v2i32");
// Global -> LDS without registers: lane i writes `size` (4, 12 or 16) bytes at
// lds + i * size (lds wave-uniform); counts on vmcnt like any buffer load.
__device__ void kq_rbl_lds(i32x4 rsrc, __attribute__((address_space(3))) void* lds, int32_t size,
                           int32_t voff, int32_t soff, int32_t off, int32_t aux)
    __asm("llvm.amdgcn.raw.buffer.load.lds");
namespace kq {

constexpr int32_t kAuxNT = 2;

KQ_DEV i32x4 make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)(uintptr_t)base;
  i32x4 r;
  r[0] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((int32_t)(uint32_t)(a >> 32));  // stride 0
  r[2] = __builtin_amdgcn_readfirstlane((int32_t)bytes);
  r[3] = 0x00020000;  // gfx9 buffer format word (32-bit data, no swizzle)
  return r;
}

// ------------------------------------------------------------- wave helpers
KQ_DEV int lane_id() { return (int)(threadIdx.x & 63); }
KQ_DEV int wave_id() { return (int)(threadIdx.x >> 6); }

// Wave-wide maximum of a 32-bit key, uniform result.  Within each row of 16
// lanes: quad exchanges (xor 1, xor 2), then half-row and row mirrors through
// DPP (register-to-register, no LDS round trip); the four row maxima are then
// read from lanes 0, 16, 32, 48.
template <int CTRL>
KQ_DEV uint32_t dpp_max_u32(uint32_t v) {
  return max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false));
}

KQ_DEV uint32_t wave_max_u32_dpp(uint32_t v) {
  v = dpp_max_u32<0xB1>(v);    // quad_perm [1,0,3,2]
  v = dpp_max_u32<0x4E>(v);    // quad_perm [2,3,0,1]
  v = dpp_max_u32<0x141>(v);   // row_half_mirror
  v = dpp_max_u32<0x140>(v);   // row_mirror
  uint32_t best = (uint32_t)__builtin_amdgcn_readlane((int)v, 0);
#pragma unroll
  for (int r = 1; r < 4; ++r) best = max(best, (uint32_t)__builtin_amdgcn_readlane((int)v, 16 * r));
  return best;
}

KQ_DEV float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

// Map a linear block id so that consecutive logical tiles land on the same
// XCD (gfx950 dispatches workgroups round-robin over 8 XCDs with separate L2s).
KQ_DEV int xcd_swizzle(int bid, int nblocks) {
  const int kXcd = 8;
  if (nblocks < kXcd || (nblocks % kXcd) != 0) return bid;
  int per = nblocks / kXcd;
  return (bid % kXcd) * per + (bid / kXcd);
}

}  // namespace kq
