// W4A16 (AWQ / GPTQ int4 weights, fp16/bf16 activations) for gfx950.
//
// Contract (reference kairyu/kernels/quant_gemm_gpu.py:224-407):
//   w[k, n] = fp16( (q - z) * s )       q, z 4-bit; s fp16 checkpoint scale
//   x       = fp16(x)   (bf16 finite values saturate to +-65504 first)
//   out     = sum_k x * w  accumulated in fp32, + bias, cast to x's dtype.
//
// Dequant happens in registers, two nibbles per 32-bit lane word: OR-ing a
// nibble into 0x6400 gives the fp16 value 1024+q, so (1024+q) - (1024+z) is
// exact and one packed fp16 multiply yields the same correctly rounded
// fp16((q-z)*s) as the reference's fp32 product rounded to fp16.
//
// Kernel (M <= 64 per row block): a workgroup owns 64 output columns; its
// waves take contiguous K ranges and each lane dequantizes straight into the
// B operand of v_mfma_f32_16x16x32_f16 (no LDS for weights); the waves reduce
// through LDS in fixed order.  Shapes with too few column tiles also split K
// across workgroups (partials + a separate reduce kernel).  Act-order GPTQ
// gathers x through the load-time permutation once per call into an fp16
// workspace buffer.  Larger M runs one grid row per 64-row block.
//
//   GPTQ (qweight [K/8, N], 8 consecutive k per word): lane (j = l%16,
//     kb = l/16) loads 4 adjacent columns' words of packed row kb; word t is
//     directly the B operand of MFMA t (k order [0,4,1,5,2,6,3,7], matched in
//     the A operand).  Output column of MFMA t, lane jj: base + 4*jj + t.
//   AWQ (qweight [K, N/8], 8 columns per word, order [0,2,4,6,1,3,5,7]): lane
//     loads the word of octet o = j%8 for rows k..k+7, keeps the column half
//     h = j/8 (4 columns), and transposes 2x2 fp16 blocks with v_perm_b32 so
//     each column's 8 k values form one B operand.  Output column of MFMA i,
//     lane jj: base + 8*(jj%8) + 4*(jj/8) + i.
#include "kq_common.h"
#include "kq_splitk.h"

#include <algorithm>

namespace kq {

enum { kAwq = 0, kGptq = 1 };
enum { kGroupsUniform = 0, kGroupsPermuted = 1, kGroupsPerK = 2 };

constexpr int kW4Cols = 64;   // columns per workgroup tile

struct W4Args {
  const uint16_t* x;
  int x_dtype;
  int ldx;
  bool x_vec;
  const uint32_t* qw;
  const uint32_t* qz;
  const uint16_t* sc;
  const int32_t* gidx;
  const int32_t* perm;
  const void* bias;
  int bias_dtype;
  uint16_t* out;
  int out_dtype;
  int M, N, K, G;
  int steps_per_split;
  int splits;
  float* partials;  // [splits][M][N] when splits > 1
};

KQ_DEV uint32_t pk_sub_mul(uint32_t q, uint32_t z, uint32_t s) {
  f16x2 r = (__builtin_bit_cast(f16x2, q) - __builtin_bit_cast(f16x2, z)) *
            __builtin_bit_cast(f16x2, s);
  return __builtin_bit_cast(uint32_t, r);
}

KQ_DEV uint32_t perm_lo(uint32_t hi_word, uint32_t lo_word) {
  return __builtin_amdgcn_perm(hi_word, lo_word, 0x05040100u);
}
KQ_DEV uint32_t perm_hi(uint32_t hi_word, uint32_t lo_word) {
  return __builtin_amdgcn_perm(hi_word, lo_word, 0x07060302u);
}

KQ_DEV uint16_t act_bits(uint16_t b, int dtype) {
  return __builtin_bit_cast(uint16_t, act_to_f16(b, dtype));
}

KQ_DEV uint32_t act_pair(uint32_t raw, int dtype) {
  if (dtype == KQ_DTYPE_F16) return raw;
  return (uint32_t)act_bits((uint16_t)(raw & 0xffffu), dtype) |
         ((uint32_t)act_bits((uint16_t)(raw >> 16), dtype) << 16);
}

// Eight fp16 activation values x[m][k..k+7] (natural k order), zero beyond
// the matrix.
KQ_DEV u32x4 load_x8(const W4Args& a, int m, int k) {
  u32x4 v = {0u, 0u, 0u, 0u};
  if (m >= a.M) return v;
  const uint16_t* row = a.x + (int64_t)m * a.ldx;
  if (a.x_vec && k + 8 <= a.K) {
    u32x4 raw = *(const u32x4*)(row + k);
#pragma unroll
    for (int d = 0; d < 4; ++d) v[d] = act_pair(raw[d], a.x_dtype);
    return v;
  }
  uint16_t h[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) h[e] = (k + e < a.K) ? act_bits(row[k + e], a.x_dtype) : 0;
#pragma unroll
  for (int d = 0; d < 4; ++d) v[d] = (uint32_t)h[2 * d] | ((uint32_t)h[2 * d + 1] << 16);
  return v;
}

// GPTQ A operand order [0,4,1,5,2,6,3,7] from natural pairs.
KQ_DEV u32x4 gptq_order(u32x4 n) {
  return u32x4{perm_lo(n[2], n[0]), perm_hi(n[2], n[0]), perm_lo(n[3], n[1]),
               perm_hi(n[3], n[1])};
}

KQ_DEV f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }

// Per-element dequant used by the arbitrary-g_idx path.
KQ_DEV uint16_t dq1(uint32_t q, uint32_t z, uint16_t s) {
  _Float16 d = (_Float16)((float)q - (float)z);  // exact small integer
  _Float16 r = d * __builtin_bit_cast(_Float16, s);
  return __builtin_bit_cast(uint16_t, r);
}

template <int FMT, int MT, int GMODE, int WAVES>
__global__ void __launch_bounds__(64 * WAVES)
w4a16_skinny_kernel(W4Args a) {
  __shared__ float red[(WAVES - 1) * MT * 16 * 64];
  const int lane = lane_id(), wave = wave_id();
  const int j = lane & 15, kb = lane >> 4;
  const int tile = blockIdx.x / a.splits, split = blockIdx.x % a.splits;
  const int colbase = tile * kW4Cols;
  const int mbase = blockIdx.y * (MT * 16);
  const int nsteps = (a.K + 31) / 32;
  const int sbeg = split * a.steps_per_split;
  const int send = min(nsteps, sbeg + a.steps_per_split);
  const int per_wave = (send - sbeg + WAVES - 1) / WAVES;
  const int wbeg = sbeg + wave * per_wave;
  const int wend = min(send, wbeg + per_wave);

  // columns handled by this lane
  const int o = j & 7, h = j >> 3;                    // AWQ octet / half
  const int gcol = colbase + 4 * j;                   // GPTQ first column
  const int acol = colbase + 8 * o + 4 * h;           // AWQ first column
  const bool col_ok = (FMT == kGptq ? gcol : acol) < a.N;
  const int n8 = a.N / 8;

  f32x4 acc[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  constexpr int U = FMT == kGptq ? 4 : 2;
  for (int st0 = wbeg; st0 < wend; st0 += U) {
    // ---- issue all weight loads of U steps first
    u32x4 wq[U];
    uint32_t wd[U][8];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int k = (st0 + u) * 32 + 8 * kb;
      const bool step_ok = (st0 + u) < wend;
      if constexpr (FMT == kGptq) {
        wq[u] = (step_ok && col_ok && k < a.K)
                    ? *(const u32x4*)(a.qw + (int64_t)(k >> 3) * a.N + gcol)
                    : u32x4{0u, 0u, 0u, 0u};
      } else {
#pragma unroll
        for (int t = 0; t < 8; ++t)
          wd[u][t] = (step_ok && col_ok && k + t < a.K)
                         ? a.qw[(int64_t)(k + t) * n8 + (colbase >> 3) + o]
                         : 0u;
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if ((st0 + u) >= wend) break;
      const int k = (st0 + u) * 32 + 8 * kb;
      u32x4 B[4];
      if constexpr (FMT == kGptq) {
        if constexpr (GMODE != kGroupsPerK) {
          const int g = min(k, a.K - 1) / a.G;
          const u32x2 sv = col_ok ? *(const u32x2*)(a.sc + (int64_t)g * a.N + gcol) : u32x2{0u, 0u};
          const uint32_t zw = col_ok ? a.qz[(int64_t)g * n8 + (gcol >> 3)] : 0u;
          const int zsh = 4 * (gcol & 7);
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const uint32_t z = ((zw >> (zsh + 4 * t)) & 0xfu) + 1u;
            const uint32_t zz = 0x64006400u + (z | (z << 16));
            const uint32_t s16 = (t & 1) ? (sv[t >> 1] >> 16) : (sv[t >> 1] & 0xffffu);
            const uint32_t ss = s16 | (s16 << 16);
            const uint32_t w = wq[u][t];
            B[t] = u32x4{pk_sub_mul((w & 0x000f000fu) | 0x64006400u, zz, ss),
                         pk_sub_mul(((w >> 4) & 0x000f000fu) | 0x64006400u, zz, ss),
                         pk_sub_mul(((w >> 8) & 0x000f000fu) | 0x64006400u, zz, ss),
                         pk_sub_mul(((w >> 12) & 0x000f000fu) | 0x64006400u, zz, ss)};
          }
        } else {
          // arbitrary g_idx: per element group, natural -> [0,4,1,5,...] order
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            uint16_t hv[8];
            const uint32_t w = wq[u][t];
            const int col = gcol + t;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const int kk = min(k + e, a.K - 1);
              const int g = a.gidx[kk];
              const uint32_t z = col_ok ? ((a.qz[(int64_t)g * n8 + (col >> 3)] >> (4 * (col & 7))) & 0xfu) + 1u : 0u;
              const uint16_t s = col_ok ? a.sc[(int64_t)g * a.N + col] : 0;
              hv[e] = dq1((w >> (4 * e)) & 0xfu, z, s);
            }
            B[t] = u32x4{(uint32_t)hv[0] | ((uint32_t)hv[4] << 16),
                         (uint32_t)hv[1] | ((uint32_t)hv[5] << 16),
                         (uint32_t)hv[2] | ((uint32_t)hv[6] << 16),
                         (uint32_t)hv[3] | ((uint32_t)hv[7] << 16)};
          }
        }
      } else {
        uint32_t wa[8], wb[8];
        const int zsh = 8 * h;
        // group parameters: (zero pair, scale pair) for columns 4h..4h+1 and
        // 4h+2..4h+3 of the octet; one group per 8-row chunk unless the
        // per-k path re-reads them for every row.
        u32x2 sv = {0u, 0u};
        uint32_t zp0 = 0u, zp1 = 0u;
        auto group_params = [&](int row) {
          const int g = min(row, a.K - 1) / a.G;
          sv = col_ok ? *(const u32x2*)(a.sc + (int64_t)g * a.N + acol) : u32x2{0u, 0u};
          const uint32_t zw = col_ok ? a.qz[(int64_t)g * n8 + (colbase >> 3) + o] : 0u;
          zp0 = ((zw >> zsh) & 0x000f000fu) | 0x64006400u;
          zp1 = ((zw >> (zsh + 4)) & 0x000f000fu) | 0x64006400u;
        };
        if constexpr (GMODE != kGroupsPerK) group_params(k);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          if constexpr (GMODE == kGroupsPerK) group_params(k + t);
          const uint32_t x = wd[u][t] >> zsh;
          wa[t] = pk_sub_mul((x & 0x000f000fu) | 0x64006400u, zp0, sv[0]);
          wb[t] = pk_sub_mul(((x >> 4) & 0x000f000fu) | 0x64006400u, zp1, sv[1]);
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          B[0][p] = perm_lo(wa[2 * p + 1], wa[2 * p]);
          B[1][p] = perm_hi(wa[2 * p + 1], wa[2 * p]);
          B[2][p] = perm_lo(wb[2 * p + 1], wb[2 * p]);
          B[3][p] = perm_hi(wb[2 * p + 1], wb[2 * p]);
        }
      }
#pragma unroll
      for (int t = 0; t < MT; ++t) {
        u32x4 xv = load_x8(a, mbase + t * 16 + j, k);
        if constexpr (FMT == kGptq) xv = gptq_order(xv);
        const f16x8 A = as_f16x8(xv);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[t][i] = mfma_f16(A, as_f16x8(B[i]), acc[t][i]);
      }
    }
  }

  // ---- reduce the waves' K ranges in fixed order through LDS
  constexpr int E = MT * 16;  // floats per lane
  if (wave > 0) {
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          red[((wave - 1) * E + (t * 16 + i * 4 + r)) * 64 + lane] = acc[t][i][r];
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w = 1; w < WAVES; ++w)
#pragma unroll
    for (int t = 0; t < MT; ++t)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          acc[t][i][r] = __fadd_rn(acc[t][i][r], red[((w - 1) * E + (t * 16 + i * 4 + r)) * 64 + lane]);

  // ---- epilogue (+ bias, cast) or raw partial for the reduce kernel
  float* part = a.splits > 1 ? a.partials + (size_t)split * a.M * a.N : nullptr;
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int n = FMT == kGptq ? colbase + 4 * j + i : colbase + 8 * (j & 7) + 4 * (j >> 3) + i;
      if (n >= a.N) continue;
      const bool has_bias = a.bias_dtype != KQ_DTYPE_NONE && part == nullptr;
      const float bv = has_bias ? load_as_f32(a.bias, a.bias_dtype, n) : 0.0f;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = mbase + t * 16 + kb * 4 + r;
        if (m >= a.M) continue;
        float v = acc[t][i][r];
        if (part) {
          part[(int64_t)m * a.N + n] = v;
          continue;
        }
        if (has_bias) v = __fadd_rn(v, bv);
        a.out[(int64_t)m * a.N + n] = f32_to_out(v, a.out_dtype);
      }
    }
}

// x16[m][j] = fp16(x[m][perm[j]]) (act-order gather + W4A16 activation
// conversion), 8 elements per thread.
__global__ void w4a16_prep_x_kernel(const uint16_t* __restrict__ x, int dtype, int ldx,
                                    const int32_t* __restrict__ perm, int M, int K,
                                    uint16_t* __restrict__ x16) {
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (idx >= (int64_t)M * K) return;
  const int m = (int)(idx / K), k0 = (int)(idx % K);
  const uint16_t* row = x + (int64_t)m * ldx;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = k0 + e;
    if (k < K) x16[(int64_t)m * K + k] = act_bits(row[perm ? perm[k] : k], dtype);
  }
}

// Act-order repack: unpacked row j of the output = unpacked row perm[j].
__global__ void gptq_permute_kernel(const uint32_t* __restrict__ qw, const int32_t* __restrict__ perm,
                                    uint32_t* __restrict__ out, int N, int K) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)(K / 8) * N;
  if (idx >= total) return;
  const int n = (int)(idx % N);
  const int row8 = (int)(idx / N);
  uint32_t word = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int src = perm[row8 * 8 + e];
    const uint32_t q = (qw[(int64_t)(src >> 3) * N + n] >> (4 * (src & 7))) & 0xfu;
    word |= q << (4 * e);
  }
  out[idx] = word;
}

struct W4Plan {
  int mt, waves, mblocks, tiles, splits, steps_per_split;
  size_t x16_bytes, partial_bytes;
};

static W4Plan plan_w4(int M, int N, int K, bool needs_x16, size_t ws_bytes, bool have_ws) {
  W4Plan p{};
  const int mt_needed = M >= 64 ? 4 : (M + 15) / 16;
  p.mt = mt_needed <= 1 ? 1 : (mt_needed <= 2 ? 2 : 4);
  p.waves = p.mt == 1 ? 8 : 4;
  p.mblocks = (M + p.mt * 16 - 1) / (p.mt * 16);
  p.tiles = (N + kW4Cols - 1) / kW4Cols;
  p.x16_bytes = needs_x16 ? ((size_t)M * K * 2 + 255) / 256 * 256 : 0;
  const int nsteps = (K + 31) / 32;
  p.splits = 1;
  const size_t plane = (size_t)M * N * 4;
  while (have_ws && (int64_t)p.tiles * p.mblocks * p.splits < 256 &&
         nsteps / (p.splits * 2 * p.waves) >= 2 &&
         p.x16_bytes + plane * p.splits * 2 <= ws_bytes)
    p.splits *= 2;
  p.partial_bytes = p.splits > 1 ? plane * p.splits : 0;
  p.steps_per_split = (nsteps + p.splits - 1) / p.splits;
  return p;
}

template <int FMT, int GMODE>
static void launch_w4(const W4Args& a, const W4Plan& p, hipStream_t stream) {
  dim3 grid(p.tiles * p.splits, p.mblocks);
  if (p.mt == 1)
    hipLaunchKernelGGL((w4a16_skinny_kernel<FMT, 1, GMODE, 8>), grid, dim3(512), 0, stream, a);
  else if (p.mt == 2)
    hipLaunchKernelGGL((w4a16_skinny_kernel<FMT, 2, GMODE, 4>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((w4a16_skinny_kernel<FMT, 4, GMODE, 4>), grid, dim3(256), 0, stream, a);
}

static int run_w4(const char* what, int fmt, W4Args a, int gmode, void* workspace,
                  size_t ws_bytes, hipStream_t stream) {
  if (a.x_dtype != KQ_DTYPE_F16 && a.x_dtype != KQ_DTYPE_BF16) {
    set_error("%s: activation dtype must be fp16 or bf16", what);
    return KQ_EUNSUPPORTED;
  }
  if (a.M < 0 || a.N < 8 || a.K < 1 || (a.N % 8) != 0 || a.G < 1 || a.ldx < a.K) {
    set_error("%s: bad shape m=%d n=%d k=%d group=%d", what, a.M, a.N, a.K, a.G);
    return KQ_EINVAL;
  }
  if (fmt == kGptq && (a.K % 8) != 0) {
    set_error("%s: GPTQ needs k %% 8 == 0 (k=%d)", what, a.K);
    return KQ_EINVAL;
  }
  if (fmt == kAwq && (a.K % a.G) != 0) {
    set_error("%s: AWQ needs k %% group_size == 0", what);
    return KQ_EINVAL;
  }
  if (a.M == 0) return KQ_OK;
  const bool needs_x16 = gmode == kGroupsPermuted;
  W4Plan p = plan_w4(a.M, a.N, a.K, needs_x16, ws_bytes, workspace != nullptr);
  if (p.x16_bytes + p.partial_bytes > (workspace ? ws_bytes : 0)) {
    set_error("%s: workspace of %zu bytes is smaller than the %zu bytes this call needs", what,
              workspace ? ws_bytes : (size_t)0, p.x16_bytes + p.partial_bytes);
    return KQ_EWORKSPACE;
  }
  if (needs_x16) {
    uint16_t* x16 = (uint16_t*)workspace;
    const int64_t threads = ((int64_t)a.M * a.K + 7) / 8;
    hipLaunchKernelGGL(w4a16_prep_x_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       stream, a.x, a.x_dtype, a.ldx, a.perm, a.M, a.K, x16);
    a.x = x16;
    a.x_dtype = KQ_DTYPE_F16;
    a.ldx = a.K;
  }
  a.x_vec = ((uintptr_t)a.x % 16) == 0 && (a.ldx % 8) == 0;
  a.splits = p.splits;
  a.steps_per_split = p.steps_per_split;
  a.partials = p.splits > 1 ? (float*)((uint8_t*)workspace + p.x16_bytes) : nullptr;
  if (fmt == kGptq) {
    if (gmode == kGroupsPerK) launch_w4<kGptq, kGroupsPerK>(a, p, stream);
    else launch_w4<kGptq, kGroupsUniform>(a, p, stream);
  } else {
    if (gmode == kGroupsPerK) launch_w4<kAwq, kGroupsPerK>(a, p, stream);
    else launch_w4<kAwq, kGroupsUniform>(a, p, stream);
  }
  if (p.splits > 1) {
    ReduceArgs r{a.partials, p.splits, a.M, a.N, nullptr, nullptr, 0, a.bias, a.bias_dtype,
                 a.out, a.out_dtype, nullptr};
    launch_splitk_reduce(kReduceW4, r, stream);
  }
  return check_launch(what);
}

}  // namespace kq

using namespace kq;

extern "C" size_t kq_w4a16_workspace_size(int64_t m, int64_t n, int64_t k, int gidx_mode) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  // a generous workspace lets the planner choose split-K freely
  const W4Plan p = plan_w4((int)m, (int)n, (int)k, gidx_mode == kGroupsPermuted,
                           (size_t)1 << 40, true);
  return p.x16_bytes + p.partial_bytes;
}

extern "C" int kq_w4a16_awq_gemm(const void* x, int x_dtype, const int32_t* qweight,
                                 const int32_t* qzeros, const void* scales, const void* bias,
                                 int bias_dtype, void* out, int64_t m, int64_t n, int64_t k,
                                 int group_size, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) {
    set_error("kq_w4a16_awq_gemm: dimensions exceed int32");
    return KQ_EINVAL;
  }
  W4Args a{};
  a.x = (const uint16_t*)x; a.x_dtype = x_dtype; a.ldx = (int)k;
  a.qw = (const uint32_t*)qweight; a.qz = (const uint32_t*)qzeros; a.sc = (const uint16_t*)scales;
  a.bias = bias; a.bias_dtype = bias_dtype; a.out = (uint16_t*)out; a.out_dtype = x_dtype;
  a.M = (int)m; a.N = (int)n; a.K = (int)k; a.G = group_size;
  // the fast path needs every aligned 8-row chunk inside one group
  const int gmode = (group_size % 8 == 0) ? kGroupsUniform : kGroupsPerK;
  return run_w4("kq_w4a16_awq_gemm", kAwq, a, gmode, workspace, workspace_bytes,
                (hipStream_t)stream);
}

extern "C" int kq_w4a16_gptq_gemm(const void* x, int x_dtype, const int32_t* qweight,
                                  const int32_t* qzeros, const void* scales,
                                  const int32_t* g_idx, const int32_t* perm, int gidx_mode,
                                  const void* bias, int bias_dtype, void* out, int64_t m,
                                  int64_t n, int64_t k, int group_size, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) {
    set_error("kq_w4a16_gptq_gemm: dimensions exceed int32");
    return KQ_EINVAL;
  }
  if (gidx_mode < 0 || gidx_mode > 2 || (gidx_mode == 1 && perm == nullptr) ||
      (gidx_mode == 2 && g_idx == nullptr)) {
    set_error("kq_w4a16_gptq_gemm: bad gidx_mode %d", gidx_mode);
    return KQ_EINVAL;
  }
  if (gidx_mode != 2 && group_size % 8 != 0) {
    set_error("kq_w4a16_gptq_gemm: gidx_mode %d needs group_size %% 8 == 0", gidx_mode);
    return KQ_EINVAL;
  }
  W4Args a{};
  a.x = (const uint16_t*)x; a.x_dtype = x_dtype; a.ldx = (int)k;
  a.qw = (const uint32_t*)qweight; a.qz = (const uint32_t*)qzeros; a.sc = (const uint16_t*)scales;
  a.gidx = g_idx; a.perm = perm;
  a.bias = bias; a.bias_dtype = bias_dtype; a.out = (uint16_t*)out; a.out_dtype = x_dtype;
  a.M = (int)m; a.N = (int)n; a.K = (int)k; a.G = group_size;
  return run_w4("kq_w4a16_gptq_gemm", kGptq, a, gidx_mode, workspace, workspace_bytes,
                (hipStream_t)stream);
}

extern "C" int kq_gptq_permute_qweight(const int32_t* qweight, const int32_t* perm, int32_t* out,
                                       int64_t n, int64_t k, void* stream) {
  if (n < 1 || k < 8 || (k % 8) != 0 || n > 0x7fffffff || k > 0x7fffffff) {
    set_error("kq_gptq_permute_qweight: bad shape n=%lld k=%lld", (long long)n, (long long)k);
    return KQ_EINVAL;
  }
  const int64_t total = (k / 8) * n;
  hipLaunchKernelGGL(gptq_permute_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint32_t*)qweight, perm, (uint32_t*)out, (int)n,
                     (int)k);
  return check_launch("kq_gptq_permute_qweight");
}
