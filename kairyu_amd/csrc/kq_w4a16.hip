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
// Kernels:
//   * decode GEMV (M <= 16, K % 128 == 0, load-time tiled weights): 16-wave
//     workgroups, x held in registers, weights streamed through buffer loads
//     with three 16-column blocks in flight; K beyond 4096 split across
//     workgroups (below);
//   * skinny kernel (every other shape, checkpoint or tiled layout), next.
//
// Skinny kernel (M <= 64 per row block): a workgroup owns 64 output columns; its
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
#include "kq_tile_gemm.h"  // LDS-DMA helpers (tg_dma16 / tg_dma4), kTgOob

#include <algorithm>
#include <mutex>

namespace kq {

enum { kAwq = 0, kGptq = 1 };
// Host-side group modes (ABI gidx_mode) ...
enum { kGroupsUniform = 0, kGroupsPermuted = 1, kGroupsPerK = 2 };
// ... and the kernel's group addressing: one group per step for the whole
// wave (group_size % 32 == 0, computed on the scalar unit), one group per
// lane's 8-k chunk (group_size % 8 == 0), or a group per element (g_idx).
enum { kGStep = 0, kGLane = 1, kGElem = 2 };
enum { kXF16 = 0, kXBF16 = 1 };
// qweight layouts (8 consecutive k per word, LSB first): [K/8][N] words
// (checkpoint GPTQ order) or 16-column tiles [ceil(N/16)][K/8][16] (each
// tile's words contiguous, built at load time by kq_w4a16_tile_weights)
enum { kLayoutRows = 0, kLayoutTiles = 1 };
// decode GEMV only: tiles whose table holds scales alone (one zero for all)
constexpr int kLayoutTilesZu = 2;

constexpr int kW4Cols = 64;   // columns per workgroup tile

// Load-time tile layout of the W4A16 weights ("tiles"): 16-column tiles of
// 128-k stages.  Within a tile's stage (16 packed rows of 8 k x 16 columns =
// 1 KB), word (row 4s + kb, column c) sits at (kb * 16 + c) * 4 + s: the four
// steps (32 k each) a lane (c, kb) of a 16x16x32 MFMA B operand consumes are
// one contiguous 16 bytes.  Tile u, stage t starts at word (u * T + t) * 256
// with T = ceil(K / 128) stages (rows past K / 8 are zero).
__host__ __device__ inline int w4_stages(int K) { return (K + 127) / 128; }
__host__ __device__ inline int64_t w4_tile_words(int N, int K) {
  return (int64_t)((N + 15) / 16) * w4_stages(K) * 256;
}
// The tiled operand continues with a scale/zero table read by the decode
// GEMV: for tile u and group pair p (groups 2p, 2p + 1), 16 columns x 2
// groups of one word each, scale bits | (zero nibble + zero offset) << 16, at
// word (u * P + p) * 32 + c * 2 + (g & 1), P = ceil(groups / 2); groups past
// the last and columns past N are 0.  A lane (c, kb) gets the scales and
// zeros of its column for two consecutive groups with one 8-byte load.
// With one zero for every group and column (symmetric checkpoints, "zu") the
// table holds the scales alone, word (u * P + p) * 16 + c = scale of group 2p
// | scale of group 2p + 1 << 16 (4 bytes per lane and group pair, 2 bytes per
// group and column as in the checkpoint), followed by groups x N/8 zero
// words of nibble 0 (the zero is then the zero offset) for the kernels that
// read zero words.
__host__ __device__ inline int w4_group_pairs(int K, int G) { return ((K + G - 1) / G + 1) / 2; }
__host__ __device__ inline int64_t w4_table_words(int N, int K, int G, bool zu) {
  return (int64_t)((N + 15) / 16) * w4_group_pairs(K, G) * (zu ? 16 : 32);
}
__host__ __device__ inline int64_t w4_zero_area_words(int N, int K, int G, bool zu) {
  return zu ? (int64_t)((K + G - 1) / G) * (N / 8) : 0;
}
__host__ __device__ inline int64_t w4_tiled_words(int N, int K, int G, bool zu) {
  return w4_tile_words(N, K) + w4_table_words(N, K, G, zu) + w4_zero_area_words(N, K, G, zu);
}

struct W4Args {
  const uint16_t* x;     // activation rows (fp16 or bf16 per kernel template)
  int ldx;
  int x_dtype;           // caller's activation dtype
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
  uint64_t gmagic;       // floor(k / G) == (k * gmagic) >> 40 for k < 2^24
  int steps_per_split;
  int splits;
  float* partials;       // [splits][M][N] when splits > 1
  uint32_t zoff;         // added to stored zero nibbles (GPTQ 1, natural-order AWQ 0)
  int layout;            // kLayoutRows (qweight [K/8][N]) or kLayoutTiles
  int zu;                // tiles built with one zero for every group and column (zoff)
  int swiglu;            // N = 2I gate/up columns interleaved by 16; out [M][I] = silu(gate) * up
  int swiglu_split;      // the same output from the split-K reduce of a plain GEMV over those columns
};

KQ_DEV int group_of(const W4Args& a, int k) {
  return (int)(((uint64_t)(uint32_t)k * a.gmagic) >> 40);
}

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

// bf16 -> fp16 with finite saturation to +-65504, inf/nan kept (see act_to_f16)
KQ_DEV _Float16 bf16f_to_f16_sat(float f) {
  const float c = __builtin_amdgcn_fmed3f(f, -65504.0f, 65504.0f);
  // class mask: signaling/quiet nan (0x3) | -inf (0x4) | +inf (0x200)
  const bool keep = __builtin_amdgcn_class(f, 0x207);
  return (_Float16)(keep ? f : c);
}

KQ_DEV uint32_t bf16x2_to_f16x2(uint32_t raw) {
  const _Float16 lo = bf16f_to_f16_sat(__uint_as_float(raw << 16));
  const _Float16 hi = bf16f_to_f16_sat(__uint_as_float(raw & 0xffff0000u));
  return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

template <int XDT>
KQ_DEV u32x4 x_to_f16(u32x4 raw) {
  if constexpr (XDT == kXF16) return raw;
  return u32x4{bf16x2_to_f16x2(raw[0]), bf16x2_to_f16x2(raw[1]), bf16x2_to_f16x2(raw[2]),
               bf16x2_to_f16x2(raw[3])};
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

// Register batch of U consecutive 32-k steps for one lane: packed weights,
// the group's scale/zero words and the raw activation chunks.
template <int FMT, int MT, int U>
struct W4Batch {
  u32x4 wq[FMT == kGptq ? U : 1];      // GPTQ: 4 columns' words of packed row
  uint32_t wd[FMT == kAwq ? U : 1][8]; // AWQ: octet word of rows k..k+7
  u32x2 sv[U];                         // fp16 scales of the lane's 4 columns
  uint32_t zw[U];                      // zero word holding those columns
  u32x4 xv[U][MT];                     // raw x[m][k..k+7]
};

// Load through a base pointer plus a 32-bit byte offset; with a wave-uniform
// base this is the global_load "saddr" form (no per-lane 64-bit addressing).
template <typename T>
KQ_DEV T ldb(const void* base, uint32_t byte_off) {
  return *(const T*)((const char*)base + byte_off);
}
template <typename T, bool NT>
KQ_DEV T ldw(const void* base, uint32_t byte_off) {
  if constexpr (NT) return __builtin_nontemporal_load((const T*)((const char*)base + byte_off));
  else return *(const T*)((const char*)base + byte_off);
}

// (x & mask) | magic in one VOP3 (gfx9 allows a single SGPR/literal operand,
// so the magic constant lives in a VGPR).
KQ_DEV uint32_t and_or(uint32_t x, uint32_t mask, uint32_t magic) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(x), "s"(mask), "v"(magic));
  return r;
}

// silu(gate) * up as torch computes it on fp16 / bf16 tensors (layers.py
// `silu(gate_proj(x)) * up_proj(x)`, kairyu/models/layers.py:243-244): gate and
// up rounded to the activation dtype, silu in fp32 (x / (1 + exp(-x)), IEEE
// division) rounded, the product in fp32 rounded.

// Nibble pairs of a 32-bit word as fp16 (base + q) pairs: OR-ing the nibble at
// bits 0-3 of each half into 0x6400 gives 1024+q; the nibble at bits 4-7 into
// 0x5400 gives 64+q (the nibble lands on the mantissa's unit place in both
// binades).  Bits 8-15 would reach the exponent field, so the upper byte of
// each half is shifted down first.
struct NibbleConsts {
  uint32_t m0, m1;  // SGPR masks 0x000f000f, 0x00f000f0
  uint32_t c0, c1;  // VGPR magics: fp16 pairs (1024, 1024), (64, 64)
};

// PRED = false: every step of the kernel is a full 32-k step and x rows are
// 16-byte aligned; loads carry no predicates (columns and rows are clamped to
// valid addresses and the surplus results are never stored).  PRED = true
// guards every load (K tails, unaligned x).  U = steps per register batch
// (two batches in flight), NT = weights streamed with non-temporal loads.
template <int FMT, int MT, int GM, int XDT, bool PRED, int WAVES, int U, bool NT>
__global__ void __launch_bounds__(64 * WAVES)
w4a16_skinny_kernel(W4Args a) {
  __shared__ float red[(WAVES - 1) * MT * 16 * 64];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int j = lane & 15, kb = lane >> 4;
  const int tile = blockIdx.x / a.splits, split = blockIdx.x % a.splits;
  const int colbase = tile * kW4Cols;
  const int mbase = blockIdx.y * (MT * 16);
  const int nsteps = (a.K + 31) / 32;
  const int sbeg = split * a.steps_per_split;
  const int send = min(nsteps, sbeg + a.steps_per_split);
  // waves take contiguous, batch-aligned step ranges
  const int per_wave = ((send - sbeg + WAVES - 1) / WAVES + U - 1) / U * U;
  const int wbeg = sbeg + wave * per_wave;
  const int wend = min(send, wbeg + per_wave);

  // the lane's 4 columns, clamped to valid memory
  const int o = j & 7, h = j >> 3;                        // AWQ octet / half
  const int lcol = FMT == kGptq ? colbase + 4 * j : colbase + 8 * o + 4 * h;
  const bool col_ok = lcol < a.N;
  const int lcol_c = col_ok ? lcol : a.N - 4;
  const int n8 = a.N / 8;
  const int zword = lcol_c >> 3;
  const int zsh = FMT == kGptq ? 4 * (lcol_c & 7) : 8 * h;
  NibbleConsts nc;
  nc.m0 = __builtin_amdgcn_readfirstlane(0x000f000fu);
  nc.m1 = __builtin_amdgcn_readfirstlane(0x00f000f0u);
  nc.c0 = 0x64006400u + (uint32_t)(lane & 0);  // keep the magics in VGPRs
  nc.c1 = 0x54005400u + (uint32_t)(lane & 0);

  // loop-invariant 32-bit byte offsets of this lane; tiles: the word of
  // column lcol_c at stage 0, step 0 (column lcol_c + i is 16 bytes further,
  // step s of stage t (t * 1024 + s * 4) bytes)
  const bool tiles = FMT == kGptq && a.layout == kLayoutTiles;
  const uint32_t w_boff = tiles
                             ? (uint32_t)(((lcol_c >> 4) * w4_stages(a.K) * 64 + kb * 16 + (lcol_c & 15)) * 16)
                         : FMT == kGptq ? (uint32_t)(kb * a.N + lcol_c) * 4u
                                       : (uint32_t)(8 * kb * n8 + zword) * 4u;
  const uint32_t s_boff = (uint32_t)lcol_c * 2u;
  const uint32_t z_boff = (uint32_t)zword * 4u;
  uint32_t x_boff[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
    x_boff[t] = (uint32_t)(min(mbase + t * 16 + j, a.M - 1) * a.ldx + 8 * kb) * 2u;

  f32x4 acc[MT][4];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto step_group = [&](int st, int k) -> int {
    if constexpr (GM == kGStep) return __builtin_amdgcn_readfirstlane(group_of(a, st * 32));
    else return group_of(a, PRED ? min(k, a.K - 1) : k);
  };

  auto load_weights_step = [&](W4Batch<FMT, MT, U>& b, int u, int st) {
    const int k = st * 32 + 8 * kb;
    const bool ok = !PRED || (k < a.K && col_ok);
    if constexpr (FMT == kGptq) {
      if (tiles) {
        // the 4 columns' words of this step, 16 bytes apart
        const uint32_t* base = a.qw + (int64_t)(st >> 2) * 256 + (st & 3);
#pragma unroll
        for (int i = 0; i < 4; ++i) b.wq[u][i] = ok ? ldw<uint32_t, NT>(base, w_boff + 16u * i) : 0u;
      } else {
        // rows: word row st*4 + kb starts at (st*4)*N
        const uint32_t* base = a.qw + (int64_t)st * 4 * a.N;
        b.wq[u] = ok ? ldw<u32x4, NT>(base, w_boff) : u32x4{0u, 0u, 0u, 0u};
      }
    } else {
      const uint32_t* base = a.qw + (int64_t)st * 32 * n8;
#pragma unroll
      for (int t = 0; t < 8; ++t)
        b.wd[u][t] = (!PRED || (ok && k + t < a.K)) ? ldw<uint32_t, NT>(base, w_boff + (uint32_t)(t * n8 * 4)) : 0u;
    }
  };
  auto load_rest = [&](W4Batch<FMT, MT, U>& b, int u, int st) {
    const int k = st * 32 + 8 * kb;
    if constexpr (GM == kGLane) {
      const int g = step_group(st, k);
      b.sv[u] = ldb<u32x2>(a.sc + (int64_t)g * a.N, s_boff);
      b.zw[u] = ldb<uint32_t>(a.qz + (int64_t)g * n8, z_boff);
    } else if constexpr (GM == kGStep) {
      // derive() reads a step's scale/zero words only where the group changes:
      // at a batch's first step (the previous batch may have ended a group or
      // this is the wave's first step) and at a group's first step
      const int g = step_group(st, k);
      if (u == 0 || group_of(a, st * 32) != group_of(a, st * 32 - 32)) {
        b.sv[u] = ldb<u32x2>(a.sc + (int64_t)g * a.N, s_boff);
        b.zw[u] = ldb<uint32_t>(a.qz + (int64_t)g * n8, z_boff);
      }
    }
    const uint16_t* xb = a.x + (int64_t)st * 32;
#pragma unroll
    for (int t = 0; t < MT; ++t) {
      if constexpr (!PRED) {
        b.xv[u][t] = ldb<u32x4>(xb, x_boff[t]);
      } else {
        uint32_t hv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
          hv[e] = (k + e < a.K) ? (uint32_t)ldb<uint16_t>(xb, x_boff[t] + 2u * e) : 0u;
#pragma unroll
        for (int d = 0; d < 4; ++d) b.xv[u][t][d] = hv[2 * d] | (hv[2 * d + 1] << 16);
      }
    }
  };

  auto load_step = [&](W4Batch<FMT, MT, U>& b, int u, int st) {
    load_weights_step(b, u, st);
    load_rest(b, u, st);
  };

  // derived per-group operands: zero pairs for the two magics and the
  // broadcast scale pair of each of the lane's 4 columns (GPTQ), or the zero
  // / scale pairs of its 4 columns (AWQ)
  uint32_t zq[4][2], sq[4];
  int gcur = -1;
  auto derive = [&](const W4Batch<FMT, MT, U>& b, int u) {
    if constexpr (FMT == kGptq) {
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const uint32_t z = ((b.zw[u] >> (zsh + 4 * t)) & 0xfu) + a.zoff;
        zq[t][0] = nc.c0 + z * 0x00010001u;   // (1024 + z) pair
        zq[t][1] = nc.c1 + z * 0x00100010u;   // (64 + z) pair: z on the nibble's bit place
        const uint32_t s16 = (t & 1) ? (b.sv[u][t >> 1] >> 16) : (b.sv[u][t >> 1] & 0xffffu);
        sq[t] = s16 * 0x00010001u;
      }
    } else {
      const uint32_t x = b.zw[u] >> zsh;
      zq[0][0] = and_or(x, nc.m0, nc.c0);   // zero pair of columns 4h, 4h+1 as 1024+z
      zq[1][0] = and_or(x, nc.m1, nc.c1);   // columns 4h+2, 4h+3 as 64+z
      sq[0] = b.sv[u][0];
      sq[1] = b.sv[u][1];
    }
  };

  auto compute_step = [&](const W4Batch<FMT, MT, U>& b, int u, int st) {
    const int k = st * 32 + 8 * kb;
    u32x4 B[4];
    if constexpr (GM == kGStep) {
      const int g = __builtin_amdgcn_readfirstlane(group_of(a, st * 32));
      if (g != gcur) {
        derive(b, u);
        gcur = g;
      }
    } else if constexpr (GM == kGLane) {
      derive(b, u);
    }
    if constexpr (FMT == kGptq) {
      if constexpr (GM != kGElem) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const uint32_t w = b.wq[u][t], y = w >> 8;
          B[t] = u32x4{pk_sub_mul(and_or(w, nc.m0, nc.c0), zq[t][0], sq[t]),   // k+0, k+4
                       pk_sub_mul(and_or(w, nc.m1, nc.c1), zq[t][1], sq[t]),   // k+1, k+5
                       pk_sub_mul(and_or(y, nc.m0, nc.c0), zq[t][0], sq[t]),   // k+2, k+6
                       pk_sub_mul(and_or(y, nc.m1, nc.c1), zq[t][1], sq[t])};  // k+3, k+7
        }
      } else {
        // arbitrary g_idx: per-element group; natural -> [0,4,1,5,...] order
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          uint16_t hv[8];
          const uint32_t w = b.wq[u][t];
          const int col = lcol_c + t;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int g = a.gidx[min(k + e, a.K - 1)];
            const uint32_t z = ((a.qz[(int64_t)g * n8 + (col >> 3)] >> (4 * (col & 7))) & 0xfu) + a.zoff;
            hv[e] = dq1((w >> (4 * e)) & 0xfu, z, a.sc[(int64_t)g * a.N + col]);
          }
          B[t] = u32x4{(uint32_t)hv[0] | ((uint32_t)hv[4] << 16),
                       (uint32_t)hv[1] | ((uint32_t)hv[5] << 16),
                       (uint32_t)hv[2] | ((uint32_t)hv[6] << 16),
                       (uint32_t)hv[3] | ((uint32_t)hv[7] << 16)};
        }
      }
    } else {
      uint32_t wa[8], wb[8];
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        if constexpr (GM == kGElem) {
          // a group boundary inside the 8-row chunk: per-row parameters
          W4Batch<FMT, MT, U> tmp;
          const int g = group_of(a, min(k + t, a.K - 1));
          tmp.sv[0] = ldb<u32x2>(a.sc + (int64_t)g * a.N, s_boff);
          tmp.zw[0] = ldb<uint32_t>(a.qz + (int64_t)g * n8, z_boff);
          derive(tmp, 0);
        }
        const uint32_t x = b.wd[u][t] >> zsh;
        wa[t] = pk_sub_mul(and_or(x, nc.m0, nc.c0), zq[0][0], sq[0]);
        wb[t] = pk_sub_mul(and_or(x, nc.m1, nc.c1), zq[1][0], sq[1]);
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
      u32x4 xv = x_to_f16<XDT>(b.xv[u][t]);
      if constexpr (FMT == kGptq) xv = gptq_order(xv);
      const f16x8 A = as_f16x8(xv);
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[t][i] = mfma_f16(A, as_f16x8(B[i]), acc[t][i]);
    }
  };

  auto load = [&](W4Batch<FMT, MT, U>& b, int st0) {
#pragma unroll
    for (int u = 0; u < U; ++u) load_step(b, u, st0 + u);
  };
  // tiles, a stage-aligned batch of 4 steps: one 16-byte load per column
  // holds its words of all 4 steps
  auto load_batch = [&](W4Batch<FMT, MT, U>& b, int st0) {
    if constexpr (FMT == kGptq && U == 4 && !PRED) {
      if (tiles && (st0 & 3) == 0) {
        const uint32_t* base = a.qw + (int64_t)(st0 >> 2) * 256;
        u32x4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = ldw<u32x4, NT>(base, w_boff + 16u * i);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
#pragma unroll
          for (int i = 0; i < 4; ++i) b.wq[u][i] = v[i][u];
          load_rest(b, u, st0 + u);
        }
        return;
      }
    }
    load(b, st0);
  };
  auto compute = [&](const W4Batch<FMT, MT, U>& b, int st0) {
#pragma unroll
    for (int u = 0; u < U; ++u) compute_step(b, u, st0 + u);
  };

  // full batches: two register batches in flight (load b+1 while computing b)
  const int nfull = max(0, wend - wbeg) / U;
  W4Batch<FMT, MT, U> b0, b1;
  int st = wbeg;
  if (nfull > 0) load_batch(b0, st);
  int bi = 0;
  for (; bi + 2 <= nfull; bi += 2, st += 2 * U) {
    load_batch(b1, st + U);
    compute(b0, st);
    if (bi + 2 < nfull) load_batch(b0, st + 2 * U);
    compute(b1, st + U);
  }
  if (bi < nfull) {
    compute(b0, st);
    st += U;
  }
  // remaining single steps
  for (; st < wend; ++st) {
    load_step(b0, 0, st);
    gcur = -1;
    compute_step(b0, 0, st);
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

// ---------------------------------------------------------------------------
// Decode GEMV (M <= 16, K % 128 == 0 in windows of S steps x 32 with S in
// {2, 4, 8}, group_size a multiple of 32 whose boundaries fall at fixed steps
// of every wave's window).
//
// A 16-wave workgroup (one per CU) owns a balanced run of 16-column blocks
// and one K chunk of at most 16 windows (all of K up to 4096 at S = 8; longer
// K runs several chunks, grid y, whose fp32 partials a reduce pass adds in
// chunk order).  Wave w owns steps [c0 + w*S, c0 + w*S + S) of the chunk
// starting at step c0 (none when that lies past the chunk or past K: the
// wave then loads nothing and adds zeros): it loads those x chunks once as MFMA A
// operands and keeps them in registers while it streams the weights of every
// column block of the workgroup with D blocks in flight, so x is read once
// per wave rather than once per column block.  Lane (j = l%16, kb = l/16)
// dequantizes the packed word of column block*16 + j, packed row step*4 + kb:
// the B operand of one v_mfma_f32_16x16x32_f16 (k order [0,4,1,5,2,6,3,7],
// matched in A).  The 16 waves' partial sums meet in LDS and are added in
// wave order, so results do not depend on timing; they meet once per round of
// 2*D blocks (one round covers a workgroup's share for typical N), so the
// waves stream without barriers in between.  Weights, scales and zeros
// are read through buffer resources: every address is a scalar base and
// offset plus one fixed 32-bit lane offset; reads past a buffer return 0 and
// columns past N are computed but never stored.
//
// Weight layouts: LAYOUT_ROWS = qweight [K/8][N] (checkpoint GPTQ order);
// LAYOUT_TILES = the lane-major stage tiles (w4_stages): a lane's words of a
// stage are one 16-byte load.
constexpr int kGvWaves = 16;

struct GvPlan {
  int wgs, units;
  int splits, sps;  // K splits (grid y) and steps of 32 per split
};

template <int S, int SPG>
struct GvShape {
  static constexpr int kGroups = SPG >= S ? 1 : S / SPG;        // group slots per window
  // blocks in flight per wave.  S = 8 (K = 4096): 3, measured on C2
  // (N = 28672, M = 16): 13.8 us against 14.3 us with 4 and 13.9 with 2; more
  // requests in flight do not add bandwidth here, they delay the first block.
  static constexpr int kDepth = (S + 2 * kGroups) > 16 ? 2
                                : (S >= 8 || (S + 2 * kGroups) > 12) ? 3 : 4;
  static constexpr int kRound = kDepth;  // blocks per reduction round (several rounds)
  // a share of at most kShort blocks has all of them in flight at once
  static constexpr int kShort = kDepth + 1;
  // a workgroup's whole share in one round (at least 8 blocks: 7 on C2)
  static constexpr int kOneRound = 2 * kDepth < 8 ? 8 : 2 * kDepth;
};

template <int S, int SPG>
struct GvBlock {
  uint32_t w[S];
  uint32_t sv[GvShape<S, SPG>::kGroups];  // LAYOUT_ROWS: scale bits
  uint32_t zw[GvShape<S, SPG>::kGroups];  // LAYOUT_ROWS: zero word; tiles: table word
};

struct GvCtx {
  i32x4 rw, rs, rz;      // buffer resources: qweight (tiles: + table), scales, qzeros
  i32x4 rnull;           // zero-size resource (dead blocks)
  int32_t wlane;         // lane byte offset inside a step (layout dependent)
  int32_t slane, zlane;  // lane byte offsets of its scale / zero (tiles: table) word
  int32_t tbase;         // tiles: byte offset of the scale/zero table
  int pairs;             // tiles: group pairs per column tile
  int st0;               // first step of this wave
  int g0;                // group of the first step
  bool wlive;            // the wave's window lies inside K (else it loads nothing)
};

// Loads of one block in the order its compute consumes them (the group's
// scale and zero words, then the weight steps); the scheduling barrier keeps
// the compiler from regrouping loads across blocks, so waiting for a block
// never waits for a later block's loads (vector loads complete in order).
// A block that is not `live` (past the workgroup's share) reads through a
// zero-size resource instead: every lane is out of range, reads 0 and sends
// no memory request, and the code stays branch-free.
KQ_DEV i32x4 select_rsrc(bool live, const i32x4& r, const i32x4& dead) {
  i32x4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = __builtin_amdgcn_readfirstlane(live ? r[i] : dead[i]);
  return o;
}

template <int S, int SPG, int LAYOUT>
KQ_DEV void gv_load(const W4Args& a, const GvCtx& c, int unit, bool live, GvBlock<S, SPG>& b) {
  constexpr int NG = GvShape<S, SPG>::kGroups;
  live = live && c.wlive;
  const i32x4 rw = select_rsrc(live, c.rw, c.rnull);
  if constexpr (LAYOUT == kLayoutTilesZu) {
    // scales alone: one 2-byte scale (a single group) or 4 bytes per group pair
    const int32_t so = c.tbase + (unit * c.pairs + (c.g0 >> 1)) * 64;
    if constexpr (NG == 1) {
      b.zw[0] = (uint16_t)kq_rbl_i16(rw, c.zlane, so + (c.g0 & 1) * 2, 0);
    } else {
#pragma unroll
      for (int i = 0; i < NG / 2; ++i) b.zw[i] = (uint32_t)kq_rbl_i32(rw, c.zlane, so + i * 64, 0);
    }
  } else if constexpr (LAYOUT == kLayoutTiles) {
    // the window's scale/zero words from the table behind the tiles: one
    // word (a single group) or 8 bytes per group pair (g0 is then even)
    const int32_t so = c.tbase + (unit * c.pairs + (c.g0 >> 1)) * 128;
    if constexpr (NG == 1) {
      b.zw[0] = (uint32_t)kq_rbl_i32(rw, c.zlane, so + (c.g0 & 1) * 4, 0);
    } else {
#pragma unroll
      for (int i = 0; i < NG / 2; ++i) {
        const i32x2 v = kq_rbl_v2i32(rw, c.zlane, so + i * 128, 0);
        b.zw[2 * i] = (uint32_t)v[0];
        b.zw[2 * i + 1] = (uint32_t)v[1];
      }
    }
  } else {
    const i32x4 rs = select_rsrc(live, c.rs, c.rnull);
    const i32x4 rz = select_rsrc(live, c.rz, c.rnull);
#pragma unroll
    for (int i = 0; i < NG; ++i) {
      const int g = c.g0 + i;
      b.sv[i] = (uint16_t)kq_rbl_i16(rs, c.slane, (g * a.N + unit * 16) * 2, 0);
      b.zw[i] = (uint32_t)kq_rbl_i32(rz, c.zlane, (g * (a.N / 8) + unit * 2) * 4, 0);
    }
  }
  if constexpr (LAYOUT != kLayoutRows) {
    // a lane's steps of one stage are 16 contiguous bytes: one load per
    // stage (S = 2: the wave's half of a stage, 8 bytes)
    const int T = w4_stages(a.K);
    if constexpr (S >= 4) {
#pragma unroll
      for (int h = 0; h < S / 4; ++h) {
        const int32_t so = (unit * T + (c.st0 >> 2) + h) * 1024;
        const i32x4 v = kq_rbl_v4i32(rw, c.wlane, so, kAuxNT);
#pragma unroll
        for (int e = 0; e < 4; ++e) b.w[4 * h + e] = (uint32_t)v[e];
      }
    } else {
      const int32_t so = (unit * T + (c.st0 >> 2)) * 1024 + (c.st0 & 3) * 4;
      const i32x2 v = kq_rbl_v2i32(rw, c.wlane, so, kAuxNT);
      b.w[0] = (uint32_t)v[0];
      b.w[1] = (uint32_t)v[1];
    }
  } else {
#pragma unroll
    for (int s = 0; s < S; ++s) {
      const int32_t so = (c.st0 + s) * 16 * a.N + unit * 64;
      b.w[s] = (uint32_t)kq_rbl_i32(rw, c.wlane, so, kAuxNT);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
}

template <int S, int SPG, int LAYOUT>
KQ_DEV f32x4 gv_compute(const W4Args& a, const NibbleConsts& nc, uint32_t zsh,
                        const GvBlock<S, SPG>& b, const u32x4 (&A)[S]) {
  f32x4 acc{0.f, 0.f, 0.f, 0.f};
  uint32_t zq0 = 0, zq1 = 0, sq = 0;
#pragma unroll
  for (int s = 0; s < S; ++s) {
    if (SPG >= S ? s == 0 : (s % SPG) == 0) {
      const int i = SPG >= S ? 0 : s / SPG;
      uint32_t z;
      if constexpr (LAYOUT == kLayoutTilesZu) {
        z = a.zoff;                                          // the operand's one zero
        sq = GvShape<S, SPG>::kGroups == 1 ? b.zw[0] * 0x00010001u
                            : __builtin_amdgcn_perm(b.zw[i >> 1], b.zw[i >> 1],
                                                    (i & 1) ? 0x07060706u : 0x05040504u);
      } else if constexpr (LAYOUT == kLayoutTiles) {
        z = b.zw[i] >> 16;                                   // zero offset included
        sq = __builtin_amdgcn_perm(b.zw[i], b.zw[i], 0x05040504u);  // (scale, scale)
      } else {
        z = ((b.zw[i] >> zsh) & 0xfu) + a.zoff;
        sq = b.sv[i] * 0x00010001u;
      }
      zq0 = nc.c0 + z * 0x00010001u;   // (1024 + z) pair
      zq1 = nc.c1 + z * 0x00100010u;   // (64 + z) pair
    }
    const uint32_t w = b.w[s], y = w >> 8;
    const u32x4 B{pk_sub_mul(and_or(w, nc.m0, nc.c0), zq0, sq),   // k+0, k+4
                  pk_sub_mul(and_or(w, nc.m1, nc.c1), zq1, sq),   // k+1, k+5
                  pk_sub_mul(and_or(y, nc.m0, nc.c0), zq0, sq),   // k+2, k+6
                  pk_sub_mul(and_or(y, nc.m1, nc.c1), zq1, sq)};  // k+3, k+7
    acc = mfma_f16(as_f16x8(A[s]), as_f16x8(B), acc);
  }
  return acc;
}

// MODE kGvOne: the launch guarantees ncb <= kOneRound blocks per workgroup,
// so one round with the accumulators of all of them in registers (no outer
// loop).
// kGvShort: ncb <= kShort (one more than the streaming depth), one round with
// all of them in flight at once (Llama-3-8B gate, N = 14336, K = 4096: 9.0 ->
// 8.3 us at M = 1; down, K = 14336 in 4 chunks: 12.0 -> 11.0 us).  kGvSingle: every workgroup owns
// exactly one block (D = U = 1).  The modes keep the slots past a share few:
// their out-of-range loads move no data but still cost address-unit issue
// slots.  kGvRounds: several rounds of U blocks.
enum { kGvRounds = 0, kGvOne = 1, kGvSingle = 2, kGvShort = 3 };

// SWIGLU (one-round mode, tiled operand over gate/up columns interleaved by
// 16): workgroup shares are whole gate/up unit pairs and the epilogue writes
// silu(gate) * up into out [M][N/2].
template <int XDT, int S, int SPG, int LAYOUT, int MODE, bool SWIGLU = false>
__global__ void __launch_bounds__(64 * kGvWaves)
w4a16_gemv_kernel(W4Args a, GvPlan p) {
  constexpr bool ONE = MODE != kGvRounds;
  constexpr int D = MODE == kGvSingle ? 1 : MODE == kGvShort ? GvShape<S, SPG>::kShort : GvShape<S, SPG>::kDepth;
  constexpr int U = MODE == kGvSingle ? 1
                    : MODE == kGvShort ? D
                    : (MODE == kGvOne ? GvShape<S, SPG>::kOneRound : GvShape<S, SPG>::kRound);
  // LDS: per wave, first its x slice (16 rows x S*32 halves, rows padded by
  // 16 bytes), later its row of partial sums; the wave is done with x before
  // it writes partial sums, so the two share the wave's region.
  constexpr int kXRow = S * 64 + 16;                       // bytes per staged x row
  constexpr int kWaveLds = (16 * kXRow > U * 4 * 64 * 4) ? 16 * kXRow : U * 4 * 64 * 4;
  __shared__ __attribute__((aligned(16))) char lds[kGvWaves * kWaveLds];
  static_assert(kGvWaves * kWaveLds <= 160 * 1024, "LDS");
  auto red = [&](int w, int i) -> float* { return (float*)(lds + w * kWaveLds) + i * 64; };
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int j = lane & 15, kb = lane >> 4;
  // balanced unit range of this workgroup (SWIGLU: balanced in unit pairs)
  constexpr int kUnitsPer = SWIGLU ? 2 : 1;
  const int items = p.units / kUnitsPer;
  const int base = items / p.wgs, rem = items % p.wgs;
  const int bid = blockIdx.x;
  const int u0 = (bid * base + min(bid, rem)) * kUnitsPer;
  const int ncb = (base + (bid < rem ? 1 : 0)) * kUnitsPer;
  static_assert(!SWIGLU || (MODE == kGvOne && U % 2 == 0), "SwiGLU GEMV runs one round of unit pairs");

  NibbleConsts nc;
  nc.m0 = __builtin_amdgcn_readfirstlane(0x000f000fu);
  nc.m1 = __builtin_amdgcn_readfirstlane(0x00f000f0u);
  nc.c0 = 0x64006400u + (uint32_t)(lane & 0);
  nc.c1 = 0x54005400u + (uint32_t)(lane & 0);

  GvCtx c;
  const int ngroups = (a.K + a.G - 1) / a.G;
  c.rw = make_rsrc(a.qw, LAYOUT != kLayoutRows
                            ? (uint32_t)(w4_tiled_words(a.N, a.K, a.G, LAYOUT == kLayoutTilesZu) * 4)
                            : (uint32_t)((a.K / 8) * a.N * 4));
  c.rs = make_rsrc(a.sc, (uint32_t)(ngroups * a.N * 2));
  c.rz = make_rsrc(a.qz, (uint32_t)(ngroups * (a.N / 8) * 4));
  c.rnull = make_rsrc(a.qw, 0u);
  c.wlane = LAYOUT != kLayoutRows ? lane * 16 : (kb * a.N + j) * 4;
  c.slane = j * 2;
  c.zlane = LAYOUT == kLayoutTilesZu ? j * 4 : LAYOUT == kLayoutTiles ? j * 8 : (j >> 3) * 4;
  c.tbase = (int32_t)(w4_tile_words(a.N, a.K) * 4);
  c.pairs = w4_group_pairs(a.K, a.G);
  // K split blockIdx.y covers steps [cs0, cs1) (one split: all of K); its
  // windows start at multiples of S, and windows past cs1 belong to inactive
  // waves, whose loads go through the zero-size resource and whose x is
  // zeroed (gv_plan: K % (32 * S) == 0, steps per split a multiple of S)
  const int split = blockIdx.y;
  const int cs0 = split * a.steps_per_split;
  const int cs1 = min(cs0 + a.steps_per_split, a.K / 32);
  c.st0 = cs0 + wave * S;
  c.wlive = c.st0 < cs1;
  const int xst0 = c.wlive ? c.st0 : 0;
  c.g0 = __builtin_amdgcn_readfirstlane(group_of(a, xst0 * 32));
  const uint32_t zsh = 4u * (uint32_t)(j & 7);

  // x chunks of this wave's steps, loaded once and kept for every block.
  // They are requested before the weights: loads complete in issue order, so
  // the first block's compute then waits for x and that block only, not for
  // every block in flight (which would leave HBM idle between the first
  // window and the loads the compute issues).  The loads read whole 128-byte
  // lines (8 lanes per row, 8 rows per instruction: half the line requests
  // of the MFMA lane order, which reads 64 bytes of 16 rows); the wave then
  // moves them into the MFMA lane order through its own LDS region (no
  // barrier: only this wave reads it).  Measured: C1 (N = K = 4096, M = 16,
  // one column block per workgroup, x 80% of a workgroup's bytes) 6.47 ->
  // 5.30 us; C2 M = 16 13.85 -> 13.50 us.
  u32x4 X[S];
  {
    const int rsub = lane >> 3, csub = lane & 7;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int q = i * 8 + rsub;                 // row chunk: row q % 16, 128 B chunk q / 16
      const int row = q & 15, cc = q >> 4;
      X[i] = *(const u32x4*)(a.x + (int64_t)min(row, a.M - 1) * a.ldx + xst0 * 32 + cc * 64 + csub * 8);
    }
  }

  // rolling window: block q's weights were requested D blocks earlier.  No
  // load sits under a branch (blocks past the share read through the
  // zero-size resource), so the code stays straight-line and the compiler
  // waits for exactly the block about to be computed.  (Under a branch the
  // wait count is merged at the join, and each compute then waits for every
  // load in flight.)
  GvBlock<S, SPG> buf[D];
#pragma unroll
  for (int d = 0; d < D; ++d) gv_load<S, SPG, LAYOUT>(a, c, u0 + d, d < ncb, buf[d]);

  // x in the MFMA lane order (the weight loads above stay in flight)
  {
    const int rsub = lane >> 3, csub = lane & 7;
    char* mine = lds + wave * kWaveLds;
#pragma unroll
    for (int i = 0; i < S; ++i) {
      const int q = i * 8 + rsub;
      *(u32x4*)(mine + (q & 15) * kXRow + (q >> 4) * 128 + csub * 16) = X[i];
    }
#pragma unroll
    for (int s = 0; s < S; ++s) X[s] = *(const u32x4*)(mine + j * kXRow + s * 64 + kb * 16);
  }

  u32x4 A[S];
#pragma unroll
  for (int s = 0; s < S; ++s) {
    A[s] = gptq_order(x_to_f16<XDT>(X[s]));
    if (!c.wlive) A[s] = u32x4{0u, 0u, 0u, 0u};  // (a non-finite x would turn 0 * x into NaN)
  }

  for (int q0 = 0; q0 < (ONE ? 1 : ncb); q0 += U) {
    // U blocks per round (U a multiple of D, so block q0+q sits in buf[q % D])
    f32x4 acc[U];
#pragma unroll
    for (int q = 0; q < U; ++q) {
      acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
      // Issue priority falls as the wave completes blocks: the SIMD otherwise
      // favours its oldest ready wave, which then runs ahead, and the last
      // waves of the workgroup finish alone with few loads in flight.
      // Measured on C2 (N = 28672, K = 4096): 13.31 -> 13.04 us at M = 16,
      // 12.69 -> 12.47 us at M = 1; raising it around the load issue too
      // changed nothing.
      if (q < 2) __builtin_amdgcn_s_setprio(3);
      else if (q < 4) __builtin_amdgcn_s_setprio(2);
      else if (q < 6) __builtin_amdgcn_s_setprio(1);
      else __builtin_amdgcn_s_setprio(0);
      if (q0 + q < ncb) acc[q] = gv_compute<S, SPG, LAYOUT>(a, nc, zsh, buf[q % D], A);
      // (ONE: the share has at most U blocks, so slots past U are never loaded)
      if (!ONE || q + D < U) gv_load<S, SPG, LAYOUT>(a, c, u0 + q0 + q + D, q0 + q + D < ncb, buf[q % D]);
    }
    // fixed-order reduction of the 16 waves' partial sums (the next round's
    // loads stay in flight across the barriers)
#pragma unroll
    for (int q = 0; q < U; ++q)
#pragma unroll
      for (int r = 0; r < 4; ++r) red(wave, q * 4 + r)[lane] = acc[q][r];
    __syncthreads();
    if constexpr (SWIGLU) {
      // one gate/up pair per thread: unit 2pp holds gate columns, 2pp + 1 up
      const int width = a.N / 2;
      for (int i = wave; i < (U / 2) * 4; i += kGvWaves) {
        const int pp = i >> 2, r = i & 3, qg = 2 * pp, qu = qg + 1;
        if (qu >= ncb) continue;
        float g = red(0, qg * 4 + r)[lane], u = red(0, qu * 4 + r)[lane];
#pragma unroll
        for (int w = 1; w < kGvWaves; ++w) {
          g = __fadd_rn(g, red(w, qg * 4 + r)[lane]);
          u = __fadd_rn(u, red(w, qu * 4 + r)[lane]);
        }
        const int m = 4 * kb + r;
        const int col = (u0 + qg) * 16 + j;  // gate column of the interleaved operand
        if (m < a.M) {
          if (a.bias_dtype != KQ_DTYPE_NONE) {
            g = __fadd_rn(g, load_as_f32(a.bias, a.bias_dtype, col));
            u = __fadd_rn(u, load_as_f32(a.bias, a.bias_dtype, col + 16));
          }
          a.out[(int64_t)m * width + ((u0 + qg) >> 1) * 16 + j] = swiglu_bits(g, u, a.out_dtype);
        }
      }
      return;
    }
    for (int i = wave; i < U * 4; i += kGvWaves) {   // one output per thread
      const int q = i >> 2, r = i & 3;
      if (q0 + q >= ncb) continue;
      float v = red(0, i)[lane];
#pragma unroll
      for (int w = 1; w < kGvWaves; ++w) v = __fadd_rn(v, red(w, i)[lane]);
      const int m = 4 * kb + r;
      const int n = (u0 + q0 + q) * 16 + j;
      if (m < a.M && n < a.N) {
        if (a.splits > 1) {
          // this split's fp32 partial; the reduce pass adds the splits in
          // order and applies bias and the cast
          a.partials[((int64_t)split * a.M + m) * a.N + n] = v;
        } else {
          if (a.bias_dtype != KQ_DTYPE_NONE) v = __fadd_rn(v, load_as_f32(a.bias, a.bias_dtype, n));
          a.out[(int64_t)m * a.N + n] = f32_to_out(v, a.out_dtype);
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Prefill GEMM (M > 16, load-time tiled weights, K % 128 == 0, group_size a
// multiple of 128).  Output tile BM = 16*TM*WM activation rows x BN =
// 16*TN*(8/WM) columns, 8 waves as WM x (8/WM); wave (wm, wn) owns TM row
// blocks x TN column tiles of 16.  Measured floor (C2 M = 512): without the
// dequant and the MFMAs the kernel still takes 80% of its time, i.e. the
// LDS fragment reads, the copies and the per-stage barrier bound it.  K advances 128 per stage; a stage holds
//   x16  BM rows x 256 bytes (fp16, k in MFMA order, 16-byte chunk c of row r
//        at c ^ (r & 15): the 16 lanes of one k-group read 16 banks),
//   W    BN/16 column tiles x 1 KB (their tiled words of the stage's 4 steps),
//   the stage's group scales (BN fp16) and zero words (BN/8),
// all copied global -> LDS with buffer_load ... lds through an NS-stage ring:
// stages k+1 .. k+NS-1 are in flight while k computes (one barrier per stage).  The
// dequantized weights are the MFMA A operand (v_mfma_f32_16x16x32_f16), x the
// B operand, so a lane's four results are four consecutive columns of one row.
// Dequantization is the GEMV's (exact fp16((q-z)*s)).  x16 is written by
// w4a16_prep_x_mma_kernel: fp16, act-order gathered, and each 8-k chunk in
// the [0,4,1,5,2,6,3,7] order of the weight nibble pairs.
// vmcnt(N) (expcnt and lgkmcnt 0): the gfx9 immediate splits vmcnt in bits
// 0-3 and 14-15
template <int N>
KQ_DEV void w4p_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14));
}
// wait until at most `after` stages of OPS copies each remain in flight
template <int OPS, int C>
KQ_DEV void w4p_wait_stages(int after) {
  if constexpr (C > 0) {
    if (after >= C) {
      w4p_wait<C * OPS>();
      return;
    }
    w4p_wait_stages<OPS, C - 1>(after);
  } else {
    w4p_wait<0>();
  }
}

template <int TM, int TN, int WM>
struct W4pShape {
  static constexpr int WN = 8 / WM;
  static constexpr int BM = 16 * TM * WM;
  static constexpr int BN = 16 * TN * WN;
  static constexpr int XBytes = BM * 256;
  static constexpr int WBytes = BN * 64;           // BN/16 tiles x 1 KB
  static constexpr int SBytes = BN * 2;            // scales
  static constexpr int ZBytes = BN / 2;            // zero words (BN/8 x 4)
  static constexpr int Stage = XBytes + WBytes + SBytes + 256;  // zeros padded to one DMA4
  static constexpr int XOps = BM / 4 / 8;          // 1 KB DMA16 per wave per stage
  static constexpr int WOps = BN / 16 / 8;
  static constexpr int SOps = SBytes / 256;        // DMA4 (256 bytes) instructions
  static constexpr int Ops = XOps + WOps + 1;      // + one DMA4 per wave (scales, zeros or spare)
  static_assert(XOps >= 1 && WOps >= 1 && SOps + 1 <= 8, "tile shape");
};

// SWIGLU: the operand interleaves gate and up 16-column tiles (2p gate, 2p + 1
// up), so each pair of a wave's column tiles (TN = 2 or 4) holds both halves
// of 16 output columns and the epilogue writes silu(gate) * up into
// out [M][N/2].
template <int TM, int TN, int WM, int NS, bool SWIGLU = false>
__global__ void __launch_bounds__(512)
w4a16_prefill_kernel(W4Args a, int mblocks, int tiles, int ksplit) {
  using S = W4pShape<TM, TN, WM>;
  static_assert(!SWIGLU || TN % 2 == 0, "the SwiGLU epilogue pairs a wave's column tiles");
  __shared__ __attribute__((aligned(16))) uint8_t smem[NS * S::Stage + 8 * 256];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int wm = wave / S::WN, wn = wave % S::WN;
  const int c = lane & 15, g = lane >> 4;
  // XCD-contiguous unit ranges (row block fastest: an XCD's consecutive tiles
  // share weight tiles in its L2; the K splits of a tile are consecutive units)
  const int total = tiles * ksplit;
  const int per = (total + 7) / 8;
  const int u = (blockIdx.x & 7) * per + (blockIdx.x >> 3);
  if (u >= total) return;
  const int t = u / ksplit, split = u - t * ksplit;
  const int mb = t % mblocks, nb = t / mblocks;
  const int m0 = mb * S::BM, n0 = nb * S::BN;
  const int K = a.K, nst = K / 128;
  // this unit's stages [kb0, kb1) (ksplit <= nst / 2: at least two)
  const int kb0 = (int)((int64_t)nst * split / ksplit), kb1 = (int)((int64_t)nst * (split + 1) / ksplit);
  const int ngroups = K / a.G;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;

  // buffer resources: reads past them return zeros
  const i32x4 rx = make_rsrc(a.x, (uint32_t)((uint64_t)a.M * K * 2));
  const i32x4 rw = make_rsrc(a.qw, (uint32_t)(w4_tile_words(a.N, K) * 4));
  const i32x4 rs = make_rsrc(a.sc, (uint32_t)((uint64_t)ngroups * a.N * 2));
  const i32x4 rz = make_rsrc(a.qz, (uint32_t)((uint64_t)ngroups * (a.N / 8) * 4));

  // per-lane DMA offsets (stage-independent parts)
  int32_t xoff[S::XOps];
#pragma unroll
  for (int i = 0; i < S::XOps; ++i) {
    const int blk = wave * S::XOps + i;           // 1 KB = 4 rows x 256 bytes
    const int r = blk * 4 + (lane >> 4), pc = lane & 15;
    const int lc = pc ^ (r & 15);                 // logical 16-byte chunk (8 k)
    xoff[i] = m0 + r < a.M ? ((m0 + r) * K + lc * 8) * 2 : kTgOob;
  }
  int32_t woff[S::WOps];
#pragma unroll
  for (int i = 0; i < S::WOps; ++i) {
    const int u = n0 / 16 + wave * S::WOps + i;   // column tile
    woff[i] = u * 16 < a.N ? u * (K * 8) + lane * 16 : kTgOob;
  }
  // one DMA4 per wave: waves < SOps copy 256 bytes of scales, wave SOps the
  // zero words, the rest a spare (out of range -> zeros) so that every wave
  // issues S::Ops instructions per stage
  int32_t aoff;
  i32x4 ra;
  uint32_t alds;
  if (wave < S::SOps) {
    ra = rs;
    aoff = n0 + wave * 128 + 2 * lane < a.N ? (n0 + wave * 128 + 2 * lane) * 2 : kTgOob;
    alds = S::XBytes + S::WBytes + wave * 256;
  } else {
    ra = rz;
    aoff = (wave == S::SOps && lane < S::BN / 8 && n0 + lane * 8 < a.N) ? (n0 / 8 + lane) * 4 : kTgOob;
    alds = wave == S::SOps ? S::XBytes + S::WBytes + S::SBytes : NS * S::Stage + wave * 256;
  }
  auto issue = [&](int kb, int slot) {
    const uint32_t b = lds0 + slot * S::Stage;
#pragma unroll
    for (int i = 0; i < S::XOps; ++i) tg_dma16(rx, b + (wave * S::XOps + i) * 1024, xoff[i], kb * 256);
#pragma unroll
    for (int i = 0; i < S::WOps; ++i) tg_dma16(rw, b + S::XBytes + (wave * S::WOps + i) * 1024, woff[i], kb * 1024);
    const int grp = (kb * 128) / a.G;
    const int32_t so = wave < S::SOps ? grp * a.N * 2 : grp * (a.N / 8) * 4;
    const uint32_t dst = wave <= S::SOps ? b + alds : lds0 + alds;
    tg_dma4(ra, dst, aoff, so);
  };

  NibbleConsts nc;
  nc.m0 = __builtin_amdgcn_readfirstlane(0x000f000fu);
  nc.m1 = __builtin_amdgcn_readfirstlane(0x00f000f0u);
  nc.c0 = 0x64006400u + (uint32_t)(lane & 0);
  nc.c1 = 0x54005400u + (uint32_t)(lane & 0);
  const uint32_t zsh = 4u * (uint32_t)(c & 7);

  f32x4 acc[TN][TM];
#pragma unroll
  for (int tn = 0; tn < TN; ++tn)
#pragma unroll
    for (int i = 0; i < TM; ++i) acc[tn][i] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int i = 0; i < NS - 1; ++i)
    if (kb0 + i < kb1) issue(kb0 + i, (kb0 + i) % NS);
  w4p_wait_stages<S::Ops, NS - 2>(min(NS - 2, kb1 - kb0 - 1));
  __syncthreads();

  for (int kb = kb0; kb < kb1; ++kb) {
    const int slot = kb % NS;
    if (kb + NS - 1 < kb1) issue(kb + NS - 1, (kb + NS - 1) % NS);
    const uint8_t* st = smem + slot * S::Stage;
    // this stage's scales and zeros of the wave's column tiles (one group)
    uint32_t zq0[TN], zq1[TN], sq[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int col = (wn * TN + tn) * 16 + c;
      const uint32_t sv = *(const uint16_t*)(st + S::XBytes + S::WBytes + col * 2);
      const uint32_t zw = *(const uint32_t*)(st + S::XBytes + S::WBytes + S::SBytes + (col >> 3) * 4);
      const uint32_t z = ((zw >> zsh) & 0xfu) + a.zoff;
      zq0[tn] = nc.c0 + z * 0x00010001u;
      zq1[tn] = nc.c1 + z * 0x00100010u;
      sq[tn] = sv * 0x00010001u;
    }
    // the stage's four weight words of each column tile (one 16-byte read)
    u32x4 W[TN];
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) W[tn] = *(const u32x4*)(st + S::XBytes + (wn * TN + tn) * 1024 + lane * 16);
#pragma unroll
    for (int s4 = 0; s4 < 4; ++s4) {
      // The step's activation fragments are read first and land while its
      // weights dequantize; the fences keep that order (left alone, the
      // scheduler keeps two fragments in flight and each pair's LDS latency
      // stalls the MFMAs).  C2 (N = 28672, K = 4096): M = 128 67.7 -> 61.1 us,
      // M = 512 116 -> 113 us, M = 64 33.0 -> 31.2 us.
      u32x4 B[TM];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = (wm * TM + i) * 16 + c;
        B[i] = *(const u32x4*)(st + r * 256 + (((s4 * 4 + g) ^ c) << 4));
      }
      __builtin_amdgcn_sched_barrier(0);
      u32x4 A[TN];
#pragma unroll
      for (int tn = 0; tn < TN; ++tn) {
        const uint32_t w = W[tn][s4];
        const uint32_t y = w >> 8;
        A[tn] = u32x4{pk_sub_mul(and_or(w, nc.m0, nc.c0), zq0[tn], sq[tn]),
                      pk_sub_mul(and_or(w, nc.m1, nc.c1), zq1[tn], sq[tn]),
                      pk_sub_mul(and_or(y, nc.m0, nc.c0), zq0[tn], sq[tn]),
                      pk_sub_mul(and_or(y, nc.m1, nc.c1), zq1[tn], sq[tn])};
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int tn = 0; tn < TN; ++tn) acc[tn][i] = mfma_f16(as_f16x8(A[tn]), as_f16x8(B[i]), acc[tn][i]);
      __builtin_amdgcn_sched_barrier(0);
    }
    // stage kb+1 landed (the stages issued after it may stay in flight), and
    // every wave is done with stage kb before it is refilled
    w4p_wait_stages<S::Ops, NS - 2>(min(NS - 2, kb1 - 2 - kb));
    __syncthreads();
  }

  // epilogue: lane (c, g) of block (tn, i) holds rows m = .. + c, columns
  // n = .. + 4g .. 4g+3
  if constexpr (SWIGLU) {
    const int width = a.N / 2;
#pragma unroll
    for (int pp = 0; pp < TN / 2; ++pp) {
      // pair pp: gate column tile wn * TN + 2 pp of the interleaved operand,
      // its up tile the next one; output columns 16 of them
      const int ng = n0 + (wn * TN + 2 * pp) * 16 + 4 * g;
      const int oc = n0 / 2 + (wn * TN / 2 + pp) * 16 + 4 * g;
      float bg[4] = {0.f, 0.f, 0.f, 0.f}, bu[4] = {0.f, 0.f, 0.f, 0.f};
      if (a.bias_dtype != KQ_DTYPE_NONE)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          bg[q] = ng + q < a.N ? load_as_f32(a.bias, a.bias_dtype, ng + q) : 0.f;
          bu[q] = ng + 16 + q < a.N ? load_as_f32(a.bias, a.bias_dtype, ng + 16 + q) : 0.f;
        }
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = m0 + (wm * TM + i) * 16 + c;
        if (m >= a.M) continue;
        uint16_t o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          float gv = acc[2 * pp][i][q], uv = acc[2 * pp + 1][i][q];
          if (a.bias_dtype != KQ_DTYPE_NONE) {
            gv = __fadd_rn(gv, bg[q]);
            uv = __fadd_rn(uv, bu[q]);
          }
          o[q] = swiglu_bits(gv, uv, a.out_dtype);
        }
        uint16_t* dst = a.out + (int64_t)m * width + oc;
        if (oc + 3 < width) {
          *(u32x2*)dst = u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (oc + q < width) dst[q] = o[q];
        }
      }
    }
    return;
  }
  if (ksplit > 1) {
    // this split's fp32 partial sums; the W4 split-K reduce adds the splits in
    // order and applies bias and the cast
#pragma unroll
    for (int tn = 0; tn < TN; ++tn) {
      const int n = n0 + (wn * TN + tn) * 16 + 4 * g;
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int m = m0 + (wm * TM + i) * 16 + c;
        if (m >= a.M || n >= a.N) continue;
        float* dst = a.partials + ((int64_t)split * a.M + m) * a.N + n;
        if (n + 3 < a.N) {
          *(f32x4*)dst = acc[tn][i];
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (n + q < a.N) dst[q] = acc[tn][i][q];
        }
      }
    }
    return;
  }
#pragma unroll
  for (int tn = 0; tn < TN; ++tn) {
    const int n = n0 + (wn * TN + tn) * 16 + 4 * g;
    float bv[4] = {0.f, 0.f, 0.f, 0.f};
    if (a.bias_dtype != KQ_DTYPE_NONE)
#pragma unroll
      for (int q = 0; q < 4; ++q) bv[q] = n + q < a.N ? load_as_f32(a.bias, a.bias_dtype, n + q) : 0.f;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int m = m0 + (wm * TM + i) * 16 + c;
      if (m >= a.M) continue;
      uint16_t o[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v = acc[tn][i][q];
        if (a.bias_dtype != KQ_DTYPE_NONE) v = __fadd_rn(v, bv[q]);
        o[q] = f32_to_out(v, a.out_dtype);
      }
      uint16_t* dst = a.out + (int64_t)m * a.N + n;
      if (n + 3 < a.N) {
        *(u32x2*)dst = u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
      } else {
#pragma unroll
        for (int q = 0; q < 4; ++q)
          if (n + q < a.N) dst[q] = o[q];
      }
    }
  }
}

// x16[m][8j + e] = fp16(x[m][perm(8j + o[e])]) with o = [0,4,1,5,2,6,3,7]
// (perm = identity when null): the prefill kernel's activation operand.
__global__ void __launch_bounds__(256)
w4a16_prep_x_mma_kernel(const uint16_t* __restrict__ x, int dtype, int ldx,
                        const int32_t* __restrict__ perm, int M, int K, uint16_t* __restrict__ x16) {
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (idx >= (int64_t)M * K) return;
  const int m = (int)(idx / K), k0 = (int)(idx % K);
  const uint16_t* row = x + (int64_t)m * ldx;
  uint16_t h[8];
  if (perm) {
    const i32x4 p0 = *(const i32x4*)(perm + k0);
    const i32x4 p1 = *(const i32x4*)(perm + k0 + 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[e] = act_bits(row[p0[e]], dtype);
      h[e + 4] = act_bits(row[p1[e]], dtype);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) h[e] = act_bits(row[k0 + e], dtype);
  }
  const u32x4 v{(uint32_t)h[0] | ((uint32_t)h[4] << 16), (uint32_t)h[1] | ((uint32_t)h[5] << 16),
                (uint32_t)h[2] | ((uint32_t)h[6] << 16), (uint32_t)h[3] | ((uint32_t)h[7] << 16)};
  *(u32x4*)(x16 + idx) = v;
}

// x16[m][j] = fp16(x[m][perm[j]]) (act-order gather + W4A16 activation
// conversion); each thread writes 8 consecutive outputs with one 16-byte store.
__global__ void __launch_bounds__(64)
w4a16_prep_x_kernel(const uint16_t* __restrict__ x, int dtype, int ldx,
                    const int32_t* __restrict__ perm, int M, int K, uint16_t* __restrict__ x16) {
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (idx >= (int64_t)M * K) return;
  const int m = (int)(idx / K), k0 = (int)(idx % K);
  const uint16_t* row = x + (int64_t)m * ldx;
  if (k0 + 8 <= K && (K % 8) == 0) {
    const i32x4 p0 = *(const i32x4*)(perm + k0);
    const i32x4 p1 = *(const i32x4*)(perm + k0 + 4);
    uint16_t h[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      h[e] = act_bits(row[p0[e]], dtype);
      h[e + 4] = act_bits(row[p1[e]], dtype);
    }
    u32x4 v;
#pragma unroll
    for (int d = 0; d < 4; ++d) v[d] = (uint32_t)h[2 * d] | ((uint32_t)h[2 * d + 1] << 16);
    *(u32x4*)(x16 + (int64_t)m * K + k0) = v;
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int k = k0 + e;
    if (k < K) x16[(int64_t)m * K + k] = act_bits(row[perm[k]], dtype);
  }
}

// The act-order gather of the decode GEMV (M <= 16, K % 8 == 0, 16-byte
// aligned x rows): workgroup (c, m) stages row m of x in LDS while the perm
// slice it gathers is in flight (one memory round trip, where reading perm
// and then x through it takes two), then gathers 1024 outputs from LDS, 8
// consecutive ones per thread with one 16-byte store.
__global__ void __launch_bounds__(128)
w4a16_prep_x_row_kernel(const uint16_t* __restrict__ x, int dtype, int ldx,
                        const int32_t* __restrict__ perm, int K, uint16_t* __restrict__ x16) {
  extern __shared__ __attribute__((aligned(16))) uint16_t srow[];  // K halves
  const int m = blockIdx.y;
  const int j0 = blockIdx.x * 1024 + (int)threadIdx.x * 8;
  const bool mine = j0 < K;
  i32x4 p0{0, 0, 0, 0}, p1{0, 0, 0, 0};
  if (mine) {
    p0 = *(const i32x4*)(perm + j0);
    p1 = *(const i32x4*)(perm + j0 + 4);
  }
  const uint16_t* row = x + (int64_t)m * ldx;
#pragma unroll 4
  for (int c = threadIdx.x; c < K / 8; c += 128) *(u32x4*)(srow + 8 * c) = *(const u32x4*)(row + 8 * c);
  __syncthreads();
  if (!mine) return;
  uint16_t h[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    h[e] = act_bits(srow[p0[e]], dtype);
    h[e + 4] = act_bits(srow[p1[e]], dtype);
  }
  u32x4 v;
#pragma unroll
  for (int d = 0; d < 4; ++d) v[d] = (uint32_t)h[2 * d] | ((uint32_t)h[2 * d + 1] << 16);
  *(u32x4*)(x16 + (int64_t)m * K + j0) = v;
}

// out[m][n] = silu(gate) * up (swiglu_bits) from a [M][2I] gate/up output:
// gate column n and up column I + n, or (interleaved) the 16-column blocks of
// gate and up alternating.  Two outputs per thread.
__global__ void __launch_bounds__(256)
swiglu_kernel(const uint16_t* __restrict__ src, int64_t ld_src, int interleaved, int dtype,
              uint16_t* __restrict__ dst, int64_t M, int64_t I) {
  const int64_t idx = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 2;
  if (idx >= M * I) return;
  const int64_t m = idx / I, n = idx % I;  // I even: both outputs in row m
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const int64_t c = n + e;
    const int64_t gc = interleaved ? (c >> 4) * 32 + (c & 15) : c;
    const int64_t uc = interleaved ? gc + 16 : I + c;
    const float g = load_as_f32(src + m * ld_src, dtype, gc);
    const float u = load_as_f32(src + m * ld_src, dtype, uc);
    dst[m * I + c] = swiglu_bits(g, u, dtype);
  }
}

// AWQ word (k, c) holds column 8c + [0,2,4,6,1,3,5,7][i] in nibble i, so
// column offset o sits at nibble (o % 2) * 4 + o / 2 (kairyu/quant/awq.py:14-36).
KQ_DEV uint32_t awq_shift(int o) { return 4u * (uint32_t)((o & 1) * 4 + (o >> 1)); }

// Load-time tiling into the lane-major stage layout (see w4_stages): the
// word of packed row r, column n holds q[row(8r + e)][n] in nibble e, with
// row(k) = perm[k] (act-order) or k; rows past K/8 and columns past N are 0.
// Source: GPTQ qweight [K/8][N] (LSB-first along k) or AWQ qweight [K][N/8].
__global__ void w4_tile_kernel(const uint32_t* __restrict__ src, int awq, const int32_t* __restrict__ perm,
                               uint32_t* __restrict__ out, int N, int K) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int T = w4_stages(K);
  if (idx >= w4_tile_words(N, K)) return;
  const int s4 = (int)(idx & 3);
  const int lane = (int)((idx >> 2) & 63);
  const int c = lane & 15, kb = lane >> 4;
  const int t = (int)((idx >> 8) % T);
  const int u = (int)((idx >> 8) / T);
  const int r = t * 16 + s4 * 4 + kb;   // packed row: k = 8r .. 8r + 7
  const int n = u * 16 + c;
  uint32_t word = 0;
  if (n < N && r < K / 8) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int k = perm ? perm[8 * r + e] : 8 * r + e;
      const uint32_t q = awq ? (src[(int64_t)k * (N / 8) + (n >> 3)] >> awq_shift(n & 7)) & 0xfu
                             : (src[(int64_t)(k >> 3) * N + n] >> (4 * (k & 7))) & 0xfu;
      word |= q << (4 * e);
    }
  }
  out[idx] = word;
}

// The scale/zero table behind the tiles (see w4_tiled_words), from natural
// nibble order zeros [groups][N/8] (null: one zero, zoff) and fp16 scales
// [groups][N]; with one zero the scale-only table and the zero-word area.
__global__ void w4_scale_zero_kernel(const uint32_t* __restrict__ qz, uint32_t zoff,
                                     const uint16_t* __restrict__ sc, uint32_t* __restrict__ out,
                                     int N, int K, int G) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const bool zu = qz == nullptr;
  const int P = w4_group_pairs(K, G), groups = (K + G - 1) / G;
  const int64_t table = w4_table_words(N, K, G, zu);
  if (idx >= table) {
    if (idx < table + w4_zero_area_words(N, K, G, zu)) out[idx] = 0u;  // zero nibbles
    return;
  }
  auto scale = [&](int g, int n) -> uint32_t {
    return g < groups && n < N ? (uint32_t)sc[(int64_t)g * N + n] : 0u;
  };
  if (zu) {
    const int c = (int)(idx & 15), p = (int)((idx >> 4) % P), u = (int)((idx >> 4) / P);
    const int n = 16 * u + c;
    out[idx] = scale(2 * p, n) | (scale(2 * p + 1, n) << 16);
    return;
  }
  const int h = (int)(idx & 1), c = (int)((idx >> 1) & 15);
  const int p = (int)((idx >> 5) % P), u = (int)((idx >> 5) / P);
  const int g = 2 * p + h, n = 16 * u + c;
  uint32_t v = 0;
  if (g < groups && n < N) {
    const uint32_t z = ((qz[(int64_t)g * (N / 8) + (n >> 3)] >> (4 * (n & 7))) & 0xfu) + zoff;
    v = scale(g, n) | (z << 16);
  }
  out[idx] = v;
}

// AWQ zeros -> natural nibble order (column 8c + i in nibble i), values kept.
__global__ void awq_natural_zeros_kernel(const uint32_t* __restrict__ qz, uint32_t* __restrict__ out,
                                         int64_t words) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= words) return;
  const uint32_t w = qz[idx];
  uint32_t r = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) r |= ((w >> awq_shift(i)) & 0xfu) << (4 * i);
  out[idx] = r;
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
  p.waves = 4;
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
  // whole 128-k stages per split, so that the tiled layout's 16-byte stage
  // loads stay aligned (a split past the end gets no steps and stores zeros)
  p.steps_per_split = ((nsteps + p.splits - 1) / p.splits + 3) / 4 * 4;
  return p;
}

template <int FMT, int GM, int XDT, bool PRED>
static void launch_w4_mt(const W4Args& a, const W4Plan& p, hipStream_t stream) {
  dim3 grid(p.tiles * p.splits, p.mblocks);
  if (p.mt == 1)
    hipLaunchKernelGGL((w4a16_skinny_kernel<FMT, 1, GM, XDT, PRED, 4, 4, false>), grid, dim3(256), 0, stream, a);
  else if (p.mt == 2)
    hipLaunchKernelGGL((w4a16_skinny_kernel<FMT, 2, GM, XDT, PRED, 4, 4, false>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((w4a16_skinny_kernel<FMT, 4, GM, XDT, PRED, 4, 4, false>), grid, dim3(256), 0, stream, a);
}

template <int FMT, int GM>
static void launch_w4(const W4Args& a, const W4Plan& p, int xdt, bool pred, hipStream_t stream) {
  if (pred) {
    if (xdt == kXF16) launch_w4_mt<FMT, GM, kXF16, true>(a, p, stream);
    else launch_w4_mt<FMT, GM, kXBF16, true>(a, p, stream);
  } else {
    if (xdt == kXF16) launch_w4_mt<FMT, GM, kXF16, false>(a, p, stream);
    else launch_w4_mt<FMT, GM, kXBF16, false>(a, p, stream);
  }
}

static int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) dev = 0;
  const int slot = dev & 63;
  if (cached[slot] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      n = 256;
    cached[slot] = n;
  }
  return cached[slot];
}

// The decode GEMV covers M <= 16 with K % 128 == 0: 16 waves, each a window
// of S steps of 32 (S = 2, 4 or 8: half, one or two stages; 8 from 17 stages
// up when K % 256 == 0, else 4), 16-byte aligned x rows, and group boundaries
// at fixed steps of every window.  K beyond one pass of the 16 windows (4096
// at S = 8, 2048 at S = 4) is split across workgroups in chunks of whole
// windows (fp32 partials, then the W4 split-K reduce); waves whose window lies
// past K or past their chunk stay inactive (K = 3584: 14 of 16).  Every unit
// count works: with fewer 16-column units than CUs each workgroup owns one
// unit, and with K splits the workgroups per split fill the CUs together.
// *S and *SPG receive the kernel's template values.
static bool gv_plan(const W4Args& a, int fmt, int gmode, GvPlan* p, int* S, int* SPG) {
  if (fmt != kGptq || a.M > 16 || gmode == kGroupsPerK) return false;
  if (a.K % 128 != 0 || (a.K > 4096 && a.swiglu)) return false;
  const int stages = a.K / 128;
  const int s = stages > 16 ? (a.K % 256 == 0 ? 8 : 4) : (stages > 8 ? 4 : 2);
  if (a.K % (32 * s) != 0) return false;
  const int nsteps = a.K / 32;
  p->splits = (nsteps + 16 * s - 1) / (16 * s);
  p->sps = ((nsteps + p->splits - 1) / p->splits + s - 1) / s * s;
  p->splits = (nsteps + p->sps - 1) / p->sps;
  if (a.G % 32 != 0) return false;
  const int spg = a.G / 32;
  int tspg;
  if (spg >= s) {
    if (spg % s != 0) return false;
    tspg = 8;  // one group per window
  } else {
    if (s % spg != 0) return false;
    tspg = spg;
  }
  if (((uintptr_t)a.x % 16) != 0 || (a.ldx % 8) != 0) return false;
  if ((uint64_t)w4_tiled_words(a.N, a.K, a.G, a.zu != 0) * 4u >= ((uint64_t)1 << 31)) return false;
  const int cus = device_cus();
  p->units = (a.N + 15) / 16;
  if (a.swiglu) {
    // whole gate/up unit pairs per workgroup, one round (at most 8 units)
    if (a.layout != kLayoutTiles || (a.N % 32) != 0) return false;
    const int pairs = p->units / 2;
    p->wgs = std::min(cus, pairs);
    if (2 * ((pairs + p->wgs - 1) / p->wgs) > 8) return false;
    *S = s;
    *SPG = tspg;
    return true;
  }
  // with K splits, workgroups per split so that all splits together fill the CUs
  p->wgs = std::min(p->units, std::max(1, cus / p->splits));
  if (p->splits > 1 && (p->units + p->wgs - 1) / p->wgs > GvShape<8, 4>::kOneRound) {
    p->wgs = (p->units + GvShape<8, 4>::kOneRound - 1) / GvShape<8, 4>::kOneRound;
  }
  *S = s;
  *SPG = tspg;
  return true;
}

// fp32 partial bytes of a split-K decode GEMV call (0 without splits); an
// upper bound the workspace sizing uses without the device's CU count.
static size_t gv_split_bytes(int64_t m, int64_t n, int64_t k) {
  if (m > 16 || k % 128 != 0 || k <= 2048) return 0;
  const int64_t s = k % 256 == 0 ? 8 : 4;
  const int64_t nsteps = k / 32;
  int64_t splits = (nsteps + 16 * s - 1) / (16 * s);
  if (splits <= 1) return 0;
  const int64_t sps = ((nsteps + splits - 1) / splits + s - 1) / s * s;
  splits = (nsteps + sps - 1) / sps;
  return ((size_t)splits * (size_t)m * (size_t)n * 4 + 255) / 256 * 256;
}

// Prefill GEMM conditions: tiled weights, M above the GEMV's range, whole
// 128-k stages and groups, 32-bit byte offsets for x16 and the tiled weights.
static bool prefill_applies(const W4Args& a, int gmode) {
  return a.layout == kLayoutTiles && a.M > 16 && gmode != kGroupsPerK && a.K % 128 == 0 &&
         a.G % 128 == 0 && (int64_t)a.M * a.K < ((int64_t)1 << 30) &&
         (uint64_t)w4_tile_words(a.N, a.K) * 4u < ((uint64_t)1 << 31);
}

template <int TM, int TN, int WM, int NS, bool SWIGLU = false>
static void launch_prefill_shape(const W4Args& a, hipStream_t stream, int ksplit = 1) {
  using S = W4pShape<TM, TN, WM>;
  const int mblocks = (a.M + S::BM - 1) / S::BM;
  const int tiles = mblocks * ((a.N + S::BN - 1) / S::BN);
  const int grid = 8 * ((tiles * ksplit + 7) / 8);
  hipLaunchKernelGGL((w4a16_prefill_kernel<TM, TN, WM, NS, SWIGLU>), dim3(grid), dim3(512), 0, stream, a,
                     mblocks, tiles, ksplit);
}

// Tile shapes: 64 x 128 (4-stage ring), 128 x 128 and 128 x 256 (3 stages),
// 128 x 512 (2 stages of 65 KB), all with the 8 waves side by side along N
// (each weight word dequantized once per tile).  Larger tiles copy fewer
// bytes per MFMA but are fewer; the launch takes the shape with the least
// estimated time, rounds of tiles over the CUs times a tile's time under
// full load, measured on C2 (N = 28672, K = 4096): 33, 45, 65 and 112 us.
// Against 128 x 256 tiles from M = 65 on (same process, outputs
// bit-identical): C2 M = 128 61.1 -> 45.3 us (128 x 128), M = 512
// 138 -> 119 us, M = 1024 281 -> 236, M = 2048 511 -> 474 (128 x 512);
// N = 4096 M = 512 63.4 -> 33.2 us and N = 14336 M = 128 61.0 -> 31.2 us
// (64 x 128).  (M = 64: the 4-stage ring 34.4 -> 33.4 us against 3 stages;
// 2 x 4 waves of 64 x 64 took M = 512 152 against 140 us.)
enum { kPfSmall = 0, kPfSquare = 1, kPfNarrow = 2, kPfWide = 3 };
static int prefill_shape(const W4Args& a) {
  if (a.M <= 64) return kPfSmall;
  const int64_t cus = device_cus();
  auto rounds = [&](int64_t bm, int64_t bn) {
    return ((a.M + bm - 1) / bm * ((a.N + bn - 1) / bn) + cus - 1) / cus;
  };
  const int64_t t[4] = {33 * rounds(64, 128), 45 * rounds(128, 128), 65 * rounds(128, 256),
                        112 * rounds(128, 512)};
  int best = kPfWide;  // ties: the larger tile (fewer bytes)
  for (int s = kPfNarrow; s >= kPfSmall; --s)
    if (t[s] < t[best]) best = s;
  return best;
}

// K splits of the 64 x 128 tiles where they leave at least half the CUs idle
// (M <= 64 on narrow projections, e.g. Llama-3-8B down N = 4096: 32 tiles
// over K = 14336): up to 16 splits of at least two stages whose fp32 partials
// fit past the staged activations in `avail` bytes and, together with them,
// in KQ_W4A16_NOALLOC_SCRATCH_BYTES (so the allocation-free entry splits as
// the workspace entry does); the W4 split-K reduce sums them.
static int prefill_splits(const W4Args& a, size_t avail) {
  if (a.swiglu || prefill_shape(a) != kPfSmall) return 1;
  const int64_t cus = device_cus();
  const int64_t tiles = (a.M + 63) / 64 * ((a.N + 127) / 128);
  if (2 * tiles > cus) return 1;
  const size_t x16 = ((size_t)a.M * (size_t)a.K * 2 + 255) / 256 * 256;
  const size_t cap = x16 < (size_t)KQ_W4A16_NOALLOC_SCRATCH_BYTES ? (size_t)KQ_W4A16_NOALLOC_SCRATCH_BYTES - x16 : 0;
  avail = std::min(avail, cap);
  int64_t s = std::min<int64_t>({16, cus / tiles, (a.K / 128) / 2});
  while (s > 1 && (size_t)s * (size_t)a.M * (size_t)a.N * 4 > avail) --s;
  return (int)std::max<int64_t>(1, s);
}

static void launch_prefill(const W4Args& a, int ksplit, hipStream_t stream) {
  if (a.swiglu) {
    // M > 64 (kq_w4a16_tiled_swiglu_gemm): each pair of a wave's column tiles
    // is a gate/up pair; 64 x 256 (4 stages), 128 x 256 or 128 x 512 tiles by
    // the same estimate as prefill_shape, a 64 x 256 round taking 45 us on
    // C2's K.  Gate/up I = 14336 at M = 80 / 128 took 59.3 / 62.0 us on
    // 128 x 256 tiles and 45.0 / 45.6 us on 64 x 256 ones (outputs
    // bit-identical).  (At M <= 64 the fused 64 x 256 form is not used: it took
    // 45.3 us against 41.8 us for the 64 x 128 GEMM and the elementwise pass.)
    const int64_t cus = device_cus();
    auto rounds = [&](int64_t bm, int64_t bn) {
      return ((a.M + bm - 1) / bm * ((a.N + bn - 1) / bn) + cus - 1) / cus;
    };
    const int64_t ts = 45 * rounds(64, 256), tn = 65 * rounds(128, 256), tw = 112 * rounds(128, 512);
    if (tw <= tn && tw <= ts) launch_prefill_shape<8, 4, 1, 2, true>(a, stream);
    else if (tn <= ts) launch_prefill_shape<8, 2, 1, 3, true>(a, stream);
    else launch_prefill_shape<4, 2, 1, 4, true>(a, stream);
    return;
  }
  switch (prefill_shape(a)) {
    case kPfSmall: launch_prefill_shape<4, 1, 1, 4>(a, stream, ksplit); break;
    case kPfSquare: launch_prefill_shape<8, 1, 1, 3>(a, stream); break;
    case kPfNarrow: launch_prefill_shape<8, 2, 1, 3>(a, stream); break;
    default: launch_prefill_shape<8, 4, 1, 2>(a, stream); break;
  }
}

template <int XDT, int S, int SPG>
static void launch_gv_s(const W4Args& a, const GvPlan& p, int layout, hipStream_t st) {
  const int per = (p.units + p.wgs - 1) / p.wgs;
  const int mode = per <= 1                         ? kGvSingle
                   : per <= GvShape<S, SPG>::kShort    ? kGvShort
                   : per <= GvShape<S, SPG>::kOneRound ? kGvOne
                                                       : kGvRounds;
  const dim3 g(p.wgs, p.splits), b(64 * kGvWaves);
#define KQ_GV_LAUNCH(L, M) hipLaunchKernelGGL((w4a16_gemv_kernel<XDT, S, SPG, L, M>), g, b, 0, st, a, p)
  if (a.swiglu) {
    // (gv_plan: tiled operand, at most kOneRound units per workgroup)
    if (a.zu) hipLaunchKernelGGL((w4a16_gemv_kernel<XDT, S, SPG, kLayoutTilesZu, kGvOne, true>), g, b, 0, st, a, p);
    else hipLaunchKernelGGL((w4a16_gemv_kernel<XDT, S, SPG, kLayoutTiles, kGvOne, true>), g, b, 0, st, a, p);
    return;
  }
  if (layout == kLayoutTiles && a.zu) {
    if (mode == kGvSingle) KQ_GV_LAUNCH(kLayoutTilesZu, kGvSingle);
    else if (mode == kGvShort) KQ_GV_LAUNCH(kLayoutTilesZu, kGvShort);
    else if (mode == kGvOne) KQ_GV_LAUNCH(kLayoutTilesZu, kGvOne);
    else KQ_GV_LAUNCH(kLayoutTilesZu, kGvRounds);
  } else if (layout == kLayoutTiles) {
    if (mode == kGvSingle) KQ_GV_LAUNCH(kLayoutTiles, kGvSingle);
    else if (mode == kGvShort) KQ_GV_LAUNCH(kLayoutTiles, kGvShort);
    else if (mode == kGvOne) KQ_GV_LAUNCH(kLayoutTiles, kGvOne);
    else KQ_GV_LAUNCH(kLayoutTiles, kGvRounds);
  } else {
    if (mode == kGvSingle) KQ_GV_LAUNCH(kLayoutRows, kGvSingle);
    else if (mode == kGvShort) KQ_GV_LAUNCH(kLayoutRows, kGvShort);
    else if (mode == kGvOne) KQ_GV_LAUNCH(kLayoutRows, kGvOne);
    else KQ_GV_LAUNCH(kLayoutRows, kGvRounds);
  }
#undef KQ_GV_LAUNCH
}

// Steps per group as gv_plan returns them: 8 = one group per window, else a
// divisor of S below S.
template <int XDT, int S>
static void launch_gv_spg(const W4Args& a, const GvPlan& p, int spg, int layout, hipStream_t st) {
  if constexpr (S >= 4) {
    if (spg == 2) return launch_gv_s<XDT, S, 2>(a, p, layout, st);
  }
  if constexpr (S >= 8) {
    if (spg == 4) return launch_gv_s<XDT, S, 4>(a, p, layout, st);
  }
  if (spg == 1) return launch_gv_s<XDT, S, 1>(a, p, layout, st);
  launch_gv_s<XDT, S, 8>(a, p, layout, st);
}

template <int XDT>
static void launch_gv_x(const W4Args& a, const GvPlan& p, int S, int spg, int layout, hipStream_t st) {
  if (S == 2) launch_gv_spg<XDT, 2>(a, p, spg, layout, st);
  else if (S == 4) launch_gv_spg<XDT, 4>(a, p, spg, layout, st);
  else launch_gv_spg<XDT, 8>(a, p, spg, layout, st);
}

static void launch_gv(const W4Args& a, const GvPlan& p, int xdt, int S, int spg, int layout,
                      hipStream_t st) {
  if (xdt == kXF16) launch_gv_x<kXF16>(a, p, S, spg, layout, st);
  else launch_gv_x<kXBF16>(a, p, S, spg, layout, st);
}

static int run_w4(const char* what, int fmt, W4Args a, int gmode, void* workspace,
                  size_t ws_bytes, hipStream_t stream) {
  if (a.x_dtype != KQ_DTYPE_F16 && a.x_dtype != KQ_DTYPE_BF16) {
    set_error("%s: activation dtype must be fp16 or bf16", what);
    return KQ_EUNSUPPORTED;
  }
  if (a.M < 0 || a.N < 8 || a.K < 1 || (a.N % 8) != 0 || a.G < 1 || a.ldx < a.K ||
      a.K >= (1 << 24) || a.G >= (1 << 16)) {
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
  // floor(k / G) = (k * ceil(2^40 / G)) >> 40, exact for k < 2^24, G < 2^16
  a.gmagic = (((uint64_t)1 << 40) + (uint64_t)a.G - 1) / (uint64_t)a.G;
  const bool needs_x16 = gmode == kGroupsPermuted;
  GvPlan gp{};
  int gv_s = 0, gv_spg = 0;
  if (gv_plan(a, fmt, gmode, &gp, &gv_s, &gv_spg)) {
    int xdt = a.x_dtype == KQ_DTYPE_F16 ? kXF16 : kXBF16;
    // act-order x gather first, then the split partials
    const size_t x16_bytes = needs_x16 ? ((size_t)a.M * a.K * 2 + 255) / 256 * 256 : 0;
    const size_t part_bytes = gp.splits > 1 ? (size_t)gp.splits * a.M * a.N * 4 : 0;
    if (x16_bytes + part_bytes > 0 && (workspace == nullptr || ws_bytes < x16_bytes + part_bytes)) {
      set_error("%s: workspace of %zu bytes is smaller than the %zu bytes this call needs", what,
                workspace ? ws_bytes : (size_t)0, x16_bytes + part_bytes);
      return KQ_EWORKSPACE;
    }
    a.splits = gp.splits;
    a.steps_per_split = gp.sps;
    a.partials = gp.splits > 1 ? (float*)((uint8_t*)workspace + x16_bytes) : nullptr;
    if (needs_x16) {
      // act-order: gather x through the permutation once per call
      uint16_t* x16 = (uint16_t*)workspace;
      // (gv_plan: M <= 16, K % 128 == 0, 16-byte aligned x rows)
      hipLaunchKernelGGL(w4a16_prep_x_row_kernel, dim3((unsigned)((a.K + 1023) / 1024), (unsigned)a.M),
                         dim3(128), (size_t)a.K * 2, stream, a.x, a.x_dtype, a.ldx, a.perm, a.K, x16);
      a.x = x16;
      a.ldx = a.K;
      xdt = kXF16;
    }
    launch_gv(a, gp, xdt, gv_s, gv_spg, a.layout, stream);
    if (gp.splits > 1) {
      ReduceArgs r{a.partials, gp.splits, a.M, a.N, nullptr, nullptr, 0, a.bias, a.bias_dtype,
                   a.out, a.out_dtype, nullptr, a.swiglu_split ? 2 : 0};
      launch_splitk_reduce(kReduceW4, r, stream);
    }
    return check_launch(what);
  }
  if (prefill_applies(a, gmode)) {
    const size_t x16_bytes = (size_t)a.M * a.K * 2;
    if (workspace == nullptr || ws_bytes < x16_bytes) {
      set_error("%s: workspace of %zu bytes is smaller than the %zu bytes this call needs", what,
                workspace ? ws_bytes : (size_t)0, x16_bytes);
      return KQ_EWORKSPACE;
    }
    uint16_t* x16 = (uint16_t*)workspace;
    const size_t x16_al = (x16_bytes + 255) / 256 * 256;
    const int ks = prefill_splits(a, ws_bytes > x16_al ? ws_bytes - x16_al : 0);
    a.partials = ks > 1 ? (float*)((uint8_t*)workspace + x16_al) : nullptr;
    const int64_t threads = (int64_t)a.M * a.K / 8;
    hipLaunchKernelGGL(w4a16_prep_x_mma_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       stream, a.x, a.x_dtype, a.ldx, gmode == kGroupsPermuted ? a.perm : nullptr,
                       a.M, a.K, x16);
    a.x = x16;
    a.ldx = a.K;
    launch_prefill(a, ks, stream);
    if (ks > 1) {
      ReduceArgs r{a.partials, ks, a.M, a.N, nullptr, nullptr, 0, a.bias, a.bias_dtype,
                   a.out, a.out_dtype, nullptr};
      launch_splitk_reduce(kReduceW4, r, stream);
    }
    return check_launch(what);
  }
  W4Plan p = plan_w4(a.M, a.N, a.K, needs_x16, ws_bytes, workspace != nullptr);
  if (p.x16_bytes + p.partial_bytes > (workspace ? ws_bytes : 0)) {
    set_error("%s: workspace of %zu bytes is smaller than the %zu bytes this call needs", what,
              workspace ? ws_bytes : (size_t)0, p.x16_bytes + p.partial_bytes);
    return KQ_EWORKSPACE;
  }
  int xdt = a.x_dtype == KQ_DTYPE_F16 ? kXF16 : kXBF16;
  if (needs_x16) {
    uint16_t* x16 = (uint16_t*)workspace;
    const int64_t threads = ((int64_t)a.M * a.K + 7) / 8;
    hipLaunchKernelGGL(w4a16_prep_x_kernel, dim3((unsigned)((threads + 63) / 64)), dim3(64), 0,
                       stream, a.x, a.x_dtype, a.ldx, a.perm, a.M, a.K, x16);
    a.x = x16;
    a.ldx = a.K;
    xdt = kXF16;
  }
  const bool pred = (a.K % 32) != 0 || ((uintptr_t)a.x % 16) != 0 || (a.ldx % 8) != 0;
  a.splits = p.splits;
  a.steps_per_split = p.steps_per_split;
  a.partials = p.splits > 1 ? (float*)((uint8_t*)workspace + p.x16_bytes) : nullptr;
  // kernel group addressing: per element (g_idx, or a group boundary inside
  // an 8-row chunk), per lane chunk, or per step for the whole wave
  const int gm = gmode == kGroupsPerK ? kGElem : ((a.G % 32) == 0 ? kGStep : kGLane);
  if (fmt == kGptq) {
    if (gm == kGElem) launch_w4<kGptq, kGElem>(a, p, xdt, pred, stream);
    else if (gm == kGStep) launch_w4<kGptq, kGStep>(a, p, xdt, pred, stream);
    else launch_w4<kGptq, kGLane>(a, p, xdt, pred, stream);
  } else {
    if (gm == kGElem) launch_w4<kAwq, kGElem>(a, p, xdt, pred, stream);
    else if (gm == kGStep) launch_w4<kAwq, kGStep>(a, p, xdt, pred, stream);
    else launch_w4<kAwq, kGLane>(a, p, xdt, pred, stream);
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

// The scratch a call needs at least (the prefill GEMM without K splits).
static size_t w4_min_workspace(int64_t m, int64_t n, int64_t k, int gidx_mode) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  // a generous workspace lets the planner choose split-K freely
  const W4Plan p = plan_w4((int)m, (int)n, (int)k, gidx_mode == kGroupsPermuted,
                           (size_t)1 << 40, true);
  // the prefill GEMM (M > 16, tiled weights) stages fp16 x in the workspace;
  // the decode GEMV keeps the act-order gather and its split partials there
  const size_t x16 = m > 16 ? ((size_t)m * (size_t)k * 2 + 255) / 256 * 256 : 0;
  const size_t gv = (gidx_mode == kGroupsPermuted ? ((size_t)m * (size_t)k * 2 + 255) / 256 * 256 : 0) +
                    gv_split_bytes(m, n, k);
  return std::max({p.x16_bytes + p.partial_bytes, x16, gv});
}

extern "C" size_t kq_w4a16_workspace_size(int64_t m, int64_t n, int64_t k, int gidx_mode) {
  const size_t need = w4_min_workspace(m, n, k, gidx_mode);
  if (need == 0 || m <= 16 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) return need;
  // the prefill GEMM's K-split partials past its staged activations
  W4Args a{};
  a.M = (int)m;
  a.N = (int)n;
  a.K = (int)k;
  const int ks = prefill_splits(a, (size_t)1 << 40);
  const size_t x16 = ((size_t)m * (size_t)k * 2 + 255) / 256 * 256;
  return ks > 1 ? std::max(need, x16 + (size_t)ks * (size_t)m * (size_t)n * 4) : need;
}

// Offset of the SwiGLU two-pass intermediate: after the GEMM's own scratch.
static size_t swiglu_ws_offset(int64_t m, int64_t n, int64_t k, int gmode) {
  return (kq_w4a16_workspace_size(m, n, k, gmode) + 255) / 256 * 256;
}

extern "C" size_t kq_w4a16_swiglu_workspace_size(int64_t m, int64_t i_width, int64_t k,
                                                 int gidx_mode) {
  if (m <= 0 || i_width <= 0 || k <= 0) return 0;
  return swiglu_ws_offset(m, 2 * i_width, k, gidx_mode) + (size_t)m * (size_t)(2 * i_width) * 2;
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
  a.M = (int)m; a.N = (int)n; a.K = (int)k; a.G = group_size; a.zoff = 0u;
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
  a.M = (int)m; a.N = (int)n; a.K = (int)k; a.G = group_size; a.zoff = 1u;
  return run_w4("kq_w4a16_gptq_gemm", kGptq, a, gidx_mode, workspace, workspace_bytes,
                (hipStream_t)stream);
}

// Shapes the tiled operand supports (32-bit k and group arithmetic of the
// kernels; whole packed rows and 8-row group chunks).
static bool tiled_shape_ok(int64_t n, int64_t k, int64_t group_size) {
  return n >= 8 && k >= 8 && (n % 8) == 0 && (k % 8) == 0 && n <= 0x7fffffff && k < (1 << 24) &&
         group_size >= 8 && (group_size % 8) == 0 && group_size < (1 << 16);
}

// Arguments of the tiled entry points (validated; a.layout = tiles).
static int tiled_args(const char* what, const void* x, int x_dtype, const int32_t* tiles,
                      const int32_t* qzeros, int zero_offset, const void* scales,
                      const int32_t* perm, const void* bias, int bias_dtype, void* out, int64_t m,
                      int64_t n, int64_t k, int group_size, W4Args* args) {
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) {
    set_error("%s: dimensions exceed int32", what);
    return KQ_EINVAL;
  }
  const bool zu = qzeros == nullptr;
  if (k % 8 != 0 || group_size % 8 != 0 || zero_offset < 0 || zero_offset > (zu ? 16 : 1)) {
    set_error("%s: needs k %% 8 == 0, group_size %% 8 == 0, zero_offset 0 or 1 (0..16 without "
              "qzeros)", what);
    return KQ_EINVAL;
  }
  if (!tiled_shape_ok(n, k, group_size) ||
      (uint64_t)w4_tiled_words((int)n, (int)k, group_size, zu) * 4u >= ((uint64_t)1 << 32)) {
    set_error("%s: tiled weight exceeds 4 GiB or bad shape", what);
    return KQ_EINVAL;
  }
  W4Args a{};
  a.x = (const uint16_t*)x; a.x_dtype = x_dtype; a.ldx = (int)k;
  a.qw = (const uint32_t*)tiles; a.qz = (const uint32_t*)qzeros; a.sc = (const uint16_t*)scales;
  // one zero: the other kernels read the operand's zero-nibble words
  if (zu)
    a.qz = (const uint32_t*)tiles + w4_tile_words((int)n, (int)k) +
           w4_table_words((int)n, (int)k, group_size, true);
  a.zu = zu ? 1 : 0;
  a.perm = perm;
  a.bias = bias; a.bias_dtype = bias_dtype; a.out = (uint16_t*)out; a.out_dtype = x_dtype;
  a.M = (int)m; a.N = (int)n; a.K = (int)k; a.G = group_size; a.zoff = (uint32_t)zero_offset;
  a.layout = kLayoutTiles;
  *args = a;
  return KQ_OK;
}

extern "C" int kq_w4a16_tiled_gemm(const void* x, int x_dtype, const int32_t* tiles,
                                   const int32_t* qzeros, int zero_offset, const void* scales,
                                   const int32_t* perm, const void* bias, int bias_dtype, void* out,
                                   int64_t m, int64_t n, int64_t k, int group_size, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  W4Args a{};
  const int status = tiled_args("kq_w4a16_tiled_gemm", x, x_dtype, tiles, qzeros, zero_offset,
                                scales, perm, bias, bias_dtype, out, m, n, k, group_size, &a);
  if (status != KQ_OK) return status;
  return run_w4("kq_w4a16_tiled_gemm", kGptq, a, perm ? kGroupsPermuted : kGroupsUniform,
                workspace, workspace_bytes, (hipStream_t)stream);
}

// Packed gate/up projection with SwiGLU (layers.py:243-244): the tiled operand
// covers 2I columns, 16-column blocks of gate and up alternating.  Decode
// shapes run the GEMV with the SwiGLU epilogue; others the tiled GEMM into
// the workspace (after its own scratch) and the elementwise pass.
static size_t swiglu_ws_offset(int64_t m, int64_t n, int64_t k, int gmode);

extern "C" int kq_w4a16_tiled_swiglu_gemm(const void* x, int x_dtype, const int32_t* tiles,
                                          const int32_t* qzeros, int zero_offset,
                                          const void* scales, const int32_t* perm,
                                          const void* bias, int bias_dtype, void* out, int64_t m,
                                          int64_t i_width, int64_t k, int group_size,
                                          void* workspace, size_t workspace_bytes, void* stream) {
  const char* what = "kq_w4a16_tiled_swiglu_gemm";
  if (i_width < 16 || (i_width % 16) != 0 || i_width > 0x3fffffff) {
    set_error("%s: the activation width must be a positive multiple of 16 (got %lld)", what,
              (long long)i_width);
    return KQ_EINVAL;
  }
  const int64_t n = 2 * i_width;
  W4Args a{};
  int status = tiled_args(what, x, x_dtype, tiles, qzeros, zero_offset, scales, perm, bias,
                          bias_dtype, out, m, n, k, group_size, &a);
  if (status != KQ_OK) return status;
  const int gmode = perm ? kGroupsPermuted : kGroupsUniform;
  GvPlan gp{};
  int s_ = 0, spg_ = 0;
  a.swiglu = 1;
  // decode GEMV or (M > 64) prefill GEMM with the SwiGLU epilogue: one launch
  // (plus the activation staging pass), out written directly.  Llama-3-8B
  // gate/up (K = 4096, I = 14336, act-order), graph replay: M = 512 169 ->
  // 135 us, 2048 636 -> 495 us, 4096 1333 -> 1015 us against the GEMM and the
  // elementwise pass
  if (a.M > 0 && (gv_plan(a, kGptq, gmode, &gp, &s_, &spg_) || (a.M > 64 && prefill_applies(a, gmode))))
    return run_w4(what, kGptq, a, gmode, workspace, workspace_bytes, (hipStream_t)stream);
  a.swiglu = 0;
  // decode shapes whose K takes more than one GEMV pass (K > 4096): the plain
  // GEMV's K chunks meet in the split-K reduce, which pairs each gate column
  // with its up column 16 on and stores silu(gate) * up (the bits of the
  // reduce's store followed by the elementwise pass)
  if (a.M > 0 && gv_plan(a, kGptq, gmode, &gp, &s_, &spg_) && gp.splits > 1) {
    a.swiglu_split = 1;
    return run_w4(what, kGptq, a, gmode, workspace, workspace_bytes, (hipStream_t)stream);
  }
  // two passes: [m][2I] in the activation dtype after the GEMM's scratch
  if (m == 0) return KQ_OK;
  const size_t off = swiglu_ws_offset(m, n, k, gmode);
  const size_t need = off + (size_t)m * (size_t)n * 2;
  if (workspace == nullptr || workspace_bytes < need) {
    set_error("%s: workspace of %zu bytes is smaller than the %zu bytes this call needs", what,
              workspace ? workspace_bytes : (size_t)0, need);
    return KQ_EWORKSPACE;
  }
  uint16_t* mid = (uint16_t*)((char*)workspace + off);
  a.out = mid;
  status = run_w4(what, kGptq, a, gmode, workspace, off, (hipStream_t)stream);
  if (status != KQ_OK) return status;
  const int64_t pairs = m * i_width / 2;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)mid, n, 1, x_dtype, (uint16_t*)out, m,
                     i_width);
  return check_launch(what);
}

extern "C" int kq_swiglu(const void* src, int64_t ld_src, int interleaved, int dtype, void* dst,
                         int64_t m, int64_t i_width, void* stream) {
  if (m < 0 || i_width < 2 || (i_width % 2) != 0 || ld_src < 2 * i_width ||
      (interleaved && (i_width % 16) != 0) || (dtype != KQ_DTYPE_F16 && dtype != KQ_DTYPE_BF16)) {
    set_error("kq_swiglu: bad arguments m=%lld i=%lld ld=%lld dtype=%d", (long long)m,
              (long long)i_width, (long long)ld_src, dtype);
    return KQ_EINVAL;
  }
  if (m == 0) return KQ_OK;
  const int64_t pairs = m * i_width / 2;
  hipLaunchKernelGGL(swiglu_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint16_t*)src, ld_src, interleaved, dtype,
                     (uint16_t*)dst, m, i_width);
  return check_launch("kq_swiglu");
}

// ---------------------------------------------------------------------------
// Allocation-free form of kq_w4a16_tiled_gemm.  Its scratch (the act-order
// activation gather, the prefill GEMM's staged activations, split-K partial
// sums) lives in this fixed array, which the runtime places once on every
// device the library is loaded on.  Every scratch byte a call reads is written
// earlier in the same call (gathers and partial planes are written in full),
// so nothing needs clearing between calls; calls that overlap on one device
// share the array and race.
static __device__ __align__(256) uint8_t scratch[KQ_W4A16_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kScratchDevices] = {};
}  // namespace

// Device address of `scratch` on the current device, resolved once per device
// (the symbol's host-side name is not a device address).
static int current_scratch(const char* what, void** ptr) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kScratchDevices) {
    set_error("%s: no current device (or device index %d beyond %d)", what, dev, kScratchDevices);
    return KQ_EUNSUPPORTED;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_ptr[dev] == nullptr) {
    void* address = nullptr;
    const hipError_t err = hipGetSymbolAddress(&address, HIP_SYMBOL(scratch));
    if (err != hipSuccess || address == nullptr) {
      set_error("%s: hipGetSymbolAddress(scratch) failed on device %d: %s", what, dev,
                hipGetErrorString(err));
      return KQ_ELAUNCH;
    }
    g_scratch_ptr[dev] = address;
  }
  *ptr = g_scratch_ptr[dev];
  return KQ_OK;
}

extern "C" int kq_w4a16_tiled_gemm_noalloc(const void* x, int x_dtype, const int32_t* tiles,
                                           const int32_t* qzeros, int zero_offset,
                                           const void* scales, const int32_t* perm,
                                           const void* bias, int bias_dtype, void* out, int64_t m,
                                           int64_t n, int64_t k, int group_size, void* stream) {
  const char* what = "kq_w4a16_tiled_gemm_noalloc";
  W4Args a{};
  int status = tiled_args(what, x, x_dtype, tiles, qzeros, zero_offset, scales, perm, bias,
                          bias_dtype, out, m, n, k, group_size, &a);
  if (status != KQ_OK) return status;
  const size_t need = kq_w4a16_workspace_size(m, n, k, perm ? kGroupsPermuted : kGroupsUniform);
  if (need > (size_t)KQ_W4A16_NOALLOC_SCRATCH_BYTES) {
    set_error("%s: m=%lld n=%lld k=%lld needs %zu bytes of scratch, more than the fixed %zu "
              "(use kq_w4a16_tiled_gemm with a workspace)", what, (long long)m, (long long)n,
              (long long)k, need, (size_t)KQ_W4A16_NOALLOC_SCRATCH_BYTES);
    return KQ_EWORKSPACE;
  }
  void* buffer = nullptr;
  status = current_scratch(what, &buffer);
  if (status != KQ_OK) return status;
  return run_w4(what, kGptq, a, perm ? kGroupsPermuted : kGroupsUniform, buffer,
                (size_t)KQ_W4A16_NOALLOC_SCRATCH_BYTES, (hipStream_t)stream);
}

extern "C" int64_t kq_w4a16_tiled_words(int64_t n, int64_t k, int group_size, int one_zero) {
  if (!tiled_shape_ok(n, k, group_size)) return -1;
  return w4_tiled_words((int)n, (int)k, group_size, one_zero != 0);
}

extern "C" int kq_w4a16_tile_weights(const int32_t* qweight, int src_format, const int32_t* perm,
                                     const int32_t* qzeros, int zero_offset, const void* scales,
                                     int32_t* tiles, int64_t n, int64_t k, int group_size,
                                     void* stream) {
  const bool zu = qzeros == nullptr;
  if (!tiled_shape_ok(n, k, group_size) || (src_format != 0 && src_format != 1) ||
      zero_offset < 0 || zero_offset > (zu ? 16 : 1)) {
    set_error("kq_w4a16_tile_weights: bad arguments n=%lld k=%lld group=%d format=%d zero_offset=%d",
              (long long)n, (long long)k, group_size, src_format, zero_offset);
    return KQ_EINVAL;
  }
  if ((uint64_t)w4_tiled_words((int)n, (int)k, group_size, zu) * 4u >= ((uint64_t)1 << 32)) {
    set_error("kq_w4a16_tile_weights: tiled weight exceeds 4 GiB");
    return KQ_EINVAL;
  }
  const int64_t words = w4_tile_words((int)n, (int)k);
  hipLaunchKernelGGL(w4_tile_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint32_t*)qweight, src_format == 0 ? 1 : 0, perm,
                     (uint32_t*)tiles, (int)n, (int)k);
  const int64_t table = w4_tiled_words((int)n, (int)k, group_size, zu) - words;
  hipLaunchKernelGGL(w4_scale_zero_kernel, dim3((unsigned)((table + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint32_t*)qzeros, (uint32_t)zero_offset,
                     (const uint16_t*)scales, (uint32_t*)tiles + words, (int)n, (int)k, group_size);
  return check_launch("kq_w4a16_tile_weights");
}

extern "C" int kq_awq_natural_zeros(const int32_t* qzeros, int32_t* qzeros_n, int64_t n,
                                    int64_t groups, void* stream) {
  if (n < 8 || (n % 8) != 0 || groups < 1) {
    set_error("kq_awq_natural_zeros: bad shape n=%lld groups=%lld", (long long)n, (long long)groups);
    return KQ_EINVAL;
  }
  const int64_t words = groups * (n / 8);
  hipLaunchKernelGGL(awq_natural_zeros_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, (const uint32_t*)qzeros, (uint32_t*)qzeros_n, words);
  return check_launch("kq_awq_natural_zeros");
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
