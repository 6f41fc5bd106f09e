// Block-scaled FP8 MoE experts and the dense block-FP8 linear for gfx950.
//
// Contract (Qwen3-MoE sparse block, reference kairyu/models/moe.py:27-119,
// 255-273, kairyu/models/grouped_moe.py:239-330, moe_parallel.py:255-283):
//   route:   top-k experts by a stable descending sort of the router logits
//            (ties -> smaller expert id); weights = fp32 softmax over the
//            selected logits, or over all logits gathered at the selection;
//   expert:  y = down(silu(gate(x)) * up(x)) in the hidden dtype (bf16 or
//            fp16 rounding after each step), every projection a block-FP8
//            linear: weight e4m3 [out, in] with fp32 scales per 128x128 block
//            (W = q * S[n/128][k/128]), activations quantized per token per
//            128-wide K block (s = max(amax, 1e-12) / 448, q = e4m3(x / s)),
//            each projection's output rounded to the activation dtype;
//   combine: out = sum over slots, in slot order, of fp32(y) * w, in fp32,
//            one final cast.
//
// Pipeline on the device, no host synchronization (graph-capturable):
//   1. moe_count / moe_scan / moe_scatter: stable sort of the T*k routed rows
//      by expert (per-chunk histograms, one-workgroup scan that also lays out
//      the grid's M tiles, per-chunk ranks); every output row keeps the
//      ascending flat order inside its expert segment.
//   2. act_quant_fp8_blocks: each token quantized once (not once per slot).
//   3. grouped GEMM 1 (gate_up): A rows gathered through the sorted order,
//      B = the expert's stacked [gate; up] weight.  A 64 x 256 tile pairs
//      gate columns [n0, n0+128) with up columns [I+n0, I+n0+128), so the
//      epilogue forms bf16 SwiGLU and quantizes the finished 128-column
//      activation block to e4m3 in registers (no bf16 intermediate in HBM).
//   4. grouped GEMM 2 (down): 64 x 256 tiles -> expert outputs (bf16/fp16).
//   5. combine: fp32 slot-order weighted sum per token.
// Both GEMMs use v_mfma_scale_f32_16x16x128_f8f6f4 (unit E8M0 scales): one
// MFMA spans one 128-wide K block, and its fp32 result is scaled by
// s_act[row][kb] * s_w[nb][kb] before it is added to the accumulator.
#include "kq_common.h"

#include <algorithm>

namespace kq {

// ------------------------------------------------------------------ routing
constexpr int kRouteMaxPerLane = 8;   // experts <= 512
constexpr int kRouteMaxTopK = 32;

// Sortable key of a float: larger value -> larger key; -0 == +0; NaN largest.
KQ_DEV uint32_t float_key(float v) {
  if (v == 0.0f) v = 0.0f;
  const uint32_t u = __float_as_uint(v);
  if (v != v) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

KQ_DEV uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)v, off, 64);
    const uint32_t hi = __shfl_xor((uint32_t)(v >> 32), off, 64);
    const uint64_t o = ((uint64_t)hi << 32) | lo;
    v = o > v ? o : v;
  }
  return v;
}

KQ_DEV float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

KQ_DEV float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// One wave per token: k rounds of a wave-wide max over (value key, -expert);
// every lane sees each round's winner, lane r keeps slot r's logit.
__global__ void __launch_bounds__(256)
moe_route_kernel(const void* __restrict__ logits, int dtype, int T, int E, int k, int norm,
                 int32_t* __restrict__ idx, float* __restrict__ w) {
  const int lane = lane_id();
  const int t = blockIdx.x * 4 + wave_id();
  if (t >= T) return;
  float v[kRouteMaxPerLane];
  bool live[kRouteMaxPerLane];
#pragma unroll
  for (int i = 0; i < kRouteMaxPerLane; ++i) {
    const int e = lane + 64 * i;
    live[i] = e < E;
    v[i] = live[i] ? load_as_f32(logits, dtype, (int64_t)t * E + e) : 0.0f;
  }
  float my_sel = 0.0f, first = 0.0f, denom = 0.0f;
  for (int r = 0; r < k; ++r) {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < kRouteMaxPerLane; ++i) {
      if (!live[i]) continue;
      const uint64_t key = ((uint64_t)float_key(v[i]) << 32) |
                           (uint32_t)(0xffffffffu - (uint32_t)(lane + 64 * i));
      best = key > best ? key : best;
    }
    best = wave_max_u64(best);
    const int e = (int)(0xffffffffu - (uint32_t)best);
    const float val = key_float((uint32_t)(best >> 32));
#pragma unroll
    for (int i = 0; i < kRouteMaxPerLane; ++i)
      if (lane + 64 * i == e) live[i] = false;
    if (lane == 0) idx[(int64_t)t * k + r] = e;
    if (lane == r) my_sel = val;
    if (r == 0) first = val;
    if (norm) denom = __fadd_rn(denom, expf(val - first));  // slot order, uniform
  }
  // fp32 softmax over the selected logits, or over all logits gathered
  float mx = first;
  if (!norm) {
    float m = -__builtin_inff();
#pragma unroll
    for (int i = 0; i < kRouteMaxPerLane; ++i)
      if (lane + 64 * i < E) m = fmaxf(m, v[i]);
    mx = wave_max(m);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kRouteMaxPerLane; ++i)
      if (lane + 64 * i < E) sum += expf(v[i] - mx);
    denom = wave_sum(sum);
  }
  if (lane < k) w[(int64_t)t * k + lane] = __fdiv_rn(expf(my_sel - mx), denom);
}

// -------------------------------------------------------------- stable sort
constexpr int kSortChunk = 1024;

// Per-chunk expert histogram: counts[c][e].
__global__ void __launch_bounds__(256)
moe_count_kernel(const int32_t* __restrict__ idx, int R, int E, int32_t* __restrict__ counts) {
  extern __shared__ int hist[];
  for (int i = threadIdx.x; i < E; i += 256) hist[i] = 0;
  __syncthreads();
  const int c = blockIdx.x;
  for (int j = threadIdx.x; j < kSortChunk; j += 256) {
    const int r = c * kSortChunk + j;
    if (r < R) {
      const int e = idx[r];
      if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < E; i += 256) counts[(int64_t)c * E + i] = hist[i];
}

// One workgroup: expert offsets, per-chunk output bases and the M-tile table
// (tile i -> (expert, first row)); unused table entries get expert -1.
__global__ void __launch_bounds__(1024)
moe_scan_kernel(const int32_t* __restrict__ counts, int C, int E, int BM, int max_tiles,
                int32_t* __restrict__ offsets, int32_t* __restrict__ base, int32_t* __restrict__ tiles) {
  __shared__ int tot[1024], ntile[1024], off[1024], tstart[1024];
  __shared__ int total_tiles;
  for (int e = threadIdx.x; e < E; e += 1024) {
    int s = 0;
    for (int c = 0; c < C; ++c) {
      base[(int64_t)c * E + e] = s;
      s += counts[(int64_t)c * E + e];
    }
    tot[e] = s;
    ntile[e] = (s + BM - 1) / BM;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0, trun = 0;
    for (int e = 0; e < E; ++e) {
      off[e] = run;
      offsets[e] = run;
      run += tot[e];
      tstart[e] = trun;
      trun += ntile[e];
    }
    offsets[E] = run;
    total_tiles = trun;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < E; e += 1024) {
    for (int c = 0; c < C; ++c) base[(int64_t)c * E + e] += off[e];
    for (int i = 0; i < ntile[e] && tstart[e] + i < max_tiles; ++i) {
      tiles[2 * (tstart[e] + i)] = e;
      tiles[2 * (tstart[e] + i) + 1] = off[e] + i * BM;
    }
  }
  for (int i = total_tiles + threadIdx.x; i < max_tiles; i += 1024) {
    tiles[2 * i] = -1;
    tiles[2 * i + 1] = 0;
  }
}

// One wave per chunk: sorted position of flat row r = base[c][e] + its rank
// among the chunk's earlier rows routed to the same expert.
__global__ void __launch_bounds__(64)
moe_scatter_kernel(const int32_t* __restrict__ idx, int R, int E, const int32_t* __restrict__ base,
                   int32_t* __restrict__ sorted_rows, int32_t* __restrict__ inv) {
  extern __shared__ int running[];
  for (int i = threadIdx.x; i < E; i += 64) running[i] = 0;
  __syncthreads();
  const int c = blockIdx.x, lane = threadIdx.x;
  for (int g = 0; g < kSortChunk / 64; ++g) {
    const int r = c * kSortChunk + g * 64 + lane;
    const int e = r < R ? idx[r] : -1;
    const bool ok = e >= 0 && e < E;
    int rank = 0;
    for (int d = 1; d < 64; ++d) {
      const int o = __shfl(e, (lane - d) & 63, 64);
      rank += (d <= lane && o == e) ? 1 : 0;
    }
    const int before = ok ? running[e] : 0;
    __syncthreads();
    if (ok) {
      const int pos = base[(int64_t)c * E + e] + before + rank;
      sorted_rows[pos] = r;
      inv[r] = pos;
      atomicAdd(&running[e], 1);
    } else if (r < R) {
      inv[r] = -1;
    }
    __syncthreads();
  }
}

// --------------------------------------------------- 1x128 activation quant
// Grid (rows, ceil(K / 2048)); 256 threads x 8 elements; 16 threads per block.
__global__ void __launch_bounds__(256)
act_quant_fp8_blocks_kernel(const uint16_t* __restrict__ x, int dtype, int K, int64_t ldx, bool vec,
                            uint8_t* __restrict__ xq, float* __restrict__ xs) {
  const int64_t row = blockIdx.x;
  const int k0 = blockIdx.y * 2048 + threadIdx.x * 8;
  const uint16_t* xr = x + row * ldx;
  float v[8];
  if (vec && k0 + 8 <= K) {
    const u32x4 raw = *(const u32x4*)(xr + k0);
#pragma unroll
    for (int d = 0; d < 4; ++d) {
      v[2 * d] = dtype == KQ_DTYPE_BF16 ? bf16_to_f32(raw[d] & 0xffffu) : f16_to_f32(raw[d] & 0xffffu);
      v[2 * d + 1] = dtype == KQ_DTYPE_BF16 ? bf16_to_f32(raw[d] >> 16) : f16_to_f32(raw[d] >> 16);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      v[e] = k0 + e < K ? (dtype == KQ_DTYPE_BF16 ? bf16_to_f32(xr[k0 + e]) : f16_to_f32(xr[k0 + e])) : 0.0f;
  }
  float amax = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off, 64));
  if (k0 >= K) return;
  const float s = __fdiv_rn(fmaxf(amax, 1e-12f), 448.0f);
  uint32_t lo = 0, hi = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float q = __fdiv_rn(v[e], s);
    q = q < -448.0f ? -448.0f : (q > 448.0f ? 448.0f : q);
    const uint32_t b = f32_to_e4m3(q);
    if (e < 4) lo |= b << (8 * e);
    else hi |= b << (8 * (e - 4));
  }
  uint8_t* qr = xq + row * (int64_t)K;
  if (k0 + 8 <= K && (K % 8) == 0) {
    *(u32x2*)(qr + k0) = u32x2{lo, hi};
  } else {
    for (int e = 0; e < 8 && k0 + e < K; ++e) qr[k0 + e] = (uint8_t)(((e < 4 ? lo : hi) >> (8 * (e & 3))) & 0xffu);
  }
  if ((threadIdx.x & 15) == 0) xs[row * ((K + 127) / 128) + k0 / 128] = s;
}

// ------------------------------------------------------------ grouped GEMM
constexpr int kBM = 64;     // rows per tile
constexpr int kBN = 256;    // weight rows per tile
constexpr int kBK = 128;    // one scale block of K per step
enum { kModeGateUp = 0, kModeDown = 1 };

struct MoeGemmArgs {
  const uint8_t* a;        // e4m3 activation rows of length K
  const float* as;         // activation block scales [rows][K/128]
  const int32_t* rows;     // sorted row -> flat routed row (token = flat / topk); null: identity
  int topk;
  const uint8_t* w;        // [E][N][K] e4m3
  const float* ws;         // [E][N/128][K/128]
  const int32_t* tiles;    // [max_tiles][2] (expert, first row); null: dense tiles of M rows
  const int32_t* offsets;  // [E+1] expert row offsets; null: dense
  int M;                   // dense row count
  int N, K, I;             // weight rows, K, activation width (gate_up: N = 2I)
  int mtiles, ntiles;
  uint8_t* actq;           // gate_up: e4m3 activations [rows][I] (out_dtype: their dtype)
  float* acts;             // gate_up: their block scales [rows][I/128]
  void* out;               // down: [rows][N] in out_dtype
  int out_dtype;
  const void* bias;        // down (dense linear only)
  int bias_dtype;
};

KQ_DEV int tswz(int r, int c) { return r * 128 + ((c ^ (r & 7)) << 4); }

// Round to the activation dtype (bf16 or fp16) and back.
KQ_DEV float round_act(float v, int dtype) {
  return dtype == KQ_DTYPE_BF16 ? bf16_to_f32(f32_to_bf16(v)) : f16_to_f32(f32_to_f16(v));
}

template <int MODE>
__global__ void __launch_bounds__(256)
moe_gemm_kernel(MoeGemmArgs a) {
  // one LDS stage (40 KB: up to three workgroups per CU); the next K block
  // is fetched into registers while this one is multiplied
  __shared__ __attribute__((aligned(16))) uint8_t sA[kBM * kBK];
  __shared__ __attribute__((aligned(16))) uint8_t sB[kBN * kBK];
  __shared__ float sS[kBM];
  __shared__ float sRed[4][kBM];
  const int tid = threadIdx.x, lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  // tiles sharing an n-tile and an expert are adjacent and land on one XCD
  const int nblk = a.mtiles * a.ntiles;
  const int L = xcd_swizzle(blockIdx.x, nblk);
  const int ntile = L / a.mtiles, mtile = L % a.mtiles;
  int e, row0, row_end;
  if (a.tiles) {
    e = a.tiles[2 * mtile];
    if (e < 0) return;
    row0 = a.tiles[2 * mtile + 1];
    row_end = a.offsets[e + 1];
  } else {
    e = 0;
    row0 = mtile * kBM;
    row_end = a.M;
  }
  const int KB = a.K / kBK;
  const int NB = (a.N + 127) / 128;
  const int n0 = MODE == kModeGateUp ? ntile * 128 : ntile * kBN;
  const uint8_t* wexp = a.w + (int64_t)e * a.N * a.K;
  const float* wsexp = a.ws + (int64_t)e * NB * KB;

  // global -> register staging of one K block: 2 A chunks, 8 B chunks, 1 scale
  int64_t a_src[2];
  bool a_ok[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int q = tid + 256 * i, r = row0 + (q >> 3);
    a_ok[i] = r < row_end;
    int64_t src = 0;
    if (a_ok[i]) src = a.rows ? (int64_t)(a.rows[r] / a.topk) : (int64_t)r;
    a_src[i] = src * a.K + (q & 7) * 16;
  }
  int64_t s_src = -1;
  if (tid < kBM && row0 + tid < row_end)
    s_src = (a.rows ? (int64_t)(a.rows[row0 + tid] / a.topk) : (int64_t)(row0 + tid)) * KB;
  int64_t b_src[8];
  bool b_ok[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int q = tid + 256 * i, j = q >> 3;
    const int wrow = MODE == kModeGateUp ? (j < 128 ? n0 + j : a.I + n0 + (j - 128)) : n0 + j;
    b_ok[i] = wrow < a.N;
    b_src[i] = (int64_t)(b_ok[i] ? wrow : 0) * a.K + (q & 7) * 16;
  }
  i32x4 ra[2], rb[8];
  float rs = 0.0f;
  auto gload = [&](int kb) {
    const int64_t ko = (int64_t)kb * kBK;
#pragma unroll
    for (int i = 0; i < 2; ++i) ra[i] = a_ok[i] ? *(const i32x4*)(a.a + a_src[i] + ko) : i32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; ++i) rb[i] = b_ok[i] ? *(const i32x4*)(wexp + b_src[i] + ko) : i32x4{0, 0, 0, 0};
    rs = s_src >= 0 ? a.as[s_src + kb] : 0.0f;
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int q = tid + 256 * i;
      *(i32x4*)(&sA[tswz(q >> 3, q & 7)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int q = tid + 256 * i;
      *(i32x4*)(&sB[tswz(q >> 3, q & 7)]) = rb[i];
    }
    if (tid < kBM) sS[tid] = rs;
  };

  // this wave's four 16-column blocks of the tile's 256 weight rows
  int cbr[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    cbr[c] = MODE == kModeGateUp ? (c < 2 ? 32 * wave + 16 * c : 128 + 32 * wave + 16 * (c - 2))
                                 : 64 * wave + 16 * c;
  // their weight scale blocks (row block of weight row n0 + cbr[c])
  int cnb[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const int j = cbr[c];
    const int wrow = MODE == kModeGateUp ? (j < 128 ? n0 + j : a.I + n0 + (j - 128)) : n0 + j;
    cnb[c] = min(wrow, a.N - 1) / 128;
  }

  f32x4 acc[4][4];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, kc = (lane >> 4) * 2;  // operand row and 16-byte chunk pair
  gload(0);
  sstore();
  __syncthreads();
  for (int kb = 0; kb < KB; ++kb) {
    if (kb + 1 < KB) gload(kb + 1);
    float sw[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) sw[c] = wsexp[cnb[c] * KB + kb];
    i32x8 B[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int row = cbr[c] + lr;
      const i32x4 lo = *(const i32x4*)(&sB[tswz(row, kc)]);
      const i32x4 hi = *(const i32x4*)(&sB[tswz(row, kc + 1)]);
      B[c] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int row = 16 * r + lr;
      const i32x4 lo = *(const i32x4*)(&sA[tswz(row, kc)]);
      const i32x4 hi = *(const i32x4*)(&sA[tswz(row, kc + 1)]);
      const i32x8 A = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      // activation scales of the four output rows this lane holds
      const f32x4 sx = *(const f32x4*)(&sS[16 * r + 4 * (lane >> 4)]);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 blk = mfma_fp8(A, B[c], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[r][c][q] = fmaf(blk[q], sx[q] * sw[c], acc[r][c][q]);
      }
    }
    if (kb + 1 < KB) {
      __syncthreads();  // every wave is done reading this stage
      sstore();
    }
    __syncthreads();
  }

  if constexpr (MODE == kModeGateUp) {
    // SwiGLU in the activation dtype (out_dtype), then 1x128 e4m3 quantization of
    // the tile's finished 128 activation columns
    float act[4][2][4];
    float rmax[4][4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int q = 0; q < 4; ++q) rmax[r][q] = 0.0f;
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float gb = round_act(acc[r][g][q], a.out_dtype);
          const float ub = round_act(acc[r][2 + g][q], a.out_dtype);
          const float sl = round_act(gb / (1.0f + expf(-gb)), a.out_dtype);
          const float av = round_act(sl * ub, a.out_dtype);
          act[r][g][q] = av;
          rmax[r][q] = fmaxf(rmax[r][q], fabsf(av));
        }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) rmax[r][q] = fmaxf(rmax[r][q], __shfl_xor(rmax[r][q], off, 64));
      if (lr == 0)
#pragma unroll
        for (int q = 0; q < 4; ++q) sRed[wave][16 * r + 4 * (lane >> 4) + q] = rmax[r][q];
    }
    __syncthreads();
    const int IB = a.I / 128;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lrow = 16 * r + 4 * (lane >> 4) + q;
        const int grow = row0 + lrow;
        if (grow >= row_end) continue;
        const float amax = fmaxf(fmaxf(sRed[0][lrow], sRed[1][lrow]), fmaxf(sRed[2][lrow], sRed[3][lrow]));
        const float s = __fdiv_rn(fmaxf(amax, 1e-12f), 448.0f);
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          float v = __fdiv_rn(act[r][g][q], s);
          v = v < -448.0f ? -448.0f : (v > 448.0f ? 448.0f : v);
          a.actq[(int64_t)grow * a.I + n0 + 32 * wave + 16 * g + lr] = (uint8_t)f32_to_e4m3(v);
        }
        if (wave == 0 && lr == 0) a.acts[(int64_t)grow * IB + n0 / 128] = s;
      }
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int n = n0 + cbr[c] + lr;
        if (n >= a.N) continue;
        const float bv = a.bias_dtype != KQ_DTYPE_NONE ? load_as_f32(a.bias, a.bias_dtype, n) : 0.0f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int grow = row0 + 16 * r + 4 * (lane >> 4) + q;
          if (grow >= row_end) continue;
          float v = acc[r][c][q];
          if (a.bias_dtype != KQ_DTYPE_NONE) v = __fadd_rn(v, bv);
          ((uint16_t*)a.out)[(int64_t)grow * a.N + n] = f32_to_out(v, a.out_dtype);
        }
      }
  }
}

// ------------------------------------------------------------------ combine
// out[t] = sum over slots s (in order) of fp32(y[inv[t*k+s]]) * w[t*k+s].
__global__ void __launch_bounds__(256)
moe_combine_kernel(const uint16_t* __restrict__ y, int y_dtype, const int32_t* __restrict__ inv,
                   const float* __restrict__ w, int k, int H, uint16_t* __restrict__ out) {
  const int64_t t = blockIdx.x;
  for (int h = threadIdx.x * 8; h < H; h += 256 * 8) {
    float acc[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[e] = 0.0f;
    for (int s = 0; s < k; ++s) {
      const int pos = inv[t * k + s];
      const float wv = w[t * k + s];
      if (pos < 0) continue;
      const uint16_t* yr = y + (int64_t)pos * H + h;
      float yv[8];
      if (h + 8 <= H) {
        const u32x4 raw = *(const u32x4*)yr;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          yv[2 * d] = y_dtype == KQ_DTYPE_BF16 ? bf16_to_f32(raw[d] & 0xffffu) : f16_to_f32(raw[d] & 0xffffu);
          yv[2 * d + 1] = y_dtype == KQ_DTYPE_BF16 ? bf16_to_f32(raw[d] >> 16) : f16_to_f32(raw[d] >> 16);
        }
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          yv[e] = h + e < H ? (y_dtype == KQ_DTYPE_BF16 ? bf16_to_f32(yr[e]) : f16_to_f32(yr[e])) : 0.0f;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = __fadd_rn(acc[e], __fmul_rn(yv[e], wv));
    }
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (h + e < H) out[t * H + h + e] = f32_to_out(acc[e], y_dtype);
  }
}

// ------------------------------------------------------------------- host
struct MoeWorkspace {
  size_t counts, base, offsets, tiles, sorted, inv, xq, xs, actq, acts, y, total;
};

static size_t align256(size_t v) { return (v + 255) / 256 * 256; }

static MoeWorkspace moe_layout(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k) {
  const int64_t R = T * k;
  const int64_t C = (R + kSortChunk - 1) / kSortChunk;
  const int64_t max_tiles = (R + kBM - 1) / kBM + E;
  MoeWorkspace w{};
  size_t p = 0;
  auto take = [&](size_t bytes) { const size_t at = p; p += align256(bytes); return at; };
  w.counts = take((size_t)C * E * 4);
  w.base = take((size_t)C * E * 4);
  w.offsets = take((size_t)(E + 1) * 4);
  w.tiles = take((size_t)max_tiles * 8);
  w.sorted = take((size_t)R * 4);
  w.inv = take((size_t)R * 4);
  w.xq = take((size_t)T * H);
  w.xs = take((size_t)T * (H / 128) * 4);
  w.actq = take((size_t)R * I);
  w.acts = take((size_t)R * (I / 128) * 4);
  w.y = take((size_t)R * H * 2);
  w.total = p;
  return w;
}

static bool quant_dtype_ok(int d) { return d == KQ_DTYPE_F16 || d == KQ_DTYPE_BF16; }

static void launch_act_quant_blocks(const void* x, int dtype, int64_t rows, int64_t K, int64_t ldx,
                                    uint8_t* xq, float* xs, hipStream_t st) {
  const bool vec = ((uintptr_t)x % 16) == 0 && (ldx % 8) == 0;
  const dim3 grid((unsigned)rows, (unsigned)((K + 2047) / 2048));
  hipLaunchKernelGGL(act_quant_fp8_blocks_kernel, grid, dim3(256), 0, st, (const uint16_t*)x, dtype,
                     (int)K, ldx, vec, xq, xs);
}

}  // namespace kq

using namespace kq;

extern "C" int kq_moe_route_topk(const void* logits, int dtype, int64_t tokens, int64_t experts,
                                 int top_k, int norm_topk_prob, int32_t* topk_idx, float* topk_w,
                                 void* stream) {
  if (dtype != KQ_DTYPE_F16 && dtype != KQ_DTYPE_BF16 && dtype != KQ_DTYPE_F32) {
    set_error("kq_moe_route_topk: logits must be fp16, bf16 or fp32");
    return KQ_EUNSUPPORTED;
  }
  if (tokens < 0 || experts < 1 || experts > 64 * kRouteMaxPerLane || top_k < 1 ||
      top_k > kRouteMaxTopK || top_k > experts || tokens > 0x7fffffffLL / 64) {
    set_error("kq_moe_route_topk: bad shape tokens=%lld experts=%lld top_k=%d", (long long)tokens,
              (long long)experts, top_k);
    return KQ_EINVAL;
  }
  if (tokens == 0) return KQ_OK;
  hipLaunchKernelGGL(moe_route_kernel, dim3((unsigned)((tokens + 3) / 4)), dim3(256), 0,
                     (hipStream_t)stream, logits, dtype, (int)tokens, (int)experts, top_k,
                     norm_topk_prob ? 1 : 0, topk_idx, topk_w);
  return check_launch("kq_moe_route_topk");
}

extern "C" int kq_act_quant_fp8_blocks(const void* x, int x_dtype, int64_t rows, int64_t k,
                                       int64_t ldx, uint8_t* xq, float* xs, void* stream) {
  if (!quant_dtype_ok(x_dtype)) {
    set_error("kq_act_quant_fp8_blocks: activation dtype must be fp16 or bf16");
    return KQ_EUNSUPPORTED;
  }
  if (rows < 0 || k < 1 || ldx < k || rows > 0x7fffffffLL || k > 0x7fffffffLL) {
    set_error("kq_act_quant_fp8_blocks: bad shape rows=%lld k=%lld", (long long)rows, (long long)k);
    return KQ_EINVAL;
  }
  if (rows == 0) return KQ_OK;
  launch_act_quant_blocks(x, x_dtype, rows, k, ldx, xq, xs, (hipStream_t)stream);
  return check_launch("kq_act_quant_fp8_blocks");
}

extern "C" int kq_block_fp8_gemm(const uint8_t* xq, const float* xs, const uint8_t* w,
                                 const float* ws, const void* bias, int bias_dtype, void* out,
                                 int out_dtype, int64_t m, int64_t n, int64_t k, void* stream) {
  if (!quant_dtype_ok(out_dtype)) {
    set_error("kq_block_fp8_gemm: output dtype must be fp16 or bf16");
    return KQ_EUNSUPPORTED;
  }
  if (m < 0 || n < 1 || k < kBK || (k % kBK) != 0 || m > 0x7fffffffLL || n > 0x7fffffffLL ||
      k > 0x7fffffffLL) {
    set_error("kq_block_fp8_gemm: bad shape m=%lld n=%lld k=%lld (k must be a multiple of 128)",
              (long long)m, (long long)n, (long long)k);
    return KQ_EINVAL;
  }
  if (m == 0) return KQ_OK;
  MoeGemmArgs a{};
  a.a = xq; a.as = xs; a.rows = nullptr; a.topk = 1;
  a.w = w; a.ws = ws; a.tiles = nullptr; a.offsets = nullptr;
  a.M = (int)m; a.N = (int)n; a.K = (int)k; a.I = 0;
  a.mtiles = (int)((m + kBM - 1) / kBM);
  a.ntiles = (int)((n + kBN - 1) / kBN);
  a.out = out; a.out_dtype = out_dtype; a.bias = bias; a.bias_dtype = bias_dtype;
  hipLaunchKernelGGL(moe_gemm_kernel<kModeDown>, dim3((unsigned)(a.mtiles * a.ntiles)), dim3(256), 0,
                     (hipStream_t)stream, a);
  return check_launch("kq_block_fp8_gemm");
}

extern "C" size_t kq_moe_workspace_size(int64_t tokens, int64_t hidden, int64_t inter,
                                        int64_t experts, int top_k) {
  if (tokens < 1 || hidden < 1 || inter < 1 || experts < 1 || top_k < 1) return 0;
  return moe_layout(tokens, hidden, inter, experts, top_k).total;
}

extern "C" int kq_moe_block_fp8_experts(const void* hidden, int dtype, int64_t tokens,
                                        int64_t hidden_size, int64_t inter, int64_t experts,
                                        int top_k, const int32_t* topk_idx, const float* topk_w,
                                        const uint8_t* w13, const float* s13, const uint8_t* w2,
                                        const float* s2, void* out, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  if (!quant_dtype_ok(dtype)) {
    set_error("kq_moe_block_fp8_experts: hidden dtype must be fp16 or bf16");
    return KQ_EUNSUPPORTED;
  }
  if (tokens < 0 || hidden_size < kBK || (hidden_size % kBK) != 0 || inter < kBK ||
      (inter % kBK) != 0 || experts < 1 || experts > 1024 || top_k < 1 || top_k > experts ||
      tokens * top_k > 0x7fffffffLL || hidden_size * 2 * inter > 0x7fffffffLL) {
    set_error("kq_moe_block_fp8_experts: bad shape tokens=%lld hidden=%lld inter=%lld experts=%lld "
              "top_k=%d (hidden and inter must be multiples of 128)",
              (long long)tokens, (long long)hidden_size, (long long)inter, (long long)experts, top_k);
    return KQ_EINVAL;
  }
  if (tokens == 0) return KQ_OK;
  const MoeWorkspace L = moe_layout(tokens, hidden_size, inter, experts, top_k);
  if (workspace == nullptr || workspace_bytes < L.total) {
    set_error("kq_moe_block_fp8_experts: workspace of %zu bytes is smaller than the %zu bytes "
              "this call needs", workspace ? workspace_bytes : (size_t)0, L.total);
    return KQ_EWORKSPACE;
  }
  hipStream_t st = (hipStream_t)stream;
  uint8_t* ws = (uint8_t*)workspace;
  int32_t* counts = (int32_t*)(ws + L.counts);
  int32_t* base = (int32_t*)(ws + L.base);
  int32_t* offsets = (int32_t*)(ws + L.offsets);
  int32_t* tiles = (int32_t*)(ws + L.tiles);
  int32_t* sorted = (int32_t*)(ws + L.sorted);
  int32_t* inv = (int32_t*)(ws + L.inv);
  uint8_t* xq = ws + L.xq;
  float* xs = (float*)(ws + L.xs);
  uint8_t* actq = ws + L.actq;
  float* acts = (float*)(ws + L.acts);
  uint16_t* y = (uint16_t*)(ws + L.y);
  const int R = (int)(tokens * top_k);
  const int C = (R + kSortChunk - 1) / kSortChunk;
  const int E = (int)experts;
  const int max_tiles = (R + kBM - 1) / kBM + E;

  hipLaunchKernelGGL(moe_count_kernel, dim3(C), dim3(256), E * sizeof(int), st, topk_idx, R, E, counts);
  hipLaunchKernelGGL(moe_scan_kernel, dim3(1), dim3(1024), 0, st, counts, C, E, kBM, max_tiles, offsets,
                     base, tiles);
  hipLaunchKernelGGL(moe_scatter_kernel, dim3(C), dim3(64), E * sizeof(int), st, topk_idx, R, E, base,
                     sorted, inv);
  launch_act_quant_blocks(hidden, dtype, tokens, hidden_size, hidden_size, xq, xs, st);

  MoeGemmArgs g{};
  g.a = xq; g.as = xs; g.rows = sorted; g.topk = top_k;
  g.w = w13; g.ws = s13; g.tiles = tiles; g.offsets = offsets;
  g.N = (int)(2 * inter); g.K = (int)hidden_size; g.I = (int)inter;
  g.mtiles = max_tiles; g.ntiles = (int)(inter / 128);
  g.actq = actq; g.acts = acts; g.out_dtype = dtype;
  hipLaunchKernelGGL(moe_gemm_kernel<kModeGateUp>, dim3((unsigned)(g.mtiles * g.ntiles)), dim3(256), 0,
                     st, g);

  MoeGemmArgs d{};
  d.a = actq; d.as = acts; d.rows = nullptr; d.topk = 1;
  d.w = w2; d.ws = s2; d.tiles = tiles; d.offsets = offsets;
  d.N = (int)hidden_size; d.K = (int)inter; d.I = 0;
  d.mtiles = max_tiles; d.ntiles = (int)((hidden_size + kBN - 1) / kBN);
  d.out = y; d.out_dtype = dtype; d.bias = nullptr; d.bias_dtype = KQ_DTYPE_NONE;
  hipLaunchKernelGGL(moe_gemm_kernel<kModeDown>, dim3((unsigned)(d.mtiles * d.ntiles)), dim3(256), 0,
                     st, d);

  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)tokens), dim3(256), 0, st, y, dtype, inv, topk_w,
                     top_k, (int)hidden_size, (uint16_t*)out);
  return check_launch("kq_moe_block_fp8_experts");
}
