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
constexpr int kSortChunk = 256;   // rows per chunk = threads per sort workgroup

// Per-chunk expert histogram: counts[c][e].
__global__ void __launch_bounds__(kSortChunk)
moe_count_kernel(const int32_t* __restrict__ idx, int R, int E, int32_t* __restrict__ counts) {
  extern __shared__ int hist[];
  for (int i = threadIdx.x; i < E; i += kSortChunk) hist[i] = 0;
  __syncthreads();
  const int r = blockIdx.x * kSortChunk + threadIdx.x;
  if (r < R) {
    const int e = idx[r];
    if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < E; i += kSortChunk) counts[(int64_t)blockIdx.x * E + i] = hist[i];
}

// Exclusive prefix sum of v[0..n) in LDS (n <= 1024, 1024 threads); returns the total.
KQ_DEV int block_exclusive_scan(int* v, int* tmp, int n) {
  const int t = threadIdx.x;
  int x = t < n ? v[t] : 0;
  tmp[t] = x;
  __syncthreads();
  for (int off = 1; off < 1024; off <<= 1) {
    const int y = t >= off ? tmp[t - off] : 0;
    __syncthreads();
    tmp[t] += y;
    __syncthreads();
  }
  const int total = tmp[1023];
  if (t < n) v[t] = tmp[t] - x;
  __syncthreads();
  return total;
}

// One 1024-thread workgroup: column-wise exclusive scan of counts[C][E] into
// base[c][e] (sorted position of chunk c's first row of expert e), expert
// offsets, and the M-tile table (tile i -> (expert, first row); unused
// entries get expert -1).  Thread (slice, e) scans a contiguous run of chunks.
__global__ void __launch_bounds__(1024)
moe_scan_kernel(const int32_t* __restrict__ counts, int C, int E, int BM, int max_tiles,
                int32_t* __restrict__ offsets, int32_t* __restrict__ base, int32_t* __restrict__ tiles) {
  __shared__ int part[1024], tot[1024], ntile[1024], tmp[1024];
  const int t = threadIdx.x;
  int slices = 1;
  while (slices * 2 * E <= 1024) slices *= 2;
  const int per = (C + slices - 1) / slices;
  const int e = t % E, sl = t / E;
  const bool active = sl < slices;
  const int c0 = active ? sl * per : 0, c1 = active ? min(C, c0 + per) : 0;
  int sum = 0;
  for (int c = c0; c < c1; ++c) sum += counts[(int64_t)c * E + e];
  part[t] = sum;
  __syncthreads();
  if (t < E) {
    int run = 0;
    for (int q = 0; q < slices; ++q) {
      const int v = part[q * E + t];
      part[q * E + t] = run;   // slice start within the expert
      run += v;
    }
    tot[t] = run;
    ntile[t] = (run + BM - 1) / BM;
  }
  __syncthreads();
  const int total_rows = block_exclusive_scan(tot, tmp, E);     // tot -> expert offsets
  const int total_tiles = block_exclusive_scan(ntile, tmp, E);  // ntile -> first tile
  (void)total_rows;
  if (active) {
    int run = tot[e] + part[t];
    for (int c = c0; c < c1; ++c) {
      base[(int64_t)c * E + e] = run;
      run += counts[(int64_t)c * E + e];
    }
  }
  if (t < E) {
    offsets[t] = tot[t];
    if (t == E - 1) offsets[E] = total_rows;
    const int rows = (t == E - 1 ? total_rows : tot[t + 1]) - tot[t];
    const int nt = (rows + BM - 1) / BM;
    for (int i = 0; i < nt && ntile[t] + i < max_tiles; ++i) {
      tiles[2 * (ntile[t] + i)] = t;
      tiles[2 * (ntile[t] + i) + 1] = tot[t] + i * BM;
    }
  }
  for (int i = total_tiles + t; i < max_tiles; i += 1024) {
    tiles[2 * i] = -1;
    tiles[2 * i + 1] = 0;
  }
}

// Sorted position of row r = base[chunk][e] + its rank among the chunk's
// earlier rows routed to the same expert (stable).
__global__ void __launch_bounds__(kSortChunk)
moe_scatter_kernel(const int32_t* __restrict__ idx, int R, int E, const int32_t* __restrict__ base,
                   int32_t* __restrict__ sorted_rows, int32_t* __restrict__ inv) {
  __shared__ int ids[kSortChunk];
  const int c = blockIdx.x, t = threadIdx.x;
  const int r = c * kSortChunk + t;
  const int e = r < R ? idx[r] : -1;
  ids[t] = e;
  __syncthreads();
  if (r >= R) return;
  if (e < 0 || e >= E) {
    inv[r] = -1;
    return;
  }
  int rank = 0;
  for (int j = 0; j < t; ++j) rank += ids[j] == e ? 1 : 0;
  const int pos = base[(int64_t)c * E + e] + rank;
  sorted_rows[pos] = r;
  inv[r] = pos;
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
// A tile is up to 256 rows of one expert x 256 weight rows; eight waves in a
// 2 (row halves of 128) x 4 (column quarters of 64) grid.  Each wave keeps its
// four B operands of a K block in registers while its eight 16-row A blocks
// stream from LDS (~24 KB of LDS reads per wave per K block).  A, B and the
// activation scales move global -> LDS with buffer_load ... lds (no register
// staging), double-buffered: K block kb+1 is in flight while kb is
// multiplied.  The loop is unrolled by two so the two LDS stages are distinct
// arrays and reads of one stage never wait for the other stage's loads.
// Tiles of one expert and column range are adjacent and land on one XCD, so
// a second row chunk of an expert finds the weights in that XCD's L2.
constexpr int kBM = 256;    // rows per tile
constexpr int kBN = 256;    // weight rows per tile
constexpr int kBK = 128;    // one scale block of K per step
constexpr int kGemmThreads = 512;
constexpr int32_t kOob = (int32_t)0x80000000u;  // buffer offset past every resource: reads 0
enum { kModeGateUp = 0, kModeDown = 1 };

struct MoeGemmArgs {
  const uint8_t* a;        // e4m3 activation rows of length K
  const float* as;         // activation block scales [rows][K/128]
  int a_rows;              // rows of a / as (resource bounds)
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

// Global -> LDS copy of 16 (or 4) bytes per lane with buffer_load ... lds:
// lane i writes at LDS byte lds + i * size.  Written as inline asm so the
// compiler does not make every later LDS read wait for it (it cannot tell the
// two stages apart); the kernel waits with s_waitcnt + s_barrier before it
// reads a stage.  M0 carries the wave-uniform LDS address.
KQ_DEV void dma_lds16(i32x4 rsrc, uint32_t lds, int32_t voff, int32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
               ::"s"(lds), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
}
KQ_DEV void dma_lds4(i32x4 rsrc, uint32_t lds, int32_t voff, int32_t soff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
               ::"s"(lds), "v"(voff), "s"(rsrc), "s"(soff) : "memory", "m0");
}

// LDS map: two A stages, two B stages, two scale stages.
constexpr int kMaxKB = 128;   // K <= 16384
constexpr int kLdsA = 0, kLdsB = 2 * kBM * kBK, kLdsS = kLdsB + 2 * kBN * kBK;
constexpr int kLdsW = kLdsS + 2 * kBM * 4;            // the tile's two weight-scale rows
constexpr int kLdsBytes = kLdsW + 2 * kMaxKB * 4;

template <int MODE>
__global__ void __launch_bounds__(kGemmThreads)
moe_gemm_kernel(MoeGemmArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[kLdsBytes];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int wr = wave >> 2, wc = wave & 3;
  const int nblk = a.mtiles * a.ntiles;
  const int L = xcd_swizzle(blockIdx.x, nblk);
  const int ntile = L / a.mtiles, mtile = L % a.mtiles;
  int e, row0, row_end;
  if (a.tiles) {
    e = a.tiles[2 * mtile];
    if (e < 0) return;
    row0 = a.tiles[2 * mtile + 1];
    row_end = min(a.offsets[e + 1], row0 + kBM);
  } else {
    e = 0;
    row0 = mtile * kBM;
    row_end = min(a.M, row0 + kBM);
  }
  const int KB = a.K / kBK;
  const int NB = (a.N + 127) / 128;
  const int n0 = MODE == kModeGateUp ? ntile * 128 : ntile * kBN;
  const i32x4 ra = make_rsrc(a.a, (uint32_t)((uint64_t)a.a_rows * a.K));
  const i32x4 rsc = make_rsrc(a.as, (uint32_t)((uint64_t)a.a_rows * KB * 4));
  const i32x4 rw = make_rsrc(a.w + (int64_t)e * a.N * a.K, (uint32_t)((uint64_t)a.N * a.K));
  const float* wsexp = a.ws + (int64_t)e * NB * KB;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;

  // lane offsets of this wave's four 1 KB DMA blocks of the A and B stages:
  // LDS slot p = block*64 + lane holds chunk c = (p & 7) ^ (row & 7) of row p / 8
  int32_t a_off[4], b_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int p = (wave * 4 + i) * 64 + lane, row = p >> 3, c = (p & 7) ^ (row & 7);
    const int r = row0 + row;
    a_off[i] = kOob;
    if (r < row_end) {
      const int src = a.rows ? a.rows[r] / a.topk : r;
      a_off[i] = src * a.K + c * 16;
    }
    const int wrow = MODE == kModeGateUp ? (row < 128 ? n0 + row : a.I + n0 + (row - 128)) : n0 + row;
    b_off[i] = wrow < a.N ? wrow * a.K + c * 16 : kOob;
  }
  int32_t s_off = kOob;  // waves 0-3 fetch the 256 activation scales
  if (wave < 4) {
    const int r = row0 + wave * 64 + lane;
    if (r < row_end) s_off = (a.rows ? a.rows[r] / a.topk : r) * KB * 4;
  }
  auto issue = [&](int kb, int st) {
    const uint32_t la = lds0 + kLdsA + st * (kBM * kBK) + wave * 4096;
    const uint32_t lb = lds0 + kLdsB + st * (kBN * kBK) + wave * 4096;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dma_lds16(ra, la + i * 1024, a_off[i], kb * kBK);
      dma_lds16(rw, lb + i * 1024, b_off[i], kb * kBK);
    }
    if (wave < 4) dma_lds4(rsc, lds0 + kLdsS + st * (kBM * 4) + wave * 256, s_off, kb * 4);
  };

  // this wave's four 16-column blocks of the tile's 256 weight rows
  int cbr[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
    cbr[c] = MODE == kModeGateUp ? (c < 2 ? 32 * wc + 16 * c : 128 + 32 * wc + 16 * (c - 2))
                                 : 64 * wc + 16 * c;
  // the tile's weight rows span two 128-row scale blocks (gate_up: the gate
  // block and the up block; down: n0/128 and the next); stage both scale rows
  // for every K block in LDS before the loop
  float* sWs = (float*)(smem + kLdsW);
  {
    const int nb0 = (MODE == kModeGateUp ? n0 : n0) / 128;
    const int nb1 = MODE == kModeGateUp ? (a.I + n0) / 128 : min(n0 / 128 + 1, NB - 1);
    for (int t = threadIdx.x; t < 2 * KB; t += kGemmThreads)
      sWs[t] = wsexp[(t < KB ? nb0 : nb1) * KB + (t % KB)];
  }
  int cslot[4];  // which staged scale row each of the wave's column blocks uses
#pragma unroll
  for (int c = 0; c < 4; ++c) cslot[c] = MODE == kModeGateUp ? (c < 2 ? 0 : 1) : (wc >> 1);

  f32x4 acc[8][4];
#pragma unroll
  for (int r = 0; r < 8; ++r)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[r][c] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, kc = (lane >> 4) * 2;  // operand row and 16-byte chunk pair
  const int rbase = 128 * wr;
  // rows 16*r + lr share (row & 7), so one swizzled offset serves all blocks
  const int a_lo = tswz(rbase + lr, kc), a_hi = tswz(rbase + lr, kc + 1);
  const int b_lo = tswz(lr, kc), b_hi = tswz(lr, kc + 1);

  issue(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int kb = 0; kb < KB; ++kb) {
    const int st = kb & 1;
    if (kb + 1 < KB) issue(kb + 1, st ^ 1);
    const uint8_t* sA = smem + kLdsA + st * (kBM * kBK);
    const uint8_t* sB = smem + kLdsB + st * (kBN * kBK);
    const float* sS = (const float*)(smem + kLdsS + st * (kBM * 4));
    float sw[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) sw[c] = sWs[cslot[c] * KB + kb];
    i32x8 B[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const i32x4 lo = *(const i32x4*)(sB + cbr[c] * 128 + b_lo);
      const i32x4 hi = *(const i32x4*)(sB + cbr[c] * 128 + b_hi);
      B[c] = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const i32x4 lo = *(const i32x4*)(sA + r * 2048 + a_lo);
      const i32x4 hi = *(const i32x4*)(sA + r * 2048 + a_hi);
      const i32x8 A = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      // activation scales of the four output rows this lane holds
      const f32x4 sx = *(const f32x4*)(&sS[rbase + 16 * r + 4 * (lane >> 4)]);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const f32x4 blk = mfma_fp8(A, B[c], f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
        for (int q = 0; q < 4; ++q) acc[r][c][q] = fmaf(blk[q], sx[q] * sw[c], acc[r][c][q]);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of stage kb+1 have landed
    __syncthreads();                 // ... and everyone's; stage kb is free again
  }

  if constexpr (MODE == kModeGateUp) {
    // SwiGLU in the activation dtype (out_dtype), then 1x128 e4m3 quantization
    // of the tile's finished 128 activation columns; act overwrites acc[r][0..1]
    float (*sRed)[kBM] = (float (*)[kBM])smem;  // stages are free after the loop
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      float rmax[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float gb = round_act(acc[r][g][q], a.out_dtype);
          const float ub = round_act(acc[r][2 + g][q], a.out_dtype);
          const float sl = round_act(gb / (1.0f + expf(-gb)), a.out_dtype);
          const float av = round_act(sl * ub, a.out_dtype);
          acc[r][g][q] = av;
          rmax[q] = fmaxf(rmax[q], fabsf(av));
        }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int off = 8; off > 0; off >>= 1) rmax[q] = fmaxf(rmax[q], __shfl_xor(rmax[q], off, 64));
      if (lr == 0)
#pragma unroll
        for (int q = 0; q < 4; ++q) sRed[wc][rbase + 16 * r + 4 * (lane >> 4) + q] = rmax[q];
    }
    __syncthreads();
    const int IB = a.I / 128;
#pragma unroll
    for (int r = 0; r < 8; ++r)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int lrow = rbase + 16 * r + 4 * (lane >> 4) + q;
        const int grow = row0 + lrow;
        if (grow >= row_end) continue;
        const float amax = fmaxf(fmaxf(sRed[0][lrow], sRed[1][lrow]), fmaxf(sRed[2][lrow], sRed[3][lrow]));
        const float s = __fdiv_rn(fmaxf(amax, 1e-12f), 448.0f);
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          float v = __fdiv_rn(acc[r][g][q], s);
          v = v < -448.0f ? -448.0f : (v > 448.0f ? 448.0f : v);
          a.actq[(int64_t)grow * a.I + n0 + 32 * wc + 16 * g + lr] = (uint8_t)f32_to_e4m3(v);
        }
        if (wc == 0 && lr == 0) a.acts[(int64_t)grow * IB + n0 / 128] = s;
      }
  } else {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const int n = n0 + cbr[c] + lr;
      if (n >= a.N) continue;
      const float bv = a.bias_dtype != KQ_DTYPE_NONE ? load_as_f32(a.bias, a.bias_dtype, n) : 0.0f;
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int grow = row0 + rbase + 16 * r + 4 * (lane >> 4) + q;
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
  if (m < 0 || n < 1 || k < kBK || (k % kBK) != 0 || k > kBK * kMaxKB || m > 0x7fffffffLL ||
      n > 0x7fffffffLL || n * k > 0x7fffffffLL) {
    set_error("kq_block_fp8_gemm: bad shape m=%lld n=%lld k=%lld (k must be a multiple of 128)",
              (long long)m, (long long)n, (long long)k);
    return KQ_EINVAL;
  }
  if (m == 0) return KQ_OK;
  MoeGemmArgs a{};
  a.a = xq; a.as = xs; a.a_rows = (int)m; a.rows = nullptr; a.topk = 1;
  a.w = w; a.ws = ws; a.tiles = nullptr; a.offsets = nullptr;
  a.M = (int)m; a.N = (int)n; a.K = (int)k; a.I = 0;
  a.mtiles = (int)((m + kBM - 1) / kBM);
  a.ntiles = (int)((n + kBN - 1) / kBN);
  a.out = out; a.out_dtype = out_dtype; a.bias = bias; a.bias_dtype = bias_dtype;
  hipLaunchKernelGGL(moe_gemm_kernel<kModeDown>, dim3((unsigned)(a.mtiles * a.ntiles)), dim3(kGemmThreads), 0,
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
      hidden_size > kBK * kMaxKB || inter > kBK * kMaxKB || tokens * top_k > 0x7fffffffLL ||
      hidden_size * 2 * inter > 0x7fffffffLL || tokens * hidden_size > 0x7fffffffLL ||
      tokens * top_k * inter > 0x7fffffffLL) {
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

  hipLaunchKernelGGL(moe_count_kernel, dim3(C), dim3(kSortChunk), E * sizeof(int), st, topk_idx, R, E,
                     counts);
  hipLaunchKernelGGL(moe_scan_kernel, dim3(1), dim3(1024), 0, st, counts, C, E, kBM, max_tiles, offsets,
                     base, tiles);
  hipLaunchKernelGGL(moe_scatter_kernel, dim3(C), dim3(kSortChunk), 0, st, topk_idx, R, E, base, sorted,
                     inv);
  launch_act_quant_blocks(hidden, dtype, tokens, hidden_size, hidden_size, xq, xs, st);

  MoeGemmArgs g{};
  g.a = xq; g.as = xs; g.a_rows = (int)tokens; g.rows = sorted; g.topk = top_k;
  g.w = w13; g.ws = s13; g.tiles = tiles; g.offsets = offsets;
  g.N = (int)(2 * inter); g.K = (int)hidden_size; g.I = (int)inter;
  g.mtiles = max_tiles; g.ntiles = (int)(inter / 128);
  g.actq = actq; g.acts = acts; g.out_dtype = dtype;
  hipLaunchKernelGGL(moe_gemm_kernel<kModeGateUp>, dim3((unsigned)(g.mtiles * g.ntiles)), dim3(kGemmThreads), 0,
                     st, g);

  MoeGemmArgs d{};
  d.a = actq; d.as = acts; d.a_rows = R; d.rows = nullptr; d.topk = 1;
  d.w = w2; d.ws = s2; d.tiles = tiles; d.offsets = offsets;
  d.N = (int)hidden_size; d.K = (int)inter; d.I = 0;
  d.mtiles = max_tiles; d.ntiles = (int)((hidden_size + kBN - 1) / kBN);
  d.out = y; d.out_dtype = dtype; d.bias = nullptr; d.bias_dtype = KQ_DTYPE_NONE;
  hipLaunchKernelGGL(moe_gemm_kernel<kModeDown>, dim3((unsigned)(d.mtiles * d.ntiles)), dim3(kGemmThreads), 0,
                     st, d);

  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)tokens), dim3(256), 0, st, y, dtype, inv, topk_w,
                     top_k, (int)hidden_size, (uint16_t*)out);
  return check_launch("kq_moe_block_fp8_experts");
}
