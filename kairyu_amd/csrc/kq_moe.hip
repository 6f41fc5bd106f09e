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
//   3. grouped GEMM 1 (gate_up), kq_tile_gemm.h: activation rows gathered
//      through the sorted order, weights = the expert's stacked [gate; up].
//      A 320 x 256 or 256 x 256 tile (rows of one expert; moe_nrb picks the
//      height) pairs gate columns [n0, n0+128) with up columns
//      [I+n0, I+n0+128), so the epilogue forms the SwiGLU in the activation
//      dtype and quantizes the finished 128-column block to e4m3 in registers
//      (no bf16 intermediate in HBM).
//   4. grouped GEMM 2 (down): the same row tiles x 256 -> expert outputs
//      (bf16/fp16).
//   5. combine: fp32 slot-order weighted sum per token.
// Both GEMMs use v_mfma_scale_f32_16x16x128_f8f6f4 (unit E8M0 scales): one
// MFMA spans one 128-wide K block, and its fp32 result is scaled by
// s_act[row][kb] * s_w[nb][kb] before it is added to the accumulator.
#include "kq_common.h"
#include "kq_tile_gemm.h"

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


KQ_DEV float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

KQ_DEV float key_float(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// One wave routes TW tokens at once (their selection chains interleave):
// per token, k rounds of a wave-wide max of the value keys, ties to the
// smallest expert (a ballot of the lanes holding the maximum); every lane
// sees each round's winner, lane r keeps slot r's logit.  v[j][i] holds token
// t[j]'s logit of expert lane + 64 i; tokens j >= live are computed on a
// repeated row and not written.  `sids`, when given, receives token j's k
// experts in slot order at sids[j * sstride] (the sort chunk's row ids).
template <int PL, int TW>
KQ_DEV void route_tokens(const float (&v)[TW][PL], const int (&t)[TW], int live, int E, int k, int norm,
                         int32_t* __restrict__ idx, float* __restrict__ w, int* sids, int sstride) {
  const int lane = lane_id();
  // value keys of the live experts; 0 marks a dead slot (no float maps to 0)
  uint32_t key[TW][PL];
  float my_sel[TW], first[TW], denom[TW];
#pragma unroll
  for (int j = 0; j < TW; ++j) {
#pragma unroll
    for (int i = 0; i < PL; ++i) key[j][i] = lane + 64 * i < E ? float_key(v[j][i]) : 0u;
    my_sel[j] = first[j] = denom[j] = 0.0f;
  }
  for (int r = 0; r < k; ++r) {
#pragma unroll
    for (int j = 0; j < TW; ++j) {
      // the largest key, then the smallest expert holding it: slot i covers
      // experts 64i..64i+63, so the first slot with a match holds the smallest
      uint32_t m = key[j][0];
#pragma unroll
      for (int i = 1; i < PL; ++i) m = max(m, key[j][i]);
      m = wave_max_u32_dpp(m);
      int e = -1;
#pragma unroll
      for (int i = PL - 1; i >= 0; --i) {
        const uint64_t hit = __ballot(key[j][i] == m);
        if (hit) e = 64 * i + (int)__builtin_ctzll(hit);
      }
      const float val = key_float(m);
#pragma unroll
      for (int i = 0; i < PL; ++i)
        if (lane + 64 * i == e) key[j][i] = 0u;
      if (lane == 0 && j < live) {
        idx[(int64_t)t[j] * k + r] = e;
        if (sids) sids[j * sstride + r] = e;
      }
      if (lane == r) my_sel[j] = val;
      if (r == 0) first[j] = val;
      if (norm) denom[j] = __fadd_rn(denom[j], expf(val - first[j]));  // slot order, uniform
    }
  }
  // fp32 softmax over the selected logits, or over all logits gathered
#pragma unroll
  for (int j = 0; j < TW; ++j) {
    float mx = first[j];
    if (!norm) {
      float m = -__builtin_inff();
#pragma unroll
      for (int i = 0; i < PL; ++i)
        if (lane + 64 * i < E) m = fmaxf(m, v[j][i]);
      mx = wave_max(m);
      float sum = 0.0f;
#pragma unroll
      for (int i = 0; i < PL; ++i)
        if (lane + 64 * i < E) sum += expf(v[j][i] - mx);
      denom[j] = wave_sum(sum);
    }
    if (lane < k && j < live) w[(int64_t)t[j] * k + lane] = __fdiv_rn(expf(my_sel[j] - mx), denom[j]);
  }
}

// The router logits of token t, widened; experts past E read as 0 (never
// selected: their keys are dead).
template <int PL>
KQ_DEV void route_load(const void* __restrict__ logits, int dtype, int t, int E, float (&v)[PL]) {
  const int lane = lane_id();
#pragma unroll
  for (int i = 0; i < PL; ++i) {
    const int e = lane + 64 * i;
    v[i] = e < E ? load_as_f32(logits, dtype, (int64_t)t * E + e) : 0.0f;
  }
}

template <int PL>   // logits per lane: E <= 64 * PL
__global__ void __launch_bounds__(256)
moe_route_kernel(const void* __restrict__ logits, int dtype, int T, int E, int k, int norm,
                 int32_t* __restrict__ idx, float* __restrict__ w) {
  const int t = blockIdx.x * 4 + wave_id();
  if (t >= T) return;
  float v[1][PL];
  route_load<PL>(logits, dtype, t, E, v[0]);
  const int tt[1] = {t};
  route_tokens<PL, 1>(v, tt, 1, E, k, norm, idx, w, nullptr, 0);
}

// -------------------------------------------------------------- stable sort
constexpr int kSortChunk = 256;   // threads per sort workgroup (>= rows per chunk)
// Rows per sort chunk: whole tokens (kSortChunk / k of them, their rows
// consecutive in the flat routed order r = token * k + slot), so one
// workgroup can route a chunk's tokens and count its experts; 256 rows for
// k > 256 (expert ids given by the caller).
__host__ __device__ inline int moe_chunk_rows(int k) {
  return k <= kSortChunk ? (kSortChunk / k) * k : kSortChunk;
}
// Chunks x experts up to which one launch both scans the chunk histograms and
// scatters (every workgroup reads the whole histogram table: 128 KB at most).
constexpr int kFusedScanMax = 32768;

// Row tiles of the expert GEMMs: 64 * moe_nrb rows.  320-row tiles (NRB 5)
// when the routing averages more than 192 rows per expert: an even top-k
// routing then spreads the experts' rows over ~256 +- 50, which 256-row tiles
// split into a full tile and a tail of a few rows that streams the same
// weights and unbalances the persistent schedule (C5: 368 -> 295 us).  With
// fewer rows every expert fits one 256-row tile, which costs less than a
// 320-row one (measured 3-6% at 16 to 1024 tokens of the C5 layer).
static inline int moe_nrb(int64_t routed_rows, int64_t experts) {
  return routed_rows > 192 * experts ? 5 : 4;
}

// Per-chunk expert histogram of the CR rows of chunk c: counts[c][e]
// (hist: E ints of LDS).
KQ_DEV void moe_count_chunk(const int32_t* __restrict__ idx, int R, int CR, int E, int32_t* __restrict__ counts,
                            int c, int* hist) {
  for (int i = threadIdx.x; i < E; i += kSortChunk) hist[i] = 0;
  __syncthreads();
  const int r = c * CR + (int)threadIdx.x;
  if ((int)threadIdx.x < CR && r < R) {
    const int e = idx[r];
    if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < E; i += kSortChunk) counts[(int64_t)c * E + i] = hist[i];
}

// Exclusive prefix sum of v[0..n) in LDS (n <= 1024); returns the total.
// Wave 0 scans (each lane a run of consecutive entries, lane totals through a
// shuffle scan) while the other waves wait at the barrier: two barriers
// instead of a workgroup-wide Hillis-Steele scan's twenty.  tmp[0] carries
// the total.
KQ_DEV int block_exclusive_scan(int* v, int* tmp, int n) {
  if (wave_id() == 0) {
    const int lane = lane_id();
    const int per = (n + 63) / 64;
    const int b = min(n, lane * per), e = min(n, b + per);
    int sum = 0;
    for (int i = b; i < e; ++i) sum += v[i];
    int inc = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(inc, off, 64);
      if (lane >= off) inc += y;
    }
    int run = inc - sum;
    for (int i = b; i < e; ++i) {
      const int x = v[i];
      v[i] = run;
      run += x;
    }
    if (lane == 63) tmp[0] = inc;
  }
  __syncthreads();
  const int total = tmp[0];
  __syncthreads();  // tmp and v are reused by the caller
  return total;
}

// The row-tile table from the experts' row counts: tile i -> (expert, first
// row, end row, 0); unused entries get expert -1; tile_count = tiles in use.
// Thread t < E writes expert t's tiles (first[t]: its first tile index,
// start[t]: its first sorted row, rows[t]: its row count); all threads clear
// the unused entries.
KQ_DEV void moe_write_tiles(const int* first, const int* start, const int* rows, int E, int BM, int total_tiles,
                            int max_tiles, int32_t* __restrict__ tiles, int32_t* __restrict__ tile_count) {
  const int t = threadIdx.x;
  if (t < E) {
    const int nt = (rows[t] + BM - 1) / BM;
    for (int i = 0; i < nt && first[t] + i < max_tiles; ++i) {
      int32_t* d = tiles + 4 * (first[t] + i);
      d[0] = t;
      d[1] = start[t] + i * BM;
      d[2] = min(start[t] + rows[t], start[t] + (i + 1) * BM);
      d[3] = 0;
    }
  }
  if (t == 0) tile_count[0] = min(total_tiles, max_tiles);
  for (int i = total_tiles + t; i < max_tiles; i += blockDim.x) {
    tiles[4 * i] = -1;
    tiles[4 * i + 1] = 0;
    tiles[4 * i + 2] = 0;
    tiles[4 * i + 3] = 0;
  }
}

// Chunk slices of the scan: the largest power of two with 2 * slices * E <=
// 1024 (at least 1), so slices * E threads each scan one run of chunks.
__host__ __device__ inline int moe_scan_slices(int E) {
  int slices = 1;
  while (slices * 2 * E <= 1024) slices *= 2;
  return slices;
}

// One 1024-thread workgroup (chunk tables too large for moe_scan_scatter):
// column-wise exclusive scan of counts[C][E] into base[c][e] (sorted position
// of chunk c's first row of expert e), expert offsets and the row-tile table.
// Thread (slice, e) scans a contiguous run of chunks.  PER > 0: the run has
// at most PER chunks, and the thread issues all its count loads at once into
// registers (unconditional loads from clamped, in-range addresses, so no load
// sits under a branch and they overlap) and keeps them for the second pass;
// PER = 0: any run length, one load at a time.
template <int PER>
__global__ void __launch_bounds__(1024)
moe_scan_kernel(const int32_t* __restrict__ counts, int C, int E, int BM, int max_tiles,
                int32_t* __restrict__ offsets, int32_t* __restrict__ base, int32_t* __restrict__ tiles,
                int32_t* __restrict__ tile_count) {
  __shared__ int part[1024], tot[1024], rows[1024], ntile[1024], tmp[1024];
  const int t = threadIdx.x;
  const int slices = moe_scan_slices(E);
  const int per = (C + slices - 1) / slices;
  const int e = t % E, sl = t / E;
  const bool active = sl < slices;
  const int c0 = active ? sl * per : 0, c1 = active ? min(C, c0 + per) : 0;
  int cnt[PER > 0 ? PER : 1];
  int sum = 0;
  if constexpr (PER > 0) {
    const int last = max(c1 - 1, 0);   // C >= 1, so chunk 0 always exists
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int v = counts[(int64_t)min(c0 + i, last) * E + e];
      cnt[i] = c0 + i < c1 ? v : 0;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) sum += cnt[i];
  } else {
    for (int c = c0; c < c1; ++c) sum += counts[(int64_t)c * E + e];
  }
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
    rows[t] = run;
    ntile[t] = (run + BM - 1) / BM;
  }
  __syncthreads();
  const int total_rows = block_exclusive_scan(tot, tmp, E);     // tot -> expert offsets
  const int total_tiles = block_exclusive_scan(ntile, tmp, E);  // ntile -> first tile
  if (active) {
    int run = tot[e] + part[t];
    if constexpr (PER > 0) {
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        if (c0 + i < c1) base[(int64_t)(c0 + i) * E + e] = run;
        run += cnt[i];
      }
    } else {
      for (int c = c0; c < c1; ++c) {
        base[(int64_t)c * E + e] = run;
        run += counts[(int64_t)c * E + e];
      }
    }
  }
  if (t < E) offsets[t] = tot[t];
  if (t == 0) offsets[E] = total_rows;
  moe_write_tiles(ntile, tot, rows, E, BM, total_tiles, max_tiles, tiles, tile_count);
}

// Sorted position of row r = base[e] (chunk c's first row of expert e) + its
// rank among the chunk's earlier rows routed to the same expert (stable).
// The rank is the rows of expert e in the chunk's earlier waves (per-wave
// counts in LDS, whist[w][e]) plus the earlier lanes of this wave with expert
// e: one ballot per bit of the expert id leaves the mask of lanes whose id
// equals this lane's.  sorted_tok[pos] is the token of the routed row at
// sorted position pos (the gate_up GEMM's row source), inv[r] the sorted
// position of routed row r.
KQ_DEV void moe_scatter_chunk(const int32_t* __restrict__ idx, int R, int CR, int E, int top_k, int c,
                              const int32_t* base, int* whist, int32_t* __restrict__ sorted_tok,
                              int32_t* __restrict__ inv) {
  const int t = threadIdx.x;
  const int w = t >> 6, lane = t & 63;
  const int r = c * CR + t;
  const bool in = t < CR && r < R;
  const int e = in ? idx[r] : -1;
  const bool ok = e >= 0 && e < E;
  for (int i = t; i < (kSortChunk / 64) * E; i += kSortChunk) whist[i] = 0;
  const int nbits = E > 1 ? 32 - __builtin_clz((unsigned)(E - 1)) : 0;
  uint64_t same = __ballot(ok);
  for (int b = 0; b < nbits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t m = __ballot(bit);
    same &= bit ? m : ~m;
  }
  const int rank_in = __popcll(same & ((1ull << lane) - 1ull));
  __syncthreads();   // whist cleared
  if (ok && rank_in == 0) whist[w * E + e] = __popcll(same);
  __syncthreads();
  if (!in) return;
  if (!ok) {
    inv[r] = -1;
    return;
  }
  int rank = rank_in;
  for (int w2 = 0; w2 < w; ++w2) rank += whist[w2 * E + e];
  const int pos = base[e] + rank;
  // (pos < R always holds for a consistent base table; the check keeps a
  // position outside the buffer from ever being written or combined)
  if (pos < R) sorted_tok[pos] = r / top_k;
  inv[r] = pos < R ? pos : -1;
}

__global__ void __launch_bounds__(kSortChunk)
moe_scatter_kernel(const int32_t* __restrict__ idx, int R, int CR, int E, int top_k,
                   const int32_t* __restrict__ base, int32_t* __restrict__ sorted_tok, int32_t* __restrict__ inv) {
  extern __shared__ int whist[];   // [kSortChunk / 64][E]
  const int c = blockIdx.x;
  moe_scatter_chunk(idx, R, CR, E, top_k, c, base + (int64_t)c * E, whist, sorted_tok, inv);
}

// Scan and scatter in one launch (E <= 256, C * E <= kFusedScanMax): chunk
// c's workgroup sums the histogram table itself — per expert, the rows of the
// chunks before c and of all chunks (thread (slice, e) one run of chunks, 16
// loads in flight) — scans the expert totals into offsets, and scatters its
// rows; workgroup 0 also writes the expert offsets and the row-tile table.
// Every workgroup derives the same totals, so the positions are those of the
// two-launch form.
__global__ void __launch_bounds__(kSortChunk)
moe_scan_scatter_kernel(const int32_t* __restrict__ idx, int R, int CR, int E, int top_k,
                        const int32_t* __restrict__ counts, int C, int BM, int max_tiles,
                        int32_t* __restrict__ offsets, int32_t* __restrict__ tiles,
                        int32_t* __restrict__ tile_count, int32_t* __restrict__ sorted_tok,
                        int32_t* __restrict__ inv) {
  __shared__ int part_pre[4 * kSortChunk], part_tot[4 * kSortChunk], sbase[kSortChunk], soff[kSortChunk];
  __shared__ int srows[kSortChunk], sfirst[kSortChunk], tmp[kSortChunk];
  __shared__ int whist[(kSortChunk / 64) * kSortChunk];
  const int c = blockIdx.x, t = threadIdx.x;
  // thread (slice, q) sums experts [VW q, VW q + VW) over one run of chunks
  // (16-byte loads of four experts when E % 4 == 0)
  const int VW = E % 4 == 0 ? 4 : 1;
  const int Q = E / VW, S = kSortChunk / Q;  // chunk slices (E <= kSortChunk)
  const int q = t % Q, sl = t / Q;
  int pre[4] = {0, 0, 0, 0}, tot[4] = {0, 0, 0, 0};
  if (sl < S) {
    const int c0 = (int)((int64_t)C * sl / S), c1 = (int)((int64_t)C * (sl + 1) / S);
    for (int cc = c0; cc < c1; cc += 16) {
      if (VW == 4) {
        i32x4 v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = *(const i32x4*)(counts + (int64_t)min(cc + u, c1 - 1) * E + 4 * q);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int x = cc + u < c1 ? v[u][i] : 0;
            tot[i] += x;
            pre[i] += cc + u < c ? x : 0;
          }
        }
      } else {
        int v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = counts[(int64_t)min(cc + u, c1 - 1) * E + q];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
          const int x = cc + u < c1 ? v[u] : 0;
          tot[0] += x;
          pre[0] += cc + u < c ? x : 0;
        }
      }
    }
    for (int i = 0; i < VW; ++i) {
      part_pre[sl * E + VW * q + i] = pre[i];
      part_tot[sl * E + VW * q + i] = tot[i];
    }
  }
  __syncthreads();
  if (t < E) {
    int before = 0, rows = 0;
    for (int s2 = 0; s2 < S; ++s2) {
      before += part_pre[s2 * E + t];
      rows += part_tot[s2 * E + t];
    }
    sbase[t] = before;
    srows[t] = rows;
    soff[t] = rows;
    sfirst[t] = (rows + BM - 1) / BM;
  }
  __syncthreads();
  const int total_rows = block_exclusive_scan(soff, tmp, E);      // soff -> expert offsets
  const int total_tiles = block_exclusive_scan(sfirst, tmp, E);   // sfirst -> first tile
  if (t < E) sbase[t] += soff[t];
  if (c == 0) {
    if (t < E) offsets[t] = soff[t];
    if (t == 0) offsets[E] = total_rows;
    moe_write_tiles(sfirst, soff, srows, E, BM, total_tiles, max_tiles, tiles, tile_count);
  }
  __syncthreads();   // sbase complete
  moe_scatter_chunk(idx, R, CR, E, top_k, c, sbase, whist, sorted_tok, inv);
}

// --------------------------------------------------- 1x128 activation quant
// A quantization unit is kQuantRows consecutive rows x one 2048-element span
// (256 threads x 8 elements, 16 threads per 1x128 block): the threads issue
// the rows' 16-byte loads back to back, then quantize row by row.  (One row
// per 256-thread workgroup left the C5 token pass latency-bound at 9 us.)
constexpr int kQuantRows = 4;

// Raw 16-bit elements of thread tx in span y of rows [row0, row0 +
// kQuantRows) (rows past `rows` repeat the last row; elements past K read 0).
KQ_DEV void aq_load_rows(const uint16_t* __restrict__ x, int K, int64_t ldx, bool vec, int64_t row0,
                         int64_t rows, int y, int tx, u32x4 (&raw)[kQuantRows]) {
  const int k0 = y * 2048 + tx * 8;
  if (vec && k0 + 8 <= K) {
#pragma unroll
    for (int j = 0; j < kQuantRows; ++j) raw[j] = *(const u32x4*)(x + min(row0 + j, rows - 1) * ldx + k0);
  } else {
#pragma unroll
    for (int j = 0; j < kQuantRows; ++j) {
      const uint16_t* xr = x + min(row0 + j, rows - 1) * ldx;
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) h[e] = k0 + e < K ? xr[k0 + e] : 0u;
      raw[j] = u32x4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
    }
  }
}

// 1x128 block scale of thread tx's 16-lane group (s = max(amax, 1e-12) /
// 448), e4m3 values of its 8 elements, stored with the block's scale.
KQ_DEV void aq_quant8(const u32x4 raw, int dtype, int K, uint8_t* __restrict__ xq, float* __restrict__ xs,
                      int64_t row, int y, int tx) {
  const int k0 = y * 2048 + tx * 8;
  float v[8];
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    v[2 * d] = dtype == KQ_DTYPE_BF16 ? bf16_to_f32(raw[d] & 0xffffu) : f16_to_f32(raw[d] & 0xffffu);
    v[2 * d + 1] = dtype == KQ_DTYPE_BF16 ? bf16_to_f32(raw[d] >> 16) : f16_to_f32(raw[d] >> 16);
  }
  // block amax as an integer max of |bits|: inf and NaN order above every
  // finite magnitude, so a NaN in the block makes the scale NaN (torch's amax
  // and clamp propagate it) and a non-finite block takes the IEEE path below
  uint32_t abits = 0;
#pragma unroll
  for (int e = 0; e < 8; ++e) abits = max(abits, __float_as_uint(v[e]) & 0x7fffffffu);
#pragma unroll
  for (int off = 8; off > 0; off >>= 1) abits = max(abits, (uint32_t)__shfl_xor((int)abits, off, 64));
  if (k0 >= K) return;
  const float s = __fdiv_rn(max_keep_nan(__uint_as_float(abits), 1e-12f), 448.0f);
  uint32_t lo = 0, hi = 0;
  if (abits < 0x7f800000u) {
    // finite block: reciprocal + fma remainder (IEEE quotient wherever it
    // matters) and the hardware e4m3 converter
    const float rs = __fdiv_rn(1.0f, s);
    float q[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) q[e] = fminf(fmaxf(div_by_recip(v[e], s, rs), -448.0f), 448.0f);
    lo = pack4_e4m3(q[0], q[1], q[2], q[3]);
    hi = pack4_e4m3(q[4], q[5], q[6], q[7]);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      float q = __fdiv_rn(v[e], s);
      q = q < -448.0f ? -448.0f : (q > 448.0f ? 448.0f : q);
      const uint32_t b = f32_to_e4m3(q);
      if (e < 4) lo |= b << (8 * e);
      else hi |= b << (8 * (e - 4));
    }
  }
  uint8_t* qr = xq + row * (int64_t)K;
  if (k0 + 8 <= K && (K % 8) == 0) {
    *(u32x2*)(qr + k0) = u32x2{lo, hi};
  } else {
    for (int e = 0; e < 8 && k0 + e < K; ++e) qr[k0 + e] = (uint8_t)(((e < 4 ? lo : hi) >> (8 * (e & 3))) & 0xffu);
  }
  if ((tx & 15) == 0) xs[row * ((K + 127) / 128) + k0 / 128] = s;
}

// Rows [row0, row0 + kQuantRows) of `rows`, span y, by the 256 threads tx =
// 0..255 (whole waves; the row-count test is uniform over them).
KQ_DEV void act_quant_fp8_blocks_unit(const uint16_t* __restrict__ x, int dtype, int K, int64_t ldx, bool vec,
                                      int64_t row0, int64_t rows, int y, uint8_t* __restrict__ xq,
                                      float* __restrict__ xs, int tx) {
  u32x4 raw[kQuantRows];
  aq_load_rows(x, K, ldx, vec, row0, rows, y, tx, raw);
#pragma unroll
  for (int j = 0; j < kQuantRows; ++j)
    if (row0 + j < rows) aq_quant8(raw[j], dtype, K, xq, xs, row0 + j, y, tx);
}

// Grid (row groups, spans): blockIdx.y is the span, blockIdx.x strides over
// groups of kQuantRows rows.
__global__ void __launch_bounds__(256)
act_quant_fp8_blocks_kernel(const uint16_t* __restrict__ x, int dtype, int K, int64_t ldx, bool vec, int64_t rows,
                            uint8_t* __restrict__ xq, float* __restrict__ xs) {
  for (int64_t g = blockIdx.x; g * kQuantRows < rows; g += gridDim.x)
    act_quant_fp8_blocks_unit(x, dtype, K, ldx, vec, g * kQuantRows, rows, (int)blockIdx.y, xq, xs, threadIdx.x);
}

// Quantization unit u of a MoE call's tokens: row group u / KY, span u % KY.
KQ_DEV void moe_quant_unit(const uint16_t* __restrict__ x, int dtype, int K, bool vec, int KY, int u, int64_t rows,
                           uint8_t* __restrict__ xq, float* __restrict__ xs, int tx) {
  const int y = u % KY, g = u / KY;
  act_quant_fp8_blocks_unit(x, dtype, K, K, vec, (int64_t)g * kQuantRows, rows, y, xq, xs, tx);
}

// MoE with the caller's routing: the chunk histograms (workgroups [0, C))
// and the token quantization (one unit per workgroup after them) in one
// launch; neither reads the other's output.
static_assert(kSortChunk == 256, "a sort chunk and a quantization unit both take 256 threads");
__global__ void __launch_bounds__(256)
moe_count_quant_kernel(const int32_t* __restrict__ idx, int R, int CR, int E, int32_t* __restrict__ counts, int C,
                       const uint16_t* __restrict__ x, int dtype, int K, bool vec, int KY, int64_t T,
                       uint8_t* __restrict__ xq, float* __restrict__ xs) {
  extern __shared__ int hist[];
  const int b = blockIdx.x;
  if (b < C) moe_count_chunk(idx, R, CR, E, counts, b, hist);
  else moe_quant_unit(x, dtype, K, vec, KY, b - C, T, xq, xs, threadIdx.x);
}

// MoE from router logits, 1024-thread workgroups: workgroup c < C routes the
// chunk's TPC tokens, writes topk_idx / topk_w and the chunk's expert
// histogram; each of the other workgroups quantizes four token units (256
// threads per unit).  TPC <= 16: one token per wave; more: wave w takes
// tokens w, w + 16, ... two at a time, their selection chains interleaved.
// Routing needs many waves in flight: one chunk per 256-thread workgroup (8
// tokens per wave in turn) took 24.7 us for C5's 4096 tokens, 32-token chunks
// (2 per wave) 15.4 us, where the one-token-per-wave routing kernel takes
// 6 us.
constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;

// Tokens per sort chunk of the routed call: one per route wave where the
// chunk table still fits the one-launch scan (and a chunk holds at most
// kSortChunk rows), else kSortChunk / k.
static inline int moe_routed_chunk_tokens(int64_t T, int k, int64_t E) {
  const int full = kSortChunk / k;  // k <= kRouteMaxTopK
  if (full > kRouteWaves && E <= kSortChunk && (T + kRouteWaves - 1) / kRouteWaves * E <= kFusedScanMax)
    return kRouteWaves;
  return full;
}

template <int PL>
__global__ void __launch_bounds__(kRouteThreads)
moe_route_count_quant_kernel(const void* __restrict__ logits, int ldtype, int T, int E, int k, int norm,
                             int TPC, int32_t* __restrict__ idx, float* __restrict__ w,
                             int32_t* __restrict__ counts, int C, const uint16_t* __restrict__ x, int dtype,
                             int K, bool vec, int KY, int units, uint8_t* __restrict__ xq,
                             float* __restrict__ xs) {
  extern __shared__ int hist[];   // E counters, then the chunk's expert ids (kSortChunk)
  const int b = blockIdx.x;
  if (b >= C) {
    // four quantization units, one per 256 threads
    const int u = (b - C) * (kRouteThreads / 256) + (int)(threadIdx.x >> 8);
    if (u < units) moe_quant_unit(x, dtype, K, vec, KY, u, T, xq, xs, threadIdx.x & 255);
    return;
  }
  int* sids = hist + E;
  for (int i = threadIdx.x; i < E; i += kRouteThreads) hist[i] = 0;
  const int t0 = b * TPC, nt = min(TPC, T - t0);
  const int wv = wave_id();
  if (TPC <= kRouteWaves) {
    if (wv < nt) {
      float v[1][PL];
      route_load<PL>(logits, ldtype, t0 + wv, E, v[0]);
      const int tt[1] = {t0 + wv};
      route_tokens<PL, 1>(v, tt, 1, E, k, norm, idx, w, sids + wv * k, 0);
    }
  } else for (int i = wv; i < nt; i += 2 * kRouteWaves) {
    const int i1 = min(i + kRouteWaves, nt - 1);
    float v[2][PL];
    route_load<PL>(logits, ldtype, t0 + i, E, v[0]);
    route_load<PL>(logits, ldtype, t0 + i1, E, v[1]);
    const int tt[2] = {t0 + i, t0 + i1};
    const int live = i + kRouteWaves < nt ? 2 : 1;
    route_tokens<PL, 2>(v, tt, live, E, k, norm, idx, w, sids + i * k, kRouteWaves * k);
  }
  __syncthreads();   // hist cleared, the chunk's ids in LDS
  if ((int)threadIdx.x < nt * k) {
    const int e = sids[threadIdx.x];
    if (e >= 0 && e < E) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  for (int i = threadIdx.x; i < E; i += kRouteThreads) counts[(int64_t)b * E + i] = hist[i];
}

// ------------------------------------------------------------------ combine
// out[t] = sum over slots s (in order) of fp32(y[inv[t*k+s]]) * w[t*k+s].
KQ_DEV void widen8_out(u32x4 raw, int dtype, float v[8]) {
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    v[2 * d] = dtype == KQ_DTYPE_BF16 ? bf16_to_f32(raw[d] & 0xffffu) : f16_to_f32(raw[d] & 0xffffu);
    v[2 * d + 1] = dtype == KQ_DTYPE_BF16 ? bf16_to_f32(raw[d] >> 16) : f16_to_f32(raw[d] >> 16);
  }
}

__global__ void __launch_bounds__(256)
moe_combine_kernel(const uint16_t* __restrict__ y, int y_dtype, const int32_t* __restrict__ inv,
                   const float* __restrict__ w, int k, int H, uint16_t* __restrict__ out) {
  const int64_t t = blockIdx.x;
  if (k == 8 && (H & 7) == 0 && (((uintptr_t)out | (uintptr_t)y) & 15) == 0) {
    // the common top-8 case: all eight rows are requested before the first
    // is summed (the generic loop below has one row in flight per thread)
    for (int h = threadIdx.x * 8; h < H; h += 256 * 8) {
      int pos[8];
      float wv[8];
      u32x4 raw[8];
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        pos[s] = inv[t * 8 + s];
        wv[s] = w[t * 8 + s];
      }
#pragma unroll
      for (int s = 0; s < 8; ++s) raw[s] = *(const u32x4*)(y + (int64_t)max(pos[s], 0) * H + h);
      float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        float yv[8];
        widen8_out(raw[s], y_dtype, yv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float sum = __fadd_rn(acc[e], __fmul_rn(yv[e], wv[s]));
          acc[e] = pos[s] < 0 ? acc[e] : sum;  // an unrouted slot adds nothing
        }
      }
      u32x4 o;
#pragma unroll
      for (int d = 0; d < 4; ++d)
        o[d] = (uint32_t)f32_to_out(acc[2 * d], y_dtype) | ((uint32_t)f32_to_out(acc[2 * d + 1], y_dtype) << 16);
      *(u32x4*)(out + t * H + h) = o;
    }
    return;
  }
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
  size_t counts, base, offsets, tiles, tile_count, sorted, inv, xq, xs, actq, acts, y, total;
};

static size_t align256(size_t v) { return (v + 255) / 256 * 256; }

static MoeWorkspace moe_layout(int64_t T, int64_t H, int64_t I, int64_t E, int64_t k) {
  const int64_t R = T * k;
  const int64_t CR = moe_chunk_rows((int)k);
  // chunks of either call: the caller's routing (CR rows) or the routed call
  int64_t C = (R + CR - 1) / CR;
  if (k <= kRouteMaxTopK) {
    const int64_t tpc = moe_routed_chunk_tokens(T, (int)k, E);
    C = std::max(C, (T + tpc - 1) / tpc);
  }
  const int64_t BM = 64 * moe_nrb(R, E);
  const int64_t max_tiles = (R + BM - 1) / BM + E;
  MoeWorkspace w{};
  size_t p = 0;
  auto take = [&](size_t bytes) { const size_t at = p; p += align256(bytes); return at; };
  w.counts = take((size_t)C * E * 4);
  w.base = take((size_t)C * E * 4);
  w.offsets = take((size_t)(E + 1) * 4);
  w.tiles = take((size_t)max_tiles * 16);
  w.tile_count = take(4);
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
  const int64_t groups = (rows + kQuantRows - 1) / kQuantRows;
  const dim3 grid((unsigned)std::min<int64_t>(groups, 1 << 20), (unsigned)((K + 2047) / 2048));
  hipLaunchKernelGGL(act_quant_fp8_blocks_kernel, grid, dim3(256), 0, st, (const uint16_t*)x, dtype, (int)K, ldx,
                     vec, rows, xq, xs);
}

// Shapes of one MoE call and its workspace pointers.
struct MoeCall {
  const void* hidden;
  int dtype, top_k;
  int64_t tokens, H, I, E;
  int R, CR, C, nrb, BM, max_tiles, KY;
  int tpc;              // routed call: tokens per sort chunk (CR = tpc * top_k)
  int units;            // token quantization units (kQuantRows rows x one 2048-element span)
  bool vec;
  int32_t *counts, *base, *offsets, *tiles, *tile_count, *sorted, *inv;
  uint8_t *xq, *actq;
  float *xs, *acts;
  uint16_t* y;
};

static MoeCall moe_call(const void* hidden, int dtype, int64_t tokens, int64_t H, int64_t I, int64_t E,
                        int top_k, void* workspace, bool routed) {
  const MoeWorkspace L = moe_layout(tokens, H, I, E, top_k);
  uint8_t* ws = (uint8_t*)workspace;
  MoeCall m{};
  m.hidden = hidden; m.dtype = dtype; m.top_k = top_k;
  m.tokens = tokens; m.H = H; m.I = I; m.E = E;
  m.R = (int)(tokens * top_k);
  m.tpc = routed ? moe_routed_chunk_tokens(tokens, top_k, E) : 0;
  m.CR = routed ? m.tpc * top_k : moe_chunk_rows(top_k);
  m.C = (m.R + m.CR - 1) / m.CR;
  m.nrb = moe_nrb(m.R, E);
  m.BM = 64 * m.nrb;
  m.max_tiles = (m.R + m.BM - 1) / m.BM + (int)E;
  m.KY = (int)((H + 2047) / 2048);
  m.units = (int)((tokens + kQuantRows - 1) / kQuantRows) * m.KY;
  m.vec = ((uintptr_t)hidden % 16) == 0 && (H % 8) == 0;
  m.counts = (int32_t*)(ws + L.counts);
  m.base = (int32_t*)(ws + L.base);
  m.offsets = (int32_t*)(ws + L.offsets);
  m.tiles = (int32_t*)(ws + L.tiles);
  m.tile_count = (int32_t*)(ws + L.tile_count);
  m.sorted = (int32_t*)(ws + L.sorted);
  m.inv = (int32_t*)(ws + L.inv);
  m.xq = ws + L.xq;
  m.xs = (float*)(ws + L.xs);
  m.actq = ws + L.actq;
  m.acts = (float*)(ws + L.acts);
  m.y = (uint16_t*)(ws + L.y);
  return m;
}

// After the chunk histograms and the token quantization: the stable sort's
// scan and scatter (one launch when the histogram table is small, else the
// one-workgroup scan and the scatter), both grouped GEMMs and the combine.
static void moe_sort_experts_combine(const MoeCall& m, const int32_t* topk_idx, const float* topk_w,
                                     const uint8_t* w13, const float* s13, const uint8_t* w2,
                                     const float* s2, void* out, hipStream_t st) {
  const int E = (int)m.E;
  if (E <= kSortChunk && (int64_t)m.C * E <= kFusedScanMax) {
    hipLaunchKernelGGL(moe_scan_scatter_kernel, dim3(m.C), dim3(kSortChunk), 0, st, topk_idx, m.R, m.CR, E,
                       m.top_k, m.counts, m.C, m.BM, m.max_tiles, m.offsets, m.tiles, m.tile_count, m.sorted,
                       m.inv);
  } else {
    const int scan_per = (m.C + moe_scan_slices(E) - 1) / moe_scan_slices(E);
    if (scan_per <= 16)
      hipLaunchKernelGGL(moe_scan_kernel<16>, dim3(1), dim3(1024), 0, st, m.counts, m.C, E, m.BM, m.max_tiles,
                         m.offsets, m.base, m.tiles, m.tile_count);
    else if (scan_per <= 64)
      hipLaunchKernelGGL(moe_scan_kernel<64>, dim3(1), dim3(1024), 0, st, m.counts, m.C, E, m.BM, m.max_tiles,
                         m.offsets, m.base, m.tiles, m.tile_count);
    else
      hipLaunchKernelGGL(moe_scan_kernel<0>, dim3(1), dim3(1024), 0, st, m.counts, m.C, E, m.BM, m.max_tiles,
                         m.offsets, m.base, m.tiles, m.tile_count);
    hipLaunchKernelGGL(moe_scatter_kernel, dim3(m.C), dim3(kSortChunk), (kSortChunk / 64) * E * sizeof(int), st,
                       topk_idx, m.R, m.CR, E, m.top_k, m.base, m.sorted, m.inv);
  }

  TileGemmArgs g{};
  g.x = m.xq; g.xs = m.xs; g.x_rows = (int)m.tokens; g.gather = m.sorted; g.gather_rows = m.R;
  g.w = w13; g.ws = s13; g.mtile_table = m.tiles; g.mtile_count = m.tile_count;
  g.N = (int)(2 * m.I); g.K = (int)m.H; g.I = (int)m.I;
  g.mtiles = m.max_tiles; g.ntiles = (int)(m.I / 128);
  g.actq = m.actq; g.acts = m.acts; g.out_dtype = m.dtype; g.bias_dtype = KQ_DTYPE_NONE;
  if (m.nrb == 5) tg_launch<kTgFp8, true, kTgEpiSwiGluQuant, 5, true>(g, st);
  else tg_launch<kTgFp8, true, kTgEpiSwiGluQuant, 4, true>(g, st);

  TileGemmArgs d{};
  d.x = m.actq; d.xs = m.acts; d.x_rows = m.R; d.gather = nullptr;
  d.w = w2; d.ws = s2; d.mtile_table = m.tiles; d.mtile_count = m.tile_count;
  d.N = (int)m.H; d.K = (int)m.I; d.I = 0;
  d.mtiles = m.max_tiles; d.ntiles = (int)((m.H + kTgBN - 1) / kTgBN);
  d.out = m.y; d.out_dtype = m.dtype; d.bias = nullptr; d.bias_dtype = KQ_DTYPE_NONE;
  if (m.nrb == 5) tg_launch<kTgFp8, true, kTgEpiStore, 5, true>(d, st);
  else tg_launch<kTgFp8, true, kTgEpiStore, 4, true>(d, st);

  hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)m.tokens), dim3(256), 0, st, m.y, m.dtype, m.inv, topk_w,
                     m.top_k, (int)m.H, (uint16_t*)out);
}

// Shape checks shared by both MoE entry points; 0 or an error code.
static int moe_check_shape(const char* name, int dtype, int64_t tokens, int64_t hidden_size, int64_t inter,
                           int64_t experts, int top_k, void* workspace, size_t workspace_bytes) {
  if (!quant_dtype_ok(dtype)) {
    set_error("%s: hidden dtype must be fp16 or bf16", name);
    return KQ_EUNSUPPORTED;
  }
  if (tokens < 0 || hidden_size < kTgBK || (hidden_size % kTgBK) != 0 || inter < kTgBK ||
      (inter % kTgBK) != 0 || experts < 1 || experts > 1024 || top_k < 1 || top_k > experts ||
      hidden_size > kTgBK * kTgMaxKB || inter > kTgBK * kTgMaxKB || tokens * top_k > 0x7fffffffLL ||
      hidden_size * 2 * inter > 0x7fffffffLL || tokens * hidden_size > 0x7fffffffLL ||
      tokens * top_k * inter > 0x7fffffffLL) {
    set_error("%s: bad shape tokens=%lld hidden=%lld inter=%lld experts=%lld top_k=%d (hidden and inter "
              "must be multiples of 128)",
              name, (long long)tokens, (long long)hidden_size, (long long)inter, (long long)experts, top_k);
    return KQ_EINVAL;
  }
  if (tokens == 0) return KQ_OK;
  const MoeWorkspace L = moe_layout(tokens, hidden_size, inter, experts, top_k);
  if (workspace == nullptr || workspace_bytes < L.total) {
    set_error("%s: workspace of %zu bytes is smaller than the %zu bytes this call needs", name,
              workspace ? workspace_bytes : (size_t)0, L.total);
    return KQ_EWORKSPACE;
  }
  return KQ_OK;
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
  const dim3 grid((unsigned)((tokens + 3) / 4)), block(256);
  hipStream_t st = (hipStream_t)stream;
  const int T = (int)tokens, E = (int)experts, norm = norm_topk_prob ? 1 : 0;
  if (E <= 64)
    hipLaunchKernelGGL(moe_route_kernel<1>, grid, block, 0, st, logits, dtype, T, E, top_k, norm, topk_idx, topk_w);
  else if (E <= 128)
    hipLaunchKernelGGL(moe_route_kernel<2>, grid, block, 0, st, logits, dtype, T, E, top_k, norm, topk_idx, topk_w);
  else if (E <= 256)
    hipLaunchKernelGGL(moe_route_kernel<4>, grid, block, 0, st, logits, dtype, T, E, top_k, norm, topk_idx, topk_w);
  else
    hipLaunchKernelGGL(moe_route_kernel<kRouteMaxPerLane>, grid, block, 0, st, logits, dtype, T, E, top_k, norm,
                       topk_idx, topk_w);
  return check_launch("kq_moe_route_topk");
}

extern "C" int kq_act_quant_fp8_blocks(const void* x, int x_dtype, int64_t rows, int64_t k,
                                       int64_t ldx, uint8_t* xq, float* xs, void* stream) {
  if (!quant_dtype_ok(x_dtype)) {
    set_error("kq_act_quant_fp8_blocks: activation dtype must be fp16 or bf16");
    return KQ_EUNSUPPORTED;
  }
  if (rows < 0 || k < 1 || ldx < k || rows > 0x7fffffffLL || k > 65535LL * 2048) {
    set_error("kq_act_quant_fp8_blocks: bad shape rows=%lld k=%lld (k <= 65535 * 2048)", (long long)rows,
              (long long)k);
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
  if (m < 0 || n < 1 || k < kTgBK || (k % kTgBK) != 0 || k > kTgBK * kTgMaxKB || m > 0x7fffffffLL ||
      n > 0x7fffffffLL || n * k > 0x7fffffffLL || m * k > 0x7fffffffLL) {
    set_error("kq_block_fp8_gemm: bad shape m=%lld n=%lld k=%lld (k must be a multiple of 128)",
              (long long)m, (long long)n, (long long)k);
    return KQ_EINVAL;
  }
  if (m == 0) return KQ_OK;
  TileGemmArgs a{};
  a.x = xq; a.xs = xs; a.x_rows = (int)m; a.gather = nullptr;
  a.w = w; a.ws = ws; a.mtile_table = nullptr; a.mtile_count = nullptr;
  a.M = (int)m; a.N = (int)n; a.K = (int)k; a.I = 0;
  a.mtiles = (int)((m + kTgBM - 1) / kTgBM);
  a.ntiles = (int)((n + kTgBN - 1) / kTgBN);
  a.out = out; a.out_dtype = out_dtype; a.bias = bias; a.bias_dtype = bias_dtype;
  tg_launch<kTgFp8, true, kTgEpiStore>(a, (hipStream_t)stream);
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
  const int bad = moe_check_shape("kq_moe_block_fp8_experts", dtype, tokens, hidden_size, inter, experts,
                                  top_k, workspace, workspace_bytes);
  if (bad != KQ_OK || tokens == 0) return bad;
  hipStream_t st = (hipStream_t)stream;
  const MoeCall m = moe_call(hidden, dtype, tokens, hidden_size, inter, experts, top_k, workspace, false);
  // chunk histograms and the token quantization share one launch
  const int64_t blocks = (int64_t)m.C + m.units;
  hipLaunchKernelGGL(moe_count_quant_kernel, dim3((unsigned)blocks), dim3(kSortChunk), m.E * sizeof(int), st,
                     topk_idx, m.R, m.CR, (int)m.E, m.counts, m.C, (const uint16_t*)hidden, dtype, (int)m.H, m.vec,
                     m.KY, m.tokens, m.xq, m.xs);
  moe_sort_experts_combine(m, topk_idx, topk_w, w13, s13, w2, s2, out, st);
  return check_launch("kq_moe_block_fp8_experts");
}

extern "C" int kq_moe_routed_block_fp8_experts(const void* logits, int logits_dtype, int norm_topk_prob,
                                               const void* hidden, int dtype, int64_t tokens,
                                               int64_t hidden_size, int64_t inter, int64_t experts,
                                               int top_k, const uint8_t* w13, const float* s13,
                                               const uint8_t* w2, const float* s2, int32_t* topk_idx,
                                               float* topk_w, void* out, void* workspace,
                                               size_t workspace_bytes, void* stream) {
  if (logits_dtype != KQ_DTYPE_F16 && logits_dtype != KQ_DTYPE_BF16 && logits_dtype != KQ_DTYPE_F32) {
    set_error("kq_moe_routed_block_fp8_experts: logits must be fp16, bf16 or fp32");
    return KQ_EUNSUPPORTED;
  }
  if (experts > 64 * kRouteMaxPerLane || top_k > kRouteMaxTopK || tokens > 0x7fffffffLL / 64) {
    set_error("kq_moe_routed_block_fp8_experts: routing supports experts <= %d and top_k <= %d "
              "(experts=%lld top_k=%d)", 64 * kRouteMaxPerLane, kRouteMaxTopK, (long long)experts, top_k);
    return KQ_EINVAL;
  }
  const int bad = moe_check_shape("kq_moe_routed_block_fp8_experts", dtype, tokens, hidden_size, inter, experts,
                                  top_k, workspace, workspace_bytes);
  if (bad != KQ_OK || tokens == 0) return bad;
  if (logits == nullptr || topk_idx == nullptr || topk_w == nullptr) {
    set_error("kq_moe_routed_block_fp8_experts: logits, topk_idx and topk_w are required");
    return KQ_EINVAL;
  }
  hipStream_t st = (hipStream_t)stream;
  const MoeCall m = moe_call(hidden, dtype, tokens, hidden_size, inter, experts, top_k, workspace, true);
  // routing, the chunk histograms and the token quantization in one launch
  const int64_t per_block = kRouteThreads / 256;
  const int64_t blocks = (int64_t)m.C + (m.units + per_block - 1) / per_block;
  const size_t lds = (size_t)(m.E + kSortChunk) * sizeof(int);
  const int T = (int)tokens, E = (int)experts, norm = norm_topk_prob ? 1 : 0;
  const dim3 grid((unsigned)blocks), block(kRouteThreads);
#define KQ_ROUTE_LAUNCH(PL)                                                                                    \
  hipLaunchKernelGGL(moe_route_count_quant_kernel<PL>, grid, block, lds, st, logits, logits_dtype, T, E, top_k, \
                     norm, m.tpc, topk_idx, topk_w, m.counts, m.C, (const uint16_t*)hidden, dtype, (int)m.H,    \
                     m.vec, m.KY, m.units, m.xq, m.xs)
  if (E <= 64) KQ_ROUTE_LAUNCH(1);
  else if (E <= 128) KQ_ROUTE_LAUNCH(2);
  else if (E <= 256) KQ_ROUTE_LAUNCH(4);
  else KQ_ROUTE_LAUNCH(kRouteMaxPerLane);
#undef KQ_ROUTE_LAUNCH
  moe_sort_experts_combine(m, topk_idx, topk_w, w13, s13, w2, s2, out, st);
  return check_launch("kq_moe_routed_block_fp8_experts");
}
