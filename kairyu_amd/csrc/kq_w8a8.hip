// W8A8 GEMMs for gfx950: INT8 (v_mfma_i32_16x16x64_i8) and FP8 e4m3
// (v_mfma_scale_f32_16x16x128_f8f6f4 with unit scales).
//
//   out[m, n] = epilogue( sum_k xq[m, k] * w[n, k] )
//   INT8: fp32(acc) * xscale[m] * wscale[n] (+ bias[n]), int32 accumulation
//         exact; each multiply/add rounded separately (no FMA contraction), the
//         CPU oracle's op order (kairyu/quant/int8.py:33-41, linear.py:547-553).
//   FP8 : acc (fp32) * xscale[m] * wscale[n or 0] (+ bias[n])
//         (kairyu/quant/fp8.py:48-56, linear.py:463-469).
//
// Kernels:
//   * skinny (M <= 64): a workgroup owns 16 output columns; its 8 waves split
//     K, stream weight rows straight into MFMA B-operand registers and reduce
//     through LDS.  Small-N shapes also split K across workgroups, finished
//     by a separate reduce kernel (no inter-workgroup sync).  HBM-bound.
//   * M > 64 with at least one 256x256 tile per CU: the persistent tile
//     engine of kq_tile_gemm.h (LDS DMA double buffering, XCD-grouped tiles).
//   * other M > 64: 128x128x128 workgroup tiles, 4 waves of 64x64, LDS
//     double buffer with an XOR chunk swizzle (twice the workgroups of the
//     256x256 engine for shapes that would leave CUs idle).
#include "kq_common.h"
#include "kq_splitk.h"
#include "kq_tile_gemm.h"

namespace kq {

enum { kFmtI8 = 0, kFmtFp8 = 1 };

template <int FMT> struct W8Traits;
template <> struct W8Traits<kFmtI8> {
  static constexpr int kStep = 64;   // K per MFMA
  static constexpr int kLane = 16;   // bytes per lane per operand
  using Acc = i32x4;
  using Frag = i32x4;
};
template <> struct W8Traits<kFmtFp8> {
  static constexpr int kStep = 128;
  static constexpr int kLane = 32;
  using Acc = f32x4;
  using Frag = i32x8;
};

struct Epi {
  const float* xscale;
  const float* wscale;
  int ws_per_channel;
  const void* bias;
  int bias_dtype;
  void* out;
  int out_dtype;
  int32_t* acc_out;
  int M, N;
  // decode kernels only: N = 2I packed gate / up weight rows [gate; up], the
  // output out[M][I] = silu(gate) * up (SwiGLU epilogue); 0: out[M][N]
  int swiglu;
};

template <int FMT>
KQ_DEV void epi_store(const Epi& ep, int m, int n, typename W8Traits<FMT>::Acc acc, int r) {
  if (m >= ep.M || n >= ep.N) return;
  float v;
  if constexpr (FMT == kFmtI8) {
    if (ep.acc_out) ep.acc_out[(int64_t)m * ep.N + n] = acc[r];
    v = (float)acc[r];
  } else {
    v = acc[r];
  }
  v = __fmul_rn(v, ep.xscale[m]);
  v = __fmul_rn(v, ep.ws_per_channel ? ep.wscale[n] : ep.wscale[0]);
  if (ep.bias_dtype != KQ_DTYPE_NONE) v = __fadd_rn(v, load_as_f32(ep.bias, ep.bias_dtype, n));
  ((uint16_t*)ep.out)[(int64_t)m * ep.N + n] = f32_to_out(v, ep.out_dtype);
}

// Decode tiles with the SwiGLU epilogue: tile t pairs gate rows [8t, 8t + 8)
// (tile rows 0..7) with up rows [I + 8t, I + 8t + 8) (tile rows 8..15), so a
// lane's column j and column j ^ 8 are one gate / up pair.  Weight row of tile
// row r, or -1 past the I activation columns.
KQ_DEV int swiglu_row(int t, int r, int I) {
  const int c = 8 * t + (r & 7);
  return c < I ? (r < 8 ? c : I + c) : -1;
}

// The decode epilogue with SwiGLU: the store epilogue's ((acc * xs) * ws) +
// bias for both columns of a pair, then swiglu_bits (the elementwise pass's
// roundings) -- the bits of the packed linear followed by kq_swiglu.  Lane
// (j, kg) holds column j of tile t for rows m0 + 4kg .. m0 + 4kg + 3; all 64
// lanes take part (the pair exchange is a cross-lane read).
template <int FMT>
KQ_DEV void epi_swiglu(const Epi& ep, const float* xs, int t, int m0, int j, int kg,
                       typename W8Traits<FMT>::Acc acc) {
  const int I = ep.N >> 1;
  const int n = swiglu_row(t, j, I);
  const float ws = n >= 0 ? (ep.ws_per_channel ? ep.wscale[n] : ep.wscale[0]) : 0.0f;
  const float b = n >= 0 && ep.bias_dtype != KQ_DTYPE_NONE ? load_as_f32(ep.bias, ep.bias_dtype, n) : 0.0f;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = m0 + kg * 4 + r;
    float v = 0.0f;
    if (n >= 0 && m < ep.M) {
      v = __fmul_rn(__fmul_rn((float)acc[r], xs[m]), ws);
      if (ep.bias_dtype != KQ_DTYPE_NONE) v = __fadd_rn(v, b);
    }
    const float u = __shfl_xor(v, 8, 64);
    if (j < 8 && n >= 0 && m < ep.M)
      ((uint16_t*)ep.out)[(int64_t)m * I + 8 * t + j] = swiglu_bits(v, u, ep.out_dtype);
  }
}

// Raw 32-bit pattern of accumulator element r.  (Goes through a scalar
// conversion: a bit cast applied directly to an ext-vector element selected
// element 0 for every r with this compiler.)
KQ_DEV uint32_t acc_bits(i32x4 a, int r) { return (uint32_t)(int)a[r]; }
KQ_DEV uint32_t acc_bits(f32x4 a, int r) { return __float_as_uint((float)a[r]); }

template <int FMT>
KQ_DEV typename W8Traits<FMT>::Frag load_frag(const uint8_t* p, bool lo_ok, bool hi_ok) {
  using Frag = typename W8Traits<FMT>::Frag;
  Frag f;
  if constexpr (FMT == kFmtI8) {
    f = lo_ok ? *(const i32x4*)p : i32x4{0, 0, 0, 0};
  } else {
    i32x4 lo = lo_ok ? *(const i32x4*)p : i32x4{0, 0, 0, 0};
    i32x4 hi = hi_ok ? *(const i32x4*)(p + 16) : i32x4{0, 0, 0, 0};
    f = i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  }
  return f;
}

template <int FMT>
KQ_DEV typename W8Traits<FMT>::Acc mfma_w8(typename W8Traits<FMT>::Frag a,
                                           typename W8Traits<FMT>::Frag b,
                                           typename W8Traits<FMT>::Acc c) {
  if constexpr (FMT == kFmtI8) return mfma_i8(a, b, c);
  else return mfma_fp8(a, b, c);
}

// ------------------------------------------------------------------ skinny
// Workgroup = NT tiles of 16 output columns x a K range; its waves split the
// K range.  Lane (j, kg) streams 16 (INT8) or 32 (FP8) contiguous weight
// bytes of row n = ct*16 + j of each column tile ct straight into the MFMA B
// operand, and each activation fragment (MT row tiles of 16) feeds the NT
// column tiles' MFMAs: the activation rows of a K range are read once per NT
// column tiles (x is re-read by every workgroup of a K range, so NT divides
// that traffic).  The waves' partial sums meet in LDS; the wave that owns a
// 16 x 16 block adds the eight partials in wave order (fixed order).
constexpr int kSkinnyWaves = 8;
constexpr int kSkinnyCols = 16;

template <typename T>
KQ_DEV T ldb(const void* base, uint32_t byte_off) {
  return *(const T*)((const char*)base + byte_off);
}

// PRED = false: K is a multiple of the MFMA step, so loads need no guards
// (rows beyond M / N are clamped to valid memory and never stored).
// SW: the SwiGLU epilogue (Epi::swiglu) with the weight rows of swiglu_row;
// split partials go to the [M][2I] plane by weight row, and the reduce pairs
// gate column c with up column I + c.
template <int FMT, int MT, int NT, int U, bool PRED, bool SW>
__global__ void __launch_bounds__(64 * kSkinnyWaves)
w8a8_skinny_kernel(const uint8_t* __restrict__ xq, const uint8_t* __restrict__ w, int K,
                   int steps_per_split, int splits, Epi ep, void* __restrict__ partials) {
  using T = W8Traits<FMT>;
  using Acc = typename T::Acc;
  using Frag = typename T::Frag;
  constexpr int NB = MT * NT;  // 16 x 16 output blocks of a workgroup
  __shared__ uint32_t red[kSkinnyWaves * NB * 4 * 64];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int j = lane & 15, kg = lane >> 4;
  const int tile = blockIdx.x / splits, split = blockIdx.x % splits;  // tile: NT column tiles
  const int I = ep.N >> 1;
  auto col_of = [&](int nt) -> int {  // weight row of lane column j in column tile nt, -1: none
    const int ct = tile * NT + nt;
    if constexpr (SW) return swiglu_row(ct, j, I);
    const int n = ct * kSkinnyCols + j;
    return n < ep.N ? n : -1;
  };
  const int nsteps = (K + T::kStep - 1) / T::kStep;
  const int sbeg = split * steps_per_split;
  const int send = min(nsteps, sbeg + steps_per_split);
  const int per_wave = (send - sbeg + kSkinnyWaves - 1) / kSkinnyWaves;
  const int wbeg = sbeg + wave * per_wave;
  const int wend = min(send, wbeg + per_wave);
  // loop-invariant 32-bit byte offsets (rows clamped to valid memory)
  uint32_t w_boff[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int n = col_of(nt);
    w_boff[nt] = (uint32_t)((n >= 0 ? n : ep.N - 1) * K + kg * T::kLane);
  }
  uint32_t x_boff[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) x_boff[t] = (uint32_t)(min(t * 16 + j, ep.M - 1) * K + kg * T::kLane);

  Acc acc[MT][NT];
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) acc[t][nt] = Acc{0, 0, 0, 0};

  auto frag = [&](const uint8_t* base, uint32_t off, int k) -> Frag {
    if constexpr (!PRED) {
      if constexpr (FMT == kFmtI8) {
        return ldb<i32x4>(base, off);
      } else {
        const i32x4 lo = ldb<i32x4>(base, off), hi = ldb<i32x4>(base, off + 16);
        return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
      }
    } else {
      return load_frag<FMT>(base + off, k < K, k + 16 < K);
    }
  };
  // two register batches of U steps: load batch b+1 while computing batch b
  struct Batch {
    Frag b[U][NT];
    Frag a[U][MT];
  };
  auto load = [&](Batch& bt, int st0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int st = min(st0 + u, wend - 1);  // surplus steps reload; never computed
      const int k = st * T::kStep + kg * T::kLane;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) bt.b[u][nt] = frag(w + (int64_t)st * T::kStep, w_boff[nt], k);
#pragma unroll
      for (int t = 0; t < MT; ++t) bt.a[u][t] = frag(xq + (int64_t)st * T::kStep, x_boff[t], k);
    }
  };
  auto compute = [&](const Batch& bt, int st0) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (st0 + u >= wend) break;
#pragma unroll
      for (int t = 0; t < MT; ++t)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[t][nt] = mfma_w8<FMT>(bt.a[u][t], bt.b[u][nt], acc[t][nt]);
    }
  };
  Batch b0, b1;
  if (wbeg < wend) load(b0, wbeg);
  for (int st = wbeg; st < wend; st += 2 * U) {
    if (st + U < wend) load(b1, st + U);
    compute(b0, st);
    if (st + 2 * U < wend) load(b0, st + 2 * U);
    compute(b1, st + U);
  }

  // fixed-order reduction of the waves' K ranges: every wave parks its
  // partials, then the owner of block b (wave b % 8) adds waves 0..7 in order
#pragma unroll
  for (int t = 0; t < MT; ++t)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[((wave * NB + t * NT + nt) * 4 + r) * 64 + lane] = acc_bits(acc[t][nt], r);
  __syncthreads();
  for (int bk = wave; bk < NB; bk += kSkinnyWaves) {
    const int t = bk / NT, nt = bk - t * NT;
    Acc v;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t b0 = red[((0 * NB + bk) * 4 + r) * 64 + lane];
      if constexpr (FMT == kFmtI8) v[r] = (int)b0;
      else v[r] = __uint_as_float(b0);
      for (int w2 = 1; w2 < kSkinnyWaves; ++w2) {
        const uint32_t bits = red[((w2 * NB + bk) * 4 + r) * 64 + lane];
        if constexpr (FMT == kFmtI8) v[r] += (int)bits;
        else v[r] = __fadd_rn(v[r], __uint_as_float(bits));
      }
    }
    const int n = col_of(nt);
    if (splits == 1) {
      if constexpr (SW) {
        epi_swiglu<FMT>(ep, ep.xscale, tile * NT + nt, t * 16, j, kg, v);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n >= 0) epi_store<FMT>(ep, t * 16 + kg * 4 + r, n, v, r);
      }
    } else {
      uint32_t* part = (uint32_t*)partials + (size_t)split * ep.M * ep.N;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = t * 16 + kg * 4 + r;
        if (m < ep.M && n >= 0) part[(int64_t)m * ep.N + n] = acc_bits(v, r);
      }
    }
  }
}

// ------------------------------------------------------------------ decode
// M <= 16, K a multiple of 128: a workgroup owns 16 output columns, its NW
// waves split K into contiguous ranges of 128-byte stages.  Each wave keeps a
// private ring of R LDS stages; one stage holds 128 bytes of K for the 16
// weight rows and the (up to) 16 activation rows, fetched by LDS DMA with 8
// rows x 128 bytes per instruction (whole cache lines, where direct MFMA
// fragment loads touch 16 half-lines each), and read back as MFMA fragments
// through the tile engine's chunk swizzle.  No barrier in the K loop: a wave
// only waits (vmcnt) for its own stage.  Rows beyond M or N load as zeros
// (buffer offsets past the resource), so no lane branches on shape.
template <int N_>
KQ_DEV void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N_) : "memory");
}

constexpr int kDecStage = 4096;  // 2 KB weight block + 2 KB activation block

// SW: the SwiGLU epilogue (Epi::swiglu); workgroup t holds the 16 weight rows
// of swiglu_row (the whole weight is one buffer: 2I * K < 2^31), otherwise
// rows [16t, 16t + 16).
template <int FMT, int R, int NW, int XH, bool SW>
__global__ void __launch_bounds__(64 * NW)
w8a8_decode_kernel(const uint8_t* __restrict__ xq, const uint8_t* __restrict__ w, int K, Epi ep) {
  constexpr int TF = FMT == kFmtFp8 ? kTgFp8 : kTgI8;
  constexpr int OPS = 2 + XH;  // DMA instructions per stage
  using Acc = typename W8Traits<FMT>::Acc;
  __shared__ __attribute__((aligned(16))) uint8_t ring[NW * R * kDecStage];
  __shared__ uint32_t red[(NW > 1 ? NW - 1 : 1) * 4 * 64];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int j = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * kSkinnyCols;
  const int nst = K / 128;
  const int per_wave = (nst + NW - 1) / NW;
  const int sbeg = wave * per_wave;
  const int nmy = max(0, min(nst, sbeg + per_wave) - sbeg);
  const i32x4 rw = SW ? make_rsrc(w, (uint32_t)(ep.N * K))
                      : make_rsrc(w + (int64_t)n0 * K, (uint32_t)(min(kSkinnyCols, ep.N - n0) * K));
  const i32x4 rx = make_rsrc(xq, (uint32_t)(ep.M * K));
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring +
                        wave * R * kDecStage;
  // DMA lane -> (row 8h + lane/8, physical chunk lane%8 holding logical chunk c)
  int32_t vw[2], vx[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = 8 * h + (lane >> 3), c = tg_chunk<TF>(r, lane & 7);
    if constexpr (SW) {
      const int n = swiglu_row((int)blockIdx.x, r, ep.N >> 1);
      vw[h] = n >= 0 ? n * K + c * 16 : kTgOob;
    } else {
      vw[h] = r * K + c * 16;
    }
    vx[h] = r < ep.M ? r * K + c * 16 : kTgOob;
  }
  auto issue = [&](int st, int q) {
    const uint32_t b = lds0 + q * kDecStage;
    const int32_t so = __builtin_amdgcn_readfirstlane(st * 128);
#pragma unroll
    for (int h = 0; h < 2; ++h) tg_dma16(rw, b + h * 1024, vw[h], so);
#pragma unroll
    for (int h = 0; h < XH; ++h) tg_dma16(rx, b + 2048 + h * 1024, vx[h], so);
  };
  const uint8_t* mine = ring + wave * R * kDecStage;
  if constexpr (XH == 1) {  // activation rows 8..15 are never loaded: zero once
#pragma unroll
    for (int q = 0; q < R; ++q) *(i32x4*)(mine + q * kDecStage + 3072 + lane * 16) = i32x4{0, 0, 0, 0};
  }
  const int o_lo = j * 128 + (tg_chunk<TF>(j, FMT == kFmtFp8 ? 2 * kg : kg) << 4);
  const int o_hi = j * 128 + (tg_chunk<TF>(j, FMT == kFmtFp8 ? 2 * kg + 1 : 4 + kg) << 4);

  Acc acc = Acc{0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < R - 1; ++i)
    if (i < nmy) issue(sbeg + i, i);
  for (int i = 0; i < nmy; ++i) {
    // stage i + R - 1 reuses the slot read in iteration i - 1 (its reads are
    // complete: their MFMA has consumed them)
    if (i + R - 1 < nmy) issue(sbeg + i + R - 1, (i + R - 1) % R);
    const int ahead = min(R - 1, nmy - 1 - i);  // stages issued after stage i
    if (ahead >= 3) wait_vm<3 * OPS>();
    else if (ahead == 2) wait_vm<2 * OPS>();
    else if (ahead == 1) wait_vm<OPS>();
    else wait_vm<0>();
    const uint8_t* q = mine + (i % R) * kDecStage;
    const i32x4 wl = *(const i32x4*)(q + o_lo), wh = *(const i32x4*)(q + o_hi);
    const i32x4 xl = *(const i32x4*)(q + 2048 + o_lo), xh = *(const i32x4*)(q + 2048 + o_hi);
    if constexpr (FMT == kFmtFp8) {
      acc = mfma_fp8(i32x8{xl[0], xl[1], xl[2], xl[3], xh[0], xh[1], xh[2], xh[3]},
                     i32x8{wl[0], wl[1], wl[2], wl[3], wh[0], wh[1], wh[2], wh[3]}, acc);
    } else {
      acc = mfma_i8(xl, wl, acc);
      acc = mfma_i8(xh, wh, acc);
    }
  }

  // fixed-order reduction of the waves' K ranges (wave 0 first)
  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[((wave - 1) * 4 + r) * 64 + lane] = acc_bits(acc, r);
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w2 = 1; w2 < NW; ++w2)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t bits = red[((w2 - 1) * 4 + r) * 64 + lane];
      if constexpr (FMT == kFmtI8) acc[r] += (int)bits;
      else acc[r] = __fadd_rn(acc[r], __uint_as_float(bits));
    }
  if constexpr (SW) {
    epi_swiglu<FMT>(ep, ep.xscale, (int)blockIdx.x, 0, j, kg, acc);
  } else {
#pragma unroll
    for (int r = 0; r < 4; ++r) epi_store<FMT>(ep, kg * 4 + r, n0 + j, acc, r);
  }
}

// Workgroups of a decode launch: one per 16 weight rows; with the SwiGLU
// epilogue one per 8 activation columns (8 gate + 8 up rows).
static dim3 decode_grid(const Epi& ep) {
  return ep.swiglu ? dim3((unsigned)((ep.N / 2 + 7) / 8)) : dim3((unsigned)((ep.N + kSkinnyCols - 1) / kSkinnyCols));
}

template <int FMT, int R, int NW, bool SW>
static void launch_decode_sw(const uint8_t* xq, const uint8_t* w, int K, const Epi& ep,
                             hipStream_t stream) {
  const dim3 grid = decode_grid(ep), block(64 * NW);
  if (ep.M <= 8)
    hipLaunchKernelGGL((w8a8_decode_kernel<FMT, R, NW, 1, SW>), grid, block, 0, stream, xq, w, K, ep);
  else
    hipLaunchKernelGGL((w8a8_decode_kernel<FMT, R, NW, 2, SW>), grid, block, 0, stream, xq, w, K, ep);
}

template <int FMT, int R, int NW>
static void launch_decode_nw(const uint8_t* xq, const uint8_t* w, int K, const Epi& ep,
                             hipStream_t stream) {
  if (ep.swiglu) launch_decode_sw<FMT, R, NW, true>(xq, w, K, ep, stream);
  else launch_decode_sw<FMT, R, NW, false>(xq, w, K, ep, stream);
}

// Waves and ring depth of the decode kernels.  With at least one workgroup
// per CU (N >= 16 * CUs) by the stage count, each wave keeping >= ~4 stages
// in its range, rings of 4 stages; the 2-wave form's short ranges take 3
// stages with 16-row activation stages (M > 8) and 2 otherwise: measured on
// C4's shape (N = 18944, K = 3584) M = 16 15.5 -> 15.2 us with 3, M = 4 and 8
// 3% slower with 3, and slower still with 4 or 6 stages or 4 waves; N = K =
// 4096 (one tile per CU) runs 4 waves 10% faster than 8.  With fewer tiles
// than CUs, 8 waves with 4-stage rings (Qwen2-7B q_proj, N = K = 3584: every
// stage of a tile in flight at once; 4.9 -> 4.6 us at M = 1 against the
// skinny kernel), and with at most half a tile per CU and K <= 4096, 16 waves
// of two stages with 2-stage rings (Llama-3-8B k_proj, N = 1024: every stage
// of the 64 tiles in flight at once; 6.0 -> 3.7 us at M = 1).
struct DecForm {
  int nw, r;
};

static DecForm decode_form(int64_t n, int K, int M) {
  const int64_t tiles = (n + kSkinnyCols - 1) / kSkinnyCols;
  const int cus = tg_device_cus();
  const int nst = K / 128;
  if (tiles >= (int64_t)cus) {
    if (nst >= 64) return {8, 4};
    if (nst >= 32) return {4, 4};
    return {2, M > 8 ? 3 : 2};
  }
  if (2 * tiles <= cus && nst <= 32) return {16, 2};
  return {8, 4};
}

template <int FMT>
static void launch_decode(const uint8_t* xq, const uint8_t* w, int K, const Epi& ep,
                          hipStream_t stream) {
  const DecForm f = decode_form(ep.N, K, ep.M);
  if (f.nw == 16) launch_decode_nw<FMT, 2, 16>(xq, w, K, ep, stream);
  else if (f.nw == 8) launch_decode_nw<FMT, 4, 8>(xq, w, K, ep, stream);
  else if (f.nw == 4) launch_decode_nw<FMT, 4, 4>(xq, w, K, ep, stream);
  else if (f.r == 3) launch_decode_nw<FMT, 3, 2>(xq, w, K, ep, stream);
  else launch_decode_nw<FMT, 2, 2>(xq, w, K, ep, stream);
}

// ------------------------------------------------------ decode, fused quant
// Small M with unquantized fp16 / bf16 activations: the per-token quantization
// runs inside the decode launch.  Every workgroup reads the M rows once for
// their amax (after its first weight copies are issued), then each wave copies
// 128-element slices of raw rows 0..3 into its ring next to the weights (one
// 1 KB instruction per stage), quantizes the first MR rows in place into the
// fragment layout of the plain decode kernel (64/MR lanes per row, 2*MR
// elements per lane) and runs the same MFMAs; fragment rows >= MR read a zero
// block.  The bytes are the per-token quantizers' (kq_act_quant.hip): an
// element takes the reciprocal path when it is finite and the row scale lies
// in [2^-60, FLT_MAX] (there both paths give the same byte), otherwise IEEE
// division -- decided per wave and stage, so they match the quantizer's
// row-level choice; the row scale enters in the epilogue.  SW: the SwiGLU
// epilogue and weight rows of w8a8_decode_kernel<..., true>.
template <int FMT, int R, int NW, int MR, bool SW>
__global__ void __launch_bounds__(64 * NW)
w8a8_decode_quant_kernel(const uint16_t* __restrict__ x, int x_dtype, int ldx, int scale_mode,
                         const float* __restrict__ scale_in, const uint8_t* __restrict__ w, int K,
                         Epi ep) {
  constexpr int TF = FMT == kFmtFp8 ? kTgFp8 : kTgI8;
  constexpr int OPS = 3;            // 2 weight + 1 activation DMA instructions per stage
  constexpr int LPR = 64 / MR;      // quantizing lanes per row
  constexpr int EPL = 128 / LPR;    // elements per lane and stage
  constexpr float QMAX = FMT == kFmtFp8 ? 448.0f : 127.0f;
  using Acc = typename W8Traits<FMT>::Acc;
  __shared__ __attribute__((aligned(16))) uint8_t ring[NW * R * kDecStage];
  __shared__ __attribute__((aligned(16))) uint8_t zero_rows[128];
  __shared__ uint32_t red[(NW > 1 ? NW - 1 : 1) * 4 * 64];
  __shared__ uint32_t wmax[NW][MR];
  __shared__ float srow[MR];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int j = lane & 15, kg = lane >> 4;
  const int n0 = blockIdx.x * kSkinnyCols;
  const int M = ep.M;
  const int nst = K / 128;
  const int per_wave = (nst + NW - 1) / NW;
  const int sbeg = wave * per_wave;
  const int nmy = max(0, min(nst, sbeg + per_wave) - sbeg);
  const i32x4 rw = SW ? make_rsrc(w, (uint32_t)(ep.N * K))
                      : make_rsrc(w + (int64_t)n0 * K, (uint32_t)(min(kSkinnyCols, ep.N - n0) * K));
  const i32x4 rx = make_rsrc(x, (uint32_t)(((int64_t)(M - 1) * ldx + K) * 2));
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)ring +
                        wave * R * kDecStage;
  int32_t vw[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = 8 * h + (lane >> 3), c = tg_chunk<TF>(r, lane & 7);
    if constexpr (SW) {
      const int n = swiglu_row((int)blockIdx.x, r, ep.N >> 1);
      vw[h] = n >= 0 ? n * K + c * 16 : kTgOob;
    } else {
      vw[h] = r * K + c * 16;
    }
  }
  const int xr = lane >> 4;  // raw rows 0..3, 16 chunks of 8 elements each
  const int32_t vx = xr < M ? (xr * ldx + (lane & 15) * 8) * 2 : kTgOob;
  auto issue = [&](int st, int q) {
    const uint32_t b = lds0 + q * kDecStage;
    const int32_t sw = __builtin_amdgcn_readfirstlane(st * 128);
    const int32_t sx = __builtin_amdgcn_readfirstlane(st * 256);
#pragma unroll
    for (int h = 0; h < 2; ++h) tg_dma16(rw, b + h * 1024, vw[h], sw);
    tg_dma16(rx, b + 2048, vx, sx);
  };
#pragma unroll
  for (int i = 0; i < R - 1; ++i)
    if (i < nmy) issue(sbeg + i, i);
  if (threadIdx.x < 8) *(i32x4*)(zero_rows + threadIdx.x * 16) = i32x4{0, 0, 0, 0};

  // row scales
  if (scale_mode == 0) {
#pragma unroll
    for (int r = 0; r < MR; ++r) {
      uint32_t mx = 0;
      if (r < M) {
        for (int c = (int)threadIdx.x; c < K / 8; c += 64 * NW) {
          const u32x4 raw = *(const u32x4*)(x + (int64_t)r * ldx + c * 8);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint16_t lo = (uint16_t)(raw[e] & 0xffffu), hi = (uint16_t)(raw[e] >> 16);
            const float flo = x_dtype == KQ_DTYPE_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
            const float fhi = x_dtype == KQ_DTYPE_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
            mx = max(mx, max(__float_as_uint(flo) & 0x7fffffffu, __float_as_uint(fhi) & 0x7fffffffu));
          }
        }
      }
      mx = wave_max_u32_dpp(mx);
      if (lane == 0) wmax[wave][r] = mx;
    }
    __syncthreads();
    if ((int)threadIdx.x < min(M, MR)) {
      uint32_t mx = wmax[0][threadIdx.x];
      for (int w2 = 1; w2 < NW; ++w2) mx = max(mx, wmax[w2][threadIdx.x]);
      srow[threadIdx.x] = __fdiv_rn(max_keep_nan(__uint_as_float(mx), 1e-12f), QMAX);
    }
  } else if ((int)threadIdx.x < min(M, MR)) {
    srow[threadIdx.x] = scale_mode == 1 ? scale_in[0] : scale_in[threadIdx.x];
  }
  __syncthreads();

  // this lane's quantization row and EPL-element slice of every stage
  const int qr = lane / LPR, qe = (lane % LPR) * EPL;
  const float s = qr < M ? srow[qr] : 1.0f;
  const float rs = __fdiv_rn(1.0f, s);
  const bool s_ok = s >= 0x1p-60f && s <= 3.4028235e38f;
  const int qdst = 2048 + qr * 128 + (tg_chunk<TF>(qr, qe >> 4) << 4) + (qe & 15);
  // fragment offsets: rows < MR in the stage, rows >= MR in the zero block
  const int o_lo = j * 128 + (tg_chunk<TF>(j, FMT == kFmtFp8 ? 2 * kg : kg) << 4);
  const int o_hi = j * 128 + (tg_chunk<TF>(j, FMT == kFmtFp8 ? 2 * kg + 1 : 4 + kg) << 4);
  const uint8_t* mine = ring + wave * R * kDecStage;

  Acc acc = Acc{0, 0, 0, 0};
  for (int i = 0; i < nmy; ++i) {
    if (i + R - 1 < nmy) issue(sbeg + i + R - 1, (i + R - 1) % R);
    const int ahead = min(R - 1, nmy - 1 - i);
    if (ahead >= 3) wait_vm<3 * OPS>();
    else if (ahead == 2) wait_vm<2 * OPS>();
    else if (ahead == 1) wait_vm<OPS>();
    else wait_vm<0>();
    uint8_t* q = (uint8_t*)mine + (i % R) * kDecStage;
    {
      const uint8_t* src = q + 2048 + qr * 256 + qe * 2;
      uint32_t raw[EPL / 2];
      if constexpr (EPL == 8) {
        const u32x4 t = *(const u32x4*)src;
        raw[0] = t[0]; raw[1] = t[1]; raw[2] = t[2]; raw[3] = t[3];
      } else if constexpr (EPL == 4) {
        const u32x2 t = *(const u32x2*)src;
        raw[0] = t[0]; raw[1] = t[1];
      } else {
        raw[0] = *(const uint32_t*)src;
      }
      float v[EPL];
#pragma unroll
      for (int e = 0; e < EPL / 2; ++e) {
        const uint16_t lo = (uint16_t)(raw[e] & 0xffffu), hi = (uint16_t)(raw[e] >> 16);
        v[2 * e] = x_dtype == KQ_DTYPE_BF16 ? bf16_to_f32(lo) : f16_to_f32(lo);
        v[2 * e + 1] = x_dtype == KQ_DTYPE_BF16 ? bf16_to_f32(hi) : f16_to_f32(hi);
      }
      bool fast = s_ok;
#pragma unroll
      for (int e = 0; e < EPL; ++e) fast = fast && (__float_as_uint(v[e]) & 0x7fffffffu) < 0x7f800000u;
      uint32_t b[EPL];
      if (__builtin_amdgcn_read_exec() == __ballot(fast)) {
        float t[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) t[e] = fminf(fmaxf(div_by_recip(v[e], s, rs), -QMAX), QMAX);
        if constexpr (FMT == kFmtFp8) {
#pragma unroll
          for (int e = 0; e < EPL; e += 2) {
            const uint32_t pk = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(t[e], t[e + 1], 0, false);
            b[e] = pk & 0xffu;
            b[e + 1] = (pk >> 8) & 0xffu;
          }
        } else {
#pragma unroll
          for (int e = 0; e < EPL; ++e) b[e] = (uint32_t)(int32_t)__builtin_rintf(t[e]) & 0xffu;
        }
      } else {
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
          const float t = clamp_keep_nan(__fdiv_rn(v[e], s), QMAX);
          b[e] = FMT == kFmtFp8 ? f32_to_e4m3(t) : ((uint32_t)(int32_t)__builtin_rintf(t) & 0xffu);
        }
      }
      // in place: this wave's reads of the raw slice precede its writes
      if constexpr (EPL == 8) {
        *(u32x2*)(q + qdst) = u32x2{b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24),
                                    b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24)};
      } else if constexpr (EPL == 4) {
        *(uint32_t*)(q + qdst) = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
      } else {
        *(uint16_t*)(q + qdst) = (uint16_t)(b[0] | (b[1] << 8));
      }
    }
    const uint8_t* fx = j < MR ? q + 2048 : zero_rows;
    const int xo_lo = j < MR ? o_lo : (o_lo & 127), xo_hi = j < MR ? o_hi : (o_hi & 127);
    const i32x4 wl = *(const i32x4*)(q + o_lo), wh = *(const i32x4*)(q + o_hi);
    const i32x4 xl = *(const i32x4*)(fx + xo_lo), xh = *(const i32x4*)(fx + xo_hi);
    if constexpr (FMT == kFmtFp8) {
      acc = mfma_fp8(i32x8{xl[0], xl[1], xl[2], xl[3], xh[0], xh[1], xh[2], xh[3]},
                     i32x8{wl[0], wl[1], wl[2], wl[3], wh[0], wh[1], wh[2], wh[3]}, acc);
    } else {
      acc = mfma_i8(xl, wl, acc);
      acc = mfma_i8(xh, wh, acc);
    }
  }

  if (wave > 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) red[((wave - 1) * 4 + r) * 64 + lane] = acc_bits(acc, r);
  }
  __syncthreads();
  if (wave != 0) return;
  for (int w2 = 1; w2 < NW; ++w2)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t bits = red[((w2 - 1) * 4 + r) * 64 + lane];
      if constexpr (FMT == kFmtI8) acc[r] += (int)bits;
      else acc[r] = __fadd_rn(acc[r], __uint_as_float(bits));
    }
  if constexpr (SW) {
    epi_swiglu<FMT>(ep, srow, (int)blockIdx.x, 0, j, kg, acc);
    return;
  }
  const int n = n0 + j;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = kg * 4 + r;
    if (m >= M || n >= ep.N) continue;
    float v;
    if constexpr (FMT == kFmtI8) {
      if (ep.acc_out) ep.acc_out[(int64_t)m * ep.N + n] = acc[r];
      v = (float)acc[r];
    } else {
      v = acc[r];
    }
    v = __fmul_rn(v, srow[m]);
    v = __fmul_rn(v, ep.ws_per_channel ? ep.wscale[n] : ep.wscale[0]);
    if (ep.bias_dtype != KQ_DTYPE_NONE) v = __fadd_rn(v, load_as_f32(ep.bias, ep.bias_dtype, n));
    ((uint16_t*)ep.out)[(int64_t)m * ep.N + n] = f32_to_out(v, ep.out_dtype);
  }
}

template <int FMT, int MR, bool SW>
static void launch_decode_quant_sw(const uint16_t* x, int x_dtype, int ldx, int scale_mode,
                                   const float* scale_in, const uint8_t* w, int K, const Epi& ep,
                                   hipStream_t stream) {
  const DecForm f = decode_form(ep.N, K, ep.M);
  const dim3 grid = decode_grid(ep);
  if (f.nw == 16)
    hipLaunchKernelGGL((w8a8_decode_quant_kernel<FMT, 2, 16, MR, SW>), grid, dim3(1024), 0, stream, x,
                       x_dtype, ldx, scale_mode, scale_in, w, K, ep);
  else if (f.nw == 8)
    hipLaunchKernelGGL((w8a8_decode_quant_kernel<FMT, 4, 8, MR, SW>), grid, dim3(512), 0, stream, x,
                       x_dtype, ldx, scale_mode, scale_in, w, K, ep);
  else if (f.nw == 4)
    hipLaunchKernelGGL((w8a8_decode_quant_kernel<FMT, 4, 4, MR, SW>), grid, dim3(256), 0, stream, x,
                       x_dtype, ldx, scale_mode, scale_in, w, K, ep);
  else
    hipLaunchKernelGGL((w8a8_decode_quant_kernel<FMT, 2, 2, MR, SW>), grid, dim3(128), 0, stream, x,
                       x_dtype, ldx, scale_mode, scale_in, w, K, ep);
}

template <int FMT, int MR>
static void launch_decode_quant_mr(const uint16_t* x, int x_dtype, int ldx, int scale_mode,
                                   const float* scale_in, const uint8_t* w, int K, const Epi& ep,
                                   hipStream_t stream) {
  if (ep.swiglu) launch_decode_quant_sw<FMT, MR, true>(x, x_dtype, ldx, scale_mode, scale_in, w, K, ep, stream);
  else launch_decode_quant_sw<FMT, MR, false>(x, x_dtype, ldx, scale_mode, scale_in, w, K, ep, stream);
}

// One activation row (MR = 1); the kernel also takes MR = 2 and 4.
template <int FMT>
static void launch_decode_quant(const uint16_t* x, int x_dtype, int ldx, int scale_mode,
                                const float* scale_in, const uint8_t* w, int K, const Epi& ep,
                                hipStream_t stream) {
  launch_decode_quant_mr<FMT, 1>(x, x_dtype, ldx, scale_mode, scale_in, w, K, ep, stream);
}

// ------------------------------------------------------------------- tiled
constexpr int kTile = 128;      // BM = BN = BK(bytes) = 128
constexpr int kTileBytes = kTile * kTile;

// byte offset of 16-byte chunk `c` (0..7) of row `r` in a swizzled tile
KQ_DEV int swz(int r, int c) { return r * kTile + ((c ^ (r & 7)) << 4); }

template <int FMT>
__global__ void __launch_bounds__(256)
w8a8_tile_kernel(const uint8_t* __restrict__ xq, const uint8_t* __restrict__ w, int K,
                 int tiles_n, Epi ep) {
  using T = W8Traits<FMT>;
  using Acc = typename T::Acc;
  using Frag = typename T::Frag;
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][2][kTileBytes];

  const int tid = threadIdx.x, lane = lane_id(), wave = wave_id();
  const int j = lane & 15, kg = lane >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  // grouped tile order: 8 row-tiles share each sweep over column tiles
  const int nblocks = gridDim.x;
  const int pid = xcd_swizzle(blockIdx.x, nblocks);
  const int tiles_m = (ep.M + kTile - 1) / kTile;
  const int group = 8 * tiles_n;
  const int gid = pid / group;
  const int first_m = gid * 8;
  const int gsize = min(tiles_m - first_m, 8);
  const int tm = first_m + (pid % group) % gsize;
  const int tn = (pid % group) / gsize;
  const int m0 = tm * kTile, n0 = tn * kTile;

  Acc acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b) acc[a][b] = Acc{0, 0, 0, 0};

  i32x4 ra[4], rb[4];
  auto gload = [&](int k0) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q;
      const int row = c >> 3, ch = c & 7;
      const int kc = k0 + ch * 16;
      const int m = m0 + row, n = n0 + row;
      ra[q] = (m < ep.M && kc < K) ? *(const i32x4*)(xq + (int64_t)m * K + kc) : i32x4{0, 0, 0, 0};
      rb[q] = (n < ep.N && kc < K) ? *(const i32x4*)(w + (int64_t)n * K + kc) : i32x4{0, 0, 0, 0};
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q;
      const int row = c >> 3, ch = c & 7;
      *(i32x4*)(&smem[buf][0][swz(row, ch)]) = ra[q];
      *(i32x4*)(&smem[buf][1][swz(row, ch)]) = rb[q];
    }
  };
  auto lfrag = [&](const uint8_t* s, int row, int ch0) -> Frag {
    if constexpr (FMT == kFmtI8) {
      return *(const i32x4*)(s + swz(row, ch0));
    } else {
      i32x4 lo = *(const i32x4*)(s + swz(row, ch0));
      i32x4 hi = *(const i32x4*)(s + swz(row, ch0 + 1));
      return i32x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    }
  };

  const int nk = (K + kTile - 1) / kTile;
  gload(0);
  sstore(0);
  __syncthreads();
  for (int s = 0; s < nk; ++s) {
    const int cur = s & 1;
    if (s + 1 < nk) gload((s + 1) * kTile);
    const uint8_t* sa = smem[cur][0];
    const uint8_t* sb = smem[cur][1];
    constexpr int kSteps = kTile / T::kStep;
#pragma unroll
    for (int ks = 0; ks < kSteps; ++ks) {
      const int ch0 = ks * (T::kStep / 16) + kg * (T::kLane / 16);
      Frag fa[4], fb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) fa[i] = lfrag(sa, wm * 64 + i * 16 + j, ch0);
#pragma unroll
      for (int i = 0; i < 4; ++i) fb[i] = lfrag(sb, wn * 64 + i * 16 + j, ch0);
#pragma unroll
      for (int a = 0; a < 4; ++a)
#pragma unroll
        for (int b = 0; b < 4; ++b) acc[a][b] = mfma_w8<FMT>(fa[a], fb[b], acc[a][b]);
    }
    if (s + 1 < nk) sstore(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int a = 0; a < 4; ++a)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        epi_store<FMT>(ep, m0 + wm * 64 + a * 16 + kg * 4 + r, n0 + wn * 64 + b * 16 + j,
                       acc[a][b], r);
}

// --------------------------------------------------------------- generic
// One thread per output; any K.  Used only when K is not a multiple of 16.
template <int FMT>
__global__ void w8a8_generic_kernel(const uint8_t* __restrict__ xq, const uint8_t* __restrict__ w,
                                    int K, Epi ep) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)ep.M * ep.N) return;
  const int m = (int)(idx / ep.N), n = (int)(idx % ep.N);
  typename W8Traits<FMT>::Acc acc = {0, 0, 0, 0};
  if constexpr (FMT == kFmtI8) {
    int s = 0;
    for (int k = 0; k < K; ++k)
      s += (int)(int8_t)xq[(int64_t)m * K + k] * (int)(int8_t)w[(int64_t)n * K + k];
    acc[0] = s;
  } else {
    float s = 0.0f;
    for (int k = 0; k < K; ++k)
      s = __fadd_rn(s, __fmul_rn(e4m3_to_f32(xq[(int64_t)m * K + k]),
                                 e4m3_to_f32(w[(int64_t)n * K + k])));
    acc[0] = s;
  }
  epi_store<FMT>(ep, m, n, acc, 0);
}

// ------------------------------------------------------------------ host
// Column tiles per skinny workgroup: with MT >= 2 activation row tiles the
// activation traffic of a K range (every workgroup reads all its rows)
// outweighs the weights', so NT column tiles share each activation fragment:
// FP8 4 with two row tiles and 2 with four (its 32-byte fragments in two
// register batches would spill at 4), INT8 2 with two row tiles and 4 with
// four (measured, C4's N = 18944: INT8 M = 17 / 32 29.4 / 33.0 us at 4 and
// 25.1 / 29.8 at 2, M = 64 43.3 at 4 and 45.7 at 2; FP8 N = 28672 M = 32 33.6
// at 4 and 38.7 at 2); the one-row-tile form (M <= 16 with K % 128 != 0)
// keeps NT = 1.  kSkinnyNT (the largest) bounds the split count.
constexpr int kSkinnyNT = 4;
template <int FMT, int MT>
constexpr int skinny_nt() {
  if (MT == 1) return 1;
  return (FMT == kFmtFp8) == (MT == 2) ? kSkinnyNT : 2;
}

template <int FMT, int MT>
static void launch_skinny(const uint8_t* xq, const uint8_t* w, int K, const Epi& ep,
                          void* workspace, size_t ws_bytes, hipStream_t stream) {
  using T = W8Traits<FMT>;
  constexpr int NTG = skinny_nt<FMT, MT>();
  // (SwiGLU: 8 gate + 8 up rows per column tile, as many tiles)
  const int ctiles = ep.swiglu ? (ep.N / 2 + 7) / 8 : (ep.N + kSkinnyCols - 1) / kSkinnyCols;
  const int nsteps = (K + T::kStep - 1) / T::kStep;
  const size_t plane = (size_t)ep.M * ep.N * 4;
  // Fill the 256 CUs: split K across workgroups only when there are fewer
  // tiles than CUs and every wave keeps >= 2 MFMA steps.
  auto splits_for = [&](int tiles) {
    int s = 1;
    while (workspace && tiles * s < 256 && nsteps / (s * 2 * kSkinnyWaves) >= 2 &&
           plane * s * 2 <= ws_bytes)
      s *= 2;
    return s;
  };
  // Grouped column tiles only where they keep as many workgroups as single
  // tiles do (up to 256): a small N leaves too few (N = 1024, K = 4096,
  // FP8 M = 32: 32 workgroups, 8.5 -> 11.1 us).
  const int tiles_g = (ctiles + NTG - 1) / NTG, splits_g = splits_for(tiles_g);
  const int splits_1 = splits_for(ctiles);
  const bool grouped = NTG > 1 && tiles_g * splits_g >= std::min(256, ctiles * splits_1);
  const int tiles = grouped ? tiles_g : ctiles, splits = grouped ? splits_g : splits_1;
  const int steps_per_split = (nsteps + splits - 1) / splits;
  constexpr int U1 = MT == 4 ? (FMT == kFmtI8 ? 2 : 1) : (FMT == kFmtI8 ? 4 : 2);
  constexpr int UG = FMT == kFmtI8 ? 2 : 1;
#define KQ_SKINNY(NT, U, PRED, SW)                                                                \
  hipLaunchKernelGGL((w8a8_skinny_kernel<FMT, MT, NT, U, PRED, SW>), dim3(tiles * splits),        \
                     dim3(64 * kSkinnyWaves), 0, stream, xq, w, K, steps_per_split, splits, ep, \
                     workspace)
#define KQ_SKINNY_NT(PRED, SW)                 \
  if constexpr (NTG > 1) {                       \
    if (grouped) KQ_SKINNY(NTG, UG, PRED, SW);   \
    else KQ_SKINNY(1, U1, PRED, SW);             \
  } else {                                       \
    KQ_SKINNY(1, U1, PRED, SW);                  \
  }
  if (K % T::kStep == 0) {
    if (ep.swiglu) { KQ_SKINNY_NT(false, true) }
    else { KQ_SKINNY_NT(false, false) }
  } else {
    if (ep.swiglu) { KQ_SKINNY_NT(true, true) }
    else { KQ_SKINNY_NT(true, false) }
  }
#undef KQ_SKINNY_NT
#undef KQ_SKINNY
  if (splits > 1) {
    ReduceArgs r{workspace, splits, ep.M, ep.N, ep.xscale, ep.wscale, ep.ws_per_channel,
                 ep.bias, ep.bias_dtype, ep.out, ep.out_dtype, ep.acc_out, ep.swiglu};
    launch_splitk_reduce(FMT == kFmtI8 ? kReduceI8 : kReduceFp8, r, stream);
  }
}

// Work units per 256x256 tile for the tile engine at M > 64, 0 when it does
// not apply: 1 with at least one tile per CU; otherwise the K range is split
// (2..4 ways, >= 8 K blocks each) when that fills at least half the CUs, else
// up to 8 ways with >= 4 K blocks each, where the workspace holds the
// fp32/int32 partials.  Shapes it declines take the 128x128 kernel.
static int tile_engine_splits(int64_t m, int64_t n, int K, const void* workspace, size_t ws_bytes) {
  if (m * K >= ((int64_t)1 << 31) || n * K >= ((int64_t)1 << 31)) return 0;
  const int64_t tiles = ((m + kTgBM - 1) / kTgBM) * ((n + kTgBN - 1) / kTgBN);
  const int cus = tg_device_cus();
  if (tiles >= cus) return 1;
  const int kb = (K + kTgBK - 1) / kTgBK;
  for (int s = (int)std::min<int64_t>(4, cus / tiles); s >= 2; --s)
    if (kb / s >= 8 && tiles * s * 2 >= cus && workspace &&
        (size_t)s * (size_t)(m * n) * 4 <= ws_bytes)
      return s;
  // Too few tiles to fill half the CUs that way: split K up to 8 ways (at
  // least 4 K blocks per unit) rather than run the 128x128 kernel with a
  // workgroup per 128x128 tile.  N = K = 4096 (same process, outputs
  // bit-identical): FP8 M = 128 56.1 -> 26.4 us, M = 256 55.7 -> 28.9, INT8
  // M = 128 51.1 -> 27.2; N = 1024 M = 512 45.9 -> 28.9.  (Where the rule
  // above applies, 8 ways were slower: M = 512 34.8 -> 38.8 us.)
  for (int s = (int)std::min<int64_t>(8, cus / tiles); s >= 2; --s)
    if (kb / s >= 4 && workspace && (size_t)s * (size_t)(m * n) * 4 <= ws_bytes) return s;
  return 0;
}

template <int FMT>
static int run_w8a8(const char* what, const uint8_t* xq, const uint8_t* w, int64_t m,
                    int64_t n, int64_t k, const Epi& ep, void* workspace, size_t ws_bytes,
                    hipStream_t stream) {
  if (m < 0 || n < 1 || k < 1 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff ||
      m * k > 0x7fffffffffffLL) {
    set_error("%s: bad shape m=%lld n=%lld k=%lld", what, (long long)m, (long long)n,
              (long long)k);
    return KQ_EINVAL;
  }
  if (ep.out_dtype != KQ_DTYPE_F16 && ep.out_dtype != KQ_DTYPE_BF16) {
    set_error("%s: output dtype must be fp16 or bf16", what);
    return KQ_EUNSUPPORTED;
  }
  if (m == 0) return KQ_OK;
  const int K = (int)k;
  if (ep.swiglu && !(m <= 64 && K % 16 == 0 && ((uintptr_t)xq % 16) == 0 && ((uintptr_t)w % 16) == 0 &&
                     n * k < ((int64_t)1 << 31) && m * k < ((int64_t)1 << 31))) {
    set_error("%s: the SwiGLU epilogue runs in the decode and skinny kernels only (m=%lld k=%lld)",
              what, (long long)m, (long long)k);
    return KQ_EINVAL;
  }
  if ((K % 16) != 0 || ((uintptr_t)xq % 16) || ((uintptr_t)w % 16)) {
    const int64_t total = m * n;
    hipLaunchKernelGGL(w8a8_generic_kernel<FMT>, dim3((unsigned)((total + 255) / 256)),
                       dim3(256), 0, stream, xq, w, K, ep);
    return check_launch(what);
  }
  if (m <= 64 && (n * k >= ((int64_t)1 << 32) || m * k >= ((int64_t)1 << 32))) {
    set_error("%s: weight or activation exceeds the 4 GiB addressing of the skinny kernel", what);
    return KQ_EINVAL;
  }
  if (m <= 16 && K % 128 == 0)
    launch_decode<FMT>(xq, w, K, ep, stream);
  else if (m <= 16) launch_skinny<FMT, 1>(xq, w, K, ep, workspace, ws_bytes, stream);
  else if (m <= 32) launch_skinny<FMT, 2>(xq, w, K, ep, workspace, ws_bytes, stream);
  else if (m <= 64) launch_skinny<FMT, 4>(xq, w, K, ep, workspace, ws_bytes, stream);
  else if (const int splits = tile_engine_splits(m, n, K, workspace, ws_bytes)) {
    // persistent 256x256 MFMA tiles (kq_tile_gemm.h), scales in the epilogue;
    // with fewer tiles than CUs each tile's K range is split over `splits`
    // work units whose raw accumulators the split-K reduce sums in order
    TileGemmArgs a{};
    a.x = xq; a.x_rows = (int)m; a.xs = ep.xscale; a.gather = nullptr;
    a.w = w; a.ws = ep.wscale; a.ws_per_channel = ep.ws_per_channel;
    a.mtile_table = nullptr; a.mtile_count = nullptr;
    a.M = (int)m; a.N = (int)n; a.K = K; a.I = 0;
    a.mtiles = (int)((m + kTgBM - 1) / kTgBM);
    a.ntiles = (int)((n + kTgBN - 1) / kTgBN);
    a.out = ep.out; a.out_dtype = ep.out_dtype; a.bias = ep.bias; a.bias_dtype = ep.bias_dtype;
    a.acc_out = ep.acc_out;
    a.ksplit = splits;
    a.partials = splits > 1 ? (uint32_t*)workspace : nullptr;
    tg_launch<FMT == kFmtI8 ? kTgI8 : kTgFp8, false, kTgEpiStore>(a, stream);
    if (splits > 1) {
      ReduceArgs r{workspace, splits, ep.M, ep.N, ep.xscale, ep.wscale, ep.ws_per_channel,
                   ep.bias, ep.bias_dtype, ep.out, ep.out_dtype, ep.acc_out};
      launch_splitk_reduce(FMT == kFmtI8 ? kReduceI8 : kReduceFp8, r, stream);
    }
  } else {
    const int tiles_m = (int)((m + kTile - 1) / kTile);
    const int tiles_n = (int)((n + kTile - 1) / kTile);
    hipLaunchKernelGGL(w8a8_tile_kernel<FMT>, dim3(tiles_m * tiles_n), dim3(256), 0, stream, xq,
                       w, K, tiles_n, ep);
  }
  return check_launch(what);
}

}  // namespace kq

using namespace kq;

// Rows up to which the fused decode path quantizes inside the GEMM launch.
// Every workgroup repeats the quantization of its K slices, so the saved
// launch pays only for one row (graph replay, C3 / C4 shapes: FP8 14.2 vs
// 16.2 us, INT8 15.9 vs 17.1 us at M = 1; even at M = 2; slower from M = 3).
constexpr int kFusedMaxRows = 1;

// Quantize + GEMM: the fused decode launch where it applies, otherwise the
// per-token quantizer into the workspace (bytes, then fp32 row scales) and
// the GEMM dispatch of run_w8a8 on the rest of the workspace.
template <int FMT>
static int run_linear(const char* what, const void* x, int x_dtype, int64_t ldx, int scale_mode,
                      const float* scale_in, const uint8_t* w, int64_t m, int64_t n, int64_t k,
                      Epi ep, void* workspace, size_t ws_bytes, hipStream_t stream) {
  if (x_dtype != KQ_DTYPE_F16 && x_dtype != KQ_DTYPE_BF16) {
    set_error("%s: activation dtype must be fp16 or bf16 (code %d)", what, x_dtype);
    return KQ_EUNSUPPORTED;
  }
  if (m < 0 || n < 1 || k < 1 || ldx < k || m > 0x7fffffff || n > 0x7fffffff || k > 65536) {
    set_error("%s: bad shape m=%lld n=%lld k=%lld ldx=%lld", what, (long long)m, (long long)n,
              (long long)k, (long long)ldx);
    return KQ_EINVAL;
  }
  if (ep.out_dtype != KQ_DTYPE_F16 && ep.out_dtype != KQ_DTYPE_BF16) {
    set_error("%s: output dtype must be fp16 or bf16", what);
    return KQ_EUNSUPPORTED;
  }
  if (m == 0) return KQ_OK;
  if (m > 0 && x == nullptr) {
    set_error("%s: null activation", what);
    return KQ_EINVAL;
  }
  const int K = (int)k;
  if (m <= kFusedMaxRows && K % 128 == 0 &&
      ((uintptr_t)x % 16) == 0 && (ldx % 8) == 0 && ((uintptr_t)w % 16) == 0 &&
      ((m - 1) * ldx + k) * 2 < ((int64_t)1 << 31) && n * k < ((int64_t)1 << 32)) {
    ep.xscale = nullptr;
    launch_decode_quant<FMT>((const uint16_t*)x, x_dtype, (int)ldx, scale_mode, scale_in, w, K, ep,
                             stream);
    return check_launch(what);
  }
  const size_t xq_bytes = ((size_t)m * (size_t)k + 255) / 256 * 256;
  const size_t xs_bytes = ((size_t)m * 4 + 255) / 256 * 256;
  if (workspace == nullptr || ws_bytes < xq_bytes + xs_bytes) {
    set_error("%s: workspace of %zu bytes is smaller than the %zu bytes this call needs", what,
              workspace ? ws_bytes : (size_t)0, xq_bytes + xs_bytes);
    return KQ_EWORKSPACE;
  }
  uint8_t* xq = (uint8_t*)workspace;
  float* xs = (float*)(xq + xq_bytes);
  const int rc = FMT == kFmtI8
                     ? kq_act_quant_i8(x, x_dtype, m, k, ldx, (int8_t*)xq, xs, stream)
                     : kq_act_quant_fp8(x, x_dtype, m, k, ldx, scale_in, scale_mode, xq, xs, stream);
  if (rc != KQ_OK) return rc;
  ep.xscale = xs;
  return run_w8a8<FMT>(what, xq, w, m, n, k, ep, xq + xq_bytes + xs_bytes,
                       ws_bytes - xq_bytes - xs_bytes, stream);
}

extern "C" size_t kq_w8a8_workspace_size(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0 || m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff) return 0;
  const size_t plane = (size_t)m * (size_t)n * 4;
  if (m <= 64) {
    // skinny split-K as launch_skinny doubles it (the INT8 K step is the
    // smaller one, so it bounds both formats; M > 16 groups kSkinnyNT column
    // tiles per workgroup)
    const int64_t ctiles = (n + kSkinnyCols - 1) / kSkinnyCols;
    const int64_t tiles = m > 16 ? (ctiles + kSkinnyNT - 1) / kSkinnyNT : ctiles;
    const int64_t nsteps = (k + W8Traits<kFmtI8>::kStep - 1) / W8Traits<kFmtI8>::kStep;
    int64_t s = 1;
    while (tiles * s < 256 && nsteps / (s * 2 * kSkinnyWaves) >= 2) s *= 2;
    return s > 1 ? plane * (size_t)s : 0;
  }
  const int s = tile_engine_splits(m, n, (int)k, (const void*)1, (size_t)-1);
  return s > 1 ? plane * (size_t)s : 0;
}

extern "C" int kq_w8a8_i8_gemm(const int8_t* xq, const float* xscale, const int8_t* w,
                               const float* wscale, const void* bias, int bias_dtype,
                               void* out, int out_dtype, int32_t* acc_out, int64_t m, int64_t n,
                               int64_t k, void* workspace, size_t workspace_bytes,
                               void* stream) {
  Epi ep{xscale, wscale, 1, bias, bias_dtype, out, out_dtype, acc_out, (int)m, (int)n};
  return run_w8a8<kFmtI8>("kq_w8a8_i8_gemm", (const uint8_t*)xq, (const uint8_t*)w, m, n, k, ep,
                          workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int kq_w8a8_fp8_gemm(const uint8_t* xq, const float* xscale, const uint8_t* w,
                                const float* wscale, int wscale_per_channel, const void* bias,
                                int bias_dtype, void* out, int out_dtype, int64_t m, int64_t n,
                                int64_t k, void* workspace, size_t workspace_bytes,
                                void* stream) {
  Epi ep{xscale, wscale, wscale_per_channel, bias, bias_dtype, out, out_dtype, nullptr,
         (int)m, (int)n};
  return run_w8a8<kFmtFp8>("kq_w8a8_fp8_gemm", xq, w, m, n, k, ep, workspace, workspace_bytes,
                           (hipStream_t)stream);
}

extern "C" size_t kq_w8a8_linear_workspace_size(int64_t m, int64_t n, int64_t k) {
  if (m <= 0 || n <= 0 || k <= 0) return 0;
  return ((size_t)m * (size_t)k + 255) / 256 * 256 + ((size_t)m * 4 + 255) / 256 * 256 +
         kq_w8a8_workspace_size(m, n, k);
}

extern "C" int kq_w8a8_i8_linear(const void* x, int x_dtype, int64_t ldx, const int8_t* w,
                                 const float* wscale, const void* bias, int bias_dtype, void* out,
                                 int out_dtype, int32_t* acc_out, int64_t m, int64_t n, int64_t k,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  Epi ep{nullptr, wscale, 1, bias, bias_dtype, out, out_dtype, acc_out, (int)m, (int)n};
  return run_linear<kFmtI8>("kq_w8a8_i8_linear", x, x_dtype, ldx, 0, nullptr,
                            (const uint8_t*)w, m, n, k, ep, workspace, workspace_bytes,
                            (hipStream_t)stream);
}

extern "C" int kq_w8a8_fp8_linear(const void* x, int x_dtype, int64_t ldx, const float* scale_in,
                                  int scale_mode, const uint8_t* w, const float* wscale,
                                  int wscale_per_channel, const void* bias, int bias_dtype,
                                  void* out, int out_dtype, int64_t m, int64_t n, int64_t k,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  if (scale_mode < 0 || scale_mode > 2 || (scale_mode != 0 && scale_in == nullptr)) {
    set_error("kq_w8a8_fp8_linear: bad scale_mode %d", scale_mode);
    return KQ_EINVAL;
  }
  Epi ep{nullptr, wscale, wscale_per_channel, bias, bias_dtype, out, out_dtype, nullptr, (int)m,
         (int)n};
  return run_linear<kFmtFp8>("kq_w8a8_fp8_linear", x, x_dtype, ldx, scale_mode, scale_in, w, m, n,
                             k, ep, workspace, workspace_bytes, (hipStream_t)stream);
}

// ------------------------------------------------------------------ SwiGLU
// A packed (gate, up) projection with SwiGLU, out[m][c] = silu(g) * up for
// gate column c and up column I + c of the packed weight w [2I][K] (the
// reference MLP's act_fn(gate(x)) * up(x), kairyu/models/layers.py:243-244,
// over its packed projections, kairyu/models/packed_linear.py:58-149).
// Prefill shapes (M > 64, I % 128 == 0, enough 256 x 256 tiles for half the
// CUs) run the tile engine with the SwiGLU store epilogue: each tile pairs
// gate columns [n0, n0 + 128) with up columns [I + n0, I + n0 + 128), so the
// [M, 2I] projection output never reaches memory.  Shapes of M <= 64 run the
// decode or skinny kernels with the SwiGLU epilogue (each workgroup's 16
// weight rows are 8 gate rows and the matching 8 up rows; split-K partials
// meet in the reduce, which pairs the columns).  Other shapes run the packed
// linear into the workspace and the elementwise pass.  All produce the bits
// of the packed linear followed by kq_swiglu.
static bool swiglu_fused_applies(int64_t m, int64_t i_width, int64_t k, const void* x, int64_t ldx,
                                 const void* w) {
  if (m <= 64 || i_width % 128 != 0 || k % 16 != 0 || ((uintptr_t)w % 16) != 0) return false;
  if (m * k >= ((int64_t)1 << 31) || 2 * i_width * k >= ((int64_t)1 << 31)) return false;
  const int64_t tiles = ((m + kTgBM - 1) / kTgBM) * (i_width / 128);
  return 2 * tiles >= tg_device_cus();
}

template <int FMT>
static int run_swiglu_linear(const char* what, const void* x, int x_dtype, int64_t ldx, int scale_mode,
                             const float* scale_in, const uint8_t* w, const float* wscale,
                             int ws_per_channel, const void* bias, int bias_dtype, void* out,
                             int64_t m, int64_t i_width, int64_t k, void* workspace, size_t ws_bytes,
                             hipStream_t stream) {
  if (i_width < 1 || i_width > 0x3fffffff) {
    set_error("%s: bad width %lld", what, (long long)i_width);
    return KQ_EINVAL;
  }
  const int64_t n = 2 * i_width;
  Epi ep{nullptr, wscale, ws_per_channel, bias, bias_dtype, out, x_dtype, nullptr, (int)m, (int)n};
  if (m > 0 && m <= 0x7fffffff && k >= 1 && k <= 65536 && ldx >= k && x != nullptr &&
      (x_dtype == KQ_DTYPE_F16 || x_dtype == KQ_DTYPE_BF16) &&
      swiglu_fused_applies(m, i_width, k, x, ldx, w)) {
    const size_t xq_bytes = ((size_t)m * (size_t)k + 255) / 256 * 256;
    const size_t xs_bytes = ((size_t)m * 4 + 255) / 256 * 256;
    if (workspace == nullptr || ws_bytes < xq_bytes + xs_bytes) {
      set_error("%s: workspace of %zu bytes is smaller than the %zu bytes this call needs", what,
                workspace ? ws_bytes : (size_t)0, xq_bytes + xs_bytes);
      return KQ_EWORKSPACE;
    }
    uint8_t* xq = (uint8_t*)workspace;
    float* xs = (float*)(xq + xq_bytes);
    const int rc = FMT == kFmtI8
                       ? kq_act_quant_i8(x, x_dtype, m, k, ldx, (int8_t*)xq, xs, stream)
                       : kq_act_quant_fp8(x, x_dtype, m, k, ldx, scale_in, scale_mode, xq, xs, stream);
    if (rc != KQ_OK) return rc;
    TileGemmArgs a{};
    a.x = xq; a.x_rows = (int)m; a.xs = xs; a.gather = nullptr;
    a.w = w; a.ws = wscale; a.ws_per_channel = ws_per_channel;
    a.mtile_table = nullptr; a.mtile_count = nullptr;
    a.M = (int)m; a.N = (int)n; a.K = (int)k; a.I = (int)i_width;
    a.mtiles = (int)((m + kTgBM - 1) / kTgBM);
    a.ntiles = (int)(i_width / 128);
    a.out = out; a.out_dtype = x_dtype; a.bias = bias; a.bias_dtype = bias_dtype;
    a.acc_out = nullptr;
    a.ksplit = 1;
    tg_launch<FMT == kFmtI8 ? kTgI8 : kTgFp8, false, kTgEpiSwiGluStore>(a, stream);
    return check_launch(what);
  }
  if (m >= 1 && m <= 64 && k % 16 == 0 && k <= 65536 && ((uintptr_t)w % 16) == 0 &&
      ((uintptr_t)workspace % 16) == 0 && n * k < ((int64_t)1 << 31)) {
    // decode shapes: the decode or skinny kernels (one-row fused quantization
    // or the per-token quantizer first) with the SwiGLU epilogue
    ep.swiglu = 1;
    return run_linear<FMT>(what, x, x_dtype, ldx, scale_mode, scale_in, w, m, n, k, ep, workspace,
                           ws_bytes, stream);
  }
  // two passes: the packed projection [m][2I] in the activation dtype, then SwiGLU
  const size_t tmp_bytes = ((size_t)(m > 0 ? m : 0) * (size_t)n * 2 + 255) / 256 * 256;
  if (m > 0 && (workspace == nullptr || ws_bytes < tmp_bytes)) {
    set_error("%s: workspace of %zu bytes is smaller than the %zu bytes this call needs", what,
              workspace ? ws_bytes : (size_t)0, tmp_bytes);
    return KQ_EWORKSPACE;
  }
  ep.out = workspace;
  const int rc = run_linear<FMT>(what, x, x_dtype, ldx, scale_mode, scale_in, w, m, n, k, ep,
                                 (uint8_t*)workspace + tmp_bytes, ws_bytes - tmp_bytes, stream);
  if (rc != KQ_OK || m == 0) return rc;
  return kq_swiglu(workspace, n, 0, x_dtype, out, m, i_width, stream);
}

extern "C" size_t kq_w8a8_swiglu_workspace_size(int64_t m, int64_t i_width, int64_t k) {
  if (m <= 0 || i_width <= 0 || k <= 0) return 0;
  const size_t fused = ((size_t)m * (size_t)k + 255) / 256 * 256 + ((size_t)m * 4 + 255) / 256 * 256;
  const size_t tmp = ((size_t)m * (size_t)(2 * i_width) * 2 + 255) / 256 * 256;
  return std::max(fused, tmp + kq_w8a8_linear_workspace_size(m, 2 * i_width, k));
}

extern "C" int kq_w8a8_i8_swiglu_linear(const void* x, int x_dtype, int64_t ldx, const int8_t* w,
                                        const float* wscale, const void* bias, int bias_dtype, void* out,
                                        int64_t m, int64_t i_width, int64_t k, void* workspace,
                                        size_t workspace_bytes, void* stream) {
  return run_swiglu_linear<kFmtI8>("kq_w8a8_i8_swiglu_linear", x, x_dtype, ldx, 0, nullptr,
                                   (const uint8_t*)w, wscale, 1, bias, bias_dtype, out, m, i_width, k,
                                   workspace, workspace_bytes, (hipStream_t)stream);
}

extern "C" int kq_w8a8_fp8_swiglu_linear(const void* x, int x_dtype, int64_t ldx, const float* scale_in,
                                         int scale_mode, const uint8_t* w, const float* wscale,
                                         int wscale_per_channel, const void* bias, int bias_dtype,
                                         void* out, int64_t m, int64_t i_width, int64_t k,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  if (scale_mode < 0 || scale_mode > 2 || (scale_mode != 0 && scale_in == nullptr)) {
    set_error("kq_w8a8_fp8_swiglu_linear: bad scale_mode %d", scale_mode);
    return KQ_EINVAL;
  }
  return run_swiglu_linear<kFmtFp8>("kq_w8a8_fp8_swiglu_linear", x, x_dtype, ldx, scale_mode, scale_in,
                                    w, wscale, wscale_per_channel, bias, bias_dtype, out, m, i_width, k,
                                    workspace, workspace_bytes, (hipStream_t)stream);
}
