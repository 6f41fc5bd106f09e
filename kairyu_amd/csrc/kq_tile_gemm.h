// Persistent fp8 / int8 MFMA tile engine for gfx950.
//
//   D[m, n] = sum_k X[m, k] * W[n, k]        (X: activation rows, W: weight rows,
//                                            both K-contiguous bytes)
//
// Used by the grouped block-FP8 MoE expert GEMMs, the dense block-FP8 linear
// and the W8A8 (FP8 / INT8) prefill GEMMs.
//
// Work decomposition
//   * Tiles of BM = 64 * NRB activation rows x 256 weight rows: NRB = 4
//     (256 rows) for the dense GEMMs, NRB = 5 (320 rows) for MoE experts of
//     many rows, where one 320-row tile holds every row of an expert at an
//     even top-8 routing (≈256 ± 50 rows) that 256-row tiles split into a
//     full tile and a tail of a few rows streaming the same weights (MoE
//     experts of fewer rows take NRB = 4).  The grid is persistent
//     (one 512-thread workgroup per CU).  Workgroup b runs on XCD b % 8; XCD x
//     owns the contiguous slice [x*T/8, (x+1)*T/8) of the T tiles, walked by
//     its workgroups in order, so the 32 tiles an XCD has in flight are
//     neighbours: the column tiles of one row tile (shared activation rows)
//     and the row tiles of one expert / column range (shared weight rows) meet
//     in that XCD's L2.  T may come from device memory (MoE: the number of
//     row tiles the routing produced), so the host launches no empty tiles.
//   * Eight waves: wn = wave / 4 owns 128 weight rows (8 blocks of 16),
//     wm = wave % 4 owns the NRB activation row blocks 4 * mb + wm (16 rows
//     each; interleaved, so a ragged tile's rows spread over the four SIMDs).
//     Weights are the MFMA A operand and activations the B operand, so a
//     lane's four results are four consecutive output columns of one row: one
//     activation scale and one weight scale cover all four (one multiply per
//     16x16 block and K block for block scaling), and stores are 8 bytes wide.
//
// Memory pipeline
//   K advances in 128-byte blocks.  W blocks (32 KB) and X blocks (BM x 128
//   bytes) move global -> LDS with buffer_load ... lds (no registers),
//   double-buffered: block kb+1 is in flight while kb is multiplied.  Rows are 128 bytes in LDS, their
//   16-byte chunks permuted by an XOR of row bits chosen per operand pattern
//   (measured with ds_read_b128 on gfx950: FP8 lanes read chunk pairs
//   (2g, 2g+1) of 16 rows -> c ^ (r & 7) ^ ((r >> 3) & 1); INT8 lanes read
//   chunks g and 4+g -> c ^ ((r >> 1) & 7); both run at the conflict-free
//   rate, where c ^ (r & 7) alone costs 1.7x).  A DMA lane writes LDS slot
//   M0 + 16 * lane, so each lane fetches the global chunk that belongs in its
//   slot.
//
// Numerics
//   FP8, block scales : per K block t = mfma(Wq, Xq) (exact e4m3 products, fp32
//                       sums), acc = fma(t, xs[m, kb] * ws[n/128, kb], acc).
//   FP8, plain        : acc accumulates in the MFMA; the epilogue applies
//                       ((acc * xs[m]) * ws[n]) (+ bias) with separate roundings.
//   INT8              : int32 accumulation, exact; same epilogue on fp32(acc).
#pragma once

#include "kq_common.h"

#include <type_traits>

namespace kq {

constexpr int kTgBM = 256;        // activation rows per tile of the dense GEMMs (NRB = 4)
constexpr int kTgBN = 256;        // weight rows per tile
constexpr int kTgBK = 128;        // K bytes per pipeline stage (one block-scale block)
constexpr int kTgThreads = 512;
constexpr int kTgMaxKB = 128;     // K <= 16384 for block scaling (weight scale rows in LDS)
constexpr int32_t kTgOob = (int32_t)0x80000000u;  // buffer offset past every resource: reads 0
constexpr int kTgGroupM = 8;  // dense tile order: row tiles per group
constexpr int kTgLag = 2;     // block scaling: MFMAs between a result and its scale FMA

enum { kTgFp8 = 0, kTgI8 = 1 };
// Epilogues: store the outputs; SwiGLU of each gate / up column pair
// quantized to e4m3 1x128 blocks (MoE gate_up); SwiGLU of each pair stored
// in the activation dtype (a dense packed gate / up projection).  Both SwiGLU
// forms pair weight rows [n0, n0 + 128) with [I + n0, I + n0 + 128).
enum { kTgEpiStore = 0, kTgEpiSwiGluQuant = 1, kTgEpiSwiGluStore = 2 };

// LDS map (bytes) of a tile of 64 * NRB activation rows
template <int NRB>
struct TgLds {
  static constexpr int BM = 64 * NRB;
  static constexpr int W = 0;                           // 2 stages x 256 weight rows x 128
  static constexpr int X = W + 2 * kTgBN * kTgBK;       // 2 stages x BM activation rows x 128
  static constexpr int Xs = X + 2 * BM * kTgBK;         // 2 stages x BM activation block scales
  static constexpr int Ws = Xs + 2 * BM * 4;            // 2 tiles x 2 weight-scale rows x kTgMaxKB
  static constexpr int Red = Ws + 4 * kTgMaxKB * 4;     // 2 x BM row maxima (SwiGLU quant)
  static constexpr int Epi = Red + 2 * BM * 4;          // 2 tiles x {row scale, column scale, bias} x 256
  static constexpr int Gat = Epi + 2 * 3 * 256 * 4;     // the next tile's BM row sources (gathered rows)
  static constexpr int Bytes = Gat + BM * 4;
  static_assert(Bytes <= 160 * 1024, "the tile's LDS exceeds a CU's 160 KB");
};

struct TileGemmArgs {
  // activations (MFMA B operand)
  const uint8_t* x;          // [x_rows][K]
  int x_rows;                // rows addressable through x (buffer bound)
  const float* xs;           // block scaling: [x_rows][ceil(K/128)]; otherwise per-row scale [M]
  const int32_t* gather;     // tile row -> source row of x; null: identity
  int gather_rows;           // entries of gather
  // weights (MFMA A operand)
  const uint8_t* w;          // [E][N][K]
  const float* ws;           // block scaling: [E][ceil(N/128)][K/128]; otherwise [N] or [1]
  int ws_per_channel;
  // tiles: row tile i covers rows [row0, row_end) of expert e
  const int32_t* mtile_table;   // [mtiles][4] (expert, first row, end row, 0); null: dense rows 256*i
  const int32_t* mtile_count;   // device count of row tiles in use; null: mtiles
  int mtiles, ntiles;
  int M;                     // dense row count (mtile_table == null)
  int N, K, I;               // weight rows, K bytes, activation width I (SwiGLU: N = 2I)
  // epilogue
  void* out;                 // [rows][N] in out_dtype
  int out_dtype;
  const void* bias;          // [N] or null
  int bias_dtype;
  int32_t* acc_out;          // INT8: raw int32 accumulators [M][N] or null (store epilogue)
  int ksplit;                // dense, per-channel scales only: K split across this many
                             // work units per tile (0/1: none); each stores raw 32-bit
  uint32_t* partials;        // accumulators to partials[split][M][N], reduced afterwards
  uint8_t* actq;             // SwiGLU: e4m3 activations [rows][I]
  float* acts;               // SwiGLU: their 1x128 block scales [rows][I/128]
};

// physical 16-byte chunk of logical chunk c in LDS row r (an involution)
template <int FMT>
KQ_DEV int tg_chunk(int r, int c) {
  if constexpr (FMT == kTgFp8) return c ^ (r & 7) ^ ((r >> 3) & 1);
  else return c ^ ((r >> 1) & 7);
}

// Output staging rows of 128 bytes (the epilogues): unit u of row r at unit
// u ^ (r & 15) (8-byte units) or u ^ ((r & 15) << 1) (4-byte units).  The
// 16 consecutive lanes of an epilogue write hold the same unit of 16 rows;
// XOR-ing by the row puts them on 16 distinct units, i.e. all 32 four-byte
// banks of a 128-byte bank row.  (A permutation of 16-byte chunks leaves the
// 16 lanes on 8 chunks at one half-chunk offset: a two-way conflict on every
// staging write, 0.46 of the MoE down GEMM's LDS-active cycles.)  The
// read-back takes row r's 16-byte chunk c from chunk c ^ ((r & 15) >> 1),
// whose two 8-byte halves are swapped when r is odd.
KQ_DEV int tg_stage_off8(int r, int u) { return r * 128 + ((u ^ (r & 15)) << 3); }
KQ_DEV int tg_stage_off4(int r, int u) { return r * 128 + ((u ^ ((r & 15) << 1)) << 2); }
KQ_DEV i32x4 tg_stage_read(const uint8_t* stg, int r, int c) {
  const i32x4 v = *(const i32x4*)(stg + r * 128 + ((c ^ ((r & 15) >> 1)) << 4));
  return (r & 1) ? i32x4{v[2], v[3], v[0], v[1]} : v;
}

// Global -> LDS copies of 16 / 4 bytes per lane (buffer_load ... lds): lane i
// of the wave writes at LDS byte address lds + i * size; `lds` is wave-uniform
// (the compiler places it in m0).
typedef __attribute__((address_space(3))) void* tg_lds_ptr;
KQ_DEV void tg_dma16(i32x4 rsrc, uint32_t lds, int32_t voff, int32_t soff) {
  kq_rbl_lds(rsrc, (tg_lds_ptr)(uintptr_t)lds, 16, voff, soff, 0, 0);
}
// The same with the non-temporal hint: weights that one work unit streams
// once (MoE experts: each expert's rows meet one or two row tiles).
KQ_DEV void tg_dma16nt(i32x4 rsrc, uint32_t lds, int32_t voff, int32_t soff) {
  kq_rbl_lds(rsrc, (tg_lds_ptr)(uintptr_t)lds, 16, voff, soff, 0, kAuxNT);
}
KQ_DEV void tg_dma4(i32x4 rsrc, uint32_t lds, int32_t voff, int32_t soff) {
  kq_rbl_lds(rsrc, (tg_lds_ptr)(uintptr_t)lds, 4, voff, soff, 0, 0);
}

// Two values rounded (to nearest even) to the 16-bit dtype and packed, low
// half first: one v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32.
typedef __bf16 tg_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 tg_f16x2 __attribute__((ext_vector_type(2)));
typedef float tg_f32x2 __attribute__((ext_vector_type(2)));
KQ_DEV uint32_t tg_pack2(float lo, float hi, int dtype) {
  const tg_f32x2 v = {lo, hi};
  if (dtype == KQ_DTYPE_BF16) return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, tg_bf16x2));
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, tg_f16x2));
}
// The two values of a packed pair, widened to fp32.
KQ_DEV float tg_lo(uint32_t p, int dtype) {
  if (dtype == KQ_DTYPE_BF16) return __uint_as_float(p << 16);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)p);
}
KQ_DEV float tg_hi(uint32_t p, int dtype) {
  if (dtype == KQ_DTYPE_BF16) return __uint_as_float(p & 0xffff0000u);
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(p >> 16));
}


template <int FMT> struct TgTraits;
template <> struct TgTraits<kTgFp8> { using Acc = f32x4; };
template <> struct TgTraits<kTgI8> { using Acc = i32x4; };

// Operand fragment of one 16-row block: FP8 uses chunks 2g, 2g+1 (32 bytes of
// K 32g..32g+31 for the 16x16x128 MFMA); INT8 uses chunk g (K 16g..) for the
// first 16x16x64 MFMA and chunk 4+g for the second.
struct TgFrag {
  i32x4 lo, hi;
};

KQ_DEV TgFrag tg_load(const uint8_t* blk, int off_lo, int off_hi) {
  TgFrag f;
  f.lo = *(const i32x4*)(blk + off_lo);
  f.hi = *(const i32x4*)(blk + off_hi);
  return f;
}

// Wave-uniform description of one tile.
struct TgTile {
  int e, row0, row_end, ntile;
  int split, kb0, kb1;  // K blocks [kb0, kb1) of this work unit
};

// WNT: weight copies carry the non-temporal hint (the MoE GEMMs, whose
// 600 MB of expert weights otherwise displace the expert outputs the combine
// reads next from the MALL: C5 292 -> 282 us).
template <int FMT, bool BLOCK, int EPI, int NRB, bool WNT>
__global__ void __launch_bounds__(kTgThreads)
tile_gemm_kernel(TileGemmArgs a) {
  // 320-row tiles only where no per-row epilogue constants are needed
  static_assert(NRB == 4 || (NRB == 5 && BLOCK), "row blocks per wave: 4, or 5 with block scaling");
  using Acc = typename TgTraits<FMT>::Acc;
  using L = TgLds<NRB>;
  constexpr int BM = L::BM;
  __shared__ __attribute__((aligned(16))) uint8_t smem[L::Bytes];
  const int lane = lane_id();
  const int wave = __builtin_amdgcn_readfirstlane(wave_id());
  const int wn = wave >> 2, wm = wave & 3;
  const int lr = lane & 15, lg = lane >> 4;
  const uint32_t lds0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) uint8_t*)smem;
  const int K = a.K;
  const int KB = (K + kTgBK - 1) / kTgBK;
  const int ktail = K - (KB - 1) * kTgBK;  // bytes of K in the last block (16..128)
  const int NB = (a.N + 127) / 128;

  const int mt_used = a.mtile_count ? __builtin_amdgcn_readfirstlane(*a.mtile_count) : a.mtiles;
  const int ksplit = (!BLOCK && EPI == kTgEpiStore && !a.mtile_table && a.ksplit > 1) ? a.ksplit : 1;
  const int tiles = min(mt_used, a.mtiles) * a.ntiles;
  const int total = tiles * ksplit;
  const int xcd = blockIdx.x & 7, per = gridDim.x >> 3, slot = blockIdx.x >> 3;
  const int t_lo = (int)((int64_t)total * xcd / 8), t_hi = (int)((int64_t)total * (xcd + 1) / 8);
  int t = t_lo + slot;
  if (t >= t_hi) return;

  const i32x4 rx = make_rsrc(a.x, (uint32_t)((uint64_t)a.x_rows * K));
  const i32x4 rxs = make_rsrc(a.xs, BLOCK ? (uint32_t)((uint64_t)a.x_rows * KB * 4) : 0u);
  const i32x4 rtab = make_rsrc(a.mtile_table, a.mtile_table ? (uint32_t)a.mtiles * 16u : 0u);
  const i32x4 rgat = make_rsrc(a.gather, a.gather ? (uint32_t)((uint64_t)a.gather_rows * 4) : 0u);
  // block scales: every offset below addresses a weight-scale row of an
  // expert in the tile table (the buffer bound is not the check)
  const i32x4 rws = make_rsrc(a.ws, BLOCK ? 0x7fffffffu : 0u);

  // lane-constant parts of the operand reads: row lr of a 16-row block
  const int o_lo = lr * kTgBK + (tg_chunk<FMT>(lr, FMT == kTgFp8 ? 2 * lg : lg) << 4);
  const int o_hi = lr * kTgBK + (tg_chunk<FMT>(lr, FMT == kTgFp8 ? 2 * lg + 1 : 4 + lg) << 4);

  float* sRed = (float*)(smem + L::Red);

  // ---- tile metadata.  A row tile's table entry is (expert, first row, end
  // row, 0); lane l < 3 of a table word holds entry word l.
  auto load_tab = [&](int tt) -> int {
    if (!a.mtile_table) return 0;
    return kq_rbl_i32(rtab, (4 * ((tt % tiles) / a.ntiles) + (lane & 3)) * 4, 0, 0);
  };
  auto tile_of = [&](int tt, int tab) -> TgTile {
    TgTile r;
    // split s of every tile before split s + 1: an XCD's range shares K blocks
    r.split = tt / tiles;
    tt -= r.split * tiles;
    r.kb0 = (int)((int64_t)KB * r.split / ksplit);
    r.kb1 = (int)((int64_t)KB * (r.split + 1) / ksplit);
    if (a.mtile_table) {
      r.ntile = tt % a.ntiles;
      r.e = __builtin_amdgcn_readlane(tab, 0);
      r.row0 = __builtin_amdgcn_readlane(tab, 1);
      r.row_end = __builtin_amdgcn_readlane(tab, 2);
    } else {
      // dense: groups of kTgGroupM row tiles, row tile fastest, so an XCD's
      // contiguous range of tiles covers a near-square block of the output
      // (its operand rows come through its own L2 once) instead of a few row
      // tiles against every weight row
      const int gsz = kTgGroupM * a.ntiles, g = tt / gsz, rr = tt - g * gsz;
      const int gm = min(kTgGroupM, a.mtiles - g * kTgGroupM);
      r.ntile = rr / gm;
      r.e = 0;
      r.row0 = (g * kTgGroupM + rr % gm) * BM;
      r.row_end = min(a.M, r.row0 + BM);
    }
    return r;
  };
  // the two 128-row weight-scale blocks a tile spans: SwiGLU the gate and the
  // up block of activation columns ntile*128; otherwise n0/128 and the next
  auto scale_block = [&](const TgTile& tl, int half) -> int {
    if constexpr (EPI == kTgEpiSwiGluQuant) return half ? (a.I + tl.ntile * 128) / 128 : tl.ntile;
    else return min(tl.ntile * 2 + half, NB - 1);
  };

  // ---- per-tile loads, issued one tile ahead so that they land under the
  // current tile's K loop.  Row sources (gathered rows) and block weight
  // scales move global -> LDS by DMA (no registers held across the K loop);
  // the store epilogue's constants load into registers.
  float pf_exs = 1.0f, pf_ews = 1.0f, pf_eb = -0.0f;  // (no bias: adds -0.0, the identity)
  auto prefetch = [&](const TgTile& tl, int wsbuf) {
    if (a.gather && wave < NRB) {
      // LDS int t of the Gat region holds tile row t's flat routed row
      const int r = tl.row0 + 64 * wave + lane;
      tg_dma4(rgat, lds0 + L::Gat + wave * 256, r < tl.row_end ? r * 4 : kTgOob, 0);
    }
    if (BLOCK && 64 * wave < 2 * KB) {
      // LDS float t of weight-scale buffer wsbuf: t < KB the first 128-row
      // block's scale of K block t, then the second block's
      const int tt = (int)threadIdx.x, half = tt >= KB, kb = tt - half * KB;
      const int off = tt < 2 * KB ? ((tl.e * NB + scale_block(tl, half)) * KB + kb) * 4 : kTgOob;
      tg_dma4(rws, lds0 + L::Ws + wsbuf * (2 * kTgMaxKB * 4) + wave * 256, off, 0);
    }
    if (EPI != kTgEpiSwiGluQuant && threadIdx.x < 256) {
      // epilogue constants of tile row / column t: loaded here, one tile
      // ahead, so the epilogue issues no global loads between its stores
      // (loads and stores share vmcnt: a load would wait for every store).
      // SwiGLU store: column t < 128 is gate column ntile * 128 + t, the
      // others the up columns I + ntile * 128 + t - 128.
      const int t = (int)threadIdx.x, r = tl.row0 + t;
      const int n = EPI == kTgEpiSwiGluStore ? min((t >> 7) * a.I + tl.ntile * 128 + (t & 127), a.N - 1)
                                             : min(tl.ntile * kTgBN + t, a.N - 1);
      if (!BLOCK) {
        pf_exs = r < tl.row_end ? a.xs[r] : 0.0f;
        pf_ews = a.ws_per_channel ? a.ws[n] : a.ws[0];
      }
      if (a.bias_dtype != KQ_DTYPE_NONE) pf_eb = load_as_f32(a.bias, a.bias_dtype, n);
    }
  };

  // ---- DMA state of the tile being loaded (after its prefetch has landed)
  i32x4 rw;
  int32_t w_off[4], x_off[NRB], xs_off = kTgOob;
  const int32_t* sGat = (const int32_t*)(smem + L::Gat);
  auto row_src = [&](const TgTile& tl, int row) -> int {
    const int r = tl.row0 + row;
    return r < tl.row_end ? (a.gather ? sGat[row] : r) : -1;
  };
  auto set_offsets = [&](const TgTile& tl) {
    rw = make_rsrc(a.w + (int64_t)tl.e * a.N * K, (uint32_t)((uint64_t)a.N * K));
    // lane terms formed per tile (see the epilogue)
    int ln = lane;
    asm volatile("" : "+v"(ln));
    // this wave fills 1 KB blocks 4*wave+i of each 32 KB weight stage and
    // NRB*wave+i of each activation stage; slot p = block*64 + lane is row
    // p/8, physical chunk p%8
#pragma unroll
    for (int i = 0; i < NRB; ++i) {
      const int p = (wave * NRB + i) * 64 + ln, row = p >> 3;
      const int src = row_src(tl, row);
      x_off[i] = src >= 0 ? src * K + tg_chunk<FMT>(row, p & 7) * 16 : kTgOob;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int p = (wave * 4 + i) * 64 + ln, row = p >> 3;
      const int c = tg_chunk<FMT>(row, p & 7);
      int n;
      if constexpr (EPI != kTgEpiStore) {
        // wave half wn: blocks j < 4 gate rows, j >= 4 up rows of activation
        // columns ntile*128 + 64*wn + 16*(j&3) + (row&15)
        const int j = (row >> 4) & 7;
        const int col = tl.ntile * 128 + 64 * (row >> 7) + 16 * (j & 3) + (row & 15);
        n = j < 4 ? col : a.I + col;
      } else {
        n = tl.ntile * kTgBN + row;
      }
      w_off[i] = n < a.N ? n * K + c * 16 : kTgOob;
    }
    if (BLOCK && wave < NRB) {
      // LDS scale float r of a stage holds tile row r (64 rows per wave)
      const int src = row_src(tl, 64 * wave + ln);
      xs_off = src >= 0 ? src * KB * 4 : kTgOob;
    }
  };
  auto stage_ws = [&](int buf) {
    if (EPI != kTgEpiSwiGluQuant && threadIdx.x < 256) {
      float* e = (float*)(smem + L::Epi) + buf * 3 * 256 + (int)threadIdx.x;
      e[0] = pf_exs;
      e[256] = pf_ews;
      e[512] = pf_eb;
    }
  };
  auto issue = [&](int kb, int st) {
    const uint32_t lw = lds0 + L::W + st * (kTgBN * kTgBK) + wave * 4096;
    const uint32_t lx = lds0 + L::X + st * (BM * kTgBK) + wave * (NRB * 1024);
    const int soff = kb * kTgBK;
    if (!BLOCK && kb == KB - 1 && ktail < kTgBK) {
      // ragged last block: chunks past K read zeros (K % 16 == 0; block
      // scaling takes K % 128 == 0)
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        if (i < 4) {
          const int row = (wave * 4 + i) * 8 + (lane >> 3);
          const bool ok = tg_chunk<FMT>(row, lane & 7) * 16 < ktail;
          tg_dma16(rw, lw + i * 1024, ok ? w_off[i] : kTgOob, soff);
        }
        const int row = (wave * NRB + i) * 8 + (lane >> 3);
        const bool ok = tg_chunk<FMT>(row, lane & 7) * 16 < ktail;
        tg_dma16(rx, lx + i * 1024, ok ? x_off[i] : kTgOob, soff);
      }
    } else {
#pragma unroll
      for (int i = 0; i < NRB; ++i) {
        if (i < 4) {
          if constexpr (WNT) tg_dma16nt(rw, lw + i * 1024, w_off[i], soff);
          else tg_dma16(rw, lw + i * 1024, w_off[i], soff);
        }
        tg_dma16(rx, lx + i * 1024, x_off[i], soff);
      }
    }
    if (BLOCK && wave < NRB) tg_dma4(rxs, lds0 + L::Xs + st * (BM * 4) + wave * 256, xs_off, kb * 4);
  };

  // ---- first tile: synchronous set-up
  TgTile cur = tile_of(t, load_tab(t));
  int buf = 0, st = 0;
  prefetch(cur, buf);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();  // the first tile's row sources are in LDS
  set_offsets(cur);
  stage_ws(buf);
  issue(cur.kb0, st);
  int tn = t + per;
  int pf_tab = tn < t_hi ? load_tab(tn) : 0;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  while (true) {
    const bool has_next = tn < t_hi;
    TgTile nxt = cur;
    if (has_next) {
      // the next tile's row sources and weight scales load under this tile's
      // K loop; the table word of the tile after it as well
      nxt = tile_of(tn, pf_tab);
      prefetch(nxt, buf ^ 1);
      if (tn + per < t_hi) pf_tab = load_tab(tn + per);
    }
    int wslot = 0;  // block scaling: staged weight-scale row of this wave's blocks j < 4
    if (BLOCK && EPI != kTgEpiSwiGluQuant) wslot = wn;
    const float* sWs = (const float*)(smem + L::Ws) + buf * 2 * kTgMaxKB;

    Acc acc[8][NRB];
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int mb = 0; mb < NRB; ++mb) acc[j][mb] = Acc{0, 0, 0, 0};

    // The next tile's prefetch loads are still in flight here.  Where the
    // register allocator reuses one of their destination registers inside the
    // K loop (the store epilogue variants), the compiler would otherwise wait
    // for all vector-memory operations (the next block's copies included) in
    // every K step; one wait per tile here lets it drop that.
    if constexpr (EPI != kTgEpiSwiGluQuant) __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    // Block scaling (MoE experts, block-FP8 linear): row block 4 * mb + wm of
    // a ragged row tile holds rows while 16 * (4 * mb + wm) < rows, so the
    // first `live` of this wave's row blocks hold rows.  A wave without any
    // skips its fragment reads and MFMAs (its accumulators stay 0 and are
    // never stored) and takes part in every copy and barrier; the SwiGLU
    // epilogue skips the blocks past `live`.  (Skipping single row blocks in
    // the K loop takes one loop body per live count, and the compiler's
    // register copies between those bodies cost more than the MFMAs saved;
    // the W8A8 prefill instantiations keep the unbranched loop: same speed
    // without the branch, measured.)
    const int live = BLOCK ? __builtin_amdgcn_readfirstlane(
                                 min(NRB, max(0, (cur.row_end - cur.row0 - 16 * wm + 63) >> 6)))
                           : NRB;
    for (int kb = cur.kb0; kb < cur.kb1; ++kb) {
      if (kb + 1 < cur.kb1) issue(kb + 1, st ^ 1);
      const uint8_t* sW = smem + L::W + st * (kTgBN * kTgBK) + (128 * wn) * kTgBK;
      // row block mb of this wave: tile rows 16 * (4 * mb + wm) ...
      const uint8_t* sX = smem + L::X + st * (BM * kTgBK) + (16 * wm) * kTgBK;
      // block scaling: the scale of row block mb and W rows j * 16 is
      // sx[mb] * sw[j >> 2]; 256-row tiles form the products once per K
      // block, 320-row tiles (160 accumulators: registers are short) form
      // each at its use
      float sx[NRB], sw[2] = {0.f, 0.f}, prod[2][NRB];
      if constexpr (BLOCK) {
        // 16 lanes read 16 consecutive floats (the other lane groups the same
        // ones): conflict-free
        const float* sxs = (const float*)(smem + L::Xs + st * (BM * 4)) + 16 * wm + lr;
#pragma unroll
        for (int mb = 0; mb < NRB; ++mb) sx[mb] = sxs[64 * mb];
        if constexpr (EPI == kTgEpiSwiGluQuant) {
          sw[0] = sWs[kb];
          sw[1] = sWs[KB + kb];
        } else {
          sw[0] = sw[1] = sWs[wslot * KB + kb];
        }
        if constexpr (NRB == 4) {
#pragma unroll
          for (int mb = 0; mb < NRB; ++mb) {
            prod[0][mb] = sx[mb] * sw[0];
            prod[1][mb] = sx[mb] * sw[1];
          }
        }
      }
      // fragment reads and MFMAs of the wave's NRB row blocks
      auto kstep = [&]() {
        TgFrag xf[NRB];
        f32x4 blk[kTgLag + 1];
#pragma unroll
        for (int mb = 0; mb < NRB; ++mb) xf[mb] = tg_load(sX + mb * 64 * kTgBK, o_lo, o_hi);
        // 256-row tiles: the next weight fragment's LDS read goes out before
        // this one's MFMAs, and the fence keeps the scheduler from sinking it
        // to its use (otherwise each fragment's read latency stalls its MFMAs:
        // C3 M = 8192 377 -> 362 us, C4 M = 4096 272 -> 265 us; a second
        // fragment ahead measured the same).  320-row tiles have no registers
        // for the second buffer.
        constexpr bool PF = NRB == 4;
        TgFrag wfb[2];
        if constexpr (PF) wfb[0] = tg_load(sW, o_lo, o_hi);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          TgFrag wf;
          if constexpr (PF) {
            if (j + 1 < 8) wfb[(j + 1) & 1] = tg_load(sW + (j + 1) * 16 * kTgBK, o_lo, o_hi);
            __builtin_amdgcn_sched_barrier(0);
            wf = wfb[j & 1];
          } else {
            wf = tg_load(sW + j * 16 * kTgBK, o_lo, o_hi);
          }
#pragma unroll
          for (int mb = 0; mb < NRB; ++mb) {
            if constexpr (FMT == kTgI8) {
              acc[j][mb] = mfma_i8(wf.lo, xf[mb].lo, acc[j][mb]);
              acc[j][mb] = mfma_i8(wf.hi, xf[mb].hi, acc[j][mb]);
            } else {
              const i32x8 A = i32x8{wf.lo[0], wf.lo[1], wf.lo[2], wf.lo[3], wf.hi[0], wf.hi[1], wf.hi[2], wf.hi[3]};
              const i32x8 B = i32x8{xf[mb].lo[0], xf[mb].lo[1], xf[mb].lo[2], xf[mb].lo[3],
                                    xf[mb].hi[0], xf[mb].hi[1], xf[mb].hi[2], xf[mb].hi[3]};
              if constexpr (BLOCK) {
                // scale-accumulate kTgLag MFMAs behind, from rotating
                // temporaries: with one MFMA of lag the FMAs read a result
                // the matrix core is still producing and the next MFMA into
                // that temporary waits for them (two MFMAs in flight at most)
                const int idx = j * NRB + mb;
                constexpr int R = kTgLag + 1;
                blk[idx % R] = mfma_fp8(A, B, f32x4{0.f, 0.f, 0.f, 0.f});
                // keep the FMAs of result idx - kTgLag after this MFMA (the
                // scheduler would otherwise hoist them next to their MFMA)
                __builtin_amdgcn_sched_barrier(0);
                auto fold = [&](int d) {
                  const int pj = d / NRB, pm = d % NRB;
                  const float sc = NRB == 4 ? prod[pj >> 2][pm] : sx[pm] * sw[pj >> 2];
#pragma unroll
                  for (int q = 0; q < 4; ++q) acc[pj][pm][q] = fmaf(blk[d % R][q], sc, acc[pj][pm][q]);
                };
                if (idx >= kTgLag) fold(idx - kTgLag);
                if (idx == 8 * NRB - 1) {
#pragma unroll
                  for (int d = 8 * NRB - kTgLag; d < 8 * NRB; ++d) fold(d);
                }
              } else {
                acc[j][mb] = mfma_fp8(A, B, acc[j][mb]);
              }
            }
          }
        }
      };
      if (live > 0) kstep();
      __builtin_amdgcn_s_waitcnt(0);  // this wave's copies of the next block have landed
      __syncthreads();                 // ... and everyone's; stage st is free again
      st ^= 1;
    }

    if (has_next) {
      // the next tile's first K block loads while this tile's epilogue runs
      set_offsets(nxt);
      stage_ws(buf ^ 1);
      issue(nxt.kb0, st);
    }

    // ------------------------------------------------------------ epilogue
    // One copy per output dtype (a uniform branch picks it), so every
    // rounding and conversion below is a single fixed instruction sequence.
    auto epilogue = [&](auto odt) {
      constexpr int ODT = decltype(odt)::value;
      // The epilogue's lane-derived addresses are formed here, once per tile:
      // an opaque copy of the lane id keeps the compiler from computing them
      // before the tile loop and holding them in registers across the K loop.
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const int lr = ln & 15, lg = ln >> 4, tid = 64 * wave + ln;
      auto trow = [&](int mb) { return 16 * (4 * mb + wm) + lr; };
      // lane holds tile rows trow(mb) = 16*(4*mb + wm) + lr, columns 128*wn + 16*j + 4*lg + q
      const int row0 = cur.row0, row_end = cur.row_end, ntile = cur.ntile;
      if constexpr (EPI == kTgEpiSwiGluQuant) {
        // SwiGLU rounded to the activation dtype at each step (as torch does for
        // bf16 / fp16 tensors), then 1x128 e4m3 quantization of the tile's 128
        // activation columns: s = max(amax, 1e-12) / 448, q = e4m3(clamp(v / s)).
        // Row blocks without rows keep their zero accumulators.
        // The products are held as 16-bit pairs of the activation dtype (the
        // value each rounds to), so the 80 gate and 80 up accumulators of a
        // 320-row tile give way to 40 registers.
        float amax[NRB];
        uint32_t pv[4][NRB][2];
  #pragma unroll
        for (int mb = 0; mb < NRB; ++mb) {
          amax[mb] = 0.f;
  #pragma unroll
          for (int j = 0; j < 4; ++j) pv[j][mb][0] = pv[j][mb][1] = 0u;
          if (mb >= live) continue;
  #pragma unroll
          for (int j = 0; j < 4; ++j) {
  #pragma unroll
            for (int h = 0; h < 2; ++h) {
              // the pair q = 2h, 2h + 1, each rounding a packed conversion
              const uint32_t gp = tg_pack2(acc[j][mb][2 * h], acc[j][mb][2 * h + 1], ODT);
              const uint32_t up = tg_pack2(acc[j + 4][mb][2 * h], acc[j + 4][mb][2 * h + 1], ODT);
              const float g0 = tg_lo(gp, ODT), g1 = tg_hi(gp, ODT);
              const uint32_t sp = tg_pack2(g0 * __builtin_amdgcn_rcpf(1.0f + __expf(-g0)),
                                           g1 * __builtin_amdgcn_rcpf(1.0f + __expf(-g1)), ODT);
              const uint32_t vp = tg_pack2(tg_lo(sp, ODT) * tg_lo(up, ODT), tg_hi(sp, ODT) * tg_hi(up, ODT), ODT);
              amax[mb] = fmaxf(amax[mb], fmaxf(fabsf(tg_lo(vp, ODT)), fabsf(tg_hi(vp, ODT))));
              pv[j][mb][h] = vp;
            }
          }
        }
  #pragma unroll
        for (int mb = 0; mb < NRB; ++mb) {
          amax[mb] = fmaxf(amax[mb], __shfl_xor(amax[mb], 16, 64));
          amax[mb] = fmaxf(amax[mb], __shfl_xor(amax[mb], 32, 64));
          if (lg == 0) sRed[wn * BM + trow(mb)] = amax[mb];
        }
        __syncthreads();
        const int IB = a.I / 128;
        // the tile's BM x 128 e4m3 block goes through the idle pipeline stage
        // (row r at r*128, 4-byte units permuted by tg_stage_off4) so that the global
        // stores below write whole 128-byte rows
        uint8_t* stg = smem + L::X + (st ^ 1) * (BM * kTgBK);
  #pragma unroll
        for (int mb = 0; mb < NRB; ++mb) {
          const int lrow = trow(mb);
          const float am = fmaxf(sRed[lrow], sRed[BM + lrow]);
          const float s = __fdiv_rn(fmaxf(am, 1e-12f), 448.0f);
          const float rs = __fdiv_rn(1.0f, s);
  #pragma unroll
          for (int j = 0; j < 4; ++j) {
            float v[4];
  #pragma unroll
            for (int q = 0; q < 4; ++q)
              v[q] = fminf(fmaxf(div_by_recip((q & 1) ? tg_hi(pv[j][mb][q >> 1], ODT) : tg_lo(pv[j][mb][q >> 1], ODT), s, rs),
                                 -448.0f), 448.0f);
            const int col = 64 * wn + 16 * j + 4 * lg;
            *(uint32_t*)(stg + tg_stage_off4(lrow, col >> 2)) =
                pack4_e4m3(v[0], v[1], v[2], v[3]);
          }
          if (wn == 0 && lg == 0 && row0 + lrow < row_end) a.acts[(int64_t)(row0 + lrow) * IB + ntile] = s;
        }
        __syncthreads();
  #pragma unroll
        for (int i = 0; i < NRB; ++i) {
          const int r = 64 * i + (tid >> 3), c = tid & 7;
          if (row0 + r < row_end)
            *(i32x4*)(a.actq + (int64_t)(row0 + r) * a.I + ntile * 128 + c * 16) =
                tg_stage_read(stg, r, c);
        }
      } else if constexpr (EPI == kTgEpiSwiGluStore) {
        // gate and up of activation column 64 * wn + 16 * j + 4 * lg + q
        // (j < 4: gate rows, j + 4 the up rows) with the store epilogue's
        // arithmetic, ((acc * xs) * ws) + bias, then SwiGLU with the
        // elementwise pass's roundings (swiglu_bits): the bits the packed
        // GEMM followed by kq_swiglu produce, without the [M, 2I] round trip
        const float* eX = (const float*)(smem + L::Epi) + buf * 3 * 256;
        const int I = a.I;
  #pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int cl = 64 * wn + 16 * j + 4 * lg;
          const int col = ntile * 128 + cl;
          const f32x4 wsg = *(const f32x4*)(eX + 256 + cl), wsu = *(const f32x4*)(eX + 256 + 128 + cl);
          const f32x4 bg = *(const f32x4*)(eX + 512 + cl), bu = *(const f32x4*)(eX + 512 + 128 + cl);
  #pragma unroll
          for (int mb = 0; mb < NRB; ++mb) {
            const int grow = row0 + trow(mb);
            const float xsc = eX[trow(mb)];
            uint16_t o[4];
  #pragma unroll
            for (int q = 0; q < 4; ++q) {
              const float g = __fadd_rn(__fmul_rn(__fmul_rn((float)acc[j][mb][q], xsc), wsg[q]), bg[q]);
              const float u = __fadd_rn(__fmul_rn(__fmul_rn((float)acc[j + 4][mb][q], xsc), wsu[q]), bu[q]);
              o[q] = swiglu_bits(g, u, ODT);
            }
            if (grow < row_end && col < I)
              *(u32x2*)((uint16_t*)a.out + (int64_t)grow * I + col) =
                  u32x2{(uint32_t)o[0] | ((uint32_t)o[1] << 16), (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
          }
        }
      } else if (ksplit > 1) {
        // raw 32-bit accumulators of this work unit's K range; a reduce pass
        // sums the splits in order and applies the scales
        uint32_t* pb = a.partials + (int64_t)cur.split * a.M * a.N;
        const bool vec = (a.N & 3) == 0;
  #pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int n = ntile * kTgBN + 128 * wn + 16 * j + 4 * lg;
  #pragma unroll
          for (int mb = 0; mb < NRB; ++mb) {
            const int grow = row0 + trow(mb);
            if (grow >= row_end) continue;
            uint32_t v[4];
  #pragma unroll
            for (int q = 0; q < 4; ++q) {
              if constexpr (FMT == kTgI8) v[q] = (uint32_t)(int)acc[j][mb][q];
              else v[q] = __float_as_uint((float)acc[j][mb][q]);
            }
            uint32_t* dst = pb + (int64_t)grow * a.N + n;
            if (vec && n + 3 < a.N) {
              *(u32x4*)dst = u32x4{v[0], v[1], v[2], v[3]};
            } else {
  #pragma unroll
              for (int q = 0; q < 4; ++q)
                if (n + q < a.N) dst[q] = v[q];
            }
          }
        }
      } else {
        const float* eX = (const float*)(smem + L::Epi) + buf * 3 * 256;
        // each wave's output rows go through its 8 KB of the idle pipeline
        // stage in passes of up to four row blocks by 64 columns ([m][64
        // columns], 8-byte units permuted by tg_stage_off8), so every global
        // store writes whole 128-byte row segments; rows of 8-aligned N only
        // (others store directly)
        uint8_t* stg = smem + (wave < 4 ? L::W : L::X) + (st ^ 1) * (wave < 4 ? kTgBN * kTgBK : BM * kTgBK) +
                       (wave & 3) * 8192;
        const bool staged = (a.N & 7) == 0;
  #pragma unroll
        for (int half = 0; half < 2; ++half) {
  #pragma unroll
          for (int mg = 0; mg < NRB; mg += 4) {
            constexpr int kPass = 4;
  #pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
              const int j = 4 * half + jj;
              const int nl = 128 * wn + 16 * j + 4 * lg;  // tile column of q = 0
              const int n = ntile * kTgBN + nl;
              const f32x4 wsc = *(const f32x4*)(eX + 256 + nl);
              const f32x4 bv = *(const f32x4*)(eX + 512 + nl);
  #pragma unroll
              for (int mb = mg; mb < NRB && mb < mg + kPass; ++mb) {
                const int ml = 16 * (mb - mg) + lr;  // staging row
                const int grow = row0 + trow(mb);
                const float xsc = BLOCK ? 1.0f : eX[trow(mb)];
                // bias: -0.0 when the call has none (v + -0 == v for every v,
                // signed zeros and NaNs included), so no branch or select
                float v[4];
  #pragma unroll
                for (int q = 0; q < 4; ++q) {
                  v[q] = (float)acc[j][mb][q];
                  if (!BLOCK) v[q] = __fmul_rn(__fmul_rn(v[q], xsc), wsc[q]);
                  v[q] = __fadd_rn(v[q], bv[q]);
                }
                const u32x2 word = u32x2{tg_pack2(v[0], v[1], ODT), tg_pack2(v[2], v[3], ODT)};
                const uint16_t o[4] = {(uint16_t)word[0], (uint16_t)(word[0] >> 16), (uint16_t)word[1],
                                       (uint16_t)(word[1] >> 16)};
                if (staged) {
                  const int cb = 32 * jj + 8 * lg;  // byte column within the 128-byte row
                  *(u32x2*)(stg + tg_stage_off8(ml, cb >> 3)) = word;
                } else if (grow < row_end) {
                  uint16_t* dst = (uint16_t*)a.out + (int64_t)grow * a.N + n;
  #pragma unroll
                  for (int q = 0; q < 4; ++q)
                    if (n + q < a.N) dst[q] = o[q];
                }
                if constexpr (FMT == kTgI8) {
                  if (a.acc_out && grow < row_end) {
                    int32_t* ad = a.acc_out + (int64_t)grow * a.N + n;
  #pragma unroll
                    for (int q = 0; q < 4; ++q)
                      if (n + q < a.N) ad[q] = acc[j][mb][q];
                  }
                }
              }
            }
            if (staged) {
              // 8 rows of 8 chunks per instruction over the pass's rows
              const int prow = 16 * (NRB - mg < kPass ? NRB - mg : kPass);
  #pragma unroll
              for (int i = 0; i < prow / 8; ++i) {
                const int ml = 8 * i + (ln >> 3), c = ln & 7;
                const int grow = row0 + 16 * (4 * (mg + (ml >> 4)) + wm) + (ml & 15);
                const int n = ntile * kTgBN + 128 * wn + 64 * half + 8 * c;
                const i32x4 v = tg_stage_read(stg, ml, c);
                if (grow < row_end && n < a.N) *(i32x4*)((uint16_t*)a.out + (int64_t)grow * a.N + n) = v;
              }
            }
          }
        }
      }
    };
    if (a.out_dtype == KQ_DTYPE_BF16) epilogue(std::integral_constant<int, KQ_DTYPE_BF16>{});
    else epilogue(std::integral_constant<int, KQ_DTYPE_F16>{});
    if (!has_next) break;
    __builtin_amdgcn_s_waitcnt(0);  // the next tile's first block has landed
    __syncthreads();
    cur = nxt;
    buf ^= 1;
    tn += per;
  }
}

// ------------------------------------------------------------------ host
static inline int tg_device_cus() {
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

// Persistent launch: one workgroup per CU (never more than the tiles), a
// multiple of 8 so every XCD gets the same number of workgroups.  NRB = 5:
// row tiles of 320 rows (a.mtiles counts them).
template <int FMT, bool BLOCK, int EPI, int NRB = 4, bool WNT = false>
static void tg_launch(const TileGemmArgs& a, hipStream_t stream) {
  const int64_t max_total = (int64_t)a.mtiles * a.ntiles * (a.ksplit > 1 ? a.ksplit : 1);
  int64_t grid = max_total < tg_device_cus() ? max_total : tg_device_cus();
  grid = (grid + 7) / 8 * 8;
  hipLaunchKernelGGL((tile_gemm_kernel<FMT, BLOCK, EPI, NRB, WNT>), dim3((unsigned)grid), dim3(kTgThreads), 0,
                     stream, a);
}

}  // namespace kq
