// Split-K without inter-workgroup synchronization.
//
// When a GEMV-shaped problem has too few output tiles to fill the 256 CUs,
// workgroups of one tile take disjoint K ranges and store raw partial
// accumulators to a workspace ([splits][M][N], 32-bit).  A second, small
// kernel sums the partials in fixed split order 0..S-1 and runs the
// epilogue; the kernel boundary orders the two, so no device-scope fence or
// counter is needed inside either kernel.
#pragma once

#include "kq_common.h"

namespace kq {

enum { kReduceW4 = 0, kReduceI8 = 1, kReduceFp8 = 2 };

struct ReduceArgs {
  const void* partials;  // [splits][M][N] float (W4, FP8) or int32 (I8)
  int splits, M, N;
  const float* xscale;   // W8A8 epilogue
  const float* wscale;
  int ws_per_channel;
  const void* bias;
  int bias_dtype;
  void* out;
  int out_dtype;
  int32_t* acc_out;      // I8: optional raw accumulators
  // N = 2I packed gate / up columns, out [M][I] = silu(gate) * up (the
  // elementwise pass's roundings), no acc_out: 1 gate column c with up column
  // I + c (W8A8 packs), 2 gate / up 16-column blocks alternating (the W4A16
  // interleaved operand); 0 none
  int swiglu;
};

// Launches the reduce kernel on `stream` (grid over M*N, 4 outputs/thread).
void launch_splitk_reduce(int mode, const ReduceArgs& a, hipStream_t stream);

}  // namespace kq
