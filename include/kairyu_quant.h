/*
 * kairyu_quant.h - C ABI of the MI355X (gfx950) quantized-linear kernels.
 *
 * Drop-in boundary for the reference's kernel layer
 * (reference: kairyu/kernels/quant_gemm_gpu.py).  Every entry point takes raw
 * device pointers, element counts and a hipStream_t (passed as void*), never
 * a framework type, launches asynchronously on that stream and returns
 * KQ_OK or an error code; kq_last_error() gives the message of the calling
 * thread's most recent failure.  Host wrappers map KQ_EINVAL to ValueError and
 * every other code to RuntimeError, the reference's fail-closed convention
 * (quant_gemm_gpu.py:418-520).
 *
 * Conventions
 *   - Matrices are row-major with unit stride in the last dimension; `ld*`
 *     arguments give the row pitch in elements where a caller may pass views.
 *   - dtype codes: KQ_DTYPE_F16, KQ_DTYPE_BF16, KQ_DTYPE_F32; KQ_DTYPE_NONE
 *     marks an absent optional operand (bias).
 *   - FP8 means OCP e4m3fn bytes (torch.float8_e4m3fn).
 *   - `workspace` is scratch device memory (split-K partial sums, the
 *     act-order activation gather).  It may be NULL or short for the W8A8
 *     entry points (no split-K then; kq_w8a8_workspace_size() bytes enable
 *     every split-K form); W4A16 calls need kq_w4a16_workspace_size() bytes.
 *     Calls that share one workspace must be ordered on one stream.
 */
#ifndef KAIRYU_QUANT_H
#define KAIRYU_QUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KQ_OK 0
#define KQ_EINVAL 1       /* bad shape / layout / argument (ValueError)   */
#define KQ_EUNSUPPORTED 2 /* device or dtype not supported (RuntimeError) */
#define KQ_ELAUNCH 3      /* HIP launch failure (RuntimeError)            */
#define KQ_EWORKSPACE 4   /* workspace too small (RuntimeError)           */

#define KQ_DTYPE_NONE (-1)
#define KQ_DTYPE_F16 0
#define KQ_DTYPE_BF16 1
#define KQ_DTYPE_F32 2

/* Library version (major*10000 + minor*100 + patch). */
int kq_version(void);

/* Message of the calling thread's last failed call ("" if none). */
const char* kq_last_error(void);

/* 1 when `device` is a gfx950 GPU this library was built for, else 0.
 * Replaces the SM capability floors of quant_gemm_gpu.py:409-415. */
int kq_device_supported(int device);

/* Per-row fp32 absolute maximum of x[rows, k] (fp16/bf16).
 * Replaces _row_amax_kernel / fp8_activation_amax (quant_gemm_gpu.py:79-94,575-593). */
int kq_row_amax(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                float* amax, void* stream);

/* Dynamic per-token symmetric INT8 quantization: scale = max(amax,1e-12)/127
 * (IEEE division), q = rint(clamp(x/scale, +-127)).
 * Replaces _scaled_activation_quant_kernel with ROUND_TO_INT
 * (quant_gemm_gpu.py:26-76,538-572; CPU oracle kairyu/quant/int8.py:25-30). */
int kq_act_quant_i8(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                    int8_t* xq, float* xscale, void* stream);

/* Per-token FP8 e4m3 quantization q = e4m3(clamp(x/scale, +-448)).
 * scale_mode 0: dynamic, scale = max(amax,1e-12)/448 (kairyu/quant/fp8.py:33-45)
 * scale_mode 1: static scalar scale_in[0] (checkpoint input_scale)
 * scale_mode 2: given per row scale_in[rows] (TP global amax, linear.py:496-518)
 * The scale used for each row is written to xscale[rows].
 * Replaces _scaled_activation_quant_kernel without ROUND_TO_INT. */
int kq_act_quant_fp8(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                     const float* scale_in, int scale_mode, uint8_t* xq, float* xscale,
                     void* stream);

/* INT8 W8A8: acc = xq[m,k] . w[n,k] exactly in int32, then
 * out = fp32(acc) * xscale[m] * wscale[n] (+ bias[n]), each step rounded
 * separately, cast to out_dtype.  acc_out (optional, int32 [m,n]) receives
 * the raw accumulators.  Replaces _int8_w8a8_kernel / int8_linear_forward
 * (quant_gemm_gpu.py:160-221,657-687; oracle kairyu/quant/int8.py:33-41). */
int kq_w8a8_i8_gemm(const int8_t* xq, const float* xscale, const int8_t* w,
                    const float* wscale, const void* bias, int bias_dtype, void* out,
                    int out_dtype, int32_t* acc_out, int64_t m, int64_t n, int64_t k,
                    void* workspace, size_t workspace_bytes, void* stream);

/* FP8 W8A8: out = (xq . w in fp32) * xscale[m] * wscale[n or 0] (+ bias).
 * wscale_per_channel selects wscale[n] vs a per-tensor wscale[0].
 * Replaces torch._scaled_mm / _fp8_w8a8_kernel of fp8_linear_forward
 * (quant_gemm_gpu.py:97-157,596-654; oracle kairyu/quant/fp8.py:48-56). */
int kq_w8a8_fp8_gemm(const uint8_t* xq, const float* xscale, const uint8_t* w,
                     const float* wscale, int wscale_per_channel, const void* bias,
                     int bias_dtype, void* out, int out_dtype, int64_t m, int64_t n,
                     int64_t k, void* workspace, size_t workspace_bytes, void* stream);

/* Per-token activation quantization fused with the W8A8 GEMM: x fp16/bf16
 * [m, k] (row pitch ldx) is quantized exactly as kq_act_quant_i8 /
 * kq_act_quant_fp8 would (INT8 dynamic; FP8 scale_mode 0 dynamic, 1 static
 * scale_in[0], 2 per-row scale_in[m]) and multiplied with w as
 * kq_w8a8_i8_gemm / kq_w8a8_fp8_gemm do.  Small decode batches quantize
 * inside the GEMM launch; other shapes stage the quantized rows in the
 * workspace (kq_w8a8_linear_workspace_size bytes).  Replaces the
 * _quantize_activation + GEMM pair of int8_linear_forward / fp8_linear_forward
 * (quant_gemm_gpu.py:538-572, :596-687). */
int kq_w8a8_i8_linear(const void* x, int x_dtype, int64_t ldx, const int8_t* w,
                      const float* wscale, const void* bias, int bias_dtype, void* out,
                      int out_dtype, int32_t* acc_out, int64_t m, int64_t n, int64_t k,
                      void* workspace, size_t workspace_bytes, void* stream);
int kq_w8a8_fp8_linear(const void* x, int x_dtype, int64_t ldx, const float* scale_in,
                       int scale_mode, const uint8_t* w, const float* wscale,
                       int wscale_per_channel, const void* bias, int bias_dtype, void* out,
                       int out_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                       size_t workspace_bytes, void* stream);
/* Workspace bytes for kq_w8a8_{i8,fp8}_linear of this shape (quantized rows,
 * row scales, and every split-K form).  No counterpart in the reference. */
size_t kq_w8a8_linear_workspace_size(int64_t m, int64_t n, int64_t k);

/* Packed (gate, up) W8A8 projection with SwiGLU: w holds the gate rows then
 * the up rows, [2 * i_width][k] (wscale and bias over the same 2 * i_width
 * rows), and out [m][i_width] (activation dtype) = silu(g) * u for gate
 * column c and up column i_width + c, with the roundings of
 * kq_w8a8_*_linear followed by kq_swiglu (bit-identical to that pair).
 * Prefill shapes apply SwiGLU in the tile engine's epilogue and shapes of
 * m <= 64 in the decode or skinny GEMM's (or the reduce of their K splits):
 * the [m][2I] projection never reaches memory; other shapes run the pair
 * through the workspace.  Replaces the reference MLP's act_fn(gate(x)) *
 * up(x) (kairyu/models/layers.py:243-244) over its packed projections
 * (kairyu/models/packed_linear.py:58-149) for FP8 / INT8 W8A8. */
int kq_w8a8_i8_swiglu_linear(const void* x, int x_dtype, int64_t ldx, const int8_t* w,
                             const float* wscale, const void* bias, int bias_dtype, void* out,
                             int64_t m, int64_t i_width, int64_t k, void* workspace,
                             size_t workspace_bytes, void* stream);
int kq_w8a8_fp8_swiglu_linear(const void* x, int x_dtype, int64_t ldx, const float* scale_in,
                              int scale_mode, const uint8_t* w, const float* wscale,
                              int wscale_per_channel, const void* bias, int bias_dtype, void* out,
                              int64_t m, int64_t i_width, int64_t k, void* workspace,
                              size_t workspace_bytes, void* stream);
/* Workspace bytes for kq_w8a8_*_swiglu_linear of this shape.  No counterpart
 * in the reference. */
size_t kq_w8a8_swiglu_workspace_size(int64_t m, int64_t i_width, int64_t k);

/* Bytes of workspace with which every split-K form of the two W8A8 entry
 * points is available for this shape (0: none applies).  No counterpart in
 * the reference (its GPU path calls torch._scaled_mm / Triton, which allocate
 * through torch). */
size_t kq_w8a8_workspace_size(int64_t m, int64_t n, int64_t k);

/* AWQ W4A16 ("gemm" layout): qweight int32 [k, n/8] packed along n in order
 * [0,2,4,6,1,3,5,7], qzeros int32 [k/g, n/8] same packing, scales fp16 [k/g, n].
 * w = fp16((q - z) * s); x is fed to the dot as fp16 (bf16 saturated to
 * +-65504); fp32 accumulation; out in x_dtype.
 * Replaces _awq_w4a16_kernel / awq_linear_forward (quant_gemm_gpu.py:224-315,690-724;
 * format kairyu/quant/awq.py:14-74). */
int kq_w4a16_awq_gemm(const void* x, int x_dtype, const int32_t* qweight,
                      const int32_t* qzeros, const void* scales, const void* bias,
                      int bias_dtype, void* out, int64_t m, int64_t n, int64_t k,
                      int group_size, void* workspace, size_t workspace_bytes,
                      void* stream);

/* GPTQ W4A16: qweight int32 [k/8, n] packed LSB-first along k, qzeros int32
 * [groups, n/8] packed along n storing z-1, scales fp16 [groups, n].
 * w = fp16((q - (z_stored + 1)) * s[group(k)]).
 * gidx_mode 0: group(k) = k / group_size, qweight rows in checkpoint order.
 * gidx_mode 1: qweight rows were permuted by kq_gptq_permute_qweight with
 *              `perm`; permuted row j reads x[:, perm[j]] and has group
 *              j / group_size.
 * gidx_mode 2: arbitrary g_idx[k] (per-element group lookup).
 * Replaces _gptq_w4a16_kernel / gptq_linear_forward (quant_gemm_gpu.py:318-407,
 * 727-761; format kairyu/quant/gptq.py:15-90). */
int kq_w4a16_gptq_gemm(const void* x, int x_dtype, const int32_t* qweight,
                       const int32_t* qzeros, const void* scales, const int32_t* g_idx,
                       const int32_t* perm, int gidx_mode, const void* bias,
                       int bias_dtype, void* out, int64_t m, int64_t n, int64_t k,
                       int group_size, void* workspace, size_t workspace_bytes,
                       void* stream);

/* Load-time tiled operand of a W4A16 weight for the tiled kernels:
 * kq_w4a16_tiled_words(n, k, group_size) int32 words.  The first
 * ceil(n/16) * ceil(k/128) * 256 words hold 16-column tiles of 128-k stages:
 * the word of packed row r (k = 8r .. 8r+7) and column 16u + c holds
 * q[row(8r + e)][16u + c] in nibble e; within tile u's stage t = r / 16 it
 * sits at word (u * ceil(k/128) + t) * 256 + (kb * 16 + c) * 4 + s for
 * r % 16 = 4s + kb, so the 4 words a lane (c, kb) of a 16x16x32 MFMA operand
 * needs for a stage are 16 contiguous bytes.  row(k) = perm[k] when perm is
 * given (GPTQ act-order: the stable argsort of g_idx, so permuted row j has
 * group j / group_size), else k; rows past k/8 and columns past n are 0.
 * A scale/zero table follows: for tile u and group pair p, word
 * (u * P + p) * 32 + c * 2 + (g & 1) = scales[g][16u + c] bits |
 * (zero nibble + zero_offset) << 16 for g = 2p, 2p + 1, with
 * P = ceil(ceil(k / group_size) / 2) (0 past the last group and past n).
 * With qzeros null (one zero, zero_offset in 0..16, for every group and
 * column: symmetric checkpoints) the table holds scales alone, word
 * (u * P + p) * 16 + c = scales[2p][16u + c] | scales[2p + 1][16u + c] << 16,
 * followed by ceil(k / group_size) * n/8 words of zero nibbles.
 * src_format 0: AWQ qweight [k, n/8]; 1: GPTQ qweight [k/8, n].  qzeros
 * [groups, n/8] in natural nibble order (or null) and zero_offset as for
 * kq_w4a16_tiled_gemm, scales fp16 [groups, n]; the tiled GEMM must be given
 * the same three.  Derived operand only; checkpoint buffers are untouched (the
 * reference caches derived runtime operands the same way,
 * quant_gemm_gpu.py:802-850; formats kairyu/quant/awq.py:14-36,
 * kairyu/quant/gptq.py:15-46). */
int kq_w4a16_tile_weights(const int32_t* qweight, int src_format, const int32_t* perm,
                          const int32_t* qzeros, int zero_offset, const void* scales,
                          int32_t* tiles, int64_t n, int64_t k, int group_size, void* stream);

/* int32 words of kq_w4a16_tile_weights' operand (one_zero: built with qzeros
 * null), or -1 for an unsupported shape (n, k multiples of 8, group_size a
 * multiple of 8 below 65536, k below 2^24).  Sizing helper; no reference
 * counterpart. */
int64_t kq_w4a16_tiled_words(int64_t n, int64_t k, int group_size, int one_zero);

/* AWQ qzeros [groups, n/8] (AWQ nibble order) -> natural nibble order
 * (column 8w + i in nibble i), values unchanged: the zero operand of
 * kq_w4a16_tiled_gemm with zero_offset 0 (kairyu/quant/awq.py:14-36). */
int kq_awq_natural_zeros(const int32_t* qzeros, int32_t* qzeros_n, int64_t n, int64_t groups,
                         void* stream);

/* W4A16 on kq_w4a16_tile_weights' operand (built from the same qzeros,
 * zero_offset and scales as this call gets): w = fp16((q - z) * s[group]) with
 * z = stored nibble + zero_offset (GPTQ qzeros: 1; AWQ natural zeros: 0;
 * qzeros null: z = zero_offset in 0..16 everywhere, for an operand tiled so),
 * qzeros [groups, n/8] natural nibble order, scales fp16 [groups, n],
 * group = row / group_size of the (permuted) row; x fed to the dot as fp16
 * (bf16 saturated to +-65504), fp32 accumulation, out in x_dtype.  perm
 * (nullable) is the act-order permutation the tiles were built with: x is
 * gathered through it (workspace: m*k*2 bytes).  M <= 16 with k in
 * {1024, 2048, 4096} runs the persistent decode GEMV.
 * Replaces _awq_w4a16_kernel / _gptq_w4a16_kernel and awq_linear_forward /
 * gptq_linear_forward (quant_gemm_gpu.py:224-407,690-761). */
int kq_w4a16_tiled_gemm(const void* x, int x_dtype, const int32_t* tiles, const int32_t* qzeros,
                        int zero_offset, const void* scales, const int32_t* perm, const void* bias,
                        int bias_dtype, void* out, int64_t m, int64_t n, int64_t k, int group_size,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Packed gate/up projection with SwiGLU: out[m][n] = silu(gate) * up for
 * n < i_width, computed as torch does on fp16/bf16 tensors (gate and up
 * rounded to x_dtype, silu = g / (1 + exp(-g)) in fp32 rounded, the product
 * rounded; kairyu/models/layers.py:243-244 `silu(gate_proj(x)) *
 * up_proj(x)`).  `tiles` is kq_w4a16_tile_weights' operand over 2 * i_width
 * columns in which 16-column blocks of gate (block b: gate columns 16b..16b+15)
 * and up alternate; qzeros / scales / bias (nullable) are in that column
 * order too.  Decode shapes (the GEMV's conditions, at most 8 column blocks
 * per CU) apply SwiGLU in the GEMV's epilogue, or with K > 4096 in the reduce
 * of its K chunks, and prefill shapes (M > 64) in the prefill GEMM's; other
 * shapes run the tiled GEMM into the workspace and one elementwise pass
 * (kq_w4a16_swiglu_workspace_size bytes).  No reference counterpart: the
 * reference packs gate/up only for dense and NVFP4 projections
 * (kairyu/models/packed_linear.py:58-149) and applies SwiGLU separately. */
int kq_w4a16_tiled_swiglu_gemm(const void* x, int x_dtype, const int32_t* tiles,
                               const int32_t* qzeros, int zero_offset, const void* scales,
                               const int32_t* perm, const void* bias, int bias_dtype, void* out,
                               int64_t m, int64_t i_width, int64_t k, int group_size,
                               void* workspace, size_t workspace_bytes, void* stream);
size_t kq_w4a16_swiglu_workspace_size(int64_t m, int64_t i_width, int64_t k, int gidx_mode);

/* dst[m][n] = silu(gate) * up (as kq_w4a16_tiled_swiglu_gemm) from src
 * [m][2 * i_width] (row stride ld_src elements, dtype fp16 or bf16): gate
 * column n and up column i_width + n, or with `interleaved` 16-column blocks
 * of gate and up alternating.  SwiGLU of a packed W8A8 gate/up output
 * (kairyu/models/layers.py:243-244). */
int kq_swiglu(const void* src, int64_t ld_src, int interleaved, int dtype, void* dst, int64_t m,
              int64_t i_width, void* stream);

/* Allocation-free form of kq_w4a16_tiled_gemm, same arguments and results
 * except `workspace`: the call's scratch (act-order activation gather, the
 * prefill GEMM's staged activations, split-K partial sums) lives in a fixed
 * device array of KQ_W4A16_NOALLOC_SCRATCH_BYTES that the library holds on
 * every GPU it runs on until the process ends.  A shape whose
 * kq_w4a16_workspace_size() exceeds that size fails with KQ_EWORKSPACE before
 * anything is launched.  The call allocates nothing (no hipMalloc, no
 * allocating library routine), for callers that cannot allocate: code under
 * HIP graph capture, tight serving loops, harnesses that forbid allocation.
 * Calls on one GPU share its array: calls that overlap on one GPU (two
 * streams, or two threads) race; order them on one stream.  The first call on
 * each GPU resolves the array's device address (hipGetSymbolAddress), so make
 * one eager call per GPU before capturing this entry in a HIP graph; captured
 * launches then replay with no host work.  No counterpart in the reference. */
#define KQ_W4A16_NOALLOC_SCRATCH_BYTES (16u << 20)
int kq_w4a16_tiled_gemm_noalloc(const void* x, int x_dtype, const int32_t* tiles,
                                const int32_t* qzeros, int zero_offset, const void* scales,
                                const int32_t* perm, const void* bias, int bias_dtype, void* out,
                                int64_t m, int64_t n, int64_t k, int group_size, void* stream);

/* Bytes of `workspace` a W4A16 call of this shape needs (gidx_mode as for
 * kq_w4a16_gptq_gemm; AWQ uses 0).  No reference counterpart: sizing helper
 * for the caller-owned scratch buffer. */
size_t kq_w4a16_workspace_size(int64_t m, int64_t n, int64_t k, int gidx_mode);

/* Load-time act-order repack: out row j of the unpacked [k, n] nibble matrix
 * is source row perm[j]; packing stays GPTQ (k/8 words, LSB-first).  Derived
 * operand only; checkpoint buffers are untouched (the reference caches derived
 * runtime operands the same way, quant_gemm_gpu.py:802-850). */
int kq_gptq_permute_qweight(const int32_t* qweight, const int32_t* perm, int32_t* out,
                            int64_t n, int64_t k, void* stream);

/* ------------------------------------------------ block-FP8 and MoE experts
 * Block FP8: weight e4m3 [n, k] with fp32 weight_scale_inv [ceil(n/128),
 * ceil(k/128)], W = q * S[n/128][k/128]; activations quantized per token per
 * 128-wide K block, s = max(amax, 1e-12) / 448, q = e4m3(clamp(x / s, +-448))
 * (the finegrained_fp8_linear(..., block_size=[128, 128]) convention the
 * reference calls at kairyu/kernels/deepseek_v4_moe_gpu.py:60-74). */

/* Per token, per 128-wide block quantization of x [rows, k] (fp16/bf16,
 * k <= 65535 * 2048): xq e4m3 [rows, k], xs fp32 [rows, ceil(k/128)].  Replaces the activation
 * side of finegrained_fp8_linear (deepseek_v4_moe_gpu.py:60-74). */
int kq_act_quant_fp8_blocks(const void* x, int x_dtype, int64_t rows, int64_t k, int64_t ldx,
                            uint8_t* xq, float* xs, void* stream);

/* Dense block-FP8 linear: out[m, n] = sum over 128-wide K blocks b of
 * (xq . w) * xs[m][b] * ws[n/128][b] (fp32) + bias, cast to out_dtype;
 * k % 128 == 0.  Replaces finegrained_fp8_linear (deepseek_v4_moe_gpu.py:60-74)
 * for BlockFp8Linear. */
int kq_block_fp8_gemm(const uint8_t* xq, const float* xs, const uint8_t* w, const float* ws,
                      const void* bias, int bias_dtype, void* out, int out_dtype, int64_t m,
                      int64_t n, int64_t k, void* stream);

/* Qwen3 routing of logits [tokens, experts] (fp16/bf16/fp32; experts <= 512,
 * top_k <= 32): stable descending top-k (ties -> smaller expert id) into
 * topk_idx int32 [tokens, top_k]; topk_w fp32 = softmax of the selected
 * logits (norm_topk_prob != 0) or the full softmax gathered at the
 * selection.  Replaces route_experts' Qwen3 branch (kairyu/models/moe.py:255-273). */
int kq_moe_route_topk(const void* logits, int dtype, int64_t tokens, int64_t experts, int top_k,
                      int norm_topk_prob, int32_t* topk_idx, float* topk_w, void* stream);

/* Bytes of workspace kq_moe_block_fp8_experts and
 * kq_moe_routed_block_fp8_experts need for this shape. */
size_t kq_moe_workspace_size(int64_t tokens, int64_t hidden, int64_t inter, int64_t experts,
                             int top_k);

/* Routed block-FP8 SwiGLU experts + combine: for token t and slot s with
 * expert e = topk_idx[t, s], y = down_e(bf16(silu(gate_e(x_t))) * up_e(x_t))
 * (each projection a block-FP8 linear rounded to the hidden dtype); out[t] =
 * sum over s in slot order of fp32(y) * topk_w[t, s], one final cast.
 * w13 e4m3 [experts, 2*inter, hidden] (gate rows then up rows), s13 fp32
 * [experts, 2*inter/128, hidden/128]; w2 e4m3 [experts, hidden, inter], s2
 * fp32 [experts, hidden/128, inter/128]; hidden, inter multiples of 128.
 * Device-side stable sort by expert, grouped GEMMs, no host synchronization.
 * Replaces _mix_experts / GroupedExpertPack.forward / the EP slot-order
 * combine (kairyu/models/moe.py:86-119, grouped_moe.py:239-330,
 * moe_parallel.py:255-283) for block-FP8 experts. */
int kq_moe_block_fp8_experts(const void* hidden, int dtype, int64_t tokens, int64_t hidden_size,
                             int64_t inter, int64_t experts, int top_k, const int32_t* topk_idx,
                             const float* topk_w, const uint8_t* w13, const float* s13,
                             const uint8_t* w2, const float* s2, void* out, void* workspace,
                             size_t workspace_bytes, void* stream);

/* The Qwen3 sparse block from its router logits: kq_moe_route_topk's routing
 * (logits fp16/bf16/fp32 [tokens, experts], experts <= 512, top_k <= 32;
 * topk_idx int32 and topk_w fp32 [tokens, top_k] are written as that call
 * writes them) followed by kq_moe_block_fp8_experts, with the same outputs
 * bit for bit.  The routing, the sort's expert histograms and the token
 * quantization share one launch.  Replaces route_experts + _mix_experts of
 * the sparse block's forward (kairyu/models/moe.py:255-273, 86-119,
 * 324-332). */
int kq_moe_routed_block_fp8_experts(const void* logits, int logits_dtype, int norm_topk_prob,
                                    const void* hidden, int dtype, int64_t tokens,
                                    int64_t hidden_size, int64_t inter, int64_t experts, int top_k,
                                    const uint8_t* w13, const float* s13, const uint8_t* w2,
                                    const float* s2, int32_t* topk_idx, float* topk_w, void* out,
                                    void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- ceilings
 * Measurement aids, no counterpart in the reference: the box's own ceilings
 * that bench.py --peaks reports next to the vendor peaks.  `sink` is device
 * memory of workgroups * 256 uint32 (written only if a fold of the data hits
 * a fixed value, which keeps the work live). */

/* Streaming read of `bytes` (a positive multiple of 16, 16-byte aligned) from
 * `src`: 256-thread workgroups, grid-strided 16-byte loads, 8 in flight per
 * thread.  Bytes moved per launch = `bytes`. */
int kq_peak_stream_read(const void* src, int64_t bytes, int workgroups, void* sink, void* stream);

/* Register-only MFMA loop: every wave of `workgroups` 256-thread workgroups
 * runs `iterations` x KQ_PEAK_MFMA_CHAINS independent MFMAs of `kind`:
 *   KQ_PEAK_FP16  v_mfma_f32_16x16x32_f16            16384 FLOP each
 *   KQ_PEAK_FP8   v_mfma_scale_f32_16x16x128_f8f6f4  65536 FLOP each (e4m3)
 *   KQ_PEAK_INT8  v_mfma_i32_16x16x64_i8             32768 OP each
 * (the instructions the W4A16, FP8 and INT8 GEMMs issue). */
#define KQ_PEAK_FP16 0
#define KQ_PEAK_FP8 1
#define KQ_PEAK_INT8 2
#define KQ_PEAK_MFMA_CHAINS 8
int kq_peak_mfma(int kind, int64_t iterations, int workgroups, void* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KAIRYU_QUANT_H */
