/*
 * dflash.h - C ABI of the MI355X (gfx950) DeBERTa disentangled-attention library.
 *
 * Plain pointers and sizes only: every tensor argument is a device pointer to
 * memory the caller owns; the library allocates nothing (the split-key form
 * takes a workspace from the caller) and launches on the HIP stream it is
 * given (NULL = the default stream).  Calls are asynchronous
 * with respect to the host, like the kernel launch they replace.
 *
 * Return value: 0 on success, a negative DFLASH_ERR_* code for an argument
 * error detected on the host (nothing is launched), or a positive hipError_t
 * from the launch.  dflash_error_string() turns either into text.
 *
 * dtype codes: 0 = fp16, 1 = bf16, 2 = fp32.  Head dimension D is 32, 64 or 128.
 */
#ifndef DFLASH_H_
#define DFLASH_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DFLASH_API __attribute__((visibility("default")))

#define DFLASH_ABI_VERSION 7

#define DFLASH_DTYPE_FP16 0
#define DFLASH_DTYPE_BF16 1
#define DFLASH_DTYPE_FP32 2

#define DFLASH_OK 0
#define DFLASH_ERR_NULL (-1)
#define DFLASH_ERR_SHAPE (-2)
#define DFLASH_ERR_HEAD_DIM (-3)
#define DFLASH_ERR_DTYPE (-4)
#define DFLASH_ERR_ALIGN (-5)
#define DFLASH_ERR_TOO_LARGE (-6)
#define DFLASH_ERR_WORKSPACE (-7)
#define DFLASH_ERR_SCRATCH (-8)
#define DFLASH_ERR_BUSY (-9)

/* Activation codes of the ConvLayer tail (the module's conv_act). */
#define DFLASH_ACT_GELU 0 /* exact erf form, Hugging Face ACT2FN["gelu"] */
#define DFLASH_ACT_TANH 1
#define DFLASH_ACT_RELU 2

/*
 * Fused attention over precomputed relative-score tables.
 *
 * Replaces the reference op torch.ops.gliner2_attention.deberta_attention
 * (/root/reference/src/disentangled_flash/kernel.py:368-438, kernel body
 * kernel.py:137-345) argument for argument:
 *   query, key, value : [B, H, L, D] contiguous, dtype `dtype`
 *   c2p, p2c          : [B, H, L, S] contiguous, unscaled Q.Kr^T / K.Qr^T over
 *                       the active slots; ignored (may be NULL) when the mode is off
 *   delta_to_local    : int32 [2L-1], local slot of delta i-j at index i-j+L-1
 *   attention_mask    : uint8 [B, L], nonzero = kept token (the reference's bool mask)
 *   out               : [B, L, H*D], dtype `dtype`
 *   score_scale_log2  : log2(e) / sqrt(D * (1 + has_c2p + has_p2c))  (kernel.py:587-588)
 *   strict_fp32       : fp32 only: 1 = fp32-accurate products (as for the
 *                       relative entry points below); 0 = the reference's
 *                       TF32 mode (kernel.py:211-223), here QK and PV as three
 *                       bf16 products each (about 2^-16 relative error per
 *                       product, against TF32's 2^-11).  Ignored for fp16/bf16.
 * B == 0 is a no-op that returns 0 (pointers are not inspected), like the
 * reference's launch over an empty grid.  query, key, value and out must be
 * 16-byte aligned (DFLASH_ERR_ALIGN); one (b, h) slice of a table,
 * L * S * sizeof(element), must stay below 2^31 bytes (DFLASH_ERR_TOO_LARGE).
 * Entries of delta_to_local outside [0, S) give undefined values (they read
 * slot S - 1); every read stays inside the c2p / p2c tensors.
 */
DFLASH_API int dflash_attention_fwd(const void* query, const void* key, const void* value,
                         const void* c2p, const void* p2c, const int32_t* delta_to_local,
                         const uint8_t* attention_mask, void* out, int B, int H, int L, int D,
                         int S, float score_scale_log2, int has_c2p, int has_p2c, int dtype,
                         int strict_fp32, void* stream);

/*
 * Fused attention computing the relative scores inside the kernel.
 *
 * Same output contract as dflash_attention_fwd, but it takes the projected
 * active relative rows instead of the [B, H, L, S] tables, so the separate
 * C2P/P2C GEMMs of the reference's forward_prepared
 * (/root/reference/src/disentangled_flash/kernel.py:574-585) and their
 * 2 x B*H*L*S HBM round trip disappear:
 *   query/key/value   : element (b, h, i, :) at base + b*stride_b + h*stride_h + i*stride_l,
 *                       D contiguous elements; strides in elements, 16-byte aligned.
 *                       Pass the three column blocks of the fused QKV projection
 *                       output [B, L, 3*H*D] directly (stride_b = 3*H*D*L,
 *                       stride_h = D, stride_l = 3*H*D) - no head reshape copy.
 *   pos_key, pos_query: [H, S, D] contiguous, the plan's pos_key / pos_query
 *                       (kernel.py:461-468, 522-523)
 *   delta_to_local    : as above; any table (the kernel builds its relative
 *                       windows per delta, gathering rows through the table).
 *   strict_fp32       : fp32 only.  1 = the reference's strict mode
 *                       (input_precision="ieee", kernel.py:216): fp32-accurate
 *                       products, IEEE fp32 MFMA (v_mfma_f32_16x16x4_f32) at
 *                       D = 128 with the c2p term and, otherwise, six bf16
 *                       MFMAs over a
 *                       three-way bf16 split of each operand (all 24 significand
 *                       bits; the dropped part products are below 2^-24 of the
 *                       leading one).  0 = the reference's fast mode, which is
 *                       TF32 there (kernel.py:222); gfx950 has no TF32 matrix
 *                       path, so each fp32 operand is split into bf16 hi + lo
 *                       and the product runs as three bf16 MFMAs (relative error
 *                       about 2^-16 per product, below TF32's 2^-11).
 * B == 0 is a no-op that returns 0 (pointers are not inspected).
 * DFLASH_ERR_TOO_LARGE when L * stride_l elements or the S * D elements of one
 * head's relative rows reach 2^31 bytes (the kernel's 32-bit buffer offsets).
 */
DFLASH_API int dflash_attention_rel_fwd(const void* query, const void* key, const void* value,
                             int64_t stride_b, int64_t stride_h, int64_t stride_l,
                             const void* pos_key, const void* pos_query,
                             const int32_t* delta_to_local, const uint8_t* attention_mask,
                             void* out, int B, int H, int L, int D, int S,
                             float score_scale_log2, int has_c2p, int has_p2c, int dtype,
                             int strict_fp32, void* stream);

/*
 * Split-key plan for dflash_attention_rel_fwd_split on the current device.
 *
 * No counterpart in the reference, whose launch grid is always
 * (cdiv(L, BM), B*H) (/root/reference/src/disentangled_flash/kernel.py:405-417).
 * When that grid leaves most of the GPU idle (small batches: B=1, L=512, H=12
 * gives 48 workgroups for 256 CUs), splitting the key range of every query
 * block over `splits` workgroups and merging their partial rows fills it.  *splits on entry: 0 = choose for this shape and the current
 * device, 1..8 = the caller's count.  On return *splits is the count the split
 * form runs (1 = no split; fewer than requested when L has fewer key tiles)
 * and *workspace_bytes the workspace it needs (0 for 1).
 */
DFLASH_API int dflash_attention_rel_split_plan(int B, int H, int L, int D, int* splits,
                                               size_t* workspace_bytes);

/*
 * dflash_attention_rel_fwd with the key range of every query block split over
 * `splits` workgroups (1..8; fewer are used when L has fewer key tiles).
 * Same arguments, output and numerics contract; in addition:
 *   splits          : the split count, normally from dflash_attention_rel_split_plan
 *   workspace       : device memory of at least the plan's workspace_bytes for this
 *                     split count, 16-byte aligned, owned by the caller; it holds the
 *                     partial rows (fp32) between the kernel and the merge, both
 *                     launched on `stream`.  Calls that share a workspace must not
 *                     overlap.  May be NULL when splits <= 1.
 * splits <= 1 and dtype fp32 (which has no split form) run dflash_attention_rel_fwd
 * unchanged.
 * Returns DFLASH_ERR_WORKSPACE when workspace_bytes is too small.
 */
DFLASH_API int dflash_attention_rel_fwd_split(const void* query, const void* key,
                                              const void* value, int64_t stride_b,
                                              int64_t stride_h, int64_t stride_l,
                                              const void* pos_key, const void* pos_query,
                                              const int32_t* delta_to_local,
                                              const uint8_t* attention_mask, void* out, int B,
                                              int H, int L, int D, int S, float score_scale_log2,
                                              int has_c2p, int has_p2c, int dtype,
                                              int strict_fp32, int splits, void* workspace,
                                              size_t workspace_bytes, void* stream);

/*
 * dflash_attention_rel_fwd_split without a caller workspace and without any
 * allocation.
 *
 * No counterpart in the reference.  It is for callers that cannot allocate
 * device memory at call time (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The partial rows of the split-key
 * form live in a static device array of the library,
 * dflash_attention_rel_noalloc_scratch_bytes() bytes (16 MiB) per GPU, held
 * until the process ends; its address is looked up once per device at the
 * first call on that device.  The function calls no hipMalloc, hipFree or
 * allocating library routine.
 *   splits : 0 = the count dflash_attention_rel_split_plan would choose on the
 *            current device; 1..8 = the caller's count (as in
 *            dflash_attention_rel_fwd_split).  fp32 never splits.
 * Returns DFLASH_ERR_SCRATCH (nothing launched) when the split workspace of
 * that count exceeds the scratch.  With splits = 0 on a 256-CU MI355X the
 * plan never needs more than 8.7 MB, so only forced counts on large shapes
 * are refused.
 * All calls on one GPU share that GPU's scratch.  Calls on one stream are
 * ordered by it.  A split call issued from another stream while the last split
 * call's kernels are still pending returns DFLASH_ERR_BUSY and launches nothing
 * (the library records an event after each split call and queries it).  While
 * the stream is being captured into a HIP graph nothing is recorded or checked:
 * replays of graphs that use the scratch must not overlap each other or another
 * split call on the same GPU.  The scratch keeps the last call's contents; every
 * call writes all the partial rows it reads, so nothing needs clearing.
 */
DFLASH_API int dflash_attention_rel_fwd_noalloc(const void* query, const void* key,
                                                const void* value, int64_t stride_b,
                                                int64_t stride_h, int64_t stride_l,
                                                const void* pos_key, const void* pos_query,
                                                const int32_t* delta_to_local,
                                                const uint8_t* attention_mask, void* out, int B,
                                                int H, int L, int D, int S,
                                                float score_scale_log2, int has_c2p, int has_p2c,
                                                int dtype, int strict_fp32, int splits,
                                                void* stream);

/* Size in bytes of the per-GPU static scratch of dflash_attention_rel_fwd_noalloc. */
DFLASH_API size_t dflash_attention_rel_noalloc_scratch_bytes(void);

/*
 * Fused residual add + LayerNorm of an encoder layer output.
 *
 * Replaces the tail of DebertaV2SelfOutput.forward and DebertaV2Output.forward,
 * LayerNorm(dense(x) + input_tensor)
 * (/root/reference/src/disentangled_flash/_reference.py:108-112 and 482-485;
 * the dropout between them is the identity in inference), for the encoder
 * loop of DebertaV2InferenceEncoder.forward_prepared
 * (/root/reference/src/disentangled_flash/deberta.py:262-276):
 *   x, residual, out : [rows, hidden], dtype `dtype`, contiguous
 *   gamma, beta      : [hidden], dtype `dtype` (the LayerNorm weight and bias)
 *   out = LayerNorm(T(x + residual)) with eps, statistics in fp32.
 *   residual may be NULL: out = LayerNorm(x) (x already holds the sum, e.g. from
 *   dflash_linear_fwd with DFLASH_GEMM_BIAS_ADD).
 * hidden must be a multiple of 4 and at most 4096; pointers 4-element aligned.
 * rows == 0 is a no-op (pointers are not inspected).
 */
DFLASH_API int dflash_add_layernorm_fwd(const void* x, const void* residual, const void* gamma,
                                        const void* beta, void* out, int rows, int hidden,
                                        float eps, int dtype, void* stream);

/*
 * Tail of the ConvLayer applied after the first encoder layer.
 *
 * Replaces ConvLayer.forward (/root/reference/src/disentangled_flash/_reference.py:536-566)
 * as called by the encoder loop (/root/reference/src/disentangled_flash/deberta.py:272-273),
 * from the convolution output on, for Conv1d(hidden, hidden, 3, padding=1, groups=1):
 *   z          : [B*L, 3*hidden], dtype `z_dtype` (fp32, or `dtype`): the products of
 *                the layer input rows with the three taps, z[:, k*hidden + o] =
 *                sum_i x[:, i] * conv.weight[o, i, k]
 *   residual   : [B*L, hidden], dtype `dtype` (the layer-0 output, residual_states)
 *   conv_bias, gamma, beta : [hidden], dtype `dtype` (conv.bias, LayerNorm weight/bias)
 *   mask       : int64 [B, L], the caller's attention mask (a bool mask passed as 0/1)
 *   out        : [B*L, hidden], dtype `dtype`
 *   act        : DFLASH_ACT_* (the module's conv_act)
 * out = T(LayerNorm(T(residual + T(act(T(conv) or 0 where mask != 1)))) * T(mask)), conv
 * summed in fp32 from the taps at l-1, l, l+1 of the same sequence plus conv_bias.
 * hidden must be a multiple of 4 and at most 4096; pointers 4-element aligned, mask
 * 8-byte aligned.  B*L == 0 is a no-op.
 */
DFLASH_API int dflash_conv_layer_tail_fwd(const void* z, int z_dtype, const void* residual,
                                          const void* conv_bias, const void* gamma,
                                          const void* beta, const int64_t* mask, void* out,
                                          int B, int L, int hidden, float eps, int act, int dtype,
                                          void* stream);

/* Epilogue codes of dflash_linear_fwd. */
#define DFLASH_GEMM_BIAS 0      /* y = T(x.W^T + b) */
#define DFLASH_GEMM_BIAS_GELU 1 /* y = T(gelu_erf(T(x.W^T + b))) */
#define DFLASH_GEMM_BIAS_ADD 2  /* y = T(T(x.W^T + b) + residual) */

/*
 * Dense projection with a fused epilogue: y[M, N] = epilogue(x[M, K] . W[N, K]^T + bias).
 *
 * Replaces the nn.Linear calls of the encoder layer (F.linear = hipBLASLt in
 * the reference's torch path) together with what follows them:
 *   DFLASH_GEMM_BIAS      : the fused QKV projection of forward_prepared
 *                           (/root/reference/src/disentangled_flash/_torch.py:284-297,
 *                           weight concatenated at _torch.py:112-123)
 *   DFLASH_GEMM_BIAS_GELU : DebertaV2Intermediate, dense then exact-erf GELU
 *                           (/root/reference/src/disentangled_flash/_reference.py:470-471)
 *   DFLASH_GEMM_BIAS_ADD  : dense + residual of DebertaV2SelfOutput/DebertaV2Output
 *                           before their LayerNorm (_reference.py:108-112, 482-485)
 * The sum is rounded to the dtype before the epilogue, as nn.Linear's output is.
 *   x        : [M, K] row-major; weight: [N, K] row-major (the nn.Linear weight)
 *   bias     : [N]; residual: [M, N] row-major (DFLASH_GEMM_BIAS_ADD only, else may be NULL)
 *   y        : [M, N] row-major
 *   dtype    : fp16 or bf16 (fp32 is not supported: DFLASH_ERR_DTYPE)
 * N must be a multiple of 64 and K of 32 (DFLASH_ERR_SHAPE otherwise; every
 * projection of DeBERTa base/large/xlarge qualifies; the automatic configuration
 * runs the 64 x 64 tiles when N is a multiple of neither 128 nor 192, at any M);
 * x, weight, residual, y
 * 16-byte aligned, bias 8-byte aligned.  M == 0 is a no-op.
 *   epilogue : the code above in bits 0-7; bits 8 and up select a tile
 *              configuration (0 = automatic by N and epilogue): 1 = 256 x 192
 *              tiles, 4 wavefronts (N % 192 == 0); 2 = 256 x 128 at two workgroups per CU
 *              (N % 128 == 0); 3 = 256 x 192, 8 wavefronts (N % 192 == 0);
 *              4 = 64 x 128 at three per CU (N % 128 == 0); 5 = 64 x 64 at four
 *              per CU (N % 64 == 0).  The 64-row forms give four times the tiles
 *              for few rows.  A configuration that does not fit N returns
 *              DFLASH_ERR_SHAPE.
 */
DFLASH_API int dflash_linear_fwd(const void* x, const void* weight, const void* bias,
                                 const void* residual, void* y, int M, int N, int K,
                                 int epilogue, int dtype, void* stream);

/* Text for a return code of any dflash_* entry point. */
DFLASH_API const char* dflash_error_string(int code);

/* DFLASH_ABI_VERSION of the loaded library. */
DFLASH_API int dflash_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DFLASH_H_ */
