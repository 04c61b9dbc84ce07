/*
 * shape_aware_hip.h - C ABI of the MI355X (gfx950) Transformer forward hot path.
 *
 * Every entry point takes raw device pointers, int64 sizes and strides (in
 * elements), scalars and a hipStream_t.  None of them allocates, synchronizes
 * or throws: work is enqueued asynchronously on `stream` and the return value
 * is a status code (SAH_OK on success).  sah_last_error() returns a
 * thread-local description of the most recent failure on the calling thread.
 *
 * The reference project binds the equivalent kernels from Python through
 * torch.library custom ops; the Python side of this project binds these
 * symbols with ctypes (solution/kernels/hip/_library.py) and registers the same
 * kind of custom ops around them.
 */
#ifndef SHAPE_AWARE_HIP_H_
#define SHAPE_AWARE_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* hipStream_t is an opaque pointer; declared here so the header does not need
 * the HIP headers (a NULL stream is the legacy default stream). */
typedef struct ihipStream_t* sah_stream_t;

#define SAH_ABI_VERSION 1

typedef enum {
  SAH_DTYPE_F32 = 0,
  SAH_DTYPE_F16 = 1,
  SAH_DTYPE_BF16 = 2
} sah_dtype;

typedef enum {
  SAH_OK = 0,
  SAH_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size, bad stride, bad alignment */
  SAH_ERR_UNSUPPORTED = 2,      /* shape/dtype/launch outside the implemented kernels */
  SAH_ERR_HIP = 3,              /* a HIP runtime call or launch failed */
  SAH_ERR_WORKSPACE = 4         /* workspace missing or too small */
} sah_status;

typedef enum {
  SAH_NORM_LAYER = 0, /* y = (x - mean) * rsqrt(var + eps) * weight + bias, biased var */
  SAH_NORM_RMS = 1    /* y = x * rsqrt(mean(x^2) + eps) * weight (+ bias if given)     */
} sah_norm_kind;

/* Library identity. */
int sah_abi_version(void);
const char* sah_last_error(void);

/*
 * Causal multi-head attention forward with head_dim 64 and the output written
 * directly in [B, S, H*64] ("BSD") layout.
 *
 * Replaces the reference's
 *   _streaming_dh64_causal_attention_bsd_op  (solution/shape14/triton_streaming_dh64.py:200-242)
 *   _streaming_dh64_causal_attention_kernel (solution/shape14/triton_streaming_dh64.py:69-190)
 * with the same meaning of every argument: query/key/value are [B, H, S, 64]
 * tensors given by pointer + strides (the packed-QKV view of
 * solution/operators/projection/qkv_layout.py:22-50 is accepted as is),
 * `scale` multiplies QK^T before the causal softmax, softmax statistics and
 * accumulation are fp32, and P is rounded to the input dtype before PV.
 *
 * dtype: SAH_DTYPE_BF16 or SAH_DTYPE_F16 for q, k, v and output.
 * q/k: the head_dim stride must be 1, the seq stride a multiple of 8 and the
 *      base 16-byte aligned; the key seq stride must lie in [0, 2^24).
 * v:   either head_dim-contiguous (v_stride_d == 1, the reference layout,
 *      any key stride in [0, 2^24) such as the packed QKV view's; read as
 *      given, the PV operand transposed on its way out of LDS) or
 *      seq-contiguous (v_stride_s == 1, a V^T buffer, any v_stride_d that is
 *      a multiple of 8; first copied key-major into `workspace`).  Tiles of
 *      64 key rows are addressed at 32-bit offsets; a larger key stride
 *      returns SAH_ERR_UNSUPPORTED.
 * workspace: 16-byte aligned, at least sah_causal_attention_workspace_bytes();
 *      may be null when that is 0.  Sequences of 4096 keys or more keep
 *      there, written by one preparation launch over Q and K: a table
 *      of the largest key norm of every 64-key tile, which bounds every score
 *      so that most tiles skip their row maximum, tables of the largest key
 *      and query norm of every 512-row block, and the keys times
 *      scale * log2(e) in fp16.  A block of 512 query rows whose bound
 *      scale * log2(e) * max|q| * max|k| is at most 32 (15 for fp16) computes
 *      its scores on the fp16 MFMA from those keys and takes P = exp2(score)
 *      without a shift; other blocks keep the shifted path.
 * out: [B, S, H*64], element stride 1 on the feature axis.
 * Launch parameters: (block_m query rows, num_warps wavefronts) per workgroup
 *      in {(128, 4), (256, 4), (256, 8), (512, 8)} (32 or 64 query rows per
 *      wavefront), block_n == 64 keys per tile, num_stages 1 or 2 (LDS
 *      buffers), or 3 for (128, 4) (the software-pipelined kernel)
 *      (sah_causal_attention_launch_supported() reports the implemented set).
 */
int sah_causal_attention_bsd(
    const void* query, const void* key, const void* value, void* output,
    int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
    int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
    int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s, int64_t v_stride_d,
    int64_t o_stride_b, int64_t o_stride_s,
    float scale, int dtype,
    int block_m, int block_n, int num_warps, int num_stages,
    void* workspace, size_t workspace_bytes,
    sah_stream_t stream);

/* Workspace bytes sah_causal_attention_bsd needs (the most over its
 * launches): for seq_len >= 4096 the key-norm table (4 bytes per 64-key tile
 * per head, rounded up to 256), the key and query block-norm tables (8 bytes
 * per 512-row block per head, rounded up to 256) and the fp16 scaled keys
 * (128 bytes per key, seq_len rounded up to 64, per head), then, for a
 * seq-contiguous value, its key-major copy (128 bytes per key per head);
 * 0 for a head_dim-contiguous value shorter than 4096 keys.  The pipelined
 * launch (num_stages 3) uses at most the copy. */
size_t sah_causal_attention_workspace_bytes(
    int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
    int64_t v_stride_s, int64_t v_stride_d, int dtype);

/*
 * sah_causal_attention_bsd for callers that cannot allocate device memory.
 *
 * No counterpart in the reference (its Triton launcher allocates nothing
 * beyond the output).  It is for callers that may not call hipMalloc: code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation.  Arguments are those of sah_causal_attention_bsd without the
 * workspace pair: the workspace is a static device array of
 * SAH_ATTENTION_STATIC_WORKSPACE_BYTES (64 MiB) that each GPU holds for the
 * life of the process.  A call whose workspace (that of
 * sah_causal_attention_bsd: norm tables and fp16 scaled keys from 4096 keys
 * on, the key-major copy of a seq-contiguous V) fits the array runs as one
 * call.  A larger one runs in chunks of heads of one batch row whose
 * workspace fits (for example BASELINE C4's B16 H32 S4096, 268 MB of scaled
 * keys: one call per batch row of 32 heads); heads are independent and each
 * takes its path from its own tables, so the result is bitwise that of
 * sah_causal_attention_bsd.  When even one head's prepared layout is above
 * the array, every chunk runs the shifted path without the preparation
 * launch, as below 4096 keys (equal to sah_causal_attention_bsd's result to
 * the 16-bit tolerance, not bitwise).  A call for which one head's workspace
 * still exceeds the array (a seq-contiguous V of more than 524288 keys)
 * returns SAH_ERR_WORKSPACE before any launch.  All calls on one GPU share its
 * array:
 * calls that may overlap on that GPU (different streams, or host threads)
 * race on it and must be serialized by the caller.  Nothing in it needs to
 * start at zero; every call writes what it reads.
 */
#define SAH_ATTENTION_STATIC_WORKSPACE_BYTES (64ull << 20)
int sah_causal_attention_bsd_static_workspace(
    const void* query, const void* key, const void* value, void* output,
    int64_t batch, int64_t heads, int64_t seq_len, int64_t head_dim,
    int64_t q_stride_b, int64_t q_stride_h, int64_t q_stride_s,
    int64_t k_stride_b, int64_t k_stride_h, int64_t k_stride_s,
    int64_t v_stride_b, int64_t v_stride_h, int64_t v_stride_s, int64_t v_stride_d,
    int64_t o_stride_b, int64_t o_stride_s,
    float scale, int dtype,
    int block_m, int block_n, int num_warps, int num_stages,
    sah_stream_t stream);

/* 1 when (block_m, block_n, num_warps, num_stages) is an implemented launch. */
int sah_causal_attention_launch_supported(int block_m, int block_n, int num_warps,
                                          int num_stages);

/*
 * Fused residual add + LayerNorm / RMSNorm over the last axis:
 *   residual   = round_to(value_dtype, value + update)
 *   normalized = round_to(normalized_dtype, norm(residual) * weight + bias)
 * Statistics are fp32, computed in one pass over HBM (per-lane Welford states
 * merged across the wavefront).  Both outputs may not alias the inputs.
 *
 * Replaces the reference's
 *   _residual_layer_norm_kernel        (solution/kernels/norm/triton_residual.py:39-71)        fp32 stream
 *   _mixed_residual_layer_norm_kernel  (solution/kernels/norm/triton_mixed_residual.py:41-76)  fp32 stream + 16-bit update
 *   residual_add + nn.LayerNorm        (solution/operators/norm/residual_add.py:28-39,
 *                                       solution/transformer.py:1629-1632)                      same-dtype stream
 * Implemented dtype combinations (value, update, normalized):
 *   (bf16,bf16,bf16) (f16,f16,f16) (f32,f32,f32)
 *   (f32,f16,f16) (f32,f16,f32) (f32,bf16,bf16) (f32,bf16,f32)
 * weight/bias: param_dtype (f32 or the value dtype); either may be NULL
 * (weight 1, bias 0).  width: 128, 256 or 512 x {1, 2, 4, 8, 16} for 16-bit
 * value dtypes, 128 or 256 x {1, 2, 4, 8, 16} for f32.  Rows are contiguous
 * (row stride == width).
 * block_rows rows per workgroup of num_warps wavefronts; block_rows must be a
 * multiple of num_warps; num_warps in {1, 2, 4, 8}.
 */
int sah_residual_norm(
    const void* value, const void* update, const void* weight, const void* bias,
    void* residual, void* normalized,
    int64_t rows, int64_t width, float eps,
    int value_dtype, int update_dtype, int normalized_dtype, int param_dtype,
    int norm_kind, int block_rows, int num_warps,
    sah_stream_t stream);

/*
 * LayerNorm / RMSNorm without a residual (the layer-0 "initial" norm):
 *   normalized = round_to(normalized_dtype, norm(value) * weight + bias)
 *
 * Replaces the reference's
 *   _initial_fp16_layer_norm_kernel (solution/kernels/norm/triton_initial.py:39-63)
 *   the TORCH initial norm           (solution/transformer.py:1403-1409)
 * Implemented (value, normalized): (bf16,bf16) (f16,f16) (f32,f32) (f32,f16) (f32,bf16).
 * Same width / launch rules as sah_residual_norm.
 */
int sah_norm(
    const void* value, const void* weight, const void* bias, void* normalized,
    int64_t rows, int64_t width, float eps,
    int value_dtype, int normalized_dtype, int param_dtype,
    int norm_kind, int block_rows, int num_warps,
    sah_stream_t stream);

typedef enum {
  SAH_ACTIVATION_NONE = 0,
  SAH_ACTIVATION_GELU_EXACT = 1 /* 0.5 v (1 + erf(v / sqrt(2))) */
} sah_activation;

/*
 * Linear layer with a fused epilogue:
 *   y = round_to(dtype, act(x weight^T + bias))
 * fp32 accumulation; the bias (optional, NULL for none) is added in fp32 and
 * the activation evaluated in fp32 before the single rounding.
 *
 * Replaces the reference's
 *   _linear_exact_gelu_kernel + prevalidated_triton_linear_exact_gelu
 *     (solution/kernels/ffn/triton_linear_exact_gelu.py:69-137, 182-234)   activation = GELU_EXACT
 *   the FFN input projection + exact GELU of the TORCH path
 *     (solution/transformer.py:828-842)
 * x: [rows, in_features] with row stride x_row_stride; weight: [out_features,
 * in_features] contiguous (nn.Linear layout); bias: [out_features]; y: [rows,
 * out_features] with row stride y_row_stride.  x, weight, bias and y share
 * dtype (SAH_DTYPE_BF16 or SAH_DTYPE_F16).  in_features must be a multiple of
 * 64 and out_features of 256; strides multiples of 8 elements; x, weight and y
 * 16-byte aligned, bias 8-byte aligned.  Launch: (block_m, block_n, block_k,
 * num_warps, num_stages) = (256, 256, 64, 8, 2), see
 * sah_linear_launch_supported().
 */
int sah_linear(
    const void* x, const void* weight, const void* bias, void* y,
    int64_t rows, int64_t in_features, int64_t out_features,
    int64_t x_row_stride, int64_t y_row_stride,
    int dtype, int activation,
    int block_m, int block_n, int block_k, int num_warps, int num_stages,
    sah_stream_t stream);

/* 1 if sah_linear implements this launch, else 0 (mirrors the reference's
 * _launch_config_is_valid, solution/kernels/ffn/triton_linear_exact_gelu.py:29-45). */
int sah_linear_launch_supported(int block_m, int block_n, int block_k, int num_warps,
                                int num_stages);

/*
 * Exact GELU of a contiguous 16-bit tensor: y = round_to(dtype, GELU(x)),
 * GELU(v) = 0.5 v (1 + erf(v / sqrt(2))) evaluated in fp32.  y may be x.
 *
 * Replaces the reference's
 *   _exact_gelu_kernel + prevalidated_triton_exact_gelu
 *     (solution/kernels/ffn/triton_exact_gelu.py:50-118)
 *   F.gelu(approximate="none") of the TORCH FFN path (solution/transformer.py:828-831)
 * x, y: n elements of dtype SAH_DTYPE_BF16 or SAH_DTYPE_F16, 16-byte aligned.
 * block_size elements per workgroup of num_warps wavefronts; block_size must be
 * 512 x num_warps x {1, 2, 4, 8}, num_warps in {1, 2, 4, 8}.
 */
int sah_gelu(const void* x, void* y, int64_t n, int dtype, int block_size, int num_warps,
             sah_stream_t stream);

/* 1 if sah_gelu implements (block_size, num_warps), else 0. */
int sah_gelu_launch_supported(int block_size, int num_warps);

/* Value layouts sah_qkv_projection can write. */
typedef enum {
  SAH_QKV_VALUE_BHSD = 0,     /* [B, H, S, head_dim] contiguous, like query and key */
  SAH_QKV_VALUE_SEQ_MAJOR = 1 /* [B, H, head_dim, value_seq_stride]: seq-contiguous
                                 (V^T; sah_causal_attention_bsd copies it key-major) */
} sah_qkv_value_layout;

/*
 * Packed QKV projection with a head-major epilogue:
 *   qkv = round_to(dtype, x weight^T + bias)   (fp32 accumulation, bias in fp32)
 * with output column c of [0, 3 d_model) written to
 *   query (c < d_model), key (c < 2 d_model) or value, head (c % d_model) / head_dim,
 *   element (c % d_model) % head_dim,
 * and row r to token (r / seq_len, r % seq_len).  No [B, S, 3 d_model]
 * intermediate exists.
 *
 * Replaces the reference's
 *   _qkv_native_bhsd_kernel + prevalidated_triton_qkv_native_bhsd
 *     (solution/kernels/projection/triton_qkv_layout.py:60-115, 170-230)
 *   the packed QKV projection + split_qkv of the default path
 *     (solution/transformer.py:432-435; solution/operators/projection/qkv_layout.py:22-50)
 * x: [batch * seq_len, d_model] with row stride x_row_stride; weight:
 * [3 d_model, d_model] contiguous (the packed qkv_proj weight, rows q | k | v);
 * bias: [3 d_model] or NULL; query, key: [batch, heads, seq_len, head_dim]
 * contiguous; value: the same, or (value_layout SAH_QKV_VALUE_SEQ_MAJOR)
 * [batch, heads, head_dim, value_seq_stride] with tokens [seq_len,
 * value_seq_stride) left untouched.  Shared dtype SAH_DTYPE_BF16 or
 * SAH_DTYPE_F16.  d_model must be a multiple of 256 and head_dim = d_model /
 * heads a multiple of 8; batch * seq_len below 2^31; x_row_stride and
 * value_seq_stride multiples of 8; all tensors 16-byte aligned, bias 8-byte.
 * Launch: (block_m, block_n, block_k, num_warps) = (256, 256, 64, 8), see
 * sah_qkv_launch_supported().
 */
int sah_qkv_projection(
    const void* x, const void* weight, const void* bias,
    void* query, void* key, void* value,
    int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads,
    int64_t x_row_stride, int value_layout, int64_t value_seq_stride,
    int dtype, int block_m, int block_n, int block_k, int num_warps,
    sah_stream_t stream);

/*
 * The model's first LayerNorm fused into the packed QKV projection:
 *   y   = round_to(dtype, (x - mean) * rstd * ln_weight + ln_bias)
 *         (mean, rstd = 1 / sqrt(var + ln_eps) of each x row in fp32, biased
 *          variance; y stays on chip)
 *   qkv = round_to(dtype, y weight^T + bias), stored as sah_qkv_projection does.
 * The row statistics are formed exactly as sah_norm forms them, so the outputs
 * equal those of sah_norm (LayerNorm, same weight, bias, eps, dtype) followed
 * by sah_qkv_projection, bit for bit.  Two launches on the stream: the row
 * statistics (mean, rstd as two floats per row) into the workspace, then the
 * projection, which normalizes x as it stages it.
 *
 * Replaces the reference's
 *   _initial_norm_qkv_native_bhsd_kernel + the fused initial-norm QKV launch
 *     (solution/kernels/projection/triton_shape07_initial_norm_qkv.py:67-140,
 *      173-218), which the reference plans as initial_norm TRITON_FUSED_QKV
 *      (solution/plan_builder.py:1097-1160) and calls for layer 0
 *      (solution/transformer.py:1364-1440).
 * Arguments as sah_qkv_projection, plus ln_weight / ln_bias: [d_model] in
 * dtype, 16-byte aligned, both required; ln_eps finite and >= 0; workspace:
 * device memory of at least sah_norm_qkv_workspace_bytes(batch, seq_len)
 * bytes, 16-byte aligned, else SAH_ERR_WORKSPACE before any launch (it only
 * carries the statistics between the two launches; calls that share one
 * workspace must not overlap).  d_model must be 512, 1024, 2048 or 4096.
 */
int sah_norm_qkv_projection(
    const void* x, const void* ln_weight, const void* ln_bias, float ln_eps,
    const void* weight, const void* bias,
    void* query, void* key, void* value,
    int64_t batch, int64_t seq_len, int64_t d_model, int64_t heads,
    int64_t x_row_stride, int value_layout, int64_t value_seq_stride,
    int dtype, int block_m, int block_n, int block_k, int num_warps,
    void* workspace, size_t workspace_bytes, sah_stream_t stream);

/* Workspace sah_norm_qkv_projection needs: 8 bytes per token (0 for an empty
 * or invalid size). */
size_t sah_norm_qkv_workspace_bytes(int64_t batch, int64_t seq_len);

/* 1 if sah_qkv_projection implements the launch, else 0 (mirrors the
 * reference's _launch_config_is_valid,
 * solution/kernels/projection/triton_qkv_layout.py:29-43). */
int sah_qkv_launch_supported(int block_m, int block_n, int block_k, int num_warps);

/*
 * Fused Linear + residual add + LayerNorm / RMSNorm boundary:
 *   update     = round_to(dtype, x weight^T + bias)   (fp32 accumulation, bias in fp32)
 *   residual   = round_to(dtype, value + update)
 *   normalized = round_to(dtype, norm(residual) * gamma + beta)
 * The update never reaches HBM.  The residual and norm arithmetic are those
 * of sah_residual_norm (statistics in fp32 over the rounded residual).
 *
 * Replaces the reference's
 *   _linear_residual_norm_kernel + triton_linear_residual_norm
 *     (solution/kernels/boundary/triton_linear_residual_norm.py:34-109, 197-245)
 *   the out_proj / ffn_out projection + _apply_residual_norm pair of the
 *   default path (solution/transformer.py:727-730, 1515-1644)
 * x: [rows, in_features] with row stride x_row_stride; weight: [width,
 * in_features] contiguous; bias, gamma, beta: [width] or NULL (0, 1, 0);
 * value, residual, normalized: [rows, width] contiguous, residual and
 * normalized not aliasing any input.  Shared dtype SAH_DTYPE_BF16 or
 * SAH_DTYPE_F16; norm_kind SAH_NORM_LAYER or SAH_NORM_RMS.  width 512 or
 * 1024, in_features a multiple of 64, x_row_stride a multiple of 8; tensors
 * 16-byte aligned, bias 8-byte.  Launch: block_rows = 65536 / width whole rows
 * per workgroup of num_warps = 8 wavefronts, see
 * sah_linear_residual_norm_launch_supported().
 */
int sah_linear_residual_norm(
    const void* x, const void* weight, const void* bias,
    const void* value, const void* gamma, const void* beta,
    void* residual, void* normalized,
    int64_t rows, int64_t in_features, int64_t width, int64_t x_row_stride,
    float eps, int dtype, int norm_kind, int block_rows, int num_warps,
    sah_stream_t stream);

/* 1 if sah_linear_residual_norm implements (width, block_rows, num_warps),
 * else 0 (mirrors the reference's _launch_is_valid,
 * solution/kernels/boundary/triton_linear_residual_norm.py:114-119). */
int sah_linear_residual_norm_launch_supported(int64_t width, int block_rows, int num_warps);

/*
 * The whole FFN fused through its residual add and LayerNorm / RMSNorm
 * boundary:
 *   hidden     = round_to(dtype, GELU(x w1^T + b1))   (fp32 accumulation, exact GELU)
 *   update     = round_to(dtype, hidden w2^T + b2)
 *   residual   = round_to(dtype, value + update)
 *   normalized = round_to(dtype, norm(residual) * gamma + beta)
 * Neither the hidden activation nor the update reaches HBM.  For a given
 * update, residual and normalized equal those of sah_residual_norm (same
 * norm, parameters, eps and dtype).
 *
 * Replaces the reference's
 *   _ffn_residual_norm_kernel + triton_ffn_residual_norm
 *     (solution/kernels/boundary/triton_ffn_residual_norm.py:44-135, 211-268),
 *   planned as FFNBackend TRITON_FUSED_MLP_BOUNDARY
 *   (solution/plan_builder.py:783-800; solution/transformer.py:844-896).
 * x: [rows, width] with row stride x_row_stride; w1: [ffn, width] and w2:
 * [width, ffn] contiguous (the ffn_in / ffn_out weights); b1 [ffn], b2, gamma,
 * beta [width], each may be NULL (0, 0, 1, 0); value, residual, normalized:
 * [rows, width] contiguous, residual and normalized not aliasing any input.
 * Shared dtype SAH_DTYPE_BF16 or SAH_DTYPE_F16; norm_kind SAH_NORM_LAYER or
 * SAH_NORM_RMS.  width 128 or 256 (the reference's kernel: 128), ffn a
 * multiple of 64; x_row_stride a multiple of 8; tensors 16-byte aligned,
 * biases 8-byte.  Launch: block_rows = 64 rows per workgroup of num_warps = 4
 * wavefronts, see sah_mlp_residual_norm_launch_supported().
 */
int sah_mlp_residual_norm(
    const void* x, const void* w1, const void* b1, const void* w2, const void* b2,
    const void* value, const void* gamma, const void* beta,
    void* residual, void* normalized,
    int64_t rows, int64_t width, int64_t ffn, int64_t x_row_stride,
    float eps, int dtype, int norm_kind, int block_rows, int num_warps,
    sah_stream_t stream);

/* 1 if sah_mlp_residual_norm implements (width, block_rows, num_warps), else 0
 * (mirrors the reference's _launch_is_valid,
 * solution/kernels/boundary/triton_ffn_residual_norm.py:30-38). */
int sah_mlp_residual_norm_launch_supported(int64_t width, int block_rows, int num_warps);

#ifdef __cplusplus
}
#endif

#endif /* SHAPE_AWARE_HIP_H_ */
