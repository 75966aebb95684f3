/*
 * qattn.h - C ABI of the MI355X (gfx950) quantized attention library (libqattn.so).
 *
 * Drop-in for the SageAttention-2 path TeleFuser reaches through
 * telefuser/ops/attention/attention_impl.py:245-283 -> tf_kernel.sageattn2 -> torch.ops.tf_kernel.*.
 * Every entry point takes device pointers, element strides and sizes, never allocates, launches
 * asynchronously on the given HIP stream and returns a status code (0 = OK).  On error the
 * message of the calling thread's last failure is available from qattn_last_error().
 *
 * Tensor views: a "sequence tensor" holds element (b, l, h, d) at
 *     data[b * sb + l * sl + h * sh + d]
 * with the head dim contiguous.  NHD ([B, L, H, D]) and HND ([B, H, L, D]) layouts are both
 * expressed by choosing the strides (reference tensor_layout 0/1, fused.cu:476-492).
 */
#ifndef QATTN_H_
#define QATTN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* qattn_stream_t; /* == hipStream_t */

/* element strides of a sequence tensor (head dim contiguous) */
typedef struct qattn_seq {
  void* data;
  int64_t sb, sl, sh;
} qattn_seq;

enum qattn_status {
  QATTN_OK = 0,
  QATTN_ERR_DTYPE = 1,      /* unsupported dtype code */
  QATTN_ERR_SHAPE = 2,      /* inconsistent or unsupported sizes */
  QATTN_ERR_STRIDE = 3,     /* strides not representable / not 16-byte aligned rows */
  QATTN_ERR_ALIGN = 4,      /* base pointer misaligned */
  QATTN_ERR_HEAD_DIM = 5,   /* head_dim other than 128 (or 64 where supported): callers pad the others */
  QATTN_ERR_HEAD_RATIO = 6, /* num_qo_heads % num_kv_heads != 0 */
  QATTN_ERR_WORKSPACE = 7,  /* workspace missing or too small */
  QATTN_ERR_LAUNCH = 8,     /* HIP launch error */
  QATTN_ERR_ARG = 9         /* other invalid argument */
};

enum qattn_dtype { QATTN_BF16 = 0, QATTN_FP16 = 1 };

/* Q/K scale granularity: the reference's QuantGranularity codes (attn_utils.cuh:41-64) */
enum qattn_gran {
  QATTN_GRAN_BLOCK = 1,
  QATTN_GRAN_WARP = 2,
  QATTN_GRAN_THREAD = 3,
  /* the same granularities with the scale tables of the reference's sm90 entry (sageattn2.py:1608-1624):
   * 64-row Q blocks of four 16-row warps, 128-row K blocks (shapes at qattn_quant_qk_per_warp_int8_ex) */
  QATTN_GRAN_WARP_SM90 = 4,
  QATTN_GRAN_THREAD_SM90 = 5
};

/* scale-table layout of the per-warp / per-thread quantizers (the *_ex entries) */
enum qattn_scale_layout {
  QATTN_SCALES_SM89 = 0, /* BLKQ 128, WARPQ 32, BLKK 64: the sm80/sm89 kernels' tables */
  QATTN_SCALES_SM90 = 1  /* BLKQ 64, WARPQ 16, BLKK 128 (WARPK 128): the sm90 kernel's tables */
};

/* V operand of qattn_fwd_ex */
enum qattn_v_kind { QATTN_V_FP8 = 0, QATTN_V_BF16 = 1, QATTN_V_FP16 = 2 };

/* rounding / smoothing semantics of the per-block INT8 quantizer */
enum qattn_quant_variant {
  QATTN_QUANT_CUDA = 0,  /* QuantInt8Kernel: fp32 (x - km) * sm_scale, amax floor 1e-7, RNE + saturate */
  QATTN_QUANT_TRITON = 1 /* quant_per_block_int8_kernel: half-rounded (x - km), no floor, round half away */
};

const char* qattn_last_error(void);
int qattn_version(void);

/*
 * Per-block INT8 quantization of one tensor.
 * Replaces torch.ops.tf_kernel.quant_per_block_int8_cuda_with_sm_scale, quant_per_block_int8_cuda and
 * quant_per_block_int8_fuse_sub_mean_cuda (tf-kernel/csrc/common_extension.cc:168-187,
 * tf-kernel/csrc/sageattn2/fused/fused.cu:447-696) and, with variant QATTN_QUANT_TRITON, the Triton
 * quant_per_block_int8_kernel (tf-kernel/tf_kernel/triton/quant_per_block.py:22-71).
 *   in:    sequence tensor [B, L, H, D] (bf16/fp16), D = 64 or 128
 *   mean:  NULL or [B, H, D] contiguous, same dtype as in (subtracted before quantization)
 *   out:   int8 sequence tensor (same sizes)
 *   scale: fp32 [B, H, ceil(L / block_size)] contiguous
 *   has_sm_scale: multiply by sm_scale (callers pass sm_scale * 1.44269504 for Q)
 *   block_size: 32, 64 or 128
 */
int qattn_quant_per_block_int8(qattn_seq in, int dtype, int64_t B, int64_t L, int64_t H, int64_t D,
                               const void* mean, qattn_seq out, float* scale, float sm_scale, int has_sm_scale,
                               int block_size, int variant, qattn_stream_t stream);

/*
 * Q and K quantized in one launch: Q with sm_scale folded in (block blkq), K with the optional mean
 * subtracted (block blkk).  Replaces the pair of launches in per_block_int8
 * (tf-kernel/tf_kernel/sageattn2.py:96-187).
 */
int qattn_quant_qk_per_block_int8(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t Lq, int64_t Lk,
                                  int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean, qattn_seq q_out,
                                  qattn_seq k_out, float* q_scale, float* k_scale, float sm_scale, int blkq,
                                  int blkk, int variant, qattn_stream_t stream);

/*
 * Per-warp INT8 quantization of Q and K in one launch: sageattn2.per_warp_int8 (sageattn2.py:190-280 ->
 * quant_per_warp_int8_cuda fused.cu:698-780 for Q, QuantInt8Kernel per 64-row block for K).  The
 * QuantInt8Kernel rounding (amax floor 1e-7, RNE + saturate), no sm_scale folded in:
 *   q_scale [B, Hq, ceil(Lq/128)*4]: one scale per 32 rows (empty trailing warp blocks: 1e-7/127);
 *   k_scale [B, Hkv, ceil(Lk/64)], K = k - k_mean in fp32 when k_mean is given.
 */
int qattn_quant_qk_per_warp_int8(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t Lq, int64_t Lk,
                                 int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean, qattn_seq q_out,
                                 qattn_seq k_out, float* q_scale, float* k_scale, qattn_stream_t stream);

/*
 * Per-thread INT8 quantization of Q and K in one launch: the Triton per_thread_int8 of the reference's
 * default SAGE_ATTN_2_8_8 path (tf-kernel/tf_kernel/triton/quant_per_thread.py:22-158,267-369;
 * chosen at sageattn2.py:1360-1365).  Scales follow the NVIDIA mma fragment a thread holds:
 *   q_scale [B, Hq, ceil(Lq/128)*32]: 32-row warp blocks, rows with equal row % 8 share a scale
 *     (index (row / 32) * 8 + row % 8; trailing warp blocks of the last 128-row block get 1e-7);
 *   k_scale [B, Hkv, ceil(Lk/64)*4]: 64-row blocks, rows with equal (row % 8) / 2 share a scale
 *     (index (row / 64) * 4 + (row % 8) / 2).
 * scale = amax / 127 + 1e-7, q = round-half-away(x / scale); K = half-rounded (k - k_mean) when k_mean
 * is given; sm_scale is not folded in (qattn_fwd_ex applies it, qk_quant_gran = QATTN_GRAN_THREAD).
 */
int qattn_quant_qk_per_thread_int8(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t Lq, int64_t Lk,
                                   int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean, qattn_seq q_out,
                                   qattn_seq k_out, float* q_scale, float* k_scale, qattn_stream_t stream);

/*
 * The two quantizers above with a choice of scale layout.  QATTN_SCALES_SM89 is what the plain entries
 * do.  QATTN_SCALES_SM90 gives the tables of the reference's sm90 entry, which calls
 * per_warp_int8(BLKQ=64, WARPQ=16, BLKK=128) and per_thread_int8(BLKQ=64, WARPQ=16, BLKK=128, WARPK=128)
 * (tf-kernel/tf_kernel/sageattn2.py:1608-1624, quant_per_thread.py:267-369):
 *   per-warp:   q_scale [B, Hq, ceil(Lq/64)*4]  (index row / 16),
 *               k_scale [B, Hkv, ceil(Lk/128)]   (index row / 128);
 *   per-thread: q_scale [B, Hq, ceil(Lq/64)*32] (index (row / 16) * 8 + row % 8),
 *               k_scale [B, Hkv, ceil(Lk/128)*4] (index (row / 128) * 4 + (row % 8) / 2).
 * Rounding and smoothing are those of the plain entry.  qattn_fwd_ex reads these tables with
 * qk_quant_gran QATTN_GRAN_WARP_SM90 / QATTN_GRAN_THREAD_SM90.
 */
int qattn_quant_qk_per_warp_int8_ex(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t Lq, int64_t Lk,
                                    int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean, qattn_seq q_out,
                                    qattn_seq k_out, float* q_scale, float* k_scale, int scale_layout,
                                    qattn_stream_t stream);
int qattn_quant_qk_per_thread_int8_ex(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t Lq, int64_t Lk,
                                      int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean, qattn_seq q_out,
                                      qattn_seq k_out, float* q_scale, float* k_scale, int scale_layout,
                                      qattn_stream_t stream);

/*
 * Mean over the sequence, rounded to the input dtype: mean[b, h, d] (contiguous [B, H, D]).
 * Replaces k.mean(dim=seq) in sageattn_qk_int8_pv_fp8_cuda (tf-kernel/tf_kernel/sageattn2.py:1329-1330).
 * Deterministic (fixed reduction order).  Needs workspace of qattn_seq_mean_workspace_size bytes.
 */
size_t qattn_seq_mean_workspace_size(int64_t B, int64_t L, int64_t H, int64_t D);
int qattn_seq_mean(qattn_seq in, int dtype, int64_t B, int64_t L, int64_t H, int64_t D, void* mean,
                   void* workspace, size_t workspace_bytes, qattn_stream_t stream);

/*
 * Per-channel FP8 (OCP e4m3) quantization of V.
 * Replaces per_channel_fp8 = transpose_pad_permute_cuda + scale_fuse_quant_cuda
 * (tf-kernel/tf_kernel/sageattn2.py:320-407, fused.cu:265-330,332-445,863-1010).
 *   v8:      [B, H, D, Lpad] bytes, Lpad = ceil(L / 64) * 64.  Within every 64-key tile the keys are
 *            stored in the order the attention kernel's FP8 MFMA A-operand reads them: key
 *            kappa = 32*kb + 8*g + 4*hf + t sits at position 32*hf + 16*kb + 4*g + t.
 *   v_scale: fp32 [B, H, D]; v ~= e4m3(v8) * v_scale
 */
size_t qattn_per_channel_fp8_workspace_size(int64_t B, int64_t L, int64_t H, int64_t D);
int qattn_per_channel_fp8(qattn_seq v, int dtype, int64_t B, int64_t L, int64_t H, int64_t D, float scale_max,
                          uint8_t* v8, int64_t Lpad, float* v_scale, void* workspace, size_t workspace_bytes,
                          qattn_stream_t stream);
/*
 * qattn_per_channel_fp8 with the reference's optional V smoothing (per_channel_fp8(smooth_v=True) ->
 * mean_scale_fuse_quant_cuda, MeanScaleKernel<sub_mean> fused.cu:362-445): with smooth_v != 0,
 *   v_mean = sum over the L tokens / (L rounded up to 16)        (fp32 [B, H, D], written)
 *   amax   = max(|max - v_mean|, |min - v_mean|), max / min including the zero pad tokens up to 16
 *   v8     = e4m3((v - v_mean) * scale_max / amax),  v_scale = amax / scale_max
 * and the attention adds v_mean back to its output (qattn_fwd_ex2).  smooth_v == 0: qattn_per_channel_fp8.
 */
int qattn_per_channel_fp8_ex(qattn_seq v, int dtype, int64_t B, int64_t L, int64_t H, int64_t D, float scale_max,
                             int smooth_v, uint8_t* v8, int64_t Lpad, float* v_scale, float* v_mean, void* workspace,
                             size_t workspace_bytes, qattn_stream_t stream);

/*
 * Quantized attention: INT8 Q.K^T on MFMA, fp32 online softmax (exp2 domain, FP8 offset 8.807),
 * FP8 P.V on MFMA with fp32 accumulation, v_scale fused into the epilogue.
 * Replaces torch.ops.tf_kernel.qk_int8_sv_f8_accum_f32_fuse_v_scale_attn(_inst_buf)
 * (tf-kernel/csrc/common_extension.cc:239-258, qattn/qk_int_sv_f8_cuda_sm89.cuh:66-841).
 *   q8, k8:   int8 sequence tensors; q_scale [B, Hq, ceil(Lq/128)], k_scale [B, Hkv, ceil(Lk/64)]
 *   v8/v_scale as produced by qattn_per_channel_fp8 (Lpad >= ceil(Lk/64)*64)
 *   o:        output sequence tensor [B, Lq, Hq, D] of out_dtype
 *   qk_mult:  extra logit multiplier (1.0 when sm_scale*log2e was folded into Q by the quantizer)
 *   causal:   mask kv_idx > q_idx + q_offset (reference is_causal is top-left aligned, q_offset 0)
 *   kv_valid: NULL or device int32 [B]: keys >= kv_valid[b] are masked (key padding)
 *   lse:      NULL or fp32 [B, Hq, Lq] receiving log2(sum 2^s) of the quantized logits
 *   num_splits: 0 = automatic, 1 = no KV split, n > 1 = split keys over n workgroups
 *   workspace: needed when splitting, qattn_fwd_workspace_size bytes
 * D is 128, or 64 for FP8 V (dense launches: qattn_fwd / qattn_fwd_ex / _ex2 / _noalloc with v_kind FP8).
 * Callers pad other heads as sageattn2.py:1307-1316 does: D < 64 to 64, 64 < D < 128 to 128.  Head
 * dimension 64 runs the ping-pong kernel (unsplit or KV-split) with half the MFMA work and bytes per key
 * tile; the kernel queries below (qattn_fwd_ex_kernel, the split counts) describe D = 128.
 */
size_t qattn_fwd_workspace_size(int64_t B, int64_t Lq, int64_t Hq, int64_t D, int num_splits);
int qattn_fwd_num_splits(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq);
int qattn_fwd(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale, const uint8_t* v8,
              int64_t Lpad, const float* v_scale, qattn_seq o, int out_dtype, int64_t B, int64_t Lq, int64_t Lk,
              int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int causal, int64_t q_offset,
              const int32_t* kv_valid, float* lse, int num_splits, void* workspace, size_t workspace_bytes,
              qattn_stream_t stream);

/*
 * V (bf16/fp16) copied into the same transposed, tile-permuted layout as qattn_per_channel_fp8 uses,
 * in its own dtype: v16 [B, H, D, Lpad].  Replaces the V preparation of the reference's fp16-P.V
 * paths (sageattn_qk_int8_pv_fp16_cuda / _triton, tf-kernel/tf_kernel/sageattn2.py:551-769,930-1194).
 */
int qattn_v_tile_half(qattn_seq v, int dtype, int64_t B, int64_t L, int64_t H, int64_t D, uint16_t* v16,
                      int64_t Lpad, qattn_stream_t stream);

/*
 * The prologue of the INT8-QK / FP8-PV path in four launches: one pass over K and V for their column
 * statistics (K sum when smooth_k; V max |v|, or sum / max / min when smooth_v), one finalize (k_mean
 * [B, Hkv, D] in the input dtype, v_scale, v_mean), V to FP8 tiles (as qattn_per_channel_fp8_ex), and K then
 * Q to INT8 in one launch (qk_quant_gran 1: per block, Q times q_sm_scale = sm_scale * log2(e), CUDA
 * rounding; 2: per warp; 3: per thread, as qattn_quant_qk_per_warp_int8 / _per_thread_int8; 4 / 5: per warp /
 * per thread with the sm90 tables, as the *_ex quantizers with QATTN_SCALES_SM90).  Outputs are
 * bit-identical to qattn_seq_mean + the quantizer + qattn_per_channel_fp8_ex.  Replaces the quantization
 * block of sageattn_qk_int8_pv_fp8_cuda (tf-kernel/tf_kernel/sageattn2.py:1334-1383), which the reference
 * runs as separate kernels.  workspace: qattn_sage_quant_workspace_size bytes.
 */
size_t qattn_sage_quant_workspace_size(int64_t B, int64_t Lk, int64_t Hkv, int64_t D);
int qattn_sage_quant(qattn_seq q, qattn_seq k, qattn_seq v, int dtype, int64_t B, int64_t Lq, int64_t Lk, int64_t Hq,
                     int64_t Hkv, int64_t D, int qk_quant_gran, float q_sm_scale, int smooth_k, float scale_max,
                     int smooth_v, qattn_seq q_out, float* q_scale, qattn_seq k_out, float* k_scale, void* k_mean,
                     uint8_t* v8, int64_t Lpad, float* v_scale, float* v_mean, void* workspace,
                     size_t workspace_bytes, qattn_stream_t stream);

/*
 * Packed variable-length batches: sequence b spans rows cu_seqlens[b] .. cu_seqlens[b + 1] of a packed
 * [total, H, D] tensor (int32 device tables of B + 1 entries, read only on the device).  Every kernel
 * clamps a sequence to rows [0, total) of its tensor and to max_seqlen rows, so a malformed table cannot
 * make it address memory outside the packed tensors (the reference leaves such tables undefined).
 *
 * qattn_varlen_offsets: seq_q / seq_k = the sequence tables made non-decreasing and clamped to [0, total]
 * (so that sequences are disjoint row ranges of the packed tensors whatever the input), and the block
 * offsets cu_qs[b] = sum over earlier sequences of ceil(len_q / 128), cu_ks[b] = cu_vt[b] = the same of
 * ceil(len_k / 64), with len = min(rows, max_seqlen) (all B + 1 entries); replaces the cumsum of
 * quant_per_block_varlen.py:92-107 (tf-kernel/tf_kernel/).  The three kernels below take seq_q / seq_k
 * as their cu_seqlens_q / cu_seqlens_k.
 *
 * qattn_quant_qk_varlen_int8: per-sequence INT8 blocks of 128 Q rows and 64 K rows, with the Triton rounding
 * of variant; q_scale [cu_qs[B], Hq] and k_scale [cu_ks[B], Hkv] (block-major, the reference's layout);
 * k_mean [1, Hkv, D] (shared by every sequence) or NULL; q scaled by sm_scale.  max_lq / max_lk bound every
 * sequence's length.  Replaces per_block_int8_varlen (quant_per_block_varlen.py:72-127).
 *
 * qattn_v_tile_half_varlen: V into the tile layout of qattn_v_tile_half as one entry [1, H, D, Lpad], sequence
 * b's tiles at tile columns cu_vt[b] ..; Lpad >= 64 * (cu_vt[B]) (an upper bound such as
 * 64 * (ceil(total_k / 64) + B) is fine).
 *
 * qattn_fwd_varlen: INT8 Q.K^T and fp16 P.V per sequence in one launch, causal top-left aligned per sequence;
 * q8/k8/o are the packed [1, total, H, D] views (their batch stride is ignored), v16 from
 * qattn_v_tile_half_varlen.  Rows of sequences with no keys are left untouched.  Replaces
 * attn_qk_int8_block_varlen.forward (attn_qk_int8_block_varlen.py:157-200).
 */
int qattn_varlen_offsets(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t B, int64_t total_q,
                         int64_t total_k, int64_t max_lq, int64_t max_lk, int32_t* seq_q, int32_t* seq_k,
                         int32_t* cu_qs, int32_t* cu_ks, int32_t* cu_vt, qattn_stream_t stream);
int qattn_quant_qk_varlen_int8(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t total_q, int64_t total_k,
                               int64_t max_lq, int64_t max_lk, int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean,
                               const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, const int32_t* cu_qs,
                               const int32_t* cu_ks, qattn_seq q_out, qattn_seq k_out, float* q_scale, float* k_scale,
                               float sm_scale, int variant, qattn_stream_t stream);
int qattn_v_tile_half_varlen(qattn_seq v, int dtype, int64_t B, int64_t total_k, int64_t max_lk, int64_t H, int64_t D,
                             const int32_t* cu_seqlens_k, const int32_t* cu_vt, uint16_t* v16, int64_t Lpad,
                             qattn_stream_t stream);
int qattn_fwd_varlen(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale, const uint16_t* v16,
                     int64_t Lpad, qattn_seq o, int out_dtype, int64_t B, int64_t total_q, int64_t total_k,
                     int64_t max_lq, int64_t max_lk, int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int causal,
                     const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, const int32_t* cu_qs,
                     const int32_t* cu_ks, const int32_t* cu_vt, qattn_stream_t stream);

/*
 * Quantized attention with INT8 Q.K^T and P.V in the half dtype of V (P rounded to that dtype,
 * fp32 accumulation, no FP8 offset or v_scale): the math of the reference's INT8-QK / FP16-PV kernels
 * (qk_int8_sv_f16_accum_f32_attn, common_extension.cc:214-218; Triton attn_qk_int8_per_block.py:46-101).
 * Arguments as qattn_fwd, with v16 from qattn_v_tile_half and v_dtype its dtype.
 */
int qattn_fwd_pv16(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale, const uint16_t* v16,
                   int v_dtype, int64_t Lpad, qattn_seq o, int out_dtype, int64_t B, int64_t Lq, int64_t Lk,
                   int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int causal, int64_t q_offset,
                   const int32_t* kv_valid, float* lse, int num_splits, void* workspace, size_t workspace_bytes,
                   qattn_stream_t stream);

/*
 * Streaming KV cache, V side: FP8 V with a running ("sticky") per-channel amax.
 * The cache keeps V in its own dtype (v: sequence tensor over cache slots [0, fill)) next to an FP8
 * copy v8 [B, H, D, Lpad] in the tile layout of qattn_per_channel_fp8.  After the caller has written
 * new rows into the slot ranges [begin0, end0) and [begin1, end1) (either may be empty), this call
 *   amax[b, h, d] = max(amax, max |v| over the new rows);   v_scale = amax / scale_max
 * and re-encodes, with scale_max / amax, the FP8 tiles that overlap the new rows - or every tile of a
 * (b, h) whose amax grew.  amax (fp32 [B, H, D], zero-initialised by the caller) persists across
 * calls.  No host synchronisation.  Replaces the per-step per_channel_fp8 of the whole attention
 * window that the reference's streaming self-attention performs through attention()
 * (telefuser/models/lingbot_world_fast_dit.py:150-183; sageattn2.py:320-407).
 */
size_t qattn_v_fp8_cache_workspace_size(int64_t B, int64_t n0, int64_t n1, int64_t H, int64_t D);
int qattn_v_fp8_cache_update(qattn_seq v, int dtype, int64_t B, int64_t fill, int64_t H, int64_t D, int64_t begin0,
                             int64_t end0, int64_t begin1, int64_t end1, float scale_max, float* amax, uint8_t* v8,
                             int64_t Lpad, float* v_scale, void* workspace, size_t workspace_bytes,
                             qattn_stream_t stream);

/*
 * Attention on half-precision Q (bf16 / fp16, the output's dtype), quantized inside the attention kernel as
 * the reference's per_thread_int8 (qk_quant_gran QATTN_GRAN_THREAD, Triton rounding,
 * quant_per_thread.py:22-158), per_warp_int8 (QATTN_GRAN_WARP, QuantInt8Kernel rounding, fused.cu:698-780) or
 * per_block_int8 (QATTN_GRAN_BLOCK, QuantInt8Kernel rounding with sm_scale folded in, fused.cu:59-194) would
 * -- bit-identical codes and scales -- by the resident-K/V or the ping-pong kernel (per block, the four
 * waves that hold a 128-row query block exchange their maxima through LDS), so int8 Q is never written out
 * and read back.  K and V are prepared as for qattn_fwd_ex with the
 * same granularity (k_scale per 64-key block, or 4 lane-pair classes per block for per-thread).  Arguments
 * as qattn_fwd_ex (causal, q_offset, kv_valid, lse, num_splits with its workspace sized by
 * qattn_fwd_ex_num_splits / qattn_fwd_workspace_size); qk_mult = sm_scale * 1.44269504 (per block it is the
 * factor multiplied into Q before quantization, and the logits take 1).  Runs when the
 * automatic kernel rule gives one of those two kernels for the launch and head_dim is 128, or for
 * any launch with head_dim 64 (the ping-pong kernel's D = 64 form) (qattn_fwd_q16_supported), else returns
 * QATTN_ERR_SHAPE.  Replaces the quantize-then-attend sequence of
 * sageattn_qk_int8_pv_fp8_cuda (sageattn2.py:1334-1446); no counterpart op in the reference.
 */
int qattn_fwd_q16_supported(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int64_t D, int qk_quant_gran, int causal);
int qattn_fwd_q16(qattn_seq q, qattn_seq k8, const float* k_scale, const uint8_t* v8, int64_t Lpad,
                  const float* v_scale, const float* v_mean, qattn_seq o, int dtype, int64_t B, int64_t Lq, int64_t Lk,
                  int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int qk_quant_gran, int causal, int64_t q_offset,
                  const int32_t* kv_valid, float* lse, int num_splits, void* workspace, size_t workspace_bytes,
                  qattn_stream_t stream);

/*
 * General form of qattn_fwd / qattn_fwd_pv16 with the Q/K scale granularity of the reference's kernels
 * (the qk_quant_gran argument of qk_int8_sv_f8_accum_f32_fuse_v_scale_attn(_inst_buf) and
 * qk_int8_sv_f16_accum_f32_attn, common_extension.cc:214-258; sm89 kernel :136,318-323):
 *   QATTN_GRAN_BLOCK:  q_scale [B, Hq, ceil(Lq/128)],     k_scale [B, Hkv, ceil(Lk/64)]
 *   QATTN_GRAN_WARP:   q_scale [B, Hq, ceil(Lq/128)*4],   k_scale [B, Hkv, ceil(Lk/64)]
 *   QATTN_GRAN_THREAD: q_scale [B, Hq, ceil(Lq/128)*32],  k_scale [B, Hkv, ceil(Lk/64)*4]
 * (layouts of qattn_quant_qk_per_warp_int8 / qattn_quant_qk_per_thread_int8), and the sm90 tables of
 * qk_int8_sv_f8_accum_f32_fuse_v_scale_attn_inst_buf (sageattn2.py:1608-1624,1676-1689):
 *   QATTN_GRAN_WARP_SM90:   q_scale [B, Hq, ceil(Lq/64)*4],   k_scale [B, Hkv, ceil(Lk/128)]
 *   QATTN_GRAN_THREAD_SM90: q_scale [B, Hq, ceil(Lq/64)*32],  k_scale [B, Hkv, ceil(Lk/128)*4]
 * (qattn_quant_qk_per_warp_int8_ex / _per_thread_int8_ex with QATTN_SCALES_SM90; FP8 or half V, dense
 * sequences only).  For per-warp and
 * per-thread scales sm_scale is not in Q: pass qk_mult = sm_scale * 1.44269504.
 *   v_kind QATTN_V_FP8: v = e4m3 tile layout + v_scale;  QATTN_V_BF16 / _FP16: v from qattn_v_tile_half.
 * The number of KV splits depends on v_kind and the granularity: size the workspace with
 * qattn_fwd_ex_num_splits (or pass an explicit num_splits >= it).
 */
int qattn_fwd_ex_num_splits(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int v_kind, int qk_quant_gran);
/*
 * Query blocks (128 rows) one workgroup of qattn_fwd_ex streams through a single K/V pipeline for an
 * automatic-split call with these sizes (1 = one block per workgroup).  Short, non-causal FP8 P.V key
 * ranges (fewer than 24 key tiles) over grids larger than the resident 512 workgroups use several, so the
 * per-workgroup start-up and the epilogue overlap the next block's work; the result does not depend on
 * it.  No counterpart in the reference (its launch is one CTA per query block).
 */
int qattn_fwd_ex_blocks_per_workgroup(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int v_kind, int qk_quant_gran,
                                      int causal);
/*
 * Which kernel a qattn_fwd_ex launch runs (no counterpart in the reference, whose launch is one CTA
 * kernel per query block; for benchmarks and tests):
 *   QATTN_KERNEL_ONE_BLOCK:   one query block (128 rows, 4 waves) per workgroup; half-P.V and
 *                             block-sparse launches always run it, KV-split launches unless they fit
 *                             one round of 128-256 ping-pong workgroups
 *   QATTN_KERNEL_MULTI_BLOCK: several query blocks of a head per workgroup through one K/V pipeline
 *                             (short, non-causal FP8 key ranges; see qattn_fwd_ex_blocks_per_workgroup)
 *   QATTN_KERNEL_PINGPONG:    two query blocks per workgroup (8 waves) whose wave groups alternate
 *                             matrix and vector stages; dense unsplit FP8 launches whose rounds of 256 CUs cost no more
 *                             than the one-block grid's, and KV-split FP8 launches of 128-256 workgroups
 *   QATTN_KERNEL_RESIDENT:    the whole key range (at most 8 tiles of 64 keys) held in LDS, 12 waves per
 *                             workgroup each walking its own 32-row query blocks without barriers;
 *                             non-causal FP8 launches with Lk <= 512
 * All four give identical results for a launch they can run.  qattn_fwd_ex_kernel returns the kernel the
 * automatic rule picks for these sizes; qattn_set_kernel(k) forces k for the calling thread's later
 * FP8, dense, unsplit launches (QATTN_KERNEL_AUTO restores the rule; MULTI_BLOCK and RESIDENT only where
 * they apply)
 * and returns the previous setting; qattn_last_kernel() is the kernel of the calling thread's last launch.
 */
enum qattn_kernel {
  QATTN_KERNEL_AUTO = 0,
  QATTN_KERNEL_ONE_BLOCK = 1,
  QATTN_KERNEL_MULTI_BLOCK = 2,
  QATTN_KERNEL_PINGPONG = 3,
  QATTN_KERNEL_RESIDENT = 4
};
int qattn_fwd_ex_kernel(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int v_kind, int qk_quant_gran, int causal,
                        int num_splits);
int qattn_set_kernel(int kernel);
int qattn_last_kernel(void);
int qattn_fwd_ex(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale, const void* v, int v_kind,
                 int64_t Lpad, const float* v_scale, qattn_seq o, int out_dtype, int64_t B, int64_t Lq, int64_t Lk,
                 int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int qk_quant_gran, int causal, int64_t q_offset,
                 const int32_t* kv_valid, float* lse, int num_splits, void* workspace, size_t workspace_bytes,
                 qattn_stream_t stream);
/*
 * qattn_fwd_ex plus the V-mean epilogue of the reference's fuse_v_mean kernel
 * (qk_int8_sv_f8_accum_f32_fuse_v_scale_fuse_v_mean_attn, common_extension.cc; sm89 kernel :742-761):
 * out = O / l * v_scale + v_mean, with v_mean fp32 [B, Hkv, D] from qattn_per_channel_fp8_ex (FP8 V
 * only; NULL = qattn_fwd_ex).
 */
int qattn_fwd_ex2(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale, const void* v, int v_kind,
                  int64_t Lpad, const float* v_scale, const float* v_mean, qattn_seq o, int out_dtype, int64_t B,
                  int64_t Lq, int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int qk_quant_gran,
                  int causal, int64_t q_offset, const int32_t* kv_valid, float* lse, int num_splits, void* workspace,
                  size_t workspace_bytes, qattn_stream_t stream);

/*
 * qattn_fwd_ex without a workspace argument, for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops).  No counterpart in the reference.  KV-split partials go to a
 * device array inside the library (one per GPU, held until the process ends) of at most
 * qattn_fwd_noalloc_max_scratch() bytes (128 MiB): a launch whose qattn_fwd_workspace_size(B, Lq, Hq, D,
 * splits) exceeds it fails with QATTN_ERR_WORKSPACE.  Calls never allocate device memory.  Launches that use
 * the array (KV-split launches) are ordered on the GPU in the order the host issues them, also from different
 * streams or threads: each waits (hipStreamWaitEvent, no host wait) for the previous one's completion event.
 * On a stream under graph capture that ordering is left to the graph: replays of a captured graph must not
 * overlap other users of the array on the same GPU.  The array exists on every GPU where the library's code
 * object is loaded, whether or not this entry is called.  Results equal qattn_fwd_ex's.
 */
size_t qattn_fwd_noalloc_max_scratch(void);
int qattn_fwd_ex_noalloc(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale, const void* v,
                         int v_kind, int64_t Lpad, const float* v_scale, qattn_seq o, int out_dtype, int64_t B,
                         int64_t Lq, int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int qk_quant_gran,
                         int causal, int64_t q_offset, const int32_t* kv_valid, float* lse, int num_splits,
                         qattn_stream_t stream);

/*
 * Block-sparse quantized attention: like qattn_fwd_pv16, but a query block (128 rows) only visits the
 * key tiles (64 keys) whose mask byte is non-zero - the k_block_id skip of the reference's
 * sparse_int8_attn forward (telefuser/kernel/triton/sparse_int8_attn.py:22-280, called from
 * sparse_sageattn, telefuser/ops/attention/sparse_sage.py:25-80).
 *   tile_mask: int8, element (b, kv head hk, query block i, key tile j) at
 *              tile_mask[(b * Hkv + hk) * mask_sbh + i * mask_sq + j]  (key tiles contiguous)
 * A query row whose blocks are all masked gets a zero output.  The KV split count must come from
 * qattn_fwd_block_sparse_num_splits (a workgroup holds the ids of at most 1024 active tiles).
 */
int qattn_fwd_block_sparse_num_splits(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq);
int qattn_fwd_block_sparse(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale, const uint16_t* v16,
                           int v_dtype, int64_t Lpad, qattn_seq o, int out_dtype, int64_t B, int64_t Lq, int64_t Lk,
                           int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int causal, const int8_t* tile_mask,
                           int64_t mask_sbh, int64_t mask_sq, float* lse, int num_splits, void* workspace,
                           size_t workspace_bytes, qattn_stream_t stream);

/*
 * Fused prologue of the Wan self-attention projections (the step before the path:
 * telefuser/models/wan_video_dit.py:196-207 norm_q/norm_k -> rope_apply -> attention):
 *   x: linear output [B, L, H*D] viewed as a sequence tensor [B, L, H, D] (row of H*D contiguous values)
 *   rstd: qattn_row_rstd of x (RMSNorm over the whole H*D row; fp64-exact sum of squares, fp32 after)
 *   y = half((x * rstd) * w), then interleaved RoPE on y with cos/sin [L, D/2] fp32 (rows cs_stride
 *   floats): (y1, y2) -> half(fma(-y2, sin, y1*cos)), half(fma(y1, sin, y2*cos))
 *   (telefuser/kernel/triton/norm.py:469-507 and rotary.py:21-88), then per-block INT8 quantization as
 *   qattn_quant_qk_per_block_int8 (Q blocks of 128 with sm_scale folded, K blocks of 64 with k_mean).
 * The normalized / rotated bf16 tensors are never written.  qattn_norm_rope_seq_mean gives the K mean
 * of the rotated values (smoothing vector) in one pass over x.
 */
int qattn_row_rstd(const void* x, int dtype, int64_t rows, int64_t row_stride, int64_t n, float eps, float* rstd,
                   qattn_stream_t stream);
int qattn_norm_rope_seq_mean(qattn_seq x, int dtype, int64_t B, int64_t L, int64_t H, int64_t D, const float* rstd,
                             const void* w, const float* cs, const float* sn, int64_t cs_stride, void* mean,
                             void* workspace, size_t workspace_bytes, qattn_stream_t stream);
int qattn_norm_rope_quant_qk(qattn_seq xq, qattn_seq xk, int dtype, int64_t B, int64_t L, int64_t H, int64_t D,
                             const float* rstd_q, const float* rstd_k, const void* wq, const void* wk, const float* cs,
                             const float* sn, int64_t cs_stride, const void* k_mean, qattn_seq q_out,
                             qattn_seq k_out, float* q_scale, float* k_scale, float sm_scale, int variant,
                             qattn_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QATTN_H_ */
