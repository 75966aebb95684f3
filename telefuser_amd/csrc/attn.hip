// Quantized attention forward for gfx950: INT8 Q.K^T and FP8 P.V on MFMA, fp32 online softmax.
//
// Math (the reference's sm89 kernel, tf-kernel/csrc/sageattn2/qattn/qk_int_sv_f8_cuda_sm89.cuh:342-840,
// attn_utils.cuh:362-452 update_mdo, :469-481 RS_32_to_8, :711-756 normalize_d):
//   s    = int32(Q8 . K8^T) * (q_scale * k_scale * qk_mult)          (log2 domain)
//   m'   = max(m, rowmax(s) - 8.807);   p = exp2(s - m')  in (0, 448]
//          (here with a lazy update rule: m' = rowmax(s) - 5.807 only if that exceeds m by > 3, which
//          keeps p <= 448 and skips the O rescale on almost every tile; oracle/ restates the rule)
//   l    = l * exp2(m - m') + sum(p)
//   O    = O * exp2(m - m') + e4m3(p) . e4m3(V)                        (fp32 accumulation)
//   out  = O / l * v_scale[d]
//   (the FP8 P.V kernels form e4m3(p) straight from s - m' without an exponential, p_e4m3_x4 below,
//   and sum that rounded P; the half P.V kernels use exp2)
//
// MI355X design (not a translation of the NVIDIA tiling):
//   * qattn_fwd_kernel: workgroup = 4 wave64s = 128 query rows (one Q quantization block, so one q_scale);
//     each wave owns 32 rows.  Key tiles of 64 keys (one K quantization block, one k_scale).
//   * S^T = K . Q^T with v_mfma_i32_32x32x32_i8 (A = K from LDS, B = Q held in VGPRs for the whole
//     loop).  In the 32x32 result each lane owns one query column and 16 key rows, so the row max
//     is an in-lane max plus one lane^32 exchange, and the running sum stays per lane until the end.
//   * O^T = V^T . P^T with v_mfma_f32_32x32x64_f8f6f4 (A = V^T from LDS, B = P^T straight from the
//     softmax registers).  The FP8 V quantizer stores every 64-key tile in exactly the key order the
//     B operand inherits from the S^T layout, so P never goes through LDS.
//   * K/V tiles are multi-buffered in LDS, fragment-major (each 1 KiB block holds one MFMA operand
//     fragment of all 64 lanes), and fetched by LDS DMA (buffer_load_dwordx4 ... lds) issued before the
//     current tile's MFMA/softmax work, so staging costs neither VGPRs nor VALU slots and a lane reads
//     its fragments from one base address plus constant offsets.
//   * Large dense launches run the ping-pong kernel (two 4-wave groups per workgroup, 256 rows, whose
//     waves alternate matrix and vector stages on each SIMD); the per-element arithmetic is the same.
//   * blockIdx -> tile mapping is XCD-aware: the hardware deals workgroups round-robin over the 8
//     XCDs, so consecutive tiles of one (batch, head) are gathered onto one XCD and share its L2.
//   * Optional KV split (flash-decoding style) for grids that cannot fill 256 CUs; a combine kernel
//     merges the partial (O, m, l) triples.
#include <algorithm>
#include <mutex>
#include <type_traits>

#include "common.h"

namespace qattn {

constexpr int kD = 128;
constexpr int kBQ = 128;  // query quantization block
constexpr int kWavesPerSimd = 2;  // occupancy target: 2 workgroups of 4 waves per CU
constexpr int kPrefetch = 2;      // K/V tiles in flight ahead of the one being computed
constexpr int kNBuf = kPrefetch + 1;
// k_scales staged in LDS per workgroup (floats).  Sized so that two workgroups per CU still fit in the
// 160 KiB of LDS next to the K/V buffers: 24 + 24 + 30 KiB (FP8 V) or 24 + 48 + 6 KiB (half V).
template <int PV> constexpr int ks_lds_floats() { return PV == 0 ? 7680 : 1536; }
// block-sparse launches (half P.V only) stage the active tiles' ids next to their scales
constexpr int kSpMaxTiles = 1024;
// multi-block launches (one workgroup streams up to kMqMaxBlocks query blocks of one head through one
// K/V pipeline): short key ranges only, so their k_scales and q_scales are staged whole in LDS
constexpr int kMqMaxTiles = 64;
// the automatic rule picks multi-block launches below this many key tiles: from 32 tiles on the ping-pong
// kernel is 4-12 % faster (32760 x 2048 x 12, 8192 x 4096 x 16), at 12 and 16 tiles the two tie
constexpr int kMqAutoMaxTiles = 24;
constexpr int kMqMaxBlocks = 64;
// per-thread K scales: 4 per 64-key tile (one per mma lane-pair class), otherwise 1
constexpr int ks_per_tile(bool kt) { return kt ? 4 : 1; }
constexpr int kBK = 64;
constexpr int kThreads = 256;
constexpr float kFp8Offset = 8.807f;  // attn_utils.cuh:35 S_FP8_OFFSET
constexpr float kMInit = -3.0e38f;
// Lazy-rescale threshold (log2 units), see the softmax below.  After a move of the running max the largest p of
// the row is 448 / 2^kLazyTau.  Measured against 1 (C4, text cross attention over 512 keys: a few tiles per
// row, so the max moves on most of them at 1): 8 % faster at 3, RMS error against float64 truth 3.84 % ->
// 3.90 % (cosine 0.99926 -> 0.99924); C2 / C5 within 1 %, error unchanged.
constexpr float kLazyTau = 3.0f;
// The QK accumulators start at kAccBiasBits instead of 0: the int32 result bias + s, read as fp32,
// is exactly kAccBias + s for |s| < 2^22 (here |s| <= 2^21), so the logits reach the softmax as floats
// without an int -> float conversion per element; the bias is folded into the exp2 offset.
constexpr int kAccBiasBits = 0x4B400000;
constexpr float kAccBias = 12582912.0f;
// a masked logit as -inf: as int32 (-2^23) it lies below every biased logit, as fp32 its exp2 is 0
constexpr int kMaskedLogitBits = (int)0xFF800000u;

struct AttnParams {
  const int8_t* q8;
  int64_t qsb, qsl, qsh;
  const int8_t* k8;
  int64_t ksb, ksl, ksh;
  const void* v;  // tile-layout V: e4m3 (PV_FP8) or the half dtype, [B, Hkv, D, Lpad]
  int64_t Lpad;
  const float* q_scale;  // [B, Hq, nQS]: per 128-row block, per 32-row warp block, or per thread class
  const float* k_scale;  // [B, Hkv, nKS]: per 64-key tile, or 4 lane-pair classes per tile
  const float* v_scale;  // [B, Hkv, D] (FP8 P.V only)
  const float* v_mean;   // [B, Hkv, D] or null: added to the output (smoothed V, FP8 P.V only)
  void* o;
  int64_t osb, osl, osh;
  float* lse;  // [B, Hq, Lq] or null
  const int32_t* kv_valid;
  const int8_t* tile_mask;  // block-sparse: [B, Hkv, nQB, nKB] (strides tm_s1 per (b, kv head), tm_s2 per Q block)
  int64_t tm_s1, tm_s2;
  float* ws_o;   // split partials [split][B][Hq][Lq][D]
  float* ws_ml;  // [split][B][Hq][Lq][2]
  int64_t B, Lq, Lk, Hq, Hkv, nQB, nKB;
  int64_t nQS, nKS;  // scale entries per (b, h)
  int qgran;         // QATTN_GRAN_BLOCK / _WARP / _THREAD (q_scale indexing)
  float q_sm_scale;  // Q quantized per block inside the kernel: the factor multiplied into Q first
  int qrs;           // log2 of the rows of a warp cell of q_scale: 5 (sm89 tables) or 4 (sm90 tables)
  int kts;           // key tiles (64 keys) per k_scale block, as a shift: 0 (64-key blocks) or 1 (128)
  int64_t q_offset;
  int group;
  int nsplit;
  int tiles_per_split;
  int qpw;       // multi-block launches: query blocks per workgroup
  int64_t nQC;   // multi-block launches: workgroups per (batch, head)
  int causal;
  float qk_mult;
  // packed variable-length batches (null otherwise): sequence b has query rows cu_q[b] .. cu_q[b + 1] and key
  // rows cu_k[b] .. cu_k[b + 1] of the packed [1, total, H, D] tensors, its scales start at block cu_qs[b] /
  // cu_ks[b] of [total_blocks, H] tables, and its V tiles at tile cu_vt[b] of the [1, Hkv, D, Lpad] tile layout
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* cu_qs;
  const int32_t* cu_ks;
  const int32_t* cu_vt;
  int64_t var_tq, var_tk;  // rows of the packed Q / K tensors
  // resident-K/V launches: each workgroup takes wb_per_wg consecutive 32-row wave blocks of one head,
  // n_chunk workgroups per (batch, head)
  int64_t wb_per_wg;
  int64_t n_chunk;
};

__device__ __forceinline__ int64_t xcd_remap(int64_t bid, int64_t n) {
  const int64_t q = n / 8, r = n % 8;
  const int64_t xcd = bid % 8, idx = bid / 8;
  return xcd * q + (xcd < r ? xcd : r) + idx;
}

// Buffer resource (V#) for raw, unswizzled byte addressing of [base, base + bytes): loads whose offset
// is at or past `bytes` return zeros instead of touching memory.
// q_scale entry of query row `row` (< nQB * 128): one per 128-row block, per warp cell of 2^qrs rows, or
// per row class (rows of a warp cell with equal row % 8: the reference's per-thread grouping).  Clamped
// to the table: the sm90 tables cover ceil(Lq / 64) * 64 rows, and the rows past that are masked.
__device__ __forceinline__ int64_t q_scale_index(const AttnParams& p, int64_t row) {
  const int64_t i = p.qgran == QATTN_GRAN_THREAD ? ((row >> p.qrs) << 3) + (row & 7)
                    : p.qgran == QATTN_GRAN_WARP ? row >> p.qrs
                                                 : row >> 7;
  return i < p.nQS ? i : p.nQS - 1;
}

// k_scale entry c (< ks) of key tile t in a table of ks entries per k_scale block
__device__ __forceinline__ int64_t k_scale_index(const AttnParams& p, int64_t t, int c, int ks) {
  return (t >> p.kts) * ks + c;
}

__device__ __forceinline__ v4u make_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = reinterpret_cast<uint64_t>(base);
  v4u r;
  r[0] = __builtin_amdgcn_readfirstlane((uint32_t)a);
  r[1] = __builtin_amdgcn_readfirstlane((uint32_t)(a >> 32) & 0xffffu);
  r[2] = __builtin_amdgcn_readfirstlane(bytes);
  r[3] = 0x00020000u;  // raw buffer, 32-bit data format
  return r;
}

// One 16-byte-per-lane buffer -> LDS DMA (buffer_load_dwordx4 ... lds): lane j's 16 bytes, read at
// base + soff + voff_j, land at LDS address lds + 16 j.  The per-lane offsets are loop-invariant
// VGPRs and the tile advance is a scalar offset, so issuing a tile costs no VALU work.  Issued through
// inline asm so the compiler does not treat every later LDS read as a possible alias of the in-flight
// DMA (it would otherwise put an s_waitcnt vmcnt(0) in front of them and serialise the prefetch);
// completion is tracked with explicit vmcnt waits instead.
__device__ __forceinline__ void lds_dma16(uint32_t voff, v4u rsrc, uint32_t soff, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dwordx4 %0, %1, %2 offen lds"
      :
      : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds)
      : "memory", "m0");
}

// The 4-byte form (buffer_load_dword ... lds): lane j's dword lands at lds + 4 j.
__device__ __forceinline__ void lds_dma4(uint32_t voff, v4u rsrc, uint32_t soff, uint32_t lds) {
  asm volatile(
      "s_mov_b32 m0, %3\n\t"
      "s_nop 0\n\t"
      "buffer_load_dword %0, %1, %2 offen lds"
      :
      : "v"(voff), "s"(rsrc), "s"(soff), "s"(lds)
      : "memory", "m0");
}

// two floats -> two round-to-nearest-even halves (bf16: v_cvt_pk_bf16_f32), low word first
template <bool IS_FP16>
__device__ __forceinline__ uint32_t pack_half2(float a, float b) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  uint32_t r;
  if constexpr (IS_FP16) {
    const h2 v = __builtin_convertvector(f2{a, b}, h2);
    __builtin_memcpy(&r, &v, 4);
  } else {
    const b2 v = __builtin_convertvector(f2{a, b}, b2);
    __builtin_memcpy(&r, &v, 4);
  }
  return r;
}

// One output value: O / l * v_scale (+ v_mean for smoothed V), rounded after every operation (no fused
// multiply-add), so that every kernel and the split combine produce the same bits.
template <bool ADD_MEAN>
__device__ __forceinline__ float epilogue_value(float o, float inv_l, float sc, float vm) {
#pragma clang fp contract(off)
  const float x = o * inv_l * sc;
  if constexpr (ADD_MEAN) return x + vm;
  else return x;
}

// P of the FP8 P.V without an exponential.  u = 8 (x - kPLinShift) + 56, rounded to an integer k (RNE) and
// clamped to [0, 255] by v_cvt_pk_u8_f32, is read as the e4m3 byte of P: exponent field floor(y) + 7 and
// mantissa round(8 frac(y)) for y = x - kPLinShift, i.e. 2^floor(y) (1 + frac(y)) rounded to the e4m3 grid.
// This is Schraudolph's exponential ("A fast, compact approximation of the exponential function", Neural
// Computation 11, 1999: the argument scaled into the exponent field, the mantissa interpolating 2^f
// linearly) at e4m3 precision.  (1 + f) / 2^f lies in [1, 1.0861] with mean 1.040685 over f in [0, 1); the
// shift kPLinShift = log2(1.040685) removes that mean, so P is unbiased against exp2(x) on average and within
// -4.0 % / +4.4 % of it before the e4m3 rounding (RMS 3.15 % relative including the rounding, against
// 2.66 % for exp2(x) rounded to e4m3).  x <= 8.807 (the FP8 offset) gives k <= 126 (448); k = 127 would
// be NaN.  x < -7 gives 0; k < 8 are the e4m3 subnormals (P < 2^-6, linear in k).  Costs one full-rate
// conversion per element against a quarter-rate v_exp_f32 plus half a quarter-rate fp8 pack (measured:
// 10.3 against 23.9 cycles per element with the fma, two waves per SIMD).
constexpr float kPLinShift = 0.057539f;
constexpr float kPLinBias = 56.0f - 8.0f * kPLinShift;  // e4m3 exponent bias 7, in units of 1/8
__device__ __forceinline__ int p_e4m3_x4(float u0, float u1, float u2, float u3) {
  uint32_t t = __builtin_amdgcn_cvt_pk_u8_f32(u0, 0, 0u);
  t = __builtin_amdgcn_cvt_pk_u8_f32(u1, 1, t);
  t = __builtin_amdgcn_cvt_pk_u8_f32(u2, 2, t);
  return (int)__builtin_amdgcn_cvt_pk_u8_f32(u3, 3, t);
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(__attribute__((address_space(3))) const void*)p);
}

// Row sums of P on the matrix pipe (FP8 P.V): one v_mfma_scale_f32_16x16x128_f8f6f4 per tile, D += A . B with
// B the e4m3 P^T operand of the P.V MFMA read in the 16 x 16 x 128 layout (lane l feeds column l % 16; its 32
// bytes are, in the 32 x 32 layout, 32 keys of query l % 32, so columns collect query c from lanes c and
// c + 32 and query c + 16 from lanes c + 16 and c + 48) and A an fp4 (e2m1) selector.  In this layout fp4
// nibbles 0-15 of A lane 16 a + r meet bytes 0-15 (a = 0, 1: of B lane groups 0, 2) or 16-31 (a = 2, 3) of
// lane groups 0 / 2, and nibbles 16-31 the same bytes of lane groups 1 / 3 (measured on gfx950).  So row 0 of
// A is 1.0 on nibbles 0-15 of lanes 0, 16, 32, 48 and row 1 on nibbles 16-31 of lanes 1, 17, 33, 49: row 0
// of the result is the running sum l of queries 0..15, row 1 that of queries 16..31, and lane c < 16 holds
// them in elements 0 and 1.  l is thus the sum of the e4m3-rounded P (the reference's accumulate_d sums p
// before rounding; the difference is the mean FP8 rounding error of P, far inside the attention tolerance);
// the row sums leave the softmax's VALU stream, and the MFMA costs half the 32 x 32 x 64 form.
__device__ __forceinline__ v8i row_sum_selector() {
  const int r = threadIdx.x & 15;
  const int lo = r == 0 ? 0x22222222 : 0, hi = r == 1 ? 0x22222222 : 0;
  return v8i{lo, lo, hi, hi, 0, 0, 0, 0};
}
__device__ __forceinline__ v4f row_sum_mfma(const v4f& acc, const v8i& pf, const v8i& sel) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(sel, pf, acc, 4, 0, 0, 0, 0, 0);
}
// online-softmax rescale of the row sums: element 0 of lane c belongs to query c (the lane's own), element 1
// to query c + 16, whose factor lane c + 16 holds
__device__ __forceinline__ void row_sum_rescale(v4f& acc, float alpha) {
  const int lane = threadIdx.x & 63;
  const float a_hi = __int_as_float(__builtin_amdgcn_ds_bpermute(((lane & 15) + 16) * 4, __float_as_int(alpha)));
  acc[0] *= alpha;
  acc[1] *= a_hi;
}
// the row sum of query lq (lanes lq and lq + 32 both get it)
__device__ __forceinline__ float row_sum_value(const v4f& acc, int lq) {
  const int src = (lq & 15) * 4;
  const float v0 = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(acc[0])));
  const float v1 = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(acc[1])));
  return lq < 16 ? v0 : v1;
}

// P.V flavours: e4m3 P x e4m3 V (the reference's fp8 kernel, with the 8.807 offset and v_scale), or
// P rounded to the half dtype of V x V as given (the Triton / SAGE_ATTN_2_8_16 style), fp32 accumulation.
enum PvKind { PV_FP8 = 0, PV_BF16 = 1, PV_FP16 = 2 };

template <bool IS_FP16_OUT, bool SPLIT, int PV, bool KT, bool SP = false, bool MQ = false>
__global__ __launch_bounds__(kThreads, kWavesPerSimd) void qattn_fwd_kernel(AttnParams p) {
  static_assert(!SP || (PV != PV_FP8 && !KT), "block-sparse launches use half P.V and per-block scales");
  static_assert(!MQ || (PV == PV_FP8 && !SPLIT && !SP), "multi-block launches: FP8 P.V, no split, dense");
  constexpr int KS = ks_per_tile(KT);
  constexpr int kVBytes = PV == PV_FP8 ? 1 : 2;    // bytes per V element
  constexpr int kVDma = 2 * kVBytes;                // V DMA instructions per wave per tile
  constexpr float kOffset = PV == PV_FP8 ? kFp8Offset : 0.f;
  __shared__ __align__(16) uint8_t lds_k[kNBuf][kBK * kD];
  __shared__ __align__(16) uint8_t lds_v[kNBuf][kD * kBK * kVBytes];
  __shared__ float lds_ks[SP ? kSpMaxTiles : MQ ? kMqMaxTiles * 4 : ks_lds_floats<PV>()];  // k_scales of its key tiles
  // multi-block launches: a wave-private 4 KiB region per wave that receives the next query block's Q
  // rows by DMA and then stages the finished block's O rows; and the q_scales of all its blocks
  __shared__ __align__(16) uint8_t lds_qo[MQ ? 4 * 4096 : 16];
  __shared__ float lds_qs[MQ ? kMqMaxBlocks * 32 : 1];
  __shared__ __align__(16) float lds_vs[PV == PV_FP8 ? kD : 4];  // v_scale of this head (epilogue)
  __shared__ __align__(16) float lds_vm[PV == PV_FP8 ? kD : 4];  // v_mean of this head (smoothed V)
  __shared__ int16_t lds_tid[SP ? kSpMaxTiles : 1];                  // block-sparse: ids of the active tiles
  __shared__ int lds_nact;

  const int64_t tile_id = xcd_remap(blockIdx.x, gridDim.x);
  int64_t qb, qb_end;  // query blocks [qb, qb_end) of this workgroup
  int64_t rest;
  int split = 0;
  if constexpr (MQ) {
    qb = (tile_id % p.nQC) * p.qpw;
    qb_end = min(p.nQB, qb + p.qpw);
    rest = tile_id / p.nQC;
  } else {
    qb = tile_id % p.nQB;
    qb_end = qb + 1;
    rest = tile_id / p.nQB;
    split = (int)(rest % p.nsplit);
    rest /= p.nsplit;
  }
  const int64_t qb0 = qb;
  const int64_t h = rest % p.Hq;
  const int64_t b = rest / p.Hq;
  const int64_t hk = h / p.group;

  // the batch entry's view: a dense batch, or one sequence of a packed variable-length batch
  int64_t Lq = p.Lq, Lk = p.Lk;
  const int8_t* q8b = p.q8 + b * p.qsb;
  const int8_t* k8b = p.k8 + b * p.ksb;
  int64_t vcol0 = 0;  // first key column of this entry in the V tile layout
  const float* qs_tab = p.q_scale + (b * p.Hq + h) * p.nQS;
  const float* ks_tab = p.k_scale + (b * p.Hkv + hk) * p.nKS;
  int64_t qs_stride = 1, ks_stride = 1;
  uint16_t* ob = static_cast<uint16_t*>(p.o) + b * p.osb;
  if (p.cu_q) {
    int64_t q0, k0s;
    varlen_range(p.cu_q, b, p.var_tq, p.Lq, q0, Lq);
    varlen_range(p.cu_k, b, p.var_tk, p.Lk, k0s, Lk);
    // (a V tile range past Lpad, from a too small Lpad, leaves the sequence's rows untouched)
    if (qb * kBQ >= Lq || Lk <= 0 || ((int64_t)p.cu_vt[b] + (Lk + kBK - 1) / kBK) * kBK > p.Lpad) return;
    q8b = p.q8 + q0 * p.qsl;
    k8b = p.k8 + k0s * p.ksl;
    vcol0 = (int64_t)p.cu_vt[b] * kBK;
    qs_tab = p.q_scale + (int64_t)p.cu_qs[b] * p.Hq + h;
    ks_tab = p.k_scale + (int64_t)p.cu_ks[b] * p.Hkv + hk;
    qs_stride = p.Hq;
    ks_stride = p.Hkv;
    ob = static_cast<uint16_t*>(p.o) + q0 * p.osl;
  }

  const int tid = threadIdx.x;
  // (wave index in a scalar register, so that every per-wave quantity and branch stays scalar)
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, lq = lane & 31, hf = lane >> 5;

  // key range of this workgroup
  int64_t q_first = qb * kBQ;
  int64_t kv_end = Lk;
  if (p.kv_valid) kv_end = min(kv_end, (int64_t)p.kv_valid[b]);
  if (p.causal) kv_end = min(kv_end, q_first + kBQ + p.q_offset);
  const int64_t n_tiles = kv_end > 0 ? (kv_end + kBK - 1) / kBK : 0;
  // The loop runs over "slots": every key tile (dense), or the tiles the block-sparse mask keeps for
  // this query block, in key order (sparse_int8_attn.py:57-58 skips a tile whose k_block_id is 0).
  int64_t t_begin = SPLIT ? (int64_t)split * p.tiles_per_split : 0;
  int64_t n_slots = n_tiles;
  if constexpr (SP) {
    if (w == 0) {  // wave 0 compacts the mask row with ballots; only this split's slots are stored
      const int8_t* mrow = p.tile_mask + (b * p.Hkv + hk) * p.tm_s1 + qb * p.tm_s2;
      int64_t cnt = 0;
      for (int64_t base = 0; base < n_tiles; base += 64) {
        const int64_t t = base + lane;
        const bool act = t < n_tiles && mrow[t] != 0;
        const uint64_t bal = __ballot(act);
        const int64_t slot = cnt + __popcll(bal & ((1ull << lane) - 1ull));
        if (act && slot >= t_begin && slot < t_begin + (SPLIT ? p.tiles_per_split : kSpMaxTiles))
          lds_tid[slot - t_begin] = (int16_t)t;
        cnt += __popcll(bal);
      }
      if (lane == 0) lds_nact = (int)cnt;
    }
    __syncthreads();
    n_slots = lds_nact;
  }
  const int64_t t_end = SPLIT ? min(n_slots, t_begin + p.tiles_per_split) : n_slots;
  // key tile of slot t (wave-uniform)
  auto tile_of = [&](int64_t t) -> int64_t {
    if constexpr (SP) return __builtin_amdgcn_readfirstlane((int)lds_tid[t - t_begin]);
    else return t;
  };

  // Q fragment (B operand of S^T = K.Q^T): lane owns query row lq of this wave, bytes
  // d = 32*m + 16*hf .. +16 for m = 0..3
  int64_t wrow0 = q_first + w * 32;
  int64_t qrow = wrow0 + lq;
  // Q fragments: the wave's 32 rows are read row-contiguously (8 lanes x 16 B per 128-byte row, full
  // cache lines) into a wave-private LDS stage, then each lane picks its MFMA B-operand bytes
  // d = 32 m + 16 hf .. +16 of row lq.  Stage rows are 128 B with the 16-byte chunk c stored at
  // chunk c ^ (row & 7), so both the row writes and the fragment reads are bank-conflict free.
  uint8_t* stage = (MQ ? &lds_qo[0] : &lds_k[0][0]) + w * 4096;  // 32 rows x 128 B per wave (lds_k is free here)
  v4i qf[4];
  {
    const int8_t* qbase = q8b + h * p.qsh;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = i * 8 + (lane >> 3), c = lane & 7;
      const int64_t row = wrow0 + r;
      const v4i val = row < Lq ? *reinterpret_cast<const v4i*>(qbase + row * p.qsl + c * 16) : v4i{0, 0, 0, 0};
      *reinterpret_cast<v4i*>(stage + r * 128 + ((c ^ (r & 7)) << 4)) = val;
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int m = 0; m < 4; m++) {
      const int c = 2 * m + hf;
      qf[m] = *reinterpret_cast<const v4i*>(stage + lq * 128 + ((c ^ (lq & 7)) << 4));
    }
    // consume the loads here: otherwise the compiler's wait for them lands at their first use inside
    // the key loop
#pragma unroll
    for (int m = 0; m < 4; m++) asm volatile("" ::"v"(qf[m]));
  }
  // q_scale of this lane's query row
  float qs = qs_tab[q_scale_index(p, qb * kBQ + w * 32 + lq) * qs_stride] * p.qk_mult;
  // q_scale entries per query block, and this lane's entry within its block
  const int qs_per = p.qgran == QATTN_GRAN_THREAD ? (kBQ >> p.qrs) * 8 : p.qgran == QATTN_GRAN_WARP ? kBQ >> p.qrs : 1;
  const int qs_sub = p.qgran == QATTN_GRAN_BLOCK ? 0 : (int)q_scale_index(p, w * 32 + lq);
  const float* ks_ptr = ks_tab;

  // global -> LDS copies go through the LDS-DMA path (buffer_load_dwordx4 ... lds): lane j of a wave
  // writes the 16 bytes at LDS slot (wave base + 16 j).  The tiles are fragment-major: 1 KiB block f holds
  // MFMA operand fragment f of all 64 lanes (lane l at 16 l), so a lane reads its fragments at one base
  // address plus constant offsets, each read a contiguous, conflict-free 1 KiB:
  //   K block j (0..7): lane l gets K row (j & 1) * 32 + l % 32, bytes 16 (2 (j >> 1) + l / 32) .. + 16
  //   FP8 V block 2 dblk + h: lane l gets V^T row dblk * 32 + l % 32, bytes 16 (2 (l / 32) + h) .. + 16
  //   half V block 4 dblk + c: lane l gets V^T row dblk * 32 + l % 32, bytes 16 (4 (l / 32) + c) .. + 16
  // DMA instruction i of wave w fills block 4 i + w.  Each wave moves 2 x 1 KiB of K and kVDma x 1 KiB of V
  // per tile; no VGPRs are spent on staging.
  // The K resource of a tile starts at the tile's first row, so K rows at or past Lk fall outside its
  // range and arrive as zeros (masked anyway) without being read (the range check covers the
  // per-lane offset, not the scalar one).
  const int8_t* kbase = k8b + hk * p.ksh;
  const uint8_t* vbase = static_cast<const uint8_t*>(p.v) + ((p.cu_q ? 0 : b) * p.Hkv + hk) * (int64_t)kD * p.Lpad * kVBytes +
                         vcol0 * kVBytes;
  const int64_t kbytes = (Lk - 1) * p.ksl + kD;
  const v4u vrsrc = make_rsrc(vbase, (uint32_t)(((int64_t)kD * p.Lpad - vcol0) * kVBytes));
  // per-lane byte offsets relative to the tile start (first K row / first V column)
  uint32_t koff[2], voff[kVDma];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int j = i * 4 + w;
    koff[i] = (uint32_t)(((j & 1) * 32 + lq) * p.ksl + (2 * (j >> 1) + hf) * 16);
  }
#pragma unroll
  for (int i = 0; i < kVDma; i++) {
    const int f = i * 4 + w;
    if constexpr (PV == PV_FP8) voff[i] = (uint32_t)(((f >> 1) * 32 + lq) * p.Lpad + (2 * hf + (f & 1)) * 16);
    else voff[i] = (uint32_t)(((f >> 2) * 32 + lq) * p.Lpad * 2 + (4 * hf + (f & 3)) * 16);
  }
  const int64_t k_step = kBK * p.ksl;
  const uint32_t lds_k0 = lds_addr(&lds_k[0][0]) + __builtin_amdgcn_readfirstlane(w) * 1024;
  const uint32_t lds_v0 = lds_addr(&lds_v[0][0]) + __builtin_amdgcn_readfirstlane(w) * 1024;
  auto dma_tile = [&](int64_t t, int buf) {
    const int64_t kso = t * k_step;
    const v4u krsrc = make_rsrc(kbase + kso, (uint32_t)(kbytes - kso));
    const uint32_t vso = (uint32_t)t * (kBK * kVBytes);
    const uint32_t kl = lds_k0 + buf * (kBK * kD), vl = lds_v0 + buf * (kD * kBK * kVBytes);
#pragma unroll
    for (int i = 0; i < 2; i++) lds_dma16(koff[i], krsrc, 0, kl + i * 4096);
#pragma unroll
    for (int i = 0; i < kVDma; i++) lds_dma16(voff[i], vrsrc, vso, vl + i * 4096);
  };
  // multi-block launches: the wave's 32 rows of the next query block go by DMA into its region of
  // lds_qo, in the stage layout (LDS slot (r, c') receives global chunk c' ^ (r & 7)); the resource
  // covers exactly the rows below Lq, the others arrive as zeros
  uint32_t qoff[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int slot = i * 64 + lane, r = slot >> 3;
    qoff[i] = (uint32_t)(r * p.qsl + (((slot & 7) ^ (r & 7)) << 4));
  }
  const int8_t* qhead = q8b + h * p.qsh;
  const int wu = __builtin_amdgcn_readfirstlane(w);
  auto dma_q = [&](int64_t blk) {
    const int64_t r0 = blk * kBQ + wu * 32;
    const int64_t nr = min((int64_t)32, Lq - r0);
    const v4u qr = make_rsrc(qhead + (nr > 0 ? r0 * p.qsl : 0), nr > 0 ? (uint32_t)((nr - 1) * p.qsl + kD) : 0u);
    const uint32_t ql = lds_addr(&lds_qo[0]) + wu * 4096;
#pragma unroll
    for (int i = 0; i < 4; i++) lds_dma16(qoff[i], qr, 0, ql + i * 1024);
  };

  v16f o[4];
#pragma unroll
  for (int i = 0; i < 4; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[i][r] = 0.f;
  float m_run = kMInit, l_run = 0.f;
  v4f lacc = {0.f, 0.f, 0.f, 0.f};  // FP8 P.V: row sums of P on the matrix pipe (row_sum_mfma)
  const v8i rs_sel = row_sum_selector();
  v16i kbias;
#pragma unroll
  for (int r = 0; r < 16; r++) kbias[r] = kAccBiasBits;

  // K/V tiles run kPrefetch tiles ahead of the compute through kNBuf = kPrefetch + 1 LDS buffers:
  // iteration t issues tile t + kPrefetch into buffer (t + kPrefetch) % kNBuf, which was last read in
  // iteration t - 1.  The k_scales of all tiles are staged in LDS once, so the only VMEM traffic in the
  // loop is the 4 DMA instructions per tile and the vmcnt accounting below is exact.
  __syncthreads();  // every wave has its Q fragments out of the LDS stage before the DMA reuses it
  if constexpr (SP) {
    for (int64_t i = tid; i < t_end - t_begin; i += kThreads) lds_ks[i] = ks_ptr[lds_tid[i] * ks_stride];
  } else {
    for (int64_t i = tid; i < (t_end - t_begin) * KS; i += kThreads) lds_ks[i] = ks_ptr[k_scale_index(p, t_begin + i / KS, i % KS, KS) * ks_stride];
  }
  if constexpr (PV == PV_FP8 && !SPLIT)
    if (tid < kD) {
      lds_vs[tid] = p.v_scale[(b * p.Hkv + hk) * kD + tid];
      lds_vm[tid] = p.v_mean ? p.v_mean[(b * p.Hkv + hk) * kD + tid] : 0.f;
    }
  if constexpr (MQ) {
    const float* qsp = p.q_scale + (b * p.Hq + h) * p.nQS + qb0 * qs_per;
    const int64_t n_qs = std::min<int64_t>((qb_end - qb0) * qs_per, p.nQS - qb0 * qs_per);
    for (int64_t i = tid; i < n_qs; i += kThreads) lds_qs[i] = qsp[i];
  }
  // The loop runs over (query block, key tile) pairs: a multi-block launch walks the same key tiles once
  // per query block, and its DMA stream runs on across the block boundaries.
  const int64_t n_kt = t_end - t_begin;
  const int64_t total = MQ ? (qb_end - qb0) * n_kt : n_kt;
#pragma unroll
  for (int d = 0; d < kPrefetch; d++)
    if (d < total) dma_tile(tile_of(t_begin + (MQ ? d % n_kt : d)), d);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  // ---- epilogue of the current query block: O / l * v_scale out through the wave's LDS stage ----
  auto finish = [&]() {
    float l_tot;
    if constexpr (PV == PV_FP8) {
      l_tot = row_sum_value(lacc, lq);
    } else {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(l_run), __float_as_uint(l_run), false, false);
      l_tot = __uint_as_float(sw[0]) + __uint_as_float(sw[1]);
    }
    if (SPLIT) {
      if (qrow >= Lq) return;
      const int64_t row = (((int64_t)split * p.B + b) * p.Hq + h) * p.Lq + qrow;
      float* wo = p.ws_o + row * kD;
#pragma unroll
      for (int dblk = 0; dblk < 4; dblk++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int d = dblk * 32 + g * 8 + hf * 4;
          *reinterpret_cast<v4f*>(wo + d) =
              v4f{o[dblk][g * 4 + 0], o[dblk][g * 4 + 1], o[dblk][g * 4 + 2], o[dblk][g * 4 + 3]};
        }
      if (hf == 0) {
        p.ws_ml[row * 2 + 0] = m_run;
        p.ws_ml[row * 2 + 1] = l_tot;
      }
      return;
    }
    const float inv_l = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    // O goes out through the wave-private LDS stage (the K/V buffers are idle after the loop's last
    // barrier; multi-block launches use their own region), 64 channels per pass, so that every row is
    // stored as whole 128-byte lines
    uint16_t* obase = ob + h * p.osh;
    auto store = [&](auto mean_t) {
    constexpr bool kMean = decltype(mean_t)::value;
#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
#pragma unroll
      for (int db = 0; db < 2; db++) {
        const int dblk = pass * 2 + db;
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int d = dblk * 32 + g * 8 + hf * 4;
          const v4f sc = PV == PV_FP8 ? *reinterpret_cast<const v4f*>(&lds_vs[d]) : v4f{1.f, 1.f, 1.f, 1.f};
          float f[4];
          const v4f vm = kMean ? *reinterpret_cast<const v4f*>(&lds_vm[d]) : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int e = 0; e < 4; e++) f[e] = epilogue_value<kMean>(o[dblk][g * 4 + e], inv_l, sc[e], vm[e]);
          const v2u packed{pack_half2<IS_FP16_OUT>(f[0], f[1]), pack_half2<IS_FP16_OUT>(f[2], f[3])};
          const int c = db * 4 + g;  // 16-byte chunk of the staged 128-byte row (8 channels)
          *reinterpret_cast<v2u*>(stage + lq * 128 + ((c ^ (lq & 7)) << 4) + hf * 8) = packed;
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int r = i * 8 + (lane >> 3), c = lane & 7;
        const v4u val = *reinterpret_cast<const v4u*>(stage + r * 128 + ((c ^ (r & 7)) << 4));
        const int64_t row = wrow0 + r;
        if (row < Lq) *reinterpret_cast<v4u*>(obase + row * p.osl + pass * 64 + c * 8) = val;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    };
    if (PV == PV_FP8 && p.v_mean) store(std::true_type{});
    else store(std::false_type{});
    if (p.lse && hf == 0 && qrow < Lq)
      p.lse[(b * p.Hq + h) * p.Lq + qrow] = l_tot > 0.f ? __builtin_log2f(l_tot) + m_run : -INFINITY;
  };
  [[maybe_unused]] auto next_block = [&]() {
    qb++;
    q_first = qb * kBQ;
    wrow0 = q_first + w * 32;
    qrow = wrow0 + lq;
    qs = lds_qs[(qb - qb0) * qs_per + qs_sub] * p.qk_mult;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) o[i][r] = 0.f;
    m_run = kMInit;
    l_run = 0.f;
    lacc = v4f{0.f, 0.f, 0.f, 0.f};
  };

  int buf = 0;
  int64_t t = t_begin;                            // key slot being computed
  int64_t pt = t_begin + (MQ && total > 0 ? kPrefetch % n_kt : kPrefetch);  // next slot to fetch
  for (int64_t it = 0; it < total; it++) {
    const bool issue = it + kPrefetch < total;
    // (issued before this iteration's K/V DMA, so the iteration's final vmcnt wait covers it)
    if constexpr (MQ)
      if (t == 0 && qb + 1 < qb_end) dma_q(qb + 1);
    if (issue) {
      dma_tile(tile_of(pt), buf == 0 ? kNBuf - 1 : buf - 1);
      pt++;
      if (MQ && pt == t_end) pt = t_begin;
    }
    // logit scale(s) of this lane: with per-thread K scales, key kappa of the tile belongs to class
    // (kappa % 8) / 2 = 2 hf + (r & 3) / 2 for accumulator element r, so a lane needs two of them
    float cs_a, cs_b;
    if constexpr (KT) {
      cs_a = qs * lds_ks[(t - t_begin) * 4 + 2 * hf];
      cs_b = qs * lds_ks[(t - t_begin) * 4 + 2 * hf + 1];
    } else {
      cs_a = cs_b = qs * lds_ks[t - t_begin];
    }

    // ---- S^T = K . Q^T: two 32-key blocks x 4 MFMAs over D = 128; K fragments streamed from LDS ----
    v16i s[2];
    {
      v4i kf[8];  // all K fragments first: the LDS latency is paid once per tile
#pragma unroll
      for (int j = 0; j < 8; j++)
        kf[j] = *reinterpret_cast<const v4i*>(&lds_k[buf][j * 1024 + lane * 16]);
      // The QK MFMAs run at raised wave priority: when the other wave of the SIMD is in its softmax
      // VALU phase, the scheduler then keeps the matrix pipe fed from this wave (measured ~6 % faster
      // than equal priorities).
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int m = j >> 1, kb = j & 1;
        s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[j], qf[m], m == 0 ? kbias : s[kb], 0, 0, 0);
      }
      __builtin_amdgcn_s_setprio(0);
    }

    // ---- masking (tail tile, key padding, causal diagonal) ----
    const int64_t k0 = tile_of(t) * kBK;
    const bool masked = (k0 + kBK > kv_end) || (p.causal && k0 + kBK - 1 > wrow0 + p.q_offset);
    if (masked) {
      // element r of block kb holds key k0 + c + 4 hf with c = 32 kb + 8 (r / 4) + r % 4; it is masked
      // when key >= kv_end or (causal) key > qrow + q_offset, i.e. when c >= lim for this lane's lim
      int lim = (int)min(kv_end - k0, (int64_t)kBK);
      if (p.causal) lim = min(lim, (int)max(min(qrow + p.q_offset + 1 - k0, (int64_t)kBK), (int64_t)-1));
      lim -= hf * 4;
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          if (kb * 32 + (r >> 2) * 8 + (r & 3) >= lim) s[kb][r] = INT32_MIN;
    }

    // ---- online softmax ----
    float m_tile;
    if constexpr (!KT) {
      int mx = max(s[0][0], s[0][1]);
#pragma unroll
      for (int r = 2; r < 16; r++) mx = max(mx, s[0][r]);
#pragma unroll
      for (int r = 0; r < 16; r++) mx = max(mx, s[1][r]);
      {  // lanes l and l^32 hold the two key halves of the same query row
        const auto sw = __builtin_amdgcn_permlane32_swap(mx, mx, false, false);
        mx = max((int)sw[0], (int)sw[1]);
      }
      // Lazy rescale: the running max m is only moved when the tile max exceeds it by more than
      // kLazyTau (log2 units), per row.  With the offset lowered by the same tau, p = exp2(s - m) stays
      // <= 2^8.807 = 448 (the e4m3 maximum), so the FP8 range is honoured while the O rescale (64
      // multiplies per lane) is skipped on almost every tile.  A row whose keys in this tile are all
      // masked never moves m.
      m_tile = mx == INT32_MIN ? kMInit : fmaf(__int_as_float(mx), cs_a, -fmaf(kAccBias, cs_a, kOffset - kLazyTau));
    } else {  // two scale classes per lane: max per class, scaled, then across the lane pair
      int ma = INT32_MIN, mb = INT32_MIN;
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          if ((r & 3) < 2) ma = max(ma, s[kb][r]);
          else mb = max(mb, s[kb][r]);
        }
      const float fa = ma == INT32_MIN ? kMInit : fmaf(__int_as_float(ma), cs_a, -fmaf(kAccBias, cs_a, kOffset - kLazyTau));
      const float fb = mb == INT32_MIN ? kMInit : fmaf(__int_as_float(mb), cs_b, -fmaf(kAccBias, cs_b, kOffset - kLazyTau));
      float mt = fmaxf(fa, fb);
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
      m_tile = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    const bool grow = m_tile > m_run + kLazyTau;
    if (__any(grow)) {
      const float m_new = grow ? m_tile : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      l_run *= alpha;
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] *= alpha;
      if constexpr (PV == PV_FP8) row_sum_rescale(lacc, alpha);
      m_run = m_new;
    }
    const float nc_a = -fmaf(kAccBias, cs_a, m_run), nc_b = -fmaf(kAccBias, cs_b, m_run);
    // p = exp2(s * cs - m); masked logits (INT32_MIN) become p = 0 exactly (the sentinel times a tiny
    // block scale is not necessarily very negative)
    auto p4 = [&](int j, float (&pv)[4], auto mk) {
      const int kb = j >> 2, r0 = (j & 3) * 4;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int sv = s[kb][r0 + e];
        pv[e] = __builtin_amdgcn_exp2f(fmaf(__int_as_float(sv), e < 2 ? cs_a : cs_b, e < 2 ? nc_a : nc_b));
        if constexpr (decltype(mk)::value) pv[e] = sv == INT32_MIN ? 0.f : pv[e];
      }
    };
    if constexpr (PV == PV_FP8) {
      v8i pf;  // P^T as the e4m3 B operand: byte s of the lane = slot s = 16 kb + r
      // u = 8 (s * cs - m - kPLinShift) + 56 (p_e4m3_x4); masked logits give u = -1, P = 0
      const float cs8_a = 8.0f * cs_a, cs8_b = 8.0f * cs_b;
      const float nu_a = fmaf(-8.0f, fmaf(kAccBias, cs_a, m_run), kPLinBias);
      const float nu_b = fmaf(-8.0f, fmaf(kAccBias, cs_b, m_run), kPLinBias);
      auto body = [&](auto mk) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int kb = j >> 2, r0 = (j & 3) * 4;
          float u[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int sv = s[kb][r0 + e];
            u[e] = fmaf(__int_as_float(sv), e < 2 ? cs8_a : cs8_b, e < 2 ? nu_a : nu_b);
            if constexpr (decltype(mk)::value) u[e] = sv == INT32_MIN ? -1.f : u[e];
          }
          pf[j] = p_e4m3_x4(u[0], u[1], u[2], u[3]);
        }
      };
      if (masked) body(std::true_type{});
      else body(std::false_type{});

      // ---- O^T += V^T . P^T (FP8 MFMA, K = 64 keys) ----
      v8i vf[4];
#pragma unroll
      for (int dblk = 0; dblk < 4; dblk++) {
        const v4i a0 = *reinterpret_cast<const v4i*>(&lds_v[buf][(2 * dblk) * 1024 + lane * 16]);
        const v4i a1 = *reinterpret_cast<const v4i*>(&lds_v[buf][(2 * dblk + 1) * 1024 + lane * 16]);
        vf[dblk] = v8i{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      }
#pragma unroll
      for (int dblk = 0; dblk < 4; dblk++)
        o[dblk] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf[dblk], pf, o[dblk], 0, 0, 0, 0, 0, 0);
      lacc = row_sum_mfma(lacc, pf, rs_sel);
    } else {
      // P^T in the half dtype: chunk c (16 keys of the MFMA's K dimension) = slots 8c .. 8c+7
      typedef __attribute__((ext_vector_type(8))) __bf16 v8bf;
      typedef __attribute__((ext_vector_type(8))) _Float16 v8h;
      using HV = std::conditional_t<PV == PV_BF16, v8bf, v8h>;
      using HS = std::conditional_t<PV == PV_BF16, __bf16, _Float16>;
      HV ph[4];
      auto body = [&](auto mk) {
        float lsum = 0.f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
          float pv[4];
          p4(j, pv, mk);
          lsum += (pv[0] + pv[1]) + (pv[2] + pv[3]);
#pragma unroll
          for (int e = 0; e < 4; e++) ph[j >> 1][(j & 1) * 4 + e] = (HS)pv[e];  // RNE
        }
        l_run += lsum;
      };
      if (masked) body(std::true_type{});
      else body(std::false_type{});

      // ---- O^T += V^T . P^T (half MFMA 32x32x16, 4 K-chunks per 32-channel block) ----
#pragma unroll
      for (int dblk = 0; dblk < 4; dblk++) {
        HV vf[4];
#pragma unroll
        for (int c = 0; c < 4; c++)
          vf[c] = *reinterpret_cast<const HV*>(&lds_v[buf][(4 * dblk + c) * 1024 + lane * 16]);
#pragma unroll
        for (int c = 0; c < 4; c++) {
          if constexpr (PV == PV_BF16) o[dblk] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[c], ph[c], o[dblk], 0, 0, 0);
          else o[dblk] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vf[c], ph[c], o[dblk], 0, 0, 0);
        }
      }
    }

    // tile t+1 must have landed; the DMAs of the tiles after it may stay in flight
    if (issue) asm volatile("s_waitcnt vmcnt(%0)" ::"n"((2 + kVDma) * (kPrefetch - 1)) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    buf = buf + 1 == kNBuf ? 0 : buf + 1;
    t++;
    if constexpr (MQ) {
      if (t == t_end && qb + 1 < qb_end) {
        // block boundary: the next block's Q rows (landed with this iteration's wait) leave the region
        // before the finished block's O goes out through it
        v4i qn[4];
#pragma unroll
        for (int m = 0; m < 4; m++) {
          const int c = 2 * m + hf;
          qn[m] = *reinterpret_cast<const v4i*>(stage + lq * 128 + ((c ^ (lq & 7)) << 4));
        }
        finish();
#pragma unroll
        for (int m = 0; m < 4; m++) qf[m] = qn[m];
        next_block();
        t = t_begin;
      }
    }
  }
  if constexpr (MQ) {
    // no key tiles at all (kv_valid 0): every block of the workgroup gets the empty-row output
    if (total == 0)
      while (qb + 1 < qb_end) {
        finish();
        next_block();
      }
  }
  finish();
}

// ---- ping-pong workgroups: two groups of four waves, one wave of each group per SIMD ----
//
// In qattn_fwd_kernel the two waves of a SIMD belong to different workgroups and fall into step with
// each other: both run their softmax on the VALU, then both run their MFMAs, so a SIMD spends the sum
// of the two phases per tile.  Here one workgroup holds two query blocks of the same head (group 0 =
// waves 0-3, group 1 = waves 4-7; wave w runs on SIMD w % 4) and the groups alternate through workgroup
// barriers, half a tile apart:
//
//   group 0:  M(0) | V(0) | M(1) | V(1) | ...        M(t) = P(t-1).V(t-1), row sum, Q.K(t)^T (matrix pipe)
//   group 1:    -  | M(0) | V(0) | M(1) | ...        V(t) = mask, softmax, P(t) to e4m3  (VALU)
//
// so at every step one wave of a SIMD feeds the matrix pipe while the other runs the VALU softmax, and
// a SIMD spends about max(MFMA, VALU) per step instead of their sum.  Per element the arithmetic is
// that of qattn_fwd_kernel (32 rows per wave, same MFMA chains, lazy running max, FP8 offset, row sums
// on the matrix pipe), so both kernels give identical results.
//
// K/V tiles come in by LDS DMA, four buffers, two tiles ahead: every wave moves 1 KiB of K and 1 KiB of
// V of tile t + 2 at the start of its stage M(t) and has its share of tile t + 1 landed by the end of
// M(t); tile t is read as K in M(t) and as V during V(t) (operands of M(t + 1)), so its buffer is free
// once both groups have finished M(t + 1).
constexpr int kPPThreads = 512;
constexpr int kPPNBuf = 4;

// QF: Q as int8 with its scale table (0), or Q in the output's half type quantized inside the attention
// kernel: with the per-thread classes of the Triton quantizer (QF_THREAD: rows with equal row % 8 of a wave's
// 32 share a scale, round half away from x / scale), the per-warp blocks of the CUDA one (QF_WARP: a wave's
// 32 rows share a scale, RNE of x * 127 / amax), or its per-block form (QF_BLOCK: the
// 128 rows of a query block, held by four waves of one workgroup, share a scale, x multiplied by
// sm_scale * log2(e) first) -- the codes and
// scales of per_thread_int8 / per_warp_int8 / per_block_int8 bit for bit, without writing int8 Q out and
// reading it back.
constexpr int QF_INT8 = 0, QF_THREAD = 1, QF_WARP = 2, QF_BLOCK = 3;

// Lane (lq, hf) of a wave whose 32 query rows are lq = lane % 32: the raw half words of its row (row
// pointer rowp; zeros when !valid) at 32 m + 16 hf .. + 16, m < NQF.
template <int NQF>
__device__ __forceinline__ void quant_q_raw(const uint16_t* rowp, bool valid, int hf, v4u (&r)[NQF][2]) {
#pragma unroll
  for (int m = 0; m < NQF; m++) {
    r[m][0] = r[m][1] = v4u{0, 0, 0, 0};
    if (valid) {
      r[m][0] = *reinterpret_cast<const v4u*>(rowp + m * 32 + hf * 16);
      r[m][1] = *reinterpret_cast<const v4u*>(rowp + m * 32 + hf * 16 + 8);
    }
  }
}

// Those values as fp32, times mul when MUL.
template <bool IS_FP16, int NQF, bool MUL>
__device__ __forceinline__ void quant_q_unpack(const v4u (&r)[NQF][2], float mul, float (&x)[NQF][16]) {
#pragma unroll
  for (int m = 0; m < NQF; m++) {
#pragma unroll
    for (int e = 0; e < 4; e++) {
      x[m][2 * e] = half_to_f32<IS_FP16>((uint16_t)(r[m][0][e] & 0xffffu));
      x[m][2 * e + 1] = half_to_f32<IS_FP16>((uint16_t)(r[m][0][e] >> 16));
      x[m][8 + 2 * e] = half_to_f32<IS_FP16>((uint16_t)(r[m][1][e] & 0xffffu));
      x[m][8 + 2 * e + 1] = half_to_f32<IS_FP16>((uint16_t)(r[m][1][e] >> 16));
    }
    if constexpr (MUL) {
#pragma unroll
      for (int e = 0; e < 16; e++) x[m][e] = x[m][e] * mul;
    }
  }
}

// The |x| maximum over the lane's scale group within the wave (per-thread class: lanes lq ^ 8, lq ^ 16 and
// the other half-row; per-warp / per-block: all 64 lanes, from the CUDA quantizer's 1e-7 floor).
template <int QF, int NQF>
__device__ __forceinline__ float quant_q_amax(const float (&x)[NQF][16]) {
  float am = QF == QF_THREAD ? 0.f : 0.0000001f;
#pragma unroll
  for (int m = 0; m < NQF; m++)
#pragma unroll
    for (int e = 0; e < 16; e++) am = fmaxf(am, fabsf(x[m][e]));
  if constexpr (QF != QF_THREAD) {
    am = fmaxf(am, __shfl_xor(am, 1, 64));
    am = fmaxf(am, __shfl_xor(am, 2, 64));
    am = fmaxf(am, __shfl_xor(am, 4, 64));
  }
  am = fmaxf(am, __shfl_xor(am, 8, 64));
  am = fmaxf(am, __shfl_xor(am, 16, 64));
  am = fmaxf(am, __shfl_xor(am, 32, 64));
  return am;
}

// The three steps at once: the lane's values x (times mul when MUL) and their group maximum.
template <bool IS_FP16, int QF, int NQF, bool MUL = false>
__device__ __forceinline__ float quant_q_load(const uint16_t* rowp, bool valid, int hf, float mul, float (&x)[NQF][16]) {
  v4u r[NQF][2];
  quant_q_raw<NQF>(rowp, valid, hf, r);
  quant_q_unpack<IS_FP16, NQF, MUL>(r, mul, x);
  return quant_q_amax<QF, NQF>(x);
}

// The scale of a group with |x| maximum am (returned) and the int8 codes as the MFMA B fragments qf.
template <int QF, int NQF>
__device__ __forceinline__ float quant_q_codes(const float (&x)[NQF][16], float am, v4i (&qf)[NQF]) {
  constexpr bool TRITON = QF == QF_THREAD;
  const float sc = TRITON ? quant_scale_triton(am) : quant_scale_cuda(am);
  const float iv = TRITON ? refined_rcp(sc) : quant_recip_cuda(am);
#pragma unroll
  for (int m = 0; m < NQF; m++) {
    int c[16];
#pragma unroll
    for (int e = 0; e < 16; e++) c[e] = TRITON ? quant_code_triton(x[m][e], sc, iv) : quant_code_cuda(x[m][e], iv);
#pragma unroll
    for (int g = 0; g < 4; g++)
      qf[m][g] = (c[4 * g] & 0xff) | ((c[4 * g + 1] & 0xff) << 8) | ((c[4 * g + 2] & 0xff) << 16) | (c[4 * g + 3] << 24);
  }
  return sc;
}

// per-thread / per-warp: both steps within the wave
template <bool IS_FP16, int QF, int NQF>
__device__ __forceinline__ float quant_q_rows(const uint16_t* rowp, bool valid, int hf, v4i (&qf)[NQF]) {
  static_assert(QF == QF_THREAD || QF == QF_WARP, "wave-local scale groups");
  float x[NQF][16];
  const float am = quant_q_load<IS_FP16, QF, NQF>(rowp, valid, hf, 1.f, x);
  return quant_q_codes<QF, NQF>(x, am, qf);
}

// workgroup barrier that the compiler neither crosses with memory operations nor schedules around
__device__ __forceinline__ void pp_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

template <bool IS_FP16_OUT, bool KT, bool SPLIT, int HD, int QF = QF_INT8>
__device__ __forceinline__ void qattn_fwd_pp(const AttnParams& p) {
  // HD: head dimension, 128 or 64.  Per 64-key tile a wave runs HD / 16 Q.K^T MFMAs (two key blocks x HD / 32
  // k-steps) and HD / 32 P.V MFMAs; K and V tiles are HD / 16 fragments of 1 KiB each.
  static_assert(HD == 128 || HD == 64, "head_dim 128 or 64");
  constexpr int NQF = HD / 32;  // Q fragments (k-steps of 32) = P.V output blocks of 32 dims
  constexpr int NKF = HD / 16;  // K fragments per tile = V fragments per tile
  constexpr int ROWB = HD;      // bytes of one int8 Q row
  constexpr int KS = ks_per_tile(KT);
  constexpr int NB = kPPNBuf;
  // the K buffers double as the waves' Q / O stage (4 KiB per wave), so they span at least 32 KiB
  constexpr int kKBytes = NB * kBK * HD > 8 * 4096 ? NB * kBK * HD : 8 * 4096;
  __shared__ __align__(16) uint8_t lds_kbuf[kKBytes];
  auto lds_k = reinterpret_cast<uint8_t (*)[kBK * HD]>(lds_kbuf);
  __shared__ __align__(16) uint8_t lds_v[NB][HD * kBK];
  auto buf_of = [](int t) { return (int)((unsigned)t % (unsigned)NB); };
  __shared__ float lds_ks[ks_lds_floats<PV_FP8>()];
  __shared__ __align__(16) float lds_vs[HD];
  __shared__ __align__(16) float lds_vm[HD];

  const int64_t nQP = (p.nQB + 1) / 2;
  const int64_t wg_id = xcd_remap(blockIdx.x, gridDim.x);
  // KV split: split-major order, so the workgroups of one key range of a head run next to each other
  const int64_t n_pairs = p.B * p.Hq * nQP;
  const int split = SPLIT ? (int)(wg_id / n_pairs) : 0;
  const int64_t tile_id = SPLIT ? wg_id - (int64_t)split * n_pairs : wg_id;
  const int64_t qp = tile_id % nQP;
  const int64_t rest = tile_id / nQP;
  const int64_t h = rest % p.Hq;
  const int64_t b = rest / p.Hq;
  const int64_t hk = h / p.group;

  const int tid = threadIdx.x;
  // (wave index in a scalar register, so that every per-wave quantity and branch stays scalar)
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, lq = lane & 31, hf = lane >> 5;
  const int grp = w >> 2, wl = w & 3;
  const int64_t qb = qp * 2 + grp;  // == nQB for the empty second group of an odd block count
  const int64_t q_first = qb * kBQ;
  const int64_t wrow0 = q_first + wl * 32;
  const int64_t qrow = wrow0 + lq;

  // key range of this group, and of the workgroup (its last non-empty group)
  int64_t kv_lim = p.Lk;
  if (p.kv_valid) kv_lim = min(kv_lim, (int64_t)p.kv_valid[b]);
  int64_t kv_end = kv_lim, kv_end_wg = kv_lim;
  if (p.causal) {
    kv_end = min(kv_lim, q_first + kBQ + p.q_offset);
    kv_end_wg = min(kv_lim, min(qp * 2 + 1, p.nQB - 1) * kBQ + kBQ + p.q_offset);
  }
  // (wave-uniform values in scalar registers: kv_valid comes through a vector load)
  const int kv_end_s = __builtin_amdgcn_readfirstlane((int)kv_end);
  // last key that the wave's first row may see (causal), clamped so that adding a row index stays in range
  constexpr int kNoDiag = INT32_MAX - 128;
  const int diag_s = p.causal ? __builtin_amdgcn_readfirstlane((int)min(wrow0 + p.q_offset, (int64_t)kNoDiag)) : kNoDiag;
  const int n_tiles = __builtin_amdgcn_readfirstlane(kv_end_wg > 0 ? (int)((kv_end_wg + kBK - 1) / kBK) : 0);
  // this workgroup's key tiles t_lo .. t_end - 1 (the split's run, as in qattn_fwd_kernel)
  const int t_lo = SPLIT ? split * p.tiles_per_split : 0;
  const int t_end = SPLIT ? min(n_tiles, t_lo + p.tiles_per_split) : n_tiles;

  // Q fragments through the wave-private LDS stage (rows row-contiguous, 16-byte chunk c of row r at
  // c ^ (r % chunks per row))
  constexpr int QC = ROWB / 16;  // 16-byte chunks per Q row
  uint8_t* stage = &lds_k[0][0] + w * 4096;
  v4i qf[NQF];
  float qs;
  auto load_q = [&]() {
  if constexpr (QF == QF_BLOCK) {
    // half Q quantized per 128-row block: the four waves of a group exchange their maxima through LDS
    // (q_sm_scale = sm_scale * log2(e) multiplied in first; the logits then take qk_mult = 1)
    __shared__ float lds_qam[8];
    const uint16_t* qh16 = reinterpret_cast<const uint16_t*>(p.q8) + b * p.qsb + h * p.qsh;
    float x[NQF][16];
    const float am_w = quant_q_load<IS_FP16_OUT, QF, NQF, true>(qh16 + qrow * p.qsl, qrow < p.Lq, hf, p.q_sm_scale, x);
    if (lane == 0) lds_qam[w] = am_w;
    __syncthreads();
    const float am = fmaxf(fmaxf(lds_qam[grp * 4], lds_qam[grp * 4 + 1]), fmaxf(lds_qam[grp * 4 + 2], lds_qam[grp * 4 + 3]));
    qs = quant_q_codes<QF, NQF>(x, am, qf) * p.qk_mult;
  } else if constexpr (QF != QF_INT8) {
    // half Q quantized by the wave itself (see quant_q_rows)
    const uint16_t* qh16 = reinterpret_cast<const uint16_t*>(p.q8) + b * p.qsb + h * p.qsh;
    qs = quant_q_rows<IS_FP16_OUT, QF, NQF>(qh16 + qrow * p.qsl, qrow < p.Lq, hf, qf) * p.qk_mult;
  } else {
    const int8_t* qbase = p.q8 + b * p.qsb + h * p.qsh;
#pragma unroll
    for (int i = 0; i < 32 * QC / 64; i++) {
      const int r = i * (64 / QC) + lane / QC, c = lane % QC;
      const int64_t row = wrow0 + r;
      const v4i val = row < p.Lq ? *reinterpret_cast<const v4i*>(qbase + row * p.qsl + c * 16) : v4i{0, 0, 0, 0};
      *reinterpret_cast<v4i*>(stage + r * ROWB + ((c ^ (r % QC)) << 4)) = val;
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int m = 0; m < NQF; m++) {
      const int c = 2 * m + hf;
      qf[m] = *reinterpret_cast<const v4i*>(stage + lq * ROWB + ((c ^ (lq % QC)) << 4));
    }
#pragma unroll
    for (int m = 0; m < NQF; m++) asm volatile("" ::"v"(qf[m]));
    const int64_t qbs = min(qb, p.nQB - 1);
    const int64_t qsi = q_scale_index(p, qbs * kBQ + wl * 32 + lq);
    qs = p.q_scale[(b * p.Hq + h) * p.nQS + qsi] * p.qk_mult;
  }
  };
  // int8 Q goes through the LDS stage, which the first DMAs overwrite: it is loaded first.  Half Q is
  // quantized in registers, so its loads are issued behind the first DMAs and their latencies overlap.
  if constexpr (QF == QF_INT8) load_q();
  const float* ks_ptr = p.k_scale + (b * p.Hkv + hk) * p.nKS;

  // K/V tiles in LDS, fragment-major: 1 KiB block j holds MFMA operand fragment j of all 64 lanes (lane l
  // at 16 l), so a lane reads its fragments at one per-tile base address plus constant offsets (no
  // per-fragment address arithmetic) and every read is a contiguous, conflict-free 1 KiB.
  //   K block j (0..7): lane l gets K row (j & 1) * 32 + l % 32, bytes 16 (2 (j >> 1) + l / 32) .. + 16
  //   V block 2 dblk + h (h = 0, 1): lane l gets V^T row dblk * 32 + l % 32, bytes 16 (2 (l / 32) + h) .. + 16
  //     of the tile (the two halves of the lane's P.V A operand)
  // LDS DMA: with HD = 128 wave w fills block w of the K tile and block w of the V tile (two DMAs per wave
  // and tile); with HD = 64 the tiles have four blocks each, waves 0-3 fill the K blocks and waves 4-7 the
  // V blocks (one DMA per wave and tile).
  constexpr int kDmaPerTile = HD == 128 ? 2 : 1;
  const int8_t* kbase = p.k8 + b * p.ksb + hk * p.ksh;
  const uint8_t* vbase = static_cast<const uint8_t*>(p.v) + (b * p.Hkv + hk) * (int64_t)HD * p.Lpad;
  const int64_t kbytes = (p.Lk - 1) * p.ksl + HD;
  const v4u vrsrc = make_rsrc(vbase, (uint32_t)((int64_t)HD * p.Lpad));
  const int wu = __builtin_amdgcn_readfirstlane(w);
  const int kblk = HD == 128 ? wu : wu & 3;  // the K block and V block this wave fills
  uint32_t koff, voff;
  {
    const int kr = (kblk & 1) * 32 + lq, kc = 2 * (kblk >> 1) + hf;
    koff = (uint32_t)(kr * p.ksl + kc * 16);
    const int vd = (kblk >> 1) * 32 + lq, vc = 2 * hf + (kblk & 1);
    voff = (uint32_t)(vd * p.Lpad + vc * 16);
  }
  const int64_t k_step = kBK * p.ksl;
  const uint32_t lds_k0 = lds_addr(&lds_k[0][0]) + kblk * 1024;
  const uint32_t lds_v0 = lds_addr(&lds_v[0][0]) + kblk * 1024;
  const bool dma_k = HD == 128 || wu < 4, dma_v = HD == 128 || wu >= 4;
  auto dma_tile = [&](int t) {
    const int buf = buf_of(t);
    const int64_t kso = (int64_t)t * k_step;
    if (dma_k) lds_dma16(koff, make_rsrc(kbase + kso, (uint32_t)(kbytes - kso)), 0, lds_k0 + buf * (kBK * HD));
    if (dma_v) lds_dma16(voff, vrsrc, (uint32_t)t * kBK, lds_v0 + buf * (HD * kBK));
  };

  v16f o[NQF];
#pragma unroll
  for (int i = 0; i < NQF; i++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[i][r] = 0.f;
  float m_run = kMInit;
  v4f lacc = {0.f, 0.f, 0.f, 0.f};
  const v8i rs_sel = row_sum_selector();
  v16i kbias;
#pragma unroll
  for (int r = 0; r < 16; r++) kbias[r] = kAccBiasBits;

  if constexpr (QF == QF_INT8) __syncthreads();  // Q fragments are out of the LDS stage before the DMA reuses it
  // the key scales of tiles t_lo .. t_end - 1, from lds_ks[0]
  for (int i = tid; i < (t_end - t_lo) * KS; i += kPPThreads) lds_ks[i] = ks_ptr[k_scale_index(p, t_lo + i / KS, i % KS, KS)];
  if (tid < HD) {
    lds_vs[tid] = p.v_scale[(b * p.Hkv + hk) * HD + tid];
    lds_vm[tid] = p.v_mean ? p.v_mean[(b * p.Hkv + hk) * HD + tid] : 0.f;
  }
  for (int t = t_lo; t < min(t_end, t_lo + 2); t++) dma_tile(t);
  if constexpr (QF != QF_INT8) load_q();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();

  v16i s[2];
  v8i pf, vf[NQF];
  v4i kf[NKF];
  float cs_a, cs_b;  // logit scales of the tile in the softmax
  auto read_k = [&](int t) {
    const uint8_t* kb = &lds_k[buf_of(t)][lane * 16];
#pragma unroll
    for (int j = 0; j < NKF; j++) kf[j] = *reinterpret_cast<const v4i*>(kb + j * 1024);
  };
  auto read_cs = [&](int t) {
    if constexpr (KT) {
      cs_a = qs * lds_ks[(t - t_lo) * 4 + 2 * hf];
      cs_b = qs * lds_ks[(t - t_lo) * 4 + 2 * hf + 1];
    } else {
      cs_a = cs_b = qs * lds_ks[t - t_lo];
    }
  };
  auto read_v = [&](int t) {
    const uint8_t* vb = &lds_v[buf_of(t)][lane * 16];
#pragma unroll
    for (int dblk = 0; dblk < NQF; dblk++) {
      const v4i a0 = *reinterpret_cast<const v4i*>(vb + (2 * dblk) * 1024);
      const v4i a1 = *reinterpret_cast<const v4i*>(vb + (2 * dblk + 1) * 1024);
      vf[dblk] = v8i{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
    }
  };
  // stage M: P(t-1).V(t-1) and its row sum (operands from the previous stage V), then S^T(t) = K(t).Q^T
  auto pv = [&]() {
#pragma unroll
    for (int dblk = 0; dblk < NQF; dblk++)
      o[dblk] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf[dblk], pf, o[dblk], 0, 0, 0, 0, 0, 0);
    lacc = row_sum_mfma(lacc, pf, rs_sel);
  };
  auto qk = [&]() {
#pragma unroll
    for (int j = 0; j < NKF; j++) {
      const int m = j >> 1, kb = j & 1;
      s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf[j], qf[m], m == 0 ? kbias : s[kb], 0, 0, 0);
    }
  };
  auto stage_m = [&](int t, auto first_t) {
    constexpr bool kFirst = decltype(first_t)::value;
    if (!kFirst) read_v(t - 1);
    read_k(t);
    if (!kFirst) pv();
    qk();
    // the logit scales of the tile, for the softmax of the next stage
    read_cs(t);
    if constexpr (!kFirst && HD == 128) {
      // LDS reads three ahead of the MFMA that consumes them: 3 reads, then (1 MFMA, 2 reads) x 7,
      // then the remaining MFMAs (16 fragment reads + the key-scale read; 13 MFMAs with the row sum)
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
#pragma unroll
      for (int i = 0; i < 7; i++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, 6, 0);
    }
  };
  // stage V: V(t) fragments out of LDS (operands of the next stage M), mask, online softmax, P(t) to e4m3
  auto stage_v = [&](int t) {
    const int k0 = t * kBK;
    const bool masked = (k0 + kBK > kv_end_s) || (k0 + kBK - 1 > diag_s);
    if (masked) {
      int lim = max(min(kv_end_s - k0, kBK), -1);
      lim = min(lim, max(min(diag_s + lq + 1 - k0, kBK), -1));
      lim -= hf * 4;
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++)
          if (kb * 32 + (r >> 2) * 8 + (r & 3) >= lim) s[kb][r] = INT32_MIN;
    }
    float m_tile;
    if constexpr (!KT) {
      int mx = max(s[0][0], s[0][1]);
#pragma unroll
      for (int r = 2; r < 16; r++) mx = max(mx, s[0][r]);
#pragma unroll
      for (int r = 0; r < 16; r++) mx = max(mx, s[1][r]);
      const auto sw = __builtin_amdgcn_permlane32_swap(mx, mx, false, false);
      mx = max((int)sw[0], (int)sw[1]);
      m_tile = mx == INT32_MIN ? kMInit : fmaf(__int_as_float(mx), cs_a, -fmaf(kAccBias, cs_a, kFp8Offset - kLazyTau));
    } else {
      int ma = INT32_MIN, mb = INT32_MIN;
#pragma unroll
      for (int kb = 0; kb < 2; kb++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          if ((r & 3) < 2) ma = max(ma, s[kb][r]);
          else mb = max(mb, s[kb][r]);
        }
      const float fa = ma == INT32_MIN ? kMInit : fmaf(__int_as_float(ma), cs_a, -fmaf(kAccBias, cs_a, kFp8Offset - kLazyTau));
      const float fb = mb == INT32_MIN ? kMInit : fmaf(__int_as_float(mb), cs_b, -fmaf(kAccBias, cs_b, kFp8Offset - kLazyTau));
      const float mt = fmaxf(fa, fb);
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
      m_tile = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
    }
    const bool grow = m_tile > m_run + kLazyTau;
    if (__any(grow)) {
      const float m_new = grow ? m_tile : m_run;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
      for (int i = 0; i < NQF; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] *= alpha;
      row_sum_rescale(lacc, alpha);
      m_run = m_new;
    }
    // u = 8 (s * cs - m - kPLinShift) + 56 (p_e4m3_x4); masked logits give u = -1, P = 0
    const float cs8_a = 8.0f * cs_a, cs8_b = 8.0f * cs_b;
    const float nu_a = fmaf(-8.0f, fmaf(kAccBias, cs_a, m_run), kPLinBias);
    const float nu_b = fmaf(-8.0f, fmaf(kAccBias, cs_b, m_run), kPLinBias);
    auto body = [&](auto mk) {
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const int kb = j >> 2, r0 = (j & 3) * 4;
        float u[4];
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int sv = s[kb][r0 + e];
          u[e] = fmaf(__int_as_float(sv), e < 2 ? cs8_a : cs8_b, e < 2 ? nu_a : nu_b);
          if constexpr (decltype(mk)::value) u[e] = sv == INT32_MIN ? -1.f : u[e];
        }
        pf[j] = p_e4m3_x4(u[0], u[1], u[2], u[3]);
      }
    };
    if (masked) body(std::true_type{});
    else body(std::false_type{});
  };

  auto step = [&](int t, auto first_t) {
    const bool issue = t + 2 < t_end;
    if (issue) dma_tile(t + 2);
    // the matrix stage runs at raised wave priority: the vector-stage wave of the SIMD then cannot
    // delay the issue of its MFMAs (measured faster than equal priorities)
    __builtin_amdgcn_s_setprio(1);
    stage_m(t, first_t);
    __builtin_amdgcn_s_setprio(0);
    // this wave's share of tile t + 1 has landed (tile t + 2 may stay in flight)
    if (issue) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kDmaPerTile) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    pp_barrier();
    stage_v(t);
    pp_barrier();
  };
  if (grp == 1) pp_barrier();
  // the first tile has no P.V of a previous one: peeled, so the loop body has no branch on it
  if (t_lo < t_end) step(t_lo, std::true_type{});
  for (int t = t_lo + 1; t < t_end; t++) step(t, std::false_type{});
  if (grp == 0) pp_barrier();
  if (t_end > t_lo) {
    read_v(t_end - 1);
#pragma unroll
    for (int dblk = 0; dblk < NQF; dblk++)
      o[dblk] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf[dblk], pf, o[dblk], 0, 0, 0, 0, 0, 0);
    lacc = row_sum_mfma(lacc, pf, rs_sel);
  }

  const float l_tot = row_sum_value(lacc, lq);
  if constexpr (SPLIT) {
    // the split's partial (unnormalised O, m, l) for the combine kernel, in qattn_fwd_kernel's layout
    if (qrow >= p.Lq) return;
    const int64_t row = (((int64_t)split * p.B + b) * p.Hq + h) * p.Lq + qrow;
    float* wo = p.ws_o + row * HD;
#pragma unroll
    for (int dblk = 0; dblk < NQF; dblk++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int d = dblk * 32 + g * 8 + hf * 4;
        *reinterpret_cast<v4f*>(wo + d) = v4f{o[dblk][g * 4 + 0], o[dblk][g * 4 + 1], o[dblk][g * 4 + 2], o[dblk][g * 4 + 3]};
      }
    if (hf == 0) {
      p.ws_ml[row * 2 + 0] = m_run;
      p.ws_ml[row * 2 + 1] = l_tot;
    }
    return;
  }

  // ---- epilogue: O / l * v_scale out through the wave's LDS stage (the K buffers are idle now) ----
  const float inv_l = l_tot > 0.f ? 1.0f / l_tot : 0.f;
  uint16_t* obase = static_cast<uint16_t*>(p.o) + b * p.osb + h * p.osh;
  auto store = [&](auto mean_t) {
  constexpr bool kMean = decltype(mean_t)::value;
#pragma unroll
  for (int pass = 0; pass < HD / 64; pass++) {
#pragma unroll
    for (int db = 0; db < 2; db++) {
      const int dblk = pass * 2 + db;
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int d = dblk * 32 + g * 8 + hf * 4;
        const v4f sc = *reinterpret_cast<const v4f*>(&lds_vs[d]);
        float f[4];
        const v4f vm = kMean ? *reinterpret_cast<const v4f*>(&lds_vm[d]) : v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; e++) f[e] = epilogue_value<kMean>(o[dblk][g * 4 + e], inv_l, sc[e], vm[e]);
        const v2u packed{pack_half2<IS_FP16_OUT>(f[0], f[1]), pack_half2<IS_FP16_OUT>(f[2], f[3])};
        const int c = db * 4 + g;
        *reinterpret_cast<v2u*>(stage + lq * 128 + ((c ^ (lq & 7)) << 4) + hf * 8) = packed;
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = i * 8 + (lane >> 3), c = lane & 7;
      const v4u val = *reinterpret_cast<const v4u*>(stage + r * 128 + ((c ^ (r & 7)) << 4));
      const int64_t row = wrow0 + r;
      if (row < p.Lq) *reinterpret_cast<v4u*>(obase + row * p.osl + pass * 64 + c * 8) = val;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  };
  if (p.v_mean) store(std::true_type{});
  else store(std::false_type{});
  if (p.lse && hf == 0 && qrow < p.Lq)
    p.lse[(b * p.Hq + h) * p.Lq + qrow] = l_tot > 0.f ? __builtin_log2f(l_tot) + m_run : -INFINITY;
}

template <bool IS_FP16_OUT, bool KT, bool SPLIT, int HD = kD, int QF = QF_INT8>
__global__ __launch_bounds__(kPPThreads) void qattn_fwd_pp_kernel(AttnParams p) {
  qattn_fwd_pp<IS_FP16_OUT, KT, SPLIT, HD, QF>(p);
}

// ---- resident K/V: short key ranges (at most kResMaxTiles tiles, e.g. text cross-attention) ----
//
// The whole key range of a head (K int8 and e4m3 V, fragment-major as in the streaming kernels) is
// loaded into LDS once per workgroup; then each of the 12 waves walks its own 32-row query blocks over
// the resident tiles with no workgroup barrier at all: Q fragments come straight from global memory, the
// three waves of a SIMD drift apart freely so that one's softmax and Q loads overlap the others' MFMAs,
// and O leaves through a 2 KiB wave-private LDS stage as whole 64-byte row segments.  Twelve waves leave
// each 168 VGPRs: K and V fragments are read from LDS next to their MFMAs, and the next block's Q is not
// prefetched into registers (three waves per SIMD hide its latency better than two waves with prefetch:
// C4 0.63 -> 0.615 ms).  Per element the arithmetic is that of qattn_fwd_kernel
// (same MFMA chains, masking, lazy running max, FP8 offset, row sums on the matrix pipe), so the
// results are identical to it.
constexpr int kResMaxTiles = 8;
constexpr int kResThreads = 768;
constexpr int kResWaves = kResThreads / 64;

template <bool IS_FP16_OUT, bool KT, int QF = QF_INT8>
__global__ __launch_bounds__(kResThreads) void qattn_fwd_res_kernel(AttnParams p) {
  constexpr int KS = ks_per_tile(KT);
  constexpr int NW = kResThreads / 64;
  __shared__ __align__(16) uint8_t lds_k[kResMaxTiles][kBK * kD];
  __shared__ __align__(16) uint8_t lds_v[kResMaxTiles][kD * kBK];
  __shared__ __align__(16) uint8_t lds_o[NW][32 * 64];
  __shared__ __align__(16) uint8_t lds_pf[QF == QF_BLOCK ? NW : 1][256];  // landing slots of the Q prefetch, never read
  __shared__ float lds_ks[kResMaxTiles * 4];
  __shared__ __align__(16) float lds_vs[kD];
  __shared__ __align__(16) float lds_vm[kD];

  const int64_t wg = xcd_remap(blockIdx.x, gridDim.x);
  const int64_t chunk = wg % p.n_chunk;
  const int64_t h = (wg / p.n_chunk) % p.Hq;
  const int64_t b = wg / (p.n_chunk * p.Hq);
  const int64_t hk = h / p.group;
  const int tid = threadIdx.x;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, lq = lane & 31, hf = lane >> 5;
  const v8i rs_sel = row_sum_selector();

  // key range (wave-uniform, in scalar registers: kv_valid comes through a vector load)
  int64_t kv_lim = p.Lk;
  if (p.kv_valid) kv_lim = min(kv_lim, (int64_t)p.kv_valid[b]);
  const int64_t kv_end = __builtin_amdgcn_readfirstlane((int)max(kv_lim, (int64_t)0));
  const int n_tiles = (int)((kv_end + kBK - 1) / kBK);

  // ---- the key range into LDS: tile t of K / V in lds_k[t] / lds_v[t], fragment-major ----
  {
    const int8_t* kbase = p.k8 + b * p.ksb + hk * p.ksh;
    const uint8_t* vbase = static_cast<const uint8_t*>(p.v) + (b * p.Hkv + hk) * (int64_t)kD * p.Lpad;
    const int64_t kbytes = (p.Lk - 1) * p.ksl + kD;
    const v4u vrsrc = make_rsrc(vbase, (uint32_t)((int64_t)kD * p.Lpad));
    // per tile, wave w < 8 fills 1 KiB block w of the K tile and block w of the V tile (one DMA
    // instruction each), so waves 0-7 cover both tiles
    const int j = w;
    const uint32_t koff = (uint32_t)(((j & 1) * 32 + lq) * p.ksl + (2 * (j >> 1) + hf) * 16);
    const uint32_t voff = (uint32_t)(((j >> 1) * 32 + lq) * p.Lpad + (2 * hf + (j & 1)) * 16);
    const uint32_t lk0 = lds_addr(&lds_k[0][0]) + w * 1024, lv0 = lds_addr(&lds_v[0][0]) + w * 1024;
    if (w < 8) {
      for (int t = 0; t < n_tiles; t++) {
        const int64_t kso = (int64_t)t * kBK * p.ksl;
        const v4u krsrc = make_rsrc(kbase + kso, (uint32_t)(kbytes - kso));
        lds_dma16(koff, krsrc, 0, lk0 + t * (kBK * kD));
        lds_dma16(voff, vrsrc, (uint32_t)t * kBK, lv0 + t * (kD * kBK));
      }
    }
    const float* ks_ptr = p.k_scale + (b * p.Hkv + hk) * p.nKS;
    if (tid < n_tiles * KS) lds_ks[tid] = ks_ptr[k_scale_index(p, tid / KS, tid % KS, KS)];
    if (tid < kD) {
      lds_vs[tid] = p.v_scale[(b * p.Hkv + hk) * kD + tid];
      lds_vm[tid] = p.v_mean ? p.v_mean[(b * p.Hkv + hk) * kD + tid] : 0.f;
    }
  }

  // this wave's 32-row blocks: wb = wb0 + w, wb0 + w + NW, ... below wb_end
  const int64_t n_wb = (p.Lq + 31) / 32;
  const int64_t wb0 = chunk * p.wb_per_wg;
  const int64_t wb_end = min(n_wb, wb0 + p.wb_per_wg);
  const int8_t* qhead = p.q8 + b * p.qsb + h * p.qsh;
  const float* qs_tab = p.q_scale + (b * p.Hq + h) * p.nQS;
  // lane (lq, hf) holds bytes 32 m + 16 hf .. + 16 of query row lq (the MFMA B operand)
  auto load_q = [&](int64_t wb, v4i (&qf)[4]) {
    const int64_t row = wb * 32 + lq;
#pragma unroll
    for (int m = 0; m < 4; m++)
      qf[m] = row < p.Lq ? *reinterpret_cast<const v4i*>(qhead + row * p.qsl + m * 32 + hf * 16) : v4i{0, 0, 0, 0};
  };
  const uint16_t* qhead16 = reinterpret_cast<const uint16_t*>(p.q8) + b * p.qsb + h * p.qsh;
  v4i qf[4];
  int64_t wb = wb0 + w;
  v16i kbias;
#pragma unroll
  for (int r = 0; r < 16; r++) kbias[r] = kAccBiasBits;
  uint8_t* stage = &lds_o[w][0];
  uint16_t* obase = static_cast<uint16_t*>(p.o) + b * p.osb + h * p.osh;

  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();  // every wave's share of the key range has landed

  // per-block Q (QF_BLOCK): the layout starts every chunk on a 128-row block, so in each round waves 4 g ..
  // 4 g + 3 hold the four 32-row blocks of one Q block and exchange their maxima through LDS; every wave
  // runs all rounds of the chunk (a wave past the chunk's end takes zero rows, contributes 0 to the maxima,
  // joins the barrier and stores nothing)
  const int64_t wb_lim = QF == QF_BLOCK ? wb0 + (wb_end - wb0 + NW - 1) / NW * NW : wb_end;
  for (int rnd = 0; wb < wb_lim; rnd++, wb += NW) {
    const bool live = QF != QF_BLOCK || wb < wb_end;
    float qs;
    if constexpr (QF == QF_INT8) {
      load_q(wb, qf);
      qs = qs_tab[q_scale_index(p, wb * 32 + lq)] * p.qk_mult;
    } else if constexpr (QF == QF_BLOCK) {
      // (double-buffered by round: a wave writes round r + 2's maximum only after the barrier of round r + 1,
      // which every wave reaches after reading round r's)
      // (only the raw half words stay live across the barrier, and the values are formed again after it:
      // 64 fp32 values per lane would not fit beside the kernel's other registers)
      __shared__ float lds_qam[2][NW];
      const int64_t row = wb * 32 + lq;
      v4u raw[4][2];
      quant_q_raw<4>(qhead16 + row * p.qsl, live && row < p.Lq, hf, raw);
      float am_w;
      {
        float x[4][16];
        quant_q_unpack<IS_FP16_OUT, 4, true>(raw, p.q_sm_scale, x);
        am_w = quant_q_amax<QF, 4>(x);
      }
      if (lane == 0) lds_qam[rnd & 1][w] = am_w;
      __syncthreads();
      const float* g4 = &lds_qam[rnd & 1][w & ~3];
      const float am = fmaxf(fmaxf(g4[0], g4[1]), fmaxf(g4[2], g4[3]));
#pragma unroll
      for (int m = 0; m < 4; m++) asm volatile("" : "+v"(raw[m][0]), "+v"(raw[m][1]));  // (no reuse of the first unpack)
      float x[4][16];
      quant_q_unpack<IS_FP16_OUT, 4, true>(raw, p.q_sm_scale, x);
      qs = quant_q_codes<QF, 4>(x, am, qf) * p.qk_mult;
    } else {
      const int64_t row = wb * 32 + lq;
      qs = quant_q_rows<IS_FP16_OUT, QF, 4>(qhead16 + row * p.qsl, row < p.Lq, hf, qf) * p.qk_mult;
    }
    const int64_t wrow0 = wb * 32, qrow = wrow0 + lq;
    // Per block, the round barrier lines the waves up, so all of them would load their next Q rows at once
    // and wait out the HBM latency together: the wave's next 32 rows go into L2 while this block runs, one
    // dword of every 128-byte line (lane (lq, hf): row lq, line hf) DMA'd into the wave's landing slot so
    // that no register waits for it.  (The free-running forms stagger their loads by themselves: the
    // prefetch measured no gain there.)
    if constexpr (QF == QF_BLOCK) {
      if (wb + NW < wb_end) {
        constexpr int kQB = 2;  // bytes per Q element
        const int64_t nrow0 = (wb + NW) * 32;
        const uint8_t* nbase = reinterpret_cast<const uint8_t*>(p.q8) + (b * p.qsb + h * p.qsh + nrow0 * p.qsl) * kQB;
        const int64_t rem = ((p.Lq - 1 - nrow0) * p.qsl + kD) * kQB;  // bytes to the end of the last row
        lds_dma4((uint32_t)((lq * p.qsl + hf * 64) * kQB), make_rsrc(nbase, (uint32_t)min(rem, (int64_t)UINT32_MAX)), 0,
                 lds_addr(&lds_pf[w][0]));
      }
    }

    v16f o[4];
    v4f lacc;
    float m_run = kMInit;
    // One key tile.  The first tile of a block is peeled: its running max is the tile max and its P.V
    // starts from zero accumulators, which is what the general step computes there (the rescale factor
    // exp2(kMInit - m) is 0 while O and l are still 0, and a first tile always holds a valid key),
    // without zeroing O and l and without the O rescale.
    auto tile = [&](int t, auto first_t) {
      constexpr bool kFirst = decltype(first_t)::value;
      float cs_a, cs_b;
      if constexpr (KT) {
        cs_a = qs * lds_ks[t * 4 + 2 * hf];
        cs_b = qs * lds_ks[t * 4 + 2 * hf + 1];
      } else {
        cs_a = cs_b = qs * lds_ks[t];
      }
      v16i s[2];
      {
        __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int m = j >> 1, kb = j & 1;
          const v4i kf = *reinterpret_cast<const v4i*>(&lds_k[t][j * 1024 + lane * 16]);
          s[kb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf[m], m == 0 ? kbias : s[kb], 0, 0, 0);
        }
        __builtin_amdgcn_s_setprio(0);
      }
      const int64_t k0 = (int64_t)t * kBK;
      const bool masked = k0 + kBK > kv_end;
      // Masked logits become -inf (as int32 below every biased logit, so the max skips them), whose
      // exp2 is exactly 0: no per-logit select in the softmax.  A zero logit scale (an all-zero block
      // under the Triton rounding) would turn -inf into NaN there, so a wave with one falls back to
      // INT32_MIN and the select.
      bool select_mask = false;
      if (masked) {
        select_mask = !__all(cs_a > 0.f && cs_b > 0.f);
        const int mval = select_mask ? INT32_MIN : kMaskedLogitBits;
        int lim = (int)min(kv_end - k0, (int64_t)kBK) - hf * 4;
        asm volatile("" : "+v"(lim));  // (compared here, not as 32 lane masks kept in registers across the loops)
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
          for (int r = 0; r < 16; r++)
            if (kb * 32 + (r >> 2) * 8 + (r & 3) >= lim) s[kb][r] = mval;
      }
      auto all_masked = [](int x) { return x == INT32_MIN || x == kMaskedLogitBits; };
      float m_tile;
      if constexpr (!KT) {
        int mx = max(s[0][0], s[0][1]);
#pragma unroll
        for (int r = 2; r < 16; r++) mx = max(mx, s[0][r]);
#pragma unroll
        for (int r = 0; r < 16; r++) mx = max(mx, s[1][r]);
        const auto sw = __builtin_amdgcn_permlane32_swap(mx, mx, false, false);
        mx = max((int)sw[0], (int)sw[1]);
        m_tile = all_masked(mx) ? kMInit : fmaf(__int_as_float(mx), cs_a, -fmaf(kAccBias, cs_a, kFp8Offset - kLazyTau));
      } else {
        int ma = INT32_MIN, mb = INT32_MIN;
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            if ((r & 3) < 2) ma = max(ma, s[kb][r]);
            else mb = max(mb, s[kb][r]);
          }
        const float fa = all_masked(ma) ? kMInit : fmaf(__int_as_float(ma), cs_a, -fmaf(kAccBias, cs_a, kFp8Offset - kLazyTau));
        const float fb = all_masked(mb) ? kMInit : fmaf(__int_as_float(mb), cs_b, -fmaf(kAccBias, cs_b, kFp8Offset - kLazyTau));
        const float mt = fmaxf(fa, fb);
        const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mt), __float_as_uint(mt), false, false);
        m_tile = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
      }
      if constexpr (kFirst) {
        m_run = m_tile;
      } else {
        const bool grow = m_tile > m_run + kLazyTau;
        if (__any(grow)) {
          const float m_new = grow ? m_tile : m_run;
          const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
#pragma unroll
          for (int i = 0; i < 4; i++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[i][r] *= alpha;
          row_sum_rescale(lacc, alpha);
          m_run = m_new;
        }
      }
      // u = 8 (s * cs - m - kPLinShift) + 56 (p_e4m3_x4); masked logits give u = -1, P = 0
      const float cs8_a = 8.0f * cs_a, cs8_b = 8.0f * cs_b;
      const float nu_a = fmaf(-8.0f, fmaf(kAccBias, cs_a, m_run), kPLinBias);
      const float nu_b = fmaf(-8.0f, fmaf(kAccBias, cs_b, m_run), kPLinBias);
      v8i pf;
      auto body = [&](auto mk) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
          const int kb = j >> 2, r0 = (j & 3) * 4;
          float u[4];
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int sv = s[kb][r0 + e];
            u[e] = fmaf(__int_as_float(sv), e < 2 ? cs8_a : cs8_b, e < 2 ? nu_a : nu_b);
            if constexpr (decltype(mk)::value) u[e] = sv == INT32_MIN ? -1.f : u[e];
          }
          pf[j] = p_e4m3_x4(u[0], u[1], u[2], u[3]);
        }
      };
      if (select_mask) body(std::true_type{});
      else body(std::false_type{});
      const v16f zero = {};
#pragma unroll
      for (int dblk = 0; dblk < 4; dblk++) {
        const v4i a0 = *reinterpret_cast<const v4i*>(&lds_v[t][(2 * dblk) * 1024 + lane * 16]);
        const v4i a1 = *reinterpret_cast<const v4i*>(&lds_v[t][(2 * dblk + 1) * 1024 + lane * 16]);
        const v8i vf = v8i{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
        o[dblk] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pf, kFirst ? zero : o[dblk], 0, 0, 0, 0, 0, 0);
      }
      lacc = row_sum_mfma(kFirst ? v4f{0.f, 0.f, 0.f, 0.f} : lacc, pf, rs_sel);
    };
    if (n_tiles > 0) {
      tile(0, std::true_type{});
      for (int t = 1; t < n_tiles; t++) tile(t, std::false_type{});
    } else {
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[i][r] = 0.f;
      lacc = v4f{0.f, 0.f, 0.f, 0.f};
    }

    // ---- epilogue: O / l * v_scale (+ v_mean), 32 channels per pass through the 2 KiB stage ----
    const float l_tot = row_sum_value(lacc, lq);
    const float inv_l = l_tot > 0.f ? 1.0f / l_tot : 0.f;
    auto store = [&](auto mean_t) {
    constexpr bool kMean = decltype(mean_t)::value;
#pragma unroll
    for (int dblk = 0; dblk < 4; dblk++) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int d = dblk * 32 + g * 8 + hf * 4;
        const v4f sc = *reinterpret_cast<const v4f*>(&lds_vs[d]);
        const v4f vm = kMean ? *reinterpret_cast<const v4f*>(&lds_vm[d]) : v4f{0.f, 0.f, 0.f, 0.f};
        float f[4];
#pragma unroll
        for (int e = 0; e < 4; e++) f[e] = epilogue_value<kMean>(o[dblk][g * 4 + e], inv_l, sc[e], vm[e]);
        const v2u packed{pack_half2<IS_FP16_OUT>(f[0], f[1]), pack_half2<IS_FP16_OUT>(f[2], f[3])};
        // stage row lq: 4 chunks of 16 B (8 channels), chunk g stored at g ^ (lq & 3)
        *reinterpret_cast<v2u*>(stage + lq * 64 + ((g ^ (lq & 3)) << 4) + hf * 8) = packed;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const int id = i * 64 + lane, r = id >> 2, c = id & 3;
        const v4u val = *reinterpret_cast<const v4u*>(stage + r * 64 + ((c ^ (r & 3)) << 4));
        const int64_t row = wrow0 + r;
        if (live && row < p.Lq) *reinterpret_cast<v4u*>(obase + row * p.osl + dblk * 32 + c * 8) = val;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    };
    if (p.v_mean) store(std::true_type{});
    else store(std::false_type{});
    if (p.lse && hf == 0 && live && qrow < p.Lq)
      p.lse[(b * p.Hq + h) * p.Lq + qrow] = l_tot > 0.f ? __builtin_log2f(l_tot) + m_run : -INFINITY;
  }
  if constexpr (QF == QF_BLOCK) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no prefetch left in flight
}

// Merge the KV-split partials: one wave per query row, 2 channels per lane.
template <bool IS_FP16_OUT, int HD = kD>
__global__ __launch_bounds__(256) void qattn_combine_kernel(AttnParams p) {
  constexpr int E = HD / 64;  // output elements per lane
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);  // over B*Hq*Lq
  const int lane = threadIdx.x & 63;
  const int64_t total = p.B * p.Hq * p.Lq;
  if (row >= total) return;
  const int64_t qrow = row % p.Lq;
  const int64_t h = (row / p.Lq) % p.Hq;
  const int64_t b = row / (p.Lq * p.Hq);
  const int64_t hk = h / p.group;
  const int64_t sstride = total;
  float M = kMInit;
  for (int s = 0; s < p.nsplit; s++) M = fmaxf(M, p.ws_ml[(s * sstride + row) * 2]);
  float L = 0.f, a[E];
#pragma unroll
  for (int e = 0; e < E; e++) a[e] = 0.f;
  for (int s = 0; s < p.nsplit; s++) {
    const float ms = p.ws_ml[(s * sstride + row) * 2], ls = p.ws_ml[(s * sstride + row) * 2 + 1];
    const float f = __builtin_amdgcn_exp2f(ms - M);
    L += ls * f;
    const float* wo = p.ws_o + (s * sstride + row) * HD + lane * E;
#pragma unroll
    for (int e = 0; e < E; e++) a[e] += wo[e] * f;
  }
  const float inv = L > 0.f ? 1.0f / L : 0.f;
  const float* vs = p.v_scale ? p.v_scale + (b * p.Hkv + hk) * HD + lane * E : nullptr;
  uint16_t* orow = static_cast<uint16_t*>(p.o) + b * p.osb + qrow * p.osl + h * p.osh + lane * E;
  const float* vm = p.v_mean ? p.v_mean + (b * p.Hkv + hk) * HD + lane * E : nullptr;
#pragma unroll
  for (int e = 0; e < E; e++) {
    const float r = vm ? epilogue_value<true>(a[e], inv, vs ? vs[e] : 1.f, vm[e])
                       : epilogue_value<false>(a[e], inv, vs ? vs[e] : 1.f, 0.f);
    orow[e] = f32_to_half<IS_FP16_OUT>(r);
  }
  if (p.lse && lane == 0) p.lse[(b * p.Hq + h) * p.Lq + qrow] = L > 0.f ? __builtin_log2f(L) + M : -INFINITY;
}

}  // namespace qattn

using namespace qattn;

static bool is_thread_gran(int g) { return g == QATTN_GRAN_THREAD || g == QATTN_GRAN_THREAD_SM90; }

// key tiles one workgroup can cover (its k_scales are staged in LDS)
static int64_t max_tiles_per_split(int pv, bool kt) {
  const int floats = pv == PV_FP8 ? ks_lds_floats<PV_FP8>() : ks_lds_floats<PV_BF16>();
  return floats / ks_per_tile(kt);
}

// Ping-pong KV-split launches take whole pairs of query blocks; an odd block count leaves the last pair's
// second wave group idle, allowed when that is at most 1/6 of the groups.
static bool pp_split_fits(int64_t nqb) { return nqb % 2 == 0 || nqb >= 5; }

static int num_splits_for(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int64_t max_tiles, bool pp) {
  const int64_t nqb = (Lq + kBQ - 1) / kBQ;
  const int64_t wgs = B * Hq * nqb;
  const int64_t nkb = (Lk + kBK - 1) / kBK;
  if (wgs <= 0 || nkb <= 0) return 1;
  // 256 CUs x 2 resident workgroups.  Split only when the grid leaves CUs without any workgroup: at
  // 256 or more workgroups the combine traffic of a split costs more than the idle half-slots it fills
  // (C5, 444 workgroups: 0.63 ms unsplit against 0.79 ms with 3 splits); every split still gets at least
  // 8 key tiles
  const int64_t target = 1024;
  const int64_t min_s = (nkb + max_tiles - 1) / max_tiles;
  if (wgs >= target / 4) return (int)min_s;
  if (pp && pp_split_fits(nqb)) {
    // FP8 dense launches: splits for one round of at most 256 ping-pong workgroups (one per CU).  Against
    // the earlier count (about 1024 one-block workgroups) 5-27 % faster at 512-4680 queries over 8k-32k keys,
    // with either kernel (fewer splits, less combine traffic)
    const int64_t pairs = B * Hq * ((nqb + 1) / 2);
    const int64_t s = std::min<int64_t>(std::min<int64_t>(256 / pairs, nkb / 8), 32);
    return (int)std::max<int64_t>(min_s, std::max<int64_t>(s, 1));
  }
  int64_t s = (target + wgs - 1) / wgs;
  s = std::min<int64_t>(s, nkb / 8);
  return (int)std::max<int64_t>(min_s, std::min<int64_t>(s, 32));
}

extern "C" int qattn_fwd_num_splits(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq) {
  return num_splits_for(B, Lq, Lk, Hq, max_tiles_per_split(PV_FP8, false), true);
}

extern "C" int qattn_fwd_ex_num_splits(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int v_kind, int qk_quant_gran) {
  return num_splits_for(B, Lq, Lk, Hq, max_tiles_per_split(v_kind, is_thread_gran(qk_quant_gran)),
                        v_kind == QATTN_V_FP8);
}

static int blocks_per_workgroup(int64_t bh, int64_t nqb, int64_t nkb);

extern "C" int qattn_fwd_ex_blocks_per_workgroup(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int v_kind,
                                                 int qk_quant_gran, int causal) {
  if (v_kind != QATTN_V_FP8 || causal || B <= 0 || Lq <= 0 || Lk <= 0 || Hq <= 0) return 1;
  const int64_t nkb = (Lk + kBK - 1) / kBK, nqb = (Lq + kBQ - 1) / kBQ;
  if (nkb >= kMqAutoMaxTiles) return 1;
  if (num_splits_for(B, Lq, Lk, Hq, max_tiles_per_split(PV_FP8, is_thread_gran(qk_quant_gran)), true) != 1)
    return 1;
  return blocks_per_workgroup(B * Hq, nqb, nkb);
}

extern "C" size_t qattn_fwd_workspace_size(int64_t B, int64_t Lq, int64_t Hq, int64_t D, int num_splits) {
  if (num_splits <= 1) return 0;
  return (size_t)num_splits * B * Hq * Lq * (D + 2) * sizeof(float);
}

// Kernel selection.  Dense FP8 launches without a KV split run the ping-pong kernel when its grid (one
// workgroup per two query blocks, one workgroup per CU) fills the 256 CUs, the multi-block variant of
// qattn_fwd_kernel for short key ranges (blocks_per_workgroup > 1), and qattn_fwd_kernel otherwise;
// split, half-P.V and block-sparse launches always run qattn_fwd_kernel.  A thread-local override
// (qattn_set_kernel) forces one of the applicable kernels, so tests can compare them on small shapes.
static thread_local int t_kernel_override = QATTN_KERNEL_AUTO;
static thread_local int t_last_kernel = QATTN_KERNEL_AUTO;

extern "C" int qattn_set_kernel(int kernel) {
  const int prev = t_kernel_override;
  if (kernel >= QATTN_KERNEL_AUTO && kernel <= QATTN_KERNEL_RESIDENT) t_kernel_override = kernel;
  return prev;
}

extern "C" int qattn_last_kernel(void) { return t_last_kernel; }

// the kernel a launch runs, given its split count and whether the multi-block / resident layouts apply
static int pick_kernel(int pv, bool sparse, int ns, int causal, int64_t B, int64_t Hq, int64_t nQB, int qpw_auto,
                       bool mq_ok, bool res_ok) {
  if (pv != PV_FP8 || sparse) return QATTN_KERNEL_ONE_BLOCK;
  const int ov = t_kernel_override;
  // KV-split launches: the ping-pong kernel when its grid of pairs x splits is one round of 128 to 256
  // workgroups over whole pairs (the split count the automatic rule picks for it: 3-5 % faster than the
  // one-block kernel with the same splits), else the one-block kernel (also for tiny grids such as C1's
  // 16 ping-pong workgroups, where its 32 run 1 us faster)
  if (ns > 1) {
    if (ov == QATTN_KERNEL_PINGPONG) return QATTN_KERNEL_PINGPONG;
    const int64_t g = B * Hq * ((nQB + 1) / 2) * ns;
    const bool pp = ov == QATTN_KERNEL_AUTO && pp_split_fits(nQB) && g >= 128 && g <= 256;
    return pp ? QATTN_KERNEL_PINGPONG : QATTN_KERNEL_ONE_BLOCK;
  }
  if (ov == QATTN_KERNEL_PINGPONG || ov == QATTN_KERNEL_ONE_BLOCK) return ov;
  if (ov == QATTN_KERNEL_MULTI_BLOCK && mq_ok && !causal) return QATTN_KERNEL_MULTI_BLOCK;
  if (ov == QATTN_KERNEL_RESIDENT && res_ok) return QATTN_KERNEL_RESIDENT;
  if (res_ok) return QATTN_KERNEL_RESIDENT;
  if (qpw_auto > 1) return QATTN_KERNEL_MULTI_BLOCK;
  // The ping-pong kernel (one workgroup of two 128-row query blocks per CU) against one-block workgroups
  // (one query block, two per CU), in rounds of the 256 CUs: a ping-pong round takes about T (one pair
  // over the whole key range), a full round of one-block workgroups ~1.1 T (C2: 3.9 against 3.45 ms for
  // the same rounds), a last round with a single one-block workgroup on a CU ~0.9 T (one wave per SIMD:
  // 0.454 against 0.512 ms at 2048 x 32760 x 12).  At the C5 chunk shape with 8, 10, 11 and 12 heads (152
  // to 228 pairs) the ping-pong grid is 4-9 % faster.
  const int64_t pairs = B * Hq * ((nQB + 1) / 2), blocks = B * Hq * nQB;
  const double pp_cost = (double)((pairs + 255) / 256);
  const int64_t rem = blocks % 512;
  const double ob_cost = (double)(blocks / 512) * 1.1 + (rem == 0 ? 0.0 : rem > 256 ? 1.1 : 0.9);
  return pp_cost <= ob_cost ? QATTN_KERNEL_PINGPONG : QATTN_KERNEL_ONE_BLOCK;
}

// Resident-K/V launches: the 32-row wave blocks of each (batch, head) are cut into n_chunk workgroups
// of wb_per_wg blocks.  One workgroup runs per CU (its LDS holds the key range), its kResWaves waves each
// taking every kResWaves-th block; the cut minimises full rounds of 256 workgroups x (wave rounds per
// workgroup + one round of start-up for the key-range load).
static void resident_layout(int64_t bh, int64_t n_wb, int64_t& wb_per_wg, int64_t& n_chunk, int64_t align = 1) {
  double best = 1e300;
  wb_per_wg = (n_wb + align - 1) / align * align;
  n_chunk = 1;
  for (int64_t c = 1; c <= std::max<int64_t>(1, (n_wb + kResWaves - 1) / kResWaves); c++) {
    const int64_t per = ((n_wb + c - 1) / c + align - 1) / align * align;
    const int64_t chunks = (n_wb + per - 1) / per;
    const int64_t rounds = (bh * chunks + 255) / 256;
    const double cost = (double)rounds * (double)((per + kResWaves - 1) / kResWaves + 1);
    if (cost < best) {
      best = cost;
      wb_per_wg = per;
      n_chunk = chunks;
    }
  }
}

template <int PV, bool KT, bool SP = false>
static int launch_fwd(AttnParams& p, int out_dtype, int ns, void* workspace, size_t workspace_bytes, hipStream_t st,
                      int64_t D, int kernel) {
  t_last_kernel = kernel;
  if constexpr (PV == PV_FP8 && !SP) {
    if (kernel == QATTN_KERNEL_MULTI_BLOCK) {
      p.nsplit = 1;
      p.tiles_per_split = (int)p.nKB;
      p.nQC = (p.nQB + p.qpw - 1) / p.qpw;
      const int64_t g = p.B * p.Hq * p.nQC;
      QATTN_REQUIRE(g < (1ll << 31), QATTN_ERR_SHAPE, "grid too large");
      if (out_dtype == QATTN_BF16) qattn_fwd_kernel<false, false, PV, KT, false, true><<<g, kThreads, 0, st>>>(p);
      else qattn_fwd_kernel<true, false, PV, KT, false, true><<<g, kThreads, 0, st>>>(p);
      return check_launch("qattn_fwd");
    }
    if (kernel == QATTN_KERNEL_RESIDENT) {
      p.nsplit = 1;
      p.tiles_per_split = (int)p.nKB;
      resident_layout(p.B * p.Hq, (p.Lq + 31) / 32, p.wb_per_wg, p.n_chunk);
      const int64_t g = p.B * p.Hq * p.n_chunk;
      QATTN_REQUIRE(g < (1ll << 31), QATTN_ERR_SHAPE, "grid too large");
      if (out_dtype == QATTN_BF16) qattn_fwd_res_kernel<false, KT><<<g, kResThreads, 0, st>>>(p);
      else qattn_fwd_res_kernel<true, KT><<<g, kResThreads, 0, st>>>(p);
      return check_launch("qattn_fwd");
    }
    if (kernel == QATTN_KERNEL_PINGPONG) {
      const int64_t g = p.B * p.Hq * ((p.nQB + 1) / 2) * ns;
      QATTN_REQUIRE(g < (1ll << 31), QATTN_ERR_SHAPE, "grid too large");
      p.nsplit = ns;
      p.tiles_per_split = (int)((p.nKB + ns - 1) / ns);
      if (ns > 1) {
        QATTN_REQUIRE(workspace && workspace_bytes >= qattn_fwd_workspace_size(p.B, p.Lq, p.Hq, D, ns),
                      QATTN_ERR_WORKSPACE, "qattn_fwd with %d KV splits needs %zu workspace bytes", ns,
                      qattn_fwd_workspace_size(p.B, p.Lq, p.Hq, D, ns));
        p.ws_o = static_cast<float*>(workspace);
        p.ws_ml = p.ws_o + (int64_t)ns * p.B * p.Hq * p.Lq * D;
        const int64_t rows = p.B * p.Hq * p.Lq;
        if (D == 64) {
          if (out_dtype == QATTN_BF16) qattn_fwd_pp_kernel<false, KT, true, 64><<<g, kPPThreads, 0, st>>>(p);
          else qattn_fwd_pp_kernel<true, KT, true, 64><<<g, kPPThreads, 0, st>>>(p);
          if (out_dtype == QATTN_BF16) qattn_combine_kernel<false, 64><<<(rows + 3) / 4, 256, 0, st>>>(p);
          else qattn_combine_kernel<true, 64><<<(rows + 3) / 4, 256, 0, st>>>(p);
        } else {
          if (out_dtype == QATTN_BF16) qattn_fwd_pp_kernel<false, KT, true><<<g, kPPThreads, 0, st>>>(p);
          else qattn_fwd_pp_kernel<true, KT, true><<<g, kPPThreads, 0, st>>>(p);
          if (out_dtype == QATTN_BF16) qattn_combine_kernel<false><<<(rows + 3) / 4, 256, 0, st>>>(p);
          else qattn_combine_kernel<true><<<(rows + 3) / 4, 256, 0, st>>>(p);
        }
      } else if (D == 64) {
        if (out_dtype == QATTN_BF16) qattn_fwd_pp_kernel<false, KT, false, 64><<<g, kPPThreads, 0, st>>>(p);
        else qattn_fwd_pp_kernel<true, KT, false, 64><<<g, kPPThreads, 0, st>>>(p);
      } else {
        if (out_dtype == QATTN_BF16) qattn_fwd_pp_kernel<false, KT, false><<<g, kPPThreads, 0, st>>>(p);
        else qattn_fwd_pp_kernel<true, KT, false><<<g, kPPThreads, 0, st>>>(p);
      }
      return check_launch("qattn_fwd");
    }
  }
  const int64_t grid = p.B * p.Hq * p.nQB * ns;
  QATTN_REQUIRE(grid < (1ll << 31), QATTN_ERR_SHAPE, "grid too large");
  p.nsplit = ns;
  p.tiles_per_split = (int)((p.nKB + ns - 1) / ns);
  if (ns > 1) {
    QATTN_REQUIRE(workspace && workspace_bytes >= qattn_fwd_workspace_size(p.B, p.Lq, p.Hq, D, ns), QATTN_ERR_WORKSPACE,
                  "qattn_fwd with %d KV splits needs %zu workspace bytes", ns,
                  qattn_fwd_workspace_size(p.B, p.Lq, p.Hq, D, ns));
    p.ws_o = static_cast<float*>(workspace);
    p.ws_ml = p.ws_o + (int64_t)ns * p.B * p.Hq * p.Lq * D;
    if (out_dtype == QATTN_BF16) qattn_fwd_kernel<false, true, PV, KT, SP><<<grid, kThreads, 0, st>>>(p);
    else qattn_fwd_kernel<true, true, PV, KT, SP><<<grid, kThreads, 0, st>>>(p);
    const int64_t rows = p.B * p.Hq * p.Lq;
    if (out_dtype == QATTN_BF16) qattn_combine_kernel<false><<<(rows + 3) / 4, 256, 0, st>>>(p);
    else qattn_combine_kernel<true><<<(rows + 3) / 4, 256, 0, st>>>(p);
  } else {
    if (out_dtype == QATTN_BF16) qattn_fwd_kernel<false, false, PV, KT, SP><<<grid, kThreads, 0, st>>>(p);
    else qattn_fwd_kernel<true, false, PV, KT, SP><<<grid, kThreads, 0, st>>>(p);
  }
  return check_launch("qattn_fwd");
}

// Short key ranges: one workgroup streams several query blocks of a head through one K/V pipeline, so
// the per-workgroup start-up (Q load, scale staging, first DMA round trip) and the epilogue overlap the
// next block's work.  Picks the blocks per workgroup that minimise the modelled makespan: full rounds
// of 512 resident workgroups (256 CUs x 2), each block costing its key tiles plus about one tile of
// epilogue, each workgroup about four tiles of start-up.
static int blocks_per_workgroup(int64_t bh, int64_t nqb, int64_t nkb) {
  int best = 1;
  double best_cost = 1e300;
  for (int64_t q = 1; q <= std::min<int64_t>(nqb, kMqMaxBlocks); q++) {
    const int64_t wgs = bh * ((nqb + q - 1) / q);
    const int64_t rounds = (wgs + 511) / 512;
    const double cost = (double)rounds * (double)(q * (nkb + 1) + 4);
    if (cost < best_cost) {
      best_cost = cost;
      best = (int)q;
    }
  }
  return best;
}

// Split count, query blocks per workgroup and kernel of a launch (rows of 128 queries, tiles of 64 keys).
static void plan_fwd(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int pv, int gran, int causal, bool sparse,
                     int num_splits, int& ns, int& qpw, int& kernel) {
  const int64_t nQB = (Lq + kBQ - 1) / kBQ, nKB = (Lk + kBK - 1) / kBK;
  const int64_t max_tiles = sparse ? kSpMaxTiles : max_tiles_per_split(pv, is_thread_gran(gran));
  ns = num_splits > 0 ? num_splits : num_splits_for(B, Lq, Lk, Hq, max_tiles, pv == PV_FP8 && !sparse);
  ns = (int)std::min<int64_t>(ns, nKB);
  if (ns < 1) ns = 1;
  // a workgroup stages the k_scales of at most max_tiles key tiles
  ns = (int)std::max<int64_t>(ns, (nKB + max_tiles - 1) / max_tiles);
  // (the multi-block kernel stages at most 32 q_scales per query block)
  const bool mq_ok = ns == 1 && !sparse && !causal && pv == PV_FP8 && nKB <= kMqMaxTiles &&
                     gran != QATTN_GRAN_THREAD_SM90;
  const bool res_ok = ns == 1 && !sparse && !causal && pv == PV_FP8 && nKB <= kResMaxTiles;
  const int qpw_mq = mq_ok ? blocks_per_workgroup(B * Hq, nQB, nKB) : 1;
  const int qpw_auto = nKB < kMqAutoMaxTiles ? qpw_mq : 1;
  kernel = pick_kernel(pv, sparse, ns, causal, B, Hq, nQB, qpw_auto, mq_ok, res_ok);
  qpw = kernel == QATTN_KERNEL_MULTI_BLOCK ? qpw_mq : 1;
}

extern "C" int qattn_fwd_ex_kernel(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int v_kind, int qk_quant_gran,
                                   int causal, int num_splits) {
  if (B <= 0 || Lq <= 0 || Lk <= 0 || Hq <= 0) return QATTN_KERNEL_AUTO;
  const int pv = v_kind == QATTN_V_FP8 ? PV_FP8 : v_kind == QATTN_V_BF16 ? PV_BF16 : PV_FP16;
  int ns, qpw, kernel;
  plan_fwd(B, Lq, Lk, Hq, pv, qk_quant_gran, causal, false, num_splits, ns, qpw, kernel);
  return kernel;
}

static int setup_fwd(AttnParams& p, int& ns, qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale,
                     const void* v, int64_t Lpad, qattn_seq o, int out_dtype, int64_t B, int64_t Lq, int64_t Lk,
                     int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int causal, int64_t q_offset,
                     const int32_t* kv_valid, float* lse, int num_splits, int pv, int gran, int& kernel,
                     bool sparse = false) {
  QATTN_REQUIRE(out_dtype == QATTN_BF16 || out_dtype == QATTN_FP16, QATTN_ERR_DTYPE, "out dtype must be bf16 or fp16");
  QATTN_REQUIRE(D == kD || (D == 64 && pv == PV_FP8 && !sparse), QATTN_ERR_HEAD_DIM,
                "qattn_fwd needs head_dim 128, or 64 with FP8 V on a dense launch (pad other heads), got %lld",
                (long long)D);
  QATTN_REQUIRE(gran >= QATTN_GRAN_BLOCK && gran <= QATTN_GRAN_THREAD_SM90, QATTN_ERR_ARG,
                "qk_quant_gran must be 1 (per block), 2 (per warp), 3 (per thread), 4 (per warp, sm90 tables) or "
                "5 (per thread, sm90 tables), got %d", gran);
  QATTN_REQUIRE(B >= 0 && Lq >= 0 && Lk >= 0 && Hq > 0 && Hkv > 0, QATTN_ERR_SHAPE, "bad sizes");
  QATTN_REQUIRE(Hq % Hkv == 0, QATTN_ERR_HEAD_RATIO, "num_qo_heads (%lld) must be divisible by num_kv_heads (%lld)",
                (long long)Hq, (long long)Hkv);
  if (B * Lq == 0) return -1;  // nothing to do
  QATTN_REQUIRE(Lk > 0, QATTN_ERR_SHAPE, "kv_len must be positive");
  QATTN_REQUIRE(Lpad % kBK == 0 && Lpad >= (Lk + kBK - 1) / kBK * kBK, QATTN_ERR_SHAPE,
                "Lpad must be a multiple of 64 covering kv_len");
  for (const qattn_seq* sq : {&q8, &k8}) {
    QATTN_REQUIRE(sq->data && aligned16(sq->data), QATTN_ERR_ALIGN, "q8/k8 must be 16-byte aligned");
    QATTN_REQUIRE(sq->sb % 16 == 0 && sq->sl % 16 == 0 && sq->sh % 16 == 0, QATTN_ERR_STRIDE,
                  "q8/k8 strides must be multiples of 16 bytes");
  }
  QATTN_REQUIRE(o.data && aligned16(o.data), QATTN_ERR_ALIGN, "output must be 16-byte aligned");
  QATTN_REQUIRE(o.sb % 8 == 0 && o.sl % 8 == 0 && o.sh % 8 == 0, QATTN_ERR_STRIDE,
                "output strides must be multiples of 16 bytes");
  QATTN_REQUIRE(v && aligned16(v) && q_scale && k_scale, QATTN_ERR_ARG, "null scale or V pointer");
  QATTN_REQUIRE(!causal || q_offset >= 0, QATTN_ERR_ARG, "q_offset must be >= 0");
  // the kernel addresses one (batch, kv head) of K and V through 32-bit buffer offsets
  QATTN_REQUIRE((Lk - 1) * k8.sl + D < (1ll << 32) && D * Lpad * 2 < (1ll << 32), QATTN_ERR_SHAPE,
                "K/V of one (batch, head) must span less than 4 GiB");

  p = AttnParams{};
  p.q8 = static_cast<const int8_t*>(q8.data);
  p.qsb = q8.sb; p.qsl = q8.sl; p.qsh = q8.sh;
  p.k8 = static_cast<const int8_t*>(k8.data);
  p.ksb = k8.sb; p.ksl = k8.sl; p.ksh = k8.sh;
  p.v = v; p.Lpad = Lpad;
  p.q_scale = q_scale; p.k_scale = k_scale;
  p.o = o.data; p.osb = o.sb; p.osl = o.sl; p.osh = o.sh;
  p.lse = lse; p.kv_valid = kv_valid;
  p.B = B; p.Lq = Lq; p.Lk = Lk; p.Hq = Hq; p.Hkv = Hkv;
  p.nQB = (Lq + kBQ - 1) / kBQ;
  p.nKB = (Lk + kBK - 1) / kBK;
  const bool sm90 = gran == QATTN_GRAN_WARP_SM90 || gran == QATTN_GRAN_THREAD_SM90;
  p.qgran = sm90 ? gran - 2 : gran;
  p.qrs = sm90 ? 4 : 5;
  p.kts = sm90 ? 1 : 0;
  if (sm90) {
    // 64-row Q blocks of four 16-row warps, 128-key K blocks
    const int64_t nq64 = (Lq + 63) / 64, nk128 = (Lk + 127) / 128;
    p.nQS = p.qgran == QATTN_GRAN_THREAD ? nq64 * 32 : nq64 * 4;
    p.nKS = p.qgran == QATTN_GRAN_THREAD ? nk128 * 4 : nk128;
  } else {
    p.nQS = gran == QATTN_GRAN_THREAD ? p.nQB * 32 : gran == QATTN_GRAN_WARP ? p.nQB * 4 : p.nQB;
    p.nKS = gran == QATTN_GRAN_THREAD ? p.nKB * 4 : p.nKB;
  }
  p.q_offset = q_offset;
  p.group = (int)(Hq / Hkv);
  p.causal = causal ? 1 : 0;
  p.qk_mult = qk_mult;

  plan_fwd(B, Lq, Lk, Hq, pv, gran, causal, sparse, num_splits, ns, p.qpw, kernel);
  if (D == 64) {
    // head_dim 64 runs the ping-pong kernel only (its unsplit and KV-split forms)
    QATTN_REQUIRE(t_kernel_override == QATTN_KERNEL_AUTO || t_kernel_override == QATTN_KERNEL_PINGPONG,
                  QATTN_ERR_HEAD_DIM, "head_dim 64 runs the ping-pong kernel only (kernel override %d)",
                  t_kernel_override);
    kernel = QATTN_KERNEL_PINGPONG;
    p.qpw = 1;
  }
  return QATTN_OK;
}

template <int PV>
static int launch_gran(AttnParams& p, int gran, int out_dtype, int ns, void* ws, size_t wsb, hipStream_t st,
                       int64_t D, int kernel) {
  if (is_thread_gran(gran)) return launch_fwd<PV, true>(p, out_dtype, ns, ws, wsb, st, D, kernel);
  return launch_fwd<PV, false>(p, out_dtype, ns, ws, wsb, st, D, kernel);
}

extern "C" int qattn_fwd_ex(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale, const void* v,
                            int v_kind, int64_t Lpad, const float* v_scale, qattn_seq o, int out_dtype, int64_t B,
                            int64_t Lq, int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, float qk_mult,
                            int qk_quant_gran, int causal, int64_t q_offset, const int32_t* kv_valid, float* lse,
                            int num_splits, void* workspace, size_t workspace_bytes, qattn_stream_t stream) {
  return qattn_fwd_ex2(q8, q_scale, k8, k_scale, v, v_kind, Lpad, v_scale, nullptr, o, out_dtype, B, Lq, Lk, Hq, Hkv,
                       D, qk_mult, qk_quant_gran, causal, q_offset, kv_valid, lse, num_splits, workspace,
                       workspace_bytes, stream);
}

extern "C" int qattn_fwd_ex2(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale, const void* v,
                             int v_kind, int64_t Lpad, const float* v_scale, const float* v_mean, qattn_seq o,
                             int out_dtype, int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D,
                             float qk_mult, int qk_quant_gran, int causal, int64_t q_offset, const int32_t* kv_valid,
                             float* lse, int num_splits, void* workspace, size_t workspace_bytes,
                             qattn_stream_t stream) {
  QATTN_REQUIRE(!v_mean || v_kind == QATTN_V_FP8, QATTN_ERR_ARG, "v_mean needs the FP8 V path");
  QATTN_REQUIRE(v_kind == QATTN_V_FP8 || v_kind == QATTN_V_BF16 || v_kind == QATTN_V_FP16, QATTN_ERR_DTYPE,
                "v_kind must be 0 (fp8), 1 (bf16) or 2 (fp16), got %d", v_kind);
  AttnParams p;
  int ns = 1, kernel = QATTN_KERNEL_AUTO;
  const int pv = v_kind == QATTN_V_FP8 ? PV_FP8 : v_kind == QATTN_V_BF16 ? PV_BF16 : PV_FP16;
  const int rc = setup_fwd(p, ns, q8, q_scale, k8, k_scale, v, Lpad, o, out_dtype, B, Lq, Lk, Hq, Hkv, D, qk_mult,
                           causal, q_offset, kv_valid, lse, num_splits, pv, qk_quant_gran, kernel);
  if (rc < 0) return QATTN_OK;
  if (rc) return rc;
  hipStream_t st = (hipStream_t)stream;
  if (pv == PV_FP8) {
    QATTN_REQUIRE(v_scale, QATTN_ERR_ARG, "v_scale is null");
    p.v_scale = v_scale;
    p.v_mean = v_mean;
    return launch_gran<PV_FP8>(p, qk_quant_gran, out_dtype, ns, workspace, workspace_bytes, st, D, kernel);
  }
  p.v_scale = nullptr;
  if (pv == PV_BF16) return launch_gran<PV_BF16>(p, qk_quant_gran, out_dtype, ns, workspace, workspace_bytes, st, D, kernel);
  return launch_gran<PV_FP16>(p, qk_quant_gran, out_dtype, ns, workspace, workspace_bytes, st, D, kernel);
}

// ---- half Q quantized inside the attention kernel (resident or ping-pong) ----
// the kernel a qattn_fwd_q16 launch runs: the automatic rule's, when it is one of the two with a fused-Q form
static int q16_kernel(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int64_t D, int gran, int causal) {
  if ((D != kD && D != 64) || B <= 0 || Lq <= 0 || Lk <= 0 || Hq <= 0) return QATTN_KERNEL_AUTO;
  if (D == 64) return QATTN_KERNEL_PINGPONG;  // (head_dim 64 runs the ping-pong kernel only)
  int ns, qpw, kernel;
  plan_fwd(B, Lq, Lk, Hq, PV_FP8, gran, causal, false, 0, ns, qpw, kernel);
  return kernel == QATTN_KERNEL_RESIDENT || kernel == QATTN_KERNEL_PINGPONG ? kernel : QATTN_KERNEL_AUTO;
}

extern "C" int qattn_fwd_q16_supported(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int64_t D, int qk_quant_gran,
                                       int causal) {
  if (qk_quant_gran < QATTN_GRAN_BLOCK || qk_quant_gran > QATTN_GRAN_THREAD) return 0;
  return q16_kernel(B, Lq, Lk, Hq, D, qk_quant_gran, causal) != QATTN_KERNEL_AUTO ? 1 : 0;
}

template <int QF, int HD>
static void launch_pp_q16(AttnParams& p, int dtype, int ns, hipStream_t st) {
  constexpr bool KT = QF == QF_THREAD;
  const int64_t g = p.B * p.Hq * ((p.nQB + 1) / 2) * ns;
  if (ns > 1) {
    const int64_t rows = p.B * p.Hq * p.Lq;
    if (dtype == QATTN_BF16) qattn_fwd_pp_kernel<false, KT, true, HD, QF><<<g, kPPThreads, 0, st>>>(p);
    else qattn_fwd_pp_kernel<true, KT, true, HD, QF><<<g, kPPThreads, 0, st>>>(p);
    if (dtype == QATTN_BF16) qattn_combine_kernel<false, HD><<<(rows + 3) / 4, 256, 0, st>>>(p);
    else qattn_combine_kernel<true, HD><<<(rows + 3) / 4, 256, 0, st>>>(p);
  } else {
    if (dtype == QATTN_BF16) qattn_fwd_pp_kernel<false, KT, false, HD, QF><<<g, kPPThreads, 0, st>>>(p);
    else qattn_fwd_pp_kernel<true, KT, false, HD, QF><<<g, kPPThreads, 0, st>>>(p);
  }
}
template <int QF>
static void launch_pp_q16(AttnParams& p, int dtype, int ns, hipStream_t st, int64_t D) {
  if (D == 64) launch_pp_q16<QF, 64>(p, dtype, ns, st);
  else launch_pp_q16<QF, kD>(p, dtype, ns, st);
}

extern "C" int qattn_fwd_q16(qattn_seq q, qattn_seq k8, const float* k_scale, const uint8_t* v8, int64_t Lpad,
                             const float* v_scale, const float* v_mean, qattn_seq o, int dtype, int64_t B,
                             int64_t Lq, int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, float qk_mult,
                             int qk_quant_gran, int causal, int64_t q_offset, const int32_t* kv_valid, float* lse,
                             int num_splits, void* workspace, size_t workspace_bytes, qattn_stream_t stream) {
  QATTN_REQUIRE(qk_quant_gran >= QATTN_GRAN_BLOCK && qk_quant_gran <= QATTN_GRAN_THREAD, QATTN_ERR_ARG,
                "qattn_fwd_q16 quantizes Q per block (1), per warp (2) or per thread (3), got %d", qk_quant_gran);
  QATTN_REQUIRE(v8 && v_scale, QATTN_ERR_ARG, "null V or v_scale");
  if (B * Lq == 0) return QATTN_OK;
  const int kernel = q16_kernel(B, Lq, Lk, Hq, D, qk_quant_gran, causal);
  QATTN_REQUIRE(kernel != QATTN_KERNEL_AUTO, QATTN_ERR_SHAPE,
                "qattn_fwd_q16 runs the resident or ping-pong kernel: head_dim 64, or 128 and a launch the automatic "
                "rule gives one of them (see qattn_fwd_q16_supported)");
  AttnParams p;
  int ns = 1, kplan = QATTN_KERNEL_AUTO;
  // (q's scale table is formed inside the kernel: k_scale stands in for the pointer setup_fwd checks)
  const int rc = setup_fwd(p, ns, q, k_scale, k8, k_scale, v8, Lpad, o, dtype, B, Lq, Lk, Hq, Hkv, D, qk_mult, causal,
                           q_offset, kv_valid, lse, num_splits, PV_FP8, qk_quant_gran, kplan);
  if (rc < 0) return QATTN_OK;
  if (rc) return rc;
  QATTN_REQUIRE(kplan == kernel, QATTN_ERR_ARG, "qattn_fwd_q16: num_splits %d moves the launch off its kernel",
                num_splits);
  p.v_scale = v_scale;
  p.v_mean = v_mean;
  if (qk_quant_gran == QATTN_GRAN_BLOCK) {
    // per-block scales carry sm_scale * log2(e): it is multiplied into Q, the logits take 1
    p.q_sm_scale = qk_mult;
    p.qk_mult = 1.0f;
  }
  hipStream_t st = (hipStream_t)stream;
  t_last_kernel = kernel;
  if (kernel == QATTN_KERNEL_RESIDENT) {
    p.nsplit = 1;
    p.tiles_per_split = (int)p.nKB;
    // (chunks of whole 128-row Q blocks for per-block scales)
    resident_layout(p.B * p.Hq, (p.Lq + 31) / 32, p.wb_per_wg, p.n_chunk, qk_quant_gran == QATTN_GRAN_BLOCK ? 4 : 1);
    const int64_t g = p.B * p.Hq * p.n_chunk;
    QATTN_REQUIRE(g < (1ll << 31), QATTN_ERR_SHAPE, "grid too large");
    if (qk_quant_gran == QATTN_GRAN_BLOCK) {
      if (dtype == QATTN_BF16) qattn_fwd_res_kernel<false, false, QF_BLOCK><<<g, kResThreads, 0, st>>>(p);
      else qattn_fwd_res_kernel<true, false, QF_BLOCK><<<g, kResThreads, 0, st>>>(p);
    } else if (qk_quant_gran == QATTN_GRAN_THREAD) {
      if (dtype == QATTN_BF16) qattn_fwd_res_kernel<false, true, QF_THREAD><<<g, kResThreads, 0, st>>>(p);
      else qattn_fwd_res_kernel<true, true, QF_THREAD><<<g, kResThreads, 0, st>>>(p);
    } else {
      if (dtype == QATTN_BF16) qattn_fwd_res_kernel<false, false, QF_WARP><<<g, kResThreads, 0, st>>>(p);
      else qattn_fwd_res_kernel<true, false, QF_WARP><<<g, kResThreads, 0, st>>>(p);
    }
    return check_launch("qattn_fwd_q16");
  }
  const int64_t g = p.B * p.Hq * ((p.nQB + 1) / 2) * ns;
  QATTN_REQUIRE(g < (1ll << 31), QATTN_ERR_SHAPE, "grid too large");
  p.nsplit = ns;
  p.tiles_per_split = (int)((p.nKB + ns - 1) / ns);
  if (ns > 1) {
    QATTN_REQUIRE(workspace && workspace_bytes >= qattn_fwd_workspace_size(p.B, p.Lq, p.Hq, D, ns),
                  QATTN_ERR_WORKSPACE, "qattn_fwd_q16 with %d KV splits needs %zu workspace bytes", ns,
                  qattn_fwd_workspace_size(p.B, p.Lq, p.Hq, D, ns));
    p.ws_o = static_cast<float*>(workspace);
    p.ws_ml = p.ws_o + (int64_t)ns * p.B * p.Hq * p.Lq * D;
  }
  if (qk_quant_gran == QATTN_GRAN_THREAD) launch_pp_q16<QF_THREAD>(p, dtype, ns, st, D);
  else if (qk_quant_gran == QATTN_GRAN_WARP) launch_pp_q16<QF_WARP>(p, dtype, ns, st, D);
  else launch_pp_q16<QF_BLOCK>(p, dtype, ns, st, D);
  return check_launch("qattn_fwd_q16");
}

// ---- packed variable-length batches ----
// One launch over every sequence of a packed batch (attn_qk_int8_block_varlen.py:68-155): the grid covers
// max_seqlen_q rows per sequence and head, and each workgroup reads its sequence's row range, scale
// offsets and V tile column from the device tables, so the host never reads cu_seqlens.
extern "C" int qattn_fwd_varlen(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale,
                                const uint16_t* v16, int64_t Lpad, qattn_seq o, int out_dtype, int64_t B,
                                int64_t total_q, int64_t total_k, int64_t max_lq, int64_t max_lk, int64_t Hq,
                                int64_t Hkv, int64_t D, float qk_mult,
                                int causal, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                const int32_t* cu_qs, const int32_t* cu_ks, const int32_t* cu_vt,
                                qattn_stream_t stream) {
  QATTN_REQUIRE(cu_seqlens_q && cu_seqlens_k && cu_qs && cu_ks && cu_vt, QATTN_ERR_ARG, "null sequence table");
  QATTN_REQUIRE(total_q >= 0 && total_k >= 0, QATTN_ERR_SHAPE, "negative packed size");
  AttnParams p;
  int ns = 1, kernel = QATTN_KERNEL_AUTO;
  const int rc = setup_fwd(p, ns, q8, q_scale, k8, k_scale, v16, Lpad, o, out_dtype, B, max_lq, max_lk, Hq, Hkv, D,
                           qk_mult, causal, 0, nullptr, nullptr, 1, PV_FP16, QATTN_GRAN_BLOCK, kernel);
  if (rc < 0) return QATTN_OK;
  if (rc) return rc;
  p.cu_q = cu_seqlens_q;
  p.cu_k = cu_seqlens_k;
  p.cu_qs = cu_qs;
  p.cu_ks = cu_ks;
  p.cu_vt = cu_vt;
  p.var_tq = total_q;
  p.var_tk = total_k;
  p.v_scale = nullptr;
  p.qpw = 1;
  return launch_fwd<PV_FP16, false>(p, out_dtype, 1, nullptr, 0, (hipStream_t)stream, D, QATTN_KERNEL_ONE_BLOCK);
}

// ---- allocation-free form of qattn_fwd_ex ----
// KV-split launches keep their partial (O, m, l) rows in this file-scope device array instead of a caller
// workspace.  Every GPU the library runs on holds its own copy for the life of the process; host code
// reaches it only through the address hipGetSymbolAddress returns on that device (the array's name is a
// host-side stand-in, not a device address).
constexpr size_t kScratchBytes = 128ull << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;  // guards the per-device tables and orders the scratch users (below)
static void* g_scratch_ptr[kMaxDevices];
// Completion of the last launch that used a device's scratch.  Each launch that uses the scratch first makes
// its stream wait for this event and then records it again, so launches from different streams (or threads)
// take the array one after the other in the order the host issued them (hipStreamWaitEvent is asynchronous:
// no host wait).  Created with the symbol lookup on the first call that needs the scratch on the device.
static hipEvent_t g_scratch_done[kMaxDevices];

// the scratch address and its ordering event on the calling thread's current device, set up once per device;
// the caller holds g_scratch_mu
static int scratch_on_current_device(void** out, int* dev_out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  QATTN_REQUIRE(e == hipSuccess && dev >= 0 && dev < kMaxDevices, QATTN_ERR_LAUNCH, "hipGetDevice failed: %s",
                hipGetErrorString(e));
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    QATTN_REQUIRE(e == hipSuccess && ptr, QATTN_ERR_LAUNCH, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(e));
    hipEvent_t ev = nullptr;
    e = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
    QATTN_REQUIRE(e == hipSuccess && ev, QATTN_ERR_LAUNCH, "hipEventCreate failed on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_done[dev] = ev;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  *dev_out = dev;
  return QATTN_OK;
}

extern "C" size_t qattn_fwd_noalloc_max_scratch(void) { return kScratchBytes; }

extern "C" int qattn_fwd_ex_noalloc(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale,
                                    const void* v, int v_kind, int64_t Lpad, const float* v_scale, qattn_seq o,
                                    int out_dtype, int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int64_t Hkv,
                                    int64_t D, float qk_mult, int qk_quant_gran, int causal, int64_t q_offset,
                                    const int32_t* kv_valid, float* lse, int num_splits, qattn_stream_t stream) {
  QATTN_REQUIRE(v_kind == QATTN_V_FP8 || v_kind == QATTN_V_BF16 || v_kind == QATTN_V_FP16, QATTN_ERR_DTYPE,
                "v_kind must be 0 (fp8), 1 (bf16) or 2 (fp16), got %d", v_kind);
  AttnParams p;
  int ns = 1, kernel = QATTN_KERNEL_AUTO;
  const int pv = v_kind == QATTN_V_FP8 ? PV_FP8 : v_kind == QATTN_V_BF16 ? PV_BF16 : PV_FP16;
  const int rc = setup_fwd(p, ns, q8, q_scale, k8, k_scale, v, Lpad, o, out_dtype, B, Lq, Lk, Hq, Hkv, D, qk_mult,
                           causal, q_offset, kv_valid, lse, num_splits, pv, qk_quant_gran, kernel);
  if (rc < 0) return QATTN_OK;
  if (rc) return rc;
  const size_t need = qattn_fwd_workspace_size(B, Lq, Hq, D, ns);
  QATTN_REQUIRE(need <= kScratchBytes, QATTN_ERR_WORKSPACE,
                "qattn_fwd_ex_noalloc: %d KV splits need %zu bytes of scratch, more than its %zu-byte limit "
                "(use qattn_fwd_ex with a workspace, or fewer splits)", ns, need, kScratchBytes);
  if (need == 0)  // no KV split: nothing of the scratch is used
    return qattn_fwd_ex(q8, q_scale, k8, k_scale, v, v_kind, Lpad, v_scale, o, out_dtype, B, Lq, Lk, Hq, Hkv, D,
                        qk_mult, qk_quant_gran, causal, q_offset, kv_valid, lse, ns, nullptr, 0, stream);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  void* ws = nullptr;
  int dev = -1;
  int e = scratch_on_current_device(&ws, &dev);
  if (e) return e;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // Order this launch after the previous scratch user on the device.  A stream under graph capture is left
  // to the graph's own order (waiting there on an event recorded outside the capture is not allowed):
  // replays of a captured graph must not overlap other users of the scratch.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t he = hipStreamIsCapturing(st, &cap);
  QATTN_REQUIRE(he == hipSuccess, QATTN_ERR_LAUNCH, "hipStreamIsCapturing failed: %s", hipGetErrorString(he));
  const bool order = cap == hipStreamCaptureStatusNone;
  if (order) {
    he = hipStreamWaitEvent(st, g_scratch_done[dev], 0);
    QATTN_REQUIRE(he == hipSuccess, QATTN_ERR_LAUNCH, "hipStreamWaitEvent failed: %s", hipGetErrorString(he));
  }
  // the same launch as qattn_fwd_ex with this split count and the device array as its workspace
  e = qattn_fwd_ex(q8, q_scale, k8, k_scale, v, v_kind, Lpad, v_scale, o, out_dtype, B, Lq, Lk, Hq, Hkv, D, qk_mult,
                   qk_quant_gran, causal, q_offset, kv_valid, lse, ns, ws, need, stream);
  if (e) return e;
  if (order) {
    he = hipEventRecord(g_scratch_done[dev], st);
    QATTN_REQUIRE(he == hipSuccess, QATTN_ERR_LAUNCH, "hipEventRecord failed: %s", hipGetErrorString(he));
  }
  return QATTN_OK;
}

extern "C" int qattn_fwd(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale, const uint8_t* v8,
                         int64_t Lpad, const float* v_scale, qattn_seq o, int out_dtype, int64_t B, int64_t Lq,
                         int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int causal,
                         int64_t q_offset, const int32_t* kv_valid, float* lse, int num_splits, void* workspace,
                         size_t workspace_bytes, qattn_stream_t stream) {
  return qattn_fwd_ex(q8, q_scale, k8, k_scale, v8, QATTN_V_FP8, Lpad, v_scale, o, out_dtype, B, Lq, Lk, Hq, Hkv, D,
                      qk_mult, QATTN_GRAN_BLOCK, causal, q_offset, kv_valid, lse, num_splits, workspace,
                      workspace_bytes, stream);
}

extern "C" int qattn_fwd_pv16(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale,
                              const uint16_t* v16, int v_dtype, int64_t Lpad, qattn_seq o, int out_dtype, int64_t B,
                              int64_t Lq, int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, float qk_mult, int causal,
                              int64_t q_offset, const int32_t* kv_valid, float* lse, int num_splits, void* workspace,
                              size_t workspace_bytes, qattn_stream_t stream) {
  QATTN_REQUIRE(v_dtype == QATTN_BF16 || v_dtype == QATTN_FP16, QATTN_ERR_DTYPE, "V dtype must be bf16 or fp16");
  return qattn_fwd_ex(q8, q_scale, k8, k_scale, v16, v_dtype == QATTN_BF16 ? QATTN_V_BF16 : QATTN_V_FP16, Lpad,
                      nullptr, o, out_dtype, B, Lq, Lk, Hq, Hkv, D, qk_mult, QATTN_GRAN_BLOCK, causal, q_offset,
                      kv_valid, lse, num_splits, workspace, workspace_bytes, stream);
}

extern "C" int qattn_fwd_block_sparse_num_splits(int64_t B, int64_t Lq, int64_t Lk, int64_t Hq) {
  return num_splits_for(B, Lq, Lk, Hq, kSpMaxTiles, false);
}

extern "C" int qattn_fwd_block_sparse(qattn_seq q8, const float* q_scale, qattn_seq k8, const float* k_scale,
                                      const uint16_t* v16, int v_dtype, int64_t Lpad, qattn_seq o, int out_dtype,
                                      int64_t B, int64_t Lq, int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D,
                                      float qk_mult, int causal, const int8_t* tile_mask, int64_t mask_sbh,
                                      int64_t mask_sq, float* lse, int num_splits, void* workspace,
                                      size_t workspace_bytes, qattn_stream_t stream) {
  QATTN_REQUIRE(v_dtype == QATTN_BF16 || v_dtype == QATTN_FP16, QATTN_ERR_DTYPE, "V dtype must be bf16 or fp16");
  QATTN_REQUIRE(tile_mask != nullptr, QATTN_ERR_ARG, "tile_mask is null");
  QATTN_REQUIRE(mask_sbh >= 0 && mask_sq >= 0, QATTN_ERR_STRIDE, "negative mask stride");
  AttnParams p;
  int ns = 1, kernel = QATTN_KERNEL_AUTO;
  const int pv = v_dtype == QATTN_BF16 ? PV_BF16 : PV_FP16;
  const int rc = setup_fwd(p, ns, q8, q_scale, k8, k_scale, v16, Lpad, o, out_dtype, B, Lq, Lk, Hq, Hkv, D, qk_mult,
                           causal, 0, nullptr, lse, num_splits, pv, QATTN_GRAN_BLOCK, kernel, true);
  if (rc < 0) return QATTN_OK;
  if (rc) return rc;
  p.v_scale = nullptr;
  p.tile_mask = tile_mask;
  p.tm_s1 = mask_sbh;
  p.tm_s2 = mask_sq;
  hipStream_t st = (hipStream_t)stream;
  if (pv == PV_BF16) return launch_fwd<PV_BF16, false, true>(p, out_dtype, ns, workspace, workspace_bytes, st, D, kernel);
  return launch_fwd<PV_FP16, false, true>(p, out_dtype, ns, workspace, workspace_bytes, st, D, kernel);
}
