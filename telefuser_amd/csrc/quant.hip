// Quantizers of the SageAttention-2 path, written for gfx950 (wave64, 16-byte vector loads):
//   * per-block INT8 quantization of Q and K (one launch for both), with optional K-mean smoothing
//     and sm_scale folding - semantics of QuantInt8Kernel (tf-kernel/csrc/sageattn2/fused/fused.cu:59-194)
//     or of the Triton quant_per_block_int8_kernel (tf-kernel/tf_kernel/triton/quant_per_block.py:22-71);
//   * the sequence mean of K used for smoothing (sageattn2.py:1329-1330);
//   * per-channel FP8 e4m3 quantization of V into the attention kernel's tile layout
//     (semantics of MeanScaleKernel, fused.cu:332-445, with scale_max = 448).
// All of them are HBM-bound streaming kernels: one pass over the input, coalesced row reads,
// reductions in registers + wave shuffles + a tiny LDS step.
#include "common.h"

namespace qattn {

// ------------------------------------------------------------------------------------------------
// per-block INT8 quantizer
// ------------------------------------------------------------------------------------------------

// Prologue of the Wan self-attention projections, applied on the fly to a 16-byte chunk (8 elements,
// 4 rotation pairs) of head h, row l of the linear output x:
//   RMSNorm over the full H*D row: y = half((x * rstd[b, l]) * w[h*D + d])  (norm_infer,
//     telefuser/kernel/triton/norm.py:469-507: x * rstd in fp32, times the weight, stored in x's dtype)
//   interleaved RoPE on the stored y: (y1, y2) -> half(fma(-y2, sin, y1*cos)), half(fma(y1, sin, y2*cos))
//     (telefuser/kernel/triton/rotary.py:21-88), cos/sin as fp32 per (row, pair)
// rstd == nullptr: no prologue (the chunk is used as loaded).
struct NormRope {
  const float* rstd;     // [B * L]
  const uint16_t* w;     // [H * D], x's dtype
  const float* cs;       // [L, D / 2] rows of cs_stride floats
  const float* sn;
  int64_t cs_stride;
};

template <bool IS_FP16>
__device__ __forceinline__ void norm_rope8(const NormRope& nr, int64_t b, int64_t L, int64_t l, int64_t h, int D,
                                           int dc, uint16_t (&hv)[8]) {
  const float r = nr.rstd[b * L + l];
  const v4u wr = *reinterpret_cast<const v4u*>(nr.w + h * D + dc * 8);
  uint16_t wv[8];
  __builtin_memcpy(wv, &wr, 16);
  const v4f c4 = *reinterpret_cast<const v4f*>(nr.cs + l * nr.cs_stride + dc * 4);
  const v4f s4 = *reinterpret_cast<const v4f*>(nr.sn + l * nr.cs_stride + dc * 4);
  float y[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float xr = half_to_f32<IS_FP16>(hv[e]) * r;
    y[e] = half_to_f32<IS_FP16>(f32_to_half<IS_FP16>(xr * half_to_f32<IS_FP16>(wv[e])));
  }
#pragma unroll
  for (int p = 0; p < 4; p++) {
    const float y1 = y[2 * p], y2 = y[2 * p + 1];
    const float a = y1 * c4[p], bb = y2 * c4[p];
    hv[2 * p] = f32_to_half<IS_FP16>(fmaf(-y2, s4[p], a));
    hv[2 * p + 1] = f32_to_half<IS_FP16>(fmaf(y1, s4[p], bb));
  }
}

// One quantizer job (Q or K).  A workgroup covers blk rows of one (batch entry, head): one scale block of
// the quantizer's block size (128, 64 or 32 rows), or, with nsub = 4, blk = 4 cr rows that are four cr-row
// scale blocks (the warp blocks of the per-warp / per-thread Q layouts: cr = 32, or 16 in the sm90 layout).
struct QuantJob {
  const uint16_t* in;
  int64_t sb, sl, sh;
  int8_t* out;
  int64_t ob, ol, oh;
  float* scale;  // [B, H, scale_blocks, ncls]
  const uint16_t* mean;  // [B, H, D] or null
  int64_t L, H;
  int64_t nblk;          // workgroup blocks per (batch entry, head)
  int64_t scale_blocks;  // scale blocks per (batch entry, head) in the scale tensor
  int blk, nsub;
  int cr;  // rows per scale cell of a grouped block (32 or 16), 0 for one scale per block
  int has_sm_scale;
  float sm_scale;
  int64_t nwg;  // B * H * nblk
  int ncls;     // scale classes per scale block: 1 (per block), 8 (per-thread Q), 4 (per-thread K)
  int cls_shift;  // class of row r = (r % 8) >> cls_shift  (3, 0, 1 for the cases above)
  NormRope nr;    // optional RMSNorm + RoPE prologue on the loaded chunks
  // packed variable-length input (null otherwise): entry b is rows cu_seq[b] .. cu_seq[b + 1] of batch 0, its
  // block n's scale goes to scale[(cu_blk[b] + n) * H + h] (quant_per_block_varlen.py:22-70)
  const int32_t* cu_seq;
  const int32_t* cu_blk;
  int64_t total;  // rows of the packed tensor
};

struct QuantArgs {
  QuantJob job[2];
  int njobs;
};

// Rounding of the Triton per-thread quantizer (quant_per_thread.py:63-70): scale = amax/127 + 1e-7,
// half-rounded K - km, round half away.  Used with per-thread scale classes only.
constexpr int QATTN_QUANT_TRITON_THREAD = 2;
// threads per quantizer workgroup: 512 (4 chunks of 16 bytes per thread at 128 rows and D = 128)
template <int VARIANT> constexpr int quant_threads() { return 512; }

// fp32 -> half dtype -> fp32, round to nearest even (bf16 through v_cvt_pk_bf16_f32: one instruction
// instead of the integer sequence; the two differ only in the payload of a NaN, which quantizes to 0)
template <bool IS_FP16>
__device__ __forceinline__ float round_to_half(float v) {
  if constexpr (IS_FP16) {
    return f16_to_f32(f32_to_f16(v));
  } else {
    const __bf16 h = (__bf16)v;
    return (float)h;
  }
}

// One workgroup per block of one (batch entry, head) of a job; a launch covers up to two jobs (Q and K)
// of equal cell layout (cr): workgroups [0, job[0].nwg) take job 0, the rest job 1.  Two passes over registers: |x|
// maxima, then the scales and the quantized bytes.  GROUPED (CR = 32 or 16 rows per cell, nsub = blk / CR
// cells): the block's rows are cells of CR rows with scales of their own, e.g. four
// 32-row scale blocks; a wave's rows of one pass lie in one of them.
// The plain kernel is held to 64 VGPRs: 4 workgroups (8 waves per SIMD) per CU instead of 3, worth more than
// the two registers it spills.
template <bool IS_FP16, int VARIANT, int D, int CR>
__global__ __launch_bounds__(quant_threads<VARIANT>()) __attribute__((amdgpu_waves_per_eu(CR ? 7 : 8)))
void quant_per_block_kernel(QuantArgs args) {
  constexpr bool GROUPED = CR != 0;
  constexpr int NCELL = GROUPED ? 128 / CR : 1;  // cells of a 128-row block
  constexpr int kQuantThreads = quant_threads<VARIANT>();
  constexpr int TPR = D / 8;                       // threads (16-byte chunks) per row
  constexpr int MAXC = 128 * TPR / kQuantThreads;  // chunks per thread at 128 rows
  constexpr int RPP = kQuantThreads / TPR;         // rows per pass: chunk i of a thread is row RPP i + tid / TPR
  constexpr int RPW = 64 / TPR;                    // rows per wave and pass
  constexpr int NW = kQuantThreads / 64;
  constexpr int NA = GROUPED ? MAXC : 1;           // |x| maxima kept per thread
  static_assert(RPP % 32 == 0 && 32 % RPW == 0 && MAXC * RPP == 128, "row cells");

  // index math in 32 bits (the grid is below 2^31 workgroups)
  uint32_t wg = blockIdx.x;
  int j = 0;
  if (args.njobs > 1 && wg >= (uint32_t)args.job[0].nwg) {
    wg -= (uint32_t)args.job[0].nwg;
    j = 1;
  }
  const QuantJob& J = args.job[j];
  const uint32_t H = (uint32_t)J.H, NB = (uint32_t)J.nblk;
  // Heads interleaved inside a row (sequence-major layouts): the heads of one row block run next to
  // each other, so concurrent workgroups read contiguous row segments; head-major layouts walk blocks.
  uint32_t n, h, b;
  if (J.sh < J.sl) {
    const uint32_t q = wg / H;
    h = wg - q * H;
    b = q / NB;
    n = q - b * NB;
  } else {
    const uint32_t bh = wg / NB;
    n = wg - bh * NB;
    b = bh / H;
    h = bh - b * H;
  }
  const int tid = threadIdx.x;
  const int blk = J.blk;
  // this entry's rows: in_b[l * sl], l < Lb (a dense batch entry, or one packed sequence)
  const uint16_t* in_b = J.in + (int64_t)b * J.sb;
  int8_t* out_b = J.out + (int64_t)b * J.ob;
  int64_t Lb = J.L;
  float* scale_at = J.scale + (((int64_t)b * J.H + h) * J.scale_blocks + (int64_t)n * J.nsub) * J.ncls;
  int64_t mb = b;  // batch entry of the mean (packed sequences share entry 0)
  if (J.cu_seq) {
    mb = 0;
    int64_t r0;
    varlen_range(J.cu_seq, b, J.total, J.L, r0, Lb);
    if ((int64_t)n * blk >= Lb) return;  // uniform over the workgroup
    in_b = J.in + r0 * J.sl;
    out_b = J.out + r0 * J.ol;
    scale_at = J.scale + ((int64_t)J.cu_blk[b] + n) * J.H + h;
  }

  // the scale class of a row: rows r with equal (r % 8) / (8 / ncls) share a scale.  Every thread
  // touches rows of a single class (RPP is a multiple of 8).
  const int cls = ((tid / TPR) & 7) >> J.cls_shift;
  const int row0 = tid / TPR, dc = tid % TPR;

  float x[MAXC][8];
  const float amax0 = VARIANT == QATTN_QUANT_CUDA ? 0.0000001f : 0.f;
  float am[NA];  // |x| maximum of each chunk (GROUPED), or of all of them
#pragma unroll
  for (int i = 0; i < NA; i++) am[i] = amax0;
#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int r = row0 + RPP * i;
    const int64_t l = (int64_t)n * blk + r;
#pragma unroll
    for (int e = 0; e < 8; e++) x[i][e] = 0.f;
    if (r < blk && l < Lb) {
      v4u raw = *reinterpret_cast<const v4u*>(in_b + l * J.sl + (int64_t)h * J.sh + dc * 8);
      uint16_t hv[8];
      __builtin_memcpy(hv, &raw, 16);
      if (J.nr.rstd) norm_rope8<IS_FP16>(J.nr, b, J.L, l, h, D, dc, hv);
      float mv[8];
      if (J.mean) {
        v4u mraw = *reinterpret_cast<const v4u*>(J.mean + (mb * J.H + h) * D + dc * 8);
        uint16_t mh[8];
        __builtin_memcpy(mh, &mraw, 16);
#pragma unroll
        for (int e = 0; e < 8; e++) mv[e] = half_to_f32<IS_FP16>(mh[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; e++) {
        float v = half_to_f32<IS_FP16>(hv[e]);
        if (J.mean) {
          v = v - mv[e];
          // Triton paths: k - km is a torch op on half tensors, rounded back to the half type
          if constexpr (VARIANT != QATTN_QUANT_CUDA) v = round_to_half<IS_FP16>(v);
        }
        if (J.has_sm_scale) v = v * J.sm_scale;
        x[i][e] = v;
        am[GROUPED ? i : 0] = fmaxf(am[GROUPED ? i : 0], fabsf(v));
      }
    }
  }

  // IEEE division (hipcc default: correctly rounded)
  auto scale_of = [](float a) {
    if constexpr (VARIANT == QATTN_QUANT_TRITON_THREAD) return quant_scale_triton(a);
    else return quant_scale_cuda(a);
  };
  // per chunk (GROUPED) or per thread: the scale (Triton rounding) or 127 / amax (CUDA rounding)
  float sc[NA];
  if constexpr (VARIANT == QATTN_QUANT_TRITON_THREAD) {
    // per-thread scale classes: each row's maximum (over its TPR lanes) into LDS, then the maximum over
    // the rows of a class in the row's scale block (ungrouped: rows r, r + RPP, ... already share theirs)
    __shared__ float row_max[GROUPED ? 128 : RPP];
#pragma unroll
    for (int i = 0; i < NA; i++) {
      float a = am[i];
#pragma unroll
      for (int o = 1; o < TPR; o <<= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
      if (dc == 0) row_max[RPP * i + row0] = a;
    }
    __syncthreads();
    // rows r of class k in scale block g: (r % 8) in [k * cw, (k + 1) * cw), cw = 8 / ncls (a loop over
    // those rows only)
    const int cw = 1 << J.cls_shift;
    auto class_max = [&](int g, int k) {
      float a = 0.f;
      const int r0 = GROUPED ? CR * g : 0, r1 = GROUPED ? r0 + CR : RPP;
      for (int o = r0; o < r1; o += 8)
        for (int m = 0; m < cw; m++) a = fmaxf(a, row_max[o + k * cw + m]);
      return a;
    };
#pragma unroll
    for (int i = 0; i < NA; i++) sc[i] = scale_of(class_max(GROUPED ? (RPP * i + row0) / (GROUPED ? CR : 1) : 0, cls));
    if (tid < J.nsub * J.ncls) scale_at[tid] = scale_of(class_max(tid / J.ncls, tid % J.ncls));
  } else {  // one scale per scale block: wave maxima, then over the waves (of each 32-row cell)
    __shared__ float wave_maxes[NA][NW];
#pragma unroll
    for (int i = 0; i < NA; i++) {
      const float a = wave_max(am[i]);
      if ((tid & 63) == 0) wave_maxes[i][tid >> 6] = a;
    }
    __syncthreads();
    float cell[NCELL];  // cell c: rows [CR c, CR c + CR) = the waves w of chunk i with (RPP i + RPW w) / CR == c
#pragma unroll
    for (int c = 0; c < NCELL; c++) {
      cell[c] = amax0;
#pragma unroll
      for (int i = 0; i < NA; i++)
#pragma unroll
        for (int ww = 0; ww < NW; ww++)
          if (!GROUPED || (RPP * i + RPW * ww) / (GROUPED ? CR : 1) == c) cell[c] = fmaxf(cell[c], wave_maxes[i][ww]);
    }
#pragma unroll
    for (int i = 0; i < NA; i++) {
      float a = cell[0];
      if constexpr (CR == 32) {
        // this thread's cell of chunk i: (RPP i + row0) / 32, row0 / 32 = RPW (tid / 64) / 32
        a = cell[(RPP * i) / 32];
        if constexpr (RPP > 32) {
          if ((RPW * (tid >> 6)) / 32 == 1) a = cell[(RPP * i) / 32 + 1];
        }
      } else if constexpr (GROUPED) {
        // this wave's cell of chunk i (a wave's RPW rows of a pass lie in one cell)
        const int idx = (RPP * i + RPW * (tid >> 6)) / CR;
#pragma unroll
        for (int c = 1; c < NCELL; c++)
          if (idx == c) a = cell[c];
      }
      sc[i] = VARIANT == QATTN_QUANT_CUDA ? quant_recip_cuda(a) : scale_of(a);
    }
#pragma unroll
    for (int c = 0; c < NCELL; c++)
      if (tid == c && c < J.nsub) scale_at[c] = scale_of(cell[c]);
  }

#pragma unroll
  for (int i = 0; i < MAXC; i++) {
    const int r = row0 + RPP * i;
    const int64_t l = (int64_t)n * blk + r;
    if (r < blk && l < Lb) {
      const float s = sc[GROUPED ? i : 0];
      const float iv = VARIANT == QATTN_QUANT_CUDA ? s : refined_rcp(s);
      int8_t qv[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        // |x| <= amax, so the quotients stay within [-127, 127] before rounding (no saturation step);
        // NaN converts to 0
        if constexpr (VARIANT == QATTN_QUANT_CUDA) {
          // cvt.rni.sat.s8.f32: round to nearest even
          qv[e] = (int8_t)quant_code_cuda(x[i][e], iv);
        } else {
          // Triton: t + 0.5 * sign(t) in fp32, truncate toward zero
          qv[e] = (int8_t)quant_code_triton(x[i][e], s, iv);
        }
      }
      v2u packed;
      __builtin_memcpy(&packed, qv, 8);
      *reinterpret_cast<v2u*>(out_b + l * J.ol + (int64_t)h * J.oh + dc * 8) = packed;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// column reductions over the sequence: partial sums (mean of K) or partial abs-max (scale of V)
// ------------------------------------------------------------------------------------------------

constexpr int kColChunk = 256;  // sequence rows per workgroup

// MODE 0: sum; 1: max |x|; 2: sum, max and min (V smoothing), stored as three D-vectors per chunk
template <bool IS_FP16, int MODE, int D>
__device__ __forceinline__ void col_partial_body(const NormRope& nr, const uint16_t* in, int64_t sb, int64_t sl,
                                                 int64_t sh, int64_t L, int64_t H, int64_t nchunk, float* part,
                                                 int64_t c, int64_t h, int64_t b) {
  constexpr int TPR = D / 8;
  constexpr int RPP = 256 / TPR;  // rows per pass
  __shared__ float red[RPP][D + 1];
  const int tid = threadIdx.x, r0 = tid / TPR, dc = tid % TPR;
  float acc[8], amx[8], amn[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    acc[e] = 0.f;
    amx[e] = -INFINITY;
    amn[e] = INFINITY;
  }
  // rows r0, r0 + RPP, ... of the chunk, loaded four at a time (four loads in flight per thread) and
  // accumulated in row order
  constexpr int kU = 4;
  for (int r = r0; r < kColChunk; r += kU * RPP) {
    v4u raw[kU];
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int64_t l = c * kColChunk + r + u * RPP;
      raw[u] = v4u{0u, 0u, 0u, 0u};
      if (r + u * RPP < kColChunk && l < L) raw[u] = *reinterpret_cast<const v4u*>(in + b * sb + l * sl + h * sh + dc * 8);
    }
#pragma unroll
    for (int u = 0; u < kU; u++) {
      const int64_t l = c * kColChunk + r + u * RPP;
      if (r + u * RPP < kColChunk && l < L) {
        uint16_t hv[8];
        __builtin_memcpy(hv, &raw[u], 16);
        if (nr.rstd) norm_rope8<IS_FP16>(nr, b, L, l, h, D, dc, hv);
#pragma unroll
        for (int e = 0; e < 8; e++) {
          float v = half_to_f32<IS_FP16>(hv[e]);
          if constexpr (MODE == 1) {
            acc[e] = fmaxf(acc[e], fabsf(v));
          } else {
            acc[e] += v;
            if constexpr (MODE == 2) {
              amx[e] = fmaxf(amx[e], v);
              amn[e] = fminf(amn[e], v);
            }
          }
        }
      }
    }
  }
  constexpr int NV = MODE == 2 ? 3 : 1;
#pragma unroll
  for (int k = 0; k < NV; k++) {
    if (k) __syncthreads();
#pragma unroll
    for (int e = 0; e < 8; e++) red[r0][dc * 8 + e] = k == 0 ? acc[e] : k == 1 ? amx[e] : amn[e];
    __syncthreads();
    if (tid < D) {
      float s = red[0][tid];
      for (int r = 1; r < RPP; r++) {
        const float x = red[r][tid];
        s = (MODE == 1 || k == 1) ? fmaxf(s, x) : k == 2 ? fminf(s, x) : s + x;
      }
      part[(((b * H + h) * nchunk + c) * NV + k) * D + tid] = s;
    }
  }
}

template <bool IS_FP16, int MODE, int D>
__global__ __launch_bounds__(256) void col_partial_kernel(NormRope nr, const uint16_t* in, int64_t sb, int64_t sl, int64_t sh,
                                                          int64_t L, int64_t H, int64_t nchunk, float* part) {
  col_partial_body<IS_FP16, MODE, D>(nr, in, sb, sl, sh, L, H, nchunk, part, blockIdx.x, blockIdx.y, blockIdx.z);
}

// The column passes of the SAGE prologue in one launch: z < B sums K (the smoothing mean), z >= B reduces
// V (max |v|, or sum / max / min when V is smoothed).  Same per-chunk work and order as col_partial_kernel.
template <bool IS_FP16, int VMODE, int D>
__global__ __launch_bounds__(256) void prep_col_kernel(const uint16_t* k, int64_t ksb, int64_t ksl, int64_t ksh,
                                                       const uint16_t* v, int64_t vsb, int64_t vsl, int64_t vsh,
                                                       int64_t L, int64_t H, int64_t B, int64_t nchunk, float* kpart,
                                                       float* vpart, int64_t zoff) {
  const int64_t z = blockIdx.z + zoff;  // zoff = B: no K mean, V only
  if (z >= B) col_partial_body<IS_FP16, VMODE, D>(NormRope{}, v, vsb, vsl, vsh, L, H, nchunk, vpart, blockIdx.x, blockIdx.y, z - B);
  else col_partial_body<IS_FP16, 0, D>(NormRope{}, k, ksb, ksl, ksh, L, H, nchunk, kpart, blockIdx.x, blockIdx.y, z);
}

// Chunk partials -> one value per (b, h, d).  One workgroup per (b, h), one thread per channel; the
// loop over chunks keeps 4 independent loads in flight (it is latency-bound, not bandwidth-bound).
// MODE 0: sum, 1: max, 2: min.  Chunk c's vector is at part + ((bh * nchunk + c) * NV + k) * D.
template <int MODE, int D, int NV = 1>
__device__ __forceinline__ float reduce_chunks(const float* part, int64_t bh, int64_t nchunk, int d, int k = 0) {
  const float init = MODE == 0 ? 0.f : MODE == 1 ? -INFINITY : INFINITY;
  float a[4] = {init, init, init, init};
  auto op = [](float x, float y) { return MODE == 0 ? x + y : MODE == 1 ? fmaxf(x, y) : fminf(x, y); };
  auto at = [&](int64_t c) { return part[((bh * nchunk + c) * NV + k) * D + d]; };
  int64_t c = 0;
  // 32 chunks per step: all loads first, then the same accumulation order as one chunk at a time
  for (; c + 32 <= nchunk; c += 32) {
    float x[32];
#pragma unroll
    for (int u = 0; u < 32; u++) x[u] = at(c + u);
#pragma unroll
    for (int u = 0; u < 32; u++) a[u & 3] = op(a[u & 3], x[u]);
  }
  for (; c + 4 <= nchunk; c += 4)
#pragma unroll
    for (int u = 0; u < 4; u++) a[u] = op(a[u], at(c + u));
  for (; c < nchunk; c++) a[0] = op(a[0], at(c));
  return op(op(a[0], a[1]), op(a[2], a[3]));
}

template <bool IS_FP16, int D>
__global__ void mean_finalize_kernel(const float* part, int64_t nchunk, int64_t L, uint16_t* mean) {
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x;
  mean[bh * D + d] = f32_to_half<IS_FP16>(reduce_chunks<0, D>(part, bh, nchunk, d) / (float)L);
}

// V smoothing (MeanScaleKernel<sub_mean>, fused.cu:362-416): the mean divides the sum by the token count
// rounded up to 16 and the max / min cover those zero pad tokens too; amax = max(|max - mean|, |min - mean|).
template <int D>
__global__ void vsmooth_finalize_kernel(const float* part, int64_t nchunk, int64_t L, float scale_max, float* v_scale,
                                        float* recp, float* v_mean) {
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x;
  const float sum = reduce_chunks<0, D, 3>(part, bh, nchunk, d, 0);
  float mx = reduce_chunks<1, D, 3>(part, bh, nchunk, d, 1);
  float mn = reduce_chunks<2, D, 3>(part, bh, nchunk, d, 2);
  const int64_t l16 = (L + 15) / 16 * 16;
  if (l16 != L) {
    mx = fmaxf(mx, 0.f);
    mn = fminf(mn, 0.f);
  }
  const float mean = sum / (float)l16;
  const float a = fmaxf(fabsf(mx - mean), fabsf(mn - mean));
  v_mean[bh * D + d] = mean;
  v_scale[bh * D + d] = a / scale_max;
  recp[bh * D + d] = scale_max / a;
}

// The finalize steps of the SAGE prologue in one launch: blocks [0, BH) write the K mean (when kpart is
// given), blocks [BH, 2 BH) the V scales (and mean, when V is smoothed); same arithmetic as
// mean_finalize_kernel, vscale_finalize_kernel and vsmooth_finalize_kernel.
template <bool IS_FP16, bool SMOOTH_V, int D>
__global__ void prep_finalize_kernel(const float* kpart, const float* vpart, int64_t nchunk, int64_t L, int64_t BH,
                                     uint16_t* kmean, float scale_max, float* v_scale, float* recp, float* v_mean,
                                     int64_t boff) {
  const int64_t blk = blockIdx.x + boff;  // boff = BH: no K mean, V only
  const int64_t bh = blk % BH;
  const int d = threadIdx.x;
  if (blk < BH) {
    kmean[bh * D + d] = f32_to_half<IS_FP16>(reduce_chunks<0, D>(kpart, bh, nchunk, d) / (float)L);
    return;
  }
  if constexpr (SMOOTH_V) {
    const float sum = reduce_chunks<0, D, 3>(vpart, bh, nchunk, d, 0);
    float mx = reduce_chunks<1, D, 3>(vpart, bh, nchunk, d, 1);
    float mn = reduce_chunks<2, D, 3>(vpart, bh, nchunk, d, 2);
    const int64_t l16 = (L + 15) / 16 * 16;
    if (l16 != L) {
      mx = fmaxf(mx, 0.f);
      mn = fminf(mn, 0.f);
    }
    const float mean = sum / (float)l16;
    const float a = fmaxf(fabsf(mx - mean), fabsf(mn - mean));
    v_mean[bh * D + d] = mean;
    v_scale[bh * D + d] = a / scale_max;
    recp[bh * D + d] = scale_max / a;
  } else {
    const float a = reduce_chunks<1, D>(vpart, bh, nchunk, d);
    v_scale[bh * D + d] = a / scale_max;
    recp[bh * D + d] = scale_max / a;
  }
}

template <int D>
__global__ void vscale_finalize_kernel(const float* part, int64_t nchunk, float scale_max, float* v_scale,
                                       float* recp) {
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x;
  const float a = reduce_chunks<1, D>(part, bh, nchunk, d);
  v_scale[bh * D + d] = a / scale_max;
  recp[bh * D + d] = scale_max / a;
}

// Streaming cache: fold the amax of the freshly written rows (two partial sets, one per slot range)
// into the running per-channel amax, publish v_scale / recp from it, and flag the (b, h) whose amax
// grew - their whole FP8 V must be rewritten with the new scale.
template <int D>
__global__ void vcache_scale_kernel(const float* part0, int64_t nchunk0, const float* part1, int64_t nchunk1,
                                    float scale_max, float* amax, float* v_scale, float* recp, int* grown) {
  const int64_t bh = blockIdx.x;
  const int d = threadIdx.x;
  float a = 0.f;
  if (nchunk0) a = reduce_chunks<1, D>(part0, bh, nchunk0, d);
  if (nchunk1) a = fmaxf(a, reduce_chunks<1, D>(part1, bh, nchunk1, d));
  const float old = amax[bh * D + d];
  const float now = fmaxf(old, a);
  amax[bh * D + d] = now;
  v_scale[bh * D + d] = now / scale_max;
  recp[bh * D + d] = scale_max / now;
  const int g = __syncthreads_or(now > old);
  if (d == 0) grown[bh] = g;
}

// ------------------------------------------------------------------------------------------------
// V -> FP8 in the attention kernel's tile layout
// ------------------------------------------------------------------------------------------------

// position of key kappa (0..63) inside its 64-key tile; see qattn.h
__host__ __device__ __forceinline__ int vtile_pos(int kappa) {
  const int kb = kappa >> 5, g = (kappa >> 3) & 3, hf = (kappa >> 2) & 1, t = kappa & 3;
  return hf * 32 + kb * 16 + g * 4 + t;
}

__device__ __forceinline__ uint8_t f32_to_e4m3_sat(float y) {
  if (y != y) return 0x7f;
  y = fminf(fmaxf(y, -448.f), 448.f);
  return (uint8_t)(__builtin_amdgcn_cvt_pk_fp8_f32(y, 0.f, 0, false) & 0xff);
}

// Tiles a streaming-cache update must rewrite: every tile of a (b, h) whose scale grew, otherwise
// only the tiles that overlap the freshly written slot ranges [r[0], r[1]) and [r[2], r[3]).
struct VTileFilter {
  const int* grown;  // [B, H] or null (= rewrite every tile)
  int64_t r[4];
};

// 64-key tiles per workgroup of v_fp8_kernel: the loads of all of them are issued before any is converted
constexpr int kVTilesPerWG = 2;

template <bool IS_FP16, int D>
__global__ __launch_bounds__(256) void v_fp8_kernel(const uint16_t* in, int64_t sb, int64_t sl, int64_t sh,
                                                    int64_t L, int64_t H, const float* recp, uint8_t* v8,
                                                    int64_t Lpad, int64_t ntiles, VTileFilter filt,
                                                    const float* vmean = nullptr) {
  constexpr int TPR = D / 8;
  static_assert(16 * TPR <= 256, "one key quad x 8 channels per thread");
  // The tile as 4-byte words: word w of channel d holds the tile-permuted key slots 4w .. 4w + 3.  Its
  // 16-byte chunks (4 words) are XOR-swizzled by the channel group (d / 8) & 3, so that the word stores
  // of a wave (16 channel groups x 4 key quads) spread over the banks and each chunk is still read back
  // with one 16-byte load.
  __shared__ __align__(16) uint32_t tile[kVTilesPerWG][D][16];
  const int64_t h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  bool act[kVTilesPerWG];  // uniform over the workgroup
#pragma unroll
  for (int tt = 0; tt < kVTilesPerWG; tt++) {
    const int64_t t = (int64_t)blockIdx.x * kVTilesPerWG + tt;
    act[tt] = t < ntiles;
    if (act[tt] && filt.grown && !filt.grown[b * H + h]) {
      const int64_t lo = t * 64, hi = lo + 64;
      act[tt] = (filt.r[0] < hi && lo < filt.r[1]) || (filt.r[2] < hi && lo < filt.r[3]);
    }
  }
  // thread: key quad q (keys 4q .. 4q + 3 of a tile, which occupy consecutive slots) x 8 channels
  const int q = tid / TPR, dc = tid % TPR;
  const bool lane = tid < 16 * TPR;
  uint16_t hv[kVTilesPerWG][4][8];
#pragma unroll
  for (int tt = 0; tt < kVTilesPerWG; tt++) {
    const int64_t t = (int64_t)blockIdx.x * kVTilesPerWG + tt;
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int64_t l = t * 64 + 4 * q + r;
      v4u raw = {0u, 0u, 0u, 0u};
      if (act[tt] && lane && l < L) raw = *reinterpret_cast<const v4u*>(in + b * sb + l * sl + h * sh + dc * 8);
      __builtin_memcpy(hv[tt][r], &raw, 16);
    }
  }
  const float* rc = recp + (b * H + h) * D;
  const float* mn = vmean ? vmean + (b * H + h) * D : nullptr;
  const int wi = vtile_pos(4 * q) >> 2;
  const int sw = (dc & 3) << 2;
  if (lane) {
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const int d = dc * 8 + e;
      const float s = rc[d];
      const float m = mn ? mn[d] : 0.f;
#pragma unroll
      for (int tt = 0; tt < kVTilesPerWG; tt++) {
        const int64_t t = (int64_t)blockIdx.x * kVTilesPerWG + tt;
        uint32_t word = 0;
#pragma unroll
        for (int r = 0; r < 4; r++) {
          // x * recp or (x - mean) * recp as MeanScaleKernel computes it; key slots past L are zero (they
          // are masked, and a zero byte keeps P.V finite there even for an all-zero channel's recp = inf)
          const float x = half_to_f32<IS_FP16>(hv[tt][r][e]);
          const float y = t * 64 + 4 * q + r < L ? (mn ? (x - m) * s : x * s) : 0.f;
          word |= (uint32_t)f32_to_e4m3_sat(y) << (8 * r);
        }
        tile[tt][d][wi ^ sw] = word;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int tt = 0; tt < kVTilesPerWG; tt++) {
    if (!act[tt]) continue;
    const int64_t t = (int64_t)blockIdx.x * kVTilesPerWG + tt;
    for (int c = tid; c < D * 4; c += 256) {
      const int d = c / 4, cc = c % 4;
      const int sc = cc ^ ((d >> 3) & 3);
      *reinterpret_cast<v4u*>(v8 + ((b * H + h) * D + d) * Lpad + t * 64 + cc * 16) =
          *reinterpret_cast<const v4u*>(&tile[tt][d][sc * 4]);
    }
  }
}

// V to FP8 tiles: tiles [0, ntiles) of every (batch entry, head)
static void launch_v_fp8(int dtype, int64_t D, const uint16_t* p, const qattn_seq& v, int64_t L, int64_t B, int64_t H,
                         const float* recp, uint8_t* v8, int64_t Lpad, int64_t ntiles, const VTileFilter& filt,
                         const float* mean, hipStream_t st) {
  dim3 grid((unsigned)((ntiles + kVTilesPerWG - 1) / kVTilesPerWG), (unsigned)H, (unsigned)B);
#define QATTN_VF(F16, DD) \
  v_fp8_kernel<F16, DD><<<grid, 256, 0, st>>>(p, v.sb, v.sl, v.sh, L, H, recp, v8, Lpad, ntiles, filt, mean)
  if (dtype == QATTN_BF16) {
    if (D == 128) QATTN_VF(false, 128);
    else QATTN_VF(false, 64);
  } else {
    if (D == 128) QATTN_VF(true, 128);
    else QATTN_VF(true, 64);
  }
#undef QATTN_VF
}

template <int D>
__global__ __launch_bounds__(256) void v_tile_half_kernel(const uint16_t* in, int64_t sb, int64_t sl, int64_t sh,
                                                          int64_t L, int64_t H, uint16_t* v16, int64_t Lpad,
                                                          const int32_t* cu_k = nullptr, const int32_t* cu_vt = nullptr,
                                                          int64_t total_k = 0) {
  constexpr int TPR = D / 8;
  __shared__ __align__(16) uint16_t tile[D][64];
  int64_t t = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  int64_t tcol = t;  // tile column in v16
  if (cu_k) {  // packed variable-length keys: sequence b's tile t goes to tile column cu_vt[b] + t of entry 0
    int64_t k0;
    varlen_range(cu_k, b, total_k, L, k0, L);
    tcol = (int64_t)cu_vt[b] + t;
    if (t * 64 >= L || (tcol + 1) * 64 > Lpad) return;  // (a too small Lpad drops tiles, never overruns)
    in += k0 * sl;
    b = 0;
  }
#pragma unroll
  for (int i = 0; i < 64 * TPR / 256; i++) {
    const int c = tid + i * 256;
    const int row = c / TPR, dc = c % TPR;
    const int64_t l = t * 64 + row;
    uint16_t hv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (l < L) {
      v4u raw = *reinterpret_cast<const v4u*>(in + b * sb + l * sl + h * sh + dc * 8);
      __builtin_memcpy(hv, &raw, 16);
    }
    const int pos = vtile_pos(row);
#pragma unroll
    for (int e = 0; e < 8; e++) tile[dc * 8 + e][pos] = hv[e];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < D * 8 / 256; i++) {
    const int c = tid + i * 256;
    const int d = c / 8, cc = c % 8;
    *reinterpret_cast<v4u*>(v16 + ((b * H + h) * D + d) * Lpad + tcol * 64 + cc * 8) =
        *reinterpret_cast<const v4u*>(&tile[d][cc * 8]);
  }
}

// ------------------------------------------------------------------------------------------------
// RMSNorm statistics: rstd = 1 / sqrt(mean(x^2) + eps) per row, one wave per row.  The squares of half
// values are exact in fp64 and so is their sum for any realistic row, which makes the mean independent
// of the summation order; var is then rounded to fp32 and the rest is IEEE fp32 (sqrt, division).
// ------------------------------------------------------------------------------------------------
template <bool IS_FP16>
__global__ __launch_bounds__(256) void row_rstd_kernel(const uint16_t* x, int64_t rows, int64_t row_stride, int64_t n,
                                                       float eps, float* rstd) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= rows) return;
  const uint16_t* xr = x + row * row_stride;
  double acc = 0.0;
  for (int64_t c = lane; c * 8 < n; c += 64) {
    const v4u raw = *reinterpret_cast<const v4u*>(xr + c * 8);
    uint16_t hv[8];
    __builtin_memcpy(hv, &raw, 16);
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const double v = (double)half_to_f32<IS_FP16>(hv[e]);
      acc += v * v;
    }
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o, 64);
  if (lane == 0) {
    const float var = (float)(acc / (double)n);
    rstd[row] = 1.0f / sqrtf(var + eps);
  }
}

// ------------------------------------------------------------------------------------------------
// host side
// ------------------------------------------------------------------------------------------------

static int check_seq(const char* name, const qattn_seq& s, int elem_bytes) {
  QATTN_REQUIRE(s.data != nullptr, QATTN_ERR_ARG, "%s: null data pointer", name);
  QATTN_REQUIRE(aligned16(s.data), QATTN_ERR_ALIGN, "%s: data pointer must be 16-byte aligned", name);
  QATTN_REQUIRE((s.sb * elem_bytes) % 16 == 0 && (s.sl * elem_bytes) % 16 == 0 && (s.sh * elem_bytes) % 16 == 0,
                QATTN_ERR_STRIDE, "%s: batch/seq/head strides must be multiples of 16 bytes", name);
  return QATTN_OK;
}

static bool fill_job(QuantJob& J, const qattn_seq& in, const qattn_seq& out, int64_t B, int64_t L, int64_t H,
                     const void* mean, float* scale, float sm_scale, int has_sm, int blk) {
  J.in = static_cast<const uint16_t*>(in.data);
  J.sb = in.sb; J.sl = in.sl; J.sh = in.sh;
  J.out = static_cast<int8_t*>(out.data);
  J.ob = out.sb; J.ol = out.sl; J.oh = out.sh;
  J.scale = scale;
  J.mean = static_cast<const uint16_t*>(mean);
  J.L = L; J.H = H;
  J.blk = blk;
  J.nsub = 1;
  J.cr = 0;
  J.nblk = (L + blk - 1) / blk;
  J.scale_blocks = J.nblk;
  J.has_sm_scale = has_sm;
  J.sm_scale = sm_scale;
  J.nwg = B * H * J.nblk;
  J.ncls = 1;
  J.cls_shift = 3;
  J.nr = NormRope{};
  J.cu_seq = J.cu_blk = nullptr;
  J.total = 0;
  return true;
}

// Q in the per-warp / per-thread layouts: the reference grid's 128-row CTA blocks, each four 32-row warp
// blocks with scales of their own (trailing warp blocks past L get the scale of an empty block).  One
// workgroup covers a CTA block.
static void warp_block_job(QuantJob& J, int64_t B, int warp_rows = 32) {
  // warp_rows 32: the sm80/sm89 layout (128-row blocks of four 32-row warps); 16: the sm90 layout
  // (64-row blocks of four 16-row warps, sageattn2.py:1608-1624)
  J.blk = warp_rows * 4;
  J.nsub = 4;
  J.cr = warp_rows;
  J.nblk = (J.L + J.blk - 1) / J.blk;
  J.scale_blocks = J.nblk * 4;
  J.nwg = B * J.H * J.nblk;
}

template <int D, int CR>
static void launch_quant(const QuantArgs& a, int dtype, int variant, int64_t nwg, hipStream_t st) {
  dim3 grid((unsigned)nwg);
#define QATTN_QK(F16, V) quant_per_block_kernel<F16, V, D, CR><<<grid, quant_threads<V>(), 0, st>>>(a)
  if (dtype == QATTN_BF16) {
    if (variant == QATTN_QUANT_CUDA) QATTN_QK(false, QATTN_QUANT_CUDA);
    else if (variant == QATTN_QUANT_TRITON) QATTN_QK(false, QATTN_QUANT_TRITON);
    else QATTN_QK(false, QATTN_QUANT_TRITON_THREAD);
  } else {
    if (variant == QATTN_QUANT_CUDA) QATTN_QK(true, QATTN_QUANT_CUDA);
    else if (variant == QATTN_QUANT_TRITON) QATTN_QK(true, QATTN_QUANT_TRITON);
    else QATTN_QK(true, QATTN_QUANT_TRITON_THREAD);
  }
#undef QATTN_QK
}

// One launch per scale-block layout among the jobs (Q in warp blocks next to K in plain blocks takes two:
// each kernel keeps the register budget of its own layout).
static int run_quant(QuantArgs& a, int dtype, int64_t D, int variant, hipStream_t st) {
  for (int cr : {0, 32, 16}) {
    QuantArgs s{};
    s.njobs = 0;
    int64_t nwg = 0;
    for (int j = 0; j < a.njobs; j++)
      if (a.job[j].cr == cr && a.job[j].nwg > 0) {
        s.job[s.njobs++] = a.job[j];
        nwg += a.job[j].nwg;
      }
    if (nwg == 0) continue;
    QATTN_REQUIRE(nwg < (1ll << 31), QATTN_ERR_SHAPE, "quantizer grid too large");
    if (cr == 32) {
      if (D == 128) launch_quant<128, 32>(s, dtype, variant, nwg, st);
      else launch_quant<64, 32>(s, dtype, variant, nwg, st);
    } else if (cr == 16) {
      if (D == 128) launch_quant<128, 16>(s, dtype, variant, nwg, st);
      else launch_quant<64, 16>(s, dtype, variant, nwg, st);
    } else {
      if (D == 128) launch_quant<128, 0>(s, dtype, variant, nwg, st);
      else launch_quant<64, 0>(s, dtype, variant, nwg, st);
    }
  }
  return check_launch("quant_per_block_int8");
}

static int check_common(int dtype, int64_t D, int variant, int blk) {
  QATTN_REQUIRE(dtype == QATTN_BF16 || dtype == QATTN_FP16, QATTN_ERR_DTYPE, "dtype must be bf16 (0) or fp16 (1)");
  QATTN_REQUIRE(D == 64 || D == 128, QATTN_ERR_HEAD_DIM, "head_dim must be 64 or 128, got %lld", (long long)D);
  QATTN_REQUIRE(variant == QATTN_QUANT_CUDA || variant == QATTN_QUANT_TRITON, QATTN_ERR_ARG, "unknown variant %d",
                variant);
  QATTN_REQUIRE(blk == 32 || blk == 64 || blk == 128, QATTN_ERR_ARG, "block_size must be 32, 64 or 128, got %d", blk);
  return QATTN_OK;
}

}  // namespace qattn

using namespace qattn;

extern "C" int qattn_quant_per_block_int8(qattn_seq in, int dtype, int64_t B, int64_t L, int64_t H, int64_t D,
                                          const void* mean, qattn_seq out, float* scale, float sm_scale,
                                          int has_sm_scale, int block_size, int variant, qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, variant, block_size))) return rc;
  QATTN_REQUIRE(B >= 0 && L >= 0 && H >= 0, QATTN_ERR_SHAPE, "negative size");
  if (B * L * H == 0) return QATTN_OK;
  if ((rc = check_seq("input", in, 2)) || (rc = check_seq("output", out, 1))) return rc;
  QATTN_REQUIRE(scale != nullptr, QATTN_ERR_ARG, "scale is null");
  QATTN_REQUIRE(mean == nullptr || aligned16(mean), QATTN_ERR_ALIGN, "mean must be 16-byte aligned");
  QuantArgs a{};
  a.njobs = 1;
  fill_job(a.job[0], in, out, B, L, H, mean, scale, sm_scale, has_sm_scale, block_size);
  return run_quant(a, dtype, D, variant, (hipStream_t)stream);
}

extern "C" int qattn_quant_qk_per_block_int8(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t Lq,
                                             int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean,
                                             qattn_seq q_out, qattn_seq k_out, float* q_scale, float* k_scale,
                                             float sm_scale, int blkq, int blkk, int variant,
                                             qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, variant, blkq)) || (rc = check_common(dtype, D, variant, blkk))) return rc;
  QATTN_REQUIRE(B >= 0 && Lq >= 0 && Lk >= 0 && Hq >= 0 && Hkv >= 0, QATTN_ERR_SHAPE, "negative size");
  QuantArgs a{};
  a.njobs = 0;
  if (B * Lq * Hq > 0) {
    if ((rc = check_seq("q", q, 2)) || (rc = check_seq("q_out", q_out, 1))) return rc;
    QATTN_REQUIRE(q_scale != nullptr, QATTN_ERR_ARG, "q_scale is null");
    fill_job(a.job[a.njobs++], q, q_out, B, Lq, Hq, nullptr, q_scale, sm_scale, 1, blkq);
  }
  if (B * Lk * Hkv > 0) {
    if ((rc = check_seq("k", k, 2)) || (rc = check_seq("k_out", k_out, 1))) return rc;
    QATTN_REQUIRE(k_scale != nullptr, QATTN_ERR_ARG, "k_scale is null");
    QATTN_REQUIRE(k_mean == nullptr || aligned16(k_mean), QATTN_ERR_ALIGN, "k_mean must be 16-byte aligned");
    fill_job(a.job[a.njobs++], k, k_out, B, Lk, Hkv, k_mean, k_scale, 1.0f, 0, blkk);
  }
  if (a.njobs == 0) return QATTN_OK;
  return run_quant(a, dtype, D, variant, (hipStream_t)stream);
}

extern "C" int qattn_quant_qk_per_warp_int8_ex(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t Lq,
                                                int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean,
                                                qattn_seq q_out, qattn_seq k_out, float* q_scale, float* k_scale,
                                                int scale_layout, qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, QATTN_QUANT_CUDA, 64))) return rc;
  QATTN_REQUIRE(scale_layout == QATTN_SCALES_SM89 || scale_layout == QATTN_SCALES_SM90, QATTN_ERR_ARG,
                "scale_layout must be 0 (sm89) or 1 (sm90), got %d", scale_layout);
  QATTN_REQUIRE(B >= 0 && Lq >= 0 && Lk >= 0 && Hq >= 0 && Hkv >= 0, QATTN_ERR_SHAPE, "negative size");
  QATTN_REQUIRE(q_scale && k_scale, QATTN_ERR_ARG, "scale is null");
  const bool sm90 = scale_layout == QATTN_SCALES_SM90;
  QuantArgs a{};
  a.njobs = 0;
  if (B * Lq * Hq > 0) {
    if ((rc = check_seq("q", q, 2)) || (rc = check_seq("q_out", q_out, 1))) return rc;
    QuantJob& J = a.job[a.njobs++];
    fill_job(J, q, q_out, B, Lq, Hq, nullptr, q_scale, 1.0f, 0, 32);
    warp_block_job(J, B, sm90 ? 16 : 32);
  }
  if (B * Lk * Hkv > 0) {
    if ((rc = check_seq("k", k, 2)) || (rc = check_seq("k_out", k_out, 1))) return rc;
    QATTN_REQUIRE(k_mean == nullptr || aligned16(k_mean), QATTN_ERR_ALIGN, "k_mean must be 16-byte aligned");
    fill_job(a.job[a.njobs++], k, k_out, B, Lk, Hkv, k_mean, k_scale, 1.0f, 0, sm90 ? 128 : 64);
  }
  if (a.njobs == 0) return QATTN_OK;
  return run_quant(a, dtype, D, QATTN_QUANT_CUDA, (hipStream_t)stream);
}

extern "C" int qattn_quant_qk_per_warp_int8(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t Lq, int64_t Lk,
                                             int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean, qattn_seq q_out,
                                             qattn_seq k_out, float* q_scale, float* k_scale, qattn_stream_t stream) {
  return qattn_quant_qk_per_warp_int8_ex(q, k, dtype, B, Lq, Lk, Hq, Hkv, D, k_mean, q_out, k_out, q_scale, k_scale,
                                         QATTN_SCALES_SM89, stream);
}

extern "C" int qattn_quant_qk_per_thread_int8_ex(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t Lq,
                                                  int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean,
                                                  qattn_seq q_out, qattn_seq k_out, float* q_scale, float* k_scale,
                                                  int scale_layout, qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, QATTN_QUANT_TRITON, 64))) return rc;
  QATTN_REQUIRE(scale_layout == QATTN_SCALES_SM89 || scale_layout == QATTN_SCALES_SM90, QATTN_ERR_ARG,
                "scale_layout must be 0 (sm89) or 1 (sm90), got %d", scale_layout);
  QATTN_REQUIRE(B >= 0 && Lq >= 0 && Lk >= 0 && Hq >= 0 && Hkv >= 0, QATTN_ERR_SHAPE, "negative size");
  QATTN_REQUIRE(q_scale && k_scale, QATTN_ERR_ARG, "scale is null");
  const bool sm90 = scale_layout == QATTN_SCALES_SM90;
  QuantArgs a{};
  a.njobs = 0;
  if (B * Lq * Hq > 0) {
    if ((rc = check_seq("q", q, 2)) || (rc = check_seq("q_out", q_out, 1))) return rc;
    QuantJob& J = a.job[a.njobs++];
    fill_job(J, q, q_out, B, Lq, Hq, nullptr, q_scale, 1.0f, 0, 32);
    warp_block_job(J, B, sm90 ? 16 : 32);
    J.ncls = 8;
    J.cls_shift = 0;
  }
  if (B * Lk * Hkv > 0) {
    if ((rc = check_seq("k", k, 2)) || (rc = check_seq("k_out", k_out, 1))) return rc;
    QATTN_REQUIRE(k_mean == nullptr || aligned16(k_mean), QATTN_ERR_ALIGN, "k_mean must be 16-byte aligned");
    QuantJob& J = a.job[a.njobs++];
    fill_job(J, k, k_out, B, Lk, Hkv, k_mean, k_scale, 1.0f, 0, sm90 ? 128 : 64);
    J.ncls = 4;
    J.cls_shift = 1;
  }
  if (a.njobs == 0) return QATTN_OK;
  return run_quant(a, dtype, D, QATTN_QUANT_TRITON_THREAD, (hipStream_t)stream);
}

extern "C" int qattn_quant_qk_per_thread_int8(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t Lq,
                                               int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, const void* k_mean,
                                               qattn_seq q_out, qattn_seq k_out, float* q_scale, float* k_scale,
                                               qattn_stream_t stream) {
  return qattn_quant_qk_per_thread_int8_ex(q, k, dtype, B, Lq, Lk, Hq, Hkv, D, k_mean, q_out, k_out, q_scale,
                                           k_scale, QATTN_SCALES_SM89, stream);
}

static int64_t col_chunks(int64_t L) { return (L + kColChunk - 1) / kColChunk; }

extern "C" size_t qattn_seq_mean_workspace_size(int64_t B, int64_t L, int64_t H, int64_t D) {
  return (size_t)(B * H * col_chunks(L) * D) * sizeof(float);
}

template <int MODE>
static void launch_col(const qattn_seq& in, int dtype, int64_t B, int64_t L, int64_t H, int64_t D, int64_t nchunk,
                       float* part, hipStream_t st, const NormRope& nr = NormRope{}) {
  dim3 grid((unsigned)nchunk, (unsigned)H, (unsigned)B);
  const uint16_t* p = static_cast<const uint16_t*>(in.data);
#define QATTN_COL(F16, DD) col_partial_kernel<F16, MODE, DD><<<grid, 256, 0, st>>>(nr, p, in.sb, in.sl, in.sh, L, H, nchunk, part)
  if (dtype == QATTN_BF16) { if (D == 128) QATTN_COL(false, 128); else QATTN_COL(false, 64); }
  else { if (D == 128) QATTN_COL(true, 128); else QATTN_COL(true, 64); }
#undef QATTN_COL
}

extern "C" int qattn_seq_mean(qattn_seq in, int dtype, int64_t B, int64_t L, int64_t H, int64_t D, void* mean,
                              void* workspace, size_t workspace_bytes, qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, QATTN_QUANT_CUDA, 64))) return rc;
  QATTN_REQUIRE(B > 0 && L > 0 && H > 0, QATTN_ERR_SHAPE, "seq_mean needs non-empty input");
  if ((rc = check_seq("input", in, 2))) return rc;
  QATTN_REQUIRE(mean != nullptr, QATTN_ERR_ARG, "mean is null");
  const int64_t nchunk = col_chunks(L);
  QATTN_REQUIRE(workspace && workspace_bytes >= qattn_seq_mean_workspace_size(B, L, H, D), QATTN_ERR_WORKSPACE,
                "seq_mean workspace too small");
  hipStream_t st = (hipStream_t)stream;
  float* part = static_cast<float*>(workspace);
  launch_col<0>(in, dtype, B, L, H, D, nchunk, part, st);
  uint16_t* m = static_cast<uint16_t*>(mean);
  if (dtype == QATTN_BF16) {
    if (D == 128) mean_finalize_kernel<false, 128><<<B * H, 128, 0, st>>>(part, nchunk, L, m);
    else mean_finalize_kernel<false, 64><<<B * H, 64, 0, st>>>(part, nchunk, L, m);
  } else {
    if (D == 128) mean_finalize_kernel<true, 128><<<B * H, 128, 0, st>>>(part, nchunk, L, m);
    else mean_finalize_kernel<true, 64><<<B * H, 64, 0, st>>>(part, nchunk, L, m);
  }
  return check_launch("seq_mean");
}

extern "C" size_t qattn_per_channel_fp8_workspace_size(int64_t B, int64_t L, int64_t H, int64_t D) {
  // (three partial vectors per chunk: enough for the smoothed form too)
  return (size_t)(3 * B * H * col_chunks(L) * D + B * H * D) * sizeof(float);
}

extern "C" int qattn_per_channel_fp8(qattn_seq v, int dtype, int64_t B, int64_t L, int64_t H, int64_t D,
                                     float scale_max, uint8_t* v8, int64_t Lpad, float* v_scale, void* workspace,
                                     size_t workspace_bytes, qattn_stream_t stream) {
  return qattn_per_channel_fp8_ex(v, dtype, B, L, H, D, scale_max, 0, v8, Lpad, v_scale, nullptr, workspace,
                                  workspace_bytes, stream);
}

extern "C" int qattn_per_channel_fp8_ex(qattn_seq v, int dtype, int64_t B, int64_t L, int64_t H, int64_t D,
                                        float scale_max, int smooth_v, uint8_t* v8, int64_t Lpad, float* v_scale,
                                        float* v_mean, void* workspace, size_t workspace_bytes,
                                        qattn_stream_t stream) {
  int rc;
  QATTN_REQUIRE(!smooth_v || v_mean, QATTN_ERR_ARG, "smooth_v needs a v_mean output");
  if ((rc = check_common(dtype, D, QATTN_QUANT_CUDA, 64))) return rc;
  QATTN_REQUIRE(B > 0 && L > 0 && H > 0, QATTN_ERR_SHAPE, "per_channel_fp8 needs non-empty input");
  if ((rc = check_seq("v", v, 2))) return rc;
  QATTN_REQUIRE(Lpad >= (L + 63) / 64 * 64 && Lpad % 64 == 0, QATTN_ERR_SHAPE,
                "Lpad must be a multiple of 64 and >= L rounded up to 64");
  QATTN_REQUIRE(v8 && aligned16(v8) && v_scale, QATTN_ERR_ALIGN, "v8 must be non-null and 16-byte aligned");
  QATTN_REQUIRE(workspace && workspace_bytes >= qattn_per_channel_fp8_workspace_size(B, L, H, D),
                QATTN_ERR_WORKSPACE, "per_channel_fp8 workspace too small");
  hipStream_t st = (hipStream_t)stream;
  const int64_t nchunk = col_chunks(L);
  float* part = static_cast<float*>(workspace);
  float* recp = part + 3 * B * H * nchunk * D;
  const float* mean = smooth_v ? v_mean : nullptr;
  if (smooth_v) {
    launch_col<2>(v, dtype, B, L, H, D, nchunk, part, st);
    if (D == 128) vsmooth_finalize_kernel<128><<<B * H, 128, 0, st>>>(part, nchunk, L, scale_max, v_scale, recp, v_mean);
    else vsmooth_finalize_kernel<64><<<B * H, 64, 0, st>>>(part, nchunk, L, scale_max, v_scale, recp, v_mean);
  } else {
    launch_col<1>(v, dtype, B, L, H, D, nchunk, part, st);
    if (D == 128) vscale_finalize_kernel<128><<<B * H, 128, 0, st>>>(part, nchunk, scale_max, v_scale, recp);
    else vscale_finalize_kernel<64><<<B * H, 64, 0, st>>>(part, nchunk, scale_max, v_scale, recp);
  }
  const VTileFilter nof{nullptr, {0, 0, 0, 0}};
  launch_v_fp8(dtype, D, static_cast<const uint16_t*>(v.data), v, L, B, H, recp, v8, Lpad, Lpad / 64, nof, mean, st);
  return check_launch("per_channel_fp8");
}

extern "C" int qattn_v_tile_half(qattn_seq v, int dtype, int64_t B, int64_t L, int64_t H, int64_t D, uint16_t* v16,
                                 int64_t Lpad, qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, QATTN_QUANT_CUDA, 64))) return rc;
  QATTN_REQUIRE(B > 0 && L > 0 && H > 0, QATTN_ERR_SHAPE, "v_tile_half needs non-empty input");
  if ((rc = check_seq("v", v, 2))) return rc;
  QATTN_REQUIRE(Lpad >= (L + 63) / 64 * 64 && Lpad % 64 == 0, QATTN_ERR_SHAPE,
                "Lpad must be a multiple of 64 and >= L rounded up to 64");
  QATTN_REQUIRE(v16 && aligned16(v16), QATTN_ERR_ALIGN, "v16 must be non-null and 16-byte aligned");
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)(Lpad / 64), (unsigned)H, (unsigned)B);
  const uint16_t* p = static_cast<const uint16_t*>(v.data);
  if (D == 128) v_tile_half_kernel<128><<<grid, 256, 0, st>>>(p, v.sb, v.sl, v.sh, L, H, v16, Lpad);
  else v_tile_half_kernel<64><<<grid, 256, 0, st>>>(p, v.sb, v.sl, v.sh, L, H, v16, Lpad);
  return check_launch("v_tile_half");
}


extern "C" size_t qattn_v_fp8_cache_workspace_size(int64_t B, int64_t n0, int64_t n1, int64_t H, int64_t D) {
  return (size_t)(B * H * (col_chunks(n0) + col_chunks(n1)) * D + B * H * D + B * H) * sizeof(float);
}

extern "C" int qattn_v_fp8_cache_update(qattn_seq v, int dtype, int64_t B, int64_t fill, int64_t H, int64_t D,
                                        int64_t begin0, int64_t end0, int64_t begin1, int64_t end1,
                                        float scale_max, float* amax, uint8_t* v8, int64_t Lpad, float* v_scale,
                                        void* workspace, size_t workspace_bytes, qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, QATTN_QUANT_CUDA, 64))) return rc;
  QATTN_REQUIRE(B > 0 && H > 0 && fill > 0, QATTN_ERR_SHAPE, "v_fp8_cache_update needs a non-empty cache");
  QATTN_REQUIRE(0 <= begin0 && begin0 <= end0 && end0 <= fill && 0 <= begin1 && begin1 <= end1 && end1 <= fill,
                QATTN_ERR_ARG, "slot ranges must lie inside [0, fill)");
  if ((rc = check_seq("v", v, 2))) return rc;
  QATTN_REQUIRE(Lpad >= (fill + 63) / 64 * 64 && Lpad % 64 == 0, QATTN_ERR_SHAPE,
                "Lpad must be a multiple of 64 and >= fill rounded up to 64");
  QATTN_REQUIRE(v8 && aligned16(v8) && v_scale && amax, QATTN_ERR_ALIGN, "v8 must be non-null and 16-byte aligned");
  const int64_t n0 = end0 - begin0, n1 = end1 - begin1;
  QATTN_REQUIRE(workspace && workspace_bytes >= qattn_v_fp8_cache_workspace_size(B, n0, n1, H, D),
                QATTN_ERR_WORKSPACE, "v_fp8_cache_update workspace too small");
  hipStream_t st = (hipStream_t)stream;
  const int64_t c0 = col_chunks(n0), c1 = col_chunks(n1);
  float* part0 = static_cast<float*>(workspace);
  float* part1 = part0 + B * H * c0 * D;
  float* recp = part1 + B * H * c1 * D;
  int* grown = reinterpret_cast<int*>(recp + B * H * D);
  const int esz = 2;
  auto range_view = [&](int64_t begin) {
    qattn_seq s = v;
    s.data = static_cast<char*>(v.data) + begin * v.sl * esz;
    return s;
  };
  if (n0) launch_col<1>(range_view(begin0), dtype, B, n0, H, D, c0, part0, st);
  if (n1) launch_col<1>(range_view(begin1), dtype, B, n1, H, D, c1, part1, st);
  if (D == 128)
    vcache_scale_kernel<128><<<B * H, 128, 0, st>>>(part0, c0, part1, c1, scale_max, amax, v_scale, recp, grown);
  else
    vcache_scale_kernel<64><<<B * H, 64, 0, st>>>(part0, c0, part1, c1, scale_max, amax, v_scale, recp, grown);
  const VTileFilter filt{grown, {begin0, end0, begin1, end1}};
  launch_v_fp8(dtype, D, static_cast<const uint16_t*>(v.data), v, fill, B, H, recp, v8, Lpad, (fill + 63) / 64, filt,
               nullptr, st);
  return check_launch("v_fp8_cache_update");
}

extern "C" int qattn_row_rstd(const void* x, int dtype, int64_t rows, int64_t row_stride, int64_t n, float eps,
                              float* rstd, qattn_stream_t stream) {
  QATTN_REQUIRE(dtype == QATTN_BF16 || dtype == QATTN_FP16, QATTN_ERR_DTYPE, "dtype must be bf16 (0) or fp16 (1)");
  QATTN_REQUIRE(rows >= 0 && n > 0 && n % 8 == 0, QATTN_ERR_SHAPE, "row length must be a positive multiple of 8");
  if (rows == 0) return QATTN_OK;
  QATTN_REQUIRE(x && aligned16(x) && row_stride % 8 == 0, QATTN_ERR_ALIGN, "rows must be 16-byte aligned");
  QATTN_REQUIRE(rstd != nullptr, QATTN_ERR_ARG, "rstd is null");
  hipStream_t st = (hipStream_t)stream;
  const unsigned grid = (unsigned)((rows + 3) / 4);
  const uint16_t* p = static_cast<const uint16_t*>(x);
  if (dtype == QATTN_BF16) row_rstd_kernel<false><<<grid, 256, 0, st>>>(p, rows, row_stride, n, eps, rstd);
  else row_rstd_kernel<true><<<grid, 256, 0, st>>>(p, rows, row_stride, n, eps, rstd);
  return check_launch("row_rstd");
}

static int make_norm_rope(NormRope& nr, const float* rstd, const void* w, const float* cs, const float* sn,
                          int64_t cs_stride, int64_t D) {
  QATTN_REQUIRE(rstd && w && cs && sn, QATTN_ERR_ARG, "norm/rope operands must be non-null");
  QATTN_REQUIRE(aligned16(w) && aligned16(cs) && aligned16(sn) && cs_stride % 4 == 0 && cs_stride >= D / 2,
                QATTN_ERR_ALIGN, "weight / cos / sin must be 16-byte aligned with cos/sin rows of >= D/2 floats");
  nr.rstd = rstd;
  nr.w = static_cast<const uint16_t*>(w);
  nr.cs = cs;
  nr.sn = sn;
  nr.cs_stride = cs_stride;
  return QATTN_OK;
}

extern "C" int qattn_norm_rope_seq_mean(qattn_seq x, int dtype, int64_t B, int64_t L, int64_t H, int64_t D,
                                        const float* rstd, const void* w, const float* cs, const float* sn,
                                        int64_t cs_stride, void* mean, void* workspace, size_t workspace_bytes,
                                        qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, QATTN_QUANT_CUDA, 64))) return rc;
  QATTN_REQUIRE(B > 0 && L > 0 && H > 0, QATTN_ERR_SHAPE, "norm_rope_seq_mean needs non-empty input");
  if ((rc = check_seq("x", x, 2))) return rc;
  NormRope nr{};
  if ((rc = make_norm_rope(nr, rstd, w, cs, sn, cs_stride, D))) return rc;
  QATTN_REQUIRE(mean != nullptr, QATTN_ERR_ARG, "mean is null");
  QATTN_REQUIRE(workspace && workspace_bytes >= qattn_seq_mean_workspace_size(B, L, H, D), QATTN_ERR_WORKSPACE,
                "norm_rope_seq_mean workspace too small");
  hipStream_t st = (hipStream_t)stream;
  const int64_t nchunk = col_chunks(L);
  float* part = static_cast<float*>(workspace);
  launch_col<0>(x, dtype, B, L, H, D, nchunk, part, st, nr);
  uint16_t* m = static_cast<uint16_t*>(mean);
  if (dtype == QATTN_BF16) {
    if (D == 128) mean_finalize_kernel<false, 128><<<B * H, 128, 0, st>>>(part, nchunk, L, m);
    else mean_finalize_kernel<false, 64><<<B * H, 64, 0, st>>>(part, nchunk, L, m);
  } else {
    if (D == 128) mean_finalize_kernel<true, 128><<<B * H, 128, 0, st>>>(part, nchunk, L, m);
    else mean_finalize_kernel<true, 64><<<B * H, 64, 0, st>>>(part, nchunk, L, m);
  }
  return check_launch("norm_rope_seq_mean");
}

extern "C" int qattn_norm_rope_quant_qk(qattn_seq xq, qattn_seq xk, int dtype, int64_t B, int64_t L, int64_t H,
                                        int64_t D, const float* rstd_q, const float* rstd_k, const void* wq,
                                        const void* wk, const float* cs, const float* sn, int64_t cs_stride,
                                        const void* k_mean, qattn_seq q_out, qattn_seq k_out, float* q_scale,
                                        float* k_scale, float sm_scale, int variant, qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, variant, 64))) return rc;
  QATTN_REQUIRE(B >= 0 && L >= 0 && H >= 0, QATTN_ERR_SHAPE, "negative size");
  if (B * L * H == 0) return QATTN_OK;
  if ((rc = check_seq("xq", xq, 2)) || (rc = check_seq("xk", xk, 2)) || (rc = check_seq("q_out", q_out, 1)) ||
      (rc = check_seq("k_out", k_out, 1)))
    return rc;
  QATTN_REQUIRE(q_scale && k_scale, QATTN_ERR_ARG, "scale is null");
  QATTN_REQUIRE(k_mean == nullptr || aligned16(k_mean), QATTN_ERR_ALIGN, "k_mean must be 16-byte aligned");
  QuantArgs a{};
  a.njobs = 2;
  fill_job(a.job[0], xq, q_out, B, L, H, nullptr, q_scale, sm_scale, 1, 128);
  fill_job(a.job[1], xk, k_out, B, L, H, k_mean, k_scale, 1.0f, 0, 64);
  if ((rc = make_norm_rope(a.job[0].nr, rstd_q, wq, cs, sn, cs_stride, D))) return rc;
  if ((rc = make_norm_rope(a.job[1].nr, rstd_k, wk, cs, sn, cs_stride, D))) return rc;
  return run_quant(a, dtype, D, variant, (hipStream_t)stream);
}

// ------------------------------------------------------------------------------------------------
// packed variable-length batches
// ------------------------------------------------------------------------------------------------

namespace qattn {
// Sanitised sequence tables and block offsets of a packed batch, by one thread (B is small).  The
// sanitised tables are the caller's cu_seqlens made non-decreasing and clamped to [0, total], so that the
// sequences are disjoint row ranges of the packed tensors whatever the input; the other varlen kernels read
// only these.  cu_qs[b] = sum of ceil(len_q / 128), cu_ks[b] = cu_vt[b] = sum of ceil(len_k / 64) over the
// sequences before b, with len = min(rows of the sequence, max_seqlen) (the cumsum of
// quant_per_block_varlen.py:92-107).
__global__ void varlen_offsets_kernel(const int32_t* cu_q, const int32_t* cu_k, int64_t B, int64_t total_q,
                                      int64_t total_k, int64_t max_lq, int64_t max_lk, int32_t* sq, int32_t* sk,
                                      int32_t* cu_qs, int32_t* cu_ks, int32_t* cu_vt) {
  if (threadIdx.x != 0) return;
  int64_t pq = 0, pk = 0;
  for (int64_t b = 0; b <= B; b++) {
    pq = min(max((int64_t)cu_q[b], pq), total_q);
    pk = min(max((int64_t)cu_k[b], pk), total_k);
    sq[b] = (int32_t)pq;
    sk[b] = (int32_t)pk;
  }
  int32_t aq = 0, ak = 0;
  for (int64_t b = 0; b <= B; b++) {
    cu_qs[b] = aq;
    cu_ks[b] = ak;
    cu_vt[b] = ak;
    if (b < B) {
      int64_t s, lq, lk;
      varlen_range(sq, b, total_q, max_lq, s, lq);
      varlen_range(sk, b, total_k, max_lk, s, lk);
      aq += (int32_t)((lq + 127) / 128);
      ak += (int32_t)((lk + 63) / 64);
    }
  }
}
}  // namespace qattn

extern "C" int qattn_varlen_offsets(const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int64_t B,
                                    int64_t total_q, int64_t total_k, int64_t max_lq, int64_t max_lk,
                                    int32_t* seq_q, int32_t* seq_k, int32_t* cu_qs, int32_t* cu_ks, int32_t* cu_vt,
                                    qattn_stream_t stream) {
  QATTN_REQUIRE(B > 0 && total_q >= 0 && total_k >= 0 && max_lq >= 0 && max_lk >= 0, QATTN_ERR_SHAPE,
                "varlen batch must hold at least one sequence; sizes must be non-negative");
  QATTN_REQUIRE(total_q < (1ll << 31) && total_k < (1ll << 31), QATTN_ERR_SHAPE, "packed tensors too long");
  QATTN_REQUIRE(cu_seqlens_q && cu_seqlens_k && seq_q && seq_k && cu_qs && cu_ks && cu_vt, QATTN_ERR_ARG,
                "null pointer");
  varlen_offsets_kernel<<<1, 64, 0, (hipStream_t)stream>>>(cu_seqlens_q, cu_seqlens_k, B, total_q, total_k, max_lq,
                                                           max_lk, seq_q, seq_k, cu_qs, cu_ks, cu_vt);
  return check_launch("varlen_offsets");
}

extern "C" int qattn_quant_qk_varlen_int8(qattn_seq q, qattn_seq k, int dtype, int64_t B, int64_t total_q,
                                          int64_t total_k, int64_t max_lq, int64_t max_lk, int64_t Hq, int64_t Hkv,
                                          int64_t D, const void* k_mean,
                                          const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                          const int32_t* cu_qs, const int32_t* cu_ks, qattn_seq q_out,
                                          qattn_seq k_out, float* q_scale, float* k_scale, float sm_scale,
                                          int variant, qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, variant, 128))) return rc;
  QATTN_REQUIRE(B > 0 && total_q >= 0 && total_k >= 0 && max_lq >= 0 && max_lk >= 0 && Hq > 0 && Hkv > 0,
                QATTN_ERR_SHAPE, "bad sizes");
  QATTN_REQUIRE(cu_seqlens_q && cu_seqlens_k && cu_qs && cu_ks && q_scale && k_scale, QATTN_ERR_ARG, "null pointer");
  if ((rc = check_seq("q", q, 2)) || (rc = check_seq("q_out", q_out, 1)) || (rc = check_seq("k", k, 2)) ||
      (rc = check_seq("k_out", k_out, 1)))
    return rc;
  QATTN_REQUIRE(k_mean == nullptr || aligned16(k_mean), QATTN_ERR_ALIGN, "k_mean must be 16-byte aligned");
  QuantArgs a{};
  a.njobs = 0;
  if (max_lq > 0) {
    QuantJob& J = a.job[a.njobs++];
    fill_job(J, q, q_out, B, max_lq, Hq, nullptr, q_scale, sm_scale, 1, 128);
    J.cu_seq = cu_seqlens_q;
    J.cu_blk = cu_qs;
    J.total = total_q;
  }
  if (max_lk > 0) {
    QuantJob& J = a.job[a.njobs++];
    fill_job(J, k, k_out, B, max_lk, Hkv, k_mean, k_scale, 1.0f, 0, 64);
    J.cu_seq = cu_seqlens_k;
    J.cu_blk = cu_ks;
    J.total = total_k;
  }
  if (a.njobs == 0) return QATTN_OK;
  return run_quant(a, dtype, D, variant, (hipStream_t)stream);
}

extern "C" int qattn_v_tile_half_varlen(qattn_seq v, int dtype, int64_t B, int64_t total_k, int64_t max_lk, int64_t H,
                                        int64_t D,
                                        const int32_t* cu_seqlens_k, const int32_t* cu_vt, uint16_t* v16,
                                        int64_t Lpad, qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, QATTN_QUANT_CUDA, 64))) return rc;
  QATTN_REQUIRE(B > 0 && total_k >= 0 && max_lk > 0 && H > 0, QATTN_ERR_SHAPE, "v_tile_half_varlen needs non-empty input");
  if ((rc = check_seq("v", v, 2))) return rc;
  QATTN_REQUIRE(Lpad % 64 == 0, QATTN_ERR_SHAPE, "Lpad must be a multiple of 64");
  QATTN_REQUIRE(v16 && aligned16(v16) && cu_seqlens_k && cu_vt, QATTN_ERR_ARG, "null or misaligned pointer");
  hipStream_t st = (hipStream_t)stream;
  dim3 grid((unsigned)((max_lk + 63) / 64), (unsigned)H, (unsigned)B);
  const uint16_t* p = static_cast<const uint16_t*>(v.data);
  if (D == 128) v_tile_half_kernel<128><<<grid, 256, 0, st>>>(p, v.sb, v.sl, v.sh, max_lk, H, v16, Lpad, cu_seqlens_k, cu_vt, total_k);
  else v_tile_half_kernel<64><<<grid, 256, 0, st>>>(p, v.sb, v.sl, v.sh, max_lk, H, v16, Lpad, cu_seqlens_k, cu_vt,
                                                    total_k);
  return check_launch("v_tile_half_varlen");
}

// ------------------------------------------------------------------------------------------------
// the whole SAGE prologue: K mean, Q/K INT8, V FP8 in four launches
// ------------------------------------------------------------------------------------------------

extern "C" size_t qattn_sage_quant_workspace_size(int64_t B, int64_t Lk, int64_t Hkv, int64_t D) {
  const int64_t n = B * Hkv * col_chunks(Lk) * D;
  return (size_t)(n + 3 * n + B * Hkv * D) * sizeof(float);
}

extern "C" int qattn_sage_quant(qattn_seq q, qattn_seq k, qattn_seq v, int dtype, int64_t B, int64_t Lq, int64_t Lk,
                                int64_t Hq, int64_t Hkv, int64_t D, int qk_quant_gran, float q_sm_scale, int smooth_k,
                                float scale_max, int smooth_v, qattn_seq q_out, float* q_scale, qattn_seq k_out,
                                float* k_scale, void* k_mean, uint8_t* v8, int64_t Lpad, float* v_scale,
                                float* v_mean, void* workspace, size_t workspace_bytes, qattn_stream_t stream) {
  int rc;
  if ((rc = check_common(dtype, D, QATTN_QUANT_CUDA, 64))) return rc;
  QATTN_REQUIRE(qk_quant_gran >= 1 && qk_quant_gran <= 5, QATTN_ERR_ARG,
                "qk_quant_gran must be 1 (per block), 2 (per warp), 3 (per thread), 4 (per warp, sm90 tables) or "
                "5 (per thread, sm90 tables), got %d", qk_quant_gran);
  // Lq = 0: K and V only (Q is quantized by the attention kernel, qattn_fwd_q16)
  QATTN_REQUIRE(B > 0 && Lq >= 0 && Lk > 0 && Hq > 0 && Hkv > 0, QATTN_ERR_SHAPE, "sage_quant needs non-empty K / V");
  // the sm90 tables: 64-row Q blocks of 16-row warps, 128-row K blocks (as the *_ex quantizers)
  const bool sm90 = qk_quant_gran >= 4;
  if (sm90) qk_quant_gran -= 2;
  if ((Lq > 0 && ((rc = check_seq("q", q, 2)) || (rc = check_seq("q_out", q_out, 1)))) ||
      (rc = check_seq("k", k, 2)) || (rc = check_seq("v", v, 2)) || (rc = check_seq("k_out", k_out, 1)))
    return rc;
  QATTN_REQUIRE((Lq == 0 || q_scale) && k_scale && v_scale && v8 && aligned16(v8), QATTN_ERR_ARG,
                "null or misaligned output");
  QATTN_REQUIRE(!smooth_k || (k_mean && aligned16(k_mean)), QATTN_ERR_ALIGN, "smooth_k needs an aligned k_mean output");
  QATTN_REQUIRE(!smooth_v || v_mean, QATTN_ERR_ARG, "smooth_v needs a v_mean output");
  QATTN_REQUIRE(Lpad >= (Lk + 63) / 64 * 64 && Lpad % 64 == 0, QATTN_ERR_SHAPE,
                "Lpad must be a multiple of 64 and >= Lk rounded up to 64");
  QATTN_REQUIRE(workspace && workspace_bytes >= qattn_sage_quant_workspace_size(B, Lk, Hkv, D), QATTN_ERR_WORKSPACE,
                "sage_quant workspace too small");
  hipStream_t st = (hipStream_t)stream;
  const int64_t nchunk = col_chunks(Lk), BH = B * Hkv;
  float* kpart = static_cast<float*>(workspace);
  float* vpart = kpart + BH * nchunk * D;
  float* recp = vpart + 3 * BH * nchunk * D;
  const uint16_t* kp = static_cast<const uint16_t*>(k.data);
  const uint16_t* vp = static_cast<const uint16_t*>(v.data);
  uint16_t* km = static_cast<uint16_t*>(k_mean);

  // 1. column partials of K (sum) and V (max |v|, or sum / max / min), one launch
  {
    const int64_t zoff = smooth_k ? 0 : B;
    dim3 grid((unsigned)nchunk, (unsigned)Hkv, (unsigned)(2 * B - zoff));
#define QATTN_PC(F16, VM, DD)                                                                                       \
  prep_col_kernel<F16, VM, DD><<<grid, 256, 0, st>>>(kp, k.sb, k.sl, k.sh, vp, v.sb, v.sl, v.sh, Lk, Hkv, B, nchunk, \
                                                     kpart, vpart, zoff)
#define QATTN_PC2(F16, DD) \
  if (smooth_v) QATTN_PC(F16, 2, DD); else QATTN_PC(F16, 1, DD)
    if (dtype == QATTN_BF16) { if (D == 128) { QATTN_PC2(false, 128); } else { QATTN_PC2(false, 64); } }
    else { if (D == 128) { QATTN_PC2(true, 128); } else { QATTN_PC2(true, 64); } }
#undef QATTN_PC2
#undef QATTN_PC
  }
  // 2. K mean and V scales, one launch
  {
    const int64_t boff = smooth_k ? 0 : BH;
    const unsigned g = (unsigned)(2 * BH - boff);
#define QATTN_PF(F16, SV, DD) \
  prep_finalize_kernel<F16, SV, DD><<<g, DD, 0, st>>>(kpart, vpart, nchunk, Lk, BH, km, scale_max, v_scale, recp, v_mean, boff)
#define QATTN_PF2(F16, DD) \
  if (smooth_v) QATTN_PF(F16, true, DD); else QATTN_PF(F16, false, DD)
    if (dtype == QATTN_BF16) { if (D == 128) { QATTN_PF2(false, 128); } else { QATTN_PF2(false, 64); } }
    else { if (D == 128) { QATTN_PF2(true, 128); } else { QATTN_PF2(true, 64); } }
#undef QATTN_PF2
#undef QATTN_PF
  }
  // 3. V to FP8 tiles (V was read by step 1 just before: its second read finds much of it in cache)
  {
    const VTileFilter nof{nullptr, {0, 0, 0, 0}};
    launch_v_fp8(dtype, D, vp, v, Lk, B, Hkv, recp, v8, Lpad, Lpad / 64, nof, smooth_v ? v_mean : nullptr, st);
  }
  // 4. K then Q to INT8 in one launch (K first: its rows were read by step 1 as well)
  QuantArgs a{};
  a.njobs = 0;
  // per-thread scales: the Triton rounding for K (and Q); otherwise the CUDA rounding
  const int variant = qk_quant_gran == 3 ? QATTN_QUANT_TRITON_THREAD : QATTN_QUANT_CUDA;
  const void* kmean_in = smooth_k ? k_mean : nullptr;
  {
    QuantJob& J = a.job[a.njobs++];
    fill_job(J, k, k_out, B, Lk, Hkv, kmean_in, k_scale, 1.0f, 0, sm90 ? 128 : 64);
    if (qk_quant_gran == 3) {
      J.ncls = 4;
      J.cls_shift = 1;
    }
  }
  if (Lq > 0) {
    QuantJob& J = a.job[a.njobs++];
    if (qk_quant_gran == 1) {
      fill_job(J, q, q_out, B, Lq, Hq, nullptr, q_scale, q_sm_scale, 1, 128);
    } else {
      fill_job(J, q, q_out, B, Lq, Hq, nullptr, q_scale, 1.0f, 0, 32);
      warp_block_job(J, B, sm90 ? 16 : 32);
      if (qk_quant_gran == 3) {
        J.ncls = 8;
        J.cls_shift = 0;
      }
    }
  }
  if ((rc = check_launch("sage_quant"))) return rc;
  return run_quant(a, dtype, D, variant, st);
}
