/*
 * CPU restatement of the reference's SageAttention-2 quantized-attention math.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load this library, and only as the checker (or as the
 * timed "reference CPU path" baseline).  The product path never calls it.
 *
 * Reference files followed (paths relative to the TeleFuser tree):
 *   tf-kernel/csrc/sageattn2/fused/fused.cu:59-194      QuantInt8Kernel (per-block INT8 quantizer)
 *   tf-kernel/csrc/sageattn2/fused/fused.cu:332-445     MeanScaleKernel (per-channel FP8 V quantizer)
 *   tf-kernel/csrc/sageattn2/numeric_conversion.cuh:47-58,147-151  rounding semantics
 *        (cvt.rn.satfinite.e4m3x2.f32, cvt.rni.sat.s8.f32)
 *   tf-kernel/tf_kernel/triton/quant_per_block.py:22-166  Triton per-block quantizer
 *   tf-kernel/csrc/sageattn2/qattn/qk_int_sv_f8_cuda_sm89.cuh:136-470,711-840  attention main loop
 *   tf-kernel/csrc/sageattn2/qattn/attn_utils.cuh:35,316-452,469-534,711-875  update_mdo / RS_32_to_8 /
 *        accumulate_d / normalize_d
 *   tf-kernel/tf_kernel/triton/attn_qk_int8_per_block.py:46-101  Triton inner loop (bf16/fp16 P.V mode)
 *
 * Parity pins (see tests/test_oracle_kat.py): every function here is checked against closed-form
 * known-answer cases, torch's float8_e4m3fn / bfloat16 casts, brute-force float64 attention and
 * softmax invariances.  The reference ships no golden vectors for this path.
 *
 * Build: oracle/Makefile (gcc -O3 -fopenmp, no -ffast-math: IEEE division and rounding are part
 * of the bit-exact contract).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------ */
/* scalar conversions                                                                          */
/* ------------------------------------------------------------------------------------------ */

static inline float u32_as_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f32_as_u32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float oq_bf16_to_f32(uint16_t h) { return u32_as_f32(((uint32_t)h) << 16); }

float oq_f16_to_f32(uint16_t h) {
  uint32_t s = (h >> 15) & 1, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  float v;
  if (e == 0) v = ldexpf((float)m, -24);
  else if (e == 31) v = m ? NAN : INFINITY;
  else v = ldexpf((float)(m | 0x400), (int)e - 25);
  return s ? -v : v;
}

/* round-to-nearest-even fp32 -> bf16 (NaN kept quiet) */
uint16_t oq_f32_to_bf16(float f) {
  uint32_t u = f32_as_u32(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  uint32_t lsb = (u >> 16) & 1u;
  u += 0x7fffu + lsb;
  return (uint16_t)(u >> 16);
}

/* OCP E4M3FN decode: 1-4-3, bias 7, no infinities, 0x7f/0xff are NaN, max 448 */
float oq_e4m3_to_f32(uint8_t b) {
  int s = b >> 7, e = (b >> 3) & 0xf, m = b & 7;
  float v;
  if (e == 0xf && m == 7) return NAN;
  if (e == 0) v = ldexpf((float)m, -9);
  else v = ldexpf((float)(8 + m), e - 10);
  return s ? -v : v;
}

/* fp32 -> E4M3FN, round-to-nearest-even, saturate finite values to +-448 (PTX
 * cvt.rn.satfinite.e4m3x2.f32 semantics, numeric_conversion.cuh:47-58).  NaN -> 0x7f.
 * Bit-level: normals keep 3 mantissa bits with RNE on the 20 dropped bits; values below 2^-6
 * are multiples of 2^-9 (a*512 is exact, rintf is RNE; n == 8 encodes 2^-6 correctly). */
uint8_t oq_f32_to_e4m3(float f) {
  if (isnan(f)) return 0x7f;
  uint32_t u = f32_as_u32(f);
  uint8_t sign = (u >> 31) ? 0x80 : 0;
  float a = fabsf(f);
  if (a >= 448.f) return sign | 0x7e;
  if (a < 0.015625f) return sign | (uint8_t)(int)rintf(a * 512.f);
  uint32_t ua = u & 0x7fffffffu;
  int e4 = (int)(ua >> 23) - 127 + 7;
  uint32_t man = ua & 0x7fffffu;
  uint32_t m = man >> 20, rem = man & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (m & 1u))) m++;
  if (m == 8) { m = 0; e4++; }
  return sign | (uint8_t)((e4 << 3) | m);
}

/* fp32 -> IEEE half bits, round-to-nearest-even (used for the Triton fp16 K - km rounding) */
uint16_t oq_f32_to_f16(float f) {
  uint32_t u = f32_as_u32(f);
  uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  uint32_t ua = u & 0x7fffffffu;
  if (ua > 0x7f800000u) return sign | 0x7e00;
  if (ua >= 0x477ff000u) return sign | 0x7c00; /* >= 65520 rounds to inf */
  float a = fabsf(f);
  if (a < 6.103515625e-05f) return sign | (uint16_t)(int)rintf(a * 16777216.f); /* subnormal: 2^-24 steps */
  int e5 = (int)(ua >> 23) - 127 + 15;
  uint32_t man = ua & 0x7fffffu;
  uint32_t m = man >> 13, rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (m & 1u))) m++;
  if (m == 0x400u) { m = 0; e5++; }
  return sign | (uint16_t)((e5 << 10) | m);
}

/* cvt.rni.sat.s8.f32: round to nearest even, saturate to [-128, 127]; NaN -> 0 */
int8_t oq_f32_to_s8_rne_sat(float x) {
  if (isnan(x)) return 0;
  float r = rintf(x); /* default FE_TONEAREST = RNE */
  if (r > 127.f) r = 127.f;
  if (r < -128.f) r = -128.f;
  return (int8_t)r;
}

/* Triton: x += 0.5*sign(x>=0 ? 1 : -1); x.to(int8) = truncation toward zero.  NaN -> 0. */
int8_t oq_f32_to_s8_half_away(float x) {
  if (isnan(x)) return 0;
  float t = x + (x >= 0.f ? 0.5f : -0.5f);
  float r = truncf(t);
  if (r > 127.f) r = 127.f;
  if (r < -128.f) r = -128.f;
  return (int8_t)r;
}

static inline float load_h(const uint16_t* p, int is_fp16) {
  return is_fp16 ? oq_f16_to_f32(*p) : oq_bf16_to_f32(*p);
}

/* ------------------------------------------------------------------------------------------ */
/* per-block INT8 quantizers                                                                   */
/* ------------------------------------------------------------------------------------------ */

/*
 * CUDA QuantInt8Kernel semantics (fused.cu:59-194, launchers :447-696):
 *   x = float(in); if km: x -= float(km[d]); if has_sm_scale: x *= sm_scale   (fp32, in that order)
 *   tail rows (token >= L) are x = 0 and are not stored
 *   amax = max(1e-7f, max|x|); scale = amax / 127.f (IEEE); inv = 127.f / amax (IEEE)
 *   q = cvt.rni.sat.s8(x * inv)
 * Layout: element (b, l, h, d) at in[b*sb + l*sl + h*sh + d]; scale is contiguous [B, H, nblk].
 */
void oq_quant_per_block_int8(const uint16_t* in, int is_fp16, int64_t B, int64_t L, int64_t H, int64_t D,
                             int64_t sb, int64_t sl, int64_t sh, const uint16_t* km, int64_t kmb, int64_t kmh,
                             float sm_scale, int has_sm_scale, int64_t blk, int8_t* out, int64_t ob, int64_t ol,
                             int64_t oh, float* scale) {
  int64_t nblk = (L + blk - 1) / blk;
#pragma omp parallel for collapse(3) schedule(static)
  for (int64_t b = 0; b < B; b++)
    for (int64_t h = 0; h < H; h++)
      for (int64_t n = 0; n < nblk; n++) {
        float* xs = (float*)malloc(sizeof(float) * blk * D);
        float amax = 0.0000001f;
        for (int64_t r = 0; r < blk; r++) {
          int64_t l = n * blk + r;
          for (int64_t d = 0; d < D; d++) {
            float x = 0.f;
            if (l < L) {
              x = load_h(in + b * sb + l * sl + h * sh + d, is_fp16);
              if (km) x -= load_h(km + b * kmb + h * kmh + d, is_fp16);
              if (has_sm_scale) x *= sm_scale;
            }
            xs[r * D + d] = x;
            amax = fmaxf(amax, fabsf(x));
          }
        }
        volatile float a = amax;
        float sc = a / 127.0f;
        float inv = 127.0f / a;
        scale[(b * H + h) * nblk + n] = sc;
        for (int64_t r = 0; r < blk; r++) {
          int64_t l = n * blk + r;
          if (l >= L) break;
          for (int64_t d = 0; d < D; d++) {
            volatile float p = xs[r * D + d] * inv;
            out[b * ob + l * ol + h * oh + d] = oq_f32_to_s8_rne_sat(p);
          }
        }
        free(xs);
      }
}

/*
 * Triton quant_per_block_int8_kernel semantics (triton/quant_per_block.py:22-166):
 *   K path: k = k - km is a torch op on half tensors -> fp32 difference rounded to the input dtype
 *   x = float(x) * sm_scale (sm_scale = 1.0 for K); masked tail rows load as 0
 *   scale = max|x| / 127 (no floor: an all-zero block gives scale 0 and q = 0 here)
 *   q = trunc(x/scale + 0.5*sign)   (round half away from zero)
 */
void oq_quant_per_block_int8_triton(const uint16_t* in, int is_fp16, int64_t B, int64_t L, int64_t H, int64_t D,
                                    int64_t sb, int64_t sl, int64_t sh, const uint16_t* km, int64_t kmb,
                                    int64_t kmh, float sm_scale, int64_t blk, int8_t* out, int64_t ob, int64_t ol,
                                    int64_t oh, float* scale) {
  int64_t nblk = (L + blk - 1) / blk;
#pragma omp parallel for collapse(3) schedule(static)
  for (int64_t b = 0; b < B; b++)
    for (int64_t h = 0; h < H; h++)
      for (int64_t n = 0; n < nblk; n++) {
        float* xs = (float*)malloc(sizeof(float) * blk * D);
        float amax = 0.f;
        for (int64_t r = 0; r < blk; r++) {
          int64_t l = n * blk + r;
          for (int64_t d = 0; d < D; d++) {
            float x = 0.f;
            if (l < L) {
              x = load_h(in + b * sb + l * sl + h * sh + d, is_fp16);
              if (km) {
                float diff = x - load_h(km + b * kmb + h * kmh + d, is_fp16);
                if (is_fp16) {
                  x = oq_f16_to_f32(oq_f32_to_f16(diff));
                } else {
                  x = oq_bf16_to_f32(oq_f32_to_bf16(diff));
                }
              }
              volatile float xm = x * sm_scale;
              x = xm;
            }
            xs[r * D + d] = x;
            amax = fmaxf(amax, fabsf(x));
          }
        }
        volatile float a = amax;
        float sc = a / 127.0f;
        scale[(b * H + h) * nblk + n] = sc;
        for (int64_t r = 0; r < blk; r++) {
          int64_t l = n * blk + r;
          if (l >= L) break;
          for (int64_t d = 0; d < D; d++) {
            volatile float t = xs[r * D + d] / sc;
            out[b * ob + l * ol + h * oh + d] = oq_f32_to_s8_half_away(t);
          }
        }
        free(xs);
      }
}

/*
 * Triton per-thread quantizer (tf-kernel/tf_kernel/triton/quant_per_thread.py:22-158, wrapper :267-369).
 * The scale groups follow the NVIDIA mma fragment a thread holds:
 *   query (is_key = 0): 32-row warp blocks; rows r with the same r % 8 share a scale (4 rows x D);
 *     scale index = block * 8 + r % 8; the scale array has ceil(L / 128) * 4 * 8 entries per (b, h)
 *     (trailing blocks with no rows get scale 1e-7), no sm_scale folded in;
 *   key (is_key = 1): 64-row blocks; rows with the same (r % 8) / 2 share a scale (16 rows x D);
 *     scale index = block * 4 + (r % 8) / 2; ceil(L / 64) * 4 entries per (b, h).
 *   k - km is a torch op on half tensors (rounded to the input dtype, :285-286);
 *   scale = max|x| / 127 + 1e-7; q = trunc(x / scale + 0.5 * sign)  (:63-70, :145-158)
 * Masked tail rows load as 0 and do not change the max.
 */
/*
 * General form: scale blocks of blk rows (WARPQ for queries; WARPK = BLKK for keys), nblk of them per
 * (b, h) (ceil(L / BLKQ) * (BLKQ / WARPQ) for queries, ceil(L / BLKK) for keys: the grid of
 * quant_per_thread.py:317-350).  The sm90 entry calls it with BLKQ 64, WARPQ 16, BLKK = WARPK = 128
 * (sageattn2.py:1614-1624).
 */
void oq_quant_per_thread_int8_ex(const uint16_t* in, int is_fp16, int64_t B, int64_t L, int64_t H, int64_t D,
                                 int64_t sb, int64_t sl, int64_t sh, const uint16_t* km, int64_t kmb, int64_t kmh,
                                 int is_key, int64_t blk, int64_t nblk, int8_t* out, int64_t ob, int64_t ol,
                                 int64_t oh, float* scale) {
  const int64_t ncls = is_key ? 4 : 8;
#pragma omp parallel for collapse(3) schedule(static)
  for (int64_t b = 0; b < B; b++)
    for (int64_t h = 0; h < H; h++)
      for (int64_t n = 0; n < nblk; n++)
        for (int64_t c = 0; c < ncls; c++) {
          float amax = 0.f;
          for (int64_t r = 0; r < blk; r++) {
            const int64_t cls = is_key ? (r % 8) / 2 : r % 8;
            const int64_t l = n * blk + r;
            if (cls != c || l >= L) continue;
            for (int64_t d = 0; d < D; d++) {
              float x = load_h(in + b * sb + l * sl + h * sh + d, is_fp16);
              if (km) {
                float diff = x - load_h(km + b * kmb + h * kmh + d, is_fp16);
                x = is_fp16 ? oq_f16_to_f32(oq_f32_to_f16(diff)) : oq_bf16_to_f32(oq_f32_to_bf16(diff));
              }
              amax = fmaxf(amax, fabsf(x));
            }
          }
          volatile float q127 = amax / 127.0f;
          volatile float sc = q127 + 0.0000001f;
          scale[(b * H + h) * nblk * ncls + n * ncls + c] = sc;
          for (int64_t r = 0; r < blk; r++) {
            const int64_t cls = is_key ? (r % 8) / 2 : r % 8;
            const int64_t l = n * blk + r;
            if (cls != c || l >= L) continue;
            for (int64_t d = 0; d < D; d++) {
              float x = load_h(in + b * sb + l * sl + h * sh + d, is_fp16);
              if (km) {
                float diff = x - load_h(km + b * kmb + h * kmh + d, is_fp16);
                x = is_fp16 ? oq_f16_to_f32(oq_f32_to_f16(diff)) : oq_bf16_to_f32(oq_f32_to_bf16(diff));
              }
              volatile float t = x / sc;
              out[b * ob + l * ol + h * oh + d] = oq_f32_to_s8_half_away(t);
            }
          }
        }
}

void oq_quant_per_thread_int8(const uint16_t* in, int is_fp16, int64_t B, int64_t L, int64_t H, int64_t D,
                              int64_t sb, int64_t sl, int64_t sh, const uint16_t* km, int64_t kmb, int64_t kmh,
                              int is_key, int8_t* out, int64_t ob, int64_t ol, int64_t oh, float* scale) {
  oq_quant_per_thread_int8_ex(in, is_fp16, B, L, H, D, sb, sl, sh, km, kmb, kmh, is_key, is_key ? 64 : 32,
                              is_key ? (L + 63) / 64 : (L + 127) / 128 * 4, out, ob, ol, oh, scale);
}

/*
 * Prologue of the Wan self-attention projections (telefuser/models/wan_video_dit.py:196-207):
 * RMSNorm over the whole row of N = H*D values, then interleaved RoPE per head.
 *   norm (Triton norm_infer, telefuser/kernel/triton/norm.py:469-507): var = sum(x^2) / N,
 *     rstd = 1 / sqrt(var + eps), y = (x * rstd) * w stored in x's dtype.  The sum is taken exactly (fp64:
 *     the squares of half values and their sum are exact for any realistic row) and var rounded to fp32
 *     - the reference's fp32 tree sum differs from it in the last bits: parity of this step is pinned
 *     to the mathematics, not to that reduction order;
 *   rope (telefuser/kernel/triton/rotary.py:21-88): pairs (y[2i], y[2i+1]) of each head with cos/sin[l][i]
 *     (fp32): o1 = fma(-y2, sin, y1*cos), o2 = fma(y1, sin, y2*cos), stored in x's dtype.
 * x, out: [B, L, N] contiguous half bits; w: [N]; cs, sn: [L, D/2] fp32.
 */
void oq_norm_rope(const uint16_t* x, int is_fp16, int64_t B, int64_t L, int64_t N, int64_t D, const uint16_t* w,
                  const float* cs, const float* sn, float eps, uint16_t* out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; b++)
    for (int64_t l = 0; l < L; l++) {
      const uint16_t* xr = x + (b * L + l) * N;
      uint16_t* orow = out + (b * L + l) * N;
      double acc = 0.0;
      for (int64_t i = 0; i < N; i++) {
        const double v = load_h(xr + i, is_fp16);
        acc += v * v;
      }
      volatile float var = (float)(acc / (double)N);
      volatile float den = sqrtf(var + eps);
      const float rstd = 1.0f / den;
      for (int64_t i = 0; i < N; i += 2) {
        float y[2];
        for (int e = 0; e < 2; e++) {
          volatile float xr_ = load_h(xr + i + e, is_fp16) * rstd;
          volatile float yw = xr_ * load_h(w + i + e, is_fp16);
          y[e] = is_fp16 ? oq_f16_to_f32(oq_f32_to_f16(yw)) : oq_bf16_to_f32(oq_f32_to_bf16(yw));
        }
        const int64_t pair = (i % D) / 2;
        const float c = cs[l * (D / 2) + pair], s = sn[l * (D / 2) + pair];
        volatile float a = y[0] * c, bb = y[1] * c;
        const float o1 = fmaf(-y[1], s, a), o2 = fmaf(y[0], s, bb);
        orow[i] = is_fp16 ? oq_f32_to_f16(o1) : oq_f32_to_bf16(o1);
        orow[i + 1] = is_fp16 ? oq_f32_to_f16(o2) : oq_f32_to_bf16(o2);
      }
    }
}

/* ------------------------------------------------------------------------------------------ */
/* per-channel FP8 V quantizer                                                                 */
/* ------------------------------------------------------------------------------------------ */

/*
 * MeanScaleKernel<_, sub_mean=false> semantics (fused.cu:332-445):
 *   per (b, h, d): amax = max(|max_l v|, |min_l v|) over all tokens (padding zeros never change it)
 *   v_scale = amax / scale_max; recp = scale_max / amax; v8 = e4m3_rn_satfinite(v * recp)
 *   (no floor: an all-zero channel yields 0/0 = NaN, as in the reference)
 * Output here is the plain transposed layout v8[b][h][d][l] with Lpad >= L columns (pad = 0x00);
 * the device kernel's in-tile key permutation is a storage detail undone by the tests.
 */
/* Per-channel e4m3 quantization of V (MeanScaleKernel, fused.cu:332-445).  The reference reduces over the
 * tokens padded with zeros up to a multiple of 16 (fp8_padded_num_tokens, :362-366).  smooth != 0 is the
 * sub_mean form (:388-411,430-436): mean = sum / ceil16(L), amax = max(|max - mean|, |min - mean|),
 * v8 = e4m3((x - mean) * recp); the mean comes from mean_in when given (its fp32 value depends on the
 * reduction order, which the reference leaves to its block reduction), else from a float64 sum, and is
 * written to mean_out.  Key slots past L are written as zero. */
void oq_per_channel_fp8_ex(const uint16_t* in, int is_fp16, int64_t B, int64_t L, int64_t H, int64_t D, int64_t sb,
                           int64_t sl, int64_t sh, float scale_max, int smooth, const float* mean_in, float* mean_out,
                           uint8_t* v8, int64_t Lpad, float* v_scale) {
  const int64_t l16 = (L + 15) / 16 * 16;
#pragma omp parallel for collapse(3) schedule(static)
  for (int64_t b = 0; b < B; b++)
    for (int64_t h = 0; h < H; h++)
      for (int64_t d = 0; d < D; d++) {
        float mx = -1000000.0f, mn = 1000000.0f;
        double sum = 0.0;
        for (int64_t l = 0; l < L; l++) {
          float x = load_h(in + b * sb + l * sl + h * sh + d, is_fp16);
          mx = fmaxf(mx, x);
          mn = fminf(mn, x);
          sum += x;
        }
        if (l16 > L) {
          mx = fmaxf(mx, 0.f);
          mn = fminf(mn, 0.f);
        }
        const int64_t i = (b * H + h) * D + d;
        volatile float mean = 0.f;
        volatile float amax;
        if (smooth) {
          mean = mean_in ? mean_in[i] : (float)(sum / (double)l16);
          if (mean_out) mean_out[i] = mean;
          volatile float a1 = mx - mean, a2 = mn - mean;
          amax = fmaxf(fabsf(a1), fabsf(a2));
        } else {
          amax = fmaxf(fabsf(mx), fabsf(mn));
        }
        v_scale[i] = amax / scale_max;
        volatile float recp = scale_max / amax;
        uint8_t* row = v8 + i * Lpad;
        for (int64_t l = 0; l < Lpad; l++) {
          if (l >= L) {
            row[l] = 0;
            continue;
          }
          volatile float x = load_h(in + b * sb + l * sl + h * sh + d, is_fp16);
          if (smooth) x = x - mean;
          volatile float y = x * recp;
          row[l] = oq_f32_to_e4m3(y);
        }
      }
}

void oq_per_channel_fp8(const uint16_t* in, int is_fp16, int64_t B, int64_t L, int64_t H, int64_t D, int64_t sb,
                        int64_t sl, int64_t sh, float scale_max, uint8_t* v8, int64_t Lpad, float* v_scale) {
  oq_per_channel_fp8_ex(in, is_fp16, B, L, H, D, sb, sl, sh, scale_max, 0, NULL, NULL, v8, Lpad, v_scale);
}

/* ------------------------------------------------------------------------------------------ */
/* quantized attention forward                                                                 */
/* ------------------------------------------------------------------------------------------ */

#define OQ_FP8_OFFSET 8.807 /* attn_utils.cuh:35 S_FP8_OFFSET */

/*
 * Quantized attention with the reference's tile structure (qk_int_sv_f8_cuda_sm89.cuh:342-840):
 *   for each 64-key tile (blkk):  s = float(Q8.K8^T) * (q_scale * k_scale) * qk_mult
 *     m_new = max(m, rowmax(s) - offset);  p = exp2(s - m_new);  d = d*exp2(m - m_new) + sum(p)
 *     pv_mode 0: O = O*exp2(m-m_new) + e4m3(p) . e4m3(V)   (offset = 8.807, V per-channel fp8)
 *     pv_mode 1: O = O*exp2(m-m_new) + half(p) . Vh         (offset = 0, V = bf16/fp16 input values,
 *                P rounded to the same half type as V)
 *   end: O /= d; pv_mode 0: O *= v_scale[d]
 * Everything not rounded by the reference is carried in double.
 *
 * q8: element (b,l,h,d) at q8[b*qsb + l*qsl + h*qsh + d]; k8 likewise with ks*.
 * Scale granularity (the reference's QuantGranularity codes, attn_utils.cuh:41-64):
 *   q_gran 1: q_scale [B,Hq,nQB] with block blkq;  2 (per warp): one scale per 32 rows, ceil(Lq/128)*4
 *   entries;  3 (per thread): (row / 32) * 8 + row % 8, ceil(Lq/128)*32 entries.
 *   k_gran 1 / 2: k_scale [B,Hkv,nKB] one per key tile (blkk);  3: tile * 4 + (key % 8) / 2, nKB*4 entries.
 *   (per-warp K is per-block K; quant_per_thread.py:267-369, fused.cu:698-780.)
 *   The sm90 entry's tables (BLKQ 64, WARPQ 16, BLKK = WARPK 128; sageattn2.py:1608-1624):
 *   q_gran 4 (per warp): row / 16, ceil(Lq/64)*4 entries;  5 (per thread): (row / 16) * 8 + row % 8,
 *   ceil(Lq/64)*32 entries;  k_gran 4: key / 128, ceil(Lk/128) entries;  5: (key / 128) * 4 + (key % 8) / 2,
 *   ceil(Lk/128)*4 entries.
 * pv_mode 0: v8 is the plain transposed [B,Hkv,D,Lpad] e4m3 tensor, v_scale [B,Hkv,D].
 * pv_mode 1: vh is (b,l,h,d) at vh[b*vsb + l*vsl + h*vsh + d] (bf16 or fp16 bits).
 * kv_valid: per-batch number of valid keys (NULL = Lk); causal: top-left aligned kv > q + q_offset masked.
 * out: float [B, Lq, Hq, D] contiguous; lse2 (optional): log2-domain row LSE [B, Hq, Lq] of the
 * quantized logits (log2(d) + m).
 * If qrows_limit > 0 only the first qrows_limit query rows of every (b, h) are computed (CPU timing).
 * lazy_tau >= 0 restates the lazy running-max rule of the device kernel: m moves to rowmax(s) -
 * (offset - tau) only when that exceeds the current m by more than tau (p stays <= 2^offset);
 * lazy_tau < 0 is the reference rule m = max(m, rowmax(s) - offset) of update_mdo.
 * lsum_rounded != 0 sums the rounded P (what the device kernel's MFMA row sum computes) instead of
 * the unrounded p the reference's accumulate_d sums.
 * p_linear != 0 (pv_mode 0) restates the device kernels' P: oq_p_linear_byte(s - m) read as e4m3, no exp2.
 * tiles_per_split > 0 restates the KV-split schedule: every run of tiles_per_split key tiles keeps its
 * own (m, d, O) and the partials are merged at the end with weights exp2(m_s - max m).
 *
 * Loop order: (b, h, 128-row query block) x key tile, with the tile's V decoded once into floats, so the
 * same code doubles as the timed CPU baseline.
 */
/*
 * The FP8 P of the device kernels (attn.hip p_e4m3_x4): the byte k = RNE(8 (x - 0.057539) + 56), clamped to
 * [0, 255] (v_cvt_pk_u8_f32), taken as an e4m3 encoding.  For y = x - 0.057539 the byte holds exponent
 * field floor(y) + 7 and mantissa round(8 frac(y)): 2^floor(y) (1 + frac(y)) on the e4m3 grid, the linear
 * interpolation of 2^y between powers of two (Schraudolph, Neural Computation 11, 1999).  0.057539 =
 * log2(1.040685), the mean of (1 + f) / 2^f over f in [0, 1).
 */
static uint8_t oq_p_linear_byte(double x) {
  const double u = 8.0 * (x - 0.057539) + 56.0;
  if (!(u > 0.0)) return 0;
  if (u >= 255.0) return 255;
  return (uint8_t)nearbyint(u); /* default rounding mode: ties to even */
}

void oq_qattn_fwd(const int8_t* q8, int64_t qsb, int64_t qsl, int64_t qsh, const float* q_scale, int64_t blkq,
                  const int8_t* k8, int64_t ksb, int64_t ksl, int64_t ksh, const float* k_scale, int64_t blkk,
                  const uint8_t* v8, int64_t Lpad, const float* v_scale, const uint16_t* vh, int is_fp16,
                  int64_t vsb, int64_t vsl, int64_t vsh, int64_t B, int64_t Lq, int64_t Lk, int64_t Hq,
                  int64_t Hkv, int64_t D, double qk_mult, int pv_mode, int causal, int64_t q_offset,
                  const int32_t* kv_valid, int64_t h_begin, int64_t h_end, int64_t qrows_limit, int64_t tiles_per_split,
                  double lazy_tau, int lsum_rounded, int q_gran, int k_gran, const int8_t* tile_mask, int64_t tm_s1,
                  int64_t tm_s2, const float* v_mean, int pv_f16_tile, int p_linear, float* out, float* lse2) {
  const int64_t RB = 128; /* query rows per work item */
  int64_t nQB = (Lq + blkq - 1) / blkq;
  int64_t nKB = (Lk + blkk - 1) / blkk;
  /* scale entries per (b, h): per-block / per-warp (32 rows) / per-thread (32-row block x 8 classes) */
  const int64_t nQS = q_gran == 5   ? (Lq + 63) / 64 * 32
                      : q_gran == 4 ? (Lq + 63) / 64 * 4
                      : q_gran == 3 ? (Lq + 127) / 128 * 32
                      : q_gran == 2 ? (Lq + 127) / 128 * 4
                                    : nQB;
  const int64_t nKS = k_gran == 5 ? (Lk + 127) / 128 * 4 : k_gran == 4 ? (Lk + 127) / 128 : k_gran == 3 ? nKB * 4 : nKB;
  int64_t group = Hq / Hkv;
  int64_t rows = qrows_limit > 0 && qrows_limit < Lq ? qrows_limit : Lq;
  int64_t nRB = (rows + RB - 1) / RB;
  if (h_end <= 0 || h_end > Hq) h_end = Hq;
  if (tiles_per_split <= 0) tiles_per_split = nKB > 0 ? nKB : 1;
  double offset = pv_mode == 0 ? OQ_FP8_OFFSET : 0.0;
#pragma omp parallel for collapse(3) schedule(dynamic, 1)
  for (int64_t b = 0; b < B; b++)
    for (int64_t h = h_begin; h < h_end; h++)
      for (int64_t rb = 0; rb < nRB; rb++) {
        int64_t hk = h / group;
        int64_t i0 = rb * RB, i1 = i0 + RB < rows ? i0 + RB : rows, nr = i1 - i0;
        int64_t valid = kv_valid ? kv_valid[b] : Lk;
        if (valid > Lk) valid = Lk;
        double* o = (double*)calloc((size_t)(nr * D), sizeof(double));   /* current split */
        double* oacc = (double*)calloc((size_t)(nr * D), sizeof(double)); /* merged splits */
        double* m = (double*)malloc(sizeof(double) * nr);
        double* dsum = (double*)malloc(sizeof(double) * nr);
        double* macc = (double*)malloc(sizeof(double) * nr);
        double* dacc = (double*)calloc((size_t)nr, sizeof(double));
        int* has = (int*)calloc((size_t)nr, sizeof(int));
        int* hasacc = (int*)calloc((size_t)nr, sizeof(int));
        double* vt = (double*)malloc(sizeof(double) * blkk * D);
        double s[1024];
        /* key tiles this query block visits, in order: all of them, or the ones the block-sparse mask
         * keeps (sparse_int8_attn.py:57-58); KV splits group consecutive visited tiles */
        int64_t* act = (int64_t*)malloc(sizeof(int64_t) * (nKB > 0 ? nKB : 1));
        int64_t nact = 0;
        for (int64_t t = 0; t < nKB && t * blkk < valid; t++)
          if (!tile_mask || tile_mask[(b * Hkv + hk) * tm_s1 + (i0 / RB) * tm_s2 + t]) act[nact++] = t;
        const int64_t tps = tiles_per_split < nKB ? tiles_per_split : (nKB > 0 ? nKB : 1);
        for (int64_t r = 0; r < nr; r++) macc[r] = -INFINITY;
        for (int64_t a0 = 0; a0 < nact; a0 += tps) {
          int64_t a1 = a0 + tps < nact ? a0 + tps : nact;
          for (int64_t r = 0; r < nr; r++) { m[r] = -5000000.0; dsum[r] = 0.0; has[r] = 0; }
          memset(o, 0, sizeof(double) * nr * D);
          for (int64_t ai = a0; ai < a1; ai++) {
            const int64_t t = act[ai];
            int64_t k0 = t * blkk, kend = k0 + blkk < valid ? k0 + blkk : valid;
            const float* ksrow = k_scale + (b * Hkv + hk) * nKS;
            for (int64_t j = k0; j < kend; j++)
              for (int64_t d = 0; d < D; d++) {
                double vv;
                if (pv_mode == 0) vv = oq_e4m3_to_f32(v8[((b * Hkv + hk) * D + d) * Lpad + j]);
                else vv = load_h(vh + b * vsb + j * vsl + hk * vsh + d, is_fp16);
                vt[(j - k0) * D + d] = vv;
              }
            for (int64_t r = 0; r < nr; r++) {
              int64_t i = i0 + r;
              int64_t k1 = kend;
              if (causal && i + q_offset + 1 < k1) k1 = i + q_offset + 1;
              if (k1 <= k0) continue;
              const int8_t* qrow = q8 + b * qsb + i * qsl + h * qsh;
              const int64_t qi = q_gran == 5   ? (i / 16) * 8 + i % 8
                                 : q_gran == 4 ? i / 16
                                 : q_gran == 3 ? (i / 32) * 8 + i % 8
                                 : q_gran == 2 ? i / 32
                                               : i / blkq;
              const double qsv = (double)q_scale[(b * Hq + h) * nQS + qi];
              double mx = -1e300;
              for (int64_t j = k0; j < k1; j++) {
                const int8_t* krow = k8 + b * ksb + j * ksl + hk * ksh;
                int32_t acc = 0;
                for (int64_t d = 0; d < D; d++) acc += (int32_t)qrow[d] * (int32_t)krow[d];
                const double ks = ksrow[k_gran == 5   ? (j / 128) * 4 + (j % 8) / 2
                                        : k_gran == 4 ? j / 128
                                        : k_gran == 3 ? t * 4 + (j % 8) / 2
                                                      : t];
                s[j - k0] = (double)acc * (qsv * ks * qk_mult);
                if (s[j - k0] > mx) mx = s[j - k0];
              }
              double m_new;
              if (lazy_tau < 0) {
                m_new = mx - offset > m[r] ? mx - offset : m[r];
              } else { /* lazy rule: move m only when the tile max exceeds it by more than tau */
                double mt = mx - (offset - lazy_tau);
                m_new = (!has[r] || mt > m[r] + lazy_tau) ? mt : m[r];
              }
              double alpha = has[r] ? exp2(m[r] - m_new) : 0.0;
              double* orow = o + r * D;
              dsum[r] *= alpha;
              for (int64_t d = 0; d < D; d++) orow[d] *= alpha;
              m[r] = m_new;
              has[r] = 1;
              double part[2][128];
              if (pv_f16_tile) memset(part, 0, sizeof(part));
              for (int64_t j = k0; j < k1; j++) {
                double p = exp2(s[j - k0] - m_new);
                double pr = pv_mode == 0 ? oq_e4m3_to_f32(oq_f32_to_e4m3((float)p))
                            : is_fp16   ? oq_f16_to_f32(oq_f32_to_f16((float)p))
                                        : oq_bf16_to_f32(oq_f32_to_bf16((float)p));
                if (pv_mode == 0 && p_linear) pr = oq_e4m3_to_f32(oq_p_linear_byte(s[j - k0] - m_new));
                dsum[r] += lsum_rounded ? pr : p;
                const double* vr = vt + (j - k0) * D;
                if (pv_f16_tile) {
                  double* pp = part[(j - k0) >= 32];
                  for (int64_t d = 0; d < D; d++) pp[d] += pr * vr[d];
                } else {
                  for (int64_t d = 0; d < D; d++) orow[d] += pr * vr[d];
                }
              }
              if (pv_f16_tile) {
                /* the tile's P.V as two k = 32 MMAs with an fp16 accumulator (compute_fp8_sv_inst_buf_fp16_accu,
                 * attn_utils.cuh:886-953): each MMA's sum rounded to fp16, then added to the fp32 O */
                for (int64_t d = 0; d < D; d++) {
                  const float a = oq_f16_to_f32(oq_f32_to_f16((float)part[0][d]));
                  const float b2 = oq_f16_to_f32(oq_f32_to_f16((float)(a + part[1][d])));
                  orow[d] += b2;
                }
              }
            }
          }
          /* merge this split into the accumulator */
          for (int64_t r = 0; r < nr; r++) {
            if (!has[r]) continue;
            double M = m[r] > macc[r] ? m[r] : macc[r];
            double fa = hasacc[r] ? exp2(macc[r] - M) : 0.0, fs = exp2(m[r] - M);
            dacc[r] = dacc[r] * fa + dsum[r] * fs;
            for (int64_t d = 0; d < D; d++) oacc[r * D + d] = oacc[r * D + d] * fa + o[r * D + d] * fs;
            macc[r] = M;
            hasacc[r] = 1;
          }
        }
        for (int64_t r = 0; r < nr; r++) {
          int64_t i = i0 + r;
          float* orow = out + ((b * Lq + i) * Hq + h) * D;
          for (int64_t d = 0; d < D; d++) {
            double v = hasacc[r] && dacc[r] > 0 ? oacc[r * D + d] / dacc[r] : 0.0;
            if (pv_mode == 0) v *= (double)v_scale[(b * Hkv + hk) * D + d];
            if (pv_mode == 0 && v_mean) v += (double)v_mean[(b * Hkv + hk) * D + d];
            orow[d] = (float)v;
          }
          if (lse2) lse2[(b * Hq + h) * Lq + i] = hasacc[r] && dacc[r] > 0 ? (float)(log2(dacc[r]) + macc[r]) : -INFINITY;
        }
        free(o); free(oacc); free(m); free(dsum); free(macc); free(dacc); free(has); free(hasacc); free(vt); free(act);
      }
}

/* float64 exact softmax attention on half inputs (the unquantized truth), same layouts as above. */
void oq_attn_fp64(const uint16_t* q, const uint16_t* k, const uint16_t* v, int is_fp16, int64_t B, int64_t Lq,
                  int64_t Lk, int64_t Hq, int64_t Hkv, int64_t D, double sm_scale, int causal, int64_t q_offset,
                  const int32_t* kv_valid, float* out) {
  int64_t group = Hq / Hkv;
#pragma omp parallel for collapse(3) schedule(dynamic, 4)
  for (int64_t b = 0; b < B; b++)
    for (int64_t h = 0; h < Hq; h++)
      for (int64_t i = 0; i < Lq; i++) {
        int64_t hk = h / group;
        int64_t last = kv_valid ? kv_valid[b] : Lk;
        if (last > Lk) last = Lk;
        if (causal && i + q_offset + 1 < last) last = i + q_offset + 1;
        double* s = (double*)malloc(sizeof(double) * (Lk > 0 ? Lk : 1));
        double* o = (double*)calloc((size_t)D, sizeof(double));
        double mx = -1e300;
        for (int64_t j = 0; j < last; j++) {
          double acc = 0;
          for (int64_t d = 0; d < D; d++)
            acc += (double)load_h(q + ((b * Lq + i) * Hq + h) * D + d, is_fp16) *
                   (double)load_h(k + ((b * Lk + j) * Hkv + hk) * D + d, is_fp16);
          s[j] = acc * sm_scale;
          if (s[j] > mx) mx = s[j];
        }
        double den = 0;
        for (int64_t j = 0; j < last; j++) {
          double p = exp(s[j] - mx);
          den += p;
          for (int64_t d = 0; d < D; d++) o[d] += p * (double)load_h(v + ((b * Lk + j) * Hkv + hk) * D + d, is_fp16);
        }
        for (int64_t d = 0; d < D; d++) out[((b * Lq + i) * Hq + h) * D + d] = last > 0 ? (float)(o[d] / den) : 0.f;
        free(s);
        free(o);
      }
}

int oq_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Threads that actually run an OpenMP parallel region (for the CPU-baseline report), and a setter for the
 * thread count of later regions (n <= 0 leaves it unchanged). */
int oq_parallel_threads(void) {
  int n = 1;
#ifdef _OPENMP
#pragma omp parallel
  {
#pragma omp single
    n = omp_get_num_threads();
  }
#endif
  return n;
}

void oq_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* Element-wise conversions over an array (kind 0: e4m3 bytes, 1: bf16 bits, 2: s8 RNE-sat,
 * 3: s8 half-away (Triton), 4: fp16 bits).  Lets tests sweep millions of values in one call. */
void oq_cvt_array(const float* x, int64_t n, int kind, void* out) {
  for (int64_t i = 0; i < n; i++) {
    switch (kind) {
      case 0: ((uint8_t*)out)[i] = oq_f32_to_e4m3(x[i]); break;
      case 1: ((uint16_t*)out)[i] = oq_f32_to_bf16(x[i]); break;
      case 2: ((int8_t*)out)[i] = oq_f32_to_s8_rne_sat(x[i]); break;
      case 3: ((int8_t*)out)[i] = oq_f32_to_s8_half_away(x[i]); break;
      default: ((uint16_t*)out)[i] = oq_f32_to_f16(x[i]); break;
    }
  }
}
