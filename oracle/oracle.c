/* oracle.c -- CPU restatement of the PULSAR-ASM hot path (test infrastructure).
 *
 * ONLY tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load this library, and only as the test reference / CPU baseline. The product
 * (pulsar-asm_amd/) never links or calls it.
 *
 * Citations are relative to the PULSAR-ASM tree. The orders the build defines
 * itself (R1 GEMV, split-K flash decode, pairwise norm tree) are spelled out at
 * each function; the HIP kernels implement the same orders bit for bit.
 *
 * Compiled with -ffp-contract=off: every fused multiply-add is an explicit
 * fmaf(), every other a*b+c rounds twice.
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>

/* The OpenMP team size the oracle's parallel loops use (reported beside the CPU baseline). */
int orc_max_threads(void) { return omp_get_max_threads(); }
#endif

/* ===================================================================== scalars */

/* bf16 -> f32: the bf16 bits are the top half of the f32 (lfm3_nanode.cu:115). */
float orc_bf2f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* f32 -> bf16 round-to-nearest-even; inf/nan pass their top half through
 * (lfm3_nanode.cu:116-121, lfm3_elem_test.c:26-31). Pinned by: closed-form
 * cases in test_oracle_scalars (ties to even, carry into the exponent). */
uint16_t orc_f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if (((u >> 23) & 0xffu) == 0xffu) return (uint16_t)(u >> 16);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

/* binary16 -> f32, exact (pq2_host.c:9-20 pq2_h2f). Pinned by: numpy float16
 * conversion over all 65536 bit patterns. */
float orc_h2f(uint16_t h) {
  const uint32_t s = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t o;
  if (e == 0) {
    if (m == 0) { o = s; }
    else {
      float f = (float)m * 5.9604644775390625e-8f;      /* m * 2^-24, exact */
      memcpy(&o, &f, 4);
      o |= s;
    }
  } else if (e == 31) {
    o = s | 0x7f800000u | (m << 13);
  } else {
    o = s | ((e + 112u) << 23) | (m << 13);
  }
  float r;
  memcpy(&r, &o, 4);
  return r;
}

/* f32 -> binary16, IEEE round-to-nearest-even, subnormals kept, overflow to
 * inf. Written from the binary16 definition (IEEE 754-2008 3.6). Pinned by:
 * numpy float32->float16 casts over random and edge patterns. */
uint16_t orc_f2h(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u;
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u)                                 /* inf / nan */
    return (uint16_t)(sign | 0x7c00u | (a > 0x7f800000u ? (0x200u | ((a >> 13) & 0x3ffu)) : 0u));
  if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);   /* >= 65520 rounds to inf */
  if (a < 0x38800000u) {                                 /* below 2^-14: subnormal */
    if (a < 0x33000000u) return (uint16_t)sign;          /* < 2^-25 -> 0 */
    const uint32_t e = a >> 23, m = (a & 0x7fffffu) | 0x800000u;
    const uint32_t sh = 126u - e;                        /* 14..24 */
    uint32_t q = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
  }
  const uint32_t r = a - 0x38000000u;                    /* rebias 127 -> 15 */
  uint32_t q = r >> 13;
  const uint32_t rem = r & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
  return (uint16_t)(sign | q);
}

/* e^x shared by softmax, silu and the sigmoid gate; the device kernels carry
 * the same function. Method: Cody & Waite argument reduction (Cody, Waite,
 * "Software Manual for the Elementary Functions", 1980, ch. 6):
 *   n = rint(x * log2(e)), r = (x - n*ln2_hi) - n*ln2_lo  (two fmaf),
 * e^r from the degree-7 Taylor polynomial sum r^k/k! in Horner form (fmaf),
 * |r| <= ln2/2 so the truncation error is < r^8/8! = 5.3e-9 relative.
 * 2^n is applied as two exact power-of-two factors 2^(n/2) * 2^(n-n/2), so
 * only the final multiply rounds (also into the subnormal range).
 * Pinned by: |orc_expf - exp| <= 2 ulp over a dense sweep (test_oracle_scalars).
 * The reference calls CUDA's expf (lfm3_nanode.cu:824, 578); a CPU/GPU pair
 * must share one definition to be bit-identical, hence this one. */
float orc_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -104.0f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(n, -0.693145751953125f, x);
  r = fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.98412698412698412e-4f;             /* 1/7! */
  p = fmaf(p, r, 1.38888888888888889e-3f);       /* 1/6! */
  p = fmaf(p, r, 8.33333333333333333e-3f);       /* 1/5! */
  p = fmaf(p, r, 4.16666666666666667e-2f);       /* 1/4! */
  p = fmaf(p, r, 1.66666666666666667e-1f);       /* 1/3! */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int a = ni / 2, b = ni - a;
  uint32_t ua = (uint32_t)(a + 127) << 23, ub = (uint32_t)(b + 127) << 23;
  float fa, fb;
  memcpy(&fa, &ua, 4);
  memcpy(&fb, &ub, 4);
  return (p * fa) * fb;
}

/* =================================================================== generator
 * splitmix64 (Steele, Lea, Flood, "Fast splittable pseudorandom number
 * generators", OOPSLA 2014): output n of a stream seeded with `seed` is
 * mix(seed + (n+1)*GAMMA), so any element can be generated independently and
 * a tensor is generated in parallel. The product's synthetic-model generator
 * restates the same definition; test_synth checks they agree bit for bit.
 *   codes:   element i = 16-bit lane i%4 of word i/4, c = (u16*255)>>16 - 127
 *   normal:  word i -> u1 = (hi32+1)/2^32, u2 = lo32/2^32,
 *            z = sqrt(-2 ln u1) cos(2 pi u2) in double, rounded to float
 *   scales:  f16(fl(|z| * mult))
 *   ternary: code i = byte i%8 of word i/8, c = (u8*3)>>8 in {0,1,2}
 * The reference generates its fixtures in-process too (xorshift32 in
 * q8_gemv_neon_test.c:57-65, LCG in pq1t_parity.c:13-14). */
#define SM_GAMMA 0x9e3779b97f4a7c15ull
static inline uint64_t sm_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
uint64_t orc_sm64_at(uint64_t seed, uint64_t n) { return sm_mix(seed + (n + 1) * SM_GAMMA); }

void orc_gen_codes(uint64_t seed, int8_t *out, size_t n) {
  const size_t nw = (n + 3) / 4;
#pragma omp parallel for schedule(static)
  for (size_t w = 0; w < nw; w++) {
    const uint64_t v = orc_sm64_at(seed, w);
    for (int k = 0; k < 4; k++) {
      const size_t i = w * 4 + (size_t)k;
      if (i < n) out[i] = (int8_t)((int)((((v >> (16 * k)) & 0xffffu) * 255u) >> 16) - 127);
    }
  }
}

static inline float sm_normal(uint64_t v) {
  const double u1 = ((double)(v >> 32) + 1.0) * (1.0 / 4294967296.0);
  const double u2 = (double)(v & 0xffffffffu) * (1.0 / 4294967296.0);
  return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925 * u2));
}

void orc_gen_normal(uint64_t seed, float *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; i++) out[i] = sm_normal(orc_sm64_at(seed, i));
}

void orc_gen_scales(uint64_t seed, uint16_t *out, size_t n, float mult) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; i++) out[i] = orc_f2h(fabsf(sm_normal(orc_sm64_at(seed, i))) * mult);
}

void orc_gen_affine(uint64_t seed, float *out, size_t n, float a, float b) {
  for (size_t i = 0; i < n; i++) out[i] = a + b * sm_normal(orc_sm64_at(seed, i));
}

void orc_gen_ternary(uint64_t seed, uint8_t *out, size_t nbytes) {
#pragma omp parallel for schedule(static)
  for (size_t by = 0; by < nbytes; by++) {
    uint8_t o = 0;
    for (int k = 0; k < 4; k++) {
      const size_t i = by * 4 + (size_t)k;
      const uint64_t v = orc_sm64_at(seed, i / 8);
      const uint32_t u8 = (uint32_t)(v >> (8 * (i % 8))) & 0xffu;
      o |= (uint8_t)(((u8 * 3u) >> 8) << (2 * k));
    }
    out[by] = o;
  }
}

void orc_gen_tokens(uint64_t seed, int32_t *out, int n, int vocab) {
  for (int i = 0; i < n; i++) out[i] = (int32_t)((orc_sm64_at(seed, (uint64_t)i) >> 32) % (uint64_t)vocab);
}

/* ================================================================= quantizers */

/* Q8_0 activation quantizer, one row of K (K % 32 == 0). Per 32-block:
 *   amax = max|x_j|, d = fl(amax / 127), q_j = rne(fl(x_j / d)) clamped to
 *   [-127,127]; d == 0 writes q = 0 and d = 0.
 * This is the Q8_0 rule of q8_gemv_cpu.c:63-81 (quant_row) with an fp32
 * scale (export_lfm3_q8.py:50-66 keeps fp32 scales) and rne = lrintf there /
 * np.round there. Pinned by: closed-form cases (|q| <= 127, the amax element
 * maps to +-127, all-zero block) and |q*d - x| <= d/2 on random rows. */
void orc_q8_quant(const float *x, int K, int8_t *qx, float *dx) {
  for (int b = 0; b < K / ORC_QBLK; b++) {
    const float *xb = x + (size_t)b * ORC_QBLK;
    float amax = 0.0f;
    for (int j = 0; j < ORC_QBLK; j++) { const float a = fabsf(xb[j]); if (a > amax) amax = a; }
    const float d = amax / 127.0f;
    dx[b] = d;
    for (int j = 0; j < ORC_QBLK; j++) {
      int v = 0;
      if (d != 0.0f) {
        v = (int)rintf(xb[j] / d);
        if (v > 127) v = 127;
        if (v < -127) v = -127;
      }
      qx[(size_t)b * ORC_QBLK + j] = (int8_t)v;
    }
  }
}

void orc_q8_quant_bf16(const uint16_t *x, int K, int8_t *qx, float *dx) {
  float buf[ORC_QBLK];
  for (int b = 0; b < K / ORC_QBLK; b++) {
    for (int j = 0; j < ORC_QBLK; j++) buf[j] = orc_bf2f(x[(size_t)b * ORC_QBLK + j]);
    orc_q8_quant(buf, ORC_QBLK, qx + (size_t)b * ORC_QBLK, dx + b);
  }
}

/* Q8_K activation quantizer (fwd8.c:61-137, the fork's quantize_row_q8_K_ref):
 * per 256-block, max = x at the FIRST index reaching amax (strict-> scan),
 * iscale = -127/max, q = min(127, nearest_int(iscale*x)) where nearest_int is
 * the 1.5*2^23 magic add (fwd8.c:63-67), 16 int16 bsums, d = 1/iscale.
 * All-zero block: d = 0 and qs = 0 (the fork leaves bsums stale; here they
 * are zeroed -- the GEMV never reads them). */
static inline int orc_nearest_int(float fval) {
  const float val = fval + 12582912.f;
  int32_t i;
  memcpy(&i, &val, 4);
  return (i & 0x007fffff) - 0x00400000;
}
void orc_q8k_quant(const float *x, int K, uint8_t *out) {
  for (int bk = 0; bk < K / ORC_Q8K_BLK; bk++) {
    const float *xb = x + (size_t)bk * ORC_Q8K_BLK;
    uint8_t *yb = out + (size_t)bk * ORC_Q8K_BYTES;
    int8_t *qs = (int8_t *)(yb + 4);
    int16_t bs[16];
    float amax = 0.0f, max = 0.0f;
    for (int j = 0; j < ORC_Q8K_BLK; j++) {
      const float ax = fabsf(xb[j]);
      if (ax > amax) { amax = ax; max = xb[j]; }
    }
    if (amax == 0.0f) {
      memset(yb, 0, ORC_Q8K_BYTES);
      continue;
    }
    const float iscale = -127.f / max;
    for (int j = 0; j < ORC_Q8K_BLK; j++) {
      int v = orc_nearest_int(iscale * xb[j]);
      qs[j] = (int8_t)(v < 127 ? v : 127);
    }
    for (int g = 0; g < 16; g++) {
      int s = 0;
      for (int i = 0; i < 16; i++) s += qs[g * 16 + i];
      bs[g] = (int16_t)s;
    }
    memcpy(yb + 4 + 256, bs, 32);
    const float d = 1.0f / iscale;
    memcpy(yb, &d, 4);
  }
}

/* ================================================================ GEMV / GEMM */

static inline int32_t blk_dot(const int8_t *w, const int8_t *x) {
  int32_t s = 0;
  for (int j = 0; j < ORC_QBLK; j++) s += (int32_t)w[j] * (int32_t)x[j];
  return s;
}

/* Q8_0 x Q8_0 GEMV in the R1 order, one output row:
 *   isum_b = sum_j W[32b+j]*qx[32b+j]                (int32, exact)
 *   s_b    = fl(f16tof32(S_b) * dx_b)
 *   chunk c = blocks [8c, min(8c+8, nb)):  a = 0; a = fmaf(s_b, (float)isum_b, a)
 *   y = 0; y = fl(y + a_c) for c ascending
 * The per-block scale fused into the accumulator mirrors the reference's
 * acc = fmaf(s_b, dot, acc) (lfm3_nanode.cu:312-323); the chunk partials
 * combined ascending from 0 mirror KCHUNK + k_combine_* (lfm3_nanode.cu:
 * 1763, 336-374). The int8 x int8 block dot with an fp32 scale chain is the
 * pattern of pq2_host.c:100. Pinned by: exact int64/double recomputation on
 * random inputs (<= 1e-5 relative to sum|terms|), the reference's own A11
 * loop (oracle/_ref, q8_gemv_cpu.c) within 1e-5 on dequantized x, and
 * hand-computed single-block / single-chunk cases. */
static float q8_row_r1(const int8_t *w, const uint16_t *s, const int8_t *qx, const float *dx,
                       int K) {
  const int nb = K / ORC_QBLK;
  float y = 0.0f;
  for (int c0 = 0; c0 < nb; c0 += ORC_CHUNK) {
    const int c1 = c0 + ORC_CHUNK < nb ? c0 + ORC_CHUNK : nb;
    float a = 0.0f;
    for (int b = c0; b < c1; b++) {
      const int32_t is = blk_dot(w + (size_t)b * ORC_QBLK, qx + (size_t)b * ORC_QBLK);
      const float sb = orc_h2f(s[b]) * dx[b];
      a = fmaf(sb, (float)is, a);
    }
    y = y + a;
  }
  return y;
}

void orc_q8_gemv(const int8_t *W, const uint16_t *S, const int8_t *qx, const float *dx,
                 float *y, int N, int K) {
  const int nb = K / ORC_QBLK;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < N; r++)
    y[r] = q8_row_r1(W + (size_t)r * K, S + (size_t)r * nb, qx, dx, K);
}

/* T positions against one weight stream: y[t][r] is exactly orc_q8_gemv of
 * position t (the batched == per-position invariant of prefill_chunk_test,
 * lfm3_nanode.cu:3020-3106). Row-outer so each weight row is reused from cache. */
void orc_q8_gemm(const int8_t *W, const uint16_t *S, const int8_t *qx, const float *dx,
                 float *y, int N, int K, int T) {
  const int nb = K / ORC_QBLK;
#pragma omp parallel for schedule(dynamic, 16)
  for (int r = 0; r < N; r++)
    for (int t = 0; t < T; t++)
      y[(size_t)t * N + r] = q8_row_r1(W + (size_t)r * K, S + (size_t)r * nb,
                                       qx + (size_t)t * K, dx + (size_t)t * nb, K);
}

/* A11: the reference's CPU Q8 GEMV (q8_gemv_cpu.c:29-58): fp32 x, per block
 * p += q_j * x_j for j ascending (32 unfused terms), acc += s_b * p. Used as the
 * 1e-5 cross-check of R1 and as the shape of the CPU baseline loop. */
void orc_q8_gemv_a11(const int8_t *W, const float *S, const float *x, float *y, int N, int K) {
  const int nb = K / ORC_QBLK;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < N; r++) {
    const int8_t *qr = W + (size_t)r * K;
    const float *sr = S + (size_t)r * nb;
    float acc = 0.0f;
    for (int b = 0; b < nb; b++) {
      float p = 0.0f;
      for (int j = 0; j < ORC_QBLK; j++) p += (float)qr[b * ORC_QBLK + j] * x[b * ORC_QBLK + j];
      acc += sr[b] * p;
    }
    y[r] = acc;
  }
}

/* R2, the reference's own GEMV numerics (q8_partial<bf16, FMA=1> and
 * k_combine_bf / k_combine_f, lfm3_nanode.cu:222-374, with the chunk rule of
 * pick(), 1750-1782): x is bf16 widened to fp32, weight scales are fp32.
 * Per chunk of KC = 2048 of K (K >= 2048 and K % 2048 == 0; otherwise all of
 * K): leaf L = 0..31 folds blocks b = L, L+32, ... of the chunk in ascending
 * order, each block's dot an fmaf chain over its 32 codes ascending from 0
 * (274-323), acc_L = fmaf(s_b, dot_b, acc_L) from 0; the chunk partial is the
 * shfl_down tree over the leaves, offsets 16, 8, 4, 2, 1 with
 * v_i = v_i + v_{i+o} (326); y = ((0 + p_0) + p_1) + ... over the chunks
 * ascending (338-345). The tiled prefill twin (q8_partial_TLb, 4051-4509, and
 * its transcription cpuchk_run, 4658-4684) runs only on single-chunk shapes
 * (pf_tilable, 4533-4542) and gives the same bits: its bit-reversed leaf
 * order with the binary counter is this tree. y[t][r] for T positions. */
static float q8r_row(const int8_t *w, const float *s, const float *x, int K) {
  const int KC = (K >= 2048 && K % 2048 == 0) ? 2048 : K;
  const int nbc = KC / ORC_QBLK;
  float y = 0.0f;
  for (int c = 0; c < K / KC; c++) {
    float leaf[32];
    for (int L = 0; L < 32; L++) {
      float acc = 0.0f;
      for (int b = L; b < nbc; b += 32) {
        const int k0 = c * KC + b * ORC_QBLK;
        float dot = 0.0f;
        for (int j = 0; j < ORC_QBLK; j++) dot = fmaf((float)w[k0 + j], x[k0 + j], dot);
        acc = fmaf(s[c * nbc + b], dot, acc);
      }
      leaf[L] = acc;
    }
    for (int o = 16; o > 0; o >>= 1)
      for (int i = 0; i < o; i++) leaf[i] = leaf[i] + leaf[i + o];
    y = y + leaf[0];
  }
  return y;
}

void orc_q8r_gemm(const int8_t *W, const float *S, const uint16_t *x, float *y, int N, int K, int T) {
  const int nb = K / ORC_QBLK;
  float *xf = (float *)malloc(sizeof(float) * (size_t)K * T);
  for (size_t i = 0; i < (size_t)K * T; i++) xf[i] = orc_bf2f(x[i]);
#pragma omp parallel for schedule(dynamic, 16)
  for (int r = 0; r < N; r++)
    for (int t = 0; t < T; t++)
      y[(size_t)t * N + r] = q8r_row(W + (size_t)r * K, S + (size_t)r * nb, xf + (size_t)t * K, K);
  free(xf);
}

/* Q4 / Q5 low-bit GEMV, the reference's order (k_qlow + k_qlow_combine,
 * lfm3_qlow.cuh:39-113, with qlow_gemv's K split, lfm3_nanode.cu:1894-1915).
 * Per 32-group along K: w = d*q + mn, q in [0, 2^B), stored d' = 128*d and
 * mn (fp16). x is bf16 widened to fp32. K is cut into KS slices of whole
 * groups, KS = 4 for K >= 4096 else 2; per slice from 0, groups ascending:
 *   sg  = the group's 32 x summed in order from 0 (k_qlow's sx, 68-73);
 *   a_b = fmaf chain from 0 over k = b, b+4, ..., b+28 of (1 + q_k/128)*x_k,
 *         b = 0..3 (qlow_group: the code read as the float 1 + q/128, 22-37);
 *   acc = (a0 + a1) + (a2 + a3);
 *   y_s = fmaf(d', acc - sg, fmaf(mn, sg, y_s))                   (99-101);
 * then y = ((0 + y_0) + y_1) + ... over the slices (107-112). Codes Q
 * [N][K], one value per byte (row-major, unpacked); S [N][K/32][2] fp16 bits
 * (d', mn). y fp32; the reference stores bf16(y). */
void orc_qlow_gemv(const uint8_t *Q, const uint16_t *S, const uint16_t *x, float *y, int N, int K) {
  const int G = K / ORC_QBLK, KS = K >= 4096 ? 4 : 2, GL = G / KS;
  float *xf = (float *)malloc(sizeof(float) * (size_t)K);
  float *sx = (float *)malloc(sizeof(float) * (size_t)G);
  for (int i = 0; i < K; i++) xf[i] = orc_bf2f(x[i]);
  for (int g = 0; g < G; g++) {
    float t = 0.0f;
    for (int k = 0; k < ORC_QBLK; k++) t += xf[g * ORC_QBLK + k];
    sx[g] = t;
  }
#pragma omp parallel for schedule(static)
  for (int r = 0; r < N; r++) {
    const uint8_t *qr = Q + (size_t)r * K;
    float yt = 0.0f;
    for (int sl = 0; sl < KS; sl++) {
      float ys = 0.0f;
      for (int g = sl * GL; g < (sl + 1) * GL; g++) {
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int k = 0; k < ORC_QBLK; k++)
          a[k & 3] = fmaf(1.0f + (float)qr[g * ORC_QBLK + k] / 128.0f, xf[g * ORC_QBLK + k], a[k & 3]);
        const float acc = (a[0] + a[1]) + (a[2] + a[3]);
        const float dp = orc_h2f(S[((size_t)r * G + g) * 2]), mn = orc_h2f(S[((size_t)r * G + g) * 2 + 1]);
        ys = fmaf(dp, acc - sx[g], fmaf(mn, sx[g], ys));
      }
      yt = yt + ys;
    }
    y[r] = yt;
  }
  free(xf);
  free(sx);
}

/* The bf16-table LM head (k_gemv_bf16, lfm3_nanode.cu:3504-3534, as
 * lm_head_bf16 launches it, 3536-3573): W bf16 [N][K], x bf16 [K] widened to
 * fp32. Per row, leaf L = 0..31 sums k = L, L+32, L+64, ... ascending from 0,
 * each product rounded before its add (__fmul_rn, __fadd_rn); the 32 leaves
 * then combine as the shfl_down tree 16, 8, 4, 2, 1 (leaf i += leaf i+o for
 * i < o). y fp32. */
void orc_bf16_gemv(const uint16_t *W, const uint16_t *x, float *y, int N, int K) {
  float *xf = (float *)malloc(sizeof(float) * (size_t)K);
  for (int i = 0; i < K; i++) xf[i] = orc_bf2f(x[i]);
#pragma omp parallel for schedule(static)
  for (int r = 0; r < N; r++) {
    const uint16_t *wr = W + (size_t)r * K;
    float leaf[32];
    for (int L = 0; L < 32; L++) {
      float s = 0.0f;
      for (int k = L; k < K; k += 32) {
        const float p = orc_bf2f(wr[k]) * xf[k];
        s = s + p;
      }
      leaf[L] = s;
    }
    for (int o = 16; o > 0; o >>= 1)
      for (int i = 0; i < o; i++) leaf[i] = leaf[i] + leaf[i + o];
    y[r] = leaf[0];
  }
  free(xf);
}

/* Exact value of the quantized product, sum_b (S_b*dx_b as real) * isum_b, in
 * double (every term is exact in double: S_b and dx_b have 11 and 24 bit
 * mantissas, isum_b < 2^20; the sum rounds at most nb times at 2^-53). */
void orc_q8_gemv_exact(const int8_t *W, const uint16_t *S, const int8_t *qx, const float *dx,
                       double *y, int N, int K) {
  const int nb = K / ORC_QBLK;
  for (int r = 0; r < N; r++) {
    double acc = 0.0;
    for (int b = 0; b < nb; b++) {
      const int32_t is = blk_dot(W + (size_t)r * K + (size_t)b * ORC_QBLK, qx + (size_t)b * ORC_QBLK);
      acc += (double)orc_h2f(S[(size_t)r * nb + b]) * (double)dx[b] * (double)is;
    }
    y[r] = acc;
  }
}

/* PQ2_0 x Q8_K ternary GEMV (pq2_host.c:82-104 pq2_gemv_cpu): codes u8
 * [N][K/4] (weight i of a byte = bits 2i..2i+1, value = code-1), fp16 scale
 * per 128-group, activations Q8_K (292 B per 256; group g uses block g>>1,
 * half g&1). Per row, groups ascending:
 *   isum = sum (code-1)*qs  (int32),  acc = fl(acc + fl(fl(ws*db) * (float)isum))
 * Pinned by: bit-exact against the reference's own pq2_gemv_cpu built into
 * oracle/_ref from pq2_host.c. */
void orc_tq2_gemv(const uint8_t *codes, const uint16_t *S, const uint8_t *xq, float *y,
                  int N, int K) {
  const int ng = K / ORC_TQ_GROUP;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < N; r++) {
    const uint8_t *cd = codes + (size_t)r * (K / 4);
    float acc = 0.0f;
    for (int g = 0; g < ng; g++) {
      const uint8_t *qb = xq + (size_t)(g >> 1) * ORC_Q8K_BYTES;
      float db;
      memcpy(&db, qb, 4);
      const int8_t *qs = (const int8_t *)(qb + 4 + (g & 1) * 128);
      const float ws = orc_h2f(S[(size_t)r * ng + g]);
      const uint8_t *c = cd + (size_t)g * 32;
      int32_t isum = 0;
      for (int i = 0; i < 128; i++) isum += (((c[i >> 2] >> ((i & 3) * 2)) & 3) - 1) * (int32_t)qs[i];
      const float t = ws * db;
      const float u = t * (float)isum;
      acc = acc + u;
    }
    y[r] = acc;
  }
}

/* ============================================================ layer primitives */

/* Pairwise (balanced binary) sum in natural order: n == 1 -> v[0], else
 * fl(pw(first floor(n/2)) + pw(rest)). For n a power of two this is exactly
 * the xor-butterfly across lanes the attention kernels use for a split's
 * softmax denominator. */
float orc_pairwise(const float *v, int n) {
  if (n == 1) return v[0];
  const int h = n / 2;
  return orc_pairwise(v, h) + orc_pairwise(v + h, n - h);
}

/* The shfl_down tree of a 32-thread warp (lfm3_nanode.cu:398, 470): at
 * offset o = 16, 8, 4, 2, 1 thread l < o adds thread l + o's value; thread 0
 * ends with the warp's sum. */
static float orc_warp_tree(float *s) {
  for (int o = 16; o > 0; o >>= 1)
    for (int l = 0; l < o; l++) s[l] = s[l] + s[l + o];
  return s[0];
}

/* The sum of squares of rmsnorm_body (lfm3_nanode.cu:383-440): thread l of
 * warp w holds elements 256w + 8l .. 256w + 8l + 7 and sums their squares
 * pairwise, the warp's 32 sums go through the shfl_down tree, and the n/256
 * warp partials add in order from warp 0. n a multiple of 256 (the reference
 * runs n = 2048: 256 threads, 8 warps). */
float orc_rms_sumsq(const uint16_t *x, int n) {
  float tot = 0.0f;
  for (int w = 0; w < n / 256; w++) {
    float s[32];
    for (int l = 0; l < 32; l++) {
      float q[8];
      for (int j = 0; j < 8; j++) {
        const float v = orc_bf2f(x[256 * w + 8 * l + j]);
        q[j] = v * v;
      }
      s[l] = ((q[0] + q[1]) + (q[2] + q[3])) + ((q[4] + q[5]) + (q[6] + q[7]));
    }
    const float p = orc_warp_tree(s);
    tot = w == 0 ? p : tot + p;
  }
  return tot;
}

/* RMSNorm, bf16 in/out, fp32 weight (lfm3_nanode.cu:383-440 rmsnorm_body):
 *   ss = orc_rms_sumsq(x), v = fl(fl(ss * fl(1/n)) + eps), rs = fl(1 / fl(sqrt(v)))
 *   y_i = bf16(fl(w_i * bf16(fl(x_i * rs))))   -- round BEFORE the weight
 * The reference takes rs = rsqrtf(v) on the device (an approximation CUDA
 * does not specify bit for bit) and 1/sqrtf on the CPU (lfm3_elem_test.c:45);
 * both sides here use the correctly rounded 1/sqrtf. n a multiple of 256. */
void orc_rmsnorm(const uint16_t *x, const float *w, uint16_t *y, int n, float eps) {
  const float ss = orc_rms_sumsq(x, n);
  const float rs = 1.0f / sqrtf(ss * (1.0f / (float)n) + eps);
  for (int i = 0; i < n; i++) {
    const float rounded = orc_bf2f(orc_f2bf(orc_bf2f(x[i]) * rs));
    y[i] = orc_f2bf(w[i] * rounded);
  }
}

/* The sum of squares of k_headnorm (lfm3_nanode.cu:460-479) over one head:
 * 32 threads of e = hd/32 consecutive elements (4 at hd = 128, the
 * reference's; 2 at hd = 64, which it does not run), their squares summed
 * pairwise (the reference's trailing + 0 leaves a sum of squares unchanged),
 * then the shfl_down tree. */
float orc_head_sumsq(const uint16_t *x, int hd) {
  const int e = hd / 32;
  float s[32];
  for (int l = 0; l < 32; l++) {
    float q[4];
    for (int j = 0; j < e; j++) {
      const float v = orc_bf2f(x[e * l + j]);
      q[j] = v * v;
    }
    s[l] = e == 4 ? (q[0] + q[1]) + (q[2] + q[3]) : q[0] + q[1];
  }
  return orc_warp_tree(s);
}

/* Per-head RMSNorm over head_dim, in place (k_headnorm): orc_head_sumsq, then
 * the rounding steps of orc_rmsnorm with n = hd. */
void orc_headnorm(uint16_t *x, const float *w, int nheads, int hd, float eps) {
  for (int h = 0; h < nheads; h++) {
    uint16_t *xr = x + (size_t)h * hd;
    const float rs = 1.0f / sqrtf(orc_head_sumsq(xr, hd) * (1.0f / (float)hd) + eps);
    for (int i = 0; i < hd; i++) xr[i] = orc_f2bf(w[i] * orc_bf2f(orc_f2bf(orc_bf2f(xr[i]) * rs)));
  }
}

/* RoPE inverse frequencies as the reference's host builds them
 * (lfm3_nanode.cu:3719-3723 build_invf, dim = head_dim): in float,
 * invf_i = 1.0f / powf(theta, (float)(2i) / (float)hd) for i < rot/2, and 0
 * past them (the zero tail). */
void orc_rope_invf(float *invf, int hd, int rot, float theta) {
  for (int i = 0; i < hd / 2; i++)
    invf[i] = i < rot / 2 ? 1.0f / powf(theta, (float)(2 * i) / (float)hd) : 0.0f;
}

/* RoPE table [pos][rot/2][cos, sin]: the angle is the fp32 product
 * fl((float)pos * invf_i) (k_rope, lfm3_nanode.cu:483-498), and cos/sin of
 * that float angle are evaluated in double and rounded once to float (the
 * reference evaluates cosf/sinf on the device and notes it could not match
 * torch's cos/sin there, lfm3_nanode.cu:43-44; a table read on both sides
 * fixes one value). */
void orc_rope_table(float *cs, int maxpos, int hd, int rot, float theta) {
  const int half = rot / 2;
  float invf[512];
  orc_rope_invf(invf, hd, rot, theta);
  for (int p = 0; p < maxpos; p++)
    for (int i = 0; i < half; i++) {
      const float ang = (float)p * invf[i];
      cs[((size_t)p * half + i) * 2 + 0] = (float)cos((double)ang);
      cs[((size_t)p * half + i) * 2 + 1] = (float)sin((double)ang);
    }
}

/* Zero-tail partial rotation (lfm3_nanode.cu:483-498): pairs (i, i + hd/2) for
 * i < rot/2, lo' = bf16(fl(lo*c) - fl(hi*s)), hi' = bf16(fl(hi*c) + fl(lo*s)). */
void orc_rope(uint16_t *x, const float *cs, int pos, int nheads, int hd, int rot) {
  const int half = rot / 2;
  for (int h = 0; h < nheads; h++) {
    uint16_t *xr = x + (size_t)h * hd;
    for (int i = 0; i < half; i++) {
      const float c = cs[((size_t)pos * half + i) * 2], s = cs[((size_t)pos * half + i) * 2 + 1];
      const float lo = orc_bf2f(xr[i]), hi = orc_bf2f(xr[i + hd / 2]);
      xr[i] = orc_f2bf(lo * c - hi * s);
      xr[i + hd / 2] = orc_f2bf(hi * c + lo * s);
    }
  }
}

/* Split-K flash-decode over an fp16 KV cache [npos][nkv][hd] (the fp16-KV
 * online-softmax precedent is pq1_host.c:385-430 pq1_fa16_head; the GQA head
 * map h -> h / (nh/nkv) is lfm3_nanode.cu:520). Order, per q head:
 *   dot_p = fmaf chain over d ascending of bf16(q_d) * f16(k_pd), from 0
 *   s_p   = fl(dot_p * scale)
 *   split j = positions [64j, min(64j+64, npos)):
 *     m_j = max s_p;  e_p = expf(fl(s_p - m_j))
 *     l_j = pairwise sum over the 64 slots (e_p, zero past npos)
 *     o_jd = fmaf chain over p ascending of e_p * f16(v_pd), from 0
 *   M = max m_j; for j ascending: w = expf(fl(m_j - M)),
 *     L = fmaf(l_j, w, L), O_d = fmaf(o_jd, w, O_d)   (from 0)
 *   out_d = bf16(fl(O_d / L))
 * win > 0 (sliding-window layers): only keys [lo, npos) take part, see below.
 * Pinned by: a double-precision two-pass softmax (orc_attn_twopass) over the
 * same keys within bf16 rounding, npos = 1 (out = v_0 exactly up to bf16) and
 * win = 1 (out = v_{npos-1}). */
void orc_attn(const uint16_t *q, const uint16_t *Kc, const uint16_t *Vc, uint16_t *out,
              int npos, int nh, int nkv, int hd, float scale, int win) {
  const int grp = nh / nkv;
  /* sliding window: the query at position npos-1 sees keys [lo, npos), with
   * the reference's lo = (win > 0 && npos > win) ? npos - win : 0
   * (k_attn_head, lfm3_nanode.cu:515). The splits stay the 64-aligned blocks
   * of absolute positions; slots outside [lo, npos) hold nothing (e = 0, not
   * in the max, skipped in the value chain), and splits with no visible
   * position are left out of the merge. */
  const int lo = (win > 0 && npos > win) ? npos - win : 0;
  const int j0 = lo / ORC_ATT_SPLIT;
  const int nsplit = (npos + ORC_ATT_SPLIT - 1) / ORC_ATT_SPLIT;
  float *m = (float *)malloc(sizeof(float) * (size_t)nsplit);
  float *l = (float *)malloc(sizeof(float) * (size_t)nsplit);
  float *o = (float *)malloc(sizeof(float) * (size_t)nsplit * hd);
  float e[ORC_ATT_SPLIT], sc[ORC_ATT_SPLIT];
  for (int h = 0; h < nh; h++) {
    const int g = h / grp;
    const uint16_t *qh = q + (size_t)h * hd;
    for (int j = j0; j < nsplit; j++) {
      const int p0 = j * ORC_ATT_SPLIT;
      const int pn = npos - p0 < ORC_ATT_SPLIT ? npos - p0 : ORC_ATT_SPLIT;
      const int i0 = lo > p0 ? lo - p0 : 0;   /* first visible slot */
      float mj = -INFINITY;
      for (int i = i0; i < pn; i++) {
        const uint16_t *kr = Kc + ((size_t)(p0 + i) * nkv + g) * hd;
        float dot = 0.0f;
        for (int d = 0; d < hd; d++) dot = fmaf(orc_bf2f(qh[d]), orc_h2f(kr[d]), dot);
        sc[i] = dot * scale;
        if (sc[i] > mj) mj = sc[i];
      }
      for (int i = 0; i < ORC_ATT_SPLIT; i++) e[i] = i >= i0 && i < pn ? orc_expf(sc[i] - mj) : 0.0f;
      m[j] = mj;
      l[j] = orc_pairwise(e, ORC_ATT_SPLIT);
      for (int d = 0; d < hd; d++) {
        float acc = 0.0f;
        for (int i = i0; i < pn; i++)
          acc = fmaf(e[i], orc_h2f(Vc[((size_t)(p0 + i) * nkv + g) * hd + d]), acc);
        o[(size_t)j * hd + d] = acc;
      }
    }
    float M = -INFINITY;
    for (int j = j0; j < nsplit; j++) if (m[j] > M) M = m[j];
    float L = 0.0f;
    float O[1024];
    for (int d = 0; d < hd; d++) O[d] = 0.0f;
    for (int j = j0; j < nsplit; j++) {
      const float w = orc_expf(m[j] - M);
      L = fmaf(l[j], w, L);
      for (int d = 0; d < hd; d++) O[d] = fmaf(o[(size_t)j * hd + d], w, O[d]);
    }
    for (int d = 0; d < hd; d++) out[(size_t)h * hd + d] = orc_f2bf(O[d] / L);
  }
  free(m); free(l); free(o);
}

/* Attention in k_attn_head's order (lfm3_nanode.cu:503-602) over a bf16 cache
 * [npos][nkv][hd], for the query at position npos - 1 (keys lo .. npos - 1, lo
 * from win as in orc_attn). Per q head, the reference's 256 threads being 8
 * warps of 32 lanes:
 *  - key i's score: lane l's chain over dims e*l .. e*l + e - 1 (e = hd/32),
 *    s = fl(s + fl(q_d * k_d)) from 0; the shfl_down tree over the 32 lanes;
 *    fl(s * scale);
 *  - m = the largest of -1e30 and the scores;
 *  - e_i = orc_expf(s_i - m) (CUDA's expf in the reference); thread t sums
 *    e_i over i = t, t + 256, ... in order, each warp's 32 sums go through the
 *    shfl_down tree, the 8 warp sums through the tree of offsets 4, 2, 1;
 *    inv = fl(1 / sum);
 *  - per dim d, segment g of 8 sums fl(fl(e_i * inv) * v_id) over i = g,
 *    g + 8, ... in order from 0, and out_d = bf16 of the segments added
 *    pairwise, ((g0 + g1) + (g2 + g3)) + ((g4 + g5) + (g6 + g7)).
 * i counts from lo. */
void orc_attn_ref(const uint16_t *q, const uint16_t *Kc, const uint16_t *Vc, uint16_t *out,
                  int npos, int nh, int nkv, int hd, float scale, int win) {
  const int grp = nh / nkv, e = hd / 32;
  const int lo = (win > 0 && npos > win) ? npos - win : 0, np = npos - lo;
  float *sl = (float *)malloc(sizeof(float) * (size_t)np);
  for (int h = 0; h < nh; h++) {
    const int g = h / grp;
    const uint16_t *qh = q + (size_t)h * hd;
    for (int i = 0; i < np; i++) {
      const uint16_t *kr = Kc + ((size_t)(lo + i) * nkv + g) * hd;
      float s[32];
      for (int l = 0; l < 32; l++) {
        float a = 0.0f;
        for (int j = 0; j < e; j++) a = a + orc_bf2f(qh[e * l + j]) * orc_bf2f(kr[e * l + j]);
        s[l] = a;
      }
      sl[i] = orc_warp_tree(s) * scale;
    }
    float m = -1e30f;
    for (int i = 0; i < np; i++) m = fmaxf(m, sl[i]);
    for (int i = 0; i < np; i++) sl[i] = orc_expf(sl[i] - m);
    float th[256], ws[8];
    for (int t = 0; t < 256; t++) {
      th[t] = 0.0f;
      for (int i = t; i < np; i += 256) th[t] = th[t] + sl[i];
    }
    for (int w = 0; w < 8; w++) ws[w] = orc_warp_tree(th + 32 * w);
    const float inv = 1.0f / (((ws[0] + ws[4]) + (ws[2] + ws[6])) + ((ws[1] + ws[5]) + (ws[3] + ws[7])));
    for (int d = 0; d < hd; d++) {
      float sg[8];
      for (int k = 0; k < 8; k++) {
        float acc = 0.0f;
        for (int i = k; i < np; i += 8) acc = acc + (sl[i] * inv) * orc_bf2f(Vc[((size_t)(lo + i) * nkv + g) * hd + d]);
        sg[k] = acc;
      }
      out[(size_t)h * hd + d] = orc_f2bf(((sg[0] + sg[1]) + (sg[2] + sg[3])) + ((sg[4] + sg[5]) + (sg[6] + sg[7])));
    }
  }
  free(sl);
}

/* Two-pass softmax attention in double (the structure of k_attn_head,
 * lfm3_nanode.cu:503-602, without its rounding steps): the referee for
 * orc_attn. out is fp32 [nh][hd]. */
void orc_attn_twopass(const uint16_t *q, const uint16_t *Kc, const uint16_t *Vc, float *out,
                      int npos, int nh, int nkv, int hd, float scale, int win) {
  const int grp = nh / nkv;
  const int lo = (win > 0 && npos > win) ? npos - win : 0;
  double *s = (double *)malloc(sizeof(double) * (size_t)npos);
  for (int h = 0; h < nh; h++) {
    const int g = h / grp;
    double mx = -INFINITY;
    for (int p = lo; p < npos; p++) {
      double dot = 0.0;
      for (int d = 0; d < hd; d++)
        dot += (double)orc_bf2f(q[(size_t)h * hd + d]) * (double)orc_h2f(Kc[((size_t)p * nkv + g) * hd + d]);
      s[p] = dot * (double)scale;
      if (s[p] > mx) mx = s[p];
    }
    double sum = 0.0;
    for (int p = lo; p < npos; p++) { s[p] = exp(s[p] - mx); sum += s[p]; }
    for (int d = 0; d < hd; d++) {
      double acc = 0.0;
      for (int p = lo; p < npos; p++) acc += s[p] * (double)orc_h2f(Vc[((size_t)p * nkv + g) * hd + d]);
      out[(size_t)h * hd + d] = (float)(acc / sum);
    }
  }
  free(s);
}

/* Gated short conv, one position (lfm3_nanode.cu:892-911 k_shift_in + k_conv7,
 * and the layer_body sequence 3790-3817): bcx = in_proj output [B | C | x],
 * ring [ntaps][H] bf16 with the newest slot last.
 *   bx = bf16(fl(B*x)); ring shifts down, slot ntaps-1 = bx
 *   acc = 0; acc = fl(acc + fl(tap_k * ring_k)) for k ascending; cy = bf16(acc)
 *   out = bf16(fl(C * cy))
 * Pinned by: ntaps-step impulse responses (a unit bx appears scaled by tap_k
 * k steps later) and the CPU conv reference order (lfm3_conv_test.c:30-39). */
void orc_conv_step(uint16_t *ring, const float *taps, const uint16_t *bcx, uint16_t *out,
                   int H, int ntaps) {
  for (int i = 0; i < H; i++) {
    const uint16_t bx = orc_f2bf(orc_bf2f(bcx[i]) * orc_bf2f(bcx[2 * H + i]));
    for (int k = 0; k < ntaps - 1; k++) ring[(size_t)k * H + i] = ring[(size_t)(k + 1) * H + i];
    ring[(size_t)(ntaps - 1) * H + i] = bx;
    float acc = 0.0f;
    for (int k = 0; k < ntaps; k++) acc = acc + taps[(size_t)i * ntaps + k] * orc_bf2f(ring[(size_t)k * H + i]);
    const uint16_t cy = orc_f2bf(acc);
    out[i] = orc_f2bf(orc_bf2f(bcx[H + i]) * orc_bf2f(cy));
  }
}

/* Elementwise ops, one bf16 rounding each (lfm3_nanode.cu:811-888). */
void orc_add(const uint16_t *a, const uint16_t *b, uint16_t *y, int n) {
  for (int i = 0; i < n; i++) y[i] = orc_f2bf(orc_bf2f(a[i]) + orc_bf2f(b[i]));
}
void orc_mul(const uint16_t *a, const uint16_t *b, uint16_t *y, int n) {
  for (int i = 0; i < n; i++) y[i] = orc_f2bf(orc_bf2f(a[i]) * orc_bf2f(b[i]));
}
/* silu(a)*b: sg = fl(1 / fl(1 + expf(-a))), y = bf16(fl(fl(a*sg) * b)) (821-829). */
void orc_silu_mul(const uint16_t *a, const uint16_t *b, uint16_t *y, int n) {
  for (int i = 0; i < n; i++) {
    const float av = orc_bf2f(a[i]);
    const float sg = 1.0f / (1.0f + orc_expf(-av));
    y[i] = orc_f2bf((av * sg) * orc_bf2f(b[i]));
  }
}
/* attn[h][:] *= sigmoid(g_h), s = fl(1 / fl(1 + expf(-g))) (852-859). */
void orc_sigmoid_gate(const uint16_t *g, uint16_t *attn, int nh, int hd) {
  for (int h = 0; h < nh; h++) {
    const float s = 1.0f / (1.0f + orc_expf(-orc_bf2f(g[h])));
    for (int d = 0; d < hd; d++)
      attn[(size_t)h * hd + d] = orc_f2bf(orc_bf2f(attn[(size_t)h * hd + d]) * s);
  }
}

/* Greedy argmax as k_argmax (lfm3_nanode.cu:942-964) picks it: thread t of
 * 256 scans i = t, t + 256, ... keeping the first value strictly above its
 * best (from -1e30, index -1); the 32 lanes of each warp then fold with the
 * shfl_down tree, lane l < o taking lane l + o's pair only when its value is
 * strictly larger, and the 8 warp pairs fold the same way. -1 when no value
 * exceeds -1e30. */
int orc_argmax(const float *v, int n) {
  float bv[256];
  int bi[256];
  for (int t = 0; t < 256; t++) {
    bv[t] = -1e30f;
    bi[t] = -1;
    for (int i = t; i < n; i += 256)
      if (v[i] > bv[t]) { bv[t] = v[i]; bi[t] = i; }
  }
  float wv[8];
  int wi[8];
  for (int w = 0; w < 8; w++) {
    float *sv = bv + 32 * w;
    int *si = bi + 32 * w;
    for (int o = 16; o > 0; o >>= 1)
      for (int l = 0; l < o; l++)
        if (sv[l + o] > sv[l]) { sv[l] = sv[l + o]; si[l] = si[l + o]; }
    wv[w] = sv[0];
    wi[w] = si[0];
  }
  for (int o = 4; o > 0; o >>= 1)
    for (int l = 0; l < o; l++)
      if (wv[l + o] > wv[l]) { wv[l] = wv[l + o]; wi[l] = wi[l + o]; }
  return wi[0];
}

/* Embedding row from the tied Q8 table: bf16(fl(code * scale)) (lfm3_nanode.cu:
 * 138-142 k_dequant_row). */
void orc_embed_row(const int8_t *W, const uint16_t *S, int tok, int K, uint16_t *out) {
  const int8_t *c = W + (size_t)tok * K;
  const uint16_t *s = S + (size_t)tok * (K / ORC_QBLK);
  for (int i = 0; i < K; i++) out[i] = orc_f2bf((float)c[i] * orc_h2f(s[i / ORC_QBLK]));
}
