/* oracle.h -- CPU restatement of the PULSAR-ASM LFM3/Bonsai hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the test reference for the HIP path:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * it. The product library never links, calls or falls back to it.
 *
 * Every function names the reference file:line whose behaviour it restates
 * (paths relative to the PULSAR-ASM tree). Where the build defines its own
 * order (the Q8_0 x Q8_0 "R1" order, split-K flash-decode, the pairwise
 * norm tree) the definition is written out in the comment and is the
 * contract the GPU kernels implement bit for bit.
 *
 * Pinning (what checks each function independently of its own formula) is
 * listed per function under "pinned by"; the tests in tests/test_oracle_*.py
 * carry those checks out.
 *
 * Build: -O3 -ffp-contract=off -fopenmp (see oracle/build.py). With
 * -ffp-contract=off every fused multiply-add below is an explicit fmaf().
 */
#ifndef PULSAR_ORACLE_H
#define PULSAR_ORACLE_H
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORC_QBLK 32          /* Q8_0 block (lfm3_nanode.cu:74 Q8_BLK)        */
#define ORC_CHUNK 8          /* R1 chunk, in blocks (256 K-elements)         */
#define ORC_ATT_SPLIT 64     /* flash-decode split, in positions             */
#define ORC_TQ_GROUP 128     /* PQ2_0 group (pq2_wrap.h:9-12)                */
#define ORC_Q8K_BLK 256      /* Q8_K block (fwd8.c:72)                       */
#define ORC_Q8K_BYTES 292    /* 4 B d + 256 qs + 16 x int16 bsums            */

/* ---------------------------------------------------------------- scalars */
float    orc_bf2f(uint16_t b);        /* lfm3_nanode.cu:115                   */
uint16_t orc_f2bf(float f);           /* lfm3_nanode.cu:116-121 (RNE, nan/inf passthrough) */
float    orc_h2f(uint16_t h);         /* pq2_host.c:9-20 pq2_h2f              */
uint16_t orc_f2h(float f);            /* IEEE binary16 RNE (overflow -> inf)  */
float    orc_expf(float x);           /* Cody-Waite + Taylor, see oracle.c    */

/* ------------------------------------------------------------- generator */
uint64_t orc_sm64_at(uint64_t seed, uint64_t n);     /* splitmix64 output n   */
void orc_gen_codes(uint64_t seed, int8_t *out, size_t n);          /* [-127,127] */
void orc_gen_normal(uint64_t seed, float *out, size_t n);          /* N(0,1)     */
void orc_gen_scales(uint64_t seed, uint16_t *out, size_t n, float mult); /* f16(|z|*mult) */
void orc_gen_affine(uint64_t seed, float *out, size_t n, float a, float b); /* a + b*z */
void orc_gen_ternary(uint64_t seed, uint8_t *out, size_t nbytes);  /* codes {0,1,2} */
void orc_gen_tokens(uint64_t seed, int32_t *out, int n, int vocab);

/* ------------------------------------------------------------ quantizers */
void orc_q8_quant(const float *x, int K, int8_t *qx, float *dx);
void orc_q8_quant_bf16(const uint16_t *x, int K, int8_t *qx, float *dx);
void orc_q8k_quant(const float *x, int K, uint8_t *out);            /* fwd8.c:72-137 */

/* ------------------------------------------------------------ GEMV / GEMM */
void orc_q8_gemv(const int8_t *W, const uint16_t *S, const int8_t *qx, const float *dx,
                 float *y, int N, int K);
void orc_q8_gemm(const int8_t *W, const uint16_t *S, const int8_t *qx, const float *dx,
                 float *y, int N, int K, int T);
void orc_q8_gemv_a11(const int8_t *W, const float *S, const float *x, float *y, int N, int K);
/* R2: the reference's own GEMV order (bf16 x, fp32 scales, 32-leaf tree); y [T][N] */
void orc_q8r_gemm(const int8_t *W, const float *S, const uint16_t *x, float *y, int N, int K, int T);
/* Q4/Q5 low-bit GEMV in the reference's order; Q [N][K] one code per byte, S [N][K/32][2] fp16 (d', mn) */
void orc_qlow_gemv(const uint8_t *Q, const uint16_t *S, const uint16_t *x, float *y, int N, int K);
void orc_bf16_gemv(const uint16_t *W, const uint16_t *x, float *y, int N, int K);
void orc_q8_gemv_exact(const int8_t *W, const uint16_t *S, const int8_t *qx, const float *dx,
                       double *y, int N, int K);
void orc_tq2_gemv(const uint8_t *codes, const uint16_t *S, const uint8_t *xq, float *y,
                  int N, int K);

/* ------------------------------------------------------ layer primitives */
float orc_pairwise(const float *v, int n);
float orc_rms_sumsq(const uint16_t *x, int n);
float orc_head_sumsq(const uint16_t *x, int hd);
void orc_rmsnorm(const uint16_t *x, const float *w, uint16_t *y, int n, float eps);
void orc_headnorm(uint16_t *x, const float *w, int nheads, int hd, float eps);
int orc_max_threads(void);
void orc_rope_invf(float *invf, int hd, int rot, float theta);
void orc_rope_table(float *cs, int maxpos, int hd, int rot, float theta);
void orc_rope(uint16_t *x, const float *cs, int pos, int nheads, int hd, int rot);
void orc_attn(const uint16_t *q, const uint16_t *Kc, const uint16_t *Vc, uint16_t *out,
              int npos, int nh, int nkv, int hd, float scale, int win);
void orc_attn_ref(const uint16_t *q, const uint16_t *Kc, const uint16_t *Vc, uint16_t *out,
                  int npos, int nh, int nkv, int hd, float scale, int win);
void orc_attn_twopass(const uint16_t *q, const uint16_t *Kc, const uint16_t *Vc, float *out,
                      int npos, int nh, int nkv, int hd, float scale, int win);
void orc_conv_step(uint16_t *ring, const float *taps, const uint16_t *bcx, uint16_t *out,
                   int H, int ntaps);
void orc_add(const uint16_t *a, const uint16_t *b, uint16_t *y, int n);
void orc_mul(const uint16_t *a, const uint16_t *b, uint16_t *y, int n);
void orc_silu_mul(const uint16_t *a, const uint16_t *b, uint16_t *y, int n);
void orc_sigmoid_gate(const uint16_t *g, uint16_t *attn, int nh, int hd);
int  orc_argmax(const float *v, int n);
void orc_embed_row(const int8_t *W, const uint16_t *S, int tok, int K, uint16_t *out);

/* ------------------------------------------------------------- backbone */
typedef struct orc_cfg {
  int hidden, ffn, vocab, nlayers;
  int nh, nkv, hd, rot;      /* rot = rotated dims (partial factor * hd)     */
  int ntaps;                 /* short-conv kernel size                        */
  int ctx;                   /* KV capacity                                   */
  float eps, theta;
  uint64_t seed;
  uint32_t attn_mask;        /* bit L set -> layer L is attention, else conv  */
  int numerics;              /* 0: Q8_0 x Q8_0 (R1); 1: the reference's GEMV
                                order (R2: bf16 x, fp32 scales)               */
  uint32_t slide_mask;       /* bit L set -> layer L is sliding-window attention */
  int slide_win;             /* keys a sliding layer sees (the last slide_win)  */
  int slide_rot;             /* rotated dims of a sliding layer                */
  float slide_theta;         /* RoPE base of a sliding layer                   */
  int emb_bf16;              /* 1: the tied table is bf16 (the exporter's --emb-bf16):
                                embedding rows copied, LM head orc_bf16_gemv   */
  int lowbit;                /* 0, 4 or 5: the bits of the low-bit tensors      */
  uint32_t lowbit_mask;      /* bit L set -> layer L's linears are low-bit (all
                                but the attention gate_proj); needs numerics 1 */
} orc_cfg;

typedef struct orc_model orc_model;
orc_model *orc_model_create(const orc_cfg *cfg);
void orc_model_free(orc_model *m);
void orc_model_reset(orc_model *m);
/* Feed n tokens starting at the model's current position; returns the
 * greedy id after the last one (the argmax of its logits). logits may be
 * NULL or receive the vocab logits of the last position. */
int orc_model_feed(orc_model *m, const int32_t *tok, int n, float *logits);
/* prompt -> greedy ids of n_steps decode steps (the first id comes from the
 * prompt's last position). */
void orc_model_greedy(orc_model *m, const int32_t *prompt, int n_prompt, int n_steps,
                      int32_t *ids);
/* Tensor access for tests (row-major codes [N][K], fp16 scales [N][K/32]). */
int orc_model_tensor(orc_model *m, int layer, int slot, const void **p0, const void **p1,
                     int *N, int *K);
int orc_model_debug_hidden(orc_model *m, uint16_t *out);   /* residual of last position */
/* The source tensors of a slot (0 mixer in, 1 mixer out, 2 gate/up, 3 down) as
 * the .lfm3q8 file lists them: up to 4 (row offset, rows, bits: 8 = Q8, 4 / 5 =
 * low-bit). Returns their count, or -1. */
int orc_model_parts(orc_model *m, int layer, int slot, int *r0, int *n, int *bits);
/* A slot's low-bit codes (uint8 [N][K], one per byte) and scales ([N][K/32][2]
 * fp16: d' = 128 d, mn), for every row (the low-bit parts' rows are the ones
 * used); -1 if the slot has no low-bit part. */
int orc_model_lowbit(orc_model *m, int layer, int slot, const uint8_t **q, const uint16_t **s, int *N, int *K);

#ifdef __cplusplus
}
#endif
#endif
