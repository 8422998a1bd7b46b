/* oracle_model.c -- CPU restatement of the LFM3-style backbone (test infrastructure).
 *
 * The layer sequence restates layer_body (lfm3_nanode.cu:3739-3856) with the
 * hot-path numerics of oracle.c: Q8_0 x Q8_0 GEMVs (activations quantized per
 * 32-block; or, with numerics = 1, the reference's own GEMV order on bf16 x
 * and fp32 scales, orc_q8r_gemm), fp16 KV cache with split-K flash decode (with
 * numerics = 1: the bf16 cache and k_attn_head's order, orc_attn_ref), table
 * RoPE, one expf.
 *   operator_norm -> {attention | gated conv} -> post_operator_norm -> +residual
 *   ffn_norm -> gate/up GEMV -> silu(gate)*up -> down GEMV -> post_ffn_norm -> +residual
 * Attention: fused [q | k | v | gate] GEMV (gate = one value per q head), per-head
 * q/k RMSNorm, zero-tail partial RoPE, KV write, attention, sigmoid gate, o_proj.
 * Conv: in_proj [B | C | x] GEMV, gated short conv, out_proj.
 * Sliding-window attention layers (slide_mask) use their own RoPE table
 * (slide_theta, slide_rot) and see only the last slide_win keys.
 * After the last layer: embedding_norm -> tied LM head (fp32 logits) -> argmax
 * (lfm3_nanode.cu:6183, 5171-5179, 6229).
 *
 * Synthetic weights (no checkpoint exists offline): tensor t of the model draws
 * from seed + 4*t + part (part 0 codes, 1 scales, 2 fp32 parameters) with the
 * generators of oracle.c; t = 16*layer + slot, embedding t = 4000, final norm
 * t = 4001. Slots: 0 mixer in, 1 mixer out, 2 gate/up, 3 down, 4 operator_norm,
 * 5 post_operator_norm, 6 ffn_norm, 7 post_ffn_norm, 8 q_norm, 9 k_norm,
 * 10 conv taps. Norm weights are 1 + 0.1 z except the two post-mixer norms,
 * which are 4 + 0.4 z: with 1 + 0.1 z the tied embedding dominates the final
 * residual and greedy decoding locks onto the input token. Conv taps are 0.5 z.
 *
 * Prompts are processed layer-major (all positions of a layer, then the next),
 * which gives the same values as one position at a time: every operation of a
 * position reads only that position's inputs and earlier KV / ring state.
 */
#include "oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  int8_t *w;
  uint16_t *s;   /* fp16 scales (the R1 GEMV)                          */
  float *sf;     /* the same scales widened to fp32 (the R2 GEMV)      */
  int N, K;
  /* the slot's source tensors (row offset, rows, bits: 8 = Q8, 4 / 5 =
   * low-bit) and, when one is low-bit, its codes / scales for every row */
  int np, pr0[4], pn[4], pbits[4];
  uint8_t *lq;     /* [N][K], one code per byte                          */
  uint16_t *ls;    /* [N][K/32][2] fp16: d' = 128 d, mn                  */
} q8t;

typedef struct {
  int attn, slide;       /* slide: a sliding-window attention layer */
  q8t in, out, ug, down;
  float *op_norm, *post_op_norm, *ffn_norm, *post_ffn_norm, *q_norm, *k_norm, *taps;
  uint16_t *kc, *vc;    /* fp16 (numerics 1: bf16) [ctx][nkv][hd] */
  uint16_t *ring;       /* bf16 [ntaps][H]      */
} layer_t;

struct orc_model {
  orc_cfg c;
  layer_t *L;
  q8t emb;
  uint16_t *emb16;   /* emb_bf16: the tied table as bf16 [vocab][H] */
  float *final_norm;
  float *rope, *rope_slide;   /* cos/sin tables: full-attention and sliding layers */
  int pos;
  uint16_t *last_hidden;
};

static uint64_t tseed(const orc_cfg *c, int t, int part) { return c->seed + 4ull * (uint64_t)t + (uint64_t)part; }

static void q8_make(q8t *q, const orc_cfg *c, int t, int N, int K) {
  q->N = N; q->K = K;
  q->w = (int8_t *)malloc((size_t)N * K);
  q->s = (uint16_t *)malloc((size_t)N * (K / ORC_QBLK) * 2);
  orc_gen_codes(tseed(c, t, 0), q->w, (size_t)N * K);
  orc_gen_scales(tseed(c, t, 1), q->s, (size_t)N * (K / ORC_QBLK), 0.01f);
  q->sf = (float *)malloc(sizeof(float) * (size_t)N * (K / ORC_QBLK));
  for (size_t i = 0; i < (size_t)N * (K / ORC_QBLK); i++) q->sf[i] = orc_h2f(q->s[i]);
}

/* The slot's source tensors (the .lfm3q8 names, in row order): nsrc of them
 * with the given row counts. A source is low-bit (cfg.lowbit bits) when its
 * layer is in lowbit_mask, its rows are a multiple of 32 and K of 256 (the
 * exporter's dtype 6 / 7 rule, lfm3_nanode.cu:1494-1496) and it is not the
 * attention gate_proj (skip: its index, or -1), which stays Q8 as in the real
 * LFM3 shapes (16 rows). The low-bit parameters of tensor t come from their
 * own streams (t + 5000): codes uniform in [0, 2^B), d' = f16(|z| * 2560 / 2^B)
 * (so w = d q + mn spreads like the Q8 weights), mn = f16(-(2^B - 1)/2 * d'/128
 * + 0.02 z), centring w. */
static void parts_make(q8t *q, const orc_cfg *c, int t, int layer, const int *rows, int nsrc, int skip) {
  const int low = c->lowbit && ((c->lowbit_mask >> layer) & 1u);
  int r0 = 0, any = 0;
  q->np = nsrc;
  for (int i = 0; i < nsrc; i++) {
    q->pr0[i] = r0;
    q->pn[i] = rows[i];
    q->pbits[i] = (low && i != skip && rows[i] % 32 == 0 && q->K % 256 == 0) ? c->lowbit : 8;
    any |= q->pbits[i] != 8;
    r0 += rows[i];
  }
  if (!any) return;
  const int B = c->lowbit, G = q->K / ORC_QBLK;
  const size_t n = (size_t)q->N * q->K, ng = (size_t)q->N * G;
  q->lq = (uint8_t *)malloc(n);
  q->ls = (uint16_t *)malloc(ng * 4);
  const uint64_t sq = tseed(c, 5000 + t, 0), sd = tseed(c, 5000 + t, 1), sm = tseed(c, 5000 + t, 2);
  for (size_t i = 0; i < n; i++) q->lq[i] = (uint8_t)(orc_sm64_at(sq, i) >> (64 - B));
  uint16_t *dp = (uint16_t *)malloc(ng * 2);
  float *z = (float *)malloc(sizeof(float) * ng);
  orc_gen_scales(sd, dp, ng, 2560.0f / (float)(1 << B));
  orc_gen_normal(sm, z, ng);
  for (size_t g = 0; g < ng; g++) {
    q->ls[2 * g] = dp[g];
    q->ls[2 * g + 1] = orc_f2h(-(float)((1 << B) - 1) * 0.5f * orc_h2f(dp[g]) / 128.0f + 0.02f * z[g]);
  }
  free(dp);
  free(z);
}

static float *vec_make(const orc_cfg *c, int t, int n, float a, float b) {
  float *v = (float *)malloc(sizeof(float) * (size_t)n);
  orc_gen_affine(tseed(c, t, 2), v, (size_t)n, a, b);
  return v;
}

orc_model *orc_model_create(const orc_cfg *cfg) {
  /* the bf16 table and low-bit tensors take bf16 activations: the reference's
   * own GEMV numerics (numerics 1) */
  if ((cfg->emb_bf16 || cfg->lowbit) && cfg->numerics != 1) return NULL;
  if (cfg->lowbit != 0 && cfg->lowbit != 4 && cfg->lowbit != 5) return NULL;
  orc_model *m = (orc_model *)calloc(1, sizeof(orc_model));
  m->c = *cfg;
  const orc_cfg *c = &m->c;
  const int H = c->hidden, F = c->ffn, qd = c->nh * c->hd, kvd = c->nkv * c->hd;
  m->L = (layer_t *)calloc((size_t)c->nlayers, sizeof(layer_t));
  for (int l = 0; l < c->nlayers; l++) {
    layer_t *L = &m->L[l];
    const int t0 = 16 * l;
    L->attn = (int)((c->attn_mask >> l) & 1u);
    L->slide = L->attn && ((c->slide_mask >> l) & 1u);
    if (L->attn) {
      const int rin[4] = {qd, kvd, kvd, c->nh};
      q8_make(&L->in, c, t0 + 0, qd + 2 * kvd + c->nh, H);
      parts_make(&L->in, c, t0 + 0, l, rin, 4, 3);
      q8_make(&L->out, c, t0 + 1, H, qd);
      parts_make(&L->out, c, t0 + 1, l, &H, 1, -1);
      L->q_norm = vec_make(c, t0 + 8, c->hd, 1.0f, 0.1f);
      L->k_norm = vec_make(c, t0 + 9, c->hd, 1.0f, 0.1f);
      L->kc = (uint16_t *)calloc((size_t)c->ctx * kvd, 2);
      L->vc = (uint16_t *)calloc((size_t)c->ctx * kvd, 2);
    } else {
      const int rin = 3 * H;
      q8_make(&L->in, c, t0 + 0, 3 * H, H);
      parts_make(&L->in, c, t0 + 0, l, &rin, 1, -1);
      q8_make(&L->out, c, t0 + 1, H, H);
      parts_make(&L->out, c, t0 + 1, l, &H, 1, -1);
      L->taps = vec_make(c, t0 + 10, H * c->ntaps, 0.0f, 0.5f);
      L->ring = (uint16_t *)calloc((size_t)c->ntaps * H, 2);
    }
    const int rug[2] = {F, F};
    q8_make(&L->ug, c, t0 + 2, 2 * F, H);
    parts_make(&L->ug, c, t0 + 2, l, rug, 2, -1);
    q8_make(&L->down, c, t0 + 3, H, F);
    parts_make(&L->down, c, t0 + 3, l, &H, 1, -1);
    L->op_norm = vec_make(c, t0 + 4, H, 1.0f, 0.1f);
    L->post_op_norm = vec_make(c, t0 + 5, H, 4.0f, 0.4f);
    L->ffn_norm = vec_make(c, t0 + 6, H, 1.0f, 0.1f);
    L->post_ffn_norm = vec_make(c, t0 + 7, H, 4.0f, 0.4f);
  }
  q8_make(&m->emb, c, 4000, c->vocab, H);
  if (c->emb_bf16) {   /* the bf16 table: each row is the Q8 table's embedding row */
    m->emb16 = (uint16_t *)malloc((size_t)c->vocab * H * 2);
    for (int v = 0; v < c->vocab; v++) orc_embed_row(m->emb.w, m->emb.s, v, H, m->emb16 + (size_t)v * H);
  }
  m->final_norm = vec_make(c, 4001, H, 1.0f, 0.1f);
  m->rope = (float *)malloc(sizeof(float) * (size_t)c->ctx * (c->rot / 2) * 2 + 8);
  orc_rope_table(m->rope, c->ctx, c->hd, c->rot, c->theta);
  if (c->slide_mask) {
    m->rope_slide = (float *)malloc(sizeof(float) * (size_t)c->ctx * (c->slide_rot / 2) * 2 + 8);
    orc_rope_table(m->rope_slide, c->ctx, c->hd, c->slide_rot, c->slide_theta);
  }
  m->last_hidden = (uint16_t *)calloc((size_t)H, 2);
  m->pos = 0;
  return m;
}

void orc_model_reset(orc_model *m) {
  const orc_cfg *c = &m->c;
  for (int l = 0; l < c->nlayers; l++) {
    layer_t *L = &m->L[l];
    if (L->attn) {
      memset(L->kc, 0, (size_t)c->ctx * c->nkv * c->hd * 2);
      memset(L->vc, 0, (size_t)c->ctx * c->nkv * c->hd * 2);
    } else {
      memset(L->ring, 0, (size_t)c->ntaps * c->hidden * 2);
    }
  }
  m->pos = 0;
}

static void q8_free(q8t *q) { free(q->w); free(q->s); free(q->sf); free(q->lq); free(q->ls); }

void orc_model_free(orc_model *m) {
  if (!m) return;
  for (int l = 0; l < m->c.nlayers; l++) {
    layer_t *L = &m->L[l];
    q8_free(&L->in); q8_free(&L->out); q8_free(&L->ug); q8_free(&L->down);
    free(L->op_norm); free(L->post_op_norm); free(L->ffn_norm); free(L->post_ffn_norm);
    free(L->q_norm); free(L->k_norm); free(L->taps); free(L->kc); free(L->vc); free(L->ring);
  }
  free(m->L);
  q8_free(&m->emb);
  free(m->emb16);
  free(m->final_norm); free(m->rope); free(m->rope_slide); free(m->last_hidden);
  free(m);
}

int orc_model_tensor(orc_model *m, int layer, int slot, const void **p0, const void **p1,
                     int *N, int *K) {
  if (layer == -1) {
    if (slot == 0) { *p0 = m->emb.w; *p1 = m->emb.s; *N = m->emb.N; *K = m->emb.K; return 0; }
    if (slot == 1) { *p0 = m->final_norm; *p1 = NULL; *N = 1; *K = m->c.hidden; return 0; }
    if (slot == 2) { *p0 = m->rope; *p1 = NULL; *N = m->c.ctx; *K = m->c.rot; return 0; }
    if (slot == 3 && m->emb16) { *p0 = m->emb16; *p1 = NULL; *N = m->c.vocab; *K = m->c.hidden; return 0; }
    return -1;
  }
  if (layer < 0 || layer >= m->c.nlayers) return -1;
  layer_t *L = &m->L[layer];
  q8t *q = NULL;
  const float *v = NULL;
  int n = m->c.hidden;
  switch (slot) {
    case 0: q = &L->in; break;
    case 1: q = &L->out; break;
    case 2: q = &L->ug; break;
    case 3: q = &L->down; break;
    case 4: v = L->op_norm; break;
    case 5: v = L->post_op_norm; break;
    case 6: v = L->ffn_norm; break;
    case 7: v = L->post_ffn_norm; break;
    case 8: v = L->q_norm; n = m->c.hd; break;
    case 9: v = L->k_norm; n = m->c.hd; break;
    case 10: v = L->taps; n = m->c.hidden * m->c.ntaps; break;
    default: return -1;
  }
  if (q) { *p0 = q->w; *p1 = q->s; *N = q->N; *K = q->K; return 0; }
  if (!v) return -1;
  *p0 = v; *p1 = NULL; *N = 1; *K = n;
  return 0;
}

static q8t *slot_q8(orc_model *m, int layer, int slot) {
  if (layer < 0 || layer >= m->c.nlayers) return NULL;
  layer_t *L = &m->L[layer];
  switch (slot) {
    case 0: return &L->in;
    case 1: return &L->out;
    case 2: return &L->ug;
    case 3: return &L->down;
    default: return NULL;
  }
}

int orc_model_parts(orc_model *m, int layer, int slot, int *r0, int *n, int *bits) {
  const q8t *q = slot_q8(m, layer, slot);
  if (!q) return -1;
  for (int i = 0; i < q->np; i++) { r0[i] = q->pr0[i]; n[i] = q->pn[i]; bits[i] = q->pbits[i]; }
  return q->np;
}

int orc_model_lowbit(orc_model *m, int layer, int slot, const uint8_t **qq, const uint16_t **ss, int *N, int *K) {
  const q8t *q = slot_q8(m, layer, slot);
  if (!q || !q->lq) return -1;
  *qq = q->lq; *ss = q->ls; *N = q->N; *K = q->K;
  return 0;
}

int orc_model_debug_hidden(orc_model *m, uint16_t *out) {
  memcpy(out, m->last_hidden, (size_t)m->c.hidden * 2);
  return 0;
}

/* y_f32[T][N] = W . x_bf16[T][K] in the model's GEMV numerics: R1 quantizes
 * each position's row to Q8_0 and runs the R1 GEMM; R2 runs the reference's
 * own order on bf16 x and fp32 scales (orc_q8r_gemm). */
static int g_numerics;   /* set per feed from the model's configuration */
static void gemm_f32(const q8t *W, const uint16_t *x, float *y, int T, int8_t *qx, float *dx) {
  const int K = W->K, N = W->N, nb = K / ORC_QBLK;
  if (g_numerics == 1 && W->lq) {
    /* per source tensor (gemv per name, layer_body 3739-3856): a Q8 part in
     * the R2 order, a low-bit part one position at a time (pf_gemv_T,
     * lfm3_nanode.cu:4846-4848) in the Q4 / Q5 order */
    float *tmp = (float *)malloc(sizeof(float) * (size_t)T * N);
    for (int i = 0; i < W->np; i++) {
      const int r0 = W->pr0[i], n = W->pn[i];
      if (W->pbits[i] == 8) {
        orc_q8r_gemm(W->w + (size_t)r0 * K, W->sf + (size_t)r0 * nb, x, tmp, n, K, T);
      } else {
        for (int t = 0; t < T; t++)
          orc_qlow_gemv(W->lq + (size_t)r0 * K, W->ls + (size_t)r0 * nb * 2, x + (size_t)t * K, tmp + (size_t)t * n,
                        n, K);
      }
      for (int t = 0; t < T; t++) memcpy(y + (size_t)t * N + r0, tmp + (size_t)t * n, sizeof(float) * (size_t)n);
    }
    free(tmp);
    return;
  }
  if (g_numerics == 1) {
    orc_q8r_gemm(W->w, W->sf, x, y, N, K, T);
    return;
  }
  for (int t = 0; t < T; t++) orc_q8_quant_bf16(x + (size_t)t * K, K, qx + (size_t)t * K, dx + (size_t)t * nb);
  orc_q8_gemm(W->w, W->s, qx, dx, y, N, K, T);
}

/* y_bf16[T][N] = bf16 of the GEMM above (k_combine_bf, 336-343). */
static void gemm_bf16(const q8t *W, const uint16_t *x, uint16_t *y, int T, float *scratch_f,
                      int8_t *qx, float *dx) {
  gemm_f32(W, x, scratch_f, T, qx, dx);
  for (size_t i = 0; i < (size_t)T * W->N; i++) y[i] = orc_f2bf(scratch_f[i]);
}

int orc_model_feed(orc_model *m, const int32_t *tok, int T, float *logits_out) {
  const orc_cfg *c = &m->c;
  const int H = c->hidden, F = c->ffn, qd = c->nh * c->hd, kvd = c->nkv * c->hd;
  const int nin = qd + 2 * kvd + c->nh;
  int wmax = 3 * H > 2 * F ? 3 * H : 2 * F;
  if (nin > wmax) wmax = nin;
  int kmax = F > H ? F : H;
  if (qd > kmax) kmax = qd;
  if (m->pos + T > c->ctx) return -1;
  g_numerics = c->numerics;
  uint16_t *X = (uint16_t *)malloc((size_t)T * H * 2);
  uint16_t *H1 = (uint16_t *)malloc((size_t)T * kmax * 2);
  uint16_t *H2 = (uint16_t *)malloc((size_t)T * kmax * 2);
  uint16_t *H3 = (uint16_t *)malloc((size_t)T * H * 2);
  uint16_t *W = (uint16_t *)malloc((size_t)T * wmax * 2);
  float *yf = (float *)malloc(sizeof(float) * (size_t)T * (wmax > c->vocab ? wmax : c->vocab));
  int8_t *qx = (int8_t *)malloc((size_t)T * kmax);
  float *dx = (float *)malloc(sizeof(float) * (size_t)T * (kmax / ORC_QBLK));

  for (int t = 0; t < T; t++) {
    if (m->emb16) {   /* the bf16 row as stored (lfm3_nanode.cu:6062-6076); an id off the table: zeros */
      if (tok[t] >= 0 && tok[t] < c->vocab) memcpy(X + (size_t)t * H, m->emb16 + (size_t)tok[t] * H, (size_t)H * 2);
      else memset(X + (size_t)t * H, 0, (size_t)H * 2);
    } else {
      orc_embed_row(m->emb.w, m->emb.s, tok[t], H, X + (size_t)t * H);
    }
  }

  for (int l = 0; l < c->nlayers; l++) {
    layer_t *L = &m->L[l];
    for (int t = 0; t < T; t++) orc_rmsnorm(X + (size_t)t * H, L->op_norm, H1 + (size_t)t * H, H, c->eps);
    if (L->attn) {
      gemm_bf16(&L->in, H1, W, T, yf, qx, dx);                 /* [T][nin] */
      for (int t = 0; t < T; t++) {
        uint16_t *row = W + (size_t)t * nin;
        uint16_t *q = row, *k = row + qd, *v = row + qd + kvd, *g = row + qd + 2 * kvd;
        const int pos = m->pos + t;
        orc_headnorm(q, L->q_norm, c->nh, c->hd, c->eps);
        orc_headnorm(k, L->k_norm, c->nkv, c->hd, c->eps);
        /* per layer type (lfm3_nanode.cu:3756-3765, 5416-5422, 5486-5487): full
         * attention rotates rot dims with theta; sliding attention its own
         * rot (all of hd) with its own base and sees a window of keys */
        const float *rt = L->slide ? m->rope_slide : m->rope;
        const int rot = L->slide ? c->slide_rot : c->rot;
        orc_rope(q, rt, pos, c->nh, c->hd, rot);
        orc_rope(k, rt, pos, c->nkv, c->hd, rot);
        /* R1: fp16 cache, split-K flash decode; numerics 1: the bf16 rows as
         * k_kv_write copies them and k_attn_head's order */
        for (int i = 0; i < kvd; i++) {
          L->kc[(size_t)pos * kvd + i] = c->numerics == 1 ? k[i] : orc_f2h(orc_bf2f(k[i]));
          L->vc[(size_t)pos * kvd + i] = c->numerics == 1 ? v[i] : orc_f2h(orc_bf2f(v[i]));
        }
        uint16_t *a = H2 + (size_t)t * qd;
        if (c->numerics == 1)
          orc_attn_ref(q, L->kc, L->vc, a, pos + 1, c->nh, c->nkv, c->hd, 1.0f / sqrtf((float)c->hd),
                       L->slide ? c->slide_win : 0);
        else
          orc_attn(q, L->kc, L->vc, a, pos + 1, c->nh, c->nkv, c->hd, 1.0f / sqrtf((float)c->hd),
                   L->slide ? c->slide_win : 0);
        orc_sigmoid_gate(g, a, c->nh, c->hd);
      }
      gemm_bf16(&L->out, H2, H1, T, yf, qx, dx);               /* [T][H] */
    } else {
      gemm_bf16(&L->in, H1, W, T, yf, qx, dx);                 /* [T][3H] */
      for (int t = 0; t < T; t++)
        orc_conv_step(L->ring, L->taps, W + (size_t)t * 3 * H, H2 + (size_t)t * H, H, c->ntaps);
      gemm_bf16(&L->out, H2, H1, T, yf, qx, dx);
    }
    for (int t = 0; t < T; t++) {
      orc_rmsnorm(H1 + (size_t)t * H, L->post_op_norm, H3 + (size_t)t * H, H, c->eps);
      orc_add(X + (size_t)t * H, H3 + (size_t)t * H, X + (size_t)t * H, H);
      orc_rmsnorm(X + (size_t)t * H, L->ffn_norm, H1 + (size_t)t * H, H, c->eps);
    }
    gemm_bf16(&L->ug, H1, W, T, yf, qx, dx);                   /* [T][2F] */
    for (int t = 0; t < T; t++)
      orc_silu_mul(W + (size_t)t * 2 * F, W + (size_t)t * 2 * F + F, H2 + (size_t)t * F, F);
    gemm_bf16(&L->down, H2, H1, T, yf, qx, dx);                /* [T][H] */
    for (int t = 0; t < T; t++) {
      orc_rmsnorm(H1 + (size_t)t * H, L->post_ffn_norm, H3 + (size_t)t * H, H, c->eps);
      orc_add(X + (size_t)t * H, H3 + (size_t)t * H, X + (size_t)t * H, H);
    }
  }
  const uint16_t *xl = X + (size_t)(T - 1) * H;
  memcpy(m->last_hidden, xl, (size_t)H * 2);
  orc_rmsnorm(xl, m->final_norm, H1, H, c->eps);
  if (m->emb16) orc_bf16_gemv(m->emb16, H1, yf, c->vocab, H);   /* lm_head_bf16 (3536-3573) */
  else gemm_f32(&m->emb, H1, yf, 1, qx, dx);
  const int id = orc_argmax(yf, c->vocab);
  if (logits_out) memcpy(logits_out, yf, sizeof(float) * (size_t)c->vocab);
  m->pos += T;
  free(X); free(H1); free(H2); free(H3); free(W); free(yf); free(qx); free(dx);
  return id;
}

void orc_model_greedy(orc_model *m, const int32_t *prompt, int n_prompt, int n_steps,
                      int32_t *ids) {
  orc_model_reset(m);
  int id = orc_model_feed(m, prompt, n_prompt, NULL);
  ids[0] = id;
  for (int s = 1; s < n_steps; s++) {
    const int32_t t = id;
    id = orc_model_feed(m, &t, 1, NULL);
    ids[s] = id;
  }
}
