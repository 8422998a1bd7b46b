// engine.cpp -- the C++ host side of the LFM3-style backbone on one MI355X.
//
// Keeps the reference's host contract (lfm3_nanode.cu): arenas allocated once
// and never resized (5431), one launch stream, a per-layer call sequence that
// restates layer_body (3739-3856) for T=1 and layer_chunk_T (4997-5131) for a
// prefill chunk, the embedding_norm + tied LM head + argmax after the last layer
// (6183, 5171-5179, 6229). Every device step is a C-ABI entry point of this
// library; the engine owns buffers and ordering only.
//
// Layer (attention):  rmsnorm(op_norm) -> Q8 -> [q|k|v|gate] GEMV -> q/k norm +
//   RoPE + fp16 KV write -> split-K attention + sigmoid gate -> Q8 -> o_proj
// Layer (conv):       rmsnorm(op_norm) -> Q8 -> [B|C|x] GEMV -> gated conv -> Q8
//   -> out_proj
// then:  post_operator_norm + residual + ffn_norm -> Q8 -> gate/up GEMV ->
//   silu(gate)*up -> Q8 -> down GEMV -> post_ffn_norm + residual + next norm -> Q8.
// The residual adds are fused into the following norm (one kernel per
// "rms1 -> eadd -> rms1" triple of layer_body, same values and roundings).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <memory>
#include <string>
#include <vector>

#include "pq_host.h"
#include "pq_internal.h"

namespace pq {

// A source tensor of a slot as the .lfm3q8 file lists it (layer_body runs one
// gemv per name, 3739-3856): rows r0 .. r0 + n of the slot; bits 8 = Q8 (the
// slot's own row-major arrays), 4 / 5 = the exporter's pre-tiled Q4 / Q5
// payload (dtype 6 / 7, pc and ps on the device), which gemv hands to
// qlow_gemv (1916-1923).
struct Part {
  int r0 = 0, n = 0, bits = 8;
  uint8_t *pc = nullptr;
  uint16_t *ps = nullptr;
};

// A Q8 weight on the device. PQ_NUMERICS_Q8: packed tiles (pc) and fp16
// scales (ps). PQ_NUMERICS_REF: row-major codes (pc) and fp32 scales (sf), as
// the .lfm3q8 file stores them.
struct Q8Dev {
  int8_t *pc = nullptr;
  uint16_t *ps = nullptr;
  float *sf = nullptr;
  int N = 0, K = 0;
  bool gate_up = false;  // Q8: packed by pq_q8_pack_gate_up (rows interleaved in groups of 32)
  std::vector<Part> parts;   // non-empty when a source is low-bit: each part runs its own GEMV
  bool split() const { return !parts.empty(); }
};

struct LayerDev {
  int attn = 0, slide = 0;   // slide: sliding-window attention (its own RoPE table, rot and window)
  Q8Dev in, out, ug, down;
  float *op_norm = nullptr, *post_op_norm = nullptr, *ffn_norm = nullptr, *post_ffn_norm = nullptr;
  float *q_norm = nullptr, *k_norm = nullptr, *taps = nullptr;
  uint16_t *kc = nullptr, *vc = nullptr;
  uint16_t *rings[2] = {nullptr, nullptr};  // conv ring ping-pong pair; rings[rc] is current
  int rc = 0;
  uint16_t *ring() const { return rings[rc]; }
};

struct Engine {
  pq_model_cfg c{};
  hipStream_t st = nullptr;
  std::vector<LayerDev> L;
  Q8Dev emb;
  float *final_norm = nullptr, *rope = nullptr, *rope_slide = nullptr;
  int pos = 0, tmax = 0, qd = 0, kvd = 0, nin = 0, last_t = 1;
  bool fused = false;             // T=1 steps through the fused kernels (when supported)
  bool graph = true;              // fused steps replay as captured HIP graphs
  int32_t *ctr = nullptr;         // device [id slot, position] of the replayed step
  int32_t hctr[2] = {0, 0};       // its host source (outlives the async upload)
  hipGraphExec_t gexec[2] = {nullptr, nullptr};  // the step, by conv-ring parity
  uint16_t *Xd[2] = {nullptr, nullptr};  // decode residual ping-pong
  const uint16_t *last_resid = nullptr;
  const uint16_t *step_resid = nullptr;  // where a replayed decode step leaves the residual
  float *parts = nullptr;
  int nparts = 0;
  // activations: the residual stream X, the layer input qin/din (Q8_0) and
  // the prompt's token ids tokd hold every position of the context; the rest
  // is sized for one chunk of tmax positions
  uint16_t *X = nullptr, *Hb = nullptr, *Wd = nullptr, *A = nullptr;
  int8_t *qx = nullptr, *qin = nullptr;
  uint16_t *xin = nullptr;        // PQ_NUMERICS_REF: the bf16 layer input of every position
  float *dx = nullptr, *din = nullptr, *logits = nullptr;
  int32_t *tok = nullptr, *tokd = nullptr, *ids = nullptr;
  int max_ids = 0;
  void *attn_ws = nullptr;
  size_t attn_ws_bytes = 0;
  void *gemm_ws = nullptr;
  size_t gemm_ws_bytes = 0;
  // from a blob (PQ_NUMERICS_REF only): the tied table as bf16 [vocab][H]
  // (dtype 3; null for a Q8 table), the Q4 / Q5 GEMV workspace and the
  // [tmax][wide] staging of a part's rows at T > 1
  uint16_t *emb16 = nullptr;
  bool emb_bf16 = false;
  void *qlow_ws = nullptr;
  size_t qlow_ws_bytes = 0;
  char *ptmp = nullptr;
  int nparts16 = 0;
  std::vector<void *> allocs;
  bool loaded = false;

  ~Engine() {
    if (st) hipStreamSynchronize(st);
    for (hipGraphExec_t g : gexec)
      if (g) hipGraphExecDestroy(g);
    for (void *p : allocs) hipFree(p);
    if (st) hipStreamDestroy(st);
  }

  // frees an allocation dalloc made (null: nothing)
  void dfree(void *p) {
    if (!p) return;
    for (size_t i = 0; i < allocs.size(); i++)
      if (allocs[i] == p) {
        hipFree(p);
        allocs.erase(allocs.begin() + (long)i);
        return;
      }
  }

  template <typename T>
  int dalloc(T **p, size_t count) {
    void *q = nullptr;
    const size_t bytes = count * sizeof(T) ? count * sizeof(T) : 16;
    const hipError_t e = hipMalloc(&q, bytes);
    if (e != hipSuccess) return fail(PQ_ERR_LAUNCH, "hipMalloc(%zu) failed: %s", bytes, hipGetErrorString(e));
    allocs.push_back(q);
    *p = static_cast<T *>(q);
    return PQ_OK;
  }
};

#define PQ_TRY(expr)             \
  do {                           \
    const int _rc = (expr);      \
    if (_rc != PQ_OK) return _rc; \
  } while (0)

static bool ref_numerics(const Engine &E) { return E.c.numerics == PQ_NUMERICS_REF; }

static int alloc_q8(Engine &E, Q8Dev &q, int N, int K) {
  q.N = N;
  q.K = K;
  if (ref_numerics(E)) {
    PQ_TRY(E.dalloc(&q.pc, (size_t)N * K));
    PQ_TRY(E.dalloc(&q.sf, (size_t)N * (K / 32)));
    return PQ_OK;
  }
  PQ_TRY(E.dalloc(&q.pc, pq_q8_packed_codes_bytes(N, K)));
  PQ_TRY(E.dalloc(&q.ps, pq_q8_packed_scales_bytes(N, K) / 2));
  return PQ_OK;
}

static int create(Engine &E, const pq_model_cfg &c) {
  E.c = c;
  const int H = c.hidden, F = c.ffn;
  E.qd = c.nh * c.hd;
  E.kvd = c.nkv * c.hd;
  E.nin = E.qd + 2 * E.kvd + c.nh;
  E.tmax = c.prefill_chunk;
  if (hipStreamCreateWithFlags(&E.st, hipStreamNonBlocking) != hipSuccess)
    return fail(PQ_ERR_LAUNCH, "hipStreamCreate failed");
  E.L.resize(c.nlayers);
  for (int l = 0; l < c.nlayers; l++) {
    LayerDev &D = E.L[l];
    D.attn = (int)((c.attn_mask >> l) & 1u);
    D.slide = D.attn && ((c.slide_mask >> l) & 1u);
    if (D.attn) {
      PQ_TRY(alloc_q8(E, D.in, E.nin, H));
      PQ_TRY(alloc_q8(E, D.out, H, E.qd));
      PQ_TRY(E.dalloc(&D.q_norm, c.hd));
      PQ_TRY(E.dalloc(&D.k_norm, c.hd));
      PQ_TRY(E.dalloc(&D.kc, (size_t)c.ctx * E.kvd));
      PQ_TRY(E.dalloc(&D.vc, (size_t)c.ctx * E.kvd));
    } else {
      PQ_TRY(alloc_q8(E, D.in, 3 * H, H));
      PQ_TRY(alloc_q8(E, D.out, H, H));
      PQ_TRY(E.dalloc(&D.taps, (size_t)H * c.ntaps));
      PQ_TRY(E.dalloc(&D.rings[0], (size_t)H * c.ntaps));
      PQ_TRY(E.dalloc(&D.rings[1], (size_t)H * c.ntaps));
    }
    PQ_TRY(alloc_q8(E, D.ug, 2 * F, H));
    D.ug.gate_up = true;
    PQ_TRY(alloc_q8(E, D.down, H, F));
    PQ_TRY(E.dalloc(&D.op_norm, H));
    PQ_TRY(E.dalloc(&D.post_op_norm, H));
    PQ_TRY(E.dalloc(&D.ffn_norm, H));
    PQ_TRY(E.dalloc(&D.post_ffn_norm, H));
  }
  PQ_TRY(alloc_q8(E, E.emb, c.vocab, H));
  PQ_TRY(E.dalloc(&E.final_norm, H));
  PQ_TRY(E.dalloc(&E.rope, (size_t)c.ctx * (c.rot / 2) * 2 + 2));
  if (c.slide_mask) PQ_TRY(E.dalloc(&E.rope_slide, (size_t)c.ctx * (c.slide_rot / 2) * 2 + 2));
  const int T = E.tmax;
  const int wide = std::max(std::max(3 * H, 2 * F), E.nin);
  const int kmax = std::max(std::max(H, F), E.qd);
  const size_t npos = (size_t)std::max(c.ctx, T);
  PQ_TRY(E.dalloc(&E.X, npos * H));
  PQ_TRY(E.dalloc(&E.qin, npos * H));
  PQ_TRY(E.dalloc(&E.din, npos * (H / 32)));
  PQ_TRY(E.dalloc(&E.tokd, npos));
  if (ref_numerics(E)) PQ_TRY(E.dalloc(&E.xin, npos * H));
  PQ_TRY(E.dalloc(&E.Xd[0], (size_t)H));
  PQ_TRY(E.dalloc(&E.Xd[1], (size_t)H));
  E.nparts = ref_numerics(E) ? pq_q8r_gemv_parts(c.vocab) : pq_q8_gemv_parts(c.vocab, H);
  E.nparts16 = pq_bf16_gemv_parts(c.vocab);
  PQ_TRY(E.dalloc(&E.parts, (size_t)std::max(E.nparts, E.nparts16) * 2));
  PQ_TRY(E.dalloc(&E.Hb, (size_t)T * H));
  PQ_TRY(E.dalloc(&E.Wd, (size_t)T * wide));
  PQ_TRY(E.dalloc(&E.A, (size_t)T * kmax));
  PQ_TRY(E.dalloc(&E.qx, (size_t)T * kmax));
  PQ_TRY(E.dalloc(&E.dx, (size_t)T * kmax / 32));
  PQ_TRY(E.dalloc(&E.logits, (size_t)c.vocab));
  PQ_TRY(E.dalloc(&E.tok, (size_t)T));
  E.max_ids = c.ctx + 1;
  PQ_TRY(E.dalloc(&E.ids, (size_t)E.max_ids));
  PQ_TRY(E.dalloc(&E.ctr, 2));
  E.attn_ws_bytes = pq_attn_workspace_bytes(c.nh, c.hd, c.ctx, T);
  PQ_TRY(E.dalloc(reinterpret_cast<char **>(&E.attn_ws), E.attn_ws_bytes));
  // the split-K GEMM workspace: the largest of the layer shapes at any chunk
  // size up to tmax (pq_engine_set_chunk may shrink the chunk, and the small
  // chunks are the ones that split K)
  const int shapes[6][2] = {{E.nin, H}, {3 * H, H}, {H, E.qd}, {H, H}, {2 * F, H}, {H, F}};
  for (int t = 1; t <= T; t++)
    for (const auto &nk : shapes)
      E.gemm_ws_bytes = std::max(E.gemm_ws_bytes, pq_q8_gemm_workspace_bytes(nk[0], nk[1], t));
  if (E.gemm_ws_bytes) PQ_TRY(E.dalloc(reinterpret_cast<char **>(&E.gemm_ws), E.gemm_ws_bytes));
  return PQ_OK;
}

// ------------------------------------------------------------ weight upload
static float host_h2f(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
  uint32_t u;
  if (e == 0x1f) u = sign | 0x7f800000u | (m << 13);
  else if (e) u = sign | ((e + 112u) << 23) | (m << 13);
  else if (m == 0) u = sign;
  else {   // subnormal: normalize
    int ex = -1;
    uint32_t mm = m;
    do { mm <<= 1; ex++; } while (!(mm & 0x400u));
    u = sign | ((uint32_t)(112 - ex) << 23) | ((mm & 0x3ffu) << 13);
  }
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// fp32 -> binary16 bits, round to nearest even (overflow to inf, NaN kept).
static uint16_t host_f2h(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t sign = (u >> 16) & 0x8000u, e = (u >> 23) & 0xffu, m = u & 0x7fffffu;
  if (e == 0xff) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u | (m >> 13) : 0u));
  const int ex = (int)e - 127 + 15;
  if (ex >= 31) return (uint16_t)(sign | 0x7c00u);
  if (ex <= 0) {   // binary16 subnormal (or zero): shift the full mantissa, round to even
    if (ex < -10) return (uint16_t)sign;
    const uint32_t mm = m | 0x800000u;
    const int sh = 14 - ex;
    uint32_t q = mm >> sh;
    const uint32_t rem = mm & ((1u << sh) - 1), half = 1u << (sh - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    return (uint16_t)(sign | q);
  }
  uint32_t q = ((uint32_t)ex << 10) | (m >> 13);
  const uint32_t rem = m & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;   // a carry into the exponent is still right
  return (uint16_t)(sign | q);
}

// One Q8 weight, row-major codes [N][K] with scales [N][K/32] given either as
// fp16 bits (s16) or as fp32 (s32), onto the device in the engine's format:
// Q8 numerics pack it (fp32 scales must be fp16 values: the GEMV's scales
// are fp16, and a scale fp16 cannot hold is refused with a count instead of
// being rounded); reference numerics keep the codes as they are and the
// scales as fp32 (fp16 widens exactly).
static int upload_q8(Engine &E, Q8Dev &q, const int8_t *codes, const uint16_t *s16, const float *s32) {
  const size_t nc = (size_t)q.N * q.K, ns = (size_t)q.N * (q.K / 32);
  if (ref_numerics(E)) {
    std::vector<float> wide;
    if (s16) {
      wide.resize(ns);
      for (size_t i = 0; i < ns; i++) wide[i] = host_h2f(s16[i]);
      s32 = wide.data();
    }
    if (hipMemcpyAsync(q.pc, codes, nc, hipMemcpyHostToDevice, E.st) != hipSuccess ||
        hipMemcpyAsync(q.sf, s32, ns * 4, hipMemcpyHostToDevice, E.st) != hipSuccess ||
        hipStreamSynchronize(E.st) != hipSuccess)
      return fail(PQ_ERR_LAUNCH, "weight upload failed");
    return PQ_OK;
  }
  std::vector<uint16_t> narrow;
  if (!s16) {
    narrow.resize(ns);
    size_t inexact = 0, tiny = 0;
    for (size_t i = 0; i < ns; i++) {
      narrow[i] = host_f2h(s32[i]);
      uint32_t a, b;
      const float back = host_h2f(narrow[i]);
      memcpy(&a, &s32[i], 4);
      memcpy(&b, &back, 4);
      if (a != b) {
        inexact++;
        if (fabsf(s32[i]) < 6.103515625e-05f) tiny++;   // below the fp16 normal range
      }
    }
    if (inexact)
      return fail(PQ_ERR_DATA,
                  "%zu of %zu fp32 weight scales of a [%d x %d] tensor are not fp16 values (%zu below the fp16 "
                  "normal range); the Q8 numerics would round them -- use PQ_NUMERICS_REF, which keeps fp32 scales",
                  inexact, ns, q.N, q.K, tiny);
    s16 = narrow.data();
  }
  int8_t *dc = nullptr;
  uint16_t *ds = nullptr;
  if (hipMalloc(&dc, nc) != hipSuccess) return fail(PQ_ERR_LAUNCH, "hipMalloc staging failed");
  if (hipMalloc(&ds, ns * 2) != hipSuccess) {
    hipFree(dc);
    return fail(PQ_ERR_LAUNCH, "hipMalloc staging failed");
  }
  int rc = PQ_OK;
  if (hipMemcpyAsync(dc, codes, nc, hipMemcpyHostToDevice, E.st) != hipSuccess ||
      hipMemcpyAsync(ds, s16, ns * 2, hipMemcpyHostToDevice, E.st) != hipSuccess)
    rc = fail(PQ_ERR_LAUNCH, "weight upload failed");
  if (rc == PQ_OK)
    rc = q.gate_up ? pq_q8_pack_gate_up(dc, ds, q.N / 2, q.K, q.pc, q.ps, E.st)
                   : pq_q8_pack(dc, ds, q.N, q.K, q.pc, q.ps, E.st);
  if (hipStreamSynchronize(E.st) != hipSuccess && rc == PQ_OK) rc = fail(PQ_ERR_LAUNCH, "weight pack failed");
  hipFree(dc);
  hipFree(ds);
  return rc;
}

static int upload_f32(Engine &E, float *dst, const float *src, size_t n) {
  if (hipMemcpyAsync(dst, src, n * 4, hipMemcpyHostToDevice, E.st) != hipSuccess ||
      hipStreamSynchronize(E.st) != hipSuccess)
    return fail(PQ_ERR_LAUNCH, "upload failed");
  return PQ_OK;
}

static Q8Dev *q8_slot(Engine &E, int layer, int slot) {
  if (layer == -1) return slot == 0 ? &E.emb : nullptr;
  if (layer < 0 || layer >= (int)E.L.size()) return nullptr;
  LayerDev &D = E.L[layer];
  switch (slot) {
    case 0: return &D.in;
    case 1: return &D.out;
    case 2: return &D.ug;
    case 3: return &D.down;
    default: return nullptr;
  }
}

static float *vec_slot(Engine &E, int layer, int slot, size_t *n) {
  const int H = E.c.hidden;
  if (layer == -1) {
    if (slot == 1) { *n = H; return E.final_norm; }
    return nullptr;
  }
  if (layer < 0 || layer >= (int)E.L.size()) return nullptr;
  LayerDev &D = E.L[layer];
  *n = H;
  switch (slot) {
    case 4: return D.op_norm;
    case 5: return D.post_op_norm;
    case 6: return D.ffn_norm;
    case 7: return D.post_ffn_norm;
    case 8: *n = E.c.hd; return D.q_norm;
    case 9: *n = E.c.hd; return D.k_norm;
    case 10: *n = (size_t)H * E.c.ntaps; return D.taps;
    default: return nullptr;
  }
}

static void rope_table(std::vector<float> &cs, int ctx, int hd, int rot, float theta) {
  const int half = rot / 2;
  cs.assign((size_t)ctx * half * 2 + 2, 0.0f);
  for (int p = 0; p < ctx; p++)
    for (int i = 0; i < half; i++) {
      // build_invf (lfm3_nanode.cu:3719-3723): float powf and a float divide.
      const float invf = 1.0f / powf(theta, (float)(2 * i) / (float)hd);
      const float ang = (float)p * invf;
      cs[((size_t)p * half + i) * 2] = (float)cos((double)ang);
      cs[((size_t)p * half + i) * 2 + 1] = (float)sin((double)ang);
    }
}

// Synthetic weights: tensor t draws from seed + 4t + part (0 codes, 1 scales,
// 2 fp32 parameters); t = 16*layer + slot, embedding 4000, final norm 4001.
static int load_synthetic(Engine &E) {
  const pq_model_cfg &c = E.c;
  auto seed = [&](int t, int part) { return c.seed + 4ull * (uint64_t)t + (uint64_t)part; };
  std::vector<int8_t> codes;
  std::vector<uint16_t> scales;
  std::vector<float> vec;
  auto q8 = [&](Q8Dev &q, int t) -> int {
    codes.resize((size_t)q.N * q.K);
    scales.resize((size_t)q.N * (q.K / 32));
    pq_synth_fill(PQ_SYNTH_CODES, seed(t, 0), codes.data(), codes.size(), 0, 0);
    pq_synth_fill(PQ_SYNTH_SCALES, seed(t, 1), scales.data(), scales.size(), 0.01f, 0);
    return upload_q8(E, q, codes.data(), scales.data(), nullptr);
  };
  auto fv = [&](float *dst, int t, size_t n, float a, float b) -> int {
    vec.resize(n);
    pq_synth_fill(PQ_SYNTH_AFFINE, seed(t, 2), vec.data(), n, a, b);
    return upload_f32(E, dst, vec.data(), n);
  };
  const int H = c.hidden;
  for (int l = 0; l < c.nlayers; l++) {
    LayerDev &D = E.L[l];
    const int t0 = 16 * l;
    PQ_TRY(q8(D.in, t0 + 0));
    PQ_TRY(q8(D.out, t0 + 1));
    PQ_TRY(q8(D.ug, t0 + 2));
    PQ_TRY(q8(D.down, t0 + 3));
    PQ_TRY(fv(D.op_norm, t0 + 4, H, 1.0f, 0.1f));
    PQ_TRY(fv(D.post_op_norm, t0 + 5, H, 4.0f, 0.4f));
    PQ_TRY(fv(D.ffn_norm, t0 + 6, H, 1.0f, 0.1f));
    PQ_TRY(fv(D.post_ffn_norm, t0 + 7, H, 4.0f, 0.4f));
    if (D.attn) {
      PQ_TRY(fv(D.q_norm, t0 + 8, c.hd, 1.0f, 0.1f));
      PQ_TRY(fv(D.k_norm, t0 + 9, c.hd, 1.0f, 0.1f));
    } else {
      PQ_TRY(fv(D.taps, t0 + 10, (size_t)H * c.ntaps, 0.0f, 0.5f));
    }
  }
  PQ_TRY(q8(E.emb, 4000));
  PQ_TRY(fv(E.final_norm, 4001, H, 1.0f, 0.1f));
  return PQ_OK;
}

// One table per attention layer type: full attention (theta, rot) and, with
// sliding layers, their own (slide_theta, slide_rot) -- the reference's
// invf_full / invf_slide (lfm3_nanode.cu:5486-5487).
static int upload_rope(Engine &E) {
  std::vector<float> cs;
  rope_table(cs, E.c.ctx, E.c.hd, E.c.rot, E.c.theta);
  PQ_TRY(upload_f32(E, E.rope, cs.data(), cs.size()));
  if (!E.rope_slide) return PQ_OK;
  rope_table(cs, E.c.ctx, E.c.hd, E.c.slide_rot, E.c.slide_theta);
  return upload_f32(E, E.rope_slide, cs.data(), cs.size());
}

// The attention layer's RoPE table, rotated dims and window.
static const float *layer_rope(const Engine &E, const LayerDev &D) { return D.slide ? E.rope_slide : E.rope; }
static int layer_rot(const Engine &E, const LayerDev &D) { return D.slide ? E.c.slide_rot : E.c.rot; }
static int layer_win(const Engine &E, const LayerDev &D) { return D.slide ? E.c.slide_win : 0; }

// Zero KV caches and conv rings with a kernel-free copy of a zero host buffer
// (allocated once per reset; reset is not on the decode path).
static int reset(Engine &E) {
  std::vector<uint16_t> z;
  for (LayerDev &D : E.L) {
    const size_t n = D.attn ? (size_t)E.c.ctx * E.kvd : (size_t)E.c.hidden * E.c.ntaps;
    z.assign(n, 0);
    if (D.attn) {
      if (hipMemcpyAsync(D.kc, z.data(), n * 2, hipMemcpyHostToDevice, E.st) != hipSuccess ||
          hipMemcpyAsync(D.vc, z.data(), n * 2, hipMemcpyHostToDevice, E.st) != hipSuccess)
        return fail(PQ_ERR_LAUNCH, "reset copy failed");
    } else {
      D.rc = 0;
      if (hipMemcpyAsync(D.rings[0], z.data(), n * 2, hipMemcpyHostToDevice, E.st) != hipSuccess ||
          hipMemcpyAsync(D.rings[1], z.data(), n * 2, hipMemcpyHostToDevice, E.st) != hipSuccess)
        return fail(PQ_ERR_LAUNCH, "reset copy failed");
    }
    if (hipStreamSynchronize(E.st) != hipSuccess) return fail(PQ_ERR_LAUNCH, "reset sync failed");
  }
  E.pos = 0;
  return PQ_OK;
}

// ---------------------------------------------------------------- forward
static int gemm_T(Engine &E, const Q8Dev &w, const int8_t *qx, const float *dx, void *y, int T) {
  if (T == 1) return pq_q8_gemv(w.pc, w.ps, qx, dx, y, PQ_DTYPE_BF16, w.N, w.K, E.st);
  return pq_q8_gemm_ws(w.pc, w.ps, qx, dx, y, PQ_DTYPE_BF16, w.N, w.K, T, E.gemm_ws, E.gemm_ws_bytes, E.st);
}

// Runs n positions whose token ids are in toks (device) through all layers and
// leaves the greedy id of the last position in *next (device). Layer-major: a
// layer runs every chunk of up to tmax positions before the next layer starts,
// so its weights serve all the chunks while they are warm in the Infinity
// Cache (the reference's layer-major prefill order, lfm3_nanode.cu:5935-5955).
// The residual stream X and the layer input qin/din hold every position; the
// chunk's attention sees the KV entries its earlier chunks wrote at this layer
// and the conv ring carries from chunk to chunk, so every position's
// arithmetic is the chunk-major (and the one-position-at-a-time) arithmetic.
// Per chunk the sequence restates layer_body (3739-3856) / layer_chunk_T
// (4997-5131); the "rms1 -> eadd -> rms1" triple that ends a layer writes the
// next layer's Q8_0 input for the chunk's rows.
static int forward(Engine &E, const int32_t *toks, int n, int32_t *next) {
  const pq_model_cfg &c = E.c;
  const int H = c.hidden, F = c.ffn;
  if (n <= 0 || E.pos + n > c.ctx) return fail(PQ_ERR_STATE, "context full: %d + %d > %d", E.pos, n, c.ctx);
  PQ_TRY(pq_embed(E.emb.pc, E.emb.ps, toks, E.X, H, c.vocab, n, E.st));
  PQ_TRY(pq_rmsnorm(E.X, nullptr, E.L[0].op_norm, nullptr, nullptr, E.qin, E.din, H, n, c.eps, E.st));
  const float scale = 1.0f / sqrtf((float)c.hd);
  for (int l = 0; l < c.nlayers; l++) {
    LayerDev &D = E.L[l];
    const float *next_norm = l + 1 < c.nlayers ? E.L[l + 1].op_norm : E.final_norm;
    for (int c0 = 0; c0 < n; c0 += E.tmax) {
      const int T = std::min(E.tmax, n - c0);
      const int pos0 = E.pos + c0;
      uint16_t *Xc = E.X + (size_t)c0 * H;
      int8_t *qin = E.qin + (size_t)c0 * H;
      float *din = E.din + (size_t)c0 * (H / 32);
      PQ_TRY(gemm_T(E, D.in, qin, din, E.Wd, T));
      if (D.attn) {
        PQ_TRY(pq_qk_prep(E.Wd, E.nin, D.q_norm, D.k_norm, layer_rope(E, D), D.kc, D.vc, pos0, c.nh, c.nkv, c.hd,
                          layer_rot(E, D), T, c.eps, E.st));
        PQ_TRY(pq_attn_decode(E.Wd, E.nin, D.kc, D.vc, E.Wd + E.qd + 2 * E.kvd, E.nin, nullptr, 0, E.qx, E.dx, pos0,
                              c.nh, c.nkv, c.hd, T, scale, layer_win(E, D), E.attn_ws, E.attn_ws_bytes, E.st));
      } else {
        PQ_TRY(pq_conv(D.ring(), D.taps, E.Wd, E.A, H, T, c.ntaps, E.st));
        PQ_TRY(pq_q8_quant_bf16(E.A, E.qx, E.dx, H, T, E.st));
      }
      PQ_TRY(gemm_T(E, D.out, E.qx, E.dx, E.Hb, T));
      PQ_TRY(pq_rmsnorm(Xc, E.Hb, D.post_op_norm, D.ffn_norm, nullptr, E.qx, E.dx, H, T, c.eps, E.st));
      PQ_TRY(gemm_T(E, D.ug, E.qx, E.dx, E.Wd, T));
      PQ_TRY(pq_silu_mul_interleaved(E.Wd, nullptr, E.qx, E.dx, F, T, E.st));
      PQ_TRY(gemm_T(E, D.down, E.qx, E.dx, E.Hb, T));
      PQ_TRY(pq_rmsnorm(Xc, E.Hb, D.post_ffn_norm, next_norm, nullptr, qin, din, H, T, c.eps, E.st));
    }
  }
  // tied LM head on the last position's final-normed row
  PQ_TRY(pq_q8_gemv(E.emb.pc, E.emb.ps, E.qin + (size_t)(n - 1) * H, E.din + (size_t)(n - 1) * (H / 32), E.logits,
                    PQ_DTYPE_F32, c.vocab, H, E.st));
  PQ_TRY(pq_argmax(E.logits, c.vocab, next, E.st));
  E.pos += n;
  E.last_t = n;
  E.last_resid = E.X + (size_t)(n - 1) * H;
  return PQ_OK;
}

// Whether an attention layer's decode mixer is one launch (pq_attn_layer_decode:
// head_dim 64 or 128, any window) -- its LDS holds the split partials of the
// whole context; otherwise q/k prep + the split-K attention pair.
static bool mixer_fused_cfg(const pq_model_cfg &c, bool slide) {
  (void)slide;
  const size_t ns = ((size_t)c.ctx + 63) / 64;
  return (c.hd == 64 || c.hd == 128) && ((size_t)c.hd + 8 * 64 + ns * (c.hd + 2)) * 4 + 2 * (size_t)c.hd * 2 <=
                                            160 * 1024;
}
static bool mixer_fused(const Engine &E, const LayerDev &D) { return mixer_fused_cfg(E.c, D.slide != 0); }

// The same layer sequence under PQ_NUMERICS_REF: every GEMV is pq_q8r_gemv
// (the reference's own order on bf16 activations and fp32 scales, row-major
// codes) and the activations between ops stay bf16, as in layer_body; the
// bf16 layer input xin holds every position (the Q8_0 qin's counterpart).
static int gemm_r2(Engine &E, const Q8Dev &w, const uint16_t *x, void *y, int y_dtype, int T) {
  if (!w.split()) return pq_q8r_gemv(w.pc, w.sf, x, y, y_dtype, w.N, w.K, T, E.st);
  // one GEMV per source tensor (gemv per name): a Q8 part over its rows of the
  // slot's arrays; a Q4 / Q5 part, which pf_gemv_T runs one position at a
  // time (4846-4848), as one pq_qlow_gemm over the T positions (the same bits
  // per position) writing y's [T][N] rows in place; at T > 1 a Q8 part's
  // [T][n] rows go through ptmp into y's rows by one strided copy
  const size_t es = y_dtype == PQ_DTYPE_F32 ? 4 : 2;
  for (const Part &p : w.parts) {
    char *dst = T == 1 ? static_cast<char *>(y) + (size_t)p.r0 * es : E.ptmp;
    if (p.bits != 8) {
      if (T == 1)
        PQ_TRY(pq_qlow_gemv_ws(p.pc, p.ps, x, dst, y_dtype, p.n, w.K, p.bits, E.qlow_ws, E.qlow_ws_bytes, E.st));
      else
        PQ_TRY(pq_qlow_gemm(p.pc, p.ps, x, static_cast<char *>(y) + (size_t)p.r0 * es, y_dtype, p.n, w.K, T, w.N,
                            p.bits, E.st));
      continue;
    }
    PQ_TRY(pq_q8r_gemv(w.pc + (size_t)p.r0 * w.K, w.sf + (size_t)p.r0 * (w.K / 32), x, dst, y_dtype, p.n, w.K, T,
                       E.st));
    if (T > 1 && hipMemcpy2DAsync(static_cast<char *>(y) + (size_t)p.r0 * es, (size_t)w.N * es, dst,
                                  (size_t)p.n * es, (size_t)p.n * es, (size_t)T, hipMemcpyDeviceToDevice,
                                  E.st) != hipSuccess)
      return fail(PQ_ERR_LAUNCH, "part copy failed");
  }
  return PQ_OK;
}

// The embedding rows of n device token ids and the tied head on one final-normed
// row, from the Q8 table or the bf16 one.
static int embed_r2(Engine &E, const int32_t *toks, uint16_t *out, int n) {
  if (E.emb_bf16) return pq_embed_bf16(E.emb16, toks, out, E.c.hidden, E.c.vocab, n, E.st);
  return pq_embed_rows(E.emb.pc, E.emb.sf, toks, out, E.c.hidden, E.c.vocab, n, E.st);
}
static int head_r2(Engine &E, const uint16_t *x, float *parts) {
  if (E.emb_bf16) return pq_bf16_gemv(E.emb16, x, E.logits, E.c.vocab, E.c.hidden, parts, E.st);   // lm_head_bf16
  if (parts) return fail(PQ_ERR_ARG, "head_r2: argmax parts come from the fused GEMV");
  return gemm_r2(E, E.emb, x, E.logits, PQ_DTYPE_F32, 1);
}

static int forward_r2(Engine &E, const int32_t *toks, int n, int32_t *next) {
  const pq_model_cfg &c = E.c;
  const int H = c.hidden, F = c.ffn;
  if (n <= 0 || E.pos + n > c.ctx) return fail(PQ_ERR_STATE, "context full: %d + %d > %d", E.pos, n, c.ctx);
  PQ_TRY(embed_r2(E, toks, E.X, n));
  PQ_TRY(pq_rmsnorm(E.X, nullptr, E.L[0].op_norm, nullptr, E.xin, nullptr, nullptr, H, n, c.eps, E.st));
  const float scale = 1.0f / sqrtf((float)c.hd);
  for (int l = 0; l < c.nlayers; l++) {
    LayerDev &D = E.L[l];
    const float *next_norm = l + 1 < c.nlayers ? E.L[l + 1].op_norm : E.final_norm;
    for (int c0 = 0; c0 < n; c0 += E.tmax) {
      const int T = std::min(E.tmax, n - c0);
      const int pos0 = E.pos + c0;
      uint16_t *Xc = E.X + (size_t)c0 * H;
      uint16_t *xin = E.xin + (size_t)c0 * H;
      PQ_TRY(gemm_r2(E, D.in, xin, E.Wd, PQ_DTYPE_BF16, T));
      if (D.attn) {   // k_attn_head's order over the bf16 cache
        PQ_TRY(pq_qk_prep_ref(E.Wd, E.nin, D.q_norm, D.k_norm, layer_rope(E, D), D.kc, D.vc, pos0, c.nh, c.nkv, c.hd,
                              layer_rot(E, D), T, c.eps, E.st));
        PQ_TRY(pq_attn_ref(E.Wd, E.nin, D.kc, D.vc, E.Wd + E.qd + 2 * E.kvd, E.nin, E.A, E.qd, pos0, c.nh, c.nkv,
                           c.hd, T, scale, layer_win(E, D), E.st));
      } else {
        PQ_TRY(pq_conv(D.ring(), D.taps, E.Wd, E.A, H, T, c.ntaps, E.st));
      }
      PQ_TRY(gemm_r2(E, D.out, E.A, E.Hb, PQ_DTYPE_BF16, T));
      PQ_TRY(pq_rmsnorm(Xc, E.Hb, D.post_op_norm, D.ffn_norm, E.A, nullptr, nullptr, H, T, c.eps, E.st));
      PQ_TRY(gemm_r2(E, D.ug, E.A, E.Wd, PQ_DTYPE_BF16, T));      // [gate | up] rows
      PQ_TRY(pq_silu_mul(E.Wd, E.A, nullptr, nullptr, F, T, E.st));
      PQ_TRY(gemm_r2(E, D.down, E.A, E.Hb, PQ_DTYPE_BF16, T));
      PQ_TRY(pq_rmsnorm(Xc, E.Hb, D.post_ffn_norm, next_norm, xin, nullptr, nullptr, H, T, c.eps, E.st));
    }
  }
  // tied LM head (gemv_f, or lm_head_bf16 for a bf16 table: fp32 logits) on
  // the last position's final-normed row
  PQ_TRY(head_r2(E, E.xin + (size_t)(n - 1) * H, nullptr));
  PQ_TRY(pq_argmax(E.logits, c.vocab, next, E.st));
  E.pos += n;
  E.last_t = n;
  E.last_resid = E.X + (size_t)(n - 1) * H;
  return PQ_OK;
}

static int forward_any(Engine &E, const int32_t *toks, int n, int32_t *next) {
  return ref_numerics(E) ? forward_r2(E, toks, n, next) : forward(E, toks, n, next);
}

static bool pow2_range(int v) { return v >= 1024 && v <= 8192 && (v & (v - 1)) == 0; }


// Whether the fused decode kernels take this configuration: a power-of-two
// hidden width of 1024..8192 (the fused GEMV prologues), an FFN width that is
// a multiple of 32 (the SwiGLU epilogue's 32-row groups; a width that is not
// a power of two runs its down projection as the plain Q8_0 GEMV), 3 or 7
// conv taps, and attention the split-K kernels can run (GQA group 1..8).
// Under PQ_NUMERICS_REF the same holds, and the conv prologue (conv layers)
// takes hidden <= 4096.
static bool fused_supported(const pq_model_cfg &c, const char **why) {
  bool conv = false, attn = false;
  for (int l = 0; l < c.nlayers; l++) ((c.attn_mask >> l) & 1u ? attn : conv) = true;
  const int G = c.nkv > 0 ? c.nh / c.nkv : 0;
  *why = nullptr;
  if (!pow2_range(c.hidden)) *why = "hidden must be a power of two in 1024..8192";
  else if (c.ffn % 32 != 0) *why = "ffn must be a multiple of 32";
  else if (conv && c.ntaps != 3 && c.ntaps != 7) *why = "the fused conv prologue takes 3 or 7 taps";
  else if (conv && c.numerics == PQ_NUMERICS_REF && c.hidden > 4096)
    *why = "the reference-numerics conv prologue takes hidden <= 4096";
  else if (attn && G != 1 && G != 2 && G != 4 && G != 8) *why = "GQA group 1, 2, 4 or 8";
  return *why == nullptr;
}

static int forward_decode_r2(Engine &E, bool dev);

// One T=1 decode step through the fused kernels: four GEMV launches per conv
// layer, five per attention layer (incl. the attention mixer), the LM head with
// per-workgroup argmax partials and the final argmax -- 106 launches for the
// 24-layer backbone. Reads the token from E.tok and writes the next one there.
// dev: the position comes from E.ctr[1] and the id is appended at E.ids[E.ctr[0]]
// on the device (the form captured for replay); otherwise E.pos is passed.
static int forward_decode(Engine &E, bool dev) {
  if (ref_numerics(E)) return forward_decode_r2(E, dev);
  const pq_model_cfg &c = E.c;
  const int H = c.hidden;
  if (E.pos + 1 > c.ctx) return fail(PQ_ERR_STATE, "context full: %d + 1 > %d", E.pos, c.ctx);
  uint16_t *xa = E.Xd[0], *xb = E.Xd[1];
  pq_gemv_prologue p;
  auto resnorm = [&](const float *w0, const float *w1) {
    p = pq_gemv_prologue{};
    p.kind = PQ_PRO_RESNORM;
    p.h = E.Hb;
    p.x_in = xa;
    p.x_out = xb;
    p.w0 = w0;
    p.w1 = w1;
    p.eps = c.eps;
    std::swap(xa, xb);
  };
  auto gemv = [&](const Q8Dev &w, void *y, int dt, float *parts) {
    return pq_q8_gemv_fused(w.pc, w.ps, &p, y, dt, w.N, w.K, parts, E.st);
  };
  const float scale = 1.0f / sqrtf((float)c.hd);
  for (int l = 0; l < c.nlayers; l++) {
    LayerDev &D = E.L[l];
    if (l == 0) {
      p = pq_gemv_prologue{};
      p.kind = PQ_PRO_EMBED;
      p.tok = E.tok;
      p.emb_pc = E.emb.pc;
      p.emb_ps = E.emb.ps;
      p.vocab = c.vocab;
      p.x_out = xa;
      p.w0 = D.op_norm;
      p.eps = c.eps;
    } else {
      resnorm(E.L[l - 1].post_ffn_norm, D.op_norm);
    }
    PQ_TRY(gemv(D.in, E.Wd, PQ_DTYPE_BF16, nullptr));
    p = pq_gemv_prologue{};
    if (D.attn && mixer_fused(E, D)) {
      if (dev)
        PQ_TRY(attn_layer_decode_dev(E.Wd, D.q_norm, D.k_norm, layer_rope(E, D), D.kc, D.vc, E.ctr + 1, c.ctx, c.nh,
                                     c.nkv, c.hd, layer_rot(E, D), layer_win(E, D), c.eps, scale, nullptr, E.qx, E.dx,
                                     E.st));
      else
        PQ_TRY(pq_attn_layer_decode(E.Wd, D.q_norm, D.k_norm, layer_rope(E, D), D.kc, D.vc, E.pos, c.nh, c.nkv, c.hd,
                                    layer_rot(E, D), layer_win(E, D), c.eps, scale, nullptr, E.qx, E.dx, E.st));
    } else if (D.attn) {
      // head_dim 128 or a sliding window: q/k prep and the split-K attention
      // (two launches), the position read on the device in the captured step
      const int32_t *pd = dev ? E.ctr + 1 : nullptr;
      PQ_TRY(qk_prep_launch(E.Wd, E.nin, D.q_norm, D.k_norm, layer_rope(E, D), D.kc, D.vc, E.pos, pd, c.nh, c.nkv,
                            c.hd, layer_rot(E, D), 1, c.eps, E.st));
      if (dev)
        PQ_TRY(attn_decode_dev(E.Wd, E.nin, D.kc, D.vc, E.Wd + E.qd + 2 * E.kvd, E.nin, nullptr, 0, E.qx, E.dx, pd,
                               c.ctx, c.nh, c.nkv, c.hd, scale, layer_win(E, D), E.attn_ws, E.attn_ws_bytes, E.st));
      else
        PQ_TRY(pq_attn_decode(E.Wd, E.nin, D.kc, D.vc, E.Wd + E.qd + 2 * E.kvd, E.nin, nullptr, 0, E.qx, E.dx, E.pos,
                              c.nh, c.nkv, c.hd, 1, scale, layer_win(E, D), E.attn_ws, E.attn_ws_bytes, E.st));
    }
    if (D.attn) {
      p.kind = PQ_PRO_Q8;
      p.qx = E.qx;
      p.dx = E.dx;
    } else {
      p.kind = PQ_PRO_CONV;
      p.bcx = E.Wd;
      p.ring_in = D.rings[D.rc];
      p.ring_out = D.rings[1 - D.rc];
      p.taps = D.taps;
      p.ntaps = c.ntaps;
      D.rc = 1 - D.rc;
    }
    PQ_TRY(gemv(D.out, E.Hb, PQ_DTYPE_BF16, nullptr));
    resnorm(D.post_op_norm, D.ffn_norm);
    PQ_TRY(pq_q8_gemv_fused_swiglu(D.ug.pc, D.ug.ps, &p, E.qx, E.dx, c.ffn, H, E.st));
    if (pow2_range(D.down.K)) {
      p = pq_gemv_prologue{};
      p.kind = PQ_PRO_Q8;
      p.qx = E.qx;
      p.dx = E.dx;
      PQ_TRY(gemv(D.down, E.Hb, PQ_DTYPE_BF16, nullptr));
    } else {   // FFN widths that are not powers of two (LFM3: 7680): the Q8_0 GEMV, the same bits
      PQ_TRY(pq_q8_gemv(D.down.pc, D.down.ps, E.qx, E.dx, E.Hb, PQ_DTYPE_BF16, D.down.N, D.down.K, E.st));
    }
  }
  resnorm(E.L[c.nlayers - 1].post_ffn_norm, E.final_norm);
  PQ_TRY(gemv(E.emb, E.logits, PQ_DTYPE_F32, E.parts));
  if (dev) PQ_TRY(argmax_parts_step(E.parts, E.nparts, E.tok, E.ids, E.ctr, E.st));
  else PQ_TRY(pq_argmax_parts(E.parts, E.nparts, E.tok, E.st));
  E.pos += 1;
  E.last_t = 1;
  E.last_resid = xa;
  (void)H;
  return PQ_OK;
}

// forward_r2's T=1 step through the fused reference-numerics kernels, the
// same bits: the embedding row, the norm + residual pairs and the conv run as
// the prologues of the GEMVs that read them, silu(gate) * up as the gate/up
// GEMV's epilogue, and the LM head writes per-workgroup argmax pairs: per
// attention layer the in GEMV, the attention mixer, o_proj, gate/up and down
// (five launches), per conv layer four (the conv is the out GEMV's
// prologue), plus the LM head and the argmax. A slot with a low-bit source
// tensor (a Q4 / Q5 blob) runs its parts' GEMVs on the op's bf16 output
// instead (pq_rmsnorm's residual form, pq_conv on a copy of the ring,
// pq_silu_mul: the same values), and a bf16 table takes the row copy and
// pq_bf16_gemv. The position and id slot as in forward_decode (dev: on the
// device, so the step can be captured and replayed).
// Whether a split slot's parts take a prologue (pq_qlow_gemv_fused for the
// low-bit parts, pq_q8r_gemv_fused for the Q8 ones): K of 2048, 4096 or 8192,
// K <= 4096 for CONV.
static bool parts_fusable(const Q8Dev &w, int kind) {
  return (w.K == 2048 || w.K == 4096 || w.K == 8192) && (kind != PQ_PRO_CONV || w.K <= 4096);
}

// A split slot's GEMVs at T = 1 with the prologue pro, each part writing its
// rows of y (bf16). Every launch runs the prologue; the vectors it writes once
// (x_out, ring_out) get the same values from each, from unchanged inputs.
// (A second part forked onto another stream inside the captured step, to run
// beside the first, cost about 22 us per fork and join: 0.728 -> 0.909 ms per
// token of the Q4 backbone, whose attention gate rows stay Q8.)
static int parts_fused(Engine &E, const Q8Dev &w, const pq_gemv_prologue &pro, uint16_t *y,
                       const Part *skip = nullptr) {
  for (const Part &p : w.parts) {
    if (&p == skip) continue;
    if (p.bits == 8)
      PQ_TRY(pq_q8r_gemv_fused(w.pc + (size_t)p.r0 * w.K, w.sf + (size_t)p.r0 * (w.K / 32), &pro, y + p.r0,
                               PQ_DTYPE_BF16, p.n, w.K, nullptr, E.st));
    else
      PQ_TRY(pq_qlow_gemv_fused(p.pc, p.ps, &pro, y + p.r0, PQ_DTYPE_BF16, p.n, w.K, p.bits, E.st));
  }
  return PQ_OK;
}

// A gate/up slot whose [gate | up] rows are one low-bit part (w1 | w3 of one
// width, tile after tile): pq_qlow_gemv_fused_swiglu writes silu(gate) * up
// directly (PQ_QLOW_SWIGLU=0: the GEMV, then down's SILU prologue).
static bool qlow_swiglu(const Q8Dev &w) {
  static const bool off = [] {
    const char *e = getenv("PQ_QLOW_SWIGLU");
    return e != nullptr && atoi(e) == 0;
  }();
  return !off && w.parts.size() == 1 && w.parts[0].bits != 8 && w.parts[0].n == w.N && (w.N / 2) % 32 == 0 &&
         parts_fusable(w, PQ_PRO_RESNORM);
}

// The decode token's q/k prep inside its attention launch
// (PQ_ATTN_PREP=0: pq_qk_prep_ref's kernel, then the attention).
static bool attn_prep_fused() {
  static const bool off = [] {
    const char *e = getenv("PQ_ATTN_PREP");
    return e != nullptr && atoi(e) == 0;
  }();
  return !off;
}

// An attention layer's in-slot whose last part is the gate rows in Q8 (rows
// qd + 2 kvd .., one per q head, K = 2048; a low-bit blob keeps gate_proj in
// Q8): the decode attention forms the gates itself from those rows and the
// residual (pq_attn_decode_ref's gate form), so the slot's launches leave
// them out (PQ_ATTN_GATE=0: the part's own GEMV, as the unfused step runs it).
static const Part *attn_gate_part(const Engine &E, const LayerDev &D) {
  static const bool off = [] {
    const char *e = getenv("PQ_ATTN_GATE");
    return e != nullptr && atoi(e) == 0;
  }();
  if (off || !D.attn || !D.in.split() || D.in.parts.size() < 2 || D.in.K != 2048 || !attn_prep_fused()) return nullptr;
  const Part &g = D.in.parts.back();
  return g.bits == 8 && g.r0 == E.qd + 2 * E.kvd && g.n == E.c.nh ? &g : nullptr;
}

static int forward_decode_r2(Engine &E, bool dev) {
  const pq_model_cfg &c = E.c;
  const int H = c.hidden;
  if (E.pos + 1 > c.ctx) return fail(PQ_ERR_STATE, "context full: %d + 1 > %d", E.pos, c.ctx);
  uint16_t *xa = E.Xd[0], *xb = E.Xd[1];
  pq_gemv_prologue p;
  auto resnorm = [&](const float *w0, const float *w1) {
    p = pq_gemv_prologue{};
    p.kind = PQ_PRO_RESNORM;
    p.h = E.Hb;
    p.x_in = xa;
    p.x_out = xb;
    p.w0 = w0;
    p.w1 = w1;
    p.eps = c.eps;
    std::swap(xa, xb);
  };
  // the unfused "rms1 -> eadd -> rms1" triple: xa += rmsnorm(Hb, w0) in place,
  // y = rmsnorm(xa, w1) as bf16
  auto resnorm_to = [&](const float *w0, const float *w1, uint16_t *y) {
    return pq_rmsnorm(xa, E.Hb, w0, w1, y, nullptr, nullptr, H, 1, c.eps, E.st);
  };
  auto gemv = [&](const Q8Dev &w, void *y, int dt, float *parts) {
    return pq_q8r_gemv_fused(w.pc, w.sf, &p, y, dt, w.N, w.K, parts, E.st);
  };
  auto plain = [&](const Q8Dev &w, const uint16_t *x, uint16_t *y) {
    return gemm_r2(E, w, x, y, PQ_DTYPE_BF16, 1);
  };
  const float scale = 1.0f / sqrtf((float)c.hd);
  for (int l = 0; l < c.nlayers; l++) {
    LayerDev &D = E.L[l];
    if (l == 0 && (E.emb_bf16 || D.in.split())) {   // the row into xa, then its norm
      PQ_TRY(embed_r2(E, E.tok, xa, 1));
      if (D.in.split() && !parts_fusable(D.in, PQ_PRO_NORM)) {
        PQ_TRY(pq_rmsnorm(xa, nullptr, D.op_norm, nullptr, E.A, nullptr, nullptr, H, 1, c.eps, E.st));
        PQ_TRY(plain(D.in, E.A, E.Wd));
      } else {
        p = pq_gemv_prologue{};
        p.kind = PQ_PRO_NORM;
        p.x_in = xa;
        p.w0 = D.op_norm;
        p.eps = c.eps;
        if (D.in.split()) PQ_TRY(parts_fused(E, D.in, p, E.Wd, attn_gate_part(E, D)));
        else PQ_TRY(gemv(D.in, E.Wd, PQ_DTYPE_BF16, nullptr));
      }
    } else if (l == 0) {   // the token's embedding row (written once to xa), normalized
      p = pq_gemv_prologue{};
      p.kind = PQ_PRO_EMBED;
      p.tok = E.tok;
      p.emb_pc = E.emb.pc;
      p.emb_sf = E.emb.sf;
      p.vocab = c.vocab;
      p.x_out = xa;
      p.w0 = D.op_norm;
      p.eps = c.eps;
      PQ_TRY(gemv(D.in, E.Wd, PQ_DTYPE_BF16, nullptr));
    } else if (D.in.split() && parts_fusable(D.in, PQ_PRO_RESNORM)) {
      resnorm(E.L[l - 1].post_ffn_norm, D.op_norm);
      PQ_TRY(parts_fused(E, D.in, p, E.Wd, attn_gate_part(E, D)));
    } else if (D.in.split()) {
      PQ_TRY(resnorm_to(E.L[l - 1].post_ffn_norm, D.op_norm, E.A));
      PQ_TRY(plain(D.in, E.A, E.Wd));
    } else {
      resnorm(E.L[l - 1].post_ffn_norm, D.op_norm);
      PQ_TRY(gemv(D.in, E.Wd, PQ_DTYPE_BF16, nullptr));
    }
    if (D.attn) {   // k_attn_head's order over the bf16 cache
      const int32_t *pd = dev ? E.ctr + 1 : nullptr;
      const uint16_t *gate = E.Wd + E.qd + 2 * E.kvd;
      // the gates' rows left out of the in-slot above (the fused prologue forms: layer 0's NORM, RESNORM)
      const bool fused_in = D.in.split() && (l == 0 ? parts_fusable(D.in, PQ_PRO_NORM) : parts_fusable(D.in, PQ_PRO_RESNORM));
      const Part *gp = fused_in ? attn_gate_part(E, D) : nullptr;
      if (gp != nullptr) {   // y = rmsnorm(xa, op_norm): xa is the layer input's residual (written by the in-slot)
        const AttnGateQ8 g{D.in.pc + (size_t)gp->r0 * D.in.K, D.in.sf + (size_t)gp->r0 * (D.in.K / 32), xa,
                           D.op_norm, c.eps, D.in.K};
        PQ_TRY(attn_decode_ref_dev(E.Wd, D.q_norm, D.k_norm, layer_rope(E, D), D.kc, D.vc, nullptr, E.A, E.pos, pd,
                                   c.ctx, c.nh, c.nkv, c.hd, layer_rot(E, D), c.eps, scale, layer_win(E, D), E.st,
                                   &g));
      } else if (attn_prep_fused()) {
        PQ_TRY(attn_decode_ref_dev(E.Wd, D.q_norm, D.k_norm, layer_rope(E, D), D.kc, D.vc, gate, E.A, E.pos, pd,
                                   c.ctx, c.nh, c.nkv, c.hd, layer_rot(E, D), c.eps, scale, layer_win(E, D), E.st));
      } else {
        PQ_TRY(qk_prep_launch(E.Wd, E.nin, D.q_norm, D.k_norm, layer_rope(E, D), D.kc, D.vc, E.pos, pd, c.nh,
                              c.nkv, c.hd, layer_rot(E, D), 1, c.eps, E.st, true));
        if (dev)
          PQ_TRY(attn_ref_dev(E.Wd, E.nin, D.kc, D.vc, gate, E.nin, E.A, E.qd, pd, c.ctx, c.nh, c.nkv, c.hd, scale,
                              layer_win(E, D), E.st));
        else
          PQ_TRY(pq_attn_ref(E.Wd, E.nin, D.kc, D.vc, gate, E.nin, E.A, E.qd, E.pos, c.nh, c.nkv, c.hd, 1, scale,
                             layer_win(E, D), E.st));
      }
      PQ_TRY(plain(D.out, E.A, E.Hb));
    } else if (D.out.split() && parts_fusable(D.out, PQ_PRO_CONV)) {
      p = pq_gemv_prologue{};
      p.kind = PQ_PRO_CONV;
      p.bcx = E.Wd;
      p.ring_in = D.rings[D.rc];
      p.ring_out = D.rings[1 - D.rc];
      p.taps = D.taps;
      p.ntaps = c.ntaps;
      D.rc = 1 - D.rc;
      PQ_TRY(parts_fused(E, D.out, p, E.Hb));
    } else if (D.out.split()) {
      // the ring ping-pong as the CONV prologue keeps it: the shifted ring goes
      // to the other buffer (a copy, then the conv updates it in place)
      const size_t rb = (size_t)c.ntaps * H * 2;
      if (hipMemcpyAsync(D.rings[1 - D.rc], D.rings[D.rc], rb, hipMemcpyDeviceToDevice, E.st) != hipSuccess)
        return fail(PQ_ERR_LAUNCH, "ring copy failed");
      D.rc = 1 - D.rc;
      PQ_TRY(pq_conv(D.rings[D.rc], D.taps, E.Wd, E.A, H, 1, c.ntaps, E.st));
      PQ_TRY(plain(D.out, E.A, E.Hb));
    } else {
      p = pq_gemv_prologue{};
      p.kind = PQ_PRO_CONV;
      p.bcx = E.Wd;
      p.ring_in = D.rings[D.rc];
      p.ring_out = D.rings[1 - D.rc];
      p.taps = D.taps;
      p.ntaps = c.ntaps;
      D.rc = 1 - D.rc;
      PQ_TRY(gemv(D.out, E.Hb, PQ_DTYPE_BF16, nullptr));
    }
    // a split gate/up slot: its parts with the RESNORM prologue write the
    // [gate | up] rows, and down takes silu(gate) * up as its SILU prologue
    const bool down_silu = D.down.split() ? parts_fusable(D.down, PQ_PRO_SILU) : pow2_range(D.down.K);
    if (qlow_swiglu(D.ug)) {
      resnorm(D.post_op_norm, D.ffn_norm);
      const Part &pu = D.ug.parts[0];
      PQ_TRY(pq_qlow_gemv_fused_swiglu(pu.pc, pu.ps, &p, E.A, c.ffn, H, pu.bits, E.st));
      PQ_TRY(plain(D.down, E.A, E.Hb));
      continue;
    }
    if (D.ug.split() && parts_fusable(D.ug, PQ_PRO_RESNORM) && down_silu) {
      resnorm(D.post_op_norm, D.ffn_norm);
      PQ_TRY(parts_fused(E, D.ug, p, E.Wd));                        // [gate | up] rows
      p = pq_gemv_prologue{};
      p.kind = PQ_PRO_SILU;
      p.gu = E.Wd;
      if (D.down.split()) PQ_TRY(parts_fused(E, D.down, p, E.Hb));
      else PQ_TRY(gemv(D.down, E.Hb, PQ_DTYPE_BF16, nullptr));
      continue;
    }
    if (D.ug.split()) {
      PQ_TRY(resnorm_to(D.post_op_norm, D.ffn_norm, E.A));
      PQ_TRY(plain(D.ug, E.A, E.Wd));                               // [gate | up] rows
      PQ_TRY(pq_silu_mul(E.Wd, E.A, nullptr, nullptr, c.ffn, 1, E.st));
    } else {
      resnorm(D.post_op_norm, D.ffn_norm);
      PQ_TRY(pq_q8r_gemv_fused_swiglu(D.ug.pc, D.ug.sf, &p, E.A, c.ffn, H, E.st));
    }
    PQ_TRY(plain(D.down, E.A, E.Hb));
  }
  const float *last_post = E.L[c.nlayers - 1].post_ffn_norm;
  int nparts = E.nparts;
  if (E.emb_bf16) {
    PQ_TRY(resnorm_to(last_post, E.final_norm, E.A));
    PQ_TRY(head_r2(E, E.A, E.parts));
    nparts = E.nparts16;
  } else {
    resnorm(last_post, E.final_norm);
    PQ_TRY(gemv(E.emb, E.logits, PQ_DTYPE_F32, E.parts));
  }
  if (dev) PQ_TRY(argmax_parts_step(E.parts, nparts, E.tok, E.ids, E.ctr, E.st));
  else PQ_TRY(pq_argmax_parts(E.parts, nparts, E.tok, E.st));
  E.pos += 1;
  E.last_t = 1;
  E.last_resid = xa;
  return PQ_OK;
}

// The prompt, uploaded once (the copy is waited for: the caller's host buffer
// may go away when the call returns), then run layer-major in chunks of tmax
// positions with no further host synchronization; the greedy id after the
// last position goes to *next.
static int prefill(Engine &E, const int32_t *prompt, int n, int32_t *next) {
  if (hipMemcpyAsync(E.tokd, prompt, (size_t)n * 4, hipMemcpyHostToDevice, E.st) != hipSuccess ||
      hipStreamSynchronize(E.st) != hipSuccess)
    return fail(PQ_ERR_LAUNCH, "token upload failed");
  return forward_any(E, E.tokd, n, next);
}

// n decode steps from the device-resident token *E.tok: step s feeds the id
// of step s-1 and writes its own into ids[s] and E.tok (no host round trip).
// The conv rings' parity: every conv layer flips its ping-pong pair each step.
static int ring_parity(const Engine &E) {
  for (const LayerDev &D : E.L)
    if (!D.attn) return D.rc;
  return 0;
}
static void set_ring_parity(Engine &E, int rc) {
  for (LayerDev &D : E.L)
    if (!D.attn) D.rc = rc;
}

// Capture the fused step (device position and id slot) for ring parity p. The
// capture only records: the host-side state it advances is put back.
static int capture_step(Engine &E, int p) {
  const int pos = E.pos, rc = ring_parity(E), last_t = E.last_t;
  const uint16_t *last_resid = E.last_resid;
  set_ring_parity(E, p);
  hipGraph_t g = nullptr;
  if (hipStreamBeginCapture(E.st, hipStreamCaptureModeThreadLocal) != hipSuccess)
    return fail(PQ_ERR_LAUNCH, "hipStreamBeginCapture failed");
  const int rc_step = forward_decode(E, true);
  const hipError_t ec = hipStreamEndCapture(E.st, &g);
  E.step_resid = E.last_resid;   // the residual buffer a step ends in
  E.pos = pos;
  E.last_t = last_t;
  E.last_resid = last_resid;
  set_ring_parity(E, rc);
  if (rc_step != PQ_OK) {
    if (g) hipGraphDestroy(g);
    return rc_step;
  }
  if (ec != hipSuccess || g == nullptr) return fail(PQ_ERR_LAUNCH, "hipStreamEndCapture failed");
  const hipError_t ei = hipGraphInstantiate(&E.gexec[p], g, nullptr, nullptr, 0);
  hipGraphDestroy(g);
  if (ei != hipSuccess) return fail(PQ_ERR_LAUNCH, "hipGraphInstantiate failed: %s", hipGetErrorString(ei));
  return PQ_OK;
}

// n decode steps from the device-resident token *E.tok: step s feeds the id
// of step s-1 and writes its own into ids[first_slot + s] and E.tok (no host
// round trip). Fused steps replay a captured graph per step.
static int decode(Engine &E, int n, int first_slot) {
  if (E.fused && E.graph) {
    if (E.pos + n > E.c.ctx) return fail(PQ_ERR_STATE, "context full: %d + %d > %d", E.pos, n, E.c.ctx);
    for (int p = 0; p < 2; p++)
      if (!E.gexec[p]) PQ_TRY(capture_step(E, p));
    E.hctr[0] = first_slot;
    E.hctr[1] = E.pos;
    if (hipMemcpyAsync(E.ctr, E.hctr, sizeof E.hctr, hipMemcpyHostToDevice, E.st) != hipSuccess)
      return fail(PQ_ERR_LAUNCH, "counter upload failed");
    const int rc0 = ring_parity(E);
    for (int s = 0; s < n; s++)
      if (hipGraphLaunch(E.gexec[(rc0 + s) & 1], E.st) != hipSuccess) return fail(PQ_ERR_LAUNCH, "hipGraphLaunch failed");
    // the host-side state the steps advanced
    E.pos += n;
    E.last_t = 1;
    E.last_resid = E.step_resid;
    set_ring_parity(E, (rc0 + n) & 1);
    return PQ_OK;
  }
  for (int s = 0; s < n; s++) {
    if (E.fused) PQ_TRY(forward_decode(E, false));
    else PQ_TRY(forward_any(E, E.tok, 1, E.tok));
    if (hipMemcpyAsync(E.ids + first_slot + s, E.tok, 4, hipMemcpyDeviceToDevice, E.st) != hipSuccess)
      return fail(PQ_ERR_LAUNCH, "id copy failed");
  }
  return PQ_OK;
}

}  // namespace pq

using namespace pq;

static void drop_graphs(Engine &E);
static void clear_blob_extras(Engine &E);
static void clear_parts(Engine &E, Q8Dev &q);

extern "C" void *pq_engine_create(const pq_model_cfg *cfg) {
  if (!cfg) { fail(PQ_ERR_ARG, "pq_engine_create: null config"); return nullptr; }
  const pq_model_cfg &c = *cfg;
  const bool ok = c.hidden >= 256 && (c.hidden & (c.hidden - 1)) == 0 && c.hidden <= 8192 && c.ffn % 256 == 0 &&
                  c.ffn > 0 && c.vocab > 0 && c.nlayers > 0 && c.nlayers <= 32 && (c.hd == 64 || c.hd == 128) &&
                  c.nkv > 0 &&
                  c.nh % c.nkv == 0 && c.nh * c.hd % 64 == 0 && c.rot >= 0 && c.rot <= c.hd && c.rot % 2 == 0 &&
                  (c.ntaps == 2 || c.ntaps == 3 || c.ntaps == 4 || c.ntaps == 7) && c.ctx > 0 &&
                  c.prefill_chunk > 0 && c.prefill_chunk <= 512 &&
                  (c.numerics == PQ_NUMERICS_Q8 || c.numerics == PQ_NUMERICS_REF);
  if (!ok) { fail(PQ_ERR_ARG, "pq_engine_create: unsupported configuration"); return nullptr; }
  if (c.slide_mask != 0 && ((c.slide_mask & ~c.attn_mask) != 0 || c.slide_win <= 0 || c.slide_rot < 0 ||
                            c.slide_rot > c.hd || c.slide_rot % 2 != 0 || !(c.slide_theta > 0.0f))) {
    fail(PQ_ERR_ARG, "pq_engine_create: sliding layers must be attention layers with a window, rot and theta");
    return nullptr;
  }
  auto E = std::make_unique<Engine>();
  if (create(*E, c) != PQ_OK) return nullptr;
  if (upload_rope(*E) != PQ_OK || reset(*E) != PQ_OK) return nullptr;
  const char *why;
  E->fused = fused_supported(c, &why);
  return E.release();
}

extern "C" int pq_engine_destroy(void *h) {
  delete static_cast<Engine *>(h);
  return PQ_OK;
}

extern "C" int pq_engine_load_synthetic(void *h) {
  PQ_REQUIRE(h, PQ_ERR_ARG, "null engine");
  Engine &E = *static_cast<Engine *>(h);
  drop_graphs(E);
  clear_blob_extras(E);
  PQ_TRY(load_synthetic(E));
  E.loaded = true;
  return PQ_OK;
}

extern "C" int pq_engine_set_q8(void *h, int layer, int slot, const int8_t *codes, const uint16_t *scales) {
  PQ_REQUIRE(h && codes && scales, PQ_ERR_ARG, "pq_engine_set_q8: null pointer");
  Engine &E = *static_cast<Engine *>(h);
  Q8Dev *q = q8_slot(E, layer, slot);
  PQ_REQUIRE(q, PQ_ERR_ARG, "pq_engine_set_q8: no Q8 tensor at layer %d slot %d", layer, slot);
  drop_graphs(E);
  clear_parts(E, *q);
  return upload_q8(E, *q, codes, scales, nullptr);
}

extern "C" int pq_engine_set_q8_f32(void *h, int layer, int slot, const int8_t *codes, const float *scales) {
  PQ_REQUIRE(h && codes && scales, PQ_ERR_ARG, "pq_engine_set_q8_f32: null pointer");
  Engine &E = *static_cast<Engine *>(h);
  Q8Dev *q = q8_slot(E, layer, slot);
  PQ_REQUIRE(q, PQ_ERR_ARG, "pq_engine_set_q8_f32: no Q8 tensor at layer %d slot %d", layer, slot);
  drop_graphs(E);
  clear_parts(E, *q);
  return upload_q8(E, *q, codes, nullptr, scales);
}

extern "C" int pq_engine_set_f32(void *h, int layer, int slot, const float *v, size_t n) {
  PQ_REQUIRE(h && v, PQ_ERR_ARG, "pq_engine_set_f32: null pointer");
  Engine &E = *static_cast<Engine *>(h);
  size_t want = 0;
  float *dst = vec_slot(E, layer, slot, &want);
  PQ_REQUIRE(dst && n == want, PQ_ERR_ARG, "pq_engine_set_f32: layer %d slot %d expects %zu values", layer, slot, want);
  return upload_f32(E, dst, v, n);
}

// ------------------------------------------------------------ .lfm3q8 load
namespace {
struct BlobSrc {
  std::string name;
  long long n0, n1;   // Q8: rows, columns; fp32: element count in n0
};
struct BlobTarget {
  int layer, slot;
  bool q8;
  std::vector<BlobSrc> src;
};
}  // namespace

// Discards the captured decode steps (they hold the weights' addresses); the
// next decode captures them again.
static void drop_graphs(Engine &E) {
  if (E.st) hipStreamSynchronize(E.st);
  for (hipGraphExec_t &g : E.gexec)
    if (g) {
      hipGraphExecDestroy(g);
      g = nullptr;
    }
}

// Frees what a blob load adds beyond the create-time arenas: low-bit parts,
// the bf16 table, their workspaces; the slots are plain Q8 again.
static void clear_parts(Engine &E, Q8Dev &q) {
  if (q.parts.empty()) return;
  if (E.st) hipStreamSynchronize(E.st);
  for (const Part &pt : q.parts) {
    E.dfree(pt.pc);
    E.dfree(pt.ps);
  }
  q.parts.clear();
}

static void clear_blob_extras(Engine &E) {
  if (E.st) hipStreamSynchronize(E.st);
  for (LayerDev &D : E.L)
    for (Q8Dev *q : {&D.in, &D.out, &D.ug, &D.down}) clear_parts(E, *q);
  E.dfree(E.emb16);
  E.emb16 = nullptr;
  E.emb_bf16 = false;
  E.dfree(E.qlow_ws);
  E.qlow_ws = nullptr;
  E.qlow_ws_bytes = 0;
  E.dfree(E.ptmp);
  E.ptmp = nullptr;
}

// The reference's tensor names (layer_body, lfm3_nanode.cu:3739-3856; the
// exporter's table) onto the engine's slots: q|k|v|gate_proj stack into the
// attention layer's input GEMV, w1 (gate) and w3 (up) into gate/up. The fp32
// weight scales stay fp32 under PQ_NUMERICS_REF; under PQ_NUMERICS_Q8 they
// must be fp16 values (a blob written from fp16 scales), else the load is
// refused with a count of the scales fp16 cannot hold. The blob's layer_types
// must match the engine's layer kinds.
static int load_blob(Engine &E, void *blob) {
  const pq_model_cfg &c = E.c;
  const long long H = c.hidden, F = c.ffn;
  // the header's layer_types (conv / full_attention / sliding_attention, as
  // the reference reads them, lfm3_nanode.cu:5404-5424) must be the engine's
  {
    const char *js = pq_blob_config(blob);
    const char *lt = strstr(js, "\"layer_types\":[");
    if (lt) {
      const char *q = lt + strlen("\"layer_types\":[");
      for (int l = 0; l < c.nlayers; l++) {
        const char *a = strchr(q, '"');
        const char *b = a ? strchr(a + 1, '"') : nullptr;
        PQ_REQUIRE(a && b, PQ_ERR_ARG, "pq_engine_load_blob: layer_types has fewer than %d entries", c.nlayers);
        const std::string ty(a + 1, b);
        const LayerDev &D = E.L[l];
        const char *want = !D.attn ? "conv" : D.slide ? "sliding_attention" : "full_attention";
        PQ_REQUIRE(ty == want, PQ_ERR_ARG, "pq_engine_load_blob: layer %d is %s in the blob, %s in the engine", l,
                   ty.c_str(), want);
        q = b + 1;
      }
    }
  }
  auto LN = [](int l, const char *suf) { return "lfm.model.layers." + std::to_string(l) + "." + suf; };
  std::vector<BlobTarget> T;
  T.push_back({-1, 0, true, {{"lfm.model.embed_tokens.weight", c.vocab, H}}});
  for (int l = 0; l < c.nlayers; l++) {
    if (E.L[l].attn) {
      T.push_back({l, 0, true, {{LN(l, "self_attn.q_proj.weight"), (long long)c.nh * c.hd, H},
                                {LN(l, "self_attn.k_proj.weight"), (long long)c.nkv * c.hd, H},
                                {LN(l, "self_attn.v_proj.weight"), (long long)c.nkv * c.hd, H},
                                {LN(l, "self_attn.gate_proj.weight"), (long long)c.nh, H}}});
      T.push_back({l, 1, true, {{LN(l, "self_attn.o_proj.weight"), H, (long long)c.nh * c.hd}}});
      T.push_back({l, 8, false, {{LN(l, "self_attn.q_norm.weight"), c.hd, 0}}});
      T.push_back({l, 9, false, {{LN(l, "self_attn.k_norm.weight"), c.hd, 0}}});
    } else {
      T.push_back({l, 0, true, {{LN(l, "conv.in_proj.weight"), 3 * H, H}}});
      T.push_back({l, 1, true, {{LN(l, "conv.out_proj.weight"), H, H}}});
      T.push_back({l, 10, false, {{LN(l, "conv.conv.weight"), H * c.ntaps, 0}}});
    }
    T.push_back({l, 2, true, {{LN(l, "feed_forward.w1.weight"), F, H}, {LN(l, "feed_forward.w3.weight"), F, H}}});
    T.push_back({l, 3, true, {{LN(l, "feed_forward.w2.weight"), H, F}}});
    T.push_back({l, 4, false, {{LN(l, "operator_norm.weight"), H, 0}}});
    T.push_back({l, 5, false, {{LN(l, "post_operator_norm.weight"), H, 0}}});
    T.push_back({l, 6, false, {{LN(l, "ffn_norm.weight"), H, 0}}});
    T.push_back({l, 7, false, {{LN(l, "post_ffn_norm.weight"), H, 0}}});
  }
  T.push_back({-1, 1, false, {{"lfm.model.embedding_norm.weight", H, 0}}});
  // every source present, with the dtype and shape its slot needs: a linear is
  // Q8 (dtype 1) or, under the reference numerics, Q4 / Q5 (6 / 7); the tied
  // table Q8 or, under the reference numerics, bf16 (3)
  std::vector<int> order, dtypes;
  for (const BlobTarget &t : T)
    for (const BlobSrc &s : t.src) {
      const int i = pq::blob_find(blob, s.name.c_str());
      PQ_REQUIRE(i >= 0, PQ_ERR_ARG, "pq_engine_load_blob: the blob has no %s", s.name.c_str());
      pq_blob_tensor ti;
      PQ_TRY(pq_blob_tensor_info(blob, i, &ti));
      long long elems = 1;
      for (int d = 0; d < ti.ndim; d++) elems *= ti.ne[d];
      if (t.q8) {
        const bool emb = t.layer == -1, low = ti.dtype == 6 || ti.dtype == 7;
        PQ_REQUIRE((ti.dtype == 1 || (low && !emb) || (ti.dtype == 3 && emb)) && ti.ndim == 2 && ti.ne[0] == s.n0 &&
                       ti.ne[1] == s.n1,
                   PQ_ERR_ARG,
                   "pq_engine_load_blob: %s is dtype %d [%lld x %lld], the engine needs [%lld x %lld] as Q8 (dtype 1)"
                   "%s",
                   s.name.c_str(), ti.dtype, ti.ne[0], ti.ndim > 1 ? ti.ne[1] : 0, s.n0, s.n1,
                   emb ? " or bf16 (dtype 3)" : " or Q4 / Q5 (dtype 6 / 7)");
        PQ_REQUIRE(ti.dtype == 1 || ref_numerics(E), PQ_ERR_ARG,
                   "pq_engine_load_blob: %s is %s, which is not supported under the Q8_0 numerics (its GEMV takes "
                   "bf16 activations): load it into an engine created with PQ_NUMERICS_REF",
                   s.name.c_str(), low ? "a Q4 / Q5 tensor (dtype 6 / 7)" : "the bf16 table (dtype 3)");
      } else {
        PQ_REQUIRE(ti.dtype == 2 && elems == s.n0, PQ_ERR_ARG,
                   "pq_engine_load_blob: %s is dtype %d with %lld values, the engine needs %lld fp32", s.name.c_str(),
                   ti.dtype, elems, s.n0);
      }
      order.push_back(i);
      dtypes.push_back(ti.dtype);
    }
  // a new load replaces what an earlier one set up (the captured steps hold
  // the old parts' addresses)
  drop_graphs(E);
  clear_blob_extras(E);
  // read ahead on a thread of its own while the tensors before convert and upload
  pq::BlobReader rd(blob, order, 2);
  std::vector<char> buf;
  std::vector<int8_t> codes;
  std::vector<float> sc32;
  size_t si = 0;   // index of the next source in order / dtypes
  for (const BlobTarget &t : T) {
    if (!t.q8) {
      si++;
      PQ_TRY(rd.take(buf));
      size_t n = 0;
      float *dst = vec_slot(E, t.layer, t.slot, &n);
      PQ_REQUIRE(dst && n == (size_t)t.src[0].n0, PQ_ERR_ARG, "pq_engine_load_blob: slot %d of layer %d", t.slot,
                 t.layer);
      PQ_TRY(upload_f32(E, dst, reinterpret_cast<const float *>(buf.data()), n));
      continue;
    }
    Q8Dev *q = q8_slot(E, t.layer, t.slot);
    long long rows = 0;
    for (const BlobSrc &s : t.src) rows += s.n0;
    PQ_REQUIRE(q && q->N == rows && q->K == t.src[0].n1, PQ_ERR_ARG,
               "pq_engine_load_blob: slot %d of layer %d holds [%d x %d]", t.slot, t.layer, q ? q->N : 0,
               q ? q->K : 0);
    if (t.layer == -1 && dtypes[si] == 3) {   // the bf16 table, as stored
      si++;
      PQ_TRY(rd.take(buf));
      if (!E.emb16) PQ_TRY(E.dalloc(&E.emb16, (size_t)c.vocab * H));
      if (hipMemcpyAsync(E.emb16, buf.data(), buf.size(), hipMemcpyHostToDevice, E.st) != hipSuccess ||
          hipStreamSynchronize(E.st) != hipSuccess)
        return fail(PQ_ERR_LAUNCH, "bf16 table upload failed");
      E.emb_bf16 = true;
      continue;
    }
    // Q8 sources into the slot's row-major arrays (rows of low-bit sources stay
    // zero there, unused), low-bit sources onto the device as the exporter laid
    // them out. Adjacent low-bit sources of one width share a part (their
    // 32-row tiles are stored tile after tile, so one payload holds both):
    // q|k|v_proj or w1|w3 run as one GEMV.
    codes.assign((size_t)rows * q->K, 0);
    sc32.assign((size_t)rows * (q->K / 32), 0.0f);
    std::vector<Part> parts;
    std::vector<int> part_of;   // the part of each source
    {
      size_t rr = 0;
      for (size_t k = 0; k < t.src.size(); k++) {
        const int dt = dtypes[si + k], bits = dt == 1 ? 8 : dt == 6 ? 4 : 5;
        if (bits != 8 && !parts.empty() && parts.back().bits == bits) {
          parts.back().n += (int)t.src[k].n0;
        } else {
          Part pt;
          pt.r0 = (int)rr;
          pt.n = (int)t.src[k].n0;
          pt.bits = bits;
          parts.push_back(pt);
        }
        part_of.push_back((int)parts.size() - 1);
        rr += (size_t)t.src[k].n0;
      }
    }
    bool low = false;
    for (Part &pt : parts)
      if (pt.bits != 8) {
        PQ_TRY(E.dalloc(&pt.pc, pq_qlow_packed_codes_bytes(pt.n, q->K, pt.bits)));
        PQ_TRY(E.dalloc(&pt.ps, pq_qlow_packed_scales_bytes(pt.n, q->K, pt.bits) / 2));
        E.qlow_ws_bytes = std::max(E.qlow_ws_bytes, pq_qlow_workspace_bytes(pt.n, q->K, pt.bits));
        low = true;
      }
    size_t r0 = 0;
    for (size_t k = 0; k < t.src.size(); k++) {
      const BlobSrc &s = t.src[k];
      const int dt = dtypes[si++];
      PQ_TRY(rd.take(buf));
      const size_t nc = (size_t)s.n0 * s.n1, ns = nc / 32;
      if (dt == 1) {
        memcpy(codes.data() + r0 * q->K, buf.data(), nc);
        memcpy(sc32.data() + r0 * (q->K / 32), buf.data() + nc, ns * 4);
      } else {
        const Part &pt = parts[(size_t)part_of[k]];
        const size_t pcb = pq_qlow_packed_codes_bytes((int)s.n0, (int)s.n1, pt.bits);
        const size_t psb = pq_qlow_packed_scales_bytes((int)s.n0, (int)s.n1, pt.bits);
        PQ_REQUIRE(pcb + psb == buf.size(), PQ_ERR_ARG, "pq_engine_load_blob: %s: %zu payload bytes, want %zu",
                   s.name.c_str(), buf.size(), pcb + psb);
        // the source's tiles follow those of the part's earlier sources
        const size_t t0 = (r0 - (size_t)pt.r0) / 32;
        const size_t ct = pq_qlow_packed_codes_bytes(32, q->K, pt.bits), st = pq_qlow_packed_scales_bytes(32, q->K, pt.bits);
        if (hipMemcpyAsync(pt.pc + t0 * ct, buf.data(), pcb, hipMemcpyHostToDevice, E.st) != hipSuccess ||
            hipMemcpyAsync(reinterpret_cast<char *>(pt.ps) + t0 * st, buf.data() + pcb, psb, hipMemcpyHostToDevice,
                           E.st) != hipSuccess ||
            hipStreamSynchronize(E.st) != hipSuccess)
          return fail(PQ_ERR_LAUNCH, "low-bit upload failed");
      }
      r0 += (size_t)s.n0;
    }
    if (low) q->parts = std::move(parts);
    const int rc = upload_q8(E, *q, codes.data(), nullptr, sc32.data());
    if (rc != PQ_OK) {
      if (rc == PQ_ERR_DATA) {   // name the tensor in the message
        const std::string why = pq_last_error();
        return fail(PQ_ERR_DATA, "pq_engine_load_blob: %s: %s", t.src[0].name.c_str(), why.c_str());
      }
      return rc;
    }
  }
  // the low-bit GEMV workspace and the staging of a part's rows at T > 1
  bool split = false;
  for (const LayerDev &D : E.L) split = split || D.in.split() || D.out.split() || D.ug.split() || D.down.split();
  if (split) {
    PQ_TRY(E.dalloc(reinterpret_cast<char **>(&E.qlow_ws), std::max<size_t>(E.qlow_ws_bytes, 16)));
    const size_t wide = (size_t)std::max(std::max(3 * H, 2 * F), (long long)E.nin);
    PQ_TRY(E.dalloc(&E.ptmp, (size_t)E.tmax * wide * 4));
  }
  return PQ_OK;
}

extern "C" int pq_engine_load_blob(void *h, const char *path) {
  PQ_REQUIRE(h && path, PQ_ERR_ARG, "pq_engine_load_blob: null argument");
  Engine &E = *static_cast<Engine *>(h);
  void *blob = pq_blob_open(path);
  if (!blob) return PQ_ERR_ARG;
  E.loaded = false;
  const int rc = load_blob(E, blob);
  pq_blob_close(blob);
  if (rc != PQ_OK) return rc;
  E.loaded = true;
  return PQ_OK;
}

extern "C" int pq_engine_mark_loaded(void *h) {
  PQ_REQUIRE(h, PQ_ERR_ARG, "null engine");
  static_cast<Engine *>(h)->loaded = true;
  return PQ_OK;
}

extern "C" int pq_engine_reset(void *h) {
  PQ_REQUIRE(h, PQ_ERR_ARG, "null engine");
  return reset(*static_cast<Engine *>(h));
}

extern "C" int pq_engine_feed(void *h, const int32_t *tokens, int n, int32_t *next_id, float *logits) {
  PQ_REQUIRE(h && tokens && n > 0, PQ_ERR_ARG, "pq_engine_feed: bad arguments");
  Engine &E = *static_cast<Engine *>(h);
  PQ_REQUIRE(E.loaded, PQ_ERR_STATE, "pq_engine_feed: weights not loaded");
  // refused before the first chunk, so a prompt too long for the context
  // leaves the KV cache, the conv rings and the position as they were
  PQ_REQUIRE(n <= E.c.ctx - E.pos, PQ_ERR_STATE, "pq_engine_feed: %d tokens at position %d exceed the context %d", n,
             E.pos, E.c.ctx);
  PQ_TRY(prefill(E, tokens, n, E.tok));
  // the copies go on the engine's stream (a non-blocking stream: a null-stream
  // copy would not wait for the forward pass) and are waited for
  if (next_id && hipMemcpyAsync(next_id, E.tok, 4, hipMemcpyDeviceToHost, E.st) != hipSuccess)
    return fail(PQ_ERR_LAUNCH, "id copy failed");
  if (logits && hipMemcpyAsync(logits, E.logits, (size_t)E.c.vocab * 4, hipMemcpyDeviceToHost, E.st) != hipSuccess)
    return fail(PQ_ERR_LAUNCH, "logits copy failed");
  if ((next_id || logits) && hipStreamSynchronize(E.st) != hipSuccess) return fail(PQ_ERR_LAUNCH, "stream sync failed");
  return PQ_OK;
}

extern "C" int pq_engine_greedy(void *h, const int32_t *prompt, int n_prompt, int n_steps, int32_t *ids) {
  PQ_REQUIRE(h && prompt && ids && n_prompt > 0 && n_steps > 0, PQ_ERR_ARG, "pq_engine_greedy: bad arguments");
  Engine &E = *static_cast<Engine *>(h);
  PQ_REQUIRE(E.loaded, PQ_ERR_STATE, "pq_engine_greedy: weights not loaded");
  PQ_REQUIRE(n_steps <= E.max_ids && n_prompt + n_steps - 1 <= E.c.ctx, PQ_ERR_STATE,
             "pq_engine_greedy: %d + %d positions exceed the context %d", n_prompt, n_steps, E.c.ctx);
  PQ_TRY(reset(E));
  PQ_TRY(prefill(E, prompt, n_prompt, E.tok));
  if (hipMemcpyAsync(E.ids, E.tok, 4, hipMemcpyDeviceToDevice, E.st) != hipSuccess)
    return fail(PQ_ERR_LAUNCH, "id copy failed");
  PQ_TRY(decode(E, n_steps - 1, 1));
  if (hipMemcpyAsync(ids, E.ids, (size_t)n_steps * 4, hipMemcpyDeviceToHost, E.st) != hipSuccess ||
      hipStreamSynchronize(E.st) != hipSuccess)
    return fail(PQ_ERR_LAUNCH, "ids copy failed");
  return PQ_OK;
}

extern "C" int pq_engine_decode(void *h, int n_steps, int32_t *ids) {
  PQ_REQUIRE(h && n_steps > 0, PQ_ERR_ARG, "pq_engine_decode: bad arguments");
  Engine &E = *static_cast<Engine *>(h);
  PQ_REQUIRE(E.loaded, PQ_ERR_STATE, "pq_engine_decode: weights not loaded");
  PQ_REQUIRE(n_steps <= E.max_ids && E.pos + n_steps <= E.c.ctx, PQ_ERR_STATE, "pq_engine_decode: context full");
  PQ_TRY(decode(E, n_steps, 0));
  if (ids && (hipMemcpyAsync(ids, E.ids, (size_t)n_steps * 4, hipMemcpyDeviceToHost, E.st) != hipSuccess ||
              hipStreamSynchronize(E.st) != hipSuccess))
    return fail(PQ_ERR_LAUNCH, "ids copy failed");
  return PQ_OK;
}

extern "C" int pq_engine_set_fused(void *h, int on) {
  PQ_REQUIRE(h, PQ_ERR_ARG, "null engine");
  Engine &E = *static_cast<Engine *>(h);
  const char *why;
  if (on && !fused_supported(E.c, &why)) return fail(PQ_ERR_ARG, "pq_engine_set_fused: %s", why);
  E.fused = on != 0;
  return PQ_OK;
}

extern "C" int pq_engine_set_chunk(void *h, int n) {
  PQ_REQUIRE(h, PQ_ERR_ARG, "null engine");
  Engine &E = *static_cast<Engine *>(h);
  PQ_REQUIRE(n >= 1 && n <= E.c.prefill_chunk, PQ_ERR_ARG,
             "pq_engine_set_chunk: %d positions (1..%d, the prefill_chunk the engine was created with)", n,
             E.c.prefill_chunk);
  E.tmax = n;
  return PQ_OK;
}

extern "C" int pq_engine_set_graph(void *h, int on) {
  PQ_REQUIRE(h, PQ_ERR_ARG, "null engine");
  static_cast<Engine *>(h)->graph = on != 0;
  return PQ_OK;
}

extern "C" int pq_engine_sync(void *h) {
  PQ_REQUIRE(h, PQ_ERR_ARG, "null engine");
  return hipStreamSynchronize(static_cast<Engine *>(h)->st) == hipSuccess ? PQ_OK
                                                                          : fail(PQ_ERR_LAUNCH, "stream sync failed");
}

extern "C" void *pq_engine_stream(void *h) { return h ? static_cast<Engine *>(h)->st : nullptr; }

extern "C" int pq_engine_position(void *h) { return h ? static_cast<Engine *>(h)->pos : -1; }

extern "C" int pq_engine_hidden(void *h, uint16_t *out) {
  PQ_REQUIRE(h && out, PQ_ERR_ARG, "pq_engine_hidden: null pointer");
  Engine &E = *static_cast<Engine *>(h);
  // The residual stream of the last position fed.
  if (!E.last_resid) return fail(PQ_ERR_STATE, "pq_engine_hidden: nothing fed yet");
  return hipMemcpyAsync(out, E.last_resid, (size_t)E.c.hidden * 2, hipMemcpyDeviceToHost, E.st) == hipSuccess &&
                 hipStreamSynchronize(E.st) == hipSuccess
             ? PQ_OK
             : fail(PQ_ERR_LAUNCH, "hidden copy failed");
}

extern "C" size_t pq_engine_weight_bytes(void *h) {
  if (!h) return 0;
  Engine &E = *static_cast<Engine *>(h);
  size_t b = 0;
  const size_t sb = ref_numerics(E) ? 4 : 2;   // fp32 or fp16 scale per 32
  // the bytes a decode step reads: each part's own (a low-bit part its packed
  // payload), the bf16 table at 2 bytes per weight
  auto rows = [&](int n, int K, int bits) {
    if (bits == 8) return (size_t)n * K + (size_t)n * (K / 32) * sb;
    return pq_qlow_packed_codes_bytes(n, K, bits) + pq_qlow_packed_scales_bytes(n, K, bits);
  };
  auto q8 = [&](const Q8Dev &q) {
    if (!q.split()) b += rows(q.N, q.K, 8);
    for (const Part &pt : q.parts) b += rows(pt.n, q.K, pt.bits);
  };
  for (const LayerDev &D : E.L) {
    q8(D.in); q8(D.out); q8(D.ug); q8(D.down);
  }
  if (E.emb_bf16) b += (size_t)E.c.vocab * E.c.hidden * 2;
  else q8(E.emb);
  return b;
}
