// layer_ops.hip -- the non-GEMV steps of one LFM3-style decoder layer on gfx950:
// RMSNorm (optionally fused with the residual add and with the Q8_0
// quantization of its output), per-head q/k norm + RoPE + fp16 KV write, the
// gated short conv, silu(gate)*up, argmax and the embedding row lookup.
//
// Every op keeps the reference's rounding points (one bf16 round per op,
// RMSNorm rounding before the weight multiply) and its orders where they are
// fixed ones: sums of squares as rmsnorm_body / k_headnorm add them, argmax
// ties as k_argmax breaks them; e^x is pq::expf_pq, 1/sqrt the correctly
// rounded 1.0f / sqrtf (the reference's rsqrtf is the one step not restated).
#include "pq_device.h"
#include "pq_host.h"
#include "pq_internal.h"

namespace pq {

// ------------------------------------------------------------------ helpers
// Q8_0 quantization of a thread's E consecutive bf16 outputs (E <= 32, 32/E
// threads per block): amax over the block's threads (xor butterfly of max),
// d = amax/127, q = rne(v/d) clamped -- the same rule as q8_quant_kernel.
template <int E>
__device__ __forceinline__ void quant_store(const float *v, int8_t *qx, float *dx, int e0) {
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < E; i++) a = fmaxf(a, fabsf(v[i]));
#pragma unroll
  for (int o = 1; o < 32 / E; o <<= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
  const float d = a / 127.0f;
  int8_t q[E];
  const float dd = d != 0.0f ? d : 1.0f;   // d = 0: the block is all zero (q = 0), no branch
#pragma unroll
  for (int i = 0; i < E; i++) {
    int t = (int)__builtin_rintf(v[i] / dd);
    t = t > 127 ? 127 : (t < -127 ? -127 : t);
    q[i] = (int8_t)t;
  }
#pragma unroll
  for (int i = 0; i < E; i++) qx[e0 + i] = q[i];
  if ((e0 & 31) == 0) dx[e0 >> 5] = d;
}

// ---------------------------------------------------------------- RMSNorm
// One workgroup per row of H = 8 * blockDim elements, thread t holding 8
// consecutive ones as rmsnorm_body's threads do (H = 2048: its 256 threads).
// Optional residual form: h3 = rmsnorm(h, w0); x = bf16(x + h3) (written
// back); out = rmsnorm(x, w1). The output goes to y (bf16) and/or (qx, dx).
template <bool RESID>
__global__ __launch_bounds__(1024) void rmsnorm_kernel(uint16_t *__restrict__ x, const uint16_t *__restrict__ h,
                                                        const float *__restrict__ w0, const float *__restrict__ w1,
                                                        uint16_t *__restrict__ y, int8_t *__restrict__ qx,
                                                        float *__restrict__ dx, int H, float eps) {
  constexpr int E = 8;
  __shared__ __align__(16) float part[64];   // the warp partials of the two sums (H / 256 <= 32 each)
  const int nparts = H / 256;
  const size_t row = blockIdx.x;
  const int e0 = threadIdx.x * E;
  float v[E];
  const float inv_n = 1.0f / (float)H;  // exact: H is a power of two
  if (RESID) {
    float hv[E];
#pragma unroll
    for (int i = 0; i < E; i++) hv[i] = bf2f(h[row * H + e0 + i]);
    const float ss = ref_sumsq<E, false>(hv, part, nparts);
    const float rs = 1.0f / sqrtf(ss * inv_n + eps);
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float h3 = bf2f(f2bf(w0[e0 + i] * bf2f(f2bf(hv[i] * rs))));
      const uint16_t xn = f2bf(bf2f(x[row * H + e0 + i]) + h3);
      v[i] = bf2f(xn);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < E; i++) x[row * H + e0 + i] = f2bf(v[i]);
  } else {
#pragma unroll
    for (int i = 0; i < E; i++) v[i] = bf2f(x[row * H + e0 + i]);
  }
  const float *w = RESID ? w1 : w0;
  const float ss = ref_sumsq<E, false>(v, part + 32, nparts);
  const float rs = 1.0f / sqrtf(ss * inv_n + eps);
  float o[E];
#pragma unroll
  for (int i = 0; i < E; i++) o[i] = bf2f(f2bf(w[e0 + i] * bf2f(f2bf(v[i] * rs))));
  if (y != nullptr) {
#pragma unroll
    for (int i = 0; i < E; i++) y[row * H + e0 + i] = f2bf(o[i]);
  }
  if (qx != nullptr) quant_store<E>(o, qx + row * H, dx + row * (H / 32), e0);
}

// ------------------------------------------------- q/k norm, RoPE, KV write
// One wave per (head, position); lane l holds dimensions l + 64e, e < HD/64
// (HD = 64 or 128). Heads [0, nh) are q (norm + rope, in place), [nh, nh+nkv)
// k (norm + rope, then written to the fp16 cache), [nh+nkv, nh+2nkv) v
// (written to the cache). The sum of squares is k_headnorm's (head_sumsq).
// RoPE pairs (i, i + HD/2) for i < rot/2 (k_rope,
// lfm3_nanode.cu:483-498): a lane-pair exchange at HD = 64, the lane's own two
// values at HD = 128. cs is the layer's [pos][rot/2][cos, sin] table. KVB: the
// cache holds the bf16 values as the reference's k_kv_write copies them
// (157-162); else fp16 of them.
template <int HD, bool KVB>
__global__ __launch_bounds__(64) void qk_prep_kernel(uint16_t *__restrict__ qkv, int row_stride,
                                                      const float *__restrict__ qn, const float *__restrict__ kn,
                                                      const float *__restrict__ cs, uint16_t *__restrict__ kc,
                                                      uint16_t *__restrict__ vc, int pos0, int nh, int nkv, int rot,
                                                      float eps, const int32_t *__restrict__ pos_dev) {
  constexpr int E = HD / 64;
  const int head = blockIdx.x, t = blockIdx.y, l = threadIdx.x;
  const int pos = (pos_dev != nullptr ? *pos_dev : pos0) + t;
  uint16_t *row = qkv + (size_t)t * row_stride;
  const int kvd = nkv * HD;
  if (head >= nh + nkv) {  // v: straight to the cache
    const int g = head - nh - nkv;
#pragma unroll
    for (int e = 0; e < E; e++) {
      const uint16_t vb = row[nh * HD + kvd + g * HD + l + 64 * e];
      vc[(size_t)pos * kvd + g * HD + l + 64 * e] = KVB ? vb : f2h(bf2f(vb));
    }
    return;
  }
  const bool isq = head < nh;
  uint16_t *xr = isq ? row + head * HD : row + nh * HD + (head - nh) * HD;
  const float *w = isq ? qn : kn;
  float x[E], v[E];
#pragma unroll
  for (int e = 0; e < E; e++) x[e] = bf2f(xr[l + 64 * e]);
  const float rs = 1.0f / sqrtf(head_sumsq<HD>(x) * (1.0f / (float)HD) + eps);
#pragma unroll
  for (int e = 0; e < E; e++) v[e] = bf2f(f2bf(w[l + 64 * e] * bf2f(f2bf(x[e] * rs))));
  const int half = rot / 2;
  float r[E];
  if constexpr (HD == 64) {
    const float up = __shfl_down(v[0], 32, 64);     // partner for d < 32
    const float dn = __shfl_up(v[0], 32, 64);       // partner for d >= 32
    const int i = l & 31;
    r[0] = v[0];
    if (i < half) {
      const float c = cs[((size_t)pos * half + i) * 2], sn = cs[((size_t)pos * half + i) * 2 + 1];
      r[0] = l < 32 ? v[0] * c - up * sn : v[0] * c + dn * sn;
    }
  } else {   // HD = 128: the pair (l, l + 64) is the lane's own
    r[0] = v[0];
    r[1] = v[1];
    if (l < half) {
      const float c = cs[((size_t)pos * half + l) * 2], sn = cs[((size_t)pos * half + l) * 2 + 1];
      r[0] = v[0] * c - v[1] * sn;
      r[1] = v[1] * c + v[0] * sn;
    }
  }
#pragma unroll
  for (int e = 0; e < E; e++) {
    const uint16_t vb = f2bf(r[e]);
    if (isq) xr[l + 64 * e] = vb;
    else kc[(size_t)pos * kvd + (head - nh) * HD + l + 64 * e] = KVB ? vb : f2h(bf2f(vb));
  }
}

// ------------------------------------------------------------ short conv
// k_conv_chunk (lfm3_nanode.cu:917-941): per channel, bx = bf16(B*x); the
// window of the last NT bx values (the ring holds the NT before the chunk,
// newest last); acc = sum_k fl(tap_k * bx_{t-NT+1+k}) ascending from 0;
// cy = bf16(acc); out = bf16(C*cy). The positions are independent once bx is
// known, so a workgroup owns 64 channels x kConvTP positions [t0, t0 + TP):
// its threads first form the bx values the tile's windows need (positions
// t0 - NT + 1 .. t0 + TP - 1, each once, from the ring before the chunk) into
// LDS, then each output from LDS. The new ring (the last NT bx values) is
// written by the tile at t0 = 0, after a workgroup barrier: it is the only
// tile that reads the old ring, so the in-place update cannot race.
constexpr int kConvTP = 32;   // positions per workgroup

template <int NT>
__global__ __launch_bounds__(512) void conv_kernel(uint16_t *__restrict__ ring, const float *__restrict__ taps,
                                                    const uint16_t *__restrict__ bcx, uint16_t *__restrict__ out,
                                                    int H, int T) {
  constexpr int NW = kConvTP + NT - 1;   // window positions of the tile
  __shared__ uint16_t sbx[NW][64];
  const int lc = threadIdx.x & 63, c = blockIdx.x * 64 + lc;
  const int w = threadIdx.x >> 6, W = blockDim.x >> 6;
  const int t0 = blockIdx.y * kConvTP;
  const bool live = c < H;
  auto bx = [&](int tau) -> uint16_t {   // tau < 0: the ring (tau = -1 is its newest entry)
    if (tau < 0) return ring[(size_t)(NT + tau) * H + c];
    const uint16_t *row = bcx + (size_t)tau * 3 * H;
    return f2bf(bf2f(row[c]) * bf2f(row[2 * H + c]));
  };
  const int tend = T - t0 < kConvTP ? T - t0 : kConvTP;   // positions of this tile
  if (live)
    for (int i = w; i < tend + NT - 1; i += W) sbx[i][lc] = bx(t0 - (NT - 1) + i);
  float tp[NT];
#pragma unroll
  for (int k = 0; k < NT; k++) tp[k] = live ? taps[(size_t)c * NT + k] : 0.0f;
  uint16_t nr[NT];
  if (blockIdx.y == 0 && live && w == 0) {   // the new ring, from the old one where T < NT
#pragma unroll
    for (int k = 0; k < NT; k++) nr[k] = bx(T - NT + k);
  }
  __syncthreads();   // the window is in LDS; every read of the old ring is done
  if (live) {
    for (int i = w; i < tend; i += W) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < NT; k++) acc = acc + tp[k] * bf2f(sbx[i + k][lc]);
      const uint16_t cy = f2bf(acc);
      const int t = t0 + i;
      out[(size_t)t * H + c] = f2bf(bf2f(bcx[(size_t)t * 3 * H + H + c]) * bf2f(cy));
    }
  }
  if (blockIdx.y == 0 && live && w == 0) {
#pragma unroll
    for (int k = 0; k < NT; k++) ring[(size_t)k * H + c] = nr[k];
  }
}

// ------------------------------------------------------- silu(gate) * up
// Rows of the fused gate/up GEMV output: gate = row[0:F], up = row[F:2F].
// One workgroup of F/E threads per position; E consecutive elements per
// thread so the Q8_0 output can be formed in the same pass.
// IL: the row holds the gate/up pair interleaved in groups of 32 (the output
// of weights packed by pq_q8_pack_gate_up): gate element i at 64*(i/32) + i%32,
// up element i 32 further.
template <int E, bool IL>
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t *__restrict__ gu, uint16_t *__restrict__ y,
                                                        int8_t *__restrict__ qx, float *__restrict__ dx, int F) {
  const size_t t = blockIdx.y;
  const int e0 = (blockIdx.x * blockDim.x + threadIdx.x) * E;
  const uint16_t *g = gu + t * 2 * F + (IL ? 32 * (e0 / 32) : 0);
  const uint16_t *u = IL ? g + 32 : g + F;
  float o[E];
#pragma unroll
  for (int i = 0; i < E; i++) {
    const float a = bf2f(g[e0 + i]);
    const float sg = 1.0f / (1.0f + expf_pq(-a));
    o[i] = bf2f(f2bf((a * sg) * bf2f(u[e0 + i])));
  }
  if (y != nullptr) {
#pragma unroll
    for (int i = 0; i < E; i++) y[t * F + e0 + i] = f2bf(o[i]);
  }
  if (qx != nullptr) quant_store<E>(o, qx + t * F, dx + t * (F / 32), e0);
}

// ------------------------------------------------------------------ argmax
// The pick of k_argmax (am_better: the largest value above kAmFloor, ties in
// its thread-slot order; -1 when there is none), by any tree: a scan per
// thread, then the wave butterfly and the waves in order.
__global__ __launch_bounds__(1024) void argmax_kernel(const float *__restrict__ v, int n, int32_t *__restrict__ out) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  float best = kAmFloor;
  int idx = -1;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    float cv;
    int ci;
    am_leaf(v[i], i, cv, ci);
    if (am_better(cv, ci, best, idx)) { best = cv; idx = ci; }
  }
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const float ob = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (am_better(ob, oi, best, idx)) { best = ob; idx = oi; }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { bv[wave] = best; bi[wave] = idx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < (int)(blockDim.x >> 6); w++)
      if (am_better(bv[w], bi[w], best, idx)) { best = bv[w]; idx = bi[w]; }
    *out = idx;
  }
}

// --------------------------------------------------------------- embedding
// Row tok of the tied Q8_0 table, read from the packed layout:
// bf16(fl(code * scale)) (k_dequant_row, lfm3_nanode.cu:138-142). Tokens
// outside [0, vocab) give a zero row.
__global__ __launch_bounds__(256) void embed_kernel(const int8_t *__restrict__ pc, const uint16_t *__restrict__ ps,
                                                     const int32_t *__restrict__ tok, uint16_t *__restrict__ out,
                                                     int H, int vocab) {
  const int t = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= H) return;
  const int id = tok[t];
  if (id < 0 || id >= vocab) {
    out[(size_t)t * H + k] = 0;
    return;
  }
  const int nb = H / 32, nch = (nb + 7) / 8;
  const int tile = id / 64, r = id % 64, b = k / 32, h = (k % 32) / 16, j = k % 16;
  const int8_t c = pc[(((size_t)tile * nb + b) * 2 + h) * 1024 + r * 16 + j];
  const uint16_t s = ps[(((size_t)tile * nch + b / 8) * 64 + r) * 8 + (b % 8)];
  out[(size_t)t * H + k] = f2bf((float)c * h2f(s));
}

// The same lookup on the table as the .lfm3q8 file stores it (row-major
// codes [vocab][H], one fp32 scale per 32): the reference-numerics engine's
// table, k_dequant_row exactly as the reference calls it.
__global__ __launch_bounds__(256) void embed_rows_kernel(const int8_t *__restrict__ codes,
                                                          const float *__restrict__ scales,
                                                          const int32_t *__restrict__ tok, uint16_t *__restrict__ out,
                                                          int H, int vocab) {
  const int t = blockIdx.y;
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= H) return;
  const int id = tok[t];
  if (id < 0 || id >= vocab) {
    out[(size_t)t * H + k] = 0;
    return;
  }
  const int8_t c = codes[(size_t)id * H + k];
  const float s = scales[(size_t)id * (H / 32) + k / 32];
  out[(size_t)t * H + k] = f2bf((float)c * s);
}

}  // namespace pq

using namespace pq;

static bool pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

extern "C" int pq_rmsnorm(uint16_t *x, const uint16_t *h, const float *w0, const float *w1, uint16_t *y, int8_t *qx,
                          float *dx, int H, int T, float eps, void *stream) {
  PQ_REQUIRE(x && w0 && (y || qx), PQ_ERR_ARG, "pq_rmsnorm: null pointer");
  PQ_REQUIRE(!h || w1, PQ_ERR_ARG, "pq_rmsnorm: the residual form needs w1");
  PQ_REQUIRE(!qx || dx, PQ_ERR_ARG, "pq_rmsnorm: qx without dx");
  PQ_REQUIRE(pow2(H) && H >= 256 && H <= 8192 && T > 0, PQ_ERR_ARG, "pq_rmsnorm: H=%d (power of two, 256..8192)",
             H);
  hipStream_t st = as_stream(stream);
  const dim3 grid(T), block(H / 8);
  if (h) launch(rmsnorm_kernel<true>, grid, block, 0, st, x, h, w0, w1, y, qx, dx, H, eps);
  else launch(rmsnorm_kernel<false>, grid, block, 0, st, x, h, w0, w1, y, qx, dx, H, eps);
  return check_launch("pq_rmsnorm");
}

static int qk_prep_entry(uint16_t *qkv, int row_stride, const float *q_norm, const float *k_norm,
                         const float *rope_cs, uint16_t *kcache, uint16_t *vcache, int pos0, int nh, int nkv, int hd,
                         int rot, int T, float eps, void *stream, bool kv_bf16, const char *who) {
  PQ_REQUIRE(qkv && q_norm && k_norm && rope_cs && kcache && vcache, PQ_ERR_ARG, "%s: null pointer", who);
  PQ_REQUIRE(hd == 64 || hd == 128, PQ_ERR_ARG, "%s: head_dim %d (64 or 128)", who, hd);
  PQ_REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && rot >= 0 && rot <= hd && rot % 2 == 0 && T > 0 && pos0 >= 0,
             PQ_ERR_ARG, "%s: nh=%d nkv=%d rot=%d T=%d pos0=%d", who, nh, nkv, rot, T, pos0);
  PQ_REQUIRE(row_stride >= (nh + 2 * nkv) * hd, PQ_ERR_ARG, "%s: row stride %d too small", who, row_stride);
  return qk_prep_launch(qkv, row_stride, q_norm, k_norm, rope_cs, kcache, vcache, pos0, nullptr, nh, nkv, hd, rot, T,
                        eps, as_stream(stream), kv_bf16);
}

extern "C" int pq_qk_prep(uint16_t *qkv, int row_stride, const float *q_norm, const float *k_norm, const float *rope_cs,
                          uint16_t *kcache, uint16_t *vcache, int pos0, int nh, int nkv, int hd, int rot, int T,
                          float eps, void *stream) {
  return qk_prep_entry(qkv, row_stride, q_norm, k_norm, rope_cs, kcache, vcache, pos0, nh, nkv, hd, rot, T, eps,
                       stream, false, "pq_qk_prep");
}

extern "C" int pq_qk_prep_ref(uint16_t *qkv, int row_stride, const float *q_norm, const float *k_norm,
                              const float *rope_cs, uint16_t *kcache, uint16_t *vcache, int pos0, int nh, int nkv,
                              int hd, int rot, int T, float eps, void *stream) {
  return qk_prep_entry(qkv, row_stride, q_norm, k_norm, rope_cs, kcache, vcache, pos0, nh, nkv, hd, rot, T, eps,
                       stream, true, "pq_qk_prep_ref");
}

namespace pq {
int qk_prep_launch(uint16_t *qkv, int row_stride, const float *q_norm, const float *k_norm, const float *rope_cs,
                   uint16_t *kcache, uint16_t *vcache, int pos0, const int32_t *pos_dev, int nh, int nkv, int hd,
                   int rot, int T, float eps, hipStream_t st, bool kv_bf16) {
#define PQ_QKP(HH, KB)                                                                                             \
  launch(qk_prep_kernel<HH, KB>, dim3(nh + 2 * nkv, T), dim3(64), 0, st, qkv, row_stride, q_norm, k_norm, rope_cs, \
         kcache, vcache, pos0, nh, nkv, rot, eps, pos_dev)
  if (hd == 64) {
    if (kv_bf16) PQ_QKP(64, true);
    else PQ_QKP(64, false);
  } else {
    if (kv_bf16) PQ_QKP(128, true);
    else PQ_QKP(128, false);
  }
#undef PQ_QKP
  return check_launch("pq_qk_prep");
}
}  // namespace pq

extern "C" int pq_conv(uint16_t *ring, const float *taps, const uint16_t *bcx, uint16_t *out, int H, int T, int ntaps,
                       void *stream) {
  PQ_REQUIRE(ring && taps && bcx && out, PQ_ERR_ARG, "pq_conv: null pointer");
  PQ_REQUIRE(H > 0 && T > 0, PQ_ERR_ARG, "pq_conv: H=%d T=%d", H, T);
  // 64 channels x 32 positions per workgroup; up to 8 waves over the positions
  const int waves = T < 8 ? T : 8;
  const dim3 grid((H + 63) / 64, (T + kConvTP - 1) / kConvTP), block(64 * waves);
  hipStream_t st = as_stream(stream);
  switch (ntaps) {
    case 2: launch(conv_kernel<2>, grid, block, 0, st, ring, taps, bcx, out, H, T); break;
    case 3: launch(conv_kernel<3>, grid, block, 0, st, ring, taps, bcx, out, H, T); break;
    case 4: launch(conv_kernel<4>, grid, block, 0, st, ring, taps, bcx, out, H, T); break;
    case 7: launch(conv_kernel<7>, grid, block, 0, st, ring, taps, bcx, out, H, T); break;
    default: return fail(PQ_ERR_ARG, "pq_conv: ntaps %d (2, 3, 4 or 7)", ntaps);
  }
  return check_launch("pq_conv");
}

static int silu_mul(const uint16_t *gu, uint16_t *y, int8_t *qx, float *dx, int F, int T, bool il, void *stream,
                    const char *who) {
  PQ_REQUIRE(gu && (y || qx) && (!qx || dx), PQ_ERR_ARG, "%s: null pointer", who);
  PQ_REQUIRE(F > 0 && F % 256 == 0 && T > 0, PQ_ERR_ARG, "%s: F=%d (a multiple of 256)", who, F);
  constexpr int E = 8;
  // threads per workgroup: the largest of 256, 128, 64, 32 that divides the
  // F/E thread count (F % 256 == 0 makes 32 always one), so the grid covers F
  // exactly -- F = 7680 (the LFM3 FFN) runs 15 workgroups of 64
  int threads = 256;
  while ((F / E) % threads != 0) threads >>= 1;
  if (il)
    launch(silu_mul_kernel<E, true>, dim3(F / E / threads, T), dim3(threads), 0, as_stream(stream), gu, y, qx, dx, F);
  else
    launch(silu_mul_kernel<E, false>, dim3(F / E / threads, T), dim3(threads), 0, as_stream(stream), gu, y, qx, dx, F);
  return check_launch(who);
}

extern "C" int pq_silu_mul(const uint16_t *gu, uint16_t *y, int8_t *qx, float *dx, int F, int T, void *stream) {
  return silu_mul(gu, y, qx, dx, F, T, false, stream, "pq_silu_mul");
}

extern "C" int pq_silu_mul_interleaved(const uint16_t *gu, uint16_t *y, int8_t *qx, float *dx, int F, int T,
                                       void *stream) {
  return silu_mul(gu, y, qx, dx, F, T, true, stream, "pq_silu_mul_interleaved");
}

extern "C" int pq_argmax(const float *v, int n, int32_t *out, void *stream) {
  PQ_REQUIRE(v && out && n > 0, PQ_ERR_ARG, "pq_argmax: n=%d", n);
  launch(argmax_kernel, dim3(1), dim3(1024), 0, as_stream(stream), v, n, out);
  return check_launch("pq_argmax");
}

extern "C" int pq_embed(const int8_t *pcodes, const uint16_t *pscales, const int32_t *tokens, uint16_t *out, int H,
                        int vocab, int T, void *stream) {
  PQ_REQUIRE(pcodes && pscales && tokens && out, PQ_ERR_ARG, "pq_embed: null pointer");
  PQ_REQUIRE(H > 0 && H % 32 == 0 && vocab > 0 && T > 0, PQ_ERR_ARG, "pq_embed: H=%d vocab=%d T=%d", H, vocab, T);
  launch(embed_kernel, dim3((H + 255) / 256, T), dim3(256), 0, as_stream(stream), pcodes, pscales, tokens, out, H,
         vocab);
  return check_launch("pq_embed");
}

extern "C" int pq_embed_rows(const int8_t *codes, const float *scales, const int32_t *tokens, uint16_t *out, int H,
                             int vocab, int T, void *stream) {
  PQ_REQUIRE(codes && scales && tokens && out, PQ_ERR_ARG, "pq_embed_rows: null pointer");
  PQ_REQUIRE(H > 0 && H % 32 == 0 && vocab > 0 && T > 0, PQ_ERR_ARG, "pq_embed_rows: H=%d vocab=%d T=%d", H, vocab,
             T);
  launch(embed_rows_kernel, dim3((H + 255) / 256, T), dim3(256), 0, as_stream(stream), codes, scales, tokens, out, H,
         vocab);
  return check_launch("pq_embed_rows");
}
