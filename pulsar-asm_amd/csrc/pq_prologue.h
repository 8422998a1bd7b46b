// pq_prologue.h -- the activation prologues of the fused GEMVs (gfx950): the
// small ops of a decode step (residual add + RMSNorm, RMSNorm, SiLU * up, the
// gated short conv, the embedding row) computed by the GEMV that consumes
// them, redundantly in every workgroup, with the unfused ops' arithmetic and
// order (sums of squares in rmsnorm_body's order, the same bf16 roundings), so a fused step is
// bit-identical to the unfused one. Shared by the Q8_0, reference-numerics and
// Q4 / Q5 GEMVs.
#pragma once

#include "pq_device.h"
#include "pq_host.h"
#include "q8_common.h"

namespace pq {

// --------------------------------------------------------- block helpers

// E contiguous bf16 (E = 4, 8 or 16) as E/2 packed dwords, one 8- or 16-byte
// vector load per 8 elements; lo/hi unpack to fp32.
template <int E>
__device__ __forceinline__ void ld_raw(const uint16_t *__restrict__ p, uint32_t *o) {
  if constexpr (E == 4) {
    const uint2 u = *reinterpret_cast<const uint2 *>(p);
    o[0] = u.x; o[1] = u.y;
  } else {
#pragma unroll
    for (int i = 0; i < E / 8; i++) {
      const uint4 u = reinterpret_cast<const uint4 *>(p)[i];
      o[4 * i] = u.x; o[4 * i + 1] = u.y; o[4 * i + 2] = u.z; o[4 * i + 3] = u.w;
    }
  }
}
__device__ __forceinline__ float bf_at(const uint32_t *w, int i) {
  return __uint_as_float((i & 1) ? (w[i >> 1] & 0xffff0000u) : (w[i >> 1] << 16));
}
template <int E>
__device__ __forceinline__ void ld_f32(const float *__restrict__ p, float *o) {
#pragma unroll
  for (int i = 0; i < E / 4; i++) {
    const float4 f = reinterpret_cast<const float4 *>(p)[i];
    o[4 * i] = f.x; o[4 * i + 1] = f.y; o[4 * i + 2] = f.z; o[4 * i + 3] = f.w;
  }
}

// E bf16 already packed in pairs (E/2 dwords)
template <int E>
__device__ __forceinline__ void st_bf16w(uint16_t *__restrict__ p, const uint32_t *w) {
  if constexpr (E == 4) {
    *reinterpret_cast<uint2 *>(p) = make_uint2(w[0], w[1]);
  } else {
#pragma unroll
    for (int i = 0; i < E / 8; i++)
      reinterpret_cast<uint4 *>(p)[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
  }
}

// The sum of squares of a norm prologue over K = E * blockDim elements, in
// rmsnorm_body's order (ref_sumsq); red holds kNormSlots partials per sum,
// so the two sums of RESNORM take red and red + kNormSlots (K <= 8192).
constexpr int kNormSlots = 32;
template <int E>
__device__ __forceinline__ float pro_sumsq(const float *v, float *red, int K) {
  return ref_sumsq<E, true>(v, red, K / 256);
}

// y = bf16(w * bf16(x * rs)) for the thread's E values.
template <int E>
__device__ __forceinline__ void norm_apply(float *x, const float *w, float ss, int K, float eps) {
  const float rs = 1.0f / sqrtf(ss * (1.0f / (float)K) + eps);
#pragma unroll
  for (int i = 0; i < E; i += 2) {
    float a = x[i] * rs, b = x[i + 1] * rs;
    bfr2(a, b);
    x[i] = w[i] * a;
    x[i + 1] = w[i + 1] * b;
    bfr2(x[i], x[i + 1]);
  }
}

// ------------------------------------------------------------- prologues
// Phase 1 (pro_load) issues every global load of the thread's E elements, raw;
// the GEMV then issues its weight loads; phase 2 (pro_compute) does the math
// with LDS-only barriers and leaves the Q8_0 x in LDS.
// The CONV prologue comes in two tap counts (3: the synthetic backbone; 7:
// LFM3's conv_L_cache): the template kind kProConv7 is PQ_PRO_CONV with 7 taps.
constexpr int kProConv7 = 0x100 | PQ_PRO_CONV;
constexpr int kProEmbedR = 0x100 | PQ_PRO_EMBED;   // EMBED on the row-major table (the R2 GEMV)
constexpr int pro_base(int pro) { return pro & 0xff; }
constexpr int conv_taps(int pro) { return pro == kProConv7 ? 7 : 3; }

template <int E, int NT>
struct ProRegs {
  uint32_t u0[E / 2], u1[E / 2], u2[E / 2];
  uint32_t ring[NT - 1][E / 2];
  float f0[E], f1[E];
  float taps[E * NT];
  uint32_t emb_c[E / 4];
  uint16_t emb_s;
  float emb_f;
};

template <int PRO, int E>
__device__ __forceinline__ void pro_load(const pq_gemv_prologue &p, int e0, int K,
                                         ProRegs<E, conv_taps(PRO)> &r) {
  constexpr int NT = conv_taps(PRO);
  if constexpr (PRO == PQ_PRO_Q8) {
#pragma unroll
    for (int i = 0; i < E / 4; i++) r.emb_c[i] = reinterpret_cast<const uint32_t *>(p.qx + e0)[i];
    r.f0[0] = (e0 & 31) == 0 ? p.dx[e0 >> 5] : 0.0f;
  } else if constexpr (PRO == PQ_PRO_F32) {
    ld_f32<E>(p.xf + e0, r.f0);
  } else if constexpr (PRO == PQ_PRO_RESNORM) {
    ld_raw<E>(p.h + e0, r.u0);
    ld_raw<E>(p.x_in + e0, r.u1);
    ld_f32<E>(p.w0 + e0, r.f0);
    ld_f32<E>(p.w1 + e0, r.f1);
  } else if constexpr (PRO == PQ_PRO_NORM) {
    ld_raw<E>(p.x_in + e0, r.u0);
    ld_f32<E>(p.w0 + e0, r.f0);
  } else if constexpr (PRO == PQ_PRO_EMBED) {
    const int id = *p.tok;
    const bool ok = id >= 0 && id < p.vocab;
    const int nb = K / kQ, nch = nchunks(K), tile = ok ? id / kTR : 0, rr = ok ? id % kTR : 0;
    const int b = e0 / kQ;   // E <= 32 elements, all in block b
#pragma unroll
    for (int i = 0; i < E / 4; i++) {   // element e0+4i: half (e % 32) / 16 of the block's slab
      const int e = e0 + 4 * i, hh = (e % kQ) / 16, jj = e % 16;
      const int8_t *src = p.emb_pc + (((size_t)tile * nb + b) * 2 + hh) * (kTR * 16) + rr * 16 + jj;
      r.emb_c[i] = ok ? *reinterpret_cast<const uint32_t *>(src) : 0u;
    }
    r.emb_s = ok ? p.emb_ps[(((size_t)tile * nch + b / kCB) * kTR + rr) * kCB + (b % kCB)] : (uint16_t)0;
    ld_f32<E>(p.w0 + e0, r.f0);
  } else if constexpr (PRO == kProEmbedR) {
    const int id = *p.tok;
    const bool ok = id >= 0 && id < p.vocab;   // an id outside the table gives a zero row
    const uint32_t *src = reinterpret_cast<const uint32_t *>(p.emb_pc + (size_t)(ok ? id : 0) * K + e0);
#pragma unroll
    for (int i = 0; i < E / 4; i++) r.emb_c[i] = ok ? src[i] : 0u;
    r.emb_f = ok ? p.emb_sf[(size_t)id * (K / kQ) + e0 / kQ] : 0.0f;   // E <= 32: one block
    ld_f32<E>(p.w0 + e0, r.f0);
  } else if constexpr (PRO == PQ_PRO_SILU) {
    ld_raw<E>(p.gu + e0, r.u0);
    ld_raw<E>(p.gu + K + e0, r.u1);
  } else if constexpr (pro_base(PRO) == PQ_PRO_CONV) {
    ld_raw<E>(p.bcx + e0, r.u0);          // B
    ld_raw<E>(p.bcx + K + e0, r.u1);      // C
    ld_raw<E>(p.bcx + 2 * K + e0, r.u2);  // x
#pragma unroll
    for (int k = 1; k < NT; k++) ld_raw<E>(p.ring_in + (size_t)k * K + e0, r.ring[k - 1]);
    ld_f32<E * NT>(p.taps + (size_t)e0 * NT, r.taps);
  }
}

// The prologue's x values for the thread's E elements (every kind but Q8),
// bf16-rounded where the unfused op rounds; the vectors it writes once
// (x_out, ring_out) are written by workgroup 0.
template <int PRO, int E>
__device__ __forceinline__ void pro_values(const pq_gemv_prologue &p, int e0, int K, ProRegs<E, conv_taps(PRO)> &r,
                                           float *red, float *v) {
  constexpr int NT = conv_taps(PRO);
  const bool writer = blockIdx.x == 0 && blockIdx.y == 0;
  if constexpr (PRO == PQ_PRO_RESNORM) {
#pragma unroll
    for (int i = 0; i < E; i++) v[i] = bf_at(r.u0, i);
    const float ss = pro_sumsq<E>(v, red, K);
    const float rs = 1.0f / sqrtf(ss * (1.0f / (float)K) + p.eps);
    uint32_t xn[E / 2];
#pragma unroll
    for (int i = 0; i < E; i += 2) {
      float a = v[i] * rs, b = v[i + 1] * rs;
      bfr2(a, b);
      a = r.f0[i] * a;
      b = r.f0[i + 1] * b;
      bfr2(a, b);   // h3
      v[i] = bf_at(r.u1, i) + a;
      v[i + 1] = bf_at(r.u1, i + 1) + b;
      xn[i >> 1] = bfr2(v[i], v[i + 1]);
    }
    if (writer) st_bf16w<E>(p.x_out + e0, xn);
    norm_apply<E>(v, r.f1, pro_sumsq<E>(v, red + kNormSlots, K), K, p.eps);
  } else if constexpr (PRO == PQ_PRO_F32) {
#pragma unroll
    for (int i = 0; i < E; i++) v[i] = r.f0[i];
  } else if constexpr (PRO == PQ_PRO_NORM) {
#pragma unroll
    for (int i = 0; i < E; i++) v[i] = bf_at(r.u0, i);
    norm_apply<E>(v, r.f0, pro_sumsq<E>(v, red, K), K, p.eps);
  } else if constexpr (PRO == PQ_PRO_EMBED) {
    const float sc = h2f(r.emb_s);
    uint32_t xb[E / 2];
#pragma unroll
    for (int i = 0; i < E; i++) v[i] = (float)(int8_t)((r.emb_c[i >> 2] >> (8 * (i & 3))) & 0xffu) * sc;
#pragma unroll
    for (int i = 0; i < E; i += 2) xb[i >> 1] = bfr2(v[i], v[i + 1]);
    if (writer) st_bf16w<E>(p.x_out + e0, xb);
    norm_apply<E>(v, r.f0, pro_sumsq<E>(v, red, K), K, p.eps);
  } else if constexpr (PRO == kProEmbedR) {   // pq_embed_rows' bf16(code * scale), then the norm
    uint32_t xb[E / 2];
#pragma unroll
    for (int i = 0; i < E; i++) v[i] = (float)(int8_t)((r.emb_c[i >> 2] >> (8 * (i & 3))) & 0xffu) * r.emb_f;
#pragma unroll
    for (int i = 0; i < E; i += 2) xb[i >> 1] = bfr2(v[i], v[i + 1]);
    if (writer) st_bf16w<E>(p.x_out + e0, xb);
    norm_apply<E>(v, r.f0, pro_sumsq<E>(v, red, K), K, p.eps);
  } else if constexpr (PRO == PQ_PRO_SILU) {
#pragma unroll
    for (int i = 0; i < E; i++) {
      const float a = bf_at(r.u0, i);
      const float sg = 1.0f / (1.0f + expf_pq(-a));
      v[i] = (a * sg) * bf_at(r.u1, i);
    }
#pragma unroll
    for (int i = 0; i < E; i += 2) bfr2(v[i], v[i + 1]);
  } else if constexpr (pro_base(PRO) == PQ_PRO_CONV) {
    // the shifted ring keeps the stored bf16 bits; its new entry is bx = bf16(B*x)
    uint32_t bxw[E / 2];
#pragma unroll
    for (int i = 0; i < E; i += 2) {
      float a = bf_at(r.u0, i) * bf_at(r.u2, i), b = bf_at(r.u0, i + 1) * bf_at(r.u2, i + 1);
      bxw[i >> 1] = bfr2(a, b);
    }
#pragma unroll
    for (int i = 0; i < E; i++) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < NT; k++)
        acc = acc + r.taps[i * NT + k] * bf_at(k + 1 < NT ? r.ring[k] : bxw, i);
      v[i] = acc;
    }
#pragma unroll
    for (int i = 0; i < E; i += 2) {
      bfr2(v[i], v[i + 1]);   // cy
      v[i] = bf_at(r.u1, i) * v[i];
      v[i + 1] = bf_at(r.u1, i + 1) * v[i + 1];
      bfr2(v[i], v[i + 1]);
    }
    if (writer) {
#pragma unroll
      for (int k = 0; k + 1 < NT; k++) st_bf16w<E>(p.ring_out + (size_t)k * K + e0, r.ring[k]);
      st_bf16w<E>(p.ring_out + (size_t)(NT - 1) * K + e0, bxw);
    }
  }
}

}  // namespace pq
