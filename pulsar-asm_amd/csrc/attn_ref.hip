// attn_ref.hip -- the attention of the reference-numerics engine (gfx950), in
// the reference's own order: k_attn_head (lfm3_nanode.cu:503-602) over a bf16
// KV cache [pos][nkv][hd] (written by pq_qk_prep_ref, as k_kv_write copies the
// bf16 rows, 157-162), then k_sigmoid_gate's gate (852-858). For one decode
// token the same kernel also forms the position's q, k and v rows itself
// (pq_attn_decode_ref: the PREP form below), bit for bit the two launches.
//
// One workgroup per (q head, query position t), as the reference launches a
// block of 256 per head (blockIdx.y the chunk position). Threads 0..255 are
// the reference's: its 8 warps of 32 are the 32-lane halves of waves 0-3
// (lane = tid & 31, warp = tid >> 5), so every sum keeps its place. The scores
// do not depend on which warp forms them, so all 32 warps of the 1024 threads
// share them (a quarter of the key rounds, four waves a SIMD to hide latency):
//   score p (warp p mod 32): lane l's chain s = fl(s + fl(q_d * k_d)) over its
//     hd/32 dims from 0, the shfl_down tree over the 32 lanes, fl(s * scale);
//   m = the largest score (a max: any order gives it);
//   e_p = e^(s_p - m) by pq::expf_pq, the build's e^x, where the reference
//     calls CUDA's expf (not restated bit for bit); thread t sums e over
//     p = t, t + 256, ... in order, the shfl_down tree per warp, the 8 warp
//     sums by the tree of offsets 4, 2, 1; inv = 1 / sum;
//   the value sum: warp g (segment g) accumulates fl(w_p * v_pd), w_p =
//     fl(e_p * inv), over p = g, g + 8, ... in order for the lane's hd/32
//     dims; out_d = bf16 of the 8 segments added pairwise.
// p counts from the window's first key lo (the reference's i and p). head_dim
// 128 is the reference's (4 dims a lane); 64 takes 2.
#include "pq_device.h"
#include "pq_host.h"
#include "pq_internal.h"
#include "pq_prologue.h"
#include "q8_common.h"
#include "q8r_common.h"


namespace pq {

constexpr int kArRound = 8;          // keys a warp loads per round
constexpr int kArMaxKeys = 32768;    // keys in one window (LDS: 4 bytes each)

// the shfl_down tree of a 32-lane warp (offsets 16 .. 1): lane 0 of each half
// of the wave ends with its warp's sum
__device__ __forceinline__ float warp_tree32(float s) {
  s = add_down<16>(s);
  s = add_down<8>(s);
  s = add_down<4>(s);
  s = add_down<2>(s);
  return add_down<1>(s);
}

// E consecutive bf16 values of a cache row: one 8-byte (E = 4) or 4-byte load
template <int E>
struct KVPiece {
  using T = uint2;
};
template <>
struct KVPiece<2> {
  using T = uint32_t;
};
// the lane's piece at byte offset off of a cache resource (zeros past its end)
template <int E>
__device__ __forceinline__ typename KVPiece<E>::T kv_load(__amdgpu_buffer_rsrc_t r, int off) {
  if constexpr (E == 4) {
    const v2i v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
    return make_uint2((uint32_t)v.x, (uint32_t)v.y);
  } else {
    return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
  }
}
template <int E>
__device__ __forceinline__ void kv_unpack(const typename KVPiece<E>::T &w, float *f) {
  if constexpr (E == 4) {
    f[0] = __uint_as_float(w.x << 16);
    f[1] = __uint_as_float(w.x & 0xffff0000u);
    f[2] = __uint_as_float(w.y << 16);
    f[3] = __uint_as_float(w.y & 0xffff0000u);
  } else {
    f[0] = __uint_as_float(w << 16);
    f[1] = __uint_as_float(w & 0xffff0000u);
  }
}

constexpr int kArThreads = 1024;     // 32 warps for the scores; the first 256 are the reference's

// The decode launch's own q/k prep (attn_ref_kernel<HD, true>): the inputs of
// qk_prep_kernel for the token's q, k and v rows.
struct AttnPrep {
  const float *qn, *kn;   // q and k head-norm weights [hd]
  const float *cs;        // RoPE (cos, sin) pairs [pos][rot / 2]
  int rot;                // rotated dims
  float eps;
};

// GQ (with PREP): the head's gate is not read from the row but formed here,
// for a layer whose gate rows are a Q8 part of their own (a low-bit blob keeps
// gate_proj in Q8): rows [nh][kGateK] of codes and fp32 block scales, applied
// to y = rmsnorm(x, w) of the residual x (bf16 [kGateK]) in rmsnorm_body's
// order, with the arithmetic of the reference-numerics GEMV (its RESNORM
// prologue's second norm, the 32 leaf chains, the leaf tree, bf16 of 0 +
// the sum): the same bits as that GEMV's launch, which the layer then skips.
// Waves 4-7 form y while waves 0-2 prepare q, k, v; wave 8 dots the gate row
// while waves 0-3 form the softmax sums.
constexpr int kGateK = 2048;
struct AttnGate {
  const int8_t *codes;     // [nh][kGateK] int8
  const float *scales;     // [nh][kGateK / 32]
  const uint16_t *x;       // the residual, bf16 [kGateK]
  const float *w;          // the norm weight [kGateK]
  float eps;
};

// PREP (one decode token, T = 1): q is the token's projected row [q | k | v]
// (nh, nkv, nkv heads), and the workgroup first forms the position's q, k and
// v rows as qk_prep_kernel does (head norm and RoPE for q and k, v as it is):
// q into qs, bf16 k and v into kvn, and the k and v rows into the cache by the
// group's first q head. The cache reads stop before that row, which no
// workgroup reads back; each workgroup takes the position's key and value from
// kvn instead, as the last key of its score warp and of its value segment, so
// every sum keeps the order of the unfused pair (pq_qk_prep_ref, then the
// attention of this kernel without PREP).
template <int HD, bool PREP, bool GQ>
__global__ __launch_bounds__(kArThreads) void attn_ref_kernel(const uint16_t *__restrict__ q, int q_stride,
                                                        uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                                                        const uint16_t *__restrict__ gate, int gate_stride,
                                                        uint16_t *__restrict__ out, int out_stride, int pos0,
                                                        const int32_t *__restrict__ pos_dev, int nh, int nkv,
                                                        float scale, int win, AttnPrep pp, AttnGate gq) {
  static_assert(PREP || !GQ, "the gate is formed in the one-token form");
  constexpr int E = HD / 32;
  using KT = typename KVPiece<E>::T;
  extern __shared__ __align__(16) float sl[];   // the window's scores, then their e
  __shared__ float red[kArThreads / 64];
  __shared__ float seg[8][HD];
  __shared__ float qs[PREP ? HD : 1];                      // PREP: the position's q
  __shared__ __align__(16) uint16_t kvn[PREP ? 2 * HD : 2];   // PREP: its bf16 k, then v
  __shared__ __align__(16) float gpart[GQ ? 8 : 1];                      // GQ: y's sum-of-squares partials
  __shared__ __align__(16) float gxs[GQ ? (kGateK / kQ) * kRXStride : 4];   // GQ: y in the leaves' layout
  __shared__ float gval;                                                  // GQ: the gate (bf16 value)
  const int h = blockIdx.x, t = blockIdx.y, tid = threadIdx.x, lane = tid & 31, wid = tid >> 5;
  const int npos = (pos_dev != nullptr ? *pos_dev : pos0) + t + 1;
  const int lo = window_lo(npos, win), np = npos - lo;
  const int kvd = nkv * HD, kvh = h / (nh / nkv);
  const size_t kvo = (size_t)kvh * HD + lane * E;   // the lane's dims within a cache row
  // the caches up to the query's position (PREP: before it): keys past read zeros
  const int nrow = PREP ? npos - 1 : npos;
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(kc, (short)0, nrow * kvd * 2, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(vc, (short)0, nrow * kvd * 2, kRsrcWord3);
  // score warp w's keys: lo + w + 32j; value segment w's (w < 8): lo + w + 8j.
  // Rounds of kArRound keys whose loads all go out before the round is
  // computed; the first round of value rows is loaded before the softmax,
  // which hides its latency. The kernel is bound by instruction latency, so
  // short rounds (the fewest key slots issued past the window) measured
  // fastest: 290 keys at 256 threads 7.8 us at 8 a round, 8.4 at 16, 10.5 at 64
  // (head_dim 64).
  constexpr int B = kArRound;
  constexpr int W = kArThreads / 32;   // score warps
  const int nks = np > wid ? (np - wid + W - 1) / W : 0;   // this warp's keys: lo + wid + W j
  const int nk = np > wid ? (np - wid + 7) / 8 : 0;        // segment wid's keys (wid < 8): lo + wid + 8 j
  auto ld = [&](__amdgpu_buffer_rsrc_t r, KT *w, int j0, int stride) {
#pragma unroll
    for (int b = 0; b < B; b++)
      w[b] = kv_load<E>(r, (int)(((size_t)(lo + wid + stride * (j0 + b)) * kvd + kvo) * 2));
  };
  KT wk[B], wv[B];
  if (nks > 0) ld(rk, wk, 0, W);   // the first round's keys load during the prep
  float qv[E];
  float gy[8], gw[8];   // GQ, threads 256..511: 8 elements of the residual and of the norm weight
  RBlocks gB;           // GQ, wave 8: the head's gate row (leaf L: blocks L and L + 32)
  if constexpr (GQ) {
    if (tid >= 256 && tid < 512) {
      const int e0 = (tid - 256) * 8;
      const uint4 u = *reinterpret_cast<const uint4 *>(gq.x + e0);
      const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        gy[2 * i] = __uint_as_float(uw[i] << 16);
        gy[2 * i + 1] = __uint_as_float(uw[i] & 0xffff0000u);
      }
      const float4 w0 = *reinterpret_cast<const float4 *>(gq.w + e0);
      const float4 w1 = *reinterpret_cast<const float4 *>(gq.w + e0 + 4);
      gw[0] = w0.x; gw[1] = w0.y; gw[2] = w0.z; gw[3] = w0.w;
      gw[4] = w1.x; gw[5] = w1.y; gw[6] = w1.z; gw[7] = w1.w;
    } else if (tid >= 512 && tid < 576) {
      const __amdgpu_buffer_rsrc_t gc = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(gq.codes), (short)0,
                                                                          nh * kGateK, kRsrcWord3);
      const __amdgpu_buffer_rsrc_t gs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(gq.scales), (short)0,
                                                                          nh * (kGateK / kQ) * 4, kRsrcWord3);
      q8r_load<2>(gB, gc, gs, h, nh, kGateK, kGateK / kQ, kGateK / kQ, 0, lane);
    }
  }
  if constexpr (PREP) {
    if (tid < 192) {   // wave 0: q, wave 1: k, wave 2: v
      constexpr int EH = HD / 64;
      const int l = tid & 63, part = tid >> 6, pos = npos - 1;
      const uint16_t *src = q + (part == 0 ? h * HD : nh * HD + (part - 1) * kvd + kvh * HD);
      uint16_t *dst = (part == 1 ? kc : vc) + (size_t)pos * kvd + kvh * HD;
      const bool writer = h % (nh / nkv) == 0;
      if (part == 2) {
#pragma unroll
        for (int e = 0; e < EH; e++) {
          const uint16_t vb = src[l + 64 * e];
          kvn[HD + l + 64 * e] = vb;
          if (writer) dst[l + 64 * e] = vb;
        }
      } else {
        const float *w = part == 0 ? pp.qn : pp.kn;
        float x[EH], wn[EH], r[EH];
#pragma unroll
        for (int e = 0; e < EH; e++) {
          x[e] = bf2f(src[l + 64 * e]);
          wn[e] = w[l + 64 * e];
        }
        const int half = pp.rot / 2, pair = HD == 64 ? (l & 31) : l;
        float c = 1.0f, sn = 0.0f;
        if (pair < half) {
          c = pp.cs[((size_t)pos * half + pair) * 2];
          sn = pp.cs[((size_t)pos * half + pair) * 2 + 1];
        }
        norm_rope<HD>(x, wn, c, sn, pp.rot, pp.eps, l, r);
#pragma unroll
        for (int e = 0; e < EH; e++) {
          if (part == 0) {
            qs[l + 64 * e] = r[e];
          } else {
            const uint16_t kb = f2bf(r[e]);
            kvn[l + 64 * e] = kb;
            if (writer) dst[l + 64 * e] = kb;
          }
        }
      }
    }
    if constexpr (GQ) {
      if (tid >= 256 && tid < 512) ref_sumsq_part<8>(gy, gpart, tid - 256);
    }
    __syncthreads();
    if constexpr (GQ) {   // y = rmsnorm(x, w) as the GEMV prologue forms it, into the leaves' layout
      if (tid >= 256 && tid < 512) {
        norm_apply<8>(gy, gw, ordered_sum(gpart, 8), kGateK, gq.eps);
        const int e0 = (tid - 256) * 8;
        float *d = gxs + (e0 >> 5) * kRXStride + (e0 & 31);
        *reinterpret_cast<float4 *>(d) = make_float4(gy[0], gy[1], gy[2], gy[3]);
        *reinterpret_cast<float4 *>(d + 4) = make_float4(gy[4], gy[5], gy[6], gy[7]);
      }
    }
#pragma unroll
    for (int j = 0; j < E; j++) qv[j] = qs[lane * E + j];
  } else {
#pragma unroll
    for (int j = 0; j < E; j++) qv[j] = bf2f(q[(size_t)t * q_stride + (size_t)h * HD + lane * E + j]);
  }
  for (int j0 = 0; j0 < nks; j0 += B) {
    if (j0 > 0) ld(rk, wk, j0, W);
    float s[B];
#pragma unroll
    for (int b = 0; b < B; b++) {
      float kf[E];
      kv_unpack<E>(wk[b], kf);
      s[b] = 0.0f;
#pragma unroll
      for (int j = 0; j < E; j++) s[b] = s[b] + qv[j] * kf[j];
    }
    // the trees of the round's keys step by step (independent chains side by side)
#pragma unroll
    for (int b = 0; b < B; b++) s[b] = add_down<16>(s[b]);
#pragma unroll
    for (int b = 0; b < B; b++) s[b] = add_down<8>(s[b]);
#pragma unroll
    for (int b = 0; b < B; b++) s[b] = add_down<4>(s[b]);
#pragma unroll
    for (int b = 0; b < B; b++) s[b] = add_down<2>(s[b]);
#pragma unroll
    for (int b = 0; b < B; b++) s[b] = add_down<1>(s[b]);
    if (lane == 0) {
#pragma unroll
      for (int b = 0; b < B; b++) {
        const int i = wid + W * (j0 + b);
        if (i < np) sl[i] = s[b] * scale;
      }
    }
  }
  if constexpr (PREP) {   // the position's own key (read as zeros above), from kvn
    const int ws = (np - 1) % W;
    if ((wid >> 1) == (ws >> 1)) {   // its whole wave, for the tree
      float s = 0.0f;
#pragma unroll
      for (int j = 0; j < E; j++) s = s + qv[j] * __uint_as_float((uint32_t)kvn[lane * E + j] << 16);
      s = warp_tree32(s);
      if (wid == ws && lane == 0) sl[np - 1] = s * scale;
    }
  }
  if (wid < 8) ld(rv, wv, 0, 8);
  __syncthreads();
  float mx = -1e30f;
  for (int i = tid; i < np; i += kArThreads) mx = fmaxf(mx, sl[i]);
  mx = wave_max(mx);
  if ((tid & 63) == 0) red[tid >> 6] = mx;
  __syncthreads();
  float m = red[0];
#pragma unroll
  for (int w = 1; w < kArThreads / 64; w++) m = fmaxf(m, red[w]);
  __syncthreads();
  if constexpr (GQ) {   // the head's gate row on y (wave 8; y was written before two barriers)
    if (tid >= 512 && tid < 576) {
      const float a = leaf_tree32(q8r_leaf<2>(gB, gxs, kGateK / kQ, 0, lane));
      if (tid == 512) gval = bf2f(f2bf(0.0f + a));
    }
  }
  if (tid < 256) {   // the reference's threads: e over keys tid, tid + 256, ..., then the warp trees
    float sum = 0.0f;
    for (int i = tid; i < np; i += 256) {
      const float e = expf_pq(sl[i] - m);
      sl[i] = e;
      sum = sum + e;
    }
    sum = warp_tree32(sum);
    if (lane == 0) red[wid] = sum;
  }
  __syncthreads();
  const float inv = 1.0f / (((red[0] + red[4]) + (red[2] + red[6])) + ((red[1] + red[5]) + (red[3] + red[7])));
  // the value sum of segment wid over keys wid, wid + 8, ... (from lo); PREP
  // leaves the last key to the step after the loop
  const int npv = PREP ? np - 1 : np;
  float acc[E];
#pragma unroll
  for (int j = 0; j < E; j++) acc[j] = 0.0f;
  for (int j0 = 0; j0 < (wid < 8 ? nk : 0); j0 += B) {
    if (j0 > 0) ld(rv, wv, j0, 8);
    // branch-free, so the round's weight reads from LDS go out together: keys
    // past the window read a clamped slot and leave acc as it is (a select)
#pragma unroll
    for (int b = 0; b < B; b++) {
      const int i = wid + 8 * (j0 + b);
      const float wt = sl[i < np ? i : np - 1] * inv;
      float vf[E];
      kv_unpack<E>(wv[b], vf);
#pragma unroll
      for (int j = 0; j < E; j++) {
        const float a = acc[j] + wt * vf[j];
        acc[j] = i < npv ? a : acc[j];
      }
    }
  }
  if constexpr (PREP) {   // the position's own value row: its segment's last key
    if (wid == (np - 1) % 8) {
      const float wt = sl[np - 1] * inv;
#pragma unroll
      for (int j = 0; j < E; j++) acc[j] = acc[j] + wt * __uint_as_float((uint32_t)kvn[HD + lane * E + j] << 16);
    }
  }
  if (wid < 8) {
#pragma unroll
    for (int j = 0; j < E; j++) seg[wid][lane * E + j] = acc[j];
  }
  __syncthreads();
  if (tid < HD) {
    const float o = ((seg[0][tid] + seg[1][tid]) + (seg[2][tid] + seg[3][tid])) +
                    ((seg[4][tid] + seg[5][tid]) + (seg[6][tid] + seg[7][tid]));
    uint16_t ob = f2bf(o);
    if (GQ || gate != nullptr) {   // k_sigmoid_gate: bf16(out * 1 / (1 + e^-g))
      const float g = GQ ? gval : bf2f(gate[(size_t)t * gate_stride + h]);
      const float sg = 1.0f / (1.0f + expf_pq(-g));
      ob = f2bf(bf2f(ob) * sg);
    }
    out[(size_t)t * out_stride + (size_t)h * HD + tid] = ob;
  }
}

// pp non-null: the PREP kernel (T = 1); gq non-null (with pp): the GQ form
static int attn_ref_launch(const uint16_t *q, int q_stride, const uint16_t *kcache, const uint16_t *vcache,
                           const uint16_t *gate, int gate_stride, uint16_t *out, int out_stride, int pos0,
                           const int32_t *pos_dev, int keys, int nh, int nkv, int hd, int T, float scale, int win,
                           const AttnPrep *pp, const AttnGate *gq, hipStream_t st) {
  const dim3 grid((unsigned)nh, (unsigned)T), block(kArThreads);
  const size_t lds = (size_t)keys * sizeof(float);
  uint16_t *kc = const_cast<uint16_t *>(kcache), *vc = const_cast<uint16_t *>(vcache);
  const AttnPrep p = pp != nullptr ? *pp : AttnPrep{};
  const AttnGate g = gq != nullptr ? *gq : AttnGate{};
#define PQ_AR(HH, PR, GG)                                                                                  \
  launch(attn_ref_kernel<HH, PR, GG>, grid, block, lds, st, q, q_stride, kc, vc, gate, gate_stride, out, \
         out_stride, pos0, pos_dev, nh, nkv, scale, win, p, g)
  if (hd == 64) {
    if (pp != nullptr && gq != nullptr) PQ_AR(64, true, true);
    else if (pp != nullptr) PQ_AR(64, true, false);
    else PQ_AR(64, false, false);
  } else {
    if (pp != nullptr && gq != nullptr) PQ_AR(128, true, true);
    else if (pp != nullptr) PQ_AR(128, true, false);
    else PQ_AR(128, false, false);
  }
#undef PQ_AR
  return check_launch(pp != nullptr ? "pq_attn_decode_ref" : "pq_attn_ref");
}

static int attn_ref_check(const uint16_t *q, const uint16_t *kcache, const uint16_t *vcache, const uint16_t *out,
                          int nh, int nkv, int hd, int T, int win, int keys, const char *who) {
  PQ_REQUIRE(q && kcache && vcache && out, PQ_ERR_ARG, "%s: null pointer", who);
  PQ_REQUIRE(hd == 64 || hd == 128, PQ_ERR_ARG, "%s: head_dim %d (64 or 128)", who, hd);
  PQ_REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && T > 0 && win >= 0, PQ_ERR_ARG, "%s: nh=%d nkv=%d T=%d win=%d",
             who, nh, nkv, T, win);
  PQ_REQUIRE(aligned(kcache, 16) && aligned(vcache, 16), PQ_ERR_ALIGN, "%s: KV cache must be 16-byte aligned", who);
  PQ_REQUIRE(keys <= kArMaxKeys, PQ_ERR_ARG, "%s: %d keys in a window (at most %d)", who, keys, kArMaxKeys);
  return PQ_OK;
}

static int attn_prep_check(const float *q_norm, const float *k_norm, const float *rope_cs, int hd, int rot,
                           const char *who) {
  PQ_REQUIRE(q_norm && k_norm && rope_cs, PQ_ERR_ARG, "%s: null pointer", who);
  PQ_REQUIRE(rot >= 0 && rot <= hd && rot % 2 == 0, PQ_ERR_ARG, "%s: rot=%d (even, at most head_dim)", who, rot);
  return PQ_OK;
}

// pq_attn_ref at the device position *pos_dev: LDS for the keys of any
// position below ctx.
int attn_ref_dev(const uint16_t *q, int q_stride, const uint16_t *kcache, const uint16_t *vcache,
                 const uint16_t *gate, int gate_stride, uint16_t *out, int out_stride, const int32_t *pos_dev,
                 int ctx, int nh, int nkv, int hd, float scale, int win, hipStream_t st) {
  const int keys = win > 0 && win < ctx ? win : ctx;
  PQ_REQUIRE(pos_dev && ctx > 0, PQ_ERR_ARG, "attn_ref_dev: no position");
  const int rc = attn_ref_check(q, kcache, vcache, out, nh, nkv, hd, 1, win, keys, "attn_ref_dev");
  if (rc) return rc;
  return attn_ref_launch(q, q_stride, kcache, vcache, gate, gate_stride, out, out_stride, 0, pos_dev, keys, nh, nkv,
                         hd, 1, scale, win, nullptr, nullptr, st);
}

// pq_attn_decode_ref at the device position *pos_dev (pos_dev null: pos):
// LDS for the keys of any position below ctx.
int attn_decode_ref_dev(const uint16_t *qkv, const float *q_norm, const float *k_norm, const float *rope_cs,
                        uint16_t *kcache, uint16_t *vcache, const uint16_t *gate, uint16_t *out, int pos,
                        const int32_t *pos_dev, int ctx, int nh, int nkv, int hd, int rot, float eps, float scale,
                        int win, hipStream_t st, const AttnGateQ8 *gq8) {
  const int keys = win > 0 && win < ctx ? win : ctx;
  PQ_REQUIRE(ctx > 0 && (pos_dev || (pos >= 0 && pos < ctx)), PQ_ERR_ARG, "pq_attn_decode_ref: pos=%d ctx=%d",
             pos, ctx);
  int rc = attn_ref_check(qkv, kcache, vcache, out, nh, nkv, hd, 1, win, keys, "pq_attn_decode_ref");
  if (rc) return rc;
  rc = attn_prep_check(q_norm, k_norm, rope_cs, hd, rot, "pq_attn_decode_ref");
  if (rc) return rc;
  const AttnPrep pp{q_norm, k_norm, rope_cs, rot, eps};
  if (gq8 != nullptr) {
    PQ_REQUIRE(gq8->codes && gq8->scales && gq8->x && gq8->w && gq8->K == kGateK, PQ_ERR_ARG,
               "pq_attn_decode_ref: the Q8 gate rows need codes, scales, x, w and K = %d (K = %d)", kGateK, gq8->K);
    PQ_REQUIRE(aligned(gq8->codes, 16) && aligned(gq8->x, 16) && aligned(gq8->w, 16) && aligned(gq8->scales, 4),
               PQ_ERR_ALIGN, "pq_attn_decode_ref: Q8 gate pointer alignment");
    const AttnGate g{gq8->codes, gq8->scales, gq8->x, gq8->w, gq8->eps};
    return attn_ref_launch(qkv, 0, kcache, vcache, nullptr, 0, out, 0, pos, pos_dev, keys, nh, nkv, hd, 1, scale,
                           win, &pp, &g, st);
  }
  return attn_ref_launch(qkv, 0, kcache, vcache, gate, 0, out, 0, pos, pos_dev, keys, nh, nkv, hd, 1, scale, win,
                         &pp, nullptr, st);
}

}  // namespace pq

using namespace pq;

extern "C" int pq_attn_ref(const uint16_t *q, int q_stride, const uint16_t *kcache, const uint16_t *vcache,
                           const uint16_t *gate, int gate_stride, uint16_t *out, int out_stride, int pos0, int nh,
                           int nkv, int hd, int T, float scale, int win, void *stream) {
  PQ_REQUIRE(pos0 >= 0, PQ_ERR_ARG, "pq_attn_ref: pos0=%d", pos0);
  const int last = pos0 + T;   // keys of the chunk's last query
  const int keys = win > 0 && win < last ? win : last;
  const int rc = attn_ref_check(q, kcache, vcache, out, nh, nkv, hd, T, win, keys, "pq_attn_ref");
  if (rc) return rc;
  return attn_ref_launch(q, q_stride, kcache, vcache, gate, gate_stride, out, out_stride, pos0, nullptr, keys, nh,
                         nkv, hd, T, scale, win, nullptr, nullptr, as_stream(stream));
}

extern "C" int pq_attn_decode_ref_q8gate(const uint16_t *qkv, const float *q_norm, const float *k_norm,
                                         const float *rope_cs, uint16_t *kcache, uint16_t *vcache,
                                         const int8_t *gate_codes, const float *gate_scales, const uint16_t *x,
                                         const float *x_norm, uint16_t *out, int pos, int nh, int nkv, int hd, int rot,
                                         float eps, float scale, int win, void *stream) {
  const AttnGateQ8 g{gate_codes, gate_scales, x, x_norm, eps, kGateK};
  return attn_decode_ref_dev(qkv, q_norm, k_norm, rope_cs, kcache, vcache, nullptr, out, pos, nullptr, pos + 1, nh, nkv,
                             hd, rot, eps, scale, win, as_stream(stream), &g);
}

extern "C" int pq_attn_decode_ref(const uint16_t *qkv, const float *q_norm, const float *k_norm,
                                  const float *rope_cs, uint16_t *kcache, uint16_t *vcache, const uint16_t *gate,
                                  uint16_t *out, int pos, int nh, int nkv, int hd, int rot, float eps, float scale,
                                  int win, void *stream) {
  return attn_decode_ref_dev(qkv, q_norm, k_norm, rope_cs, kcache, vcache, gate, out, pos, nullptr, pos + 1, nh, nkv,
                             hd, rot, eps, scale, win, as_stream(stream), nullptr);
}
