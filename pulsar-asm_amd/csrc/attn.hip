// attn.hip -- split-K flash-decode attention over an fp16 KV cache (gfx950).
//
// Positions are cut into splits of 64; pass 1 computes, per (kv head, split,
// query), the G = nh/nkv heads' partial softmax state, pass 2 merges the
// splits of each head in ascending order and applies the per-head sigmoid
// gate (optionally emitting the Q8_0 input of o_proj). head_dim 64 or 128; a
// sliding-window layer (win > 0) sees keys [npos - win, npos) once npos > win.
// Order (the same on the host side):
//   dot_p = fmaf chain over d ascending of q_d * f16(k_pd), s_p = fl(dot_p * scale)
//   split j: m_j = max s_p, e_p = expf(fl(s_p - m_j)), l_j = pairwise sum of the
//            64 slots (zero past npos), o_jd = fmaf chain over p ascending of e_p * v_pd
//   M = max m_j; w_j = expf(fl(m_j - M)); L = fmaf(l_j, w_j, L); O_d = fmaf(o_jd, w_j, O_d)
//   out_d = bf16(fl(O_d / L)), then bf16(out_d * sigmoid(gate_h)).
// Query t of a T-position call sits at position pos0 + t and sees keys
// [0, pos0 + t] (causal), so a prefill chunk and T single-position calls give
// the same bits. The GQA head map h -> h / (nh/nkv) is lfm3_nanode.cu:520.
#include "pq_device.h"
#include "pq_host.h"
#include "pq_internal.h"

namespace pq {

constexpr int kSplit = 64;

// One wave per (kv head g, split j, query t); lane p = position 64j + p for the
// scores, lane l = dimensions l + 64e (e < HD/64) for the value sums; the G
// heads of the group share every K and V load. Splits with no key in the
// window write nothing (the merge starts at the window's first split); the
// slots before lo are absent (no score, e = 0, skipped in the value chain).
template <int G, int HD>
__global__ __launch_bounds__(64) void attn_split_kernel(const uint16_t *__restrict__ q, int q_stride,
                                                         const uint16_t *__restrict__ kc,
                                                         const uint16_t *__restrict__ vc, float *__restrict__ part,
                                                         int pos0, int nh, int nkv, int nsplit_max, float scale,
                                                         int win, const int32_t *__restrict__ pos_dev) {
  constexpr int E = HD / 64, PART = HD + 2;
  __shared__ __align__(16) float qs[G][HD];
  __shared__ float es[G][kSplit];
  const int g = blockIdx.x, j = blockIdx.y, t = blockIdx.z, lane = threadIdx.x;
  const int npos = (pos_dev != nullptr ? *pos_dev : pos0) + t + 1;
  const int lo = window_lo(npos, win);
  const int p0 = j * kSplit;
  if (p0 >= npos || p0 + kSplit <= lo) return;
  const int pn = npos - p0 < kSplit ? npos - p0 : kSplit;
  const int i0 = lo > p0 ? lo - p0 : 0;
  const int kvd = nkv * HD;
#pragma unroll
  for (int h = 0; h < G; h++)
#pragma unroll
    for (int e = 0; e < E; e++) qs[h][lane + 64 * e] = bf2f(q[(size_t)t * q_stride + (g * G + h) * HD + lane + 64 * e]);
  __syncthreads();
  const bool valid = lane >= i0 && lane < pn;
  float dot[G];
#pragma unroll
  for (int h = 0; h < G; h++) dot[h] = 0.0f;
  if (valid) {
    const uint16_t *kr = kc + (size_t)(p0 + lane) * kvd + g * HD;
    for (int d0 = 0; d0 < HD; d0 += 8) {
      const uint4 k8 = *reinterpret_cast<const uint4 *>(kr + d0);
      const uint32_t kw[4] = {k8.x, k8.y, k8.z, k8.w};
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float kf = h2f((uint16_t)(kw[i >> 1] >> (16 * (i & 1))));
#pragma unroll
        for (int h = 0; h < G; h++) dot[h] = __builtin_fmaf(qs[h][d0 + i], kf, dot[h]);
      }
    }
  }
  float m[G], l[G];
#pragma unroll
  for (int h = 0; h < G; h++) {
    const float sc = valid ? dot[h] * scale : -__builtin_inff();
    m[h] = wave_max(sc);
    const float e = valid ? expf_pq(sc - m[h]) : 0.0f;
    l[h] = wave_pairwise_sum(e);
    es[h][lane] = e;
  }
  __syncthreads();
  float o[G][E];
#pragma unroll
  for (int h = 0; h < G; h++)
#pragma unroll
    for (int e = 0; e < E; e++) o[h][e] = 0.0f;
  for (int p = i0; p < pn; p++) {
#pragma unroll
    for (int e = 0; e < E; e++) {
      const float v = h2f(vc[(size_t)(p0 + p) * kvd + g * HD + lane + 64 * e]);
#pragma unroll
      for (int h = 0; h < G; h++) o[h][e] = __builtin_fmaf(es[h][p], v, o[h][e]);
    }
  }
#pragma unroll
  for (int h = 0; h < G; h++) {
    float *pp = part + (((size_t)t * nh + g * G + h) * nsplit_max + j) * PART;
#pragma unroll
    for (int e = 0; e < E; e++) pp[lane + 64 * e] = o[h][e];
    if (lane == 0) {
      pp[HD] = m[h];
      pp[HD + 1] = l[h];
    }
  }
}

// One wave per (head, query); lane l = dimensions l + 64e. The window's
// splits merge in ascending order.
template <int HD>
__global__ __launch_bounds__(64) void attn_merge_kernel(const float *__restrict__ part, int pos0, int nh,
                                                         int nsplit_max, const uint16_t *__restrict__ gate,
                                                         int gate_stride, uint16_t *__restrict__ out, int out_stride,
                                                         int8_t *__restrict__ qx, float *__restrict__ dx, int win,
                                                         const int32_t *__restrict__ pos_dev) {
  constexpr int E = HD / 64, PART = HD + 2;
  const int h = blockIdx.x, t = blockIdx.y, d = threadIdx.x;
  const int npos = (pos_dev != nullptr ? *pos_dev : pos0) + t + 1;
  const int j0 = window_lo(npos, win) / kSplit;
  const int ns = (npos + kSplit - 1) / kSplit;
  const float *pp = part + ((size_t)t * nh + h) * nsplit_max * PART;
  float M = -__builtin_inff();
  for (int j = j0; j < ns; j++) M = fmaxf(M, pp[j * PART + HD]);
  float L = 0.0f, O[E];
#pragma unroll
  for (int e = 0; e < E; e++) O[e] = 0.0f;
  for (int j = j0; j < ns; j++) {
    const float w = expf_pq(pp[j * PART + HD] - M);
    L = __builtin_fmaf(pp[j * PART + HD + 1], w, L);
#pragma unroll
    for (int e = 0; e < E; e++) O[e] = __builtin_fmaf(pp[j * PART + d + 64 * e], w, O[e]);
  }
  const float gs = gate != nullptr ? 1.0f / (1.0f + expf_pq(-bf2f(gate[(size_t)t * gate_stride + h]))) : 0.0f;
#pragma unroll
  for (int e = 0; e < E; e++) {
    uint16_t r = f2bf(O[e] / L);
    if (gate != nullptr) r = f2bf(bf2f(r) * gs);
    const int dd = d + 64 * e;
    if (out != nullptr) out[(size_t)t * out_stride + h * HD + dd] = r;
    if (qx != nullptr) {
      const float v = bf2f(r);
      float a = fabsf(v);
#pragma unroll
      for (int o = 1; o < 32; o <<= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
      const float dq = a / 127.0f;
      // d = 0 only when every |x| of the block is below 127 * 2^-149: dividing
      // by 1 then gives q = 0 as the zero-block rule does, with no branch
      int qv = (int)__builtin_rintf(v / (dq != 0.0f ? dq : 1.0f));
      qv = qv > 127 ? 127 : (qv < -127 ? -127 : qv);
      const size_t K = (size_t)nh * HD;
      qx[(size_t)t * K + h * HD + dd] = (int8_t)qv;
      if ((d & 31) == 0) dx[(size_t)t * (K / 32) + (h * HD + dd) / 32] = dq;
    }
  }
}

}  // namespace pq

using namespace pq;

extern "C" size_t pq_attn_workspace_bytes(int nh, int hd, int max_pos, int T) {
  if (nh <= 0 || (hd != 64 && hd != 128) || max_pos <= 0 || T <= 0) return 0;
  const size_t ns = (size_t)(max_pos + kSplit - 1) / kSplit;
  return (size_t)T * nh * ns * (hd + 2) * sizeof(float);
}

template <int HD>
static int attn_launch(const uint16_t *q, int q_stride, const uint16_t *kcache, const uint16_t *vcache,
                       const uint16_t *gate, int gate_stride, uint16_t *out, int out_stride, int8_t *qx, float *dx,
                       int pos0, const int32_t *pos_dev, int nh, int nkv, int T, float scale, int win, float *part,
                       int nsplit, hipStream_t st) {
  const int G = nh / nkv;
  const dim3 g1(nkv, nsplit, T), b1(64);
  switch (G) {
    case 1: launch(attn_split_kernel<1, HD>, g1, b1, 0, st, q, q_stride, kcache, vcache, part, pos0, nh, nkv, nsplit, scale, win, pos_dev); break;
    case 2: launch(attn_split_kernel<2, HD>, g1, b1, 0, st, q, q_stride, kcache, vcache, part, pos0, nh, nkv, nsplit, scale, win, pos_dev); break;
    case 4: launch(attn_split_kernel<4, HD>, g1, b1, 0, st, q, q_stride, kcache, vcache, part, pos0, nh, nkv, nsplit, scale, win, pos_dev); break;
    case 8: launch(attn_split_kernel<8, HD>, g1, b1, 0, st, q, q_stride, kcache, vcache, part, pos0, nh, nkv, nsplit, scale, win, pos_dev); break;
    default: return fail(PQ_ERR_ARG, "pq_attn_decode: %d q heads per kv head (1, 2, 4 or 8)", G);
  }
  int rc = check_launch("pq_attn_decode split");
  if (rc) return rc;
  launch(attn_merge_kernel<HD>, dim3(nh, T), dim3(64), 0, st, part, pos0, nh, nsplit, gate, gate_stride, out,
         out_stride, qx, dx, win, pos_dev);
  return check_launch("pq_attn_decode merge");
}

extern "C" int pq_attn_decode(const uint16_t *q, int q_stride, const uint16_t *kcache, const uint16_t *vcache,
                              const uint16_t *gate, int gate_stride, uint16_t *out, int out_stride, int8_t *qx,
                              float *dx, int pos0, int nh, int nkv, int hd, int T, float scale, int win, void *ws,
                              size_t ws_bytes, void *stream) {
  PQ_REQUIRE(q && kcache && vcache && (out || qx) && (!qx || dx), PQ_ERR_ARG, "pq_attn_decode: null pointer");
  PQ_REQUIRE(hd == 64 || hd == 128, PQ_ERR_ARG, "pq_attn_decode: head_dim %d (64 or 128)", hd);
  PQ_REQUIRE(nh > 0 && nkv > 0 && nh % nkv == 0 && T > 0 && pos0 >= 0 && win >= 0, PQ_ERR_ARG,
             "pq_attn_decode: nh=%d nkv=%d T=%d pos0=%d win=%d", nh, nkv, T, pos0, win);
  PQ_REQUIRE(aligned(kcache, 16) && aligned(vcache, 16), PQ_ERR_ALIGN, "pq_attn_decode: KV cache must be 16-byte aligned");
  const int max_pos = pos0 + T;
  const int nsplit = (max_pos + kSplit - 1) / kSplit;
  const size_t need = pq_attn_workspace_bytes(nh, hd, max_pos, T);
  PQ_REQUIRE(ws && ws_bytes >= need, PQ_ERR_WORKSPACE, "pq_attn_decode: workspace of %zu bytes needed (got %zu)", need,
             ws_bytes);
  float *part = reinterpret_cast<float *>(ws);
  hipStream_t st = as_stream(stream);
  if (hd == 64)
    return attn_launch<64>(q, q_stride, kcache, vcache, gate, gate_stride, out, out_stride, qx, dx, pos0, nullptr, nh,
                           nkv, T, scale, win, part, nsplit, st);
  return attn_launch<128>(q, q_stride, kcache, vcache, gate, gate_stride, out, out_stride, qx, dx, pos0, nullptr, nh,
                          nkv, T, scale, win, part, nsplit, st);
}

namespace pq {
// One query (T = 1) at the position *pos_dev holds: the split grid and the
// workspace cover positions below ctx, and the splits past the position
// return at once, so a captured launch replays for any position.
int attn_decode_dev(const uint16_t *q, int q_stride, const uint16_t *kcache, const uint16_t *vcache,
                    const uint16_t *gate, int gate_stride, uint16_t *out, int out_stride, int8_t *qx, float *dx,
                    const int32_t *pos_dev, int ctx, int nh, int nkv, int hd, float scale, int win, void *ws,
                    size_t ws_bytes, hipStream_t st) {
  PQ_REQUIRE(q && kcache && vcache && pos_dev && (out || qx) && (!qx || dx) && ctx > 0, PQ_ERR_ARG,
             "attn_decode_dev: bad arguments");
  PQ_REQUIRE(hd == 64 || hd == 128, PQ_ERR_ARG, "attn_decode_dev: head_dim %d", hd);
  const int nsplit = (ctx + kSplit - 1) / kSplit;
  PQ_REQUIRE(ws && ws_bytes >= pq_attn_workspace_bytes(nh, hd, ctx, 1), PQ_ERR_WORKSPACE,
             "attn_decode_dev: workspace too small");
  float *part = reinterpret_cast<float *>(ws);
  if (hd == 64)
    return attn_launch<64>(q, q_stride, kcache, vcache, gate, gate_stride, out, out_stride, qx, dx, 0, pos_dev, nh,
                           nkv, 1, scale, win, part, nsplit, st);
  return attn_launch<128>(q, q_stride, kcache, vcache, gate, gate_stride, out, out_stride, qx, dx, 0, pos_dev, nh,
                          nkv, 1, scale, win, part, nsplit, st);
}
}  // namespace pq
