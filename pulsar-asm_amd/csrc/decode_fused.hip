// decode_fused.hip -- the T=1 decode step with its small ops fused into the
// kernels that consume them (gfx950).
//
// A decode step of the reference is ~15 launches per layer (layer_body,
// lfm3_nanode.cu:3739-3856). Here the GEMV that consumes an activation computes
// it in its own prologue, redundantly in every workgroup (the vectors are 2K-8K
// elements), after issuing its first weight loads so the prologue hides under
// their latency:
//   RESNORM  h3 = rmsnorm(h, w0); x' = bf16(x + h3) (workgroup 0 writes x');
//            y = rmsnorm(x', w1)          -- "rms1 -> eadd -> rms1" of layer_body
//   NORM     y = rmsnorm(x, w0)
//   EMBED    x = embedding row of the device token (workgroup 0 writes x);
//            y = rmsnorm(x, w0)
//   SILU     y = silu(gate) * up
//   CONV     the gated short conv; workgroup 0 writes the shifted ring into the
//            other buffer of a ping-pong pair
//   Q8       y already quantized (qx, dx)
//   F32      y = fp32 x, quantized here
// then quantizes y to Q8_0 in LDS and runs the GEMV of q8.hip on it. Every op
// keeps the unfused kernels' arithmetic and order (the sums of squares in
// rmsnorm_body's order, the same roundings), so the fused step is
// bit-identical to the unfused one.
// The attention mixer of a decode step is one kernel per layer
// (attn_layer_kernel): q/k norm, RoPE, KV write, every split, the ordered
// merge, the sigmoid gate and the Q8_0 output for o_proj.
#include <type_traits>

#include "pq_device.h"
#include "pq_host.h"
#include "q8_common.h"
#include "q8r_common.h"
#include "pq_internal.h"
#include "pq_prologue.h"

namespace pq {

// --------------------------------------------------------- block helpers
// (the prologue kinds and their helpers, pro_load and pro_values, are in
// pq_prologue.h)

// E int8 codes (E/4 dwords) of elements e0.. into the staged-x layout in LDS:
// chunk c at c*kXStride, block i of the chunk at i*32.
template <int E>
__device__ __forceinline__ void store_q8_lds(const uint32_t *w, int e0, int8_t *xs) {
  const int b = e0 >> 5;
  int8_t *dst = xs + (b >> 3) * kXStride + (b & 7) * kQ + (e0 & 31);
  if constexpr (E == 4) {
    *reinterpret_cast<uint32_t *>(dst) = w[0];
  } else {
#pragma unroll
    for (int i = 0; i < E / 8; i++) *reinterpret_cast<uint2 *>(dst + 8 * i) = make_uint2(w[2 * i], w[2 * i + 1]);
  }
}

// The max over each aligned group of L lanes (L a power of two, 1..32), by
// DPP within 16-lane rows and the row-pair swap (all 64 lanes active).
template <int L>
__device__ __forceinline__ float group_max(float a) {
  if constexpr (L >= 2) a = fmaxf(a, dpp_f<kDppXor1>(a));
  if constexpr (L >= 4) a = fmaxf(a, dpp_f<kDppXor2>(a));
  if constexpr (L >= 8) a = fmaxf(a, dpp_f<kDppHalfMirror>(a));
  if constexpr (L >= 16) a = fmaxf(a, dpp_f<kDppMirror>(a));
  if constexpr (L >= 32) a = max_row_pair(a);
  return a;
}

// Q8_0 of the thread's E values (elements e0 .. e0+E-1) into the staged-x
// layout in LDS (chunk c at c*kXStride, block i of the chunk at i*32) and dxs:
// amax over the block's 32/E threads, d = amax/127, q = rne(x/d) clamped.
template <int E>
__device__ __forceinline__ void quant_lds(const float *v, int e0, int8_t *xs, float *dxs) {
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < E; i++) a = fmaxf(a, fabsf(v[i]));
  a = group_max<32 / E>(a);
  const float d = a / 127.0f;
  const Q8Div qd(d);
  uint32_t w[E / 4];
#pragma unroll
  for (int i = 0; i < E / 4; i++) w[i] = 0u;
#pragma unroll
  for (int i = 0; i < E; i++) w[i >> 2] |= (uint32_t)(uint8_t)q8_code(qd.div(v[i])) << (8 * (i & 3));
  store_q8_lds<E>(w, e0, xs);
  if ((e0 & 31) == 0) dxs[e0 >> 5] = d;
}


template <int PRO, int E>
__device__ __forceinline__ void pro_compute(const pq_gemv_prologue &p, int e0, int K, ProRegs<E, conv_taps(PRO)> &r,
                                            float *red, int8_t *xs, float *dxs) {
  if constexpr (PRO == PQ_PRO_Q8) {
    store_q8_lds<E>(r.emb_c, e0, xs);
    if ((e0 & 31) == 0) dxs[e0 >> 5] = r.f0[0];
    lds_barrier();
  } else {
    float v[E];
    pro_values<PRO, E>(p, e0, K, r, red, v);
    quant_lds<E>(v, e0, xs, dxs);
    lds_barrier();
  }
}

// The fused GEMV's outputs from wave 0 (lane l < R holds row tile*64 + l's
// y): the SwiGLU epilogue when qo is given (R = 64, rows interleaved by
// pq_q8_pack_gate_up: lane l < 32 holds gate row 32*tile + l, lane l + 32 its
// up row; writes the Q8_0 block tile of silu(gate) * up as silu_mul_kernel +
// quant_store form it), else y (bf16 or fp32) and, with parts, the (value,
// index) of the pick among its outputs in k_argmax's order (am_better) at
// parts[2*part].
template <int R>
__device__ __forceinline__ void fused_epilogue(float yv, int lane, int tile, int row, int part, void *__restrict__ y,
                                               int y_bf16, int N, float *__restrict__ parts, int8_t *__restrict__ qo,
                                               float *__restrict__ dqo) {
  if (qo != nullptr) {
    if constexpr (R == 64) {
      const float u = bf2f(f2bf(__shfl_down(yv, 32, 64)));
      const float a = bf2f(f2bf(yv));
      const float sg = 1.0f / (1.0f + expf_pq(-a));
      const float o = bf2f(f2bf((a * sg) * u));
      const float m = wave_max(lane < 32 ? fabsf(o) : 0.0f);
      const float d = m / 127.0f;
      int q = (int)__builtin_rintf(o / (d != 0.0f ? d : 1.0f));   // d = 0: the block is all zero
      q = q > 127 ? 127 : (q < -127 ? -127 : q);
      if (lane < 32) qo[32 * tile + lane] = (int8_t)q;
      if (lane == 0) dqo[tile] = d;
    }
    return;
  }
  if (lane < R && row < N) {
    if (y_bf16) reinterpret_cast<uint16_t *>(y)[row] = f2bf(yv);
    else reinterpret_cast<float *>(y)[row] = yv;
  }
  if (parts != nullptr) {
    float v;
    int idx;
    am_leaf((lane < R && row < N) ? yv : kAmFloor, row, v, idx);
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const float ov = __shfl_xor(v, o, 64);
      const int oi = __shfl_xor(idx, o, 64);
      if (am_better(ov, oi, v, idx)) { v = ov; idx = oi; }
    }
    if (lane == 0) {
      parts[2 * part] = v;
      parts[2 * part + 1] = __int_as_float(idx);
    }
  }
}

// ------------------------------------------------------------ fused GEMV
// The GEMV of q8.hip (R rows per workgroup, chunk slots per lane, rounds with an
// ordered LDS fold) with x from the prologue: 64*W threads, E = K/(64*W)
// contiguous elements of the prologue per thread. Optional argmax partials:
// each workgroup writes the (value, index) of its outputs' pick in
// k_argmax's order (am_better) for pq_argmax_parts.
template <int R, int PRO, int E>
__global__ __launch_bounds__(512) void q8_gemv_fused_kernel(const int8_t *__restrict__ pc,
                                                             const uint16_t *__restrict__ ps, pq_gemv_prologue p,
                                                             void *__restrict__ y, int y_bf16, int N, int K,
                                                             float *__restrict__ parts, int8_t *__restrict__ qo,
                                                             float *__restrict__ dqo) {
  constexpr int C = 64 / R;
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ __align__(16) float red[2 * kNormSlots];
  const int nb = K / kQ, nch = nchunks(K);  // K a power of two >= 1024: every chunk is full
  const int W = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int cs = lane / R, r = lane % R;
  const int tile = blockIdx.x / C, trow = (blockIdx.x % C) * R + r;
  const int row = tile * kTR + trow;
  float *sp = reinterpret_cast<float *>(smem);                       // [W*C][R]
  int8_t *xs = reinterpret_cast<int8_t *>(smem + (size_t)W * 64 * 4);
  float *dxs = reinterpret_cast<float *>(xs + (size_t)nch * kXStride);
  const int per_round = W * C;
  const int nrounds = (nch + per_round - 1) / per_round;
  const int slot = wave * C + cs;
  const int e0 = threadIdx.x * E;
  // 1. the prologue's global loads, then round 0's weight loads, then the
  //    prologue math: its waits leave the weight loads in flight
  ProRegs<E, conv_taps(PRO)> pr;
  pro_load<PRO, E>(p, e0, K, pr);
  const TileRsrc tr = tile_rsrc(pc, ps, tile, nb, nch);
  int c = slot;
  ChunkRegs regs;
  load_chunk_rsrc(regs, tr, c, nch, trow);
  pro_compute<PRO, E>(p, e0, K, pr, red, xs, dxs);
  // 2. the GEMV: rounds of W*C chunks, each folded in chunk order
  float yv = 0.0f;
  for (int rd = 0; rd < nrounds; rd++) {
    if (rd > 0) {
      c = rd * per_round + slot;
      load_chunk_rsrc(regs, tr, c, nch, trow);
    }
    float a = 0.0f;
    if (c < nch) {
      const int8_t *xc = xs + (size_t)c * kXStride;
      const int b0 = c * kCB;
      auto XS = [&](int i, int *x) {
        const v4i lo = *reinterpret_cast<const v4i *>(xc + i * 32);
        const v4i hi = *reinterpret_cast<const v4i *>(xc + i * 32 + 16);
        x[0] = lo.x; x[1] = lo.y; x[2] = lo.z; x[3] = lo.w;
        x[4] = hi.x; x[5] = hi.y; x[6] = hi.z; x[7] = hi.w;
      };
      auto DX = [&](int i) { return dxs[b0 + i]; };
      a = dot_chunk(regs, XS, DX);
    }
    sp[slot * R + r] = a;
    __syncthreads();
    if (wave == 0 && lane < R) {
      const int n = nch - rd * per_round < per_round ? nch - rd * per_round : per_round;
      for (int k = 0; k < n; k++) yv = yv + sp[k * R + lane];
    }
    if (rd + 1 < nrounds) __syncthreads();
  }
  if (wave == 0) fused_epilogue<R>(yv, lane, tile, row, (int)blockIdx.x, y, y_bf16, N, parts, qo, dqo);
}

// ------------------------------------ the reference-numerics fused GEMV
// q8r_gemv_kernel at T = 1 with x from a prologue. The prologue's E = K/256
// values per thread (bf16-rounded where the unfused op rounds them) go to LDS
// as fp32 in the 36-float padded blocks the leaf chains read -- the same
// values the unfused op writes as bf16 and the plain kernel widens -- once
// per workgroup: the workgroup then walks row tiles blockIdx.x, + gridDim.x,
// ... (ntiles in all), each tile's 2048-wide chunks in order: its units
// (tile, chunk) u = 0, 1, ... With NS = 2 block sets rotated by name, unit
// u + 1 loads while unit u folds (unit 0 before the prologue; a third set,
// two units ahead, measured slower in the decode step: 0.712 against 0.687
// ms); NS = 1 is the one unit of a single-tile, single-chunk workgroup.
// SWI: the tile is 4 gate rows t*4 + w and their up rows F + t*4 + w (codes
// [2F][K], F = N/2), wave w holding gate row t*4 + w in lanes 0-31 and its up
// row in lanes 32-63; lane 0 forms silu_mul_kernel's output from the bf16
// gate and up values (no barrier per tile). Else, with parts: the (y, row) of
// the workgroup's pick in k_argmax's order (am_better) at parts[2 * blockIdx.x].
template <int BPL, int PRO, int E, int NS, bool SWI>
__global__ __launch_bounds__(kRThreads) void q8r_gemv_fused_kernel(const int8_t *__restrict__ codes,
                                                                   const float *__restrict__ scales,
                                                                   pq_gemv_prologue p, void *__restrict__ y,
                                                                   int y_bf16, int N, int K, int ntiles,
                                                                   float *__restrict__ parts) {
  constexpr int W = kRThreads / 64;
  extern __shared__ __align__(16) float rxs[];   // [nb][kRXStride]
  __shared__ __align__(16) float red[2 * kNormSlots];
  const int nb = K / kQ, KC = q8r_chunk(K), nbc = KC / kQ, nch = K / KC;
  const int r = threadIdx.x >> 5, L = threadIdx.x & 31, F = N >> 1;
  auto row_of = [&](int t) { return SWI ? ((r & 1) ? F : 0) + t * (kRRows / 2) + (r >> 1) : t * kRRows + r; };
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(codes), (short)0, N * K, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(scales), (short)0, N * nb * 4, kRsrcWord3);
  const int e0 = threadIdx.x * E;
  const int nu = nch * ((ntiles - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x);   // units
  auto load_u = [&](RBlocks &B, int u) {
    q8r_load<BPL>(B, rc, rs, row_of((int)blockIdx.x + (u / nch) * (int)gridDim.x), N, K, nb, nbc, u % nch, L);
  };
  ProRegs<E, conv_taps(PRO)> pr;
  pro_load<PRO, E>(p, e0, K, pr);
  RBlocks Ba, Bb;
  load_u(Ba, 0);
  {
    float v[E];
    pro_values<PRO, E>(p, e0, K, pr, red, v);
    float *d = rxs + (size_t)(e0 >> 5) * kRXStride + (e0 & 31);   // E divides 32: one block
#pragma unroll
    for (int i = 0; i < E; i += 4) *reinterpret_cast<float4 *>(d + i) = make_float4(v[i], v[i + 1], v[i + 2], v[i + 3]);
  }
  lds_barrier();
  float yv = 0.0f, best = kAmFloor;
  int bidx = -1;
  // fold chunk cc of tile tt (lane L = 0 of each row holds the partial); the
  // tile's last chunk writes its outputs
  auto step = [&](const RBlocks &B, int tt, int cc) {
    yv = yv + leaf_tree32(q8r_leaf<BPL>(B, rxs, nbc, cc, L));
    if (cc + 1 < nch) return;
    if constexpr (SWI) {
      const float u = bf2f(f2bf(__shfl_down(yv, 32, 64)));   // the up row's sum, from lane 32
      if ((threadIdx.x & 63) == 0) {
        const float a = bf2f(f2bf(yv));
        const float sg = 1.0f / (1.0f + expf_pq(-a));
        reinterpret_cast<uint16_t *>(y)[tt * (kRRows / 2) + (threadIdx.x >> 6)] = f2bf((a * sg) * u);
      }
    } else {
      const int row = tt * kRRows + r;
      if (L == 0 && row < N) {
        if (y_bf16) reinterpret_cast<uint16_t *>(y)[row] = f2bf(yv);
        else reinterpret_cast<float *>(y)[row] = yv;
        float cv;
        int ci;
        am_leaf(yv, row, cv, ci);
        if (am_better(cv, ci, best, bidx)) { best = cv; bidx = ci; }
      }
    }
    yv = 0.0f;
  };
  auto step_u = [&](const RBlocks &B, int u) { step(B, (int)blockIdx.x + (u / nch) * (int)gridDim.x, u % nch); };
  if constexpr (NS == 1) {
    step_u(Ba, 0);
  } else {
    for (int u = 0; u < nu; u += 2) {
      if (u + 1 < nu) load_u(Bb, u + 1);
      step_u(Ba, u);
      if (u + 1 >= nu) break;
      if (u + 2 < nu) load_u(Ba, u + 2);
      step_u(Bb, u + 1);
    }
  }
  if constexpr (!SWI) {
    if (parts != nullptr) {   // uniform: every thread reaches the barrier
      __shared__ float pb[kRRows];
      __shared__ int pi[kRRows];
      if (L == 0) { pb[r] = best; pi[r] = bidx; }
      lds_barrier();
      if (threadIdx.x == 0) {
        for (int i = 1; i < kRRows; i++)
          if (am_better(pb[i], pi[i], best, bidx)) { best = pb[i]; bidx = pi[i]; }
        parts[2 * blockIdx.x] = best;
        parts[2 * blockIdx.x + 1] = __int_as_float(bidx);
      }
    }
  }
}

// (value, index) partials -> the pick in k_argmax's order (am_better); -1
// when no output exceeds kAmFloor.
// With ctr (the engine's replayed decode step): also ids[ctr[0]++] = the id and
// ctr[1]++ (the position).
__global__ __launch_bounds__(1024) void argmax_parts_kernel(const float *__restrict__ parts, int n,
                                                             int32_t *__restrict__ out, int32_t *__restrict__ ids,
                                                             int32_t *__restrict__ ctr) {
  __shared__ float bv[16];
  __shared__ int bi[16];
  float best = kAmFloor;
  int idx = -1;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const float v = parts[2 * i];
    const int j = __float_as_int(parts[2 * i + 1]);
    if (am_better(v, j, best, idx)) { best = v; idx = j; }
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
    const int id = idx;
    *out = id;
    if (ctr != nullptr) {
      ids[ctr[0]] = id;
      ctr[0] += 1;
      ctr[1] += 1;
    }
  }
}

// --------------------------------------------------------- attention mixer
// One workgroup of 8 waves per q head hq (kv head g = hq / G) at T=1, position
// pos (keys lo..pos, lo = pos + 1 - win for a sliding window). Wave w owns the
// splits j0 + w, j0 + w + 8, ... (64 positions each, j0 = lo / 64). Every
// global load a wave needs for its first split is issued before anything
// waits: the step-1 inputs, the gate, then the K and V blocks of its split, 8
// lanes per 128-byte row slice (whole cache lines per load), through buffer
// resources that end at position pos (rows >= pos read zeros, no branch).
//  1. wave 0 norms + ropes q into LDS; wave 1 norms + ropes k, wave 2 rounds
//     v, both into LDS as fp16 bits and (workgroup G*g only) to the cache.
//  2. per split, per 64-dim slice of the head: the K slice goes through LDS
//     so lane p holds key p (s = q.k, one fmaf chain over d ascending), then
//     m, e, l; each V slice goes through the same LDS buffer so lane d runs
//     the fmaf chain over positions for o of dim d (+ 64 per slice).
//  3. wave 0 merges the splits in ascending order, applies the sigmoid gate
//     and writes the head's bf16 output and/or o_proj's Q8_0 blocks.
constexpr int kSplitF = 64;   // positions per attention split
constexpr int kVRow = 64 + 8;  // padded fp16 row of a 64-dim K/V block slice in LDS

// the amax of each 32-lane half of a wave (one Q8_0 block): DPP within
// 16-lane rows, then the row-pair swap
__device__ __forceinline__ float block_amax(float v) {
  float a = fabsf(v);
  a = fmaxf(a, dpp_f<kDppXor1>(a));
  a = fmaxf(a, dpp_f<kDppXor2>(a));
  a = fmaxf(a, dpp_f<kDppHalfMirror>(a));
  a = fmaxf(a, dpp_f<kDppMirror>(a));
  return max_row_pair(a);
}

// One 64-position split j of a q head, by one wave: the K slices go through
// the wave's LDS buffer bw so lane p holds key p (s = q.k, one fmaf chain over
// d ascending), then m, e, l; each V slice goes through the same buffer so
// lane d runs the fmaf chain over positions for o of dim d (+ 64 per slice).
// kr/vr hold the split's K and V blocks (lane l: 16-byte chunk l%8 of rows
// 8i + l/8, slice h), rows at and past pos zero; the row at pos comes from
// kvnew. Writes (o[HD], m, l) to sj (LDS or global).
template <int HD>
__device__ __forceinline__ void split_partial(const v4i (&kr)[HD / 64][8], const v4i (&vr)[HD / 64][8],
                                              const float *qs, const uint16_t *kvnew, uint16_t *bw, float *eww, int pos,
                                              int npos, int lo, int j, int lane, float scale, float *sj) {
  constexpr int E = HD / 64;
  const int lr = lane >> 3, lc = lane & 7;
  const int p0 = j * kSplitF;
  const int pn = npos - p0 < kSplitF ? npos - p0 : kSplitF;
  const int i0 = lo > p0 ? lo - p0 : 0;
  const bool valid = lane >= i0 && lane < pn;
  // K slices -> LDS -> lane p's row (the row at pos from kvnew); one chain over d
  float d = 0.0f;
#pragma unroll
  for (int h = 0; h < E; h++) {
    if (h > 0) {   // the previous slice's reads precede this slice's writes
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
#pragma unroll
    for (int i = 0; i < 8; i++) *reinterpret_cast<v4i *>(bw + (8 * i + lr) * kVRow + lc * 8) = kr[h][i];
    const uint16_t *krow = p0 + lane == pos ? kvnew + 64 * h : bw + lane * kVRow;
    float kf[64];
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const v4i w4 = *reinterpret_cast<const v4i *>(krow + 8 * q);
      const uint32_t kw[4] = {(uint32_t)w4.x, (uint32_t)w4.y, (uint32_t)w4.z, (uint32_t)w4.w};
#pragma unroll
      for (int i = 0; i < 8; i++) kf[8 * q + i] = h2f((uint16_t)(kw[i >> 1] >> (16 * (i & 1))));
    }
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float4 q4 = reinterpret_cast<const float4 *>(qs + 64 * h)[i];
      d = __builtin_fmaf(q4.x, kf[4 * i], d);
      d = __builtin_fmaf(q4.y, kf[4 * i + 1], d);
      d = __builtin_fmaf(q4.z, kf[4 * i + 2], d);
      d = __builtin_fmaf(q4.w, kf[4 * i + 3], d);
    }
  }
  const float sc = valid ? d * scale : -__builtin_inff();
  const float m = wave_max(sc);
  const float e = valid ? expf_pq(sc - m) : 0.0f;
  const float l = wave_pairwise_sum(e);
  eww[lane] = e;
#pragma unroll
  for (int h = 0; h < E; h++) {
    // V slice h -> the same LDS buffer (this wave's earlier reads of it
    // precede it in LDS order); the row at pos from kvnew
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < 8; i++) *reinterpret_cast<v4i *>(bw + (8 * i + lr) * kVRow + lc * 8) = vr[h][i];
    if (pos - p0 < kSplitF && lane < 8)
      *reinterpret_cast<v4i *>(bw + (pos - p0) * kVRow + lane * 8) =
          reinterpret_cast<const v4i *>(kvnew + HD + 64 * h)[lane];
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    // o = sum_p e[p] v[p][64h + lane] (fmaf chain over i0 <= p < pn), 16
    // positions per batch, the next batch's LDS reads issued before this
    // batch's fmafs. Rows past pos read as zeros (the buffer bound) with
    // e = 0, and fmaf(0, +0, o) = o, so the last batch runs whole; rows
    // below i0 (the window's first split) are skipped, a cache row there
    // may hold an fp16 infinity
    auto vchain = [&](auto FULL) {
      float o = 0.0f;
      uint16_t vb[16];
      float4 e4[4];
#pragma unroll
      for (int i = 0; i < 16; i++) vb[i] = bw[i * kVRow + lane];
#pragma unroll
      for (int k = 0; k < 4; k++) e4[k] = reinterpret_cast<const float4 *>(eww)[k];
      for (int b0 = 0; b0 < pn; b0 += 16) {
        const int nb0 = b0 + 16 < kSplitF ? b0 + 16 : b0;
        uint16_t vn[16];
        float4 en[4];
#pragma unroll
        for (int i = 0; i < 16; i++) vn[i] = bw[(nb0 + i) * kVRow + lane];
#pragma unroll
        for (int k = 0; k < 4; k++) en[k] = reinterpret_cast<const float4 *>(eww + nb0)[k];
#pragma unroll
        for (int i = 0; i < 16; i++)
          if (FULL || b0 + i >= i0) {
            const float4 &q = e4[i >> 2];
            const float ei = (i & 3) == 0 ? q.x : (i & 3) == 1 ? q.y : (i & 3) == 2 ? q.z : q.w;
            o = __builtin_fmaf(ei, h2f(vb[i]), o);
          }
#pragma unroll
        for (int i = 0; i < 16; i++) vb[i] = vn[i];
#pragma unroll
        for (int k = 0; k < 4; k++) e4[k] = en[k];
      }
      return o;
    };
    const float o = i0 == 0 ? vchain(std::true_type{}) : vchain(std::false_type{});
    sj[64 * h + lane] = o;
  }
  if (lane == 0) {
    sj[HD] = m;
    sj[HD + 1] = l;
  }
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Merge the splits j0 .. ns-1 of q head hq (partials (o[HD], m, l) at st, PART
// floats apart) by one wave, in ascending order; then the sigmoid gate, the
// bf16 output and/or the Q8_0 blocks of o_proj's input.
template <int HD>
__device__ __forceinline__ void merge_splits(const float *st, int j0, int ns, int lane, uint16_t graw, int hq,
                                             uint16_t *__restrict__ out, int8_t *__restrict__ qx,
                                             float *__restrict__ dx) {
  constexpr int E = HD / 64, PART = HD + 2;
  // M = max m_j; w_j = e^(m_j - M) for 64 splits at a time, one per lane;
  // then L and O as fmaf chains over j ascending (w_j, l_j by v_readlane)
  float M = -__builtin_inff();
  for (int jb = j0; jb < ns; jb += 64)
    M = fmaxf(M, wave_max(jb + lane < ns ? st[(size_t)(jb + lane) * PART + HD] : -__builtin_inff()));
  float L = 0.0f, O[E];
#pragma unroll
  for (int h = 0; h < E; h++) O[h] = 0.0f;
  for (int jb = j0; jb < ns; jb += 64) {
    const int jl = jb + lane < ns ? jb + lane : ns - 1;
    const float w = expf_pq(st[(size_t)jl * PART + HD] - M);
    const float lj = st[(size_t)jl * PART + HD + 1];
    const int n = ns - jb < 64 ? ns - jb : 64;
    for (int b = 0; b < n; b += 8) {
      float oj[8][E];
#pragma unroll
      for (int i = 0; i < 8; i++)
#pragma unroll
        for (int h = 0; h < E; h++) oj[i][h] = st[(size_t)(jb + (b + i < n ? b + i : 0)) * PART + 64 * h + lane];
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int i = 0; i < 8; i++)
        if (b + i < n) {
          const float wi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), b + i));
          L = __builtin_fmaf(__int_as_float(__builtin_amdgcn_readlane(__float_as_int(lj), b + i)), wi, L);
#pragma unroll
          for (int h = 0; h < E; h++) O[h] = __builtin_fmaf(oj[i][h], wi, O[h]);
        }
    }
  }
  const float gs = 1.0f / (1.0f + expf_pq(-bf2f(graw)));
#pragma unroll
  for (int h = 0; h < E; h++) {
    const int dd = hq * HD + 64 * h + lane;
    const uint16_t rb = f2bf(bf2f(f2bf(O[h] / L)) * gs);
    if (out != nullptr) out[dd] = rb;
    if (qx != nullptr) {   // the Q8_0 blocks of o_proj's input (a caller may ask for bf16 only)
      const float v = bf2f(rb);
      const float dq = block_amax(v) / 127.0f;
      qx[dd] = (int8_t)q8_code(Q8Div(dq).div(v));
      if ((lane & 31) == 0) dx[dd / 32] = dq;
    }
  }
}

template <int HD>
__global__ __launch_bounds__(512) void attn_head_kernel(const uint16_t *__restrict__ qkvg, const float *__restrict__ qn,
                                                         const float *__restrict__ kn, const float *__restrict__ cs,
                                                         uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                                                         int pos_arg, const int32_t *__restrict__ pos_dev, int nh,
                                                         int nkv, int rot, int win, float eps, float scale,
                                                         uint16_t *__restrict__ out, int8_t *__restrict__ qx,
                                                         float *__restrict__ dx) {
  constexpr int E = HD / 64, PART = HD + 2;
  extern __shared__ __align__(16) unsigned char smem[];
  float *qs = reinterpret_cast<float *>(smem);                      // [HD] q
  float *ew = qs + HD;                                               // [8 waves][64] e
  uint16_t *kvnew = reinterpret_cast<uint16_t *>(ew + 8 * kSplitF);  // [2][HD] fp16 k, v at pos
  uint16_t *blk = kvnew + 2 * HD;                                    // [8 waves][64][kVRow] K, then V slices
  float *st = reinterpret_cast<float *>(blk + 8 * kSplitF * kVRow);  // [nsplit][HD + 2]
  const int pos = pos_dev != nullptr ? __builtin_amdgcn_readfirstlane(*pos_dev) : pos_arg;
  // workgroups go round-robin over the 8 XCDs (XCD = id % 8): with nh a
  // multiple of 8, XCD x takes q heads x*nh/8 .. +nh/8, so the q heads of a kv
  // group share an L2 (or two) and their K/V blocks come from HBM once per L2
  const int hq = nh % 8 == 0 ? (int)(blockIdx.x % 8) * (nh / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
  const int G = nh / nkv, g = hq / G;
  const bool writer = hq % G == 0;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int kvd = nkv * HD;
  const int npos = pos + 1;
  const int lo = window_lo(npos, win);
  const int j0 = lo / kSplitF, ns = (npos + kSplitF - 1) / kSplitF;
  const int half = rot / 2;
  // step-1 and step-3 inputs: wave 0 q, wave 1 k, others v (valid addresses)
  const int xoff = wave == 0 ? hq * HD : wave == 1 ? nh * HD + g * HD : nh * HD + kvd + g * HD;
  uint16_t xraw[E];
  float wv[E];
#pragma unroll
  for (int e = 0; e < E; e++) {
    xraw[e] = qkvg[xoff + lane + 64 * e];
    wv[e] = (wave == 1 ? kn : qn)[lane + 64 * e];
  }
  const int pair = HD == 64 ? (lane & 31) : lane;
  const __amdgpu_buffer_rsrc_t rcs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(cs), (short)0, (pos + 1) * half * 8, kRsrcWord3);
  const v2i csw = __builtin_amdgcn_raw_buffer_load_b64(rcs, (pos * half + max(0, min(pair, half - 1))) * 8, 0, 0);
  const uint16_t graw = qkvg[nh * HD + 2 * kvd + hq];
  // K, V blocks of split J: slice h, lane l loads 16 B (chunk l%8) of rows 8i + l/8
  const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(kc, (short)0, pos * kvd * 2, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(vc, (short)0, pos * kvd * 2, kRsrcWord3);
  const int lr = lane >> 3, lc = lane & 7;
  v4i kr[E][8], vr[E][8];
  auto load_blocks = [&](int J) {
    const int off = ((J * kSplitF + lr) * kvd + g * HD) * 2 + lc * 16;
#pragma unroll
    for (int h = 0; h < E; h++)
#pragma unroll
      for (int i = 0; i < 8; i++) kr[h][i] = __builtin_amdgcn_raw_buffer_load_b128(rk, off + h * 128 + i * 8 * kvd * 2, 0, 0);
#pragma unroll
    for (int h = 0; h < E; h++)
#pragma unroll
      for (int i = 0; i < 8; i++) vr[h][i] = __builtin_amdgcn_raw_buffer_load_b128(rv, off + h * 128 + i * 8 * kvd * 2, 0, 0);
  };
  __builtin_amdgcn_sched_barrier(0);   // the step-1 inputs' loads first,
  load_blocks(j0 + wave);
  __builtin_amdgcn_sched_barrier(0);   // and every load is issued before anything waits
  // 1. q/k norm + rope, KV write. The empty asm uses the norm weights and
  //    the RoPE pair in every wave, so that their loads stay ahead of the K/V
  //    loads in issue order (a wait for them leaves the K/V loads in flight).
#pragma unroll
  for (int e = 0; e < E; e++) asm volatile("" ::"v"(wv[e]));
  asm volatile("" ::"v"(csw.x), "v"(csw.y));
  float x1[E], r[E];
#pragma unroll
  for (int e = 0; e < E; e++) x1[e] = bf2f(xraw[e]);
  if (wave < 2) norm_rope<HD>(x1, wv, __int_as_float(csw.x), __int_as_float(csw.y), rot, eps, lane, r);
  if (wave == 0) {
#pragma unroll
    for (int e = 0; e < E; e++) qs[lane + 64 * e] = r[e];
  } else if (wave == 1) {
#pragma unroll
    for (int e = 0; e < E; e++) {
      const uint16_t k = f2h(r[e]);
      if (writer) kc[(size_t)pos * kvd + g * HD + lane + 64 * e] = k;
      kvnew[lane + 64 * e] = k;
    }
  } else if (wave == 2) {
#pragma unroll
    for (int e = 0; e < E; e++) {
      const uint16_t v = f2h(x1[e]);
      if (writer) vc[(size_t)pos * kvd + g * HD + lane + 64 * e] = v;
      kvnew[HD + lane + 64 * e] = v;
    }
  }
  lds_barrier();
  // 2. splits
  uint16_t *bw = blk + wave * kSplitF * kVRow;
  for (int j = j0 + wave; j < ns; j += 8) {
    if (j != j0 + wave) load_blocks(j);
    split_partial<HD>(kr, vr, qs, kvnew, bw, ew + wave * kSplitF, pos, npos, lo, j, lane, scale, st + (size_t)j * PART);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
  lds_barrier();
  // 3. merge, gate, outputs
  if (wave == 0) merge_splits<HD>(st, j0, ns, lane, graw, hq, out, qx, dx);
}

// ------------------------------------- attention mixer, head_dim 64 or 128
// The one-launch decode mixer for the shapes attn_head_kernel does not take
// (GQA group 8, or contexts whose splits overflow its LDS): the arithmetic of qk_prep_kernel +
// attn_split_kernel + attn_merge_kernel in one workgroup of 8 waves per q
// head. Waves 0-2 form q (norm + RoPE from the layer's table), k (norm + RoPE,
// fp16, written to the cache by the group's first workgroup) and v; wave w
// then owns the splits j0 + w, j0 + w + 8, ... of the window. Per split lane p
// loads key row p (whole cache lines) and every lane loads its E = HD/64
// adjacent value dims of all 64 positions up front, so a split waits on
// memory about once; the row at pos, which this launch writes, comes from LDS.
// Wave 0 merges the splits in ascending order, gates, and writes the head's
// bf16 output and/or its Q8_0 blocks.
template <int HD>
__device__ __forceinline__ void mixer_norm_rope(const float *x, const float *__restrict__ w,
                                                const float *__restrict__ cs, int pos, int rot, float eps, int lane,
                                                float *r) {
  constexpr int E = HD / 64;
  float wv[E];
#pragma unroll
  for (int e = 0; e < E; e++) wv[e] = w[lane + 64 * e];
  const int half = rot / 2, pair = HD == 64 ? (lane & 31) : lane;
  float c = 0.0f, sn = 0.0f;
  if (pair < half) {
    c = cs[((size_t)pos * half + pair) * 2];
    sn = cs[((size_t)pos * half + pair) * 2 + 1];
  }
  norm_rope<HD>(x, wv, c, sn, rot, eps, lane, r);
}

template <int HD>
__global__ __launch_bounds__(512) void attn_mixer_kernel(const uint16_t *__restrict__ qkvg, const float *__restrict__ qn,
                                                          const float *__restrict__ kn, const float *__restrict__ cs,
                                                          uint16_t *__restrict__ kc, uint16_t *__restrict__ vc,
                                                          int pos_arg, const int32_t *__restrict__ pos_dev, int nh,
                                                          int nkv, int rot, int win, float eps, float scale,
                                                          uint16_t *__restrict__ out, int8_t *__restrict__ qx,
                                                          float *__restrict__ dx) {
  constexpr int E = HD / 64, PART = HD + 2;
  using VT = typename std::conditional<E == 2, uint32_t, uint16_t>::type;   // a lane's E adjacent fp16
  extern __shared__ __align__(16) unsigned char smem[];
  float *qs = reinterpret_cast<float *>(smem);                      // [HD] q
  float *ew = qs + HD;                                               // [8 waves][64] e
  uint16_t *kvnew = reinterpret_cast<uint16_t *>(ew + 8 * kSplitF);  // [2][HD] fp16 k, v at pos
  float *st = reinterpret_cast<float *>(kvnew + 2 * HD);            // [nsplit][HD + 2]
  const int pos = pos_dev != nullptr ? __builtin_amdgcn_readfirstlane(*pos_dev) : pos_arg;
  const int hq = blockIdx.x, G = nh / nkv, g = hq / G;
  const bool writer = hq % G == 0;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int kvd = nkv * HD;
  const int npos = pos + 1;
  const int lo = window_lo(npos, win);
  const int j0 = lo / kSplitF, ns = (npos + kSplitF - 1) / kSplitF;
  // 1. q, k (norm + RoPE) and v of position pos
  if (wave < 3) {
    const int base = wave == 0 ? hq * HD : wave == 1 ? nh * HD + g * HD : nh * HD + kvd + g * HD;
    float x[E];
#pragma unroll
    for (int e = 0; e < E; e++) x[e] = bf2f(qkvg[base + lane + 64 * e]);
    if (wave == 2) {
#pragma unroll
      for (int e = 0; e < E; e++) {
        const uint16_t v = f2h(x[e]);
        kvnew[HD + lane + 64 * e] = v;
        if (writer) vc[(size_t)pos * kvd + g * HD + lane + 64 * e] = v;
      }
    } else {
      float r[E];
      mixer_norm_rope<HD>(x, wave == 0 ? qn : kn, cs, pos, rot, eps, lane, r);
#pragma unroll
      for (int e = 0; e < E; e++) {
        if (wave == 0) {
          qs[lane + 64 * e] = r[e];
        } else {
          const uint16_t k = f2h(r[e]);
          kvnew[lane + 64 * e] = k;
          if (writer) kc[(size_t)pos * kvd + g * HD + lane + 64 * e] = k;
        }
      }
    }
  }
  __syncthreads();
  // 2. the window's splits
  float *eww = ew + wave * kSplitF;
  for (int j = j0 + wave; j < ns; j += 8) {
    const int p0 = j * kSplitF;
    const int pn = npos - p0 < kSplitF ? npos - p0 : kSplitF;
    const int i0 = lo > p0 ? lo - p0 : 0;
    const bool valid = lane >= i0 && lane < pn;
    VT vr[kSplitF];
    {
      const VT *vb = reinterpret_cast<const VT *>(vc + (size_t)p0 * kvd + g * HD) + lane;
#pragma unroll
      for (int p = 0; p < kSplitF; p++)
        vr[p] = p >= i0 && p < pn && p0 + p != pos ? vb[(size_t)p * (kvd / E)] : (VT)0;
    }
    uint4 k8[HD / 8];
    {
      const bool from_cache = valid && p0 + lane != pos;
      const uint4 *kr = from_cache ? reinterpret_cast<const uint4 *>(kc + (size_t)(p0 + lane) * kvd + g * HD)
                                   : reinterpret_cast<const uint4 *>(kvnew);
#pragma unroll
      for (int i = 0; i < HD / 8; i++) k8[i] = kr[i];
    }
    float d = 0.0f;
#pragma unroll
    for (int i = 0; i < HD / 8; i++) {
      const uint32_t kw[4] = {k8[i].x, k8[i].y, k8[i].z, k8[i].w};
#pragma unroll
      for (int u = 0; u < 8; u++) d = __builtin_fmaf(qs[8 * i + u], h2f((uint16_t)(kw[u >> 1] >> (16 * (u & 1)))), d);
    }
    const float sc = valid ? d * scale : -__builtin_inff();
    const float m = wave_max(sc);
    const float e = valid ? expf_pq(sc - m) : 0.0f;
    const float l = wave_pairwise_sum(e);
    eww[lane] = e;
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
    float o[E];
#pragma unroll
    for (int k = 0; k < E; k++) o[k] = 0.0f;
    const VT vpos = reinterpret_cast<const VT *>(kvnew + HD)[lane];
#pragma unroll
    for (int p = 0; p < kSplitF; p++)
      if (p >= i0 && p < pn) {
        const uint32_t bits = (uint32_t)(p0 + p == pos ? vpos : vr[p]);
        const float ep = eww[p];
#pragma unroll
        for (int k = 0; k < E; k++) o[k] = __builtin_fmaf(ep, h2f((uint16_t)(bits >> (16 * k))), o[k]);
      }
    float *sj = st + (size_t)j * PART;
#pragma unroll
    for (int k = 0; k < E; k++) sj[E * lane + k] = o[k];
    if (lane == 0) {
      sj[HD] = m;
      sj[HD + 1] = l;
    }
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }
  __syncthreads();
  // 3. ordered merge, gate, outputs
  if (wave == 0) {
    float M = -__builtin_inff();
    for (int j = j0; j < ns; j++) M = fmaxf(M, st[(size_t)j * PART + HD]);
    float L = 0.0f, O[E];
#pragma unroll
    for (int k = 0; k < E; k++) O[k] = 0.0f;
    for (int j = j0; j < ns; j++) {
      const float w = expf_pq(st[(size_t)j * PART + HD] - M);
      L = __builtin_fmaf(st[(size_t)j * PART + HD + 1], w, L);
#pragma unroll
      for (int k = 0; k < E; k++) O[k] = __builtin_fmaf(st[(size_t)j * PART + lane + 64 * k], w, O[k]);
    }
    const float gs = 1.0f / (1.0f + expf_pq(-bf2f(qkvg[nh * HD + 2 * kvd + hq])));
#pragma unroll
    for (int k = 0; k < E; k++) {
      const int dd = hq * HD + lane + 64 * k;
      const uint16_t rb = f2bf(bf2f(f2bf(O[k] / L)) * gs);
      if (out != nullptr) out[dd] = rb;
      if (qx != nullptr) {
        const float v = bf2f(rb);
        float a = fabsf(v);
#pragma unroll
        for (int o = 1; o < 32; o <<= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
        const float dq = a / 127.0f;
        qx[dd] = (int8_t)q8_code(Q8Div(dq).div(v));
        if ((lane & 31) == 0) dx[dd / 32] = dq;
      }
    }
  }
}

}  // namespace pq

using namespace pq;

static int fused_rows(int N, int K);

extern "C" int pq_q8_gemv_parts(int N, int K) {
  if (N <= 0 || K <= 0 || K % kQ) return 0;
  return ntiles(N) * (64 / fused_rows(N, K));
}

// Argument checks shared by the fused GEMV entry points (out: y or qx).
static int check_fused_args(const int8_t *pcodes, const uint16_t *pscales, const pq_gemv_prologue *pro,
                            const void *out, int N, int K, const char *who) {
  PQ_REQUIRE(pcodes && pscales && pro && out, PQ_ERR_ARG, "%s: null pointer", who);
  PQ_REQUIRE(N > 0 && K >= 1024 && K <= 8192 && (K & (K - 1)) == 0, PQ_ERR_ARG,
             "%s: N=%d K=%d (K a power of two, 1024..8192)", who, N, K);
  PQ_REQUIRE(aligned(pcodes, 16) && aligned(pscales, 16), PQ_ERR_ALIGN, "%s: packed weights alignment", who);
  const pq_gemv_prologue &p = *pro;
  switch (p.kind) {
    case PQ_PRO_Q8:
      PQ_REQUIRE(p.qx && p.dx && aligned(p.qx, 16), PQ_ERR_ARG, "%s: Q8 prologue needs aligned qx, dx", who);
      break;
    case PQ_PRO_RESNORM:
      PQ_REQUIRE(p.h && p.x_in && p.x_out && p.w0 && p.w1 && p.x_in != p.x_out, PQ_ERR_ARG,
                 "%s: RESNORM needs h, x_in, x_out (distinct), w0, w1", who);
      break;
    case PQ_PRO_NORM:
      PQ_REQUIRE(p.x_in && p.w0, PQ_ERR_ARG, "%s: NORM needs x_in, w0", who);
      break;
    case PQ_PRO_EMBED:
      PQ_REQUIRE(p.tok && p.emb_pc && p.emb_ps && p.x_out && p.w0 && p.vocab > 0, PQ_ERR_ARG,
                 "%s: EMBED needs tok, the table, x_out, w0", who);
      break;
    case PQ_PRO_SILU:
      PQ_REQUIRE(p.gu, PQ_ERR_ARG, "%s: SILU needs gu", who);
      break;
    case PQ_PRO_F32:
      PQ_REQUIRE(p.xf && aligned(p.xf, 16), PQ_ERR_ARG, "%s: F32 prologue needs 16-byte aligned xf", who);
      break;
    case PQ_PRO_CONV:
      PQ_REQUIRE(p.bcx && p.ring_in && p.ring_out && p.taps && p.ring_in != p.ring_out &&
                     (p.ntaps == 3 || p.ntaps == 7) && aligned(p.taps, 16),
                 PQ_ERR_ARG, "%s: CONV needs bcx, taps, distinct ring_in / ring_out, ntaps 3 or 7", who);
      break;
    default:
      return fail(PQ_ERR_ARG, "%s: prologue kind %d", who, p.kind);
  }
  return PQ_OK;
}

// Rows per workgroup of a fused GEMV: the largest R of 64, 32, 16, 8 that
// still gives at least 192 workgroups for K <= 4096 (256 for longer rows).
// Every workgroup repeats the prologue, so fewer and longer workgroups win
// until too few are left to keep HBM busy. Measured per decode launch at
// K = 2048: conv in_proj 6144 rows with the RESNORM prologue 5.0 us at R = 32
// (192 workgroups) against 5.7 at R = 16 and 6.1 at R = 64; q|k|v|gate 3136
// rows 4.5 us at R = 16 against 5.5 at R = 8; 2048-row shapes equal at R = 8
// and 16; at K = 8192 (down) R = 8 is fastest. PQ_GEMV_R forces R,
// PQ_FUSED_MINWG the workgroup target.
static int fused_rows(int N, int K) {
  static const int fR = env_int("PQ_GEMV_R"), fM = env_int("PQ_FUSED_MINWG");
  if (fR == 8 || fR == 16 || fR == 32 || fR == 64) return fR;
  const int target = fM > 0 ? fM : (K <= 4096 ? 192 : 256);
  const long long nt = ntiles(N);
  int R = 64;
  while (R > 8 && nt * (64 / R) < target) R >>= 1;
  return R;
}

// Launch shape of a fused GEMV: W waves (4 or 8; fewer waves leave each
// thread a longer prologue and measured slower, even where a wave has no chunk
// of its own and only issues loads that read nothing), enough to give every
// chunk slot of the R-row slice a lane, and E = K/(64W) prologue elements per
// thread, 4..16.
static int fused_waves(int R, int K) {
  static const int fW = env_int("PQ_FUSED_W");   // launch-shape override for sweeps (4 or 8)
  const int C = 64 / R;
  const int need = (nchunks(K) + C - 1) / C;
  int W = need > 4 ? 8 : 4;
  if (fW == 4 || fW == 8) W = fW;
  if (K / (64 * W) > 16) W = 8;
  if (K / (64 * W) < 4) W = 4;
  return W;
}

template <int R, int PRO, int E>
static void launch_fused_t(dim3 grid, dim3 block, size_t lds, hipStream_t st, const int8_t *pcodes,
                           const uint16_t *pscales, const pq_gemv_prologue &p, void *y, int yb, int N, int K,
                           float *parts, int8_t *qo, float *dqo) {
  launch(q8_gemv_fused_kernel<R, PRO, E>, grid, block, lds, st, pcodes, pscales, p, y, yb, N, K, parts, qo, dqo);
}

template <int R, int PRO>
static void launch_fused_e(int E, dim3 grid, dim3 block, size_t lds, hipStream_t st, const int8_t *pcodes,
                           const uint16_t *pscales, const pq_gemv_prologue &p, void *y, int yb, int N, int K,
                           float *parts, int8_t *qo, float *dqo) {
  switch (E) {
    case 4: launch_fused_t<R, PRO, 4>(grid, block, lds, st, pcodes, pscales, p, y, yb, N, K, parts, qo, dqo); break;
    case 8: launch_fused_t<R, PRO, 8>(grid, block, lds, st, pcodes, pscales, p, y, yb, N, K, parts, qo, dqo); break;
    default: launch_fused_t<R, PRO, 16>(grid, block, lds, st, pcodes, pscales, p, y, yb, N, K, parts, qo, dqo); break;
  }
}

template <int PRO>
static void launch_fused_r(int R, int E, dim3 grid, dim3 block, size_t lds, hipStream_t st, const int8_t *pcodes,
                           const uint16_t *pscales, const pq_gemv_prologue &p, void *y, int yb, int N, int K,
                           float *parts, int8_t *qo, float *dqo) {
  switch (R) {
    case 64: launch_fused_e<64, PRO>(E, grid, block, lds, st, pcodes, pscales, p, y, yb, N, K, parts, qo, dqo); break;
    case 32: launch_fused_e<32, PRO>(E, grid, block, lds, st, pcodes, pscales, p, y, yb, N, K, parts, qo, dqo); break;
    case 16: launch_fused_e<16, PRO>(E, grid, block, lds, st, pcodes, pscales, p, y, yb, N, K, parts, qo, dqo); break;
    default: launch_fused_e<8, PRO>(E, grid, block, lds, st, pcodes, pscales, p, y, yb, N, K, parts, qo, dqo); break;
  }
}

static int launch_fused(const int8_t *pcodes, const uint16_t *pscales, const pq_gemv_prologue &p, void *y, int yb,
                        int N, int K, float *parts, int8_t *qo, float *dqo, int R, hipStream_t st, const char *who) {
  const int C = 64 / R;
  const int W = fused_waves(R, K);
  const int E = K / (64 * W);
  PQ_REQUIRE(E >= 4 && E <= 16 && 64 * W * E == K, PQ_ERR_ARG, "%s: no launch shape for K=%d", who, K);
  const int nch = nchunks(K), nb = K / kQ;
  const size_t lds = (size_t)W * 64 * 4 + (size_t)nch * kXStride + (size_t)nb * 4;
  const dim3 grid((unsigned)(ntiles(N) * C)), block(64 * W);
#define PQ_FUSED(PP) \
  launch_fused_r<PP>(R, E, grid, block, lds, st, pcodes, pscales, p, y, yb, N, K, parts, qo, dqo)
  switch (p.kind) {
    case PQ_PRO_Q8: PQ_FUSED(PQ_PRO_Q8); break;
    case PQ_PRO_RESNORM: PQ_FUSED(PQ_PRO_RESNORM); break;
    case PQ_PRO_NORM: PQ_FUSED(PQ_PRO_NORM); break;
    case PQ_PRO_EMBED: PQ_FUSED(PQ_PRO_EMBED); break;
    case PQ_PRO_SILU: PQ_FUSED(PQ_PRO_SILU); break;
    case PQ_PRO_F32: PQ_FUSED(PQ_PRO_F32); break;
    default:
      if (p.ntaps == 7) PQ_FUSED(kProConv7);
      else PQ_FUSED(PQ_PRO_CONV);
      break;
  }
#undef PQ_FUSED
  return check_launch(who);
}

extern "C" int pq_q8_gemv_fused(const int8_t *pcodes, const uint16_t *pscales, const pq_gemv_prologue *pro, void *y,
                                int y_dtype, int N, int K, float *argmax_parts, void *stream) {
  const int rc = check_fused_args(pcodes, pscales, pro, y, N, K, "pq_q8_gemv_fused");
  if (rc) return rc;
  PQ_REQUIRE(y_dtype == PQ_DTYPE_F32 || y_dtype == PQ_DTYPE_BF16, PQ_ERR_ARG, "pq_q8_gemv_fused: y_dtype %d", y_dtype);
  const pq_gemv_prologue &p = *pro;
  return launch_fused(pcodes, pscales, p, y, y_dtype == PQ_DTYPE_BF16 ? 1 : 0, N, K, argmax_parts, nullptr, nullptr,
                      fused_rows(N, K), as_stream(stream), "pq_q8_gemv_fused");
}

extern "C" int pq_q8_gemv_fused_swiglu(const int8_t *pcodes, const uint16_t *pscales, const pq_gemv_prologue *pro,
                                       int8_t *qx, float *dx, int F, int K, void *stream) {
  PQ_REQUIRE(pro && qx && dx, PQ_ERR_ARG, "pq_q8_gemv_fused_swiglu: null pointer");
  PQ_REQUIRE(F > 0 && F % 32 == 0, PQ_ERR_ARG, "pq_q8_gemv_fused_swiglu: F=%d (a multiple of 32)", F);
  PQ_REQUIRE(aligned(dx, 4), PQ_ERR_ALIGN, "pq_q8_gemv_fused_swiglu: dx alignment");
  const int rc = check_fused_args(pcodes, pscales, pro, qx, 2 * F, K, "pq_q8_gemv_fused_swiglu");
  if (rc) return rc;
  return launch_fused(pcodes, pscales, *pro, nullptr, 0, 2 * F, K, nullptr, qx, dx, 64, as_stream(stream),
                      "pq_q8_gemv_fused_swiglu");
}

// Workgroups of the fused reference-numerics GEMV: ntiles row tiles over at
// most 512 workgroups (two per CU), so a large N pays its prologue once per
// workgroup, not once per 8 rows (512 measured faster than 1024 and 2048 for
// the 16384- and 65536-row shapes).
static int q8r_fused_grid(int ntiles) {
  static const int cap = [] {
    const char *e = getenv("PQ_Q8RF_GRID");
    const int v = e ? atoi(e) : 0;
    return v >= 64 ? v : 512;
  }();
  return std::min(ntiles, cap);
}

template <int PRO, bool SWI>
static void launch_q8r_fused(int K, int ntiles, size_t lds, hipStream_t st, const int8_t *codes, const float *scales,
                             const pq_gemv_prologue &p, void *y, int yb, int N, float *parts) {
  const int G = q8r_fused_grid(ntiles);
  const bool one = G == ntiles && K <= 2048;   // one unit per workgroup
  const dim3 grid((unsigned)G), blk(kRThreads);
  // K = 256 E; chunks of 2048 (one for K <= 2048): BPL = 1 at K = 1024, else 2
#define PQ_Q8RF(BPL, E, NS) \
  launch(q8r_gemv_fused_kernel<BPL, PRO, E, NS, SWI>, grid, blk, lds, st, codes, scales, p, y, yb, N, K, ntiles, \
         parts)
#define PQ_Q8RF_W(BPL, E)        \
  do {                           \
    if (one) PQ_Q8RF(BPL, E, 1); \
    else PQ_Q8RF(BPL, E, 2);     \
  } while (0)
  switch (K) {
    case 1024: PQ_Q8RF_W(1, 4); break;
    case 2048: PQ_Q8RF_W(2, 8); break;
    case 4096: PQ_Q8RF(2, 16, 2); break;
    default:
      if constexpr (pro_base(PRO) != PQ_PRO_CONV) PQ_Q8RF(2, 32, 2);
      break;
  }
#undef PQ_Q8RF_W
#undef PQ_Q8RF
}

template <bool SWI>
static int q8r_fused_entry(const int8_t *codes, const float *scales, const pq_gemv_prologue *pro, void *y, int y_dtype,
                           int N, int K, float *parts, void *stream, const char *who) {
  PQ_REQUIRE(codes && scales && pro && y, PQ_ERR_ARG, "%s: null pointer", who);
  PQ_REQUIRE(N > 0 && (K == 1024 || K == 2048 || K == 4096 || K == 8192), PQ_ERR_ARG,
             "%s: N=%d K=%d (K 1024, 2048, 4096 or 8192)", who, N, K);
  PQ_REQUIRE((long long)N * K < (1ll << 31), PQ_ERR_ARG, "%s: N=%d K=%d too large", who, N, K);
  PQ_REQUIRE(aligned(codes, 16) && aligned(scales, 16), PQ_ERR_ALIGN, "%s: codes, scales alignment", who);
  PQ_REQUIRE(y_dtype == PQ_DTYPE_F32 || y_dtype == PQ_DTYPE_BF16, PQ_ERR_ARG, "%s: y_dtype %d", who, y_dtype);
  const pq_gemv_prologue &p = *pro;
  PQ_REQUIRE(p.kind == PQ_PRO_RESNORM || p.kind == PQ_PRO_NORM ||
                 (!SWI && (p.kind == PQ_PRO_SILU || p.kind == PQ_PRO_CONV || p.kind == PQ_PRO_EMBED)),
             PQ_ERR_ARG, "%s: prologue kind %d (RESNORM, NORM%s)", who, p.kind, SWI ? "" : ", SILU, CONV or EMBED");
  PQ_REQUIRE(p.kind != PQ_PRO_CONV || K <= 4096, PQ_ERR_ARG, "%s: the CONV prologue takes K <= 4096", who);
  if (p.kind == PQ_PRO_EMBED) {   // the row-major table (emb_pc codes, emb_sf fp32 scales)
    PQ_REQUIRE(p.tok && p.emb_pc && p.emb_sf && p.x_out && p.w0 && p.vocab > 0 && aligned(p.emb_pc, 4), PQ_ERR_ARG,
               "%s: EMBED needs tok, emb_pc (4-byte aligned), emb_sf, x_out, w0 and vocab", who);
  } else {
    const int rc = check_fused_args(codes, reinterpret_cast<const uint16_t *>(scales), pro, y, N, K, who);
    if (rc) return rc;
  }
  const size_t lds = (size_t)(K / kQ) * kRXStride * sizeof(float);
  const int ntiles = SWI ? N / kRRows : (N + kRRows - 1) / kRRows;
  const int yb = y_dtype == PQ_DTYPE_BF16 ? 1 : 0;
  hipStream_t st = as_stream(stream);
  switch (p.kind) {
    case PQ_PRO_RESNORM: launch_q8r_fused<PQ_PRO_RESNORM, SWI>(K, ntiles, lds, st, codes, scales, p, y, yb, N, parts); break;
    case PQ_PRO_NORM: launch_q8r_fused<PQ_PRO_NORM, SWI>(K, ntiles, lds, st, codes, scales, p, y, yb, N, parts); break;
    default:
      if constexpr (!SWI) {
        if (p.kind == PQ_PRO_EMBED) launch_q8r_fused<kProEmbedR, false>(K, ntiles, lds, st, codes, scales, p, y, yb, N, parts);
        else if (p.kind == PQ_PRO_SILU) launch_q8r_fused<PQ_PRO_SILU, false>(K, ntiles, lds, st, codes, scales, p, y, yb, N, parts);
        else if (p.ntaps == 7) launch_q8r_fused<kProConv7, false>(K, ntiles, lds, st, codes, scales, p, y, yb, N, parts);
        else launch_q8r_fused<PQ_PRO_CONV, false>(K, ntiles, lds, st, codes, scales, p, y, yb, N, parts);
      }
      break;
  }
  return check_launch(who);
}

extern "C" int pq_q8r_gemv_parts(int N) { return N > 0 ? q8r_fused_grid((N + kRRows - 1) / kRRows) : 0; }

extern "C" int pq_q8r_gemv_fused(const int8_t *codes, const float *scales, const pq_gemv_prologue *pro, void *y,
                                 int y_dtype, int N, int K, float *argmax_parts, void *stream) {
  return q8r_fused_entry<false>(codes, scales, pro, y, y_dtype, N, K, argmax_parts, stream, "pq_q8r_gemv_fused");
}

extern "C" int pq_q8r_gemv_fused_swiglu(const int8_t *codes, const float *scales, const pq_gemv_prologue *pro,
                                        uint16_t *y, int F, int K, void *stream) {
  PQ_REQUIRE(F > 0 && F % (kRRows / 2) == 0, PQ_ERR_ARG, "pq_q8r_gemv_fused_swiglu: F=%d (a multiple of 4)", F);
  return q8r_fused_entry<true>(codes, scales, pro, y, PQ_DTYPE_BF16, 2 * F, K, nullptr, stream,
                               "pq_q8r_gemv_fused_swiglu");
}

extern "C" int pq_argmax_parts(const float *parts, int nparts, int32_t *out, void *stream) {
  PQ_REQUIRE(parts && out && nparts > 0, PQ_ERR_ARG, "pq_argmax_parts: nparts=%d", nparts);
  launch(argmax_parts_kernel, dim3(1), dim3(1024), 0, as_stream(stream), parts, nparts, out, nullptr, nullptr);
  return check_launch("pq_argmax_parts");
}

namespace pq {
int argmax_parts_step(const float *parts, int nparts, int32_t *out, int32_t *ids, int32_t *ctr, hipStream_t st) {
  PQ_REQUIRE(parts && out && ids && ctr && nparts > 0, PQ_ERR_ARG, "argmax_parts_step: bad arguments");
  launch(argmax_parts_kernel, dim3(1), dim3(1024), 0, st, parts, nparts, out, ids, ctr);
  return check_launch("argmax_parts_step");
}
}  // namespace pq

static int attn_layer(const uint16_t *qkvg, const float *q_norm, const float *k_norm, const float *rope_cs,
                      uint16_t *kcache, uint16_t *vcache, int pos, const int32_t *pos_dev, int ctx, int nh, int nkv,
                      int hd, int rot, int win, float eps, float scale, uint16_t *out, int8_t *qx, float *dx,
                      hipStream_t st) {
  PQ_REQUIRE(qkvg && q_norm && k_norm && rope_cs && kcache && vcache && (qx || out) && (!qx || dx), PQ_ERR_ARG,
             "pq_attn_layer_decode: null pointer");
  PQ_REQUIRE((hd == 64 || hd == 128) && nh > 0 && nkv > 0 && nh % nkv == 0 && pos >= 0 && rot >= 0 && rot <= hd &&
                 win >= 0,
             PQ_ERR_ARG, "pq_attn_layer_decode: hd=%d nh=%d nkv=%d pos=%d win=%d", hd, nh, nkv, pos, win);
  PQ_REQUIRE(aligned(kcache, 16) && aligned(vcache, 16), PQ_ERR_ALIGN, "pq_attn_layer_decode: cache alignment");
  const int G = nh / nkv;
  const int ns = (ctx + kSplitF - 1) / kSplitF;   // LDS for the splits of positions 0..ctx-1
  if (G == 1 || G == 2 || G == 4) {
    // the K/V blocks pass through LDS (attn_head_kernel)
    const size_t lds = ((size_t)hd + 8 * (size_t)kSplitF + (size_t)ns * (hd + 2)) * 4 +
                       (2 * (size_t)hd + 8 * (size_t)kSplitF * kVRow) * 2;
    if (lds <= kMaxLds) {
      if (hd == 64)
        launch(attn_head_kernel<64>, dim3(nh), dim3(512), lds, st, qkvg, q_norm, k_norm, rope_cs, kcache, vcache, pos,
               pos_dev, nh, nkv, rot, win, eps, scale, out, qx, dx);
      else
        launch(attn_head_kernel<128>, dim3(nh), dim3(512), lds, st, qkvg, q_norm, k_norm, rope_cs, kcache, vcache,
               pos, pos_dev, nh, nkv, rot, win, eps, scale, out, qx, dx);
      return check_launch("pq_attn_layer_decode");
    }
  }
  const size_t lds = ((size_t)hd + 8 * (size_t)kSplitF + (size_t)ns * (hd + 2)) * 4 + 2 * (size_t)hd * 2;
  PQ_REQUIRE(lds <= kMaxLds, PQ_ERR_ARG, "pq_attn_layer_decode: %d positions need %zu B of LDS", ctx, lds);
  if (hd == 64)
    launch(attn_mixer_kernel<64>, dim3(nh), dim3(512), lds, st, qkvg, q_norm, k_norm, rope_cs, kcache, vcache, pos,
           pos_dev, nh, nkv, rot, win, eps, scale, out, qx, dx);
  else
    launch(attn_mixer_kernel<128>, dim3(nh), dim3(512), lds, st, qkvg, q_norm, k_norm, rope_cs, kcache, vcache, pos,
           pos_dev, nh, nkv, rot, win, eps, scale, out, qx, dx);
  return check_launch("pq_attn_layer_decode");
}

extern "C" int pq_attn_layer_decode(const uint16_t *qkvg, const float *q_norm, const float *k_norm,
                                    const float *rope_cs, uint16_t *kcache, uint16_t *vcache, int pos, int nh, int nkv,
                                    int hd, int rot, int win, float eps, float scale, uint16_t *out, int8_t *qx,
                                    float *dx, void *stream) {
  return attn_layer(qkvg, q_norm, k_norm, rope_cs, kcache, vcache, pos, nullptr, pos + 1, nh, nkv, hd, rot, win, eps,
                    scale, out, qx, dx, as_stream(stream));
}

namespace pq {
int attn_layer_decode_dev(const uint16_t *qkvg, const float *q_norm, const float *k_norm, const float *rope_cs,
                          uint16_t *kcache, uint16_t *vcache, const int32_t *pos_dev, int ctx, int nh, int nkv, int hd,
                          int rot, int win, float eps, float scale, uint16_t *out, int8_t *qx, float *dx,
                          hipStream_t st) {
  PQ_REQUIRE(pos_dev && ctx > 0, PQ_ERR_ARG, "attn_layer_decode_dev: bad arguments");
  return attn_layer(qkvg, q_norm, k_norm, rope_cs, kcache, vcache, 0, pos_dev, ctx, nh, nkv, hd, rot, win, eps, scale,
                    out, qx, dx, st);
}
}  // namespace pq
