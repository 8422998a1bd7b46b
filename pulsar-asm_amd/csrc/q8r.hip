// q8r.hip -- the reference's own Q8_0 GEMV numerics (R2) on gfx950.
//
// The arithmetic of q8_partial<bf16, FMA=1> + k_combine_bf / k_combine_f
// (lfm3_nanode.cu:222-374), as gemv / gemv_f call them (1916-1966,
// 3634-3663), on the reference's untiled data: codes int8 [N][K] row-major and
// one fp32 scale per 32-block [N][K/32] (the .lfm3q8 tensors), x bf16 [T][K]
// position-first, y [T][N] bf16 or fp32. Per output (row r, position t):
//   chunks of KC = 2048 of K (all of K when K is not a multiple of 2048);
//   in each chunk, leaf L = 0..31 folds blocks L, L+32, ... ascending:
//     dot = fmaf((float)c_j, x_j, dot) over the block's 32 codes, from 0,
//     acc = fmaf(s_b, dot, acc), from 0;
//   the chunk partial is the shfl_down tree over the leaves (offsets 16, 8,
//   4, 2, 1: v_i = v_i + v_{i+o});
//   y = ((0 + p_0) + p_1) + ... over the chunks; out = bf16(y) or y.
//
// As in the reference, 32 lanes own a row and lane L owns leaf L, so a row's
// lanes read 32 consecutive blocks (1 KB of whole cache lines) per load. Two
// rows per wave, 8 rows per workgroup. x is staged once per workgroup as
// fp32 in LDS with each 32-element block padded to 36 floats, so the 16-byte
// reads of any 8 consecutive lanes cover all 32 banks. A lane's weight loads
// for a chunk are issued before the previous chunk's arithmetic.
#include <algorithm>

#include "pq_device.h"
#include "pq_host.h"
#include "q8_common.h"
#include "q8r_common.h"

namespace pq {

// BPL = blocks per leaf per chunk (ceil(chunk blocks / 32)); MC: K holds
// several chunks (a second block set in flight; with one chunk the kernel
// keeps the registers, and the occupancy, of one).
template <int BPL, bool MC>
__global__ __launch_bounds__(kRThreads) void q8r_gemv_kernel(const int8_t *__restrict__ codes,
                                                           const float *__restrict__ scales,
                                                           const uint16_t *__restrict__ x, void *__restrict__ y,
                                                           int y_bf16, int N, int K) {
  extern __shared__ __align__(16) float xs[];   // [nb][kRXStride]
  const int t = blockIdx.y;
  const int nb = K / kQ, KC = q8r_chunk(K), nbc = KC / kQ, nch = K / KC;
  const int row = blockIdx.x * kRRows + (threadIdx.x >> 5);
  const int L = threadIdx.x & 31;
  // wave-uniform resources over the whole tensors; a row past N reads at an
  // offset past them
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(codes), (short)0, N * K, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(scales), (short)0, N * nb * 4, kRsrcWord3);
  RBlocks Ba, Bb;
  q8r_load<BPL>(Ba, rc, rs, row, N, K, nb, nbc, 0, L);
  // x of position t: 8 bf16 per thread per step, widened into the padded blocks
  const uint16_t *xt = x + (size_t)t * K;
  for (int e = threadIdx.x * 8; e < K; e += kRThreads * 8) {
    const uint4 u = *reinterpret_cast<const uint4 *>(xt + e);
    const uint32_t v[4] = {u.x, u.y, u.z, u.w};
    float f[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      f[2 * k] = __uint_as_float(v[k] << 16);
      f[2 * k + 1] = __uint_as_float(v[k] & 0xffff0000u);
    }
    float *d = xs + (size_t)(e >> 5) * kRXStride + (e & 31);
    *reinterpret_cast<float4 *>(d) = make_float4(f[0], f[1], f[2], f[3]);
    *reinterpret_cast<float4 *>(d + 4) = make_float4(f[4], f[5], f[6], f[7]);
  }
  __syncthreads();
  // chunks in order, the next chunk's blocks in flight during this one's
  // arithmetic; the two block sets alternate by name (a register copy of a
  // set still being loaded would wait for its loads)
  float yv = 0.0f;
  auto chunk = [&](const RBlocks &B, int c) {
    const float acc = leaf_tree32(q8r_leaf<BPL>(B, xs, nbc, c, L));
    yv = yv + acc;   // lane L = 0 holds the chunk partial
  };
  if constexpr (!MC) {
    chunk(Ba, 0);
  } else {
    for (int c = 0; c < nch; c += 2) {
      if (c + 1 < nch) q8r_load<BPL>(Bb, rc, rs, row, N, K, nb, nbc, c + 1, L);
      chunk(Ba, c);
      if (c + 1 >= nch) break;
      if (c + 2 < nch) q8r_load<BPL>(Ba, rc, rs, row, N, K, nb, nbc, c + 2, L);
      chunk(Bb, c + 1);
    }
  }
  if (L == 0 && row < N) {
    if (y_bf16) reinterpret_cast<uint16_t *>(y)[(size_t)t * N + row] = f2bf(yv);
    else reinterpret_cast<float *>(y)[(size_t)t * N + row] = yv;
  }
}

// q8r_gemv_kernel for rows of several 2048-wide chunks when N alone gives too
// few workgroups (down, K = 8192: N/8 workgroups of one CU each): CW half-waves
// per row, half-wave g taking chunks g, g + CW, ... (the next one loading while
// this one folds), each chunk's partial (lane 0 after the tree) into LDS; then
// one thread per row adds them in chunk order from 0, y = ((0 + p0) + p1) + ...
// as the single-walker kernel does. x is staged once per 8 rows as there.
template <int CW>
__global__ __launch_bounds__(kRThreads * CW) void q8r_gemv_kc_kernel(const int8_t *__restrict__ codes,
                                                                    const float *__restrict__ scales,
                                                                    const uint16_t *__restrict__ x,
                                                                    void *__restrict__ y, int y_bf16, int N, int K) {
  constexpr int BPL = 2;   // 2048-wide chunks: 64 blocks over 32 lanes
  extern __shared__ __align__(16) float xs[];   // [nb][kRXStride]
  __shared__ float pp[kRRows][kRMaxChunks];
  const int t = blockIdx.y;
  const int nb = K / kQ, nbc = 2048 / kQ, nch = K / 2048;
  const int hw = threadIdx.x >> 5, L = threadIdx.x & 31, r = hw / CW, g = hw % CW;
  const int row = blockIdx.x * kRRows + r;
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(codes), (short)0, N * K, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(scales), (short)0, N * nb * 4, kRsrcWord3);
  RBlocks Ba, Bb;
  q8r_load<BPL>(Ba, rc, rs, row, N, K, nb, nbc, g, L);
  const uint16_t *xt = x + (size_t)t * K;
  for (int e = threadIdx.x * 8; e < K; e += kRThreads * CW * 8) {
    const uint4 u = *reinterpret_cast<const uint4 *>(xt + e);
    const uint32_t v[4] = {u.x, u.y, u.z, u.w};
    float f[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      f[2 * k] = __uint_as_float(v[k] << 16);
      f[2 * k + 1] = __uint_as_float(v[k] & 0xffff0000u);
    }
    float *d = xs + (size_t)(e >> 5) * kRXStride + (e & 31);
    *reinterpret_cast<float4 *>(d) = make_float4(f[0], f[1], f[2], f[3]);
    *reinterpret_cast<float4 *>(d + 4) = make_float4(f[4], f[5], f[6], f[7]);
  }
  __syncthreads();
  auto chunk = [&](const RBlocks &B, int c) {
    const float acc = leaf_tree32(q8r_leaf<BPL>(B, xs, nbc, c, L));
    if (L == 0) pp[r][c] = acc;
  };
  for (int c = g; c < nch; c += 2 * CW) {
    if (c + CW < nch) q8r_load<BPL>(Bb, rc, rs, row, N, K, nb, nbc, c + CW, L);
    chunk(Ba, c);
    if (c + CW >= nch) break;
    if (c + 2 * CW < nch) q8r_load<BPL>(Ba, rc, rs, row, N, K, nb, nbc, c + 2 * CW, L);
    chunk(Bb, c + CW);
  }
  lds_barrier();
  if (threadIdx.x < kRRows) {
    const int rw = blockIdx.x * kRRows + threadIdx.x;
    float yv = 0.0f;
    for (int c = 0; c < nch; c++) yv = yv + pp[threadIdx.x][c];
    if (rw < N) {
      if (y_bf16) reinterpret_cast<uint16_t *>(y)[(size_t)t * N + rw] = f2bf(yv);
      else reinterpret_cast<float *>(y)[(size_t)t * N + rw] = yv;
    }
  }
}

// The T-wide form (T > 1): the same per-output arithmetic, with each weight
// load serving many positions. A workgroup takes 8 rows x up to kRTPW
// positions; per chunk of K its lanes load their leaves' blocks once (CVT:
// codes widened to fp32 once, for up to 2 blocks per leaf), then the
// positions' x of that chunk are staged in LDS tp at a time (bf16 widened to
// fp32, 36-float padded blocks) and every position runs the leaf chains and
// the tree of the single-position kernel. The chunk partials of a (position,
// row) go to an LDS running sum in chunk order, y = ((0 + p_0) + p_1) + ...
constexpr int kRTPW = 32;      // positions per workgroup

template <int BPL, bool CVT>
__global__ __launch_bounds__(kRThreads) void q8r_gemm_kernel(const int8_t *__restrict__ codes,
                                                             const float *__restrict__ scales,
                                                             const uint16_t *__restrict__ x, void *__restrict__ y,
                                                             int y_bf16, int N, int K, int T, int tp) {
  extern __shared__ __align__(16) float rsm[];
  const int nb = K / kQ, KC = q8r_chunk(K), nbc = KC / kQ, nch = K / KC;
  float *ysum = rsm;                                   // [kRTPW][kRRows] running sums
  float *xs = rsm + kRTPW * kRRows;                    // [tp][nbc][kRXStride]
  const int wr = threadIdx.x >> 5, L = threadIdx.x & 31;
  const int row = blockIdx.x * kRRows + wr;
  const int t0 = blockIdx.y * kRTPW, tn = T - t0 < kRTPW ? T - t0 : kRTPW;
  const __amdgpu_buffer_rsrc_t rc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(codes), (short)0, N * K, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(scales), (short)0, N * nb * 4, kRsrcWord3);
  for (int i = threadIdx.x; i < kRTPW * kRRows; i += kRThreads) ysum[i] = 0.0f;
  for (int c = 0; c < nch; c++) {
    RBlocks B;
    q8r_load<BPL>(B, rc, rs, row, N, K, nb, nbc, c, L);
    float cf[CVT ? BPL : 1][32];
    if constexpr (CVT) {
#pragma unroll
      for (int i = 0; i < BPL; i++) {
        const uint32_t w[8] = {(uint32_t)B.c[2 * i].x,     (uint32_t)B.c[2 * i].y,     (uint32_t)B.c[2 * i].z,
                               (uint32_t)B.c[2 * i].w,     (uint32_t)B.c[2 * i + 1].x, (uint32_t)B.c[2 * i + 1].y,
                               (uint32_t)B.c[2 * i + 1].z, (uint32_t)B.c[2 * i + 1].w};
#pragma unroll
        for (int k = 0; k < 32; k++) cf[i][k] = (float)(int8_t)((w[k >> 2] >> (8 * (k & 3))) & 0xffu);
      }
    }
    for (int tt = 0; tt < tn; tt += tp) {
      const int np = tn - tt < tp ? tn - tt : tp;
      __syncthreads();   // the previous tile's reads of xs are done (and ysum is zeroed)
      // x of positions t0+tt .. +np, chunk c: 8 bf16 per thread per step
      for (int e = threadIdx.x * 8; e < np * KC; e += kRThreads * 8) {
        const int p = e / KC, k = e % KC;
        const uint4 u = *reinterpret_cast<const uint4 *>(x + (size_t)(t0 + tt + p) * K + (size_t)c * KC + k);
        const uint32_t v[4] = {u.x, u.y, u.z, u.w};
        float f[8];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          f[2 * q] = __uint_as_float(v[q] << 16);
          f[2 * q + 1] = __uint_as_float(v[q] & 0xffff0000u);
        }
        float *d = xs + ((size_t)p * nbc + (k >> 5)) * kRXStride + (k & 31);
        *reinterpret_cast<float4 *>(d) = make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4 *>(d + 4) = make_float4(f[4], f[5], f[6], f[7]);
      }
      __syncthreads();
      for (int p = 0; p < np; p++) {
        const float *xp = xs + (size_t)p * nbc * kRXStride;
        float acc = 0.0f;
#pragma unroll
        for (int i = 0; i < BPL; i++) {
          const int b = L + 32 * i;
          // a block past the chunk has zero codes and scale: fmaf(0, 0, acc) = acc
          const float *xb = xp + (size_t)(b < nbc ? b : 0) * kRXStride;
          float dot = 0.0f;
#pragma unroll
          for (int q = 0; q < 8; q++) {
            const float4 x4 = *reinterpret_cast<const float4 *>(xb + 4 * q);
            if constexpr (CVT) {
              dot = __builtin_fmaf(cf[i][4 * q], x4.x, dot);
              dot = __builtin_fmaf(cf[i][4 * q + 1], x4.y, dot);
              dot = __builtin_fmaf(cf[i][4 * q + 2], x4.z, dot);
              dot = __builtin_fmaf(cf[i][4 * q + 3], x4.w, dot);
            } else {
              // the code word passes through an empty asm per position: otherwise the converts,
              // invariant in p, are hoisted out of the position loop and their 32 * BPL
              // values held (BPL = 8: 256 VGPRs, one wave per SIMD; with this 105, four)
              uint32_t w = (uint32_t)(q < 4 ? B.c[2 * i][q] : B.c[2 * i + 1][q - 4]);
              asm volatile("" : "+v"(w));
              dot = __builtin_fmaf((float)(int8_t)(w & 0xffu), x4.x, dot);
              dot = __builtin_fmaf((float)(int8_t)((w >> 8) & 0xffu), x4.y, dot);
              dot = __builtin_fmaf((float)(int8_t)((w >> 16) & 0xffu), x4.z, dot);
              dot = __builtin_fmaf((float)(int8_t)(w >> 24), x4.w, dot);
            }
          }
          acc = __builtin_fmaf(B.s[i], dot, acc);
        }
        acc = leaf_tree32(acc);
        if (L == 0) ysum[(tt + p) * kRRows + wr] += acc;
      }
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < tn * kRRows; i += kRThreads) {
    const int t = i / kRRows, r = blockIdx.x * kRRows + i % kRRows;
    if (r < N) {
      const float v = ysum[i];
      if (y_bf16) reinterpret_cast<uint16_t *>(y)[(size_t)(t0 + t) * N + r] = f2bf(v);
      else reinterpret_cast<float *>(y)[(size_t)(t0 + t) * N + r] = v;
    }
  }
}

}  // namespace pq

using namespace pq;

extern "C" int pq_q8r_gemv(const int8_t *codes, const float *scales, const uint16_t *x, void *y, int y_dtype, int N,
                           int K, int T, void *stream) {
  PQ_REQUIRE(codes && scales && x && y, PQ_ERR_ARG, "pq_q8r_gemv: null pointer");
  PQ_REQUIRE(N > 0 && T > 0 && K >= kQ && K % kQ == 0, PQ_ERR_ARG, "pq_q8r_gemv: N=%d K=%d T=%d (K a multiple of 32)",
             N, K, T);
  PQ_REQUIRE(y_dtype == PQ_DTYPE_F32 || y_dtype == PQ_DTYPE_BF16, PQ_ERR_ARG, "pq_q8r_gemv: y_dtype %d", y_dtype);
  PQ_REQUIRE(aligned(codes, 16) && aligned(scales, 4) && aligned(x, 16) && K % 8 == 0, PQ_ERR_ALIGN,
             "pq_q8r_gemv: codes and x must be 16-byte aligned");
  const int KC = q8r_chunk(K), bpl = (KC / kQ + 31) / 32;
  PQ_REQUIRE(bpl <= 8, PQ_ERR_ARG, "pq_q8r_gemv: K=%d (above 8192, K must be a multiple of 2048)", K);
  PQ_REQUIRE((long long)N * K < (1ll << 31), PQ_ERR_ARG, "pq_q8r_gemv: N=%d K=%d too large", N, K);
  const size_t lds = (size_t)(K / kQ) * kRXStride * sizeof(float);
  PQ_REQUIRE(lds <= kMaxLds, PQ_ERR_ARG, "pq_q8r_gemv: K=%d too large for LDS", K);
  const int yb = y_dtype == PQ_DTYPE_BF16 ? 1 : 0;
  hipStream_t st = as_stream(stream);
  static const int env_t = env_int("PQ_Q8R_POSWISE");   // 1: one position per workgroup row at any T
  if (T > 1 && env_t != 1) {   // the T-wide form: each weight load serves up to 32 positions
    // positions per LDS tile: as many 36-float padded chunks as fit 18 KB, at most 8 (small tiles keep
    // several workgroups per CU: a 256-token prompt through 24 layers of hidden 2048 / FFN 8192 takes
    // 41 ms with 72 KB tiles, 25 ms with 18 KB)
    const size_t per = (size_t)(KC / kQ) * kRXStride * sizeof(float);
    static const int env_kb = env_int("PQ_Q8R_TILE_KB");
    const size_t budget = (size_t)(env_kb > 0 ? env_kb : 18) * 1024;
    const int tp = (int)std::min<size_t>(8, std::max<size_t>(1, budget / per));
    const size_t lds_t = (size_t)kRTPW * kRRows * sizeof(float) + (size_t)tp * per;
    PQ_REQUIRE(lds_t <= kMaxLds, PQ_ERR_ARG, "pq_q8r_gemv: K=%d too large for LDS", K);
    const dim3 gt((unsigned)((N + kRRows - 1) / kRRows), (unsigned)((T + kRTPW - 1) / kRTPW)), bt(kRThreads);
    if (bpl <= 1) launch(q8r_gemm_kernel<1, true>, gt, bt, lds_t, st, codes, scales, x, y, yb, N, K, T, tp);
    else if (bpl <= 2) launch(q8r_gemm_kernel<2, true>, gt, bt, lds_t, st, codes, scales, x, y, yb, N, K, T, tp);
    else if (bpl <= 4) launch(q8r_gemm_kernel<4, false>, gt, bt, lds_t, st, codes, scales, x, y, yb, N, K, T, tp);
    else launch(q8r_gemm_kernel<8, false>, gt, bt, lds_t, st, codes, scales, x, y, yb, N, K, T, tp);
    return check_launch("pq_q8r_gemv");
  }
  const dim3 grid((unsigned)((N + kRRows - 1) / kRRows), (unsigned)T), block(kRThreads);
  const bool mc = K / KC > 1;
  // rows of 2..8 chunks on fewer than 1024 workgroups: CW = 2 half-waves per row (PQ_Q8R_CW: 1, 2 or
  // 4). Measured per launch with cold weights: down 2048 x 8192 7.53 / 6.75 / 6.78 us at CW = 1 / 2 /
  // 4, 4096 x 12288 13.5 / 12.6 / 15.9 us, 2048 x 4096 5.0 / 4.7 / 4.7 us
  static const int env_cw = env_int("PQ_Q8R_CW");
  const int nch = K / KC;
  const bool cw_ok = env_cw == 1 || env_cw == 2 || env_cw == 4;   // any other value: the default
  int cw = cw_ok ? env_cw : (mc && nch <= kRMaxChunks && grid.x * T < 1024 ? 2 : 1);
  if (nch < 4) cw = std::min(cw, 2);   // no idle half-waves
  if (mc && nch <= kRMaxChunks && cw > 1) {
    const dim3 bk(kRThreads * cw);
    if (cw == 2) launch(q8r_gemv_kc_kernel<2>, grid, bk, lds, st, codes, scales, x, y, yb, N, K);
    else launch(q8r_gemv_kc_kernel<4>, grid, bk, lds, st, codes, scales, x, y, yb, N, K);
    return check_launch("pq_q8r_gemv");
  }
  // several chunks only with 2048-wide chunks, i.e. 2 blocks per lane
  if (mc) launch(q8r_gemv_kernel<2, true>, grid, block, lds, st, codes, scales, x, y, yb, N, K);
  else if (bpl <= 1) launch(q8r_gemv_kernel<1, false>, grid, block, lds, st, codes, scales, x, y, yb, N, K);
  else if (bpl <= 2) launch(q8r_gemv_kernel<2, false>, grid, block, lds, st, codes, scales, x, y, yb, N, K);
  else if (bpl <= 4) launch(q8r_gemv_kernel<4, false>, grid, block, lds, st, codes, scales, x, y, yb, N, K);
  else launch(q8r_gemv_kernel<8, false>, grid, block, lds, st, codes, scales, x, y, yb, N, K);
  return check_launch("pq_q8r_gemv");
}
