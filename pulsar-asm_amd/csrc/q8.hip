// q8.hip -- Q8_0 activation quantizer, weight packing, the T=1 decode GEMV and
// the T-wide prefill GEMM for gfx950.
//
// Packed weight layout (64-row tiles, nb = K/32 blocks, nch = ceil(nb/8)):
//   codes  [tile][b][h][r][16 B] = codes[64*tile + r][32*b + 16*h .. +16]
//   scales [tile][c][r][8] fp16  = scale[64*tile + r][8*c + i]
// One (tile, b, h) slab is 1 KB: a wave64 load of 16 B per lane. The decode
// GEMV gives each lane one row (thread-per-row, the reference's TL kernels'
// mapping, lfm3_nanode.cu:4051-4123); the MFMA GEMM reads the same slabs as
// the 32x32x32 B operand (lane = row % 32, k-half = lane / 32).
//
// Numerics (R1), per output (row, position):
//   isum_b = sum_j w[32b+j] * qx[32b+j]          int32, exact (v_dot4)
//   s_b    = fl(f16(scale_b) * dx_b)
//   a_c    = fmaf(s_b, (float)isum_b, a_c)       blocks of chunk c ascending, from 0
//   y      = fl(y + a_c)                          chunks ascending, from 0
#include "pq_device.h"
#include "pq_host.h"
#include "q8_common.h"

namespace pq {

// ------------------------------------------------------------------ quantizer
// One 32-lane half wave per block: lane j holds x_j, amax by an xor-butterfly
// max (order-free), d = amax/127, q = rne(x/d) clamped.
template <typename TX>
__device__ __forceinline__ float load_act(const TX *p);
template <>
__device__ __forceinline__ float load_act<float>(const float *p) { return *p; }
template <>
__device__ __forceinline__ float load_act<uint16_t>(const uint16_t *p) { return bf2f(*p); }

template <typename TX>
__global__ __launch_bounds__(256) void q8_quant_kernel(const TX *__restrict__ x, int8_t *__restrict__ qx,
                                                        float *__restrict__ dx, long long nblk) {
  const long long gt = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long blk = gt >> 5;
  const int j = (int)(gt & 31);
  const bool valid = blk < nblk;
  const float v = valid ? load_act<TX>(x + blk * kQ + j) : 0.0f;
  float a = fabsf(v);
#pragma unroll
  for (int o = 1; o < 32; o <<= 1) a = fmaxf(a, __shfl_xor(a, o, 32));
  const float d = a / 127.0f;
  int q = 0;
  if (d != 0.0f) {
    q = (int)__builtin_rintf(v / d);
    q = q > 127 ? 127 : (q < -127 ? -127 : q);
  }
  if (valid) {
    qx[blk * kQ + j] = (int8_t)q;
    if (j == 0) dx[blk] = d;
  }
}

// -------------------------------------------------------------------- packing
// One thread per 16-byte slab piece (tile, b, h, r).
// Source row of packed row `row`: itself, or with il = F > 0 the gate/up pair
// interleave (packed rows 64t..64t+31 = gate rows 32t.., 64t+32.. = up rows
// F+32t..).
__device__ __forceinline__ long long src_row(long long row, int il) {
  if (il == 0) return row;
  const long long t = row / kTR, r = row % kTR;
  return r < 32 ? 32 * t + r : il + 32 * t + (r - 32);
}

__global__ __launch_bounds__(256) void q8_pack_codes_kernel(const int8_t *__restrict__ codes, int8_t *__restrict__ pc,
                                                             int N, int K, long long npieces, int il) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= npieces) return;
  const int nb = K / kQ;
  const int r = (int)(i % kTR);
  const int h = (int)((i / kTR) % 2);
  const long long tb = i / (2 * kTR);
  const int b = (int)(tb % nb);
  const long long tile = tb / nb;
  const long long row = tile * kTR + r;
  int4 v = make_int4(0, 0, 0, 0);
  if (row < N) v = *reinterpret_cast<const int4 *>(codes + src_row(row, il) * K + (long long)b * kQ + 16 * h);
  *reinterpret_cast<int4 *>(pc + i * 16) = v;
}

// One thread per (tile, chunk, row): its 8 scales.
__global__ __launch_bounds__(256) void q8_pack_scales_kernel(const uint16_t *__restrict__ sc, uint16_t *__restrict__ ps,
                                                              int N, int K, long long nitems, int il) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= nitems) return;
  const int nb = K / kQ, nch = nchunks(K);
  const int r = (int)(i % kTR);
  const long long tc = i / kTR;
  const int c = (int)(tc % nch);
  const long long tile = tc / nch;
  const long long row = tile * kTR + r;
  uint16_t v[8];
#pragma unroll
  for (int k = 0; k < 8; k++) {
    const int b = c * kCB + k;
    v[k] = (row < N && b < nb) ? sc[src_row(row, il) * nb + b] : (uint16_t)0;
  }
  uint4 o;
  o.x = v[0] | ((uint32_t)v[1] << 16);
  o.y = v[2] | ((uint32_t)v[3] << 16);
  o.z = v[4] | ((uint32_t)v[5] << 16);
  o.w = v[6] | ((uint32_t)v[7] << 16);
  *reinterpret_cast<uint4 *>(ps + i * 8) = o;
}

// ------------------------------------------------------------- decode GEMV
// Workgroup = R rows (a slice of one 64-row tile) x every chunk of K, so each
// workgroup writes finished outputs and no reduction crosses workgroups. Lane
// l handles row r = l % R of the slice and chunk slot cs = l / R (C = 64/R
// slots per wave); in round rd, wave w's lanes take chunks
// (rd*W + w)*C + cs. Each lane computes its chunk partial a_c; the round's
// partials go to LDS in chunk order and lanes 0..R-1 of wave 0 fold them into
// y = y + a_c. With R = 64 a wave's chunk is wave-uniform and x / dx come in
// through scalar loads; with R < 64 the workgroup stages x and dx in LDS.
template <int R>
__global__ __launch_bounds__(512) void q8_gemv_kernel(const int8_t *__restrict__ pc, const uint16_t *__restrict__ ps,
                                                       const int8_t *__restrict__ qx, const float *__restrict__ dx,
                                                       void *__restrict__ y, int y_bf16, int N, int K) {
  constexpr int C = 64 / R;
  extern __shared__ __align__(16) unsigned char smem[];
  const int nb = K / kQ, nch = nchunks(K);
  const int W = blockDim.x >> 6;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int cs = lane / R, r = lane % R;
  const int tile = blockIdx.x / C, trow = (blockIdx.x % C) * R + r;
  const int row = tile * kTR + trow;
  float *sp = reinterpret_cast<float *>(smem);                   // [W*C][R] partials of one round
  int8_t *xs = reinterpret_cast<int8_t *>(smem + (size_t)W * 64 * 4);
  float *dxs = reinterpret_cast<float *>(xs + (size_t)nch * kXStride);
  const int per_round = W * C;
  const int nrounds = (nch + per_round - 1) / per_round;
  const int slot = wave * C + cs;
  float yv = 0.0f;
  for (int rd = 0; rd < nrounds; rd++) {
    const int c = rd * per_round + slot;
    const int b0 = c * kCB;
    const bool full = c < nch && b0 + kCB <= nb;
    const int8_t *slab0 = pc + ((size_t)tile * nb + b0) * kSlab;
    const uint16_t *sp8 = ps + (((size_t)tile * nch + c) * kTR + trow) * 8;
    ChunkRegs regs;
    if (full) load_chunk(regs, slab0, sp8, trow);   // in flight while x is staged
    if (C > 1 && rd == 0) {
      for (int i = threadIdx.x; i < nb * 2; i += blockDim.x)
        *reinterpret_cast<v4i *>(xs + (i >> 4) * kXStride + (i & 15) * 16) = *reinterpret_cast<const v4i *>(qx + i * 16);
      for (int i = threadIdx.x; i < nb; i += blockDim.x) dxs[i] = dx[i];
      __syncthreads();
    }
    float a = 0.0f;
    if (c < nch) {
      if (C == 1) {
        const int *xg = reinterpret_cast<const int *>(qx + (size_t)b0 * kQ);
        auto XS = [&](int i, int *x) {
#pragma unroll
          for (int k = 0; k < 8; k++) x[k] = xg[i * 8 + k];
        };
        auto DX = [&](int i) { return dx[b0 + i]; };
        a = full ? dot_chunk(regs, XS, DX) : tail_chunk(slab0, sp8, nb - b0, trow, XS, DX);
      } else {
        const int8_t *xc = xs + (size_t)c * kXStride;
        auto XS = [&](int i, int *x) {
          const v4i lo = *reinterpret_cast<const v4i *>(xc + i * 32);
          const v4i hi = *reinterpret_cast<const v4i *>(xc + i * 32 + 16);
          x[0] = lo.x; x[1] = lo.y; x[2] = lo.z; x[3] = lo.w;
          x[4] = hi.x; x[5] = hi.y; x[6] = hi.z; x[7] = hi.w;
        };
        auto DX = [&](int i) { return dxs[b0 + i]; };
        a = full ? dot_chunk(regs, XS, DX) : tail_chunk(slab0, sp8, nb - b0, trow, XS, DX);
      }
    }
    sp[slot * R + r] = a;
    __syncthreads();
    if (wave == 0 && lane < R) {
      const int n = nch - rd * per_round < per_round ? nch - rd * per_round : per_round;
      for (int k = 0; k < n; k++) yv = yv + sp[k * R + lane];
    }
    __syncthreads();
  }
  if (wave == 0 && lane < R && row < N) {
    if (y_bf16) reinterpret_cast<uint16_t *>(y)[row] = f2bf(yv);
    else reinterpret_cast<float *>(y)[row] = yv;
  }
}

// ------------------------------------------------------------ prefill GEMM
// Workgroup = one 32-row half of a 64-row tile x 32 positions x all of K, W
// waves. In round rd wave w takes R1 chunk c = rd*W + w: per block one
// v_mfma_i32_32x32x32_i8 with A = activations (i = position) and B = weights
// (j = row), so lane l holds D[i][j] for j = l % 32 and
// i = 8(r/4) + 4(l/32) + r%4 (r = 0..15), and folds its 16 outputs into the
// chunk partial a = fmaf(fl(dw*dx), (float)isum, a). The round's partials go
// to LDS and the workgroup adds them to y in chunk order (y = y + a_c), each
// thread owning 1024/(64W) of the 32x32 outputs. dx of the round's chunks is
// staged in LDS as [wave][block][position].
template <int W>
__global__ __launch_bounds__(64 * W) void q8_gemm_kernel(const int8_t *__restrict__ pc,
                                                          const uint16_t *__restrict__ ps,
                                                          const int8_t *__restrict__ qx, const float *__restrict__ dx,
                                                          void *__restrict__ y, int y_bf16, int N, int K, int T) {
  constexpr int EPT = 1024 / (64 * W);          // outputs folded per thread
  __shared__ float part[W][16][64];
  __shared__ __align__(16) float dxs[W][kCB][32];
  const int nb = K / kQ, nch = nchunks(K);
  const int tile = blockIdx.x >> 1, sub = blockIdx.x & 1;
  const int p0 = blockIdx.y * 32;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int h = lane >> 5, l32 = lane & 31;
  const int jrow = sub * 32 + l32;
  const int apos = p0 + l32;
  const bool aval = apos < T;
  const int8_t *arow = qx + (size_t)(aval ? apos : 0) * K + 16 * h;
  float yv[EPT];
#pragma unroll
  for (int k = 0; k < EPT; k++) yv[k] = 0.0f;
  const int nrounds = (nch + W - 1) / W;
  for (int rd = 0; rd < nrounds; rd++) {
    const int c = rd * W + wave;
    const int b0 = c * kCB;
    const int nbc = c < nch ? (b0 + kCB <= nb ? kCB : nb - b0) : 0;
    for (int i = lane; i < kCB * 32; i += 64) {
      const int bi = i >> 5, p = i & 31, pos = p0 + p;
      dxs[wave][bi][p] = (bi < nbc && pos < T) ? dx[(size_t)pos * nb + b0 + bi] : 0.0f;
    }
    __syncthreads();
    float a[16];
#pragma unroll
    for (int r = 0; r < 16; r++) a[r] = 0.0f;
    if (nbc > 0) {
      const uint4 sv = *reinterpret_cast<const uint4 *>(ps + (((size_t)tile * nch + c) * kTR + jrow) * 8);
      const uint32_t sw[4] = {sv.x, sv.y, sv.z, sv.w};
      v4i bw[kCB], av[kCB];
#pragma unroll
      for (int i = 0; i < kCB; i++) {
        if (i < nbc) {
          bw[i] = __builtin_nontemporal_load(
              reinterpret_cast<const v4i *>(pc + ((size_t)tile * nb + b0 + i) * kSlab + (h * kTR + jrow) * 16));
          av[i] = aval ? *reinterpret_cast<const v4i *>(arow + (size_t)(b0 + i) * kQ) : v4i{0, 0, 0, 0};
        }
      }
#pragma unroll
      for (int i = 0; i < kCB; i++) {
        if (i < nbc) {
          v16i acc = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
          acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(av[i], bw[i], acc, 0, 0, 0);
          const float dw = half_of(sw[i >> 1], i & 1);
#pragma unroll
          for (int g = 0; g < 4; g++) {
            const float4 d4 = *reinterpret_cast<const float4 *>(&dxs[wave][i][8 * g + 4 * h]);
            const float dv[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
            for (int k = 0; k < 4; k++) a[4 * g + k] = __builtin_fmaf(dw * dv[k], (float)acc[4 * g + k], a[4 * g + k]);
          }
        }
      }
    }
#pragma unroll
    for (int r = 0; r < 16; r++) part[wave][r][lane] = a[r];
    __syncthreads();
    const int nvalid = nch - rd * W < W ? nch - rd * W : W;
#pragma unroll
    for (int k = 0; k < EPT; k++) {
      const int e = threadIdx.x + k * 64 * W;
      const int r = e >> 6, l = e & 63;
      for (int w = 0; w < nvalid; w++) yv[k] = yv[k] + part[w][r][l];
    }
    __syncthreads();
  }
#pragma unroll
  for (int k = 0; k < EPT; k++) {
    const int e = threadIdx.x + k * 64 * W;
    const int r = e >> 6, l = e & 63;
    const int pos = p0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    const int row = tile * kTR + sub * 32 + (l & 31);
    if (pos < T && row < N) {
      if (y_bf16) reinterpret_cast<uint16_t *>(y)[(size_t)pos * N + row] = f2bf(yv[k]);
      else reinterpret_cast<float *>(y)[(size_t)pos * N + row] = yv[k];
    }
  }
}

}  // namespace pq

using namespace pq;

extern "C" size_t pq_q8_packed_codes_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || K % kQ) return 0;
  return (size_t)ntiles(N) * (K / kQ) * kSlab;
}

extern "C" size_t pq_q8_packed_scales_bytes(int N, int K) {
  if (N <= 0 || K <= 0 || K % kQ) return 0;
  return (size_t)ntiles(N) * nchunks(K) * kTR * 8 * sizeof(uint16_t);
}

extern "C" int pq_q8_quant_f32(const float *x, int8_t *qx, float *dx, int K, int T, void *stream) {
  PQ_REQUIRE(x && qx && dx, PQ_ERR_ARG, "pq_q8_quant_f32: null pointer");
  PQ_REQUIRE(K > 0 && K % kQ == 0 && T > 0, PQ_ERR_ARG, "pq_q8_quant_f32: K=%d T=%d (K must be a multiple of 32)", K, T);
  const long long nblk = (long long)T * (K / kQ);
  const long long threads = nblk * 32;
  launch(q8_quant_kernel<float>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, as_stream(stream),
                     x, qx, dx, nblk);
  return check_launch("pq_q8_quant_f32");
}

extern "C" int pq_q8_quant_bf16(const uint16_t *x, int8_t *qx, float *dx, int K, int T, void *stream) {
  PQ_REQUIRE(x && qx && dx, PQ_ERR_ARG, "pq_q8_quant_bf16: null pointer");
  PQ_REQUIRE(K > 0 && K % kQ == 0 && T > 0, PQ_ERR_ARG, "pq_q8_quant_bf16: K=%d T=%d (K must be a multiple of 32)", K, T);
  const long long nblk = (long long)T * (K / kQ);
  const long long threads = nblk * 32;
  launch(q8_quant_kernel<uint16_t>, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     as_stream(stream), x, qx, dx, nblk);
  return check_launch("pq_q8_quant_bf16");
}

static int pack(const int8_t *codes, const uint16_t *scales, int N, int K, int8_t *pcodes, uint16_t *pscales, int il,
                void *stream, const char *who) {
  PQ_REQUIRE(codes && scales && pcodes && pscales, PQ_ERR_ARG, "%s: null pointer", who);
  PQ_REQUIRE(N > 0 && K > 0 && K % kQ == 0, PQ_ERR_ARG, "%s: N=%d K=%d", who, N, K);
  PQ_REQUIRE(aligned(codes, 16) && aligned(pcodes, 16) && aligned(pscales, 16), PQ_ERR_ALIGN,
             "%s: codes and packed buffers must be 16-byte aligned", who);
  const long long npieces = (long long)ntiles(N) * (K / kQ) * 2 * kTR;
  launch(q8_pack_codes_kernel, dim3((unsigned)((npieces + 255) / 256)), dim3(256), 0, as_stream(stream),
                     codes, pcodes, N, K, npieces, il);
  int rc = check_launch(who);
  if (rc) return rc;
  const long long nitems = (long long)ntiles(N) * nchunks(K) * kTR;
  launch(q8_pack_scales_kernel, dim3((unsigned)((nitems + 255) / 256)), dim3(256), 0, as_stream(stream),
                     scales, pscales, N, K, nitems, il);
  return check_launch(who);
}

extern "C" int pq_q8_pack(const int8_t *codes, const uint16_t *scales, int N, int K, int8_t *pcodes,
                          uint16_t *pscales, void *stream) {
  return pack(codes, scales, N, K, pcodes, pscales, 0, stream, "pq_q8_pack");
}

extern "C" int pq_q8_pack_gate_up(const int8_t *codes, const uint16_t *scales, int F, int K, int8_t *pcodes,
                                  uint16_t *pscales, void *stream) {
  PQ_REQUIRE(F > 0 && F % 32 == 0, PQ_ERR_ARG, "pq_q8_pack_gate_up: F=%d (a multiple of 32)", F);
  return pack(codes, scales, 2 * F, K, pcodes, pscales, F, stream, "pq_q8_pack_gate_up");
}

extern "C" int pq_q8_gemv(const int8_t *pcodes, const uint16_t *pscales, const int8_t *qx, const float *dx, void *y,
                          int y_dtype, int N, int K, void *stream) {
  PQ_REQUIRE(pcodes && pscales && qx && dx && y, PQ_ERR_ARG, "pq_q8_gemv: null pointer");
  PQ_REQUIRE(N > 0 && K > 0 && K % kQ == 0, PQ_ERR_ARG, "pq_q8_gemv: N=%d K=%d (K must be a multiple of 32)", N, K);
  PQ_REQUIRE(y_dtype == PQ_DTYPE_F32 || y_dtype == PQ_DTYPE_BF16, PQ_ERR_ARG, "pq_q8_gemv: y_dtype %d", y_dtype);
  PQ_REQUIRE(aligned(pcodes, 16) && aligned(pscales, 16) && aligned(qx, 16) && aligned(dx, 4), PQ_ERR_ALIGN,
             "pq_q8_gemv: packed weights and qx must be 16-byte aligned");
  const GemvShape g = gemv_shape(N, K);
  const int C = 64 / g.R;
  const size_t lds = (size_t)g.W * 64 * 4 + (C > 1 ? (size_t)nchunks(K) * kXStride + (size_t)(K / kQ) * 4 : 0);
  const dim3 grid((unsigned)(ntiles(N) * C)), block(64 * g.W);
  const int yb = y_dtype == PQ_DTYPE_BF16 ? 1 : 0;
  hipStream_t st = as_stream(stream);
  switch (g.R) {
    case 64: launch(q8_gemv_kernel<64>, grid, block, lds, st, pcodes, pscales, qx, dx, y, yb, N, K); break;
    case 32: launch(q8_gemv_kernel<32>, grid, block, lds, st, pcodes, pscales, qx, dx, y, yb, N, K); break;
    case 16: launch(q8_gemv_kernel<16>, grid, block, lds, st, pcodes, pscales, qx, dx, y, yb, N, K); break;
    default: launch(q8_gemv_kernel<8>, grid, block, lds, st, pcodes, pscales, qx, dx, y, yb, N, K); break;
  }
  return check_launch("pq_q8_gemv");
}

extern "C" int pq_q8_gemm(const int8_t *pcodes, const uint16_t *pscales, const int8_t *qx, const float *dx, void *y,
                          int y_dtype, int N, int K, int T, void *stream) {
  PQ_REQUIRE(pcodes && pscales && qx && dx && y, PQ_ERR_ARG, "pq_q8_gemm: null pointer");
  PQ_REQUIRE(N > 0 && K > 0 && K % kQ == 0 && T > 0, PQ_ERR_ARG, "pq_q8_gemm: N=%d K=%d T=%d", N, K, T);
  PQ_REQUIRE(y_dtype == PQ_DTYPE_F32 || y_dtype == PQ_DTYPE_BF16, PQ_ERR_ARG, "pq_q8_gemm: y_dtype %d", y_dtype);
  PQ_REQUIRE(aligned(pcodes, 16) && aligned(pscales, 16) && aligned(qx, 16) && aligned(dx, 4), PQ_ERR_ALIGN,
             "pq_q8_gemm: packed weights and qx must be 16-byte aligned");
  const int nch = nchunks(K);
  const int W = nch >= 8 ? 8 : (nch >= 4 ? 4 : (nch >= 2 ? 2 : 1));
  const dim3 grid((unsigned)(ntiles(N) * 2), (unsigned)((T + 31) / 32));
  const int yb = y_dtype == PQ_DTYPE_BF16 ? 1 : 0;
  hipStream_t st = as_stream(stream);
  switch (W) {
    case 8: launch(q8_gemm_kernel<8>, grid, dim3(512), 0, st, pcodes, pscales, qx, dx, y, yb, N, K, T); break;
    case 4: launch(q8_gemm_kernel<4>, grid, dim3(256), 0, st, pcodes, pscales, qx, dx, y, yb, N, K, T); break;
    case 2: launch(q8_gemm_kernel<2>, grid, dim3(128), 0, st, pcodes, pscales, qx, dx, y, yb, N, K, T); break;
    default: launch(q8_gemm_kernel<1>, grid, dim3(64), 0, st, pcodes, pscales, qx, dx, y, yb, N, K, T); break;
  }
  return check_launch("pq_q8_gemm");
}
