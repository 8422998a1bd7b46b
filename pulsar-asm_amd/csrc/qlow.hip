// qlow.hip -- Q4 / Q5 low-bit backbone GEMV (gfx950), the reference's order.
//
// Format (lfm3_qlow.cuh:1-16), per 32-group along K: w = d*q + mn, q in
// [0, 2^B) (B = 4 or 5), d' = 128*d and mn fp16. The payload is tiled by 32
// rows: for tile t, group g, 32 x 16 bytes of nibbles (row r's 32 codes: byte
// b of word i holds weight 8i+b in its low nibble and 8i+4+b in its high
// nibble), for B = 5 then 32 x uint32 high planes (bit 8b+p = bit 4 of weight
// 4p+b); scales [tile][g][32 rows] half2 (d', mn).
//
// Numerics of k_qlow + k_qlow_combine (lfm3_qlow.cuh:39-113) with
// qlow_gemv's K split (lfm3_nanode.cu:1894-1915), per row:
//   KS = 4 slices of whole groups for K >= 4096, else 2;
//   sg = the group's 32 x summed in order from 0;
//   a_b = fmaf chain over k = b, b+4, ..., b+28 of (1 + q_k/128) * x_k from
//   0 (the code read as the float 1 + q/128), acc = (a0 + a1) + (a2 + a3);
//   y_s = fmaf(d', acc - sg, fmaf(mn, sg, y_s)) over the slice's groups from 0;
//   y = ((0 + y_0) + y_1) + ...; out bf16(y) or y.
//
// A workgroup owns one 32-row tile: lane r of each of the 16 32-lane slots
// takes row r, slot j takes groups j, j+16, ... (a slot's 32 lanes read a
// tile-group's 512 contiguous bytes), computes acc - sg into LDS; then one
// lane per (row, slice) runs the slice's fmaf chain, and the slices add in
// order.
#include "pq_device.h"
#include "pq_host.h"
#include "q8_common.h"

namespace pq {

constexpr int kLoThreads = 512;
constexpr int kLoSlots = kLoThreads / 32;   // group slots per round

__host__ __device__ inline int qlow_ks(int K) { return K >= 4096 ? 4 : 2; }
__host__ __device__ inline int qlow_gw(int B) { return B == 4 ? 32 : 40; }   // 16-byte units per tile-group

// The code byte q as the float 1 + q/128 (q < 128: exponent of 1.0, q in
// mantissa bits 16..22).
__device__ __forceinline__ float qlow_f(uint32_t m, int b) {
  return __uint_as_float(0x3F800000u | (((m >> (8 * b)) & 0xffu) << 16));
}

template <int B>
__device__ __forceinline__ float qlow_acc(v4i w4, uint32_t hp, const float *__restrict__ xg) {
  const uint32_t w[4] = {(uint32_t)w4.x, (uint32_t)w4.y, (uint32_t)w4.z, (uint32_t)w4.w};
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      uint32_t m = (hf ? (w[i] >> 4) : w[i]) & 0x0F0F0F0Fu;
      if constexpr (B == 5) {   // bit 4 of quad p's four codes from the plane's bits p, 8+p, 16+p, 24+p
        const int p = 2 * i + hf;
        const uint32_t hs = p <= 4 ? (hp << (4 - p)) : (hp >> (p - 4));
        m |= hs & 0x10101010u;
      }
      const float4 xv = *reinterpret_cast<const float4 *>(xg + 8 * i + 4 * hf);
      a0 = __builtin_fmaf(qlow_f(m, 0), xv.x, a0);
      a1 = __builtin_fmaf(qlow_f(m, 1), xv.y, a1);
      a2 = __builtin_fmaf(qlow_f(m, 2), xv.z, a2);
      a3 = __builtin_fmaf(qlow_f(m, 3), xv.w, a3);
    }
  }
  return (a0 + a1) + (a2 + a3);
}

// With ws (the split form): workgroup (tile, s) covers only slice s =
// blockIdx.y and writes its y_s to ws[s][N]; qlow_combine_kernel adds the
// slices in order. Without ws: one workgroup per tile, all slices.
template <int B>
__global__ __launch_bounds__(kLoThreads) void qlow_gemv_kernel(const uint8_t *__restrict__ pc,
                                                              const uint32_t *__restrict__ ps,
                                                              const uint16_t *__restrict__ x, void *__restrict__ y,
                                                              int y_bf16, int N, int K, float *__restrict__ ws) {
  extern __shared__ __align__(16) float lsm[];
  const int GA = K / kQ, KSA = qlow_ks(K), GW = qlow_gw(B);
  // the groups this workgroup covers: [gb, gb + G), in KS slices of GL
  const int KS = ws ? 1 : KSA, G = ws ? GA / KSA : GA, GL = G / KS, gb = ws ? (int)blockIdx.y * G : 0;
  float *xs = lsm;                      // [G*32]
  float *sx = xs + G * kQ;              // [G]
  float *u = sx + G;                    // [32 rows][G + 1]: acc - sg
  float *ys = u + 32 * (G + 1);         // [KS][32]
  uint32_t *scl = reinterpret_cast<uint32_t *>(ys + KS * 32);   // [G][32] half2 (d', mn)
  const int tid = threadIdx.x, tile = blockIdx.x;
  const int r = tid & 31, slot = tid >> 5;
  // the tile's codes and scales from group gb (wave-uniform resources)
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(pc + ((size_t)tile * GA + gb) * GW * 16), (short)0, G * GW * 16, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t *>(ps + ((size_t)tile * GA + gb) * 32), (short)0, G * 32 * 4, kRsrcWord3);
  x += (size_t)gb * kQ;
  K = G * kQ;
  // this lane's first PF groups' codes, before anything waits
  constexpr int PF = 4;
  v4i w[PF];
  uint32_t hpl[PF];
#pragma unroll
  for (int k = 0; k < PF; k++) {
    const int g = slot + kLoSlots * k;
    w[k] = __builtin_amdgcn_raw_buffer_load_b128(rc, g < G ? (g * GW + r) * 16 : kRsrcOob, 0, kAuxNT);
    hpl[k] = B == 5 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, g < G ? (g * GW + 32) * 16 + r * 4 : kRsrcOob, 0,
                                                                     kAuxNT)
                    : 0u;
  }
  // the tile's scales into LDS (16-byte loads over the contiguous [G][32])
  for (int i = tid; i < G * 8; i += kLoThreads) {
    const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rsc, i * 16, 0, 0);
    *reinterpret_cast<v4i *>(scl + 4 * i) = v;
  }
  // x widened into LDS, then each group's sum of x in order
  for (int e = tid * 8; e < K; e += kLoThreads * 8) {
    const uint4 v = *reinterpret_cast<const uint4 *>(x + e);
    const uint32_t vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int k = 0; k < 4; k++) {
      xs[e + 2 * k] = __uint_as_float(vv[k] << 16);
      xs[e + 2 * k + 1] = __uint_as_float(vv[k] & 0xffff0000u);
    }
  }
  __syncthreads();
  for (int g = tid; g < G; g += kLoThreads) {
    float t = 0.0f;
    for (int k = 0; k < kQ; k++) t += xs[g * kQ + k];
    sx[g] = t;
  }
  __syncthreads();
  // group partials acc - sg, PF groups of loads in flight
  for (int g0 = 0; g0 < G; g0 += kLoSlots * PF) {
    v4i wn[PF];
    uint32_t hn[PF];
    const bool more = g0 + kLoSlots * PF < G;
    if (more) {
#pragma unroll
      for (int k = 0; k < PF; k++) {
        const int g = g0 + kLoSlots * PF + slot + kLoSlots * k;
        wn[k] = __builtin_amdgcn_raw_buffer_load_b128(rc, g < G ? (g * GW + r) * 16 : kRsrcOob, 0, kAuxNT);
        hn[k] = B == 5 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                             rc, g < G ? (g * GW + 32) * 16 + r * 4 : kRsrcOob, 0, kAuxNT)
                       : 0u;
      }
    }
#pragma unroll
    for (int k = 0; k < PF; k++) {
      const int g = g0 + slot + kLoSlots * k;
      if (g < G) u[r * (G + 1) + g] = qlow_acc<B>(w[k], hpl[k], xs + g * kQ) - sx[g];
    }
    if (more) {
#pragma unroll
      for (int k = 0; k < PF; k++) { w[k] = wn[k]; hpl[k] = hn[k]; }
    }
  }
  __syncthreads();
  // per (row, slice): the slice's chain over its groups in order
  if (tid < 32 * KS) {
    const int s = tid >> 5;
    float yv = 0.0f;
    for (int g = s * GL; g < (s + 1) * GL; g++) {
      const uint32_t sc = scl[g * 32 + r];
      const float dp = h2f((uint16_t)(sc & 0xffffu)), mn = h2f((uint16_t)(sc >> 16));
      yv = __builtin_fmaf(dp, u[r * (G + 1) + g], __builtin_fmaf(mn, sx[g], yv));
    }
    ys[s * 32 + r] = yv;
  }
  __syncthreads();
  if (tid < 32) {
    const int row = tile * 32 + r;
    if (ws) {
      if (row < N) ws[(size_t)blockIdx.y * N + row] = ys[r];
      return;
    }
    float yt = 0.0f;
    for (int s = 0; s < KS; s++) yt = yt + ys[s * 32 + r];
    if (row < N) {
      if (y_bf16) reinterpret_cast<uint16_t *>(y)[row] = f2bf(yt);
      else reinterpret_cast<float *>(y)[row] = yt;
    }
  }
}

// y = ((0 + ws[0]) + ws[1]) + ... (k_qlow_combine, lfm3_qlow.cuh:107-113).
__global__ __launch_bounds__(256) void qlow_combine_kernel(const float *__restrict__ ws, void *__restrict__ y,
                                                            int y_bf16, int N, int KS) {
  const int row = blockIdx.x * blockDim.x + threadIdx.x;
  if (row >= N) return;
  float yt = 0.0f;
  for (int s = 0; s < KS; s++) yt = yt + ws[(size_t)s * N + row];
  if (y_bf16) reinterpret_cast<uint16_t *>(y)[row] = f2bf(yt);
  else reinterpret_cast<float *>(y)[row] = yt;
}

// Row-major codes q [N][K] (one per byte) and scales [N][K/32][2] fp16 ->
// the tiled payload above; one thread per (row, group).
__global__ void qlow_pack_kernel(const uint8_t *__restrict__ q, const uint16_t *__restrict__ s,
                                 uint8_t *__restrict__ pc, uint32_t *__restrict__ ps, int N, int K, int B) {
  const int G = K / kQ, GW = qlow_gw(B);
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long long)N * G) return;
  const int row = (int)(i / G), g = (int)(i % G), tile = row >> 5, r = row & 31;
  const uint8_t *qg = q + (size_t)row * K + g * kQ;
  uint32_t w[4] = {0u, 0u, 0u, 0u}, hp = 0u;
  for (int i4 = 0; i4 < 4; i4++)
    for (int b = 0; b < 4; b++) {
      const uint32_t lo = qg[8 * i4 + b], hi = qg[8 * i4 + 4 + b];
      w[i4] |= ((lo & 15u) | ((hi & 15u) << 4)) << (8 * b);
    }
  if (B == 5)
    for (int p = 0; p < 8; p++)
      for (int b = 0; b < 4; b++) hp |= ((uint32_t)(qg[4 * p + b] >> 4) & 1u) << (8 * b + p);
  uint8_t *dst = pc + (((size_t)tile * G + g) * GW) * 16;
  *reinterpret_cast<uint4 *>(dst + r * 16) = make_uint4(w[0], w[1], w[2], w[3]);
  if (B == 5) reinterpret_cast<uint32_t *>(dst + 32 * 16)[r] = hp;
  ps[((size_t)tile * G + g) * 32 + r] = (uint32_t)s[((size_t)row * G + g) * 2] | ((uint32_t)s[((size_t)row * G + g) * 2 + 1] << 16);
}

}  // namespace pq

using namespace pq;

static bool qlow_shape(int N, int K, int bits) {
  return (bits == 4 || bits == 5) && N > 0 && N % 32 == 0 && K > 0 && K % 256 == 0 && K <= 16384;
}

extern "C" size_t pq_qlow_packed_codes_bytes(int N, int K, int bits) {
  if (!qlow_shape(N, K, bits)) return 0;
  return (size_t)N / 32 * (K / kQ) * qlow_gw(bits) * 16;
}

extern "C" size_t pq_qlow_packed_scales_bytes(int N, int K, int bits) {
  if (!qlow_shape(N, K, bits)) return 0;
  return (size_t)N * (K / kQ) * 4;
}

extern "C" int pq_qlow_pack(const uint8_t *codes, const uint16_t *scales, int N, int K, int bits, uint8_t *pcodes,
                            uint16_t *pscales, void *stream) {
  PQ_REQUIRE(codes && scales && pcodes && pscales, PQ_ERR_ARG, "pq_qlow_pack: null pointer");
  PQ_REQUIRE(qlow_shape(N, K, bits), PQ_ERR_ARG, "pq_qlow_pack: N=%d K=%d bits=%d (N %% 32, K %% 256, bits 4 or 5)", N,
             K, bits);
  PQ_REQUIRE(aligned(pcodes, 16) && aligned(pscales, 4) && aligned(scales, 2), PQ_ERR_ALIGN,
             "pq_qlow_pack: packed buffers must be 16-byte aligned");
  const long long n = (long long)N * (K / kQ);
  launch(qlow_pack_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream), codes, scales, pcodes,
         reinterpret_cast<uint32_t *>(pscales), N, K, bits);
  return check_launch("pq_qlow_pack");
}

extern "C" size_t pq_qlow_workspace_bytes(int N, int K, int bits) {
  if (!qlow_shape(N, K, bits)) return 0;
  return (size_t)qlow_ks(K) * N * sizeof(float);
}

extern "C" int pq_qlow_gemv(const uint8_t *pcodes, const uint16_t *pscales, const uint16_t *x, void *y, int y_dtype,
                            int N, int K, int bits, void *stream) {
  return pq_qlow_gemv_ws(pcodes, pscales, x, y, y_dtype, N, K, bits, nullptr, 0, stream);
}

extern "C" int pq_qlow_gemv_ws(const uint8_t *pcodes, const uint16_t *pscales, const uint16_t *x, void *y,
                               int y_dtype, int N, int K, int bits, void *ws, size_t ws_bytes, void *stream) {
  PQ_REQUIRE(pcodes && pscales && x && y, PQ_ERR_ARG, "pq_qlow_gemv: null pointer");
  PQ_REQUIRE(qlow_shape(N, K, bits), PQ_ERR_ARG, "pq_qlow_gemv: N=%d K=%d bits=%d (N %% 32, K %% 256, bits 4 or 5)", N,
             K, bits);
  PQ_REQUIRE(y_dtype == PQ_DTYPE_F32 || y_dtype == PQ_DTYPE_BF16, PQ_ERR_ARG, "pq_qlow_gemv: y_dtype %d", y_dtype);
  PQ_REQUIRE(aligned(pcodes, 16) && aligned(pscales, 4) && aligned(x, 16), PQ_ERR_ALIGN,
             "pq_qlow_gemv: packed codes and x must be 16-byte aligned");
  const int KS = qlow_ks(K);
  auto lds_of = [&](int G, int ks) {
    return ((size_t)G * kQ + G + 32 * (size_t)(G + 1) + (size_t)ks * 32 + 32 * (size_t)G) * sizeof(float);
  };
  // the split form (one workgroup per (tile, slice), then the ordered
  // combine): for long rows on too few tiles to fill the chip (K = 2048 rows
  // measured faster whole), or when a whole row's staging exceeds LDS
  const bool whole_fits = lds_of(K / kQ, KS) <= kMaxLds;
  const bool split = ws != nullptr && ws_bytes >= pq_qlow_workspace_bytes(N, K, bits) &&
                     ((N / 32 < 256 && K >= 4096) || !whole_fits);
  PQ_REQUIRE(!split || aligned(ws, 4), PQ_ERR_ALIGN, "pq_qlow_gemv: workspace alignment");
  const int G = split ? K / kQ / KS : K / kQ, KSW = split ? 1 : KS;
  const size_t lds = lds_of(G, KSW);
  PQ_REQUIRE(lds <= kMaxLds, PQ_ERR_ARG, "pq_qlow_gemv: K=%d needs the workspace form", K);
  const dim3 grid((unsigned)(N / 32), split ? (unsigned)KS : 1u), block(kLoThreads);
  const int yb = y_dtype == PQ_DTYPE_BF16 ? 1 : 0;
  float *wsf = split ? static_cast<float *>(ws) : nullptr;
  hipStream_t st = as_stream(stream);
  if (bits == 4)
    launch(qlow_gemv_kernel<4>, grid, block, lds, st, pcodes, reinterpret_cast<const uint32_t *>(pscales), x, y, yb,
           N, K, wsf);
  else
    launch(qlow_gemv_kernel<5>, grid, block, lds, st, pcodes, reinterpret_cast<const uint32_t *>(pscales), x, y, yb,
           N, K, wsf);
  int rc = check_launch("pq_qlow_gemv");
  if (rc || !split) return rc;
  launch(qlow_combine_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, st, wsf, y, yb, N, KS);
  return check_launch("pq_qlow_gemv combine");
}
