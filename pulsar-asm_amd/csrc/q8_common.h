// q8_common.h -- building blocks shared by the Q8_0 GEMV / GEMM kernels: the
// packed-layout constants and the per-chunk load / dot / fold steps of the R1
// order (see q8.hip for the layout and the order).
#pragma once
#include <stdlib.h>

#include "pq_device.h"
#include "pq_host.h"
#include "../../include/pulsar_amd.h"

namespace pq {

constexpr int kQ = PQ_QBLK;             // 32 codes per block
constexpr int kCB = PQ_CHUNK_BLOCKS;    // 8 blocks per R1 chunk
constexpr int kTR = PQ_TILE_ROWS;       // 64 rows per tile
constexpr int kSlab = 2 * kTR * 16;     // bytes per (tile, block): 2 halves x 64 rows x 16 B

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float f4v __attribute__((ext_vector_type(4)));

__host__ __device__ inline int nchunks(int K) { return (K / kQ + kCB - 1) / kCB; }
__host__ __device__ inline int ntiles(int N) { return (N + kTR - 1) / kTR; }

__device__ __forceinline__ float half_of(uint32_t w, int hi) { return h2f((uint16_t)(hi ? (w >> 16) : (w & 0xffffu))); }

// One row's chunk partial a_c, in two phases so a workgroup can issue its
// weight loads before it waits on anything else: load_chunk issues the 16
// 16-byte code loads (and the 8 scales) of a full chunk; dot_chunk folds the
// blocks ascending, each an exact int32 dot (8 v_dot4 over the lane's two
// halves) folded into a = fmaf(fl(dw*dx), (float)isum, a). XS(i, x) yields the
// 8 x dwords of block b0+i and DX(i) its scale (scalar registers when the
// chunk is wave-uniform, LDS otherwise).
struct ChunkRegs {
  v4i w[2 * kCB];
  uint32_t sw[4];
};

__device__ __forceinline__ void load_chunk(ChunkRegs &R, const int8_t *__restrict__ slab0,
                                           const uint16_t *__restrict__ sp8, int trow) {
#pragma unroll
  for (int i = 0; i < kCB; i++) {
    R.w[2 * i] = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(slab0 + (size_t)i * kSlab + trow * 16));
    R.w[2 * i + 1] =
        __builtin_nontemporal_load(reinterpret_cast<const v4i *>(slab0 + (size_t)i * kSlab + kTR * 16 + trow * 16));
  }
  const uint4 sv = *reinterpret_cast<const uint4 *>(sp8);
  R.sw[0] = sv.x; R.sw[1] = sv.y; R.sw[2] = sv.z; R.sw[3] = sv.w;
}

// The same loads through buffer resources over one 64-row tile's codes and
// scales. A slot without a chunk (c >= nch) reads at an offset past
// num_records, which returns zeros without a memory access: every lane issues
// the same loads with no branch, so the waits the compiler counts for loads
// issued earlier stay exact.
constexpr int kRsrcWord3 = 0x00020000;  // gfx9 buffer descriptor word 3 (32-bit data format)
constexpr int kRsrcOob = 0x40000000;    // an offset past every tile's num_records
constexpr int kAuxNT = 2;               // nontemporal cache policy
struct TileRsrc {
  __amdgpu_buffer_rsrc_t codes, scales;
};
__device__ __forceinline__ TileRsrc tile_rsrc(const int8_t *pc, const uint16_t *ps, int tile, int nb, int nch) {
  TileRsrc t;
  t.codes = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t *>(pc + (size_t)tile * nb * kSlab), (short)0,
                                              nb * kSlab, kRsrcWord3);
  t.scales = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(ps + (size_t)tile * nch * kTR * 8), (short)0,
                                               nch * kTR * 16, kRsrcWord3);
  return t;
}
__device__ __forceinline__ void load_chunk_rsrc(ChunkRegs &R, const TileRsrc &t, int c, int nch, int trow) {
  const int oc = c < nch ? c * kCB * kSlab + trow * 16 : kRsrcOob;
  const int os = c < nch ? (c * kTR + trow) * 16 : kRsrcOob;
#pragma unroll
  for (int i = 0; i < kCB; i++) {
    R.w[2 * i] = __builtin_amdgcn_raw_buffer_load_b128(t.codes, oc + i * kSlab, 0, kAuxNT);
    R.w[2 * i + 1] = __builtin_amdgcn_raw_buffer_load_b128(t.codes, oc + i * kSlab + kTR * 16, 0, kAuxNT);
  }
  const v4i sv = __builtin_amdgcn_raw_buffer_load_b128(t.scales, os, 0, 0);
  R.sw[0] = sv.x; R.sw[1] = sv.y; R.sw[2] = sv.z; R.sw[3] = sv.w;
}

__device__ __forceinline__ int dot8(v4i w0, v4i w1, const int *x) {
  int t = 0;
  t = __builtin_amdgcn_sdot4(w0.x, x[0], t, false);
  t = __builtin_amdgcn_sdot4(w0.y, x[1], t, false);
  t = __builtin_amdgcn_sdot4(w0.z, x[2], t, false);
  t = __builtin_amdgcn_sdot4(w0.w, x[3], t, false);
  t = __builtin_amdgcn_sdot4(w1.x, x[4], t, false);
  t = __builtin_amdgcn_sdot4(w1.y, x[5], t, false);
  t = __builtin_amdgcn_sdot4(w1.z, x[6], t, false);
  t = __builtin_amdgcn_sdot4(w1.w, x[7], t, false);
  return t;
}

template <typename XF, typename DF>
__device__ __forceinline__ float dot_chunk(const ChunkRegs &R, XF XS, DF DX) {
  int is[kCB];
#pragma unroll
  for (int i = 0; i < kCB; i++) {
    int x[8];
    XS(i, x);
    is[i] = dot8(R.w[2 * i], R.w[2 * i + 1], x);
  }
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < kCB; i++) a = __builtin_fmaf(half_of(R.sw[i >> 1], i & 1) * DX(i), (float)is[i], a);
  return a;
}

// The last chunk of a K that is not a multiple of 256: blocks b0 .. nb-1.
template <typename XF, typename DF>
__device__ __forceinline__ float tail_chunk(const int8_t *__restrict__ slab0, const uint16_t *__restrict__ sp8, int nbc,
                                            int trow, XF XS, DF DX) {
  float a = 0.0f;
  for (int i = 0; i < nbc; i++) {
    const v4i w0 = *reinterpret_cast<const v4i *>(slab0 + (size_t)i * kSlab + trow * 16);
    const v4i w1 = *reinterpret_cast<const v4i *>(slab0 + (size_t)i * kSlab + kTR * 16 + trow * 16);
    int x[8];
    XS(i, x);
    const int t = dot8(w0, w1, x);
    a = __builtin_fmaf(h2f(sp8[i]) * DX(i), (float)t, a);
  }
  return a;
}

constexpr int kXStride = 256 + 16;    // LDS bytes per staged x chunk (the pad spreads chunks over banks)
constexpr int kMaxStagedK = 32768;     // x staged in LDS only up to this K (35 KB)
constexpr size_t kMaxLds = 160 * 1024;  // LDS one gfx950 workgroup may allocate


// Decode GEMV launch shape: R rows per workgroup (64, or narrower slices when
// there are too few 64-row tiles to give each of the 256 CUs a workgroup) and
// W waves, enough to give every chunk of K a lane.
struct GemvShape { int R, W; };
inline GemvShape gemv_shape(int N, int K) {
  static const int fR = env_int("PQ_GEMV_R"), fW = env_int("PQ_GEMV_W");
  const int nt = ntiles(N), nch = nchunks(K);
  int R = 64;
  while (R > 8 && (long long)nt * (64 / R) < 256) R >>= 1;
  if (fR == 8 || fR == 16 || fR == 32 || fR == 64) R = fR;
  if (K > kMaxStagedK) R = 64;
  const int C = 64 / R;
  int W = (nch + C - 1) / C;
  W = W < 1 ? 1 : (W > 8 ? 8 : W);
  if (fW >= 1 && fW <= 8) W = fW;
  return {R, W};
}

}  // namespace pq
