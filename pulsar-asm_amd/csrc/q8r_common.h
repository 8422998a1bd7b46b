// q8r_common.h -- device pieces of the reference-numerics (R2) Q8_0 GEMV
// shared by its plain kernels (q8r.hip) and its fused-prologue form
// (decode_fused.hip): the workgroup shape, a lane's block loads, its leaf
// chain over the staged fp32 x and the 32-lane leaf tree. The arithmetic
// is q8_partial<bf16, FMA=1> + k_combine (lfm3_nanode.cu:222-374).
#pragma once

#include "pq_device.h"
#include "q8_common.h"

namespace pq {

constexpr int kRRows = 8;        // rows per workgroup
constexpr int kRThreads = 32 * kRRows;
constexpr int kRXStride = 36;    // LDS floats per staged 32-block of x
constexpr int kRMaxChunks = 8;   // 2048-wide chunks a row may hold in the chunk-split form

__host__ __device__ inline int q8r_chunk(int K) { return (K >= 2048 && K % 2048 == 0) ? 2048 : K; }

struct RBlocks {
  v4i c[2 * 8];
  float s[8];
};

// The lane's BPL blocks of chunk c (block L + 32 i of the chunk; blocks past
// the chunk, and rows past N, read zeros: offsets past num_records).
template <int BPL>
__device__ __forceinline__ void q8r_load(RBlocks &B, __amdgpu_buffer_rsrc_t rc, __amdgpu_buffer_rsrc_t rs, int row,
                                         int N, int K, int nb, int nbc, int c, int L) {
#pragma unroll
  for (int i = 0; i < BPL; i++) {
    const int b = L + 32 * i;
    const bool ok = b < nbc && row < N;
    const int g = c * nbc + b;
    const int oc = ok ? row * K + g * kQ : kRsrcOob;
    B.c[2 * i] = __builtin_amdgcn_raw_buffer_load_b128(rc, oc, 0, kAuxNT);
    B.c[2 * i + 1] = __builtin_amdgcn_raw_buffer_load_b128(rc, ok ? oc + 16 : kRsrcOob, 0, kAuxNT);
    B.s[i] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, ok ? (row * nb + g) * 4 : kRsrcOob, 0, 0));
  }
}

// The reference's leaf tree over each 32-lane half of a wave: offsets 16, 8,
// 4, 2, 1, v_i = v_i + v_{i+o}; lanes 0 and 32 end with their half's sum. The
// 16-step crosses 16-lane rows (the row-pair swap: the sum is commutative, so
// both rows get v_i + v_{i+16}); the others are DPP row shifts (lane i reads
// lane i + o of its row), in place of cross-lane permutes through LDS.
__device__ __forceinline__ float leaf_tree32(float v) {
  v = add_row_pair(v);
  v = v + dpp_f<0x108>(v);   // row_shl:8
  v = v + dpp_f<0x104>(v);   // row_shl:4
  v = v + dpp_f<0x102>(v);   // row_shl:2
  return v + dpp_f<0x101>(v);   // row_shl:1
}

template <int BPL>
__device__ __forceinline__ float q8r_leaf(const RBlocks &B, const float *__restrict__ xs, int nbc, int c, int L) {
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < BPL; i++) {
    const int b = L + 32 * i;
    // a block past the chunk has zero codes and scale: fmaf(0, 0, acc) = acc
    // exactly (acc is never -0), so it is folded without a branch
    const float *xb = xs + (size_t)(b < nbc ? c * nbc + b : 0) * kRXStride;
    const uint32_t w[8] = {(uint32_t)B.c[2 * i].x, (uint32_t)B.c[2 * i].y, (uint32_t)B.c[2 * i].z,
                           (uint32_t)B.c[2 * i].w, (uint32_t)B.c[2 * i + 1].x, (uint32_t)B.c[2 * i + 1].y,
                           (uint32_t)B.c[2 * i + 1].z, (uint32_t)B.c[2 * i + 1].w};
    float dot = 0.0f;
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const float4 x4 = *reinterpret_cast<const float4 *>(xb + 4 * q);
      dot = __builtin_fmaf((float)(int8_t)(w[q] & 0xffu), x4.x, dot);
      dot = __builtin_fmaf((float)(int8_t)((w[q] >> 8) & 0xffu), x4.y, dot);
      dot = __builtin_fmaf((float)(int8_t)((w[q] >> 16) & 0xffu), x4.z, dot);
      dot = __builtin_fmaf((float)(int8_t)(w[q] >> 24), x4.w, dot);
    }
    acc = __builtin_fmaf(B.s[i], dot, acc);
  }
  return acc;
}

}  // namespace pq
