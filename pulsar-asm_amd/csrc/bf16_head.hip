// bf16_head.hip -- the tied bf16 embedding table (gfx950): the embedding row of a
// token and the LM head over the table.
//
// The reference's exporter can keep the tied embedding as bf16 (dtype 3,
// export_lfm3_q8.py --emb-bf16); the engine then copies the token's row as it
// is (lfm3_nanode.cu:6062-6076) and runs the head as k_gemv_bf16 (3517-3534):
// per row, leaf L = 0..31 sums the products of elements L, L+32, L+64, ... in
// order, each product rounded before its add, and the 32 leaves combine as the
// shfl_down tree 16, 8, 4, 2, 1. The products of two bf16 values are exact in
// fp32, so only the adds round, and the result depends only on that order.
//
// Layout of the GEMV: a workgroup of 4 waves takes 16 rows, each wave two rows
// at a time (lanes 0-31 row a, lanes 32-63 row a + 1; lane & 31 is the leaf).
// x is widened to fp32 once per workgroup into LDS. A row pair's 2048-element
// slice is read with 16-byte loads (one 1 KB load per wave instruction, whole
// cache lines), stored to the wave's own LDS region, and each lane then walks
// its leaf's elements L, L+32, ... from LDS (the stride that a coalesced
// register load cannot give one lane); the next slice's loads are issued before
// this slice's walk. HBM-bound: 2 bytes per weight.
#include "pq_device.h"
#include "pq_host.h"

namespace pq {

constexpr int kB16Waves = 4;
constexpr int kB16Rows = 16;              // rows per workgroup
constexpr int kB16Slice = 2048;           // elements of a row per LDS slice
constexpr int kB16LoadsPerRow = kB16Slice * 2 / (64 * 16);   // 16-byte loads per lane per row slice: 4

typedef int b16v4 __attribute__((ext_vector_type(4)));

// The 16-byte pieces of rows r0 and r0 + 1, elements k0 .. k0 + 2047, that
// lane l loads: piece l + 64 i of row r0 + (i >= 4), i = 0..7 (rows past N and
// elements past K read zeros through the buffer resource's bound).
struct SliceRegs {
  b16v4 v[2 * kB16LoadsPerRow];
};

__device__ __forceinline__ void slice_load(SliceRegs &s, __amdgpu_buffer_rsrc_t w, int r0, int N, int K, int k0,
                                           int lane) {
#pragma unroll
  for (int i = 0; i < 2 * kB16LoadsPerRow; i++) {
    const int r = r0 + i / kB16LoadsPerRow;
    const int e = k0 + 8 * (lane + 64 * (i % kB16LoadsPerRow));   // first element of the piece
    const int off = (r < N && e < K) ? (int)(((size_t)r * K + e) * 2) : 0x7ffffff0;
    s.v[i] = __builtin_amdgcn_raw_buffer_load_b128(w, off, 0, 2);
  }
}

// Per workgroup: y for its rows and, with parts, the (y, row) of its rows'
// pick in k_argmax's order (am_better) at parts[2 * blockIdx.x].
__global__ __launch_bounds__(64 * kB16Waves) void bf16_gemv_kernel(const uint16_t *__restrict__ W,
                                                                     const uint16_t *__restrict__ x,
                                                                     float *__restrict__ y, int N, int K,
                                                                     float *__restrict__ parts) {
  extern __shared__ __align__(16) unsigned char smem[];
  float *xs = reinterpret_cast<float *>(smem);                                  // [K]
  uint16_t *ws = reinterpret_cast<uint16_t *>(smem + (size_t)K * 4);             // [waves][2][kB16Slice]
  __shared__ float bv[kB16Waves];
  __shared__ int bi[kB16Waves];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, leaf = lane & 31, half = lane >> 5;
  uint16_t *wl = ws + (size_t)wave * 2 * kB16Slice;
  const __amdgpu_buffer_rsrc_t wr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(W), (short)0, N * K * 2, 0x00020000);   // <= 0x7fff0000: below every rejected offset
  const int row0 = blockIdx.x * kB16Rows;
  const int nsl = (K + kB16Slice - 1) / kB16Slice;
  const int npairs = kB16Rows / (2 * kB16Waves);   // row pairs per wave: 2
  // the first slice's loads go out before x is staged
  SliceRegs cur;
  slice_load(cur, wr, row0 + 2 * wave, N, K, 0, lane);
  for (int i = threadIdx.x; i < K; i += 64 * kB16Waves) xs[i] = bf2f(x[i]);
  __syncthreads();
  float best = kAmFloor;
  int besti = -1;
  for (int pp = 0; pp < npairs; pp++) {
    const int ra = row0 + 2 * wave + 2 * kB16Waves * pp;   // this pass's row pair: ra, ra + 1
    float s = 0.0f;
    for (int sl = 0; sl < nsl; sl++) {
      // stage the slice in the wave's LDS region: row h at wl + h * kB16Slice
#pragma unroll
      for (int i = 0; i < 2 * kB16LoadsPerRow; i++)
        *reinterpret_cast<b16v4 *>(wl + (i / kB16LoadsPerRow) * kB16Slice + 8 * (lane + 64 * (i % kB16LoadsPerRow))) =
            cur.v[i];
      // the next slice (or the next pair's first slice) loads while this one is walked
      const bool more = sl + 1 < nsl || pp + 1 < npairs;
      if (more) {
        if (sl + 1 < nsl) slice_load(cur, wr, ra, N, K, (sl + 1) * kB16Slice, lane);
        else slice_load(cur, wr, ra + 2 * kB16Waves, N, K, 0, lane);
      }
      const uint16_t *wrow = wl + half * kB16Slice;
      const float *xk = xs + sl * kB16Slice;
      const int n = min(kB16Slice, K - sl * kB16Slice);
      for (int k = leaf; k < n; k += 32) {
        const float p = bf2f(wrow[k]) * xk[k];
        s = s + p;
      }
    }
    // the leaf tree within each 32-lane row: leaf i += leaf i + o, o = 16 .. 1
#pragma unroll
    for (int o = 16; o > 0; o >>= 1) s = s + __shfl_down(s, o, 32);
    const int r = ra + half;
    if (leaf == 0 && r < N) {
      y[r] = s;
      float cv;
      int ci;
      am_leaf(s, r, cv, ci);
      if (am_better(cv, ci, best, besti)) { best = cv; besti = ci; }
    }
  }
  if (parts == nullptr) return;
  // (value, row) of the workgroup's pick in k_argmax's order (am_better)
  {
    const float ov = __shfl(best, 32, 64);
    const int oi = __shfl(besti, 32, 64);
    if (am_better(ov, oi, best, besti)) { best = ov; besti = oi; }
  }
  if (lane == 0) { bv[wave] = best; bi[wave] = besti; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float v = bv[0];
    int idx = bi[0];
    for (int w = 1; w < kB16Waves; w++)
      if (am_better(bv[w], bi[w], v, idx)) { v = bv[w]; idx = bi[w]; }
    parts[2 * blockIdx.x] = v;
    parts[2 * blockIdx.x + 1] = __int_as_float(idx);
  }
}

// Rows of T token ids from the bf16 table, copied as stored; an id outside
// [0, vocab) gives a zero row. One workgroup per position, 8 bytes per thread.
__global__ void embed_bf16_kernel(const uint16_t *__restrict__ table, const int32_t *__restrict__ tokens,
                                  uint16_t *__restrict__ out, int H, int vocab) {
  const int t = blockIdx.x, id = tokens[t];
  const bool ok = id >= 0 && id < vocab;
  for (int i = threadIdx.x * 4; i < H; i += blockDim.x * 4) {
    const uint2 v = ok ? *reinterpret_cast<const uint2 *>(table + (size_t)id * H + i) : make_uint2(0u, 0u);
    *reinterpret_cast<uint2 *>(out + (size_t)t * H + i) = v;
  }
}

}  // namespace pq

using namespace pq;

extern "C" int pq_bf16_gemv_parts(int N) { return N > 0 ? (N + kB16Rows - 1) / kB16Rows : 0; }

extern "C" int pq_bf16_gemv(const uint16_t *W, const uint16_t *x, float *y, int N, int K, float *argmax_parts,
                            void *stream) {
  PQ_REQUIRE(W && x && y, PQ_ERR_ARG, "pq_bf16_gemv: null pointer");
  PQ_REQUIRE(N > 0 && K >= 32 && K % 32 == 0 && K <= 16384, PQ_ERR_ARG, "pq_bf16_gemv: N=%d K=%d (K a multiple of 32, "
             "at most 16384)", N, K);
  PQ_REQUIRE((long long)N * K * 2 <= 0x7fff0000ll, PQ_ERR_ARG, "pq_bf16_gemv: N=%d K=%d: the table exceeds 2 GiB", N,
             K);
  PQ_REQUIRE(aligned(W, 16) && aligned(x, 4) && aligned(y, 4), PQ_ERR_ALIGN, "pq_bf16_gemv: alignment");
  const size_t lds = (size_t)K * 4 + (size_t)kB16Waves * 2 * kB16Slice * 2;
  const dim3 grid((unsigned)((N + kB16Rows - 1) / kB16Rows)), block(64 * kB16Waves);
  launch(bf16_gemv_kernel, grid, block, lds, as_stream(stream), W, x, y, N, K, argmax_parts);
  return check_launch("pq_bf16_gemv");
}

extern "C" int pq_embed_bf16(const uint16_t *table, const int32_t *tokens, uint16_t *out, int H, int vocab, int T,
                             void *stream) {
  PQ_REQUIRE(table && tokens && out && H > 0 && H % 4 == 0 && vocab > 0 && T > 0, PQ_ERR_ARG,
             "pq_embed_bf16: bad arguments (H=%d vocab=%d T=%d)", H, vocab, T);
  PQ_REQUIRE(aligned(table, 8) && aligned(out, 8), PQ_ERR_ALIGN, "pq_embed_bf16: alignment");
  launch(embed_bf16_kernel, dim3((unsigned)T), dim3(256), 0, as_stream(stream), table, tokens, out, H, vocab);
  return check_launch("pq_embed_bf16");
}
