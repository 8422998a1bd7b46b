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

#include <mutex>
#include <type_traits>

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
  int q = (int)__builtin_rintf(v / (d != 0.0f ? d : 1.0f));   // d = 0: the block is all zero (q = 0)
  q = q > 127 ? 127 : (q < -127 ? -127 : q);
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
// Persistent workgroups of 8 waves. A work item is a group of 8 32-row slices
// (256 rows) x one K split x one 32-position block; wave w of the workgroup
// takes slice w of the group and walks the split's chunks in order, so each
// output's chunk partials fold into y = y + a_c in registers -- no barrier
// between waves. The activations of 8 chunks (2048 K) x 32 positions (64 KB)
// and their dx sit in LDS, shared by the 8 waves; they are re-staged only when
// the chunks or positions move out of them (with K <= 2048, one split and
// T <= 32: once per workgroup). Each wave keeps the weights of its next two
// chunks in flight -- across item boundaries -- while it computes one. Per
// block one v_mfma_i32_32x32x32_i8 with A = activations (i = position) and B =
// weights (j = row): lane l holds D[i][j] for j = l % 32 and
// i = 8(r/4) + 4(l/32) + r%4 (r = 0..15), and folds its 16 outputs into the
// chunk partial a = fmaf(fl(dw*dx), (float)isum, a).
// Several K splits (small N): every chunk partial goes to the workspace
// [nch][T][N] and q8_gemm_fold_kernel adds them in chunk order.
// Weights and scales come through buffer resources (rows past N and absent
// chunks read zeros, no branch).
// One chunk (up to 8 blocks) of a 32 x 32 (position x row) MFMA tile into the
// lane's 16 chunk partials: per block b one v_mfma_i32_32x32x32_i8 (A = the
// activations AV(b), B = the weights w[b]), then a = fmaf(fl(dw*dx), (float)isum, a)
// for the lane's 16 outputs (row = lane % 32, positions 8(r/4) + 4(lane/32) + r%4;
// dx of block b at dxs[kb0 + b][position]). Block b+1's MFMA and LDS reads are
// issued before block b's fold, so the matrix core and the LDS work while the
// VALU folds; the fold order per output is unchanged.
// The pipelined form: block b+1's MFMA is issued, then block b+2's activations
// and block b+1's dx are read from LDS, then block b is folded -- so each LDS
// read has a whole fold to arrive in, and the MFMA result it folds was issued
// one fold earlier. The scheduling barriers keep the reads ahead of the fold.
// NB = kCB compiles the whole-chunk case without the per-block bounds. Only
// the first NQ position quads (outputs a[0 .. 4*NQ)) are folded: NQ = 2 when
// the tile's A operand holds 16 positions.
template <int NB, int NQ, typename AF>
__device__ __forceinline__ void mfma_chunk_pipe(float *a, const v4i *w, const v4i sv, AF AV,
                                                const float (*dxs)[32], int kb0, int h, int nbc_rt) {
  const int nbc = NB ? NB : nbc_rt;
  const uint32_t sw[4] = {(uint32_t)sv.x, (uint32_t)sv.y, (uint32_t)sv.z, (uint32_t)sv.w};
  const v16i zero = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  v16i acc[2];
  f4v d[2][4];
  v4i an;   // the activations of the next block's MFMA
  const lds_ptr<f4v> dp = lds_base(reinterpret_cast<const f4v *>(&dxs[kb0][4 * h]));   // block i, q: dp[8i + 2q]
  if (nbc > 0) {
    acc[0] = __builtin_amdgcn_mfma_i32_32x32x32_i8(AV(0), w[0], zero, 0, 0, 0);
    if (nbc > 1) an = AV(1);
#pragma unroll
    for (int q = 0; q < NQ; q++) d[0][q] = dp[2 * q];
  }
#pragma unroll
  for (int i = 0; i < kCB; i++) {
    if (i + 1 < kCB && i + 1 < nbc) {
      acc[(i + 1) & 1] = __builtin_amdgcn_mfma_i32_32x32x32_i8(an, w[i + 1], zero, 0, 0, 0);
      if (i + 2 < kCB && i + 2 < nbc) an = AV(i + 2);
#pragma unroll
      for (int q = 0; q < NQ; q++) d[(i + 1) & 1][q] = dp[8 * (i + 1) + 2 * q];
    }
    __builtin_amdgcn_sched_barrier(0);
    if (i < nbc) {
      const float dw = half_of(sw[i >> 1], i & 1);
      const v16i &ac = acc[i & 1];
#pragma unroll
      for (int q = 0; q < NQ; q++) {
        const float dq[4] = {d[i & 1][q].x, d[i & 1][q].y, d[i & 1][q].z, d[i & 1][q].w};
#pragma unroll
        for (int k = 0; k < 4; k++) a[4 * q + k] = __builtin_fmaf(dw * dq[k], (float)ac[4 * q + k], a[4 * q + k]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

template <bool PIPE, int NQ = 4, typename AF>
__device__ __forceinline__ void mfma_chunk(float *a, const v4i *w, const v4i sv, AF AV, const float (*dxs)[32],
                                           int kb0, int h, int nbc) {
  if constexpr (!PIPE) {   // one MFMA result live at a time (for a tight register budget)
    const uint32_t sw[4] = {(uint32_t)sv.x, (uint32_t)sv.y, (uint32_t)sv.z, (uint32_t)sv.w};
#pragma unroll
    for (int i = 0; i < kCB; i++) {
      if (i < nbc) {
        v16i acc = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(AV(i), w[i], acc, 0, 0, 0);
        const float dw = half_of(sw[i >> 1], i & 1);
#pragma unroll
        for (int q = 0; q < NQ; q++) {
          const float4 d4 = *reinterpret_cast<const float4 *>(&dxs[kb0 + i][8 * q + 4 * h]);
          const float dq[4] = {d4.x, d4.y, d4.z, d4.w};
#pragma unroll
          for (int k = 0; k < 4; k++) a[4 * q + k] = __builtin_fmaf(dw * dq[k], (float)acc[4 * q + k], a[4 * q + k]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    return;
  }
  if (nbc == kCB) mfma_chunk_pipe<kCB, NQ>(a, w, sv, AV, dxs, kb0, h, kCB);   // whole chunks: no branches
  else mfma_chunk_pipe<0, NQ>(a, w, sv, AV, dxs, kb0, h, nbc);
}

constexpr int kGemmWaves = 8;
constexpr int kGemmThreads = 64 * kGemmWaves;
constexpr int kGemmSegChunks = 8;                          // chunks of K staged at once
constexpr int kGemmSegK = kGemmSegChunks * kCB * kQ;       // 2048
constexpr int kGemmARow = kGemmSegK + 16;                  // padded LDS row (bytes)
constexpr size_t kGemmLds = 32 * (size_t)kGemmARow + (size_t)kGemmSegChunks * kCB * 32 * 4;

struct GemmW {
  v4i w[kCB];
  v4i s;
};

struct GemmCur {     // one chunk step of a wave: item it, 32-row slice, chunk c
  int it, slice, c0, c1, p0, c;
  bool ok;
};

__global__ __launch_bounds__(kGemmThreads) void q8_gemm_kernel(const int8_t *__restrict__ pc,
                                                                const uint16_t *__restrict__ ps,
                                                                const int8_t *__restrict__ qx,
                                                                const float *__restrict__ dx, void *__restrict__ y,
                                                                int y_bf16, int N, int K, int T,
                                                                float *__restrict__ ws, int cps) {
  extern __shared__ __align__(16) unsigned char gsm[];
  int8_t(*as)[kGemmARow] = reinterpret_cast<int8_t(*)[kGemmARow]>(gsm);              // [32 positions]
  float(*dxs)[32] = reinterpret_cast<float(*)[32]>(gsm + 32 * kGemmARow);            // [64 blocks][32]
  const int nb = K / kQ, nch = nchunks(K);
  const int nsl = (N + 31) / 32, ngr = (nsl + kGemmWaves - 1) / kGemmWaves;
  const int S = (nch + cps - 1) / cps;
  const int P = (T + 31) / 32, nitems = ngr * S * P;
  // Item it -> (group, split) gs and position block pb. Workgroups are placed
  // on the 8 XCDs round-robin (XCD = id % 8) and a workgroup's items are
  // gridDim.x apart, so with several position blocks the items are laid out to
  // give the P position blocks of one (group, split) to P workgroups of one
  // XCD at the same time: the group's weights are read from HBM once and from
  // that XCD's L2 P-1 times, and each workgroup keeps its position block's
  // activations. A bijection on [0, nitems) whenever 8 divides ngr * S.
  const bool xcd_map = P > 1 && (ngr * S) % 8 == 0;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int h = lane >> 5, l32 = lane & 31;
  if ((int)blockIdx.x >= nitems) return;
  auto item = [&](int it, GemmCur &g) {
    int gs, pb;
    if (xcd_map) {
      const int j = it >> 3;
      pb = j % P;
      gs = (j / P) * 8 + (it & 7);
    } else {
      gs = it % (ngr * S);
      pb = it / (ngr * S);
    }
    const int gr = gs % ngr, s = gs / ngr;
    g.it = it;
    g.slice = gr * kGemmWaves + wave;
    g.p0 = pb * 32;
    g.c0 = s * cps;
    g.c1 = min(nch, g.c0 + cps);
    g.c = g.c0;
  };
  auto next = [&](GemmCur g) {
    if (!g.ok) return g;
    if (++g.c >= g.c1) {
      const int it = g.it + (int)gridDim.x;
      g.ok = it < nitems;
      if (g.ok) item(it, g);
    }
    return g;
  };
  auto wload = [&](GemmW &w, const GemmCur &g) {
    const bool live = g.ok && g.slice < nsl;
    const int tile = live ? g.slice >> 1 : 0;
    const int jt = (g.slice & 1) * 32 + l32;
    const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int8_t *>(pc + (size_t)tile * nb * kSlab), (short)0, live ? nb * kSlab : 0, kRsrcWord3);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(ps + (size_t)tile * nch * kTR * 8), (short)0, live ? nch * kTR * 16 : 0, kRsrcWord3);
    const int oc = g.c * kCB * kSlab + (h * kTR + jt) * 16;
#pragma unroll
    for (int i = 0; i < kCB; i++) w.w[i] = __builtin_amdgcn_raw_buffer_load_b128(rc, oc + i * kSlab, 0, kAuxNT);
    w.s = __builtin_amdgcn_raw_buffer_load_b128(rs, (g.c * kTR + jt) * 16, 0, 0);
  };
  GemmCur g0;
  g0.ok = true;
  item(blockIdx.x, g0);
  GemmCur g1 = next(g0);
  GemmW wa, wb, wc;   // the three chunk buffers of the pipeline, rotated by name (see below)
  int seg_k = -1, seg_c1 = 0, seg_p = -1;   // staged chunks [seg_k, min(seg_k + 8, seg_c1)), position block
  float yv[16];
#pragma unroll
  for (int r = 0; r < 16; r++) yv[r] = 0.0f;
  // One chunk step of the wave. Loads are issued in the order they are needed:
  // a new segment's activations first, then (first step only) the weights of
  // chunks 0 and 1, then the weights two chunks ahead -- so staging waits only
  // on the activations. The first step is a separate copy (FIRST) so every
  // wait the compiler places stays exact. w0 holds the weights of the chunk
  // computed, w1 and w2 those of the next two; the loop below passes the three
  // buffers in rotated order instead of copying them, since a copy of a
  // register that a load is still filling waits for that load.
  auto step = [&](auto FIRST, GemmW &w0, GemmW &w1, GemmW &w2) -> bool {
    const int c = g0.c;
    // activations and dx: the 8 chunks from c of position block p0 (uniform:
    // every wave of the workgroup walks the same chunk sequence)
    const bool restage =
        seg_k < 0 || c < seg_k || c >= seg_k + kGemmSegChunks || c >= seg_c1 || g0.p0 != seg_p;
    const bool had = seg_k >= 0;
    v4i av[8];
    float dv[4];
    const int t = threadIdx.x;
    if (restage) {
      seg_k = c;
      seg_c1 = g0.c1;
      seg_p = g0.p0;
      const int np = T - seg_p < 32 ? T - seg_p : 32;
      const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<int8_t *>(qx + (size_t)seg_p * K), (short)0, np * K, kRsrcWord3);
      const __amdgpu_buffer_rsrc_t rdx = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<float *>(dx + (size_t)seg_p * nb), (short)0, np * nb * 4, kRsrcWord3);
      const int kb0 = seg_k * kCB * kQ;          // byte offset of the segment in a row
      const int kend = min(K, min(g0.c1, seg_k + kGemmSegChunks) * kCB * kQ);   // the item's part of it
      const int bend = kend / kQ;
#pragma unroll
      for (int i = 0; i < 8; i++) {              // 32 rows x 128 pieces of 16 B: thread t, pieces t + 512 i
        const int pc16 = t + i * kGemmThreads;
        const int p = pc16 >> 7, q = pc16 & 127;
        av[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, kb0 + q * 16 < kend ? p * K + kb0 + q * 16 : kRsrcOob, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {              // 32 positions x 64 blocks: thread t, entries t + 512 i
        const int e = t + i * kGemmThreads;
        const int p = e >> 6, b = seg_k * kCB + (e & 63);
        dv[i] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rdx, b < bend ? (p * nb + b) * 4 : kRsrcOob, 0, 0));
      }
    }
    auto stage_store = [&]() {
      if (had) lds_barrier();   // every wave is done with the previous segment
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const int pc16 = t + i * kGemmThreads;
        *reinterpret_cast<v4i *>(&as[pc16 >> 7][(pc16 & 127) * 16]) = av[i];
      }
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int e = t + i * kGemmThreads;
        dxs[e & 63][e >> 6] = dv[i];
      }
      lds_barrier();
    };
    GemmCur g2;
    if constexpr (decltype(FIRST)::value) {
      // first step: only chunk 0's weights go out with the activations (a
      // deeper prefetch from every CU queues ahead of them in memory)
      wload(w0, g0);
      stage_store();
      wload(w1, g1);
      g2 = next(g1);
      wload(w2, g2);
    } else {
      g2 = next(g1);
      wload(w2, g2);
      if (restage) stage_store();
    }
    // chunk c of this wave's slice
    float a[16];
#pragma unroll
    for (int r = 0; r < 16; r++) a[r] = 0.0f;
    {
      const int kb0 = (c - seg_k) * kCB;   // the chunk's first block within the staged segment
      const lds_ptr<v4i> ap = lds_base(reinterpret_cast<const v4i *>(&as[l32][kb0 * kQ + 16 * h]));
      auto AV = [&](int i) { return ap[2 * i]; };   // block i: 32 bytes on
      mfma_chunk<true>(a, w0.w, w0.s, AV, dxs, kb0, h, min(kCB, nb - c * kCB));
    }
    const int row = g0.slice * 32 + l32;
    if (ws == nullptr) {
#pragma unroll
      for (int r = 0; r < 16; r++) yv[r] = yv[r] + a[r];
      if (c + 1 >= g0.c1) {   // the slice's last chunk: write y
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int pos = g0.p0 + 8 * (r >> 2) + 4 * h + (r & 3);
          if (pos < T && row < N) {
            if (y_bf16) reinterpret_cast<uint16_t *>(y)[(size_t)pos * N + row] = f2bf(yv[r]);
            else reinterpret_cast<float *>(y)[(size_t)pos * N + row] = yv[r];
          }
          yv[r] = 0.0f;
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int pos = g0.p0 + 8 * (r >> 2) + 4 * h + (r & 3);
        if (pos < T && row < N) ws[((size_t)c * T + pos) * N + row] = a[r];
      }
    }
    if (!g1.ok) return false;
    g0 = g1;
    g1 = g2;
    return true;
  };
  const std::integral_constant<bool, false> rest;
  if (step(std::integral_constant<bool, true>{}, wa, wb, wc))
    while (step(rest, wb, wc, wa) && step(rest, wc, wa, wb) && step(rest, wa, wb, wc)) {
    }
}

// The tile-parallel form (small and mid-sized N): a workgroup = S 32-row
// slices x 32 positions, 8*S waves; wave w takes slice w % S and chunk
// 8*rd + w / S of round rd, so a round's 8 chunks of every slice load at once.
// Per round the 32 positions' activations (2048 K) and dx are loaded first,
// then the wave's weights, so the staging waits only on the activations; the
// 8 chunk partials then fold into y through LDS in chunk order (the partials
// reuse the activation buffer once every wave has read it, which leaves room
// for two workgroups per CU). Same numerics as the walking form.
// PH = 16 gives a workgroup 16 positions (the A operand's other 16 rows read
// zeros and their outputs are neither folded nor written): twice the
// workgroups and half the fold per wave, for GEMMs with few slices. AUX is the
// weight loads' cache policy: nontemporal, or cached where many position
// blocks' workgroups re-read the same weights.
constexpr int kTileSlots = 8;
constexpr size_t kTileActBytes = 32 * (size_t)kGemmARow;
constexpr size_t kTileLds = kTileActBytes + (size_t)kTileSlots * kCB * 32 * 4;

template <int S, bool PIPE, int PH = 32, int AUX = kAuxNT>
__global__ __launch_bounds__(64 * kTileSlots * S) void q8_gemm_tile_kernel(const int8_t *__restrict__ pc,
                                                                        const uint16_t *__restrict__ ps,
                                                                        const int8_t *__restrict__ qx,
                                                                        const float *__restrict__ dx,
                                                                        void *__restrict__ y, int y_bf16, int N,
                                                                        int K, int T) {
  constexpr int NT = 64 * kTileSlots * S;
  constexpr int APT = 32 * (kGemmSegK / 16) / NT;   // 16-byte activation pieces per thread per round
  constexpr int DPT = 32 * kTileSlots * kCB / NT;   // dx entries per thread per round
  static_assert(kTileSlots * S * 16 * 64 * 4 <= kTileActBytes, "partials must fit the activation buffer");
  extern __shared__ __align__(16) unsigned char gsm[];
  int8_t(*as)[kGemmARow] = reinterpret_cast<int8_t(*)[kGemmARow]>(gsm);
  float(*part)[S][16][64] = reinterpret_cast<float(*)[S][16][64]>(gsm);   // aliases as
  float(*dxs)[32] = reinterpret_cast<float(*)[32]>(gsm + kTileActBytes);
  const int nb = K / kQ, nch = nchunks(K);
  static_assert(PH == 32 || PH == 16, "16 or 32 positions per workgroup");
  constexpr int NQ = PH / 8;                          // position quads folded per lane
  const int p0 = blockIdx.z * PH;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int sub = wave % S, slot = wave / S;
  const int h = lane >> 5, l32 = lane & 31;
  const int sl = blockIdx.x * S + sub;                 // 32-row slice
  const bool live = sl * 32 < N;
  const int tile = live ? sl >> 1 : 0, jt = (sl & 1) * 32 + l32;
  const int np = T - p0 < PH ? T - p0 : PH;   // rows past np of the A operand read zeros
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t *>(pc + (size_t)tile * nb * kSlab), (short)0, live ? nb * kSlab : 0, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(ps + (size_t)tile * nch * kTR * 8), (short)0, live ? nch * kTR * 16 : 0, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<int8_t *>(qx + (size_t)p0 * K), (short)0, np * K, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rdx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(dx + (size_t)p0 * nb), (short)0, np * nb * 4, kRsrcWord3);
  const int nrounds = (nch + kTileSlots - 1) / kTileSlots;
  const int t = threadIdx.x;
  float yv[2] = {0.0f, 0.0f};
  for (int rd = 0; rd < nrounds; rd++) {
    const int rbase = rd * kTileSlots;
    const int c = rbase + slot;
    const bool valid = c < nch;
    // the round's activations (piece q = t + NT*i: position q / 128, bytes
    // 16*(q % 128) of the round's 2048) and dx, then this wave's weights
    v4i av[APT];
#pragma unroll
    for (int i = 0; i < APT; i++) {
      const int q = t + NT * i, p = q >> 7, col = rbase * kCB * kQ + (q & 127) * 16;
      av[i] = __builtin_amdgcn_raw_buffer_load_b128(ra, col < K ? p * K + col : kRsrcOob, 0, 0);
    }
    float dv[DPT];
#pragma unroll
    for (int i = 0; i < DPT; i++) {
      const int e = t + NT * i, p = e >> 6, b = rbase * kCB + (e & 63);
      dv[i] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rdx, b < nb ? (p * nb + b) * 4 : kRsrcOob, 0, 0));
    }
    v4i wv[kCB];
    const int oc = valid ? c * kCB * kSlab + (h * kTR + jt) * 16 : kRsrcOob;
#pragma unroll
    for (int i = 0; i < kCB; i++) wv[i] = __builtin_amdgcn_raw_buffer_load_b128(rc, oc + i * kSlab, 0, AUX);
    const v4i sv = __builtin_amdgcn_raw_buffer_load_b128(rs, valid ? (c * kTR + jt) * 16 : kRsrcOob, 0, 0);
    if (rd > 0) lds_barrier();   // the previous round's fold reads of the partials are done
#pragma unroll
    for (int i = 0; i < APT; i++) {
      const int q = t + NT * i;
      *reinterpret_cast<v4i *>(&as[q >> 7][(q & 127) * 16]) = av[i];
    }
#pragma unroll
    for (int i = 0; i < DPT; i++) {
      const int e = t + NT * i;
      dxs[e & 63][e >> 6] = dv[i];
    }
    lds_barrier();
    float a[16];
#pragma unroll
    for (int r = 0; r < 16; r++) a[r] = 0.0f;
    if (valid) {
      const int kb0 = slot * kCB;
      const lds_ptr<v4i> ap = lds_base(reinterpret_cast<const v4i *>(&as[l32][kb0 * kQ + 16 * h]));
      auto AV = [&](int i) { return ap[2 * i]; };   // block i: 32 bytes on
      mfma_chunk<PIPE, NQ>(a, wv, sv, AV, dxs, kb0, h, min(kCB, nb - c * kCB));
    }
    lds_barrier();   // every wave is done with the activations: the partials overwrite them
#pragma unroll
    for (int r = 0; r < 16; r++) part[slot][sub][r][lane] = a[r];
    lds_barrier();
    const int n = nch - rbase < kTileSlots ? nch - rbase : kTileSlots;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      const int e = t + k * NT;
      const int s2 = e >> 10, r = (e >> 6) & 15, l = e & 63;
      if ((r >> 2) < NQ)
        for (int w = 0; w < n; w++) yv[k] = yv[k] + part[w][s2][r][l];
    }
  }
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int e = t + k * NT;
    const int s2 = e >> 10, r = (e >> 6) & 15, l = e & 63;
    const int pos = p0 + 8 * (r >> 2) + 4 * (l >> 5) + (r & 3);
    const int row = (blockIdx.x * S + s2) * 32 + (l & 31);
    if ((r >> 2) < NQ && pos < T && row < N) {
      if (y_bf16) reinterpret_cast<uint16_t *>(y)[(size_t)pos * N + row] = f2bf(yv[k]);
      else reinterpret_cast<float *>(y)[(size_t)pos * N + row] = yv[k];
    }
  }
}

// y[pos][row] = sum over chunks of the workspace partials, chunk order, from 0.
__global__ __launch_bounds__(256) void q8_gemm_fold_kernel(const float *__restrict__ ws, void *__restrict__ y,
                                                            int y_bf16, long long TN, int nch) {
  const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= TN) return;
  float v = 0.0f;
  for (int c0 = 0; c0 < nch; c0 += 8) {   // 8 loads in flight, then their adds in chunk order
    float p[8];
#pragma unroll
    for (int k = 0; k < 8; k++) p[k] = c0 + k < nch ? ws[(size_t)(c0 + k) * TN + i] : 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++)
      if (c0 + k < nch) v = v + p[k];
  }
  if (y_bf16) reinterpret_cast<uint16_t *>(y)[i] = f2bf(v);
  else reinterpret_cast<float *>(y)[i] = v;
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

// K splits for the T-wide GEMM: with a workspace, enough 8-slice work items
// to give every CU one.
static int gemm_splits(int N, int K, int T, bool have_ws) {
  const int nch = nchunks(K), tb = (T + 31) / 32;
  const long long items = (long long)((N + 255) / 256) * tb;
  int cps = nch;
  if (have_ws)
    while (cps > 1 && items * ((nch + cps - 1) / cps) < 256) cps = (cps + 1) / 2;
  return cps;
}

// Which form runs a T-wide GEMM: 1 = the walking form (persistent, split K
// with a workspace), 2 = tile form over 64-row tiles, 3 = tile form over 32-row
// slices. PQ_GEMM_FORM (1..3) overrides the choice.
enum { kFormWalk = 1, kFormTile = 2, kFormSlice = 3 };
// Measured on the LFM-style shapes (hidden 2048): 32-row slices win at one
// position block with K <= 2048 (one round), the walking form for the LM head
// and for deeper K at one position block (split over workgroups), 64-row
// tiles for mid-sized N over many position blocks.
static int gemm_form(int N, int K, int T) {
  static const int env = env_int("PQ_GEMM_FORM");
  if (env >= kFormWalk && env <= kFormSlice) return env;
  if (N >= 32768) return kFormWalk;
  if (T <= 32) return K > kGemmSegK ? kFormWalk : kFormSlice;
  return N >= 16384 ? kFormWalk : kFormTile;
}

extern "C" size_t pq_q8_gemm_workspace_bytes(int N, int K, int T) {
  if (N <= 0 || K <= 0 || K % kQ || T <= 0) return 0;
  if (gemm_form(N, K, T) != kFormWalk) return 0;
  const int nch = nchunks(K);
  return gemm_splits(N, K, T, true) < nch ? (size_t)nch * T * N * sizeof(float) : 0;
}

extern "C" int pq_q8_gemm_ws(const int8_t *pcodes, const uint16_t *pscales, const int8_t *qx, const float *dx, void *y,
                             int y_dtype, int N, int K, int T, void *ws, size_t ws_bytes, void *stream) {
  PQ_REQUIRE(pcodes && pscales && qx && dx && y, PQ_ERR_ARG, "pq_q8_gemm: null pointer");
  PQ_REQUIRE(N > 0 && K > 0 && K % kQ == 0 && T > 0, PQ_ERR_ARG, "pq_q8_gemm: N=%d K=%d T=%d", N, K, T);
  PQ_REQUIRE(y_dtype == PQ_DTYPE_F32 || y_dtype == PQ_DTYPE_BF16, PQ_ERR_ARG, "pq_q8_gemm: y_dtype %d", y_dtype);
  PQ_REQUIRE(aligned(pcodes, 16) && aligned(pscales, 16) && aligned(qx, 16) && aligned(dx, 4), PQ_ERR_ALIGN,
             "pq_q8_gemm: packed weights and qx must be 16-byte aligned");
  PQ_REQUIRE((long long)T * K < (1ll << 31) && (long long)ntiles(N) * (K / kQ) * kSlab < (1ll << 31), PQ_ERR_ARG,
             "pq_q8_gemm: N=%d K=%d T=%d too large", N, K, T);
  const int nch = nchunks(K);
  const size_t need = pq_q8_gemm_workspace_bytes(N, K, T);
  const bool split = ws != nullptr && need > 0 && ws_bytes >= need;
  const int cps = gemm_splits(N, K, T, split);
  const int S = (nch + cps - 1) / cps;
  const long long items = (long long)((N + 255) / 256) * S * ((T + 31) / 32);
  PQ_REQUIRE(items < (1ll << 31), PQ_ERR_ARG, "pq_q8_gemm: N=%d T=%d too large", N, T);
  const int yb = y_dtype == PQ_DTYPE_BF16 ? 1 : 0;
  hipStream_t st = as_stream(stream);
  const int form = gemm_form(N, K, T);
  if (form == kFormTile) {   // with 8+ position blocks the weights' re-reads are served from cache (measured)
    const dim3 grid((unsigned)ntiles(N), 1, (unsigned)((T + 31) / 32));
    if (grid.z >= 8)
      launch(q8_gemm_tile_kernel<2, false, 32, 0>, grid, dim3(64 * kTileSlots * 2), kTileLds, st, pcodes, pscales, qx,
             dx, y, yb, N, K, T);
    else
      launch(q8_gemm_tile_kernel<2, false>, grid, dim3(64 * kTileSlots * 2), kTileLds, st, pcodes, pscales, qx, dx, y,
             yb, N, K, T);
    return check_launch("pq_q8_gemm");
  }
  if (form == kFormSlice) {
    // the pipelined fold holds two MFMA results (one workgroup per CU): worth it
    // while there is at most one workgroup per CU anyway; with at most 128
    // (slice, 32 positions) items, 16 positions per workgroup spread them over
    // twice the CUs (PQ_GEMM_PH = 32 / 16 overrides)
    static const int env_ph = env_int("PQ_GEMM_PH");
    const long long items32 = (long long)((N + 31) / 32) * ((T + 31) / 32);
    if (env_ph != 32 && (env_ph == 16 ? items32 <= 256 : items32 <= 128))
      launch(q8_gemm_tile_kernel<1, true, 16>, dim3((unsigned)((N + 31) / 32), 1, (unsigned)((T + 15) / 16)),
             dim3(64 * kTileSlots), kTileLds, st, pcodes, pscales, qx, dx, y, yb, N, K, T);
    else if (items32 <= 256)
      launch(q8_gemm_tile_kernel<1, true>, dim3((unsigned)((N + 31) / 32), 1, (unsigned)((T + 31) / 32)),
             dim3(64 * kTileSlots), kTileLds, st, pcodes, pscales, qx, dx, y, yb, N, K, T);
    else
      launch(q8_gemm_tile_kernel<1, false>, dim3((unsigned)((N + 31) / 32), 1, (unsigned)((T + 31) / 32)),
             dim3(64 * kTileSlots), kTileLds, st, pcodes, pscales, qx, dx, y, yb, N, K, T);
    return check_launch("pq_q8_gemm");
  }
  const unsigned grid = (unsigned)(items < 256 ? items : 256);   // one persistent workgroup per CU
  launch(q8_gemm_kernel, dim3(grid), dim3(kGemmThreads), kGemmLds, st, pcodes, pscales, qx, dx, y, yb, N, K, T,
         split ? static_cast<float *>(ws) : nullptr, cps);
  int rc = check_launch("pq_q8_gemm");
  if (rc || !split) return rc;
  const long long TN = (long long)T * N;
  launch(q8_gemm_fold_kernel, dim3((unsigned)((TN + 255) / 256)), dim3(256), 0, st, static_cast<const float *>(ws), y,
         yb, TN, nch);
  return check_launch("pq_q8_gemm fold");
}

extern "C" int pq_q8_gemm(const int8_t *pcodes, const uint16_t *pscales, const int8_t *qx, const float *dx, void *y,
                          int y_dtype, int N, int K, int T, void *stream) {
  return pq_q8_gemm_ws(pcodes, pscales, qx, dx, y, y_dtype, N, K, T, nullptr, 0, stream);
}

// ------------------------------------------------- the allocation-free GEMM
// pq_q8_gemm_ws with its split-K partials in a library-owned device array
// instead of a caller workspace, for callers that cannot allocate. The array
// is one per GPU (each device gets its own copy of the module's globals) and
// lives until the process ends. Its device address comes from
// hipGetSymbolAddress once per device, with that device current, and only
// that address is ever handed to kernels: in host code `scratch` names a
// host-side stand-in, not device memory.
namespace pq {
constexpr size_t kScratchBytes = (size_t)16 << 20;   // 16 MiB per GPU
static __device__ __align__(256) float scratch[kScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void *g_scratch_ptr[kMaxDevices];

// The scratch array's device address on the current device (looked up on the
// first call there). The stream, if given, must belong to the current device.
static int scratch_address(hipStream_t st, void **out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(PQ_ERR_LAUNCH, "pq_q8_gemm_noalloc: no current device");
  if (st != nullptr) {
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(st, &sdev) != hipSuccess || sdev != dev)
      return fail(PQ_ERR_ARG, "pq_q8_gemm_noalloc: the stream does not belong to the current device %d", dev);
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    // the lookup is a runtime call that a stream capture must not record or
    // refuse halfway: it is made on a call outside capture
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (st != nullptr && hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return fail(PQ_ERR_ARG,
                  "pq_q8_gemm_noalloc: the first call on device %d is under stream capture; make one call "
                  "outside capture first (it looks up the scratch array's address)",
                  dev);
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(PQ_ERR_LAUNCH, "pq_q8_gemm_noalloc: hipGetSymbolAddress failed on device %d: %s", dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PQ_OK;
}
}  // namespace pq

extern "C" size_t pq_q8_gemm_scratch_bytes(void) { return kScratchBytes; }

extern "C" int pq_q8_gemm_noalloc(const int8_t *pcodes, const uint16_t *pscales, const int8_t *qx, const float *dx,
                                  void *y, int y_dtype, int N, int K, int T, void *stream) {
  PQ_REQUIRE(N > 0 && K > 0 && K % kQ == 0 && T > 0, PQ_ERR_ARG, "pq_q8_gemm_noalloc: N=%d K=%d T=%d", N, K, T);
  const size_t need = pq_q8_gemm_workspace_bytes(N, K, T);
  PQ_REQUIRE(need <= kScratchBytes, PQ_ERR_WORKSPACE,
             "pq_q8_gemm_noalloc: N=%d K=%d T=%d splits K into %zu bytes of partials, more than the %zu-byte "
             "scratch array (call pq_q8_gemm_ws with a workspace)",
             N, K, T, need, kScratchBytes);
  void *ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address(as_stream(stream), &ws);
    if (rc != PQ_OK) return rc;
  }
  // every partial the split writes is written before the fold reads it, so
  // nothing in the array needs clearing between calls
  return pq_q8_gemm_ws(pcodes, pscales, qx, dx, y, y_dtype, N, K, T, ws, need, stream);
}
