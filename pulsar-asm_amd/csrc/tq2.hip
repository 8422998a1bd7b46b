// tq2.hip -- ternary PQ2_0 x Q8_K GEMV and the Q8_K activation quantizer (gfx950).
//
// Weights: the reference's split layout (pq2_wrap.h:9-17, pq2_split_repack):
// codes u8 [N][K/4], weight i of a byte in bits 2i..2i+1, value = code - 1;
// fp16 scale per 128-weight group [N][K/128]. Activations: Q8_K blocks of 256
// (fp32 d, 256 int8 qs, 16 int16 bsums; 292 B). Per row, groups ascending
// (pq2_host.c:82-104):
//   isum_g = sum (code-1) * qs            int32, exact
//   acc    = fl(acc + fl(fl(ws_g * db_g) * (float)isum_g))     from 0
// where db_g is the d of Q8_K block g/2 and qs its half g%2.
//
// The int32 group dots run lane-parallel; the fp32 chain is sequential per row
// over all groups, so each workgroup owns whole rows (16 rows of 32 lanes, 8
// of 64 for long rows): the lanes compute the group partials p_g into LDS,
// then, after one barrier, lane i of wave 0 folds row i in group order.
//
// Group dot without unpacking the codes to bytes: for a code dword w (16
// weights), w & 0x33333333 holds the even weights' codes in its nibbles and
// (w >> 2) & 0x33333333 the odd ones'; each activation is split x = 16 h + l
// (h the signed high nibble, l the unsigned low one) and staged in LDS as four
// nibble-packed dwords per 16 weights, so sum code*x = 16 * (two v_dot8_i32_i4)
// + (two v_dot8_u32_u4), exact, and isum = that - sum x over the group.
#include "pq_device.h"
#include "pq_host.h"
#include "q8_common.h"

namespace pq {

constexpr int kTqGroup = 128;
constexpr int kQ8K = 256;
constexpr int kQ8KBytes = 292;

// Row stride (floats) of the group partials in LDS: rows 4 banks apart, so the
// fold's lanes (one row each, reading 16 bytes at a time) spread over the banks
// instead of all reading the same four (rows of 32 or 96 floats).
__host__ __device__ inline int tq2_pgs(int ng) { return ng + 4; }

// The activations' Q8_K row staged once per workgroup: permuted qs (dword k of
// each 16 = x[k], x[k+4], x[k+8], x[k+12]), per-group sums from the bsums
// (exact int16 sums of 16), and each group's block scale d. Split in two: the
// loads (XR runs of 16 qs per thread, one group's bsums and d per thread),
// issued before the weight codes so they return first, then the LDS stores.
template <int XR>
struct TqX {
  v4i run[XR];
  v4i bs;
  uint32_t d;
};

template <int XR, int NT>
__device__ __forceinline__ void tq2_load_x(const uint8_t *__restrict__ xq, int K, TqX<XR> &t) {
  const int ng = K / kTqGroup, nrun = K / 16;
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(xq), (short)0,
                                                                      (K / kQ8K) * kQ8KBytes, kRsrcWord3);
#pragma unroll
  for (int i = 0; i < XR; i++) {   // run m: 16 qs of block m/16
    const int m = threadIdx.x + i * NT;
    t.run[i] = __builtin_amdgcn_raw_buffer_load_b128(rx, m < nrun ? (m >> 4) * kQ8KBytes + 4 + (m & 15) * 16 : kRsrcOob,
                                                     0, 0);
  }
  // group g = threadIdx.x: bsums 8*half .. 8*half+7 of its block (16 bytes at
  // an even offset) and the block's d
  const int g = threadIdx.x, blk = g >> 1, half = g & 1;
  t.bs = __builtin_amdgcn_raw_buffer_load_b128(rx, g < ng ? blk * kQ8KBytes + 4 + kQ8K + 16 * half : kRsrcOob, 0, 0);
  t.d = __builtin_amdgcn_raw_buffer_load_b32(rx, g < ng ? blk * kQ8KBytes : kRsrcOob, 0, 0);
}

// A run of 16 qs (bytes x0..x15 in dwords w0..w3) regrouped by byte permutes:
// A = x0 x4 x8 x12, B = x2 x6 x10 x14, C = x1 x5 x9 x13, D = x3 x7 x11 x15
// (the byte form's dwords k = 0, 2, 1, 3: byte j of dword k = x[k + 4j]).
struct TqRun {
  uint32_t A, B, C, D;
};
__device__ __forceinline__ TqRun tq2_regroup(uint32_t w0, uint32_t w1, uint32_t w2, uint32_t w3) {
  const uint32_t e01 = __builtin_amdgcn_perm(w1, w0, 0x06020400u);   // x0 x4 x2 x6
  const uint32_t e23 = __builtin_amdgcn_perm(w3, w2, 0x06020400u);   // x8 x12 x10 x14
  const uint32_t o01 = __builtin_amdgcn_perm(w1, w0, 0x07030501u);   // x1 x5 x3 x7
  const uint32_t o23 = __builtin_amdgcn_perm(w3, w2, 0x07030501u);   // x9 x13 x11 x15
  TqRun r;
  r.A = __builtin_amdgcn_perm(e23, e01, 0x05040100u);
  r.B = __builtin_amdgcn_perm(e23, e01, 0x07060302u);
  r.C = __builtin_amdgcn_perm(o23, o01, 0x05040100u);
  r.D = __builtin_amdgcn_perm(o23, o01, 0x07060302u);
  return r;
}

// The D8 form of a run: each x = 16 h + l with h = x >> 4 (a signed nibble,
// -8..7) and l = x & 15 (an unsigned one), packed as the nibbles of the code
// masks w & 0x33333333 (nibble n = code 2n) and (w >> 2) & 0x33333333 (code
// 2n + 1) line up: dword 0 = h of x0, x2, ..., x14 (nibble 2k from A, 2k + 1
// from B); 1 = h of the odd x (C, D); 2, 3 = l of the even and the odd x.
__device__ __forceinline__ int4 tq2_d8_run(const TqRun &r) {
  const uint32_t he = ((r.A >> 4) & 0x0f0f0f0fu) | (r.B & 0xf0f0f0f0u);
  const uint32_t ho = ((r.C >> 4) & 0x0f0f0f0fu) | (r.D & 0xf0f0f0f0u);
  const uint32_t le = (r.A & 0x0f0f0f0fu) | ((r.B & 0x0f0f0f0fu) << 4);
  const uint32_t lo = (r.C & 0x0f0f0f0fu) | ((r.D & 0x0f0f0f0fu) << 4);
  return make_int4((int)he, (int)ho, (int)le, (int)lo);
}

// The staged x in LDS: the 4 runs of a 64-weight piece (16 dwords) at a piece
// stride of kXPieceDw dwords, so the pieces that consecutive lanes read start
// on different banks (a 16-dword stride put every even piece on the same four
// banks: 16-way conflicts).
constexpr int kXPieceDw = 20;
__host__ __device__ constexpr int tq2_xbytes(int K) { return K / 64 * kXPieceDw * 4; }
__device__ __forceinline__ int tq2_run_dw(int m) { return (m >> 2) * kXPieceDw + (m & 3) * 4; }

template <int XR, int NT>
__device__ __forceinline__ void tq2_store_x(const TqX<XR> &t, int K, int *xperm, int *gsum, float *db) {
  const int ng = K / kTqGroup, nrun = K / 16;
#pragma unroll
  for (int i = 0; i < XR; i++) {
    const int m = threadIdx.x + i * NT;
    if (m < nrun) {
      const TqRun rr = tq2_regroup(t.run[i].x, t.run[i].y, t.run[i].z, t.run[i].w);
      *reinterpret_cast<int4 *>(xperm + tq2_run_dw(m)) = tq2_d8_run(rr);
    }
  }
  const int g = threadIdx.x;
  if (g < ng) {
    const int v[4] = {t.bs.x, t.bs.y, t.bs.z, t.bs.w};
    int s = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) s += (int)(int16_t)(v[i] & 0xffff) + (int)(int16_t)((uint32_t)v[i] >> 16);
    gsum[g] = s;
    db[g] = __int_as_float(t.d);
  }
}

// Up to three tensors of one K over the same activations in one launch (the
// reference's batched launch for projections that read the same vector): the
// workgroups of tensor i are wg0[i] .. wg0[i+1]-1, so each workgroup's rows
// are one tensor's and every row runs the single-tensor arithmetic.
constexpr int kTqBatch = 3;
struct TqBatch {
  const uint8_t *codes[kTqBatch];
  const uint16_t *scales[kTqBatch];
  float *y[kTqBatch];
  int rows[kTqBatch];
  int wg0[kTqBatch + 1];
};

// LPR lanes per row (16, 32 or 64), NT/LPR rows per workgroup of NT threads. Lane gs of a row
// reads the row's 16-byte pieces gs, gs + LPR, ... (a row's lanes cover
// 16*LPR contiguous bytes per load, whole cache lines): piece p is half p % 2 of group p / 2, so lanes
// gs and gs ^ 1 hold the two halves of the same groups; their exact int32
// half-dots add across the pair, and the even lane forms the group partial.
// PPL pieces per lane per round (LPR*PPL pieces = 64*LPR*PPL of K).
// The group dots are nibble dots (v_dot8: codes w & 0x33333333 and
// (w >> 2) & 0x33333333 against x's signed high and unsigned low nibbles,
// sum code*x = 16 sum code*h + sum code*l: 7 VALU per 16 weights, against 11
// for four byte masks and sdot4). The codes load nontemporal.
// NB > 1: the batch's NB tensors have the same row count and a workgroup
// takes the same row block of each (x staged once for all of them, and the
// launch holds a third of the workgroups of one per tensor and row block);
// NB = 1: a workgroup's rows are one tensor's, selected from the workgroup id.
template <int LPR, int PPL, int XR, int NT, int NB>
__global__ __launch_bounds__(NT) void tq2_gemv_kernel(TqBatch bt, const uint8_t *__restrict__ xq, int K) {
  static_assert(64 % LPR == 0, "a row's lanes must sit in one wave");
  constexpr int kRows = NT / LPR;   // rows per workgroup and tensor
  extern __shared__ __align__(16) unsigned char smem[];
  const int ng = K / kTqGroup, npc = 2 * ng;                 // groups, 16-byte pieces per row
  int *xperm = reinterpret_cast<int *>(smem);                  // tq2_xbytes(K): K bytes, permuted, padded
  int *gsum = reinterpret_cast<int *>(smem + tq2_xbytes(K));   // [ng] sum of qs over the group
  float *db = reinterpret_cast<float *>(gsum + ng);            // [ng] Q8_K d of the group's block
  const int pgs = tq2_pgs(ng);                                 // padded row stride of the partials
  float *pg = db + ng;                                         // [NB][kRows][pgs] group partials
  const int tid = threadIdx.x;
  const int r = tid / LPR, gs = tid % LPR;
  // the first tensor and the row block (workgroup-uniform)
  const int t0 = NB > 1 ? 0 : (int)blockIdx.x >= bt.wg0[2] ? 2 : (int)blockIdx.x >= bt.wg0[1] ? 1 : 0;
  const int rb = (int)blockIdx.x - (NB > 1 ? 0 : bt.wg0[t0]);
  const int N = bt.rows[t0];   // every tensor's when NB > 1
  const int row = rb * kRows + r;
  const bool live = row < N;
  // one resource per tensor (workgroup-uniform: scalar registers, no per-row
  // waterfall); a row past N reads at an offset past num_records: zeros
  __amdgpu_buffer_rsrc_t rc[NB], rsc[NB];
#pragma unroll
  for (int i = 0; i < NB; i++) {
    rc[i] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(bt.codes[t0 + i]), (short)0,
                                              (int)((size_t)N * (K / 4)), kRsrcWord3);
    rsc[i] = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(bt.scales[t0 + i]), (short)0,
                                               (int)((size_t)N * ng * 2), kRsrcWord3);
  }
  const int crow = live ? row * (K / 4) : kRsrcOob, srow = live ? row * ng * 2 : kRsrcOob;
  TqX<XR> xt;
  tq2_load_x<XR, NT>(xq, K, xt);
  for (int p0 = 0; p0 < npc; p0 += LPR * PPL) {
    // this round's codes (16 B per piece) and, on even lanes, the scale pair
    // of each piece's group, for every tensor, before anything waits
    v4i c[NB][PPL];
    uint32_t sc[NB][PPL];
#pragma unroll
    for (int i = 0; i < NB; i++)
#pragma unroll
      for (int j = 0; j < PPL; j++) {
        const int pc = p0 + j * LPR + gs, g = pc >> 1;
        c[i][j] = __builtin_amdgcn_raw_buffer_load_b128(rc[i], pc < npc && live ? crow + pc * 16 : kRsrcOob, 0,
                                                        kAuxNT);
        // every lane loads (the odd lane of a pair discards it): no branch, so
        // the waits on the earlier x loads count exactly
        sc[i][j] = __builtin_amdgcn_raw_buffer_load_b32(rsc[i], pc < npc && live ? srow + (g & ~1) * 2 : kRsrcOob, 0,
                                                        0);
      }
    if (p0 == 0) {
      tq2_store_x<XR, NT>(xt, K, xperm, gsum, db);
      __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < NB; i++)
#pragma unroll
      for (int j = 0; j < PPL; j++) {
        const int pc = p0 + j * LPR + gs, g = pc >> 1;
        const uint32_t w[4] = {(uint32_t)c[i][j].x, (uint32_t)c[i][j].y, (uint32_t)c[i][j].z, (uint32_t)c[i][j].w};
        const int *xp = xperm + (pc < npc ? pc : 0) * kXPieceDw;
        int ah = 0;
        uint32_t al = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          const int4 xv = *reinterpret_cast<const int4 *>(xp + 4 * q);
          const int m0 = (int)(w[q] & 0x33333333u), m1 = (int)((w[q] >> 2) & 0x33333333u);
          ah = __builtin_amdgcn_sdot8(m0, xv.x, ah, false);
          ah = __builtin_amdgcn_sdot8(m1, xv.y, ah, false);
          al = __builtin_amdgcn_udot8(m0, xv.z, al, false);
          al = __builtin_amdgcn_udot8(m1, xv.w, al, false);
        }
        int sacc = 16 * ah + (int)al;
        sacc += __builtin_amdgcn_update_dpp(0, sacc, kDppXor1, 0xf, 0xf, false);   // the group's two halves
        if ((gs & 1) == 0 && pc < npc) {
          const int isum = sacc - gsum[g];
          const float t = h2f((uint16_t)(sc[i][j] >> (16 * (g & 1)))) * db[g];
          pg[(i * kRows + r) * pgs + g] = t * (float)isum;
        }
      }
  }
  // after one workgroup barrier, lane l of wave 0 folds row l % kRows of
  // tensor l / kRows: every row of the workgroup in one wave's instruction
  // stream (a fold per wave, with 2 of its lanes busy, measured 0.1-0.3 us
  // slower per launch)
  __syncthreads();
  const int fi = tid / kRows, fr = tid % kRows, frow = rb * kRows + fr;
  if (tid < NB * kRows && frow < N) {   // groups ascending; partials read 8 at a time
    float acc = 0.0f;
    const float *pr = pg + (fi * kRows + fr) * pgs;
    const int ng8 = (ng & 7) == 0 ? ng : 0;   // 16-byte aligned rows when ng % 8 == 0
    for (int g = ng8; g < ng; g++) acc = acc + pr[g];
    for (int g = 0; g < ng8; g += 8) {
      const float4 a4 = reinterpret_cast<const float4 *>(pr + g)[0];
      const float4 b4 = reinterpret_cast<const float4 *>(pr + g)[1];
      acc = acc + a4.x; acc = acc + a4.y; acc = acc + a4.z; acc = acc + a4.w;
      acc = acc + b4.x; acc = acc + b4.y; acc = acc + b4.z; acc = acc + b4.w;
    }
    bt.y[t0 + fi][frow] = acc;
  }
}

// Q8_K quantizer (fwd8.c:61-137, the fork's quantize_row_q8_K_ref): one wave
// per 256-block, 4 consecutive elements per lane. max = the x at the FIRST
// index reaching amax; iscale = -127/max; q = min(127, nearest_int(iscale*x))
// with nearest_int the 1.5*2^23 magic add; bsums of 16; d = 1/iscale. An
// all-zero block writes d = 0, qs = 0 and zero bsums.
__global__ __launch_bounds__(64) void q8k_quant_kernel(const float *__restrict__ x, uint8_t *__restrict__ out) {
  const int blk = blockIdx.x, lane = threadIdx.x;
  const float *xb = x + (size_t)blk * kQ8K;
  uint8_t *ob = out + (size_t)blk * kQ8KBytes;
  const float4 v4 = *reinterpret_cast<const float4 *>(xb + 4 * lane);
  const float v[4] = {v4.x, v4.y, v4.z, v4.w};
  float a = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
  a = wave_max(a);
  int idx = 0x7fffffff;
#pragma unroll
  for (int i = 3; i >= 0; i--)
    if (fabsf(v[i]) == a) idx = 4 * lane + i;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) idx = min(idx, __shfl_xor(idx, o, 64));
  int8_t *qs = reinterpret_cast<int8_t *>(ob + 4);
  int16_t *bs = reinterpret_cast<int16_t *>(ob + 4 + kQ8K);
  if (a == 0.0f) {
    *reinterpret_cast<uint32_t *>(qs + 4 * lane) = 0u;
    if (lane < 16) bs[lane] = 0;
    if (lane == 0) *reinterpret_cast<float *>(ob) = 0.0f;
    return;
  }
  const float mx = xb[idx];
  const float iscale = -127.f / mx;
  int q[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float val = iscale * v[i] + 12582912.f;
    const int n = (__float_as_int(val) & 0x007fffff) - 0x00400000;
    q[i] = n < 127 ? n : 127;
  }
  *reinterpret_cast<uint32_t *>(qs + 4 * lane) =
      (uint32_t)(uint8_t)q[0] | ((uint32_t)(uint8_t)q[1] << 8) | ((uint32_t)(uint8_t)q[2] << 16) |
      ((uint32_t)(uint8_t)q[3] << 24);
  int s = q[0] + q[1] + q[2] + q[3];
  s += __shfl_xor(s, 1, 64);
  s += __shfl_xor(s, 2, 64);
  if ((lane & 3) == 0) bs[lane >> 2] = (int16_t)s;
  if (lane == 0) *reinterpret_cast<float *>(ob) = 1.0f / iscale;
}

}  // namespace pq

using namespace pq;

extern "C" int pq_q8k_quant(const float *x, uint8_t *out, int K, int T, void *stream) {
  PQ_REQUIRE(x && out, PQ_ERR_ARG, "pq_q8k_quant: null pointer");
  PQ_REQUIRE(K > 0 && K % kQ8K == 0 && T > 0, PQ_ERR_ARG, "pq_q8k_quant: K=%d (a multiple of 256)", K);
  PQ_REQUIRE(aligned(x, 16) && aligned(out, 4), PQ_ERR_ALIGN, "pq_q8k_quant: x must be 16-byte aligned");
  launch(q8k_quant_kernel, dim3((unsigned)((size_t)T * (K / kQ8K))), dim3(64), 0, as_stream(stream), x, out);
  return check_launch("pq_q8k_quant");
}

// The launch for a batch of n tensors (rows and pointers checked by the caller).
static int tq2_launch(TqBatch bt, int n, const uint8_t *xq, int K, hipStream_t st, const char *who) {
  const int ng = K / kTqGroup;
  // lanes per row by row length: 64 from 192 pieces (K = 12288), 32 from 64
  // pieces (K = 4096), else 16 (measured at 256 and at 512 threads); PPL
  // covers a row in one round up to K = 12288
  static const int env = env_int("PQ_TQ2_LPR");
  const int lpr = env == 16 || env == 32 || env == 64 ? env : (2 * ng >= 192 ? 64 : 2 * ng >= 64 ? 32 : 16);
  const int ppl = (2 * ng + lpr - 1) / lpr;   // pieces per lane for one round
  static const int envt = env_int("PQ_TQ2_NT");
  // 512 threads per workgroup: every workgroup stages x (K bytes permuted,
  // the group sums), which more rows amortize; measured per shape (gate/up
  // 12288x4096 5.8 us against 6.0 at 256 and 6.7 at 1024 threads, down
  // 4096x12288 6.0 against 6.8 and 6.7)
  const int nt = envt == 256 || envt == 512 || envt == 1024 ? envt : 512;
  const int rows = nt / lpr;
  // tensors of equal row count share workgroups: each takes the same row
  // block of all of them (x staged once; gate+up 12288x4096 as one batch:
  // 768 workgroups, all resident at once, instead of 1536); PQ_TQ2_NB1=1
  // keeps one tensor per workgroup
  static const int env_nb1 = env_int("PQ_TQ2_NB1");
  bool same = n > 1 && env_nb1 != 1 && nt == 512;   // (instantiated at 512 threads)
  for (int i = 1; i < n; i++) same = same && bt.rows[i] == bt.rows[0];
  const int nb = same ? n : 1;
  const size_t lds = (size_t)tq2_xbytes(K) + (size_t)ng * 8 + (size_t)nb * rows * tq2_pgs(ng) * 4;
  bt.wg0[0] = 0;
  for (int i = 0; i < kTqBatch; i++) bt.wg0[i + 1] = bt.wg0[i] + (i < n ? (bt.rows[i] + rows - 1) / rows : 0);
  for (int i = n; i < kTqBatch; i++) bt.wg0[i + 1] = 0x7fffffff;   // never selected
  const dim3 grid((unsigned)(same ? (bt.rows[0] + rows - 1) / rows : bt.wg0[n])), block(nt);
  // 16-qs runs of x per thread (K/16 runs over nt threads)
  const int runs = (K / 16 + nt - 1) / nt, xr = runs <= 1 ? 1 : runs <= 2 ? 2 : runs <= 4 ? 4 : 8;
#define PQ_TQ2_X1(L, P, X, T) launch(tq2_gemv_kernel<L, P, X, T, 1>, grid, block, lds, st, bt, xq, K)
#define PQ_TQ2_X(L, P, X, T)                                                                \
  do {                                                                                      \
    if (nb == 2) launch(tq2_gemv_kernel<L, P, X, T, 2>, grid, block, lds, st, bt, xq, K);   \
    else if (nb == 3) launch(tq2_gemv_kernel<L, P, X, T, 3>, grid, block, lds, st, bt, xq, K); \
    else PQ_TQ2_X1(L, P, X, T);                                                             \
  } while (0)
#define PQ_TQ2_T(L, P)                                             \
  do {                                                             \
    if (nt == 1024) {                                              \
      if (xr <= 1) PQ_TQ2_X1(L, P, 1, 1024);                       \
      else PQ_TQ2_X1(L, P, 2, 1024);                               \
    } else if (nt == 512) {                                        \
      if (xr <= 1) PQ_TQ2_X(L, P, 1, 512);                         \
      else if (xr <= 2) PQ_TQ2_X(L, P, 2, 512);                    \
      else PQ_TQ2_X(L, P, 4, 512);                                 \
    } else {                                                       \
      if (xr <= 1) PQ_TQ2_X1(L, P, 1, 256);                        \
      else if (xr <= 2) PQ_TQ2_X1(L, P, 2, 256);                   \
      else if (xr <= 4) PQ_TQ2_X1(L, P, 4, 256);                   \
      else PQ_TQ2_X1(L, P, 8, 256);                                \
    }                                                              \
  } while (0)
  if (lpr == 16) {
    if (ppl <= 4) PQ_TQ2_T(16, 4);
    else if (ppl <= 8) PQ_TQ2_T(16, 8);
    else PQ_TQ2_T(16, 12);
  } else if (lpr == 32) {
    if (ppl <= 2) PQ_TQ2_T(32, 2);
    else if (ppl <= 4) PQ_TQ2_T(32, 4);
    else PQ_TQ2_T(32, 6);
  } else {
    if (ppl <= 1) PQ_TQ2_T(64, 1);
    else if (ppl <= 2) PQ_TQ2_T(64, 2);
    else PQ_TQ2_T(64, 3);
  }
#undef PQ_TQ2_T
#undef PQ_TQ2_X
#undef PQ_TQ2_X1
  return check_launch(who);
}

extern "C" int pq_tq2_gemv(const uint8_t *codes, const uint16_t *scales, const uint8_t *xq, float *y, int K, int N,
                           void *stream) {
  PQ_REQUIRE(codes && scales && xq && y, PQ_ERR_ARG, "pq_tq2_gemv: null pointer");
  PQ_REQUIRE(N > 0 && K > 0 && K % kQ8K == 0 && K <= 32768, PQ_ERR_ARG,
             "pq_tq2_gemv: N=%d K=%d (K a multiple of 256, at most 32768)", N, K);
  PQ_REQUIRE(aligned(codes, 16) && aligned(xq, 4), PQ_ERR_ALIGN, "pq_tq2_gemv: codes must be 16-byte aligned");
  PQ_REQUIRE((long long)N * (K / 4) < kRsrcOob, PQ_ERR_ARG, "pq_tq2_gemv: N=%d K=%d: codes beyond 1 GiB", N, K);
  TqBatch bt{};
  bt.codes[0] = codes;
  bt.scales[0] = scales;
  bt.y[0] = y;
  bt.rows[0] = N;
  return tq2_launch(bt, 1, xq, K, as_stream(stream), "pq_tq2_gemv");
}

extern "C" int pq_tq2_gemv_batch(const uint8_t *const *codes, const uint16_t *const *scales, const uint8_t *xq,
                                 float *const *ys, int K, const int *rows, int n, void *stream) {
  PQ_REQUIRE(codes && scales && xq && ys && rows && n >= 1 && n <= kTqBatch, PQ_ERR_ARG,
             "pq_tq2_gemv_batch: null pointer or n=%d (1..3)", n);
  PQ_REQUIRE(K > 0 && K % kQ8K == 0 && K <= 32768, PQ_ERR_ARG,
             "pq_tq2_gemv_batch: K=%d (a multiple of 256, at most 32768)", K);
  PQ_REQUIRE(aligned(xq, 4), PQ_ERR_ALIGN, "pq_tq2_gemv_batch: xq alignment");
  TqBatch bt{};
  long long wgs = 0;
  for (int i = 0; i < n; i++) {
    PQ_REQUIRE(codes[i] && scales[i] && ys[i] && rows[i] > 0, PQ_ERR_ARG,
               "pq_tq2_gemv_batch: tensor %d: null pointer or rows=%d", i, rows[i]);
    PQ_REQUIRE(aligned(codes[i], 16), PQ_ERR_ALIGN, "pq_tq2_gemv_batch: tensor %d codes must be 16-byte aligned", i);
    PQ_REQUIRE((long long)rows[i] * (K / 4) < kRsrcOob, PQ_ERR_ARG, "pq_tq2_gemv_batch: tensor %d: codes beyond 1 GiB",
               i);
    bt.codes[i] = codes[i];
    bt.scales[i] = scales[i];
    bt.y[i] = ys[i];
    bt.rows[i] = rows[i];
    wgs += rows[i];
  }
  PQ_REQUIRE(wgs < (1ll << 30), PQ_ERR_ARG, "pq_tq2_gemv_batch: %lld rows in all", wgs);
  return tq2_launch(bt, n, xq, K, as_stream(stream), "pq_tq2_gemv_batch");
}
