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
// A workgroup of NT = 512 threads owns an RS-row slice of a 32-row tile (RS =
// 32, 16 or 8 by N): lane r of each of its NT/RS slots takes row r of the
// slice, slot j takes groups j, j + NT/RS, ... (a slot's
// lanes read 16*RS contiguous bytes of the tile-group, whole 128-byte lines),
// and computes acc - sg into LDS; then one lane per (row, slice of K) runs
// that slice's fmaf chain, and the K slices add in order (through lane reads
// when all chain lanes are wave 0's). The slices of a tile run on one XCD
// (workgroups go round-robin over the 8 XCDs), so the tile's scale and bit-4
// plane lines, which all of them read, are fetched into one L2. Two codes
// become two fp16 values 1 + q/128 by one byte permute, which the FMA widens
// exactly (v_fma_mix_f32).
#include "pq_device.h"
#include "pq_host.h"
#include "q8_common.h"
#include "pq_prologue.h"

namespace pq {


__host__ __device__ inline int qlow_ks(int K) { return K >= 4096 ? 4 : 2; }
__host__ __device__ inline int qlow_gw(int B) { return B == 4 ? 32 : 40; }   // 16-byte units per tile-group

// LDS row stride (floats) of the per-row partials and scale pairs: rows 4
// banks apart and 16-byte aligned (a stride of 8 banks for 8-row slices,
// tried, gave more bank-conflict cycles: down 379K -> 412K).
__host__ __device__ inline int qlow_gp(int G, int RS) { return (void)RS, G + 4; }

// The code q (< 128) as the fp16 1 + q/128, bits 0x3C00 | q << 3: mq holds
// four codes at bits 3-6 (and 7) of its bytes; one byte permute interleaves
// bytes 2j and 2j + 1 with 0x3C into two such halves. An FMA with an fp16
// operand (v_fma_mix_f32) widens it exactly, so fmaf(1 + q/128, x, a) is the
// fp32 fmaf of the code's float.
typedef _Float16 qh2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ qh2 qlow_h2(uint32_t mq, int j) {
  return __builtin_bit_cast(qh2, __builtin_amdgcn_perm(0x3C3C3C3Cu, mq, j ? 0x04030402u : 0x04010400u));
}

template <int B>
__device__ __forceinline__ float qlow_acc(v4i w4, uint32_t hp, const float *__restrict__ xg) {
  const uint32_t w[4] = {(uint32_t)w4.x, (uint32_t)w4.y, (uint32_t)w4.z, (uint32_t)w4.w};
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      // quad p = 2i + hf: codes of weights 8i + 4hf + b (b = 0..3) at bits 3-6 of byte b
      uint32_t m = (hf ? (w[i] >> 1) : (w[i] << 3)) & 0x78787878u;
      if constexpr (B == 5) {   // bit 4 of quad p's codes: the plane's bits 8b + p, to bit 7 of byte b
        const int p = 2 * i + hf;
        m |= (hp << (7 - p)) & 0x80808080u;
      }
      const float4 xv = *reinterpret_cast<const float4 *>(xg + 8 * i + 4 * hf);
      const qh2 q01 = qlow_h2(m, 0), q23 = qlow_h2(m, 1);
      a0 = __builtin_fmaf((float)q01.x, xv.x, a0);
      a1 = __builtin_fmaf((float)q01.y, xv.y, a1);
      a2 = __builtin_fmaf((float)q23.x, xv.z, a2);
      a3 = __builtin_fmaf((float)q23.y, xv.w, a3);
    }
  }
  return (a0 + a1) + (a2 + a3);
}

// One step of a slice's chain: y = fmaf(d', acc - sg, fmaf(mn, sg, y)), the
// scale pair sc = (d', mn) as half2.
__device__ __forceinline__ float qlow_step(float y, float u, float sg, uint32_t sc) {
  const float dp = h2f((uint16_t)(sc & 0xffffu)), mn = h2f((uint16_t)(sc >> 16));
  return __builtin_fmaf(dp, u, __builtin_fmaf(mn, sg, y));
}

// A slice's chain from 0 over its GL groups in order: per group the partial
// up[g] = acc - sg, the scale pair cp[g] and the group sum sp[g] (16-byte
// aligned LDS). With GL a multiple of 16 the operands come in blocks of 8
// groups held in two register sets, each block's reads issued 8 steps before
// its first use (the chain's two dependent FMAs per step then never wait on
// LDS); otherwise two groups per read, one read ahead.
__device__ __forceinline__ float qlow_chain(const float *__restrict__ up, const uint32_t *__restrict__ cp,
                                            const float *__restrict__ sp, int GL) {
  float yv = 0.0f;
  if (GL % 16 == 0) {
    struct Blk {
      float4 u0, u1, s0, s1;
      uint4 c0, c1;
    };
    auto ld = [&](Blk &k, int i) {
      k.u0 = *reinterpret_cast<const float4 *>(up + 8 * i);
      k.u1 = *reinterpret_cast<const float4 *>(up + 8 * i + 4);
      k.s0 = *reinterpret_cast<const float4 *>(sp + 8 * i);
      k.s1 = *reinterpret_cast<const float4 *>(sp + 8 * i + 4);
      k.c0 = *reinterpret_cast<const uint4 *>(cp + 8 * i);
      k.c1 = *reinterpret_cast<const uint4 *>(cp + 8 * i + 4);
    };
    auto run = [&](const Blk &k) {
      yv = qlow_step(yv, k.u0.x, k.s0.x, k.c0.x);
      yv = qlow_step(yv, k.u0.y, k.s0.y, k.c0.y);
      yv = qlow_step(yv, k.u0.z, k.s0.z, k.c0.z);
      yv = qlow_step(yv, k.u0.w, k.s0.w, k.c0.w);
      yv = qlow_step(yv, k.u1.x, k.s1.x, k.c1.x);
      yv = qlow_step(yv, k.u1.y, k.s1.y, k.c1.y);
      yv = qlow_step(yv, k.u1.z, k.s1.z, k.c1.z);
      yv = qlow_step(yv, k.u1.w, k.s1.w, k.c1.w);
    };
    // The empty asm statements with a memory clobber pin each block's reads
    // where they stand: without them the compiler turns a register set
    // carried round the loop into reads at the top of the next iteration,
    // right before their use.
    const int n = GL / 8;   // even
    Blk A, B;
    ld(A, 0);
    ld(B, 1);
    asm volatile("" ::: "memory");
    for (int i = 0; i < n; i += 2) {
      // the reads past the slice's last block repeat it (unconditional reads
      // keep the LDS wait counts exact)
      run(A);
      ld(A, i + 2 < n ? i + 2 : n - 2);
      asm volatile("" ::: "memory");
      run(B);
      ld(B, i + 3 < n ? i + 3 : n - 1);
      asm volatile("" ::: "memory");
    }
    return yv;
  }
  const int n = GL / 2;   // G is a multiple of 8 and KS of 2 or 4: GL is even
  float2 uq = *reinterpret_cast<const float2 *>(up), sq = *reinterpret_cast<const float2 *>(sp);
  uint2 cq = *reinterpret_cast<const uint2 *>(cp);
  for (int it = 0; it < n; it++) {
    const int nx = (it + 1 < n ? it + 1 : it) * 2;
    const float2 un = *reinterpret_cast<const float2 *>(up + nx), sn = *reinterpret_cast<const float2 *>(sp + nx);
    const uint2 cn = *reinterpret_cast<const uint2 *>(cp + nx);
    yv = qlow_step(yv, uq.x, sq.x, cq.x);
    yv = qlow_step(yv, uq.y, sq.y, cq.y);
    uq = un;
    sq = sn;
    cq = cn;
  }
  return yv;
}

// Workgroup b -> (tile, RS-row slice of it): with a multiple of 8 tiles, the
// 32/RS slices of a tile get workgroup ids equal mod 8 (one XCD).
template <int RS>
__device__ __forceinline__ void qlow_place(int b, int ntiles, int &tile, int &sub) {
  constexpr int SUBS = 32 / RS;
  if (ntiles % 8 == 0) {
    tile = (b / (8 * SUBS)) * 8 + (b % 8);
    sub = (b / 8) % SUBS;
  } else {
    tile = b / SUBS;
    sub = b % SUBS;
  }
}

// With ws (the split form): workgroup (slice of rows, s) covers only K slice
// s = blockIdx.y and writes its y_s to ws[s][N]; qlow_combine_kernel adds the
// slices in order. Without ws: all K slices in one workgroup.
//
// PRO: x is the bf16 vector x (kProPlain), or comes from a fused prologue
// (pq_prologue.h: RESNORM, NORM, SILU, CONV; whole rows only, K = NT * E):
// thread t computes elements tE .. tE + E - 1 as the bf16 values the unfused
// op would store, which the staging below then widens and sums exactly as it
// does x.
constexpr int kProPlain = -1;

// SWI: the FFN's gate/up GEMV with the SwiGLU epilogue. The tensor's N = 2F
// rows are [gate | up]; a workgroup takes RS rows of a gate tile with its first
// NT/2 threads and the same rows of the up tile (F/32 tiles on) with the
// others, and writes y = bf16(silu(bf16 g) * bf16 u) for its RS rows [F]: the
// GEMV, bf16 outputs and pq_silu_mul in one launch, the same bits.
template <int B, int RS, int XL, int NT, int PF, int PRO = kProPlain, int E = 8, bool SWI = false>
__global__ __launch_bounds__(NT) void qlow_gemv_kernel(const uint8_t *__restrict__ pc,
                                                              const uint32_t *__restrict__ ps,
                                                              const uint16_t *__restrict__ x, void *__restrict__ y,
                                                              int y_bf16, int N, int K, float *__restrict__ ws,
                                                              pq_gemv_prologue p) {
  constexpr bool kPro = PRO != kProPlain;
  extern __shared__ __align__(16) float lsm[];
  __shared__ __align__(16) float red[2 * kNormSlots];   // the prologue's workgroup reductions
  const int GA = K / kQ, KSA = qlow_ks(K), GW = qlow_gw(B);
  // the groups this workgroup covers: [gb, gb + G), in KS slices of GL
  const int KS = ws ? 1 : KSA, G = ws ? GA / KSA : GA, GL = G / KS, gb = ws ? (int)blockIdx.y * G : 0;
  // per row, the groups' partials and scale pairs at the padded stride GP
  constexpr int kHalf = SWI ? NT / 2 : NT;   // threads per row set (SWI: the gate rows', then the up rows')
  constexpr int kLoSlots = kHalf / RS;       // group slots per round (kHalf/RS slots of RS rows)
  constexpr int kRows = SWI ? 2 * RS : RS;   // rows staged in LDS
  const int GP = qlow_gp(G, RS);
  float *xs = lsm;                      // [G*32]
  float *sx = xs + G * kQ;              // [G]
  float *u = sx + G;                    // [kRows][GP]: acc - sg
  uint32_t *scl = reinterpret_cast<uint32_t *>(u + kRows * GP);   // [kRows][GP] half2 (d', mn)
  float *ys = reinterpret_cast<float *>(scl + kRows * GP);          // [KS][RS] (SWI: [RS] up outputs)
  const int tid = threadIdx.x;
  const int half = SWI ? tid / kHalf : 0, tih = SWI ? tid % kHalf : tid;   // wave-uniform half
  int tile, sub;
  qlow_place<RS>(blockIdx.x, (SWI ? N / 2 : N) / 32, tile, sub);
  if (SWI && half) tile += N / 64;      // the up rows' tile
  const int r = tih % RS, slot = tih / RS;
  const int tr = sub * RS + r;          // this lane's row within the tile
  // the tile's codes and scales from group gb (wave-uniform resources)
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(pc + ((size_t)tile * GA + gb) * GW * 16), (short)0, G * GW * 16, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t *>(ps + ((size_t)tile * GA + gb) * 32), (short)0, G * 32 * 4, kRsrcWord3);
  x += (size_t)gb * kQ;
  K = G * kQ;
  // Loads in the order their data is needed (they return in issue order):
  // x (8 bf16 per 16-byte load, XL loads per thread: K <= 2048 XL), this
  // lane's first PF groups' codes, then the slice's scale pairs (4 rows per
  // 16-byte load, up to kScl loads per thread; any more come after the
  // partials). Codes and scales load nontemporal (read once per launch; the
  // scale lines a tile's slices share are read close together in time).
  constexpr int kXLoads = kPro ? 1 : XL, kScl = 4;
  constexpr int HQ = RS / 4;
  uint4 xr[kXLoads];
  ProRegs<E, conv_taps(PRO)> pr;
  if constexpr (kPro) {
    pro_load<PRO, E>(p, tid * E, K, pr);   // the prologue's global loads
  } else {
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(x), (short)0, K * 2, kRsrcWord3);
#pragma unroll
    for (int it = 0; it < kXLoads; it++) {
      const int e = tid * 8 + it * NT * 8;
      const v4i v = __builtin_amdgcn_raw_buffer_load_b128(rx, e < K ? e * 2 : kRsrcOob, 0, 0);
      xr[it] = make_uint4((uint32_t)v.x, (uint32_t)v.y, (uint32_t)v.z, (uint32_t)v.w);
    }
  }
  v4i w[PF];
  uint32_t hpl[PF];
#pragma unroll
  for (int k = 0; k < PF; k++) {
    const int g = slot + kLoSlots * k;
    w[k] = __builtin_amdgcn_raw_buffer_load_b128(rc, g < G ? (g * GW + tr) * 16 : kRsrcOob, 0, kAuxNT);
    hpl[k] = B == 5 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, g < G ? (g * GW + 32) * 16 + tr * 4 : kRsrcOob,
                                                                     0, kAuxNT)
                    : 0u;
  }
  v4i sr[kScl];
#pragma unroll
  for (int k = 0; k < kScl; k++) {
    const int i = tih + k * kHalf;
    sr[k] = __builtin_amdgcn_raw_buffer_load_b128(
        rsc, i < G * HQ ? ((i / HQ) * 32 + sub * RS + 4 * (i % HQ)) * 4 : kRsrcOob, 0, kAuxNT);
  }
  // x widened into LDS, and each group's sum of x in order from 0: a group's
  // 32 elements are the 8-element pieces of 4 adjacent lanes (K is a multiple
  // of 256), so lane j of the 4 continues the chain of lane j - 1 (a row shift
  // by one lane) and the group's last lane holds the sum. From a prologue: the
  // E-element pieces of 32/E adjacent lanes, chained the same way.
  if constexpr (kPro) {
    float v[E];
    pro_values<PRO, E>(p, tid * E, K, pr, red, v);
    const int e0 = tid * E;
    constexpr int LG = 32 / E;
#pragma unroll
    for (int i = 0; i < E / 4; i++)
      *reinterpret_cast<float4 *>(xs + e0 + 4 * i) = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
    float c = 0.0f;
#pragma unroll
    for (int k = 0; k < E; k++) c = c + v[k];
#pragma unroll
    for (int j = 1; j < LG; j++) {
      float cj = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), kDppRowShr1, 0xf, 0xf, false));
#pragma unroll
      for (int k = 0; k < E; k++) cj = cj + v[k];
      if ((tid & (LG - 1)) == j) c = cj;
    }
    if ((tid & (LG - 1)) == LG - 1) sx[e0 / kQ] = c;
  }
#pragma unroll
  for (int it = 0; it < (kPro ? 0 : kXLoads); it++) {
    const int e = tid * 8 + it * NT * 8;
    const uint32_t vv[4] = {xr[it].x, xr[it].y, xr[it].z, xr[it].w};
    float f[8];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      f[2 * k] = __uint_as_float(vv[k] << 16);
      f[2 * k + 1] = __uint_as_float(vv[k] & 0xffff0000u);
    }
    if (e < K) {
      *reinterpret_cast<float4 *>(xs + e) = make_float4(f[0], f[1], f[2], f[3]);
      *reinterpret_cast<float4 *>(xs + e + 4) = make_float4(f[4], f[5], f[6], f[7]);
    }
    float c = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) c = c + f[k];
#pragma unroll
    for (int j = 1; j < 4; j++) {
      float cj = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), kDppRowShr1, 0xf, 0xf, false));
#pragma unroll
      for (int k = 0; k < 8; k++) cj = cj + f[k];
      if ((tid & 3) == j) c = cj;
    }
    if ((tid & 3) == 3 && e < K) sx[e / kQ] = c;
  }
  __syncthreads();
  // group partials acc - sg, PF groups of loads in flight: the rounds
  // alternate between two register sets passed by name (w / hpl, then wb /
  // hb), each round's loads issued before the round before it is computed and
  // unconditionally (groups past G read zeros through the resource bound), so
  // no copy of a register still being filled waits for its load
  auto ld_round = [&](v4i *wr, uint32_t *hr, int g0) {
#pragma unroll
    for (int k = 0; k < PF; k++) {
      const int g = g0 + slot + kLoSlots * k;
      wr[k] = __builtin_amdgcn_raw_buffer_load_b128(rc, g < G ? (g * GW + tr) * 16 : kRsrcOob, 0, kAuxNT);
      hr[k] = B == 5 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                           rc, g < G ? (g * GW + 32) * 16 + tr * 4 : kRsrcOob, 0, kAuxNT)
                     : 0u;
    }
  };
  auto do_round = [&](const v4i *wr, const uint32_t *hr, int g0) {
#pragma unroll
    for (int k = 0; k < PF; k++) {
      const int g = g0 + slot + kLoSlots * k;
      if (g < G) u[(half * RS + r) * GP + g] = qlow_acc<B>(wr[k], hr[k], xs + g * kQ) - sx[g];
    }
  };
  constexpr int kRound = kLoSlots * PF;   // groups per round
  v4i wb[PF];
  uint32_t hb[PF];
  if (G <= 2 * kRound) {   // one or two rounds (every decode shape): straight-line code, exact waits
    ld_round(wb, hb, kRound);
    do_round(w, hpl, 0);
    do_round(wb, hb, kRound);
  } else {
    for (int g0 = 0; g0 < G; g0 += 2 * kRound) {
      ld_round(wb, hb, g0 + kRound);
      do_round(w, hpl, g0);
      if (g0 + kRound >= G) break;
      ld_round(w, hpl, g0 + 2 * kRound);
      do_round(wb, hb, g0 + kRound);
    }
  }
  // the scale pairs, each row's to its row
  auto put_scales = [&](int i, v4i v) {
    const int g = i / HQ, h = half * RS + 4 * (i % HQ);
    scl[h * GP + g] = (uint32_t)v.x;
    scl[(h + 1) * GP + g] = (uint32_t)v.y;
    scl[(h + 2) * GP + g] = (uint32_t)v.z;
    scl[(h + 3) * GP + g] = (uint32_t)v.w;
  };
#pragma unroll
  for (int k = 0; k < kScl; k++)
    if (tih + k * kHalf < G * HQ) put_scales(tih + k * kHalf, sr[k]);
  for (int i = tih + kScl * kHalf; i < G * HQ; i += kHalf)
    put_scales(i, __builtin_amdgcn_raw_buffer_load_b128(rsc, ((i / HQ) * 32 + sub * RS + 4 * (i % HQ)) * 4, 0,
                                                        kAuxNT));
  __syncthreads();
  // per (row, K slice): the slice's chain over its groups in order, one lane
  // each. With at most 64 such lanes (every shape but 32-row slices of K >=
  // 4096) they are wave 0's, and the slices add in order through lane reads:
  // no barrier and no LDS pass
  if constexpr (SWI) {   // wave 0: the gate rows' chains, wave 1 the up rows' (RS * KS <= 64 each)
    const int wv = tid >> 6, ln = tid & 63;
    float yv = 0.0f, yt = 0.0f;
    if (wv < 2 && ln < RS * KS) {
      const int s = ln / RS, rr = ln % RS;
      yv = qlow_chain(u + (wv * RS + rr) * GP + s * GL, scl + (wv * RS + rr) * GP + s * GL, sx + s * GL, GL);
    }
    if (wv < 2)
      for (int s = 0; s < KS; s++) yt = yt + __shfl(yv, s * RS + ln % RS, 64);
    if (wv == 1 && ln < RS) ys[ln] = yt;
    __syncthreads();
    if (wv == 0 && ln < RS) {   // silu_mul of the two bf16 outputs (silu_mul_kernel's arithmetic)
      const float a = bf2f(f2bf(yt)), uu = bf2f(f2bf(ys[ln]));
      const float sg = 1.0f / (1.0f + expf_pq(-a));
      reinterpret_cast<uint16_t *>(y)[tile * 32 + sub * RS + ln] = f2bf((a * sg) * uu);
    }
    return;
  }
  const int row = tile * 32 + sub * RS + tid % RS;
  if (RS * KS <= 64) {
    if (tid >= 64) return;
    float yv = 0.0f;
    if (tid < RS * KS) {
      const int s = tid / RS, rr = tid % RS;
      yv = qlow_chain(u + rr * GP + s * GL, scl + rr * GP + s * GL, sx + s * GL, GL);
    }
    if (ws) {   // one K slice per workgroup
      if (tid < RS && row < N) ws[(size_t)blockIdx.y * N + row] = yv;
      return;
    }
    float yt = 0.0f;
    for (int s = 0; s < KS; s++) yt = yt + __shfl(yv, s * RS + tid % RS, 64);
    if (tid < RS && row < N) {
      if (y_bf16) reinterpret_cast<uint16_t *>(y)[row] = f2bf(yt);
      else reinterpret_cast<float *>(y)[row] = yt;
    }
    return;
  }
  if (tid < RS * KS) {
    const int s = tid / RS, rr = tid % RS;
    ys[s * RS + rr] = qlow_chain(u + rr * GP + s * GL, scl + rr * GP + s * GL, sx + s * GL, GL);
  }
  __syncthreads();
  if (tid < RS) {
    if (ws) {
      if (row < N) ws[(size_t)blockIdx.y * N + row] = ys[tid];
      return;
    }
    float yt = 0.0f;
    for (int s = 0; s < KS; s++) yt = yt + ys[s * RS + tid];
    if (row < N) {
      if (y_bf16) reinterpret_cast<uint16_t *>(y)[row] = f2bf(yt);
      else reinterpret_cast<float *>(y)[row] = yt;
    }
  }
}

// ---------------------------------------------------------- T positions
// The GEMV of TB positions per workgroup, one position block per blockIdx.y
// (a prompt's low-bit linears, which the reference runs one position at a
// time): every position's arithmetic is the single-position kernel's, in the
// same order, so y[t] equals pq_qlow_gemv of x[t] bit for bit. A group's codes
// become their 16 fp16 pairs once and serve the TB positions. LDS: TB
// positions' x and group sums, TB x RS rows of partials, RS rows of scales.

// The 32 codes of a group as 16 fp16 pairs 1 + q/128 (quads in qlow_acc's
// order: pair 2p + j holds codes 4p + 2j and 4p + 2j + 1 of quad p).
template <int B>
__device__ __forceinline__ void qlow_codes(v4i w4, uint32_t hp, qh2 *q) {
  const uint32_t w[4] = {(uint32_t)w4.x, (uint32_t)w4.y, (uint32_t)w4.z, (uint32_t)w4.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      uint32_t m = (hf ? (w[i] >> 1) : (w[i] << 3)) & 0x78787878u;
      if constexpr (B == 5) {
        const int pq = 2 * i + hf;
        m |= (hp << (7 - pq)) & 0x80808080u;
      }
      q[4 * i + 2 * hf] = qlow_h2(m, 0);
      q[4 * i + 2 * hf + 1] = qlow_h2(m, 1);
    }
  }
}

// acc of one position from the group's pairs: qlow_acc's four chains.
__device__ __forceinline__ float qlow_dot(const qh2 *q, const float *__restrict__ xg) {
  float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; i++) {
#pragma unroll
    for (int hf = 0; hf < 2; hf++) {
      const float4 xv = *reinterpret_cast<const float4 *>(xg + 8 * i + 4 * hf);
      const qh2 q01 = q[4 * i + 2 * hf], q23 = q[4 * i + 2 * hf + 1];
      a0 = __builtin_fmaf((float)q01.x, xv.x, a0);
      a1 = __builtin_fmaf((float)q01.y, xv.y, a1);
      a2 = __builtin_fmaf((float)q23.x, xv.z, a2);
      a3 = __builtin_fmaf((float)q23.y, xv.w, a3);
    }
  }
  return (a0 + a1) + (a2 + a3);
}

constexpr int kQgNT = 512;   // threads per workgroup of the T-position form

template <int B, int RS, int TB, int XL>
__global__ __launch_bounds__(kQgNT) void qlow_gemm_kernel(const uint8_t *__restrict__ pc,
                                                           const uint32_t *__restrict__ ps,
                                                           const uint16_t *__restrict__ x, void *__restrict__ y,
                                                           int y_bf16, int N, int K, int T, int ldy) {
  constexpr int NT = kQgNT, kLoSlots = NT / RS, HQ = RS / 4, kScl = 4;
  extern __shared__ __align__(16) float lsm[];
  const int G = K / kQ, KS = qlow_ks(K), GL = G / KS, GW = qlow_gw(B), GP = qlow_gp(G, RS);
  float *xs = lsm;                                             // [TB][G*32]
  float *sx = xs + TB * G * kQ;                                // [TB][G]
  float *u = sx + TB * G;                                      // [TB][RS][GP]: acc - sg
  uint32_t *scl = reinterpret_cast<uint32_t *>(u + TB * RS * GP);   // [RS][GP]
  float *ys = reinterpret_cast<float *>(scl + RS * GP);              // [TB][KS][RS] (slices across waves)
  const int tid = threadIdx.x;
  int tile, sub;
  qlow_place<RS>(blockIdx.x, N / 32, tile, sub);
  const int r = tid % RS, slot = tid / RS, tr = sub * RS + r;
  const int t0 = (int)blockIdx.y * TB, nt = T - t0 < TB ? T - t0 : TB;   // positions of this block
  const __amdgpu_buffer_rsrc_t rc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(pc + (size_t)tile * G * GW * 16), (short)0, G * GW * 16, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rsc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t *>(ps + (size_t)tile * G * 32), (short)0, G * 32 * 4, kRsrcWord3);
  // Loads in the order their data is needed: the block's x rows (positions
  // past T read zeros; 8 bf16 per 16-byte load, XL per thread and position),
  // the lane's first group of codes, the scale pairs.
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t *>(x + (size_t)t0 * K), (short)0, nt * K * 2, kRsrcWord3);
  v4i xr[TB][XL];
#pragma unroll
  for (int t = 0; t < TB; t++)
#pragma unroll
    for (int it = 0; it < XL; it++) {
      const int e = tid * 8 + it * NT * 8;
      xr[t][it] = __builtin_amdgcn_raw_buffer_load_b128(rx, e < K ? (t * K + e) * 2 : kRsrcOob, 0, 0);
    }
  int g = slot;
  v4i wc = __builtin_amdgcn_raw_buffer_load_b128(rc, g < G ? (g * GW + tr) * 16 : kRsrcOob, 0, kAuxNT);
  uint32_t hc = B == 5 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rc, g < G ? (g * GW + 32) * 16 + tr * 4
                                                                                : kRsrcOob, 0, kAuxNT)
                       : 0u;
  v4i sr[kScl];
#pragma unroll
  for (int k = 0; k < kScl; k++) {
    const int i = tid + k * NT;
    sr[k] = __builtin_amdgcn_raw_buffer_load_b128(
        rsc, i < G * HQ ? ((i / HQ) * 32 + sub * RS + 4 * (i % HQ)) * 4 : kRsrcOob, 0, kAuxNT);
  }
  // staging, position by position: x widened into LDS and its group sums in
  // order from 0 (a group's 32 elements are the 8-element pieces of 4
  // adjacent lanes; lane j continues lane j - 1's chain by a DPP row shift)
#pragma unroll
  for (int t = 0; t < TB; t++)
#pragma unroll
    for (int it = 0; it < XL; it++) {
      const int e = tid * 8 + it * NT * 8;
      const uint32_t vv[4] = {(uint32_t)xr[t][it].x, (uint32_t)xr[t][it].y, (uint32_t)xr[t][it].z,
                              (uint32_t)xr[t][it].w};
      float f[8];
#pragma unroll
      for (int k = 0; k < 4; k++) {
        f[2 * k] = __uint_as_float(vv[k] << 16);
        f[2 * k + 1] = __uint_as_float(vv[k] & 0xffff0000u);
      }
      float *xt = xs + t * G * kQ;
      if (e < K) {
        *reinterpret_cast<float4 *>(xt + e) = make_float4(f[0], f[1], f[2], f[3]);
        *reinterpret_cast<float4 *>(xt + e + 4) = make_float4(f[4], f[5], f[6], f[7]);
      }
      float c = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; k++) c = c + f[k];
#pragma unroll
      for (int j = 1; j < 4; j++) {
        float cj = __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(c), kDppRowShr1, 0xf, 0xf, false));
#pragma unroll
        for (int k = 0; k < 8; k++) cj = cj + f[k];
        if ((tid & 3) == j) c = cj;
      }
      if ((tid & 3) == 3 && e < K) sx[t * G + e / kQ] = c;
    }
  // the scale pairs, each row's to its row
  auto put_scales = [&](int i, v4i v) {
    const int gg = i / HQ, h = i % HQ;
    scl[(4 * h) * GP + gg] = (uint32_t)v.x;
    scl[(4 * h + 1) * GP + gg] = (uint32_t)v.y;
    scl[(4 * h + 2) * GP + gg] = (uint32_t)v.z;
    scl[(4 * h + 3) * GP + gg] = (uint32_t)v.w;
  };
#pragma unroll
  for (int k = 0; k < kScl; k++)
    if (tid + k * NT < G * HQ) put_scales(tid + k * NT, sr[k]);
  for (int i = tid + kScl * NT; i < G * HQ; i += NT)
    put_scales(i, __builtin_amdgcn_raw_buffer_load_b128(rsc, ((i / HQ) * 32 + sub * RS + 4 * (i % HQ)) * 4, 0,
                                                        kAuxNT));
  __syncthreads();
  // group partials: each (row, group) of the lane converts its codes once,
  // then forms acc - sg for the block's positions; the next group's codes
  // load before this one's arithmetic
  for (; g < G; g += kLoSlots) {
    const int gn = g + kLoSlots;
    const v4i wn = __builtin_amdgcn_raw_buffer_load_b128(rc, gn < G ? (gn * GW + tr) * 16 : kRsrcOob, 0, kAuxNT);
    const uint32_t hn = B == 5 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                                     rc, gn < G ? (gn * GW + 32) * 16 + tr * 4 : kRsrcOob, 0, kAuxNT)
                               : 0u;
    qh2 q[16];
    qlow_codes<B>(wc, hc, q);
#pragma unroll
    for (int t = 0; t < TB; t++)
      u[(t * RS + r) * GP + g] = qlow_dot(q, xs + t * G * kQ + g * kQ) - sx[t * G + g];
    wc = wn;
    hc = hn;
  }
  __syncthreads();
  // per (position, K slice, row): the slice's chain; lane ((t * KS + s) * RS + rr)
  const int nl = TB * KS * RS;
  float yv = 0.0f;
  int tt = 0, ss = 0, rr = 0;
  if (tid < nl) {
    rr = tid % RS;
    ss = (tid / RS) % KS;
    tt = tid / (RS * KS);
    yv = qlow_chain(u + (tt * RS + rr) * GP + ss * GL, scl + rr * GP + ss * GL, sx + tt * G + ss * GL, GL);
  }
  const int row = tile * 32 + sub * RS + rr;
  auto put = [&](float yt) {
    if (tt < nt && row < N) {
      const size_t o = (size_t)(t0 + tt) * ldy + row;
      if (y_bf16) reinterpret_cast<uint16_t *>(y)[o] = f2bf(yt);
      else reinterpret_cast<float *>(y)[o] = yt;
    }
  };
  if (KS * RS <= 64) {   // a (position, row)'s slices sit in one wave: they add in order by lane reads
    float yt = 0.0f;
    const int base = tid - ss * RS;
    for (int s = 0; s < KS; s++) yt = yt + __shfl(yv, base + s * RS, 64);
    if (tid < nl && ss == 0) put(yt);
    return;
  }
  if (tid < nl) ys[(tt * KS + ss) * RS + rr] = yv;
  __syncthreads();
  if (tid < nl && ss == 0) {
    float yt = 0.0f;
    for (int s = 0; s < KS; s++) yt = yt + ys[(tt * KS + s) * RS + rr];
    put(yt);
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

// Rows per workgroup: 32 (whole tiles) when that still gives 512
// workgroups, else 16 when that gives 192, else 8. Each workgroup stages x
// and its group sums, which longer row slices amortize; small N needs the
// short slices to fill the chip (measured at 512 threads, Q4: gate+up 16384
// rows 8.0 us at 32 rows against 10.1 at 16; q|k|v 3072 rows 4.75 at 16
// against 5.2 at 8 and 5.4 at 32; o_proj and down 2048 rows 4.4 and 7.6 at 8).
// PQ_QLOW_RS forces 8, 16 or 32.
static int qlow_rows(int N) {
  static const int fR = env_int("PQ_QLOW_RS");
  if (fR == 8 || fR == 16 || fR == 32) return fR;
  return N / 32 >= 512 ? 32 : N / 16 >= 192 ? 16 : 8;
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
  const int RS = qlow_rows(N);
  auto lds_of = [&](int G, int ks) {
    return ((size_t)G * kQ + G + 2 * RS * (size_t)qlow_gp(G, RS) + (size_t)ks * RS) * sizeof(float);
  };
  // the split form (one workgroup per (8 rows, K slice), then the ordered
  // combine): for long rows on too few row slices to fill the chip, or when
  // a whole row's staging exceeds LDS
  // PQ_QLOW_SPLIT=1 takes the split form whenever the workspace allows, 2 only
  // when a whole row's staging exceeds LDS
  static const int env_split = env_int("PQ_QLOW_SPLIT");
  const bool whole_fits = lds_of(K / kQ, KS) <= kMaxLds;
  const bool want_split = env_split == 1   ? true
                          : env_split == 2 ? !whole_fits
                                           : (N / RS < 128 && K >= 4096) || !whole_fits;
  const bool split = ws != nullptr && ws_bytes >= pq_qlow_workspace_bytes(N, K, bits) && want_split;
  PQ_REQUIRE(!split || aligned(ws, 4), PQ_ERR_ALIGN, "pq_qlow_gemv: workspace alignment");
  const int G = split ? K / kQ / KS : K / kQ, KSW = split ? 1 : KS;
  const size_t lds = lds_of(G, KSW);
  PQ_REQUIRE(lds <= kMaxLds, PQ_ERR_ARG, "pq_qlow_gemv: K=%d needs the workspace form", K);
  static const int envt = env_int("PQ_QLOW_NT");
  const int NT = envt == 256 || envt == 512 ? envt : 512;   // threads per workgroup (512 measured faster)
  const dim3 grid((unsigned)(N / RS), split ? (unsigned)KS : 1u), block(NT);
  const int yb = y_dtype == PQ_DTYPE_BF16 ? 1 : 0;
  float *wsf = split ? static_cast<float *>(ws) : nullptr;
  hipStream_t st = as_stream(stream);
  const uint32_t *ps32 = reinterpret_cast<const uint32_t *>(pscales);
  const pq_gemv_prologue np0{};   // no prologue: x given
  // x loads per thread for the K one workgroup covers (NT threads x 8)
  const int xl = (G * kQ + 8 * NT - 1) / (8 * NT), XL = xl <= 1 ? 1 : xl <= 2 ? 2 : xl <= 4 ? 4 : 8;
  // PF groups of loads in flight per slot: 2 (the partials of one round overlap the next
  // round's loads); per config-2 step Q4 22.9 / 21.9 / 22.4 us at PF = 4 / 2 / 1, Q5 24.2 / 23.5 /
  // 23.9 us (PQ_QLOW_PF: 1, 2 or 4)
  static const int env_pf = env_int("PQ_QLOW_PF");
  const int pf = env_pf == 1 || env_pf == 4 ? env_pf : 2;
#define PQ_QLOW(BB, RR, XX, TT)                                                                            \
  do {                                                                                                     \
    if (pf == 1) launch(qlow_gemv_kernel<BB, RR, XX, TT, 1>, grid, block, lds, st, pcodes, ps32, x, y, yb, N, K, wsf, np0); \
    else if (pf == 2) launch(qlow_gemv_kernel<BB, RR, XX, TT, 2>, grid, block, lds, st, pcodes, ps32, x, y, yb, N, K, wsf, np0); \
    else launch(qlow_gemv_kernel<BB, RR, XX, TT, 4>, grid, block, lds, st, pcodes, ps32, x, y, yb, N, K, wsf, np0); \
  } while (0)
#define PQ_QLOW_X(BB, RR)                                  \
  if (NT == 512) {                                         \
    switch (XL) {                                          \
      case 1: PQ_QLOW(BB, RR, 1, 512); break;              \
      case 2: PQ_QLOW(BB, RR, 2, 512); break;              \
      default: PQ_QLOW(BB, RR, 4, 512); break;             \
    }                                                      \
  } else {                                                 \
    switch (XL) {                                          \
      case 1: PQ_QLOW(BB, RR, 1, 256); break;              \
      case 2: PQ_QLOW(BB, RR, 2, 256); break;              \
      case 4: PQ_QLOW(BB, RR, 4, 256); break;              \
      default: PQ_QLOW(BB, RR, 8, 256); break;             \
    }                                                      \
  }
  if (bits == 4) {
    if (RS == 32) PQ_QLOW_X(4, 32)
    else if (RS == 16) PQ_QLOW_X(4, 16)
    else PQ_QLOW_X(4, 8)
  } else {
    if (RS == 32) PQ_QLOW_X(5, 32)
    else if (RS == 16) PQ_QLOW_X(5, 16)
    else PQ_QLOW_X(5, 8)
  }
#undef PQ_QLOW_X
#undef PQ_QLOW
  int rc = check_launch("pq_qlow_gemv");
  if (rc || !split) return rc;
  launch(qlow_combine_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0, st, wsf, y, yb, N, KS);
  return check_launch("pq_qlow_gemv combine");
}

// The Q4 / Q5 GEMV with x from a prologue (RESNORM, NORM, SILU, CONV), whole
// rows per workgroup (no K split): K = 512 * E for E = 4, 8 or 16, CONV with
// K <= 4096.
extern "C" int pq_qlow_gemv_fused(const uint8_t *pcodes, const uint16_t *pscales, const pq_gemv_prologue *pro,
                                  void *y, int y_dtype, int N, int K, int bits, void *stream) {
  PQ_REQUIRE(pcodes && pscales && pro && y, PQ_ERR_ARG, "pq_qlow_gemv_fused: null pointer");
  PQ_REQUIRE(qlow_shape(N, K, bits) && (K == 2048 || K == 4096 || K == 8192), PQ_ERR_ARG,
             "pq_qlow_gemv_fused: N=%d K=%d bits=%d (N %% 32, K 2048, 4096 or 8192, bits 4 or 5)", N, K, bits);
  PQ_REQUIRE(y_dtype == PQ_DTYPE_F32 || y_dtype == PQ_DTYPE_BF16, PQ_ERR_ARG, "pq_qlow_gemv_fused: y_dtype %d",
             y_dtype);
  PQ_REQUIRE(aligned(pcodes, 16) && aligned(pscales, 4), PQ_ERR_ALIGN,
             "pq_qlow_gemv_fused: packed codes must be 16-byte aligned");
  const pq_gemv_prologue &p = *pro;
  switch (p.kind) {
    case PQ_PRO_RESNORM:
      PQ_REQUIRE(p.h && p.x_in && p.x_out && p.w0 && p.w1 && p.x_in != p.x_out, PQ_ERR_ARG,
                 "pq_qlow_gemv_fused: RESNORM needs h, x_in, x_out (distinct), w0, w1");
      PQ_REQUIRE(aligned(p.h, 16) && aligned(p.x_in, 16) && aligned(p.x_out, 16) && aligned(p.w0, 16) &&
                     aligned(p.w1, 16),
                 PQ_ERR_ALIGN, "pq_qlow_gemv_fused: RESNORM vectors must be 16-byte aligned");
      break;
    case PQ_PRO_NORM:
      PQ_REQUIRE(p.x_in && p.w0, PQ_ERR_ARG, "pq_qlow_gemv_fused: NORM needs x_in, w0");
      PQ_REQUIRE(aligned(p.x_in, 16) && aligned(p.w0, 16), PQ_ERR_ALIGN,
                 "pq_qlow_gemv_fused: NORM vectors must be 16-byte aligned");
      break;
    case PQ_PRO_SILU:
      PQ_REQUIRE(p.gu && aligned(p.gu, 16), PQ_ERR_ARG, "pq_qlow_gemv_fused: SILU needs a 16-byte aligned gu");
      break;
    case PQ_PRO_CONV:
      PQ_REQUIRE(p.bcx && p.ring_in && p.ring_out && p.taps && p.ring_in != p.ring_out &&
                     (p.ntaps == 3 || p.ntaps == 7) && K <= 4096,
                 PQ_ERR_ARG, "pq_qlow_gemv_fused: CONV needs bcx, taps, distinct ring_in / ring_out, ntaps 3 or 7, "
                             "K <= 4096");
      PQ_REQUIRE(aligned(p.bcx, 16) && aligned(p.ring_in, 16) && aligned(p.ring_out, 16) && aligned(p.taps, 16),
                 PQ_ERR_ALIGN, "pq_qlow_gemv_fused: CONV vectors must be 16-byte aligned");
      break;
    default:
      return fail(PQ_ERR_ARG, "pq_qlow_gemv_fused: prologue kind %d (RESNORM, NORM, SILU or CONV)", p.kind);
  }
  const int RS = qlow_rows(N), G = K / kQ, KS = qlow_ks(K);
  const size_t lds = ((size_t)G * kQ + G + 2 * RS * (size_t)qlow_gp(G, RS) + (size_t)KS * RS) * sizeof(float);
  PQ_REQUIRE(lds <= kMaxLds, PQ_ERR_ARG, "pq_qlow_gemv_fused: K=%d exceeds the workgroup's LDS", K);
  const dim3 grid((unsigned)(N / RS)), block(512);
  const int yb = y_dtype == PQ_DTYPE_BF16 ? 1 : 0;
  hipStream_t st = as_stream(stream);
  const uint32_t *ps32 = reinterpret_cast<const uint32_t *>(pscales);
  const int kind = p.kind == PQ_PRO_CONV && p.ntaps == 7 ? kProConv7 : p.kind;
  // one instantiation per (bits, rows per workgroup, prologue, E = K / 512)
#define PQ_QLF(BB, RR, PP, EE) \
  launch(qlow_gemv_kernel<BB, RR, 1, 512, 2, PP, EE>, grid, block, lds, st, pcodes, ps32, nullptr, y, yb, N, K, \
         (float *)nullptr, p)
#define PQ_QLF_E(BB, RR, PP)                  \
  do {                                        \
    if (K == 2048) PQ_QLF(BB, RR, PP, 4);     \
    else if (K == 4096) PQ_QLF(BB, RR, PP, 8); \
    else PQ_QLF(BB, RR, PP, 16);              \
  } while (0)
#define PQ_QLF_CONV(BB, RR, PP)               \
  do {                                        \
    if (K == 2048) PQ_QLF(BB, RR, PP, 4);     \
    else PQ_QLF(BB, RR, PP, 8);               \
  } while (0)
#define PQ_QLF_P(BB, RR)                                                \
  do {                                                                  \
    switch (kind) {                                                     \
      case PQ_PRO_RESNORM: PQ_QLF_E(BB, RR, PQ_PRO_RESNORM); break;     \
      case PQ_PRO_NORM: PQ_QLF_E(BB, RR, PQ_PRO_NORM); break;           \
      case PQ_PRO_SILU: PQ_QLF_E(BB, RR, PQ_PRO_SILU); break;           \
      case kProConv7: PQ_QLF_CONV(BB, RR, kProConv7); break;            \
      default: PQ_QLF_CONV(BB, RR, PQ_PRO_CONV); break;                 \
    }                                                                   \
  } while (0)
  if (bits == 4) {
    if (RS == 32) PQ_QLF_P(4, 32);
    else if (RS == 16) PQ_QLF_P(4, 16);
    else PQ_QLF_P(4, 8);
  } else {
    if (RS == 32) PQ_QLF_P(5, 32);
    else if (RS == 16) PQ_QLF_P(5, 16);
    else PQ_QLF_P(5, 8);
  }
#undef PQ_QLF_P
#undef PQ_QLF_CONV
#undef PQ_QLF_E
#undef PQ_QLF
  return check_launch("pq_qlow_gemv_fused");
}

// The T-position form's shape: rows per workgroup RS and positions per
// workgroup TB, the most positions first (x staged once per position block
// serves RS rows; TB positions share each group's code conversion), then the
// longest row slice, within the LDS and with TB * KS * RS chain lanes <= 512.
static size_t qlow_gemm_lds(int G, int RS, int TB) {
  return ((size_t)TB * G * kQ + (size_t)TB * G + (size_t)TB * RS * qlow_gp(G, RS) + (size_t)RS * qlow_gp(G, RS) +
          (size_t)TB * qlow_ks(G * kQ) * RS) * sizeof(float);
}
static void qlow_gemm_shape(int N, int K, int T, int &RS, int &TB) {
  const int G = K / kQ, KS = qlow_ks(K), XL = (K / 8 + kQgNT - 1) / kQgNT;
  const int tbmax = XL == 1 ? 8 : XL == 2 ? 2 : 1;   // the instantiated (TB, XL) pairs
  RS = 8;
  TB = 1;
  for (int tb = tbmax; tb >= 1; tb >>= 1) {
    if (tb > 1 && tb > T) continue;
    for (int rs = 32; rs >= 8; rs >>= 1)
      if (tb * KS * rs <= kQgNT && qlow_gemm_lds(G, rs, tb) <= kMaxLds && (rs == 8 || N / rs >= 64)) {
        RS = rs;
        TB = tb;
        return;
      }
  }
}

extern "C" int pq_qlow_gemm(const uint8_t *pcodes, const uint16_t *pscales, const uint16_t *x, void *y,
                            int y_dtype, int N, int K, int T, int ldy, int bits, void *stream) {
  PQ_REQUIRE(pcodes && pscales && x && y, PQ_ERR_ARG, "pq_qlow_gemm: null pointer");
  PQ_REQUIRE(qlow_shape(N, K, bits) && T > 0 && ldy >= N, PQ_ERR_ARG,
             "pq_qlow_gemm: N=%d K=%d T=%d ldy=%d bits=%d (N %% 32, K %% 256, K <= 16384, ldy >= N, bits 4 or 5)", N, K,
             T, ldy, bits);
  PQ_REQUIRE((long long)T * K < (1ll << 30) && (long long)T * ldy < (1ll << 31), PQ_ERR_ARG,
             "pq_qlow_gemm: T=%d too large", T);
  PQ_REQUIRE(y_dtype == PQ_DTYPE_F32 || y_dtype == PQ_DTYPE_BF16, PQ_ERR_ARG, "pq_qlow_gemm: y_dtype %d", y_dtype);
  PQ_REQUIRE(aligned(pcodes, 16) && aligned(pscales, 4) && aligned(x, 16), PQ_ERR_ALIGN,
             "pq_qlow_gemm: packed codes and x must be 16-byte aligned");
  int RS, TB;
  qlow_gemm_shape(N, K, T, RS, TB);
  const int G = K / kQ, XL = (K / 8 + kQgNT - 1) / kQgNT;
  const size_t lds = qlow_gemm_lds(G, RS, TB);
  PQ_REQUIRE(lds <= kMaxLds && TB * XL <= 8, PQ_ERR_ARG, "pq_qlow_gemm: K=%d exceeds the workgroup's LDS", K);
  const dim3 grid((unsigned)(N / RS), (unsigned)((T + TB - 1) / TB)), block(kQgNT);
  const int yb = y_dtype == PQ_DTYPE_BF16 ? 1 : 0;
  hipStream_t st = as_stream(stream);
  const uint32_t *ps32 = reinterpret_cast<const uint32_t *>(pscales);
#define PQ_QG(BB, RR, TT, XX) \
  launch(qlow_gemm_kernel<BB, RR, TT, XX>, grid, block, lds, st, pcodes, ps32, x, y, yb, N, K, T, ldy)
#define PQ_QG_T(BB, RR)                                  \
  do {                                                   \
    if (XL == 1) {                                       \
      if (TB == 8) PQ_QG(BB, RR, 8, 1);                  \
      else if (TB == 4) PQ_QG(BB, RR, 4, 1);             \
      else if (TB == 2) PQ_QG(BB, RR, 2, 1);             \
      else PQ_QG(BB, RR, 1, 1);                          \
    } else if (XL == 2) {                                \
      if (TB >= 2) PQ_QG(BB, RR, 2, 2);                  \
      else PQ_QG(BB, RR, 1, 2);                          \
    } else {                                             \
      PQ_QG(BB, RR, 1, 4);                               \
    }                                                    \
  } while (0)
  if (bits == 4) {
    if (RS == 32) PQ_QG_T(4, 32);
    else if (RS == 16) PQ_QG_T(4, 16);
    else PQ_QG_T(4, 8);
  } else {
    if (RS == 32) PQ_QG_T(5, 32);
    else if (RS == 16) PQ_QG_T(5, 16);
    else PQ_QG_T(5, 8);
  }
#undef PQ_QG_T
#undef PQ_QG
  return check_launch("pq_qlow_gemm");
}

// The FFN's gate/up GEMV on a low-bit [gate | up] tensor (N = 2F rows) with a
// RESNORM or NORM prologue and the SwiGLU epilogue: y bf16 [F] = silu(gate) *
// up as pq_silu_mul forms it from the bf16 outputs.
extern "C" int pq_qlow_gemv_fused_swiglu(const uint8_t *pcodes, const uint16_t *pscales, const pq_gemv_prologue *pro,
                                         uint16_t *y, int F, int K, int bits, void *stream) {
  PQ_REQUIRE(pcodes && pscales && pro && y, PQ_ERR_ARG, "pq_qlow_gemv_fused_swiglu: null pointer");
  PQ_REQUIRE(F > 0 && F % 32 == 0 && qlow_shape(2 * F, K, bits) && (K == 2048 || K == 4096 || K == 8192), PQ_ERR_ARG,
             "pq_qlow_gemv_fused_swiglu: F=%d K=%d bits=%d (F %% 32, K 2048, 4096 or 8192, bits 4 or 5)", F, K, bits);
  PQ_REQUIRE(aligned(pcodes, 16) && aligned(pscales, 4), PQ_ERR_ALIGN,
             "pq_qlow_gemv_fused_swiglu: packed codes must be 16-byte aligned");
  const pq_gemv_prologue &p = *pro;
  if (p.kind == PQ_PRO_RESNORM) {
    PQ_REQUIRE(p.h && p.x_in && p.x_out && p.w0 && p.w1 && p.x_in != p.x_out, PQ_ERR_ARG,
               "pq_qlow_gemv_fused_swiglu: RESNORM needs h, x_in, x_out (distinct), w0, w1");
    PQ_REQUIRE(aligned(p.h, 16) && aligned(p.x_in, 16) && aligned(p.x_out, 16) && aligned(p.w0, 16) &&
                   aligned(p.w1, 16),
               PQ_ERR_ALIGN, "pq_qlow_gemv_fused_swiglu: RESNORM vectors must be 16-byte aligned");
  } else if (p.kind == PQ_PRO_NORM) {
    PQ_REQUIRE(p.x_in && p.w0 && aligned(p.x_in, 16) && aligned(p.w0, 16), PQ_ERR_ARG,
               "pq_qlow_gemv_fused_swiglu: NORM needs 16-byte aligned x_in, w0");
  } else {
    return fail(PQ_ERR_ARG, "pq_qlow_gemv_fused_swiglu: prologue kind %d (RESNORM or NORM)", p.kind);
  }
  const int G = K / kQ, KS = qlow_ks(K);
  // rows of each half per workgroup: qlow_rows of the 2F rows, at most 64 / KS
  // (a half's slice chains sit in one wave). Measured, Q4 F = 8192, K = 2048:
  // 32 rows a half (256 workgroups) 8.03 us, as the plain gate/up GEMV's 8.06,
  // against 8.87 at 16 and 12.0 at 8.
  int RS = qlow_rows(2 * F);
  while (RS * KS > 64) RS >>= 1;
  const size_t lds = ((size_t)G * kQ + G + 2 * 2 * RS * (size_t)qlow_gp(G, RS) + (size_t)KS * RS) * sizeof(float);
  PQ_REQUIRE(lds <= kMaxLds, PQ_ERR_ARG, "pq_qlow_gemv_fused_swiglu: K=%d exceeds the workgroup's LDS", K);
  const dim3 grid((unsigned)(F / RS)), block(512);
  hipStream_t st = as_stream(stream);
  const uint32_t *ps32 = reinterpret_cast<const uint32_t *>(pscales);
#define PQ_QSW(BB, RR, PP, EE)                                                                                  \
  launch(qlow_gemv_kernel<BB, RR, 1, 512, 2, PP, EE, true>, grid, block, lds, st, pcodes, ps32, nullptr, y, 1, \
         2 * F, K, (float *)nullptr, p)
#define PQ_QSW_E(BB, RR, PP)                  \
  do {                                        \
    if (K == 2048) PQ_QSW(BB, RR, PP, 4);     \
    else if (K == 4096) PQ_QSW(BB, RR, PP, 8); \
    else PQ_QSW(BB, RR, PP, 16);              \
  } while (0)
#define PQ_QSW_P(BB, RR)                                                          \
  do {                                                                            \
    if (p.kind == PQ_PRO_RESNORM) PQ_QSW_E(BB, RR, PQ_PRO_RESNORM);               \
    else PQ_QSW_E(BB, RR, PQ_PRO_NORM);                                           \
  } while (0)
  if (bits == 4) {
    if (RS == 32) PQ_QSW_P(4, 32);
    else if (RS == 16) PQ_QSW_P(4, 16);
    else PQ_QSW_P(4, 8);
  } else {
    if (RS == 32) PQ_QSW_P(5, 32);
    else if (RS == 16) PQ_QSW_P(5, 16);
    else PQ_QSW_P(5, 8);
  }
#undef PQ_QSW_P
#undef PQ_QSW_E
#undef PQ_QSW
  return check_launch("pq_qlow_gemv_fused_swiglu");
}
