// pq_device.h -- device-side scalar helpers shared by every gfx950 kernel.
//
// All HIP sources are compiled with -ffp-contract=off: a fused multiply-add is
// written as __builtin_fmaf, every other a*b+c rounds twice. Division and
// sqrtf are the correctly rounded forms (hipcc's default for HIP), so host and
// device agree on them bit for bit.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pq {

// bf16 <-> f32. bf16 is raw 16-bit storage; f32 -> bf16 is round-to-nearest-
// even with inf/nan passed through (lfm3_nanode.cu:114-121), written out in
// integer steps here (f2bf_bits) and done by gfx950's v_cvt_pk_bf16_f32 in
// f2bf / f2bf2 (pq_check_bf16_cvt compares the two over all 2^32 inputs).
__device__ __forceinline__ float bf2f(uint16_t v) { return __uint_as_float(((uint32_t)v) << 16); }
__device__ __forceinline__ uint16_t f2bf_bits(float v) {
  const uint32_t u = __float_as_uint(v);
  if (((u >> 23) & 0xffu) == 0xffu) return (uint16_t)(u >> 16);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
typedef float pq_f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 pq_bf16x2 __attribute__((ext_vector_type(2)));
// (bf16(a), bf16(b)) packed low, high: one v_cvt_pk_bf16_f32
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
  const pq_f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, pq_bf16x2));
}
__device__ __forceinline__ uint16_t f2bf(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }
// x rounded to bf16 and back
__device__ __forceinline__ float bfr(float v) { return bf2f(f2bf(v)); }
// a, b rounded to bf16 in place (one convert for the pair); returns the pair's
// bf16 bits packed low, high
__device__ __forceinline__ uint32_t bfr2(float &a, float &b) {
  const uint32_t w = f2bf2(a, b);
  a = __uint_as_float(w << 16);
  b = __uint_as_float(w & 0xffff0000u);
  return w;
}

// Correctly rounded a / d for many a over one divisor d with
// 2^-90 <= |d| <= 2^100: the divide sequence with the divisor's part done
// once -- r = rcp(d) refined by one Newton step, then per quotient q = a*r and
// two remainder corrections q += r*(a - d*q), each an fma. In that range the
// hardware divide's operand scaling is the identity and its fixup passes a
// finite quotient through, so the steps are the same as a / d's.
struct SharedDiv {
  float d, r;
  __device__ __forceinline__ explicit SharedDiv(float dv) : d(dv) {
    const float r0 = __builtin_amdgcn_rcpf(dv);
    r = __builtin_fmaf(__builtin_fmaf(-dv, r0, 1.0f), r0, r0);
  }
  __device__ __forceinline__ float div(float a) const {
    float q = a * r;
    q = __builtin_fmaf(__builtin_fmaf(-d, q, a), r, q);
    return __builtin_fmaf(__builtin_fmaf(-d, q, a), r, q);
  }
};
// The Q8_0 quotient x / d of a block (d = amax/127), without branches: a d
// outside SharedDiv's range is brought into it by an exact power-of-two scale
// of both operands (the quotient of the scaled pair is the same real number,
// so the same rounded one; x is at most ~127.5 |d|, so scaling it up cannot
// overflow, and an x that underflows when scaled down is below 2^-100 |d|,
// whose code is 0 either way). d = 0 (an all-zero block up to values below
// 127 * 2^-149) divides by 1, whose codes are 0 as the zero-block rule wants.
// pq_check_quant_div compares the codes with x / d's on the GPU.
struct Q8Div {
  float sc;
  SharedDiv sd;
  __device__ __forceinline__ static float scale_of(float d) {
    const float m = __builtin_fabsf(d);
    return m < 0x1p-90f ? 0x1p64f : (m > 0x1p100f ? 0x1p-64f : 1.0f);
  }
  __device__ __forceinline__ explicit Q8Div(float d)
      : sc(scale_of(d != 0.0f ? d : 1.0f)), sd((d != 0.0f ? d : 1.0f) * scale_of(d != 0.0f ? d : 1.0f)) {}
  __device__ __forceinline__ float div(float x) const { return sd.div(x * sc); }
};
// Q8_0 code of x in a block with scale d (d = amax/127; d = 0 only for an
// all-zero block, whose codes are 0): rne(x/d) clamped to [-127, 127]
__device__ __forceinline__ int q8_code(float q) {
  const int c = (int)__builtin_rintf(q);
  return c > 127 ? 127 : (c < -127 ? -127 : c);
}

// binary16 <-> f32 through the hardware converts (v_cvt_f32_f16 is exact;
// v_cvt_f16_f32 rounds to nearest even and keeps subnormals).
__device__ __forceinline__ float h2f(uint16_t h) {
  return __builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f2h(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// e^x with the build's one definition: Cody & Waite reduction
// n = rint(x*log2 e), r = (x - n*ln2_hi) - n*ln2_lo, degree-7 Taylor
// polynomial in Horner form, then two exact power-of-two factors so only the
// last multiply rounds. Identical operation sequence on the host side.
__device__ __forceinline__ float expf_pq(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return __builtin_inff();
  if (x < -104.0f) return 0.0f;
  const float n = __builtin_rintf(x * 1.44269502162933349609375f);
  float r = __builtin_fmaf(n, -0.693145751953125f, x);
  r = __builtin_fmaf(n, -1.428606765330187045e-06f, r);
  float p = 1.98412698412698412e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int a = ni / 2, b = ni - a;
  const float fa = __uint_as_float((uint32_t)(a + 127) << 23);
  const float fb = __uint_as_float((uint32_t)(b + 127) << 23);
  return (p * fa) * fb;
}

// Wave64 xor-butterfly reductions. After step k every aligned group of 2^k
// lanes holds the same value, so the partner of step k can be any lane of the
// neighbouring group: steps 1-2 are DPP quad permutes (lane ^ 1, lane ^ 2),
// steps 3-4 DPP half-row / row mirrors (lane i <-> 7-i, 15-i), steps 5-6 the
// gfx950 permlane16/32 swaps. Every lane ends with the pairwise (balanced
// binary) sum of the 64 lanes' values in lane order -- the order the host side
// writes as a recursive halving sum. All 64 lanes must be active.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppXor1 = 0xb1, kDppXor2 = 0x4e, kDppHalfMirror = 0x141, kDppMirror = 0x140;
constexpr int kDppRowShr1 = 0x111;   // lane i takes lane i - 1 of its 16-lane row

// v + (the value of the other 16-lane row of the pair), rows uniform
__device__ __forceinline__ float add_row_pair(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_half_pair(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float max_row_pair(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_half_pair(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float wave_pairwise_sum(float v) {
  v = v + dpp_f<kDppXor1>(v);
  v = v + dpp_f<kDppXor2>(v);
  v = v + dpp_f<kDppHalfMirror>(v);
  v = v + dpp_f<kDppMirror>(v);
  v = add_row_pair(v);
  return add_half_pair(v);
}
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  v = max_row_pair(v);
  return max_half_pair(v);
}

// Workgroup barrier over LDS only: waits for this wave's LDS operations, not for
// its outstanding global loads, so weight loads issued before a prologue stay
// in flight while the prologue runs.
__device__ __forceinline__ void lds_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0); vmcnt and expcnt left alone
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// An LDS pointer whose address sits in one VGPR the optimizer cannot split
// into a uniform and a per-lane part: reads at constant offsets from it fold
// into the DS instruction's offset field, where a split address costs one
// VALU add per read. p must point into LDS.
template <typename T>
using lds_ptr = const __attribute__((address_space(3))) T *;
template <typename T>
__device__ __forceinline__ lds_ptr<T> lds_base(const T *p) {
  uint32_t a = (uint32_t)(size_t)(lds_ptr<T>)p;
  asm("" : "+v"(a));
  return (lds_ptr<T>)(size_t)a;
}

// Keys a query at npos - 1 sees: [lo, npos), lo = npos - win for a sliding
// layer whose window the context has outgrown (k_attn_head, lfm3_nanode.cu:515).
__device__ __forceinline__ int window_lo(int npos, int win) { return (win > 0 && npos > win) ? npos - win : 0; }

// ------------------------------------------ the reference's reduction orders
// v + (the value D lanes up), exact at every lane l with l mod 2D < D (the
// lanes a shfl_down tree step reads on): D = 1, 2 by quad permutes, 4 and 8
// by 16-lane row rotates (row_ror:n reads lane l - n mod 16), 16 and 32 by the
// permlane row / half swaps (lane for lane).
template <int D>
__device__ __forceinline__ float add_down(float v) {
  if constexpr (D == 1) return v + dpp_f<kDppXor1>(v);
  else if constexpr (D == 2) return v + dpp_f<kDppXor2>(v);
  else if constexpr (D == 4) return v + dpp_f<0x12c>(v);   // row_ror:12
  else if constexpr (D == 8) return v + dpp_f<0x128>(v);   // row_ror:8
  else if constexpr (D == 16) return add_row_pair(v);
  else return add_half_pair(v);
}

// One step (offset O, in reference threads) of the shfl_down tree of
// rmsnorm_body over a thread's t[R] (R reference threads per lane, or LPR
// lanes per reference thread).
template <int E, int O>
__device__ __forceinline__ void ref_tree_step(float *t) {
  constexpr int R = E >= 8 ? E / 8 : 1, LPR = E >= 8 ? 1 : 8 / E;
  if constexpr (O >= R) {
#pragma unroll
    for (int j = 0; j < R; j++) t[j] = add_down<(O / R) * LPR>(t[j]);
  } else {
#pragma unroll
    for (int j = 0; j + O < R; j++) t[j] = t[j] + t[j + O];
  }
}

// ((p[0] + p[1]) + p[2]) + ... over NP values of LDS, all read first.
template <int NP>
__device__ __forceinline__ float ordered_sum_n(const float *p) {
  float v[NP];
  if constexpr (NP % 4 == 0) {
#pragma unroll
    for (int i = 0; i < NP / 4; i++) {
      const float4 q = reinterpret_cast<const float4 *>(p)[i];
      v[4 * i] = q.x;
      v[4 * i + 1] = q.y;
      v[4 * i + 2] = q.z;
      v[4 * i + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NP; i++) v[i] = p[i];
  }
  float t = v[0];
#pragma unroll
  for (int i = 1; i < NP; i++) t = t + v[i];
  return t;
}
// the same for n = 1, 2, 4, .. 32 (a uniform branch); p 16-byte aligned
__device__ __forceinline__ float ordered_sum(const float *p, int n) {
  switch (n) {
    case 1: return p[0];
    case 2: return ordered_sum_n<2>(p);
    case 4: return ordered_sum_n<4>(p);
    case 8: return ordered_sum_n<8>(p);
    case 16: return ordered_sum_n<16>(p);
    default: return ordered_sum_n<32>(p);
  }
}

// The sum of squares of RMSNorm in the reference's order (rmsnorm_body,
// lfm3_nanode.cu:383-440): a thread of 8 consecutive elements sums their
// squares pairwise, a warp of 32 such threads folds them with the shfl_down
// tree (offsets 16, 8, 4, 2, 1: s_l + s_{l+o}), and the warp partials (one per
// 256 elements) add in order from the first. Here workgroup thread t holds
// elements tE .. tE + E - 1 (E = 4 .. 32): a reference thread is a lane pair
// (E = 4) or an 8-element piece of a lane, and the tree's offsets become lane
// offsets or sums within the lane. part (16-byte aligned LDS) gets the
// nparts = n/256 partials (1, 2, 4, .. 32; one barrier, LDS-only with LDSB);
// every thread returns the total. ref_sumsq_part is the part before the
// barrier for threads t = 0, 1, .. of a group that starts at a wave boundary
// (t = threadIdx.x - a multiple of 64).
template <int E>
__device__ __forceinline__ void ref_sumsq_part(const float *v, float *part, int t_in_group) {
  static_assert(E == 4 || E == 8 || E == 16 || E == 32, "4 .. 32 elements per thread");
  constexpr int R = E >= 8 ? E / 8 : 1, LPR = E >= 8 ? 1 : 8 / E;
  float t[R];
  if constexpr (E == 4) {
    t[0] = add_down<1>((v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]));
  } else {
#pragma unroll
    for (int j = 0; j < R; j++) {
      const float *e = v + 8 * j;
      t[j] = ((e[0] * e[0] + e[1] * e[1]) + (e[2] * e[2] + e[3] * e[3])) +
             ((e[4] * e[4] + e[5] * e[5]) + (e[6] * e[6] + e[7] * e[7]));
    }
  }
  ref_tree_step<E, 16>(t);
  ref_tree_step<E, 8>(t);
  ref_tree_step<E, 4>(t);
  ref_tree_step<E, 2>(t);
  ref_tree_step<E, 1>(t);
  constexpr int S = 32 * LPR / R;   // lanes per reference warp
  const int lane = threadIdx.x & 63;
  if ((lane & (S - 1)) == 0) part[(t_in_group >> 6) * (64 / S) + lane / S] = t[0];
}
template <int E, bool LDSB>
__device__ __forceinline__ float ref_sumsq(const float *v, float *part, int nparts) {
  ref_sumsq_part<E>(v, part, threadIdx.x);
  if constexpr (LDSB) lds_barrier();
  else __syncthreads();
  return ordered_sum(part, nparts);
}

// The sum of squares of a head norm in the reference's order (k_headnorm,
// lfm3_nanode.cu:460-479): 32 threads of HD/32 consecutive elements (4 at
// HD = 128; HD = 64, which the reference does not run, takes 2), each summed
// pairwise, then the shfl_down tree; the trailing + 0 of the reference leaves
// a sum of squares unchanged. Lane l of the wave holds elements l and l + 64
// (x[0], x[1]) at HD = 128, element l at HD = 64; every lane gets lane 0's
// total.
template <int HD>
__device__ __forceinline__ float head_sumsq(const float *x) {
  float s;
  if constexpr (HD == 128) {   // thread m < 16: lanes 4m..4m+3 of x[0]; m >= 16: of x[1]
    float a = x[0] * x[0], b = x[1] * x[1];
    a = add_down<2>(add_down<1>(a));
    b = add_down<2>(add_down<1>(b));
    s = a + b;                 // offset 16: threads m and m + 16 share lane 4m
    s = add_down<32>(s);       // 8
    s = add_down<16>(s);       // 4
    s = add_down<8>(s);        // 2
    s = add_down<4>(s);        // 1
  } else {                     // thread m: lanes 2m, 2m + 1
    s = add_down<1>(x[0] * x[0]);
    s = add_down<32>(s);
    s = add_down<16>(s);
    s = add_down<8>(s);
    s = add_down<4>(s);
    s = add_down<2>(s);
  }
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 0));
}

// q/k head norm + RoPE from preloaded inputs: x[e] and wv[e] are element
// lane + 64e of the head and of its norm weight, (c, sn) the cos/sin of the
// lane's RoPE pair: pair lane & 31 for head_dim 64 (elements i and i + 32
// sit in lanes i and i + 32), pair lane for head_dim 128 (elements lane and
// lane + 64 in one lane). The arithmetic of qk_prep_kernel
// (shared by the fused attention launches).
template <int HD>
__device__ __forceinline__ void norm_rope(const float *x, const float *wv, float c, float sn, int rot, float eps,
                                          int lane, float *r) {
  constexpr int E = HD / 64;
  float v[E];
  const float rs = 1.0f / sqrtf(head_sumsq<HD>(x) * (1.0f / (float)HD) + eps);
#pragma unroll
  for (int e = 0; e < E; e++) v[e] = bf2f(f2bf(wv[e] * bf2f(f2bf(x[e] * rs))));
  const int half = rot / 2;
  if constexpr (HD == 64) {
    const float up = __shfl_down(v[0], 32, 64);
    const float dn = __shfl_up(v[0], 32, 64);
    r[0] = v[0];
    if ((lane & 31) < half) r[0] = lane < 32 ? v[0] * c - up * sn : v[0] * c + dn * sn;
  } else {
    r[0] = v[0];
    r[1] = v[1];
    if (lane < half) {
      r[0] = v[0] * c - v[1] * sn;
      r[1] = v[1] * c + v[0] * sn;
    }
  }
#pragma unroll
  for (int e = 0; e < E; e++) r[e] = bf2f(f2bf(r[e]));
}

// Greedy argmax in the reference's order (k_argmax, lfm3_nanode.cu:942-964):
// its 256 threads scan i = tid, tid + 256, ... keeping the first strict
// maximum above -1e30 (kAmFloor), then two shfl_down trees (the 32 lanes of a
// warp, then the 8 warps) keep the lower lane's pair unless the other's value
// is strictly larger. Among equal maxima the last tree step weighs most: the
// pick has the smallest (bitrev3(warp), bitrev5(lane)) of its thread slot
// i mod 256, then the smallest i. am_key orders indices that way (no index,
// -1: the largest key); the pick is the largest value, then the smallest key,
// a total order that any reduction tree reproduces. No value above kAmFloor
// gives -1, as the reference's does.
constexpr float kAmFloor = -1e30f;
__device__ __forceinline__ uint32_t am_key(int i) {
  if (i < 0) return 0xffffffffu;
  const uint32_t s = (uint32_t)i & 255u, w = s >> 5, l = s & 31u;
  const uint32_t bw = ((w & 1u) << 2) | (w & 2u) | (w >> 2);
  const uint32_t bl = ((l & 1u) << 4) | ((l & 2u) << 2) | (l & 4u) | ((l >> 2) & 2u) | (l >> 4);
  return (((bw << 5) | bl) << 24) | ((uint32_t)i >> 8);
}
// (v, i) picked over (bv, bi)
__device__ __forceinline__ bool am_better(float v, int i, float bv, int bi) {
  return v > bv || (v == bv && am_key(i) < am_key(bi));
}
// a candidate (v, i): itself when v > kAmFloor, else no index
__device__ __forceinline__ void am_leaf(float v, int i, float &bv, int &bi) {
  const bool ok = v > kAmFloor;
  bv = ok ? v : kAmFloor;
  bi = ok ? i : -1;
}

}  // namespace pq
