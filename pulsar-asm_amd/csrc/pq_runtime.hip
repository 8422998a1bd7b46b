// pq_runtime.hip -- error state and version of the C ABI.
#include <string.h>

#include "pq_device.h"
#include "pq_host.h"

namespace pq {

static thread_local char g_err[512] = "";

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

TimedLaunch &timed_launch() {
  static thread_local TimedLaunch t;
  return t;
}

// Block b checks the float bit patterns [b*2^16, (b+1)*2^16): the hardware
// conversion (single and packed forms) against the integer-step rounding.
// Writes the block's mismatch count and its lowest mismatching pattern
// (0xffffffff if none). Per-thread vector stores only.
__global__ __launch_bounds__(256) void bf16_cvt_check_kernel(uint32_t *__restrict__ counts,
                                                             uint32_t *__restrict__ first) {
  __shared__ uint32_t sc[256], sf[256];
  const uint32_t base = (uint32_t)blockIdx.x << 16;
  uint32_t n = 0, f = 0xffffffffu;
  for (uint32_t j = 0; j < 256; j += 2) {
    const uint32_t u0 = base + threadIdx.x + 256u * j, u1 = u0 + 256u;
    const float a = __uint_as_float(u0), b = __uint_as_float(u1);
    const uint32_t want = (uint32_t)f2bf_bits(a) | ((uint32_t)f2bf_bits(b) << 16);
    const uint32_t pk = f2bf2(a, b);
    const uint32_t sg = (uint32_t)f2bf(a) | ((uint32_t)f2bf(b) << 16);
    const bool bad0 = (pk & 0xffffu) != (want & 0xffffu) || (sg & 0xffffu) != (want & 0xffffu);
    const bool bad1 = (pk >> 16) != (want >> 16) || (sg >> 16) != (want >> 16);
    n += (uint32_t)bad0 + (uint32_t)bad1;
    if (bad0 && u0 < f) f = u0;
    if (bad1 && u1 < f) f = u1;
  }
  sc[threadIdx.x] = n;
  sf[threadIdx.x] = f;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      sc[threadIdx.x] += sc[threadIdx.x + o];
      sf[threadIdx.x] = sf[threadIdx.x] < sf[threadIdx.x + o] ? sf[threadIdx.x] : sf[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    counts[blockIdx.x] = sc[0];
    first[blockIdx.x] = sf[0];
  }
}

__device__ __forceinline__ uint32_t mix32(uint32_t x) {   // an integer hash (xorshift-multiply rounds)
  x ^= x >> 16;
  x *= 0x7feb352du;
  x ^= x >> 15;
  x *= 0x846ca68bu;
  x ^= x >> 16;
  return x;
}

// Each thread draws a block maximum amax (exponent field 0..254 -- subnormal
// to the largest binade -- and mantissa at random; thread 0 of each block
// takes amax = 0), d = amax/127 as the quantizers form it, and 64 values v of
// that block: uniform multiples of d in [-128d, 128d], the rounded
// half-integers (k + 1/2)*d and their neighbours within 2 ulps, small values,
// and +-amax, each clamped to [-amax, amax]. A mismatch: the Q8_0 code of Q8Div's quotient differs from that
// of v / d (v / 1 for d = 0), or (for |v| >= 2^-20 |d| and a normal v) the
// quotients differ at all.
__global__ __launch_bounds__(256) void quant_div_check_kernel(uint32_t *__restrict__ counts,
                                                              uint32_t *__restrict__ first, uint32_t seed) {
  __shared__ uint32_t sc[256], sf[256];
  const uint32_t tid = blockIdx.x * 256u + threadIdx.x;
  uint32_t h = mix32(tid ^ mix32(seed));
  const uint32_t e = h % 255u;
  h = mix32(h);
  const float amax = threadIdx.x == 0 ? 0.0f : __uint_as_float((e << 23) | (h & 0x7fffffu));
  const float d = amax / 127.0f;
  uint32_t n = 0, f = 0xffffffffu;
  {
    const Q8Div qd(d);
    const float dd = d != 0.0f ? d : 1.0f;
    for (uint32_t j = 0; j < 64; j++) {
      h = mix32(h + j);
      const float sgn = (h & 1u) ? -1.0f : 1.0f;
      float v;
      switch (j & 3u) {
        case 0: v = d * ((float)(h >> 8) * 0x1p-24f * 256.0f - 128.0f); break;
        case 1: {
          const float t = d * ((float)((int)((h >> 4) & 255u) - 128) + 0.5f);
          v = __uint_as_float(__float_as_uint(t) + ((h >> 12) % 5u) - 2u);
          break;
        }
        case 2: v = sgn * d * __uint_as_float(((127u - 1u - ((h >> 4) % 60u)) << 23) | ((h >> 9) & 0x7fffffu)); break;
        default: v = sgn * amax; break;
      }
      v = fminf(fmaxf(v, -amax), amax);   // a block's values lie within its amax
      const float qi = v / dd, qs = qd.div(v);
      const bool exact = __builtin_fabsf(v) >= __builtin_fabsf(d) * 0x1p-20f && __builtin_fabsf(v) >= 0x1p-126f;
      const bool bad = q8_code(qi) != q8_code(qs) || (exact && __float_as_uint(qi) != __float_as_uint(qs));
      n += bad ? 1u : 0u;
      if (bad && tid < f) f = tid;
    }
  }
  sc[threadIdx.x] = n;
  sf[threadIdx.x] = f;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) {
      sc[threadIdx.x] += sc[threadIdx.x + o];
      sf[threadIdx.x] = sf[threadIdx.x] < sf[threadIdx.x + o] ? sf[threadIdx.x] : sf[threadIdx.x + o];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    counts[blockIdx.x] = sc[0];
    first[blockIdx.x] = sf[0];
  }
}

// One wave: shader clock cycles (s_memtime) against the 100 MHz real-time
// counter (s_memrealtime) over a bounded dependent-FMA loop of ~0.2 ms.
__global__ __launch_bounds__(64) void clock_probe_kernel(float *__restrict__ out, int iters) {
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), r0 = wall_clock64();
  float x = (float)threadIdx.x;
  for (int i = 0; i < iters; i++) x = __builtin_fmaf(x, 0.999999f, 1e-7f);
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), r1 = wall_clock64();
  if (threadIdx.x == 0) {
    out[0] = (float)((double)(c1 - c0) / (double)(r1 - r0) * 100.0);   // MHz
    out[1] = x;   // keeps the loop
  }
}

// A plain streaming read of n16 16-byte pieces: 1024 workgroups of 512
// threads, one nontemporal 16-byte load per lane per grid-stride step and no
// arithmetic beyond an xor, so its launch period is what a kernel that only
// streams the same bytes achieves -- the practical ceiling a GEMV launch of
// that size is read against. sink is written only if the xor of the data hits
// a value it cannot for the caller's buffers (the loads stay live).
typedef int piece16 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(512) void stream_read_kernel(const piece16 *__restrict__ p, long long n16,
                                                          float *__restrict__ sink) {
  int acc = 0;
  for (long long i = (long long)blockIdx.x * 512 + threadIdx.x; i < n16; i += (long long)gridDim.x * 512) {
    const piece16 v = __builtin_nontemporal_load(p + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x7eadbeef) sink[0] = (float)acc;
}

}  // namespace pq

extern "C" int pq_stream_read(const void *p, size_t bytes, float *sink, void *stream) {
  PQ_REQUIRE(p && sink && bytes % 16 == 0, PQ_ERR_ARG, "pq_stream_read: p, sink and a multiple of 16 bytes");
  PQ_REQUIRE(pq::aligned(p, 16), PQ_ERR_ALIGN, "pq_stream_read: p must be 16-byte aligned");
  pq::launch(pq::stream_read_kernel, dim3(1024), dim3(512), 0, pq::as_stream(stream),
             static_cast<const pq::piece16 *>(p), (long long)(bytes / 16), sink);
  return pq::check_launch("pq_stream_read");
}

extern "C" int pq_clock_mhz(float *out, void *stream) {
  PQ_REQUIRE(out, PQ_ERR_ARG, "pq_clock_mhz: null pointer");
  pq::launch(pq::clock_probe_kernel, dim3(1), dim3(64), 0, pq::as_stream(stream), out, 50000);
  return pq::check_launch("pq_clock_mhz");
}

extern "C" int pq_check_quant_div(uint32_t *counts, uint32_t *first, uint32_t seed, void *stream) {
  PQ_REQUIRE(counts && first, PQ_ERR_ARG, "pq_check_quant_div: null pointer");
  pq::launch(pq::quant_div_check_kernel, dim3(65536), dim3(256), 0, pq::as_stream(stream), counts, first, seed);
  return pq::check_launch("pq_check_quant_div");
}

extern "C" int pq_check_bf16_cvt(uint32_t *counts, uint32_t *first, void *stream) {
  PQ_REQUIRE(counts && first, PQ_ERR_ARG, "pq_check_bf16_cvt: null pointer");
  pq::launch(pq::bf16_cvt_check_kernel, dim3(65536), dim3(256), 0, pq::as_stream(stream), counts, first);
  return pq::check_launch("pq_check_bf16_cvt");
}

extern "C" const char *pq_version(void) { return "pulsar-amd 0.1 gfx950"; }

extern "C" const char *pq_last_error(void) { return pq::g_err; }

extern "C" int pq_time_next_launch(void *start_event, void *stop_event) {
  PQ_REQUIRE((start_event == nullptr) == (stop_event == nullptr), PQ_ERR_ARG,
             "pq_time_next_launch: pass both events or neither");
  pq::TimedLaunch &t = pq::timed_launch();
  t.start = reinterpret_cast<hipEvent_t>(start_event);
  t.stop = reinterpret_cast<hipEvent_t>(stop_event);
  return PQ_OK;
}
