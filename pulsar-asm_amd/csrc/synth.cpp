// synth.cpp -- synthetic-model generator (host side): the stand-in for a
// checkpoint, since none is available offline.
//
// splitmix64 (Steele, Lea, Flood, OOPSLA 2014) used counter-style: output n of
// a stream seeded with s is mix(s + (n+1)*GAMMA), so any element is generated
// independently and tensors are filled by several threads.
//   codes:   element i = 16-bit lane i%4 of word i/4, c = (u16*255)>>16 - 127
//   normal:  word i -> u1 = (hi32+1)/2^32, u2 = lo32/2^32,
//            z = sqrt(-2 ln u1) cos(2 pi u2) in double, rounded to float
//   scales:  f16(fl(|z| * mult))
//   affine:  fl(a + fl(b * z))
//   ternary: code i = byte i%8 of word i/8, c = (u8*3)>>8 in {0,1,2}
//   tokens:  (word i >> 32) % vocab
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <algorithm>
#include <thread>
#include <vector>

#include "../../include/pulsar_amd.h"

namespace pq {

static constexpr uint64_t kGamma = 0x9e3779b97f4a7c15ull;

static inline uint64_t mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}
static inline uint64_t at(uint64_t seed, uint64_t n) { return mix(seed + (n + 1) * kGamma); }

static inline float normal(uint64_t v) {
  const double u1 = ((double)(v >> 32) + 1.0) * (1.0 / 4294967296.0);
  const double u2 = (double)(v & 0xffffffffu) * (1.0 / 4294967296.0);
  return (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586476925 * u2));
}

static inline uint16_t to_half(float f) {
  const _Float16 h = (_Float16)f;  // IEEE round-to-nearest-even
  uint16_t b;
  memcpy(&b, &h, 2);
  return b;
}

template <typename F>
static void parallel_for(size_t n, F fn) {
  const unsigned hw = std::max(1u, std::min(32u, std::thread::hardware_concurrency()));
  if (n < (1u << 16) || hw == 1) {
    fn((size_t)0, n);
    return;
  }
  std::vector<std::thread> th;
  const size_t step = (n + hw - 1) / hw;
  for (unsigned t = 0; t < hw; t++) {
    const size_t a = t * step, b = std::min(n, a + step);
    if (a < b) th.emplace_back(fn, a, b);
  }
  for (auto &x : th) x.join();
}

}  // namespace pq

using namespace pq;

extern "C" int pq_synth_fill(int kind, uint64_t seed, void *out, size_t n, float a, float b) {
  if (out == nullptr && n > 0) return PQ_ERR_ARG;
  switch (kind) {
    case PQ_SYNTH_CODES: {
      int8_t *o = static_cast<int8_t *>(out);
      parallel_for((n + 3) / 4, [&](size_t w0, size_t w1) {
        for (size_t w = w0; w < w1; w++) {
          const uint64_t v = at(seed, w);
          for (int k = 0; k < 4; k++) {
            const size_t i = w * 4 + k;
            if (i < n) o[i] = (int8_t)((int)((((v >> (16 * k)) & 0xffffu) * 255u) >> 16) - 127);
          }
        }
      });
      return PQ_OK;
    }
    case PQ_SYNTH_NORMAL: {
      float *o = static_cast<float *>(out);
      parallel_for(n, [&](size_t i0, size_t i1) {
        for (size_t i = i0; i < i1; i++) o[i] = normal(at(seed, i));
      });
      return PQ_OK;
    }
    case PQ_SYNTH_SCALES: {
      uint16_t *o = static_cast<uint16_t *>(out);
      parallel_for(n, [&](size_t i0, size_t i1) {
        for (size_t i = i0; i < i1; i++) o[i] = to_half(fabsf(normal(at(seed, i))) * a);
      });
      return PQ_OK;
    }
    case PQ_SYNTH_AFFINE: {
      float *o = static_cast<float *>(out);
      for (size_t i = 0; i < n; i++) {
        const float z = normal(at(seed, i));
        const float bz = b * z;
        o[i] = a + bz;
      }
      return PQ_OK;
    }
    case PQ_SYNTH_TERNARY: {
      uint8_t *o = static_cast<uint8_t *>(out);
      parallel_for(n, [&](size_t b0, size_t b1) {
        for (size_t by = b0; by < b1; by++) {
          uint8_t r = 0;
          for (int k = 0; k < 4; k++) {
            const size_t i = by * 4 + k;
            const uint32_t u8 = (uint32_t)(at(seed, i / 8) >> (8 * (i % 8))) & 0xffu;
            r |= (uint8_t)(((u8 * 3u) >> 8) << (2 * k));
          }
          o[by] = r;
        }
      });
      return PQ_OK;
    }
    case PQ_SYNTH_TOKENS: {
      int32_t *o = static_cast<int32_t *>(out);
      const uint64_t vocab = (uint64_t)a;
      if (vocab == 0) return PQ_ERR_ARG;
      for (size_t i = 0; i < n; i++) o[i] = (int32_t)((at(seed, i) >> 32) % vocab);
      return PQ_OK;
    }
    default:
      return PQ_ERR_ARG;
  }
}
