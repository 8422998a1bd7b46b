// pq_internal.h -- entry points the engine shares with the kernels' files but
// that are not part of the C ABI: the decode step with its position and id slot
// on the device, so a captured step replays unchanged.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <memory>
#include <vector>

namespace pq {

// pq_attn_layer_decode with the position read from *pos_dev on the device; LDS
// sized for any position below ctx.
int attn_layer_decode_dev(const uint16_t *qkvg, const float *q_norm, const float *k_norm, const float *rope_cs,
                          uint16_t *kcache, uint16_t *vcache, const int32_t *pos_dev, int ctx, int nh, int nkv, int hd,
                          int rot, int win, float eps, float scale, uint16_t *out, int8_t *qx, float *dx,
                          hipStream_t st);

// pq_qk_prep (pq_qk_prep_ref with kv_bf16) with the launch stream given;
// pos_dev (if not NULL) holds the position of row 0 on the device instead of
// pos0.
int qk_prep_launch(uint16_t *qkv, int row_stride, const float *q_norm, const float *k_norm, const float *rope_cs,
                   uint16_t *kcache, uint16_t *vcache, int pos0, const int32_t *pos_dev, int nh, int nkv, int hd,
                   int rot, int T, float eps, hipStream_t st, bool kv_bf16 = false);

// pq_attn_ref for one query at the device position *pos_dev (keys up to it,
// window win); LDS sized for positions below ctx.
int attn_ref_dev(const uint16_t *q, int q_stride, const uint16_t *kcache, const uint16_t *vcache,
                 const uint16_t *gate, int gate_stride, uint16_t *out, int out_stride, const int32_t *pos_dev,
                 int ctx, int nh, int nkv, int hd, float scale, int win, hipStream_t st);

// The gate rows of a layer as a Q8 part of their own, for the attention to
// form: [nh][K] int8 codes, [nh][K/32] fp32 scales, applied to
// rmsnorm(x, w) of the bf16 residual x (K = 2048).
struct AttnGateQ8 {
  const int8_t *codes;
  const float *scales;
  const uint16_t *x;
  const float *w;
  float eps;
  int K;
};

// pq_attn_decode_ref at the device position *pos_dev (null: at pos); LDS
// sized for positions below ctx. gq8 non-null: the head gates formed in the
// launch from those rows (gate is then not read).
int attn_decode_ref_dev(const uint16_t *qkv, const float *q_norm, const float *k_norm, const float *rope_cs,
                        uint16_t *kcache, uint16_t *vcache, const uint16_t *gate, uint16_t *out, int pos,
                        const int32_t *pos_dev, int ctx, int nh, int nkv, int hd, int rot, float eps, float scale,
                        int win, hipStream_t st, const AttnGateQ8 *gq8 = nullptr);

// pq_attn_decode for one query at the device position *pos_dev (keys up to
// it, window win), sized for positions below ctx.
int attn_decode_dev(const uint16_t *q, int q_stride, const uint16_t *kcache, const uint16_t *vcache,
                    const uint16_t *gate, int gate_stride, uint16_t *out, int out_stride, int8_t *qx, float *dx,
                    const int32_t *pos_dev, int ctx, int nh, int nkv, int hd, float scale, int win, void *ws,
                    size_t ws_bytes, hipStream_t st);

// pq_argmax_parts that also appends the id: ids[ctr[0]++] = id, ctr[1]++.
int argmax_parts_step(const float *parts, int nparts, int32_t *out, int32_t *ids, int32_t *ctr, hipStream_t st);

// zlib-compatible crc32 (blob.cpp).
uint32_t crc32_update(uint32_t crc, const void *data, size_t n);

// Index of the blob tensor called name, or -1.
int blob_find(void *blob, const char *name);

// Reads the blob tensors listed in order (table indices) on a thread of its
// own, each into a host buffer (codes then scales) with its crc checked, at
// most depth ahead of the caller; take() hands them over in order.
class BlobReader {
 public:
  BlobReader(void *blob, const std::vector<int> &order, size_t depth);
  ~BlobReader();
  int take(std::vector<char> &out);

 private:
  struct Impl;
  std::unique_ptr<Impl> impl;
};

}  // namespace pq
