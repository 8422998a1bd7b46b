/* pulsar_amd.h -- C ABI of the MI355X (gfx950) hot path of PULSAR-ASM's LFM3 engine.
 *
 * Plain pointers and sizes only. All pointers are DEVICE pointers unless a
 * parameter says host. Every entry point:
 *   - launches on the HIP stream passed as `stream` (a hipStream_t; NULL = the
 *     null stream) and returns without synchronizing;
 *   - returns 0 on success or a negative PQ_ERR_* code, and never exits or
 *     prints (pq_last_error() gives the message of the calling thread's last
 *     failure) -- the reference prints and exit(2)s (lfm3_nanode.cu:1927-1929)
 *     or returns 1 (lfm3_nanode.cu:4956-4967);
 *   - allocates nothing (buffers are the caller's).
 * Paths in comments are relative to the PULSAR-ASM tree.
 */
#ifndef PULSAR_AMD_H
#define PULSAR_AMD_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PQ_OK 0
#define PQ_ERR_ARG (-1)        /* bad size, null pointer or unsupported shape   */
#define PQ_ERR_ALIGN (-2)      /* a pointer misses its required alignment       */
#define PQ_ERR_WORKSPACE (-3)  /* workspace missing or too small                */
#define PQ_ERR_LAUNCH (-4)     /* the HIP launch or a HIP runtime call failed   */
#define PQ_ERR_STATE (-5)      /* engine state (context full, not loaded, ...)  */

#define PQ_QBLK 32             /* Q8_0 block: 32 codes, one fp16 scale           */
#define PQ_CHUNK_BLOCKS 8      /* R1 chunk: the fp32 partial covers 8 blocks     */
#define PQ_TILE_ROWS 64        /* rows per tile of the packed weight layout      */

#define PQ_DTYPE_F32 0
#define PQ_DTYPE_BF16 1

/* Library version string and the calling thread's last error message. */
const char *pq_version(void);
const char *pq_last_error(void);

/* Profiling hook: the calling thread's next kernel launch records the two
 * hipEvent_t on its own dispatch (hipExtLaunchKernel), so their elapsed time
 * is that kernel's duration. NULL, NULL disarms. The counterpart of the
 * reference's LFM_KTIME per-statement event brackets (lfm3_nanode.cu:1030-1051). */
int pq_time_next_launch(void *start_event, void *stop_event);

/* --------------------------------------------------------- Q8_0 activations
 * x [T][K] -> qx [T][K] int8, dx [T][K/32] fp32. Per 32-block:
 * d = amax/127, q = rne(x/d) clamped to [-127,127]; an all-zero block gives
 * d = 0, q = 0. New entry point: the reference's decode GEMV reads bf16 x
 * directly (lfm3_nanode.cu:250-276); the Q8_0 x Q8_0 path quantizes first
 * (the rule of .auto/lfm3/q8_gemv_cpu.c:63-81 with an fp32 scale). */
int pq_q8_quant_f32(const float *x, int8_t *qx, float *dx, int K, int T, void *stream);
int pq_q8_quant_bf16(const uint16_t *x, int8_t *qx, float *dx, int K, int T, void *stream);

/* ---------------------------------------------------------- weight packing
 * Row-major Q8_0 weights (codes [N][K] int8, fp16 scales [N][K/32]) -> the
 * packed tile layout every GEMV/GEMM entry point reads:
 *   codes: [N/64 tiles][K/32 blocks][2 halves][64 rows][16 B]
 *   scales:[N/64 tiles][ceil(K/256) chunks][64 rows][8] fp16
 * (rows past N and blocks past K/32 are zero). Replaces the loader's
 * 32-row tile repack (lfm3_nanode.cu:1359-1391, 4510-4568 k_tile_q/k_tile_s,
 * pf_tile). */
size_t pq_q8_packed_codes_bytes(int N, int K);
size_t pq_q8_packed_scales_bytes(int N, int K);
int pq_q8_pack(const int8_t *codes, const uint16_t *scales, int N, int K,
               int8_t *pcodes, uint16_t *pscales, void *stream);

/* ------------------------------------------------------------ Q8_0 GEMV, T=1
 * y[N] = W[N][K] . x, W packed, x as (qx, dx) from pq_q8_quant_*. y_dtype
 * PQ_DTYPE_F32 (LM head logits) or PQ_DTYPE_BF16 (RNE of the fp32 value).
 * Order per output (R1): isum_b exact int32; s_b = fl(f16(W.s_b) * dx_b);
 * per 8-block chunk a = fmaf(s_b, (float)isum_b, a) from 0; y = y + a_c over
 * chunks ascending from 0. y may alias the buffer qx was quantized from.
 * Each workgroup owns whole rows (no cross-workgroup reduction, no scratch).
 * Replaces gemv / gemv_f / tlb_decode (lfm3_nanode.cu:1916-1966, 3634-3663,
 * 4524-4530) and their kernels q8_partial + k_combine_* (222-374). */
int pq_q8_gemv(const int8_t *pcodes, const uint16_t *pscales, const int8_t *qx, const float *dx,
               void *y, int y_dtype, int N, int K, void *stream);

/* ------------------------------------------------------- Q8_0 GEMM, T wide
 * y[T][N] for T positions (qx [T][K], dx [T][K/32], position-first), each
 * output bit-identical to pq_q8_gemv of that position. int8 MFMA
 * (v_mfma_i32_32x32x32_i8) with the R1 epilogue. Replaces pf_gemv_T
 * (lfm3_nanode.cu:4840-4968) and the q8_partial_TL{b,f,g}/Tb/Tp kernels. */
int pq_q8_gemm(const int8_t *pcodes, const uint16_t *pscales, const int8_t *qx, const float *dx,
               void *y, int y_dtype, int N, int K, int T, void *stream);

#ifdef __cplusplus
}
#endif
#endif
