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
#define PQ_ERR_DATA (-6)       /* stored data failed its check (a blob's crc32)  */

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

/* Self-check of the hardware f32 -> bf16 conversion the kernels use
 * (v_cvt_pk_bf16_f32) against the reference's rounding (round to nearest
 * even, inf/nan passed through; lfm3_nanode.cu:114-121) over all 2^32 float
 * bit patterns. counts, first: device arrays of 65536 uint32; block b reports
 * its mismatches among patterns [b*65536, (b+1)*65536) and the lowest one
 * (0xffffffff if none). Expected: exactly the 2*(2^22 - 1) signaling NaNs
 * differ (the hardware quiets them; the kernels never convert one). No
 * counterpart in the reference. */
int pq_check_bf16_cvt(uint32_t *counts, uint32_t *first, void *stream);
/* Self-check of the quantizers' shared-divisor division against x / d: 2^24
 * random Q8_0 blocks (d = amax/127), 64 values each (ties +-2 ulps, tiny
 * values, +-amax among them); counts/first per 256-block group as above
 * (first = the lowest mismatching thread). No counterpart in the reference. */
int pq_check_quant_div(uint32_t *counts, uint32_t *first, uint32_t seed, void *stream);
/* The shader clock in MHz, measured by one wave over ~0.2 ms (cycle counter
 * against the 100 MHz real-time counter). out: 2 floats of device memory,
 * out[0] = MHz. No counterpart in the reference. */
int pq_clock_mhz(float *out, void *stream);
/* A plain streaming read of `bytes` (a multiple of 16) from p: 1024 x 512
 * threads, one nontemporal 16-byte load per lane per grid-stride step, no
 * arithmetic. Its launch period is the practical ceiling of any kernel that
 * reads that many bytes in one launch; sink (one float of device memory) is
 * never written for real data. No counterpart in the reference. */
int pq_stream_read(const void *p, size_t bytes, float *sink, void *stream);

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
/* The fused gate/up weight [2F][K] (gate rows 0..F-1, up rows F..2F-1, as
 * the MERGE:gate_up tensor, lfm3_nanode.cu:3825-3833) packed with its rows
 * interleaved in groups of 32: packed rows 64t..64t+31 are gate rows
 * 32t..32t+31, rows 64t+32..64t+63 the up rows F+32t... Every GEMV/GEMM over
 * it returns its outputs in that order; pq_silu_mul_interleaved and
 * pq_q8_gemv_fused_swiglu read it. F a multiple of 32. */
int pq_q8_pack_gate_up(const int8_t *codes, const uint16_t *scales, int F, int K,
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
/* The same with a workspace: when N is too small to fill the chip, K is split
 * over workgroups that write each 256-wide chunk's partial to ws [nch][T][N]
 * fp32, then a fold adds them in chunk order -- the same bits. ws_bytes from
 * pq_q8_gemm_workspace_bytes (0: no split for this shape; ws may be NULL). The
 * counterpart of the reference's chunked partials + k_combine_bf_T
 * (lfm3_nanode.cu:4840-4968). */
size_t pq_q8_gemm_workspace_bytes(int N, int K, int T);
int pq_q8_gemm_ws(const int8_t *pcodes, const uint16_t *pscales, const int8_t *qx, const float *dx,
                  void *y, int y_dtype, int N, int K, int T, void *ws, size_t ws_bytes, void *stream);

/* The same GEMM without a workspace argument, for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the split-K partials go to a library-owned device array
 * of pq_q8_gemm_scratch_bytes() (16 MiB) per GPU, held until the process ends.
 * No counterpart in the reference. It calls no allocator. Shapes whose split
 * needs more than the array (pq_q8_gemm_workspace_bytes > the array) are
 * refused with PQ_ERR_WORKSPACE. Every call on one GPU shares that GPU's
 * array: calls that overlap on one GPU (other streams, other threads) race
 * and must be serialized by the caller (one stream per GPU). The stream must
 * belong to the current device. The first call on each device looks up the
 * array's device address (hipGetSymbolAddress) and must be made outside
 * stream capture (under capture it is refused with PQ_ERR_ARG); later calls
 * may be captured into a graph. Same bits as pq_q8_gemm_ws. */
size_t pq_q8_gemm_scratch_bytes(void);
int pq_q8_gemm_noalloc(const int8_t *pcodes, const uint16_t *pscales, const int8_t *qx, const float *dx,
                       void *y, int y_dtype, int N, int K, int T, void *stream);

/* The reference's own GEMV numerics (R2), the order of its CPU transcription
 * (cpuchk_run, lfm3_nanode.cu:4658-4684): codes int8 [N][K] row-major and an
 * fp32 scale per 32-block [N][K/32] (the .lfm3q8 tensors, untiled); x bf16
 * [T][K] position-first; y [T][N] bf16 or fp32. Per output: chunks of 2048 of
 * K (all of K when K is not a multiple of 2048), 32 leaves per chunk (leaf L
 * folds blocks L, L+32, ...: dot = fmaf((float)c_j, x_j, dot) over j
 * ascending, acc = fmaf(s_b, dot, acc)), the shfl_down tree 16..1 over the
 * leaves, chunk partials summed in order from 0. K a multiple of 32, and of
 * 2048 above 8192. Replaces q8_partial<bf16, FMA=1> + k_combine_bf /
 * k_combine_f (lfm3_nanode.cu:222-374) as gemv / gemv_f call them
 * (1916-1966, 3634-3663); T > 1 gives the tiled prefill twin's bits
 * (q8_partial_TLb, 4051-4509) on the shapes that use it. */
int pq_q8r_gemv(const int8_t *codes, const float *scales, const uint16_t *x, void *y, int y_dtype, int N,
                int K, int T, void *stream);

/* ====================================================== Q4 / Q5 low-bit GEMV
 * The reference's low-bit backbone format and order (lfm3_qlow.cuh:1-113,
 * qlow_gemv lfm3_nanode.cu:1894-1915). Per 32-group along K: w = d*q + mn,
 * q in [0, 2^bits) (bits 4 or 5), d' = 128*d and mn fp16. N a multiple of
 * 32, K a multiple of 256 (at most 16384). pq_qlow_pack turns row-major codes
 * (one per byte, [N][K]) and scales ([N][K/32][2] fp16 bits: d', mn) into the
 * reference's tiled payload (the exporter's dtype 6 / 7 tensors: 32-row
 * tiles of nibbles, the bit-4 plane for Q5, half2 scales per row and group). */
size_t pq_qlow_packed_codes_bytes(int N, int K, int bits);
size_t pq_qlow_packed_scales_bytes(int N, int K, int bits);
int pq_qlow_pack(const uint8_t *codes, const uint16_t *scales, int N, int K, int bits, uint8_t *pcodes,
                 uint16_t *pscales, void *stream);
/* y [N] (bf16 or fp32) from x bf16 [K] on the packed payload: K in KS = 4
 * slices for K >= 4096, else 2; per slice and group: acc from four fmaf
 * chains over (1 + q/128) * x (elements b, b+4, ...), (a0 + a1) + (a2 + a3);
 * y_s = fmaf(d', acc - sg, fmaf(mn, sg, y_s)) with sg the group's sum of x;
 * slices added in order from 0. Replaces k_qlow + k_qlow_combine
 * (lfm3_qlow.cuh:39-113) as qlow_gemv launches them. */
int pq_qlow_gemv(const uint8_t *pcodes, const uint16_t *pscales, const uint16_t *x, void *y, int y_dtype, int N,
                 int K, int bits, void *stream);
/* The same with a workspace (ws_bytes >= pq_qlow_workspace_bytes: KS x N
 * fp32, the reference's part): for K >= 4096 on fewer than 256 tiles, or a K
 * whose whole-row staging exceeds LDS, one workgroup per (tile, slice) writes
 * the slice sums there and a second pass adds them in order -- the same bits.
 * Without the workspace such a K is rejected with PQ_ERR_ARG. */
size_t pq_qlow_workspace_bytes(int N, int K, int bits);
int pq_qlow_gemv_ws(const uint8_t *pcodes, const uint16_t *pscales, const uint16_t *x, void *y, int y_dtype,
                    int N, int K, int bits, void *ws, size_t ws_bytes, void *stream);
/* pq_qlow_gemv of T positions in one launch: x [T][K] bf16 (16-byte aligned),
 * y row t at y + t * ldy (ldy >= N, y_dtype fp32 or bf16), each row equal to
 * pq_qlow_gemv of x[t] bit for bit. Replaces the per-position qlow_gemv calls
 * of pf_gemv_T for a low-bit source tensor (lfm3_nanode.cu:4846-4848). */
int pq_qlow_gemm(const uint8_t *pcodes, const uint16_t *pscales, const uint16_t *x, void *y, int y_dtype, int N,
                 int K, int T, int ldy, int bits, void *stream);

/* ============================================================ weight blob
 * The .lfm3q8 file the reference's exporter writes (export_lfm3_q8.py) and
 * load_blob reads (lfm3_nanode.cu:1219-1733): 8-byte magic "LFM3Q8\x01\x00",
 * uint32 header length, a JSON header {cfg, table: [{name, dtype, ne, off,
 * ncodes, nscales, crc}]}, then each tensor's payload (dtype 1: int8 codes
 * then one fp32 scale per 32; 2: fp32; 3: bf16) with the zlib crc32 of its
 * bytes. Host-side only: no GPU is needed to open or read one. */
typedef struct pq_blob_tensor {
  char name[128];
  int dtype;          /* 1 Q8 (codes + fp32 scales), 2 fp32, 3 bf16, 6 / 7 Q4 / Q5 (the
                         exporter's pre-tiled payload, pq_qlow_pack's layout: codes, then
                         (d', mn) fp16 scales; N a multiple of 32, K of 256) */
  int ndim;
  long long ne[4];    /* shape, as the table lists it ([N][K] for a Linear) */
  long long ncodes;   /* payload bytes: codes (or the fp32 / bf16 values) */
  long long nscales;  /* then the fp32 scales (dtype 1) */
  unsigned crc;
} pq_blob_tensor;
void *pq_blob_open(const char *path);    /* NULL on error (pq_last_error) */
int pq_blob_close(void *blob);
int pq_blob_count(void *blob);
int pq_blob_find(void *blob, const char *name);   /* table index, or -1 */
int pq_blob_tensor_info(void *blob, int i, pq_blob_tensor *out);
/* Tensor i's payload into host memory: ncodes bytes to codes, nscales bytes
 * to scales; PQ_ERR_DATA when the crc32 of the bytes read differs from the
 * table's (the reference's load-time check, 1358-1362). */
int pq_blob_read(void *blob, int i, void *codes, void *scales);
/* The header's "cfg" object, re-serialized as JSON (valid until close). */
const char *pq_blob_config(void *blob);
unsigned pq_crc32(unsigned crc, const void *data, size_t n);

/* ======================================================= layer operations
 * bf16 activations are raw uint16 bits. T positions are rows of the given
 * stride (position-first). Each op rounds once to bf16 where the reference's
 * kernel does (lfm3_nanode.cu:383-498, 811-941). */

/* RMSNorm of T rows of H (a power of two, 256..8192), the sum of squares in
 * rmsnorm_body's order (threads of 8 consecutive elements summed pairwise,
 * the shfl_down tree over 32 threads, the partials of each 256 elements in
 * order), rs = 1/sqrtf(ss * (1/H) + eps), y = bf16(w * bf16(x * rs)) (the
 * reference's rsqrtf is the one step taken correctly rounded instead).
 * Residual form (h != NULL): h3 = rmsnorm(h, w0); x = bf16(x + h3) (x is
 * updated in place); out = rmsnorm(x, w1) -- one call for layer_body's
 * "rms1(post_norm) -> eadd -> rms1(next_norm)" triple (3819-3851). The
 * output goes to y (bf16) and/or to (qx, dx) as Q8_0 for the next GEMV.
 * Replaces k_rmsnorm / k_rmsnorm_T / rmsnorm_body (383-456) and k_add_bf(4). */
int pq_rmsnorm(uint16_t *x, const uint16_t *h, const float *w0, const float *w1, uint16_t *y,
               int8_t *qx, float *dx, int H, int T, float eps, void *stream);

/* Per-head q/k RMSNorm, zero-tail partial RoPE from a [pos][rot/2][cos,sin]
 * table, and the fp16 KV-cache write of k and v at positions pos0..pos0+T-1.
 * qkv rows hold [q (nh*hd) | k (nkv*hd) | v (nkv*hd) | ...] with row_stride
 * elements; q is updated in place. head_dim 64 or 128; the table and rot are
 * the layer type's (full attention: partial rotation, theta 1e6; sliding:
 * full rotation, theta 1e4 -- lfm3_nanode.cu:3756-3765). The head norm's sum
 * of squares is k_headnorm's: 32 threads of hd/32 consecutive elements summed
 * pairwise, then the shfl_down tree. Replaces k_headnorm, k_rope and the KV
 * write (460-498, 157-162, 3749-3778). */
int pq_qk_prep(uint16_t *qkv, int row_stride, const float *q_norm, const float *k_norm,
               const float *rope_cs, uint16_t *kcache, uint16_t *vcache, int pos0, int nh, int nkv,
               int hd, int rot, int T, float eps, void *stream);

/* Split-K flash-decode attention over the fp16 cache [ctx][nkv][hd]: query t
 * (row t of q, stride q_stride) at position pos0+t attends keys lo..pos0+t,
 * lo = pos0+t+1-win when win > 0 and the context has outgrown the window
 * (a sliding-window layer, as k_attn_head's win, lfm3_nanode.cu:515), else 0.
 * Splits of 64 positions, merged in ascending order; then the per-head
 * sigmoid gate (gate row t, stride gate_stride; NULL for none). Output to
 * out (bf16, stride out_stride) and/or (qx, dx) as Q8_0 for o_proj. ws holds
 * the split partials (pq_attn_workspace_bytes). head_dim 64 or 128. Replaces
 * k_attn_head(G) and k_sigmoid_gate(4) (503-809, 852-888). */
size_t pq_attn_workspace_bytes(int nh, int hd, int max_pos, int T);
int pq_attn_decode(const uint16_t *q, int q_stride, const uint16_t *kcache, const uint16_t *vcache,
                   const uint16_t *gate, int gate_stride, uint16_t *out, int out_stride, int8_t *qx,
                   float *dx, int pos0, int nh, int nkv, int hd, int T, float scale, int win, void *ws,
                   size_t ws_bytes, void *stream);

/* The reference-numerics arm's attention, in k_attn_head's own order
 * (lfm3_nanode.cu:503-602), then k_sigmoid_gate (852-858): pq_qk_prep_ref is
 * pq_qk_prep with the cache holding the bf16 k and v rows as k_kv_write copies
 * them (157-162); pq_attn_ref attends query t (row t of q) at position pos0+t
 * to keys lo..pos0+t of that bf16 cache (lo as in pq_attn_decode) with one
 * 1024-thread workgroup per (head, t): each score a chain over the lane's
 * hd/32 dims and the shfl_down tree of a 32-lane warp (32 warps share the
 * keys); then its first 256 threads keep the reference's places: the softmax
 * sum per thread over keys t, t+256, ..., the warp tree, the 8 warps' tree;
 * the probabilities normalized before an 8-segment value sum added pairwise. e^x is the build's expf_pq where the reference
 * calls CUDA's expf. head_dim 64 or 128; at most 32768 keys in a window;
 * gate NULL for none; out bf16 [T] rows of stride out_stride. */
int pq_qk_prep_ref(uint16_t *qkv, int row_stride, const float *q_norm, const float *k_norm,
                   const float *rope_cs, uint16_t *kcache, uint16_t *vcache, int pos0, int nh, int nkv,
                   int hd, int rot, int T, float eps, void *stream);
int pq_attn_ref(const uint16_t *q, int q_stride, const uint16_t *kcache, const uint16_t *vcache,
                const uint16_t *gate, int gate_stride, uint16_t *out, int out_stride, int pos0, int nh,
                int nkv, int hd, int T, float scale, int win, void *stream);

/* One decode token's pq_qk_prep_ref + pq_attn_ref in a single launch, with
 * the same results (outputs and cache rows bit for bit): qkv is the token's
 * projected row [q (nh hd) | k (nkv hd) | v (nkv hd)] (left unchanged; the
 * rotated q stays on chip), the token at position pos; the k and v rows of pos
 * go to the cache and into each workgroup's LDS, and its key and value are
 * taken from there, so no workgroup waits on another's cache write. gate NULL
 * for none (one bf16 per head); out bf16 [nh hd]. Replaces k_headnorm,
 * k_rope, k_kv_write, k_attn_head and k_sigmoid_gate of one decode step
 * (lfm3_nanode.cu:460-498, 157-162, 503-602, 852-858). */
int pq_attn_decode_ref(const uint16_t *qkv, const float *q_norm, const float *k_norm,
                       const float *rope_cs, uint16_t *kcache, uint16_t *vcache, const uint16_t *gate,
                       uint16_t *out, int pos, int nh, int nkv, int hd, int rot, float eps, float scale,
                       int win, void *stream);

/* pq_attn_decode_ref for a layer whose gate rows are a Q8 tensor of their own
 * (a low-bit blob keeps gate_proj in Q8): the launch forms each head's gate
 * itself, with the bits of the reference-numerics GEMV of those rows on
 * rmsnorm(x, x_norm) (pq_q8r_gemv_fused with the NORM prologue: rmsnorm_body's
 * order, then the 32 leaf chains of q8_partial<bf16, FMA=1> and k_combine's
 * bf16), so that GEMV's launch is not needed. gate_codes [nh][2048] int8 and
 * gate_scales [nh][64] fp32 row-major as the .lfm3q8 file stores them; x the
 * bf16 residual [2048] (hidden 2048), x_norm its norm weight; eps serves both
 * norms. Replaces, for one decode step, the gate rows' gemv (lfm3_nanode.cu
 * 222-374, 383-440) with the kernels pq_attn_decode_ref replaces. */
int pq_attn_decode_ref_q8gate(const uint16_t *qkv, const float *q_norm, const float *k_norm,
                              const float *rope_cs, uint16_t *kcache, uint16_t *vcache,
                              const int8_t *gate_codes, const float *gate_scales, const uint16_t *x,
                              const float *x_norm, uint16_t *out, int pos, int nh, int nkv, int hd, int rot,
                              float eps, float scale, int win, void *stream);

/* Gated short conv over T positions: bcx rows [B | C | x] (3H), ring
 * [ntaps][H] bf16 (newest last, updated), out [T][H] bf16 = bf16(C * conv(B*x)).
 * ntaps 2, 3, 4 or 7. Replaces k_shift_in + k_conv7 / k_conv_chunk (892-941). */
int pq_conv(uint16_t *ring, const float *taps, const uint16_t *bcx, uint16_t *out, int H, int T,
            int ntaps, void *stream);

/* silu(gate) * up over rows [gate (F) | up (F)]; output bf16 and/or Q8_0.
 * Replaces k_silu_mul_bf(v) (821-847). */
int pq_silu_mul(const uint16_t *gu, uint16_t *y, int8_t *qx, float *dx, int F, int T, void *stream);
/* The same over rows in the pq_q8_pack_gate_up order (gate element i at
 * 64*(i/32) + i%32, up element i 32 further). */
int pq_silu_mul_interleaved(const uint16_t *gu, uint16_t *y, int8_t *qx, float *dx, int F, int T,
                            void *stream);

/* Greedy id: k_argmax's pick among v[n] (942-964): the largest value above
 * -1e30, ties in its order -- the smallest (bitrev3(i/32 mod 8), bitrev5(i mod
 * 32)), then the smallest i -- and -1 when no value exceeds -1e30. Replaces
 * k_argmax. */
int pq_argmax(const float *v, int n, int32_t *out, void *stream);

/* Embedding rows of T token ids (device) from the packed tied Q8_0 table:
 * bf16(code * scale); ids outside [0, vocab) give zero rows. Replaces
 * k_dequant_row (138-142). */
int pq_embed(const int8_t *pcodes, const uint16_t *pscales, const int32_t *tokens, uint16_t *out,
             int H, int vocab, int T, void *stream);
/* The same from the table as an .lfm3q8 file stores it: row-major codes
 * [vocab][H] and one fp32 scale per 32 ([vocab][H/32]). Replaces k_dequant_row
 * (138-142) on the blob's tensor, as the reference runs it. */
int pq_embed_rows(const int8_t *codes, const float *scales, const int32_t *tokens, uint16_t *out, int H,
                  int vocab, int T, void *stream);

/* The tied table kept as bf16 [vocab][H] (the exporter's --emb-bf16, dtype 3).
 * pq_embed_bf16: rows of T token ids (device) copied as stored, zero rows for
 * ids outside [0, vocab) -- the reference's bf16 row copy (lfm3_nanode.cu:
 * 6062-6076). pq_bf16_gemv: y [N] fp32 = W . x for x bf16 [K] (K a multiple
 * of 32, at most 16384), in k_gemv_bf16's order (3517-3534, as lm_head_bf16
 * launches it, 3536-3573): per row, leaf L = 0..31 sums the products of
 * elements L, L+32, ... in order, each rounded before its add, then the
 * shfl_down tree 16, 8, 4, 2, 1 over the leaves. argmax_parts (NULL or
 * 2 * pq_bf16_gemv_parts(N) floats) receives each workgroup's (y, row) pick
 * in pq_argmax's order for pq_argmax_parts. */
int pq_embed_bf16(const uint16_t *table, const int32_t *tokens, uint16_t *out, int H, int vocab, int T,
                  void *stream);
int pq_bf16_gemv_parts(int N);
int pq_bf16_gemv(const uint16_t *W, const uint16_t *x, float *y, int N, int K, float *argmax_parts,
                 void *stream);


/* ================================================== fused decode kernels
 * The T=1 decode step with the small ops folded into the GEMV that consumes
 * their output (each workgroup recomputes the vector in its prologue, after
 * issuing its first weight loads). Same arithmetic and order as the unfused
 * calls, so the results are bit-identical. Prologue kinds:
 *   PQ_PRO_Q8       x given as (qx, dx)
 *   PQ_PRO_RESNORM  h3 = rmsnorm(h, w0); x_out = bf16(x_in + h3) (written once);
 *                   x = rmsnorm(x_out, w1)            -- rms1 -> eadd -> rms1
 *   PQ_PRO_NORM     x = rmsnorm(x_in, w0)
 *   PQ_PRO_EMBED    x_out = embedding row of *tok (packed table, written once);
 *                   x = rmsnorm(x_out, w0)
 *   PQ_PRO_SILU     x = silu(gu[0:K]) * gu[K:2K]
 *   PQ_PRO_CONV     gated short conv of bcx [B|C|x] with ring_in -> ring_out
 *                   (the shifted ring, written once; a ping-pong pair);
 *                   ntaps 3 or 7, taps f32 [K][ntaps] 16-byte aligned
 *   PQ_PRO_F32      x = xf, fp32 [K] (16-byte aligned), quantized in-kernel
 *                   exactly as pq_q8_quant_f32
 * K is the GEMV's K (a power of two, 1024..8192). argmax_parts (optional,
 * 2 floats per workgroup, pq_q8_gemv_parts(N, K) of them) receives each
 * workgroup's (value, index) pick in pq_argmax's order for pq_argmax_parts --
 * the LM head + k_argmax. The norms' sums of squares are pq_rmsnorm's. */
#define PQ_PRO_Q8 0
#define PQ_PRO_RESNORM 1
#define PQ_PRO_NORM 2
#define PQ_PRO_EMBED 3
#define PQ_PRO_SILU 4
#define PQ_PRO_CONV 5
#define PQ_PRO_F32 6
typedef struct pq_gemv_prologue {
  int kind;
  const int8_t *qx;
  const float *dx;
  const uint16_t *h, *x_in;
  uint16_t *x_out;
  const float *w0, *w1;
  float eps;
  const uint16_t *gu;
  const uint16_t *bcx, *ring_in;
  uint16_t *ring_out;
  const float *taps;
  int ntaps;
  const int8_t *emb_pc;
  const uint16_t *emb_ps;
  const int32_t *tok;
  int vocab;
  const float *xf;
  const float *emb_sf;   /* PQ_PRO_EMBED under pq_q8r_gemv_fused: the row-major table's fp32 scales */
} pq_gemv_prologue;
int pq_q8_gemv_parts(int N, int K);
int pq_q8_gemv_fused(const int8_t *pcodes, const uint16_t *pscales, const pq_gemv_prologue *pro,
                     void *y, int y_dtype, int N, int K, float *argmax_parts, void *stream);
int pq_argmax_parts(const float *parts, int nparts, int32_t *out, void *stream);
/* pq_q8r_gemv at T = 1 (the reference's own GEMV order on row-major codes and
 * fp32 scales) with x from a prologue: RESNORM, NORM, SILU or CONV (K <= 4096
 * for CONV), computed exactly as the kinds above and handed to the GEMV as the
 * bf16 values the unfused op would store. K is 1024, 2048, 4096 or 8192; y
 * bf16 or fp32; argmax_parts as for pq_q8_gemv_fused. Replaces the rmsnorm_body / k_silu_mul_bf / k_conv7 + gemv
 * pairs of layer_body (lfm3_nanode.cu:3739-3856) under the reference numerics. */
/* (PQ_PRO_EMBED here reads the row-major .lfm3q8 table, emb_pc codes
 * [vocab][K] and emb_sf fp32 scales [vocab][K/32]: x_out = bf16(code * scale)
 * of row *tok, zeros for an id outside [0, vocab), as pq_embed_rows;
 * k_dequant_row, lfm3_nanode.cu:138-142.) */
int pq_q8r_gemv_fused(const int8_t *codes, const float *scales, const pq_gemv_prologue *pro, void *y,
                      int y_dtype, int N, int K, float *argmax_parts, void *stream);
/* Workgroups of pq_q8r_gemv_fused for N rows: the (value, index) pairs it
 * writes to argmax_parts (if not NULL) for pq_argmax_parts. */
int pq_q8r_gemv_parts(int N);
/* The FFN's gate/up GEMV under the reference numerics: codes [2F][K] (gate
 * rows 0..F-1, up rows F..2F-1, row-major), fp32 scales, x from a RESNORM or
 * NORM prologue, and y [F] bf16 = silu_mul of the bf16 gate and up outputs --
 * the gemv + k_silu_mul_bf pair (lfm3_nanode.cu:821-829) of layer_body
 * (3739-3856) in one launch, the same bits. F a multiple of 4. */
int pq_q8r_gemv_fused_swiglu(const int8_t *codes, const float *scales, const pq_gemv_prologue *pro,
                             uint16_t *y, int F, int K, void *stream);
/* The Q4 / Q5 GEMV (pq_qlow_gemv's payload and order) at T = 1 with x from a
 * prologue: RESNORM, NORM, SILU or CONV (3 or 7 taps, K <= 4096), computed
 * as the kinds above and handed to the GEMV as the bf16 values the unfused op
 * would store. K is 2048, 4096 or 8192 (whole rows per workgroup, no K split);
 * y bf16 or fp32. Replaces the rmsnorm_body / k_silu_mul_bf / k_conv7 +
 * qlow_gemv pairs of layer_body (lfm3_nanode.cu:3739-3856, qlow_gemv
 * 1894-1915) for a low-bit source tensor. */
int pq_qlow_gemv_fused(const uint8_t *pcodes, const uint16_t *pscales, const pq_gemv_prologue *pro, void *y,
                       int y_dtype, int N, int K, int bits, void *stream);
/* The FFN's gate/up GEMV on a low-bit [w1 | w3] payload (pq_qlow_pack of the
 * 2F rows, gate rows first) with a RESNORM or NORM prologue and y [F] bf16 =
 * silu_mul of the bf16 gate and up outputs: the qlow_gemv (1894-1915) +
 * k_silu_mul_bf (821-829) pair of layer_body (lfm3_nanode.cu:3830-3833) in
 * one launch, the same bits as pq_qlow_gemv_fused (N = 2F, bf16) followed by
 * pq_silu_mul. F a multiple of 32; K 2048, 4096 or 8192. */
int pq_qlow_gemv_fused_swiglu(const uint8_t *pcodes, const uint16_t *pscales, const pq_gemv_prologue *pro,
                              uint16_t *y, int F, int K, int bits, void *stream);
/* The FFN's gate/up GEMV (weights from pq_q8_pack_gate_up, N = 2F) with the
 * prologue pro and silu(gate) * up as its epilogue: writes the Q8_0 row
 * (qx [F], dx [F/32]) that the down projection reads (PQ_PRO_Q8) -- the
 * gemv(gate_up), k_silu_mul_bf sequence of layer_body (3830-3833).
 * Same bits as the GEMV, pq_silu_mul_interleaved and its Q8_0 output. */
int pq_q8_gemv_fused_swiglu(const int8_t *pcodes, const uint16_t *pscales, const pq_gemv_prologue *pro,
                            int8_t *qx, float *dx, int F, int K, void *stream);
/* The attention mixer of one decode step (T=1, position pos) in one launch:
 * q/k norm + RoPE, fp16 KV write at pos, every 64-position split of the
 * window (win as in pq_attn_decode; 0 = full attention), the ordered merge,
 * the sigmoid gate, and the Q8_0 row (qx, dx) of o_proj's input and/or out
 * (bf16) with the gated attention output. qkvg is the fused [q | k | v | gate]
 * GEMV row; head_dim 64 or 128. Same numerics as pq_qk_prep + pq_attn_decode.
 * Replaces k_headnorm, k_rope, the KV write, k_attn_head and k_sigmoid_gate of
 * layer_body (lfm3_nanode.cu:3749-3786). */
int pq_attn_layer_decode(const uint16_t *qkvg, const float *q_norm, const float *k_norm,
                         const float *rope_cs, uint16_t *kcache, uint16_t *vcache, int pos, int nh,
                         int nkv, int hd, int rot, int win, float eps, float scale, uint16_t *out,
                         int8_t *qx, float *dx, void *stream);

/* ======================================================= ternary GEMV
 * PQ2_0 x Q8_K, the Bonsai ternary path. codes u8 [N][K/4] (weight i of a
 * byte = bits 2i..2i+1, value = code - 1), fp16 scale per 128 weights
 * [N][K/128] -- the split layout of pq2_split_repack (pq2_host.c:40-57);
 * xq = Q8_K activations (292 B per 256: fp32 d, 256 int8, 16 int16 bsums).
 * y[N] fp32, per row groups ascending: acc = fl(acc + fl(fl(ws*db) * isum))
 * with isum the exact int32 group dot (pq2_host.c:82-104). K a multiple of
 * 256, at most 32768. Replaces pq2_gemv_sm53_launch (pq2_wrap.h:24-28) with
 * its arguments in its order -- (..., y, K, N, stream) -- and its convention
 * of a negative status on error. */
int pq_tq2_gemv(const uint8_t *codes, const uint16_t *scales, const uint8_t *xq, float *y, int K,
                int N, void *stream);
/* n = 1..3 ternary tensors of the same K over the same xq in one launch
 * (codes[i], scales[i], ys[i]: device pointers in host arrays; rows[i] rows
 * each), every output the bits pq_tq2_gemv gives it: the gate and up
 * projections of an FFN, or q, k and v. Replaces the batched launch the
 * reference's engine makes for projections that read one activation
 * (pq2_gemv_batch, pq2_fwd8_shim.h:16, called from gemvP_multi, fwd8.c:303-310
 * and 857-861; the device form is pq1_gemv_batch_launch,
 * pq1_swar_sm53.cu:1480-1680). */
int pq_tq2_gemv_batch(const uint8_t *const *codes, const uint16_t *const *scales, const uint8_t *xq,
                      float *const *ys, int K, const int *rows, int n, void *stream);
/* x [T][K] fp32 -> Q8_K blocks (quantize_row_q8_K_ref as restated in
 * fwd8.c:61-137); K a multiple of 256. */
int pq_q8k_quant(const float *x, uint8_t *out, int K, int T, void *stream);

/* ==================================================== synthetic generator
 * Host-side fill of a synthetic tensor (there is no checkpoint offline):
 * splitmix64 output n = mix(seed + (n+1)*0x9e3779b97f4a7c15), used as
 *   CODES   int8 in [-127,127]   SCALES fp16 bits of |N(0,1)| * a
 *   NORMAL  float N(0,1)         AFFINE float a + b * N(0,1)
 *   TERNARY PQ2_0 code bytes, codes in {0,1,2}   TOKENS int32 in [0, a) */
#define PQ_SYNTH_CODES 0
#define PQ_SYNTH_NORMAL 1
#define PQ_SYNTH_SCALES 2
#define PQ_SYNTH_AFFINE 3
#define PQ_SYNTH_TERNARY 4
#define PQ_SYNTH_TOKENS 5
int pq_synth_fill(int kind, uint64_t seed, void *out_host, size_t n, float a, float b);

/* ================================================================ engine
 * The backbone on one GPU: weights resident in HBM (packed Q8_0), fp16 KV
 * cache, conv rings, a prefill path that runs the prompt layer by layer in
 * chunks of up to prefill_chunk positions (the batched MFMA GEMM; the
 * reference's layer-major order, lfm3_nanode.cu:5935-5955) and a T=1 decode
 * path (the GEMV), all on the engine's own stream. Layer kinds come from attn_mask (bit L set = attention layer).
 * Host pointers: tokens, ids, logits, tensors passed to pq_engine_set_*.
 * The call sequence restates lfm3_nanode.cu main()/layer_body (3739-3856,
 * 5828-6340) with the reference's host contract: arenas allocated once at
 * create, errors returned instead of exit(2). */
typedef struct pq_model_cfg {
  int hidden, ffn, vocab, nlayers;
  int nh, nkv, hd, rot;      /* rot = rotated dims (partial rotary factor * hd) */
  int ntaps, ctx;            /* conv kernel size; KV capacity                   */
  float eps, theta;
  uint64_t seed;             /* synthetic weights                              */
  uint32_t attn_mask;
  int prefill_chunk;         /* positions per prefill launch (32)               */
  int numerics;              /* PQ_NUMERICS_Q8 or PQ_NUMERICS_REF               */
  uint32_t slide_mask;       /* bit L set = sliding-window attention layer     */
  int slide_win;             /* keys a sliding layer sees (the last slide_win)  */
  int slide_rot;             /* rotated dims of a sliding layer                 */
  float slide_theta;         /* RoPE base of a sliding layer                    */
} pq_model_cfg;
/* numerics: PQ_NUMERICS_Q8 runs the Q8_0 x Q8_0 GEMVs (activations quantized
 * per 32-block, fp16 weight scales, the packed tile layout, int8 MFMA for
 * prefill, the fused decode kernels); PQ_NUMERICS_REF keeps the .lfm3q8
 * tensors as stored (row-major codes, fp32 scales) and runs every GEMV through
 * pq_q8r_gemv on bf16 activations -- the reference's own GEMV order
 * (gemv / gemv_f, lfm3_nanode.cu:1916-1966, 3634-3663) -- with unfused T=1
 * steps. */
#define PQ_NUMERICS_Q8 0
#define PQ_NUMERICS_REF 1

void *pq_engine_create(const pq_model_cfg *cfg);             /* NULL on failure */
int pq_engine_destroy(void *engine);
int pq_engine_load_synthetic(void *engine);
/* Load one tensor from host memory (the blob loader's boundary, lfm3_nanode.cu:
 * 1294-1402): Q8 slots 0 mixer in, 1 mixer out, 2 gate/up, 3 down (layer -1
 * slot 0 = tied embedding); fp32 slots 4..7 norms, 8/9 q/k norm, 10 conv taps
 * (layer -1 slot 1 = final norm). Call pq_engine_mark_loaded when done. */
int pq_engine_set_q8(void *engine, int layer, int slot, const int8_t *codes, const uint16_t *scales);
/* The same with fp32 scales (the .lfm3q8 form). Under PQ_NUMERICS_Q8 every
 * scale must be an fp16 value: otherwise PQ_ERR_DATA, with the count of those
 * that are not (and of those below fp16's normal range) in pq_last_error. */
int pq_engine_set_q8_f32(void *engine, int layer, int slot, const int8_t *codes, const float *scales);
int pq_engine_set_f32(void *engine, int layer, int slot, const float *v, size_t n);
int pq_engine_mark_loaded(void *engine);
/* Every backbone tensor from an .lfm3q8 blob (the reference's load_blob,
 * lfm3_nanode.cu:1404-1733, on the names layer_body reads, 3739-3856): each
 * payload's crc32 is checked (PQ_ERR_DATA on a mismatch) on a reader thread
 * that stays ahead of the uploads; q/k/v/gate_proj stack into the attention
 * input GEMV, feed_forward.w1 / w3 into gate/up. The fp32 weight scales are
 * kept under PQ_NUMERICS_REF; under PQ_NUMERICS_Q8 they must be fp16 values
 * (a blob written from fp16 scales), else PQ_ERR_DATA naming the tensor and
 * counting the scales fp16 cannot hold -- nothing is rounded silently. The
 * tied embedding must be Q8 (dtype 1). Shapes must match the engine's
 * configuration; sliding-window attention layers are refused.
 * Marks the engine loaded on success. */
int pq_engine_load_blob(void *engine, const char *path);
int pq_engine_reset(void *engine);
/* Feed n tokens (prefill chunks); the greedy id after the last one and its
 * fp32 logits (either may be NULL) come back to the host. */
int pq_engine_feed(void *engine, const int32_t *tokens, int n, int32_t *next_id, float *logits);
/* reset, prompt, then n_steps greedy ids (ids[0] from the prompt's last position). */
int pq_engine_greedy(void *engine, const int32_t *prompt, int n_prompt, int n_steps, int32_t *ids);
/* n_steps T=1 decode steps from the current device-side token; ids may be NULL. */
int pq_engine_decode(void *engine, int n_steps, int32_t *ids);
/* Route T=1 steps through the fused decode kernels (1) or the unfused per-op
 * calls (0); both give the same bits. The default is 1 where the fused kernels
 * take the configuration (hidden and ffn powers of two in 1024..8192, 3 conv
 * taps, GQA group 1/2/4, the context's splits in LDS); set_fused(1) on another
 * configuration returns PQ_ERR_ARG. */
int pq_engine_set_fused(void *engine, int on);
/* Positions per prefill chunk from now on: 1 .. the configuration's
 * prefill_chunk (the arenas' size). Any chunk size gives the same bits; the
 * prompt runs layer by layer over its chunks, so larger chunks read each
 * layer's weights fewer times. */
int pq_engine_set_chunk(void *engine, int n);
/* Fused decode steps replay a captured HIP graph (1, the default; the position
 * and the id slot live on the device) or launch kernel by kernel (0); both give
 * the same bits. */
int pq_engine_set_graph(void *engine, int on);
int pq_engine_sync(void *engine);
void *pq_engine_stream(void *engine);
int pq_engine_position(void *engine);
int pq_engine_hidden(void *engine, uint16_t *out_host);
size_t pq_engine_weight_bytes(void *engine);

#ifdef __cplusplus
}
#endif
#endif
