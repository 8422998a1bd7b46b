/* ref_shim.c -- exports the reference's own CPU routines for the oracle checks.
 *
 * TEST INFRASTRUCTURE ONLY. oracle/build.py compiles this file against the
 * reference sources where they lie (their paths come in as REF_Q8_CPU and
 * REF_PQ2_HOST); nothing of the reference is copied into this repository.
 * The output goes to oracle/_ref/ and is used only to pin the oracle:
 *   ref_q8_gemv   -> gemv_q8   (.auto/lfm3/q8_gemv_cpu.c:29-58)
 *   ref_q8_quant  -> quant_row (.auto/lfm3/q8_gemv_cpu.c:63-81)
 *   ref_set_threads / ref_max_threads -> the OpenMP team size
 *   pq2_gemv_cpu / pq2_h2f are exported by pulsar_arm/bonsai2/pq2_host.c itself;
 *   bq1_quant_row_i8 by pulsar_arm/bonsai2/bq1_cpu.c itself (bq1_cpu.c:40-54,
 *   the Q8_K rule of fwd8.c:72-137 over one block of K values).
 */
#include <omp.h>

#define main q8_gemv_cpu_reference_main
#include REF_Q8_CPU
#undef main

/* OpenMP team size for the routines below (the CPU baseline times all cores and one). */
void ref_set_threads(int n) { omp_set_num_threads(n); }
int ref_max_threads(void) { return omp_get_max_threads(); }

void ref_q8_gemv(const signed char *q, const float *s, const float *x, float *y, int N, int K) {
  gemv_q8(q, s, x, y, N, K);
}

void ref_q8_quant(const float *w, int K, signed char *q, float *s) { quant_row(w, K, q, s); }

/* The reference's pq2_gemv_cpu (pulsar_arm/bonsai2/pq2_host.c:82-104) is
 * serial; rows are independent, so the CPU baseline runs it on row slices in
 * an OpenMP team (same outputs, row for row). */
#include <stdint.h>
void pq2_gemv_cpu(int rows, int K, const uint8_t *w_codes, const uint16_t *w_scales_h, const uint8_t *xq, float *y);

void ref_pq2_gemv_rows(int rows, int K, const uint8_t *w_codes, const uint16_t *w_scales_h, const uint8_t *xq,
                       float *y) {
  const int nb = omp_get_max_threads() * 4;
#pragma omp parallel for schedule(static)
  for (int b = 0; b < nb; b++) {
    const long r0 = (long)rows * b / nb, r1 = (long)rows * (b + 1) / nb;
    if (r1 > r0)
      pq2_gemv_cpu((int)(r1 - r0), K, w_codes + r0 * (K / 4), w_scales_h + r0 * (K / 128), xq, y + r0);
  }
}
