// pq_runtime.cpp -- error state, version and workspace initialisation.
#include <string.h>

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

// Zero fill as a kernel: a hipMemsetAsync node misbehaves on replay when a
// caller captures this stream into a HIP graph.
__global__ void fill_u32_kernel(uint32_t *p, size_t n, uint32_t v) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = v;
}

}  // namespace pq

extern "C" const char *pq_version(void) { return "pulsar-amd 0.1 gfx950"; }

extern "C" const char *pq_last_error(void) { return pq::g_err; }

extern "C" int pq_workspace_init(void *ws, size_t ws_bytes, void *stream) {
  PQ_REQUIRE(ws != nullptr && ws_bytes >= 4, PQ_ERR_WORKSPACE, "pq_workspace_init: null or empty workspace");
  PQ_REQUIRE(pq::aligned(ws, 4), PQ_ERR_ALIGN, "pq_workspace_init: workspace must be 4-byte aligned");
  const size_t n = ws_bytes / 4;
  const unsigned grid = (unsigned)((n + 255) / 256 < 4096 ? (n + 255) / 256 : 4096);
  hipLaunchKernelGGL(pq::fill_u32_kernel, dim3(grid), dim3(256), 0, pq::as_stream(stream),
                     (uint32_t *)ws, n, 0u);
  return pq::check_launch("pq_workspace_init");
}
