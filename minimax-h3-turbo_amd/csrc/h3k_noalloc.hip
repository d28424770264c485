// h3k_w4a8_linear without a workspace, for callers that cannot allocate device memory: the scratch is a static
// device array (one copy per GPU), found once per device with hipGetSymbolAddress.
#include <mutex>

#include "h3k_common.hpp"

namespace h3k {
size_t w4a8_linear_base_workspace(int64_t m, int64_t n, int64_t k);
}
using namespace h3k;

// The scratch of h3k_w4a8_linear_noalloc: a file-scope device array, one copy per GPU the library runs on, held
// until the process ends.  In host code `scratch` names a host-side stand-in, not device memory: the device address
// of each GPU's copy comes from hipGetSymbolAddress, once per device with that device current, and only that
// address is ever passed to kernels.
static constexpr size_t kNoAllocScratchBytes = size_t(128) << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[64] = {};
}  // namespace

static int noalloc_scratch(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= 64) return fail(H3K_ELAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr)
      return fail(H3K_ELAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return H3K_OK;
}

extern "C" int h3k_w4a8_linear_noalloc(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const void* q,
                                       int64_t ldq, const void* s_rel, int s_dtype, int64_t lds, const float* s_ch,
                                       const float* codebook, int64_t n, int group, int rot, const void* bias, int mode,
                                       void* out, int out_dtype, int64_t ldo, void* stream) {
  // the required part of the workspace; the packed GEMM's split tail is used when the scratch holds it as well
  const size_t need = w4a8_linear_base_workspace(m, n, k);
  if (need > kNoAllocScratchBytes)
    return fail(H3K_ESPACE, "h3k_w4a8_linear_noalloc: m=%lld n=%lld k=%lld needs %zu bytes of scratch, the static "
                "scratch holds %zu: split the rows or use h3k_w4a8_linear with a workspace",
                (long long)m, (long long)n, (long long)k, need, kNoAllocScratchBytes);
  if (m == 0 || n == 0) return H3K_OK;
  void* ws = nullptr;
  const int rc = noalloc_scratch(&ws);
  if (rc) return rc;
  return h3k_w4a8_linear(x, x_dtype, m, k, ldx, q, ldq, s_rel, s_dtype, lds, s_ch, codebook, n, group, rot, bias, mode,
                         out, out_dtype, ldo, ws, kNoAllocScratchBytes, stream);
}

