// C ABI glue: error reporting, the fused W4A8 linear entry point and the streaming copy.
#include "h3k_common.hpp"

namespace h3k {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

int fail(int code, const char* fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(H3K_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  return H3K_OK;
}

int gemm_a8w8_launch(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8, int64_t ldw, const float* s_ch,
                     const void* bias, int64_t m, int64_t n, int64_t k, int mode, void* out, int out_dtype, int64_t ldo,
                     int32_t* acc_out, hipStream_t st);

static inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

int64_t w8p_bytes(int64_t n, int64_t k);
bool w8p_serves(int64_t m, int64_t n, int64_t k);
int64_t w8p_split_bytes(int64_t m, int64_t n, int64_t k);
size_t w4a8_linear_base_workspace(int64_t m, int64_t n, int64_t k);
void gemm_w8p_launch(const int8_t* a, int64_t lda, const float* xs, const int8_t* w8p, const float* s_ch,
                     const void* bias, int m, int n, int k, int mode, void* out, int odt, int64_t ldo, int32_t* acc_out,
                     int32_t* part, hipStream_t st);

}  // namespace h3k

using namespace h3k;

extern "C" int h3k_version(void) { return 7; }

extern "C" const char* h3k_last_error(void) { return g_last_error.c_str(); }

// Calls of at most this many rows may take the fused int4 GEMM (fused_few_rows below).
static constexpr int64_t kFewRows = 32;

// The weight region holds the decoded int8 grid (row-major, or packed: n rounded up to 256 rows), or for the fused
// few-row GEMM its split-K accumulators (only calls that can take that GEMM reserve them).
static size_t weight_region(int64_t m, int64_t n, int64_t k) {
  const size_t grid = static_cast<size_t>((n + 255) / 256 * 256) * k;
  const size_t acc = m <= kFewRows ? static_cast<size_t>(h3k_gemm_w4a8_workspace(m, n, k)) : 0;
  return grid > acc ? grid : acc;
}

// The packed grid and its GEMM: shapes with enough 256 x 256 tiles, the rotate+quant output (lda = k) addressable
// by one buffer descriptor, and a packed weight the packed decode can read.
static bool packed_route(int64_t m, int64_t n, int64_t k, const void* q, int64_t ldq, int group) {
  return w8p_serves(m, n, k) && (m - 1) * k + k < (int64_t(1) << 32) && aligned(q, 16) && ldq % 16 == 0 &&
         group >= 4 && k % group == 0 && ((16 % group) == 0 || (group % 16) == 0);
}

// Chunks of up to 32 rows take the fused int4 GEMM; from 64 rows the decode + int8 GEMM pair is faster (N=13824,
// K=5120: 35 against 42 us at 64 rows), at 16 the fused GEMM (15 against 34 us).
static bool fused_few_rows(int64_t m, int64_t k, int group, const void* q, int64_t ldq) {
  return m <= kFewRows && k % 64 == 0 && (group == 16 || group == 32 || (group > 0 && group % 64 == 0)) && k % group == 0 &&
         aligned(q, 16) && ldq % 16 == 0;
}

// Activations, their scales and the weight region: what every call needs.
size_t h3k::w4a8_linear_base_workspace(int64_t m, int64_t n, int64_t k) {
  if (m < 0 || n < 0 || k < 0) return 0;
  return round_up(static_cast<size_t>(m) * k, 256) + round_up(static_cast<size_t>(m) * 4, 256) +
         round_up(weight_region(m, n, k), 256);
}

// The packed GEMM's split-tail partial sums, for the shapes whose route takes it (the caller checks the rest).
static size_t split_region(int64_t m, int64_t n, int64_t k) {
  return m > kFewRows && w8p_serves(m, n, k) ? round_up(static_cast<size_t>(w8p_split_bytes(m, n, k)), 256) : 0;
}

extern "C" size_t h3k_w4a8_linear_workspace(int64_t m, int64_t n, int64_t k) {
  if (m < 0 || n < 0 || k < 0) return 0;
  return w4a8_linear_base_workspace(m, n, k) + split_region(m, n, k);
}

extern "C" int h3k_w4a8_linear(const void* x, int x_dtype, int64_t m, int64_t k, int64_t ldx, const void* q,
                               int64_t ldq, const void* s_rel, int s_dtype, int64_t lds, const float* s_ch,
                               const float* codebook, int64_t n, int group, int rot, const void* bias, int mode,
                               void* out, int out_dtype, int64_t ldo, void* workspace, size_t workspace_bytes,
                               void* stream) {
  const size_t need = w4a8_linear_base_workspace(m, n, k);
  if (workspace_bytes < need)
    return fail(H3K_ESPACE, "workspace of %zu bytes, %zu needed", workspace_bytes, need);
  if (m == 0 || n == 0) return H3K_OK;
  if (!workspace || !aligned(workspace, 256)) return fail(H3K_EINVAL, "workspace must be 256-byte aligned");
  char* ws = static_cast<char*>(workspace);
  int8_t* aq = reinterpret_cast<int8_t*>(ws);
  float* xs = reinterpret_cast<float*>(ws + round_up(static_cast<size_t>(m) * k, 256));
  int8_t* w8 = reinterpret_cast<int8_t*>(ws + round_up(static_cast<size_t>(m) * k, 256) + round_up(static_cast<size_t>(m) * 4, 256));
  int rc = h3k_rotate_quant(x, x_dtype, m, k, ldx, rot, mode, aq, k, xs, stream);
  if (rc) return rc;
  if (fused_few_rows(m, k, group, q, ldq))  // int4 decoded in registers: no int8 grid
    return h3k_gemm_w4a8(aq, k, xs, q, ldq, s_rel, s_dtype, lds, codebook, group, s_ch, bias, m, n, k, mode, out,
                         out_dtype, ldo, reinterpret_cast<int32_t*>(w8), nullptr, stream);
  if (packed_route(m, n, k, q, ldq, group) && aligned(s_ch, 16) && (bias == nullptr || aligned(bias, 16)) &&
      ldo >= n && (mode == H3K_MODE_CK || mode == H3K_MODE_EAGER) &&
      (out_dtype == H3K_BF16 || out_dtype == H3K_F16 || out_dtype == H3K_F32) && out) {
    rc = h3k_decode_w4_packed(q, ldq, s_rel, s_dtype, lds, codebook, n, k, group, w8, stream);
    if (rc) return rc;
    const size_t split = split_region(m, n, k);  // taken when the workspace holds it
    int32_t* part = split > 0 && workspace_bytes >= need + split ? reinterpret_cast<int32_t*>(ws + need) : nullptr;
    gemm_w8p_launch(aq, k, xs, w8, s_ch, bias, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k), mode, out,
                    out_dtype, ldo, nullptr, part, static_cast<hipStream_t>(stream));
    return check_launch("gemm_a8w8_packed");
  }
  rc = h3k_decode_w4(q, ldq, s_rel, s_dtype, lds, codebook, n, k, group, w8, k, stream);
  if (rc) return rc;
  return gemm_a8w8_launch(aq, k, xs, w8, k, s_ch, bias, m, n, k, mode, out, out_dtype, ldo, nullptr,
                          static_cast<hipStream_t>(stream));
}

extern "C" int h3k_copy_h2d_async(void* dst, const void* src, size_t nbytes, void* stream) {
  if (nbytes == 0) return H3K_OK;
  if (!dst || !src) return fail(H3K_EINVAL, "NULL pointer");
  const hipError_t e = hipMemcpyAsync(dst, src, nbytes, hipMemcpyHostToDevice, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return fail(H3K_ELAUNCH, "hipMemcpyAsync: %s", hipGetErrorString(e));
  return H3K_OK;
}
