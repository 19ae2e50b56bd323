// C ABI of libpare_amd.so: host-side argument validation, error reporting and
// kernel dispatch. Declarations and reference citations: include/pare_amd.h.
#include "../../include/pare_amd.h"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "pmi_launch.h"

namespace {

thread_local char g_err[512] = "";
std::atomic<int> g_kernel_override{0};

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int ok() {
  g_err[0] = '\0';
  return PMI_OK;
}

int from_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return ok();
  return fail(PMI_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

// Shared shape rules of the packed INT4 format and the kernels' tiling.
int check_shape(int64_t N, int64_t K, int64_t gs, const char* fn) {
  if (N < 0 || K <= 0 || gs <= 0)
    return fail(PMI_ERR_INVALID, "%s: need N >= 0, K > 0, group_size > 0 (N=%lld K=%lld gs=%lld)",
                fn, (long long)N, (long long)K, (long long)gs);
  if (K % gs != 0)
    return fail(PMI_ERR_INVALID, "%s: K=%lld must be divisible by group_size=%lld", fn,
                (long long)K, (long long)gs);
  if (gs % 32 != 0)
    return fail(PMI_ERR_UNSUPPORTED, "%s: group_size=%lld must be a multiple of 32", fn,
                (long long)gs);
  if (K > (1ll << 30) || N > (1ll << 31) - 1 || N * (K / 2) >= (1ll << 31))
    return fail(PMI_ERR_UNSUPPORTED, "%s: shape too large (N=%lld K=%lld)", fn, (long long)N,
                (long long)K);
  return PMI_OK;
}

int check_zero_dtype(int zero_dtype, const char* fn) {
  if (zero_dtype != PMI_F32 && zero_dtype != PMI_U8)
    return fail(PMI_ERR_INVALID, "%s: zero dtype must be PMI_F32 or PMI_U8 (got %d)", fn,
                zero_dtype);
  return PMI_OK;
}

}  // namespace

extern "C" {

int pmi_abi_version(void) { return PMI_ABI_VERSION; }

const char* pmi_last_error(void) { return g_err; }

int pmi_device_supported(int device) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n <= 0)
    return fail(PMI_ERR_NO_DEVICE, "pmi_device_supported: no HIP device");
  if (device < 0 || device >= n) {
    fail(PMI_OK, "pmi_device_supported: device %d out of range (count %d)", device, n);
    return 0;
  }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess)
    return fail(PMI_ERR_HIP, "pmi_device_supported: hipGetDeviceProperties failed");
  ok();
  return strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int pmi_repack_int4_for_kernel(const uint8_t* packed, uint8_t* out, const int32_t* perm,
                               int64_t N, int64_t K, int64_t group_size, void* stream) {
  const char* fn = "pmi_repack_int4_for_kernel";
  if (int rc = check_shape(N, K, group_size, fn)) return rc;
  if (N == 0) return ok();
  if (!packed || !out) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (packed == out) return fail(PMI_ERR_INVALID, "%s: in-place repack is not supported", fn);
  if (!aligned(out, 4)) return fail(PMI_ERR_INVALID, "%s: out must be 4-byte aligned", fn);
  return from_hip(pmi::launch_repack(packed, out, perm, N, K, group_size, (hipStream_t)stream), fn);
}

int pmi_zeros_to_u8(const float* zeros, uint8_t* zeros_u8, int32_t* bad_count, int64_t count,
                    void* stream) {
  const char* fn = "pmi_zeros_to_u8";
  if (count < 0) return fail(PMI_ERR_INVALID, "%s: count < 0", fn);
  if (count == 0) return ok();
  if (!zeros || !zeros_u8) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  return from_hip(pmi::launch_zeros_to_u8(zeros, zeros_u8, bad_count, count, (hipStream_t)stream),
                  fn);
}

int pmi_perm_u16(const int32_t* perm, uint16_t* perm16, int32_t* bad_count, int64_t K,
                 void* stream) {
  const char* fn = "pmi_perm_u16";
  if (K < 0 || K > 65536)
    return fail(PMI_ERR_INVALID, "%s: need 0 <= K <= 65536 (K=%lld)", fn, (long long)K);
  if (K == 0) return ok();
  if (!perm || !perm16) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(perm, 4)) return fail(PMI_ERR_INVALID, "%s: perm must be 4-byte aligned", fn);
  if (!aligned(perm16, 16)) return fail(PMI_ERR_INVALID, "%s: perm16 must be 16-byte aligned", fn);
  return from_hip(pmi::launch_perm_u16(perm, perm16, bad_count, K, (hipStream_t)stream), fn);
}

namespace {
int check_awq(int64_t N, int64_t K, int64_t gs, const char* fn) {
  if (int rc = check_shape(N, K, gs, fn)) return rc;
  if (N % 8 != 0)
    return fail(PMI_ERR_INVALID, "%s: N=%lld must be divisible by 8 (eight columns per int32)",
                fn, (long long)N);
  return PMI_OK;
}
}  // namespace

int pmi_awq_gemm_to_storage(const int32_t* qweight, const int32_t* qzeros, const void* scales,
                            uint8_t* packed, float* scale, float* zero, int64_t N, int64_t K,
                            int64_t group_size, void* stream) {
  const char* fn = "pmi_awq_gemm_to_storage";
  if (int rc = check_awq(N, K, group_size, fn)) return rc;
  if (N == 0) return ok();
  if (!qweight || !qzeros || !scales || !packed || !scale || !zero)
    return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(qweight, 4) || !aligned(qzeros, 4) || !aligned(scales, 2) || !aligned(scale, 4) ||
      !aligned(zero, 4) || !aligned(packed, 16))
    return fail(PMI_ERR_INVALID, "%s: misaligned buffer (packed needs 16 bytes)", fn);
  return from_hip(pmi::launch_awq_to_storage(qweight, qzeros, scales, packed, scale, zero, N, K,
                                             group_size, (hipStream_t)stream),
                  fn);
}

int pmi_storage_to_awq_gemm(const uint8_t* packed, const float* scale, const void* zero,
                            int zero_dtype, int32_t* qweight, int32_t* qzeros, void* scales,
                            int32_t* bad_count, int64_t N, int64_t K, int64_t group_size,
                            void* stream) {
  const char* fn = "pmi_storage_to_awq_gemm";
  if (int rc = check_awq(N, K, group_size, fn)) return rc;
  if (int rc = check_zero_dtype(zero_dtype, fn)) return rc;
  if (N == 0) return ok();
  if (!qweight || !qzeros || !scales || !packed || !scale || !zero)
    return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(qweight, 4) || !aligned(qzeros, 4) || !aligned(scales, 2) || !aligned(scale, 4) ||
      !aligned(zero, zero_dtype == PMI_F32 ? 4 : 1) || !aligned(packed, 16))
    return fail(PMI_ERR_INVALID, "%s: misaligned buffer (packed needs 16 bytes)", fn);
  return from_hip(pmi::launch_storage_to_awq(packed, scale, zero, zero_dtype == PMI_U8, qweight,
                                             qzeros, scales, bad_count, N, K, group_size,
                                             (hipStream_t)stream),
                  fn);
}

int pmi_set_kernel_override(int kernel) {
  if (kernel < 0 || kernel > 6)
    return fail(PMI_ERR_INVALID, "pmi_set_kernel_override: unknown kernel %d", kernel);
  ok();
  return g_kernel_override.exchange(kernel);
}

int pmi_matmul_kernel_choice(int64_t M, int64_t N, int64_t K, int64_t group_size, int flags) {
  const int forced = g_kernel_override.load();
  if (forced) return forced;
  const bool has_tiled = flags & PMI_CHOICE_TILED, has_perm = flags & PMI_CHOICE_PERM;
  // The tiled-weight GEMM (a contiguous weight stream, no K split), measured
  // on MI355X against the GEMV, skinny kernel and MFMA GEMM over 8-48 weight
  // copies beyond the MALL:
  // - 5..32 rows: it wins at every N while its workgroups take one pass over
  //   the CUs (N <= 16384; 1024 x 4096 at M = 16: 6.9 against 10.7 us for the
  //   MFMA GEMM; 512 x 3584 at M = 8: 5.3 against 7.3 us for the skinny
  //   kernel), and past that up to 12 rows (fused gate/up 28672 x 4096 at
  //   M = 8: 15.5 against 17.5 us; 18944 x 3584 at M = 16: 15.1 against
  //   13.9 us for the MFMA GEMM). K <= 8192: with longer rows its activation
  //   reloads per 16-row tile outweigh the weights.
  // - 3..4 rows: from N = 3072 (narrower layers: the GEMV, 4.3 against 5.1
  //   us at 1024 x 4096).
  // - 2 rows: for 8192 <= N <= 20480 (gate: 8.1 against 9.3 us for the GEMV).
  // - act_order up to 16 rows (X[:, perm] gathered inside the kernel when it
  //   fits LDS): from 3 rows at any N (512 x 3584 at M = 4: 6.0 against 7.5
  //   us for the GEMV, which gathers too), and at 2 rows from N = 3072.
  // - 33..64 rows (64-row activation blocks, every B operand feeding four
  //   activation tiles) while the workgroups take one pass (gate 14336 x 4096
  //   at M = 64: 15.9 against 17.6 us for the MFMA GEMM; 4096 x 4096: 10.5
  //   against 11.8 us).
  // - past one pass over the CUs (N > 16384), up to 12 rows, and up to 16 where
  //   ranges of 5-6 tiles per workgroup cover the tiles in one pass (Qwen gate/up
  //   18944 x 3584 at M = 16: 13.6 against 13.9 us; with act_order 13.3 against
  //   17.4 for the MFMA GEMM with its gather launch).
  const int64_t panels = (N + 63) / 64, cus = pmi::device_cu_count();
  const bool ranged = panels > cus && 4 * panels <= 6 * cus && group_size % 128 == 0;
  if (has_tiled && M >= 2 && M <= 64 && pmi::tgemm_supported(M, N, K, group_size) && K <= 8192 &&
      (N <= 16384 || M <= 12 || (ranged && M <= 16))) {
    const bool gathers = has_perm && M <= 16 && pmi::tgemm_gather_supported(M, K);
    if (gathers ? (M >= 3 || N >= 3072) : (M >= 5 || (M >= 3 && N >= 3072) || (N >= 8192 && N <= 20480)))
      return 5;
  }
  // Long rows (K > 8192, down_proj) up to 16 rows, where the tiled GEMM splits
  // K four ways over 64-row workgroups: Llama down 4096 x 14336 at M = 4 / 16
  // takes 10.3 / 11.8 against 14.0 us for the MFMA GEMM; Qwen down 3584 x 18944
  // 11.9 / 12.9 against 15.8 / 15.3. With act_order past 2 rows X[:, perm] is
  // gathered into the workspace first (M = 16: 17.6 against 20.0 us).
  if (has_tiled && M >= 2 && M <= 16 && K > 8192 && pmi::tgemm_supported(M, N, K, group_size)) {
    const pmi::TgemmConfig c =
        pmi::tgemm_config(M, N, K, group_size, has_perm && pmi::tgemm_gather_supported(M, K));
    if (c.splits > 1 && c.ntw == 4) return 5;
  }
  // Many activation rows (prefill): the big-tile GEMM, 256 weight rows x 128
  // activation rows per workgroup, where its tiles fill three quarters of
  // the CUs in one pass or more.
  if (has_tiled && M > 64 && group_size % 128 == 0 && pmi::tgemm_supported(M, N, K, group_size)) {
    const pmi::BgemmConfig b = pmi::bgemm_config(M, N, K, group_size);
    if (b.ok && (int64_t)b.n_bands * b.grid_m * 4 >= 3 * cus) return 6;
  }
  // Past 64 rows on narrow layers, while the tiled GEMM's 64-row blocks still
  // take one pass over the CUs: against the register-streamed GEMM, whose K
  // splits these layers need, k/v 1024 x 4096 at M = 256 takes 10.3 against
  // 17.0 us and 512 x 3584 at M = 512 takes 9.5 against 15.9 us; with a second
  // pass it loses (1024 x 4096 at M = 512: 19.4 against 16.3 us).
  if (has_tiled && M > 64 && K <= 8192 && pmi::tgemm_supported(M, N, K, group_size) &&
      pmi::tgemm_config(M, N, K, group_size, false).grid <= cus)
    return 5;
  // Group sizes 32 and 64 have no other matrix-core kernel: past 4 rows the
  // tiled GEMM (one activation block of 32 rows after another) replaces the
  // GEMV, which would stream the weights once per 4 rows.
  if (has_tiled && M > 4 && !pmi::gemm_supported(K, group_size) &&
      pmi::tgemm_supported(M, N, K, group_size))
    return 5;
  // Measured on MI355X (gate/up/down and q/k/v/o shapes): the GEMV wins up to
  // M = 2, and up to M = 4 for N < 8192 with K <= 8192, where the GEMM's K
  // splits cost more than its matrix cores save. With long rows the GEMV's
  // four activation rows cost more than the splits: down_proj at M = 4 takes
  // 16.5 against 15.0 us (4096 x 14336) and 31.9 against 16.2 us (3584 x
  // 18944; 20.2 against 16.2 at M = 3). The skinny kernel wins over the GEMM
  // for N <= 8192 while the activations fit its LDS.
  const bool gemm = pmi::gemm_supported(K, group_size);
  if (M <= 2 || (M <= 4 && ((N < 8192 && K <= 8192) || !gemm))) return 1;
  if (M >= 5 && N <= 8192 && pmi::skinny_supported(M, N, K, group_size)) return 3;
  // The register-streamed GEMM beats the MFMA GEMM by 3-8 % from M = 128 on
  // (Llama and Qwen shapes up to M = 512), and at 33-64 rows when its 128-row
  // blocks alone fill the CUs (fused gate/up at M = 64: 26.7 us against
  // 28.4 us); with a K split at M <= 64 it loses (gate_proj at M = 64: 23.2
  // us against 19.2 us).
  if (pmi::gemm64_supported(M, K, group_size)) {
    if (M > 64) return 4;
    if (M > 32 && pmi::gemm64_config(M, N, K).splits == 1 &&
        pmi::gemm64_config(M, N, K).grid >= 7 * pmi::device_cu_count() / 8)
      return 4;
  }
  return gemm ? 2 : 1;
}

int pmi_matmul_w4a16_glu(const void* gate_up, const uint8_t* w, const float* scales,
                         const void* zeros, int zero_dtype, void* y, int64_t M, int64_t N,
                         int64_t K, int64_t group_size, void* stream) {
  const char* fn = "pmi_matmul_w4a16_glu";
  if (int rc = check_shape(N, K, group_size, fn)) return rc;
  if (zero_dtype != PMI_U8)
    return fail(PMI_ERR_UNSUPPORTED, "%s: zero points must be PMI_U8 (got %d)", fn, zero_dtype);
  if (M < 0) return fail(PMI_ERR_INVALID, "%s: M < 0", fn);
  if (M > 4) return fail(PMI_ERR_UNSUPPORTED, "%s: the gated GEMV takes M <= 4 (got %lld)", fn,
                         (long long)M);
  if (M == 0 || N == 0) return ok();
  if (!gate_up || !w || !scales || !zeros || !y) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(gate_up, 16)) return fail(PMI_ERR_INVALID, "%s: gate_up must be 16-byte aligned", fn);
  if (!aligned(w, 16)) return fail(PMI_ERR_INVALID, "%s: packed weight must be 16-byte aligned", fn);
  if (!aligned(scales, 4)) return fail(PMI_ERR_INVALID, "%s: scales must be 4-byte aligned", fn);
  if (!aligned(y, 2)) return fail(PMI_ERR_INVALID, "%s: y must be 2-byte aligned", fn);
  pmi::GemvXform xf;
  xf.mode = 2;
  return from_hip(pmi::launch_gemv(gate_up, w, scales, zeros, 1, nullptr, y, M, N, K, group_size,
                                   (hipStream_t)stream, &xf),
                  fn);
}

int pmi_gate_up_silu_supported(int64_t M, int64_t N, int64_t K, int64_t group_size) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0 || K % group_size != 0) return 0;
  return pmi::tgemm_glu_supported(M, N, K, group_size) ? 1 : 0;
}

int pmi_matmul_w4a16_gate_up_silu(const void* x, const uint8_t* w_tiled, const float* scales_gm,
                                  const uint8_t* zeros_gm, void* y, int64_t M, int64_t N,
                                  int64_t K, int64_t group_size, void* stream) {
  const char* fn = "pmi_matmul_w4a16_gate_up_silu";
  if (int rc = check_shape(N, K, group_size, fn)) return rc;
  if (M < 0) return fail(PMI_ERR_INVALID, "%s: M < 0", fn);
  if (M == 0 || N == 0) return ok();
  if (!pmi::tgemm_glu_supported(M, N, K, group_size))
    return fail(PMI_ERR_UNSUPPORTED, "%s: shape not on the four-tile tiled GEMM (M=%lld N=%lld "
                "K=%lld gs=%lld; see pmi_gate_up_silu_supported)", fn, (long long)M, (long long)N,
                (long long)K, (long long)group_size);
  if (!x || !w_tiled || !scales_gm || !zeros_gm || !y) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(x, 16) || !aligned(w_tiled, 16) || !aligned(scales_gm, 16) || !aligned(y, 4))
    return fail(PMI_ERR_INVALID, "%s: x, w_tiled and scales_gm must be 16-byte aligned, y 4-byte", fn);
  return from_hip(pmi::launch_tgemm_glu(x, w_tiled, scales_gm, zeros_gm, y, M, N, K, group_size,
                                        (hipStream_t)stream),
                  fn);
}

int pmi_tiled_rmsnorm_supported(int64_t M, int64_t N, int64_t K, int64_t group_size, int glu) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0 || K % group_size != 0) return 0;
  return pmi::tgemm_norm_supported(M, N, K, group_size, glu != 0) ? 1 : 0;
}

int pmi_matmul_w4a16_tiled_rmsnorm(const void* x, const void* residual, const void* norm_weight,
                                   float eps, void* h_out, const uint8_t* w_tiled,
                                   const float* scales_gm, const uint8_t* zeros_gm, void* y,
                                   int64_t M, int64_t N, int64_t K, int64_t group_size, int glu,
                                   void* stream) {
  const char* fn = "pmi_matmul_w4a16_tiled_rmsnorm";
  if (int rc = check_shape(N, K, group_size, fn)) return rc;
  if (M < 0) return fail(PMI_ERR_INVALID, "%s: M < 0", fn);
  if (M == 0 || N == 0) return ok();
  if (!pmi::tgemm_norm_supported(M, N, K, group_size, glu != 0))
    return fail(PMI_ERR_UNSUPPORTED, "%s: shape not on the fused-norm tiled GEMM (M=%lld N=%lld "
                "K=%lld gs=%lld glu=%d; see pmi_tiled_rmsnorm_supported)", fn, (long long)M,
                (long long)N, (long long)K, (long long)group_size, glu);
  if (!x || !norm_weight || !w_tiled || !scales_gm || !zeros_gm || !y)
    return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (residual && !h_out) return fail(PMI_ERR_INVALID, "%s: a residual needs h_out", fn);
  if (!aligned(x, 16) || (residual && !aligned(residual, 16)) || !aligned(norm_weight, 16) ||
      (h_out && !aligned(h_out, 16)) || !aligned(w_tiled, 16) || !aligned(scales_gm, 16) ||
      !aligned(y, 8))
    return fail(PMI_ERR_INVALID, "%s: x, residual, norm_weight, h_out, w_tiled and scales_gm must "
                "be 16-byte aligned, y 8-byte", fn);
  return from_hip(pmi::launch_tgemm_norm(x, residual, norm_weight, eps, h_out, w_tiled, scales_gm,
                                         zeros_gm, y, M, N, K, group_size, glu != 0,
                                         (hipStream_t)stream),
                  fn);
}

int pmi_residual_stats_count(int64_t N, int64_t K, int glu) {
  if (N <= 0 || K <= 0 || K % 32 != 0) return 0;
  const pmi::GemvConfig c = pmi::gemv_config(1, N, K, glu ? 2 : 0);
  if (c.slice_waves < 2 || c.grid > pmi::kGemvMaxStats) return 0;
  return c.grid;
}

int pmi_matmul_w4a16_residual(const void* x, int glu, const void* residual, float* stats,
                              const uint8_t* w, const float* scales, const uint8_t* zeros_u8,
                              void* h, int64_t N, int64_t K, int64_t group_size, void* stream) {
  const char* fn = "pmi_matmul_w4a16_residual";
  if (int rc = check_shape(N, K, group_size, fn)) return rc;
  if (N == 0) return ok();
  if (pmi_residual_stats_count(N, K, glu) == 0)
    return fail(PMI_ERR_UNSUPPORTED, "%s: needs rows of at least two GEMV slices and at most %d "
                "workgroups (N=%lld K=%lld; see pmi_residual_stats_count)", fn, pmi::kGemvMaxStats,
                (long long)N, (long long)K);
  if (!x || !residual || !stats || !w || !scales || !zeros_u8 || !h)
    return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(x, 16) || !aligned(w, 16))
    return fail(PMI_ERR_INVALID, "%s: x and the packed weight must be 16-byte aligned", fn);
  if (!aligned(scales, 4) || !aligned(stats, 4) || !aligned(h, 2) || !aligned(residual, 2))
    return fail(PMI_ERR_INVALID, "%s: scales and stats must be 4-byte aligned, h and residual 2-byte",
                fn);
  pmi::GemvXform xf;
  xf.mode = glu ? 2 : 0;
  xf.res = residual;
  xf.stats = stats;
  return from_hip(pmi::launch_gemv(x, w, scales, zeros_u8, 1, nullptr, h, 1, N, K, group_size,
                                   (hipStream_t)stream, &xf),
                  fn);
}

int pmi_matmul_w4a16_prenormed(const void* x, const float* stats, int n_stats,
                               const void* norm_weight, float eps, const uint8_t* w,
                               const float* scales, const uint8_t* zeros_u8, void* y, int64_t N,
                               int64_t K, int64_t group_size, void* stream) {
  const char* fn = "pmi_matmul_w4a16_prenormed";
  if (int rc = check_shape(N, K, group_size, fn)) return rc;
  if (N == 0) return ok();
  if (n_stats < 1 || n_stats > pmi::kGemvMaxStats)
    return fail(PMI_ERR_INVALID, "%s: n_stats must be in [1, %d] (got %d)", fn, pmi::kGemvMaxStats,
                n_stats);
  if (!x || !stats || !norm_weight || !w || !scales || !zeros_u8 || !y)
    return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(x, 16) || !aligned(norm_weight, 16) || !aligned(w, 16))
    return fail(PMI_ERR_INVALID, "%s: x, norm_weight and the packed weight must be 16-byte aligned",
                fn);
  if (!aligned(scales, 4) || !aligned(stats, 4) || !aligned(y, 2))
    return fail(PMI_ERR_INVALID, "%s: scales and stats must be 4-byte aligned, y 2-byte", fn);
  pmi::GemvXform xf;
  xf.mode = 5;
  xf.w = norm_weight;
  xf.eps = eps;
  xf.stats = const_cast<float*>(stats);
  xf.n_stats = n_stats;
  return from_hip(pmi::launch_gemv(x, w, scales, zeros_u8, 1, nullptr, y, 1, N, K, group_size,
                                   (hipStream_t)stream, &xf),
                  fn);
}

int pmi_matmul_w4a16_rmsnorm(const void* x, const void* residual, const void* norm_weight,
                             float eps, void* h_out, const uint8_t* w, const float* scales,
                             const void* zeros, int zero_dtype, void* y, int64_t M, int64_t N,
                             int64_t K, int64_t group_size, void* stream) {
  const char* fn = "pmi_matmul_w4a16_rmsnorm";
  if (int rc = check_shape(N, K, group_size, fn)) return rc;
  if (zero_dtype != PMI_U8)
    return fail(PMI_ERR_UNSUPPORTED, "%s: zero points must be PMI_U8 (got %d)", fn, zero_dtype);
  if (M < 0) return fail(PMI_ERR_INVALID, "%s: M < 0", fn);
  if (M > 4) return fail(PMI_ERR_UNSUPPORTED, "%s: the fused GEMV takes M <= 4 (got %lld)", fn,
                         (long long)M);
  if (M == 0 || N == 0) return ok();
  if (!x || !norm_weight || !w || !scales || !zeros || !y)
    return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (residual && !h_out) return fail(PMI_ERR_INVALID, "%s: a residual needs h_out", fn);
  if (!aligned(x, 16) || (residual && !aligned(residual, 16)) || !aligned(norm_weight, 16) ||
      (h_out && !aligned(h_out, 16)))
    return fail(PMI_ERR_INVALID, "%s: x, residual, norm_weight and h_out must be 16-byte aligned",
                fn);
  if (!aligned(w, 16)) return fail(PMI_ERR_INVALID, "%s: packed weight must be 16-byte aligned", fn);
  if (!aligned(scales, 4)) return fail(PMI_ERR_INVALID, "%s: scales must be 4-byte aligned", fn);
  if (!aligned(y, 2)) return fail(PMI_ERR_INVALID, "%s: y must be 2-byte aligned", fn);
  pmi::GemvXform xf;
  xf.mode = 3;
  xf.r = residual;
  xf.w = norm_weight;
  xf.eps = eps;
  xf.h_out = h_out;
  return from_hip(pmi::launch_gemv(x, w, scales, zeros, 1, nullptr, y, M, N, K, group_size,
                                   (hipStream_t)stream, &xf),
                  fn);
}

size_t pmi_tiled_bytes(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0) return 0;
  return pmi::tiled_bytes(N, K);
}

int pmi_tile_w4a16(const uint8_t* w_kernel, uint8_t* w_tiled, int64_t N, int64_t K,
                   int64_t group_size, void* stream) {
  const char* fn = "pmi_tile_w4a16";
  if (int rc = check_shape(N, K, group_size, fn)) return rc;
  if (K % 128 != 0)
    return fail(PMI_ERR_UNSUPPORTED, "%s: K=%lld must be a multiple of 128", fn, (long long)K);
  if (group_size != 32 && group_size != 64 && group_size % 128 != 0)
    return fail(PMI_ERR_UNSUPPORTED, "%s: group_size must be 32, 64 or a multiple of 128 (got %lld)",
                fn, (long long)group_size);
  if ((int64_t)pmi::tiled_bytes(N, K) >= (1ll << 31))
    return fail(PMI_ERR_UNSUPPORTED, "%s: shape too large (N=%lld K=%lld)", fn, (long long)N,
                (long long)K);
  if (N == 0) return ok();
  if (!w_kernel || !w_tiled) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (w_kernel == w_tiled) return fail(PMI_ERR_INVALID, "%s: in-place tiling is not supported", fn);
  if (!aligned(w_kernel, 16) || !aligned(w_tiled, 16))
    return fail(PMI_ERR_INVALID, "%s: buffers must be 16-byte aligned", fn);
  return from_hip(pmi::launch_tile(w_kernel, w_tiled, N, K, group_size, (hipStream_t)stream), fn);
}

namespace {

// Workspace of the tiled GEMM (when a caller has the tiled copy): the act_order
// gather of X where the kernel does not gather itself, and the split-K
// partial tiles after it.
size_t tgemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group_size, bool has_perm) {
  if (!pmi::tgemm_supported(M, N, K, group_size)) return 0;
  const bool gathers = has_perm && pmi::tgemm_gather_supported(M, K);
  const size_t xg = has_perm && !gathers ? pmi::ws_perm_bytes(M, K) : 0;
  const size_t split = pmi::tgemm_config(M, N, K, group_size, gathers).ws_split;
  return xg + split ? pmi::kWsCounterBytes + xg + split : 0;
}

size_t other_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group_size, int has_perm) {
  const int choice = pmi_matmul_kernel_choice(M, N, K, group_size, 0);
  if (choice == 2 && pmi::gemm_supported(K, group_size))
    return pmi::gemm_workspace_bytes(M, N, K, group_size, has_perm != 0);
  if (choice == 4 && pmi::gemm64_supported(M, K, group_size)) {
    const size_t split = pmi::gemm64_config(M, N, K).ws_split;
    const size_t perm = has_perm ? pmi::ws_perm_bytes(M, K) : 0;
    return split + perm ? pmi::kWsCounterBytes + perm + split : 0;
  }
  // the GEMV reads act_order activations gathered once into the workspace
  // where its rows do not fit LDS (the size is reported either way, so that a
  // caller's workspace covers a forced or fallback launch)
  if ((choice == 1 || choice == 4) && has_perm)
    return pmi::kWsCounterBytes + pmi::ws_perm_bytes(M, K);
  // choice 3 (skinny) gathers in LDS; a tiled-GEMM launch with perm needs the
  // gather of X in the workspace
  if (has_perm && pmi::tgemm_supported(M, N, K, group_size))
    return pmi::kWsCounterBytes + pmi::ws_perm_bytes(M, K);
  return 0;
}

}  // namespace

int pmi_tgemm_splits(int64_t M, int64_t N, int64_t K, int64_t group_size, int has_perm) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0 || K % group_size != 0 ||
      !pmi::tgemm_supported(M, N, K, group_size))
    return 1;
  return pmi::tgemm_config(M, N, K, group_size, has_perm && pmi::tgemm_gather_supported(M, K)).splits;
}

size_t pmi_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group_size,
                                  int has_perm) {
  if (M <= 0 || N <= 0 || K <= 0 || group_size <= 0 || K % group_size != 0) return 0;
  // enough for whichever kernel runs, with or without the tiled copy, and
  // with act_order for the gather of X[:, perm] (bf16 activations always
  // gather into the workspace)
  const size_t other = other_workspace_bytes(M, N, K, group_size, has_perm);
  const size_t tiled = tgemm_workspace_bytes(M, N, K, group_size, has_perm != 0);
  size_t need = other > tiled ? other : tiled;
  if (has_perm && need < pmi::kWsCounterBytes + pmi::ws_perm_bytes(M, K))
    need = pmi::kWsCounterBytes + pmi::ws_perm_bytes(M, K);
  return need;
}

int pmi_sz_group_major(const float* scales, const void* zeros, int zero_dtype, float* scales_gm,
                       uint8_t* zeros_gm, int32_t* bad_count, int64_t N, int64_t G,
                       void* stream) {
  const char* fn = "pmi_sz_group_major";
  if (int rc = check_zero_dtype(zero_dtype, fn)) return rc;
  if (N < 0 || G <= 0) return fail(PMI_ERR_INVALID, "%s: need N >= 0 and G > 0", fn);
  if (N * G >= (1ll << 31)) return fail(PMI_ERR_UNSUPPORTED, "%s: N*G too large", fn);
  if (N == 0) return ok();
  if (!scales || !zeros || !scales_gm || !zeros_gm) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  return from_hip(pmi::launch_sz_group_major(scales, zeros, zero_dtype == PMI_U8, scales_gm,
                                             zeros_gm, bad_count, N, G, (hipStream_t)stream),
                  fn);
}

int pmi_matmul_w4a16(const void* x, int x_dtype, const uint8_t* w, const float* scales,
                     const void* zeros, int zero_dtype, const int32_t* perm,
                     const uint16_t* perm16, const float* scales_gm, const uint8_t* zeros_gm, const uint8_t* w_tiled, void* y,
                     int y_dtype, int64_t M, int64_t N, int64_t K, int64_t group_size,
                     void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "pmi_matmul_w4a16";
  if (int rc = check_shape(N, K, group_size, fn)) return rc;
  if (int rc = check_zero_dtype(zero_dtype, fn)) return rc;
  if (M < 0) return fail(PMI_ERR_INVALID, "%s: M < 0", fn);
  const bool bf = x_dtype == PMI_BF16;
  if (!((x_dtype == PMI_F16 && y_dtype == PMI_F16) || (bf && y_dtype == PMI_BF16)))
    return fail(PMI_ERR_UNSUPPORTED, "%s: x and y must both be fp16 or both bf16 (got x=%d y=%d)",
                fn, x_dtype, y_dtype);
  if (M > (1ll << 31) - 1) return fail(PMI_ERR_UNSUPPORTED, "%s: M too large", fn);
  if (M == 0 || N == 0) return ok();
  if (!x || !w || !scales || !zeros || !y) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(x, 16)) return fail(PMI_ERR_INVALID, "%s: x must be 16-byte aligned", fn);
  if (!aligned(w, 16)) return fail(PMI_ERR_INVALID, "%s: packed weight must be 16-byte aligned", fn);
  if (!aligned(scales, 4)) return fail(PMI_ERR_INVALID, "%s: scales must be 4-byte aligned", fn);
  if (zero_dtype == PMI_F32 && !aligned(zeros, 4))
    return fail(PMI_ERR_INVALID, "%s: fp32 zeros must be 4-byte aligned", fn);
  if (!aligned(y, 2)) return fail(PMI_ERR_INVALID, "%s: y must be 2-byte aligned", fn);
  if (perm && !aligned(perm, 4)) return fail(PMI_ERR_INVALID, "%s: perm must be 4-byte aligned", fn);
  if (perm16 && !perm) return fail(PMI_ERR_INVALID, "%s: perm16 is given with perm", fn);
  if (perm16 && (K > 65536 || !aligned(perm16, 16)))
    return fail(PMI_ERR_INVALID, "%s: perm16 needs K <= 65536 and 16-byte alignment", fn);
  if (!scales_gm != !zeros_gm)
    return fail(PMI_ERR_INVALID, "%s: scales_gm and zeros_gm are given together or not at all", fn);
  if (scales_gm && (!aligned(scales_gm, 4) || !aligned(zeros_gm, 4)))
    return fail(PMI_ERR_INVALID, "%s: scales_gm and zeros_gm must be 4-byte aligned", fn);
  if (workspace_bytes && (!workspace || !aligned(workspace, 256)))
    return fail(PMI_ERR_INVALID, "%s: workspace must be non-null and 256-byte aligned", fn);
  if (w_tiled && !aligned(w_tiled, 16))
    return fail(PMI_ERR_INVALID, "%s: w_tiled must be 16-byte aligned", fn);

  hipStream_t s = (hipStream_t)stream;
  const int zu8 = zero_dtype == PMI_U8;
  const int forced = g_kernel_override.load();
  if (bf) {
    // bf16 activations (the native bf16 extension): with the tiled copy, the
    // rows an fp16 call would run on the tiled GEMM's 16-row blocks (no
    // act_order) take its bf16 variant; the rest run on the GEMV, four
    // activation rows per launch, act_order rows gathered into the workspace
    // first (2-byte elements, as for fp16)
    if (forced && forced != 1 && forced != 5)
      return fail(PMI_ERR_UNSUPPORTED, "%s: bf16 activations run on the GEMV or the tiled GEMM only "
                  "(kernel %d forced)", fn, forced);
    const bool bf_tiled = w_tiled && scales_gm && zeros_gm && N % 4 == 0 && !perm && aligned(y, 8) &&
                          pmi::tgemm_bf16_supported(M, N, K, group_size);
    if (forced == 5 && !bf_tiled)
      return fail(PMI_ERR_UNSUPPORTED, "%s: the tiled GEMM's bf16 variant needs w_tiled, scales_gm and "
                  "zeros_gm, no perm, y 8-byte aligned, group_size %% 128 == 0 and 16-row blocks", fn);
    if (bf_tiled && (forced == 5 || (!forced && pmi_matmul_kernel_choice(M, N, K, group_size,
                                                                         PMI_CHOICE_TILED) == 5)))
      return from_hip(pmi::launch_tgemm(x, nullptr, nullptr, w_tiled, scales_gm, zeros_gm, y, M, N,
                                        K, group_size, nullptr, 0, 0, s, true),
                      fn);
    const uint16_t* xp = (const uint16_t*)x;
    if (perm) {
      if (workspace_bytes < pmi::kWsCounterBytes + pmi::ws_perm_bytes(M, K))
        return fail(PMI_ERR_UNSUPPORTED, "%s: bf16 with perm needs a workspace of "
                    "pmi_matmul_workspace_bytes() bytes", fn);
      uint16_t* xg = (uint16_t*)((uint8_t*)workspace + pmi::kWsCounterBytes);
      hipError_t e = pmi::launch_gather_cols(x, perm, xg, M, K, s);
      if (e != hipSuccess) return from_hip(e, fn);
      xp = xg;
    }
    pmi::GemvXform bxf;
    bxf.mode = 6;
    uint16_t* yp = (uint16_t*)y;
    for (int64_t m = 0; m < M; m += 4) {
      const int64_t mt = M - m < 4 ? M - m : 4;
      hipError_t e = pmi::launch_gemv(xp + m * K, w, scales, zeros, zu8, nullptr, yp + m * N, mt, N, K,
                                      group_size, s, &bxf);
      if (e != hipSuccess) return from_hip(e, fn);
    }
    return ok();
  }
  // the tiled GEMM reads the tiled weights and the group-major scale/zero copies
  const bool has_tiled = w_tiled && scales_gm && zeros_gm && N % 4 == 0;
  int choice = pmi_matmul_kernel_choice(
      M, N, K, group_size, (has_tiled ? PMI_CHOICE_TILED : 0) | (perm ? PMI_CHOICE_PERM : 0));
  // the tiled GEMM's epilogue (both variants) stores up to four fp16 outputs
  // (8 bytes) per lane
  if ((choice == 5 || choice == 6) && !aligned(y, 8)) {
    if (forced) return fail(PMI_ERR_INVALID, "%s: the tiled GEMM needs y 8-byte aligned", fn);
    choice = pmi_matmul_kernel_choice(M, N, K, group_size, perm ? PMI_CHOICE_PERM : 0);
  }
  if (choice == 6) {
    if (!has_tiled || !pmi::tgemm_supported(M, N, K, group_size) || group_size % 128 != 0 ||
        !pmi::bgemm_config(M, N, K, group_size).ok)
      return fail(PMI_ERR_UNSUPPORTED, "%s: the big-tile GEMM needs w_tiled, scales_gm and zeros_gm, "
                  "N %% 4 == 0, K %% 512 == 0, K >= 1536, group_size %% 128 == 0 and M * K < 2^30", fn);
    // act_order: X[:, perm] gathered into the workspace first
    const void* xs = x;
    if (perm) {
      if (workspace_bytes < pmi::kWsCounterBytes + pmi::ws_perm_bytes(M, K))
        return fail(PMI_ERR_UNSUPPORTED, "%s: the big-tile GEMM with perm needs a workspace of "
                    "pmi_matmul_workspace_bytes() bytes", fn);
      void* xg = (uint8_t*)workspace + pmi::kWsCounterBytes;
      hipError_t e = pmi::launch_gather_cols(x, perm, xg, M, K, s);
      if (e != hipSuccess) return from_hip(e, fn);
      xs = xg;
    }
    return from_hip(pmi::launch_bgemm(xs, w_tiled, scales_gm, zeros_gm, y, M, N, K, group_size, s), fn);
  }
  if (choice == 5) {
    if (!has_tiled || !pmi::tgemm_supported(M, N, K, group_size))
      return fail(PMI_ERR_UNSUPPORTED, "%s: the tiled GEMM needs w_tiled, scales_gm and zeros_gm, "
                  "N %% 4 == 0, K %% 512 == 0, K >= 1536 and group_size 32, 64 or a "
                  "multiple of 128", fn);
    // act_order: up to 16 rows the kernel gathers X[:, perm] itself (from
    // LDS); past that X[:, perm] is gathered into the workspace first
    // (the split-K partial tiles follow the counters, or the gathered X)
    void* ws = workspace_bytes >= pmi::kWsCounterBytes ? workspace : nullptr;
    if (!perm || pmi::tgemm_gather_supported(M, K))
      return from_hip(pmi::launch_tgemm(x, perm, perm16, w_tiled, scales_gm, zeros_gm, y, M, N, K,
                                        group_size, ws, workspace_bytes, pmi::kWsCounterBytes, s),
                      fn);
    if (workspace_bytes >= pmi::kWsCounterBytes + pmi::ws_perm_bytes(M, K)) {
      void* xg = (uint8_t*)workspace + pmi::kWsCounterBytes;
      hipError_t e = pmi::launch_gather_cols(x, perm, xg, M, K, s);
      if (e != hipSuccess) return from_hip(e, fn);
      return from_hip(pmi::launch_tgemm(xg, nullptr, nullptr, w_tiled, scales_gm, zeros_gm, y, M, N,
                                        K, group_size, ws, workspace_bytes,
                                        pmi::kWsCounterBytes + pmi::ws_perm_bytes(M, K), s),
                      fn);
    }
    if (forced) return fail(PMI_ERR_UNSUPPORTED, "%s: forced tiled GEMM with perm needs a "
                            "workspace of pmi_matmul_workspace_bytes() bytes", fn);
    choice = pmi_matmul_kernel_choice(M, N, K, group_size, 0);
  }
  // act_order on the GEMM gathers X[:, perm] into the workspace; without one
  // the automatic choice falls back to the GEMV.
  const bool perm_fits = !perm || !pmi::gemm_supported(K, group_size) ||
                         workspace_bytes >= pmi::gemm_workspace_bytes(M, N, K, group_size, true) -
                                                pmi::gemm_config(M, N, K, group_size, true).ws_split;
  if (choice == 2 && !perm_fits) {
    if (forced) return fail(PMI_ERR_UNSUPPORTED, "%s: forced MFMA GEMM with perm needs a workspace "
                            "of pmi_matmul_workspace_bytes() bytes", fn);
    choice = 1;
  }
  if (choice == 4 && !pmi::gemm64_supported(M, K, group_size))
    return fail(PMI_ERR_UNSUPPORTED, "%s: forced register-streamed GEMM needs group_size == 128 "
                "and M*K*2 < 2^31", fn);
  if (choice == 4) {
    // act_order: X[:, perm] is gathered into the workspace first (as for the
    // MFMA GEMM); the split-K partial tiles follow it
    const void* xs = x;
    size_t part_offset = pmi::kWsCounterBytes;
    if (perm) {
      if (workspace_bytes < pmi::kWsCounterBytes + pmi::ws_perm_bytes(M, K))
        return fail(PMI_ERR_UNSUPPORTED, "%s: register-streamed GEMM with perm needs a workspace "
                    "of pmi_matmul_workspace_bytes() bytes", fn);
      void* xg = (uint8_t*)workspace + pmi::kWsCounterBytes;
      hipError_t e = pmi::launch_gather_cols(x, perm, xg, M, K, s);
      if (e != hipSuccess) return from_hip(e, fn);
      xs = xg;
      part_offset += pmi::ws_perm_bytes(M, K);
    }
    return from_hip(pmi::launch_gemm64(xs, w, scales, zeros, zu8, scales_gm, zeros_gm, y, M, N, K,
                                       workspace_bytes >= pmi::kWsCounterBytes ? workspace : nullptr,
                                       workspace_bytes, part_offset, s), fn);
  }
  if (choice == 3 && !pmi::skinny_supported(M, N, K, group_size))
    return fail(PMI_ERR_UNSUPPORTED, "%s: forced skinny kernel needs M <= 16, group_size %% 128 "
                "== 0 and the activations within 64 KiB of LDS", fn);
  if (choice == 2 && !pmi::gemm_supported(K, group_size))
    return fail(PMI_ERR_UNSUPPORTED, "%s: forced MFMA GEMM needs group_size %% 128 == 0 and "
                "K %% 256 == 0", fn);
  if (choice == 3)
    return from_hip(pmi::launch_skinny(x, w, scales, zeros, zu8, perm, y, M, N, K, group_size, s),
                    fn);
  if (choice == 2)
    return from_hip(pmi::launch_gemm(x, w, scales, zeros, zu8, scales_gm, zeros_gm, perm, y, M, N,
                                     K, group_size, workspace, workspace_bytes, s), fn);
  // GEMV, four activation rows per launch. With act_order, every workgroup
  // stages X in LDS and gathers X[:, perm] from there when the rows fit
  // (64 KiB); otherwise X[:, perm] is gathered once into the workspace by a
  // launch of its own, or, without room in the workspace, every lane gathers
  // its columns from global memory. The LDS gather reads the 16-bit copy of
  // the permutation when the caller gives one (half the bytes every
  // workgroup reads before its first gather).
  const uint16_t* xp = (const uint16_t*)x;
  uint16_t* yp = (uint16_t*)y;
  pmi::GemvXform perm_xf;
  perm_xf.mode = perm16 ? 8 : 4;
  const bool perm_lds = perm && pmi::gemv_perm_lds_ok(M, N, K);
  const int32_t* gemv_perm = perm_lds && perm16 ? reinterpret_cast<const int32_t*>(perm16) : perm;
  if (perm && !perm_lds && workspace_bytes >= pmi::kWsCounterBytes + pmi::ws_perm_bytes(M, K)) {
    uint16_t* xg = (uint16_t*)((uint8_t*)workspace + pmi::kWsCounterBytes);
    hipError_t e = pmi::launch_gather_cols(x, perm, xg, M, K, s);
    if (e != hipSuccess) return from_hip(e, fn);
    xp = xg;
    gemv_perm = nullptr;
  }
  for (int64_t m = 0; m < M; m += 4) {
    const int64_t mt = M - m < 4 ? M - m : 4;
    hipError_t e = pmi::launch_gemv(xp + m * K, w, scales, zeros, zu8, gemv_perm, yp + m * N, mt, N,
                                    K, group_size, s, perm_lds ? &perm_xf : nullptr);
    if (e != hipSuccess) return from_hip(e, fn);
  }
  return ok();
}

}  // extern "C"

// ---- allocation-free matmul ---------------------------------------------------
// The scratch of pmi_matmul_w4a16_noalloc: a file-scope device array, one copy
// per GPU, held until the process ends. In host code `scratch` only names the
// symbol; its device address on the current GPU comes from
// hipGetSymbolAddress, once per device, and only that address is ever passed
// to a kernel. Layout as a pmi_matmul_w4a16 workspace: the split-K counter
// block first (zero between calls; cleared by a fill kernel the first time a
// device is used), then the act_order gather of X and the partial tiles.
namespace {
constexpr size_t kScratchBytes = 16u << 20;
}  // namespace

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {

constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

__global__ void scratch_clear_kernel(uint32_t* p, int words) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < words) p[i] = 0u;
}

// Device address of `scratch` on the current device (set up on first use,
// with its counter block cleared on `stream` ahead of the caller's launches).
int scratch_ptr(void** out, hipStream_t stream, const char* fn) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return from_hip(e, fn);
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(PMI_ERR_UNSUPPORTED, "%s: device %d is beyond the %d devices served", fn, dev,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return from_hip(e, fn);
    if (!p) return fail(PMI_ERR_HIP, "%s: hipGetSymbolAddress gave a null address", fn);
    const int words = (int)(pmi::kWsCounterBytes / 4);
    hipLaunchKernelGGL(scratch_clear_kernel, dim3((words + 255) / 256), dim3(256), 0, stream,
                       (uint32_t*)p, words);
    e = hipGetLastError();
    if (e != hipSuccess) return from_hip(e, fn);
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return PMI_OK;
}

}  // namespace

extern "C" {

int pmi_matmul_w4a16_noalloc(const void* x, int x_dtype, const uint8_t* w, const float* scales,
                             const void* zeros, int zero_dtype, const int32_t* perm,
                             const uint16_t* perm16, const float* scales_gm, const uint8_t* zeros_gm,
                             const uint8_t* w_tiled, void* y,
                             int y_dtype, int64_t M, int64_t N, int64_t K, int64_t group_size,
                             void* stream) {
  const char* fn = "pmi_matmul_w4a16_noalloc";
  if (int rc = check_shape(N, K, group_size, fn)) return rc;
  if (M < 0) return fail(PMI_ERR_INVALID, "%s: M < 0", fn);
  if (M == 0 || N == 0) return ok();
  const size_t need = pmi_matmul_workspace_bytes(M, N, K, group_size, perm != nullptr);
  if (need > kScratchBytes)
    return fail(PMI_ERR_UNSUPPORTED, "%s: this shape needs %zu bytes of scratch (M=%lld N=%lld "
                "K=%lld%s), more than the library's fixed %zu; call pmi_matmul_w4a16 with a "
                "workspace of pmi_matmul_workspace_bytes() bytes", fn, need, (long long)M,
                (long long)N, (long long)K, perm ? ", act_order" : "", kScratchBytes);
  void* ws = nullptr;
  if (need) {
    if (int rc = scratch_ptr(&ws, (hipStream_t)stream, fn)) return rc;
  }
  const int rc = pmi_matmul_w4a16(x, x_dtype, w, scales, zeros, zero_dtype, perm, perm16, scales_gm,
                                  zeros_gm, w_tiled, y, y_dtype, M, N, K, group_size, ws,
                                  need ? kScratchBytes : 0, stream);
  if (rc) {
    // keep the message, name this entry point
    char msg[sizeof(g_err)];
    snprintf(msg, sizeof(msg), "%s", g_err);
    return fail(rc, "%s: %s", fn, msg);
  }
  return ok();
}

int pmi_dequant_w4a16(const uint8_t* w, int layout, const float* scales, const void* zeros,
                      int zero_dtype, const int32_t* idx, void* w_out, int out_dtype, int64_t N,
                      int64_t K, int64_t group_size, void* stream) {
  const char* fn = "pmi_dequant_w4a16";
  if (N < 0 || K <= 0 || group_size <= 0 || K % group_size != 0 || K % 2 != 0)
    return fail(PMI_ERR_INVALID, "%s: need K even and divisible by group_size (N=%lld K=%lld gs=%lld)",
                fn, (long long)N, (long long)K, (long long)group_size);
  if (layout != PMI_LAYOUT_STORAGE && layout != PMI_LAYOUT_KERNEL)
    return fail(PMI_ERR_INVALID, "%s: unknown layout %d", fn, layout);
  if (layout == PMI_LAYOUT_KERNEL && group_size % 2 != 0)
    return fail(PMI_ERR_INVALID, "%s: kernel layout needs an even group_size", fn);
  if (int rc = check_zero_dtype(zero_dtype, fn)) return rc;
  if (out_dtype != PMI_F16 && out_dtype != PMI_BF16 && out_dtype != PMI_F32)
    return fail(PMI_ERR_INVALID, "%s: out dtype must be PMI_F16, PMI_BF16 or PMI_F32", fn);
  if (N == 0) return ok();
  if (!w || !scales || !zeros || !w_out) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  return from_hip(pmi::launch_dequant(w, layout, scales, zeros, zero_dtype == PMI_U8, idx, w_out,
                                      out_dtype, N, K, group_size, (hipStream_t)stream),
                  fn);
}

int pmi_rtn_quantize(const void* w, int w_dtype, uint8_t* packed, float* scale, float* zero,
                     int64_t N, int64_t K, int64_t group_size, int sym, void* stream) {
  const char* fn = "pmi_rtn_quantize";
  if (N < 0 || K <= 0 || group_size <= 0 || K % group_size != 0)
    return fail(PMI_ERR_INVALID, "%s: in_features=%lld is not divisible by group_size=%lld", fn,
                (long long)K, (long long)group_size);
  if (group_size % 2 != 0 || K % 2 != 0)
    return fail(PMI_ERR_INVALID, "%s: INT4 packing needs an even group_size and K", fn);
  if (w_dtype != PMI_F32 && w_dtype != PMI_F16 && w_dtype != PMI_BF16)
    return fail(PMI_ERR_INVALID, "%s: weight dtype must be PMI_F32, PMI_F16 or PMI_BF16", fn);
  if (sym < 0 || sym > 2) return fail(PMI_ERR_INVALID, "%s: sym must be 0, 1 or 2", fn);
  if (N == 0) return ok();
  if (!w || !packed || !scale || !zero) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  return from_hip(pmi::launch_rtn(w, w_dtype, packed, scale, zero, N, K, group_size, sym,
                                  (hipStream_t)stream),
                  fn);
}

// ---- GPTQ producer -----------------------------------------------------------

int pmi_gptq_group_params(const float* w, int64_t ldw, int64_t N, int64_t col0, int64_t cols,
                          int sym, float* scale, float* zero, int64_t G, int64_t g, void* stream) {
  const char* fn = "pmi_gptq_group_params";
  if (N < 0 || cols <= 0 || col0 < 0 || col0 + cols > ldw || G <= 0 || g < 0 || g >= G)
    return fail(PMI_ERR_INVALID, "%s: need N >= 0, 0 <= col0, col0 + cols <= ldw, 0 <= g < G", fn);
  if (sym < 0 || sym > 2) return fail(PMI_ERR_INVALID, "%s: sym must be 0, 1 or 2", fn);
  if (N == 0) return ok();
  if (!w || !scale || !zero) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  return from_hip(pmi::launch_gptq_group_params(w, ldw, N, col0, cols, sym, scale, zero, G, g,
                                                (hipStream_t)stream),
                  fn);
}

int pmi_gptq_block(const float* w, const float* c, const int32_t* colg, const float* scale,
                   const float* zero, uint8_t* codes, float* errors, int64_t N, int64_t K,
                   int64_t G, int64_t b0, int64_t count, void* stream) {
  const char* fn = "pmi_gptq_block";
  if (N < 0 || K <= 0 || K % 16 != 0 || G <= 0)
    return fail(PMI_ERR_INVALID, "%s: need N >= 0, K > 0 with K %% 16 == 0, G > 0", fn);
  if (b0 < 0 || b0 % 16 != 0 || count <= 0 || count > 128 || count % 16 != 0 || b0 + count > K)
    return fail(PMI_ERR_INVALID,
                "%s: the block [b0, b0 + count) must lie in [0, K) with b0 and count multiples "
                "of 16 and count <= 128 (b0=%lld count=%lld K=%lld)",
                fn, (long long)b0, (long long)count, (long long)K);
  if (N == 0) return ok();
  if (!w || !c || !colg || !scale || !zero || !codes || !errors)
    return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(w, 16)) return fail(PMI_ERR_INVALID, "%s: w must be 16-byte aligned", fn);
  return from_hip(pmi::launch_gptq_block(w, c, colg, scale, zero, codes, errors, N, K, G, b0,
                                         (int)count, (hipStream_t)stream),
                  fn);
}

int pmi_gptq_pack(const uint8_t* codes, const int32_t* inv_perm, uint8_t* packed, int64_t N,
                  int64_t K, void* stream) {
  const char* fn = "pmi_gptq_pack";
  if (N < 0 || K <= 0 || K % 8 != 0)
    return fail(PMI_ERR_INVALID, "%s: need N >= 0 and K > 0 with K %% 8 == 0", fn);
  if (N == 0) return ok();
  if (!codes || !packed) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(packed, 4)) return fail(PMI_ERR_INVALID, "%s: packed must be 4-byte aligned", fn);
  return from_hip(pmi::launch_gptq_pack(codes, inv_perm, packed, N, K, (hipStream_t)stream), fn);
}

// ---- caller-side decoder ops ---------------------------------------------

int pmi_add_rmsnorm_f16(const void* x, const void* residual, const void* weight, void* y,
                        void* residual_out, int64_t rows, int64_t dim, float eps, void* stream) {
  const char* fn = "pmi_add_rmsnorm_f16";
  if (rows < 0 || dim <= 0 || dim % 8 != 0 || dim > 8192)
    return fail(PMI_ERR_INVALID, "%s: need rows >= 0 and 0 < dim <= 8192, dim %% 8 == 0", fn);
  if (rows == 0) return ok();
  if (!x || !weight || !y || (!residual != !residual_out))
    return fail(PMI_ERR_INVALID, "%s: null buffer (residual and residual_out go together)", fn);
  for (const void* p : {x, residual, weight, (const void*)y, (const void*)residual_out})
    if (p && !aligned(p, 16)) return fail(PMI_ERR_INVALID, "%s: buffers must be 16-byte aligned", fn);
  return from_hip(pmi::launch_add_rmsnorm(x, residual, weight, y, residual_out, rows, dim, eps,
                                          (hipStream_t)stream), fn);
}

int pmi_rope_kv_f16(const void* qkv, const float* cos_t, const float* sin_t, const int64_t* pos,
                    void* q_out, void* cache_k, void* cache_v, int64_t B, int64_t T, int64_t H,
                    int64_t KV, int64_t D, int64_t L, void* stream) {
  const char* fn = "pmi_rope_kv_f16";
  if (B < 0 || T <= 0 || H <= 0 || KV <= 0 || H % KV != 0 || D <= 0 || D % 2 != 0 || L <= 0)
    return fail(PMI_ERR_INVALID, "%s: bad shape (B=%lld T=%lld H=%lld KV=%lld D=%lld L=%lld)", fn,
                (long long)B, (long long)T, (long long)H, (long long)KV, (long long)D, (long long)L);
  if (B == 0) return ok();
  if (!qkv || !cos_t || !sin_t || !pos || !q_out || !cache_k || !cache_v)
    return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (B * T * (H + 2 * KV) * D >= (1ll << 31) || B * KV * L * D >= (1ll << 31))
    return fail(PMI_ERR_UNSUPPORTED, "%s: shape too large", fn);
  return from_hip(pmi::launch_rope_kv(qkv, cos_t, sin_t, pos, q_out, cache_k, cache_v, B, T, H,
                                      KV, D, L, (hipStream_t)stream), fn);
}

size_t pmi_decode_attention_workspace_bytes(int64_t B, int64_t H, int64_t KV, int64_t L) {
  if (B <= 0 || H <= 0 || KV <= 0 || L <= 0) return 0;
  return pmi::decode_attention_ws_bytes(B, H, KV, L);
}

int pmi_decode_attention_f16(const void* q, const void* cache_k, const void* cache_v,
                             const int64_t* pos, void* out, int64_t B, int64_t H, int64_t KV,
                             int64_t D, int64_t L, float scale, void* workspace,
                             size_t workspace_bytes, void* stream) {
  const char* fn = "pmi_decode_attention_f16";
  if (B < 0 || H <= 0 || KV <= 0 || H % KV != 0 || L <= 0)
    return fail(PMI_ERR_INVALID, "%s: bad shape", fn);
  if (D != 128 || H / KV > 4)
    return fail(PMI_ERR_UNSUPPORTED, "%s: needs head_dim 128 and at most 4 query heads per KV head",
                fn);
  const size_t need = pmi::decode_attention_ws_bytes(B, H, KV, L);  // 0: B * KV too large
  const bool split = workspace && need && workspace_bytes >= need;
  if (split && !aligned(workspace, 256))
    return fail(PMI_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  if (split && need >= (1ull << 31))
    return fail(PMI_ERR_UNSUPPORTED, "%s: workspace partials exceed 2 GiB", fn);
  const int64_t group = H / KV, span = (L + 3) / 4;
  if (!split && (group * 4 * span + group * 4 * (2 + D)) * 4 > 64 * 1024)
    return fail(PMI_ERR_UNSUPPORTED,
                "%s: cache length %lld needs the split kernel (pass a workspace of "
                "pmi_decode_attention_workspace_bytes)", fn, (long long)L);
  if (B == 0) return ok();
  if (!q || !cache_k || !cache_v || !pos || !out) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(q, 16) || !aligned(cache_k, 16) || !aligned(cache_v, 16) || !aligned(out, 4))
    return fail(PMI_ERR_INVALID, "%s: q and the caches must be 16-byte aligned", fn);
  if (B * KV * L * D >= (1ll << 31)) return fail(PMI_ERR_UNSUPPORTED, "%s: cache too large", fn);
  return from_hip(pmi::launch_decode_attention(q, cache_k, cache_v, pos, out, B, H, KV, L, scale,
                                               split ? workspace : nullptr, workspace_bytes,
                                               (hipStream_t)stream), fn);
}

int pmi_decode_attention_rope_f16(const void* qkv, const float* cos, const float* sin,
                                  const int64_t* pos, void* cache_k, void* cache_v, void* out,
                                  int64_t B, int64_t H, int64_t KV, int64_t D, int64_t L,
                                  float scale, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  const char* fn = "pmi_decode_attention_rope_f16";
  if (B < 0 || H <= 0 || KV <= 0 || H % KV != 0 || L <= 0)
    return fail(PMI_ERR_INVALID, "%s: bad shape", fn);
  if (D != 128 || H / KV > 4)
    return fail(PMI_ERR_UNSUPPORTED, "%s: needs head_dim 128 and at most 4 query heads per KV head",
                fn);
  const size_t need = pmi::decode_attention_ws_bytes(B, H, KV, L);
  if (!need)
    return fail(PMI_ERR_UNSUPPORTED, "%s: B * KV = %lld exceeds the %lld split counters", fn,
                (long long)(B * KV), (long long)pmi::kOpsMaxCounters);
  if (!workspace || workspace_bytes < need)
    return fail(PMI_ERR_INVALID, "%s: needs a workspace of pmi_decode_attention_workspace_bytes "
                "(%zu) bytes", fn, need);
  if (!aligned(workspace, 256)) return fail(PMI_ERR_INVALID, "%s: workspace must be 256-byte aligned", fn);
  if (need >= (1ull << 31)) return fail(PMI_ERR_UNSUPPORTED, "%s: workspace partials exceed 2 GiB", fn);
  if (B == 0) return ok();
  if (!qkv || !cos || !sin || !pos || !cache_k || !cache_v || !out)
    return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(cache_k, 16) || !aligned(cache_v, 16) || !aligned(out, 4) || !aligned(qkv, 2) ||
      !aligned(cos, 4) || !aligned(sin, 4))
    return fail(PMI_ERR_INVALID, "%s: the caches must be 16-byte aligned", fn);
  if (B * KV * L * D >= (1ll << 31)) return fail(PMI_ERR_UNSUPPORTED, "%s: cache too large", fn);
  return from_hip(pmi::launch_decode_attention(qkv, cache_k, cache_v, pos, out, B, H, KV, L, scale,
                                               workspace, workspace_bytes, (hipStream_t)stream,
                                               cos, sin),
                  fn);
}

size_t pmi_argmax_workspace_bytes(int64_t rows, int64_t n) {
  if (rows <= 0 || n <= 0) return 0;
  return pmi::argmax_ws_bytes(rows, n);
}

int pmi_argmax_f16(const void* x, int64_t rows, int64_t n, int64_t* out, int64_t out_stride,
                   void* workspace, size_t workspace_bytes, void* stream) {
  const char* fn = "pmi_argmax_f16";
  if (rows < 0 || n <= 0 || n % 8 != 0 || n >= (1ll << 31) || out_stride < 1)
    return fail(PMI_ERR_INVALID, "%s: need rows >= 0, 0 < n < 2^31 with n %% 8 == 0, out_stride >= 1",
                fn);
  if (rows == 0) return ok();
  if (rows > pmi::kOpsMaxCounters)
    return fail(PMI_ERR_UNSUPPORTED, "%s: at most %lld rows", fn, (long long)pmi::kOpsMaxCounters);
  const size_t need = pmi::argmax_ws_bytes(rows, n);
  if (!workspace || workspace_bytes < need)
    return fail(PMI_ERR_INVALID, "%s: needs a zero-filled workspace of pmi_argmax_workspace_bytes "
                "(%zu) bytes", fn, need);
  if (!x || !out) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(x, 16) || !aligned(out, 8) || !aligned(workspace, 256))
    return fail(PMI_ERR_INVALID, "%s: x 16-byte, out 8-byte and workspace 256-byte aligned", fn);
  return from_hip(pmi::launch_argmax(x, rows, n, out, out_stride, workspace, (hipStream_t)stream),
                  fn);
}

int pmi_read_probe(const void* buf, int64_t bytes, int64_t grid, uint32_t* sink, void* stream) {
  const char* fn = "pmi_read_probe";
  if (bytes < 0 || bytes % 16 != 0 || grid <= 0 || grid > (1 << 20))
    return fail(PMI_ERR_INVALID, "%s: need bytes %% 16 == 0 and 0 < grid <= 2^20", fn);
  if (bytes == 0) return ok();
  if (!buf || !sink) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(buf, 16) || !aligned(sink, 4)) return fail(PMI_ERR_INVALID, "%s: misaligned", fn);
  return from_hip(pmi::launch_read_probe(buf, bytes, grid, sink, (hipStream_t)stream), fn);
}

int pmi_silu_mul_f16(const void* gate_up, void* out, int64_t rows, int64_t F, void* stream) {
  const char* fn = "pmi_silu_mul_f16";
  if (rows < 0 || F <= 0 || F % 8 != 0)
    return fail(PMI_ERR_INVALID, "%s: need F > 0, F %% 8 == 0", fn);
  if (rows == 0) return ok();
  if (!gate_up || !out) return fail(PMI_ERR_INVALID, "%s: null buffer", fn);
  if (!aligned(gate_up, 16) || !aligned(out, 16))
    return fail(PMI_ERR_INVALID, "%s: buffers must be 16-byte aligned", fn);
  if (rows * F * 2 >= (1ll << 31)) return fail(PMI_ERR_UNSUPPORTED, "%s: too large", fn);
  return from_hip(pmi::launch_silu_mul(gate_up, out, rows, F, (hipStream_t)stream), fn);
}

}  // extern "C"
