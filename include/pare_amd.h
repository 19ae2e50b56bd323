/*
 * pare_amd.h — C ABI of the MI355X (gfx950) INT4 W4A16 dequant-matmul library
 * (libpare_amd.so).
 *
 * This library is a drop-in for the kernel path of Pare's QuantizedLinear
 * (use_kernel=True). Every entry point below names the reference interface it
 * replaces, as /root/reference file:line.
 *
 * Conventions shared by all entry points
 *  - Pointers are device pointers (HIP), except where noted. Shapes are int64.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream). All
 *    work is enqueued asynchronously on it; nothing synchronises the host.
 *  - Return value: PMI_OK (0) or a negative PMI_ERR_* code. On error a
 *    message is available from pmi_last_error() (thread-local). Argument
 *    validation happens on the host before anything is launched, so an
 *    invalid call has no device side effects.
 *  - No entry point allocates device memory.
 *
 * Data layouts (identical to the reference buffers)
 *  - packed "storage" layout, u8 [N, K/2]: byte b of row n holds
 *    q[n,2b] in bits 0-3 and q[n,2b+1] in bits 4-7      (pare/core/pack.py:29-48)
 *  - packed "kernel" layout, u8 [N, K/2]: inside every group_size-wide tile
 *    starting at column k0, byte j (0 <= j < gs/2) holds q[n,k0+j] in bits 0-3
 *    and q[n,k0+gs/2+j] in bits 4-7                      (pare/core/pack.py:88-132)
 *  - scales fp32 [N, G] with G = K / group_size            (pare/kernels/matmul_int4.py:219-228)
 *  - zeros  fp32 [N, G] (integer values in [0,15]) or u8 [N, G]
 *  - Dequantisation: w = (float(q) - zero) * scale in fp32  (pare/core/functional.py:78-91)
 */
#ifndef PARE_AMD_H
#define PARE_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PMI_ABI_VERSION 16

#if defined(__GNUC__)
#define PMI_API __attribute__((visibility("default")))
#else
#define PMI_API
#endif

/* status codes */
#define PMI_OK               0
#define PMI_ERR_INVALID     -1 /* bad argument (shape, dtype, alignment, null pointer) */
#define PMI_ERR_UNSUPPORTED -2 /* well-formed but outside what the kernels implement   */
#define PMI_ERR_HIP         -3 /* the HIP runtime reported an error                     */
#define PMI_ERR_NO_DEVICE   -4 /* no usable gfx950 device                               */

/* element types */
#define PMI_F16  0
#define PMI_BF16 1
#define PMI_F32  2
#define PMI_U8   3

/* packed weight layouts */
#define PMI_LAYOUT_STORAGE 0 /* pack_int4 order            */
#define PMI_LAYOUT_KERNEL  1 /* repack_int4_for_kernel order */

/* Library version (PMI_ABI_VERSION). No reference counterpart. */
PMI_API int pmi_abi_version(void);

/* Message of the last error on the calling thread ("" if none). Host-only. */
PMI_API const char* pmi_last_error(void);

/* 1 if `device` exists and is a gfx950 GPU, 0 if not, PMI_ERR_NO_DEVICE when
 * no HIP device is present at all.
 * Replaces: triton_available()                 pare/kernels/matmul_int4.py:246-248 */
PMI_API int pmi_device_supported(int device);

/* Storage layout -> kernel layout, one device pass.
 * perm (nullable, int32 [K], a permutation of 0..K-1): when given, the
 * output holds the columns in the order q[:, perm[0]], q[:, perm[1]], ...
 * before the kernel-layout repack (used for act_order / g_idx layers).
 * Requires K % group_size == 0, group_size % 32 == 0.
 * Replaces: repack_int4_for_kernel(packed, group_size)  pare/core/pack.py:88-132 */
PMI_API int pmi_repack_int4_for_kernel(const uint8_t* packed, uint8_t* out, const int32_t* perm,
                               int64_t N, int64_t K, int64_t group_size, void* stream);

/* fp32 zero points -> u8. Values must be integers in [0,15]; the number of
 * elements that are not is added to *bad_count (device int32, nullable).
 * Replaces: the per-call zeros.float() of _to_2d   pare/kernels/matmul_int4.py:219-228 */
PMI_API int pmi_zeros_to_u8(const float* zeros, uint8_t* zeros_u8, int32_t* bad_count,
                    int64_t count, void* stream);

/* act_order permutation int32 [K] -> its 16-bit copy perm16 uint16 [K]
 * (16-byte aligned, K <= 65536), for pmi_matmul_w4a16's perm16 argument.
 * Entries outside [0, K) become 0, as the kernels clamp them at use; their
 * number is added to *bad_count (device int32, nullable). Built once per layer.
 * No reference counterpart: a derived per-layer copy of the act_order
 * permutation (from g_idx, pare/schemes/gptq.py:196-201,258-261), like the
 * kernel-layout weight the reference caches (pare/layers/linear.py:148-151). */
PMI_API int pmi_perm_u16(const int32_t* perm, uint16_t* perm16, int32_t* bad_count, int64_t K,
                         void* stream);

/* AWQ-GEMM checkpoint tensors -> the buffers above, one device pass each.
 * qweight int32 [K, N/8] and qzeros int32 [G, N/8] hold eight 4-bit codes per
 * word along N: column 8c + order[i] in bits 4i..4i+3 of word c, order =
 * [0,2,4,6,1,3,5,7]; scales fp16 [G, N]. Writes packed (storage layout,
 * u8 [N, K/2], 16-byte aligned), scale and zero (fp32 [N, G]; the zeros are
 * the integer codes). Lossless: the AWQ convention is w = (q - z) * s, the
 * same affine form. Requires N % 8 == 0, K % group_size == 0,
 * group_size % 32 == 0 (group_size = K for one group per row).
 * No reference counterpart in this direction: it inverts
 * _pack_awq / _to_awq_linear   pare/model/export_awq.py:37-49,75-94, so an
 * AWQ-GEMM checkpoint (the format vLLM and AutoAWQ load) runs on this path. */
PMI_API int pmi_awq_gemm_to_storage(const int32_t* qweight, const int32_t* qzeros,
                                    const void* scales, uint8_t* packed, float* scale, float* zero,
                                    int64_t N, int64_t K, int64_t group_size, void* stream);

/* The reverse: storage layout + scale fp32 [N,G] + zero (PMI_F32 or PMI_U8
 * [N,G]) -> qweight, qzeros (int32, AWQ order) and scales fp16 [G, N] (round to
 * nearest even). fp32 zeros are rounded half-to-even first, as the reference
 * does; a zero outside [0,15] after rounding is added to *bad_count (device
 * int32, nullable) and packed as 0 (the reference's shift would spill it
 * into the neighbouring nibble). Same shape rules as above.
 * Replaces: _to_awq_linear (qweight, qzeros, scales)   pare/model/export_awq.py:75-94 */
PMI_API int pmi_storage_to_awq_gemm(const uint8_t* packed, const float* scale, const void* zero,
                                    int zero_dtype, int32_t* qweight, int32_t* qzeros,
                                    void* scales, int32_t* bad_count, int64_t N, int64_t K,
                                    int64_t group_size, void* stream);

/* [N,G] scales (fp32) and zero points (PMI_F32 or PMI_U8) -> group-major
 * copies scales_gm fp32 [G,N] and zeros_gm u8 [G,N], for pmi_matmul_w4a16.
 * Zero points must be integers in [0,15]; the number that are not is added
 * to *bad_count (device int32, nullable) and they are written as 0.
 * No reference counterpart: a derived, per-layer layout like the kernel-layout
 * weight of pare/layers/linear.py:148-151 (the reference kernel reads [N,G]
 * per program, pare/kernels/matmul_int4.py:145-164). */
PMI_API int pmi_sz_group_major(const float* scales, const void* zeros, int zero_dtype,
                               float* scales_gm, uint8_t* zeros_gm, int32_t* bad_count,
                               int64_t N, int64_t G, void* stream);

/* Bytes of the tiled copy of an [N,K] INT4 weight (64-row panels, N padded to
 * a multiple of 64): ceil(N/64) * 64 * K/2. Host-only. No reference counterpart. */
PMI_API size_t pmi_tiled_bytes(int64_t N, int64_t K);

/* Kernel-layout weight (group size group_size, act_order permutation already
 * applied) -> tiled copy for the tiled-weight GEMM that pmi_matmul_w4a16 runs
 * for 2..64 activation rows: for every 64-row panel p and 128-column unit u
 * one 4 KiB block of 4 tiles x 64 lanes x 16 bytes; lane n + 16h of tile j
 * holds row 64p + 4n + j, and its byte b carries columns 128u + (b < 8 ?
 * 8h + b : 32 + 8h + b - 8) (low nibble) and that + 64 (high nibble); rows
 * past N are zero. w_tiled: pmi_tiled_bytes(N, K) bytes, 16-byte aligned;
 * K % 128 == 0; group_size 32, 64 or a multiple of 128. Built once per layer.
 * No reference counterpart: a derived per-layer layout, like the kernel-layout
 * weight the reference caches (pare/layers/linear.py:148-151), laid out so a
 * wave reads contiguous 1 KiB runs straight into MFMA operands. */
PMI_API int pmi_tile_w4a16(const uint8_t* w_kernel, uint8_t* w_tiled, int64_t N, int64_t K,
                           int64_t group_size, void* stream);

/* Y[M,N] = X[M,K] . dequant(W)^T with the dequantisation fused into the
 * matmul. x: fp16 [M,K] row-major, 16-byte aligned; w: kernel layout;
 * x_dtype and y_dtype: both PMI_F16, or both PMI_BF16 (native bf16
 * activations: an extension with no reference counterpart, where the
 * reference casts bf16 activations to fp16, pare/layers/linear.py:154-156;
 * y rounded to bf16; with w_tiled and no perm, the rows an fp16 call would
 * run on the tiled GEMM's 16-row blocks take its bf16 variant (one K range,
 * group_size % 128 == 0), the rest run on the GEMV, four activation rows per
 * launch, and with perm it needs the workspace for the gather of X[:, perm]);
 * zeros: PMI_F32 or PMI_U8 [N,G]; perm (nullable, int32 [K]): act_order
 * gather, X is read as X[:, perm[j]] for weight column j (w must then be
 * repacked with the same perm); y: fp16 [M,N].
 * perm16 (nullable; only with perm): the pmi_perm_u16 copy of perm (uint16
 * [K], 16-byte aligned, K <= 65536). The GEMV's act_order launches that stage
 * X in LDS, and the tiled GEMM's in-kernel gather (up to 16 rows), read it
 * instead of perm: half the table bytes every workgroup reads before its
 * first gather; same results. Every other kernel reads perm.
 * scales_gm, zeros_gm (nullable, both or neither): the pmi_sz_group_major
 * copies of scales and zeros; the MFMA GEMM reads them (one contiguous run per
 * group) instead of gathering [N,G] rows when N % 4 == 0. The other kernels
 * read scales and zeros.
 * w_tiled (nullable): the pmi_tile_w4a16 copy of w. With it (and scales_gm,
 * zeros_gm) 2..64 activation rows (more on narrow layers) run on the
 * tiled-weight GEMM where that wins (pmi_matmul_kernel_choice 5); without it
 * those rows take the other kernels. The tiled GEMM stores up to 8 bytes per
 * lane: with y not 8-byte aligned (a view at an odd offset) the call runs on
 * the kernel it would pick without w_tiled (an error if the tiled GEMM is
 * forced); y needs only 2-byte alignment otherwise.
 * workspace (nullable when workspace_bytes == 0): device scratch of
 * pmi_matmul_workspace_bytes() bytes, 256-byte aligned, zero-filled before
 * its first use; every call leaves it zero-filled again (it holds split-K
 * counters, partial tiles and the act_order gather of X). A smaller or null
 * workspace is accepted: the GEMM then runs without split-K, and act_order
 * shapes fall back to the GEMV. Calls that may run concurrently (other
 * streams) must not share a workspace.
 * Requires K % group_size == 0, group_size % 32 == 0, K % 32 == 0.
 * Replaces: matmul_w4a16(x, packed_weight, scales, zeros, group_size)
 *           pare/kernels/matmul_int4.py:183-243 (kernel :66-176) */
PMI_API int pmi_matmul_w4a16(const void* x, int x_dtype, const uint8_t* w, const float* scales,
                     const void* zeros, int zero_dtype, const int32_t* perm,
                     const uint16_t* perm16, const float* scales_gm, const uint8_t* zeros_gm, const uint8_t* w_tiled, void* y,
                     int y_dtype, int64_t M, int64_t N, int64_t K, int64_t group_size,
                     void* workspace, size_t workspace_bytes, void* stream);

/* pmi_matmul_w4a16 without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). Same arguments, kernels and results as
 * pmi_matmul_w4a16 given a workspace of pmi_matmul_workspace_bytes() bytes.
 * The scratch is a fixed 16 MiB array the library holds on each GPU it runs
 * on until the process ends (found with hipGetSymbolAddress on the first call
 * on a device, which also clears its counter block: make that first call
 * outside graph capture). Shapes whose pmi_matmul_workspace_bytes() exceeds
 * 16 MiB (large-M act_order layers) fail with PMI_ERR_UNSUPPORTED. Allocates
 * nothing. Every call on one GPU shares that GPU's scratch, so calls that
 * may overlap on one GPU (other streams, other threads) race; calls on one
 * stream are ordered and safe.
 * No reference counterpart: an allocation-free form of
 *           matmul_w4a16  pare/kernels/matmul_int4.py:183-243, for the callers above. */
PMI_API int pmi_matmul_w4a16_noalloc(const void* x, int x_dtype, const uint8_t* w,
                                     const float* scales, const void* zeros, int zero_dtype,
                                     const int32_t* perm, const uint16_t* perm16,
                                     const float* scales_gm,
                                     const uint8_t* zeros_gm, const uint8_t* w_tiled, void* y,
                                     int y_dtype, int64_t M,
                                     int64_t N, int64_t K, int64_t group_size, void* stream);

/* y = (silu(gate) * up) . dequant(W)^T for M <= 4, the down projection of a
 * gated MLP fused with its activation: gate_up is fp16 [M, 2K] (gate in
 * columns 0..K-1, up in K..2K-1, the output of a fused gate/up matmul), and
 * the GEMV forms each activation as pmi_silu_mul_f16 does (silu(gate) rounded
 * to fp16, times up, rounded to fp16), so y equals pmi_silu_mul_f16 followed
 * by pmi_matmul_w4a16 bit for bit. w: kernel layout; zeros PMI_U8 [N,G]; no
 * act_order. Every wave forms its own slice of the activations, so it pays
 * off at M = 1 (one launch less); from M = 2 on the two launches are faster. No reference counterpart: the reference runs SiLU and the
 * product as HuggingFace PyTorch ops before QuantizedLinear
 * (pare/eval/throughput.py:84-126). */
PMI_API int pmi_matmul_w4a16_glu(const void* gate_up, const uint8_t* w, const float* scales,
                                 const void* zeros, int zero_dtype, void* y, int64_t M, int64_t N,
                                 int64_t K, int64_t group_size, void* stream);

/* y = silu(x . dequant(Wg)^T) * (x . dequant(Wu)^T), the fused gate/up
 * projection of a gated MLP with its activation in the epilogue (one launch
 * instead of the matmul and pmi_silu_mul_f16). x: fp16 [M, K]; y: fp16
 * [M, N / 2], each element formed as pmi_silu_mul_f16 forms it from the fp16
 * gate and up outputs, so y equals pmi_matmul_w4a16 on the fused [Wg; Wu]
 * followed by pmi_silu_mul_f16 bit for bit. w_tiled, scales_gm, zeros_gm:
 * the pmi_tile_w4a16 and pmi_sz_group_major copies of the fused weight with
 * its rows interleaved in fours: row 64p + 4n + j holds gate row 32p + 2n + j
 * for j < 2 and up row 32p + 2n + j - 2 for j >= 2 (p < N / 64, n < 16).
 * For the shapes pmi_gate_up_silu_supported accepts (the tiled GEMM with four
 * 16-row tiles per workgroup: M <= 16, N % 64 == 0; no act_order), else
 * PMI_ERR_UNSUPPORTED. No reference counterpart: the reference runs SiLU and
 * the product as HuggingFace PyTorch ops after QuantizedLinear
 * (pare/eval/throughput.py:84-126). */
PMI_API int pmi_matmul_w4a16_gate_up_silu(const void* x, const uint8_t* w_tiled,
                                          const float* scales_gm, const uint8_t* zeros_gm,
                                          void* y, int64_t M, int64_t N, int64_t K,
                                          int64_t group_size, void* stream);

/* 1 when pmi_matmul_w4a16_gate_up_silu runs this shape, else 0. Host-only. */
PMI_API int pmi_gate_up_silu_supported(int64_t M, int64_t N, int64_t K, int64_t group_size);

/* y = (RMSNorm(x + residual) * norm_weight) . dequant(W)^T for M <= 4: a
 * decoder's residual add and pre-norm fused into the GEMV that consumes them.
 * x, residual (nullable), h_out: fp16 [M, K]; norm_weight fp16 [K]. With a
 * residual, h = x + residual (fp16) is written to h_out. Each activation is
 * formed as pmi_add_rmsnorm_f16 forms it (h rounded to fp16; y = h *
 * rsqrt(mean(h^2) + eps) * w rounded to fp16); the mean is summed in another
 * order, so activations can differ from pmi_add_rmsnorm_f16 by one fp16 ulp.
 * w: kernel layout; zeros PMI_U8 [N,G]; no act_order. Every wave forms the
 * norm for its rows after one workgroup barrier; it pays off at M = 1. No
 * reference counterpart (the reference runs the norm in PyTorch,
 * pare/eval/throughput.py:84-126). */
PMI_API int pmi_matmul_w4a16_rmsnorm(const void* x, const void* residual, const void* norm_weight,
                                     float eps, void* h_out, const uint8_t* w, const float* scales,
                                     const void* zeros, int zero_dtype, void* y, int64_t M,
                                     int64_t N, int64_t K, int64_t group_size, void* stream);

/* The residual add moved into the launch that forms the residual stream, one
 * activation row: h = residual + (x . dequant(W)^T), each element rounded to
 * fp16 and then added as pmi_add_rmsnorm_f16 adds (h may alias residual);
 * with glu != 0, x is the fused gate/up output [1, 2K] consumed as
 * SiLU(gate) * up (as pmi_matmul_w4a16_glu). stats[g] receives workgroup g's
 * sum of h^2 over its rows, pmi_residual_stats_count(N, K, glu) floats, for a
 * following pmi_matmul_w4a16_prenormed. zeros u8 [N, G], kernel layout, no
 * act_order. PMI_ERR_UNSUPPORTED where the count is 0 (rows of one GEMV
 * slice, K <= 2048). No reference counterpart (the reference adds the
 * residual in PyTorch, pare/eval/throughput.py:84-126). */
PMI_API int pmi_matmul_w4a16_residual(const void* x, int glu, const void* residual, float* stats,
                                      const uint8_t* w, const float* scales,
                                      const uint8_t* zeros_u8, void* h, int64_t N, int64_t K,
                                      int64_t group_size, void* stream);

/* Number of stats floats pmi_matmul_w4a16_residual writes for this shape, 0
 * when it does not run it. Host-only. */
PMI_API int pmi_residual_stats_count(int64_t N, int64_t K, int glu);

/* y = (RMSNorm(x) * norm_weight) . dequant(W)^T for one activation row x
 * fp16 [1, K] that a pmi_matmul_w4a16_residual launch formed, with its n_stats
 * partial sums of x^2 (1 <= n_stats <= 512): every wave adds them in one fixed
 * order, so the launch needs no whole-row reduction or barrier before its
 * first weight batch. The activations are formed as pmi_add_rmsnorm_f16 forms
 * them; the mean's sum runs in another order, so an activation can differ by
 * one fp16 ulp. norm_weight fp16 [K]; zeros u8 [N, G]; kernel layout; no
 * act_order. No reference counterpart (pare/eval/throughput.py:84-126). */
PMI_API int pmi_matmul_w4a16_prenormed(const void* x, const float* stats, int n_stats,
                                       const void* norm_weight, float eps, const uint8_t* w,
                                       const float* scales, const uint8_t* zeros_u8, void* y,
                                       int64_t N, int64_t K, int64_t group_size, void* stream);

/* The same residual add and pre-norm on the tiled GEMM, for up to 4 rows:
 * y = (RMSNorm(x + residual) * norm_weight) . dequant(W)^T, or with glu != 0
 * (the gate/up layout of pmi_matmul_w4a16_gate_up_silu) y = SiLU(gate) * up of
 * it, [M, N/2]. x, residual (nullable), h_out: fp16 [M, K]; norm_weight fp16
 * [K]; w_tiled / scales_gm / zeros_gm as for pmi_matmul_w4a16's tiled GEMM.
 * Every workgroup forms the normalised rows in LDS once, before its first
 * weight batch, with the rounding and the summation order of
 * pmi_add_rmsnorm_f16, so y equals pmi_add_rmsnorm_f16 followed by the
 * matmul (or the gate/up launch) bit for bit; workgroup 0 writes h = x +
 * residual to h_out. For the shapes pmi_tiled_rmsnorm_supported accepts (M <=
 * 4, K <= 4096, group_size % 128 == 0, one 16-row activation block), else
 * PMI_ERR_UNSUPPORTED. No reference counterpart (the reference runs the norm
 * in PyTorch, pare/eval/throughput.py:84-126). */
PMI_API int pmi_matmul_w4a16_tiled_rmsnorm(const void* x, const void* residual,
                                           const void* norm_weight, float eps, void* h_out,
                                           const uint8_t* w_tiled, const float* scales_gm,
                                           const uint8_t* zeros_gm, void* y, int64_t M,
                                           int64_t N, int64_t K, int64_t group_size, int glu,
                                           void* stream);

/* 1 when pmi_matmul_w4a16_tiled_rmsnorm runs this shape, else 0. Host-only. */
PMI_API int pmi_tiled_rmsnorm_supported(int64_t M, int64_t N, int64_t K, int64_t group_size,
                                        int glu);

/* Workspace bytes pmi_matmul_w4a16 uses at full speed for this shape (0 when
 * the chosen kernel needs none). Host-only. No reference counterpart: the
 * Triton kernel allocates nothing besides Y (pare/kernels/matmul_int4.py:230). */
PMI_API size_t pmi_matmul_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t group_size,
                                  int has_perm);

/* Full dequantised weight W_hat[N,K] in the original column order, cast to
 * out_dtype (PMI_F16 / PMI_BF16 with round-to-nearest-even, or PMI_F32).
 * layout PMI_LAYOUT_STORAGE: idx (nullable) is g_idx int32 [K], the group of
 *   each column (default k / group_size).
 * layout PMI_LAYOUT_KERNEL: idx (nullable) is the perm given to
 *   pmi_repack_int4_for_kernel.
 * Replaces: QuantizedLinear.dequantize().to(dtype)   pare/layers/linear.py:101-118,129
 *           (unpack_int4 pare/core/pack.py:51-67, dequantize_tensor
 *            pare/core/functional.py:78-91) */
PMI_API int pmi_dequant_w4a16(const uint8_t* w, int layout, const float* scales, const void* zeros,
                      int zero_dtype, const int32_t* idx, void* w_out, int out_dtype,
                      int64_t N, int64_t K, int64_t group_size, void* stream);

/* RTN INT4 quantisation of W[N,K] (fp32, fp16 or bf16) with per-group
 * min/max scales: writes packed (storage layout, u8 [N,K/2]), scale and zero
 * (fp32 [N, K/group_size]). sym=0: asymmetric; sym=1: the reference's
 * symmetric rule on the unsigned grid (zero 0: negative weights clamp to code
 * 0); sym=2: offset-8 symmetric (zero 8, scale = 2 max|w| / 15, no reference
 * counterpart). Use group_size = K for per-channel.
 * Replaces: compute_scale(..., per_group) + quantize_tensor + pack_int4
 *           pare/core/scale.py:24-137, pare/core/functional.py:46-75,
 *           pare/core/pack.py:29-48, as called by pare/schemes/rtn.py:46-65 */
PMI_API int pmi_rtn_quantize(const void* w, int w_dtype, uint8_t* packed, float* scale, float* zero,
                     int64_t N, int64_t K, int64_t group_size, int sym, void* stream);

/* ---- GPTQ producer ---------------------------------------------------------
 * The device half of one GPTQ layer (pare/schemes/gptq.py:156-263). The host
 * computes the upper Cholesky factor C of the damped (and, with act_order,
 * permuted) inverse Hessian, calls pmi_gptq_block once per 128-column block
 * and applies the lazy update W[:, b0+count:] -= E^T C[b0:b0+count, b0+count:]
 * with a GEMM between blocks, then packs with pmi_gptq_pack. */

/* scale[n*G + g], zero[n*G + g] for every row n from w[n*ldw + col0 ..
 * col0 + cols - 1] (fp32), with the min/max rule of pmi_rtn_quantize (sym 0,
 * 1 or 2). Used for groups formed in processing order (act_order with g_idx,
 * AutoGPTQ desc_act), whose scale comes from the partly updated W.
 * Replaces: compute_scale on one group   pare/core/scale.py:24-137 */
PMI_API int pmi_gptq_group_params(const float* w, int64_t ldw, int64_t N, int64_t col0,
                                  int64_t cols, int sym, float* scale, float* zero, int64_t G,
                                  int64_t g, void* stream);

/* The column loop of one block, columns b0 .. b0 + count - 1 of w (fp32
 * [N, K], row-major, 16-byte aligned; w is read, not written). For each
 * column j in order: q = clamp(rint(w / s + z), 0, 15) with s, z the
 * scale/zero [N, G] of group colg[j] (int32 [K]; values are clamped into
 * [0, G)); e = (w - (q - z) s) / C[j, j]; then w[:, j'] -= e * C[j, j'] for
 * every later column j' of the block, one column at a time. c: fp32 [K, K]
 * row-major. Writes codes[j*N + n] (u8, column-major [K, N]) and errors[(j-b0)*N
 * + n] (fp32 [count, N]). b0 and count are multiples of 16, count <= 128.
 * Replaces: the loop of _gptq_one_layer   pare/schemes/gptq.py:218-249 */
PMI_API int pmi_gptq_block(const float* w, const float* c, const int32_t* colg,
                           const float* scale, const float* zero, uint8_t* codes, float* errors,
                           int64_t N, int64_t K, int64_t G, int64_t b0, int64_t count,
                           void* stream);

/* codes (u8 [K, N], processed column order) -> packed (storage layout
 * u8 [N, K/2], original column order): column k was processed at step
 * inv_perm[k] (int32 [K], nullable = identity; out-of-range entries read
 * step k). K % 8 == 0.
 * Replaces: Q_int[:, invperm] + pack_int4   pare/schemes/gptq.py:258-261,
 *           pare/core/pack.py:29-48 */
PMI_API int pmi_gptq_pack(const uint8_t* codes, const int32_t* inv_perm, uint8_t* packed,
                          int64_t N, int64_t K, void* stream);

/* Flags of pmi_matmul_kernel_choice: the call passes the tiled copy (with
 * scales_gm and zeros_gm), and an act_order perm. */
#define PMI_CHOICE_TILED 1
#define PMI_CHOICE_PERM  2

/* Which kernel pmi_matmul_w4a16 would run for this shape: 1 = split-K GEMV,
 * 2 = MFMA GEMM (group_size % 128 == 0 and K % 256 == 0), 3 = skinny MFMA
 * kernel (M <= 16), 4 = register-streamed MFMA GEMM (group_size == 128,
 * K % 512 == 0), 5 = tiled-weight MFMA GEMM (K % 512 == 0, K >= 1536,
 * N % 4 == 0, group_size 32, 64 or a multiple of 128; needs the w_tiled copy,
 * so it is chosen only with PMI_CHOICE_TILED in flags; with PMI_CHOICE_PERM
 * as well, up to 16 rows it gathers X[:, perm] itself when M (2K + 16) + 4K
 * bytes fit its LDS, which widens where it wins), 6 = the tiled GEMM's
 * big-tile variant (same buffers; many activation rows, group_size % 128 ==
 * 0: 256 weight rows x 128 activation rows per workgroup, B formed as
 * fp16((q - z) * s) as the reference dequantises; with PMI_CHOICE_PERM
 * X[:, perm] is gathered into the workspace first). flags 0 and 1 keep the
 * meaning of the former has_tiled argument. Host-only; no reference
 * counterpart (the reference has one Triton kernel). */
PMI_API int pmi_matmul_kernel_choice(int64_t M, int64_t N, int64_t K, int64_t group_size,
                                     int flags);

/* The K ranges the tiled-weight GEMM (kernel 5) splits this shape into when
 * the call has a workspace of pmi_matmul_workspace_bytes() bytes. Up to 16
 * rows: four ranges where its one-tile workgroups fill at most a quarter of
 * the CUs (narrow layers), and four ranges over four-tile workgroups for
 * K > 8192 (and at 13-16 rows for N <= 4096 without act_order). Each range
 * runs on its own workgroup; the last to finish adds the fp32 partial tiles
 * in range order. 1 = unsplit (always without a workspace). has_perm: an
 * act_order perm. Host-only diagnostic; no reference counterpart. */
PMI_API int pmi_tgemm_splits(int64_t M, int64_t N, int64_t K, int64_t group_size, int has_perm);

/* Forces pmi_matmul_w4a16 onto one kernel (1 to 6 as above; 0 restores the
 * automatic choice) for every thread of the process; returns the previous
 * setting, or PMI_ERR_INVALID for an unknown value. A test and benchmarking
 * hook with no reference counterpart. A forced kernel that cannot run a shape
 * makes pmi_matmul_w4a16 return PMI_ERR_UNSUPPORTED. */
PMI_API int pmi_set_kernel_override(int kernel);

/* ---- Caller-side fp16 ops of the end-to-end decoder ----------------------
 * The model around the INT4 linears, one launch each. No reference
 * counterpart: the reference runs these parts of the model as HuggingFace
 * PyTorch ops (pare/eval/throughput.py:84-126 times HF generate). fp32
 * arithmetic inside; buffers 16-byte aligned. */

/* h = x (+ residual); residual_out = h (residual and residual_out both or
 * neither); y = h * rsqrt(mean(h^2) + eps) * weight. x, y [rows, dim] fp16,
 * weight [dim] fp16; dim % 8 == 0, dim <= 8192. */
PMI_API int pmi_add_rmsnorm_f16(const void* x, const void* residual, const void* weight, void* y,
                                void* residual_out, int64_t rows, int64_t dim, float eps,
                                void* stream);

/* RoPE (rotate_half on the two halves of the head dim) and the KV-cache
 * write. qkv [B*T, (H + 2*KV)*D] fp16 (fused q/k/v rows), cos/sin fp32
 * [L, D/2], pos int64 [T] (device) cache positions of the T tokens; writes
 * q_out [B, H, T, D] rotated and the rotated k and the v into cache_k,
 * cache_v [B, KV, L, D]. */
PMI_API int pmi_rope_kv_f16(const void* qkv, const float* cos, const float* sin, const int64_t* pos,
                            void* q_out, void* cache_k, void* cache_v, int64_t B, int64_t T,
                            int64_t H, int64_t KV, int64_t D, int64_t L, void* stream);

/* One-token grouped-query attention over cache positions 0..*pos (device
 * int64): out[b, h] = softmax(q[b, h] . k^T * scale) v with KV head h/(H/KV).
 * q, out [B, H, 128] fp16; caches [B, KV, L, 128] fp16; H/KV <= 4.
 * workspace (nullable): device scratch of
 * pmi_decode_attention_workspace_bytes(B, H, KV, L) bytes, 256-byte aligned
 * and zero-filled before its first use (each call leaves its counters at
 * zero). With it the positions are split over workgroups of 64 positions
 * each, combined by the last workgroup of each (b, KV head) in split order;
 * without it (or when smaller) one workgroup per (b, KV head) runs, for
 * L up to about 3000. The workspace starts with a fixed 16 KiB block of
 * counters (one per (b, KV head), so the split needs B * KV <= 4096) that no
 * shape's partials overlap: one workspace may serve calls of any shapes in
 * turn. Calls that may run concurrently must not share a workspace. */
PMI_API int pmi_decode_attention_f16(const void* q, const void* cache_k, const void* cache_v,
                                     const int64_t* pos, void* out, int64_t B, int64_t H,
                                     int64_t KV, int64_t D, int64_t L, float scale,
                                     void* workspace, size_t workspace_bytes, void* stream);

/* pmi_rope_kv_f16 and pmi_decode_attention_f16 of one new token in one
 * launch: qkv [B, (H + 2*KV)*128] fp16 is the token's fused q/k/v row, cos/sin
 * fp32 [L, 64] the RoPE tables, *pos (device int64) its cache position. Writes
 * the rotated k and the v into cache_k / cache_v at *pos and out [B, H, 128]
 * = the attention of the rotated q over positions 0..*pos, equal to the two
 * separate calls bit for bit. Needs the workspace of
 * pmi_decode_attention_workspace_bytes (same rules). No reference counterpart. */
PMI_API int pmi_decode_attention_rope_f16(const void* qkv, const float* cos, const float* sin,
                                          const int64_t* pos, void* cache_k, void* cache_v,
                                          void* out, int64_t B, int64_t H, int64_t KV, int64_t D,
                                          int64_t L, float scale, void* workspace,
                                          size_t workspace_bytes, void* stream);

/* Workspace bytes of the split pmi_decode_attention_f16 (0 for bad shapes and
 * for B * KV > 4096, where the split is unavailable). Host-only. */
PMI_API size_t pmi_decode_attention_workspace_bytes(int64_t B, int64_t H, int64_t KV, int64_t L);

/* Greedy decoding's argmax: out[r * out_stride] (int64) = index of the largest
 * value of x[r, 0:n] (fp16, rows 16-byte aligned, n % 8 == 0), the first one
 * on ties, NaN counted as largest (torch.argmax's rule). workspace: device
 * scratch of pmi_argmax_workspace_bytes(rows, n) bytes, 256-byte aligned and
 * zero-filled before its first use; each call leaves it zero-filled again.
 * It starts with the same fixed 16 KiB counter block (one per row, rows <=
 * 4096), so one workspace may serve calls of any shapes in turn. Calls that
 * may run concurrently must not share it. */
PMI_API int pmi_argmax_f16(const void* x, int64_t rows, int64_t n, int64_t* out,
                           int64_t out_stride, void* workspace, size_t workspace_bytes,
                           void* stream);
PMI_API size_t pmi_argmax_workspace_bytes(int64_t rows, int64_t n);

/* out[r, c] = silu(gate_up[r, c]) * gate_up[r, F + c]; gate_up [rows, 2F],
 * out [rows, F] fp16; F % 8 == 0. */
PMI_API int pmi_silu_mul_f16(const void* gate_up, void* out, int64_t rows, int64_t F, void* stream);

/* ---- Measurement hook ------------------------------------------------------
 * Reads `bytes` (a multiple of 16) of device memory at `buf` once, with at most
 * `grid` workgroups of 8 waves (the GEMV's workgroup shape) each streaming one
 * contiguous range in 16-byte loads, and
 * computes nothing from it: the read floor that a kernel reading the same bytes
 * on the same grid can reach. sink: device uint32 [grid] (never written in
 * practice; it keeps the loads live). No reference counterpart. */
PMI_API int pmi_read_probe(const void* buf, int64_t bytes, int64_t grid, uint32_t* sink,
                           void* stream);

#ifdef __cplusplus
}
#endif
#endif /* PARE_AMD_H */
