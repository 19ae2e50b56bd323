// Host-side launchers shared between the kernel sources and the C ABI layer.
// Every launcher assumes its arguments were validated by capi.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pmi {

struct GemvConfig {
  int rows_per_wave;    // U: rows per batch of one wave (x stays in registers)
  int depth;            // D: batches in a wave's register ring (D - 1 in flight)
  int slices_per_wave;  // 1, or 2 when K needs more than 8 slices
  int slice_waves;      // waves that split one row's K range (1 slice = 2048 columns)
  int row_waves;        // waves that take different rows of the same slices
  int n_slices;         // ceil(K / 2048)
  int rows_per_wg;      // contiguous rows owned by one workgroup
  int grid;             // workgroups
  int lds_bytes;        // per-row partials of the slice waves (0 with one slice wave)
};

struct GemmConfig {
  int m_tiles;      // 16-row MFMA activation tiles per workgroup (1, 2 or 4)
  int n_t;          // 16-row weight tiles per compute wave (4: 128-row tiles, 2: 64-row)
  int n_tiles;      // 128-row weight tiles
  int grid_m;       // activation row blocks of 16 * m_tiles
  int splits;       // workgroups sharing one tile's K range
  int grid;         // workgroups
  size_t ws_split;  // workspace bytes for the partial tiles (splits > 1)
  size_t ws_perm;   // workspace bytes for X[:, perm] (act_order)
};

struct TgemmConfig {
  int mt;      // 16-row activation tiles (1: activations in registers, 2: LDS ring)
  int ntw;     // 16-row weight tiles per workgroup (4, 2 or 1; 5 or 6 for ranges)
  bool rng;    // ntw consecutive tiles per workgroup across panels (up to 16 rows)
  int n_wg;    // weight workgroups
  int grid_m;  // activation blocks
  int splits;  // K ranges per weight workgroup (up to 16 rows on narrow layers), else 1
  int grid;    // workgroups
  size_t ws_split;  // workspace bytes of the split-K partial tiles (0 unsplit)
};

struct SkinnyConfig {
  int k_waves;         // waves of a workgroup splitting the K groups
  int n_waves;         // waves of a workgroup taking different weight tiles
  int tiles_per_wave;  // 16-row weight tiles per wave (NB)
  int grid;            // workgroups
  size_t lds;          // dynamic LDS bytes
};

// Compute units of the current device (cached; 256 when the query fails).
int device_cu_count();

// xmode: the activation transform (GemvXform::mode). Modes whose per-workgroup
// prologue reads all of X once (4 and 8: act_order staged in LDS, 3: RMSNorm
// over the row) take fewer, larger workgroups on some shapes.
GemvConfig gemv_config(int64_t M, int64_t N, int64_t K, int xmode = 0);
bool skinny_supported(int64_t M, int64_t N, int64_t K, int64_t gs);
SkinnyConfig skinny_config(int64_t M, int64_t N, int64_t K, int64_t gs);

hipError_t launch_skinny(const void* x, const uint8_t* w, const float* scales, const void* zeros,
                         int zero_u8, const int32_t* perm, void* y, int64_t M, int64_t N,
                         int64_t K, int64_t gs, hipStream_t stream);
// The matmul workspace starts with a block of split-K counters that nothing
// else writes (zero between calls); the act_order gather X[:, perm] follows it.
constexpr size_t kWsCounterBytes = 64 * 1024;
inline size_t ws_align(size_t v) { return (v + 255) & ~(size_t)255; }
inline size_t ws_perm_bytes(int64_t M, int64_t K) { return ws_align((size_t)M * K * 2); }

// X[:, perm] -> out (fp16 [M, K], K % 8 == 0), one pass.
hipError_t launch_gather_cols(const void* x, const int32_t* perm, void* out, int64_t M, int64_t K,
                              hipStream_t stream);

// The register-streamed GEMM (blocks of 64 activation rows) runs whole
// 128-column groups; its activation offsets are int32.
inline bool gemm64_supported(int64_t M, int64_t K, int64_t gs) {
  return gs == 128 && K % 128 == 0 && M * K * 2 < (1ll << 31);
}
struct Gemm64Config {
  int n_blocks;     // 128-row weight blocks
  int grid_m;       // 64-row activation blocks
  int splits;       // workgroups sharing one block's K range
  int grid;         // workgroups
  size_t ws_split;  // workspace bytes for the partial tiles (splits > 1)
};
Gemm64Config gemm64_config(int64_t M, int64_t N, int64_t K);
// workspace (nullable): zero-filled counter block first, partial tiles at
// part_offset; too small for them -> unsplit.
hipError_t launch_gemm64(const void* x, const uint8_t* w, const float* scales, const void* zeros,
                         int zero_u8, const float* scales_gm, const uint8_t* zeros_gm, void* y,
                         int64_t M, int64_t N, int64_t K, void* workspace, size_t ws_bytes,
                         size_t part_offset, hipStream_t stream);

// The MFMA GEMM runs whole 128-column groups, consumed two at a time.
inline bool gemm_supported(int64_t K, int64_t gs) { return gs % 128 == 0 && K % 256 == 0; }
GemmConfig gemm_config(int64_t M, int64_t N, int64_t K, int64_t gs, bool has_perm);
size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t gs, bool has_perm);

// Activation transforms of the GEMV (modes 2 and 3: u8 zero points, no perm):
//   mode 2: x is the fused gate/up output [M, 2K], consumed as silu(gate) * up;
//   mode 3: x is the residual stream [M, K], consumed as RMSNorm(x + r) * w
//           (r nullable; h = x + r written to h_out when r is given);
//   mode 5: x is a residual stream, consumed as RMSNorm(x) * w, with sum(x^2)
//           from per-workgroup partials a launch with `res` left;
//   mode 6: x and y bf16 [M, K] / [M, N] (no perm; act_order rows are
//           gathered by the caller first);
//   mode 4: act_order, x[:, perm] gathered from a copy of x staged in LDS by
//           each workgroup (needs gemv_perm_lds_fits), instead of every lane
//           gathering from global memory;
//   mode 8: mode 4 with the 16-bit copy of the permutation: the perm argument
//           then points at uint16 [K] (16-byte aligned, K <= 65536).
constexpr int kGemvLdsChunks = 8;  // 16-byte activation chunks staged per thread (modes 4, 8)
inline bool gemv_perm_lds_fits(int64_t mt, int64_t K, int64_t threads) {
  return K % 8 == 0 && mt * K * 2 <= 64 * 1024 && mt * K / 8 <= kGemvLdsChunks * threads;
}
// Plain activations staged in LDS (mode 7): one 16-byte chunk per thread at
// most, so that a workgroup's start-up issues one load per wave for them.
constexpr int kGemvXLdsChunks = 1;
inline bool gemv_x_lds_fits(int64_t mt, int64_t K, int64_t threads) {
  return K % 8 == 0 && mt * K * 2 <= 64 * 1024 && mt * K / 8 <= kGemvXLdsChunks * threads;
}
// Mode 4 fits every launch of an M-row GEMV (launched four rows at a time).
bool gemv_perm_lds_ok(int64_t M, int64_t N, int64_t K);
struct GemvXform {
  int mode = 0;
  const void* r = nullptr;
  const void* w = nullptr;
  float eps = 0.f;
  void* h_out = nullptr;
  // mode 5: the partial sums of h^2 (n_stats of them, at most kGemvMaxStats)
  // left by the launch that formed x; with res (one row, at least two slice
  // waves): y = y + res, and that launch's partials are written to stats
  const void* res = nullptr;
  float* stats = nullptr;
  int n_stats = 0;
};
constexpr int kGemvMaxStats = 512;
hipError_t launch_gemv(const void* x, const uint8_t* w, const float* scales, const void* zeros,
                       int zero_u8, const int32_t* perm, void* y, int64_t M, int64_t N,
                       int64_t K, int64_t gs, hipStream_t stream,
                       const GemvXform* xform = nullptr);

// workspace: zero-filled before first use, left zeroed; may be smaller than
// gemm_workspace_bytes() (then unsplit) but must hold the counter block and
// ws_perm when perm is set. scales_gm / zeros_gm (nullable): group-major
// copies fp32 [G, N] / u8 [G, N], used when both are given and N % 4 == 0.
hipError_t launch_gemm(const void* x, const uint8_t* w, const float* scales, const void* zeros,
                       int zero_u8, const float* scales_gm, const uint8_t* zeros_gm,
                       const int32_t* perm, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                       void* workspace, size_t ws_bytes, hipStream_t stream);

// [N, G] scales and zero points -> group-major fp32 [G, N] and u8 [G, N]
// (zeros must hold integers in [0, 15]; others are counted into *bad).
hipError_t launch_sz_group_major(const float* scales, const void* zeros, int zero_u8,
                                 float* scales_gm, uint8_t* zeros_gm, int32_t* bad, int64_t N,
                                 int64_t G, hipStream_t stream);

// Caller-side decoder ops (decode_ops.hip).
hipError_t launch_add_rmsnorm(const void* x, const void* r, const void* w, void* y, void* r_out,
                              int64_t rows, int64_t dim, float eps, hipStream_t stream);
hipError_t launch_rope_kv(const void* qkv, const float* cos_t, const float* sin_t,
                          const int64_t* pos, void* q_out, void* cache_k, void* cache_v,
                          int64_t B, int64_t T, int64_t H, int64_t KV, int64_t D, int64_t L,
                          hipStream_t stream);
// Workspaces of the split attention and the argmax start with a fixed block of
// int32 counters (zero between calls) that no shape's partials ever overlap:
// a workspace shared by calls of different shapes keeps every counter of
// every shape at zero. Counter i serves (sequence, KV head) i, or row i.
constexpr size_t kOpsCounterBytes = 16 * 1024;
constexpr int64_t kOpsMaxCounters = kOpsCounterBytes / 4;
// Split attention workspace: the counter block, then the per-split partials.
// 0 when B * KV exceeds the counter block (the split kernel is then unavailable).
size_t decode_attention_ws_bytes(int64_t B, int64_t H, int64_t KV, int64_t L);
// workspace (nullable): too small or null runs the one-workgroup-per-KV-head kernel.
hipError_t launch_decode_attention(const void* q, const void* cache_k, const void* cache_v,
                                   const int64_t* pos, void* out, int64_t B, int64_t H,
                                   int64_t KV, int64_t L, float scale, void* workspace,
                                   size_t ws_bytes, hipStream_t stream,
                                   const float* cos_t = nullptr, const float* sin_t = nullptr);
// Greedy argmax over fp16 rows; workspace: the counter block, then (value,
// index) per (row, chunk). 0 when rows exceed the counter block.
size_t argmax_ws_bytes(int64_t rows, int64_t n);
hipError_t launch_argmax(const void* x, int64_t rows, int64_t n, int64_t* out, int64_t out_stride,
                         void* workspace, hipStream_t stream);
hipError_t launch_silu_mul(const void* gu, void* out, int64_t rows, int64_t F, hipStream_t stream);

hipError_t launch_repack(const uint8_t* packed, uint8_t* out, const int32_t* perm, int64_t N,
                         int64_t K, int64_t gs, hipStream_t stream);

hipError_t launch_zeros_to_u8(const float* zeros, uint8_t* out, int32_t* bad, int64_t count,
                              hipStream_t stream);

// int32 permutation [K] -> uint16 [K] (K <= 65536), entries outside [0, K) as 0.
hipError_t launch_perm_u16(const int32_t* perm, uint16_t* out, int32_t* bad, int64_t K,
                           hipStream_t stream);

// AWQ-GEMM int32 layout <-> storage layout + fp32 [N,G] scales and zeros.
hipError_t launch_awq_to_storage(const int32_t* qweight, const int32_t* qzeros, const void* scales,
                                 uint8_t* packed, float* scale, float* zero, int64_t N, int64_t K,
                                 int64_t gs, hipStream_t stream);
hipError_t launch_storage_to_awq(const uint8_t* packed, const float* scale, const void* zero,
                                 int zero_u8, int32_t* qweight, int32_t* qzeros, void* scales,
                                 int32_t* bad, int64_t N, int64_t K, int64_t gs,
                                 hipStream_t stream);

hipError_t launch_dequant(const uint8_t* w, int layout, const float* scales, const void* zeros,
                          int zero_u8, const int32_t* idx, void* out, int out_dtype, int64_t N,
                          int64_t K, int64_t gs, hipStream_t stream);

// GPTQ producer (gptq.hip).
hipError_t launch_gptq_group_params(const float* w, int64_t ldw, int64_t N, int64_t c0,
                                    int64_t cols, int sym, float* scale, float* zero, int64_t G,
                                    int64_t g, hipStream_t stream);
hipError_t launch_gptq_block(const float* w, const float* c, const int32_t* colg,
                             const float* scale, const float* zero, uint8_t* qt, float* et,
                             int64_t N, int64_t K, int64_t G, int64_t b0, int count,
                             hipStream_t stream);
hipError_t launch_gptq_pack(const uint8_t* qt, const int32_t* inv_perm, uint8_t* packed, int64_t N,
                            int64_t K, hipStream_t stream);

// Streaming read of `bytes` (multiple of 16) over at most `grid` workgroups
// (probes.hip); sink: `grid` uint32 (written only in a case that never occurs).
hipError_t launch_read_probe(const void* buf, int64_t bytes, int64_t grid, uint32_t* sink,
                             hipStream_t stream);

hipError_t launch_rtn(const void* w, int w_dtype, uint8_t* packed, float* scale, float* zero,
                      int64_t N, int64_t K, int64_t gs, int sym, hipStream_t stream);

}  // namespace pmi

namespace pmi {

// ---- tiled weight layout and its GEMM (w4a16_tgemm.hip) ----------------------
// Bytes of the tiled copy of an [N, K] INT4 weight: 64-row panels, N padded.
inline size_t tiled_bytes(int64_t N, int64_t K) { return (size_t)((N + 63) / 64) * 64 * (size_t)(K / 2); }
// kernel layout (group size gs) -> tiled layout
hipError_t launch_tile(const uint8_t* w_kernel, uint8_t* w_tiled, int64_t N, int64_t K, int64_t gs,
                       hipStream_t stream);
bool tgemm_supported(int64_t M, int64_t N, int64_t K, int64_t gs);
// act_order inside the tiled GEMM: X rows and the perm table fit its LDS
constexpr int kTgemmXGLds = 160 * 1024 - 1024;
bool tgemm_gather_supported(int64_t M, int64_t K);
TgemmConfig tgemm_config(int64_t M, int64_t N, int64_t K, int64_t gs, bool gather);
// The big-tile variant of the tiled GEMM (w4a16_bgemm.hip), for many
// activation rows: 256 weight rows (four panels) x 128 activation rows per
// workgroup over all of K, B formed as fp16((q - z) * s); no workspace.
struct BgemmConfig {
  bool ok;      // the shape is within the kernel's limits (gs % 128 == 0, K % 128 == 0)
  int n_bands;  // bands of four 64-row panels
  int grid_m;   // 128-row activation blocks
  int chunk;    // (activation block, band) pairs per XCD
  int grid;     // workgroups (8 chunk)
};
BgemmConfig bgemm_config(int64_t M, int64_t N, int64_t K, int64_t gs);
hipError_t launch_bgemm(const void* x, const uint8_t* w_tiled, const float* scales_gm,
                        const uint8_t* zeros_gm, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                        hipStream_t stream);
// perm: act_order columns, gathered in the kernel (tgemm_gather_supported), or null;
// perm16 (nullable, with perm): its 16-bit copy, which the gather then reads instead.
// workspace: counters (zero between calls) at its start and the split-K partial
// tiles at part_offset; null or too small for them, the kernel runs unsplit.
// bf16: x and y bf16 (tgemm_bf16_supported, no perm; always one K range).
hipError_t launch_tgemm(const void* x, const int32_t* perm, const uint16_t* perm16,
                        const uint8_t* w_tiled, const float* scales_gm, const uint8_t* zeros_gm,
                        void* y, int64_t M, int64_t N, int64_t K, int64_t gs, void* workspace,
                        size_t ws_bytes, size_t part_offset, hipStream_t stream,
                        bool bf16 = false);
bool tgemm_bf16_supported(int64_t M, int64_t N, int64_t K, int64_t gs);
// silu(gate) * up from a fused gate/up weight whose rows are interleaved in
// groups of four (rows 4n + {0, 1} of a 64-row panel p: gate rows 32 p + 2 n +
// {0, 1}; rows 4n + {2, 3}: the matching up rows), y fp16 [M, N / 2]; for the
// shapes the tiled GEMM runs with four tiles per workgroup, no K split
bool tgemm_glu_supported(int64_t M, int64_t N, int64_t K, int64_t gs);
hipError_t launch_tgemm_glu(const void* x, const uint8_t* w_tiled, const float* scales_gm,
                            const uint8_t* zeros_gm, void* y, int64_t M, int64_t N, int64_t K,
                            int64_t gs, hipStream_t stream);
// The residual add + RMSNorm fused into the tiled GEMM's activation load (y =
// (RMSNorm(x + r) * norm_w) . W^T, or its silu(gate) * up with glu), up to 4
// rows, K <= 4096, gs % 128 == 0; h = x + r to h_out when r is given.
bool tgemm_norm_supported(int64_t M, int64_t N, int64_t K, int64_t gs, bool glu);
hipError_t launch_tgemm_norm(const void* x, const void* r, const void* norm_w, float eps, void* h_out,
                             const uint8_t* w_tiled, const float* scales_gm, const uint8_t* zeros_gm,
                             void* y, int64_t M, int64_t N, int64_t K, int64_t gs, bool glu,
                             hipStream_t stream);

}  // namespace pmi
