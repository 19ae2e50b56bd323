// Big-tile GEMM: the tiled-weight INT4 W4A16 GEMM for many activation rows
// (prefill), gfx950 (v_mfma_f32_16x16x32_f16). A variant of the tiled GEMM
// (w4a16_tgemm.hip) over the same buffers: tiled weights, group-major scales
// and zero points.
//
// Work. A workgroup owns a 256 x 128 output tile (four 64-row weight panels x
// 128 activation rows) over all of K, with eight compute waves, two per SIMD:
// wave w takes the 16-row weight tiles 2 (w % 2) and 2 (w % 2) + 1 of panel
// w / 2 against all 128 activation rows (eight MFMA row tiles). Per 128-column
// unit a workgroup moves 32 KiB of activations and 16 KiB of codes for 8.4
// MFLOP; each B operand is formed once and feeds eight MFMAs. Against four
// panels x two activation halves (every B operand formed by two waves, four
// MFMAs each) this is 35 % fewer VALU instructions for twice the LDS A-operand
// reads, and 4-8 % faster (4096 x 4096 at M = 2048: 81 against 85 us). With
// two waves on a SIMD, one wave's MFMAs can run while the other forms B
// operands.
//
// Placement. The workgroups are numbered activation block by activation
// block and dealt to the 8 XCDs in contiguous ranges (the dispatcher deals
// workgroups round-robin, so workgroup 8 k + x runs on XCD x): the bands that
// share an activation block share an XCD and read its rows from that XCD's
// L2. The activation rows are twice the weight bytes of a workgroup, so they
// are the operand kept local. A placement preference only.
//
// Operands. Each unit's activation rows (128 x 256 bytes), the band's four
// 4 KiB weight blocks and its scales and zero points go global -> registers
// -> LDS, double-buffered in LDS: every wave writes its eighth of unit s + 1 to
// the other slot after computing unit s, then loads the codes of unit s + 2
// and the activations of unit s + 3 (two register stages for the
// activations, whose loads otherwise stalled the slot writes; 79 against 81
// us at 4096 x 4096, M = 2048); one barrier per unit. In a slot, the 16-byte chunk
// c of activation row r sits at chunk c ^ (r % 16), so the 16 rows an
// A-operand read touches at one column fall in 16 different bank groups.
//
// Numerics: those of the tiled GEMM. B = 8 fp16 (q - z), exact (v_perm_b32
// under a 0x64 exponent byte, one packed subtract); the products x (q - z)
// are exact in fp32; per unit y += s * sum x (q - z) in fp32, the reference's
// w = (q - z) * s with fp32 accumulation (pare/kernels/matmul_int4.py:145-176).
#include <atomic>

#include "pmi_common.h"
#include "pmi_launch.h"

namespace pmi {
namespace {

constexpr int kBWaves = 8;  // compute waves: 4 panels x 2 activation halves
constexpr int kBMT = 8;     // 16-row activation tiles per wave (all 128 rows)
// one LDS slot: activations, the four panels' weight blocks, scales, zero points
constexpr int kBX = 128 * 256;          // 32 KiB: 128 rows x 256 bytes
constexpr int kBWo = kBX;               // weights: 4 panels x 4 KiB
constexpr int kBSo = kBWo + 4 * 4096;   // scales: 256 rows x 4 bytes
constexpr int kBZo = kBSo + 1024;       // zero points: 256 rows x 1 byte
constexpr int kBSlot = kBZo + 256;
static_assert(2 * kBSlot <= 160 * 1024, "two slots fit LDS");

struct BgemmArgs {
  const f16* x;
  const uint8_t* wt;    // tiled weights
  const float* s_gm;    // fp32 [G, N]
  const uint8_t* z_gm;  // u8 [G, N]
  f16* y;
  int M, N, K, gs;
  int n_panels;  // 64-row panels of the tiled weights
  int n_bands;   // bands of four panels
  int grid_m;    // 128-row activation blocks
  int chunk;     // (activation block, band) pairs per XCD
};

// s_waitcnt lgkmcnt(0), the other counters left alone (gfx9 encoding)
PMI_DEV void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xF | 0x70 | (3 << 14)); }

__global__ __launch_bounds__(kBWaves * 64, 1) void w4a16_bgemm_kernel(BgemmArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];

  const int tid = threadIdx.x, l = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // workgroup 8 k + x -> pair L = x chunk + k of XCD x's range; L runs band
  // fastest, so an XCD holds consecutive bands of an activation block
  const int x8 = blockIdx.x % 8, k8 = blockIdx.x / 8;
  const int L = x8 * a.chunk + k8;
  if (k8 >= a.chunk || L >= a.n_bands * a.grid_m) return;  // padding workgroups (uniform)
  const int band = L % a.n_bands, mb = L / a.n_bands;
  const int M = a.M, N = a.N, K = a.K;
  const int U = K >> 7;
  const int G = K / a.gs;
  const int upg = a.gs >> 7;  // units per group
  const int m0 = 128 * mb;
  const int ln = l & 15, h = l >> 4;

  // ---- staging: wave w moves activation pieces 4 w .. 4 w + 3 (rows 16 w ..
  // 16 w + 15; lane l: chunk l % 16 of row 4 g + l / 16, read from activation
  // chunk (l % 16) ^ (row % 16)), weight pieces 2 w, 2 w + 1 (panel i / 4, 1 KiB
  // piece i % 4; panels past the last read past the buffer's end, where the
  // buffer resource returns zeros), and wave 0 the band's scales, wave 1 its
  // zero points
  const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (int64_t)M * K * 2);
  const __amdgpu_buffer_rsrc_t rw = rsrc(a.wt, (int64_t)a.n_panels * 64 * (K >> 1));
  const __amdgpu_buffer_rsrc_t rs = rsrc(a.s_gm, (int64_t)G * N * 4);
  const __amdgpu_buffer_rsrc_t rz = rsrc(a.z_gm, (int64_t)G * N);
  int vx[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * wv + 4 * i + (l >> 4);
    const int mg = m0 + row < M ? m0 + row : M - 1;
    vx[i] = mg * K * 2 + 16 * ((l & 15) ^ (row & 15));
  }
  int vwp[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int pc = 2 * wv + i;
    vwp[i] = (band * 4 + pc / 4) * U * 4096 + (pc % 4) * 1024 + 16 * l;
  }
  const int vsz = wv == 0 ? (256 * band + 4 * l) * 4 : 256 * band + 4 * l;
  // The activation rows are staged two units ahead, in two register stages;
  // the codes, scales and zero points one unit ahead.
  struct XStage {
    u32x4 x[4];
  };
  struct WStage {
    u32x4 w[2], sz;
  };
  auto clamp_unit = [&](int u) {
    u = u < U ? u : U - 1;  // past K: re-read the last unit (never used)
    return __builtin_amdgcn_readfirstlane(u);
  };
  auto load_x = [&](XStage& st, int u) {
    const int uu = clamp_unit(u);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      st.x[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rx, vx[i], uu * 256, 0));
  };
  auto load_w = [&](WStage& st, int u) {
    const int uu = clamp_unit(u);
#pragma unroll
    for (int i = 0; i < 2; ++i)
      st.w[i] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, vwp[i], uu * 4096, 0));
    const int g = uu / upg;
    if (wv == 0)
      st.sz = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, vsz, g * N * 4, 0));
    else if (wv == 1)
      st.sz = u32x4{__builtin_amdgcn_raw_buffer_load_b32(rz, vsz, g * N, 0), 0u, 0u, 0u};
  };
  auto stage_write = [&](const XStage& xs, const WStage& ws, uint8_t* base) {
#pragma unroll
    for (int i = 0; i < 4; ++i) *reinterpret_cast<u32x4*>(base + (4 * wv + i) * 1024 + 16 * l) = xs.x[i];
#pragma unroll
    for (int i = 0; i < 2; ++i) *reinterpret_cast<u32x4*>(base + kBWo + (2 * wv + i) * 1024 + 16 * l) = ws.w[i];
    if (wv == 0) *reinterpret_cast<u32x4*>(base + kBSo + 16 * l) = ws.sz;
    else if (wv == 1) *reinterpret_cast<uint32_t*>(base + kBZo + 4 * l) = ws.sz[0];
  };

  // ---- compute: tiles 2 jh, 2 jh + 1 of panel pw, all 128 activation rows
  const int pw = wv >> 1, jh = wv & 1;
  const int p = band * 4 + pw;
  const int row0 = 64 * p + 4 * ln + 2 * jh;
  f32x4 acc[kBMT][2];
#pragma unroll
  for (int mt = 0; mt < kBMT; ++mt)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const uint8_t* base) {
    u32x4 w[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
      w[j] = *reinterpret_cast<const u32x4*>(base + kBWo + pw * 4096 + (2 * jh + j) * 1024 + 16 * l);
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 sc = *reinterpret_cast<const f32x2*>(base + kBSo + (64 * pw + 4 * ln + 2 * jh) * 4);
    const uint32_t zq = *reinterpret_cast<const uint16_t*>(base + kBZo + 64 * pw + 4 * ln + 2 * jh);
    f16x2 nz[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) nz[j] = as_f16x2(neg_magic_zero_x2((zq >> (8 * j)) & 0xFFu));
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 cg[kBMT][2];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int run = t >> 1, half = t & 1;
      // the step's two B operands, then each activation tile read once for both
      f16x8 B[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const uint32_t w0 = w[j][2 * half], w1 = w[j][2 * half + 1];
        const uint32_t t0 = (run ? (w0 >> 4) : w0) & 0x0F0F0F0Fu;
        const uint32_t t1 = (run ? (w1 >> 4) : w1) & 0x0F0F0F0Fu;
        B[j] = b_operand(t0, t1, nz[j]);
      }
#pragma unroll
      for (int i = 0; i < kBMT; ++i) {
        const f16x8 A = *reinterpret_cast<const f16x8*>(base + (16 * i + ln) * 256 + (((4 * t + h) ^ ln) << 4));
#pragma unroll
        for (int j = 0; j < 2; ++j)
          cg[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B[j], t == 0 ? zero4 : cg[i][j], 0, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int i = 0; i < kBMT; ++i)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[i][j][e] = fmaf(sc[j], cg[i][j][e], acc[i][j][e]);
  };

  // Unit u: activations in xs[u % 2] (loaded during unit u - 2), codes in ws
  // (loaded during unit u - 1). Issue order within a step is codes, then
  // activations, so the wait for the codes leaves the younger activations in
  // flight.
  XStage xs[2];
  WStage ws;
  load_x(xs[0], 0);
  load_w(ws, 0);
  stage_write(xs[0], ws, lds);
  load_x(xs[1], 1);
  load_w(ws, 1);
  load_x(xs[0], 2);
  wait_lgkm0();
  barrier_only();
  // step s: compute unit s, write unit s + 1 to the other slot (whose unit
  // s - 1 every wave finished before the last barrier), fetch the codes of
  // s + 2 and the activations of s + 3
  auto step = [&](int s, XStage& x1) {
    compute(lds + (s & 1) * kBSlot);
    __builtin_amdgcn_sched_barrier(0);
    stage_write(x1, ws, lds + ((s + 1) & 1) * kBSlot);
    load_w(ws, s + 2);
    load_x(x1, s + 3);
    // the slot writes have landed before any wave passes (LDS operations
    // complete in order per wave; the barrier makes them visible)
    wait_lgkm0();
    barrier_only();
    __builtin_amdgcn_sched_barrier(0);
  };
  // whole pairs of steps with no exit inside, then the last two units (U is
  // even and at least 12: K % 512 == 0, K >= 1536)
  int s = 0;
  for (; s < U - 2; s += 2) {
    step(s, xs[1]);
    step(s + 1, xs[0]);
  }
  step(U - 2, xs[1]);
  compute(lds + ((U - 1) & 1) * kBSlot);
  if (p >= a.n_panels || row0 >= N) return;

  // lane (n, h): activation rows m0 + 16 i + 4 h + e, weight rows row0 + j
#pragma unroll
  for (int i = 0; i < kBMT; ++i)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int m = m0 + 16 * i + 4 * h + e;
      if (m >= M) continue;
      const uint32_t v0 = __builtin_bit_cast(uint16_t, f32_to_f16_rne(acc[i][0][e]));
      const uint32_t v1 = __builtin_bit_cast(uint16_t, f32_to_f16_rne(acc[i][1][e]));
      *reinterpret_cast<uint32_t*>(a.y + (size_t)m * N + row0) = v0 | (v1 << 16);
    }
}

}  // namespace

BgemmConfig bgemm_config(int64_t M, int64_t N, int64_t K, int64_t gs) {
  BgemmConfig c{};
  c.ok = false;
  if (M < 1 || N % 4 != 0 || K % 128 != 0 || K < 128 || gs % 128 != 0 || K % gs != 0) return c;
  if ((int64_t)M * K * 2 >= (1ll << 31) || ((N + 63) / 64) * 64 * (K / 2) >= (1ll << 31)) return c;
  const int64_t bands = ((N + 63) / 64 + 3) / 4;
  const int64_t gm = (M + 127) / 128;
  const int64_t chunk = (bands * gm + 7) / 8;
  if (8 * chunk >= (1ll << 31)) return c;
  c.ok = true;
  c.n_bands = (int)bands;
  c.grid_m = (int)gm;
  c.chunk = (int)chunk;
  c.grid = (int)(8 * chunk);
  return c;
}

hipError_t launch_bgemm(const void* x, const uint8_t* w_tiled, const float* scales_gm,
                        const uint8_t* zeros_gm, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                        hipStream_t stream) {
  const BgemmConfig c = bgemm_config(M, N, K, gs);
  if (!c.ok) return hipErrorInvalidValue;
  static std::atomic<uint64_t> allowed{0};
  int dev = 0;
  if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
  const uint64_t bit = 1ull << (dev & 63);
  const size_t lds = 2 * (size_t)kBSlot;
  if (!(allowed.load() & bit)) {
    if (hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&w4a16_bgemm_kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        e != hipSuccess)
      return e;
    allowed.fetch_or(bit);
  }
  BgemmArgs a;
  a.x = (const f16*)x;
  a.wt = w_tiled;
  a.s_gm = scales_gm;
  a.z_gm = zeros_gm;
  a.y = (f16*)y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.gs = (int)gs;
  a.n_panels = (int)((N + 63) / 64);
  a.n_bands = c.n_bands;
  a.grid_m = c.grid_m;
  a.chunk = c.chunk;
  hipLaunchKernelGGL(w4a16_bgemm_kernel, dim3(c.grid), dim3(kBWaves * 64), lds, stream, a);
  return hipGetLastError();
}

}  // namespace pmi
