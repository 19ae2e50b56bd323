// Register-streamed MFMA INT4 W4A16 GEMM for blocks of up to 64 activation
// rows, gfx950 (v_mfma_f32_32x32x16_f16), group size 128.
//
// Why a second GEMM. At 16-64 activation rows the weights still dominate the
// traffic (gate_proj at M = 64: 29 MB of codes against 0.5 MB of activations),
// so the kernel must stream them at the HBM rate the split-K GEMV reaches:
// straight into registers, 16 bytes per lane per load, with every CU streaming
// its own bytes. Weight copies through LDS (buffer_load ... lds) measured far
// slower per CU.
//
// Work layout. A workgroup owns 128 weight rows (four 32-row MFMA tiles, one
// per "N wave") and up to 64 activation rows (MT = 1 or 2 row tiles of 32),
// over a range of K. K is cut into 128-column stages (one quantisation
// group); two "K waves" take alternate stages, so a 128-byte weight line (two
// groups) is requested by both at the same step. A workgroup has 8 compute
// waves; the two K-wave tiles are added through LDS at the end, and two more
// waves, one per K wave, only copy activations into LDS. When 128-row blocks
// alone would leave CUs idle, K is also split over `splits` workgroups: each
// stores its fp32 tile in the caller's workspace and the last to arrive adds
// them in split order (deterministic) and writes fp16 Y.
//
// Operands. Lane l of a compute wave owns weight row n = l % 32 of its tile
// and holds, per stage, bytes 32h..32h+31 (h = l / 32) of the row's 64-byte
// group tile (kernel layout: byte b carries column b in its low nibble and
// column 64 + b in its high nibble): two 16-byte loads per stage. MFMA k-step
// j < 4 takes the low nibbles of bytes 32h + 8j .. +7, step j >= 4 the high
// nibbles of bytes 32h + 8(j-4) .. +7, as the B operand (fp16 q - z, exact,
// built with v_perm_b32 under a 0x64 exponent byte and one packed add). The
// matching A operand is 8 consecutive activations of row m = l % 32 of the
// row tile, one 16-byte LDS read. Products x * (q - z) are exact in fp32; per
// stage y += s * sum x*(q - z), the reference's w = (q - z) * s with fp32
// accumulation.
//
// Pipeline. Compute waves keep a 4-deep register ring of weight stages: the
// loads of stage s + 3 are issued before stage s is computed. The activation
// producer of a K wave keeps a 4-deep LDS ring (64 rows x 256 bytes per stage,
// 16-byte chunks XOR-swizzled by row so the A reads of a wave are bank-
// conflict free) with three stages in flight: at every step it waits for the
// oldest, all waves cross one s_barrier, and it issues stage s + 3. Compute
// waves never issue LDS copies, so none of their LDS reads wait on the copy
// queue.
//
// Semantics follow the reference Triton kernel (pare/kernels/matmul_int4.py:
// 105-176): w = (q - zero) * scale per group, fp32 accumulation, fp16 output.
#include <type_traits>

#include "pmi_common.h"
#include "pmi_launch.h"

namespace pmi {
namespace {

constexpr int kNW = 4;                      // N waves (32 weight rows each)
constexpr int kKW = 2;                      // K waves (alternate stages)
constexpr int kCompute = kNW * kKW;         // compute waves
constexpr int kWaves = kCompute + kKW;      // + one activation producer per K wave
constexpr int kThreads = kWaves * 64;
constexpr int kBN = 32 * kNW;               // weight rows per workgroup
constexpr int kBM = 64;                     // activation rows per block
constexpr int kDW = 4;                      // weight stages in a compute wave's ring
constexpr int kDX = 4;                      // activation stages per K wave in LDS
constexpr int kXRow = 256;                  // bytes of one activation row of a stage
constexpr int kXStage = kBM * kXRow;        // 16 KiB
constexpr int kXCopies = kXStage / 1024;    // copies of 64 lanes x 16 bytes per stage

typedef float f32x16 __attribute__((ext_vector_type(16)));

struct Gemm64Args {
  const f16* x;
  const uint8_t* w;
  const float* s;
  const void* z;
  const float* s_gm;    // optional group-major copies: fp32 [G, N]
  const uint8_t* z_gm;  //                              u8 [G, N]
  f16* y;
  float* part;    // split-K partial tiles (splits > 1)
  int* counters;  // one per (n block, m block), zero between calls
  int M, N, K, n_blocks, grid_m, splits;
  // udiv_magic of splits, 8 grid_m and n_blocks % 8 (the divisors of the
  // workgroup numbering), so that no wave divides before its first load
  uint32_t split_m, span_m, rem_m;
};

// One weight stage of a compute lane: 32 bytes of its row, the row's scale
// and raw zero point (u8, or fp32 bits), widened only where it is used.
template <bool ZB>
struct WStage {
  u32x4 w[2];
  float s;
  typename std::conditional<ZB, uint8_t, uint32_t>::type z;
};

// SZT: scales and zero points from the group-major copies (32 rows of one
// group are 128 + 32 contiguous bytes) instead of a gather over the [N, G]
// arrays. ZU8: u8 zero points (fp32 otherwise); with SZT they are always u8.
template <int MT, bool ZU8, bool SZT>
__global__ __launch_bounds__(kThreads, 1) void w4a16_gemm64_kernel(Gemm64Args a) {
  constexpr bool ZB = ZU8 || SZT;
  __shared__ __attribute__((aligned(16))) uint8_t xring[kKW * kDX * kXStage];
  __shared__ int last_flag;

  const int tid = threadIdx.x, l = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // (n block, m block, split) of this workgroup. Splits of a tile are
  // consecutive; workgroups are dealt to the 8 XCDs round-robin by index, so
  // the m blocks of one n block, numbered 8 tiles apart, share an XCD and its
  // L2 (a placement preference only).
  // The arguments the prologue reads, pinned in SGPRs at entry so that they
  // arrive in one round trip to the kernel-argument memory.
  asm volatile("" ::"s"(a.M), "s"(a.N), "s"(a.K), "s"(a.n_blocks), "s"(a.grid_m), "s"(a.splits),
               "s"(a.split_m), "s"(a.span_m), "s"(a.rem_m), "s"(a.x), "s"(a.w));
  const int bid = blockIdx.x;
  const int tl = (int)udiv(bid, a.splits, a.split_m);
  const int sp = bid - tl * a.splits;
  int nb, mb;
  {
    const int gm = a.grid_m, full = a.n_blocks & ~7;
    if (gm == 1) {
      nb = tl;
      mb = 0;
    } else if (tl < full * gm) {
      const int q = (int)udiv(tl, 8 * gm, a.span_m), r = tl - q * 8 * gm;
      nb = q * 8 + (r & 7);
      mb = r >> 3;
    } else {
      const int rem = a.n_blocks - full, r = tl - full * gm;
      const int q = (int)udiv(r, rem, a.rem_m);
      nb = full + (r - q * rem);
      mb = q;
    }
  }
  const int M = a.M, N = a.N, K = a.K;
  const int G = K >> 7;  // groups = 128-column stages
  // groups [g_lo, g_hi) of this split, in K-wave pairs; K wave k takes
  // g_lo + k, g_lo + k + 2, ... (stage s of K wave k is group g_lo + 2s + k)
  const int pairs = (G + 1) >> 1;
  const int g_lo = 2 * (int)udiv(sp * pairs, a.splits, a.split_m);
  const int g_hi_raw = 2 * (int)udiv((sp + 1) * pairs, a.splits, a.split_m);
  const int g_hi = g_hi_raw < G ? g_hi_raw : G;
  const int S = (g_hi - g_lo + 1) >> 1;  // steps (stages of K wave 0)
  const int row_bytes = K >> 1;

  f32x16 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[mt][i] = 0.f;

  if (wv >= kCompute) {
    // ---- activation producer of K wave kp: copy c covers stage rows 4c..4c+3
    // (lane l: row 4c + l/16, LDS chunk p = l%16 holding activation chunk
    // p ^ (row % 16)); rows past M repeat row M - 1, stages past the split's
    // range repeat its last group
    const int kp = wv - kCompute;
    const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (int64_t)M * K * 2);
    int vx[kXCopies];
#pragma unroll
    for (int c = 0; c < kXCopies; ++c) {
      const int row = 4 * c + (l >> 4);
      int mg = mb * kBM + row;
      mg = mg < M ? mg : M - 1;
      vx[c] = mg * K * 2 + 16 * ((l & 15) ^ (row & 15));
    }
    uint8_t* xbase = xring + kp * kDX * kXStage;
    auto issue = [&](int slot, int st) {
      int g = g_lo + 2 * st + kp;
      g = g < g_hi ? g : g_hi - 1;
      const int soff = __builtin_amdgcn_readfirstlane(g * 256);
#pragma unroll
      for (int c = 0; c < kXCopies; ++c)
        copy_to_lds<16>(rx, xbase + slot * kXStage + c * 1024, vx[c], soff);
    };
#pragma unroll
    for (int d = 0; d < kDX - 1; ++d) issue(d, d);
    for (int s = 0; s < S; ++s) {
      wait_vmcnt<(kDX - 2) * kXCopies>();  // stage s has landed
      barrier_only();                      // ... for both K waves; stage s-1 is free
      issue((s + kDX - 1) & (kDX - 1), s + kDX - 1);
    }
    wait_vmcnt<0>();  // the clamped copies past the last stage
  } else {
    // ---- compute wave (N wave nw, K wave kw) -------------------------------
    const int nw = wv & (kNW - 1), kw = wv / kNW;
    const int h = l >> 5, ln = l & 31;
    int n = nb * kBN + 32 * nw + ln;
    n = n < N ? n : N - 1;
    const __amdgpu_buffer_rsrc_t rw = rsrc(a.w, (int64_t)N * row_bytes);
    const int vw = n * row_bytes + 32 * h;
    __amdgpu_buffer_rsrc_t rs, rz;
    int vs, vz, gs_mul, gz_mul;  // lane offsets; bytes per group (SGPR offsets)
    if constexpr (SZT) {
      rs = rsrc(a.s_gm, (int64_t)G * N * 4);
      rz = rsrc(a.z_gm, (int64_t)G * N);
      vs = 4 * n, vz = n, gs_mul = 4 * N, gz_mul = N;
    } else {
      rs = rsrc(a.s, (int64_t)N * G * 4);
      rz = rsrc(a.z, (int64_t)N * G * (ZU8 ? 1 : 4));
      vs = 4 * n * G, vz = n * G * (ZU8 ? 1 : 4), gs_mul = 4, gz_mul = ZU8 ? 1 : 4;
    }
    // stages of this K wave (the other may have one more)
    const int S_own = (g_hi - g_lo - kw + 1) >> 1;

    auto issue_w = [&](WStage<ZB>& ws, int st) {
      int g = g_lo + 2 * st + kw;
      g = g < g_hi ? g : g_hi - 1;  // past the range: re-read the last group (unused)
      const int woff = __builtin_amdgcn_readfirstlane(g * 64);
      ws.w[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, vw, woff, 0));
      ws.w[1] =
          __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, vw + 16, woff, 0));
      ws.s = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                           rs, vs, __builtin_amdgcn_readfirstlane(g * gs_mul), 0));
      if constexpr (ZB)
        ws.z = __builtin_amdgcn_raw_buffer_load_b8(rz, vz, __builtin_amdgcn_readfirstlane(g * gz_mul), 0);
      else
        ws.z = __builtin_amdgcn_raw_buffer_load_b32(rz, vz, __builtin_amdgcn_readfirstlane(g * gz_mul), 0);
    };

    const int xrow = ln * kXRow;
    const uint8_t* xk = xring + kw * kDX * kXStage;

    // A operands of k-step j: row r = 32 mt + ln, chunk q ^ (r % 16) with
    // q = (j < 4 ? 0 : 8) + 4h + (j & 3). They are read one k-step ahead of
    // their MFMAs so the LDS latency overlaps the matrix work.
    auto load_a = [&](const uint8_t* xb, int j, f16x8 (&A)[MT]) {
      const int q = (j < 4 ? 0 : 8) + 4 * h + (j & 3);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        A[mt] = *reinterpret_cast<const f16x8*>(xb + mt * 32 * kXRow + xrow + ((q ^ (ln & 15)) << 4));
    };
    auto compute = [&](const WStage<ZB>& ws, int xslot) {
      const uint8_t* xb = xk + xslot * kXStage;
      uint32_t zi;
      if constexpr (ZB) zi = (uint32_t)ws.z;
      else zi = (uint32_t)(int)__builtin_bit_cast(float, ws.z);
      const f16x2 nz = as_f16x2(neg_magic_zero_x2(zi));
      f32x16 cg[MT];
      f16x8 A[2][MT];
      load_a(xb, 0, A[0]);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        if (j + 1 < 8) load_a(xb, j + 1, A[(j + 1) & 1]);
        const u32x4& wq = ws.w[(j & 3) >> 1];
        const uint32_t w0 = wq[2 * (j & 1)], w1 = wq[2 * (j & 1) + 1];
        const uint32_t t0 = (j < 4 ? w0 : (w0 >> 4)) & 0x0F0F0F0Fu;
        const uint32_t t1 = (j < 4 ? w1 : (w1 >> 4)) & 0x0F0F0F0Fu;
        const f16x8 B = b_operand(t0, t1, nz);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (j == 0) {
            f32x16 zero16;
#pragma unroll
            for (int i = 0; i < 16; ++i) zero16[i] = 0.f;
            cg[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[0][mt], B, zero16, 0, 0, 0);
          } else {
            cg[mt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(A[j & 1][mt], B, cg[mt], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[mt][i] = fmaf(ws.s, cg[mt][i], acc[mt][i]);
    };

    // Ring: stages 0..2 in flight before the loop; step s issues stage s + 3
    // into the slot stage s - 1 used, then waits (the compiler's vmcnt for the
    // slot it reads) and crosses the step barrier. Unrolled by the ring depth
    // so every slot is a fixed register set.
    static_assert(kDW == kDX, "weight and activation rings step together");
    WStage<ZB> ring[kDW];
#pragma unroll
    for (int d = 0; d < kDW - 1; ++d) issue_w(ring[d], d);
    __builtin_amdgcn_sched_barrier(0);
    for (int s0 = 0; s0 < S; s0 += kDW) {
#pragma unroll
      for (int d = 0; d < kDW; ++d) {
        const int s = s0 + d;
        if (s >= S) break;
        issue_w(ring[(d + kDW - 1) % kDW], s + kDW - 1);
        __builtin_amdgcn_sched_barrier(0);
        barrier_only();  // activations of step s are in LDS
        if (s < S_own) compute(ring[d], d);
      }
    }
  }

  // ---- K-wave reduction through LDS (the activation ring is free) ----------
  __syncthreads();
  const int nw = wv & (kNW - 1), kw = wv / kNW;
  const int h = l >> 5, ln = l & 31;
  float* red = reinterpret_cast<float*>(xring);  // [nw][mt][i][lane]
  if (wv < kCompute && kw == 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) red[((nw * MT + mt) * 16 + i) * 64 + l] = acc[mt][i];
  }
  __syncthreads();
  const bool lead = wv < kNW;  // compute waves of K wave 0 hold the tile
  if (lead) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[mt][i] += red[((nw * MT + mt) * 16 + i) * 64 + l];
  }

  if (a.splits > 1) {
    // Partial tile of split sp: [nw][mt][i / 4][lane] x 16 bytes, each lane's
    // 4 values contiguous, a wave's store one 1 KiB run. Stores and loads use
    // the device-scope cache policy (sc1), like agent-scope atomics: coherent
    // across the XCDs' L2 caches without a release fence. The s_waitcnt makes
    // every store of this thread complete before the barrier, which orders
    // them before the counter increment.
    constexpr int kPartBytes = kNW * MT * 16 * 64 * 4;
    const __amdgpu_buffer_rsrc_t rp =
        rsrc(a.part + (size_t)tl * a.splits * (kPartBytes / 4), (int64_t)a.splits * kPartBytes);
    const int vlane = nw * MT * 4096 + l * 16;
    constexpr int kSc1 = 16;
    if (lead) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const f32x4 v = {acc[mt][4 * b], acc[mt][4 * b + 1], acc[mt][4 * b + 2], acc[mt][4 * b + 3]};
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rp,
                                                 vlane + (mt * 4 + b) * 1024,
                                                 __builtin_amdgcn_readfirstlane(sp * kPartBytes), kSc1);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const int old = __hip_atomic_fetch_add(&a.counters[tl], 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
      last_flag = old == a.splits - 1;
    }
    __syncthreads();
    if (!last_flag || !lead) return;
    // Last to arrive: add the partials in split order (deterministic). Every
    // split's partial, this one's included, is in the workspace; the loads of
    // kB splits are issued together (one round trip per kB splits).
    constexpr int kB = MT >= 2 ? 2 : 4;
    f32x16 tot[MT] = {};
    for (int q0 = 0; q0 < a.splits; q0 += kB) {
      f32x16 part[kB][MT];
#pragma unroll
      for (int sb = 0; sb < kB; ++sb) {
        const int q = q0 + sb < a.splits ? q0 + sb : a.splits - 1;  // past the end: loaded, not added
        const int soff = __builtin_amdgcn_readfirstlane(q * kPartBytes);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            const f32x4 v = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, vlane + (mt * 4 + b) * 1024, soff, kSc1));
#pragma unroll
            for (int e = 0; e < 4; ++e) part[sb][mt][4 * b + e] = v[e];
          }
      }
      // the adds select rather than break: behind the break the compiler sank
      // the loads of later splits to their adds, one round trip per split
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int sb = 0; sb < kB; ++sb) {
        const bool use = q0 + sb < a.splits;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const f32x16 t = q0 + sb == 0 ? part[sb][mt] : tot[mt] + part[sb][mt];
          tot[mt] = use ? t : tot[mt];
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = tot[mt];
    if (tid == 0) __hip_atomic_store(&a.counters[tl], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!lead) return;

  // ---- epilogue: lane (ln, h) holds rows 32 mt + 8 (i / 4) + 4 h + i % 4 of
  // weight row ln of its tile
  const int ncol = nb * kBN + 32 * nw + ln;
  if (ncol >= N) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = mb * kBM + 32 * mt + 8 * (i >> 2) + 4 * h + (i & 3);
      if (m < M) a.y[(size_t)m * N + ncol] = f32_to_f16_rne(acc[mt][i]);
    }
}

template <int MT>
hipError_t launch_mt(const Gemm64Args& a, int grid, int zero_u8, hipStream_t stream) {
  if (a.s_gm)
    hipLaunchKernelGGL((w4a16_gemm64_kernel<MT, true, true>), dim3(grid), dim3(kThreads), 0, stream, a);
  else if (zero_u8)
    hipLaunchKernelGGL((w4a16_gemm64_kernel<MT, true, false>), dim3(grid), dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((w4a16_gemm64_kernel<MT, false, false>), dim3(grid), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

int device_cu_count() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

Gemm64Config gemm64_config(int64_t M, int64_t N, int64_t K) {
  Gemm64Config c;
  c.n_blocks = (int)((N + kBN - 1) / kBN);
  c.grid_m = (int)((M + kBM - 1) / kBM);
  const int64_t tiles = (int64_t)c.n_blocks * c.grid_m;
  const int64_t pairs = (K / 128 + 1) / 2;
  // Split K while the tiles alone leave CUs idle, at most one split per K-wave
  // pair of groups (and no more tiles than the counter block holds).
  int64_t s = device_cu_count() / tiles;
  if (s > pairs) s = pairs;
  if (s > 16) s = 16;
  if (s < 1 || tiles > (int64_t)(kWsCounterBytes / 4)) s = 1;
  c.splits = (int)s;
  c.grid = (int)(tiles * c.splits);
  c.ws_split = c.splits > 1 ? ws_align((size_t)tiles * c.splits * kBN * (M <= 32 ? 32 : 64) * 4) : 0;
  return c;
}

hipError_t launch_gemm64(const void* x, const uint8_t* w, const float* scales, const void* zeros,
                         int zero_u8, const float* scales_gm, const uint8_t* zeros_gm, void* y,
                         int64_t M, int64_t N, int64_t K, void* workspace, size_t ws_bytes,
                         size_t part_offset, hipStream_t stream) {
  Gemm64Config c = gemm64_config(M, N, K);
  Gemm64Args a;
  a.x = (const f16*)x;
  a.w = w;
  a.s = scales;
  a.z = zeros;
  a.s_gm = scales_gm;
  a.z_gm = zeros_gm;
  a.y = (f16*)y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.n_blocks = c.n_blocks;
  a.grid_m = c.grid_m;
  // workspace: [counters, kWsCounterBytes][X[:, perm] (act_order)][partial tiles]
  // with the partial tiles at part_offset; without room for them the kernel
  // runs unsplit
  if (c.splits > 1 && (!workspace || ws_bytes < part_offset + c.ws_split)) {
    c.splits = 1;
    c.grid = c.n_blocks * c.grid_m;
  }
  a.splits = c.splits;
  a.split_m = udiv_magic((uint32_t)c.splits);
  a.span_m = udiv_magic(8u * (uint32_t)c.grid_m);
  a.rem_m = udiv_magic((uint32_t)(c.n_blocks % 8 ? c.n_blocks % 8 : 1));
  a.counters = (int*)workspace;
  a.part = c.splits > 1 ? (float*)((uint8_t*)workspace + part_offset) : nullptr;
  if (M <= 32) return launch_mt<1>(a, c.grid, zero_u8, stream);
  return launch_mt<2>(a, c.grid, zero_u8, stream);
}

}  // namespace pmi
