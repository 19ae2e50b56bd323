// Tiled-weight MFMA INT4 W4A16 GEMM for 2..64 activation rows (more as
// 16-row blocks on narrow layers), gfx950 (v_mfma_f32_16x16x32_f16).
//
// Why a tiled copy of the weights. At these row counts the kernel is a weight
// stream, and how the stream meets the DRAM decides its speed: on MI355X a
// grid that reads the gate_proj weights (29 MB) as 64-byte pieces of many rows
// per load (the MFMA operand layout of the row-major kernel layout) moves them
// in 8.7 us; the same bytes read as contiguous 4 KiB blocks take 6.1 us. The
// tiled copy (`pmi_tile_w4a16`, built once per layer like the kernel-layout
// weight) stores, for every 64-row panel p and 128-column unit u, one 4 KiB
// block that a wave loads with four contiguous 1 KiB loads straight into MFMA
// operand registers:
//   block (p, u) = tile j (4) x lane L = n + 16 h (64) x 16 bytes;
//   lane (n, h) of tile j holds row 64 p + 4 n + j, unit bytes b < 8:
//   columns 128 u + 8 h + b (low nibble) and + 64 (high nibble); b >= 8:
//   columns 128 u + 32 + 8 h + (b - 8) and + 64.
// MFMA k-step t < 4 of a unit then covers columns 128 u + 32 t + [0, 32):
// steps 0 and 1 take the low nibbles of bytes 0-7 and 8-15, steps 2 and 3 the
// high nibbles, so every step lies inside one group of 32, 64 or 128 columns
// and the per-group scale applies after the steps of its group.
//
// Work layout. A workgroup owns NTW 16-row tiles of one panel (16 NTW weight
// rows) for all activation rows and the whole K range. Its four compute waves
// take the units u = 4 s + w (w = wave) and are added through LDS at the end;
// the four waves of a workgroup read four consecutive blocks at every step.
// NTW is the largest of 4, 2, 1 that still gives about a workgroup per CU.
// Up to 16 rows, layers whose workgroups would leave most CUs idle (narrow
// layers; long rows, K > 8192, with four tiles per workgroup) split K: four
// workgroups per tile set take ranges of unit quads, and the last to finish
// adds the fp32 partial tiles in range order (combine_splits).
//
// Activations. Up to 16 rows (MT = 1) every compute wave loads the A operands
// of its own units with the weights (16 rows x 256 bytes per unit, L2
// resident), so the kernel has no LDS staging and no barrier in its loop.
// 17-32 rows (MT = 2) would need twice the registers; there two producer
// waves copy the activations of each step (the four units of the four waves)
// into a four-deep LDS ring with buffer_load ... lds, and all waves cross one
// s_barrier per step. 33-64 rows (MT = 4) use the same ring with half units
// per slot (64 columns; 32 KiB a slot, 128 KiB for four), two barriers per
// step: every B operand then feeds four activation tiles, and the ring stays
// four slots deep (gate_proj at M = 64: 15.9 against 17.6 us for the MFMA
// GEMM of w4a16_gemm.hip; with full-unit slots, two fit: 16.4 us).
//
// act_order (GATHER, up to 16 rows). The tiled weights hold their columns in perm
// order, so the A operand of column c is x[:, perm[c]]. Every workgroup copies
// the M activation rows (row stride 2K + 16 bytes, which puts the 16 rows of
// one column in 16 different LDS banks) and the perm table (as byte offsets
// 2 perm[c], out-of-range entries read column 0) into LDS once, before its
// loop; each lane then gathers its 8 columns per k-step with 2-byte LDS reads,
// one step ahead of the MFMAs. A workgroup reads X once either way, so the
// gather adds the 4K-byte table to its L2 traffic and no launch; 2K bytes with
// the 16-bit copy of the permutation (GATHER 2; GATHER 1 reads the int32 one).
//
// Residual add + RMSNorm (NORM, up to 4 rows, K <= 4096). Every workgroup
// reads the rows of x and of the residual ahead of its first weight loads,
// forms h = x + r, the per-row statistic and the normalised rows exactly as
// the add + RMSNorm kernel does (same per-thread chunks and summation order),
// and keeps them in LDS; the compute waves read their A operands there. The
// launch then equals the norm launch followed by the plain one bit for bit.
//
// Pipeline. Each compute wave keeps a three-deep register ring of units
// (weights, scales, zero points and, for MT = 1, activations): the loads of
// step s + 2 are issued before step s is computed. The loop runs whole rounds
// of three steps with no exit inside a round and every load unconditional
// (past the range it re-reads the last unit), so the compiler waits for
// exactly the two younger steps; a deeper ring measured slower (more requests
// in flight per CU spread the DRAM pages).
//
// Operands and numerics are those of the MFMA GEMM: B = 8 fp16 (q - z), exact,
// from v_perm_b32 under a 0x64 exponent byte and one packed subtract; the
// products x * (q - z) are exact in fp32; per group y += s * sum x*(q - z) in
// fp32, the reference's w = (q - z) * s with fp32 accumulation
// (pare/kernels/matmul_int4.py:105-176).
#include <stdlib.h>

#include <atomic>
#include <type_traits>

#include "pmi_common.h"
#include "pmi_launch.h"

namespace pmi {
namespace {

constexpr int kKW = 4;     // compute waves (units u = 4 s + w)
constexpr int kDW = 3;     // register ring depth (steps)
constexpr int kDX = 4;     // LDS ring depth (slots), MT = 2 and 4
constexpr int kProd = 2;   // activation producer waves, MT = 2 and 4
constexpr int kXGLds = kTgemmXGLds;  // LDS of the act_order variant (X rows + perm table)
constexpr int kXGPermIt = 8;         // perm-table entries per thread / 4 (K <= 8192)

struct TgemmArgs {
  const f16* x;
  const int32_t* perm;  // act_order columns (GATHER 1), their uint16 copy (GATHER 2), else null
  const uint8_t* wt;    // tiled weights
  const float* s_gm;    // fp32 [G, N]
  const uint8_t* z_gm;  // u8 [G, N]
  f16* y;
  int M, N, K, gs;
  int n_wg;    // weight workgroups (16 NTW rows each)
  int grid_m;  // activation blocks of 16 MT rows
  int n_tiles; // RNG: 16-row tiles (4 per 64-row panel)
  int splits;  // K ranges per weight workgroup (MT = 1, one activation block), else 1
  int* counters;  // splits > 1: one per weight workgroup, zero between calls
  float* part;    // splits > 1: [n_wg][splits][NTW] partial 16 x 16 fp32 tiles
  int glu;        // NTW = 4: rows 4n + {0, 1} of a panel are gate, 4n + {2, 3} the
                  // matching up rows; y is [M, N / 2] = silu(gate) * up
  // NORM: the activations are RMSNorm(x + r) * nw (r nullable), formed once
  // per workgroup into LDS; workgroup 0 writes h = x + r to h_out when r is
  // given
  const f16* r;
  const f16* nw;
  f16* h_out;
  float eps;
  // Quotients and reciprocal constants the host works out (derive_args), so
  // that no wave divides before its first load (an integer division is a
  // ~25-instruction dependent chain): n / d = umulhi(n, ceil(2^32 / d)) for
  // d >= 2 and n d < 2^32, and n / d = (n ceil(2^16 / d)) >> 16 for n d < 2^16.
  int groups;           // K / gs
  uint32_t upg_magic;   // units per group (gs >= 128: gs / 128, else 1), 16-bit form
  uint32_t span_magic;  // grid_m > 1: 8 grid_m, 32-bit form
  uint32_t split_magic; // splits > 1: splits, 32-bit form
  int perm_u16;         // host dispatch: perm points at the 16-bit copy (GATHER 2)
};

// Fills the derived fields of `a`; false when a quotient would leave the range
// in which its constant is exact.
inline bool derive_args(TgemmArgs& a) {
  const uint32_t upg = a.gs >= 128 ? (uint32_t)a.gs / 128u : 1u;
  const uint64_t units = (uint64_t)a.K / 128u;
  const uint64_t grid = (uint64_t)(a.n_wg + 8) * (uint64_t)(a.grid_m > 0 ? a.grid_m : 1) *
                        (uint64_t)(a.splits > 0 ? a.splits : 1);
  const uint64_t span = 8ull * (uint64_t)(a.grid_m > 0 ? a.grid_m : 1);
  if (a.gs <= 0 || units * upg >= (1ull << 16) || grid * span >= (1ull << 32) ||
      grid * (uint64_t)(a.splits > 0 ? a.splits : 1) >= (1ull << 32) ||
      (units / kKW) * (uint64_t)(a.splits > 0 ? a.splits : 1) >= (1ull << 32))
    return false;
  a.groups = a.K / a.gs;
  a.upg_magic = (65536u + upg - 1u) / upg;
  a.span_magic = span >= 2 ? (uint32_t)(((1ull << 32) + span - 1) / span) : 0u;
  a.split_magic = a.splits >= 2 ? (uint32_t)(((1ull << 32) + (uint64_t)a.splits - 1) / (uint64_t)a.splits) : 0u;
  return true;
}

// One unit of a compute wave: activations (MT = 1), weights, and for each of
// the GPU groups of the unit the NTW scales and zero points of the lane's rows
// (RNG: one scale and zero point per tile, the tiles' rows are not adjacent).
// The zero points stay as wide as their load (8 bits for one row, 16 for two)
// and are widened where they are used: loaded into 32-bit ring registers,
// the compiler narrowed the loop-carried copies and masked them before the
// loop, a wait for every load in flight there (the whole ring drained before
// the first step).
template <int NTW>
using ZeroT = std::conditional_t<NTW == 1, uint8_t, std::conditional_t<NTW == 2, uint16_t, uint32_t>>;
template <int MT, int NTW, int GPU, bool RNG = false>
struct Unit {
  u32x4 xa[MT == 1 ? 4 : 1];
  u32x4 w[NTW];
  f32x4 s[RNG ? 1 : GPU];
  ZeroT<NTW> z[RNG ? 1 : GPU];
  float sr[RNG ? NTW : 1];
  uint8_t zr[RNG ? NTW : 1];
  int xo;  // NORM: byte offset of the unit's 128 columns in an LDS activation row
};

// K split: the NTW partial 16 x 16 tiles of split sp go to the workspace;
// the last split of weight workgroup wg to arrive adds all of them in split
// order (so the result does not depend on the arrival order) and returns
// true with the sums in `sum`. Stores and loads carry the device-scope cache
// policy (sc1), as agent-scope atomics do, so they are coherent across the
// XCDs' L2 caches without a release fence: the stores complete (s_waitcnt)
// before the counter increment, and the last split loads only after its
// increment has returned the count. All kMaxSplits loads of a tile are issued
// together (one round trip; past the last split they re-read it).
constexpr int kMaxSplits = 4;
template <int NTW>
__device__ __forceinline__ bool combine_splits(const TgemmArgs& a, int wg, int sp, int l, f32x4 (&sum)[NTW]) {
  constexpr int kTile = 1024;  // bytes of a 16 x 16 fp32 tile
  constexpr int kSc1 = 16;
  const __amdgpu_buffer_rsrc_t rp =
      rsrc(a.part + (size_t)wg * a.splits * NTW * (kTile / 4), (int64_t)a.splits * NTW * kTile);
#pragma unroll
  for (int j = 0; j < NTW; ++j)
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, sum[j]), rp, 16 * l,
                                           __builtin_amdgcn_readfirstlane((sp * NTW + j) * kTile), kSc1);
  // The compiler barriers keep the partial stores above the wait and the
  // counter increment, and the partial loads below the returned count: the
  // waitcnt intrinsic alone is no memory clobber, and a relaxed RMW orders
  // no plain accesses at the language level.
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_waitcnt(0);
  asm volatile("" ::: "memory");
  int old = 0;
  if (l == 0)
    old = __hip_atomic_fetch_add(&a.counters[wg], 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  old = __builtin_amdgcn_readfirstlane(old);
  if (old != a.splits - 1) return false;
  asm volatile("" ::: "memory");
  f32x4 v[kMaxSplits][NTW];
#pragma unroll
  for (int q = 0; q < kMaxSplits; ++q) {
    const int qq = q < a.splits ? q : a.splits - 1;
#pragma unroll
    for (int j = 0; j < NTW; ++j)
      v[q][j] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                              rp, 16 * l, __builtin_amdgcn_readfirstlane((qq * NTW + j) * kTile), kSc1));
  }
  // the adds select rather than branch: behind a branch per split the
  // compiler sank each load to its add, one round trip per split
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < NTW; ++j) {
    sum[j] = v[0][j];
#pragma unroll
    for (int q = 1; q < kMaxSplits; ++q) {
      const f32x4 t = sum[j] + v[q][j];
      sum[j] = q < a.splits ? t : sum[j];
    }
  }
  if (l == 0) __hip_atomic_store(&a.counters[wg], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return true;
}

// RNG: the workgroup takes NTW consecutive 16-row tiles t0 = wg NTW .. of the
// 4 n_panels tiles (5 or 6 of them, so that one pass over the CUs covers more
// than one 64-row panel per CU), the last ones clamped and not stored.
// SPLIT: a K range of a split weight workgroup (a.splits > 1); a variant of its
// own, so that unsplit launches carry none of its index arithmetic.
// BF: bf16 activations and output (the native bf16 extension), up to 16 rows
// per activation block, one K range, gs % 128 == 0. gfx950 has no packed bf16
// subtract, so B is the bf16 128 + q, exact (v_perm_b32 under a 0x43 byte),
// and each k-step adds a second MFMA whose B operand is -(128 + z) in every
// element: its products x (-(128 + z)) are exact in fp32, so the group's sum
// is sum x (q - z) up to the fp32 rounding of the accumulation; the fold and
// the combine are those of fp16, and y is rounded to bf16 (nearest even).
template <int MT, int NTW, int GPU, int GATHER, bool RNG, bool SPLIT = false, bool NORM = false,
          bool BF = false>
__global__ __launch_bounds__((kKW + (MT == 1 ? 0 : kProd)) * 64, 1) void w4a16_tgemm_kernel(TgemmArgs a) {
  static_assert(!GATHER || MT == 1, "the act_order gather is built for up to 16 rows");
  static_assert(!NORM || (MT == 1 && GPU == 1 && !GATHER && !RNG && !SPLIT),
                "the fused norm is built for up to 4 rows, gs % 128 == 0, one K range");
  static_assert(!RNG || (MT == 1 && GPU == 1), "tile ranges are built for up to 16 rows, gs >= 128");
  static_assert(!SPLIT || (MT == 1 && !RNG), "the K split is built for up to 16 rows");
  static_assert(!BF || (MT == 1 && GPU == 1 && !GATHER && !RNG && !SPLIT && !NORM),
                "bf16 activations are built for 16-row blocks, gs % 128 == 0, one K range");
  using UnitT = Unit<MT, NTW, GPU, RNG>;
  constexpr bool RING = MT > 1;
  // MT = 4: the ring holds half units (64 columns, k-steps 0-1 or 2-3), two
  // slots per unit, so that the same 128 KiB hold four slots
  constexpr bool HALF = MT == 4;
  constexpr int BM = 16 * MT;
  constexpr int RB = HALF ? 128 : 256;  // bytes of an activation row in a slot
  constexpr int XBYTES = BM * RB;       // activation bytes of a slot (RING)
  constexpr int CPU = XBYTES / 1024;    // 1 KiB copies per slot (RING)
  constexpr int RPC = 1024 / RB;        // activation rows per copy
  constexpr int CH = RB / 16;           // 16-byte chunks per row in a slot
  constexpr int SUBS = 4 / NTW;  // workgroups per panel
  constexpr int TPG = 4 / GPU;   // MFMA k-steps per group
  // activation ring (MT = 2, 4), reused after the loop for the partial tiles of
  // three waves
  constexpr int kRing = RING ? kKW * kDX * XBYTES : 0;
  constexpr int kRed = kKW * MT * NTW * 64 * 16;  // partial tiles, indexed by source wave
  constexpr int kLds0 = kRing > kRed ? kRing : kRed;
  // GATHER: the activation rows and the perm table in dynamic LDS sized by the
  // host (max(M (2K + 16) + 4K, the partial tiles)), so that small row counts
  // leave room for other workgroups; reused after the loop for the partial tiles
  // NORM: the normalised activation rows (stride 2K + 16 bytes) in dynamic LDS
  // of max(M (2K + 16), the partial tiles)
  __shared__ __attribute__((aligned(16))) uint8_t lds_s[GATHER || NORM ? 16 : kLds0];
  extern __shared__ __attribute__((aligned(16))) uint8_t lds_d[];
  uint8_t* const lds = GATHER || NORM ? lds_d : lds_s;
  __shared__ float npart[NORM ? 4 * kKW : 1];  // NORM: per-row, per-wave sums of h^2

  // The arguments the prologue reads, pinned in SGPRs at entry so that they
  // arrive in one round trip: left to itself the compiler loads each group
  // where it is first used, and every group behind a branch waited for its
  // own trip to the kernel-argument memory before the first weight load.
  asm volatile("" ::"s"(a.M), "s"(a.N), "s"(a.K), "s"(a.n_wg), "s"(a.grid_m), "s"(a.splits),
               "s"(a.groups), "s"(a.upg_magic), "s"(a.span_magic), "s"(a.split_magic), "s"(a.x),
               "s"(a.wt), "s"(a.s_gm), "s"(a.z_gm));
  const int tid = threadIdx.x, l = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  // (weight workgroup, activation block). Workgroups are dealt to the 8 XCDs
  // round-robin by index, so the activation blocks of one weight workgroup
  // are numbered 8 apart: they share an XCD, and the second read of its
  // weights mostly hits that XCD's L2 (a placement preference only).
  int wg = blockIdx.x, mb = 0, sp = 0;
  if constexpr (SPLIT) {
    // K split (one activation block): the splits of a weight workgroup are
    // consecutive blocks
    wg = (int)__umulhi(blockIdx.x, a.split_magic);  // blockIdx.x / splits
    sp = blockIdx.x - wg * a.splits;
  } else if (a.grid_m > 1) {
    const int span = 8 * a.grid_m;
    const int q = (int)__umulhi(blockIdx.x, a.span_magic), r = blockIdx.x - q * span;
    wg = 8 * q + (r & 7);
    mb = r >> 3;
  }
  const int panel = RNG ? 0 : wg / SUBS, jb = RNG ? 0 : (wg % SUBS) * NTW;
  const int M = a.M, N = a.N, K = a.K;
  // padding workgroups: past the weight workgroups, or past the last rows (uniform)
  if (wg >= a.n_wg || (!RNG && 64 * panel + jb >= N)) return;
  const int m0 = mb * BM;  // first activation row of this block
  const int U = K >> 7;              // units (U % 4 == 0)
  // steps of this workgroup: the unit quads q_lo .. q_lo + steps - 1 (all of
  // them unsplit; split sp takes quads Q sp / splits .. Q (sp + 1) / splits - 1)
  const int Q = U / kKW;
  const int q_lo = SPLIT ? (int)__umulhi((uint32_t)(sp * Q), a.split_magic) : 0;
  const int steps = SPLIT ? (int)__umulhi((uint32_t)((sp + 1) * Q), a.split_magic) - q_lo : Q;
  const int ln = l & 15, h = l >> 4;
  const int row0 = 64 * panel + 4 * ln + jb;  // first of the lane's NTW rows
  // RNG: tile j of the range (clamped to the last tile), its lane row and the
  // wave-uniform byte offset of its 1 KiB in every 4 KiB block
  int trow[RNG ? NTW : 1], tbase[RNG ? NTW : 1];
  if constexpr (RNG) {
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      int t = wg * NTW + j;
      t = t < a.n_tiles ? t : a.n_tiles - 1;
      trow[j] = 64 * (t >> 2) + 4 * ln + (t & 3);
      tbase[j] = (t >> 2) * (K >> 7) * 4096 + 1024 * (t & 3);
    }
  }

  f32x4 acc[MT][NTW];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (RING && wv >= kKW) {
    // ---- activation producer p: per slot the units 4 s .. 4 s + 3 (MT = 4:
    // their halves), copy c of unit k covers rows RPC c + l / CH; LDS chunk
    // l % CH of a row holds activation chunk (l % CH) ^ (row % 16) (MT = 4:
    // ^ ((row / 2) % 8), so that each 16 lanes of an A read, rows n = 0..15,
    // hit 16 different bank groups)
    const int p = wv - kKW;
    const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (int64_t)M * K * 2);
    int vx[CPU];
#pragma unroll
    for (int c = 0; c < CPU; ++c) {
      const int r = RPC * c + l / CH;
      const int mg = m0 + r < M ? m0 + r : M - 1;
      vx[c] = mg * K * 2 + 16 * ((l % CH) ^ ((HALF ? r >> 1 : r) % CH));
    }
    constexpr int CPS = kKW * CPU / kProd;  // copies per producer per step
    static_assert((kDX - 1) * CPS < 64, "copies in flight fit vmcnt");
    auto issue = [&](int slot, int st) {
#pragma unroll
      for (int q = 0; q < CPS; ++q) {
        const int cc = q * kProd + p;
        const int k = cc / CPU, c = cc % CPU;
        int u = kKW * (HALF ? st >> 1 : st) + k;
        u = u < U ? u : U - 1;
        copy_to_lds<16>(rx, lds + (k * kDX + slot) * XBYTES + c * 1024, vx[c],
                        __builtin_amdgcn_readfirstlane(u * 256 + (HALF ? (st & 1) * 128 : 0)));
      }
    };
    for (int d = 0; d < kDX - 1; ++d) issue(d, d);
    int slot = kDX - 1;
    for (int s = 0; s < (HALF ? 2 * steps : steps); ++s) {
      wait_vmcnt<(kDX - 2) * CPS>();  // slot s has landed
      barrier_only();                 // ... and every wave is done with step s - 1
      issue(slot, s + kDX - 1);
      slot = slot + 1 == kDX ? 0 : slot + 1;
    }
    wait_vmcnt<0>();  // clamped copies past the last step
  } else {
    // ---- compute wave kw: units u = 4 s + kw
    const int kw = wv;
    const int G = a.groups;
    const int rowc = row0 < N ? row0 : N - 4 + jb;  // clamped for the scale/zero loads
    const __amdgpu_buffer_rsrc_t rw = rsrc(a.wt, (int64_t)((N + 63) / 64) * 64 * (K >> 1));
    const __amdgpu_buffer_rsrc_t rs = rsrc(a.s_gm, (int64_t)G * N * 4);
    const __amdgpu_buffer_rsrc_t rz = rsrc(a.z_gm, (int64_t)G * N);
    const int vw = panel * U * 4096 + 1024 * jb + 16 * l;
    const int vs = rowc * 4, vz = rowc;
    __amdgpu_buffer_rsrc_t rxd;
    int vxd = 0;
    const int xstride = 2 * K + 16;   // GATHER: LDS bytes per activation row
    const int xtab = M * xstride;     // GATHER: LDS offset of the perm table
    int xrow = 0;                     // GATHER: LDS offset of the lane's row
    if constexpr (MT == 1) {
      const int mg = m0 + ln < M ? m0 + ln : M - 1;
      if constexpr (GATHER || NORM) {
        xrow = mg * xstride;
      } else {
        rxd = rsrc(a.x, (int64_t)M * K * 2);
        vxd = mg * K * 2 + 16 * h;
      }
    }
    // GATHER: X rows in 1 KiB copies (K % 512 == 0), dealt to the waves, and
    // the perm table through registers (clamped, scaled to byte offsets; the
    // table is written after the ring's first weight loads are issued, so
    // that the latencies overlap). From the 16-bit copy of the permutation
    // each 16-byte load holds 8 entries instead of 4: half the loads.
    u32x4 pv[GATHER ? kXGPermIt : 1];
    auto stage_issue = [&]() {
      if constexpr (GATHER) {
        const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (int64_t)M * K * 2);
        const int cpr = K >> 9;
        for (int c = kw; c < M * cpr; c += kKW) {
          const int m = c / cpr, q = c - m * cpr;
          copy_to_lds<16>(rx, lds + m * xstride + q * 1024, 16 * l,
                          __builtin_amdgcn_readfirstlane(m * K * 2 + q * 1024));
        }
        if constexpr (GATHER == 2) {
          const __amdgpu_buffer_rsrc_t rp = rsrc(a.perm, (int64_t)K * 2);
#pragma unroll
          for (int i = 0; i < kXGPermIt / 2; ++i) {
            const int e = tid + i * kKW * 64;  // entries 8 e .. 8 e + 7
            pv[i] = 8 * e < K ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, 16 * e, 0, 0))
                              : u32x4{0u, 0u, 0u, 0u};
          }
        } else {
          const __amdgpu_buffer_rsrc_t rp = rsrc(a.perm, (int64_t)K * 4);
#pragma unroll
          for (int i = 0; i < kXGPermIt; ++i) {
            const int e = tid + i * kKW * 64;  // entries 4 e .. 4 e + 3
            pv[i] = 4 * e < K ? __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, 16 * e, 0, 0))
                              : u32x4{0u, 0u, 0u, 0u};
          }
        }
      }
    };
    // GATHER: the A operands of a step come from LDS in three stages, each one
    // step ahead of the next so that no LDS read waits inside a step: the
    // perm-table offsets of step s + 2 (8 per k-step: lane (n, h), k-step t
    // takes columns perm[128 u + 32 t + 8 h + i], i < 8, of row n), the
    // 2-byte gathers of step s + 1, and the packing of step s.
    uint32_t poff[GATHER ? 32 : 1], graw[GATHER ? 32 : 1];
    auto table_read = [&](int s) {
      if constexpr (GATHER) {
        const int u = kKW * (q_lo + (s < steps ? s : steps - 1)) + kw;
        const uint8_t* pt = lds + xtab + (u * 128 + 8 * h) * 4;
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(pt + 128 * (q >> 1) + 16 * (q & 1));
#pragma unroll
          for (int c = 0; c < 4; ++c) poff[4 * q + c] = v[c];
        }
      }
    };
    auto gather_issue = [&]() {
      if constexpr (GATHER) {
        const uint8_t* xr = lds + xrow;
#pragma unroll
        for (int k = 0; k < 32; ++k) graw[k] = *reinterpret_cast<const uint16_t*>(xr + poff[k]);
      }
    };
    auto pack = [&](UnitT& un) {
      if constexpr (GATHER) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          un.xa[t] = u32x4{graw[8 * t] | (graw[8 * t + 1] << 16), graw[8 * t + 2] | (graw[8 * t + 3] << 16),
                           graw[8 * t + 4] | (graw[8 * t + 5] << 16), graw[8 * t + 6] | (graw[8 * t + 7] << 16)};
      }
    };
    auto issue = [&](UnitT& un, int s) {
      // past the range: re-read the wave's last unit (loaded, never computed)
      const int u = kKW * (q_lo + (s < steps ? s : steps - 1)) + kw;
      const int uu = __builtin_amdgcn_readfirstlane(u);
      if constexpr (MT == 1 && !GATHER && !NORM) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
          un.xa[t] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rxd, vxd, uu * 256 + 64 * t, 0));
      }
      if constexpr (NORM) un.xo = uu * 256;
      if constexpr (RNG) {
        const int g = (int)(((uint32_t)uu * a.upg_magic) >> 16);  // uu / upg
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          un.w[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(
              rw, 16 * l, __builtin_amdgcn_readfirstlane(tbase[j] + uu * 4096), 2));
          const int rc = trow[j] < N ? trow[j] : N - 1;
          un.sr[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, rc * 4, g * 4 * N, 0));
          un.zr[j] = __builtin_amdgcn_raw_buffer_load_b8(rz, rc, g * N, 0);
        }
        return;
      }
#pragma unroll
      for (int j = 0; j < NTW; ++j)
        un.w[j] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, vw + 1024 * j, uu * 4096, 2));
#pragma unroll
      for (int gp = 0; gp < GPU; ++gp) {
        const int g = GPU > 1 ? uu * GPU + gp : (int)(((uint32_t)uu * a.upg_magic) >> 16);
        // the vector result is converted as a whole: hipcc 7.2 mis-reads the
        // lanes of a u32x4 bit-cast element by element to float
        if constexpr (NTW == 4) {
          un.s[gp] = __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, vs, g * 4 * N, 0));
          un.z[gp] = __builtin_amdgcn_raw_buffer_load_b32(rz, vz, g * N, 0);
        } else if constexpr (NTW == 2) {
          typedef float f32x2 __attribute__((ext_vector_type(2)));
          const f32x2 v = __builtin_bit_cast(f32x2, __builtin_amdgcn_raw_buffer_load_b64(rs, vs, g * 4 * N, 0));
          un.s[gp] = f32x4{v[0], v[1], 0.f, 0.f};
          un.z[gp] = __builtin_amdgcn_raw_buffer_load_b16(rz, vz, g * N, 0);
        } else {
          un.s[gp] = f32x4{__builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, vs, g * 4 * N, 0)),
                           0.f, 0.f, 0.f};
          un.z[gp] = __builtin_amdgcn_raw_buffer_load_b8(rz, vz, g * N, 0);
        }
      }
    };
    f32x4 cg[MT][NTW];  // the current group's products (kept across the halves of MT = 4)
    auto compute = [&](const UnitT& un, const uint8_t* xb, int half) {
      const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        if (HALF && (t >> 1) != half) continue;
        const int gp = t / TPG;
        const int run = t >> 1, half = t & 1;
        f16x8 A[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if constexpr (NORM)
            A[mt] = *reinterpret_cast<const f16x8*>(lds + xrow + un.xo + 64 * t + 16 * h);
          else if constexpr (MT == 1) A[mt] = __builtin_bit_cast(f16x8, un.xa[t]);
          else if constexpr (HALF)
            A[mt] = *reinterpret_cast<const f16x8*>(xb + (16 * mt + ln) * RB +
                                                     (((4 * (t & 1) + h) ^ ((ln >> 1) % CH)) << 4));
          else A[mt] = *reinterpret_cast<const f16x8*>(xb + (16 * mt + ln) * 256 + (((4 * t + h) ^ ln) << 4));
        }
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
          const uint32_t zq = RNG ? (uint32_t)un.zr[j] : ((uint32_t)un.z[gp] >> (8 * j)) & 0xFFu;
          const f16x2 nz = as_f16x2(neg_magic_zero_x2(zq));
          const uint32_t w0 = un.w[j][2 * half], w1 = un.w[j][2 * half + 1];
          const uint32_t t0 = (run ? (w0 >> 4) : w0) & 0x0F0F0F0Fu;
          const uint32_t t1 = (run ? (w1 >> 4) : w1) & 0x0F0F0F0Fu;
          if constexpr (BF) {
            const bf16x8 Bq = b_operand_bf16(t0, t1);
            const uint32_t nzb = (0xC300u | zq) * 0x00010001u;  // bf16 -(128 + z), twice
            const bf16x8 Bz = __builtin_bit_cast(bf16x8, u32x4{nzb, nzb, nzb, nzb});
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
              const bf16x8 Ab = __builtin_bit_cast(bf16x8, A[mt]);
              cg[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ab, Bq, t % TPG == 0 ? zero4 : cg[mt][j], 0,
                                                                  0, 0);
              cg[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(Ab, Bz, cg[mt][j], 0, 0, 0);
            }
          } else {
            const f16x8 B = b_operand(t0, t1, nz);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              cg[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mt], B, t % TPG == 0 ? zero4 : cg[mt][j],
                                                                 0, 0, 0);
          }
        }
        if (t % TPG == TPG - 1) {
#pragma unroll
          for (int j = 0; j < NTW; ++j) {
            const float sc = RNG ? un.sr[j] : un.s[gp][j];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
              for (int i = 0; i < 4; ++i) acc[mt][j][i] = fmaf(sc, cg[mt][j][i], acc[mt][j][i]);
          }
        }
      }
    };

    UnitT ring[kDW];
    if constexpr (GATHER) {
      stage_issue();
      __builtin_amdgcn_sched_barrier(0);
    }
    // NORM: x, r and the norm weight of every thread's columns, issued ahead
    // of the ring's first loads so that waiting for them leaves those in
    // flight. Thread t holds columns (i * 256 + t) * 8 .. + 7 of every row,
    // i < 2, the chunks pmi_add_rmsnorm_f16's thread t holds (K <= 4096).
    u32x4 nx[NORM ? 4 : 1][2], nr[NORM ? 4 : 1][2], nwv[2];
    if constexpr (NORM) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        const int c = (i * 256 + tid) * 8, cc = c < K ? c : 0;
        nwv[i] = *reinterpret_cast<const u32x4*>(a.nw + cc);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int mm = m < M ? m : M - 1;
          nx[m][i] = *reinterpret_cast<const u32x4*>(a.x + (size_t)mm * K + cc);
          if (a.r) nr[m][i] = *reinterpret_cast<const u32x4*>(a.r + (size_t)mm * K + cc);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int d = 0; d < kDW - 1; ++d) {
      issue(ring[d], d);
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (NORM) {
      // h = x + r rounded to fp16 and sum(h^2) per row in the order of
      // pmi_add_rmsnorm_f16 (each thread's chunks in column order, then the
      // wave butterfly, then the four waves in order), so that the normalised
      // activations are bit-identical to its output
      wait_vmcnt_lgkm0<(kDW - 1) * (NTW + 2 * GPU)>();
      __builtin_amdgcn_sched_barrier(0);
      f16x8 hv[4][2];
      float ss[4];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        ss[m] = 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int c = (i * 256 + tid) * 8;
          const f16x8 xv = __builtin_bit_cast(f16x8, nx[m][i]);
          f16x8 hh = xv;
          if (a.r) {
            const f16x8 rv = __builtin_bit_cast(f16x8, nr[m][i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) hh[e] = (f16)((float)xv[e] + (float)rv[e]);
          }
          hv[m][i] = hh;
          if (c < K && m < M) {
#pragma unroll
            for (int e = 0; e < 8; ++e) ss[m] += (float)hh[e] * (float)hh[e];
            if (a.r && blockIdx.x == 0) *reinterpret_cast<f16x8*>(a.h_out + (size_t)m * K + c) = hh;
          }
        }
        ss[m] = wave_sum(ss[m]);
        if (l == 0) npart[4 * m + wv] = ss[m];
      }
      wait_vmcnt_lgkm0<(kDW - 1) * (NTW + 2 * GPU)>();
      barrier_only();
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        if (m >= M) break;
        const float inv = rsqrtf((npart[4 * m] + npart[4 * m + 1] + npart[4 * m + 2] + npart[4 * m + 3]) /
                                     (float)K + a.eps);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          const int c = (i * 256 + tid) * 8;
          if (c >= K) continue;
          const f16x8 wv8 = __builtin_bit_cast(f16x8, nwv[i]);
          f16x8 o;
#pragma unroll
          for (int e = 0; e < 8; ++e) o[e] = (f16)((float)hv[m][i][e] * inv * (float)wv8[e]);
          *reinterpret_cast<f16x8*>(lds + m * xstride + 2 * c) = o;
        }
      }
      // every row is in LDS before any wave reads it; the scheduling fences
      // keep the loop's work below the barrier
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt_lgkm0<(kDW - 1) * (NTW + 2 * GPU)>();
      barrier_only();
      __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (GATHER) {
      if constexpr (GATHER == 2) {
#pragma unroll
        for (int i = 0; i < kXGPermIt / 2; ++i) {
          const int e = tid + i * kKW * 64;  // entries 8 e .. 8 e + 7 (K % 8 == 0)
          if (8 * e < K) {
            u32x4 o0, o1;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              const uint32_t lo = pv[i][c] & 0xFFFFu, hi = pv[i][c] >> 16;
              const uint32_t olo = lo < (uint32_t)K ? 2u * lo : 0u;
              const uint32_t ohi = hi < (uint32_t)K ? 2u * hi : 0u;
              if (c < 2) { o0[2 * c] = olo; o0[2 * c + 1] = ohi; }
              else { o1[2 * c - 4] = olo; o1[2 * c - 3] = ohi; }
            }
            *reinterpret_cast<u32x4*>(lds + xtab + 32 * e) = o0;
            *reinterpret_cast<u32x4*>(lds + xtab + 32 * e + 16) = o1;
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < kXGPermIt; ++i) {
          const int e = tid + i * kKW * 64;  // entries 4 e .. 4 e + 3
          if (4 * e < K) {
            u32x4 o;
#pragma unroll
            for (int c = 0; c < 4; ++c) o[c] = pv[i][c] < (uint32_t)K ? 2u * pv[i][c] : 0u;
            *reinterpret_cast<u32x4*>(lds + xtab + 16 * e) = o;
          }
        }
      }
      // this wave's X copies have landed (only the ring's loads may still be
      // in flight) and its table writes are done; after the barrier so are
      // every wave's. The scheduling fences keep step 0's unpacking below the
      // barrier: hoisted above it, it made every wave wait for the first
      // weight batch before the barrier, and the first gathers started only
      // then (Qwen q_o 3584 x 3584, M = 16: 8.6 against 8.2 us).
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt_lgkm0<(kDW - 1) * (RNG ? 3 * NTW : NTW + 2 * GPU)>();
      barrier_only();
      __builtin_amdgcn_sched_barrier(0);
      table_read(0);
      gather_issue();
      table_read(1);
    }
    int xslot = 0;
    auto step = [&](const UnitT& un) {
      const uint8_t* xb = nullptr;
      if constexpr (RING) {
        barrier_only();  // the activations of this step are in LDS
        xb = lds + (kw * kDX + xslot) * XBYTES;
        xslot = xslot + 1 == kDX ? 0 : xslot + 1;
      }
      compute(un, xb, 0);
      if constexpr (HALF) {
        barrier_only();  // ... and of its second half
        xb = lds + (kw * kDX + xslot) * XBYTES;
        xslot = xslot + 1 == kDX ? 0 : xslot + 1;
        compute(un, xb, 1);
      }
    };
    // Whole rounds of kDW steps, then a tail already in flight (a K split may
    // leave fewer than kDW steps: then only the tail).
    int s0 = 0;
    if (steps >= kDW) do {
#pragma unroll
      for (int d = 0; d < kDW; ++d) {
        issue(ring[(d + kDW - 1) % kDW], s0 + d + kDW - 1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (GATHER) {
          pack(ring[d]);
          gather_issue();
          table_read(s0 + d + 2);
          __builtin_amdgcn_sched_barrier(0);
        }
        step(ring[d]);
      }
      s0 += kDW;
    } while (s0 + kDW <= steps);
#pragma unroll
    for (int d = 0; d < kDW - 1; ++d) {
      if (s0 + d >= steps) break;
      if constexpr (GATHER) {
        pack(ring[d]);
        gather_issue();
        table_read(s0 + d + 2);
      }
      step(ring[d]);
    }
  }

  // ---- the four waves' partial tiles are added through LDS (a unit past K,
  // re-read by a clamped load, is never computed: steps * 4 covers U exactly
  // only when U % 4 == 0, which the host requires)
  // Activation tile mt is finished by compute wave mt % 4 (all by wave 0 at
  // MT = 1): every compute wave stores its partial tiles, and the finishing
  // wave adds the four in wave order 0..3 (no register array is indexed by
  // the wave number, which would put it in scratch memory).
  __syncthreads();
  f32x4* red = reinterpret_cast<f32x4*>(lds);
  if (wv < kKW) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < NTW; ++j) red[((wv * MT + mt) * NTW + j) * 64 + l] = acc[mt][j];
  }
  __syncthreads();
  if (wv >= kKW) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    if ((MT == 1 ? 0 : mt % kKW) != wv) continue;
    f32x4 sum[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
      sum[j] = red[(mt * NTW + j) * 64 + l];
#pragma unroll
      for (int k = 1; k < kKW; ++k) sum[j] += red[((k * MT + mt) * NTW + j) * 64 + l];
    }
    if constexpr (SPLIT) {
      if (!combine_splits<NTW>(a, wg, sp, l, sum)) return;
    }
    if (!RNG && row0 >= N) return;
    // lane (n, h): rows 16 mt + 4 h + i of the activations, weight rows row0 + j
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m0 + 16 * mt + 4 * h + i;
      if (m >= M) continue;
      if constexpr (RNG) {
        // one 2-byte store per tile: the range's rows are 4 apart per tile
#pragma unroll
        for (int j = 0; j < NTW; ++j)
          if (wg * NTW + j < a.n_tiles && trow[j] < N) a.y[(size_t)m * N + trow[j]] = f32_to_f16_rne(sum[j][i]);
        continue;
      }
      uint16_t v[4] = {0, 0, 0, 0};
#pragma unroll
      for (int j = 0; j < NTW && j < 4; ++j)
        v[j] = BF ? f32_to_bf16_rne(sum[j][i]) : __builtin_bit_cast(uint16_t, f32_to_f16_rne(sum[j][i]));
      if constexpr (NTW == 4) {
        if (a.glu) {
          // columns 32 p + 2 n and + 1 of the activation, each formed as
          // pmi_silu_mul_f16 forms it from the fp16 gate and up outputs
          *reinterpret_cast<uint32_t*>(a.y + (size_t)m * (N >> 1) + 32 * panel + 2 * ln) =
              glu_pair((uint32_t)v[0] | ((uint32_t)v[1] << 16), (uint32_t)v[2] | ((uint32_t)v[3] << 16));
          continue;
        }
      }
      f16* dst = a.y + (size_t)m * N + row0;
      if constexpr (NTW == 4) {
        *reinterpret_cast<uint2*>(dst) = uint2{(uint32_t)v[0] | ((uint32_t)v[1] << 16),
                                               (uint32_t)v[2] | ((uint32_t)v[3] << 16)};
      } else if constexpr (NTW == 2) {
        *reinterpret_cast<uint32_t*>(dst) = (uint32_t)v[0] | ((uint32_t)v[1] << 16);
      } else {
        *reinterpret_cast<uint16_t*>(dst) = v[0];
      }
    }
  }
}

// Launches one kernel variant; GATHER variants get their dynamic LDS beyond
// the 64 KiB default allowed once per variant and device.
template <int MT, int NTW, int GPU, int GATHER, bool RNG, bool SPLIT>
hipError_t launch_variant(const TgemmConfig& c, const TgemmArgs& a, hipStream_t stream) {
  const dim3 block((kKW + (MT == 1 ? 0 : kProd)) * 64);
  size_t lds = 0;
  if constexpr (GATHER) {
    static std::atomic<uint64_t> allowed{0};
    int dev = 0;
    if (hipError_t e = hipGetDevice(&dev); e != hipSuccess) return e;
    const uint64_t bit = 1ull << (dev & 63);
    if (!(allowed.load() & bit)) {
      if (hipError_t e = hipFuncSetAttribute(
              reinterpret_cast<const void*>(&w4a16_tgemm_kernel<MT, NTW, GPU, true, RNG, SPLIT>),
              hipFuncAttributeMaxDynamicSharedMemorySize, kXGLds);
          e != hipSuccess)
        return e;
      allowed.fetch_or(bit);
    }
    const size_t need = (size_t)a.M * (2 * a.K + 16) + 4 * (size_t)a.K;
    const size_t red = (size_t)kKW * NTW * 64 * 16;
    lds = need > red ? need : red;
  }
  hipLaunchKernelGGL((w4a16_tgemm_kernel<MT, NTW, GPU, GATHER, RNG, SPLIT>), dim3(c.grid), block, lds,
                     stream, a);
  return hipGetLastError();
}

// The fused-norm variants (one activation block, one K range): the
// normalised rows in dynamic LDS, at most 4 (2 * 4096 + 16) bytes, within the
// default limit.
template <int NTW>
hipError_t launch_norm_variant(const TgemmConfig& c, const TgemmArgs& a, hipStream_t stream) {
  const size_t need = (size_t)a.M * (2 * a.K + 16);
  const size_t red = (size_t)kKW * NTW * 64 * 16;
  hipLaunchKernelGGL((w4a16_tgemm_kernel<1, NTW, 1, false, false, false, true>), dim3(c.grid),
                     dim3(kKW * 64), need > red ? need : red, stream, a);
  return hipGetLastError();
}

template <int MT, int NTW, int GPU, bool RNG = false>
hipError_t launch_cfg(const TgemmConfig& c, const TgemmArgs& a, hipStream_t stream) {
  if constexpr (MT == 1) {
    // K split: one tile per workgroup at every group size, 2 or 4 at gs >= 128
    if constexpr (!RNG && (NTW == 1 || GPU == 1)) {
      if (a.splits > 1) {
        if (a.perm && a.perm_u16) return launch_variant<1, NTW, GPU, 2, false, true>(c, a, stream);
        if (a.perm) return launch_variant<1, NTW, GPU, 1, false, true>(c, a, stream);
        return launch_variant<1, NTW, GPU, false, false, true>(c, a, stream);
      }
    }
    if (a.perm && a.perm_u16) return launch_variant<1, NTW, GPU, 2, RNG, false>(c, a, stream);
    if (a.perm) return launch_variant<1, NTW, GPU, 1, RNG, false>(c, a, stream);
  }
  return launch_variant<MT, NTW, GPU, false, RNG, false>(c, a, stream);
}

template <int MT, int NTW>
hipError_t launch_gpu(const TgemmConfig& c, const TgemmArgs& a, hipStream_t stream) {
  if (a.gs == 32) return launch_cfg<MT, NTW, 4>(c, a, stream);
  if (a.gs == 64) return launch_cfg<MT, NTW, 2>(c, a, stream);
  return launch_cfg<MT, NTW, 1>(c, a, stream);
}

template <int MT>
hipError_t launch_mt(const TgemmConfig& c, const TgemmArgs& a, hipStream_t stream) {
  if constexpr (MT == 1) {
    if (c.rng) {
      switch (c.ntw) {
        case 5: return launch_cfg<1, 5, 1, true>(c, a, stream);
        case 6: return launch_cfg<1, 6, 1, true>(c, a, stream);
        default: return hipErrorInvalidValue;
      }
    }
  }
  if (c.ntw == 4) return launch_gpu<MT, 4>(c, a, stream);
  if (c.ntw == 2) return launch_gpu<MT, 2>(c, a, stream);
  return launch_gpu<MT, 1>(c, a, stream);
}

}  // namespace

bool tgemm_supported(int64_t M, int64_t N, int64_t K, int64_t gs) {
  // K % 512 == 0: every compute wave gets the same number of units, at least
  // the ring depth of them (K >= 1536)
  // The last two bounds keep the host's reciprocal constants exact
  // (derive_args): units times units per group, workgroups times the span
  // of one weight workgroup's activation blocks.
  const int64_t wgs = ((N + 63) / 64 * 4 + 8) * ((M + 15) / 16);
  return M >= 1 && N % 4 == 0 && K % 512 == 0 && K >= 1536 &&
         (gs == 32 || gs == 64 || gs % 128 == 0) &&
         K % gs == 0 && (int64_t)M * K * 2 < (1ll << 31) && ((N + 63) / 64) * 64 * (K / 2) < (1ll << 31) &&
         wgs < (1ll << 31) && (K / 128) * (gs >= 128 ? gs / 128 : 1) < (1ll << 16) &&
         wgs * 8 * ((M + 15) / 16) < (1ll << 32);
}

TgemmConfig tgemm_config(int64_t M, int64_t N, int64_t K, int64_t gs, bool gather) {
  TgemmConfig c;
  c.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  // tuning override (benchmark sweeps only)
  static const int env_mt = [] { const char* e = getenv("PMI_TGEMM_MT"); return e ? atoi(e) : 0; }();
  if ((env_mt == 1 || env_mt == 2 || env_mt == 4) && !gather) c.mt = env_mt;
  c.rng = false;
  // the most rows per workgroup that still give about one workgroup per CU
  const int64_t cus = device_cu_count();
  const int64_t panels = (N + 63) / 64;
  c.ntw = panels >= (cus * 3) / 4 ? 4 : (2 * panels >= (cus * 3) / 4 ? 2 : 1);
  // tuning override (benchmark sweeps only)
  static const int env_ntw = [] { const char* e = getenv("PMI_TGEMM_NTW"); return e ? atoi(e) : 0; }();
  // Past 24 rows, 16-row activation blocks (MT = 1: activations straight from
  // L2 into registers, no LDS ring or barriers; the blocks of one weight
  // workgroup share an XCD, so its weights come from HBM once) wherever the
  // blocks and the weight workgroups fit one pass over the CUs, with the
  // narrowest weight tiles that do. Against the 32- and 64-row LDS-ring
  // kernels (us): 4096 x 4096 at M = 32 / 48 / 64 7.3 / 8.6 / 8.6 against 8.5 /
  // 10.0 / 10.5; 2048 x 4096 at M = 64 7.4 against 9.7; 1024 x 4096 at M = 64 /
  // 256 7.2 / 8.4 against 9.5 / 10.1. Where they do not fit (gate 14336 x 4096
  // at M = 32 / 64: 15.8 / 26.3 against 11.8 / 14.7) the ring kernels stay,
  // and at 17-24 rows, where the second block is mostly empty (4096 x 4096 at
  // M = 17: 7.5 against 7.2; 3584 x 3584 at M = 24: 7.0 against 6.8).
  if (M > 24 && !gather && env_mt == 0 && env_ntw == 0) {
    const int64_t gm = (M + 15) / 16;
    for (int ntw = 1; ntw <= 4; ntw *= 2) {
      const int64_t n_wg = panels * (4 / ntw);
      if ((n_wg + 7) / 8 * 8 * gm <= cus) {
        c.mt = 1;
        c.ntw = ntw;
        break;
      }
    }
  }
  if (env_ntw == 1 || env_ntw == 2 || env_ntw == 4) c.ntw = env_ntw;
  c.n_wg = (int)(panels * (4 / c.ntw));
  // Up to 16 rows with more panels than CUs: ranges of 5 or 6 consecutive
  // 16-row tiles per workgroup, so that one pass over the CUs covers every
  // tile. Measured on Qwen gate/up 18944 x 3584: with the act_order gather
  // (whose LDS keeps one workgroup per CU) 13.3 against 19.2 us at M = 16 and
  // 12.4 against 14.0 at M = 4; without it 13.6 against 15.0 at M = 16 and
  // 12.7 against 13.0 at M = 8, but 13.9 against 12.6 at M = 4, where two
  // workgroups per CU already share the passes. Ranges of 7 (fused gate/up
  // 28672 rows) measured slower than two passes (18.6 against 15.5 at M = 8).
  static const int env_rng = [] { const char* e = getenv("PMI_TGEMM_RANGE"); return e ? atoi(e) : -1; }();
  if (c.mt == 1 && gs % 128 == 0 && panels > cus && env_rng != 0 && (gather || M >= 8)) {
    const int64_t tiles = 4 * panels;
    const int64_t per = (tiles + cus - 1) / cus;
    if (per <= 6) {
      c.rng = true;
      c.ntw = (int)(per < 5 ? 5 : per);
      c.n_wg = (int)((tiles + c.ntw - 1) / c.ntw);
    }
  }
  c.grid_m = (int)((M + 16 * c.mt - 1) / (16 * c.mt));
  c.grid = c.grid_m == 1 ? c.n_wg : (int)((c.n_wg + 7) / 8 * 8 * c.grid_m);
  // Up to 16 rows with the weight workgroups on at most a quarter of the CUs
  // (narrow layers): split K into kMaxSplits ranges of whole unit quads; the
  // last split of each workgroup adds the partial tiles (one round trip for
  // all of them). Measured on MI355X (us, unsplit -> 4 splits): 512 x 3584 at
  // M = 8 / 16 5.3 / 6.6 -> 4.9 / 5.2 (act_order 6.6 / 8.0 -> 6.0 / 6.8), 1024 x
  // 4096 at M = 16 6.9 -> 5.9 (act_order 8.7 -> 7.9), 512 x 8192 at M = 8 8.8 ->
  // 5.8. Two splits gained nothing (2048 x 4096 at M = 16: 7.0 either way), and
  // more than one pass over the CUs loses (three there: 9.4).
  c.splits = 1;
  c.ws_split = 0;
  static const int env_split = [] { const char* e = getenv("PMI_TGEMM_SPLIT"); return e ? atoi(e) : -1; }();
  // Long rows (K > 8192) up to 16 rows, where 64-row workgroups fill at most a
  // quarter of the CUs (down_proj: N <= 4096): four 16-row tiles per
  // workgroup, K split four ways, so that each workgroup reads a quarter of
  // the activation rows once for four tiles (unsplit, every tile re-reads all
  // of them). Against the MFMA GEMM (us): Llama down 4096 x 14336 at M = 4 / 8
  // / 16 10.3 / 10.5 / 11.8 against 14.0; Qwen down 3584 x 18944 11.9 / 11.9 /
  // 12.9 against 15.8 / 15.5 / 15.3. Two splits, or four tiles unsplit, lose.
  // The same at 13-16 rows for shorter rows where one-tile workgroups already
  // fill more than a quarter of the CUs (1024 < N <= 4096; not with the
  // act_order gather, whose every workgroup stages all of X): 2048 x 4096 at
  // M = 16 6.2 against 6.9 us, Qwen q_o 3584 x 3584 6.6 against 7.0, 4096 x
  // 4096 7.1 against 7.2; at M = 8 it loses (4096 x 4096: 7.0 against 6.0).
  const bool wide_split = K > 8192 || (M > 12 && !gather && 4 * panels * kMaxSplits > cus);
  if (c.mt == 1 && c.grid_m == 1 && !c.rng && gs % 128 == 0 && wide_split && env_split != 0 &&
      env_ntw == 0 && panels * kMaxSplits <= cus && panels <= (int64_t)(kWsCounterBytes / 4)) {
    c.ntw = 4;
    c.n_wg = (int)panels;
    c.grid = c.n_wg;
  }
  if (c.mt == 1 && c.grid_m == 1 && !c.rng && (c.ntw == 1 || (gs % 128 == 0 && (env_split > 0 || wide_split))) &&
      env_split != 0 && c.n_wg <= (int64_t)(kWsCounterBytes / 4)) {
    int64_t s = env_split > 0 ? env_split : (cus / c.n_wg >= kMaxSplits ? kMaxSplits : 1);
    if (s > (K >> 9)) s = K >> 9;
    if (s > kMaxSplits) s = kMaxSplits;
    if (s >= 2) {
      c.splits = (int)s;
      c.grid = c.n_wg * c.splits;
      c.ws_split = ws_align((size_t)c.n_wg * c.splits * c.ntw * 1024);
    }
  }
  return c;
}

// The bf16 variant: the configuration the fp16 call would take, when it is
// one unsplit K range of 16-row blocks without tile ranges.
bool tgemm_bf16_supported(int64_t M, int64_t N, int64_t K, int64_t gs) {
  if (!tgemm_supported(M, N, K, gs) || gs % 128 != 0) return false;
  const TgemmConfig c = tgemm_config(M, N, K, gs, false);
  return c.mt == 1 && !c.rng;
}

bool tgemm_gather_supported(int64_t M, int64_t K) {
  return M >= 1 && M <= 16 && K <= 4 * 64 * kXGPermIt * 4 && M * (2 * K + 16) + 4 * K <= kXGLds;
}

hipError_t launch_tgemm(const void* x, const int32_t* perm, const uint16_t* perm16,
                        const uint8_t* w_tiled, const float* scales_gm, const uint8_t* zeros_gm,
                        void* y, int64_t M, int64_t N, int64_t K, int64_t gs, void* workspace,
                        size_t ws_bytes, size_t part_offset, hipStream_t stream, bool bf16) {
  if (perm && !tgemm_gather_supported(M, K)) return hipErrorInvalidValue;
  if (bf16 && (perm || !tgemm_bf16_supported(M, N, K, gs))) return hipErrorInvalidValue;
  TgemmConfig c = tgemm_config(M, N, K, gs, perm != nullptr);
  if (bf16) {
    // one K range (no workspace): a split configuration runs unsplit
    c.splits = 1;
    c.grid = c.grid_m == 1 ? c.n_wg : (int)((c.n_wg + 7) / 8 * 8 * c.grid_m);
  }
  if (c.splits > 1 && (!workspace || ws_bytes < part_offset + c.ws_split)) {
    c.splits = 1;
    c.grid = c.n_wg;
  }
  TgemmArgs a;
  a.x = (const f16*)x;
  a.perm = perm && perm16 ? reinterpret_cast<const int32_t*>(perm16) : perm;
  a.perm_u16 = perm && perm16 ? 1 : 0;
  a.wt = w_tiled;
  a.s_gm = scales_gm;
  a.z_gm = zeros_gm;
  a.y = (f16*)y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.gs = (int)gs;
  a.n_wg = c.n_wg;
  a.grid_m = c.grid_m;
  a.n_tiles = (int)(4 * ((N + 63) / 64));
  a.splits = c.splits;
  a.counters = (int*)workspace;
  a.part = c.splits > 1 ? (float*)((uint8_t*)workspace + part_offset) : nullptr;
  a.glu = 0;
  if (!derive_args(a)) return hipErrorInvalidValue;
  if (bf16) {
    const dim3 block(kKW * 64);
#define PMI_TG_BF(NTW_)                                                                               \
  hipLaunchKernelGGL((w4a16_tgemm_kernel<1, NTW_, 1, false, false, false, false, true>), dim3(c.grid), \
                     block, 0, stream, a)
    if (c.ntw == 4) PMI_TG_BF(4);
    else if (c.ntw == 2) PMI_TG_BF(2);
    else PMI_TG_BF(1);
#undef PMI_TG_BF
    return hipGetLastError();
  }
  if (c.mt == 1) return launch_mt<1>(c, a, stream);
  if (c.mt == 2) return launch_mt<2>(c, a, stream);
  return launch_mt<4>(c, a, stream);
}


bool tgemm_glu_supported(int64_t M, int64_t N, int64_t K, int64_t gs) {
  if (!tgemm_supported(M, N, K, gs) || M > 16 || N % 64 != 0) return false;
  const TgemmConfig c = tgemm_config(M, N, K, gs, false);
  return c.mt == 1 && c.ntw == 4 && !c.rng && c.splits == 1 && c.grid_m == 1;
}

hipError_t launch_tgemm_glu(const void* x, const uint8_t* w_tiled, const float* scales_gm,
                            const uint8_t* zeros_gm, void* y, int64_t M, int64_t N, int64_t K,
                            int64_t gs, hipStream_t stream) {
  if (!tgemm_glu_supported(M, N, K, gs)) return hipErrorInvalidValue;
  const TgemmConfig c = tgemm_config(M, N, K, gs, false);
  TgemmArgs a;
  a.x = (const f16*)x;
  a.perm = nullptr;
  a.perm_u16 = 0;
  a.wt = w_tiled;
  a.s_gm = scales_gm;
  a.z_gm = zeros_gm;
  a.y = (f16*)y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.gs = (int)gs;
  a.n_wg = c.n_wg;
  a.grid_m = c.grid_m;
  a.n_tiles = (int)(4 * (N / 64));
  a.splits = 1;
  a.counters = nullptr;
  a.part = nullptr;
  a.glu = 1;
  if (!derive_args(a)) return hipErrorInvalidValue;
  return launch_mt<1>(c, a, stream);
}

// The residual add and RMSNorm in the tiled GEMM (up to 4 rows, K <= 4096,
// gs % 128 == 0), where the plain launch takes one K range and one activation
// block (so that both add the same products in the same order; a K split
// would also form the norm once per range).
bool tgemm_norm_supported(int64_t M, int64_t N, int64_t K, int64_t gs, bool glu) {
  if (!tgemm_supported(M, N, K, gs) || M > 4 || K > 4096 || gs % 128 != 0) return false;
  const TgemmConfig c = tgemm_config(M, N, K, gs, false);
  if (c.mt != 1 || c.rng || c.grid_m != 1 || c.splits > 1) return false;
  return !glu || (c.ntw == 4 && N % 64 == 0);
}

hipError_t launch_tgemm_norm(const void* x, const void* r, const void* norm_w, float eps, void* h_out,
                             const uint8_t* w_tiled, const float* scales_gm, const uint8_t* zeros_gm,
                             void* y, int64_t M, int64_t N, int64_t K, int64_t gs, bool glu,
                             hipStream_t stream) {
  if (!tgemm_norm_supported(M, N, K, gs, glu)) return hipErrorInvalidValue;
  const TgemmConfig c = tgemm_config(M, N, K, gs, false);
  TgemmArgs a;
  a.x = (const f16*)x;
  a.perm = nullptr;
  a.perm_u16 = 0;
  a.wt = w_tiled;
  a.s_gm = scales_gm;
  a.z_gm = zeros_gm;
  a.y = (f16*)y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.gs = (int)gs;
  a.n_wg = c.n_wg;
  a.grid_m = 1;
  a.n_tiles = (int)(4 * ((N + 63) / 64));
  a.splits = 1;
  a.counters = nullptr;
  a.part = nullptr;
  a.glu = glu ? 1 : 0;
  a.r = (const f16*)r;
  a.nw = (const f16*)norm_w;
  a.h_out = (f16*)h_out;
  a.eps = eps;
  if (!derive_args(a)) return hipErrorInvalidValue;
  if (c.ntw == 4) return launch_norm_variant<4>(c, a, stream);
  if (c.ntw == 2) return launch_norm_variant<2>(c, a, stream);
  return launch_norm_variant<1>(c, a, stream);
}

}  // namespace pmi
