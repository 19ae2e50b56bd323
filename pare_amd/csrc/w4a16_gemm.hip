// Split-K MFMA INT4 W4A16 GEMM for M > 4, gfx950 (v_mfma_f32_16x16x32_f16).
//
// Work layout. A workgroup is 4 compute waves and 4 producer waves (two waves
// per SIMD) and owns 128 weight rows (a "tile"; 64 with NT = 2) for up to 64
// activation rows (MT MFMA row tiles of 16), over a contiguous range of
// "units". A unit is 128
// columns of K: 64 bytes of every packed row (kernel layout), i.e. columns
// k0+64c+b (low nibble of byte b) and k0+gs/2+64c+b (high nibble), b < 64, of
// the group starting at k0. Units are consumed in pairs: compute wave w takes
// weight rows 16 NT (w&1)..+16 NT - 1 (NT 16-row MFMA tiles) of the pair's unit w>>1,
// so each wave reads from LDS only the activations of its own units and every
// activation fragment it reads feeds four weight tiles. The two k-parities
// are added through LDS at the end. The producer waves only issue the copies
// and wait for them. With K split over `splits` workgroups per tile, the grid
// is tiles x splits.
//
// Operands. Lane l holds 16 bytes of each of its four weight tiles per unit
// (row l%16, bytes 16*(l/16)..+15). Each k-step takes 8 of those bytes and one
// nibble run (low or high): the B operand is 8 fp16 halves (1024 + q) -
// (1024 + z) = q - z, exact, built with v_perm_b32 under a 0x64 exponent byte
// and one packed subtract per pair. Their columns are 8 consecutive
// activations, so the A operand is one 16-byte LDS read. Products x*(q - z) are
// exact in fp32; per unit y += s * sum x*(q - z), the reference's
// w = (q - z) * s with fp32 accumulation.
//
// Pipeline. Everything a unit needs - its activation tile (16*MT rows x 256
// bytes, 16-byte chunks XOR-swizzled per row so the A reads of 16 rows hit 16
// bank groups), its 128 x 64 weight bytes, and the scale and zero-point words
// of its 128 rows - goes straight from memory into an LDS slot with
// buffer_load ... lds (no VGPRs in flight). P pairs of slots form a ring; at
// each step the producers wait for their copies of the oldest pair with an
// explicit vmcnt, everyone crosses one plain s_barrier (which also frees the
// pair computed in the previous step), the producers issue the pair P-1
// steps ahead and the compute waves compute. Loads are unconditional (ranges
// are clamped, never branched around) and the steady-state loops are
// straight-line code.
//
// Split-K. Every split stores its fp32 partial tile (lane-contiguous, coalesced)
// in the caller's workspace and bumps the tile's counter; the last workgroup to
// arrive adds the partials in split order (deterministic), writes fp16 Y and
// resets the counter, so the workspace stays valid for the next call.
//
// Semantics follow the reference Triton kernel (pare/kernels/matmul_int4.py:
// 105-176): w = (q - zero) * scale per group, fp32 accumulation, fp16 output.
#include <stdlib.h>

#include <type_traits>

#include "pmi_common.h"
#include "pmi_launch.h"

namespace pmi {
namespace {

constexpr int kWaves = 4;               // compute waves per workgroup
constexpr int kProducers = 4;           // copy-issuing waves per workgroup
constexpr int kBN = 128;                // weight rows per workgroup
constexpr int kThreads = (kWaves + kProducers) * 64;

// LDS rings (units are consumed in pairs, one unit per k parity):
//   weights of a pair - 128 rows x 128 bytes, each row's 8 chunks of 16 bytes
//   XOR-swizzled by row % 8 - then the scale and zero words of its two units,
//   kWPair bytes, PW slots;
//   activations of a unit, kX bytes, 2*PX slots.
// Weights come from HBM and get the deep ring; activations are re-read from
// L2 by every workgroup and get a shallow one. A pair's two units are 128
// contiguous bytes of every packed row: each weight copy fetches whole cache
// lines (8 rows x 128 bytes), which the DRAM serves far better than the 64-byte
// halves one unit would give.
template <int MT, int NT>
struct Tiling {
  static constexpr int R = 16 * MT;                             // activation rows
  static constexpr int kX = R * 256;                            // activation tile of a unit
  static constexpr int PW = MT == 4 ? 5 : 6;                    // weight pairs in the ring
  // activation pairs in the ring: with 64-row weight tiles (NT = 2) the
  // weight slots are half as large, which leaves room for a third activation
  // pair (M = 64 gate_proj on MI355X: 18.6 us against 20.2 us with two)
  static constexpr int PX = MT == 4 ? (NT == 2 ? 3 : 2) : 3;
  // per weight producer per pair: 2 NT copies of 8 rows, NT scale/zero copies
  static constexpr int kWCopies = 3 * NT;
  static constexpr int kXCopies = 4 * MT;                       // per activation producer per pair
};

struct GemmArgs {
  const f16* x;
  const uint8_t* w;
  const float* s;
  const void* z;
  const float* s_gm;    // optional group-major copies: fp32 [G, N]
  const uint8_t* z_gm;  //                              u8 [G, N]
  f16* y;
  float* part;    // split-K partial tiles (splits > 1)
  int* counters;  // one per (m-block, tile), zero between calls
  int M, N, K, gs, splits, n_tiles, grid_m;
};

template <int I, int N, class F>
PMI_DEV void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// SZT: scales and zero points come from the group-major copies (one unit's
// 128 rows are 512 + 128 contiguous bytes) instead of a gather over 128 rows
// of the [N, G] arrays. NT: 16-row weight tiles per compute wave, 4 (tiles of
// 128 rows) or 2 (tiles of 64 rows, twice the tiles for the same N: with
// MT = 4 one pass over the CUs without a K split at 33-64 activation rows).
template <int MT, bool ZU8, bool SZT, int NT>
__global__ __launch_bounds__(kThreads, 1) void w4a16_gemm_kernel(GemmArgs a) {
  constexpr int kNT = NT, kBN = 32 * NT, R2 = 16 * NT, HALVES = NT / 2;
  constexpr int kSBytes = kBN * 4, kZBytes = kBN * 4;
  constexpr int kWLines = kBN * 128, kWPair = kWLines + 2 * (kSBytes + kZBytes);
  using T = Tiling<MT, NT>;
  constexpr int R = T::R, kX = T::kX, PW = T::PW, PX = T::PX;
  constexpr int kWC = T::kWCopies, kXC = T::kXCopies;
  static_assert(PW >= 2 && (PW - 1) * kWC < 64 && PX >= 2 && (PX - 1) * kXC < 64,
                "copies in flight per producer wave fit vmcnt (63)");
  static_assert(PW * kWPair + 2 * PX * kX <= 160 * 1024, "LDS budget");
  static_assert(2 * MT * kNT * 64 * 16 <= PW * kWPair, "k-parity reduction fits the weight ring");
  __shared__ __attribute__((aligned(16))) uint8_t wring[PW * kWPair];
  __shared__ __attribute__((aligned(16))) uint8_t xring[2 * PX * kX];
  __shared__ int last_flag;

  const int tid = threadIdx.x, l = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the copies' LDS base is M0
  // waves 0..3 compute, 4 and 5 copy weights (+ scales, zero points), 6 and 7
  // copy activations
  const bool producer = wv >= kWaves;
  const bool wprod = wv == 4 || wv == 5, xprod = wv >= 6;
  const int pw = wv & 1;                                     // index within a producer pair
  const int rh = wv & 1;                                     // compute: row half
  const int kp = producer ? 2 : (wv >> 1);                   // compute: k parity
  const int kq = l >> 4, ln = l & 15;
  const int bid = blockIdx.x;
  const int sp = bid % a.splits;
  // (tile, m-block) of this workgroup. Workgroups are dealt to the 8 XCDs
  // round-robin by index, so the m-blocks of one tile are numbered 8 apart:
  // they then share an XCD and its L2, and the second read of the tile's
  // weights hits there. (Only a placement preference: correctness does not
  // depend on it.)
  const int tl = bid / a.splits;
  int tile, mb;
  {
    const int gm = a.grid_m, full = (a.n_tiles / 8) * 8;
    if (tl < full * gm) {
      const int r = tl % (8 * gm);
      tile = (tl / (8 * gm)) * 8 + (r & 7);
      mb = r >> 3;
    } else {
      const int rem = a.n_tiles - full, r = tl - full * gm;
      tile = full + r % rem;
      mb = r / rem;
    }
  }
  const int M = a.M, N = a.N, K = a.K, gs = a.gs;
  const int units = K >> 7;  // even (K % 256 == 0): every pair is whole
  const int u_begin = 2 * (int)((int64_t)sp * (units >> 1) / a.splits);
  const int u_end = 2 * (int)((int64_t)(sp + 1) * (units >> 1) / a.splits);
  const int upg = gs >> 7;
  const int G = K / gs;
  const int row_bytes = K >> 1;
  const int n_pairs = (u_end - u_begin) >> 1;

  f32x4 acc[MT][kNT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < kNT; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  if (wprod) {
    // ---- weight producer pw: rows R2*pw .. +R2-1 as 2 NT copies of 8 rows x
    // 128 bytes (lane l: row 8i + l/8, chunk l%8 of the LDS row, which holds
    // the pair's chunk (l%8) ^ (row%8)), and the scale (pw 0) or zero-point
    // (pw 1) words of the tile's rows, 64 per copy, of both units
    const __amdgpu_buffer_rsrc_t rw = rsrc(a.w, (int64_t)N * row_bytes);
    int vl[2 * NT];
#pragma unroll
    for (int i = 0; i < 2 * NT; ++i) {
      const int rloc = R2 * pw + 8 * i + (l >> 3);
      int n = tile * kBN + rloc;
      n = n < N ? n : N - 1;
      vl[i] = n * row_bytes + 16 * ((l & 7) ^ (rloc & 7));
    }
    const bool scale = pw == 0;
    __amdgpu_buffer_rsrc_t rsz;
    int gmul, vsz[HALVES];
    if constexpr (SZT) {
      // scales: rows h*64 + l; zero bytes: rows h*64 + 4l .. +3 (lanes 16..63
      // repeat lanes 0..15; rows past N are clamped into the array, N % 4 == 0)
      rsz = scale ? rsrc(a.s_gm, (int64_t)G * N * 4) : rsrc(a.z_gm, (int64_t)G * N);
      gmul = scale ? 4 * N : N;  // bytes per group
#pragma unroll
      for (int h = 0; h < HALVES; ++h) {
        int n = scale ? tile * kBN + 64 * h + l : tile * kBN + 64 * h + 4 * (l & 15);
        const int nmax = scale ? N - 1 : N - 4;
        n = n < nmax ? n : nmax;
        vsz[h] = scale ? 4 * n : n;
      }
    } else {
      // u8 zero points are fetched as the aligned word holding the byte; an
      // aligned word never crosses a page, so it lies in the zeros' allocation
      rsz = scale ? rsrc(a.s, (int64_t)N * G * 4)
                  : rsrc(a.z, ZU8 ? (((int64_t)N * G + 3) & ~(int64_t)3) : (int64_t)N * G * 4);
      gmul = (scale || !ZU8) ? 4 : 1;  // bytes per (row, group) entry
#pragma unroll
      for (int h = 0; h < HALVES; ++h) {
        int n = tile * kBN + 64 * h + l;
        n = n < N ? n : N - 1;
        vsz[h] = n * G * gmul;
      }
    }
    // slot: [weight lines 128 x 128 B][unit 0: scales, zero words][unit 1: ...]
    auto issue_pair = [&](int slot, int q) {
      uint8_t* base = wring + slot * kWPair;
      int u0 = u_begin + 2 * q;
      u0 = u0 < u_end - 2 ? u0 : u_end - 2;
      const int woff = __builtin_amdgcn_readfirstlane(u0 * 64);
#pragma unroll
      for (int i = 0; i < 2 * NT; ++i)
        copy_to_lds<16>(rw, base + (R2 * pw + 8 * i) * 128, vl[i], woff);
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int g = (u0 + e) / upg;
        uint8_t* sz = base + kWLines + e * (kSBytes + kZBytes) + pw * kSBytes;
#pragma unroll
        for (int h = 0; h < HALVES; ++h) {
          if constexpr (SZT)
            copy_to_lds<4>(rsz, sz + h * 256, vsz[h], __builtin_amdgcn_readfirstlane(g * gmul));
          else
            copy_to_lds<4>(rsz, sz + h * 256, (vsz[h] + g * gmul) & ~3, 0);
        }
      }
    };
    // pairs 0 .. PW-2 in flight; step q waits for pair q and issues pair
    // q+PW-1 (clamped past the range) into the slot pair q-1 used
    for (int q = 0; q < PW - 1; ++q) issue_pair(q, q);
    int slot = PW - 1;
    for (int q = 0; q < n_pairs; ++q) {
      wait_vmcnt<(PW - 2) * kWC>();
      barrier_only();
      issue_pair(slot, q + PW - 1);
      slot = slot + 1 == PW ? 0 : slot + 1;
    }
    wait_vmcnt<0>();  // clamped copies past the range may still be landing
  } else if (xprod) {
    // ---- activation producer pw: tile rows 4*(pw*2*MT + r) .. +3, 16 chunks
    // each; LDS chunk p of row m holds activation chunk p ^ (m % 16)
    const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (int64_t)M * K * 2);
    int vx[2 * MT];
#pragma unroll
    for (int r = 0; r < 2 * MT; ++r) {
      const int mloc = 4 * (pw * 2 * MT + r) + (l >> 4);
      const int c = (l & 15) ^ (mloc & 15);
      int mg = mb * R + mloc;
      mg = mg < M ? mg : M - 1;
      vx[r] = mg * K * 2 + (c >> 3) * gs + 16 * (c & 7);
    }
    auto issue_unit = [&](int slot, int u) {
      uint8_t* base = xring + slot * kX;
      u = u < u_end ? u : u_end - 1;
      const int g = u / upg;
      const int xoff = __builtin_amdgcn_readfirstlane((g * gs + 64 * (u - g * upg)) * 2);
#pragma unroll
      for (int r = 0; r < 2 * MT; ++r)
        copy_to_lds<16>(rx, base + (pw * 2 * MT + r) * 1024, vx[r], xoff);
    };
    for (int q = 0; q < PX - 1; ++q) {
      issue_unit(2 * q, u_begin + 2 * q);
      issue_unit(2 * q + 1, u_begin + 2 * q + 1);
    }
    int slot = 2 * (PX - 1);
    for (int q = 0; q < n_pairs; ++q) {
      wait_vmcnt<(PX - 2) * kXC>();
      barrier_only();
      issue_unit(slot, u_begin + 2 * (q + PX - 1));
      issue_unit(slot + 1, u_begin + 2 * (q + PX - 1) + 1);
      slot = slot + 2 == 2 * PX ? 0 : slot + 2;
    }
    wait_vmcnt<0>();
  } else {
    // ---- compute wave (row half rh, k parity kp): no copies of its own, so
    // its LDS reads never wait on the copy queue; the step barrier orders them
    int zrow[kNT];
#pragma unroll
    for (int j = 0; j < kNT; ++j) {
      int n = tile * kBN + R2 * rh + 16 * j + ln;
      n = n < N ? n : N - 1;
      zrow[j] = n * G;
    }
    int wslot = 0, xslot = kp;
    for (int q = 0; q < n_pairs; ++q) {
      barrier_only();  // every copy of pair q is in; every wave is done with pair q-1
      const int u = u_begin + 2 * q + kp;
      if (u < u_end) {
        const uint8_t* wb = wring + wslot * kWPair;
        const uint8_t* szb = wb + kWLines + kp * (kSBytes + kZBytes);
        const uint8_t* xb = xring + xslot * kX;
        const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
        const int g = u / upg;
        u32x4 w[kNT];
        f16x2 nz[kNT];
        float sc[kNT];
#pragma unroll
        for (int j = 0; j < kNT; ++j) {
          const int row = R2 * rh + 16 * j + ln;
          // 16 bytes of this unit: chunk 4*kp + kq of the row's 128, swizzled
          w[j] = *reinterpret_cast<const u32x4*>(wb + row * 128 + 16 * ((4 * kp + kq) ^ (row & 7)));
          sc[j] = *reinterpret_cast<const float*>(szb + 4 * row);
          uint32_t z;
          if constexpr (SZT) {
            z = szb[kSBytes + 256 * (row >> 6) + (row & 63)];  // rows 64h + 4l.. at 256h + 4l
          } else {
            const uint32_t zw = *reinterpret_cast<const uint32_t*>(szb + kSBytes + 4 * row);
            z = ZU8 ? (zw >> (((zrow[j] + g) & 3) * 8)) & 0xFFu
                    : (uint32_t)(int)__builtin_bit_cast(float, zw);
          }
          nz[j] = as_f16x2(neg_magic_zero_x2(z));
        }
        f32x4 cg[MT][kNT];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const int run = t >> 1, half = t & 1;
          const int c = run * 8 + 2 * kq + half;
          f16x8 A[MT];
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
            A[mt] = *reinterpret_cast<const f16x8*>(xb + (16 * mt + ln) * 256 + ((c ^ ln) << 4));
#pragma unroll
          for (int j = 0; j < kNT; ++j) {
            const uint32_t w0 = w[j][2 * half], w1 = w[j][2 * half + 1];
            const uint32_t t0 = (run ? (w0 >> 4) : w0) & 0x0F0F0F0Fu;
            const uint32_t t1 = (run ? (w1 >> 4) : w1) & 0x0F0F0F0Fu;
            const f16x8 B = b_operand(t0, t1, nz[j]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              cg[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mt], B, t == 0 ? zero4 : cg[mt][j],
                                                                 0, 0, 0);
          }
        }
#pragma unroll
        for (int j = 0; j < kNT; ++j)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mt][j][i] = fmaf(sc[j], cg[mt][j][i], acc[mt][j][i]);
      }
      wslot = wslot + 1 == PW ? 0 : wslot + 1;
      xslot = xslot + 2 >= 2 * PX ? xslot + 2 - 2 * PX : xslot + 2;
    }
  }

  // ---- k-parity reduction through LDS --------------------------------------
  __syncthreads();
  {
    f32x4* red = reinterpret_cast<f32x4*>(wring);
    if (kp == 1) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < kNT; ++j) red[((rh * MT + mt) * kNT + j) * 64 + l] = acc[mt][j];
    }
    __syncthreads();
    if (kp == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < kNT; ++j) acc[mt][j] += red[((rh * MT + mt) * kNT + j) * 64 + l];
    }
  }

  // ---- epilogue (waves of k parity 0 hold the sums) ------------------------
  const int n0 = tile * kBN + R2 * rh + ln;
  const int m0 = mb * R + 4 * kq;
  if (a.splits > 1) {
    // Partial tile of split sp: [row half][mt][j][lane] x 16 bytes (each lane's
    // f32x4 contiguous, a wave's store one 1 KiB run). Stores and loads carry
    // the device-scope cache policy (sc1), like agent-scope atomics: they are
    // coherent across the XCDs' L2 caches without a release fence, whose L2
    // write-back would cost far more than the tile. The s_waitcnt makes every
    // store of this thread complete before the barrier, and the barrier
    // orders them before the counter increment.
    constexpr int kPartBytes = 2 * MT * kNT * 64 * 16;
    const __amdgpu_buffer_rsrc_t rp =
        rsrc(a.part + (size_t)tl * a.splits * (kPartBytes / 4), (int64_t)a.splits * kPartBytes);
    const int vlane = (rh * MT * kNT * 64 + l) * 16;
    constexpr int kSc1 = 16;
    if (kp == 0) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < kNT; ++j)
          __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mt][j]), rp,
                                                 vlane + (mt * kNT + j) * 1024,
                                                 __builtin_amdgcn_readfirstlane(sp * kPartBytes), kSc1);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const int old = __hip_atomic_fetch_add(&a.counters[tl], 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
      last_flag = old == a.splits - 1;
    }
    __syncthreads();
    if (!last_flag) return;
    if (kp != 0) return;
    // Last to arrive: sum the partials in split order (deterministic). Every
    // split's partial, this one's included, is in the workspace. The loads of
    // kB splits are issued together, so the sum costs one round trip per kB
    // splits rather than one per split; kB keeps them within 64 VGPRs.
    constexpr int kB = MT * kNT >= 16 ? 1 : 16 / (MT * kNT);
    f32x4 tot[MT][kNT] = {};
    for (int q0 = 0; q0 < a.splits; q0 += kB) {
      f32x4 part[kB][MT][kNT];
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const int q = q0 + b < a.splits ? q0 + b : a.splits - 1;  // past the end: loaded, not added
        const int soff = __builtin_amdgcn_readfirstlane(q * kPartBytes);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < kNT; ++j)
            part[b][mt][j] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, vlane + (mt * kNT + j) * 1024, soff, kSc1));
      }
      // the adds select rather than break: behind the break the compiler sank
      // the loads of later splits to their adds, one round trip per split
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int b = 0; b < kB; ++b) {
        const bool use = q0 + b < a.splits;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < kNT; ++j) {
            const f32x4 t = q0 + b == 0 ? part[b][mt][j] : tot[mt][j] + part[b][mt][j];
            tot[mt][j] = use ? t : tot[mt][j];
          }
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < kNT; ++j) acc[mt][j] = tot[mt][j];
    if (tid == 0) __hip_atomic_store(&a.counters[tl], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (kp != 0) return;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < kNT; ++j) {
      const int n = n0 + 16 * j;
      if (n >= N) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * mt + i;
        if (m < M) a.y[(size_t)m * N + n] = f32_to_f16_rne(acc[mt][j][i]);
      }
    }
}

// X[:, perm] for act_order layers, 8 columns per thread.
__global__ void gather_cols_kernel(const f16* __restrict__ x, const int32_t* __restrict__ perm,
                                   f16* __restrict__ out, int M, int K) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_row = K / 8;
  if (i >= (int64_t)M * per_row) return;
  const int m = (int)(i / per_row), k0 = (int)(i % per_row) * 8;
  const f16* row = x + (size_t)m * K;
  f16x8 v;
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = row[perm_col(perm, k0 + e, K)];
  *reinterpret_cast<f16x8*>(out + (size_t)m * K + k0) = v;
}

int env_int(const char* name, int dflt) {
  const char* s = getenv(name);
  return (s && *s) ? atoi(s) : dflt;
}

int device_cus() {
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

// The workspace starts with a fixed block of split-K counters that nothing else
// ever writes, so counters left at zero by one call are zero for the next one
// whatever shapes the workspace served in between.
constexpr size_t kCounterBytes = kWsCounterBytes;
constexpr int64_t kMaxCounters = kCounterBytes / 4;

template <int MT, int NT>
hipError_t launch_mt(const GemmConfig& c, const GemmArgs& a, int zero_u8, hipStream_t stream) {
  if (a.s_gm)
    hipLaunchKernelGGL((w4a16_gemm_kernel<MT, true, true, NT>), dim3(c.grid), dim3(kThreads), 0,
                       stream, a);
  else if (zero_u8)
    hipLaunchKernelGGL((w4a16_gemm_kernel<MT, true, false, NT>), dim3(c.grid), dim3(kThreads), 0,
                       stream, a);
  else
    hipLaunchKernelGGL((w4a16_gemm_kernel<MT, false, false, NT>), dim3(c.grid), dim3(kThreads), 0,
                       stream, a);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_gather_cols(const void* x, const int32_t* perm, void* out, int64_t M, int64_t K,
                              hipStream_t stream) {
  const int64_t threads = M * (K / 8);
  hipLaunchKernelGGL(gather_cols_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     stream, (const f16*)x, perm, (f16*)out, (int)M, (int)K);
  return hipGetLastError();
}

GemmConfig gemm_config(int64_t M, int64_t N, int64_t K, int64_t gs, bool has_perm) {
  (void)gs;
  GemmConfig c;
  // 33..64 rows: two 32-row m-blocks per tile when that grid still fits one
  // pass over the CUs (it needs fewer K splits, whose partial tiles are added
  // at the end); otherwise one 64-row block, which reads the weights once.
  static const int env_mt = env_int("PMI_GEMM_MT", 0);
  static const int env_nt = env_int("PMI_GEMM_NT", 0);
  const int64_t n_tiles = (N + kBN - 1) / kBN;
  // 33..64 rows with N <= 16384: one 64-row block over 64-row weight tiles
  // (NT = 2): twice the tiles of 128-row ones, and every B operand built once
  // for four activation tiles instead of two. Measured on MI355X at M = 64
  // (48 weight copies beyond the MALL): o/q 12.2 us against 12.9 us for two
  // 32-row blocks, fused q/k/v 13.8 against 14.7, gate 20.0 against 20.3.
  const bool wide64 = M > 32 && M <= 64 && N <= 16384;
  c.m_tiles = M <= 16 ? 1 : (M <= 32 ? 2 : (wide64 ? 4 : (M <= 64 && 2 * n_tiles <= device_cus() ? 2 : 4)));
  if (env_mt == 1 || env_mt == 2 || env_mt == 4) c.m_tiles = env_mt;
  const int64_t bm = 16 * c.m_tiles;
  c.grid_m = (int)((M + bm - 1) / bm);
  c.n_t = c.m_tiles == 4 && (env_nt == 2 || (env_nt == 0 && wide64)) ? 2 : 4;
  const int64_t bn = 32 * c.n_t;
  c.n_tiles = (int)((N + bn - 1) / bn);
  const int64_t units = K / 128;
  const int64_t tiles = (int64_t)c.n_tiles * c.grid_m;
  static const int env_s = env_int("PMI_GEMM_SPLITS", 0);
  static const int env_occ = env_int("PMI_GEMM_OCC", 1);
  int64_t s = env_s > 0 ? env_s : ((int64_t)device_cus() * (env_occ > 0 ? env_occ : 1)) / tiles;
  if (s > units / 2) s = units / 2;
  if (s > 16) s = 16;
  if (s < 1 || tiles > kMaxCounters) s = 1;
  c.splits = (int)s;
  c.grid = (int)(tiles * c.splits);
  c.ws_perm = has_perm ? ws_perm_bytes(M, K) : 0;
  c.ws_split = c.splits > 1 ? ws_align((size_t)tiles * c.splits * bm * bn * 4) : 0;
  return c;
}

size_t gemm_workspace_bytes(int64_t M, int64_t N, int64_t K, int64_t gs, bool has_perm) {
  const GemmConfig c = gemm_config(M, N, K, gs, has_perm);
  if (c.ws_split + c.ws_perm == 0) return 0;
  return kCounterBytes + c.ws_perm + c.ws_split;
}

hipError_t launch_gemm(const void* x, const uint8_t* w, const float* scales, const void* zeros,
                       int zero_u8, const float* scales_gm, const uint8_t* zeros_gm,
                       const int32_t* perm, void* y, int64_t M, int64_t N, int64_t K, int64_t gs,
                       void* workspace, size_t ws_bytes, hipStream_t stream) {
  GemmConfig c = gemm_config(M, N, K, gs, perm != nullptr);
  // workspace: [counters, kCounterBytes][X[:, perm] (act_order)][partial tiles]
  uint8_t* ws = (uint8_t*)workspace;
  if (c.ws_perm && ws_bytes < kCounterBytes + c.ws_perm) return hipErrorInvalidValue;
  // Without room for the partial tiles the kernel runs unsplit.
  if (c.splits > 1 && ws_bytes < kCounterBytes + c.ws_perm + c.ws_split) {
    c.splits = 1;
    c.grid = c.n_tiles * c.grid_m;
  }
  const f16* xp = (const f16*)x;
  if (perm) {
    // act_order: gather X[:, perm] once into the workspace
    f16* xg = (f16*)(ws + kCounterBytes);
    hipError_t e = launch_gather_cols(xp, perm, xg, M, K, stream);
    if (e != hipSuccess) return e;
    xp = xg;
  }
  GemmArgs a;
  a.x = xp;
  a.w = w;
  a.s = scales;
  a.z = zeros;
  // the group-major copies are read as whole words of 4 rows
  const bool gm = scales_gm && zeros_gm && N % 4 == 0;
  a.s_gm = gm ? scales_gm : nullptr;
  a.z_gm = gm ? zeros_gm : nullptr;
  a.y = (f16*)y;
  a.counters = (int*)ws;
  a.part = c.splits > 1 ? (float*)(ws + kCounterBytes + c.ws_perm) : nullptr;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.gs = (int)gs;
  a.splits = c.splits;
  a.n_tiles = c.n_tiles;
  a.grid_m = c.grid_m;
  if (c.m_tiles == 1) return launch_mt<1, 4>(c, a, zero_u8, stream);
  if (c.m_tiles == 2) return launch_mt<2, 4>(c, a, zero_u8, stream);
  if (c.n_t == 2) return launch_mt<4, 2>(c, a, zero_u8, stream);
  return launch_mt<4, 4>(c, a, zero_u8, stream);
}

}  // namespace pmi
