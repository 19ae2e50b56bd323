// Split-K MFMA INT4 W4A16 GEMM for M > 4, gfx950 (v_mfma_f32_16x16x32_f16).
//
// Work layout. A workgroup is 4 waves and owns 128 weight rows (a "tile") for up
// to 64 activation rows (MT MFMA row tiles of 16), over a contiguous range of
// "units". A unit is 128 columns of K: 64 bytes of every packed row (kernel
// layout), i.e. columns k0+64c+b (low nibble of byte b) and k0+gs/2+64c+b (high
// nibble), b < 64, of the group starting at k0. Units are consumed in pairs:
// wave w takes weight rows 64*(w&1)..+63 (four 16-row MFMA tiles) of the pair's
// unit w>>1, so each wave reads from LDS only the activations of its own units
// and every activation fragment it reads feeds four weight tiles. The two
// k-parities are added through LDS at the end. With K split over `splits`
// workgroups per tile, the grid is tiles x splits.
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
// buffer_load ... lds (no VGPRs in flight). P pairs of slots form a ring; each
// step waits for its own copies of the oldest pair with an explicit vmcnt,
// crosses one plain s_barrier (which also frees the pair computed in the
// previous step) and issues the pair P-1 steps ahead. Loads are
// unconditional (ranges are clamped, never branched around) and the
// steady-state loop is straight-line code.
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

constexpr int kWaves = 4;               // waves per workgroup
constexpr int kNT = 4;                  // 16-row weight tiles per wave
constexpr int kBN = 128;                // weight rows per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kWBytes = kBN * 64;       // weight bytes of one unit
constexpr int kSBytes = kBN * 4;        // scales of one unit
constexpr int kZBytes = kBN * 4;        // zero-point words of one unit

template <int MT>
struct Tiling {
  static constexpr int R = 16 * MT;                          // activation rows
  static constexpr int kX = R * 256;                         // activation tile of a unit
  static constexpr int kSlot = kX + kWBytes + kSBytes + kZBytes;
  static constexpr int kPair = 2 * kSlot;
  static constexpr int P = MT == 1 ? 5 : (MT == 2 ? 4 : 3);  // unit pairs in the ring
  static constexpr int kCopies = MT + 3;                     // copies per wave per unit
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
  int M, N, K, gs, splits, n_tiles;
};

typedef __attribute__((address_space(3))) void* lds_ptr;

PMI_DEV __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
PMI_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | 0xF00 | ((N >> 4) << 14));
}

// BYTES (4 or 16) per lane from a buffer straight into LDS (buffer_load_dword /
// _dwordx4 ... lds): lane i writes lds + BYTES*i; `lds` must be wave-uniform
// (it is M0). The builtin only exists for the device; the host pass, which
// only needs the kernels' launch stubs, sees an empty body.
template <int BYTES>
PMI_DEV void copy_to_lds(__amdgpu_buffer_rsrc_t r, void* lds, int voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  static_assert(BYTES == 4 || BYTES == 16, "dword or dwordx4 copies");
  if constexpr (BYTES == 16)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)lds, 16, voff, soff, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)lds, 4, voff, soff, 0, 0);
#else
  (void)r, (void)lds, (void)voff, (void)soff;
#endif
}

template <int I, int N, class F>
PMI_DEV void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

// Workgroup barrier without the fence of __syncthreads(): that fence counts
// in-flight buffer->LDS copies as pending LDS stores and would drain the whole
// ring at every step. Callers order memory themselves (vmcnt waits before,
// operands consumed before); the clobber keeps the compiler from moving
// memory accesses across it.
PMI_DEV void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// The value of v, hidden from the optimiser (no instruction is emitted).
PMI_DEV int opaque(int v) {
  asm("" : "+v"(v));
  return v;
}

// B operand: 8 nibbles (one run of two words) as fp16 (q - z).
PMI_DEV f16x8 b_operand(uint32_t t0, uint32_t t1, f16x2 nz) {
  const uint32_t K = 0x64646464u;
  const f16x2 h0 = as_f16x2(__builtin_amdgcn_perm(K, t0, 0x04010400u)) + nz;
  const f16x2 h1 = as_f16x2(__builtin_amdgcn_perm(K, t0, 0x04030402u)) + nz;
  const f16x2 h2 = as_f16x2(__builtin_amdgcn_perm(K, t1, 0x04010400u)) + nz;
  const f16x2 h3 = as_f16x2(__builtin_amdgcn_perm(K, t1, 0x04030402u)) + nz;
  const u32x4 r = {as_u32(h0), as_u32(h1), as_u32(h2), as_u32(h3)};
  return __builtin_bit_cast(f16x8, r);
}

// SZT: scales and zero points come from the group-major copies (one unit's
// 128 rows are 512 + 128 contiguous bytes) instead of a gather over 128 rows
// of the [N, G] arrays.
template <int MT, bool ZU8, bool SZT>
__global__ __launch_bounds__(kThreads, 1) void w4a16_gemm_kernel(GemmArgs a) {
  using T = Tiling<MT>;
  constexpr int R = T::R, kX = T::kX, kSlot = T::kSlot, P = T::P;
  constexpr int kPairCopies = 2 * T::kCopies;
  static_assert(P >= 2 && P <= 5 && (P - 1) * kPairCopies < 64, "pipeline depth");
  static_assert(P * T::kPair <= 160 * 1024, "LDS budget");
  static_assert(2 * MT * kNT * 64 * 16 <= T::kPair, "k-parity reduction fits one pair");
  // one LDS array per pair of ring slots: the compiler tracks each pair's
  // copies apart, so reading one pair never waits for copies into another
  __shared__ __attribute__((aligned(16))) uint8_t lp0[T::kPair], lp1[T::kPair], lp2[T::kPair],
      lp3[T::kPair], lp4[T::kPair];
  __shared__ int last_flag;
  auto pair_ptr = [&](auto PAIR) -> uint8_t* {
    constexpr int q = decltype(PAIR)::value;
    if constexpr (q == 0) return lp0;
    else if constexpr (q == 1) return lp1;
    else if constexpr (q == 2) return lp2;
    else if constexpr (q == 3) return lp3;
    else return lp4;
  };

  const int tid = threadIdx.x, l = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the copies' LDS base is M0
  const int rh = wv & 1, kp = wv >> 1;                       // row half, k parity
  const int kq = l >> 4, ln = l & 15;
  const int bid = blockIdx.x;
  const int sp = bid % a.splits;
  const int tl = bid / a.splits;
  const int tile = tl % a.n_tiles, mb = tl / a.n_tiles;
  const int M = a.M, N = a.N, K = a.K, gs = a.gs;
  const int units = K >> 7;
  const int u_begin = (int)((int64_t)sp * units / a.splits);
  const int u_end = (int)((int64_t)(sp + 1) * units / a.splits);
  const int upg = gs >> 7;
  const int G = K / gs;
  const int row_bytes = K >> 1;

  const __amdgpu_buffer_rsrc_t rw = rsrc(a.w, (int64_t)N * row_bytes);
  const __amdgpu_buffer_rsrc_t rs = rsrc(a.s, (int64_t)N * G * 4);
  // u8 zero points are fetched as the aligned word holding the byte; an
  // aligned word never crosses a page, so it lies in the zeros' allocation
  const __amdgpu_buffer_rsrc_t rz =
      rsrc(a.z, ZU8 ? (((int64_t)N * G + 3) & ~(int64_t)3) : (int64_t)N * G * 4);
  const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (int64_t)M * K * 2);

  // Copies of this wave per unit: weight tiles 2*wv, 2*wv+1; activation rows
  // 4*(wv*MT + r) .. +3 (16 chunks each; LDS chunk p of row m holds activation
  // chunk p ^ (m % 16)); the scale (waves 0, 1) or zero-point (waves 2, 3)
  // words of rows 64*(wv&1) + l.
  int vw[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    int n = tile * kBN + (2 * wv + j) * 16 + ln;
    n = n < N ? n : N - 1;
    vw[j] = n * row_bytes + 16 * kq;
  }
  int vx[MT];
#pragma unroll
  for (int r = 0; r < MT; ++r) {
    const int mloc = 4 * (wv * MT + r) + (l >> 4);
    const int c = (l & 15) ^ (mloc & 15);
    int mg = mb * R + mloc;
    mg = mg < M ? mg : M - 1;
    vx[r] = mg * K * 2 + (c >> 3) * gs + 16 * (c & 7);
  }
  const bool sz_scale = wv < 2;
  __amdgpu_buffer_rsrc_t rsz;
  int gmul, vsz;
  if constexpr (SZT) {
    // waves 0, 1: scales of rows 64*wv + l; waves 2, 3: the zero bytes of rows
    // 64*(wv-2) + 4l .. +3 (lanes 16..63 repeat lanes 0..15; rows past N are
    // clamped into the array, N % 4 == 0)
    rsz = sz_scale ? rsrc(a.s_gm, (int64_t)G * N * 4) : rsrc(a.z_gm, (int64_t)G * N);
    gmul = sz_scale ? 4 * N : N;  // bytes per group
    int n = sz_scale ? tile * kBN + 64 * (wv & 1) + l : tile * kBN + 64 * (wv & 1) + 4 * (l & 15);
    const int nmax = sz_scale ? N - 1 : N - 4;
    n = n < nmax ? n : nmax;
    vsz = sz_scale ? 4 * n : n;
  } else {
    rsz = sz_scale ? rs : rz;
    gmul = (sz_scale || !ZU8) ? 4 : 1;  // bytes per (row, group) entry
    int n = tile * kBN + 64 * (wv & 1) + l;
    n = n < N ? n : N - 1;
    vsz = n * G * gmul;
  }

  // everything unit u needs -> the slot at `base`
  auto issue_unit = [&](uint8_t* base, int u) {
    u = u < u_end ? u : u_end - 1;
    const int g = u / upg;
    const int xoff = __builtin_amdgcn_readfirstlane((g * gs + 64 * (u - g * upg)) * 2);
    const int woff = __builtin_amdgcn_readfirstlane(u * 64);
#pragma unroll
    for (int r = 0; r < MT; ++r) copy_to_lds<16>(rx, base + (wv * MT + r) * 1024, vx[r], xoff);
#pragma unroll
    for (int j = 0; j < 2; ++j) copy_to_lds<16>(rw, base + kX + (2 * wv + j) * 1024, vw[j], woff);
    if constexpr (SZT)
      copy_to_lds<4>(rsz, base + kX + kWBytes + wv * 256, vsz, __builtin_amdgcn_readfirstlane(g * gmul));
    else
      copy_to_lds<4>(rsz, base + kX + kWBytes + wv * 256, (vsz + g * gmul) & ~3, 0);
  };
  auto issue_pair = [&](auto PAIR, int q) {
    uint8_t* base = pair_ptr(PAIR);
    issue_unit(base, u_begin + 2 * q);
    issue_unit(base + kSlot, u_begin + 2 * q + 1);
  };

  // per-lane constants of the compute: this wave's rows and their zero words
  int zrow[kNT];
#pragma unroll
  for (int j = 0; j < kNT; ++j) {
    int n = tile * kBN + 64 * rh + 16 * j + ln;
    n = n < N ? n : N - 1;
    zrow[j] = n * G;
  }

  f32x4 acc[MT][kNT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < kNT; ++j) acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const uint8_t* base, int u) {
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    const int g = u / upg;
    u32x4 w[kNT];
    f16x2 nz[kNT];
    float sc[kNT];
#pragma unroll
    for (int j = 0; j < kNT; ++j) {
      const int row = 64 * rh + 16 * j + ln;
      // Every per-tile LDS offset goes through opaque(): each read is then one
      // offset from the pair array. Folded into a chain of offsets, the later
      // reads lose the LDS alias information and the compiler would wait for
      // every copy in flight before them.
      w[j] = *reinterpret_cast<const u32x4*>(base + opaque(kX + (4 * rh + j) * 1024 + 16 * l));
      sc[j] = *reinterpret_cast<const float*>(base + opaque(kX + kWBytes + 4 * row));
      uint32_t z;
      if constexpr (SZT) {
        z = base[opaque(kX + kWBytes + kSBytes + 256 * rh + 16 * j + ln)];
      } else {
        const uint32_t zw =
            *reinterpret_cast<const uint32_t*>(base + opaque(kX + kWBytes + kSBytes + 4 * row));
        z = ZU8 ? (zw >> (((zrow[j] + g) & 3) * 8)) & 0xFFu : (uint32_t)(int)__builtin_bit_cast(float, zw);
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
        A[mt] = *reinterpret_cast<const f16x8*>(base + (16 * mt + ln) * 256 + ((c ^ ln) << 4));
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
  };

  // Pipeline: pairs 0 .. P-2 in flight before the loop; step q waits for pair
  // q, computes one unit of it per wave and issues pair q+P-1 into the pair
  // array that step q-1 finished with.
  const int nu = u_end - u_begin;
  const int full_pairs = nu >> 1, n_pairs = (nu + 1) >> 1;
  static_for<0, P - 1>([&](auto I) { issue_pair(I, (int)I); });

  int q0 = 0;
  for (; q0 + P <= full_pairs; q0 += P) {
    static_for<0, P>([&](auto I) {
      constexpr int i = decltype(I)::value;
      // pairs q0+i .. q0+i+P-2 are in flight: wait for the oldest
      wait_vmcnt<(P - 2) * kPairCopies>();
      barrier_only();  // every wave's copies of pair q0+i are in; pair array (i+P-1)%P is free
      issue_pair(std::integral_constant<int, (i + P - 1) % P>{}, q0 + i + P - 1);
      compute(pair_ptr(I) + kp * kSlot, u_begin + 2 * (q0 + i) + kp);
    });
  }
  // Remainder: at most P pairs, the last possibly a single unit; only the
  // first can still need its successor issued.
  static_for<0, P>([&](auto I) {
    constexpr int i = decltype(I)::value;
    if (q0 + i < n_pairs) {
      wait_vmcnt<0>();
      barrier_only();
      if (q0 + i + P - 1 < n_pairs) issue_pair(std::integral_constant<int, (i + P - 1) % P>{}, q0 + i + P - 1);
      const int u = u_begin + 2 * (q0 + i) + kp;
      if (u < u_end) compute(pair_ptr(I) + kp * kSlot, u);
    }
  });

  // ---- k-parity reduction through LDS --------------------------------------
  wait_vmcnt<0>();  // clamped copies past the range may still be landing
  __syncthreads();
  {
    f32x4* red = reinterpret_cast<f32x4*>(lp0);
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
  const int n0 = tile * kBN + 64 * rh + ln;
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
    // Last to arrive: sum the partials in split order (deterministic), one
    // round trip per split.
    f32x4 tot[MT][kNT];
    for (int q = 0; q < a.splits; ++q) {
      f32x4 part[MT][kNT];
      if (q == sp) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < kNT; ++j) part[mt][j] = acc[mt][j];
      } else {
        const int soff = __builtin_amdgcn_readfirstlane(q * kPartBytes);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < kNT; ++j)
            part[mt][j] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, vlane + (mt * kNT + j) * 1024, soff, kSc1));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < kNT; ++j) tot[mt][j] = q == 0 ? part[mt][j] : tot[mt][j] + part[mt][j];
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

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

// The workspace starts with a fixed block of split-K counters that nothing else
// ever writes, so counters left at zero by one call are zero for the next one
// whatever shapes the workspace served in between.
constexpr size_t kCounterBytes = 64 * 1024;
constexpr int64_t kMaxCounters = kCounterBytes / 4;

template <int MT>
hipError_t launch_mt(const GemmConfig& c, const GemmArgs& a, int zero_u8, hipStream_t stream) {
  if (a.s_gm)
    hipLaunchKernelGGL((w4a16_gemm_kernel<MT, true, true>), dim3(c.grid), dim3(kThreads), 0, stream, a);
  else if (zero_u8)
    hipLaunchKernelGGL((w4a16_gemm_kernel<MT, true, false>), dim3(c.grid), dim3(kThreads), 0, stream, a);
  else
    hipLaunchKernelGGL((w4a16_gemm_kernel<MT, false, false>), dim3(c.grid), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

}  // namespace

GemmConfig gemm_config(int64_t M, int64_t N, int64_t K, int64_t gs, bool has_perm) {
  (void)gs;
  GemmConfig c;
  c.m_tiles = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int64_t bm = 16 * c.m_tiles;
  c.grid_m = (int)((M + bm - 1) / bm);
  c.n_tiles = (int)((N + kBN - 1) / kBN);
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
  c.ws_perm = has_perm ? align256((size_t)M * K * 2) : 0;
  c.ws_split = c.splits > 1 ? align256((size_t)tiles * c.splits * bm * kBN * 4) : 0;
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
    const int64_t threads = M * (K / 8);
    hipLaunchKernelGGL(gather_cols_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                       stream, xp, perm, xg, (int)M, (int)K);
    hipError_t e = hipGetLastError();
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
  if (c.m_tiles == 1) return launch_mt<1>(c, a, zero_u8, stream);
  if (c.m_tiles == 2) return launch_mt<2>(c, a, zero_u8, stream);
  return launch_mt<4>(c, a, zero_u8, stream);
}

}  // namespace pmi
