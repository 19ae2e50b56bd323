// Split-K MFMA INT4 W4A16 GEMM for M > 4, gfx950 (v_mfma_f32_16x16x32_f16).
//
// Work layout. A workgroup is 4 waves and owns 128 weight rows (a "tile"; each
// wave 2 x 16 rows) for up to 64 activation rows (MT MFMA row tiles of 16), over
// a contiguous range of "units". A unit is 128 columns of K: 64 bytes of every
// packed row (kernel layout), i.e. columns k0+64c+b (low nibble of byte b) and
// k0+gs/2+64c+b (high nibble), b < 64, of the group starting at k0. With K
// split over `splits` workgroups per tile, the grid is tiles x splits.
//
// Operands. Lane l loads 16 bytes of each of its two 16-row weight tiles per
// unit (row l%16, bytes 16*(l/16)..+15) with one buffer_load_dwordx4. Each
// k-step takes 8 bytes of them and one nibble run (low or high): the B operand
// is 8 fp16 halves (1024 + q) - (1024 + z) = q - z, exact, built with v_perm_b32
// under a 0x64 exponent byte and one packed subtract per pair. Their columns
// are 8 consecutive activations, so the A operand is one 16-byte LDS read.
// Products x*(q - z) are exact in fp32; per group y += s * sum x*(q - z), the
// reference's w = (q - z) * s with fp32 accumulation.
//
// Pipeline. The activation tile of a unit (16*MT rows x 256 bytes) is copied
// straight from memory into LDS by the waves' buffer_load ... lds (no VGPRs),
// into D LDS slots with a per-row XOR swizzle of its 16-byte chunks (the A reads
// of 16 rows hit 16 different bank groups). Weights, scales and zero points go
// to a D-deep register ring. Every stage is issued D-1 units ahead with
// unconditional loads (ranges are clamped, never branched around) in a
// straight-line steady-state loop, so each wave waits for exactly its oldest
// stage; one barrier per unit publishes the activation slot and frees the one
// the next DMA overwrites.
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

constexpr int kWaves = 4;              // waves per workgroup
constexpr int kNB = 2;                 // 16-row weight tiles per wave
constexpr int kBN = kWaves * kNB * 16; // weight rows per workgroup
constexpr int kThreads = kWaves * 64;

struct GemmArgs {
  const f16* x;
  const uint8_t* w;
  const float* s;
  const void* z;
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

// 16 bytes per lane from a buffer straight into LDS (buffer_load_dwordx4 ...
// lds): lane i writes lds + 16*i; `lds` must be wave-uniform (it is M0). The
// builtin only exists for the device; the host pass, which only needs the
// kernels' launch stubs, sees an empty body.
PMI_DEV void copy16_to_lds(__amdgpu_buffer_rsrc_t r, void* lds, int voff, int soff) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_ptr)lds, 16, voff, soff, 0, 0);
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
// activation ring at every unit. Callers order memory themselves (vmcnt waits
// before, operands consumed before); the clobber keeps the compiler from
// moving memory accesses across it.
PMI_DEV void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

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

template <int MT, int D, bool UPG1, bool ZU8>
__global__ __launch_bounds__(kThreads, 1) void w4a16_gemm_kernel(GemmArgs a) {
  constexpr int R = 16 * MT;                 // activation rows per workgroup
  constexpr int kXBytes = R * 256;           // activation tile of one unit
  constexpr int kSlot = kXBytes + kWaves * kNB * 1024;  // + weight tiles of one unit
  constexpr int kCopies = MT + kNB;          // buffer->LDS copies per wave per unit
  constexpr int kBatch = 2 * kNB * D;        // scale + zero loads per wave per block
  static_assert(D >= 3 && (D - 2) * kCopies + kBatch < 64, "pipeline depth");
  // one LDS array per ring slot: the compiler tracks each slot's copies apart
  __shared__ __attribute__((aligned(16))) uint8_t xs0[kSlot], xs1[kSlot], xs2[kSlot], xs3[kSlot],
      xs4[kSlot], xs5[kSlot], xs6[kSlot], xs7[kSlot];
  static_assert(D <= 8, "at most 8 LDS slots");
  __shared__ int last_flag;
  auto slot_ptr = [&](auto SLOT) -> uint8_t* {
    constexpr int q = decltype(SLOT)::value;
    if constexpr (q == 0) return xs0;
    else if constexpr (q == 1) return xs1;
    else if constexpr (q == 2) return xs2;
    else if constexpr (q == 3) return xs3;
    else if constexpr (q == 4) return xs4;
    else if constexpr (q == 5) return xs5;
    else if constexpr (q == 6) return xs6;
    else return xs7;
  };

  const int tid = threadIdx.x, l = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: the copies' LDS base is M0
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
  const __amdgpu_buffer_rsrc_t rz = rsrc(a.z, (int64_t)N * G * (ZU8 ? 1 : 4));
  const __amdgpu_buffer_rsrc_t rx = rsrc(a.x, (int64_t)M * K * 2);

  int vw[kNB], vs[kNB], vz[kNB];
#pragma unroll
  for (int j = 0; j < kNB; ++j) {
    int n = tile * kBN + wv * 32 + j * 16 + ln;
    n = n < N ? n : N - 1;
    vw[j] = n * row_bytes + 16 * kq;
    vs[j] = n * G * 4;
    vz[j] = n * G * (ZU8 ? 1 : 4);
  }
  // Copy r of this wave fills tile rows 4*(wv*MT + r) .. +3, 16 chunks each;
  // LDS chunk p of row m holds activation chunk p ^ (m % 16).
  int vx[MT];
#pragma unroll
  for (int r = 0; r < MT; ++r) {
    const int mloc = 4 * (wv * MT + r) + (l >> 4);
    const int c = (l & 15) ^ (mloc & 15);
    int mg = mb * R + mloc;
    mg = mg < M ? mg : M - 1;
    vx[r] = mg * K * 2 + (c >> 3) * gs + 16 * (c & 7);
  }

  // activation and weight tiles of unit u -> LDS slot SLOT
  auto issue = [&](auto SLOT, int u) {
    uint8_t* base = slot_ptr(SLOT);
    u = u < u_end ? u : u_end - 1;
    const int g = u / upg;
    const int xoff = __builtin_amdgcn_readfirstlane((g * gs + 64 * (u - g * upg)) * 2);
    const int woff = __builtin_amdgcn_readfirstlane(u * 64);
#pragma unroll
    for (int r = 0; r < MT; ++r) copy16_to_lds(rx, base + (wv * MT + r) * 1024, vx[r], xoff);
#pragma unroll
    for (int j = 0; j < kNB; ++j) copy16_to_lds(rw, base + kXBytes + (wv * kNB + j) * 1024, vw[j], woff);
  };

  // scales and zero points of units ub .. ub+D-1
  auto load_sz = [&](float (&sc)[D][kNB], uint32_t (&zr)[D][kNB], int ub) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      int u = ub + d;
      u = u < u_end ? u : u_end - 1;
      const int g = __builtin_amdgcn_readfirstlane(u / upg);
#pragma unroll
      for (int j = 0; j < kNB; ++j) {
        sc[d][j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, vs[j], g * 4, 0));
        if constexpr (ZU8)
          zr[d][j] = __builtin_amdgcn_raw_buffer_load_b8(rz, vz[j], g, 0);
        else
          zr[d][j] = __builtin_amdgcn_raw_buffer_load_b32(rz, vz[j], g * 4, 0);
      }
    }
  };

  f32x4 acc[MT][kNB];
  f32x4 cg[MT][kNB];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < kNB; ++j) {
      acc[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      cg[mt][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

  auto compute = [&](auto SLOT, const float (&sc)[kNB], const uint32_t (&zr)[kNB], int u) {
    const uint8_t* xb = slot_ptr(SLOT);
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    u32x4 w[kNB];
    f16x2 nz[kNB];
#pragma unroll
    for (int j = 0; j < kNB; ++j) {
      w[j] = *reinterpret_cast<const u32x4*>(xb + kXBytes + (wv * kNB + j) * 1024 + 16 * l);
      const uint32_t z = ZU8 ? zr[j] : (uint32_t)(int)__builtin_bit_cast(float, zr[j]);
      nz[j] = as_f16x2(neg_magic_zero_x2(z));
    }
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int run = t >> 1, half = t & 1;
      const int c = run * 8 + 2 * kq + half;
      f16x8 A[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
        A[mt] = *reinterpret_cast<const f16x8*>(xb + (16 * mt + ln) * 256 + ((c ^ ln) << 4));
#pragma unroll
      for (int j = 0; j < kNB; ++j) {
        const uint32_t w0 = w[j][2 * half], w1 = w[j][2 * half + 1];
        const uint32_t t0 = (run ? (w0 >> 4) : w0) & 0x0F0F0F0Fu;
        const uint32_t t1 = (run ? (w1 >> 4) : w1) & 0x0F0F0F0Fu;
        const f16x8 B = b_operand(t0, t1, nz[j]);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          cg[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              A[mt], B, (UPG1 && t == 0) ? zero4 : cg[mt][j], 0, 0, 0);
      }
    }
    // scale at the end of a group (every unit when gs == 128); selects keep the
    // steady-state loop free of branches
    const bool flush = UPG1 || ((u + 1) % upg == 0) || (u + 1 == u_end);
#pragma unroll
    for (int j = 0; j < kNB; ++j) {
      const float sf = flush ? sc[j] : 0.f;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[mt][j][i] = fmaf(sf, cg[mt][j][i], acc[mt][j][i]);
          if (!UPG1) cg[mt][j][i] = flush ? 0.f : cg[mt][j][i];
        }
    }
  };

  // Pipeline: the tiles of D-1 units ahead are in flight in LDS, the scales
  // and zero points one block of D units ahead in registers. Registers carried
  // around the loop only ever hold loads that have completed.
  float cs[D][kNB], ns[D][kNB];
  uint32_t cz[D][kNB], nz_[D][kNB];
  load_sz(cs, cz, u_begin);
  static_for<0, D - 1>([&](auto I) { issue(I, u_begin + I); });

  // Steady state: whole blocks of D units as straight-line code (a branch in
  // the block would make the compiler drain the load ring at the join).
  int u0 = u_begin;
  for (; u0 + D <= u_end; u0 += D) {
    load_sz(ns, nz_, u0 + D);
    static_for<0, D>([&](auto I) {
      constexpr int i = decltype(I)::value;
      // copies of unit u0+i done (loads issued after them: D-2 units' copies,
      // plus the scale batch when unit u0+i was issued before it)
      wait_vmcnt<(D - 2) * kCopies + (i <= D - 2 ? kBatch : 0)>();
      barrier_only();  // every wave's copies are in; slot (i+D-1)%D is free
      issue(std::integral_constant<int, (i + D - 1) % D>{}, u0 + i + D - 1);
      compute(I, cs[i], cz[i], u0 + i);
    });
#pragma unroll
    for (int d = 0; d < D; ++d)
#pragma unroll
      for (int j = 0; j < kNB; ++j) {
        cs[d][j] = ns[d][j];
        cz[d][j] = nz_[d][j];
      }
  }
  // Remainder: fewer than D units, already in ring slots 0..rem-1.
  const int rem = u_end - u0;
  static_for<0, D - 1>([&](auto I) {
    constexpr int i = decltype(I)::value;
    if (i < rem) {
      wait_vmcnt<0>();
      barrier_only();
      compute(I, cs[i], cz[i], u0 + i);
    }
  });

  // ---- epilogue ---------------------------------------------------------
  const int n0 = tile * kBN + wv * 32 + ln;
  const int m0 = mb * R + 4 * kq;
  if (a.splits > 1) {
    // Partial tile of split sp: [wave][mt][j][lane] x 16 bytes (each lane's
    // f32x4 contiguous, a wave's store one 1 KiB run). Stores and loads carry
    // the device-scope cache policy (sc1), like agent-scope atomics: they are
    // coherent across the XCDs' L2 caches without a release fence, whose L2
    // write-back would cost far more than the tile. The s_waitcnt makes every
    // store of this thread complete before the barrier, and the barrier
    // orders them before the counter increment.
    constexpr int kPartBytes = kWaves * MT * kNB * 64 * 16;
    const __amdgpu_buffer_rsrc_t rp =
        rsrc(a.part + (size_t)tl * a.splits * (kPartBytes / 4), (int64_t)a.splits * kPartBytes);
    const int vlane = (wv * MT * kNB * 64 + l) * 16;
    constexpr int kSc1 = 16;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < kNB; ++j)
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[mt][j]), rp,
                                               vlane + (mt * kNB + j) * 1024,
                                               __builtin_amdgcn_readfirstlane(sp * kPartBytes), kSc1);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (tid == 0) {
      const int old = __hip_atomic_fetch_add(&a.counters[tl], 1, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
      last_flag = old == a.splits - 1;
    }
    __syncthreads();
    if (!last_flag) return;
    // Last to arrive: sum the partials in split order (deterministic), one
    // round trip per split.
    f32x4 tot[MT][kNB];
    for (int q = 0; q < a.splits; ++q) {
      f32x4 part[MT][kNB];
      if (q == sp) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < kNB; ++j) part[mt][j] = acc[mt][j];
      } else {
        const int soff = __builtin_amdgcn_readfirstlane(q * kPartBytes);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int j = 0; j < kNB; ++j)
            part[mt][j] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, vlane + (mt * kNB + j) * 1024, soff, kSc1));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < kNB; ++j) tot[mt][j] = q == 0 ? part[mt][j] : tot[mt][j] + part[mt][j];
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < kNB; ++j) acc[mt][j] = tot[mt][j];
    if (tid == 0) __hip_atomic_store(&a.counters[tl], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < kNB; ++j) {
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

template <int MT, int D, bool UPG1, bool ZU8>
hipError_t launch_cfg(const GemmConfig& c, const GemmArgs& a, hipStream_t stream) {
  hipLaunchKernelGGL((w4a16_gemm_kernel<MT, D, UPG1, ZU8>), dim3(c.grid), dim3(kThreads), 0, stream, a);
  return hipGetLastError();
}

template <int MT, int D>
hipError_t launch_mt(const GemmConfig& c, const GemmArgs& a, int zero_u8, hipStream_t stream) {
  const bool upg1 = a.gs == 128;
  if (upg1) {
    if (zero_u8) return launch_cfg<MT, D, true, true>(c, a, stream);
    return launch_cfg<MT, D, true, false>(c, a, stream);
  }
  if (zero_u8) return launch_cfg<MT, D, false, true>(c, a, stream);
  return launch_cfg<MT, D, false, false>(c, a, stream);
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
                       int zero_u8, const int32_t* perm, void* y, int64_t M, int64_t N,
                       int64_t K, int64_t gs, void* workspace, size_t ws_bytes,
                       hipStream_t stream) {
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
  a.y = (f16*)y;
  a.counters = (int*)ws;
  a.part = c.splits > 1 ? (float*)(ws + kCounterBytes + c.ws_perm) : nullptr;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.gs = (int)gs;
  a.splits = c.splits;
  a.n_tiles = c.n_tiles;
  if (c.m_tiles == 1) return launch_mt<1, 8>(c, a, zero_u8, stream);
  if (c.m_tiles == 2) return launch_mt<2, 8>(c, a, zero_u8, stream);
  return launch_mt<4, 6>(c, a, zero_u8, stream);
}

}  // namespace pmi
