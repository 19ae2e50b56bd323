// INT4 W4A16 matmul for skinny activations (M = 1..16: decode and small
// batches) on the gfx950 matrix cores, v_mfma_f32_16x16x32_f16.
//
// Orientation. The MFMA computes C[m][n] = sum_k A[m][k] B[k][n] with the
// activations as A (16 rows m, zero-padded past M) and 16 weight rows as B.
// Lane l then holds C[4*(l/16)+i][l%16]: every lane owns ONE weight row n, so
// the group scale and zero point are one value per lane, and the reduction
// over K happens inside the MFMA (no cross-lane reduction per row).
//
// Weights. Lane group lg (= l/16) of lane l loads 16 bytes of row n at byte
// 16*lg of a 64-byte block of the kernel layout; word t covers columns
// c = block start + 16*lg + 4t + {0..3} (low nibbles) and c + gs/2 (high
// nibbles). A nibble zero-extended into an fp16 half is the subnormal
// q * 2^-24, exact; v_perm_b32 places two of them per register in natural
// column order, so the B operand of one MFMA is the low (or high) nibbles of
// two consecutive words: 8 consecutive columns. Per 32-bit word: 3 bit ops +
// 4 v_perm_b32. MFMA keeps subnormal inputs and accumulates exactly in fp32.
//
// Zero points and scales. sum_k x (q - z) s = s * (2^24 * sum_k x q2^-24 - z Sx)
// where Sx sums the activations; it is applied per 128-column unit (the
// group's scale and zero with the unit's Sx), so each unit adds
// s * (2^24 * C_unit - z * Sx_unit): 2 FMAs per output row and unit. The unit
// sums are computed once per workgroup while x is staged (DPP reduction over
// the 16 lanes holding a unit's 16 chunks).
//
// Activations are staged once per workgroup into LDS in natural order (for
// act_order layers gathered through the permutation), so each A operand is one
// 16-byte LDS read shared by all weight tiles of the wave.
//
// Work split. A workgroup is k_waves x n_waves waves; the k_waves waves split
// the K groups of the same NB weight tiles (16 rows each), each wave keeps a
// ring of D prefetched 64-byte units per tile in registers (buffer loads, row
// offsets in SGPRs), and the partial tiles are summed over the k_waves waves
// through LDS once at the end in a fixed order: deterministic, no workspace.
// The weight prefetch is issued before the activation staging so that the HBM
// latency overlaps it.
//
// Semantics of the reference kernel (pare/kernels/matmul_int4.py:105-176):
// w = (q - zero) * scale per group, fp32 accumulation, fp16 output.
#include "pmi_common.h"
#include "pmi_launch.h"

namespace pmi {
namespace {

constexpr int kSkMaxWaves = 8;

// Low and high nibbles of one word as fp16 subnormals, natural column order:
// lo01 = (q[c], q[c+1]), lo23 = (q[c+2], q[c+3]), hi.. the same for c + gs/2.
PMI_DEV void unpack_natural(uint32_t w, uint32_t& lo01, uint32_t& lo23, uint32_t& hi01,
                            uint32_t& hi23) {
  const uint32_t t = w & 0x0F0F0F0Fu;
  const uint32_t u = (w >> 4) & 0x0F0F0F0Fu;
  // selector byte 0x0C yields 0x00
  lo01 = __builtin_amdgcn_perm(t, t, 0x0C010C00u);
  lo23 = __builtin_amdgcn_perm(t, t, 0x0C030C02u);
  hi01 = __builtin_amdgcn_perm(u, u, 0x0C010C00u);
  hi23 = __builtin_amdgcn_perm(u, u, 0x0C030C02u);
}

PMI_DEV f16x8 halves8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(f16x8, u32x4{a, b, c, d});
}

PMI_DEV __amdgpu_buffer_rsrc_t sk_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// One prefetched 64-byte unit of NB weight tiles: 16 bytes of weights and the
// raw scale / zero of its group per lane.
template <int NB>
struct SkUnit {
  u32x4 w[NB];
  uint32_t s[NB];
  uint32_t z[NB];
};

template <int NB, bool ZU8>
PMI_DEV void sk_load(SkUnit<NB>& su, __amdgpu_buffer_rsrc_t rw, __amdgpu_buffer_rsrc_t rs,
                     __amdgpu_buffer_rsrc_t rz, int unit, int bpg, int hgs, const int (&vw)[NB],
                     const int (&vs)[NB]) {
  const int g = unit / bpg;
  const int woff = g * hgs + (unit - g * bpg) * 64;  // byte offset inside the row
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    su.w[nb] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rw, vw[nb], woff, 0));
    su.s[nb] = __builtin_amdgcn_raw_buffer_load_b32(rs, vs[nb], g * 4, 0);
    if constexpr (ZU8)
      su.z[nb] = __builtin_amdgcn_raw_buffer_load_b8(rz, vs[nb] >> 2, g, 0);
    else
      su.z[nb] = __builtin_amdgcn_raw_buffer_load_b32(rz, vs[nb], g * 4, 0);
  }
}

template <int MI, int NB, bool ZU8>
PMI_DEV void sk_process(const SkUnit<NB>& su, int unit, int bpg, int hgs, int lg,
                        const f16* __restrict__ xrow, const float* __restrict__ sx_lds,
                        f32x4 (&acc)[NB]) {
  const int g = unit / bpg;
  const int blk = unit - g * bpg;
  const int c0 = g * 2 * hgs + blk * 64 + 16 * lg;  // first low-nibble column of the lane
  // A operands: 8 consecutive activations each, shared by all NB tiles
  const f16x8 a_lo0 = *reinterpret_cast<const f16x8*>(xrow + c0);
  const f16x8 a_lo1 = *reinterpret_cast<const f16x8*>(xrow + c0 + 8);
  const f16x8 a_hi0 = *reinterpret_cast<const f16x8*>(xrow + c0 + hgs);
  const f16x8 a_hi1 = *reinterpret_cast<const f16x8*>(xrow + c0 + hgs + 8);
  // Sx of the unit's 128 columns for the lane's rows m = 4*lg + i
  const f32x4 sx = *reinterpret_cast<const f32x4*>(sx_lds + unit * 16 + 4 * lg);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    uint32_t l0[4], l1[4], h0[4], h1[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) unpack_natural(su.w[nb][t], l0[t], l1[t], h0[t], h1[t]);
    f32x4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo0, halves8(l0[0], l1[0], l0[1], l1[1]),
                                                     f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_lo1, halves8(l0[2], l1[2], l0[3], l1[3]), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi0, halves8(h0[0], h1[0], h0[1], h1[1]), c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_hi1, halves8(h0[2], h1[2], h0[3], h1[3]), c, 0, 0, 0);
    // acc += s * (2^24 * c - z * Sx): the unit's share of its group's term
    const float s = __builtin_bit_cast(float, su.s[nb]);
    const float s24 = s * 16777216.0f;
    const float zs = -s * (ZU8 ? (float)su.z[nb] : __builtin_bit_cast(float, su.z[nb]));
#pragma unroll
    for (int i = 0; i < MI; ++i) acc[nb][i] = fmaf(zs, sx[i], fmaf(s24, c[i], acc[nb][i]));
  }
}

template <int MI, int NB, int D, bool PERM, bool ZU8>
__global__ void __launch_bounds__(kSkMaxWaves * 64)
w4a16_skinny_kernel(const f16* __restrict__ x, const uint8_t* __restrict__ w,
                    const float* __restrict__ scales, const void* __restrict__ zeros,
                    const int32_t* __restrict__ perm, f16* __restrict__ y, int M, int N, int K,
                    int gs, int k_waves, int n_waves) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kw = wave % k_waves;
  const int nw = wave / k_waves;
  const int li = lane & 15, lg = lane >> 4;
  const int G = K / gs, hgs = gs >> 1, bpg = gs >> 7;
  const int xs = K + 8;  // LDS row stride in halves (16-byte pad spreads banks)
  f16* x_lds = reinterpret_cast<f16*>(smem);
  float* sx_lds = reinterpret_cast<float*>(smem + (size_t)M * xs * 2);  // [K/128][16]

  // ---- this wave: NB tiles, a contiguous range of K groups ----
  const int tile0 = (blockIdx.x * n_waves + nw) * NB;
  const int g_begin = (G * kw) / k_waves, g_end = (G * (kw + 1)) / k_waves;
  const int u_begin = g_begin * bpg;
  const int n_units = (g_end - g_begin) * bpg;
  const int row_bytes = K >> 1;
  const __amdgpu_buffer_rsrc_t rw = sk_rsrc(w, (uint32_t)N * (uint32_t)row_bytes);
  const __amdgpu_buffer_rsrc_t rs = sk_rsrc(scales, (uint32_t)N * (uint32_t)G * 4u);
  const __amdgpu_buffer_rsrc_t rz = sk_rsrc(zeros, (uint32_t)N * (uint32_t)G * (ZU8 ? 1u : 4u));
  int vw[NB], vs[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int n = min((tile0 + nb) * 16 + li, N - 1);  // rows past N re-read row N-1
    vw[nb] = n * row_bytes + 16 * lg;
    vs[nb] = n * G * 4;
  }

  // Weight prefetch first: the HBM latency overlaps the activation staging.
  SkUnit<NB> ring[D];
  const int u_last = min(u_begin + max(n_units, 1), G * bpg) - 1;
#pragma unroll
  for (int d = 0; d < D; ++d)
    sk_load<NB, ZU8>(ring[d], rw, rs, rz, min(u_begin + d, u_last), bpg, hgs, vw, vs);
  __builtin_amdgcn_sched_barrier(0);

  // ---- stage the activations (gathered for act_order) and unit sums ----
  // Chunk c (8 halves) of row m sits in lane c % 64; the 16 chunks of one
  // 128-column unit are 16 consecutive lanes, reduced with DPP in-row steps.
  const int kc8 = K >> 3;
  const int n_chunks = M * kc8;
  for (int c0 = 0; c0 < n_chunks; c0 += blockDim.x) {
    const int c = c0 + threadIdx.x;
    float part = 0.f;
    if (c < n_chunks) {
      const int m = c / kc8, k = (c - m * kc8) * 8;
      u32x4 v;
      if constexpr (PERM) {
        const uint16_t* xr = reinterpret_cast<const uint16_t*>(x) + (int64_t)m * K;
        uint32_t p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i)
          p[i] = (uint32_t)xr[perm_col(perm, k + 2 * i, K)] |
                 ((uint32_t)xr[perm_col(perm, k + 2 * i + 1, K)] << 16);
        v = u32x4{p[0], p[1], p[2], p[3]};
      } else {
        v = *reinterpret_cast<const u32x4*>(x + (int64_t)m * K + k);
      }
      *reinterpret_cast<u32x4*>(x_lds + m * xs + k) = v;
      part = dot2_acc(as_f16x2(0x3C003C00u), v.x, part);
      part = dot2_acc(as_f16x2(0x3C003C00u), v.y, part);
      part = dot2_acc(as_f16x2(0x3C003C00u), v.z, part);
      part = dot2_acc(as_f16x2(0x3C003C00u), v.w, part);
    }
    part += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, part), 0xB1, 0xf, 0xf, false));
    part += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, part), 0x4E, 0xf, 0xf, false));
    part += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, part), 0x141, 0xf, 0xf, false));
    part += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, part), 0x140, 0xf, 0xf, false));
    if (c < n_chunks && (c & 15) == 0) {
      const int m = c / kc8, u = (c - m * kc8) >> 4;
      sx_lds[u * 16 + m] = part;
    }
  }
  // rows m >= M of the unit sums are zero
  for (int e = threadIdx.x; e < (K >> 7) * 16; e += blockDim.x)
    if ((e & 15) >= M) sx_lds[e] = 0.f;
  __syncthreads();

  const f16* xrow = x_lds + min(li, M - 1) * xs;  // A operand row m = l % 16

  f32x4 acc[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // steady state: every refill is a real unit, so loads are unconditional
  int u0 = 0;
  for (; u0 + 2 * D <= n_units; u0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      sk_process<MI, NB, ZU8>(ring[d], u_begin + u0 + d, bpg, hgs, lg, xrow, sx_lds, acc);
      sk_load<NB, ZU8>(ring[d], rw, rs, rz, u_begin + u0 + D + d, bpg, hgs, vw, vs);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  // tail: fewer than 2*D units left
#pragma unroll
  for (int d = 0; d < D; ++d) {
    if (u0 + d < n_units)
      sk_process<MI, NB, ZU8>(ring[d], u_begin + u0 + d, bpg, hgs, lg, xrow, sx_lds, acc);
    if (u0 + D + d < n_units)
      sk_load<NB, ZU8>(ring[d], rw, rs, rz, u_begin + u0 + D + d, bpg, hgs, vw, vs);
  }
#pragma unroll
  for (int d = 0; d < D; ++d)
    if (u0 + D + d < n_units)
      sk_process<MI, NB, ZU8>(ring[d], u_begin + u0 + D + d, bpg, hgs, lg, xrow, sx_lds, acc);

  // ---- sum the k_waves partial tiles through LDS (reusing the x region) ----
  __syncthreads();
  float* red = reinterpret_cast<float*>(smem);  // [k_waves][n_waves*NB][64][MI]
  const int tiles = n_waves * NB;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb)
#pragma unroll
    for (int i = 0; i < MI; ++i)
      red[((kw * tiles + nw * NB + nb) * 64 + lane) * MI + i] = acc[nb][i];
  __syncthreads();
  const int outs = tiles * 16 * M;
  for (int e = threadIdx.x; e < outs; e += blockDim.x) {
    const int t = e / (16 * M);
    const int rem = e - t * 16 * M;
    const int m = rem / 16, r = rem - (rem / 16) * 16;
    const int l = r + 16 * (m >> 2), i = m & 3;
    float s = 0.f;
    for (int q = 0; q < k_waves; ++q) s += red[((q * tiles + t) * 64 + l) * MI + i];
    const int n = (blockIdx.x * tiles + t) * 16 + r;
    if (n < N) y[(int64_t)m * N + n] = f32_to_f16_rne(s);
  }
}

template <int MI, int NB, int D, bool ZU8>
hipError_t sk_launch(const SkinnyConfig& c, const void* x, const uint8_t* w, const float* scales,
                     const void* zeros, const int32_t* perm, void* y, int M, int N, int K, int gs,
                     hipStream_t stream) {
  const dim3 block(64 * c.k_waves * c.n_waves);
  if (perm)
    hipLaunchKernelGGL((w4a16_skinny_kernel<MI, NB, D, true, ZU8>), dim3(c.grid), block, c.lds,
                       stream, (const f16*)x, w, scales, zeros, perm, (f16*)y, M, N, K, gs,
                       c.k_waves, c.n_waves);
  else
    hipLaunchKernelGGL((w4a16_skinny_kernel<MI, NB, D, false, ZU8>), dim3(c.grid), block, c.lds,
                       stream, (const f16*)x, w, scales, zeros, perm, (f16*)y, M, N, K, gs,
                       c.k_waves, c.n_waves);
  return hipGetLastError();
}

template <int MI, int NB>
hipError_t sk_launch_z(const SkinnyConfig& c, const void* x, const uint8_t* w,
                       const float* scales, const void* zeros, int zero_u8,
                       const int32_t* perm, void* y, int M, int N, int K, int gs,
                       hipStream_t stream) {
  if (zero_u8) return sk_launch<MI, NB, 4, true>(c, x, w, scales, zeros, perm, y, M, N, K, gs, stream);
  return sk_launch<MI, NB, 4, false>(c, x, w, scales, zeros, perm, y, M, N, K, gs, stream);
}

template <int MI>
hipError_t sk_launch_nb(const SkinnyConfig& c, const void* x, const uint8_t* w,
                        const float* scales, const void* zeros, int zero_u8,
                        const int32_t* perm, void* y, int M, int N, int K, int gs,
                        hipStream_t stream) {
  if (c.tiles_per_wave == 2)
    return sk_launch_z<MI, 2>(c, x, w, scales, zeros, zero_u8, perm, y, M, N, K, gs, stream);
  return sk_launch_z<MI, 1>(c, x, w, scales, zeros, zero_u8, perm, y, M, N, K, gs, stream);
}

int sk_env(const char* name) {
  const char* s = getenv(name);
  return (s && *s) ? atoi(s) : 0;
}

}  // namespace

// LDS bytes the kernel needs for M activation rows of length K.
static size_t skinny_lds_bytes(int64_t M, int64_t K, int64_t gs, int k_waves, int tiles) {
  (void)gs;
  const size_t stage = (size_t)M * (K + 8) * 2 + (size_t)(K / 128) * 16 * 4;
  const size_t red = (size_t)k_waves * tiles * 64 * (M < 4 ? M : 4) * 4;
  return stage > red ? stage : red;
}

bool skinny_supported(int64_t M, int64_t N, int64_t K, int64_t gs) {
  (void)N;
  if (M < 1 || M > 16 || gs % 128 != 0) return false;
  // k_waves * n_waves = 8 and at most 2 tiles per wave: k_waves * tiles <= 16
  return skinny_lds_bytes(M, K, gs, kSkMaxWaves, 2) <= 64 * 1024;
}

SkinnyConfig skinny_config(int64_t M, int64_t N, int64_t K, int64_t gs) {
  SkinnyConfig c;
  const int64_t tiles = (N + 15) / 16;
  const int64_t units = K / 128;  // 64-byte units per row
  static const int env_kw = sk_env("PMI_SK_KWAVES");
  static const int env_nb = sk_env("PMI_SK_NB");
  // K split across up to 8 waves of a workgroup, at least 2 units per wave
  const int64_t groups = K / gs;
  int kw = 8;
  while (kw > 1 && (units / kw < 2 || groups < kw)) kw /= 2;
  if ((env_kw == 1 || env_kw == 2 || env_kw == 4 || env_kw == 8) && env_kw <= groups) kw = env_kw;
  c.k_waves = kw;
  c.n_waves = kSkMaxWaves / kw;
  c.tiles_per_wave = tiles >= 2 * 256 * c.n_waves ? 2 : 1;
  if (env_nb == 1 || env_nb == 2) c.tiles_per_wave = env_nb;
  const int64_t per_wg = (int64_t)c.n_waves * c.tiles_per_wave;
  c.grid = (int)((tiles + per_wg - 1) / per_wg);
  c.lds = skinny_lds_bytes(M, K, gs, c.k_waves, (int)per_wg);
  return c;
}

hipError_t launch_skinny(const void* x, const uint8_t* w, const float* scales, const void* zeros,
                         int zero_u8, const int32_t* perm, void* y, int64_t M, int64_t N,
                         int64_t K, int64_t gs, hipStream_t stream) {
  const SkinnyConfig c = skinny_config(M, N, K, gs);
  const int m = (int)M, n = (int)N, k = (int)K, g = (int)gs;
  switch (M < 4 ? M : 4) {
    case 1: return sk_launch_nb<1>(c, x, w, scales, zeros, zero_u8, perm, y, m, n, k, g, stream);
    case 2: return sk_launch_nb<2>(c, x, w, scales, zeros, zero_u8, perm, y, m, n, k, g, stream);
    case 3: return sk_launch_nb<3>(c, x, w, scales, zeros, zero_u8, perm, y, m, n, k, g, stream);
    default: return sk_launch_nb<4>(c, x, w, scales, zeros, zero_u8, perm, y, m, n, k, g, stream);
  }
}

}  // namespace pmi
