// INT4 W4A16 GEMM on the gfx950 matrix cores (M > 4), v_mfma_f32_16x16x32_f16.
//
// The reduction dimension of an MFMA may be permuted freely as long as A and
// B use the same permutation. This kernel picks the permutation that falls
// out of the kernel-layout nibble order: a lane of lane group g (= lane/16)
// loads the 16 bytes at offset 16g of a 64-byte block of its weight row; word
// t of those bytes unpacks (unpack_word_minus_zero) into the eight fp16
// values (q - z) of columns k+{0,2,1,3} and k+gs/2+{0,2,1,3}, k = block start
// + 16g + 4t. That is the B operand of MFMA step t, straight from registers:
// the weights never pass through LDS and each byte is loaded by one lane.
// The activation tile is staged in LDS already reordered into the same
// column order, so each A operand is one 16-byte LDS read.
//
// (q - z) is exact in fp16, so each group's MFMA chain accumulates
// sum x * (q - z) exactly as fp32 products; the group scale is applied once
// per group and output element (4 FMAs per 16x16 tile per lane), as in
// sum_g s_g * sum_k x_k (q_k - z_g). This needs every 64-byte block inside one
// group, i.e. group_size % 128 == 0 (checked by the host).
//
// Reference semantics: pare/kernels/matmul_int4.py:105-176.
#include "pmi_common.h"
#include "pmi_launch.h"

namespace pmi {
namespace {

constexpr int kWaves = 4;
constexpr int kARowBytes = 256 + 16;  // 128 fp16 per activation row + pad (bank spread)

template <int MB, int NB, bool PERM>
__global__ void __launch_bounds__(kWaves * 64)
w4a16_gemm_kernel(const f16* __restrict__ x, const uint8_t* __restrict__ w,
                  const float* __restrict__ scales, const void* __restrict__ zeros, int zero_u8,
                  const int32_t* __restrict__ perm, f16* __restrict__ y, int M, int N, int K,
                  int gs) {
  constexpr int BM = 16 * MB;
  constexpr int BN = 16 * NB * kWaves;
  __shared__ __attribute__((aligned(16))) uint8_t a_lds[BM * kARowBytes];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int lg = lane >> 4;
  const int m0 = blockIdx.y * BM;
  const int nw0 = blockIdx.x * BN + wave * 16 * NB;
  const int hgs = gs >> 1;
  const int G = K / gs;
  const int blocks_per_group = gs >> 7;
  const int64_t row_bytes = K >> 1;
  const uint16_t* xs = reinterpret_cast<const uint16_t*>(x);

  f32x4 acc[MB][NB];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) acc[i][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

  for (int g = 0; g < G; ++g) {
    float sc[NB];
    uint32_t nz[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int n = nw0 + nb * 16 + li;
      if (n < N) {
        sc[nb] = scales[(int64_t)n * G + g];
        nz[nb] = neg_magic_zero_x2(load_zero(zeros, zero_u8, (int64_t)n * G + g));
      } else {
        sc[nb] = 0.f;
        nz[nb] = neg_magic_zero_x2(0u);
      }
    }
    f32x4 part[MB][NB];
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) part[i][nb] = f32x4{0.f, 0.f, 0.f, 0.f};

    for (int blk = 0; blk < blocks_per_group; ++blk) {
      const int jb = blk * 64;      // byte offset inside the group tile
      const int kb = g * gs + jb;   // column of the low nibble of byte jb

      // Weights first, so their HBM latency overlaps the activation staging.
      u32x4 wv[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int n = nw0 + nb * 16 + li;
        wv[nb] = n < N ? *reinterpret_cast<const u32x4*>(w + (int64_t)n * row_bytes +
                                                          (int64_t)g * hgs + jb + 16 * lg)
                       : u32x4{0u, 0u, 0u, 0u};
      }

      __syncthreads();
      for (int e = threadIdx.x; e < BM * 16; e += kWaves * 64) {
        const int m = e >> 4, eg = (e >> 2) & 3, et = e & 3;
        const int kk = kb + 16 * eg + 4 * et;
        uint32_t l0 = 0, l1 = 0, h0 = 0, h1 = 0;
        if (m0 + m < M) {
          const int64_t xr = (int64_t)(m0 + m) * K;
          if constexpr (PERM) {
            const uint16_t* xrow = xs + xr;
            l0 = (uint32_t)xrow[perm_col(perm, kk, K)] |
                 ((uint32_t)xrow[perm_col(perm, kk + 1, K)] << 16);
            l1 = (uint32_t)xrow[perm_col(perm, kk + 2, K)] |
                 ((uint32_t)xrow[perm_col(perm, kk + 3, K)] << 16);
            h0 = (uint32_t)xrow[perm_col(perm, kk + hgs, K)] |
                 ((uint32_t)xrow[perm_col(perm, kk + hgs + 1, K)] << 16);
            h1 = (uint32_t)xrow[perm_col(perm, kk + hgs + 2, K)] |
                 ((uint32_t)xrow[perm_col(perm, kk + hgs + 3, K)] << 16);
          } else {
            const uint2 lo = *reinterpret_cast<const uint2*>(xs + xr + kk);
            const uint2 hi = *reinterpret_cast<const uint2*>(xs + xr + kk + hgs);
            l0 = lo.x; l1 = lo.y; h0 = hi.x; h1 = hi.y;
          }
        }
        const u32x4 v = u32x4{pair_lo(l0, l1), pair_hi(l0, l1), pair_lo(h0, h1), pair_hi(h0, h1)};
        *reinterpret_cast<u32x4*>(a_lds + m * kARowBytes + eg * 64 + et * 16) = v;
      }
      __syncthreads();

#pragma unroll
      for (int t = 0; t < 4; ++t) {
        f16x8 bop[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          f16x2 d0, d1, d2, d3;
          unpack_word_minus_zero(wv[nb][t], nz[nb], d0, d1, d2, d3);
          bop[nb] = f16x8{d0.x, d0.y, d1.x, d1.y, d2.x, d2.y, d3.x, d3.y};
        }
#pragma unroll
        for (int i = 0; i < MB; ++i) {
          const f16x8 aop =
              *reinterpret_cast<const f16x8*>(a_lds + (16 * i + li) * kARowBytes + lg * 64 + t * 16);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
            part[i][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop[nb], part[i][nb], 0, 0, 0);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < MB; ++i)
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
#pragma unroll
        for (int v = 0; v < 4; ++v) acc[i][nb][v] = fmaf(sc[nb], part[i][nb][v], acc[i][nb][v]);
  }

  // Output tile: lane holds rows 4*lg + v, column li of each 16x16 tile.
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int n = nw0 + nb * 16 + li;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = m0 + 16 * i + 4 * lg + v;
        if (m < M && n < N) y[(int64_t)m * N + n] = f32_to_f16_rne(acc[i][nb][v]);
      }
    }
}

template <int MB, int NB>
hipError_t launch_mb_nb(const GemmConfig& c, const void* x, const uint8_t* w, const float* scales,
                        const void* zeros, int zero_u8, const int32_t* perm, void* y, int M, int N,
                        int K, int gs, hipStream_t stream) {
  const dim3 grid(c.grid_n, c.grid_m);
  const dim3 block(kWaves * 64);
  if (perm)
    hipLaunchKernelGGL((w4a16_gemm_kernel<MB, NB, true>), grid, block, 0, stream, (const f16*)x, w,
                       scales, zeros, zero_u8, perm, (f16*)y, M, N, K, gs);
  else
    hipLaunchKernelGGL((w4a16_gemm_kernel<MB, NB, false>), grid, block, 0, stream, (const f16*)x, w,
                       scales, zeros, zero_u8, perm, (f16*)y, M, N, K, gs);
  return hipGetLastError();
}

}  // namespace

GemmConfig gemm_config(int64_t M, int64_t N, int64_t K) {
  (void)K;
  GemmConfig c;
  c.m_tiles = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int64_t bm = 16 * c.m_tiles;
  c.grid_m = (int)((M + bm - 1) / bm);
  c.n_tiles = (N / (16 * 2 * kWaves)) * c.grid_m >= 256 ? 2 : 1;
  const int64_t bn = 16 * c.n_tiles * kWaves;
  c.grid_n = (int)((N + bn - 1) / bn);
  return c;
}

hipError_t launch_gemm(const void* x, const uint8_t* w, const float* scales, const void* zeros,
                       int zero_u8, const int32_t* perm, void* y, int64_t M, int64_t N,
                       int64_t K, int64_t gs, hipStream_t stream) {
  const GemmConfig c = gemm_config(M, N, K);
  const int m = (int)M, n = (int)N, k = (int)K, g = (int)gs;
  if (c.m_tiles == 1) {
    if (c.n_tiles == 1) return launch_mb_nb<1, 1>(c, x, w, scales, zeros, zero_u8, perm, y, m, n, k, g, stream);
    return launch_mb_nb<1, 2>(c, x, w, scales, zeros, zero_u8, perm, y, m, n, k, g, stream);
  }
  if (c.m_tiles == 2) {
    if (c.n_tiles == 1) return launch_mb_nb<2, 1>(c, x, w, scales, zeros, zero_u8, perm, y, m, n, k, g, stream);
    return launch_mb_nb<2, 2>(c, x, w, scales, zeros, zero_u8, perm, y, m, n, k, g, stream);
  }
  if (c.n_tiles == 1) return launch_mb_nb<4, 1>(c, x, w, scales, zeros, zero_u8, perm, y, m, n, k, g, stream);
  return launch_mb_nb<4, 2>(c, x, w, scales, zeros, zero_u8, perm, y, m, n, k, g, stream);
}

}  // namespace pmi
