// Layout and producer kernels around the INT4 matmul:
//   repack   storage layout -> kernel layout (+ optional act_order permutation)
//   zeros    fp32 zero points -> u8, counting values that are not integers in [0,15]
//   dequant  packed INT4 -> fp16 / bf16 / fp32 weights (bit-exact with the reference)
//   rtn      fp weights -> (packed, scale, zero) with per-group min/max RTN
//   awq      AWQ-GEMM int32 words <-> storage layout, fp16 [G,N] <-> fp32 [N,G]
// All are integer/byte or elementwise work bound by HBM bandwidth; none uses LDS.
#include "../../include/pare_amd.h"
#include "pmi_common.h"
#include "pmi_launch.h"

namespace pmi {
namespace {

constexpr int kBlock = 256;

PMI_DEV uint32_t nibble_at(const uint8_t* __restrict__ row, int64_t col) {
  return (row[col >> 1] >> ((col & 1) * 4)) & 0xFu;
}

PMI_DEV int64_t safe_col(const int32_t* __restrict__ perm, int64_t k, int64_t K) {
  if (!perm) return k;
  const int32_t p = perm[k];
  return (p >= 0 && p < K) ? (int64_t)p : k;
}

// Output byte j of a row holds, inside its group tile t (hgs = gs/2 bytes),
// column t*gs + (j - t*hgs) in bits 0-3 and that column + hgs in bits 4-7
// (pare/core/pack.py:123-130). One thread writes 4 consecutive output bytes.
__global__ void repack_kernel(const uint8_t* __restrict__ packed, uint8_t* __restrict__ out,
                              const int32_t* __restrict__ perm, int64_t N, int64_t K, int64_t gs) {
  const int64_t row_bytes = K >> 1;
  const int64_t words_per_row = row_bytes >> 2;
  const int64_t hgs = gs >> 1;
  const int64_t total = N * words_per_row;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = idx / words_per_row;
    const int64_t jw = (idx - n * words_per_row) << 2;
    const uint8_t* src = packed + n * row_bytes;
    uint32_t word = 0;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t j = jw + b;
      const int64_t t = j / hgs;
      const int64_t k_lo = t * gs + (j - t * hgs);
      const uint32_t lo = nibble_at(src, safe_col(perm, k_lo, K));
      const uint32_t hi = nibble_at(src, safe_col(perm, k_lo + hgs, K));
      word |= (lo | (hi << 4)) << (8 * b);
    }
    *reinterpret_cast<uint32_t*>(out + n * row_bytes + jw) = word;
  }
}

__global__ void zeros_to_u8_kernel(const float* __restrict__ zeros, uint8_t* __restrict__ out,
                                   int32_t* __restrict__ bad, int64_t count) {
  int local_bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float z = zeros[i];
    const bool ok = z >= 0.f && z <= 15.f && z == rintf(z);  // false for NaN
    local_bad += ok ? 0 : 1;
    out[i] = ok ? (uint8_t)(int)z : (uint8_t)0;
  }
  if (bad && local_bad) atomicAdd(bad, local_bad);
}

// int32 act_order permutation -> its 16-bit copy (K <= 65536) for the GEMV's
// LDS gather. Entries outside [0, K) become 0, as the kernels clamp them at
// use, and are counted into *bad (nullable).
__global__ void perm_u16_kernel(const int32_t* __restrict__ perm, uint16_t* __restrict__ out,
                                int32_t* __restrict__ bad, int64_t K) {
  int local_bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < K;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t p = perm[i];
    const bool ok = p >= 0 && (int64_t)p < K;
    local_bad += ok ? 0 : 1;
    out[i] = ok ? (uint16_t)p : (uint16_t)0;
  }
  if (bad && local_bad) atomicAdd(bad, local_bad);
}

// [N, G] -> [G, N] copies of the scales and zero points (zeros to u8, values
// that are not integers in [0, 15] counted like zeros_to_u8_kernel). One
// thread per output element: writes are coalesced, reads strided; it runs
// once per layer.
__global__ void sz_group_major_kernel(const float* __restrict__ scales,
                                      const void* __restrict__ zeros, int zero_u8,
                                      float* __restrict__ s_gm, uint8_t* __restrict__ z_gm,
                                      int32_t* __restrict__ bad, int64_t N, int64_t G) {
  int local_bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < N * G;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t g = i / N, n = i - g * N;
    s_gm[i] = scales[n * G + g];
    if (zero_u8) {
      const uint8_t z = ((const uint8_t*)zeros)[n * G + g];
      local_bad += z <= 15 ? 0 : 1;
      z_gm[i] = z <= 15 ? z : (uint8_t)0;
    } else {
      const float z = ((const float*)zeros)[n * G + g];
      const bool ok = z >= 0.f && z <= 15.f && z == rintf(z);  // false for NaN
      local_bad += ok ? 0 : 1;
      z_gm[i] = ok ? (uint8_t)(int)z : (uint8_t)0;
    }
  }
  if (bad && local_bad) atomicAdd(bad, local_bad);
}

// w_hat = (float(q) - zero) * scale in fp32, then one rounding to out dtype
// (pare/core/functional.py:90-91, pare/layers/linear.py:129).
template <int OUT>
__global__ void dequant_kernel(const uint8_t* __restrict__ w, int layout,
                               const float* __restrict__ scales, const void* __restrict__ zeros,
                               int zero_u8, const int32_t* __restrict__ idx,
                               void* __restrict__ out, int64_t N, int64_t K, int64_t gs) {
  const int64_t row_bytes = K >> 1;
  const int64_t hgs = gs >> 1;
  const int64_t G = K / gs;
  const int64_t total = N * K;
  for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (int64_t)gridDim.x * blockDim.x) {
    const int64_t n = e / K;
    const int64_t j = e - n * K;
    const uint8_t* row = w + n * row_bytes;
    uint32_t q;
    int64_t g, col;
    if (layout == PMI_LAYOUT_KERNEL) {
      const int64_t t = j / gs;
      const int64_t r = j - t * gs;
      const int64_t byte = t * hgs + (r < hgs ? r : r - hgs);
      q = (row[byte] >> (r < hgs ? 0 : 4)) & 0xFu;
      g = t;
      col = safe_col(idx, j, K);
    } else {
      q = nibble_at(row, j);
      g = idx ? (int64_t)idx[j] : j / gs;
      col = j;
    }
    float v;
    if (g < 0 || g >= G) {
      v = __builtin_nanf("");
    } else {
      const int64_t sz = n * G + g;
      const float z = zero_u8 ? (float)((const uint8_t*)zeros)[sz] : ((const float*)zeros)[sz];
      v = ((float)q - z) * scales[sz];
    }
    const int64_t o = n * K + col;
    if constexpr (OUT == PMI_F32) {
      ((float*)out)[o] = v;
    } else if constexpr (OUT == PMI_F16) {
      ((f16*)out)[o] = f32_to_f16_rne(v);
    } else {
      ((uint16_t*)out)[o] = f32_to_bf16_rne(v);
    }
  }
}

// AWQ-GEMM int32 words (pare/model/export_awq.py:37-49): word c of a row packs
// output columns 8c..8c+7, column 8c + order[i] in bits 4i..4i+3 with
// order = [0,2,4,6,1,3,5,7]. awq_slot(o) is the inverse: the nibble index of
// column 8c + o.
PMI_DEV int awq_slot(int o) { return (o >> 1) | ((o & 1) << 2); }

// qweight int32 [K, N/8] -> storage layout u8 [N, K/2]. One thread per
// (32-column block kb of K, word column c): 32 coalesced word loads down K,
// then eight 16-byte row writes (rows 8c..8c+7, bytes 16kb..16kb+15).
__global__ void awq_to_storage_kernel(const int32_t* __restrict__ qweight,
                                      uint8_t* __restrict__ packed, int64_t N, int64_t K) {
  const int64_t NC = N >> 3;
  const int64_t total = (K >> 5) * NC;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t kb = idx / NC, c = idx - kb * NC;
    const int32_t* src = qweight + (kb << 5) * NC + c;
    uint32_t out[8][4];
#pragma unroll
    for (int o = 0; o < 8; ++o)
#pragma unroll
      for (int s = 0; s < 4; ++s) out[o][s] = 0;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int t = 0; t < 8; ++t) {
        const uint32_t w = (uint32_t)src[(int64_t)(8 * s + t) * NC];
#pragma unroll
        for (int o = 0; o < 8; ++o) out[o][s] |= ((w >> (4 * awq_slot(o))) & 0xFu) << (4 * t);
      }
    }
#pragma unroll
    for (int o = 0; o < 8; ++o) {
      u32x4 v = {out[o][0], out[o][1], out[o][2], out[o][3]};
      *reinterpret_cast<u32x4*>(packed + (8 * c + o) * (K >> 1) + (kb << 4)) = v;
    }
  }
}

// qzeros int32 [G, N/8], scales fp16 [G, N] -> zero, scale fp32 [N, G].
__global__ void awq_sz_to_rows_kernel(const int32_t* __restrict__ qzeros,
                                      const f16* __restrict__ scales, float* __restrict__ scale,
                                      float* __restrict__ zero, int64_t N, int64_t G) {
  const int64_t NC = N >> 3;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < G * NC;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t g = idx / NC, c = idx - g * NC;
    const uint32_t z = (uint32_t)qzeros[idx];
#pragma unroll
    for (int o = 0; o < 8; ++o) {
      const int64_t n = 8 * c + o;
      zero[n * G + g] = (float)((z >> (4 * awq_slot(o))) & 0xFu);
      scale[n * G + g] = (float)scales[g * N + n];
    }
  }
}

// Storage layout u8 [N, K/2] -> qweight int32 [K, N/8]; the inverse of
// awq_to_storage_kernel with the same thread mapping (coalesced word stores).
__global__ void storage_to_awq_kernel(const uint8_t* __restrict__ packed,
                                      int32_t* __restrict__ qweight, int64_t N, int64_t K) {
  const int64_t NC = N >> 3;
  const int64_t total = (K >> 5) * NC;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t kb = idx / NC, c = idx - kb * NC;
    u32x4 in[8];
#pragma unroll
    for (int o = 0; o < 8; ++o)
      in[o] = *reinterpret_cast<const u32x4*>(packed + (8 * c + o) * (K >> 1) + (kb << 4));
    int32_t* dst = qweight + (kb << 5) * NC + c;
#pragma unroll
    for (int t = 0; t < 32; ++t) {
      uint32_t w = 0;
#pragma unroll
      for (int o = 0; o < 8; ++o)
        w |= ((in[o][t >> 3] >> (4 * (t & 7))) & 0xFu) << (4 * awq_slot(o));
      dst[(int64_t)t * NC] = (int32_t)w;
    }
  }
}

// zero (PMI_F32 or PMI_U8) and scale fp32 [N, G] -> qzeros int32 [G, N/8] and
// scales fp16 [G, N]. fp32 zeros are rounded half-to-even first
// (pare/model/export_awq.py:85); a zero outside [0, 15] after rounding is
// counted in *bad and packed as 0.
__global__ void awq_sz_from_rows_kernel(const float* __restrict__ scale,
                                        const void* __restrict__ zero, int zero_u8,
                                        int32_t* __restrict__ qzeros, f16* __restrict__ scales,
                                        int32_t* __restrict__ bad, int64_t N, int64_t G) {
  const int64_t NC = N >> 3;
  int local_bad = 0;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < G * NC;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t g = idx / NC, c = idx - g * NC;
    uint32_t w = 0;
#pragma unroll
    for (int o = 0; o < 8; ++o) {
      const int64_t n = 8 * c + o;
      uint32_t z;
      if (zero_u8) {
        z = ((const uint8_t*)zero)[n * G + g];
      } else {
        const float r = rintf(((const float*)zero)[n * G + g]);
        z = (r >= 0.f && r <= 15.f) ? (uint32_t)(int)r : 16u;  // NaN -> 16
      }
      local_bad += z <= 15u ? 0 : 1;
      w |= (z <= 15u ? z : 0u) << (4 * awq_slot(o));
      scales[g * N + n] = f32_to_f16_rne(scale[n * G + g]);
    }
    qzeros[idx] = (int32_t)w;
  }
  if (bad && local_bad) atomicAdd(bad, local_bad);
}

template <int IN>
PMI_DEV float load_as_f32(const void* p, int64_t i) {
  if constexpr (IN == PMI_F32) {
    return ((const float*)p)[i];
  } else if constexpr (IN == PMI_F16) {
    return (float)((const f16*)p)[i];
  } else {
    return __builtin_bit_cast(float, (uint32_t)((const uint16_t*)p)[i] << 16);
  }
}

PMI_DEV float wave_min(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fminf(v, __shfl_xor(v, o, 64));
  return v;
}
PMI_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// One wave per (row, group): min/max -> (scale, zero) -> q -> packed bytes.
// Formulas of pare/core/scale.py:73-91 and pare/core/functional.py:68-75 with
// qmin = 0, qmax = 15 (unsigned INT4); rintf is round-half-to-even like
// torch.round.
template <int IN>
__global__ void rtn_kernel(const void* __restrict__ w, uint8_t* __restrict__ packed,
                           float* __restrict__ scale_out, float* __restrict__ zero_out, int64_t N,
                           int64_t K, int64_t gs, int sym) {
  const int lane = threadIdx.x & 63;
  const int64_t G = K / gs;
  const int64_t unit = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (unit >= N * G) return;
  const int64_t n = unit / G;
  const int64_t g = unit - n * G;
  const int64_t base = n * K + g * gs;
  const int64_t pairs = gs >> 1;

  float mn = __builtin_inff(), mx = -__builtin_inff();
  for (int64_t p = lane; p < pairs; p += 64) {
    const float a = load_as_f32<IN>(w, base + 2 * p);
    const float b = load_as_f32<IN>(w, base + 2 * p + 1);
    mn = fminf(mn, fminf(a, b));
    mx = fmaxf(mx, fmaxf(a, b));
  }
  mn = wave_min(mn);
  mx = wave_max(mx);

  float scale, zero;
  scale_zero_from_minmax(mn, mx, sym, scale, zero);
  if (lane == 0) {
    scale_out[unit] = scale;
    zero_out[unit] = zero;
  }
  for (int64_t p = lane; p < pairs; p += 64) {
    const float a = load_as_f32<IN>(w, base + 2 * p);
    const float b = load_as_f32<IN>(w, base + 2 * p + 1);
    const float qa = fminf(fmaxf(rintf(a / scale + zero), 0.0f), 15.0f);
    const float qb = fminf(fmaxf(rintf(b / scale + zero), 0.0f), 15.0f);
    packed[(base >> 1) + p] = (uint8_t)((int)qa | ((int)qb << 4));
  }
}

// Kernel layout (group size gs) -> tiled layout of the tiled-weight GEMM.
// Output chunk i (16 bytes) of block (panel p, unit u): tile j = (i / 64) % 4,
// lane L = i % 64 = n + 16 h, row 64 p + 4 n + j (zero past N); its byte b
// holds columns c = 128 u + (b < 8 ? 8 h + b : 32 + 8 h + b - 8) in the low
// nibble and c + 64 in the high nibble. In the kernel layout column k of a row
// lies in the gs-wide tile starting at k0 = k - k % gs, byte k0 / 2 + k % (gs/2),
// low nibble for k % gs < gs / 2, high nibble otherwise. One thread per chunk.
__device__ __forceinline__ uint32_t kernel_nibble(const uint8_t* __restrict__ row, int k, int gs) {
  const int k0 = k - k % gs, j = k - k0, hg = gs >> 1;
  const uint8_t b = row[(k0 >> 1) + (j < hg ? j : j - hg)];
  return j < hg ? (b & 0xFu) : (b >> 4);
}

__global__ void tile_kernel(const uint8_t* __restrict__ wk, uint8_t* __restrict__ wt, int64_t N,
                            int64_t K, int gs) {
  const int64_t U = K >> 7;
  const int64_t chunks = (N + 63) / 64 * U * 256;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < chunks;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int L = (int)(i & 63), j = (int)((i >> 6) & 3);
    const int64_t pu = i >> 8;
    const int64_t u = pu % U, p = pu / U;
    const int n = L & 15, h = L >> 4;
    const int64_t row = 64 * p + 4 * n + j;
    uint32_t w[4] = {0u, 0u, 0u, 0u};
    if (row < N) {
      const uint8_t* src = wk + row * (K >> 1);
      if (gs == 128) {
        // the unit is one group: its bytes carry columns c and c + 64 already
        const uint32_t* a = reinterpret_cast<const uint32_t*>(src + 64 * u + 8 * h);
        const uint32_t* b = reinterpret_cast<const uint32_t*>(src + 64 * u + 32 + 8 * h);
        w[0] = a[0], w[1] = a[1], w[2] = b[0], w[3] = b[1];
      } else {
#pragma unroll
        for (int bb = 0; bb < 16; ++bb) {
          const int c = (int)(128 * u) + (bb < 8 ? 8 * h + bb : 32 + 8 * h + bb - 8);
          const uint32_t v = kernel_nibble(src, c, gs) | (kernel_nibble(src, c + 64, gs) << 4);
          w[bb >> 2] |= v << (8 * (bb & 3));
        }
      }
    }
    reinterpret_cast<u32x4*>(wt)[i] = u32x4{w[0], w[1], w[2], w[3]};
  }
}

int grid_for(int64_t work, int per_thread = 1) {
  int64_t blocks = (work / per_thread + kBlock - 1) / kBlock;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  return (int)blocks;
}

}  // namespace

hipError_t launch_repack(const uint8_t* packed, uint8_t* out, const int32_t* perm, int64_t N,
                         int64_t K, int64_t gs, hipStream_t stream) {
  hipLaunchKernelGGL(repack_kernel, dim3(grid_for(N * (K / 8))), dim3(kBlock), 0, stream, packed,
                     out, perm, N, K, gs);
  return hipGetLastError();
}

hipError_t launch_tile(const uint8_t* w_kernel, uint8_t* w_tiled, int64_t N, int64_t K, int64_t gs,
                       hipStream_t stream) {
  hipLaunchKernelGGL(tile_kernel, dim3(grid_for((N + 63) / 64 * (K / 128) * 256)), dim3(kBlock), 0,
                     stream, w_kernel, w_tiled, N, K, (int)gs);
  return hipGetLastError();
}

hipError_t launch_zeros_to_u8(const float* zeros, uint8_t* out, int32_t* bad, int64_t count,
                              hipStream_t stream) {
  hipLaunchKernelGGL(zeros_to_u8_kernel, dim3(grid_for(count)), dim3(kBlock), 0, stream, zeros,
                     out, bad, count);
  return hipGetLastError();
}

hipError_t launch_perm_u16(const int32_t* perm, uint16_t* out, int32_t* bad, int64_t K,
                           hipStream_t stream) {
  hipLaunchKernelGGL(perm_u16_kernel, dim3(grid_for(K)), dim3(kBlock), 0, stream, perm, out, bad,
                     K);
  return hipGetLastError();
}

hipError_t launch_sz_group_major(const float* scales, const void* zeros, int zero_u8,
                                 float* scales_gm, uint8_t* zeros_gm, int32_t* bad, int64_t N,
                                 int64_t G, hipStream_t stream) {
  hipLaunchKernelGGL(sz_group_major_kernel, dim3(grid_for(N * G)), dim3(kBlock), 0, stream, scales,
                     zeros, zero_u8, scales_gm, zeros_gm, bad, N, G);
  return hipGetLastError();
}

hipError_t launch_awq_to_storage(const int32_t* qweight, const int32_t* qzeros, const void* scales,
                                 uint8_t* packed, float* scale, float* zero, int64_t N, int64_t K,
                                 int64_t gs, hipStream_t stream) {
  hipLaunchKernelGGL(awq_to_storage_kernel, dim3(grid_for((K / 32) * (N / 8))), dim3(kBlock), 0,
                     stream, qweight, packed, N, K);
  if (hipError_t e = hipGetLastError()) return e;
  const int64_t G = K / gs;
  hipLaunchKernelGGL(awq_sz_to_rows_kernel, dim3(grid_for(G * (N / 8))), dim3(kBlock), 0, stream,
                     qzeros, (const f16*)scales, scale, zero, N, G);
  return hipGetLastError();
}

hipError_t launch_storage_to_awq(const uint8_t* packed, const float* scale, const void* zero,
                                 int zero_u8, int32_t* qweight, int32_t* qzeros, void* scales,
                                 int32_t* bad, int64_t N, int64_t K, int64_t gs,
                                 hipStream_t stream) {
  hipLaunchKernelGGL(storage_to_awq_kernel, dim3(grid_for((K / 32) * (N / 8))), dim3(kBlock), 0,
                     stream, packed, qweight, N, K);
  if (hipError_t e = hipGetLastError()) return e;
  const int64_t G = K / gs;
  hipLaunchKernelGGL(awq_sz_from_rows_kernel, dim3(grid_for(G * (N / 8))), dim3(kBlock), 0, stream,
                     scale, zero, zero_u8, qzeros, (f16*)scales, bad, N, G);
  return hipGetLastError();
}

hipError_t launch_dequant(const uint8_t* w, int layout, const float* scales, const void* zeros,
                          int zero_u8, const int32_t* idx, void* out, int out_dtype, int64_t N,
                          int64_t K, int64_t gs, hipStream_t stream) {
  const dim3 grid(grid_for(N * K)), block(kBlock);
  switch (out_dtype) {
    case PMI_F16:
      hipLaunchKernelGGL(dequant_kernel<PMI_F16>, grid, block, 0, stream, w, layout, scales, zeros,
                         zero_u8, idx, out, N, K, gs);
      break;
    case PMI_BF16:
      hipLaunchKernelGGL(dequant_kernel<PMI_BF16>, grid, block, 0, stream, w, layout, scales,
                         zeros, zero_u8, idx, out, N, K, gs);
      break;
    default:
      hipLaunchKernelGGL(dequant_kernel<PMI_F32>, grid, block, 0, stream, w, layout, scales, zeros,
                         zero_u8, idx, out, N, K, gs);
  }
  return hipGetLastError();
}

hipError_t launch_rtn(const void* w, int w_dtype, uint8_t* packed, float* scale, float* zero,
                      int64_t N, int64_t K, int64_t gs, int sym, hipStream_t stream) {
  const int64_t units = N * (K / gs);
  const int waves_per_block = 4;
  const dim3 grid((unsigned)((units + waves_per_block - 1) / waves_per_block));
  const dim3 block(64 * waves_per_block);
  switch (w_dtype) {
    case PMI_F32:
      hipLaunchKernelGGL(rtn_kernel<PMI_F32>, grid, block, 0, stream, w, packed, scale, zero, N, K,
                         gs, sym);
      break;
    case PMI_F16:
      hipLaunchKernelGGL(rtn_kernel<PMI_F16>, grid, block, 0, stream, w, packed, scale, zero, N, K,
                         gs, sym);
      break;
    default:
      hipLaunchKernelGGL(rtn_kernel<PMI_BF16>, grid, block, 0, stream, w, packed, scale, zero, N,
                         K, gs, sym);
  }
  return hipGetLastError();
}

}  // namespace pmi
