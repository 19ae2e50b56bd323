// GPTQ producer kernels (pare/schemes/gptq.py:156-263): the sequential column
// loop of one 128-column block, the per-group scale/zero of the dynamic-group
// (desc_act) variant, and the final un-permute + INT4 pack. The Cholesky chain
// and the lazy update of the columns right of a block are library work
// (rocSOLVER / rocBLAS through torch) driven by the host.
//
// Rows are independent in GPTQ: row n's codes depend only on W[n, :] and the
// shared factor C. A workgroup owns 128 rows, one per lane, and keeps the
// block's transposed C (66 KB, padded) and its rows' block of W (64 KB) in LDS.
#include "../../include/pare_amd.h"
#include "pmi_common.h"
#include "pmi_launch.h"

namespace pmi {
namespace {

constexpr int kRows = 128;      // rows (lanes) per workgroup
constexpr int kBlk = 128;       // GPTQ block (gptq.py:42)
constexpr int kSub = 16;        // columns held in registers at a time
constexpr int kCtStride = 132;  // padded row of the transposed C block (floats)

// scale[n, g], zero[n, g] from W[n, c0 : c0 + cols] (row stride ldw), one
// wave per row.
__global__ void group_params_kernel(const float* __restrict__ w, int64_t ldw, int64_t N,
                                    int64_t c0, int64_t cols, int sym, float* __restrict__ scale,
                                    float* __restrict__ zero, int64_t G, int64_t g) {
  const int lane = threadIdx.x & 63;
  const int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  if (n >= N) return;
  const float* row = w + n * ldw + c0;
  float mn = __builtin_inff(), mx = -__builtin_inff();
  for (int64_t c = lane; c < cols; c += 64) {
    mn = fminf(mn, row[c]);
    mx = fmaxf(mx, row[c]);
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    mn = fminf(mn, __shfl_xor(mn, o, 64));
    mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  }
  float s, z;
  scale_zero_from_minmax(mn, mx, sym, s, z);
  if (lane == 0) {
    scale[n * G + g] = s;
    zero[n * G + g] = z;
  }
}

// One GPTQ block, columns b0 .. b0 + count - 1 of the permuted W [N, K]:
// per column j, q = clamp(rint(w / s + z), 0, 15) with the scale/zero of group
// colg[j]; e = (w - (q - z) s) / C[j, j]; every later column of the block
// gets w -= e * C[j, later], in order of j (one rounded product and one
// subtraction per step, as gptq.py:241-249 computes it). Writes the codes to
// qt [K, N] (processed column order, column-major so stores coalesce) and the
// errors to et [count, N] for the host's lazy update.
__global__ void __launch_bounds__(kRows) gptq_block_kernel(
    const float* __restrict__ w, const float* __restrict__ c, const int32_t* __restrict__ colg,
    const float* __restrict__ scale, const float* __restrict__ zero, uint8_t* __restrict__ qt,
    float* __restrict__ et, int64_t N, int64_t K, int64_t G, int64_t b0, int count) {
  __shared__ __attribute__((aligned(16))) float ct[kBlk * kCtStride];  // C[b0 + k][b0 + j] at [j][k]
  __shared__ float wl[kBlk * kRows];                                    // W[row][b0 + j] at [j][lane]
  const int t = threadIdx.x;
  const int64_t n = (int64_t)blockIdx.x * kRows + t;
  const bool live = n < N;

  // transposed C block: thread t reads row k = (i / count) contiguous in j
  for (int i = t; i < count * count; i += kRows) {
    const int k = i / count, j = i - k * count;
    ct[j * kCtStride + k] = c[(b0 + k) * K + b0 + j];
  }
  {
    const float* row = w + (live ? n : 0) * K + b0;
    for (int j = 0; j < count; j += 4) {
      float4 v = live ? *reinterpret_cast<const float4*>(row + j) : float4{0.f, 0.f, 0.f, 0.f};
      wl[(j + 0) * kRows + t] = v.x;
      wl[(j + 1) * kRows + t] = v.y;
      wl[(j + 2) * kRows + t] = v.z;
      wl[(j + 3) * kRows + t] = v.w;
    }
  }
  __syncthreads();

  for (int sb = 0; sb < count; sb += kSub) {
    float wr[kSub], er[kSub];
#pragma unroll
    for (int i = 0; i < kSub; ++i) wr[i] = wl[(sb + i) * kRows + t];
#pragma unroll
    for (int i = 0; i < kSub; ++i) {
      const int j = sb + i;
      const int64_t g = min(max((int64_t)colg[b0 + j], (int64_t)0), G - 1);
      float s = 1.f, z = 0.f;
      if (live) {
        s = scale[n * G + g];
        z = zero[n * G + g];
      }
      const float q = fminf(fmaxf(rintf(wr[i] / s + z), 0.0f), 15.0f);
      const float e = (wr[i] - (q - z) * s) / ct[j * kCtStride + j];
      er[i] = e;
      if (live) {
        qt[(b0 + j) * N + n] = (uint8_t)(int)q;
        et[(int64_t)j * N + n] = e;
      }
#pragma unroll
      for (int i2 = i + 1; i2 < kSub; ++i2) {
        const float p = e * ct[(sb + i2) * kCtStride + j];
        wr[i2] = wr[i2] - p;
      }
    }
    // later columns of the block: this sub-block's errors in column order
    for (int j2 = sb + kSub; j2 < count; ++j2) {
      const float* crow = ct + j2 * kCtStride + sb;
      float v = wl[j2 * kRows + t];
#pragma unroll
      for (int i = 0; i < kSub; ++i) {
        const float p = er[i] * crow[i];
        v = v - p;
      }
      wl[j2 * kRows + t] = v;
    }
  }
}

// packed[n, :] (storage layout, original column order) from the codes qt
// [K, N] in processed order: original column k was processed at step
// inv_perm[k] (identity when inv_perm is null). One thread per (n, 8 columns).
__global__ void gptq_pack_kernel(const uint8_t* __restrict__ qt, const int32_t* __restrict__ inv_perm,
                                 uint8_t* __restrict__ packed, int64_t N, int64_t K) {
  const int64_t words = K >> 3;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < words * N;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t wd = idx / N, n = idx - wd * N;
    uint32_t v = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int64_t k = wd * 8 + i;
      const int64_t p = inv_perm ? (int64_t)inv_perm[k] : k;
      const int64_t j = (p >= 0 && p < K) ? p : k;
      v |= ((uint32_t)qt[j * N + n] & 0xFu) << (4 * i);
    }
    *reinterpret_cast<uint32_t*>(packed + n * (K >> 1) + wd * 4) = v;
  }
}

}  // namespace

hipError_t launch_gptq_group_params(const float* w, int64_t ldw, int64_t N, int64_t c0,
                                    int64_t cols, int sym, float* scale, float* zero, int64_t G,
                                    int64_t g, hipStream_t stream) {
  const int waves = 4;
  hipLaunchKernelGGL(group_params_kernel, dim3((unsigned)((N + waves - 1) / waves)),
                     dim3(64 * waves), 0, stream, w, ldw, N, c0, cols, sym, scale, zero, G, g);
  return hipGetLastError();
}

hipError_t launch_gptq_block(const float* w, const float* c, const int32_t* colg,
                             const float* scale, const float* zero, uint8_t* qt, float* et,
                             int64_t N, int64_t K, int64_t G, int64_t b0, int count,
                             hipStream_t stream) {
  hipLaunchKernelGGL(gptq_block_kernel, dim3((unsigned)((N + kRows - 1) / kRows)), dim3(kRows), 0,
                     stream, w, c, colg, scale, zero, qt, et, N, K, G, b0, count);
  return hipGetLastError();
}

hipError_t launch_gptq_pack(const uint8_t* qt, const int32_t* inv_perm, uint8_t* packed, int64_t N,
                            int64_t K, hipStream_t stream) {
  int64_t blocks = ((K / 8) * N + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks < 1) blocks = 1;
  hipLaunchKernelGGL(gptq_pack_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, qt, inv_perm,
                     packed, N, K);
  return hipGetLastError();
}

}  // namespace pmi
