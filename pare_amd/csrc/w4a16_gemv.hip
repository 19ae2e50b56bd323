// Split-K INT4 W4A16 GEMV for decode (M = 1..4), gfx950.
//
// Work layout. A packed weight row (kernel layout, K/2 bytes) is cut into
// 16-byte chunks; 64 consecutive chunks (2048 columns) form a "slice", the
// K range one wave covers with one 128-bit load per lane. Because the kernel
// layout keeps each 16-byte chunk inside one quantisation group, lane l of a
// wave always needs the same 32 activation values for every row: it loads
// them once, reorders them into fp16 pairs that line up with the nibble
// unpack, and keeps them in registers while the wave walks R weight rows.
// Per row and lane: one 16-byte weight load, one scale and one zero load,
// 4 x (7 bit ops + 4 packed-fp16 subtracts + 4 v_dot2_f32_f16), one fp32 FMA
// with the group scale (the scale is factored out of the group sum).
//
// A workgroup is slice_waves x row_waves waves. The partial sums of a row
// are reduced across the 64 lanes with a transpose-style butterfly, then
// across the slice waves through LDS in a fixed order, so results are
// deterministic and no workspace or atomics are needed.
//
// Semantics follow the reference Triton kernel (pare/kernels/matmul_int4.py:
// 105-176): w = (q - zero) * scale per group, fp32 accumulation, fp16 output.
#include "pmi_common.h"
#include "pmi_launch.h"

namespace pmi {
namespace {

constexpr int kSliceChunks = 64;  // 16-byte chunks per slice (one per lane)

template <int V>
struct Pow2Ceil {
  static constexpr int value = V <= 1 ? 1 : 2 * Pow2Ceil<(V + 1) / 2>::value;
};
template <>
struct Pow2Ceil<1> {
  static constexpr int value = 1;
};

template <int P>
struct Log2 {
  static constexpr int value = 1 + Log2<P / 2>::value;
};
template <>
struct Log2<1> {
  static constexpr int value = 0;
};

// The 32 activations of one row that match this lane's chunk: columns
// k_lo..k_lo+15 (low nibbles) and k_hi..k_hi+15 (high nibbles), reordered so
// xp[4i+c] pairs with d_c of weight word i (see unpack_word_minus_zero).
template <bool PERM>
PMI_DEV void load_x_pairs(const f16* __restrict__ xrow, const int32_t* __restrict__ perm,
                          int k_lo, int k_hi, uint32_t (&xp)[16]) {
  uint32_t a[8], b[8];
  if constexpr (!PERM) {
    const u32x4* pa = reinterpret_cast<const u32x4*>(xrow + k_lo);
    const u32x4* pb = reinterpret_cast<const u32x4*>(xrow + k_hi);
    const u32x4 a0 = pa[0], a1 = pa[1], b0 = pb[0], b1 = pb[1];
    a[0] = a0.x; a[1] = a0.y; a[2] = a0.z; a[3] = a0.w;
    a[4] = a1.x; a[5] = a1.y; a[6] = a1.z; a[7] = a1.w;
    b[0] = b0.x; b[1] = b0.y; b[2] = b0.z; b[3] = b0.w;
    b[4] = b1.x; b[5] = b1.y; b[6] = b1.z; b[7] = b1.w;
  } else {
    const uint16_t* xs = reinterpret_cast<const uint16_t*>(xrow);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = (uint32_t)xs[perm[k_lo + 2 * i]] | ((uint32_t)xs[perm[k_lo + 2 * i + 1]] << 16);
      b[i] = (uint32_t)xs[perm[k_hi + 2 * i]] | ((uint32_t)xs[perm[k_hi + 2 * i + 1]] << 16);
    }
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xp[4 * i + 0] = pair_lo(a[2 * i], a[2 * i + 1]);
    xp[4 * i + 1] = pair_hi(a[2 * i], a[2 * i + 1]);
    xp[4 * i + 2] = pair_lo(b[2 * i], b[2 * i + 1]);
    xp[4 * i + 3] = pair_hi(b[2 * i], b[2 * i + 1]);
  }
}

// Reduces VP values per lane across the wave. Afterwards every lane holds the
// wave-wide sum of value index (lane >> (6 - log2 VP)) in v[0].
template <int VP>
PMI_DEV void wave_transpose_reduce(float (&v)[VP], int lane) {
#pragma unroll
  for (int step = 0; step < 6; ++step) {
    const int o = 32 >> step;
    const int cnt = VP >> step;  // values still held per lane
    if (cnt > 1) {
      const int half = cnt / 2;
      const bool upper = (lane & o) != 0;
#pragma unroll
      for (int i = 0; i < half; ++i) {
        const float send = upper ? v[i] : v[i + half];
        const float keep = upper ? v[i + half] : v[i];
        v[i] = keep + __shfl_xor(send, o, 64);
      }
    } else {
      v[0] += __shfl_xor(v[0], o, 64);
    }
  }
}

template <int MT, int R, bool PERM>
__global__ void __launch_bounds__(512)
w4a16_gemv_kernel(const f16* __restrict__ x, const uint8_t* __restrict__ w,
                  const float* __restrict__ scales, const void* __restrict__ zeros, int zero_u8,
                  const int32_t* __restrict__ perm, f16* __restrict__ y, int N, int K, int gs,
                  int n_slices, int slice_waves, int row_waves) {
  constexpr int V = R * MT;
  constexpr int VP = Pow2Ceil<V>::value;
  constexpr int LOGV = Log2<VP>::value;
  extern __shared__ float red[];  // [row_waves][slice_waves][V]

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int ws = wave % slice_waves;
  const int wr = wave / slice_waves;
  const int row_chunks = K >> 5;
  const int hgs = gs >> 1;  // bytes per group tile
  const int G = K / gs;
  const int64_t row_bytes = K >> 1;
  const int n0 = (blockIdx.x * row_waves + wr) * R;

  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.f;

  for (int s = ws; s < n_slices; s += slice_waves) {
    const int chunk = s * kSliceChunks + lane;
    if (chunk < row_chunks) {
      const int b = chunk << 4;  // byte offset inside the row
      const int t = b / hgs;     // group (tile) index
      const int j = b - t * hgs;
      const int k_lo = t * gs + j;
      const int k_hi = k_lo + hgs;

      u32x4 wv[R];
      float sc[R];
      uint32_t nz[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const int n = n0 + r;
        if (n < N) {
          wv[r] = *reinterpret_cast<const u32x4*>(w + (int64_t)n * row_bytes + b);
          sc[r] = scales[(int64_t)n * G + t];
          nz[r] = neg_magic_zero_x2(load_zero(zeros, zero_u8, (int64_t)n * G + t));
        } else {
          wv[r] = u32x4{0u, 0u, 0u, 0u};
          sc[r] = 0.f;
          nz[r] = neg_magic_zero_x2(0u);
        }
      }

      uint32_t xp[MT][16];
#pragma unroll
      for (int m = 0; m < MT; ++m) load_x_pairs<PERM>(x + (int64_t)m * K, perm, k_lo, k_hi, xp[m]);

#pragma unroll
      for (int r = 0; r < R; ++r) {
        float p[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) p[m] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          f16x2 d0, d1, d2, d3;
          unpack_word_minus_zero(wv[r][i], nz[r], d0, d1, d2, d3);
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            p[m] = dot2_acc(d0, xp[m][4 * i + 0], p[m]);
            p[m] = dot2_acc(d1, xp[m][4 * i + 1], p[m]);
            p[m] = dot2_acc(d2, xp[m][4 * i + 2], p[m]);
            p[m] = dot2_acc(d3, xp[m][4 * i + 3], p[m]);
          }
        }
#pragma unroll
        for (int m = 0; m < MT; ++m) acc[r][m] = fmaf(p[m], sc[r], acc[r][m]);
      }
    }
  }

  float v[VP];
#pragma unroll
  for (int i = 0; i < VP; ++i) v[i] = 0.f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) v[r * MT + m] = acc[r][m];
  wave_transpose_reduce<VP>(v, lane);

  const int idx = LOGV == 0 ? 0 : (lane >> (6 - LOGV));
  const bool writer = (lane & ((64 >> LOGV) - 1)) == 0 && idx < V;
  if (slice_waves == 1) {
    if (writer) {
      const int r = idx / MT, m = idx - (idx / MT) * MT;
      const int n = n0 + r;
      if (n < N) y[(int64_t)m * N + n] = (f16)v[0];
    }
    return;
  }
  if (writer) red[(wr * slice_waves + ws) * V + idx] = v[0];
  __syncthreads();
  for (int e = threadIdx.x; e < row_waves * V; e += blockDim.x) {
    const int wr2 = e / V, id2 = e - (e / V) * V;
    float s = 0.f;
    for (int q = 0; q < slice_waves; ++q) s += red[(wr2 * slice_waves + q) * V + id2];
    const int r = id2 / MT, m = id2 - (id2 / MT) * MT;
    const int n = (blockIdx.x * row_waves + wr2) * R + r;
    if (n < N) y[(int64_t)m * N + n] = (f16)s;
  }
}

template <int MT, int R>
hipError_t launch_mt_r(const GemvConfig& c, const void* x, const uint8_t* w, const float* scales,
                       const void* zeros, int zero_u8, const int32_t* perm, void* y, int N, int K,
                       int gs, hipStream_t stream) {
  const dim3 block(64 * c.slice_waves * c.row_waves);
  const size_t lds = c.slice_waves > 1 ? sizeof(float) * c.row_waves * c.slice_waves * R * MT : 0;
  if (perm)
    hipLaunchKernelGGL((w4a16_gemv_kernel<MT, R, true>), dim3(c.grid), block, lds, stream,
                       (const f16*)x, w, scales, zeros, zero_u8, perm, (f16*)y, N, K, gs,
                       c.n_slices, c.slice_waves, c.row_waves);
  else
    hipLaunchKernelGGL((w4a16_gemv_kernel<MT, R, false>), dim3(c.grid), block, lds, stream,
                       (const f16*)x, w, scales, zeros, zero_u8, perm, (f16*)y, N, K, gs,
                       c.n_slices, c.slice_waves, c.row_waves);
  return hipGetLastError();
}

template <int MT>
hipError_t launch_mt(const GemvConfig& c, const void* x, const uint8_t* w, const float* scales,
                     const void* zeros, int zero_u8, const int32_t* perm, void* y, int N, int K,
                     int gs, hipStream_t stream) {
  switch (c.rows_per_wave) {
    case 1: return launch_mt_r<MT, 1>(c, x, w, scales, zeros, zero_u8, perm, y, N, K, gs, stream);
    case 2: return launch_mt_r<MT, 2>(c, x, w, scales, zeros, zero_u8, perm, y, N, K, gs, stream);
    case 4: return launch_mt_r<MT, 4>(c, x, w, scales, zeros, zero_u8, perm, y, N, K, gs, stream);
    default: return launch_mt_r<MT, 8>(c, x, w, scales, zeros, zero_u8, perm, y, N, K, gs, stream);
  }
}

int env_int(const char* name, int dflt) {
  const char* s = getenv(name);
  return (s && *s) ? atoi(s) : dflt;
}

}  // namespace

GemvConfig gemv_config(int64_t M, int64_t N, int64_t K) {
  (void)M;
  GemvConfig c;
  const int64_t row_chunks = K / 32;
  c.n_slices = (int)((row_chunks + kSliceChunks - 1) / kSliceChunks);
  // At most 8 waves per workgroup (512 threads) so a wave may use 256 VGPRs.
  c.slice_waves = c.n_slices < 8 ? c.n_slices : 8;
  c.row_waves = 8 / c.slice_waves;
  // Tuning overrides (benchmark sweeps only).
  static const int env_r = env_int("PMI_GEMV_R", 0);
  static const int env_wr = env_int("PMI_GEMV_ROW_WAVES", 0);
  if (env_wr > 0 && env_wr * c.slice_waves <= 8) c.row_waves = env_wr;
  int R = 8;
  while (R > 1 && (N + (int64_t)c.row_waves * R - 1) / ((int64_t)c.row_waves * R) < 512) R /= 2;
  if (env_r == 1 || env_r == 2 || env_r == 4 || env_r == 8) R = env_r;
  c.rows_per_wave = R;
  c.grid = (int)((N + (int64_t)c.row_waves * R - 1) / ((int64_t)c.row_waves * R));
  return c;
}

hipError_t launch_gemv(const void* x, const uint8_t* w, const float* scales, const void* zeros,
                       int zero_u8, const int32_t* perm, void* y, int64_t M, int64_t N,
                       int64_t K, int64_t gs, hipStream_t stream) {
  const GemvConfig c = gemv_config(M, N, K);
  switch (M) {
    case 1: return launch_mt<1>(c, x, w, scales, zeros, zero_u8, perm, y, (int)N, (int)K, (int)gs, stream);
    case 2: return launch_mt<2>(c, x, w, scales, zeros, zero_u8, perm, y, (int)N, (int)K, (int)gs, stream);
    case 3: return launch_mt<3>(c, x, w, scales, zeros, zero_u8, perm, y, (int)N, (int)K, (int)gs, stream);
    case 4: return launch_mt<4>(c, x, w, scales, zeros, zero_u8, perm, y, (int)N, (int)K, (int)gs, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pmi
