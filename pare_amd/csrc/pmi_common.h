// Shared device helpers for the gfx950 INT4 W4A16 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

#define PMI_DEV __device__ __forceinline__

// fp16 bit pattern 0x6400 is 1024.0; a nibble q in its low mantissa bits
// gives exactly 1024 + q.

PMI_DEV f16x2 as_f16x2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
PMI_DEV uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// Packed -(1024 + z) in both halves, for an integer zero point z in [0, 15]:
// 1024 + z has bit pattern 0x6400 | z, and the sign bit makes it 0xE400 | z.
PMI_DEV uint32_t neg_magic_zero_x2(uint32_t z) { return (0xE400u | z) * 0x00010001u; }

// Four half2 values (q - z) from one 32-bit word w of packed nibbles.
// With bytes b0..b3 of w (byte i = lo_i | hi_i << 4) the results are
//   d0 = (lo0, lo2), d1 = (lo1, lo3), d2 = (hi0, hi2), d3 = (hi1, hi3).
// The nibbles are first spread to one per byte; v_perm_b32 then places each
// nibble under a 0x64 high byte, giving the fp16 value 1024 + q. Every
// result is an integer in [-15, 15], so the fp16 subtraction is exact.
// 7 bit ops + 4 packed-fp16 subtracts per word.
PMI_DEV void unpack_word_minus_zero(uint32_t w, uint32_t nz, f16x2& d0, f16x2& d1,
                                    f16x2& d2, f16x2& d3) {
  const f16x2 z2 = as_f16x2(nz);
  const uint32_t lo = w & 0x0F0F0F0Fu;
  const uint32_t hi = (w >> 4) & 0x0F0F0F0Fu;
  // selector bytes 0..3 pick from the second operand, 4 picks 0x64
  d0 = as_f16x2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04020400u)) + z2;
  d1 = as_f16x2(__builtin_amdgcn_perm(0x64646464u, lo, 0x04030401u)) + z2;
  d2 = as_f16x2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04020400u)) + z2;
  d3 = as_f16x2(__builtin_amdgcn_perm(0x64646464u, hi, 0x04030401u)) + z2;
}

// (a.lo16, b.lo16) and (a.hi16, b.hi16) of two words holding consecutive
// fp16 pairs: turns x[4i..4i+3] into the pairs (x0,x2) and (x1,x3) that
// line up with d0/d1 (or d2/d3) above.
PMI_DEV uint32_t pair_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
PMI_DEV uint32_t pair_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// silu(g) * u of two fp16 pairs, each half rounded as pmi_silu_mul_f16 rounds
// it: the gate's silu to fp16 first, then the product.
PMI_DEV uint32_t glu_pair(uint32_t g, uint32_t u) {
  const f16x2 gh = as_f16x2(g), uh = as_f16x2(u);
  f16x2 o;
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const float gf = (float)gh[e];
    const float sg = (float)(f16)(gf * __builtin_amdgcn_rcpf(1.f + __expf(-gf)));
    o[e] = (f16)(sg * (float)uh[e]);
  }
  return as_u32(o);
}

PMI_DEV float dot2_acc(f16x2 a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(a, as_f16x2(b), c, false);
}

// fp32 -> fp16, round to nearest even, from a materialised fp32 value. The
// empty asm keeps the backend from folding the producer of v into the
// conversion: (f16)(a * b) would otherwise become one v_fma_mixlo_f16 that
// rounds the exact product once, where the reference rounds to fp32 first
// and then to fp16 (they differ when the fp32 product is an fp16 tie).
PMI_DEV f16 f32_to_f16_rne(float v) {
  asm volatile("" : "+v"(v));
  return (f16)v;
}

// fp32 -> bf16 bits, round to nearest even (NaN kept quiet).
PMI_DEV uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// Loads a zero point for (row n, group g) as an integer 0..15.
PMI_DEV uint32_t load_zero(const void* zeros, int zero_u8, int64_t idx) {
  if (zero_u8) return (uint32_t)((const uint8_t*)zeros)[idx];
  return (uint32_t)(int)((const float*)zeros)[idx];
}

// Column index read from a caller-supplied permutation, clamped into [0, K)
// so a malformed permutation cannot make a kernel read outside the row.
PMI_DEV int perm_col(const int32_t* __restrict__ perm, int k, int K) {
  const int p = perm[k];
  return (unsigned)p < (unsigned)K ? p : 0;
}

// ---- buffer resources, LDS DMA and barriers (MFMA GEMM kernels) -----------

typedef __attribute__((address_space(3))) void* lds_ptr;

// Division by a launch constant d >= 1 without a division sequence in the
// kernel (one is ~25 dependent instructions): the host passes
// m = udiv_magic(d) = ceil(2^32 / d) (0 for d = 1), and umulhi(n, m) is
// floor(n / d) or one more; one compare corrects it. Exact for n < 2^31.
inline uint32_t udiv_magic(uint32_t d) {
  return d <= 1 ? 0u : (uint32_t)(((1ull << 32) + d - 1) / d);
}
PMI_DEV uint32_t udiv(uint32_t n, uint32_t d, uint32_t m) {
  if (m == 0) return n;
  const uint32_t q = __umulhi(n, m);
  return q * d > n ? q - 1 : q;
}

// Raw buffer resource over `bytes` bytes (untyped dword access, no swizzle).
PMI_DEV __amdgpu_buffer_rsrc_t rsrc(const void* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding).
template <int N>
PMI_DEV void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | 0xF00 | ((N >> 4) << 14));
}

// s_waitcnt vmcnt(N) lgkmcnt(0): all but the N youngest vector-memory
// operations and every LDS operation of this wave are complete
template <int N>
PMI_DEV void wait_vmcnt_lgkm0() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | 0x70 | ((N >> 4) << 14));
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

// Workgroup barrier without the fence of __syncthreads(): that fence counts
// in-flight buffer->LDS copies as pending LDS stores and would drain the whole
// ring at every step. Callers order memory themselves (vmcnt waits before,
// operands consumed before); the clobber keeps the compiler from moving
// memory accesses across it.
PMI_DEV void barrier_only() { asm volatile("s_barrier" ::: "memory"); }

// Sum over the 64 lanes of a wave, halving distances 32 .. 1: the order of
// the additions is part of the residual RMSNorm's result, which both the
// add + RMSNorm kernel and the tiled GEMM's fused norm prologue form with it.
PMI_DEV float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// MFMA B operand: 8 nibbles (the low nibbles of the bytes of t0, t1, already
// masked to 0x0F0F0F0F) as fp16 (q - z) in byte order, exact: v_perm_b32 puts
// each nibble under a 0x64 exponent byte (1024 + q) and a packed add of
// nz = -(1024 + z) in both halves subtracts the zero point.
PMI_DEV f16x8 b_operand(uint32_t t0, uint32_t t1, f16x2 nz) {
  const uint32_t K = 0x64646464u;
  const f16x2 h0 = as_f16x2(__builtin_amdgcn_perm(K, t0, 0x04010400u)) + nz;
  const f16x2 h1 = as_f16x2(__builtin_amdgcn_perm(K, t0, 0x04030402u)) + nz;
  const f16x2 h2 = as_f16x2(__builtin_amdgcn_perm(K, t1, 0x04010400u)) + nz;
  const f16x2 h3 = as_f16x2(__builtin_amdgcn_perm(K, t1, 0x04030402u)) + nz;
  const u32x4 r = {as_u32(h0), as_u32(h1), as_u32(h2), as_u32(h3)};
  return __builtin_bit_cast(f16x8, r);
}

// The same 8 nibbles as bf16 128 + q, exact: v_perm_b32 under a 0x43 byte
// (bf16 has no packed subtract on gfx950; the zero point is taken off by a
// separate MFMA whose operand is -(128 + z)).
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
PMI_DEV bf16x8 b_operand_bf16(uint32_t t0, uint32_t t1) {
  const uint32_t K = 0x43434343u;
  const u32x4 r = {__builtin_amdgcn_perm(K, t0, 0x04010400u), __builtin_amdgcn_perm(K, t0, 0x04030402u),
                   __builtin_amdgcn_perm(K, t1, 0x04010400u), __builtin_amdgcn_perm(K, t1, 0x04030402u)};
  return __builtin_bit_cast(bf16x8, r);
}

// (scale, zero) of an INT4 group from its min and max, qmin = 0, qmax = 15.
// sym 0: asymmetric (pare/core/scale.py:83-91); 1: the reference's symmetric
// rule on the unsigned grid (scale.py:73-82: zero 0, so negative weights clamp
// to code 0); 2: offset-8 symmetric, zero 8 and scale 2 max|w| / 15.
PMI_DEV void scale_zero_from_minmax(float mn, float mx, int sym, float& scale, float& zero) {
  if (sym == 2) {
    const float amax = fmaxf(fmaxf(fabsf(mn), fabsf(mx)), 1e-8f);
    scale = 2.0f * amax / 15.0f;
    zero = 8.0f;
  } else if (sym == 1) {
    const float amax = fmaxf(fmaxf(fabsf(mn), fabsf(mx)), 1e-8f);
    scale = amax / 15.0f;
    zero = 0.0f;
  } else {
    mn = fminf(mn, 0.0f);
    mx = fmaxf(mx, 0.0f);
    scale = fmaxf((mx - mn) / 15.0f, 1e-8f);
    zero = fminf(fmaxf(rintf(-mn / scale + 0.0f), 0.0f), 15.0f);
  }
}
