// Split-K INT4 W4A16 GEMV for decode (M = 1..4), gfx950.
//
// Work layout. A packed weight row (kernel layout, K/2 bytes) is cut into
// 16-byte chunks; 64 consecutive chunks (2048 columns) form a "slice", the K
// range one wave covers with one 128-bit load per lane. The kernel layout keeps
// every 16-byte chunk inside one quantisation group, so lane l of a wave needs
// the same 32 activations for every weight row: it loads them once, reorders
// them into fp16 pairs that line up with the nibble unpack, and keeps them in
// registers for the life of the wave, together with their sum Sx.
//
// Arithmetic. A nibble masked into an fp16 half in place is a subnormal:
// bits 0-3 give q * 2^-24, bits 4-7 give q * 2^-20, both exact.
// v_dot2_f32_f16 on those halves and the activation pairs forms exact products
// with fp32 sums; low and high nibbles go to separate accumulators, and the
// group term is s * (2^24 * sum_lo + 2^20 * sum_hi - z * Sx) = s * sum x*(q - z).
// Per 32-bit word of nibbles: 5 bit ops + 4 v_dot2_f32_f16.
//
// Pipeline. A workgroup is slice_waves x row_waves waves and owns a contiguous
// range of rows. Each wave walks its rows in batches of U through a D-deep
// register ring: buffer loads of batch i+D-1 (row offsets in SGPRs, so no
// address VALU) are issued before batch i is unpacked and reduced. Every load
// is unconditional, so the compiler waits for exactly the older batch. The
// weight loads are non-temporal: each 16-byte chunk is read once, and keeping
// the stream out of the caches' normal replacement gave 3-5 % on every shape.
//
// Reduction. Partial sums of a batch are reduced across the 64 lanes with a
// transpose butterfly (v_permlane32_swap / v_permlane16_swap for the two wide
// steps, DPP row_mirror / row_half_mirror / quad_perm for the rest). Waves of
// one workgroup do not synchronise while streaming: per-row partials of the
// slice waves wait in LDS and are added in a fixed order after one barrier at
// the end. Results are deterministic and no workspace or atomics are used.
//
// bf16 activations (XM 6, the native bf16 extension): the weight operand is
// the bf16 128 + q, exact, one v_perm_b32 per pair under a 0x43 byte (bf16
// has no packed subtract on gfx950), and v_dot2_f32_bf16 forms the exact
// products x (128 + q); per group the lane's term is s * (sum x (128 + q) -
// (128 + z) * Sx) with the bracket formed by one fma, which equals
// s * sum x (q - z) up to the fp32 rounding of the accumulated sums; y is
// rounded to bf16 (nearest even).
//
// Semantics follow the reference Triton kernel (pare/kernels/matmul_int4.py:
// 105-176): w = (q - zero) * scale per group, fp32 accumulation, fp16 output.
#include "pmi_common.h"
#include "pmi_launch.h"

#include <type_traits>

namespace pmi {
namespace {

constexpr int kSliceChunks = 64;  // 16-byte chunks per slice (one per lane)
constexpr int kMaxWaves = 8;      // waves per workgroup

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
// k_lo..k_lo+15 (low nibbles) and k_hi..k_hi+15 (high nibbles), as raw
// consecutive pairs a[i] = (x[k_lo+2i], x[k_lo+2i+1]), b[i] likewise at k_hi.
template <bool PERM>
PMI_DEV void load_x_raw(const f16* __restrict__ xrow, const int32_t* __restrict__ perm, int k_lo,
                        int k_hi, int K, uint32_t (&a)[8], uint32_t (&b)[8]) {
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
      a[i] = (uint32_t)xs[perm_col(perm, k_lo + 2 * i, K)] |
             ((uint32_t)xs[perm_col(perm, k_lo + 2 * i + 1, K)] << 16);
      b[i] = (uint32_t)xs[perm_col(perm, k_hi + 2 * i, K)] |
             ((uint32_t)xs[perm_col(perm, k_hi + 2 * i + 1, K)] << 16);
    }
  }
}

// act_order through LDS (XM 4, 8): the permuted column indices of this lane's
// chunk (k_lo..k_lo+15, k_hi..k_hi+15), clamped into [0, K); the activations
// themselves are staged in LDS by the whole workgroup and gathered from there.
PMI_DEV void load_perm(const int32_t* __restrict__ perm, int k_lo, int k_hi, int K, int (&pl)[16],
                       int (&ph)[16]) {
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    pl[i] = perm_col(perm, k_lo + i, K);
    ph[i] = perm_col(perm, k_hi + i, K);
  }
}

// The same from the 16-bit copy of the permutation (XM 8): two 16-byte loads
// per 16 columns instead of four (k_lo and k_hi are multiples of 16 and the
// host checks the table's 16-byte alignment), entries past K clamped to 0 as
// perm_col clamps them.
PMI_DEV void load_perm16(const uint16_t* __restrict__ p16, int k_lo, int k_hi, int K,
                         int (&pl)[16], int (&ph)[16]) {
  const u32x4* ql = reinterpret_cast<const u32x4*>(p16 + k_lo);
  const u32x4* qh = reinterpret_cast<const u32x4*>(p16 + k_hi);
  const u32x4 l0 = ql[0], l1 = ql[1], h0 = qh[0], h1 = qh[1];
  const uint32_t lw[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
  const uint32_t hw[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const int a = (int)((lw[i >> 1] >> (16 * (i & 1))) & 0xFFFFu);
    const int b = (int)((hw[i >> 1] >> (16 * (i & 1))) & 0xFFFFu);
    pl[i] = a < K ? a : 0;
    ph[i] = b < K ? b : 0;
  }
}

// Reorders the raw pairs so xp[4i+c] lines up with nibble pair c of weight
// word i: (x0,x2), (x1,x3) from the low half, the same from the high half.
PMI_DEV void pair_x(const uint32_t (&a)[8], const uint32_t (&b)[8], uint32_t (&xp)[16]) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xp[4 * i + 0] = pair_lo(a[2 * i], a[2 * i + 1]);
    xp[4 * i + 1] = pair_hi(a[2 * i], a[2 * i + 1]);
    xp[4 * i + 2] = pair_lo(b[2 * i], b[2 * i + 1]);
    xp[4 * i + 3] = pair_hi(b[2 * i], b[2 * i + 1]);
  }
}

// dst = keep + (value of `send` in the partner lane), partner given by a DPP
// control that pairs lanes differing in the step's lane bit.
template <int CTRL>
PMI_DEV float dpp_add(float keep, float send) {
  const int moved = __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, send), CTRL, 0xf, 0xf,
                                                false);
  return keep + __builtin_bit_cast(float, moved);
}

// The sum of v over the 64 lanes, the same value in every lane: within each
// row of 16 lanes by DPP (pairs, quads, halves, rows: quad_perm [1,0,3,2],
// quad_perm [2,3,0,1], row_half_mirror, row_mirror), then the four rows read
// out in order. A fixed order, so every wave of every workgroup forms the
// same float; no LDS round trip (a ds_bpermute butterfly took six).
PMI_DEV float wave_total(float v) {
  v = dpp_add<0xB1>(v, v);
  v = dpp_add<0x4E>(v, v);
  v = dpp_add<0x141>(v, v);
  v = dpp_add<0x140>(v, v);
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

// One transpose step with partner lane^o for o = 32 or 16. After
// v_permlane{32,16}_swap_b32 a, b the pair (a, b) holds, per lane, the own
// and the partner value of one index, so a + b is the pair sum of index i on
// the lower lane and of index i + half on the upper lane. Written as inline
// asm on two tied registers: the compiler builtin's two results were read
// back as the same register when summed (hipcc 7.2), doubling the own value.
// The s_nops cover the VALU-write -> permlane-read hazard on both sides.
template <int O>
PMI_DEV float swap_add(float lo, float hi) {
  uint32_t a = __builtin_bit_cast(uint32_t, lo), b = __builtin_bit_cast(uint32_t, hi);
  if constexpr (O == 32)
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  else
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
  return __builtin_bit_cast(float, a) + __builtin_bit_cast(float, b);
}

// DPP partner controls for lane bits 3, 2, 1, 0: row_mirror (l <-> 15-l),
// row_half_mirror (l <-> 7-l), quad_perm [2,3,0,1], quad_perm [1,0,3,2]. The
// mirrors also flip lower lane bits, which is harmless because the steps run
// from the high bit down and lower bits have not split the values yet.
template <int STEP>
struct DppCtrl;
template <> struct DppCtrl<2> { static constexpr int v = 0x140; };
template <> struct DppCtrl<3> { static constexpr int v = 0x141; };
template <> struct DppCtrl<4> { static constexpr int v = 0x4E; };
template <> struct DppCtrl<5> { static constexpr int v = 0xB1; };

template <int VP, int STEP>
PMI_DEV void reduce_step(float (&v)[VP], int lane) {
  constexpr int o = 32 >> STEP;
  constexpr int cnt = VP >> STEP;  // values still held per lane
  if constexpr (STEP < 2) {
    if constexpr (cnt > 1) {
#pragma unroll
      for (int i = 0; i < cnt / 2; ++i) v[i] = swap_add<o>(v[i], v[i + cnt / 2]);
    } else {
      v[0] = swap_add<o>(v[0], v[0]);
    }
  } else {
    if constexpr (cnt > 1) {
      const bool upper = (lane & o) != 0;
#pragma unroll
      for (int i = 0; i < cnt / 2; ++i) {
        const float send = upper ? v[i] : v[i + cnt / 2];
        const float keep = upper ? v[i + cnt / 2] : v[i];
        v[i] = dpp_add<DppCtrl<STEP>::v>(keep, send);
      }
    } else {
      v[0] = dpp_add<DppCtrl<STEP>::v>(v[0], v[0]);
    }
  }
}

// Reduces VP values per lane across the wave. Afterwards every lane holds the
// wave-wide sum of value index (lane >> (6 - log2 VP)) in v[0].
template <int VP>
PMI_DEV void wave_transpose_reduce(float (&v)[VP], int lane) {
  reduce_step<VP, 0>(v, lane);
  reduce_step<VP, 1>(v, lane);
  reduce_step<VP, 2>(v, lane);
  reduce_step<VP, 3>(v, lane);
  reduce_step<VP, 4>(v, lane);
  reduce_step<VP, 5>(v, lane);
}

// One batch of U weight rows for the SPW slices a lane covers. z holds the raw
// zero point (u8 value or fp32 bits) and is widened and converted only where
// the batch is reduced: widening a u8 load where it is issued made the
// compiler mask the loop-carried registers of the ring before the streaming
// loop, which waits for every load in flight.
template <int U, int SPW, bool ZU8>
struct Batch {
  u32x4 w[SPW][U];
  float s[SPW][U];
  typename std::conditional<ZU8, uint8_t, uint32_t>::type z[SPW][U];
};

struct Rsrc {
  __amdgpu_buffer_rsrc_t w, s, z;
};

// A launch's geometry as the kernel reads it (GemvConfig plus the quotients
// and reciprocals the host works out, gemv_geom).
struct GemvGeom {
  int n_slices, slice_waves, row_waves, rows_per_wg;
  int groups;          // K / gs
  int n_batches;       // ceil(rows_per_wg / (row_waves * U))
  uint32_t sw_magic;   // ceil(2^16 / slice_waves): wave / slice_waves, wave < 16
  uint32_t hgs_magic;  // ceil(2^32 / (gs / 2)): b / (gs / 2) for b * (gs / 2) < 2^32
};

// Raw buffer resource over `bytes` bytes (untyped dword access).
PMI_DEV __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

// Every load is unconditional: rows past the workgroup's range re-read its
// last row (their results are never written) and inactive lanes read byte
// offset 0 (their activations are zero). Row offsets are wave-uniform and go
// in the SGPR offset of the buffer load; lane offsets are fixed per wave.
// The weights are read non-temporally (each byte once per launch); SZNT marks
// the scale and zero-point loads non-temporal too, on plain activations (modes
// 0 and 7, no residual epilogue). Measured in the decode step of four launches
// per layer (graphs over 32 distinct layers, two boxes, A/B/C in one process
// type): 903.7-914.4 us against 919.2-927.2 without the hint, the seven-launch
// step 1137-1140 against 1158-1162, although the down projection alone is
// 0.05-0.15 us slower with it; the launch that follows finds more of L2 free.
// The fused decoder modes keep cached loads (batch-1 decoding 619 against 623
// tok/s with the hint on them).
template <int U, int SPW, bool ZU8, bool SZNT = false>
PMI_DEV void load_batch(Batch<U, SPW, ZU8>& bt, const Rsrc& rs, int first_row, int row_last,
                        int row_bytes, int G, const int (&boff)[SPW], const int (&grp)[SPW]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int n = min(first_row + u, row_last);
#pragma unroll
    for (int sp = 0; sp < SPW; ++sp) {
      const u32x4 wv = __builtin_bit_cast(
          u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs.w, boff[sp], n * row_bytes, 2));
      bt.w[sp][u] = wv;
      constexpr int kAux = SZNT ? 2 : 0;
      bt.s[sp][u] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rs.s, grp[sp] * 4, n * G * 4, kAux));
      if constexpr (ZU8)
        bt.z[sp][u] = __builtin_amdgcn_raw_buffer_load_b8(rs.z, grp[sp], n * G, kAux);
      else
        bt.z[sp][u] = __builtin_amdgcn_raw_buffer_load_b32(rs.z, grp[sp] * 4, n * G * 4, kAux);
    }
  }
}

template <bool ZU8>
PMI_DEV float zero_value(uint32_t raw) {
  if constexpr (ZU8) return (float)raw;
  return __builtin_bit_cast(float, raw);
}

// Unpacks and reduces one batch. Each nibble pair of a weight word is masked
// into an fp16x2 operand in place: low nibbles (bits 0-3 of a half) are the
// subnormals q * 2^-24, high nibbles (bits 4-7) the subnormals q * 2^-20; both
// stay inside the mantissa, so the values are exact and v_dot2_f32_f16 forms
// exact products. The two scales go to separate accumulators, combined per
// row as s * (2^24 * sum_lo + 2^20 * sum_hi - z * Sx). 5 bit ops + 4 dot2 per
// word. After the wave reduction, lane `idx`-writers hold row u's value for
// activation row m in v[0] (idx = u * MT + m).
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

PMI_DEV float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a), __builtin_bit_cast(bf16x2, b), c,
                                         false);
}

template <int MT, int U, int SPW, bool ZU8, bool BF = false>
PMI_DEV void reduce_batch(const Batch<U, SPW, ZU8>& bt, const uint32_t (&xp)[SPW][MT][16],
                          const float (&sx)[SPW][MT], float (&out)[Pow2Ceil<U * MT>::value],
                          int lane) {
  constexpr int VP = Pow2Ceil<U * MT>::value;
  float (&v)[VP] = out;
#pragma unroll
  for (int i = 0; i < VP; ++i) v[i] = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u) {
#pragma unroll
    for (int sp = 0; sp < SPW; ++sp) {
      if constexpr (BF) {
        // bf16: weight pairs (128 + q) in column order, one accumulator
        float pa[MT];
#pragma unroll
        for (int m = 0; m < MT; ++m) pa[m] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t wd = bt.w[sp][u][i];
          const uint32_t lo = wd & 0x0F0F0F0Fu, hi = (wd >> 4) & 0x0F0F0F0Fu;
          const uint32_t b0 = __builtin_amdgcn_perm(0x43434343u, lo, 0x04010400u);
          const uint32_t b1 = __builtin_amdgcn_perm(0x43434343u, lo, 0x04030402u);
          const uint32_t b2 = __builtin_amdgcn_perm(0x43434343u, hi, 0x04010400u);
          const uint32_t b3 = __builtin_amdgcn_perm(0x43434343u, hi, 0x04030402u);
#pragma unroll
          for (int m = 0; m < MT; ++m) {
            pa[m] = dot2_bf16(b0, xp[sp][m][4 * i + 0], pa[m]);
            pa[m] = dot2_bf16(b1, xp[sp][m][4 * i + 1], pa[m]);
            pa[m] = dot2_bf16(b2, xp[sp][m][4 * i + 2], pa[m]);
            pa[m] = dot2_bf16(b3, xp[sp][m][4 * i + 3], pa[m]);
          }
        }
        const float sc = bt.s[sp][u];
        const float zb = -(128.f + zero_value<ZU8>(bt.z[sp][u]));  // -(128 + z), exact
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          float& acc = v[u * MT + m];
          acc = fmaf(sc, fmaf(zb, sx[sp][m], pa[m]), acc);
        }
        continue;
      }
      float pl[MT], ph[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) pl[m] = ph[m] = 0.f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t wd = bt.w[sp][u][i];
        const uint32_t w8 = wd >> 8;
        // (lo0,lo2) (lo1,lo3) as q * 2^-24; (hi0,hi2) (hi1,hi3) as q * 2^-20
        const f16x2 h0 = as_f16x2(wd & 0x000F000Fu);
        const f16x2 h1 = as_f16x2(w8 & 0x000F000Fu);
        const f16x2 h2 = as_f16x2(wd & 0x00F000F0u);
        const f16x2 h3 = as_f16x2(w8 & 0x00F000F0u);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
          pl[m] = dot2_acc(h0, xp[sp][m][4 * i + 0], pl[m]);
          pl[m] = dot2_acc(h1, xp[sp][m][4 * i + 1], pl[m]);
          ph[m] = dot2_acc(h2, xp[sp][m][4 * i + 2], ph[m]);
          ph[m] = dot2_acc(h3, xp[sp][m][4 * i + 3], ph[m]);
        }
      }
      const float sc = bt.s[sp][u];
      const float s24 = sc * 16777216.0f;  // s * 2^24, exact
      const float s20 = sc * 1048576.0f;   // s * 2^20, exact
      const float sz = -sc * zero_value<ZU8>(bt.z[sp][u]);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float& acc = v[u * MT + m];
        acc = fmaf(pl[m], s24, acc);
        acc = fmaf(ph[m], s20, acc);
        acc = fmaf(sz, sx[sp][m], acc);
      }
    }
  }
  wave_transpose_reduce<VP>(v, lane);
}

// Workgroup: slice_waves x row_waves waves owning rows_per_wg contiguous rows.
// Wave (ws, wr) covers slices ws, ws + slice_waves, ... (SPW of them) of rows
// row0 + wr*U + b*stride + u, batch b = 0, 1, ... Batches stream through a
// D-deep register ring: batch b + D - 1 is issued before batch b is reduced,
// so D - 1 batches stay in flight. D = 1 (no ring) is for launches in which
// every wave holds one batch. Waves never synchronise until the end:
// with one slice wave the results go straight to y, otherwise each wave
// parks its per-row partial in LDS and one barrier precedes the fixed-order
// sum over slice waves (deterministic; no atomics, no workspace).
// h = x + r per fp16 pair, rounded as add_rmsnorm_kernel rounds it.
PMI_DEV uint32_t add_pair(uint32_t x, uint32_t r) {
  const f16x2 xh = as_f16x2(x), rh = as_f16x2(r);
  f16x2 o;
  o[0] = (f16)((float)xh[0] + (float)rh[0]);
  o[1] = (f16)((float)xh[1] + (float)rh[1]);
  return as_u32(o);
}

// (f16)(h * inv * w) per fp16 pair, as add_rmsnorm_kernel forms it.
PMI_DEV uint32_t norm_pair(uint32_t h, uint32_t w, float inv) {
  const f16x2 hh = as_f16x2(h), wh = as_f16x2(w);
  f16x2 o;
  o[0] = (f16)((float)hh[0] * inv * (float)wh[0]);
  o[1] = (f16)((float)hh[1] * inv * (float)wh[1]);
  return as_u32(o);
}

PMI_DEV float sq_pairs(const uint32_t (&v)[8], float acc) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const f16x2 h = as_f16x2(v[i]);
    acc = fmaf((float)h[0], (float)h[0], acc);
    acc = fmaf((float)h[1], (float)h[1], acc);
  }
  return acc;
}

// One output: fp16, or with BF the bf16 bits in the same 2-byte slot; both
// round to nearest even.
template <bool BF>
PMI_DEV void store_y(f16* p, float v) {
  if constexpr (BF) *reinterpret_cast<uint16_t*>(p) = f32_to_bf16_rne(v);
  else *p = f32_to_f16_rne(v);
}

// XM selects the activation source: 0 x [M, K]; 1 x[:, perm] (act_order),
// gathered by every lane from global memory; 4 the same, x staged in LDS once
// per workgroup (16-byte loads) and gathered from there; 8 as 4 with the
// 16-bit copy of the permutation (perm then points at uint16 [K]), which
// halves the table every workgroup reads before its first gather;
// 2 the fused gate/up output [M, 2K], consumed as silu(gate) * up;
// 3 RMSNorm(x + r) * w of the residual stream (xf.r nullable), with
// h = x + r written to xf.h_out by workgroup 0; 5 RMSNorm(x) * w of a
// residual stream x whose sum of squares the launch that formed it left as
// per-workgroup partials (xf.stats, xf.n_stats of them): every wave adds them
// in the same fixed order, so no workgroup reduces the row or waits at a
// barrier first; 6 bf16 x [M, K], y bf16 (the native bf16 extension);
// 7 x [M, K] as 0, staged in LDS with one 16-byte load per thread and read
// from there: a workgroup's start-up then puts 8 KiB (K = 4096) of activation
// reads in front of its weight stream, not 8 waves x 4 KiB.
// Epilogue (xf.res, one activation row, slice_waves > 1): y = h = y + res
// rounded as add_rmsnorm_kernel forms h, and xf.stats[blockIdx.x] = the sum of
// h^2 over the workgroup's rows (fixed order), for a mode-5 launch to read.
//
// The launch geometry comes with the divisions a wave would otherwise do
// before its first load worked out on the host (an integer division is ~25
// dependent instructions, and the first weight batch waited for three of
// them): wave / slice_waves = (wave * sw_magic) >> 16 and a lane's byte
// offset b / (gs / 2) = umulhi(b, hgs_magic), both exact in the ranges the
// host checks (gemv_geom).
template <int MT, int U, int D, int SPW, int XM, bool ZU8, bool RES = false>
__global__ void __launch_bounds__(kMaxWaves * 64)
w4a16_gemv_kernel(const f16* __restrict__ x, const uint8_t* __restrict__ w,
                  const float* __restrict__ scales, const void* __restrict__ zeros,
                  const int32_t* __restrict__ perm, f16* __restrict__ y, int N, int K, int gs,
                  GemvGeom gg, GemvXform xf) {
  extern __shared__ float part[];  // [rows_per_wg][slice_waves][MT] when slice_waves > 1
  __shared__ float nrm[XM == 3 ? kMaxWaves * 4 : 1];  // per-wave sums of h^2 (XM 3)
  __shared__ float hred[RES ? kMaxWaves : 1];          // per-wave sums of h^2 (RES)
  constexpr int VP = Pow2Ceil<U * MT>::value;
  constexpr int LOGV = Log2<VP>::value;

  const int n_slices = gg.n_slices, slice_waves = gg.slice_waves;
  const int row_waves = gg.row_waves, rows_per_wg = gg.rows_per_wg;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wr = (int)(((uint32_t)wave * gg.sw_magic) >> 16);
  const int ws = wave - wr * slice_waves;
  const int row_chunks = K >> 5;
  const int hgs = gs >> 1;  // bytes per group tile
  const int G = gg.groups;
  const int row_bytes = K >> 1;
  const int row0 = blockIdx.x * rows_per_wg;
  const int row_lim = min(N, row0 + rows_per_wg);
  const int stride = row_waves * U;
  const int n_batches = gg.n_batches;

  Rsrc rs;
  rs.w = make_rsrc(w, (uint32_t)N * (uint32_t)row_bytes);
  rs.s = make_rsrc(scales, (uint32_t)N * (uint32_t)G * 4u);
  rs.z = make_rsrc(zeros, (uint32_t)N * (uint32_t)G * (ZU8 ? 1u : 4u));

  // Issue order matters: activation loads, then the first weight batches,
  // and only then wait for the activations, so the HBM stream starts at once.
  // sched_barrier keeps the scheduler from sinking loads below the waits.
  int boff[SPW], grp[SPW];
  bool act[SPW];
  uint32_t xa[SPW][MT][8], xb[SPW][MT][8];
  constexpr int kXS = XM == 2 || XM == 3 ? SPW : 1, kXM = XM == 2 || XM == 3 ? MT : 1;
  constexpr int kNS = XM == 3 || XM == 5 ? SPW : 1;
  uint32_t ua[kXS][kXM][8], ub[kXS][kXM][8];  // up (XM 2) or residual (XM 3)
  uint32_t wa[kNS][8], wb[kNS][8];            // norm weight (XM 3, 5)
  constexpr bool kPG = XM == 4 || XM == 8;    // act_order gathered from LDS
  constexpr int kPS = kPG ? SPW : 1;
  int pl[kPS][16], ph[kPS][16];                // permuted columns (XM 4, 8)
  int klo[SPW];
#pragma unroll
  for (int sp = 0; sp < SPW; ++sp) {
    const int s = ws + sp * slice_waves;
    const int chunk = s * kSliceChunks + lane;
    act[sp] = s < n_slices && chunk < row_chunks;
    const int b = act[sp] ? chunk << 4 : 0;
    const int t = (int)__umulhi((uint32_t)b, gg.hgs_magic);  // b / hgs
    const int j = b - t * hgs;
    boff[sp] = b;
    grp[sp] = t;
    const int k_lo = t * gs + j;
    klo[sp] = k_lo;
    if constexpr (XM == 3 || XM == 5)
      load_x_raw<false>(reinterpret_cast<const f16*>(xf.w), perm, k_lo, k_lo + hgs, K, wa[sp],
                        wb[sp]);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
      if constexpr (XM == 3) {
        load_x_raw<false>(x + (int64_t)m * K, perm, k_lo, k_lo + hgs, K, xa[sp][m], xb[sp][m]);
        if (xf.r)
          load_x_raw<false>(reinterpret_cast<const f16*>(xf.r) + (int64_t)m * K, perm, k_lo,
                            k_lo + hgs, K, ua[sp][m], ub[sp][m]);
      } else if constexpr (XM == 2) {
        load_x_raw<false>(x + (int64_t)m * 2 * K, perm, k_lo, k_lo + hgs, K, xa[sp][m], xb[sp][m]);
        load_x_raw<false>(x + (int64_t)m * 2 * K + K, perm, k_lo, k_lo + hgs, K, ua[sp][m],
                          ub[sp][m]);
      } else if constexpr (XM == 4) {
        if (m == 0) load_perm(perm, k_lo, k_lo + hgs, K, pl[sp], ph[sp]);
      } else if constexpr (XM == 8) {
        if (m == 0)
          load_perm16(reinterpret_cast<const uint16_t*>(perm), k_lo, k_lo + hgs, K, pl[sp], ph[sp]);
      } else if constexpr (XM != 7) {
        load_x_raw<XM == 1>(x + (int64_t)m * K, perm, k_lo, k_lo + hgs, K, xa[sp][m], xb[sp][m]);
      }
    }
  }
  // XM 4, 7, 8: the MT activation rows ([MT, K], contiguous) in 16-byte chunks,
  // at most kXCh per thread (the host checks MT * K / 8 <= kXCh * blockDim.x),
  // loaded here and written to LDS after the first weight batch is issued.
  constexpr bool kXL = kPG || XM == 7;
  constexpr bool kSZNT = (XM == 0 || XM == 7) && !RES;  // non-temporal scale / zero loads
  constexpr int kXCh = kPG ? kGemvLdsChunks : XM == 7 ? kGemvXLdsChunks : 1;
  u32x4 xst[kXCh];
  const int n_xch = MT * K / 8;
  f16* lds_x = reinterpret_cast<f16*>(
      reinterpret_cast<uint8_t*>(part) +
      (((slice_waves > 1 ? rows_per_wg * slice_waves * MT * 4 : 0) + 15) & ~15));
  if constexpr (kXL) {
#pragma unroll
    for (int i = 0; i < kXCh; ++i) {
      const int c = (int)threadIdx.x + i * (int)blockDim.x;
      if constexpr (XM == 7) {
        // one chunk per thread, loaded and written without a branch (threads
        // past the rows re-read the last chunk and write it to a spare slot
        // after the rows): in a branch the compiler sank the load below the
        // weight batches and drained them before the write
        xst[i] = reinterpret_cast<const u32x4*>(x)[c < n_xch ? c : n_xch - 1];
      } else {
        xst[i] = c < n_xch ? reinterpret_cast<const u32x4*>(x)[c] : u32x4{0u, 0u, 0u, 0u};
      }
    }
    // issued ahead of the weight batches: a staging load scheduled after them
    // would make its LDS write wait for every batch in flight
    __builtin_amdgcn_sched_barrier(0);
  }
  // XM 5: the producing launch's partials of sum(h^2), lane l holding
  // l, l + 64, ... (the host checks 1 <= n_stats <= 64 kSt). The loads are
  // unconditional (clamped index) and the entries past n_stats are dropped
  // only in setup_x, below the ring's first weight loads: selected here, the
  // values made the compiler wait for these loads before issuing the ring.
  constexpr int kSt = XM == 5 ? 8 : 1;
  float st[kSt];
  if constexpr (XM == 5) {
#pragma unroll
    for (int i = 0; i < kSt; ++i) {
      const int q = lane + 64 * i;
      st[i] = xf.stats[q < xf.n_stats ? q : xf.n_stats - 1];
    }
  }
  // RES: each thread's first output row of the residual, fetched now
  // (clamped to the workgroup's last row; used only by threads that own a
  // row). A template flag, so that no other launch carries this code.
  static_assert(!RES || MT == 1, "the residual epilogue is built for one activation row");
  f16 rpre = (f16)0.f;
  if constexpr (RES) {
    const int e = min((int)threadIdx.x, (row_lim - row0) * MT - 1);
    const int lr = e / MT, m = e - lr * MT;
    rpre = reinterpret_cast<const f16*>(xf.res)[(int64_t)m * N + row0 + lr];
  }

  const int my_row0 = row0 + wr * U;
  const int row_last = row_lim - 1;
  uint32_t xp[SPW][MT][16];
  float sx[SPW][MT];
  // Pairs the activations with the nibble order and sums each lane's 32.
  // XM 4, 8: stage the activations in LDS, then gather this lane's columns;
  // XM 7: stage them in LDS, then read this lane's two 16-column runs
  auto stage_x = [&]() {
    if constexpr (kXL) {
#pragma unroll
      for (int i = 0; i < kXCh; ++i) {
        const int c = (int)threadIdx.x + i * (int)blockDim.x;
        if constexpr (XM == 7)
          reinterpret_cast<u32x4*>(lds_x)[c < n_xch ? c : n_xch] = xst[i];
        else if (c < n_xch)
          reinterpret_cast<u32x4*>(lds_x)[c] = xst[i];
      }
      // own LDS writes done (lgkmcnt(0)), then a bare s_barrier (no vmcnt
      // wait: the weight batches stay in flight)
      __builtin_amdgcn_s_waitcnt(0xC07F);
      barrier_only();
    }
    if constexpr (XM == 7) {
#pragma unroll
      for (int sp = 0; sp < SPW; ++sp)
#pragma unroll
        for (int m = 0; m < MT; ++m)
          load_x_raw<false>(lds_x + m * K, perm, klo[sp], klo[sp] + hgs, K, xa[sp][m], xb[sp][m]);
    }
    if constexpr (kPG) {
      const uint16_t* xs = reinterpret_cast<const uint16_t*>(lds_x);
#pragma unroll
      for (int sp = 0; sp < SPW; ++sp)
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            xa[sp][m][i] = (uint32_t)xs[m * K + pl[sp][2 * i]] |
                           ((uint32_t)xs[m * K + pl[sp][2 * i + 1]] << 16);
            xb[sp][m][i] = (uint32_t)xs[m * K + ph[sp][2 * i]] |
                           ((uint32_t)xs[m * K + ph[sp][2 * i + 1]] << 16);
          }
    }
  };
  auto setup_x = [&]() {
    if constexpr (XM == 3) {
      // h = x + r; the RMS of every activation row over all K columns: each
      // wave sums h^2 over its slices, the slice waves of row-wave group 0
      // (which together cover K once) are added after one barrier.
      float ss[MT];
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        ss[m] = 0.f;
#pragma unroll
        for (int sp = 0; sp < SPW; ++sp) {
          if (xf.r) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
              xa[sp][m][i] = add_pair(xa[sp][m][i], ua[sp][m][i]);
              xb[sp][m][i] = add_pair(xb[sp][m][i], ub[sp][m][i]);
            }
          }
          if (act[sp]) ss[m] = sq_pairs(xb[sp][m], sq_pairs(xa[sp][m], ss[m]));
        }
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) ss[m] += __shfl_xor(ss[m], o, 64);
      }
      if (lane == 0) {
#pragma unroll
        for (int m = 0; m < MT; ++m) nrm[wave * 4 + m] = ss[m];
      }
      // LDS writes done (lgkmcnt(0)), then a bare s_barrier: __syncthreads()
      // would also wait for every weight load in flight (vmcnt(0)) and drain
      // the ring this prologue overlaps
      __builtin_amdgcn_s_waitcnt(0xC07F);
      barrier_only();
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        float tot = 0.f;
        for (int q = 0; q < slice_waves; ++q) tot += nrm[q * 4 + m];
        const float inv = rsqrtf(tot / (float)K + xf.eps);
#pragma unroll
        for (int sp = 0; sp < SPW; ++sp) {
          if (xf.r && blockIdx.x == 0 && wr == 0 && act[sp]) {
            f16* hrow = reinterpret_cast<f16*>(xf.h_out) + (int64_t)m * K;
            u32x4* ha = reinterpret_cast<u32x4*>(hrow + klo[sp]);
            u32x4* hb = reinterpret_cast<u32x4*>(hrow + klo[sp] + hgs);
            ha[0] = u32x4{xa[sp][m][0], xa[sp][m][1], xa[sp][m][2], xa[sp][m][3]};
            ha[1] = u32x4{xa[sp][m][4], xa[sp][m][5], xa[sp][m][6], xa[sp][m][7]};
            hb[0] = u32x4{xb[sp][m][0], xb[sp][m][1], xb[sp][m][2], xb[sp][m][3]};
            hb[1] = u32x4{xb[sp][m][4], xb[sp][m][5], xb[sp][m][6], xb[sp][m][7]};
          }
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            xa[sp][m][i] = norm_pair(xa[sp][m][i], wa[sp][i], inv);
            xb[sp][m][i] = norm_pair(xb[sp][m][i], wb[sp][i], inv);
          }
        }
      }
    }
    if constexpr (XM == 5) {
      // the whole row's sum of squares from the partials, the same fixed
      // order in every wave; then RMSNorm(x) * w rounded as add_rmsnorm_kernel
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < kSt; ++i) acc += lane + 64 * i < xf.n_stats ? st[i] : 0.f;
      const float inv = rsqrtf(wave_total(acc) / (float)K + xf.eps);
#pragma unroll
      for (int sp = 0; sp < SPW; ++sp)
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            xa[sp][m][i] = norm_pair(xa[sp][m][i], wa[sp][i], inv);
            xb[sp][m][i] = norm_pair(xb[sp][m][i], wb[sp][i], inv);
          }
    }
#pragma unroll
    for (int sp = 0; sp < SPW; ++sp)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if constexpr (XM == 2) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            xa[sp][m][i] = glu_pair(xa[sp][m][i], ua[sp][m][i]);
            xb[sp][m][i] = glu_pair(xb[sp][m][i], ub[sp][m][i]);
          }
        }
        if constexpr (XM == 6) {
          // bf16: the pairs in column order, as the weight pairs are formed
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            xp[sp][m][4 * i + 0] = xa[sp][m][2 * i];
            xp[sp][m][4 * i + 1] = xa[sp][m][2 * i + 1];
            xp[sp][m][4 * i + 2] = xb[sp][m][2 * i];
            xp[sp][m][4 * i + 3] = xb[sp][m][2 * i + 1];
          }
        } else {
          pair_x(xa[sp][m], xb[sp][m], xp[sp][m]);
        }
        if (!act[sp]) {
#pragma unroll
          for (int i = 0; i < 16; ++i) xp[sp][m][i] = 0u;
        }
        float acc = 0.f;
        if constexpr (XM == 6) {
#pragma unroll
          for (int i = 0; i < 16; ++i) acc = dot2_bf16(0x3F803F80u, xp[sp][m][i], acc);
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) acc = dot2_acc(as_f16x2(0x3C003C00u), xp[sp][m][i], acc);
        }
        sx[sp][m] = acc;
      }
  };
  const int idx = LOGV == 0 ? 0 : (lane >> (6 - LOGV));
  const bool writer = (lane & ((64 >> LOGV) - 1)) == 0 && idx < U * MT;
  const int wu = idx / MT, wm = idx - (idx / MT) * MT;
  // Reduces batch b and stores (or parks) its results.
  auto finish = [&](const Batch<U, SPW, ZU8>& bt, int b) {
    float v[VP];
    reduce_batch<MT, U, SPW, ZU8, XM == 6>(bt, xp, sx, v, lane);
    if (writer) {
      const int lr = wr * U + b * stride + wu;  // row within the workgroup
      if (row0 + lr < row_lim) {
        if (slice_waves == 1)
          store_y<XM == 6>(y + (int64_t)wm * N + row0 + lr, v[0]);
        else
          part[(lr * slice_waves + ws) * MT + wm] = v[0];
      }
    }
  };

  if constexpr (D == 1) {
    // No ring (the host picks it when every wave has one batch): batches go
    // one after the other, the first load ahead of the activation setup.
    Batch<U, SPW, ZU8> bt;
    load_batch<U, SPW, ZU8, kSZNT>(bt, rs, my_row0, row_last, row_bytes, G, boff, grp);
    __builtin_amdgcn_sched_barrier(0);
    stage_x();
    setup_x();
    finish(bt, 0);
    for (int b = 1; b < n_batches; ++b) {
      load_batch<U, SPW, ZU8, kSZNT>(bt, rs, my_row0 + b * stride, row_last, row_bytes, G, boff, grp);
      finish(bt, b);
    }
  } else {
    Batch<U, SPW, ZU8> ring[D];
#pragma unroll
    for (int d = 0; d < D - 1; ++d)
      load_batch<U, SPW, ZU8, kSZNT>(ring[d], rs, my_row0 + d * stride, row_last, row_bytes, G, boff,
                              grp);
    __builtin_amdgcn_sched_barrier(0);
    stage_x();
    setup_x();
    // Steady state, unrolled by D so every ring slot is a fixed register set.
    // Step b issues the loads of batch b + D - 1 unconditionally (past the
    // last batch it re-reads the last row), so the wait before a reduction is
    // always for exactly the D - 1 younger batches. Whole rounds of D steps
    // first, with no exit inside a round: an exit path into the loop head made
    // the compiler wait for all but one batch at the first step of every
    // round. The last n_batches % D steps only reduce: every batch they would
    // load lies past the end.
    const int n_full = n_batches - n_batches % D;
    int i = 0;
    for (; i < n_full; i += D) {
#pragma unroll
      for (int d = 0; d < D; ++d) {
        load_batch<U, SPW, ZU8, kSZNT>(ring[(d + D - 1) % D], rs, my_row0 + (i + d + D - 1) * stride,
                                row_last, row_bytes, G, boff, grp);
        __builtin_amdgcn_sched_barrier(0);
        finish(ring[d], i + d);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
#pragma unroll
    for (int d = 0; d < D - 1; ++d)
      if (i + d < n_batches) finish(ring[d], i + d);
  }
  if (slice_waves == 1) return;
  __syncthreads();
  const int nr = row_lim - row0;
  float hsq = 0.f;
  for (int e = threadIdx.x; e < nr * MT; e += blockDim.x) {
    const int lr = e / MT, m = e - (e / MT) * MT;
    float s = 0.f;
    for (int q = 0; q < slice_waves; ++q) s += part[(lr * slice_waves + q) * MT + m];
    if constexpr (XM == 6) {
      store_y<true>(y + (int64_t)m * N + row0 + lr, s);
      continue;
    }
    f16 yv = f32_to_f16_rne(s);
    if constexpr (RES) {
      const f16 rv = e == (int)threadIdx.x ? rpre
                                           : reinterpret_cast<const f16*>(xf.res)[(int64_t)m * N + row0 + lr];
      yv = (f16)((float)yv + (float)rv);
      hsq = fmaf((float)yv, (float)yv, hsq);
    }
    y[(int64_t)m * N + row0 + lr] = yv;
  }
  if constexpr (RES) {
    // the workgroup's sum of h^2: per wave, then the waves in order; when its
    // rows fit wave 0 (one row per lane above), wave 0 alone, no barrier
    if (nr * MT <= 64) {
      if (wave == 0) {
        const float t = wave_total(hsq);
        if (lane == 0) xf.stats[blockIdx.x] = t;
      }
    } else {
      hsq = wave_total(hsq);
      if (lane == 0) hred[wave] = hsq;
      __syncthreads();
      if (threadIdx.x == 0) {
        float t = 0.f;
        for (int q = 0; q < (int)(blockDim.x >> 6); ++q) t += hred[q];
        xf.stats[blockIdx.x] = t;
      }
    }
  }
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

// The kernel's geometry for a launch of U rows per batch; false when a
// quotient would leave the range in which its reciprocal is exact (rows of
// 2^17 columns or more).
bool gemv_geom(const GemvConfig& c, int U, int K, int gs, GemvGeom& g) {
  const uint32_t hgs = (uint32_t)gs / 2u;
  if (c.slice_waves < 1 || c.slice_waves > kMaxWaves || hgs < 1 ||
      (uint64_t)(K / 2) * hgs >= (1ull << 32))
    return false;
  const int stride = c.row_waves * U;
  g.n_slices = c.n_slices;
  g.slice_waves = c.slice_waves;
  g.row_waves = c.row_waves;
  g.rows_per_wg = c.rows_per_wg;
  g.groups = K / gs;
  g.n_batches = (c.rows_per_wg + stride - 1) / stride;
  g.sw_magic = (65536u + (uint32_t)c.slice_waves - 1u) / (uint32_t)c.slice_waves;
  g.hgs_magic = (uint32_t)(((1ull << 32) + hgs - 1) / hgs);
  return true;
}

template <int MT, int U, int D, int SPW>
hipError_t launch_cfg(const GemvConfig& c, const void* x, const uint8_t* w, const float* scales,
                      const void* zeros, int zero_u8, const int32_t* perm, void* y, int N, int K,
                      int gs, const GemvXform& xf, hipStream_t stream) {
  const dim3 block(64 * c.slice_waves * c.row_waves);
  GemvGeom gg;
  if (!gemv_geom(c, U, K, gs, gg)) return hipErrorInvalidValue;
  // XM 4 and 8 (xf.mode 4, 8): the activation rows staged in LDS after the partials;
  // plain activations (XM 7 for 0) likewise where several row waves would
  // each load the same slices, the rows fit one chunk per thread, and either
  // a ring or several workgroups per CU multiply those loads (A/B on MI355X,
  // us: fused q/k/v, three workgroups per CU, 5.01 -> 4.75; gate 7.75 ->
  // 7.67; fused gate/up 12.5 -> 12.45). One workgroup per CU with one batch
  // per wave (q/o, k/v) lost 0.1-0.2 to the barrier and keeps its registers.
  const bool perm_lds = perm && (xf.mode == 4 || xf.mode == 8);
  if (perm_lds && !gemv_perm_lds_fits(MT, K, (int)block.x)) return hipErrorInvalidValue;
  static const bool env_xlds = env_int("PMI_GEMV_XLDS", 1) != 0;  // benchmark sweeps only
  const bool x_lds = env_xlds && !perm && xf.mode == 0 && c.row_waves > 1 &&
                     (D > 1 || c.grid > device_cus()) && gemv_x_lds_fits(MT, K, (int)block.x);
  // (XM 7 writes one spare 16-byte slot after the rows)
  const size_t lds = perm_lds || x_lds
                         ? (((size_t)c.lds_bytes + 15) & ~(size_t)15) + (size_t)MT * K * 2 +
                               (x_lds ? 16 : 0)
                         : (size_t)c.lds_bytes;
#define PMI_GEMV_LAUNCH(XM, Z)                                                                  \
  hipLaunchKernelGGL((w4a16_gemv_kernel<MT, U, D, SPW, XM, Z>), dim3(c.grid), block, lds, stream, \
                     (const f16*)x, w, scales, zeros, perm, (f16*)y, N, K, gs, gg, xf)
  if (xf.res) {
    // the residual epilogue: one activation row, plain or SiLU(gate) * up
    // activations, u8 zero points, no permutation
    if constexpr (MT == 1) {
      if (!zero_u8 || perm || (xf.mode != 0 && xf.mode != 2) || c.slice_waves < 2)
        return hipErrorInvalidValue;
      if (xf.mode == 2)
        hipLaunchKernelGGL((w4a16_gemv_kernel<MT, U, D, SPW, 2, true, true>), dim3(c.grid), block,
                           lds, stream, (const f16*)x, w, scales, zeros, perm, (f16*)y, N, K, gs,
                           gg, xf);
      else
        hipLaunchKernelGGL((w4a16_gemv_kernel<MT, U, D, SPW, 0, true, true>), dim3(c.grid), block,
                           lds, stream, (const f16*)x, w, scales, zeros, perm, (f16*)y, N, K, gs,
                           gg, xf);
      return hipGetLastError();
    } else {
      return hipErrorInvalidValue;
    }
  }
  if (xf.mode == 2 || xf.mode == 3 || xf.mode == 5) {
    // the transformed activations are built for u8 zero points and no permutation only
    if (!zero_u8 || perm) return hipErrorInvalidValue;
    if (xf.mode == 2) PMI_GEMV_LAUNCH(2, true);
    else if (xf.mode == 3) PMI_GEMV_LAUNCH(3, true);
    else PMI_GEMV_LAUNCH(5, true);
  } else if (xf.mode == 6) {
    // bf16 activations: plain rows (act_order is gathered by the caller first)
    if (perm) return hipErrorInvalidValue;
    if (zero_u8) PMI_GEMV_LAUNCH(6, true);
    else PMI_GEMV_LAUNCH(6, false);
  } else if (perm_lds && xf.mode == 8) {
    if (zero_u8) PMI_GEMV_LAUNCH(8, true);
    else PMI_GEMV_LAUNCH(8, false);
  } else if (perm_lds) {
    if (zero_u8) PMI_GEMV_LAUNCH(4, true);
    else PMI_GEMV_LAUNCH(4, false);
  } else if (perm) {
    if (zero_u8) PMI_GEMV_LAUNCH(1, true);
    else PMI_GEMV_LAUNCH(1, false);
  } else if (x_lds) {
    if (zero_u8) PMI_GEMV_LAUNCH(7, true);
    else PMI_GEMV_LAUNCH(7, false);
  } else {
    if (zero_u8) PMI_GEMV_LAUNCH(0, true);
    else PMI_GEMV_LAUNCH(0, false);
  }
#undef PMI_GEMV_LAUNCH
  return hipGetLastError();
}

// The (U, D) pairs instantiated: one activation row keeps one, two or four
// rows per batch (a three-deep ring with one or two); more activation rows
// keep a two-deep ring with one, two or (one slice per lane) four rows, and
// only one row when a lane holds more than four activation-row slices, which
// bounds the registers per lane. Every U but the last also comes without a
// ring (D = 1) for launches of one batch per wave.
template <int MT, int SPW>
hipError_t launch_ud(const GemvConfig& c, const void* x, const uint8_t* w, const float* scales,
                     const void* zeros, int zero_u8, const int32_t* perm, void* y, int N, int K,
                     int gs, const GemvXform& xf, hipStream_t stream) {
#define PMI_GEMV_UD(U_, D_) \
  if (c.rows_per_wave == U_ && c.depth == D_) \
    return launch_cfg<MT, U_, D_, SPW>(c, x, w, scales, zeros, zero_u8, perm, y, N, K, gs, xf, \
                                       stream)
  if constexpr (MT == 1) {
    PMI_GEMV_UD(4, 2);
    PMI_GEMV_UD(2, 3);
    PMI_GEMV_UD(1, 3);
    PMI_GEMV_UD(4, 1);
    PMI_GEMV_UD(2, 1);
    PMI_GEMV_UD(1, 1);
  } else if constexpr (MT * SPW > 4) {
    PMI_GEMV_UD(1, 2);
  } else {
    if constexpr (SPW == 1) {
      PMI_GEMV_UD(4, 2);
      PMI_GEMV_UD(4, 1);
    }
    PMI_GEMV_UD(2, 2);
    PMI_GEMV_UD(1, 2);
    PMI_GEMV_UD(2, 1);
    PMI_GEMV_UD(1, 1);
  }
#undef PMI_GEMV_UD
  return hipErrorInvalidValue;  // gemv_config only yields the pairs above
}

template <int MT>
hipError_t launch_mt(const GemvConfig& c, const void* x, const uint8_t* w, const float* scales,
                     const void* zeros, int zero_u8, const int32_t* perm, void* y, int N, int K,
                     int gs, const GemvXform& xf, hipStream_t stream) {
  if (c.slices_per_wave == 2)
    return launch_ud<MT, 2>(c, x, w, scales, zeros, zero_u8, perm, y, N, K, gs, xf, stream);
  return launch_ud<MT, 1>(c, x, w, scales, zeros, zero_u8, perm, y, N, K, gs, xf, stream);
}


constexpr int kMaxPartBytes = 32 * 1024;  // LDS for the per-row partials

}  // namespace

GemvConfig gemv_config(int64_t M, int64_t N, int64_t K, int xmode) {
  GemvConfig c;
  const int mt = (int)(M < 4 ? M : 4);
  const int64_t row_chunks = K / 32;
  c.n_slices = (int)((row_chunks + kSliceChunks - 1) / kSliceChunks);
  // At most 8 waves per workgroup; more than 8 slices -> two slices per wave.
  c.slices_per_wave = c.n_slices > kMaxWaves ? 2 : 1;
  c.slice_waves = (c.n_slices + c.slices_per_wave - 1) / c.slices_per_wave;
  c.row_waves = kMaxWaves / c.slice_waves;
  // Rows per batch (U) and workgroups per CU, from sweeps of every built
  // variant on MI355X at M = 1 with non-temporal weight loads (graph-timed,
  // 8-64 weight copies beyond the MALL, three sweeps). Rows longer than 16384
  // columns (two slices per wave, e.g. K = 18944): single rows at two per CU
  // (10.2 us against 11.4-11.7 for four rows at one). Long rows (three or more
  // slice waves, e.g. K = 14336): four rows, one workgroup per CU (8.0 us).
  // Otherwise by rows per CU: >= 48 (N = 14336 and 28672) pairs at one per CU
  // (7.9 and 12.7-13.0 us; three per CU gave 13.8-14.3 us at N = 28672);
  // plain activations (with the host-side quotients and, where it applies, the
  // activation staging of mode 7) instead take four-row batches at >= 96
  // (N = 28672: median 12.11-12.30 against 12.32-12.36 us, three A/B rounds)
  // and single rows at two per CU below (N = 14336: 7.51-7.55 against
  // 7.62-7.68 us),
  // >= 20 (N = 6144) pairs at three per CU (5.0 us against 5.3-5.5 for single
  // rows at two). Fewer rows (q/o, k/v): one batch per wave, of the most rows
  // that still give every CU a workgroup (N = 4096: four rows, 4.25 us;
  // N = 1024: one row, 3.1 us).
  // Tuning overrides (benchmark sweeps only), restricted to what is built.
  static const int env_u = env_int("PMI_GEMV_U", 0);
  static const int env_wr = env_int("PMI_GEMV_ROW_WAVES", 0);
  static const int env_wpc = env_int("PMI_GEMV_WG_PER_CU", 0);
  static const int env_spw = env_int("PMI_GEMV_SPW", 0);
  if (env_spw == 2 && c.n_slices > 1 && c.slices_per_wave == 1) {
    c.slices_per_wave = 2;
    c.slice_waves = (c.n_slices + 1) / 2;
    c.row_waves = kMaxWaves / c.slice_waves;
  }
  if (env_wr > 0 && env_wr * c.slice_waves <= kMaxWaves) c.row_waves = env_wr;
  const int lanes_x = mt * c.slices_per_wave;  // activation-row slices per lane
  const int max_u = lanes_x > 4 ? 1 : (c.slices_per_wave == 1 || lanes_x <= 2 ? 4 : 2);
  int wpc = 2;
  const int64_t cus = device_cus();
  const int64_t rows_per_cu = N / cus;
  bool one_batch = false;
  // act_order gather (mode 4) on such rows: one per CU, since every workgroup
  // reads the activations (2K bytes) and the permutation (4K) from L2 once
  // (Qwen down 3584 x 18944: 13.8 against 18.1 us at two per CU); with the
  // 16-bit permutation (mode 8, 2K bytes) two per CU up to K = 20480 (3584 x
  // 18944: 11.58-11.68 against 11.70-11.72 us; 4096 x 18944: 12.30-12.34
  // against 12.78-12.81), one beyond (3584 x 32768: 15.0 against 15.3-15.4)
  if (mt == 1 && c.slices_per_wave == 2) {
    c.rows_per_wave = 1;
    wpc = xmode == 4 || (xmode == 8 && K > 20480) ? 1 : 2;
  }
  else if (mt == 1 && c.slice_waves >= 3) { c.rows_per_wave = 4; wpc = 1; }
  else if (mt == 1 && rows_per_cu >= 96 && xmode == 0) { c.rows_per_wave = 4; wpc = 1; }
  else if (mt == 1 && rows_per_cu >= 48 && xmode == 0) { c.rows_per_wave = 1; wpc = 2; }
  else if (mt == 1 && rows_per_cu >= 48) { c.rows_per_wave = 2; wpc = 1; }
  // with the RMSNorm prologue (mode 3) every workgroup first reduces the whole
  // row: single rows at two per CU (fused q/k/v in the decoder: 8.0 against
  // 9.1 us for pairs at three)
  else if (mt == 1 && rows_per_cu >= 20 && xmode == 3) { c.rows_per_wave = 1; wpc = 2; }
  // act_order staged in LDS (mode 4) reads X and the int32 permutation once per
  // workgroup: one per CU (6144 x 4096: 6.7 against 9.4 us at three); so does
  // the norm from partials (mode 5), whose prologue then overlaps a three-deep
  // ring instead of a wave's only batch (6.2 against 7.3 us)
  else if (mt == 1 && rows_per_cu >= 20) {
    c.rows_per_wave = 2;
    wpc = xmode == 4 || xmode == 8 || xmode == 5 ? 1 : 3;
  }
  else if (mt > 1 && rows_per_cu >= 48) { c.rows_per_wave = 2; wpc = 2; }
  else one_batch = true;
  if (one_batch || c.rows_per_wave > max_u) {
    c.rows_per_wave = max_u;
    while (c.rows_per_wave > 1 &&
           N < (int64_t)c.row_waves * c.rows_per_wave * cus * 7 / 8)
      c.rows_per_wave /= 2;
  }
  if ((env_u == 1 || env_u == 2 || env_u == 4) && env_u <= max_u) c.rows_per_wave = env_u;
  if (env_wpc > 0) wpc = env_wpc;
  c.depth = (mt == 1 && c.rows_per_wave != 4) ? 3 : 2;
  const int64_t target = cus * wpc;
  const int64_t stride = (int64_t)c.row_waves * c.rows_per_wave;
  int64_t rows = (N + target - 1) / target;
  if (rows < stride) rows = stride;  // every wave of a workgroup gets rows
  if (c.slice_waves > 1) {
    const int64_t per_row = (int64_t)c.slice_waves * mt * 4;
    const int64_t cap = kMaxPartBytes / per_row / stride * stride;
    if (rows > cap) rows = cap;
  }
  c.rows_per_wg = (int)rows;
  c.grid = (int)((N + rows - 1) / rows);
  if (rows <= stride && lanes_x <= 4) c.depth = 1;  // one batch per wave: no ring
  c.lds_bytes = c.slice_waves > 1 ? (int)(rows * c.slice_waves * mt * 4) : 0;
  return c;
}

bool gemv_perm_lds_ok(int64_t M, int64_t N, int64_t K) {
  const int64_t full = M < 4 ? M : 4, rem = M > 4 ? M % 4 : 0;
  for (const int64_t mt : {full, rem}) {
    if (mt == 0) continue;
    const GemvConfig c = gemv_config(mt, N, K);
    if (!gemv_perm_lds_fits(mt, K, 64 * c.slice_waves * c.row_waves)) return false;
  }
  return true;
}

hipError_t launch_gemv(const void* x, const uint8_t* w, const float* scales, const void* zeros,
                       int zero_u8, const int32_t* perm, void* y, int64_t M, int64_t N,
                       int64_t K, int64_t gs, hipStream_t stream, const GemvXform* xform) {
  const GemvXform xf = xform ? *xform : GemvXform{};
  // bf16 activations (mode 6) take the plain tuning
  const int tune_mode =
      xf.mode == 6 ? 0 : (perm || (xf.mode != 4 && xf.mode != 8) ? xf.mode : 0);
  const GemvConfig c = gemv_config(M, N, K, tune_mode);
  const int n = (int)N, k = (int)K, g = (int)gs;
  switch (M) {
    case 1: return launch_mt<1>(c, x, w, scales, zeros, zero_u8, perm, y, n, k, g, xf, stream);
    case 2: return launch_mt<2>(c, x, w, scales, zeros, zero_u8, perm, y, n, k, g, xf, stream);
    case 3: return launch_mt<3>(c, x, w, scales, zeros, zero_u8, perm, y, n, k, g, xf, stream);
    case 4: return launch_mt<4>(c, x, w, scales, zeros, zero_u8, perm, y, n, k, g, xf, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace pmi
