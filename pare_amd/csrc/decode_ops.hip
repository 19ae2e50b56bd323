// Caller-side fp16 ops of the end-to-end decoder (the model around the INT4
// linears): residual add + RMSNorm, RoPE + KV-cache write, grouped-query
// decode attention, SiLU-gate multiply. One launch each, so a decoder layer is
// about ten launches (four of them INT4 linears) instead of ~50 PyTorch
// elementwise kernels. fp32 arithmetic inside, fp16 in and out.
//
// None of these has a counterpart in the reference's W4A16 path: the
// reference runs the model around QuantizedLinear with HuggingFace PyTorch
// ops (pare/eval/throughput.py:84-126 times HF generate).
#include "pmi_common.h"
#include "pmi_launch.h"

namespace pmi {
namespace {

PMI_DEV float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// h = x (+ r); r_out = h (when r is given); y = h * rsqrt(mean(h^2) + eps) * w.
// One workgroup of 256 threads per row; dim % 8 == 0, dim <= 8192.
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const f16* __restrict__ x,
                                                          const f16* __restrict__ r,
                                                          const f16* __restrict__ w,
                                                          f16* __restrict__ y,
                                                          f16* __restrict__ r_out, int dim,
                                                          float eps) {
  __shared__ float part[4];
  const int row = blockIdx.x, t = threadIdx.x;
  const f16* xr = x + (size_t)row * dim;
  const f16* rr = r ? r + (size_t)row * dim : nullptr;
  constexpr int kPer = 32;  // up to 8192 / 256 values per thread
  float h[kPer];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < kPer / 8; ++i) {
    const int c = (i * 256 + t) * 8;
    if (c < dim) {
      const f16x8 xv = *reinterpret_cast<const f16x8*>(xr + c);
      f16x8 hv = xv;
      if (rr) {
        const f16x8 rv = *reinterpret_cast<const f16x8*>(rr + c);
#pragma unroll
        for (int e = 0; e < 8; ++e) hv[e] = (f16)((float)xv[e] + (float)rv[e]);
        *reinterpret_cast<f16x8*>(r_out + (size_t)row * dim + c) = hv;
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        h[i * 8 + e] = (float)hv[e];
        ss += h[i * 8 + e] * h[i * 8 + e];
      }
    }
  }
  ss = wave_sum(ss);
  if ((t & 63) == 0) part[t >> 6] = ss;
  __syncthreads();
  const float inv = rsqrtf((part[0] + part[1] + part[2] + part[3]) / (float)dim + eps);
#pragma unroll
  for (int i = 0; i < kPer / 8; ++i) {
    const int c = (i * 256 + t) * 8;
    if (c < dim) {
      const f16x8 wv = *reinterpret_cast<const f16x8*>(w + c);
      f16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (f16)(h[i * 8 + e] * inv * (float)wv[e]);
      *reinterpret_cast<f16x8*>(y + (size_t)row * dim + c) = o;
    }
  }
}

// qkv: [B*T, (H + 2*KV) * D] (fused q/k/v output); token bt = b*T + t sits at
// cache position pos[t]. Writes q_out [B, H, T, D] rotated, and the rotated k
// and the v of every token into cache_k / cache_v [B, KV, L, D]. Rotation on
// the two halves of D (rotate_half), cos/sin fp32 [L, D/2] indexed by position.
// One thread per (token, head, pair i < D/2) over all H + KV heads.
__global__ void rope_kv_kernel(const f16* __restrict__ qkv, const float* __restrict__ cos_t,
                               const float* __restrict__ sin_t, const int64_t* __restrict__ pos,
                               f16* __restrict__ q_out, f16* __restrict__ cache_k,
                               f16* __restrict__ cache_v, int B, int T, int H, int KV, int D,
                               int L) {
  const int half = D / 2;
  const int64_t n = (int64_t)B * T * (H + KV) * half;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int d = (int)(i % half);
  const int hh = (int)((i / half) % (H + KV));
  const int bt = (int)(i / ((int64_t)half * (H + KV)));
  const int b = bt / T, t = bt - (bt / T) * T;
  int64_t p = pos[t];
  p = p < 0 ? 0 : (p >= L ? L - 1 : p);
  const int row = (H + 2 * KV) * D;
  const f16* src = qkv + (size_t)bt * row + (size_t)hh * D;
  const float x1 = (float)src[d], x2 = (float)src[d + half];
  const float c = cos_t[p * half + d], s = sin_t[p * half + d];
  const f16 o1 = (f16)(x1 * c - x2 * s), o2 = (f16)(x2 * c + x1 * s);
  if (hh < H) {
    f16* dst = q_out + (((size_t)b * H + hh) * T + t) * D;
    dst[d] = o1;
    dst[d + half] = o2;
  } else {
    const int kh = hh - H;
    f16* dk = cache_k + (((size_t)b * KV + kh) * L + p) * D;
    dk[d] = o1;
    dk[d + half] = o2;
    const f16* sv = qkv + (size_t)bt * row + (size_t)(H + KV + kh) * D;
    f16* dv = cache_v + (((size_t)b * KV + kh) * L + p) * D;
    dv[d] = sv[d];
    dv[d + half] = sv[d + half];
  }
}

// Decode attention, one query token per sequence: out[b, h, :] = softmax(q k^T
// * scale over cache positions 0..*pos) v, query head h reading KV head
// h / (H / KV). One workgroup per (b, KV head); wave (g, c) takes query head
// g of the group and quarter c of the positions (kQuarters waves per head).
// Scores: lane-parallel over positions, each lane a full 128-dim dot product
// (q held in registers as fp16 pairs, v_dot2_f32_f16), stored in LDS. Then
// exp and sum in fp32, and P V with lanes split over positions and 8-dim
// chunks of V. The quarters are combined through LDS with the usual max/sum
// rescaling.
constexpr int kHeadDim = 128;
constexpr int kQuarters = 4;

__global__ __launch_bounds__(1024) void decode_attention_kernel(
    const f16* __restrict__ q, const f16* __restrict__ cache_k, const f16* __restrict__ cache_v,
    const int64_t* __restrict__ pos, f16* __restrict__ out, int H, int KV, int L, float scale) {
  constexpr int D = kHeadDim;
  extern __shared__ float smem[];  // scores [group * kQuarters][span], then partials
  const int b = blockIdx.x / KV, kh = blockIdx.x - (blockIdx.x / KV) * KV;
  const int group = H / KV;
  const int wv = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int g = wv / kQuarters, c = wv - (wv / kQuarters) * kQuarters;
  const int64_t p = *pos;
  const int len = (int)(p < 0 ? 1 : (p >= L ? L : p + 1));
  const int span = (L + kQuarters - 1) / kQuarters;
  const int j0 = c * ((len + kQuarters - 1) / kQuarters);
  const int j1 = min(len, j0 + (len + kQuarters - 1) / kQuarters);
  const int h = kh * group + g;
  const f16* kb = cache_k + ((size_t)b * KV + kh) * L * D;
  const f16* vb = cache_v + ((size_t)b * KV + kh) * L * D;
  float* s = smem + wv * span;
  float* partial = smem + group * kQuarters * span;  // [wave][2 + D]

  // q, pre-scaled, as 64 fp16 pairs in every lane
  uint32_t qp[D / 2];
  {
    const u32x4* q4 = reinterpret_cast<const u32x4*>(q + ((size_t)b * H + h) * D);
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
      const u32x4 v = q4[i];
      qp[4 * i] = v.x; qp[4 * i + 1] = v.y; qp[4 * i + 2] = v.z; qp[4 * i + 3] = v.w;
    }
  }
  float mx = -INFINITY;
  for (int j = j0 + l; j < j1; j += 64) {
    const u32x4* k4 = reinterpret_cast<const u32x4*>(kb + (size_t)j * D);
    float d = 0.f;
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
      const u32x4 kv = k4[i];
      d = dot2_acc(as_f16x2(kv.x), qp[4 * i], d);
      d = dot2_acc(as_f16x2(kv.y), qp[4 * i + 1], d);
      d = dot2_acc(as_f16x2(kv.z), qp[4 * i + 2], d);
      d = dot2_acc(as_f16x2(kv.w), qp[4 * i + 3], d);
    }
    d *= scale;
    s[j - j0] = d;
    mx = fmaxf(mx, d);
  }
  mx = wave_max(mx);
  float sum = 0.f;
  for (int j = j0 + l; j < j1; j += 64) {
    const float e = mx == -INFINITY ? 0.f : __expf(s[j - j0] - mx);
    s[j - j0] = e;
    sum += e;
  }
  sum = wave_sum(sum);
  // P V: lane (ps = l / 16, dc = l % 16) accumulates output dims 8dc..8dc+7
  // over positions j = ps (mod 4), 16 positions per round and two rounds of
  // 16-byte loads in flight; the four position groups are then added with
  // cross-lane shuffles.
  const int ps = l >> 4, dc = l & 15;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  for (int jb = j0; jb < j1; jb += 32) {
    u32x4 vv[8];
    float pp[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int j = jb + 4 * k + ps;
      const bool ok = j < j1;
      const int jj = ok ? j : j0;
      vv[k] = *reinterpret_cast<const u32x4*>(vb + (size_t)jj * D + 8 * dc);
      pp[k] = ok ? s[jj - j0] : 0.f;
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const f16x8 h8 = __builtin_bit_cast(f16x8, vv[k]);
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[e] = fmaf(pp[k], (float)h8[e], acc[e]);
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    acc[e] += __shfl_xor(acc[e], 16);
    acc[e] += __shfl_xor(acc[e], 32);
  }
  float* mine = partial + wv * (2 + D);
  if (l == 0) {
    mine[0] = mx;
    mine[1] = sum;
  }
  if (l < 16) {
#pragma unroll
    for (int e = 0; e < 8; ++e) mine[2 + 8 * dc + e] = acc[e];
  }
  __syncthreads();
  if (c != 0) return;
  float m = -INFINITY;
#pragma unroll
  for (int qq = 0; qq < kQuarters; ++qq) m = fmaxf(m, partial[(wv + qq) * (2 + D)]);
  float tot = 0.f, o0 = 0.f, o1 = 0.f;
#pragma unroll
  for (int qq = 0; qq < kQuarters; ++qq) {
    const float* pq = partial + (wv + qq) * (2 + D);
    const float f = pq[0] == -INFINITY ? 0.f : __expf(pq[0] - m);
    tot = fmaf(pq[1], f, tot);
    o0 = fmaf(pq[2 + 2 * l], f, o0);
    o1 = fmaf(pq[3 + 2 * l], f, o1);
  }
  const float inv = 1.f / tot;
  f16x2 o;
  o[0] = (f16)(o0 * inv);
  o[1] = (f16)(o1 * inv);
  *reinterpret_cast<f16x2*>(out + ((size_t)b * H + h) * D + 2 * l) = o;
}

// Decode attention split over the cache positions (flash-decoding), for
// batches too small to fill the chip with one workgroup per (b, KV head).
// Workgroup (split s, b * KV + kh) takes positions 64 s .. 64 s + 63, one
// wave per query head of the group and one lane per position for the
// scores; the split's K and V rows are staged in LDS once for all its waves
// (coalesced buffer -> LDS copies issued first thing). It writes the split's
// partial (max m, sum l, unnormalised P V) to
// the workspace; the last workgroup of a (b, kh) to arrive, counted with an
// agent-scope atomic, combines the splits in order (deterministic) and
// resets the counter. Partials are stored and loaded with the device-scope
// cache policy (sc1), coherent across the XCDs' L2 caches.
constexpr int kSplitPos = 64;                   // cache positions per workgroup
constexpr int kPartFloats = kHeadDim + 4;       // acc[128], m, l, 2 pad (528 bytes)
constexpr int kSc1 = 16;

// ROPE: q is the fused q/k/v row [B, (H + 2 KV) D] of the new token instead
// of rotated q [B, H, D]. The kernel then does rope_kv_kernel's work itself:
// every wave rotates its head's q into LDS, and the workgroup whose split holds
// the new token's cache row rotates its k and writes k and v to the caches,
// using them from LDS for that row (the same fp16 roundings as rope_kv_kernel,
// so the result equals rope_kv + attention bit for bit).
template <bool ROPE>
__global__ __launch_bounds__(256) void decode_attention_split_kernel(
    const f16* __restrict__ q, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
    f16* __restrict__ cache_k, f16* __restrict__ cache_v, const int64_t* __restrict__ pos,
    f16* __restrict__ out, int H, int KV, int L, int S, float scale, int* __restrict__ counters,
    float* __restrict__ part) {
  constexpr int D = kHeadDim;
  __shared__ int last_flag;
  __shared__ __attribute__((aligned(16))) f16 qrot[ROPE ? 4 : 1][D];
  __shared__ __attribute__((aligned(16))) f16 kvnew[ROPE ? 2 : 1][D];
  // the split's K and V rows (64 x 256 bytes each); 16-byte chunk c of row r
  // sits in slot c ^ (r % 16) of the row, so that the 16 lanes reading chunk c
  // of 16 different rows, and the 16 lanes reading 16 chunks of one row, hit
  // 16 different bank groups
  __shared__ __attribute__((aligned(16))) uint8_t kvs[2][kSplitPos * D * 2];
  const int sidx = blockIdx.x, bk = blockIdx.y;
  const int b = bk / KV, kh = bk - (bk / KV) * KV;
  const int group = H / KV;
  const int g = threadIdx.x >> 6, l = threadIdx.x & 63;
  const int h = kh * group + g;
  const int64_t p = *pos;
  const int len = (int)(p < 0 ? 1 : (p >= L ? L : p + 1));
  const int j0 = sidx * kSplitPos;
  const int j1 = min(len, j0 + kSplitPos);  // j1 <= j0: an empty split
  const f16* kb = cache_k + ((size_t)b * KV + kh) * L * D;
  const f16* vb = cache_v + ((size_t)b * KV + kh) * L * D;
  const int64_t part_bytes = (int64_t)gridDim.y * group * S * kPartFloats * 4;
  const __amdgpu_buffer_rsrc_t rp = rsrc(part, part_bytes);
  // byte offset of this split's record (wave-uniform)
  const int rec = __builtin_amdgcn_readfirstlane(((b * H + h) * S + sidx) * kPartFloats * 4);
  const int pc = (int)(p < 0 ? 0 : (p >= L ? L - 1 : p));  // the new token's cache row

  // Stage the split's K and V rows once for all query-head waves, straight
  // into LDS, before anything waits: 16 copies of 1 KiB (4 rows) per tensor,
  // dealt to the waves; rows past the cache are clamped into it (read, never
  // used). Every lane then reads its rows from LDS: loaded by each lane from
  // L2 (a 256-byte row per lane, the same rows in every wave) the score loads
  // touched 64 lines per instruction.
  {
    const __amdgpu_buffer_rsrc_t rk = rsrc(kb, (int64_t)L * D * 2);
    const __amdgpu_buffer_rsrc_t rv = rsrc(vb, (int64_t)L * D * 2);
    const int nwv = (int)(blockDim.x >> 6);
    for (int c = g; c < kSplitPos / 4; c += nwv) {
      const int r = 4 * c + (l >> 4);
      const int jr = min(j0 + r, L - 1);
      const int voff = jr * (D * 2) + 16 * ((l & 15) ^ (r & 15));
      copy_to_lds<16>(rk, kvs[0] + c * 1024, voff, 0);
      copy_to_lds<16>(rv, kvs[1] + c * 1024, voff, 0);
    }
  }

  if constexpr (ROPE) {
    if (j1 > j0) {
      const f16* src = q + (size_t)b * (H + 2 * KV) * D;
      const int d = l;  // rotation pair (d, d + D/2)
      const float c = cos_t[(size_t)pc * (D / 2) + d], sn = sin_t[(size_t)pc * (D / 2) + d];
      {
        const float x1 = (float)src[h * D + d], x2 = (float)src[h * D + d + D / 2];
        qrot[g][d] = (f16)(x1 * c - x2 * sn);
        qrot[g][d + D / 2] = (f16)(x2 * c + x1 * sn);
      }
      if (g == 0 && pc >= j0 && pc < j1) {
        const float x1 = (float)src[(H + kh) * D + d], x2 = (float)src[(H + kh) * D + d + D / 2];
        const f16 o1 = (f16)(x1 * c - x2 * sn), o2 = (f16)(x2 * c + x1 * sn);
        const f16 v1 = src[(H + KV + kh) * D + d], v2 = src[(H + KV + kh) * D + d + D / 2];
        kvnew[0][d] = o1;
        kvnew[0][d + D / 2] = o2;
        kvnew[1][d] = v1;
        kvnew[1][d + D / 2] = v2;
        const size_t crow = (((size_t)b * KV + kh) * L + pc) * D;
        cache_k[crow + d] = o1;
        cache_k[crow + d + D / 2] = o2;
        cache_v[crow + d] = v1;
        cache_v[crow + d + D / 2] = v2;
      }
    }
  }
  // the staged rows (counted as pending LDS stores by the fence) and the
  // rotated q / new row are in LDS
  __syncthreads();

  float m = -INFINITY, lsum = 0.f;
  float acc[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = 0.f;
  const int ps = l >> 4, dc = l & 15;
  if (j1 > j0) {
    uint32_t qp[D / 2];
    const u32x4* q4 = ROPE ? reinterpret_cast<const u32x4*>(&qrot[ROPE ? g : 0][0])
                           : reinterpret_cast<const u32x4*>(q + ((size_t)b * H + h) * D);
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
      const u32x4 v = q4[i];
      qp[4 * i] = v.x; qp[4 * i + 1] = v.y; qp[4 * i + 2] = v.z; qp[4 * i + 3] = v.w;
    }
    const int j = j0 + l;
    const bool live = j < j1;
    float sc = -INFINITY;
    if (live) {
      // row l of the split, or the new token's k (LDS under ROPE)
      const bool fresh = ROPE && j == pc;
      const uint8_t* krow = fresh ? reinterpret_cast<const uint8_t*>(&kvnew[0][0]) : kvs[0] + l * (D * 2);
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < D / 8; ++i) {
        const u32x4 kv = *reinterpret_cast<const u32x4*>(krow + 16 * (fresh ? i : (i ^ (l & 15))));
        d = dot2_acc(as_f16x2(kv.x), qp[4 * i], d);
        d = dot2_acc(as_f16x2(kv.y), qp[4 * i + 1], d);
        d = dot2_acc(as_f16x2(kv.z), qp[4 * i + 2], d);
        d = dot2_acc(as_f16x2(kv.w), qp[4 * i + 3], d);
      }
      sc = d * scale;
    }
    m = wave_max(sc);
    const float e = live ? __expf(sc - m) : 0.f;
    lsum = wave_sum(e);
    // P V: lane (ps, dc) takes dims 8 dc .. 8 dc + 7 of positions j0 + 4 k + ps
    // (positions past j1 read row 0 of the split, weighted 0)
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int jv = j0 + 4 * k + ps;
      const int r = jv < j1 ? 4 * k + ps : 0;
      const bool fresh = ROPE && j0 + r == pc;
      const u32x4 vv = *reinterpret_cast<const u32x4*>(
          fresh ? reinterpret_cast<const uint8_t*>(&kvnew[ROPE ? 1 : 0][0]) + 16 * dc
                : kvs[1] + r * (D * 2) + 16 * (dc ^ (r & 15)));
      const float pk = __shfl(e, 4 * k + ps);  // 0 for positions past j1
      const f16x8 h8 = __builtin_bit_cast(f16x8, vv);
#pragma unroll
      for (int x = 0; x < 8; ++x) acc[x] = fmaf(pk, (float)h8[x], acc[x]);
    }
#pragma unroll
    for (int x = 0; x < 8; ++x) {
      acc[x] += __shfl_xor(acc[x], 16);
      acc[x] += __shfl_xor(acc[x], 32);
    }
  }
  if (l < 16) {
    const f32x4 a0 = {acc[0], acc[1], acc[2], acc[3]}, a1 = {acc[4], acc[5], acc[6], acc[7]};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, a0), rp, 32 * dc, rec, kSc1);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, a1), rp, 32 * dc + 16, rec,
                                           kSc1);
  } else if (l == 16) {
    const f32x4 ml = {m, lsum, 0.f, 0.f};
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, ml), rp, 4 * D, rec, kSc1);
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(&counters[bk], 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    last_flag = old == S - 1;
  }
  __syncthreads();
  if (!last_flag) return;

  // Last to arrive: combine the S splits of head h in split order, with the
  // running max rescaling, sixteen splits per round of loads (each lane reads
  // the splits' (m, l) and its dims 2l and 2l + 1): one round trip up to 1024
  // cache positions.
  const int rec0 = __builtin_amdgcn_readfirstlane((b * H + h) * S * kPartFloats * 4);
  float mx = -INFINITY, tot = 0.f, o0 = 0.f, o1 = 0.f;
  for (int s0 = 0; s0 < S; s0 += 16) {
    float ms[16], ls[16], a0[16], a1[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int sk = min(s0 + k, S - 1);  // past the end: skipped below
      const int off = __builtin_amdgcn_readfirstlane(rec0 + sk * kPartFloats * 4);
      ms[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, 4 * D, off, kSc1));
      ls[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, 4 * D + 4, off, kSc1));
      a0[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, 8 * l, off, kSc1));
      a1[k] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, 8 * l + 4, off, kSc1));
    }
    // the updates select rather than skip: behind a branch on the loaded max
    // the compiler sank the later splits' loads to their updates, one round
    // trip each
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const bool use = s0 + k < S && ms[k] != -INFINITY;  // uniform across the wave
      const float nm = fmaxf(mx, ms[k]);
      const float fo = mx == -INFINITY ? 0.f : __expf(mx - nm);
      const float fn = __expf(ms[k] - nm);
      const float t = fmaf(tot, fo, ls[k] * fn);
      const float p0 = fmaf(o0, fo, a0[k] * fn);
      const float p1 = fmaf(o1, fo, a1[k] * fn);
      tot = use ? t : tot;
      o0 = use ? p0 : o0;
      o1 = use ? p1 : o1;
      mx = use ? nm : mx;
    }
  }
  const float inv = 1.f / tot;
  f16x2 o;
  o[0] = (f16)(o0 * inv);
  o[1] = (f16)(o1 * inv);
  *reinterpret_cast<f16x2*>(out + ((size_t)b * H + h) * D + 2 * l) = o;
  if (threadIdx.x == 0)
    __hip_atomic_store(&counters[bk], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Greedy token choice: out[r * out_stride] = the index of the largest value of
// x[r, 0:n] (the first one on ties; NaN counts as largest, as torch.argmax
// treats it). Workgroup (chunk c, row r) scans 8192 values with 16-byte loads;
// its (value, index) goes to the workspace with device-scope (sc1) stores and
// the last workgroup of the row, counted with an agent-scope atomic, combines
// the chunks and resets the counter.
constexpr int kArgChunk = 8192;

PMI_DEV bool arg_better(float v, int i, float b, int bi) {
  if (bi < 0) return true;
  if (v != v) return b == b || i < bi;  // NaN beats numbers; the first NaN wins
  if (b != b) return false;
  return v > b || (v == b && i < bi);
}

PMI_DEV void arg_wave_reduce(float& v, int& i) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float ov = __shfl_xor(v, o);
    const int oi = __shfl_xor(i, o);
    if (oi >= 0 && arg_better(ov, oi, v, i)) {
      v = ov;
      i = oi;
    }
  }
}

__global__ __launch_bounds__(256) void argmax_kernel(const f16* __restrict__ x, int n, int chunks,
                                                     int64_t* __restrict__ out, int64_t out_stride,
                                                     int* __restrict__ counters,
                                                     float* __restrict__ part) {
  __shared__ float sv[4];
  __shared__ int si[4];
  __shared__ int last_flag;
  const int c = blockIdx.x, r = blockIdx.y, t = threadIdx.x, l = t & 63, w = t >> 6;
  const f16* row = x + (size_t)r * n;
  const int c0 = c * kArgChunk, c1 = min(n, c0 + kArgChunk);
  float best = 0.f;
  int bi = -1;
#pragma unroll
  for (int k = 0; k < kArgChunk / 2048; ++k) {
    const int i0 = c0 + (k * 256 + t) * 8;
    if (i0 < c1) {  // n % 8 == 0: a chunk of 8 is whole
      const f16x8 v8 = *reinterpret_cast<const f16x8*>(row + i0);
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (arg_better((float)v8[e], i0 + e, best, bi)) {
          best = (float)v8[e];
          bi = i0 + e;
        }
    }
  }
  arg_wave_reduce(best, bi);
  if (l == 0) {
    sv[w] = best;
    si[w] = bi;
  }
  __syncthreads();
  const __amdgpu_buffer_rsrc_t rp = rsrc(part, (int64_t)gridDim.y * chunks * 8);
  if (t == 0) {
    for (int q = 1; q < 4; ++q)
      if (si[q] >= 0 && arg_better(sv[q], si[q], best, bi)) {
        best = sv[q];
        bi = si[q];
      }
    const int off = (r * chunks + c) * 8;
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, best), rp, off, 0, kSc1);
    __builtin_amdgcn_raw_buffer_store_b32((uint32_t)bi, rp, off + 4, 0, kSc1);
    // compiler barriers: the stores stay above the wait and the increment
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0);
    asm volatile("" ::: "memory");
    const int old = __hip_atomic_fetch_add(&counters[r], 1, __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
    last_flag = old == chunks - 1;
  }
  __syncthreads();
  if (!last_flag || w != 0) return;
  // last to arrive: lane q takes chunks q, q + 64, ...
  float v = 0.f;
  int vi = -1;
  for (int q = l; q < chunks; q += 64) {
    const int off = (r * chunks + q) * 8;
    const float qv = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rp, off, 0, kSc1));
    const int qi = (int)__builtin_amdgcn_raw_buffer_load_b32(rp, off + 4, 0, kSc1);
    if (qi >= 0 && arg_better(qv, qi, v, vi)) {
      v = qv;
      vi = qi;
    }
  }
  arg_wave_reduce(v, vi);
  if (l == 0) {
    out[(int64_t)r * out_stride] = vi;
    __hip_atomic_store(&counters[r], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// out[r, c] = silu(gu[r, c]) * gu[r, F + c] for c < F.
__global__ void silu_mul_kernel(const f16* __restrict__ gu, f16* __restrict__ out, int rows,
                                int F) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
  if (i >= (int64_t)rows * F) return;
  const int r = (int)(i / F), c = (int)(i - (i / F) * F);
  const f16x8 g = *reinterpret_cast<const f16x8*>(gu + (size_t)r * 2 * F + c);
  const f16x8 u = *reinterpret_cast<const f16x8*>(gu + (size_t)r * 2 * F + F + c);
  f16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gf = (float)g[e];
    const float sg = (float)(f16)(gf * __builtin_amdgcn_rcpf(1.f + __expf(-gf)));
    o[e] = (f16)(sg * (float)u[e]);
  }
  *reinterpret_cast<f16x8*>(out + (size_t)r * F + c) = o;
}

}  // namespace

hipError_t launch_add_rmsnorm(const void* x, const void* r, const void* w, void* y, void* r_out,
                              int64_t rows, int64_t dim, float eps, hipStream_t stream) {
  hipLaunchKernelGGL(add_rmsnorm_kernel, dim3((unsigned)rows), dim3(256), 0, stream, (const f16*)x,
                     (const f16*)r, (const f16*)w, (f16*)y, (f16*)r_out, (int)dim, eps);
  return hipGetLastError();
}

hipError_t launch_rope_kv(const void* qkv, const float* cos_t, const float* sin_t,
                          const int64_t* pos, void* q_out, void* cache_k, void* cache_v,
                          int64_t B, int64_t T, int64_t H, int64_t KV, int64_t D, int64_t L,
                          hipStream_t stream) {
  const int64_t n = B * T * (H + KV) * (D / 2);
  hipLaunchKernelGGL(rope_kv_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     (const f16*)qkv, cos_t, sin_t, pos, (f16*)q_out, (f16*)cache_k,
                     (f16*)cache_v, (int)B, (int)T, (int)H, (int)KV, (int)D, (int)L);
  return hipGetLastError();
}

size_t decode_attention_ws_bytes(int64_t B, int64_t H, int64_t KV, int64_t L) {
  if (B * KV > kOpsMaxCounters) return 0;
  const int64_t S = (L + kSplitPos - 1) / kSplitPos;
  return kOpsCounterBytes + (size_t)(B * H * S * kPartFloats * 4);
}

hipError_t launch_decode_attention(const void* q, const void* cache_k, const void* cache_v,
                                   const int64_t* pos, void* out, int64_t B, int64_t H,
                                   int64_t KV, int64_t L, float scale, void* workspace,
                                   size_t ws_bytes, hipStream_t stream, const float* cos_t,
                                   const float* sin_t) {
  const int group = (int)(H / KV);
  const bool rope = cos_t != nullptr;
  const size_t need = decode_attention_ws_bytes(B, H, KV, L);
  if (workspace && need && ws_bytes >= need) {
    const int S = (int)((L + kSplitPos - 1) / kSplitPos);
    int* counters = (int*)workspace;
    float* part = (float*)((char*)workspace + kOpsCounterBytes);
    const dim3 grid((unsigned)S, (unsigned)(B * KV)), block(64 * group);
    if (rope)
      hipLaunchKernelGGL(decode_attention_split_kernel<true>, grid, block, 0, stream, (const f16*)q,
                         cos_t, sin_t, (f16*)cache_k, (f16*)cache_v, pos, (f16*)out, (int)H,
                         (int)KV, (int)L, S, scale, counters, part);
    else
      hipLaunchKernelGGL(decode_attention_split_kernel<false>, grid, block, 0, stream,
                         (const f16*)q, nullptr, nullptr, (f16*)cache_k, (f16*)cache_v, pos,
                         (f16*)out, (int)H, (int)KV, (int)L, S, scale, counters, part);
    return hipGetLastError();
  }
  if (rope) return hipErrorInvalidValue;  // the fused RoPE needs the split kernel
  const int span = (int)((L + kQuarters - 1) / kQuarters);
  const size_t lds = ((size_t)group * kQuarters * span + (size_t)group * kQuarters * (2 + kHeadDim)) * 4;
  hipLaunchKernelGGL(decode_attention_kernel, dim3((unsigned)(B * KV)),
                     dim3(64 * group * kQuarters), lds, stream, (const f16*)q,
                     (const f16*)cache_k, (const f16*)cache_v, pos, (f16*)out, (int)H, (int)KV,
                     (int)L, scale);
  return hipGetLastError();
}

size_t argmax_ws_bytes(int64_t rows, int64_t n) {
  if (rows > kOpsMaxCounters) return 0;
  const int64_t chunks = (n + kArgChunk - 1) / kArgChunk;
  return kOpsCounterBytes + (size_t)(rows * chunks * 8);
}

hipError_t launch_argmax(const void* x, int64_t rows, int64_t n, int64_t* out, int64_t out_stride,
                         void* workspace, hipStream_t stream) {
  const int chunks = (int)((n + kArgChunk - 1) / kArgChunk);
  int* counters = (int*)workspace;
  float* part = (float*)((char*)workspace + kOpsCounterBytes);
  hipLaunchKernelGGL(argmax_kernel, dim3((unsigned)chunks, (unsigned)rows), dim3(256), 0, stream,
                     (const f16*)x, (int)n, chunks, out, out_stride, counters, part);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const void* gu, void* out, int64_t rows, int64_t F,
                           hipStream_t stream) {
  const int64_t n = rows * F / 8;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                     (const f16*)gu, (f16*)out, (int)rows, (int)F);
  return hipGetLastError();
}

}  // namespace pmi
