// moe_common.hpp — device helpers shared by the gfx950 MoE kernels.
//
// Element types are the storage types of FFAI's DType (f32 / f16 / bf16,
// Sources/FFAI/DType.swift:20-39). Every kernel accumulates in fp32 and rounds
// to the storage type (round-to-nearest-even) where the reference stores a
// tensor in the activation dtype.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "moe_internal.hpp"

namespace moe {

constexpr int kWave = 64;

typedef __bf16 bf16_t;
typedef _Float16 f16_t;
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// ---------------------------------------------------------------- convert --
template <typename T> __device__ __forceinline__ float to_f(T v) { return (float)v; }
template <> __device__ __forceinline__ float to_f<bf16_t>(bf16_t v) {
  return __uint_as_float((uint32_t)__builtin_bit_cast(uint16_t, v) << 16);
}
template <typename T> __device__ __forceinline__ T from_f(float v) { return (T)v; }

template <typename T> __device__ __forceinline__ float round_to(float v) { return to_f<T>(from_f<T>(v)); }

// --------------------------------------------------------- wave reductions --
__device__ __forceinline__ float wave_sum_width(float v, int width) {
  for (int off = width >> 1; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

// DPP lane moves (GFX9 encodings): quad_perm [1,0,3,2] = 0xB1, [2,3,0,1] =
// 0x4E, row_half_mirror = 0x141, row_mirror = 0x140, row_bcast:15 = 0x142,
// row_bcast:31 = 0x143. Rows outside ROW_MASK return `old`.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f32(float old, float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(x), CTRL,
                                                    ROW_MASK, 0xF, false));
}

// Maximum over the wave, returned wave-uniform; as with fmaxf (v_max_f32 in
// IEEE mode), NaN lanes are ignored unless every lane is NaN.
__device__ __forceinline__ float wave_max_f32(float x) {
  x = fmaxf(x, dpp_f32<0xB1, 0xF>(x, x));
  x = fmaxf(x, dpp_f32<0x4E, 0xF>(x, x));
  x = fmaxf(x, dpp_f32<0x141, 0xF>(x, x));
  x = fmaxf(x, dpp_f32<0x140, 0xF>(x, x));
  x = fmaxf(x, dpp_f32<0x142, 0xA>(x, x));
  x = fmaxf(x, dpp_f32<0x143, 0xC>(x, x));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), 63));
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ int dpp_i32(int old, int x) {
  return __builtin_amdgcn_update_dpp(old, x, CTRL, ROW_MASK, 0xF, false);
}

// Maximum over the wave, returned wave-uniform.
__device__ __forceinline__ int wave_max_i32(int x) {
  x = max(x, dpp_i32<0xB1, 0xF>(x, x));
  x = max(x, dpp_i32<0x4E, 0xF>(x, x));
  x = max(x, dpp_i32<0x141, 0xF>(x, x));
  x = max(x, dpp_i32<0x140, 0xF>(x, x));
  x = max(x, dpp_i32<0x142, 0xA>(x, x));
  x = max(x, dpp_i32<0x143, 0xC>(x, x));
  return __builtin_amdgcn_readlane(x, 63);
}

// Lane r's value (r wave-uniform), through a scalar register.
__device__ __forceinline__ float lane_f32(float x, int r) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), r));
}

// Inclusive prefix sum over the wave by DPP: row_shr 1, 2, 4, 8 within each
// row of 16 lanes (lanes without a source add 0), then row 0's total into
// row 1 and row 2's into row 3 (row_bcast:15), then rows 0-1's into rows
// 2-3 (row_bcast:31).
__device__ __forceinline__ uint32_t wave_scan_u32(uint32_t x) {
  int v = (int)x;
  v += dpp_i32<0x111, 0xF>(0, v);
  v += dpp_i32<0x112, 0xF>(0, v);
  v += dpp_i32<0x114, 0xF>(0, v);
  v += dpp_i32<0x118, 0xF>(0, v);
  v += dpp_i32<0x142, 0xA>(0, v);
  v += dpp_i32<0x143, 0xC>(0, v);
  return (uint32_t)v;
}

// Order-preserving map of non-NaN floats onto signed ints (an involution):
// a < b as floats iff key(a) < key(b), with -0 canonicalised to +0 first so
// that the two zeros tie as they do in float comparisons.
__device__ __forceinline__ int f32_key(float f) {
  const int b = __float_as_int(f + 0.0f);
  return b ^ ((b >> 31) & 0x7FFFFFFF);
}
__device__ __forceinline__ float key_f32(int k) { return __int_as_float(k ^ ((k >> 31) & 0x7FFFFFFF)); }

// Sum over each aligned group of 2^lg lanes (lg wave-uniform, 0..6). The
// sum is valid in the group's last lane (lane % 2^lg == 2^lg - 1); groups of
// up to 16 lanes hold it in every lane. The summation tree is fixed, so the
// result is deterministic.
__device__ __forceinline__ float group_sum(float v, int lg) {
  if (lg >= 1) v += dpp_f32<0xB1, 0xF>(0.f, v);
  if (lg >= 2) v += dpp_f32<0x4E, 0xF>(0.f, v);
  if (lg >= 3) v += dpp_f32<0x141, 0xF>(0.f, v);
  if (lg >= 4) v += dpp_f32<0x140, 0xF>(0.f, v);
  if (lg >= 5) v += dpp_f32<0x142, 0xA>(0.f, v);
  if (lg >= 6) v += dpp_f32<0x143, 0xC>(0.f, v);
  return v;
}

// Block barrier ordering LDS only: loads from global memory stay in flight
// across it (a full __syncthreads would wait for them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// ------------------------------------------------------- buffer resources --
// Raw buffer view of [base, base + bytes): loads take a 32-bit lane offset
// against a wave-uniform base held in SGPRs, and a load whose lane offset is
// at or past `bytes` returns zero instead of touching memory.
typedef __amdgpu_buffer_rsrc_t rsrc_t;
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x3_t __attribute__((ext_vector_type(3)));
// AUX: the cache policy of the load. kStream (non-temporal) is for expert
// weights that a call reads once in whole lines per instruction (the one-token
// and few-row GEMVs): they then stop evicting what later launches read again,
// such as the next layers' router rows (GPT-OSS decode 23.9 -> 23.0 us per
// layer, Qwen3 16.0 -> 14.9). Kernels that re-read weights (the grouped GEMM
// across row tiles) or read parts of lines per lane (the matrix-core GEMV)
// measured slower with it.
constexpr int kStream = 2;
template <int AUX = 0>
__device__ __forceinline__ u32x4_t bload128(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ u32x3_t bload96(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b96(r, off, 0, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ u32x2_t bload64(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ uint32_t bload32(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ uint16_t bload16(rsrc_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, AUX);
}
// A store whose lane offset is at or past the view's end is dropped.
__device__ __forceinline__ void bstore128(rsrc_t r, uint32_t off, u32x4_t v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, 0);
}

// Eight bf16 values (16 bytes) -> f16 * 2^-SHIFT, rounded to nearest even:
// the grouped GEMM's A operand of a bf16 layer, converted as its epilogue
// converts the intermediate activation (to_a16 in gemm.hip). Exact for
// magnitudes 2^(SHIFT-14) ... 65504 * 2^SHIFT (f16's normal range after the
// scale); below, f16 subnormals round to nearest (absolute error at most
// 2^(SHIFT-25)); finite values beyond saturate to +-65504 * 2^SHIFT;
// infinities and NaNs pass through.
template <int SHIFT>
__device__ __forceinline__ uint4 bf16x8_to_a16(uint4 v) {
  const uint32_t in[4] = {v.x, v.y, v.z, v.w};
  uint32_t o[4];
  auto cvt = [](float f) -> uint32_t {
    f = __builtin_ldexpf(f, -SHIFT);
    if (__builtin_fabsf(f) > 65504.0f && __builtin_isfinite(f)) f = __builtin_copysignf(65504.0f, f);
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
  };
#pragma unroll
  for (int q = 0; q < 4; q++)
    o[q] = cvt(__uint_as_float(in[q] << 16)) | (cvt(__uint_as_float(in[q] & 0xFFFF0000u)) << 16);
  return make_uint4(o[0], o[1], o[2], o[3]);
}

// ------------------------------------------------------ deterministic exp --
// Cody-Waite reduction by ln2 plus Moshier's degree-5 polynomial (Cephes
// expf), written as explicit fused/unfused fp32 operations so that the CPU
// restatement of the router evaluates the identical bits.
__device__ __forceinline__ float det_expf(float x) {
#pragma clang fp contract(off)
  if (x > 88.0f) return __builtin_huge_valf();
  if (x < -87.0f) return 0.0f;
  float n = __builtin_rintf(x * 1.44269504088896341f);
  float r = __builtin_fmaf(n, -0.693359375f, x);
  r = __builtin_fmaf(n, 2.12194440e-4f, r);
  float p = 1.9875691500e-4f;
  p = __builtin_fmaf(p, r, 1.3981999507e-3f);
  p = __builtin_fmaf(p, r, 8.3334519073e-3f);
  p = __builtin_fmaf(p, r, 4.1665795894e-2f);
  p = __builtin_fmaf(p, r, 1.6666665459e-1f);
  p = __builtin_fmaf(p, r, 5.0000001201e-1f);
  float r2 = r * r;
  float y = __builtin_fmaf(p, r2, r) + 1.0f;
  return __builtin_ldexpf(y, (int)n);
}

// ------------------------------------------------------------ bias words --
// A per-expert bias element's raw bits through a buffer view (no bias: an
// empty view, which reads 0 without touching memory), converted only where
// the bias is added (bias_f). Converting it where it is loaded makes the wave
// wait for it, and for every load issued before it, ahead of the loads that
// follow (vector loads complete in issue order).
template <typename XT>
__device__ __forceinline__ uint32_t bias_raw(const XT* bias, int e) {
  const rsrc_t r = make_rsrc(bias ? bias + e : nullptr, bias ? (uint32_t)sizeof(XT) : 0u);
  if constexpr (sizeof(XT) == 2) return (uint32_t)bload16(r, 0u);
  else return bload32(r, 0u);
}
template <typename XT>
__device__ __forceinline__ float bias_f(uint32_t raw) {
  if constexpr (sizeof(XT) == 2) return to_f<XT>(__builtin_bit_cast(XT, (uint16_t)raw));
  else return __uint_as_float(raw);
}

// ------------------------------------------------------------ wave top-k --
// Makes LDS writes of this wave visible to its other lanes.
__device__ __forceinline__ void wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
}

constexpr int kTopkMaxE = 512;           // experts a wave can route
constexpr int kTopkEPL = kTopkMaxE / 64; // logits held per lane

// MoERouter.route for one token with one full wave (MoELayer.swift:140-205,
// heap order of :223-296). Lane r < k returns the r-th selected expert in
// (value desc, index asc) order in *sel and its combine weight in *w
// (weights only when want_weights). Softmax sums run in index / rank order
// on one lane with det_expf, so the results are reproducible bit for bit.
// sc: this wave's LDS scratch of at least E floats (full-softmax mode).
// masks (nullable): wave-uniform selection bitmaps, bit l of masks[j] set
// iff expert 64 j + l was selected (kTopkEPL entries). EPL: logits per lane,
// a compile-time bound on E (E <= 64 EPL) that removes the per-slot range
// checks from the k selection rounds.
template <typename XT, int EPL = kTopkEPL>
__device__ void wave_topk(const XT* __restrict__ row, int E, int k, const RouteOpts& ro, float* sc,
                          bool want_weights, int* sel, float* w, uint64_t* masks = nullptr) {
  const int lane = threadIdx.x & 63;
  const int gating = ro.gating, norm = ro.norm;
  const float* __restrict__ ebias = ro.ebias;
  const bool sigmoid = gating == 2;
  const bool on_logits = !sigmoid && ((gating == 1) || (norm && ebias == nullptr));
  const float NEG = -__builtin_huge_valf();
  float v[EPL];
  float m = NEG;
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    const int i = lane + 64 * j;
    v[j] = NEG;
    if (j * 64 < E) {  // wave-uniform; the load itself is clamped, not branched
      const float lv = to_f<XT>(row[min(i, E - 1)]) * ro.logit_scale;
      v[j] = (i < E) ? lv : NEG;
      m = (i < E) ? fmaxf(m, lv) : m;
    }
  }
  // sigmoid mode: v becomes the selection score, raw[] the unbiased sigmoid
  float raw[EPL];
  if (sigmoid) {
#pragma unroll
    for (int j = 0; j < EPL; j++) {
      const int i = lane + 64 * j;
      raw[j] = 1.0f / (1.0f + det_expf(-v[j]));
      v[j] = (i < E) ? (ebias ? raw[j] + ebias[min(i, E - 1)] : raw[j]) : NEG;
    }
  }
  if (!on_logits && !sigmoid) {
    // full softmax (+ expert bias): MoELayer.swift:174-195
    m = wave_max_f32(m);
#pragma unroll
    for (int j = 0; j < EPL; j++) {
      const int i = lane + 64 * j;
      if (i < E) {
        v[j] = det_expf(v[j] - m);
        sc[i] = v[j];
      }
    }
    wave_sync();
    float s = 0.f;
    if (lane == 0)
      for (int i = 0; i < E; i++) s += sc[i];
    s = lane_f32(s, 0);
#pragma unroll
    for (int j = 0; j < EPL; j++) {
      const int i = lane + 64 * j;
      if (i < E) {
        v[j] = (s > 0.f) ? v[j] / s : 1.0f / (float)E;
        if (ebias) v[j] = v[j] + ebias[min(i, E - 1)];
      }
    }
    wave_sync();
  }
  // NaN sorts as -inf so the order is total and every lane agrees. k rounds
  // of a wave argmax over integer keys: the largest remaining key by a DPP
  // max, the smallest index holding it by ballots (index = lane + 64 j).
  constexpr int NONE = (int)0x80000000;  // below the key of -inf
  int key[EPL];
#pragma unroll
  for (int j = 0; j < EPL; j++) {
    const bool ok = (j * 64 < E) && (lane + 64 * j < E);
    key[j] = ok ? f32_key(v[j] != v[j] ? NEG : v[j]) : NONE;
  }
  uint32_t taken = 0;
  int my_sel = 0, my_key = NONE;
  float my_raw = NEG;  // the selected logit (sigmoid: unbiased score), lane r < k
  for (int r = 0; r < k; r++) {
    int bk = key[0];
#pragma unroll
    for (int j = 1; j < EPL; j++)
      if (j * 64 < E) bk = max(bk, key[j]);
    const int mk = wave_max_i32(bk);
    int win = 0;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
      if (j * 64 < E) {
        const uint64_t b = __ballot(key[j] == mk);
        if (b) {
          win = j * 64 + __ffsll((unsigned long long)b) - 1;
          break;
        }
      }
    }
    win = __builtin_amdgcn_readfirstlane(win);
    const int wj = win >> 6;
    const bool mine = (win & 63) == lane;
    float rv = sigmoid ? raw[0] : v[0];
#pragma unroll
    for (int j = 1; j < EPL; j++) rv = (j == wj) ? (sigmoid ? raw[j] : v[j]) : rv;
    rv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rv), win & 63));
#pragma unroll
    for (int j = 0; j < EPL; j++) {
      if (j == wj && mine) {
        key[j] = NONE;
        taken |= 1u << j;
      }
    }
    if (lane == r) {
      my_sel = win;
      my_key = mk;
      my_raw = rv;
    }
  }
  const float my_val = key_f32(my_key);
  if (masks) {
#pragma unroll
    for (int j = 0; j < kTopkEPL; j++) masks[j] = (j < EPL && j * 64 < E) ? __ballot((taken >> j) & 1u) : 0ull;
  }
  *sel = my_sel;
  if (!want_weights) return;
  // combine weights; lane 0 accumulates in rank order
  float wv;
  if (on_logits) {
    // softmax over the k picked raw logits — MoELayer.swift:166-172,197-203
    // (the values travelled with the selection: no second read of the row)
    // (the max by DPP and the rank-order sum by readlane: shuffles would put
    // an LDS round trip per step on the routing chain)
    const float lv = (lane < k) ? my_raw : NEG;
    const float mx = wave_max_f32(lv);
    const float ex = (lane < k) ? det_expf(lv - mx) : 0.f;
    float s = 0.f;
    for (int r = 0; r < k; r++) s += lane_f32(ex, r);
    wv = (s > 0.f) ? ex / s : 1.0f / (float)k;
  } else if (sigmoid) {
    // raw sigmoid of the pick, / (sum in rank order + 1e-20) when norm, k > 1
    wv = my_raw;
    if (norm && k > 1) {
      float s = 0.f;
      for (int r = 0; r < k; r++) s += lane_f32(my_raw, r);
      wv = wv / (s + 1e-20f);
    }
  } else {
    wv = my_val;
    if (norm) {
      float s = 0.f;
      for (int r = 0; r < k; r++) s += lane_f32(my_val, r);
      if (s > 0.f) wv = wv / s;
    }
  }
  wv = wv * ro.routed_scale;
  if (ro.escale) wv = wv * ro.escale[min(my_sel, E - 1)];
  *w = wv;
}

// ------------------------------------------------------------ activations --
enum { ACT_SWIGLU = 0, ACT_GPTOSS = 1, ACT_GEGLU = 2, ACT_RELU2 = 3 };

// Tanh-form GELU, 0.5 g (1 + tanh(y)) with y = sqrt(2/pi) (g + 0.044715 g^3),
// evaluated as g * logistic(2y): the same function without the cancellation
// of 1 + tanh(y) for negative g, and finite at both ends (exp overflows to
// inf, the reciprocal to 0).
__device__ __forceinline__ float gelu_tanh(float g) {
  const float y = 0.7978845608f * (g + 0.044715f * g * g * g);
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-2.0f * y));
}

// The gated activation of one expert row, returned in fp32 before the final
// rounding to the storage type XT:
//   SwiGLU silu(g) u (Ops.swift:6400-6411);
//   GPT-OSS min(g, limit) sigma(alpha g) (clamp(u, +-limit) + 1)
//     (GPTOSSText.swift:1415-1431);
//   GEGLU gelu(g) rounded to XT, times u (Gemma4Text.swift:965 stores the
//     GELU before the product);
//   ReLU^2 max(u, 0)^2, no gate projection (NemotronHText.swift:756-761).
// The logistic uses the hardware reciprocal (v_rcp_f32, 1 ulp) in place of an
// IEEE divide: the result is rounded to a 16-bit storage type right after.
template <typename XT>
__device__ __forceinline__ float apply_act(float g, float u, int act, float alpha, float limit) {
  if (act == ACT_GPTOSS) {
    g = fminf(g, limit);
    u = fminf(fmaxf(u, -limit), limit);
    const float glu = g * __builtin_amdgcn_rcpf(1.0f + __expf(-alpha * g));
    return glu * (u + 1.0f);
  }
  if (act == ACT_GEGLU) return round_to<XT>(gelu_tanh(g)) * u;
  if (act == ACT_RELU2) {
    const float r = fmaxf(u, 0.0f);
    return r * r;
  }
  return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
}

// ------------------------------------------------------ affine bit stream --
// A "unit" is 32 consecutive values of one weight row: BITS u32 words of the
// little-endian bit stream (value i at bit offset i*BITS). Units never
// straddle a scale group because group sizes are multiples of 32.
//
// unpack_pairs<BITS> turns a unit into 16 code pairs, each u32 holding two
// codes in its low bits of the 16-bit halves: pair j = (q_a, q_b) with the
// sub-block pairing (i, i + P/2) inside blocks of P values, P = 16 for 2-bit,
// 8 for 3/4-bit and 4 for 5/6/8-bit. Activations are stored in the same
// pair order (pair_pos) so a dot2 multiplies matching values.
template <int BITS> struct Pairing;
template <> struct Pairing<2> { static constexpr int P = 16; };
template <> struct Pairing<3> { static constexpr int P = 8; };
template <> struct Pairing<4> { static constexpr int P = 8; };
template <> struct Pairing<5> { static constexpr int P = 4; };
template <> struct Pairing<6> { static constexpr int P = 4; };
template <> struct Pairing<8> { static constexpr int P = 4; };

// Position of value v (0..31 within a unit) in the pair-ordered layout.
template <int BITS> __host__ __device__ __forceinline__ int pair_pos(int v) {
  constexpr int P = Pairing<BITS>::P, H = P / 2;
  int blk = v / P, i = v % P;
  return blk * P + (i < H ? 2 * i : 2 * (i - H) + 1);
}

// (hi:lo) >> sh for sh in [0, 32), one v_alignbit_b32. (A 64-bit shift here
// let the compiler merge neighbouring words of a unit into 64-bit loads from
// the unit array, which then stayed a memory array instead of registers.)
__device__ __forceinline__ uint32_t funnel(uint32_t hi, uint32_t lo, int sh) {
  return __builtin_amdgcn_alignbit(hi, lo, (uint32_t)sh);
}

// A VGPR copy of c that the compiler cannot fold back into a literal: GFX9
// VOP3 encodings take no literal operand, so `(x & M) | C` only becomes one
// v_and_or_b32 when C already sits in a register.
__device__ __forceinline__ uint32_t opaque_vgpr(uint32_t c) {
  uint32_t r;
  asm("v_mov_b32 %0, %1" : "=v"(r) : "s"(c));
  return r;
}

// MAGIC is or-ed into every pair in the same and-or (see Magic below).
template <int BITS, uint32_t MAGIC_C = 0u>
__device__ __forceinline__ void unpack_pairs(const uint32_t (&w)[BITS], uint32_t (&cp)[16]) {
  const uint32_t MAGIC = MAGIC_C ? opaque_vgpr(MAGIC_C) : 0u;
  if constexpr (BITS == 2) {
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int i = 0; i < 8; i++) cp[j * 8 + i] = ((w[j] >> (2 * i)) & 0x00030003u) | MAGIC;
  } else if constexpr (BITS == 4) {
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
      for (int i = 0; i < 4; i++) cp[j * 4 + i] = ((w[j] >> (4 * i)) & 0x000F000Fu) | MAGIC;
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int j = 0; j < 8; j++)
#pragma unroll
      for (int i = 0; i < 2; i++) cp[j * 2 + i] = ((w[j] >> (8 * i)) & 0x00FF00FFu) | MAGIC;
  } else if constexpr (BITS == 3) {
    // 4 sub-blocks of 24 bits (8 values); spread the upper 12 bits to bit 16
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int bit = 24 * j, lo = bit >> 5, sh = bit & 31;
      uint32_t s = (sh + 24 <= 32) ? (w[lo] >> sh) : funnel(w[lo + 1], w[lo], sh);
      s &= 0xFFFFFFu;
      uint32_t t = (s & 0xFFFu) | ((s & 0xFFF000u) << 4);
#pragma unroll
      for (int i = 0; i < 4; i++) cp[j * 4 + i] = ((t >> (3 * i)) & 0x00070007u) | MAGIC;
    }
  } else if constexpr (BITS == 6) {
    // 8 sub-blocks of 24 bits (4 values)
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int bit = 24 * j, lo = bit >> 5, sh = bit & 31;
      uint32_t s = (sh + 24 <= 32) ? (w[lo] >> sh) : funnel(w[lo + 1], w[lo], sh);
      s &= 0xFFFFFFu;
      uint32_t t = (s & 0xFFFu) | ((s & 0xFFF000u) << 4);
#pragma unroll
      for (int i = 0; i < 2; i++) cp[j * 2 + i] = ((t >> (6 * i)) & 0x003F003Fu) | MAGIC;
    }
  } else if constexpr (BITS == 5) {
    // 8 sub-blocks of 20 bits (4 values); spread the upper 10 bits to bit 16
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int bit = 20 * j, lo = bit >> 5, sh = bit & 31;
      uint32_t s = (sh + 20 <= 32) ? (w[lo] >> sh) : funnel(w[lo + 1], w[lo], sh);
      s &= 0xFFFFFu;
      uint32_t t = (s & 0x3FFu) | ((s & 0xFFC00u) << 6);
#pragma unroll
      for (int i = 0; i < 2; i++) cp[j * 2 + i] = ((t >> (5 * i)) & 0x001F001Fu) | MAGIC;
    }
  }
}

// Loads one unit (BITS consecutive u32) with the widest loads its alignment
// allows (rows start 16-byte aligned: k is a multiple of 32).
template <int BITS>
__device__ __forceinline__ void load_unit(const uint32_t* __restrict__ p, uint32_t (&w)[BITS]) {
  if constexpr (BITS == 2) {
    uint2 v = *reinterpret_cast<const uint2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else if constexpr (BITS == 3) {
    w[0] = p[0]; w[1] = p[1]; w[2] = p[2];
  } else if constexpr (BITS == 4) {
    uint4 v = *reinterpret_cast<const uint4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (BITS == 5) {
    // 20-byte units are only 4-byte aligned
    w[0] = p[0]; w[1] = p[1]; w[2] = p[2]; w[3] = p[3]; w[4] = p[4];
  } else if constexpr (BITS == 6) {
    uint2 a = *reinterpret_cast<const uint2*>(p);
    uint2 b = *reinterpret_cast<const uint2*>(p + 2);
    uint2 c = *reinterpret_cast<const uint2*>(p + 4);
    w[0] = a.x; w[1] = a.y; w[2] = b.x; w[3] = b.y; w[4] = c.x; w[5] = c.y;
  } else {
    uint4 a = *reinterpret_cast<const uint4*>(p);
    uint4 b = *reinterpret_cast<const uint4*>(p + 4);
    w[0] = a.x; w[1] = a.y; w[2] = a.z; w[3] = a.w;
    w[4] = b.x; w[5] = b.y; w[6] = b.z; w[7] = b.w;
  }
}

// Buffer form of load_unit: byte offset `off` of a raw buffer view. Units of
// 3, 5 and 6 bits are 12, 20 and 24 bytes, 4- or 8-byte aligned; buffer
// loads of several dwords need only dword alignment, so each unit takes one
// or two loads (a 96-bit load, or a 128-bit load and the rest) instead of one
// per word.
template <int BITS, int AUX = 0>
__device__ __forceinline__ void bload_unit(rsrc_t r, uint32_t off, uint32_t (&w)[BITS]) {
  if constexpr (BITS == 2) {
    const u32x2_t v = bload64<AUX>(r, off);
    w[0] = v[0]; w[1] = v[1];
  } else if constexpr (BITS == 3) {
    const u32x3_t v = bload96<AUX>(r, off);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2];
  } else if constexpr (BITS == 4) {
    const u32x4_t v = bload128<AUX>(r, off);
    w[0] = v[0]; w[1] = v[1]; w[2] = v[2]; w[3] = v[3];
  } else if constexpr (BITS == 5) {
    const u32x4_t a = bload128<AUX>(r, off);
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
    w[4] = bload32<AUX>(r, off + 16);
  } else if constexpr (BITS == 6) {
    const u32x4_t a = bload128<AUX>(r, off);
    const u32x2_t b = bload64<AUX>(r, off + 16);
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3]; w[4] = b[0]; w[5] = b[1];
  } else if constexpr (BITS == 8) {
    const u32x4_t a = bload128<AUX>(r, off), b = bload128<AUX>(r, off + 16);
    w[0] = a[0]; w[1] = a[1]; w[2] = a[2]; w[3] = a[3];
    w[4] = b[0]; w[5] = b[1]; w[6] = b[2]; w[7] = b[3];
  } else {
    // 16: plain 16-bit weights (dense projections), 32 values = 64 bytes
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const u32x4_t v = bload128<AUX>(r, off + 16u * q);
      w[4 * q] = v[0]; w[4 * q + 1] = v[1]; w[4 * q + 2] = v[2]; w[4 * q + 3] = v[3];
    }
  }
}

// Number of selected experts with an id below e (selection bitmaps from
// wave_topk); e may equal the expert count.
__device__ __forceinline__ int selected_below(const uint64_t (&m)[kTopkEPL], int e) {
  int c = 0;
#pragma unroll
  for (int j = 0; j < kTopkEPL; j++) {
    const int lo = j * 64;
    if (e >= lo + 64) c += __popcll(m[j]);
    else if (e > lo) c += __popcll(m[j] & ((1ull << (e - lo)) - 1ull));
  }
  return c;
}

// The s-th smallest selected expert id (wave-uniform s and bitmaps).
__device__ __forceinline__ int selected_nth(const uint64_t (&m)[kTopkEPL], int s) {
  int e = 0;
  bool found = false;
#pragma unroll
  for (int j = 0; j < kTopkEPL; j++) {
    const int c = __popcll(m[j]);
    if (!found && s < c) {
      uint64_t b = m[j];
      for (int t = 0; t < s; t++) b &= b - 1ull;
      e = j * 64 + __ffsll((unsigned long long)b) - 1;
      found = true;
    } else if (!found) {
      s -= c;
    }
  }
  return e;
}

// --------------------------------------------------------- unit dot product --
// D = sum over the unit of (MAGIC + q) * x for 16-bit activations: codes are
// or-ed into the mantissa of MAGIC = 128.0 (bf16, exact for codes < 128) or
// 1024.0 (f16, exact for codes < 1024), and v_dot2 multiplies two pairs at a
// time with fp32 accumulation. 8-bit codes with bf16 activations, and f32
// activations, use exact integer->fp32 conversion instead (MAGIC = 0). The
// caller removes MAGIC * sum(x) through the bias term.
template <int BITS, typename XT> struct Magic {
  static constexpr bool dot2 = !__is_same(XT, float) && !(BITS == 8 && __is_same(XT, bf16_t));
  static constexpr uint32_t bits = !dot2 ? 0u : (__is_same(XT, bf16_t) ? 0x43004300u : 0x64006400u);
  static constexpr float value = !dot2 ? 0.0f : (__is_same(XT, bf16_t) ? 128.0f : 1024.0f);
};

// a.lo b.lo + a.hi b.hi + c for two packed 16-bit pairs of type T
// (v_dot2_f32_bf16 / v_dot2_f32_f16).
template <typename T>
__device__ __forceinline__ float dot2_16(uint32_t a, uint32_t b, float c) {
  if constexpr (__is_same(T, bf16_t))
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                           __builtin_bit_cast(bf16x2_t, b), c, false);
  else
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c,
                                  false);
}

// x16: the unit's 32 activations in pair order, as 16 u32 (16-bit types);
// cp: code pairs from unpack_pairs<BITS, Magic<BITS, XT>::bits>.
template <int BITS, typename XT>
__device__ __forceinline__ float unit_dot16(const uint32_t (&cp)[16], const uint32_t (&x16)[16]) {
  float d = 0.f;
  if constexpr (Magic<BITS, XT>::dot2) {
#pragma unroll
    for (int i = 0; i < 16; i++) {
      if constexpr (__is_same(XT, bf16_t))
        d = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, cp[i]),
                                            __builtin_bit_cast(bf16x2_t, x16[i]), d, false);
      else
        d = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, cp[i]),
                                   __builtin_bit_cast(f16x2_t, x16[i]), d, false);
    }
  } else {
    // bf16 activations with 8-bit codes
#pragma unroll
    for (int i = 0; i < 16; i++) {
      const float xa = __uint_as_float(x16[i] << 16), xb = __uint_as_float(x16[i] & 0xFFFF0000u);
      d = __builtin_fmaf((float)(cp[i] & 0xFFFFu), xa, d);
      d = __builtin_fmaf((float)(cp[i] >> 16), xb, d);
    }
  }
  return d;
}

// f32 activations: x32 in pair order.
__device__ __forceinline__ float unit_dot32(const uint32_t (&cp)[16], const float (&x32)[32]) {
  float d0 = 0.f, d1 = 0.f;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    d0 = __builtin_fmaf((float)(cp[i] & 0xFFFFu), x32[2 * i], d0);
    d1 = __builtin_fmaf((float)(cp[i] >> 16), x32[2 * i + 1], d1);
  }
  return d0 + d1;
}

// Scale/bias element loads (scale dtype independent of activations).
template <typename ST> __device__ __forceinline__ float ld_sb(const void* p, size_t i) {
  return to_f<ST>(reinterpret_cast<const ST*>(p)[i]);
}

}  // namespace moe
