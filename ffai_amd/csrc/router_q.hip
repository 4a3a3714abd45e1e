// router_q.hip — router projection with affine-quantised weights (an mlx
// QuantizedLinear router or shared-expert gate, Sources/FFAI/Layers.swift:
// 371-400; loaded by Models/Text/Qwen3xText.swift:605-606, 660-661), on
// gfx950. One translation unit per bit width (MOE_BITS).
//
//   logits[t, e] = round(sum_k (s[e, g(k)] q[e, k] + b[e, g(k)]) x[t, k])
//                  (+ bias: round(logit + bias[e]))
//
// The weights are never rounded: codes enter the products exactly, as
// MAGIC + q in the 16-bit activation type (MAGIC = 128 for bf16, 1024 for
// f16; 8-bit codes with bf16 activations convert exactly without it), and the
// affine scale and bias apply per 32-value unit in fp32:
//   sum((s q + b) x) = s * sum((MAGIC + q) x) + (b - MAGIC s) * sum(x).
// Two kernels:
//  - router_qrow_kernel, few tokens: one wave per (expert, up to 8 tokens);
//    lane l takes units l + 64 j of the expert's row (v_dot2 over code pairs,
//    as the decode GEMVs do);
//  - router_qgemm_kernel, many tokens: a 32-token x 32-expert tile per block
//    on v_mfma_f32_32x32x16, the four waves splitting the hidden dimension in
//    64-value chunks; per 32 values one MFMA pair gives sum((MAGIC + q) x) and
//    one against all-ones gives sum(x), so the scale and bias of each unit
//    apply in fp32 to a fresh partial product.
#include <hip/hip_runtime.h>

#include "moe_common.hpp"
#include "moe_internal.hpp"
#include "decode_units.hpp"

#ifndef MOE_BITS
#define MOE_BITS 4
#endif

namespace moe {

// ------------------------------------------------------------- few tokens --
template <int BITS, typename XT, typename ST, int UR>
__global__ __launch_bounds__(256) void router_qrow_kernel(const XT* __restrict__ x, const GemvProj W,
                                                          const XT* __restrict__ bias,
                                                          XT* __restrict__ logits, int T, int H,
                                                          int E, int gsh, int tchunks) {
  // wave-uniform (readfirstlane keeps the buffer resources below scalar)
  const int gw = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
  const int e = gw / tchunks, tc = gw - e * tchunks;
  if (e >= E) return;  // the kernel has no block barrier
  const int lane = threadIdx.x & 63;
  const int t0 = tc * 8, nt = min(8, T - t0);
  const int CU = H >> 5, groups = CU >> gsh, row_words = CU * BITS;
  const uint32_t bv = bias_raw<XT>(bias, e);  // converted where it is added
  const ProjView V = proj_view<BITS, ST>(W, 0u, E, row_words, groups);
  const uint32_t wstep = (uint32_t)(64 * BITS * 4), sstep = (uint32_t)((64 >> gsh) * sizeof(ST));
  WUnit<BITS, ST> w[UR];
  bload_units<BITS, ST, UR>(V, unit_addr<BITS, ST>((uint32_t)e, row_words, groups, lane, gsh), wstep,
                            sstep, w);
  float acc[8];
#pragma unroll
  for (int t = 0; t < 8; t++) {
    acc[t] = 0.f;
    if (t < nt) {  // wave-uniform
      const rsrc_t xr = make_rsrc(x + (size_t)(t0 + t) * H, (uint32_t)(H * sizeof(XT)));
      XUnit<XT> xu[UR];
      float xs[UR];
      bload_x_units<BITS, XT, UR>(xr, lane, 64, xu, xs);
      acc[t] = group_sum(dot_units<BITS, XT, ST, UR>(w, xu, xs, lane, 64, CU), 6);
    }
  }
  if (lane == 63) {
    for (int t = 0; t < nt; t++) {
      float l = round_to<XT>(acc[t]);
      if (bias) l = round_to<XT>(l + bias_f<XT>(bv));
      logits[(size_t)(t0 + t) * E + e] = from_f<XT>(l);
    }
  }
}

// ------------------------------------------------------------ many tokens --
typedef float f32x16_t __attribute__((ext_vector_type(16)));
constexpr int kRqWaves = 4;

template <typename XT> struct RqMfma;
template <> struct RqMfma<bf16_t> {
  typedef __bf16 V __attribute__((ext_vector_type(8)));
  static constexpr uint32_t kOnes = 0x3F803F80u;  // (1.0, 1.0)
  static __device__ __forceinline__ f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(V, a), __builtin_bit_cast(V, b), c, 0, 0, 0);
  }
};
template <> struct RqMfma<f16_t> {
  typedef _Float16 V __attribute__((ext_vector_type(8)));
  static constexpr uint32_t kOnes = 0x3C003C00u;
  static __device__ __forceinline__ f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(V, a), __builtin_bit_cast(V, b), c, 0, 0, 0);
  }
};

// The unit's bit stream with its first 8 values dropped when `drop` (lane
// half h = 1 takes values 8..15 and 24..31 of each 16-value step pair).
template <int BITS>
__device__ __forceinline__ void drop8(const uint32_t (&w)[BITS], bool drop, uint32_t (&o)[BITS]) {
  constexpr int S = (8 * BITS) / 32, SH = (8 * BITS) % 32;
#pragma unroll
  for (int i = 0; i < BITS; i++) {
    const uint32_t lo = (i + S < BITS) ? w[i + S] : 0u;
    const uint32_t hi = (i + S + 1 < BITS) ? w[i + S + 1] : 0u;
    const uint32_t d = SH ? ((lo >> SH) | (hi << (32 - SH))) : lo;
    o[i] = drop ? d : w[i];
  }
}

// Values v0 .. v0 + 7 (compile-time v0) of a unit as four 16-bit pairs in
// natural order, each code or-ed into MAGIC (exact), or, without a magic
// offset (8-bit codes, bf16), converted exactly.
template <int BITS, typename XT>
__device__ __forceinline__ u32x4_t code_frag(const uint32_t (&w)[BITS], int v0) {
  constexpr bool kMagic = Magic<BITS, XT>::dot2;
  constexpr uint32_t M = Magic<BITS, XT>::bits & 0xFFFFu;
  uint32_t c[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const int bit = (v0 + e) * BITS, lo = bit >> 5, sh = bit & 31;
    uint32_t v = w[lo] >> sh;
    if (sh + BITS > 32) v |= w[lo + 1] << (32 - sh);
    c[e] = v & ((1u << BITS) - 1u);
  }
  u32x4_t r;
#pragma unroll
  for (int p = 0; p < 4; p++) {
    uint32_t a, b;
    if constexpr (kMagic) {
      a = c[2 * p] | M;
      b = c[2 * p + 1] | M;
    } else {  // bf16 of an integer below 256 is exact
      a = __float_as_uint((float)c[2 * p]) >> 16;
      b = __float_as_uint((float)c[2 * p + 1]) >> 16;
    }
    r[p] = a | (b << 16);
  }
  return r;
}

template <int BITS, typename XT, typename ST>
__global__ __launch_bounds__(64 * kRqWaves) void router_qgemm_kernel(const XT* __restrict__ x,
                                                                    const GemvProj W,
                                                                    const XT* __restrict__ bias,
                                                                    XT* __restrict__ logits, int T,
                                                                    int H, int E, int gsh) {
  __shared__ float part[kRqWaves][32 * 33];
  constexpr float MAGIC = Magic<BITS, XT>::value;
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int col = lane & 31, h = lane >> 5;
  const int t0 = blockIdx.x * 32, e0 = blockIdx.y * 32;
  const uint32_t row = (uint32_t)min(t0 + col, T - 1);  // rows past T repeat the last token
  const uint32_t ex = (uint32_t)min(e0 + col, E - 1);  // experts past E repeat the last one
  const int CU = H >> 5, groups = CU >> gsh, row_words = CU * BITS;
  const rsrc_t xr = make_rsrc(x, (uint32_t)((size_t)T * H * sizeof(XT)));
  const rsrc_t wr = make_rsrc(W.w, (uint32_t)((size_t)E * row_words * 4));
  const rsrc_t sr = make_rsrc(W.s, (uint32_t)((size_t)E * groups * sizeof(ST)));
  const rsrc_t br = make_rsrc(W.b, (uint32_t)((size_t)E * groups * sizeof(ST)));
  const uint32_t xo = (row * (uint32_t)H + 8u * (uint32_t)h) * 2u;
  const uint32_t wo = ex * (uint32_t)row_words * 4u;
  const uint32_t so = ex * (uint32_t)groups;
  const int G = H >> 6;
  const int ng = (G - wv + kRqWaves - 1) / kRqWaves;  // chunks wv + 4 i, i < ng

  struct Set {
    u32x4_t a[4];
    uint32_t w[2][BITS];
    ST s[2], b[2];
  };
  auto load = [&](int i, Set& st) __attribute__((always_inline)) {
    const int c = min(wv + kRqWaves * i, G - 1);  // clamped: in bounds, never multiplied
    const uint32_t kb = (uint32_t)c * 128u;
#pragma unroll
    for (int q = 0; q < 4; q++) st.a[q] = bload128(xr, xo + kb + 32u * (uint32_t)q);
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int unit = 2 * c + u;
      bload_unit<BITS>(wr, wo + (uint32_t)(unit * BITS) * 4u, st.w[u]);
      const uint32_t gi = (so + (uint32_t)(unit >> gsh)) * (uint32_t)sizeof(ST);
      st.s[u] = __builtin_bit_cast(ST, bload16(sr, gi));
      st.b[u] = __builtin_bit_cast(ST, bload16(br, gi));
    }
  };
  const u32x4_t ones = {RqMfma<XT>::kOnes, RqMfma<XT>::kOnes, RqMfma<XT>::kOnes, RqMfma<XT>::kOnes};
  f32x16_t acc = {};
  auto run = [&](const Set& st) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 2; u++) {
      uint32_t wd[BITS];
      drop8<BITS>(st.w[u], h != 0, wd);
      f32x16_t P = {}, Q = {};
#pragma unroll
      for (int m = 0; m < 2; m++) {
        const u32x4_t b = code_frag<BITS, XT>(wd, 16 * m);
        P = RqMfma<XT>::mma(st.a[2 * u + m], b, P);
        Q = RqMfma<XT>::mma(st.a[2 * u + m], ones, Q);
      }
      const float s = to_f<ST>(st.s[u]);
      const float c = to_f<ST>(st.b[u]) - MAGIC * s;
#pragma unroll
      for (int r = 0; r < 16; r++) acc[r] = __builtin_fmaf(s, P[r], __builtin_fmaf(c, Q[r], acc[r]));
    }
  };
  Set s0, s1;
  load(0, s0);
  for (int i = 0; i < ng; i += 2) {  // ng is wave-uniform: scalar branches
    load(i + 1, s1);
    run(s0);
    if (i + 1 >= ng) break;
    load(i + 2, s0);
    run(s1);
  }

  // lane (col, h) holds token rows 8 (r / 4) + 4 h + r % 4 of expert column col
#pragma unroll
  for (int r = 0; r < 16; r++) part[wv][(8 * (r >> 2) + 4 * h + (r & 3)) * 33 + col] = acc[r];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 1024 / (64 * kRqWaves); j++) {
    const int o = threadIdx.x + 64 * kRqWaves * j;
    const int r = o >> 5, c = o & 31;
    float v = part[0][r * 33 + c];
#pragma unroll
    for (int w = 1; w < kRqWaves; w++) v += part[w][r * 33 + c];
    if (t0 + r < T && e0 + c < E) {
      float l = round_to<XT>(v);
      if (bias) l = round_to<XT>(l + to_f<XT>(bias[e0 + c]));
      logits[(size_t)(t0 + r) * E + e0 + c] = from_f<XT>(l);
    }
  }
}

// ---------------------------------------------------------------- launch --
template <int BITS, typename XT, typename ST>
static hipError_t launch_rq_t(const void* x, int T, int H, const GemvProj& W, int gsh,
                              const void* bias, int E, void* logits, hipStream_t st) {
  // the matrix-core kernel views x as one buffer with 32-bit offsets: beyond
  // 4 GiB of input rows the per-row kernel (64-bit row addresses) runs
  if (T >= 32 && H % 64 == 0 && (size_t)T * H * sizeof(XT) < (1ull << 32)) {
    hipLaunchKernelGGL((router_qgemm_kernel<BITS, XT, ST>), dim3((T + 31) / 32, (E + 31) / 32),
                       dim3(64 * kRqWaves), 0, st, (const XT*)x, W, (const XT*)bias, (XT*)logits,
                       T, H, E, gsh);
    return hipGetLastError();
  }
  const int tchunks = (T + 7) / 8;
  const long waves = (long)E * tchunks;
  const int wpb = (T <= 8) ? 1 : 4;  // small batches: spread the experts over the CUs
  const int grid = (int)((waves + wpb - 1) / wpb);
  const int ur = (H / 32 + 63) / 64;
#define MOE_RQ(UR)                                                                             \
  hipLaunchKernelGGL((router_qrow_kernel<BITS, XT, ST, UR>), dim3(grid), dim3(64 * wpb), 0, st, \
                     (const XT*)x, W, (const XT*)bias, (XT*)logits, T, H, E, gsh, tchunks);    \
  return hipGetLastError();
  if (ur <= 1) { MOE_RQ(1) }
  if (ur <= 2) { MOE_RQ(2) }
  if (ur <= 3) { MOE_RQ(3) }
  if (ur <= 4) { MOE_RQ(4) }
#undef MOE_RQ
  return hipErrorInvalidValue;
}

#define MOE_CAT2(a, b) a##b
#define MOE_CAT(a, b) MOE_CAT2(a, b)

// x, logits, bias in xdt (16-bit); W: one stacked projection [1, E, H]
// (W.ob unused); H % 32 == 0, H <= 8192.
hipError_t MOE_CAT(launch_router_q_b, MOE_BITS)(const void* x, int xdt, int T, int H,
                                                 const GemvProj& W, int sbdt, int gsh,
                                                 const void* bias, int E, void* logits,
                                                 hipStream_t st) {
  if (xdt == DT_BF16 && sbdt == DT_BF16) return launch_rq_t<MOE_BITS, bf16_t, bf16_t>(x, T, H, W, gsh, bias, E, logits, st);
  if (xdt == DT_BF16 && sbdt == DT_F16) return launch_rq_t<MOE_BITS, bf16_t, f16_t>(x, T, H, W, gsh, bias, E, logits, st);
  if (xdt == DT_F16 && sbdt == DT_F16) return launch_rq_t<MOE_BITS, f16_t, f16_t>(x, T, H, W, gsh, bias, E, logits, st);
  if (xdt == DT_F16 && sbdt == DT_BF16) return launch_rq_t<MOE_BITS, f16_t, bf16_t>(x, T, H, W, gsh, bias, E, logits, st);
  return hipErrorInvalidValue;
}

}  // namespace moe
