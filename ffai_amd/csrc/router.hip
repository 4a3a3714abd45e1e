// router.hip — router projection and top-k selection for gfx950.
//
// Replaces the gate GEMV + host readback + MoERouter.route of
// Sources/FFAI/Models/MoELayer.swift:540-573 (decode), :689-750 (prefill) and
// the GPU router Ops.moeRouterTopKMany (Sources/FFAI/Ops/Ops.swift:2589-2662),
// generalised to every gating mode of MoERouter.route (MoELayer.swift:
// 140-205) and to GPT-OSS's biased router (Models/Text/GPTOSSText.swift:
// 345-366,1349-1361). Selection order is (value desc, index asc): the
// reference heap's tie rule (MoELayer.swift:223-296).
#include "moe_common.hpp"
#include "moe_internal.hpp"

namespace moe {

// 8 consecutive elements at byte offset `off` of a raw buffer view, as fp32;
// elements past the view read as zero.
template <typename T>
__device__ __forceinline__ void bload8(rsrc_t r, uint32_t off, float (&v)[8]) {
  if constexpr (__is_same(T, float)) {
    const u32x4_t a = bload128(r, off), b = bload128(r, off + 16);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[j] = __uint_as_float(a[j]);
      v[4 + j] = __uint_as_float(b[j]);
    }
  } else {
    const u32x4_t a = bload128(r, off);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[2 * j] = to_f<T>(__builtin_bit_cast(T, (uint16_t)(a[j] & 0xFFFFu)));
      v[2 * j + 1] = to_f<T>(__builtin_bit_cast(T, (uint16_t)(a[j] >> 16)));
    }
  }
}

// logits[t, e] = round(W[e] . x[t]) (+ bias: round(logit + b)). One wave per
// (expert, chunk of up to 8 tokens); lane l takes the 8-element chunks
// l + 64 j, j < NL, of the hidden dimension (NL * 512 >= H; chunks past H
// read zeros), so the whole weight row is requested in one round trip.
// Weights and activations of one 16-bit type multiply pairwise with v_dot2
// (fp32 accumulate) in chunk order; other type pairs use fp32 fma.
template <typename XT, typename WT, int NL>
__global__ __launch_bounds__(256) void router_logits_kernel(const XT* __restrict__ x,
                                                            const WT* __restrict__ W,
                                                            const XT* __restrict__ bias,
                                                            XT* __restrict__ logits, int T, int H,
                                                            int E, int tchunks) {
  // wave-uniform (readfirstlane keeps the buffer resources below scalar)
  const int gw = __builtin_amdgcn_readfirstlane(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6));
  const int e = gw / tchunks, tc = gw - e * tchunks;
  if (e >= E) return;  // the kernel has no block barrier
  const int lane = threadIdx.x & 63;
  const int t0 = tc * 8, nt = min(8, T - t0);
  const float bv = bias ? to_f<XT>(bias[e]) : 0.f;  // issued before the row loads
  const rsrc_t wr = make_rsrc(W + (size_t)e * H, (uint32_t)(H * sizeof(WT)));
  float acc[8];
  if constexpr (__is_same(XT, WT) && !__is_same(XT, float)) {
    u32x4_t wv[NL];
#pragma unroll
    for (int j = 0; j < NL; j++) wv[j] = bload128(wr, (uint32_t)((lane + 64 * j) * 16));
#pragma unroll
    for (int t = 0; t < 8; t++) {
      acc[t] = 0.f;
      if (t < nt) {  // wave-uniform
        const rsrc_t xr = make_rsrc(x + (size_t)(t0 + t) * H, (uint32_t)(H * sizeof(XT)));
#pragma unroll
        for (int j = 0; j < NL; j++) {
          const u32x4_t xv = bload128(xr, (uint32_t)((lane + 64 * j) * 16));
#pragma unroll
          for (int i = 0; i < 4; i++) acc[t] = dot2_16<XT>(wv[j][i], xv[i], acc[t]);
        }
        acc[t] = group_sum(acc[t], 6);
      }
    }
  } else {
    float wv[NL][8];
#pragma unroll
    for (int j = 0; j < NL; j++) bload8<WT>(wr, (uint32_t)((lane + 64 * j) * 8 * sizeof(WT)), wv[j]);
#pragma unroll
    for (int t = 0; t < 8; t++) {
      acc[t] = 0.f;
      if (t < nt) {  // wave-uniform
        const rsrc_t xr = make_rsrc(x + (size_t)(t0 + t) * H, (uint32_t)(H * sizeof(XT)));
#pragma unroll
        for (int j = 0; j < NL; j++) {
          float xv[8];
          bload8<XT>(xr, (uint32_t)((lane + 64 * j) * 8 * sizeof(XT)), xv);
#pragma unroll
          for (int i = 0; i < 8; i++) acc[t] = __builtin_fmaf(wv[j][i], xv[i], acc[t]);
        }
        acc[t] = group_sum(acc[t], 6);
      }
    }
  }
  if (lane == 63) {
    for (int t = 0; t < nt; t++) {
      float l = round_to<XT>(acc[t]);
      if (bias) l = round_to<XT>(l + bv);
      logits[(size_t)(t0 + t) * E + e] = from_f<XT>(l);
    }
  }
}

// One wave per token row (wave_topk); weights are reproducible bit for bit.
template <typename XT>
__global__ __launch_bounds__(256) void router_topk_kernel(const XT* __restrict__ logits, int T,
                                                          int E, int k, const RouteOpts ro,
                                                          uint32_t* __restrict__ idx_out,
                                                          float* __restrict__ w_out) {
  __shared__ float sc[4][kTopkMaxE];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wv;
  if (t >= T) return;  // wave-uniform; the kernel has no block barrier
  int sel;
  float w;
  wave_topk<XT>(logits + (size_t)t * E, E, k, ro, sc[wv], true, &sel, &w);
  if (lane < k) {
    idx_out[(size_t)t * k + lane] = (uint32_t)sel;
    w_out[(size_t)t * k + lane] = w;
  }
}

template <typename XT, typename WT>
static hipError_t launch_rl(const void* x, int T, int H, const void* W, const void* bias, int E,
                            void* logits, hipStream_t st) {
  const int tchunks = (T + 7) / 8;
  const long waves = (long)E * tchunks;
  // small batches: one wave per block spreads the experts over the CUs
  const int wpb = (T <= 8) ? 1 : 4;
  const int grid = (int)((waves + wpb - 1) / wpb);
  const int nl = (H + 511) / 512;
#define MOE_RL(NL)                                                                            \
  hipLaunchKernelGGL((router_logits_kernel<XT, WT, NL>), dim3(grid), dim3(64 * wpb), 0, st,  \
                     (const XT*)x, (const WT*)W, (const XT*)bias, (XT*)logits, T, H, E,       \
                     tchunks);                                                                \
  return hipGetLastError();
  if (nl <= 1) { MOE_RL(1) }
  if (nl <= 2) { MOE_RL(2) }
  if (nl <= 4) { MOE_RL(4) }
  if (nl <= 8) { MOE_RL(8) }
  if (nl <= 16) { MOE_RL(16) }
#undef MOE_RL
  return hipErrorInvalidValue;
}

hipError_t launch_router_logits(const void* x, int xdt, int T, int H, const void* W, int wdt,
                                const void* bias, int E, void* logits, hipStream_t st) {
#define MOE_RL2(XT, WT) return launch_rl<XT, WT>(x, T, H, W, bias, E, logits, st);
  if (xdt == DT_BF16) {
    if (wdt == DT_BF16) { MOE_RL2(bf16_t, bf16_t) }
    if (wdt == DT_F16) { MOE_RL2(bf16_t, f16_t) }
    if (wdt == DT_F32) { MOE_RL2(bf16_t, float) }
  } else if (xdt == DT_F16) {
    if (wdt == DT_BF16) { MOE_RL2(f16_t, bf16_t) }
    if (wdt == DT_F16) { MOE_RL2(f16_t, f16_t) }
    if (wdt == DT_F32) { MOE_RL2(f16_t, float) }
  } else if (xdt == DT_F32) {
    if (wdt == DT_BF16) { MOE_RL2(float, bf16_t) }
    if (wdt == DT_F16) { MOE_RL2(float, f16_t) }
    if (wdt == DT_F32) { MOE_RL2(float, float) }
  }
#undef MOE_RL2
  return hipErrorInvalidValue;
}

hipError_t launch_router_topk(const void* logits, int dt, int T, int E, int k,
                              const RouteOpts& ro, uint32_t* idx, float* w, hipStream_t st) {
  const int grid = (T + 3) / 4;
#define MOE_TK(XT)                                                                          \
  hipLaunchKernelGGL((router_topk_kernel<XT>), dim3(grid), dim3(256), 0, st,               \
                     (const XT*)logits, T, E, k, ro, idx, w);                              \
  return hipGetLastError();
  if (dt == DT_BF16) { MOE_TK(bf16_t) }
  if (dt == DT_F16) { MOE_TK(f16_t) }
  if (dt == DT_F32) { MOE_TK(float) }
#undef MOE_TK
  return hipErrorInvalidValue;
}

}  // namespace moe
