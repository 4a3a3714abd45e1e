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

template <typename T>
__device__ __forceinline__ void load8(const T* __restrict__ p, float (&v)[8]) {
  if constexpr (__is_same(T, float)) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[2 * j] = to_f<T>(__builtin_bit_cast(T, (uint16_t)(w[j] & 0xFFFFu)));
      v[2 * j + 1] = to_f<T>(__builtin_bit_cast(T, (uint16_t)(w[j] >> 16)));
    }
  }
}

// logits[t, e] = round(W[e] . x[t]) (+ bias: round(logit + b)). One wave per
// (expert, chunk of 8 tokens); lanes stride over hidden 8 values at a time.
template <typename XT, typename WT>
__global__ __launch_bounds__(256) void router_logits_kernel(const XT* __restrict__ x,
                                                            const WT* __restrict__ W,
                                                            const XT* __restrict__ bias,
                                                            XT* __restrict__ logits, int T, int H,
                                                            int E, int tchunks) {
  const int gw = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
  const int e = gw / tchunks, tc = gw - e * tchunks;
  if (e >= E) return;
  const int lane = threadIdx.x & 63;
  const int t0 = tc * 8, nt = min(8, T - t0);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const WT* w = W + (size_t)e * H;
  constexpr int UNR = 4;  // hidden chunks in flight per lane
  for (int h0 = lane * 8; h0 < H; h0 += 512 * UNR) {
    float wv[UNR][8];
#pragma unroll
    for (int u = 0; u < UNR; u++)
      if (h0 + u * 512 < H) load8<WT>(w + h0 + u * 512, wv[u]);
#pragma unroll
    for (int t = 0; t < 8; t++) {
      if (t < nt) {
        float xv[UNR][8];
#pragma unroll
        for (int u = 0; u < UNR; u++)
          if (h0 + u * 512 < H) load8<XT>(x + (size_t)(t0 + t) * H + h0 + u * 512, xv[u]);
#pragma unroll
        for (int u = 0; u < UNR; u++)
          if (h0 + u * 512 < H)
#pragma unroll
            for (int j = 0; j < 8; j++) acc[t] = __builtin_fmaf(wv[u][j], xv[u][j], acc[t]);
      }
    }
  }
#pragma unroll
  for (int t = 0; t < 8; t++)
    if (t < nt) acc[t] = wave_sum_width(acc[t], 64);
  if (lane == 0) {
    for (int t = 0; t < nt; t++) {
      float l = round_to<XT>(acc[t]);
      if (bias) l = round_to<XT>(l + to_f<XT>(bias[e]));
      logits[(size_t)(t0 + t) * E + e] = from_f<XT>(l);
    }
  }
}

// One wave per token row (wave_topk); weights are reproducible bit for bit.
template <typename XT>
__global__ __launch_bounds__(256) void router_topk_kernel(const XT* __restrict__ logits, int T,
                                                          int E, int k, int gating, int norm,
                                                          const float* __restrict__ ebias,
                                                          uint32_t* __restrict__ idx_out,
                                                          float* __restrict__ w_out) {
  __shared__ float sc[4][kTopkMaxE];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wv;
  if (t >= T) return;  // wave-uniform; the kernel has no block barrier
  int sel;
  float w;
  wave_topk<XT>(logits + (size_t)t * E, E, k, gating, norm, ebias, sc[wv], true, &sel, &w);
  if (lane < k) {
    idx_out[(size_t)t * k + lane] = (uint32_t)sel;
    w_out[(size_t)t * k + lane] = w;
  }
}

hipError_t launch_router_logits(const void* x, int xdt, int T, int H, const void* W, int wdt,
                                const void* bias, int E, void* logits, hipStream_t st) {
  const int tchunks = (T + 7) / 8;
  const long waves = (long)E * tchunks;
  const int grid = (int)((waves + 3) / 4);
#define MOE_RL(XT, WT)                                                                      \
  hipLaunchKernelGGL((router_logits_kernel<XT, WT>), dim3(grid), dim3(256), 0, st,         \
                     (const XT*)x, (const WT*)W, (const XT*)bias, (XT*)logits, T, H, E,     \
                     tchunks);                                                              \
  return hipGetLastError();
  if (xdt == DT_BF16) {
    if (wdt == DT_BF16) { MOE_RL(bf16_t, bf16_t) }
    if (wdt == DT_F16) { MOE_RL(bf16_t, f16_t) }
    if (wdt == DT_F32) { MOE_RL(bf16_t, float) }
  } else if (xdt == DT_F16) {
    if (wdt == DT_BF16) { MOE_RL(f16_t, bf16_t) }
    if (wdt == DT_F16) { MOE_RL(f16_t, f16_t) }
    if (wdt == DT_F32) { MOE_RL(f16_t, float) }
  } else if (xdt == DT_F32) {
    if (wdt == DT_BF16) { MOE_RL(float, bf16_t) }
    if (wdt == DT_F16) { MOE_RL(float, f16_t) }
    if (wdt == DT_F32) { MOE_RL(float, float) }
  }
#undef MOE_RL
  return hipErrorInvalidValue;
}

hipError_t launch_router_topk(const void* logits, int dt, int T, int E, int k, int gating,
                              int norm, const float* ebias, uint32_t* idx, float* w,
                              hipStream_t st) {
  const int grid = (T + 3) / 4;
#define MOE_TK(XT)                                                                          \
  hipLaunchKernelGGL((router_topk_kernel<XT>), dim3(grid), dim3(256), 0, st,               \
                     (const XT*)logits, T, E, k, gating, norm, ebias, idx, w);              \
  return hipGetLastError();
  if (dt == DT_BF16) { MOE_TK(bf16_t) }
  if (dt == DT_F16) { MOE_TK(f16_t) }
  if (dt == DT_F32) { MOE_TK(float) }
#undef MOE_TK
  return hipErrorInvalidValue;
}

}  // namespace moe
