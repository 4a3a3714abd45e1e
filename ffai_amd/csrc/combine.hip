// combine.hip — weighted combine back to token order, shared-expert add,
// elementwise activation and standalone affine dequantisation for gfx950.
//
//   unpermute      Ops.moeUnpermute (Sources/FFAI/Ops/Ops.swift:5030-5110) with
//                  the combine weights rounded to the activation dtype first
//                  (Sources/FFAI/Models/MoELayer.swift:921-935)
//   shared add     MoELayer.swift:620-624 (unconditional add) and
//                  Ops.sigmoidScalarFMA (Ops.swift:6256-6317; Qwen3xText.swift:
//                  1054-1103): y = round(routed + sigmoid(g) * shared)
//   activation     Ops.swiglu (Ops.swift:6411-6460) / GPT-OSS clamped swish
//   dequantize     QuantizedOps.dequantizeAffine (QuantizedOps.swift:62-221)
//   add + RMSNorm  Ops.addAndRmsNorm (Ops.swift:676-730), the decoder step
//                  before the MoE block (Qwen3xText.swift:2650-2660)
//   residual       the decoder step after it folded into the final store:
//                  Ops.sigmoidScalarFMAResidual (OpsFused.swift:699-753),
//                  y = round(residual + routed + sigmoid(g) * shared), or
//                  y = round(residual + routed) without a shared expert
#include <algorithm>

#include "moe_common.hpp"
#include "moe_internal.hpp"

namespace moe {

template <typename T> struct Vec8 {
  static __device__ __forceinline__ void load(const T* p, float (&v)[8]) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      v[2 * j] = to_f<T>(__builtin_bit_cast(T, (uint16_t)(w[j] & 0xFFFFu)));
      v[2 * j + 1] = to_f<T>(__builtin_bit_cast(T, (uint16_t)(w[j] >> 16)));
    }
  }
  static __device__ __forceinline__ void store(T* p, const float (&v)[8]) {
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint16_t lo = __builtin_bit_cast(uint16_t, from_f<T>(v[2 * j]));
      const uint16_t hi = __builtin_bit_cast(uint16_t, from_f<T>(v[2 * j + 1]));
      w[j] = (uint32_t)lo | ((uint32_t)hi << 16);
    }
    *reinterpret_cast<uint4*>(p) = make_uint4(w[0], w[1], w[2], w[3]);
  }
};
template <> struct Vec8<float> {
  static __device__ __forceinline__ void load(const float* p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  }
  static __device__ __forceinline__ void store(float* p, const float (&v)[8]) {
    reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
  }
};

// shared_mode: 0 none, 1 unconditional add, 2 sigmoid-gated add.
template <typename XT>
__device__ __forceinline__ float shared_gate(int mode, const XT* logit, int t) {
  if (mode == 2) return 1.0f / (1.0f + __expf(-to_f<XT>(logit[t])));
  return 1.0f;
}

constexpr int kCombineBatch = 8;  // expert ranks whose rows load together

// One block per token; threads stride over hidden 8 values at a time.
// res (nullable): the decoder residual added before the final rounding.
template <typename XT>
__global__ __launch_bounds__(256) void unpermute_kernel(const XT* __restrict__ Y,
                                                        const uint32_t* __restrict__ inv,
                                                        const float* __restrict__ w, int T, int H,
                                                        int k, XT* __restrict__ out,
                                                        const XT* __restrict__ sout,
                                                        const XT* __restrict__ slogit, int smode,
                                                        const XT* __restrict__ res) {
  const int t = blockIdx.x;
  const uint32_t M = (uint32_t)T * (uint32_t)k;
  const float g = smode ? shared_gate<XT>(smode, slogit, t) : 0.f;
  for (int h = threadIdx.x * 8; h < H; h += blockDim.x * 8) {
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    // ranks in batches of kCombineBatch: every position, then every row of a
    // batch in flight before its fused multiply-adds (in rank order, as the
    // loop over the ranks one at a time contracted them); a position past M
    // reads row 0 and leaves the sum unchanged
    for (int s0 = 0; s0 < k; s0 += kCombineBatch) {
      uint32_t p[kCombineBatch];
      float ws[kCombineBatch];
#pragma unroll
      for (int q = 0; q < kCombineBatch; q++) {
        const int s = min(s0 + q, k - 1);
        p[q] = inv[(size_t)t * k + s];
        ws[q] = round_to<XT>(w[(size_t)t * k + s]);
      }
      float y[kCombineBatch][8];
#pragma unroll
      for (int q = 0; q < kCombineBatch; q++)
        Vec8<XT>::load(Y + (size_t)(p[q] < M ? p[q] : 0u) * H + h, y[q]);
#pragma unroll
      for (int q = 0; q < kCombineBatch; q++) {
        const bool valid = s0 + q < k && p[q] < M;
#pragma unroll
        for (int j = 0; j < 8; j++) acc[j] = valid ? __builtin_fmaf(ws[q], y[q][j], acc[j]) : acc[j];
      }
    }
#pragma unroll
    for (int j = 0; j < 8; j++) acc[j] = round_to<XT>(acc[j]);
    if (res) {
      float rv[8];
      Vec8<XT>::load(res + (size_t)t * H + h, rv);
#pragma unroll
      for (int j = 0; j < 8; j++) acc[j] = rv[j] + acc[j];
    }
    if (smode) {
      float sv[8];
      Vec8<XT>::load(sout + (size_t)t * H + h, sv);
#pragma unroll
      for (int j = 0; j < 8; j++) acc[j] = acc[j] + g * sv[j];
    }
    Vec8<XT>::store(out + (size_t)t * H + h, acc);
  }
}

template <typename XT>
__global__ __launch_bounds__(256) void add_shared_kernel(XT* __restrict__ y,
                                                         const XT* __restrict__ sout,
                                                         const XT* __restrict__ slogit, int smode,
                                                         int H, const XT* __restrict__ res) {
  const int t = blockIdx.x;
  const float g = shared_gate<XT>(smode, slogit, t);
  for (int h = threadIdx.x * 8; h < H; h += blockDim.x * 8) {
    float a[8], b[8];
    Vec8<XT>::load(y + (size_t)t * H + h, a);
    Vec8<XT>::load(sout + (size_t)t * H + h, b);
    if (res) {
      float rv[8];
      Vec8<XT>::load(res + (size_t)t * H + h, rv);
#pragma unroll
      for (int j = 0; j < 8; j++) a[j] = rv[j] + a[j];
    }
#pragma unroll
    for (int j = 0; j < 8; j++) a[j] = a[j] + g * b[j];
    Vec8<XT>::store(y + (size_t)t * H + h, a);
  }
}

template <typename XT>
__global__ __launch_bounds__(256) void activation_kernel(const XT* __restrict__ g,
                                                         const XT* __restrict__ u,
                                                         XT* __restrict__ out, int64_t n, int act,
                                                         float alpha, float limit) {
  // squared ReLU reads the up projection only; g may be null for it
  const bool gated = act != ACT_RELU2;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float gv = gated ? to_f<XT>(g[i]) : 0.0f;
    out[i] = from_f<XT>(apply_act<XT>(gv, to_f<XT>(u[i]), act, alpha, limit));
  }
}

// bf16 rows -> the f16 A operand of the grouped GEMM (bf16x8_to_a16), 8
// values per thread and step.
__global__ __launch_bounds__(256) void to_a16_kernel(const uint4* __restrict__ x,
                                                     uint4* __restrict__ y, int64_t n8) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n8;
       i += (int64_t)gridDim.x * blockDim.x)
    y[i] = bf16x8_to_a16<kA16Shift>(x[i]);
}

hipError_t launch_to_a16(const void* x, void* y, int64_t n, hipStream_t st) {
  if (n % 8 != 0) return hipErrorInvalidValue;
  const int64_t n8 = n / 8;
  const int grid = (int)std::min<int64_t>((n8 + 255) / 256, 4096);
  hipLaunchKernelGGL(to_a16_kernel, dim3(grid), dim3(256), 0, st,
                     reinterpret_cast<const uint4*>(x), reinterpret_cast<uint4*>(y), n8);
  return hipGetLastError();
}

// One block per row: s = round(a + b) stored to res, then
// xn = round(s / sqrt(mean(s^2) + eps) * w) stored to xn. A thread keeps its
// (up to kNormChunks) 8-value chunks in registers between the two halves.
constexpr int kNormChunks = 4;  // rows up to 256 * 8 * 4 = 8192 values

template <typename XT>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const XT* __restrict__ a,
                                                          const XT* __restrict__ b,
                                                          const XT* __restrict__ w, float eps,
                                                          int H, XT* __restrict__ res,
                                                          XT* __restrict__ xn) {
  __shared__ float part[4];
  const size_t row = (size_t)blockIdx.x * H;
  float sv[kNormChunks][8];
  float ssq = 0.f;
#pragma unroll
  for (int c = 0; c < kNormChunks; c++) {
    const int h = (threadIdx.x + c * 256) * 8;
    if (h < H) {
      float av[8], bv[8];
      Vec8<XT>::load(a + row + h, av);
      Vec8<XT>::load(b + row + h, bv);
#pragma unroll
      for (int j = 0; j < 8; j++) {
        sv[c][j] = round_to<XT>(av[j] + bv[j]);
        ssq = __builtin_fmaf(sv[c][j], sv[c][j], ssq);
      }
      Vec8<XT>::store(res + row + h, sv[c]);
    }
  }
  ssq = group_sum(ssq, 6);
  if ((threadIdx.x & 63) == 63) part[threadIdx.x >> 6] = ssq;
  __syncthreads();
  const float tot = (part[0] + part[1]) + (part[2] + part[3]);
  const float rms = sqrtf(tot / (float)H + eps);
#pragma unroll
  for (int c = 0; c < kNormChunks; c++) {
    const int h = (threadIdx.x + c * 256) * 8;
    if (h < H) {
      float wv[8], o[8];
      Vec8<XT>::load(w + h, wv);
#pragma unroll
      for (int j = 0; j < 8; j++) o[j] = sv[c][j] / rms * wv[j];
      Vec8<XT>::store(xn + row + h, o);
    }
  }
}

template <typename ST, typename OT>
__global__ __launch_bounds__(256) void dequantize_kernel(const uint32_t* __restrict__ w,
                                                         const ST* __restrict__ s,
                                                         const ST* __restrict__ b, int bits,
                                                         int gs, int64_t numel,
                                                         OT* __restrict__ out) {
#pragma clang fp contract(off)
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < numel;
       i += (int64_t)gridDim.x * blockDim.x) {
    const uint64_t bit = (uint64_t)i * (uint64_t)bits;
    const uint64_t word = bit >> 5;
    const uint32_t sh = (uint32_t)(bit & 31u);
    uint64_t win = w[word];
    if (sh + (uint32_t)bits > 32u) win |= (uint64_t)w[word + 1] << 32;
    const float q = (float)((uint32_t)(win >> sh) & ((1u << bits) - 1u));
    const int64_t g = i / gs;
    const float sq = to_f<ST>(s[g]) * q;
    out[i] = from_f<OT>(sq + to_f<ST>(b[g]));
  }
}

#define MOE_BY_DT(dt, MACRO)          \
  if ((dt) == DT_BF16) { MACRO(bf16_t) } \
  if ((dt) == DT_F16) { MACRO(f16_t) }   \
  if ((dt) == DT_F32) { MACRO(float) }

hipError_t launch_unpermute(const void* Y, const uint32_t* inv, const float* w, int T, int H,
                            int k, void* out, int dt, const void* shared_out,
                            const void* shared_logit, int shared_mode, hipStream_t st,
                            const void* res) {
#define MOE_UP(XT)                                                                            \
  hipLaunchKernelGGL((unpermute_kernel<XT>), dim3(T), dim3(256), 0, st, (const XT*)Y, inv, w, \
                     T, H, k, (XT*)out, (const XT*)shared_out, (const XT*)shared_logit,       \
                     shared_mode, (const XT*)res);                                            \
  return hipGetLastError();
  MOE_BY_DT(dt, MOE_UP)
#undef MOE_UP
  return hipErrorInvalidValue;
}

hipError_t launch_add_shared(void* y, const void* shared_out, const void* shared_logit,
                             int shared_mode, int T, int H, int dt, hipStream_t st,
                             const void* res) {
#define MOE_AS(XT)                                                                        \
  hipLaunchKernelGGL((add_shared_kernel<XT>), dim3(T), dim3(256), 0, st, (XT*)y,          \
                     (const XT*)shared_out, (const XT*)shared_logit, shared_mode, H,       \
                     (const XT*)res);                                                      \
  return hipGetLastError();
  MOE_BY_DT(dt, MOE_AS)
#undef MOE_AS
  return hipErrorInvalidValue;
}

hipError_t launch_add_rmsnorm(const void* a, const void* b, const void* w, float eps, int T,
                              int H, int dt, void* res, void* xn, hipStream_t st) {
  if (H % 8 != 0 || H > 256 * 8 * kNormChunks) return hipErrorInvalidValue;
#define MOE_AN(XT)                                                                          \
  hipLaunchKernelGGL((add_rmsnorm_kernel<XT>), dim3(T), dim3(256), 0, st, (const XT*)a,     \
                     (const XT*)b, (const XT*)w, eps, H, (XT*)res, (XT*)xn);                \
  return hipGetLastError();
  MOE_BY_DT(dt, MOE_AN)
#undef MOE_AN
  return hipErrorInvalidValue;
}

hipError_t launch_activation(const void* g, const void* u, void* out, int64_t n, int dt, int act,
                             float alpha, float limit, hipStream_t st) {
  const int64_t blocks64 = (n + 255) / 256;
  const int grid = (int)(blocks64 < 65536 ? blocks64 : 65536);
#define MOE_ACT(XT)                                                                          \
  hipLaunchKernelGGL((activation_kernel<XT>), dim3(grid), dim3(256), 0, st, (const XT*)g,   \
                     (const XT*)u, (XT*)out, n, act, alpha, limit);                         \
  return hipGetLastError();
  MOE_BY_DT(dt, MOE_ACT)
#undef MOE_ACT
  return hipErrorInvalidValue;
}

hipError_t launch_dequantize(const uint32_t* w, const void* s, const void* b, int sbdt, int bits,
                             int gs, int64_t numel, void* out, int odt, hipStream_t st) {
  const int64_t blocks64 = (numel + 255) / 256;
  const int grid = (int)(blocks64 < 65536 ? blocks64 : 65536);
#define MOE_DQ2(ST, OT)                                                                     \
  hipLaunchKernelGGL((dequantize_kernel<ST, OT>), dim3(grid), dim3(256), 0, st, w,         \
                     (const ST*)s, (const ST*)b, bits, gs, numel, (OT*)out);               \
  return hipGetLastError();
#define MOE_DQ(ST)                              \
  if (odt == DT_BF16) { MOE_DQ2(ST, bf16_t) }   \
  if (odt == DT_F16) { MOE_DQ2(ST, f16_t) }     \
  if (odt == DT_F32) { MOE_DQ2(ST, float) }
  MOE_BY_DT(sbdt, MOE_DQ)
#undef MOE_DQ
#undef MOE_DQ2
  return hipErrorInvalidValue;
}

}  // namespace moe
