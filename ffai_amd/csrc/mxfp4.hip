// mxfp4.hip — MXFP4 expert weights to mlx affine 4-bit on the GPU.
//
// GPT-OSS checkpoints ship their experts as MXFP4: 32 fp4 (e2m1) codes per
// group, packed 8 per u32 little-endian, and one e8m0 exponent byte per group
// (value = LUT[code] * 2^(e8m0 - 127)). The reference transcodes them on the
// CPU at load (Sources/FFAI/Models/Text/GPTOSSText.swift:1040-1236) into an
// affine grid fitted per group:
//   lo, hi  = min / max of LUT[code] over the group (scanned in code order;
//             LUT = 0, 0.5, 1, 1.5, 2, 3, 4, 6 for codes 0-7, negated for 8-15,
//             the mlx-lm gpt_oss table, GPTOSSText.swift:947-954)
//   bias    = lo * mx,  scale = (hi - lo) * mx / 15  (0 for a flat group)
//   q       = clamp(round((LUT[code] - lo) * (mx * (1 / scale))), 0, 15)
// stored as an mlx affine triplet with group size 32. Code i sits in the same
// nibble of the same word in both formats, so the weight words transcode in
// place. One thread per group: one 16-byte load, one exponent byte, an
// integer min/max over the 32 codes, the 16 possible levels computed once,
// then a nibble table lookup per code (17 bytes read and 16 + 2 *
// sizeof(scale) written per group).
#include "moe_common.hpp"
#include "moe_internal.hpp"

namespace moe {

// from_f with the sign of zero kept: the f32 -> f16 conversion as compiled
// here turns -0.0 into +0.0, and the reference stores a -0.0 bias for a
// group whose first minimal code is -0. The sign bit of a 16-bit result
// equals the f32 sign for every non-NaN value, so it is or-ed back in.
template <typename ST>
__device__ __forceinline__ ST from_f_signed(float v) {
  const ST r = from_f<ST>(v);
  if constexpr (sizeof(ST) == 2) {
    const uint16_t b = __builtin_bit_cast(uint16_t, r) | (uint16_t)((__float_as_uint(v) >> 16) & 0x8000u);
    return __builtin_bit_cast(ST, b);
  }
  return r;
}

// Twice the table value of a code: magnitudes 0, 1, 2, 3, 4, 6, 8, 12 held in
// the nibbles of one constant, the sign from bit 3 (code 8, -0.0, gives 0).
__device__ __forceinline__ int mxfp4_val2(uint32_t c) {
  const int mag = (int)((0xC8643210u >> (4u * (c & 7u))) & 15u);
  return (c & 8u) ? -mag : mag;
}

// 1 when the first code whose value is zero (low three bits zero: +0 or
// -0) is -0. Per word, ((w & 0x77777777) + 0x77777777) & 0x88888888 sets
// bit 3 of each nibble whose low three bits are non-zero (no carries cross
// nibbles); the complement marks the zero codes, the lowest one first.
__device__ __forceinline__ uint32_t first_zero_is_negative(const uint32_t (&w)[4]) {
#pragma unroll
  for (int k = 0; k < 4; k++) {
    const uint32_t z = ~(((w[k] & 0x77777777u) + 0x77777777u) & 0x88888888u) & 0x88888888u;
    if (z) return (w[k] >> __builtin_ctz(z)) & 1u;
  }
  return 0u;
}

template <typename ST>
__global__ __launch_bounds__(256) void mxfp4_affine_kernel(const uint32_t* __restrict__ packed,
                                                           const uint8_t* __restrict__ e8m0,
                                                           int64_t groups,
                                                           uint32_t* __restrict__ out_w,
                                                           ST* __restrict__ out_s,
                                                           ST* __restrict__ out_b) {
#pragma clang fp contract(off)
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
       g += (int64_t)gridDim.x * blockDim.x) {
    const uint4 wv = reinterpret_cast<const uint4*>(packed)[g];
    const uint32_t words[4] = {wv.x, wv.y, wv.z, wv.w};
    // 2^(e - 127) exactly, subnormals included (e = 0 gives 2^-127)
    const int e = (int)e8m0[g];
    const float mx = __builtin_ldexpf(1.0f, e - 127);
    // pass 1: min / max over the group, in integers (twice the values)
    int lo2 = 1 << 30, hi2 = -(1 << 30);
#pragma unroll
    for (int i = 0; i < 32; i++) {
      const int v = mxfp4_val2((words[i >> 3] >> (4 * (i & 7))) & 15u);
      lo2 = min(lo2, v);
      hi2 = max(hi2, v);
    }
    // the reference's scan keeps the first of equal minima: a zero minimum
    // carries the sign of the first zero code (the maximum's sign never
    // reaches a result)
    float lo = 0.5f * (float)lo2;
    if (lo2 == 0 && first_zero_is_negative(words)) lo = -0.0f;
    const float hi = 0.5f * (float)hi2;
    const float bias = lo * mx;
    const float span = (hi - lo) * mx;
    const float scale = span > 0.0f ? span / 15.0f : 0.0f;
    const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
    const float cs = mx * inv;
    // the affine level of each of the 16 codes, as the reference computes it
    // per code: round((value - lo) * cs), clamped; 4 bits each in a u64
    uint64_t lvl = 0;
#pragma unroll
    for (int c = 0; c < 16; c++) {
      float q = roundf((0.5f * (float)mxfp4_val2((uint32_t)c) - lo) * cs);
      q = fminf(fmaxf(q, 0.0f), 15.0f);
      lvl |= (uint64_t)(uint32_t)q << (4 * c);
    }
    // pass 2: every code through the table, nibble for nibble
    uint32_t ow[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
      uint32_t o = 0;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const uint32_t c = (words[k] >> (4 * j)) & 15u;
        o |= (uint32_t)((lvl >> (4u * c)) & 15u) << (4 * j);
      }
      ow[k] = o;
    }
    reinterpret_cast<uint4*>(out_w)[g] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
    out_s[g] = from_f_signed<ST>(scale);
    out_b[g] = from_f_signed<ST>(bias);
  }
}

// dst[i] = src[i] converted between float types (per-row expert biases).
template <typename S, typename D>
__global__ __launch_bounds__(256) void convert_kernel(const S* __restrict__ src, D* __restrict__ dst,
                                                      int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    dst[i] = from_f<D>(to_f<S>(src[i]));
}

hipError_t launch_mxfp4_affine(const uint32_t* packed, const uint8_t* e8m0, int64_t groups,
                               uint32_t* out_w, void* out_s, void* out_b, int sbdt,
                               hipStream_t st) {
  const int64_t blocks = (groups + 255) / 256;
  const int grid = (int)(blocks < 65536 ? blocks : 65536);
#define MOE_MX(ST)                                                                        \
  hipLaunchKernelGGL((mxfp4_affine_kernel<ST>), dim3(grid), dim3(256), 0, st, packed, e8m0, \
                     groups, out_w, (ST*)out_s, (ST*)out_b);                               \
  return hipGetLastError();
  if (sbdt == DT_BF16) { MOE_MX(bf16_t) }
  if (sbdt == DT_F16) { MOE_MX(f16_t) }
  if (sbdt == DT_F32) { MOE_MX(float) }
#undef MOE_MX
  return hipErrorInvalidValue;
}

hipError_t launch_convert(const void* src, int sdt, void* dst, int ddt, int64_t n,
                          hipStream_t st) {
  const int64_t blocks = (n + 255) / 256;
  const int grid = (int)(blocks < 65536 ? blocks : 65536);
#define MOE_CV2(S, D)                                                                       \
  hipLaunchKernelGGL((convert_kernel<S, D>), dim3(grid), dim3(256), 0, st, (const S*)src,   \
                     (D*)dst, n);                                                           \
  return hipGetLastError();
#define MOE_CV(S)                              \
  if (ddt == DT_BF16) { MOE_CV2(S, bf16_t) }   \
  if (ddt == DT_F16) { MOE_CV2(S, f16_t) }     \
  if (ddt == DT_F32) { MOE_CV2(S, float) }
  if (sdt == DT_BF16) { MOE_CV(bf16_t) }
  if (sdt == DT_F16) { MOE_CV(f16_t) }
  if (sdt == DT_F32) { MOE_CV(float) }
#undef MOE_CV
#undef MOE_CV2
  return hipErrorInvalidValue;
}

}  // namespace moe
