// gemv.hip — decode-side grouped dequant GEMV for gfx950.
//
// Replaces FFAI's expert GEMVs on the decode path:
//   Ops.dequantGemvInt4ExpertIndexed(Many)  Sources/FFAI/Ops/Ops.swift:2444-2587
//   MoELayer.swiGLU / batchedSwiGLU         Sources/FFAI/Models/MoELayer.swift:992-1155
//   Ops.moeDownSwigluAccumInt4Chain8        Sources/FFAI/Ops/OpsFused.swift:545-697
// generalised to 2/3/4/5/6/8-bit mlx affine weights, any stacked expert count
// and an activation dtype independent of the scale dtype.
//
// The work is HBM-bound: every packed weight byte is read once. A lane reads
// whole 32-value units (bits x 4 bytes, contiguous across the lanes of a row),
// unpacks them to code pairs in registers and multiplies with v_dot2_f32_bf16
// (or _f16) against activations kept in the same pair order. The affine
// bias is folded in per unit: sum((s q + b) x) = s * D + (b - MAGIC s) * sum(x)
// with D = sum((MAGIC + q) x).
//
// Lane layout: a wave is split into 64/L sub-groups of L lanes; a sub-group
// owns one output row and its lanes stride over the row's K/32 units; a
// shuffle reduction over L lanes finishes the row.
#include "moe_common.hpp"
#include "moe_internal.hpp"

#ifndef MOE_BITS
#define MOE_BITS 4
#endif

namespace moe {

constexpr int kUMax = 8;  // units per lane (host picks L so ceil(K/32/L) <= 8)

// ---------------------------------------------------------------------------
// activation loads in pair order
// ---------------------------------------------------------------------------

// 16-bit activations: 32 values = 16 natural u32 words -> 16 pair words.
template <int BITS>
__device__ __forceinline__ void natural_to_pairs(const uint32_t (&n)[16], uint32_t (&x16)[16]) {
  constexpr int P = Pairing<BITS>::P, H = P / 2;
#pragma unroll
  for (int q = 0; q < 16; q++) {
    const int b = (2 * q) / P, i = q % H;
    const int va = b * P + i, vb = va + H;
    const uint32_t lo = (n[va >> 1] >> ((va & 1) * 16)) & 0xFFFFu;
    const uint32_t hi = (n[vb >> 1] >> ((vb & 1) * 16)) & 0xFFFFu;
    x16[q] = lo | (hi << 16);
  }
}

__device__ __forceinline__ float sum16(const uint32_t (&n)[16], bool bf16) {
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; j++) {
    float lo, hi;
    if (bf16) {
      lo = __uint_as_float(n[j] << 16);
      hi = __uint_as_float(n[j] & 0xFFFF0000u);
    } else {
      lo = (float)__builtin_bit_cast(f16_t, (uint16_t)(n[j] & 0xFFFFu));
      hi = (float)__builtin_bit_cast(f16_t, (uint16_t)(n[j] >> 16));
    }
    s += lo + hi;
  }
  return s;
}

// One unit's activations, pair order, for either storage class.
template <typename XT> struct XUnit;
template <> struct XUnit<bf16_t> { uint32_t v[16]; };
template <> struct XUnit<f16_t> { uint32_t v[16]; };
template <> struct XUnit<float> { float v[32]; };

template <int BITS, typename XT>
__device__ __forceinline__ float dot_unit(const uint32_t (&cp)[16], const XUnit<XT>& x) {
  if constexpr (__is_same(XT, float)) return unit_dot32(cp, x.v);
  else return unit_dot16<BITS, XT>(cp, x.v);
}

// Loads unit u of an activation row straight from global memory into pair
// order and returns its sum.
template <int BITS, typename XT>
__device__ __forceinline__ float load_x_unit(const XT* __restrict__ row, int u, XUnit<XT>& x) {
  if constexpr (__is_same(XT, float)) {
    const float4* p = reinterpret_cast<const float4*>(row + u * 32);
    float n[32];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      float4 v = p[j];
      n[4 * j] = v.x; n[4 * j + 1] = v.y; n[4 * j + 2] = v.z; n[4 * j + 3] = v.w;
    }
    float s = 0.f;
#pragma unroll
    for (int v = 0; v < 32; v++) {
      x.v[pair_pos<BITS>(v)] = n[v];
      s += n[v];
    }
    return s;
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(row + u * 32);
    uint32_t n[16];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint4 v = p[j];
      n[4 * j] = v.x; n[4 * j + 1] = v.y; n[4 * j + 2] = v.z; n[4 * j + 3] = v.w;
    }
    natural_to_pairs<BITS>(n, x.v);
    return sum16(n, __is_same(XT, bf16_t));
  }
}

// Reads unit u of a staged (already pair-ordered) LDS row.
template <typename XT>
__device__ __forceinline__ void lds_x_unit(const XT* row, int u, XUnit<XT>& x) {
  if constexpr (__is_same(XT, float)) {
    const float4* p = reinterpret_cast<const float4*>(row + u * 32);
#pragma unroll
    for (int j = 0; j < 8; j++) {
      float4 v = p[j];
      x.v[4 * j] = v.x; x.v[4 * j + 1] = v.y; x.v[4 * j + 2] = v.z; x.v[4 * j + 3] = v.w;
    }
  } else {
    const uint4* p = reinterpret_cast<const uint4*>(row + u * 32);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint4 v = p[j];
      x.v[4 * j] = v.x; x.v[4 * j + 1] = v.y; x.v[4 * j + 2] = v.z; x.v[4 * j + 3] = v.w;
    }
  }
}

// One weight unit with its group scale and folded bias.
template <int BITS> struct WUnit {
  uint32_t w[BITS];
  float s, b;
};

template <int BITS, typename ST>
__device__ __forceinline__ void load_w_unit(const GemvProj& p, size_t row, int row_words, int groups,
                                            int gs, int u, WUnit<BITS>& wu) {
  load_unit<BITS>(p.w + row * row_words + u * BITS, wu.w);
  const size_t gi = row * groups + (u * 32) / gs;
  wu.s = ld_sb<ST>(p.s, gi);
  wu.b = ld_sb<ST>(p.b, gi);
}

template <typename XT>
__device__ __forceinline__ float finish_proj(float acc, const void* ob, size_t obi) {
  float v = round_to<XT>(acc);
  if (ob) v = round_to<XT>(v + to_f<XT>(reinterpret_cast<const XT*>(ob)[obi]));
  return v;
}

// ---------------------------------------------------------------------------
// grouped GEMV, activations staged in LDS (any number of rows per expert)
// ---------------------------------------------------------------------------

template <int BITS, typename XT>
__device__ void stage_rows(const XT* __restrict__ x, const uint32_t* __restrict__ perm, int topk,
                           uint32_t p_first, int nt, int K, XT* xs, float* xsum) {
  const int tid = threadIdx.x, nthr = blockDim.x;
  const int total = nt * K;
  for (int i = tid; i < total; i += nthr) {
    const int t = i / K, c = i - t * K;
    const uint32_t p = p_first + (uint32_t)t;
    const uint32_t row = perm ? perm[p] / (uint32_t)topk : p;
    xs[t * K + (c & ~31) + pair_pos<BITS>(c & 31)] = x[(size_t)row * K + c];
  }
  __syncthreads();
  const int CU = K >> 5;
  for (int i = tid; i < nt * CU; i += nthr) {
    const XT* src = xs + i * 32;
    float s = 0.f;
    for (int j = 0; j < 32; j++) s += to_f<XT>(src[j]);
    xsum[i] = s;
  }
  __syncthreads();
}

template <int BITS, typename XT, typename ST, bool GATEUP, int TOKMAX>
__global__ __launch_bounds__(256) void gemv_grouped_kernel(const GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int slot = blockIdx.x / a.row_blocks, rb = blockIdx.x - slot * a.row_blocks;
  if ((uint32_t)slot >= a.used[0]) return;
  const uint32_t e = a.used[1 + slot];
  const uint32_t pbeg = a.offsets[e], pend = a.offsets[e + 1];
  const int N = a.N, K = a.K, CU = K >> 5, groups = K / a.gs, row_words = CU * BITS;
  const int r_begin = rb * a.rows_per_block;
  const int r_end = min(N, r_begin + a.rows_per_block);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int L = 1 << a.lg, SG = 64 >> a.lg;
  const int sg = lane >> a.lg, li = lane & (L - 1);
  XT* xs = reinterpret_cast<XT*>(smem);
  float* xsum = reinterpret_cast<float*>(smem + (size_t)a.tok_chunk * K * sizeof(XT));
  const XT* x = reinterpret_cast<const XT*>(a.x);
  XT* out = reinterpret_cast<XT*>(a.out);
  constexpr float MAGIC = Magic<BITS, XT>::value;
  const size_t ebase = (size_t)e * N;

  for (uint32_t pc = pbeg; pc < pend; pc += (uint32_t)a.tok_chunk) {
    const int nt = min((int)(pend - pc), a.tok_chunk);
    __syncthreads();
    stage_rows<BITS, XT>(x, a.perm, a.topk, pc, nt, K, xs, xsum);
    for (int r0 = r_begin + wave * SG; r0 < r_end; r0 += nwaves * SG) {
      const int r = r0 + sg;
      if (r >= r_end) continue;
      const size_t row = ebase + (size_t)r;
      float acc0[TOKMAX], acc1[TOKMAX];
#pragma unroll
      for (int t = 0; t < TOKMAX; t++) acc0[t] = acc1[t] = 0.f;
      WUnit<BITS> w0[kUMax], w1[kUMax];
#pragma unroll
      for (int j = 0; j < kUMax; j++) {
        const int u = li + j * L;
        if (u < CU) {
          load_w_unit<BITS, ST>(a.p0, row, row_words, groups, a.gs, u, w0[j]);
          if constexpr (GATEUP) load_w_unit<BITS, ST>(a.p1, row, row_words, groups, a.gs, u, w1[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < kUMax; j++) {
        const int u = li + j * L;
        if (u < CU) {
          uint32_t cp0[16], cp1[16];
          unpack_pairs<BITS>(w0[j].w, cp0);
          const float bb0 = w0[j].b - MAGIC * w0[j].s;
          float bb1 = 0.f;
          if constexpr (GATEUP) {
            unpack_pairs<BITS>(w1[j].w, cp1);
            bb1 = w1[j].b - MAGIC * w1[j].s;
          }
#pragma unroll
          for (int t = 0; t < TOKMAX; t++) {
            if (t < nt) {
              XUnit<XT> xu;
              lds_x_unit<XT>(xs + t * K, u, xu);
              const float xsu = xsum[t * CU + u];
              acc0[t] += w0[j].s * dot_unit<BITS, XT>(cp0, xu) + bb0 * xsu;
              if constexpr (GATEUP) acc1[t] += w1[j].s * dot_unit<BITS, XT>(cp1, xu) + bb1 * xsu;
            }
          }
        }
      }
#pragma unroll
      for (int t = 0; t < TOKMAX; t++) {
        if (t < nt) {
          acc0[t] = wave_sum_width(acc0[t], L);
          if constexpr (GATEUP) acc1[t] = wave_sum_width(acc1[t], L);
        }
      }
      if (li == 0) {
#pragma unroll
        for (int t = 0; t < TOKMAX; t++) {
          if (t < nt) {
            const size_t o = (size_t)(pc + t) * N + r;
            const float g = finish_proj<XT>(acc0[t], a.p0.ob, row);
            if constexpr (GATEUP) {
              const float u = finish_proj<XT>(acc1[t], a.p1.ob, row);
              out[o] = from_f<XT>(apply_act(g, u, a.act, a.alpha, a.limit));
            } else {
              out[o] = from_f<XT>(g);
            }
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// one activation row per expert (decode T = 1): activations live in registers
// for the lifetime of the wave, no LDS, no barrier.
// ---------------------------------------------------------------------------

template <int BITS, typename XT, typename ST, bool GATEUP>
__global__ __launch_bounds__(256) void gemv_single_kernel(const GemvArgs a) {
  const int slot = blockIdx.x / a.row_blocks, rb = blockIdx.x - slot * a.row_blocks;
  if ((uint32_t)slot >= a.used[0]) return;
  const uint32_t e = a.used[1 + slot];
  const uint32_t p = a.offsets[e];
  if (a.offsets[e + 1] == p) return;
  const int N = a.N, K = a.K, CU = K >> 5, groups = K / a.gs, row_words = CU * BITS;
  const int r_begin = rb * a.rows_per_block;
  const int r_end = min(N, r_begin + a.rows_per_block);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int L = 1 << a.lg, SG = 64 >> a.lg;
  const int sg = lane >> a.lg, li = lane & (L - 1);
  constexpr float MAGIC = Magic<BITS, XT>::value;
  constexpr int UR = 4;  // host guarantees ceil(CU / L) <= 4 for this kernel
  const uint32_t xrow = a.perm ? a.perm[p] / (uint32_t)a.topk : p;
  const XT* x = reinterpret_cast<const XT*>(a.x) + (size_t)xrow * K;
  XT* out = reinterpret_cast<XT*>(a.out);
  const size_t ebase = (size_t)e * N;

  XUnit<XT> xu[UR];
  float xs[UR];
#pragma unroll
  for (int j = 0; j < UR; j++) {
    const int u = li + j * L;
    xs[j] = 0.f;
    if (u < CU) xs[j] = load_x_unit<BITS, XT>(x, u, xu[j]);
  }
  for (int r0 = r_begin + wave * SG; r0 < r_end; r0 += nwaves * SG) {
    const int r = r0 + sg;
    if (r >= r_end) continue;
    const size_t row = ebase + (size_t)r;
    WUnit<BITS> w0[UR], w1[UR];
#pragma unroll
    for (int j = 0; j < UR; j++) {
      const int u = li + j * L;
      if (u < CU) {
        load_w_unit<BITS, ST>(a.p0, row, row_words, groups, a.gs, u, w0[j]);
        if constexpr (GATEUP) load_w_unit<BITS, ST>(a.p1, row, row_words, groups, a.gs, u, w1[j]);
      }
    }
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int j = 0; j < UR; j++) {
      const int u = li + j * L;
      if (u < CU) {
        uint32_t cp[16];
        unpack_pairs<BITS>(w0[j].w, cp);
        acc0 += w0[j].s * dot_unit<BITS, XT>(cp, xu[j]) + (w0[j].b - MAGIC * w0[j].s) * xs[j];
        if constexpr (GATEUP) {
          unpack_pairs<BITS>(w1[j].w, cp);
          acc1 += w1[j].s * dot_unit<BITS, XT>(cp, xu[j]) + (w1[j].b - MAGIC * w1[j].s) * xs[j];
        }
      }
    }
    acc0 = wave_sum_width(acc0, L);
    if constexpr (GATEUP) acc1 = wave_sum_width(acc1, L);
    if (li == 0) {
      const size_t o = (size_t)p * N + r;
      const float g = finish_proj<XT>(acc0, a.p0.ob, row);
      if constexpr (GATEUP) {
        const float u = finish_proj<XT>(acc1, a.p1.ob, row);
        out[o] = from_f<XT>(apply_act(g, u, a.act, a.alpha, a.limit));
      } else {
        out[o] = from_f<XT>(g);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// fused down projection + weighted combine, one token
//   out[r] = round( sum_p round(w_p) * (W_down[e_p] . act_p)[r] )
// Sub-group g handles sorted positions g, g + 64/L, ...; a full-wave
// reduction adds the slots. Activations live in registers.
// ---------------------------------------------------------------------------

template <int BITS, typename XT, typename ST>
__global__ __launch_bounds__(256) void down_combine_kernel(const DownCombineArgs a) {
  const int N = a.N, K = a.K, CU = K >> 5, groups = K / a.gs, row_words = CU * BITS;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int L = 1 << a.lg, SG = 64 >> a.lg;
  const int sg = lane >> a.lg, li = lane & (L - 1);
  constexpr float MAGIC = Magic<BITS, XT>::value;
  constexpr int UR = 4;   // units per lane
  constexpr int PR = 2;   // positions per sub-group (host: k <= 2 * 64/L)
  const int r_begin = blockIdx.x * a.rows_per_block;
  const int r_end = min(N, r_begin + a.rows_per_block);
  XT* out = reinterpret_cast<XT*>(a.out);

  XUnit<XT> xu[PR][UR];
  float xs[PR][UR], wsl[PR];
  uint32_t ex[PR];
#pragma unroll
  for (int q = 0; q < PR; q++) {
    const int p = sg + q * SG;
    wsl[q] = 0.f;
    ex[q] = 0;
    if (p < a.k) {
      const uint32_t src = a.perm[p];
      ex[q] = a.idx[src];
      wsl[q] = round_to<XT>(a.w[src]);
      const XT* row = reinterpret_cast<const XT*>(a.act) + (size_t)p * K;
#pragma unroll
      for (int j = 0; j < UR; j++) {
        const int u = li + j * L;
        xs[q][j] = 0.f;
        if (u < CU) xs[q][j] = load_x_unit<BITS, XT>(row, u, xu[q][j]);
      }
    }
  }
  for (int r = r_begin + wave; r < r_end; r += nwaves) {
    WUnit<BITS> wu[PR][UR];
#pragma unroll
    for (int q = 0; q < PR; q++) {
      const int p = sg + q * SG;
      if (p < a.k) {
        const size_t row = (size_t)ex[q] * N + r;
#pragma unroll
        for (int j = 0; j < UR; j++) {
          const int u = li + j * L;
          if (u < CU) load_w_unit<BITS, ST>(a.p, row, row_words, groups, a.gs, u, wu[q][j]);
        }
      }
    }
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < PR; q++) {
      const int p = sg + q * SG;
      float part = 0.f;
      if (p < a.k) {
#pragma unroll
        for (int j = 0; j < UR; j++) {
          const int u = li + j * L;
          if (u < CU) {
            uint32_t cp[16];
            unpack_pairs<BITS>(wu[q][j].w, cp);
            part += wu[q][j].s * dot_unit<BITS, XT>(cp, xu[q][j]) +
                    (wu[q][j].b - MAGIC * wu[q][j].s) * xs[q][j];
          }
        }
      }
      // the expert's down output is rounded to the activation dtype before
      // it is weighted, as the unfused path stores it (MoELayer.swift:895-939)
      part = wave_sum_width(part, L);
      if (p < a.k && li == 0) {
        const float yv = finish_proj<XT>(part, a.p.ob, (size_t)ex[q] * N + r);
        acc += wsl[q] * yv;
      }
    }
    acc = wave_sum_width(acc, 64);
    if (lane == 0) out[r] = from_f<XT>(acc);
  }
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

template <int BITS, typename XT, typename ST>
static hipError_t launch_gemv_t(bool gateup, int tokmax, const GemvArgs& a, int grid,
                                hipStream_t st) {
  if (tokmax <= 1) {
    if (gateup)
      hipLaunchKernelGGL((gemv_single_kernel<BITS, XT, ST, true>), dim3(grid), dim3(256), 0, st, a);
    else
      hipLaunchKernelGGL((gemv_single_kernel<BITS, XT, ST, false>), dim3(grid), dim3(256), 0, st, a);
  } else {
    const size_t smem = gemv_smem_bytes(__is_same(XT, float) ? DT_F32 : DT_BF16, a.K, a.tok_chunk);
    if (gateup)
      hipLaunchKernelGGL((gemv_grouped_kernel<BITS, XT, ST, true, 8>), dim3(grid), dim3(256), smem,
                         st, a);
    else
      hipLaunchKernelGGL((gemv_grouped_kernel<BITS, XT, ST, false, 8>), dim3(grid), dim3(256), smem,
                         st, a);
  }
  return hipGetLastError();
}

template <int BITS>
static hipError_t launch_gemv_bits(int xdt, int sbdt, bool gateup, int tokmax, const GemvArgs& a,
                                   int grid, hipStream_t st) {
  if (xdt == DT_BF16 && sbdt == DT_BF16) return launch_gemv_t<BITS, bf16_t, bf16_t>(gateup, tokmax, a, grid, st);
  if (xdt == DT_BF16 && sbdt == DT_F16) return launch_gemv_t<BITS, bf16_t, f16_t>(gateup, tokmax, a, grid, st);
  if (xdt == DT_F16 && sbdt == DT_F16) return launch_gemv_t<BITS, f16_t, f16_t>(gateup, tokmax, a, grid, st);
  if (xdt == DT_F16 && sbdt == DT_BF16) return launch_gemv_t<BITS, f16_t, bf16_t>(gateup, tokmax, a, grid, st);
  if (xdt == DT_F32 && sbdt == DT_F32) return launch_gemv_t<BITS, float, float>(gateup, tokmax, a, grid, st);
  return hipErrorInvalidValue;
}

template <int BITS>
static hipError_t launch_down_combine_bits(int xdt, int sbdt, const DownCombineArgs& a, int grid,
                                           hipStream_t st) {
#define MOE_DC(XT, ST)                                                                         \
  hipLaunchKernelGGL((down_combine_kernel<BITS, XT, ST>), dim3(grid), dim3(256), 0, st, a); \
  return hipGetLastError();
  if (xdt == DT_BF16 && sbdt == DT_BF16) { MOE_DC(bf16_t, bf16_t) }
  if (xdt == DT_BF16 && sbdt == DT_F16) { MOE_DC(bf16_t, f16_t) }
  if (xdt == DT_F16 && sbdt == DT_F16) { MOE_DC(f16_t, f16_t) }
  if (xdt == DT_F16 && sbdt == DT_BF16) { MOE_DC(f16_t, bf16_t) }
  if (xdt == DT_F32 && sbdt == DT_F32) { MOE_DC(float, float) }
#undef MOE_DC
  return hipErrorInvalidValue;
}

// One translation unit per bit width (MOE_BITS) keeps compile times short;
// the per-width entry points are stitched together in api.cpp.
#define MOE_CAT2(a, b) a##b
#define MOE_CAT(a, b) MOE_CAT2(a, b)

hipError_t MOE_CAT(launch_gemv_b, MOE_BITS)(int xdt, int sbdt, bool gateup, int tokmax,
                                             const GemvArgs& a, int grid, hipStream_t st) {
  return launch_gemv_bits<MOE_BITS>(xdt, sbdt, gateup, tokmax, a, grid, st);
}

hipError_t MOE_CAT(launch_down_combine_b, MOE_BITS)(int xdt, int sbdt, const DownCombineArgs& a,
                                                     int grid, hipStream_t st) {
  return launch_down_combine_bits<MOE_BITS>(xdt, sbdt, a, grid, st);
}

}  // namespace moe
