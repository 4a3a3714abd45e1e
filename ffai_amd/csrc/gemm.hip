// gemm.hip — prefill-side grouped dequant GEMM on the gfx950 matrix cores.
//
// Replaces Ops.moeGatherDequantGemmInt4 bm8/bm16/bm64/m1
// (Sources/FFAI/Ops/Ops.swift:4553-5201, 6499-6585) with the tile choice of
// MoELayer.swift:855-882, generalised to 2/3/4/5/6/8-bit weights, any
// group size in {32, 64, 128} and scale dtypes independent of the
// activation dtype:
//   gate/up:  act[p, n] = act_fn(round(Wg[e(p)][n] . x[row(p)]),
//                                round(Wu[e(p)][n] . x[row(p)]))
//   single:   out[p, n] = round(W[e(p)][n] . a[p])
// over the expert-sorted positions p of a dispatch plan.
//
// Work: a tile list of (expert, 128 consecutive sorted positions); block =
// one tile x one column slice. The block stages the tile's 128 activation
// rows, 64 values at a time, in LDS (padded rows, double-buffered); every
// wave owns 32 output columns for one or two weight matrices and all 128
// rows (4 x v_mfma_f32_32x32x16 tiles per matrix). A wave dequantises its
// weight fragments straight from HBM into the MFMA B-operand registers, so
// each weight value is converted exactly once per tile and no LDS traffic is
// spent on weights: codes -> fp32 (exact) -> s*q + b (fp32) -> bf16 / f16.
//
// K order inside a 64-value chunk: lane half h of the wave takes values
// [32h, 32h + 32) — one whole 32-value unit, a single contiguous load — and
// step s (0..3) of the 16-deep MFMA reduction feeds values 32h + 8s + e,
// e < 8; the A fragments are read from LDS in the same order.
#include <hip/hip_ext.h>

#include "moe_common.hpp"
#include "moe_internal.hpp"

#ifndef MOE_BITS
#define MOE_BITS 4
#endif

namespace moe {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

struct ProjViewG {
  rsrc_t w, s, b;
};

constexpr int kGBM = kGemmRows;  // rows per tile
constexpr int kGBK = 64;       // values per K chunk
constexpr int kGAS = 72;       // LDS row stride in elements (64 + 8: conflict-free b128 reads)

template <typename XT> struct MfmaOp;
template <> struct MfmaOp<bf16_t> {
  typedef bf16x8_t V;
  static __device__ __forceinline__ f32x16_t mma(V a, V b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct MfmaOp<f16_t> {
  typedef f16x8_t V;
  static __device__ __forceinline__ f32x16_t mma(V a, V b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// Code e (0..7) of step s (0..3) of a 32-value unit, as an exact float.
template <int BITS>
__device__ __forceinline__ float unit_code(const uint32_t (&w)[BITS], int s, int e) {
  const int bit = (8 * s + e) * BITS;
  const int lo = bit >> 5, sh = bit & 31;
  uint32_t v = w[lo] >> sh;
  if (sh + BITS > 32) v |= w[lo + 1] << (32 - sh);
  return (float)(v & ((1u << BITS) - 1u));
}

// Eight dequantised weights of step s: w = s * q + b rounded to the MFMA
// operand type. 4-bit codes are split into byte lanes first so every code
// converts with one v_cvt_f32_ubyte.
template <int BITS, typename XT>
__device__ __forceinline__ typename MfmaOp<XT>::V dequant8(const uint32_t (&w)[BITS], int s,
                                                          float sc, float bi) {
  float q[8];
  if constexpr (BITS == 4) {
    const uint32_t lo = w[s] & 0x0F0F0F0Fu, hi = (w[s] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      q[2 * j] = (float)((lo >> (8 * j)) & 0xFFu);
      q[2 * j + 1] = (float)((hi >> (8 * j)) & 0xFFu);
    }
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int e = 0; e < 8; e++) q[e] = (float)((w[2 * s + (e >> 2)] >> (8 * (e & 3))) & 0xFFu);
  } else {
#pragma unroll
    for (int e = 0; e < 8; e++) q[e] = unit_code<BITS>(w, s, e);
  }
  typename MfmaOp<XT>::V r;
#pragma unroll
  for (int e = 0; e < 8; e++) r[e] = from_f<XT>(__builtin_fmaf(sc, q[e], bi));
  return r;
}

// One weight matrix slice held by a lane for one K chunk.
template <int BITS, typename ST> struct BFrag {
  uint32_t w[BITS];
  ST s, b;
};

template <int BITS, typename ST>
__device__ __forceinline__ void load_bfrag(const ProjViewG& v, uint32_t row, int row_words,
                                           int groups, int chunk, int h, int gsh,
                                           BFrag<BITS, ST>& f) {
  const int unit = 2 * chunk + h;  // 32-value unit index within the row
  bload_unit<BITS>(v.w, (row * (uint32_t)row_words + (uint32_t)(unit * BITS)) * 4u, f.w);
  const uint32_t gi = row * (uint32_t)groups + (uint32_t)(unit >> gsh);
  f.s = __builtin_bit_cast(ST, bload16(v.s, gi * (uint32_t)sizeof(ST)));
  f.b = __builtin_bit_cast(ST, bload16(v.b, gi * (uint32_t)sizeof(ST)));
}

template <int BITS, typename ST>
__device__ __forceinline__ ProjViewG proj_view_g(const GemvProj& p, uint32_t e, int N,
                                                 int row_words, int groups) {
  const size_t rows = (size_t)e * (size_t)N;
  ProjViewG v;
  v.w = make_rsrc(p.w + rows * row_words, (uint32_t)N * (uint32_t)row_words * 4u);
  v.s = make_rsrc(reinterpret_cast<const ST*>(p.s) + rows * groups,
                  (uint32_t)N * (uint32_t)groups * (uint32_t)sizeof(ST));
  v.b = make_rsrc(reinterpret_cast<const ST*>(p.b) + rows * groups,
                  (uint32_t)N * (uint32_t)groups * (uint32_t)sizeof(ST));
  return v;
}

// GATEUP: matrix 0 = gate, matrix 1 = up, both for columns n0 + lane%32
// (the activation is applied in the epilogue, output [M, N]); otherwise
// one matrix with two 32-column sets n0 + lane%32 and n0 + 32 + lane%32.
template <int BITS, typename XT, typename ST, bool GATEUP>
__global__ __launch_bounds__(256) void gemm_grouped_kernel(const GemmArgs a) {
  __shared__ __align__(16) XT As[2][kGBM * kGAS];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nb_cols = GATEUP ? 128 : 256;  // output columns per block
  const int n_tiles = (a.N + nb_cols - 1) / nb_cols;

  // blocks b, b + 8, b + 16, ... share an XCD (and its L2): give them
  // consecutive work items, column slices of one row tile first
  const uint32_t per = gridDim.x >> 3;
  const uint32_t wi = (blockIdx.x & 7u) * per + (blockIdx.x >> 3);
  const uint32_t ntile = a.tiles[0];
  if (wi >= ntile * (uint32_t)n_tiles) return;
  const uint32_t tile = wi / (uint32_t)n_tiles;
  const int bn = (int)(wi - tile * (uint32_t)n_tiles);
  // tile fields are block-uniform; readfirstlane keeps the buffer resources
  // built from them scalar
  const uint32_t e = __builtin_amdgcn_readfirstlane(a.tiles[1 + 2 * tile]);
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(a.tiles[2 + 2 * tile]);
  const uint32_t pend = __builtin_amdgcn_readfirstlane(a.offsets[e + 1]);

  const int N = a.N, K = a.K, CU = K >> 5, groups = CU >> a.gsh, row_words = CU * BITS;
  const int nchunks = K / kGBK;
  const int col = lane & 31, h = lane >> 5;
  const int n0 = bn * nb_cols + wave * (GATEUP ? 32 : 64);
  // B rows of the two column sets (clamped: columns past N compute garbage
  // that is never stored)
  const uint32_t r0 = (uint32_t)min(n0 + col, N - 1);
  const uint32_t r1 = GATEUP ? r0 : (uint32_t)min(n0 + 32 + col, N - 1);
  const ProjViewG P0 = proj_view_g<BITS, ST>(a.p0, e, N, row_words, groups);
  const ProjViewG P1 = GATEUP ? proj_view_g<BITS, ST>(a.p1, e, N, row_words, groups) : P0;

  // A staging: thread t copies row t/2, values [32 (t%2), +32) of a chunk
  const int arow = threadIdx.x >> 1, ahalf = threadIdx.x & 1;
  const uint32_t ap = min(m0 + (uint32_t)arow, pend - 1);
  const uint32_t xrow = a.perm ? a.perm[ap] / (uint32_t)a.topk : ap;
  // rows differ per lane, so these are plain global loads (a buffer
  // resource must be wave-uniform)
  const u32x4_t* xsrc = reinterpret_cast<const u32x4_t*>(reinterpret_cast<const XT*>(a.x) +
                                                         (size_t)xrow * K + 32 * ahalf);
  auto load_a = [&](int c, u32x4_t (&v)[4]) {
#pragma unroll
    for (int j = 0; j < 4; j++) v[j] = xsrc[c * (kGBK * (int)sizeof(XT) / 16) + j];
  };
  auto store_a = [&](int buf, const u32x4_t (&v)[4]) {
    u32x4_t* dst = reinterpret_cast<u32x4_t*>(&As[buf][arow * kGAS + 32 * ahalf]);
#pragma unroll
    for (int j = 0; j < 4; j++) dst[j] = v[j];
  };

  f32x16_t acc0[4], acc1[4];
#pragma unroll
  for (int t = 0; t < 4; t++) {
    acc0[t] = f32x16_t{};
    acc1[t] = f32x16_t{};
  }

  BFrag<BITS, ST> f0, f1, g0, g1;
  u32x4_t av[4];
  load_a(0, av);
  load_bfrag<BITS, ST>(P0, r0, row_words, groups, 0, h, a.gsh, f0);
  load_bfrag<BITS, ST>(P1, r1, row_words, groups, 0, h, a.gsh, f1);
  store_a(0, av);
  __syncthreads();

  typedef typename MfmaOp<XT>::V V;
  for (int c = 0; c < nchunks; c++) {
    const int buf = c & 1;
    const bool more = c + 1 < nchunks;
    if (more) {
      load_a(c + 1, av);
      load_bfrag<BITS, ST>(P0, r0, row_words, groups, c + 1, h, a.gsh, g0);
      load_bfrag<BITS, ST>(P1, r1, row_words, groups, c + 1, h, a.gsh, g1);
    }
    const float s0 = to_f<ST>(f0.s), b0 = to_f<ST>(f0.b);
    const float s1 = to_f<ST>(f1.s), b1 = to_f<ST>(f1.b);
    const XT* at = &As[buf][0];
#pragma unroll
    for (int s = 0; s < 4; s++) {
      const V bq0 = dequant8<BITS, XT>(f0.w, s, s0, b0);
      const V bq1 = dequant8<BITS, XT>(f1.w, s, s1, b1);
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const V av8 = *reinterpret_cast<const V*>(at + (t * 32 + col) * kGAS + 32 * h + 8 * s);
        acc0[t] = MfmaOp<XT>::mma(av8, bq0, acc0[t]);
        acc1[t] = MfmaOp<XT>::mma(av8, bq1, acc1[t]);
      }
    }
    if (more) {
      store_a(buf ^ 1, av);
      f0 = g0;
      f1 = g1;
    }
    __syncthreads();
  }

  // epilogue: lane holds column col, rows 8 (r / 4) + 4 h + r % 4 of each
  // 32 x 32 tile
  XT* out = reinterpret_cast<XT*>(a.out);
  const XT* ob0 = reinterpret_cast<const XT*>(a.p0.ob);
  const XT* ob1 = reinterpret_cast<const XT*>(GATEUP ? a.p1.ob : a.p0.ob);
  const int c0 = n0 + col, c1 = GATEUP ? c0 : n0 + 32 + col;
  const float obv0 = (ob0 && c0 < N) ? to_f<XT>(ob0[(size_t)e * N + c0]) : 0.f;
  const float obv1 = (ob1 && c1 < N) ? to_f<XT>(ob1[(size_t)e * N + c1]) : 0.f;
#pragma unroll
  for (int t = 0; t < 4; t++) {
#pragma unroll
    for (int r = 0; r < 16; r++) {
      const uint32_t p = m0 + (uint32_t)(t * 32 + 8 * (r >> 2) + 4 * h + (r & 3));
      if (p >= pend) continue;
      float v0 = round_to<XT>(acc0[t][r]);
      if (ob0) v0 = round_to<XT>(v0 + obv0);
      float v1 = round_to<XT>(acc1[t][r]);
      if (ob1) v1 = round_to<XT>(v1 + obv1);
      if constexpr (GATEUP) {
        if (c0 < N) out[(size_t)p * N + c0] = from_f<XT>(apply_act(v0, v1, a.act, a.alpha, a.limit));
      } else {
        if (c0 < N) out[(size_t)p * N + c0] = from_f<XT>(v0);
        if (c1 < N) out[(size_t)p * N + c1] = from_f<XT>(v1);
      }
    }
  }
}

template <int BITS, typename XT, typename ST>
static hipError_t launch_gemm_t(bool gateup, const GemmArgs& a, int grid, hipStream_t st,
                                KEvents ev) {
  if (gateup)
    hipExtLaunchKernelGGL((gemm_grouped_kernel<BITS, XT, ST, true>), dim3(grid), dim3(256), 0, st,
                          ev.start, ev.stop, 0, a);
  else
    hipExtLaunchKernelGGL((gemm_grouped_kernel<BITS, XT, ST, false>), dim3(grid), dim3(256), 0, st,
                          ev.start, ev.stop, 0, a);
  return hipGetLastError();
}

#define MOE_CAT2(a, b) a##b
#define MOE_CAT(a, b) MOE_CAT2(a, b)

hipError_t MOE_CAT(launch_gemm_b, MOE_BITS)(int xdt, int sbdt, bool gateup, const GemmArgs& a,
                                             int grid, hipStream_t st, KEvents ev) {
  if (xdt == DT_BF16 && sbdt == DT_BF16) return launch_gemm_t<MOE_BITS, bf16_t, bf16_t>(gateup, a, grid, st, ev);
  if (xdt == DT_BF16 && sbdt == DT_F16) return launch_gemm_t<MOE_BITS, bf16_t, f16_t>(gateup, a, grid, st, ev);
  if (xdt == DT_F16 && sbdt == DT_F16) return launch_gemm_t<MOE_BITS, f16_t, f16_t>(gateup, a, grid, st, ev);
  if (xdt == DT_F16 && sbdt == DT_BF16) return launch_gemm_t<MOE_BITS, f16_t, bf16_t>(gateup, a, grid, st, ev);
  return hipErrorInvalidValue;
}

}  // namespace moe
