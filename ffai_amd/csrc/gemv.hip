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
// decode of one token: gate/up with in-wave routing, then down + combine
// ---------------------------------------------------------------------------

template <int BITS, typename ST, int UR>
__device__ __forceinline__ void load_units(const GemvProj& p, size_t row, int row_words, int groups,
                                           int gs, int li, int L, int CU,
                                           WUnit<BITS> (&w)[UR]) {
#pragma unroll
  for (int j = 0; j < UR; j++) {
    const int u = li + j * L;
    if (u < CU) load_w_unit<BITS, ST>(p, row, row_words, groups, gs, u, w[j]);
  }
}

template <int BITS, typename XT, int UR>
__device__ __forceinline__ float dot_units(const WUnit<BITS> (&w)[UR],
                                           const XUnit<XT> (&xu)[UR], const float (&xs)[UR],
                                           int li, int L, int CU) {
  constexpr float MAGIC = Magic<BITS, XT>::value;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < UR; j++) {
    const int u = li + j * L;
    if (u < CU) {
      uint32_t cp[16];
      unpack_pairs<BITS>(w[j].w, cp);
      acc += w[j].s * dot_unit<BITS, XT>(cp, xu[j]) + (w[j].b - MAGIC * w[j].s) * xs[j];
    }
  }
  return acc;
}

template <int BITS, typename XT, typename ST, int UR>
__global__ __launch_bounds__(256) void gateup1_kernel(const Decode1Args a) {
  __shared__ float sc[4][kTopkMaxE];
  __shared__ int sel_lds[64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int slot = blockIdx.x / a.row_blocks, rb = blockIdx.x - slot * a.row_blocks;
  const bool writer = (blockIdx.x == 0 && wave == 0);
  const XT* logits = reinterpret_cast<const XT*>(a.logits);

  // every wave routes the token itself (identical, deterministic results)
  int sel;
  float wgt = 0.f;
  wave_topk<XT>(logits, a.E, a.k, a.gating, a.norm, a.ebias, sc[wave], writer, &sel, &wgt);
  int pos = 0;
  for (int r = 0; r < a.k; r++) pos += (__shfl(sel, r, 64) < sel) ? 1 : 0;
  const uint64_t hit = __ballot(lane < a.k && pos == slot);
  if (hit == 0) return;
  const int e = __shfl(sel, __ffsll((unsigned long long)hit) - 1, 64);
  if (writer) {
    if (lane < a.k) {
      a.idx[lane] = (uint32_t)sel;
      a.w[lane] = wgt;
      a.perm[pos] = (uint32_t)lane;
      sel_lds[lane] = sel;
    }
    if (a.offsets) {
      wave_sync();
      for (int ee = lane; ee <= a.E; ee += 64) {
        int c = 0;
        for (int r = 0; r < a.k; r++) c += (sel_lds[r] < ee) ? 1 : 0;
        a.offsets[ee] = (uint32_t)c;
      }
    }
  }

  const int N = a.N, K = a.K, CU = K >> 5, groups = K / a.gs, row_words = CU * BITS;
  const int L = 1 << a.lg, SG = 64 >> a.lg;
  const int sg = lane >> a.lg, li = lane & (L - 1);
  const int r_begin = rb * a.rows_per_block;
  const int r_end = min(N, r_begin + a.rows_per_block);
  const int stride = nwaves * SG;
  const size_t ebase = (size_t)e * N;
  XT* act = reinterpret_cast<XT*>(a.act) + (size_t)slot * N;

  int r = r_begin + wave * SG + sg;
  WUnit<BITS> A0[UR], A1[UR], B0[UR], B1[UR];
  if (r < r_end) {
    load_units<BITS, ST, UR>(a.g, ebase + r, row_words, groups, a.gs, li, L, CU, A0);
    load_units<BITS, ST, UR>(a.u, ebase + r, row_words, groups, a.gs, li, L, CU, A1);
  }
  XUnit<XT> xu[UR];
  float xs[UR];
  const XT* x = reinterpret_cast<const XT*>(a.x);
#pragma unroll
  for (int j = 0; j < UR; j++) {
    const int u = li + j * L;
    xs[j] = 0.f;
    if (u < CU) xs[j] = load_x_unit<BITS, XT>(x, u, xu[j]);
  }
  auto finish = [&](int rr, float g, float u) {
    g = wave_sum_width(g, L);
    u = wave_sum_width(u, L);
    if (li == 0) {
      const float gv = finish_proj<XT>(g, a.g.ob, ebase + rr);
      const float uv = finish_proj<XT>(u, a.u.ob, ebase + rr);
      act[rr] = from_f<XT>(apply_act(gv, uv, a.act_kind, a.alpha, a.limit));
    }
  };
  while (r < r_end) {
    int rn = r + stride;
    if (rn < r_end) {
      load_units<BITS, ST, UR>(a.g, ebase + rn, row_words, groups, a.gs, li, L, CU, B0);
      load_units<BITS, ST, UR>(a.u, ebase + rn, row_words, groups, a.gs, li, L, CU, B1);
    }
    finish(r, dot_units<BITS, XT, UR>(A0, xu, xs, li, L, CU), dot_units<BITS, XT, UR>(A1, xu, xs, li, L, CU));
    r = rn;
    if (r >= r_end) break;
    rn = r + stride;
    if (rn < r_end) {
      load_units<BITS, ST, UR>(a.g, ebase + rn, row_words, groups, a.gs, li, L, CU, A0);
      load_units<BITS, ST, UR>(a.u, ebase + rn, row_words, groups, a.gs, li, L, CU, A1);
    }
    finish(r, dot_units<BITS, XT, UR>(B0, xu, xs, li, L, CU), dot_units<BITS, XT, UR>(B1, xu, xs, li, L, CU));
    r = rn;
  }
}

template <int BITS, typename ST, int PR, int UR>
__device__ __forceinline__ void down1_load_row(const GemvProj& P, int N, int k, int gs,
                                               const uint32_t (&ex)[PR], int r, int sg, int SG,
                                               int li, int L, int CU, int row_words, int groups,
                                               WUnit<BITS> (&w)[PR][UR]) {
#pragma unroll
  for (int q = 0; q < PR; q++)
    if (sg + q * SG < k)
      load_units<BITS, ST, UR>(P, (size_t)ex[q] * N + r, row_words, groups, gs, li, L, CU, w[q]);
}

// One output row: each expert's output is rounded to the activation dtype
// before it is weighted, as the unfused path stores it (MoELayer.swift:
// 895-939); a full-wave reduction adds the k experts.
template <int BITS, typename XT, int PR, int UR>
__device__ __forceinline__ void down1_row(const void* ob, XT* out, int N, int k,
                                          const uint32_t (&ex)[PR], const float (&wsl)[PR],
                                          const XUnit<XT> (&xu)[PR][UR], const float (&xs)[PR][UR],
                                          const WUnit<BITS> (&w)[PR][UR], int r, int sg, int SG,
                                          int li, int L, int CU, int lane) {
  float acc = 0.f;
#pragma unroll
  for (int q = 0; q < PR; q++) {
    const int p = sg + q * SG;
    float part = 0.f;
    if (p < k) part = dot_units<BITS, XT, UR>(w[q], xu[q], xs[q], li, L, CU);
    part = wave_sum_width(part, L);
    if (p < k && li == 0) acc += wsl[q] * finish_proj<XT>(part, ob, (size_t)ex[q] * N + r);
  }
  acc = wave_sum_width(acc, 64);
  if (lane == 0) out[r] = from_f<XT>(acc);
}

template <int BITS, typename XT, typename ST, int PR, int UR>
__global__ __launch_bounds__(256) void down1_kernel(const Down1Args a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int N = a.N, K = a.K, CU = K >> 5, groups = K / a.gs, row_words = CU * BITS;
  const int L = 1 << a.lg, SG = 64 >> a.lg;
  const int sg = lane >> a.lg, li = lane & (L - 1);
  const int r_begin = blockIdx.x * a.rows_per_block;
  const int r_end = min(N, r_begin + a.rows_per_block);
  XT* al = reinterpret_cast<XT*>(smem);
  const GemvProj P = a.p;
  const int kk = a.k, gs = a.gs;
  XT* out = reinterpret_cast<XT*>(a.out);

  // stage the k activation rows (natural order) while the weights stream in
  constexpr int EPV = 16 / sizeof(XT);
  constexpr int NPRE = 4;
  const int nvec = a.k * K / EPV;
  const uint4* src = reinterpret_cast<const uint4*>(a.act);
  uint4* dst = reinterpret_cast<uint4*>(al);
  uint4 stage[NPRE];
#pragma unroll
  for (int j = 0; j < NPRE; j++) {
    const int i = threadIdx.x + j * blockDim.x;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (i < nvec) v = src[i];
    stage[j] = v;
  }

  uint32_t ex[PR];
  float wsl[PR];
#pragma unroll
  for (int q = 0; q < PR; q++) {
    const int p = sg + q * SG;
    ex[q] = 0;
    wsl[q] = 0.f;
    if (p < a.k) {
      const uint32_t s = a.perm[p];
      ex[q] = a.idx[s];
      wsl[q] = round_to<XT>(a.w[s]);
    }
  }
  int r = r_begin + wave;
  WUnit<BITS> A[PR][UR], B[PR][UR];
  if (r < r_end) down1_load_row<BITS, ST, PR, UR>(P, N, kk, gs, ex, r, sg, SG, li, L, CU, row_words, groups, A);

#pragma unroll
  for (int j = 0; j < NPRE; j++) {
    const int i = threadIdx.x + j * blockDim.x;
    if (i < nvec) dst[i] = stage[j];
  }
  for (int i = threadIdx.x + NPRE * blockDim.x; i < nvec; i += blockDim.x) dst[i] = src[i];
  __syncthreads();

  XUnit<XT> xu[PR][UR];
  float xs[PR][UR];
#pragma unroll
  for (int q = 0; q < PR; q++) {
    const int p = sg + q * SG;
#pragma unroll
    for (int j = 0; j < UR; j++) {
      const int u = li + j * L;
      xs[q][j] = 0.f;
      if (p < a.k && u < CU) xs[q][j] = load_x_unit<BITS, XT>(al + (size_t)p * K, u, xu[q][j]);
    }
  }
  while (r < r_end) {
    int rn = r + nwaves;
    if (rn < r_end) down1_load_row<BITS, ST, PR, UR>(P, N, kk, gs, ex, rn, sg, SG, li, L, CU, row_words, groups, B);
    down1_row<BITS, XT, PR, UR>(P.ob, out, N, kk, ex, wsl, xu, xs, A, r, sg, SG, li, L, CU, lane);
    r = rn;
    if (r >= r_end) break;
    rn = r + nwaves;
    if (rn < r_end) down1_load_row<BITS, ST, PR, UR>(P, N, kk, gs, ex, rn, sg, SG, li, L, CU, row_words, groups, A);
    down1_row<BITS, XT, PR, UR>(P.ob, out, N, kk, ex, wsl, xu, xs, B, r, sg, SG, li, L, CU, lane);
    r = rn;
  }
}

template <int BITS, typename XT, typename ST, int UR>
static hipError_t launch_dec1_u(bool down, int pr, const void* args, int grid, size_t smem,
                                hipStream_t st) {
  if (!down)
    hipLaunchKernelGGL((gateup1_kernel<BITS, XT, ST, UR>), dim3(grid), dim3(256), 0, st,
                       *reinterpret_cast<const Decode1Args*>(args));
  else if (pr == 1)
    hipLaunchKernelGGL((down1_kernel<BITS, XT, ST, 1, UR>), dim3(grid), dim3(256), smem, st,
                       *reinterpret_cast<const Down1Args*>(args));
  else
    hipLaunchKernelGGL((down1_kernel<BITS, XT, ST, 2, UR>), dim3(grid), dim3(256), smem, st,
                       *reinterpret_cast<const Down1Args*>(args));
  return hipGetLastError();
}

template <int BITS, typename XT, typename ST>
static hipError_t launch_dec1_t(bool down, int pr, int ur, const void* args, int grid, size_t smem,
                                hipStream_t st) {
  switch (ur) {
    case 1: return launch_dec1_u<BITS, XT, ST, 1>(down, pr, args, grid, smem, st);
    case 2: return launch_dec1_u<BITS, XT, ST, 2>(down, pr, args, grid, smem, st);
    case 3: return launch_dec1_u<BITS, XT, ST, 3>(down, pr, args, grid, smem, st);
    case 4: return launch_dec1_u<BITS, XT, ST, 4>(down, pr, args, grid, smem, st);
  }
  return hipErrorInvalidValue;
}

template <int BITS>
static hipError_t launch_dec1_bits(int xdt, int sbdt, bool down, int pr, int ur, const void* args,
                                   int grid, size_t smem, hipStream_t st) {
  if (xdt == DT_BF16 && sbdt == DT_BF16) return launch_dec1_t<BITS, bf16_t, bf16_t>(down, pr, ur, args, grid, smem, st);
  if (xdt == DT_BF16 && sbdt == DT_F16) return launch_dec1_t<BITS, bf16_t, f16_t>(down, pr, ur, args, grid, smem, st);
  if (xdt == DT_F16 && sbdt == DT_F16) return launch_dec1_t<BITS, f16_t, f16_t>(down, pr, ur, args, grid, smem, st);
  if (xdt == DT_F16 && sbdt == DT_BF16) return launch_dec1_t<BITS, f16_t, bf16_t>(down, pr, ur, args, grid, smem, st);
  return hipErrorInvalidValue;
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

// One translation unit per bit width (MOE_BITS) keeps compile times short;
// the per-width entry points are stitched together in api.cpp.
#define MOE_CAT2(a, b) a##b
#define MOE_CAT(a, b) MOE_CAT2(a, b)

hipError_t MOE_CAT(launch_gemv_b, MOE_BITS)(int xdt, int sbdt, bool gateup, int tokmax,
                                             const GemvArgs& a, int grid, hipStream_t st) {
  return launch_gemv_bits<MOE_BITS>(xdt, sbdt, gateup, tokmax, a, grid, st);
}

hipError_t MOE_CAT(launch_dec1_b, MOE_BITS)(int xdt, int sbdt, bool down, int pr, int ur,
                                             const void* args, int grid, size_t smem,
                                             hipStream_t st) {
  return launch_dec1_bits<MOE_BITS>(xdt, sbdt, down, pr, ur, args, grid, smem, st);
}

}  // namespace moe
