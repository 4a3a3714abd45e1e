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
#include <hip/hip_ext.h>

#include "moe_common.hpp"
#include "moe_internal.hpp"
#include "decode_units.hpp"

#ifndef MOE_BITS
#define MOE_BITS 4
#endif

namespace moe {

constexpr int kUMax = 8;  // units per lane (host picks L so ceil(K/32/L) <= 8)

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
  const int N = a.N, K = a.K, CU = K >> 5, groups = CU >> a.gsh, row_words = CU * BITS;
  const int r_begin = rb * a.rows_per_block;
  const int r_end = min(N, r_begin + a.rows_per_block);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int L = 1 << a.lg, SG = 64 >> a.lg;
  const int sg = lane >> a.lg, li = lane & (L - 1);
  const GemvProj p0 = expert_proj<BITS, ST>(a.p0, e, N, row_words, groups);
  const GemvProj p1 = expert_proj<BITS, ST>(a.p1, e, N, row_words, groups);
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
      const uint32_t row = (uint32_t)r;
      float acc0[TOKMAX], acc1[TOKMAX];
#pragma unroll
      for (int t = 0; t < TOKMAX; t++) acc0[t] = acc1[t] = 0.f;
      WUnit<BITS, ST> w0[kUMax], w1[kUMax];
#pragma unroll
      for (int j = 0; j < kUMax; j++) {
        const int u = li + j * L;
        if (u < CU) {
          load_w_unit<BITS, ST>(p0, row, row_words, groups, a.gsh, u, w0[j]);
          if constexpr (GATEUP) load_w_unit<BITS, ST>(p1, row, row_words, groups, a.gsh, u, w1[j]);
        }
      }
#pragma unroll
      for (int j = 0; j < kUMax; j++) {
        const int u = li + j * L;
        if (u < CU) {
          uint32_t cp0[16], cp1[16];
          unpack_pairs<BITS, Magic<BITS, XT>::bits>(w0[j].w, cp0);
          const float bb0 = w0[j].b() - MAGIC * w0[j].s();
          float bb1 = 0.f;
          if constexpr (GATEUP) {
            unpack_pairs<BITS, Magic<BITS, XT>::bits>(w1[j].w, cp1);
            bb1 = w1[j].b() - MAGIC * w1[j].s();
          }
#pragma unroll
          for (int t = 0; t < TOKMAX; t++) {
            if (t < nt) {
              XUnit<XT> xu;
              lds_x_unit<XT>(xs + t * K, u, xu);
              const float xsu = xsum[t * CU + u];
              acc0[t] += w0[j].s() * dot_unit<BITS, XT>(cp0, xu) + bb0 * xsu;
              if constexpr (GATEUP) acc1[t] += w1[j].s() * dot_unit<BITS, XT>(cp1, xu) + bb1 * xsu;
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
            const float g = finish_proj<XT>(acc0[t], a.p0.ob, ebase + r);
            if constexpr (GATEUP) {
              const float u = finish_proj<XT>(acc1[t], a.p1.ob, ebase + r);
              out[o] = from_f<XT>(apply_act<XT>(g, u, a.act, a.alpha, a.limit));
            } else {
              // single projection: only ReLU^2 acts on it (no gate)
              out[o] = from_f<XT>(a.act == ACT_RELU2 ? apply_act<XT>(0.f, g, ACT_RELU2, 0.f, 0.f) : g);
            }
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// grouped GEMV for a few rows per expert (batched decode), 16-bit activations
//
// LDS holds a pass's activation units quad-major ([token][quad][unit], 16
// bytes each), so the lanes of a row group, which take consecutive units,
// read consecutive 16 bytes (a unit-major layout put them 64 bytes apart, on
// the same banks).
// Block (slot, rb): expert used[1 + slot] and rows_per_block weight rows,
// taken in iterations of R1 = 4 SG RM rows (lane rows as in gateup1_kernel:
// wave w, sub-group sg, it < RM). The expert's sorted positions go through
// in passes of up to TM rows; per pass the block stages the activation rows
// into LDS once, in pair order with the per-unit sums (one thread per
// 64-byte unit, 16-byte loads), and every iteration multiplies against them,
// so the staging is shared by all the block's rows. Two register sets of
// weights alternate: iteration i + 1's loads (output biases first) are in
// flight while iteration i multiplies. The dot products run unit by unit,
// token by token, so one LDS read of an activation unit serves every row and
// both projections of the lane. A pass's activation loads are issued before
// its first weight loads: loads retire in order, so staging waits for them
// alone, and the block barriers order LDS only.
// ---------------------------------------------------------------------------

// Items q0 and q0 + 256 of a pass, (token q / CU, unit q % CU): the loads
// (stage_load; past the pass they repeat its last item) and the pair-order
// LDS rows with their sums (stage_store).
template <typename XT>
__device__ __forceinline__ void stage_load(const XT* __restrict__ x, const uint32_t* __restrict__ perm,
                                           int topk, uint32_t pc, int nt, int K, int CU, int q0,
                                           uint32_t (&n)[2][16]) {
  const int total = nt * CU;
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const int q = min(q0 + 256 * r, total - 1);
    const int t = q / CU, u = q - t * CU;
    const uint32_t p = pc + (uint32_t)t;
    const uint32_t row = perm ? perm[p] / (uint32_t)topk : p;
    const uint4* src = reinterpret_cast<const uint4*>(x + (size_t)row * K + (size_t)u * 32);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint4 v = src[j];
      n[r][4 * j] = v.x; n[r][4 * j + 1] = v.y; n[r][4 * j + 2] = v.z; n[r][4 * j + 3] = v.w;
    }
  }
}

template <int BITS, typename XT>
__device__ __forceinline__ void stage_store(const uint32_t (&n)[2][16], int nt, int CU, int q0,
                                            uint32_t* xl, float* xsl) {
  const int total = nt * CU;
#pragma unroll
  for (int r = 0; r < 2; r++) {
    const int q = q0 + 256 * r;
    if (q < total) {
      uint32_t pw[16];
      natural_to_pairs<BITS>(n[r], pw);
      // quad j of (token t, unit u) at uint4 (4 t + j) CU + u: lanes that
      // read consecutive units of one quad hit consecutive 16 bytes
      const int t = q / CU, u = q - t * CU;
      uint4* dst = reinterpret_cast<uint4*>(xl);
#pragma unroll
      for (int j = 0; j < 4; j++)
        dst[(size_t)(4 * t + j) * CU + u] = make_uint4(pw[4 * j], pw[4 * j + 1], pw[4 * j + 2], pw[4 * j + 3]);
      xsl[q] = sum16(n[r], __is_same(XT, bf16_t));
    }
  }
}

template <int BITS, typename XT, typename ST, bool GATEUP, int UR, int RM, int TM>
__global__ __launch_bounds__(256, 2) void gemv_multi_kernel(const GemvArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int slot = blockIdx.x / a.row_blocks, rb = blockIdx.x - slot * a.row_blocks;
  if ((uint32_t)slot >= a.used[0]) return;  // block-uniform, before any barrier
  const uint32_t e = __builtin_amdgcn_readfirstlane(a.used[1 + slot]);
  const uint32_t pbeg = __builtin_amdgcn_readfirstlane(a.offsets[e]);
  const uint32_t pend = __builtin_amdgcn_readfirstlane(a.offsets[e + 1]);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int N = a.N, K = a.K, CU = K >> 5, groups = CU >> a.gsh, row_words = CU * BITS;
  const int L = 1 << a.lg, SG = 64 >> a.lg;
  const int sg = lane >> a.lg, li = lane & (L - 1);
  // the block's rows go through in iterations of R1 = 4 SG RM rows: row
  // rbase + i R1 + it 4 SG of iteration i
  const int R1 = 4 * SG * RM, nit = a.rows_per_block / R1;
  const int r_end = min(N, (rb + 1) * a.rows_per_block);
  const int rbase = rb * a.rows_per_block + wave * SG + sg, stride = 4 * SG;
  uint32_t* xl = reinterpret_cast<uint32_t*>(smem);                         // [TM][4][CU][4]
  float* xsl = reinterpret_cast<float*>(smem + (size_t)TM * CU * 64);      // [TM][CU]
  const XT* x = reinterpret_cast<const XT*>(a.x);
  XT* out = reinterpret_cast<XT*>(a.out);
  constexpr float MAGIC = Magic<BITS, XT>::value;
  const ProjView P0 = proj_view<BITS, ST>(a.p0, e, N, row_words, groups);
  const ProjView P1 = GATEUP ? proj_view<BITS, ST>(a.p1, e, N, row_words, groups) : P0;
  const uint32_t wstep = (uint32_t)(L * BITS * 4), sstep = (uint32_t)((L >> a.gsh) * sizeof(ST));
  const size_t ebase = (size_t)e * N;
  constexpr int RM1 = GATEUP ? RM : 1;

  // weights (and output biases) of one iteration's rows
  struct WSet {
    WUnit<BITS, ST> w0[RM][UR], w1[RM1][UR];
    float ob0[RM], ob1[RM];
  };
  auto load_w = [&](int i, WSet& ws) __attribute__((always_inline)) {
#pragma unroll
    for (int it = 0; it < RM; it++) {
      const int row = min(rbase + i * R1 + it * stride, N - 1);
      ws.ob0[it] = a.p0.ob ? to_f<XT>(reinterpret_cast<const XT*>(a.p0.ob)[ebase + row]) : 0.f;
      ws.ob1[it] = (GATEUP && a.p1.ob) ? to_f<XT>(reinterpret_cast<const XT*>(a.p1.ob)[ebase + row]) : 0.f;
      const UnitAddr ad = unit_addr<BITS, ST>((uint32_t)row, row_words, groups, li, a.gsh);
      bload_units<BITS, ST, UR, kStream>(P0, ad, wstep, sstep, ws.w0[it]);
      if constexpr (GATEUP) bload_units<BITS, ST, UR, kStream>(P1, ad, wstep, sstep, ws.w1[it]);
    }
  };
  // iteration i's rows against the nt staged activation rows of pass pc
  auto compute = [&](int i, const WSet& ws, uint32_t pc, int nt) __attribute__((always_inline)) {
    float acc0[RM][TM], acc1[RM1][TM];
#pragma unroll
    for (int it = 0; it < RM; it++)
#pragma unroll
      for (int t = 0; t < TM; t++) {
        acc0[it][t] = 0.f;
        if constexpr (GATEUP) acc1[it][t] = 0.f;
      }
#pragma unroll
    for (int j = 0; j < UR; j++) {
      const int u = li + j * L;
      const bool valid = u < CU;
      const int uc = min(u, CU - 1);
      uint32_t cp0[RM][16], cp1[RM1][16];
      float s0[RM], b0[RM], s1[RM1], b1[RM1];
#pragma unroll
      for (int it = 0; it < RM; it++) {
        unpack_pairs<BITS, Magic<BITS, XT>::bits>(ws.w0[it][j].w, cp0[it]);
        s0[it] = ws.w0[it][j].s();
        b0[it] = ws.w0[it][j].b() - MAGIC * s0[it];
        if constexpr (GATEUP) {
          unpack_pairs<BITS, Magic<BITS, XT>::bits>(ws.w1[it][j].w, cp1[it]);
          s1[it] = ws.w1[it][j].s();
          b1[it] = ws.w1[it][j].b() - MAGIC * s1[it];
        }
      }
#pragma unroll
      for (int t = 0; t < TM; t++) {
        if (t < nt) {  // block-uniform
          XUnit<XT> xu;
          const uint4* xq = reinterpret_cast<const uint4*>(xl) + (size_t)(4 * t) * CU + uc;
#pragma unroll
          for (int q = 0; q < 4; q++) {
            const uint4 v = xq[(size_t)q * CU];
            xu.v[4 * q] = v.x; xu.v[4 * q + 1] = v.y; xu.v[4 * q + 2] = v.z; xu.v[4 * q + 3] = v.w;
          }
          const float xs = xsl[t * CU + uc];
#pragma unroll
          for (int it = 0; it < RM; it++) {
            const float v0 = s0[it] * dot_unit<BITS, XT>(cp0[it], xu) + b0[it] * xs;
            acc0[it][t] += valid ? v0 : 0.f;
            if constexpr (GATEUP) {
              const float v1 = s1[it] * dot_unit<BITS, XT>(cp1[it], xu) + b1[it] * xs;
              acc1[it][t] += valid ? v1 : 0.f;
            }
          }
        }
      }
    }
#pragma unroll
    for (int it = 0; it < RM; it++) {
      const int row = rbase + i * R1 + it * stride;
#pragma unroll
      for (int t = 0; t < TM; t++) {
        if (t < nt) {
          float g = group_sum(acc0[it][t], a.lg);
          float v;
          if constexpr (GATEUP) {
            float uu = group_sum(acc1[it][t], a.lg);
            g = round_to<XT>(g);
            uu = round_to<XT>(uu);
            if (a.p0.ob) g = round_to<XT>(g + ws.ob0[it]);
            if (a.p1.ob) uu = round_to<XT>(uu + ws.ob1[it]);
            v = apply_act<XT>(g, uu, a.act, a.alpha, a.limit);
          } else {
            g = round_to<XT>(g);
            if (a.p0.ob) g = round_to<XT>(g + ws.ob0[it]);
            // single projection: only ReLU^2 acts on it (no gate)
            v = a.act == ACT_RELU2 ? apply_act<XT>(0.f, g, ACT_RELU2, 0.f, 0.f) : g;
          }
          if (li == L - 1 && row < r_end) out[(size_t)(pc + t) * N + row] = from_f<XT>(v);
        }
      }
    }
  };

  WSet wa, wb;
  // (reading iteration 0's weights before the rows' range and positions, as
  // gemv_mma_kernel does, measured slower here: Qwen3 16 tokens gate/up 43.2
  // -> 51.2 us)
  for (uint32_t pc = pbeg; pc < pend;) {
    const int nt = min((int)(pend - pc), TM);
    // this pass's first activation loads, then iteration 0's weights, then
    // the activations into LDS once every wave is done with the last pass
    uint32_t xn[2][16];
    stage_load<XT>(x, a.perm, a.topk, pc, nt, K, CU, (int)threadIdx.x, xn);
    load_w(0, wa);
    __builtin_amdgcn_sched_barrier(0);
    lds_barrier();  // LDS only: the weight loads stay in flight
    stage_store<BITS, XT>(xn, nt, CU, (int)threadIdx.x, xl, xsl);
    for (int q0 = threadIdx.x + 512; q0 < nt * CU; q0 += 512) {
      stage_load<XT>(x, a.perm, a.topk, pc, nt, K, CU, q0, xn);
      stage_store<BITS, XT>(xn, nt, CU, q0, xl, xsl);
    }
    lds_barrier();
    // iteration i + 1's weights load while iteration i multiplies (a form
    // with no break and loads past the last iteration that read nothing, as
    // in gemv_mma_kernel, measured slower here: blocks have one or two
    // iterations, Qwen3 batch 4 43.1 -> 45.7 us per layer step)
    for (int i = 0; i < nit; i += 2) {
      if (i + 1 < nit) load_w(i + 1, wb);
      compute(i, wa, pc, nt);
      if (i + 1 >= nit) break;
      if (i + 2 < nit) load_w(i + 2, wa);
      compute(i + 1, wb, pc, nt);
    }
    pc += (uint32_t)nt;
  }
}

#define MOE_CAT2(a, b) a##b
#define MOE_CAT(a, b) MOE_CAT2(a, b)

#if MOE_BITS <= 6
// ---------------------------------------------------------------------------
// grouped GEMV for a few rows per expert on the matrix cores (4-bit weights,
// 16-bit activations)
//
// Block (slot, rb): expert used[1 + slot] and 64 LDS weight rows (a gate/up
// pair: 32 rows of each; else 64 rows of one projection); the expert's
// sorted positions go through in passes of up to 16 rows. Wave w owns 16
// weight rows and computes C[t][r] = sum_k x[t][k] W[r][k] with
// v_mfma_f32_16x16x32: A = 16 activation rows, B = the 16 weight rows' codes
// with the magic offset (MAGIC + q exact in the 16-bit type), per 32-value
// unit. A second MFMA against all-ones gives the unit's activation sums Q, so
// the affine scale and bias apply per group in fp32 on the accumulators:
// acc = fma(b - MAGIC s, Q, fma(s, P, acc)). Lane (r, kb) = (lane % 16,
// lane / 16) supplies the codes of 8-value block kb of weight row r (bits
// [8 kb BITS, +8 BITS) of the unit's BITS words; for 4 bits, word kb), whose
// pairs (j, j + 4) match the activations' pair order, and
// quad kb of activation row r; it ends with rows 4 kb + i of output column r.
// K runs in chunks of 8 units through double-buffered LDS: per chunk the
// block copies 64 rows x 8 units of codes (BITS words each), their 16-bit
// scale/bias pairs and 16 rows x 8 units of activations (permuted to pair
// order), with global loads two chunks ahead of the MFMAs.
// ---------------------------------------------------------------------------

typedef float f32x4_t __attribute__((ext_vector_type(4)));

template <typename XT> struct Mma16;
template <> struct Mma16<bf16_t> {
  typedef __bf16 V __attribute__((ext_vector_type(8)));
  static constexpr uint32_t ones = 0x3F803F80u;
  static __device__ __forceinline__ f32x4_t mma(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(V, a), __builtin_bit_cast(V, b), c, 0, 0, 0);
  }
};
template <> struct Mma16<f16_t> {
  typedef _Float16 V __attribute__((ext_vector_type(8)));
  static constexpr uint32_t ones = 0x3C003C00u;
  static __device__ __forceinline__ f32x4_t mma(u32x4_t a, u32x4_t b, f32x4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(V, a), __builtin_bit_cast(V, b), c, 0, 0, 0);
  }
};

constexpr int kMmaU = 8;      // units per K chunk
constexpr int kMmaRows = 64;  // LDS weight rows per block
constexpr int kMmaTok = 16;   // activation rows per pass

// Codes of 8-value block kb of a unit as four magic-offset pairs (j, j + 4).
// mf: the pair's field mask ((1 << BITS) - 1) * 0x10001 and ml (2 and 3
// bits) the low-half mask (1 << 4 BITS) - 1, held by the caller in scalar
// registers, with MB in a vector register: gfx9's three-operand
// v_and_or_b32 / v_bfi_b32 take no literal, so with compile-time constants
// each step cost two two-operand instructions.
// 2 and 3 bits take all 8 BITS <= 24 bits of the block with one funnel
// shift, then merge values 4..7 up to bit 16 (the bits between the two
// halves hold no field a pair reads): checked equal to the per-value
// extraction for every block of 200,000 random units on the CPU.
template <int BITS>
__device__ __forceinline__ uint32_t mma_funnel(const uint32_t* unit, int bit) {
  const int i0 = bit >> 5, i1 = i0 + 1 < BITS ? i0 + 1 : BITS - 1;
  return __builtin_amdgcn_alignbit(unit[i1], unit[i0], (uint32_t)(bit & 31));
}
template <int BITS>
__device__ __forceinline__ u32x4_t mma_codes(const uint32_t* unit, int kb, uint32_t MB, uint32_t mf,
                                             uint32_t ml) {
  if constexpr (BITS == 4) {
    const uint32_t w = unit[kb];
    return u32x4_t{(w & mf) | MB, ((w >> 4) & mf) | MB, ((w >> 8) & mf) | MB, ((w >> 12) & mf) | MB};
  } else if constexpr (BITS <= 3) {
    const uint32_t v = mma_funnel<BITS>(unit, 8 * kb * BITS);
    const uint32_t m = (v & ml) | ((v << (16 - 4 * BITS)) & ~ml);
    return u32x4_t{(m & mf) | MB, ((m >> BITS) & mf) | MB, ((m >> (2 * BITS)) & mf) | MB,
                   ((m >> (3 * BITS)) & mf) | MB};
  } else {
    // 8 BITS <= 48 bits from bit 8 kb BITS: two consecutive words of the
    // unit hold them after the in-word shift (at most 24). (Two funnel shifts
    // merged as for 2 and 3 bits cut the 6-bit unpack by a third, but the
    // kernel then kept its accumulators in AGPRs and the down projection of
    // the mixed-bit layer went 67.1 -> 70.9 us at 256 tokens.)
    (void)mf;
    const int bit = 8 * kb * BITS, i0 = bit >> 5;
    const int i1 = i0 + 1 < BITS ? i0 + 1 : BITS - 1;
    const uint64_t v = ((uint64_t)unit[i0] | ((uint64_t)unit[i1] << 32)) >> (bit & 31);
    constexpr uint32_t m = (1u << BITS) - 1u;
    u32x4_t r;
#pragma unroll
    for (int j = 0; j < 4; j++)
      r[j] = ((uint32_t)(v >> (BITS * j)) & m) | (((uint32_t)(v >> (BITS * (j + 4))) & m) << 16) | MB;
    return r;
  }
}

// Four waves per SIMD where that fits in 128 VGPRs without spills (2- and
// 4-bit, 3-bit gate/up); the compiler's own choice elsewhere.
template <int BITS, bool GATEUP>
constexpr int kMmaWavesPerEu = (BITS == 2 || BITS == 4 || (BITS == 3 && GATEUP)) ? 4 : 1;

// GSH: log2(group size / 32), the launch's a.gsh (group sizes 32, 64, 128).
template <int BITS, typename XT, typename ST, bool GATEUP, int GSH>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kMmaWavesPerEu<BITS, GATEUP>)))
void gemv_mma_kernel(const GemvArgs a) {
  __shared__ __align__(16) uint32_t wl[2][kMmaRows * kMmaU * BITS];  // [row][unit slot][BITS words]
  __shared__ __align__(16) uint32_t sl[2][kMmaRows * kMmaU];      // [row][unit]: s | b << 16
  __shared__ __align__(16) uint32_t xl[2][kMmaU * kMmaTok * 16];  // [unit][row][quad slot][4 words]
  __shared__ float gl[32 * kMmaTok];                              // gate outputs of a pass
  const int slot = blockIdx.x / a.row_blocks, rb = blockIdx.x - slot * a.row_blocks;
  if ((uint32_t)slot >= a.used[0]) return;  // block-uniform, before any barrier
  const uint32_t e = __builtin_amdgcn_readfirstlane(a.used[1 + slot]);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = a.N, K = a.K, CU = K >> 5, groups = CU >> GSH, row_words = CU * BITS;
  constexpr int UPG = 1 << GSH;  // units per scale group
  const int nchunks = (CU + kMmaU - 1) / kMmaU;
  constexpr int RPB = GATEUP ? 32 : 64;  // output rows per block
  const int r_begin = rb * RPB;
  const ProjView P0 = proj_view<BITS, ST>(a.p0, e, N, row_words, groups);
  const ProjView P1 = GATEUP ? proj_view<BITS, ST>(a.p1, e, N, row_words, groups) : P0;
  // activation rows through a buffer view (the host keeps x_rows K 16-bit
  // values below 2^31 bytes): the rows of a pass past its end read zero at a
  // dead offset instead of repeating its last row, and offsets stay 32-bit
  const rsrc_t xr = make_rsrc(a.x, (uint32_t)((size_t)a.x_rows * (size_t)K * sizeof(XT)));
  // MAGIC + q is exact in the 16-bit type for q < 128 (bf16) / 1024 (f16)
  constexpr float MAGIC = Magic<BITS, XT>::value;
  constexpr uint32_t MB = Magic<BITS, XT>::bits;
  static_assert(Magic<BITS, XT>::dot2, "magic-offset codes");
  const int r = lane & 15, kb = lane >> 4;
  // this lane's LDS weight row and output row
  const int lr = GATEUP ? (wave >> 1) * 32 + (wave & 1) * 16 + r : wave * 16 + r;
  const int orow = r_begin + (GATEUP ? (wave & 1) * 16 : wave * 16) + r;

  // staging items of this thread, j < 2: codes and scales of LDS row
  // (tid >> 3) + 32 j, unit slot tid & 7; activation quad q = tid + 256 j:
  // unit q >> 6, row (q >> 2) & 15 (the same for both j), quad q & 3
  const int s_lr0 = tid >> 3, s_us = tid & 7;
  const int x_t = (tid >> 2) & 15, x_kb = tid & 3, x_us0 = wave;  // x_us0 scalar
  struct Stage {
    uint32_t w[2][BITS];
    u32x4_t x[2];
    uint32_t s[2], b[2];  // 16-bit scale and bias, merged only when stored (no early wait)
  };
  auto gw_row = [&](int slr) -> uint32_t {
    const int g = GATEUP ? r_begin + (slr & 31) : r_begin + slr;
    return (uint32_t)min(g, N - 1);
  };
  // chunks past the last load their weights at offsets past the views' ends
  // (2^31 and more: the views of one expert are far smaller), which read zero
  // without touching memory, so the loop below issues the same loads on every
  // trip. (Selecting views of zero bytes instead cost eight VGPRs.)
  auto load_w_stage = [&](int c, Stage& st) __attribute__((always_inline)) {
    const int cc = min(c, nchunks - 1);
    const uint32_t dead = c < nchunks ? 0u : 0x80000000u;  // block-uniform
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int slr = s_lr0 + 32 * j;
      const ProjView& pv = (GATEUP && j == 1) ? P1 : P0;
      const uint32_t grow = gw_row(slr);
      const int uu = kMmaU * cc + s_us;
      const uint32_t u = (uint32_t)min(uu, CU - 1);
      bload_unit<BITS>(pv.w, (grow * (uint32_t)row_words + u * (uint32_t)BITS) * 4u + dead, st.w[j]);
      // units past K (the last chunk's tail) read a zero scale and bias, so
      // their products with the clamped unit's codes and activations add
      // zero (for finite activations; a non-finite one in a row's last unit
      // makes its outputs non-finite either way)
      const uint32_t sdead = uu < CU ? dead : 0x80000000u;
      const uint32_t gi = (grow * (uint32_t)groups + (u >> GSH)) * (uint32_t)sizeof(ST) + sdead;
      st.s[j] = (uint32_t)bload16(pv.s, gi);
      st.b[j] = (uint32_t)bload16(pv.b, gi);
    }
  };
  auto load_x_stage = [&](int c, uint32_t xbase, Stage& st) __attribute__((always_inline)) {
    const int cc = min(c, nchunks - 1);
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int ux = min(kMmaU * cc + x_us0 + 4 * j, CU - 1);
      st.x[j] = bload128(xr, xbase + (uint32_t)ux * 64u + (uint32_t)x_kb * 16u);
    }
  };
  auto load_stage = [&](int c, uint32_t xbase, Stage& st) __attribute__((always_inline)) {
    load_w_stage(c, st);
    load_x_stage(c, xbase, st);
  };
  auto store_stage = [&](const Stage& st, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int slr = s_lr0 + 32 * j;
      uint32_t* wd = &wl[buf][(slr * kMmaU + ((s_us + slr) & 7)) * BITS];
      if constexpr (BITS == 4) {
        *reinterpret_cast<u32x4_t*>(wd) = u32x4_t{st.w[j][0], st.w[j][1], st.w[j][2], st.w[j][3]};
      } else {
#pragma unroll
        for (int q = 0; q < BITS; q++) wd[q] = st.w[j][q];
      }
      sl[buf][slr * kMmaU + s_us] = st.s[j] | (st.b[j] << 16);
      // natural values x0..x7 -> pairs (x0, x4), (x1, x5), (x2, x6), (x3, x7)
      const u32x4_t n = st.x[j];
      const u32x4_t pw = {(n[0] & 0xFFFFu) | (n[2] << 16), (n[0] >> 16) | (n[2] & 0xFFFF0000u),
                          (n[1] & 0xFFFFu) | (n[3] << 16), (n[1] >> 16) | (n[3] & 0xFFFF0000u)};
      const int us = x_us0 + 4 * j;
      *reinterpret_cast<u32x4_t*>(&xl[buf][((us * kMmaTok + x_t) * 4 + (x_kb ^ ((x_t >> 2) & 3))) * 4]) = pw;
    }
  };
  const u32x4_t ones = {Mma16<XT>::ones, Mma16<XT>::ones, Mma16<XT>::ones, Mma16<XT>::ones};
  // opaque copies of the unpack's constants (see mma_codes)
  uint32_t mf, ml, mbv;
  asm("s_mov_b32 %0, %1" : "=s"(mf) : "i"(((1u << BITS) - 1u) * 0x10001u));
  asm("s_mov_b32 %0, %1" : "=s"(ml) : "i"((1u << (4 * (BITS < 4 ? BITS : 4))) - 1u));
  asm("v_mov_b32 %0, %1" : "=v"(mbv) : "i"(MB));
  f32x4_t acc;
  // Every chunk runs the same straight-line code: K is a multiple of the
  // group size, so groups never straddle the end of K, and the units past it
  // carry zero scales and biases. A group's first unit starts P and Q from a
  // zero accumulator (no register clears), its last applies the group's
  // scale and bias; with the group size a runtime value the compiler kept
  // both per unit behind branches, with eight register clears per group.
  auto compute = [&](int buf) __attribute__((always_inline)) {
    f32x4_t P = {}, Q = {};
#pragma unroll
    for (int us = 0; us < kMmaU; us++) {
      const u32x4_t bop = mma_codes<BITS>(&wl[buf][(lr * kMmaU + ((us + lr) & 7)) * BITS], kb, mbv, mf, ml);
      const u32x4_t aop =
          *reinterpret_cast<const u32x4_t*>(&xl[buf][((us * kMmaTok + r) * 4 + (kb ^ ((r >> 2) & 3))) * 4]);
      P = Mma16<XT>::mma(aop, bop, us % UPG == 0 ? f32x4_t{} : P);
      Q = Mma16<XT>::mma(aop, ones, us % UPG == 0 ? f32x4_t{} : Q);
      if ((us + 1) % UPG == 0) {
        const uint32_t sb = sl[buf][lr * kMmaU + us];
        const float sc = to_f<ST>(__builtin_bit_cast(ST, (uint16_t)(sb & 0xFFFFu)));
        const float bi = to_f<ST>(__builtin_bit_cast(ST, (uint16_t)(sb >> 16))) - MAGIC * sc;
        // two chained fmas per output (the sum s P + bi Q as written cost a
        // multiply, an fma and an add)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = __builtin_fmaf(bi, Q[i], __builtin_fmaf(sc, P[i], acc[i]));
      }
    }
  };

  XT* out = reinterpret_cast<XT*>(a.out);
  Stage s0, s1;
  // chunk 0 and 1 weights need only the expert: the first pass's go out
  // before its rows' range and positions are read (two dependent loads),
  // each later pass's at the end of the pass before
  load_w_stage(0, s0);
  load_w_stage(1, s1);
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t pbeg = __builtin_amdgcn_readfirstlane(a.offsets[e]);
  const uint32_t pend = __builtin_amdgcn_readfirstlane(a.offsets[e + 1]);
  for (uint32_t pc = pbeg; pc < pend; pc += kMmaTok) {
    const int nt = min((int)(pend - pc), kMmaTok);
    const uint32_t p = pc + (uint32_t)min(x_t, nt - 1);
    const uint32_t xrow = a.perm ? a.perm[p] / (uint32_t)a.topk : p;
    const uint32_t xbase = x_t < nt ? xrow * (uint32_t)K * (uint32_t)sizeof(XT) : 0x80000000u;
    load_x_stage(0, xbase, s0);
    load_x_stage(1, xbase, s1);
    lds_barrier();  // the last pass's LDS reads (and gl) are done; loads stay in flight
    store_stage(s0, 0);
    load_stage(2, xbase, s0);
    lds_barrier();
    acc = f32x4_t{};
    // No break in this loop: with one, the compiler's wait counts at the loop
    // head took the break path's state (chunk c + 3's loads youngest) and the
    // stores of chunk c + 1 waited for chunk c + 2's loads as well. An odd
    // chunk count runs a last trip whose second chunk is skipped (its weight
    // loads read nothing, its stores land in a buffer nothing reads). Peeling
    // that chunk off the loop instead cost eight VGPRs and one wave per SIMD.
    for (int c = 0; c < nchunks; c += 2) {
      compute(0);
      store_stage(s1, 1);  // chunk c + 1
      load_stage(c + 3, xbase, s1);
      lds_barrier();
      if (c + 1 < nchunks) compute(1);
      store_stage(s0, 0);  // chunk c + 2
      load_stage(c + 4, xbase, s0);
      lds_barrier();
    }
    // lane (r, kb): output column orow, activation rows 4 kb + i of the pass
    const size_t ob_i = (size_t)e * N + (size_t)min(orow, N - 1);
    if constexpr (GATEUP) {
      if (wave < 2) {
        const float ob = a.p0.ob ? to_f<XT>(reinterpret_cast<const XT*>(a.p0.ob)[ob_i]) : 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          float g = round_to<XT>(acc[i]);
          if (a.p0.ob) g = round_to<XT>(g + ob);
          gl[((wave & 1) * 16 + r) * kMmaTok + 4 * kb + i] = g;
        }
      }
      __syncthreads();
      if (wave >= 2) {
        const float ob = a.p1.ob ? to_f<XT>(reinterpret_cast<const XT*>(a.p1.ob)[ob_i]) : 0.f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int t = 4 * kb + i;
          float u = round_to<XT>(acc[i]);
          if (a.p1.ob) u = round_to<XT>(u + ob);
          const float g = gl[((wave & 1) * 16 + r) * kMmaTok + t];
          if (t < nt && orow < N)
            out[(size_t)(pc + t) * N + orow] = from_f<XT>(apply_act<XT>(g, u, a.act, a.alpha, a.limit));
        }
      }
    } else {
      const float ob = a.p0.ob ? to_f<XT>(reinterpret_cast<const XT*>(a.p0.ob)[ob_i]) : 0.f;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int t = 4 * kb + i;
        float g = round_to<XT>(acc[i]);
        if (a.p0.ob) g = round_to<XT>(g + ob);
        // single projection: only ReLU^2 acts on it (no gate)
        const float v = a.act == ACT_RELU2 ? apply_act<XT>(0.f, g, ACT_RELU2, 0.f, 0.f) : g;
        if (t < nt && orow < N) out[(size_t)(pc + t) * N + orow] = from_f<XT>(v);
      }
    }
    if (pc + kMmaTok < pend) {  // the next pass's chunk 0 and 1 weights (block-uniform)
      load_w_stage(0, s0);
      load_w_stage(1, s1);
    }
  }
}

template <typename XT, typename ST, int GSH>
static hipError_t launch_mma_g(bool gateup, const GemvArgs& a, int grid, hipStream_t st, KEvents ev) {
  if (gateup)
    hipExtLaunchKernelGGL((gemv_mma_kernel<MOE_BITS, XT, ST, true, GSH>), dim3(grid), dim3(256), 0, st,
                          ev.start, ev.stop, 0, a);
  else
    hipExtLaunchKernelGGL((gemv_mma_kernel<MOE_BITS, XT, ST, false, GSH>), dim3(grid), dim3(256), 0, st,
                          ev.start, ev.stop, 0, a);
  return hipGetLastError();
}

hipError_t MOE_CAT(launch_mma_b, MOE_BITS)(int xdt, int sbdt, bool gateup, const GemvArgs& a,
                                            int grid, hipStream_t st, KEvents ev) {
#define MOE_MMA(XT, ST)                                                \
  switch (a.gsh) {                                                     \
    case 0: return launch_mma_g<XT, ST, 0>(gateup, a, grid, st, ev);   \
    case 1: return launch_mma_g<XT, ST, 1>(gateup, a, grid, st, ev);   \
    case 2: return launch_mma_g<XT, ST, 2>(gateup, a, grid, st, ev);   \
    default: return hipErrorInvalidValue;                              \
  }
  if (xdt == DT_BF16 && sbdt == DT_BF16) { MOE_MMA(bf16_t, bf16_t) }
  if (xdt == DT_BF16 && sbdt == DT_F16) { MOE_MMA(bf16_t, f16_t) }
  if (xdt == DT_F16 && sbdt == DT_F16) { MOE_MMA(f16_t, f16_t) }
  if (xdt == DT_F16 && sbdt == DT_BF16) { MOE_MMA(f16_t, bf16_t) }
#undef MOE_MMA
  return hipErrorInvalidValue;
}
#endif  // MOE_BITS <= 6

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
  const int N = a.N, K = a.K, CU = K >> 5, groups = CU >> a.gsh, row_words = CU * BITS;
  const int r_begin = rb * a.rows_per_block;
  const int r_end = min(N, r_begin + a.rows_per_block);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nwaves = blockDim.x >> 6;
  const int L = 1 << a.lg, SG = 64 >> a.lg;
  const int sg = lane >> a.lg, li = lane & (L - 1);
  const GemvProj p0 = expert_proj<BITS, ST>(a.p0, e, N, row_words, groups);
  const GemvProj p1 = expert_proj<BITS, ST>(a.p1, e, N, row_words, groups);
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
    const uint32_t row = (uint32_t)r;
    WUnit<BITS, ST> w0[UR], w1[UR];
#pragma unroll
    for (int j = 0; j < UR; j++) {
      const int u = li + j * L;
      if (u < CU) {
        load_w_unit<BITS, ST>(p0, row, row_words, groups, a.gsh, u, w0[j]);
        if constexpr (GATEUP) load_w_unit<BITS, ST>(p1, row, row_words, groups, a.gsh, u, w1[j]);
      }
    }
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int j = 0; j < UR; j++) {
      const int u = li + j * L;
      if (u < CU) {
        uint32_t cp[16];
        unpack_pairs<BITS, Magic<BITS, XT>::bits>(w0[j].w, cp);
        acc0 += w0[j].s() * dot_unit<BITS, XT>(cp, xu[j]) + (w0[j].b() - MAGIC * w0[j].s()) * xs[j];
        if constexpr (GATEUP) {
          unpack_pairs<BITS, Magic<BITS, XT>::bits>(w1[j].w, cp);
          acc1 += w1[j].s() * dot_unit<BITS, XT>(cp, xu[j]) + (w1[j].b() - MAGIC * w1[j].s()) * xs[j];
        }
      }
    }
    acc0 = wave_sum_width(acc0, L);
    if constexpr (GATEUP) acc1 = wave_sum_width(acc1, L);
    if (li == 0) {
      const size_t o = (size_t)p * N + r;
      const float g = finish_proj<XT>(acc0, a.p0.ob, ebase + r);
      if constexpr (GATEUP) {
        const float u = finish_proj<XT>(acc1, a.p1.ob, ebase + r);
        out[o] = from_f<XT>(apply_act<XT>(g, u, a.act, a.alpha, a.limit));
      } else {
        out[o] = from_f<XT>(a.act == ACT_RELU2 ? apply_act<XT>(0.f, g, ACT_RELU2, 0.f, 0.f) : g);
      }
    }
  }
}

// ---------------------------------------------------------------------------
// decode of one token in two launches: gate/up with in-wave routing, then
// down + combine
// ---------------------------------------------------------------------------

// gate/up for one token. Block (slot, rb): the slot-th smallest selected
// expert, rows [rb * rows_per_block, ...). Wave w, sub-group sg owns rows
// r_begin + w SG + sg + it 4 SG for it < RM; every load of those rows is
// issued before the first dot product. The routing runs once per block, in
// wave 0, with the logits as its first load, while the other waves copy the
// activation row into LDS once; each lane reads its units from there after
// its weight loads are in flight (per-lane global loads of the same row
// would occupy the CU's load path for about a microsecond before routing).
// The shared expert's sigmoid gate logit, round(x . w) over one dense row in
// the activation dtype: each thread takes 8-value pieces in index order,
// then the sums go through a fixed DPP tree and the four waves in order.
template <typename XT>
__device__ void shared_gate_logit(const XT* x, const XT* w, int K, XT* out) {
  __shared__ float part[4];
  const rsrc_t xr = make_rsrc(x, (uint32_t)(K * sizeof(XT)));
  const rsrc_t wr = make_rsrc(w, (uint32_t)(K * sizeof(XT)));
  float acc = 0.f;
#pragma unroll 1
  for (int c = threadIdx.x; c < K / 8; c += blockDim.x) {
    const u32x4_t xv = bload128(xr, (uint32_t)c * 16u), wv = bload128(wr, (uint32_t)c * 16u);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      acc = fmaf(to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(xv[q] & 0xFFFFu))),
                 to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(wv[q] & 0xFFFFu))), acc);
      acc = fmaf(to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(xv[q] >> 16))),
                 to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(wv[q] >> 16))), acc);
    }
  }
  acc = group_sum(acc, 6);
  if ((threadIdx.x & 63) == 63) part[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    float t = 0.f;
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) t += part[i];
    out[0] = from_f<XT>(t);
  }
}

template <int BITS, typename XT, typename ST, int UR, int RM, int EPL, bool SH>
__global__ __launch_bounds__(256) void gateup1_kernel(const Decode1Args a) {
  __shared__ float sc[kTopkMaxE];
  __shared__ int route[2];
  __shared__ __align__(16) uint32_t xl[kDec1MaxHidden / 2];
  __shared__ float xsm[kDec1MaxHidden / 32];
  const int routed_blocks = a.k * a.row_blocks;
  // the shared expert's gate logit block (the last, with a dense gate row)
  if (SH && a.sgw && (int)blockIdx.x == routed_blocks + a.s_blocks) {
    shared_gate_logit<XT>(reinterpret_cast<const XT*>(a.x), reinterpret_cast<const XT*>(a.sgw),
                          a.K, reinterpret_cast<XT*>(a.s_logit));
    return;
  }
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // scalar branches below
  const int t = blockIdx.y;  // the token (a shared expert in the launch: T = 1)
  // blocks from routed_blocks on hold rows of the shared expert (expert 0 of
  // its one-expert projections); the rest a slot of the routed experts
  const bool shb = SH && (int)blockIdx.x >= routed_blocks;
  const int slot = shb ? 0 : (int)blockIdx.x / a.row_blocks;
  const int rb = shb ? (int)blockIdx.x - routed_blocks : (int)blockIdx.x - slot * a.row_blocks;
  const int N = shb ? a.SN : a.N;
  const int K = a.K, CU = K >> 5, groups = CU >> a.gsh, row_words = CU * BITS;
  const int L = 1 << a.lg, SG = 64 >> a.lg;
  const int sg = lane >> a.lg, li = lane & (L - 1);
  const int r_begin = rb * a.rows_per_block;
  const int r_end = min(N, r_begin + a.rows_per_block);
  const int r0 = r_begin + wave * SG + sg, stride = 4 * SG;
  const GemvProj pg = shb ? a.sg : a.g, pu = shb ? a.su : a.u;
  const XT* ob_g = reinterpret_cast<const XT*>(pg.ob);
  const XT* ob_u = reinterpret_cast<const XT*>(pu.ob);

  // wave 0 routes the token (every block computes identical, deterministic
  // results); block 0 publishes the routing. Meanwhile the other waves stage
  // the activation row in LDS in pair order with its unit sums, so that the
  // lanes' dot products after the weight stream read their units as they are.
  if (wave != 0)
    stage_x_pairs<BITS, XT, 2>([&](int) { return reinterpret_cast<const XT*>(a.x) + (size_t)t * K; },
                               1, K, xl, xsm, threadIdx.x - 64, blockDim.x - 64);
  if (wave == 0 && shb) {
    if (lane == 0) {
      route[0] = 0;
      route[1] = 0;
    }
  } else if (wave == 0) {
    const bool writer = blockIdx.x == 0;
    int sel;
    float wgt = 0.f;
    uint64_t masks[kTopkEPL];
    wave_topk<XT, EPL>(reinterpret_cast<const XT*>(a.logits) + (size_t)t * a.E, a.E, a.k, a.ro, sc,
                       writer, &sel, &wgt, masks);
    const int e = __builtin_amdgcn_readfirstlane(selected_nth(masks, slot));
    const uint64_t hit = __ballot(lane < a.k && sel == e);
    if (lane == 0) {
      route[0] = e;
      route[1] = __ffsll((unsigned long long)hit) - 1;
    }
    if (writer) {
      if (lane < a.k) {
        a.idx[t * a.k + lane] = (uint32_t)sel;
        a.w[t * a.k + lane] = wgt;
        if (a.perm) a.perm[selected_below(masks, sel)] = (uint32_t)lane;
      }
      if (a.offsets)
        for (int ee = lane; ee <= a.E; ee += 64) a.offsets[ee] = (uint32_t)selected_below(masks, ee);
    }
  }
  __syncthreads();
  const int e = __builtin_amdgcn_readfirstlane(route[0]);
  const int rank = __builtin_amdgcn_readfirstlane(route[1]);

  // output biases first (a missing one through an empty view, which reads
  // zero), kept raw until every weight load is out: converting them here
  // would wait for them, and for every load issued before them, ahead of the
  // weight stream
  uint16_t obg_raw[RM], obu_raw[RM];
  {
    const rsrc_t gr = make_rsrc(ob_g ? ob_g + (size_t)e * N : nullptr, ob_g ? (uint32_t)(N * sizeof(XT)) : 0u);
    const rsrc_t ur = make_rsrc(ob_u ? ob_u + (size_t)e * N : nullptr, ob_u ? (uint32_t)(N * sizeof(XT)) : 0u);
#pragma unroll
    for (int it = 0; it < RM; it++) {
      const uint32_t off = (uint32_t)min(r0 + it * stride, N - 1) * (uint32_t)sizeof(XT);
      obg_raw[it] = bload16(gr, off);
      obu_raw[it] = bload16(ur, off);
    }
  }
  // squared-ReLU experts have no gate projection (g.w null): the gate reads
  // go to empty buffer views, which return zeros without touching memory
  // (no branch around the loads), and the activation reads u only
  const ProjView U = proj_view<BITS, ST>(pu, (uint32_t)e, N, row_words, groups);
  const rsrc_t none = make_rsrc(pu.w, 0u);
  const ProjView G = pg.w ? proj_view<BITS, ST>(pg, (uint32_t)e, N, row_words, groups)
                          : ProjView{none, none, none};
  const uint32_t wstep = (uint32_t)(L * BITS * 4), sstep = (uint32_t)((L >> a.gsh) * sizeof(ST));
  WUnit<BITS, ST> gw[RM][UR], uw[RM][UR];
#pragma unroll
  for (int it = 0; it < RM; it++) {
    const UnitAddr ad = unit_addr<BITS, ST>((uint32_t)(r0 + it * stride), row_words, groups, li, a.gsh);
    bload_units<BITS, ST, UR, kStream>(G, ad, wstep, sstep, gw[it]);
    bload_units<BITS, ST, UR, kStream>(U, ad, wstep, sstep, uw[it]);
  }
  // every weight load is issued before the first dot product: without the
  // fence the scheduler interleaves loads with math to save registers, and
  // each wave then waits out the memory latency more than once
  __builtin_amdgcn_sched_barrier(0);
  XUnit<XT> xu[UR];
  float xs[UR];
  lds_x_units_pairs<XT, UR>(xl, xsm, 0, li, L, CU, xu, xs);

  XT* act = shb ? reinterpret_cast<XT*>(a.s_act)
                : reinterpret_cast<XT*>(a.act) + ((size_t)t * a.k + rank) * N;
#pragma unroll
  for (int it = 0; it < RM; it++) {
    float g = group_sum(dot_units<BITS, XT, ST, UR>(gw[it], xu, xs, li, L, CU), a.lg);
    float u = group_sum(dot_units<BITS, XT, ST, UR>(uw[it], xu, xs, li, L, CU), a.lg);
    const int row = r0 + it * stride;
    if (li == L - 1 && row < r_end) {
      g = round_to<XT>(g);
      u = round_to<XT>(u);
      if (ob_g) g = round_to<XT>(g + to_f<XT>(__builtin_bit_cast(XT, obg_raw[it])));
      if (ob_u) u = round_to<XT>(u + to_f<XT>(__builtin_bit_cast(XT, obu_raw[it])));
      act[row] = from_f<XT>(apply_act<XT>(g, u, a.act_kind, a.alpha, a.limit));
    }
  }
}

// down projection + weighted combine for one token. Block = k waves (SH:
// k + m); wave q < k takes the rank-q expert and its activation row
// (registers, pair order), wave k + j the j-th column slice of the shared
// expert, and all waves share the block's rows: sub-group sg owns rows
// r_begin + sg + it SG for it < RM. Each routed expert's output is rounded
// to the activation dtype (then its output bias added and rounded) before it
// is weighted, as the unfused path stores it (MoELayer.swift:895-939); the
// weighted outputs are added in rank order. The shared expert's slices are
// summed in fp32 and rounded once, then added to the rounded routed sum with
// its gate weight, as the shared add does after a separate shared expert.
template <int BITS, typename XT, typename ST, int UR, int RM, bool SH>
__global__ __launch_bounds__(SH ? 64 * kDec1MaxWaves : 64 * kDec1MaxK) void down1_kernel(
    const Down1Args a) {
  __shared__ float ys[(SH ? kDec1MaxWaves : kDec1MaxK) * kDec1MaxRows * 64];
  __shared__ float wr[kDec1MaxK];
  // wave-uniform by construction; readfirstlane tells the compiler, so the
  // buffer resources built from it stay scalar
  const int lane = threadIdx.x & 63, q = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int N = a.N, K = a.K, CU = K >> 5, groups = CU >> a.gsh, row_words = CU * BITS;
  const int L = 1 << a.lg, SG = 64 >> a.lg;
  const int sg = lane >> a.lg, li = lane & (L - 1);
  const int rpb = a.rows_per_block;  // RM * SG
  const int r_begin = blockIdx.x * rpb;
  const bool shw = SH && q >= a.k;  // a shared-expert wave
  const int j = q - a.k;            // its column slice
  const int t = blockIdx.y;         // the token (a shared expert in the launch: T = 1)
  const XT* ob = reinterpret_cast<const XT*>(a.p.ob);

  // The activation units go out first: they need no routing, and their
  // conversion to pair order then runs while the weights stream instead of
  // after them (loads complete in issue order).
  const XT* act = shw ? reinterpret_cast<const XT*>(a.s_act) + (size_t)j * K
                      : reinterpret_cast<const XT*>(a.act) + ((size_t)t * a.k + q) * K;
  u32x4_t xraw[UR][4];
  {
    const rsrc_t xr = make_rsrc(act, (uint32_t)(K * sizeof(XT)));
#pragma unroll
    for (int jj = 0; jj < UR; jj++)
#pragma unroll
      for (int q4 = 0; q4 < 4; q4++) xraw[jj][q4] = bload128(xr, (uint32_t)(li + jj * L) * 64u + 16u * q4);
  }
  __builtin_amdgcn_sched_barrier(0);

  uint32_t e = 0;
  ProjView P;
  UnitAddr base{0u, 0u};
  int rw = row_words, grp = groups;
  // output biases kept raw until the weight loads are out (converting them
  // here would wait for them, and for the activation loads before them,
  // ahead of the weight stream); shared waves and a missing bias read zero
  // through an empty view
  uint16_t obraw[RM];
  if (shw) {
    rw = a.m * row_words;
    grp = a.m * groups;
    P = proj_view<BITS, ST>(a.sp, 0u, N, rw, grp);
    base.w0 = (uint32_t)(j * row_words * 4);
    base.s0 = (uint32_t)(j * groups * (int)sizeof(ST));
#pragma unroll
    for (int it = 0; it < RM; it++) obraw[it] = 0;
  } else {
    e = __builtin_amdgcn_readfirstlane(a.idx[t * a.k + q]);
    if (lane == 0) wr[q] = round_to<XT>(a.w[t * a.k + q]);
    const rsrc_t obr = make_rsrc(ob ? ob + (size_t)e * N : nullptr, ob ? (uint32_t)(N * sizeof(XT)) : 0u);
#pragma unroll
    for (int it = 0; it < RM; it++)
      obraw[it] = bload16(obr, (uint32_t)min(r_begin + sg + it * SG, N - 1) * (uint32_t)sizeof(XT));
    P = proj_view<BITS, ST>(a.p, e, N, row_words, groups);
  }
  const uint32_t wstep = (uint32_t)(L * BITS * 4), sstep = (uint32_t)((L >> a.gsh) * sizeof(ST));
  WUnit<BITS, ST> w[RM][UR];
#pragma unroll
  for (int it = 0; it < RM; it++) {
    UnitAddr ad = unit_addr<BITS, ST>((uint32_t)(r_begin + sg + it * SG), rw, grp, li, a.gsh);
    ad.w0 += base.w0;
    ad.s0 += base.s0;
    bload_units<BITS, ST, UR, kStream>(P, ad, wstep, sstep, w[it]);
  }
  __builtin_amdgcn_sched_barrier(0);  // all loads in flight before the conversion and the math
  XUnit<XT> xu[UR];
  float xs[UR];
#pragma unroll
  for (int jj = 0; jj < UR; jj++) {
    uint32_t n[16];
#pragma unroll
    for (int q4 = 0; q4 < 4; q4++) {
      n[4 * q4] = xraw[jj][q4][0]; n[4 * q4 + 1] = xraw[jj][q4][1];
      n[4 * q4 + 2] = xraw[jj][q4][2]; n[4 * q4 + 3] = xraw[jj][q4][3];
    }
    natural_to_pairs<BITS>(n, xu[jj].v);
    xs[jj] = sum16(n, __is_same(XT, bf16_t));
  }
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int it = 0; it < RM; it++) {
    float y = group_sum(dot_units<BITS, XT, ST, UR>(w[it], xu, xs, li, L, CU), a.lg);
    if (!shw) {
      y = round_to<XT>(y);
      if (ob) y = round_to<XT>(y + to_f<XT>(__builtin_bit_cast(XT, obraw[it])));
    }
    if (li == L - 1) ys[q * rpb + sg + it * SG] = y;
  }
  __syncthreads();
  XT* out = reinterpret_cast<XT*>(a.out) + (size_t)t * N;
  const XT* res = a.res ? reinterpret_cast<const XT*>(a.res) + (size_t)t * N : nullptr;
  const XT* sob = reinterpret_cast<const XT*>(a.sp.ob);
  const float gate = (SH && a.s_logit)
                         ? 1.0f / (1.0f + __expf(-to_f<XT>(reinterpret_cast<const XT*>(a.s_logit)[0])))
                         : 1.0f;
  for (int t = threadIdx.x; t < rpb; t += blockDim.x) {
    const int row = r_begin + t;
    if (row >= N) break;
    float acc = 0.f;
    for (int qq = 0; qq < a.k; qq++) acc += wr[qq] * ys[qq * rpb + t];
    if constexpr (SH) {
      float sv = 0.f;
      for (int jj = 0; jj < a.m; jj++) sv += ys[(a.k + jj) * rpb + t];
      sv = round_to<XT>(sv);
      if (sob) sv = round_to<XT>(sv + to_f<XT>(sob[row]));
      acc = round_to<XT>(acc);
      if (res) acc = to_f<XT>(res[row]) + acc;
      acc = acc + gate * sv;
    } else {
      if (res) acc = to_f<XT>(res[row]) + round_to<XT>(acc);
    }
    out[row] = from_f<XT>(acc);
  }
}

template <int BITS, typename XT, typename ST, int UR, int RM, bool SH>
static hipError_t launch_gateup1_e(int E, const Decode1Args& a, int grid, hipStream_t st,
                                   KEvents ev) {
  if (E <= 64)
    hipExtLaunchKernelGGL((gateup1_kernel<BITS, XT, ST, UR, RM, 1, SH>), dim3(grid, a.T), dim3(256), 0,
                          st, ev.start, ev.stop, 0, a);
  else if (E <= 128)
    hipExtLaunchKernelGGL((gateup1_kernel<BITS, XT, ST, UR, RM, 2, SH>), dim3(grid, a.T), dim3(256), 0,
                          st, ev.start, ev.stop, 0, a);
  else
    hipExtLaunchKernelGGL((gateup1_kernel<BITS, XT, ST, UR, RM, kTopkEPL, SH>), dim3(grid, a.T),
                          dim3(256), 0, st, ev.start, ev.stop, 0, a);
  return hipGetLastError();
}

template <int BITS, typename XT, typename ST, int UR>
static hipError_t launch_dec1_u(bool down, int var, const void* args, int grid, size_t smem,
                                hipStream_t st, KEvents ev) {
  (void)smem;
  if (!down) {
    const Decode1Args& a = *reinterpret_cast<const Decode1Args*>(args);
    const bool sh = a.s_blocks > 0;
    switch (var) {
      case 1: return sh ? launch_gateup1_e<BITS, XT, ST, UR, 1, true>(a.E, a, grid, st, ev)
                        : launch_gateup1_e<BITS, XT, ST, UR, 1, false>(a.E, a, grid, st, ev);
      case 2: return sh ? launch_gateup1_e<BITS, XT, ST, UR, 2, true>(a.E, a, grid, st, ev)
                        : launch_gateup1_e<BITS, XT, ST, UR, 2, false>(a.E, a, grid, st, ev);
      default: return hipErrorInvalidValue;
    }
  }
  const Down1Args& a = *reinterpret_cast<const Down1Args*>(args);
  const bool sh = a.m > 0;
  const dim3 block(64 * (a.k + a.m));
#define MOE_DN(RM)                                                                           \
  if (sh)                                                                                    \
    hipExtLaunchKernelGGL((down1_kernel<BITS, XT, ST, UR, RM, true>), dim3(grid, a.T), block, 0, \
                          st, ev.start, ev.stop, 0, a);                                      \
  else                                                                                       \
    hipExtLaunchKernelGGL((down1_kernel<BITS, XT, ST, UR, RM, false>), dim3(grid, a.T), block, 0, \
                          st, ev.start, ev.stop, 0, a);
  switch (var) {
    case 1: MOE_DN(1) break;
    case 2: MOE_DN(2) break;
    default: return hipErrorInvalidValue;
  }
#undef MOE_DN
  return hipGetLastError();
}

template <int BITS, typename XT, typename ST>
static hipError_t launch_dec1_t(bool down, int var, int ur, const void* args, int grid, size_t smem,
                                hipStream_t st, KEvents ev) {
  switch (ur) {
    case 1: return launch_dec1_u<BITS, XT, ST, 1>(down, var, args, grid, smem, st, ev);
    case 2: return launch_dec1_u<BITS, XT, ST, 2>(down, var, args, grid, smem, st, ev);
    case 3: return launch_dec1_u<BITS, XT, ST, 3>(down, var, args, grid, smem, st, ev);
    case 4: return launch_dec1_u<BITS, XT, ST, 4>(down, var, args, grid, smem, st, ev);
  }
  return hipErrorInvalidValue;
}

// var: rows per lane (1..kDec1MaxRows).
template <int BITS>
static hipError_t launch_dec1_bits(int xdt, int sbdt, bool down, int var, int ur, const void* args,
                                   int grid, size_t smem, hipStream_t st, KEvents ev = {}) {
  if (xdt == DT_BF16 && sbdt == DT_BF16) return launch_dec1_t<BITS, bf16_t, bf16_t>(down, var, ur, args, grid, smem, st, ev);
  if (xdt == DT_BF16 && sbdt == DT_F16) return launch_dec1_t<BITS, bf16_t, f16_t>(down, var, ur, args, grid, smem, st, ev);
  if (xdt == DT_F16 && sbdt == DT_F16) return launch_dec1_t<BITS, f16_t, f16_t>(down, var, ur, args, grid, smem, st, ev);
  if (xdt == DT_F16 && sbdt == DT_BF16) return launch_dec1_t<BITS, f16_t, bf16_t>(down, var, ur, args, grid, smem, st, ev);
  return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------

template <int BITS, typename XT, typename ST>
static hipError_t launch_gemv_t(bool gateup, int tokmax, const GemvArgs& a, int grid,
                                hipStream_t st, KEvents ev) {
  if (tokmax <= 1) {
    if (gateup)
      hipExtLaunchKernelGGL((gemv_single_kernel<BITS, XT, ST, true>), dim3(grid), dim3(256), 0, st,
                            ev.start, ev.stop, 0, a);
    else
      hipExtLaunchKernelGGL((gemv_single_kernel<BITS, XT, ST, false>), dim3(grid), dim3(256), 0, st,
                            ev.start, ev.stop, 0, a);
  } else {
    const uint32_t smem = (uint32_t)gemv_smem_bytes(__is_same(XT, float) ? DT_F32 : DT_BF16, a.K,
                                                    a.tok_chunk);
    if (gateup)
      hipExtLaunchKernelGGL((gemv_grouped_kernel<BITS, XT, ST, true, 8>), dim3(grid), dim3(256),
                            smem, st, ev.start, ev.stop, 0, a);
    else
      hipExtLaunchKernelGGL((gemv_grouped_kernel<BITS, XT, ST, false, 8>), dim3(grid), dim3(256),
                            smem, st, ev.start, ev.stop, 0, a);
  }
  return hipGetLastError();
}

// gemv_multi_kernel: ur = units per lane (1..4), tm = rows per pass (4 or 8),
// kMultiRows(gate/up) weight rows per lane, smem = tm * (K / 32) * 68 bytes.
template <int BITS, typename XT, typename ST, bool GU, int UR>
static hipError_t launch_multi_u(int tm, const GemvArgs& a, int grid, size_t smem, hipStream_t st,
                                 KEvents ev) {
  constexpr int RM = kMultiRows(GU);
  if (tm <= 4)
    hipExtLaunchKernelGGL((gemv_multi_kernel<BITS, XT, ST, GU, UR, RM, 4>), dim3(grid), dim3(256),
                          (uint32_t)smem, st, ev.start, ev.stop, 0, a);
  else
    hipExtLaunchKernelGGL((gemv_multi_kernel<BITS, XT, ST, GU, UR, RM, 8>), dim3(grid), dim3(256),
                          (uint32_t)smem, st, ev.start, ev.stop, 0, a);
  return hipGetLastError();
}

template <int BITS, typename XT, typename ST>
static hipError_t launch_multi_t(bool gateup, int ur, int tm, const GemvArgs& a, int grid,
                                 size_t smem, hipStream_t st, KEvents ev) {
#define MOE_MU(UR)                                                                     \
  case UR:                                                                             \
    return gateup ? launch_multi_u<BITS, XT, ST, true, UR>(tm, a, grid, smem, st, ev)  \
                  : launch_multi_u<BITS, XT, ST, false, UR>(tm, a, grid, smem, st, ev);
  switch (ur) { MOE_MU(1) MOE_MU(2) MOE_MU(3) MOE_MU(4) }
#undef MOE_MU
  return hipErrorInvalidValue;
}

template <int BITS>
static hipError_t launch_multi_bits(int xdt, int sbdt, bool gateup, int ur, int tm,
                                    const GemvArgs& a, int grid, size_t smem, hipStream_t st,
                                    KEvents ev) {
  if (xdt == DT_BF16 && sbdt == DT_BF16) return launch_multi_t<BITS, bf16_t, bf16_t>(gateup, ur, tm, a, grid, smem, st, ev);
  if (xdt == DT_BF16 && sbdt == DT_F16) return launch_multi_t<BITS, bf16_t, f16_t>(gateup, ur, tm, a, grid, smem, st, ev);
  if (xdt == DT_F16 && sbdt == DT_F16) return launch_multi_t<BITS, f16_t, f16_t>(gateup, ur, tm, a, grid, smem, st, ev);
  if (xdt == DT_F16 && sbdt == DT_BF16) return launch_multi_t<BITS, f16_t, bf16_t>(gateup, ur, tm, a, grid, smem, st, ev);
  return hipErrorInvalidValue;
}

template <int BITS>
static hipError_t launch_gemv_bits(int xdt, int sbdt, bool gateup, int tokmax, const GemvArgs& a,
                                   int grid, hipStream_t st, KEvents ev) {
  if (xdt == DT_BF16 && sbdt == DT_BF16) return launch_gemv_t<BITS, bf16_t, bf16_t>(gateup, tokmax, a, grid, st, ev);
  if (xdt == DT_BF16 && sbdt == DT_F16) return launch_gemv_t<BITS, bf16_t, f16_t>(gateup, tokmax, a, grid, st, ev);
  if (xdt == DT_F16 && sbdt == DT_F16) return launch_gemv_t<BITS, f16_t, f16_t>(gateup, tokmax, a, grid, st, ev);
  if (xdt == DT_F16 && sbdt == DT_BF16) return launch_gemv_t<BITS, f16_t, bf16_t>(gateup, tokmax, a, grid, st, ev);
  if (xdt == DT_F32 && sbdt == DT_F32) return launch_gemv_t<BITS, float, float>(gateup, tokmax, a, grid, st, ev);
  return hipErrorInvalidValue;
}

// One translation unit per bit width (MOE_BITS) keeps compile times short;
// the per-width entry points are stitched together in api.cpp.

hipError_t MOE_CAT(launch_gemv_b, MOE_BITS)(int xdt, int sbdt, bool gateup, int tokmax,
                                             const GemvArgs& a, int grid, hipStream_t st,
                                             KEvents ev) {
  return launch_gemv_bits<MOE_BITS>(xdt, sbdt, gateup, tokmax, a, grid, st, ev);
}

hipError_t MOE_CAT(launch_multi_b, MOE_BITS)(int xdt, int sbdt, bool gateup, int ur, int tm,
                                              const GemvArgs& a, int grid, size_t smem,
                                              hipStream_t st, KEvents ev) {
  return launch_multi_bits<MOE_BITS>(xdt, sbdt, gateup, ur, tm, a, grid, smem, st, ev);
}

hipError_t MOE_CAT(launch_dec1_b, MOE_BITS)(int xdt, int sbdt, bool down, int rm, int ur,
                                             const void* args, int grid, size_t smem,
                                             hipStream_t st, KEvents ev) {
  return launch_dec1_bits<MOE_BITS>(xdt, sbdt, down, rm, ur, args, grid, smem, st, ev);
}

}  // namespace moe
