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
// Work: a tile list of (expert, up to 256 consecutive sorted positions; the
// last tile of an expert with at most 128 rows is a half tile); block = one
// tile x one column slice (256 weight rows). Per 64-value chunk of K the
// block stages the tile's activation rows and the slice's weights,
// dequantised once per block to the MFMA operand type, in double-buffered
// LDS; 8 waves multiply with v_mfma_f32_32x32x16 (see the kernel comment).
// Dequantisation: codes -> fp32 (exact) -> s*q + b (fp32) -> bf16 / f16.
//
// K order inside a 64-value chunk: lane half h of the wave takes values
// [32h, 32h + 32) — one whole 32-value unit — and step s (0..3) of the
// 16-deep MFMA reduction feeds values 16 s + 8 h + e, e < 8 (LDS chunk
// 2 s + h of the row); A and B fragments are read in the same order.
#include <hip/hip_ext.h>

#include <type_traits>

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

constexpr int kGBK = 64;  // values per K chunk

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
  if constexpr (BITS == 16) {
    // plain weights already in the operand type
    (void)sc;
    (void)bi;
    return __builtin_bit_cast(typename MfmaOp<XT>::V, u32x4_t{w[4 * s], w[4 * s + 1], w[4 * s + 2], w[4 * s + 3]});
  }
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

// LDS tile of 256 rows x 64 values (16-bit), 128 B per row. The banks
// repeat every 256 B (two rows) and a 16-byte read serves 16 lanes per
// cycle, so the 16-byte chunk c of row r sits at slot c ^ ((r >> 1) & 7):
// 16 consecutive rows reading the same chunk then cover every bank once.
constexpr int kTR = 256;
__device__ __forceinline__ int tile_swz(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ uint32_t tile_off(int r, int c) {
  return (uint32_t)(r * 128 + ((c ^ tile_swz(r)) << 4));
}

// Block tile: 256 rows x 256 weight rows (gate/up: 128 output columns of
// gate and of up; otherwise 256 output columns), 8 waves in a 4 x 2 grid:
// wave (wm, wn) owns rows [64 wm, +64) as 2 MFMA row tiles and 4 MFMA column
// tiles (gate/up: gate columns [64 wn, +64) and the matching up columns), so
// its accumulators fit 128 registers and two waves share each SIMD. Row
// tiles past the expert's last position skip their MFMAs. A half tile (the
// last tile of an expert, at most 128 rows) gives each wave the 32-row band
// [32 wm, +32) instead, so its rows are spread over all four SIMDs.
//
// Per 64-value chunk: every thread copies 64 bytes of activation rows and
// dequantises one 32-value unit of one weight row into LDS, once for the
// whole block, and each wave runs 4 steps x 8 v_mfma_f32_32x32x16. Global
// loads run two chunks ahead of the MFMAs; chunk c + 1 is written to LDS
// (its weights dequantised between the MFMA steps) while chunk c is
// multiplied.
// All operand rows of a lane are congruent mod 16, so one swizzled chunk
// offset per step serves every LDS read (immediate row offsets).
template <int BITS, typename XT, typename ST, bool GATEUP>
__global__ __launch_bounds__(512) void gemm_grouped_kernel(const GemmArgs a) {
  __shared__ __align__(16) unsigned char As[2][kTR * 128];
  __shared__ __align__(16) unsigned char Bs[2][kTR * 128];
  typedef typename MfmaOp<XT>::V V;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int ncols = GATEUP ? 128 : 256;  // output columns per block
  const int n_tiles = (a.N + ncols - 1) / ncols;

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
  const uint32_t ef = __builtin_amdgcn_readfirstlane(a.tiles[1 + 2 * tile]);
  const uint32_t e = ef & ~kHalfTile;
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(a.tiles[2 + 2 * tile]);
  // rows per wave band: 64 (two MFMA row tiles) in a full 256-row tile, 32
  // (one) in a half tile, so that all four SIMDs share a short tile's rows
  const int band = (ef & kHalfTile) ? 32 : 64;
  const uint32_t pend = __builtin_amdgcn_readfirstlane(a.offsets[e + 1]);

  const int N = a.N, K = a.K, CU = K >> 5, groups = CU >> a.gsh, row_words = CU * BITS;
  const int nchunks = K / kGBK;

  // ---- activation rows: thread (wave, lane) copies, for i < 4, 16 bytes
  // of LDS row 32 wave + 8 i + lane / 8, slot lane % 8 (logical chunk
  // (lane % 8) ^ tile_swz(row)); two register sets keep chunk c + 2 in flight
  // one wave-uniform buffer resource over all activation rows; per-lane
  // 32-bit byte offsets of the four rows this lane copies
  const rsrc_t xr = make_rsrc(a.x, (uint32_t)min((size_t)a.x_rows * K * sizeof(XT), (size_t)0xFFFFFFFFu));
  uint32_t xoff[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 32 * wave + 8 * i + (lane >> 3);
    const uint32_t p = min(m0 + (uint32_t)r, pend - 1);
    const uint32_t xrow = a.perm ? a.perm[p] / (uint32_t)a.topk : p;
    const int c = (lane & 7) ^ tile_swz(r);
    xoff[i] = (xrow * (uint32_t)K + (uint32_t)(8 * c)) * (uint32_t)sizeof(XT);
  }
  // LDS byte offset of load i: row 32 wave + 8 i + lane / 8, slot lane % 8
  const uint32_t aoff0 = (uint32_t)((32 * wave + (lane >> 3)) * 128 + ((lane & 7) << 4));
  struct ARegs {
    u32x4_t v[4];
  };
  auto load_a = [&](int chunk, ARegs& ar) {
#pragma unroll
    for (int i = 0; i < 4; i++)
      ar.v[i] = bload128(xr, xoff[i] + (uint32_t)(chunk * kGBK * (int)sizeof(XT)));
  };
  auto store_a = [&](const ARegs& ar, int buf) {
#pragma unroll
    for (int i = 0; i < 4; i++) *reinterpret_cast<u32x4_t*>(&As[buf][aoff0 + 1024 * i]) = ar.v[i];
  };

  // ---- weights: thread t dequantises unit t % 2 (values [32 (t % 2), +32)
  // of the chunk) of LDS weight row t / 2
  const int brl = threadIdx.x >> 1, bu = threadIdx.x & 1;
  const bool upper = GATEUP && wave >= 4;  // LDS rows 128..255 hold up (wave-uniform)
  const int wrow = GATEUP ? bn * 128 + (brl & 127) : bn * 256 + brl;
  const uint32_t brow = (uint32_t)min(wrow, N - 1);
  const ProjViewG PB = proj_view_g<BITS, ST>(upper ? a.p1 : a.p0, e, N, row_words, groups);
  // packed codes, scale and bias of one unit: two register sets so that
  // chunk c + 2 is in flight while chunk c + 1 is dequantised
  struct BUnit {
    uint32_t w[BITS];
    ST s, b;
  };
  auto load_b = [&](int chunk, BUnit& u) {
    const int unit = 2 * chunk + bu;
    bload_unit<BITS>(PB.w, (brow * (uint32_t)row_words + (uint32_t)(unit * BITS)) * 4u, u.w);
    if constexpr (BITS != 16) {
      const uint32_t gi = brow * (uint32_t)groups + (uint32_t)(unit >> a.gsh);
      u.s = __builtin_bit_cast(ST, bload16(PB.s, gi * (uint32_t)sizeof(ST)));
      u.b = __builtin_bit_cast(ST, bload16(PB.b, gi * (uint32_t)sizeof(ST)));
    }
  };
  // 8 values [8 s, 8 s + 8) of the unit -> LDS chunk 4 bu + s
  auto store_b = [&](const BUnit& u, int s, int buf) {
    const V v = BITS == 16 ? dequant8<BITS, XT>(u.w, s, 0.f, 0.f)
                           : dequant8<BITS, XT>(u.w, s, to_f<ST>(u.s), to_f<ST>(u.b));
    *reinterpret_cast<V*>(&Bs[buf][tile_off(brl, 4 * bu + s)]) = v;
  };

  f32x16_t acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 4; j++) acc[i][j] = f32x16_t{};

  // row tiles of this wave's band that hold positions of the expert
  const uint32_t bstart = m0 + (uint32_t)(band * wm);
  const int mvalid = (bstart >= pend) ? 0 : (band == 32 || bstart + 32u >= pend) ? 1 : 2;

  // MFMA operand rows of this lane: A rows band wm + 32 i + col, B rows
  // (gate/up) 64 wn + 32 j + col and 128 + 64 wn + 32 (j - 2) + col, or
  // 128 wn + 32 j + col; all congruent to col mod 16, so they share
  // tile_swz(col)
  const int col = lane & 31, h = lane >> 5;
  const uint32_t arow0 = (uint32_t)(band * wm + col) * 128u;
  const uint32_t brow0 = (uint32_t)((GATEUP ? 64 * wn : 128 * wn) + col) * 128u;
  auto boff = [&](int j) -> uint32_t {
    return GATEUP ? (uint32_t)((j < 2 ? 32 * j : 128 + 32 * (j - 2)) * 128) : (uint32_t)(32 * j * 128);
  };

  // One chunk: MFMAs on LDS buffer `buf`. First chunk c + 1's activations
  // (loaded during chunk c - 1) go from `ar` to the other buffer, which
  // chunk c - 1's closing barrier freed, and `ar` takes chunk c + 2's loads;
  // chunk c + 1's weights (set nb) are dequantised into the other buffer
  // between the MFMA steps, and chunk c + 2's weights load into the set cb
  // that chunk c used. One activation register set suffices.
  // Loads and LDS writes are unconditional (past the end they repeat the
  // last chunk, in bounds and never read) so that the compiler can count
  // outstanding loads exactly and never waits for the newest ones.
  // MV: row tiles of this wave with positions of the expert (0..2), a
  // compile-time constant so that each version of the loop is straight-line
  // code the compiler can schedule across steps (a branch per row tile split
  // every step into blocks that serialised LDS reads and MFMAs)
  auto chunk_step = [&](auto mv, int c, int buf, ARegs& ar, BUnit& cb, const BUnit& nb) {
    constexpr int MV = decltype(mv)::value;
    const int cp = min(c + 2, nchunks - 1);
    store_a(ar, buf ^ 1);
    load_a(cp, ar);
    load_b(cp, cb);
    // keep chunk c + 2's loads issued here: sunk below the first weight
    // dequantisation they turned its wait for chunk c + 1's weights into a
    // wait for every load in flight
    __builtin_amdgcn_sched_barrier(0);
    const unsigned char* Ab = &As[buf][0];
    const unsigned char* Bb = &Bs[buf][0];
    // operand fragments of step s + 1 are read while step s multiplies
    V bf[2][4], af[2][2];
    auto read_frags = [&](int s, V (&b)[4], V (&a2)[2]) {
      const uint32_t sw = (uint32_t)(((2 * s + h) ^ tile_swz(col)) << 4);
#pragma unroll
      for (int j = 0; j < 4; j++) b[j] = *reinterpret_cast<const V*>(Bb + brow0 + boff(j) + sw);
#pragma unroll
      for (int i = 0; i < 2; i++) a2[i] = *reinterpret_cast<const V*>(Ab + arow0 + 32 * 128 * i + sw);
    };
    read_frags(0, bf[0], af[0]);
#pragma unroll
    for (int s = 0; s < 4; s++) {
      if (s < 3) read_frags(s + 1, bf[(s + 1) & 1], af[(s + 1) & 1]);
#pragma unroll
      for (int i = 0; i < MV; i++) {
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = MfmaOp<XT>::mma(af[s & 1][i], bf[s & 1][j], acc[i][j]);
      }
      store_b(nb, s, buf ^ 1);
    }
    lds_barrier();
  };

  ARegs ar;
  BUnit u0, u1;
  load_a(0, ar);
  load_b(0, u0);
  load_b(min(1, nchunks - 1), u1);
  store_a(ar, 0);
  load_a(min(1, nchunks - 1), ar);
#pragma unroll
  for (int s = 0; s < 4; s++) store_b(u0, s, 0);
  lds_barrier();

  auto run = [&](auto mv) {
    for (int c = 0; c < nchunks; c += 2) {
      chunk_step(mv, c, 0, ar, u0, u1);
      if (c + 1 < nchunks) chunk_step(mv, c + 1, 1, ar, u1, u0);
    }
  };
  // mvalid is wave-uniform: one scalar branch picks the loop
  if (mvalid == 2) run(std::integral_constant<int, 2>{});
  else if (mvalid == 1) run(std::integral_constant<int, 1>{});
  else run(std::integral_constant<int, 0>{});

  // epilogue: lane holds column col, rows 8 (r / 4) + 4 h + r % 4 of each
  // 32 x 32 tile. The wave's finished outputs (64 rows x OC columns) go
  // through LDS (free after the last barrier) so that the global stores are
  // 16 contiguous bytes of one output row per lane instead of 2-byte stores.
  XT* out = reinterpret_cast<XT*>(a.out);
  const XT* ob0 = reinterpret_cast<const XT*>(a.p0.ob);
  const XT* ob1 = reinterpret_cast<const XT*>(GATEUP ? a.p1.ob : a.p0.ob);
  constexpr int OC = GATEUP ? 64 : 128;  // output columns per wave
  const int cbase = GATEUP ? bn * 128 + 64 * wn : bn * 256 + 128 * wn;
  const uint32_t prow0 = bstart;
  // 8 waves x 64 x OC 16-bit values: As holds waves 0-3, Bs waves 4-7
  XT* wt = reinterpret_cast<XT*>(wave < 4 ? &As[0][0] : &Bs[0][0]) + (wave & 3) * 64 * OC;
#pragma unroll
  for (int j = 0; j < (GATEUP ? 2 : 4); j++) {
    const int cn = cbase + 32 * j + col;
    const float obg = (ob0 && cn < N) ? to_f<XT>(ob0[(size_t)e * N + cn]) : 0.f;
    const float obu = (GATEUP && ob1 && cn < N) ? to_f<XT>(ob1[(size_t)e * N + cn]) : 0.f;
#pragma unroll
    for (int i = 0; i < 2; i++) {
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
        float v = round_to<XT>(acc[i][j][r]);
        if (ob0) v = round_to<XT>(v + obg);
        if constexpr (GATEUP) {
          float u = round_to<XT>(acc[i][j + 2][r]);
          if (ob1) u = round_to<XT>(u + obu);
          v = apply_act<XT>(v, u, a.act, a.alpha, a.limit);
        } else if (a.act == ACT_RELU2) {  // single projection: ReLU^2 only
          v = apply_act<XT>(0.f, v, ACT_RELU2, 0.f, 0.f);
        }
        wt[row * OC + 32 * j + col] = from_f<XT>(v);
      }
    }
  }
  // each lane: 16 bytes (8 columns) of one row per step; the wave reads only
  // its own region, so no block barrier is needed
  constexpr int C8 = OC / 8;
#pragma unroll
  for (int t = 0; t < 64 * C8 / 64; t++) {
    const int q = 64 * t + lane;
    const int row = q / C8, c8 = q - row * C8;
    const uint32_t p = prow0 + (uint32_t)row;
    const int cn0 = cbase + 8 * c8;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(wt + row * OC + 8 * c8);
    // rows past the band belong to the next wave (half tiles)
    if (row < band && p < pend && cn0 < N)  // N % 8 == 0 (host check): whole 16-byte groups
      *reinterpret_cast<u32x4_t*>(out + (size_t)p * N + cn0) = v;
  }
}

template <int BITS, typename XT, typename ST>
static hipError_t launch_gemm_t(bool gateup, const GemmArgs& a, int grid, hipStream_t st,
                                KEvents ev) {
  if (gateup)
    hipExtLaunchKernelGGL((gemm_grouped_kernel<BITS, XT, ST, true>), dim3(grid), dim3(512), 0, st,
                          ev.start, ev.stop, 0, a);
  else
    hipExtLaunchKernelGGL((gemm_grouped_kernel<BITS, XT, ST, false>), dim3(grid), dim3(512), 0, st,
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

#if MOE_BITS == 4
// Dense 16-bit weights of the activation type (the router projection over
// many tokens): the same kernel with the dequantisation replaced by a copy.
hipError_t launch_gemm_dense(int xdt, const GemmArgs& a, int grid, hipStream_t st) {
  if (xdt == DT_BF16)
    hipLaunchKernelGGL((gemm_grouped_kernel<16, bf16_t, bf16_t, false>), dim3(grid), dim3(512), 0,
                       st, a);
  else if (xdt == DT_F16)
    hipLaunchKernelGGL((gemm_grouped_kernel<16, f16_t, f16_t, false>), dim3(grid), dim3(512), 0,
                       st, a);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}
#endif

}  // namespace moe
