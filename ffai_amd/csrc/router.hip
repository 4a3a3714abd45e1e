// router.hip — router projection and top-k selection for gfx950.
//
// Replaces the gate GEMV + host readback + MoERouter.route of
// Sources/FFAI/Models/MoELayer.swift:540-573 (decode), :689-750 (prefill) and
// the GPU router Ops.moeRouterTopKMany (Sources/FFAI/Ops/Ops.swift:2589-2662),
// generalised to every gating mode of MoERouter.route (MoELayer.swift:
// 140-205) and to GPT-OSS's biased router (Models/Text/GPTOSSText.swift:
// 345-366,1349-1361). Selection order is (value desc, index asc): the
// reference heap's tie rule (MoELayer.swift:223-296).
#include <algorithm>

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
  const uint32_t bv = bias_raw<XT>(bias, e);  // issued before the row loads, converted at the end
  const rsrc_t wr = make_rsrc(W + (size_t)e * H, (uint32_t)(H * sizeof(WT)));
  float acc[8];
  if constexpr (__is_same(XT, WT) && !__is_same(XT, float)) {
    u32x4_t wv[NL];
#pragma unroll
    for (int j = 0; j < NL; j++) wv[j] = bload128(wr, (uint32_t)((lane + 64 * j) * 16));
    // tokens in batches of TB: every activation load of a batch goes out
    // before its dot products (a branch per token made each token's loads
    // wait for the token before); tokens past nt repeat the last one and
    // are not stored
    constexpr int TB = NL <= 4 ? 8 : (NL <= 8 ? 4 : 2);
#pragma unroll
    for (int tb = 0; tb < 8; tb += TB) {
      if (tb < nt) {  // wave-uniform
        u32x4_t xv[TB][NL];
#pragma unroll
        for (int q = 0; q < TB; q++) {
          const int t = min(tb + q, nt - 1);
          const rsrc_t xr = make_rsrc(x + (size_t)(t0 + t) * H, (uint32_t)(H * sizeof(XT)));
#pragma unroll
          for (int j = 0; j < NL; j++) xv[q][j] = bload128(xr, (uint32_t)((lane + 64 * j) * 16));
        }
        __builtin_amdgcn_sched_barrier(0);  // the batch's loads stay ahead of its math
#pragma unroll
        for (int q = 0; q < TB; q++) {
          float a = 0.f;
#pragma unroll
          for (int j = 0; j < NL; j++)
#pragma unroll
            for (int i = 0; i < 4; i++) a = dot2_16<XT>(wv[j][i], xv[q][j][i], a);
          acc[tb + q] = group_sum(a, 6);
        }
      } else {
#pragma unroll
        for (int q = 0; q < TB; q++) acc[tb + q] = 0.f;
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
      if (bias) l = round_to<XT>(l + bias_f<XT>(bv));
      logits[(size_t)(t0 + t) * E + e] = from_f<XT>(l);
    }
  }
}

// One token with the decoder step before the MoE block folded in: the
// residual add and RMSNorm of Ops.addAndRmsNorm (Sources/FFAI/Ops/Ops.swift:
// 676-730; Models/Text/Qwen3xText.swift:2650-2660), s = round(h + m),
// xn = round(s * (1 / sqrt(mean(s^2) + eps)) * nw), then
// logits[e] = round(W[e] . xn) (+ bias). One 256-thread block per expert;
// thread i takes the 8-element chunks i + 256 j, j < NL, so the per-thread
// chain is short; the sum of squares and the dot product are reduced over the
// four waves through LDS. Every block computes the same normalised row from
// the same loads, and the expert-0 block writes s and xn for the kernels that
// follow. Weights, activations and the norm weight share one 16-bit type.
template <typename XT, int NL>
__global__ __launch_bounds__(256) void router_logits_norm_kernel(
    const XT* __restrict__ h, const XT* __restrict__ m, const XT* __restrict__ nw, float eps,
    const XT* __restrict__ W, const XT* __restrict__ bias, XT* __restrict__ logits,
    XT* __restrict__ res_out, XT* __restrict__ xn_out, int H, int E) {
  __shared__ float part[2][4];
  const int e = blockIdx.x;  // grid == E
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t bv = bias_raw<XT>(bias, e);  // converted where it is added
  const uint32_t rb = (uint32_t)(H * sizeof(XT));
  const rsrc_t wr = make_rsrc(W + (size_t)e * H, rb);
  const rsrc_t hr = make_rsrc(h, rb), mr = make_rsrc(m, rb), nr = make_rsrc(nw, rb);
  u32x4_t wq[NL], hv[NL], mv[NL], nv[NL];
#pragma unroll
  for (int j = 0; j < NL; j++) {
    const uint32_t off = (uint32_t)((tid + 256 * j) * 16);
    hv[j] = bload128(hr, off);
    mv[j] = bload128(mr, off);
    nv[j] = bload128(nr, off);
    wq[j] = bload128(wr, off);
  }
  // s = round(h + m); chunks past H read zeros and add nothing
  float sv[NL][8];
  float ssq = 0.f;
#pragma unroll
  for (int j = 0; j < NL; j++) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float h0 = to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(hv[j][i] & 0xFFFFu)));
      const float h1 = to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(hv[j][i] >> 16)));
      const float m0 = to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(mv[j][i] & 0xFFFFu)));
      const float m1 = to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(mv[j][i] >> 16)));
      sv[j][2 * i] = round_to<XT>(h0 + m0);
      sv[j][2 * i + 1] = round_to<XT>(h1 + m1);
      ssq = __builtin_fmaf(sv[j][2 * i], sv[j][2 * i], ssq);
      ssq = __builtin_fmaf(sv[j][2 * i + 1], sv[j][2 * i + 1], ssq);
    }
  }
  ssq = group_sum(ssq, 6);
  if (lane == 63) part[0][wv] = ssq;
  __syncthreads();
  const float tot = (part[0][0] + part[0][1]) + (part[0][2] + part[0][3]);
  const float inv = 1.0f / sqrtf(tot / (float)H + eps);
  u32x4_t sp[NL], xp[NL];
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NL; j++) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const float n0 = to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(nv[j][i] & 0xFFFFu)));
      const float n1 = to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(nv[j][i] >> 16)));
      const uint16_t x0 = __builtin_bit_cast(uint16_t, from_f<XT>(sv[j][2 * i] * inv * n0));
      const uint16_t x1 = __builtin_bit_cast(uint16_t, from_f<XT>(sv[j][2 * i + 1] * inv * n1));
      const uint16_t s0 = __builtin_bit_cast(uint16_t, from_f<XT>(sv[j][2 * i]));
      const uint16_t s1 = __builtin_bit_cast(uint16_t, from_f<XT>(sv[j][2 * i + 1]));
      xp[j][i] = (uint32_t)x0 | ((uint32_t)x1 << 16);
      sp[j][i] = (uint32_t)s0 | ((uint32_t)s1 << 16);
      acc = dot2_16<XT>(wq[j][i], xp[j][i], acc);
    }
  }
  acc = group_sum(acc, 6);
  if (lane == 63) part[1][wv] = acc;
  if (e == 0) {
#pragma unroll
    for (int j = 0; j < NL; j++) {
      const int c = tid + 256 * j;  // 8-element chunk; H is a multiple of 8
      if (c * 8 < H) {
        *reinterpret_cast<u32x4_t*>(res_out + (size_t)c * 8) = sp[j];
        *reinterpret_cast<u32x4_t*>(xn_out + (size_t)c * 8) = xp[j];
      }
    }
  }
  __syncthreads();
  if (tid == 0) {
    float l = round_to<XT>((part[1][0] + part[1][1]) + (part[1][2] + part[1][3]));
    if (bias) l = round_to<XT>(l + bias_f<XT>(bv));
    logits[e] = from_f<XT>(l);
  }
}

// One token, one 256-thread block per expert: thread i takes the 8-element
// chunks i + 256 j, j < NL, so each lane issues a quarter of the loads of the
// one-wave form; the four partial sums are added through LDS in wave order.
// Weights and activations share one 16-bit type.
template <typename XT, int NL>
__global__ __launch_bounds__(256) void router_logits_row_kernel(const XT* __restrict__ x,
                                                                const XT* __restrict__ W,
                                                                const XT* __restrict__ bias,
                                                                XT* __restrict__ logits, int H,
                                                                int E) {
  __shared__ float part[4];
  const int e = blockIdx.x;  // grid == E
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t bv = bias_raw<XT>(bias, e);  // converted where it is added
  const uint32_t rb = (uint32_t)(H * sizeof(XT));
  const rsrc_t wr = make_rsrc(W + (size_t)e * H, rb), xr = make_rsrc(x, rb);
  u32x4_t wq[NL], xq[NL];
#pragma unroll
  for (int j = 0; j < NL; j++) {
    const uint32_t off = (uint32_t)((tid + 256 * j) * 16);
    xq[j] = bload128(xr, off);
    wq[j] = bload128(wr, off);
  }
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < NL; j++)
#pragma unroll
    for (int i = 0; i < 4; i++) acc = dot2_16<XT>(wq[j][i], xq[j][i], acc);
  acc = group_sum(acc, 6);
  if (lane == 63) part[wv] = acc;
  __syncthreads();
  if (tid == 0) {
    float l = round_to<XT>((part[0] + part[1]) + (part[2] + part[3]));
    if (bias) l = round_to<XT>(l + bias_f<XT>(bv));
    logits[e] = from_f<XT>(l);
  }
}

// Router logits for many tokens on the matrix cores. Block = one tile of 32
// tokens x 32 experts; its 4 waves split the hidden dimension into 64-value
// groups g = wave + 4 i and each accumulates its groups with
// v_mfma_f32_32x32x16 (lane (c, h) of step q holds values 16 q + 8 h .. + 8
// of token row c (A) and of expert row c (B)). The four partial tiles are
// added in wave order through LDS, then rounded as router_logits_kernel
// rounds (product, then + bias). Needs H % 64 == 0 and T * H, E * H below
// 2^31 elements (32-bit byte offsets); the last expert tile repeats expert
// E - 1 past E and stores nothing there.
// Split K (KS > 1, `psum` non-null): the grid holds KS copies of the tiles,
// copy s over chunks [s * cps, (s + 1) * cps) of the hidden dimension, and
// each writes its unrounded fp32 tile to psum[s][T][E] (the second
// projection's after them, psum[KS * T * E + (s * T + t) * E2 + e]);
// router_topk_kernel adds the KS partials in split order, rounds and routes.
// A batch of 32-255 tokens has only 1-8 token tiles, too few blocks to hide
// the chunk loop's latency.
//
// Both tiles pass through LDS in chunks of 256 values: a wave's load
// instruction covers two rows x 512 contiguous bytes (whole cache lines),
// where fragment-order loads straight from memory touched 32 rows x 32 bytes
// per instruction and ran the one-column shared gate of a 2048-token call at
// 25 us. Chunks c + 1 and c + 2 are in registers while chunk c is multiplied
// from LDS. Rows are stored with their 16-byte pieces XORed by the row's low
// four bits, so the 16 rows a fragment read touches at once hit distinct
// banks.
constexpr int kRgWaves = 4;
constexpr int kRgChunk = 256;                  // values of K per LDS chunk
constexpr int kRgPieces = kRgChunk / 8;        // 16-byte pieces per row chunk
constexpr int kRgLoads = 32 * kRgPieces / (64 * kRgWaves);  // pieces per thread per tile
typedef float f32x16_t __attribute__((ext_vector_type(16)));

template <typename XT> struct RgMfma;
template <> struct RgMfma<bf16_t> {
  typedef __bf16 V __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(V, a), __builtin_bit_cast(V, b), c, 0, 0, 0);
  }
};
template <> struct RgMfma<f16_t> {
  typedef _Float16 V __attribute__((ext_vector_type(8)));
  static __device__ __forceinline__ f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(V, a), __builtin_bit_cast(V, b), c, 0, 0, 0);
  }
};

__device__ __forceinline__ int rg_slot(int row, int piece) {
  return row * kRgPieces + (piece ^ (row & 15));
}

template <typename XT>
__global__ __launch_bounds__(64 * kRgWaves) void router_gemm_kernel(const XT* __restrict__ x,
                                                                    const XT* __restrict__ W,
                                                                    const XT* __restrict__ bias,
                                                                    XT* __restrict__ logits, int T,
                                                                    int H, int E,
                                                                    uint4* __restrict__ x16,
                                                                    const XT* __restrict__ W2,
                                                                    XT* __restrict__ logits2, int E2,
                                                                    float* __restrict__ psum, int KS) {
  // token tile and expert tile of one chunk; the partial tiles of the
  // epilogue (rows padded to 33 floats) reuse the same bytes
  __shared__ u32x4_t stage[2][32 * kRgPieces];
  static_assert(sizeof(stage) >= kRgWaves * 32 * 33 * sizeof(float), "epilogue fits the stage");
  // Blocks go to the eight XCDs round robin (block b to XCD b % 8). The nE
  // expert tiles of one token tile take ids 8 apart inside a window of 8 nE
  // ids, so they run close together on one XCD and read the token rows from
  // its L2 after the first of them has fetched them.
  // Expert tiles past the first ceil(E / 32) belong to a second projection
  // of the same rows (W2: E2 rows, no bias, into logits2), such as a shared
  // expert's gate, so that it costs no launch of its own.
  const int nE1 = (E + 31) >> 5, nE = nE1 + ((E2 + 31) >> 5);
  const int nB = (int)gridDim.x / KS, ks = (int)blockIdx.x / nB;  // K split of this block
  const int b = (int)blockIdx.x - ks * nB, win = b / (8 * nE), slot = b - win * 8 * nE;
  const int tt = win * 8 + (slot & 7), et = slot >> 3;
  if (tt * 32 >= T) return;  // padding of the last window; uniform over the block
  const bool second = et >= nE1;
  const XT* __restrict__ Wt = second ? W2 : W;
  const XT* __restrict__ bt = second ? nullptr : bias;
  XT* __restrict__ out = second ? logits2 : logits;
  const int Et = second ? E2 : E;
  const int t0 = tt * 32, e0 = (second ? et - nE1 : et) * 32;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int col = lane & 31, h = lane >> 5;
  const int G = H >> 6, nC = (H + kRgChunk - 1) / kRgChunk;
  const int cps = (nC + KS - 1) / KS, c0 = ks * cps, c1 = min(nC, c0 + cps);  // this split's chunks
  const rsrc_t xr = make_rsrc(x, (uint32_t)((size_t)T * H * sizeof(XT)));
  const rsrc_t wr = make_rsrc(Wt, (uint32_t)((size_t)Et * H * sizeof(XT)));
  // thread piece j: row (j * 64 * kRgWaves + tid) / kRgPieces of the tile,
  // piece (...) % kRgPieces of the chunk. Rows past T repeat the last token
  // and experts past E the last expert (never stored); pieces past H read
  // the next row or, for the buffer's last row, zero, and are never used.
  uint32_t xo[kRgLoads], wo[kRgLoads];
  int prow[kRgLoads], ppc[kRgLoads];
#pragma unroll
  for (int j = 0; j < kRgLoads; j++) {
    const int P = j * 64 * kRgWaves + tid;
    prow[j] = P / kRgPieces;
    ppc[j] = P % kRgPieces;
    const uint32_t tr = (uint32_t)min(t0 + prow[j], T - 1), er = (uint32_t)min(e0 + prow[j], Et - 1);
    xo[j] = (tr * (uint32_t)H + 8u * (uint32_t)ppc[j]) * 2u;
    wo[j] = (er * (uint32_t)H + 8u * (uint32_t)ppc[j]) * 2u;
  }
  struct Tile {
    u32x4_t a[kRgLoads], b[kRgLoads];
  };
  auto load = [&](int c, Tile& s) __attribute__((always_inline)) {
    const uint32_t kb = (uint32_t)min(c, c1 - 1) * (uint32_t)(kRgChunk * 2);
#pragma unroll
    for (int j = 0; j < kRgLoads; j++) {
      s.a[j] = bload128(xr, xo[j] + kb);
      s.b[j] = bload128(wr, wo[j] + kb);
    }
  };
  // the f16 A operand of the expert GEMMs (bf16 rows only), as a by-product:
  // the nE expert tiles of a token tile convert a share of its rows each.
  // Stores go through a buffer view of x16 with the offsets of pieces outside
  // the share (or past H) set to the view's end, where they are dropped: no
  // branches, so the loads of later chunks keep their exact wait counts.
  const int per = (32 + nE - 1) / nE;
  const int cv0 = et * per, cv1 = min(min(cv0 + per, 32), T - t0);
  const uint32_t x16_bytes = x16 ? (uint32_t)((size_t)T * H * 2) : 0u;
  const rsrc_t cr = make_rsrc(x16, x16_bytes);
  auto put = [&](int c, const Tile& s) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < kRgLoads; j++) {
      stage[0][rg_slot(prow[j], ppc[j])] = s.a[j];
      stage[1][rg_slot(prow[j], ppc[j])] = s.b[j];
    }
#pragma unroll
    for (int j = 0; j < kRgLoads; j++) {
      const int k8 = c * kRgPieces + ppc[j];  // piece of the whole row
      const bool mine = prow[j] >= cv0 && prow[j] < cv1 && 8 * k8 < H && c < c1;
      const uint32_t off = mine ? ((uint32_t)(t0 + prow[j]) * (uint32_t)(H / 8) + (uint32_t)k8) * 16u : x16_bytes;
      const uint4 v = bf16x8_to_a16<kA16Shift>(make_uint4(s.a[j].x, s.a[j].y, s.a[j].z, s.a[j].w));
      bstore128(cr, off, u32x4_t{v.x, v.y, v.z, v.w});
    }
  };
  f32x16_t acc = {};
  auto mma = [&](int c) __attribute__((always_inline)) {
    if (c < c1 && 4 * c + wv < G) {  // wave-uniform: the wave's group of chunk c
      u32x4_t fa[4], fb[4];
#pragma unroll
      for (int q = 0; q < 4; q++) {
        const int p = 8 * wv + 2 * q + h;
        fa[q] = stage[0][rg_slot(col, p)];
        fb[q] = stage[1][rg_slot(col, p)];
      }
#pragma unroll
      for (int q = 0; q < 4; q++) acc = RgMfma<XT>::mma(fa[q], fb[q], acc);
    }
  };
  // LDS-only barriers: the next chunks' loads stay in flight across them
  // (the scheduling barrier keeps chunk 0's loads ahead of chunk 1's, so the
  // first stores to LDS wait for chunk 0 only)
  Tile s0, s1;
  load(c0, s0);
  __builtin_amdgcn_sched_barrier(0);
  load(c0 + 1, s1);
  __builtin_amdgcn_sched_barrier(0);
  // Chunk c from s0, chunk c + 1 from s1; each set reloads two chunks on.
  // With an odd chunk count the last trip's second chunk is past the split:
  // its loads repeat the last chunk, its x16 stores are dropped and no wave
  // has a group in it (no break in the loop, which would cost the wait counts
  // their exactness).
  for (int c = c0; c < c1; c += 2) {  // c0 and c1 are uniform: a scalar loop
    put(c, s0);
    lds_barrier();
    load(c + 2, s0);
    mma(c);
    lds_barrier();
    put(c + 1, s1);
    lds_barrier();
    load(c + 3, s1);
    mma(c + 1);
    lds_barrier();
  }

  float* part = reinterpret_cast<float*>(&stage[0][0]);  // [kRgWaves][32 * 33]
  // lane (col, h) holds rows 8 (r / 4) + 4 h + r % 4 of column col
#pragma unroll
  for (int r = 0; r < 16; r++) part[wv * 32 * 33 + (8 * (r >> 2) + 4 * h + (r & 3)) * 33 + col] = acc[r];
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 1024 / (64 * kRgWaves); j++) {
    const int o = tid + 64 * kRgWaves * j;
    const int r = o >> 5, c = o & 31;
    float s = part[r * 33 + c];
#pragma unroll
    for (int w = 1; w < kRgWaves; w++) s += part[w * 32 * 33 + r * 33 + c];
    if (t0 + r < T && e0 + c < Et) {
      if (psum) {  // block-uniform
        float* pp = second ? psum + (size_t)KS * T * E + (size_t)ks * T * E2 : psum + (size_t)ks * T * E;
        pp[(size_t)(t0 + r) * Et + e0 + c] = s;
        continue;
      }
      float l = round_to<XT>(s);
      if (bt) l = round_to<XT>(l + to_f<XT>(bt[e0 + c]));
      out[(size_t)(t0 + r) * Et + e0 + c] = from_f<XT>(l);
    }
  }
}

// One wave per token row (wave_topk); weights are reproducible bit for bit.
// With the partial tiles of a split-K router_gemm_kernel (rp.part), the wave
// first adds the token's KS partials in split order, rounds as the router
// kernels round (sum, then + bias), and writes the logits row (and the
// second projection's row) before routing it from LDS.
struct RouterPartials {
  const float* part;  // [KS][T][E], then [KS][T][E2]
  int KS;
  const void* bias;   // router bias (XT), nullable
  void* logits2;      // second projection's logits (XT), when E2 > 0
  int E2;
};

// The sum over KS <= MAXKS partials at p[q * stride], in split order: all
// loads first (splits past KS repeat the last one), then the adds.
template <int MAXKS>
__device__ __forceinline__ float split_sum(const float* __restrict__ p, size_t stride, int KS) {
  float v[MAXKS];
#pragma unroll
  for (int q = 0; q < MAXKS; q++) v[q] = p[(size_t)min(q, KS - 1) * stride];
  float s = v[0];
#pragma unroll
  for (int q = 1; q < MAXKS; q++) s = q < KS ? s + v[q] : s;
  return s;
}

// MAXKS: 1 without partials, else a bound on rp.KS; EPL: logits per lane
// (E <= 64 EPL)
template <typename XT, int MAXKS, int EPL>
__global__ __launch_bounds__(256) void router_topk_kernel(XT* __restrict__ logits, int T,
                                                          int E, int k, const RouteOpts ro,
                                                          uint32_t* __restrict__ idx_out,
                                                          float* __restrict__ w_out,
                                                          const RouterPartials rp) {
  __shared__ float sc[4][kTopkMaxE];
  __shared__ XT lrow[MAXKS > 1 ? 4 : 1][MAXKS > 1 ? kTopkMaxE : 1];
  const int wv = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + wv;
  if (t >= T) return;  // wave-uniform; the kernel has no block barrier
  const XT* row = logits + (size_t)t * E;
  if constexpr (MAXKS > 1) {
    const XT* bias = reinterpret_cast<const XT*>(rp.bias);
    const size_t stride = (size_t)T * E;
#pragma unroll
    for (int j = 0; j < EPL; j++) {
      if (64 * j >= E) break;  // wave-uniform
      const int e = lane + 64 * j, ec = min(e, E - 1);
      float l = round_to<XT>(split_sum<MAXKS>(rp.part + (size_t)t * E + ec, stride, rp.KS));
      if (bias) l = round_to<XT>(l + to_f<XT>(bias[ec]));
      if (e < E) {
        logits[(size_t)t * E + e] = from_f<XT>(l);
        lrow[wv][e] = from_f<XT>(l);
      }
    }
    if (lane < rp.E2) {
      const float* p2 = rp.part + (size_t)rp.KS * stride + (size_t)t * rp.E2 + lane;
      const float s = split_sum<MAXKS>(p2, (size_t)T * rp.E2, rp.KS);
      reinterpret_cast<XT*>(rp.logits2)[(size_t)t * rp.E2 + lane] = from_f<XT>(s);
    }
    wave_sync();
    row = lrow[wv];
  }
  int sel;
  float w;
  wave_topk<XT, EPL>(row, E, k, ro, sc[wv], true, &sel, &w);
  if (lane < k) {
    idx_out[(size_t)t * k + lane] = (uint32_t)sel;
    w_out[(size_t)t * k + lane] = w;
  }
}

// Token x expert tiles below which router_gemm_kernel splits K: splits
// until about this many blocks run (at most one per 256-value chunk).
constexpr int kRgSplitBlocks = 256;
constexpr int kRgMaxSplits = 16;

template <typename XT, typename WT>
static hipError_t launch_rl(const void* x, int T, int H, const void* W, const void* bias, int E,
                            void* logits, hipStream_t st, void* x16, bool* x16_done,
                            const void* W2, int E2, void* logits2, bool* second_done,
                            float* part, size_t part_bytes, int* splits) {
  if constexpr (__is_same(XT, WT) && !__is_same(XT, float)) {
    if (T >= 32 && H % 64 == 0 && (size_t)T * H < (1ull << 31) && (size_t)E * H < (1ull << 31)) {
      const bool conv = x16 && __is_same(XT, bf16_t);
      const bool two = W2 && logits2 && E2 > 0 && (size_t)E2 * H < (1ull << 31);
      const int windows = (T + 255) / 256;  // eight token tiles each
      const int tiles = (E + 31) / 32 + (two ? (E2 + 31) / 32 : 0);
      const int nC = (H + kRgChunk - 1) / kRgChunk, active = (T + 31) / 32 * tiles;
      int KS = 1;
      if (part && splits && active < kRgSplitBlocks) {
        KS = std::min(std::min(nC, kRgMaxSplits), (kRgSplitBlocks + active - 1) / active);
        const int cps = (nC + KS - 1) / KS;  // chunks per split
        KS = (nC + cps - 1) / cps;           // no split without chunks
        if ((size_t)KS * T * (E + (two ? E2 : 0)) * sizeof(float) > part_bytes) KS = 1;
      }
      hipLaunchKernelGGL((router_gemm_kernel<XT>), dim3(KS * windows * 8 * tiles),
                         dim3(64 * kRgWaves), 0, st, (const XT*)x, (const XT*)W, (const XT*)bias,
                         (XT*)logits, T, H, E, conv ? (uint4*)x16 : nullptr,
                         two ? (const XT*)W2 : nullptr, two ? (XT*)logits2 : nullptr,
                         two ? E2 : 0, KS > 1 ? part : nullptr, KS);
      if (x16_done) *x16_done = conv;
      if (second_done) *second_done = two;
      if (splits) *splits = KS;
      return hipGetLastError();
    }
    if (T == 1 && H <= 4 * 2048) {
      const int nl4 = (H + 2047) / 2048;
#define MOE_RLR(NL)                                                                         \
  hipLaunchKernelGGL((router_logits_row_kernel<XT, NL>), dim3(E), dim3(256), 0, st,         \
                     (const XT*)x, (const XT*)W, (const XT*)bias, (XT*)logits, H, E);       \
  return hipGetLastError();
      if (nl4 <= 1) { MOE_RLR(1) }
      if (nl4 <= 2) { MOE_RLR(2) }
      MOE_RLR(4)
#undef MOE_RLR
    }
  }
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
                                const void* bias, int E, void* logits, hipStream_t st, void* x16,
                                bool* x16_done, const void* W2, int E2, void* logits2,
                                bool* second_done, float* part, size_t part_bytes, int* splits) {
  if (x16_done) *x16_done = false;
  if (second_done) *second_done = false;
  if (splits) *splits = 1;
#define MOE_RL2(XT, WT)                                                                        \
  return launch_rl<XT, WT>(x, T, H, W, bias, E, logits, st, x16, x16_done, W2, E2, logits2, \
                           second_done, part, part_bytes, splits);
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

hipError_t launch_router_logits_norm(const void* h, const void* m, const void* nw, float eps,
                                     int xdt, int H, const void* W, int wdt, const void* bias,
                                     int E, void* logits, void* res_out, void* xn_out,
                                     hipStream_t st) {
  if (xdt != wdt || xdt == DT_F32 || H % 8 != 0 || H > 4 * 2048) return hipErrorInvalidValue;
  const int nl = (H + 2047) / 2048;
#define MOE_RLN(XT, NL)                                                                        \
  hipLaunchKernelGGL((router_logits_norm_kernel<XT, NL>), dim3(E), dim3(256), 0, st,           \
                     (const XT*)h, (const XT*)m, (const XT*)nw, eps, (const XT*)W,             \
                     (const XT*)bias, (XT*)logits, (XT*)res_out, (XT*)xn_out, H, E);           \
  return hipGetLastError();
#define MOE_RLN_NL(XT)            \
  if (nl <= 1) { MOE_RLN(XT, 1) } \
  if (nl <= 2) { MOE_RLN(XT, 2) } \
  MOE_RLN(XT, 4)
  if (xdt == DT_BF16) { MOE_RLN_NL(bf16_t) }
  MOE_RLN_NL(f16_t)
#undef MOE_RLN_NL
#undef MOE_RLN
}

hipError_t launch_router_topk(void* logits, int dt, int T, int E, int k, const RouteOpts& ro,
                              uint32_t* idx, float* w, hipStream_t st, const float* part, int KS,
                              const void* bias, void* logits2, int E2) {
  const int grid = (T + 3) / 4;
  const RouterPartials rp{KS > 1 ? part : nullptr, KS, bias, logits2, KS > 1 && logits2 ? E2 : 0};
  if (rp.part && (E > kTopkMaxE || E2 > 64 || KS > kRgMaxSplits || dt == DT_F32))
    return hipErrorInvalidValue;
#define MOE_TK3(XT, MK, EPL)                                                                \
  hipLaunchKernelGGL((router_topk_kernel<XT, MK, EPL>), dim3(grid), dim3(256), 0, st,      \
                     (XT*)logits, T, E, k, ro, idx, w, rp);                                \
  return hipGetLastError();
#define MOE_TK2(XT, MK)                   \
  if (E <= 64) { MOE_TK3(XT, MK, 1) }     \
  if (E <= 128) { MOE_TK3(XT, MK, 2) }    \
  if (E <= 256) { MOE_TK3(XT, MK, 4) }    \
  MOE_TK3(XT, MK, kTopkEPL)
#define MOE_TK(XT)                                 \
  if (!rp.part) { MOE_TK2(XT, 1) }                 \
  if constexpr (!__is_same(XT, float)) {           \
    if (KS <= 4) { MOE_TK2(XT, 4) }                \
    if (KS <= 8) { MOE_TK2(XT, 8) }                \
    MOE_TK2(XT, kRgMaxSplits)                      \
  }
  if (dt == DT_BF16) { MOE_TK(bf16_t) }
  if (dt == DT_F16) { MOE_TK(f16_t) }
  if (dt == DT_F32) { MOE_TK(float) }
#undef MOE_TK
#undef MOE_TK2
#undef MOE_TK3
  return hipErrorInvalidValue;
}

}  // namespace moe
