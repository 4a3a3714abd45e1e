// gemm.hip — prefill-side grouped dequant GEMM on the gfx950 matrix cores.
//
// Replaces Ops.moeGatherDequantGemmInt4 bm8/bm16/bm64/m1
// (Sources/FFAI/Ops/Ops.swift:4553-5201, 6499-6585) with the tile choice of
// MoELayer.swift:855-882, generalised to 2/3/4/5/6/8-bit weights, group sizes
// 32/64/128 and scale dtypes independent of the activation dtype:
//   gate/up:  act[p, n] = act_fn(round(Wg[e(p)][n] . x[row(p)]),
//                                round(Wu[e(p)][n] . x[row(p)]))
//   single:   out[p, n] = round(W[e(p)][n] . a[p])
// over the expert-sorted positions p of a dispatch plan.
//
// Operands are f16 on v_mfma_f32_32x32x16_f16:
//  - weights are dequantised exactly to s * q + b rounded once to f16
//    (2^-12 relative; bf16 operands would round them to 2^-9): 4-bit codes
//    become f16 q through the scaled fp8 conversion, other widths enter as
//    1024 + q (exact in f16) less 1024; one packed fma gives s * q + b;
//  - activations of an f16 layer are used as they are; those of a bf16 layer
//    are scaled by 2^-8 into f16 range (exact for magnitudes 2^-6 .. 1.6e7,
//    saturating beyond) beforehand (launch_to_a16, and the gate/up epilogue
//    writes its activation in that form for the down GEMM); the epilogue
//    multiplies the fp32 sums by 2^8.
//
// Work: a list of items (expert, first sorted position, column block) built
// on the device from the CSR offsets (launch_gemm_items). An expert's rows go
// in tiles of 256, and a last tile of at most 128 rows takes the half shape:
//   shape 0: 256 rows x 256 weight rows, waves 4 x 2, 64 x 128 per wave;
//   shape 1: 128 rows x 256 weight rows, waves 2 x 4, 64 x 64 per wave.
// A wave owns 64 rows x NJ * 32 weight rows (gate/up: half gate, half up, so
// the epilogue pairs them in one lane); a wave whose rows hold no position of
// the expert skips its MFMAs. Both shapes dequantise 256 weight rows per
// chunk, one unit per thread, so a block's cost is set mostly by K; a
// 64-row shape over 512 weight rows would need LDS for two more weight rows
// per thread than the three activation stages leave. Blocks b, b + 8, ...
// run on one XCD: the items are split into 8 contiguous ranges at run time,
// one per XCD, so neighbouring column blocks of a row tile share its L2.
//
// Per 64-value chunk of K the block holds the tile's activation rows (copied
// from memory straight into a ring of three LDS stages, two chunks ahead) and
// its weight rows (codes, scales and biases loaded three chunks ahead into
// registers, dequantised once per block into two LDS buffers between the MFMA
// steps of the chunk before). One block barrier per chunk.
#include <hip/hip_ext.h>

#include <type_traits>

#include "moe_common.hpp"
#include "moe_internal.hpp"

#ifndef MOE_BITS
#define MOE_BITS 4
#endif

namespace moe {

typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16_t mma_f16(u32x4_t a, u32x4_t b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, a),
                                                __builtin_bit_cast(f16x8_t, b), c, 0, 0, 0);
}

constexpr int kGBK = 64;  // values per K chunk (128 bytes of an LDS row)

// vector-memory instructions of one bload_unit
template <int BITS>
constexpr int kUnitLoads = (BITS == 5 || BITS == 6 || BITS == 8) ? 2 : 1;

// s_waitcnt for at most N outstanding vector-memory operations (gfx9
// encoding: vmcnt in bits 3:0 and 15:14; expcnt 6:4 and lgkmcnt 11:8 left
// at their maxima)
template <int N>
__device__ __forceinline__ void vmcnt_wait() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Block barrier for LDS written by this block's LDS stores and by its
// memory-to-LDS copies of earlier chunks: waits for the wave's own LDS
// operations (lgkmcnt 0) only. A release fence on LDS would also wait for
// every memory-to-LDS copy in flight, including the ones issued for chunks
// two ahead; the callers wait for the copies that must have landed
// (vmcnt_wait) themselves. The signal fences keep the compiler from moving
// memory operations across the barrier.
__device__ __forceinline__ void lds_barrier_copies_in_flight() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt and expcnt at their maxima
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// LDS tiles are 128 B per row. The banks repeat every 256 B (two rows) and a
// 16-byte read serves 16 lanes per cycle, so the 16-byte chunk c of row r
// sits at slot c ^ ((r >> 1) & 7) ^ 2 (r & 1): 16 consecutive rows reading
// the same chunk then cover every bank once, and so do the weight stores (a
// lane pair per row, chunks s and 4 + s). Measured with the bank-conflict
// counter on gfx950: (r >> 1) & 7 alone keeps the reads conflict-free but
// gives the stores 1.6 conflict cycles per LDS-active cycle (96 against 80
// shader cycles per store instruction), r & 7 the reverse (reads 64 against
// 50); this form is conflict-free for both.
__device__ __forceinline__ int tile_swz(int r) { return ((r >> 1) & 7) ^ ((r & 1) << 1); }
__device__ __forceinline__ uint32_t tile_off(int r, int c) {
  return (uint32_t)(r * 128 + ((c ^ tile_swz(r)) << 4));
}

template <int S> struct GShape;
template <> struct GShape<0> { static constexpr int MR = 256, NR = 256, WMN = 4, NJ = 4; };
template <> struct GShape<1> { static constexpr int MR = 128, NR = 256, WMN = 2, NJ = 2; };
// 64 rows: the waves split the weight rows only (32 each; for a gate/up pair
// waves 0-3 hold gate rows and 4-7 the matching up rows, paired through LDS
// in the epilogue), so every wave has MFMA work.
template <> struct GShape<2> { static constexpr int MR = 64, NR = 256, WMN = 1, NJ = 1; };

// LDS: three activation stages (one object each, so that the compiler tracks
// the memory-to-LDS copies into each stage on their own and waits for only
// the stage a read needs) and the two weight buffers.
constexpr int kAStageBytes = 256 * 128, kBBufBytes = 256 * 128;
struct GemmLds {
  unsigned char *a0, *a1, *a2, *b;
};

struct ProjViewG {
  rsrc_t w, s, b;
};
template <int BITS>
__device__ __forceinline__ ProjViewG proj_view_g(const GemvProj& p, uint32_t e, int N, int row_words,
                                                 int groups) {
  const size_t rows = (size_t)e * (size_t)N;
  ProjViewG v;
  v.w = make_rsrc(p.w + rows * row_words, (uint32_t)N * (uint32_t)row_words * 4u);
  v.s = make_rsrc(reinterpret_cast<const uint16_t*>(p.s) + rows * groups, (uint32_t)N * (uint32_t)groups * 2u);
  v.b = make_rsrc(reinterpret_cast<const uint16_t*>(p.b) + rows * groups, (uint32_t)N * (uint32_t)groups * 2u);
  return v;
}

// Values 8 s + 2 p and 8 s + 2 p + 1 (p < 4) of a 32-value unit as 16-bit
// pairs 0x6400 | q, i.e. 1024 + q in f16 (exact for q < 1024).
template <int BITS>
__device__ __forceinline__ void quarter_pairs(const uint32_t (&w)[BITS], int s, uint32_t (&pr)[4]) {
  const uint32_t M = opaque_vgpr(0x64006400u);
  if constexpr (BITS == 4) {
    // word s holds the quarter: nibbles 0, 2, 4, 6 in the bytes of t, 1, 3, 5, 7 in u
    const uint32_t t = w[s] & 0x0F0F0F0Fu, u = (w[s] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
    for (int p = 0; p < 4; p++)  // bytes [t.p, 0, u.p, 0]
      pr[p] = __builtin_amdgcn_perm(u, t, (uint32_t)p | 0x0C00u | ((uint32_t)(4 + p) << 16) | 0x0C000000u) | M;
  } else if constexpr (BITS == 8) {
#pragma unroll
    for (int p = 0; p < 4; p++) {  // bytes [b(2p), 0, b(2p+1), 0] of word 2 s + p / 2
      const int bb = 2 * (p & 1);
      pr[p] = __builtin_amdgcn_perm(0u, w[2 * s + (p >> 1)],
                                    (uint32_t)bb | 0x0C00u | ((uint32_t)(bb + 1) << 16) | 0x0C000000u) | M;
    }
  } else if constexpr (BITS <= 3) {
    // Two pairs per 4 * BITS-bit field y (values a, b, c, d from bit 0):
    // m = y | y << (16 - BITS) has a at bit 0, b at bit 16, c at bit 2 * BITS
    // and d at bit 16 + 2 * BITS, and the two copies of y do not overlap
    // (4 * BITS <= 16 - BITS), so one mask per pair picks them out.
    constexpr uint32_t kField = (1u << (4 * BITS)) - 1u, kPair = ((1u << BITS) - 1u) * 0x10001u;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int bit = (2 * s + h) * 4 * BITS, lo = bit >> 5, sh = bit & 31;
      uint32_t y;
      if (sh + 4 * BITS <= 32)
        y = (w[lo] >> sh) & kField;
      else
        y = __builtin_amdgcn_alignbit(w[lo + 1], w[lo], (uint32_t)sh) & kField;
      const uint32_t m = y | (y << (16 - BITS));
      pr[2 * h] = (m & kPair) | M;
      pr[2 * h + 1] = ((m >> (2 * BITS)) & kPair) | M;
    }
  } else if constexpr (BITS == 5 || BITS == 6) {
    // A pair's 2 * BITS bits lie inside the 16 bits from the byte holding its
    // first bit: one byte permute puts those 16 bits in both halves, and one
    // packed 16-bit shift right by (o, o + BITS) brings each value to the
    // bottom of its half.
    typedef unsigned short u16x2_t __attribute__((ext_vector_type(2)));
    constexpr uint32_t kPair = ((1u << BITS) - 1u) * 0x10001u;
#pragma unroll
    for (int p = 0; p < 4; p++) {
      const int bit = (8 * s + 2 * p) * BITS, byte = bit >> 3, o = bit & 7;
      const int wi = byte >> 2, bw = byte & 3, wj = wi + 1 < BITS ? wi + 1 : BITS - 1;
      const uint32_t sel = (uint32_t)bw | ((uint32_t)(bw + 1) << 8) | ((uint32_t)bw << 16) |
                           ((uint32_t)(bw + 1) << 24);
      const u16x2_t z = __builtin_bit_cast(u16x2_t, __builtin_amdgcn_perm(w[wj], w[wi], sel));
      const u16x2_t t = z >> u16x2_t{(unsigned short)o, (unsigned short)(o + BITS)};
      pr[p] = (__builtin_bit_cast(uint32_t, t) & kPair) | M;
    }
  } else {
#pragma unroll
    for (int p = 0; p < 4; p++) {
      uint32_t c[2];
#pragma unroll
      for (int k = 0; k < 2; k++) {
        const int bit = (8 * s + 2 * p + k) * BITS, lo = bit >> 5, sh = bit & 31;
        uint32_t v = w[lo] >> sh;
        if (sh + BITS > 32) v |= w[lo + 1] << (32 - sh);
        c[k] = v & ((1u << BITS) - 1u);
      }
      pr[p] = (c[0] | (c[1] << 16)) | M;
    }
  }
}

// Codes of values 8 s + 2 p and 8 s + 2 p + 1 (p < 4) of a 32-value unit as
// f16 pairs. 4-bit: the nibbles are spread one per byte, and a byte q < 16 is
// the OCP e4m3 number q * 2^-9 (subnormal below 8), so the scaled fp8
// conversion at 2^9 gives q exactly, two values per instruction. Other widths:
// 1024 + q pairs less 1024.
template <int BITS>
__device__ __forceinline__ void quarter_codes(const uint32_t (&w)[BITS], int s, h2_t (&q)[4]) {
  if constexpr (BITS == 4) {
    const uint32_t t = w[s] & 0x0F0F0F0Fu, u = (w[s] >> 4) & 0x0F0F0F0Fu;
    const uint32_t z0 = __builtin_amdgcn_perm(u, t, 0x05010400u);  // bytes [t0, u0, t1, u1]
    const uint32_t z1 = __builtin_amdgcn_perm(u, t, 0x07030602u);  // bytes [t2, u2, t3, u3]
    q[0] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(z0, 512.0f, false);
    q[1] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(z0, 512.0f, true);
    q[2] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(z1, 512.0f, false);
    q[3] = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(z1, 512.0f, true);
  } else {
    uint32_t pr[4];
    quarter_pairs<BITS>(w, s, pr);
#pragma unroll
    for (int p = 0; p < 4; p++)
      q[p] = __builtin_bit_cast(h2_t, pr[p]) - h2_t{(_Float16)1024.0f, (_Float16)1024.0f};
  }
}

// A 16-bit scale or bias (bf16 or f16 storage) as an f16 pair. Both
// conversions are computed and one is selected (a branch on the storage type
// here split every chunk of the main loop into a dozen basic blocks).
__device__ __forceinline__ h2_t sb_h2(uint32_t raw16, bool bf16) {
  const uint16_t from_bf = __builtin_bit_cast(uint16_t, (_Float16)__uint_as_float(raw16 << 16));
  const uint32_t h = bf16 ? (uint32_t)from_bf : raw16;  // bf16: exact inside f16's range
  return __builtin_bit_cast(h2_t, h | (h << 16));
}

// One stored output value (fp32, already in the output's units) as the f16 A
// operand of the next GEMM: round to the layer dtype first (the reference
// stores the activation in it), then scale into f16 range, saturating.
template <typename XT>
__device__ __forceinline__ _Float16 to_a16(float v) {
  v = round_to<XT>(v);
  if constexpr (__is_same(XT, bf16_t)) {
    v = __builtin_ldexpf(v, -kA16Shift);
    v = fminf(fmaxf(v, -65504.0f), 65504.0f);
  }
  return (_Float16)v;
}

// Gate/up epilogue of the 64-row shape: wave w < 4 holds gate columns
// 32 w + col of the block, wave w + 4 the matching up columns. Each wave
// stores its projections, rounded as the other shapes round them, into a
// [64 rows][256] 16-bit table in the weight buffers (free after the last
// barrier); after a block barrier every thread pairs gate and up for 8
// consecutive output columns of a row and stores them as 16 bytes.
template <typename XT>
__device__ __forceinline__ void gateup_epilogue_split(const GemmArgs& a, const GemmLds L,
                                                      const f32x16_t (&acc)[2][1], uint32_t e,
                                                      uint32_t m0, int bn, uint32_t pend, int wn,
                                                      int col, int h, float oscale) {
  const int N = a.N;
  uint16_t* tb = reinterpret_cast<uint16_t*>(L.b);
  const int cn = bn * 128 + 32 * (wn & 3) + col;  // output column of this lane
  const XT* ob = reinterpret_cast<const XT*>(wn < 4 ? a.p0.ob : a.p1.ob);
  // without an output bias (ob is wave-uniform) the sum is rounded once
  auto stage_out = [&](auto biasc) {
    constexpr bool BIAS = decltype(biasc)::value;
    const float obv = (BIAS && cn < N) ? to_f<XT>(ob[(size_t)e * N + cn]) : -0.0f;
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const int row = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
        float v = acc[i][0][r] * oscale;
        if constexpr (BIAS) v = round_to<XT>(round_to<XT>(v) + obv);
        tb[row * 256 + 32 * wn + col] = __builtin_bit_cast(uint16_t, from_f<XT>(v));
      }
  };
  if (ob) stage_out(std::true_type{});
  else stage_out(std::false_type{});
  __syncthreads();
  uint16_t* out = reinterpret_cast<uint16_t*>(a.out);
  auto finish = [&](auto actc) {
    constexpr int ACT = decltype(actc)::value;
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const int q = (int)threadIdx.x + 512 * t;  // 64 rows x 16 pieces of 8 columns
      const int row = q >> 4, c8 = q & 15;
      const u32x4_t gv = *reinterpret_cast<const u32x4_t*>(tb + row * 256 + 8 * c8);
      const u32x4_t uv = *reinterpret_cast<const u32x4_t*>(tb + row * 256 + 128 + 8 * c8);
      u32x4_t o;
#pragma unroll
      for (int k = 0; k < 4; k++) {
        uint32_t pk = 0;
#pragma unroll
        for (int half = 0; half < 2; half++) {
          const float g = to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(gv[k] >> (16 * half))));
          const float u = to_f<XT>(__builtin_bit_cast(XT, (uint16_t)(uv[k] >> (16 * half))));
          const uint16_t bits = __builtin_bit_cast(uint16_t, to_a16<XT>(apply_act<XT>(g, u, ACT, a.alpha, a.limit)));
          pk |= (uint32_t)bits << (16 * half);
        }
        o[k] = pk;
      }
      const uint32_t p = m0 + (uint32_t)row;
      const int cn0 = bn * 128 + 8 * c8;
      if (p < pend && cn0 < N)  // N % 8 == 0 (host check): whole 16-byte groups
        *reinterpret_cast<u32x4_t*>(out + (size_t)p * N + cn0) = o;
    }
  };
  if (a.act == ACT_GPTOSS) finish(std::integral_constant<int, ACT_GPTOSS>{});
  else if (a.act == ACT_GEGLU) finish(std::integral_constant<int, ACT_GEGLU>{});
  else finish(std::integral_constant<int, ACT_SWIGLU>{});
}

// One block's tile: rows [m0, m0 + MR) of expert e (positions below pend),
// weight rows of column block bn.
template <int S, int BITS, typename XT, bool GATEUP>
__device__ __forceinline__ void gemm_tile(const GemmArgs& a, const GemmLds L, uint32_t e, uint32_t m0,
                                          int bn, uint32_t pend) {
  typedef GShape<S> G;
  constexpr int MR = G::MR, NR = G::NR, WMN = G::WMN, WN = 8 / WMN, NJ = G::NJ;
  constexpr int BBUF = NR * 128;
  constexpr int AI = MR / 64;       // activation copies of 16 B per thread per chunk
  constexpr int BI = NR * 2 / 512;  // weight units per thread per chunk
  static_assert(MR * 128 <= kAStageBytes && 2 * BBUF <= kBBufBytes * 2, "LDS layout");
  constexpr float OSCALE = __is_same(XT, bf16_t) ? (float)(1 << kA16Shift) : 1.0f;
  unsigned char* Bs = L.b;  // two weight buffers of BBUF bytes
  // activation stage ST (compile time: each stage is its own LDS object)
  auto stage = [&](auto st) -> unsigned char* {
    constexpr int ST = decltype(st)::value;
    return ST == 0 ? L.a0 : (ST == 1 ? L.a1 : L.a2);
  };
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int N = a.N, K = a.K, CU = K >> 5, groups = CU >> a.gsh, row_words = CU * BITS;
  const int nchunks = K / kGBK;
  const bool sb_bf16 = a.sb_bf16 != 0;

  // ---- activation rows go from memory straight to LDS (buffer loads with
  // the LDS flag: lane l of a wave writes the 16 bytes at M0 + 16 l). Thread
  // t fills, for i < AI, slot t % 8 of LDS row t / 8 + 64 i with the row's
  // logical 16-byte chunk (t % 8) ^ tile_swz(row); a wave's 64 lanes cover 8
  // consecutive rows, one contiguous KB of LDS.
  const rsrc_t xr = make_rsrc(a.x, (uint32_t)min((size_t)a.x_rows * K * 2u, (size_t)0xFFFFFFFFu));
  // the rows' plan entries, loaded without a branch (a view of zero bytes
  // when there is no gather: loads return 0) and first of all, since the
  // copies wait for them; turned into row offsets once the weights' first
  // loads are out (set_xoff)
  const rsrc_t permv = make_rsrc(a.perm, (uint32_t)__builtin_amdgcn_readfirstlane(a.perm ? -1 : 0));
  uint32_t xpos[AI], praw[AI], xoff[AI];
#pragma unroll
  for (int i = 0; i < AI; i++) {
    xpos[i] = min(m0 + (uint32_t)((threadIdx.x >> 3) + 64 * i), pend - 1);
    praw[i] = bload32(permv, xpos[i] * 4u);
  }
  auto set_xoff = [&]() {
#pragma unroll
    for (int i = 0; i < AI; i++) {
      const int r = (threadIdx.x >> 3) + 64 * i;
      const uint32_t xrow = a.perm ? praw[i] / (uint32_t)a.topk : xpos[i];
      const int c = (threadIdx.x & 7) ^ tile_swz(r);
      xoff[i] = (xrow * (uint32_t)K + (uint32_t)(8 * c)) * 2u;
    }
  };
  auto dma_a = [&](int chunk, auto st) {
#pragma unroll
    for (int i = 0; i < AI; i++) {
      unsigned char* dst = stage(st) + (64 * i + 8 * wave) * 128;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(xr, (__attribute__((address_space(3))) void*)dst, 16,
                                               xoff[i] + (uint32_t)(chunk * kGBK * 2), 0, 0, 0);
    }
  };

  // ---- weights: thread t dequantises, for i < BI, unit t % 2 (values
  // [32 (t % 2), +32) of the chunk) of LDS weight row t / 2 + 256 i. Gate/up:
  // LDS rows below NR / 2 hold gate rows, the rest up rows (for shape 0 that
  // splits at wave 4, for the others at i = 1: wave-uniform either way).
  const int bu = threadIdx.x & 1;
  int brl[BI];
  uint32_t brow[BI];
  ProjViewG PB[BI];
  const uint32_t* SB[BI];
#pragma unroll
  for (int i = 0; i < BI; i++) {
    brl[i] = (threadIdx.x >> 1) + 256 * i;
    int wrow;
    bool upper = false;
    if constexpr (GATEUP) {
      upper = brl[i] >= NR / 2;
      wrow = bn * (NR / 2) + (brl[i] & (NR / 2 - 1));
    } else {
      wrow = bn * NR + brl[i];
    }
    brow[i] = (uint32_t)min(wrow, N - 1);
    // upper is wave-uniform (see above); the branch keeps the views scalar
    const GemvProj& pj = (GATEUP && __builtin_amdgcn_readfirstlane((int)upper)) ? a.p1 : a.p0;
    PB[i] = proj_view_g<BITS>(pj, e, N, row_words, groups);
    // the lane pair of a weight row (bu = 0, 1) loads its scales and its
    // biases respectively (4-byte aligned arrays, host check; the expert's
    // first group is even since N % 8 == 0)
    SB[i] = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint16_t*>(bu ? pj.b : pj.s) +
                                              (size_t)e * N * groups);
  }
  // packed codes and the scale or bias word of a thread's units: three
  // register sets, so chunks c + 2 and c + 3 are in flight while chunk c + 1
  // is dequantised
  struct BUnits {
    uint32_t w[BI][BITS];
    uint32_t sb[BI];  // the 32-bit word holding the unit's 16-bit scale (bu = 0) or bias (bu = 1)
  };
  // group element of a thread's unit in chunk `chunk` (row-major [N][groups]):
  // for 32-value groups the pair's two groups share one word (groups is even:
  // K % 64 == 0), for larger ones both lanes want the same group
  auto sb_el = [&](int i, int chunk) -> uint32_t {
    return brow[i] * (uint32_t)groups + (uint32_t)((2 * chunk + bu) >> a.gsh);
  };
  auto load_sb = [&](int chunk, BUnits& u) {
#pragma unroll
    for (int i = 0; i < BI; i++) u.sb[i] = SB[i][sb_el(i, chunk) >> 1];
  };
  auto load_w = [&](int chunk, BUnits& u) {
    const int unit = 2 * chunk + bu;
#pragma unroll
    for (int i = 0; i < BI; i++)
      bload_unit<BITS>(PB[i].w, (brow[i] * (uint32_t)row_words + (uint32_t)(unit * BITS)) * 4u, u.w[i]);
  };
  // values [8 s, 8 s + 8) of each unit -> LDS chunk 4 bu + s of its row
  auto store_b = [&](const BUnits& u, const h2_t (&s2)[BI], const h2_t (&b2)[BI], int s, int buf) {
#pragma unroll
    for (int i = 0; i < BI; i++) {
      h2_t q[4];
      quarter_codes<BITS>(u.w[i], s, q);
      u32x4_t v;
#pragma unroll
      for (int p = 0; p < 4; p++)
        v[p] = __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(q[p], s2[i], b2[i]));
      *reinterpret_cast<u32x4_t*>(Bs + buf * BBUF + tile_off(brl[i], 4 * bu + s)) = v;
    }
  };
  // the unit's scale and bias: the lane pair swaps its words (DPP quad_perm
  // [1, 0, 3, 2]) and each lane takes its 16-bit half
  auto sb_pairs = [&](const BUnits& u, int chunk, h2_t (&s2)[BI], h2_t (&b2)[BI]) {
#pragma unroll
    for (int i = 0; i < BI; i++) {
      const uint32_t other = (uint32_t)__builtin_amdgcn_mov_dpp((int)u.sb[i], 0xB1, 0xF, 0xF, false);
      const uint32_t sw = bu ? other : u.sb[i], bw = bu ? u.sb[i] : other;
      const uint32_t sh = (sb_el(i, chunk) & 1u) * 16u;
      s2[i] = sb_h2((sw >> sh) & 0xFFFFu, sb_bf16);
      b2[i] = sb_h2((bw >> sh) & 0xFFFFu, sb_bf16);
    }
  };

  f32x16_t acc[2][NJ];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < NJ; j++) acc[i][j] = f32x16_t{};

  // row tiles of this wave's 64-row band that hold positions of the expert
  const uint32_t bstart = m0 + 64u * (uint32_t)wm;
  const int mvalid = (bstart >= pend) ? 0 : (bstart + 32u >= pend ? 1 : 2);

  // MFMA operand rows of this lane: A rows 64 wm + 32 i + col, B rows (LDS)
  // 32 j + col within the wave's weight rows; all congruent to col mod 32, so
  // they share tile_swz(col)
  const int col = lane & 31, h = lane >> 5;
  const uint32_t arow0 = (uint32_t)(64 * wm + col) * 128u;
  auto boff = [&](int j) -> uint32_t {
    int r;
    if constexpr (S == 2) {
      r = 32 * wn + 32 * j;  // gate rows below NR / 2: waves 0-3 gate, 4-7 up
    } else if constexpr (GATEUP) {
      constexpr int HJ = NJ / 2;  // gate tiles, then the matching up tiles
      r = (j < HJ ? 0 : NR / 2) + 32 * HJ * wn + 32 * (j % HJ);
    } else {
      r = 32 * NJ * wn + 32 * j;
    }
    return (uint32_t)(r + col) * 128u;
  };

  // the operand fragments of one 16-value step of a chunk: activations from
  // stage st, weights from buffer buf
  struct Frags {
    u32x4_t b[NJ], a[2];
  };
  auto read_frags = [&](auto st, int buf, int s, Frags& f) {
    const unsigned char* Ab = stage(st);
    const unsigned char* Bb = Bs + buf * BBUF;
    const uint32_t sw = (uint32_t)(((2 * s + h) ^ tile_swz(col)) << 4);
#pragma unroll
    for (int j = 0; j < NJ; j++) f.b[j] = *reinterpret_cast<const u32x4_t*>(Bb + boff(j) + sw);
#pragma unroll
    for (int i = 0; i < 2; i++) f.a[i] = *reinterpret_cast<const u32x4_t*>(Ab + arow0 + 32 * 128 * i + sw);
  };
  auto mma_step = [&](auto mv, const Frags& f) {
    constexpr int MV = decltype(mv)::value;
#pragma unroll
    for (int i = 0; i < MV; i++)
#pragma unroll
      for (int j = 0; j < NJ; j++) acc[i][j] = mma_f16(f.a[i], f.b[j], acc[i][j]);
  };
  // vector-memory instructions per thread: a chunk's activation copies, and
  // one chunk's scales, biases and codes
  constexpr int kCopyLoads = AI, kUnitSetLoads = BI * (1 + kUnitLoads<BITS>);
  // A chunk's activations were issued one chunk before its barrier, ahead of
  // that chunk's weight loads (in the program, and sched_barriers keep them
  // there); at most the weight loads of that chunk plus everything the next
  // chunk issued may then be outstanding.
  constexpr int kCopyWait = kCopyLoads + 2 * kUnitSetLoads;
  // Chunk c: activations in stage ST = c % 3, weights in buffer buf = c % 2.
  // Its first fragments are read as soon as the previous chunk's barrier has
  // passed, and the previous chunk's last MFMA step (operands already in
  // registers, `last`) is issued behind those reads, so the matrix cores work
  // while this chunk's first operands arrive. Then chunk c + 2's activations
  // go to stage (c + 2) % 3, which held chunk c - 1 (free since that
  // barrier), and chunk c + 3's scales, biases and codes to the register set
  // cb that chunk c used; chunk c + 1's weights (set nb) are dequantised into
  // the other buffer between the MFMA steps. This chunk's own last step is
  // left in `last`. Loads are unconditional (past the end they repeat the
  // last chunk, in bounds and never read) so that the compiler can count
  // outstanding loads exactly. MV: row tiles of this wave with positions of
  // the expert (0..2), a compile-time constant, so each version of the loop
  // is straight-line code.
  // TAIL: one of the last chunks, which issues only the loads of chunks that
  // exist and drains all loads before its barrier.
  auto chunk_step = [&](auto mv, auto pending, auto st, auto tail, int c, BUnits& cb,
                        const BUnits& nb, Frags& last) {
    constexpr int ST = decltype(st)::value;
    constexpr bool TAIL = decltype(tail)::value;
    const int buf = c & 1;
    Frags f0, f1;
    read_frags(st, buf, 0, f0);
    if constexpr (decltype(pending)::value) mma_step(mv, last);
    if (!TAIL || c + 2 < nchunks)
      dma_a(min(c + 2, nchunks - 1), std::integral_constant<int, (ST + 2) % 3>{});
    __builtin_amdgcn_sched_barrier(0);
    if (!TAIL || c + 3 < nchunks) {
      load_sb(min(c + 3, nchunks - 1), cb);
      load_w(min(c + 3, nchunks - 1), cb);
    }
    // keep chunk c + 3's loads issued here (sunk below the first weight
    // dequantisation they would turn its wait into a wait for every load)
    __builtin_amdgcn_sched_barrier(0);
    h2_t s2[BI], b2[BI];
    sb_pairs(nb, c + 1, s2, b2);
    read_frags(st, buf, 1, f1);
    mma_step(mv, f0);
    store_b(nb, s2, b2, 0, buf ^ 1);
    read_frags(st, buf, 2, f0);
    mma_step(mv, f1);
    store_b(nb, s2, b2, 1, buf ^ 1);
    read_frags(st, buf, 3, last);
    mma_step(mv, f0);
    store_b(nb, s2, b2, 2, buf ^ 1);
    store_b(nb, s2, b2, 3, buf ^ 1);
    // this wave's copies of chunk c + 1's activations have landed; the
    // barrier then publishes every wave's (the first chunk's follow only
    // its own loads: the prologue issued the copies last)
    if constexpr (TAIL) vmcnt_wait<0>();
    else if constexpr (!decltype(pending)::value) vmcnt_wait<kCopyLoads + kUnitSetLoads>();
    else vmcnt_wait<kCopyWait>();
    lds_barrier_copies_in_flight();
  };

  using S0_ = std::integral_constant<int, 0>;
  using S1_ = std::integral_constant<int, 1>;
  using S2_ = std::integral_constant<int, 2>;
  // The weights of chunks 0-2 need only the item; the activation copies
  // wait for the rows' positions (perm): weights first, copies last.
  BUnits u0, u1, u2;
  load_sb(0, u0);
  load_w(0, u0);
  load_sb(min(1, nchunks - 1), u1);
  load_w(min(1, nchunks - 1), u1);
  load_sb(min(2, nchunks - 1), u2);
  load_w(min(2, nchunks - 1), u2);
  __builtin_amdgcn_sched_barrier(0);
  set_xoff();
  dma_a(0, S0_{});
  dma_a(min(1, nchunks - 1), S1_{});
  __builtin_amdgcn_sched_barrier(0);
  {
    h2_t s2[BI], b2[BI];
    sb_pairs(u0, 0, s2, b2);
#pragma unroll
    for (int s = 0; s < 4; s++) store_b(u0, s2, b2, s, 0);
  }
  vmcnt_wait<kCopyLoads>();  // chunk 0's activations (only chunk 1's copies may remain)
  lds_barrier_copies_in_flight();

  // The trips of the loop issue every load unconditionally (each loads
  // chunks that exist); the last up to five chunks run as tail steps, which
  // issue no loads past the end, so that no load is still in flight when the
  // epilogue starts.
  auto run = [&](auto mv) {
    using Y = std::true_type;
    using F = std::false_type;
    Frags last;
    chunk_step(mv, F{}, S0_{}, F{}, 0, u0, u1, last);
    int c = 1;
    for (; c + 5 < nchunks; c += 3) {
      chunk_step(mv, Y{}, S1_{}, F{}, c, u1, u2, last);
      chunk_step(mv, Y{}, S2_{}, F{}, c + 1, u2, u0, last);
      chunk_step(mv, Y{}, S0_{}, F{}, c + 2, u0, u1, last);
    }
    if (c < nchunks) chunk_step(mv, Y{}, S1_{}, Y{}, c, u1, u2, last);
    if (c + 1 < nchunks) chunk_step(mv, Y{}, S2_{}, Y{}, c + 1, u2, u0, last);
    if (c + 2 < nchunks) chunk_step(mv, Y{}, S0_{}, Y{}, c + 2, u0, u1, last);
    if (c + 3 < nchunks) chunk_step(mv, Y{}, S1_{}, Y{}, c + 3, u1, u2, last);
    if (c + 4 < nchunks) chunk_step(mv, Y{}, S2_{}, Y{}, c + 4, u2, u0, last);
    mma_step(mv, last);
  };
  // mvalid is wave-uniform: one scalar branch picks the loop
  if (mvalid == 2) run(std::integral_constant<int, 2>{});
  else if (mvalid == 1) run(std::integral_constant<int, 1>{});
  else run(std::integral_constant<int, 0>{});
  // No load is in flight here unless K is a single chunk (the first step's
  // clamped copies), and the epilogue reuses LDS: drain them (the last
  // step's barrier already ordered every wave's reads of the staging areas)
  vmcnt_wait<0>();

  if constexpr (GATEUP && S == 2) {
    gateup_epilogue_split<XT>(a, L, acc, e, m0, bn, pend, wn, col, h, OSCALE);
    return;
  }
  // epilogue: lane holds column col, rows 8 (r / 4) + 4 h + r % 4 of each
  // 32 x 32 tile. The wave's outputs (64 rows x OC columns, 16-bit) go
  // through LDS (free after the last barrier) so that the global stores are
  // 16 contiguous bytes of one output row per lane.
  constexpr int OC = GATEUP ? NJ * 16 : NJ * 32;  // output columns per wave
  constexpr int HJ = GATEUP ? NJ / 2 : NJ;
  const int cbase = GATEUP ? bn * (NR / 2) + wn * OC : bn * NR + wn * OC;
  const XT* ob0 = reinterpret_cast<const XT*>(a.p0.ob);
  const XT* ob1 = reinterpret_cast<const XT*>(GATEUP ? a.p1.ob : a.p0.ob);
  // a wave's 64 x OC outputs take at most 16 KB: waves 0-3 stage them in the
  // weight buffers, waves 4-7 in the first two activation stages (each LDS
  // object holds only its own bytes)
  static_assert(64 * OC * 2 <= 16384, "epilogue staging");
  unsigned char* wreg = wave < 4 ? L.b + wave * 16384 : (wave < 6 ? L.a0 : L.a1) + (wave & 1) * 16384;
  uint16_t* wt = reinterpret_cast<uint16_t*>(wreg);
  // Straight-line per activation kind (a runtime switch inside the loop left
  // a branch per output), and per presence of an output bias: without one,
  // the sum is rounded once (adding -0, the identity, and rounding the
  // rounded value again would change nothing). A single projection that
  // writes the layer dtype (the routed down GEMM) takes its own copy too,
  // one conversion per output instead of both forms and a select.
  auto epilogue = [&](auto actc, auto biasc, auto xtc) {
    constexpr int ACT = decltype(actc)::value;
    constexpr bool BIAS = decltype(biasc)::value, XT_ONLY = decltype(xtc)::value;
#pragma unroll
    for (int j = 0; j < HJ; j++) {
      const int cn = cbase + 32 * j + col;
      float obg = -0.0f, obu = -0.0f;
      if constexpr (BIAS) {
        obg = (ob0 && cn < N) ? to_f<XT>(ob0[(size_t)e * N + cn]) : -0.0f;
        obu = (GATEUP && ob1 && cn < N) ? to_f<XT>(ob1[(size_t)e * N + cn]) : -0.0f;
      }
#pragma unroll
      for (int i = 0; i < 2; i++) {
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const int row = 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
          if constexpr (!GATEUP && !BIAS && XT_ONLY && ACT != ACT_RELU2) {
            // the stored value is the sum rounded once: one conversion
            wt[row * OC + 32 * j + col] = __builtin_bit_cast(uint16_t, from_f<XT>(acc[i][j][r] * OSCALE));
            continue;
          }
          float v = round_to<XT>(acc[i][j][r] * OSCALE);
          if constexpr (BIAS) v = round_to<XT>(v + obg);
          uint16_t bits;
          if constexpr (GATEUP) {
            float u = round_to<XT>(acc[i][j + HJ][r] * OSCALE);
            if constexpr (BIAS) u = round_to<XT>(u + obu);
            bits = __builtin_bit_cast(uint16_t, to_a16<XT>(apply_act<XT>(v, u, ACT, a.alpha, a.limit)));
          } else {
            // single projections: squared ReLU only
            const float y = ACT == ACT_RELU2 ? apply_act<XT>(0.f, v, ACT_RELU2, 0.f, 0.f) : v;
            const uint16_t as_xt = __builtin_bit_cast(uint16_t, from_f<XT>(y));
            if constexpr (XT_ONLY) {
              bits = as_xt;
            } else {
              const uint16_t as_a16 = __builtin_bit_cast(uint16_t, to_a16<XT>(y));
              bits = a.out_a16 ? as_a16 : as_xt;
            }
          }
          wt[row * OC + 32 * j + col] = bits;
        }
      }
    }
  };
  using kNo = std::false_type;
  using kYes = std::true_type;
  const bool has_bias = ob0 != nullptr || (GATEUP && ob1 != nullptr);
  auto by_bias = [&](auto actc, auto xtc) {
    if (has_bias) epilogue(actc, kYes{}, xtc);
    else epilogue(actc, kNo{}, xtc);
  };
  if constexpr (GATEUP) {
    if (a.act == ACT_GPTOSS) by_bias(std::integral_constant<int, ACT_GPTOSS>{}, kNo{});
    else if (a.act == ACT_GEGLU) by_bias(std::integral_constant<int, ACT_GEGLU>{}, kNo{});
    else by_bias(std::integral_constant<int, ACT_SWIGLU>{}, kNo{});
  } else {
    auto by_out = [&](auto actc) {
      if (a.out_a16) by_bias(actc, kNo{});
      else by_bias(actc, kYes{});
    };
    if (a.act == ACT_RELU2) by_out(std::integral_constant<int, ACT_RELU2>{});
    else by_out(std::integral_constant<int, ACT_SWIGLU>{});
  }
  // each lane: 16 bytes (8 columns) of one row per step; the wave reads only
  // its own region, so no block barrier is needed
  uint16_t* out = reinterpret_cast<uint16_t*>(a.out);
  constexpr int C8 = OC / 8;
#pragma unroll
  for (int t = 0; t < C8; t++) {
    const int q = 64 * t + lane;
    const int row = q / C8, c8 = q - row * C8;
    const uint32_t p = bstart + (uint32_t)row;
    const int cn0 = cbase + 8 * c8;
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(wt + row * OC + 8 * c8);
    if (p < pend && cn0 < N)  // N % 8 == 0 (host check): whole 16-byte groups
      *reinterpret_cast<u32x4_t*>(out + (size_t)p * N + cn0) = v;
  }
}

template <int BITS, typename XT, bool GATEUP>
__global__ __launch_bounds__(512) void gemm_grouped_kernel(const GemmArgs a) {
  __shared__ __align__(16) unsigned char a0[kAStageBytes], a1[kAStageBytes], a2[kAStageBytes];
  __shared__ __align__(16) unsigned char b[2 * kBBufBytes];
  // the items split into 8 contiguous ranges, one per XCD (blocks b, b + 8,
  // ... share an XCD)
  const uint32_t n = __builtin_amdgcn_readfirstlane(a.items[0]);
  const uint32_t per = (n + 7u) >> 3;
  const uint32_t j = blockIdx.x >> 3;
  if (j >= per) return;
  const uint32_t wi = (blockIdx.x & 7u) * per + j;
  if (wi >= n) return;
  const uint32_t tag = __builtin_amdgcn_readfirstlane(a.items[4 + 4 * wi]);
  const uint32_t m0 = __builtin_amdgcn_readfirstlane(a.items[5 + 4 * wi]);
  const int bn = (int)__builtin_amdgcn_readfirstlane(a.items[6 + 4 * wi]);
  const uint32_t pend = __builtin_amdgcn_readfirstlane(a.items[7 + 4 * wi]);
  const uint32_t e = tag & 0x3FFFFFFFu, shape = tag >> 30;
  const GemmLds L{a0, a1, a2, b};
  if (shape == 0) gemm_tile<0, BITS, XT, GATEUP>(a, L, e, m0, bn, pend);
  else if (shape == 1) gemm_tile<1, BITS, XT, GATEUP>(a, L, e, m0, bn, pend);
  else gemm_tile<2, BITS, XT, GATEUP>(a, L, e, m0, bn, pend);
}

template <int BITS, typename XT, bool GATEUP>
static hipError_t launch_gemm_v(const GemmArgs& a, int grid, hipStream_t st, KEvents ev) {
  hipExtLaunchKernelGGL((gemm_grouped_kernel<BITS, XT, GATEUP>), dim3(grid), dim3(512), 0, st,
                        ev.start, ev.stop, 0, a);
  return hipGetLastError();
}

#define MOE_CAT2(a, b) a##b
#define MOE_CAT(a, b) MOE_CAT2(a, b)

// A rows are f16 operands (A16 for a bf16 layer) in every case.
hipError_t MOE_CAT(launch_gemm_b, MOE_BITS)(int xdt, bool gateup, const GemmArgs& a, int grid,
                                             hipStream_t st, KEvents ev) {
  if (xdt == DT_BF16)
    return gateup ? launch_gemm_v<MOE_BITS, bf16_t, true>(a, grid, st, ev)
                  : launch_gemm_v<MOE_BITS, bf16_t, false>(a, grid, st, ev);
  if (xdt == DT_F16)
    return gateup ? launch_gemm_v<MOE_BITS, f16_t, true>(a, grid, st, ev)
                  : launch_gemm_v<MOE_BITS, f16_t, false>(a, grid, st, ev);
  return hipErrorInvalidValue;
}

}  // namespace moe
