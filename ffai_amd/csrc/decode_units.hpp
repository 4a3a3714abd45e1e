// decode_units.hpp — per-unit building blocks of the decode kernels
// (gemv.hip): activation units in pair order, packed weight
// units with their group scale and bias, and the wave-uniform expert views
// the one-token kernels address their loads through.
#pragma once

#include "moe_common.hpp"
#include "moe_internal.hpp"

namespace moe {
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

// One weight unit with its group scale and bias. Scale and bias stay in
// their storage type until use, so loads are not forced to complete early.
template <int BITS, typename ST> struct WUnit {
  uint32_t w[BITS];
  ST s_raw, b_raw;
  __device__ __forceinline__ float s() const { return to_f<ST>(s_raw); }
  __device__ __forceinline__ float b() const { return to_f<ST>(b_raw); }
};

// p points at one expert (see expert_proj); row < N, so the offsets fit in
// 32 bits and the loads use a scalar base with a 32-bit vector offset.
template <int BITS, typename ST>
__device__ __forceinline__ void load_w_unit(const GemvProj& p, uint32_t row, int row_words, int groups,
                                            int gsh, int u, WUnit<BITS, ST>& wu) {
  load_unit<BITS>(p.w + (row * (uint32_t)row_words + (uint32_t)(u * BITS)), wu.w);
  const uint32_t gi = row * (uint32_t)groups + (uint32_t)(u >> gsh);
  wu.s_raw = reinterpret_cast<const ST*>(p.s)[gi];
  wu.b_raw = reinterpret_cast<const ST*>(p.b)[gi];
}

// The projection of expert e alone (pointers advanced to its first row).
template <int BITS, typename ST>
__device__ __forceinline__ GemvProj expert_proj(const GemvProj& p, uint32_t e, int N, int row_words,
                                                int groups) {
  GemvProj q;
  q.w = p.w + (size_t)e * N * row_words;
  q.s = reinterpret_cast<const ST*>(p.s) + (size_t)e * N * groups;
  q.b = reinterpret_cast<const ST*>(p.b) + (size_t)e * N * groups;
  q.ob = p.ob;
  return q;
}

template <typename XT>
__device__ __forceinline__ float finish_proj(float acc, const void* ob, size_t obi) {
  float v = round_to<XT>(acc);
  if (ob) v = round_to<XT>(v + to_f<XT>(reinterpret_cast<const XT*>(ob)[obi]));
  return v;
}

// ---------------------------------------------------------------------------
// one-token kernels: expert views and unit loads
//
// The one-token kernels hold one expert per wave at a time, so the expert's weight,
// scale and bias arrays are addressed through wave-uniform buffer resources
// and every load is a 32-bit lane offset (no per-unit 64-bit address math).
// A lane's units are u = li + j L; units at or past CU read the next row's
// bytes, or zeros past the expert's end, and are masked out of the sums.
// ---------------------------------------------------------------------------

struct ProjView {
  rsrc_t w, s, b;
};

template <int BITS, typename ST>
__device__ __forceinline__ ProjView proj_view(const GemvProj& p, uint32_t e, int N, int row_words,
                                              int groups) {
  const size_t rows = (size_t)e * (size_t)N;
  ProjView v;
  v.w = make_rsrc(p.w + rows * row_words, (uint32_t)N * (uint32_t)row_words * 4u);
  v.s = make_rsrc(reinterpret_cast<const ST*>(p.s) + rows * groups,
                  (uint32_t)N * (uint32_t)groups * (uint32_t)sizeof(ST));
  v.b = make_rsrc(reinterpret_cast<const ST*>(p.b) + rows * groups,
                  (uint32_t)N * (uint32_t)groups * (uint32_t)sizeof(ST));
  return v;
}

// Byte offsets of a lane's first unit in `row`; unit j adds j * wstep and
// j * sstep (wstep = L * BITS * 4, sstep = (L >> gsh) * sizeof(ST); the host
// keeps L a multiple of the units per scale group, 1 << gsh).
struct UnitAddr {
  uint32_t w0, s0;
};

template <int BITS, typename ST>
__device__ __forceinline__ UnitAddr unit_addr(uint32_t row, int row_words, int groups, int li,
                                              int gsh) {
  UnitAddr a;
  a.w0 = row * (uint32_t)(row_words * 4) + (uint32_t)(li * BITS * 4);
  a.s0 = (row * (uint32_t)groups + (uint32_t)(li >> gsh)) * (uint32_t)sizeof(ST);
  return a;
}

template <int BITS, typename ST, int UR, int AUX = 0>
__device__ __forceinline__ void bload_units(const ProjView& v, UnitAddr ad, uint32_t wstep,
                                            uint32_t sstep, WUnit<BITS, ST> (&u)[UR]) {
#pragma unroll
  for (int j = 0; j < UR; j++) {
    bload_unit<BITS, AUX>(v.w, ad.w0 + (uint32_t)j * wstep, u[j].w);
    u[j].s_raw = __builtin_bit_cast(ST, bload16<AUX>(v.s, ad.s0 + (uint32_t)j * sstep));
    u[j].b_raw = __builtin_bit_cast(ST, bload16<AUX>(v.b, ad.s0 + (uint32_t)j * sstep));
  }
}

template <int BITS, typename XT, typename ST, int UR>
__device__ __forceinline__ float dot_units(const WUnit<BITS, ST> (&w)[UR],
                                           const XUnit<XT> (&xu)[UR], const float (&xs)[UR],
                                           int li, int L, int CU) {
  constexpr float MAGIC = Magic<BITS, XT>::value;
  float acc = 0.f;
#pragma unroll
  for (int j = 0; j < UR; j++) {
    uint32_t cp[16];
    unpack_pairs<BITS, Magic<BITS, XT>::bits>(w[j].w, cp);
    const float sc = w[j].s();
    const float v = sc * dot_unit<BITS, XT>(cp, xu[j]) + (w[j].b() - MAGIC * sc) * xs[j];
    acc += (li + j * L < CU) ? v : 0.f;
  }
  return acc;
}

// One activation row (16-bit types) into registers in pair order; units past
// the row read zeros.
template <int BITS, typename XT, int UR>
__device__ __forceinline__ void bload_x_units(rsrc_t xr, int li, int L, XUnit<XT> (&xu)[UR],
                                              float (&xs)[UR]) {
#pragma unroll
  for (int j = 0; j < UR; j++) {
    const uint32_t off = (uint32_t)(li + j * L) * 64u;
    uint32_t n[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const u32x4_t v = bload128(xr, off + 16u * q);
      n[4 * q] = v[0]; n[4 * q + 1] = v[1]; n[4 * q + 2] = v[2]; n[4 * q + 3] = v[3];
    }
    natural_to_pairs<BITS>(n, xu[j].v);
    xs[j] = sum16(n, __is_same(XT, bf16_t));
  }
}

// Cooperative copy of one 16-bit activation row (K % 32 == 0) into LDS by
// threads t = 0..nt-1 of a block: every load is issued before the first LDS
// write (one round trip). Needs NPT nt >= K / 8; offsets past the row read
// zeros without touching memory and are not written.
template <typename XT, int NPT>
__device__ __forceinline__ void stage_x_row(const XT* x, int K, uint32_t* xl, int t, int nt) {
  const int n16 = K * (int)sizeof(XT) / 16;
  const rsrc_t r = make_rsrc(x, (uint32_t)(K * sizeof(XT)));
  u32x4_t v[NPT];
#pragma unroll
  for (int j = 0; j < NPT; j++) v[j] = bload128(r, (uint32_t)(t + j * nt) * 16u);
#pragma unroll
  for (int j = 0; j < NPT; j++) {
    const int i = t + j * nt;
    if (i < n16) *reinterpret_cast<uint4*>(xl + 4 * i) = make_uint4(v[j][0], v[j][1], v[j][2], v[j][3]);
  }
}

// Cooperative copy of `rows` 16-bit activation rows of K values (row r at
// src_r(r)) into LDS already in pair order: unit u of row r is 16 pair words
// at xl + (r CU + u) 16 and its sum at xs[r CU + u], so that the lanes that
// multiply the unit read it as it is. Threads t = 0..nt-1 of a block take
// units t, t + nt, ...; each batch of up to NB units has every load issued
// before its first conversion.
template <int BITS, typename XT, int NB, typename SRC>
__device__ __forceinline__ void stage_x_pairs(SRC src_r, int rows, int K, uint32_t* xl, float* xs,
                                              int t, int nt) {
  const int CU = K >> 5, total = rows * CU;
  for (int base = t; base < total; base += NB * nt) {
    u32x4_t v[NB][4];
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const int g = min(base + b * nt, total - 1), r = g / CU, u = g - r * CU;
      const rsrc_t rr = make_rsrc(src_r(r), (uint32_t)(K * sizeof(XT)));
#pragma unroll
      for (int q = 0; q < 4; q++) v[b][q] = bload128(rr, (uint32_t)u * 64u + 16u * q);
    }
#pragma unroll
    for (int b = 0; b < NB; b++) {
      const int g = base + b * nt;
      if (g < total) {
        uint32_t n[16], x16[16];
#pragma unroll
        for (int q = 0; q < 4; q++) {
          n[4 * q] = v[b][q][0]; n[4 * q + 1] = v[b][q][1];
          n[4 * q + 2] = v[b][q][2]; n[4 * q + 3] = v[b][q][3];
        }
        natural_to_pairs<BITS>(n, x16);
        uint4* d = reinterpret_cast<uint4*>(xl + 16 * g);
#pragma unroll
        for (int q = 0; q < 4; q++) d[q] = make_uint4(x16[4 * q], x16[4 * q + 1], x16[4 * q + 2], x16[4 * q + 3]);
        xs[g] = sum16(n, __is_same(XT, bf16_t));
      }
    }
  }
}

// Units li + j L (j < UR) of row r staged by stage_x_pairs; units past CU
// repeat the last unit (the dot products mask them out).
template <typename XT, int UR>
__device__ __forceinline__ void lds_x_units_pairs(const uint32_t* xl, const float* xs, int r, int li,
                                                  int L, int CU, XUnit<XT> (&xu)[UR],
                                                  float (&xsum)[UR]) {
#pragma unroll
  for (int j = 0; j < UR; j++) {
    const int g = r * CU + min(li + j * L, CU - 1);
    const uint4* p = reinterpret_cast<const uint4*>(xl + 16 * g);
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint4 v = p[q];
      xu[j].v[4 * q] = v.x; xu[j].v[4 * q + 1] = v.y; xu[j].v[4 * q + 2] = v.z; xu[j].v[4 * q + 3] = v.w;
    }
    xsum[j] = xs[g];
  }
}

// Units li + j L (j < UR) of a 16-bit activation row staged in LDS (natural
// order, 16 dwords per unit) into pair order with their sums. Units past CU
// repeat the last unit; the dot products mask them out.
template <int BITS, typename XT, int UR>
__device__ __forceinline__ void lds_x_units_nat(const uint32_t* row, int li, int L, int CU,
                                                XUnit<XT> (&xu)[UR], float (&xs)[UR]) {
#pragma unroll
  for (int j = 0; j < UR; j++) {
    const uint4* p = reinterpret_cast<const uint4*>(row + 16 * min(li + j * L, CU - 1));
    uint32_t n[16];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint4 v = p[q];
      n[4 * q] = v.x; n[4 * q + 1] = v.y; n[4 * q + 2] = v.z; n[4 * q + 3] = v.w;
    }
    natural_to_pairs<BITS>(n, xu[j].v);
    xs[j] = sum16(n, __is_same(XT, bf16_t));
  }
}

}  // namespace moe
