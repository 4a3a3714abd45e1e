// dispatch.hip — deterministic token->expert dispatch plan for gfx950.
//
// Replaces the host plan of MoELayer.decodeMany (Sources/FFAI/Models/
// MoELayer.swift:752-792: token-major (expert, token, slot) tuples, a stable
// sort by expert, inv_perm) and the host CSR offsets of the m1 path
// (:1035-1058), with no host round trip:
//   1. histogram of expert ids (LDS atomics: counts are order independent),
//   2. exclusive scan -> CSR offsets, plus the ascending list of used experts,
//   3. stable permute: entries are ranked inside each wave with ballots over
//      the expert-id bits, waves are ordered inside a tile, tiles in order, so
//      position = offsets[e] + (#earlier entries with expert e). The result is
//      the stable order (expert asc, token asc, slot asc) bit for bit.
//
// Small plans run in one workgroup. Large plans (prefill) split the entries
// into chunks: a per-chunk histogram pass, a scan pass, and a scatter pass
// that starts every chunk at its own per-expert base.
#include "moe_common.hpp"
#include "moe_internal.hpp"

namespace moe {

constexpr int kPlanThreads = 256;
constexpr int kPlanMaxE = 1024;
constexpr int kChunk = 1024;             // entries per chunk in the multi-block plan
constexpr int kSingleBlockMax = 4096;    // M at or below which one workgroup plans

// Exclusive scan of cnt[0..E) over NT threads (4 experts per thread).
// Writes offsets[0..E], counts, the used list, and base[e] = offsets[e].
template <int NT = kPlanThreads>
__device__ void scan_experts(const uint32_t* cnt, int E, uint32_t* counts, uint32_t* offsets,
                             uint32_t* used, uint32_t* base) {
  __shared__ uint32_t wsum[NT / 64], wused[NT / 64];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  uint32_t c[4], f[4], tot = 0, ftot = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int e = tid * 4 + j;
    c[j] = e < E ? cnt[e] : 0u;
    f[j] = c[j] > 0 ? 1u : 0u;
    tot += c[j];
    ftot += f[j];
  }
  // inclusive wave scan of (tot, ftot) by DPP (shuffles put an LDS round
  // trip per step on the plan's chain)
  const uint32_t s = wave_scan_u32(tot), fs = wave_scan_u32(ftot);
  if (lane == 63) {
    wsum[wave] = s;
    wused[wave] = fs;
  }
  __syncthreads();
  // the earlier waves' totals, all read at once
  uint32_t wb = 0, fb = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; w++) {
    const uint32_t a = wsum[w], b = wused[w];
    wb += w < wave ? a : 0u;
    fb += w < wave ? b : 0u;
  }
  uint32_t run = wb + s - tot, frun = fb + fs - ftot;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int e = tid * 4 + j;
    if (e < E) {
      counts[e] = c[j];
      offsets[e] = run;
      base[e] = run;
      if (f[j]) used[1 + frun] = (uint32_t)e;
    }
    run += c[j];
    frun += f[j];
  }
  if (tid == NT - 1) {
    offsets[E] = run;
    used[0] = frun;
  }
  __syncthreads();
}

// Rank of this lane's entry among earlier lanes of the wave with the same
// expert, and the number of such lanes in the wave (valid lanes only).
__device__ __forceinline__ void wave_peers(uint32_t e, bool valid, int nbits, uint32_t* rank,
                                           uint32_t* count, bool* last) {
  const int lane = threadIdx.x & 63;
  uint64_t peers = __ballot(valid);
  for (int b = 0; b < nbits; b++) {
    const bool bit = (e >> b) & 1u;
    const uint64_t bal = __ballot(valid && bit);
    peers &= bit ? bal : ~bal;
  }
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  *rank = (uint32_t)__popcll(peers & below);
  *count = (uint32_t)__popcll(peers);
  *last = (peers >> lane) == 1ull;
}

// Ranks the entries [begin, end) in order and scatters them starting from
// cursor[e]; cursor ends advanced by the number of entries of each expert.
// NT threads; the waves take turns at the cursors, only those with entries.
template <int NT = kPlanThreads>
__device__ void stable_scatter(const uint32_t* __restrict__ idx, int begin, int end, int E,
                               int nbits, uint32_t* cursor, uint32_t* __restrict__ perm,
                               uint32_t* __restrict__ inv) {
  const int tid = threadIdx.x, wave = tid >> 6;
  for (int base = begin; base < end; base += NT) {
    const int m = base + tid;
    uint32_t e = m < end ? idx[m] : 0xffffffffu;
    const bool valid = m < end && e < (uint32_t)E;
    uint32_t rank, count;
    bool last;
    wave_peers(e, valid, nbits, &rank, &count, &last);
    const int nw = min(NT, end - base + 63) / 64;  // block-uniform
    for (int w = 0; w < nw; w++) {
      if (wave == w && valid) {
        const uint32_t pos = cursor[e] + rank;
        perm[pos] = (uint32_t)m;
        inv[m] = pos;
        if (last) cursor[e] += count;
      }
      __syncthreads();
    }
  }
}

// stable_scatter over entries [begin, begin + n) whose ids thread t already
// holds: ev[i] = the id of entry begin + t + NT i (n <= NT * PER), loaded
// all at once up front. Loading them tile by tile, after each tile's
// barriers, put one memory round trip per NT entries on the plan's
// critical path.
template <int NT, int PER>
__device__ void stable_scatter_held(const uint32_t (&ev)[PER], int begin, int n, int E, int nbits,
                                    uint32_t* cursor, uint32_t* __restrict__ perm,
                                    uint32_t* __restrict__ inv) {
  const int tid = threadIdx.x, wave = tid >> 6;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int base = i * NT;
    if (base >= n) break;  // block-uniform
    const int o = base + tid, m = begin + o;
    const uint32_t e = o < n ? ev[i] : 0xffffffffu;
    const bool valid = o < n && e < (uint32_t)E;
    uint32_t rank, count;
    bool last;
    wave_peers(e, valid, nbits, &rank, &count, &last);
    const int nw = min(NT, n - base + 63) / 64;  // block-uniform
    for (int w = 0; w < nw; w++) {
      if (wave == w && valid) {
        const uint32_t pos = cursor[e] + rank;
        perm[pos] = (uint32_t)m;
        inv[m] = pos;
        if (last) cursor[e] += count;
      }
      __syncthreads();
    }
  }
}

__device__ __forceinline__ int id_bits(int E) {
  int nb = 0;
  while ((1 << nb) < E) nb++;
  return nb;
}

__global__ __launch_bounds__(kPlanThreads) void plan_single_kernel(
    const uint32_t* __restrict__ idx, int M, int E, uint32_t* counts, uint32_t* offsets,
    uint32_t* perm, uint32_t* inv, uint32_t* used) {
  __shared__ uint32_t cnt[kPlanMaxE], cursor[kPlanMaxE];
  constexpr int PER = kSingleBlockMax / kPlanThreads;
  const int tid = threadIdx.x;
  // every id of this thread's entries in flight at once, kept for the scatter
  uint32_t ev[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int m = tid + i * kPlanThreads;
    ev[i] = m < M ? idx[m] : 0xffffffffu;
  }
  for (int e = tid; e < E; e += kPlanThreads) cnt[e] = 0;
  __syncthreads();
#pragma unroll
  for (int i = 0; i < PER; i++)
    if (ev[i] < (uint32_t)E) atomicAdd(&cnt[ev[i]], 1u);
  __syncthreads();
  scan_experts(cnt, E, counts, offsets, used, cursor);
  stable_scatter_held<kPlanThreads, PER>(ev, 0, M, E, id_bits(E), cursor, perm, inv);
}

// Routing and dispatch plan of a small batch in one launch: the NT / 64
// waves route tokens t = wave, wave + NT / 64, ... exactly as
// router_topk_kernel does (wave_topk, same results bit for bit), then the
// block plans the T * k entries as plan_single_kernel does, reading the ids
// from LDS. One wave per token past four tokens: the routing chain of a
// wave outlasts the launch it saves once a wave routes two tokens or more of
// a larger batch (Qwen3 shape, per layer step: 16 tokens on 4 waves 96.5 us
// against 90.7 us for the top-k and plan launches; 64 tokens on 16 waves
// 142.9 us against 133.6 us; 16 tokens on 16 waves 83.6 us against 84.4 us).
constexpr int kRoutePlanMaxT = 16;
constexpr int kRoutePlanMaxM = 1024;

template <typename XT, int EPL, int NT>
__global__ __launch_bounds__(NT) void route_plan_kernel(
    const XT* __restrict__ logits, int T, int E, int k, const RouteOpts ro, uint32_t* idx, float* w,
    uint32_t* counts, uint32_t* offsets, uint32_t* perm, uint32_t* inv, uint32_t* used) {
  __shared__ float sc[NT / 64][kTopkMaxE];
  __shared__ uint32_t sidx[kRoutePlanMaxM];
  __shared__ uint32_t cnt[kPlanMaxE], cursor[kPlanMaxE];
  const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
  const int M = T * k;
  for (int e = tid; e < E; e += NT) cnt[e] = 0;
  for (int t = wv; t < T; t += NT / 64) {  // wave-uniform
    int sel;
    float wt;
    wave_topk<XT, EPL>(logits + (size_t)t * E, E, k, ro, sc[wv], true, &sel, &wt);
    if (lane < k) {
      idx[t * k + lane] = (uint32_t)sel;
      w[t * k + lane] = wt;
      sidx[t * k + lane] = (uint32_t)sel;
    }
  }
  __syncthreads();
  for (int m = tid; m < M; m += NT) {
    const uint32_t e = sidx[m];
    if (e < (uint32_t)E) atomicAdd(&cnt[e], 1u);
  }
  __syncthreads();
  scan_experts<NT>(cnt, E, counts, offsets, used, cursor);
  stable_scatter<NT>(sidx, 0, M, E, id_bits(E), cursor, perm, inv);
}

hipError_t launch_route_plan(const void* logits, int dt, int T, int E, int k, const RouteOpts& ro,
                             uint32_t* idx, float* w, uint32_t* counts, uint32_t* offsets,
                             uint32_t* perm, uint32_t* inv, uint32_t* used, hipStream_t st) {
  if (T > kRoutePlanMaxT || T * k > kRoutePlanMaxM || E > kTopkMaxE || k > 64)
    return hipErrorInvalidValue;
#define MOE_RP(XT, EPL)                                                                          \
  if (T <= 4)                                                                                    \
    hipLaunchKernelGGL((route_plan_kernel<XT, EPL, kPlanThreads>), dim3(1), dim3(kPlanThreads),  \
                       0, st, (const XT*)logits, T, E, k, ro, idx, w, counts, offsets, perm, inv, \
                       used);                                                                    \
  else if (T <= 8)                                                                               \
    hipLaunchKernelGGL((route_plan_kernel<XT, EPL, 512>), dim3(1), dim3(512), 0, st,             \
                       (const XT*)logits, T, E, k, ro, idx, w, counts, offsets, perm, inv, used); \
  else                                                                                           \
    hipLaunchKernelGGL((route_plan_kernel<XT, EPL, 1024>), dim3(1), dim3(1024), 0, st,           \
                       (const XT*)logits, T, E, k, ro, idx, w, counts, offsets, perm, inv, used); \
  return hipGetLastError();
#define MOE_RP_E(XT)                  \
  if (E <= 64) { MOE_RP(XT, 1) }      \
  if (E <= 128) { MOE_RP(XT, 2) }     \
  if (E <= 256) { MOE_RP(XT, 4) }     \
  MOE_RP(XT, kTopkEPL)
  if (dt == DT_BF16) { MOE_RP_E(bf16_t) }
  if (dt == DT_F16) { MOE_RP_E(f16_t) }
  if (dt == DT_F32) { MOE_RP_E(float) }
#undef MOE_RP_E
#undef MOE_RP
  return hipErrorInvalidValue;
}

// Multi-block pass 1: per-chunk histograms, hist[c * E + e].
__global__ __launch_bounds__(kPlanThreads) void plan_hist_kernel(const uint32_t* __restrict__ idx,
                                                                 int M, int E,
                                                                 uint32_t* __restrict__ hist) {
  __shared__ uint32_t cnt[kPlanMaxE];
  const int tid = threadIdx.x, c = blockIdx.x;
  for (int e = tid; e < E; e += kPlanThreads) cnt[e] = 0;
  __syncthreads();
  const int begin = c * kChunk, end = min(M, begin + kChunk);
  for (int m = begin + tid; m < end; m += kPlanThreads) {
    const uint32_t e = idx[m];
    if (e < (uint32_t)E) atomicAdd(&cnt[e], 1u);
  }
  __syncthreads();
  for (int e = tid; e < E; e += kPlanThreads) hist[(size_t)c * E + e] = cnt[e];
}

// Multi-block pass 2 (one block): totals, scan, and each chunk's starting
// position per expert, written back over hist.
__global__ __launch_bounds__(kPlanThreads) void plan_scan_kernel(int nchunks, int E,
                                                                 uint32_t* __restrict__ hist,
                                                                 uint32_t* counts, uint32_t* offsets,
                                                                 uint32_t* used) {
  __shared__ uint32_t cnt[kPlanMaxE], base[kPlanMaxE];
  const int tid = threadIdx.x;
  // chunks in batches of kScanBatch: a batch's loads are all in flight
  // before the first add (one round trip per batch, not per chunk)
  constexpr int kScanBatch = 16;
  for (int e = tid; e < E; e += kPlanThreads) {
    uint32_t s = 0;
    for (int c0 = 0; c0 < nchunks; c0 += kScanBatch) {
      uint32_t h[kScanBatch];
#pragma unroll
      for (int j = 0; j < kScanBatch; j++)
        h[j] = (c0 + j < nchunks) ? hist[(size_t)(c0 + j) * E + e] : 0u;
#pragma unroll
      for (int j = 0; j < kScanBatch; j++) s += h[j];
    }
    cnt[e] = s;
  }
  __syncthreads();
  scan_experts(cnt, E, counts, offsets, used, base);
  for (int e = tid; e < E; e += kPlanThreads) {
    uint32_t run = base[e];
    for (int c0 = 0; c0 < nchunks; c0 += kScanBatch) {
      uint32_t h[kScanBatch];
#pragma unroll
      for (int j = 0; j < kScanBatch; j++)
        h[j] = (c0 + j < nchunks) ? hist[(size_t)(c0 + j) * E + e] : 0u;
#pragma unroll
      for (int j = 0; j < kScanBatch; j++) {
        if (c0 + j < nchunks) hist[(size_t)(c0 + j) * E + e] = run;
        run += h[j];
      }
    }
  }
}

// Multi-block pass 3: stable scatter of each chunk from its own bases.
__global__ __launch_bounds__(kPlanThreads) void plan_scatter_kernel(
    const uint32_t* __restrict__ idx, int M, int E, const uint32_t* __restrict__ hist,
    uint32_t* perm, uint32_t* inv) {
  __shared__ uint32_t cursor[kPlanMaxE];
  constexpr int PER = kChunk / kPlanThreads;
  const int tid = threadIdx.x, c = blockIdx.x;
  const int begin = c * kChunk, end = min(M, begin + kChunk);
  uint32_t ev[PER];  // the chunk's ids, all loads in flight at once
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int m = begin + tid + i * kPlanThreads;
    ev[i] = m < end ? idx[m] : 0xffffffffu;
  }
  for (int e = tid; e < E; e += kPlanThreads) cursor[e] = hist[(size_t)c * E + e];
  __syncthreads();
  stable_scatter_held<kPlanThreads, PER>(ev, begin, end - begin, E, id_bits(E), cursor, perm, inv);
}

__global__ void identity_plan_kernel(uint32_t* offsets, uint32_t* used, int M) {
  if (threadIdx.x == 0) {
    offsets[0] = 0;
    offsets[1] = (uint32_t)M;
    used[0] = 1;
    used[1] = 0;
  }
}

__global__ __launch_bounds__(kPlanThreads) void used_from_offsets_kernel(const uint32_t* offsets,
                                                                         int E, uint32_t* used) {
  __shared__ uint32_t cnt[kPlanMaxE], dummy_off[kPlanMaxE + 1], dummy_cnt[kPlanMaxE],
      dummy_base[kPlanMaxE];
  for (int e = threadIdx.x; e < E; e += kPlanThreads) cnt[e] = offsets[e + 1] - offsets[e];
  __syncthreads();
  scan_experts(cnt, E, dummy_cnt, dummy_off, used, dummy_base);
}

size_t dispatch_scratch_bytes(int T, int k, int E) {
  const long M = (long)T * k;
  if (M <= kSingleBlockMax) return 0;
  const long nchunks = (M + kChunk - 1) / kChunk;
  return (size_t)(nchunks * E * 4);
}

constexpr int kItemBlocks = 8;  // blocks writing the GEMM work items

struct ItemCols {
  int nb[2][kGemmShapes];  // column blocks per tile shape, for each of the two lists
};

// Work items of the grouped GEMM over an expert-sorted plan (the list format
// is described at launch_gemm_items). Thread t counts the items of experts
// t * EPT .. + EPT; a block scan gives every expert's first item (in LDS),
// the same in every block; then the threads of all blocks write items in a
// strided loop, each finding its expert by a binary search over those starts.
__device__ void gemm_items_body(const uint32_t* __restrict__ offsets, int E, const ItemCols& ic,
                                uint32_t* __restrict__ items0, uint32_t* __restrict__ items1,
                                int blk, int nblk) {
  __shared__ uint32_t scan[2][kPlanThreads];
  __shared__ uint32_t start[2][kPlanMaxE + 1];  // first item of each expert, per list
  __shared__ uint32_t first_pos[kPlanMaxE], rows_of[kPlanMaxE];
  constexpr int EPT = kPlanMaxE / kPlanThreads;  // experts per thread
  const int t = threadIdx.x;
  uint32_t cnt[2][EPT], tot0 = 0, tot1 = 0;
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const int e = t * EPT + j;
    uint32_t rows = 0, first = 0;
    if (e < E) {
      first = offsets[e];
      rows = offsets[e + 1] - first;
      first_pos[e] = first;
      rows_of[e] = rows;
    }
    const uint32_t full = rows / 256u, rem = rows % 256u;
    // the remainder takes the smallest shape that holds it
    const int rs = gemm_shape_for((int)rem);
    cnt[0][j] = full * (uint32_t)ic.nb[0][0] + (rem ? (uint32_t)ic.nb[0][rs] : 0u);
    cnt[1][j] = full * (uint32_t)ic.nb[1][0] + (rem ? (uint32_t)ic.nb[1][rs] : 0u);
    tot0 += cnt[0][j];
    tot1 += cnt[1][j];
  }
  scan[0][t] = tot0;
  scan[1][t] = tot1;
  __syncthreads();
  for (int off = 1; off < kPlanThreads; off <<= 1) {
    const uint32_t v0 = t >= off ? scan[0][t - off] : 0u;
    const uint32_t v1 = t >= off ? scan[1][t - off] : 0u;
    __syncthreads();
    scan[0][t] += v0;
    scan[1][t] += v1;
    __syncthreads();
  }
  uint32_t b0 = scan[0][t] - tot0, b1 = scan[1][t] - tot1;
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const int e = t * EPT + j;
    if (e < E) {
      start[0][e] = b0;
      start[1][e] = b1;
    }
    b0 += cnt[0][j];
    b1 += cnt[1][j];
  }
  const uint32_t n[2] = {scan[0][kPlanThreads - 1], scan[1][kPlanThreads - 1]};
  if (t == 0) {
    start[0][E] = n[0];
    start[1][E] = n[1];
    if (blk == 0) {
      items0[0] = n[0];
      if (items1) items1[0] = n[1];
    }
  }
  __syncthreads();
#pragma unroll
  for (int l = 0; l < 2; l++) {
    uint32_t* items = l ? items1 : items0;
    if (!items) continue;
    const uint32_t nb0 = (uint32_t)ic.nb[l][0];
    for (uint32_t i = (uint32_t)blk * kPlanThreads + (uint32_t)t; i < n[l];
         i += (uint32_t)nblk * kPlanThreads) {
      // the last expert whose first item is at or before i (experts without
      // items share their start with the next one)
      int lo = 0, hi = E - 1;
      while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (start[l][mid] <= i) lo = mid;
        else hi = mid - 1;
      }
      const uint32_t e = (uint32_t)lo, k = i - start[l][lo];
      const uint32_t rows = rows_of[e], full = rows / 256u;
      uint32_t tile, b, shape;
      if (k < full * nb0) {
        tile = k / nb0;
        b = k - tile * nb0;
        shape = 0u;
      } else {
        const uint32_t rem = rows % 256u;
        tile = full;
        b = k - full * nb0;
        shape = (uint32_t)gemm_shape_for((int)rem);
      }
      uint32_t* it = items + 4 + 4 * i;
      it[0] = e | (shape << 30);
      it[1] = first_pos[e] + tile * 256u;
      it[2] = b;
      it[3] = first_pos[e] + rows;
    }
  }
}

__global__ __launch_bounds__(kPlanThreads) void gemm_items_kernel(
    const uint32_t* __restrict__ offsets, int E, const ItemCols ic, uint32_t* __restrict__ items0,
    uint32_t* __restrict__ items1) {
  gemm_items_body(offsets, E, ic, items0, items1, (int)blockIdx.x, (int)gridDim.x);
}

// Multi-block pass 3 with the grouped GEMM's work items: each block scatters
// its chunk as plan_scatter_kernel does, then writes a strided share of the
// items as gemm_items_kernel does (they need only the offsets, which the
// scan pass wrote). One launch fewer per prefill step.
__global__ __launch_bounds__(kPlanThreads) void plan_scatter_items_kernel(
    const uint32_t* __restrict__ idx, int M, int E, const uint32_t* __restrict__ hist,
    uint32_t* perm, uint32_t* inv, const uint32_t* __restrict__ offsets, const ItemCols ic,
    uint32_t* __restrict__ items0, uint32_t* __restrict__ items1) {
  __shared__ uint32_t cursor[kPlanMaxE];
  constexpr int PER = kChunk / kPlanThreads;
  const int tid = threadIdx.x, c = blockIdx.x;
  const int begin = c * kChunk, end = min(M, begin + kChunk);
  uint32_t ev[PER];  // the chunk's ids, all loads in flight at once
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int m = begin + tid + i * kPlanThreads;
    ev[i] = m < end ? idx[m] : 0xffffffffu;
  }
  for (int e = tid; e < E; e += kPlanThreads) cursor[e] = hist[(size_t)c * E + e];
  __syncthreads();
  stable_scatter_held<kPlanThreads, PER>(ev, begin, end - begin, E, id_bits(E), cursor, perm, inv);
  gemm_items_body(offsets, E, ic, items0, items1, c, (int)gridDim.x);
}

static ItemCols item_cols(int N0, bool gateup0, int N1, bool gateup1, bool two) {
  ItemCols ic{};
  for (int sh = 0; sh < kGemmShapes; sh++) {
    ic.nb[0][sh] = (N0 + gemm_cols(sh, gateup0) - 1) / gemm_cols(sh, gateup0);
    ic.nb[1][sh] = two ? (N1 + gemm_cols(sh, gateup1) - 1) / gemm_cols(sh, gateup1) : 0;
  }
  return ic;
}

hipError_t launch_dispatch_plan(const uint32_t* idx, int T, int k, int E, uint32_t* counts,
                                uint32_t* offsets, uint32_t* perm, uint32_t* inv_perm,
                                uint32_t* used, void* scratch, size_t scratch_bytes,
                                hipStream_t st, const GemmItemsReq* items, bool* items_done) {
  if (items_done) *items_done = false;
  const int M = T * k;
  if (E > kPlanMaxE) return hipErrorInvalidValue;
  if (M <= kSingleBlockMax) {
    hipLaunchKernelGGL(plan_single_kernel, dim3(1), dim3(kPlanThreads), 0, st, idx, M, E, counts,
                       offsets, perm, inv_perm, used);
    return hipGetLastError();
  }
  const int nchunks = (M + kChunk - 1) / kChunk;
  if (scratch == nullptr || scratch_bytes < (size_t)nchunks * E * 4) return hipErrorInvalidValue;
  uint32_t* hist = reinterpret_cast<uint32_t*>(scratch);
  hipLaunchKernelGGL(plan_hist_kernel, dim3(nchunks), dim3(kPlanThreads), 0, st, idx, M, E, hist);
  hipLaunchKernelGGL(plan_scan_kernel, dim3(1), dim3(kPlanThreads), 0, st, nchunks, E, hist,
                     counts, offsets, used);
  if (items) {
    const ItemCols ic = item_cols(items->N0, items->gateup0, items->N1, items->gateup1,
                                  items->items1 != nullptr);
    hipLaunchKernelGGL(plan_scatter_items_kernel, dim3(nchunks), dim3(kPlanThreads), 0, st, idx,
                       M, E, hist, perm, inv_perm, offsets, ic, items->items0, items->items1);
    if (items_done) *items_done = true;
  } else {
    hipLaunchKernelGGL(plan_scatter_kernel, dim3(nchunks), dim3(kPlanThreads), 0, st, idx, M, E,
                       hist, perm, inv_perm);
  }
  return hipGetLastError();
}

hipError_t launch_gemm_items(const uint32_t* offsets, int E, int N0, bool gateup0,
                             uint32_t* items0, int N1, bool gateup1, uint32_t* items1,
                             hipStream_t st) {
  if (E > kPlanMaxE) return hipErrorInvalidValue;
  const ItemCols ic = item_cols(N0, gateup0, N1, gateup1, items1 != nullptr);
  // every block scans the experts' item counts (cheap) and writes a strided
  // share of the items
  hipLaunchKernelGGL(gemm_items_kernel, dim3(kItemBlocks), dim3(kPlanThreads), 0, st, offsets, E, ic, items0,
                     items1);
  return hipGetLastError();
}

hipError_t launch_identity_plan(uint32_t* offsets, uint32_t* used, int M, hipStream_t st) {
  hipLaunchKernelGGL(identity_plan_kernel, dim3(1), dim3(64), 0, st, offsets, used, M);
  return hipGetLastError();
}

hipError_t launch_used_from_offsets(const uint32_t* offsets, int E, uint32_t* used,
                                    hipStream_t st) {
  if (E > kPlanMaxE) return hipErrorInvalidValue;
  hipLaunchKernelGGL(used_from_offsets_kernel, dim3(1), dim3(kPlanThreads), 0, st, offsets, E,
                     used);
  return hipGetLastError();
}

}  // namespace moe
