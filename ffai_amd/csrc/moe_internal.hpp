// moe_internal.hpp — argument blocks and launchers shared between the C-ABI
// layer (api.cpp) and the kernel translation units. Host code only sees
// plain pointers; every launcher returns hipSuccess or the launch error.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace moe {

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2 };

// The thread-local text behind moe_last_error_string() (api.cpp), shared by
// every translation unit of the C ABI.
void set_error_text(const char* msg);
void clear_error_text();

// Optional events recorded by the dispatch of one kernel itself (its start
// and end timestamps, hipExtLaunchKernel); null entries record nothing.
struct KEvents {
  hipEvent_t start = nullptr, stop = nullptr;
};

// Routing options beyond the gating mode (the families after MoERouter):
//   gating 0 softmax -> top-k, 1 top-k -> softmax (MoELayer.swift:140-205),
//          2 sigmoid scores, ebias added for the selection only, weights the
//          raw sigmoids, renormalised by their sum + 1e-20 when norm and
//          k > 1 (NemotronHText.swift:700-725, 838-868);
//   logit_scale multiplies the logits in fp32 before anything else (Gemma 4
//          folds hidden^-0.5 there, Gemma4Text.swift:938-944);
//   routed_scale multiplies the final weights (NemotronH
//          routed_scaling_factor), then escale[e] (nullable, Gemma 4
//          per_expert_scale, Gemma4Text.swift:945-950).
struct RouteOpts {
  int gating, norm;
  const float* ebias;
  float logit_scale, routed_scale;
  const float* escale;
};

// ------------------------------------------------------------------ GEMV --
// Expert-grouped dequant GEMV over a dispatch plan. Block b handles expert
// slot b / row_blocks (the slot-th used expert) and rows
// [rb*rows_per_block, ...) of its N output rows for every sorted position of
// that expert.
struct GemvProj {
  const uint32_t* w;     // [E, N, K*bits/32]
  const void* s;         // [E, N, K/gs] sb dtype
  const void* b;         // [E, N, K/gs] sb dtype
  const void* ob;        // nullable [E, N] activation dtype
};

struct GemvArgs {
  GemvProj p0, p1;           // p0 = gate (or the single projection), p1 = up
  const void* x;             // activation rows, [rows, K]
  const uint32_t* perm;      // nullable: row(p) = perm[p] / topk, else row(p) = p
  int topk;
  const uint32_t* offsets;   // [E+1] CSR over sorted positions
  const uint32_t* used;      // [1+E]: used[0] = U, used[1..U] = expert ids
  void* out;                 // [M, N]
  int N, K;
  int gsh;                   // log2(group size / 32)
  int row_blocks, rows_per_block;
  int lg;                    // log2(lanes per row)
  int tok_chunk;             // activation rows staged per pass (<= TOKMAX)
  int act;                   // activation (gate/up pair only)
  float alpha, limit;
  int x_rows;                // rows of x (gemv_mma_kernel reads them through a buffer view)
};

// Decode of one token (T = 1). gate/up kernel: every wave selects the top-k
// from the router logits itself; block 0 publishes the routing. down kernel:
// fused weighted combine over the k experts.
// The one-token kernels over T tokens (grid.y = T): block row t routes and
// computes token t on its own (its slots' weights are read once per token,
// so a few tokens at most).
struct Decode1Args {
  const void* logits;        // [T, E] activation dtype
  int E, k, T;
  RouteOpts ro;
  uint32_t* idx;             // [T, k] out: experts in rank order
  float* w;                  // [T, k] out: combine weights
  uint32_t* perm;            // nullable [k] out (T = 1): sorted position -> rank
  uint32_t* offsets;         // nullable [E+1] out (T = 1): CSR offsets of the plan
  const void* x;             // [T, K]
  GemvProj g, u;             // gate / up
  void* act;                 // [T, k, N] in rank order
  int N, K, gsh, row_blocks, rows_per_block, lg;
  int act_kind;
  float alpha, limit;
  // A shared expert in the same launch (s_blocks > 0, T = 1 only): blocks k * row_blocks
  // onwards compute its SN gate/up rows (one-expert projections sg / su,
  // same bits, group size and scale dtype as g / u) into s_act; with sgw (a
  // dense gate row [K] in the activation dtype) one more block computes the
  // sigmoid gate's logit into s_logit[0].
  GemvProj sg, su;
  void* s_act;               // [SN]
  int SN, s_blocks;
  const void* sgw;           // nullable
  void* s_logit;             // [1]
};

struct Down1Args {
  const uint32_t* idx;       // [T, k] experts in rank order
  const float* w;            // [T, k] combine weights in rank order
  const void* act;           // [T, k, K] in rank order
  GemvProj p;
  void* out;                 // [T, N]
  const void* res;           // nullable [T, N]: residual added before the final rounding
  int k, N, K, gsh, rows_per_block, lg, T;
  // A shared expert as m more waves (m > 0, T = 1 only): wave k + j reads columns
  // [j K, (j + 1) K) of the rows of sp (one expert, m K columns, same bits,
  // group size and scale dtype as p) against s_act[j K, ...); the waves'
  // sum is rounded (then its output bias added and rounded) and added to
  // the rounded routed combine with the weight sigmoid(s_logit[0]) (1 when
  // s_logit is null), as the separate shared-expert path adds it.
  GemvProj sp;
  const void* s_act;         // [m K]
  const void* s_logit;       // nullable [1]
  int m;
};

// Launch limits of the decode kernels: a block has one wave per selected
// expert (down) and each lane holds at most kDec1MaxRows rows of at most 4
// units each.
constexpr int kDec1MaxK = 8;
// Waves of a down1_kernel block with a shared expert: k routed + m shared.
constexpr int kDec1MaxWaves = 12;
constexpr int kDec1MaxRows = 2;
constexpr int kDec1MaxHidden = 8192;  // activation row staged in LDS
// Weight rows per lane of gemv_multi_kernel: one, for a gate/up pair and for
// a single projection alike. Two rows per lane for a single projection held
// the down kernel at 208 VGPRs (two waves per SIMD) and measured 1-3 % slower
// per layer step on every batched decode shape (Qwen3 16 tokens 87.4 ->
// 84.8 us, GPT-OSS 16 tokens 173.2 -> 169.8 us with one row).
constexpr int kMultiRows(bool gateup) { return gateup ? 1 : 1; }

// rm: rows per lane (rows_per_block = rm * 4 * SG for gate/up, rm * SG for
// down).
hipError_t launch_gateup1(int bits, int xdt, int sbdt, const Decode1Args& a, int rm, int grid,
                          hipStream_t st, KEvents ev = {});
hipError_t launch_down1(int bits, int xdt, int sbdt, const Down1Args& a, int rm, int grid,
                        hipStream_t st, KEvents ev = {});

hipError_t launch_gemv(int bits, int xdt, int sbdt, bool gateup, int tokmax, const GemvArgs& a,
                       int grid, hipStream_t st, KEvents ev = {});
size_t gemv_smem_bytes(int xdt, int K, int tok_chunk);

// ---------------------------------------------------------------- router --
// x16 (nullable): where the many-token matrix-core kernel, for bf16 rows,
// also writes the rows as the expert GEMMs' f16 operand (launch_to_a16's
// values); *x16_done tells whether it did. W2 / E2 / logits2 (nullable): a
// second projection of the same rows with weights of W's type and no bias
// (a shared expert's gate), which that kernel computes in the same launch;
// *second_done tells whether it did (else the caller launches it).
// part / part_bytes / splits: fp32 scratch that a batch of few token tiles on
// the matrix cores may split K over; *splits > 1 then means that neither
// logits nor logits2 is written yet: launch_router_topk with the same part,
// splits, bias and logits2 adds the partials, rounds and writes both.
hipError_t launch_router_logits(const void* x, int xdt, int T, int H, const void* W, int wdt,
                                const void* bias, int E, void* logits, hipStream_t st,
                                void* x16 = nullptr, bool* x16_done = nullptr,
                                const void* W2 = nullptr, int E2 = 0, void* logits2 = nullptr,
                                bool* second_done = nullptr, float* part = nullptr,
                                size_t part_bytes = 0, int* splits = nullptr);
hipError_t launch_router_topk(void* logits, int dt, int T, int E, int k, const RouteOpts& ro,
                              uint32_t* idx, float* w, hipStream_t st, const float* part = nullptr,
                              int KS = 1, const void* bias = nullptr, void* logits2 = nullptr,
                              int E2 = 0);
// One token: res = round(h + m), xn = round(rmsnorm(res) * nw), then the
// router logits of xn, in one launch. 16-bit x and W of one type, H <= 8192;
// hipErrorInvalidValue otherwise (launch_add_rmsnorm + launch_router_logits).
hipError_t launch_router_logits_norm(const void* h, const void* m, const void* nw, float eps,
                                     int xdt, int H, const void* W, int wdt, const void* bias,
                                     int E, void* logits, void* res_out, void* xn_out,
                                     hipStream_t st);

// Router logits with an affine-quantised weight W (one stacked projection
// [1, E, H], codes of `bits`, scales in sbdt, log2(group size / 32) = gsh):
// 16-bit x / bias / logits of type xdt, H % 32 == 0, H <= 8192.
hipError_t launch_router_q(int bits, const void* x, int xdt, int T, int H, const GemvProj& W,
                           int sbdt, int gsh, const void* bias, int E, void* logits,
                           hipStream_t st);

// ------------------------------------------------------------- dispatch --
// Writes counts, offsets, perm, inv_perm and the used-expert list.
// launch_router_topk + launch_dispatch_plan in one workgroup for T <= 16,
// T * k <= 1024, E <= 512 and k <= 64 (hipErrorInvalidValue otherwise,
// nothing launched).
hipError_t launch_route_plan(const void* logits, int dt, int T, int E, int k, const RouteOpts& ro,
                             uint32_t* idx, float* w, uint32_t* counts, uint32_t* offsets,
                             uint32_t* perm, uint32_t* inv, uint32_t* used, hipStream_t st);
// The grouped GEMM's work items (launch_gemm_items arguments) to be written
// by the plan's last launch.
struct GemmItemsReq {
  int N0;
  bool gateup0;
  uint32_t* items0;
  int N1;
  bool gateup1;
  uint32_t* items1;  // nullptr: one list
};
// With `items`, a multi-block plan also writes the GEMM work items (then
// *items_done is set; a one-workgroup plan leaves them to launch_gemm_items).
hipError_t launch_dispatch_plan(const uint32_t* idx, int T, int k, int E, uint32_t* counts,
                                uint32_t* offsets, uint32_t* perm, uint32_t* inv_perm,
                                uint32_t* used, void* scratch, size_t scratch_bytes,
                                hipStream_t st, const GemmItemsReq* items = nullptr,
                                bool* items_done = nullptr);
size_t dispatch_scratch_bytes(int T, int k, int E);
// Fills offsets {0, M}, used {1, 0} for a single-expert identity plan.
hipError_t launch_identity_plan(uint32_t* offsets, uint32_t* used, int M, hipStream_t st);
// Builds the used list from CSR offsets only (caller-supplied plans).
hipError_t launch_used_from_offsets(const uint32_t* offsets, int E, uint32_t* used,
                                    hipStream_t st);

// -------------------------------------------------------------- combine --
hipError_t launch_unpermute(const void* Y, const uint32_t* inv, const float* w, int T, int H,
                            int k, void* out, int dt, const void* shared_out,
                            const void* shared_logit, int shared_mode, hipStream_t st,
                            const void* res = nullptr);
hipError_t launch_add_shared(void* y, const void* shared_out, const void* shared_logit,
                             int shared_mode, int T, int H, int dt, hipStream_t st,
                             const void* res = nullptr);
// Per row: res = round(a + b), xn = round(res / sqrt(mean(res^2) + eps) * w);
// H a multiple of 8, at most 8192; rows 16-byte aligned.
hipError_t launch_add_rmsnorm(const void* a, const void* b, const void* w, float eps, int T,
                              int H, int dt, void* res, void* xn, hipStream_t st);
hipError_t launch_activation(const void* g, const void* u, void* out, int64_t n, int dt,
                             int act, float alpha, float limit, hipStream_t st);
hipError_t launch_dequantize(const uint32_t* w, const void* s, const void* b, int sbdt, int bits,
                             int gs, int64_t numel, void* out, int odt, hipStream_t st);

// ---------------------------------------------------------------- MXFP4 --
// MXFP4 groups (4 packed u32 + 1 e8m0 byte each) -> affine 4-bit, group 32;
// out_w may be `packed` itself (the codes keep their nibbles).
hipError_t launch_mxfp4_affine(const uint32_t* packed, const uint8_t* e8m0, int64_t groups,
                               uint32_t* out_w, void* out_s, void* out_b, int sbdt,
                               hipStream_t st);
// Elementwise float conversion between the DT_* types.
hipError_t launch_convert(const void* src, int sdt, void* dst, int ddt, int64_t n,
                          hipStream_t st);

// ----------------------------------------------------------------- GEMM --
// Grouped dequant GEMM over a dispatch plan on the matrix cores, f16
// operands. The A rows are f16: activations of an f16 layer as they are, or
// of a bf16 layer scaled by 2^-8 (kA16Shift) into f16 range (launch_to_a16),
// which the kernel copies into LDS as they are. Gate/up pairs write their
// activation in that same f16 form (the down GEMM's A rows); a single
// projection writes out_dtype rows.
constexpr int kA16Shift = 8;
struct GemmArgs {
  GemvProj p0, p1;           // gate/up pair (p1 = up) or a single projection
  const void* x;             // activation rows [x_rows, K]
  int x_rows;
  const uint32_t* perm;      // nullable: row(p) = perm[p] / topk, else p
  int topk;
  const uint32_t* offsets;   // [E+1] CSR over sorted positions
  const uint32_t* items;     // work items (launch_gemm_items)
  void* out;                 // [M, N]
  int N, K, gsh;
  int sb_bf16;               // scales / biases stored as bf16 (else f16)
  int out_a16;               // a single projection writes f16 A rows (the first
                             // stage of squared-ReLU experts), else its dtype
  int act;
  float alpha, limit;
};
// Block shapes (activation rows x weight rows per block, 8 waves): an
// expert's rows go in 256-row tiles, and its last tile is the smallest shape
// that holds what is left.
constexpr int kGemmShapes = 3;
constexpr int kGemmShapeRows[kGemmShapes] = {256, 128, 64};
constexpr int kGemmShapeWRows[kGemmShapes] = {256, 256, 256};
__host__ __device__ inline int gemm_shape_for(int rows) {
  return rows > 128 ? 0 : (rows > 64 ? 1 : 2);
}
// Output columns per block: half the weight rows for a gate/up pair.
inline int gemm_cols(int shape, bool gateup) {
  return gateup ? kGemmShapeWRows[shape] / 2 : kGemmShapeWRows[shape];
}
// Upper bound on the work items of a plan of M rows over E experts (shapes
// 0 and 1 have the most column blocks).
inline long gemm_max_items(int M, int E, int N, bool gateup) {
  const long tiles = (M + 255) / 256 + (long)E;
  return tiles * ((N + gemm_cols(0, gateup) - 1) / gemm_cols(0, gateup));
}
inline size_t gemm_items_bytes(int M, int E, int N, bool gateup) {
  return (size_t)(4 + 4 * gemm_max_items(M, E, N, gateup)) * 4;
}
// items[0] = count (items[1..3] unused), then per item, 16-byte aligned,
// {expert | shape << 30, first sorted position, column block, end of the
// expert's positions}: experts ascending, an expert's row tiles in order, a
// tile's column blocks in order (neighbouring items share activation rows).
// Writes the list for (N0, gateup0) into items0 and, when items1 is
// non-NULL, the list for (N1, gateup1) over the same tiles into items1.
hipError_t launch_gemm_items(const uint32_t* offsets, int E, int N0, bool gateup0,
                             uint32_t* items0, int N1, bool gateup1, uint32_t* items1,
                             hipStream_t st);
// grid: 8 * ceil(gemm_max_items / 8) blocks (items are split evenly over the
// XCDs at run time; blocks without an item return at once).
hipError_t launch_gemm(int bits, int xdt, int sbdt, bool gateup, const GemmArgs& a, int grid,
                       hipStream_t st, KEvents ev = {});
// Elementwise bf16 -> f16 * 2^-kA16Shift (saturating), n a multiple of 8,
// 16-byte aligned buffers.
hipError_t launch_to_a16(const void* x, void* y, int64_t n, hipStream_t st);

}  // namespace moe
