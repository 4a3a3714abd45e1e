// api.cpp — the C ABI of libmoehip.so (include/moe_hip.h) and the host-side
// MoELayer that mirrors FFAI's Swift block (Sources/FFAI/Models/MoELayer.swift).
//
// Everything here is host code: argument validation (the reference's Swift
// preconditions and validators), workspace layout, launch geometry, and the
// stream-ordered sequence of kernels for one layer call. No call on the hot
// path allocates, synchronises or copies to the host.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cmath>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/moe_hip.h"
#include "moe_internal.hpp"

namespace moe {
hipError_t launch_gemv_b2(int, int, bool, int, const GemvArgs&, int, hipStream_t, KEvents);
hipError_t launch_gemv_b3(int, int, bool, int, const GemvArgs&, int, hipStream_t, KEvents);
hipError_t launch_gemv_b4(int, int, bool, int, const GemvArgs&, int, hipStream_t, KEvents);
hipError_t launch_gemv_b5(int, int, bool, int, const GemvArgs&, int, hipStream_t, KEvents);
hipError_t launch_gemv_b6(int, int, bool, int, const GemvArgs&, int, hipStream_t, KEvents);
hipError_t launch_gemv_b8(int, int, bool, int, const GemvArgs&, int, hipStream_t, KEvents);
hipError_t launch_dec1_b2(int, int, bool, int, int, const void*, int, size_t, hipStream_t, KEvents);
hipError_t launch_dec1_b3(int, int, bool, int, int, const void*, int, size_t, hipStream_t, KEvents);
hipError_t launch_dec1_b4(int, int, bool, int, int, const void*, int, size_t, hipStream_t, KEvents);
hipError_t launch_dec1_b5(int, int, bool, int, int, const void*, int, size_t, hipStream_t, KEvents);
hipError_t launch_dec1_b6(int, int, bool, int, int, const void*, int, size_t, hipStream_t, KEvents);
hipError_t launch_dec1_b8(int, int, bool, int, int, const void*, int, size_t, hipStream_t, KEvents);
hipError_t launch_multi_b2(int, int, bool, int, int, const GemvArgs&, int, size_t, hipStream_t, KEvents);
hipError_t launch_multi_b3(int, int, bool, int, int, const GemvArgs&, int, size_t, hipStream_t, KEvents);
hipError_t launch_multi_b4(int, int, bool, int, int, const GemvArgs&, int, size_t, hipStream_t, KEvents);
hipError_t launch_multi_b5(int, int, bool, int, int, const GemvArgs&, int, size_t, hipStream_t, KEvents);
hipError_t launch_multi_b6(int, int, bool, int, int, const GemvArgs&, int, size_t, hipStream_t, KEvents);
hipError_t launch_multi_b8(int, int, bool, int, int, const GemvArgs&, int, size_t, hipStream_t, KEvents);
hipError_t launch_mma_b2(int, int, bool, const GemvArgs&, int, hipStream_t, KEvents);
hipError_t launch_mma_b3(int, int, bool, const GemvArgs&, int, hipStream_t, KEvents);
hipError_t launch_mma_b4(int, int, bool, const GemvArgs&, int, hipStream_t, KEvents);
hipError_t launch_mma_b5(int, int, bool, const GemvArgs&, int, hipStream_t, KEvents);
hipError_t launch_mma_b6(int, int, bool, const GemvArgs&, int, hipStream_t, KEvents);

static hipError_t launch_mma(int bits, int xdt, int sbdt, bool gateup, const GemvArgs& a,
                             int grid, hipStream_t st, KEvents ev) {
  switch (bits) {
    case 2: return launch_mma_b2(xdt, sbdt, gateup, a, grid, st, ev);
    case 3: return launch_mma_b3(xdt, sbdt, gateup, a, grid, st, ev);
    case 4: return launch_mma_b4(xdt, sbdt, gateup, a, grid, st, ev);
    case 5: return launch_mma_b5(xdt, sbdt, gateup, a, grid, st, ev);
    case 6: return launch_mma_b6(xdt, sbdt, gateup, a, grid, st, ev);
    default: return hipErrorInvalidValue;
  }
}

static hipError_t launch_multi(int bits, int xdt, int sbdt, bool gateup, int ur, int tm,
                               const GemvArgs& a, int grid, size_t smem, hipStream_t st,
                               KEvents ev) {
  switch (bits) {
    case 2: return launch_multi_b2(xdt, sbdt, gateup, ur, tm, a, grid, smem, st, ev);
    case 3: return launch_multi_b3(xdt, sbdt, gateup, ur, tm, a, grid, smem, st, ev);
    case 4: return launch_multi_b4(xdt, sbdt, gateup, ur, tm, a, grid, smem, st, ev);
    case 5: return launch_multi_b5(xdt, sbdt, gateup, ur, tm, a, grid, smem, st, ev);
    case 6: return launch_multi_b6(xdt, sbdt, gateup, ur, tm, a, grid, smem, st, ev);
    case 8: return launch_multi_b8(xdt, sbdt, gateup, ur, tm, a, grid, smem, st, ev);
  }
  return hipErrorInvalidValue;
}


hipError_t launch_router_q_b2(const void*, int, int, int, const GemvProj&, int, int, const void*, int, void*, hipStream_t);
hipError_t launch_router_q_b3(const void*, int, int, int, const GemvProj&, int, int, const void*, int, void*, hipStream_t);
hipError_t launch_router_q_b4(const void*, int, int, int, const GemvProj&, int, int, const void*, int, void*, hipStream_t);
hipError_t launch_router_q_b5(const void*, int, int, int, const GemvProj&, int, int, const void*, int, void*, hipStream_t);
hipError_t launch_router_q_b6(const void*, int, int, int, const GemvProj&, int, int, const void*, int, void*, hipStream_t);
hipError_t launch_router_q_b8(const void*, int, int, int, const GemvProj&, int, int, const void*, int, void*, hipStream_t);

hipError_t launch_router_q(int bits, const void* x, int xdt, int T, int H, const GemvProj& W,
                           int sbdt, int gsh, const void* bias, int E, void* logits,
                           hipStream_t st) {
  switch (bits) {
    case 2: return launch_router_q_b2(x, xdt, T, H, W, sbdt, gsh, bias, E, logits, st);
    case 3: return launch_router_q_b3(x, xdt, T, H, W, sbdt, gsh, bias, E, logits, st);
    case 4: return launch_router_q_b4(x, xdt, T, H, W, sbdt, gsh, bias, E, logits, st);
    case 5: return launch_router_q_b5(x, xdt, T, H, W, sbdt, gsh, bias, E, logits, st);
    case 6: return launch_router_q_b6(x, xdt, T, H, W, sbdt, gsh, bias, E, logits, st);
    case 8: return launch_router_q_b8(x, xdt, T, H, W, sbdt, gsh, bias, E, logits, st);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemm_b2(int, bool, const GemmArgs&, int, hipStream_t, KEvents);
hipError_t launch_gemm_b3(int, bool, const GemmArgs&, int, hipStream_t, KEvents);
hipError_t launch_gemm_b4(int, bool, const GemmArgs&, int, hipStream_t, KEvents);
hipError_t launch_gemm_b5(int, bool, const GemmArgs&, int, hipStream_t, KEvents);
hipError_t launch_gemm_b6(int, bool, const GemmArgs&, int, hipStream_t, KEvents);
hipError_t launch_gemm_b8(int, bool, const GemmArgs&, int, hipStream_t, KEvents);

hipError_t launch_gemm(int bits, int xdt, int sbdt, bool gateup, const GemmArgs& a0, int grid,
                       hipStream_t st, KEvents ev) {
  if (sbdt != DT_BF16 && sbdt != DT_F16) return hipErrorInvalidValue;
  GemmArgs a = a0;
  a.sb_bf16 = sbdt == DT_BF16;
  switch (bits) {
    case 2: return launch_gemm_b2(xdt, gateup, a, grid, st, ev);
    case 3: return launch_gemm_b3(xdt, gateup, a, grid, st, ev);
    case 4: return launch_gemm_b4(xdt, gateup, a, grid, st, ev);
    case 5: return launch_gemm_b5(xdt, gateup, a, grid, st, ev);
    case 6: return launch_gemm_b6(xdt, gateup, a, grid, st, ev);
    case 8: return launch_gemm_b8(xdt, gateup, a, grid, st, ev);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gemv(int bits, int xdt, int sbdt, bool gateup, int tokmax, const GemvArgs& a,
                       int grid, hipStream_t st, KEvents ev) {
  switch (bits) {
    case 2: return launch_gemv_b2(xdt, sbdt, gateup, tokmax, a, grid, st, ev);
    case 3: return launch_gemv_b3(xdt, sbdt, gateup, tokmax, a, grid, st, ev);
    case 4: return launch_gemv_b4(xdt, sbdt, gateup, tokmax, a, grid, st, ev);
    case 5: return launch_gemv_b5(xdt, sbdt, gateup, tokmax, a, grid, st, ev);
    case 6: return launch_gemv_b6(xdt, sbdt, gateup, tokmax, a, grid, st, ev);
    case 8: return launch_gemv_b8(xdt, sbdt, gateup, tokmax, a, grid, st, ev);
  }
  return hipErrorInvalidValue;
}

static hipError_t launch_dec1(int bits, int xdt, int sbdt, bool down, int rm, int ur,
                              const void* args, int grid, size_t smem, hipStream_t st,
                              KEvents ev) {
  switch (bits) {
    case 2: return launch_dec1_b2(xdt, sbdt, down, rm, ur, args, grid, smem, st, ev);
    case 3: return launch_dec1_b3(xdt, sbdt, down, rm, ur, args, grid, smem, st, ev);
    case 4: return launch_dec1_b4(xdt, sbdt, down, rm, ur, args, grid, smem, st, ev);
    case 5: return launch_dec1_b5(xdt, sbdt, down, rm, ur, args, grid, smem, st, ev);
    case 6: return launch_dec1_b6(xdt, sbdt, down, rm, ur, args, grid, smem, st, ev);
    case 8: return launch_dec1_b8(xdt, sbdt, down, rm, ur, args, grid, smem, st, ev);
  }
  return hipErrorInvalidValue;
}

hipError_t launch_gateup1(int bits, int xdt, int sbdt, const Decode1Args& a, int rm, int grid,
                          hipStream_t st, KEvents ev) {
  const int L = 1 << a.lg, ur = (a.K / 32 + L - 1) / L;
  return launch_dec1(bits, xdt, sbdt, false, rm, ur, &a, grid, 0, st, ev);
}

hipError_t launch_down1(int bits, int xdt, int sbdt, const Down1Args& a, int rm, int grid,
                        hipStream_t st, KEvents ev) {
  const int L = 1 << a.lg, ur = (a.K / 32 + L - 1) / L;
  return launch_dec1(bits, xdt, sbdt, true, rm, ur, &a, grid, 0, st, ev);
}

size_t gemv_smem_bytes(int xdt, int K, int tok_chunk) {
  const size_t xs = (xdt == DT_F32) ? 4 : 2;
  return (size_t)tok_chunk * ((size_t)K * xs + (size_t)(K / 32) * 4);
}

}  // namespace moe

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
namespace moe {

thread_local std::string g_err;

void set_error_text(const char* msg) { g_err = msg; }
void clear_error_text() { g_err.clear(); }

}  // namespace moe

using namespace moe;

namespace {

moe_status fail(moe_status s, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  set_error_text(buf);
  return s;
}

moe_status ok() {
  clear_error_text();
  return MOE_OK;
}

moe_status hip_check(hipError_t e, const char* what) {
  if (e == hipSuccess) return MOE_OK;
  return fail(MOE_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define MOE_TRY(expr)                    \
  do {                                   \
    moe_status _s = (expr);              \
    if (_s != MOE_OK) return _s;         \
  } while (0)

#define MOE_HIP(expr, what) MOE_TRY(hip_check((expr), (what)))

bool dt_ok(int dt) { return dt == MOE_F32 || dt == MOE_F16 || dt == MOE_BF16; }
size_t dt_size(int dt) { return dt == MOE_F32 ? 4u : 2u; }
bool bits_ok(int b) { return b == 2 || b == 3 || b == 4 || b == 5 || b == 6 || b == 8; }

// activation dtype x scale dtype pairs built into the kernels
bool pair_ok(int xdt, int sbdt) {
  if (xdt == MOE_F32) return sbdt == MOE_F32;
  return sbdt == MOE_F16 || sbdt == MOE_BF16;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

bool gating_ok(int g) {
  return g == MOE_SOFTMAX_THEN_TOPK || g == MOE_TOPK_THEN_SOFTMAX || g == MOE_SIGMOID_TOPK;
}
bool act_ok(int a) {
  return a == MOE_ACT_SWIGLU || a == MOE_ACT_GPTOSS || a == MOE_ACT_GEGLU || a == MOE_ACT_RELU2;
}
bool scales_ok(float logit_scale, float routed_scale) {
  return std::isfinite(logit_scale) && std::isfinite(routed_scale);
}

// Routing options of the device router; a zero scale reads as 1.0.
RouteOpts route_opts(int gating, int norm, const float* ebias, float logit_scale,
                     float routed_scale, const float* escale) {
  RouteOpts r{};
  r.gating = gating;
  r.norm = norm;
  r.ebias = ebias;
  r.logit_scale = logit_scale == 0.f ? 1.f : logit_scale;
  r.routed_scale = routed_scale == 0.f ? 1.f : routed_scale;
  r.escale = escale;
  return r;
}
RouteOpts route_opts(const moe_layer_desc* d) {
  return route_opts(d->gating, d->norm_topk_prob, d->expert_bias, d->logit_scale, d->routed_scale,
                    d->expert_scale);
}

moe_status validate_qproj_named(const moe_qproj* p, const char* name) {
  if (!p) return fail(MOE_ERR_INVALID, "%s: descriptor is NULL", name);
  if (!p->weight || !p->scales || !p->biases)
    return fail(MOE_ERR_INVALID, "%s: weight/scales/biases must be non-NULL", name);
  if (!bits_ok(p->bits))
    return fail(MOE_ERR_INVALID, "%s: bits=%d unsupported — must be 2 / 3 / 4 / 5 / 6 / 8", name,
                p->bits);
  if (p->group_size <= 0) return fail(MOE_ERR_INVALID, "%s: group_size must be positive", name);
  if (p->n <= 0 || p->k <= 0 || p->n_experts <= 0)
    return fail(MOE_ERR_INVALID, "%s: n=%d k=%d n_experts=%d must be positive", name, p->n, p->k,
                p->n_experts);
  if (p->k % p->group_size)
    return fail(MOE_ERR_INVALID, "%s: k=%d must be a multiple of group_size=%d", name, p->k,
                p->group_size);
  if (((long)p->k * p->bits) % 32)
    return fail(MOE_ERR_INVALID, "%s: k*bits must be a multiple of 32 (u32 bit-stream alignment)",
                name);
  if (!dt_ok(p->sb_dtype)) return fail(MOE_ERR_INVALID, "%s: bad scale dtype %d", name, p->sb_dtype);
  // reference-valid shapes this build does not implement
  if (p->group_size != 32 && p->group_size != 64 && p->group_size != 128)
    return fail(MOE_ERR_UNSUPPORTED, "%s: group_size=%d not built (32, 64, 128 are)", name,
                p->group_size);
  if (p->k % 32) return fail(MOE_ERR_UNSUPPORTED, "%s: k=%d must be a multiple of 32", name, p->k);
  if ((uintptr_t)p->weight % 16)
    return fail(MOE_ERR_INVALID, "%s: weight pointer must be 16-byte aligned", name);
  if ((uintptr_t)p->scales % dt_size(p->sb_dtype) || (uintptr_t)p->biases % dt_size(p->sb_dtype))
    return fail(MOE_ERR_INVALID, "%s: scales/biases pointers misaligned", name);
  return MOE_OK;
}

}  // namespace

// ---------------------------------------------------------------------------
// diagnostics + validation
// ---------------------------------------------------------------------------
extern "C" const char* moe_last_error_string(void) { return g_err.c_str(); }
extern "C" const char* moe_version(void) { return "moehip 0.1 gfx950"; }

extern "C" moe_status moe_validate_qproj(const moe_qproj* p) {
  MOE_TRY(validate_qproj_named(p, "qproj"));
  return ok();
}

extern "C" moe_status moe_derive_bits(int64_t packed_cols, int64_t scale_cols, int32_t group_size,
                                      int32_t* bits_out) {
  const int64_t in_features = scale_cols * (int64_t)group_size;
  if (in_features <= 0)
    return fail(MOE_ERR_INVALID, "deriveAffineQuantBits: non-positive in-features");
  if ((32 * packed_cols) % in_features)
    return fail(MOE_ERR_INVALID,
                "deriveAffineQuantBits: %lld packed columns are inconsistent with %lld in-features",
                (long long)packed_cols, (long long)in_features);
  if (bits_out) *bits_out = (int32_t)((32 * packed_cols) / in_features);
  return ok();
}

namespace {

// A quantised router or shared gate: a one-expert stack [1, n, hidden].
moe_status validate_router_q(const moe_qproj* q, int n, int hidden, int xdt, const char* name) {
  MOE_TRY(validate_qproj_named(q, name));
  if (q->n_experts != 1 || q->n != n || q->k != hidden)
    return fail(MOE_ERR_INVALID, "%s: quantised weight must be [1, %d, %d] (got [%d, %d, %d])", name,
                n, hidden, q->n_experts, q->n, q->k);
  if (q->out_bias) return fail(MOE_ERR_INVALID, "%s: the router bias goes in router_bias", name);
  if (xdt != MOE_F16 && xdt != MOE_BF16)
    return fail(MOE_ERR_UNSUPPORTED, "%s: quantised router needs f16 or bf16 activations", name);
  if (!pair_ok(xdt, q->sb_dtype))
    return fail(MOE_ERR_UNSUPPORTED, "%s: scale dtype %d with activation dtype %d is not built",
                name, q->sb_dtype, xdt);
  if (hidden > 8192) return fail(MOE_ERR_UNSUPPORTED, "%s: hidden above 8192", name);
  return MOE_OK;
}

constexpr int kMaxExperts = 512;
constexpr int kMaxHidden = 8192;  // router rows are read in one round trip of 16 loads per lane

moe_status validate_layer_impl(const moe_layer_desc* d) {
  if (!d) return fail(MOE_ERR_INVALID, "MoELayer: descriptor is NULL");
  if (d->n_experts <= 0) return fail(MOE_ERR_INVALID, "MoERouter: nExperts must be positive");
  if (d->top_k <= 0 || d->top_k > d->n_experts)
    return fail(MOE_ERR_INVALID, "MoERouter: topK (%d) must be in 1...nExperts (%d)", d->top_k,
                d->n_experts);
  if (d->hidden <= 0 || d->intermediate <= 0)
    return fail(MOE_ERR_INVALID, "MoELayer: hidden and intermediate must be positive");
  if (d->hidden > kMaxHidden)
    return fail(MOE_ERR_UNSUPPORTED, "MoELayer: hidden (%d) above %d", d->hidden, kMaxHidden);
  if (!dt_ok(d->act_dtype) || !dt_ok(d->router_dtype))
    return fail(MOE_ERR_INVALID, "MoELayer: bad dtype");
  const bool rq = d->router_q.weight != nullptr;
  if (!d->router_weight && !rq) return fail(MOE_ERR_INVALID, "MoELayer: router weight is NULL");
  if (d->router_weight && rq)
    return fail(MOE_ERR_INVALID,
                "MoELayer: give the router as a dense weight or as a quantised triplet, not both");
  if (rq) MOE_TRY(validate_router_q(&d->router_q, d->n_experts, d->hidden, d->act_dtype, "gate"));
  if (!gating_ok(d->gating)) return fail(MOE_ERR_INVALID, "MoERouter: bad gating mode %d", d->gating);
  if (!act_ok(d->activation))
    return fail(MOE_ERR_INVALID, "MoELayer: bad activation %d", d->activation);
  if (!scales_ok(d->logit_scale, d->routed_scale))
    return fail(MOE_ERR_INVALID, "MoERouter: logit/routed scales must be finite");
  // squared-ReLU experts have no gate projection (NemotronHText.swift:756-761)
  const bool gated = d->activation != MOE_ACT_RELU2;
  if (!gated && (d->gate.weight || (d->has_shared && d->shared_gate.weight)))
    return fail(MOE_ERR_INVALID, "MoELayer: squared-ReLU experts take no gate projection");
  if (gated) MOE_TRY(validate_qproj_named(&d->gate, "gate_proj"));
  MOE_TRY(validate_qproj_named(&d->up, "up_proj"));
  MOE_TRY(validate_qproj_named(&d->down, "down_proj"));
  const moe_qproj* u = &d->up;
  const moe_qproj* g = gated ? &d->gate : u;
  const moe_qproj* dn = &d->down;
  if (g->n_experts != d->n_experts || u->n_experts != d->n_experts || dn->n_experts != d->n_experts)
    return fail(MOE_ERR_INVALID, "MoELayer: gate/up/down expert counts must equal nExperts (%d)",
                d->n_experts);
  if (g->n != d->intermediate || u->n != d->intermediate || g->k != d->hidden || u->k != d->hidden)
    return fail(MOE_ERR_INVALID, "MoELayer: gate/up must be [intermediate=%d, hidden=%d]",
                d->intermediate, d->hidden);
  if (dn->n != d->hidden || dn->k != d->intermediate)
    return fail(MOE_ERR_INVALID, "MoELayer: down must be [hidden=%d, intermediate=%d]", d->hidden,
                d->intermediate);
  if (g->bits != u->bits || g->group_size != u->group_size || g->sb_dtype != u->sb_dtype)
    return fail(MOE_ERR_UNSUPPORTED, "MoELayer: gate and up must share bits/group size/scale dtype");
  if (!pair_ok(d->act_dtype, g->sb_dtype) || !pair_ok(d->act_dtype, dn->sb_dtype))
    return fail(MOE_ERR_UNSUPPORTED,
                "MoELayer: activation dtype %d with scale dtype %d/%d is not built", d->act_dtype,
                g->sb_dtype, dn->sb_dtype);
  if (d->n_experts > kMaxExperts)
    return fail(MOE_ERR_UNSUPPORTED, "MoELayer: nExperts=%d above %d", d->n_experts, kMaxExperts);
  if (d->top_k > 64) return fail(MOE_ERR_UNSUPPORTED, "MoELayer: topK=%d above 64", d->top_k);
  if (d->has_shared) {
    if (gated) MOE_TRY(validate_qproj_named(&d->shared_gate, "shared_expert.gate_proj"));
    MOE_TRY(validate_qproj_named(&d->shared_up, "shared_expert.up_proj"));
    MOE_TRY(validate_qproj_named(&d->shared_down, "shared_expert.down_proj"));
    const moe_qproj* su = &d->shared_up;
    const moe_qproj* sg = gated ? &d->shared_gate : su;
    const moe_qproj* sd = &d->shared_down;
    if (sg->n_experts != 1 || su->n_experts != 1 || sd->n_experts != 1)
      return fail(MOE_ERR_INVALID, "MoELayer: shared expert projections hold exactly one expert");
    if (sg->k != d->hidden || su->k != d->hidden || su->n != sg->n || sd->k != sg->n ||
        sd->n != d->hidden)
      return fail(MOE_ERR_INVALID, "MoELayer: shared expert shapes do not chain hidden->I->hidden");
    if (sg->bits != su->bits || sg->group_size != su->group_size || sg->sb_dtype != su->sb_dtype)
      return fail(MOE_ERR_UNSUPPORTED, "MoELayer: shared gate/up must share bits/group/dtype");
    if (!pair_ok(d->act_dtype, sg->sb_dtype) || !pair_ok(d->act_dtype, sd->sb_dtype))
      return fail(MOE_ERR_UNSUPPORTED, "MoELayer: shared expert scale dtype not built");
    if (d->shared_gate_q.weight) {
      if (d->shared_gate_weight)
        return fail(MOE_ERR_INVALID,
                    "MoELayer: give shared_expert_gate as a dense weight or a quantised triplet, "
                    "not both");
      MOE_TRY(validate_router_q(&d->shared_gate_q, 1, d->hidden, d->act_dtype,
                                "shared_expert_gate"));
    }
  } else if (d->shared_gate_q.weight || d->shared_gate_weight) {
    return fail(MOE_ERR_INVALID, "MoELayer: shared_expert_gate given without a shared expert");
  }
  return MOE_OK;
}

// ---------------------------------------------------------------------------
// launch geometry
// ---------------------------------------------------------------------------

// log2 of the lanes per output row: the best lane utilisation of the K/32
// units with at most umax units per lane; ties go to fewer lanes (more rows
// in flight per wave, fewer shuffle steps).
int pick_lg(int CU, int umax, int min_lg = 0) {
  int best = 6;
  double best_eff = -1.0;
  for (int lg = min_lg; lg <= 6; lg++) {
    const int L = 1 << lg;
    const int upl = (CU + L - 1) / L;
    if (upl > umax) continue;
    const double eff = (double)CU / (double)(L * upl);
    if (eff > best_eff + 1e-9) {
      best_eff = eff;
      best = lg;
    }
  }
  return best;
}

constexpr int kTargetBlocks = 1024;

struct GemvGeom {
  int lg, row_blocks, rows_per_block, grid, tokmax, tok_chunk;
};

GemvGeom gemv_geom(int N, int K, int gsh, int slots, bool single, int M, int xdt) {
  GemvGeom g{};
  const int CU = K / 32;
  g.tokmax = single ? 1 : 8;
  g.lg = pick_lg(CU, single ? 4 : 8, gsh);
  const int SG = 64 >> g.lg;
  g.tok_chunk = 1;
  if (!single) {
    const size_t per_tok = gemv_smem_bytes(xdt, K, 1);
    int cap = (int)std::min<size_t>(8, 65536 / per_tok);
    g.tok_chunk = std::max(1, std::min(cap, M));
  }
  const int rows_per_iter = 4 * SG;
  const int max_rb = std::max(1, (N + rows_per_iter - 1) / rows_per_iter);
  int rb = std::max(1, (kTargetBlocks + slots - 1) / slots);
  rb = std::min(rb, max_rb);
  g.rows_per_block = (N + rb - 1) / rb;
  g.row_blocks = (N + g.rows_per_block - 1) / g.rows_per_block;
  g.grid = slots * g.row_blocks;
  return g;
}

// log2(group size / 32); group sizes are validated to 32, 64 or 128.
int group_shift(int gs) { return gs == 128 ? 2 : (gs == 64 ? 1 : 0); }

// ---------------------------------------------------------------------------
// workspace
// ---------------------------------------------------------------------------

struct Workspace {
  size_t logits, idx, w, counts, offsets, used, perm, inv, act, Y, plan_scratch;
  size_t items_gu, items_dn;  // grouped-GEMM work items of the routed experts
  size_t x16;                 // the layer input as the GEMMs' f16 operand
  size_t s_off, s_used, s_act, s_out, s_logit, s_items_gu, s_items_dn;
  size_t xn, res;  // decoder step before the block: normalised rows, residual
  size_t total;
};

Workspace layout(const moe_layer_desc* d, int T) {
  Workspace w{};
  const size_t A = 256, ds = dt_size(d->act_dtype);
  const size_t E = (size_t)d->n_experts, k = (size_t)d->top_k, M = (size_t)T * k;
  const size_t H = (size_t)d->hidden, I = (size_t)d->intermediate;
  size_t o = 0;
  auto take = [&](size_t bytes) {
    size_t at = o;
    o = align_up(o + std::max<size_t>(bytes, 1), A);
    return at;
  };
  w.logits = take((size_t)T * E * ds);
  w.idx = take(M * 4);
  w.w = take(M * 4);
  w.counts = take(E * 4);
  w.offsets = take((E + 1) * 4);
  w.used = take((E + 1) * 4);
  w.perm = take(M * 4);
  w.inv = take(M * 4);
  w.act = take(M * I * ds);
  w.Y = take(M * H * ds);
  w.plan_scratch = take(dispatch_scratch_bytes(T, (int)k, (int)E));
  w.items_gu = take(gemm_items_bytes((int)M, (int)E, (int)I, true));
  w.items_dn = take(gemm_items_bytes((int)M, (int)E, (int)H, false));
  w.x16 = take((size_t)T * H * 2);
  if (d->has_shared) {
    const size_t SI = (size_t)d->shared_up.n;
    w.s_off = take(2 * 4);
    w.s_used = take(2 * 4);
    w.s_act = take((size_t)T * SI * ds);
    w.s_out = take((size_t)T * H * ds);
    w.s_logit = take((size_t)T * ds);
    w.s_items_gu = take(gemm_items_bytes(T, 1, (int)SI, true));
    w.s_items_dn = take(gemm_items_bytes(T, 1, (int)H, false));
  }
  w.xn = take((size_t)T * H * ds);
  w.res = take((size_t)T * H * ds);
  w.total = o;
  return w;
}

template <typename P> P* at(void* base, size_t off) {
  return reinterpret_cast<P*>(reinterpret_cast<char*>(base) + off);
}

GemvProj to_proj(const moe_qproj& q) { return GemvProj{q.weight, q.scales, q.biases, q.out_bias}; }

int pick_lg_dec1(int CU, int gsh);

// Row iterations per gemv_multi_kernel block (each shares the block's staged
// activation rows; the next iteration's weights load while one multiplies)
// and the block count below which fewer are used. Swept over (iterations,
// floor) = (1, 2, 4, 8) x (1024, 512), µs per layer step at 4 / 16 tokens:
// (4, 512) GPT-OSS 72.4 / 158.7, Qwen3 41.8 / 84.0, against (2, 1024) 77.1 /
// 169.3 and 42.9 / 84.7; one iteration or eight are slower.
constexpr int kMultiIters = 4;
constexpr int kMultiBlocks = 512;

// Rows per used expert from which the batched GEMV runs on the matrix cores
// (Qwen3 shape, 4 per expert: 192 -> 154 us per layer step; GPT-OSS, 8 per
// expert: 409 -> 208 us; at 1 per expert gemv_multi_kernel is faster).
// Codes of other widths cost gemv_multi_kernel more unpacking, so they move
// from 2 rows per expert (mixed 3/6-bit layer, 64 tokens: 317 -> 231 us).
// One expert alone (a shared expert) gets only ceil(N / 32) matrix-core
// blocks, so it moves only once a pass fills the 16 activation rows.
// 4-bit thresholds re-measured after the matrix-core GEMV's loop and
// occupancy changes: a gate/up pair from 2 rows per used expert (Qwen3 32
// tokens 124.3 -> 117.6 us, GPT-OSS 16 tokens gate/up 96.8 -> 85.1 us), a
// single projection from 3 (GPT-OSS 16 tokens, 2 per expert: down 45.5 on
// gemv_multi_kernel against 50.0; at 24 tokens 58.8 against 52.5).
// Thresholds in tenths of a row per used expert. With the matrix-core GEMV's
// straight-line chunks the 4-bit crossovers moved down again (µs per launch,
// gemv_multi_kernel against gemv_mma_kernel): a gate/up pair is as fast or
// faster on the matrix cores at every measured count (Qwen3 12 tokens, 1.2
// rows per used expert: 36.2 / 34.6; 16 tokens, 1.56 rows: 42.7 / 39.4; 24
// tokens, 1.94 rows: 56.3 / 46.1; GPT-OSS 8 tokens, 1.45 rows: 62.1 / 60.1;
// 12 tokens: 79.6 / 68.9), a single projection from 1.8 rows (Qwen3 16
// tokens: 23.1 / 24.5; 20 tokens, 1.72 rows: 26.3 / 26.9; 24 tokens: 30.6 /
// 28.8; GPT-OSS 8 tokens: 29.6 / 33.4; 16 tokens, 2.2 rows: 45.9 / 43.3).
// Layer steps, old thresholds / these: Qwen3 16 tokens 80.0 / 77.7, 24
// tokens 99.7 / 90.3, GPT-OSS 12 tokens 129.0 / 120.7. Other widths stay at
// 2 (mixed-bit 16 tokens: gate/up 37.3 / 41.6).
constexpr int kMmaMinRowsPair10 = 10;
constexpr int kMmaMinRowsSingle10 = 18;
constexpr int kMmaMinRowsOther10 = 20;
constexpr int kMmaMinRowsSingleExpert10 = 160;

// gemv_mma_kernel applies: 2- to 6-bit codes (exact with the magic offset in
// either 16-bit type), 16-bit activations at 16-byte aligned rows, and
// expert-local byte offsets below 2^31.
bool mma_ok(const moe_qproj& p0, const moe_qproj* p1, bool x_aligned, int xdt) {
  if (p0.bits < 2 || p0.bits > 6 || (p1 && p1->bits != p0.bits)) return false;
  if (xdt == MOE_F32 || p0.sb_dtype == MOE_F32 || !x_aligned) return false;
  return ((size_t)p0.n + 64) * ((size_t)p0.k * p0.bits / 8) < (1ull << 31);
}

// gemv_multi_kernel applies: 16-bit activations at 16-byte aligned rows, at
// most 4 units per lane, a pass of tm rows in 64 KB of LDS, expert-local byte
// offsets below 2^31.
bool multi_ok(const moe_qproj& p0, bool x_aligned, int xdt, int tm) {
  if (xdt == MOE_F32 || p0.sb_dtype == MOE_F32 || !x_aligned) return false;
  const int CU = p0.k / 32;
  const int L = 1 << pick_lg_dec1(CU, group_shift(p0.group_size));
  if ((CU + L - 1) / L > 4) return false;
  if ((size_t)tm * CU * 68 > 65536) return false;
  return ((size_t)p0.n + 256) * ((size_t)p0.k * p0.bits / 8) < (1ull << 31);
}

// Rows per pass of gemv_multi_kernel: 4 when no expert, or the average used
// expert, has more (fewer accumulators: three blocks per CU instead of two;
// the few experts above the average take a second pass), else 8.
int multi_rows_per_pass(int max_rows, int rows, int slots) {
  return (max_rows <= 4 || (long)rows / std::max(1, slots) <= 4) ? 4 : 8;
}

// The GEMV kernel run_gemv takes for M rows over `slots` used experts.
enum GemvKind { kGemvGrouped = 0, kGemvMulti = 1, kGemvMma = 2 };
GemvKind gemv_kind(const moe_qproj& p0, const moe_qproj* p1, bool x_aligned, int xdt, int slots,
                   int M, bool single, int max_rows) {
  if (single) return kGemvGrouped;
  // the matrix cores once the used experts average enough rows: below that
  // the K-chunk pipeline's latency outweighs the VALU it saves
  const int min_rows10 = slots <= 1 ? kMmaMinRowsSingleExpert10
                        : p0.bits != 4 ? kMmaMinRowsOther10
                                       : (p1 ? kMmaMinRowsPair10 : kMmaMinRowsSingle10);
  // (its activation view holds at most M rows of K 16-bit values in 32-bit offsets)
  if (10L * M >= (long)min_rows10 * std::max(1, slots) && mma_ok(p0, p1, x_aligned, xdt) &&
      (size_t)M * (size_t)p0.k * 2 < (1ull << 31))
    return kGemvMma;
  const int tm = multi_rows_per_pass(std::min(max_rows, M), M, slots);
  if (multi_ok(p0, x_aligned, xdt, tm)) return kGemvMulti;
  return kGemvGrouped;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// gemv_multi_kernel for a few rows per expert (16-bit activations):
// kMultiRows weight rows per lane, lanes per row as for the one-token
// kernels, up to 4 or 8 activation rows per pass (rows in all, max_rows at
// most for one expert), activation units staged in at most 64 KB of LDS.
// The caller has checked multi_ok.
void run_multi(const moe_qproj& p0, const moe_qproj* p1, const void* x, int xdt,
               const uint32_t* perm, int topk, const uint32_t* offsets, const uint32_t* used,
               int slots, int max_rows, void* out, int act, float alpha, float limit,
               hipStream_t st, KEvents ev, moe_status* status, int rows) {
  const int gsh = group_shift(p0.group_size);
  const int CU = p0.k / 32;
  const int lg = pick_lg_dec1(CU, gsh);
  const int L = 1 << lg, ur = (CU + L - 1) / L;
  const int tm = multi_rows_per_pass(max_rows, rows, slots);
  const size_t smem = (size_t)tm * CU * 68;
  // R1 rows per iteration; up to kMultiIters iterations per block, fewer
  // while that leaves under kMultiBlocks blocks for the used experts
  const int SG = 64 >> lg, R1 = 4 * SG * kMultiRows(p1 != nullptr);
  const int groups_per_expert = (p0.n + R1 - 1) / R1;
  const int nit = std::max(1, std::min(kMultiIters, groups_per_expert * slots / kMultiBlocks));
  const int rows_per_block = nit * R1;
  const int row_blocks = (p0.n + rows_per_block - 1) / rows_per_block;
  GemvArgs a{};
  a.p0 = to_proj(p0);
  if (p1) a.p1 = to_proj(*p1);
  a.x = x;
  a.perm = perm;
  a.topk = topk;
  a.offsets = offsets;
  a.used = used;
  a.out = out;
  a.N = p0.n;
  a.K = p0.k;
  a.gsh = gsh;
  a.row_blocks = row_blocks;
  a.rows_per_block = rows_per_block;
  a.lg = lg;
  a.tok_chunk = tm;
  a.act = act;
  a.alpha = alpha;
  a.limit = limit;
  const hipError_t err = launch_multi(p0.bits, xdt, p0.sb_dtype, p1 != nullptr, ur, tm, a,
                                     slots * row_blocks, smem, st, ev);
  *status = hip_check(err, "grouped GEMV launch");
}

// gemv_mma_kernel (matrix cores) for 2- to 6-bit weights and 16-bit
// activations: 32 rows of a gate/up pair or 64 rows of one projection per
// block, 16 activation rows per pass. The caller has checked mma_ok.
void run_mma(const moe_qproj& p0, const moe_qproj* p1, const void* x, int xdt,
             const uint32_t* perm, int topk, const uint32_t* offsets, const uint32_t* used, int slots,
             int x_rows, void* out, int act, float alpha, float limit, hipStream_t st, KEvents ev,
             moe_status* status) {
  const int rows_per_block = p1 ? 32 : 64;
  const int row_blocks = (p0.n + rows_per_block - 1) / rows_per_block;
  GemvArgs a{};
  a.p0 = to_proj(p0);
  if (p1) a.p1 = to_proj(*p1);
  a.x = x;
  a.perm = perm;
  a.topk = topk;
  a.offsets = offsets;
  a.used = used;
  a.out = out;
  a.N = p0.n;
  a.K = p0.k;
  a.gsh = group_shift(p0.group_size);
  a.row_blocks = row_blocks;
  a.rows_per_block = rows_per_block;
  a.act = act;
  a.alpha = alpha;
  a.limit = limit;
  a.x_rows = x_rows;
  *status = hip_check(launch_mma(p0.bits, xdt, p0.sb_dtype, p1 != nullptr, a, slots * row_blocks, st, ev),
                      "grouped GEMV launch");
}

// out[p] = W[e(p)] . a[row(p)] over a plan; optionally a gate/up pair with
// the activation fused. max_rows bounds the rows of any one expert (T for
// routed tokens, which pick an expert at most once each).
moe_status run_gemv(const moe_qproj& p0, const moe_qproj* p1, const void* x, int xdt,
                    const uint32_t* perm, int topk, const uint32_t* offsets, const uint32_t* used,
                    int slots, int M, bool single, void* out, int act, float alpha, float limit,
                    hipStream_t st, KEvents ev = {}, int max_rows = 1 << 30) {
  const GemvKind kind = gemv_kind(p0, p1, aligned16(x), xdt, slots, M, single, max_rows);
  if (kind == kGemvMma) {
    moe_status status = MOE_OK;
    // the activation rows: one per token on the gather path (M = T topk)
    const int x_rows = perm ? (M + topk - 1) / topk : M;
    run_mma(p0, p1, x, xdt, perm, topk, offsets, used, slots, x_rows, out, act, alpha, limit, st,
            ev, &status);
    return status;
  }
  if (kind == kGemvMulti) {
    moe_status status = MOE_OK;
    run_multi(p0, p1, x, xdt, perm, topk, offsets, used, slots, std::min(max_rows, M), out, act,
              alpha, limit, st, ev, &status, M);
    return status;
  }
  const int gsh = group_shift(p0.group_size);
  GemvGeom g = gemv_geom(p0.n, p0.k, gsh, slots, single, M, xdt);
  GemvArgs a{};
  a.p0 = to_proj(p0);
  if (p1) a.p1 = to_proj(*p1);
  a.x = x;
  a.perm = perm;
  a.topk = topk;
  a.offsets = offsets;
  a.used = used;
  a.out = out;
  a.N = p0.n;
  a.K = p0.k;
  a.gsh = gsh;
  a.row_blocks = g.row_blocks;
  a.rows_per_block = g.rows_per_block;
  a.lg = g.lg;
  a.tok_chunk = g.tok_chunk;
  a.act = act;
  a.alpha = alpha;
  a.limit = limit;
  MOE_HIP(launch_gemv(p0.bits, xdt, p0.sb_dtype, p1 != nullptr, g.tokmax, a, g.grid, st, ev),
          "grouped GEMV launch");
  return MOE_OK;
}

// The MFMA grouped GEMM pays off once the used experts average enough rows
// to fill a good part of its 64-row tiles; below that the matrix-core GEMV,
// which reads every weight once per 16 rows, is faster. Swept at 16 / 24 /
// 32+ rows per expert (µs per layer step, GEMV against GEMM): 16 rows
// Qwen3 192.8 / 184.4, GPT-OSS 254.0 / 301.9, mixed-bit 317.3 / 320.0; 24
// rows Qwen3 242.0 / 191.8, GPT-OSS 323.9 / 305.3, mixed-bit 381.2 / 321.1.
// The same count moves a shared expert (one expert, T rows) onto the side
// stream and the GEMM (mixed-bit layer at 24 tokens: 147.6 -> 121.0 us).
// With the GEMM's epilogues at one rounding per output, layers of many
// small experts cross over at 16 rows (GEMV against GEMM: 16 rows Qwen3
// 192.9 / 180.5, mixed-bit 309.0 / 303.9; 20 rows 221.7 / 183.9 and 345.7 /
// 297.1; 14 rows 177.1 / 178.5 and 281.6 / 300.6; 12 rows 163.5 / 176.0 and
// 257.3 / 297.5), while GPT-OSS's 32 large experts keep the GEMV up to 23
// rows (16 rows 254.8 / 299.8, 20 rows 282.9 / 301.4): its GEMM blocks run
// 45 K chunks each in few rounds over the CUs.
constexpr int kGemmMinRows = 24;
constexpr int kGemmMinRowsMany = 16, kGemmManyExperts = 64;
// Rows from which a shared expert forks onto the side stream, whatever
// kernel it then runs (mixed-bit layer, µs per layer step in order / forked:
// 8 tokens 85.8 / 79.7, 16 tokens 111.7 / 99.0; 4 tokens 58.3 either way).
constexpr int kSideMinRows = 8;

// The matrix-core GEMM reads a weight row's scales and biases as 32-bit words
// (two 16-bit groups each): both arrays 4-byte aligned.
bool sb_words_ok(const moe_qproj& p) {
  return ((reinterpret_cast<uintptr_t>(p.scales) | reinterpret_cast<uintptr_t>(p.biases)) & 3) == 0;
}

// The matrix-core GEMM writes whole 16-byte groups of an output row: N is a
// multiple of 8 and the output 16-byte aligned (workspace buffers always are).
bool gemm_ok(const moe_qproj& p, int xdt, int M, const void* out = nullptr) {
  const int slots = std::min(p.n_experts, M);
  // activation rows are addressed with 32-bit byte offsets
  const bool fits = (size_t)M * (size_t)p.k * 2 < (1ull << 32);
  return xdt != MOE_F32 && p.k % 64 == 0 && p.n % 8 == 0 && p.n_experts <= 1024 && fits && sb_words_ok(p) &&
         M >= (p.n_experts >= kGemmManyExperts ? kGemmMinRowsMany : kGemmMinRows) * slots &&
         (reinterpret_cast<uintptr_t>(out) & 15) == 0;
}

// out[p] = W[e(p)] . a[row(p)] (or the gate/up pair with the activation)
// over a plan, on the matrix cores. `items` must hold the work list written by
// launch_gemm_items for the same offsets and (N, gate/up). The A rows x are
// f16 A operands (kA16Shift); a gate/up pair writes its activation as A
// rows.
// The routed experts / the shared expert of a layer call of T rows take the
// grouped GEMM (gate/up and down together: the gate/up epilogue writes the
// down GEMM's f16 operand).
bool routed_gemm(const moe_layer_desc* d, int T) {
  const moe_qproj& p0 = d->activation == MOE_ACT_RELU2 ? d->up : d->gate;
  const int M = T * d->top_k;
  return gemm_ok(p0, d->act_dtype, M) && gemm_ok(d->down, d->act_dtype, M) &&
         (d->activation == MOE_ACT_RELU2 || sb_words_ok(d->up));
}
bool shared_gemm(const moe_layer_desc* d, int T) {
  if (!d->has_shared) return false;
  const moe_qproj& p0 = d->activation == MOE_ACT_RELU2 ? d->shared_up : d->shared_gate;
  return gemm_ok(p0, d->act_dtype, T) && gemm_ok(d->shared_down, d->act_dtype, T) &&
         (d->activation == MOE_ACT_RELU2 || sb_words_ok(d->shared_up));
}

// out_a16: a single projection writes A rows for a following GEMM (the
// first stage of squared-ReLU experts).
moe_status run_gemm(const moe_qproj& p0, const moe_qproj* p1, const void* x, int xdt, bool out_a16, const uint32_t* perm, int topk, const uint32_t* offsets,
                    const uint32_t* items, int M, void* out, int act, float alpha, float limit,
                    hipStream_t st, KEvents ev = {}) {
  GemmArgs a{};
  a.out_a16 = out_a16;
  a.p0 = to_proj(p0);
  if (p1) a.p1 = to_proj(*p1);
  a.x = x;
  a.x_rows = perm ? (M + topk - 1) / topk : M;
  a.perm = perm;
  a.topk = topk;
  a.offsets = offsets;
  a.items = items;
  a.out = out;
  a.N = p0.n;
  a.K = p0.k;
  a.gsh = group_shift(p0.group_size);
  a.act = act;
  a.alpha = alpha;
  a.limit = limit;
  const bool gu = p1 != nullptr;
  const long items_max = gemm_max_items(M, p0.n_experts, p0.n, gu);
  const int grid = (int)((items_max + 7) / 8 * 8);  // a multiple of the 8 XCDs
  MOE_HIP(launch_gemm(p0.bits, xdt, p0.sb_dtype, gu, a, grid, st, ev),
          "grouped GEMM launch");
  return MOE_OK;
}

}  // namespace

extern "C" moe_status moe_validate_layer(const moe_layer_desc* d) {
  MOE_TRY(validate_layer_impl(d));
  return ok();
}

// ---------------------------------------------------------------------------
// kernels
// ---------------------------------------------------------------------------

extern "C" moe_status moe_router_logits(const void* x, int32_t x_dtype, int32_t T, int32_t hidden,
                                        const void* weight, int32_t w_dtype, const void* bias,
                                        int32_t n_experts, void* logits, hipStream_t stream) {
  if (!x || !weight || !logits) return fail(MOE_ERR_INVALID, "router_logits: NULL pointer");
  if (T <= 0 || hidden <= 0 || n_experts <= 0)
    return fail(MOE_ERR_INVALID, "router_logits: T, hidden and n_experts must be positive");
  if (!dt_ok(x_dtype) || !dt_ok(w_dtype)) return fail(MOE_ERR_INVALID, "router_logits: bad dtype");
  if (hidden % 8) return fail(MOE_ERR_UNSUPPORTED, "router_logits: hidden must be a multiple of 8");
  if (hidden > kMaxHidden)
    return fail(MOE_ERR_UNSUPPORTED, "router_logits: hidden (%d) above %d", hidden, kMaxHidden);
  MOE_HIP(launch_router_logits(x, x_dtype, T, hidden, weight, w_dtype, bias, n_experts, logits,
                               stream),
          "router logits launch");
  return ok();
}

extern "C" moe_status moe_router_logits_q(const void* x, int32_t x_dtype, int32_t T,
                                          int32_t hidden, const moe_qproj* w, const void* bias,
                                          int32_t n_experts, void* logits, hipStream_t stream) {
  if (!x || !w || !logits) return fail(MOE_ERR_INVALID, "router_logits_q: NULL pointer");
  if (T <= 0 || hidden <= 0 || n_experts <= 0)
    return fail(MOE_ERR_INVALID, "router_logits_q: T, hidden and n_experts must be positive");
  MOE_TRY(validate_router_q(w, n_experts, hidden, x_dtype, "router_logits_q"));
  MOE_HIP(launch_router_q(w->bits, x, x_dtype, T, hidden, to_proj(*w), w->sb_dtype,
                          group_shift(w->group_size), bias, n_experts, logits, stream),
          "quantised router launch");
  return ok();
}

extern "C" moe_status moe_router_topk(const void* logits, int32_t dtype, int32_t T,
                                      int32_t n_experts, int32_t k, int32_t gating,
                                      int32_t norm_topk_prob, const float* expert_bias,
                                      uint32_t* topk_idx, float* topk_weight, hipStream_t stream) {
  return moe_router_topk_scaled(logits, dtype, T, n_experts, k, gating, norm_topk_prob,
                                expert_bias, 1.f, 1.f, nullptr, topk_idx, topk_weight, stream);
}

extern "C" moe_status moe_router_topk_scaled(const void* logits, int32_t dtype, int32_t T,
                                             int32_t n_experts, int32_t k, int32_t gating,
                                             int32_t norm_topk_prob, const float* expert_bias,
                                             float logit_scale, float routed_scale,
                                             const float* expert_scale, uint32_t* topk_idx,
                                             float* topk_weight, hipStream_t stream) {
  if (!logits || !topk_idx || !topk_weight) return fail(MOE_ERR_INVALID, "router_topk: NULL pointer");
  if (T <= 0) return fail(MOE_ERR_INVALID, "Ops.moeRouterTopKMany: t must be positive");
  if (n_experts <= 0) return fail(MOE_ERR_INVALID, "MoERouter: nExperts must be positive");
  if (k <= 0 || k > n_experts)
    return fail(MOE_ERR_INVALID, "MoERouter: topK (%d) must be in 1...nExperts (%d)", k, n_experts);
  if (!gating_ok(gating)) return fail(MOE_ERR_INVALID, "router_topk: bad gating mode");
  if (!scales_ok(logit_scale, routed_scale))
    return fail(MOE_ERR_INVALID, "router_topk: logit/routed scales must be finite");
  if (!dt_ok(dtype)) return fail(MOE_ERR_INVALID, "router_topk: bad dtype");
  if (n_experts > kMaxExperts)
    return fail(MOE_ERR_UNSUPPORTED, "router_topk: nExperts=%d above %d", n_experts, kMaxExperts);
  if (k > 64) return fail(MOE_ERR_UNSUPPORTED, "router_topk: k=%d above 64", k);
  const RouteOpts ro = route_opts(gating, norm_topk_prob, expert_bias, logit_scale, routed_scale,
                                  expert_scale);
  // no partials: the logits are only read
  MOE_HIP(launch_router_topk(const_cast<void*>(logits), dtype, T, n_experts, k, ro, topk_idx,
                             topk_weight, stream),
          "router top-k launch");
  return ok();
}

extern "C" size_t moe_dispatch_workspace_bytes(int32_t T, int32_t k, int32_t n_experts) {
  if (T <= 0 || k <= 0 || n_experts <= 0) return 0;
  return align_up((size_t)(n_experts + 1) * 4, 256) + dispatch_scratch_bytes(T, k, n_experts);
}

extern "C" moe_status moe_dispatch_plan(const uint32_t* topk_idx, int32_t T, int32_t k,
                                        int32_t n_experts, uint32_t* counts, uint32_t* offsets,
                                        uint32_t* perm, uint32_t* inv_perm, void* workspace,
                                        size_t workspace_bytes, hipStream_t stream) {
  if (!topk_idx || !counts || !offsets || !perm || !inv_perm)
    return fail(MOE_ERR_INVALID, "dispatch_plan: NULL pointer");
  if (T <= 0 || k <= 0 || n_experts <= 0)
    return fail(MOE_ERR_INVALID, "dispatch_plan: T, k and n_experts must be positive");
  if ((long)T * k > 0x7fffffffL) return fail(MOE_ERR_INVALID, "dispatch_plan: T*k too large");
  if (n_experts > 1024) return fail(MOE_ERR_UNSUPPORTED, "dispatch_plan: n_experts above 1024");
  const size_t need = moe_dispatch_workspace_bytes(T, k, n_experts);
  if (!workspace || workspace_bytes < need)
    return fail(MOE_ERR_WORKSPACE, "dispatch_plan: workspace of %zu bytes needed", need);
  uint32_t* used = reinterpret_cast<uint32_t*>(workspace);
  void* scratch = reinterpret_cast<char*>(workspace) + align_up((size_t)(n_experts + 1) * 4, 256);
  MOE_HIP(launch_dispatch_plan(topk_idx, T, k, n_experts, counts, offsets, perm, inv_perm, used,
                               scratch, workspace_bytes - align_up((size_t)(n_experts + 1) * 4, 256),
                               stream),
          "dispatch plan launch");
  return ok();
}

extern "C" moe_status moe_dequantize_affine(const uint32_t* weight, const void* scales,
                                            const void* biases, int32_t sb_dtype, int32_t bits,
                                            int32_t group_size, int64_t numel, void* out,
                                            int32_t out_dtype, hipStream_t stream) {
  if (!weight || !scales || !biases || !out) return fail(MOE_ERR_INVALID, "dequantize: NULL pointer");
  if (numel <= 0) return fail(MOE_ERR_INVALID, "numel must be positive (got %lld)", (long long)numel);
  if (group_size <= 0)
    return fail(MOE_ERR_INVALID, "groupSize must be positive (got %d)", group_size);
  if (numel % group_size)
    return fail(MOE_ERR_INVALID, "numel=%lld must be a multiple of groupSize=%d", (long long)numel,
                group_size);
  if (bits == 2 || bits == 4 || bits == 8) {
    if (group_size % (32 / bits))
      return fail(MOE_ERR_INVALID, "groupSize=%d must be a multiple of pack_factor=%d for bits=%d",
                  group_size, 32 / bits, bits);
  } else if (bits == 3 || bits == 5 || bits == 6) {
    if ((group_size * bits) % 32)
      return fail(MOE_ERR_INVALID,
                  "groupSize=%d x bits=%d must be a multiple of 32 (u32 bit-stream alignment)",
                  group_size, bits);
  } else {
    return fail(MOE_ERR_INVALID, "bits=%d unsupported — must be 2 / 3 / 4 / 5 / 6 / 8", bits);
  }
  if ((numel * bits) % 32)
    return fail(MOE_ERR_INVALID, "numel=%lld x bits=%d must be a multiple of 32", (long long)numel,
                bits);
  if (!dt_ok(sb_dtype) || !dt_ok(out_dtype)) return fail(MOE_ERR_INVALID, "dequantize: bad dtype");
  MOE_HIP(launch_dequantize(weight, scales, biases, sb_dtype, bits, group_size, numel, out,
                            out_dtype, stream),
          "dequantize launch");
  return ok();
}

extern "C" moe_status moe_mxfp4_to_affine(const uint32_t* packed, const uint8_t* e8m0,
                                          int64_t n_groups, uint32_t* out_weight,
                                          void* out_scales, void* out_biases, int32_t sb_dtype,
                                          hipStream_t stream) {
  if (!packed || !e8m0 || !out_weight || !out_scales || !out_biases)
    return fail(MOE_ERR_INVALID, "mxfp4_to_affine: NULL pointer");
  if (n_groups <= 0) return fail(MOE_ERR_INVALID, "mxfp4_to_affine: n_groups must be positive");
  if (!dt_ok(sb_dtype)) return fail(MOE_ERR_INVALID, "mxfp4_to_affine: bad scale dtype");
  if ((reinterpret_cast<uintptr_t>(packed) & 15) || (reinterpret_cast<uintptr_t>(out_weight) & 15))
    return fail(MOE_ERR_INVALID, "mxfp4_to_affine: packed words must be 16-byte aligned");
  MOE_HIP(launch_mxfp4_affine(packed, e8m0, n_groups, out_weight, out_scales, out_biases, sb_dtype,
                              stream),
          "MXFP4 transcode launch");
  return ok();
}

// [used list / CSR copy][GEMM work list][bf16 rows as f16 operands]
extern "C" size_t moe_expert_matmul_workspace_bytes(const moe_qproj* p, int32_t a_dtype, int32_t M) {
  if (!p || M <= 0 || validate_qproj_named(p, "expert_matmul") != MOE_OK || !dt_ok(a_dtype)) return 0;
  size_t bytes = align_up((size_t)(p->n_experts + 1) * 4, 256) +
                 align_up(gemm_items_bytes(M, p->n_experts, p->n, false), 256);
  if (a_dtype == MOE_BF16) bytes += align_up((size_t)M * p->k * 2, 256);
  return bytes;
}

extern "C" moe_status moe_expert_matmul(const moe_qproj* p, const void* a, int32_t a_dtype,
                                        const uint32_t* perm, int32_t top_k, int32_t M,
                                        const uint32_t* offsets, void* out, void* workspace,
                                        size_t workspace_bytes, hipStream_t stream) {
  MOE_TRY(validate_qproj_named(p, "expert_matmul"));
  if (!a || !offsets || !out) return fail(MOE_ERR_INVALID, "expert_matmul: NULL pointer");
  if (M <= 0) return fail(MOE_ERR_INVALID, "expert_matmul: M must be positive");
  if (perm && top_k <= 0) return fail(MOE_ERR_INVALID, "expert_matmul: top_k must be positive");
  if (!dt_ok(a_dtype) || !pair_ok(a_dtype, p->sb_dtype))
    return fail(MOE_ERR_UNSUPPORTED, "expert_matmul: activation/scale dtype pair not built");
  if (p->n_experts > 1024) return fail(MOE_ERR_UNSUPPORTED, "expert_matmul: n_experts above 1024");
  const size_t need = moe_expert_matmul_workspace_bytes(p, a_dtype, M);
  if (!workspace || workspace_bytes < need)
    return fail(MOE_ERR_WORKSPACE, "expert_matmul: workspace of %zu bytes needed", need);
  if (gemm_ok(*p, a_dtype, M, out)) {
    char* wsc = reinterpret_cast<char*>(workspace);
    const size_t items_at = align_up((size_t)(p->n_experts + 1) * 4, 256);
    uint32_t* items = reinterpret_cast<uint32_t*>(wsc + items_at);
    MOE_HIP(launch_gemm_items(offsets, p->n_experts, p->n, false, items, 0, false, nullptr, stream),
            "GEMM work list launch");
    const void* a16 = a;
    if (a_dtype == MOE_BF16) {  // the GEMM's f16 operand: bf16 rows scaled by 2^-kA16Shift
      void* x16 = wsc + items_at + align_up(gemm_items_bytes(M, p->n_experts, p->n, false), 256);
      const int64_t rows = perm ? (M + top_k - 1) / top_k : M;
      MOE_HIP(launch_to_a16(a, x16, rows * p->k, stream), "f16 operand launch");
      a16 = x16;
    }
    MOE_TRY(run_gemm(*p, nullptr, a16, a_dtype, false, perm, top_k, offsets, items, M, out, 0, 0.f,
                     0.f, stream));
    return ok();
  }
  uint32_t* used = reinterpret_cast<uint32_t*>(workspace);
  MOE_HIP(launch_used_from_offsets(offsets, p->n_experts, used, stream), "used list launch");
  const int slots = std::min(p->n_experts, M);
  MOE_TRY(run_gemv(*p, nullptr, a, a_dtype, perm, top_k, offsets, used, slots, M, false, out, 0,
                   0.f, 0.f, stream));
  return ok();
}

extern "C" moe_status moe_activation_apply(const void* gate, const void* up, void* out, int64_t n,
                                           int32_t dtype, int32_t activation, float alpha,
                                           float limit, hipStream_t stream) {
  if (!up || !out) return fail(MOE_ERR_INVALID, "activation: NULL pointer");
  if (n <= 0) return fail(MOE_ERR_INVALID, "activation: n must be positive");
  if (!dt_ok(dtype)) return fail(MOE_ERR_INVALID, "activation: bad dtype");
  if (!act_ok(activation)) return fail(MOE_ERR_INVALID, "activation: bad kind");
  if (!gate && activation != MOE_ACT_RELU2) return fail(MOE_ERR_INVALID, "activation: NULL gate");
  MOE_HIP(launch_activation(gate, up, out, n, dtype, activation, alpha, limit, stream),
          "activation launch");
  return ok();
}

extern "C" moe_status moe_unpermute(const void* Y, const uint32_t* inv_perm,
                                    const float* topk_weight, int32_t T, int32_t hidden, int32_t k,
                                    void* out, int32_t dtype, hipStream_t stream) {
  if (!Y || !inv_perm || !topk_weight || !out) return fail(MOE_ERR_INVALID, "unpermute: NULL pointer");
  if (T <= 0 || hidden <= 0 || k <= 0)
    return fail(MOE_ERR_INVALID, "unpermute: T, hidden and k must be positive");
  if (hidden % 8) return fail(MOE_ERR_UNSUPPORTED, "unpermute: hidden must be a multiple of 8");
  if (!dt_ok(dtype)) return fail(MOE_ERR_INVALID, "unpermute: bad dtype");
  MOE_HIP(launch_unpermute(Y, inv_perm, topk_weight, T, hidden, k, out, dtype, nullptr, nullptr, 0,
                           stream),
          "unpermute launch");
  return ok();
}

// ---------------------------------------------------------------------------
// whole layer
// ---------------------------------------------------------------------------

extern "C" size_t moe_layer_workspace_bytes(const moe_layer_desc* d, int32_t max_tokens) {
  if (!d || max_tokens <= 0 || validate_layer_impl(d) != MOE_OK) return 0;
  return layout(d, max_tokens).total;
}

namespace {

moe_status copy_trace(const moe_layer_desc* d, int T, void* ws, const Workspace& w,
                      const moe_layer_trace* tr, hipStream_t st) {
  if (!tr) return MOE_OK;
  const size_t M = (size_t)T * d->top_k, E = (size_t)d->n_experts;
  auto cp = [&](void* dst, size_t off, size_t bytes) -> moe_status {
    if (!dst) return MOE_OK;
    return hip_check(hipMemcpyAsync(dst, at<char>(ws, off), bytes, hipMemcpyDeviceToDevice, st),
                     "trace copy");
  };
  MOE_TRY(cp(tr->logits, w.logits, (size_t)T * E * dt_size(d->act_dtype)));
  MOE_TRY(cp(tr->topk_idx, w.idx, M * 4));
  MOE_TRY(cp(tr->topk_weight, w.w, M * 4));
  MOE_TRY(cp(tr->perm, w.perm, M * 4));
  MOE_TRY(cp(tr->offsets, w.offsets, (E + 1) * 4));
  return MOE_OK;
}

// Shared expert (Qwen3xText.swift:928-1104; MoELayer.swift:620-624;
// NemotronHText.swift:855-862): gate/up + the layer's activation (or the
// single up projection with squared ReLU), down, and the optional sigmoid
// gate logit, into the workspace. Returns the combine mode: 0 none, 1
// unconditional add, 2 sigmoid-gated.
// Work that may overlap the routed experts (the shared expert: it reads the
// layer input only and writes its own workspace regions) runs on a side
// stream: forked from the caller's stream, joined back before the combine
// that reads its output. Each device keeps a small pool of non-blocking,
// default-priority side streams (each with two events), created on first use
// outside any capture and kept for the process lifetime. A side stream that
// joins a stream capture stays part of that capture until the capture ends,
// so a call takes a pooled stream only if it is not being captured, or is
// being captured by the caller's own capture (same capture id): an eager call
// and a capture, or two captures, never share one. Each call holds its side
// stream's lock from fork to join, so calls from several host threads never
// interleave its events. Under stream capture the fork and join become graph
// edges. Without a usable side stream (none idle and the caller is being
// captured, or creation failed) the work stays on the caller's stream, in
// order.
class SideFork {
 public:
  SideFork(bool want, hipStream_t st) : st_(st), side_(st) {
    if (!want) return;
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
      (void)hipGetLastError();
      return;
    }
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    unsigned long long cid = 0;
    if (hipStreamGetCaptureInfo(st, &cs, &cid) != hipSuccess) {
      (void)hipGetLastError();
      return;
    }
    const bool capturing = cs != hipStreamCaptureStatusNone;
    Slot* t = nullptr;
    {
      std::lock_guard<std::mutex> g(pool_mu());
      std::vector<Slot*>& pool = pools()[dev];
      for (Slot* c : pool) {
        std::unique_lock<std::mutex> l(c->mu, std::try_to_lock);
        if (!l.owns_lock()) continue;  // another call holds it
        hipStreamCaptureStatus xs = hipStreamCaptureStatusNone;
        unsigned long long xid = 0;
        if (hipStreamGetCaptureInfo(c->s, &xs, &xid) != hipSuccess) {
          (void)hipGetLastError();
          continue;
        }
        const bool usable = xs == hipStreamCaptureStatusNone ||
                            (capturing && xs == hipStreamCaptureStatusActive && xid == cid);
        if (!usable) continue;
        lock_ = std::move(l);
        t = c;
        break;
      }
      // a new side stream, never inside a capture (that call stays in order)
      if (!t && !capturing && pool.size() < kMaxPool) {
        hipStream_t s = nullptr;
        hipEvent_t f = nullptr, j = nullptr;
        if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&f, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&j, hipEventDisableTiming) != hipSuccess) {
          (void)hipGetLastError();
          if (j) (void)hipEventDestroy(j);
          if (f) (void)hipEventDestroy(f);
          if (s) (void)hipStreamDestroy(s);
        } else {
          Slot* c = new (std::nothrow) Slot{s, f, j, {}};
          if (!c) {
            (void)hipEventDestroy(j);
            (void)hipEventDestroy(f);
            (void)hipStreamDestroy(s);
          } else {
            pool.push_back(c);
            lock_ = std::unique_lock<std::mutex>(c->mu);
            t = c;
          }
        }
      }
    }
    if (!t) return;
    slot_ = t;
    status_ = hip_check(hipEventRecord(t->fork, st), "side stream fork");
    if (status_ == MOE_OK) status_ = hip_check(hipStreamWaitEvent(t->s, t->fork, 0), "side stream fork");
    if (status_ == MOE_OK) side_ = t->s;
  }
  moe_status status() const { return status_; }
  hipStream_t stream() const { return side_; }
  // after the side work: the point the caller's stream waits for
  moe_status mark() {
    return slot_ && side_ != st_ ? hip_check(hipEventRecord(slot_->join, side_), "side stream join")
                                 : MOE_OK;
  }
  // the caller's stream waits for the side work from here on
  moe_status join() {
    if (!slot_ || side_ == st_) return MOE_OK;
    const moe_status r = hip_check(hipStreamWaitEvent(st_, slot_->join, 0), "side stream join");
    slot_ = nullptr;
    if (lock_.owns_lock()) lock_.unlock();
    return r;
  }

 private:
  static constexpr size_t kMaxPool = 8;  // side streams per device
  struct Slot {
    hipStream_t s;
    hipEvent_t fork, join;
    std::mutex mu;
  };
  static std::mutex& pool_mu() {
    static std::mutex m;
    return m;
  }
  // never destroyed: the side streams live until the process ends
  static std::map<int, std::vector<Slot*>>& pools() {
    static std::map<int, std::vector<Slot*>>* m = new std::map<int, std::vector<Slot*>>();
    return *m;
  }
  hipStream_t st_, side_;
  Slot* slot_ = nullptr;
  std::unique_lock<std::mutex> lock_;
  moe_status status_ = MOE_OK;
};

// The shared expert's sigmoid gate logits (Qwen3xText.swift:947-951) into
// the workspace, from a dense or a quantised gate row; none without a gate.
moe_status shared_gate_logits(const moe_layer_desc* d, const void* x, int T, void* ws,
                              const Workspace& w, hipStream_t st) {
  const int xdt = d->act_dtype;
  if (d->shared_gate_q.weight)
    MOE_HIP(launch_router_q(d->shared_gate_q.bits, x, xdt, T, d->hidden, to_proj(d->shared_gate_q),
                            d->shared_gate_q.sb_dtype, group_shift(d->shared_gate_q.group_size),
                            nullptr, 1, at<void>(ws, w.s_logit), st),
            "shared gate launch");
  else if (d->shared_gate_weight)
    MOE_HIP(launch_router_logits(x, xdt, T, d->hidden, d->shared_gate_weight, d->router_dtype,
                                 nullptr, 1, at<void>(ws, w.s_logit), st),
            "shared gate launch");
  return MOE_OK;
}

// x16: the layer input as the GEMMs' f16 operand (written before the fork
// when the grouped GEMM runs for the shared expert).
// gate_done: the router launch already wrote the shared gate's logits.
moe_status shared_expert(const moe_layer_desc* d, const void* x, const void* x16, int T, void* ws,
                         const Workspace& w, hipStream_t st, int* smode, bool gate_done) {
  *smode = 0;
  if (!d->has_shared) return MOE_OK;
  const int xdt = d->act_dtype;
  const bool single = (T == 1);
  *smode = (d->shared_gate_weight || d->shared_gate_q.weight) ? 2 : 1;
  MOE_HIP(launch_identity_plan(at<uint32_t>(ws, w.s_off), at<uint32_t>(ws, w.s_used), T, st),
          "identity plan launch");
  const bool gated = d->activation != MOE_ACT_RELU2;
  const moe_qproj& p0 = gated ? d->shared_gate : d->shared_up;
  const moe_qproj* p1 = gated ? &d->shared_up : nullptr;
  if (shared_gemm(d, T)) {
    // many tokens through one expert: the matrix-core path
    MOE_HIP(launch_gemm_items(at<uint32_t>(ws, w.s_off), 1, p0.n, p1 != nullptr,
                              at<uint32_t>(ws, w.s_items_gu), d->hidden, false,
                              at<uint32_t>(ws, w.s_items_dn), st),
            "shared GEMM work list launch");
    MOE_TRY(run_gemm(p0, p1, x16, xdt, true, nullptr, 1, at<uint32_t>(ws, w.s_off),
                     at<uint32_t>(ws, w.s_items_gu), T, at<void>(ws, w.s_act), d->activation,
                     d->act_alpha, d->act_limit, st));
    MOE_TRY(run_gemm(d->shared_down, nullptr, at<void>(ws, w.s_act), xdt, false, nullptr, 1,
                     at<uint32_t>(ws, w.s_off), at<uint32_t>(ws, w.s_items_dn), T,
                     at<void>(ws, w.s_out), 0, 0.f, 0.f, st));
  } else {
    MOE_TRY(run_gemv(p0, p1, x, xdt, nullptr, 1, at<uint32_t>(ws, w.s_off),
                     at<uint32_t>(ws, w.s_used), 1, T, single, at<void>(ws, w.s_act),
                     d->activation, d->act_alpha, d->act_limit, st));
    MOE_TRY(run_gemv(d->shared_down, nullptr, at<void>(ws, w.s_act), xdt, nullptr, 1,
                     at<uint32_t>(ws, w.s_off), at<uint32_t>(ws, w.s_used), 1, T, single,
                     at<void>(ws, w.s_out), 0, 0.f, 0.f, st));
  }
  return gate_done ? MOE_OK : shared_gate_logits(d, x, T, ws, w, st);
}

// Decode (T = 1) launch geometry. Lanes per row: the best unit utilisation
// with at most 4 units per lane (and whole scale groups per lane stride).
// Rows per lane rm: every load of a lane's rows is in flight before its
// first dot product, so rm trades waves in flight against the work each
// wave amortises its routing and activation loads over; about 3000 waves
// (3 per SIMD) measured best on the GPT-OSS and Qwen3 decode shapes.
struct Dec1Geom {
  int lg, rm, rows_per_block, grid;
};

constexpr int kDec1TargetWaves = 3000;

// Lanes per row for the one-token kernels: the best unit utilisation with at
// most 4 units per lane; among equals, 2-3 units per lane (enough loads in
// flight per lane without long shuffle-free dot chains), then fewer lanes.
int pick_lg_dec1(int CU, int gsh) {
  int best = -1;
  double best_eff = -1.0, best_pen = 0.0;
  for (int lg = gsh; lg <= 6; lg++) {
    const int L = 1 << lg, upl = (CU + L - 1) / L;
    if (upl > 4) continue;
    const double eff = (double)CU / (double)(L * upl);
    const double pen = (upl == 2 || upl == 3) ? 0.0 : 1.0;
    if (eff > best_eff + 1e-9 || (eff > best_eff - 1e-9 && pen < best_pen)) {
      best = lg;
      best_eff = eff;
      best_pen = pen;
    }
  }
  return best < 0 ? 6 : best;
}

Dec1Geom dec1_geom(int N, int K, int gsh, int k, bool down, int T = 1) {
  Dec1Geom g{};
  g.lg = pick_lg_dec1(K / 32, gsh);
  const int SG = 64 >> g.lg;
  const int rows_per_wave = down ? SG : 4 * SG;  // rows one rm step covers per block
  const double waves1 = (double)T * k * N / SG;
  g.rm = std::max(1, std::min(kDec1MaxRows, (int)(waves1 / kDec1TargetWaves + 0.5)));
  g.rows_per_block = g.rm * rows_per_wave;
  const int row_blocks = (N + g.rows_per_block - 1) / g.rows_per_block;
  g.grid = down ? row_blocks : k * row_blocks;
  return g;
}

// Calls of a few tokens take the one-token kernels, each token routed and
// streamed by its own blocks (grid.y): T tokens read T k expert slices where
// the dispatch plan and the grouped GEMVs read each used expert once, about
// E (1 - (1 - k / E)^T) of them under uniform routing. Measured, us per
// layer step, one-token kernels against plan + grouped GEMVs: Qwen3 T = 2
// 19.1 / 32.7, 4 29.5 / 42.2, 8 47.8 / 62.8; GPT-OSS 2 35.3 / 50.4, 4 60.5 /
// 71.9, 8 109.0 / 107.1; mixed-bit 2 36.0 / 46.1, 4 45.6 / 58.4, 8 68.6 /
// 74.4. The one-token kernels win up to about 1.35 slices per distinct
// expert (GPT-OSS at 8 tokens: 1.52).
constexpr int kDec1MaxT = 8;
constexpr double kDec1MaxSlicesPerExpert = 1.35;

bool dec1_tokens(const moe_layer_desc* d, int T) {
  if (T == 1) return true;
  if (T < 1 || T > kDec1MaxT) return false;
  const double E = d->n_experts, k = d->top_k;
  const double distinct = E * (1.0 - std::pow(1.0 - k / E, (double)T));
  return (double)T * k <= kDec1MaxSlicesPerExpert * distinct;
}

bool dec1_supported(const moe_layer_desc* d) {
  if (d->act_dtype == MOE_F32 || d->top_k > kDec1MaxK) return false;
  if (d->hidden > 8192 || d->intermediate > 8192) return false;
  // expert-local byte offsets stay below 2^31 (with a row block of slack)
  const moe_qproj* ps[2] = {&d->up, &d->down};  // gate, when present, is shaped as up
  for (const moe_qproj* p : ps) {
    const size_t row_bytes = (size_t)p->k * p->bits / 8;
    if (((size_t)p->n + 256) * row_bytes >= (1ull << 31)) return false;
  }
  return true;
}

// The shared expert of a one-token call inside the two one-token launches
// (its gate/up rows as more gate/up blocks, its down rows as m = SI / I more
// waves of each down block, the gated add in the down kernel's combine)
// instead of five launches of its own: when each shared projection has the
// bits, group size and scale dtype of its routed counterpart, SI is a
// multiple of I and k + m waves fit a block. in_kernel_gate: the sigmoid
// gate's logit comes from one more gate/up block (a dense gate row in the
// activation dtype, 16-byte aligned); otherwise its own launch writes it.
struct Dec1Shared {
  bool on = false, in_kernel_gate = false;
  int m = 0;
};

Dec1Shared dec1_shared(const moe_layer_desc* d) {
  Dec1Shared r;
  if (!d->has_shared) return r;
  const bool gated = d->activation != MOE_ACT_RELU2;
  auto same = [](const moe_qproj& a, const moe_qproj& b) {
    return a.bits == b.bits && a.group_size == b.group_size && a.sb_dtype == b.sb_dtype;
  };
  if ((gated && !same(d->gate, d->shared_gate)) || !same(d->up, d->shared_up) ||
      !same(d->down, d->shared_down))
    return r;
  const int I = d->intermediate, SI = d->shared_up.n;
  if (SI <= 0 || SI % I != 0 || SI > 8192 || d->top_k + SI / I > kDec1MaxWaves) return r;
  // shared byte offsets below 2^31, as for the routed stacks
  const size_t up_row = (size_t)d->shared_up.k * d->shared_up.bits / 8;
  const size_t dn_row = (size_t)d->shared_down.k * d->shared_down.bits / 8;
  if (((size_t)SI + 256) * up_row >= (1ull << 31) ||
      ((size_t)d->hidden + 256) * dn_row >= (1ull << 31))
    return r;
  r.on = true;
  r.m = SI / I;
  r.in_kernel_gate = d->shared_gate_weight && !d->shared_gate_q.weight &&
                     d->router_dtype == d->act_dtype &&
                     reinterpret_cast<uintptr_t>(d->shared_gate_weight) % 16 == 0;
  return r;
}

// down projection + weighted combine of one token (down1_kernel), with the
// shared expert's down rows and gated add when fs.on.
moe_status run_down1(const moe_layer_desc* d, int T, void* y, const uint32_t* idx, const float* w,
                     const void* act, hipStream_t st, KEvents ev, const void* res = nullptr,
                     const Dec1Shared& fs = Dec1Shared{}, const void* s_act = nullptr,
                     const void* s_logit = nullptr) {
  const int k = d->top_k, H = d->hidden, I = d->intermediate;
  const Dec1Geom dg = dec1_geom(H, I, group_shift(d->down.group_size), k, true, T);
  Down1Args dn{};
  dn.T = T;
  if (fs.on) {
    dn.sp = to_proj(d->shared_down);
    dn.s_act = s_act;
    dn.s_logit = s_logit;
    dn.m = fs.m;
  }
  dn.idx = idx;
  dn.w = w;
  dn.act = act;
  dn.p = to_proj(d->down);
  dn.out = y;
  dn.res = res;
  dn.k = k;
  dn.N = H;
  dn.K = I;
  dn.gsh = group_shift(d->down.group_size);
  dn.lg = dg.lg;
  dn.rows_per_block = dg.rows_per_block;
  MOE_HIP(launch_down1(d->down.bits, d->act_dtype, d->down.sb_dtype, dn, dg.rm, dg.grid, st, ev),
          "down+combine decode launch");
  return MOE_OK;
}

// The decoder steps around the block (Qwen3xText.swift:2640-2670,
// 1015-1035): x = rmsnorm(h + m) * nw is what the block reads, and the
// residual h + m is added to its output before the final rounding.
struct DecoderStep {
  const void* h;
  const void* m;
  const void* nw;
  float eps;
  void* res_out;  // nullable: the residual row(s), else workspace
};

// rx: the router's input rows (x for every family but Gemma 4). With `step`,
// x and rx are ignored: both read the normalised rows.
// allow_side: the shared expert may fork onto a side stream (created on a
// stream's first such call); false keeps every launch on `st`.
moe_status layer_forward(const moe_layer_desc* d, const void* x, const void* rx, int T, void* y,
                         void* ws, size_t ws_bytes, const moe_layer_trace* tr, hipStream_t st,
                         const DecoderStep* step = nullptr, bool allow_side = true) {
  MOE_TRY(validate_layer_impl(d));
  if (step) {
    if (!step->h || !step->m || !step->nw)
      return fail(MOE_ERR_INVALID, "Ops.addAndRmsNorm: input is NULL");
    if (d->hidden % 8 != 0)
      return fail(MOE_ERR_UNSUPPORTED, "Ops.addAndRmsNorm: hidden (%d) must be a multiple of 8",
                  d->hidden);
    if (!(step->eps >= 0.f) || !std::isfinite(step->eps))
      return fail(MOE_ERR_INVALID, "Ops.addAndRmsNorm: eps must be finite and non-negative");
    x = rx = step->h;  // placeholders until the normalised rows exist
  }
  if (!x || !rx || !y) return fail(MOE_ERR_INVALID, "MoELayer: input/output is NULL");
  if (T <= 0) return fail(MOE_ERR_INVALID, "MoELayer.decodeMany: T must be positive");
  const Workspace w = layout(d, T);
  if (!ws || ws_bytes < w.total)
    return fail(MOE_ERR_WORKSPACE, "MoELayer: workspace of %zu bytes needed for T=%d", w.total, T);
  const int E = d->n_experts, k = d->top_k, H = d->hidden, I = d->intermediate;
  const int M = T * k, xdt = d->act_dtype;
  // dispatch-timestamped events of the routed gate/up and down kernels
  auto kev = [&](int i) -> KEvents {
    KEvents ev;
    if (tr) {
      ev.start = reinterpret_cast<hipEvent_t>(tr->events[2 * i]);
      ev.stop = reinterpret_cast<hipEvent_t>(tr->events[2 * i + 1]);
    }
    return ev;
  };

  // 0. the decoder step before the block: residual add + RMSNorm, fused into
  //    the router projection for one token (Qwen3xText.swift:2650-2660)
  const void* res = nullptr;
  bool logits_done = false;
  if (step) {
    void* xn = at<void>(ws, w.xn);
    void* rs = step->res_out ? step->res_out : at<void>(ws, w.res);
    res = rs;
    if (T == 1 && !d->router_q.weight &&
        launch_router_logits_norm(step->h, step->m, step->nw, step->eps, xdt, H,
                                            d->router_weight, d->router_dtype, d->router_bias, E,
                                            at<void>(ws, w.logits), rs, xn, st) == hipSuccess) {
      logits_done = true;
    } else {
      (void)hipGetLastError();  // a refused fused launch leaves no error behind
      MOE_HIP(launch_add_rmsnorm(step->h, step->m, step->nw, step->eps, T, H, xdt, rs, xn, st),
              "add + RMSNorm launch");
    }
    x = rx = xn;
  }

  // the grouped GEMMs read the layer input as f16 operands: a bf16 input is
  // scaled into f16 range once, for the routed and the shared expert (by the
  // router's matrix-core kernel when it reads the same rows, else on its own)
  const bool gemm = !(T == 1 && dec1_supported(d)) && routed_gemm(d, T);
  const bool want_x16 = (gemm || shared_gemm(d, T)) && xdt == MOE_BF16;
  bool x16_done = false, sgate_done = false;
  int rsplits = 1;  // > 1: the router left partial sums for the top-k launch

  // 1. router projection (MoELayer.swift:540 / 689-690)
  if (logits_done) {
    // done above
  } else if (d->router_q.weight) {
    const moe_qproj& q = d->router_q;
    MOE_HIP(launch_router_q(q.bits, rx, xdt, T, H, to_proj(q), q.sb_dtype, group_shift(q.group_size),
                            d->router_bias, E, at<void>(ws, w.logits), st),
            "quantised router launch");
  } else {
    // a dense shared gate of the router's type, applied to the same rows, is
    // computed by the router launch when that runs on the matrix cores
    const bool gate2 = d->has_shared && d->shared_gate_weight && !d->shared_gate_q.weight && rx == x;
    // a split-K router writes fp32 partials into the down projection's
    // output rows (Y, unused until the down projection), which the top-k
    // launch below reduces
    MOE_HIP(launch_router_logits(rx, xdt, T, H, d->router_weight, d->router_dtype, d->router_bias,
                                 E, at<void>(ws, w.logits), st,
                                 want_x16 && rx == x ? at<void>(ws, w.x16) : nullptr, &x16_done,
                                 gate2 ? d->shared_gate_weight : nullptr, 1,
                                 gate2 ? at<void>(ws, w.s_logit) : nullptr, &sgate_done,
                                 at<float>(ws, w.Y), (size_t)T * k * H * dt_size(xdt), &rsplits),
            "router logits launch");
  }

  const void* x16 = x;
  if (want_x16) {
    if (!x16_done)
      MOE_HIP(launch_to_a16(x, at<void>(ws, w.x16), (int64_t)T * H, st), "f16 operand launch");
    x16 = at<void>(ws, w.x16);
  }

  const bool dec1 = (dec1_tokens(d, T) && dec1_supported(d));
  int smode = 0;
  // a shared expert of kSideMinRows or more rows overlaps the routed experts
  // (MoELayer.swift:620-624: it only joins at the combine); a smaller one
  // stays in order (the fork and join cost a one-token NemotronH-shaped layer
  // 3.5 us more than they saved)
  SideFork side(allow_side && d->has_shared && T >= kSideMinRows, st);
  MOE_TRY(side.status());
  // one token: the shared expert inside the two one-token launches when its
  // formats allow (its gate logit from its own launch unless dense)
  const Dec1Shared fs = (dec1 && T == 1) ? dec1_shared(d) : Dec1Shared{};
  if (fs.on) {
    if (!fs.in_kernel_gate) MOE_TRY(shared_gate_logits(d, x, T, ws, w, st));
  } else if (dec1) {
    MOE_TRY(shared_expert(d, x, x16, T, ws, w, side.stream(), &smode, sgate_done));
  }
  if (dec1) MOE_TRY(side.mark());
  if (dec1) {
    // 2. one token: routing inside the gate/up kernel (MoELayer.swift:1167-1282
    //    without a host round trip), then the fused down + combine
    // gate/up rows (the up projection alone for squared-ReLU experts: the
    // kernel reads zeros for the missing gate)
    const moe_qproj& gu = d->activation == MOE_ACT_RELU2 ? d->up : d->gate;
    const Dec1Geom gg = dec1_geom(I, H, group_shift(gu.group_size), k, false, T);
    Decode1Args g{};
    g.logits = at<void>(ws, w.logits);
    g.E = E;
    g.k = k;
    g.T = T;
    g.ro = route_opts(d);
    g.idx = at<uint32_t>(ws, w.idx);
    g.w = at<float>(ws, w.w);
    // the plan over several tokens comes from its own launch (below), when a
    // trace asks for it
    g.perm = T == 1 ? at<uint32_t>(ws, w.perm) : nullptr;
    g.offsets = T == 1 ? at<uint32_t>(ws, w.offsets) : nullptr;
    g.x = x;
    g.g = to_proj(d->gate);
    g.u = to_proj(d->up);
    g.act = at<void>(ws, w.act);
    g.N = I;
    g.K = H;
    g.gsh = group_shift(gu.group_size);
    g.lg = gg.lg;
    g.rows_per_block = gg.rows_per_block;
    g.row_blocks = gg.grid / k;
    g.act_kind = d->activation;
    g.alpha = d->act_alpha;
    g.limit = d->act_limit;
    int grid = gg.grid;
    const bool sgate = fs.on && (d->shared_gate_weight || d->shared_gate_q.weight);
    if (fs.on) {
      g.sg = to_proj(d->shared_gate);
      g.su = to_proj(d->shared_up);
      g.s_act = at<void>(ws, w.s_act);
      g.SN = d->shared_up.n;
      g.s_blocks = (g.SN + gg.rows_per_block - 1) / gg.rows_per_block;
      g.s_logit = at<void>(ws, w.s_logit);
      g.sgw = fs.in_kernel_gate ? d->shared_gate_weight : nullptr;
      grid += g.s_blocks + (fs.in_kernel_gate ? 1 : 0);
    }
    MOE_HIP(launch_gateup1(gu.bits, xdt, gu.sb_dtype, g, gg.rm, grid, st, kev(0)),
            "gate/up decode launch");
    // the residual goes into the last store: down1's without a separate
    // shared expert
    MOE_TRY(run_down1(d, T, y, g.idx, g.w, g.act, st, kev(1), smode ? nullptr : res, fs,
                      at<void>(ws, w.s_act), sgate ? at<void>(ws, w.s_logit) : nullptr));
    // several tokens: the dispatch plan only for a trace that asks for it
    // (the kernels above route each token themselves)
    if (T > 1 && tr && (tr->perm || tr->offsets))
      MOE_HIP(launch_dispatch_plan(at<uint32_t>(ws, w.idx), T, k, E, at<uint32_t>(ws, w.counts),
                                   at<uint32_t>(ws, w.offsets), at<uint32_t>(ws, w.perm),
                                   at<uint32_t>(ws, w.inv), at<uint32_t>(ws, w.used),
                                   at<void>(ws, w.plan_scratch), dispatch_scratch_bytes(T, k, E),
                                   st, nullptr, nullptr),
              "dispatch plan launch");
    MOE_TRY(side.join());
    if (smode)
      MOE_HIP(launch_add_shared(y, at<void>(ws, w.s_out), at<void>(ws, w.s_logit), smode, T, H, xdt,
                                st, res),
              "shared add launch");
  } else {
    // squared-ReLU experts: the single up projection (NemotronHText.swift:756-761)
    const bool gated = d->activation != MOE_ACT_RELU2;
    const moe_qproj& p0 = gated ? d->gate : d->up;
    const moe_qproj* p1 = gated ? &d->up : nullptr;
    // the GEMM work lists, written by the plan's last launch when it can
    const GemmItemsReq ireq{p0.n, p1 != nullptr, at<uint32_t>(ws, w.items_gu),
                            H,    false,         at<uint32_t>(ws, w.items_dn)};
    bool items_done = false;
    // 2. selection + dispatch plan (MoELayer.swift:706-792): one launch for a
    //    small batch, else the top-k and plan kernels (past 8 tokens the GEMM
    //    path keeps the plan kernel, whose last launch writes the work lists)
    if ((T > 8 && gemm) || rsplits > 1 ||
        launch_route_plan(at<void>(ws, w.logits), xdt, T, E, k, route_opts(d),
                          at<uint32_t>(ws, w.idx), at<float>(ws, w.w), at<uint32_t>(ws, w.counts),
                          at<uint32_t>(ws, w.offsets), at<uint32_t>(ws, w.perm),
                          at<uint32_t>(ws, w.inv), at<uint32_t>(ws, w.used), st) != hipSuccess) {
      (void)hipGetLastError();  // a refused fused launch leaves no error behind
      MOE_HIP(launch_router_topk(at<void>(ws, w.logits), xdt, T, E, k, route_opts(d),
                                 at<uint32_t>(ws, w.idx), at<float>(ws, w.w), st,
                                 at<float>(ws, w.Y), rsplits, d->router_bias,
                                 sgate_done ? at<void>(ws, w.s_logit) : nullptr, 1),
              "router top-k launch");
      MOE_HIP(launch_dispatch_plan(at<uint32_t>(ws, w.idx), T, k, E, at<uint32_t>(ws, w.counts),
                                   at<uint32_t>(ws, w.offsets), at<uint32_t>(ws, w.perm),
                                   at<uint32_t>(ws, w.inv), at<uint32_t>(ws, w.used),
                                   at<void>(ws, w.plan_scratch), dispatch_scratch_bytes(T, k, E),
                                   st, gemm ? &ireq : nullptr, &items_done),
              "dispatch plan launch");
    }
    const int slots = std::min(E, M);
    // 3. gate/up + activation over the plan (MoELayer.swift:883-893)
    if (gemm) {
      if (!items_done)
        MOE_HIP(launch_gemm_items(at<uint32_t>(ws, w.offsets), E, ireq.N0, ireq.gateup0,
                                  ireq.items0, ireq.N1, ireq.gateup1, ireq.items1, st),
                "GEMM work list launch");
      MOE_TRY(run_gemm(p0, p1, x16, xdt, true, at<uint32_t>(ws, w.perm), k,
                       at<uint32_t>(ws, w.offsets), at<uint32_t>(ws, w.items_gu), M,
                       at<void>(ws, w.act), d->activation, d->act_alpha, d->act_limit, st, kev(0)));
    } else {
      MOE_TRY(run_gemv(p0, p1, x, xdt, at<uint32_t>(ws, w.perm), k,
                       at<uint32_t>(ws, w.offsets), at<uint32_t>(ws, w.used), slots, M, T == 1,
                       at<void>(ws, w.act), d->activation, d->act_alpha, d->act_limit, st, kev(0),
                       T));
    }
    // 4. down projection, then the weighted combine (MoELayer.swift:899-939)
    if (gemm) {
      MOE_TRY(run_gemm(d->down, nullptr, at<void>(ws, w.act), xdt, false, nullptr, 1,
                       at<uint32_t>(ws, w.offsets), at<uint32_t>(ws, w.items_dn), M,
                       at<void>(ws, w.Y), 0, 0.f, 0.f, st, kev(1)));
    } else {
      MOE_TRY(run_gemv(d->down, nullptr, at<void>(ws, w.act), xdt, nullptr, 1,
                       at<uint32_t>(ws, w.offsets), at<uint32_t>(ws, w.used), slots, M, T == 1,
                       at<void>(ws, w.Y), 0, 0.f, 0.f, st, kev(1), T));
    }
    // The shared expert is enqueued after the routed launches (its fork point
    // is still the router step). Replaying a HIP graph captured from this
    // call, the runtime ran the branch captured first after the fork on the
    // router's hardware queue and the other on a second queue (rocprofv3
    // traces); that first branch should be the routed chain, which sets the
    // step's length. Enqueued first, the shared branch took the router's
    // queue and the routed chain's top-k started 11 us after the router
    // ended (mixed-bit prefill step 373.8 -> 366.7 us with this order).
    MOE_TRY(shared_expert(d, x, x16, T, ws, w, side.stream(), &smode, sgate_done));
    MOE_TRY(side.mark());
    MOE_TRY(side.join());
    MOE_HIP(launch_unpermute(at<void>(ws, w.Y), at<uint32_t>(ws, w.inv), at<float>(ws, w.w), T, H,
                             k, y, xdt, smode ? at<void>(ws, w.s_out) : nullptr,
                             smode ? at<void>(ws, w.s_logit) : nullptr, smode, st, res),
            "unpermute launch");
  }
  MOE_TRY(copy_trace(d, T, ws, w, tr, st));
  return MOE_OK;
}

// The kernels layer_forward runs for T rows (the same predicates it uses).
moe_layer_paths layer_paths(const moe_layer_desc* d, int T, bool x_aligned) {
  moe_layer_paths p{};
  const int E = d->n_experts, k = d->top_k, M = T * k, xdt = d->act_dtype;
  const bool gated = d->activation != MOE_ACT_RELU2;
  auto gk = [](GemvKind kd) { return (int32_t)(kd == kGemvMma ? MOE_PATH_GEMV_MMA : MOE_PATH_GEMV); };
  const moe_qproj& p0 = gated ? d->gate : d->up;
  const moe_qproj* p1 = gated ? &d->up : nullptr;
  const bool dec1 = dec1_tokens(d, T) && dec1_supported(d);
  if (dec1) {
    p.gate_up = p.down = MOE_PATH_DECODE1;
  } else if (routed_gemm(d, T)) {
    p.gate_up = p.down = MOE_PATH_GEMM;
  } else {
    const int slots = std::min(E, M);
    p.gate_up = gk(gemv_kind(p0, p1, x_aligned, xdt, slots, M, T == 1, T));
    p.down = gk(gemv_kind(d->down, nullptr, true, xdt, slots, M, T == 1, T));
  }
  if (d->has_shared) {
    const moe_qproj& s0 = gated ? d->shared_gate : d->shared_up;
    const moe_qproj* s1 = gated ? &d->shared_up : nullptr;
    if (dec1 && T == 1 && dec1_shared(d).on) {
      p.shared_gate_up = p.shared_down = MOE_PATH_DECODE1;
    } else if (shared_gemm(d, T)) {
      p.shared_gate_up = p.shared_down = MOE_PATH_GEMM;
    } else {
      p.shared_gate_up = gk(gemv_kind(s0, s1, x_aligned, xdt, 1, T, T == 1, 1 << 30));
      p.shared_down = gk(gemv_kind(d->shared_down, nullptr, true, xdt, 1, T, T == 1, 1 << 30));
    }
  }
  return p;
}

}  // namespace

namespace moe {
// moe_layer_forward with every launch on `stream` (no side stream is created)
// and the workspace given by the caller; for allocation-free callers.
moe_status layer_forward_in_order(const moe_layer_desc* d, const void* x, int32_t T, void* y,
                                  void* ws, size_t ws_bytes, const moe_layer_trace* tr,
                                  hipStream_t st) {
  MOE_TRY(layer_forward(d, x, x, T, y, ws, ws_bytes, tr, st, nullptr, false));
  return ok();
}
size_t layer_workspace_bytes(const moe_layer_desc* d, int32_t T) {
  if (!d || T <= 0 || validate_layer_impl(d) != MOE_OK) return 0;
  return layout(d, T).total;
}
}  // namespace moe

extern "C" moe_status moe_layer_path(const moe_layer_desc* d, int32_t T, moe_layer_paths* out) {
  MOE_TRY(validate_layer_impl(d));
  if (!out) return fail(MOE_ERR_INVALID, "moe_layer_path: out is NULL");
  if (T <= 0) return fail(MOE_ERR_INVALID, "MoELayer.decodeMany: T must be positive");
  *out = layer_paths(d, T, true);
  return ok();
}

extern "C" moe_status moe_layer_forward(const moe_layer_desc* d, const void* x, int32_t T, void* y,
                                        void* workspace, size_t workspace_bytes,
                                        const moe_layer_trace* trace, hipStream_t stream) {
  MOE_TRY(layer_forward(d, x, x, T, y, workspace, workspace_bytes, trace, stream));
  return ok();
}

extern "C" moe_status moe_layer_forward_residual(const moe_layer_desc* d, const void* h,
                                                 const void* mixer_out, const void* norm_weight,
                                                 float eps, int32_t T, void* y,
                                                 void* residual_out, void* workspace,
                                                 size_t workspace_bytes,
                                                 const moe_layer_trace* trace,
                                                 hipStream_t stream) {
  const DecoderStep step{h, mixer_out, norm_weight, eps, residual_out};
  MOE_TRY(layer_forward(d, nullptr, nullptr, T, y, workspace, workspace_bytes, trace, stream,
                        &step));
  return ok();
}

extern "C" moe_status moe_add_rmsnorm(const void* a, const void* b, const void* weight, float eps,
                                      int32_t n_rows, int32_t row_size, int32_t dtype,
                                      void* residual_out, void* normed_out, hipStream_t stream) {
  if (!a || !b || !weight || !residual_out || !normed_out)
    return fail(MOE_ERR_INVALID, "Ops.addAndRmsNorm: NULL pointer");
  if (n_rows <= 0 || row_size <= 0)
    return fail(MOE_ERR_INVALID, "Ops.addAndRmsNorm: n must be positive (got %d)", row_size);
  if (!dt_ok(dtype)) return fail(MOE_ERR_INVALID, "Ops.addAndRmsNorm: bad dtype");
  if (row_size % 8 != 0 || row_size > kMaxHidden)
    return fail(MOE_ERR_UNSUPPORTED,
                "Ops.addAndRmsNorm: row size %d must be a multiple of 8 and at most %d", row_size,
                kMaxHidden);
  if (!(eps >= 0.f) || !std::isfinite(eps))
    return fail(MOE_ERR_INVALID, "Ops.addAndRmsNorm: eps must be finite and non-negative");
  MOE_HIP(launch_add_rmsnorm(a, b, weight, eps, n_rows, row_size, dtype, residual_out, normed_out,
                             stream),
          "add + RMSNorm launch");
  return ok();
}

extern "C" moe_status moe_layer_forward_routed(const moe_layer_desc* d, const void* x,
                                               const void* router_x, int32_t T, void* y,
                                               void* workspace, size_t workspace_bytes,
                                               const moe_layer_trace* trace, hipStream_t stream) {
  MOE_TRY(layer_forward(d, x, router_x ? router_x : x, T, y, workspace, workspace_bytes, trace,
                        stream));
  return ok();
}

// ---------------------------------------------------------------------------
// MoELayer handle
// ---------------------------------------------------------------------------

// Host-side mirror of the reference's MoELayer instance: it holds the layer
// description and lazily sized scratch (MoELayer.swift:408-429). Calls are
// stream-ordered and the instance is not reentrant (MoELayer.swift:311-318).
struct moe_layer {
  moe_layer_desc desc;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  int ws_tokens = 0;
  bool ws_async = false;          // ws came from hipMallocAsync
  hipStream_t last_st = nullptr;  // the stream of the latest call

  // Grows the scratch to T rows, stream-ordered: the old scratch is freed on
  // the stream of the latest call (after that call, whose side-stream work
  // joins back into it, has finished with it) and the new one allocated on
  // `st`, so growing stalls no other stream. A device without memory pools
  // falls back to a device-wide wait and hipFree. Allocating is refused while
  // `st` is being captured: a handle that is captured must have run once,
  // eagerly, at its largest T.
  moe_status reserve(int T, hipStream_t st) {
    if (T <= ws_tokens) return MOE_OK;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    MOE_HIP(hipStreamIsCapturing(st, &cs), "MoELayer scratch resize");
    if (cs != hipStreamCaptureStatusNone)
      return fail(MOE_ERR_WORKSPACE,
                  "MoELayer: scratch for T=%d (reserved for %d) cannot grow under stream capture; "
                  "run the handle once at its largest T before capturing",
                  T, ws_tokens);
    const size_t need = moe_layer_workspace_bytes(&desc, T);
    if (ws) {
      hipError_t e;
      if (ws_async) {
        e = hipFreeAsync(ws, last_st);
      } else {
        e = hipDeviceSynchronize();
        if (e == hipSuccess) e = hipFree(ws);
      }
      ws = nullptr;
      ws_bytes = 0;
      ws_tokens = 0;
      MOE_HIP(e, "MoELayer scratch free");
    }
    if (hipMallocAsync(&ws, need, st) == hipSuccess) {
      ws_async = true;
    } else {
      (void)hipGetLastError();  // no memory pools: a plain allocation
      ws = nullptr;
      ws_async = false;
      MOE_HIP(hipMalloc(&ws, need), "MoELayer scratch allocation");
    }
    ws_bytes = need;
    ws_tokens = T;
    return MOE_OK;
  }

  moe_status decode_many(const void* h, int T, void* out, hipStream_t st) {
    if (T <= 0) return fail(MOE_ERR_INVALID, "MoELayer.decodeMany: T must be positive");
    MOE_TRY(reserve(T, st));
    last_st = st;
    return layer_forward(&desc, h, h, T, out, ws, ws_bytes, nullptr, st);
  }
};

extern "C" moe_status moe_layer_create(const moe_layer_desc* d, moe_layer_t* out) {
  if (!out) return fail(MOE_ERR_INVALID, "moe_layer_create: out is NULL");
  *out = nullptr;
  MOE_TRY(validate_layer_impl(d));
  moe_layer* L = new (std::nothrow) moe_layer();
  if (!L) return fail(MOE_ERR_INVALID, "moe_layer_create: out of host memory");
  L->desc = *d;
  *out = L;
  return ok();
}

extern "C" void moe_layer_destroy(moe_layer_t layer) {
  if (!layer) return;
  if (layer->ws) {
    (void)hipDeviceSynchronize();
    if (layer->ws_async) {
      (void)hipFreeAsync(layer->ws, nullptr);
      (void)hipStreamSynchronize(nullptr);
    } else {
      (void)hipFree(layer->ws);
    }
  }
  delete layer;
}

extern "C" moe_status moe_layer_decode(moe_layer_t layer, const void* h, void* out,
                                       hipStream_t stream) {
  if (!layer) return fail(MOE_ERR_INVALID, "MoELayer.decode: layer is NULL");
  MOE_TRY(layer->decode_many(h, 1, out, stream));
  return ok();
}

extern "C" moe_status moe_layer_decode_many(moe_layer_t layer, const void* h, int32_t T, void* out,
                                            hipStream_t stream) {
  if (!layer) return fail(MOE_ERR_INVALID, "MoELayer.decodeMany: layer is NULL");
  MOE_TRY(layer->decode_many(h, T, out, stream));
  return ok();
}
