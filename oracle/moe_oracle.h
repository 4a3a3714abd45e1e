/*
 * moe_oracle.h — CPU restatement of FFAI's mixture-of-experts layer.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the correctness checker for the
 * HIP path in ffai_amd/ and the timed CPU baseline in bench.py. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it. The
 * product (libmoehip.so) never links, loads or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the FFAI checkout, Sources/FFAI/...).
 *
 * Parity status of each part (what pins it) is listed in moe_oracle.c's
 * header; no function here is "parity unpinned".
 */
#ifndef MOE_ORACLE_H
#define MOE_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types — same numbering as moe_dtype in include/moe_hip.h. */
enum { OR_F32 = 0, OR_F16 = 1, OR_BF16 = 2 };

/* Gating behaviours of MoERouter.route (MoELayer.swift:71-78,140-205) and
 * the NemotronH sigmoid router (NemotronHText.swift:838-868). */
enum { OR_SOFTMAX_THEN_TOPK = 0, OR_TOPK_THEN_SOFTMAX = 1, OR_SIGMOID_TOPK = 2 };

/* Expert activations: SwiGLU (Ops.swift:6400-6411), GPT-OSS clamped
 * alpha-swish (GPTOSSText.swift:1415-1431), Gemma 4 GELU-gated
 * (Gemma4Text.swift:965) and NemotronH squared ReLU of the single up
 * projection (NemotronHText.swift:756-761). */
enum { OR_ACT_SWIGLU = 0, OR_ACT_GPTOSS = 1, OR_ACT_GEGLU = 2, OR_ACT_RELU2 = 3 };

/* ---- scalar conversions (Tensor.swift:146-150 for bf16 RNE) ------------ */
float    or_bf16_to_f32(uint16_t h);
uint16_t or_f32_to_bf16(float f);
float    or_f16_to_f32(uint16_t h);
uint16_t or_f32_to_f16(float f);
float    or_round_dt(float v, int dt);
void     or_load(const void* src, int dt, size_t n, float* dst);
void     or_store(const float* src, int dt, size_t n, void* dst);

/* ---- deterministic exp used by the router softmax ---------------------- */
float or_expf(float x);

/* ---- affine bit-stream format (Layers.swift:134-143, QuantizedOps.swift:
 *      33-45, QuantizedOpsValidation.swift:34-110) ------------------------ */
int  or_unpack_codes(const uint32_t* w, int bits, size_t n, uint8_t* codes);
int  or_pack_codes(const uint8_t* codes, int bits, size_t n, uint32_t* w);
long or_packed_u32_count(long numel, int bits);
int  or_derive_bits(long packed_cols, long scale_cols, long group_size);
int  or_dequantize_affine(const uint32_t* w, const void* scales, const void* biases,
                          int sb_dt, int bits, int group_size, size_t numel, float* out);

/* ---- router (MoELayer.swift:140-296, GPTOSSText.swift:345-366,1349-1361) */
void or_router_logits(const void* x, int x_dt, int T, int H,
                      const void* W, int w_dt, const void* bias, int E,
                      float* logits);
int  or_topk_indices(const float* v, int n, int k, int* out);
void or_softmax(const float* x, int n, float* out);
int  or_route(const float* logits, int T, int E, int k, int gating, int norm_topk,
              const float* expert_bias, uint32_t* idx, float* weights);
/* or_route with logits * logit_scale first (Gemma4Text.swift:938-944) and
 * the final weights * routed_scale (NemotronH routed_scaling_factor,
 * NemotronHText.swift:867) then * expert_scale[e] when non-NULL
 * (Gemma4Text.swift:945-950). */
int  or_route_scaled(const float* logits, int T, int E, int k, int gating, int norm_topk,
                     const float* expert_bias, float logit_scale, float routed_scale,
                     const float* expert_scale, uint32_t* idx, float* weights);

/* ---- dispatch plan (MoELayer.swift:752-792) ----------------------------- */
int or_dispatch_plan(const uint32_t* idx, int T, int k, int E,
                     uint32_t* counts, uint32_t* offsets,
                     uint32_t* perm, uint32_t* inv_perm);

/* ---- stacked affine projection ----------------------------------------- */
typedef struct or_qproj {
    const uint32_t* weight;  /* [E, N, K*bits/32] */
    const void* scales;      /* [E, N, K/gs] in sb_dt */
    const void* biases;      /* [E, N, K/gs] in sb_dt */
    const void* out_bias;    /* nullable [E, N] in the activation dtype */
    int bits, group_size, sb_dt, n, k;
} or_qproj;

/* The router projection with an affine-quantised weight (QuantizedLinear,
 * Layers.swift:371-400): row e of W dequantised as or_qgemm_rows does
 * (w = s*q + b in fp32), dot products in double, then rounded as
 * or_router_logits rounds. W is a one-expert stack with W->n = E. */
int or_router_logits_q(const void* x, int x_dt, int T, int H, const or_qproj* W,
                       const void* bias, int E, float* logits);

/* out[m, :] = W[row_expert[m]] · a[m, :]  (fp32 dequant, double accumulate) */
int or_qgemm_rows(const or_qproj* p, const float* a, int M,
                  const uint32_t* row_expert, float* out);

/* Tanh-form GELU (Tests/FFAITests/Ops/OpsTests.swift:254-273). */
float or_gelu(float g);
/* The activation before its final rounding to dt; GEGLU rounds the GELU to
 * dt before the product (Gemma4Text.swift:965: Ops.mul(Ops.gelu(g), u)).
 * RELU2 reads u only. or_act is or_act_dt at OR_F32. */
float or_act_dt(float g, float u, int act, float alpha, float limit, int dt);
float or_act(float g, float u, int act, float alpha, float limit);

/* out[t,:] = Σ_s w[t,s] · Y[inv_perm[t*k+s], :] (Ops.swift:5030-5110) */
void or_unpermute(const float* Y, const uint32_t* inv_perm, const float* w,
                  int T, int H, int k, int dt, float* out);

/* ---- whole layer (MoELayer.decodeMany, MoELayer.swift:677-969; shared
 *      expert Qwen3xText.swift:1047-1104 / MoELayer.swift:620-624) --------- */
typedef struct or_layer {
    int hidden, n_experts, top_k, intermediate;
    int act_dt;
    const void* router_weight; int router_dt; const void* router_bias;
    int gating, norm_topk; const float* expert_bias;
    or_qproj gate, up, down;
    int activation; float alpha, limit;
    int has_shared;
    or_qproj shared_gate, shared_up, shared_down;
    const void* shared_gate_weight;   /* nullable [H] in router_dt */
    float logit_scale, routed_scale;  /* 0 reads as 1 */
    const float* expert_scale;        /* nullable [E] */
    /* quantised router / shared gate (QuantizedLinear, Layers.swift:371-400):
     * used instead of router_weight / shared_gate_weight when .weight is
     * non-NULL; one-expert stacks [1, E, H] and [1, 1, H] */
    or_qproj router_q, shared_gate_q;
} or_layer;

/* If given_logits is non-NULL it replaces the router projection (used to
 * route from the logits a GPU run produced). Any of the trace pointers may
 * be NULL. Returns 0 on success. */
int or_moe_layer(const or_layer* L, const void* x, int T, void* y,
                 const float* given_logits,
                 float* logits_out, uint32_t* idx_out, float* w_out);
/* The same with the router reading router_x while the experts read x
 * (Gemma4Text.swift:932-936, 960). */
int or_moe_layer_routed(const or_layer* L, const void* x, const void* router_x, int T,
                        void* y, const float* given_logits,
                        float* logits_out, uint32_t* idx_out, float* w_out);

/* ---- decoder steps around the block (Qwen3xText.swift:2640-2670,
 *      1015-1035) --------------------------------------------------------- */
void or_add_rmsnorm(const float* a, const float* b, const float* w, float eps, int T, int H,
                    int dt, float* res_out, float* xn_out);
void or_residual_combine(const float* res, const float* base, const float* value, float gate,
                         int n, int dt, float* out);
int or_moe_layer_residual(const or_layer* L, const void* h, const void* m, const float* nw,
                          float eps, int T, void* y, const float* given_logits,
                          float* xn_out, float* res_out, float* logits_out, uint32_t* idx_out,
                          float* w_out);

/* ---- MXFP4 -> affine 4-bit transcode (GPTOSSText.swift:941-1236) ------- */
float or_mxfp4_value(int code);
void or_mxfp4_to_affine(const uint32_t* packed, const uint8_t* e8m0, long groups,
                        uint32_t* out_w, void* out_s, void* out_b, int sb_dt);

#ifdef __cplusplus
}
#endif
#endif
