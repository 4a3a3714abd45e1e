/*
 * moe_hip.h — C ABI of libmoehip.so, the MI355X (gfx950) mixture-of-experts
 * feed-forward layer.
 *
 * This is the drop-in boundary for FFAI's MoE block. A Swift package imports
 * it through `module CMoEHIP { header "moe_hip.h" link "moehip" export * }`.
 * Every entry point below names the reference interface it replaces
 * (paths relative to the FFAI checkout).
 *
 * Conventions
 *  - Plain pointers and sizes only. Device pointers are HIP device memory;
 *    every launch is stream-ordered and asynchronous on `stream`.
 *  - The caller owns every buffer. The layer entry points take a
 *    caller-provided workspace and never allocate on the hot path; the
 *    MoELayer handle (moe_layer_create) owns a lazily sized workspace the
 *    way the reference's MoELayer owns its scratch tensors
 *    (Sources/FFAI/Models/MoELayer.swift:408-429).
 *  - Shapes, bit widths, group sizes and dtypes are validated on the host
 *    before any launch; a violation returns a status and launches nothing
 *    (the reference traps in a precondition instead, e.g.
 *    Sources/FFAI/Ops/Ops.swift:4585-4615). moe_last_error_string() gives
 *    the reason (thread-local).
 *  - Not reentrant per workspace / layer handle (MoELayer.swift:311-318).
 */
#ifndef MOE_HIP_H
#define MOE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

typedef enum moe_status {
    MOE_OK = 0,
    MOE_ERR_INVALID = 1,     /* shape / argument contract violated */
    MOE_ERR_UNSUPPORTED = 2, /* valid for the reference, not built here */
    MOE_ERR_WORKSPACE = 3,   /* workspace missing or too small */
    MOE_ERR_HIP = 4          /* the HIP runtime reported an error */
} moe_status;

/* Element types (Sources/FFAI/DType.swift:20-39). */
typedef enum moe_dtype { MOE_F32 = 0, MOE_F16 = 1, MOE_BF16 = 2 } moe_dtype;

/* MoEGatingMode (Sources/FFAI/Models/MoELayer.swift:71-78), plus the
 * NemotronH sigmoid router (Models/Text/NemotronHText.swift:700-725,
 * 838-868): scores sigmoid(logit), expert_bias added for the selection
 * only, weights the unbiased sigmoids, divided by their sum + 1e-20 when
 * norm_topk_prob and k > 1. */
typedef enum moe_gating {
    MOE_SOFTMAX_THEN_TOPK = 0,
    MOE_TOPK_THEN_SOFTMAX = 1,
    MOE_SIGMOID_TOPK = 2
} moe_gating;

/* Expert activation:
 *   SWIGLU  silu(g)*u (Ops.swift:6400-6411);
 *   GPTOSS  clamped alpha-swish g*sigmoid(alpha*g)*(u+1) with g<=limit,
 *           |u|<=limit (Models/Text/GPTOSSText.swift:1415-1431);
 *   GEGLU   gelu(g)*u, tanh-form GELU rounded to the activation dtype
 *           before the product (Gemma4Text.swift:965, the GELU of
 *           Tests/FFAITests/Ops/OpsTests.swift:254-273);
 *   RELU2   relu(u)^2 of a single up projection, no gate projection
 *           (NemotronHText.swift:756-761). */
typedef enum moe_activation {
    MOE_ACT_SWIGLU = 0,
    MOE_ACT_GPTOSS = 1,
    MOE_ACT_GEGLU = 2,
    MOE_ACT_RELU2 = 3
} moe_activation;

/* Stacked mlx-affine projection of n_experts experts
 * (MoELayer.StackedInt4Experts, MoELayer.swift:347-390, generalised to
 * 2/3/4/5/6/8 bits):
 *   weight   [n_experts, n, k*bits/32] u32, little-endian bit stream per row
 *   scales   [n_experts, n, k/group_size] in sb_dtype
 *   biases   [n_experts, n, k/group_size] in sb_dtype
 *   out_bias [n_experts, n] in the activation dtype, nullable (GPT-OSS
 *            per-expert projection bias, GPTOSSText.swift:1403-1410)
 * Dequantised weight: w = scale * q + bias (QuantizedOps.swift:33-45). */
typedef struct moe_qproj {
    const uint32_t* weight;
    const void* scales;
    const void* biases;
    const void* out_bias;
    int32_t bits;
    int32_t group_size;
    int32_t sb_dtype;
    int32_t n;
    int32_t k;
    int32_t n_experts;
} moe_qproj;

/* MoELayer + MoERouter configuration (MoELayer.swift:97-124,440-498;
 * GPT-OSS GPTOSSMoELayer, GPTOSSText.swift:1302-1340; Qwen3.5 shared
 * expert Qwen35MoEFFN, Qwen3xText.swift:870-928; NemotronHMoELayer,
 * NemotronHText.swift:694-868; Gemma4MoEFFN, Gemma4Text.swift:928-978).
 * With MOE_ACT_RELU2 the gate projections (routed and shared) are absent:
 * gate.weight and shared_gate.weight are NULL. */
typedef struct moe_layer_desc {
    int32_t hidden;
    int32_t n_experts;
    int32_t top_k;
    int32_t intermediate;
    int32_t act_dtype;             /* activations, logits, outputs */
    /* router projection: dense [n_experts, hidden] */
    const void* router_weight;
    int32_t router_dtype;
    const void* router_bias;       /* nullable [n_experts] in act_dtype */
    int32_t gating;                /* moe_gating */
    int32_t norm_topk_prob;
    const float* expert_bias;      /* nullable [n_experts] f32 (LFM2) */
    /* routed experts */
    moe_qproj gate, up, down;      /* gate/up: n=intermediate,k=hidden */
    int32_t activation;            /* moe_activation */
    float act_alpha, act_limit;    /* GPT-OSS: 1.702, 7.0 */
    /* optional always-on shared expert (n_experts = 1 in each proj) */
    int32_t has_shared;
    moe_qproj shared_gate, shared_up, shared_down;
    const void* shared_gate_weight; /* nullable dense [hidden] in
                                       router_dtype: sigmoid gate */
    /* routing scales (0 reads as 1.0, so zero-initialised descriptors
     * keep the plain MoERouter behaviour) */
    float logit_scale;             /* logits * s in f32 before gating
                                      (Gemma 4 hidden^-0.5,
                                      Gemma4Text.swift:938-944) */
    float routed_scale;            /* final weights * s (NemotronH
                                      routed_scaling_factor) */
    const float* expert_scale;     /* nullable [n_experts] f32: final
                                      weight * expert_scale[e] (Gemma 4
                                      per_expert_scale,
                                      Gemma4Text.swift:945-950) */
    /* Affine-quantised router and shared-expert gate: the mlx
     * QuantizedLinear that loadLinear returns for a quantised checkpoint
     * (Layers.swift:371-400; Qwen3xText.swift:605-606, 660-661). When
     * router_q.weight is non-NULL the router projection is this one-expert
     * stack [1, n_experts, hidden] (n = n_experts, k = hidden, n_experts =
     * 1, out_bias NULL) and router_weight must be NULL; router_bias still
     * applies. Likewise shared_gate_q ([1, 1, hidden]) replaces
     * shared_gate_weight. Dequantised inside the router kernels (the weights
     * are never rounded); 16-bit activations only. */
    moe_qproj router_q;
    moe_qproj shared_gate_q;
} moe_layer_desc;

/* Optional device outputs of a layer call, for callers and tests that need
 * the routing decisions. Any pointer may be NULL. */
typedef struct moe_layer_trace {
    void* logits;          /* [T, n_experts] act_dtype */
    uint32_t* topk_idx;    /* [T, top_k] */
    float* topk_weight;    /* [T, top_k] */
    uint32_t* perm;        /* [T*top_k] sorted position -> token-major entry */
    uint32_t* offsets;     /* [n_experts + 1] */
    /* hipEvent_t handles (each nullable) recorded by the dispatch of the
     * routed expert kernels themselves, so that their elapsed time is the
     * kernel's own execution: [0]/[1] start/end of the gate/up kernel,
     * [2]/[3] start/end of the down kernel (fused with the combine on the
     * one-token path). For timing the expert weight streaming. */
    void* events[4];
} moe_layer_trace;

/* ---- diagnostics ------------------------------------------------------- */
const char* moe_last_error_string(void);
const char* moe_version(void);

/* ---- host-only validation (no GPU needed) ------------------------------ */

/* QuantizedOpsValidation.validateAffineDequantize + OpsValidation
 * validateDequantGemv (QuantizedOpsValidation.swift:64-110,
 * OpsValidation.swift:339-380) for one stacked projection. */
moe_status moe_validate_qproj(const moe_qproj* p);
/* MoERouter.init + MoELayer.init preconditions (MoELayer.swift:105-124,
 * 449-484). */
moe_status moe_validate_layer(const moe_layer_desc* d);
/* deriveAffineQuantBits (Sources/FFAI/Layers.swift:348-363). */
moe_status moe_derive_bits(int64_t packed_cols, int64_t scale_cols,
                           int32_t group_size, int32_t* bits_out);

/* ---- kernels ----------------------------------------------------------- */

/* Router projection logits = round(W x) [+ bias], one row per token
 * (QuantizedLinear/Linear callAsFunction, Layers.swift:201; GPT-OSS
 * GPTOSSBiasedLinear, GPTOSSText.swift:345-366). */
moe_status moe_router_logits(const void* x, int32_t x_dtype, int32_t T, int32_t hidden,
                             const void* weight, int32_t w_dtype, const void* bias,
                             int32_t n_experts, void* logits, hipStream_t stream);

/* moe_router_logits with an affine-quantised weight (QuantizedLinear,
 * Layers.swift:371-400): w is a one-expert stack [1, n_experts, hidden]
 * (w->n = n_experts, w->k = hidden, w->n_experts = 1). x, bias and logits
 * in x_dtype (f16 or bf16). */
moe_status moe_router_logits_q(const void* x, int32_t x_dtype, int32_t T, int32_t hidden,
                               const moe_qproj* w, const void* bias, int32_t n_experts,
                               void* logits, hipStream_t stream);

/* MoERouter.route on the GPU for every token row: Ops.moeRouterTopKMany
 * (Ops.swift:2589-2662) generalised to all gating modes of
 * MoELayer.swift:140-205 (expert_bias nullable). Output order: value desc,
 * index asc. Weights are f32. */
moe_status moe_router_topk(const void* logits, int32_t dtype, int32_t T, int32_t n_experts,
                           int32_t k, int32_t gating, int32_t norm_topk_prob,
                           const float* expert_bias, uint32_t* topk_idx, float* topk_weight,
                           hipStream_t stream);
/* moe_router_topk with the routing scales of moe_layer_desc (logit_scale,
 * routed_scale: 0 reads as 1.0; expert_scale nullable): the NemotronH and
 * Gemma 4 routers (NemotronHText.swift:838-868, Gemma4Text.swift:938-950). */
moe_status moe_router_topk_scaled(const void* logits, int32_t dtype, int32_t T,
                                  int32_t n_experts, int32_t k, int32_t gating,
                                  int32_t norm_topk_prob, const float* expert_bias,
                                  float logit_scale, float routed_scale,
                                  const float* expert_scale, uint32_t* topk_idx,
                                  float* topk_weight, hipStream_t stream);

/* Deterministic token->expert plan replacing the host sort of
 * MoELayer.decodeMany (MoELayer.swift:752-792): stable order (expert asc,
 * token asc, slot asc). perm[p] = t*k+s at sorted position p, inv_perm its
 * inverse, offsets the CSR start of each expert. Entries with an id >=
 * n_experts are dropped (their perm / inv_perm slots are left unwritten and
 * sum(counts) < T*k), so a bad id can never index out of bounds. */
size_t moe_dispatch_workspace_bytes(int32_t T, int32_t k, int32_t n_experts);
moe_status moe_dispatch_plan(const uint32_t* topk_idx, int32_t T, int32_t k, int32_t n_experts,
                             uint32_t* counts, uint32_t* offsets, uint32_t* perm,
                             uint32_t* inv_perm, void* workspace, size_t workspace_bytes,
                             hipStream_t stream);

/* QuantizedOps.dequantizeAffine (QuantizedOps.swift:62-221): numel values
 * of one packed stream to out_dtype. */
moe_status moe_dequantize_affine(const uint32_t* weight, const void* scales, const void* biases,
                                 int32_t sb_dtype, int32_t bits, int32_t group_size,
                                 int64_t numel, void* out, int32_t out_dtype, hipStream_t stream);

/* Expert-grouped dequant product over the rows of a dispatch plan:
 *   out[p, :] = W[e(p)] . a[row(p), :]   for every sorted position p,
 * e(p) = the expert whose CSR range [offsets[e], offsets[e+1]) holds p,
 * row(p) = perm[p] / top_k when perm is non-NULL (activation gather), else
 * p. With perm, a holds ceil(M / top_k) rows and every perm[p] < M (a plan
 * of M = T * top_k positions over T rows, as moe_dispatch_plan writes it);
 * without, a holds M rows. Replaces Ops.dequantGemvInt4ExpertIndexed(Many) (Ops.swift:2444-2587)
 * and Ops.moeGatherDequantGemmInt4 bm8/bm16/bm64/m1 (Ops.swift:4553-5201,
 * 6499-6585). Picks the HBM-streaming GEMV or the MFMA GEMM by rows per
 * expert. out and a are in a_dtype. The workspace holds the GEMM's work list
 * and, for bf16 rows, their f16 operand copy; its size depends on the
 * projection, the activation dtype and M (0 for invalid arguments). */
size_t moe_expert_matmul_workspace_bytes(const moe_qproj* p, int32_t a_dtype, int32_t M);
moe_status moe_expert_matmul(const moe_qproj* p, const void* a, int32_t a_dtype,
                             const uint32_t* perm, int32_t top_k, int32_t M,
                             const uint32_t* offsets, void* out, void* workspace,
                             size_t workspace_bytes, hipStream_t stream);

/* Ops.swiglu (Ops.swift:6411-6460) and the other moe_activation kinds,
 * elementwise over n values. MOE_ACT_RELU2 reads `up` only (gate may be
 * NULL). */
moe_status moe_activation_apply(const void* gate, const void* up, void* out, int64_t n,
                                int32_t dtype, int32_t activation, float alpha, float limit,
                                hipStream_t stream);

/* Ops.moeUnpermute (Ops.swift:5030-5110):
 *   out[t,:] = sum_s round(w[t,s]) * Y[inv_perm[t*k+s], :]. */
moe_status moe_unpermute(const void* Y, const uint32_t* inv_perm, const float* topk_weight,
                         int32_t T, int32_t hidden, int32_t k, void* out, int32_t dtype,
                         hipStream_t stream);

/* GPT-OSS's MXFP4 -> affine 4-bit transcode (transcodeStackedExperts,
 * Models/Text/GPTOSSText.swift:1040-1236), on the GPU. n_groups groups of 32
 * fp4 codes: packed [n_groups * 4] u32 (8 codes per word, low nibble first),
 * e8m0 [n_groups] exponent bytes (value = LUT[code] * 2^(e8m0 - 127)). Per
 * group: lo/hi = min/max table value, bias = lo * 2^(e-127), scale =
 * (hi - lo) * 2^(e-127) / 15, code = clamp(round((LUT[code] - lo) *
 * 2^(e-127) / scale), 0, 15) in the same nibble. Writes an mlx affine 4-bit
 * triplet with group size 32: out_weight (may equal packed), out_scales and
 * out_biases [n_groups] in sb_dtype. packed and out_weight 16-byte aligned.
 * Bit-exact with the reference's f32 arithmetic for e8m0 in 3..254; for
 * e8m0 0..2 (magnitudes below 2^-124) the reference's intermediates are
 * subnormal and the GPU flushes them (the result stays finite); e8m0 = 255
 * (2^128) is outside the format's finite range. */
moe_status moe_mxfp4_to_affine(const uint32_t* packed, const uint8_t* e8m0, int64_t n_groups,
                               uint32_t* out_weight, void* out_scales, void* out_biases,
                               int32_t sb_dtype, hipStream_t stream);

/* Ops.addAndRmsNorm (Ops.swift:676-730): per row, residual = a + b and
 * normed = residual / sqrt(mean(residual^2) + eps) * weight, each rounded to
 * dtype. [n_rows, row_size] rows (16-byte aligned), weight [row_size];
 * row_size a multiple of 8, at most 8192. */
moe_status moe_add_rmsnorm(const void* a, const void* b, const void* weight, float eps,
                           int32_t n_rows, int32_t row_size, int32_t dtype, void* residual_out,
                           void* normed_out, hipStream_t stream);

/* ---- whole layer ------------------------------------------------------- */

/* Workspace for moe_layer_forward at up to max_tokens rows. */
size_t moe_layer_workspace_bytes(const moe_layer_desc* d, int32_t max_tokens);

/* MoELayer.decode / decodeMany (MoELayer.swift:530-634,677-969) with the
 * router, plan, expert products and combine all on the device, plus the
 * optional shared expert (Qwen3xText.swift:928-1104). x [T, hidden],
 * y [T, hidden] in act_dtype. trace is nullable. */
moe_status moe_layer_forward(const moe_layer_desc* d, const void* x, int32_t T, void* y,
                             void* workspace, size_t workspace_bytes,
                             const moe_layer_trace* trace, hipStream_t stream);
/* moe_layer_forward with the router reading its own input rows router_x
 * [T, hidden] (nullable: x) while the experts read x: Gemma 4 routes on
 * rmsNorm(h, router.scale) and feeds the experts preNorm2(h)
 * (Gemma4Text.swift:932-936, 960). */
moe_status moe_layer_forward_routed(const moe_layer_desc* d, const void* x,
                                    const void* router_x, int32_t T, void* y, void* workspace,
                                    size_t workspace_bytes, const moe_layer_trace* trace,
                                    hipStream_t stream);

/* moe_layer_forward for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). No counterpart in the reference: the workspace is a static
 * device array of moe_layer_noalloc_max_bytes() bytes (16 MiB) that each GPU
 * holds for the life of the process, instead of a caller buffer; a call
 * whose workspace (moe_layer_workspace_bytes) would exceed it returns
 * MOE_ERR_WORKSPACE before any launch. Every launch stays on `stream` (no
 * side stream). All calls on one GPU share the array: calls that overlap on
 * a GPU (other streams, other host threads) race and must be serialised by
 * the caller. */
moe_status moe_layer_forward_noalloc(const moe_layer_desc* d, const void* x, int32_t T, void* y,
                                     const moe_layer_trace* trace, hipStream_t stream);
size_t moe_layer_noalloc_max_bytes(void);

/* The MoE block with the decoder steps on either side folded in: the
 * post-attention residual add + RMSNorm before it (Ops.addAndRmsNorm,
 * Qwen3xText.swift:2640-2660) and the residual add after it
 * (Ops.sigmoidScalarFMAResidual, OpsFused.swift:699-753; Qwen3xText.swift:
 * 1015-1035):
 *   r  = h + mixer_out                      (rounded; written to residual_out
 *                                            when non-NULL)
 *   xn = r / sqrt(mean(r^2) + eps) * norm_weight   (rounded)
 *   y  = r + MoE(xn) [+ sigmoid(gate) * shared(xn)]   (one rounding)
 * h, mixer_out, y [T, hidden]; norm_weight [hidden]; all in act_dtype and
 * 16-byte aligned; hidden a multiple of 8. For one token the add and norm
 * run inside the router launch. */
moe_status moe_layer_forward_residual(const moe_layer_desc* d, const void* h,
                                      const void* mixer_out, const void* norm_weight, float eps,
                                      int32_t T, void* y, void* residual_out, void* workspace,
                                      size_t workspace_bytes, const moe_layer_trace* trace,
                                      hipStream_t stream);

/* The kernels a layer call of T rows runs, per stage, for 16-byte aligned
 * activation rows. No reference counterpart: the reference picks its tile
 * kernels internally (MoELayer.swift:855-882); callers and tests use this
 * to know which kernel a configuration exercises. 0 = stage absent. */
typedef enum moe_path {
    MOE_PATH_NONE = 0,
    MOE_PATH_DECODE1 = 1,   /* one token, or a few (up to 8, while the
                               T * top_k expert slices stay within 1.35 per
                               distinct expert expected under uniform
                               routing): gate/up with in-kernel routing per
                               token, fused down + combine, no dispatch plan
                               (for the shared stages, one token only: the
                               shared expert runs inside those two
                               launches) */
    MOE_PATH_GEMV = 2,      /* HBM-streaming grouped GEMV (VALU dot2) */
    MOE_PATH_GEMV_MMA = 3,  /* batched grouped GEMV on the matrix cores */
    MOE_PATH_GEMM = 4       /* grouped GEMM on the matrix cores */
} moe_path;
typedef struct moe_layer_paths {
    int32_t gate_up, down, shared_gate_up, shared_down; /* moe_path */
} moe_layer_paths;
moe_status moe_layer_path(const moe_layer_desc* d, int32_t T, moe_layer_paths* out);

/* ---- MoELayer handle (owns its workspace like the reference instance) -- */
typedef struct moe_layer* moe_layer_t;

/* MoELayer.init (MoELayer.swift:440-498). The descriptor is copied; the
 * weight buffers it points to must outlive the handle. */
moe_status moe_layer_create(const moe_layer_desc* d, moe_layer_t* out);
void moe_layer_destroy(moe_layer_t layer);
/* MoELayer.decode (MoELayer.swift:530): one token. */
moe_status moe_layer_decode(moe_layer_t layer, const void* h, void* out, hipStream_t stream);
/* MoELayer.decodeMany (MoELayer.swift:677): T tokens. */
moe_status moe_layer_decode_many(moe_layer_t layer, const void* h, int32_t T, void* out,
                                 hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* MOE_HIP_H */
