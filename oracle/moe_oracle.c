/*
 * moe_oracle.c — CPU restatement of FFAI's MoE feed-forward layer.
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the HIP path and the timed CPU
 * baseline. The product never loads it; only tests/, smoke() and bench.py's
 * cpu_baseline leg do.
 *
 * The reference (thewafflehaus/FFAI) is Swift + Metal and cannot be built
 * here, so this file restates its semantics in plain C. Build flags keep the
 * arithmetic literal: -ffp-contract=off, no fast-math.
 *
 * What pins each part (tests/test_oracle_golden.py):
 *   conversions     IEEE special values + exhaustive f16/bf16 round trips
 *   or_expf         |or_expf(x) - exp(x)| <= 2 ulp over a dense sweep
 *   bit stream      the reference's own byte-level packers
 *                   (Tests/FFAITests/Ops/QuantizedOpsTests.swift:33-121),
 *                   dequant KAT (QuantizedOpsAffineTests.swift:124-159),
 *                   deriveAffineQuantBits cases (LayersTests.swift:79-98)
 *   router          KATs MoELayerTests.swift:36-110, QuantizedOpsTests.swift:
 *                   999-1028, brute-force full stable sort
 *   dispatch plan   brute-force sort + invariants
 *   grouped GEMM    numpy float64 matmul of the dequantised dense matrix on
 *                   the reference's generators (MoEBgemmBm64MppTests.swift:
 *                   159-271, QuantizedOpsTests.swift:126-438)
 *   activations     KATs OpsSpecialPathTests.swift:314-354; GPT-OSS closed
 *                   form at hand-picked points (clamp branches)
 *   combine         KAT OpsSpecialPathTests.swift:1080-1122
 *   whole layer     KATs MoELayerTests.swift:147-265 (scalar experts)
 */
#include "moe_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* conversions                                                              */
/* ------------------------------------------------------------------------ */

float or_bf16_to_f32(uint16_t h) {
    uint32_t x = (uint32_t)h << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* Round-to-nearest-even, the bias trick of Tensor.swift:146-150 and
 * MoELayer.swift:927-931. NaN stays NaN. */
uint16_t or_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u);
    uint32_t r = x + 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(r >> 16);
}

float or_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, x;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31) x = sign | 0x7f800000u | (m << 13);
    else x = sign | ((e + 112u) << 23) | (m << 13);
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t or_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
    if (ax < 0x38800000u) {                                    /* below 2^-14 */
        float a;
        memcpy(&a, &ax, 4);
        uint32_t m = (uint32_t)nearbyintf(a * 16777216.0f); /* units of 2^-24, RNE */
        return (uint16_t)(sign | m);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t mant = ax & 0x7fffffu;
    uint32_t h = (e << 10) | (mant >> 13);
    uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float or_round_dt(float v, int dt) {
    if (dt == OR_BF16) return or_bf16_to_f32(or_f32_to_bf16(v));
    if (dt == OR_F16) return or_f16_to_f32(or_f32_to_f16(v));
    return v;
}

void or_load(const void* src, int dt, size_t n, float* dst) {
    if (dt == OR_F32) {
        memcpy(dst, src, n * 4);
    } else if (dt == OR_F16) {
        const uint16_t* s = (const uint16_t*)src;
        for (size_t i = 0; i < n; i++) dst[i] = or_f16_to_f32(s[i]);
    } else {
        const uint16_t* s = (const uint16_t*)src;
        for (size_t i = 0; i < n; i++) dst[i] = or_bf16_to_f32(s[i]);
    }
}

void or_store(const float* src, int dt, size_t n, void* dst) {
    if (dt == OR_F32) {
        memcpy(dst, src, n * 4);
    } else if (dt == OR_F16) {
        uint16_t* d = (uint16_t*)dst;
        for (size_t i = 0; i < n; i++) d[i] = or_f32_to_f16(src[i]);
    } else {
        uint16_t* d = (uint16_t*)dst;
        for (size_t i = 0; i < n; i++) d[i] = or_f32_to_bf16(src[i]);
    }
}

static float load1(const void* p, int dt, size_t i) {
    if (dt == OR_F32) return ((const float*)p)[i];
    if (dt == OR_F16) return or_f16_to_f32(((const uint16_t*)p)[i]);
    return or_bf16_to_f32(((const uint16_t*)p)[i]);
}

/* ------------------------------------------------------------------------ */
/* deterministic exp                                                        */
/* ------------------------------------------------------------------------ */

/* Cody-Waite reduction by ln2 and Moshier's degree-5 minimax polynomial
 * (Cephes expf). Every step is an explicit fused or unfused single-precision
 * operation, so the GPU router (which evaluates the same sequence) returns
 * the identical bits. The reference calls Foundation.exp
 * (MoELayer.swift:213); the two agree to within 2 ulp. */
float or_expf(float x) {
    if (x > 88.0f) return INFINITY;
    if (x < -87.0f) return 0.0f;
    float n = rintf(x * 1.44269504088896341f);
    float r = fmaf(n, -0.693359375f, x);
    r = fmaf(n, 2.12194440e-4f, r);
    float p = 1.9875691500e-4f;
    p = fmaf(p, r, 1.3981999507e-3f);
    p = fmaf(p, r, 8.3334519073e-3f);
    p = fmaf(p, r, 4.1665795894e-2f);
    p = fmaf(p, r, 1.6666665459e-1f);
    p = fmaf(p, r, 5.0000001201e-1f);
    float r2 = r * r;
    float y = fmaf(p, r2, r) + 1.0f;
    return ldexpf(y, (int)n);
}

/* ------------------------------------------------------------------------ */
/* affine bit stream                                                        */
/* ------------------------------------------------------------------------ */

static int bits_ok(int bits) {
    return bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
}

/* Value i of a row lives at bit offset i*bits of the little-endian u32
 * stream (Layers.swift:134-143; QuantizedOpsTests.swift:33-121 packers);
 * 3/5/6-bit values straddle byte and word boundaries. */
static inline uint32_t get_code(const uint32_t* w, int bits, size_t i) {
    size_t bit = i * (size_t)bits;
    size_t word = bit >> 5;
    unsigned sh = (unsigned)(bit & 31u);
    uint64_t win = w[word];
    if (sh + (unsigned)bits > 32u) win |= (uint64_t)w[word + 1] << 32;
    return (uint32_t)(win >> sh) & ((1u << bits) - 1u);
}

int or_unpack_codes(const uint32_t* w, int bits, size_t n, uint8_t* codes) {
    if (!bits_ok(bits) || (n * (size_t)bits) % 32u) return -1;
    for (size_t i = 0; i < n; i++) codes[i] = (uint8_t)get_code(w, bits, i);
    return 0;
}

int or_pack_codes(const uint8_t* codes, int bits, size_t n, uint32_t* w) {
    if (!bits_ok(bits) || (n * (size_t)bits) % 32u) return -1;
    memset(w, 0, n * (size_t)bits / 8);
    for (size_t i = 0; i < n; i++) {
        uint64_t v = (uint64_t)(codes[i] & ((1u << bits) - 1u));
        size_t bit = i * (size_t)bits;
        size_t word = bit >> 5;
        unsigned sh = (unsigned)(bit & 31u);
        w[word] |= (uint32_t)(v << sh);
        if (sh + (unsigned)bits > 32u) w[word + 1] |= (uint32_t)(v >> (32u - sh));
    }
    return 0;
}

/* QuantizedOpsValidation.packedUInt32Count (QuantizedOpsValidation.swift:52-57) */
long or_packed_u32_count(long numel, int bits) {
    if (!bits_ok(bits)) return -1;
    long bitcount = numel * bits;
    if (bitcount % 32) return -1;
    return bitcount / 32;
}

/* deriveAffineQuantBits (Layers.swift:348-363): bits = 32*packed/(scale*gs).
 * Returns -1 where the Swift code traps. */
int or_derive_bits(long packed_cols, long scale_cols, long group_size) {
    long in_features = scale_cols * group_size;
    if (in_features <= 0) return -1;
    if ((32 * packed_cols) % in_features) return -1;
    return (int)((32 * packed_cols) / in_features);
}

/* QuantizedOps.dequantizeAffine (QuantizedOps.swift:62-221) with the
 * validator of QuantizedOpsValidation.swift:64-110: w = scale*q + bias. */
int or_dequantize_affine(const uint32_t* w, const void* scales, const void* biases,
                         int sb_dt, int bits, int group_size, size_t numel, float* out) {
    if (!bits_ok(bits) || group_size <= 0 || numel % (size_t)group_size) return -1;
    if (bits == 2 || bits == 4 || bits == 8) {
        if (group_size % (32 / bits)) return -1;
    } else if ((group_size * bits) % 32) {
        return -1;
    }
    for (size_t i = 0; i < numel; i++) {
        size_t g = i / (size_t)group_size;
        float s = load1(scales, sb_dt, g), b = load1(biases, sb_dt, g);
        float q = (float)get_code(w, bits, i);
        float sq = s * q;
        out[i] = sq + b;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* router                                                                   */
/* ------------------------------------------------------------------------ */

/* Router projection (Layers.swift:201, GPTOSSText.swift:361-365):
 * logits = round_dt(W x), then with a bias round_dt(logits + b), both in the
 * activation dtype. Dot products accumulate in double. */
void or_router_logits(const void* x, int x_dt, int T, int H,
                      const void* W, int w_dt, const void* bias, int E,
                      float* logits) {
    float* xr = (float*)malloc(sizeof(float) * (size_t)H);
    float* wr = (float*)malloc(sizeof(float) * (size_t)H * (size_t)E);
    or_load(W, w_dt, (size_t)H * (size_t)E, wr);
    for (int t = 0; t < T; t++) {
        or_load((const char*)x + (size_t)t * H * (x_dt == OR_F32 ? 4 : 2), x_dt, (size_t)H, xr);
        for (int e = 0; e < E; e++) {
            double acc = 0.0;
            const float* w = wr + (size_t)e * H;
            for (int h = 0; h < H; h++) acc += (double)w[h] * (double)xr[h];
            float l = or_round_dt((float)acc, x_dt);
            if (bias) l = or_round_dt(l + load1(bias, x_dt, (size_t)e), x_dt);
            logits[(size_t)t * E + e] = l;
        }
    }
    free(xr);
    free(wr);
}

/* Dequantised row r of a stacked projection: w = s * q + b in fp32
 * (QuantizedOps.swift:33-45), the form or_qgemm_rows multiplies. */
static void dequant_row(const or_qproj* p, size_t r, float* wrow) {
    int K = p->k, gs = p->group_size, bits = p->bits, groups = K / gs;
    const uint32_t* wr = p->weight + r * ((size_t)K * bits / 32);
    for (int g = 0; g < groups; g++) {
        float s = load1(p->scales, p->sb_dt, r * groups + g);
        float b = load1(p->biases, p->sb_dt, r * groups + g);
        for (int j = 0; j < gs; j++) {
            float q = (float)get_code(wr, bits, (size_t)g * gs + j);
            float sq = s * q;
            wrow[g * gs + j] = sq + b;
        }
    }
}

int or_router_logits_q(const void* x, int x_dt, int T, int H, const or_qproj* W,
                       const void* bias, int E, float* logits) {
    if (!W || !bits_ok(W->bits) || W->k != H || W->n != E || W->group_size <= 0 ||
        H % W->group_size || ((long)H * W->bits) % 32)
        return -1;
    float* xr = (float*)malloc(sizeof(float) * (size_t)H);
    float* wr = (float*)malloc(sizeof(float) * (size_t)H * (size_t)E);
    for (int e = 0; e < E; e++) dequant_row(W, (size_t)e, wr + (size_t)e * H);
    for (int t = 0; t < T; t++) {
        or_load((const char*)x + (size_t)t * H * (x_dt == OR_F32 ? 4 : 2), x_dt, (size_t)H, xr);
        for (int e = 0; e < E; e++) {
            double acc = 0.0;
            const float* w = wr + (size_t)e * H;
            for (int h = 0; h < H; h++) acc += (double)w[h] * (double)xr[h];
            float l = or_round_dt((float)acc, x_dt);
            if (bias) l = or_round_dt(l + load1(bias, x_dt, (size_t)e), x_dt);
            logits[(size_t)t * E + e] = l;
        }
    }
    free(xr);
    free(wr);
    return 0;
}

/* Numerically-stable softmax with the uniform fallback
 * (MoELayer.swift:210-219); the sum runs in index order. */
void or_softmax(const float* x, int n, float* out) {
    if (n <= 0) return;
    float m = x[0];
    for (int i = 1; i < n; i++) m = x[i] > m ? x[i] : m;
    float s = 0.0f;
    for (int i = 0; i < n; i++) {
        out[i] = or_expf(x[i] - m);
        s += out[i];
    }
    if (!(s > 0.0f)) {
        for (int i = 0; i < n; i++) out[i] = 1.0f / (float)n;
        return;
    }
    for (int i = 0; i < n; i++) out[i] = out[i] / s;
}

/* Heap top-k of MoELayer.swift:223-296: a k-sized min-heap ordered by
 * (value asc, index desc), drained and sorted by (value desc, index asc). */
typedef struct { float v; int i; } vi_t;

static int vi_less(vi_t a, vi_t b) { /* a is the easier evict */
    if (a.v != b.v) return a.v < b.v;
    return a.i > b.i;
}

static int vi_cmp_desc(const void* pa, const void* pb) {
    vi_t a = *(const vi_t*)pa, b = *(const vi_t*)pb;
    if (a.v != b.v) return a.v > b.v ? -1 : 1;
    return a.i < b.i ? -1 : (a.i > b.i);
}

int or_topk_indices(const float* v, int n, int k, int* out) {
    if (k <= 0 || k > n) return -1;
    vi_t* heap = (vi_t*)malloc(sizeof(vi_t) * (size_t)k);
    int cnt = 0;
    for (int i = 0; i < n; i++) {
        vi_t e = {v[i], i};
        if (cnt < k) {
            int j = cnt++;
            heap[j] = e;
            while (j > 0) {
                int p = (j - 1) >> 1;
                if (vi_less(heap[j], heap[p])) {
                    vi_t t = heap[j]; heap[j] = heap[p]; heap[p] = t;
                    j = p;
                } else {
                    break;
                }
            }
        } else if (vi_less(heap[0], e)) {
            heap[0] = e;
            int j = 0;
            for (;;) {
                int l = 2 * j + 1, r = 2 * j + 2, s = j;
                if (l < cnt && vi_less(heap[l], heap[s])) s = l;
                if (r < cnt && vi_less(heap[r], heap[s])) s = r;
                if (s == j) break;
                vi_t t = heap[j]; heap[j] = heap[s]; heap[s] = t;
                j = s;
            }
        }
    }
    qsort(heap, (size_t)cnt, sizeof(vi_t), vi_cmp_desc);
    for (int j = 0; j < k; j++) out[j] = heap[j].i;
    free(heap);
    return 0;
}

/* MoERouter.route (MoELayer.swift:140-205). GPT-OSS's router
 * (GPTOSSText.swift:1349-1361: full stable sort, top-k, softmax over the k)
 * is the topKThenSoftmax branch. */
int or_route(const float* logits, int T, int E, int k, int gating, int norm_topk,
             const float* expert_bias, uint32_t* idx, float* weights) {
    return or_route_scaled(logits, T, E, k, gating, norm_topk, expert_bias, 1.0f, 1.0f, NULL,
                           idx, weights);
}

/* NemotronH routing (NemotronHText.swift:844-867): sigmoid scores with the
 * correction bias added for the selection only, ties to the lower index, the
 * unbiased sigmoids as weights, divided by (their sum in rank order + 1e-20)
 * when norm_topk and k > 1. The sigmoid uses or_expf, the exp of the
 * softmax. */
static void route_sigmoid(const float* l, int E, int k, int norm_topk, const float* expert_bias,
                          float* raw, float* score, int* sel, float* ow) {
    for (int e = 0; e < E; e++) {
        raw[e] = 1.0f / (1.0f + or_expf(-l[e]));
        score[e] = expert_bias ? raw[e] + expert_bias[e] : raw[e];
    }
    or_topk_indices(score, E, k, sel);
    for (int j = 0; j < k; j++) ow[j] = raw[sel[j]];
    if (k > 1 && norm_topk) {
        float s = 0.0f;
        for (int j = 0; j < k; j++) s += ow[j];
        s = s + 1e-20f;
        for (int j = 0; j < k; j++) ow[j] = ow[j] / s;
    }
}

int or_route_scaled(const float* logits, int T, int E, int k, int gating, int norm_topk,
                    const float* expert_bias, float logit_scale, float routed_scale,
                    const float* expert_scale, uint32_t* idx, float* weights) {
    if (E <= 0 || k <= 0 || k > E) return -1;
    if (gating < OR_SOFTMAX_THEN_TOPK || gating > OR_SIGMOID_TOPK) return -1;
    int* sel = (int*)malloc(sizeof(int) * (size_t)k);
    float* probs = (float*)malloc(sizeof(float) * (size_t)E);
    float* score = (float*)malloc(sizeof(float) * (size_t)E);
    float* pick = (float*)malloc(sizeof(float) * (size_t)k);
    float* lrow = (float*)malloc(sizeof(float) * (size_t)E);
    for (int t = 0; t < T; t++) {
        const float* l = lrow;
        for (int e = 0; e < E; e++) lrow[e] = logits[(size_t)t * E + e] * logit_scale;
        uint32_t* oi = idx + (size_t)t * k;
        float* ow = weights + (size_t)t * k;
        if (gating == OR_SIGMOID_TOPK) {
            route_sigmoid(l, E, k, norm_topk, expert_bias, probs, score, sel, ow);
        } else if (gating == OR_TOPK_THEN_SOFTMAX ||
            (gating == OR_SOFTMAX_THEN_TOPK && norm_topk && !expert_bias)) {
            or_topk_indices(l, E, k, sel);
            for (int j = 0; j < k; j++) pick[j] = l[sel[j]];
            or_softmax(pick, k, ow);
        } else {
            or_softmax(l, E, probs);
            if (expert_bias)
                for (int e = 0; e < E; e++) probs[e] = probs[e] + expert_bias[e];
            or_topk_indices(probs, E, k, sel);
            for (int j = 0; j < k; j++) ow[j] = probs[sel[j]];
            if (norm_topk) {
                float s = 0.0f;
                for (int j = 0; j < k; j++) s += ow[j];
                if (s > 0.0f)
                    for (int j = 0; j < k; j++) ow[j] = ow[j] / s;
            }
        }
        for (int j = 0; j < k; j++) {
            oi[j] = (uint32_t)sel[j];
            ow[j] = ow[j] * routed_scale;
            if (expert_scale) ow[j] = ow[j] * expert_scale[sel[j]];
        }
    }
    free(sel);
    free(probs);
    free(score);
    free(pick);
    free(lrow);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* dispatch plan                                                            */
/* ------------------------------------------------------------------------ */

typedef struct { uint32_t e, src; } plan_t;

/* Stable merge sort by expert id. */
static void plan_sort(plan_t* a, plan_t* tmp, size_t n) {
    if (n < 2) return;
    size_t h = n / 2;
    plan_sort(a, tmp, h);
    plan_sort(a + h, tmp, n - h);
    size_t i = 0, j = h, o = 0;
    while (i < h && j < n) tmp[o++] = (a[j].e < a[i].e) ? a[j++] : a[i++];
    while (i < h) tmp[o++] = a[i++];
    while (j < n) tmp[o++] = a[j++];
    memcpy(a, tmp, n * sizeof(plan_t));
}

/* MoELayer.decodeMany's plan (MoELayer.swift:752-792): the T*k entries are
 * listed token-major, then stably sorted by expert. perm[p] is the
 * token-major entry (t*k + s) at sorted position p; inv_perm is its inverse;
 * offsets is the CSR row start of each expert. */
int or_dispatch_plan(const uint32_t* idx, int T, int k, int E,
                     uint32_t* counts, uint32_t* offsets,
                     uint32_t* perm, uint32_t* inv_perm) {
    size_t M = (size_t)T * (size_t)k;
    for (size_t m = 0; m < M; m++)
        if (idx[m] >= (uint32_t)E) return -1;
    plan_t* a = (plan_t*)malloc(sizeof(plan_t) * (M ? M : 1));
    plan_t* tmp = (plan_t*)malloc(sizeof(plan_t) * (M ? M : 1));
    for (size_t m = 0; m < M; m++) {
        a[m].e = idx[m];
        a[m].src = (uint32_t)m;
    }
    plan_sort(a, tmp, M);
    for (int e = 0; e < E; e++) counts[e] = 0;
    for (size_t p = 0; p < M; p++) {
        perm[p] = a[p].src;
        inv_perm[a[p].src] = (uint32_t)p;
        counts[a[p].e]++;
    }
    offsets[0] = 0;
    for (int e = 0; e < E; e++) offsets[e + 1] = offsets[e] + counts[e];
    free(a);
    free(tmp);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* grouped dequant GEMM                                                     */
/* ------------------------------------------------------------------------ */

/* Restates the CPU m1 oracle of MoEBgemmBm64MppTests.swift:82-114
 * generalised to every bit width: w = s*q + b in fp32, dot products in
 * double. Rows are processed expert by expert so each dequantised weight row
 * is built once. */
int or_qgemm_rows(const or_qproj* p, const float* a, int M,
                  const uint32_t* row_expert, float* out) {
    int N = p->n, K = p->k, gs = p->group_size, bits = p->bits;
    if (!bits_ok(bits) || gs <= 0 || K % gs || (K * bits) % 32 || M < 0) return -1;
    int E = 0;
    for (int m = 0; m < M; m++)
        if ((int)row_expert[m] + 1 > E) E = (int)row_expert[m] + 1;
    int* cnt = (int*)calloc((size_t)E + 1, sizeof(int));
    int* start = (int*)calloc((size_t)E + 1, sizeof(int));
    int* rows = (int*)malloc(sizeof(int) * ((size_t)M + 1));
    for (int m = 0; m < M; m++) cnt[row_expert[m]]++;
    for (int e = 0; e < E; e++) start[e + 1] = start[e] + cnt[e];
    for (int e = 0; e < E; e++) cnt[e] = 0;
    for (int m = 0; m < M; m++) rows[start[row_expert[m]] + cnt[row_expert[m]]++] = m;
    float* wrow = (float*)malloc(sizeof(float) * (size_t)K);
    for (int e = 0; e < E; e++) {
        if (start[e + 1] == start[e]) continue;
        for (int n = 0; n < N; n++) {
            dequant_row(p, (size_t)e * N + n, wrow);
            for (int i = start[e]; i < start[e + 1]; i++) {
                int m = rows[i];
                const float* x = a + (size_t)m * K;
                double acc0 = 0.0, acc1 = 0.0, acc2 = 0.0, acc3 = 0.0;
                int kk = 0;
                for (; kk + 4 <= K; kk += 4) {
                    acc0 += (double)wrow[kk] * (double)x[kk];
                    acc1 += (double)wrow[kk + 1] * (double)x[kk + 1];
                    acc2 += (double)wrow[kk + 2] * (double)x[kk + 2];
                    acc3 += (double)wrow[kk + 3] * (double)x[kk + 3];
                }
                for (; kk < K; kk++) acc0 += (double)wrow[kk] * (double)x[kk];
                out[(size_t)m * N + n] = (float)((acc0 + acc1) + (acc2 + acc3));
            }
        }
    }
    free(cnt);
    free(start);
    free(rows);
    free(wrow);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* activations and combine                                                  */
/* ------------------------------------------------------------------------ */

/* 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))), the form the
 * reference's GELU test states (OpsTests.swift:262-267). */
float or_gelu(float g) {
    const float c = 0.7978845608028654f; /* sqrt(2/pi) */
    float inner = c * (g + 0.044715f * g * g * g);
    return 0.5f * g * (1.0f + tanhf(inner));
}

float or_act(float g, float u, int act, float alpha, float limit) {
    return or_act_dt(g, u, act, alpha, limit, OR_F32);
}

/* SwiGLU silu(g)*u in fp32 (Ops.swift:6400-6411); GPT-OSS clamped
 * alpha-swish with the upper-only gate clamp (GPTOSSText.swift:1415-1431);
 * GEGLU with the GELU stored in dt before the product (Gemma4Text.swift:
 * 965); squared ReLU relu(u) * relu(u) (NemotronHText.swift:759-760). */
float or_act_dt(float g, float u, int act, float alpha, float limit, int dt) {
    if (act == OR_ACT_GEGLU) return or_round_dt(or_gelu(g), dt) * u;
    if (act == OR_ACT_RELU2) {
        float r = u > 0.0f ? u : 0.0f;
        return r * r;
    }
    if (act == OR_ACT_GPTOSS) {
        if (g > limit) g = limit;
        if (u > limit) u = limit;
        if (u < -limit) u = -limit;
        float ag = alpha * g;
        float glu = g / (1.0f + expf(-ag));
        return glu * (u + 1.0f);
    }
    float silu = g / (1.0f + expf(-g));
    return silu * u;
}

/* mt_moe_unpermute (Ops.swift:5030-5110) with the combine weights rounded to
 * the activation dtype first (MoELayer.swift:921-935); fp32 accumulation in
 * slot order, one rounding at the store. */
void or_unpermute(const float* Y, const uint32_t* inv_perm, const float* w,
                  int T, int H, int k, int dt, float* out) {
    for (int t = 0; t < T; t++) {
        for (int h = 0; h < H; h++) {
            float acc = 0.0f;
            for (int s = 0; s < k; s++) {
                float ws = or_round_dt(w[(size_t)t * k + s], dt);
                float prod = ws * Y[(size_t)inv_perm[(size_t)t * k + s] * H + h];
                acc = acc + prod;
            }
            out[(size_t)t * H + h] = or_round_dt(acc, dt);
        }
    }
}

/* ------------------------------------------------------------------------ */
/* whole layer                                                              */
/* ------------------------------------------------------------------------ */

/* Rounds a [M, N] projection output to dt and applies the optional
 * per-expert projection bias (GPTOSSText.swift:1403-1410,1439-1441:
 * round(round(Wx) + b)). */
static void finish_proj(const or_qproj* p, float* v, int M, const uint32_t* row_expert, int dt) {
    int N = p->n;
    for (int m = 0; m < M; m++) {
        for (int n = 0; n < N; n++) {
            float r = or_round_dt(v[(size_t)m * N + n], dt);
            if (p->out_bias) {
                float b = load1(p->out_bias, dt, (size_t)row_expert[m] * N + n);
                r = or_round_dt(r + b, dt);
            }
            v[(size_t)m * N + n] = r;
        }
    }
}

int or_moe_layer(const or_layer* L, const void* x, int T, void* y,
                 const float* given_logits,
                 float* logits_out, uint32_t* idx_out, float* w_out) {
    return or_moe_layer_routed(L, x, x, T, y, given_logits, logits_out, idx_out, w_out);
}

/* The gate/up pair (or the single up projection of squared-ReLU experts)
 * and the activation, rounded to dt, into g [M, I]. */
static void expert_act(const or_layer* L, const or_qproj* gate, const or_qproj* up,
                       const float* a, int M, const uint32_t* rexp, float* g) {
    const int I = up->n, dt = L->act_dt;
    float* u = (float*)malloc(sizeof(float) * (size_t)M * I);
    or_qgemm_rows(up, a, M, rexp, u);
    finish_proj(up, u, M, rexp, dt);
    if (L->activation == OR_ACT_RELU2) {
        memset(g, 0, sizeof(float) * (size_t)M * I);
    } else {
        or_qgemm_rows(gate, a, M, rexp, g);
        finish_proj(gate, g, M, rexp, dt);
    }
    for (size_t i = 0; i < (size_t)M * I; i++)
        g[i] = or_round_dt(or_act_dt(g[i], u[i], L->activation, L->alpha, L->limit, dt), dt);
    free(u);
}

/* Ops.addAndRmsNorm (Ops.swift:676-730; the reference's CPU check in
 * OpsTests.swift:1009-1060): r = round(a + b), ssq summed in row order,
 * xn = round(r / sqrt(ssq / n + eps) * w). */
void or_add_rmsnorm(const float* a, const float* b, const float* w, float eps, int T, int H,
                    int dt, float* res_out, float* xn_out) {
    for (int t = 0; t < T; t++) {
        const float* ar = a + (size_t)t * H;
        const float* br = b + (size_t)t * H;
        float* rr = res_out + (size_t)t * H;
        float ssq = 0.0f;
        for (int i = 0; i < H; i++) {
            rr[i] = or_round_dt(ar[i] + br[i], dt);
            ssq += rr[i] * rr[i];
        }
        float rms = sqrtf(ssq / (float)H + eps);
        for (int i = 0; i < H; i++)
            xn_out[(size_t)t * H + i] = or_round_dt(rr[i] / rms * w[i], dt);
    }
}

/* out[i] = round((residual[i] + base[i]) + gate * value[i]): Ops.
 * sigmoidScalarFMAResidual (OpsFused.swift:699-753) with gate = sigmoid of
 * the shared-expert gate logit; a NULL residual is Ops.sigmoidScalarFMA, a
 * NULL value the residual add alone. */
void or_residual_combine(const float* res, const float* base, const float* value, float gate,
                         int n, int dt, float* out) {
    for (int i = 0; i < n; i++) {
        float v = base[i];
        if (res) v = res[i] + v;
        if (value) v = v + gate * value[i];
        out[i] = or_round_dt(v, dt);
    }
}

static int layer_impl(const or_layer* L, const void* x, const void* router_x, int T, void* y,
                      const float* given_logits, float* logits_out, uint32_t* idx_out,
                      float* w_out, const float* res);

int or_moe_layer_routed(const or_layer* L, const void* x, const void* router_x, int T,
                        void* y, const float* given_logits,
                        float* logits_out, uint32_t* idx_out, float* w_out) {
    return layer_impl(L, x, router_x, T, y, given_logits, logits_out, idx_out, w_out, NULL);
}

/* The block between the decoder steps (Qwen3xText.swift:2640-2670,
 * 1015-1035): r = round(h + m), xn = rmsnorm(r) * nw, y = round(r + MoE(xn)
 * [+ gate * shared(xn)]). xn_out and res_out (nullable) receive the rows. */
int or_moe_layer_residual(const or_layer* L, const void* h, const void* m, const float* nw,
                          float eps, int T, void* y, const float* given_logits,
                          float* xn_out, float* res_out, float* logits_out, uint32_t* idx_out,
                          float* w_out) {
    int H = L->hidden, dt = L->act_dt;
    if (T <= 0 || H <= 0) return -1;
    size_t n = (size_t)T * H;
    float* hf = (float*)malloc(sizeof(float) * n);
    float* mf = (float*)malloc(sizeof(float) * n);
    float* r = (float*)malloc(sizeof(float) * n);
    float* xn = (float*)malloc(sizeof(float) * n);
    void* xs = malloc(n * (dt == OR_F32 ? 4 : 2));
    or_load(h, dt, n, hf);
    or_load(m, dt, n, mf);
    or_add_rmsnorm(hf, mf, nw, eps, T, H, dt, r, xn);
    or_store(xn, dt, n, xs);
    int rc = layer_impl(L, xs, xs, T, y, given_logits, logits_out, idx_out, w_out, r);
    if (xn_out) memcpy(xn_out, xn, sizeof(float) * n);
    if (res_out) memcpy(res_out, r, sizeof(float) * n);
    free(hf); free(mf); free(r); free(xn); free(xs);
    return rc;
}

static int layer_impl(const or_layer* L, const void* x, const void* router_x, int T, void* y,
                      const float* given_logits, float* logits_out, uint32_t* idx_out,
                      float* w_out, const float* res) {
    int H = L->hidden, E = L->n_experts, k = L->top_k, I = L->intermediate, dt = L->act_dt;
    if (T <= 0 || H <= 0 || E <= 0 || k <= 0 || k > E || I <= 0) return -1;
    size_t M = (size_t)T * k;
    float* xf = (float*)malloc(sizeof(float) * (size_t)T * H);
    or_load(x, dt, (size_t)T * H, xf);

    /* 1. router projection */
    float* logits = (float*)malloc(sizeof(float) * (size_t)T * E);
    if (given_logits) memcpy(logits, given_logits, sizeof(float) * (size_t)T * E);
    else if (L->router_q.weight)
        or_router_logits_q(router_x, dt, T, H, &L->router_q, L->router_bias, E, logits);
    else or_router_logits(router_x, dt, T, H, L->router_weight, L->router_dt, L->router_bias, E,
                          logits);

    /* 2. routing */
    uint32_t* idx = (uint32_t*)malloc(sizeof(uint32_t) * M);
    float* w = (float*)malloc(sizeof(float) * M);
    or_route_scaled(logits, T, E, k, L->gating, L->norm_topk, L->expert_bias,
                    L->logit_scale == 0.0f ? 1.0f : L->logit_scale,
                    L->routed_scale == 0.0f ? 1.0f : L->routed_scale, L->expert_scale, idx, w);

    /* 3. plan */
    uint32_t* counts = (uint32_t*)malloc(sizeof(uint32_t) * (size_t)E);
    uint32_t* offsets = (uint32_t*)malloc(sizeof(uint32_t) * ((size_t)E + 1));
    uint32_t* perm = (uint32_t*)malloc(sizeof(uint32_t) * M);
    uint32_t* inv = (uint32_t*)malloc(sizeof(uint32_t) * M);
    or_dispatch_plan(idx, T, k, E, counts, offsets, perm, inv);

    /* 4. gather + gate/up + activation (MoELayer.swift:843-893) */
    uint32_t* rexp = (uint32_t*)malloc(sizeof(uint32_t) * M);
    float* a = (float*)malloc(sizeof(float) * M * H);
    for (size_t p = 0; p < M; p++) {
        rexp[p] = idx[perm[p]];
        memcpy(a + p * H, xf + (size_t)(perm[p] / k) * H, sizeof(float) * (size_t)H);
    }
    float* g = (float*)malloc(sizeof(float) * M * I);
    expert_act(L, &L->gate, &L->up, a, (int)M, rexp, g);

    /* 5. down projection (MoELayer.swift:899-902) */
    float* Y = (float*)malloc(sizeof(float) * M * H);
    or_qgemm_rows(&L->down, g, (int)M, rexp, Y);
    finish_proj(&L->down, Y, (int)M, rexp, dt);

    /* 6. weighted combine (MoELayer.swift:936-939) */
    float* out = (float*)malloc(sizeof(float) * (size_t)T * H);
    or_unpermute(Y, inv, w, T, H, k, dt, out);

    /* 7. shared expert: Granite-style unconditional add (MoELayer.swift:
     * 620-624), Qwen3.5's sigmoid gate (Qwen3xText.swift:1047-1104), or
     * NemotronH's squared-ReLU expert (NemotronHText.swift:855-862); the
     * shared expert uses the routed experts' activation. The decoder
     * residual, when given, joins the same final rounding. */
    if (res && !L->has_shared)
        for (int t = 0; t < T; t++)
            or_residual_combine(res + (size_t)t * H, out + (size_t)t * H, NULL, 0.0f, H, dt,
                                out + (size_t)t * H);
    if (L->has_shared) {
        int SI = L->shared_up.n;
        uint32_t* zero = (uint32_t*)calloc((size_t)T, sizeof(uint32_t));
        float* sg = (float*)malloc(sizeof(float) * (size_t)T * SI);
        float* so = (float*)malloc(sizeof(float) * (size_t)T * H);
        expert_act(L, &L->shared_gate, &L->shared_up, xf, T, zero, sg);
        or_qgemm_rows(&L->shared_down, sg, T, zero, so);
        finish_proj(&L->shared_down, so, T, zero, dt);
        float* gl = NULL;
        if (L->shared_gate_q.weight) {
            gl = (float*)malloc(sizeof(float) * (size_t)T);
            or_router_logits_q(x, dt, T, H, &L->shared_gate_q, NULL, 1, gl);
        } else if (L->shared_gate_weight) {
            gl = (float*)malloc(sizeof(float) * (size_t)T);
            or_router_logits(x, dt, T, H, L->shared_gate_weight, L->router_dt, NULL, 1, gl);
        }
        for (int t = 0; t < T; t++) {
            float gate = 1.0f;
            if (gl) gate = 1.0f / (1.0f + expf(-gl[t]));
            or_residual_combine(res ? res + (size_t)t * H : NULL, out + (size_t)t * H,
                                so + (size_t)t * H, gate, H, dt, out + (size_t)t * H);
        }
        free(zero); free(sg); free(so); free(gl);
    }
    or_store(out, dt, (size_t)T * H, y);

    if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)T * E);
    if (idx_out) memcpy(idx_out, idx, sizeof(uint32_t) * M);
    if (w_out) memcpy(w_out, w, sizeof(float) * M);
    free(xf); free(logits); free(idx); free(w); free(counts); free(offsets);
    free(perm); free(inv); free(rexp); free(a); free(g); free(Y); free(out);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* MXFP4 -> affine 4-bit (GPTOSSText.swift:1040-1236)                       */
/* ------------------------------------------------------------------------ */

/* The mlx-lm gpt_oss MXFP4 table (GPTOSSText.swift:947-954). */
static const float kMxfp4Lut[16] = {+0.0f, +0.5f, +1.0f, +1.5f, +2.0f, +3.0f, +4.0f, +6.0f,
                                    -0.0f, -0.5f, -1.0f, -1.5f, -2.0f, -3.0f, -4.0f, -6.0f};

float or_mxfp4_value(int code) { return kMxfp4Lut[code & 15]; }

/* Per 32-code group, the reference's two passes: min / max of the table
 * values in byte order (low nibble first), bias = lo * 2^(e - 127),
 * scale = (hi - lo) * mx / 15 (0 when flat), q = clamp(round((v - lo) *
 * (mx * (1 / scale))), 0, 15) into the same nibble; scale and bias stored in
 * sb_dt. packed/out_w hold groups * 4 words, e8m0 one byte per group. */
void or_mxfp4_to_affine(const uint32_t* packed, const uint8_t* e8m0, long groups,
                        uint32_t* out_w, void* out_s, void* out_b, int sb_dt) {
    for (long g = 0; g < groups; g++) {
        const uint8_t* bytes = (const uint8_t*)(packed + 4 * g);
        float mx = (float)exp2((double)((int)e8m0[g] - 127));
        float lo = 1e30f, hi = -1e30f;
        for (int b = 0; b < 16; b++) {
            float v0 = kMxfp4Lut[bytes[b] & 0x0F];
            float v1 = kMxfp4Lut[bytes[b] >> 4];
            if (v0 < lo) lo = v0;
            if (v0 > hi) hi = v0;
            if (v1 < lo) lo = v1;
            if (v1 > hi) hi = v1;
        }
        float bias = lo * mx;
        float span = (hi - lo) * mx;
        float scale = span > 0 ? span / 15.0f : 0;
        float inv = scale > 0 ? 1.0f / scale : 0;
        float cs = mx * inv;
        uint8_t* ob = (uint8_t*)(out_w + 4 * g);
        uint8_t src[16];
        memcpy(src, bytes, 16); /* out_w may alias packed */
        for (int b = 0; b < 16; b++) {
            long q0 = lroundf((kMxfp4Lut[src[b] & 0x0F] - lo) * cs);
            long q1 = lroundf((kMxfp4Lut[src[b] >> 4] - lo) * cs);
            if (q0 < 0) q0 = 0;
            if (q0 > 15) q0 = 15;
            if (q1 < 0) q1 = 0;
            if (q1 > 15) q1 = 15;
            ob[b] = (uint8_t)(q0 | (q1 << 4));
        }
        float sv = scale, bv = bias;
        or_store(&sv, sb_dt, 1, (char*)out_s + (size_t)g * (sb_dt == OR_F32 ? 4 : 2));
        or_store(&bv, sb_dt, 1, (char*)out_b + (size_t)g * (sb_dt == OR_F32 ? 4 : 2));
    }
}

