/* CPU oracle of the vision encoder and its mergers -- TEST INFRASTRUCTURE ONLY.
 *
 * Restates the reference's Qwen3-VL vision tower as its engine evaluates it
 * (Sources/Engine/Engine.swift:189-246 grid tables, 317-473 schedule; Shaders.swift:59-454
 * kernels), following tools/reference/qwen3vl_ref.py:25-85 and 165-216 for the math.  The
 * engine rounds to fp16 where it stores half tensors, and so does this file:
 *  - patches (Shaders.swift:84-111);
 *  - LayerNorm outputs (116-199);
 *  - q / k after 2D RoPE and v (207-290);
 *  - softmax probabilities and the attention output (294-395);
 *  - GELU outputs of fc1 (398-447).
 * Everything else is float32.  Dot products of fp16 operands accumulate their exact float
 * products in double and are rounded once to float32.  Reductions run in index order by one
 * thread, so results do not depend on the OpenMP thread count. */
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define VH OR_VH
#define VFF OR_VFF
#define VNH OR_VNH
#define VHD OR_VHD
#define VQKV OR_VQKV
#define VPATCH OR_VPATCH
#define MH OR_MH

/* Tensor-table slots of the vision tensors (Sources/Engine/ModelFile.swift:64-87). */
enum {
    T_PATCH_W = 0,
    T_PATCH_B = 1,
    T_POS = 2,
    T_VIT_BASE = 3,
    T_VIT_PER = 12,
    T_MERGER_BASE = T_VIT_BASE + OR_VLAYERS * T_VIT_PER,
    T_MERGER_PER = 6,
    T_COUNT_ALL = 710
};

static float g_h2f[65536];
static int g_lut_ready = 0;
static void lut_init(void) {
    if (g_lut_ready) return;
    for (int i = 0; i < 65536; ++i) g_h2f[i] = or_h2f((uint16_t)i);
    g_lut_ready = 1;
}

/* k_vit_patchify_rgb (Shaders.swift:84-111): patch p in 2x2 merge-block order, element
 * i = c * 256 + dy * 16 + dx, value fp16(u8 * (2 / 255) - 1) in float32 (qwen3vl_ref.py:25-38). */
void or_vit_patchify(const uint8_t* rgb, int gh, int gw, uint16_t* out) {
    const int np = gh * gw, merge_w = gw / 2, img_w = gw * 16;
    for (int p = 0; p < np; ++p) {
        const int blk = p / 4, in = p % 4;
        const int pr = (blk / merge_w) * 2 + in / 2, pc = (blk % merge_w) * 2 + in % 2;
        for (int i = 0; i < VPATCH; ++i) {
            const int c = i / 256, dy = (i % 256) / 16, dx = i % 16;
            const uint8_t v = rgb[((size_t)(pr * 16 + dy) * img_w + pc * 16 + dx) * 3 + c];
            const float a = (float)v * (2.0f / 255.0f);
            out[(size_t)p * VPATCH + i] = or_f2h(a - 1.0f);
        }
    }
}

/* prepareVisionGrid (Engine.swift:189-246): bilinear interpolation, align_corners, of the
 * 48 x 48 position table, in merge-block order, float32 in the engine's operation order. */
void or_vit_pos_interp(const float* table, int gh, int gw, float* out) {
    const int side = OR_VPOS, mw = gw / 2;
    const int np = gh * gw;
    for (int p = 0; p < np; ++p) {
        const int blk = p / 4, in = p % 4;
        const int r = (blk / mw) * 2 + in / 2, c = (blk % mw) * 2 + in % 2;
        const float y = (float)r * (float)(side - 1) / (float)(gh - 1 > 1 ? gh - 1 : 1);
        const float x = (float)c * (float)(side - 1) / (float)(gw - 1 > 1 ? gw - 1 : 1);
        const int y0 = (int)floorf(y), x0 = (int)floorf(x);
        const int y1 = y0 + 1 < side - 1 ? y0 + 1 : side - 1, x1 = x0 + 1 < side - 1 ? x0 + 1 : side - 1;
        const float dy = y - (float)y0, dx = x - (float)x0;
        const float w00 = (1.0f - dy) * (1.0f - dx), w01 = (1.0f - dy) * dx;
        const float w10 = dy * (1.0f - dx), w11 = dy * dx;
        const float* p00 = table + (size_t)(y0 * side + x0) * VH;
        const float* p01 = table + (size_t)(y0 * side + x1) * VH;
        const float* p10 = table + (size_t)(y1 * side + x0) * VH;
        const float* p11 = table + (size_t)(y1 * side + x1) * VH;
        float* d = out + (size_t)p * VH;
        for (int k = 0; k < VH; ++k) {
            float s = w00 * p00[k];
            s = s + w01 * p01[k];
            s = s + w10 * p10[k];
            s = s + w11 * p11[k];
            d[k] = s;
        }
    }
}

/* 2D vision RoPE table (Engine.swift:200-238; qwen3vl_ref.py:71-84): out[p][j] = (cos, sin) of
 * row * f_j for j < 16 and col * f_(j-16) for j >= 16, f_i = fl32(1 / 10000^(2i / 32)); the angle
 * is the float32 product, evaluated in double. */
void or_vit_rope_table(int gh, int gw, float* out) {
    float invf[16];
    for (int i = 0; i < 16; ++i) invf[i] = (float)(1.0 / pow(10000.0, (double)(2 * i) / 32.0));
    const int np = gh * gw, mw = gw / 2;
    for (int p = 0; p < np; ++p) {
        const int blk = p / 4, in = p % 4;
        const int r = (blk / mw) * 2 + in / 2, c = (blk % mw) * 2 + in % 2;
        float* d = out + (size_t)p * 64;
        for (int i = 0; i < 16; ++i) {
            const double ah = (double)((float)r * invf[i]), aw = (double)((float)c * invf[i]);
            d[2 * i] = (float)cos(ah);
            d[2 * i + 1] = (float)sin(ah);
            d[2 * (16 + i)] = (float)cos(aw);
            d[2 * (16 + i) + 1] = (float)sin(aw);
        }
    }
}

/* LayerNorm (eps 1e-6) of `rows` rows of n floats, fp16 output (Shaders.swift:116-199;
 * qwen3vl_ref.py:142-146): mean and variance in double, ((x - mean) * rstd) * w + b. */
void or_layernorm_f16(const float* x, const float* w, const float* b, int rows, int n, uint16_t* out) {
#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; ++r) {
        const float* xr = x + (size_t)r * n;
        double s = 0;
        for (int k = 0; k < n; ++k) s += xr[k];
        const double mean = s / n;
        double v = 0;
        for (int k = 0; k < n; ++k) v += (xr[k] - mean) * (xr[k] - mean);
        const double rstd = 1.0 / sqrt(v / n + 1e-6);
        for (int k = 0; k < n; ++k) out[(size_t)r * n + k] = or_f2h((float)((xr[k] - mean) * rstd * w[k] + b[k]));
    }
}

/* y[m][n] = sum_k X[m][k] * W[n][k] + bias[n]: fp16 operands, exact products summed in double,
 * one rounding to float32 (the k_vit_gemm_T product, Shaders.swift:398-447). */
void or_linear_f16(const uint16_t* X, const uint16_t* W, const float* bias, int M, int N, int K, float* y) {
    lut_init();
    float* xf = (float*)malloc(sizeof(float) * (size_t)M * K);
    for (size_t i = 0; i < (size_t)M * K; ++i) xf[i] = g_h2f[X[i]];
#pragma omp parallel
    {
        float* wr = (float*)malloc(sizeof(float) * (size_t)K);
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            for (int k = 0; k < K; ++k) wr[k] = g_h2f[W[(size_t)n * K + k]];
            for (int m = 0; m < M; ++m) {
                const float* xr = xf + (size_t)m * K;
                double acc = 0;
                for (int k = 0; k < K; ++k) acc += (double)(xr[k] * wr[k]);
                y[(size_t)m * N + n] = (float)(acc + bias[n]);
            }
        }
        free(wr);
    }
    free(xf);
}

/* gelu_tanh and gelu_exact (Shaders.swift:59-78; qwen3vl_ref.py:158-163), in double. */
float or_gelu_tanh(float x) {
    const double xd = x;
    return (float)(0.5 * xd * (1.0 + tanh(0.7978845608028654 * (xd + 0.044715 * xd * xd * xd))));
}
float or_gelu_erf(float x) {
    const double xd = x;
    return (float)(0.5 * xd * (1.0 + erf(xd * 0.7071067811865475)));
}

/* Bidirectional attention of one image (k_vit_attn, Shaders.swift:294-395; qwen3vl_ref.py:
 * 186-193).  q, k, v fp16 head-major [VNH][np][VHD]; out fp16 [np][VH].  Scores are float32,
 * scaled by 1/8; the softmax is float32 and its probabilities are rounded to fp16 before the
 * product with V. */
void or_vit_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int np, uint16_t* out) {
    lut_init();
#pragma omp parallel
    {
        float* s = (float*)malloc(sizeof(float) * (size_t)np);
        float* pr = (float*)malloc(sizeof(float) * (size_t)np);
#pragma omp for schedule(static) collapse(2)
        for (int h = 0; h < VNH; ++h)
            for (int t = 0; t < np; ++t) {
                const uint16_t* qr = q + ((size_t)h * np + t) * VHD;
                float mx = -INFINITY;
                for (int j = 0; j < np; ++j) {
                    const uint16_t* kr = k + ((size_t)h * np + j) * VHD;
                    double acc = 0;
                    for (int d = 0; d < VHD; ++d) acc += (double)(g_h2f[qr[d]] * g_h2f[kr[d]]);
                    s[j] = (float)acc * 0.125f;
                    if (s[j] > mx) mx = s[j];
                }
                double sum = 0;
                for (int j = 0; j < np; ++j) {
                    pr[j] = (float)exp((double)(s[j] - mx));
                    sum += pr[j];
                }
                const float inv = (float)(1.0 / sum);
                for (int j = 0; j < np; ++j) pr[j] = g_h2f[or_f2h(pr[j] * inv)];
                for (int d = 0; d < VHD; ++d) {
                    double acc = 0;
                    for (int j = 0; j < np; ++j) acc += (double)(pr[j] * g_h2f[v[((size_t)h * np + j) * VHD + d]]);
                    out[(size_t)t * VH + h * VHD + d] = or_f2h((float)acc);
                }
            }
        free(s);
        free(pr);
    }
}

typedef struct {
    const float *n1w, *n1b, *qkvb, *projb, *n2w, *n2b, *fc1b, *fc2b;
    const uint16_t *qkvw, *projw, *fc1w, *fc2w;
} vit_layer;
typedef struct {
    const float *nw, *nb, *fc1b, *fc2b;
    const uint16_t *fc1w, *fc2w;
} merger_w;

static const char* g_vis_err = "";
const char* or_vision_error(void) { return g_vis_err; }

/* Merger (Shaders.swift:398-454 k_merger_fc1 / k_merger_fc2; qwen3vl_ref.py:200-216): fp16 rows
 * xn [nvis][4096] -> fc1 + GELU (erf) in fp16 -> fc2 + bias, float32 out [nvis][2048]. */
static void merger_mlp(const merger_w* mw, const uint16_t* xn, int nvis, float* out) {
    float* t = (float*)malloc(sizeof(float) * (size_t)nvis * MH);
    uint16_t* h = (uint16_t*)malloc(2 * (size_t)nvis * MH);
    or_linear_f16(xn, mw->fc1w, mw->fc1b, nvis, MH, MH, t);
    for (size_t i = 0; i < (size_t)nvis * MH; ++i) h[i] = or_f2h(or_gelu_erf(t[i]));
    or_linear_f16(h, mw->fc2w, mw->fc2b, nvis, OR_H, MH, out);
    free(t);
    free(h);
}

/* One pre-norm block (Engine.swift:352-414; qwen3vl_ref.py:178-197) on the float32 residual x
 * [np][1024] in place; work buffers as sized in or_vision. */
static void vit_block(const vit_layer* W, float* x, const float* rope, int np, uint16_t* xn, float* qkv,
                      uint16_t* qh, uint16_t* att, float* t, uint16_t* hb) {
    or_layernorm_f16(x, W->n1w, W->n1b, np, VH, xn);
    or_linear_f16(xn, W->qkvw, W->qkvb, np, VQKV, VH, qkv);
    /* q and k heads rotate pairs (d, d + 32) by the patch's angle d (k_vit_qkv epilogue,
     * Shaders.swift:262-289); fp16 head-major q, k, v. */
    for (int p = 0; p < np; ++p)
        for (int hh = 0; hh < 3 * VNH; ++hh) {
            const float* src = qkv + (size_t)p * VQKV + hh * VHD;
            uint16_t* dst = qh + ((size_t)hh * np + p) * VHD;
            for (int j = 0; j < 32; ++j) {
                float a = src[j], b = src[j + 32];
                if (hh < 2 * VNH) {
                    const float c = rope[(size_t)p * 64 + 2 * j], s = rope[(size_t)p * 64 + 2 * j + 1];
                    const float a2 = a * c - b * s, b2 = b * c + a * s;
                    a = a2;
                    b = b2;
                }
                dst[j] = or_f2h(a);
                dst[j + 32] = or_f2h(b);
            }
        }
    or_vit_attention(qh, qh + (size_t)VNH * np * VHD, qh + (size_t)2 * VNH * np * VHD, np, att);
    or_linear_f16(att, W->projw, W->projb, np, VH, VH, t);
    for (size_t i = 0; i < (size_t)np * VH; ++i) x[i] = x[i] + t[i];
    or_layernorm_f16(x, W->n2w, W->n2b, np, VH, xn);
    or_linear_f16(xn, W->fc1w, W->fc1b, np, VFF, VH, t);
    for (size_t i = 0; i < (size_t)np * VFF; ++i) hb[i] = or_f2h(or_gelu_tanh(t[i]));
    or_linear_f16(hb, W->fc2w, W->fc2b, np, VH, VFF, t);
    for (size_t i = 0; i < (size_t)np * VH; ++i) x[i] = x[i] + t[i];
}

/* Vision tensors of an .icua image (ModelFile.swift:64-87); -1 with the error set if one is
 * missing or mis-sized. */
static int parse_vision(const uint8_t* img, size_t len, const uint16_t** patch_w, const float** patch_b,
                        const float** pos, vit_layer* L, merger_w* Mg) {
    const uint64_t* tab = (const uint64_t*)(img + 16);
    if (len < 16384 || ((const uint32_t*)img)[3] != T_COUNT_ALL) {
        g_vis_err = "bad header";
        return -1;
    }
#define TP(id, want)                                                                  \
    ((tab[2 * (id) + 1] == (uint64_t)(want) && tab[2 * (id)] + (want) <= len) ? (const void*)(img + tab[2 * (id)]) \
                                                                            : NULL)
    *patch_w = (const uint16_t*)TP(T_PATCH_W, (size_t)VH * VPATCH * 2);
    *patch_b = (const float*)TP(T_PATCH_B, VH * 4);
    *pos = (const float*)TP(T_POS, (size_t)OR_VPOS * OR_VPOS * VH * 4);
    if (!*patch_w || !*patch_b || !*pos) {
        g_vis_err = "image has no vision tensors";
        return -1;
    }
    for (int l = 0; l < OR_VLAYERS; ++l) {
        const int b = T_VIT_BASE + l * T_VIT_PER;
        L[l].n1w = (const float*)TP(b + 0, VH * 4);
        L[l].n1b = (const float*)TP(b + 1, VH * 4);
        L[l].qkvw = (const uint16_t*)TP(b + 2, (size_t)VQKV * VH * 2);
        L[l].qkvb = (const float*)TP(b + 3, VQKV * 4);
        L[l].projw = (const uint16_t*)TP(b + 4, (size_t)VH * VH * 2);
        L[l].projb = (const float*)TP(b + 5, VH * 4);
        L[l].n2w = (const float*)TP(b + 6, VH * 4);
        L[l].n2b = (const float*)TP(b + 7, VH * 4);
        L[l].fc1w = (const uint16_t*)TP(b + 8, (size_t)VFF * VH * 2);
        L[l].fc1b = (const float*)TP(b + 9, VFF * 4);
        L[l].fc2w = (const uint16_t*)TP(b + 10, (size_t)VH * VFF * 2);
        L[l].fc2b = (const float*)TP(b + 11, VH * 4);
        if (!L[l].n1w || !L[l].n1b || !L[l].qkvw || !L[l].qkvb || !L[l].projw || !L[l].projb || !L[l].n2w ||
            !L[l].n2b || !L[l].fc1w || !L[l].fc1b || !L[l].fc2w || !L[l].fc2b) {
            g_vis_err = "vision block tensor missing or mis-sized";
            return -1;
        }
    }
    for (int d = 0; d < 4; ++d) {
        const int b = T_MERGER_BASE + d * T_MERGER_PER;
        const int nn = d < 3 ? MH : VH;  // DeepStack mergers normalise 4096 columns, the final one 1024
        Mg[d].nw = (const float*)TP(b + 0, nn * 4);
        Mg[d].nb = (const float*)TP(b + 1, nn * 4);
        Mg[d].fc1w = (const uint16_t*)TP(b + 2, (size_t)MH * MH * 2);
        Mg[d].fc1b = (const float*)TP(b + 3, MH * 4);
        Mg[d].fc2w = (const uint16_t*)TP(b + 4, (size_t)OR_H * MH * 2);
        Mg[d].fc2b = (const float*)TP(b + 5, OR_H * 4);
        if (!Mg[d].nw || !Mg[d].nb || !Mg[d].fc1w || !Mg[d].fc1b || !Mg[d].fc2w || !Mg[d].fc2b) {
            g_vis_err = "merger tensor missing or mis-sized";
            return -1;
        }
    }
#undef TP
    return 0;
}

int or_vision(const uint8_t* img, size_t len, const uint8_t* rgb, int gh, int gw, float* pooler,
              float* const* deepstack) {
    if (gh < 2 || gw < 2 || gh % 2 || gw % 2 || gh * gw > OR_NPATCH_MAX) {
        g_vis_err = "grid must be even and hold at most 1024 patches";
        return -1;
    }
    const uint16_t* patch_w;
    const float *patch_b, *pos;
    vit_layer L[OR_VLAYERS];
    merger_w Mg[4];
    if (parse_vision(img, len, &patch_w, &patch_b, &pos, L, Mg)) return -1;
    lut_init();
    const int np = gh * gw, nvis = np / 4;
    uint16_t* patches = (uint16_t*)malloc(2 * (size_t)np * VPATCH);
    float* x = (float*)malloc(sizeof(float) * (size_t)np * VH);
    float* pe = (float*)malloc(sizeof(float) * (size_t)np * VH);
    float* rope = (float*)malloc(sizeof(float) * (size_t)np * 64);
    uint16_t* xn = (uint16_t*)malloc(2 * (size_t)np * VH);
    float* qkv = (float*)malloc(sizeof(float) * (size_t)np * VQKV);
    uint16_t* qh = (uint16_t*)malloc(2 * (size_t)3 * VNH * np * VHD);
    uint16_t* att = (uint16_t*)malloc(2 * (size_t)np * VH);
    float* t = (float*)malloc(sizeof(float) * (size_t)np * VFF);
    uint16_t* hb = (uint16_t*)malloc(2 * (size_t)np * VFF);

    or_vit_patchify(rgb, gh, gw, patches);
    or_vit_pos_interp(pos, gh, gw, pe);
    or_vit_rope_table(gh, gw, rope);
    /* Patch embedding: (X W^T + b) + pos (k_vit_patch_embed, MODE 4). */
    or_linear_f16(patches, patch_w, patch_b, np, VH, VPATCH, x);
    for (size_t i = 0; i < (size_t)np * VH; ++i) x[i] = x[i] + pe[i];

    int ds = 0;
    for (int l = 0; l < OR_VLAYERS; ++l) {
        vit_block(&L[l], x, rope, np, xn, qkv, qh, att, t, hb);
        if (l == 5 || l == 11 || l == 17) {
            /* DeepStack merger: LayerNorm over the 4096 values of each 2 x 2 block (Engine.swift:
             * 420-447; qwen3vl_ref.py:200-208). */
            or_layernorm_f16(x, Mg[ds].nw, Mg[ds].nb, nvis, MH, xn);
            if (deepstack && deepstack[ds]) merger_mlp(&Mg[ds], xn, nvis, deepstack[ds]);
            ds++;
        }
    }
    /* Final merger: LayerNorm over 1024 per patch, then 2 x 2 blocks as rows of 4096
     * (Engine.swift:450-472; qwen3vl_ref.py:210-215). */
    or_layernorm_f16(x, Mg[3].nw, Mg[3].nb, np, VH, xn);
    merger_mlp(&Mg[3], xn, nvis, pooler);

    free(patches);
    free(x);
    free(pe);
    free(rope);
    free(xn);
    free(qkv);
    free(qh);
    free(att);
    free(t);
    free(hb);
    return 0;
}

int or_vit_block(const uint8_t* img, size_t len, int l, float* x, int gh, int gw) {
    const uint16_t* patch_w;
    const float *patch_b, *pos;
    vit_layer L[OR_VLAYERS];
    merger_w Mg[4];
    if (l < 0 || l >= OR_VLAYERS || gh * gw > OR_NPATCH_MAX) {
        g_vis_err = "bad block or grid";
        return -1;
    }
    if (parse_vision(img, len, &patch_w, &patch_b, &pos, L, Mg)) return -1;
    const int np = gh * gw;
    float* rope = (float*)malloc(sizeof(float) * (size_t)np * 64);
    uint16_t* xn = (uint16_t*)malloc(2 * (size_t)np * VH);
    float* qkv = (float*)malloc(sizeof(float) * (size_t)np * VQKV);
    uint16_t* qh = (uint16_t*)malloc(2 * (size_t)3 * VNH * np * VHD);
    uint16_t* att = (uint16_t*)malloc(2 * (size_t)np * VH);
    float* t = (float*)malloc(sizeof(float) * (size_t)np * VFF);
    uint16_t* hb = (uint16_t*)malloc(2 * (size_t)np * VFF);
    or_vit_rope_table(gh, gw, rope);
    vit_block(&L[l], x, rope, np, xn, qkv, qh, att, t, hb);
    free(rope);
    free(xn);
    free(qkv);
    free(qh);
    free(att);
    free(t);
    free(hb);
    return 0;
}
