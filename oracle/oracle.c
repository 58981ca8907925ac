/* CPU oracle for the Qwen3-VL text-decoder token loop -- TEST INFRASTRUCTURE ONLY.
 * The arithmetic contract and the reference files each part follows are stated in
 * oracle.h.  Nothing in the product library links this file. */
#include "oracle.h"
#include "oracle_model.h"

#include <math.h>
#include <omp.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define OR_EPS ((double)1e-6f) /* EPS 1e-6f (Shaders.swift:36) */
#define OR_THETA 5000000.0     /* Dims.ropeTheta (ModelFile.swift:59) */

static __thread char g_err[256];
const char* or_last_error(void) { return g_err; }
static void set_err(const char* s) { snprintf(g_err, sizeof g_err, "%s", s); }

void or_set_threads(int n) {
    if (n > 0) omp_set_num_threads(n);
}
int or_get_threads(void) { return omp_get_max_threads(); }

/* ------------------------------------------------------------------------------------------ */
/* fp16 conversions (IEEE 754 binary16). */

float or_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do {
                man <<= 1;
                e++;
            } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t or_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u : 0));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                                    /* below 2^-14: subnormal half */
        if (ax < 0x33000000u) return (uint16_t)sign;           /* < 2^-25 rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e; /* value = m * 2^(e-150); half ulp = 2^-24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 127 + 15;
    uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1))) q++;
    return (uint16_t)(sign | q);
}

/* ------------------------------------------------------------------------------------------ */
/* Codecs. */

/* One row of a [rows][K] matrix to double (values are the fp32 dequantised weights). */
static void dequant_row_d(int fmt, const uint8_t* codes, const uint8_t* sb, int K, long row, double* w) {
    if (fmt == 2) { /* q4: byte j holds q[2j] (low nibble) and q[2j+1] (Convert.swift:262) */
        const uint8_t* c = codes + (size_t)row * (K / 2);
        const uint16_t* p = (const uint16_t*)sb + (size_t)row * (K / 64) * 2;
        for (int g = 0; g < K / 64; ++g) {
            float s = or_h2f(p[2 * g]), b = or_h2f(p[2 * g + 1]);
            for (int j = 0; j < 32; ++j) {
                uint8_t v = c[g * 32 + j];
                float w0 = s * (float)(v & 15) + b; /* s*q is exact in fp32, so this is fl32(s*q+b) */
                float w1 = s * (float)(v >> 4) + b;
                w[g * 64 + 2 * j] = w0;
                w[g * 64 + 2 * j + 1] = w1;
            }
        }
    } else if (fmt == 1) { /* q8 symmetric, group 32 */
        const int8_t* c = (const int8_t*)codes + (size_t)row * K;
        const uint16_t* p = (const uint16_t*)sb + (size_t)row * (K / 32);
        for (int g = 0; g < K / 32; ++g) {
            float s = or_h2f(p[g]);
            for (int j = 0; j < 32; ++j) w[g * 32 + j] = (float)(s * (float)c[g * 32 + j]);
        }
    } else {
        const uint16_t* c = (const uint16_t*)codes + (size_t)row * K;
        for (int k = 0; k < K; ++k) w[k] = or_h2f(c[k]);
    }
}

void or_dequant(int fmt, const uint8_t* codes, const uint8_t* sb, int rows, int K, float* out) {
#pragma omp parallel
    {
        double* w = (double*)malloc(sizeof(double) * K);
#pragma omp for schedule(static)
        for (long r = 0; r < rows; ++r) {
            dequant_row_d(fmt, codes, sb, K, r, w);
            for (int k = 0; k < K; ++k) out[r * (size_t)K + k] = (float)w[k];
        }
        free(w);
    }
}

typedef double v4d __attribute__((vector_size(32)));

static double dotd(const double* a, const double* b, int K) {
    v4d s0 = {0, 0, 0, 0}, s1 = {0, 0, 0, 0};
    for (int k = 0; k < K; k += 8) {
        v4d a0, a1, b0, b1;
        memcpy(&a0, a + k, 32);
        memcpy(&a1, a + k + 4, 32);
        memcpy(&b0, b + k, 32);
        memcpy(&b1, b + k + 4, 32);
        s0 += a0 * b0;
        s1 += a1 * b1;
    }
    v4d s = s0 + s1;
    return (s[0] + s[1]) + (s[2] + s[3]);
}

/* y[t][r] for t < n: rows in parallel, tokens in blocks so that the block of x stays in cache. */
static void gemv_d(int fmt, const uint8_t* codes, const uint8_t* sb, int N, int K, const double* xd, int n,
                   float* y) {
    const int TB = 16;
#pragma omp parallel
    {
        double* w = (double*)aligned_alloc(64, sizeof(double) * K);
#pragma omp for schedule(static)
        for (int r = 0; r < N; ++r) {
            dequant_row_d(fmt, codes, sb, K, r, w);
            for (int t0 = 0; t0 < n; t0 += TB) {
                int t1 = t0 + TB < n ? t0 + TB : n;
                for (int t = t0; t < t1; ++t) y[(size_t)t * N + r] = (float)dotd(w, xd + (size_t)t * K, K);
            }
        }
        free(w);
    }
}

void or_gemv(int fmt, const uint8_t* codes, const uint8_t* sb, int N, int K, const float* x, int n, float* y) {
    double* xd = (double*)aligned_alloc(64, sizeof(double) * (size_t)n * K);
    for (size_t i = 0; i < (size_t)n * K; ++i) xd[i] = x[i];
    gemv_d(fmt, codes, sb, N, K, xd, n, y);
    free(xd);
}

/* ------------------------------------------------------------------------------------------ */
/* M-RoPE table (Engine.swift:121-125 inv-freq in double; 254-298 positions and angles). */

void or_mrope_table(int maxctx, int vis_offset, int llm_h, int llm_w, float* out) {
    double invf[64];
    for (int i = 0; i < 64; ++i) invf[i] = 1.0 / pow(OR_THETA, (double)(2 * i) / (double)OR_HD);
    int n_vis = llm_h * llm_w;
    int delta = (llm_h > llm_w ? llm_h : llm_w) - n_vis;
    for (int slot = 0; slot < maxctx; ++slot) {
        int pt, ph, pw;
        if (vis_offset < 0 || slot < vis_offset) {
            pt = ph = pw = slot;
        } else if (slot < vis_offset + n_vis) {
            int v = slot - vis_offset;
            pt = vis_offset;
            ph = vis_offset + v / llm_w;
            pw = vis_offset + v % llm_w;
        } else {
            pt = ph = pw = slot + delta;
        }
        for (int i = 0; i < 64; ++i) {
            int p = (i < 60 && i % 3 == 1) ? ph : (i < 60 && i % 3 == 2) ? pw : pt;
            double ang = (double)((float)p * (float)invf[i]);
            out[(size_t)slot * 128 + 2 * i] = (float)cos(ang);
            out[(size_t)slot * 128 + 2 * i + 1] = (float)sin(ang);
        }
    }
}

/* ------------------------------------------------------------------------------------------ */
/* Model. */

enum { T_LLM_BASE = 315, T_LAYER_BASE = 318, T_PER_LAYER = 14, T_COUNT = 710 };

static size_t code_bytes(int fmt, size_t rows, size_t K) {
    return fmt == 2 ? rows * K / 2 : fmt == 1 ? rows * K : rows * K * 2;
}
static size_t sb_bytes(int fmt, size_t rows, size_t K) {
    return fmt == 2 ? rows * (K / 64) * 4 : fmt == 1 ? rows * (K / 32) * 2 : 0;
}

or_model* or_model_new(const uint8_t* img, size_t len, int maxctx) {
    if (len < 16384 || len % 16384) {
        set_err("bad image size");
        return NULL;
    }
    const uint32_t* h = (const uint32_t*)img;
    if (h[0] != 0x31554349u || h[1] != 1 || h[2] > 2 || h[3] != T_COUNT) {
        set_err("bad header");
        return NULL;
    }
    const uint64_t* tab = (const uint64_t*)(img + 16);
    or_model* m = (or_model*)calloc(1, sizeof(or_model));
    m->fmt = (int)h[2];
    m->img = img;
    m->maxctx = maxctx;
#define CHECK(id, want)                                                                    \
    do {                                                                                   \
        if (tab[2 * (id) + 1] != (uint64_t)(want) || tab[2 * (id)] + (want) > len) {       \
            snprintf(g_err, sizeof g_err, "tensor %d: size %llu, want %llu", (int)(id),    \
                     (unsigned long long)tab[2 * (id) + 1], (unsigned long long)(want));   \
            free(m);                                                                       \
            return NULL;                                                                   \
        }                                                                                  \
    } while (0)
    int fmt = m->fmt;
    CHECK(T_LLM_BASE + 0, code_bytes(fmt, OR_VOCAB, OR_H));
    CHECK(T_LLM_BASE + 1, sb_bytes(fmt, OR_VOCAB, OR_H));
    CHECK(T_LLM_BASE + 2, OR_H * 4);
    m->embed = img + tab[2 * (T_LLM_BASE + 0)];
    m->embed_sb = img + tab[2 * (T_LLM_BASE + 1)];
    m->final_norm = (const float*)(img + tab[2 * (T_LLM_BASE + 2)]);
    int nl = 0;
    while (nl < OR_MAXLAYERS && tab[2 * (T_LAYER_BASE + nl * T_PER_LAYER + 1) + 1] != 0) nl++;
    for (int l = 0; l < nl; ++l) {
        int b = T_LAYER_BASE + l * T_PER_LAYER;
        CHECK(b + 0, OR_H * 4);
        CHECK(b + 1, code_bytes(fmt, OR_QKV, OR_H));
        CHECK(b + 2, sb_bytes(fmt, OR_QKV, OR_H));
        CHECK(b + 3, OR_HD * 4);
        CHECK(b + 4, OR_HD * 4);
        CHECK(b + 5, code_bytes(fmt, OR_H, OR_H));
        CHECK(b + 6, sb_bytes(fmt, OR_H, OR_H));
        CHECK(b + 7, OR_H * 4);
        CHECK(b + 8, code_bytes(fmt, OR_GU, OR_H));
        CHECK(b + 9, sb_bytes(fmt, OR_GU, OR_H));
        CHECK(b + 10, code_bytes(fmt, OR_H, OR_FF));
        CHECK(b + 11, sb_bytes(fmt, OR_H, OR_FF));
        or_layer_w* L = &m->L[l];
        L->attn_norm = (const float*)(img + tab[2 * (b + 0)]);
        L->wqkv = img + tab[2 * (b + 1)];
        L->wqkv_sb = img + tab[2 * (b + 2)];
        L->q_norm = (const float*)(img + tab[2 * (b + 3)]);
        L->k_norm = (const float*)(img + tab[2 * (b + 4)]);
        L->wo = img + tab[2 * (b + 5)];
        L->wo_sb = img + tab[2 * (b + 6)];
        L->mlp_norm = (const float*)(img + tab[2 * (b + 7)]);
        L->wgu = img + tab[2 * (b + 8)];
        L->wgu_sb = img + tab[2 * (b + 9)];
        L->wd = img + tab[2 * (b + 10)];
        L->wd_sb = img + tab[2 * (b + 11)];
    }
#undef CHECK
    if (nl == 0) {
        set_err("no decoder layers");
        free(m);
        return NULL;
    }
    m->layers = nl;
    size_t kvn = (size_t)nl * 2 * OR_NKV * maxctx * OR_HD;
    m->kv = (uint16_t*)calloc(kvn, 2);
    m->rope = (float*)malloc(sizeof(float) * (size_t)maxctx * 128);
    if (!m->kv || !m->rope) {
        set_err("out of memory");
        free(m->kv);
        free(m->rope);
        free(m);
        return NULL;
    }
    or_mrope_table(maxctx, -1, 1, 1, m->rope);
    return m;
}

void or_model_free(or_model* m) {
    if (!m) return;
    free(m->kv);
    free(m->rope);
    free(m);
}
int or_model_layers(const or_model* m) { return m->layers; }
int or_model_format(const or_model* m) { return m->fmt; }

void or_prepare_mrope(or_model* m, int vis_offset, int llm_h, int llm_w) {
    or_mrope_table(m->maxctx, vis_offset, llm_h, llm_w, m->rope);
}

uint16_t* or_kv(or_model* m, int layer, int kind) {
    return m->kv + ((size_t)layer * 2 + kind) * OR_NKV * m->maxctx * OR_HD;
}

/* RMSNorm(H) -> fp32 GEMV input, kept as double for the dot products (qwen3vl_ref.py:148-150;
 * Shaders.swift:634-657 computes the same expression). */
static void rmsnorm_in(const float* x, const float* w, int n, double* out) {
    double ss = 0;
    for (int i = 0; i < n; ++i) ss += (double)x[i] * x[i];
    double scale = 1.0 / sqrt(ss / n + OR_EPS);
    for (int i = 0; i < n; ++i) out[i] = (float)((double)x[i] * scale * (double)w[i]);
}

/* Per-head RMSNorm(128) in place, fp32 result (Shaders.swift:764-769; qwen3vl_ref.py:254-255). */
static void head_norm(float* v, const float* w) {
    double ss = 0;
    for (int i = 0; i < OR_HD; ++i) ss += (double)v[i] * v[i];
    double scale = 1.0 / sqrt(ss / OR_HD + OR_EPS);
    for (int i = 0; i < OR_HD; ++i) v[i] = (float)((double)v[i] * scale * (double)w[i]);
}

/* rotate_half RoPE with the table row of `slot` (qwen3vl_ref.py:153-155, 257-258;
 * Shaders.swift:770-774). */
static void rope_apply(float* v, const float* cs) {
    for (int i = 0; i < 64; ++i) {
        double c = cs[2 * i], s = cs[2 * i + 1];
        double a = v[i], b = v[i + 64];
        v[i] = (float)(a * c - b * s);
        v[i + 64] = (float)(b * c + a * s);
    }
}

void or_embed(const or_model* m, int tok, float* x) {
    double w[OR_H];
    dequant_row_d(m->fmt, m->embed, m->embed_sb, OR_H, tok, w);
    for (int i = 0; i < OR_H; ++i) x[i] = (float)w[i];
}

static float* g_dbg_qkv = NULL; /* raw QKV GEMV rows [n][QKV] */
static float* g_dbg_att = NULL; /* attention output before fp16 rounding [n][H] */
static float* g_dbg_act = NULL; /* SwiGLU output before fp16 rounding [n][FF] */
void or_debug_taps(float* qkv, float* att, float* act) {
    g_dbg_qkv = qkv;
    g_dbg_att = att;
    g_dbg_act = act;
}

void or_layer(or_model* m, int l, float* x, int n, int pos) {
    const or_layer_w* L = &m->L[l];
    const int H = OR_H, FF = OR_FF;
    double* xd = (double*)aligned_alloc(64, sizeof(double) * (size_t)n * FF);
    float* qkv = (float*)malloc(sizeof(float) * (size_t)n * OR_QKV);
    float* att = (float*)malloc(sizeof(float) * (size_t)n * H);
    float* gu = (float*)malloc(sizeof(float) * (size_t)n * OR_GU);
    float* y = (float*)malloc(sizeof(float) * (size_t)n * H);
    uint16_t* kc = or_kv(m, l, 0);
    uint16_t* vc = or_kv(m, l, 1);
    const size_t mc = (size_t)m->maxctx;

    /* 1. RMSNorm -> fused QKV GEMV (Convert.swift:185-188 row order q|k|v). */
    for (int t = 0; t < n; ++t) rmsnorm_in(x + (size_t)t * H, L->attn_norm, H, xd + (size_t)t * H);
    gemv_d(m->fmt, L->wqkv, L->wqkv_sb, OR_QKV, H, xd, n, qkv);
    if (g_dbg_qkv) memcpy(g_dbg_qkv, qkv, sizeof(float) * (size_t)n * OR_QKV);

    /* 2. q_norm / k_norm, RoPE, K/V cache write in fp16. */
    for (int t = 0; t < n; ++t) {
        float* r = qkv + (size_t)t * OR_QKV;
        const float* cs = m->rope + (size_t)(pos + t) * 128;
        for (int hd = 0; hd < OR_NH; ++hd) {
            head_norm(r + hd * OR_HD, L->q_norm);
            rope_apply(r + hd * OR_HD, cs);
        }
        for (int g = 0; g < OR_NKV; ++g) {
            float* k = r + OR_H + g * OR_HD;
            const float* v = r + OR_H + OR_NKV * OR_HD + g * OR_HD;
            head_norm(k, L->k_norm);
            rope_apply(k, cs);
            for (int d = 0; d < OR_HD; ++d) {
                kc[((size_t)g * mc + pos + t) * OR_HD + d] = or_f2h(k[d]);
                vc[((size_t)g * mc + pos + t) * OR_HD + d] = or_f2h(v[d]);
            }
        }
    }

    /* 3. Causal GQA attention over cache slots 0..pos+t (qwen3vl_ref.py:262-270, 313-320);
     * Q head h reads KV group h / 2.  The fp16 cache is widened to fp32 once per layer. */
    const int L1 = pos + n;
    float* kf = (float*)malloc(sizeof(float) * (size_t)OR_NKV * L1 * OR_HD);
    float* vf = (float*)malloc(sizeof(float) * (size_t)OR_NKV * L1 * OR_HD);
#pragma omp parallel for schedule(static)
    for (int g = 0; g < OR_NKV; ++g) {
        for (size_t i = 0; i < (size_t)L1 * OR_HD; ++i) {
            kf[(size_t)g * L1 * OR_HD + i] = or_h2f(kc[(size_t)g * mc * OR_HD + i]);
            vf[(size_t)g * L1 * OR_HD + i] = or_h2f(vc[(size_t)g * mc * OR_HD + i]);
        }
    }
#pragma omp parallel
    {
        double* sc = (double*)malloc(sizeof(double) * L1);
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (int t = 0; t < n; ++t) {
            for (int hd = 0; hd < OR_NH; ++hd) {
                const float* q = qkv + (size_t)t * OR_QKV + hd * OR_HD;
                int g = hd / (OR_NH / OR_NKV);
                int len = pos + t + 1;
                const float* kg = kf + (size_t)g * L1 * OR_HD;
                const float* vg = vf + (size_t)g * L1 * OR_HD;
                double mx = -INFINITY;
                for (int j = 0; j < len; ++j) {
                    const float* kr = kg + (size_t)j * OR_HD;
                    double a = 0;
                    for (int d = 0; d < OR_HD; ++d) a += (double)q[d] * (double)kr[d];
                    a *= 1.0 / sqrt((double)OR_HD);
                    sc[j] = a;
                    if (a > mx) mx = a;
                }
                double sum = 0;
                for (int j = 0; j < len; ++j) {
                    sc[j] = exp(sc[j] - mx);
                    sum += sc[j];
                }
                double o[OR_HD];
                for (int d = 0; d < OR_HD; ++d) o[d] = 0;
                for (int j = 0; j < len; ++j) {
                    const float* vr = vg + (size_t)j * OR_HD;
                    for (int d = 0; d < OR_HD; ++d) o[d] += sc[j] * (double)vr[d];
                }
                for (int d = 0; d < OR_HD; ++d) att[(size_t)t * H + hd * OR_HD + d] = (float)(o[d] / sum);
            }
        }
        free(sc);
    }
    free(kf);
    free(vf);

    if (g_dbg_att) memcpy(g_dbg_att, att, sizeof(float) * (size_t)n * H);
    /* 4. O projection of the fp32 attention output, residual add in fp32. */
    for (size_t i = 0; i < (size_t)n * H; ++i) xd[i] = att[i];
    gemv_d(m->fmt, L->wo, L->wo_sb, H, H, xd, n, y);
    for (size_t i = 0; i < (size_t)n * H; ++i) x[i] = x[i] + y[i];

    /* 5. RMSNorm -> gate|up GEMV (Convert.swift:193-194) -> SwiGLU (fp32) -> down GEMV. */
    for (int t = 0; t < n; ++t) rmsnorm_in(x + (size_t)t * H, L->mlp_norm, H, xd + (size_t)t * H);
    gemv_d(m->fmt, L->wgu, L->wgu_sb, OR_GU, H, xd, n, gu);
    for (int t = 0; t < n; ++t) {
        for (int i = 0; i < FF; ++i) {
            double g = gu[(size_t)t * OR_GU + i], u = gu[(size_t)t * OR_GU + FF + i];
            float a = (float)(g / (1.0 + exp(-g)) * u);
            if (g_dbg_act) g_dbg_act[(size_t)t * FF + i] = a;
            xd[(size_t)t * FF + i] = a;
        }
    }
    gemv_d(m->fmt, L->wd, L->wd_sb, H, FF, xd, n, y);
    for (size_t i = 0; i < (size_t)n * H; ++i) x[i] = x[i] + y[i];

    free(xd);
    free(qkv);
    free(att);
    free(gu);
    free(y);
}

void or_lm_head(const or_model* m, const float* x, float* logits) {
    double* h = (double*)aligned_alloc(64, sizeof(double) * OR_H);
    rmsnorm_in(x, m->final_norm, OR_H, h);
    gemv_d(m->fmt, m->embed, m->embed_sb, OR_VOCAB, OR_H, h, 1, logits);
    free(h);
}

int or_argmax(const float* v, int n) {
    int bi = 0;
    for (int i = 1; i < n; ++i)
        if (v[i] > v[bi]) bi = i;
    return bi;
}

int or_pass(or_model* m, const int32_t* toks, int n, int pos, const float* pooler, int vis_offset, int n_vis,
            const float* const* deepstack, int logits_rows, float* logits) {
    if (n <= 0 || pos < 0 || pos + n > m->maxctx) {
        set_err("pass exceeds context");
        return -1;
    }
    float* x = (float*)malloc(sizeof(float) * (size_t)n * OR_H);
    for (int t = 0; t < n; ++t) {
        int v = t - vis_offset;
        if (pooler && vis_offset >= 0 && toks[t] == OR_IMAGE_PAD && v >= 0 && v < n_vis)
            memcpy(x + (size_t)t * OR_H, pooler + (size_t)v * OR_H, sizeof(float) * OR_H);
        else
            or_embed(m, toks[t], x + (size_t)t * OR_H);
    }
    for (int l = 0; l < m->layers; ++l) {
        or_layer(m, l, x, n, pos);
        if (deepstack && vis_offset >= 0 && l < 3) {
            for (int v = 0; v < n_vis && vis_offset + v < n; ++v) {
                float* xr = x + (size_t)(vis_offset + v) * OR_H;
                const float* d = deepstack[l] + (size_t)v * OR_H;
                for (int i = 0; i < OR_H; ++i) xr[i] = xr[i] + d[i];
            }
        }
    }
    if (logits_rows == 1) {
        or_lm_head(m, x + (size_t)(n - 1) * OR_H, logits);
    } else if (logits_rows == n) {
        for (int t = 0; t < n; ++t) or_lm_head(m, x + (size_t)t * OR_H, logits + (size_t)t * OR_VOCAB);
    }
    free(x);
    return 0;
}

static float top2_margin(const float* v, int n, int best) {
    float second = -INFINITY;
    for (int i = 0; i < n; ++i)
        if (i != best && v[i] > second) second = v[i];
    return v[best] - second;
}

int or_generate(or_model* m, const int32_t* toks, int n, const float* pooler, int vis_offset, int n_vis,
                const float* const* deepstack, int steps, int32_t* out_tokens, float* margins, float* top1,
                float* out_first_logits) {
    float* logits = (float*)malloc(sizeof(float) * OR_VOCAB);
    int rc = or_pass(m, toks, n, 0, pooler, vis_offset, n_vis, deepstack, 1, logits);
    if (rc) {
        free(logits);
        return rc;
    }
    if (out_first_logits) memcpy(out_first_logits, logits, sizeof(float) * OR_VOCAB);
    int tok = or_argmax(logits, OR_VOCAB);
    out_tokens[0] = tok;
    if (margins) margins[0] = top2_margin(logits, OR_VOCAB, tok);
    if (top1) top1[0] = logits[tok];
    for (int s = 1; s < steps; ++s) {
        rc = or_pass(m, &tok, 1, n + s - 1, NULL, -1, 0, NULL, 1, logits);
        if (rc) break;
        tok = or_argmax(logits, OR_VOCAB);
        out_tokens[s] = tok;
        if (margins) margins[s] = top2_margin(logits, OR_VOCAB, tok);
        if (top1) top1[s] = logits[tok];
    }
    free(logits);
    return rc;
}

static int first_step_action(int tok) {
    return tok == 3678 || tok == 7241 || tok == 12476 || tok == 10855 || tok == 11862 || tok == 1339 || tok == 1472 ||
           tok == 24769;
}

int or_generate_commit(or_model* m, const int32_t* toks, int n, const float* pooler, int vis_offset, int n_vis,
                       const float* const* deepstack, int max_steps, int eos0, int eos1, int grammar,
                       int32_t* out_tokens) {
    float* logits = (float*)malloc(sizeof(float) * OR_VOCAB);
    int32_t pass[2];
    const int32_t* pt = toks;
    int pn = n, pos = 0, step = 0;
    for (;;) {
        if (step >= max_steps) break;
        if (or_pass(m, pt, pn, pos, pooler, vis_offset, n_vis, deepstack, 1, logits)) {
            free(logits);
            return -1;
        }
        pooler = NULL; /* the visual rows belong to the prompt pass only */
        deepstack = NULL;
        vis_offset = -1;
        n_vis = 0;
        const int tok = or_argmax(logits, OR_VOCAB);
        pos += pn;
        out_tokens[step++] = tok;
        if (tok == eos0 || tok == eos1 || (grammar && tok == 8) || step >= max_steps) break;
        pass[0] = tok;
        pt = pass;
        pn = 1;
        if (grammar && ((step == 1 && first_step_action(tok)) || tok == 11)) {
            pass[1] = tok == 11 ? 220 : 7;
            out_tokens[step++] = pass[1];
            pn = 2;
        }
    }
    free(logits);
    return step;
}

/* ------------------------------------------------------------------------------------------ */
/* Quantisers of the converter (Convert.swift:214-320), float32 arithmetic in the reference's
 * order: sums run over i = 0..n-1, no contraction (the Makefile builds with
 * -ffp-contract=off), division correctly rounded, `.rounded()` = roundf (half away from zero),
 * Float16(x) = round to nearest even (or_f2h). */

/* Swift's min / max on Float: min(x, y) = y < x ? y : x, max(x, y) = y >= x ? y : x. */
static float sw_min(float x, float y) { return y < x ? y : x; }
static float sw_max(float x, float y) { return y >= x ? y : x; }

void or_quant_q8(const float* m, int rows, int cols, int8_t* codes, uint16_t* scales) {
    const int groups = cols / 32;
#pragma omp parallel for schedule(static)
    for (int ci = 0; ci < (rows + 63) / 64; ++ci) {
        for (int r = ci * 64; r < rows && r < (ci + 1) * 64; ++r) {
            for (int g = 0; g < groups; ++g) {
                const float* src = m + (size_t)r * cols + (size_t)g * 32;
                float amax = 0.0f;
                for (int i = 0; i < 32; ++i) amax = sw_max(amax, fabsf(src[i]));
                uint16_t sh = or_f2h(amax / 127.0f);
                if (or_h2f(sh) * 127.0f < amax) sh = (uint16_t)(sh + 1u); /* Convert.swift:229 */
                const float s = or_h2f(sh);
                scales[(size_t)r * groups + g] = sh;
                const float inv = s > 0.0f ? 1.0f / s : 0.0f;
                for (int i = 0; i < 32; ++i)
                    codes[(size_t)r * cols + (size_t)g * 32 + i] =
                        (int8_t)sw_max(-127.0f, sw_min(127.0f, roundf(src[i] * inv)));
            }
        }
    }
}

/* quantGroup (Convert.swift:273-319).  q_out keeps its contents when no candidate is accepted
 * (every candidate's fp16 scale rounds to 0): the caller's array then still holds the codes of
 * the chunk's previous group, as in the reference. */
static void quant_group_q4(const float* w, uint8_t* q_out, uint16_t* s_out, uint16_t* b_out) {
    static const float clips[5] = {0.0f, 0.03f, 0.06f, 0.1f, 0.15f};
    float mn = w[0], mx = w[0];
    for (int i = 1; i < 64; ++i) {
        mn = sw_min(mn, w[i]);
        mx = sw_max(mx, w[i]);
    }
    if (mx - mn < 1e-12f) {
        memset(q_out, 0, 64);
        *s_out = 0;
        *b_out = or_f2h(mn);
        return;
    }
    float best_err = INFINITY;
    uint16_t best_s = 0, best_b = 0;
    uint8_t q[64];
    const float range = mx - mn;
    for (int ai = 0; ai < 5; ++ai) {
        for (int cj = 0; cj < 5; ++cj) {
            const float lo = mn + clips[ai] * range, hi = mx - clips[cj] * range;
            if (hi <= lo) continue;
            float s = (hi - lo) / 15.0f, b = lo;
            /* Iteration 0 of the reference's two: the codes and the least-squares refit.  Its
             * iteration 1 only recomputes codes that the error pass below overwrites. */
            {
                const float inv = 1.0f / s;
                float sq = 0.0f, sw = 0.0f, sqq = 0.0f, sqw = 0.0f;
                for (int i = 0; i < 64; ++i) {
                    const float v = sw_min(15.0f, sw_max(0.0f, roundf((w[i] - b) * inv)));
                    sq += v;
                    sw += w[i];
                    sqq += v * v;
                    sqw += v * w[i];
                }
                const float den = 64.0f * sqq - sq * sq;
                if (den > 0.0f) {
                    const float s2 = (64.0f * sqw - sq * sw) / den;
                    if (s2 > 0.0f) {
                        s = s2;
                        b = (sw - s2 * sq) / 64.0f;
                    }
                }
            }
            const uint16_t sh = or_f2h(s), bh = or_f2h(b);
            const float sf = or_h2f(sh), bf = or_h2f(bh);
            if (sf <= 0.0f) continue;
            const float inv = 1.0f / sf;
            float err = 0.0f;
            for (int i = 0; i < 64; ++i) {
                const float v = sw_min(15.0f, sw_max(0.0f, roundf((w[i] - bf) * inv)));
                q[i] = (uint8_t)v;
                const float d = sf * v + bf - w[i];
                err += d * d;
            }
            if (err < best_err) {
                best_err = err;
                best_s = sh;
                best_b = bh;
                memcpy(q_out, q, 64);
            }
        }
    }
    *s_out = best_s;
    *b_out = best_b;
}

void or_quant_q4(const float* m, int rows, int cols, uint8_t* packed, uint16_t* sb) {
    const int groups = cols / 64;
#pragma omp parallel for schedule(static)
    for (int ci = 0; ci < (rows + 63) / 64; ++ci) {
        uint8_t q[64];
        memset(q, 0, 64); /* one code array per 64-row chunk (Convert.swift:251) */
        for (int r = ci * 64; r < rows && r < (ci + 1) * 64; ++r) {
            for (int g = 0; g < groups; ++g) {
                const size_t base = (size_t)r * cols + (size_t)g * 64;
                quant_group_q4(m + base, q, &sb[((size_t)r * groups + g) * 2], &sb[((size_t)r * groups + g) * 2 + 1]);
                for (int j = 0; j < 32; ++j) packed[base / 2 + j] = (uint8_t)(q[2 * j] | (q[2 * j + 1] << 4));
            }
        }
    }
}
