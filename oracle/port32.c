/* fp32 CPU port of the decoder token loop -- CPU BASELINE ONLY.
 *
 * The benchmark's CPU baseline: the reference decoder math (tools/reference/qwen3vl_ref.py:
 * 142-155, 243-336, fp32 throughout) over the oracle's model state (the same weights, fp16 KV
 * cache and M-RoPE table; oracle_model.h), written for speed on the host cores instead of as the
 * parity checker:
 *   - fp32 arithmetic and accumulation everywhere;
 *   - one-token GEMVs with the q4 / q8 dequantisation fused into the dot product (per group:
 *     s * sum q x, plus b * sum x for q4), eight lanes wide (AVX2, FMA, F16C);
 *   - many-token GEMMs dequantise a weight row once per block of 8 tokens and take the 8 dot
 *     products together;
 *   - OpenMP over weight rows and over (token, head) attention tasks.
 * Text tokens only (no visual rows, no DeepStack).  Nothing in the product library links it; the
 * checker is oracle.c, and tests/test_port32.py compares this port with it.
 */
#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#include "oracle_model.h"

#define P32_EPS 1e-6f /* EPS 1e-6f (Shaders.swift:36) */

static inline float hsum8(__m256 v) {
    __m128 a = _mm_add_ps(_mm256_castps256_ps128(v), _mm256_extractf128_ps(v, 1));
    a = _mm_add_ps(a, _mm_movehl_ps(a, a));
    a = _mm_add_ss(a, _mm_movehdup_ps(a));
    return _mm_cvtss_f32(a);
}

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }

/* ------------------------------------------------------------------------------------------ */
/* One-token GEMV, dequantisation fused into the dot product. */

/* A q4 row against x in nibble order: per 64-group, the 32 even-indexed activations, then the
 * 32 odd-indexed ones (byte j of a group holds q[2j] in its low nibble and q[2j+1] in its high
 * one, Convert.swift:262); xs[g] = the group's activation sum. */
static float dot_q4(const uint8_t* c, const uint16_t* sb, const float* xn, const float* xs, int K) {
    const __m256i m15 = _mm256_set1_epi32(15);
    __m256 y = _mm256_setzero_ps();
    float bsum = 0.f;
    for (int g = 0; g < K / 64; ++g) {
        __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
        const uint8_t* cg = c + g * 32;
        const float* xg = xn + g * 64;
        for (int j = 0; j < 32; j += 8) {
            const __m256i w = _mm256_cvtepu8_epi32(_mm_loadl_epi64((const __m128i*)(cg + j)));
            a0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_and_si256(w, m15)), _mm256_loadu_ps(xg + j), a0);
            a1 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_srli_epi32(w, 4)), _mm256_loadu_ps(xg + 32 + j), a1);
        }
        y = _mm256_fmadd_ps(_mm256_set1_ps(h2f(sb[2 * g])), _mm256_add_ps(a0, a1), y);
        bsum += h2f(sb[2 * g + 1]) * xs[g];
    }
    return hsum8(y) + bsum;
}

static float dot_q8(const int8_t* c, const uint16_t* sb, const float* x, int K) {
    __m256 y = _mm256_setzero_ps();
    for (int g = 0; g < K / 32; ++g) {
        __m256 a = _mm256_setzero_ps();
        for (int j = 0; j < 32; j += 8) {
            const __m256i w = _mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i*)(c + g * 32 + j)));
            a = _mm256_fmadd_ps(_mm256_cvtepi32_ps(w), _mm256_loadu_ps(x + g * 32 + j), a);
        }
        y = _mm256_fmadd_ps(_mm256_set1_ps(h2f(sb[g])), a, y);
    }
    return hsum8(y);
}

static float dot_f16(const uint16_t* c, const float* x, int K) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
    for (int k = 0; k < K; k += 16) {
        a0 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(c + k))), _mm256_loadu_ps(x + k), a0);
        a1 = _mm256_fmadd_ps(_mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(c + k + 8))), _mm256_loadu_ps(x + k + 8),
                             a1);
    }
    return hsum8(_mm256_add_ps(a0, a1));
}

static void gemv1(int fmt, const uint8_t* codes, const uint8_t* sb, int N, int K, const float* x, float* y) {
    float* xn = (float*)aligned_alloc(64, sizeof(float) * K);
    float* xs = (float*)malloc(sizeof(float) * (K / 64 + 1));
    if (fmt == 2) {
        for (int g = 0; g < K / 64; ++g) {
            float s = 0.f;
            for (int j = 0; j < 32; ++j) {
                xn[g * 64 + j] = x[g * 64 + 2 * j];
                xn[g * 64 + 32 + j] = x[g * 64 + 2 * j + 1];
                s += x[g * 64 + 2 * j] + x[g * 64 + 2 * j + 1];
            }
            xs[g] = s;
        }
    }
#pragma omp parallel for schedule(static)
    for (int r = 0; r < N; ++r) {
        if (fmt == 2)
            y[r] = dot_q4(codes + (size_t)r * (K / 2), (const uint16_t*)sb + (size_t)r * (K / 64) * 2, xn, xs, K);
        else if (fmt == 1)
            y[r] = dot_q8((const int8_t*)codes + (size_t)r * K, (const uint16_t*)sb + (size_t)r * (K / 32), x, K);
        else
            y[r] = dot_f16((const uint16_t*)codes + (size_t)r * K, x, K);
    }
    free(xn);
    free(xs);
}

/* ------------------------------------------------------------------------------------------ */
/* Many-token GEMM: y[t][r] for t < n. */

/* Row r dequantised to fp32 in K order (the codec values fl32(s q + b) / s q / the half). */
static void dequant_row(int fmt, const uint8_t* codes, const uint8_t* sb, int K, int r, float* w) {
    if (fmt == 2) {
        const uint8_t* c = codes + (size_t)r * (K / 2);
        const uint16_t* p = (const uint16_t*)sb + (size_t)r * (K / 64) * 2;
        for (int g = 0; g < K / 64; ++g) {
            const float s = h2f(p[2 * g]), b = h2f(p[2 * g + 1]);
            for (int j = 0; j < 32; ++j) {
                w[g * 64 + 2 * j] = s * (float)(c[g * 32 + j] & 15) + b;
                w[g * 64 + 2 * j + 1] = s * (float)(c[g * 32 + j] >> 4) + b;
            }
        }
    } else if (fmt == 1) {
        const int8_t* c = (const int8_t*)codes + (size_t)r * K;
        const uint16_t* p = (const uint16_t*)sb + (size_t)r * (K / 32);
        for (int k = 0; k < K; ++k) w[k] = h2f(p[k / 32]) * (float)c[k];
    } else {
        const uint16_t* c = (const uint16_t*)codes + (size_t)r * K;
        for (int k = 0; k < K; k += 8) _mm256_storeu_ps(w + k, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(c + k))));
    }
}

/* out[t] = w . x[t] for 8 token rows of stride K. */
static void dot8(const float* w, const float* x, int K, float* out) {
    __m256 a[8];
    for (int t = 0; t < 8; ++t) a[t] = _mm256_setzero_ps();
    for (int k = 0; k < K; k += 8) {
        const __m256 wv = _mm256_loadu_ps(w + k);
        for (int t = 0; t < 8; ++t) a[t] = _mm256_fmadd_ps(wv, _mm256_loadu_ps(x + (size_t)t * K + k), a[t]);
    }
    for (int t = 0; t < 8; ++t) out[t] = hsum8(a[t]);
}

static float dot1(const float* w, const float* x, int K) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
    for (int k = 0; k < K; k += 16) {
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(w + k), _mm256_loadu_ps(x + k), a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(w + k + 8), _mm256_loadu_ps(x + k + 8), a1);
    }
    return hsum8(_mm256_add_ps(a0, a1));
}

static void gemm(int fmt, const uint8_t* codes, const uint8_t* sb, int N, int K, const float* x, int n, float* y) {
    if (n == 1) {
        gemv1(fmt, codes, sb, N, K, x, y);
        return;
    }
#pragma omp parallel
    {
        const int nt = omp_get_num_threads(), id = omp_get_thread_num();
        const int r0 = (int)((long)N * id / nt), r1 = (int)((long)N * (id + 1) / nt);
        float* w = (float*)aligned_alloc(64, sizeof(float) * K);
        float o[8];
        for (int t0 = 0; t0 < n; t0 += 8) { /* 8 token rows stay in the core's cache */
            for (int r = r0; r < r1; ++r) {
                dequant_row(fmt, codes, sb, K, r, w);
                if (t0 + 8 <= n) {
                    dot8(w, x + (size_t)t0 * K, K, o);
                    for (int t = 0; t < 8; ++t) y[(size_t)(t0 + t) * N + r] = o[t];
                } else {
                    for (int t = t0; t < n; ++t) y[(size_t)t * N + r] = dot1(w, x + (size_t)t * K, K);
                }
            }
        }
        free(w);
    }
}

/* ------------------------------------------------------------------------------------------ */
/* Layer. */

static void rmsnorm(const float* x, const float* w, int n, float* out) {
    float ss = 0.f;
    for (int i = 0; i < n; ++i) ss += x[i] * x[i];
    const float scale = 1.0f / sqrtf(ss / (float)n + P32_EPS);
    for (int i = 0; i < n; ++i) out[i] = x[i] * scale * w[i];
}

static void head_norm_rope(float* v, const float* w, const float* cs) {
    float ss = 0.f;
    for (int i = 0; i < OR_HD; ++i) ss += v[i] * v[i];
    const float scale = 1.0f / sqrtf(ss / (float)OR_HD + P32_EPS);
    for (int i = 0; i < OR_HD; ++i) v[i] = v[i] * scale * w[i];
    for (int i = 0; i < 64; ++i) { /* rotate_half (qwen3vl_ref.py:153-155) */
        const float c = cs[2 * i], s = cs[2 * i + 1], a = v[i], b = v[i + 64];
        v[i] = a * c - b * s;
        v[i + 64] = b * c + a * s;
    }
}

static float dot_kh(const float* q, const uint16_t* k) {
    __m256 a = _mm256_setzero_ps();
    for (int d = 0; d < OR_HD; d += 8)
        a = _mm256_fmadd_ps(_mm256_loadu_ps(q + d), _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(k + d))), a);
    return hsum8(a);
}

static void p32_layer(or_model* m, int l, float* x, int n, int pos) {
    const or_layer_w* L = &m->L[l];
    const int H = OR_H, FF = OR_FF;
    const size_t mc = (size_t)m->maxctx;
    float* xn = (float*)aligned_alloc(64, sizeof(float) * (size_t)n * FF);
    float* qkv = (float*)malloc(sizeof(float) * (size_t)n * OR_QKV);
    float* att = (float*)malloc(sizeof(float) * (size_t)n * H);
    float* gu = (float*)malloc(sizeof(float) * (size_t)n * OR_GU);
    float* y = (float*)malloc(sizeof(float) * (size_t)n * H);
    uint16_t* kc = or_kv(m, l, 0);
    uint16_t* vc = or_kv(m, l, 1);

    for (int t = 0; t < n; ++t) rmsnorm(x + (size_t)t * H, L->attn_norm, H, xn + (size_t)t * H);
    gemm(m->fmt, L->wqkv, L->wqkv_sb, OR_QKV, H, xn, n, qkv);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; ++t) {
        float* r = qkv + (size_t)t * OR_QKV;
        const float* cs = m->rope + (size_t)(pos + t) * 128;
        for (int hd = 0; hd < OR_NH; ++hd) head_norm_rope(r + hd * OR_HD, L->q_norm, cs);
        for (int g = 0; g < OR_NKV; ++g) {
            float* k = r + OR_H + g * OR_HD;
            const float* v = r + OR_H + OR_NKV * OR_HD + g * OR_HD;
            head_norm_rope(k, L->k_norm, cs);
            for (int d = 0; d < OR_HD; ++d) {
                kc[((size_t)g * mc + pos + t) * OR_HD + d] = _cvtss_sh(k[d], 0);
                vc[((size_t)g * mc + pos + t) * OR_HD + d] = _cvtss_sh(v[d], 0);
            }
        }
    }

    /* Causal GQA attention (qwen3vl_ref.py:262-270): head h reads KV group h / 2. */
    const float qs = 1.0f / sqrtf((float)OR_HD);
#pragma omp parallel
    {
        float* sc = (float*)malloc(sizeof(float) * (size_t)(pos + n));
#pragma omp for schedule(dynamic, 1) collapse(2)
        for (int t = 0; t < n; ++t) {
            for (int hd = 0; hd < OR_NH; ++hd) {
                const float* q = qkv + (size_t)t * OR_QKV + hd * OR_HD;
                const int g = hd / (OR_NH / OR_NKV), len = pos + t + 1;
                const uint16_t* kg = kc + (size_t)g * mc * OR_HD;
                const uint16_t* vg = vc + (size_t)g * mc * OR_HD;
                float mx = -INFINITY;
                for (int j = 0; j < len; ++j) {
                    sc[j] = dot_kh(q, kg + (size_t)j * OR_HD) * qs;
                    mx = sc[j] > mx ? sc[j] : mx;
                }
                float sum = 0.f;
                for (int j = 0; j < len; ++j) {
                    sc[j] = expf(sc[j] - mx);
                    sum += sc[j];
                }
                __m256 o[OR_HD / 8];
                for (int d = 0; d < OR_HD / 8; ++d) o[d] = _mm256_setzero_ps();
                for (int j = 0; j < len; ++j) {
                    const __m256 p = _mm256_set1_ps(sc[j]);
                    const uint16_t* vr = vg + (size_t)j * OR_HD;
                    for (int d = 0; d < OR_HD / 8; ++d)
                        o[d] = _mm256_fmadd_ps(p, _mm256_cvtph_ps(_mm_loadu_si128((const __m128i*)(vr + 8 * d))), o[d]);
                }
                const __m256 inv = _mm256_set1_ps(1.0f / sum);
                for (int d = 0; d < OR_HD / 8; ++d)
                    _mm256_storeu_ps(att + (size_t)t * H + hd * OR_HD + 8 * d, _mm256_mul_ps(o[d], inv));
            }
        }
        free(sc);
    }

    gemm(m->fmt, L->wo, L->wo_sb, H, H, att, n, y);
    for (size_t i = 0; i < (size_t)n * H; ++i) x[i] += y[i];

    for (int t = 0; t < n; ++t) rmsnorm(x + (size_t)t * H, L->mlp_norm, H, xn + (size_t)t * H);
    gemm(m->fmt, L->wgu, L->wgu_sb, OR_GU, H, xn, n, gu);
#pragma omp parallel for schedule(static)
    for (int t = 0; t < n; ++t) {
        for (int i = 0; i < FF; ++i) {
            const float g = gu[(size_t)t * OR_GU + i], u = gu[(size_t)t * OR_GU + FF + i];
            xn[(size_t)t * FF + i] = g / (1.0f + expf(-g)) * u;
        }
    }
    gemm(m->fmt, L->wd, L->wd_sb, H, FF, xn, n, y);
    for (size_t i = 0; i < (size_t)n * H; ++i) x[i] += y[i];

    free(xn);
    free(qkv);
    free(att);
    free(gu);
    free(y);
}

int p32_pass(or_model* m, const int32_t* toks, int n, int pos, float* logits) {
    if (n <= 0 || pos < 0 || pos + n > m->maxctx) return -1;
    float* x = (float*)aligned_alloc(64, sizeof(float) * (size_t)n * OR_H);
    for (int t = 0; t < n; ++t) dequant_row(m->fmt, m->embed, m->embed_sb, OR_H, toks[t], x + (size_t)t * OR_H);
    for (int l = 0; l < m->layers; ++l) p32_layer(m, l, x, n, pos);
    float h[OR_H];
    rmsnorm(x + (size_t)(n - 1) * OR_H, m->final_norm, OR_H, h);
    gemv1(m->fmt, m->embed, m->embed_sb, OR_VOCAB, OR_H, h, logits);
    free(x);
    return 0;
}
