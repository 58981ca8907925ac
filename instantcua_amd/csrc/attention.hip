// GQA 16:8 decode / verify attention over the fp16 KV cache, gfx950.
//
// Replaces k_attention (Shaders.swift:1220-1289) and the q_norm/k_norm + M-RoPE + KV-write
// epilogue of k_attn_in (Shaders.swift:758-787).  Math follows tools/reference/qwen3vl_ref.py
// (254-270, 305-320): per-head RMSNorm(128) on q and k, rotate_half RoPE with the engine's
// M-RoPE table row of the token's cache slot, scores q.k / sqrt(128), softmax, P.V.
//
// Layout.  The cache of a layer is [NKV][maxctx][HD] fp16 (Engine.swift:110-112, 477): one
// KV group is a contiguous run of 256-byte rows.  The grid is (ATTN_SPLITS, NKV): workgroup
// (s, g) streams an equal share of the prior slots [0, pos) of group g once and serves BOTH
// query heads 2g and 2g+1 from it (the reference streams each group twice, once per head).
// Every 16-lane quarter-wave owns one cache row per step (16 x 16 B loads = 256 B), so a wave
// reads four consecutive rows = 1 KiB per instruction.
//
// The last split also owns the new rows of the pass (slots pos .. pos+M-1): it normalises,
// rotates and rounds their K/V to fp16, writes them to the cache and uses them, causally
// masked, from LDS.  Each split writes an unnormalised (o, m, l) partial; the workgroup that
// arrives last for a group merges the partials (flash-decoding) and writes the fp16 output
// row that feeds the O projection (the reference rounds it to fp16 there, Shaders.swift:659-669).
#include "icua_device.h"
#include "icua_kernels.h"

namespace icua {

constexpr int ATT_THREADS = 256;
constexpr int ATT_TQ = 2;          // query tokens per sweep over the split
constexpr int ATT_CHUNK_MAX = 256; // prior slots per split (maxctx <= ATT_CHUNK_MAX * ATTN_SPLITS)
constexpr int PART_STRIDE = HD + 2;

// Per-head RMSNorm(128) + RoPE of one 128-vector by one wave: lane i owns the rotation pair
// (i, i + 64).  Returns the pair in (a, b).
__device__ __forceinline__ void norm_rope_pair(float& a, float& b, const float* w, const float* cs, int lane) {
    const float ss = wave_sum(a * a + b * b);
    const float scale = 1.0f / sqrtf(ss / (float)HD + EPS);
    a = a * scale * w[lane];
    b = b * scale * w[lane + 64];
    const float c = cs[2 * lane], sn = cs[2 * lane + 1];
    const float a2 = a * c - b * sn;
    const float b2 = b * c + a * sn;
    a = a2;
    b = b2;
}

template <int MT>
__global__ __launch_bounds__(ATT_THREADS) void attention_kernel(AttnArgs a) {
    const State* st = a.st;
    if (st->done) return;
    const int M = a.m_fixed > 0 ? a.m_fixed : (st->n < MT ? st->n : MT);
    const int pos = st->pos;
    const int maxctx = st->maxctx;
    if (pos < 0 || pos + M > maxctx || pos > ATT_CHUNK_MAX * (int)gridDim.x) return;  // host-checked; never index past the cache
    const int s = blockIdx.x, S = gridDim.x, g = blockIdx.y;
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int quad = tid / 16, ql = tid % 16;  // 16 quarter-waves of 16 lanes
    const bool last = (s == S - 1);

    const int chunk = (pos + S - 1) / S;
    const int j0 = s * chunk < pos ? s * chunk : pos;
    const int j1 = (j0 + chunk) < pos ? (j0 + chunk) : pos;
    const int nprior = j1 - j0;
    const int ntail = last ? M : 0;
    const int P = nprior + ntail;

    __shared__ float qs[MT][2][HD];           // normalised, rotated, pre-scaled queries
    __shared__ float ktail[MT][HD];           // fp16-rounded new K/V rows (last split)
    __shared__ float vtail[MT][HD];
    __shared__ float sc[2 * ATT_TQ][ATT_CHUNK_MAX + MAXM];
    __shared__ float mrow[2 * ATT_TQ], lrow[2 * ATT_TQ];
    __shared__ float ored[16][2 * ATT_TQ][HD / 8][8];
    __shared__ int is_last;

    const float qscale = 1.0f / sqrtf((float)HD);
    // Queries (and, for the last split, the new K/V rows).
    for (int row = wave; row < 2 * M; row += ATT_THREADS / WAVE) {
        const int t = row / 2, hh = row % 2;
        const float* src = a.qkv + (size_t)t * QKV + (2 * g + hh) * HD;
        float x0 = src[lane], x1 = src[lane + 64];
        norm_rope_pair(x0, x1, a.q_norm, a.rope + (size_t)(pos + t) * 128, lane);
        qs[t][hh][lane] = x0 * qscale;
        qs[t][hh][lane + 64] = x1 * qscale;
    }
    if (last) {
        for (int t = wave; t < M; t += ATT_THREADS / WAVE) {
            const float* ksrc = a.qkv + (size_t)t * QKV + H + g * HD;
            const float* vsrc = a.qkv + (size_t)t * QKV + H + NKV * HD + g * HD;
            float k0 = ksrc[lane], k1 = ksrc[lane + 64];
            norm_rope_pair(k0, k1, a.k_norm, a.rope + (size_t)(pos + t) * 128, lane);
            const uint16_t hk0 = f2h(k0), hk1 = f2h(k1);
            const uint16_t hv0 = f2h(vsrc[lane]), hv1 = f2h(vsrc[lane + 64]);
            uint16_t* kd = a.kc + ((size_t)g * maxctx + pos + t) * HD;
            uint16_t* vd = a.vc + ((size_t)g * maxctx + pos + t) * HD;
            kd[lane] = hk0;
            kd[lane + 64] = hk1;
            vd[lane] = hv0;
            vd[lane + 64] = hv1;
            ktail[t][lane] = h2f(hk0);
            ktail[t][lane + 64] = h2f(hk1);
            vtail[t][lane] = h2f(hv0);
            vtail[t][lane + 64] = h2f(hv1);
        }
    }
    __syncthreads();

    const uint16_t* kbase = a.kc + (size_t)g * maxctx * HD;
    const uint16_t* vbase = a.vc + (size_t)g * maxctx * HD;
    float* part = a.part + (size_t)(g * S + s) * MAXM * 2 * PART_STRIDE;

    for (int t0 = 0; t0 < M; t0 += ATT_TQ) {
        const int tq = (M - t0) < ATT_TQ ? (M - t0) : ATT_TQ;
        // Lane ql of a quarter-wave holds query dims [8 ql, 8 ql + 8) of its rows.
        float qreg[ATT_TQ][2][8];
#pragma unroll
        for (int u = 0; u < ATT_TQ; ++u)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                for (int d = 0; d < 8; ++d) qreg[u][hh][d] = (u < tq) ? qs[t0 + u][hh][8 * ql + d] : 0.f;

        // 1. Scores.
        for (int p = quad; p < P; p += 16) {
            float kv[8];
            if (p < nprior) {
                const uint4 raw = *(const uint4*)(kbase + (size_t)(j0 + p) * HD + 8 * ql);
                const uint32_t d4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f16x2 h = as_h2(d4[i]);
                    kv[2 * i] = (float)h.x;
                    kv[2 * i + 1] = (float)h.y;
                }
            } else {
#pragma unroll
                for (int d = 0; d < 8; ++d) kv[d] = ktail[p - nprior][8 * ql + d];
            }
#pragma unroll
            for (int u = 0; u < ATT_TQ; ++u) {
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    float acc = 0.f;
#pragma unroll
                    for (int d = 0; d < 8; ++d) acc += qreg[u][hh][d] * kv[d];
                    acc = sum16(acc);
                    const bool masked = (u >= tq) || (p >= nprior && (p - nprior) > t0 + u);
                    if (ql == 0) sc[2 * u + hh][p] = masked ? -__builtin_inff() : acc;
                }
            }
        }
        __syncthreads();

        // 2. Split softmax statistics, one wave per (token, head) row.
        for (int row = wave; row < 2 * ATT_TQ; row += ATT_THREADS / WAVE) {
            float m = -__builtin_inff();
            for (int p = lane; p < P; p += WAVE) m = fmaxf(m, sc[row][p]);
            m = wave_max(m);
            float l = 0.f;
            for (int p = lane; p < P; p += WAVE) {
                const float e = (m == -__builtin_inff()) ? 0.f : expf(sc[row][p] - m);
                sc[row][p] = e;
                l += e;
            }
            l = wave_sum(l);
            if (lane == 0) {
                mrow[row] = m;
                lrow[row] = l;
            }
        }
        __syncthreads();

        // 3. P.V: lane ql of a quarter-wave accumulates dims [8 ql, 8 ql + 8).
        float o[2 * ATT_TQ][8];
#pragma unroll
        for (int r = 0; r < 2 * ATT_TQ; ++r)
#pragma unroll
            for (int d = 0; d < 8; ++d) o[r][d] = 0.f;
        for (int p = quad; p < P; p += 16) {
            float vv[8];
            if (p < nprior) {
                const uint4 raw = *(const uint4*)(vbase + (size_t)(j0 + p) * HD + 8 * ql);
                const uint32_t d4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f16x2 h = as_h2(d4[i]);
                    vv[2 * i] = (float)h.x;
                    vv[2 * i + 1] = (float)h.y;
                }
            } else {
#pragma unroll
                for (int d = 0; d < 8; ++d) vv[d] = vtail[p - nprior][8 * ql + d];
            }
#pragma unroll
            for (int r = 0; r < 2 * ATT_TQ; ++r) {
                const float pr = sc[r][p];
#pragma unroll
                for (int d = 0; d < 8; ++d) o[r][d] += pr * vv[d];
            }
        }
#pragma unroll
        for (int r = 0; r < 2 * ATT_TQ; ++r)
#pragma unroll
            for (int d = 0; d < 8; ++d) ored[quad][r][ql][d] = o[r][d];
        __syncthreads();
        for (int idx = tid; idx < 2 * tq * HD; idx += ATT_THREADS) {
            const int r = idx / HD, d = idx % HD;
            float acc = 0.f;
#pragma unroll
            for (int q = 0; q < 16; ++q) acc += ored[q][r][d / 8][d % 8];
            const int t = t0 + r / 2, hh = r % 2;
            float* dst = part + ((size_t)t * 2 + hh) * PART_STRIDE;
            dst[d] = acc;
            if (d == 0) {
                dst[HD] = mrow[r];
                dst[HD + 1] = lrow[r];
            }
        }
        __syncthreads();
    }

    // Last-arriving split of this group merges all partials.
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const int prev = atomicAdd(&a.counters[g], 1);
        is_last = (prev == S - 1);
    }
    __syncthreads();
    if (!is_last) return;
    __threadfence();
    const float* gpart = a.part + (size_t)g * S * MAXM * 2 * PART_STRIDE;
    for (int idx = tid; idx < M * 2 * HD; idx += ATT_THREADS) {
        const int t = idx / (2 * HD), hh = (idx / HD) % 2, d = idx % HD;
        float mx = -__builtin_inff();
        for (int ss = 0; ss < S; ++ss) mx = fmaxf(mx, gpart[((size_t)ss * MAXM * 2 + t * 2 + hh) * PART_STRIDE + HD]);
        float L = 0.f, O = 0.f;
        for (int ss = 0; ss < S; ++ss) {
            const float* pp = gpart + ((size_t)ss * MAXM * 2 + t * 2 + hh) * PART_STRIDE;
            const float m = pp[HD];
            if (m == -__builtin_inff()) continue;
            const float w = expf(m - mx);
            L += w * pp[HD + 1];
            O += w * pp[d];
        }
        a.out[(size_t)t * H + (2 * g + hh) * HD + d] = f2h(O / L);
    }
    if (tid == 0) a.counters[g] = 0;
}

hipError_t launch_attention(const AttnArgs& a, int mt, hipStream_t s) {
    const dim3 grid(ATTN_SPLITS, NKV);
    if (mt == 1)
        hipLaunchKernelGGL(attention_kernel<1>, grid, dim3(ATT_THREADS), 0, s, a);
    else
        hipLaunchKernelGGL(attention_kernel<MAXM>, grid, dim3(ATT_THREADS), 0, s, a);
    return hipGetLastError();
}

}  // namespace icua
