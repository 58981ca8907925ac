// Qwen3-VL vision tower on gfx950: patchify, patch embedding with the interpolated position
// table, 24 pre-norm blocks (2D RoPE, bidirectional attention, GELU-tanh MLP), three DeepStack
// mergers after blocks 5, 11 and 17, and the final merger (Sources/Engine/Engine.swift:317-473;
// Shaders.swift:59-454).  Weights are fp16 [out][in] matrices with float32 biases and norms.
//
// Every projection is one matrix-core GEMM (v_mfma_f32_16x16x32_f16) with its elementwise
// work in the epilogue: bias, position table, residual add, GELU (tanh or erf) with the fp16
// rounding of the next GEMM's operand, and for QKV the 2D RoPE of q and k with a head-major
// fp16 split and V stored transposed for the attention.  Attention is one flash-style kernel
// per (head, 64 queries) on the matrix cores with an online softmax.  fp16 rounding points are
// those of the reference engine: LayerNorm outputs, q / k / v, probabilities, attention output
// and fc1 activations; the residual stream is float32.
#include "icua_device.h"
#include "icua_kernels.h"

namespace icua {
namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// RGB8 [16 gh][16 gw][3] -> fp16 patches in 2 x 2 merge-block order: patch p = 4 block + 2 ir +
// ic, element c * 256 + dy * 16 + dx, value u8 * (2 / 255) - 1 (k_vit_patchify_rgb,
// Shaders.swift:84-111).
__global__ __launch_bounds__(256) void vit_patchify_kernel(const uint8_t* __restrict__ rgb, uint16_t* __restrict__ patches,
                                                           int gh, int gw) {
#pragma clang fp contract(off)
    const int p = blockIdx.x;
    const int mw = gw / 2, blk = p / 4, in = p % 4;
    const int pr = (blk / mw) * 2 + in / 2, pc = (blk % mw) * 2 + in % 2;
    const int img_w = gw * 16;
    for (int i = threadIdx.x; i < VPATCH; i += 256) {
        const int c = i / 256, dy = (i % 256) / 16, dx = i % 16;
        const uint8_t v = rgb[((size_t)(pr * 16 + dy) * img_w + pc * 16 + dx) * 3 + c];
        const float a = (float)v * (2.0f / 255.0f);
        patches[(size_t)p * VPATCH + i] = f2h(a - 1.0f);
    }
}

// LayerNorm (eps 1e-6) over N columns, one wave per row, fp16 out (k_vit_ln1024 / k_vit_ln4096,
// Shaders.swift:116-199): ((x - mean) * rstd) * w + b.
template <int N>
__global__ __launch_bounds__(256) void vit_layernorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                            const float* __restrict__ b, uint16_t* __restrict__ out,
                                                            int rows) {
#pragma clang fp contract(off)
    constexpr int NV = N / 256;
    const int r = blockIdx.x * 4 + threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
    if (r >= rows) return;
    const float4* xr = (const float4*)(x + (size_t)r * N);
    float4 v[NV];
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        v[k] = xr[lane + WAVE * k];
        s += (v[k].x + v[k].y) + (v[k].z + v[k].w);
    }
    const float mean = wave_sum(s) / (float)N;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        v[k].x -= mean;
        v[k].y -= mean;
        v[k].z -= mean;
        v[k].w -= mean;
        ss += (v[k].x * v[k].x + v[k].y * v[k].y) + (v[k].z * v[k].z + v[k].w * v[k].w);
    }
    const float rstd = 1.0f / sqrtf(wave_sum(ss) / (float)N + 1e-6f);
    uint2* o = (uint2*)(out + (size_t)r * N);
#pragma unroll
    for (int k = 0; k < NV; ++k) {
        const int i = lane + WAVE * k;
        const float4 wv = ((const float4*)w)[i], bv = ((const float4*)b)[i];
        const uint32_t h0 = f2h(v[k].x * rstd * wv.x + bv.x), h1 = f2h(v[k].y * rstd * wv.y + bv.y);
        const uint32_t h2 = f2h(v[k].z * rstd * wv.z + bv.z), h3 = f2h(v[k].w * rstd * wv.w + bv.w);
        o[i] = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
    }
}

// Barrier for LDS filled by global-to-LDS loads: this wave waits until at most `pending` of its
// vector-memory loads are outstanding (expcnt and lgkmcnt at their maximum), then all waves meet.
// __syncthreads() would also drain every load in flight, which empties the load pipeline; the
// empty asm statements keep the compiler from moving memory accesses across the barrier.
template <int pending>
__device__ __forceinline__ void dma_barrier() {
    static_assert(pending >= 0 && pending <= 63, "vmcnt");
    __builtin_amdgcn_s_waitcnt((pending & 15) | (7 << 4) | (15 << 8) | ((pending >> 4) << 14));
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

__device__ __forceinline__ float gelu_tanh(float x) {
    return 0.5f * x * (1.0f + tanhf(0.7978845608028654f * (x + 0.044715f * x * x * x)));
}
__device__ __forceinline__ float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.7071067811865475f)); }

// C[m][n] = sum_k X[m][k] W[n][k] over fp16 X [M][K] and W [N][K].  Workgroup tile BN x BM
// (outputs x tokens), 4 waves in a WN x WM grid; each wave holds TN x TM 16 x 16 accumulators.
// W rows are the A operand and X rows the B operand of v_mfma_f32_16x16x32_f16, so lane l
// ends with C[m = l % 16][n = 4 (l / 16) + i], four consecutive outputs of one token.
//
// K runs in steps of 64 through a ring of S LDS stages filled by direct global-to-LDS loads
// (global_load_lds_dwordx4, 16 bytes a lane), S - 1 steps ahead of the products.  A stage
// holds 128-byte rows; the 16-byte chunk c of row r sits at chunk c ^ (r % 8), so the 16 rows
// of a fragment read spread over the banks.  Token rows past M read row M - 1 and are not
// stored.
template <int BN, int BM, int WN, int WM, int MODE, int S = 4>
__global__ __launch_bounds__(256) void vit_gemm_kernel(VitGemmArgs g) {
#pragma clang fp contract(off)
    constexpr int TN = BN / WN / 16, TM = BM / WM / 16, BK = 64;
    constexpr int WLOADS = (BN + BM) / 8;  // 1 KiB wave loads per stage (8 rows each)
    constexpr int L = WLOADS / 4;          // per wave
    static_assert(WN * WM == 4 && TN >= 1 && TM >= 1 && WLOADS % 4 == 0 && S >= 2 && (S - 2) * L <= 63, "tile");
    static_assert(MODE != VG_QKV || (BN == 64 && WN == 1), "the RoPE pairs (d, d + 32) of a head stay in one lane");
    __shared__ __align__(1024) uint8_t ring[S][(BN + BM) * 128];
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE, r16 = lane & 15, q4 = lane >> 4;
    const int wn = wave / WM, wm = wave % WM;
    const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
    const int K = g.K, nk = K / BK;
    // Lane l of wave load j (rows 8 j .. 8 j + 7 of the stage: W rows first, then X rows) lands at
    // row 8 j + l / 8, chunk l % 8, and reads source chunk (l % 8) ^ (l / 8).
    const int lrow = lane >> 3, lchunk = (lane & 7) ^ lrow;
    auto issue = [&](int kt) __attribute__((always_inline)) {
        uint8_t* st = ring[kt % S];
        const int k0 = kt * BK + 8 * lchunk;
#pragma unroll
        for (int u = 0; u < L; ++u) {
            const int j = wave + 4 * u, row = 8 * j + lrow;
            const uint16_t* src = row < BN ? g.W + (size_t)(n0 + row) * K + k0
                                           : g.X + (size_t)min(m0 + row - BN, g.M - 1) * K + k0;
            __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(st + 1024 * j), 16, 0, 0);
        }
    };
    auto frag = [&](const uint8_t* st, int row, int chunk) __attribute__((always_inline)) {
        return *(const v8h*)(st + row * 128 + ((chunk ^ (row & 7)) << 4));
    };

    f32x4 acc[TN][TM];
#pragma unroll
    for (int a = 0; a < TN; ++a)
#pragma unroll
        for (int b = 0; b < TM; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int p = 0; p < S - 1; ++p) issue(min(p, nk - 1));
    for (int kt = 0; kt < nk; ++kt) {
        // This wave's loads of step kt have landed once at most (S - 2) * L newer ones are
        // outstanding; after the barrier every wave's have, and the stage read in step kt - 1
        // is free (its reads completed before each wave's products of that step).
        dma_barrier<(S - 2) * L>();
        issue(min(kt + S - 1, nk - 1));  // past the end: a repeat into a stage no one reads again
        const uint8_t* st = ring[kt % S];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            v8h af[TN], bf[TM];
#pragma unroll
            for (int a = 0; a < TN; ++a) af[a] = frag(st, (wn * TN + a) * 16 + r16, 4 * ks + q4);
#pragma unroll
            for (int b = 0; b < TM; ++b) bf[b] = frag(st, BN + (wm * TM + b) * 16 + r16, 4 * ks + q4);
#pragma unroll
            for (int a = 0; a < TN; ++a)
#pragma unroll
                for (int b = 0; b < TM; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[a], bf[b], acc[a][b], 0, 0, 0);
        }
    }
    __builtin_amdgcn_s_waitcnt(0);  // no load is in flight when the workgroup ends

    const int N = g.N;
#pragma unroll
    for (int b = 0; b < TM; ++b) {
        const int m = m0 + (wm * TM + b) * 16 + r16;
        if (m >= g.M) continue;
        if constexpr (MODE == VG_QKV) {
            // Head n0 / 64 of the fused rows: q heads 0-15, k heads 16-31, v heads 32-47.  Lane
            // holds dims d = 16 a + 4 q4 + i; pairs (d, d + 32) are accumulators a and a + 2.
            const int hh = blockIdx.x;
            float v[4][4];
#pragma unroll
            for (int a = 0; a < 4; ++a) {
                const float4 bv = *(const float4*)(g.bias + n0 + 16 * a + 4 * q4);
                v[a][0] = acc[a][b][0] + bv.x;
                v[a][1] = acc[a][b][1] + bv.y;
                v[a][2] = acc[a][b][2] + bv.z;
                v[a][3] = acc[a][b][3] + bv.w;
            }
            if (hh < 2 * VNH) {
#pragma unroll
                for (int a = 0; a < 2; ++a)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int d = 16 * a + 4 * q4 + i;
                        const float2 cs = *(const float2*)(g.rope + ((size_t)m * 32 + d) * 2);
                        const float x0 = v[a][i], x1 = v[a + 2][i];
                        v[a][i] = x0 * cs.x - x1 * cs.y;
                        v[a + 2][i] = x1 * cs.x + x0 * cs.y;
                    }
                uint16_t* dst = (hh < VNH ? g.q + (size_t)hh * g.ld * VHD : g.k + (size_t)(hh - VNH) * g.ld * VHD) +
                                (size_t)m * VHD;
#pragma unroll
                for (int a = 0; a < 4; ++a) {
                    const uint32_t h0 = f2h(v[a][0]), h1 = f2h(v[a][1]), h2 = f2h(v[a][2]), h3 = f2h(v[a][3]);
                    *(uint2*)(dst + 16 * a + 4 * q4) = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
                }
            } else {
                uint16_t* dst = g.vt + (size_t)(hh - 2 * VNH) * VHD * g.ld + m;
#pragma unroll
                for (int a = 0; a < 4; ++a)
#pragma unroll
                    for (int i = 0; i < 4; ++i) dst[(size_t)(16 * a + 4 * q4 + i) * g.ld] = f2h(v[a][i]);
            }
        } else {
#pragma unroll
            for (int a = 0; a < TN; ++a) {
                const int n = n0 + (wn * TN + a) * 16 + 4 * q4;
                const float4 bv = *(const float4*)(g.bias + n);
                float4 v = make_float4(acc[a][b][0] + bv.x, acc[a][b][1] + bv.y, acc[a][b][2] + bv.z, acc[a][b][3] + bv.w);
                const size_t o = (size_t)m * N + n;
                if constexpr (MODE == VG_F32) {
                    *(float4*)(g.outf + o) = v;
                } else if constexpr (MODE == VG_F32_ADD) {
                    float4 r = *(const float4*)(g.outf + o);
                    r.x += v.x;
                    r.y += v.y;
                    r.z += v.z;
                    r.w += v.w;
                    *(float4*)(g.outf + o) = r;
                } else if constexpr (MODE == VG_F32_POS) {
                    const float4 p = *(const float4*)(g.pos + o);
                    *(float4*)(g.outf + o) = make_float4(v.x + p.x, v.y + p.y, v.z + p.z, v.w + p.w);
                } else {
                    float e[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                    for (int i = 0; i < 4; ++i) e[i] = MODE == VG_GELU_TANH ? gelu_tanh(e[i]) : gelu_erf(e[i]);
                    const uint32_t h0 = f2h(e[0]), h1 = f2h(e[1]), h2 = f2h(e[2]), h3 = f2h(e[3]);
                    *(uint2*)(g.outh + o) = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
                }
            }
        }
    }
}

// Bidirectional attention of one head over all patches (k_vit_attn, Shaders.swift:294-395),
// grid (ceil(np / 64), 16 heads), 8 waves.  Waves w and w + 4 own the same 16 queries,
// 64 x + 16 (w % 4) .. + 15 (lane l: query l % 16), and split the key blocks in two halves, so the
// serial chain of block loads is half as long.  Per block of 64 keys: S^T = K . Q^T on
// v_mfma_f32_16x16x32_f16 (lane: keys 16 j + 4 (l / 16) + i of sub-block j), scaled by 1/8; an
// online softmax per query column; O^T += V^T . P^T on v_mfma_f32_16x16x16_f16 with the fp16
// probabilities straight from the score registers and V^T read from LDS.  The two halves'
// (max, sum, O) are combined through LDS.  Keys past np are masked (their rows hold finite
// values).
__global__ __launch_bounds__(512) void vit_attention_kernel(const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                            const uint16_t* __restrict__ vt, uint16_t* __restrict__ out,
                                                            int np, int ld) {
    constexpr int ROW = 72, TILE = 64 * ROW;
    // [key half][K, V^T][buffer].  V^T rows with (row / 8) odd hold their 4-key chunks pairwise
    // swapped (chunk c at c ^ 1): the P.V reads of 16 rows x one chunk then cover all 32 banks.
    __shared__ __align__(16) uint16_t lds[2][2][2][TILE];
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE, r16 = lane & 15, q4 = lane >> 4;
    const int grp = wave >> 2, gt = tid & 255;
    const int h = blockIdx.y;
    const int qt = blockIdx.x * 64 + (wave & 3) * 16 + r16;
    const uint16_t* qh = q + (size_t)h * ld * VHD;
    const uint16_t* kh = k + (size_t)h * ld * VHD;
    const uint16_t* vh = vt + (size_t)h * VHD * ld;
    const int qc = min(qt, np - 1);
    v8h qf[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) qf[ks] = *(const v8h*)(qh + (size_t)qc * VHD + 32 * ks + 8 * q4);

    // Register-staged block loads by the 256 threads of a half (macros: see vit_gemm_kernel).
    uint4 kr[2], vr[2];
#define VA_GLOAD(blk_)                                                              \
    do {                                                                            \
        _Pragma("unroll") for (int c = 0; c < 2; ++c) {                              \
            const int idx = gt + 256 * c, row = idx >> 3, col = (idx & 7) * 8;       \
            kr[c] = *(const uint4*)(kh + (size_t)(64 * (blk_) + row) * VHD + col);   \
            vr[c] = *(const uint4*)(vh + (size_t)row * ld + 64 * (blk_) + col);      \
        }                                                                           \
    } while (0)
#define VA_LSTORE(buf_)                                                             \
    do {                                                                            \
        _Pragma("unroll") for (int c = 0; c < 2; ++c) {                              \
            const int idx = gt + 256 * c, row = idx >> 3, col = (idx & 7) * 8;       \
            *(uint4*)&lds[grp][0][buf_][row * ROW + col] = kr[c];                    \
            const uint4 vv_ = ((row >> 3) & 1) ? make_uint4(vr[c].z, vr[c].w, vr[c].x, vr[c].y) : vr[c]; \
            *(uint4*)&lds[grp][1][buf_][row * ROW + col] = vv_;                      \
        }                                                                           \
    } while (0)

    const int nblk = (np + 63) / 64, nh = (nblk + 1) / 2;
    const int b0 = grp * nh, bend = min(nblk, b0 + nh);  // this half's blocks [b0, bend)
    float m_run = -__builtin_inff(), l_run = 0.f;
    f32x4 O[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) O[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    VA_GLOAD(min(b0, nblk - 1));
    VA_LSTORE(0);
    __syncthreads();
    for (int it = 0; it < nh; ++it) {
        const int blk = b0 + it, buf = it & 1;
        VA_GLOAD(min(blk + 1, nblk - 1));  // unconditional (a valid block either way)
        if (blk < bend) {
            const uint16_t* Ks = lds[grp][0][buf];
            const uint16_t* Vs = lds[grp][1][buf];
            f32x4 S[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                S[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 2; ++ks) {
                    const v8h kf = *(const v8h*)&Ks[(16 * j + r16) * ROW + 32 * ks + 8 * q4];
                    S[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qf[ks], S[j], 0, 0, 0);
                }
            }
            float mb = -__builtin_inff();
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = 64 * blk + 16 * j + 4 * q4 + i;
                    S[j][i] = key < np ? S[j][i] * 0.125f : -__builtin_inff();
                    mb = fmaxf(mb, S[j][i]);
                }
            mb = max_x4(mb);  // finite: key 64 blk < np
            const float m_new = fmaxf(m_run, mb);
            const float corr = expf(m_run - m_new);
            float ls = 0.f;
            v4h P[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float p = expf(S[j][i] - m_new);
                    ls += p;
                    P[j][i] = (_Float16)p;
                }
            l_run = l_run * corr + sum_x4(ls);
            m_run = m_new;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) O[dt][i] *= corr;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const v4h vf = *(const v4h*)&Vs[(16 * dt + r16) * ROW + 4 * ((4 * j + q4) ^ (r16 >> 3))];
                    O[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf, P[j], O[dt], 0, 0, 0);
                }
            }
        }
        VA_LSTORE(buf ^ 1);  // the last fills an idle buffer
        __syncthreads();
    }
#undef VA_GLOAD
#undef VA_LSTORE
    // Combine the halves: the second half's state goes through LDS (every tile read is done).
    float* xo = (float*)&lds[0][0][0][0];  // [256 lanes][18]
    if (grp == 1) {
        float* d = xo + (size_t)gt * 18;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
            for (int i = 0; i < 4; ++i) d[4 * dt + i] = O[dt][i];
        d[16] = m_run;
        d[17] = l_run;
    }
    __syncthreads();
    if (grp == 0 && qt < np) {
        const float* d = xo + (size_t)gt * 18;
        const float m1 = d[16], m = fmaxf(m_run, m1);
        const float f0 = expf(m_run - m), f1 = expf(m1 - m);  // m is finite: the first half is never empty
        const float inv = 1.0f / (l_run * f0 + d[17] * f1);
        uint16_t* dst = out + (size_t)qt * VH + h * VHD;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) o[i] = (O[dt][i] * f0 + d[4 * dt + i] * f1) * inv;
            const uint32_t h0 = f2h(o[0]), h1 = f2h(o[1]), h2 = f2h(o[2]), h3 = f2h(o[3]);
            *(uint2*)(dst + 16 * dt + 4 * q4) = make_uint2(h0 | (h1 << 16), h2 | (h3 << 16));
        }
    }
}

template <int BN, int BM, int WN, int WM, int MODE, int S = 4>
hipError_t gemm(const VitGemmArgs& g, hipStream_t s) {
    if (g.N % BN || g.K % 64 || g.M < 1) return hipErrorInvalidValue;
    const dim3 grid(g.N / BN, (g.M + BM - 1) / BM);
    hipLaunchKernelGGL((vit_gemm_kernel<BN, BM, WN, WM, MODE, S>), grid, dim3(256), 0, s, g);
    return hipGetLastError();
}

template <int N>
hipError_t layernorm(const float* x, const float* w, const float* b, uint16_t* out, int rows, hipStream_t s) {
    hipLaunchKernelGGL((vit_layernorm_kernel<N>), dim3((rows + 3) / 4), dim3(256), 0, s, x, w, b, out, rows);
    return hipGetLastError();
}

#define VCK(x)                            \
    do {                                  \
        const hipError_t e_ = (x);        \
        if (e_ != hipSuccess) return e_;  \
    } while (0)

hipError_t merger(const VitMerger& mg, const uint16_t* xn, int nvis, uint16_t* hbuf, float* out, hipStream_t s) {
    VitGemmArgs g{};
    g.X = xn;
    g.W = mg.fc1w;
    g.bias = mg.fc1b;
    g.outh = hbuf;
    g.M = nvis;
    g.N = MH;
    g.K = MH;
    VCK((gemm<32, 64, 2, 2, VG_GELU_ERF>(g, s)));
    g = VitGemmArgs{};
    g.X = hbuf;
    g.W = mg.fc2w;
    g.bias = mg.fc2b;
    g.outf = out;
    g.M = nvis;
    g.N = H;
    g.K = MH;
    return gemm<32, 32, 2, 2, VG_F32>(g, s);
}

}  // namespace

hipError_t launch_vision(const VitWeights& w, const VitBuffers& b, int gh, int gw, hipStream_t s) {
    const int np = gh * gw, nvis = np / 4;
    if (gh < 2 || gw < 2 || gh % 2 || gw % 2 || np > NPATCH_MAX) return hipErrorInvalidValue;
    hipLaunchKernelGGL(vit_patchify_kernel, dim3(np), dim3(256), 0, s, b.rgb, b.patches, gh, gw);
    VCK(hipGetLastError());
    VitGemmArgs g{};
    g.X = b.patches;
    g.W = w.patch_w;
    g.bias = w.patch_b;
    g.outf = b.x;
    g.pos = b.pos;
    g.M = np;
    g.N = VH;
    g.K = VPATCH;
    VCK((gemm<32, 64, 2, 2, VG_F32_POS>(g, s)));
    int ds = 0;
    for (int l = 0; l < VLAYERS; ++l) {
        const VitBlock& L = w.blk[l];
        VCK(layernorm<VH>(b.x, L.n1w, L.n1b, b.xn, np, s));
        g = VitGemmArgs{};
        g.X = b.xn;
        g.W = L.qkvw;
        g.bias = L.qkvb;
        g.rope = b.rope;
        g.q = b.q;
        g.k = b.k;
        g.vt = b.vt;
        g.ld = NPATCH_MAX;
        g.M = np;
        g.N = VQKV;
        g.K = VH;
        VCK((gemm<64, 64, 1, 4, VG_QKV>(g, s)));
        hipLaunchKernelGGL(vit_attention_kernel, dim3((np + 63) / 64, VNH), dim3(512), 0, s, b.q, b.k, b.vt, b.attn, np,
                           NPATCH_MAX);
        VCK(hipGetLastError());
        g = VitGemmArgs{};
        g.X = b.attn;
        g.W = L.projw;
        g.bias = L.projb;
        g.outf = b.x;
        g.M = np;
        g.N = VH;
        g.K = VH;
        VCK((gemm<32, 64, 2, 2, VG_F32_ADD>(g, s)));
        VCK(layernorm<VH>(b.x, L.n2w, L.n2b, b.xn, np, s));
        g = VitGemmArgs{};
        g.X = b.xn;
        g.W = L.fc1w;
        g.bias = L.fc1b;
        g.outh = b.h;
        g.M = np;
        g.N = VFF;
        g.K = VH;
        VCK((gemm<128, 64, 2, 2, VG_GELU_TANH, 3>(g, s)));
        g = VitGemmArgs{};
        g.X = b.h;
        g.W = L.fc2w;
        g.bias = L.fc2b;
        g.outf = b.x;
        g.M = np;
        g.N = VH;
        g.K = VFF;
        VCK((gemm<32, 64, 2, 2, VG_F32_ADD>(g, s)));
        if (l == 5 || l == 11 || l == 17) {
            // DeepStack merger: LayerNorm over each 2 x 2 block's 4096 values (Engine.swift:420-447).
            VCK(layernorm<MH>(b.x, w.mg[ds].nw, w.mg[ds].nb, b.xn, nvis, s));
            VCK(merger(w.mg[ds], b.xn, nvis, b.h, b.ds[ds], s));
            ++ds;
        }
    }
    // Final merger: LayerNorm per patch, then 2 x 2 blocks as rows of 4096 (Engine.swift:450-472).
    VCK(layernorm<VH>(b.x, w.mg[3].nw, w.mg[3].nb, b.xn, np, s));
    return merger(w.mg[3], b.xn, nvis, b.h, b.pooler, s);
}

}  // namespace icua
