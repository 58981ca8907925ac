// Group-wise dequant-GEMV for batch-1 decode (and passes of up to MAXM tokens), gfx950.
//
// Replaces the reference's dot64_row / reduce8 GEMV family (Shaders.swift:480-631) and the
// GEMV parts of k_attn_in, k_o_proj, k_mlp_in, k_mlp_out and k_lm_head (Shaders.swift:714-834,
// 1293-1495).
//
// Mapping.  A weight row is streamed in 1 KiB chunks: lane l of a wave loads bytes
// [1024 c + 16 l, +16) of chunk c with one 128-bit load, so one wave instruction reads 1 KiB
// of one row, fully coalesced.  For both q4 (group 64 = 32 bytes) and q8 (group 32 = 32 bytes)
// that slice lies in group 32 c + l / 2.  A wave keeps R rows in flight, accumulates per-lane
// partials in fp32 with v_dot2c_f32_f16 on exactly unpacked codes, applies the group scale
// per lane, and reduces the R rows together with permlane swaps and DPP (reduce_rows).
//
// Activations: the workgroup stages the fp16 GEMV input of every token of the pass in LDS,
// in a per-format pair order so that a 128-bit LDS read yields the f16x2 operands that match
// the unpacked code pairs.  The prologue optionally applies RMSNorm (Shaders.swift:634-657):
// x * rsqrt(mean(x^2) + eps) * w rounded to fp16, exactly the reference rounding point.
#include "icua_device.h"
#include "icua_kernels.h"

namespace icua {

template <int FMT>
struct FmtT;
template <>
struct FmtT<FMT_Q4> {
    static constexpr int E = 32;    // elements per lane per chunk
    static constexpr int BLK = 8;   // pair-permutation block
    static constexpr int XP = 16;   // f16x2 operands per lane per chunk
    static constexpr int row_bytes(int K) { return K / 2; }
};
template <>
struct FmtT<FMT_Q8> {
    static constexpr int E = 16;
    static constexpr int BLK = 4;
    static constexpr int XP = 8;
    static constexpr int row_bytes(int K) { return K; }
};
template <>
struct FmtT<FMT_F16> {
    static constexpr int E = 8;
    static constexpr int BLK = 2;
    static constexpr int XP = 4;
    static constexpr int row_bytes(int K) { return 2 * K; }
};

// Position inside a permutation block where element i of the block is stored.
template <int FMT>
__device__ __forceinline__ int perm_pos(int i) {
    if constexpr (FMT == FMT_Q4) {
        // block [x0..x7] stored as [x0 x4 x1 x5 x2 x6 x3 x7]
        return (i & 3) * 2 + (i >> 2);
    } else if constexpr (FMT == FMT_Q8) {
        // block [x0..x3] stored as [x0 x2 x1 x3]
        return (i & 1) * 2 + (i >> 1);
    } else {
        return i;
    }
}

// Stage the fp16 GEMV inputs of M rows into LDS (pair order) and the per-lane-slice sums.
template <int FMT, int K, int PRO>
__device__ __forceinline__ void stage_inputs(const GemvArgs& a, int M, int row0, uint16_t* xs, float* xsum,
                                             float* red) {
    constexpr int E = FmtT<FMT>::E, BLK = FmtT<FMT>::BLK;
    const int tid = threadIdx.x;
    const int nthr = blockDim.x;
    const int wave = tid / WAVE, lane = tid % WAVE;
    for (int t = 0; t < M; ++t) {
        float scale = 1.f;
        const int r = row0 + t;
        if constexpr (PRO == PRO_NORM) {
            const float* xr = (const float*)a.x + (size_t)r * K;
            float ss = 0.f;
            for (int k = tid; k < K; k += nthr) {
                float v = xr[k];
                ss += v * v;
            }
            ss = wave_sum(ss);
            if (lane == 0) red[wave] = ss;
            __syncthreads();
            float tot = 0.f;
            for (int w = 0; w < nthr / WAVE; ++w) tot += red[w];
            scale = 1.0f / sqrtf(tot / (float)K + EPS);
            __syncthreads();
        }
        for (int k = tid; k < K; k += nthr) {
            uint16_t hv;
            if constexpr (PRO == PRO_NORM) {
                const float* xr = (const float*)a.x + (size_t)r * K;
                hv = f2h(xr[k] * scale * a.norm_w[k]);
            } else if constexpr (PRO == PRO_F32) {
                hv = f2h(((const float*)a.x)[(size_t)r * K + k]);
            } else {
                hv = ((const uint16_t*)a.x)[(size_t)r * K + k];
            }
            const int blk = k / BLK, i = k % BLK;
            xs[t * K + blk * BLK + perm_pos<FMT>(i)] = hv;
        }
    }
    __syncthreads();
    // Per-lane-slice sums X (slices of E elements).
    constexpr int NS = K / E;
    for (int idx = tid; idx < M * NS; idx += nthr) {
        const int t = idx / NS, s = idx % NS;
        const uint16_t* p = xs + t * K + s * E;
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < E; ++i) acc += h2f(p[i]);
        xsum[idx] = acc;
    }
    __syncthreads();
}

// Per-lane partial of one row chunk for one token.
template <int FMT>
__device__ __forceinline__ float chunk_partial(const uint4& w, uint32_t sbv, const f16x2* x, float X) {
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    if constexpr (FMT == FMT_Q4) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f16x2 p[4];
            q4_unpack(d[j], p);
#pragma unroll
            for (int i = 0; i < 4; ++i) acc = dot2(p[i], x[4 * j + i], acc);
        }
        const f16x2 sb2 = as_h2(sbv);
        const float s = (float)sb2.x, b = (float)sb2.y;
        return (16.f * s) * (acc - X) + b * X;
    } else if constexpr (FMT == FMT_Q8) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f16x2 p[2];
            q8_unpack(d[j], p);
            acc = dot2(p[0], x[2 * j], acc);
            acc = dot2(p[1], x[2 * j + 1], acc);
        }
        const float s = h2f((uint16_t)sbv);
        return s * (acc - 1152.f * X);
    } else {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = dot2(as_h2(d[j]), x[j], acc);
        return acc;
    }
}

template <int FMT, int K, int R, int MT, int PRO, int EPI>
__global__ __launch_bounds__(256) void gemv_kernel(GemvArgs a) {
    const State* st = a.st;
    if (st->done) return;
    constexpr int E = FmtT<FMT>::E, XP = FmtT<FMT>::XP;
    constexpr int RB = FmtT<FMT>::row_bytes(K);
    constexpr int NCH = RB / 1024;
    static_assert(RB % 1024 == 0, "row must be a whole number of 1 KiB chunks");
    constexpr int NS = K / E;

    // Rows of the input to use: a contiguous run [row0, row0 + M).
    int M, row0;
    if (a.m_fixed > 0) {
        M = a.m_fixed;
        row0 = 0;
    } else {
        M = st->n;
        row0 = 0;
        if constexpr (EPI == EPI_ARGMAX) {
            if (st->logits_rows != M) {  // argmax (and logits) of the last row only
                row0 = M - 1;
                M = 1;
            }
        }
    }
    if (M > MT) M = MT;

    extern __shared__ __align__(16) uint8_t smem[];
    uint16_t* xs = (uint16_t*)smem;                       // [MT][K] fp16, pair order
    float* xsum = (float*)(smem + MT * K * 2);            // [MT][NS]
    float* red = xsum + MT * NS;                          // [8]
    stage_inputs<FMT, K, PRO>(a, M, row0, xs, xsum, red);

    const int lane = threadIdx.x % WAVE;
    const int wave = threadIdx.x / WAVE;
    const int waves_per_blk = blockDim.x / WAVE;
    const int gw = blockIdx.x * waves_per_blk + wave;
    const int nw = gridDim.x * waves_per_blk;
    const int nblocks = (EPI == EPI_SWIGLU) ? (FF / (R / 2)) : (a.N / R);

    // Single-token fast path keeps its operands in registers for the whole kernel.
    f16x2 xr[MT == 1 ? NCH * XP : 1];
    float Xr[MT == 1 ? NCH : 1];
    if constexpr (MT == 1) {
#pragma unroll
        for (int c = 0; c < NCH; ++c) {
            const int s = c * WAVE + lane;
            const uint4* src = (const uint4*)(xs + s * E);
#pragma unroll
            for (int q = 0; q < XP / 4; ++q) {
                uint4 v = src[q];
                xr[c * XP + 4 * q + 0] = as_h2(v.x);
                xr[c * XP + 4 * q + 1] = as_h2(v.y);
                xr[c * XP + 4 * q + 2] = as_h2(v.z);
                xr[c * XP + 4 * q + 3] = as_h2(v.w);
            }
            Xr[c] = xsum[s];
        }
    }

    float best_v[MT];
    int best_i[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        best_v[t] = -__builtin_inff();
        best_i[t] = 0x7fffffff;
    }

    for (int blk = gw; blk < nblocks; blk += nw) {
        int rows[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if constexpr (EPI == EPI_SWIGLU)
                rows[r] = (r < R / 2) ? blk * (R / 2) + r : FF + blk * (R / 2) + (r - R / 2);
            else
                rows[r] = blk * R + r;
        }
        uint4 w[R][NCH];
        uint32_t sbv[R][NCH];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const uint8_t* rowp = a.w + (size_t)rows[r] * RB;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                w[r][c] = ((const uint4*)(rowp + c * 1024))[lane];
                if constexpr (FMT == FMT_Q4)
                    sbv[r][c] = ((const uint32_t*)a.sb)[(size_t)rows[r] * (K / 64) + 32 * c + lane / 2];
                else if constexpr (FMT == FMT_Q8)
                    sbv[r][c] = ((const uint16_t*)a.sb)[(size_t)rows[r] * (K / 32) + 32 * c + lane / 2];
                else
                    sbv[r][c] = 0;
            }
        }
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t >= M) break;
            float part[R];
#pragma unroll
            for (int r = 0; r < R; ++r) part[r] = 0.f;
#pragma unroll
            for (int c = 0; c < NCH; ++c) {
                const f16x2* xp;
                float X;
                f16x2 xl[MT == 1 ? 1 : XP];
                if constexpr (MT == 1) {
                    xp = xr + c * XP;
                    X = Xr[c];
                } else {
                    const int s = c * WAVE + lane;
                    const uint4* src = (const uint4*)(xs + t * K + s * E);
#pragma unroll
                    for (int q = 0; q < XP / 4; ++q) {
                        uint4 v = src[q];
                        xl[4 * q + 0] = as_h2(v.x);
                        xl[4 * q + 1] = as_h2(v.y);
                        xl[4 * q + 2] = as_h2(v.z);
                        xl[4 * q + 3] = as_h2(v.w);
                    }
                    xp = xl;
                    X = xsum[t * NS + s];
                }
#pragma unroll
                for (int r = 0; r < R; ++r) part[r] += chunk_partial<FMT>(w[r][c], sbv[r][c], xp, X);
            }
            const float y = reduce_rows<R>(part, lane);
            const int r = lane / (WAVE / R);
            const bool writer = (lane % (WAVE / R)) == 0;
            const int tok = row0 + t;
            if constexpr (EPI == EPI_STORE) {
                if (writer) a.y[(size_t)tok * a.N + rows[r]] = y;
            } else if constexpr (EPI == EPI_RESID) {
                if (writer) {
                    float* xo = a.y + (size_t)tok * a.N + rows[r];
                    float v = *xo + y;
                    if (a.ds) {  // DeepStack residual of a visual row (Shaders.swift:696-707)
                        const int vrow = a.ds_row0 + tok - st->vis_offset;
                        if (st->vis_offset >= 0 && vrow >= 0 && vrow < st->n_vis)
                            v = v + a.ds[(size_t)vrow * H + rows[r]];
                    }
                    *xo = v;
                }
            } else if constexpr (EPI == EPI_SWIGLU) {
                const float up = __shfl_xor(y, 32);  // row r + R/2 sits 32 lanes up
                if (writer && r < R / 2) {
                    const float g = y;
                    const float act = (g / (1.f + expf(-g))) * up;
                    a.h[(size_t)tok * FF + rows[r]] = f2h(act);
                }
            } else {  // EPI_ARGMAX
                if (writer && a.logits && st->logits_rows > 0)  // single-row mode writes logits row 0
                    a.logits[(size_t)(tok - row0) * VOCAB + rows[r]] = y;
                argmax_merge(best_v[t], best_i[t], y, rows[r]);
            }
        }
    }
    if constexpr (EPI == EPI_ARGMAX) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
            if (t >= M) break;
            float v = best_v[t];
            int i = best_i[t];
            wave_argmax(v, i);
            if (lane == 0) {
                a.pval[(size_t)(row0 + t) * LMH_WAVES + gw] = v;
                a.pidx[(size_t)(row0 + t) * LMH_WAVES + gw] = i;
            }
        }
    }
}

template <int FMT, int K, int R, int MT, int PRO, int EPI>
static hipError_t launch_one(const GemvArgs& a, int blocks, hipStream_t s) {
    constexpr int E = FmtT<FMT>::E;
    size_t lds = (size_t)MT * K * 2 + (size_t)MT * (K / E) * 4 + 64;
    auto kern = gemv_kernel<FMT, K, R, MT, PRO, EPI>;
    static bool attr_set = false;
    if (!attr_set) {
        hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        attr_set = true;
    }
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(256), lds, s, a);
    return hipGetLastError();
}

// Dispatch on (format, op).  `mt` selects the single-token (1) or multi-token (MAXM) kernel.
template <int FMT>
static hipError_t gemv_fmt(GemvOp op, const GemvArgs& a, int mt, hipStream_t s) {
    const bool one = (mt == 1);
    switch (op) {
        case GEMV_QKV:  // RMSNorm -> fused QKV rows, fp32 out
            return one ? launch_one<FMT, H, 4, 1, PRO_NORM, EPI_STORE>(a, QKV / 16, s)
                       : launch_one<FMT, H, 4, MAXM, PRO_NORM, EPI_STORE>(a, QKV / 16, s);
        case GEMV_O:  // fp16 attention output -> O rows, residual add
            return one ? launch_one<FMT, H, 4, 1, PRO_F16, EPI_RESID>(a, H / 16, s)
                       : launch_one<FMT, H, 4, MAXM, PRO_F16, EPI_RESID>(a, H / 16, s);
        case GEMV_GU:  // RMSNorm -> gate|up pairs -> SwiGLU, fp16 out
            return one ? launch_one<FMT, H, 8, 1, PRO_NORM, EPI_SWIGLU>(a, FF / 16, s)
                       : launch_one<FMT, H, 8, MAXM, PRO_NORM, EPI_SWIGLU>(a, FF / 16, s);
        case GEMV_DOWN:  // fp16 SwiGLU output -> down rows, residual add
            return one ? launch_one<FMT, FF, 4, 1, PRO_F16, EPI_RESID>(a, H / 16, s)
                       : launch_one<FMT, FF, 4, MAXM, PRO_F16, EPI_RESID>(a, H / 16, s);
        case GEMV_LMHEAD:  // final RMSNorm -> tied embedding rows -> argmax partials
            return one ? launch_one<FMT, H, 8, 1, PRO_NORM, EPI_ARGMAX>(a, LMH_WAVES / 4, s)
                       : launch_one<FMT, H, 8, MAXM, PRO_NORM, EPI_ARGMAX>(a, LMH_WAVES / 4, s);
        case GEMV_PLAIN_F16IN:  // isolated GEMV: fp16 x in, fp32 y out
            return one ? launch_one<FMT, H, 8, 1, PRO_F16, EPI_STORE>(a, a.blocks, s)
                       : launch_one<FMT, H, 8, MAXM, PRO_F16, EPI_STORE>(a, a.blocks, s);
        case GEMV_PLAIN_F16IN_K6144:
            return one ? launch_one<FMT, FF, 4, 1, PRO_F16, EPI_STORE>(a, a.blocks, s)
                       : launch_one<FMT, FF, 4, MAXM, PRO_F16, EPI_STORE>(a, a.blocks, s);
    }
    return hipErrorInvalidValue;
}

hipError_t launch_gemv(int fmt, GemvOp op, const GemvArgs& a, int mt, hipStream_t s) {
    switch (fmt) {
        case FMT_Q4:
            return gemv_fmt<FMT_Q4>(op, a, mt, s);
        case FMT_Q8:
            return gemv_fmt<FMT_Q8>(op, a, mt, s);
        case FMT_F16:
            return gemv_fmt<FMT_F16>(op, a, mt, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace icua
