// Group-wise dequant-GEMV on the matrix cores, for passes of 1..8 tokens, gfx950.
//
// Replaces the reference's dot64_row / reduce8 GEMV family (Shaders.swift:480-631) and the
// GEMV parts of k_attn_in, k_o_proj, k_mlp_in, k_mlp_out and k_lm_head (Shaders.swift:714-834,
// 1293-1495); math per tools/reference/qwen3vl_ref.py (fp32 activations).
//
// Arithmetic.  y[r] = sum_g sum_{k in g} (s_rg q_rk + b_rg) x_k.  For each group g and token,
// the fp32 activations are written exactly-rounded as 22-bit integers X_k = rint(x_k 2^(21-e_g))
// (e_g = exponent of the group's largest |x|) split into three signed bytes (hi, mid, lo).
// The integer codes q times those bytes go through v_mfma_i32_16x16x64_i8 (q4, group 64) or
// v_mfma_i32_16x16x32_i8 (q8, group 32): the integer partial sums are exact.  Per group:
//   S = 65536 C_hi + 256 C_mid + C_lo,  y += (s 2^(e_g-21)) S + b (2^(e_g-21) sum X_k).
// The only roundings are the 22-bit activation quantisation (<= 2^-22 of the group max) and the
// fp32 group scaling, i.e. fp32-level accuracy with no fp16 activation rounding.  f16 weights
// use v_mfma_f32_16x16x32_f16 with the activation split into fp16 hi + lo parts.
//
// Operand roles.  A (16 "rows") holds activations: row m = 4 t + slice (t = token of the
// pass, slice 3 zero); B (16 "columns") holds 16 weight rows.  Lane l of both operands holds
// row/column l % 16 and K-slot group l / 16; the accumulator lane l holds C[4 (l/16) + i][l % 16],
// so every lane ends with the three slices of one (token, weight row) pair: no cross-lane
// reduction is needed.  A pass covers 4 tokens (int8) or 8 tokens (f16, rows hi/lo).
//
// Layout (repacked once at load, see repack_*): 16-row blocks; each 1 KiB chunk of a block
// holds, for lane l, the 16 bytes it feeds to the matrix core (q4: groups 2c and 2c+1, eight
// bytes each with nibbles ordered so that (v & 0x0F0F0F0F) and (v >> 4 & 0x0F0F0F0F) give the
// bytes in K order).  One wave load is 1 KiB contiguous.  Scales stay row-major [row][K/G].
//
// Work split.  A workgroup owns one 16-row block at a time; its KS waves split the block's
// chunks and reduce their partial sums through LDS in a fixed order (deterministic).  K is
// processed in 2048-wide segments so the activation operands of a segment fit in 32 KiB of LDS.
// Weight loads of a segment are issued before its activation staging, overlapping the
// RMSNorm / slicing prologue with the HBM latency.
#include "icua_device.h"
#include "icua_kernels.h"

namespace icua {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int SEG = 2048;

template <int FMT>
struct TileT;
template <>
struct TileT<FMT_Q4> {
    static constexpr int CHK = 128;  // K per 1 KiB chunk
    static constexpr int G = 64;     // group size
    static constexpr int TOK = 4;    // tokens per pass
};
template <>
struct TileT<FMT_Q8> {
    static constexpr int CHK = 64;
    static constexpr int G = 32;
    static constexpr int TOK = 4;
};
template <>
struct TileT<FMT_F16> {
    static constexpr int CHK = 32;
    static constexpr int G = 32;  // K of one MFMA (no scales)
    static constexpr int TOK = 8;
};

// LDS: activation operands of one segment for every pass of the launch (32 KiB int8 / 64 KiB
// f16 per pass), per-(token, group) factors, per-token RMSNorm scales, the cross-wave partial
// sums and the per-wave sums of squares.
template <int FMT>
struct Smem {
    static constexpr int A_BYTES = (FMT == FMT_F16) ? 65536 : 32768;
    static constexpr int NG = SEG / TileT<FMT>::G;
    static constexpr int TOK = TileT<FMT>::TOK;
    static constexpr int FX = TOK * NG * 2;  // floats of one pass's group factors
    static constexpr int passes(int mt) { return (mt + TOK - 1) / TOK; }
    static constexpr int bytes(int ks, int mt) {
        return passes(mt) * (A_BYTES + FX * 4) + MAXM * 4 + ks * 64 * 2 * 4 + ks * MAXM * 4;
    }
};

// Stages the activation operands of columns [col0, col0 + COLS) of segment `seg`, tokens
// [t0, t0 + TOK) of the pass, with NTHR threads, into the operand layout at Alds / fx (LDS, or
// global memory for the pre-staged operands).  Each thread's units are loaded first (one memory
// round trip), then sliced.
// With FUSE (PRO_NORM, the whole row in one call, one unit per token per thread), the RMSNorm
// scales come from the loaded values themselves: nscale is then LDS scratch of NTHR / 64 x MAXM
// floats, and the call holds one workgroup barrier.
template <int FMT, int K, int PRO, int NTHR, int COLS = SEG, bool FUSE = false>
__device__ __forceinline__ void stage(const GemvArgs& a, int seg, int t0, int M, int row0, uint8_t* Alds, float* fx,
                                      const float* nscale, int col0 = 0) {
    constexpr int TOK = TileT<FMT>::TOK;
    constexpr int G = TileT<FMT>::G;
    constexpr int NG = SEG / G;
    constexpr int NU = TOK * (COLS / 8) / NTHR;  // units per thread
    static_assert(TOK * (COLS / 8) % NTHR == 0 && COLS % 64 == 0, "whole units per thread, whole groups");
    static_assert(!FUSE || (PRO == PRO_NORM && COLS == K && NTHR == COLS / 8), "fused norm: unit j is token j's");
    const int tid = threadIdx.x;
    // One unit = 8 consecutive activations of one token; the units of a group sit in adjacent
    // lanes (G / 8 of them), so the group reductions are DPP steps.
    float vv[NU][8];
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        const int u = tid + NTHR * j;
        const int tl = u / (COLS / 8);
        const int k0 = col0 + (u % (COLS / 8)) * 8;  // within the segment
        const int t = t0 + tl;
        // Rows past the pass read row M - 1 and are zeroed: the loads stay unconditional, so the
        // compiler issues all of them before the first use.
        const float* xr = a.x + (size_t)(row0 + min(t, M - 1)) * K + seg * SEG + k0;
        const float4 p0 = ((const float4*)xr)[0], p1 = ((const float4*)xr)[1];
        const bool in = t < M;
        vv[j][0] = in ? p0.x : 0.f; vv[j][1] = in ? p0.y : 0.f; vv[j][2] = in ? p0.z : 0.f; vv[j][3] = in ? p0.w : 0.f;
        vv[j][4] = in ? p1.x : 0.f; vv[j][5] = in ? p1.y : 0.f; vv[j][6] = in ? p1.z : 0.f; vv[j][7] = in ? p1.w : 0.f;
    }
    float fsc[NU];
    if constexpr (FUSE) {
        float* red = (float*)nscale;
        const int lane = tid % 64, wave = tid / 64;
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            float ss = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += vv[j][i] * vv[j][i];
            ss = wave_sum(ss);
            if (lane == 0) red[wave * MAXM + j] = ss;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            float tot = 0.f;
            for (int w = 0; w < NTHR / 64; ++w) tot += red[w * MAXM + j];
            fsc[j] = 1.0f / sqrtf(tot / (float)K + EPS);
        }
    }
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        const int u = tid + NTHR * j;
        const int tl = u / (COLS / 8);
        const int k0 = col0 + (u % (COLS / 8)) * 8;  // within the segment
        const int t = t0 + tl;
        float* v = vv[j];
        if constexpr (PRO == PRO_NORM) {
            const float sc = FUSE ? fsc[j] : nscale[min(t, M - 1)];
            const float* w = a.norm_w + seg * SEG + k0;
            const float4 w0 = ((const float4*)w)[0], w1 = ((const float4*)w)[1];
            v[0] = v[0] * sc * w0.x; v[1] = v[1] * sc * w0.y; v[2] = v[2] * sc * w0.z; v[3] = v[3] * sc * w0.w;
            v[4] = v[4] * sc * w1.x; v[5] = v[5] * sc * w1.y; v[6] = v[6] * sc * w1.z; v[7] = v[7] * sc * w1.w;
        }
        if constexpr (FMT == FMT_F16) {
            // rows m = 2 tl + {hi, lo}; chunk c = k0 / 32, K-slot q = (k0 % 32) / 8.
            uint32_t hi[8], lo[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const f16 h = (f16)v[i];
                hi[i] = __builtin_bit_cast(uint16_t, h);
                lo[i] = __builtin_bit_cast(uint16_t, (f16)(v[i] - (float)h));
            }
            const int c = k0 / 32, q = (k0 % 32) / 8;
            uint4 Hv, Lv;
            Hv.x = hi[0] | hi[1] << 16; Hv.y = hi[2] | hi[3] << 16; Hv.z = hi[4] | hi[5] << 16; Hv.w = hi[6] | hi[7] << 16;
            Lv.x = lo[0] | lo[1] << 16; Lv.y = lo[2] | lo[3] << 16; Lv.z = lo[4] | lo[5] << 16; Lv.w = lo[6] | lo[7] << 16;
            uint4* A = (uint4*)Alds + c * 64;
            A[(2 * tl) + 16 * q] = Hv;
            A[(2 * tl + 1) + 16 * q] = Lv;
        } else {
            float amax = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
            int bits = (int)as_u32(amax);  // order of non-negative floats = order of their bits
            bits = max(bits, dpp_i<DPP_XOR1>(bits));
            bits = max(bits, dpp_i<DPP_XOR2>(bits));
            if constexpr (G == 64) bits = max(bits, dpp_i<DPP_HALF_MIRROR>(bits));
            int e = ((bits >> 23) & 0xFF) - 127;
            if (bits == 0) e = -100;  // all-zero group: X = 0 for any exponent
            const int sh = 21 - e;
            int X[8];
            int xs = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                X[i] = (int)rintf(ldexpf(v[i], sh));
                xs += X[i];
            }
            xs += dpp_i<DPP_XOR1>(xs);
            xs += dpp_i<DPP_XOR2>(xs);
            if constexpr (G == 64) xs += dpp_i<DPP_HALF_MIRROR>(xs);
            // Balanced byte slices: X = 65536 hi + 256 mid + lo, each in [-128, 127].
            uint32_t sl[3][2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint32_t p0 = 0, p1 = 0, p2 = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int x = X[4 * h + i];
                    const int lo = (int)(int8_t)(x & 0xFF);
                    const int r1 = (x - lo) >> 8;
                    const int mid = (int)(int8_t)(r1 & 0xFF);
                    const int hi = (r1 - mid) >> 8;
                    p0 |= (uint32_t)(lo & 0xFF) << (8 * i);
                    p1 |= (uint32_t)(mid & 0xFF) << (8 * i);
                    p2 |= (uint32_t)(hi & 0xFF) << (8 * i);
                }
                sl[0][h] = p0;
                sl[1][h] = p1;
                sl[2][h] = p2;
            }
            const int gl = k0 / G, kk = k0 % G;
            if constexpr (FMT == FMT_Q4) {
                const int q = kk / 16, j0 = kk % 16;  // K-slot (16 K) and byte offset 0 / 8
                uint8_t* A = Alds + gl * 1024;
                // rows m = 4 tl + {0 hi, 1 mid, 2 lo, 3 zero}
                *(uint2*)(A + ((4 * tl + 0) + 16 * q) * 16 + j0) = make_uint2(sl[2][0], sl[2][1]);
                *(uint2*)(A + ((4 * tl + 1) + 16 * q) * 16 + j0) = make_uint2(sl[1][0], sl[1][1]);
                *(uint2*)(A + ((4 * tl + 2) + 16 * q) * 16 + j0) = make_uint2(sl[0][0], sl[0][1]);
                *(uint2*)(A + ((4 * tl + 3) + 16 * q) * 16 + j0) = make_uint2(0u, 0u);
            } else {
                const int q = kk / 8;  // K-slot of 8 K
                uint8_t* A = Alds + gl * 512;
                *(uint2*)(A + ((4 * tl + 0) + 16 * q) * 8) = make_uint2(sl[2][0], sl[2][1]);
                *(uint2*)(A + ((4 * tl + 1) + 16 * q) * 8) = make_uint2(sl[1][0], sl[1][1]);
                *(uint2*)(A + ((4 * tl + 2) + 16 * q) * 8) = make_uint2(sl[0][0], sl[0][1]);
                *(uint2*)(A + ((4 * tl + 3) + 16 * q) * 8) = make_uint2(0u, 0u);
            }
            if (kk == 0) {
                const float f = ldexpf(1.0f, -sh);
                fx[(tl * NG + gl) * 2 + 0] = f;
                fx[(tl * NG + gl) * 2 + 1] = (float)xs * f;
            }
        }
    }
}

// Rows of the pass: M tokens from row row0 of the activations.
template <int EPI, int MT>
__device__ __forceinline__ void gemv_rows(const GemvArgs& a, const State* st, int& M, int& row0) {
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
}

// RMSNorm scale of every token over the full K (NTHR threads; red holds NTHR / 64 x MAXM
// floats); the tokens' loads are issued together and reduced in one round.
template <int K, int MT, int NTHR>
__device__ __forceinline__ void norm_scales(const GemvArgs& a, int M, int row0, float* nscale, float* red) {
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    float ss[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) ss[t] = 0.f;
#pragma unroll
    for (int k = tid; k < K; k += NTHR) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {  // unconditional loads (row clamped), zero past the pass
            const float v = a.x[(size_t)(row0 + min(t, M - 1)) * K + k];
            ss[t] += t < M ? v * v : 0.f;
        }
    }
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        const float w = wave_sum(ss[t]);
        if (lane == 0) red[wave * MAXM + t] = w;
    }
    __syncthreads();
    if (tid < M) {
        float tot = 0.f;
        for (int w = 0; w < NTHR / 64; ++w) tot += red[w * MAXM + tid];
        nscale[tid] = 1.0f / sqrtf(tot / (float)K + EPS);
    }
    __syncthreads();
}

// Pre-staging of a multi-row GEMV's activation operands, once per launch instead of once per
// workgroup: workgroup (segment, pass, chunk of PREP_COLS columns) writes its part of the
// operands and group factors in the LDS layout of gemv_kernel to a.apre [NSEG][NP][A_BYTES] and
// a.fxpre [NSEG][NP][FX], RMSNorm (PRO_NORM) included.
// One workgroup per (segment, pass) of SEG / 8 threads: every thread loads one unit of 8
// activations of each token of the pass, once; RMSNorm takes its sums from those registers.
template <int FMT, int K, int PRO, int EPI>
__global__ __launch_bounds__(SEG / 8) void gemv_prep_kernel(GemvArgs a) {
    const State* st = a.st;
    if (st->done) return;
    using T = TileT<FMT>;
    constexpr int NSEG = K / SEG, NP = Smem<FMT>::passes(MAXM);
    static_assert(PRO != PRO_NORM || NSEG == 1, "RMSNorm prologues take K = 2048");
    int M, row0;
    gemv_rows<EPI, MAXM>(a, st, M, row0);
    const int p = blockIdx.x % NP, seg = blockIdx.x / NP;
    if (p * T::TOK >= M) return;  // a pass the GEMV does not run
    __shared__ float red[(SEG / 8 / 64) * MAXM];
    stage<FMT, K, PRO, SEG / 8, SEG, PRO == PRO_NORM>(a, seg, p * T::TOK, M, row0,
                                                      a.apre + (size_t)(seg * NP + p) * Smem<FMT>::A_BYTES,
                                                      a.fxpre + (size_t)(seg * NP + p) * Smem<FMT>::FX, red);
}

template <int FMT, int K, int KS, int MT, int PRO, int EPI>
__global__ __launch_bounds__(KS * 64) void gemv_kernel(GemvArgs a) {
    const State* st = a.st;
    if (st->done) return;
    using T = TileT<FMT>;
    constexpr int NSEG = K / SEG;
    constexpr int CPS = SEG / T::CHK;  // chunks per segment
    constexpr int CPW = CPS / KS;      // chunks per wave per segment
    static_assert(CPS % KS == 0, "chunks per segment must split evenly over the waves");
    constexpr int NG = SEG / T::G;
    constexpr int NC = K / T::CHK;  // chunks per row block

    int M, row0;
    gemv_rows<EPI, MT>(a, st, M, row0);
    const int npass = (M + T::TOK - 1) / T::TOK;
    constexpr int NP = Smem<FMT>::passes(MT);

    extern __shared__ __align__(16) uint8_t smem[];
    uint8_t* Alds = smem;                                           // [NP][A_BYTES]
    float* fx = (float*)(smem + NP * Smem<FMT>::A_BYTES);           // [NP][FX]
    float* nscale = fx + NP * Smem<FMT>::FX;
    float* part = nscale + MAXM;      // [KS][2][64]
    float* red = part + KS * 2 * 64;  // [KS][MAXM]

    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;

    // Operands pre-staged by gemv_prep_kernel (multi-row passes): copied into LDS, no RMSNorm or
    // slicing here.
    const bool pre = MT > 1 && a.apre != nullptr;
    if constexpr (PRO == PRO_NORM) {
        if (!pre) norm_scales<K, MT, KS * 64>(a, M, row0, nscale, red);
    }

    // Activation operands of every pass, staged once per segment (once per launch when K fits
    // one segment).
    auto stage_all = [&](int seg) {
        if (pre) {
            // 1 KiB wave loads straight into LDS: the passes' operands, then their group factors.
            constexpr int AW = Smem<FMT>::A_BYTES / 1024, FW = (FMT == FMT_F16) ? 0 : Smem<FMT>::FX * 4 / 1024;
            for (int p = 0; p < npass; ++p) {
                const uint8_t* src = a.apre + (size_t)(seg * NP + p) * Smem<FMT>::A_BYTES;
                const uint8_t* fsrc = (const uint8_t*)(a.fxpre + (size_t)(seg * NP + p) * Smem<FMT>::FX);
                for (int w = wave; w < AW + FW; w += KS) {
                    const uint8_t* g = w < AW ? src + w * 1024 : fsrc + (w - AW) * 1024;
                    uint8_t* l = w < AW ? Alds + p * Smem<FMT>::A_BYTES + w * 1024
                                        : (uint8_t*)(fx + p * Smem<FMT>::FX) + (w - AW) * 1024;
                    __builtin_amdgcn_global_load_lds(g + lane * 16, (__attribute__((address_space(3))) void*)l, 16, 0,
                                                     0);
                }
            }
            __builtin_amdgcn_s_waitcnt(0);  // this wave's copies have landed (the barrier after covers all)
            return;
        }
        for (int p = 0; p < npass; ++p)
            stage<FMT, K, PRO, KS * 64>(a, seg, p * T::TOK, M, row0, Alds + p * Smem<FMT>::A_BYTES,
                                        fx + p * Smem<FMT>::FX, nscale);
    };
    const int nrb = (EPI == EPI_SWIGLU) ? (FF / 8) : (a.N / 16);
    // K in one segment: staged once, right after the first row block's weight loads are issued.
    constexpr bool stage_once = (NSEG == 1);
    bool staged = false;

    float best_v[MT];
    int best_i[MT];
#pragma unroll
    for (int t = 0; t < MT; ++t) {
        best_v[t] = -__builtin_inff();
        best_i[t] = 0x7fffffff;
    }

    const int r16 = lane % 16, lg = lane / 16;
    // K = 6144 residual GEMVs split along K: workgroup b takes segment b % NSEG of row block
    // b / NSEG, and the last of a row block's workgroups to finish adds the partials in segment
    // order (deterministic).  Every other GEMV walks whole row blocks.
    constexpr bool SPLITK = (EPI == EPI_RESID && NSEG > 1);
    const int seg_lo = SPLITK ? (int)(blockIdx.x % NSEG) : 0;
    const int seg_hi = SPLITK ? seg_lo + 1 : NSEG;
    const int rb_step = SPLITK ? nrb : (int)gridDim.x;
    // This wave's chunks of row block b, segment seg: the weight codes and the lane's row scales.
    auto load_w = [&](int b, int seg, uint4 (&wv)[CPW], uint2 (&sbv)[CPW]) {
        const uint8_t* wblk = a.w + (size_t)b * NC * 1024;
        const int row = b * 16 + r16;
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
            const int c = seg * CPS + wave * CPW + i;
            wv[i] = ((const uint4*)(wblk + (size_t)c * 1024))[lane];
        }
#pragma unroll
        for (int i = 0; i < CPW; ++i) {
            const int c = seg * CPS + wave * CPW + i;
            if constexpr (FMT == FMT_Q4)
                sbv[i] = *(const uint2*)(a.sb + ((size_t)row * (K / 64) + 2 * c) * 4);
            else if constexpr (FMT == FMT_Q8)
                sbv[i] = make_uint2(*(const uint32_t*)(a.sb + ((size_t)row * (K / 32) + 2 * c) * 2), 0u);
            else
                sbv[i] = make_uint2(0u, 0u);
        }
    };
    // With K in one segment and int8 codes (4 KiB of a block per wave) the next row block's
    // weights are requested before this one's matrix-core work (two blocks in flight per wave);
    // the last block re-requests itself.  f16 blocks (16 KiB per wave) would spill.
    constexpr bool prefetch = stage_once && FMT != FMT_F16;
    // One row block: this wave's weights are in wv / sbv; with K in one segment the next block's
    // are requested into wn / sn before the matrix-core work.  The two buffers swap roles from one
    // block to the next (the loop below is unrolled by two), so no register copy waits on them.
    auto row_block = [&](int rb, uint4 (&wv)[CPW], uint2 (&sbv)[CPW], uint4 (&wn)[CPW], uint2 (&sn)[CPW]) {
            const int row = rb * 16 + r16;  // tiled row of this lane
            float acc[2] = {0.f, 0.f};
            for (int seg = seg_lo; seg < seg_hi; ++seg) {
                // Weights of this wave's chunks, issued before the activation staging.
                if (!prefetch || !staged) load_w(rb, seg, wv, sbv);
                if (!stage_once || !staged) {
                    if (!stage_once) __syncthreads();
                    stage_all(seg);
                    __syncthreads();
                    staged = true;
                }
                if constexpr (prefetch) load_w(min(rb + rb_step, nrb - 1), seg, wn, sn);
                for (int p = 0; p < npass; ++p) {
                    const uint8_t* Ap = Alds + p * Smem<FMT>::A_BYTES;
                    const float* fxp = fx + p * Smem<FMT>::FX;
                    float pacc = 0.f, pacc2 = 0.f;
    #pragma unroll
                    for (int i = 0; i < CPW; ++i) {
                        const int cs = wave * CPW + i;  // chunk within the segment
                        if constexpr (FMT == FMT_Q4) {
    #pragma unroll
                            for (int hh = 0; hh < 2; ++hh) {
                                const uint32_t d0 = hh ? wv[i].z : wv[i].x;
                                const uint32_t d1 = hh ? wv[i].w : wv[i].y;
                                v4i B;
                                B[0] = (int)(d0 & 0x0F0F0F0Fu);
                                B[1] = (int)((d0 >> 4) & 0x0F0F0F0Fu);
                                B[2] = (int)(d1 & 0x0F0F0F0Fu);
                                B[3] = (int)((d1 >> 4) & 0x0F0F0F0Fu);
                                const int gl = 2 * cs + hh;
                                const v4i A = *(const v4i*)(Ap + gl * 1024 + lane * 16);
                                const v4i zero = {0, 0, 0, 0};
                                const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, zero, 0, 0, 0);
                                const float S = fmaf((float)C[0], 65536.f, fmaf((float)C[1], 256.f, (float)C[2]));
                                const f16x2 sb2 = as_h2(hh ? sbv[i].y : sbv[i].x);
                                const float f = fxp[(lg * NG + gl) * 2], X = fxp[(lg * NG + gl) * 2 + 1];
                                pacc = fmaf((float)sb2.x * f, S, fmaf((float)sb2.y, X, pacc));
                            }
                        } else if constexpr (FMT == FMT_Q8) {
    #pragma unroll
                            for (int hh = 0; hh < 2; ++hh) {
                                const long B = (long)(hh ? ((uint64_t)wv[i].w << 32 | wv[i].z)
                                                         : ((uint64_t)wv[i].y << 32 | wv[i].x));
                                const int gl = 2 * cs + hh;
                                const long A = *(const long*)(Ap + gl * 512 + lane * 8);
                                const v4i zero = {0, 0, 0, 0};
                                const v4i C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, zero, 0, 0, 0);
                                const float S = fmaf((float)C[0], 65536.f, fmaf((float)C[1], 256.f, (float)C[2]));
                                const f16x2 s2 = as_h2(sbv[i].x);
                                const float s = hh ? (float)s2.y : (float)s2.x;
                                pacc = fmaf(s * fxp[(lg * NG + gl) * 2], S, pacc);
                            }
                        } else {
                            const v8h B = __builtin_bit_cast(v8h, wv[i]);
                            const v8h A = *(const v8h*)(Ap + cs * 1024 + lane * 16);
                            const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                            const f32x4 C = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, B, zero, 0, 0, 0);
                            pacc += C[0] + C[1];
                            pacc2 += C[2] + C[3];
                        }
                    }
                    if constexpr (FMT == FMT_F16) {
                        acc[0] += pacc;
                        acc[1] += pacc2;
                    } else {
                        acc[p] += pacc;  // pass p covers tokens 4 p .. 4 p + 3
                    }
                }
            }
            // Cross-wave reduction in a fixed order.
            if constexpr (KS > 1) {
                part[(wave * 2 + 0) * 64 + lane] = acc[0];
                part[(wave * 2 + 1) * 64 + lane] = acc[1];
                __syncthreads();
                if (wave == 0) {
    #pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        float s = part[j * 64 + lane];
                        for (int w = 1; w < KS; ++w) s += part[(w * 2 + j) * 64 + lane];
                        acc[j] = s;
                    }
                }
                __syncthreads();
            }
            if constexpr (SPLITK) {
                // Partials go out with device-scope stores (coherent across the XCDs' L2s) and are
                // complete before the arrival is counted.
                __shared__ int is_last;
                if (wave == 0) {
    #pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int t = (FMT == FMT_F16) ? 2 * lg + j : 4 * j + lg;
                        if (t < M)
                            __hip_atomic_store(a.kpart + ((size_t)seg_lo * MAXM + t) * a.N + row, acc[j], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                    }
                    __builtin_amdgcn_s_waitcnt(0);
                }
                __syncthreads();
                if (tid == 0)
                    is_last = __hip_atomic_fetch_add(a.kcnt + rb, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == NSEG - 1;
                __syncthreads();
                if (!is_last) return;
                if (wave == 0) {
    #pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const int t = (FMT == FMT_F16) ? 2 * lg + j : 4 * j + lg;
                        float sum = 0.f;
                        if (t < M)
                            for (int sg = 0; sg < NSEG; ++sg)
                                sum += __hip_atomic_load(a.kpart + ((size_t)sg * MAXM + t) * a.N + row, __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
                        acc[j] = sum;
                    }
                    if (lane == 0) __hip_atomic_store(a.kcnt + rb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            if (wave == 0) {
    #pragma unroll
                for (int j = 0; j < 2; ++j) {
                    // int8 formats: acc[j] is token 4 j + lg; f16: token 2 lg + j.
                    const int t = (FMT == FMT_F16) ? 2 * lg + j : 4 * j + lg;
                    const bool valid = t < M;
                    const float y = acc[j];
                    if constexpr (EPI == EPI_STORE) {
                        if (valid) a.y[(size_t)(row0 + t) * a.N + row] = y;
                    } else if constexpr (EPI == EPI_RESID) {
                        if (valid) {
                            float* xo = a.y + (size_t)(row0 + t) * a.N + row;
                            float v = *xo + y;
                            if (a.ds) {  // DeepStack residual of a visual row (Shaders.swift:696-707)
                                const int vrow = a.ds_row0 + t - st->vis_offset;
                                if (st->vis_offset >= 0 && vrow >= 0 && vrow < st->n_vis)
                                    v = v + a.ds[(size_t)vrow * H + row];
                            }
                            *xo = v;
                        }
                    } else if constexpr (EPI == EPI_SWIGLU) {
                        // Block rb: gate units 8 rb .. 8 rb + 7 in columns 0-7, matching up rows in 8-15.
                        const float up = __shfl_xor(y, 8);
                        if (valid && r16 < 8) {
                            const float g = y;
                            a.h[(size_t)(row0 + t) * FF + rb * 8 + r16] = (g / (1.f + expf(-g))) * up;
                        }
                    } else {  // EPI_ARGMAX: tiled rows are the vocabulary ids
                        if (valid) {
                            if (a.logits && st->logits_rows > 0) a.logits[(size_t)t * VOCAB + row] = y;
    #pragma unroll
                            for (int tt = 0; tt < MT; ++tt)
                                if (tt == t) argmax_merge(best_v[tt], best_i[tt], y, row);
                        }
                    }
                }
            }
    
    };
    uint4 wa[CPW], wb[CPW];
    uint2 sa[CPW], sb2[CPW];
    const int rb0 = SPLITK ? (int)(blockIdx.x / NSEG) : (int)blockIdx.x;
    if constexpr (prefetch) {
        for (int rb = rb0; rb < nrb; rb += 2 * rb_step) {
            row_block(rb, wa, sa, wb, sb2);
            if (rb + rb_step >= nrb) break;
            row_block(rb + rb_step, wb, sb2, wa, sa);
        }
    } else {
        for (int rb = rb0; rb < nrb; rb += rb_step) row_block(rb, wa, sa, wb, sb2);
    }
    if constexpr (EPI == EPI_ARGMAX) {
        if (wave == 0) {
#pragma unroll
            for (int t = 0; t < MT; ++t) {
                if (t >= M) break;
                float v = best_v[t];
                int i = best_i[t];
                wave_argmax(v, i);
                if (lane == 0) {
                    a.pval[(size_t)(row0 + t) * LMH_WAVES + blockIdx.x] = v;
                    a.pidx[(size_t)(row0 + t) * LMH_WAVES + blockIdx.x] = i;
                }
            }
        }
    }
}

template <int FMT, int K, int KS, int MT, int PRO, int EPI>
static hipError_t launch_one(const GemvArgs& a, int blocks, hipStream_t s) {
    const size_t lds = Smem<FMT>::bytes(KS, MT);
    auto kern = gemv_kernel<FMT, K, KS, MT, PRO, EPI>;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(KS * 64), lds, s, a);
    return hipGetLastError();
}

template <int FMT>
static hipError_t gemv_fmt(GemvOp op, const GemvArgs& a, int mt, hipStream_t s) {
    const bool one = (mt == 1);
    switch (op) {
        case GEMV_QKV:  // RMSNorm -> fused QKV rows, fp32 out
            return one ? launch_one<FMT, H, 4, 1, PRO_NORM, EPI_STORE>(a, QKV / 16, s)
                       : launch_one<FMT, H, 4, MAXM, PRO_NORM, EPI_STORE>(a, QKV / 16, s);
        case GEMV_O:  // attention output -> O rows, residual add
            return one ? launch_one<FMT, H, 4, 1, PRO_F32, EPI_RESID>(a, H / 16, s)
                       : launch_one<FMT, H, 4, MAXM, PRO_F32, EPI_RESID>(a, H / 16, s);
        case GEMV_GU:  // RMSNorm -> gate|up pairs -> SwiGLU
            return one ? launch_one<FMT, H, 4, 1, PRO_NORM, EPI_SWIGLU>(a, FF / 8, s)
                       : launch_one<FMT, H, 4, MAXM, PRO_NORM, EPI_SWIGLU>(a, FF / 8, s);
        case GEMV_DOWN:  // SwiGLU output -> down rows, residual add; split along K in 3 segments
            if (!a.kpart || !a.kcnt) return hipErrorInvalidValue;
            return one ? launch_one<FMT, FF, 4, 1, PRO_F32, EPI_RESID>(a, H / 16 * (FF / SEG), s)
                       : launch_one<FMT, FF, 4, MAXM, PRO_F32, EPI_RESID>(a, H / 16 * (FF / SEG), s);
        case GEMV_LMHEAD:  // final RMSNorm -> tied embedding rows -> argmax partials
            return one ? launch_one<FMT, H, 4, 1, PRO_NORM, EPI_ARGMAX>(a, LMH_WAVES, s)
                       : launch_one<FMT, H, 4, MAXM, PRO_NORM, EPI_ARGMAX>(a, LMH_WAVES, s);
        case GEMV_PLAIN:  // isolated GEMV, K = 2048
            return one ? launch_one<FMT, H, 4, 1, PRO_F32, EPI_STORE>(a, a.blocks, s)
                       : launch_one<FMT, H, 4, MAXM, PRO_F32, EPI_STORE>(a, a.blocks, s);
        case GEMV_PLAIN_K6144:
            return one ? launch_one<FMT, FF, 4, 1, PRO_F32, EPI_STORE>(a, a.blocks, s)
                       : launch_one<FMT, FF, 4, MAXM, PRO_F32, EPI_STORE>(a, a.blocks, s);
    }
    return hipErrorInvalidValue;
}

template <int FMT, int K, int PRO, int EPI>
static hipError_t launch_prep_one(const GemvArgs& a, hipStream_t s) {
    constexpr int NB = (K / SEG) * Smem<FMT>::passes(MAXM);
    hipLaunchKernelGGL((gemv_prep_kernel<FMT, K, PRO, EPI>), dim3(NB), dim3(SEG / 8), 0, s, a);
    return hipGetLastError();
}

template <int FMT>
static hipError_t prep_fmt(GemvOp op, const GemvArgs& a, hipStream_t s) {
    switch (op) {
        case GEMV_QKV: return launch_prep_one<FMT, H, PRO_NORM, EPI_STORE>(a, s);
        case GEMV_O: return launch_prep_one<FMT, H, PRO_F32, EPI_RESID>(a, s);
        case GEMV_GU: return launch_prep_one<FMT, H, PRO_NORM, EPI_SWIGLU>(a, s);
        case GEMV_DOWN: return launch_prep_one<FMT, FF, PRO_F32, EPI_RESID>(a, s);
        case GEMV_LMHEAD: return launch_prep_one<FMT, H, PRO_NORM, EPI_ARGMAX>(a, s);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_gemv_prep(int fmt, GemvOp op, const GemvArgs& a, hipStream_t s) {
    if (!a.apre || !a.fxpre) return hipErrorInvalidValue;
    switch (fmt) {
        case FMT_Q4: return prep_fmt<FMT_Q4>(op, a, s);
        case FMT_Q8: return prep_fmt<FMT_Q8>(op, a, s);
        case FMT_F16: return prep_fmt<FMT_F16>(op, a, s);
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

// ------------------------------------------------------------------------------------------
// Repacking from the .icua row-major layout (Convert.swift:157-171) into 16-row MFMA tiles.

// Source row of a tiled row: identity, or for the fused gate|up matrix the interleave that puts
// gate units 8 rb .. 8 rb + 7 and their up rows into tiled block rb.
__device__ __forceinline__ int src_row(int trow, int gu_interleave) {
    if (!gu_interleave) return trow;
    const int rb = trow / 16, r = trow % 16;
    return r < 8 ? rb * 8 + r : FF + rb * 8 + (r - 8);
}

__global__ void repack_codes_kernel(int fmt, const uint8_t* src, uint8_t* dst, int N, int K, int gu) {
    const int chk = fmt == FMT_Q4 ? 128 : fmt == FMT_Q8 ? 64 : 32;
    const int nc = K / chk;
    const size_t total = (size_t)(N / 16) * nc * 64;  // one thread per 16-byte lane slice
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
         idx += (size_t)gridDim.x * blockDim.x) {
        const int l = (int)(idx % 64);
        const size_t bc = idx / 64;
        const int c = (int)(bc % nc);
        const int rb = (int)(bc / nc);
        const int r = l % 16, q = l / 16;
        const int srow = src_row(rb * 16 + r, gu);
        uint8_t out[16];
        if (fmt == FMT_Q4) {
            const uint8_t* rowp = src + (size_t)srow * (K / 2);
            for (int hh = 0; hh < 2; ++hh) {
                const int kbase = (2 * c + hh) * 64 + 16 * q;  // the 16 K of this slot
                for (int d = 0; d < 2; ++d)
                    for (int b = 0; b < 4; ++b) {
                        const int klo = kbase + 8 * d + b, khi = klo + 4;
                        const uint8_t vlo = (rowp[klo / 2] >> (4 * (klo & 1))) & 15;
                        const uint8_t vhi = (rowp[khi / 2] >> (4 * (khi & 1))) & 15;
                        out[8 * hh + 4 * d + b] = (uint8_t)(vlo | (vhi << 4));
                    }
            }
        } else if (fmt == FMT_Q8) {
            const uint8_t* rowp = src + (size_t)srow * K;
            for (int hh = 0; hh < 2; ++hh)
                for (int j = 0; j < 8; ++j) out[8 * hh + j] = rowp[(2 * c + hh) * 32 + 8 * q + j];
        } else {
            const uint16_t* rowp = (const uint16_t*)src + (size_t)srow * K;
            for (int j = 0; j < 8; ++j) {
                const uint16_t v = rowp[c * 32 + 8 * q + j];
                out[2 * j] = (uint8_t)(v & 0xFF);
                out[2 * j + 1] = (uint8_t)(v >> 8);
            }
        }
        uint4 o;
        o.x = out[0] | out[1] << 8 | out[2] << 16 | (uint32_t)out[3] << 24;
        o.y = out[4] | out[5] << 8 | out[6] << 16 | (uint32_t)out[7] << 24;
        o.z = out[8] | out[9] << 8 | out[10] << 16 | (uint32_t)out[11] << 24;
        o.w = out[12] | out[13] << 8 | out[14] << 16 | (uint32_t)out[15] << 24;
        ((uint4*)dst)[idx] = o;
    }
}

__global__ void repack_rows_kernel(const uint8_t* src, uint8_t* dst, int N, int row_bytes, int gu) {
    const size_t total = (size_t)N * row_bytes;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
        const int trow = (int)(i / row_bytes);
        const int b = (int)(i % row_bytes);
        dst[i] = src[(size_t)src_row(trow, gu) * row_bytes + b];
    }
}

hipError_t launch_repack(int fmt, const uint8_t* codes, const uint8_t* sb, uint8_t* dcodes, uint8_t* dsb, int N, int K,
                         int gu_interleave, hipStream_t s) {
    if (N % 16 || K % SEG || (gu_interleave && N != GU)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(repack_codes_kernel, dim3(2048), dim3(256), 0, s, fmt, codes, dcodes, N, K, gu_interleave);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (fmt != FMT_F16) {
        const int rbytes = fmt == FMT_Q4 ? (K / 64) * 4 : (K / 32) * 2;
        hipLaunchKernelGGL(repack_rows_kernel, dim3(2048), dim3(256), 0, s, sb, dsb, N, rbytes, gu_interleave);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace icua
