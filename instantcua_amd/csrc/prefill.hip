// Many-token prefill on the matrix cores, gfx950 (q4 weights).
//
// Replaces the reference's multi-token path (Shaders.swift:676-1216: k_rmsnorm_rows_h,
// llm_gemm_tile, k_g3_*, k_qk_norm_rope, k_prefill_attn) for prompts longer than one GEMV pass;
// math per tools/reference/qwen3vl_ref.py:243-292 (fp32 activations, fp16 KV cache).
//
// Projections.  y[t][r] = sum_g (s_rg sum_{k in g} q_rk x_tk + b_rg sum_{k in g} x_tk).  A prep
// kernel writes every activation row as exactly-rounded 21-bit integers per 64-group,
// X = rint(x 2^(20-e_g)) (e_g = exponent of the group's largest |x|), split into three signed
// bytes X = 65536 hi + 256 mid + lo, in the A-operand layout of v_mfma_i32_16x16x64_i8.  The
// GEMM multiplies 16 tokens x 16 weight rows x 64 K per instruction and chains the slices in
// the int32 accumulator: U = ((C_hi << 8) + C_mid) << 8) + C_lo = sum_k q_k X_k exactly
// (|U| <= 64 * 15 * 2^21 < 2^31), then y += (s f) float(U) + b (f sum X), f = 2^(e_g-20).  The
// only roundings are the 21-bit activation quantisation and fp32 group scaling.
//
// Attention.  Causal GQA flash attention on v_mfma_f32_16x16x32_f16: scores are computed
// transposed (S^T = K Q^T) so that the probabilities come out of the accumulator already in
// the B-operand layout of the P.V product (O^T = V^T P^T); V is transposed through LDS.  The
// fp32 queries and probabilities are split into fp16 hi + lo parts (two products each), which
// keeps them at ~22 bits against the fp16 cache.
#include "icua_device.h"
#include "icua_kernels.h"

namespace icua {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned v4u __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------
// Activation operands.  XA: [Mpad / 16][K / 64][3 slices (hi, mid, lo)][64 lanes][16 B], lane l
// holding token 16 tb + l % 16, K = 64 g + 16 (l / 16) + 0..15.  XF: [Mpad / 16][K / 64][16]
// float2 (f = 2^(e - 20), f * sum X).  One workgroup per token row (rows >= M are zero).

template <int K, bool NORM>
__global__ __launch_bounds__(256) void pf_prep_kernel(const float* __restrict__ src, const float* __restrict__ norm_w,
                                                      int M, uint8_t* __restrict__ xa, float2* __restrict__ xf) {
    constexpr int NU = K / 8 / 256;  // units of 8 activations per thread
    constexpr int NG = K / 64;
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    __shared__ float red[4];
    float v[NU][8];
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        if (t < M) {
            const float4* p = (const float4*)(src + (size_t)t * K + (tid + 256 * j) * 8);
            const float4 a0 = p[0], a1 = p[1];
            v[j][0] = a0.x; v[j][1] = a0.y; v[j][2] = a0.z; v[j][3] = a0.w;
            v[j][4] = a1.x; v[j][5] = a1.y; v[j][6] = a1.z; v[j][7] = a1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) v[j][i] = 0.f;
        }
    }
    if constexpr (NORM) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NU; ++j)
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += v[j][i] * v[j][i];
        ss = wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        const float tot = (red[0] + red[1]) + (red[2] + red[3]);
        const float scale = 1.0f / sqrtf(tot / (float)K + EPS);
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const float4* wp = (const float4*)(norm_w + (tid + 256 * j) * 8);
            const float4 w0 = wp[0], w1 = wp[1];
            const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) v[j][i] = v[j][i] * scale * w[i];
        }
    }
    const int tb = t >> 4, tr = t & 15;
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        const int k0 = (tid + 256 * j) * 8;
        // Group max over the 8 adjacent lanes holding the group's 64 values.
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[j][i]));
        int bits = (int)as_u32(amax);  // order of non-negative floats = order of their bits
        bits = max(bits, dpp_i<DPP_XOR1>(bits));
        bits = max(bits, dpp_i<DPP_XOR2>(bits));
        bits = max(bits, dpp_i<DPP_HALF_MIRROR>(bits));
        int e = ((bits >> 23) & 0xFF) - 127;
        if (bits == 0) e = -100;  // all-zero group: X = 0 for any exponent
        const int sh = 20 - e;
        int X[8], xs = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            X[i] = (int)rintf(ldexpf(v[j][i], sh));
            xs += X[i];
        }
        xs += dpp_i<DPP_XOR1>(xs);
        xs += dpp_i<DPP_XOR2>(xs);
        xs += dpp_i<DPP_HALF_MIRROR>(xs);
        // Balanced byte slices: X = 65536 hi + 256 mid + lo, mid and lo in [-128, 127], |hi| <= 32.
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
        const int g = k0 / 64, kk = k0 % 64;
        uint8_t* base = xa + (size_t)(tb * NG + g) * 3 * 1024 + (tr + 16 * (kk / 16)) * 16 + kk % 16;
        *(uint2*)(base) = make_uint2(sl[2][0], sl[2][1]);
        *(uint2*)(base + 1024) = make_uint2(sl[1][0], sl[1][1]);
        *(uint2*)(base + 2048) = make_uint2(sl[0][0], sl[0][1]);
        if (kk == 0) {
            const float f = ldexpf(1.0f, -sh);
            xf[(size_t)(tb * NG + g) * 16 + tr] = make_float2(f, (float)xs * f);
        }
    }
}

// ------------------------------------------------------------------------------------------
// q4 GEMM: a workgroup of 8 waves computes 128 tokens x 128 weight rows.  Wave w owns token
// block 8 tm + w (16 tokens) against all 8 row blocks; the row blocks' 1 KiB code chunks and
// scales of each 128-K step are staged once in LDS (double-buffered) and shared by the waves,
// the wave's activation slices stream from global memory straight into registers.  Tiles are
// numbered token-tile-major and dealt to the 8 XCDs in contiguous ranges, so the workgroups of
// one XCD share token tiles in its L2.

template <int K, int EPI>
__global__ __launch_bounds__(512) void pf_gemm_kernel(PfGemmArgs a) {
    constexpr int NG = K / 64, NC = K / 128;
    const int TN = a.N / 128, TM = a.Mpad / 128, T = TM * TN;
    const int per = (T + 7) / 8;
    const int tile = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (tile >= T) return;
    const int tm = tile / TN, tn = tile % TN;

    __shared__ uint4 Bs[2][8][64];
    __shared__ uint32_t SBs[2][2][128];  // [buffer][group of the step][row]

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane >> 4, r16 = lane & 15;
    const int tb = tm * 8 + wave;
    const uint8_t* xa = a.xa + (size_t)tb * NG * 3 * 1024 + lane * 16;
    const float* xf = a.xf + ((size_t)tb * NG * 16 + 4 * q) * 2;
    const uint8_t* wsrc = a.w + (size_t)(tn * 8 + wave) * NC * 1024 + lane * 16;
    const uint32_t* sbsrc = (const uint32_t*)a.sb + (size_t)(tn * 128 + (tid & 127)) * NG + (tid >> 7);

    float acc[8][4];
#pragma unroll
    for (int rb = 0; rb < 8; ++rb)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[rb][i] = 0.f;

    uint4 Ac[2][3], An[2][3];
    float4 Fc[2][2], Fn[2][2];
    uint4 Bn;
    uint32_t SBn = 0;
    auto gload = [&](int c, uint4(&A)[2][3], float4(&F)[2][2]) {
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
#pragma unroll
            for (int s = 0; s < 3; ++s) A[gg][s] = *(const uint4*)(xa + ((size_t)(2 * c + gg) * 3 + s) * 1024);
            F[gg][0] = *(const float4*)(xf + (size_t)(2 * c + gg) * 32);
            F[gg][1] = *(const float4*)(xf + (size_t)(2 * c + gg) * 32 + 4);
        }
        Bn = *(const uint4*)(wsrc + (size_t)c * 1024);
        if (tid < 256) SBn = sbsrc[2 * c];
    };
    auto lstore = [&](int b) {
        Bs[b][wave][lane] = Bn;
        if (tid < 256) SBs[b][tid >> 7][tid & 127] = SBn;
    };

    gload(0, Ac, Fc);
    lstore(0);
    __syncthreads();
    for (int c = 0; c < NC; ++c) {
        const int b = c & 1;
        if (c + 1 < NC) gload(c + 1, An, Fn);
#pragma unroll
        for (int rb = 0; rb < 8; ++rb) {
            const uint4 bw = Bs[b][rb][lane];
#pragma unroll
            for (int gg = 0; gg < 2; ++gg) {
                const uint32_t d0 = gg ? bw.z : bw.x, d1 = gg ? bw.w : bw.y;
                v4i B;
                B[0] = (int)(d0 & 0x0F0F0F0Fu);
                B[1] = (int)((d0 >> 4) & 0x0F0F0F0Fu);
                B[2] = (int)(d1 & 0x0F0F0F0Fu);
                B[3] = (int)((d1 >> 4) & 0x0F0F0F0Fu);
                const v4i zero = {0, 0, 0, 0};
                v4i U = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, Ac[gg][0]), B, zero, 0, 0, 0);
                U = __builtin_bit_cast(v4i, __builtin_bit_cast(v4u, U) << 8u);
                U = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, Ac[gg][1]), B, U, 0, 0, 0);
                U = __builtin_bit_cast(v4i, __builtin_bit_cast(v4u, U) << 8u);
                U = __builtin_amdgcn_mfma_i32_16x16x64_i8(__builtin_bit_cast(v4i, Ac[gg][2]), B, U, 0, 0, 0);
                const f16x2 sbv = as_h2(SBs[b][gg][rb * 16 + r16]);
                const float s = (float)sbv.x, bias = (float)sbv.y;
                const float f[4] = {Fc[gg][0].x, Fc[gg][0].z, Fc[gg][1].x, Fc[gg][1].z};
                const float xs[4] = {Fc[gg][0].y, Fc[gg][0].w, Fc[gg][1].y, Fc[gg][1].w};
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[rb][i] = fmaf(s * f[i], (float)U[i], fmaf(bias, xs[i], acc[rb][i]));
            }
        }
        if (c + 1 < NC) {
            lstore(b ^ 1);
#pragma unroll
            for (int gg = 0; gg < 2; ++gg) {
#pragma unroll
                for (int s = 0; s < 3; ++s) Ac[gg][s] = An[gg][s];
                Fc[gg][0] = Fn[gg][0];
                Fc[gg][1] = Fn[gg][1];
            }
        }
        __syncthreads();
    }

    // Epilogue: lane holds tokens 16 tb + 4 q + i of weight row 128 tn + 16 rb + r16.
#pragma unroll
    for (int rb = 0; rb < 8; ++rb) {
        const int row = tn * 128 + rb * 16 + r16;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = tb * 16 + 4 * q + i;
            const float y = acc[rb][i];
            if constexpr (EPI == EPI_STORE) {
                if (t < a.M) a.y[(size_t)t * a.N + row] = y;
            } else if constexpr (EPI == EPI_RESID) {
                if (t < a.M) {
                    float* xo = a.y + (size_t)t * a.N + row;
                    float v = *xo + y;
                    if (a.ds) {  // DeepStack residual of a visual row (Shaders.swift:696-707)
                        const int vrow = a.row0 + t - a.vis_offset;
                        if (a.vis_offset >= 0 && vrow >= 0 && vrow < a.n_vis) v = v + a.ds[(size_t)vrow * H + row];
                    }
                    *xo = v;
                }
            } else {  // EPI_SWIGLU: block 8 tn + rb = gate units 8 (8 tn + rb) + 0..7, then their up rows
                const float up = __shfl_xor(y, 8);
                if (t < a.M && r16 < 8) a.h[(size_t)t * FF + (tn * 8 + rb) * 8 + r16] = (y / (1.f + expf(-y))) * up;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// Per-head q/k RMSNorm + M-RoPE of every prompt row, K/V written to the fp16 cache, queries
// pre-scaled by 1/sqrt(128) and split into fp16 hi + lo.  Grid (M, 8): wave 4 y + w handles
// vector 4 y + w of row x (q heads 0-15, k groups 16-23, v groups 24-31).

__global__ __launch_bounds__(256) void pf_qk_kernel(PfQkArgs a) {
    const int t = blockIdx.x, lane = threadIdx.x % 64, vec = blockIdx.y * 4 + threadIdx.x / 64;
    if (t >= a.M) return;
    const int slot = a.p0 + t;
    const float* row = a.qkv + (size_t)t * QKV;
    const float* cs = a.rope + (size_t)slot * 128;
    if (vec < NH) {
        float x0 = row[vec * HD + lane], x1 = row[vec * HD + lane + 64];
        norm_rope_pair(x0, x1, a.q_norm, cs, lane);
        const float qscale = 1.0f / sqrtf((float)HD);
        x0 *= qscale;
        x1 *= qscale;
        const size_t o = ((size_t)t * NH + vec) * HD + lane;
        const f16 h0 = (f16)x0, h1 = (f16)x1;
        a.qh[o] = __builtin_bit_cast(uint16_t, h0);
        a.qh[o + 64] = __builtin_bit_cast(uint16_t, h1);
        a.ql[o] = f2h(x0 - (float)h0);
        a.ql[o + 64] = f2h(x1 - (float)h1);
    } else if (vec < NH + NKV) {
        const int g = vec - NH;
        float k0 = row[H + g * HD + lane], k1 = row[H + g * HD + lane + 64];
        norm_rope_pair(k0, k1, a.k_norm, cs, lane);
        uint16_t* kd = a.kc + ((size_t)g * a.maxctx + slot) * HD;
        kd[lane] = f2h(k0);
        kd[lane + 64] = f2h(k1);
    } else {
        const int g = vec - NH - NKV;
        const float* v = row + H + NKV * HD + g * HD;
        uint16_t* vd = a.vc + ((size_t)g * a.maxctx + slot) * HD;
        vd[lane] = f2h(v[lane]);
        vd[lane + 64] = f2h(v[lane + 64]);
    }
}

// ------------------------------------------------------------------------------------------
// Causal GQA flash attention.  Workgroup = (KV group g, 64-token query block); wave w handles
// head 2 g + w / 4 for tokens 16 (w % 4) .. + 15.  Key blocks of 64 slots are staged in LDS
// (K row-major, V transposed; double-buffered) and shared by the 8 waves.  Slots at or beyond
// p0 + M are staged as zeros; causal masking uses cache slots.

constexpr int PA_KB = 64;     // keys per block
constexpr int PA_KROW = 136;  // halves per K row in LDS (128 + 8 pad)
constexpr int PA_VROW = 68;   // halves per V^T row in LDS (64 keys + 4 pad)
constexpr int PA_BUF = PA_KB * PA_KROW + HD * PA_VROW;  // halves per buffer
constexpr size_t PA_LDS = 2 * PA_BUF * 2;

__global__ __launch_bounds__(512) void pf_attn_kernel(PfAttnArgs a) {
    extern __shared__ __align__(16) uint16_t pa_lds[];
    const int QB = (a.M + 63) / 64;
    const int g = (int)(blockIdx.x % NKV), qb = QB - 1 - (int)(blockIdx.x / NKV);
    if (qb < 0) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane >> 4, r16 = lane & 15;
    const int head = 2 * g + (wave >> 2);
    const int t0 = qb * 64 + (wave & 3) * 16;
    const int kv_end = a.p0 + a.M;
    const int nkb = (a.p0 + min(a.M, qb * 64 + 64) - 1) / PA_KB + 1;
    const bool active = t0 < a.M;
    const int w_last = a.p0 + min(a.M - 1, t0 + 15);
    const int qslot = a.p0 + t0 + r16;

    v8h Qh[4], Ql[4];
    {
        const size_t qo = ((size_t)(t0 + r16) * NH + head) * HD + 8 * q;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            Qh[ks] = *(const v8h*)(a.qh + qo + 32 * ks);
            Ql[ks] = *(const v8h*)(a.ql + qo + 32 * ks);
        }
    }
    const uint16_t* kg = a.kc + (size_t)g * a.maxctx * HD;
    const uint16_t* vg = a.vc + (size_t)g * a.maxctx * HD;

    // Staging: K key tid / 8, dims 16 (tid % 8) .. + 15; V keys 4 (tid / 32) .. + 3, dims
    // 4 (tid % 32) .. + 3 (transposed in registers, 8-byte LDS writes).
    uint4 kr[2];
    uint2 vr[4];
    auto gload = [&](int kb) {
        const int ks = kb * PA_KB + (tid >> 3);
        if (ks < kv_end) {
            const uint4* p = (const uint4*)(kg + (size_t)ks * HD + 16 * (tid & 7));
            kr[0] = p[0];
            kr[1] = p[1];
        } else {
            kr[0] = kr[1] = make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int vs = kb * PA_KB + 4 * (tid >> 5) + i;
            vr[i] = vs < kv_end ? *(const uint2*)(vg + (size_t)vs * HD + 4 * (tid & 31)) : make_uint2(0u, 0u);
        }
    };
    auto lstore = [&](int buf) {
        uint16_t* Ks = pa_lds + buf * PA_BUF;
        uint16_t* Vt = Ks + PA_KB * PA_KROW;
        uint4* kd = (uint4*)(Ks + (tid >> 3) * PA_KROW + 16 * (tid & 7));
        kd[0] = kr[0];
        kd[1] = kr[1];
        const int d0 = 4 * (tid & 31), k0 = 4 * (tid >> 5);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            uint32_t e[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) e[i] = ((j < 2 ? vr[i].x : vr[i].y) >> (16 * (j & 1))) & 0xFFFFu;
            *(uint2*)(Vt + (d0 + j) * PA_VROW + k0) = make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
        }
    };

    f32x4 O[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) O[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -__builtin_inff(), l_run = 0.f;

    gload(0);
    lstore(0);
    __syncthreads();
    for (int kb = 0; kb < nkb; ++kb) {
        const int buf = kb & 1;
        if (kb + 1 < nkb) gload(kb + 1);
        if (active && kb * PA_KB <= w_last) {
            const uint16_t* Ks = pa_lds + buf * PA_BUF;
            const uint16_t* Vt = Ks + PA_KB * PA_KROW;
            // S^T tiles: keys 16 kt + (4 q + i) of this lane, query r16.
            f32x4 S[4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                S[kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const v8h kf = *(const v8h*)(Ks + (kt * 16 + r16) * PA_KROW + 32 * ks + 8 * q);
                    S[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, Qh[ks], S[kt], 0, 0, 0);
                    S[kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, Ql[ks], S[kt], 0, 0, 0);
                }
            }
            float mb = -__builtin_inff();
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int key = kb * PA_KB + kt * 16 + 4 * q + i;
                    if (key > qslot) S[kt][i] = -__builtin_inff();
                    mb = fmaxf(mb, S[kt][i]);
                }
            mb = max_x4(mb);
            const float m_new = fmaxf(m_run, mb);  // finite: key slot 0 is in block 0
            const float corr = (m_run == -__builtin_inff()) ? 0.f : expf(m_run - m_new);
            float p[4][4], ls = 0.f;
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    p[kt][i] = (S[kt][i] == -__builtin_inff()) ? 0.f : expf(S[kt][i] - m_new);
                    ls += p[kt][i];
                }
            ls = sum_x4(ls);
            l_run = l_run * corr + ls;
            m_run = m_new;
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) O[dt][i] *= corr;
            // P^T of key tiles 2c, 2c + 1 is the B operand over keys {32 c + 4 q + i, 32 c + 16 + 4 q + i}.
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                v8h Ph, Pl;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const f16 h0 = (f16)p[2 * c][i], h1 = (f16)p[2 * c + 1][i];
                    Ph[i] = h0;
                    Ph[4 + i] = h1;
                    Pl[i] = (f16)(p[2 * c][i] - (float)h0);
                    Pl[4 + i] = (f16)(p[2 * c + 1][i] - (float)h1);
                }
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) {
                    const uint16_t* vp = Vt + (dt * 16 + r16) * PA_VROW + 32 * c + 4 * q;
                    const v4h va = *(const v4h*)vp, vb = *(const v4h*)(vp + 16);
                    const v8h vf = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
                    O[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, Ph, O[dt], 0, 0, 0);
                    O[dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, Pl, O[dt], 0, 0, 0);
                }
            }
        }
        if (kb + 1 < nkb) lstore(buf ^ 1);
        __syncthreads();
    }
    const int t = t0 + r16;
    if (active && t < a.M) {
        const float inv = 1.0f / l_run;
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const float4 o = make_float4(O[dt][0] * inv, O[dt][1] * inv, O[dt][2] * inv, O[dt][3] * inv);
            *(float4*)(a.out + (size_t)t * H + head * HD + dt * 16 + 4 * q) = o;
        }
    }
}

// ------------------------------------------------------------------------------------------

hipError_t launch_pf_prep(int K, int norm, const float* src, const float* norm_w, int M, int Mpad, uint8_t* xa,
                          float* xf, hipStream_t s) {
    if (M < 1 || Mpad < M || Mpad % 128) return hipErrorInvalidValue;
    float2* f2 = (float2*)xf;
    if (K == H && norm)
        hipLaunchKernelGGL((pf_prep_kernel<H, true>), dim3(Mpad), dim3(256), 0, s, src, norm_w, M, xa, f2);
    else if (K == H)
        hipLaunchKernelGGL((pf_prep_kernel<H, false>), dim3(Mpad), dim3(256), 0, s, src, norm_w, M, xa, f2);
    else if (K == FF && !norm)
        hipLaunchKernelGGL((pf_prep_kernel<FF, false>), dim3(Mpad), dim3(256), 0, s, src, norm_w, M, xa, f2);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_pf_gemm(int K, int epi, const PfGemmArgs& a, hipStream_t s) {
    if (a.M < 1 || a.Mpad < a.M || a.Mpad % 128 || a.N % 128) return hipErrorInvalidValue;
    const int T = (a.Mpad / 128) * (a.N / 128);
    const int grid = 8 * ((T + 7) / 8);
    if (K == H && epi == EPI_STORE)
        hipLaunchKernelGGL((pf_gemm_kernel<H, EPI_STORE>), dim3(grid), dim3(512), 0, s, a);
    else if (K == H && epi == EPI_RESID)
        hipLaunchKernelGGL((pf_gemm_kernel<H, EPI_RESID>), dim3(grid), dim3(512), 0, s, a);
    else if (K == H && epi == EPI_SWIGLU)
        hipLaunchKernelGGL((pf_gemm_kernel<H, EPI_SWIGLU>), dim3(grid), dim3(512), 0, s, a);
    else if (K == FF && epi == EPI_RESID)
        hipLaunchKernelGGL((pf_gemm_kernel<FF, EPI_RESID>), dim3(grid), dim3(512), 0, s, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_pf_qk(const PfQkArgs& a, hipStream_t s) {
    if (a.M < 1 || a.p0 < 0 || a.p0 + a.M > a.maxctx) return hipErrorInvalidValue;
    hipLaunchKernelGGL(pf_qk_kernel, dim3(a.M, (NH + 2 * NKV) / 4), dim3(256), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_pf_attn(const PfAttnArgs& a, hipStream_t s) {
    if (a.M < 1 || a.p0 < 0 || a.p0 + a.M > a.maxctx) return hipErrorInvalidValue;
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)pf_attn_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                           (int)PA_LDS);
        if (e != hipSuccess) return e;
        attr_set = true;
    }
    const int QB = (a.M + 63) / 64;
    hipLaunchKernelGGL(pf_attn_kernel, dim3(QB * NKV), dim3(512), PA_LDS, s, a);
    return hipGetLastError();
}

}  // namespace icua
