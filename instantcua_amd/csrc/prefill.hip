// Many-token prefill on the matrix cores, gfx950 (q4, q8 and f16 weights).
//
// Replaces the reference's multi-token path (Shaders.swift:676-1216: k_rmsnorm_rows_h,
// llm_gemm_tile, k_g3_*, k_qk_norm_rope, k_prefill_attn) for prompts longer than one GEMV pass;
// math per tools/reference/qwen3vl_ref.py:243-292 (fp32 activations, fp16 KV cache).
//
// Projections.  q4: y[t][r] = sum_g (s_rg sum_{k in g} q_rk x_tk + b_rg sum_{k in g} x_tk) over
// 64-groups; q8: y[t][r] = sum_g s_rg sum_{k in g} q_rk x_tk over 32-groups; f16: y = W x.  A prep
// kernel scales every activation row by a power of two that puts its largest |x| in
// [2^14, 2^15) and splits it into fp16 hi + lo parts (x'' = hi + lo to ~22 bits; the scaling
// keeps every part that matters far above the fp16 subnormal range).  The GEMM runs
// v_mfma_f32_16x16x32_f16 on (hi, lo) x the weights as fp16 B operands: the q4 and q8 integer
// codes are exact in fp16, so each group's sum C_g = sum_k q_k x''_k comes out of one
// accumulator chain; the group epilogue is acc += s C_g (q4 and q8: the q4 bias term
// sum_g b_g X_g, X_g = sum_k x''_k, runs on the matrix cores once per tile before the loop),
// f16 weights accumulate directly, and the row scale 2^(E_t - 14) is applied once at the end.
// With fp16 operands alone (ICUA_FLAG_PREFILL_FP16, the reference engine's precision) there is
// no lo part, and the B operands are the weights dequantised to fp16 (q4 fp16(s q + b), q8
// fp16(s q)), so the products accumulate straight into the outputs with no group epilogue.
//
// Attention.  Causal GQA flash attention on v_mfma_f32_16x16x32_f16: scores are computed
// transposed (S^T = K Q^T) so that the probabilities come out of the accumulator already in
// the B-operand layout of the P.V product (O^T = V^T P^T); V is transposed through LDS.  The
// fp32 queries and probabilities are split into fp16 hi + lo parts (two products each), which
// keeps them at ~22 bits against the fp16 cache (one part with fp16 operands alone).  Each wave
// holds 32 queries, so every K and V operand it reads from LDS feeds two products.
#include "icua_device.h"
#include "icua_kernels.h"

namespace icua {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v4h __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------
// Activation operands.  XA: [Mpad / 16][K / 32][2 (hi, lo)][64 lanes][8 halves], lane l
// holding token 16 tb + l % 16, K = 32 ks + 8 (l / 16) + 0..7.  XS: [Mpad / 16][K / 64][16]
// group sums of hi + lo.  TS: [Mpad] row scales 2^(E_t - 14).  One workgroup per token row
// (rows >= M are zero).  A row writes 16-byte pieces of lines that the 16 rows of its token
// block share, so rows are dealt to the 8 XCDs (workgroup i runs on XCD i % 8) in contiguous
// ranges: the lines are completed in one L2 rather than written back in parts from eight.

template <int K, bool NORM, int HL>
__global__ __launch_bounds__(256) void pf_prep_kernel(const float* __restrict__ src, const float* __restrict__ norm_w,
                                                      int M, uint16_t* __restrict__ xa, float* __restrict__ xs,
                                                      float* __restrict__ ts) {
    constexpr int NU = K / 8 / 256;  // units of 8 activations per thread
    constexpr int NG = K / 64, NKS = K / 32;
    const int t = (int)(blockIdx.x % 8) * (int)(gridDim.x / 8) + (int)(blockIdx.x / 8);  // gridDim.x % 8 == 0
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    __shared__ float red[8];
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
    // Row exponent: largest |x| in [2^E, 2^(E+1)).
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < NU; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[j][i]));
    amax = wave_max(amax);
    if (lane == 0) red[4 + wave] = amax;
    __syncthreads();
    const float rmax = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
    const int E = (rmax > 0.f) ? ((int)((as_u32(rmax) >> 23) & 0xFF) - 127) : 0;
    const int sh = 14 - E;
    const int tb = t >> 4, tr = t & 15;
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        const int k0 = (tid + 256 * j) * 8;
        uint32_t hw[4], lw[4];
        float gs = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float x0 = ldexpf(v[j][2 * i], sh), x1 = ldexpf(v[j][2 * i + 1], sh);
            const f16 h0 = (f16)x0, h1 = (f16)x1;
            const f16 l0 = (f16)(x0 - (float)h0), l1 = (f16)(x1 - (float)h1);
            if constexpr (HL == 2)
                gs += ((float)h0 + (float)l0) + ((float)h1 + (float)l1);
            else
                gs += (float)h0 + (float)h1;
            hw[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            lw[i] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
        }
        // Group sums over the 8 adjacent lanes holding the group's 64 values.
        gs += dpp<DPP_XOR1>(gs);
        gs += dpp<DPP_XOR2>(gs);
        gs += dpp<DPP_HALF_MIRROR>(gs);
        const int ks = k0 / 32, qq = (k0 % 32) / 8;
        uint16_t* base = xa + ((size_t)(tb * NKS + ks) * HL) * 512 + (tr + 16 * qq) * 8;
        *(uint4*)base = make_uint4(hw[0], hw[1], hw[2], hw[3]);
        if constexpr (HL == 2) *(uint4*)(base + 512) = make_uint4(lw[0], lw[1], lw[2], lw[3]);
        if (k0 % 64 == 0) xs[(size_t)(tb * NG + k0 / 64) * 16 + tr] = gs;
    }
    if (tid == 0) ts[t] = ldexpf(1.0f, -sh);
}

// ------------------------------------------------------------------------------------------
// GEMM: a workgroup of 8 waves computes 64 TB tokens x 16 RB weight rows (TB = 1 or 2 token
// blocks per wave, RB = 8 or 16 row blocks); wave w owns token blocks 4 TB tm + TB (w % 4) ..
// against row blocks RB / 2 (w / 4) onwards (RB / 2 row blocks), two waves per SIMD, and takes
// its row blocks in halves of four per group.  Each 128-K step, the weight chunks of the RB row
// blocks (q4 one 1 KiB chunk, q8 two, f16 four) become fp16 B operands in LDS once
// (double-buffered, 64 or 128 KiB) and are shared by the waves; the waves' activation operands
// stream from global memory straight into registers two 64-K groups ahead.  The launch takes
// the largest tile (most products per operand byte) whose count still fills the CUs evenly.
template <int FMT, int K, int EPI, int PG_RB, int TB, int HL>
__global__ __launch_bounds__(512) void pf_gemm_kernel(PfGemmArgs a) {
    static_assert((PG_RB == 8 || PG_RB == 16) && (TB == 1 || TB == 2), "tile shape");
    constexpr int NHF = PG_RB / 8;         // halves of four row blocks per wave
    constexpr int TR = 16 * PG_RB;         // rows of a tile
    constexpr int NG = K / 64, NKS = K / 32, NC = K / 128;
    constexpr int CPS = FMT == FMT_Q4 ? 1 : FMT == FMT_Q8 ? 2 : 4;  // 1 KiB chunks per 128-K step
    constexpr int NCH = NC * CPS;                                      // chunks per row block
    // DQ: the B operands are the dequantised weights in fp16 (q4 s q + b, q8 s q: the reference
    // engine's prefill precision, taken with fp16 operands alone) or the f16 weights themselves,
    // so the products accumulate straight into the outputs; otherwise q4 / q8 codes are exact
    // fp16 integers and each group's sums take their scale in an epilogue.
    constexpr bool DQ = HL == 1 || FMT == FMT_F16;
    const int TN = a.N / (16 * PG_RB), TM = a.Mpad / (64 * TB), T = TM * TN;
    const int per = (T + 7) / 8;
    const int tile = (int)(blockIdx.x % 8) * per + (int)(blockIdx.x / 8);
    if (tile >= T) return;
    const int tm = tile / TN, tn = tile % TN;

    __shared__ uint4 Bs[2][PG_RB][4][64];  // fp16 codes: [buffer][row block][k-step][lane]
    // Per-step words: [buffer][i] fp16 (scale, bias) of group 2 c + i / TR, row i % TR.
    __shared__ __attribute__((aligned(16))) uint32_t Vs[2][512];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane >> 4, r16 = lane & 15;
    const int tb0 = tm * 4 * TB + TB * (wave & 3), rb0 = (PG_RB / 2) * (wave >> 2);
    const uint16_t* xa = a.xa + (size_t)tb0 * NKS * 512 * HL + lane * 8;   // token block tb0 (+ NKS * 512 HL for tb0 + 1)
    // Staging: thread t unpacks nibble lane t % 64 of row block t / 64 (and t / 64 + 8).
    const int srb = tid >> 6;
    const uint8_t* wsrc = a.w + (size_t)(tn * PG_RB + srb) * NCH * 1024 + lane * 16;
    constexpr size_t WSRC2 = (size_t)8 * NCH * 1024;  // row block srb + 8
    // Thread t < 2 TR loads one scale word per step (stride 2 words): row t % TR of the tile, q4
    // the (scale, bias) half2 of 64-group 2 c + t / TR; q8 the scales of 32-groups
    // 4 c + 2 (t / TR), + 1 (the same word offsets: a q8 row holds K / 64 words of scale pairs).
    // f16 weights have no scales.
    const uint32_t* vsrc = (const uint32_t*)a.sb + (size_t)(tn * TR + (tid % TR)) * NG + (tid / TR);
    constexpr int vstride = 2;
    const bool vload = !DQ && (2 * TR >= 512 || tid < 2 * TR);
    // DQ q4 / q8: the unpacking thread's own scale words, row (tn RB + srb + 8 hb) 16 + lane % 16,
    // words 2 c and 2 c + 1 of step c (q4 the (scale, bias) of 64-groups 2 c, 2 c + 1; q8 the
    // scales of 32-groups 4 c .. 4 c + 3).
    const uint32_t* dsrc = (const uint32_t*)a.sb + (size_t)((tn * PG_RB + srb) * 16 + (lane & 15)) * NG;
    constexpr size_t DSRC2 = (size_t)8 * 16 * NG;  // row block srb + 8

    f32x4 acc[TB][4 * NHF];
#pragma unroll
    for (int i = 0; i < TB; ++i)
#pragma unroll
        for (int r = 0; r < 4 * NHF; ++r) acc[i][r] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Activation operands of one 64-group (two k-steps), prefetched one group ahead.
    uint4 Ae[TB][2][HL], Ao[TB][2][HL];  // [token block][k-step of the group][hi, lo]
    uint4 Wn[NHF][CPS];
    uint32_t Vn = 0;
    uint32_t Dn[NHF][2];
    auto aload = [&](int g, uint4(&A)[TB][2][HL]) {
#pragma unroll
        for (int i = 0; i < TB; ++i) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int hl = 0; hl < HL; ++hl)
                    A[i][kk][hl] = *(const uint4*)(xa + (size_t)i * NKS * 512 * HL + ((size_t)(2 * g + kk) * HL + hl) * 512);
        }
    };
    auto wload = [&](int c) {
#pragma unroll
        for (int hb = 0; hb < NHF; ++hb)
#pragma unroll
            for (int j = 0; j < CPS; ++j) Wn[hb][j] = *(const uint4*)(wsrc + hb * WSRC2 + (size_t)(c * CPS + j) * 1024);
        if (vload) Vn = vsrc[(size_t)c * vstride];
        if constexpr (DQ && FMT != FMT_F16) {
#pragma unroll
            for (int hb = 0; hb < NHF; ++hb)
#pragma unroll
                for (int j = 0; j < 2; ++j) Dn[hb][j] = dsrc[hb * DSRC2 + 2 * c + j];
        }
    };
    // Nibble lane L (row L % 16, 16-K slot L / 16 of each group) -> fp16 lanes (L % 16) + 16 (2 (slot % 2) + h)
    // of k-step 2 gg + slot / 2, h = 0 for K 0..7 of the slot, 1 for K 8..15.
    auto lstore = [&](int b) {
#pragma unroll
      for (int hb = 0; hb < NHF; ++hb) {
        const int sr = srb + 8 * hb;
        if constexpr (FMT == FMT_F16) {
            // f16 chunk j is k-step j, already in the B-operand lane layout.
#pragma unroll
            for (int j = 0; j < 4; ++j) Bs[b][sr][j][lane] = Wn[hb][j];
            continue;
        } else if constexpr (FMT == FMT_Q8) {
            // q8 chunk j: bytes 0-7 of a lane are k-step 2 j (K-slot lane / 16 of row lane % 16),
            // bytes 8-15 k-step 2 j + 1, the B-operand lane layout; a signed byte b spread into a
            // 16-bit lane, xor 0x80 and or'ed into 0x6400, is the fp16 value 1152 + b, and one
            // packed fp16 subtraction leaves b exactly.
            const f16x2 k1152 = {(f16)1152.f, (f16)1152.f};
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const uint32_t dd[4] = {Wn[hb][j].x, Wn[hb][j].y, Wn[hb][j].z, Wn[hb][j].w};
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    uint32_t o[4];
                    // DQ: k-step 2 j + h is 32-group 4 c + 2 j + h, the scale in half h of word 2 c + j.
                    const f16 sc = DQ ? (h ? as_h2(Dn[hb][j]).y : as_h2(Dn[hb][j]).x) : (f16)1.f;
                    const f16x2 sc2 = {sc, sc};
#pragma unroll
                    for (int w2 = 0; w2 < 2; ++w2) {
                        const uint32_t d = dd[2 * h + w2];
                        const uint32_t s0 = __builtin_amdgcn_perm(d, d, 0x0C010C00u);  // b0, b1
                        const uint32_t s1 = __builtin_amdgcn_perm(d, d, 0x0C030C02u);  // b2, b3
                        f16x2 q0 = as_h2((s0 ^ 0x00800080u) | 0x64006400u) - k1152;
                        f16x2 q1 = as_h2((s1 ^ 0x00800080u) | 0x64006400u) - k1152;
                        if constexpr (DQ) {
                            q0 = q0 * sc2;
                            q1 = q1 * sc2;
                        }
                        o[2 * w2] = h2_bits(q0);
                        o[2 * w2 + 1] = h2_bits(q1);
                    }
                    Bs[b][sr][2 * j + h][lane] = make_uint4(o[0], o[1], o[2], o[3]);
                }
            }
            continue;
        } else {
        const int r = lane & 15, slot = lane >> 4;
        const uint32_t dd[4] = {Wn[hb][0].x, Wn[hb][0].y, Wn[hb][0].z, Wn[hb][0].w};
#pragma unroll
        for (int gg = 0; gg < 2; ++gg) {
            // DQ: 64-group 2 c + gg of this row, (scale, bias) in word 2 c + gg.
            const f16x2 sbw = as_h2(DQ ? Dn[hb][gg] : 0x00003C00u);
            const f16x2 sc2 = {sbw.x, sbw.x}, bi2 = {sbw.y, sbw.y};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t d = dd[2 * gg + h];
                uint32_t o[4];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    // K 8 h + 2 j, + 1 are the low nibbles of bytes 2 j, 2 j + 1; K 8 h + 4 + 2 j, + 1 the
                    // high ones.  Bytes spread to 16-bit lanes, a nibble or'ed into 0x6400 is the fp16
                    // value 1024 + q, and one packed fp16 subtraction leaves q exactly.
                    const uint32_t sp = __builtin_amdgcn_perm(d, d, 0x0C000C00u | ((2u * j + 1u) << 16) | (2u * j));
                    const f16x2 k1024 = {(f16)1024.f, (f16)1024.f};
                    f16x2 qa = as_h2((sp & 0x000F000Fu) | 0x64006400u) - k1024;
                    f16x2 qb = as_h2(((sp >> 4) & 0x000F000Fu) | 0x64006400u) - k1024;
                    if constexpr (DQ) {  // one rounding each: fma in fp16
                        qa = __builtin_elementwise_fma(qa, sc2, bi2);
                        qb = __builtin_elementwise_fma(qb, sc2, bi2);
                    }
                    o[j] = h2_bits(qa);
                    o[2 + j] = h2_bits(qb);
                }
                Bs[b][sr][2 * gg + (slot >> 1)][r + 16 * (2 * (slot & 1) + h)] = make_uint4(o[0], o[1], o[2], o[3]);
            }
        }
        }
      }
        if constexpr (!DQ) Vs[b][tid] = Vn;
    };
    // One activation operand (token block tb0 + i, k-step kk of group g, hi / lo part hl).
    auto aload1 = [&](int g, int i, int kk, int hl) {
        return *(const uint4*)(xa + (size_t)i * NKS * 512 * HL + ((size_t)(2 * g + kk) * HL + hl) * 512);
    };
    // One 64-group, in halves of four row blocks: a half's 8 B fragments first, then 4 x 2
    // accumulator chains of 4 MFMAs, then its scale epilogue.  In the last half, each activation
    // register is requested again for group gn (two groups on) as soon as its last product is
    // issued, so the loads have two groups' work to land in.
    auto group = [&](int b, int gg, uint4(&Ac)[TB][2][HL], int gn) {
#pragma unroll
      for (int hf = 0; hf < NHF; ++hf) {
        v8h Bf[4][2];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) Bf[r][kk] = __builtin_bit_cast(v8h, Bs[b][rb0 + 4 * hf + r][2 * gg + kk][lane]);
        if constexpr (DQ) {
#pragma unroll
            for (int kk = 0; kk < 2; ++kk)
#pragma unroll
                for (int hl = 0; hl < HL; ++hl) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int i = 0; i < TB; ++i)
                            acc[i][4 * hf + r] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                __builtin_bit_cast(v8h, Ac[i][kk][hl]), Bf[r][kk], acc[i][4 * hf + r], 0, 0, 0);
                    if (hf == NHF - 1) {
#pragma unroll
                        for (int i = 0; i < TB; ++i) Ac[i][kk][hl] = aload1(gn, i, kk, hl);
                    }
                }
            continue;
        }
        float2 sb[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const f16x2 sb2 = as_h2(Vs[b][gg * TR + (rb0 + 4 * hf + r) * 16 + r16]);
            sb[r] = make_float2((float)sb2.x, (float)sb2.y);  // q4 (scale, bias); q8 the two 32-groups' scales
        }
        if constexpr (FMT == FMT_Q8) {
            // Two 32-groups, one k-step each.
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                f32x4 C[4][TB];
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int i = 0; i < TB; ++i) C[r][i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int hl = 0; hl < HL; ++hl) {
#pragma unroll
                    for (int r = 0; r < 4; ++r)
#pragma unroll
                        for (int i = 0; i < TB; ++i)
                            C[r][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, Ac[i][kk][hl]),
                                                                             Bf[r][kk], C[r][i], 0, 0, 0);
                    if (hf == NHF - 1) {
#pragma unroll
                        for (int i = 0; i < TB; ++i) Ac[i][kk][hl] = aload1(gn, i, kk, hl);
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int i = 0; i < TB; ++i)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[i][4 * hf + r][e] = fmaf(kk ? sb[r].y : sb[r].x, C[r][i][e], acc[i][4 * hf + r][e]);
            }
            continue;
        }
        f32x4 C[4][TB];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < TB; ++i) C[r][i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
#pragma unroll
            for (int hl = 0; hl < HL; ++hl) {
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int i = 0; i < TB; ++i)
                        C[r][i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, Ac[i][kk][hl]), Bf[r][kk],
                                                                         C[r][i], 0, 0, 0);
                if (hf == NHF - 1) {
#pragma unroll
                    for (int i = 0; i < TB; ++i) Ac[i][kk][hl] = aload1(gn, i, kk, hl);
                }
            }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int i = 0; i < TB; ++i) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // q4: the bias term sum_g b_g X_g went in before the loop
                    acc[i][4 * hf + r][e] = fmaf(sb[r].x, C[r][i][e], acc[i][4 * hf + r][e]);
                }
            }
      }
    };

    // Even groups use Ae, odd groups Ao: each register is reloaded (for two groups on) as its
    // group's last product using it issues, so no register copy waits on an outstanding load.
    aload(0, Ae);
    aload(1, Ao);
    wload(0);
    if constexpr (FMT == FMT_Q4 && !DQ) {
        // The q4 bias term sum_g b_g X_g of every output, on the matrix cores before the loop:
        // per 32 groups, A = the token block's group sums X (scaled by 2^-8 into fp16 range,
        // hi + lo parts) and B = the rows' fp16 biases, exact.  The loop's group epilogue is then
        // one fma per output (acc += s C_g).
#pragma unroll 1
        for (int cg = 0; cg < NG / 32; ++cg) {
            v8h Xh[TB], Xl[TB], Bb[4];
#pragma unroll
            for (int i = 0; i < TB; ++i) {
                const float* xp = a.xs + ((size_t)(tb0 + i) * NG + 32 * cg + 8 * q) * 16 + r16;
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float x = xp[16 * j] * 0.00390625f;  // 2^-8: a group sum of 64 values below 2^15
                    const f16 hx = (f16)x;
                    Xh[i][j] = hx;
                    Xl[i][j] = (f16)(x - (float)hx);
                }
            }
#pragma unroll
            for (int hf = 0; hf < NHF; ++hf) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint4* bp = (const uint4*)((const uint32_t*)a.sb +
                                                     (size_t)(tn * TR + (rb0 + 4 * hf + r) * 16 + r16) * NG + 32 * cg + 8 * q);
                    const uint4 w0 = bp[0], w1 = bp[1];
                    const uint32_t wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
                    for (int j = 0; j < 8; ++j) Bb[r][j] = as_h2(wv[j]).y;
                }
#pragma unroll
                for (int r = 0; r < 4; ++r)
#pragma unroll
                    for (int i = 0; i < TB; ++i) {
                        f32x4 B = f32x4{0.f, 0.f, 0.f, 0.f};
                        B = __builtin_amdgcn_mfma_f32_16x16x32_f16(Xh[i], Bb[r], B, 0, 0, 0);
                        B = __builtin_amdgcn_mfma_f32_16x16x32_f16(Xl[i], Bb[r], B, 0, 0, 0);
#pragma unroll
                        for (int e = 0; e < 4; ++e) acc[i][4 * hf + r][e] = fmaf(256.f, B[e], acc[i][4 * hf + r][e]);
                    }
            }
        }
    }
    lstore(0);
    __syncthreads();
    for (int c = 0; c < NC; ++c) {
        const int b = c & 1;
        // The next step's codes (the last step reloads step 0 into the idle buffer: no branch).
        wload(c + 1 < NC ? c + 1 : 0);
        group(b, 0, Ae, 2 * c + 2 < NG ? 2 * c + 2 : 0);
        group(b, 1, Ao, 2 * c + 3 < NG ? 2 * c + 3 : 1);
        lstore(b ^ 1);
        __syncthreads();
    }

    // Epilogue: lane holds tokens 16 tb + 4 q + e of weight row TR tn + 16 rb + r16.
#pragma unroll
    for (int i = 0; i < TB; ++i) {
        const int tq = (tb0 + i) * 16 + 4 * q;
        const float4 tsv = *(const float4*)(a.ts + tq);
        const float tsc[4] = {tsv.x, tsv.y, tsv.z, tsv.w};
#pragma unroll
        for (int r = 0; r < 4 * NHF; ++r) {
            const int rb = rb0 + r;
            const int row = tn * TR + rb * 16 + r16;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int t = tq + e;
                const float y = acc[i][r][e] * tsc[e];
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
                } else {  // EPI_SWIGLU: block RB tn + rb = gate units 8 (RB tn + rb) + 0..7, then their up rows
                    const float up = dpp<0x128>(y);  // lane r16 ^ 8 of the row of 16 (a rotation by 8)
                    const float hv = y * __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-y * 1.4426950408889634f)) * up;
                    if (t < a.M && r16 < 8) a.h[(size_t)t * FF + (tn * PG_RB + rb) * 8 + r16] = hv;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------
// Per-head q/k RMSNorm + M-RoPE of every prompt row, K/V written to the fp16 cache, queries
// pre-scaled by log2(e) / sqrt(128) and split into fp16 hi + lo.  Grid (M, 8): wave 4 y + w handles
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
        // 1/sqrt(128) and log2(e): the scores come out in base-2 units, so every softmax
        // exponential of the attention is one v_exp_f32.
        const float qscale = (1.0f / sqrtf((float)HD)) * 1.4426950408889634f;
        x0 *= qscale;
        x1 *= qscale;
        const size_t o = ((size_t)t * NH + vec) * HD + lane;
        const f16 h0 = (f16)x0, h1 = (f16)x1;
        a.qh[o] = __builtin_bit_cast(uint16_t, h0);
        a.qh[o + 64] = __builtin_bit_cast(uint16_t, h1);
        if (a.ql) {
            a.ql[o] = f2h(x0 - (float)h0);
            a.ql[o + 64] = f2h(x1 - (float)h1);
        }
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
// Causal GQA flash attention.  Workgroup = (KV group g, 64-token query block), 8 waves.  Wave w
// handles head 2 g + ((w >> 1) & 1) for tokens 32 (w & 1) .. + 31 of the block as two 16-row
// query tiles, so every K and V operand it reads from LDS feeds two products.  Each iteration
// stages 128 key slots in LDS as two 64-slot halves (K row-major, V transposed; double-buffered)
// and wave w takes half w >> 2: the two key-parity waves of a (head, tokens) pair keep separate
// running softmax states, merged through LDS after the last iteration.  Slots at or beyond the
// block's last query are masked for all of its queries; causal masking uses cache slots.  The
// softmax denominators come from the matrix cores too: a ones operand against the probabilities.

typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

constexpr int PA_KB = 64;     // keys per half
constexpr int PA_KROW = 136;  // halves per K row in LDS (128 + 8 pad)
constexpr int PA_VROW = 68;   // halves per V^T row in LDS (64 keys + 4 pad)
constexpr int PA_BUF = PA_KB * PA_KROW + HD * PA_VROW;  // halves per 64-slot half
constexpr size_t PA_LDS = 4 * PA_BUF * 2;                // two stages of two halves: 139,264 B

template <int HL>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2, 2))) void pf_attn_kernel(PfAttnArgs a) {
    extern __shared__ __align__(16) uint16_t pa_lds[];
    const int QB = (a.M + 63) / 64;
    const int g = (int)(blockIdx.x % NKV), qb = QB - 1 - (int)(blockIdx.x / NKV);
    if (qb < 0) return;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, q = lane >> 4, r16 = lane & 15;
    const int par = wave >> 2, wi = wave & 3;
    const int head = 2 * g + (wi >> 1);
    const int t0 = qb * 64 + 32 * (wi & 1);
    const int kv_lim = a.p0 + min(a.M, qb * 64 + 64);  // past the block's last query slot
    const int nkb = (kv_lim - 1) / PA_KB + 1;          // 64-slot key halves with unmasked keys
    const int nit = (nkb + 1) / 2;
    const bool active = t0 < a.M;
    const int w_first = a.p0 + t0;
    const int w_last = a.p0 + min(a.M - 1, t0 + 31);

    v8h Qh[2][4], Ql[2][4];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        const size_t qo = ((size_t)(t0 + 16 * u + r16) * NH + head) * HD + 8 * q;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            Qh[u][ks] = *(const v8h*)(a.qh + qo + 32 * ks);
            if constexpr (HL == 2) Ql[u][ks] = *(const v8h*)(a.ql + qo + 32 * ks);
        }
    }
    const uint16_t* kg = a.kc + (size_t)g * a.maxctx * HD;
    const uint16_t* vg = a.vc + (size_t)g * a.maxctx * HD;

    // Staging of half hb: K key tid / 8, dims 16 (tid % 8) .. + 15; V keys 4 (tid / 32) .. + 3,
    // dims 4 (tid % 32) .. + 3 (transposed in registers, 8-byte LDS writes).
    uint4 kr0[2], kr1[2];
    uint2 vr0[4], vr1[4];
    // Staging through buffer resources bounded at kv_lim: slots at or past it (masked for every
    // query of the block) read as zeros, with no branch.  Half hb of iteration it: K key tid / 8,
    // dims 16 (tid % 8) .. + 15; V keys 4 (tid / 32) .. + 3, dims 4 (tid % 32) .. + 3 (transposed
    // in registers, 8-byte LDS writes).
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)kg, (short)0, kv_lim * HD * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)vg, (short)0, kv_lim * HD * 2, 0x00020000);
    struct Half {
        u32x4 k0, k1;
        u32x2 v0, v1, v2, v3;
    };
    Half h0, h1;
    const int koff = ((tid >> 3) * HD + 16 * (tid & 7)) * 2, voff = (4 * (tid >> 5) * HD + 4 * (tid & 31)) * 2;
    auto gload_half = [&](int base, Half& h) {
        const int o = base * HD * 2;
        h.k0 = __builtin_amdgcn_raw_buffer_load_b128(krs, o + koff, 0, 0);
        h.k1 = __builtin_amdgcn_raw_buffer_load_b128(krs, o + koff + 16, 0, 0);
        h.v0 = __builtin_amdgcn_raw_buffer_load_b64(vrs, o + voff, 0, 0);
        h.v1 = __builtin_amdgcn_raw_buffer_load_b64(vrs, o + voff + HD * 2, 0, 0);
        h.v2 = __builtin_amdgcn_raw_buffer_load_b64(vrs, o + voff + HD * 4, 0, 0);
        h.v3 = __builtin_amdgcn_raw_buffer_load_b64(vrs, o + voff + HD * 6, 0, 0);
    };
    auto gload = [&](int it) {
        gload_half(2 * it * PA_KB, h0);
        gload_half((2 * it + 1) * PA_KB, h1);
    };
    auto lstore_half = [&](uint16_t* Ks, const Half& h) {
        uint16_t* Vt = Ks + PA_KB * PA_KROW;
        u32x4* kd = (u32x4*)(Ks + (tid >> 3) * PA_KROW + 16 * (tid & 7));
        kd[0] = h.k0;
        kd[1] = h.k1;
        const int d0 = 4 * (tid & 31), k0 = 4 * (tid >> 5);
        // Output row d0 + j holds dim d0 + j of keys k0 .. k0 + 3: byte selects from the four rows.
        const u32x2 vr[4] = {h.v0, h.v1, h.v2, h.v3};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int w = j >> 1;
            const unsigned sel = (j & 1) ? 0x07060302u : 0x05040100u;  // high or low halves of two words
            *(u32x2*)(Vt + (d0 + j) * PA_VROW + k0) =
                u32x2{__builtin_amdgcn_perm(vr[1][w], vr[0][w], sel), __builtin_amdgcn_perm(vr[3][w], vr[2][w], sel)};
        }
    };
    auto lstore = [&](int stage) {
        lstore_half(pa_lds + (2 * stage) * PA_BUF, h0);
        lstore_half(pa_lds + (2 * stage + 1) * PA_BUF, h1);
    };

    f32x4 O[2][8], Lr[2];  // Lr: the running denominator of query r16 in every element
#pragma unroll
    for (int u = 0; u < 2; ++u) {
        Lr[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) O[u][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    float m_run[2] = {-__builtin_inff(), -__builtin_inff()};
    const f16 one = (f16)1.0f;
    const v8h ones = {one, one, one, one, one, one, one, one};

    gload(0);
    lstore(0);
    __syncthreads();
    for (int it = 0; it < nit; ++it) {
        const int st = it & 1;
        if (it + 1 < nit) gload(it + 1);
        const int kb = 2 * it + par;
        if (active && kb * PA_KB <= w_last) {
            const uint16_t* Ks = pa_lds + (2 * st + par) * PA_BUF;
            const uint16_t* Vt = Ks + PA_KB * PA_KROW;
            // S^T tiles: keys 16 kt + (4 q + i) of this lane, query r16 of tile u.
            f32x4 S[2][4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                S[0][kt] = S[1][kt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const v8h kf = *(const v8h*)(Ks + (kt * 16 + r16) * PA_KROW + 32 * ks + 8 * q);
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        S[u][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, Qh[u][ks], S[u][kt], 0, 0, 0);
                        if constexpr (HL == 2)
                            S[u][kt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, Ql[u][ks], S[u][kt], 0, 0, 0);
                    }
                }
            }
            // Schedule: the K operands of key tile kt + 1 are read while tile kt's products issue.
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
            for (int kt = 0; kt < 4; ++kt) {
                __builtin_amdgcn_sched_group_barrier(0x008, 8 * HL, 0);
                if (kt < 2) __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
            }
            // Masking only where some key of the half lies past some query of the wave (a
            // wave-uniform branch: the halves below the diagonal skip it).
            if (kb * PA_KB + PA_KB - 1 > w_first) {
                asm volatile("");  // keeps the branch: the selects below are not speculated
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int qslot = w_first + 16 * u + r16;
#pragma unroll
                    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (kb * PA_KB + kt * 16 + 4 * q + i > qslot) S[u][kt][i] = -__builtin_inff();
                }
            }
            v8h Ph[2][2], Pl[2][2];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                float mb = -__builtin_inff();
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) mb = fmaxf(mb, S[u][kt][i]);
                mb = max_x4(mb);
                const float m_new = fmaxf(m_run[u], mb);
                const float corr = m_new == m_run[u] ? 1.f
                                 : m_run[u] == -__builtin_inff() ? 0.f
                                 : __builtin_amdgcn_exp2f(m_run[u] - m_new);
                // A query whose keys so far are all masked keeps m = -inf: subtract 0 there, so
                // that every masked score gives exp2(-inf) = 0 without a per-element test.
                const float m_use = m_new == -__builtin_inff() ? 0.f : m_new;
                float p[4][4];
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) p[kt][i] = __builtin_amdgcn_exp2f(S[u][kt][i] - m_use);
                m_run[u] = m_new;
                // The running maximum settles after the first blocks: rescale only when it moved.
                if (__builtin_amdgcn_ballot_w64(corr != 1.f)) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) Lr[u][i] *= corr;
#pragma unroll
                    for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                        for (int i = 0; i < 4; ++i) O[u][dt][i] *= corr;
                }
                // P^T of key tiles 2c, 2c + 1 is the B operand over keys {32 c + 4 q + i, 32 c + 16 + 4 q + i}.
#pragma unroll
                for (int c = 0; c < 2; ++c)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const f16 h0 = (f16)p[2 * c][i], h1 = (f16)p[2 * c + 1][i];
                        Ph[u][c][i] = h0;
                        Ph[u][c][4 + i] = h1;
                        if constexpr (HL == 2) {
                            Pl[u][c][i] = (f16)(p[2 * c][i] - (float)h0);
                            Pl[u][c][4 + i] = (f16)(p[2 * c + 1][i] - (float)h1);
                        }
                    }
            }
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    Lr[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, Ph[u][c], Lr[u], 0, 0, 0);
                    if constexpr (HL == 2) Lr[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ones, Pl[u][c], Lr[u], 0, 0, 0);
                }
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) {
                    const uint16_t* vp = Vt + (dt * 16 + r16) * PA_VROW + 32 * c + 4 * q;
                    const v4h va = *(const v4h*)vp, vb = *(const v4h*)(vp + 16);
                    const v8h vf = {va[0], va[1], va[2], va[3], vb[0], vb[1], vb[2], vb[3]};
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        O[u][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, Ph[u][c], O[u][dt], 0, 0, 0);
                        if constexpr (HL == 2)
                            O[u][dt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(vf, Pl[u][c], O[u][dt], 0, 0, 0);
                    }
                }
            // Schedule (fp16 operands alone; the hi + lo instance measured faster without it):
            // each group of four V operands is read two groups ahead of its products.
            if constexpr (HL == 1) {
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
                __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
                __builtin_amdgcn_sched_group_barrier(0x002 | 0x400, 200, 1);
                __builtin_amdgcn_sched_group_barrier(0x008, 4, 1);
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 8, 1);
                    if (k < 2) __builtin_amdgcn_sched_group_barrier(0x100, 4, 1);
                }
            }
        }
        if (it + 1 < nit) lstore(st ^ 1);
        __syncthreads();
    }

    // Key-parity merge: waves 4..7 hand (O, m, l) to waves 0..3 through LDS (free after the loop's
    // last barrier).  Waves 0..3 always have a finite maximum: half 0 holds key slot 0.
    float* mo = (float*)pa_lds;               // [4 waves][2 tiles][8 dim tiles][64 lanes] x 4
    float* mml = mo + 4 * 2 * 8 * 64 * 4;     // [4 waves][2 tiles][64 lanes] x (m, l)
    if (par == 1) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
#pragma unroll
            for (int dt = 0; dt < 8; ++dt) *(f32x4*)(mo + (((wi * 2 + u) * 8 + dt) * 64 + lane) * 4) = O[u][dt];
            *(float2*)(mml + ((wi * 2 + u) * 64 + lane) * 2) = make_float2(m_run[u], Lr[u][0]);
        }
    }
    __syncthreads();
    if (par == 0 && active) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            const int t = t0 + 16 * u + r16;
            const float2 ml1 = *(const float2*)(mml + ((wi * 2 + u) * 64 + lane) * 2);
            const float m = fmaxf(m_run[u], ml1.x);
            const float f0 = m == m_run[u] ? 1.f : __builtin_amdgcn_exp2f(m_run[u] - m);
            const float f1 = ml1.x == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(ml1.x - m);
            const float inv = 1.0f / (Lr[u][0] * f0 + ml1.y * f1);
            if (t < a.M) {
#pragma unroll
                for (int dt = 0; dt < 8; ++dt) {
                    const f32x4 o1 = *(const f32x4*)(mo + (((wi * 2 + u) * 8 + dt) * 64 + lane) * 4);
                    const float4 o = make_float4((O[u][dt][0] * f0 + o1[0] * f1) * inv, (O[u][dt][1] * f0 + o1[1] * f1) * inv,
                                                 (O[u][dt][2] * f0 + o1[2] * f1) * inv, (O[u][dt][3] * f0 + o1[3] * f1) * inv);
                    *(float4*)(a.out + (size_t)t * H + head * HD + dt * 16 + 4 * q) = o;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------------

template <int HL>
static hipError_t pf_prep_hl(int K, int norm, const float* src, const float* norm_w, int M, int Mpad, uint16_t* xa,
                             float* xs, float* ts, hipStream_t s) {
    if (K == H && norm)
        hipLaunchKernelGGL((pf_prep_kernel<H, true, HL>), dim3(Mpad), dim3(256), 0, s, src, norm_w, M, xa, xs, ts);
    else if (K == H)
        hipLaunchKernelGGL((pf_prep_kernel<H, false, HL>), dim3(Mpad), dim3(256), 0, s, src, norm_w, M, xa, xs, ts);
    else if (K == FF && !norm)
        hipLaunchKernelGGL((pf_prep_kernel<FF, false, HL>), dim3(Mpad), dim3(256), 0, s, src, norm_w, M, xa, xs, ts);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_pf_prep(int K, int norm, const float* src, const float* norm_w, int M, int Mpad, uint16_t* xa,
                          float* xs, float* ts, int parts, hipStream_t s) {
    if (M < 1 || Mpad < M || Mpad % 128 || (parts != 1 && parts != 2)) return hipErrorInvalidValue;
    return parts == 2 ? pf_prep_hl<2>(K, norm, src, norm_w, M, Mpad, xa, xs, ts, s)
                      : pf_prep_hl<1>(K, norm, src, norm_w, M, Mpad, xa, xs, ts, s);
}

template <int FMT, int RB, int TB, int HL>
static hipError_t pf_gemm_shape_hl(int K, int epi, const PfGemmArgs& a, hipStream_t s) {
    const int T = (a.Mpad / (64 * TB)) * (a.N / (16 * RB));
    const dim3 grid(8 * ((T + 7) / 8));
    if (K == H && epi == EPI_STORE)
        hipLaunchKernelGGL((pf_gemm_kernel<FMT, H, EPI_STORE, RB, TB, HL>), grid, dim3(512), 0, s, a);
    else if (K == H && epi == EPI_RESID)
        hipLaunchKernelGGL((pf_gemm_kernel<FMT, H, EPI_RESID, RB, TB, HL>), grid, dim3(512), 0, s, a);
    else if (K == H && epi == EPI_SWIGLU)
        hipLaunchKernelGGL((pf_gemm_kernel<FMT, H, EPI_SWIGLU, RB, TB, HL>), grid, dim3(512), 0, s, a);
    else if (K == FF && epi == EPI_RESID)
        hipLaunchKernelGGL((pf_gemm_kernel<FMT, FF, EPI_RESID, RB, TB, HL>), grid, dim3(512), 0, s, a);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

template <int FMT, int RB, int TB>
static hipError_t pf_gemm_shape(int K, int epi, const PfGemmArgs& a, hipStream_t s) {
    return a.parts == 1 ? pf_gemm_shape_hl<FMT, RB, TB, 1>(K, epi, a, s) : pf_gemm_shape_hl<FMT, RB, TB, 2>(K, epi, a, s);
}

// Tiles that fill the 256 CUs evenly: at least one each, and a whole number each or at least four.
static bool even_fill(int tiles) { return tiles >= 256 && (tiles % 256 == 0 || tiles >= 1024); }

// The largest tile whose count fills the CUs evenly: 128 tokens x 256 rows, 128 x 128, else
// 64 x 128 (small prompts, whose 128-token tiles would leave CUs idle).  f16 weights keep 128-row
// tiles (their four B chunks per step would not fit the registers of the larger tile), and so do
// fp16 operands alone: their 128-row tile needs ~110 registers and 64 KiB of LDS, so two
// workgroups share a CU (measured 21.55 -> 20.97 ms per 4096-row prefill against 256-row tiles).
template <int FMT>
static hipError_t pf_gemm_fmt(int K, int epi, const PfGemmArgs& a, hipStream_t s) {
    const int tm128 = a.Mpad / 128;
    if (FMT != FMT_F16 && a.parts == 2 && a.N % 256 == 0 && even_fill(tm128 * (a.N / 256))) {
        if constexpr (FMT != FMT_F16) return pf_gemm_shape<FMT, 16, 2>(K, epi, a, s);
    }
    if (even_fill(tm128 * (a.N / 128))) return pf_gemm_shape<FMT, 8, 2>(K, epi, a, s);
    return pf_gemm_shape<FMT, 8, 1>(K, epi, a, s);
}

hipError_t launch_pf_gemm(int fmt, int K, int epi, const PfGemmArgs& a, hipStream_t s) {
    if (a.M < 1 || a.Mpad < a.M || a.Mpad % 128 || a.N % 128 || (a.parts != 1 && a.parts != 2))
        return hipErrorInvalidValue;
    switch (fmt) {
        case FMT_Q4: return pf_gemm_fmt<FMT_Q4>(K, epi, a, s);
        case FMT_Q8: return pf_gemm_fmt<FMT_Q8>(K, epi, a, s);
        case FMT_F16: return pf_gemm_fmt<FMT_F16>(K, epi, a, s);
    }
    return hipErrorInvalidValue;
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
        for (const void* k : {(const void*)pf_attn_kernel<1>, (const void*)pf_attn_kernel<2>}) {
            hipError_t e = hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)PA_LDS);
            if (e != hipSuccess) return e;
        }
        attr_set = true;
    }
    const int QB = (a.M + 63) / 64;
    if (a.ql)
        hipLaunchKernelGGL(pf_attn_kernel<2>, dim3(QB * NKV), dim3(512), PA_LDS, s, a);
    else
        hipLaunchKernelGGL(pf_attn_kernel<1>, dim3(QB * NKV), dim3(512), PA_LDS, s, a);
    return hipGetLastError();
}

}  // namespace icua
