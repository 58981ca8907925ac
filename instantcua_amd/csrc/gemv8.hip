// Multi-token (2..8 rows) q4 / q8 dequant-GEMV for speculative-verify passes, short prompts and
// grammar-pair passes, gfx950: the GEMV family of Shaders.swift:480-631 and the multi-row parts
// of k_attn_in, k_o_proj, k_mlp_in, k_mlp_out, k_lm_head (Shaders.swift:714-834, 1293-1495).
//
// Schedule.  One 512-thread workgroup per CU stages the pass's activation rows once and then
// streams 16-row weight blocks w, w + G, ... (G = min(row blocks, 256)).  The eight waves split K
// (256 K each per 2048-wide segment); each wave's activation operands and group factors stay in
// registers for every block.  Every wave keeps DEPTH blocks' weights in flight: a block's slot is
// refilled with the block DEPTH further on as soon as its matrix-core work is issued, and the
// activation rows and the first blocks are requested before the control block is read (the rows
// first: a load waits for every load issued before it).  The waves' partial sums of DEPTH blocks meet in LDS (two halves,
// one barrier per DEPTH blocks) for the reduction and the epilogue.  K = 6144 (down) with the
// engine's partial buffers runs one workgroup per (row block, 2048-wide segment); the last of a
// row block's three to arrive adds the segments in a fixed order and applies the epilogue.
//
// Arithmetic.  Each quantisation group of each activation row t (after the RMSNorm weights but
// before the row's 1/rms, a per-row factor applied to the finished sums) is scaled by 2^(14 - E),
// E the exponent of the group's largest magnitude, and split into fp16 hi + lo parts (about 22
// significant bits of the group maximum, like the int8 slices of the one-token path).  A operand
// row m = 2 t + part, so one v_mfma_f32_16x16x32_f16 covers the eight tokens' hi and lo rows
// against 16 weight rows and 32 K.  The weight codes become fp16 B operands in registers,
// exactly (q4: 1024 + q in the 0x6400 exponent minus 1024; q8: 1152 + b minus 1152), in the lane
// layout of the repacked tiles:
//   q8  a lane's 8 bytes of a 32-group are K 8q .. 8q + 7 (q = lane / 16): the B operand of that
//       group's k-step as they are;
//   q4  a lane's 8 bytes of a 64-group are the 16 nibbles of K 16q .. 16q + 15 (low nibbles of
//       bytes 0-3, high nibbles of bytes 0-3, then the same of bytes 4-7): k-step 2g takes the
//       first 8 and k-step 2g + 1 the next 8, and the A operands are staged in that K order.
// Per group: acc += (s 2^(E - 14)) C (+ b X for q4, X the group's activation sum), then
// y = (acc_hi + acc_lo) / rms.
#include "icua_device.h"
#include "icua_kernels.h"

namespace icua {
namespace g8 {

constexpr int THREADS = 512, WAVES = 8, SEG = 2048, DEPTH = 4;
static_assert(DEPTH * 16 * MAXM == THREADS, "the reduction maps one thread to (block, token, row)");
typedef _Float16 v8h __attribute__((ext_vector_type(8)));

template <int NPART>
struct Smem {
    uint4 A[SEG / 32 * 64];               // A operands of one segment: [k-step][lane] (64 KiB)
    float X[MAXM][SEG / 64];              // q4 group sums of the activations, per token
    float ts[MAXM][SEG / 32];             // 2^(E - 14) of each (token, group) of the segment
    float red[WAVES][MAXM];               // per-wave sums of squares
    float part[NPART][WAVES][MAXM][16];   // partial sums of blocks
    float bv[THREADS / 16];               // argmax merge: one (value, id) per row of 16 lanes
    int bi[THREADS / 16];
    int last;                             // split K: this workgroup finishes the row block
};

// Sum over the wave of eight per-lane values s[t]: token t's total lands in the eight lanes
// 8 (t >> 2) + 16 ((t >> 1) & 1) + 32 (t & 1) + 0..7.
__device__ __forceinline__ float wave_sum8(const float (&s)[MAXM], int lane) {
    float r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = swap32_add(s[2 * i], s[2 * i + 1]);  // token 2 i + bit 5
    const float u0 = swap16_add(r[0], r[1]);  // token 2 bit4 + bit5
    const float u1 = swap16_add(r[2], r[3]);  // token 4 + 2 bit4 + bit5
    const bool hi8 = lane & 8;
    float w = (hi8 ? u1 : u0) + dpp<DPP_MIRROR>(hi8 ? u0 : u1);
    w += dpp<DPP_HALF_MIRROR>(w);
    w += dpp<DPP_XOR2>(w);
    w += dpp<DPP_XOR1>(w);
    return w;
}
__device__ __forceinline__ int sum8_token(int lane) { return 4 * ((lane >> 3) & 1) + 2 * ((lane >> 4) & 1) + ((lane >> 5) & 1); }

// Four consecutive activations (columns 4 tid .. of the segment) of buffer rows 0 .. MAXM - 1.
// A host-given row count (m_fixed) bounds the rows read (the ones past it repeat its last row);
// otherwise the buffer holds MAXM rows (the engine's pass buffers).  Every row is staged and
// multiplied; only the pass's rows are written (an operand row m = 2 t + part feeds output row m
// of the matrix-core product alone, so a row never touches another row's sums).
template <int K>
__device__ __forceinline__ void load_rows(const GemvArgs& a, int seg, float (&v)[MAXM][4]) {
    const int k0 = 4 * threadIdx.x;
#pragma unroll
    for (int t = 0; t < MAXM; ++t) {
        const int r = a.m_fixed > 0 ? min(t, a.m_fixed - 1) : t;
        const float4 p = *(const float4*)(a.x + (size_t)r * K + seg * SEG + k0);
        v[t][0] = p.x;
        v[t][1] = p.y;
        v[t][2] = p.z;
        v[t][3] = p.w;
    }
}

// The fp16 hi / lo split of the loaded activations (times the RMSNorm weights wn) in the
// operand layout, the (token, group) factors, the q4 group sums and, for PRO_NORM, the per-wave
// sums of squares of each row.  Ends with a barrier.
template <int FMT, int PRO, int NPART>
__device__ __forceinline__ void stage(Smem<NPART>& S, const float (&v)[MAXM][4], float4 wn) {
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int k0 = 4 * tid;  // column within the segment
    if constexpr (PRO == PRO_NORM) {
        float ss[MAXM];
#pragma unroll
        for (int t = 0; t < MAXM; ++t) {
            float s = v[t][0] * v[t][0];
            s = fmaf(v[t][1], v[t][1], s);
            s = fmaf(v[t][2], v[t][2], s);
            ss[t] = fmaf(v[t][3], v[t][3], s);
        }
        const float tot = wave_sum8(ss, lane);
        if (lane % 8 == 0) S.red[wave][sum8_token(lane)] = tot;
    }
    const float w4[4] = {wn.x, wn.y, wn.z, wn.w};
    constexpr int G = FMT == FMT_Q4 ? 64 : 32;  // the group's columns are G / 4 consecutive lanes
    int ks, q;
    if constexpr (FMT == FMT_Q4) {
        const int kk = k0 % 64;
        ks = 2 * (k0 / 64) + (kk % 16) / 8;
        q = kk / 16;
    } else {
        ks = k0 / 32;
        q = (k0 % 32) / 8;
    }
    const int j0 = k0 % 8;  // 0 or 4: halves j0 .. j0 + 3 of the lane's 8
    uint8_t* base = (uint8_t*)(S.A + ks * 64) + 16 * 16 * q + j0 * 2;
#pragma unroll
    for (int t = 0; t < MAXM; ++t) {
        float x[4], mx = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[i] = PRO == PRO_NORM ? v[t][i] * w4[i] : v[t][i];
            mx = fmaxf(mx, fabsf(x[i]));
        }
        int bits = (int)as_u32(mx);  // order of non-negative floats = order of their bits
        bits = max(bits, dpp_i<DPP_XOR1>(bits));
        bits = max(bits, dpp_i<DPP_XOR2>(bits));
        bits = max(bits, dpp_i<DPP_HALF_MIRROR>(bits));
        if constexpr (G == 64) bits = max(bits, dpp_i<DPP_MIRROR>(bits));
        // E clamped so that 2^(14 - E) and 2^(E - 14) are normal (an all-zero group gives zeros with any E).
        const int E = min(max(((bits >> 23) & 0xFF) - 127, -100), 126);
        const float sh = ldexpf(1.0f, 14 - E);
        uint32_t hw[2], lw[2];
        float gs = 0.f;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float x0 = x[2 * i] * sh, x1 = x[2 * i + 1] * sh;
            const f16 h0 = (f16)x0, h1 = (f16)x1;
            const f16 l0 = (f16)(x0 - (float)h0), l1 = (f16)(x1 - (float)h1);
            if constexpr (FMT == FMT_Q4) gs += ((float)h0 + (float)l0) + ((float)h1 + (float)l1);
            hw[i] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
            lw[i] = (uint32_t)__builtin_bit_cast(uint16_t, l0) | ((uint32_t)__builtin_bit_cast(uint16_t, l1) << 16);
        }
        *(uint2*)(base + (2 * t) * 16) = make_uint2(hw[0], hw[1]);
        *(uint2*)(base + (2 * t + 1) * 16) = make_uint2(lw[0], lw[1]);
        const float inv = ldexpf(1.0f, E - 14);
        if constexpr (FMT == FMT_Q4) {
            gs += dpp<DPP_XOR1>(gs);
            gs += dpp<DPP_XOR2>(gs);
            gs += dpp<DPP_HALF_MIRROR>(gs);
            gs += dpp<DPP_MIRROR>(gs);
            if (k0 % 64 == 0) S.X[t][k0 / 64] = gs * inv;
        }
        if (k0 % G == 0) S.ts[t][k0 / G] = inv;
    }
    __syncthreads();
}

// 8 fp16 B halves from 4 code bytes d: q4 the low nibbles then the high nibbles; q8 two words.
__device__ __forceinline__ v8h b_q4(uint32_t d) {
    const uint32_t s0 = __builtin_amdgcn_perm(d, d, 0x0C010C00u), s1 = __builtin_amdgcn_perm(d, d, 0x0C030C02u);
    const f16x2 k = {(f16)1024.f, (f16)1024.f};
    const uint32_t o0 = h2_bits(as_h2((s0 & 0x000F000Fu) | 0x64006400u) - k);
    const uint32_t o1 = h2_bits(as_h2((s1 & 0x000F000Fu) | 0x64006400u) - k);
    const uint32_t o2 = h2_bits(as_h2(((s0 >> 4) & 0x000F000Fu) | 0x64006400u) - k);
    const uint32_t o3 = h2_bits(as_h2(((s1 >> 4) & 0x000F000Fu) | 0x64006400u) - k);
    return __builtin_bit_cast(v8h, make_uint4(o0, o1, o2, o3));
}
__device__ __forceinline__ v8h b_q8(uint32_t d0, uint32_t d1) {
    const f16x2 k = {(f16)1152.f, (f16)1152.f};
    auto two = [&](uint32_t d, uint32_t sel) {
        return h2_bits(as_h2((__builtin_amdgcn_perm(d, d, sel) ^ 0x00800080u) | 0x64006400u) - k);
    };
    return __builtin_bit_cast(v8h, make_uint4(two(d0, 0x0C010C00u), two(d0, 0x0C030C02u), two(d1, 0x0C010C00u),
                                              two(d1, 0x0C030C02u)));
}

// Buffer resources of the weight codes and scales.  A request of a block that does not exist
// is given an offset past the end: it reads nothing and returns zeros, so every path issues the
// same loads and the compiler's waits on earlier loads stay exact.
struct Src {
    __amdgpu_buffer_rsrc_t w, s;
};
constexpr uint32_t OOB = 0x80000000u;
template <int FMT, int K>
__device__ __forceinline__ Src make_src(const GemvArgs& a) {
    const int nw = (int)((size_t)a.N * K / (FMT == FMT_Q4 ? 2 : 1));
    const int ns = (int)((size_t)a.N * (FMT == FMT_Q4 ? K / 64 * 4 : K / 32 * 2));
    return {__builtin_amdgcn_make_buffer_rsrc((void*)a.w, (short)0, nw, 0x00020000),
            __builtin_amdgcn_make_buffer_rsrc((void*)a.sb, (short)0, ns, 0x00020000)};
}

// One wave's share of a 16-row block in one segment: the code words and the lane's row scales.
template <int FMT>
struct WTile {
    static constexpr int NW = FMT == FMT_Q4 ? 2 : 4;  // 1 KiB chunks per wave per segment
    uint4 w[NW];
    uint4 s;  // q4: (scale, bias) of groups 4 wave .. + 3; q8: scales of groups 8 wave .. + 7
    template <int K>
    __device__ __forceinline__ void load(const Src& src, int rb, bool ok, int seg, int wave, int lane) {
        constexpr int CHK = FMT == FMT_Q4 ? 128 : 64, NCH = K / CHK;
        const uint32_t cw = ok ? (uint32_t)((rb * NCH + seg * (SEG / CHK) + wave * NW) * 1024 + lane * 16) : OOB;
        const int row = rb * 16 + (lane & 15);
        const uint32_t cs = !ok ? OOB
                            : FMT == FMT_Q4 ? (uint32_t)((row * (K / 64) + seg * (SEG / 64) + 4 * wave) * 4)
                                            : (uint32_t)((row * (K / 32) + seg * (SEG / 32) + 8 * wave) * 2);
#pragma unroll
        for (int i = 0; i < NW; ++i)
            w[i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src.w, cw + i * 1024, 0, 0));
        s = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(src.s, cs, 0, 0));
    }
};

// A wave's activation operands and (token, group) factors of one segment, for every block.
template <int FMT>
struct Ops {
    static constexpr int NG = FMT == FMT_Q4 ? 4 : 8;  // groups of the wave's 256 K
    v8h A[8];
    float t0[NG], t1[NG];  // 2^(E - 14) of tokens tq, tq + 1 (tq = 2 (lane / 16))
    float x0[NG], x1[NG];  // q4: their group sums
    template <int NPART>
    __device__ __forceinline__ void load(const Smem<NPART>& S, int wave, int lane) {
        const int tq = 2 * (lane >> 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) A[j] = __builtin_bit_cast(v8h, S.A[(8 * wave + j) * 64 + lane]);
#pragma unroll
        for (int g = 0; g < NG; ++g) {
            t0[g] = S.ts[tq][NG * wave + g];
            t1[g] = S.ts[tq + 1][NG * wave + g];
            if constexpr (FMT == FMT_Q4) {
                x0[g] = S.X[tq][NG * wave + g];
                x1[g] = S.X[tq + 1][NG * wave + g];
            }
        }
    }
};

// A wave's MAC of one block: y[p] for the lane's tokens 2 (lane / 16) + p, weight row lane % 16.
template <int FMT>
__device__ __forceinline__ void mac(const Ops<FMT>& o, const WTile<FMT>& wt, float (&y)[2]) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const uint32_t sw[4] = {wt.s.x, wt.s.y, wt.s.z, wt.s.w};
    if constexpr (FMT == FMT_Q4) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const uint4 c = wt.w[g / 2];
            const uint32_t d0 = (g & 1) ? c.z : c.x, d1 = (g & 1) ? c.w : c.y;
            f32x4 C = {0.f, 0.f, 0.f, 0.f};
            C = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.A[2 * g], b_q4(d0), C, 0, 0, 0);
            C = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.A[2 * g + 1], b_q4(d1), C, 0, 0, 0);
            const f16x2 sb = as_h2(sw[g]);
            const float s = (float)sb.x, b = (float)sb.y;
            // Rows 4 (lane / 16) + i: token tq + i / 2, (hi, lo); the bias once per token.
            const float f0 = s * o.t0[g], f1 = s * o.t1[g];
            acc[0] = fmaf(f0, C[0], fmaf(b, o.x0[g], acc[0]));
            acc[1] = fmaf(f0, C[1], acc[1]);
            acc[2] = fmaf(f1, C[2], fmaf(b, o.x1[g], acc[2]));
            acc[3] = fmaf(f1, C[3], acc[3]);
        }
    } else {
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const uint4 c = wt.w[g / 2];
            const v8h B = (g & 1) ? b_q8(c.z, c.w) : b_q8(c.x, c.y);
            const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
            const f32x4 C = __builtin_amdgcn_mfma_f32_16x16x32_f16(o.A[g], B, zero, 0, 0, 0);
            const f16x2 s2 = as_h2(sw[g / 2]);
            const float s = (g & 1) ? (float)s2.y : (float)s2.x;
            const float f0 = s * o.t0[g], f1 = s * o.t1[g];
            acc[0] = fmaf(f0, C[0], acc[0]);
            acc[1] = fmaf(f0, C[1], acc[1]);
            acc[2] = fmaf(f1, C[2], acc[2]);
            acc[3] = fmaf(f1, C[3], acc[3]);
        }
    }
    y[0] = acc[0] + acc[1];
    y[1] = acc[2] + acc[3];
}

// One step of an argmax over a row of 16 lanes.
template <int CTRL>
__device__ __forceinline__ void argmax_step(float& v, int& i) {
    const float ov = dpp<CTRL>(v);
    const int oi = dpp_i<CTRL>(i);
    argmax_merge(v, i, ov, oi);
}

// Rows of the pass: buffer rows row0 .. row0 + M - 1 (as the other GEMVs: the state's n rows, or
// only the last one for an argmax pass that writes no logits).
struct Pass {
    int done, n, logits_rows;
};
// The control block's fields the GEMV needs, requested where this is called (the staging's
// barriers keep the loads there, ahead of the staging's work).
__device__ __forceinline__ Pass read_pass(const GemvArgs& a) {
    const State* st = a.st;
    return {st->done, st->n, st->logits_rows};
}
template <int EPI>
__device__ __forceinline__ void rows_of(const GemvArgs& a, const Pass& p, int& M, int& row0) {
    if (a.m_fixed > 0) {
        M = a.m_fixed;
        row0 = 0;
    } else {
        M = p.n;
        row0 = 0;
        if constexpr (EPI == EPI_ARGMAX) {
            if (p.logits_rows != M) {
                row0 = M - 1;
                M = 1;
            }
        }
    }
    if (M > MAXM) M = MAXM;
    if (row0 > MAXM - 1) row0 = MAXM - 1;
}

// Residual add (+ the DeepStack row of a visual row, Shaders.swift:696-707) or plain store of
// output row `row` of buffer row t (pass rows start at buffer row 0 for these epilogues).
template <int EPI>
__device__ __forceinline__ void store_row(const GemvArgs& a, int t, int row, float y) {
    if constexpr (EPI == EPI_STORE) {
        a.y[(size_t)t * a.N + row] = y;
    } else {
        const State* st = a.st;
        float* xo = a.y + (size_t)t * a.N + row;
        float v = *xo + y;
        if (a.ds) {
            const int vrow = a.ds_row0 + t - st->vis_offset;
            if (st->vis_offset >= 0 && vrow >= 0 && vrow < st->n_vis) v = v + a.ds[(size_t)vrow * H + row];
        }
        *xo = v;
    }
}

// Row-block streaming form (every op; K = 6144 walks its three segments per batch of blocks).
template <int FMT, int K, int PRO, int EPI>
__global__ __launch_bounds__(THREADS, 1) void gemv8_kernel(GemvArgs a) {
    constexpr int NSEG = K / SEG;
    // Blocks per batch: K = 6144 holds two per wave (with three segments' operands staged in turn
    // the registers would not hold four).
    constexpr int DP = NSEG == 1 ? DEPTH : 2;
    constexpr int NPART = NSEG == 1 ? 2 * DEPTH : DP;
    __shared__ Smem<NPART> S;
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int G = gridDim.x, wg = blockIdx.x;
    const int nrb = EPI == EPI_SWIGLU ? FF / 8 : a.N / 16;
    const int nb = (nrb - wg + G - 1) / G;  // blocks of this workgroup (the host keeps wg < nrb)
    const Src src = make_src<FMT, K>(a);
    WTile<FMT> wl[DEPTH];
    float v[MAXM][4];
    // Reduction / epilogue role of this thread: block k0 + re of a batch, buffer row rt, row rr.
    const int re = tid / 128, rt = (tid / 16) % MAXM, rr = tid % 16;
    const int tq = 2 * (lane >> 4), r16 = lane & 15;
    float best_v = -__builtin_inff();
    int best_i = 0x7fffffff;
    float sc = 1.f;
    Ops<FMT> ops;
    Pass pass;
    if constexpr (NSEG > 1) pass = read_pass(a);
    if constexpr (NSEG == 1) {
        // The rows, then the first DEPTH blocks, then the staging: none of it waits for the
        // control block (read after the staging's barriers, so the loads stay ahead of it).
        load_rows<K>(a, 0, v);
        const float4 wn = PRO == PRO_NORM ? *(const float4*)(a.norm_w + 4 * tid) : make_float4(1.f, 1.f, 1.f, 1.f);
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) wl[k].template load<K>(src, wg + k * G, k < nb, 0, wave, lane);
        pass = read_pass(a);
        stage<FMT, PRO>(S, v, wn);
        ops.load(S, wave, lane);
        if constexpr (PRO == PRO_NORM) {
            float ss = 0.f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) ss += S.red[w][rt];
            sc = __builtin_amdgcn_rsqf(ss / (float)K + EPS);
        }
    }
    if (pass.done) return;
    int M, row0;
    rows_of<EPI>(a, pass, M, row0);
    const bool live = rt >= row0 && rt < row0 + M;  // this thread's row belongs to the pass
    for (int k0 = 0; k0 < nb; k0 += DP) {
        const int half = NSEG == 1 ? ((k0 / DP) & 1) * DP : 0;
        if constexpr (NSEG == 1) {
#pragma unroll
            for (int k = 0; k < DP; ++k) {
                if (k0 + k < nb) {
                    float y[2];
                    mac<FMT>(ops, wl[k], y);
                    S.part[half + k][wave][tq][r16] = y[0];
                    S.part[half + k][wave][tq + 1][r16] = y[1];
                }
                wl[k].template load<K>(src, wg + (k0 + k + DP) * G, k0 + k + DP < nb, 0, wave, lane);
            }
        } else {
            float yk[DP][2];
#pragma unroll
            for (int k = 0; k < DP; ++k) yk[k][0] = yk[k][1] = 0.f;
#pragma unroll 1
            for (int seg = 0; seg < NSEG; ++seg) {
                // (The weights are requested after the staging here: with the rows in flight
                // too, the registers would not hold them.)
                load_rows<K>(a, seg, v);
                __syncthreads();  // every wave has read the previous segment's operands
                stage<FMT, PRO_F32>(S, v, make_float4(1.f, 1.f, 1.f, 1.f));
#pragma unroll
                for (int k = 0; k < DP; ++k) wl[k].template load<K>(src, wg + (k0 + k) * G, k0 + k < nb, seg, wave, lane);
                ops.load(S, wave, lane);
#pragma unroll
                for (int k = 0; k < DP; ++k) {
                    if (k0 + k < nb) {
                        float y[2];
                        mac<FMT>(ops, wl[k], y);
                        yk[k][0] += y[0];
                        yk[k][1] += y[1];
                    }
                }
            }
#pragma unroll
            for (int k = 0; k < DP; ++k) {
                S.part[k][wave][tq][r16] = yk[k][0];
                S.part[k][wave][tq + 1][r16] = yk[k][1];
            }
        }
        __syncthreads();
        if (re < DP && k0 + re < nb && live) {
            const int rb = wg + (k0 + re) * G;
            const float(*pp)[MAXM][16] = S.part[half + re];
            float y = 0.f;
#pragma unroll
            for (int w = 0; w < WAVES; ++w) y += pp[w][rt][rr];
            y *= sc;
            const int row = rb * 16 + rr;
            if constexpr (EPI == EPI_STORE || EPI == EPI_RESID) {
                store_row<EPI>(a, rt, row, y);
            } else if constexpr (EPI == EPI_SWIGLU) {
                // Block rb: gate units 8 rb + 0..7 in rows 0-7, their up rows in 8-15.
                if (rr < 8) {
                    float up = 0.f;
#pragma unroll
                    for (int w = 0; w < WAVES; ++w) up += pp[w][rt][rr + 8];
                    up *= sc;
                    a.h[(size_t)rt * FF + rb * 8 + rr] = (y / (1.f + expf(-y))) * up;
                }
            } else {  // EPI_ARGMAX: tiled rows are the vocabulary ids
                if (a.logits && pass.logits_rows > 0) a.logits[(size_t)(rt - row0) * VOCAB + row] = y;
                argmax_merge(best_v, best_i, y, row);
            }
        }
        if constexpr (NSEG > 1) __syncthreads();  // the partials are read before the next batch writes them
    }
    if constexpr (EPI == EPI_ARGMAX) {
        // Each row of 16 lanes holds one token's candidates (token rt); rows rt, rt + 8, .. meet in LDS.
        argmax_step<DPP_MIRROR>(best_v, best_i);
        argmax_step<DPP_HALF_MIRROR>(best_v, best_i);
        argmax_step<DPP_XOR2>(best_v, best_i);
        argmax_step<DPP_XOR1>(best_v, best_i);
        if (rr == 0) {
            S.bv[tid / 16] = best_v;
            S.bi[tid / 16] = best_i;
        }
        __syncthreads();
        if (tid < M) {
            const int r = row0 + tid;
            float bv = S.bv[r];
            int bi = S.bi[r];
            for (int j = r + MAXM; j < THREADS / 16; j += MAXM) argmax_merge(bv, bi, S.bv[j], S.bi[j]);
            a.pval[(size_t)r * LMH_WAVES + wg] = bv;
            a.pidx[(size_t)r * LMH_WAVES + wg] = bi;
        }
        // The merge reads LMH_WAVES partials per row: the ones past this grid hold nothing.
        for (int j = wg + G; j < LMH_WAVES; j += G)
            if (tid < M) {
                a.pval[(size_t)(row0 + tid) * LMH_WAVES + j] = -__builtin_inff();
                a.pidx[(size_t)(row0 + tid) * LMH_WAVES + j] = 0x7fffffff;
            }
    }
}

// K = 6144 split form: workgroup (row block, segment) = (blockIdx % nrb, blockIdx / nrb).  Each
// stores its block's sums of its segment in a.kpart; the third to arrive at the row block's
// counter adds the three in segment order (the same result whichever arrives last), applies the
// epilogue and re-arms the counter.
template <int FMT, int EPI>
__global__ __launch_bounds__(THREADS, 1) void gemv8_split_kernel(GemvArgs a) {
    constexpr int K = FF, NSEG = K / SEG;
    __shared__ Smem<1> S;
    const int tid = threadIdx.x, lane = tid % 64, wave = tid / 64;
    const int nrb = a.N / 16, rb = blockIdx.x % nrb, seg = blockIdx.x / nrb;
    float v[MAXM][4];
    load_rows<K>(a, seg, v);
    WTile<FMT> wt;
    wt.template load<K>(make_src<FMT, K>(a), rb, true, seg, wave, lane);
    const Pass pass = read_pass(a);
    stage<FMT, PRO_F32>(S, v, make_float4(1.f, 1.f, 1.f, 1.f));
    Ops<FMT> ops;
    ops.load(S, wave, lane);
    float y2[2];
    mac<FMT>(ops, wt, y2);
    const int tq = 2 * (lane >> 4), r16 = lane & 15;
    S.part[0][wave][tq][r16] = y2[0];
    S.part[0][wave][tq + 1][r16] = y2[1];
    if (pass.done) return;
    int M, row0;
    rows_of<EPI>(a, pass, M, row0);  // row0 = 0 for these epilogues
    __syncthreads();
    const int rt = tid / 16, rr = tid % 16, row = rb * 16 + rr;
    const bool live = tid < MAXM * 16 && rt < M;
    if (live) {
        float y = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) y += S.part[0][w][rt][rr];
        __hip_atomic_store(a.kpart + ((size_t)seg * MAXM + rt) * a.N + row, y, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // the sums are stored before the arrival is counted
    __syncthreads();
    if (tid == 0)
        S.last = __hip_atomic_fetch_add(a.kcnt + rb, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == NSEG - 1;
    __syncthreads();
    if (!S.last) return;
    if (live) {
        float y = 0.f;
#pragma unroll
        for (int sg = 0; sg < NSEG; ++sg)
            y += __hip_atomic_load(a.kpart + ((size_t)sg * MAXM + rt) * a.N + row, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        store_row<EPI>(a, rt, row, y);
    }
    if (tid == 0) __hip_atomic_store(a.kcnt + rb, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int FMT, int K, int PRO, int EPI>
static hipError_t launch(const GemvArgs& a, hipStream_t s) {
    const int nrb = EPI == EPI_SWIGLU ? FF / 8 : a.N / 16;
    if constexpr (K == FF && PRO == PRO_F32 && (EPI == EPI_RESID || EPI == EPI_STORE)) {
        // The engine's partial buffers hold [3][MAXM][H] sums and H / 16 counters.
        if (a.kpart && a.kcnt && a.N == H) {
            hipLaunchKernelGGL((gemv8_split_kernel<FMT, EPI>), dim3(nrb * (K / SEG)), dim3(THREADS), 0, s, a);
            return hipGetLastError();
        }
    }
    const int G = nrb < 256 ? nrb : 256;
    hipLaunchKernelGGL((gemv8_kernel<FMT, K, PRO, EPI>), dim3(G), dim3(THREADS), 0, s, a);
    return hipGetLastError();
}

template <int FMT>
static hipError_t op_fmt(GemvOp op, const GemvArgs& a, hipStream_t s) {
    switch (op) {
        case GEMV_QKV: return launch<FMT, H, PRO_NORM, EPI_STORE>(a, s);
        case GEMV_O: return launch<FMT, H, PRO_F32, EPI_RESID>(a, s);
        case GEMV_GU: return launch<FMT, H, PRO_NORM, EPI_SWIGLU>(a, s);
        case GEMV_DOWN: return launch<FMT, FF, PRO_F32, EPI_RESID>(a, s);
        case GEMV_LMHEAD: return launch<FMT, H, PRO_NORM, EPI_ARGMAX>(a, s);
        case GEMV_PLAIN: return launch<FMT, H, PRO_F32, EPI_STORE>(a, s);
        case GEMV_PLAIN_K6144: return launch<FMT, FF, PRO_F32, EPI_STORE>(a, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace g8

bool gemv8_supports(int fmt, GemvOp op, int N) {
    if ((fmt != FMT_Q4 && fmt != FMT_Q8) || N <= 0 || N % 16) return false;
    // The weight buffers are addressed with 32-bit buffer offsets.
    const size_t K = (op == GEMV_DOWN || op == GEMV_PLAIN_K6144) ? FF : H;
    return (size_t)N * K / (fmt == FMT_Q4 ? 2 : 1) < ((size_t)1 << 31);
}

hipError_t launch_gemv8(int fmt, GemvOp op, const GemvArgs& a, hipStream_t s) {
    if (!gemv8_supports(fmt, op, a.N)) return hipErrorInvalidValue;
    return fmt == FMT_Q4 ? g8::op_fmt<FMT_Q4>(op, a, s) : g8::op_fmt<FMT_Q8>(op, a, s);
}

}  // namespace icua
