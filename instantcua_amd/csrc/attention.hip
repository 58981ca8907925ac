// GQA 16:8 decode / verify attention over the fp16 KV cache, gfx950.
//
// Replaces k_attention (Shaders.swift:1220-1289) and the q_norm/k_norm + M-RoPE + KV-write
// epilogue of k_attn_in (Shaders.swift:758-787).  Math follows tools/reference/qwen3vl_ref.py
// (254-270, 305-320): per-head RMSNorm(128) on q and k, rotate_half RoPE with the engine's
// M-RoPE table row of the token's cache slot, scores q.k / sqrt(128), softmax, P.V; fp32
// throughout, K/V stored as fp16.
//
// Layout.  The cache of a layer is [NKV][maxctx][HD] fp16 (Engine.swift:110-112, 477): one KV
// group is a contiguous run of 256-byte rows.  Grid (splits, NKV): split s < S-1 of group g
// streams prior slots [64 s, 64 s + 64) once and serves BOTH query heads 2g and 2g+1 (the
// reference streams each group twice, once per head).  Each 16-lane quarter-wave owns four
// slots and issues all of their K and V row loads (16 B per lane) before any arithmetic.
// Split S-1 owns the pass's new rows (slots pos .. pos+M-1): it normalises and rotates their
// K, rounds K/V to fp16, writes them to the cache and uses them from LDS with a causal mask.
//
// Each split writes an unnormalised partial (o[128], m, l) per (token, head); a merge kernel
// combines them (flash-decoding) with independent loads and writes the fp32 attention rows
// that feed the O projection.
#include "icua_device.h"
#include "icua_kernels.h"

namespace icua {

constexpr int ATT_THREADS = 256;
constexpr int ATT_CH = 64;  // prior slots per split: 16 quarter-waves x 4 slots
constexpr int PART_STRIDE = HD + 2;

__device__ __forceinline__ void unpack8(const uint4 raw, float* out) {
    const uint32_t d4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const f16x2 h = as_h2(d4[i]);
        out[2 * i] = (float)h.x;
        out[2 * i + 1] = (float)h.y;
    }
}

template <int MT>
__global__ __launch_bounds__(ATT_THREADS) void attention_kernel(AttnArgs a) {
    const State* st = a.st;
    if (st->done) return;
    const int M = a.m_fixed > 0 ? a.m_fixed : (st->n < MT ? st->n : MT);
    const int pos = st->pos;
    const int maxctx = st->maxctx;
    const int S = (pos + ATT_CH - 1) / ATT_CH + 1;  // prior splits + the tail split
    const int s = blockIdx.x, g = blockIdx.y;
    if (pos < 0 || pos + M > maxctx || S > (int)gridDim.x) return;  // host-checked; stay inside the cache
    if (s >= S) return;
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int quad = tid / 16, ql = tid % 16;
    const bool tail = (s == S - 1);
    const int j0 = s * ATT_CH;
    const int P = tail ? M : min(ATT_CH, pos - j0);

    constexpr int ROWS = 2 * MT;  // (token, head) rows
    __shared__ float qs[MT][2][HD];   // normalised, rotated, pre-scaled queries
    __shared__ float ktail[MT][HD];   // new K/V rows (fp16-rounded values)
    __shared__ float vtail[MT][HD];
    __shared__ float sc[ROWS][ATT_CH];
    __shared__ float mrow[ROWS], lrow[ROWS];
    __shared__ float ored[ATT_THREADS / WAVE][4][HD];

    const uint16_t* kbase = a.kc + (size_t)g * maxctx * HD;
    const uint16_t* vbase = a.vc + (size_t)g * maxctx * HD;

    // Prior K/V rows of this quarter-wave: loads first.
    uint4 kraw[4], vraw[4];
    if (!tail) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = quad + 16 * i;
            const int slot = j0 + (p < P ? p : 0);
            kraw[i] = *(const uint4*)(kbase + (size_t)slot * HD + 8 * ql);
            vraw[i] = *(const uint4*)(vbase + (size_t)slot * HD + 8 * ql);
        }
    }

    const float qscale = 1.0f / sqrtf((float)HD);
    for (int row = wave; row < 2 * M; row += ATT_THREADS / WAVE) {
        const int t = row / 2, hh = row % 2;
        const float* src = a.qkv + (size_t)t * QKV + (2 * g + hh) * HD;
        float x0 = src[lane], x1 = src[lane + 64];
        norm_rope_pair(x0, x1, a.q_norm, a.rope + (size_t)(pos + t) * 128, lane);
        qs[t][hh][lane] = x0 * qscale;
        qs[t][hh][lane + 64] = x1 * qscale;
    }
    if (tail) {
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

    float kv[4][8], vv[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int p = quad + 16 * i;
        if (!tail) {
            unpack8(kraw[i], kv[i]);
            unpack8(vraw[i], vv[i]);
        } else {
            const int pt = p < M ? p : 0;
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                kv[i][d] = ktail[pt][8 * ql + d];
                vv[i][d] = vtail[pt][8 * ql + d];
            }
        }
    }

    // 1. Scores of every (token, head) row for this quarter-wave's four slots.
    for (int t = 0; t < M; ++t) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            float q[8];
#pragma unroll
            for (int d = 0; d < 8; ++d) q[d] = qs[t][hh][8 * ql + d];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = quad + 16 * i;
                float acc = 0.f;
#pragma unroll
                for (int d = 0; d < 8; ++d) acc = fmaf(q[d], kv[i][d], acc);
                acc = sum16(acc);
                const bool valid = p < P && (!tail || p <= t);
                if (ql == 0) sc[2 * t + hh][p] = valid ? acc : -__builtin_inff();
            }
        }
    }
    __syncthreads();

    // 2. Split softmax statistics, one wave per row (P <= 64 slots = one per lane).
    for (int row = wave; row < 2 * M; row += ATT_THREADS / WAVE) {
        const float v = sc[row][lane];
        const float m = wave_max(v);
        const float e = (m == -__builtin_inff()) ? 0.f : expf(v - m);
        sc[row][lane] = e;
        const float l = wave_sum(e);
        if (lane == 0) {
            mrow[row] = m;
            lrow[row] = l;
        }
    }
    __syncthreads();

    // 3. P.V in groups of four rows; lane ql accumulates dims [8 ql, 8 ql + 8).
    float* part = a.part + (size_t)(g * gridDim.x + s) * MAXM * 2 * PART_STRIDE;
    for (int r0 = 0; r0 < 2 * M; r0 += 4) {
        float o[4][8];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int d = 0; d < 8; ++d) o[r][d] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int p = quad + 16 * i;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float pr = (r0 + r < 2 * M) ? sc[r0 + r][p] : 0.f;
#pragma unroll
                for (int d = 0; d < 8; ++d) o[r][d] = fmaf(pr, vv[i][d], o[r][d]);
            }
        }
        // Sum the four quarter-waves of the wave (lanes l, l^16, l^32, l^48 hold the same dims).
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int d = 0; d < 8; ++d) {
                const float t1 = swap16_add(o[r][d], o[r][d]);
                o[r][d] = swap32_add(t1, t1);
            }
        if (quad % 4 == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int d = 0; d < 8; ++d) ored[wave][r][8 * ql + d] = o[r][d];
        }
        __syncthreads();
        for (int idx = tid; idx < 4 * HD; idx += ATT_THREADS) {
            const int r = idx / HD, d = idx % HD;
            const int row = r0 + r;
            if (row >= 2 * M) continue;
            float acc = 0.f;
#pragma unroll
            for (int w = 0; w < ATT_THREADS / WAVE; ++w) acc += ored[w][r][d];
            float* dst = part + (size_t)row * PART_STRIDE;
            dst[d] = acc;
            if (d == 0) {
                dst[HD] = mrow[row];
                dst[HD + 1] = lrow[row];
            }
        }
        __syncthreads();
    }

}

// Multi-row passes (verify, short prompts) on the matrix cores.  Grid (NKV, NS), NS <= 32: the
// prior slots' 64-slot blocks are dealt evenly to splits 0 .. NS - 2 (four or five blocks each
// at 8192 slots, double-buffered through LDS) and split NS - 1 takes the pass's new rows; the
// 8 x 32 grid is one workgroup per CU (80 KiB of LDS and 236 registers would let two share one),
// and the tail splits, dispatched last, are the short ones.  (16 and 64 splits per group
// measured 3-4 % slower per verify pass, counting the merge.)  The 16 (token, head) rows of a KV group, column c = 2 t + head, are the B operand of
// S^T = K . Q^T (v_mfma_f32_16x16x32_f16, q split into fp16 hi + lo parts); wave w scores keys
// 16 w .. 16 w + 15 of each block, and its accumulator (lane l: keys 4 (l / 16) + i, column
// l % 16) is directly the B operand of O^T = V^T . P^T (v_mfma_f32_16x16x16_f16, P split hi + lo)
// with V transposed in LDS.  Each wave keeps an online softmax over its keys; the four waves'
// (m, l, o) are combined into the partial that the merge kernel reads.  Masked keys (past the
// split's cache rows, or later tokens of the pass in the tail split) hold finite rows, so p = 0
// contributes exactly nothing.
constexpr int VA_SPLITS = 32;                             // splits of a group (at most)
constexpr int VA_KROW = 136, VA_VROW = 72, VA_QROW = 136;  // padded LDS rows (halves)
// Column (halves) of key `key` in V^T row `row`: 4-key chunks XOR-swizzled by (row / 8) % 8, so
// the staging writes (lane l of a half-wave: rows 4 l + j, one chunk) and the P.V reads (16
// rows, one chunk) each cover all 32 banks.
__device__ __forceinline__ int va_vcol(int row, int key) { return 4 * ((key >> 2) ^ ((row >> 3) & 7)) + (key & 3); }

__global__ __launch_bounds__(ATT_THREADS) void attention_mfma_kernel(AttnArgs a) {
    typedef _Float16 v4h __attribute__((ext_vector_type(4)));
    typedef _Float16 v8h __attribute__((ext_vector_type(8)));
    const State* st = a.st;
    if (st->done) return;
    const int M = a.m_fixed > 0 ? a.m_fixed : (st->n < MAXM ? st->n : MAXM);
    const int pos = st->pos;
    const int maxctx = st->maxctx;
    const int NS = gridDim.y, s = blockIdx.y, g = blockIdx.x;
    if (pos < 0 || pos + M > maxctx) return;  // host-checked; stay inside the cache
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE, q4 = lane >> 4, r16 = lane & 15;
    const bool tail = (s == NS - 1);
    // Prior blocks [b0, b1) of this split (none for the tail; possibly none for small pos).
    const int nbt = (pos + ATT_CH - 1) / ATT_CH;
    const int b0 = tail ? 0 : s * nbt / (NS - 1), b1 = tail ? 0 : (s + 1) * nbt / (NS - 1);
    const int j0 = b0 * ATT_CH;
    const int P = tail ? M : min(b1 * ATT_CH, pos) - j0;  // keys of this split
    const int nblk = (P + ATT_CH - 1) / ATT_CH;

    // Two K tiles (keys x dims) and V^T tiles (dims x keys); after the products, the waves' o.
    constexpr int KS_BYTES = ATT_CH * VA_KROW * 2, VT_BYTES = HD * VA_VROW * 2, BUF = KS_BYTES + VT_BYTES;
    constexpr int OW_BYTES = (ATT_THREADS / WAVE) * 16 * HD * 4;
    static_assert(2 * BUF >= OW_BYTES, "the waves' o fit over the K / V tiles");
    __shared__ __align__(16) uint8_t kv_lds[2 * BUF];
    __shared__ __align__(16) uint16_t Qh[16 * VA_QROW], Ql[16 * VA_QROW];
    __shared__ float wm[ATT_THREADS / WAVE][16], wl[ATT_THREADS / WAVE][16];

    const uint16_t* kbase = a.kc + (size_t)g * maxctx * HD;
    const uint16_t* vbase = a.vc + (size_t)g * maxctx * HD;

    // Prior keys of block b: K rows 16 wave + 4 i + lane / 16, dims 8 (lane % 16) .. + 7 (each
    // load instruction reads four whole rows, 1 KiB contiguous); V keys 4 (tid / 32) + i (+ 32),
    // dims 4 (tid % 32) .. + 3, transposed in registers.  Two register sets: block b + 2
    // is requested while block b + 1 waits in registers and block b is in LDS.  Buffer loads over
    // this group's cache rows: rows past the split are cache rows too (finite; their scores are
    // masked and their weights are 0), rows past the cache and blocks past the split read zeros
    // without touching memory, and so does everything the tail split loads (its tiles come from
    // the pass's own rows).
    // (Macros, not lambdas: register arrays captured by reference stay in scratch memory.)
    const int lrow0 = tail ? 0 : j0;
    const int gbytes = tail ? 0 : maxctx * HD * 2;
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)kbase, (short)0, gbytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)vbase, (short)0, gbytes, 0x00020000);
    uint4 kr[2][4];
    uint2 vr[2][2][4];
#define VA_GLOAD(set_, b_)                                                                            \
    do {                                                                                              \
        const bool in_ = (b_) < nblk;                                                                 \
        const uint32_t kb_ = in_ ? (uint32_t)(((lrow0 + 64 * (b_) + 16 * wave + (lane >> 4)) * HD + 8 * (lane & 15)) * 2) : 0x80000000u; \
        _Pragma("unroll") for (int i = 0; i < 4; ++i)                                                 \
            kr[set_][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(krs, kb_ + 4 * i * HD * 2, 0, 0)); \
        const uint32_t vb_ = in_ ? (uint32_t)(((lrow0 + 64 * (b_) + 4 * (tid >> 5)) * HD + 4 * (tid & 31)) * 2) : 0x80000000u; \
        _Pragma("unroll") for (int h = 0; h < 2; ++h)                                                 \
            _Pragma("unroll") for (int i = 0; i < 4; ++i)                                             \
                vr[set_][h][i] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(      \
                    vrs, vb_ + (uint32_t)((32 * h + i) * HD * 2), 0, 0));                            \
    } while (0)
#define VA_LSTORE(set_, buf_)                                                                         \
    do {                                                                                              \
        uint16_t* Ks_ = (uint16_t*)(kv_lds + (buf_) * BUF);                                           \
        uint16_t* Vt_ = (uint16_t*)(kv_lds + (buf_) * BUF + KS_BYTES);                                \
        _Pragma("unroll") for (int i = 0; i < 4; ++i)                                                 \
            *(uint4*)(Ks_ + (16 * wave + 4 * i + (lane >> 4)) * VA_KROW + 8 * (lane & 15)) = kr[set_][i]; \
        const int d0_ = 4 * (tid & 31);                                                               \
        _Pragma("unroll") for (int h = 0; h < 2; ++h) {                                               \
            const int k0_ = 32 * h + 4 * (tid >> 5);                                                  \
            _Pragma("unroll") for (int j = 0; j < 4; ++j) {                                           \
                /* dim d0_ + j of keys k0_ .. + 3: half j of each key's 4 dims, paired by v_perm */   \
                const uint32_t sel_ = (j & 1) ? 0x07060302u : 0x05040100u;                           \
                const uint2* v_ = vr[set_][h];                                                        \
                const uint32_t lo_ = __builtin_amdgcn_perm(j < 2 ? v_[1].x : v_[1].y, j < 2 ? v_[0].x : v_[0].y, sel_); \
                const uint32_t hi_ = __builtin_amdgcn_perm(j < 2 ? v_[3].x : v_[3].y, j < 2 ? v_[2].x : v_[2].y, sel_); \
                *(uint2*)(Vt_ + (d0_ + j) * VA_VROW + va_vcol(d0_ + j, k0_)) = make_uint2(lo_, hi_);  \
            }                                                                                         \
        }                                                                                             \
    } while (0)

    // Query columns: normalised, rotated, scaled rows split into fp16 hi + lo; zero past the pass.
    // The wave's four columns load their rows, norm weights and rotations together (rows past the
    // pass read the last row and are zeroed), so the prologue is one memory round trip.
    // The tail split's new rows (K / V values, rotations, K norm weights) are requested first of
    // all: its two round trips (these, then the query rows) would otherwise be the kernel's
    // longest path, each queued behind the other splits' cache traffic.
    constexpr int NRW = MAXM / (ATT_THREADS / WAVE);  // new rows per wave: w and w + 4
    float k0[NRW], k1[NRW], v0[NRW], v1[NRW], c0[NRW], s0[NRW], w0 = 0.f, w1 = 0.f;
    if (tail) {
        w0 = a.k_norm[lane];
        w1 = a.k_norm[lane + 64];
#pragma unroll
        for (int i = 0; i < NRW; ++i) {
            const int t = wave + (ATT_THREADS / WAVE) * i, tc = min(t, M - 1);
            const float* ksrc = a.qkv + (size_t)tc * QKV + H + g * HD;
            const float* vsrc = a.qkv + (size_t)tc * QKV + H + NKV * HD + g * HD;
            k0[i] = ksrc[lane];
            k1[i] = ksrc[lane + 64];
            v0[i] = vsrc[lane];
            v1[i] = vsrc[lane + 64];
            const float* cs = a.rope + (size_t)(pos + tc) * 128;
            c0[i] = cs[2 * lane];
            s0[i] = cs[2 * lane + 1];
        }
    }
    // Scores come out in log2 units (q scaled by log2(e) / sqrt(128)): the softmax takes exp2.
    const float qscale = 1.4426950408889634f / sqrtf((float)HD);
    {
        constexpr int NCW = 16 / (ATT_THREADS / WAVE);  // columns per wave
        float x0[NCW], x1[NCW], qc[NCW], qs_[NCW];
        const float w0 = a.q_norm[lane], w1 = a.q_norm[lane + 64];
#pragma unroll
        for (int i = 0; i < NCW; ++i) {
            const int c = wave + (ATT_THREADS / WAVE) * i, t = c >> 1, hh = c & 1, tc = min(t, M - 1);
            const float* src = a.qkv + (size_t)tc * QKV + (2 * g + hh) * HD;
            x0[i] = src[lane];
            x1[i] = src[lane + 64];
            const float* cs = a.rope + (size_t)(pos + tc) * 128;
            qc[i] = cs[2 * lane];
            qs_[i] = cs[2 * lane + 1];
        }
        // Blocks 0 and 1 after the query rows: a load waits for every load issued before it,
        // and the query work should not wait for the cache blocks.
        VA_GLOAD(0, 0);
        VA_GLOAD(1, 1);
#pragma unroll
        for (int i = 0; i < NCW; ++i) {
            const int c = wave + (ATT_THREADS / WAVE) * i, t = c >> 1;
            float y0 = x0[i], y1 = x1[i];
            const float ss = wave_sum(y0 * y0 + y1 * y1);
            const float scale = 1.0f / sqrtf(ss / (float)HD + EPS);
            y0 = y0 * scale * w0;
            y1 = y1 * scale * w1;
            const float r0 = y0 * qc[i] - y1 * qs_[i], r1 = y1 * qc[i] + y0 * qs_[i];
            y0 = t < M ? r0 * qscale : 0.f;
            y1 = t < M ? r1 * qscale : 0.f;
            const f16 h0 = (f16)y0, h1 = (f16)y1;
            Qh[c * VA_QROW + lane] = __builtin_bit_cast(uint16_t, h0);
            Qh[c * VA_QROW + lane + 64] = __builtin_bit_cast(uint16_t, h1);
            Ql[c * VA_QROW + lane] = __builtin_bit_cast(uint16_t, (f16)(y0 - (float)h0));
            Ql[c * VA_QROW + lane + 64] = __builtin_bit_cast(uint16_t, (f16)(y1 - (float)h1));
        }
    }
    if (tail) {
        // The pass's new rows: per-head RMSNorm + RoPE on K, fp16 K/V into the cache and into
        // block 0's tiles; keys M .. 63 are zero rows.  Wave w takes rows w and w + 4, loaded
        // above (rows past the pass read the last row and are not stored).
        uint16_t* Ks = (uint16_t*)kv_lds;
        uint16_t* Vt = (uint16_t*)(kv_lds + KS_BYTES);
#pragma unroll
        for (int i = 0; i < NRW; ++i) {
            const int t = wave + (ATT_THREADS / WAVE) * i;
            uint16_t hk0 = 0, hk1 = 0, hv0 = 0, hv1 = 0;
            if (t < M) {
                // norm_rope_pair's arithmetic, with the loads hoisted
                float x0 = k0[i], x1 = k1[i];
                const float ss = wave_sum(x0 * x0 + x1 * x1);
                const float scale = 1.0f / sqrtf(ss / (float)HD + EPS);
                x0 = x0 * scale * w0;
                x1 = x1 * scale * w1;
                hk0 = f2h(x0 * c0[i] - x1 * s0[i]);
                hk1 = f2h(x1 * c0[i] + x0 * s0[i]);
                hv0 = f2h(v0[i]);
                hv1 = f2h(v1[i]);
                uint16_t* kd = a.kc + ((size_t)g * maxctx + pos + t) * HD;
                uint16_t* vd = a.vc + ((size_t)g * maxctx + pos + t) * HD;
                kd[lane] = hk0;
                kd[lane + 64] = hk1;
                vd[lane] = hv0;
                vd[lane + 64] = hv1;
            }
            Ks[t * VA_KROW + lane] = hk0;
            Ks[t * VA_KROW + lane + 64] = hk1;
            Vt[lane * VA_VROW + va_vcol(lane, t)] = hv0;
            Vt[(lane + 64) * VA_VROW + va_vcol(lane + 64, t)] = hv1;
        }
        for (int t = MAXM + wave; t < ATT_CH; t += ATT_THREADS / WAVE) {
            Ks[t * VA_KROW + lane] = 0;
            Ks[t * VA_KROW + lane + 64] = 0;
            Vt[lane * VA_VROW + va_vcol(lane, t)] = 0;
            Vt[(lane + 64) * VA_VROW + va_vcol(lane + 64, t)] = 0;
        }
        // Set 0 (zeros here) goes to the idle buffer, overwritten before it is read: a use on
        // this path too keeps the loads ahead of the query work.
        VA_LSTORE(0, 1);
    } else {
        VA_LSTORE(0, 0);
    }
    __syncthreads();

    // Online softmax of this wave's keys (16 per block) for its lane's column.
    const int col = r16, ct = col >> 1, kt = 16 * wave;
    v8h qfh[4], qfl[4];  // the query columns' operands, the same for every block
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        qfh[ks] = *(const v8h*)(Qh + r16 * VA_QROW + 32 * ks + 8 * q4);
        qfl[ks] = *(const v8h*)(Ql + r16 * VA_QROW + 32 * ks + 8 * q4);
    }
    float m_run = -__builtin_inff(), l_run = 0.f;
    f32x4 O[8];
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) O[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    // Blocks in pairs, so that each step's register set and LDS buffer are static; an odd count
    // runs a last block of masked keys.
    for (int b0 = 0; b0 < nblk; b0 += 2) {
#pragma unroll
    for (int buf = 0; buf < 2; ++buf) {
        const int b = b0 + buf;
        VA_GLOAD(buf, b + 2);  // this set held block b, already in LDS
        if (b < nblk) {
        const uint16_t* Ks = (const uint16_t*)(kv_lds + buf * BUF);
        const uint16_t* Vt = (const uint16_t*)(kv_lds + buf * BUF + KS_BYTES);
        f32x4 Sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            const v8h kf = *(const v8h*)(Ks + (kt + r16) * VA_KROW + 32 * ks + 8 * q4);
            Sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qfh[ks], Sc, 0, 0, 0);
            Sc = __builtin_amdgcn_mfma_f32_16x16x32_f16(kf, qfl[ks], Sc, 0, 0, 0);
        }
        float mb = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int key = 64 * b + kt + 4 * q4 + i;
            const bool valid = key < P && ct < M && (!tail || key <= ct);
            if (!valid) Sc[i] = -__builtin_inff();
            mb = fmaxf(mb, Sc[i]);
        }
        mb = max_x4(mb);
        const float m_new = fmaxf(m_run, mb);
        const float corr = (m_run == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(m_run - m_new);
        float p[4], ls = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            p[i] = (Sc[i] == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(Sc[i] - m_new);
            ls += p[i];
        }
        ls = sum_x4(ls);
        l_run = l_run * corr + ls;
        m_run = m_new;
        v4h Ph, Pl;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const f16 h = (f16)p[i];
            Ph[i] = h;
            Pl[i] = (f16)(p[i] - (float)h);
        }
        // Rescale only when some column's maximum moved (rare once the first blocks are in).
        if (__builtin_amdgcn_ballot_w64(corr != 1.f)) {
#pragma unroll
            for (int dt = 0; dt < 8; ++dt)
#pragma unroll
                for (int i = 0; i < 4; ++i) O[dt][i] *= corr;
        }
#pragma unroll
        for (int dt = 0; dt < 8; ++dt) {
            const v4h vf = *(const v4h*)(Vt + (16 * dt + r16) * VA_VROW + va_vcol(16 * dt + r16, kt + 4 * q4));
            O[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf, Ph, O[dt], 0, 0, 0);
            O[dt] = __builtin_amdgcn_mfma_f32_16x16x16f16(vf, Pl, O[dt], 0, 0, 0);
        }
        }
        VA_LSTORE(buf ^ 1, buf ^ 1);  // block b + 1 (zeros past the split) into the other buffer
        __syncthreads();
    }
    }
#undef VA_GLOAD
#undef VA_LSTORE
    if (q4 == 0) {
        wm[wave][col] = m_run;
        wl[wave][col] = l_run;
    }
    // The waves' o in their accumulator layout, [wave][dt][lane] float4 (lane l: column l % 16,
    // dims 16 dt + 4 (l / 16) .. + 3), so that writes and reads are each one contiguous 1 KiB
    // per wave and tile; every tile read is done.
    float4* ow = (float4*)kv_lds;
#pragma unroll
    for (int dt = 0; dt < 8; ++dt) ow[(wave * 8 + dt) * WAVE + lane] = make_float4(O[dt][0], O[dt][1], O[dt][2], O[dt][3]);
    __syncthreads();
    // Partial of column c = 2 t + head = lane % 16: thread slots (dt, lane) = tid and tid + 256.
    {
        const int c = lane & 15;
        if ((c >> 1) < M) {
            float mx = -__builtin_inff();
#pragma unroll
            for (int w = 0; w < ATT_THREADS / WAVE; ++w) mx = fmaxf(mx, wm[w][c]);
            float f[ATT_THREADS / WAVE], lsum = 0.f;
#pragma unroll
            for (int w = 0; w < ATT_THREADS / WAVE; ++w) {
                f[w] = (wm[w][c] == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(wm[w][c] - mx);
                lsum = fmaf(wl[w][c], f[w], lsum);
            }
            float* dst = a.part + ((size_t)(g * NS + s) * MAXM * 2 + c) * PART_STRIDE;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int slot = tid + ATT_THREADS * h, dt = slot / WAVE;
                float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
                for (int w = 0; w < ATT_THREADS / WAVE; ++w) {
                    const float4 o = ow[(w * 8 + dt) * WAVE + lane];
                    acc.x = fmaf(o.x, f[w], acc.x);
                    acc.y = fmaf(o.y, f[w], acc.y);
                    acc.z = fmaf(o.z, f[w], acc.z);
                    acc.w = fmaf(o.w, f[w], acc.w);
                }
                float2* d2 = (float2*)(dst + 16 * dt + 4 * (lane >> 4));  // rows of HD + 2 floats: 8-byte aligned
                d2[0] = make_float2(acc.x, acc.y);
                d2[1] = make_float2(acc.z, acc.w);
            }
            if (tid < 16) {
                dst[HD] = mx;
                dst[HD + 1] = lsum;
            }
        }
    }
}

// Merge of the split partials (flash-decoding): one workgroup per (KV group, token x head row),
// grid (NKV, 2 MT).  Runs as its own kernel: the kernel boundary publishes the partials of every
// split, which is far cheaper on a multi-XCD device than a device-scope fence in each split
// workgroup.  Thread t weights split t (t < S); the 128 output elements are summed by two
// halves of the workgroup over interleaved splits, combined in a fixed order.
template <int MT>
__global__ __launch_bounds__(ATT_THREADS) void attention_merge_kernel(AttnArgs a, int splits, int chunk) {
    const State* st = a.st;
    if (st->done) return;
    const int M = a.m_fixed > 0 ? a.m_fixed : (st->n < MT ? st->n : MT);
    const int pos = st->pos;
    const int S = (pos + chunk - 1) / chunk + 1;  // prior splits of `chunk` slots + the tail split
    if (pos < 0 || pos + M > st->maxctx || S > splits) return;
    const int g = blockIdx.x, row = blockIdx.y;
    if (row >= 2 * M) return;
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    constexpr int NS = 16384 / ATT_CH + 1;
    __shared__ float wts[NS];
    __shared__ float red[2][ATT_THREADS / WAVE];
    __shared__ float half[HD];
    const size_t split_stride = (size_t)MAXM * 2 * PART_STRIDE;
    const float* rp = a.part + (size_t)g * splits * split_stride + row * PART_STRIDE;
    // Split maxima and weights: thread t handles splits t, t + 256 (S <= 257).
    float mloc = -__builtin_inff();
    for (int ss = tid; ss < S; ss += ATT_THREADS) mloc = fmaxf(mloc, rp[ss * split_stride + HD]);
    mloc = wave_max(mloc);
    if (lane == 0) red[0][wave] = mloc;
    __syncthreads();
    float mx = red[0][0];
#pragma unroll
    for (int w = 1; w < ATT_THREADS / WAVE; ++w) mx = fmaxf(mx, red[0][w]);
    float L = 0.f;
    for (int ss = tid; ss < S; ss += ATT_THREADS) {
        const float m = rp[ss * split_stride + HD];
        const float wgt = (m == -__builtin_inff()) ? 0.f : expf(m - mx);
        wts[ss] = wgt;
        L += wgt * rp[ss * split_stride + HD + 1];
    }
    L = wave_sum(L);
    if (lane == 0) red[1][wave] = L;
    __syncthreads();
    float Lsum = 0.f;
#pragma unroll
    for (int w = 0; w < ATT_THREADS / WAVE; ++w) Lsum += red[1][w];
    // Weighted sum: threads (h, d), h = tid / 128 takes splits h, h + 2, ...
    const int h = tid / HD, d = tid % HD;
    float O = 0.f;
    int ss = h;
    for (; ss + 6 < S; ss += 8) {
        float v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) v[u] = rp[(ss + 2 * u) * split_stride + d];
#pragma unroll
        for (int u = 0; u < 4; ++u) O = fmaf(wts[ss + 2 * u], v[u], O);
    }
    for (; ss < S; ss += 2) O = fmaf(wts[ss], rp[ss * split_stride + d], O);
    if (h == 1) half[d] = O;
    __syncthreads();
    if (h == 0) {
        const int t = row / 2, hh = row % 2;
        a.out[(size_t)t * H + (2 * g + hh) * HD + d] = (O + half[d]) / Lsum;
    }
}

// Merge of the matrix-core path's NS (<= VA_SPLITS) partials of one (KV group, token x head) row,
// grid (NKV, 2 MAXM).  Their maxima are in log2 units.  Every partial's o values are requested
// up front together with the (m, l) pairs, so the merge is one memory round trip; wave 0 holds
// the NS pairs (one per lane) for the maximum and the weights.
static_assert(VA_SPLITS <= WAVE, "one lane per split");
__global__ __launch_bounds__(ATT_THREADS) void attention_merge_mfma_kernel(AttnArgs a, int NS) {
    const State* st = a.st;
    if (st->done) return;
    const int M = a.m_fixed > 0 ? a.m_fixed : (st->n < MAXM ? st->n : MAXM);
    const int pos = st->pos;
    if (pos < 0 || pos + M > st->maxctx || NS > VA_SPLITS) return;
    const int g = blockIdx.x, row = blockIdx.y;
    if (row >= 2 * M) return;
    const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
    const int h = tid / HD, d = tid % HD;  // half h of the workgroup takes splits h, h + 2, ...
    const size_t split_stride = (size_t)MAXM * 2 * PART_STRIDE;
    const float* rp = a.part + (size_t)g * NS * split_stride + row * PART_STRIDE;
    __shared__ float wts[VA_SPLITS];
    __shared__ float Lsum;
    __shared__ float half[HD];
    float ov[VA_SPLITS / 2];
#pragma unroll
    for (int u = 0; u < VA_SPLITS / 2; ++u) {
        const int ss = h + 2 * u;
        ov[u] = ss < NS ? rp[ss * split_stride + d] : 0.f;
    }
    if (wave == 0) {
        float m = -__builtin_inff(), l = 0.f;
        if (lane < NS) {
            m = rp[lane * split_stride + HD];
            l = rp[lane * split_stride + HD + 1];
        }
        const float mx = wave_max(m);  // finite: the tail split holds each row's own key
        const float wgt = (m == -__builtin_inff()) ? 0.f : __builtin_amdgcn_exp2f(m - mx);
        wts[lane] = wgt;
        const float L = wave_sum(wgt * l);
        if (lane == 0) Lsum = L;
    }
    __syncthreads();
    float O = 0.f;
#pragma unroll
    for (int u = 0; u < VA_SPLITS / 2; ++u)
        if (h + 2 * u < NS) O = fmaf(wts[h + 2 * u], ov[u], O);
    if (h == 1) half[d] = O;
    __syncthreads();
    if (h == 0) {
        const int t = row / 2, hh = row % 2;
        a.out[(size_t)t * H + (2 * g + hh) * HD + d] = (O + half[d]) / Lsum;
    }
}

int attention_splits(int maxctx) { return (maxctx + ATT_CH - 1) / ATT_CH + 1; }

hipError_t launch_attention(const AttnArgs& a, int mt, int splits, hipStream_t s) {
    if (splits > 16384 / ATT_CH + 1) return hipErrorInvalidValue;
    const dim3 grid(splits, NKV);
    if (mt == 1) {
        hipLaunchKernelGGL(attention_kernel<1>, grid, dim3(ATT_THREADS), 0, s, a);
        hipLaunchKernelGGL(attention_merge_kernel<1>, dim3(NKV, 2), dim3(ATT_THREADS), 0, s, a, splits, ATT_CH);
    } else {
        // The partial buffer holds `splits` (>= 2) splits per group.
        const int ns = splits < VA_SPLITS ? splits : VA_SPLITS;
        hipLaunchKernelGGL(attention_mfma_kernel, dim3(NKV, ns), dim3(ATT_THREADS), 0, s, a);
        hipLaunchKernelGGL(attention_merge_mfma_kernel, dim3(NKV, 2 * MAXM), dim3(ATT_THREADS), 0, s, a, ns);
    }
    return hipGetLastError();
}

}  // namespace icua
