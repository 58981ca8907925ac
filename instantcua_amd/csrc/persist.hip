// Persistent decode kernel: whole greedy decode steps (28 layers + lm_head + commit) in one
// cooperative launch, gfx950.  Same math and tile layout as gemv.hip / attention.hip; the
// difference is the schedule.
//
// Why.  As separate kernels a decode step is ~170 dependent launches whose fixed latency
// (launch, cold weight fetch, prologue, drain: 5-10 us each) dominates the 180 us the step's
// bytes need at 8 TB/s.  Here every workgroup stays resident and, before waiting for a stage's
// inputs, already issues the loads of its slice of that stage's weights (and K/V rows), so the
// HBM latency overlaps the synchronisation.
//
// Grid.  One 512-thread workgroup per CU (256).  Static work split per layer:
//   QKV   256 row blocks, block w                  (fused q|k|v rows, Convert.swift:185-188)
//   attn  KV group g = w / 32, slot range s = w % 32 of [0, pos); split 31 also owns the new row
//   merge the last split to arrive for a group merges the group's 32 partials
//   O     128 row blocks, workgroups 0..127
//   GU    768 row blocks (8 gate + 8 up rows each), blocks 3w .. 3w + 2
//   down  128 row blocks (K = 6144), workgroups 0..127
// then lm_head over 9496 row blocks (w, w + 256, ...) with per-workgroup argmax partials, and the
// commit (Shaders.swift:1501-1571) by the last workgroup to finish lm_head.
//
// Synchronisation.  Monotonic arrival counters in device memory (zeroed before the launch);
// a stage waits until the counter of its inputs reaches the count for (step, layer).  Large
// fan-ins arrive on 16 counters in separate 256-byte lines and are polled by one wave (one
// lane per counter).  Activations crossing workgroups are written and read with device-scope
// relaxed atomics (global_store/load ... sc1: coherent across the XCDs' L2s, no cache
// flushes); each arrival follows an s_waitcnt vmcnt(0) (the workgroup barrier before it), so
// a counter value implies the data it covers is visible.  Every spin is bounded: a timeout
// raises an error flag that makes all workgroups leave, and the host reports it.
#include "icua_device.h"
#include "icua_kernels.h"
#include "icua_persist.h"

namespace icua {
namespace pk {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int THREADS = 512, WAVES = 8;
constexpr int NWG = PERSIST_WGS;   // 256
constexpr int ATT_SPLITS = NWG / NKV;  // 32
constexpr int SPIN_LIMIT = 4000000;
constexpr int PART = HD + 2;
constexpr int ATT_SPQ = 8;                 // cache slots per quarter-wave per block
constexpr int ATT_BLOCK = 32 * ATT_SPQ;     // 256 slots per block

// Counter slots (each in its own 256-byte line).
enum {
    C_COMMIT = 0,
    C_QKV = 1,      // + g
    C_ATT = 9,      // + g
    C_MERGED = 17,
    C_ERR = 18,
    C_O = 32,       // 16 sub-counters each
    C_GU = 48,
    C_DOWN = 64,
    C_LM = 80,
    C_SLOTS = 96,
};
__device__ __forceinline__ unsigned* slot(unsigned* s, int i) { return s + i * 64; }

// threadIdx.x behind an empty asm: per-lane address math derived from it is recomputed where it
// is used instead of being hoisted out of the step / layer loops and held live (which spills).
__device__ __forceinline__ int my_tid() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

__device__ __forceinline__ unsigned ldc(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned addc(unsigned* p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ldf(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void stf(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int ldi(const int* p) { return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ void sti(int* p, int v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
__device__ __forceinline__ float2 ldf2(const float* p) {
    const uint64_t v = __hip_atomic_load((const uint64_t*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return make_float2(__builtin_bit_cast(float, (uint32_t)v), __builtin_bit_cast(float, (uint32_t)(v >> 32)));
}
__device__ __forceinline__ void stf2(float* p, float a, float b) {
    const uint64_t v = (uint64_t)__builtin_bit_cast(uint32_t, a) | ((uint64_t)__builtin_bit_cast(uint32_t, b) << 32);
    __hip_atomic_store((uint64_t*)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct Shared {
    uint8_t A[96 * 1024];      // activation operands (q4: 1 KiB per 64-K group, up to K = 6144)
    float fx[192 * 2];         // per-group (2^(e-21), sum X * 2^(e-21))
    float red[THREADS / 64 * 64];
    float qs[2][HD];           // attention: two query heads
    float ktail[HD], vtail[HD];
    float sc[2][256];          // attention scores of one block
    float ored[WAVES][2][HD];
    float misc[64];
    int flag;
};

// ------------------------------------------------------------------------------------------
// Waits.  Wave 0 polls; the whole workgroup learns the outcome through LDS.

__device__ bool wait_single(Shared& S, unsigned* sync, int idx, unsigned target) {
    __syncthreads();
    if (my_tid() < 64) {
        int ok = 1, it = 0;
        if (my_tid() == 0) {
            while (ldc(slot(sync, idx)) < target) {
                if ((++it & 255) == 0 && ldc(slot(sync, C_ERR)) != 0) { ok = 0; break; }
                if (it > SPIN_LIMIT) {
                    __hip_atomic_store(slot(sync, C_ERR), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    ok = 0;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            S.flag = ok;
        }
    }
    __syncthreads();
    return S.flag != 0;
}

// Fan-in over 16 sub-counters at idx..idx+15; `per_sub` arrivals per sub-counter per round.
__device__ bool wait_fan(Shared& S, unsigned* sync, int idx, unsigned per_sub_target) {
    __syncthreads();
    if (my_tid() < 64) {
        const int lane = my_tid();
        int ok = 1, it = 0;
        while (true) {
            const bool mine = (lane >= 16) || ldc(slot(sync, idx + lane)) >= per_sub_target;
            if (__all(mine)) break;
            if ((++it & 255) == 0 && ldc(slot(sync, C_ERR)) != 0) { ok = 0; break; }
            if (it > SPIN_LIMIT) {
                if (lane == 0) __hip_atomic_store(slot(sync, C_ERR), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                ok = 0;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
        if (lane == 0) S.flag = ok;
    }
    __syncthreads();
    return S.flag != 0;
}

// Arrival after this workgroup's coherent stores.  Every wave first waits until its own stores
// are acknowledged (s_waitcnt vmcnt(0): a device-scope store is then visible to every CU); the
// workgroup barrier alone does not wait for global stores on gfx950.
__device__ __forceinline__ unsigned arrive(unsigned* sync, int idx) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    unsigned old = 0;
    if (my_tid() == 0) old = addc(slot(sync, idx), 1u);
    return old;
}

// ------------------------------------------------------------------------------------------
// Activation staging for one token: fp32 vector (coherent loads) -> 22-bit slices -> A operands.
// Rows 0, 1, 2 of each group tile hold the hi, mid, lo slices; rows 3..15 stay zero (zeroed at
// kernel start).

template <int FMT>
__device__ void stage_vec(Shared& S, const float* src, int K, const float* norm_w) {
    constexpr int G = (FMT == FMT_Q4) ? 64 : 32;
    constexpr int TILE = (FMT == FMT_Q4) ? 1024 : 512;
    const int tid = my_tid(), lane = tid % 64, wave = tid / 64;
    const int nunits = K / 8;
    float v[2][8];
    float ss = 0.f;
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int u = tid + it * THREADS;
        if (u < nunits) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float2 p = ldf2(src + u * 8 + 2 * i);
                v[it][2 * i] = p.x;
                v[it][2 * i + 1] = p.y;
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) ss += v[it][i] * v[it][i];
        }
    }
    float scale = 1.f;
    if (norm_w) {
        ss = wave_sum(ss);
        if (lane == 0) S.red[wave] = ss;
        __syncthreads();
        float tot = 0.f;
        for (int w = 0; w < WAVES; ++w) tot += S.red[w];
        scale = 1.0f / sqrtf(tot / (float)K + EPS);
        __syncthreads();
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
        const int u = tid + it * THREADS;
        if (it * THREADS >= nunits) break;  // uniform across the workgroup
        const bool act = u < nunits;
        const int k0 = (act ? u : 0) * 8;
        float x[8];
        if (norm_w && act) {
            const float4 w0 = ((const float4*)(norm_w + k0))[0], w1 = ((const float4*)(norm_w + k0))[1];
            x[0] = v[it][0] * scale * w0.x; x[1] = v[it][1] * scale * w0.y; x[2] = v[it][2] * scale * w0.z;
            x[3] = v[it][3] * scale * w0.w; x[4] = v[it][4] * scale * w1.x; x[5] = v[it][5] * scale * w1.y;
            x[6] = v[it][6] * scale * w1.z; x[7] = v[it][7] * scale * w1.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) x[i] = act ? v[it][i] : 0.f;
        }
        float amax = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(x[i]));
        int bits = (int)as_u32(amax);
        bits = max(bits, dpp_i<DPP_XOR1>(bits));
        bits = max(bits, dpp_i<DPP_XOR2>(bits));
        if constexpr (G == 64) bits = max(bits, dpp_i<DPP_HALF_MIRROR>(bits));
        int e = ((bits >> 23) & 0xFF) - 127;
        if (bits == 0) e = -100;
        const int sh = 21 - e;
        int X[8], xs = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            X[i] = (int)rintf(ldexpf(x[i], sh));
            xs += X[i];
        }
        xs += dpp_i<DPP_XOR1>(xs);
        xs += dpp_i<DPP_XOR2>(xs);
        if constexpr (G == 64) xs += dpp_i<DPP_HALF_MIRROR>(xs);
        if (!act) continue;
        uint32_t sl[3][2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            uint32_t p0 = 0, p1 = 0, p2 = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int xv = X[4 * h + i];
                const int lo = (int)(int8_t)(xv & 0xFF);
                const int r1 = (xv - lo) >> 8;
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
        uint8_t* A = S.A + gl * TILE;
        if constexpr (FMT == FMT_Q4) {
            const int q = kk / 16, j0 = kk % 16;
            *(uint2*)(A + (0 + 16 * q) * 16 + j0) = make_uint2(sl[2][0], sl[2][1]);
            *(uint2*)(A + (1 + 16 * q) * 16 + j0) = make_uint2(sl[1][0], sl[1][1]);
            *(uint2*)(A + (2 + 16 * q) * 16 + j0) = make_uint2(sl[0][0], sl[0][1]);
        } else {
            const int q = kk / 8;
            *(uint2*)(A + (0 + 16 * q) * 8) = make_uint2(sl[2][0], sl[2][1]);
            *(uint2*)(A + (1 + 16 * q) * 8) = make_uint2(sl[1][0], sl[1][1]);
            *(uint2*)(A + (2 + 16 * q) * 8) = make_uint2(sl[0][0], sl[0][1]);
        }
        if (kk == 0) {
            const float f = ldexpf(1.0f, -sh);
            S.fx[gl * 2] = f;
            S.fx[gl * 2 + 1] = (float)xs * f;
        }
    }
    __syncthreads();
}

// One 1 KiB chunk of a 16-row block against the staged operands; returns the lane's partial
// (lanes 0-15 hold rows 0-15 of the block for the token).
template <int FMT>
__device__ __forceinline__ float chunk_mac(const Shared& S, uint4 wv, uint2 sbv, int c, int lane) {
    float acc = 0.f;
    if constexpr (FMT == FMT_Q4) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const uint32_t d0 = hh ? wv.z : wv.x, d1 = hh ? wv.w : wv.y;
            v4i B;
            B[0] = (int)(d0 & 0x0F0F0F0Fu);
            B[1] = (int)((d0 >> 4) & 0x0F0F0F0Fu);
            B[2] = (int)(d1 & 0x0F0F0F0Fu);
            B[3] = (int)((d1 >> 4) & 0x0F0F0F0Fu);
            const int gl = 2 * c + hh;
            const v4i A = *(const v4i*)(S.A + gl * 1024 + lane * 16);
            const v4i zero = {0, 0, 0, 0};
            const v4i C = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, zero, 0, 0, 0);
            const float Sv = fmaf((float)C[0], 65536.f, fmaf((float)C[1], 256.f, (float)C[2]));
            const f16x2 sb2 = as_h2(hh ? sbv.y : sbv.x);
            acc = fmaf((float)sb2.x * S.fx[gl * 2], Sv, fmaf((float)sb2.y, S.fx[gl * 2 + 1], acc));
        }
    } else {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const long B = (long)(hh ? ((uint64_t)wv.w << 32 | wv.z) : ((uint64_t)wv.y << 32 | wv.x));
            const int gl = 2 * c + hh;
            const long A = *(const long*)(S.A + gl * 512 + lane * 8);
            const v4i zero = {0, 0, 0, 0};
            const v4i C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, zero, 0, 0, 0);
            const float Sv = fmaf((float)C[0], 65536.f, fmaf((float)C[1], 256.f, (float)C[2]));
            const f16x2 s2 = as_h2(sbv.x);
            acc = fmaf((hh ? (float)s2.y : (float)s2.x) * S.fx[gl * 2], Sv, acc);
        }
    }
    return acc;
}

// Chunk geometry: q4 chunk = 128 K (two 64-K groups), q8 chunk = 64 K (two 32-K groups).
template <int FMT>
__device__ __forceinline__ uint2 load_sb(const uint8_t* sb, int row, int K, int c) {
    if constexpr (FMT == FMT_Q4)
        return *(const uint2*)(sb + ((size_t)row * (K / 64) + 2 * c) * 4);
    else
        return make_uint2(*(const uint32_t*)(sb + ((size_t)row * (K / 32) + 2 * c) * 2), 0u);
}

// Cross-wave sum of per-lane partials; returns the total in wave 0 (lanes 0-15 meaningful).
__device__ __forceinline__ float reduce_waves(Shared& S, float acc) {
    const int lane = my_tid() % 64, wave = my_tid() / 64;
    S.red[wave * 64 + lane] = acc;
    __syncthreads();
    float s = 0.f;
    if (wave == 0)
        for (int w = 0; w < WAVES; ++w) s += S.red[w * 64 + lane];
    __syncthreads();
    return s;
}

__device__ __forceinline__ void norm_rope(float& a, float& b, const float* w, const float* cs, int lane) {
    const float ss = wave_sum(a * a + b * b);
    const float scale = 1.0f / sqrtf(ss / (float)HD + EPS);
    a = a * scale * w[lane];
    b = b * scale * w[lane + 64];
    const float c = cs[2 * lane], sn = cs[2 * lane + 1];
    const float a2 = a * c - b * sn, b2 = b * c + a * sn;
    a = a2;
    b = b2;
}

// ------------------------------------------------------------------------------------------

template <int FMT>
__global__ __launch_bounds__(THREADS, 1) void decode_kernel(PersistArgs a) {
    constexpr int CPB2 = (FMT == FMT_Q4) ? H / 128 : H / 64;    // chunks per block, K = 2048
    constexpr int CPB6 = (FMT == FMT_Q4) ? FF / 128 : FF / 64;  // K = 6144
    constexpr int CW2 = CPB2 / WAVES, CW6 = CPB6 / WAVES;       // chunks per wave
    __shared__ Shared S;
    const int w = blockIdx.x;
    unsigned* sync = a.sync;
    for (int i = my_tid(); i < (int)sizeof(S.A) / 4; i += THREADS) ((uint32_t*)S.A)[i] = 0u;
    __syncthreads();

    const int L = a.nlayers;
    for (int step = 0; step < a.nsteps; ++step) {
        if (!wait_single(S, sync, C_COMMIT, (unsigned)step)) return;
        const int done = ldi(&a.st->done);
        const int pos = ldi(&a.st->pos);
        if (done) break;
        if (pos + 1 > a.maxctx || ldi(&a.st->n) != 1) break;  // host-checked; single-row passes only
        for (int l = 0; l < L; ++l) {
            const LayerPtrs& P = a.layers[l];
            const unsigned round = (unsigned)(step * L + l);  // completed layers before this one

            // ---------------- QKV: row block w -------------------------------------------
            {
                const int tid = my_tid(), lane = tid % 64, wave = tid / 64, r16 = lane % 16;
                (void)r16;
                const int rb = w;
                uint4 wv[CW2];
                uint2 sbv[CW2];
                const uint8_t* blk = P.wqkv + (size_t)rb * CPB2 * 1024;
#pragma unroll
                for (int i = 0; i < CW2; ++i) {
                    const int c = wave * CW2 + i;
                    wv[i] = ((const uint4*)(blk + (size_t)c * 1024))[lane];
                    sbv[i] = load_sb<FMT>(P.wqkv_sb, rb * 16 + r16, H, c);
                }
                // Layer 0 reads the embedding the commit wrote (already waited for above).
                if (l > 0 && !wait_fan(S, sync, C_DOWN, round * (NWG / 2) / 16)) return;
                stage_vec<FMT>(S, a.x, H, P.attn_norm);
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < CW2; ++i) acc += chunk_mac<FMT>(S, wv[i], sbv[i], wave * CW2 + i, lane);
                const float y = reduce_waves(S, acc);
                if (wave == 0 && lane < 16) stf(a.qkv + rb * 16 + lane, y);
                const int g = rb < 128 ? rb / 16 : rb < 192 ? (rb - 128) / 8 : (rb - 192) / 8;
                arrive(sync, C_QKV + g);
            }

            // ---------------- attention: group g, slot range s ----------------------------
            // The pos + 1 rows (cache rows 0..pos-1 and the new row pos) are split evenly over
            // the group's 32 workgroups; the one whose range holds row pos writes it.
            {
                const int tid = my_tid(), lane = tid % 64, wave = tid / 64, r16 = lane % 16;
                (void)r16;
                const int g = w / ATT_SPLITS, s = w % ATT_SPLITS;
                const int tot = pos + 1;
                const int chunk = (tot + ATT_SPLITS - 1) / ATT_SPLITS;
                const int j0 = min(s * chunk, tot), j1 = min(j0 + chunk, tot);
                const bool tail = (j0 <= pos) && (pos < j1);
                const int nprior = max(0, min(j1, pos) - j0);
                const int ntot = j1 - j0;
                const int quad = tid / 16, ql = tid % 16;  // 32 quarter-waves, 8 dims per lane
                const uint16_t* kb = a.kv + ((size_t)(l * 2 + 0) * NKV + g) * a.maxctx * HD;
                const uint16_t* vb = a.kv + ((size_t)(l * 2 + 1) * NKV + g) * a.maxctx * HD;
                // First block of K/V rows (ATT_SPQ slots per quarter-wave), issued before the wait.
                // Only rows < pos are ever loaded: row pos is written during this step by another
                // workgroup, and a line of it cached early would go stale.
                uint4 kr[ATT_SPQ], vr[ATT_SPQ];
#pragma unroll
                for (int i = 0; i < ATT_SPQ; ++i) {
                    const int p = quad + 32 * i;
                    kr[i] = make_uint4(0u, 0u, 0u, 0u);
                    vr[i] = kr[i];
                    if (p < nprior) {
                        kr[i] = *(const uint4*)(kb + (size_t)(j0 + p) * HD + 8 * ql);
                        vr[i] = *(const uint4*)(vb + (size_t)(j0 + p) * HD + 8 * ql);
                    }
                }
                if (!wait_single(S, sync, C_QKV + g, (round + 1) * 32)) return;
                const float* rope = a.rope + (size_t)pos * 128;
                if (wave < 2) {  // queries of heads 2g, 2g+1
                    const int hh = wave;
                    float x0 = ldf(a.qkv + (2 * g + hh) * HD + lane), x1 = ldf(a.qkv + (2 * g + hh) * HD + lane + 64);
                    norm_rope(x0, x1, P.q_norm, rope, lane);
                    const float qscale = 1.0f / sqrtf((float)HD);
                    S.qs[hh][lane] = x0 * qscale;
                    S.qs[hh][lane + 64] = x1 * qscale;
                } else if (wave == 2 && tail) {  // the new K/V row of this group
                    float k0 = ldf(a.qkv + H + g * HD + lane), k1 = ldf(a.qkv + H + g * HD + lane + 64);
                    norm_rope(k0, k1, P.k_norm, rope, lane);
                    const float v0 = ldf(a.qkv + H + NKV * HD + g * HD + lane);
                    const float v1 = ldf(a.qkv + H + NKV * HD + g * HD + lane + 64);
                    S.ktail[lane] = h2f(f2h(k0));
                    S.ktail[lane + 64] = h2f(f2h(k1));
                    S.vtail[lane] = h2f(f2h(v0));
                    S.vtail[lane + 64] = h2f(f2h(v1));
                }
                __syncthreads();
                if (tail && tid < 128) {
                    // The new cache row, written through to the coherence point (device-scope
                    // stores) so that any workgroup reads it in the next step.
                    const float* src = tid < 64 ? S.ktail : S.vtail;
                    uint16_t* dst = (uint16_t*)(tid < 64 ? kb : vb) + (size_t)pos * HD;
                    const int d = 2 * (tid % 64);
                    const uint32_t v = (uint32_t)f2h(src[d]) | ((uint32_t)f2h(src[d + 1]) << 16);
                    __hip_atomic_store((uint32_t*)(dst + d), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                float q[2][8];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int d = 0; d < 8; ++d) q[hh][d] = S.qs[hh][8 * ql + d];
                float m_run[2] = {-__builtin_inff(), -__builtin_inff()}, l_run[2] = {0.f, 0.f};
                float o[2][8];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int d = 0; d < 8; ++d) o[hh][d] = 0.f;
                for (int b0 = 0; b0 < ntot; b0 += ATT_BLOCK) {
                    const int nb = min(ATT_BLOCK, ntot - b0);
                    if (b0 > 0) {
#pragma unroll
                        for (int i = 0; i < ATT_SPQ; ++i) {
                            const int p = b0 + quad + 32 * i;
                            if (p < nprior) {
                                kr[i] = *(const uint4*)(kb + (size_t)(j0 + p) * HD + 8 * ql);
                                vr[i] = *(const uint4*)(vb + (size_t)(j0 + p) * HD + 8 * ql);
                            }
                        }
                    }
                    // The new row (block slot pos - j0 - b0) comes from LDS, not from the cache.
                    const int pnew = tail ? pos - j0 - b0 : -1;
#pragma unroll
                    for (int i = 0; i < ATT_SPQ; ++i) {
                        const int p = quad + 32 * i;
                        if (p == pnew) {
                            uint32_t kk[4], vv[4];
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                kk[j] = (uint32_t)f2h(S.ktail[8 * ql + 2 * j]) | ((uint32_t)f2h(S.ktail[8 * ql + 2 * j + 1]) << 16);
                                vv[j] = (uint32_t)f2h(S.vtail[8 * ql + 2 * j]) | ((uint32_t)f2h(S.vtail[8 * ql + 2 * j + 1]) << 16);
                            }
                            kr[i] = make_uint4(kk[0], kk[1], kk[2], kk[3]);
                            vr[i] = make_uint4(vv[0], vv[1], vv[2], vv[3]);
                        }
                    }
#pragma unroll
                    for (int i = 0; i < ATT_SPQ; ++i) {
                        const int p = quad + 32 * i;
                        const uint32_t dk[4] = {kr[i].x, kr[i].y, kr[i].z, kr[i].w};
                        float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const f16x2 hk = as_h2(dk[j]);
                            const float k0 = (float)hk.x, k1 = (float)hk.y;
                            acc0 = fmaf(q[0][2 * j], k0, acc0);
                            acc0 = fmaf(q[0][2 * j + 1], k1, acc0);
                            acc1 = fmaf(q[1][2 * j], k0, acc1);
                            acc1 = fmaf(q[1][2 * j + 1], k1, acc1);
                        }
                        acc0 = sum16(acc0);
                        acc1 = sum16(acc1);
                        if (ql == 0) {
                            S.sc[0][p] = (p < nb) ? acc0 : -__builtin_inff();
                            S.sc[1][p] = (p < nb) ? acc1 : -__builtin_inff();
                        }
                    }
                    __syncthreads();
                    // Block softmax statistics: waves 0 and 1, one head each, ATT_BLOCK / 64 slots
                    // per lane.
                    if (wave < 2) {
                        float sv[ATT_BLOCK / 64];
                        float mb = -__builtin_inff();
#pragma unroll
                        for (int i = 0; i < ATT_BLOCK / 64; ++i) {
                            sv[i] = S.sc[wave][lane + 64 * i];
                            mb = fmaxf(mb, sv[i]);
                        }
                        mb = wave_max(mb);
                        const float mn = fmaxf(m_run[wave], mb);
                        float ls = 0.f;
#pragma unroll
                        for (int i = 0; i < ATT_BLOCK / 64; ++i) {
                            const float e = (sv[i] == -__builtin_inff()) ? 0.f : expf(sv[i] - mn);
                            S.sc[wave][lane + 64 * i] = e;
                            ls += e;
                        }
                        ls = wave_sum(ls);
                        if (lane == 0) {
                            S.misc[wave] = mn;  // new running max
                            S.misc[2 + wave] = ls;
                        }
                    }
                    __syncthreads();
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const float mn = S.misc[hh];
                        const float corr = (m_run[hh] == -__builtin_inff()) ? 0.f : expf(m_run[hh] - mn);
                        l_run[hh] = l_run[hh] * corr + S.misc[2 + hh];
                        m_run[hh] = mn;
#pragma unroll
                        for (int d = 0; d < 8; ++d) o[hh][d] *= corr;
                    }
#pragma unroll
                    for (int i = 0; i < ATT_SPQ; ++i) {
                        const int p = quad + 32 * i;
                        const float p0 = S.sc[0][p], p1 = S.sc[1][p];
                        const uint32_t dv[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const f16x2 hv = as_h2(dv[j]);
                            const float v0 = (float)hv.x, v1 = (float)hv.y;
                            o[0][2 * j] = fmaf(p0, v0, o[0][2 * j]);
                            o[0][2 * j + 1] = fmaf(p0, v1, o[0][2 * j + 1]);
                            o[1][2 * j] = fmaf(p1, v0, o[1][2 * j]);
                            o[1][2 * j + 1] = fmaf(p1, v1, o[1][2 * j + 1]);
                        }
                    }
                    __syncthreads();
                }
                // Reduce o over the 32 quarter-waves: 4 per wave by lane swaps, 8 waves via LDS.
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int d = 0; d < 8; ++d) {
                        const float t1 = swap16_add(o[hh][d], o[hh][d]);
                        o[hh][d] = swap32_add(t1, t1);
                    }
                if (lane < 16) {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int d = 0; d < 8; ++d) S.ored[wave][hh][8 * ql + d] = o[hh][d];
                }
                __syncthreads();
                float* part = a.part + (size_t)(g * ATT_SPLITS + s) * 2 * PART;
                if (tid < 2 * HD) {
                    const int hh = tid / HD, d = tid % HD;
                    float acc = 0.f;
                    for (int ww = 0; ww < WAVES; ++ww) acc += S.ored[ww][hh][d];
                    stf(part + hh * PART + d, acc);
                    if (d == 0) {
                        stf(part + hh * PART + HD, m_run[hh]);
                        stf(part + hh * PART + HD + 1, l_run[hh]);
                    }
                }
                const unsigned old = arrive(sync, C_ATT + g);
                if (tid == 0) S.flag = (old == (round + 1) * ATT_SPLITS - 1);
                __syncthreads();
                if (S.flag) {  // last split of this group to finish: merge the 32 partials
                    const float* gp = a.part + (size_t)g * ATT_SPLITS * 2 * PART;
                    if (tid < 2 * HD) {
                        const int hh = tid / HD, d = tid % HD;
                        float m[ATT_SPLITS], lv[ATT_SPLITS], ov[ATT_SPLITS];
#pragma unroll
                        for (int ss = 0; ss < ATT_SPLITS; ++ss) {  // all loads in flight at once
                            const float* pp = gp + (ss * 2 + hh) * PART;
                            m[ss] = ldf(pp + HD);
                            lv[ss] = ldf(pp + HD + 1);
                            ov[ss] = ldf(pp + d);
                        }
                        float mx = -__builtin_inff();
#pragma unroll
                        for (int ss = 0; ss < ATT_SPLITS; ++ss) mx = fmaxf(mx, m[ss]);
                        float Lsum = 0.f, O = 0.f;
#pragma unroll
                        for (int ss = 0; ss < ATT_SPLITS; ++ss) {
                            const float wgt = (m[ss] == -__builtin_inff()) ? 0.f : expf(m[ss] - mx);
                            Lsum = fmaf(wgt, lv[ss], Lsum);
                            O = fmaf(wgt, ov[ss], O);
                        }
                        stf(a.attn + (2 * g + hh) * HD + d, O / Lsum);
                    }
                    arrive(sync, C_MERGED);
                }
            }

            // ---------------- O projection: workgroups 0..127 ------------------------------
            if (w < H / 16) {
                const int tid = my_tid(), lane = tid % 64, wave = tid / 64, r16 = lane % 16;
                (void)r16;
                const int rb = w;
                uint4 wv[CW2];
                uint2 sbv[CW2];
                const uint8_t* blk = P.wo + (size_t)rb * CPB2 * 1024;
#pragma unroll
                for (int i = 0; i < CW2; ++i) {
                    const int c = wave * CW2 + i;
                    wv[i] = ((const uint4*)(blk + (size_t)c * 1024))[lane];
                    sbv[i] = load_sb<FMT>(P.wo_sb, rb * 16 + r16, H, c);
                }
                if (!wait_single(S, sync, C_MERGED, (round + 1) * NKV)) return;
                stage_vec<FMT>(S, a.attn, H, nullptr);
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < CW2; ++i) acc += chunk_mac<FMT>(S, wv[i], sbv[i], wave * CW2 + i, lane);
                const float y = reduce_waves(S, acc);
                if (wave == 0 && lane < 16) {
                    float* xo = a.x + rb * 16 + lane;
                    stf(xo, ldf(xo) + y);
                }
                arrive(sync, C_O + (w % 16));
            }

            // ---------------- gate|up + SwiGLU: blocks 3w .. 3w + 2 ------------------------
            {
                const int tid = my_tid(), lane = tid % 64, wave = tid / 64, r16 = lane % 16;
                (void)r16;
                uint4 wv[3][CW2];
                uint2 sbv[3][CW2];
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const int rb = 3 * w + j;
                    const uint8_t* blk = P.wgu + (size_t)rb * CPB2 * 1024;
#pragma unroll
                    for (int i = 0; i < CW2; ++i) {
                        const int c = wave * CW2 + i;
                        wv[j][i] = ((const uint4*)(blk + (size_t)c * 1024))[lane];
                        sbv[j][i] = load_sb<FMT>(P.wgu_sb, rb * 16 + r16, H, c);
                    }
                }
                if (!wait_fan(S, sync, C_O, (round + 1) * (H / 16) / 16)) return;
                stage_vec<FMT>(S, a.x, H, P.mlp_norm);
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    float acc = 0.f;
#pragma unroll
                    for (int i = 0; i < CW2; ++i) acc += chunk_mac<FMT>(S, wv[j][i], sbv[j][i], wave * CW2 + i, lane);
                    const float y = reduce_waves(S, acc);
                    if (wave == 0) {
                        const float up = __shfl_xor(y, 8);
                        if (lane < 8) stf(a.h + (3 * w + j) * 8 + lane, (y / (1.f + expf(-y))) * up);
                    }
                }
                arrive(sync, C_GU + (w % 16));
            }

            // ---------------- down + residual: workgroups 0..127 ---------------------------
            if (w < H / 16) {
                const int tid = my_tid(), lane = tid % 64, wave = tid / 64, r16 = lane % 16;
                (void)r16;
                const int rb = w;
                uint4 wv[CW6];
                uint2 sbv[CW6];
                const uint8_t* blk = P.wd + (size_t)rb * CPB6 * 1024;
#pragma unroll
                for (int i = 0; i < CW6; ++i) {
                    const int c = wave * CW6 + i;
                    wv[i] = ((const uint4*)(blk + (size_t)c * 1024))[lane];
                    sbv[i] = load_sb<FMT>(P.wd_sb, rb * 16 + r16, FF, c);
                }
                if (!wait_fan(S, sync, C_GU, (round + 1) * NWG / 16)) return;
                stage_vec<FMT>(S, a.h, FF, nullptr);
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < CW6; ++i) acc += chunk_mac<FMT>(S, wv[i], sbv[i], wave * CW6 + i, lane);
                const float y = reduce_waves(S, acc);
                if (wave == 0 && lane < 16) {
                    float* xo = a.x + rb * 16 + lane;
                    stf(xo, ldf(xo) + y);
                }
                arrive(sync, C_DOWN + (w % 16));
            }
        }

        // ---------------- lm_head + argmax partials ---------------------------------------
        {
            const int tid = my_tid(), lane = tid % 64, wave = tid / 64, r16 = lane % 16;
            const unsigned round = (unsigned)((step + 1) * L);
            constexpr int NRB = VOCAB / 16;
            uint4 wv[CW2];
            uint2 sbv[CW2];
            int rb = w;
            auto load_block = [&](int b) {
                const uint8_t* blk = a.E + (size_t)b * CPB2 * 1024;
#pragma unroll
                for (int i = 0; i < CW2; ++i) {
                    const int c = wave * CW2 + i;
                    wv[i] = ((const uint4*)(blk + (size_t)c * 1024))[lane];
                    sbv[i] = load_sb<FMT>(a.Esb, b * 16 + r16, H, c);
                }
            };
            load_block(rb);
            if (!wait_fan(S, sync, C_DOWN, round * (NWG / 2) / 16)) return;
            stage_vec<FMT>(S, a.x, H, a.final_norm);
            float best = -__builtin_inff();
            int besti = 0x7fffffff;
            for (; rb < NRB; rb += NWG) {
                uint4 cur[CW2];
                uint2 csb[CW2];
#pragma unroll
                for (int i = 0; i < CW2; ++i) {
                    cur[i] = wv[i];
                    csb[i] = sbv[i];
                }
                if (rb + NWG < NRB) load_block(rb + NWG);  // next block in flight while computing
                float acc = 0.f;
#pragma unroll
                for (int i = 0; i < CW2; ++i) acc += chunk_mac<FMT>(S, cur[i], csb[i], wave * CW2 + i, lane);
                const float y = reduce_waves(S, acc);
                if (wave == 0 && lane < 16) argmax_merge(best, besti, y, rb * 16 + lane);
            }
            if (wave == 0) {
                wave_argmax(best, besti);  // lanes >= 16 hold (-inf, INT_MAX)
                if (lane == 0) {
                    stf(a.pval + w, best);
                    sti(a.pidx + w, besti);
                }
            }
            const unsigned old = arrive(sync, C_LM);
            if (tid == 0) S.flag = (old == (unsigned)((step + 1) * NWG - 1));
            __syncthreads();
            if (S.flag) {  // last workgroup: greedy commit (Shaders.swift:1501-1571)
                if (wave == 0) {
                    float bv = -__builtin_inff();
                    int bi = 0x7fffffff;
                    for (int i = lane; i < NWG; i += 64) argmax_merge(bv, bi, ldf(a.pval + i), ldi(a.pidx + i));
                    wave_argmax(bv, bi);
                    if (lane == 0) {
                        State* st = a.st;
                        int tok = bi;
                        const bool bad = tok < 0 || tok >= VOCAB;  // no finite logit (NaN model)
                        if (bad) tok = 0;
                        const int stp = ldi(&st->step);
                        int dn = 0;
                        if (stp >= ldi(&st->maxsteps)) {
                            dn = 1;
                            S.misc[8] = -1.f;
                        } else {
                            a.out_tokens[stp] = tok;
                            const int nstep = stp + 1;
                            const int npos = pos + 1;
                            sti(&st->pos, npos);
                            sti(&st->step, nstep);
                            sti(&st->vis_offset, -1);
                            sti(&st->n, 1);
                            dn = (bad || tok == ldi(&st->eos0) || tok == ldi(&st->eos1) ||
                                  nstep >= ldi(&st->maxsteps) || npos + 2 > ldi(&st->maxctx));
                            S.misc[8] = dn ? -1.f : (float)tok;
                        }
                        if (dn) sti(&st->done, 1);
                    }
                }
                __syncthreads();
                const float t = S.misc[8];
                if (t >= 0.f) {
                    const int tok = (int)t;
                    for (int i = tid; i < H; i += THREADS) stf(a.x + i, dequant_tiled(FMT, a.E, a.Esb, (size_t)tok, i, H));
                }
                arrive(sync, C_COMMIT);
            }
        }
    }
}

}  // namespace pk

hipError_t launch_persistent(int fmt, const PersistArgs& a, hipStream_t s) {
    void* args[] = {(void*)&a};
    if (fmt == FMT_Q4)
        return hipLaunchCooperativeKernel((const void*)pk::decode_kernel<FMT_Q4>, dim3(pk::NWG), dim3(pk::THREADS), args, 0, s);
    if (fmt == FMT_Q8)
        return hipLaunchCooperativeKernel((const void*)pk::decode_kernel<FMT_Q8>, dim3(pk::NWG), dim3(pk::THREADS), args, 0, s);
    return hipErrorInvalidValue;
}

size_t persistent_sync_bytes() { return (size_t)pk::C_SLOTS * 64 * sizeof(unsigned); }
int persistent_error_slot() { return pk::C_ERR * 64; }

}  // namespace icua
