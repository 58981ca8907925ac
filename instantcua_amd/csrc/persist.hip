// Persistent decode kernel: whole greedy decode steps (28 layers + lm_head + commit) in one
// cooperative launch, gfx950.  Same arithmetic and weight tiles as gemv.hip / attention.hip /
// misc.hip; the difference is the schedule.
//
// Why.  As separate kernels a decode step is ~170 dependent launches whose fixed latency
// (launch, cold weight fetch, prologue, drain: 5-10 us each) dominates the ~180 us the step's
// bytes need at 8 TB/s.  Here every workgroup stays resident and, before it waits for a stage's
// inputs, already has the loads of its slice of that stage's weights (and K/V rows) in flight.
//
// Grid.  One 512-thread workgroup per CU (256).  Static work split per layer:
//   QKV   256 row blocks of the fused q|k|v rows (Convert.swift:185-188), block w
//   attn  KV group g = w % 8, split s = w / 8: the pos + 1 cache rows of the group (rows < pos and
//         the new row) are spread evenly over the 32 splits; the split holding row pos writes it
//   merge split 31 of group g (workgroup 248 + g, which has no O / down work) merges the 32
//         partials of the group
//   O     128 row blocks, workgroups 0..127
//   GU    768 row blocks (8 gate + 8 up rows each), blocks 3w .. 3w + 2
//   down  128 row blocks (K = 6144), workgroups 0..127
// then lm_head over 9496 row blocks (w, w + 256, ...) with a per-workgroup argmax, and the greedy
// commit (Shaders.swift:1501-1571), which every workgroup evaluates redundantly from the 256
// argmax partials; workgroup 0 alone writes the control block and the token list.
//
// Data exchange.  Every value that crosses workgroups travels as a 64-bit packet (fp32 value,
// 32-bit round tag) written with one device-scope store and read with device-scope loads
// (global_store/load_dwordx2 ... sc1: coherent across the XCDs' L2s without cache flushes).  A
// consumer polls the packets it needs until each carries the tag of the round it expects, so the
// data is its own flag: no fences, counters or store acknowledgements on the critical path.
// A buffer is rewritten only after every consumer of its previous round has read it: each
// producer first consumes outputs that, through the stage chain, every such consumer produced
// after its read.  The packet area is zeroed before each launch and tags start at 1, so a tag
// never matches stale data.  The one value read with plain loads across workgroups is the new
// K/V cache row: it is stored device-scope, acknowledged before the writer's next packet, first
// read a step later, and rows >= pos are never loaded early (a line cached early would go
// stale).  Every poll is bounded: a timeout raises an error flag that makes all workgroups
// leave, and the host reports it.
#include "icua_device.h"
#include "icua_kernels.h"
#include "icua_persist.h"

namespace icua {
namespace pk {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int THREADS = 512, WAVES = 8;
constexpr int NWG = PERSIST_WGS;         // 256
constexpr int ATT_SPLITS = NWG / NKV;    // 32
constexpr int SPIN_LIMIT = 2000000;      // polls (>= ~1 us each) before a wait gives up
constexpr int PART = HD + 2;             // partial of one head: o[128], m, l
constexpr int ATT_SPQ = 8;               // cache slots per quarter-wave per block
constexpr int ATT_BLOCK = 32 * ATT_SPQ;  // 256 slots per block
constexpr int MERGER0 = NWG - NKV;       // workgroup 248 + g merges group g (its split 31)

// Packet area (64-bit packets), zeroed before every launch.
constexpr int XP = 0;                 // residual x [H]
constexpr int QKVP = XP + H;          // fused q|k|v [QKV]
constexpr int ATTNP = QKVP + QKV;     // merged attention [H]
constexpr int HP = ATTNP + H;         // SwiGLU activations [FF]
constexpr int LMP = HP + FF;          // argmax partials [NWG][2] (value, index)
constexpr int PARTP = LMP + 2 * NWG;  // attention partials [NKV][32][2][PART]
constexpr int PACKETS = PARTP + NKV * ATT_SPLITS * 2 * PART;
constexpr int ERRW = PACKETS * 2;     // error flag (32-bit word index)
static_assert(MERGER0 % NKV == 0, "merger of group g must be split 31 of group g");

// threadIdx.x behind an empty asm: per-lane address math derived from it is recomputed where it
// is used instead of being hoisted out of the step / layer loops and held live (which spills).
__device__ __forceinline__ int my_tid() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

__device__ __forceinline__ uint64_t ld64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t pack(float v, unsigned tag) { return (uint64_t)as_u32(v) | ((uint64_t)tag << 32); }
__device__ __forceinline__ uint64_t pack_i(int v, unsigned tag) { return (uint64_t)(uint32_t)v | ((uint64_t)tag << 32); }
__device__ __forceinline__ unsigned tag_of(uint64_t p) { return (unsigned)(p >> 32); }
__device__ __forceinline__ float val_of(uint64_t p) { return as_f32((uint32_t)p); }

__device__ __forceinline__ unsigned load_err(const unsigned* e) {
    return __hip_atomic_load(e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void raise_err(unsigned* e) {
    __hip_atomic_store(e, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Polls packets p[i] = src[off(i)] (i < N; off(i) < 0: unused) until each carries `tag`.  Returns
// false on timeout (after raising the error flag) or when another workgroup raised it.
template <int N, typename Off>
__device__ __forceinline__ bool poll(const uint64_t* src, Off off, unsigned tag, uint64_t (&p)[N], unsigned* err) {
    const uint64_t filler = (uint64_t)tag << 32;
#pragma unroll
    for (int i = 0; i < N; ++i) {
        const int o = off(i);
        p[i] = o >= 0 ? ld64(src + o) : filler;
    }
    for (int it = 0;; ++it) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < N; ++i) ok &= tag_of(p[i]) == tag;
        if (ok) return true;
        if (it >= SPIN_LIMIT) {
            raise_err(err);
            return false;
        }
        if ((it & 63) == 63 && load_err(err)) return false;
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int i = 0; i < N; ++i)
            if (tag_of(p[i]) != tag) p[i] = ld64(src + off(i));
    }
}

// Waits until sentinel packet src[sent(t)] carries `tag` for every thread t < nsent (one packet
// per producer store instruction), so that the bulk of a vector is read once instead of being
// polled: polling whole vectors from every workgroup floods the fabric.  Whole-workgroup call.
template <typename Sent>
__device__ __forceinline__ bool wait_sentinels(const uint64_t* src, int nsent, Sent sent, unsigned tag,
                                               unsigned* err) {
    const int tid = my_tid();
    bool ok = true;
    if (tid < nsent) {
        const uint64_t* q = src + sent(tid);
        uint64_t p = ld64(q);
        for (int it = 0; tag_of(p) != tag; ++it) {
            if (it >= SPIN_LIMIT) {
                raise_err(err);
                ok = false;
                break;
            }
            if ((it & 63) == 63 && load_err(err)) {
                ok = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
            p = ld64(q);
        }
    }
    return !__syncthreads_or(!ok);
}

// Producers of the packet vectors and their sentinels.  A sentinel only decides when to read
// the vector; the tag check of every packet read afterwards is what guarantees the data.
enum Src { SRC_X = 0, SRC_ATTN = 1, SRC_H = 2 };
// x: workgroup p < 128 stores packets 16p .. 16p + 15 with one instruction.
// attn: merger g stores head (2g + hh) elements d with waves 0-3 (64 elements each).
// h: workgroup p < 256 stores 8 packets per block 3p + j, j = 0, 1, 2; its last block is polled.
template <int SRC>
__device__ __forceinline__ int sentinel_count() {
    return SRC == SRC_X ? H / 16 : SRC == SRC_ATTN ? 4 * NKV : NWG;
}
template <int SRC>
__device__ __forceinline__ int sentinel_of(int t) {
    if constexpr (SRC == SRC_X) return 16 * t;
    else if constexpr (SRC == SRC_ATTN) return (t / 4) * 2 * HD + (t % 4) * 64;
    else return 8 * (3 * t + 2);
}

struct Shared {
    uint8_t A[96 * 1024];  // activation operands (1 KiB per q4 group / 512 B per q8 group, K <= 6144)
    float fx[192 * 2];     // per-group (2^(e-21), sum X * 2^(e-21))
    float red[WAVES * 64];
    float emb[H];          // embedding of the token being decoded
    float xown[16];        // residual rows of this workgroup's O / down block (workgroups < 128)
    float qs[2][HD];       // attention: two query heads
    float ktail[HD], vtail[HD];
    float sc[2][ATT_BLOCK];
    float ored[WAVES][2][HD];
    float misc[64];
    int imisc[64];
    uint64_t tmark[2];  // profiling builds: sentinel / packet times of the last vector staging
};

// ------------------------------------------------------------------------------------------
// Activation staging for one token: 8 consecutive activations per unit, units u = tid and
// tid + 512 (K / 8 units) -> optional RMSNorm -> 22-bit slices -> A operands.  Rows 0, 1, 2 of each
// group tile hold the hi, mid, lo slices; rows 3..15 stay zero (zeroed at kernel start).

template <int FMT>
__device__ __forceinline__ void stage_vals(Shared& S, float (&v)[2][8], int K, const float* norm_w) {
    constexpr int G = (FMT == FMT_Q4) ? 64 : 32;
    constexpr int TILE = (FMT == FMT_Q4) ? 1024 : 512;
    const int tid = my_tid(), lane = tid % 64, wave = tid / 64;
    const int nunits = K / 8;
    float scale = 1.f;
    if (norm_w) {
        float ss = 0.f;
#pragma unroll
        for (int it = 0; it < 2; ++it)
            if (tid + it * THREADS < nunits)
#pragma unroll
                for (int i = 0; i < 8; ++i) ss += v[it][i] * v[it][i];
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
        int bits = (int)as_u32(amax);  // order of non-negative floats = order of their bits
        bits = max(bits, dpp_i<DPP_XOR1>(bits));
        bits = max(bits, dpp_i<DPP_XOR2>(bits));
        if constexpr (G == 64) bits = max(bits, dpp_i<DPP_HALF_MIRROR>(bits));
        int e = ((bits >> 23) & 0xFF) - 127;
        if (bits == 0) e = -100;  // all-zero group: X = 0 for any exponent
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

// Stages a packet vector of K values (round `tag`).  false (for the whole workgroup) on error.
template <int FMT, int SRC>
__device__ __forceinline__ bool stage_packets(Shared& S, const uint64_t* src, unsigned tag, int K, const float* norm_w,
                              unsigned* err) {
    if (!wait_sentinels(src, sentinel_count<SRC>(), [](int t) { return sentinel_of<SRC>(t); }, tag, err)) return false;
#ifdef ICUA_PERSIST_TRACE
    if (my_tid() == 0) S.tmark[0] = wall_clock64();
#endif
    const int tid = my_tid();
    const int nunits = K / 8;
    uint64_t p[16];
    const bool ok = poll<16>(
        src,
        [&](int i) {
            const int u = tid + (i / 8) * THREADS;
            return u < nunits ? u * 8 + i % 8 : -1;
        },
        tag, p, err);
    if (__syncthreads_or(!ok)) return false;
#ifdef ICUA_PERSIST_TRACE
    if (my_tid() == 0) S.tmark[1] = wall_clock64();
#endif
    float v[2][8];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i / 8][i % 8] = val_of(p[i]);
    stage_vals<FMT>(S, v, K, norm_w);
    return true;
}

// Stages the embedding held in LDS (K = H).
template <int FMT>
__device__ __forceinline__ void stage_emb(Shared& S, const float* norm_w) {
    const int tid = my_tid();
    float v[2][8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        v[0][i] = tid < H / 8 ? S.emb[tid * 8 + i] : 0.f;
        v[1][i] = 0.f;
    }
    stage_vals<FMT>(S, v, H, norm_w);
}

// One 1 KiB chunk of a 16-row block against the staged operands; returns the lane's partial
// (lanes 0-15 hold rows 0-15 of the block).
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

// Scales of chunk c of tiled row `row`: q4 chunk = 128 K (two half2 (scale, bias) of 64-K
// groups), q8 chunk = 64 K (two half scales of 32-K groups).
template <int FMT>
__device__ __forceinline__ uint2 load_sb(const uint8_t* sb, int row, int K, int c) {
    if constexpr (FMT == FMT_Q4)
        return *(const uint2*)(sb + ((size_t)row * (K / 64) + 2 * c) * 4);
    else
        return make_uint2(*(const uint32_t*)(sb + ((size_t)row * (K / 32) + 2 * c) * 2), 0u);
}

// The CW chunks of wave `wave` of 16-row block rb (chunks wave * CW .. wave * CW + CW - 1).
template <int FMT, int CW>
__device__ __forceinline__ void load_block(const uint8_t* w, const uint8_t* sb, int rb, int K, int wave, int lane,
                                           uint4 (&wv)[CW], uint2 (&sbv)[CW]) {
    constexpr int CHK = (FMT == FMT_Q4) ? 128 : 64;
    const int cpb = K / CHK;
    const uint8_t* blk = w + (size_t)rb * cpb * 1024;
#pragma unroll
    for (int i = 0; i < CW; ++i) {
        const int c = wave * CW + i;
        wv[i] = ((const uint4*)(blk + (size_t)c * 1024))[lane];
        sbv[i] = load_sb<FMT>(sb, rb * 16 + lane % 16, K, c);
    }
}

template <int FMT, int CW>
__device__ __forceinline__ float block_mac(const Shared& S, const uint4 (&wv)[CW], const uint2 (&sbv)[CW], int wave,
                                           int lane) {
    float acc = 0.f;
#pragma unroll
    for (int i = 0; i < CW; ++i) acc += chunk_mac<FMT>(S, wv[i], sbv[i], wave * CW + i, lane);
    return acc;
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
// Stage timeline of the last step of a launch (per workgroup, per layer, 32 event slots; steady
// clock), compiled only with -DICUA_PERSIST_TRACE for profiling builds.  Slots 16 + 2k and
// 17 + 2k: sentinels seen and packets read by the k-th vector staging of the layer.
#ifdef ICUA_PERSIST_TRACE
__device__ uint64_t g_trace[NWG][MAX_LAYERS + 1][32];
#define PK_TRACE(layer, ev)                                                                  \
    do {                                                                                     \
        if (step == a.nsteps - 1 && my_tid() == 0) g_trace[w][layer][ev] = wall_clock64(); \
    } while (0)
#define PK_TRACE_MARKS(layer, k)                                           \
    do {                                                                   \
        if (step == a.nsteps - 1 && my_tid() == 0) {                       \
            g_trace[w][layer][16 + 2 * (k)] = S.tmark[0];                  \
            g_trace[w][layer][17 + 2 * (k)] = S.tmark[1];                  \
        }                                                                  \
    } while (0)
#else
#define PK_TRACE(layer, ev) \
    do {                    \
    } while (0)
#define PK_TRACE_MARKS(layer, k) \
    do {                         \
    } while (0)
#endif

template <int FMT>
__global__ __launch_bounds__(THREADS, 1) void decode_kernel(PersistArgs a) {
    constexpr int CHK = (FMT == FMT_Q4) ? 128 : 64;
    constexpr int CW2 = H / CHK / WAVES;   // chunks per wave, K = 2048
    constexpr int CW6 = FF / CHK / WAVES;  // K = 6144
    constexpr int NRB = VOCAB / 16;        // lm_head row blocks
    __shared__ Shared S;
    const int w = blockIdx.x;
    uint64_t* ll = a.ll;
    unsigned* err = (unsigned*)a.ll + ERRW;
    for (int i = my_tid(); i < (int)sizeof(S.A) / 4; i += THREADS) ((uint32_t*)S.A)[i] = 0u;

    // Control block and the embedding of the first token (written before this launch).
    State* st = a.st;
    if (st->done || st->n != 1) return;  // single-row passes only (checked by the host too)
    int pos = st->pos, stp = st->step;
    const int maxsteps = st->maxsteps, eos0 = st->eos0, eos1 = st->eos1, maxctx = st->maxctx;
    for (int i = my_tid(); i < H; i += THREADS) S.emb[i] = a.x[i];
    if (my_tid() < 16 && w < H / 16) S.xown[my_tid()] = a.x[w * 16 + my_tid()];
    __syncthreads();

    const int L = a.nlayers;
    for (int step = 0; step < a.nsteps; ++step) {
        if (pos + 1 > maxctx) break;  // the commit stops earlier; guards the cache row
        for (int l = 0; l < L; ++l) {
            const LayerPtrs& P = a.layers[l];
            const unsigned r = (unsigned)(step * L + l);  // round of this layer

            // Attention geometry of this workgroup (KV group g, split s) and its first block of
            // K/V rows, issued before the QKV stage so that they stream in behind it.  The pos + 1
            // rows of the group (rows < pos and the new row) are spread evenly over the 32 splits;
            // the split holding row pos writes it.  Only rows < pos are loaded from the cache.
            const int g = w % NKV, s = w / NKV;
            const int tot = pos + 1;
            const int chunk = (tot + ATT_SPLITS - 1) / ATT_SPLITS;
            const int j0 = min(s * chunk, tot), j1 = min(j0 + chunk, tot);
            const bool tail = (j0 <= pos) && (pos < j1);
            const int nprior = max(0, min(j1, pos) - j0);
            const int ntot = j1 - j0;
            const uint16_t* kb = a.kv + ((size_t)(l * 2 + 0) * NKV + g) * a.maxctx * HD;
            const uint16_t* vb = a.kv + ((size_t)(l * 2 + 1) * NKV + g) * a.maxctx * HD;
            uint4 kr[ATT_SPQ], vr[ATT_SPQ];
            {
                const int tid = my_tid(), quad = tid / 16, ql = tid % 16;
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
            }

            // ---------------- QKV: row block w ---------------------------------------------
            {
                const int tid = my_tid(), lane = tid % 64, wave = tid / 64;
                PK_TRACE(l, 0);
                uint4 wv[CW2];
                uint2 sbv[CW2];
                load_block<FMT, CW2>(P.wqkv, P.wqkv_sb, w, H, wave, lane, wv, sbv);
                if (l == 0) {
                    stage_emb<FMT>(S, P.attn_norm);
                } else if (!stage_packets<FMT, SRC_X>(S, ll + XP, 2 * r, H, P.attn_norm, err)) {
                    return;
                }
                PK_TRACE(l, 1);
                if (l > 0) PK_TRACE_MARKS(l, 0);
                const float y = reduce_waves(S, block_mac<FMT, CW2>(S, wv, sbv, wave, lane));
                if (wave == 0 && lane < 16) st64(ll + QKVP + w * 16 + lane, pack(y, r + 1));
                PK_TRACE(l, 2);
            }

            // ---------------- attention: group g, split s ----------------------------------
            {
                const int tid = my_tid(), lane = tid % 64, wave = tid / 64;
                const int quad = tid / 16, ql = tid % 16;  // 32 quarter-waves, 8 dims per lane
                // Sentinels: the 32 QKV blocks of group g (q heads 2g, 2g+1: blocks 16g..16g+15;
                // k: 128 + 8g..; v: 192 + 8g..), lane 0 of each.
                if (!wait_sentinels(
                        ll + QKVP, 32,
                        [&](int t) {
                            const int b = t < 16 ? 16 * g + t : t < 24 ? 128 + 8 * g + (t - 16) : 192 + 8 * g + (t - 24);
                            return 16 * b;
                        },
                        r + 1, err))
                    return;
                // Queries of heads 2g, 2g+1 (waves 0, 1); the tail split's wave 2 also takes the
                // new K and V rows of the group.
                {
                    const bool needs = wave < 2 || (wave == 2 && tail);
                    const int qoff = (2 * g + wave) * HD + lane;
                    const int koff = H + g * HD + lane, voff = H + NKV * HD + g * HD + lane;
                    uint64_t p[4];
                    bool ok = true;
                    if (needs)
                        ok = poll<4>(
                            ll + QKVP,
                            [&](int i) {
                                if (wave < 2) return i < 2 ? qoff + 64 * i : -1;
                                return i < 2 ? koff + 64 * i : voff + 64 * (i - 2);
                            },
                            r + 1, p, err);
                    if (__syncthreads_or(!ok)) return;
                    PK_TRACE(l, 3);
                    const float* rope = a.rope + (size_t)pos * 128;
                    if (wave < 2) {
                        float x0 = val_of(p[0]), x1 = val_of(p[1]);
                        norm_rope(x0, x1, P.q_norm, rope, lane);
                        const float qscale = 1.0f / sqrtf((float)HD);
                        S.qs[wave][lane] = x0 * qscale;
                        S.qs[wave][lane + 64] = x1 * qscale;
                    } else if (needs) {
                        float k0 = val_of(p[0]), k1 = val_of(p[1]);
                        norm_rope(k0, k1, P.k_norm, rope, lane);
                        S.ktail[lane] = h2f(f2h(k0));
                        S.ktail[lane + 64] = h2f(f2h(k1));
                        S.vtail[lane] = h2f(f2h(val_of(p[2])));
                        S.vtail[lane + 64] = h2f(f2h(val_of(p[3])));
                    }
                }
                __syncthreads();
                if (tail && tid < 128) {
                    // The new cache row (fp16), device-scope stores.
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
                        if (quad + 32 * i == pnew) {
                            uint32_t kk[4], vv[4];
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                kk[j] = (uint32_t)f2h(S.ktail[8 * ql + 2 * j]) |
                                        ((uint32_t)f2h(S.ktail[8 * ql + 2 * j + 1]) << 16);
                                vv[j] = (uint32_t)f2h(S.vtail[8 * ql + 2 * j]) |
                                        ((uint32_t)f2h(S.vtail[8 * ql + 2 * j + 1]) << 16);
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
                    // Block softmax statistics: waves 0 and 1, one head each.
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
                            S.misc[wave] = mn;
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
                // The new cache row is acknowledged before this workgroup's next packet.
                __builtin_amdgcn_s_waitcnt(0);
                __syncthreads();
                uint64_t* part = ll + PARTP + (size_t)(g * ATT_SPLITS + s) * 2 * PART;
                if (tid < 2 * HD) {
                    const int hh = tid / HD, d = tid % HD;
                    float acc = 0.f;
                    for (int ww = 0; ww < WAVES; ++ww) acc += S.ored[ww][hh][d];
                    st64(part + hh * PART + d, pack(acc, r + 1));
                    if (d == 0) {
                        st64(part + hh * PART + HD, pack(m_run[hh], r + 1));
                        st64(part + hh * PART + HD + 1, pack(l_run[hh], r + 1));
                    }
                }
                PK_TRACE(l, 4);
            }

            // ---------------- merge of group g: workgroups 248..255 ------------------------
            // Thread t: half = t / 256 (splits 16 half .. 16 half + 15), head hh, element d; the
            // threads with d < 16 also fetch (m, l) of split 16 half + d.  Each half is merged with
            // its own maximum, then the two halves are combined.
            if (w >= MERGER0) {
                const int tid = my_tid();
                const int half = tid / 256, hh = (tid / HD) & 1, d = tid % HD;
                const uint64_t* gp = ll + PARTP + (size_t)g * ATT_SPLITS * 2 * PART;
                // Sentinels: per split and head, the m packet and the o packet stored by the second
                // wave of that head (element 64).
                if (!wait_sentinels(
                        gp, 4 * ATT_SPLITS,
                        [](int t) { return ((t / 4) * 2 + (t % 4) / 2) * PART + ((t % 2) ? 64 : HD); }, r + 1,
                        err))
                    return;
                uint64_t p[18];
                const bool ok = poll<18>(
                    gp,
                    [&](int i) {
                        if (i < 16) return ((half * 16 + i) * 2 + hh) * PART + d;
                        return d < 16 ? ((half * 16 + d) * 2 + hh) * PART + HD + (i - 16) : -1;
                    },
                    r + 1, p, err);
                if (__syncthreads_or(!ok)) return;
                float* ml = &S.sc[0][0];  // [half][hh][16][2]
                if (d < 16) {
                    ml[((half * 2 + hh) * 16 + d) * 2] = val_of(p[16]);
                    ml[((half * 2 + hh) * 16 + d) * 2 + 1] = val_of(p[17]);
                }
                __syncthreads();
                const float* mlh = ml + (half * 2 + hh) * 32;
                float mx = -__builtin_inff();
#pragma unroll
                for (int j = 0; j < 16; ++j) mx = fmaxf(mx, mlh[2 * j]);
                float Lh = 0.f, Oh = 0.f;
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const float m = mlh[2 * j];
                    const float wgt = (m == -__builtin_inff()) ? 0.f : expf(m - mx);
                    Lh = fmaf(wgt, mlh[2 * j + 1], Lh);
                    Oh = fmaf(wgt, val_of(p[j]), Oh);
                }
                S.ored[half][hh][d] = Oh;
                if (d == 0) {
                    S.misc[(half * 2 + hh) * 2] = mx;
                    S.misc[(half * 2 + hh) * 2 + 1] = Lh;
                }
                __syncthreads();
                if (half == 0) {
                    const float m0 = S.misc[hh * 2], l0 = S.misc[hh * 2 + 1];
                    const float m1 = S.misc[(2 + hh) * 2], l1 = S.misc[(2 + hh) * 2 + 1];
                    const float M = fmaxf(m0, m1);  // finite: the split holding row pos is never empty
                    const float w0 = (m0 == -__builtin_inff()) ? 0.f : expf(m0 - M);
                    const float w1 = (m1 == -__builtin_inff()) ? 0.f : expf(m1 - M);
                    const float out = (w0 * Oh + w1 * S.ored[1][hh][d]) / (w0 * l0 + w1 * l1);
                    st64(ll + ATTNP + (2 * g + hh) * HD + d, pack(out, r + 1));
                }
                PK_TRACE(l, 5);
            }

            // ---------------- O projection + residual: workgroups 0..127 -------------------
            if (w < H / 16) {
                const int tid = my_tid(), lane = tid % 64, wave = tid / 64;
                uint4 wv[CW2];
                uint2 sbv[CW2];
                load_block<FMT, CW2>(P.wo, P.wo_sb, w, H, wave, lane, wv, sbv);
                if (!stage_packets<FMT, SRC_ATTN>(S, ll + ATTNP, r + 1, H, nullptr, err)) return;
                PK_TRACE(l, 6);
                PK_TRACE_MARKS(l, 1);
                const float y = reduce_waves(S, block_mac<FMT, CW2>(S, wv, sbv, wave, lane));
                if (wave == 0 && lane < 16) {
                    const float xn = S.xown[lane] + y;
                    S.xown[lane] = xn;
                    st64(ll + XP + w * 16 + lane, pack(xn, 2 * r + 1));
                }
                PK_TRACE(l, 7);
            }

            // ---------------- RMSNorm + gate|up + SwiGLU: blocks 3w .. 3w + 2 --------------
            {
                const int tid = my_tid(), lane = tid % 64, wave = tid / 64;
                uint4 wv[3][CW2];
                uint2 sbv[3][CW2];
#pragma unroll
                for (int j = 0; j < 3; ++j) load_block<FMT, CW2>(P.wgu, P.wgu_sb, 3 * w + j, H, wave, lane, wv[j], sbv[j]);
                if (!stage_packets<FMT, SRC_X>(S, ll + XP, 2 * r + 1, H, P.mlp_norm, err)) return;
                PK_TRACE(l, 8);
                PK_TRACE_MARKS(l, 2);
#pragma unroll
                for (int j = 0; j < 3; ++j) {
                    const float y = reduce_waves(S, block_mac<FMT, CW2>(S, wv[j], sbv[j], wave, lane));
                    if (wave == 0) {
                        // Block 3w + j: gate units 8 (3w + j) + 0..7 in lanes 0-7, their up rows in 8-15.
                        const float up = __shfl_xor(y, 8);
                        if (lane < 8)
                            st64(ll + HP + (3 * w + j) * 8 + lane, pack((y / (1.f + expf(-y))) * up, r + 1));
                    }
                }
                PK_TRACE(l, 9);
            }

            // ---------------- down + residual: workgroups 0..127 ---------------------------
            if (w < H / 16) {
                const int tid = my_tid(), lane = tid % 64, wave = tid / 64;
                uint4 wv[CW6];
                uint2 sbv[CW6];
                load_block<FMT, CW6>(P.wd, P.wd_sb, w, FF, wave, lane, wv, sbv);
                if (!stage_packets<FMT, SRC_H>(S, ll + HP, r + 1, FF, nullptr, err)) return;
                PK_TRACE(l, 10);
                PK_TRACE_MARKS(l, 3);
                const float y = reduce_waves(S, block_mac<FMT, CW6>(S, wv, sbv, wave, lane));
                if (wave == 0 && lane < 16) {
                    const float xn = S.xown[lane] + y;
                    S.xown[lane] = xn;
                    st64(ll + XP + w * 16 + lane, pack(xn, 2 * r + 2));
                }
                PK_TRACE(l, 11);
            }
        }

        // ---------------- final RMSNorm + lm_head + per-workgroup argmax ---------------------
        {
            const int tid = my_tid(), lane = tid % 64, wave = tid / 64;
            const unsigned r_last = (unsigned)(step * L + L - 1);
            PK_TRACE(L, 0);
            uint4 wv0[CW2], wv1[CW2];
            uint2 sb0[CW2], sb1[CW2];
            load_block<FMT, CW2>(a.E, a.Esb, w, H, wave, lane, wv0, sb0);
            load_block<FMT, CW2>(a.E, a.Esb, w + NWG, H, wave, lane, wv1, sb1);
            if (!stage_packets<FMT, SRC_X>(S, ll + XP, 2 * r_last + 2, H, a.final_norm, err)) return;
            PK_TRACE(L, 1);
            PK_TRACE_MARKS(L, 0);
            float best = -__builtin_inff();
            int besti = 0x7fffffff;
            // Two blocks in flight (static ping-pong buffers): a block computes while the block
            // two ahead loads.  Blocks w + k * 256; every workgroup has at least 37.
            for (int rb = w; rb < NRB; rb += 2 * NWG) {
                {
                    const float y = reduce_waves(S, block_mac<FMT, CW2>(S, wv0, sb0, wave, lane));
                    if (wave == 0 && lane < 16) argmax_merge(best, besti, y, rb * 16 + lane);
                    if (rb + 2 * NWG < NRB) load_block<FMT, CW2>(a.E, a.Esb, rb + 2 * NWG, H, wave, lane, wv0, sb0);
                }
                if (rb + NWG < NRB) {
                    const float y = reduce_waves(S, block_mac<FMT, CW2>(S, wv1, sb1, wave, lane));
                    if (wave == 0 && lane < 16) argmax_merge(best, besti, y, (rb + NWG) * 16 + lane);
                    if (rb + 3 * NWG < NRB) load_block<FMT, CW2>(a.E, a.Esb, rb + 3 * NWG, H, wave, lane, wv1, sb1);
                }
            }
            if (wave == 0) {
                wave_argmax(best, besti);  // lanes >= 16 hold (-inf, INT_MAX)
                if (lane == 0) {
                    st64(ll + LMP + 2 * w, pack(best, (unsigned)step + 1));
                    st64(ll + LMP + 2 * w + 1, pack_i(besti, (unsigned)step + 1));
                }
            }
            PK_TRACE(L, 2);
        }

        // ---------------- greedy commit, evaluated by every workgroup ------------------------
        {
            const int tid = my_tid(), lane = tid % 64, wave = tid / 64;
            uint64_t p[2];
            const bool ok = poll<2>(
                ll + LMP, [&](int i) { return tid < NWG ? 2 * tid + i : -1; }, (unsigned)step + 1, p, err);
            if (__syncthreads_or(!ok)) return;
            float bv = tid < NWG ? val_of(p[0]) : -__builtin_inff();
            int bi = tid < NWG ? (int)(uint32_t)p[1] : 0x7fffffff;
            wave_argmax(bv, bi);
            if (lane == 0) {
                S.misc[wave] = bv;
                S.imisc[wave] = bi;
            }
            __syncthreads();
            float b2 = S.misc[0];
            int tok = S.imisc[0];
            for (int ww = 1; ww < WAVES; ++ww) argmax_merge(b2, tok, S.misc[ww], S.imisc[ww]);
            bool stop;
            if (stp >= maxsteps) {  // nothing may be written past out_tokens[maxsteps - 1]
                stop = true;
            } else {
                const bool bad = tok < 0 || tok >= VOCAB;  // no finite logit (NaN model): stop on token 0
                if (bad) tok = 0;
                if (w == 0 && tid == 0) a.out_tokens[stp] = tok;
                stp += 1;
                pos += 1;
                stop = bad || tok == eos0 || tok == eos1 || stp >= maxsteps || pos + 2 > maxctx;
            }
            if (w == 0 && tid == 0) {
                st->pos = pos;
                st->step = stp;
                st->n = 1;
                st->vis_offset = -1;
                st->logits_rows = 0;
                if (stop) st->done = 1;
            }
            PK_TRACE(L, 3);
            if (stop) break;
            // Next token's embedding (Shaders.swift:464-476), in every workgroup.
            __syncthreads();  // every thread has read S.misc / S.imisc
            for (int i = tid; i < H; i += THREADS) S.emb[i] = dequant_tiled(FMT, a.E, a.Esb, (size_t)tok, i, H);
            __syncthreads();
            if (tid < 16 && w < H / 16) S.xown[tid] = S.emb[w * 16 + tid];
            if (w == 0 && step == a.nsteps - 1)
                for (int i = tid; i < H; i += THREADS) a.x[i] = S.emb[i];  // residual row for the host
        }
    }
}

}  // namespace pk

hipError_t launch_persistent(int fmt, const PersistArgs& a, hipStream_t s) {
    void* args[] = {(void*)&a};
    if (fmt == FMT_Q4)
        return hipLaunchCooperativeKernel((const void*)pk::decode_kernel<FMT_Q4>, dim3(pk::NWG), dim3(pk::THREADS),
                                          args, 0, s);
    if (fmt == FMT_Q8)
        return hipLaunchCooperativeKernel((const void*)pk::decode_kernel<FMT_Q8>, dim3(pk::NWG), dim3(pk::THREADS),
                                          args, 0, s);
    return hipErrorInvalidValue;
}

#ifdef ICUA_PERSIST_TRACE
extern "C" int icua_debug_persist_trace(uint64_t* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(pk::g_trace), sizeof(pk::g_trace)) == hipSuccess ? 0 : -1;
}
#endif

size_t persistent_sync_bytes() { return ((size_t)pk::PACKETS + 32) * sizeof(uint64_t); }
int persistent_error_slot() { return pk::ERRW; }

}  // namespace icua
