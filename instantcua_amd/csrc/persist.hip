// Persistent decode kernel: whole greedy decode steps (28 layers + lm_head + commit) in one
// cooperative launch, gfx950.  Same arithmetic and weight tiles as gemv.hip / attention.hip /
// misc.hip; the difference is the schedule.
//
// Why.  As separate kernels a decode step is ~170 dependent launches whose fixed latency
// (launch, cold weight fetch, prologue, drain: 5-10 us each) dominates the ~180 us the step's
// bytes need at 8 TB/s.  Here every workgroup stays resident; weights, K/V rows and norm vectors
// are requested one or two stages before they are needed, so HBM streams while the workgroups
// wait for each other.
//
// Grid.  One 512-thread workgroup per CU (256).  Static work split per layer:
//   QKV   256 row blocks of the fused q|k|v rows (Convert.swift:185-188): blocks w - 128 and w
//         in workgroups 128..255
//   attn  KV group g = w % 8, split s = w / 8: the pos + 1 cache rows of the group (rows < pos and
//         the new row) are spread evenly over the 32 splits; the split holding row pos writes it
//   merge splits 28..31 of group g (workgroups 224..255, no O work) merge the 32 partials of
//         the group, a quarter of the group's output each
//   O     128 row blocks, workgroups 0..127
//   GU    768 row blocks (8 gate + 8 up rows each), blocks 3w .. 3w + 2
//   down  128 row blocks split along K: workgroup w takes K half w / 128 of block w % 128
// then lm_head over 9496 row blocks (w, w + 256, ...) with a per-workgroup argmax, and the greedy
// commit (Shaders.swift:1501-1571), which every workgroup evaluates redundantly from the 256
// argmax partials; workgroup 0 alone writes the control block and the token list.
//
// Roles inside a workgroup.  Waves 0-3 ("math") hold the weight tiles and K/V rows in registers
// and run the matrix-core GEMV and the attention arithmetic (VALU-bound: spreading it over all
// eight waves only shares the same four SIMDs).  Waves 4-7 ("exchange") wait for the inputs of
// each stage; all eight waves stage them into LDS as matrix-core operands.  The
// split exists because a wave's vector-memory counter retires in issue order and a CU's memory
// pipeline is shared: a poll issued behind outstanding weight loads could not be seen before
// those loads land.  So bulk loads are issued where no poll follows on the CU: the next layer's
// QKV blocks while h is awaited, K/V rows after the QKV publish (workgroups 128..255), the down
// half-block into LDS after the O publish.
//
// Data exchange.  Every value that crosses workgroups travels in a 64-bit packet of two values
// written with one device-scope store and read with device-scope loads (global_store/load_dwordx2
// ... sc1: coherent across the XCDs' L2s without cache flushes).  The low word is value a rounded
// to a 19-bit mantissa whose low 4 bits carry the tag of the round (1..15), the high word value b
// exact.  The exchange waves read consecutive packets in consecutive lanes and poll until each
// carries the tag of the round they expect, so the data is its own flag.  The packet area is
// uncached device memory (the engine's pool; its all-to-all exchanges measure faster there).  A
// buffer is rewritten only after every consumer of its previous round has read it: each producer
// first consumes outputs that, through the stage chain, every such consumer produced after its
// read.  The packet area is zeroed before each launch and tags start at 1, so a tag never
// matches stale data.  The
// one value read with plain loads across workgroups is the new K/V cache row: it is stored
// device-scope, acknowledged before the writer's next packet, first read a step later, and rows
// >= pos are never loaded early (a line cached early would go stale).  Every poll is bounded: a
// timeout raises an error flag that makes all workgroups leave, and the host reports it.
#include "icua_device.h"
#include "icua_kernels.h"
#include "icua_persist.h"

namespace icua {
namespace pk {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));

constexpr int THREADS = 512, WAVES = 8;
constexpr int MW = 4;                     // math waves 0..3
constexpr int MT = MW * 64;               // math threads
constexpr int CT = THREADS - MT;          // exchange threads (waves 4..7)
constexpr int NWG = PERSIST_WGS;          // 256
constexpr int ATT_SPLITS = NWG / NKV;     // 32
constexpr int SPIN_LIMIT = 2000000;       // polls (>= ~1 us each) before a wait gives up
constexpr int PART2 = HD / 2 + 1;         // packets of one head's partial: o pairs, (l, m)
constexpr int ATT_QW = MT / 16;           // 16 quarter-waves of math threads
constexpr int ATT_SPQ = 9;                // cache slots per quarter-wave per block (P.V)
constexpr int ATT_BLOCK = ATT_QW * ATT_SPQ;  // 144 slots per block
constexpr int ATT_NT = (ATT_SPQ + 3) / 4;    // score tiles of 16 slots per math wave per block
constexpr int ATT_PAD = 192;              // merge weights row length
constexpr int MERGE_PARTS = 4;            // workgroups merging one group's partials
constexpr int MERGER0 = NWG - NKV * MERGE_PARTS;  // workgroups 224..255: splits 28..31 of each group
static_assert(MERGER0 >= H / 16, "mergers must not have O / down work");
static_assert(MERGER0 % NKV == 0, "mergers of group g are splits 28..31 of group g");
// Down is split along K: workgroup w < 128 multiplies K 0..3071 of row block w, workgroup
// w + 128 K 3072..6143 of the same rows.
constexpr int FFH = FF / 2;
static_assert(FFH / 128 / MW == 6 && FFH / 64 / MW == 12, "q4 down half: 6 chunks and 12 scale groups per math wave");

// Packet area (64-bit packets of two values, elements 2k and 2k + 1 of a vector in packet k),
// zeroed before every launch.  The residual after a layer is x = XP + XDP: XP carries the lower
// half's sum added to the residual, XDP the upper half's sum.  A pass of NR rows keeps NR copies
// of each vector area, row after row (row t of a vector of n packets at area + t n).
template <int NR>
struct Pk {
    static constexpr int XP = 0;                        // residual x [NR][H / 2] (after O: complete; after down: + lower half)
    static constexpr int XDP = XP + NR * H / 2;         // upper-half down sums [NR][H / 2]
    static constexpr int QKVP = XDP + NR * H / 2;       // fused q|k|v [NR][QKV / 2]
    static constexpr int ATTNP = QKVP + NR * QKV / 2;   // merged attention [NR][H / 2]
    static constexpr int HP = ATTNP + NR * H / 2;       // SwiGLU activations [NR][FF / 2]
    static constexpr int LMP = HP + NR * FF / 2;        // argmax partials [NWG] (index, value)
    static constexpr int PARTP = LMP + NWG;             // attention partials [NKV][32][NR][2][PART2]
    static constexpr int GROUP_PARTS = ATT_SPLITS * NR * 2 * PART2;  // packets of one group's partials
    static constexpr int PACKETS = PARTP + NKV * GROUP_PARTS;
};
constexpr int ERRW = Pk<2>::PACKETS * 2;  // error flag (32-bit word index), past either layout
// The single-row layout's areas.
constexpr int XP = Pk<1>::XP, XDP = Pk<1>::XDP, QKVP = Pk<1>::QKVP, ATTNP = Pk<1>::ATTNP, HP = Pk<1>::HP,
              LMP = Pk<1>::LMP, PARTP = Pk<1>::PARTP, GROUP_PARTS = Pk<1>::GROUP_PARTS;

// threadIdx.x behind an empty asm: per-lane address math derived from it is recomputed where it
// is used instead of being hoisted out of the step / layer loops and held live (which spills).
__device__ __forceinline__ int my_tid() {
    int t = (int)threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Wave index as a wave-uniform (scalar) value, so that role branches compile to scalar branches.
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane((int)threadIdx.x / 64); }

__device__ __forceinline__ uint64_t ld64(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st64(uint64_t* p, uint64_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// A packet holds two fp32 values and is written by one 64-bit store (single-copy atomic: a
// reader sees both values of one store).  The low word is value a rounded to a 19-bit mantissa
// whose low 4 bits carry the tag of the round (1..15: the round number mod 15, plus one; a
// cleared packet carries 0); the high word is value b, exact.  A packet is rewritten once per
// round of its area and a poll can only meet its own round or the two before it, so 15 tags
// never alias.
__device__ __forceinline__ unsigned tag4(unsigned round) { return round % 15u + 1u; }
__device__ __forceinline__ float q19(float v) { return as_f32((as_u32(v) + 8u) & ~0xFu); }
__device__ __forceinline__ uint64_t pack2(float a, float b, unsigned round) {
    return (uint64_t)(as_u32(q19(a)) | tag4(round)) | ((uint64_t)as_u32(b) << 32);
}
__device__ __forceinline__ unsigned tag_of(uint64_t p) { return (unsigned)p & 0xFu; }
__device__ __forceinline__ float lo_of(uint64_t p) { return as_f32((uint32_t)p & ~0xFu); }
__device__ __forceinline__ float hi_of(uint64_t p) { return as_f32((uint32_t)(p >> 32)); }

// 2^x (v_exp_f32): the persistent attention keeps scores in base-2 units.
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// Lane pair swaps by DPP (a VALU move, no LDS round trip): lane l receives lane l ^ 1; and, within
// each row of 16 lanes, lanes 0-7 receive lanes 8-15 and back (rotate by 8).
__device__ __forceinline__ float xor1(float v) { return dpp<DPP_XOR1>(v); }
__device__ __forceinline__ float xor8(float v) { return dpp<0x128>(v); }

// SwiGLU of a gate / up pair: g sigmoid(g) u, with 2^x and the reciprocal on the transcendental
// unit (each ~1 ulp).
__device__ __forceinline__ float swiglu(float g, float u) {
    return g * __builtin_amdgcn_rcpf(1.f + ex2(-g * 1.4426950408889634f)) * u;
}

// 16 bytes per lane from global memory straight into LDS: lane l's bytes land at lds + 16 l
// (lds is wave-uniform).  Counted by the issuing wave's vector-memory counter.
__device__ __forceinline__ void lds_dma16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

__device__ __forceinline__ unsigned load_err(const unsigned* e) {
    return __hip_atomic_load(e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void raise_err(unsigned* e) {
    __hip_atomic_store(e, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Exchange threads: loads the packets at(i) (i < NP; nullptr: no packet) until each carries the
// tag of `round`.  false on timeout (after raising the error flag) or when another workgroup
// raised it.
template <int NP, typename At>
__device__ __forceinline__ bool spin_tags(uint64_t (&p)[NP], At at, unsigned round, unsigned* err) {
    const unsigned tag = tag4(round);
    const uint64_t filler = tag;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const uint64_t* q = at(i);
        p[i] = q ? ld64(q) : filler;
    }
    for (int it = 0;; ++it) {
        bool ok = true;
#pragma unroll
        for (int i = 0; i < NP; ++i) ok &= tag_of(p[i]) == tag;
        if (ok) return true;
        if (it >= SPIN_LIMIT) {
            raise_err(err);
            return false;
        }
        if ((it & 63) == 63 && load_err(err)) return false;
#pragma unroll
        for (int i = 0; i < NP; ++i)
            if (tag_of(p[i]) != tag) p[i] = ld64(at(i));  // a filler always carries the tag
    }
}

// Exchange threads: polls packets src[k], k = ct + CT * i < n (consecutive lanes read consecutive
// packets), until each carries the tag of `round`, then writes their values to dst[2k], dst[2k + 1].
template <int NP>
__device__ __forceinline__ bool poll_vec(const uint64_t* src, int n, unsigned round, float* dst, unsigned* err) {
    const int ct = my_tid() - MT;
    uint64_t p[NP];
    if (!spin_tags(p, [&](int i) { return ct + CT * i < n ? src + ct + CT * i : nullptr; }, round, err)) return false;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int k = ct + CT * i;
        if (k < n) {
            dst[2 * k] = lo_of(p[i]);
            dst[2 * k + 1] = hi_of(p[i]);
        }
    }
    return true;
}

// Exchange threads: as poll_vec, for packets src[map(k)] of a gathered vector (k < n).
template <int NP, typename Map>
__device__ __forceinline__ bool poll_map(const uint64_t* src, int n, Map map, unsigned round, float* dst, unsigned* err) {
    const int ct = my_tid() - MT;
    uint64_t p[NP];
    if (!spin_tags(p, [&](int i) { return ct + CT * i < n ? src + map(ct + CT * i) : nullptr; }, round, err))
        return false;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int k = ct + CT * i;
        if (k < n) {
            dst[2 * k] = lo_of(p[i]);
            dst[2 * k + 1] = hi_of(p[i]);
        }
    }
    return true;
}

// Exchange threads: as poll_vec for n = NP * CT packets, the sums of two packet vectors a, b.
template <int NP>
__device__ __forceinline__ bool poll_sum(const uint64_t* a, const uint64_t* b, unsigned round, float* dst, unsigned* err) {
    const int ct = my_tid() - MT;
    uint64_t p[2 * NP];
    if (!spin_tags(p, [&](int i) { return (i < NP ? a : b) + ct + CT * (i % NP); }, round, err)) return false;
#pragma unroll
    for (int i = 0; i < NP; ++i) {
        const int k = ct + CT * i;
        dst[2 * k] = lo_of(p[i]) + lo_of(p[NP + i]);
        dst[2 * k + 1] = hi_of(p[i]) + hi_of(p[NP + i]);
    }
    return true;
}

// Compact activation operands: per group the hi, mid, lo slices of its 4 K-slots (q4: 16 bytes
// each, 192 B per 64-group; q8: 8 bytes each, 96 B per 32-group), K <= 6144.
constexpr int A_BYTES = 18432;
// Down half-block of a workgroup in LDS: 1 KiB chunks (q4 24, q8 48), then the 16 rows' scales
// in four per-wave parts of 16 x 48 B (q4: 12 (scale, bias) pairs, q8: 24 scales per row).
constexpr int WD_CODES = (FFH / 64) * 1024, WD_SB = 16 * MW * 48;
static_assert(((VOCAB / 16 + NWG - 1) / NWG) * WAVES * 16 * 4 <= WD_CODES + WD_SB, "lm_head partial sums fit the down block buffer");

struct Shared {
    // Small fields first: an LDS access reaches 64 KiB past its address register, so the fields
    // read at fixed offsets stay within the first 64 KiB of the struct.
    uint32_t zero[4];         // operand rows 3..15 of every tile (16 zero bytes)
    float misc[64];
    int imisc[64];
    int fail;                 // a wait of this workgroup failed (set only then; see sync_failed)
    int go;                   // round whose split partials a watching lane has seen complete
    float xown[2][16];        // residual rows of this workgroup's O / down block (workgroups < 128), per pass row
    float xhi[2][16];         // the upper-half down sums of those rows from the previous layer
    float aml[MW][8];         // per math wave and row: (m head 0, m head 1, l head 0, l head 1)
    float fx[192 * 2];        // per-group (2^(e-21), sum X * 2^(e-21))
    alignas(16) float red[6 * MW * 64];  // partial sums of the waves (up to 6 blocks: 3 blocks x 2 rows)
    // attention: the two query heads of each pass row t as fp16 hi and lo parts, rows 4 t + (hi 2g,
    // hi 2g + 1, lo 2g, lo 2g + 1): the A operand rows of the score tiles
    alignas(16) uint16_t qf[8][HD];
    alignas(16) float pw[MW][2][2][4][12];  // probabilities of a math wave's slots, [row][head][lane / 16][i]
    alignas(16) uint16_t ktail[2][HD];     // the pass's new K / V rows (fp16), in the cache
    alignas(16) uint16_t vtail[2][HD];     // layout: one 16-byte read is an operand's 8 dims
    float sc[2][ATT_PAD];
    float ored[MW][4][HD];    // per math wave: o of (row, head)
    float nw[H];              // RMSNorm weights of the current stage
    uint8_t A[A_BYTES];       // activation operands; the merger's fp32 partials during the merge
    float vec[FF];            // input vector of the current stage (fp32)
    float emb[2 * H];         // embeddings of the pass's tokens (row t at t H)
};

// Workgroup barrier for data exchanged through LDS only: waits for this wave's LDS accesses, not
// for its vector-memory loads (__syncthreads would drain the weight slices in flight, so a stage
// could not stage its input while its tiles land).  The empty asm statements keep the compiler
// from moving memory accesses across it.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (0 << 8) | (3 << 14));  // vmcnt 63, expcnt 7, lgkmcnt 0
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Workgroup barrier that also tells every thread whether any thread's wait failed.  The flag is
// written only on failure, so the common path is one barrier and one LDS read (the library's
// __syncthreads_or costs three barriers and three LDS operations).
__device__ __forceinline__ bool sync_failed(Shared& S, bool failed) {
    if (failed) S.fail = 1;
    __syncthreads();
    return S.fail != 0;
}

// ------------------------------------------------------------------------------------------
// Staging by the whole workgroup: units of 4 consecutive activations (u = tid + THREADS * j <
// K / 4), each multiplied by its RMSNorm weight S.nw when `normed`, become exact integers of the
// group's fixed point (|v| < 2^22, the group maximum's exponent e mapped to bit 21) and are cut
// into three int8 slices: the compact A operands (rows 0, 1, 2 of a group's tile: hi, mid, lo;
// rows 3..15 read S.zero) and the group factors (2^(e-21), sum of the integers * 2^(e-21)).  A
// group is 16 (q4) or 8 (q8) consecutive lanes, so its maximum and sum are DPP row reductions.
//
// The RMS factor 1/sqrt(mean(v^2) + eps) of a normed input is a scalar of the whole vector, so it
// is not applied here: each wave leaves its sum of v^2 in S.misc[40 + wave] and the stage's
// epilogue multiplies its sums by norm_scale().  The integer conversion is one fma with the
// magic constant 1.5 * 2^23 (round to nearest even, as rint); the slices are the bytes of
// (v + 0x808080) ^ 0x808080, which three byte permutes gather into the hi / mid / lo rows.  When
// K / 4 is not a multiple of THREADS the last unit row is held by the first waves only (whole
// waves, so whole groups).  NRS rows (src + t K) are staged with one barrier: row t's groups
// follow row t - 1's (group offset t K / G) and its sum of squares goes to S.misc[40 + 8 t + wave].
template <int FMT, int K, int NRS = 1, class SH, bool LDS_ONLY = false>
__device__ __forceinline__ void stage_c(SH& S, const float* src, bool normed) {
    constexpr int G = (FMT == FMT_Q4) ? 64 : 32;
    constexpr int TILE = (FMT == FMT_Q4) ? 192 : 96;
    constexpr int SLOT = (FMT == FMT_Q4) ? 16 : 8;  // bytes of a K-slot row
    constexpr int NU = (K / 4 + THREADS - 1) / THREADS;
    constexpr uint32_t MAGIC = 0x4B400000u;        // 1.5 * 2^23
    static_assert((K / 4) % 64 == 0, "units of whole waves");
    static_assert(NRS * (K / G) * TILE <= A_BYTES && NRS * (K / G) * 2 <= 384, "operands fit S.A / S.fx");
    const int tid = my_tid(), lane = tid % 64, wave = wave_id();
#pragma unroll
    for (int rw = 0; rw < NRS; ++rw) {
        float ss = 0.f;
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const int u = tid + THREADS * j;
            if ((K / 4) % THREADS != 0 && u >= K / 4) continue;
            const float4 a4 = ((const float4*)(src + rw * K))[u];
            float v[4] = {a4.x, a4.y, a4.z, a4.w};
            if (normed) {
                const float4 wn = ((const float4*)S.nw)[u];
                ss = fmaf(v[0], v[0], ss);
                ss = fmaf(v[1], v[1], ss);
                ss = fmaf(v[2], v[2], ss);
                ss = fmaf(v[3], v[3], ss);
                v[0] *= wn.x;
                v[1] *= wn.y;
                v[2] *= wn.z;
                v[3] *= wn.w;
            }
            const float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
            int bits = (int)as_u32(amax);  // order of non-negative floats = order of their bits
            bits = max(bits, dpp_i<DPP_XOR1>(bits));
            bits = max(bits, dpp_i<DPP_XOR2>(bits));
            bits = max(bits, dpp_i<DPP_HALF_MIRROR>(bits));
            if constexpr (G == 64) bits = max(bits, dpp_i<DPP_MIRROR>(bits));
            // e: exponent of the group maximum, clamped so that 2^(21 - e) and 2^(e - 21) are normal
            // (an all-zero group gives X = 0 with any e).
            const int e = min(max(((bits >> 23) & 0xFF) - 127, -100), 126);
            const float p = as_f32((uint32_t)(148 - e) << 23);  // 2^(21 - e)
            uint32_t t[4];
            int xs = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t f = as_u32(__builtin_fmaf(v[i], p, as_f32(MAGIC)));  // MAGIC + rint(v 2^(21-e))
                xs += (int)(f - MAGIC);
                t[i] = (f + 0x408080u) ^ 0x808080u;  // bytes: lo, mid, hi slices as int8
            }
            const uint32_t p01 = __builtin_amdgcn_perm(t[1], t[0], 0x05010400u);  // l0 l1 m0 m1
            const uint32_t p23 = __builtin_amdgcn_perm(t[3], t[2], 0x05010400u);  // l2 l3 m2 m3
            const uint32_t q01 = __builtin_amdgcn_perm(t[1], t[0], 0x0C0C0602u);  // h0 h1
            const uint32_t q23 = __builtin_amdgcn_perm(t[3], t[2], 0x0C0C0602u);  // h2 h3
            const uint32_t lo = __builtin_amdgcn_perm(p23, p01, 0x05040100u);
            const uint32_t mid = __builtin_amdgcn_perm(p23, p01, 0x07060302u);
            const uint32_t hi = __builtin_amdgcn_perm(q23, q01, 0x05040100u);
            xs += dpp_i<DPP_XOR1>(xs);
            xs += dpp_i<DPP_XOR2>(xs);
            xs += dpp_i<DPP_HALF_MIRROR>(xs);
            if constexpr (G == 64) xs += dpp_i<DPP_MIRROR>(xs);
            const int k0 = u * 4, gl = rw * (K / G) + k0 / G, kk = k0 % G;
            uint8_t* A = S.A + gl * TILE;
            const int q = kk / SLOT, j0 = kk % SLOT;
            *(uint32_t*)(A + (3 * q + 0) * SLOT + j0) = hi;
            *(uint32_t*)(A + (3 * q + 1) * SLOT + j0) = mid;
            *(uint32_t*)(A + (3 * q + 2) * SLOT + j0) = lo;
            if (kk == 0) {
                const float f = as_f32((uint32_t)(106 + e) << 23);  // 2^(e - 21)
                S.fx[gl * 2] = f;
                S.fx[gl * 2 + 1] = (float)xs * f;
            }
        }
        if (normed) {
            ss = wave_sum(ss);
            if (lane == 0) S.misc[40 + 8 * rw + wave] = ss;
        }
    }
    if constexpr (LDS_ONLY)
        lds_barrier();  // the slice-streaming form: the weight slices in flight stay in flight
    else
        __syncthreads();
}

// RMS factor of the last normed staging of a K-vector: 1/sqrt(mean(v^2) + eps) from the eight
// waves' sums (valid after the staging's barrier, until the next normed staging).
template <int K>
__device__ __forceinline__ float norm_scale(const Shared& S, int t = 0) {
    const float* m = S.misc + 40 + 8 * t;  // row t of a multi-row staging
    const float tot = ((m[0] + m[1]) + (m[2] + m[3])) + ((m[4] + m[5]) + (m[6] + m[7]));
    return __builtin_amdgcn_rsqf(tot * (1.0f / (float)K) + EPS);  // v_rsq_f32 (1 ulp)
}

// Two 1 KiB chunks (c, c + 1) of a 16-row block against the staged operands: a quad of four
// quantisation groups (q4: 2 x 64 K per chunk; q8: 2 x 32 K).  The four multiplies of a quad
// accumulate into one result: group j's operand tile puts its three slices in rows 4j .. 4j + 2
// and zeros elsewhere, so lanes 16j .. 16j + 15 end with group j's (hi, mid, lo) sums of weight
// rows 0-15, and one group scaling serves all four groups.  quad_load reads the four operand
// tiles (lane (r, q): slice r % 4 of K-slot q of group r / 4 when r % 4 < 3, else the zero
// block) and the factors (2^(e-21), sum X 2^(e-21)) of the lane's group j = lane / 16.
template <int FMT>
struct QuadOps {
    v4i A[4];  // operand tile of group position j (q8 uses the low 8 bytes)
    float f, fX;
};

template <int FMT, class SH>
__device__ __forceinline__ QuadOps<FMT> quad_load(const SH& S, int c, int lane, int g0 = 0) {
    QuadOps<FMT> o;
    const int r = lane & 15, q = lane >> 4, sl = r & 3, jr = r >> 2;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        // groups 2c, 2c + 1 (chunk c), 2c + 2, 2c + 3 (chunk c + 1) of the row staged at group g0
        const int gl = g0 + 2 * c + j;
        const bool on = jr == j && sl < 3;
        if constexpr (FMT == FMT_Q4) {
            const uint8_t* ap = on ? S.A + gl * 192 + (3 * q + sl) * 16 : (const uint8_t*)S.zero;
            o.A[j] = *(const v4i*)ap;
        } else {
            const uint8_t* ap = on ? S.A + gl * 96 + (3 * q + sl) * 8 : (const uint8_t*)S.zero;
            const long v = *(const long*)ap;
            o.A[j] = v4i{(int)(uint32_t)v, (int)(uint32_t)((uint64_t)v >> 32), 0, 0};
        }
    }
    const float2 fx = *(const float2*)(S.fx + (g0 + 2 * c + q) * 2);
    o.f = fx.x;
    o.fX = fx.y;
    return o;
}

// Integer sums of a quad against weight chunks w0 (groups j = 0, 1) and w1 (j = 2, 3):
// v_mfma_i32_16x16x64_i8 (q4) / 16x16x32 (q8), accumulated.
template <int FMT>
__device__ __forceinline__ v4i quad_mfma(const QuadOps<FMT>& o, uint4 w0, uint4 w1) {
    v4i C = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint4 wv = j < 2 ? w0 : w1;
        const int hh = j & 1;
        if constexpr (FMT == FMT_Q4) {
            const uint32_t d0 = hh ? wv.z : wv.x, d1 = hh ? wv.w : wv.y;
            v4i B;
            B[0] = (int)(d0 & 0x0F0F0F0Fu);
            B[1] = (int)((d0 >> 4) & 0x0F0F0F0Fu);
            B[2] = (int)(d1 & 0x0F0F0F0Fu);
            B[3] = (int)((d1 >> 4) & 0x0F0F0F0Fu);
            C = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.A[j], B, C, 0, 0, 0);
        } else {
            const long B = (long)(hh ? ((uint64_t)wv.w << 32 | wv.z) : ((uint64_t)wv.y << 32 | wv.x));
            const long A = (long)((uint64_t)(uint32_t)o.A[j][0] | ((uint64_t)(uint32_t)o.A[j][1] << 32));
            C = __builtin_amdgcn_mfma_i32_16x16x32_i8(A, B, C, 0, 0, 0);
        }
    }
    return C;
}

// Group scaling of a quad's sums into the lane's partial: Sv = 65536 hi + (256 mid + lo) (the
// bracket exact in int32), then acc += s (f Sv) + b (f X) with the fp16 scale / bias word `sq` of
// the lane's group (q8: the scale in the low half) read by mixed-precision fmas.
template <int FMT>
__device__ __forceinline__ float quad_scale(const QuadOps<FMT>& o, v4i C, uint32_t sq, float acc) {
    const float Sv = fmaf((float)C[0], 65536.f, (float)(C[1] * 256 + C[2]));
    const f16x2 sb2 = as_h2(sq);
    acc = fmaf((float)sb2.x, o.f * Sv, acc);
    if constexpr (FMT == FMT_Q4) acc = fmaf((float)sb2.y, o.fX, acc);
    return acc;
}

// Sum of a lane's partial with the three other lanes of its weight row (l, l ^ 16, l ^ 32,
// l ^ 48): lanes 0-15 then hold the row totals.
__device__ __forceinline__ float quad_rows(float v) { return sum_x4(v); }

// The scale word of the lane's group in a quad: row `row`, group 2c + lane / 16 (q4: the
// (scale, bias) half2; q8: the scale).
template <int FMT>
__device__ __forceinline__ uint32_t load_sq(const uint8_t* sb, int row, int K, int c, int lane) {
    if constexpr (FMT == FMT_Q4)
        return *(const uint32_t*)(sb + ((size_t)row * (K / 64) + 2 * c + (lane >> 4)) * 4);
    else
        return (uint32_t) * (const uint16_t*)(sb + ((size_t)row * (K / 32) + 2 * c + (lane >> 4)) * 2);
}

// This math wave's share (chunks mw * CW .. mw * CW + CW - 1, CW even) of 16-row block rb.
template <int FMT, int CW>
struct WB {
    static_assert(CW % 2 == 0, "whole quads");
    uint4 wv[CW];
    uint32_t sq[CW / 2];
    __device__ __forceinline__ void load(const uint8_t* w, const uint8_t* sbp, int rb, int K, int mw, int lane) {
        constexpr int CHK = (FMT == FMT_Q4) ? 128 : 64;
        const int cpb = K / CHK;
        const uint8_t* blk = w + (size_t)rb * cpb * 1024;
#pragma unroll
        for (int i = 0; i < CW; ++i) wv[i] = ((const uint4*)(blk + (size_t)(mw * CW + i) * 1024))[lane];
#pragma unroll
        for (int p = 0; p < CW / 2; ++p) sq[p] = load_sq<FMT>(sbp, rb * 16 + (lane & 15), K, mw * CW + 2 * p, lane);
    }
    // Ends the live range of the tile's registers (no instruction): a tile loaded under a
    // condition is otherwise kept alive across every path where the condition is false.
    __device__ __forceinline__ void forget() {
#pragma unroll
        for (int i = 0; i < CW; ++i) asm volatile("" : "=v"(wv[i].x), "=v"(wv[i].y), "=v"(wv[i].z), "=v"(wv[i].w));
#pragma unroll
        for (int p = 0; p < CW / 2; ++p) asm volatile("" : "=v"(sq[p]));
    }
};

// NB blocks' shares (the same chunks of NB row blocks) against the staged operands: each quad's
// operand tiles are read from LDS once for all blocks.  acc[b] is block b's total of this wave in
// lanes 0-15.
template <int FMT, int CW, int NB>
__device__ __forceinline__ void mac_blocks(const Shared& S, const WB<FMT, CW>* wb, int mw, int lane, float (&acc)[NB],
                                           int g0 = 0) {
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = 0.f;
#pragma unroll
    for (int p = 0; p < CW / 2; ++p) {
        const QuadOps<FMT> o = quad_load<FMT>(S, mw * CW + 2 * p, lane, g0);
        v4i C[NB];
#pragma unroll
        for (int b = 0; b < NB; ++b) C[b] = quad_mfma<FMT>(o, wb[b].wv[2 * p], wb[b].wv[2 * p + 1]);
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = quad_scale<FMT>(o, C[b], wb[b].sq[p], acc[b]);
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) acc[b] = quad_rows(acc[b]);
}

// mac_blocks for NR staged rows (row t at group offset t * gstride): acc[t * NB + b].  Each quad's
// weight registers are multiplied by every row before the next quad is touched, so they are free
// once the quad is done, as in the one-row loop.
template <int FMT, int CW, int NB, int NR>
__device__ __forceinline__ void mac_rows(const Shared& S, const WB<FMT, CW>* wb, int mw, int lane,
                                         float (&acc)[NR * NB], int gstride) {
#pragma unroll
    for (int b = 0; b < NR * NB; ++b) acc[b] = 0.f;
#pragma unroll
    for (int p = 0; p < CW / 2; ++p) {
#pragma unroll
        for (int t = 0; t < NR; ++t) {
            const QuadOps<FMT> o = quad_load<FMT>(S, mw * CW + 2 * p, lane, t * gstride);
            v4i C[NB];
#pragma unroll
            for (int b = 0; b < NB; ++b) C[b] = quad_mfma<FMT>(o, wb[b].wv[2 * p], wb[b].wv[2 * p + 1]);
#pragma unroll
            for (int b = 0; b < NB; ++b) acc[t * NB + b] = quad_scale<FMT>(o, C[b], wb[b].sq[p], acc[t * NB + b]);
        }
    }
#pragma unroll
    for (int b = 0; b < NR * NB; ++b) acc[b] = quad_rows(acc[b]);
}

// Down half-block `half` of row block rb straight into wdb (math wave mw requests the chunks
// and the scale columns it multiplies later, so each wave reads back only its own requests).
template <int FMT>
__device__ __forceinline__ void wd_request(uint8_t* wdb, const uint8_t* wd, const uint8_t* wd_sb, int rb, int half,
                                           int mw, int lane) {
    constexpr int CHK = (FMT == FMT_Q4) ? 128 : 64;
    constexpr int NC = FF / CHK, CWD = FFH / CHK / MW;  // chunks per row block, per wave
    const uint8_t* blk = wd + ((size_t)rb * NC + half * (NC / 2)) * 1024;
#pragma unroll
    for (int i = 0; i < CWD; ++i) {
        const int c = mw * CWD + i;
        lds_dma16(blk + (size_t)c * 1024 + lane * 16, wdb + c * 1024);
    }
    // Scales (FF / 16 bytes per row in both formats): rows 16 rb + r, bytes 192 half + 48 mw ..
    // + 47 -> 16 x 48 B at WD_CODES + 768 mw; lane j < 48 carries row j / 3, 16 B part j % 3.
    if (lane < 48)
        lds_dma16(wd_sb + (size_t)(16 * rb + lane / 3) * (FF / 16) + 192 * half + 48 * mw + 16 * (lane % 3),
                  wdb + WD_CODES + mw * 768);
}

// The math wave's share of the down half-block from wdb (after its requests have landed), a
// quad (two chunks) at a time; the total in lanes 0-15.  The wave's scale columns in LDS are
// 16 rows x 48 B: (scale, bias) words of its 12 q4 groups, or the scales of its 24 q8 groups.
template <int FMT>
__device__ __forceinline__ float wd_mac_lds(const Shared& S, const uint8_t* wdb, int mw, int lane, int g0 = 0) {
    constexpr int CHK = (FMT == FMT_Q4) ? 128 : 64;
    constexpr int CWD = FFH / CHK / MW;
    static_assert(CWD % 2 == 0, "whole quads");
    const uint8_t* sbr = wdb + WD_CODES + mw * 768 + 48 * (lane & 15);
    float acc = 0.f;
#pragma unroll
    for (int p = 0; p < CWD / 2; ++p) {
        const uint4 w0 = *(const uint4*)(wdb + (mw * CWD + 2 * p) * 1024 + lane * 16);
        const uint4 w1 = *(const uint4*)(wdb + (mw * CWD + 2 * p + 1) * 1024 + lane * 16);
        const int gq = 4 * p + (lane >> 4);  // the lane's group among the wave's
        const uint32_t sq = FMT == FMT_Q4 ? *(const uint32_t*)(sbr + 4 * gq) : (uint32_t) * (const uint16_t*)(sbr + 2 * gq);
        const QuadOps<FMT> o = quad_load<FMT>(S, mw * CWD + 2 * p, lane, g0);
        acc = quad_scale<FMT>(o, quad_mfma<FMT>(o, w0, w1), sq, acc);
    }
    return quad_rows(acc);
}

// Sum of the math waves' per-lane partials (whole-workgroup call); the total is valid in math
// wave 0 (lanes 0-15 meaningful).  One barrier: S.red is next written after the barriers of a
// later stage, so wave 0's reads need no second one.
template <bool MATH>
__device__ __forceinline__ float reduce_math(Shared& S, float acc) {
    const int tid = my_tid(), lane = tid % 64, wave = wave_id();
    if (MATH) S.red[wave * 64 + lane] = acc;
    __syncthreads();
    float s = 0.f;
    if (wave == 0) s = (S.red[lane] + S.red[64 + lane]) + (S.red[128 + lane] + S.red[192 + lane]);
    return s;
}

// The math waves' partials of N <= 6 blocks into S.red (one barrier); red_total(S, j) then reads
// block j's total (math wave 0, lanes 0-15 meaningful) where it is used, so that no wave holds
// the N totals in registers across the stage.
template <bool MATH, int N>
__device__ __forceinline__ void reduce_math_store(Shared& S, const float (&acc)[N]) {
    static_assert(N <= 6, "S.red holds six blocks");
    const int tid = my_tid(), lane = tid % 64, wave = wave_id();
    if (MATH) {
#pragma unroll
        for (int j = 0; j < N; ++j) S.red[(j * MW + wave) * 64 + lane] = acc[j];
    }
    __syncthreads();
}
__device__ __forceinline__ float red_total(const Shared& S, int j) {
    const int lane = my_tid() % 64;
    const float* r = S.red + j * MW * 64;
    return (r[lane] + r[64 + lane]) + (r[128 + lane] + r[192 + lane]);
}

// reduce_math for N <= 6 blocks at once (one barrier).
template <bool MATH, int N>
__device__ __forceinline__ void reduce_math_n(Shared& S, const float (&acc)[N], float (&out)[N]) {
    static_assert(N <= 6, "S.red holds six blocks");
    const int tid = my_tid(), lane = tid % 64, wave = wave_id();
    if (MATH) {
#pragma unroll
        for (int j = 0; j < N; ++j) S.red[(j * MW + wave) * 64 + lane] = acc[j];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int j = 0; j < N; ++j) {
            const float* r = S.red + j * MW * 64;
            out[j] = (r[lane] + r[64 + lane]) + (r[128 + lane] + r[192 + lane]);
        }
    }
}

__device__ __forceinline__ void norm_rope(float& a, float& b, float w0, float w1, float c, float sn) {
    const float ss = wave_sum(a * a + b * b);
    const float scale = __builtin_amdgcn_rsqf(ss * (1.0f / (float)HD) + EPS);  // v_rsq_f32 (1 ulp)
    a = a * scale * w0;
    b = b * scale * w1;
    const float a2 = a * c - b * sn, b2 = b * c + a * sn;
    a = a2;
    b = b2;
}

// Wave 0 of a workgroup waits until the (l, m) packets of all 32 attention splits of its KV group
// carry tag tg (lane s < 32 polls split s's packet at base + s * stride), then stores go in S.go.
// A wait that fails or runs past SPIN_LIMIT sets S.fail first (the next barrier returns).  Lanes
// leave the loop together (a ballot), so S.go is always stored.
__device__ __forceinline__ void watch_partials(Shared& S, const uint64_t* base, size_t stride, unsigned tg, int go,
                                               unsigned* err, int lane) {
    const bool mine = lane < ATT_SPLITS;
    const uint64_t* q = base + (size_t)(mine ? lane : 0) * stride;
    for (int it = 0;; ++it) {
        const bool waiting = mine && tag_of(ld64(q)) != tg;
        if (__builtin_amdgcn_ballot_w64(waiting) == 0) break;
        if (it >= SPIN_LIMIT) raise_err(err);
        if (it >= SPIN_LIMIT || ((it & 63) == 63 && load_err(err))) {
            if (lane == 0) S.fail = 1;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    if (lane == 0) __hip_atomic_store(&S.go, go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Math threads: the cache rows of one attention block (block slots 0 .. ATT_BLOCK - 1 at split
// row j0 + b0) that this lane holds; only rows < nprior come from the cache, zeros elsewhere.
//   K, for the score tiles: tile T of math wave mw has 16 columns; column c = lane % 16 is block
//     slot att_slot(T, c, mw) = 16 (4 T + c / 4) + 4 mw + c % 4, and the lane holds its 16 bytes
//     at dims 32 j + 8 (lane / 16), j = 0..3 (the B operand of v_mfma_f32_16x16x32_f16).
//   V, for P.V: block slots quad + 16 i (quad = 4 mw + lane / 16), 8 dims (16 B) at 8 (lane % 16).
// So the slot of V row (quad, i) is column 4 (i % 4) + lane / 16 of tile i / 4 of the same wave.
__device__ __forceinline__ int att_slot(int T, int c, int mw) { return 16 * (4 * T + (c >> 2)) + 4 * mw + (c & 3); }

__device__ __forceinline__ void load_kv_block(uint4 (&kt)[ATT_NT][4], uint4 (&vr)[ATT_SPQ], const uint16_t* kb,
                                              const uint16_t* vb, int j0, int b0, int nprior, int tid) {
    // Buffer loads over the split's cached rows j0 .. j0 + nprior - 1: a load past them returns
    // zeros without touching memory, so every lane issues the same loads with no branches.
    const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc((void*)(kb + (size_t)j0 * HD), (short)0, nprior * HD * 2, 0x00020000);
    const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc((void*)(vb + (size_t)j0 * HD), (short)0, nprior * HD * 2, 0x00020000);
    const int lane = tid % 64, mw = tid / 64, c = lane & 15, kq = lane >> 4, quad = tid / 16, ql = tid % 16;
#pragma unroll
    for (int T = 0; T < ATT_NT; ++T) {
        // Columns of tile 2 past i = ATT_SPQ - 1 hold no slot: their offset is pushed past the buffer.
        const int p = 4 * T + (c >> 2) < ATT_SPQ ? b0 + att_slot(T, c, mw) : (1 << 20);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(krs, (p * HD + 32 * j + 8 * kq) * 2, 0, 0);
            kt[T][j] = make_uint4(v.x, v.y, v.z, v.w);
        }
    }
#pragma unroll
    for (int i = 0; i < ATT_SPQ; ++i) {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(vrs, ((b0 + quad + ATT_QW * i) * HD + 8 * ql) * 2, 0, 0);
        vr[i] = make_uint4(v.x, v.y, v.z, v.w);
    }
}

__device__ __forceinline__ h8 as_h8(uint4 v) { return __builtin_bit_cast(h8, u32x4{v.x, v.y, v.z, v.w}); }

// Max over the 16 lanes of each row of 16 (every lane gets its row's maximum).
__device__ __forceinline__ float max16(float v) {
    v = fmaxf(v, dpp<DPP_MIRROR>(v));
    v = fmaxf(v, dpp<DPP_HALF_MIRROR>(v));
    v = fmaxf(v, dpp<DPP_XOR2>(v));
    return fmaxf(v, dpp<DPP_XOR1>(v));
}

__device__ __forceinline__ void load_norm8(float (&n)[8], const float* p) {
    const float4 n0 = ((const float4*)p)[0], n1 = ((const float4*)p)[1];
    n[0] = n0.x; n[1] = n0.y; n[2] = n0.z; n[3] = n0.w;
    n[4] = n1.x; n[5] = n1.y; n[6] = n1.z; n[7] = n1.w;
}

// ------------------------------------------------------------------------------------------
// f16 weights (Shaders.swift:459-531, the FMT == 0 branch of the reference's decode kernels).  A
// 16-row block of a K = 2048 f16 matrix is 64 KiB, four times a q4 block: it cannot wait in the
// registers ahead of its stage as the int8 tiles do, so the f16 stages stream their blocks (all
// eight waves, each a K-slice of every block) once the stage input is in, and multiply them on
// v_mfma_f32_16x16x32_f16: the repacked tile chunk is already the B operand (16 rows x 32 K), and
// the A operand is the staged vector's 32 K as fp16 hi (row 0) and lo (row 1) parts; rows 2..15
// read S.zero.  Every 32-K chunk of the staged vector is scaled by the power of two that puts its
// largest |v| in [2^14, 2^15), so that hi + lo hold ~22 bits of each value, and the chunk's two
// sums are scaled back by 2^(e - 14) as they are accumulated.

constexpr int F16_CHK = 32;  // K per 1 KiB f16 chunk

// The K values of src (fp32, times S.nw when normed) -> S.A, chunk c at c * 128 bytes: 32 fp16 hi
// parts, then 32 lo parts, of v * 2^(14 - e_c); S.fx[c] = 2^(e_c - 14); each wave's sum of squares
// to S.misc[40 + wave] (normed), as stage_c leaves them for norm_scale.  Whole workgroup, one
// barrier.  A unit is 4 consecutive values; the 8 lanes of a chunk find its maximum by DPP.
template <int K>
__device__ __forceinline__ void stage_f16(Shared& S, const float* src, bool normed) {
    static_assert((K / 4) % 64 == 0 && (K / F16_CHK) * 128 <= A_BYTES && K / F16_CHK <= 384, "operands fit S.A / S.fx");
    constexpr int NU = (K / 4 + THREADS - 1) / THREADS;
    const int tid = my_tid(), lane = tid % 64, wave = wave_id();
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < NU; ++j) {
        const int u = tid + THREADS * j;
        if ((K / 4) % THREADS != 0 && u >= K / 4) continue;  // whole waves
        const float4 a4 = ((const float4*)src)[u];
        float v[4] = {a4.x, a4.y, a4.z, a4.w};
        if (normed) {
            const float4 wn = ((const float4*)S.nw)[u];
            ss = fmaf(v[0], v[0], ss);
            ss = fmaf(v[1], v[1], ss);
            ss = fmaf(v[2], v[2], ss);
            ss = fmaf(v[3], v[3], ss);
            v[0] *= wn.x;
            v[1] *= wn.y;
            v[2] *= wn.z;
            v[3] *= wn.w;
        }
        const float amax = fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3])));
        int bits = (int)as_u32(amax);  // order of non-negative floats = order of their bits
        bits = max(bits, dpp_i<DPP_XOR1>(bits));
        bits = max(bits, dpp_i<DPP_XOR2>(bits));
        bits = max(bits, dpp_i<DPP_HALF_MIRROR>(bits));
        // e: exponent of the chunk maximum, clamped so that 2^(14 - e) and 2^(e - 14) are normal.
        const int e = min(max(((bits >> 23) & 0xFF) - 127, -100), 100);
        const float p = as_f32((uint32_t)(141 - e) << 23);  // 2^(14 - e)
        uint32_t hw[2], lw[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const float x0 = v[2 * i] * p, x1 = v[2 * i + 1] * p;
            const uint16_t h0 = f2h(x0), h1 = f2h(x1);
            hw[i] = (uint32_t)h0 | ((uint32_t)h1 << 16);
            lw[i] = (uint32_t)f2h(x0 - h2f(h0)) | ((uint32_t)f2h(x1 - h2f(h1)) << 16);
        }
        const int k0 = u * 4, c = k0 / F16_CHK, kk = k0 % F16_CHK;
        uint8_t* A = S.A + c * 128;
        *(uint2*)(A + 2 * kk) = make_uint2(hw[0], hw[1]);
        *(uint2*)(A + 64 + 2 * kk) = make_uint2(lw[0], lw[1]);
        if (kk == 0) S.fx[c] = as_f32((uint32_t)(113 + e) << 23);  // 2^(e - 14)
    }
    if (normed) {
        ss = wave_sum(ss);
        if (lane == 0) S.misc[40 + wave] = ss;
    }
    lds_barrier();
}

// A wave's K-slice of NB f16 blocks: chunks c0 + i, i < CPW, of blocks rb[b] (NCB chunks per
// block), one 16-byte lane slice each.
template <int NB, int CPW>
struct WF {
    uint4 wv[NB][CPW];
    // Blocks B0 .. B1 - 1 of the NB (all by default).
    template <int B0 = 0, int B1 = NB>
    __device__ __forceinline__ void load(const uint8_t* w, const int (&rb)[NB], int ncb, int c0, int lane) {
#pragma unroll
        for (int b = B0; b < B1; ++b)
#pragma unroll
            for (int i = 0; i < CPW; ++i)
                wv[b][i] = ((const uint4*)(w + ((size_t)rb[b] * ncb + c0 + i) * 1024))[lane];
    }
    // Ends the live range of the slice's registers (as WB::forget).
    __device__ __forceinline__ void forget() {
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int i = 0; i < CPW; ++i) asm volatile("" : "=v"(wv[b][i].x), "=v"(wv[b][i].y), "=v"(wv[b][i].z), "=v"(wv[b][i].w));
    }
};

// acc[b] += the slice's products with the staged chunks s0 + i (the slice's chunk index within the
// staged vector); the sums land in lanes 0-15 (row lane of the block), other lanes add zeros.
template <int NB, int CPW>
__device__ __forceinline__ void mac_f16(const Shared& S, const WF<NB, CPW>& wf, int s0, int lane, float (&acc)[NB]) {
    const int r = lane & 15, q = lane >> 4;
#pragma unroll
    for (int i = 0; i < CPW; ++i) {
        const int c = s0 + i;
        const uint8_t* ap = r < 2 ? S.A + c * 128 + 64 * r + 16 * q : (const uint8_t*)S.zero;
        const h8 A = *(const h8*)ap;
        const float f = S.fx[c];
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const f32x4 D = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, as_h8(wf.wv[b][i]), f32x4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            acc[b] = fmaf(D[0] + D[1], f, acc[b]);
        }
    }
}

// Slice tiles, for the forms whose stages stream their weight tiles on all eight waves (f16 and
// q8 blocks): a wave's slice of NB 16-row blocks is CPW 1 KiB chunks, chunks slice * CPW .. of each
// block (with their group scales for q8).  mac(S, slice, ...) multiplies them with the staged
// chunks slice * CPW .. (the slice's chunks within the staged vector) and leaves this wave's sum
// of block b in lanes 0-15 of acc[b].
template <int FMT, int NB, int CPW>
struct SliceTiles;
template <int NB, int CPW>
struct SliceTiles<FMT_F16, NB, CPW> {
    WF<NB, CPW> t;
    template <int B0 = 0, int B1 = NB>
    __device__ __forceinline__ void load(const uint8_t* w, const uint8_t*, const int (&rb)[NB], int K, int slice, int lane) {
        t.template load<B0, B1>(w, rb, K / F16_CHK, slice * CPW, lane);
    }
    __device__ __forceinline__ void forget() { t.forget(); }
    __device__ __forceinline__ void mac(const Shared& S, int slice, int lane, float (&acc)[NB]) const {
#pragma unroll
        for (int b = 0; b < NB; ++b) acc[b] = 0.f;
        mac_f16(S, t, slice * CPW, lane, acc);
    }
};
template <int NB, int CPW>
struct SliceTiles<FMT_Q8, NB, CPW> {
    WB<FMT_Q8, CPW> t[NB];
    template <int B0 = 0, int B1 = NB>
    __device__ __forceinline__ void load(const uint8_t* w, const uint8_t* sb, const int (&rb)[NB], int K, int slice, int lane) {
#pragma unroll
        for (int b = B0; b < B1; ++b) t[b].load(w, sb, rb[b], K, slice, lane);
    }
    __device__ __forceinline__ void forget() {
#pragma unroll
        for (int b = 0; b < NB; ++b) t[b].forget();
    }
    __device__ __forceinline__ void mac(const Shared& S, int slice, int lane, float (&acc)[NB]) const {
        mac_blocks<FMT_Q8, CPW, NB>(S, t, slice, lane, acc);
    }
};
// The staging of the slice-streaming forms (an LDS-only closing barrier).
template <int FMT, int K>
__device__ __forceinline__ void stage_slices(Shared& S, const float* src, bool normed) {
    if constexpr (FMT == FMT_F16)
        stage_f16<K>(S, src, normed);
    else
        stage_c<FMT, K, 1, Shared, true>(S, src, normed);
}

// The partials of N <= 3 blocks from the NWV waves that computed them (lanes 0-15 of the waves in
// slots 0 .. NWV - 1) into S.red as [block][row][slot], one barrier.  red_sum16 then reads a
// row's NWV partials with one or two 16-byte LDS reads (not NWV dependent ones) and adds them in
// slot order.
template <int N>
__device__ __forceinline__ void red_store16(Shared& S, const float (&acc)[N], int slot) {
    static_assert(N * WAVES * 16 <= 6 * MW * 64, "S.red holds the partials");
    const int lane = my_tid() % 64;
    if (slot >= 0 && lane < 16) {
#pragma unroll
        for (int b = 0; b < N; ++b) S.red[(b * 16 + lane) * WAVES + slot] = acc[b];
    }
    lds_barrier();
}
template <int NWV>
__device__ __forceinline__ float red_sum16(const Shared& S, int b) {
    static_assert(NWV % 4 == 0 && NWV <= WAVES && WAVES % 4 == 0, "whole 16-byte reads of a row");
    const float4* r = (const float4*)(S.red + (b * 16 + (unsigned)my_tid() % 16u) * WAVES);
    float4 v[NWV / 4];
#pragma unroll
    for (int i = 0; i < NWV / 4; ++i) v[i] = r[i];
    float t = v[0].x;
    t += v[0].y;
    t += v[0].z;
    t += v[0].w;
#pragma unroll
    for (int i = 1; i < NWV / 4; ++i) {
        t += v[i].x;
        t += v[i].y;
        t += v[i].z;
        t += v[i].w;
    }
    return t;
}

// ------------------------------------------------------------------------------------------
// Stage timeline of the last step of a launch (per workgroup, per layer, 32 event slots; steady
// clock), compiled only with -DICUA_PERSIST_TRACE for profiling builds.  PK_TRACE is recorded by
// math thread 0, PK_TRACE_X by exchange thread 0.
#ifdef ICUA_PERSIST_TRACE
__device__ uint64_t g_trace[NWG][MAX_LAYERS + 1][32];
#define PK_TRACE_AT(layer, ev, t0)                                                            \
    do {                                                                                      \
        if (step == a.nsteps - 1 && my_tid() == (t0)) g_trace[w][layer][ev] = wall_clock64(); \
    } while (0)
#else
#define PK_TRACE_AT(layer, ev, t0) \
    do {                           \
    } while (0)
#endif
#define PK_TRACE(layer, ev) PK_TRACE_AT(layer, ev, 0)
#define PK_TRACE_X(layer, ev) PK_TRACE_AT(layer, ev, MT)

// The decode loop of one role (MATH: waves 0-3, else waves 4-7): a.nsteps single-token steps.
// Each role is compiled as its own copy of the loop, so the register allocator never has to fit
// the math waves' weight tiles and the exchange waves' poll buffers side by side.  Both copies
// execute the same sequence of workgroup barriers (s_barrier counts waves, not call sites), so
// they stay in lockstep.  A commit that forces a grammar pair ends the loop with the pair pending
// (control block n = 2): the pair runs as one two-row pass (decode_pass_loop) in the next launch.
template <int FMT, bool MATH>
__device__ __forceinline__ void decode_loop(const PersistArgs& a, Shared& S, uint8_t* wdb, int w, int pos, int stp) {
    constexpr bool F16 = FMT == FMT_F16;  // f16 tiles stream through their stages (stage_f16 above)
    // The slice-streaming form (f16 and q8 weights): every wave takes a K-slice of each stage's
    // blocks; q4 blocks are held whole by the math waves.
    constexpr bool SL = F16 || FMT == FMT_Q8;
    constexpr int SF = SL ? FMT : FMT_Q8;               // slice tile format (unused by q4)
    constexpr int SCHK = F16 ? F16_CHK : 64;            // K per 1 KiB chunk of a slice
    constexpr int XW = WAVES - MW;        // exchange waves
    constexpr int CHK = (FMT == FMT_Q4) ? 128 : 64;
    constexpr int CW2 = H / CHK / MW;   // chunks per math wave, K = 2048
    constexpr int NRB = VOCAB / 16;     // lm_head row blocks
    constexpr int CW8 = H / CHK / WAVES;  // lm_head chunks per wave (all eight waves)
    constexpr int LM_DEPTH = 4;           // lm_head blocks in flight per wave
    constexpr int LM_BLOCKS = (NRB + NWG - 1) / NWG;  // 38 block slots per workgroup
    uint64_t* ll = a.ll;
    unsigned* err = (unsigned*)a.ll + ERRW;
    State* st = a.st;
    const int maxsteps = st->maxsteps, eos0 = st->eos0, eos1 = st->eos1, maxctx = st->maxctx;
    const bool grammar = (st->flags & STATE_FLAG_GRAMMAR) != 0;
    const int L = a.nlayers;
    float nreg[8];  // math threads: norm weights of the next normed stage (8 each)
    if (MATH) load_norm8(nreg, a.layers[0].attn_norm + my_tid() * 8);
    // Math waves: the two QKV blocks (workgroups 128..255) or the O block (workgroups 0..127) of
    // the current layer.
    WB<FMT, CW2> wx[2];
    // f16 / q8: the tiles of the QKV block, gate|up blocks and down half-block, requested a stage
    // ahead where the registers are free: the QKV block after the previous down publish; gate|up
    // by the O workgroups' exchange waves two blocks at the attention-output poll and one after
    // their O products, by every other wave after its attention partial, merge or O stage; the
    // down half-block's slices after the SwiGLU publish.
    constexpr int S_CPW = H / SCHK / WAVES, S_CPWD = FFH / SCHK / WAVES, S_CPWO = H / SCHK / XW;
    // q8: the exchange waves also request their QKV slices of the next layer at the down publish
    // (648 against 662 us per token at 4k context), so every wave multiplies a slice; f16 exchange
    // wave slices spill there, and the f16 math waves hold the whole block instead.
    constexpr bool QKV_AHEAD_ALL = FMT == FMT_Q8;
    // q8: workgroups 128..223 hold their gate|up requests until their KV group's last split
    // partial is out, as the q4 form holds its bulk requests there (642 against 646 us per token;
    // the f16 form measured 832 against 824 with the hold).
    constexpr bool GU_HOLD = FMT == FMT_Q8;
    // q8: the O block is multiplied by all eight waves (the math waves' slices requested after
    // their attention partial; 639 against 642 us per token); the f16 math waves' share spills,
    // so there the four exchange waves take it.
    constexpr bool O_ALL = FMT == FMT_Q8;
    // f16: the math waves hold the whole QKV block (16 chunks each); q8: every wave a slice.
    SliceTiles<SF, 1, (F16 ? 2 * S_CPW : S_CPW)> wqf;
    SliceTiles<SF, 3, S_CPW> wgf;
    SliceTiles<SF, 1, S_CPWD> wdf;
    __syncthreads();

    for (int step = 0; step < a.nsteps; ++step) {
        if (pos + 1 > maxctx) break;  // the commit stops earlier; guards the cache row
        if (!SL && MATH) {
            wx[0].forget();
            wx[1].forget();
        }
        if constexpr (SL) {
            if (MATH || QKV_AHEAD_ALL) wqf.load(a.layers[0].wqkv, a.layers[0].wqkv_sb, {w}, H, wave_id(), my_tid() % 64);
        }
        if (!SL && MATH && w >= NWG / 2) {  // layer 0's QKV blocks (no x poll follows at layer 0)
            wx[0].load(a.layers[0].wqkv, a.layers[0].wqkv_sb, w - NWG / 2, H, wave_id(), my_tid() % 64);
            wx[1].load(a.layers[0].wqkv, a.layers[0].wqkv_sb, w, H, wave_id(), my_tid() % 64);
        }
        for (int l = 0; l < L; ++l) {
            const LayerPtrs& P = a.layers[l];
            const unsigned r = (unsigned)(step * L + l);  // round of this layer
            const int tid = my_tid(), lane = tid % 64, wave = wave_id();
            constexpr bool math = MATH;
            const int mw = wave;  // math wave index (valid when math)

            // Attention geometry of this workgroup: KV group g, split s.  The pos + 1 rows of the
            // group (rows < pos and the new row) are spread evenly over the 32 splits; the split
            // holding row pos writes it.  Only rows < pos are loaded from the cache.
            const int g = w % NKV, s = w / NKV;
            const int tot = pos + 1;
            const int chunk = (tot + ATT_SPLITS - 1) / ATT_SPLITS;
            const int j0 = min(s * chunk, tot), j1 = min(j0 + chunk, tot);
            const bool tail = (j0 <= pos) && (pos < j1);
            const int nprior = max(0, min(j1, pos) - j0);
            const int ntot = j1 - j0;
            const uint16_t* kb = a.kv + ((size_t)(l * 2 + 0) * NKV + g) * a.maxctx * HD;
            const uint16_t* vb = a.kv + ((size_t)(l * 2 + 1) * NKV + g) * a.maxctx * HD;
            const int quad = tid / 16, ql = tid % 16;  // math threads: 16 quarter-waves, 8 dims per lane

            // Math-wave register tiles: each is requested while the exchange waves wait for the
            // input of its stage or of an earlier one.  The down half-block streams into LDS.
            WB<FMT, CW2> wgu[3];
            if constexpr (SL) {  // slices loaded under role conditions: last layer's values are dead
                wgf.forget();
                wdf.forget();
                if (!math && !QKV_AHEAD_ALL) wqf.forget();
            }

            // ---------------- QKV: row blocks w - 128 and w (workgroups 128..255) ------------
            // Workgroups 0..127 need no x here.  Loads issued just before the x poll of
            // workgroups 128..255 would queue ahead of it on their CU: their QKV blocks are
            // requested during the previous layer's down stage (layer 0's at the start of the
            // step) and their K/V rows after the QKV publish.
            const bool qkv_wg = SL || w >= NWG / 2;  // f16 / q8: one block per workgroup
            PK_TRACE(l, 0);
            uint4 kt[ATT_NT][4], vr[ATT_SPQ];
            float qn0 = 0.f, qn1 = 0.f, kn0 = 0.f, kn1 = 0.f, rc = 0.f, rs = 0.f;
            // Exchange waves poll the stage input first; math waves skip that branch and issue
            // their loads at once.  Keeping the loads after the poll in program order lets the
            // poll's registers and the weight tiles share the register file.
            bool ok_in = true;
            if (l > 0 && !math && qkv_wg) ok_in = poll_sum<H / 2 / CT>(ll + XP, ll + XDP, 2 * r, S.vec, err);
            if (math) {
                // This layer's norm weights into LDS; then the QKV blocks and the loads for the
                // stages ahead: the first block of K/V rows, the per-head norms and the rope row,
                // the O block and the mlp norm.
#pragma unroll
                for (int i = 0; i < 8; ++i) S.nw[tid * 8 + i] = nreg[i];
                if (!SL && !qkv_wg) {
                    wx[0].load(P.wo, P.wo_sb, w, H, mw, lane);
                    load_kv_block(kt, vr, kb, vb, j0, 0, nprior, tid);
                    // The lower down half-block of row block w into LDS: it lands long before the
                    // x' poll that a later request would delay.
                    wd_request<FMT>(wdb, P.wd, P.wd_sb, w, 0, mw, lane);
                }
                const float* rope = a.rope + (size_t)pos * 128;
                qn0 = P.q_norm[lane];
                qn1 = P.q_norm[lane + 64];
                kn0 = P.k_norm[lane];
                kn1 = P.k_norm[lane + 64];
                rc = rope[2 * lane];
                rs = rope[2 * lane + 1];
                load_norm8(nreg, P.mlp_norm + tid * 8);
            }
            if (sync_failed(S, !ok_in)) return;
            PK_TRACE_X(l, 1);
            if constexpr (SL) {
                // Row block w, in flight since the previous layer's down publish: held whole by the
                // f16 math waves (the exchange waves' slices, requested after the x poll, landed
                // last: 822 against 818 us per token at 4k context), as slices by every q8 wave.
                stage_slices<FMT, H>(S, l == 0 ? S.emb : S.vec, true);
                float acc[1] = {0.f};
                if (!F16 || math) wqf.mac(S, wave, lane, acc);
                PK_TRACE(l, 28);
                red_store16<1>(S, acc, F16 && !math ? -1 : wave);
                if (wave == 0) {  // rows 2i, 2i + 1 of the block in packet i (even lanes)
                    const float y0 = (F16 ? red_sum16<MW>(S, 0) : red_sum16<WAVES>(S, 0)) * norm_scale<H>(S);
                    const float n0 = xor1(y0);
                    if (lane < 16 && !(lane & 1)) st64(ll + QKVP + w * 8 + lane / 2, pack2(y0, n0, r + 1));
                }
                PK_TRACE(l, 30);
                if (math) load_kv_block(kt, vr, kb, vb, j0, 0, nprior, tid);
            } else if (qkv_wg) {
                stage_c<FMT, H>(S, l == 0 ? S.emb : S.vec, true);
                float acc[2] = {0.f, 0.f}, y[2] = {0.f, 0.f};
                if (math) mac_blocks<FMT, CW2, 2>(S, wx, mw, lane, acc);
                PK_TRACE(l, 28);
                reduce_math_n<MATH, 2>(S, acc, y);
                if (wave == 0) {  // rows 2i, 2i + 1 of a block in packet i (even lanes)
                    const float rs = norm_scale<H>(S);
                    y[0] *= rs;
                    y[1] *= rs;
                    const float n0 = xor1(y[0]), n1 = xor1(y[1]);
                    if (lane < 16 && !(lane & 1)) {
                        st64(ll + QKVP + (w - NWG / 2) * 8 + lane / 2, pack2(y[0], n0, r + 1));
                        st64(ll + QKVP + w * 8 + lane / 2, pack2(y[1], n1, r + 1));
                    }
                }
                PK_TRACE(l, 30);
                if (math) load_kv_block(kt, vr, kb, vb, j0, 0, nprior, tid);
            }
            PK_TRACE(l, 2);

            // ---------------- attention: group g, split s ----------------------------------
            {
                bool ok = true;
                if (!math)  // q heads 2g, 2g+1 -> vec[0..255], k -> vec[256..383], v -> vec[384..511]
                    ok = poll_map<1>(
                        ll + QKVP, 2 * HD,
                        [&](int k) {  // packet of gathered elements 2k, 2k + 1
                            const int e = 2 * k;
                            return (e < 2 * HD ? 2 * g * HD + e
                                               : e < 3 * HD ? H + g * HD + (e - 2 * HD)
                                                            : H + NKV * HD + g * HD + (e - 3 * HD)) / 2;
                        },
                        r + 1, S.vec, err);
                if (sync_failed(S, !ok)) return;
            }
            PK_TRACE_X(l, 3);
            if (math) {
                if (wave < 2) {
                    float x0 = S.vec[wave * HD + lane], x1 = S.vec[wave * HD + lane + 64];
                    norm_rope(x0, x1, qn0, qn1, rc, rs);
                    // 1/sqrt(128) and log2(e): scores come out in base-2 units, so every softmax
                    // exponential of this split and of the merge is one v_exp_f32.
                    const float qscale = (1.0f / sqrtf((float)HD)) * 1.4426950408889634f;
                    const float qa = x0 * qscale, qb = x1 * qscale;
                    const uint16_t ha = f2h(qa), hb = f2h(qb);
                    S.qf[wave][lane] = ha;
                    S.qf[wave][lane + 64] = hb;
                    S.qf[2 + wave][lane] = f2h(qa - h2f(ha));
                    S.qf[2 + wave][lane + 64] = f2h(qb - h2f(hb));
                } else if (wave == 2 && tail) {
                    float k0 = S.vec[2 * HD + lane], k1 = S.vec[2 * HD + lane + 64];
                    norm_rope(k0, k1, kn0, kn1, rc, rs);
                    S.ktail[0][lane] = f2h(k0);
                    S.ktail[0][lane + 64] = f2h(k1);
                    S.vtail[0][lane] = f2h(S.vec[3 * HD + lane]);
                    S.vtail[0][lane + 64] = f2h(S.vec[3 * HD + lane + 64]);
                }
            }
            __syncthreads();
            if (tail && !math && tid < MT + 128) {
                // The new cache row (fp16), device-scope stores by exchange threads, acknowledged
                // before this workgroup publishes its partials.
                const int c = tid - MT;
                const uint16_t* src = c < 64 ? S.ktail[0] : S.vtail[0];
                uint16_t* dst = (uint16_t*)(c < 64 ? kb : vb) + (size_t)pos * HD;
                const int d = 2 * (c % 64);
                const uint32_t v = (uint32_t)src[d] | ((uint32_t)src[d + 1] << 16);
                __hip_atomic_store((uint32_t*)(dst + d), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_s_waitcnt(0);
            }
            {
                // Scores on the matrix cores: per block, each math wave multiplies the query rows
                // (the fp16 hi and lo parts of both heads, replicated over the 16 A rows) with its
                // ATT_NT tiles of 16 cache rows (v_mfma_f32_16x16x32_f16, four products of 32 dims
                // each); every lane then holds the scores of its column's slot.  The online softmax
                // runs per wave (every lane holds the wave's running maximum and sum); the
                // probabilities move through LDS (wave-local) to the P.V layout, where each
                // quarter-wave takes 9 V rows, 8 dims per lane.
                float m_run[2] = {-__builtin_inff(), -__builtin_inff()}, l_run[2] = {0.f, 0.f};
                float o[2][8];
#pragma unroll
                for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                    for (int d = 0; d < 8; ++d) o[hh][d] = 0.f;
                PK_TRACE(l, 21);
                if (math) {
                    const int c = lane & 15, kq = lane >> 4;
#ifdef ICUA_PERSIST_TRACE
                    __builtin_amdgcn_s_waitcnt(0);
                    PK_TRACE(l, 25);
#endif
                    for (int b0 = 0; b0 < ntot; b0 += ATT_BLOCK) {
                        const int nb = min(ATT_BLOCK, ntot - b0);
                        if (b0 > 0) load_kv_block(kt, vr, kb, vb, j0, b0, nprior, tid);
                        // The new row (block slot pos - j0 - b0) comes from LDS, not from the cache.
                        if (tail) {
                            const int pnew = pos - j0 - b0;
#pragma unroll
                            for (int T = 0; T < ATT_NT; ++T)
                                if (4 * T + (c >> 2) < ATT_SPQ && att_slot(T, c, mw) == pnew) {
#pragma unroll
                                    for (int j = 0; j < 4; ++j) kt[T][j] = *(const uint4*)(S.ktail[0] + 32 * j + 8 * kq);
                                }
#pragma unroll
                            for (int i = 0; i < ATT_SPQ; ++i)
                                if (quad + ATT_QW * i == pnew) vr[i] = *(const uint4*)(S.vtail[0] + 8 * ql);
                        }
                        // D[variant][slot]: lane l holds rows 4 (l / 16) + r, i.e. variant r.
                        float sc[2][ATT_NT];
#pragma unroll
                        for (int T = 0; T < ATT_NT; ++T) {
                            f32x4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int j = 0; j < 4; ++j)  // A: the query rows (read from LDS for each tile)
                                D = __builtin_amdgcn_mfma_f32_16x16x32_f16(*(const h8*)&S.qf[lane & 3][32 * j + 8 * kq],
                                                                           as_h8(kt[T][j]), D, 0, 0, 0);
                            const bool ok = 4 * T + (c >> 2) < ATT_SPQ && att_slot(T, c, mw) < nb;
                            sc[0][T] = ok ? D[0] + D[2] : -__builtin_inff();
                            sc[1][T] = ok ? D[1] + D[3] : -__builtin_inff();
                        }
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            float mb = sc[hh][0];
#pragma unroll
                            for (int T = 1; T < ATT_NT; ++T) mb = fmaxf(mb, sc[hh][T]);
                            // mb is finite as soon as the wave has seen one valid slot.
                            mb = fmaxf(max16(mb), m_run[hh]);
                            const float corr = (m_run[hh] == -__builtin_inff()) ? 0.f : ex2(m_run[hh] - mb);
                            float ls = 0.f;
#pragma unroll
                            for (int T = 0; T < ATT_NT; ++T) {
                                sc[hh][T] = (sc[hh][T] == -__builtin_inff()) ? 0.f : ex2(sc[hh][T] - mb);
                                ls += sc[hh][T];
                            }
                            l_run[hh] = l_run[hh] * corr + sum16(ls);
                            m_run[hh] = mb;
#pragma unroll
                            for (int d = 0; d < 8; ++d) o[hh][d] *= corr;
                            if (lane < 16) {
#pragma unroll
                                for (int T = 0; T < ATT_NT; ++T) S.pw[mw][0][hh][c & 3][4 * T + (c >> 2)] = sc[hh][T];
                            }
                        }
                        // The probabilities of this wave's slots were written by its own lanes 0-15:
                        // a wave's LDS accesses complete in order, so no barrier is needed.
                        __builtin_amdgcn_wave_barrier();
                        PK_TRACE(l, 27);
#pragma unroll
                        for (int i = 0; i < ATT_SPQ; ++i) {
                            const float p0 = S.pw[mw][0][0][kq][i], p1 = S.pw[mw][0][1][kq][i];
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
                        __builtin_amdgcn_wave_barrier();
                    }
                    PK_TRACE(l, 29);
                    // The wave's 4 quarter-waves (lanes l, l ^ 16, l ^ 32, l ^ 48 hold the same
                    // dims) share the running maximum: their sums add.
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int d = 0; d < 8; ++d) o[hh][d] = sum_x4(o[hh][d]);
                    if (lane < 16) {
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                            for (int d = 0; d < 8; ++d) S.ored[mw][hh][8 * ql + d] = o[hh][d];
                    }
                    if (lane == 0) {
                        S.misc[16 + 4 * mw] = m_run[0];
                        S.misc[17 + 4 * mw] = m_run[1];
                        S.misc[18 + 4 * mw] = l_run[0];
                        S.misc[19 + 4 * mw] = l_run[1];
                    }
                }
                PK_TRACE(l, 22);
                __syncthreads();
                if (math) {
                    // The split's partial: the 4 waves rescaled to their common max.
                    uint64_t* part = ll + PARTP + (size_t)(g * ATT_SPLITS + s) * 2 * PART2;
                    const int hh = tid / HD, d = tid % HD;
                    float mx = -__builtin_inff();
#pragma unroll
                    for (int ww = 0; ww < MW; ++ww) mx = fmaxf(mx, S.misc[16 + 4 * ww + hh]);
                    float acc = 0.f, lsum = 0.f;
#pragma unroll
                    for (int ww = 0; ww < MW; ++ww) {
                        const float mwv = S.misc[16 + 4 * ww + hh];
                        const float f = (mwv == -__builtin_inff()) ? 0.f : ex2(mwv - mx);
                        acc = fmaf(S.ored[ww][hh][d], f, acc);
                        lsum = fmaf(S.misc[18 + 4 * ww + hh], f, lsum);
                    }
                    // o pairs (even lanes), then (l, m) with the maximum exact.
                    const float acc_n = xor1(acc);
                    if (!(d & 1)) st64(part + hh * PART2 + d / 2, pack2(acc, acc_n, r + 1));
                    if (d == 0) st64(part + hh * PART2 + HD / 2, pack2(lsum, mx, r + 1));
                }
                PK_TRACE(l, 20);
            }
            PK_TRACE(l, 4);
            // f16 / q8: workgroups 0..127 request their O block now (f16: the exchange waves, 64 KiB;
            // q8: every wave its slice); it lands during the merge and is multiplied after the
            // attention-output poll.
            SliceTiles<SF, 1, (O_ALL ? S_CPW : S_CPWO)> wof;
            if constexpr (SL) {
                if ((O_ALL || !math) && w < H / 16) wof.load(P.wo, P.wo_sb, {w}, H, O_ALL ? wave : wave - MW, lane);
                // Workgroups 128..223 (no O, no merge) idle until the x' poll: their exchange waves
                // request all of their gate|up slices now (q8: once their KV group's partials are
                // out, below; the mergers' after the merge: in flight during their partials poll,
                // they would delay it).
                if (!GU_HOLD && !math && w >= H / 16 && w < MERGER0) wgf.load(P.wgu, P.wgu_sb, {3 * w, 3 * w + 1, 3 * w + 2}, H, wave, lane);
            }

            // ---------------- merge of group g: workgroups 224..255 ------------------------
            // Split s = 28 + p of group g (workgroup 224 + 8p + g, no O / down work) merges part
            // p = 0..3 of the group's output: head 2g + p / 2, elements 64 (p % 2) .. + 63.
            if (w >= MERGER0) {
                const int p = s - (ATT_SPLITS - MERGE_PARTS), hh = p / 2, d0 = 64 * (p % 2);
                float* pl = (float*)S.A;  // [32][64 + 2]: o elements d0.., l, m of head hh per split
                const uint64_t* gp = ll + PARTP + (size_t)g * GROUP_PARTS;
                bool ok = true;
                if (!math)
                    ok = poll_map<(ATT_SPLITS * 33 + CT - 1) / CT>(
                        gp, ATT_SPLITS * 33,
                        [&](int k) {
                            const int sj = k / 33, e = k % 33;
                            return (sj * 2 + hh) * PART2 + (e < 32 ? d0 / 2 + e : HD / 2);
                        },
                        r + 1, pl, err);
                if (sync_failed(S, !ok)) return;
                PK_TRACE_X(l, 5);
                // Split weights exp(m_s - max) and the normaliser (math wave 0, one lane per split).
                if (math && wave == 0) {
                    const int sl = lane % ATT_SPLITS;
                    const float m = pl[sl * 66 + 65];
                    const float mx = wave_max(m);  // finite: the split holding row pos is never empty
                    const float wgt = (m == -__builtin_inff()) ? 0.f : ex2(m - mx);
                    const float lw = wave_sum(lane < ATT_SPLITS ? wgt * pl[sl * 66 + 64] : 0.f);
                    if (lane < ATT_SPLITS) S.sc[0][lane] = wgt;
                    if (lane == 0) S.misc[0] = 1.0f / lw;
                }
                __syncthreads();
                // Weighted sum of the split outputs: thread (q, e) over splits 8q .. 8q + 7, the
                // eight quarters combined through LDS.
                {
                    const int q = tid / 64, e = tid % 64;
                    float O = 0.f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const int sj = q * 4 + j;
                        O = fmaf(S.sc[0][sj], pl[sj * 66 + e], O);
                    }
                    float* q8 = &S.ored[0][0][0];  // [8][64]
                    q8[q * 64 + e] = O;
                    __syncthreads();
                    if (tid < 64) {
                        float t = 0.f;
#pragma unroll
                        for (int qq = 0; qq < 8; ++qq) t += q8[qq * 64 + tid];
                        const float v = t * S.misc[0], vn = xor1(v);
                        if (!(tid & 1)) st64(ll + ATTNP + ((2 * g + hh) * HD + d0 + tid) / 2, pack2(v, vn, r + 1));
                    }
                }
                PK_TRACE(l, 17);
                __syncthreads();  // the partials in S.A are read before the next staging
                if constexpr (SL) {
                    if (!math) wgf.load(P.wgu, P.wgu_sb, {3 * w, 3 * w + 1, 3 * w + 2}, H, wave, lane);
                }
                PK_TRACE(l, 6);
            }

            // ---------------- O projection + residual: workgroups 0..127 -------------------
            // The gate|up blocks are requested here, a stage early, by every workgroup.  The
            // residual of the O rows is xown (previous x + lower-half down sums) + xhi (the
            // upper-half sums, long published): the same two terms every x reader adds.
            //
            // Workgroups 128..223 (no O, no merge) request their next stages' weights only once
            // their KV group's split partials are all out: issued as their attention ends, these
            // ~10 MB would queue at the memory controllers ahead of the mergers' polls of those
            // partials.  Which split publishes last varies (the one holding the new cache row
            // also waits for that row's acknowledgement): their math waves' wave 0 watches the
            // (l, m) packets of all 32, and nothing else of theirs is in flight then.
            if (((!SL && math) || GU_HOLD) && w >= NWG / 2 && w < MERGER0) {
                // Wave 0 watches; the other waves taking part wait for it in LDS.
                if (wave == 0)
                    watch_partials(S, ll + PARTP + (size_t)g * ATT_SPLITS * 2 * PART2 + HD / 2, 2 * PART2, tag4(r + 1),
                                   (int)r + 1, err, lane);
                while (__hip_atomic_load(&S.go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != (int)r + 1)
                    __builtin_amdgcn_s_sleep(1);
                if constexpr (GU_HOLD) {
                    if (!math) wgf.load(P.wgu, P.wgu_sb, {3 * w, 3 * w + 1, 3 * w + 2}, H, wave, lane);
                }
            }
            {
                bool ok = true;
                if (w < H / 16 && !math) {
                    if (l > 0)
                        ok = poll_vec<1>(ll + XDP + w * 8, 8, 2 * r, S.xhi[0], err);
                    else if (tid - MT < 16)
                        S.xhi[0][tid - MT] = 0.f;
                    ok = ok && poll_vec<H / 2 / CT>(ll + ATTNP, H / 2, r + 1, S.vec, err);
                }
                if (!SL && math) {
#pragma unroll
                    for (int j = 0; j < 3; ++j) wgu[j].load(P.wgu, P.wgu_sb, 3 * w + j, H, mw, lane);
                }
                if (w < H / 16 && sync_failed(S, !ok)) return;
            }
            if (w < H / 16) {
                PK_TRACE_X(l, 7);
                float y = 0.f;
                if constexpr (SL) {
                    // Two gate|up blocks go out beside the O block's registers, the third once the O
                    // products are done (all three before them: 860 against 834 us per token at 4k
                    // context, one before them: 836).
                    if (!math) wgf.template load<0, 2>(P.wgu, P.wgu_sb, {3 * w, 3 * w + 1, 3 * w + 2}, H, wave, lane);
                    stage_slices<FMT, H>(S, S.vec, false);
                    float acc1[1] = {0.f};
                    if (O_ALL || !math) wof.mac(S, O_ALL ? wave : wave - MW, lane, acc1);
                    if (!math) wgf.template load<2, 3>(P.wgu, P.wgu_sb, {3 * w, 3 * w + 1, 3 * w + 2}, H, wave, lane);
                    red_store16<1>(S, acc1, O_ALL ? wave : math ? -1 : wave - MW);
                    y = O_ALL ? red_sum16<WAVES>(S, 0) : red_sum16<XW>(S, 0);
                } else {
                    stage_c<FMT, H>(S, S.vec, false);
                    float acc1[1] = {0.f};
                    if (math) mac_blocks<FMT, CW2, 1>(S, wx, mw, lane, acc1);
                    y = reduce_math<MATH>(S, acc1[0]);
                }
                if (wave == 0) {  // the owner keeps the residual as published (even rows rounded)
                    const float xn = lane < 16 ? (S.xown[0][lane] + S.xhi[0][lane]) + y : 0.f;
                    const float xo = xor1(xn);
                    if (lane < 16) {
                        S.xown[0][lane] = (lane & 1) ? xn : q19(xn);
                        if (!(lane & 1)) st64(ll + XP + w * 8 + lane / 2, pack2(xn, xo, 2 * r + 1));
                    }
                }
                PK_TRACE(l, 8);
            }
            // Workgroups 128..255 request the upper down half-block and the next layer's QKV
            // blocks here, where they wait for no stage input (workgroups 0..127 run O): loads
            // issued later would queue ahead of their x' and h polls.
            // f16: the math waves' gate|up slices (after the O publish on workgroups 0..127).  One
            // block requested earlier, at the attention partial, measured slower (868 against 855 us
            // per token at 4k context), and so did one at the start of the O stage (864 against 857).
            if (SL && math) wgf.load(P.wgu, P.wgu_sb, {3 * w, 3 * w + 1, 3 * w + 2}, H, wave, lane);
            if (!SL && math && qkv_wg) {
                wd_request<FMT>(wdb, P.wd, P.wd_sb, w - NWG / 2, 1, mw, lane);
                wx[0].forget();
                wx[1].forget();
                if (l + 1 < L) {
                    const LayerPtrs& Pn = a.layers[l + 1];
                    wx[0].load(Pn.wqkv, Pn.wqkv_sb, w - NWG / 2, H, mw, lane);
                    wx[1].load(Pn.wqkv, Pn.wqkv_sb, w, H, mw, lane);
                }
            }

            // ---------------- RMSNorm + gate|up + SwiGLU: blocks 3w .. 3w + 2 --------------
            {
                bool ok = true;
                if (!math) ok = poll_vec<H / 2 / CT>(ll + XP, H / 2, 2 * r + 1, S.vec, err);
                if (math) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) S.nw[tid * 8 + i] = nreg[i];
                    // The next layer's attention norm, or the final norm.
                    load_norm8(nreg, (l + 1 < L ? a.layers[l + 1].attn_norm : a.final_norm) + tid * 8);
                }
                if (sync_failed(S, !ok)) return;
                PK_TRACE_X(l, 9);
                float acc[3] = {0.f, 0.f, 0.f}, y[3] = {0.f, 0.f, 0.f};
                if constexpr (SL) {
                    // Blocks 3w .. 3w + 2 (192 KiB), every wave's slices in flight since its O work
                    // or attention ended.
                    stage_slices<FMT, H>(S, S.vec, true);
                    PK_TRACE(l, 13);
                    wgf.mac(S, wave, lane, acc);
                    PK_TRACE(l, 26);
                    red_store16<3>(S, acc, wave);
                    if (wave == 0) {
#pragma unroll
                        for (int j = 0; j < 3; ++j) y[j] = red_sum16<WAVES>(S, j);
                    }
                } else {
                    stage_c<FMT, H>(S, S.vec, true);
                    PK_TRACE(l, 13);
                    if (math) mac_blocks<FMT, CW2, 3>(S, wgu, mw, lane, acc);
                    PK_TRACE(l, 26);
                    reduce_math_n<MATH, 3>(S, acc, y);
                }
                PK_TRACE(l, 14);
                if (wave == 0) {
                    const float rs = norm_scale<H>(S);
#pragma unroll
                    for (int j = 0; j < 3; ++j) {
                        // Block 3w + j: gate units 8 (3w + j) + 0..7 in lanes 0-7, their up rows in 8-15.
                        y[j] *= rs;
                        const float hv = swiglu(y[j], xor8(y[j])), hn = xor1(hv);
                        if (lane < 8 && !(lane & 1)) st64(ll + HP + (3 * w + j) * 4 + lane / 2, pack2(hv, hn, r + 1));
                    }
                }
                PK_TRACE(l, 10);
                if constexpr (SL)  // every wave's down slices (the gate|up slices are spent)
                    wdf.load(P.wd, P.wd_sb, {w % (NWG / 2)}, FF, (w / (NWG / 2)) * WAVES + wave, lane);
            }

            // ---------------- down: K half w / 128 of row block w % 128 --------------------
            {
                const int rb = w % (NWG / 2), half = w / (NWG / 2);
                bool ok = true;
                if (!math) ok = poll_vec<FFH / 2 / CT>(ll + HP + half * (FFH / 2), FFH / 2, r + 1, S.vec, err);
                if (!SL && math && !qkv_wg) {
                    wx[0].forget();
                    wx[1].forget();
                }
                if (sync_failed(S, !ok)) return;
                PK_TRACE_X(l, 11);
                float y = 0.f;
                if constexpr (SL) {
                    // K half `half` of row block rb (96 KiB): chunks half * 96 .. of the block.
                    stage_slices<FMT, FFH>(S, S.vec, false);
                    PK_TRACE(l, 18);
                    float acc1[1] = {0.f};
                    wdf.mac(S, wave, lane, acc1);
                    PK_TRACE(l, 24);
                    red_store16<1>(S, acc1, wave);
                    y = red_sum16<WAVES>(S, 0);
                } else {
                stage_c<FMT, FFH>(S, S.vec, false);
                PK_TRACE(l, 18);
                float yd = 0.f;
                if (math) {
                    // This wave's down-block requests have landed (and the QKV prefetch, issued
                    // after them, too: vector memory counts complete in order).
                    __builtin_amdgcn_s_waitcnt(0);
                    __atomic_signal_fence(__ATOMIC_SEQ_CST);
                    PK_TRACE(l, 23);
                    yd = wd_mac_lds<FMT>(S, wdb, mw, lane);
                    PK_TRACE(l, 24);
                }
                y = reduce_math<MATH>(S, yd);
                }
                PK_TRACE(l, 19);
                if (wave == 0) {
                    const float v = lane < 16 ? (half == 0 ? S.xown[0][lane] + y : y) : 0.f;
                    const float vn = xor1(v);
                    if (lane < 16) {
                        if (half == 0) S.xown[0][lane] = (lane & 1) ? v : q19(v);
                        if (!(lane & 1)) st64(ll + (half == 0 ? XP : XDP) + rb * 8 + lane / 2, pack2(v, vn, 2 * r + 2));
                    }
                }
                PK_TRACE(l, 12);
                if constexpr (SL) {  // the math waves' (q8: every wave's) QKV slices of the next layer
                    if ((math || QKV_AHEAD_ALL) && l + 1 < L) wqf.load(a.layers[l + 1].wqkv, a.layers[l + 1].wqkv_sb, {w}, H, wave, lane);
                }
            }
        }

        // ---------------- final RMSNorm + lm_head + per-workgroup argmax ---------------------
        {
            const int tid = my_tid(), lane = tid % 64, wave = wave_id();
            constexpr bool math = MATH;
            const unsigned r_last = (unsigned)(step * L + L - 1);
            PK_TRACE(L, 0);
            // All eight waves stream the blocks w + k * 256 (chunks wave * CW8 ..), LM_DEPTH in
            // flight per wave; the exchange waves issue theirs once their poll is done.  Each
            // wave's per-block partial sums go to LDS; one reduction and argmax at the end.
            bool ok = true;
            if (!math) ok = poll_sum<H / 2 / CT>(ll + XP, ll + XDP, 2 * r_last + 2, S.vec, err);
            if (math) {
#pragma unroll
                for (int i = 0; i < 8; ++i) S.nw[tid * 8 + i] = nreg[i];
            }
            float* plm = (float*)wdb;  // [LM_BLOCKS][WAVES][16] partial sums
            if constexpr (F16) {
                // f16 embedding blocks (64 KiB): each wave's 8-chunk K-slice of blocks w + k * 256,
                // LM_DEPTH in flight, requested once x is in (a barrier before the staging would
                // otherwise wait for them).
                constexpr int CPW = H / F16_CHK / WAVES;
                WF<1, CPW> wl[LM_DEPTH];
                if (sync_failed(S, !ok)) return;
#pragma unroll
                for (int k = 0; k < LM_DEPTH; ++k) wl[k].load(a.E, {w + k * NWG}, H / F16_CHK, wave * CPW, lane);
                PK_TRACE_X(L, 1);
                stage_f16<H>(S, S.vec, true);
                for (int k0 = 0; k0 < LM_BLOCKS; k0 += LM_DEPTH) {
#pragma unroll
                    for (int k = 0; k < LM_DEPTH; ++k) {
                        const int kb = k0 + k, rb = w + kb * NWG;
                        float y1[1] = {0.f};
                        mac_f16(S, wl[k], wave * CPW, lane, y1);
                        if (rb < NRB && lane < 16) plm[(kb * WAVES + wave) * 16 + lane] = y1[0];
                        wl[k].load(a.E, {min(rb + LM_DEPTH * NWG, NRB - 1)}, H / F16_CHK, wave * CPW, lane);
                    }
                }
            } else {
            WB<FMT, CW8> wl[LM_DEPTH];
            // The exchange waves request their blocks once x is in; the math waves' requests
            // also wait for the barrier, so that no bulk load queues ahead of the x poll.
            if (!math) {
#pragma unroll
                for (int k = 0; k < LM_DEPTH; ++k) wl[k].load(a.E, a.Esb, w + k * NWG, H, wave, lane);
            }
            if (sync_failed(S, !ok)) return;
            if (math) {
#pragma unroll
                for (int k = 0; k < LM_DEPTH; ++k) wl[k].load(a.E, a.Esb, w + k * NWG, H, wave, lane);
            }
            PK_TRACE_X(L, 1);
            stage_c<FMT, H>(S, S.vec, true);
            QuadOps<FMT> lq[CW8 / 2];  // this wave's operand quads, the same for every block
#pragma unroll
            for (int p = 0; p < CW8 / 2; ++p) lq[p] = quad_load<FMT>(S, wave * CW8 + 2 * p, lane);
            // Every iteration issues the same refill (past the matrix it re-reads the last row
            // block, an L2 hit, and the sums of blocks past the matrix are dropped): with the
            // same loads on every path the compiler's waits stay exact, instead of draining every
            // block in flight before each block's scales are used.
            for (int k0 = 0; k0 < LM_BLOCKS; k0 += LM_DEPTH) {
#pragma unroll
                for (int k = 0; k < LM_DEPTH; ++k) {
                    const int kb = k0 + k, rb = w + kb * NWG;
                    float y = 0.f;
#pragma unroll
                    for (int p = 0; p < CW8 / 2; ++p)
                        y = quad_scale<FMT>(lq[p], quad_mfma<FMT>(lq[p], wl[k].wv[2 * p], wl[k].wv[2 * p + 1]),
                                            wl[k].sq[p], y);
                    y = quad_rows(y);
                    if (rb < NRB && lane < 16) plm[(kb * WAVES + wave) * 16 + lane] = y;
                    wl[k].load(a.E, a.Esb, min(rb + LM_DEPTH * NWG, NRB - 1), H, wave, lane);
                }
            }
            }
            __syncthreads();
            float best = -__builtin_inff();
            int besti = 0x7fffffff;
            const float rs = norm_scale<H>(S);
            for (int e = tid; e < LM_BLOCKS * 16; e += THREADS) {  // (block, row) pairs
                const int kb = e / 16, rw = e % 16;
                if (w + kb * NWG < NRB) {
                    const float* pp = plm + kb * WAVES * 16 + rw;
                    float y = 0.f;
#pragma unroll
                    for (int wv = 0; wv < WAVES; ++wv) y += pp[wv * 16];
                    argmax_merge(best, besti, y * rs, (w + kb * NWG) * 16 + rw);
                }
            }
            wave_argmax(best, besti);
            if (lane == 0) {
                S.misc[8 + wave] = best;
                S.imisc[8 + wave] = besti;
            }
            __syncthreads();
            if (tid == 0) {
                for (int wv = 1; wv < WAVES; ++wv) argmax_merge(best, besti, S.misc[8 + wv], S.imisc[8 + wv]);
                // (index << 4 | tag, value): the value exact, ids < 2^27 exact in the low word.
                const uint32_t lo = ((uint32_t)min(besti, 0x07FFFFFF) << 4) | tag4((unsigned)step + 1);
                st64(ll + LMP + w, (uint64_t)lo | ((uint64_t)as_u32(best) << 32));
            }
            PK_TRACE(L, 2);
            if (math) load_norm8(nreg, a.layers[0].attn_norm + tid * 8);  // for the next step
        }

        // ---------------- greedy commit, evaluated by every workgroup ------------------------
        {
            const int tid = my_tid(), lane = tid % 64, wave = wave_id();
            bool ok = true;
            if (!MATH) ok = poll_vec<NWG / CT>(ll + LMP, NWG, (unsigned)step + 1, S.vec, err);
            if (sync_failed(S, !ok)) return;
            PK_TRACE_X(L, 3);
            float bv = -__builtin_inff();
            int bi = 0x7fffffff;
            if (tid < NWG) {
                bv = S.vec[2 * tid + 1];
                bi = (int)(as_u32(S.vec[2 * tid]) >> 4);
            }
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
            int forced = -1;  // a forced pair's second token: the pair is the next launch's pass
            if (stp >= maxsteps) {  // nothing may be written past out_tokens[maxsteps - 1]
                stop = true;
            } else {
                const bool bad = tok < 0 || tok >= VOCAB;  // no finite logit (NaN model): stop on token 0
                if (bad) tok = 0;
                if (w == 0 && tid == 0) a.out_tokens[stp] = tok;
                stp += 1;
                pos += 1;
                stop = bad || tok == eos0 || tok == eos1 || (grammar && tok == 8) || stp >= maxsteps ||
                       pos + 2 > maxctx;
                // Grammar pairs: after a first-step action token, or after 11, the next token is
                // forced (7, or 220 after 11); it is committed now and fed after `tok`.
                if (!stop && grammar &&
                    ((stp == 1 && (tok == 3678 || tok == 7241 || tok == 12476 || tok == 10855 || tok == 11862 ||
                                   tok == 1339 || tok == 1472 || tok == 24769)) ||
                     tok == 11)) {
                    forced = tok == 11 ? 220 : 7;
                    if (w == 0 && tid == 0) a.out_tokens[stp] = forced;
                    stp += 1;
                    stop = stp >= maxsteps;  // the pair's pass would start at the step limit
                }
            }
            if (w == 0 && tid == 0) {
                st->pos = pos;
                st->step = stp;
                st->n = (forced >= 0 && !stop) ? 2 : 1;
                st->vis_offset = -1;
                st->logits_rows = 0;
                if (stop) st->done = 1;
            }
            if (stop) break;
            // Next token's embedding (Shaders.swift:464-476), in every workgroup.
            __syncthreads();  // every thread has read S.misc / S.imisc
            for (int i = tid; i < H; i += THREADS) S.emb[i] = dequant_tiled(FMT, a.E, a.Esb, (size_t)tok, i, H);
            __syncthreads();
            if (tid < 16 && w < H / 16) S.xown[0][tid] = S.emb[w * 16 + tid];
            if (w == 0 && (forced >= 0 || step == a.nsteps - 1)) {
                for (int i = tid; i < H; i += THREADS) a.x[i] = S.emb[i];  // residual row(s) for the next launch
                if (forced >= 0)
                    for (int i = tid; i < H; i += THREADS) a.x[H + i] = dequant_tiled(FMT, a.E, a.Esb, (size_t)forced, i, H);
            }
            PK_TRACE(L, 4);
            if (forced >= 0) break;  // the pair runs as the next launch's two-row pass
        }
    }
}

// The same stages for passes of NR token rows, used for a forced grammar pair (NR = 2,
// Shaders.swift:1537-1561: the reference's n = 2 pass, Shaders.swift:529-595 / 735-788 /
// 1304-1418): the two tokens at slots pos, pos + 1 go through every layer together, so each
// weight tile is streamed once for both rows.  Every GEMV stage stages NR rows and multiplies each
// against the same weight registers; the attention scores all NR rows' query heads in one
// matrix-core product (row 1 also sees slot pos + 1, row 0 does not); lm_head and the commit use
// the last row.  The packet areas hold NR copies of each vector (Pk<NR>).  The single-row loop
// above stays a separate function: its register allocation is tuned, and the row loops here
// would cost it spills.
template <int FMT, bool MATH, int NR>
__device__ __forceinline__ void decode_pass_loop(const PersistArgs& a, Shared& S, uint8_t* wdb, int w, int pos, int stp) {
    using PK = Pk<NR>;
    constexpr int CHK = (FMT == FMT_Q4) ? 128 : 64;
    constexpr int G = (FMT == FMT_Q4) ? 64 : 32;  // quantisation group (staged operand groups)
    constexpr int CW2 = H / CHK / MW;   // chunks per math wave, K = 2048
    constexpr int NRB = VOCAB / 16;     // lm_head row blocks
    constexpr int CW8 = H / CHK / WAVES;  // lm_head chunks per wave (all eight waves)
    constexpr int LM_DEPTH = 4;           // lm_head blocks in flight per wave
    constexpr int LM_BLOCKS = (NRB + NWG - 1) / NWG;  // 38 block slots per workgroup
    constexpr int NV = 4 * NR;            // query-operand variants: row, hi / lo, head
    uint64_t* ll = a.ll;
    unsigned* err = (unsigned*)a.ll + ERRW;
    State* st = a.st;
    const int maxsteps = st->maxsteps, eos0 = st->eos0, eos1 = st->eos1, maxctx = st->maxctx;
    const bool grammar = (st->flags & STATE_FLAG_GRAMMAR) != 0;
    const int L = a.nlayers;
    float nreg[8];  // math threads: norm weights of the next normed stage (8 each)
    if (MATH) load_norm8(nreg, a.layers[0].attn_norm + my_tid() * 8);
    // Math waves: the two QKV blocks (workgroups 128..255) or the O block (workgroups 0..127) of
    // the current layer.
    WB<FMT, CW2> wx[2];
    __syncthreads();

    for (int step = 0; step < a.nsteps; ++step) {
        if (pos + NR > maxctx) break;  // the commit stops earlier; guards the cache rows
        if (MATH) {
            wx[0].forget();
            wx[1].forget();
        }
        if (MATH && w >= NWG / 2) {  // layer 0's QKV blocks (no x poll follows at layer 0)
            wx[0].load(a.layers[0].wqkv, a.layers[0].wqkv_sb, w - NWG / 2, H, wave_id(), my_tid() % 64);
            wx[1].load(a.layers[0].wqkv, a.layers[0].wqkv_sb, w, H, wave_id(), my_tid() % 64);
        }
        for (int l = 0; l < L; ++l) {
            const LayerPtrs& P = a.layers[l];
            const unsigned r = (unsigned)(step * L + l);  // round of this layer
            const int tid = my_tid(), lane = tid % 64, wave = wave_id();
            constexpr bool math = MATH;
            const int mw = wave;  // math wave index (valid when math)

            // Attention geometry of this workgroup: KV group g, split s.  The pos + NR rows of the
            // group (rows < pos and the pass's new rows) are spread evenly over the 32 splits; the
            // split holding row pos + t writes it.  Only rows < pos are loaded from the cache.
            // Query row t sees rows <= pos + t: ntot_t of this split's rows.
            const int g = w % NKV, s = w / NKV;
            const int tot = pos + NR;
            const int chunk = (tot + ATT_SPLITS - 1) / ATT_SPLITS;
            const int j0 = min(s * chunk, tot), j1 = min(j0 + chunk, tot);
            // Recomputed where used (values kept live across the layer would cost registers).
            auto tl = [&](int t) { return (j0 <= pos + t) && (pos + t < j1); };  // row pos + t is in this split
            const bool tail = (j0 < pos + NR) && (pos < j1);                       // a new row is in this split
            const int nprior = max(0, min(j1, pos) - j0);
            const int ntot = j1 - j0;
            const uint16_t* kb = a.kv + ((size_t)(l * 2 + 0) * NKV + g) * a.maxctx * HD;
            const uint16_t* vb = a.kv + ((size_t)(l * 2 + 1) * NKV + g) * a.maxctx * HD;
            const int quad = tid / 16, ql = tid % 16;  // math threads: 16 quarter-waves, 8 dims per lane

            // Math-wave register tiles: each is requested while the exchange waves wait for the
            // input of its stage or of an earlier one.  The down half-block streams into LDS.
            WB<FMT, CW2> wgu[3];

            // ---------------- QKV: row blocks w - 128 and w (workgroups 128..255) ------------
            // Workgroups 0..127 need no x here.  Loads issued just before the x poll of
            // workgroups 128..255 would queue ahead of it on their CU: their QKV blocks are
            // requested during the previous layer's down stage (layer 0's at the start of the
            // step) and their K/V rows after the QKV publish.
            const bool qkv_wg = w >= NWG / 2;
            PK_TRACE(l, 0);
            uint4 kt[ATT_NT][4], vr[ATT_SPQ];
            float qn0 = 0.f, qn1 = 0.f, kn0 = 0.f, kn1 = 0.f, rc[NR], rs[NR];
            // Exchange waves poll the stage input first; math waves skip that branch and issue
            // their loads at once.  Keeping the loads after the poll in program order lets the
            // poll's registers and the weight tiles share the register file.
            bool ok_in = true;
            if (l > 0 && !math && qkv_wg) ok_in = poll_sum<NR * H / 2 / CT>(ll + PK::XP, ll + PK::XDP, 2 * r, S.vec, err);
            if (math) {
                // This layer's norm weights into LDS; then the QKV blocks and the loads for the
                // stages ahead: the first block of K/V rows, the per-head norms and the rope rows,
                // the O block and the mlp norm.
#pragma unroll
                for (int i = 0; i < 8; ++i) S.nw[tid * 8 + i] = nreg[i];
                if (!qkv_wg) {
                    wx[0].load(P.wo, P.wo_sb, w, H, mw, lane);
                    load_kv_block(kt, vr, kb, vb, j0, 0, nprior, tid);
                    // The lower down half-block of row block w into LDS: it lands long before the
                    // x' poll that a later request would delay.
                    wd_request<FMT>(wdb, P.wd, P.wd_sb, w, 0, mw, lane);
                }
                qn0 = P.q_norm[lane];
                qn1 = P.q_norm[lane + 64];
                kn0 = P.k_norm[lane];
                kn1 = P.k_norm[lane + 64];
#pragma unroll
                for (int t = 0; t < NR; ++t) {
                    const float* rope = a.rope + (size_t)(pos + t) * 128;
                    rc[t] = rope[2 * lane];
                    rs[t] = rope[2 * lane + 1];
                }
                load_norm8(nreg, P.mlp_norm + tid * 8);
            }
            if (sync_failed(S, !ok_in)) return;
            PK_TRACE_X(l, 1);
            if (qkv_wg) {
                stage_c<FMT, H, NR>(S, l == 0 ? S.emb : S.vec, true);
                float acc[2 * NR] = {};
                if (math) mac_rows<FMT, CW2, 2, NR>(S, wx, mw, lane, acc, H / G);
                PK_TRACE(l, 28);
                reduce_math_store<MATH, 2 * NR>(S, acc);
                if (wave == 0) {  // rows 2i, 2i + 1 of a block in packet i (even lanes)
#pragma unroll
                    for (int t = 0; t < NR; ++t) {
                        const float rsn = norm_scale<H>(S, t);
                        const float y0 = red_total(S, 2 * t) * rsn, y1 = red_total(S, 2 * t + 1) * rsn;
                        const float n0 = xor1(y0), n1 = xor1(y1);
                        if (lane < 16 && !(lane & 1)) {
                            uint64_t* q = ll + PK::QKVP + t * (QKV / 2);
                            st64(q + (w - NWG / 2) * 8 + lane / 2, pack2(y0, n0, r + 1));
                            st64(q + w * 8 + lane / 2, pack2(y1, n1, r + 1));
                        }
                    }
                }
                PK_TRACE(l, 30);
                if (math) load_kv_block(kt, vr, kb, vb, j0, 0, nprior, tid);
            }
            PK_TRACE(l, 2);

            // ---------------- attention: group g, split s ----------------------------------
            {
                bool ok = true;
                if (!math)  // row t: q heads 2g, 2g+1 -> vec[512t + 0..255], k -> +256..383, v -> +384..511
                    ok = poll_map<NR>(
                        ll + PK::QKVP, NR * 2 * HD,
                        [&](int k) {  // packet of gathered elements 2k, 2k + 1
                            const int t = k / (2 * HD), e = 2 * (k % (2 * HD));
                            return t * (QKV / 2) + (e < 2 * HD ? 2 * g * HD + e
                                                               : e < 3 * HD ? H + g * HD + (e - 2 * HD)
                                                                            : H + NKV * HD + g * HD + (e - 3 * HD)) / 2;
                        },
                        r + 1, S.vec, err);
                if (sync_failed(S, !ok)) return;
            }
            PK_TRACE_X(l, 3);
            if (math) {
                // Query rows: wave (t, h) = (wave / 2, wave % 2) of the NR rows; then the new K/V rows
                // of this split, a wave per row.  1/sqrt(128) and log2(e) are folded into q: scores
                // come out in base-2 units, so every softmax exponential of this split and of the
                // merge is one v_exp_f32.
                if (wave < 2 * NR) {
                    const int t = wave >> 1, hh = wave & 1;
                    float x0 = S.vec[512 * t + hh * HD + lane], x1 = S.vec[512 * t + hh * HD + lane + 64];
                    norm_rope(x0, x1, qn0, qn1, rc[t], rs[t]);
                    const float qscale = (1.0f / sqrtf((float)HD)) * 1.4426950408889634f;
                    const float qa = x0 * qscale, qb = x1 * qscale;
                    const uint16_t ha = f2h(qa), hb = f2h(qb);
                    S.qf[4 * t + hh][lane] = ha;
                    S.qf[4 * t + hh][lane + 64] = hb;
                    S.qf[4 * t + 2 + hh][lane] = f2h(qa - h2f(ha));
                    S.qf[4 * t + 2 + hh][lane + 64] = f2h(qb - h2f(hb));
                }
                const int kw = NR == 1 ? 2 : 0;  // first wave of the new-row normalisation
                if (wave >= kw && wave < kw + NR && tl(wave - kw)) {
                    const int t = wave - kw;
                    float k0 = S.vec[512 * t + 2 * HD + lane], k1 = S.vec[512 * t + 2 * HD + lane + 64];
                    norm_rope(k0, k1, kn0, kn1, rc[t], rs[t]);
                    S.ktail[t][lane] = f2h(k0);
                    S.ktail[t][lane + 64] = f2h(k1);
                    S.vtail[t][lane] = f2h(S.vec[512 * t + 3 * HD + lane]);
                    S.vtail[t][lane + 64] = f2h(S.vec[512 * t + 3 * HD + lane + 64]);
                }
            }
            __syncthreads();
            if (tail && !math && tid < MT + 128) {
                // The new cache rows (fp16), device-scope stores by exchange threads, acknowledged
                // before this workgroup publishes its partials.
                const int c = tid - MT;
#pragma unroll
                for (int t = 0; t < NR; ++t) {
                    if (!tl(t)) continue;
                    const uint16_t* src = c < 64 ? S.ktail[t] : S.vtail[t];
                    uint16_t* dst = (uint16_t*)(c < 64 ? kb : vb) + (size_t)(pos + t) * HD;
                    const int d = 2 * (c % 64);
                    const uint32_t v = (uint32_t)src[d] | ((uint32_t)src[d + 1] << 16);
                    __hip_atomic_store((uint32_t*)(dst + d), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                __builtin_amdgcn_s_waitcnt(0);
            }
            {
                // Scores on the matrix cores: per block, each math wave multiplies the query rows
                // (the fp16 hi and lo parts of both heads of each pass row, replicated over the 16 A
                // rows) with its ATT_NT tiles of 16 cache rows (v_mfma_f32_16x16x32_f16, four
                // products of 32 dims each); every lane then holds the scores of its column's slot
                // for pass row t = (lane / 16) % NR.  The online softmax runs per wave and row
                // (every lane holds its row's running maximum and sum); the probabilities move
                // through LDS (wave-local) to the P.V layout, where each quarter-wave takes 9 V
                // rows, 8 dims per lane, for every pass row.
                const int tq = (lane >> 4) & (NR - 1);  // pass row of this lane's scores
                float m_run[2] = {-__builtin_inff(), -__builtin_inff()}, l_run[2] = {0.f, 0.f};
                float o[NR][2][8];
#pragma unroll
                for (int t = 0; t < NR; ++t)
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                        for (int d = 0; d < 8; ++d) o[t][hh][d] = 0.f;
                PK_TRACE(l, 21);
                if (math) {
                    const int c = lane & 15, kq = lane >> 4;
#ifdef ICUA_PERSIST_TRACE
                    __builtin_amdgcn_s_waitcnt(0);
                    PK_TRACE(l, 25);
#endif
                    // Rows this lane's pass row sees (the split's rows up to slot pos + tq).
                    const int ntq = NR == 1 ? ntot : max(0, min(j1, pos + tq + 1) - j0);
                    for (int b0 = 0; b0 < ntot; b0 += ATT_BLOCK) {
                        const int nb = min(ATT_BLOCK, ntq - b0);
                        if (b0 > 0) load_kv_block(kt, vr, kb, vb, j0, b0, nprior, tid);
                        // The new rows (block slot pos + t - j0 - b0) come from LDS, not from the cache.
                        if (tail) {
#pragma unroll
                            for (int t = 0; t < NR; ++t) {
                                if (!tl(t)) continue;
                                const int pnew = pos + t - j0 - b0;
#pragma unroll
                                for (int T = 0; T < ATT_NT; ++T)
                                    if (4 * T + (c >> 2) < ATT_SPQ && att_slot(T, c, mw) == pnew) {
#pragma unroll
                                        for (int j = 0; j < 4; ++j) kt[T][j] = *(const uint4*)(S.ktail[t] + 32 * j + 8 * kq);
                                    }
#pragma unroll
                                for (int i = 0; i < ATT_SPQ; ++i)
                                    if (quad + ATT_QW * i == pnew) vr[i] = *(const uint4*)(S.vtail[t] + 8 * ql);
                            }
                        }
                        // D[variant][slot]: lane l holds rows 4 (l / 16) + r, i.e. variant
                        // (4 (l / 16) + r) % NV: row tq, hi (r = 0, 1) or lo (r = 2, 3) of head r % 2.
                        float sc[2][ATT_NT];
#pragma unroll
                        for (int T = 0; T < ATT_NT; ++T) {
                            f32x4 D = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                            for (int j = 0; j < 4; ++j)  // A: the query rows (read from LDS for each tile)
                                D = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                    *(const h8*)&S.qf[lane & (NV - 1)][32 * j + 8 * kq], as_h8(kt[T][j]), D, 0, 0, 0);
                            const bool ok = 4 * T + (c >> 2) < ATT_SPQ && att_slot(T, c, mw) < nb;
                            sc[0][T] = ok ? D[0] + D[2] : -__builtin_inff();
                            sc[1][T] = ok ? D[1] + D[3] : -__builtin_inff();
                        }
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            float mb = sc[hh][0];
#pragma unroll
                            for (int T = 1; T < ATT_NT; ++T) mb = fmaxf(mb, sc[hh][T]);
                            // mb is finite as soon as the wave has seen one valid slot of the row.
                            mb = fmaxf(max16(mb), m_run[hh]);
                            const float corr = (m_run[hh] == -__builtin_inff()) ? 0.f : ex2(m_run[hh] - mb);
                            float ls = 0.f;
#pragma unroll
                            for (int T = 0; T < ATT_NT; ++T) {
                                sc[hh][T] = (sc[hh][T] == -__builtin_inff()) ? 0.f : ex2(sc[hh][T] - mb);
                                ls += sc[hh][T];
                            }
                            l_run[hh] = l_run[hh] * corr + sum16(ls);
                            m_run[hh] = mb;
                            // o of row t is rescaled by row t's factor, which lanes 16 t .. hold.
#pragma unroll
                            for (int t = 0; t < NR; ++t) {
                                float ct = corr;
                                if constexpr (NR > 1) ct = __shfl(corr, 16 * t);
#pragma unroll
                                for (int d = 0; d < 8; ++d) o[t][hh][d] *= ct;
                            }
                            if (lane < 16 * NR) {
#pragma unroll
                                for (int T = 0; T < ATT_NT; ++T) S.pw[mw][tq][hh][c & 3][4 * T + (c >> 2)] = sc[hh][T];
                            }
                        }
                        // The probabilities of this wave's slots were written by its own lanes:
                        // a wave's LDS accesses complete in order, so no barrier is needed.
                        __builtin_amdgcn_wave_barrier();
                        PK_TRACE(l, 27);
#pragma unroll
                        for (int i = 0; i < ATT_SPQ; ++i) {
                            float p[NR][2];
#pragma unroll
                            for (int t = 0; t < NR; ++t) {
                                p[t][0] = S.pw[mw][t][0][kq][i];
                                p[t][1] = S.pw[mw][t][1][kq][i];
                            }
                            const uint32_t dv[4] = {vr[i].x, vr[i].y, vr[i].z, vr[i].w};
#pragma unroll
                            for (int j = 0; j < 4; ++j) {
                                const f16x2 hv = as_h2(dv[j]);
                                const float v0 = (float)hv.x, v1 = (float)hv.y;
#pragma unroll
                                for (int t = 0; t < NR; ++t)
#pragma unroll
                                    for (int hh = 0; hh < 2; ++hh) {
                                        o[t][hh][2 * j] = fmaf(p[t][hh], v0, o[t][hh][2 * j]);
                                        o[t][hh][2 * j + 1] = fmaf(p[t][hh], v1, o[t][hh][2 * j + 1]);
                                    }
                            }
                        }
                        __builtin_amdgcn_wave_barrier();
                    }
                    PK_TRACE(l, 29);
                    // The wave's 4 quarter-waves (lanes l, l ^ 16, l ^ 32, l ^ 48 hold the same
                    // dims) share each row's running maximum: their sums add.
#pragma unroll
                    for (int t = 0; t < NR; ++t)
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                            for (int d = 0; d < 8; ++d) o[t][hh][d] = sum_x4(o[t][hh][d]);
                    if (lane < 16) {
#pragma unroll
                        for (int t = 0; t < NR; ++t)
#pragma unroll
                            for (int hh = 0; hh < 2; ++hh)
#pragma unroll
                                for (int d = 0; d < 8; ++d) S.ored[mw][2 * t + hh][8 * ql + d] = o[t][hh][d];
                    }
                    if ((lane & 15) == 0 && lane < 16 * NR) {  // row tq's (m, l) per head
                        S.aml[mw][4 * tq + 0] = m_run[0];
                        S.aml[mw][4 * tq + 1] = m_run[1];
                        S.aml[mw][4 * tq + 2] = l_run[0];
                        S.aml[mw][4 * tq + 3] = l_run[1];
                    }
                }
                PK_TRACE(l, 22);
                __syncthreads();
                if (math) {
                    // The split's partials: per pass row and head, the 4 waves rescaled to their
                    // common max.
                    uint64_t* part = ll + PK::PARTP + (size_t)(g * ATT_SPLITS + s) * NR * 2 * PART2;
                    const int hh = tid / HD, d = tid % HD;
#pragma unroll
                    for (int t = 0; t < NR; ++t) {
                        float mx = -__builtin_inff();
#pragma unroll
                        for (int ww = 0; ww < MW; ++ww) mx = fmaxf(mx, S.aml[ww][4 * t + hh]);
                        float acc = 0.f, lsum = 0.f;
#pragma unroll
                        for (int ww = 0; ww < MW; ++ww) {
                            const float mwv = S.aml[ww][4 * t + hh];
                            const float f = (mwv == -__builtin_inff()) ? 0.f : ex2(mwv - mx);
                            acc = fmaf(S.ored[ww][2 * t + hh][d], f, acc);
                            lsum = fmaf(S.aml[ww][4 * t + 2 + hh], f, lsum);
                        }
                        // o pairs (even lanes), then (l, m) with the maximum exact.
                        uint64_t* pt = part + (2 * t + hh) * PART2;
                        const float acc_n = xor1(acc);
                        if (!(d & 1)) st64(pt + d / 2, pack2(acc, acc_n, r + 1));
                        if (d == 0) st64(pt + HD / 2, pack2(lsum, mx, r + 1));
                    }
                }
                PK_TRACE(l, 20);
            }
            PK_TRACE(l, 4);

            // ---------------- merge of group g: workgroups 224..255 ------------------------
            // Split s = 28 + p of group g (workgroup 224 + 8p + g, no O / down work) merges part
            // p = 0..3 of the group's output for every pass row: head 2g + p / 2, elements
            // 64 (p % 2) .. + 63.
            if (w >= MERGER0) {
                const int p = s - (ATT_SPLITS - MERGE_PARTS), hh = p / 2, d0 = 64 * (p % 2);
                float* pl = (float*)S.A;  // [NR][32][64 + 2]: o elements d0.., l, m of head hh per split
                static_assert(NR * ATT_SPLITS * 66 * 4 <= A_BYTES, "the merge's partials fit S.A");
                const uint64_t* gp = ll + PK::PARTP + (size_t)g * PK::GROUP_PARTS;
                bool ok = true;
                if (!math)
                    ok = poll_map<(NR * ATT_SPLITS * 33 + CT - 1) / CT>(
                        gp, NR * ATT_SPLITS * 33,
                        [&](int k) {
                            const int t = k / (ATT_SPLITS * 33), sj = (k / 33) % ATT_SPLITS, e = k % 33;
                            return (sj * NR * 2 + 2 * t + hh) * PART2 + (e < 32 ? d0 / 2 + e : HD / 2);
                        },
                        r + 1, pl, err);
                if (sync_failed(S, !ok)) return;
                PK_TRACE_X(l, 5);
#pragma unroll
                for (int t = 0; t < NR; ++t) {
                    const float* plt = pl + t * ATT_SPLITS * 66;
                    // Split weights exp(m_s - max) and the normaliser (math wave 0, one lane per split).
                    if (math && wave == 0) {
                        const int sl = lane % ATT_SPLITS;
                        const float m = plt[sl * 66 + 65];
                        const float mx = wave_max(m);  // finite: the split holding row pos + t sees a row
                        const float wgt = (m == -__builtin_inff()) ? 0.f : ex2(m - mx);
                        const float lw = wave_sum(lane < ATT_SPLITS ? wgt * plt[sl * 66 + 64] : 0.f);
                        if (lane < ATT_SPLITS) S.sc[0][lane] = wgt;
                        if (lane == 0) S.misc[0] = 1.0f / lw;
                    }
                    __syncthreads();
                    // Weighted sum of the split outputs: thread (q, e) over splits 4q .. 4q + 3, the
                    // eight quarters combined through LDS.
                    {
                        const int q = tid / 64, e = tid % 64;
                        float O = 0.f;
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const int sj = q * 4 + j;
                            O = fmaf(S.sc[0][sj], plt[sj * 66 + e], O);
                        }
                        float* q8 = &S.ored[0][0][0];  // [8][64]
                        q8[q * 64 + e] = O;
                        __syncthreads();
                        if (tid < 64) {
                            float tt = 0.f;
#pragma unroll
                            for (int qq = 0; qq < 8; ++qq) tt += q8[qq * 64 + tid];
                            const float v = tt * S.misc[0], vn = xor1(v);
                            if (!(tid & 1))
                                st64(ll + PK::ATTNP + t * (H / 2) + ((2 * g + hh) * HD + d0 + tid) / 2, pack2(v, vn, r + 1));
                        }
                    }
                    if (NR > 1) __syncthreads();  // S.sc, S.misc[0] and the sums are rewritten for the next row
                }
                PK_TRACE(l, 17);
                __syncthreads();  // the partials in S.A are read before the next staging
                PK_TRACE(l, 6);
            }

            // ---------------- O projection + residual: workgroups 0..127 -------------------
            // The gate|up blocks are requested here, a stage early, by every workgroup.  The
            // residual of the O rows is xown (previous x + lower-half down sums) + xhi (the
            // upper-half sums, long published): the same two terms every x reader adds.
            //
            // Workgroups 128..223 (no O, no merge) request their next stages' weights only once
            // their KV group's split partials are all out: issued as their attention ends, these
            // ~10 MB would queue at the memory controllers ahead of the mergers' polls of those
            // partials.  Which split publishes last varies (those holding new cache rows also
            // wait for the rows' acknowledgement): their math waves' wave 0 watches an (l, m)
            // packet of each of the 32, and nothing else of theirs is in flight then.
            if (math && w >= NWG / 2 && w < MERGER0) {
                // Wave 0 watches; the other math waves wait for it in LDS.
                if (wave == 0)
                    watch_partials(S, ll + PK::PARTP + (size_t)g * ATT_SPLITS * NR * 2 * PART2 + (NR - 1) * 2 * PART2 + HD / 2,
                                   (size_t)NR * 2 * PART2, tag4(r + 1), (int)r + 1, err, lane);
                while (__hip_atomic_load(&S.go, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != (int)r + 1)
                    __builtin_amdgcn_s_sleep(1);
            }
            {
                bool ok = true;
                if (w < H / 16 && !math) {
                    if (l > 0) {
#pragma unroll
                        for (int t = 0; t < NR; ++t)
                            ok = ok && poll_vec<1>(ll + PK::XDP + t * (H / 2) + w * 8, 8, 2 * r, S.xhi[t], err);
                    } else if (tid - MT < 16 * NR) {
                        S.xhi[(tid - MT) / 16][(tid - MT) % 16] = 0.f;
                    }
                    ok = ok && poll_vec<NR * H / 2 / CT>(ll + PK::ATTNP, NR * H / 2, r + 1, S.vec, err);
                }
                if (math) {
#pragma unroll
                    for (int j = 0; j < 3; ++j) wgu[j].load(P.wgu, P.wgu_sb, 3 * w + j, H, mw, lane);
                }
                if (w < H / 16 && sync_failed(S, !ok)) return;
            }
            if (w < H / 16) {
                PK_TRACE_X(l, 7);
                stage_c<FMT, H, NR>(S, S.vec, false);
                float acc[NR] = {};
                if (math) mac_rows<FMT, CW2, 1, NR>(S, wx, mw, lane, acc, H / G);
                reduce_math_store<MATH, NR>(S, acc);
                if (wave == 0) {  // the owner keeps the residual as published (even rows rounded)
#pragma unroll
                    for (int t = 0; t < NR; ++t) {
                        const float xn = lane < 16 ? (S.xown[t][lane] + S.xhi[t][lane]) + red_total(S, t) : 0.f;
                        const float xo = xor1(xn);
                        if (lane < 16) {
                            S.xown[t][lane] = (lane & 1) ? xn : q19(xn);
                            if (!(lane & 1)) st64(ll + PK::XP + t * (H / 2) + w * 8 + lane / 2, pack2(xn, xo, 2 * r + 1));
                        }
                    }
                }
                PK_TRACE(l, 8);
            }
            // Workgroups 128..255 request the upper down half-block and the next layer's QKV
            // blocks here, where they wait for no stage input (workgroups 0..127 run O): loads
            // issued later would queue ahead of their x' and h polls.
            if (math && qkv_wg) {
                wd_request<FMT>(wdb, P.wd, P.wd_sb, w - NWG / 2, 1, mw, lane);
                wx[0].forget();
                wx[1].forget();
                if (l + 1 < L) {
                    const LayerPtrs& Pn = a.layers[l + 1];
                    wx[0].load(Pn.wqkv, Pn.wqkv_sb, w - NWG / 2, H, mw, lane);
                    wx[1].load(Pn.wqkv, Pn.wqkv_sb, w, H, mw, lane);
                }
            }

            // ---------------- RMSNorm + gate|up + SwiGLU: blocks 3w .. 3w + 2 --------------
            {
                bool ok = true;
                if (!math) ok = poll_vec<NR * H / 2 / CT>(ll + PK::XP, NR * H / 2, 2 * r + 1, S.vec, err);
                if (math) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) S.nw[tid * 8 + i] = nreg[i];
                    // The next layer's attention norm, or the final norm.
                    load_norm8(nreg, (l + 1 < L ? a.layers[l + 1].attn_norm : a.final_norm) + tid * 8);
                }
                if (sync_failed(S, !ok)) return;
                PK_TRACE_X(l, 9);
                stage_c<FMT, H, NR>(S, S.vec, true);
                PK_TRACE(l, 13);
                float acc[3 * NR] = {};
                if (math) mac_rows<FMT, CW2, 3, NR>(S, wgu, mw, lane, acc, H / G);
                PK_TRACE(l, 26);
                reduce_math_store<MATH, 3 * NR>(S, acc);
                PK_TRACE(l, 14);
                if (wave == 0) {
#pragma unroll
                    for (int t = 0; t < NR; ++t) {
                        const float rsn = norm_scale<H>(S, t);
#pragma unroll
                        for (int j = 0; j < 3; ++j) {
                            // Block 3w + j: gate units 8 (3w + j) + 0..7 in lanes 0-7, their up rows in 8-15.
                            const float yj = red_total(S, 3 * t + j) * rsn;
                            const float hv = swiglu(yj, xor8(yj)), hn = xor1(hv);
                            if (lane < 8 && !(lane & 1))
                                st64(ll + PK::HP + t * (FF / 2) + (3 * w + j) * 4 + lane / 2, pack2(hv, hn, r + 1));
                        }
                    }
                }
                PK_TRACE(l, 10);
            }

            // ---------------- down: K half w / 128 of row block w % 128 --------------------
            {
                const int rb = w % (NWG / 2), half = w / (NWG / 2);
                bool ok = true;
                if (!math) {  // row t's half: HP + t FF / 2 + half FFH / 2 .. -> vec[t FFH ..]
                    if constexpr (NR == 1)
                        ok = poll_vec<FFH / 2 / CT>(ll + PK::HP + half * (FFH / 2), FFH / 2, r + 1, S.vec, err);
                    else
                        ok = poll_map<NR * FFH / 2 / CT>(
                            ll + PK::HP, NR * FFH / 2,
                            [&](int k) { return (k / (FFH / 2)) * (FF / 2) + half * (FFH / 2) + k % (FFH / 2); },
                            r + 1, S.vec, err);
                }
                if (math && !qkv_wg) {
                    wx[0].forget();
                    wx[1].forget();
                }
                if (sync_failed(S, !ok)) return;
                PK_TRACE_X(l, 11);
                stage_c<FMT, FFH, NR>(S, S.vec, false);
                PK_TRACE(l, 18);
                float yd[NR];
#pragma unroll
                for (int t = 0; t < NR; ++t) yd[t] = 0.f;
                if (math) {
                    // This wave's down-block requests have landed (and the QKV prefetch, issued
                    // after them, too: vector memory counts complete in order).
                    __builtin_amdgcn_s_waitcnt(0);
                    __atomic_signal_fence(__ATOMIC_SEQ_CST);
                    PK_TRACE(l, 23);
#pragma unroll
                    for (int t = 0; t < NR; ++t) yd[t] = wd_mac_lds<FMT>(S, wdb, mw, lane, t * (FFH / G));
                    PK_TRACE(l, 24);
                }
                reduce_math_store<MATH, NR>(S, yd);
                PK_TRACE(l, 19);
                if (wave == 0) {
#pragma unroll
                    for (int t = 0; t < NR; ++t) {
                        const float yt = red_total(S, t);
                        const float v = lane < 16 ? (half == 0 ? S.xown[t][lane] + yt : yt) : 0.f;
                        const float vn = xor1(v);
                        if (lane < 16) {
                            if (half == 0) S.xown[t][lane] = (lane & 1) ? v : q19(v);
                            if (!(lane & 1))
                                st64(ll + (half == 0 ? PK::XP : PK::XDP) + t * (H / 2) + rb * 8 + lane / 2,
                                     pack2(v, vn, 2 * r + 2));
                        }
                    }
                }
                PK_TRACE(l, 12);
            }
        }

        // ---------------- final RMSNorm + lm_head + per-workgroup argmax ---------------------
        // Over the pass's last row only (the reference commits the last row's argmax).
        {
            const int tid = my_tid(), lane = tid % 64, wave = wave_id();
            constexpr bool math = MATH;
            const unsigned r_last = (unsigned)(step * L + L - 1);
            PK_TRACE(L, 0);
            // All eight waves stream the blocks w + k * 256 (chunks wave * CW8 ..), LM_DEPTH in
            // flight per wave; the exchange waves issue theirs once their poll is done.  Each
            // wave's per-block partial sums go to LDS; one reduction and argmax at the end.
            WB<FMT, CW8> wl[LM_DEPTH];
            bool ok = true;
            if (!math)
                ok = poll_sum<H / 2 / CT>(ll + PK::XP + (NR - 1) * (H / 2), ll + PK::XDP + (NR - 1) * (H / 2),
                                          2 * r_last + 2, S.vec, err);
            if (math) {
#pragma unroll
                for (int i = 0; i < 8; ++i) S.nw[tid * 8 + i] = nreg[i];
            }
            // The exchange waves request their blocks once x is in; the math waves' requests
            // also wait for the barrier, so that no bulk load queues ahead of the x poll.
            if (!math) {
#pragma unroll
                for (int k = 0; k < LM_DEPTH; ++k) wl[k].load(a.E, a.Esb, w + k * NWG, H, wave, lane);
            }
            if (sync_failed(S, !ok)) return;
            if (math) {
#pragma unroll
                for (int k = 0; k < LM_DEPTH; ++k) wl[k].load(a.E, a.Esb, w + k * NWG, H, wave, lane);
            }
            PK_TRACE_X(L, 1);
            stage_c<FMT, H>(S, S.vec, true);
            float* plm = (float*)wdb;  // [LM_BLOCKS][WAVES][16] partial sums
            QuadOps<FMT> lq[CW8 / 2];  // this wave's operand quads, the same for every block
#pragma unroll
            for (int p = 0; p < CW8 / 2; ++p) lq[p] = quad_load<FMT>(S, wave * CW8 + 2 * p, lane);
            // Every iteration issues the same refill (past the matrix it re-reads the last row
            // block, an L2 hit, and the sums of blocks past the matrix are dropped): with the
            // same loads on every path the compiler's waits stay exact, instead of draining every
            // block in flight before each block's scales are used.
            for (int k0 = 0; k0 < LM_BLOCKS; k0 += LM_DEPTH) {
#pragma unroll
                for (int k = 0; k < LM_DEPTH; ++k) {
                    const int kb = k0 + k, rb = w + kb * NWG;
                    float y = 0.f;
#pragma unroll
                    for (int p = 0; p < CW8 / 2; ++p)
                        y = quad_scale<FMT>(lq[p], quad_mfma<FMT>(lq[p], wl[k].wv[2 * p], wl[k].wv[2 * p + 1]),
                                            wl[k].sq[p], y);
                    y = quad_rows(y);
                    if (rb < NRB && lane < 16) plm[(kb * WAVES + wave) * 16 + lane] = y;
                    wl[k].load(a.E, a.Esb, min(rb + LM_DEPTH * NWG, NRB - 1), H, wave, lane);
                }
            }
            __syncthreads();
            float best = -__builtin_inff();
            int besti = 0x7fffffff;
            const float rsn = norm_scale<H>(S);
            for (int e = tid; e < LM_BLOCKS * 16; e += THREADS) {  // (block, row) pairs
                const int kb = e / 16, rw = e % 16;
                if (w + kb * NWG < NRB) {
                    const float* pp = plm + kb * WAVES * 16 + rw;
                    float y = 0.f;
#pragma unroll
                    for (int wv = 0; wv < WAVES; ++wv) y += pp[wv * 16];
                    argmax_merge(best, besti, y * rsn, (w + kb * NWG) * 16 + rw);
                }
            }
            wave_argmax(best, besti);
            if (lane == 0) {
                S.misc[8 + wave] = best;
                S.imisc[8 + wave] = besti;
            }
            __syncthreads();
            if (tid == 0) {
                for (int wv = 1; wv < WAVES; ++wv) argmax_merge(best, besti, S.misc[8 + wv], S.imisc[8 + wv]);
                // (index << 4 | tag, value): the value exact, ids < 2^27 exact in the low word.
                const uint32_t lo = ((uint32_t)min(besti, 0x07FFFFFF) << 4) | tag4((unsigned)step + 1);
                st64(ll + PK::LMP + w, (uint64_t)lo | ((uint64_t)as_u32(best) << 32));
            }
            PK_TRACE(L, 2);
            if (math) load_norm8(nreg, a.layers[0].attn_norm + tid * 8);  // for the next step
        }

        // ---------------- greedy commit, evaluated by every workgroup ------------------------
        {
            const int tid = my_tid(), lane = tid % 64, wave = wave_id();
            bool ok = true;
            if (!MATH) ok = poll_vec<NWG / CT>(ll + PK::LMP, NWG, (unsigned)step + 1, S.vec, err);
            if (sync_failed(S, !ok)) return;
            PK_TRACE_X(L, 3);
            float bv = -__builtin_inff();
            int bi = 0x7fffffff;
            if (tid < NWG) {
                bv = S.vec[2 * tid + 1];
                bi = (int)(as_u32(S.vec[2 * tid]) >> 4);
            }
            wave_argmax(bv, bi);
            if (lane == 0) {
                S.misc[wave] = bv;
                S.imisc[wave] = bi;
            }
            __syncthreads();
            float b2 = S.misc[0];
            int tok = S.imisc[0];
            for (int ww = 1; ww < WAVES; ++ww) argmax_merge(b2, tok, S.misc[ww], S.imisc[ww]);
            bool stop, pair = false;
            int forced = -1;
            if (stp >= maxsteps) {  // nothing may be written past out_tokens[maxsteps - 1]
                stop = true;
            } else {
                const bool bad = tok < 0 || tok >= VOCAB;  // no finite logit (NaN model): stop on token 0
                if (bad) tok = 0;
                if (w == 0 && tid == 0) a.out_tokens[stp] = tok;
                stp += 1;
                pos += NR;
                stop = bad || tok == eos0 || tok == eos1 || (grammar && tok == 8) || stp >= maxsteps ||
                       pos + 2 > maxctx;
                // Grammar pairs: after a first-step action token, or after 11, the next token is
                // forced (7, or 220 after 11); it is committed now, and the next pass carries both
                // tokens (n = 2): this launch ends and the pair runs as one two-row pass.
                if (!stop && grammar &&
                    ((stp == 1 && (tok == 3678 || tok == 7241 || tok == 12476 || tok == 10855 || tok == 11862 ||
                                   tok == 1339 || tok == 1472 || tok == 24769)) ||
                     tok == 11)) {
                    forced = tok == 11 ? 220 : 7;
                    if (w == 0 && tid == 0) a.out_tokens[stp] = forced;
                    stp += 1;
                    pair = true;
                    stop = stp >= maxsteps;  // the pair's pass would start at the step limit
                }
            }
            if (w == 0 && tid == 0) {
                st->pos = pos;
                st->step = stp;
                st->n = pair && !stop ? 2 : 1;
                st->vis_offset = -1;
                st->logits_rows = 0;
                if (stop) st->done = 1;
            }
            if (stop) break;
            // Next token's embedding (Shaders.swift:464-476), in every workgroup.
            __syncthreads();  // every thread has read S.misc / S.imisc
            for (int i = tid; i < H; i += THREADS) S.emb[i] = dequant_tiled(FMT, a.E, a.Esb, (size_t)tok, i, H);
            __syncthreads();
            if (tid < 16 && w < H / 16) S.xown[0][tid] = S.emb[w * 16 + tid];
            if (w == 0 && (pair || step == a.nsteps - 1)) {
                for (int i = tid; i < H; i += THREADS) a.x[i] = S.emb[i];  // residual row(s) for the next launch
                if (pair)
                    for (int i = tid; i < H; i += THREADS) a.x[H + i] = dequant_tiled(FMT, a.E, a.Esb, (size_t)forced, i, H);
            }
            PK_TRACE(L, 4);
            if (pair) break;  // the pair is the next launch's pass
        }
    }
}

// ------------------------------------------------------------------------------------------
// Isolated one-token GEMV y = W x (W tiled by icua_repack, K = 2048 or 6144) on the schedule of
// the lm_head stage above: one 512-thread workgroup per CU streams 16-row blocks wg, wg + G, ...
// All eight waves split K (CW chunks each; each quad's operand tiles are read from LDS once for
// every block), DEPTH blocks are in flight per wave, and the per-block partial sums of the waves
// wait in LDS for one reduction at the end.  Every lane does useful work: the four groups of a
// quad accumulate into one matrix-core result (lanes 16j.. hold group j's sums).
constexpr int GS_MAX_BLOCKS = 160;  // row blocks per workgroup (part[] below)
// The staging state the isolated GEMV uses (the decode kernel's Shared holds the same members).
struct GemvShared {
    uint8_t A[A_BYTES];
    uint32_t zero[4];
    float fx[192 * 2];
    float nw[H];
    float misc[64];
};
template <int FMT, int K>
__global__ __launch_bounds__(THREADS, 1) void gemv_stream_kernel(const uint8_t* w, const uint8_t* sb, const float* x,
                                                                  float* y, int nrb) {
    constexpr int CHK = (FMT == FMT_Q4) ? 128 : 64;
    constexpr int CW = K / CHK / WAVES;  // chunks per wave: q4 2 / 6, q8 4 / 12
    constexpr int DEPTH = CW <= 2 ? 4 : CW <= 6 ? 2 : 1;
    __shared__ GemvShared S;
    __shared__ float part[GS_MAX_BLOCKS * WAVES * 16];
    const int wg = blockIdx.x, G = gridDim.x, tid = my_tid(), lane = tid % 64, wave = wave_id();
    const int nb = (nrb - wg + G - 1) / G;  // blocks of this workgroup (the host keeps wg < nrb)
    if (tid < 4) S.zero[tid] = 0u;
    WB<FMT, CW> wl[DEPTH];
#pragma unroll
    for (int k = 0; k < DEPTH; ++k) wl[k].load(w, sb, min(wg + k * G, nrb - 1), K, wave, lane);
    stage_c<FMT, K>(S, x, false);
    QuadOps<FMT> lq[CW / 2];
#pragma unroll
    for (int p = 0; p < CW / 2; ++p) lq[p] = quad_load<FMT>(S, wave * CW + 2 * p, lane);
    for (int k0 = 0; k0 < nb; k0 += DEPTH) {
#pragma unroll
        for (int k = 0; k < DEPTH; ++k) {
            const int kb = k0 + k;
            if (kb < nb) {
                float v = 0.f;
#pragma unroll
                for (int p = 0; p < CW / 2; ++p)
                    v = quad_scale<FMT>(lq[p], quad_mfma<FMT>(lq[p], wl[k].wv[2 * p], wl[k].wv[2 * p + 1]), wl[k].sq[p],
                                        v);
                v = quad_rows(v);
                if (lane < 16) part[(kb * WAVES + wave) * 16 + lane] = v;
                if (kb + DEPTH < nb) wl[k].load(w, sb, wg + (kb + DEPTH) * G, K, wave, lane);
            }
        }
    }
    __syncthreads();
    for (int e = tid; e < nb * 16; e += THREADS) {
        const int kb = e / 16, r = e % 16;
        const float* pp = part + kb * WAVES * 16 + r;
        float v = 0.f;
#pragma unroll
        for (int wv = 0; wv < WAVES; ++wv) v += pp[wv * 16];
        y[(size_t)(wg + kb * G) * 16 + r] = v;
    }
}

template <int FMT, int NR>
__global__ __launch_bounds__(THREADS, 1) void decode_kernel(PersistArgs a) {
    __shared__ Shared S;
    // The LDS-DMA destination (down half-block; lm_head partial sums later) is an object of its
    // own, so that LDS accesses to S need not wait for the DMA's completion.
    __shared__ __align__(16) uint8_t wdb[WD_CODES + WD_SB];
    const int w = blockIdx.x;
    if (my_tid() < 4) S.zero[my_tid()] = 0u;
    if (my_tid() == 0) {
        S.fail = 0;
        S.go = 0;
    }
    // Control block and the embeddings of the pass's tokens (written before this launch).  The
    // NR = 1 kernel runs single-row passes, the NR = 2 kernel one forced pair (checked by the host too).
    const State* st = a.st;
    if (st->done || st->n != NR) return;
    for (int i = my_tid(); i < NR * H; i += THREADS) S.emb[i] = a.x[i];
    if (my_tid() < 16 * NR && w < H / 16) S.xown[my_tid() / 16][my_tid() % 16] = a.x[(my_tid() / 16) * H + w * 16 + my_tid() % 16];
    if constexpr (NR == 1) {
        if (wave_id() < MW)
            decode_loop<FMT, true>(a, S, wdb, w, st->pos, st->step);
        else
            decode_loop<FMT, false>(a, S, wdb, w, st->pos, st->step);
    } else {
        if (wave_id() < MW)
            decode_pass_loop<FMT, true, NR>(a, S, wdb, w, st->pos, st->step);
        else
            decode_pass_loop<FMT, false, NR>(a, S, wdb, w, st->pos, st->step);
    }
}

}  // namespace pk

hipError_t launch_persistent(int fmt, int nr, const PersistArgs& a, hipStream_t s) {
    void* args[] = {(void*)&a};
    const void* k = nullptr;
    if (fmt == FMT_Q4) k = nr == 2 ? (const void*)pk::decode_kernel<FMT_Q4, 2> : (const void*)pk::decode_kernel<FMT_Q4, 1>;
    if (fmt == FMT_Q8) k = nr == 2 ? (const void*)pk::decode_kernel<FMT_Q8, 2> : (const void*)pk::decode_kernel<FMT_Q8, 1>;
    if (fmt == FMT_F16 && nr == 1) k = (const void*)pk::decode_kernel<FMT_F16, 1>;  // f16 pairs: the graph path
    if (!k || (nr != 1 && nr != 2) || (nr == 2 && a.nsteps != 1)) return hipErrorInvalidValue;
    return hipLaunchCooperativeKernel(k, dim3(pk::NWG), dim3(pk::THREADS), args, 0, s);
}

hipError_t launch_gemv_stream(int fmt, const uint8_t* w, const uint8_t* sb, const float* x, float* y, int N, int K,
                              hipStream_t s) {
    if (N <= 0 || N % 16 || (K != H && K != FF) || (fmt != FMT_Q4 && fmt != FMT_Q8)) return hipErrorInvalidValue;
    const int nrb = N / 16, G = nrb < pk::NWG ? nrb : pk::NWG;
    if (nrb > pk::GS_MAX_BLOCKS * G) return hipErrorInvalidValue;
    const void* k = fmt == FMT_Q4 ? (K == H ? (const void*)pk::gemv_stream_kernel<FMT_Q4, H>
                                            : (const void*)pk::gemv_stream_kernel<FMT_Q4, FF>)
                                  : (K == H ? (const void*)pk::gemv_stream_kernel<FMT_Q8, H>
                                            : (const void*)pk::gemv_stream_kernel<FMT_Q8, FF>);
    void* args[] = {(void*)&w, (void*)&sb, (void*)&x, (void*)&y, (void*)&nrb};
    return hipLaunchKernel(k, dim3(G), dim3(pk::THREADS), args, 0, s);
}

#ifdef ICUA_PERSIST_TRACE
extern "C" int icua_debug_persist_trace(uint64_t* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(pk::g_trace), sizeof(pk::g_trace)) == hipSuccess ? 0 : -1;
}
#endif

size_t persistent_sync_bytes() { return ((size_t)pk::Pk<2>::PACKETS + 32) * sizeof(uint64_t); }
int persistent_error_slot() { return pk::ERRW; }
size_t persistent_clear_bytes(int nr) {
    return (size_t)(nr == 2 ? pk::Pk<2>::PACKETS : pk::Pk<1>::PACKETS) * sizeof(uint64_t);
}

}  // namespace icua
