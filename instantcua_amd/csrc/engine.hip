// Host engine behind include/icua.h: model load, device buffers, pass orchestration and the
// GPU-resident greedy decode loop.  Mirrors Sources/Engine/Engine.swift (init 54-185,
// prepareMRoPE 254-298, encodeLLMLayer 476-629, encodeLMHead 631-644, encodeCommit 646-656,
// encodePrefill 658-673, encodeDecodeStep 675-681, generateVision 696-827).
//
// Differences by design: one HIP stream instead of Metal command buffers; one decode step is a
// captured HIP graph replayed per token (the reference encodes 8 steps per command buffer);
// q4 prompts longer than MAXM rows prefill through the matrix-core GEMMs and flash attention of
// prefill.hip in chunks of up to PF_CHUNK rows; other prompts run in passes of up to MAXM rows
// through the decode kernels.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "../../include/icua.h"
#include "icua_kernels.h"
#include "icua_persist.h"

using namespace icua;

namespace {

thread_local std::string g_err;

int fail(const std::string& msg) {
    g_err = msg;
    return -1;
}

#define HIPCK(call)                                                                             \
    do {                                                                                        \
        hipError_t _e = (call);                                                                 \
        if (_e != hipSuccess) return fail(std::string(#call) + ": " + hipGetErrorString(_e));   \
    } while (0)

// Tensor ids (Sources/Engine/ModelFile.swift:62-111).
constexpr int T_EMBED = 315, T_EMBED_SB = 316, T_FINAL_NORM = 317, T_LAYER_BASE = 318, T_PER_LAYER = 14;
constexpr int T_COUNT = 710;
constexpr uint32_t MAGIC = 0x31554349u;  // "ICU1"

size_t code_bytes(int fmt, size_t rows, size_t K) { return fmt == 2 ? rows * K / 2 : fmt == 1 ? rows * K : rows * K * 2; }
size_t sb_bytes(int fmt, size_t rows, size_t K) { return fmt == 2 ? rows * (K / 64) * 4 : fmt == 1 ? rows * (K / 32) * 2 : 0; }

struct LayerW {
    const float *attn_norm, *q_norm, *k_norm, *mlp_norm;
    const uint8_t *wqkv, *wqkv_sb, *wo, *wo_sb, *wgu, *wgu_sb, *wd, *wd_sb;
};

// M-RoPE table (Engine.swift:121-125, 254-298): inv-freq in double, angle = double(float(p) *
// float(invf)), cos/sin in double rounded to float.
void mrope_table(int maxctx, int vis_offset, int llm_h, int llm_w, std::vector<float>& out) {
    double invf[64];
    for (int i = 0; i < 64; ++i) invf[i] = 1.0 / std::pow(5000000.0, (double)(2 * i) / 128.0);
    const int n_vis = llm_h * llm_w;
    const int delta = std::max(llm_h, llm_w) - n_vis;
    out.resize((size_t)maxctx * 128);
    for (int slot = 0; slot < maxctx; ++slot) {
        int pt, ph, pw;
        if (vis_offset < 0 || slot < vis_offset) {
            pt = ph = pw = slot;
        } else if (slot < vis_offset + n_vis) {
            const int v = slot - vis_offset;
            pt = vis_offset;
            ph = vis_offset + v / llm_w;
            pw = vis_offset + v % llm_w;
        } else {
            pt = ph = pw = slot + delta;
        }
        for (int i = 0; i < 64; ++i) {
            // mrope_section [24, 20, 20] interleaved: H at 1:60:3, W at 2:60:3, else T.
            const int p = (i < 60 && i % 3 == 1) ? ph : (i < 60 && i % 3 == 2) ? pw : pt;
            const double ang = (double)((float)p * (float)invf[i]);
            out[(size_t)slot * 128 + 2 * i] = (float)std::cos(ang);
            out[(size_t)slot * 128 + 2 * i + 1] = (float)std::sin(ang);
        }
    }
}

constexpr int PF_CHUNK = 4096;  // rows per matrix-core prefill chunk

struct NullState {
    State* d = nullptr;
};
NullState g_null_state;  // control block for standalone kernels (done = 0)

int null_state(State** out, int n) {
    if (!g_null_state.d) HIPCK(hipMalloc(&g_null_state.d, sizeof(State)));
    State s{};
    s.n = n;
    s.maxctx = 1;
    HIPCK(hipMemcpy(g_null_state.d, &s, sizeof s, hipMemcpyHostToDevice));
    *out = g_null_state.d;
    return 0;
}

}  // namespace

// Packet areas of the persistent decode kernel live in uncached device memory: its all-to-all
// exchanges (device-scope stores polled by device-scope loads, 256 workgroups) complete about
// 10 % sooner there than in cached memory (2.28 against 2.55 us per round idle, 5.06 against
// 5.53 us with 64 KiB of loads in flight per CU).  Uncached memory that a kernel has read is
// never handed back to the allocator while the process runs: an engine returns its area to this
// per-device pool, and the next engine created on that device takes it again.
namespace {
std::mutex g_sync_mu;
std::vector<std::pair<int, void*>> g_sync_pool;  // (device, area), all persistent_sync_bytes() long
}  // namespace

static hipError_t take_sync_area(int dev, void** out) {
    {
        std::lock_guard<std::mutex> lk(g_sync_mu);
        for (size_t i = 0; i < g_sync_pool.size(); ++i)
            if (g_sync_pool[i].first == dev) {
                *out = g_sync_pool[i].second;
                g_sync_pool.erase(g_sync_pool.begin() + (long)i);
                return hipSuccess;
            }
    }
    return hipExtMallocWithFlags(out, persistent_sync_bytes(), hipDeviceMallocUncached);
}

static void return_sync_area(int dev, void* p) {
    std::lock_guard<std::mutex> lk(g_sync_mu);
    g_sync_pool.emplace_back(dev, p);
}

struct icua_engine {
    int fmt = 0, layers = 0, maxctx = 0, maxpass = 0, maxsteps = 0;
    uint32_t flags = 0;
    int eos0 = 151645, eos1 = 151643;  // Engine.swift:12
    hipStream_t stream = nullptr;
    uint8_t* d_weights = nullptr;
    size_t weight_bytes = 0;
    const uint8_t *E = nullptr, *Esb = nullptr;
    const float* final_norm = nullptr;
    LayerW L[MAX_LAYERS];
    float *x = nullptr, *qkv = nullptr, *rope = nullptr, *part = nullptr, *pval = nullptr, *logits = nullptr;
    float *attn = nullptr, *h = nullptr;
    uint16_t* kv = nullptr;
    int splits = 0;
    uint8_t* apre = nullptr;  // pre-staged GEMV operands of multi-row passes
    float* fxpre = nullptr;
    float* kpart = nullptr;  // split-K partials of the down GEMV [3][MAXM][H]
    int* kcnt = nullptr;     // its arrival counters [H / 16]
    int *counters = nullptr, *pidx = nullptr, *out_tokens = nullptr, *prompt = nullptr, *argmax_rows = nullptr;
    State* st = nullptr;
    float* pooler = nullptr;
    float* ds[3] = {nullptr, nullptr, nullptr};
    bool has_ds = false;
    int n_vis = 0;
    hipGraphExec_t graph[2] = {nullptr, nullptr};
    hipEvent_t ev0 = nullptr, ev1 = nullptr;
    icua_timing_t timing{};
    // Prefix cache key: the tokens whose K/V rows occupy slots 0..size-1 (empty: no valid prefix).
    std::vector<int32_t> cached_prefix;
    int mrope_key[3] = {-999, 0, 0};
    int last_logits_rows = 0;
    // Persistent decode kernel: packet area (from the uncached pool, on device psync_dev) and
    // availability; whether the last decode call used it.
    unsigned* psync = nullptr;
    int psync_dev = -1;
    bool last_persistent = false;
    int pair_passes = 0;  // two-row persistent launches (forced grammar pairs) since create
    bool persist_ok = false;
    // Matrix-core prefill buffers for chunks of up to pf_cap rows (allocated on first use).
    int pf_cap = 0;
    float *px = nullptr, *pqkv = nullptr, *patt = nullptr, *ph = nullptr, *pxs = nullptr, *pts = nullptr;
    uint16_t *pxa = nullptr, *pqh = nullptr, *pql = nullptr;
    // Vision tower, when the image holds it: weights, work buffers (one allocation, on first
    // use), the host copy of the position table, the prepared grid and the frame hash.
    uint8_t* d_vision = nullptr;
    size_t vision_bytes = 0;
    VitWeights vw{};
    VitBuffers vb{};
    void* vbuf = nullptr;
    std::vector<float> vit_pos_host;
    int vgrid[2] = {0, 0};
    int vis_cap = 0;  // rows of pooler / ds
    uint64_t rgb_hash = 0;
    int rgb_dims[2] = {0, 0};
    bool has_cached_vision = false;

    uint16_t* kv_ptr(int l, int kind) const { return kv + ((size_t)l * 2 + kind) * NKV * (size_t)maxctx * HD; }

    int read_state(State& s) {
        HIPCK(hipMemcpyAsync(&s, st, sizeof s, hipMemcpyDeviceToHost, stream));
        HIPCK(hipStreamSynchronize(stream));
        return 0;
    }
    int write_state(const State& s) {
        HIPCK(hipMemcpyAsync(st, &s, sizeof s, hipMemcpyHostToDevice, stream));
        HIPCK(hipStreamSynchronize(stream));
        return 0;
    }

    // One GEMV of the pass.  Multi-row q4 / q8 passes run the streaming kernel (the rows
    // staged once per workgroup, one workgroup per CU).  Multi-row f16 gate|up and lm_head passes
    // stage their activation operands once in a separate launch first: their 768 / 1024
    // workgroups would otherwise each repeat the RMSNorm and the slicing of every row.
    int gemv(GemvOp op, GemvArgs& a, int mt) {
        if (mt > 1 && gemv8_supports(fmt, op, a.N)) {
            HIPCK(launch_gemv8(fmt, op, a, stream));
            return 0;
        }
        const bool pre = mt > 1 && (op == GEMV_GU || op == GEMV_LMHEAD);
        a.apre = pre ? apre : nullptr;
        a.fxpre = pre ? fxpre : nullptr;
        if (pre) HIPCK(launch_gemv_prep(fmt, op, a, stream));
        HIPCK(launch_gemv(fmt, op, a, mt, stream));
        return 0;
    }

    // encodeLLMLayer for the rows of the current pass (pos / n from the control block).
    int enqueue_layer(int l, int mt, int row0) {
        const LayerW& w = L[l];
        GemvArgs a{};
        a.st = st;
        a.m_fixed = 0;
        // 1. RMSNorm + fused QKV.
        a.w = w.wqkv;
        a.sb = w.wqkv_sb;
        a.N = QKV;
        a.x = x;
        a.norm_w = w.attn_norm;
        a.y = qkv;
        if (gemv(GEMV_QKV, a, mt)) return -1;
        // 2. q/k norm + M-RoPE + KV write + causal GQA attention.
        AttnArgs t{};
        t.qkv = qkv;
        t.q_norm = w.q_norm;
        t.k_norm = w.k_norm;
        t.rope = rope;
        t.kc = kv_ptr(l, 0);
        t.vc = kv_ptr(l, 1);
        t.part = part;
        t.out = attn;
        t.st = st;
        HIPCK(launch_attention(t, mt, splits, stream));
        // 3. O projection + residual.
        a.w = w.wo;
        a.sb = w.wo_sb;
        a.N = H;
        a.x = attn;
        a.norm_w = nullptr;
        a.y = x;
        if (gemv(GEMV_O, a, mt)) return -1;
        // 4. RMSNorm + gate|up + SwiGLU.
        a.w = w.wgu;
        a.sb = w.wgu_sb;
        a.N = GU;
        a.x = x;
        a.norm_w = w.mlp_norm;
        a.h = h;
        if (gemv(GEMV_GU, a, mt)) return -1;
        // 5. Down projection + residual (+ DeepStack after layers 0-2 at visual rows).
        a.w = w.wd;
        a.sb = w.wd_sb;
        a.N = H;
        a.x = h;
        a.norm_w = nullptr;
        a.y = x;
        a.ds = (has_ds && l < 3) ? ds[l] : nullptr;
        a.ds_row0 = row0;
        a.kpart = kpart;
        a.kcnt = kcnt;
        if (gemv(GEMV_DOWN, a, mt)) return -1;
        return 0;
    }

    int enqueue_head(int mt, int verify_only) {
        GemvArgs a{};
        a.st = st;
        a.w = E;
        a.sb = Esb;
        a.N = VOCAB;
        a.x = x;
        a.norm_w = final_norm;
        a.pval = pval;
        a.pidx = pidx;
        a.logits = logits;
        if (gemv(GEMV_LMHEAD, a, mt)) return -1;
        CommitArgs c{};
        c.pval = pval;
        c.pidx = pidx;
        c.st = st;
        c.out_tokens = out_tokens;
        c.E = E;
        c.Esb = Esb;
        c.fmt = fmt;
        c.x = x;
        c.argmax_rows = argmax_rows;
        c.verify_only = verify_only;
        HIPCK(launch_commit(c, stream));
        return 0;
    }

    int enqueue_step(int mt) {
        for (int l = 0; l < layers; ++l)
            if (enqueue_layer(l, mt, 0)) return -1;
        return enqueue_head(mt, 0);
    }

    int decode_mt() const { return (flags & ICUA_FLAG_GRAMMAR_PAIRS) ? MAXM : 1; }

    int ensure_graph(int mt) {
        const int gi = mt == 1 ? 0 : 1;
        if (graph[gi]) return 0;
        // Eager dry run with done = 1 so every kernel and attribute is set up before capture.
        State s;
        if (read_state(s)) return -1;
        State dry = s;
        dry.done = 1;
        if (write_state(dry) || enqueue_step(mt)) return -1;
        HIPCK(hipStreamSynchronize(stream));
        if (write_state(s)) return -1;
        hipGraph_t g;
        HIPCK(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal));
        int rc = enqueue_step(mt);
        hipError_t e2 = hipStreamEndCapture(stream, &g);
        if (rc) return rc;
        HIPCK(e2);
        HIPCK(hipGraphInstantiate(&graph[gi], g, nullptr, nullptr, 0));
        HIPCK(hipGraphDestroy(g));
        return 0;
    }

    int init_device(const uint8_t* img, size_t len, int max_ctx, int max_pass, int max_steps, uint32_t fl) {
        if (len < 16384 || len % 16384) return fail("bad model size " + std::to_string(len));
        const uint32_t* hdr = (const uint32_t*)img;
        if (hdr[0] != MAGIC) return fail("not an instantcua model");
        if (hdr[1] != 1) return fail("unsupported version");
        if (hdr[2] > 2) return fail("unknown weight format");
        if (hdr[3] != (uint32_t)T_COUNT) return fail("tensor table mismatch");
        if (max_ctx < 1 || max_ctx > 16384) return fail("max_ctx must be in 1..16384");
        fmt = (int)hdr[2];
        maxctx = max_ctx;
        maxpass = max_pass;
        maxsteps = max_steps;
        flags = fl;
        const uint64_t* tab = (const uint64_t*)(img + 16);
        // Expected sizes of every decoder tensor; the layer stack ends at the first empty QKV.
        struct Want {
            int id;
            size_t bytes;
        };
        std::vector<Want> want = {{T_EMBED, code_bytes(fmt, VOCAB, H)},
                                  {T_EMBED_SB, sb_bytes(fmt, VOCAB, H)},
                                  {T_FINAL_NORM, (size_t)H * 4}};
        layers = 0;
        while (layers < MAX_LAYERS && tab[2 * (T_LAYER_BASE + layers * T_PER_LAYER + 1) + 1] != 0) layers++;
        if (layers == 0) return fail("model has no decoder layers");
        for (int l = 0; l < layers; ++l) {
            const int b = T_LAYER_BASE + l * T_PER_LAYER;
            want.push_back({b + 0, (size_t)H * 4});
            want.push_back({b + 1, code_bytes(fmt, QKV, H)});
            want.push_back({b + 2, sb_bytes(fmt, QKV, H)});
            want.push_back({b + 3, (size_t)HD * 4});
            want.push_back({b + 4, (size_t)HD * 4});
            want.push_back({b + 5, code_bytes(fmt, H, H)});
            want.push_back({b + 6, sb_bytes(fmt, H, H)});
            want.push_back({b + 7, (size_t)H * 4});
            want.push_back({b + 8, code_bytes(fmt, GU, H)});
            want.push_back({b + 9, sb_bytes(fmt, GU, H)});
            want.push_back({b + 10, code_bytes(fmt, H, FF)});
            want.push_back({b + 11, sb_bytes(fmt, H, FF)});
        }
        std::vector<size_t> dev_off(T_COUNT, 0);
        size_t total = 0;
        for (const Want& w : want) {
            const uint64_t off = tab[2 * w.id], sz = tab[2 * w.id + 1];
            if (sz != w.bytes || off + sz > len)
                return fail("tensor " + std::to_string(w.id) + ": size " + std::to_string(sz) + ", want " +
                            std::to_string(w.bytes));
            total = (total + 255) & ~(size_t)255;
            dev_off[w.id] = total;
            total += w.bytes;
        }
        weight_bytes = total;
        HIPCK(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking));
        HIPCK(hipEventCreate(&ev0));
        HIPCK(hipEventCreate(&ev1));
        HIPCK(hipMalloc(&d_weights, total));
        // Matrices are repacked into the GEMV tile layout through a staging buffer; norm vectors
        // are copied as they are.
        struct Mat {
            int codes, sb, rows, K, gu;
        };
        std::vector<Mat> mats = {{T_EMBED, T_EMBED_SB, VOCAB, H, 0}};
        for (int l = 0; l < layers; ++l) {
            const int b = T_LAYER_BASE + l * T_PER_LAYER;
            mats.push_back({b + 1, b + 2, QKV, H, 0});
            mats.push_back({b + 5, b + 6, H, H, 0});
            mats.push_back({b + 8, b + 9, GU, H, 1});
            mats.push_back({b + 10, b + 11, H, FF, 0});
        }
        std::vector<bool> is_mat(T_COUNT, false);
        size_t stage_bytes = 0;
        for (const Mat& m : mats) {
            is_mat[m.codes] = is_mat[m.sb] = true;
            stage_bytes = std::max(stage_bytes, code_bytes(fmt, m.rows, m.K) + sb_bytes(fmt, m.rows, m.K) + 256);
        }
        for (const Want& w : want)
            if (!is_mat[w.id] && w.bytes)
                HIPCK(hipMemcpy(d_weights + dev_off[w.id], img + tab[2 * w.id], w.bytes, hipMemcpyHostToDevice));
        uint8_t* staging = nullptr;
        HIPCK(hipMalloc(&staging, stage_bytes));
        for (const Mat& m : mats) {
            const size_t cb = code_bytes(fmt, m.rows, m.K), sbb = sb_bytes(fmt, m.rows, m.K);
            const size_t sb_off = (cb + 255) & ~(size_t)255;
            HIPCK(hipMemcpy(staging, img + tab[2 * m.codes], cb, hipMemcpyHostToDevice));
            if (sbb) HIPCK(hipMemcpy(staging + sb_off, img + tab[2 * m.sb], sbb, hipMemcpyHostToDevice));
            HIPCK(launch_repack(fmt, staging, staging + sb_off, d_weights + dev_off[m.codes], d_weights + dev_off[m.sb],
                                m.rows, m.K, m.gu, nullptr));
            HIPCK(hipDeviceSynchronize());
        }
        HIPCK(hipFree(staging));
        auto P = [&](int id) { return d_weights + dev_off[id]; };
        E = P(T_EMBED);
        Esb = P(T_EMBED_SB);
        final_norm = (const float*)P(T_FINAL_NORM);
        for (int l = 0; l < layers; ++l) {
            const int b = T_LAYER_BASE + l * T_PER_LAYER;
            LayerW& w = L[l];
            w.attn_norm = (const float*)P(b + 0);
            w.wqkv = P(b + 1);
            w.wqkv_sb = P(b + 2);
            w.q_norm = (const float*)P(b + 3);
            w.k_norm = (const float*)P(b + 4);
            w.wo = P(b + 5);
            w.wo_sb = P(b + 6);
            w.mlp_norm = (const float*)P(b + 7);
            w.wgu = P(b + 8);
            w.wgu_sb = P(b + 9);
            w.wd = P(b + 10);
            w.wd_sb = P(b + 11);
        }
        HIPCK(hipMalloc(&x, sizeof(float) * MAXM * H));
        HIPCK(hipMalloc(&qkv, sizeof(float) * MAXM * QKV));
        HIPCK(hipMalloc(&attn, sizeof(float) * MAXM * H));
        HIPCK(hipMalloc(&h, sizeof(float) * MAXM * FF));
        // The multi-row GEMVs stage every row of these buffers (only the pass's rows are
        // written): rows no pass has written yet hold zeros.
        HIPCK(hipMemset(x, 0, sizeof(float) * MAXM * H));
        HIPCK(hipMemset(attn, 0, sizeof(float) * MAXM * H));
        HIPCK(hipMemset(h, 0, sizeof(float) * MAXM * FF));
        const size_t kvn = (size_t)layers * 2 * NKV * maxctx * HD;
        HIPCK(hipMalloc(&kv, kvn * 2));
        HIPCK(hipMemset(kv, 0, kvn * 2));
        HIPCK(hipMalloc(&rope, sizeof(float) * (size_t)maxctx * 128));
        splits = attention_splits(maxctx);
        HIPCK(hipMalloc(&part, sizeof(float) * (size_t)NKV * splits * MAXM * 2 * (HD + 2)));
        HIPCK(hipMalloc(&apre, GEMV_PREP_BYTES));
        HIPCK(hipMalloc(&fxpre, GEMV_PREP_FX_BYTES));
        HIPCK(hipMalloc(&kpart, sizeof(float) * 3 * MAXM * H));
        HIPCK(hipMalloc(&kcnt, sizeof(int) * (H / 16)));
        HIPCK(hipMemset(kcnt, 0, sizeof(int) * (H / 16)));
        HIPCK(hipMalloc(&counters, sizeof(int) * NKV));
        HIPCK(hipMemset(counters, 0, sizeof(int) * NKV));
        HIPCK(hipMalloc(&pval, sizeof(float) * MAXM * LMH_WAVES));
        HIPCK(hipMalloc(&pidx, sizeof(int) * MAXM * LMH_WAVES));
        HIPCK(hipMalloc(&logits, sizeof(float) * (size_t)MAXM * VOCAB));
        HIPCK(hipMalloc(&out_tokens, sizeof(int) * (maxsteps + 4)));
        HIPCK(hipMemset(out_tokens, 0, sizeof(int) * (maxsteps + 4)));
        HIPCK(hipMalloc(&prompt, sizeof(int) * (size_t)std::max(maxctx, MAXM)));
        HIPCK(hipMalloc(&argmax_rows, sizeof(int) * MAXM));
        HIPCK(hipMalloc(&st, sizeof(State)));
        State s{};
        s.done = 1;
        s.n = 1;
        s.maxctx = maxctx;
        s.maxsteps = maxsteps;
        s.eos0 = eos0;
        s.eos1 = eos1;
        s.vis_offset = -1;
        if (write_state(s)) return -1;
        if (init_persistent()) return -1;
        if (init_vision(img, len, tab)) return -1;
        return prepare_mrope(-1, 1, 1);
    }

    // Vision tensors (ModelFile.swift:64-87, Convert.swift:97-152): copied as they are into one
    // device block.  An image without them (slot 0 empty) loads as a text-only model.
    int init_vision(const uint8_t* img, size_t len, const uint64_t* tab) {
        if (tab[1] == 0) return 0;
        struct Want {
            int id;
            size_t bytes;
        };
        std::vector<Want> want = {{0, (size_t)VH * VPATCH * 2}, {1, (size_t)VH * 4}, {2, (size_t)VPOS * VPOS * VH * 4}};
        for (int l = 0; l < VLAYERS; ++l) {
            const int b = 3 + 12 * l;
            const size_t sz[12] = {VH * 4,          VH * 4, (size_t)VQKV * VH * 2, VQKV * 4,
                                   (size_t)VH * VH * 2, VH * 4, VH * 4,                VH * 4,
                                   (size_t)VFF * VH * 2, VFF * 4, (size_t)VH * VFF * 2, VH * 4};
            for (int k = 0; k < 12; ++k) want.push_back({b + k, sz[k]});
        }
        for (int d = 0; d < 4; ++d) {
            const int b = 3 + 12 * VLAYERS + 6 * d;
            const size_t nn = d < 3 ? MH : VH;  // DeepStack mergers normalise 4096 columns
            const size_t sz[6] = {nn * 4, nn * 4, (size_t)MH * MH * 2, MH * 4, (size_t)H * MH * 2, H * 4};
            for (int k = 0; k < 6; ++k) want.push_back({b + k, sz[k]});
        }
        std::vector<size_t> off(want.size());
        size_t total = 0;
        for (size_t i = 0; i < want.size(); ++i) {
            const uint64_t o = tab[2 * want[i].id], sz = tab[2 * want[i].id + 1];
            if (sz != want[i].bytes || o + sz > len)
                return fail("vision tensor " + std::to_string(want[i].id) + ": size " + std::to_string(sz) + ", want " +
                            std::to_string(want[i].bytes));
            total = (total + 255) & ~(size_t)255;
            off[i] = total;
            total += want[i].bytes;
        }
        HIPCK(hipMalloc(&d_vision, total));
        vision_bytes = total;
        for (size_t i = 0; i < want.size(); ++i)
            HIPCK(hipMemcpy(d_vision + off[i], img + tab[2 * want[i].id], want[i].bytes, hipMemcpyHostToDevice));
        auto F = [&](size_t i) { return (const float*)(d_vision + off[i]); };
        auto W = [&](size_t i) { return (const uint16_t*)(d_vision + off[i]); };
        vw.patch_w = W(0);
        vw.patch_b = F(1);
        for (int l = 0; l < VLAYERS; ++l) {
            const size_t b = 3 + 12 * l;
            VitBlock& B = vw.blk[l];
            B.n1w = F(b);
            B.n1b = F(b + 1);
            B.qkvw = W(b + 2);
            B.qkvb = F(b + 3);
            B.projw = W(b + 4);
            B.projb = F(b + 5);
            B.n2w = F(b + 6);
            B.n2b = F(b + 7);
            B.fc1w = W(b + 8);
            B.fc1b = F(b + 9);
            B.fc2w = W(b + 10);
            B.fc2b = F(b + 11);
        }
        for (int d = 0; d < 4; ++d) {
            const size_t b = 3 + 12 * VLAYERS + 6 * d;
            VitMerger& M = vw.mg[d];
            M.nw = F(b);
            M.nb = F(b + 1);
            M.fc1w = W(b + 2);
            M.fc1b = F(b + 3);
            M.fc2w = W(b + 4);
            M.fc2b = F(b + 5);
        }
        vit_pos_host.resize((size_t)VPOS * VPOS * VH);
        std::memcpy(vit_pos_host.data(), img + tab[2 * 2], vit_pos_host.size() * 4);
        return 0;
    }

    // Visual rows for n rows (pooler and the three DeepStack sets), kept when large enough.
    int ensure_visual_rows(int n) {
        if (n <= vis_cap) return 0;
        if (pooler) (void)hipFree(pooler);
        for (auto& d : ds)
            if (d) {
                (void)hipFree(d);
                d = nullptr;
            }
        pooler = nullptr;
        vis_cap = 0;
        HIPCK(hipMalloc(&pooler, sizeof(float) * (size_t)n * H));
        for (auto& d : ds) HIPCK(hipMalloc(&d, sizeof(float) * (size_t)n * H));
        vis_cap = n;
        return 0;
    }

    // prepareVisionGrid (Engine.swift:189-246): the interpolated position table and the 2D RoPE
    // table of a gh x gw grid in merge-block order, in the engine's float32 operation order.
    int prepare_vision_grid(int gh, int gw) {
#pragma clang fp contract(off)
        if (vgrid[0] == gh && vgrid[1] == gw) return 0;
        const int np = gh * gw, mw = gw / 2;
        std::vector<float> pos((size_t)np * VH), rope((size_t)np * 64);
        float invf[16];
        for (int i = 0; i < 16; ++i) invf[i] = (float)(1.0 / std::pow(10000.0, (double)(2 * i) / 32.0));
        for (int p = 0; p < np; ++p) {
            const int blk = p / 4, in = p % 4;
            const int r = (blk / mw) * 2 + in / 2, c = (blk % mw) * 2 + in % 2;
            const float y = (float)r * (float)(VPOS - 1) / (float)std::max(1, gh - 1);
            const float xx = (float)c * (float)(VPOS - 1) / (float)std::max(1, gw - 1);
            const int y0 = (int)std::floor(y), x0 = (int)std::floor(xx);
            const int y1 = std::min(VPOS - 1, y0 + 1), x1 = std::min(VPOS - 1, x0 + 1);
            const float dy = y - (float)y0, dx = xx - (float)x0;
            const float w00 = (1.0f - dy) * (1.0f - dx), w01 = (1.0f - dy) * dx, w10 = dy * (1.0f - dx), w11 = dy * dx;
            const float* p00 = vit_pos_host.data() + (size_t)(y0 * VPOS + x0) * VH;
            const float* p01 = vit_pos_host.data() + (size_t)(y0 * VPOS + x1) * VH;
            const float* p10 = vit_pos_host.data() + (size_t)(y1 * VPOS + x0) * VH;
            const float* p11 = vit_pos_host.data() + (size_t)(y1 * VPOS + x1) * VH;
            float* d = pos.data() + (size_t)p * VH;
            for (int k = 0; k < VH; ++k) {
                float t = w00 * p00[k];  // one rounding per operation, as the engine
                t = t + w01 * p01[k];
                t = t + w10 * p10[k];
                t = t + w11 * p11[k];
                d[k] = t;
            }
            float* rr = rope.data() + (size_t)p * 64;
            for (int i = 0; i < 16; ++i) {
                const double ah = (double)((float)r * invf[i]), aw = (double)((float)c * invf[i]);
                rr[2 * i] = (float)std::cos(ah);
                rr[2 * i + 1] = (float)std::sin(ah);
                rr[2 * (16 + i)] = (float)std::cos(aw);
                rr[2 * (16 + i) + 1] = (float)std::sin(aw);
            }
        }
        HIPCK(hipMemcpy((void*)vb.pos, pos.data(), pos.size() * 4, hipMemcpyHostToDevice));
        HIPCK(hipMemcpy((void*)vb.rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice));
        vgrid[0] = gh;
        vgrid[1] = gw;
        return 0;
    }

    // encodeVision (Engine.swift:317-473) of an RGB8 frame [height][width][3].
    int vision(const uint8_t* rgb, int width, int height, double* ms) {
        if (!d_vision) return fail("the model file has no vision tower");
        if (width <= 0 || height <= 0 || width % 32 || height % 32)
            return fail("image sides must be positive multiples of 32");
        const int gh = height / 16, gw = width / 16, np = gh * gw;
        if (np > NPATCH_MAX) return fail("image has more than 1024 patches");
        if (!vbuf) {
            const size_t n = NPATCH_MAX;
            const size_t sz[] = {n * 256 * 3, n * VPATCH * 2, n * VH * 4, n * VH * 2, (size_t)VNH * n * VHD * 2,
                                 (size_t)VNH * n * VHD * 2, (size_t)VNH * VHD * n * 2, n * VH * 2, n * VFF * 2,
                                 n * VH * 4, n * 64 * 4};
            size_t o[11], total = 0;
            for (int i = 0; i < 11; ++i) {
                o[i] = total;
                total += (sz[i] + 255) & ~(size_t)255;
            }
            HIPCK(hipMalloc(&vbuf, total));
            HIPCK(hipMemset(vbuf, 0, total));  // padded key rows of q / k / v stay finite
            uint8_t* b = (uint8_t*)vbuf;
            vb.rgb = b + o[0];
            vb.patches = (uint16_t*)(b + o[1]);
            vb.x = (float*)(b + o[2]);
            vb.xn = (uint16_t*)(b + o[3]);
            vb.q = (uint16_t*)(b + o[4]);
            vb.k = (uint16_t*)(b + o[5]);
            vb.vt = (uint16_t*)(b + o[6]);
            vb.attn = (uint16_t*)(b + o[7]);
            vb.h = (uint16_t*)(b + o[8]);
            vb.pos = (const float*)(b + o[9]);
            vb.rope = (const float*)(b + o[10]);
        }
        if (ensure_visual_rows(NPATCH_MAX / 4)) return -1;
        vb.pooler = pooler;
        for (int i = 0; i < 3; ++i) vb.ds[i] = ds[i];
        if (prepare_vision_grid(gh, gw)) return -1;
        HIPCK(hipMemcpyAsync((void*)vb.rgb, rgb, (size_t)width * height * 3, hipMemcpyHostToDevice, stream));
        HIPCK(hipEventRecord(ev0, stream));
        HIPCK(launch_vision(vw, vb, gh, gw, stream));
        HIPCK(hipEventRecord(ev1, stream));
        HIPCK(hipEventSynchronize(ev1));
        float t = 0;
        HIPCK(hipEventElapsedTime(&t, ev0, ev1));
        if (ms) *ms = t;
        n_vis = np / 4;
        has_ds = true;
        return 0;
    }

    // The persistent kernel needs all PERSIST_WGS workgroups (one per CU) resident at once.
    int init_persistent() {
        persist_ok = false;
        int dev = 0, coop = 0, cus = 0;
        HIPCK(hipGetDevice(&dev));
        HIPCK(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, dev));
        HIPCK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
        if (!coop || cus < PERSIST_WGS) return 0;
        HIPCK(take_sync_area(dev, (void**)&psync));
        psync_dev = dev;
        persist_ok = true;
        return 0;
    }

    bool use_persistent() const { return persist_ok && !(flags & ICUA_FLAG_GRAPH_DECODE); }

    // One persistent launch: nr = 1, k single-row passes (ending early at a forced pair, which it
    // leaves pending); nr = 2, the pending pair as one two-row pass (k = 1).
    int enqueue_persistent(int k, int nr) {
        PersistArgs a{};
        for (int l = 0; l < layers; ++l) {
            const LayerW& w = L[l];
            a.layers[l] = LayerPtrs{w.attn_norm, w.q_norm, w.k_norm, w.mlp_norm, w.wqkv, w.wqkv_sb,
                                    w.wo,        w.wo_sb,  w.wgu,    w.wgu_sb,   w.wd,   w.wd_sb};
        }
        a.nlayers = layers;
        a.nsteps = k;
        a.maxctx = maxctx;
        a.E = E;
        a.Esb = Esb;
        a.final_norm = final_norm;
        a.rope = rope;
        a.kv = kv;
        a.x = x;
        a.st = st;
        a.out_tokens = out_tokens;
        a.ll = (uint64_t*)psync;
        HIPCK(hipMemsetAsync(psync, 0, persistent_clear_bytes(nr), stream));
        HIPCK(hipMemsetAsync(psync + persistent_error_slot(), 0, sizeof(unsigned), stream));
        HIPCK(launch_persistent(fmt, nr, a, stream));
        return 0;
    }

    // Error flag of the last persistent launch (a bounded wait timed out).
    int check_persistent() {
        unsigned err = 0;
        HIPCK(hipMemcpy(&err, psync + persistent_error_slot(), sizeof err, hipMemcpyDeviceToHost));
        if (err) return fail("persistent decode kernel: a synchronisation wait timed out");
        return 0;
    }

    // Any write of K/V rows below the cached prefix's end invalidates the prefix cache.
    void kv_written_from(int slot0) {
        if (slot0 < (int)cached_prefix.size()) cached_prefix.clear();
    }

    int prepare_mrope(int vis_offset, int llm_h, int llm_w) {
        if (vis_offset >= 0 && (llm_h <= 0 || llm_w <= 0)) return fail("bad visual grid");
        if (vis_offset < 0) vis_offset = -1, llm_h = llm_w = 1;  // one key for every text-only table
        if (mrope_key[0] == vis_offset && mrope_key[1] == llm_h && mrope_key[2] == llm_w) return 0;
        std::vector<float> tab;
        mrope_table(maxctx, vis_offset, llm_h, llm_w, tab);
        HIPCK(hipMemcpy(rope, tab.data(), tab.size() * sizeof(float), hipMemcpyHostToDevice));
        mrope_key[0] = vis_offset;
        mrope_key[1] = llm_h;
        mrope_key[2] = llm_w;
        return 0;
    }

    void free_pf() {
        void* bufs[] = {px, pqkv, patt, ph, pxs, pts, pxa, pqh, pql};
        for (void* b : bufs)
            if (b) (void)hipFree(b);
        px = pqkv = patt = ph = pxs = pts = nullptr;
        pxa = pqh = pql = nullptr;
        pf_cap = 0;
    }

    int ensure_pf(int rows) {
        const int cap = (rows + 127) / 128 * 128;
        if (cap <= pf_cap) return 0;
        HIPCK(hipStreamSynchronize(stream));
        free_pf();
        HIPCK(hipMalloc(&px, sizeof(float) * cap * H));
        HIPCK(hipMalloc(&pqkv, sizeof(float) * cap * QKV));
        HIPCK(hipMalloc(&patt, sizeof(float) * cap * H));
        HIPCK(hipMalloc(&ph, sizeof(float) * cap * FF));
        HIPCK(hipMalloc(&pxa, sizeof(uint16_t) * 2 * (size_t)cap * FF));
        HIPCK(hipMalloc(&pxs, sizeof(float) * (size_t)cap * (FF / 64)));
        HIPCK(hipMalloc(&pts, sizeof(float) * (size_t)cap));
        HIPCK(hipMalloc(&pqh, sizeof(uint16_t) * (size_t)cap * NH * HD));
        HIPCK(hipMalloc(&pql, sizeof(uint16_t) * (size_t)cap * NH * HD));
        // Rows beyond a chunk's M are read (never stored) by the attention kernel: keep them finite.
        HIPCK(hipMemset(pqh, 0, sizeof(uint16_t) * (size_t)cap * NH * HD));
        HIPCK(hipMemset(pql, 0, sizeof(uint16_t) * (size_t)cap * NH * HD));
        pf_cap = cap;
        return 0;
    }

    // One decoder layer over chunk rows [0, M) at cache slots p0.. (prompt rows row0..).
    int enqueue_pf_layer(int l, int M, int Mpad, int p0, int row0, int vis_offset) {
        const LayerW& w = L[l];
        PfGemmArgs g{};
        g.xa = pxa;
        g.xs = pxs;
        g.ts = pts;
        g.M = M;
        g.Mpad = Mpad;
        g.row0 = row0;
        g.vis_offset = vis_offset;
        g.n_vis = n_vis;
        // fp16 operands: hi + lo parts (~22 bits), or with ICUA_FLAG_PREFILL_FP16 the hi part alone
        // (fp16 activations, queries and probabilities: the reference engine's precision).
        const int parts = (flags & ICUA_FLAG_PREFILL_FP16) ? 1 : 2;
        g.parts = parts;
        // 1. RMSNorm + fused QKV.
        HIPCK(launch_pf_prep(H, 1, px, w.attn_norm, M, Mpad, pxa, pxs, pts, parts, stream));
        g.w = w.wqkv;
        g.sb = w.wqkv_sb;
        g.N = QKV;
        g.y = pqkv;
        HIPCK(launch_pf_gemm(fmt, H, EPI_STORE, g, stream));
        // 2. q/k norm + M-RoPE + KV write, causal flash attention.
        uint16_t* ql = parts == 2 ? pql : nullptr;
        PfQkArgs qa{pqkv, w.q_norm, w.k_norm, rope, kv_ptr(l, 0), kv_ptr(l, 1), pqh, ql, M, p0, maxctx};
        HIPCK(launch_pf_qk(qa, stream));
        PfAttnArgs aa{pqh, ql, kv_ptr(l, 0), kv_ptr(l, 1), patt, M, p0, maxctx};
        HIPCK(launch_pf_attn(aa, stream));
        // 3. O projection + residual.
        HIPCK(launch_pf_prep(H, 0, patt, nullptr, M, Mpad, pxa, pxs, pts, parts, stream));
        g.w = w.wo;
        g.sb = w.wo_sb;
        g.N = H;
        g.y = px;
        HIPCK(launch_pf_gemm(fmt, H, EPI_RESID, g, stream));
        // 4. RMSNorm + gate|up + SwiGLU.
        HIPCK(launch_pf_prep(H, 1, px, w.mlp_norm, M, Mpad, pxa, pxs, pts, parts, stream));
        g.w = w.wgu;
        g.sb = w.wgu_sb;
        g.N = GU;
        g.h = ph;
        HIPCK(launch_pf_gemm(fmt, H, EPI_SWIGLU, g, stream));
        // 5. Down projection + residual (+ DeepStack after layers 0-2 at visual rows).
        HIPCK(launch_pf_prep(FF, 0, ph, nullptr, M, Mpad, pxa, pxs, pts, parts, stream));
        g.w = w.wd;
        g.sb = w.wd_sb;
        g.N = H;
        g.y = px;
        g.ds = (has_ds && l < 3) ? ds[l] : nullptr;
        HIPCK(launch_pf_gemm(fmt, FF, EPI_RESID, g, stream));
        return 0;
    }

    // Matrix-core prefill of prompt rows [0, n) at slots start_pos.., then the last row's
    // lm_head + commit as a one-row pass.  The state was written by prefill().
    int prefill_chunks(int n, int start_pos, int vis_offset, int write_logits) {
        if (ensure_pf(std::min(n, PF_CHUNK))) return -1;
        int M = 0;
        for (int c0 = 0; c0 < n; c0 += PF_CHUNK) {
            M = std::min(PF_CHUNK, n - c0);
            const int Mpad = (M + 127) / 128 * 128;
            EmbedArgs ea{};
            ea.toks = prompt;
            ea.E = E;
            ea.Esb = Esb;
            ea.fmt = fmt;
            ea.pooler = vis_offset >= 0 ? pooler : nullptr;
            ea.row0 = c0;
            ea.x = px;
            ea.st = st;
            ea.n = M;
            HIPCK(launch_embed(ea, stream));
            for (int l = 0; l < layers; ++l)
                if (enqueue_pf_layer(l, M, Mpad, start_pos + c0, c0, vis_offset)) return -1;
        }
        HIPCK(hipMemcpyAsync(x, px + (size_t)(M - 1) * H, sizeof(float) * H, hipMemcpyDeviceToDevice, stream));
        HIPCK(launch_set_pass(st, start_pos + n - 1, 1, write_logits ? 1 : 0, stream));
        return enqueue_head(MAXM, 0);
    }

    bool use_pf(int n) const { return n > MAXM && !(flags & ICUA_FLAG_PASS_PREFILL); }

    int prefill(const int32_t* tokens, int n, int start_pos, int vis_offset, int max_new, int write_logits) {
        if (n <= 0) return fail("empty prompt");
        if (max_new < 1) max_new = 1;
        if (start_pos < 0 || start_pos + n + max_new - 1 > maxctx) return fail("prompt exceeds max context");
        for (int i = 0; i < n; ++i)
            if (tokens[i] < 0 || tokens[i] >= VOCAB) return fail("token id out of range");
        if (vis_offset >= n) return fail("vis_offset beyond the prompt");
        if (vis_offset >= 0 && n_vis <= 0) return fail("visual rows requested but no visual embeddings set");
        kv_written_from(start_pos);
        HIPCK(hipMemcpyAsync(prompt, tokens, sizeof(int32_t) * n, hipMemcpyHostToDevice, stream));
        State s{};
        s.pos = start_pos;
        s.n = std::min(n, MAXM);
        s.step = 0;
        s.done = 0;
        s.maxctx = maxctx;
        s.maxsteps = std::max(1, std::min(max_new, maxsteps));
        s.eos0 = eos0;
        s.eos1 = eos1;
        s.vis_offset = vis_offset;
        s.n_vis = vis_offset >= 0 ? n_vis : 0;
        s.rope_delta = 0;
        s.flags = (flags & ICUA_FLAG_GRAMMAR_PAIRS) ? STATE_FLAG_GRAMMAR : 0;
        s.logits_rows = 0;
        if (write_state(s)) return -1;
        HIPCK(hipEventRecord(ev0, stream));
        if (use_pf(n)) {
            if (prefill_chunks(n, start_pos, vis_offset, write_logits)) return -1;
        } else {
            if (prefill_passes(n, start_pos, vis_offset, write_logits)) return -1;
        }
        HIPCK(hipEventRecord(ev1, stream));
        HIPCK(hipEventSynchronize(ev1));
        float ms = 0;
        HIPCK(hipEventElapsedTime(&ms, ev0, ev1));
        timing.prefill_ms = ms;
        timing.prefill_tokens = n;
        last_logits_rows = write_logits ? 1 : 0;
        return 0;
    }

    int prefill_passes(int n, int start_pos, int vis_offset, int write_logits) {
        for (int r0 = 0; r0 < n; r0 += MAXM) {
            const int m = std::min(MAXM, n - r0);
            const bool last = (r0 + m == n);
            HIPCK(launch_set_pass(st, start_pos + r0, m, last && write_logits ? 1 : 0, stream));
            EmbedArgs ea{};
            ea.toks = prompt;
            ea.E = E;
            ea.Esb = Esb;
            ea.fmt = fmt;
            ea.pooler = vis_offset >= 0 ? pooler : nullptr;
            ea.row0 = r0;
            ea.x = x;
            ea.st = st;
            ea.n = m;
            HIPCK(launch_embed(ea, stream));
            for (int l = 0; l < layers; ++l)
                if (enqueue_layer(l, MAXM, r0)) return -1;
        }
        return enqueue_head(MAXM, 0);
    }

    int decode_steps(int k, double* ms_out) {
        if (k < 0) return fail("negative step count");
        bool persistent = use_persistent();
        State s;
        if (persistent) {  // single-row passes, or a pending forced pair (run as two rows)
            if (read_state(s)) return -1;
            if (s.n < 1 || s.n > 2 || (s.n == 2 && !(s.flags & STATE_FLAG_GRAMMAR))) persistent = false;
        }
        last_persistent = persistent;
        const int mt = decode_mt();
        if (!persistent && ensure_graph(mt)) return -1;
        HIPCK(hipEventRecord(ev0, stream));
        HIPCK(hipEventRecord(ev1, stream));
        if (persistent) {
            // k passes: launches of single-row passes, and each forced grammar pair as one launch
            // of a two-row pass (Shaders.swift:1553: the reference's n = 2 pass).  A single-row
            // launch ends at a commit that forces a pair; the control block then holds n = 2.
            // ev1 follows the last launch (the host reads the control block between launches).
            int left = k;
            while (left > 0 && !s.done) {
                const int nr = s.n == 2 ? 2 : 1, step0 = s.step;
                if (nr == 2 && fmt == FMT_F16) {
                    // The kernel has no two-row form for f16 weights: the pair's pass is one replay
                    // of the per-stage graph (built on first use), which runs n = 2 passes.
                    if (ensure_graph(MAXM)) return -1;
                    HIPCK(hipGraphLaunch(graph[1], stream));
                } else {
                    if (enqueue_persistent(nr == 2 ? 1 : left, nr)) return -1;
                    pair_passes += nr == 2;
                }
                HIPCK(hipEventRecord(ev1, stream));
                if (read_state(s)) return -1;  // waits for the launch
                if (check_persistent()) return -1;
                // Tokens committed, less the forced token of a pair left pending for the next pass.
                const int passes = s.step - step0 - (s.n == 2 && !s.done ? 1 : 0);
                if (passes <= 0) {
                    if (s.done) break;
                    return fail("persistent decode kernel made no progress");
                }
                left -= passes;
            }
        } else {
            for (int i = 0; i < k; ++i) HIPCK(hipGraphLaunch(graph[mt == 1 ? 0 : 1], stream));
            HIPCK(hipEventRecord(ev1, stream));
        }
        HIPCK(hipEventSynchronize(ev1));
        float ms = 0;
        HIPCK(hipEventElapsedTime(&ms, ev0, ev1));
        if (ms_out) *ms_out = ms;
        last_logits_rows = 0;
        return 0;
    }
};

// ---------------------------------------------------------------------------------------------
// C ABI

extern "C" {

const char* icua_last_error(void) { return g_err.c_str(); }

int icua_engine_create_from_memory(const void* image, size_t len, int max_ctx, int max_pass, int max_steps,
                                   uint32_t flags, icua_engine** out) {
    if (!image || !out) return fail("null argument");
    icua_engine* e = new icua_engine();
    if (e->init_device((const uint8_t*)image, len, max_ctx, max_pass, max_steps, flags)) {
        std::string msg = g_err;
        icua_engine_destroy(e);
        g_err = msg;
        return -1;
    }
    *out = e;
    return 0;
}

int icua_engine_create(const char* path, int max_ctx, int max_pass, int max_steps, uint32_t flags,
                       icua_engine** out) {
    if (!path || !out) return fail("null argument");
    int fd = open(path, O_RDONLY);
    if (fd < 0) return fail(std::string("cannot open ") + path);
    struct stat sb;
    if (fstat(fd, &sb) != 0) {
        close(fd);
        return fail(std::string("cannot stat ") + path);
    }
    const size_t size = (size_t)sb.st_size;
    void* p = mmap(nullptr, size, PROT_READ, MAP_SHARED, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return fail(std::string("mmap failed for ") + path);
    int rc = icua_engine_create_from_memory(p, size, max_ctx, max_pass, max_steps, flags, out);
    munmap(p, size);
    return rc;
}

void icua_engine_destroy(icua_engine* e) {
    if (!e) return;
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    for (auto& g : e->graph)
        if (g) (void)hipGraphExecDestroy(g);
    void* bufs[] = {e->d_weights, e->x, e->qkv, e->attn, e->h, e->kv, e->rope, e->part, e->counters, e->kpart, e->kcnt, e->apre, e->fxpre, e->pval,
                    e->pidx, e->logits, e->out_tokens, e->prompt, e->argmax_rows, e->st, e->pooler,
                    e->ds[0], e->ds[1], e->ds[2], e->d_vision, e->vbuf};
    if (e->psync) return_sync_area(e->psync_dev, e->psync);
    e->free_pf();
    for (void* b : bufs)
        if (b) (void)hipFree(b);
    if (e->ev0) (void)hipEventDestroy(e->ev0);
    if (e->ev1) (void)hipEventDestroy(e->ev1);
    if (e->stream) (void)hipStreamDestroy(e->stream);
    delete e;
}

int icua_engine_info(icua_engine* e, icua_info_t* out) {
    if (!e || !out) return fail("null argument");
    out->format = e->fmt;
    out->layers = e->layers;
    out->vision = e->d_vision != nullptr;
    out->max_context = e->maxctx;
    out->max_pass = e->maxpass;
    out->max_steps = e->maxsteps;
    out->weight_bytes = (int64_t)e->weight_bytes;
    out->kv_bytes = (int64_t)e->layers * 2 * NKV * e->maxctx * HD * 2;
    out->persistent_decode = e->persist_ok ? 1 : 0;
    out->last_decode_persistent = e->last_persistent ? 1 : 0;
    out->visual_rows = e->n_vis;
    out->pair_passes = e->pair_passes;
    return 0;
}

int icua_set_eos(icua_engine* e, int32_t eos0, int32_t eos1) {
    if (!e) return fail("null engine");
    e->eos0 = eos0;
    e->eos1 = eos1;
    return 0;
}

int icua_set_flags(icua_engine* e, uint32_t flags) {
    if (!e) return fail("null engine");
    e->flags = flags;
    return 0;
}

int icua_prepare_mrope(icua_engine* e, int vis_offset, int llm_h, int llm_w) {
    if (!e) return fail("null engine");
    return e->prepare_mrope(vis_offset, llm_h, llm_w);
}

int icua_set_visual(icua_engine* e, const float* pooler, const float* const* deepstack, int n_vis) {
    if (!e || !pooler || n_vis <= 0) return fail("bad visual inputs");
    if (n_vis > e->maxctx) return fail("too many visual rows");
    if (e->ensure_visual_rows(n_vis)) return -1;
    e->has_cached_vision = false;  // the rows no longer come from the last encoded frame
    HIPCK(hipMemcpy(e->pooler, pooler, sizeof(float) * (size_t)n_vis * H, hipMemcpyHostToDevice));
    e->has_ds = deepstack != nullptr;
    if (deepstack)
        for (int i = 0; i < 3; ++i)
            HIPCK(hipMemcpy(e->ds[i], deepstack[i], sizeof(float) * (size_t)n_vis * H, hipMemcpyHostToDevice));
    e->n_vis = n_vis;
    return 0;
}

int icua_prefill(icua_engine* e, const int32_t* tokens, int n, int start_pos, int vis_offset, int max_new,
                 int write_logits) {
    if (!e || !tokens) return fail("null argument");
    return e->prefill(tokens, n, start_pos, vis_offset, max_new, write_logits);
}

int icua_decode_steps(icua_engine* e, int k) {
    if (!e) return fail("null engine");
    double ms = 0;
    if (e->decode_steps(k, &ms)) return -1;
    e->timing.decode_ms = ms;
    return 0;
}

int icua_generate(icua_engine* e, const int32_t* tokens, int n, int vis_offset, int max_new, int32_t* out_tokens,
                  int* n_out) {
    if (!e || !tokens || !out_tokens || !n_out) return fail("null argument");
    const auto t0 = std::chrono::steady_clock::now();
    if (n <= 0) return fail("empty prompt");
    if (vis_offset >= n) return fail("vis_offset beyond the prompt");
    if (vis_offset < 0) {
        // Text only: the positions are 1-D whatever table an earlier call prepared.
        if (e->prepare_mrope(-1, 1, 1)) return -1;
    } else {
        // Visual rows: the table must be the one of this image (icua_prepare_mrope, or
        // icua_generate_vision which prepares it from the frame).
        if (e->mrope_key[0] != vis_offset || e->mrope_key[1] * e->mrope_key[2] != e->n_vis)
            return fail("the M-RoPE table was not prepared for this image: call icua_prepare_mrope(vis_offset, "
                        "llm_h, llm_w) with llm_h * llm_w visual rows first");
    }
    // System-prompt KV prefix cache (Engine.swift:719-735).  The key names the tokens whose K/V
    // rows the cache holds; it is set only after a prefill that wrote them succeeded.
    const bool use_cache = (e->flags & ICUA_FLAG_PREFIX_CACHE) && vis_offset > 0;
    const bool hit = use_cache && (int)e->cached_prefix.size() == vis_offset &&
                     std::equal(e->cached_prefix.begin(), e->cached_prefix.end(), tokens);
    const int start = hit ? vis_offset : 0;
    const int active = n - start;
    const int active_vis = vis_offset >= 0 ? vis_offset - start : -1;
    max_new = std::max(1, std::min(max_new, e->maxsteps));
    if (e->prefill(tokens + start, active, start, active_vis, max_new, (e->flags & ICUA_FLAG_FIRST_LOGITS) ? 1 : 0))
        return -1;
    if (use_cache && !hit) e->cached_prefix.assign(tokens, tokens + vis_offset);
    double dec_ms = 0;
    State s;
    if (e->read_state(s)) return -1;
    while (!s.done && s.step < s.maxsteps) {
        // Batches of 8 passes on the graph path (Engine.swift:771-792).  The persistent kernel
        // runs to the stop on the device (EOS, ')', the step limit); a pass commits at least one
        // token, so the remaining tokens bound its passes.
        const int left = s.maxsteps - s.step;
        const int count = e->use_persistent() ? left : std::min(8, left);
        const int step0 = s.step, pos0 = s.pos;
        double ms = 0;
        if (e->decode_steps(count, &ms)) return -1;
        dec_ms += ms;
        if (e->read_state(s)) return -1;
        if (!s.done && s.step == step0 && s.pos == pos0) return fail("decode made no progress");
    }
    std::vector<int32_t> toks(std::max(s.step, 1));
    HIPCK(hipMemcpy(toks.data(), e->out_tokens, sizeof(int32_t) * s.step, hipMemcpyDeviceToHost));
    int cnt = 0;
    for (int i = 0; i < s.step; ++i) {
        if (toks[i] == e->eos0 || toks[i] == e->eos1) break;
        out_tokens[cnt++] = toks[i];
    }
    *n_out = cnt;
    const auto t1 = std::chrono::steady_clock::now();
    e->timing.decode_ms = dec_ms;
    e->timing.total_ms = std::chrono::duration<double, std::milli>(t1 - t0).count();
    e->timing.generated_tokens = cnt;
    e->timing.vision_ms = 0;
    return 0;
}

int icua_vision(icua_engine* e, const uint8_t* rgb, int width, int height) {
    if (!e || !rgb) return fail("null argument");
    double ms = 0;
    if (e->vision(rgb, width, height, &ms)) return -1;
    e->timing.vision_ms = ms;
    e->has_cached_vision = false;
    return 0;
}

// hashRGB (Engine.swift:684-693): FNV-1a over the frame's whole 8-byte words.
static uint64_t hash_rgb(const uint8_t* p, size_t bytes) {
    uint64_t h = 0xcbf29ce484222325ull;
    for (size_t i = 0; i < bytes / 8; ++i) {
        uint64_t w;
        std::memcpy(&w, p + 8 * i, 8);
        h ^= w;
        h *= 0x100000001b3ull;
    }
    return h;
}

int icua_generate_vision(icua_engine* e, const uint8_t* rgb, int width, int height, const int32_t* tokens, int n,
                         int max_new, int32_t* out_tokens, int* n_out) {
    if (!e || !rgb || !tokens || !out_tokens || !n_out) return fail("null argument");
    const auto t0 = std::chrono::steady_clock::now();
    if (width <= 0 || height <= 0 || width % 32 || height % 32)
        return fail("image sides must be positive multiples of 32");
    // Vision delta cache (Engine.swift:707-716): an identical consecutive frame reuses the last
    // encoder outputs.  The frame size is part of the key here.
    const uint64_t hsh = hash_rgb(rgb, (size_t)width * height * 3);
    const bool skip = (e->flags & ICUA_FLAG_VISION_DELTA_CACHE) && e->has_cached_vision && hsh == e->rgb_hash &&
                      e->rgb_dims[0] == width && e->rgb_dims[1] == height;
    double vms = 0;
    if (!skip) {
        e->has_cached_vision = false;
        if (e->vision(rgb, width, height, &vms)) return -1;
        e->rgb_hash = hsh;
        e->rgb_dims[0] = width;
        e->rgb_dims[1] = height;
        e->has_cached_vision = true;
    }
    int vis_offset = -1;  // first <|image_pad|> (Engine.swift:718)
    for (int i = 0; i < n; ++i)
        if (tokens[i] == IMAGE_PAD_ID) {
            vis_offset = i;
            break;
        }
    if (e->prepare_mrope(vis_offset, height / 32, width / 32)) return -1;
    if (icua_generate(e, tokens, n, vis_offset, max_new, out_tokens, n_out)) return -1;
    e->timing.vision_ms = vms;
    e->timing.total_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
    return 0;
}

int icua_verify(icua_engine* e, const int32_t* draft, int m, int32_t* out_argmax, float* out_logits) {
    if (!e || !draft || !out_argmax) return fail("null argument");
    if (m < 1 || m > MAXM) return fail("verify takes 1..8 draft tokens");
    State s;
    if (e->read_state(s)) return -1;
    if (s.pos + m > e->maxctx) return fail("verify exceeds max context");
    for (int i = 0; i < m; ++i)
        if (draft[i] < 0 || draft[i] >= VOCAB) return fail("token id out of range");
    HIPCK(hipMemcpyAsync(e->prompt, draft, sizeof(int32_t) * m, hipMemcpyHostToDevice, e->stream));
    State v = s;
    v.n = m;
    v.done = 0;
    v.vis_offset = -1;
    v.logits_rows = m;
    if (e->write_state(v)) return -1;
    EmbedArgs ea{};
    ea.toks = e->prompt;
    ea.E = e->E;
    ea.Esb = e->Esb;
    ea.fmt = e->fmt;
    ea.row0 = 0;
    ea.x = e->x;
    ea.st = e->st;
    ea.n = m;
    HIPCK(launch_embed(ea, e->stream));
    for (int l = 0; l < e->layers; ++l)
        if (e->enqueue_layer(l, MAXM, 0)) return -1;
    if (e->enqueue_head(MAXM, 1)) return -1;
    HIPCK(hipStreamSynchronize(e->stream));
    HIPCK(hipMemcpy(out_argmax, e->argmax_rows, sizeof(int32_t) * m, hipMemcpyDeviceToHost));
    if (out_logits)
        HIPCK(hipMemcpy(out_logits, e->logits, sizeof(float) * (size_t)m * VOCAB, hipMemcpyDeviceToHost));
    e->last_logits_rows = m;
    return e->write_state(s);
}

int icua_set_position(icua_engine* e, int pos, int32_t next_token, int step, int max_steps) {
    if (!e) return fail("null engine");
    if (pos < 0 || pos >= e->maxctx) return fail("position out of range");
    if (next_token < 0 || next_token >= VOCAB) return fail("token out of range");
    if (step < 0 || step >= std::max(1, std::min(max_steps, e->maxsteps))) return fail("step out of range");
    e->kv_written_from(pos);  // the next step writes K/V at slot pos
    State s;
    if (e->read_state(s)) return -1;
    s.pos = pos;
    s.n = 1;
    s.done = 0;
    s.step = step;
    s.maxsteps = std::max(1, std::min(max_steps, e->maxsteps));
    s.vis_offset = -1;
    s.logits_rows = 0;
    s.flags = (e->flags & ICUA_FLAG_GRAMMAR_PAIRS) ? STATE_FLAG_GRAMMAR : 0;
    if (e->write_state(s)) return -1;
    HIPCK(hipMemcpy(e->prompt, &next_token, sizeof(int32_t), hipMemcpyHostToDevice));
    EmbedArgs ea{};
    ea.toks = e->prompt;
    ea.E = e->E;
    ea.Esb = e->Esb;
    ea.fmt = e->fmt;
    ea.row0 = 0;
    ea.x = e->x;
    ea.st = e->st;
    ea.n = 1;
    HIPCK(launch_embed(ea, e->stream));
    HIPCK(hipStreamSynchronize(e->stream));
    return 0;
}

int icua_read_state(icua_engine* e, icua_state_t* out) {
    if (!e || !out) return fail("null argument");
    State s;
    if (e->read_state(s)) return -1;
    static_assert(sizeof(icua_state_t) <= sizeof(State), "state layout");
    std::memcpy(out, &s, sizeof(icua_state_t));
    return 0;
}

int icua_read_tokens(icua_engine* e, int32_t* dst, int n) {
    if (!e || !dst) return fail("null argument");
    if (n < 0 || n > e->maxsteps + 4) return fail("token count out of range");
    HIPCK(hipMemcpy(dst, e->out_tokens, sizeof(int32_t) * n, hipMemcpyDeviceToHost));
    return 0;
}

int icua_logits(icua_engine* e, float* dst, int rows) {
    if (!e || !dst) return fail("null argument");
    if (rows < 1 || rows > MAXM) return fail("rows out of range");
    HIPCK(hipMemcpy(dst, e->logits, sizeof(float) * (size_t)rows * VOCAB, hipMemcpyDeviceToHost));
    return 0;
}

int icua_timing(icua_engine* e, icua_timing_t* out) {
    if (!e || !out) return fail("null argument");
    *out = e->timing;
    return 0;
}

int icua_layer_step(icua_engine* e, int layer, const float* x_in, int n, int pos, float* x_out) {
    if (!e || !x_in || !x_out) return fail("null argument");
    if (layer < 0 || layer >= e->layers) return fail("layer out of range");
    if (n < 1 || n > MAXM) return fail("layer_step takes 1..8 rows");
    if (pos < 0 || pos + n > e->maxctx) return fail("slots out of range");
    State s;
    if (e->read_state(s)) return -1;
    State v = s;
    v.pos = pos;
    v.n = n;
    v.done = 0;
    v.vis_offset = -1;
    if (e->write_state(v)) return -1;
    HIPCK(hipMemcpy(e->x, x_in, sizeof(float) * (size_t)n * H, hipMemcpyHostToDevice));
    if (e->enqueue_layer(layer, n == 1 ? 1 : MAXM, 0)) return -1;
    HIPCK(hipStreamSynchronize(e->stream));
    HIPCK(hipMemcpy(x_out, e->x, sizeof(float) * (size_t)n * H, hipMemcpyDeviceToHost));
    return e->write_state(s);
}

static int kv_copy(icua_engine* e, int layer, int kind, int slot0, int nslots, void* host, bool to_dev) {
    if (!e || !host) return fail("null argument");
    if (layer < 0 || layer >= e->layers || kind < 0 || kind > 1) return fail("bad layer/kind");
    if (slot0 < 0 || nslots < 0 || slot0 + nslots > e->maxctx) return fail("slots out of range");
    if (to_dev && nslots > 0) e->kv_written_from(slot0);
    for (int g = 0; g < NKV; ++g) {
        uint16_t* dev = e->kv_ptr(layer, kind) + ((size_t)g * e->maxctx + slot0) * HD;
        uint16_t* hp = (uint16_t*)host + (size_t)g * nslots * HD;
        const size_t bytes = (size_t)nslots * HD * 2;
        if (to_dev)
            HIPCK(hipMemcpy(dev, hp, bytes, hipMemcpyHostToDevice));
        else
            HIPCK(hipMemcpy(hp, dev, bytes, hipMemcpyDeviceToHost));
    }
    return 0;
}

int icua_read_kv(icua_engine* e, int layer, int kind, int slot0, int nslots, uint16_t* dst) {
    return kv_copy(e, layer, kind, slot0, nslots, dst, false);
}

int icua_write_kv(icua_engine* e, int layer, int kind, int slot0, int nslots, const uint16_t* src) {
    return kv_copy(e, layer, kind, slot0, nslots, (void*)src, true);
}

int icua_read_buffer(icua_engine* e, int which, void* dst, size_t bytes) {
    if (!e || !dst) return fail("null argument");
    const void* src = nullptr;
    size_t cap = 0;
    switch (which) {
        case ICUA_BUF_X: src = e->x; cap = sizeof(float) * MAXM * H; break;
        case ICUA_BUF_QKV: src = e->qkv; cap = sizeof(float) * MAXM * QKV; break;
        case ICUA_BUF_ATTN: src = e->attn; cap = sizeof(float) * MAXM * H; break;
        case ICUA_BUF_MLP: src = e->h; cap = sizeof(float) * MAXM * FF; break;
        case ICUA_BUF_POOLER: src = e->pooler; cap = sizeof(float) * (size_t)e->n_vis * H; break;
        case ICUA_BUF_DEEPSTACK0:
        case ICUA_BUF_DEEPSTACK0 + 1:
        case ICUA_BUF_DEEPSTACK0 + 2:
            src = e->has_ds ? e->ds[which - ICUA_BUF_DEEPSTACK0] : nullptr;
            cap = sizeof(float) * (size_t)e->n_vis * H;
            break;
        default: return fail("unknown buffer");
    }
    if (!src) return fail("buffer not set");
    if (bytes > cap) return fail("read past the buffer");
    HIPCK(hipStreamSynchronize(e->stream));
    HIPCK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return 0;
}

int icua_dev_alloc(size_t bytes, void** ptr) {
    if (!ptr) return fail("null argument");
    HIPCK(hipMalloc(ptr, bytes));
    return 0;
}
int icua_dev_free(void* ptr) {
    HIPCK(hipFree(ptr));
    return 0;
}
int icua_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    HIPCK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
    return 0;
}
int icua_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    HIPCK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
    return 0;
}
int icua_device_sync(void) {
    HIPCK(hipDeviceSynchronize());
    return 0;
}

static int gemv_setup(int fmt, int N, int K, int m, GemvArgs& a, GemvOp& op) {
    if (fmt < 0 || fmt > 2) return fail("bad format");
    if (K != H && K != FF) return fail("K must be 2048 or 6144");
    if (N <= 0 || N % 16) return fail("N must be a positive multiple of 16");
    if (m < 1 || m > MAXM) return fail("m must be 1..8");
    State* st;
    if (null_state(&st, m)) return -1;
    a = GemvArgs{};
    a.st = st;
    a.m_fixed = m;
    a.N = N;
    op = (K == H) ? GEMV_PLAIN : GEMV_PLAIN_K6144;
    a.blocks = std::max(1, std::min(N / 16, 1024));  // four workgroups per CU, row blocks strided
    return 0;
}

int icua_repack(int fmt, const void* d_codes, const void* d_sb, int N, int K, void* d_tiled_codes, void* d_tiled_sb) {
    if (fmt < 0 || fmt > 2) return fail("bad format");
    if (K != H && K != FF) return fail("K must be 2048 or 6144");
    if (N <= 0 || N % 16) return fail("N must be a positive multiple of 16");
    HIPCK(launch_repack(fmt, (const uint8_t*)d_codes, (const uint8_t*)d_sb, (uint8_t*)d_tiled_codes,
                        (uint8_t*)d_tiled_sb, N, K, 0, nullptr));
    HIPCK(hipDeviceSynchronize());
    return 0;
}

// One-token q4 / q8 GEMVs take the streaming kernel (the lm_head stage's schedule), multi-token
// ones its 8-row form (gemv8.hip); f16 the general kernel.
static bool use_stream(int fmt, int N, int m) {
    return m == 1 && (fmt == FMT_Q4 || fmt == FMT_Q8) && N / 16 <= 160 * 256;
}

int icua_gemv(int fmt, const void* d_codes, const void* d_sb, int N, int K, const float* d_x, int m, float* d_y) {
    GemvArgs a;
    GemvOp op;
    if (gemv_setup(fmt, N, K, m, a, op)) return -1;
    if (use_stream(fmt, N, m)) {
        HIPCK(launch_gemv_stream(fmt, (const uint8_t*)d_codes, (const uint8_t*)d_sb, d_x, d_y, N, K, nullptr));
    } else if (m > 1 && gemv8_supports(fmt, op, N)) {
        a.w = (const uint8_t*)d_codes;
        a.sb = (const uint8_t*)d_sb;
        a.x = d_x;
        a.y = d_y;
        HIPCK(launch_gemv8(fmt, op, a, nullptr));
    } else {
        a.w = (const uint8_t*)d_codes;
        a.sb = (const uint8_t*)d_sb;
        a.x = d_x;
        a.y = d_y;
        HIPCK(launch_gemv(fmt, op, a, m == 1 ? 1 : MAXM, nullptr));
    }
    HIPCK(hipDeviceSynchronize());
    return 0;
}

int icua_gemv_bench(int fmt, const void* const* d_codes, const void* const* d_sb, int ncopies, int N, int K,
                    const float* d_x, float* d_y, int iters, double* avg_us) {
    if (!d_codes || !d_sb || ncopies < 1 || iters < 1 || !avg_us) return fail("bad arguments");
    GemvArgs a;
    GemvOp op;
    if (gemv_setup(fmt, N, K, 1, a, op)) return -1;
    a.x = d_x;
    a.y = d_y;
    hipEvent_t e0, e1;
    HIPCK(hipEventCreate(&e0));
    HIPCK(hipEventCreate(&e1));
    const bool stream = use_stream(fmt, N, 1);
    auto launch = [&](int i) {
        a.w = (const uint8_t*)d_codes[i % ncopies];
        a.sb = (const uint8_t*)d_sb[i % ncopies];
        return stream ? launch_gemv_stream(fmt, a.w, a.sb, d_x, d_y, N, K, nullptr) : launch_gemv(fmt, op, a, 1, nullptr);
    };
    HIPCK(launch(0));  // warm-up
    HIPCK(hipEventRecord(e0, nullptr));
    for (int i = 0; i < iters; ++i) HIPCK(launch(i));
    HIPCK(hipEventRecord(e1, nullptr));
    HIPCK(hipEventSynchronize(e1));
    float ms = 0;
    HIPCK(hipEventElapsedTime(&ms, e0, e1));
    *avg_us = (double)ms * 1000.0 / iters;
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return 0;
}

static int quant_check(int fmt, const float* d_m, int rows, int cols, const void* d_codes, const void* d_sb) {
    if (fmt != FMT_Q4 && fmt != FMT_Q8) return fail("quantize: format must be q8 (1) or q4 (2)");
    const int gsz = fmt == FMT_Q4 ? 64 : 32;
    if (rows <= 0 || cols <= 0 || cols % gsz) return fail("quantize: cols must be a positive multiple of " +
                                                         std::to_string(gsz));
    if ((int64_t)rows * cols > ((int64_t)1 << 40)) return fail("quantize: matrix too large");
    if (!d_m || !d_codes || !d_sb) return fail("quantize: null buffer");
    return 0;
}

int icua_quantize(int fmt, const float* d_m, int rows, int cols, void* d_codes, void* d_sb) {
    if (quant_check(fmt, d_m, rows, cols, d_codes, d_sb)) return -1;
    uint8_t* none = nullptr;
    if (fmt == FMT_Q4) HIPCK(hipMalloc(&none, (size_t)rows * (cols / 64)));
    const hipError_t e = launch_quant(fmt, d_m, rows, cols, d_codes, d_sb, none, nullptr);
    const hipError_t e2 = hipDeviceSynchronize();
    if (none) (void)hipFree(none);
    HIPCK(e);
    HIPCK(e2);
    return 0;
}

int icua_quantize_noalloc(int fmt, const float* d_m, int rows, int cols, void* d_codes, void* d_sb) {
    if (quant_check(fmt, d_m, rows, cols, d_codes, d_sb)) return -1;
    uint8_t* none = nullptr;
    if (fmt == FMT_Q4) {
        const int64_t groups = (int64_t)rows * (cols / 64);
        if (groups > QUANT_SCRATCH_GROUPS)
            return fail("quantize_noalloc: " + std::to_string(groups) + " q4 groups exceed the static scratch of " +
                        std::to_string(QUANT_SCRATCH_GROUPS) + " groups (use icua_quantize)");
        HIPCK(quant_scratch(&none));
    }
    HIPCK(launch_quant(fmt, d_m, rows, cols, d_codes, d_sb, none, nullptr));
    HIPCK(hipDeviceSynchronize());
    return 0;
}

int icua_quantize_bench(int fmt, const float* d_m, int rows, int cols, void* d_codes, void* d_sb, int iters,
                        double* avg_us) {
    if (quant_check(fmt, d_m, rows, cols, d_codes, d_sb)) return -1;
    if (iters < 1 || !avg_us) return fail("bad arguments");
    uint8_t* none = nullptr;
    if (fmt == FMT_Q4) HIPCK(hipMalloc(&none, (size_t)rows * (cols / 64)));
    hipEvent_t e0 = nullptr, e1 = nullptr;
    hipError_t e = hipEventCreate(&e0);
    if (e == hipSuccess) e = hipEventCreate(&e1);
    if (e == hipSuccess) e = launch_quant(fmt, d_m, rows, cols, d_codes, d_sb, none, nullptr);  // warm-up
    if (e == hipSuccess) e = hipEventRecord(e0, nullptr);
    for (int i = 0; i < iters && e == hipSuccess; ++i) e = launch_quant(fmt, d_m, rows, cols, d_codes, d_sb, none, nullptr);
    if (e == hipSuccess) e = hipEventRecord(e1, nullptr);
    if (e == hipSuccess) e = hipEventSynchronize(e1);
    float ms = 0;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, e0, e1);
    if (e0) (void)hipEventDestroy(e0);
    if (e1) (void)hipEventDestroy(e1);
    (void)hipDeviceSynchronize();
    if (none) (void)hipFree(none);
    HIPCK(e);
    *avg_us = (double)ms * 1000.0 / iters;
    return 0;
}

int icua_dequant(int fmt, const void* d_codes, const void* d_sb, int K, int row0, int rows, float* d_out, int tiled) {
    if (fmt < 0 || fmt > 2) return fail("bad format");
    if (K <= 0 || K % 64 || rows < 0 || row0 < 0) return fail("bad shape");
    if (tiled && (K % 2048 || (row0 + rows) % 16 != 0)) return fail("tiled dequant takes whole 16-row blocks of K % 2048 == 0");
    HIPCK(launch_dequant(fmt, (const uint8_t*)d_codes, (const uint8_t*)d_sb, K, row0, rows, d_out, tiled, nullptr));
    HIPCK(hipDeviceSynchronize());
    return 0;
}

}  // extern "C"
