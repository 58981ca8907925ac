// Kernel launch interface used by the host engine.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "icua_shared.h"

namespace icua {

enum Prologue { PRO_NORM = 0, PRO_F32 = 1, PRO_F16 = 2 };
enum Epilogue { EPI_STORE = 0, EPI_RESID = 1, EPI_SWIGLU = 2, EPI_ARGMAX = 3 };
enum GemvOp {
    GEMV_QKV = 0,
    GEMV_O = 1,
    GEMV_GU = 2,
    GEMV_DOWN = 3,
    GEMV_LMHEAD = 4,
    GEMV_PLAIN = 5,        // K = 2048, fp32 x -> fp32 y
    GEMV_PLAIN_K6144 = 6,  // K = 6144, fp32 x -> fp32 y
};

struct GemvArgs {
    const uint8_t* w;       // codes in 16-row MFMA tiles (launch_repack)
    const uint8_t* sb;      // q4: half2 (scale, bias) [N][K/64]; q8: half [N][K/32] (tiled row order)
    int N;                  // output rows
    const float* x;         // fp32 activations [M][K] (MAXM rows when m_fixed == 0)
    const float* norm_w;    // PRO_NORM weights [K]
    float* y;               // EPI_STORE: y [M][N]; EPI_RESID: residual x [M][N] (+=)
    float* h;               // EPI_SWIGLU: [M][FF]
    const float* ds;        // EPI_RESID: DeepStack rows [n_vis][H] or null
    int ds_row0;            // prompt row of pass row 0 (DeepStack visual-row lookup)
    float* pval;            // EPI_ARGMAX partials [MAXM][LMH_WAVES]
    int* pidx;
    float* logits;          // EPI_ARGMAX optional logits [MAXM][VOCAB]
    const State* st;
    int m_fixed;            // > 0: rows of the pass given by the host, else st->n
    int blocks;             // isolated GEMV launches: grid size
    float* kpart;           // K = 6144 residual GEMV: per-segment partials [3][MAXM][N]
    int* kcnt;              // and per-row-block arrival counters [N / 16], zero between launches
    uint8_t* apre;          // multi-row passes: operands pre-staged by launch_gemv_prep (or null)
    float* fxpre;           // and their group factors
};

hipError_t launch_gemv(int fmt, GemvOp op, const GemvArgs& a, int mt, hipStream_t s);
// Multi-token (MAXM-row) q4 / q8 GEMVs on the streaming schedule (gemv8.hip): the pass's rows
// staged once per workgroup; every op of launch_gemv, K = 6144 for up to 1024 row blocks.
bool gemv8_supports(int fmt, GemvOp op, int N);
hipError_t launch_gemv8(int fmt, GemvOp op, const GemvArgs& a, hipStream_t s);
// Stages the activation operands of a multi-row (MAXM) GEMV of the same arguments into a.apre /
// a.fxpre (GEMV_PREP_BYTES / GEMV_PREP_FX_BYTES), for the GEMV launched next on the stream.
hipError_t launch_gemv_prep(int fmt, GemvOp op, const GemvArgs& a, hipStream_t s);
constexpr size_t GEMV_PREP_BYTES = 3 * 2 * 65536, GEMV_PREP_FX_BYTES = 3 * 2 * 1024 * 4;

// Repacks a row-major .icua matrix (codes + scales) into the GEMV tile layout.  gu_interleave
// reorders the fused gate|up rows so that tiled block b holds gate units 8b..8b+7 and then the
// matching up rows.  N % 16 == 0, K % 2048 == 0.
hipError_t launch_repack(int fmt, const uint8_t* codes, const uint8_t* sb, uint8_t* dcodes, uint8_t* dsb, int N, int K,
                         int gu_interleave, hipStream_t s);

struct AttnArgs {
    const float* qkv;       // raw fused QKV rows [M][QKV] fp32
    const float* q_norm;    // [HD]
    const float* k_norm;    // [HD]
    const float* rope;      // [maxctx][64] (cos, sin)
    uint16_t* kc;           // this layer's K cache [NKV][maxctx][HD] fp16
    uint16_t* vc;           // this layer's V cache
    float* part;            // split partials [NKV][splits][MAXM][2][HD + 2]
    float* out;             // attention output fp32 [M][H]
    const State* st;
    int m_fixed;
};
// Grid width for a cache of maxctx slots (64-slot splits + the tail split).
int attention_splits(int maxctx);
hipError_t launch_attention(const AttnArgs& a, int mt, int splits, hipStream_t s);

struct CommitArgs {
    const float* pval;
    const int* pidx;
    State* st;
    int* out_tokens;
    const uint8_t* E;       // embedding codes (tiled layout)
    const uint8_t* Esb;
    int fmt;
    float* x;               // residual rows to receive the next token embedding(s)
    int* argmax_rows;       // [MAXM] per-row argmax of the pass (verify), may be null
    int verify_only;        // 1: write argmax_rows and leave the state untouched
};
hipError_t launch_commit(const CommitArgs& a, hipStream_t s);

struct EmbedArgs {
    const int* toks;        // prompt tokens of the pass [n]
    const uint8_t* E;
    const uint8_t* Esb;
    int fmt;
    const float* pooler;    // visual embeddings [n_vis][H] fp32 or null
    int row0;               // prompt row of pass row 0
    float* x;               // [n][H]
    const State* st;
    int n;
};
hipError_t launch_embed(const EmbedArgs& a, hipStream_t s);

// Sets pos / n / logits_rows of the control block on the stream.
hipError_t launch_set_pass(State* st, int pos, int n, int logits_rows, hipStream_t s);

// ---- Matrix-core prefill (prefill.hip), q4 weights, passes of M <= Mpad tokens (Mpad % 128 == 0).
// Activation operands of one GEMM input: fp16 hi / lo parts of the row-scaled activations
// [Mpad / 16][K / 32][parts][64][8] (parts 2: hi and lo; 1: hi alone), group sums
// [Mpad / 16][K / 64][16] and row scales [Mpad].
hipError_t launch_pf_prep(int K, int norm, const float* src, const float* norm_w, int M, int Mpad, uint16_t* xa,
                          float* xs, float* ts, int parts, hipStream_t s);

struct PfGemmArgs {
    const uint16_t* xa;     // activation operands (launch_pf_prep)
    const float* xs;        // group sums
    const float* ts;        // row scales
    const uint8_t* w;       // codes in 16-row MFMA tiles (launch_repack)
    const uint8_t* sb;      // q4 half2 (scale, bias) [N][K / 64]; q8 half scales [N][K / 32]
    int N, M, Mpad;
    float* y;               // EPI_STORE: y [M][N]; EPI_RESID: residual x [M][N] (+=)
    float* h;               // EPI_SWIGLU: [M][FF]
    const float* ds;        // EPI_RESID: DeepStack rows [n_vis][H] or null
    int row0;               // prompt row of pass row 0
    int vis_offset, n_vis;
    int parts;              // operand parts of xa (1 or 2, as launch_pf_prep wrote them)
};
// fmt: FMT_Q4 / FMT_Q8 / FMT_F16 (sb unused for f16); epi: EPI_STORE / EPI_RESID / EPI_SWIGLU;
// K = 2048 (any epilogue) or 6144 (EPI_RESID).
hipError_t launch_pf_gemm(int fmt, int K, int epi, const PfGemmArgs& a, hipStream_t s);

struct PfQkArgs {
    const float* qkv;       // raw fused QKV rows [M][QKV]
    const float* q_norm;
    const float* k_norm;
    const float* rope;      // [maxctx][64] (cos, sin)
    uint16_t* kc;           // this layer's K / V cache [NKV][maxctx][HD] fp16
    uint16_t* vc;
    uint16_t* qh;           // queries, pre-scaled, fp16 hi / lo parts [Mpad][NH][HD]
    uint16_t* ql;
    int M, p0, maxctx;      // rows of the pass at cache slots p0 .. p0 + M - 1
};
hipError_t launch_pf_qk(const PfQkArgs& a, hipStream_t s);

struct PfAttnArgs {
    const uint16_t* qh;
    const uint16_t* ql;     // null: queries and probabilities as fp16 hi parts alone
    const uint16_t* kc;
    const uint16_t* vc;
    float* out;             // attention rows [M][H] fp32
    int M, p0, maxctx;
};
hipError_t launch_pf_attn(const PfAttnArgs& a, hipStream_t s);

// Bit-exact dequantisation of rows [row0, row0 + rows) to fp32 (w = s*q + b / s*q / half),
// from the row-major .icua layout (tiled = 0) or the GEMV tile layout (tiled = 1).
hipError_t launch_dequant(int fmt, const uint8_t* w, const uint8_t* sb, int K, int row0, int rows, float* out,
                          int tiled, hipStream_t s);

// Converter quantisers (Convert.swift:214-320) of a row-major fp32 matrix [rows][cols]: q8 codes
// + fp16 scales, or q4 packed codes + fp16 (scale, bias); `none` is a scratch byte per q4 group.
hipError_t launch_quant(int fmt, const float* m, int64_t rows, int64_t cols, void* codes, void* sb, uint8_t* none,
                        hipStream_t s);
// Device address, on the current device, of the quantiser's static scratch: one `none` byte per
// q4 group for up to QUANT_SCRATCH_GROUPS groups.  Looked up once per device.
constexpr int64_t QUANT_SCRATCH_GROUPS = (int64_t)8 << 20;
constexpr int QUANT_MAX_DEVICES = 64;
hipError_t quant_scratch(uint8_t** out);

// Vision tower (ModelFile.swift:31-45): dimensions, weights, work buffers.
constexpr int VH = 1024, VFF = 4096, VNH = 16, VHD = 64, VQKV = 3072, VPATCH = 768, MH = 4096;
constexpr int VLAYERS = 24, VPOS = 48, NPATCH_MAX = 1024;
enum { VG_F32 = 0, VG_F32_ADD = 1, VG_F32_POS = 2, VG_GELU_TANH = 3, VG_GELU_ERF = 4, VG_QKV = 5 };
struct VitGemmArgs {
    const uint16_t* X;  // fp16 [M][K]
    const uint16_t* W;  // fp16 [N][K]
    const float* bias;  // [N]
    float* outf;        // [M][N] float32 (VG_F32, VG_F32_ADD, VG_F32_POS)
    uint16_t* outh;     // [M][N] fp16 (GELU modes)
    const float* pos;   // [M][N] (VG_F32_POS)
    const float* rope;  // [M][32][2] (VG_QKV)
    uint16_t* q;        // [VNH][ld][VHD] fp16 (VG_QKV)
    uint16_t* k;        // [VNH][ld][VHD]
    uint16_t* vt;       // [VNH][VHD][ld], V transposed
    int ld, M, N, K;
};
struct VitBlock {
    const float *n1w, *n1b, *qkvb, *projb, *n2w, *n2b, *fc1b, *fc2b;
    const uint16_t *qkvw, *projw, *fc1w, *fc2w;
};
struct VitMerger {
    const float *nw, *nb, *fc1b, *fc2b;
    const uint16_t *fc1w, *fc2w;
};
struct VitWeights {
    const uint16_t* patch_w;
    const float* patch_b;
    VitBlock blk[VLAYERS];
    VitMerger mg[4];  // DeepStack mergers 0-2, final merger 3
};
struct VitBuffers {
    const uint8_t* rgb;  // [16 gh][16 gw][3]
    uint16_t* patches;   // [NPATCH_MAX][VPATCH]
    float* x;            // residual [NPATCH_MAX][VH]
    uint16_t* xn;        // LayerNorm out [NPATCH_MAX][VH] (= [NPATCH_MAX / 4][MH])
    uint16_t *q, *k, *vt;
    uint16_t* attn;      // [NPATCH_MAX][VH]
    uint16_t* h;         // [NPATCH_MAX][VFF]
    const float* pos;    // interpolated position table [np][VH]
    const float* rope;   // [np][32][2]
    float* pooler;       // [np / 4][H]
    float* ds[3];        // [np / 4][H]
};
// The whole tower for a gh x gw patch grid (even sides, at most NPATCH_MAX patches).
hipError_t launch_vision(const VitWeights& w, const VitBuffers& b, int gh, int gw, hipStream_t s);

}  // namespace icua
