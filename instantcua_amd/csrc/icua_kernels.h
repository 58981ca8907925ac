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
    GEMV_PLAIN_F16IN = 5,        // K = 2048, fp16 x -> fp32 y
    GEMV_PLAIN_F16IN_K6144 = 6,  // K = 6144, fp16 x -> fp32 y
};

struct GemvArgs {
    const uint8_t* w;       // codes [N][row bytes]
    const uint8_t* sb;      // q4: half2 (scale, bias) [N][K/64]; q8: half [N][K/32]
    int N;                  // output rows
    const void* x;          // PRO_NORM/PRO_F32: fp32 [M][K]; PRO_F16: fp16 [M][K]
    const float* norm_w;    // PRO_NORM weights [K]
    float* y;               // EPI_STORE: y [M][N]; EPI_RESID: residual x [M][N] (+=)
    uint16_t* h;            // EPI_SWIGLU: fp16 [M][FF]
    const float* ds;        // EPI_RESID: DeepStack rows [n_vis][H] or null
    int ds_row0;            // prompt row of pass row 0 (DeepStack visual-row lookup)
    float* pval;            // EPI_ARGMAX partials [MAXM][LMH_WAVES]
    int* pidx;
    float* logits;          // EPI_ARGMAX optional logits [MAXM][VOCAB]
    const State* st;
    int m_fixed;            // > 0: rows of the pass given by the host, else st->n
    int blocks;             // isolated GEMV launches: grid size
};

hipError_t launch_gemv(int fmt, GemvOp op, const GemvArgs& a, int mt, hipStream_t s);

struct AttnArgs {
    const float* qkv;       // raw fused QKV rows [M][QKV] fp32
    const float* q_norm;    // [HD]
    const float* k_norm;    // [HD]
    const float* rope;      // [maxctx][64] (cos, sin)
    uint16_t* kc;           // this layer's K cache [NKV][maxctx][HD] fp16
    uint16_t* vc;           // this layer's V cache
    float* part;            // split partials [NKV][ATTN_SPLITS][MAXM][2][HD + 2]
    int* counters;          // [NKV] arrival counters, zero between launches
    uint16_t* out;          // attention output fp16 [M][H]
    const State* st;
    int m_fixed;
};
hipError_t launch_attention(const AttnArgs& a, int mt, hipStream_t s);

struct CommitArgs {
    const float* pval;
    const int* pidx;
    State* st;
    int* out_tokens;
    const uint8_t* E;       // embedding codes
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

// Bit-exact dequantisation of rows [row0, row0 + rows) to fp32 (w = s*q + b / s*q / half).
hipError_t launch_dequant(int fmt, const uint8_t* w, const uint8_t* sb, int K, int row0, int rows, float* out,
                          hipStream_t s);

}  // namespace icua
