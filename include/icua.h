/* icua.h -- C ABI of the MI355X (gfx950) Qwen3-VL text-decoder engine.
 *
 * Drop-in boundary for instantcua's `Engine` (Sources/Engine/Engine.swift:5-827).  The Swift
 * class keeps its API and forwards to these functions, in the style of the reference's C target
 * Sources/CShim (Package.swift:14; Sources/CShim/include/cshim.h:1-4).  Plain pointers and
 * sizes only.  Every function returns 0 on success and a negative code on failure; the message
 * is available from icua_last_error() (thread-local), which the Swift wrapper maps to
 * `EngineError` (Sources/Engine/ModelFile.swift:158-161).
 *
 * Threading and ownership follow the reference: one engine is bound to one HIP stream and is
 * not thread-safe; calls are synchronous (they return after the GPU work completes, as
 * `waitUntilCompleted` does in Engine.swift:786-791); the engine owns all device memory; input
 * arrays are borrowed and copied in.
 */
#ifndef ICUA_H
#define ICUA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct icua_engine icua_engine;

/* Weight formats of the .icua file (ModelFile.swift:6-9). */
enum { ICUA_FMT_F16 = 0, ICUA_FMT_Q8 = 1, ICUA_FMT_Q4 = 2 };

/* Engine flags (icua_engine_create / icua_set_flags). */
enum {
    ICUA_FLAG_GRAMMAR_PAIRS = 1, /* forced syntax pairs + ')' stop of k_commit (Shaders.swift:1543-1560) */
    ICUA_FLAG_PREFIX_CACHE = 2,  /* reuse the KV of an identical pre-image prefix (Engine.swift:719-735) */
    ICUA_FLAG_GRAPH_DECODE = 4,  /* decode through the per-kernel HIP graph instead of the persistent kernel */
    ICUA_FLAG_PASS_PREFILL = 8,  /* prefill q4 prompts in passes of 8 rows instead of the matrix-core GEMMs */
    ICUA_FLAG_VISION_DELTA_CACHE = 16, /* icua_generate_vision skips the encoder on an identical frame (Engine.swift:707-716) */
    ICUA_FLAG_FIRST_LOGITS = 32, /* icua_generate(_vision) keep the first token's logits for icua_logits (writeFirstLogits, Engine.swift:697) */
    ICUA_FLAG_PREFILL_FP16 = 64, /* matrix-core prefill on fp16 operands alone: activations, queries and probabilities in fp16, weights dequantised to fp16 (the reference engine's precision, Shaders.swift:976-992), instead of fp16 hi + lo activations against exact codes */
};

/* Decode control block, first twelve fields as `State` (Shaders.swift:41-54). */
typedef struct {
    int32_t pos, n, step, done, maxctx, maxsteps, eos0, eos1, vis_offset, n_vis, rope_delta, npatches;
    int32_t flags, logits_rows;
} icua_state_t;

/* Engine.Timing (Engine.swift:44-52). */
typedef struct {
    double vision_ms, prefill_ms, decode_ms, total_ms;
    int64_t prefill_tokens, generated_tokens;
} icua_timing_t;

typedef struct {
    int32_t format, layers, max_context, max_pass, max_steps;
    int64_t weight_bytes, kv_bytes;
    int32_t persistent_decode; /* 1 if icua_decode_steps can use the persistent kernel on this device */
    int32_t vision; /* 1 if the model file holds the vision tower and its mergers */
    int32_t last_decode_persistent; /* 1 if the last icua_decode_steps call ran as the persistent kernel */
    int32_t visual_rows; /* rows of the pooler / DeepStack buffers (ICUA_BUF_POOLER, ...), 0 if unset */
    int32_t pair_passes; /* forced grammar pairs run as one two-row persistent launch, since create */
} icua_info_t;

/* Last error message of the calling thread ("" if none). */
const char* icua_last_error(void);

/* Engine.init(modelPath:maxContext:maxPass:maxSteps:copyWeights:pinMemory:) (Engine.swift:54-185).
 * Loads the .icua file (ModelFile.init, ModelFile.swift:124-149) and copies the decoder tensors
 * to device memory.  max_ctx <= 16384. */
int icua_engine_create(const char* path, int max_ctx, int max_pass, int max_steps, uint32_t flags,
                       icua_engine** out);
/* Same, from an in-memory .icua image (len bytes) that the caller keeps alive during the call. */
int icua_engine_create_from_memory(const void* image, size_t len, int max_ctx, int max_pass, int max_steps,
                                   uint32_t flags, icua_engine** out);
void icua_engine_destroy(icua_engine* e);
int icua_engine_info(icua_engine* e, icua_info_t* out);

/* Engine.eos (Engine.swift:12). */
int icua_set_eos(icua_engine* e, int32_t eos0, int32_t eos1);
/* Engine.usePrefixCache and the grammar option. */
int icua_set_flags(icua_engine* e, uint32_t flags);

/* Engine.prepareMRoPE(visOffset:llmH:llmW:) (Engine.swift:254-298); vis_offset < 0: text only. */
int icua_prepare_mrope(icua_engine* e, int vis_offset, int llm_h, int llm_w);

/* Replaces Engine.poolerBuf / deepstackBufs (Engine.swift:20-21): visual embeddings
 * pooler[n_vis][2048] and three DeepStack sets deepstack[i][n_vis][2048], fp32 host arrays.
 * deepstack may be NULL (no DeepStack injection). */
int icua_set_visual(icua_engine* e, const float* pooler, const float* const* deepstack, int n_vis);

/* Engine.encodePrefill (Engine.swift:658-673) run to completion: embeds tokens[0..n) at cache
 * slots start_pos.., runs every decoder layer (DeepStack after layers 0-2 at the visual rows),
 * then lm_head + greedy commit of the first generated token.  Resets step/done.  q4 prompts
 * longer than 8 rows run as many-token matrix-core GEMMs and flash attention in chunks of up to
 * 4096 rows (unless ICUA_FLAG_PASS_PREFILL); other formats and short prompts run in passes of 8.
 * vis_offset is the row of the first image-pad token in `tokens` (-1: none).
 * write_logits: keep the first-token logits for icua_logits(). */
int icua_prefill(icua_engine* e, const int32_t* tokens, int n, int start_pos, int vis_offset, int max_new,
                 int write_logits);

/* k x Engine.encodeDecodeStep (Engine.swift:675-681): k passes, GPU-resident with token feedback
 * on the device; returns after completion.  Passes after a stop are no-ops.  A pass commits one
 * token, or two when its commit forces a grammar pair, whose two tokens then go through the next
 * pass together (n = 2, Shaders.swift:1553).  The single-row passes run in one persistent
 * cooperative kernel (one workgroup per CU), and a pair's pass in a launch of the kernel's
 * two-row form (q4 / q8) or as one replay of the per-stage graph (f16); ICUA_FLAG_GRAPH_DECODE
 * replays a captured HIP graph of the per-stage kernels per pass.  All paths compute the same
 * arithmetic. */
int icua_decode_steps(icua_engine* e, int k);

/* Engine.generateVision (Engine.swift:696-827) minus the vision encoder: prefill + greedy decode
 * of up to max_new tokens; out_tokens receives them up to (excluding) EOS; *n_out their count.
 * vis_offset: first image-pad row or -1; with ICUA_FLAG_PREFIX_CACHE the KV of an identical
 * prefix tokens[0..vis_offset) is reused. */
int icua_generate(icua_engine* e, const int32_t* tokens, int n, int vis_offset, int max_new,
                  int32_t* out_tokens, int* n_out);

/* Engine.encodeVision (Engine.swift:317-473): runs the vision tower and its mergers on an RGB8
 * frame [height][width][3] (sides multiples of 32, at most 1024 16 x 16 patches) and keeps its
 * outputs as the visual rows of the next prefill: pooler and the three DeepStack sets,
 * (height / 32) * (width / 32) rows each.  Fails if the model file has no vision tower. */
int icua_vision(icua_engine* e, const uint8_t* rgb, int width, int height);

/* Engine.generateVision (Engine.swift:696-827): icua_vision on the frame (skipped with
 * ICUA_FLAG_VISION_DELTA_CACHE when the frame, by its 8-byte-word FNV hash and its size, equals
 * the last one), vis_offset = first 151655 (<|image_pad|>) in tokens, the M-RoPE table of the
 * (height / 32) x (width / 32) grid, then icua_generate.  The timing record includes vision_ms. */
int icua_generate_vision(icua_engine* e, const uint8_t* rgb, int width, int height, const int32_t* tokens, int n,
                         int max_new, int32_t* out_tokens, int* n_out);

/* Speculative verify: m <= 8 draft tokens at the current position in one pass with a causal
 * tail; out_argmax[m] gets each row's greedy token; out_logits ([m][151936]) may be NULL.
 * The cache keeps the drafts' K/V; the position is left unchanged (the caller accepts a prefix
 * and calls icua_set_position).  No reference counterpart: the reference's n = 2 grammar pass
 * (Shaders.swift:735-788) is the closest multi-token decode. */
int icua_verify(icua_engine* e, const int32_t* draft, int m, int32_t* out_argmax, float* out_logits);

/* Rewinds / advances the cache position and re-arms decoding with `next_token` as the input of
 * the next step (done = 0). */
int icua_set_position(icua_engine* e, int pos, int32_t next_token, int step, int max_steps);

/* Reads the control block / the committed tokens / the last written logits (rows x 151936). */
int icua_read_state(icua_engine* e, icua_state_t* out);
int icua_read_tokens(icua_engine* e, int32_t* dst, int n);
int icua_logits(icua_engine* e, float* dst, int rows);

/* Engine.lastTiming (Engine.swift:52, 818-825). */
int icua_timing(icua_engine* e, icua_timing_t* out);

/* Engine.encodeLLMLayer (Engine.swift:476-629) on explicit rows: runs decoder layer `layer` on
 * x_in[n][2048] (fp32) for cache slots pos..pos+n-1 (n <= 8), writes their K/V, x_out[n][2048]. */
int icua_layer_step(icua_engine* e, int layer, const float* x_in, int n, int pos, float* x_out);

/* KV cache access (kc/vc, Engine.swift:110-112): kind 0 = K, 1 = V; data [8][nslots][128] fp16. */
int icua_read_kv(icua_engine* e, int layer, int kind, int slot0, int nslots, uint16_t* dst);
int icua_write_kv(icua_engine* e, int layer, int kind, int slot0, int nslots, const uint16_t* src);

/* Pass activations of the last layer run (Engine.swift:24 x, qkvBuf, attn, hbuf): for tests.
 * ICUA_BUF_X fp32 [8][2048]; ICUA_BUF_QKV fp32 [8][4096] raw fused QKV rows; ICUA_BUF_ATTN fp32
 * [8][2048] attention output; ICUA_BUF_MLP fp32 [8][6144] SwiGLU output; ICUA_BUF_POOLER and
 * ICUA_BUF_DEEPSTACK0 + i fp32 [n_vis][2048], the visual rows of the next prefill. */
enum {
    ICUA_BUF_X = 0,
    ICUA_BUF_QKV = 1,
    ICUA_BUF_ATTN = 2,
    ICUA_BUF_MLP = 3,
    ICUA_BUF_POOLER = 4,
    ICUA_BUF_DEEPSTACK0 = 5
};
int icua_read_buffer(icua_engine* e, int which, void* dst, size_t bytes);

/* ---- standalone kernels on device buffers (isolated dequant-GEMV sweep, codec checks) ---- */
int icua_dev_alloc(size_t bytes, void** ptr);
int icua_dev_free(void* ptr);
int icua_memcpy_h2d(void* dst, const void* src, size_t bytes);
int icua_memcpy_d2h(void* dst, const void* src, size_t bytes);
int icua_device_sync(void);

/* Repacks a row-major .icua matrix [N][K] (codes + scales, Convert.swift:157-171) into the
 * engine's device layout: 16-row matrix-core tiles, same byte count; scales keep their layout.
 * K in {2048, 6144}, N % 16 == 0. */
int icua_repack(int fmt, const void* d_codes, const void* d_sb, int N, int K, void* d_tiled_codes, void* d_tiled_sb);
/* y[m][N] = W[N][K] . x[m][K]: W repacked by icua_repack, x fp32, y fp32; K in {2048, 6144},
 * N % 16 == 0, m <= 8.  The dot64_row GEMV family of Shaders.swift:480-595.  q4 / q8 products
 * run on a streaming schedule, one workgroup per CU (one token: N <= 655360; 2-8 tokens: codes
 * under 2 GiB). */
int icua_gemv(int fmt, const void* d_codes, const void* d_sb, int N, int K, const float* d_x, int m, float* d_y);
/* Times `iters` launches of icua_gemv (m = 1) cycling over `ncopies` weight copies; *avg_us per
 * launch (HIP events on the launch stream). */
int icua_gemv_bench(int fmt, const void* const* d_codes, const void* const* d_sb, int ncopies, int N, int K,
                    const float* d_x, float* d_y, int iters, double* avg_us);
/* Bit-exact dequantisation of rows [row0, row0 + rows) to fp32 (Shaders.swift:464-476), from
 * the row-major .icua layout (tiled = 0) or the repacked layout (tiled = 1). */
int icua_dequant(int fmt, const void* d_codes, const void* d_sb, int K, int row0, int rows, float* d_out, int tiled);

/* ---- converter quantisers (Convert.swift:214-320, Converter.quantizeQ8 / quantizeQ4Raw) ---- */
/* Quantises the row-major fp32 matrix d_m [rows][cols] into the .icua layout, bit-exact with the
 * reference's float32 arithmetic:
 *   ICUA_FMT_Q8: symmetric, group 32 along K: d_codes int8 [rows][cols], d_sb fp16 scales
 *                [rows][cols/32] (quantizeQ8, Convert.swift:215-241).
 *   ICUA_FMT_Q4: affine, group 64: d_codes packed [rows][cols/2] (q[2j] | q[2j+1] << 4), d_sb fp16
 *                (scale, bias) [rows][cols/64][2], each pair from the 5 x 5 clip grid with a
 *                least-squares refit (quantizeQ4Raw / quantGroup, Convert.swift:243-320).
 * cols must be a multiple of the group size.  All pointers are device buffers. */
int icua_quantize(int fmt, const float* d_m, int rows, int cols, void* d_codes, void* d_sb);
/* icua_quantize without any device allocation.  No counterpart in the reference: it is for
 * callers that must not allocate device memory (serving loops, harnesses that forbid hipMalloc).
 * It launches on the null stream and synchronises the device before returning, so it cannot be
 * recorded into a stream capture; its first call on a device looks up the scratch array's
 * address (hipGetSymbolAddress), so make that call outside any capture.  The q4 quantiser's
 * per-group scratch (one byte per 64-weight group) is a
 * static device array of 8 MiB per GPU, so rows * cols / 64 must not exceed 8,388,608 (larger
 * matrices fail with an error; icua_quantize takes any size).  Every call on one GPU shares that
 * array: calls that overlap on one GPU (other host threads, other streams) race.  Each call
 * rewrites every byte it reads, so nothing carries over from an earlier call. */
int icua_quantize_noalloc(int fmt, const float* d_m, int rows, int cols, void* d_codes, void* d_sb);
/* Times `iters` back-to-back icua_quantize launches on the same buffers; *avg_us per call (HIP
 * events on the launch stream). */
int icua_quantize_bench(int fmt, const float* d_m, int rows, int cols, void* d_codes, void* d_sb, int iters,
                        double* avg_us);

#ifdef __cplusplus
}
#endif
#endif
