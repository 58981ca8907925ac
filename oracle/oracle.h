/* CPU oracle for the Qwen3-VL text-decoder token loop -- TEST INFRASTRUCTURE ONLY.
 *
 * This library is the parity checker.  Only tests, the smoke check and the CPU-baseline
 * leg of the benchmark may load it; the product library never links or calls it.
 *
 * It restates the reference decoder math (tools/reference/qwen3vl_ref.py:142-155,
 * 243-336), which is fp32 throughout, over weights dequantised bit-exactly from the
 * reference codecs (Sources/Engine/Convert.swift:215-270; Shaders.swift:464-476), with an
 * fp16 KV cache (the reference engine's cache format, Shaders.swift:776-787, 914-921; the
 * workloads specify it) and the engine's M-RoPE table (Sources/Engine/Engine.swift:121-125,
 * 254-298).
 *
 * Arithmetic contract: every operation is evaluated in double precision and each
 * intermediate tensor is stored as float32 (round-to-nearest-even).  GEMV inputs are those
 * float32 values (the reference engine's extra fp16 rounding of GEMV inputs,
 * Shaders.swift:634-669, is not applied).  K/V rows are rounded to fp16 when written to
 * the cache.  Dot products accumulate in double: products of an fp32 weight and an fp32
 * activation are exact in double, so a dot product carries one double rounding per term.
 *
 * Results do not depend on the OpenMP thread count: every dot product and every
 * reduction is computed by one thread in a fixed order.
 */
#ifndef ICUA_ORACLE_H
#define ICUA_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Fixed decoder dimensions (Sources/Engine/ModelFile.swift:47-59). */
#define OR_H 2048
#define OR_FF 6144
#define OR_NH 16
#define OR_NKV 8
#define OR_HD 128
#define OR_QKV 4096
#define OR_GU 12288
#define OR_VOCAB 151936
#define OR_MAXLAYERS 28
#define OR_IMAGE_PAD 151655

/* fp16 <-> fp32 (IEEE binary16, round to nearest even). */
float or_h2f(uint16_t h);
uint16_t or_f2h(float f);

/* Dequantise `rows` rows of a [rows][K] matrix to fp32 (fmt 0 f16, 1 q8, 2 q4).
 * q4: w = fl32(s * q + b) (Convert.swift:245-262; Shaders.swift:470-475);
 * q8: w = s * q (Convert.swift:214-233; Shaders.swift:466-468); f16: w = half value. */
void or_dequant(int fmt, const uint8_t* codes, const uint8_t* sb, int rows, int K, float* out);

/* y[t][r] = sum_k W[r][k] * x[t][k] for t < n tokens; x fp32 [n][K];
 * double accumulation, float32 result. */
void or_gemv(int fmt, const uint8_t* codes, const uint8_t* sb, int N, int K,
             const float* x, int n, float* y);

/* Engine M-RoPE table rope[slot][64] = (cos, sin) float pairs (Engine.swift:254-298). */
void or_mrope_table(int maxctx, int vis_offset, int llm_h, int llm_w, float* out);

/* Whole-decoder state over an in-memory .icua image. */
typedef struct or_model or_model;

or_model* or_model_new(const uint8_t* img, size_t len, int maxctx);
void or_model_free(or_model* m);
int or_model_layers(const or_model* m);
int or_model_format(const or_model* m);
const char* or_last_error(void);

/* prepareMRoPE (Engine.swift:254-298); vis_offset < 0 means text-only. */
void or_prepare_mrope(or_model* m, int vis_offset, int llm_h, int llm_w);

/* KV cache of layer l: kind 0 = K, 1 = V; layout [NKV][maxctx][HD] fp16. */
uint16_t* or_kv(or_model* m, int layer, int kind);

/* Runs decoder layer `l` on n rows of the fp32 residual x[n][H] in place, for tokens at
 * cache slots pos .. pos+n-1 (causal).  Writes their K/V into the cache. */
void or_layer(or_model* m, int l, float* x, int n, int pos);

/* Test taps: when set (non-NULL), or_layer copies its raw QKV rows [n][4096], attention output
 * [n][2048] and SwiGLU output [n][6144] (fp32) into these buffers. */
void or_debug_taps(float* qkv, float* att, float* act);

/* Token embedding row (Shaders.swift:676-692 text branch) into x[H]. */
void or_embed(const or_model* m, int tok, float* x);

/* Final RMSNorm + tied lm_head of one residual row: logits[VOCAB]. */
void or_lm_head(const or_model* m, const float* x, float* logits);

/* One pass of n tokens at slots pos..pos+n-1 (prefill, decode step or verify):
 *  - token rows are embedded from E; if vis_offset >= 0, rows vis_offset..vis_offset+n_vis-1
 *    holding IMAGE_PAD take pooler rows (fp32 [n_vis][H]) instead (Shaders.swift:676-692);
 *  - after layers 0..2 the deepstack[i] rows (fp32 [n_vis][H]) are added to those rows
 *    (qwen3vl_ref.py:279-283; Shaders.swift:696-707), when deepstack is not NULL;
 *  - logits_rows = 0: none; 1: last row only; n: every row.  logits: [logits_rows][VOCAB].
 * Returns 0 on success. */
int or_pass(or_model* m, const int32_t* toks, int n, int pos, const float* pooler, int vis_offset,
            int n_vis, const float* const* deepstack, int logits_rows, float* logits);

/* Lowest index of the maximum (np.argmax semantics; Shaders.swift:1476-1488, 1509-1530). */
int or_argmax(const float* v, int n);

/* Greedy generation: prefill `toks` (n) at slot 0 with the visual inputs as in or_pass,
 * then decode until `steps` tokens are produced (the first from the prefill).  No EOS
 * stop.  out_tokens[steps]; margins[steps] (top-1 minus top-2 logit, may be NULL);
 * top1[steps] (the top-1 logit of each step, may be NULL); out_first_logits[VOCAB] (may be
 * NULL).  Returns 0 on success. */
int or_generate(or_model* m, const int32_t* toks, int n, const float* pooler, int vis_offset,
                int n_vis, const float* const* deepstack, int steps, int32_t* out_tokens,
                float* margins, float* top1, float* out_first_logits);

/* The reference's token loop (Engine.swift:741-817) with its commit rules (Shaders.swift:
 * 1531-1561): prefill `toks` (n) at slot 0 with the visual inputs as in or_pass, then passes
 * until a stop.  Each pass commits the argmax of its last row (ties to the lowest id) as
 * out_tokens[step++] and stops on eos0 / eos1 / max_steps, and on token 8 (")") when `grammar`
 * is set.  With `grammar`, a token 11, or one of {3678, 7241, 12476, 10855, 11862, 1339, 1472,
 * 24769} at step 1, is followed by a forced token (220 after 11, else 7) written as the next
 * out_tokens entry, and the next pass carries both tokens.  A pass that would start with
 * step >= max_steps (a forced token took the last slot) ends the loop: the reference commits one
 * more token there, past its max_steps-entry buffer.  Returns the number of tokens written
 * (out_tokens holds max_steps), or -1 on error. */
int or_generate_commit(or_model* m, const int32_t* toks, int n, const float* pooler, int vis_offset, int n_vis,
                       const float* const* deepstack, int max_steps, int eos0, int eos1, int grammar,
                       int32_t* out_tokens);

/* fp32 CPU port (port32.c) -- the benchmark's CPU baseline, not the checker: a pass of n text
 * tokens at slots pos .. pos+n-1 in fp32 arithmetic (fused dequantise-and-dot GEMVs, fp16 KV
 * cache written as the oracle does), logits of the last row.  Returns -1 if the pass exceeds
 * the context. */
int p32_pass(or_model* m, const int32_t* toks, int n, int pos, float* logits);

/* Group-wise quantisers of the .icua converter, restated in float32 with the reference's
 * operation order (Sources/Engine/Convert.swift:214-320; built with -ffp-contract=off).
 * m is row-major [rows][cols].
 *  or_quant_q8: symmetric, group 32 (Convert.swift:215-241): codes int8 [rows][cols], scales
 *      fp16 [rows][cols / 32].
 *  or_quant_q4: affine, group 64 (Convert.swift:243-320): packed codes [rows][cols / 2],
 *      (scale, bias) fp16 [rows][cols / 64][2].
 * Both process 64-row chunks independently (the reference's concurrentPerform iterations). */
void or_quant_q8(const float* m, int rows, int cols, int8_t* codes, uint16_t* scales);
void or_quant_q4(const float* m, int rows, int cols, uint8_t* packed, uint16_t* sb);

/* Vision encoder and mergers (oracle/vision.c; Sources/Engine/Engine.swift:189-246, 317-473;
 * Shaders.swift:59-454; tools/reference/qwen3vl_ref.py:25-85, 165-216).  Dimensions from
 * Sources/Engine/ModelFile.swift:31-45.  fp16 tensors are uint16_t bit patterns. */
#define OR_VH 1024
#define OR_VFF 4096
#define OR_VNH 16
#define OR_VHD 64
#define OR_VQKV 3072
#define OR_VPATCH 768
#define OR_VLAYERS 24
#define OR_VPOS 48
#define OR_MH 4096
#define OR_NPATCH_MAX 1024

/* RGB8 [gh * 16][gw * 16][3] -> fp16 patches [gh * gw][768] in 2 x 2 merge-block order. */
void or_vit_patchify(const uint8_t* rgb, int gh, int gw, uint16_t* out);
/* Bilinear (align_corners) interpolation of the [48 * 48][1024] position table: [gh * gw][1024]. */
void or_vit_pos_interp(const float* table, int gh, int gw, float* out);
/* 2D RoPE table [gh * gw][32] of (cos, sin): row angles for j < 16, column angles after. */
void or_vit_rope_table(int gh, int gw, float* out);
/* LayerNorm (eps 1e-6) of rows of n floats to fp16. */
void or_layernorm_f16(const float* x, const float* w, const float* b, int rows, int n, uint16_t* out);
/* y[M][N] = X[M][K] W[N][K]^T + bias, fp16 operands, float32 result. */
void or_linear_f16(const uint16_t* X, const uint16_t* W, const float* bias, int M, int N, int K, float* y);
float or_gelu_tanh(float x);
float or_gelu_erf(float x);
/* Bidirectional attention: q, k, v fp16 [16][np][64] -> out fp16 [np][1024]. */
void or_vit_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, int np, uint16_t* out);
/* The whole encoder over the vision tensors of an .icua image: pooler [np / 4][2048] and the three
 * DeepStack outputs (entries may be NULL) [np / 4][2048], float32.  Returns 0, or -1 with
 * or_vision_error() set. */
int or_vision(const uint8_t* img, size_t len, const uint8_t* rgb, int gh, int gw, float* pooler,
              float* const* deepstack);
const char* or_vision_error(void);
/* Block l of the tower on the float32 residual x [gh * gw][1024] in place (test tap). */
int or_vit_block(const uint8_t* img, size_t len, int l, float* x, int gh, int gw);

/* Threads used by the OpenMP regions (0 = library default). */
void or_set_threads(int n);
int or_get_threads(void);

#ifdef __cplusplus
}
#endif
#endif
