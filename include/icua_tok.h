/* Host tokenizer of the Qwen3-VL prompt (C ABI of libicua.so).
 *
 * Replaces the reference's Swift `Tokenizer` (Sources/Tokenizer/Tokenizer.swift:36-462, with
 * Core.swift:1-559): byte-level BPE with the Qwen2 split pattern and NFC, added tokens matched
 * on the raw text, the chat templates, decoding and the streaming detokenizer.  The file it opens
 * is written by instantcua_amd/tokenizer.py `compile` from a Hugging Face tokenizer.json, as
 * `Tokenizer.compile(tokenizerJSON:output:)` (Compile.swift:20) does for the reference's own
 * format.  All functions return 0 on success and -1 with icua_tok_last_error() set; output
 * arrays are caller-owned, and *n_out receives the full length even when cap is too small. */
#ifndef ICUA_TOK_H
#define ICUA_TOK_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Tokenizer.visionStart / visionEnd / imagePad (Tokenizer.swift:53-55). */
#define ICUA_TOK_VISION_START 151652
#define ICUA_TOK_VISION_END 151653
#define ICUA_TOK_IMAGE_PAD 151655

typedef struct icua_tok icua_tok;
typedef struct icua_tok_stream icua_tok_stream;

const char* icua_tok_last_error(void);

/* Tokenizer(path:) (Tokenizer.swift:60-125). */
int icua_tok_open(const char* path, icua_tok** out);
void icua_tok_close(icua_tok* t);
/* Tokenizer.vocabSize (57-58): token ids of the vocabulary and added tokens. */
int icua_tok_vocab_size(const icua_tok* t);
/* Id of an added token by its content ("<|im_end|>"), or -1; Tokenizer.imStart / imEnd /
 * endOfText (50-52) are looked up this way. */
int32_t icua_tok_special_id(const icua_tok* t, const char* content);

/* Tokenizer.encode (153) with with_specials = 0, encodeWithSpecials (159) with 1.  text is UTF-8. */
int icua_tok_encode(const icua_tok* t, const char* text, size_t len, int with_specials, int32_t* out, size_t cap,
                    size_t* n_out);
/* Tokenizer.encodeChat (166-186). */
int icua_tok_encode_chat(const icua_tok* t, const char* system, size_t slen, const char* user, size_t ulen, int32_t* out,
                         size_t cap, size_t* n_out);
/* Tokenizer.encodeVisionChat (192-204): *image_offset is the index of the first image-pad token. */
int icua_tok_encode_vision_chat(const icua_tok* t, const char* system, size_t slen, const char* user, size_t ulen,
                                int num_image_tokens, int32_t* out, size_t cap, size_t* n_out, int* image_offset);

/* Tokenizer.tokenBytes (334-338): raw bytes of a token, valid while t lives; empty for unknown ids. */
int icua_tok_token_bytes(const icua_tok* t, int32_t id, const uint8_t** bytes, size_t* len);
/* Tokenizer.decode (342-362): concatenated token bytes, invalid UTF-8 replaced by U+FFFD per
 * maximal subpart; unknown ids are skipped. */
int icua_tok_decode(const icua_tok* t, const int32_t* ids, size_t n, char* out, size_t cap, size_t* n_out);

/* TextStream (400-462): push one id (or -1 with final = 1 to flush) and receive the text that is
 * complete; the concatenation of every output equals icua_tok_decode of all ids. */
icua_tok_stream* icua_tok_stream_new(void);
void icua_tok_stream_free(icua_tok_stream* s);
int icua_tok_stream_push(const icua_tok* t, icua_tok_stream* s, int32_t id, int final, char* out, size_t cap,
                         size_t* n_out);

#ifdef __cplusplus
}
#endif
#endif
