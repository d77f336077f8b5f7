/* hai_tokenizer.h -- C ABI of the Qwen checkpoint tokenizer (C++ host,
 * libhybridai.so): the reference's tokenizer::QwenTokenizer
 * (src/tokenizer/qwen_tokenizer.h:15-104), which hybridai::Generator uses to
 * turn a text prompt into token ids, to build the chat prompt, to add the
 * generation config's stop ids and to decode the result
 * (src/generator.cc:423, 469-480, 1032, 1275).  Host-only: no device calls.
 *
 * Buffers: a call whose output needs more than `capacity` elements writes
 * nothing, stores the needed count in *n_out and returns
 * HAI_ERR_INVALID_ARGUMENT; a call with capacity 0 is the size query.
 * Status codes are those of hai_kernels.h.
 */
#ifndef HAI_TOKENIZER_H
#define HAI_TOKENIZER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* QwenTokenizer::load (qwen_tokenizer.h:20): <dir>/tokenizer.json (BPE
 * model, merges, added tokens) and, when present, <dir>/generation_config.json
 * (eos / pad / bos ids).  NULL on failure, with *status HAI_ERR_FILE_NOT_FOUND
 * (no tokenizer.json) or HAI_ERR_INVALID_MODEL and a message. */
void* hai_tokenizer_open(const char* dir, int32_t* status, char* message, int64_t message_capacity);
void hai_tokenizer_close(void* tokenizer);

/* QwenTokenizer::encode (qwen_tokenizer.h:28-29): ids of text[0, text_bytes). */
int32_t hai_tokenizer_encode(void* tokenizer, const char* text, int64_t text_bytes, int64_t* ids, int64_t capacity,
                             int64_t* n_out);

/* QwenTokenizer::decode (qwen_tokenizer.h:31-33): the bytes of the tokens;
 * added tokens give their content unless skip_special and they are special.
 * A terminating NUL is written when capacity exceeds the byte count. */
int32_t hai_tokenizer_decode(void* tokenizer, const int64_t* ids, int64_t n_ids, int32_t skip_special, char* out,
                             int64_t capacity, int64_t* n_out);

/* QwenTokenizer::build_chat_prompt (qwen_tokenizer.h:37-40): messages as
 * (role, content) pairs of NUL-terminated strings. */
int32_t hai_tokenizer_chat_prompt(const char* const* roles, const char* const* contents, int64_t n_messages,
                                  int32_t add_generation_prompt, int32_t enable_thinking, char* out,
                                  int64_t capacity, int64_t* n_out);

/* eos_token_ids / pad_token_id / bos_token_id (qwen_tokenizer.h:42-47); -1
 * when generation_config.json does not give pad or bos. */
int32_t hai_tokenizer_special_ids(void* tokenizer, int64_t* eos, int64_t eos_capacity, int64_t* n_eos, int64_t* pad,
                                  int64_t* bos);

/* The pre-tokenizer's pieces of a text holding no added tokens, as byte
 * offsets: piece k is [bounds[2k], bounds[2k+1]); capacity counts int64
 * elements (two per piece) and *n_out the pieces.  No reference counterpart
 * as a public call (QwenTokenizer::pre_tokenize is private there); for
 * callers that need offsets and for checking the split on its own. */
int32_t hai_tokenizer_pieces(void* tokenizer, const char* text, int64_t text_bytes, int64_t* bounds,
                             int64_t capacity, int64_t* n_out);

#ifdef __cplusplus
}
#endif

#endif /* HAI_TOKENIZER_H */
