/*
 * gs_tokens.h -- C ABI of the host-side text step after the sampler: token
 * id -> text, and the stop-token set the decode loop checks.
 *
 * Replaces, in gguf-rs-cli:
 *   Tokenizer::decode(&self, id: u32) -> String          src/tokenizer/bpe.rs:180-197
 *   build_byte_encoder() -> [char; 256]                   src/tokenizer/bpe.rs:199-208
 *   token_to_id (HashMap<String, u32>)                    src/tokenizer/bpe.rs:37-38
 *   ChatTemplate::detect(tok, chat_template) -> Self      src/tokenizer/chat.rs:9-24
 *   ChatTemplate::stop_tokens(&self, tok) -> Vec<u32>     src/tokenizer/chat.rs:57-72
 * The decode loop prints decode(next) for each sampled token
 * (src/main.rs:299-300) and stops on stop_tokens (src/main.rs:97, 281).
 *
 * Host code only (no device work).  Text is UTF-8 bytes, not NUL-terminated
 * unless stated.  Same status codes as gs_sampler.h.
 */
#ifndef GS_TOKENS_H
#define GS_TOKENS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* tokenizer.ggml.model (src/tokenizer/bpe.rs:52-56): "gpt2" -> GS_TOK_GPT2,
 * anything else -> GS_TOK_LLAMA. */
#define GS_TOK_LLAMA 0u
#define GS_TOK_GPT2  1u

/* ChatTemplate, in the reference's declaration order (src/tokenizer/chat.rs:4). */
#define GS_TMPL_CHATML 0u
#define GS_TMPL_LLAMA3 1u
#define GS_TMPL_LLAMA2 2u
#define GS_TMPL_GEMMA  3u
#define GS_TMPL_PHI3   4u
#define GS_TMPL_SIMPLE 5u

typedef struct gs_vocab gs_vocab;

/* The vocabulary: token i is the bytes data[offsets[i] .. offsets[i+1]) of
 * tokenizer.ggml.tokens; types = tokenizer.ggml.token_type (n_types entries,
 * possibly fewer than n: missing types read 0, as the reference's
 * .get(id).unwrap_or(0)).  Each token's decoded text is computed here once. */
int gs_vocab_create(const char *data, const uint64_t *offsets, size_t n, const uint32_t *types, size_t n_types,
                    uint32_t model, gs_vocab **out);
int gs_vocab_destroy(gs_vocab *v);

/* token_to_id lookup (src/tokenizer/bpe.rs:37-38; a string listed twice maps
 * to its last id).  *id = UINT32_MAX if absent. */
int gs_vocab_find(const gs_vocab *v, const char *s, size_t len, uint32_t *id);

/* Tokenizer::decode (src/tokenizer/bpe.rs:180-197): ids past the vocabulary
 * and tokens of type 2 or 3 give ""; Llama vocabularies map U+2581 to a
 * space; GPT-2 ones map each char through the byte decoder and, when every
 * char maps, return the bytes as UTF-8 with each maximal invalid subpart
 * replaced by U+FFFD (String::from_utf8_lossy), else the token unchanged.
 * Writes min(len, cap) bytes to out; *len = the full length. */
int gs_token_decode(const gs_vocab *v, uint32_t id, char *out, size_t cap, size_t *len);

/* The concatenation of gs_token_decode over n ids (the text the reference
 * prints, token by token, for a generated sequence). */
int gs_tokens_decode(const gs_vocab *v, const uint32_t *ids, size_t n, char *out, size_t cap, size_t *len);

/* ChatTemplate::detect (src/tokenizer/chat.rs:9-24): tmpl is the model's Jinja
 * template (NUL-terminated) or NULL. */
int gs_chat_template_detect(const gs_vocab *v, const char *tmpl, uint32_t *kind);

/* ChatTemplate::stop_tokens (src/tokenizer/chat.rs:57-72): the EOS ids plus
 * the template's end markers found in the vocabulary, sorted and deduplicated.
 * Writes min(count, cap) ids; *n = the full count. */
int gs_stop_tokens(const gs_vocab *v, uint32_t kind, const uint32_t *eos, size_t n_eos, uint32_t *out, size_t cap,
                   size_t *n);

#ifdef __cplusplus
}
#endif

#endif /* GS_TOKENS_H */
