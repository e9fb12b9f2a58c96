/*
 * Text -> token ids for the packed-batch executor: the SentencePiece-style
 * tokenizer of vendor/embeddinggemma.c/src/tokenizer.c (ei_tokenizer_init,
 * ei_tokenize_spm, ei_tokenizer_text_to_id) over the tokenizer.ggml.* keys
 * of a GGUF file, bit-exact with it, plus a multi-threaded batch form that
 * writes ids and offsets packed the way ei_gemma2_kfd_batch takes them.
 */
#ifndef EG2_TOKENIZER_H
#define EG2_TOKENIZER_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#include "gguf.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct eg2_tokenizer eg2_tokenizer;

/* tokenizer.c:205-269 ei_tokenizer_init over g's tokenizer.ggml.tokens /
 * .scores / .token_type (+ .merges: the ranked-merge mode of the reference's
 * embeddinggemma2 profile), .bos/eos/unknown/padding_token_id and
 * .add_bos_token / .add_eos_token / .add_space_prefix (model.c:111-120
 * defaults). The pieces are borrowed: g must outlive the tokenizer.
 * Returns NULL and "HIP: <reason>" in err when a key is missing or
 * malformed or a byte has no fallback token (where the reference dies). */
eg2_tokenizer *eg2_tokenizer_create(const ei_gguf *g, char *err, size_t len);
void eg2_tokenizer_free(eg2_tokenizer *tok);

/* tokenizer.c:184-187: the id of the piece `text` (the last id when pieces
 * repeat), or -1. */
int32_t eg2_tokenizer_text_to_id(const eg2_tokenizer *tok, const char *text, size_t len);

/* tokenizer.c:574-631 ei_tokenize_spm: special pieces split out first
 * (control and unknown ones only when parse_special), spaces escaped to
 * U+2581 with a leading one after a special (add_space_prefix), then the
 * bigram merges by score (ranked merges and newline runs in the merge
 * mode), pieces outside the vocabulary re-segmented or byte-encoded; BOS /
 * EOS by add_special and the model flags. Writes min(count, cap) ids and
 * returns count. */
size_t eg2_tokenize(const eg2_tokenizer *tok, const char *text, size_t len, bool add_special, bool parse_special,
                    int32_t *ids, size_t cap);

/* eg2_tokenize over n texts (text i = texts[text_offsets[i] ..
 * text_offsets[i+1])) on `threads` threads (0: one per hardware thread,
 * at most 32): the ids of text i go to ids[id_offsets[i] .. id_offsets[i+1])
 * (id_offsets has n + 1 entries, id_offsets[0] = 0), the packing
 * ei_gemma2_kfd_batch takes. Returns the total count, or SIZE_MAX (nothing
 * written to ids) when it exceeds cap. */
size_t eg2_tokenize_batch(const eg2_tokenizer *tok, const char *texts, const size_t *text_offsets, size_t n,
                          bool add_special, bool parse_special, int32_t *ids, size_t cap, size_t *id_offsets,
                          unsigned threads);

#ifdef __cplusplus
}
#endif
#endif
