/*
 * The output side of the embedding path: text and base64 forms of the
 * embeddings and the response body the reference's server builds from
 * them (vendor/embeddinggemma.c/src/server.c:1126-1190), for host-side
 * callers of the executor (a server, the stream runner's users).
 */
#ifndef EG2_FORMAT_H
#define EG2_FORMAT_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EG2_F32_CHARS 32u

/* float_format.c:276-308 ei_f32_to_chars: the shortest decimal that reads
 * back (round to nearest even) as exactly `value`; when several digit
 * strings of that length do, the one nearest to `value` (ties to the even
 * last digit). Laid out as float_format.c:244-274 does: "12.5", "100.0",
 * "0.00123", "1.5e+07", "-2e-05" (exponent sign always, at least two
 * exponent digits), zeros as "0.0" / "-0.0". Writes at most 32 bytes, no
 * terminator; returns the length, or 0 for a non-finite value. */
size_t eg2_f32_to_chars(char *dst, float value);

/* server.c:379-408: standard base64 ('+', '/', '=' padding) of the
 * little-endian bytes of count floats; writes 4 * ceil(4 count / 3) bytes,
 * no terminator, and returns that length. */
size_t eg2_base64_f32(const float *values, size_t count, char *dst);

typedef enum { EG2_API_OLLAMA = 0, EG2_API_OPENAI = 1 } eg2_embedding_api;
typedef enum { EG2_ENCODING_FLOAT = 0, EG2_ENCODING_BASE64 = 1 } eg2_embedding_encoding;

/* An upper bound of the bytes eg2_embeddings_response writes. */
size_t eg2_embeddings_response_bound(size_t n, unsigned dims, size_t model_len);

/* The body of an embedding response (server.c:1126-1190). embeddings holds
 * n rows of 768 floats; each row is first normalised to its first `dims`
 * values in place (kernels.c:403-407, ei_embedding_normalize_prefix; dims
 * must be 128, 256, 512 or 768), then written as a JSON array of
 * eg2_f32_to_chars values or as a quoted eg2_base64_f32 string:
 *   EG2_API_OLLAMA: {"embeddings":[E0,E1,...]}
 *   EG2_API_OPENAI: {"object":"list","data":[{"object":"embedding",
 *     "embedding":E0,"index":0},...],"model":"<model, JSON-escaped as
 *     server.c:356-377>","usage":{"prompt_tokens":P,"total_tokens":P}}
 * Writes at most cap bytes plus a terminating NUL and returns the length
 * (without the NUL); returns 0 when dims is unsupported, a value is not
 * finite, or cap is below eg2_embeddings_response_bound. */
size_t eg2_embeddings_response(float *embeddings, size_t n, unsigned dims, eg2_embedding_api api,
                               eg2_embedding_encoding encoding, const char *model, size_t model_len,
                               size_t prompt_tokens, char *dst, size_t cap);

#ifdef __cplusplus
}
#endif
#endif
