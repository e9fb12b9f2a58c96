/*
 * Deterministic wave packing and stream execution for the packed-batch
 * executor: the dynamic batcher's wave-forming rules restated for a queue
 * whose entries have all arrived, and a runner that embeds a whole stream
 * of texts wave by wave through ei_gemma2_kfd_batch.
 *
 * The reference batcher (vendor/embeddinggemma.c/src/inference_service.c)
 * decides wave boundaries with timers and condition variables
 * (:546-580); with every request already queued its choices reduce to the
 * fit rules restated here, which is what a reproducible stream benchmark
 * needs. The batcher itself is not replaced: it keeps calling the
 * executor's C ABI (gemma2_kfd.h).
 */
#ifndef EG2_STREAM_H
#define EG2_STREAM_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The batcher settings that shape waves (inference_service.c:60-70 config,
 * :892-895 environment; launcher values scripts/run.sh:17-19). */
typedef struct {
    size_t max_batch_tokens;          /* token budget of a wave (2048) */
    size_t max_batch_sequence_tokens; /* a longer sequence runs alone (2048) */
    size_t max_batch_requests;        /* sequences per wave (32) */
    unsigned lookahead;               /* EI_BATCH_LOOKAHEAD, default 1 */
    unsigned sort_longest_first;      /* EI_BATCH_SORT, default 1 */
} eg2_batch_config;

/* The launcher's settings: 2048 / 2048 / 32, lookahead and sort on. */
void eg2_batch_config_default(eg2_batch_config *cfg);

/* Splits a queue of n sequences (lengths[i] tokens, queue order) into
 * waves by inference_service.c:519-681:
 *  - a wave always takes the queue head;
 *  - lookahead (:631-663): if the head fits max_batch_sequence_tokens, the
 *    next 8 * max_batch_requests queued entries are scanned and each one
 *    that fits (its length <= max_batch_sequence_tokens and the wave total
 *    stays <= max_batch_tokens) joins, until max_batch_requests; entries
 *    passed over stay queued in order;
 *  - without lookahead (:611-630): entries join from the head in order
 *    until the first one that does not fit;
 *  - a head longer than max_batch_sequence_tokens runs alone;
 *  - sort_longest_first (:673-677): the wave runs longest sequence first
 *    (ties keep queue order).
 * Writes the sequence indices of every wave, wave after wave, to order[n]
 * and the end of wave w in order[] to wave_end[w] (wave_end needs room for
 * n entries). Returns the number of waves, or 0 on invalid arguments
 * (zero length, zero limits). */
size_t eg2_pack_waves(const size_t *lengths, size_t n, const eg2_batch_config *cfg, size_t *order,
                      size_t *wave_end);

/* kernels.c:393-407 ei_embedding_normalize_prefix on one 768-float
 * embedding: dims must be 128, 256, 512 or 768; for dims < 768 the first
 * dims values are L2-normalised in the SSE2 summation order
 * (kernels.c:82-94); 768 leaves the (already normalised) vector as is.
 * Returns false for unsupported dims. */
bool eg2_normalize_prefix(float *embedding, unsigned dims);

/* Embeds a stream of texts: text i is ids[text_offsets[i] ..
 * text_offsets[i+1]) with output width dims[i]. The texts are packed into
 * waves by eg2_pack_waves; the waves run on lanes taken from the context's
 * pool (eg2_hip.h) before the first wave: one, waited for, and as many more
 * as are free at that moment, up to the context's lane count (so that
 * concurrent callers never wait for each other's lanes). Wave w runs on the
 * (w mod taken)-th, so that up to that many waves are in flight, each
 * exactly as ei_gemma2_kfd_batch would run it (one hipGraph per lane and
 * padded wave size). Each embedding is
 * written to out[i * 768 ..] normalised to its prefix
 * (eg2_normalize_prefix; the values past dims[i] are zeroed). *n_waves (if
 * not NULL) receives the wave count. Returns false and a "HIP: ..." message
 * on any error (invalid text, unsupported dims, executor failure). */
bool eg2_stream_embed(void *ctx, const int32_t *ids, const size_t *text_offsets, size_t n_texts, const unsigned *dims,
                      const eg2_batch_config *cfg, float *out, size_t *n_waves, char *err, size_t len);

#ifdef __cplusplus
}
#endif
#endif
