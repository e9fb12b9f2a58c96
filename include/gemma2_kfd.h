/*
 * Executor C ABI of the packed-batch encoder forward, served on one MI355X
 * (gfx950) through HIP.
 *
 * Replaces: src/gemma2_kfd.h:7-10 (declarations) and src/gemma2_kfd.cpp:358-366
 * (definitions). Same three symbols, same arguments, same ownership and the
 * same error contract, so engine.c:39-45, :942-946, :1046-1049 and :216-218
 * link against this library unchanged.
 *
 *  ei_gemma2_kfd_create  g: a parsed GGUF (the engine's mmapped file) holding
 *      the `gemma-embedding` tensors with Q8_0 matrices; it must outlive the
 *      context. Returns NULL and writes "HIP: <reason>" into err on failure.
 *  ei_gemma2_kfd_free    NULL-safe.
 *  ei_gemma2_kfd_batch   ids[offsets[batch]], offsets[0] == 0, strictly
 *      increasing, 1 <= offsets[batch] <= 2048, batch <= 2048, ids in
 *      [0, 262144). Writes out[batch * 768], each row L2-normalised. Returns
 *      false and writes "HIP: <reason>" on failure; after a device failure
 *      the context is poisoned and every later call fails. Calls from
 *      several threads are safe: each runs on one of the context's lanes
 *      (eg2_hip.h), up to that many at the same time.
 */
#ifndef EG2_KFD_H
#define EG2_KFD_H
#ifdef __cplusplus
extern "C" {
#endif
#include "gguf.h"
void *ei_gemma2_kfd_create(const ei_gguf *g, char *err, size_t len);
void ei_gemma2_kfd_free(void *ctx);
bool ei_gemma2_kfd_batch(void *ctx, const int32_t *ids, const size_t *offsets,
                         size_t batch, float *out, char *err, size_t len);
#ifdef __cplusplus
}
#endif
#endif
