/*
 * GGUF v3 container types consumed by the executor ABI.
 *
 * Replaces: vendor/embeddinggemma.c/src/gguf.h:8-59 (the ei_gguf / ei_tensor /
 * ei_kv layout the engine passes to ei_gemma2_kfd_create). The field order,
 * types and scalar normalisation (unsigned -> v.u64, signed -> v.i64,
 * F32/F64 -> v.f64, BOOL -> v.b; gguf.c:46-61) are identical so the engine's
 * own mmapped ei_gguf can be handed to this library unchanged. This header
 * and the engine's share an include guard: a translation unit uses
 * whichever it includes first (engine.c includes gemma2_kfd.h, hence this
 * one, first; model.c and gguf.c use the engine's), and the two layouts
 * are identical, so records parsed by the engine's gguf.c read correctly
 * here.
 */
#ifndef EI_GGUF_H
#define EI_GGUF_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

enum ei_gguf_kv_type {
    EI_GGUF_U8 = 0, EI_GGUF_I8, EI_GGUF_U16, EI_GGUF_I16,
    EI_GGUF_U32, EI_GGUF_I32, EI_GGUF_F32, EI_GGUF_BOOL,
    EI_GGUF_STRING, EI_GGUF_ARRAY, EI_GGUF_U64, EI_GGUF_I64, EI_GGUF_F64,
};

/* ggml tensor element types (GGML ids). */
enum ei_tensor_type {
    EI_T_F32 = 0,
    EI_T_F16 = 1,
    EI_T_Q4_0 = 2,
    EI_T_Q8_0 = 8,
    EI_T_BF16 = 30,
};

typedef struct {
    const char *str; /* not NUL-terminated */
    uint64_t len;
} ei_str;

typedef struct {
    ei_str key;
    uint32_t type;
    union { uint64_t u64; int64_t i64; double f64; bool b; ei_str s; } v;
    uint32_t arr_type;
    uint64_t arr_n;
    const void *arr_data; /* packed scalars, or an ei_str index for STRING */
} ei_kv;

typedef struct {
    ei_str name;
    uint32_t n_dims;
    uint64_t ne[4]; /* ne[0] = row length */
    uint32_t type;
    uint64_t offset; /* relative to the data section */
    const void *data;
    uint64_t n_bytes;
} ei_tensor;

typedef struct {
    const uint8_t *map;
    size_t map_len;
    uint32_t version;
    uint64_t n_kv;
    uint64_t n_tensors;
    uint64_t alignment;
    uint64_t data_off;
    ei_kv *kv;
    ei_tensor *tensors;
} ei_gguf;

#endif /* EI_GGUF_H */
