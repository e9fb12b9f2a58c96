/*
 * Driver for the reference CPU path, compiled together with the reference's
 * own sources where they lie (see oracle/Makefile). Nothing from the
 * reference is copied here: gemma2.c is compiled as part of this
 * translation unit only so that its file-local Q8_0 x Q8_0 `mm`
 * (gemma2.c:142-153) can be called. The public functions of quants.c and
 * kernels.c are called directly from the shared library by the fixture
 * script (tests/golden/make_golden.py) and the cross-check tests.
 */
#include "gemma2.c"

/* y[n][m] = x[n][k] (quantized to Q8_0 by mm) . W[m][k]^T, W in GGUF Q8_0. */
void ref_mm_q8_0(const void *w_blocks, int k, int m, const float *x, int n, float *y) {
    ei_tensor t;
    memset(&t, 0, sizeof t);
    t.type = EI_T_Q8_0;
    t.n_dims = 2;
    t.ne[0] = (uint64_t)k;
    t.ne[1] = (uint64_t)m;
    t.ne[2] = 1;
    t.ne[3] = 1;
    t.data = w_blocks;
    t.n_bytes = (uint64_t)m * (uint64_t)(k / 32) * 34u;
    mm(NULL, &t, x, n, y);
}

/* input_embeddings (engine.c:288-295) for one row: dequant * sqrtf(768). */
void ref_embed_row(const void *table, int vocab, int row, float *out) {
    ei_tensor t;
    memset(&t, 0, sizeof t);
    t.type = EI_T_Q8_0;
    t.n_dims = 2;
    t.ne[0] = EI_N_EMBD;
    t.ne[1] = (uint64_t)vocab;
    t.ne[2] = 1;
    t.ne[3] = 1;
    t.data = table;
    ei_dequantize_row_q8_0_scaled(&t, row, sqrtf((float)EI_N_EMBD), out);
}

/* The reference tokenizer (tokenizer.c) over the tokenizer keys of a GGUF
 * file, read as model.c:111-120 reads them; the merge mode when the file
 * has tokenizer.ggml.merges (the embeddinggemma2 profile). */
#include "tokenizer.h"

typedef struct {
    ei_model m;
    ei_tokenizer tok;
} ref_tok;

void *ref_tokenizer_open(const char *path) {
    ref_tok *h = calloc(1, sizeof *h);
    ei_gguf_open(&h->m.gguf, path);
    const ei_gguf *g = &h->m.gguf;
    h->m.embeddinggemma2 = ei_gguf_kv(g, "tokenizer.ggml.merges", false) != NULL;
    h->m.tok_tokens = ei_gguf_kv(g, "tokenizer.ggml.tokens", true);
    h->m.tok_scores = ei_gguf_kv(g, "tokenizer.ggml.scores", true);
    h->m.tok_types = ei_gguf_kv(g, "tokenizer.ggml.token_type", true);
    h->m.bos_id = (int32_t)ei_gguf_kv_u64(g, "tokenizer.ggml.bos_token_id", 2);
    h->m.eos_id = (int32_t)ei_gguf_kv_u64(g, "tokenizer.ggml.eos_token_id", 1);
    h->m.unk_id = (int32_t)ei_gguf_kv_u64(g, "tokenizer.ggml.unknown_token_id", 3);
    h->m.pad_id = (int32_t)ei_gguf_kv_u64(g, "tokenizer.ggml.padding_token_id", 0);
    h->m.add_bos = ei_gguf_kv_bool(g, "tokenizer.ggml.add_bos_token", true);
    h->m.add_eos = ei_gguf_kv_bool(g, "tokenizer.ggml.add_eos_token", false);
    h->m.add_space_prefix = ei_gguf_kv_bool(g, "tokenizer.ggml.add_space_prefix", true);
    ei_tokenizer_init(&h->tok, &h->m);
    return h;
}

size_t ref_tokenize(void *handle, const char *text, size_t len, int add_special, int parse_special, int32_t *ids,
                    size_t cap) {
    ref_tok *h = handle;
    ei_tokens t;
    ei_tokenize_spm(&h->tok, text, len, add_special != 0, parse_special != 0, &t);
    for (size_t i = 0; i < t.n && i < cap; i++) ids[i] = t.ids[i];
    const size_t n = t.n;
    ei_tokens_free(&t);
    return n;
}

void ref_tokenizer_close(void *handle) {
    ref_tok *h = handle;
    ei_tokenizer_free(&h->tok);
    ei_gguf_close(&h->m.gguf);
    free(h);
}
