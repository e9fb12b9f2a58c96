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
