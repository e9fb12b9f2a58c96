/*
 * Launch-by-name entry point for the operator kernels that take the
 * include/abi.h records (embeddinggemma2-amdkfd_amd/csrc/kernels_abi.hip).
 *
 * Replaces: the by-name dispatch of a kernels/eg2.c code object,
 * src/gemma2_kfd.cpp:106-110 (kernel table) and :156-170 (`launch(name,
 * record, grid, block)`, the record copied as the kernarg segment), and the
 * `run` helper of tests/kernels.cpp:36-48. The same kernels are also built
 * into a stand-alone gfx950 code object whose symbols carry the reference
 * names, for loaders that dispatch by ".kd" symbol.
 *
 * Operators (name: record, workgroup size, grid in workgroups):
 *   eg2_saxpy          EgSaxpy         any     ceil(n / block)
 *   eg2_gather         EgGather        any     ceil(512 n / block)
 *   eg2_gather768      EgGather        any     ceil(768 n / block)
 *   eg2_mm             EgMM            256     (ceil(m/16), ceil(n/16))
 *   eg2_mm64           EgMM            256     (ceil(m/64), ceil(n/16))
 *   eg2_mm64x64        EgMM            256     (ceil(m/64), ceil(n/64))
 *   eg2_mmstep8        EgMM            256     (ceil(m/64), ceil(n/64))
 *   eg2_norm           EgNorm          64      rows
 *   eg2_rope           EgRope          any     ceil(n heads d/2 / block)
 *   eg2_attention256   EgAttention     64      4 n
 *   eg2_attention512   EgAttention     64      4 n
 *   eg2_attention256x3 EgAttention     64      3 n
 *   eg2_element        EgElement       any     ceil(n / block)
 *   eg2_pool           EgPool          any     ceil(768 batch / block)
 *   eg2_norm_residual  EgNormResidual  64      rows
 *   eg2_norm_rope      EgNormRope      64      rows
 * eg2_gather768 and eg2_attention256x3 are the 768-wide / 3-query-head
 * variants of the embedding-gemma 300M geometry; the others keep the
 * reference kernels' geometry (512-wide gather, 4 query heads).
 */
#ifndef EG2_OPS_H
#define EG2_OPS_H

#include <stddef.h>

#include "abi.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Kernarg layout of eg2_saxpy(float *y, const float *x, float a, unsigned n)
 * (kernels/eg2.c:31), which takes plain arguments rather than a record. */
typedef struct { float *y; const float *x; float a; unsigned n; } EgSaxpy;

/* Enqueues operator `name` with `record` (record_size bytes) on `stream`
 * (hipStream_t as void*, NULL = null stream). Returns 0 or a hipError_t
 * code; hipErrorInvalidValue (1) for an unknown name, a record of the wrong
 * size, a zero grid dimension, a workgroup size the operator does not take,
 * a NULL pointer the operator dereferences, a zero width, an odd rotary
 * width, an EgMM type other than 0/1/8/30 or an EgElement mode above 2.
 * Device pointers are not otherwise checked. Never synchronises. */
int eg2_op_launch(const char *name, const void *record, size_t record_size, unsigned grid_x, unsigned grid_y,
                  unsigned block, void *stream);

/* The operator names accepted by eg2_op_launch, index 0..eg2_op_count()-1. */
unsigned eg2_op_count(void);
const char *eg2_op_name(unsigned index);

#ifdef __cplusplus
}
#endif
#endif
