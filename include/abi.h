/*
 * Operator ABI: plain-old-data argument records, one per operator, with raw
 * device pointers and unsigned counts.
 *
 * Replaces: kernels/abi.h:3-11, field for field (same order, same types), so
 * code written against the reference's operator records compiles unchanged.
 * Semantics (kernels/eg2.c):
 *   EgGather        out[t,:] = dequant(Q8_0 row ids[t]) * sqrt(width)
 *   EgMM            out[n x m] = x[n x k] . W[m x k]^T, W type = GGML id
 *                   (0 F32, 1 F16, 8 Q8_0, 30 BF16)
 *   EgNorm          out = x*scale / sqrt(mean((x*scale)^2) + 1e-6) * weight
 *   EgRope          NeoX rotation, table row per token = [cos(d/2) | sin(d/2)]
 *   EgAttention     streaming softmax over keys [bounds[2t], bounds[2t+1])
 *                   intersected with |t - s| <= window (0 = unlimited)
 *   EgElement       mode 0 (x + other)*scale; 1 gelu(x)*other; 2 per-layer gate
 *   EgPool          mean over rows [offsets[s], offsets[s+1])
 *   EgNormResidual  out = (out + rms(x)*weight) * scale
 *   EgNormRope      per-head RMS then NeoX rotation, in place
 * The records carry no head counts: head geometry is fixed per operator
 * variant (see eg2_hip.h).
 */
#ifndef EG2_OPERATOR_ABI_H
#define EG2_OPERATOR_ABI_H
typedef struct { float *out; const void *weight; const int *ids; unsigned n; } EgGather;
typedef struct { float *out; const float *x; const void *weight; unsigned n, k, m, type; } EgMM;
typedef struct { float *out; const float *x; const float *weight; unsigned rows, d; float scale; } EgNorm;
typedef struct { float *x; const float *table; unsigned n, heads, d; } EgRope;
typedef struct { float *out; const float *q, *k, *v; const unsigned *bounds; unsigned n, window; } EgAttention;
typedef struct { float *out; const float *x, *other; unsigned n, mode, layer; float scale; } EgElement;
typedef struct { float *out; const float *x; const unsigned *offsets; unsigned batch; } EgPool;
typedef struct { float *out; const float *x, *weight; unsigned rows, d; float scale; } EgNormResidual;
typedef struct { float *x; const float *weight, *table; unsigned rows, d, heads; } EgNormRope;
#endif
