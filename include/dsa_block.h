/*
 * dsa_block.h — C ABI of the fused row kernels around the attention in
 * libdsa.so: the blocks the reference runs right before and after
 * DisentangledSelfAttention, as HBM-bound HIP kernels (the matrix products
 * between them stay plain hipBLASLt GEMMs, run by the caller):
 *
 *   add + LayerNorm   y = LayerNorm(x + bias + res) * gamma + beta
 *       DebertaV2SelfOutput / DebertaV2Output (_apply_output_residual_norm,
 *       src/deberta/modeling/deberta_v2_native.py:115-165, 733-758: dense
 *       without its bias, then bias + residual + LayerNorm here); the
 *       encoder's LayerNorm of the shared relative-embedding table
 *       (get_rel_embedding, :1036-1047: no bias, no residual); the RTD
 *       head's LayerNorm(hidden + hidden[:, 0]) (src/deberta/modeling/
 *       rtd.py:612-624: a residual read with row stride 0 per batch row).
 *   bias + GELU       y = gelu(x + bias), erf form
 *       DebertaV2Intermediate (:703-730, hidden_act "gelu") and the RTD
 *       head's dense + activation (rtd.py:622-623).
 *   RTD loss          logits = x . w + b;  loss = sum(active * BCE(logits,
 *       labels)) / max(sum(active), 1)
 *       the RTD classifier (rtd.py:624) and the discriminator loss
 *       (rtd.py:1134-1139).
 *
 * Conventions are those of dsa.h: the caller owns every buffer (the
 * backward's column-sum workspace included, sized by
 * dsa_block_workspace_bytes), work goes on the caller's stream, a nonzero
 * return carries a message in dsa_last_error().  Rows hold C contiguous
 * elements; a row stride is given per tensor.  Element types are DSA_F32
 * or DSA_BF16 per tensor; arithmetic is fp32.  Column sums (the parameter
 * gradients) are reduced in a fixed order: results are reproducible.
 */
#ifndef DSA_BLOCK_H_
#define DSA_BLOCK_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Workspace kinds for dsa_block_workspace_bytes. */
enum { DSA_BLOCK_LN = 0, DSA_BLOCK_GELU = 1, DSA_BLOCK_RTD = 2 };

typedef struct dsa_ln_args {
  /* forward inputs */
  const void* x;              /* [N, C], row stride x_stride */
  const void* bias;           /* [C] added to x, or NULL */
  const void* res;            /* residual or NULL: row r = g * rows_per_group + s at
                                 res + g * res_strides[0] + s * res_strides[1] */
  const void* gamma;          /* [C] */
  const void* beta;           /* [C] */
  int64_t x_stride;
  int64_t res_strides[2];
  int64_t rows_per_group;     /* > 0 when res is given */
  /* forward outputs */
  void* y;                    /* [N, C], row stride y_stride */
  int64_t y_stride;
  float* mean;                /* [N] */
  float* rstd;                /* [N]: 1 / sqrt(var + eps) */
  /* backward (reads x, bias, res, gamma, mean, rstd as saved) */
  const void* dy;             /* [N, C], row stride dy_stride */
  int64_t dy_stride;
  void* dz;                   /* [N, C] gradient of x + bias + res, row stride dz_stride, x's dtype */
  int64_t dz_stride;
  void* dgamma;               /* [C] or NULL, written */
  void* dbeta;                /* [C] or NULL, written */
  void* dbias;                /* [C] or NULL, written (the column sums of dz) */
  void* workspace;            /* dsa_block_workspace_bytes(DSA_BLOCK_LN, N, C) bytes */
  size_t workspace_bytes;
  int64_t N;
  int32_t C;                  /* a multiple of 4, at most 2048 */
  int32_t x_dtype, res_dtype, y_dtype, dy_dtype, dz_dtype;
  int32_t param_dtype;        /* bias, gamma, beta and their gradients */
  float eps;
} dsa_ln_args;

typedef struct dsa_gelu_args {
  const void* x;              /* [N, C], row stride x_stride */
  const void* bias;           /* [C] or NULL */
  void* y;                    /* [N, C], row stride y_stride */
  const void* dy;             /* backward: [N, C], row stride dy_stride */
  void* dz;                   /* backward: [N, C] gradient of x + bias, row stride dz_stride, x's dtype */
  void* dbias;                /* backward: [C] or NULL, written */
  int64_t x_stride, y_stride, dy_stride, dz_stride;
  void* workspace;            /* dsa_block_workspace_bytes(DSA_BLOCK_GELU, N, C) bytes */
  size_t workspace_bytes;
  int64_t N;
  int32_t C;                  /* a multiple of 4 */
  int32_t x_dtype, y_dtype, dy_dtype, dz_dtype, param_dtype;
} dsa_gelu_args;

typedef struct dsa_rtd_args {
  const void* x;              /* [N, C] classifier input, row stride x_stride */
  const void* w;              /* [C] classifier weight */
  const void* b;              /* [1] classifier bias, or NULL */
  const float* labels;        /* [N] replaced-token labels (0 / 1) */
  const uint8_t* active;      /* [N] or NULL (every token active) */
  int64_t x_stride;
  float* logits;              /* [N] forward output */
  float* loss;                /* [1] forward output */
  float* denom;               /* [1] forward output: max(sum(active), 1) */
  const float* dloss;         /* backward: [1] */
  void* dx;                   /* backward: [N, C], row stride dx_stride */
  int64_t dx_stride;
  void* dw;                   /* backward: [C], written */
  void* db;                   /* backward: [1] or NULL, written */
  void* workspace;            /* dsa_block_workspace_bytes(DSA_BLOCK_RTD, N, C) bytes */
  size_t workspace_bytes;
  int64_t N;
  int32_t C;                  /* a multiple of 4, at most 2048 */
  int32_t x_dtype, dx_dtype, param_dtype;
} dsa_rtd_args;

/* Workspace bytes of a backward (LN, GELU) or of the RTD forward and
 * backward (the same buffer serves both). */
size_t dsa_block_workspace_bytes(int kind, int64_t N, int32_t C);

/* y, mean, rstd from x, bias, res, gamma, beta. */
int dsa_add_ln_fwd(const dsa_ln_args* args, void* stream);
/* dz, dgamma, dbeta, dbias from dy and the forward's inputs and statistics. */
int dsa_add_ln_bwd(const dsa_ln_args* args, void* stream);

/* y = gelu(x + bias). */
int dsa_bias_gelu_fwd(const dsa_gelu_args* args, void* stream);
/* dz = dy * gelu'(x + bias), dbias = column sums of dz. */
int dsa_bias_gelu_bwd(const dsa_gelu_args* args, void* stream);

/* logits, loss and denom. */
int dsa_rtd_loss_fwd(const dsa_rtd_args* args, void* stream);
/* dx, dw, db from dloss (the forward's logits and denom are read). */
int dsa_rtd_loss_bwd(const dsa_rtd_args* args, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DSA_BLOCK_H_ */
