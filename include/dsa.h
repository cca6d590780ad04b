/*
 * dsa.h — C ABI of the fused disentangled self-attention library (libdsa.so).
 *
 * The library replaces the eager ATen op chain of the reference's
 * DisentangledSelfAttention (pszemraj/deberta):
 *   forward   src/deberta/modeling/deberta_v2_native.py:564-652
 *   bias      src/deberta/modeling/deberta_v2_native.py:349-562 (c2p/p2c terms)
 *   rel ids   src/deberta/modeling/deberta_v2_native.py:51-112, 235-271
 *   mask      src/deberta/modeling/mask_utils.py:8-32
 * and the autograd graph ATen records for it (the reference has no custom
 * backward).  The reference is pure Python, so there is no FFI in it to bind
 * to: the caller of these entry points is the torch.library custom op in
 * deberta_amd/ops.py (via ctypes), which keeps the reference's Python call
 * surface.
 *
 * Conventions
 *   - Ownership: the caller allocates and owns every buffer.  The library
 *     never allocates or frees device memory and keeps no tensor state.
 *   - Streams: all work is enqueued on `stream` (hipStream_t passed as void*),
 *     with no implicit device synchronisation.  Calls are re-entrant.
 *   - Errors: a nonzero return code means nothing was launched (argument
 *     error) or the launch failed; dsa_last_error() returns a thread-local
 *     message describing it.
 *   - Layouts: q/k/v/out/dq/dk/dv are [B, L, H, D] with element strides
 *     (b, l, h) given explicitly and the D axis contiguous (stride 1).  This is
 *     the natural view of a Linear output [B, L, H*D], so no permute copies
 *     are needed.  kr/qr (projected relative tables) are [H, R, D] with
 *     strides (h, r) and D contiguous; R = 2*att_span.
 *   - Relative positions: `rel_table` holds the (already bucketed) relative
 *     position of every query/key offset, rel_table[(i - j) + (Lk - 1)] for
 *     i - j in [-(Lk-1), Lq-1]: the reference's relative_pos matrix is a
 *     Toeplitz matrix (it depends on i - j only), and this is its first
 *     column and row.  The kernels derive the c2p row clamp(clamp(t,-A,A)+A,
 *     0, 2A-1) and the p2c row clamp(-clamp(t,-A,A)+A, 0, 2A-1) in registers
 *     (deberta_v2_native.py:377, 395, 407).
 *   - Masks: key_keep is a [B, Lk] byte mask (nonzero = keep) for the
 *     reference's broadcast (B,1,1,S) keep mask; pair_keep is a [B, Lq, Lk]
 *     byte mask for the pairwise (B,1,S,S) form, or [B, H, Lq, Lk] for a
 *     per-head (B,H,S,S) mask (pair_keep_stride_h).  At most one may be
 *     given.
 *     A zero batch stride broadcasts one mask over the batch.  Query liveness
 *     follows the reference (deberta_v2_native.py:625-639): key_keep[b,i]
 *     for the broadcast form, pair_keep[b,i,i] for the pairwise form; dead
 *     query rows produce exactly zero output and zero gradient.
 *     seg is a compact form of block-diagonal masks: an int32 [B, L]
 *     segment id per token (Lq == Lk), 0 for an inactive token.  Pair
 *     (i, j) is kept iff seg[b,i] != 0 and seg[b,i] == seg[b,j]; a query
 *     with seg 0 is a dead row.  With seg = document ids this is the
 *     reference's packed-document mask (training/compile.py:310-349, whose
 *     pad queries are dead rows); key_keep is the case seg = keep ? 1 : 0.
 *     The kernels skip tiles whose query and key segments cannot meet.
 *     At most one of key_keep, pair_keep and seg may be given.
 */
#ifndef DSA_H_
#define DSA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element types */
enum { DSA_F32 = 0, DSA_BF16 = 1 };

/* score terms (deberta_v2_native.py:592-598, pos_att_type) */
enum { DSA_C2P = 1, DSA_P2C = 2 };

/* backward stages, for dsa_bwd_args.stages (0 means all).  They run in the
 * order PREP, DKDV, DQ, FOLD and pass data through the workspace:
 *   PREP  rowsum(dO * O) and the relative tables gathered per offset
 *   DKDV  writes dv, dk and dS^T (into the workspace)
 *   DQ    writes dq from dS^T
 *   FOLD  adds the relative-table gradients (from dS^T) into dkr / dqr;
 *         it is TABLE (the per-offset sums, kept in the workspace) followed
 *         by SUM (their fold onto table rows, written to dkr / dqr), which
 *         may also be requested on their own, in that order
 * DQ and FOLD (or DQ and TABLE) requested in one call run their main
 * kernels as one launch.  Stages run in separate calls must keep this
 * order and share one workspace.  (Version 8: TABLE and SUM.) */
enum {
  DSA_STAGE_PREP = 1,
  DSA_STAGE_DQ = 2,
  DSA_STAGE_DKDV = 4,
  DSA_STAGE_FOLD = 8,
  DSA_STAGE_TABLE = 16,
  DSA_STAGE_SUM = 32
};

typedef struct dsa_fwd_args {
  const void* q;          /* [B, Lq, H, D] */
  const void* k;          /* [B, Lk, H, D] */
  const void* v;          /* [B, Lk, H, D] */
  const void* kr;         /* [H, R, D] pos-key table (c2p), NULL if !C2P */
  const void* qr;         /* [H, R, D] pos-query table (p2c), NULL if !P2C */
  const int32_t* rel_table; /* [Lq + Lk - 1], required when flags != 0 */
  const uint8_t* key_keep;  /* [B, Lk] or NULL */
  const uint8_t* pair_keep; /* [B, Lq, Lk] or NULL */
  void* out;              /* [B, Lq, H, D], same dtype as q */
  float* lse;             /* [B, H, Lq] contiguous, natural-log logsumexp */
  void* bias;             /* optional [B, H, round_up(Lq, 128), round_up(Lk, 128)]
                             contiguous: the relative score term c2p + p2c
                             (unscaled; fp16 for bf16 inputs, fp32 for fp32),
                             written for dsa_bwd.  NULL: not written. */
  int64_t q_strides[3];   /* element strides of b, l, h */
  int64_t k_strides[3];
  int64_t v_strides[3];
  int64_t o_strides[3];
  int64_t kr_strides[2];  /* element strides of h, r */
  int64_t qr_strides[2];
  int64_t key_keep_stride_b;
  int64_t pair_keep_strides[2]; /* b, q (k contiguous); pair_keep 16-byte aligned,
                                   both strides multiples of 16, each row's
                                   allocation reaching round_up(Lk, 16) bytes
                                   (read in 16-byte chunks) */
  int32_t B, H, Lq, Lk, D;
  int32_t att_span;       /* A; R = 2A rows in kr/qr */
  int32_t dtype;          /* DSA_F32 or DSA_BF16 */
  int32_t flags;          /* DSA_C2P | DSA_P2C */
  float scale;            /* 1/sqrt(D * scale_factor) */
  const int32_t* seg;     /* [B, L] segment ids or NULL (see Masks above) */
  int64_t seg_stride_b;
  /* Optional scratch of dsa_fwd_workspace_bytes(args) bytes (16-byte
     aligned), for two things: under key_keep or seg, the forward launches
     its workgroups heaviest first (a small cost and sort pass before the
     kernel); with c2p / p2c, it reads a copy of kr / qr laid out by 64-byte
     k-steps (one small copy kernel), whose row gathers touch half as many
     cache lines.  NULL (or a scratch of only the launch order's bytes): the
     default order and the caller's tables, same results.  Ignored by
     dsa_bwd, which has its own workspace. */
  void* workspace;
  size_t workspace_bytes;
  /* Optional [B, Lq, H, D] (element strides qc_strides, D contiguous): the
     query rows of the c2p term, which then reads qc_i . Kr[c(i-j)] instead
     of q_i . Kr[c(i-j)]; NULL means q.  The position-to-position term
     (p2p, deberta_v2_native.py:298-347: Qr[A + min(i, A-1)] . Kr[c(i-j)],
     the same Kr rows as c2p) is carried this way: qc = q + Qr[A + min(i,
     A-1)] with c2p and p2p, qc = Qr[A + min(i, A-1)] with p2p alone (flags
     then hold DSA_C2P).  The saved relative term holds the c2p term of qc. */
  const void* qc;
  int64_t qc_strides[3];
  /* Head stride of pair_keep (a multiple of 16): a per-head [B, H, Lq, Lk]
     pairwise mask, the reference's (B, H, S, S) keep mask; 0 broadcasts one
     [B, Lq, Lk] mask over the heads.  Query liveness is then per head:
     pair_keep[b, h, i, i]. */
  int64_t pair_keep_stride_h;
  /* Attention dropout on the probabilities (deberta_v2_native.py:222, 636:
     probs = dropout(probs), the reference's nn.Dropout in training).
     dropout_threshold t in [0, 65535], in units of 1/65536: each (query,
     key) probability is dropped with probability t / 65536 and the kept
     ones are scaled by 65536 / (65536 - t); 0 turns dropout off.  The keep
     bits are a function of (b, h, i, j) and dropout_seed (Philox4x32-10;
     the counter layout is stated in deberta_amd/csrc/dsa_dropout.h), so
     dsa_bwd, given the same arguments, reproduces the forward's mask.  The
     logsumexp (lse) is that of the probabilities before dropout.
     dsa_fwd_static refuses dropout and dsa_bias ignores it.  (Version 9.) */
  uint32_t dropout_threshold;
  uint64_t dropout_seed;
  /* Optional keep bits of the call, dsa_fwd_dropout_bytes(args) bytes,
     16-byte aligned: dsa_fwd writes them here and dsa_bwd (given the same
     pointer) reads them, so the backward generates nothing.  NULL: dsa_fwd
     keeps them in its workspace (dsa_fwd_workspace_bytes then counts them;
     a dropout call without that workspace is refused) and dsa_bwd
     regenerates them from the seed in its own (dsa_bwd_workspace_bytes
     counts them).  (Version 10.) */
  void* dropout_bits;
  /* Optional, bf16 only: O's rounding residual, bf16(o - bf16(o)) for
     every output element, written by dsa_fwd with out's strides (an
     allocation of out's extent, 16-byte aligned).  dsa_bwd, given the same
     pointer, takes the row sums dO . O of its preparation on bf16(o) plus
     the residual instead of bf16(o) alone.  Rounding O to bf16 otherwise
     offsets every dS element of a row alike (dS = P (dP - dO . O)), and a
     table gradient that sums nearly all pairs of a row onto one table row
     (few keys against many queries, narrow log buckets) keeps that offset
     where the other sums cancel it.  NULL: no residual; ignored for fp32.
     (Version 11.) */
  void* out_lo;
} dsa_fwd_args;

typedef struct dsa_bwd_args {
  /* forward inputs, exactly as passed to dsa_fwd */
  dsa_fwd_args fwd;
  const void* dout;       /* [B, Lq, H, D] upstream gradient */
  int64_t do_strides[3];
  /* outputs; gradient strides follow the [B, L, H, D] convention */
  void* dq;               /* [B, Lq, H, D], dtype of q */
  void* dk;               /* [B, Lk, H, D] */
  void* dv;               /* [B, Lk, H, D] */
  int64_t dq_strides[3];
  int64_t dk_strides[3];
  int64_t dv_strides[3];
  void* dkr;              /* [H, R, D] contiguous; NULL if !C2P */
  void* dqr;              /* [H, R, D] contiguous; NULL if !P2C */
  /* workspace: dsa_bwd_workspace_bytes() bytes, caller-allocated, in
     ordinary (coarse-grained) device memory such as hipMalloc returns: the
     table-gradient accumulators in it take fp32 atomic adds, which
     fine-grained or host-coherent memory does not support reliably */
  void* workspace;
  size_t workspace_bytes;
  int32_t stages;         /* DSA_STAGE_* mask; 0 = all */
  int32_t dtab_dtype;     /* dtype of dkr / dqr: DSA_F32 (0) or DSA_BF16 */
  int32_t dtab_overwrite; /* 0: dkr / dqr are fp32 and accumulated (+=) into;
                             1: they are overwritten (=), either dtype */
  /* With fwd.qc: [B, Lq, H, D], dtype of q, the gradient of qc
     (s sum_j dS_ij Kr[c(i-j)], the c2p part of dq); dq then holds only
     s sum_j dS_ij k_j.  Unused without fwd.qc. */
  void* dqc;
  int64_t dqc_strides[3];
} dsa_bwd_args;

/* Forward: out = softmax(mask((QK^T + c2p + p2c) * scale)) V and its
 * logsumexp.  Replaces DisentangledSelfAttention.forward's score/softmax/PV
 * chain (deberta_v2_native.py:592-652). */
int dsa_fwd(const dsa_fwd_args* args, void* stream);

/* Backward of dsa_fwd: dq, dk, dv and the gradients of the projected
 * relative tables (dkr, dqr: accumulated into fp32 buffers, or written in
 * fp32 or bf16, per dtab_dtype / dtab_overwrite).  Replaces ATen autograd through deberta_v2_native.py:592-652 and
 * the einsum/bmm + gather bias path (:349-528). */
int dsa_bwd(const dsa_bwd_args* args, void* stream);

/* dsa_fwd without any caller-provided scratch: no counterpart in the
 * reference.  For callers that cannot allocate device memory (tight serving
 * loops, harnesses that forbid hipMalloc): under key_keep or seg masks the
 * heaviest-first launch order's cost and order arrays (what
 * dsa_fwd_args.workspace brings to dsa_fwd) live in a library-owned static
 * device array of DSA_FWD_STATIC_SCRATCH_BYTES per GPU, held until the
 * process ends; args->workspace is ignored.  Results equal dsa_fwd's.
 * Sizes whose order needs more than the array (B * ceil(Lq / 128) > 65536
 * items) are refused with an error.  The calls of one process on one GPU
 * share the array and are serialised: each waits on its stream for the
 * previous one (a per-device event) before it writes the array, whatever
 * stream or host thread made it; calls from other processes have their own
 * copy.  Every call writes each element it reads, so nothing carries over
 * between calls.  Call with the stream's device current.  Like every entry
 * point here it refuses a stream that is capturing a HIP graph (the
 * library's launches are not supported under capture). */
#define DSA_FWD_STATIC_SCRATCH_BYTES (512u * 1024u)
int dsa_fwd_static(const dsa_fwd_args* args, void* stream);

/* The relative score term alone, the reference's bias API
 * DisentangledSelfAttention.disentangled_attention_bias
 * (deberta_v2_native.py:530-562, dispatching to :349-432 / :434-528):
 *   out[b, h, i, j] = scale * (qc_i . Kr[c(i-j)] + k_j . Qr[p(i-j)])
 * for the terms in args->flags (qc = q unless args->qc is set; p2p rides
 * on qc as in dsa_fwd_args), zeros with no flags.  Reads q (or qc), k, kr,
 * qr, rel_table, B, H, Lq, Lk, D, att_span, dtype, flags and scale from
 * args (masks, v, out, lse, bias and workspace are ignored: the reference's
 * bias is unmasked).  out: [B, H, Lq, Lk] in the dtype of q, element
 * strides out_strides = (b, h, i) and unit stride over j, 16-byte aligned. */
int dsa_bias(const dsa_fwd_args* args, void* out, const int64_t* out_strides, void* stream);

/* Workspace bytes dsa_bwd needs for these arguments. */
size_t dsa_bwd_workspace_bytes(const dsa_bwd_args* args);

/* Bytes of dsa_fwd_args.bias for these arguments (0 without c2p / p2c).
 * No counterpart in the reference, which keeps its (B, H, L, L) relative
 * terms alive for autograd instead. */
size_t dsa_fwd_bias_bytes(const dsa_fwd_args* args);

/* Bytes of dsa_fwd_args.dropout_bits for these arguments (0 without
 * dropout).  No counterpart in the reference, whose nn.Dropout keeps its
 * mask in autograd's saved tensors. */
size_t dsa_fwd_dropout_bytes(const dsa_fwd_args* args);
/* Bytes of dsa_fwd_args.workspace for these arguments: the heaviest-first
 * launch order under key_keep or seg, then the k-step copies of kr / qr with
 * c2p / p2c (0 without either).  No counterpart in the reference, whose
 * eager path has no launch order to choose and reads its tables through
 * torch's gathers. */
size_t dsa_fwd_workspace_bytes(const dsa_fwd_args* args);

/* Thread-local description of the last error (empty string if none). */
const char* dsa_last_error(void);

/* Library version, for the loader's compatibility check. */
int dsa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DSA_H_ */
