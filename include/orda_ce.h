/*
 * orda_ce.h -- C ABI of liborda_ce.so, the MI355X (gfx950) implementation of
 * the fused LM-head cross-entropy + knowledge-distillation loss.
 *
 * The reference (orda_ce_kernel, Python + Triton) has no native library; its
 * hot path is the chunk loop inside the three autograd Functions.  Each entry
 * point below replaces one piece of that loop, named in its comment as
 * reference-file:line (paths relative to the reference's src/orda_ce_kernel/).
 *
 * Conventions
 *   - Every pointer is a device pointer unless stated otherwise.  The library
 *     never allocates or frees device memory: the caller (PyTorch) owns every
 *     input, output, saved and workspace buffer.
 *   - All matrices are dense row-major with the leading dimension equal to
 *     the row length (the Python layer calls .contiguous() first, as the
 *     reference does at ops/tied_teacher.py:334-339).
 *   - Launches are asynchronous on the given stream; nothing synchronises the
 *     host.  Calls on different streams may run concurrently if they use
 *     different workspace buffers.
 *   - Return value: 0 on success, a negative ORDA_E* code otherwise; the
 *     message is available from orda_last_error() (thread-local).
 */
#ifndef ORDA_CE_H
#define ORDA_CE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORDA_ABI_VERSION 4

/* Teacher modes (reference api.py:21-52, ops/separate_teacher.py:1102). */
enum orda_mode {
  ORDA_MODE_TIED = 0,               /* student and teacher share W          */
  ORDA_MODE_SEPARATE = 1,           /* teacher (hidden_t, W_t)              */
  ORDA_MODE_PRECOMPUTED_LOGITS = 2, /* teacher logits [N x V] given         */
  ORDA_MODE_PRECOMPUTED_HIDDEN = 3, /* frozen (hidden_t, W_t), no grads     */
  ORDA_MODE_TOPK = 4                /* teacher as k (id, log-prob) pairs per
                                       row, renormalised over its ids; no
                                       counterpart in the reference (its
                                       precomputed teacher is [N x V] logits,
                                       ops/precomputed_teacher.py:336-356)   */
};

/* Element types. */
enum orda_dtype { ORDA_BF16 = 0, ORDA_F16 = 1, ORDA_F32 = 2 };

/* Divergences for the distillation term.  ORDA_DIV_FORWARD_KL is the only one
 * the reference has (ops/tied_teacher.py:182,189); the others are additions
 * selected by a keyword whose default keeps forward KL. */
enum orda_divergence {
  ORDA_DIV_FORWARD_KL = 0,
  ORDA_DIV_REVERSE_KL = 1,
  ORDA_DIV_SYMMETRIC_KL = 2,
  ORDA_DIV_SOFT_TARGET_CE = 3,
  ORDA_DIV_HELLINGER = 4,
  ORDA_DIV_BHATTACHARYYA = 5,
  ORDA_DIV_RENYI = 6,
  ORDA_DIV_AMARI_ALPHA = 7,
  ORDA_DIV_CHI_SQUARED = 8,
  ORDA_DIV_SQUARED_L2 = 9,
  ORDA_DIV_AB = 10,
  ORDA_DIV_JSD = 11,
  ORDA_DIV_SKEW_FORWARD_KL = 12,
  ORDA_DIV_SKEW_REVERSE_KL = 13,
  ORDA_DIV_TVD = 14,
  ORDA_DIV_COUNT = 15
};

/* Problem flags. */
#define ORDA_NEED_GRAD_STUDENT_HIDDEN (1u << 0)
#define ORDA_NEED_GRAD_WEIGHT (1u << 1)
#define ORDA_NEED_GRAD_TEACHER_HIDDEN (1u << 2)
#define ORDA_NEED_GRAD_TEACHER_WEIGHT (1u << 3)
#define ORDA_COMPUTE_TEACHER_CE (1u << 4) /* teacher CE value (and its grads) */
#define ORDA_COMPUTE_DIVERGENCE (1u << 5) /* kl_weight != 0                  */
#define ORDA_REDUCTION_SUM (1u << 6)      /* else mean                        */
/* Compute the requested gradients inside orda_forward, one token chunk at a
 * time, as the reference's Functions do (ops/tied_teacher.py:366-516): the
 * chunk's logits are materialised in the workspace (vocabulary-major), turned
 * into dlogits in place, and multiplied into the gradients; grad W is
 * accumulated across chunks in the weight dtype (the reference's default,
 * fp32_grad_weight_accumulation=False, ops/tied_teacher.py:354,488-495).
 * orda_backward then only multiplies the gradients by grad_output
 * (ops/tied_teacher.py:531-564).  Every mode (a precomputed teacher's logits
 * are stored beside the student's in the compute dtype) and every divergence
 * (the two-pass ones, JSD, skew KLs and TVD, take their second pass over the
 * chunk's stored logits). */
#define ORDA_GRADS_IN_FORWARD (1u << 7)
/* The student's final RMSNorm fused in front of the loss (no counterpart in
 * the reference's loss API; its producer applies the norm before calling the
 * loss, test/benchmark/src/core.py:7-14,135): student_hidden is the norm's
 * input x, and the loss is taken on
 *   y = x * rsqrt(mean_j x_j^2 + norm_eps) * student_norm_weight
 * (mean over the first norm_dim columns; y rounded to the compute dtype).
 * grad_student_hidden is then dloss/dx, and with
 * ORDA_NEED_GRAD_STUDENT_NORM_WEIGHT grad_student_norm_weight is
 * dloss/dnorm_weight.  Needs ORDA_GRADS_IN_FORWARD. */
#define ORDA_STUDENT_RMSNORM (1u << 8)
#define ORDA_NEED_GRAD_STUDENT_NORM_WEIGHT (1u << 9)
/* The scan's logits GEMM on gfx950's fp8 MFMA (no counterpart in the
 * reference; its logits GEMM is a bf16 torch.mm, ops/tied_teacher.py:444-445):
 * W and the chunk's hidden rows are rounded to OCP e4m3 with one
 * power-of-two scale per row (v_mfma_scale_f32_32x32x64_f8f6f4 applies the
 * scales), and the logits (values, softmax statistics, dlogits) come from
 * those products; the gradient GEMMs stay in the compute dtype.  Needs
 * ORDA_GRADS_IN_FORWARD, a 16-bit compute dtype, hidden a multiple of 16 and
 * > 128, and a tied teacher, precomputed logits read in place (ORDA_DIV
 * families other than the power family) or no teacher term.  Accuracy: see
 * the library's documentation of the flag (losses within ~1e-2 relative of
 * the exact values at the headline shape). */
#define ORDA_FP8_LOGITS (1u << 10)

/* Error codes. */
#define ORDA_OK 0
#define ORDA_EINVAL (-1)
#define ORDA_EWORKSPACE (-2)
#define ORDA_ELAUNCH (-3)
#define ORDA_EUNSUPPORTED (-4)

/* Shapes, dtypes and scalar arguments of one loss evaluation. */
typedef struct orda_problem {
  int32_t abi_version;    /* must equal ORDA_ABI_VERSION                      */
  int32_t mode;           /* enum orda_mode                                   */
  int32_t dtype;          /* compute dtype of hidden states and weights       */
  int32_t logits_dtype;   /* dtype of teacher logits (PRECOMPUTED_LOGITS)     */
  int64_t n_rows;         /* N = batch x sequence                             */
  int64_t vocab;          /* V                                                */
  int64_t hidden;         /* H of the student                                 */
  int64_t teacher_hidden; /* H of the teacher (== hidden for TIED)            */
  int64_t ignore_index;
  int64_t vocab_chunk;    /* V columns per backward chunk; 0 = library choice */
  uint32_t flags;         /* ORDA_* flags above                               */
  int32_t divergence;     /* enum orda_divergence                             */
  float temperature;      /* > 0                                              */
  float student_ce_weight;
  float teacher_ce_weight;
  float kl_weight;
  float div_alpha;        /* alpha of renyi, amari_alpha, ab, skew_*_kl       */
  float div_beta;         /* beta of jsd and ab                               */
  int32_t grad_hidden_splits; /* ORDA_GRADS_IN_FORWARD: split-K count of the
                             grad-hidden GEMM (contraction over V), 1..64;
                             0 = the gfx950 launch table (rule-based for
                             shapes it does not list).  Raised when needed
                             so each split's K range of its MN-major operands
                             stays below 2^31 bytes (one buffer resource)  */
  int64_t token_chunk;    /* ORDA_GRADS_IN_FORWARD: requested tokens per
                             chunk, the reference's chunk_size; the library's
                             chunk is this times the launch table's
                             chunk_scale (2; 4 when precomputed logits are
                             read in place), at most 2^21 tokens.
                             0 = library choice (chunk logits <= 512 MiB)     */
  int64_t topk;           /* ORDA_MODE_TOPK: ids per row (1 <= topk <= V);
                             the mode needs ORDA_GRADS_IN_FORWARD (with or
                             without gradients), teacher CE off and the
                             divergence ORDA_DIV_FORWARD_KL or
                             ORDA_DIV_SOFT_TARGET_CE                          */
  int64_t norm_dim;       /* ORDA_STUDENT_RMSNORM: columns the mean of x^2
                             runs over (the unpadded hidden size,
                             1 <= norm_dim <= hidden; 0 = hidden); columns
                             past it must be zero in x                        */
  float norm_eps;         /* ORDA_STUDENT_RMSNORM: >= 0                       */
} orda_problem_t;

/* Tensors of one loss evaluation.  Unused pointers may be NULL. */
typedef struct orda_tensors {
  const void* student_hidden;  /* [N x H]   dtype                            */
  const void* weight;          /* [V x H]   dtype                            */
  const void* teacher_hidden;  /* [N x Ht]  dtype (TIED: Ht == H)            */
  const void* teacher_weight;  /* [V x Ht]  dtype (SEPARATE / PRE_HIDDEN)    */
  const void* teacher_logits;  /* [N x V]   logits_dtype (PRE_LOGITS); with
                                * ORDA_GRADS_IN_FORWARD, a 16-bit compute dtype
                                * and V a multiple of 8 they are read in place
                                * and must be 16-byte aligned (else
                                * ORDA_EINVAL); logits of another dtype than
                                * the compute dtype are used rounded to it
                                * (ops/precomputed_teacher.py:343-348)        */
  const int64_t* labels;       /* [N]                                        */
  /* forward outputs: fp32 scalars */
  float* out_loss;
  float* out_student_ce;
  float* out_teacher_ce;
  float* out_kl;
  /* state kept from forward to backward: orda_saved_bytes() bytes          */
  void* saved;
  /* backward inputs / outputs */
  const float* grad_output;      /* fp32 scalar, d(total)/d(loss)           */
  void* grad_student_hidden;     /* [N x H]  dtype                          */
  void* grad_weight;             /* [V x H]  dtype                          */
  void* grad_teacher_hidden;     /* [N x Ht] dtype                          */
  void* grad_teacher_weight;     /* [V x Ht] dtype                          */
  /* ORDA_MODE_TOPK: per row, topk distinct vocabulary ids in [0, V) and the
   * teacher's log-probabilities there (temperature 1)                        */
  const int64_t* teacher_topk_indices; /* [N x topk]                          */
  const float* teacher_topk_logprobs;  /* [N x topk] fp32                     */
  /* ORDA_STUDENT_RMSNORM                                                     */
  const void* student_norm_weight;     /* [H] dtype                           */
  void* grad_student_norm_weight;      /* [H] dtype                           */
} orda_tensors_t;

/* ABI version of the loaded library (ORDA_ABI_VERSION). */
int orda_abi_version(void);

/* Message of the last failed call on this host thread ("" if none). */
const char* orda_last_error(void);

/* Bytes of the buffer that carries per-row statistics from orda_forward to
 * orda_backward.  Replaces the tensors saved by ctx.save_for_backward at
 * ops/tied_teacher.py:519 (and separate_teacher.py:696,971,
 * precomputed_teacher.py:478); this build saves O(N) statistics instead of
 * full gradients. */
size_t orda_saved_bytes(const orda_problem_t* p);

/* Scratch bytes orda_forward needs.  Replaces the per-chunk logits and loss
 * buffers of ops/tied_teacher.py:356-358,444-445. */
size_t orda_forward_workspace_bytes(const orda_problem_t* p);

/* Scratch bytes orda_backward needs for p->vocab_chunk (0: library choice).
 * Bounded by O(vocab_chunk x N + N x H): no [N x V] tensor is ever formed. */
size_t orda_backward_workspace_bytes(const orda_problem_t* p);

/* The launch plan orda_forward would use for p (host-side, no device work).
 * Replaces the reference's launch-config lookup (utils/_autotune.py:94-106
 * default_config, :255-340 select_config): the fixed gfx950 table of
 * launch_table.hpp for measured shapes, a rule for others. */
typedef struct orda_plan_info {
  int32_t grads_in_forward;      /* 1: gradients-in-forward schedule          */
  int32_t table_entry;           /* launch-table row used, -1 = rule          */
  int32_t teacher_class;         /* 0 tied, 1 staged, 2 in place, 3 other     */
  int32_t scan_engine;           /* 0 two-stage (8 waves), 1 ring (4 waves)   */
  int64_t token_chunk;           /* tokens per chunk                          */
  int64_t n_token_chunks;
  int32_t chunk_scale;           /* token_chunk / requested chunk             */
  int32_t scan_tokens_per_tile;  /* tokens of one scan workgroup tile         */
  int32_t scan_workgroups;       /* workgroups of one chunk's scan            */
  int32_t grad_hidden_splits;    /* student grad hidden split-K               */
  int32_t grad_teacher_hidden_splits;
  int32_t reserved;
  int64_t vocab_rows_per_split;  /* K rows of one grad-hidden split           */
  int64_t vocab_chunk;           /* two-phase backward vocabulary chunk       */
  uint64_t forward_workspace_bytes;
  uint64_t backward_workspace_bytes;
} orda_plan_info_t;

int orda_plan_info(const orda_problem_t* p, orda_plan_info_t* out);

/* Forward: losses and per-row statistics.  Replaces the chunk loop of
 * TiedCEFunction.forward (ops/tied_teacher.py:366-516),
 * SeparateStudentCEFunction.forward (ops/separate_teacher.py:568-693),
 * SeparateFullCEFunction.forward (ops/separate_teacher.py:828-968) and
 * PrecomputedCEFunction.forward (ops/precomputed_teacher.py:358-475): the
 * logits GEMMs (tied_teacher.py:444-445), the Triton row kernels
 * (tied_teacher.py:13-189) and the loss reduction (tied_teacher.py:499-516).
 * Writes out_loss/out_student_ce/out_teacher_ce/out_kl and `saved`.  With
 * ORDA_GRADS_IN_FORWARD it also writes every requested gradient (the grad_*
 * pointers of t), scaled by the mean scale but not yet by grad_output. */
int orda_forward(const orda_problem_t* p, const orda_tensors_t* t,
                 void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the static scratch behind orda_forward_static (64 MiB). */
#define ORDA_STATIC_SCRATCH_BYTES (64ull << 20)

/* orda_forward without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference, whose
 * Functions allocate their chunk buffers with torch (ops/tied_teacher.py:
 * 356-358).  The scratch is a file-scope device array of
 * ORDA_STATIC_SCRATCH_BYTES on each device the library runs on, held until
 * the process ends; this entry point calls no hipMalloc/hipFree.  Problems
 * whose orda_forward_workspace_bytes() exceed it are rejected with
 * ORDA_EWORKSPACE (a smaller token_chunk shrinks the gradients-in-forward
 * workspace: at V = 128256, H = 4096 a 64-token chunk fits).  Every call on a
 * device shares that device's scratch: calls that overlap on one device
 * (different streams, different host threads) race and must be serialised by
 * the caller.  The stream must belong to the current device.  Same outputs
 * as orda_forward. */
int orda_forward_static(const orda_problem_t* p, const orda_tensors_t* t, void* stream);

/* Backward: all requested gradients, already multiplied by
 * grad_output * mean_scale.  Replaces the gradient GEMMs computed inside
 * forward (ops/tied_teacher.py:468-495, separate_teacher.py:660-674,
 * 919-948, precomputed_teacher.py:443-457) and the scaling in backward
 * (ops/tied_teacher.py:531-564 and analogues).  Reads `saved` from the
 * matching orda_forward call.  With ORDA_GRADS_IN_FORWARD it only multiplies
 * the gradients orda_forward wrote by grad_output, in place (no workspace). */
int orda_backward(const orda_problem_t* p, const orda_tensors_t* t,
                  void* workspace, size_t workspace_bytes, void* stream);

/* grad *= factor[0] in place (numel elements of `dtype`, 16-byte aligned;
 * factor a device fp32 scalar, read on the device, so the host does not
 * synchronise; factor == 1 leaves grad untouched).  Replaces the
 * multiplication of the cached gradients by grad_output * mean_scale in
 * TiedCEFunction.backward (ops/tied_teacher.py:538-545, which allocates new
 * tensors) for callers that hold gradients from an ORDA_GRADS_IN_FORWARD
 * forward without its problem description: the torch.compile-friendly
 * custom op's backward. */
int orda_scale_gradient(int32_t dtype, void* grad, int64_t numel, const float* factor, void* stream);

/* Plain C = A * B^T with A [M x K], B [N x K] (both K-contiguous) and C
 * [M x N] in `dtype`, fp32 accumulation (the engine behind every GEMM of the
 * path).  Exposed for tests and for callers that want the MFMA engine alone;
 * replaces nothing in the reference directly (it stands for the torch
 * matmuls at ops/tied_teacher.py:445,473,493). */
int orda_gemm_abt(int32_t dtype, int64_t M, int64_t N, int64_t K,
                  const void* A, const void* B, void* C, void* stream);

/* General C = op(A) * op(B)^T in `dtype` with fp32 accumulation: a_mn = 0
 * means A is [M x K] K-contiguous (leading dimension lda), a_mn = 1 means A
 * is stored [K x M] (element (m, k) at A[k * lda + m]); likewise b_mn for B
 * ([N x K] or [K x N]).  C is [M x N] with leading dimension ldc.  splits > 1
 * splits K into that many fp32 partials summed in a fixed order; the
 * workspace must then hold splits * M * N floats (else it may be NULL).
 * Exposed for tests and callers that want the engine; it stands for the
 * torch matmuls of ops/tied_teacher.py:445,473,493, whose operands the
 * materialised path reads in both layouts. */
int orda_gemm(int32_t dtype, int32_t a_mn, int32_t b_mn, int64_t M, int64_t N, int64_t K, const void* A,
              int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int32_t splits, void* workspace,
              size_t workspace_bytes, void* stream);

/* Per-kernel-class timing, for benchmarks.  No counterpart in the reference,
 * whose benchmarks bracket whole steps with torch.cuda.Event
 * (test/benchmark/src/_train.py:410-419); this hook brackets each launch
 * inside the library with hipEvents on the launch stream.  Off by default;
 * the state is process-wide (backward may run on another host thread). */
enum orda_kernel_class {
  ORDA_K_SCAN = 0,      /* forward logits GEMM + online-softmax statistics */
  ORDA_K_ROWS = 1,      /* label logits, per-row merge, loss reduction     */
  ORDA_K_DLOGITS = 2,   /* backward logits recompute + dlogits epilogue    */
  ORDA_K_GEMM_W = 3,    /* grad_weight GEMMs                               */
  ORDA_K_GEMM_H = 4,    /* grad_hidden GEMMs                               */
  ORDA_K_AUX = 5,       /* transposes and fills                            */
  ORDA_K_COUNT = 6
};

typedef struct orda_timing {
  int32_t launches[ORDA_K_COUNT];
  double milliseconds[ORDA_K_COUNT];    /* summed kernel time per class   */
  double algorithmic_flops[ORDA_K_COUNT]; /* GEMM flops that count (no recompute) */
  double executed_flops[ORDA_K_COUNT];  /* GEMM flops issued to MFMA     */
} orda_timing_t;

/* Start (enable != 0) or stop recording; starting clears previous records. */
int orda_timing_enable(int enable);

/* Wait for the recorded events, fill *out with the sums since the last
 * enable/collect, and clear the records. */
int orda_timing_collect(orda_timing_t* out);

#ifdef __cplusplus
}
#endif

#endif /* ORDA_CE_H */
