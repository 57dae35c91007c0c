// launch.hpp -- parameter blocks and launcher declarations shared between
// the host entry points (abi.hip) and the per-dtype kernel objects.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace orda {

enum DType { DT_BF16 = 0, DT_F16 = 1, DT_F32 = 2 };

// Where a fused tile gets its teacher logits from.
enum TeacherSource {
  TSRC_NONE = 0,    // no teacher term (student CE only)
  TSRC_SHARED = 1,  // teacher hidden x the student's W (tied mode)
  TSRC_SEP = 2,     // teacher hidden x W_t (separate / precomputed hidden)
  TSRC_MEM = 3,     // precomputed logits [N x V]
  TSRC_L = 4,       // already in Lout's teacher columns (vocabulary-major; the
                    // 16-bit ring scan of the gradients-in-forward schedule)
  TSRC_MEM_RING = 5  // precomputed logits [N x V] of the compute dtype, read by
                     // the 16-bit ring scan, which also writes them to Lout's
                     // teacher columns (V a multiple of 4)
};

// GEMM epilogues: STORE writes C in T; ACC_FIRST / ACC / ACC_LAST build an
// fp32 sum in C32 over calls (the last one writes C); ACC_T adds into C in
// T (C = T(C + A B^T)); SPLIT writes split s's fp32 partial to
// C32 + s * split_stride.
enum GemmMode { GEMM_STORE = 0, GEMM_ACC_FIRST = 1, GEMM_ACC = 2, GEMM_ACC_LAST = 3, GEMM_ACC_T = 4, GEMM_SPLIT = 5 };

struct FusedParams {
  const void* W;
  const void* hs;
  const void* ht;
  const void* Wt;
  const void* Lt;
  const int64_t* labels;
  int64_t N, V, H, Ht, ignore_index;
  int tsrc, lt_dtype;
  int div;    // divergence code, -1 when the divergence is off
  int fam;    // family of div (FAM_NONE when off)
  int t_is_one;
  int tgrad;  // dlogits of the teacher are needed (teacher CE gradients)
  float invT, temperature, alpha, beta;
  float mix_w, mix_w1;  // mixture weight of the two-pass divergences, 1 - it
  float pa[3], pb[3];
  int npow;
  // scan
  int phase, n_ttiles, n_vranges, tiles_per_range, n_vtiles;
  float* partial;     // [n_vranges][kNStat][N]
  const float* rowp;  // [kNRowP][N]
  // dlogits
  int64_t vc0, vcc;
  float w_s, w_t, w_kl;
  const float* grad_output;
  const float* mean_scale;
  void* dLT;
  int64_t ldT, tcol;
  void* dLNs;
  void* dLNt;
  int64_t ldN;
  int w_dlt_s, w_dlt_t, w_dln_s, w_dln_t;
  // logits written by the scan of the materialised path: Lout[v][t],
  // teacher columns from tcolL (stored when store_t)
  void* Lout;
  int64_t ldL, tcolL;
  int store_t;
  // no teacher (TSRC_NONE) on the ring scan: 256 student tokens per workgroup
  int student_ring;
  // fp8 logits GEMM (launch_scan_store_f8): OCP e4m3 copies of W [V x H] and
  // of the chunk's student / teacher hidden rows [N x H], with one E8M0 scale
  // byte per row (eW, eS, eT)
  const void* W8;
  const void* hs8;
  const void* ht8;
  const uint8_t* eW;
  const uint8_t* eS;
  const uint8_t* eT;
};

struct GemmParams {
  const void* A;
  const void* B;
  void* C;
  float* C32;
  int64_t M, N, K, lda, ldb, ldc;
  int tiles_m, tiles_n, mode;
  // general GEMM (k_gemm2)
  int la, lb;                                // Layout of A and B
  const void* B1;                            // MN-major B: rows [b_kseg, K) come from B1
  int64_t ldb1, b_kseg, b_kval0, b_kval1;    // valid rows of each segment
  int splits;
  int64_t k_per_split, split_stride;         // split-K (GEMM_SPLIT partials)
};

// In-place dlogits on materialised logits (k_dlm).
struct DlmParams {
  void* L;  // [V][ldL]; student columns [0, N), teacher columns [tcol, tcol + N)
  int64_t ldL, tcol;
  const int64_t* labels;
  const float* rowp;        // [kNRowP][N]
  const float* mean_scale;  // device scalar
  int64_t N, V, ignore_index;
  int div, t_is_one, tgrad, rows_per_block;
  float invT, temperature, alpha, beta, w_s, w_t, w_kl;
  // precomputed teacher logits read in place, token-major [N][ldtm] (16-byte
  // aligned rows, ldtm a multiple of 8, rows_per_block a multiple of 8), when
  // they are not staged in L's teacher columns; else null
  const void* Ltm;
  int64_t ldtm;
  // no teacher logits at all (a top-k teacher): the dense teacher term reads
  // as zero, and its ids' share is scattered in afterwards (k_topk_scatter)
  int no_t;
};

// Per-token pass of a top-k teacher (k_topk_rows) and the scatter of its
// dlogits share (k_topk_scatter).
struct TopKParams {
  const void* hs;  // [N x H] student hidden rows of the chunk
  const void* W;   // [V x H]
  const int64_t* idx;   // [N x k] vocabulary ids
  const float* lp;      // [N x k] teacher log-probabilities (T = 1)
  const int64_t* labels;
  const float* mean_scale;
  const float* lse_sT;  // [N] student lse at T (MergeParams.lse_sT_out)
  float* rowp;          // [kNRowP][N]: row 3 (teacher lse at T) set to +inf
  float* rowv;          // [3][ldv]: row 2 (the divergence row, x T^2) written
  int64_t ldv;
  float* corr;          // [N x k]: the dlogits share at the ids
  void* L;              // [V][ldL] chunk dlogits (scatter)
  int64_t ldL;
  int64_t N, V, H, k, ignore_index;
  int div;              // DIV_FKL or DIV_SOFT
  float invT, temperature, w_kl;
};

// The student's final RMSNorm in front of the loss, per token chunk:
// y = x * rsqrt(mean(x^2) + eps) * gamma (k_rmsnorm_fwd), dloss/dgamma
// accumulated over chunks (k_rmsnorm_dgamma, then the fixed-order sum of its
// token-group partials), dloss/dx in place of dloss/dy (k_rmsnorm_bwd).
struct NormParams {
  const void* x;      // [N x H] the norm's input rows of the chunk
  const void* gamma;  // [H]
  void* y;            // [N x H] the normalised rows (compute dtype)
  float* rstd;        // [N] rsqrt(mean(x^2) + eps) per row
  void* dxy;          // [N x H] dloss/dy in; dloss/dx out (k_rmsnorm_bwd)
  float* gpart;       // [groups x H] fp32 token-group partial sums of dloss/dgamma
  float* gacc;        // [H] fp32 dloss/dgamma over the chunks so far
  void* gout;         // [H] dloss/dgamma in the compute dtype (last chunk), or null
  int64_t N, H, D;    // rows, columns (padded), columns of the mean
  int groups, first;  // token groups; first chunk (gacc stored, not added)
  float eps;
};

// Phase-1 row sums of the two-pass divergences over stored logits (k_two_rows).
struct TwoParams {
  const void* L;  // [V][ldL]; student columns [0, N), teacher columns [tcol, tcol + N)
  int64_t ldL, tcol;
  const float* rowp;  // [kNRowP][N]: rows 1 and 3 = log-sum-exps at T
  float* partial;     // [n_ranges][2][N]: x0, x1 per vocabulary range (dense)
  int64_t N, V, rows_per_range;
  int n_ranges, div;  // n_ranges <= 65535
  float invT, mix_w, mix_w1;  // mixture weight (beta for JSD, alpha for skew), 1 - it
  // precomputed teacher logits read in place, token-major [N][ldtm] (16-byte
  // aligned rows, V a multiple of 8, rows_per_range a multiple of 64); else
  // null: the teacher's logits are L's teacher columns
  const void* Ltm;
  int64_t ldtm;
};

struct LabelParams {
  const void* hs;
  const void* W;
  const void* ht;
  const void* Wt;
  const void* Lt;
  const int64_t* labels;
  int64_t N, V, H, Ht, ignore_index;
  int tsrc, lt_dtype;
  float* out;  // [2][N]
  // fp8 logits: the label logits from the same e4m3 rows and row scales as
  // the scan's (see FusedParams); W8 null otherwise
  const void* W8;
  const void* hs8;
  const void* ht8;
  const uint8_t* eW;
  const uint8_t* eS;
  const uint8_t* eT;
};

// Rows [rows x H] (compute dtype, pitch H) to OCP e4m3 bytes q [rows x H]
// and one E8M0 scale byte per row: e = the smallest power of two with
// amax(row) 2^-e <= 448 (biased by 127), q = RNE(x 2^-e).
struct QuantParams {
  const void* x;
  int64_t rows, H;
  uint8_t* q;
  uint8_t* e;
};

template <class T> hipError_t launch_scan(const FusedParams& P, int grid, hipStream_t s);
template <class T> hipError_t launch_dl(const FusedParams& P, int grid, hipStream_t s);
template <class T> hipError_t launch_gemm(const GemmParams& P, hipStream_t s);
template <class T> hipError_t launch_label(const LabelParams& P, hipStream_t s);
template <class T> hipError_t launch_scan_store(const FusedParams& P, int grid, hipStream_t s);
template <class T> hipError_t launch_scan_store_f8(const FusedParams& P, int grid, hipStream_t s);
template <class T> hipError_t launch_quant_f8(const QuantParams& P, hipStream_t s);
template <class T> hipError_t launch_gemm2(const GemmParams& P, hipStream_t s);
template <class T> hipError_t launch_dlm(const DlmParams& P, hipStream_t s);
template <class T> hipError_t launch_topk_rows(const TopKParams& P, hipStream_t s);
template <class T> hipError_t launch_topk_scatter(const TopKParams& P, hipStream_t s);
template <class T> hipError_t launch_rmsnorm_fwd(const NormParams& P, hipStream_t s);
template <class T> hipError_t launch_rmsnorm_dgamma(const NormParams& P, hipStream_t s);
template <class T> hipError_t launch_rmsnorm_bwd(const NormParams& P, hipStream_t s);
template <class T> hipError_t launch_two(const TwoParams& P, hipStream_t s);
template <class T>
hipError_t launch_splitk_reduce(const float* part, int splits, int64_t stride, void* out, int64_t ldo, int64_t M,
                                int64_t N, hipStream_t s);
template <class T> hipError_t launch_scale(void* x, int64_t n, const float* g, hipStream_t s);
template <class T>
hipError_t launch_transpose(const void* in, int64_t ldi, void* out, int64_t ldo, int64_t R, int64_t C,
                            hipStream_t s);
// The same for logits of dtype in_dtype (DT_*), rounded once to T.
template <class T>
hipError_t launch_transpose_cast(const void* in, int in_dtype, int64_t ldi, void* out, int64_t ldo, int64_t R,
                                 int64_t C, hipStream_t s);

// dtype-independent kernels (rows.hip)
struct MergeParams {
  const float* partial;
  int n_vranges;
  int64_t N, V, ignore_index;
  const int64_t* labels;
  const float* label_x;
  int phase, fam, div, t_is_one, has_t, teacher_ce, div_on;
  float invT, temperature, alpha, beta;
  float pa[3], pb[3];
  int npow;
  float* rowp;  // [kNRowP][N]
  float* rowv;  // [3][ldv]: student CE, teacher CE, T^2 * divergence
  int64_t ldv;
  // dtype the dlogits pass reads the student's / teacher's logits in when the
  // scan stored them rounded from the fp32 values its statistics came from:
  // 0 none (fp32, recomputed, or teacher logits read back from memory),
  // 1 bf16, 2 fp16
  int round_s, round_t;
  // when set: the student's log-sum-exp at T per row as the losses use it
  // (fp32 statistics, no rounding adjustment) -- a top-k teacher's rows
  float* lse_sT_out;
  // phase 1 reads k_two_rows' dense [n_vranges][2][N] pairs (else slots 6, 7
  // of the scan's [n_vranges][kNStat][N] states)
  int two_dense;
};
hipError_t launch_merge(const MergeParams& P, hipStream_t s);

struct FinalizeParams {
  const float* rowv;
  const int64_t* labels;
  int64_t N, ignore_index;
  int reduction_sum, teacher_ce, div_on;
  float w_s, w_t, w_kl;
  float* out_loss;
  float* out_ce_s;
  float* out_ce_t;
  float* out_kl;
  float* scal;  // [0] = mean_scale, [1] = count of non-ignored rows, [2] = 1
};
hipError_t launch_finalize(const FinalizeParams& P, hipStream_t s);

// scal[0] = mean scale (1 / max(count, 1), or 1 for sum), scal[1] = count of
// non-ignored labels, scal[2] = 1: the same values k_finalize writes,
// available before the loss rows exist.
hipError_t launch_count(const int64_t* labels, int64_t N, int64_t ignore_index, int reduction_sum, float* scal,
                        hipStream_t s);

// *out = a[0] * b[0] (device scalars; one thread)
hipError_t launch_mul_scalars(const float* a, const float* b, float* out, hipStream_t s);

// out[r * ld + c] = 0 for r < R, c0 <= c < c1 (element size esize bytes)
hipError_t launch_zero2d(void* out, int64_t ld, int64_t R, int64_t c0, int64_t c1, int esize, hipStream_t s);

}  // namespace orda
