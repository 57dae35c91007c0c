// abi.hip -- the C ABI of liborda_ce.so (declared in include/orda_ce.h):
// argument validation, the tile / workspace plan, and the launch sequences
// of the forward and backward passes.
#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <string>
#include <vector>
#include <atomic>
#include <mutex>

#include "../../include/orda_ce.h"
#include "launch.hpp"
#include "launch_table.hpp"
#include "orda_core.hpp"

using namespace orda;

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

inline int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }
// The mixture weight of the two-pass divergences (beta for JSD, alpha for
// the skew KLs) and 1 - weight, formed in double.
inline void set_mix(float& w, float& w1, const orda_problem_t* p) {
  if (p->divergence == ORDA_DIV_AB) {  // the second pass's exponents
    w = p->div_alpha;
    w1 = p->div_beta;
    return;
  }
  const double m = p->divergence == ORDA_DIV_JSD ? (double)p->div_beta : (double)p->div_alpha;
  w = (float)m;
  w1 = (float)(1.0 - m);
}
inline int64_t dtype_bytes(int32_t d) { return d == ORDA_F32 ? 4 : 2; }

constexpr size_t kAlign = 256;
inline size_t carve(size_t& off, size_t bytes) {
  const size_t at = (off + kAlign - 1) / kAlign * kAlign;
  off = at + bytes;
  return at;
}

// Default staging budget of one backward vocabulary chunk.
constexpr int64_t kDefaultStagingBytes = 512ll << 20;
// Target number of workgroups of a forward scan launch.
constexpr int64_t kScanTargetGroups = 2048;
// Default size of one token chunk's materialised logits (ORDA_GRADS_IN_FORWARD).
constexpr int64_t kFusedLogitsBytes = 512ll << 20;
// Workgroups of one chunk's scan and of the persistent GEMMs: one per CU of
// an MI355X (256 CUs, one 160 KiB-LDS workgroup each), so each walks a long
// run of tiles.
constexpr int64_t kPersistentGroups = 256;
// Target number of workgroups of a split-K grad-hidden GEMM (rule for shapes
// outside the launch table).
constexpr int64_t kSplitTargetGroups = 512;
// The ring engine addresses an MN-major operand's K range of one split as one
// buffer resource whose record count is a 32-bit byte count.
constexpr int64_t kRsrcBytes = 0x7fffffffll;
// Largest hidden size (K-major rows of 128 x hidden x 4 bytes stay below 2^31)
// and largest tokens per chunk (the chunk buffer's rows, 2 x chunk columns).
constexpr int64_t kMaxHidden = 1ll << 22;
constexpr int64_t kMaxChunkTokens = 1ll << 20;

struct Plan {
  int mode, dtype, eb, kelems;
  int64_t N, V, H, Ht;
  bool div_on, teacher_ce, two_pass, t1;
  int tsrc, div, fam, npow;
  float pa[3], pb[3];
  // forward
  int n_ttiles, n_vtiles, n_vranges, tiles_per_range;
  size_t off_partial, off_labelx, off_rowv, fwd_bytes;
  size_t saved_bytes;
  // backward
  bool need_gs, need_gw, need_gt, need_gwt;
  bool w_dlt_s, w_dlt_t, w_dln_s, w_dln_t, bwd_teacher;
  int bwd_tsrc;
  int64_t NP, ldT, ldh, Vc, nchunks;
  size_t off_hT, off_htT, off_dLT, off_dLNs, off_dLNt, off_WT, off_WtT, off_g32s, off_g32t, bwd_bytes;
  // gradients inside forward (materialised token chunks)
  bool fused, store_t, f_tl, f_tmem, f_sring, topk;
  // fp16: dlogits without the mean scale, gradients scaled once at the end
  bool late_scale;
  int tclass, table_entry, chunk_scale, scan_groups;
  int64_t fn, fnP, fldL, fnchunks;
  int f_nvr, f_tpr, splits_s, splits_t;
  int64_t kps_s, kps_t;
  size_t off_L, off_fpart, off_flabelx, off_frowp, off_frowv, off_split, off_fhT, off_fhtT, off_corr, off_lse;
  int64_t fldh;
  // the student's final RMSNorm in front of the loss
  bool norm, need_gnw, need_dy;
  // fp8 logits GEMM: e4m3 copies of W and of the chunk's hidden rows
  bool f8;
  size_t off_w8, off_ew, off_b8, off_eb;
  int64_t norm_dim;
  int norm_groups;
  size_t off_hn, off_rstd, off_dy, off_gpart, off_gacc;
};

constexpr int kScalFloats = 64;  // scalars at the head of the saved buffer

#define ORDA_TRY_PLAN(expr)         \
  do {                              \
    int rc_ = (expr);               \
    if (rc_ != ORDA_OK) return rc_; \
  } while (0)

// Budget of the step's extra device memory that the chunk rule keeps to
// (the headline configuration's ceiling: gradients, chunk logits and
// scratch together under 2 GB).
constexpr double kExtraMemoryBudget = 2e9;

// Chunk scale of the rule for shapes the launch table does not list: 4 when
// the chunk buffer holds only the student's 16-bit logits (teacher logits
// read in place, or none), else 2.  A large problem (a scale-2 chunk holding
// at least 256 MiB of logits) is raised from 2 to 4 when the step's extra
// memory at 4 -- the requested gradients, the chunk's logits, 4 split-K
// partials and the transposed hidden rows -- stays within
// kExtraMemoryBudget, or when no chunk keeps the budget (the gradients and a
// scale-2 chunk already exceed it) and the scale-4 chunk by itself stays
// within it: a deeper chunk halves grad W's read-modify-write passes over the
// weight.  Measured (the launch-table sweep): a separate teacher with student
// hidden 2048, 2048-token chunks at 1.69 GB against 1024 (20.9 against 22.4
// ms per step in bf16); tied hidden 8192 (gradients 2.2 GB), 72.1 against
// 75.0; tied hidden 5120, vocabulary 152064, 32768 tokens (gradients 1.89
// GB), 216-220 against 229-232; tied hidden 3584, vocabulary 152064, kept at
// 2 (1.92 GB; 2.5 GB at 4).  Smaller problems keep the plain rule (not
// swept).
inline int rule_chunk_scale(const Plan& pl, const orda_problem_t* p, int64_t ncol, int64_t Nr) {
  if (pl.f_tmem || (pl.tsrc == TSRC_NONE && pl.eb == 2)) return 4;
  if (p->token_chunk <= 0) return 2;
  const double eb = (double)pl.eb, V = (double)pl.V, H = (double)pl.H, Ht = (double)pl.Ht, N = (double)pl.N;
  const double n2 = (double)std::min<int64_t>(round_up(p->token_chunk * 2, 8), Nr);
  if (V * (double)ncol * n2 * eb < (double)(kFusedLogitsBytes / 2)) return 2;
  const double n4 = (double)std::min<int64_t>(round_up(p->token_chunk * 4, 8), Nr);
  const double grads = (pl.need_gw ? V * H * eb : 0.0) + (pl.need_gs ? N * H * eb : 0.0) +
                       (pl.need_gt ? N * Ht * eb : 0.0) + (pl.need_gwt ? V * Ht * eb : 0.0);
  auto chunk_bytes = [&](double n) { return V * (double)ncol * n * eb + 4.0 * n * H * 4.0 + 2.0 * n * H * eb; };
  const double chunk4 = chunk_bytes(n4);
  if (grads + chunk4 <= kExtraMemoryBudget) return 4;
  const bool out_of_reach = grads + chunk_bytes(n2) > kExtraMemoryBudget;
  return (out_of_reach && chunk4 <= kExtraMemoryBudget) ? 4 : 2;
}

int make_plan(const orda_problem_t* p, Plan& pl) {
  pl = Plan{};
  if (!p) return fail(ORDA_EINVAL, "problem is NULL");
  if (p->abi_version != ORDA_ABI_VERSION)
    return fail(ORDA_EINVAL, "abi_version %d does not match library version %d", p->abi_version,
                ORDA_ABI_VERSION);
  if (p->mode < ORDA_MODE_TIED || p->mode > ORDA_MODE_TOPK)
    return fail(ORDA_EINVAL, "unknown mode %d", p->mode);
  if (p->dtype < ORDA_BF16 || p->dtype > ORDA_F32) return fail(ORDA_EINVAL, "unknown dtype %d", p->dtype);
  if (p->n_rows <= 0 || p->vocab <= 0 || p->hidden <= 0)
    return fail(ORDA_EINVAL, "n_rows, vocab and hidden must be > 0 (got %lld, %lld, %lld)",
                (long long)p->n_rows, (long long)p->vocab, (long long)p->hidden);
  if (p->n_rows > (1ll << 30) || p->vocab > (1ll << 30) || p->hidden > kMaxHidden ||
      (p->mode != ORDA_MODE_TIED && p->teacher_hidden > kMaxHidden))
    return fail(ORDA_EINVAL, "shape too large (n_rows and vocab <= 2^30, hidden <= 2^22)");
  if (p->grad_hidden_splits < 0 || p->grad_hidden_splits > 64)
    return fail(ORDA_EINVAL, "grad_hidden_splits must be in [0, 64], got %d", p->grad_hidden_splits);
  if (!(p->temperature > 0.f) || !std::isfinite(p->temperature))
    return fail(ORDA_EINVAL, "temperature must be > 0, got %g", (double)p->temperature);
  if (p->student_ce_weight < 0.f || p->teacher_ce_weight < 0.f || p->kl_weight < 0.f)
    return fail(ORDA_EINVAL, "loss weights must be >= 0");
  if (p->divergence < 0 || p->divergence >= ORDA_DIV_COUNT)
    return fail(ORDA_EINVAL, "unknown divergence %d", p->divergence);

  pl.mode = p->mode;
  pl.dtype = p->dtype;
  pl.eb = p->dtype == ORDA_F32 ? 4 : 2;
  // In fp16 the dlogits times 1 / count (probabilities of ~1e-6 over ~1e4
  // counted tokens) fall below fp16's subnormals and flush to zero, which
  // drops most of grad hidden's softmax term.  The reference's fp16 path
  // stores them unscaled and applies the mean scale to the gradients
  // (ops/tied_teacher.py:532-545); so does this one.  bf16 and fp32 have
  // the range to fold the scale into the dlogits.
  pl.late_scale = p->dtype == ORDA_F16;
  pl.kelems = 16 / pl.eb;
  pl.N = p->n_rows;
  pl.V = p->vocab;
  pl.H = p->hidden;
  pl.Ht = (p->mode == ORDA_MODE_TIED) ? p->hidden : p->teacher_hidden;
  pl.div_on = (p->flags & ORDA_COMPUTE_DIVERGENCE) != 0;
  pl.teacher_ce = (p->flags & ORDA_COMPUTE_TEACHER_CE) != 0;
  pl.t1 = p->temperature == 1.0f;
  const bool need_teacher = pl.div_on || pl.teacher_ce;
  pl.topk = p->mode == ORDA_MODE_TOPK;
  if (pl.topk) {
    // the scan sees the student alone; k_topk_rows forms the divergence
    if (p->topk < 1 || p->topk > p->vocab)
      return fail(ORDA_EINVAL, "topk must be in [1, vocab], got %lld", (long long)p->topk);
    if (pl.teacher_ce) return fail(ORDA_EINVAL, "a top-k teacher has no teacher CE (teacher_ce_weight must be 0)");
    if (pl.div_on && p->divergence != ORDA_DIV_FORWARD_KL && p->divergence != ORDA_DIV_SOFT_TARGET_CE)
      return fail(ORDA_EUNSUPPORTED, "a top-k teacher supports forward KL and soft-target CE, got divergence %d",
                  p->divergence);
    if (!(p->flags & ORDA_GRADS_IN_FORWARD))
      return fail(ORDA_EINVAL, "a top-k teacher runs the gradients-in-forward schedule (ORDA_GRADS_IN_FORWARD)");
  }
  if ((p->flags & ORDA_FP8_LOGITS) && !(p->flags & ORDA_GRADS_IN_FORWARD))
    return fail(ORDA_EINVAL, "ORDA_FP8_LOGITS runs the gradients-in-forward schedule (ORDA_GRADS_IN_FORWARD)");
  pl.norm = (p->flags & ORDA_STUDENT_RMSNORM) != 0;
  pl.need_gnw = pl.norm && (p->flags & ORDA_NEED_GRAD_STUDENT_NORM_WEIGHT) != 0;
  if (!pl.norm && (p->flags & ORDA_NEED_GRAD_STUDENT_NORM_WEIGHT))
    return fail(ORDA_EINVAL, "ORDA_NEED_GRAD_STUDENT_NORM_WEIGHT needs ORDA_STUDENT_RMSNORM");
  if (pl.norm) {
    if (!(p->flags & ORDA_GRADS_IN_FORWARD))
      return fail(ORDA_EINVAL, "ORDA_STUDENT_RMSNORM runs the gradients-in-forward schedule (ORDA_GRADS_IN_FORWARD)");
    pl.norm_dim = p->norm_dim > 0 ? p->norm_dim : p->hidden;
    if (p->norm_dim < 0 || pl.norm_dim > p->hidden)
      return fail(ORDA_EINVAL, "norm_dim must be in [1, hidden] (0 = hidden), got %lld", (long long)p->norm_dim);
    if (!(p->norm_eps >= 0.f) || !std::isfinite(p->norm_eps))
      return fail(ORDA_EINVAL, "norm_eps must be finite and >= 0, got %g", (double)p->norm_eps);
  }
  if (!need_teacher || pl.topk) pl.tsrc = TSRC_NONE;
  else if (p->mode == ORDA_MODE_TIED) pl.tsrc = TSRC_SHARED;
  else if (p->mode == ORDA_MODE_PRECOMPUTED_LOGITS) pl.tsrc = TSRC_MEM;
  else pl.tsrc = TSRC_SEP;
  if (pl.tsrc == TSRC_SEP && pl.Ht <= 0) return fail(ORDA_EINVAL, "teacher_hidden must be > 0");
  if (pl.tsrc == TSRC_MEM && (p->logits_dtype < ORDA_BF16 || p->logits_dtype > ORDA_F32))
    return fail(ORDA_EINVAL, "unknown logits_dtype %d", p->logits_dtype);
  if (pl.H % pl.kelems != 0)
    return fail(ORDA_EINVAL, "hidden (%lld) must be a multiple of %d for this dtype", (long long)pl.H, pl.kelems);
  if (pl.tsrc == TSRC_SEP && pl.Ht % pl.kelems != 0)
    return fail(ORDA_EINVAL, "teacher_hidden (%lld) must be a multiple of %d for this dtype", (long long)pl.Ht,
                pl.kelems);

  // divergence
  pl.div = pl.div_on ? p->divergence : -1;
  pl.fam = pl.div_on ? div_family(p->divergence) : FAM_NONE;
  pl.two_pass = pl.fam == FAM_TWO;
  pl.npow = 0;
  for (int i = 0; i < 3; ++i) pl.pa[i] = pl.pb[i] = 0.f;
  const float a = p->div_alpha, b = p->div_beta;
  if (pl.div_on) {
    switch (p->divergence) {
      case ORDA_DIV_HELLINGER: case ORDA_DIV_BHATTACHARYYA:
        pl.npow = 1; pl.pa[0] = 0.5f; pl.pb[0] = 0.5f; break;
      case ORDA_DIV_RENYI:
        if (!(a > 0.f) || a == 1.f) return fail(ORDA_EINVAL, "renyi needs alpha > 0 and != 1, got %g", (double)a);
        pl.npow = 1; pl.pa[0] = a; pl.pb[0] = 1.f - a; break;
      case ORDA_DIV_AMARI_ALPHA:
        if (a == 0.f || a == 1.f) return fail(ORDA_EINVAL, "amari_alpha needs alpha not in {0, 1}, got %g", (double)a);
        pl.npow = 1; pl.pa[0] = a; pl.pb[0] = 1.f - a; break;
      case ORDA_DIV_CHI_SQUARED:
        pl.npow = 1; pl.pa[0] = 2.f; pl.pb[0] = -1.f; break;
      case ORDA_DIV_SQUARED_L2:
        pl.npow = 3; pl.pa[0] = 2.f; pl.pb[0] = 0.f; pl.pa[1] = 0.f; pl.pb[1] = 2.f; pl.pa[2] = 1.f; pl.pb[2] = 1.f;
        break;
      case ORDA_DIV_AB:
        if (a == 0.f || b == 0.f || a + b == 0.f)
          return fail(ORDA_EINVAL, "ab divergence needs alpha, beta, alpha+beta != 0");
        pl.npow = 3; pl.pa[0] = a; pl.pb[0] = b; pl.pa[1] = a + b; pl.pb[1] = 0.f; pl.pa[2] = 0.f; pl.pb[2] = a + b;
        break;
      case ORDA_DIV_JSD:
        if (!(b > 0.f && b < 1.f)) return fail(ORDA_EINVAL, "jsd needs 0 < beta < 1, got %g", (double)b);
        break;
      case ORDA_DIV_SKEW_FORWARD_KL: case ORDA_DIV_SKEW_REVERSE_KL:
        if (!(a >= 0.f && a < 1.f)) return fail(ORDA_EINVAL, "skew divergences need 0 <= alpha < 1, got %g", (double)a);
        break;
      default: break;
    }
  }

  // forward plan
  pl.n_ttiles = (int)cdiv(pl.N, 128);
  pl.n_vtiles = (int)cdiv(pl.V, 256);
  int64_t nvr = cdiv(kScanTargetGroups, pl.n_ttiles);  // two-phase scan
  if (nvr < 1) nvr = 1;
  if (nvr > pl.n_vtiles) nvr = pl.n_vtiles;
  pl.tiles_per_range = (int)cdiv(pl.n_vtiles, nvr);
  pl.n_vranges = (int)cdiv(pl.n_vtiles, pl.tiles_per_range);
  if ((int64_t)pl.n_ttiles * pl.n_vranges > 0x7fffffffll) return fail(ORDA_EINVAL, "grid too large");
  size_t off = 0;
  pl.off_partial = carve(off, (size_t)pl.n_vranges * kNStat * pl.N * 4);
  pl.off_labelx = carve(off, (size_t)2 * pl.N * 4);
  pl.off_rowv = carve(off, (size_t)3 * pl.N * 4);
  pl.fwd_bytes = off + kAlign;
  pl.saved_bytes = (size_t)kScalFloats * 4 + (size_t)kNRowP * pl.N * 4;

  // backward plan
  const uint32_t f = p->flags;
  const bool tied = p->mode == ORDA_MODE_TIED, sep = p->mode == ORDA_MODE_SEPARATE;
  pl.need_gs = (f & ORDA_NEED_GRAD_STUDENT_HIDDEN) != 0;
  pl.need_gw = (f & ORDA_NEED_GRAD_WEIGHT) != 0;
  pl.need_gt = (f & ORDA_NEED_GRAD_TEACHER_HIDDEN) != 0 && (tied || sep);
  pl.need_gwt = (f & ORDA_NEED_GRAD_TEACHER_WEIGHT) != 0 && sep;
  const bool tgrad = pl.teacher_ce && (tied || sep);
  pl.w_dlt_s = pl.need_gw;
  pl.w_dln_s = pl.need_gs;
  pl.w_dlt_t = tgrad && ((tied && pl.need_gw) || (sep && pl.need_gwt));
  pl.w_dln_t = tgrad && pl.need_gt;
  pl.bwd_teacher = pl.w_dlt_t || pl.w_dln_t;
  pl.bwd_tsrc = (pl.div_on || pl.bwd_teacher) ? pl.tsrc : TSRC_NONE;
  if (pl.bwd_teacher && pl.tsrc == TSRC_NONE) pl.bwd_tsrc = tied ? TSRC_SHARED : TSRC_SEP;
  pl.NP = round_up(pl.N, 8);
  pl.ldT = pl.w_dlt_t ? 2 * pl.NP : pl.NP;
  pl.ldh = (tied && pl.w_dlt_t) ? 2 * pl.NP : pl.NP;
  const int64_t Vmax = round_up(pl.V, 256);
  int64_t per_col = 0;
  if (pl.w_dlt_s || pl.w_dlt_t) per_col += pl.ldT;
  if (pl.w_dln_s) per_col += pl.N;
  if (pl.w_dln_t) per_col += pl.N;
  if (pl.need_gs || (tied && pl.w_dln_t)) per_col += pl.H;
  if (sep && pl.w_dln_t) per_col += pl.Ht;
  per_col *= pl.eb;
  if (p->vocab_chunk > 0) {
    pl.Vc = round_up(p->vocab_chunk, 256);
  } else {
    pl.Vc = per_col > 0 ? (kDefaultStagingBytes / per_col) / 256 * 256 : Vmax;
  }
  if (pl.Vc < 256) pl.Vc = 256;
  if (pl.Vc > Vmax) pl.Vc = Vmax;
  pl.nchunks = cdiv(pl.V, pl.Vc);
  off = 0;
  pl.off_hT = pl.need_gw ? carve(off, (size_t)pl.H * pl.ldh * pl.eb) : 0;
  pl.off_htT = (sep && pl.w_dlt_t) ? carve(off, (size_t)pl.Ht * pl.NP * pl.eb) : 0;
  pl.off_dLT = (pl.w_dlt_s || pl.w_dlt_t) ? carve(off, (size_t)pl.Vc * pl.ldT * pl.eb) : 0;
  pl.off_dLNs = pl.w_dln_s ? carve(off, (size_t)pl.N * pl.Vc * pl.eb) : 0;
  pl.off_dLNt = pl.w_dln_t ? carve(off, (size_t)pl.N * pl.Vc * pl.eb) : 0;
  pl.off_WT = (pl.need_gs || (tied && pl.w_dln_t)) ? carve(off, (size_t)pl.H * pl.Vc * pl.eb) : 0;
  pl.off_WtT = (sep && pl.w_dln_t) ? carve(off, (size_t)pl.Ht * pl.Vc * pl.eb) : 0;
  pl.off_g32s = (pl.need_gs && pl.nchunks > 1) ? carve(off, (size_t)pl.N * pl.H * 4) : 0;
  pl.off_g32t = (pl.w_dln_t && pl.nchunks > 1) ? carve(off, (size_t)pl.N * pl.Ht * 4) : 0;
  pl.bwd_bytes = off + kAlign;

  // gradients inside forward: one token chunk of logits at a time
  pl.fused = (f & ORDA_GRADS_IN_FORWARD) != 0;
  if (pl.fused) {
    // precomputed teachers: no teacher gradient; their logits (memory or the
    // frozen teacher GEMM) are stored next to the student's like a tied
    // teacher's
    // A separate teacher's logits (its own GEMM) or precomputed logits (cast
    // to the compute dtype when they have another) are staged into L's
    // teacher columns ahead of the scan, which
    // then runs the student GEMM alone on the ring engine, 256 tokens per
    // workgroup (16-bit, K > 64; one-pass and two-pass divergences, the power
    // family with one power term: with three its per-token state would spill
    // in every tile).  Staged logits of a computed teacher are rounded to the
    // compute dtype in L; a power term with a negative student exponent
    // (chi-squared, Renyi / Amari with alpha > 1) weighs the tail where p_s is
    // small, where that rounding moves the divergence by ~0.6% (chi-squared at
    // T = 1, against 1e-4 for the others), so those keep the two-stage scan,
    // which takes a computed teacher's logits at fp32.
    // The three-term power divergences (squared L2, AB) with such a teacher
    // run as two-pass divergences instead: the first pass only normalises
    // (no power sums in the scan's per-token state), the second pass over
    // the stored logits sums the divergence and the one row constant its
    // gradient needs (k_two_rows); computed teachers only with non-negative
    // student exponents, for the reason above.  (At C4: 29.5-31.1 ms per
    // step on the two-stage scan, 24.9-25.5 so.)
    // A tied teacher's logits are stored beside the student's anyway: the
    // same route replaces the tied ring scan's three power sums, which spill.
    const bool pb_nonneg = pl.pb[0] >= 0.f && pl.pb[1] >= 0.f && pl.pb[2] >= 0.f;
    if (pl.fam == FAM_POW && pl.npow == 3 && pl.eb == 2 && pl.H > 64 &&
        (pl.tsrc == TSRC_MEM || ((pl.tsrc == TSRC_SEP || pl.tsrc == TSRC_SHARED) && pb_nonneg))) {
      pl.fam = FAM_TWO;
      pl.two_pass = true;
    }
    const bool pow_ring = pl.npow == 1 && (pl.tsrc == TSRC_MEM || pl.pb[0] >= 0.f);
    pl.f_tl = pl.eb == 2 && pl.H > 64 && (pl.fam != FAM_POW || pow_ring) &&
              (pl.tsrc == TSRC_MEM || pl.tsrc == TSRC_SEP);
    // Precomputed 16-bit logits of the compute dtype with V a multiple of 8
    // are not staged at all: the scan (either engine), the two-pass
    // divergences' second pass and the dlogits pass all read them in place,
    // token-major (16-byte aligned rows), so L holds only the student's
    // logits and a chunk holds twice the tokens in the same memory (grad W
    // then runs half as many read-modify-write passes with twice the K).
    pl.f_tmem = pl.eb == 2 && pl.tsrc == TSRC_MEM && p->logits_dtype == p->dtype && pl.V % 8 == 0 &&
                pl.V <= 65535LL * 64;  // (k_dlm_tm's grid: one block row per 64 vocabulary rows)
    pl.store_t = pl.tsrc != TSRC_NONE && !pl.f_tmem;
    // no teacher on the scan (student CE only, or a top-k teacher): the ring
    // engine's student-only tiles, 256 tokens per workgroup (16-bit, K > 64)
    pl.f_sring = pl.eb == 2 && pl.H > 64 && pl.tsrc == TSRC_NONE;
    const int64_t ncol = pl.store_t ? 2 : 1;
    const int64_t Nr = round_up(pl.N, 8);
    // launch geometry: the gfx950 table for measured shapes, else the rule
    pl.tclass = pl.f_tmem                                           ? TC_INPLACE
                : pl.f_tl                                           ? TC_STAGED
                : (pl.tsrc == TSRC_SHARED && pl.eb == 2 && pl.H > 64) ? TC_TIED
                                                                    : TC_OTHER;
    pl.table_entry = find_launch_entry(pl.tclass, pl.dtype, pl.V, pl.H);
    const LaunchEntry* te = pl.table_entry >= 0 ? &kLaunchTable[pl.table_entry] : nullptr;
    // (the rule: 4 when the chunk buffer holds only the student's 16-bit
    // logits -- teacher logits read in place, or no teacher logits at all --
    // else 2, raised to 4 for large problems when the step's extra memory at
    // 4 stays under the 2 GB budget, or when the gradients alone exceed it;
    // see rule_chunk_scale)
    pl.chunk_scale = te ? te->chunk_scale : rule_chunk_scale(pl, p, ncol, Nr);
    pl.scan_groups = te ? te->scan_groups : (int)kPersistentGroups;
    int64_t n = p->token_chunk;
    if (n > 0) {
      n = round_up(n * pl.chunk_scale, 8);
    } else {
      n = kFusedLogitsBytes / (pl.V * ncol * pl.eb) / 128 * 128;
      if (n < 128) n = 128;
    }
    if (n > Nr) n = Nr;
    if (n > kMaxChunkTokens) n = kMaxChunkTokens;
    pl.fn = n;
    pl.fnP = round_up(n, 8);
    pl.fldL = ncol * pl.fnP;
    pl.fnchunks = cdiv(pl.N, n);
    const int64_t ntt = cdiv(n, (pl.f_tl || pl.f_sring) ? 256 : 128);
    // vocabulary ranges per token tile: the scan's ntt x nvr workgroups stay
    // within scan_groups, so they run in one wave of one per CU (rounding up
    // put 10 token tiles at 260 workgroups, the last 4 a second wave that
    // doubled the scan's time)
    int64_t nvr = pl.scan_groups / ntt;
    if (nvr < 1) nvr = 1;
    if (nvr > pl.n_vtiles) nvr = pl.n_vtiles;
    pl.f_tpr = (int)cdiv(pl.n_vtiles, nvr);
    pl.f_nvr = (int)cdiv(pl.n_vtiles, pl.f_tpr);
    // the table's split count is measured for the student's hidden size (the
    // tied teacher's too); a separate teacher's own grad hidden takes the rule
    auto split_plan = [&](int64_t cols, int& splits, int64_t& kps) -> int {
      int64_t sp = 1;
      if (p->grad_hidden_splits > 0) {
        sp = p->grad_hidden_splits;
      } else if (te && cols == pl.H) {
        sp = te->splits_h;
      } else {
        // Rule: the persistent GEMM runs its tiles x splits equal work items
        // in rounds of kPersistentGroups workgroups, so its time goes as
        // ceil(items / groups) / splits: pick the split count (1..16) that
        // minimises it (a partial last round idles CUs: 80 tiles x 7 splits
        // is 3 rounds at 73% fill, x 16 is 5 full ones), the one nearest
        // kSplitTargetGroups / tiles among equals.
        const int64_t tiles = cdiv(n, 256) * cdiv(cols, 256);
        int64_t want = cdiv(kSplitTargetGroups, tiles);
        if (want > 16) want = 16;
        double best = 1e30;
        for (int64_t c = 1; c <= 16; ++c) {
          const double cost = (double)cdiv(tiles * c, kPersistentGroups) / (double)c;
          const bool nearer = std::llabs(c - want) < std::llabs(sp - want);
          if (cost < best * (1.0 - 1e-9) || (cost <= best * (1.0 + 1e-9) && nearer)) {
            best = cost;
            sp = c;
          }
        }
      }
      // each split's K range of both MN-major operands (the chunk's dlogits,
      // ld = fldL, and the weight, ld = cols) must stay inside one 32-bit
      // buffer resource
      const int64_t ldmax = std::max<int64_t>(pl.fldL, cols) * pl.eb;
      const int64_t kmax = kRsrcBytes / ldmax / 64 * 64;
      if (kmax < 64) return fail(ORDA_EINVAL, "vocab rows of %lld bytes exceed a buffer resource", (long long)ldmax);
      const int64_t need = cdiv(pl.V, kmax);
      if (need > 64) return fail(ORDA_EINVAL, "grad hidden needs %lld splits of the vocabulary (at most 64)", (long long)need);
      if (sp < need) sp = need;
      kps = round_up(cdiv(pl.V, sp), 64);
      splits = (int)cdiv(pl.V, kps);
      return ORDA_OK;
    };
    ORDA_TRY_PLAN(split_plan(pl.H, pl.splits_s, pl.kps_s));
    ORDA_TRY_PLAN(split_plan(pl.Ht, pl.splits_t, pl.kps_t));
    size_t fo = 0;
    pl.off_L = carve(fo, (size_t)pl.V * pl.fldL * pl.eb);
    pl.off_fpart = carve(fo, (size_t)pl.f_nvr * kNStat * pl.fnP * 4);
    pl.off_flabelx = carve(fo, (size_t)2 * pl.fnP * 4);
    pl.off_frowp = carve(fo, (size_t)kNRowP * pl.fnP * 4);
    pl.off_frowv = carve(fo, (size_t)3 * pl.N * 4);
    int64_t split_cols = 0;
    if ((pl.need_gs || pl.need_gnw) && pl.splits_s > 1) split_cols = pl.splits_s * pl.H;
    if (pl.w_dln_t && pl.splits_t > 1 && pl.splits_t * pl.Ht > split_cols) split_cols = pl.splits_t * pl.Ht;
    pl.off_split = split_cols ? carve(fo, (size_t)split_cols * pl.fnP * 4) : 0;
    // the chunk's hidden states transposed (token-contiguous) for the grad-W
    // GEMMs: K-major B runs faster on the ring engine than reading them in
    // place as an MN-major B (measured at C2: 16.4 vs 17.5 ms per step, against
    // 0.3 ms of transposes)
    pl.fldh = (tied && pl.w_dlt_t) ? 2 * pl.fnP : pl.fnP;
    pl.off_fhT = pl.need_gw ? carve(fo, (size_t)pl.H * pl.fldh * pl.eb) : 0;
    pl.off_fhtT = (sep && pl.need_gwt && pl.w_dlt_t) ? carve(fo, (size_t)pl.Ht * pl.fnP * pl.eb) : 0;
    pl.off_corr = pl.topk ? carve(fo, (size_t)pl.fnP * p->topk * 4) : 0;
    pl.off_lse = pl.topk ? carve(fo, (size_t)pl.fnP * 4) : 0;
    // RMSNorm prologue: the chunk's normalised rows, their rsqrt, dloss/dy when
    // dloss/dx is not asked for, and the norm weight's gradient sums
    pl.need_dy = pl.need_gs || pl.need_gnw;
    pl.norm_groups = (int)std::min<int64_t>(128, cdiv(pl.fn, 8));
    pl.off_hn = pl.norm ? carve(fo, (size_t)pl.fnP * pl.H * pl.eb) : 0;
    pl.off_rstd = pl.norm ? carve(fo, (size_t)pl.fnP * 4) : 0;
    pl.off_dy = (pl.need_gnw && !pl.need_gs) ? carve(fo, (size_t)pl.fnP * pl.H * pl.eb) : 0;
    pl.off_gpart = pl.need_gnw ? carve(fo, (size_t)pl.norm_groups * pl.H * 4) : 0;
    pl.off_gacc = pl.need_gnw ? carve(fo, (size_t)pl.H * 4) : 0;
    // fp8 logits: W (V x H bytes + V scale bytes) once per call, the chunk's
    // student (and tied teacher) rows per chunk
    pl.f8 = (p->flags & ORDA_FP8_LOGITS) != 0;
    if (pl.f8) {
      if (pl.eb != 2) return fail(ORDA_EUNSUPPORTED, "ORDA_FP8_LOGITS needs a 16-bit compute dtype");
      if (pl.H % 16 != 0 || pl.H <= 128)
        return fail(ORDA_EUNSUPPORTED, "ORDA_FP8_LOGITS needs hidden a multiple of 16 and > 128, got %lld",
                    (long long)pl.H);
      if (pl.topk) return fail(ORDA_EUNSUPPORTED, "ORDA_FP8_LOGITS does not support a top-k teacher");
      const bool ring = (pl.tclass == TC_TIED) || (pl.f_tmem && pl.fam != FAM_POW) || pl.f_sring;
      if (!ring)
        return fail(ORDA_EUNSUPPORTED, "ORDA_FP8_LOGITS supports a tied teacher, precomputed logits read in place "
                    "(not the power-family divergences) or no teacher term");
      const int64_t nb = pl.tsrc == TSRC_SHARED ? 2 : 1;
      pl.off_w8 = carve(fo, (size_t)pl.V * pl.H);
      pl.off_ew = carve(fo, (size_t)pl.V);
      pl.off_b8 = carve(fo, (size_t)nb * pl.fnP * pl.H);
      pl.off_eb = carve(fo, (size_t)nb * pl.fnP);
    }
    pl.fwd_bytes = fo + kAlign;
    pl.bwd_bytes = 0;
  }
  return ORDA_OK;
}

inline char* aligned_base(void* ws) {
  const uintptr_t u = reinterpret_cast<uintptr_t>(ws);
  return reinterpret_cast<char*>((u + kAlign - 1) / kAlign * kAlign);
}

inline bool aligned16(const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15u) == 0; }

// ------------------------------------------------------------ timing hook
struct TimedLaunch {
  hipEvent_t start, stop;
  int kind;
  double alg, exe;
};
// Process-wide (autograd runs backward on its own device thread).
std::mutex g_timing_mu;
std::atomic<bool> g_timing{false};
std::vector<TimedLaunch> g_launches;
std::vector<hipEvent_t> g_event_pool;

// Caller holds g_timing_mu.
hipEvent_t pooled_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Brackets one launch with events on its stream when timing is enabled.
struct Timed {
  bool on;
  TimedLaunch rec;
  hipStream_t s;
  Timed(int kind, hipStream_t stream, double alg, double exe) : on(g_timing.load()), s(stream) {
    if (!on) return;
    {
      std::lock_guard<std::mutex> lk(g_timing_mu);
      rec = TimedLaunch{pooled_event(), pooled_event(), kind, alg, exe};
    }
    if (!rec.start || !rec.stop || hipEventRecord(rec.start, s) != hipSuccess) drop();
  }
  ~Timed() {
    if (!on) return;
    if (hipEventRecord(rec.stop, s) != hipSuccess) { drop(); return; }
    std::lock_guard<std::mutex> lk(g_timing_mu);
    g_launches.push_back(rec);
  }
  // a launch whose events could not be recorded is not timed (its events go
  // back to the pool)
  void drop() {
    on = false;
    std::lock_guard<std::mutex> lk(g_timing_mu);
    if (rec.start) g_event_pool.push_back(rec.start);
    if (rec.stop) g_event_pool.push_back(rec.stop);
  }
};

#define ORDA_CHECK_LAUNCH(expr)                                                        \
  do {                                                                                 \
    hipError_t e_ = (expr);                                                            \
    if (e_ != hipSuccess) return fail(ORDA_ELAUNCH, "%s: %s", #expr, hipGetErrorString(e_)); \
  } while (0)

template <class T>
int run_forward(const Plan& pl, const orda_problem_t* p, const orda_tensors_t* t, char* ws, hipStream_t s) {
  float* partial = reinterpret_cast<float*>(ws + pl.off_partial);
  float* labelx = reinterpret_cast<float*>(ws + pl.off_labelx);
  float* rowv = reinterpret_cast<float*>(ws + pl.off_rowv);
  float* scal = static_cast<float*>(t->saved);
  float* rowp = scal + kScalFloats;

  LabelParams L{};
  L.hs = t->student_hidden; L.W = t->weight; L.ht = t->teacher_hidden; L.Wt = t->teacher_weight;
  L.Lt = t->teacher_logits; L.labels = t->labels;
  L.N = pl.N; L.V = pl.V; L.H = pl.H; L.Ht = pl.Ht; L.ignore_index = p->ignore_index;
  L.tsrc = pl.tsrc; L.lt_dtype = p->logits_dtype; L.out = labelx;
  { Timed tm_(ORDA_K_ROWS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_label<T>(L, s)); }

  FusedParams F{};
  F.W = t->weight; F.hs = t->student_hidden; F.ht = t->teacher_hidden; F.Wt = t->teacher_weight;
  F.Lt = t->teacher_logits; F.labels = t->labels;
  F.N = pl.N; F.V = pl.V; F.H = pl.H; F.Ht = pl.Ht; F.ignore_index = p->ignore_index;
  F.tsrc = pl.tsrc; F.lt_dtype = p->logits_dtype;
  F.div = pl.div; F.fam = pl.fam; F.t_is_one = pl.t1; F.tgrad = 0;
  F.temperature = p->temperature; F.invT = 1.0f / p->temperature;
  F.alpha = p->div_alpha; F.beta = p->div_beta;
  set_mix(F.mix_w, F.mix_w1, p);
  for (int i = 0; i < 3; ++i) { F.pa[i] = pl.pa[i]; F.pb[i] = pl.pb[i]; }
  F.npow = pl.npow;
  F.phase = 0; F.n_ttiles = pl.n_ttiles; F.n_vranges = pl.n_vranges;
  F.tiles_per_range = pl.tiles_per_range; F.n_vtiles = pl.n_vtiles;
  F.partial = partial; F.rowp = rowp;
  const int grid = pl.n_ttiles * pl.n_vranges;
  const double scan_flops = 2.0 * (double)pl.N * (double)pl.V *
                            ((double)pl.H + ((pl.tsrc == TSRC_SHARED || pl.tsrc == TSRC_SEP) ? (double)pl.Ht : 0.0));
  { Timed tm_(ORDA_K_SCAN, s, scan_flops, scan_flops); ORDA_CHECK_LAUNCH(launch_scan<T>(F, grid, s)); }

  MergeParams M{};
  M.partial = partial; M.n_vranges = pl.n_vranges; M.N = pl.N; M.V = pl.V; M.ignore_index = p->ignore_index;
  M.labels = t->labels; M.label_x = labelx; M.phase = 0; M.fam = pl.fam; M.div = pl.div;
  M.t_is_one = pl.t1; M.has_t = pl.tsrc != TSRC_NONE; M.teacher_ce = pl.teacher_ce; M.div_on = pl.div_on;
  M.invT = F.invT; M.temperature = p->temperature; M.alpha = p->div_alpha; M.beta = p->div_beta;
  for (int i = 0; i < 3; ++i) { M.pa[i] = pl.pa[i]; M.pb[i] = pl.pb[i]; }
  M.npow = pl.npow; M.rowp = rowp; M.rowv = rowv; M.ldv = pl.N;
  { Timed tm_(ORDA_K_ROWS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_merge(M, s)); }

  if (pl.two_pass) {
    F.phase = 1;
    { Timed tm_(ORDA_K_SCAN, s, 0.0, scan_flops); ORDA_CHECK_LAUNCH(launch_scan<T>(F, grid, s)); }
    M.phase = 1;
    { Timed tm_(ORDA_K_ROWS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_merge(M, s)); }
  }

  FinalizeParams Z{};
  Z.rowv = rowv; Z.labels = t->labels; Z.N = pl.N; Z.ignore_index = p->ignore_index;
  Z.reduction_sum = (p->flags & ORDA_REDUCTION_SUM) != 0;
  Z.teacher_ce = pl.teacher_ce; Z.div_on = pl.div_on;
  Z.w_s = p->student_ce_weight; Z.w_t = p->teacher_ce_weight; Z.w_kl = p->kl_weight;
  Z.out_loss = t->out_loss; Z.out_ce_s = t->out_student_ce; Z.out_ce_t = t->out_teacher_ce; Z.out_kl = t->out_kl;
  Z.scal = scal;
  { Timed tm_(ORDA_K_ROWS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_finalize(Z, s)); }
  return ORDA_OK;
}

template <class T>
int gemm(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, float* C32, int64_t ldc, int64_t M,
         int64_t N, int64_t K, int mode, hipStream_t s, int kind = ORDA_K_AUX, double alg = 0.0) {
  GemmParams G{};
  G.A = A; G.B = B; G.C = C; G.C32 = C32;
  G.M = M; G.N = N; G.K = K; G.lda = lda; G.ldb = ldb; G.ldc = ldc;
  G.tiles_m = (int)cdiv(M, 256); G.tiles_n = (int)cdiv(N, 256); G.mode = mode;
  if ((int64_t)G.tiles_m * G.tiles_n > 0x7fffffffll) return fail(ORDA_EINVAL, "gemm grid too large");
  Timed tm_(kind, s, alg, 2.0 * (double)M * (double)N * (double)K);
  ORDA_CHECK_LAUNCH(launch_gemm<T>(G, s));
  return ORDA_OK;
}

#define ORDA_TRY(expr)      \
  do {                      \
    int rc_ = (expr);       \
    if (rc_ != ORDA_OK) return rc_; \
  } while (0)

// Every requested gradient *= factor[0] (a device scalar; the scaling kernel
// returns at once when it is 1).
template <class T>
int scale_grads(const Plan& pl, const orda_tensors_t* t, const float* factor, hipStream_t s) {
  auto sc = [&](void* g, int64_t n) -> int {
    if (!g) return ORDA_OK;
    Timed tm_(ORDA_K_AUX, s, 0.0, 0.0);
    ORDA_CHECK_LAUNCH(launch_scale<T>(g, n, factor, s));
    return ORDA_OK;
  };
  if (pl.need_gs) ORDA_TRY(sc(t->grad_student_hidden, pl.N * pl.H));
  if (pl.need_gw) ORDA_TRY(sc(t->grad_weight, pl.V * pl.H));
  if (pl.need_gt) ORDA_TRY(sc(t->grad_teacher_hidden, pl.N * pl.Ht));
  if (pl.need_gwt) ORDA_TRY(sc(t->grad_teacher_weight, pl.V * pl.Ht));
  if (pl.need_gnw) ORDA_TRY(sc(t->grad_student_norm_weight, pl.H));
  return ORDA_OK;
}

template <class T>
int run_backward(const Plan& pl, const orda_problem_t* p, const orda_tensors_t* t, char* ws, hipStream_t s) {
  const bool tied = pl.mode == ORDA_MODE_TIED, sep = pl.mode == ORDA_MODE_SEPARATE;
  const int eb = pl.eb;
  const int64_t N = pl.N, H = pl.H, Ht = pl.Ht, NP = pl.NP;
  char* hT = ws + pl.off_hT;
  char* htT = ws + pl.off_htT;
  char* dLT = ws + pl.off_dLT;
  char* dLNs = ws + pl.off_dLNs;
  char* dLNt = ws + pl.off_dLNt;
  char* WT = ws + pl.off_WT;
  char* WtT = ws + pl.off_WtT;
  float* g32s = reinterpret_cast<float*>(ws + pl.off_g32s);
  float* g32t = reinterpret_cast<float*>(ws + pl.off_g32t);
  float* scal = static_cast<float*>(t->saved);
  float* rowp = scal + kScalFloats;

  // Tied mode with teacher CE off: the teacher hidden gradient is zero
  // (reference ops/tied_teacher.py:478-479).
  if (tied && pl.need_gt && !pl.w_dln_t)
    { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(t->grad_teacher_hidden, H, N, 0, H, eb, s)); }

  const bool any = pl.w_dlt_s || pl.w_dlt_t || pl.w_dln_s || pl.w_dln_t;
  if (!any) return ORDA_OK;

  // Transposed hidden states for the grad_W GEMMs (K = tokens), with zeroed
  // padding columns so K can be rounded up to a multiple of 8.
  if (pl.need_gw) {
    { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(hT, pl.ldh, H, N, NP, eb, s)); }
    { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_transpose<T>(t->student_hidden, H, hT, pl.ldh, N, H, s)); }
    if (tied && pl.w_dlt_t) {
      { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(hT, pl.ldh, H, NP + N, 2 * NP, eb, s)); }
      { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_transpose<T>(t->teacher_hidden, H, hT + NP * eb, pl.ldh, N, H, s)); }
    }
  }
  if (sep && pl.w_dlt_t) {
    { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(htT, NP, Ht, N, NP, eb, s)); }
    { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_transpose<T>(t->teacher_hidden, Ht, htT, NP, N, Ht, s)); }
  }
  // padding columns of the staged dlogits (never written by the dL kernel)
  if (pl.w_dlt_s || pl.w_dlt_t) { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(dLT, pl.ldT, pl.Vc, N, NP, eb, s)); }
  if (pl.w_dlt_t) { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(dLT, pl.ldT, pl.Vc, NP + N, 2 * NP, eb, s)); }

  FusedParams F{};
  F.W = t->weight; F.hs = t->student_hidden; F.ht = t->teacher_hidden; F.Wt = t->teacher_weight;
  F.Lt = t->teacher_logits; F.labels = t->labels;
  F.N = N; F.V = pl.V; F.H = H; F.Ht = Ht; F.ignore_index = p->ignore_index;
  F.tsrc = pl.bwd_tsrc; F.lt_dtype = p->logits_dtype;
  F.div = pl.div; F.fam = pl.fam; F.t_is_one = pl.t1; F.tgrad = pl.bwd_teacher;
  F.temperature = p->temperature; F.invT = 1.0f / p->temperature;
  F.alpha = p->div_alpha; F.beta = p->div_beta;
  set_mix(F.mix_w, F.mix_w1, p);
  F.n_ttiles = pl.n_ttiles; F.rowp = rowp;
  F.w_s = p->student_ce_weight; F.w_t = p->teacher_ce_weight; F.w_kl = pl.div_on ? p->kl_weight : 0.f;
  // fp16: unscaled dlogits (scal[2] = 1); the gradients get grad_output x
  // mean_scale at the end
  F.grad_output = pl.late_scale ? scal + 2 : t->grad_output;
  F.mean_scale = pl.late_scale ? scal + 2 : scal;
  F.dLT = dLT; F.ldT = pl.ldT; F.tcol = NP; F.dLNs = dLNs; F.dLNt = dLNt; F.ldN = pl.Vc;
  F.w_dlt_s = pl.w_dlt_s; F.w_dlt_t = pl.w_dlt_t; F.w_dln_s = pl.w_dln_s; F.w_dln_t = pl.w_dln_t;

  const int64_t Kw = (tied && pl.w_dlt_t) ? 2 * NP : NP;
  for (int64_t c = 0; c < pl.nchunks; ++c) {
    const int64_t vc0 = c * pl.Vc;
    const int64_t vcc = (pl.V - vc0 < pl.Vc) ? pl.V - vc0 : pl.Vc;
    const int64_t vck = round_up(vcc, pl.kelems);  // K of the grad_hidden GEMMs
    const int gmode = pl.nchunks == 1 ? GEMM_STORE
                      : c == 0 ? GEMM_ACC_FIRST
                      : c == pl.nchunks - 1 ? GEMM_ACC_LAST : GEMM_ACC;
    const bool needWT = pl.need_gs || (tied && pl.w_dln_t);
    if (needWT) {
      { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_transpose<T>(static_cast<const char*>(t->weight) + vc0 * H * eb, H, WT, pl.Vc, vcc, H, s)); }
      if (vck > vcc) { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(WT, pl.Vc, H, vcc, vck, eb, s)); }
    }
    if (sep && pl.w_dln_t) {
      { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_transpose<T>(static_cast<const char*>(t->teacher_weight) + vc0 * Ht * eb, Ht, WtT, pl.Vc, vcc, Ht, s)); }
      if (vck > vcc) { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(WtT, pl.Vc, Ht, vcc, vck, eb, s)); }
    }
    if (vck > vcc) {
      if (pl.w_dln_s) { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(dLNs, pl.Vc, N, vcc, vck, eb, s)); }
      if (pl.w_dln_t) { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(dLNt, pl.Vc, N, vcc, vck, eb, s)); }
    }
    F.vc0 = vc0; F.vcc = vcc;
    const int grid = (int)(cdiv(vcc, 256) * pl.n_ttiles);
    {
      const double kt = (pl.bwd_tsrc == TSRC_SHARED || pl.bwd_tsrc == TSRC_SEP) ? (double)Ht : 0.0;
      Timed tm_(ORDA_K_DLOGITS, s, 0.0, 2.0 * (double)N * (double)vcc * ((double)H + kt));
      ORDA_CHECK_LAUNCH(launch_dl<T>(F, grid, s));
    }

    if (pl.need_gw) {
      const double kv = (tied && pl.w_dlt_t) ? 2.0 * (double)N : (double)N;
      ORDA_TRY(gemm<T>(dLT, pl.ldT, hT, pl.ldh, static_cast<char*>(t->grad_weight) + vc0 * H * eb, nullptr, H, vcc,
                       H, Kw, GEMM_STORE, s, ORDA_K_GEMM_W, 2.0 * (double)vcc * (double)H * kv));
    }
    if (sep && pl.need_gwt && pl.w_dlt_t) {
      ORDA_TRY(gemm<T>(dLT + NP * eb, pl.ldT, htT, NP, static_cast<char*>(t->grad_teacher_weight) + vc0 * Ht * eb,
                       nullptr, Ht, vcc, Ht, NP, GEMM_STORE, s, ORDA_K_GEMM_W,
                       2.0 * (double)vcc * (double)Ht * (double)N));
    }
    if (pl.need_gs) {
      ORDA_TRY(gemm<T>(dLNs, pl.Vc, WT, pl.Vc, t->grad_student_hidden, g32s, H, N, H, vck, gmode, s, ORDA_K_GEMM_H,
                       2.0 * (double)N * (double)H * (double)vcc));
    }
    if (pl.w_dln_t) {
      ORDA_TRY(gemm<T>(dLNt, pl.Vc, tied ? WT : WtT, pl.Vc, t->grad_teacher_hidden, g32t, Ht, N, Ht, vck, gmode, s,
                       ORDA_K_GEMM_H, 2.0 * (double)N * (double)Ht * (double)vcc));
    }
  }
  // separate mode, teacher weight grad requested but teacher CE off: zero
  if (sep && pl.need_gwt && !pl.w_dlt_t)
    { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(t->grad_teacher_weight, Ht, pl.V, 0, Ht, eb, s)); }
  if (sep && pl.need_gt && !pl.w_dln_t)
    { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(t->grad_teacher_hidden, Ht, N, 0, Ht, eb, s)); }
  if (pl.late_scale) {
    { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_mul_scalars(t->grad_output, scal, scal + 3, s)); }
    ORDA_TRY(scale_grads<T>(pl, t, scal + 3, s));
  }
  return ORDA_OK;
}

// One launch of the general GEMM (k_gemm2); B1/b_kseg/b_kval* describe an
// MN-major B in two row segments (b_kseg = K, b_kval0 = K, B1 = NULL for
// one).  splits > 1 writes fp32 partials [splits][M][N] to C32 (mode SPLIT).
template <class T>
int gemm2(int la, int lb, const void* A, int64_t lda, const void* B, int64_t ldb, const void* B1, int64_t ldb1,
          int64_t b_kseg, int64_t b_kval0, int64_t b_kval1, void* C, float* C32, int64_t ldc, int64_t M,
          int64_t N, int64_t K, int mode, int splits, int64_t kps, hipStream_t s, int kind, double alg) {
  GemmParams G{};
  G.A = A; G.B = B; G.C = C; G.C32 = C32;
  G.M = M; G.N = N; G.K = K; G.lda = lda; G.ldb = ldb; G.ldc = ldc;
  G.tiles_m = (int)cdiv(M, 256); G.tiles_n = (int)cdiv(N, 256); G.mode = mode;
  G.la = la; G.lb = lb; G.B1 = B1; G.ldb1 = ldb1; G.b_kseg = b_kseg; G.b_kval0 = b_kval0; G.b_kval1 = b_kval1;
  G.splits = splits < 1 ? 1 : splits;
  G.k_per_split = G.splits > 1 ? kps : K;
  G.split_stride = M * ldc;
  if ((int64_t)G.tiles_m * G.tiles_n * G.splits > 0x7fffffffll) return fail(ORDA_EINVAL, "gemm grid too large");
  Timed tm_(kind, s, alg, 2.0 * (double)M * (double)N * (double)K);
  ORDA_CHECK_LAUNCH(launch_gemm2<T>(G, s));
  return ORDA_OK;
}

// Forward with the gradients (ORDA_GRADS_IN_FORWARD), token chunk by token
// chunk: label logits, the scan with the logits stored vocabulary-major in L,
// the per-row merge, dlogits in place (k_dlm), grad W += dL^T [hs; ht]
// (A = L K-major over tokens, B = the chunk's hidden states read MN-major),
// grad hidden = dL W (A = L and B = W both MN-major, split over V).
template <class T>
int run_fused(const Plan& pl, const orda_problem_t* p, const orda_tensors_t* t, char* ws, hipStream_t s) {
  const bool tied = pl.mode == ORDA_MODE_TIED, sep = pl.mode == ORDA_MODE_SEPARATE;
  const int eb = pl.eb;
  const int64_t N = pl.N, V = pl.V, H = pl.H, Ht = pl.Ht, nP = pl.fnP, ldL = pl.fldL;
  char* L = ws + pl.off_L;
  float* part = reinterpret_cast<float*>(ws + pl.off_fpart);
  float* labelx = reinterpret_cast<float*>(ws + pl.off_flabelx);
  float* rowp = reinterpret_cast<float*>(ws + pl.off_frowp);
  float* rowv = reinterpret_cast<float*>(ws + pl.off_frowv);
  float* split = reinterpret_cast<float*>(ws + pl.off_split);
  float* scal = static_cast<float*>(t->saved);
  const bool reduction_sum = (p->flags & ORDA_REDUCTION_SUM) != 0;
  const bool tgrad = pl.w_dlt_t || pl.w_dln_t;
  const bool any_grad = pl.need_gs || pl.need_gw || pl.need_gnw || tgrad;
  const T* hs = static_cast<const T*>(t->student_hidden);
  const T* ht = static_cast<const T*>(t->teacher_hidden);
  const T* W = static_cast<const T*>(t->weight);
  const T* Wt = static_cast<const T*>(t->teacher_weight);

  if (pl.f_tmem && reinterpret_cast<uintptr_t>(t->teacher_logits) % 16 != 0)
    return fail(ORDA_EINVAL, "precomputed teacher logits must be 16-byte aligned when the vocabulary is a multiple of 8");
  uint8_t* w8 = nullptr;
  uint8_t* ew = nullptr;
  if (pl.f8) {
    // W in e4m3 with its row scales, once per call
    w8 = reinterpret_cast<uint8_t*>(ws + pl.off_w8);
    ew = reinterpret_cast<uint8_t*>(ws + pl.off_ew);
    QuantParams Q{W, V, H, w8, ew};
    Timed tm_(ORDA_K_AUX, s, 0.0, 0.0);
    ORDA_CHECK_LAUNCH(launch_quant_f8<T>(Q, s));
  }
  // mean scale first: the chunks' dlogits need it before the loss rows exist
  { Timed tm_(ORDA_K_ROWS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_count(t->labels, N, p->ignore_index, reduction_sum, scal, s)); }

  for (int64_t c = 0; c < pl.fnchunks; ++c) {
    const int64_t r0 = c * pl.fn;
    const int64_t nc = (N - r0 < pl.fn) ? N - r0 : pl.fn;

    // the chunk's student rows as the GEMMs see them: the caller's, or their
    // RMSNorm (then x is the caller's rows and hsc the normalised copy)
    const T* hsc = hs + r0 * H;
    NormParams Nm{};
    if (pl.norm) {
      Nm.x = hs + r0 * H; Nm.gamma = t->student_norm_weight; Nm.y = ws + pl.off_hn;
      Nm.rstd = reinterpret_cast<float*>(ws + pl.off_rstd);
      Nm.N = nc; Nm.H = H; Nm.D = pl.norm_dim; Nm.eps = p->norm_eps;
      Nm.groups = pl.norm_groups; Nm.first = c == 0 ? 1 : 0;
      { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_rmsnorm_fwd<T>(Nm, s)); }
      hsc = reinterpret_cast<const T*>(ws + pl.off_hn);
    }

    // fp8: the chunk's student (and tied teacher) rows in e4m3
    uint8_t* hs8 = nullptr;
    uint8_t* ht8 = nullptr;
    uint8_t *es = nullptr, *et = nullptr;
    if (pl.f8) {
      hs8 = reinterpret_cast<uint8_t*>(ws + pl.off_b8);
      es = reinterpret_cast<uint8_t*>(ws + pl.off_eb);
      QuantParams Q{hsc, nc, H, hs8, es};
      { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_quant_f8<T>(Q, s)); }
      if (pl.tsrc == TSRC_SHARED) {
        ht8 = hs8 + nP * H;
        et = es + nP;
        QuantParams Qt{ht + r0 * H, nc, H, ht8, et};
        Timed tm_(ORDA_K_AUX, s, 0.0, 0.0);
        ORDA_CHECK_LAUNCH(launch_quant_f8<T>(Qt, s));
      }
    }

    LabelParams Lb{};
    // the chunk's rows of precomputed teacher logits [N x V] (logits dtype)
    const void* Ltc = t->teacher_logits
                          ? static_cast<const char*>(t->teacher_logits) + r0 * V * dtype_bytes(p->logits_dtype)
                          : nullptr;
    Lb.hs = hsc; Lb.W = W; Lb.ht = ht ? ht + r0 * Ht : nullptr; Lb.Wt = Wt; Lb.Lt = Ltc;
    Lb.labels = t->labels + r0;
    Lb.N = nc; Lb.V = V; Lb.H = H; Lb.Ht = Ht; Lb.ignore_index = p->ignore_index;
    Lb.tsrc = pl.tsrc; Lb.lt_dtype = p->logits_dtype; Lb.out = labelx;
    Lb.W8 = w8; Lb.hs8 = hs8; Lb.ht8 = ht8; Lb.eW = ew; Lb.eS = es; Lb.eT = et;
    { Timed tm_(ORDA_K_ROWS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_label<T>(Lb, s)); }

    FusedParams F{};
    F.W = W; F.hs = hsc; F.ht = ht ? ht + r0 * Ht : nullptr; F.Wt = Wt; F.Lt = Ltc;
    F.labels = t->labels + r0;
    F.N = nc; F.V = V; F.H = H; F.Ht = Ht; F.ignore_index = p->ignore_index;
    F.tsrc = pl.tsrc; F.lt_dtype = p->logits_dtype;
    // (a top-k teacher's scan and merge see the student alone: no family)
    F.div = pl.div; F.fam = pl.topk ? FAM_NONE : pl.fam; F.t_is_one = pl.t1; F.tgrad = 0;
    F.temperature = p->temperature; F.invT = 1.0f / p->temperature;
    F.alpha = p->div_alpha; F.beta = p->div_beta;
    set_mix(F.mix_w, F.mix_w1, p);
    for (int i = 0; i < 3; ++i) { F.pa[i] = pl.pa[i]; F.pb[i] = pl.pb[i]; }
    F.npow = pl.npow;
    F.phase = 0; F.n_ttiles = (int)cdiv(nc, 128); F.n_vranges = pl.f_nvr;
    F.tiles_per_range = pl.f_tpr; F.n_vtiles = pl.n_vtiles;
    F.partial = part; F.rowp = rowp;
    F.Lout = L; F.ldL = ldL; F.tcolL = nP; F.store_t = pl.store_t;
    F.student_ring = pl.f_sring ? 1 : 0;
    F.W8 = w8; F.hs8 = hs8; F.ht8 = ht8; F.eW = ew; F.eS = es; F.eT = et;
    if (pl.f_sring) F.n_ttiles = (int)cdiv(nc, 256);
    // teacher logits from memory are no GEMM
    bool tgemm = pl.tsrc == TSRC_SHARED || pl.tsrc == TSRC_SEP;
    if (pl.f_tl) {
      // the chunk's teacher logits go to L[:, nP + t] (vocabulary-major) ahead
      // of the scan (teacher GEMM, transpose) or through it
      char* Lt = L + nP * eb;
      const bool same_dtype = p->logits_dtype == p->dtype;
      if (pl.f_tmem || (pl.tsrc == TSRC_MEM && same_dtype && V % 4 == 0 && V <= 65535 * 64 &&
                        reinterpret_cast<uintptr_t>(t->teacher_logits) % 8 == 0)) {
        // read token-major by the scan itself (8-byte loads of 4 rows through
        // a buffer resource over 256 tokens: 256 V sizeof(T) < 2^31), which
        // writes them to L on the way
        F.tsrc = TSRC_MEM_RING;
      } else if (pl.tsrc == TSRC_MEM && same_dtype) {
        Timed tm_(ORDA_K_AUX, s, 0.0, 0.0);
        ORDA_CHECK_LAUNCH(launch_transpose<T>(Ltc, V, Lt, ldL, nc, V, s));
      } else if (pl.tsrc == TSRC_MEM) {
        // logits of another dtype: cast to the compute dtype on the way into
        // L, as the reference casts each chunk (ops/precomputed_teacher.py:343-348)
        Timed tm_(ORDA_K_AUX, s, 0.0, 0.0);
        ORDA_CHECK_LAUNCH(launch_transpose_cast<T>(Ltc, p->logits_dtype, V, Lt, ldL, nc, V, s));
      } else {
        ORDA_TRY(gemm2<T>(KMAJ, KMAJ, Wt, Ht, ht + r0 * Ht, Ht, nullptr, 0, Ht, Ht, 0, Lt, nullptr, ldL, V, nc, Ht,
                          GEMM_STORE, 1, 0, s, ORDA_K_SCAN, 2.0 * (double)nc * (double)V * (double)Ht));
      }
      if (F.tsrc != TSRC_MEM_RING) F.tsrc = TSRC_L;
      F.n_ttiles = (int)cdiv(nc, 256);
      tgemm = false;
    }
    const double scan_flops = 2.0 * (double)nc * (double)V * ((double)H + (tgemm ? (double)Ht : 0.0));
    if (pl.f8) {
      if (F.tsrc != TSRC_SHARED && F.tsrc != TSRC_MEM_RING && F.tsrc != TSRC_NONE)
        return fail(ORDA_EUNSUPPORTED, "ORDA_FP8_LOGITS: this teacher's logits do not reach the fp8 ring scan");
      if constexpr (sizeof(T) == 2) {
        Timed tm_(ORDA_K_SCAN, s, scan_flops, scan_flops);
        ORDA_CHECK_LAUNCH(launch_scan_store_f8<T>(F, F.n_ttiles * pl.f_nvr, s));
      } else {
        return fail(ORDA_EUNSUPPORTED, "ORDA_FP8_LOGITS needs a 16-bit compute dtype");
      }
    } else {
      Timed tm_(ORDA_K_SCAN, s, scan_flops, scan_flops);
      ORDA_CHECK_LAUNCH(launch_scan_store<T>(F, F.n_ttiles * pl.f_nvr, s));
    }

    MergeParams M{};
    M.partial = part; M.n_vranges = pl.f_nvr; M.N = nc; M.V = V; M.ignore_index = p->ignore_index;
    M.labels = t->labels + r0; M.label_x = labelx; M.phase = 0; M.fam = F.fam; M.div = pl.div;
    M.t_is_one = pl.t1; M.has_t = pl.tsrc != TSRC_NONE; M.teacher_ce = pl.teacher_ce;
    M.div_on = pl.div_on && !pl.topk;  // a top-k teacher's divergence rows come from k_topk_rows
    M.invT = F.invT; M.temperature = p->temperature; M.alpha = p->div_alpha; M.beta = p->div_beta;
    for (int i = 0; i < 3; ++i) { M.pa[i] = pl.pa[i]; M.pb[i] = pl.pb[i]; }
    M.npow = pl.npow; M.rowp = rowp; M.rowv = rowv + r0; M.ldv = N;
    // logits the scan computed in fp32 and stored rounded: the student's, and
    // the teacher's when its GEMM ran inside the scan
    const int round_code = std::is_same<T, bf16>::value ? 1 : std::is_same<T, f16>::value ? 2 : 0;
    M.round_s = round_code;
    M.round_t = tgemm ? round_code : 0;
    M.lse_sT_out = pl.topk ? reinterpret_cast<float*>(ws + pl.off_lse) : nullptr;
    { Timed tm_(ORDA_K_ROWS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_merge(M, s)); }
    M.lse_sT_out = nullptr;
    TopKParams K{};
    if (pl.topk && pl.div_on) {
      // the teacher's k ids: divergence rows and the ids' dlogits share
      K.hs = hsc; K.W = W; K.idx = t->teacher_topk_indices + r0 * p->topk;
      K.lp = t->teacher_topk_logprobs + r0 * p->topk; K.labels = t->labels + r0; K.mean_scale = pl.late_scale ? scal + 2 : scal;
      K.lse_sT = reinterpret_cast<const float*>(ws + pl.off_lse); K.rowp = rowp; K.rowv = rowv + r0; K.ldv = N; K.corr = reinterpret_cast<float*>(ws + pl.off_corr);
      K.L = L; K.ldL = ldL; K.N = nc; K.V = V; K.H = H; K.k = p->topk; K.ignore_index = p->ignore_index;
      K.div = pl.div_on ? pl.div : DIV_FKL; K.invT = F.invT; K.temperature = p->temperature;
      K.w_kl = pl.div_on ? p->kl_weight : 0.f;
      { Timed tm_(ORDA_K_ROWS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_topk_rows<T>(K, s)); }
    }
    if (pl.two_pass) {
      // the two-pass divergences' row sums over the stored logits, then the
      // merge of their partial states into D and the dlogits row constants
      TwoParams Q{};
      Q.L = L; Q.ldL = ldL; Q.tcol = nP; Q.rowp = rowp; Q.partial = part;
      // vocabulary ranges of 64-row multiples, as many as the scan's partial
      // states hold as dense pairs (f_nvr * kNStat / 2)
      Q.N = nc; Q.V = V; Q.div = pl.div;
      Q.rows_per_range = round_up(cdiv(V, (int64_t)pl.f_nvr * (kNStat / 2)), 64);
      Q.n_ranges = (int)cdiv(V, Q.rows_per_range);
      Q.invT = F.invT;
      Q.mix_w = F.mix_w; Q.mix_w1 = F.mix_w1;
      Q.Ltm = pl.f_tmem ? Ltc : nullptr;
      Q.ldtm = V;
      { Timed tm_(ORDA_K_DLOGITS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_two<T>(Q, s)); }
      M.phase = 1; M.two_dense = 1; M.n_vranges = Q.n_ranges;
      { Timed tm_(ORDA_K_ROWS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_merge(M, s)); }
    }

    if (!any_grad) continue;

    DlmParams D{};
    D.L = L; D.ldL = ldL; D.tcol = nP; D.labels = t->labels + r0; D.rowp = rowp; D.mean_scale = pl.late_scale ? scal + 2 : scal;
    D.N = nc; D.V = V; D.ignore_index = p->ignore_index;
    D.div = pl.div; D.t_is_one = pl.t1; D.tgrad = tgrad;
    D.rows_per_block = (int)round_up(std::max<int64_t>(64, cdiv(V, 65535)), 8);  // grid.y stays <= 65535
    D.Ltm = pl.f_tmem ? Ltc : nullptr;
    D.ldtm = V;
    D.invT = F.invT; D.temperature = p->temperature; D.alpha = p->div_alpha; D.beta = p->div_beta;
    D.w_s = p->student_ce_weight; D.w_t = p->teacher_ce_weight; D.w_kl = pl.div_on ? p->kl_weight : 0.f;
    D.no_t = pl.topk ? 1 : 0;
    { Timed tm_(ORDA_K_DLOGITS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_dlm<T>(D, s)); }
    if (pl.topk && pl.div_on) { Timed tm_(ORDA_K_DLOGITS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_topk_scatter<T>(K, s)); }

    // token columns [nc, nP) of L are read by the grad-W GEMM (K = tokens):
    // keep them zero (the matching hidden rows read as zero too)
    if (nc < nP) {
      { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(L, ldL, V, nc, nP, eb, s)); }
      if (pl.store_t) { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(L, ldL, V, nP + nc, 2 * nP, eb, s)); }
    }

    // grad W (+)= dL^T [hs; ht] with both operands K-major over tokens: the
    // chunk's hidden states are transposed into hT (padding columns zero)
    const int wmode = c == 0 ? GEMM_STORE : GEMM_ACC_T;
    auto transpose_chunk = [&](const T* src, int64_t cols, char* dst, int64_t ldd, int64_t col0) -> int {
      { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_transpose<T>(src, cols, dst + col0 * eb, ldd, nc, cols, s)); }
      if (nc < nP) { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(dst, ldd, cols, col0 + nc, col0 + nP, eb, s)); }
      return ORDA_OK;
    };
    if (pl.need_gw) {
      const bool both = tied && pl.w_dlt_t;
      char* hT = ws + pl.off_fhT;
      ORDA_TRY(transpose_chunk(hsc, H, hT, pl.fldh, 0));
      if (both) ORDA_TRY(transpose_chunk(ht + r0 * H, H, hT, pl.fldh, nP));
      const int64_t K = both ? 2 * nP : nP;
      ORDA_TRY(gemm2<T>(KMAJ, KMAJ, L, ldL, hT, pl.fldh, nullptr, 0, K, K, 0, t->grad_weight, nullptr, H, V, H, K,
                        wmode, 1, 0, s, ORDA_K_GEMM_W, 2.0 * (double)V * (double)H * (double)(both ? 2 * nc : nc)));
    }
    if (sep && pl.need_gwt && pl.w_dlt_t) {
      char* htT = ws + pl.off_fhtT;
      ORDA_TRY(transpose_chunk(ht + r0 * Ht, Ht, htT, nP, 0));
      ORDA_TRY(gemm2<T>(KMAJ, KMAJ, static_cast<char*>(L) + nP * eb, ldL, htT, nP, nullptr, 0, nP, nP, 0,
                        t->grad_teacher_weight, nullptr, Ht, V, Ht, nP, wmode, 1, 0, s, ORDA_K_GEMM_W,
                        2.0 * (double)V * (double)Ht * (double)nc));
    }
    // (dst: the chunk's first output row)
    auto grad_hidden = [&](const char* Lcol, const T* Wx, int64_t Hx, T* dst, int splits, int64_t kps) -> int {
      const double fl = 2.0 * (double)nc * (double)Hx * (double)V;
      if (splits <= 1)
        return gemm2<T>(MNMAJ, MNMAJ, Lcol, ldL, Wx, Hx, nullptr, 0, V, V, 0, dst, nullptr, Hx, nc, Hx, V,
                        GEMM_STORE, 1, 0, s, ORDA_K_GEMM_H, fl);
      ORDA_TRY(gemm2<T>(MNMAJ, MNMAJ, Lcol, ldL, Wx, Hx, nullptr, 0, V, V, 0, nullptr, split, Hx, nc, Hx, V,
                        GEMM_SPLIT, splits, kps, s, ORDA_K_GEMM_H, fl));
      Timed tm_(ORDA_K_AUX, s, 0.0, 0.0);
      ORDA_CHECK_LAUNCH(launch_splitk_reduce<T>(split, splits, nc * Hx, dst, Hx, nc, Hx, s));
      return ORDA_OK;
    };
    if (pl.need_dy) {
      // dloss/dy of the chunk's rows; with the norm, then dloss/dgamma and
      // dloss/dx (in place)
      T* dy = pl.need_gs ? static_cast<T*>(t->grad_student_hidden) + r0 * H : reinterpret_cast<T*>(ws + pl.off_dy);
      ORDA_TRY(grad_hidden(L, W, H, dy, pl.splits_s, pl.kps_s));
      if (pl.norm) {
        Nm.dxy = dy;
        if (pl.need_gnw) {
          Nm.gpart = reinterpret_cast<float*>(ws + pl.off_gpart);
          Nm.gacc = reinterpret_cast<float*>(ws + pl.off_gacc);
          Nm.gout = c + 1 == pl.fnchunks ? t->grad_student_norm_weight : nullptr;
          Timed tm_(ORDA_K_AUX, s, 0.0, 0.0);
          ORDA_CHECK_LAUNCH(launch_rmsnorm_dgamma<T>(Nm, s));
        }
        if (pl.need_gs) { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_rmsnorm_bwd<T>(Nm, s)); }
      }
    }
    if (pl.w_dln_t)
      ORDA_TRY(grad_hidden(L + nP * eb, tied ? W : Wt, Ht, static_cast<T*>(t->grad_teacher_hidden) + r0 * Ht,
                           pl.splits_t, pl.kps_t));
  }

  FinalizeParams Z{};
  Z.rowv = rowv; Z.labels = t->labels; Z.N = N; Z.ignore_index = p->ignore_index;
  Z.reduction_sum = reduction_sum; Z.teacher_ce = pl.teacher_ce; Z.div_on = pl.div_on;
  Z.w_s = p->student_ce_weight; Z.w_t = p->teacher_ce_weight; Z.w_kl = p->kl_weight;
  Z.out_loss = t->out_loss; Z.out_ce_s = t->out_student_ce; Z.out_ce_t = t->out_teacher_ce; Z.out_kl = t->out_kl;
  Z.scal = scal;
  { Timed tm_(ORDA_K_ROWS, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_finalize(Z, s)); }

  // requested gradients that no loss term reaches are zero
  if (pl.need_gt && !pl.w_dln_t)
    { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(t->grad_teacher_hidden, Ht, N, 0, Ht, eb, s)); }
  if (sep && pl.need_gwt && !pl.w_dlt_t)
    { Timed tm_(ORDA_K_AUX, s, 0.0, 0.0); ORDA_CHECK_LAUNCH(launch_zero2d(t->grad_teacher_weight, Ht, V, 0, Ht, eb, s)); }
  // fp16: the chunks' dlogits were unscaled; the mean scale once here (the
  // backward applies grad_output)
  if (pl.late_scale && any_grad) ORDA_TRY(scale_grads<T>(pl, t, scal, s));
  return ORDA_OK;
}

// Backward of the ORDA_GRADS_IN_FORWARD mode: gradients *= grad_output.
template <class T>
int run_scale(const Plan& pl, const orda_tensors_t* t, hipStream_t s) {
  return scale_grads<T>(pl, t, t->grad_output, s);
}

// Each gradient pointer is read only when its flag asks for that gradient, so
// a caller that uses none of a later ABI's features may pass a struct that
// ends before their fields (the RMSNorm pointers come last).
int check_grads(const Plan& pl, const orda_tensors_t* t) {
  auto need = [](const void* g, const char* missing) -> int {
    if (!g) return fail(ORDA_EINVAL, missing);
    if (!aligned16(g)) return fail(ORDA_EINVAL, "gradient buffers must be 16-byte aligned");
    return ORDA_OK;
  };
  if (pl.need_gs) ORDA_TRY(need(t->grad_student_hidden, "grad_student_hidden is required"));
  if (pl.need_gw) ORDA_TRY(need(t->grad_weight, "grad_weight is required"));
  if (pl.need_gt) ORDA_TRY(need(t->grad_teacher_hidden, "grad_teacher_hidden is required"));
  if (pl.need_gwt) ORDA_TRY(need(t->grad_teacher_weight, "grad_teacher_weight is required"));
  if (pl.need_gnw) ORDA_TRY(need(t->grad_student_norm_weight, "grad_student_norm_weight is required"));
  return ORDA_OK;
}

int check_operands(const Plan& pl, const orda_tensors_t* t) {
  if (!t) return fail(ORDA_EINVAL, "tensors is NULL");
  if (!t->student_hidden || !t->weight || !t->labels) return fail(ORDA_EINVAL, "student_hidden, weight and labels are required");
  if (!aligned16(t->student_hidden) || !aligned16(t->weight)) return fail(ORDA_EINVAL, "student_hidden and weight must be 16-byte aligned");
  if (pl.tsrc == TSRC_SHARED && !t->teacher_hidden) return fail(ORDA_EINVAL, "tied mode needs teacher_hidden");
  if (pl.tsrc == TSRC_SEP && (!t->teacher_hidden || !t->teacher_weight))
    return fail(ORDA_EINVAL, "teacher_hidden and teacher_weight are required");
  if ((pl.tsrc == TSRC_SHARED || pl.tsrc == TSRC_SEP) && !aligned16(t->teacher_hidden))
    return fail(ORDA_EINVAL, "teacher_hidden must be 16-byte aligned");
  if (pl.tsrc == TSRC_SEP && !aligned16(t->teacher_weight)) return fail(ORDA_EINVAL, "teacher_weight must be 16-byte aligned");
  if (pl.tsrc == TSRC_MEM && !t->teacher_logits) return fail(ORDA_EINVAL, "teacher_logits are required");
  if (pl.norm && (!t->student_norm_weight || !aligned16(t->student_norm_weight)))
    return fail(ORDA_EINVAL, "student_norm_weight is required (16-byte aligned) with ORDA_STUDENT_RMSNORM");
  if (pl.topk && (!t->teacher_topk_indices || !t->teacher_topk_logprobs))
    return fail(ORDA_EINVAL, "teacher_topk_indices and teacher_topk_logprobs are required");
  if (!t->saved) return fail(ORDA_EINVAL, "saved buffer is required");
  return ORDA_OK;
}

// Scratch of orda_forward_static, the entry point for callers that cannot
// allocate (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc).  One array per device, created with the library's code object
// on that device and held until the process ends; every call on a device
// shares it, so calls that overlap on one device race.  Host code never uses
// the array's name as an address: the device address comes from
// hipGetSymbolAddress, once per device, with that device current.
constexpr size_t kStaticScratchBytes = ORDA_STATIC_SCRATCH_BYTES;
static __device__ __align__(256) char scratch[kStaticScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
char* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch.
int static_scratch(char** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(ORDA_ELAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(ORDA_EUNSUPPORTED, "device index %d is out of range", dev);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(ORDA_ELAUNCH, "hipGetSymbolAddress(scratch): %s", hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<char*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return ORDA_OK;
}

// orda_forward's work once the plan and the workspace are settled.
int forward_with(const Plan& pl, const orda_problem_t* p, const orda_tensors_t* t, void* workspace,
                 size_t workspace_bytes, void* stream) {
  ORDA_TRY(check_operands(pl, t));
  if (!t->out_loss || !t->out_student_ce || !t->out_teacher_ce || !t->out_kl)
    return fail(ORDA_EINVAL, "forward outputs are required");
  if (!workspace || workspace_bytes < pl.fwd_bytes)
    return fail(ORDA_EWORKSPACE, "forward workspace too small: need %zu bytes, got %zu", pl.fwd_bytes, workspace_bytes);
  char* ws = aligned_base(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (pl.fused) {
    ORDA_TRY(check_grads(pl, t));
    switch (pl.dtype) {
      case ORDA_BF16: return run_fused<bf16>(pl, p, t, ws, s);
      case ORDA_F16: return run_fused<f16>(pl, p, t, ws, s);
      default: return run_fused<float>(pl, p, t, ws, s);
    }
  }
  switch (pl.dtype) {
    case ORDA_BF16: return run_forward<bf16>(pl, p, t, ws, s);
    case ORDA_F16: return run_forward<f16>(pl, p, t, ws, s);
    default: return run_forward<float>(pl, p, t, ws, s);
  }
}

}  // namespace

extern "C" {

int orda_abi_version(void) { return ORDA_ABI_VERSION; }

const char* orda_last_error(void) { return g_err.c_str(); }

size_t orda_saved_bytes(const orda_problem_t* p) {
  Plan pl{};
  if (make_plan(p, pl) != ORDA_OK) return 0;
  return pl.saved_bytes;
}

size_t orda_forward_workspace_bytes(const orda_problem_t* p) {
  Plan pl{};
  if (make_plan(p, pl) != ORDA_OK) return 0;
  return pl.fwd_bytes;
}

size_t orda_backward_workspace_bytes(const orda_problem_t* p) {
  Plan pl{};
  if (make_plan(p, pl) != ORDA_OK) return 0;
  return pl.bwd_bytes;
}

int orda_plan_info(const orda_problem_t* p, orda_plan_info_t* out) {
  g_err.clear();
  if (!out) return fail(ORDA_EINVAL, "out is NULL");
  Plan pl{};
  ORDA_TRY(make_plan(p, pl));
  *out = orda_plan_info_t{};
  out->grads_in_forward = pl.fused ? 1 : 0;
  out->table_entry = pl.fused ? pl.table_entry : -1;
  out->teacher_class = pl.fused ? pl.tclass : -1;
  out->vocab_chunk = pl.Vc;
  out->forward_workspace_bytes = pl.fwd_bytes;
  out->backward_workspace_bytes = pl.bwd_bytes;
  if (pl.fused) {
    // the ring scan runs 16-bit tied teachers (two tokens per lane), teacher
    // logits from memory of the non-power families and 16-bit scans with no
    // teacher (four tokens per lane); the rest the two-stage engine
    const bool ring = pl.tclass == TC_TIED || pl.f_tl || pl.f_sring;
    out->scan_engine = ring ? 1 : 0;
    out->token_chunk = pl.fn;
    out->n_token_chunks = pl.fnchunks;
    out->chunk_scale = pl.chunk_scale;
    out->scan_tokens_per_tile = (pl.f_tl || pl.f_sring) ? 256 : 128;
    out->scan_workgroups = (int)(cdiv(pl.fn, out->scan_tokens_per_tile) * pl.f_nvr);
    out->grad_hidden_splits = pl.splits_s;
    out->grad_teacher_hidden_splits = pl.splits_t;
    out->vocab_rows_per_split = pl.kps_s;
  } else {
    out->scan_engine = 0;
    out->token_chunk = pl.N;
    out->n_token_chunks = 1;
    out->scan_tokens_per_tile = 128;
    out->scan_workgroups = pl.n_ttiles * pl.n_vranges;
  }
  return ORDA_OK;
}

int orda_forward(const orda_problem_t* p, const orda_tensors_t* t, void* workspace, size_t workspace_bytes,
                 void* stream) {
  g_err.clear();
  Plan pl{};
  ORDA_TRY(make_plan(p, pl));
  return forward_with(pl, p, t, workspace, workspace_bytes, stream);
}

int orda_forward_static(const orda_problem_t* p, const orda_tensors_t* t, void* stream) {
  g_err.clear();
  Plan pl{};
  ORDA_TRY(make_plan(p, pl));
  if (pl.fwd_bytes > kStaticScratchBytes)
    return fail(ORDA_EWORKSPACE,
                "orda_forward_static: this problem needs %zu bytes of scratch, more than the %zu of the static "
                "scratch; use orda_forward with a workspace, or a smaller token_chunk",
                pl.fwd_bytes, kStaticScratchBytes);
  char* ws = nullptr;
  ORDA_TRY(static_scratch(&ws));
  return forward_with(pl, p, t, ws, kStaticScratchBytes, stream);
}

int orda_backward(const orda_problem_t* p, const orda_tensors_t* t, void* workspace, size_t workspace_bytes,
                  void* stream) {
  g_err.clear();
  Plan pl{};
  ORDA_TRY(make_plan(p, pl));
  ORDA_TRY(check_operands(pl, t));
  if (!t->grad_output) return fail(ORDA_EINVAL, "grad_output is required");
  ORDA_TRY(check_grads(pl, t));
  if (pl.fused) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (pl.dtype) {
      case ORDA_BF16: return run_scale<bf16>(pl, t, s);
      case ORDA_F16: return run_scale<f16>(pl, t, s);
      default: return run_scale<float>(pl, t, s);
    }
  }
  if (pl.bwd_bytes > 0 && (!workspace || workspace_bytes < pl.bwd_bytes))
    return fail(ORDA_EWORKSPACE, "backward workspace too small: need %zu bytes, got %zu", pl.bwd_bytes, workspace_bytes);
  char* ws = aligned_base(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (pl.dtype) {
    case ORDA_BF16: return run_backward<bf16>(pl, p, t, ws, s);
    case ORDA_F16: return run_backward<f16>(pl, p, t, ws, s);
    default: return run_backward<float>(pl, p, t, ws, s);
  }
}

int orda_scale_gradient(int32_t dtype, void* grad, int64_t numel, const float* factor, void* stream) {
  g_err.clear();
  if (numel < 0) return fail(ORDA_EINVAL, "numel must be >= 0, got %lld", (long long)numel);
  if (numel == 0) return ORDA_OK;
  if (!grad || !factor) return fail(ORDA_EINVAL, "grad and factor are required");
  if (!aligned16(grad)) return fail(ORDA_EINVAL, "grad must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  Timed tm_(ORDA_K_AUX, s, 0.0, 0.0);
  switch (dtype) {
    case ORDA_BF16: ORDA_CHECK_LAUNCH(launch_scale<bf16>(grad, numel, factor, s)); break;
    case ORDA_F16: ORDA_CHECK_LAUNCH(launch_scale<f16>(grad, numel, factor, s)); break;
    case ORDA_F32: ORDA_CHECK_LAUNCH(launch_scale<float>(grad, numel, factor, s)); break;
    default: return fail(ORDA_EINVAL, "unknown dtype %d", dtype);
  }
  return ORDA_OK;
}

int orda_gemm_abt(int32_t dtype, int64_t M, int64_t N, int64_t K, const void* A, const void* B, void* C,
                  void* stream) {
  g_err.clear();
  if (M <= 0 || N <= 0 || K <= 0) return fail(ORDA_EINVAL, "M, N, K must be > 0");
  if (!A || !B || !C) return fail(ORDA_EINVAL, "A, B and C are required");
  if (dtype < ORDA_BF16 || dtype > ORDA_F32) return fail(ORDA_EINVAL, "unknown dtype %d", dtype);
  const int kel = dtype == ORDA_F32 ? 4 : 8;
  if (K % kel != 0) return fail(ORDA_EINVAL, "K must be a multiple of %d", kel);
  if (!aligned16(A) || !aligned16(B)) return fail(ORDA_EINVAL, "A and B must be 16-byte aligned");
  hipStream_t s = static_cast<hipStream_t>(stream);
  switch (dtype) {
    case ORDA_BF16: return gemm<bf16>(A, K, B, K, C, nullptr, N, M, N, K, GEMM_STORE, s);
    case ORDA_F16: return gemm<f16>(A, K, B, K, C, nullptr, N, M, N, K, GEMM_STORE, s);
    default: return gemm<float>(A, K, B, K, C, nullptr, N, M, N, K, GEMM_STORE, s);
  }
}

int orda_gemm(int32_t dtype, int32_t a_mn, int32_t b_mn, int64_t M, int64_t N, int64_t K, const void* A,
              int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc, int32_t splits, void* workspace,
              size_t workspace_bytes, void* stream) {
  g_err.clear();
  if (M <= 0 || N <= 0 || K <= 0) return fail(ORDA_EINVAL, "M, N, K must be > 0");
  if (!A || !B || !C) return fail(ORDA_EINVAL, "A, B and C are required");
  if (dtype < ORDA_BF16 || dtype > ORDA_F32) return fail(ORDA_EINVAL, "unknown dtype %d", dtype);
  if ((a_mn != 0 && a_mn != 1) || (b_mn != 0 && b_mn != 1)) return fail(ORDA_EINVAL, "a_mn and b_mn must be 0 or 1");
  if (splits < 1 || splits > 64) return fail(ORDA_EINVAL, "splits must be in [1, 64]");
  const int kel = dtype == ORDA_F32 ? 4 : 8;
  const int64_t eb = dtype == ORDA_F32 ? 4 : 2;
  // K-major operands load K in 16-byte chunks; MN-major ones load rows in
  // 16-byte chunks: the contiguous extent and the leading dimension must be
  // multiples of a chunk, and the bases 16-byte aligned.
  if (!a_mn && (K % kel || lda % kel || lda < K)) return fail(ORDA_EINVAL, "K-major A needs K and lda multiples of %d, lda >= K", kel);
  if (a_mn && (M % kel || lda % kel || lda < M)) return fail(ORDA_EINVAL, "MN-major A needs M and lda multiples of %d, lda >= M", kel);
  if (!b_mn && (K % kel || ldb % kel || ldb < K)) return fail(ORDA_EINVAL, "K-major B needs K and ldb multiples of %d, ldb >= K", kel);
  if (b_mn && (N % kel || ldb % kel || ldb < N)) return fail(ORDA_EINVAL, "MN-major B needs N and ldb multiples of %d, ldb >= N", kel);
  if (ldc < N || ldc % 4) return fail(ORDA_EINVAL, "ldc must be >= N and a multiple of 4");
  if (!aligned16(A) || !aligned16(B) || !aligned16(C)) return fail(ORDA_EINVAL, "A, B and C must be 16-byte aligned");
  int64_t kps = round_up(cdiv(K, splits), 64);
  const int sp = (int)cdiv(K, kps);
  float* part = nullptr;
  if (sp > 1) {
    if (N % 4) return fail(ORDA_EINVAL, "split-K needs N a multiple of 4");
    const size_t need = (size_t)sp * M * N * 4 + kAlign;
    if (!workspace || workspace_bytes < need)
      return fail(ORDA_EWORKSPACE, "gemm workspace too small: need %zu bytes, got %zu", need, workspace_bytes);
    part = reinterpret_cast<float*>(aligned_base(workspace));
  }
  (void)eb;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int la = a_mn ? MNMAJ : KMAJ, lb = b_mn ? MNMAJ : KMAJ;
  auto go = [&](auto tag) -> int {
    using T = decltype(tag);
    if (sp == 1)
      return gemm2<T>(la, lb, A, lda, B, ldb, nullptr, 0, K, K, 0, C, nullptr, ldc, M, N, K, GEMM_STORE, 1, 0, s,
                      ORDA_K_AUX, 0.0);
    if (la != MNMAJ || lb != MNMAJ) return fail(ORDA_EUNSUPPORTED, "split-K is built for MN-major A and B");
    ORDA_TRY(gemm2<T>(la, lb, A, lda, B, ldb, nullptr, 0, K, K, 0, nullptr, part, N, M, N, K, GEMM_SPLIT, sp, kps,
                      s, ORDA_K_AUX, 0.0));
    ORDA_CHECK_LAUNCH(launch_splitk_reduce<T>(part, sp, M * N, C, ldc, M, N, s));
    return ORDA_OK;
  };
  switch (dtype) {
    case ORDA_BF16: return go(bf16{});
    case ORDA_F16: return go(f16{});
    default: return go(float{});
  }
}

int orda_timing_enable(int enable) {
  std::lock_guard<std::mutex> lk(g_timing_mu);
  g_timing = enable != 0;
  if (enable) {
    for (auto& r : g_launches) { g_event_pool.push_back(r.start); g_event_pool.push_back(r.stop); }
    g_launches.clear();
  }
  return ORDA_OK;
}

int orda_timing_collect(orda_timing_t* out) {
  g_err.clear();
  if (!out) return fail(ORDA_EINVAL, "out is NULL");
  std::lock_guard<std::mutex> lk(g_timing_mu);
  *out = orda_timing_t{};
  for (auto& r : g_launches) {
    if (hipEventSynchronize(r.stop) != hipSuccess) return fail(ORDA_ELAUNCH, "hipEventSynchronize failed");
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.start, r.stop) != hipSuccess) return fail(ORDA_ELAUNCH, "hipEventElapsedTime failed");
    if (r.kind >= 0 && r.kind < ORDA_K_COUNT) {
      out->launches[r.kind] += 1;
      out->milliseconds[r.kind] += ms;
      out->algorithmic_flops[r.kind] += r.alg;
      out->executed_flops[r.kind] += r.exe;
    }
    g_event_pool.push_back(r.start);
    g_event_pool.push_back(r.stop);
  }
  g_launches.clear();
  return ORDA_OK;
}

}  // extern "C"
