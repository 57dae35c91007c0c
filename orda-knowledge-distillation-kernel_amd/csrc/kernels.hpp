// kernels.hpp -- kernel templates of liborda_ce.so, instantiated per element
// type by k_{scan,dl,gemm}_{bf16,f16,f32}.hip.
#pragma once

#include "launch.hpp"
#include "orda_core.hpp"
#include "ring4.hpp"
#include "ring4_f8.hpp"
#include "ring16.hpp"

namespace orda {

constexpr float kMinNormal = 1.17549435e-38f;  // 2^-126

// 1 / x on the hardware reciprocal (v_rcp_f32); x a normal float.
__device__ __forceinline__ float frcp(float x) { return __builtin_amdgcn_rcpf(x); }

// Per-element divergence gradient dD/dz_s (z = x/T) given normalised log
// probabilities at temperature T and the row constants c[] from the merge.
// The two-pass divergences form their mixture m in linear space from the
// probabilities (log m = log(w p + (1 - w) q)); an element whose mixture
// underflows (both probabilities below 2^-126) has a zero gradient.
template <int DIV>
__device__ __forceinline__ float div_grad(float lps, float lpt, float psT, float ptT,
                                          const float* c, float alpha, float beta) {
  if constexpr (DIV == DIV_FKL || DIV == DIV_SOFT) {
    return psT - ptT;
  } else if constexpr (DIV == DIV_RKL) {
    return psT * (lps - lpt - c[0]);
  } else if constexpr (DIV == DIV_SYM) {
    return psT - ptT + psT * (lps - lpt - c[0]);
  } else if constexpr (DIV == DIV_HELL) {
    return -0.5f * (fexp(0.5f * (lpt + lps)) - psT * fexp(c[0]));
  } else if constexpr (DIV == DIV_BHAT) {
    return -0.5f * (fexp(0.5f * (lpt + lps) - c[0]) - psT);
  } else if constexpr (DIV == DIV_RENYI) {
    return -(fexp(alpha * lpt + (1.0f - alpha) * lps - c[0]) - psT);
  } else if constexpr (DIV == DIV_AMARI) {
    return -(fexp(alpha * lpt + (1.0f - alpha) * lps) - psT * fexp(c[0])) / alpha;
  } else if constexpr (DIV == DIV_CHI2) {
    return -(fexp(2.0f * lpt - lps) - psT * fexp(c[0]));
  } else if constexpr (DIV == DIV_L2) {
    return 2.0f * (psT * psT - psT * fexp(c[1])) - 2.0f * (ptT * psT - psT * fexp(c[2]));
  } else if constexpr (DIV == DIV_AB) {
    const float q1 = fexp(alpha * lpt + beta * lps);
    const float q3 = fexp((alpha + beta) * lps);
    return -((q1 - psT * fexp(c[0])) - (q3 - psT * fexp(c[2]))) / alpha;
  } else if constexpr (DIV == DIV_JSD) {
    const float m = beta * ptT + (1.0f - beta) * psT;
    const bool ok = m >= kMinNormal;
    return ok ? (1.0f - beta) * psT * (lps - flog(ok ? m : 1.0f) - c[1]) : 0.0f;
  } else if constexpr (DIV == DIV_SKEW_F) {
    const float m = alpha * ptT + (1.0f - alpha) * psT;
    const bool ok = m >= kMinNormal;
    return ok ? -(1.0f - alpha) * psT * (ptT * frcp(ok ? m : 1.0f) - c[1]) : 0.0f;
  } else if constexpr (DIV == DIV_SKEW_R) {
    const float m = alpha * psT + (1.0f - alpha) * ptT;
    const bool ok = m >= kMinNormal;
    const float mm = ok ? m : 1.0f;
    return ok ? psT * (lps - flog(mm) - alpha * psT * frcp(mm) - c[0] + alpha * c[1]) : 0.0f;
  } else {  // DIV_TVD
    const float sg = (psT > ptT) ? 1.0f : ((psT < ptT) ? -1.0f : 0.0f);
    return 0.5f * psT * (sg - c[1]);
  }
}

// ------------------------------------------------------------- shared GEMMs
// Logits of one fused tile (256 vocabulary rows x 128 tokens): acc[.][0] =
// student logits (W rows v0.. x hs rows t0..), acc[.][1] = teacher logits of
// the same tokens (tied: same W x teacher hidden; separate: W_t x teacher
// hidden; precomputed logits: loaded from memory).
template <class T>
__device__ __forceinline__ void fused_logits(f32x16 (&acc)[4][2], char* lds, const FusedParams& P,
                                             int64_t v0, int64_t t0) {
  zero_acc(acc);
  const T* W = static_cast<const T*>(P.W);
  const T* hs = static_cast<const T*>(P.hs);
  const int64_t arows = P.V - v0, brows = P.N - t0;
  if (P.tsrc == TSRC_SHARED) {
    const T* ht = static_cast<const T*>(P.ht);
    mainloop<T, true, true>(acc, lds, W + v0 * P.H, P.H, arows, hs + t0 * P.H, P.H, brows,
                            ht + t0 * P.H, P.H, brows, P.H);
  } else {
    mainloop<T, true, false>(acc, lds, W + v0 * P.H, P.H, arows, hs + t0 * P.H, P.H, brows,
                             nullptr, 0, 0, P.H);
    if (P.tsrc == TSRC_SEP) {
      const T* Wt = static_cast<const T*>(P.Wt);
      const T* ht = static_cast<const T*>(P.ht);
      mainloop<T, false, true>(acc, lds, Wt + v0 * P.Ht, P.Ht, arows, nullptr, 0, 0,
                               ht + t0 * P.Ht, P.Ht, brows, P.Ht);
    } else if (P.tsrc == TSRC_MEM) {
      // Teacher logits [N x V] from memory into the unused teacher block.
      const int lane = threadIdx.x & 63;
      const int wm = wave_m(), wn = wave_n();
      const int64_t t = t0 + wn * 32 + (lane & 31);
      if (t < P.N) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int64_t v = v0 + wm * 128 + acc_row(mb, g * 4, lane);
            const int64_t off = t * P.V + v;
            float x[4];
            if (P.lt_dtype == DT_F32) {
              const float* src = static_cast<const float*>(P.Lt) + off;
#pragma unroll
              for (int e = 0; e < 4; ++e) x[e] = (v + e < P.V) ? src[e] : 0.f;
            } else if (P.lt_dtype == DT_BF16) {
              const bf16* src = static_cast<const bf16*>(P.Lt) + off;
#pragma unroll
              for (int e = 0; e < 4; ++e) x[e] = (v + e < P.V) ? (float)src[e] : 0.f;
            } else {
              const f16* src = static_cast<const f16*>(P.Lt) + off;
#pragma unroll
              for (int e = 0; e < 4; ++e) x[e] = (v + e < P.V) ? (float)src[e] : 0.f;
            }
            // logits of another dtype as the compute dtype T holds them (the
            // reference casts them per chunk; exact when the dtypes agree)
#pragma unroll
            for (int e = 0; e < 4; ++e) x[e] = to_f32(from_f32<T>(x[e]));
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mb][1][g * 4 + e] = x[e];
          }
      }
    }
  }
}

// ------------------------------------------------------------- scan kernel
// Where a lane's values of one token sit in the tile: kMB x kR accumulator
// elements (mb, r) at vocabulary row vlane0 + row(mb, r) (vlane0: the lane's
// first row).  32x32 blocks: 4 blocks x 16 elements, rows 8 (r / 4) + r % 4
// apart within a block; 16x16 blocks: 8 blocks x 4 consecutive rows.
struct Layout32 {
  static constexpr int kMB = 4, kR = 16;
  __device__ static constexpr int row(int mb, int r) { return mb * 32 + (r >> 2) * 8 + (r & 3); }
};
struct Layout16 {
  static constexpr int kMB = 8, kR = 4;
  __device__ static constexpr int row(int mb, int r) { return mb * 16 + r; }
};

// Logit accessors for the scan epilogues: s(mb, r) / t(mb, r) = student /
// teacher logit of the lane's token at accumulator element (mb, r) of the
// tile, laid out as Lay says.
struct AccPair2 {  // two-stage engine: acc[mb][0] student, acc[mb][1] teacher
  using Lay = Layout32;
  const f32x16 (&a)[4][2];
  __device__ __forceinline__ float s(int mb, int r) const { return a[mb][0][r]; }
  __device__ __forceinline__ float t(int mb, int r) const { return a[mb][1][r]; }
};
struct AccPair4 {  // ring engine, the lane's token j: acc[mb][j] student, acc[mb][j + 2] teacher
  using Lay = Layout32;
  const Acc4& a;
  int j;
  __device__ __forceinline__ float s(int mb, int r) const { return acc_get(a[mb][j], r); }
  __device__ __forceinline__ float t(int mb, int r) const { return acc_get(a[mb][j + 2], r); }
};

// Between a tile's two passes over an accessor's values: nothing, except for
// accessors that convert packed registers on each read (AccPairTL), which
// fence them so the converted values are formed again instead of kept live
// across the passes.
template <class AP>
__device__ __forceinline__ void acc_fence(const AP&) {}

// Phase 0: online softmax statistics of this lane's token over its
// vocabulary rows of the tile (64 or 32, AP::Lay).  Template flags remove work that the problem
// does not need (NPOW: the power family's terms, 1 or up to 3, P.npow).
template <bool HAS_T, int FAM, bool T1, bool MASK, class AP, int NPOW = 3>
__device__ __forceinline__ void scan_tile(RowState& S, const AP& acc, int vlane0, int64_t vlimit,
                                          const FusedParams& P) {
  const float invT = P.invT;
  float tms = -kInf, tmt = -kInf, tmu0 = -kInf, tmu1 = -kInf, tmu2 = -kInf;
#pragma unroll
  for (int mb = 0; mb < AP::Lay::kMB; ++mb)
#pragma unroll
    for (int r = 0; r < AP::Lay::kR; ++r) {
      if (MASK && vlane0 + AP::Lay::row(mb, r) >= vlimit) continue;
      const float xs = acc.s(mb, r);
      tms = fmaxf(tms, xs);
      if (HAS_T) {
        const float xt = acc.t(mb, r);
        tmt = fmaxf(tmt, xt);
        if (FAM == FAM_POW) {
          tmu0 = fmaxf(tmu0, P.pa[0] * xt + P.pb[0] * xs);
          if (NPOW > 1 && P.npow > 1) tmu1 = fmaxf(tmu1, P.pa[1] * xt + P.pb[1] * xs);
          if (NPOW > 2 && P.npow > 2) tmu2 = fmaxf(tmu2, P.pa[2] * xt + P.pb[2] * xs);
        }
      }
    }
  if (MASK && tms == -kInf) return;  // no valid vocabulary row in this lane
  acc_fence(acc);

  // rescale the running state to the new maxima
  const float nms = fmaxf(S.ms, tms);
  {
    const float d = S.ms - nms;
    const float cs = fexp(d);
    const float csT = T1 ? cs : fexp(d * invT);
    S.ss *= cs;
    if (!T1) S.sst *= csT;
    if (FAM == FAM_LIN) S.x[1] *= csT;
    S.ms = nms;
  }
  float nmt = 0.f;
  if (HAS_T) {
    nmt = fmaxf(S.mt, tmt);
    const float d = S.mt - nmt;
    const float ct = fexp(d);
    const float ctT = T1 ? ct : fexp(d * invT);
    if (FAM == FAM_LIN) {
      const float so = T1 ? S.st : S.stt;
      S.x[0] *= ctT;
      S.x[2] = (so == 0.f) ? 0.f : ctT * (S.x[2] + d * invT * so);
    }
    S.st *= ct;
    if (!T1) S.stt *= ctT;
    S.mt = nmt;
  }
  float nmu0 = 0.f, nmu1 = 0.f, nmu2 = 0.f;
  if (FAM == FAM_POW) {
    nmu0 = fmaxf(S.x[0], tmu0 * invT);
    S.x[1] *= fexp(S.x[0] - nmu0);
    S.x[0] = nmu0;
    if (NPOW > 1 && P.npow > 1) {
      nmu1 = fmaxf(S.x[2], tmu1 * invT);
      S.x[3] *= fexp(S.x[2] - nmu1);
      S.x[2] = nmu1;
    }
    if (NPOW > 2 && P.npow > 2) {
      nmu2 = fmaxf(S.x[4], tmu2 * invT);
      S.x[5] *= fexp(S.x[4] - nmu2);
      S.x[4] = nmu2;
    }
  }

  // accumulate this tile.  exp(x - m) = 2^(x log2e - m log2e): one fma forms
  // the exponent; the teacher's log-ratio sum (x[2]) is taken in that base-2
  // exponent and scaled by ln 2 once per tile.
  const float ms2 = nms * kLog2e, mt2 = nmt * kLog2e;
  const float cT = invT * kLog2e, msT2 = nms * cT, mtT2 = nmt * cT;
  float lx2 = 0.f;
#pragma unroll
  for (int mb = 0; mb < AP::Lay::kMB; ++mb)
#pragma unroll
    for (int r = 0; r < AP::Lay::kR; ++r) {
      if (MASK && vlane0 + AP::Lay::row(mb, r) >= vlimit) continue;
      const float xs = acc.s(mb, r);
      const float es = __builtin_amdgcn_exp2f(fmaf(xs, kLog2e, -ms2));
      S.ss += es;
      const float esT = T1 ? es : __builtin_amdgcn_exp2f(fmaf(xs, cT, -msT2));
      if (!T1) S.sst += esT;
      if (HAS_T) {
        const float xt = acc.t(mb, r);
        const float at = fmaf(xt, kLog2e, -mt2);
        const float et = __builtin_amdgcn_exp2f(at);
        S.st += et;
        const float atT = T1 ? at : fmaf(xt, cT, -mtT2);
        const float etT = T1 ? et : __builtin_amdgcn_exp2f(atT);
        if (!T1) S.stt += etT;
        if (FAM == FAM_LIN) {
          const float zd = T1 ? xt - xs : (xt - xs) * invT;
          S.x[0] += etT * zd;
          S.x[1] -= esT * zd;
          lx2 += etT * atT;
        }
        if (FAM == FAM_POW) {
          S.x[1] += fexp((P.pa[0] * xt + P.pb[0] * xs) * invT - nmu0);
          if (NPOW > 1 && P.npow > 1) S.x[3] += fexp((P.pa[1] * xt + P.pb[1] * xs) * invT - nmu1);
          if (NPOW > 2 && P.npow > 2) S.x[5] += fexp((P.pa[2] * xt + P.pb[2] * xs) * invT - nmu2);
        }
      }
    }
  if (HAS_T && FAM == FAM_LIN) S.x[2] += lx2 * kLn2;
}

// Phase-1 terms of the two-pass divergences for one vocabulary element,
// from normalised log-probabilities at temperature T.  w, w1: the mixture
// weight (beta for JSD, alpha for the skew KLs) and 1 - w.  The mixture m is
// formed in linear space (one log instead of a log-sum-exp); an element whose
// mixture underflows (both probabilities below 2^-126) adds nothing.
//   JSD:    x0 += p_t (l_t - l_m), x1 += p_s (l_s - l_m), m = b p_t + (1-b) p_s
//   skew-F: x0 += p_t (l_t - l_m), x1 += p_s p_t / m,     m = a p_t + (1-a) p_s
//   skew-R: x0 += p_s (l_s - l_m), x1 += p_s p_s / m,     m = a p_s + (1-a) p_t
//   TVD:    x0 += |p_t - p_s|,     x1 += p_s sign(p_s - p_t)
// and, as second passes of the three-term power divergences over a staged or
// in-place teacher (w = alpha, w1 = beta for AB):
//   L2:     x0 += (p_t - p_s)^2,   x1 += p_s (p_s - p_t)
//   AB:     x0 += q1 - a/(a+b) q2 - b/(a+b) q3,  x1 += q1 - q3,
//           q1 = p_t^a p_s^b, q2 = p_t^(a+b), q3 = p_s^(a+b)
// (x1: the row constant of the divergence's gradient).
template <int DIV>
__device__ __forceinline__ void two_term(float lps, float lpt, float w, float w1, float& s0, float& s1) {
  if constexpr (DIV == DIV_AB) {
    const float ab = w + w1;
    const float q1 = fexp(w * lpt + w1 * lps), q2 = fexp(ab * lpt), q3 = fexp(ab * lps);
    s0 += q1 - (w / ab) * q2 - (w1 / ab) * q3;
    s1 += q1 - q3;
    return;
  }
  const float ps = fexp(lps), pt = fexp(lpt);
  if constexpr (DIV == DIV_L2) {
    const float d = ps - pt;
    s0 += d * d;
    s1 += ps * d;
  } else if constexpr (DIV == DIV_TVD) {
    s0 += fabsf(pt - ps);
    s1 += (ps > pt) ? ps : ((ps < pt) ? -ps : 0.f);
  } else {
    const float m = DIV == DIV_SKEW_R ? w * ps + w1 * pt : w * pt + w1 * ps;
    const bool ok = m >= kMinNormal;
    const float mm = ok ? m : 1.f;
    if constexpr (DIV == DIV_JSD) {
      const float lm = flog(mm);
      s0 += ok ? pt * (lpt - lm) : 0.f;
      s1 += ok ? ps * (lps - lm) : 0.f;
    } else if constexpr (DIV == DIV_SKEW_F) {
      s0 += ok ? pt * (lpt - flog(mm)) : 0.f;
      s1 += ok ? ps * pt * frcp(mm) : 0.f;
    } else {  // DIV_SKEW_R
      s0 += ok ? ps * (lps - flog(mm)) : 0.f;
      s1 += ok ? ps * ps * frcp(mm) : 0.f;
    }
  }
}

template <int DIV, bool MASK, class AP>
__device__ __forceinline__ void rowsum_tile(RowState& S, const AP& acc, int vlane0, int64_t vlimit,
                                            float lse_sT, float lse_tT, const FusedParams& P) {
  const float invT = P.invT;
  float s0 = 0.f, s1 = 0.f;
#pragma unroll
  for (int mb = 0; mb < AP::Lay::kMB; ++mb)
#pragma unroll
    for (int r = 0; r < AP::Lay::kR; ++r) {
      if (MASK && vlane0 + AP::Lay::row(mb, r) >= vlimit) continue;
      const float lps = acc.s(mb, r) * invT - lse_sT;
      const float lpt = acc.t(mb, r) * invT - lse_tT;
      two_term<DIV>(lps, lpt, P.mix_w, P.mix_w1, s0, s1);
    }
  S.x[0] += s0;
  S.x[1] += s1;
}

// Exchange a RowState with lane l^32 of the same wave.
__device__ __forceinline__ RowState shfl32(const RowState& s) {
  RowState o;
  o.ms = __shfl_xor(s.ms, 32); o.ss = __shfl_xor(s.ss, 32);
  o.mt = __shfl_xor(s.mt, 32); o.st = __shfl_xor(s.st, 32);
  o.sst = __shfl_xor(s.sst, 32); o.stt = __shfl_xor(s.stt, 32);
#pragma unroll
  for (int i = 0; i < 6; ++i) o.x[i] = __shfl_xor(s.x[i], 32);
  return o;
}

template <bool PHASE1>
__device__ __forceinline__ void merge_any(RowState& a, const RowState& b, const FusedParams& P) {
  if (PHASE1) {
    a.x[0] += b.x[0];
    a.x[1] += b.x[1];
  } else {
    state_merge(a, b, P.fam, P.t_is_one != 0, P.invT);
  }
}

// Scan variants: which statistics a phase-0 tile accumulates.
enum ScanVariant {
  SV_STUDENT = 0,   // no teacher term
  SV_TCE_T1 = 1,    // teacher softmax only (teacher CE / two-pass lse), T == 1
  SV_TCE = 2,       // same, T != 1
  SV_LIN_T1 = 3,    // forward/reverse/symmetric KL, soft CE, T == 1
  SV_LIN = 4,       // same, T != 1
  SV_POW = 5,       // power-sum divergences
  SV_JSD = 6,       // phase 1 (second pass) of the two-pass divergences
  SV_SKEW_F = 7,
  SV_SKEW_R = 8,
  SV_TVD = 9,
  SV_STUDENT_T = 10,  // no teacher term, the student also at T != 1 (top-k teachers)
  SV_POW1 = 11        // power-sum divergences with one power term (P.npow == 1)
};
// Second-pass variants (row sums given the first pass's normalisers).
constexpr bool sv_phase1(int sv) { return sv >= SV_JSD && sv <= SV_TVD; }

template <int SV, class AP>
__device__ __forceinline__ void scan_variant(RowState& S, const AP& acc, int vlane0, int64_t vlimit,
                                             bool full, float lse_sT, float lse_tT, const FusedParams& P) {
  if constexpr (SV == SV_STUDENT) {
    if (full) scan_tile<false, FAM_NONE, true, false>(S, acc, vlane0, vlimit, P);
    else scan_tile<false, FAM_NONE, true, true>(S, acc, vlane0, vlimit, P);
  } else if constexpr (SV == SV_STUDENT_T) {
    if (full) scan_tile<false, FAM_NONE, false, false>(S, acc, vlane0, vlimit, P);
    else scan_tile<false, FAM_NONE, false, true>(S, acc, vlane0, vlimit, P);
  } else if constexpr (SV == SV_TCE_T1) {
    if (full) scan_tile<true, FAM_NONE, true, false>(S, acc, vlane0, vlimit, P);
    else scan_tile<true, FAM_NONE, true, true>(S, acc, vlane0, vlimit, P);
  } else if constexpr (SV == SV_TCE) {
    if (full) scan_tile<true, FAM_NONE, false, false>(S, acc, vlane0, vlimit, P);
    else scan_tile<true, FAM_NONE, false, true>(S, acc, vlane0, vlimit, P);
  } else if constexpr (SV == SV_LIN_T1) {
    if (full) scan_tile<true, FAM_LIN, true, false>(S, acc, vlane0, vlimit, P);
    else scan_tile<true, FAM_LIN, true, true>(S, acc, vlane0, vlimit, P);
  } else if constexpr (SV == SV_LIN) {
    if (full) scan_tile<true, FAM_LIN, false, false>(S, acc, vlane0, vlimit, P);
    else scan_tile<true, FAM_LIN, false, true>(S, acc, vlane0, vlimit, P);
  } else if constexpr (SV == SV_POW) {
    if (full) scan_tile<true, FAM_POW, false, false>(S, acc, vlane0, vlimit, P);
    else scan_tile<true, FAM_POW, false, true>(S, acc, vlane0, vlimit, P);
  } else if constexpr (SV == SV_POW1) {
    if (full) scan_tile<true, FAM_POW, false, false, AP, 1>(S, acc, vlane0, vlimit, P);
    else scan_tile<true, FAM_POW, false, true, AP, 1>(S, acc, vlane0, vlimit, P);
  } else {
    constexpr int DIV = SV == SV_JSD ? DIV_JSD : SV == SV_SKEW_F ? DIV_SKEW_F : SV == SV_SKEW_R ? DIV_SKEW_R : DIV_TVD;
    if (full) rowsum_tile<DIV, false>(S, acc, vlane0, vlimit, lse_sT, lse_tT, P);
    else rowsum_tile<DIV, true>(S, acc, vlane0, vlimit, lse_sT, lse_tT, P);
  }
}

// Logits of the tile to the vocabulary-major buffer Lout[v][t] (student
// columns from 0, teacher columns from tcolL), in T: the 4 consecutive
// vocabulary rows of a lane are transposed inside the lane quad so each lane
// stores 4 consecutive tokens of one row with one 8-byte (16-bit types) or
// 16-byte (fp32) store.  Every lane of the wave must call this (DPP).
template <class T>
__device__ __forceinline__ void store_logits(const f32x16 (&acc)[4][2], const FusedParams& P, int64_t v0,
                                             int64_t t0) {
  const int lane = opaque_lane();
  const int wm = wave_m(), wn = wave_n();
  const int q = lane & 3;
  const int64_t tb = t0 + wn * 32 + (lane & 31) - q;  // first token of the quad
  const int64_t nt = P.N - tb;
  const int ntok = nt <= 0 ? 0 : (nt >= 4 ? 4 : (int)nt);
  T* L = static_cast<T*>(P.Lout);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t v = v0 + wm * 128 + acc_row(mb, g * 4, lane) + q;
      const bool ok = v < P.V && ntok > 0;
      T* dst = L + v * P.ldL + tb;
      float x[4], o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) x[e] = acc[mb][0][g * 4 + e];
      quad_transpose(x, o);
      if (ok) store4(dst, o, ntok == 4, ntok);
      if (P.store_t) {
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = acc[mb][1][g * 4 + e];
        quad_transpose(x, o);
        if (ok) store4(dst + P.tcolL, o, ntok == 4, ntok);
      }
    }
}

// One workgroup: 128 tokens x a contiguous range of 256-row vocabulary
// tiles; writes one partial RowState per (range, token).  With STORE it also
// writes the tile's logits (store_logits) for the materialised path.
template <class T, int SV, bool STORE = false>
__global__ __launch_bounds__(kThreads) void k_scan(FusedParams P) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  f32x16 acc[4][2];
  constexpr bool kPhase1 = sv_phase1(SV);
  const int lane = threadIdx.x & 63;
  const int wm = wave_m(), wn = wave_n();
  int tt, vr;
  grouped_tile<4>(xcd_order(blockIdx.x, gridDim.x), P.n_ttiles, P.n_vranges, tt, vr);
  const int64_t t0 = (int64_t)tt * 128;
  const int vt_begin = vr * P.tiles_per_range;
  const int vt_end = min(vt_begin + P.tiles_per_range, P.n_vtiles);

  RowState st;
  state_init_fam(st, kPhase1 ? FAM_NONE : P.fam);
  const int64_t tok = t0 + wn * 32 + (lane & 31);
  float lse_sT = 0.f, lse_tT = 0.f;
  if (kPhase1 && tok < P.N) {
    lse_sT = P.rowp[1 * P.N + tok];
    lse_tT = P.rowp[3 * P.N + tok];
  }

  for (int vt = vt_begin; vt < vt_end; ++vt) {
    const int64_t v0 = (int64_t)vt * 256;
    // Opaque copy of the token base: keeps the compiler from hoisting every
    // per-row operand address out of this loop.
    int64_t t0v = t0;
    asm volatile("" : "+s"(t0v));
    fused_logits<T>(acc, lds, P, v0, t0v);
    if constexpr (STORE) store_logits<T>(acc, P, v0, t0v);
    const int vlane0 = wm * 128 + (opaque_lane() >> 5) * 4;
    const int64_t vlimit = P.V - v0;
    scan_variant<SV>(st, AccPair2{acc}, vlane0, vlimit, vlimit >= 256, lse_sT, lse_tT, P);
  }

  // combine lane l with l^32, then the two waves sharing the tokens (wm 0/1)
  {
    const RowState o = shfl32(st);
    merge_any<kPhase1>(st, o, P);
  }
  __syncthreads();
  float* xch = reinterpret_cast<float*>(lds);  // [wn][kNStat][32]
  if (wm == 1 && lane < 32) {
    float* d = xch + (wn * kNStat) * 32 + lane;
    const float* s = reinterpret_cast<const float*>(&st);
#pragma unroll
    for (int f = 0; f < kNStat; ++f) d[f * 32] = s[f];
  }
  __syncthreads();
  if (wm == 0 && lane < 32) {
    RowState o;
    float* od = reinterpret_cast<float*>(&o);
    const float* s = xch + (wn * kNStat) * 32 + lane;
#pragma unroll
    for (int f = 0; f < kNStat; ++f) od[f] = s[f * 32];
    merge_any<kPhase1>(st, o, P);
    if (tok < P.N) {
      float* dst = P.partial + (int64_t)vr * kNStat * P.N + tok;
      const float* sv = reinterpret_cast<const float*>(&st);
#pragma unroll
      for (int f = 0; f < kNStat; ++f) dst[(int64_t)f * P.N] = sv[f];
    }
  }
}

// Logits of a ring-engine tile to Lout[v][t] (see store_logits): block
typedef unsigned int u2v_t __attribute__((ext_vector_type(2)));
typedef unsigned int u4v_t __attribute__((ext_vector_type(4)));
// Workgroup barrier around LDS staging: the wave's LDS accesses complete
// before it, and neither the compiler nor the scheduler moves a memory
// access across it.
__device__ __forceinline__ void stage_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// A buffer resource over [p, p + bytes) with base and size read through
// readfirstlane, so it is scalar (p and bytes are wave-uniform, which the
// compiler cannot always see); bytes < 2^31.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const void* p, int64_t bytes) {
  const uint64_t base = reinterpret_cast<uint64_t>(p);
  const uint64_t ub = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(base >> 32)) << 32) |
                      (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)base);
  return rsrc_bytes(reinterpret_cast<const void*>(ub), __builtin_amdgcn_readfirstlane((int)bytes));
}

// The quad's 4 tokens x 1 row of accumulator block (mb, nb), group g,
// packed and transposed in the quad (lane q of the quad holds row q).
template <class T>
__device__ __forceinline__ uint2 quad_row4(const Acc4& acc, int mb, int nb, int g) {
  uint32_t x[2], o[2];
  x[0] = pack2<T>(acc_get(acc[mb][nb], g * 4 + 0), acc_get(acc[mb][nb], g * 4 + 1));
  x[1] = pack2<T>(acc_get(acc[mb][nb], g * 4 + 2), acc_get(acc[mb][nb], g * 4 + 3));
  quad_transpose16(x, o);
  return make_uint2(o[0], o[1]);
}

// acc[mb][nb] holds vocabulary rows wm * 128 + mb * 32 + acc_row.  Tokens:
// tied (TL false) wn * 64 + (nb & 1) * 32 + lane % 32, student for nb < 2,
// teacher for nb >= 2; student-only tiles (TL) col4(nb, wn) + lane % 32.
// Every store is a full 8-byte one, made by each quad whose first token is
// below N: a quad straddling N writes into the padding columns [N, nP) of its
// half, which the caller zeroes before anything reads them.  (Partial stores
// in the same loop make the compiler split every full store into a 4-byte
// and two 2-byte ones under divergent branches.)
template <class T, bool TL>
__device__ __forceinline__ void store_logits4(const Acc4& acc, const FusedParams& P, int64_t v0, int64_t t0) {
  const int lane = opaque_lane();
  const int wm = w4_m(), wn = w4_n();
  const int q = lane & 3;
  T* L = static_cast<T*>(P.Lout);
  constexpr int kTok = TL ? 256 : 128;
  if (t0 + kTok <= P.N) {
    // Every token of the block is valid: stores through a buffer resource
    // over the tile's rows of L, whose range check drops the rows past V,
    // with 32-bit offsets -- no per-store address arithmetic or guard.
    const int64_t ldb = P.ldL * (int64_t)sizeof(T);
    const int64_t rows = min<int64_t>(P.V - v0, 256);
    const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(L + v0 * P.ldL + t0, rows * ldb);
    const uint32_t lane_off = (uint32_t)(wm * 128 + (lane >> 5) * 4 + q) * (uint32_t)ldb +
                              (uint32_t)(wn * 64 + (lane & 31) - q) * (uint32_t)sizeof(T);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      if (!TL && nb >= 2 && !P.store_t) break;
      const int64_t tok = TL ? (nb >> 1) * 128 + (nb & 1) * 32 : (nb & 1) * 32 + (nb >= 2 ? P.tcolL : 0);
      const uint32_t nb_off = lane_off + (uint32_t)(tok * (int64_t)sizeof(T));
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint2 o = quad_row4<T>(acc, mb, nb, g);
          const u2v_t d = {o.x, o.y};
          __builtin_amdgcn_raw_buffer_store_b64(d, rs, (int)(nb_off + (uint32_t)(mb * 32 + g * 8) * (uint32_t)ldb), 0,
                                                0);
          __builtin_amdgcn_sched_barrier(0);
        }
    }
    return;
  }
#pragma unroll
  for (int nb = 0; nb < 4; ++nb) {
    if (!TL && nb >= 2 && !P.store_t) break;
    const int64_t tb = t0 + (TL ? col4(nb, wn) : wn * 64 + (nb & 1) * 32) + (lane & 31) - q;  // quad's first token
    const bool tok_ok = tb < P.N;
    const int64_t col = tb + (!TL && nb >= 2 ? P.tcolL : 0);
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int64_t v = v0 + wm * 128 + acc_row(mb, g * 4, lane) + q;
        const uint2 o = quad_row4<T>(acc, mb, nb, g);
        if (v < P.V && tok_ok) *reinterpret_cast<uint2*>(L + v * P.ldL + col) = o;
        __builtin_amdgcn_sched_barrier(0);
      }
  }
}

// Teacher logits of the ring scan's student-only tiles (token block nb of the
// lane: 4 x 16 values, rows as in the accumulator) come in two steps: 16 raw
// 8-byte loads (issue_teacher4), then putting them in accumulator order
// (order_teacher4).  Two blocks are in flight ahead of the one being
// scanned.  They stay packed (two 16-bit values per register) and are
// converted where the scan reads them (AccPairTL), which keeps 32 registers
// free for the power family's per-token state.
//  TL_FROM_L: Lout's teacher columns (vocabulary-major): one load holds the
//    quad's 4 tokens of one row; the in-quad transpose (the inverse of
//    store_logits4) gives the lane its token's 4 rows.
//  TL_FROM_MEM: precomputed logits [N x V] (token-major, V a multiple of 4,
//    256 V sizeof(T) < 2^31): one load holds the lane's token's 4
//    consecutive rows directly; the tile then writes them to Lout's teacher
//    columns for the dlogits pass.
// Rows past V and tokens past N read as 0 (the scan masks rows past V;
// tokens past N are never merged).  Loads and stores here are buffer
// instructions over the tile's block of rows, and a lane with nothing to
// move points past the resource (kOob) instead of branching round the
// instruction: every block issues the same 16 instructions, so the waits the
// compiler places before a block's use count exactly the younger ones and
// never the stores or loads of the blocks after it.
enum { TL_NONE = 0, TL_FROM_L = 1, TL_FROM_MEM = 2, TL_STUDENT = 3 };

// Vocabulary-major tile rows of L from v0 (columns from col0): the resource,
// and the lane's byte offset of token block nb (rows wm * 128 + 4 (lane / 32)
// + q, the quad's first token), or kOob when that token is at or past N.
// Row group (mb, g) is then a scalar offset of (mb * 32 + g * 8) rows.
struct TileRowsL {
  __amdgpu_buffer_rsrc_t rs;
  uint32_t ldb;
};
template <class T>
__device__ __forceinline__ TileRowsL tile_rows_l(const void* Lbase, const FusedParams& P, int64_t v0, int64_t col0) {
  TileRowsL r;
  const int64_t ldb = P.ldL * (int64_t)sizeof(T);
  const int64_t rows = min<int64_t>(P.V - v0, 256);
  r.rs = uniform_rsrc(static_cast<const T*>(Lbase) + v0 * P.ldL + col0, rows * ldb);
  r.ldb = (uint32_t)ldb;
  return r;
}
template <class T>
__device__ __forceinline__ uint32_t quad_off_l(const TileRowsL& r, const FusedParams& P, int64_t t0, int nb) {
  const int lane = opaque_lane();
  const int q = lane & 3;
  const int tq = col4(nb, w4_n()) + (lane & 31) - q;  // quad's first token, from t0
  return t0 + tq < P.N ? (uint32_t)(w4_m() * 128 + (lane >> 5) * 4 + q) * r.ldb + (uint32_t)tq * (uint32_t)sizeof(T)
                       : kOob;
}

template <class T, int TL>
__device__ __forceinline__ void issue_teacher4(uint2 (&raw)[16], const FusedParams& P, int64_t v0, int64_t t0,
                                               int nb) {
  const int lane = opaque_lane();
  const int wm = w4_m(), wn = w4_n();
  if constexpr (TL == TL_FROM_L) {
    const TileRowsL r = tile_rows_l<T>(P.Lout, P, v0, P.tcolL + t0);
    const uint32_t off = quad_off_l<T>(r, P, t0, nb);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const u2v_t d = __builtin_amdgcn_raw_buffer_load_b64(r.rs, off, (int)((uint32_t)((i >> 2) * 32 + (i & 3) * 8) * r.ldb), 0);
      raw[i] = make_uint2(d.x, d.y);
    }
  } else {
    // tokens t0 .. t0 + 255 of the [N x V] logits from row v0 on
    const int64_t ntok = min<int64_t>(P.N - t0, 256);
    const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(static_cast<const T*>(P.Lt) + t0 * P.V + v0,
                                                   (ntok * P.V - v0) * (int64_t)sizeof(T));
    const int tk = col4(nb, wn) + (lane & 31);  // the lane's token, from t0
    const int r0 = wm * 128 + (lane >> 5) * 4;  // the lane's row of group 0, from v0
    // offsets formed arithmetically (a select here becomes a branch round
    // each load): kOob or-ed in for a token at or past N, and for rows at or
    // past V (rows r0 + d .. + 3 with d < rowlim are in range, V % 4 == 0)
    const uint32_t dead = (t0 + tk < P.N) ? 0u : kOob;
    const int rowlim = (int)min<int64_t>(P.V - v0 - r0, 1 << 20);
    const uint32_t base = ((uint32_t)tk * (uint32_t)P.V + (uint32_t)r0) * (uint32_t)sizeof(T);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int d = (i >> 2) * 32 + (i & 3) * 8;
      const uint32_t past = (uint32_t)((rowlim - d - 1) >> 31) & kOob;  // d >= rowlim
      const uint32_t off = (base + (uint32_t)d * (uint32_t)sizeof(T)) | past | dead;
      const u2v_t x = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
      raw[i] = make_uint2(x.x, x.y);
    }
  }
}
// In place: raw[i] then holds rows 4 (i % 4) .. + 3 of accumulator block
// i / 4 for the lane's token (element r of block mb: raw[4 mb + r / 4],
// 16-bit value r % 4).
template <class T, int TL>
__device__ __forceinline__ void order_teacher4(uint2 (&raw)[16]) {
  if constexpr (TL == TL_FROM_L) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t x[2] = {raw[i].x, raw[i].y};
      uint32_t o[2];
      quad_transpose16(x, o);
      raw[i] = make_uint2(o[0], o[1]);
    }
  }
}
// Token block nb's teacher logits (ordered raw registers) to Lout's teacher
// columns, as store_logits4 writes a tied teacher's (full 8-byte stores by
// each quad whose first token is below N).
template <class T>
__device__ __forceinline__ void store_teacher4(const uint2 (&tr)[16], const FusedParams& P, int64_t v0, int64_t t0,
                                               int nb) {
  const TileRowsL r = tile_rows_l<T>(P.Lout, P, v0, P.tcolL + t0);
  const uint32_t off = quad_off_l<T>(r, P, t0, nb);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t x[2] = {tr[i].x, tr[i].y};
    uint32_t o[2];
    quad_transpose16(x, o);
    const u2v_t d = {o[0], o[1]};
    __builtin_amdgcn_raw_buffer_store_b64(d, r.rs, off, (int)((uint32_t)((i >> 2) * 32 + (i & 3) * 8) * r.ldb), 0);
  }
}
// Token block nb's student logits of a student-only tile (256 tokens) to
// Lout's student columns: full 8-byte stores by each quad whose first token
// is below N (a quad straddling N writes into the padding columns [N, nP),
// as store_logits4).
template <class T>
__device__ __forceinline__ void store_block4(const Acc4& acc, const FusedParams& P, int64_t v0, int64_t t0, int nb) {
  const TileRowsL r = tile_rows_l<T>(P.Lout, P, v0, t0);
  const uint32_t off = quad_off_l<T>(r, P, t0, nb);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint2 o = quad_row4<T>(acc, mb, nb, g);
      const u2v_t d = {o.x, o.y};
      __builtin_amdgcn_raw_buffer_store_b64(d, r.rs, off, (int)((uint32_t)(mb * 32 + g * 8) * r.ldb), 0);
      __builtin_amdgcn_sched_barrier(0);
    }
}
// A full student-only tile's logits (256 rows x 256 tokens, token column
// col4(nb, wn) + lane % 32 of block nb; every token below N) to Lout's
// student columns t0 .. t0 + 255, staged through the free ring slot `stage`
// (32 KiB) as store_tile16_staged: 4 rounds, round r holding row block r
// of both wave rows (staged row rho = 32 wm + 8 g + 4 (lane / 32) + q, the
// quads' 8-byte rows, 32-byte pieces xor-swizzled by rho % 16), each wave
// then storing 16 staged rows as whole 512-byte rows (lanes 0-15 / 16-31:
// tokens 0-127 / 128-255 of one row, 32-47 / 48-63 the next row).  A
// vocabulary tail beyond V is dropped by the buffer resource.  Ends with a
// workgroup barrier.
template <class T>
__device__ __forceinline__ void store_tile4_staged(const Acc4& acc, const FusedParams& P, int64_t v0, int64_t t0,
                                                   char* stage) {
  typedef __attribute__((address_space(3))) u2v_t lds_u2;
  typedef __attribute__((address_space(3))) u4v_t lds_u4;
  const int lane = opaque_lane();
  const int w = wave_id(), wm = w >> 1, wn = w & 1;
  const int q = lane & 3;
  const TileRowsL tr = tile_rows_l<T>(P.Lout, P, v0, t0);
  const uint32_t wrow = (uint32_t)(wm * 32 + (lane >> 5) * 4 + q);  // + 8 g
  const uint32_t wcol = (uint32_t)(2 * ((lane & 31) - q));
  const int half = (lane >> 4) & 1;
  const uint32_t rrow = (uint32_t)(w * 16 + (lane >> 5));  // + 2 i
  const uint32_t rcol = (uint32_t)(2 * (half * 128 + (lane & 15) * 8));
  const uint32_t gcol = rcol;  // student columns: token c at t0 + c
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int nb = 0; nb < 4; ++nb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint2 o = quad_row4<T>(acc, r, nb, g);
        const uint32_t rho = wrow + (uint32_t)(8 * g);
        const uint32_t col = wcol + (uint32_t)(2 * col4(nb, wn));
        *(lds_u2*)(stage + rho * 512 + (col ^ ((rho & 15) << 5))) = u2v_t{o.x, o.y};
      }
    stage_barrier();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t rho = rrow + (uint32_t)(2 * i);
      const u4v_t v = *(const lds_u4*)(stage + rho * 512 + (rcol ^ ((rho & 15) << 5)));
      const uint32_t trow = (rho >> 5) * 128 + (uint32_t)(32 * r) + (rho & 31);
      __builtin_amdgcn_raw_buffer_store_b128(v, tr.rs, (int)(trow * tr.ldb + gcol), 0, 0);
    }
    stage_barrier();
  }
}
struct AccPairS {  // student only: accumulator block nb (the teacher accessor is never used)
  using Lay = Layout32;
  const Acc4& a;
  int nb;
  __device__ __forceinline__ float s(int mb, int r) const { return acc_get(a[mb][nb], r); }
  __device__ __forceinline__ float t(int, int) const { return 0.f; }
};
template <class T>
struct AccPairTL {  // student from accumulator block nb, teacher from ordered raw registers
  using Lay = Layout32;
  const Acc4& a;
  int nb;
  const uint2 (&tr)[16];
  __device__ __forceinline__ float s(int mb, int r) const { return acc_get(a[mb][nb], r); }
  __device__ __forceinline__ float t(int mb, int r) const {
    const uint2& u = tr[mb * 4 + (r >> 2)];
    const uint32_t w = (r & 2) ? u.y : u.x;
    return (r & 1) ? hi16<T>(w) : lo16<T>(w);
  }
};
template <class T>
__device__ __forceinline__ void acc_fence(const AccPairTL<T>& p) {
  uint2* r = const_cast<uint2*>(p.tr);
#pragma unroll
  for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(r[i].x), "+v"(r[i].y));
}

// k_scan on the four-wave ring engine for 16-bit operands: the same
// workgroup -> (tokens, vocabulary range) mapping and partial output.  The B
// operand is fixed per workgroup; the vocabulary tiles of the range run as
// one persistent ring (pipeline4, MFMAs not swapped).
//  TL false (teacher sharing W, TSRC_SHARED): 128 tokens per workgroup, B =
//    student hidden rows t0.. then the teacher's; each lane holds two tokens,
//    j = 0, 1 at blocks (j, j + 2).
//  TL_FROM_L / TL_FROM_MEM (teacher logits from memory, see
//    issue_teacher4): 256 tokens per workgroup, B = 256 student hidden rows;
//    each lane holds four tokens (blocks 0..3).
template <class T, int SV, bool STORE, int TL, bool F8 = false>
__global__ __launch_bounds__(kThreads4, 1) void k_scan4(FusedParams P) {
  static_assert(TL == TL_NONE || (!sv_phase1(SV) && STORE), "teacher logits from memory: one-pass, stored");
  static_assert(TL != TL_STUDENT || SV == SV_STUDENT || SV == SV_STUDENT_T, "student-only tiles: no teacher");
  constexpr int NJ = TL ? 4 : 2;        // tokens per lane
  constexpr int kTok = TL ? 256 : 128;  // tokens per workgroup
  __shared__ __attribute__((aligned(16))) char lds[kLds4Bytes];
  Acc4 acc;
  zero_acc4(acc);
  constexpr bool kPhase1 = sv_phase1(SV);
  const int lane = threadIdx.x & 63;
  const int wm = w4_m(), wn = w4_n();
  int tt, vr;
  grouped_tile<4>(xcd_order(blockIdx.x, gridDim.x), P.n_ttiles, P.n_vranges, tt, vr);
  const int64_t t0 = (int64_t)tt * kTok;
  const int vt_begin = vr * P.tiles_per_range;
  const int ntiles = min(vt_begin + P.tiles_per_range, P.n_vtiles) - vt_begin;

  RowState st[NJ];
  int64_t tok[NJ];
  float lse_sT[NJ], lse_tT[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    state_init_fam(st[j], kPhase1 ? FAM_NONE : P.fam);
    tok[j] = t0 + (TL ? col4(j, wn) : wn * 64 + j * 32) + (lane & 31);
    lse_sT[j] = lse_tT[j] = 0.f;
    if (kPhase1 && tok[j] < P.N) {
      lse_sT[j] = P.rowp[1 * P.N + tok[j]];
      lse_tT[j] = P.rowp[3 * P.N + tok[j]];
    }
  }
  const T* W = static_cast<const T*>(P.W);
  const T* hs = static_cast<const T*>(P.hs);
  const T* ht = static_cast<const T*>(P.ht);
  KOp4 bop;
  int sb[4];  // fp8: E8M0 scale byte of B row col4(nb, wn) + lane % 32
  if constexpr (F8) {
    const uint8_t* hs8 = static_cast<const uint8_t*>(P.hs8);
    const uint8_t* ht8 = static_cast<const uint8_t*>(P.ht8);
    bop = TL ? kop4(hs8 + t0 * P.H, P.H, P.N - t0)
             : kop4_split(hs8 + t0 * P.H, P.N - t0, ht8 + t0 * P.H, P.N - t0, P.H);
#pragma unroll
    for (int nb = 0; nb < 4; ++nb) {
      const int j = col4(nb, wn) + (lane & 31);
      const bool teacher_row = !TL && j >= 128;
      const int64_t t = t0 + (teacher_row ? j - 128 : j);
      sb[nb] = t < P.N ? (int)(teacher_row ? P.eT : P.eS)[t] : 127;
    }
  } else {
    bop = TL ? kop4(hs + t0 * P.H, P.H, P.N - t0)
             : kop4_split(hs + t0 * P.H, P.N - t0, ht + t0 * P.H, P.N - t0, P.H);
  }
  struct TI {
    int v0;
    KOp4 a;
    int sa[4];  // fp8: E8M0 scale byte of A row wm * 128 + mb * 32 + lane % 32
  };
  auto tile_info = [&](int i) {
    TI x;
    x.v0 = (vt_begin + (i < ntiles ? i : 0)) * 256;
    if constexpr (F8) {
      x.a = kop4(static_cast<const uint8_t*>(P.W8) + (int64_t)x.v0 * P.H, P.H, P.V - x.v0);
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        const int64_t v = x.v0 + wm * 128 + mb * 32 + (lane & 31);
        x.sa[mb] = v < P.V ? (int)P.eW[v] : 127;
      }
    } else {
      x.a = kop4(W + (int64_t)x.v0 * P.H, P.H, P.V - x.v0);
    }
    return x;
  };
  auto opnd = [&](const TI& x, int op) { return op == 0 ? x.a : bop; };
  // (stage: the free ring slot, null from the fp8 pipeline)
  auto epilogue = [&](int, const TI& x, Acc4& c, char* stage = nullptr) __attribute__((always_inline)) {
    const int vlane0 = wm * 128 + (opaque_lane() >> 5) * 4;
    const int64_t vlimit = P.V - x.v0;
    if constexpr (TL == TL_STUDENT) {
      store_logits4<T, true>(c, P, x.v0, t0);
      static_for<0, NJ>([&](auto J) {
        constexpr int j = decltype(J)::value;
        scan_variant<SV>(st[j], AccPairS{c, j}, vlane0, vlimit, vlimit >= 256, lse_sT[j], lse_tT[j], P);
      });
    } else if constexpr (TL != TL_NONE) {
      // blocks j and j + 1 in flight while block j is scanned; block j's
      // student logits stored after its scan (their stores are younger than
      // the loads of block j + 1, so its wait does not cover them)
      // A full tile's student logits go out staged through the free ring
      // slot (whole row pieces) while the first two blocks' loads land.
      const bool staged = stage != nullptr && t0 + 256 <= P.N;
      uint2 raw[2][16];
      issue_teacher4<T, TL>(raw[0], P, x.v0, t0, 0);
      issue_teacher4<T, TL>(raw[1], P, x.v0, t0, 1);
      if (staged) store_tile4_staged<T>(c, P, x.v0, t0, stage);
      static_for<0, NJ>([&](auto J) {
        constexpr int j = decltype(J)::value;
        order_teacher4<T, TL>(raw[j & 1]);
        if constexpr (TL == TL_FROM_MEM) {
          if (P.store_t) store_teacher4<T>(raw[j & 1], P, x.v0, t0, j);  // else the dlogits pass reads them in place
        }
        scan_variant<SV>(st[j], AccPairTL<T>{c, j, raw[j & 1]}, vlane0, vlimit, vlimit >= 256, lse_sT[j], lse_tT[j],
                         P);
        if (!staged) store_block4<T>(c, P, x.v0, t0, j);
        if constexpr (j + 2 < NJ) issue_teacher4<T, TL>(raw[j & 1], P, x.v0, t0, j + 2);
      });
    } else {
      if constexpr (STORE) store_logits4<T, false>(c, P, x.v0, t0);
      static_for<0, NJ>([&](auto J) {
        constexpr int j = decltype(J)::value;
        scan_variant<SV>(st[j], AccPair4{c, j}, vlane0, vlimit, vlimit >= 256, lse_sT[j], lse_tT[j], P);
      });
    }
  };
  if constexpr (F8)
    pipeline4_f8(acc, lds, ntiles, P.H, P.H, P.H, tile_info, opnd, epilogue, sb);
  else
    pipeline4<T, KMAJ, KMAJ, true, true, false>(acc, lds, ntiles, P.H, P.H, P.H, tile_info, opnd, epilogue);

  // combine lane l with l^32 (other vocabulary rows of the same tokens), then
  // the two waves sharing the tokens (wm 0 / 1)
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const RowState o = shfl32(st[j]);
    merge_any<kPhase1>(st[j], o, P);
  }
  __syncthreads();
  float* xch = reinterpret_cast<float*>(lds);  // [wn][j][kNStat][32]
  if (wm == 1 && lane < 32) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float* d = xch + ((wn * NJ + j) * kNStat) * 32 + lane;
      const float* sv = reinterpret_cast<const float*>(&st[j]);
#pragma unroll
      for (int f = 0; f < kNStat; ++f) d[f * 32] = sv[f];
    }
  }
  __syncthreads();
  if (wm == 0 && lane < 32) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      RowState o;
      float* od = reinterpret_cast<float*>(&o);
      const float* sv = xch + ((wn * NJ + j) * kNStat) * 32 + lane;
#pragma unroll
      for (int f = 0; f < kNStat; ++f) od[f] = sv[f * 32];
      merge_any<kPhase1>(st[j], o, P);
      if (tok[j] < P.N) {
        float* dst = P.partial + (int64_t)vr * kNStat * P.N + tok[j];
        const float* v = reinterpret_cast<const float*>(&st[j]);
#pragma unroll
        for (int f = 0; f < kNStat; ++f) dst[(int64_t)f * P.N] = v[f];
      }
    }
  }
}

// ------------------------------------------- tied scan, 16x16x32 MFMAs
// The tied scan (TL_NONE: 128 tokens per workgroup, B = the student's hidden
// rows then the teacher's) on pipeline16.  Wave (wm, wn): vocabulary rows
// wm * 128 .., tokens wn * 64 + 16 j + lane % 16 (j < 4): student block j,
// teacher block j + 4; each lane holds 4 tokens x 32 rows (8 blocks x 4
// consecutive rows from 4 (lane / 16)).
struct AccPair16 {
  using Lay = Layout16;
  const Acc16& a;
  int j;
  __device__ __forceinline__ float s(int mb, int r) const { return acc16_get(a[mb][j], r); }
  __device__ __forceinline__ float t(int mb, int r) const { return acc16_get(a[mb][j + 4], r); }
};

// The quad's 4 tokens x 1 row of block (mb, nb), packed and transposed in the
// quad (lane q of the quad holds row 4 (lane / 16) + q).
template <class T>
__device__ __forceinline__ uint2 quad_row16(const Acc16& acc, int mb, int nb) {
  uint32_t x[2], o[2];
  x[0] = pack2<T>(acc16_get(acc[mb][nb], 0), acc16_get(acc[mb][nb], 1));
  x[1] = pack2<T>(acc16_get(acc[mb][nb], 2), acc16_get(acc[mb][nb], 3));
  quad_transpose16(x, o);
  return make_uint2(o[0], o[1]);
}

// The tile's logits to Lout[v][t] (student columns from 0, teacher columns
// from tcolL when store_t), as store_logits4: full 8-byte stores by each quad
// whose first token is below N (a quad straddling N writes into the padding
// columns [N, nP) of its half).
template <class T>
__device__ __forceinline__ void store_logits16(const Acc16& acc, const FusedParams& P, int64_t v0, int64_t t0) {
  const int lane = opaque_lane();
  const int wm = w4_m(), wn = w4_n();
  const int q = lane & 3;
  T* L = static_cast<T*>(P.Lout);
  if (t0 + 128 <= P.N) {
    const int64_t ldb = P.ldL * (int64_t)sizeof(T);
    const int64_t rows = min<int64_t>(P.V - v0, 256);
    const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(L + v0 * P.ldL + t0, rows * ldb);
    const uint32_t lane_off = (uint32_t)(wm * 128 + (lane >> 4) * 4 + q) * (uint32_t)ldb +
                              (uint32_t)(wn * 64 + (lane & 15) - q) * (uint32_t)sizeof(T);
#pragma unroll
    for (int nb = 0; nb < 8; ++nb) {
      if (nb >= 4 && !P.store_t) break;
      const int64_t tok = (nb & 3) * 16 + (nb >= 4 ? P.tcolL : 0);
      const uint32_t nb_off = lane_off + (uint32_t)(tok * (int64_t)sizeof(T));
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        const uint2 o = quad_row16<T>(acc, mb, nb);
        const u2v_t d = {o.x, o.y};
        __builtin_amdgcn_raw_buffer_store_b64(d, rs, (int)(nb_off + (uint32_t)(mb * 16) * (uint32_t)ldb), 0, 0);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    return;
  }
#pragma unroll
  for (int nb = 0; nb < 8; ++nb) {
    if (nb >= 4 && !P.store_t) break;
    const int64_t tb = t0 + wn * 64 + (nb & 3) * 16 + (lane & 15) - q;  // quad's first token
    const bool tok_ok = tb < P.N;
    const int64_t col = tb + (nb >= 4 ? P.tcolL : 0);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const int64_t v = v0 + wm * 128 + mb * 16 + (lane >> 4) * 4 + q;
      const uint2 o = quad_row16<T>(acc, mb, nb);
      if (v < P.V && tok_ok) *reinterpret_cast<uint2*>(L + v * P.ldL + col) = o;
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// A full tile's logits (256 vocabulary rows x 256 token columns, columns
// col16(nb, wn) + lane % 16 of block nb) to Lout, staged through the free
// ring slot `stage` (32 KiB) so that each store writes whole row pieces.
// Columns 0-127 go to Lout[v][t0 + c], columns 128-255 to Lout[v][t0 +
// second + c - 128] (a tied tile: the teacher's tokens at second = tcolL,
// written only when `both`; a student-only tile: second = 128).  Every token
// of the tile is below N (t0 + 128 <= N tied, t0 + 256 <= N student-only).
// 4 rounds; in round r each wave writes its row blocks 2r and 2r + 1 (32
// rows x its 2 x 64 token columns, the quads' 8-byte rows) into
// 64 staged rows of 256 tokens (512 bytes, row rho at rho * 512, 32-byte
// pieces xor-swizzled by rho % 16 so a write's 16 rows fall on distinct
// banks), then each wave stores 16 staged rows, two per 16-byte store: lanes
// 0-15 / 16-31 / 32-47 / 48-63 write the two column halves (256 bytes
// each) of two rows.  A vocabulary tail beyond V is dropped by the
// buffer resource, as in store_logits16.  Ends with a workgroup barrier.
template <class T>
__device__ __forceinline__ void store_tile16_staged(const Acc16& acc, const FusedParams& P, int64_t v0, int64_t t0,
                                                    int64_t second, bool both, char* stage) {
  typedef __attribute__((address_space(3))) u2v_t lds_u2;
  typedef __attribute__((address_space(3))) u4v_t lds_u4;
  const int lane = opaque_lane();
  const int w = wave_id(), wm = w >> 1, wn = w & 1;
  const int q = lane & 3;
  T* L = static_cast<T*>(P.Lout);
  const uint32_t ldb = (uint32_t)(P.ldL * (int64_t)sizeof(T));
  const int64_t rows = min<int64_t>(P.V - v0, 256);
  const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(L + v0 * P.ldL + t0, rows * (int64_t)ldb);
  char* st = stage;
  // writes: staged row wm * 32 + 16 (mb & 1) + 4 (lane / 16) + q, byte
  // column 2 (128 half + 64 wn + 16 (nb & 3) + 4 ((lane % 16) / 4))
  const uint32_t wrow = (uint32_t)(wm * 32 + (lane >> 4) * 4 + q);  // + 16 (mb & 1)
  const uint32_t wswz = (wrow & 15) << 5;                            // (mb & 1) * 16 leaves rho % 16
  const uint32_t wcol = (uint32_t)(2 * (wn * 64 + 4 * ((lane & 15) >> 2)));
  // reads: staged row w * 16 + 2 i + lane / 32, half (lane / 16) % 2
  const int half = (lane >> 4) & 1;
  const uint32_t rrow = (uint32_t)(w * 16 + (lane >> 5));  // + 2 i
  const uint32_t rcol = (uint32_t)(2 * (half * 128 + (lane & 15) * 8));
  const uint32_t gcol = (uint32_t)((half ? second : 0) + (lane & 15) * 8) * (uint32_t)sizeof(T);
  const bool rlive = both || half == 0;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int mb = 2 * r + h;
      const uint32_t rho = wrow + (uint32_t)(16 * h);
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        if (nb >= 4 && !both) break;
        const uint2 o = quad_row16<T>(acc, mb, nb);
        const uint32_t col = wcol + (uint32_t)(2 * ((nb >= 4 ? 128 : 0) + (nb & 3) * 16));
        *(lds_u2*)(st + rho * 512 + (col ^ wswz)) = u2v_t{o.x, o.y};
      }
    }
    stage_barrier();
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t rho = rrow + (uint32_t)(2 * i);
      if (rlive) {
        const u4v_t v = *(const lds_u4*)(st + rho * 512 + (rcol ^ ((rho & 15) << 5)));
        // tile row (rho / 32) * 128 + 32 r + rho % 32
        const uint32_t trow = (rho >> 5) * 128 + (uint32_t)(32 * r) + (rho & 31);
        __builtin_amdgcn_raw_buffer_store_b128(v, rs, (int)(trow * ldb + gcol), 0, 0);
      }
    }
    stage_barrier();
  }
}

// Exchange a RowState with lane l ^ m of the same wave.
__device__ __forceinline__ RowState shfl_state(const RowState& s, int m) {
  RowState o;
  o.ms = __shfl_xor(s.ms, m); o.ss = __shfl_xor(s.ss, m);
  o.mt = __shfl_xor(s.mt, m); o.st = __shfl_xor(s.st, m);
  o.sst = __shfl_xor(s.sst, m); o.stt = __shfl_xor(s.stt, m);
#pragma unroll
  for (int i = 0; i < 6; ++i) o.x[i] = __shfl_xor(s.x[i], m);
  return o;
}

// Student-only tiles on pipeline16 (TL_FROM_L, TL_FROM_MEM, TL_STUDENT): 256
// student tokens per workgroup, token block nb of wave (wm, wn) is tokens
// col16(nb, wn) .. + 15 (lane % 16), rows wm * 128 + mb * 16 + 4 (lane / 16)
// + e.  As the 32x32 ring's helpers above, with 16-row blocks: the lane's
// byte offset of block nb in a vocabulary-major tile of L (the quad's first
// token, rows 4 (lane / 16) + q), or kOob for a token at or past N.
template <class T>
__device__ __forceinline__ uint32_t quad_off_l16(const TileRowsL& r, const FusedParams& P, int64_t t0, int nb) {
  const int lane = opaque_lane();
  const int q = lane & 3;
  const int tq = col16(nb, w4_n()) + (lane & 15) - q;
  return t0 + tq < P.N ? (uint32_t)(w4_m() * 128 + (lane >> 4) * 4 + q) * r.ldb + (uint32_t)tq * (uint32_t)sizeof(T)
                       : kOob;
}
// Token block nb's teacher logits: 8 raw 8-byte loads (one per 16-row block
// mb), put in accumulator order by order_teacher16 (raw[mb] then holds rows
// 4 (lane / 16) .. + 3 of block mb for the lane's token).
template <class T, int TL>
__device__ __forceinline__ void issue_teacher16(uint2 (&raw)[8], const FusedParams& P, int64_t v0, int64_t t0,
                                                int nb) {
  const int lane = opaque_lane();
  if constexpr (TL == TL_FROM_L) {
    const TileRowsL r = tile_rows_l<T>(P.Lout, P, v0, P.tcolL + t0);
    const uint32_t off = quad_off_l16<T>(r, P, t0, nb);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const u2v_t d = __builtin_amdgcn_raw_buffer_load_b64(r.rs, off, (int)((uint32_t)(mb * 16) * r.ldb), 0);
      raw[mb] = make_uint2(d.x, d.y);
    }
  } else {
    const int64_t ntok = min<int64_t>(P.N - t0, 256);
    const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(static_cast<const T*>(P.Lt) + t0 * P.V + v0,
                                                   (ntok * P.V - v0) * (int64_t)sizeof(T));
    const int tk = col16(nb, w4_n()) + (lane & 15);  // the lane's token, from t0
    const int r0 = w4_m() * 128 + (lane >> 4) * 4;   // the lane's row of block 0, from v0
    const uint32_t dead = (t0 + tk < P.N) ? 0u : kOob;
    const int rowlim = (int)min<int64_t>(P.V - v0 - r0, 1 << 20);
    const uint32_t base = ((uint32_t)tk * (uint32_t)P.V + (uint32_t)r0) * (uint32_t)sizeof(T);
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const int d = mb * 16;
      const uint32_t past = (uint32_t)((rowlim - d - 1) >> 31) & kOob;  // d >= rowlim
      const uint32_t off = (base + (uint32_t)d * (uint32_t)sizeof(T)) | past | dead;
      const u2v_t x = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
      raw[mb] = make_uint2(x.x, x.y);
    }
  }
}
template <class T, int TL>
__device__ __forceinline__ void order_teacher16(uint2 (&raw)[8]) {
  if constexpr (TL == TL_FROM_L) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t x[2] = {raw[i].x, raw[i].y};
      uint32_t o[2];
      quad_transpose16(x, o);
      raw[i] = make_uint2(o[0], o[1]);
    }
  }
}
// Token block nb's teacher logits (ordered) to Lout's teacher columns.
template <class T>
__device__ __forceinline__ void store_teacher16(const uint2 (&tr)[8], const FusedParams& P, int64_t v0, int64_t t0,
                                                int nb) {
  const TileRowsL r = tile_rows_l<T>(P.Lout, P, v0, P.tcolL + t0);
  const uint32_t off = quad_off_l16<T>(r, P, t0, nb);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t x[2] = {tr[i].x, tr[i].y};
    uint32_t o[2];
    quad_transpose16(x, o);
    const u2v_t d = {o[0], o[1]};
    __builtin_amdgcn_raw_buffer_store_b64(d, r.rs, off, (int)((uint32_t)(i * 16) * r.ldb), 0);
  }
}
// Token block nb's student logits to Lout's student columns.
template <class T>
__device__ __forceinline__ void store_block16(const Acc16& acc, const FusedParams& P, int64_t v0, int64_t t0,
                                              int nb) {
  const TileRowsL r = tile_rows_l<T>(P.Lout, P, v0, t0);
  const uint32_t off = quad_off_l16<T>(r, P, t0, nb);
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    const uint2 o = quad_row16<T>(acc, mb, nb);
    const u2v_t d = {o.x, o.y};
    __builtin_amdgcn_raw_buffer_store_b64(d, r.rs, off, (int)((uint32_t)(mb * 16) * r.ldb), 0);
    __builtin_amdgcn_sched_barrier(0);
  }
}
struct AccPair16S {  // student only: block j (the teacher accessor is never used)
  using Lay = Layout16;
  const Acc16& a;
  int j;
  __device__ __forceinline__ float s(int mb, int r) const { return acc16_get(a[mb][j], r); }
  __device__ __forceinline__ float t(int, int) const { return 0.f; }
};
template <class T>
struct AccPair16TL {  // student from block j, teacher from ordered raw registers
  using Lay = Layout16;
  const Acc16& a;
  int j;
  const uint2 (&tr)[8];
  __device__ __forceinline__ float s(int mb, int r) const { return acc16_get(a[mb][j], r); }
  __device__ __forceinline__ float t(int mb, int r) const {
    const uint2& u = tr[mb];
    const uint32_t w = (r & 2) ? u.y : u.x;
    return (r & 1) ? hi16<T>(w) : lo16<T>(w);
  }
};
template <class T>
__device__ __forceinline__ void acc_fence(const AccPair16TL<T>& p) {
  uint2* r = const_cast<uint2*>(p.tr);
#pragma unroll
  for (int i = 0; i < 8; ++i) asm volatile("" : "+v"(r[i].x), "+v"(r[i].y));
}

// k_scan4's tied path (TL_NONE, 16-bit) on pipeline16: the same workgroup ->
// (128 tokens, vocabulary range) mapping, partial output and logits store.
template <class T, int SV, bool STORE, int TL = TL_NONE>
__global__ __launch_bounds__(kThreads4, 1) void k_scan16(FusedParams P) {
  static_assert(TL == TL_NONE || (!sv_phase1(SV) && STORE), "teacher logits from memory: one-pass, stored");
  static_assert(TL != TL_STUDENT || SV == SV_STUDENT || SV == SV_STUDENT_T, "student-only tiles: no teacher");
  constexpr int NJ = TL ? 8 : 4;        // tokens per lane
  constexpr int kTok = TL ? 256 : 128;  // tokens per workgroup
  __shared__ __attribute__((aligned(16))) char lds[kLds4Bytes];
  Acc16 acc;
  zero_acc16(acc);
  constexpr bool kPhase1 = sv_phase1(SV);
  const int lane = threadIdx.x & 63;
  const int wm = w4_m(), wn = w4_n();
  int tt, vr;
  grouped_tile<4>(xcd_order(blockIdx.x, gridDim.x), P.n_ttiles, P.n_vranges, tt, vr);
  const int64_t t0 = (int64_t)tt * kTok;
  const int vt_begin = vr * P.tiles_per_range;
  const int ntiles = min(vt_begin + P.tiles_per_range, P.n_vtiles) - vt_begin;
  // the lane's token j
  auto tok = [&](int j) { return t0 + (TL ? col16(j, wn) : wn * 64 + j * 16) + (lane & 15); };

  RowState st[NJ];
  float lse_sT[NJ], lse_tT[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    state_init_fam(st[j], kPhase1 ? FAM_NONE : P.fam);
    lse_sT[j] = lse_tT[j] = 0.f;
    if (kPhase1 && tok(j) < P.N) {
      lse_sT[j] = P.rowp[1 * P.N + tok(j)];
      lse_tT[j] = P.rowp[3 * P.N + tok(j)];
    }
  }
  const T* W = static_cast<const T*>(P.W);
  const T* hs = static_cast<const T*>(P.hs);
  const T* ht = static_cast<const T*>(P.ht);
  const KOp4 bop = TL ? kop4(hs + t0 * P.H, P.H, P.N - t0)
                      : kop4_split(hs + t0 * P.H, P.N - t0, ht + t0 * P.H, P.N - t0, P.H);
  struct TI {
    int v0;
    KOp4 a;
  };
  auto tile_info = [&](int i) {
    TI x;
    x.v0 = (vt_begin + (i < ntiles ? i : 0)) * 256;
    x.a = kop4(W + (int64_t)x.v0 * P.H, P.H, P.V - x.v0);
    return x;
  };
  auto opnd = [&](const TI& x, int op) { return op == 0 ? x.a : bop; };
  auto epilogue = [&](int, const TI& x, Acc16& c, char* stage) __attribute__((always_inline)) {
    const int vlane0 = wm * 128 + (opaque_lane() >> 4) * 4;
    const int64_t vlimit = P.V - x.v0;
    // a full student-only tile's logits go out staged (whole row pieces);
    // a tile with tokens past N stores block by block
    const bool full = t0 + 256 <= P.N;
    if constexpr (TL == TL_STUDENT) {
      if (full) store_tile16_staged<T>(c, P, x.v0, t0, 128, true, stage);
      static_for<0, NJ>([&](auto J) {
        constexpr int j = decltype(J)::value;
        if (!full) store_block16<T>(c, P, x.v0, t0, j);
        scan_variant<SV>(st[j], AccPair16S{c, j}, vlane0, vlimit, vlimit >= 256, lse_sT[j], lse_tT[j], P);
      });
    } else if constexpr (TL != TL_NONE) {
      // blocks j and j + 1 in flight while block j is scanned (the staged
      // store of the student's logits runs while the first two land); block
      // j's student logits stored after its scan when the tile is not full
      uint2 raw[2][8];
      issue_teacher16<T, TL>(raw[0], P, x.v0, t0, 0);
      issue_teacher16<T, TL>(raw[1], P, x.v0, t0, 1);
      if (full) store_tile16_staged<T>(c, P, x.v0, t0, 128, true, stage);
      static_for<0, NJ>([&](auto J) {
        constexpr int j = decltype(J)::value;
        order_teacher16<T, TL>(raw[j & 1]);
        if constexpr (TL == TL_FROM_MEM) {
          if (P.store_t) store_teacher16<T>(raw[j & 1], P, x.v0, t0, j);  // else the dlogits pass reads them in place
        }
        scan_variant<SV>(st[j], AccPair16TL<T>{c, j, raw[j & 1]}, vlane0, vlimit, vlimit >= 256, lse_sT[j],
                         lse_tT[j], P);
        if (!full) store_block16<T>(c, P, x.v0, t0, j);
        if constexpr (j + 2 < NJ) issue_teacher16<T, TL>(raw[j & 1], P, x.v0, t0, j + 2);
      });
    } else {
      if constexpr (STORE) {
        if (t0 + 128 <= P.N)
          store_tile16_staged<T>(c, P, x.v0, t0, P.tcolL, P.store_t != 0, stage);
        else
          store_logits16<T>(c, P, x.v0, t0);
      }
      static_for<0, NJ>([&](auto J) {
        constexpr int j = decltype(J)::value;
        scan_variant<SV>(st[j], AccPair16{c, j}, vlane0, vlimit, vlimit >= 256, lse_sT[j], lse_tT[j], P);
      });
    }
  };
  pipeline16<T, KMAJ, KMAJ, true, true, false>(acc, lds, ntiles, P.H, P.H, P.H, tile_info, opnd, epilogue);

  // combine lanes l ^ 16 and l ^ 32 (other vocabulary rows of the same
  // tokens), then the two waves sharing the tokens (wm 0 / 1)
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    RowState o = shfl_state(st[j], 16);
    merge_any<kPhase1>(st[j], o, P);
    o = shfl_state(st[j], 32);
    merge_any<kPhase1>(st[j], o, P);
  }
  __syncthreads();
  float* xch = reinterpret_cast<float*>(lds);  // [wn][j][kNStat][16]
  if (wm == 1 && lane < 16) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      float* d = xch + ((wn * NJ + j) * kNStat) * 16 + lane;
      const float* sv = reinterpret_cast<const float*>(&st[j]);
#pragma unroll
      for (int f = 0; f < kNStat; ++f) d[f * 16] = sv[f];
    }
  }
  __syncthreads();
  if (wm == 0 && lane < 16) {
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      RowState o;
      float* od = reinterpret_cast<float*>(&o);
      const float* sv = xch + ((wn * NJ + j) * kNStat) * 16 + lane;
#pragma unroll
      for (int f = 0; f < kNStat; ++f) od[f] = sv[f * 16];
      merge_any<kPhase1>(st[j], o, P);
      if (tok(j) < P.N) {
        float* dst = P.partial + (int64_t)vr * kNStat * P.N + tok(j);
        const float* v = reinterpret_cast<const float*>(&st[j]);
#pragma unroll
        for (int f = 0; f < kNStat; ++f) dst[(int64_t)f * P.N] = v[f];
      }
    }
  }
}

// ----------------------------------------------------------- dlogits kernel
template <class T, int DIV, bool T1>
__device__ __forceinline__ void dl_tile(const f32x16 (&acc)[4][2], const FusedParams& P, int64_t v0,
                                        int64_t t0) {
  const int lane = threadIdx.x & 63;
  const int wm = wave_m(), wn = wave_n();
  const int64_t t = t0 + wn * 32 + (lane & 31);
  // lanes past the last token stay active (the quad transpose below needs
  // every lane of a quad); they read token 0's row data, produce zeros and
  // store nothing
  const bool tok_ok = t < P.N;
  const int64_t tr = tok_ok ? t : 0;
  const float scale = P.grad_output[0] * P.mean_scale[0];
  const float invT = P.invT;
  const int64_t vend = min(P.V, P.vc0 + P.vcc);
  T* dLT = static_cast<T*>(P.dLT);
  T* dLNs = static_cast<T*>(P.dLNs);
  T* dLNt = static_cast<T*>(P.dLNt);
  const int64_t y = P.labels[tr];
  const bool ignored = !tok_ok || (y == P.ignore_index);
  const int64_t yeff = (y >= 0 && y < P.V) ? y : 0;
  const float lse_s = P.rowp[0 * P.N + tr];
  const float lse_sT = P.rowp[1 * P.N + tr];
  const float lse_t = P.rowp[2 * P.N + tr];
  const float lse_tT = P.rowp[3 * P.N + tr];
  float c[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = P.rowp[(4 + i) * P.N + tr];
  const float sc_s = ignored ? 0.f : scale * P.w_s;
  const float sc_t = ignored ? 0.f : scale * P.w_t;
  const float sc_d = ignored ? 0.f : scale * P.w_kl * P.temperature;
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int64_t vg = v0 + wm * 128 + acc_row(mb, g * 4, lane);  // 4 consecutive rows
      float gs[4], gt[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int r = g * 4 + e;
        const int64_t v = vg + e;
        const float xs = acc[mb][0][r];
        const float onehot = (v == yeff) ? 1.f : 0.f;
        const float ps1 = fexp(xs - lse_s);
        float d = sc_s * (ps1 - onehot);
        if (DIV >= 0) {
          const float xt = acc[mb][1][r];
          const float lps = xs * invT - lse_sT;
          const float lpt = xt * invT - lse_tT;
          const float psT = T1 ? ps1 : fexp(lps);
          const float ptT = fexp(lpt);
          d += sc_d * div_grad<(DIV >= 0 ? DIV : 0)>(lps, lpt, psT, ptT, c, P.alpha, P.beta);
        }
        gs[e] = ignored ? 0.f : d;
        if (P.tgrad) {
          const float xt = acc[mb][1][r];
          gt[e] = ignored ? 0.f : sc_t * (fexp(xt - lse_t) - onehot);
        } else {
          gt[e] = 0.f;
        }
      }
      const int64_t vl = vg - P.vc0;  // row inside the chunk
      const bool rows_full = vg + 3 < vend;
      // token-major staging: this lane's 4 consecutive rows are contiguous
      if (P.w_dln_s && tok_ok) store4(dLNs + t * P.ldN + vl, gs, rows_full, (int)(vend - vg));
      if (P.w_dln_t && tok_ok) store4(dLNt + t * P.ldN + vl, gt, rows_full, (int)(vend - vg));
      // row-major staging: transpose inside the lane quad so each lane
      // holds 4 consecutive tokens of one row
      if (P.w_dlt_s || P.w_dlt_t) {
        const int q = lane & 3;
        const int64_t tb = t - q;  // first token of the quad
        const int ntok = (int)min<int64_t>(P.N - tb, 4);
        const bool row_ok = vg + q < vend;
        if (P.w_dlt_s) {
          float o[4];
          quad_transpose(gs, o);
          if (row_ok) store4(dLT + (vl + q) * P.ldT + tb, o, ntok == 4, ntok);
        }
        if (P.w_dlt_t) {
          float o[4];
          quad_transpose(gt, o);
          if (row_ok) store4(dLT + (vl + q) * P.ldT + P.tcol + tb, o, ntok == 4, ntok);
        }
      }
    }
}

template <class T, int DIV, bool T1>
__global__ __launch_bounds__(kThreads) void k_dl(FusedParams P) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  f32x16 acc[4][2];
  int tt, vt;
  grouped_tile<4>(xcd_order(blockIdx.x, gridDim.x), P.n_ttiles, gridDim.x / P.n_ttiles, tt, vt);
  const int64_t t0 = (int64_t)tt * 128;
  const int64_t v0 = P.vc0 + (int64_t)vt * 256;
  fused_logits<T>(acc, lds, P, v0, t0);
  dl_tile<T, DIV, T1>(acc, P, v0, t0);
}

// -------------------------------------------------------------- plain GEMM
template <class T, int MODE>
__device__ __forceinline__ void gemm_epilogue(const f32x16 (&acc)[4][2], const GemmParams& P, int64_t m0,
                                              int64_t n0) {
  const int lane = threadIdx.x & 63;
  const int wm = wave_m(), wn = wave_n();
  // 32-bit offsets inside the tile; the tile base stays 64-bit.
  T* C = static_cast<T*>(P.C) + m0 * P.ldc + n0;
  float* C32 = P.C32 + m0 * P.ldc + n0;
  const int ldc = (int)P.ldc;
  const int mlim = (int)min<int64_t>(P.M - m0, 256), nlim = (int)min<int64_t>(P.N - n0, 256);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int n = acc_col0(nb, wn) + (lane & 31);
      const int mrow0 = wm * 128 + mb * 32 + (lane >> 5) * 4;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mrow0 + (r >> 2) * 8 + (r & 3);
        if (m < mlim && n < nlim) {
          const int o = m * ldc + n;
          const float a = acc[mb][nb][r];
          if (MODE == GEMM_STORE) C[o] = from_f32<T>(a);
          else if (MODE == GEMM_ACC_FIRST) C32[o] = a;
          else if (MODE == GEMM_ACC) C32[o] += a;
          else C[o] = from_f32<T>(C32[o] + a);
        }
      }
    }
}

// C[M x N] (= or +=) A[M x K] * B[N x K]^T.  Epilogue modes: STORE writes C
// in T; ACC_FIRST/ACC write the fp32 accumulator C32; ACC_LAST adds C32 and
// writes C in T.  Tiles are visited in bands of 8 tile rows, XCD by XCD.
template <class T>
__global__ __launch_bounds__(kThreads) void k_gemm(GemmParams P) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  f32x16 acc[4][2];
  const int t = xcd_order(blockIdx.x, gridDim.x);
  constexpr int G = 8;
  const int band = t / (G * P.tiles_n);
  const int first_m = band * G;
  const int gm = min(P.tiles_m - first_m, G);
  const int rem = t % (G * P.tiles_n);
  const int tm = first_m + rem % gm;
  const int tn = rem / gm;
  const int64_t m0 = (int64_t)tm * 256, n0 = (int64_t)tn * 256;
  const T* A = static_cast<const T*>(P.A);
  const T* B = static_cast<const T*>(P.B);
  zero_acc(acc);
  mainloop<T, true, true>(acc, lds, A + m0 * P.lda, P.lda, P.M - m0, B + n0 * P.ldb, P.ldb, P.N - n0,
                          B + (n0 + 128) * P.ldb, P.ldb, P.N - n0 - 128, P.K);
  switch (P.mode) {
    case GEMM_STORE: gemm_epilogue<T, GEMM_STORE>(acc, P, m0, n0); break;
    case GEMM_ACC_FIRST: gemm_epilogue<T, GEMM_ACC_FIRST>(acc, P, m0, n0); break;
    case GEMM_ACC: gemm_epilogue<T, GEMM_ACC>(acc, P, m0, n0); break;
    default: gemm_epilogue<T, GEMM_ACC_LAST>(acc, P, m0, n0); break;
  }
}

// ------------------------------------------------------------ general GEMM
// Load 4 consecutive elements as fp32 (one vector load when full).
template <class T>
__device__ __forceinline__ void load4(const T* p, float (&x)[4], bool full, int n) {
  if (full) {
    if constexpr (sizeof(T) == 2) {
      union { T e[4]; uint2 u; } v;
      v.u = *reinterpret_cast<const uint2*>(p);
#pragma unroll
      for (int i = 0; i < 4; ++i) x[i] = to_f32(v.e[i]);
    } else {
      const float4 f = *reinterpret_cast<const float4*>(p);
      x[0] = f.x; x[1] = f.y; x[2] = f.z; x[3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (i < n) ? to_f32(p[i]) : 0.f;
  }
}

// Epilogue with 4-wide accesses: a lane's 4 consecutive rows of one column
// are transposed inside the lane quad into 4 consecutive columns of one row
// (C row-major, ldc a multiple of 4, tile base 8-byte aligned for 16-bit C
// and 16-byte aligned for fp32).  Every lane must call this (DPP).
template <class T, int MODE>
__device__ __forceinline__ void gemm_epilogue_q(const f32x16 (&acc)[4][2], const GemmParams& P, float* C32,
                                                int64_t m0, int64_t n0) {
  const int lane = opaque_lane();
  const int wm = wave_m(), wn = wave_n();
  const int q = lane & 3;
  T* C = static_cast<T*>(P.C) + m0 * P.ldc + n0;
  float* D = C32 + m0 * P.ldc + n0;
  const int ldc = (int)P.ldc;
  const int mlim = (int)min<int64_t>(P.M - m0, 256), nlim = (int)min<int64_t>(P.N - n0, 256);
  if constexpr (MODE == GEMM_ACC_T && sizeof(T) == 2) {
    if (mlim == 256 && nlim == 256) {
      // interior tile: issue the reads of C for half the tile (two row
      // blocks) before its first add, so one memory latency covers 16 of the
      // read-modify-writes and 32 registers hold the loaded values
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint2 cv[2][2][4];
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              const int m = wm * 128 + acc_row(2 * h + j, g * 4, lane) + q;
              const int nbase = acc_col0(nb, wn) + (lane & 31) - q;
              cv[j][nb][g] = *reinterpret_cast<const uint2*>(C + m * ldc + nbase);
            }
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int nb = 0; nb < 2; ++nb)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
              float x[4], o[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) x[e] = acc[2 * h + j][nb][g * 4 + e];
              quad_transpose(x, o);
              const int m = wm * 128 + acc_row(2 * h + j, g * 4, lane) + q;
              const int nbase = acc_col0(nb, wn) + (lane & 31) - q;
              union { T e[4]; uint2 u; } v;
              v.u = cv[j][nb][g];
#pragma unroll
              for (int e = 0; e < 4; ++e) o[e] += to_f32(v.e[e]);
              store4(C + m * ldc + nbase, o, true, 4);
            }
      }
      return;
    }
  }
#pragma unroll
  for (int mb = 0; mb < 4; ++mb)
#pragma unroll
    for (int nb = 0; nb < 2; ++nb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float x[4], o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) x[e] = acc[mb][nb][g * 4 + e];
        quad_transpose(x, o);
        const int m = wm * 128 + acc_row(mb, g * 4, lane) + q;
        const int nbase = acc_col0(nb, wn) + (lane & 31) - q;
        const int rem = nlim - nbase;
        const int cnt = rem <= 0 ? 0 : (rem >= 4 ? 4 : rem);
        if (m < mlim && cnt > 0) {
          const int off = m * ldc + nbase;
          const bool full = cnt == 4;
          if constexpr (MODE == GEMM_STORE) {
            store4(C + off, o, full, cnt);
          } else if constexpr (MODE == GEMM_ACC_T) {
            float c[4];
            load4(C + off, c, full, cnt);
#pragma unroll
            for (int e = 0; e < 4; ++e) c[e] += o[e];
            store4(C + off, c, full, cnt);
          } else if constexpr (MODE == GEMM_ACC_FIRST || MODE == GEMM_SPLIT) {
            store4(D + off, o, full, cnt);
          } else {
            float c[4];
            load4(D + off, c, full, cnt);
#pragma unroll
            for (int e = 0; e < 4; ++e) c[e] += o[e];
            if constexpr (MODE == GEMM_ACC) store4(D + off, c, full, cnt);
            else store4(C + off, c, full, cnt);
          }
        }
      }
}

template <class T, int L>
__device__ __forceinline__ auto gemm_operand(const T* p, int64_t ld, int64_t row0, int64_t rows, int64_t kb,
                                             int64_t klen) {
  if constexpr (L == KMAJ) return KOperand<T>{p + row0 * ld + kb, ld, rows};
  else return MnOperand<T>{p + kb * ld + row0, nullptr, ld, 0, klen, klen, 0, rows};
}

// General GEMM: C[M x N] (mode) A * B^T with A and B each K-major or
// MN-major (Layout), split-K (split s covers K rows [s * k_per_split, ...)
// and writes its own fp32 partial in GEMM_SPLIT mode), and, for an MN-major
// B, two row segments (B rows [0, b_kseg) from B, the rest from B1): the
// student and teacher hidden states of one token chunk feeding one grad-W
// GEMM.  Persistent: workgroup b (in XCD order) owns tiles b, b + grid, ...
// in band order, run as one flattened pipeline (pipeline_tiles), so the next
// tile's first K steps load while the current one finishes and writes out.
template <class T, int LA, int LB, int MODE>
__global__ __launch_bounds__(kThreads) void k_gemm2(GemmParams P) {
  __shared__ __attribute__((aligned(16))) char lds[kLdsBytes];
  f32x16 acc[4][2];
  constexpr int BK = Traits<T>::kBK;
  const int tiles = P.tiles_m * P.tiles_n;
  const int total = tiles * P.splits;
  const int grid = gridDim.x;
  const int b = xcd_order(blockIdx.x, grid);
  const int ntiles = b < total ? (total - 1 - b) / grid + 1 : 0;
  const int nk = (int)((P.k_per_split + BK - 1) / BK);
  struct Tile { int split; int64_t m0, n0, kb, klen; };
  auto tile_of = [&](int i) {
    const int t_all = b + i * grid;
    Tile x;
    x.split = t_all / tiles;
    const int t = t_all - x.split * tiles;
    constexpr int G = 8;
    const int band = t / (G * P.tiles_n);
    const int first_m = band * G;
    const int gm = min(P.tiles_m - first_m, G);
    const int rem = t % (G * P.tiles_n);
    x.m0 = (int64_t)(first_m + rem % gm) * 256;
    x.n0 = (int64_t)(rem / gm) * 256;
    x.kb = (int64_t)x.split * P.k_per_split;
    x.klen = min<int64_t>(P.K - x.kb, P.k_per_split);
    return x;
  };
  const T* A = static_cast<const T*>(P.A);
  const T* B = static_cast<const T*>(P.B);
  const T* B1 = static_cast<const T*>(P.B1);
  using DA = typename std::conditional<LA == KMAJ, KDma<T>, MnDma<T>>::type;
  using DB = typename std::conditional<LB == KMAJ, KDma<T>, MnDma<T>>::type;
  DA da;
  DB db;
  da.init();
  db.init();
  // pipeline_tiles issues the steps once each, in order: track the tile and
  // K step of the next one instead of dividing the step index
  int in = 0, kn = 0;
  Tile x = tile_of(0);
  auto issue = [&](int, char* st) {
    if (kn == nk) {
      kn = 0;
      x = tile_of(++in);
    }
    const int64_t k0 = (int64_t)(kn++) * BK;  // inside the split
    if constexpr (LA == KMAJ) {
      if (k0 == 0) da.template place<0, 4>(P.lda, P.M - x.m0, 0);
      da.template issue<0, 4>(A + x.m0 * P.lda + x.kb, k0, x.klen, st);
    } else {
      const MnOperand<T> o{A + x.kb * P.lda + x.m0, nullptr, P.lda, 0, x.klen, x.klen, 0, P.M - x.m0};
      da.issue(o, k0, st);
    }
    if constexpr (LB == KMAJ) {
      if (k0 == 0) db.template place<0, 4>(P.ldb, P.N - x.n0, 0);
      db.template issue<0, 4>(B + x.n0 * P.ldb + x.kb, k0, x.klen, st + kTileBytes);
    } else {
      MnOperand<T> o;
      o.p0 = B + x.kb * P.ldb + x.n0;
      o.ld0 = P.ldb;
      o.kseg = P.b_kseg - x.kb;
      o.kval0 = min<int64_t>(P.b_kval0 - x.kb, x.klen);
      o.p1 = B1 ? B1 + x.n0 : nullptr;
      o.ld1 = P.ldb1;
      o.kval1 = P.b_kval1;
      o.cols = P.N - x.n0;
      db.issue(o, k0, st + kTileBytes);
    }
  };
  auto epilogue = [&](int i, f32x16 (&c)[4][2]) {
    const Tile y = tile_of(i);
    gemm_epilogue_q<T, MODE>(c, P, P.C32 + (int64_t)y.split * P.split_stride, y.m0, y.n0);
  };
  zero_acc(acc);
  pipeline_tiles<T, LA, LB, true, true, 8>(acc, lds, ntiles, nk, issue, epilogue);
}

// Lanes l (l / 16 even) and l + 16 trade halves of two adjacent blocks P
// (columns c0 + 4 (l / 16) ..) and Q (c0 + 16 + 4 (l / 16) ..): afterwards
// each lane holds 8 consecutive columns starting at c0 + g8(l), values
// x[0..3] then y[0..3].
__device__ __forceinline__ int g8(int lane) { return 16 * ((lane >> 4) & 1) + 8 * (lane >> 5); }
__device__ __forceinline__ void trade16(const f32x4& P, const f32x4& Q, float (&x)[4], float (&y)[4]) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(acc16_get(P, e)), __float_as_uint(acc16_get(Q, e)),
                                                    false, false);
    x[e] = __uint_as_float(r[0]);
    y[e] = __uint_as_float(r[1]);
  }
}

// C[M x N] (mode) A B^T for 16-bit operands on the four-wave ring engine
// with 16x16x32 MFMAs (pipeline16): A K-major and B K-major or MN-major (one
// segment; MODE GEMM_STORE: C = in T, GEMM_ACC_T: C += in T, the fp32 sum
// rounded once; one split), or both MN-major (GEMM_STORE, or GEMM_SPLIT:
// split s covers K rows [s * k_per_split, ...) and writes its fp32 partial).
// Persistent: workgroup b (in XCD order) owns work items b, b + grid, ...
// (split-major, tiles in band order, 8 row tiles wide).  The MFMAs run
// swapped (B x A^T), so each lane holds four consecutive columns of one C row
// per block; lanes l and l + 16 trade halves of two adjacent blocks
// (trade16) so interior tiles move 8 columns per 16-byte access.
// Contract as k_gemm2, plus k_per_split > 64 and, for MN-major operands,
// k_per_split * ld * sizeof(T) < 2^31.
template <class T, int LA, int LB, int MODE>
__global__ __launch_bounds__(kThreads4, 1) void k_gemm4(GemmParams P) {
  static_assert(LA == LB || (LA == KMAJ && LB == MNMAJ), "K/K, K/MN or MN/MN");
  __shared__ __attribute__((aligned(16))) char lds[kLds4Bytes];
  Acc16 acc;
  zero_acc16(acc);
  const int tiles = P.tiles_m * P.tiles_n;
  const int total = tiles * P.splits;
  const int grid = gridDim.x;
  const int b = xcd_order(blockIdx.x, grid);
  const int ntiles = b < total ? (total - 1 - b) / grid + 1 : 0;
  const T* A = static_cast<const T*>(P.A);
  const T* B = static_cast<const T*>(P.B);
  struct TI {
    int m0, n0, split;
    KOp4 a, b;
  };
  auto tile_info = [&](int i) {
    const int t_all = b + (i < ntiles ? i : 0) * grid;
    TI x;
    x.split = t_all / tiles;
    const int t = t_all - x.split * tiles;
    constexpr int G = 8;
    const int band = t / (G * P.tiles_n);
    const int first_m = band * G;
    const int gm = min(P.tiles_m - first_m, G);
    const int rem = t % (G * P.tiles_n);
    x.m0 = (first_m + rem % gm) * 256;
    x.n0 = (rem / gm) * 256;
    const int64_t kb = (int64_t)x.split * P.k_per_split;
    if constexpr (LA == KMAJ && LB == KMAJ) {
      x.a = kop4(A + (int64_t)x.m0 * P.lda + kb, P.lda, P.M - x.m0);
      x.b = kop4(B + (int64_t)x.n0 * P.ldb + kb, P.ldb, P.N - x.n0);
    } else if constexpr (LA == KMAJ) {
      x.a = kop4(A + (int64_t)x.m0 * P.lda, P.lda, P.M - x.m0);
      x.b = kop4_mn(B + x.n0, P.ldb, P.b_kval0, P.N - x.n0);
    } else {
      const int64_t klen = min<int64_t>(P.K - kb, P.k_per_split);
      x.a = kop4_mn(A + kb * P.lda + x.m0, P.lda, klen, P.M - x.m0);
      x.b = kop4_mn(B + kb * P.ldb + x.n0, P.ldb, klen, P.N - x.n0);
    }
    return x;
  };
  auto opnd = [](const TI& x, int op) { return op == 0 ? x.a : x.b; };
  auto epilogue = [&](int, const TI& x, Acc16& c, char*) __attribute__((always_inline)) {
    const int lane = opaque_lane();
    const int wm = w4_m(), wn = w4_n();
    const int64_t ldc = P.ldc;
    const int mlim = (int)min<int64_t>(P.M - x.m0, 256), nlim = (int)min<int64_t>(P.N - x.n0, 256);
    const int rl = lane & 15;          // C row of the lane within a block
    const int cq = 4 * (lane >> 4);    // first of the lane's 4 columns within a block (before the trade)
    const int cg = g8(lane);           // first of the lane's 8 columns within a block pair (after the trade)
    if constexpr (MODE == GEMM_SPLIT) {
      float* D = P.C32 + (int64_t)x.split * P.split_stride + (int64_t)x.m0 * ldc + x.n0;
      if (mlim == 256 && nlim == 256) {
#pragma unroll
        for (int mb = 0; mb < 8; ++mb) {
          float* rp = D + (int64_t)(wm * 128 + mb * 16 + rl) * ldc;
#pragma unroll
          for (int pr = 0; pr < 4; ++pr) {
            const int nb = (pr >> 1) * 4 + (pr & 1) * 2;  // block pairs (0,1) (2,3) (4,5) (6,7)
            float xv[4], yv[4];
            trade16(c[mb][nb], c[mb][nb + 1], xv, yv);
            float* p = rp + col16(nb, wn) + cg;
            *reinterpret_cast<float4*>(p) = make_float4(xv[0], xv[1], xv[2], xv[3]);
            *reinterpret_cast<float4*>(p + 4) = make_float4(yv[0], yv[1], yv[2], yv[3]);
            __builtin_amdgcn_sched_barrier(0);
          }
        }
        return;
      }
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) {
        const int mm = wm * 128 + mb * 16 + rl;
#pragma unroll
        for (int nb = 0; nb < 8; ++nb) {
          const int cc = col16(nb, wn) + cq;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const float v = acc16_get(c[mb][nb], e);
            if (mm < mlim && cc + e < nlim) D[(int64_t)mm * ldc + cc + e] = v;
          }
        }
      }
      return;
    }
    T* C = static_cast<T*>(P.C) + (int64_t)x.m0 * ldc + x.n0;
    const bool wide = sizeof(T) == 2 && ldc % 8 == 0 && reinterpret_cast<uintptr_t>(P.C) % 16 == 0;
    if (mlim == 256 && nlim == 256 && wide) {
      // GEMM_ACC_T: the old values of kRB row blocks (16 kRB rows x 256
      // bytes per wave) are loaded before the first add
      constexpr int kRB = 4;
#pragma unroll
      for (int hh = 0; hh < 8 / kRB; ++hh) {
        uint4 cv[kRB][4];
        if constexpr (MODE == GEMM_ACC_T) {
#pragma unroll
          for (int j = 0; j < kRB; ++j) {
            const T* rp = C + (int64_t)(wm * 128 + (kRB * hh + j) * 16 + rl) * ldc;
#pragma unroll
            for (int pr = 0; pr < 4; ++pr) {
              const int nb = (pr >> 1) * 4 + (pr & 1) * 2;
              cv[j][pr] = *reinterpret_cast<const uint4*>(rp + col16(nb, wn) + cg);
            }
          }
        }
#pragma unroll
        for (int j = 0; j < kRB; ++j) {
          const int mb = kRB * hh + j;
          T* rp = C + (int64_t)(wm * 128 + mb * 16 + rl) * ldc;
#pragma unroll
          for (int pr = 0; pr < 4; ++pr) {
            const int nb = (pr >> 1) * 4 + (pr & 1) * 2;
            float xv[4], yv[4];
            trade16(c[mb][nb], c[mb][nb + 1], xv, yv);
            uint4 out;
            if constexpr (MODE == GEMM_ACC_T) {
              const uint4 old = cv[j][pr];
              out.x = pack2<T>(xv[0] + lo16<T>(old.x), xv[1] + hi16<T>(old.x));
              out.y = pack2<T>(xv[2] + lo16<T>(old.y), xv[3] + hi16<T>(old.y));
              out.z = pack2<T>(yv[0] + lo16<T>(old.z), yv[1] + hi16<T>(old.z));
              out.w = pack2<T>(yv[2] + lo16<T>(old.w), yv[3] + hi16<T>(old.w));
            } else {
              out = make_uint4(pack2<T>(xv[0], xv[1]), pack2<T>(xv[2], xv[3]), pack2<T>(yv[0], yv[1]),
                               pack2<T>(yv[2], yv[3]));
            }
            *reinterpret_cast<uint4*>(rp + col16(nb, wn) + cg) = out;
            __builtin_amdgcn_sched_barrier(0);
          }
        }
      }
      return;
    }
    // edge tiles and rows that are not 16-byte aligned: 4 columns at a time
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) {
      const int mm = wm * 128 + mb * 16 + rl;
      T* rp = C + (int64_t)mm * ldc;
#pragma unroll
      for (int nb = 0; nb < 8; ++nb) {
        const int cc = col16(nb, wn) + cq;
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = acc16_get(c[mb][nb], e);
        const int rem = nlim - cc;
        const int cnt = rem <= 0 ? 0 : (rem >= 4 ? 4 : rem);
        if (mm < mlim && cnt > 0) {
          if constexpr (MODE == GEMM_ACC_T) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (e < cnt) o[e] += to_f32(rp[cc + e]);
          }
          store4(rp + cc, o, cnt == 4 && sizeof(T) == 2 && ldc % 4 == 0, cnt);
        }
      }
    }
  };
  pipeline16<T, LA, LB, true, true, true>(acc, lds, ntiles, P.k_per_split, P.lda, P.ldb,
                                          tile_info, opnd, epilogue);
}

// out[m][n] = sum over s of part[s][m][n] (fixed order), converted to T.
// Thread: 4 consecutive columns.  part has leading dimension N (dense),
// N a multiple of 4.
template <class T>
__global__ __launch_bounds__(256) void k_splitk_reduce(const float* __restrict__ part, int splits, int64_t stride,
                                                       T* __restrict__ out, int64_t ldo, int64_t M, int64_t N) {
  const int64_t nq = N / 4;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * nq) return;
  const int64_t m = i / nq, c = (i - m * nq) * 4;
  float x[4] = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < splits; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(part + s * stride + m * N + c);
    x[0] += v.x; x[1] += v.y; x[2] += v.z; x[3] += v.w;
  }
  store4(out + m * ldo + c, x, true, 4);
}

// x *= g[0] in place (n elements, n a multiple of 4, x 8-byte aligned);
// nothing to do when g[0] == 1.
template <class T>
__global__ __launch_bounds__(256) void k_scale(T* __restrict__ x, int64_t n, const float* __restrict__ g) {
  const float s = g[0];
  if (s == 1.0f) return;
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < n; i += (int64_t)gridDim.x * 256 * 4) {
    const int cnt = (int)min<int64_t>(4, n - i);  // (a ragged tail element by element)
    float v[4];
    load4(x + i, v, cnt == 4, cnt);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] *= s;
    store4(x + i, v, cnt == 4, cnt);
  }
}

// ------------------------------------------- token-major teacher tiles
// A kTmTok-token x kTmRows-row block of the caller's token-major [N x ldtm]
// 16-bit teacher logits, staged in LDS by token quads:
//   tile[q * kTmPitch + r * 4 + i] = Tm[tb + 4 q + i][v0 + r]
// (a quad's 4 values of one row are one 8-byte word; the quad pitch of 130
// dwords puts the 32 lanes of a half-wave reading rows of consecutive quads
// on distinct banks).  Loader: thread -> 16-byte piece j = tid % 8 (rows
// 8 j .. 8 j + 7) of the 4 token rows of quads tid / 8 and tid / 8 + 32 (8
// lanes cover a token's 128 contiguous bytes), transposed in registers
// (v_perm_b32) into 8 rows x 4 tokens before the LDS writes.  Requires V a
// multiple of 8 and 16-byte aligned rows (a piece is wholly in or out of V).
constexpr int kTmTok = 256, kTmRows = 64, kTmPitch = kTmRows * 4 + 4;
constexpr int kTmTileElems = (kTmTok / 4) * kTmPitch;

__device__ __forceinline__ uint32_t u4_word(const uint4& v, int k) {
  return k == 0 ? v.x : (k == 1 ? v.y : (k == 2 ? v.z : v.w));
}

template <class T>
struct TmTile {
  uint4 w[2][4];  // [quad half][token of the quad]: piece j of the token's row
  __device__ __forceinline__ void load(const T* Tm, int64_t ldtm, int64_t tb, int64_t v0, int64_t N, int64_t V) {
    const int j = threadIdx.x & 7, q0 = threadIdx.x >> 3;
    const int64_t v = v0 + j * 8;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int64_t t = tb + (q0 + 32 * h) * 4 + i;
        w[h][i] = make_uint4(0u, 0u, 0u, 0u);
        if (t < N && v < V) w[h][i] = *reinterpret_cast<const uint4*>(Tm + t * ldtm + v);
      }
  }
  __device__ __forceinline__ void put(T* tile) const {
    const int j = threadIdx.x & 7, q0 = threadIdx.x >> 3;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      T* base = tile + (q0 + 32 * h) * kTmPitch + j * 8 * 4;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        // element e of the 4 tokens' pieces: low or high half of word e / 2
        const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
        const uint32_t lo = __builtin_amdgcn_perm(u4_word(w[h][1], e >> 1), u4_word(w[h][0], e >> 1), sel);
        const uint32_t hi = __builtin_amdgcn_perm(u4_word(w[h][3], e >> 1), u4_word(w[h][2], e >> 1), sel);
        *reinterpret_cast<uint2*>(base + e * 4) = make_uint2(lo, hi);
      }
    }
  }
  // the 4 tokens of quad q at row r of the tile
  __device__ __forceinline__ static void read(const T* tile, int q, int r, float (&x)[4]) {
    const uint2 u = *reinterpret_cast<const uint2*>(tile + q * kTmPitch + r * 4);
    x[0] = lo16<T>(u.x);
    x[1] = hi16<T>(u.x);
    x[2] = lo16<T>(u.y);
    x[3] = hi16<T>(u.y);
  }
};

// 4 consecutive elements as raw bits (one 8- or 16-byte load when n == 4;
// elements past n read as zero bits), converted to fp32 at their use: the
// streaming passes keep a 16-bit row in two registers instead of four.
template <class T> struct Raw4 { typedef uint2 type; };
template <> struct Raw4<float> { typedef uint4 type; };
template <class T>
__device__ __forceinline__ typename Raw4<T>::type load_raw4(const T* p, int n) {
  if constexpr (sizeof(T) == 2) {
    if (n == 4) return *reinterpret_cast<const uint2*>(p);
    uint32_t e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = i < n ? (uint32_t)__builtin_bit_cast(unsigned short, p[i]) : 0u;
    return make_uint2(e[0] | (e[1] << 16), e[2] | (e[3] << 16));
  } else {
    if (n == 4) return *reinterpret_cast<const uint4*>(p);
    uint32_t e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) e[i] = i < n ? __float_as_uint(p[i]) : 0u;
    return make_uint4(e[0], e[1], e[2], e[3]);
  }
}
template <class T>
__device__ __forceinline__ void unpack4(const typename Raw4<T>::type& u, float (&x)[4]) {
  if constexpr (sizeof(T) == 2) {
    x[0] = lo16<T>(u.x);
    x[1] = hi16<T>(u.x);
    x[2] = lo16<T>(u.y);
    x[3] = hi16<T>(u.y);
  } else {
    x[0] = __uint_as_float(u.x);
    x[1] = __uint_as_float(u.y);
    x[2] = __uint_as_float(u.z);
    x[3] = __uint_as_float(u.w);
  }
}

// ------------------------------------- two-pass row sums on stored logits
// Phase 1 of the two-pass divergences (JSD, skew KLs, TVD) for the
// gradients-in-forward schedule: the row sums x0, x1 over a token chunk's
// stored logits L[v][t] (student columns [0, N), teacher columns
// [tcol, tcol + N)), normalised with phase 0's log-sum-exps (rowp rows 1
// and 3), with the same per-row terms as the two-phase scan (two_term).
// One partial pair per (vocabulary range, token), dense: x0 at
// partial[(range * 2) * N + t], x1 at partial[(range * 2 + 1) * N + t]
// (k_merge's phase 1 with two_dense).  Block: 4 waves over kTwoTok tokens
// (a lane's 4 consecutive tokens: 8-byte loads of 16-bit logits, 512
// contiguous bytes per wave and row); wave w takes rows w, w + 4, ... of the
// range, 4 rows per step with the next step's loads issued before this
// step's math, and the four waves' sums are added in a fixed order
// (bit-stable).
constexpr int kTwoTok = 256;
template <class T, int DIV>
__global__ __launch_bounds__(256) void k_two_rows(TwoParams P) {
  __shared__ float xch[2][4][kTwoTok];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t tb = (int64_t)blockIdx.x * kTwoTok + lane * 4;
  const int64_t v0 = (int64_t)blockIdx.y * P.rows_per_range;
  const int64_t v1 = min<int64_t>(P.V, v0 + P.rows_per_range);
  const int64_t rem = P.N - tb;
  const int nt = rem <= 0 ? 0 : (rem >= 4 ? 4 : (int)rem);
  const float invT = P.invT;
  float lse_sT[4], lse_tT[4], s0[4], s1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t t = i < nt ? tb + i : 0;
    lse_sT[i] = P.rowp[1 * P.N + t];
    lse_tT[i] = P.rowp[3 * P.N + t];
    s0[i] = 0.f;
    s1[i] = 0.f;
  }
  const T* Ls = static_cast<const T*>(P.L) + (nt > 0 ? tb : 0);
  const T* Lt = Ls + P.tcol;
  using Raw = typename Raw4<T>::type;
  auto rows = [&](const Raw& us, const Raw& ut) {
    float xs[4], xt[4];
    unpack4<T>(us, xs);
    unpack4<T>(ut, xt);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      two_term<DIV>(xs[i] * invT - lse_sT[i], xt[i] * invT - lse_tT[i], P.mix_w, P.mix_w1, s0[i], s1[i]);
  };
  if (nt > 0) {
    int64_t v = v0 + w;
    constexpr int R = 4;
    Raw xs[R], xt[R];
    auto load_rows = [&](int64_t vv) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        xs[r] = load_raw4(Ls + (vv + 4 * r) * P.ldL, nt);
        xt[r] = load_raw4(Lt + (vv + 4 * r) * P.ldL, nt);
      }
    };
    if (v + 4 * (R - 1) < v1) load_rows(v);
    for (; v + 4 * (R - 1) < v1; v += 4 * R) {
      Raw cs[R], ct[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        cs[r] = xs[r];
        ct[r] = xt[r];
      }
      if (v + 4 * R + 4 * (R - 1) < v1) load_rows(v + 4 * R);
#pragma unroll
      for (int r = 0; r < R; ++r) rows(cs[r], ct[r]);
    }
    for (; v < v1; v += 4) rows(load_raw4(Ls + v * P.ldL, nt), load_raw4(Lt + v * P.ldL, nt));
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xch[0][w][lane * 4 + i] = s0[i];
    xch[1][w][lane * 4 + i] = s1[i];
  }
  __syncthreads();
  const int tk = threadIdx.x;
  const int64_t t = (int64_t)blockIdx.x * kTwoTok + tk;
  if (t < P.N) {
    float* dst = P.partial + (int64_t)blockIdx.y * 2 * P.N + t;
    dst[0] = (xch[0][0][tk] + xch[0][1][tk]) + (xch[0][2][tk] + xch[0][3][tk]);
    dst[P.N] = (xch[1][0][tk] + xch[1][1][tk]) + (xch[1][2][tk] + xch[1][3][tk]);
  }
}

// k_two_rows with the teacher's logits read in place from the caller's
// precomputed [N x ldtm] tensor (token-major): the block walks its range in
// tiles of kTmRows rows; per tile the teacher's kTmTok x kTmRows block is
// staged in LDS by token quads (TmTile) and wave w takes rows w, w + 4, ...
// of it beside the student's 8-byte loads from L, the next tile's loads
// issued while this tile is summed.  Same partial pairs and fixed-order
// reduction as k_two_rows; rows_per_range a multiple of kTmRows.
template <class T, int DIV>
__global__ __launch_bounds__(256) void k_two_rows_tm(TwoParams P) {
  __shared__ __align__(16) T tile[kTmTileElems];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t tb = (int64_t)blockIdx.x * kTmTok;
  const int64_t t0 = tb + lane * 4;
  const int64_t v0 = (int64_t)blockIdx.y * P.rows_per_range;
  const int64_t v1 = min<int64_t>(P.V, v0 + P.rows_per_range);
  const int64_t rem = P.N - t0;
  const int nt = rem <= 0 ? 0 : (rem >= 4 ? 4 : (int)rem);
  const float invT = P.invT;
  float lse_sT[4], lse_tT[4], s0[4], s1[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t t = i < nt ? t0 + i : 0;
    lse_sT[i] = P.rowp[1 * P.N + t];
    lse_tT[i] = P.rowp[3 * P.N + t];
    s0[i] = 0.f;
    s1[i] = 0.f;
  }
  const T* Ls = static_cast<const T*>(P.L) + (nt > 0 ? t0 : 0);
  const T* Tm = static_cast<const T*>(P.Ltm);
  constexpr int M = kTmRows / 4;  // rows per wave and tile
  TmTile<T> tm;
  using Raw = typename Raw4<T>::type;
  const bool full_tok = tb + kTmTok <= P.N;  // block-uniform
  Raw xs[M];
  // one tile's loads (teacher block and the student's rows), issued for the
  // next tile right after this tile's staging, so they are in flight during
  // this tile's arithmetic
  auto load = [&](int64_t vb) {
    tm.load(Tm, P.ldtm, tb, vb, P.N, P.V);
    if (full_tok && vb + kTmRows <= v1) {  // no per-row guards
      const T* p = Ls + (vb + w) * P.ldL;
#pragma unroll
      for (int m = 0; m < M; ++m) {
        xs[m] = *reinterpret_cast<const Raw*>(p);
        p += 4 * P.ldL;
      }
    } else {
#pragma unroll
      for (int m = 0; m < M; ++m) {
        const int64_t v = vb + w + 4 * m;
        xs[m] = {};
        if (nt > 0 && v < v1) xs[m] = load_raw4(Ls + v * P.ldL, nt);
      }
    }
  };
  if (v0 < v1) load(v0);
  for (int64_t vb = v0; vb < v1; vb += kTmRows) {
    __syncthreads();  // the previous tile's LDS reads are done
    tm.put(tile);
    Raw cs[M];
#pragma unroll
    for (int m = 0; m < M; ++m) cs[m] = xs[m];
    __syncthreads();
    if (vb + kTmRows < v1) load(vb + kTmRows);
    if (nt == 0) continue;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int r = w + 4 * m;
      if (vb + r >= v1) break;
      float xsf[4], xt[4];
      unpack4<T>(cs[m], xsf);
      TmTile<T>::read(tile, lane, r, xt);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        two_term<DIV>(xsf[i] * invT - lse_sT[i], xt[i] * invT - lse_tT[i], P.mix_w, P.mix_w1, s0[i], s1[i]);
    }
  }
  __syncthreads();  // the tile's LDS becomes the exchange buffer
  float* xch = reinterpret_cast<float*>(tile);  // [2][4][kTmTok] (8 KiB)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    xch[(0 * 4 + w) * kTmTok + lane * 4 + i] = s0[i];
    xch[(1 * 4 + w) * kTmTok + lane * 4 + i] = s1[i];
  }
  __syncthreads();
  const int tk = threadIdx.x;
  const int64_t t = tb + tk;
  if (t < P.N) {
    float* dst = P.partial + (int64_t)blockIdx.y * 2 * P.N + t;
    dst[0] = (xch[0 * kTmTok + tk] + xch[1 * kTmTok + tk]) + (xch[2 * kTmTok + tk] + xch[3 * kTmTok + tk]);
    dst[P.N] = (xch[4 * kTmTok + tk] + xch[5 * kTmTok + tk]) + (xch[6 * kTmTok + tk] + xch[7 * kTmTok + tk]);
  }
}

// ------------------------------------------------- materialised dlogits
// Row parameters of 4 consecutive tokens and their dlogits for one
// vocabulary row: student w_s (p_s - 1_y) + w_kl T dD/dz_s, teacher
// w_t (p_t - 1_y), times mean_scale (the caller's grad_output is applied
// later); ignored tokens (and tokens past the quad's nt) give 0.
template <int DIV, bool T1>
struct DlmQuad {
  int64_t yeff[4];
  float lse_s[4], lse_sT[4], lse_t[4], lse_tT[4], c[4][4], sc_s[4], sc_t[4], sc_d[4];
  float invT, alpha, beta;

  __device__ __forceinline__ void init(const DlmParams& P, int64_t t0, int nt) {
    const float scale = P.mean_scale[0];
    invT = P.invT;
    alpha = P.alpha;
    beta = P.beta;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const bool ok = i < nt;
      const int64_t t = t0 + (ok ? i : 0);
      const int64_t y = P.labels[t];
      const bool ign = !ok || y == P.ignore_index;
      yeff[i] = (y >= 0 && y < P.V) ? y : 0;
      lse_s[i] = P.rowp[0 * P.N + t];
      lse_sT[i] = P.rowp[1 * P.N + t];
      lse_t[i] = P.rowp[2 * P.N + t];
      lse_tT[i] = P.rowp[3 * P.N + t];
#pragma unroll
      for (int k = 0; k < 4; ++k) c[i][k] = P.rowp[(4 + k) * P.N + t];
      sc_s[i] = ign ? 0.f : scale * P.w_s;
      sc_t[i] = ign ? 0.f : scale * P.w_t;
      sc_d[i] = ign ? 0.f : scale * P.w_kl * P.temperature;
    }
  }
  __device__ __forceinline__ void row(int64_t v, const float (&xs)[4], const float (&xt)[4], float (&ds)[4],
                                      float (&dt)[4]) const {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float onehot = (v == yeff[i]) ? 1.f : 0.f;
      const float ps1 = fexp(xs[i] - lse_s[i]);
      float d = sc_s[i] * (ps1 - onehot);
      if constexpr (DIV >= 0) {
        const float lps = xs[i] * invT - lse_sT[i];
        const float lpt = xt[i] * invT - lse_tT[i];
        const float psT = T1 ? ps1 : fexp(lps);
        const float ptT = fexp(lpt);
        d += sc_d[i] * div_grad<DIV>(lps, lpt, psT, ptT, c[i], alpha, beta);
      }
      ds[i] = d;
      dt[i] = sc_t[i] * (fexp(xt[i] - lse_t[i]) - onehot);
    }
  }
};

// In place on the logits L[v][t] of one token chunk (vocabulary-major,
// student columns [0, N), teacher columns [tcol, tcol + N)): the dlogits of
// DlmQuad.  Thread: 4 consecutive tokens x rows_per_block vocabulary rows;
// block: 256 threads = 1024 tokens.
template <class T, int DIV, bool T1, bool NO_T = false>
__global__ __launch_bounds__(256) void k_dlm(DlmParams P) {
  const int64_t t0 = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (t0 >= P.N) return;
  const int nt = (int)min<int64_t>(P.N - t0, 4);
  const int64_t v0 = (int64_t)blockIdx.y * P.rows_per_block;
  const int64_t v1 = min<int64_t>(P.V, v0 + P.rows_per_block);
  DlmQuad<DIV, T1> q;
  q.init(P, t0, nt);
  T* Ls = static_cast<T*>(P.L) + t0;
  T* Lt = Ls + P.tcol;
  // (a compile-time no-teacher variant: a run-time flag here splits the
  // interior loop's batched loads)
  const bool need_t = !NO_T && (DIV >= 0 || P.tgrad);
  int64_t v = v0;
  if (nt == 4) {
    // interior: R rows per iteration, every load issued before any use
    constexpr int R = 8;
    using Raw = typename Raw4<T>::type;
    for (; v + R <= v1; v += R) {
      Raw us[R], ut[R];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        us[r] = load_raw4(Ls + (v + r) * P.ldL, 4);
        ut[r] = need_t ? load_raw4(Lt + (v + r) * P.ldL, 4) : Raw{};
      }
#pragma unroll
      for (int r = 0; r < R; ++r) {
        float xs[4], xt[4], ds[4], dt[4];
        unpack4<T>(us[r], xs);
        unpack4<T>(ut[r], xt);
        q.row(v + r, xs, xt, ds, dt);
        store4(Ls + (v + r) * P.ldL, ds, true, 4);
        if (P.tgrad) store4(Lt + (v + r) * P.ldL, dt, true, 4);
      }
    }
  }
  // edges: the last rows of the block, or a partial token quad
  for (; v < v1; ++v) {
    float xs[4], xt[4] = {0.f, 0.f, 0.f, 0.f}, ds[4], dt[4];
    load4(Ls + v * P.ldL, xs, nt == 4, nt);
    if (need_t) load4(Lt + v * P.ldL, xt, nt == 4, nt);
    q.row(v, xs, xt, ds, dt);
    store4(Ls + v * P.ldL, ds, nt == 4, nt);
    if (P.tgrad) store4(Lt + v * P.ldL, dt, nt == 4, nt);
  }
}

// The same dlogits with the teacher's logits read in place from the caller's
// precomputed [N x ldtm] tensor (token-major; no teacher gradient): a block
// takes kTmTok tokens x kTmRows vocabulary rows.  The teacher's block is
// staged in LDS by token quads (TmTile); the student's rows come from L with
// 8-byte loads (a lane's 4 tokens, 512 contiguous bytes per wave and row;
// wave w takes rows w, w + 4, ...), issued with the teacher's before the
// staging barrier.  (Blocks of one tile: with many short blocks in flight
// the stream runs faster than with a block walking several tiles.)  Blocks
// wholly inside [0, N) x [0, V) take a path without per-row guards (pointer
// steps, packed stores): 0.35 -> 0.29 ms per 2048-token chunk at V = 128256.
template <class T, int DIV, bool T1>
__global__ __launch_bounds__(256) void k_dlm_tm(DlmParams P) {
  __shared__ __align__(16) T tile[kTmTileElems];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t tb = (int64_t)blockIdx.x * kTmTok;
  const int64_t v0 = (int64_t)blockIdx.y * kTmRows;
  TmTile<T> tm;
  tm.load(static_cast<const T*>(P.Ltm), P.ldtm, tb, v0, P.N, P.V);
  const int64_t t0 = tb + lane * 4;
  const int64_t rem = P.N - t0;
  const int nt = rem <= 0 ? 0 : (rem >= 4 ? 4 : (int)rem);
  const bool live = nt > 0;
  const bool interior = tb + kTmTok <= P.N && v0 + kTmRows <= P.V;  // block-uniform
  T* Ls = static_cast<T*>(P.L) + (live ? t0 : 0);
  constexpr int M = kTmRows / 4;  // rows per wave
  using Raw = typename Raw4<T>::type;
  const int64_t step = 4 * P.ldL;
  Raw xs[M];
  if (interior) {
    const T* p = Ls + (v0 + w) * P.ldL;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      xs[m] = *reinterpret_cast<const Raw*>(p);
      p += step;
    }
  } else {
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int64_t v = v0 + w + 4 * m;
      xs[m] = {};
      if (live && v < P.V) xs[m] = load_raw4(Ls + v * P.ldL, nt);
    }
  }
  DlmQuad<DIV, T1> q;
  q.init(P, live ? t0 : 0, nt);
  tm.put(tile);
  __syncthreads();
  if (!live) return;
  if (interior) {
    T* p = Ls + (v0 + w) * P.ldL;
#pragma unroll
    for (int m = 0; m < M; ++m) {
      const int r = w + 4 * m;
      float x[4], xt[4], ds[4], dt[4];
      unpack4<T>(xs[m], x);
      TmTile<T>::read(tile, lane, r, xt);
      q.row(v0 + r, x, xt, ds, dt);
      *reinterpret_cast<uint2*>(p) = make_uint2(pack2<T>(ds[0], ds[1]), pack2<T>(ds[2], ds[3]));
      p += step;
    }
    return;
  }
#pragma unroll
  for (int m = 0; m < M; ++m) {
    const int r = w + 4 * m;
    const int64_t v = v0 + r;
    if (v >= P.V) break;
    float x[4], xt[4], ds[4], dt[4];
    unpack4<T>(xs[m], x);
    TmTile<T>::read(tile, lane, r, xt);
    q.row(v, x, xt, ds, dt);
    store4(Ls + v * P.ldL, ds, nt == 4, nt);
  }
}

// ---------------------------------------------------------------- transpose
// out[c * ldo + r] = in[r * ldi + c] for r < R, c < C (64 x 64 LDS tiles).
// 16-bit tiles wholly inside [0, R) x [0, C) with 16-byte aligned rows on
// both sides (vec) move 16 bytes per access: thread -> rows tid / 8 and
// tid / 8 + 32, piece tid % 8 (8 columns) on the way in; output rows the same
// on the way out, each piece gathered from 8 tile rows.
template <class T>
__global__ __launch_bounds__(256) void k_transpose(const T* __restrict__ in, int64_t ldi, T* __restrict__ out,
                                                   int64_t ldo, int64_t R, int64_t C, int tiles_c, int vec) {
  __shared__ __align__(16) T tile[64][72];  // (pitch 144 bytes: 16-byte aligned rows)
  const int tr = blockIdx.x / tiles_c, tc = blockIdx.x % tiles_c;
  const int64_t r0 = (int64_t)tr * 64, c0 = (int64_t)tc * 64;
  if constexpr (sizeof(T) == 2) {
    if (vec && r0 + 64 <= R && c0 + 64 <= C) {  // block-uniform
      const int j = threadIdx.x & 7, i0 = threadIdx.x >> 3;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int i = i0 + 32 * h;
        *reinterpret_cast<uint4*>(&tile[i][j * 8]) = *reinterpret_cast<const uint4*>(in + (r0 + i) * ldi + c0 + j * 8);
      }
      __syncthreads();
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = i0 + 32 * h;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = __builtin_bit_cast(unsigned short, tile[j * 8 + 2 * e][c]);
          const uint32_t hi = __builtin_bit_cast(unsigned short, tile[j * 8 + 2 * e + 1][c]);
          w[e] = lo | (hi << 16);
        }
        *reinterpret_cast<uint4*>(out + (c0 + c) * ldo + r0 + j * 8) = make_uint4(w[0], w[1], w[2], w[3]);
      }
      return;
    }
  }
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int64_t r = r0 + i, c = c0 + tx;
    if (r < R && c < C) tile[i][tx] = in[r * ldi + c];
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (r < R && c < C) out[c * ldo + r] = tile[tx][i];
  }
}

// out[c * ldo + r] = (TO) in[r * ldi + c] for logits of another dtype TI
// (fp32 or the other 16-bit type), rounded once to the compute dtype TO, as
// the reference's per-chunk cast of precomputed teacher logits does
// (ops/precomputed_teacher.py:343-348).  fp32 into a 16-bit TO moves 16
// bytes per access in full tiles with 16-byte aligned rows: thread -> rows
// tid / 16 + 16 h (h < 4), 4 columns tid % 16 on the way in (converted into
// LDS); the way out as k_transpose's 16-bit path.
template <class TI, class TO>
__global__ __launch_bounds__(256) void k_transpose_cast(const TI* __restrict__ in, int64_t ldi, TO* __restrict__ out,
                                                        int64_t ldo, int64_t R, int64_t C, int tiles_c, int vec) {
  __shared__ __align__(16) TO tile[64][72];
  const int tr = blockIdx.x / tiles_c, tc = blockIdx.x % tiles_c;
  const int64_t r0 = (int64_t)tr * 64, c0 = (int64_t)tc * 64;
  if constexpr (sizeof(TI) == 4 && sizeof(TO) == 2) {
    if (vec && r0 + 64 <= R && c0 + 64 <= C) {  // block-uniform
      {
        const int j = threadIdx.x & 15, i0 = threadIdx.x >> 4;
#pragma unroll
        for (int h = 0; h < 4; ++h) {
          const int i = i0 + 16 * h;
          const float4 v = *reinterpret_cast<const float4*>(in + (r0 + i) * ldi + c0 + j * 4);
          *reinterpret_cast<uint2*>(&tile[i][j * 4]) = make_uint2(pack2<TO>(v.x, v.y), pack2<TO>(v.z, v.w));
        }
      }
      __syncthreads();
      const int j = threadIdx.x & 7, i0 = threadIdx.x >> 3;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = i0 + 32 * h;
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const uint32_t lo = __builtin_bit_cast(unsigned short, tile[j * 8 + 2 * e][c]);
          const uint32_t hi = __builtin_bit_cast(unsigned short, tile[j * 8 + 2 * e + 1][c]);
          w[e] = lo | (hi << 16);
        }
        *reinterpret_cast<uint4*>(out + (c0 + c) * ldo + r0 + j * 8) = make_uint4(w[0], w[1], w[2], w[3]);
      }
      return;
    }
  }
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int i = ty; i < 64; i += 4) {
    const int64_t r = r0 + i, c = c0 + tx;
    if (r < R && c < C) tile[i][tx] = from_f32<TO>(to_f32(in[r * ldi + c]));
  }
  __syncthreads();
  for (int i = ty; i < 64; i += 4) {
    const int64_t c = c0 + i, r = r0 + tx;
    if (r < R && c < C) out[c * ldo + r] = tile[tx][i];
  }
}

// ------------------------------------------------------------ label logits
// x_s[t, y_t] and x_t[t, y_t] (the logits at each row's label) as fp32 dot
// products, one wave per row: 16-byte loads (8 bf16/f16 or 4 fp32 per lane)
// when the rows allow it, four independent partial sums per lane.  Labels
// outside [0, V) use class 0, as the reference kernels do
// (ops/tied_teacher.py:42-44); ignored rows give 0.
template <class T>
__device__ __forceinline__ float row_dot(const T* a, const T* b, int64_t H, int lane) {
  constexpr int E = 16 / sizeof(T);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  if (H % E == 0 && (reinterpret_cast<uintptr_t>(a) & 15) == 0 && (reinterpret_cast<uintptr_t>(b) & 15) == 0) {
    const int64_t nc = H / E;
#pragma unroll 2
    for (int64_t c = lane; c < nc; c += 64) {
      union { uint4 u; T e[E]; } va, vb;
      va.u = *reinterpret_cast<const uint4*>(a + c * E);
      vb.u = *reinterpret_cast<const uint4*>(b + c * E);
#pragma unroll
      for (int i = 0; i < E; ++i) acc[i & 3] += to_f32(va.e[i]) * to_f32(vb.e[i]);
    }
  } else {
    for (int64_t k = lane; k < H; k += 64) acc[0] += to_f32(a[k]) * to_f32(b[k]);
  }
  return (acc[0] + acc[1]) + (acc[2] + acc[3]);
}

// ------------------------------------------------------------ fp8 operands
// One wave per row (see QuantParams): the row's amax, the E8M0 exponent e
// with amax 2^-e in (224, 448] (amax = m 2^k, m in [0.5, 1): e = k - 9, or
// k - 8 when m > 0.875), and the row scaled by 2^-e (exact) and rounded to
// e4m3 with v_cvt_pk_fp8_f32.
template <class T>
__global__ __launch_bounds__(256) void k_quant_f8(QuantParams P) {
  static_assert(sizeof(T) == 2, "16-bit rows");
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= P.rows) return;  // whole waves
  const T* x = static_cast<const T*>(P.x) + r * P.H;
  const int64_t nc = P.H / 8;  // 16-byte pieces of 8 elements
  float amax = 0.f;
  for (int64_t c = lane; c < nc; c += 64) {
    union { uint4 u; T e[8]; } v;
    v.u = *reinterpret_cast<const uint4*>(x + c * 8);
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(to_f32(v.e[i])));
  }
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o));
  int e = 0;
  if (amax > 0.f) {
    int k;
    const float m = frexpf(amax, &k);
    e = k - 9 + (m > 0.875f ? 1 : 0);
    e = e < -127 ? -127 : (e > 127 ? 127 : e);
  }
  const float sc = ldexpf(1.0f, -e);
  uint8_t* q = P.q + r * P.H;
  for (int64_t c = lane; c < nc; c += 64) {
    union { uint4 u; T e[8]; } v;
    v.u = *reinterpret_cast<const uint4*>(x + c * 8);
    int w0 = 0, w1 = 0;
    w0 = __builtin_amdgcn_cvt_pk_fp8_f32(to_f32(v.e[0]) * sc, to_f32(v.e[1]) * sc, w0, false);
    w0 = __builtin_amdgcn_cvt_pk_fp8_f32(to_f32(v.e[2]) * sc, to_f32(v.e[3]) * sc, w0, true);
    w1 = __builtin_amdgcn_cvt_pk_fp8_f32(to_f32(v.e[4]) * sc, to_f32(v.e[5]) * sc, w1, false);
    w1 = __builtin_amdgcn_cvt_pk_fp8_f32(to_f32(v.e[6]) * sc, to_f32(v.e[7]) * sc, w1, true);
    *reinterpret_cast<uint2*>(q + c * 8) = make_uint2((uint32_t)w0, (uint32_t)w1);
  }
  if (lane == 0) P.e[r] = (uint8_t)(e + 127);
}

// Lane share of the dot product of two e4m3 rows of H bytes (16-byte
// pieces; unscaled).
__device__ __forceinline__ float row_dot_f8(const uint8_t* a, const uint8_t* b, int64_t H, int lane) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  float acc = 0.f;
  for (int64_t c = lane; c < H / 16; c += 64) {
    const uint4 va = *reinterpret_cast<const uint4*>(a + c * 16);
    const uint4 vb = *reinterpret_cast<const uint4*>(b + c * 16);
    const uint32_t wa[4] = {va.x, va.y, va.z, va.w}, wb[4] = {vb.x, vb.y, vb.z, vb.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f2v a0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)wa[i], false), a1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)wa[i], true);
      const f2v b0 = __builtin_amdgcn_cvt_pk_f32_fp8((int)wb[i], false), b1 = __builtin_amdgcn_cvt_pk_f32_fp8((int)wb[i], true);
      acc += a0.x * b0.x + a0.y * b0.y + a1.x * b1.x + a1.y * b1.y;
    }
  }
  return acc;
}

template <class T>
__global__ __launch_bounds__(256) void k_label(LabelParams P) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= P.N) return;
  const int64_t y = P.labels[t];
  const int64_t yc = (y >= 0 && y < P.V) ? y : 0;
  const bool ignored = (y == P.ignore_index);
  float xs = 0.f, xt = 0.f;
  const bool f8 = P.W8 != nullptr;  // the scan's fp8 rows and scales (tied teacher: both)
  if (!ignored) {
    if (f8) {
      const uint8_t* w8 = static_cast<const uint8_t*>(P.W8) + yc * P.H;
      xs = row_dot_f8(static_cast<const uint8_t*>(P.hs8) + t * P.H, w8, P.H, lane);
      if (P.tsrc == TSRC_SHARED) xt = row_dot_f8(static_cast<const uint8_t*>(P.ht8) + t * P.H, w8, P.H, lane);
    } else {
      xs = row_dot(static_cast<const T*>(P.hs) + t * P.H, static_cast<const T*>(P.W) + yc * P.H, P.H, lane);
      if (P.tsrc == TSRC_SHARED || P.tsrc == TSRC_SEP)
        xt = row_dot(static_cast<const T*>(P.ht) + t * P.Ht,
                     static_cast<const T*>(P.tsrc == TSRC_SHARED ? P.W : P.Wt) + yc * P.Ht, P.Ht, lane);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    xs += __shfl_xor(xs, o);
    xt += __shfl_xor(xt, o);
  }
  if (f8 && !ignored) {
    xs = ldexpf(xs, (int)P.eW[yc] + (int)P.eS[t] - 254);
    if (P.tsrc == TSRC_SHARED) xt = ldexpf(xt, (int)P.eW[yc] + (int)P.eT[t] - 254);
  }
  if (lane == 0) {
    if (P.tsrc == TSRC_MEM && !ignored) {
      const int64_t off = t * P.V + yc;
      if (P.lt_dtype == DT_F32) xt = static_cast<const float*>(P.Lt)[off];
      else if (P.lt_dtype == DT_BF16) xt = (float)static_cast<const bf16*>(P.Lt)[off];
      else xt = (float)static_cast<const f16*>(P.Lt)[off];
      xt = to_f32(from_f32<T>(xt));  // as the compute dtype holds it
    }
    P.out[t] = xs;
    P.out[P.N + t] = xt;
  }
}

// ------------------------------------------------------------- launchers
// Scan variant for phase 0 (statistics) or phase 1 (two-pass row sums).
inline int scan_variant_of(const FusedParams& P) {
  if (P.phase == 1) {
    switch (P.div) {
      case DIV_JSD: return SV_JSD;
      case DIV_SKEW_F: return SV_SKEW_F;
      case DIV_SKEW_R: return SV_SKEW_R;
      default: return SV_TVD;
    }
  }
  if (P.tsrc == TSRC_NONE) return P.t_is_one ? SV_STUDENT : SV_STUDENT_T;
  if (P.fam == FAM_LIN) return P.t_is_one ? SV_LIN_T1 : SV_LIN;
  if (P.fam == FAM_POW) return P.npow == 1 ? SV_POW1 : SV_POW;
  return P.t_is_one ? SV_TCE_T1 : SV_TCE;
}

template <class T>
hipError_t launch_scan_t(const FusedParams& P, int grid, hipStream_t s);
template <class T>
hipError_t launch_dl_t(const FusedParams& P, int grid, hipStream_t s);

// The ring engine takes the 16-bit tied problems (K > 64); the rest run on
// the two-stage engine.
template <class T>
inline bool scan_on_ring(const FusedParams& P) {
  return sizeof(T) == 2 && P.tsrc == TSRC_SHARED && P.H > 64;
}
#define ORDA_SCAN_CASE(T, SV)                                                                    \
  case SV:                                                                                       \
    if constexpr (sizeof(T) == 2) {                                                              \
      if (scan_on_ring<T>(P)) {                                                                  \
        hipLaunchKernelGGL((k_scan16<T, SV, false>), dim3(grid), dim3(kThreads4), 0, s, P);      \
        break;                                                                                   \
      }                                                                                          \
    }                                                                                            \
    hipLaunchKernelGGL((k_scan<T, SV>), dim3(grid), dim3(kThreads), 0, s, P);                    \
    break;
#define ORDA_DL_CASE(T, D) \
  case D: hipLaunchKernelGGL((k_dl<T, D, false>), dim3(grid), dim3(kThreads), 0, s, P); break;

#define ORDA_INSTANTIATE_SCAN(T)                                                     \
  template <> hipError_t launch_scan<T>(const FusedParams& P, int grid, hipStream_t s) { \
    switch (scan_variant_of(P)) {                                                    \
      ORDA_SCAN_CASE(T, SV_STUDENT)                                                  \
      ORDA_SCAN_CASE(T, SV_STUDENT_T)                                                \
      ORDA_SCAN_CASE(T, SV_TCE_T1)                                                   \
      ORDA_SCAN_CASE(T, SV_TCE)                                                      \
      ORDA_SCAN_CASE(T, SV_LIN_T1)                                                   \
      ORDA_SCAN_CASE(T, SV_LIN)                                                      \
      ORDA_SCAN_CASE(T, SV_POW)                                                      \
      ORDA_SCAN_CASE(T, SV_POW1)                                                     \
      ORDA_SCAN_CASE(T, SV_JSD)                                                      \
      ORDA_SCAN_CASE(T, SV_SKEW_F)                                                   \
      ORDA_SCAN_CASE(T, SV_SKEW_R)                                                   \
      ORDA_SCAN_CASE(T, SV_TVD)                                                      \
      default: return hipErrorInvalidValue;                                          \
    }                                                                                \
    return hipGetLastError();                                                        \
  }

#define ORDA_INSTANTIATE_DL(T)                                                       \
  template <> hipError_t launch_dl<T>(const FusedParams& P, int grid, hipStream_t s) {   \
    const bool t1 = P.t_is_one != 0;                                                 \
    switch (P.div) {                                                                 \
      case -1: hipLaunchKernelGGL((k_dl<T, -1, true>), dim3(grid), dim3(kThreads), 0, s, P); break; \
      case DIV_FKL:                                                                  \
        if (t1) hipLaunchKernelGGL((k_dl<T, DIV_FKL, true>), dim3(grid), dim3(kThreads), 0, s, P); \
        else hipLaunchKernelGGL((k_dl<T, DIV_FKL, false>), dim3(grid), dim3(kThreads), 0, s, P); \
        break;                                                                       \
      case DIV_SOFT:                                                                 \
        if (t1) hipLaunchKernelGGL((k_dl<T, DIV_SOFT, true>), dim3(grid), dim3(kThreads), 0, s, P); \
        else hipLaunchKernelGGL((k_dl<T, DIV_SOFT, false>), dim3(grid), dim3(kThreads), 0, s, P); \
        break;                                                                       \
      ORDA_DL_CASE(T, DIV_RKL)                                                       \
      ORDA_DL_CASE(T, DIV_SYM)                                                       \
      ORDA_DL_CASE(T, DIV_HELL)                                                      \
      ORDA_DL_CASE(T, DIV_BHAT)                                                      \
      ORDA_DL_CASE(T, DIV_RENYI)                                                     \
      ORDA_DL_CASE(T, DIV_AMARI)                                                     \
      ORDA_DL_CASE(T, DIV_CHI2)                                                      \
      ORDA_DL_CASE(T, DIV_L2)                                                        \
      ORDA_DL_CASE(T, DIV_AB)                                                        \
      ORDA_DL_CASE(T, DIV_JSD)                                                       \
      ORDA_DL_CASE(T, DIV_SKEW_F)                                                    \
      ORDA_DL_CASE(T, DIV_SKEW_R)                                                    \
      ORDA_DL_CASE(T, DIV_TVD)                                                       \
      default: return hipErrorInvalidValue;                                          \
    }                                                                                \
    return hipGetLastError();                                                        \
  }

template <class T>
hipError_t launch_gemm(const GemmParams& P, hipStream_t s) {
  const int grid = P.tiles_m * P.tiles_n;
  hipLaunchKernelGGL(k_gemm<T>, dim3(grid), dim3(kThreads), 0, s, P);
  return hipGetLastError();
}
template <class T>
hipError_t launch_transpose(const void* in, int64_t ldi, void* out, int64_t ldo, int64_t R, int64_t C,
                            hipStream_t s) {
  const int tiles_r = (int)((R + 63) / 64), tiles_c = (int)((C + 63) / 64);
  const int vec = sizeof(T) == 2 && ldi % 8 == 0 && ldo % 8 == 0 && reinterpret_cast<uintptr_t>(in) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(out) % 16 == 0;
  hipLaunchKernelGGL(k_transpose<T>, dim3(tiles_r * tiles_c), dim3(256), 0, s, static_cast<const T*>(in), ldi,
                     static_cast<T*>(out), ldo, R, C, tiles_c, vec);
  return hipGetLastError();
}

template <class T>
hipError_t launch_transpose_cast(const void* in, int in_dtype, int64_t ldi, void* out, int64_t ldo, int64_t R,
                                 int64_t C, hipStream_t s) {
  const int tiles_r = (int)((R + 63) / 64), tiles_c = (int)((C + 63) / 64);
  const dim3 grid((unsigned)(tiles_r * tiles_c));
  const int vec = ldi % 4 == 0 && ldo % 8 == 0 && reinterpret_cast<uintptr_t>(in) % 16 == 0 &&
                  reinterpret_cast<uintptr_t>(out) % 16 == 0;
  switch (in_dtype) {
    case DT_F32:
      hipLaunchKernelGGL((k_transpose_cast<float, T>), grid, dim3(256), 0, s, static_cast<const float*>(in), ldi,
                         static_cast<T*>(out), ldo, R, C, tiles_c, vec);
      break;
    case DT_BF16:
      hipLaunchKernelGGL((k_transpose_cast<bf16, T>), grid, dim3(256), 0, s, static_cast<const bf16*>(in), ldi,
                         static_cast<T*>(out), ldo, R, C, tiles_c, 0);
      break;
    case DT_F16:
      hipLaunchKernelGGL((k_transpose_cast<f16, T>), grid, dim3(256), 0, s, static_cast<const f16*>(in), ldi,
                         static_cast<T*>(out), ldo, R, C, tiles_c, 0);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <class T>
hipError_t launch_label(const LabelParams& P, hipStream_t s) {
  const int grid = (int)((P.N + 3) / 4);
  hipLaunchKernelGGL(k_label<T>, dim3(grid), dim3(256), 0, s, P);
  return hipGetLastError();
}

// ------------------------------------------------------- top-k teachers
// Sum over the 64 lanes of a wave, in every lane.
__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
  return x;
}

// The student's logits at the teacher's ids, x_s[t][i] = <hs_t, W[id_ti]> in
// fp32, into P.corr[t][i] (k_topk_rows reads them there and overwrites them
// with the dlogits share).  One wave per (token, group of kTopkIds ids): the
// hidden row's 16-byte pieces and those of kTopkIds weight rows are loaded
// together (the rows are independent gathers, so many loads are in flight),
// then one wave sum per id.  Ids outside [0, V) are clamped into range (the
// caller's contract is distinct ids in range: no fault either way).
constexpr int kTopkIds = 4;
template <class T>
__global__ __launch_bounds__(256) void k_topk_logits(TopKParams P) {
  constexpr int E = 16 / sizeof(T);
  const int lane = threadIdx.x & 63;
  const int64_t groups = (P.k + kTopkIds - 1) / kTopkIds;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= P.N * groups) return;  // whole waves
  const int64_t t = item / groups;
  const int64_t i0 = (item - t * groups) * kTopkIds;
  const T* hs = static_cast<const T*>(P.hs) + t * P.H;
  const T* W = static_cast<const T*>(P.W);
  const T* rows[kTopkIds];
#pragma unroll
  for (int j = 0; j < kTopkIds; ++j) {
    int64_t v = i0 + j < P.k ? P.idx[t * P.k + i0 + j] : 0;
    v = (v >= 0 && v < P.V) ? v : 0;
    rows[j] = W + v * P.H;
  }
  float acc[kTopkIds];
#pragma unroll
  for (int j = 0; j < kTopkIds; ++j) acc[j] = 0.f;
  const int64_t nc = P.H / E;  // H is a multiple of E (16-byte rows)
#pragma unroll 2
  for (int64_t c = lane; c < nc; c += 64) {
    union U { uint4 u; T e[E]; };
    U h, w[kTopkIds];
    h.u = *reinterpret_cast<const uint4*>(hs + c * E);
#pragma unroll
    for (int j = 0; j < kTopkIds; ++j) w[j].u = *reinterpret_cast<const uint4*>(rows[j] + c * E);
#pragma unroll
    for (int j = 0; j < kTopkIds; ++j)
#pragma unroll
      for (int e = 0; e < E; ++e) acc[j] += to_f32(h.e[e]) * to_f32(w[j].e[e]);
  }
#pragma unroll
  for (int j = 0; j < kTopkIds; ++j) {
    const float d = wave_sum(acc[j]);
    if (lane == 0 && i0 + j < P.k) P.corr[t * P.k + i0 + j] = d;
  }
}

// Per token of the chunk (one wave each), from the student logits at its ids
// (k_topk_logits, in P.corr): the teacher renormalised over its ids at
// temperature T (online max / sum of lp / T), the divergence row D (forward
// KL: sum p_t (log p_t - log p_s^T); soft-target CE: -sum p_t log p_s^T)
// times T^2, and the ids' share of the student's dlogits,
// -mean_scale w_kl T p_t, over P.corr (each lane reads its ids' logits before
// it writes their share; scattered after the dense pass).  Ids of
// log-probability -inf add nothing.  Sets the row's teacher log-normaliser to
// +inf so the dense pass sees a zero teacher.
template <class T>
__global__ __launch_bounds__(256) void k_topk_rows(TopKParams P) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= P.N) return;  // whole waves
  const int64_t y = P.labels[t];
  const bool ignored = y == P.ignore_index;
  const float invT = P.invT;
  const float lse_sT = P.lse_sT[t];
  const float* xk = P.corr + t * P.k;
  const float* lp = P.lp + t * P.k;
  float m = -kInf, sum = 0.f, a = 0.f;
  for (int64_t c0 = 0; c0 < P.k; c0 += 64) {
    const int cnt = (int)min<int64_t>(64, P.k - c0);
    const float mine = lane < cnt ? xk[c0 + lane] : 0.f;
    const float z = lane < cnt ? lp[c0 + lane] * invT : -kInf;
    if (z > -kInf) {  // (an id of probability 0 adds nothing)
      const float nm = fmaxf(m, z);
      const float sc = m == -kInf ? 0.f : fexp(m - nm);
      const float e = fexp(z - nm);
      sum = sum * sc + e;
      a = a * sc + e * (P.div == DIV_FKL ? z - mine * invT : mine * invT);
      m = nm;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float m2 = __shfl_xor(m, off), s2 = __shfl_xor(sum, off), a2 = __shfl_xor(a, off);
    const float nm = fmaxf(m, m2);
    const float c1 = m == -kInf ? 0.f : fexp(m - nm), c2 = m2 == -kInf ? 0.f : fexp(m2 - nm);
    sum = sum * c1 + s2 * c2;
    a = a * c1 + a2 * c2;
    m = nm;
  }
  const float lse_p = m + flog(sum);
  const float D = P.div == DIV_FKL ? a / sum - lse_p + lse_sT : lse_sT - a / sum;
  if (lane == 0) {
    P.rowv[2 * P.ldv + t] = ignored ? 0.f : P.temperature * P.temperature * D;
    P.rowp[3 * P.N + t] = kInf;
  }
  // an ignored row writes exact zeros: with every id at -inf its lse_p is
  // -inf and the products below would be NaN (0 * NaN), which the scatter
  // would carry into the gradients
  const float sc = ignored ? 0.f : -P.mean_scale[0] * P.w_kl * P.temperature;
  float* corr = P.corr + t * P.k;
  for (int64_t i = lane; i < P.k; i += 64) corr[i] = ignored ? 0.f : sc * fexp(lp[i] * invT - lse_p);
}

// L[id][t] += corr[t][i] for every token t of the chunk and each of its k ids
// (the chunk's dlogits, in T; distinct ids per token, so no two threads
// touch one element).
template <class T>
__global__ __launch_bounds__(256) void k_topk_scatter(TopKParams P) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= P.N * P.k) return;
  const int64_t t = g / P.k;
  int64_t v = P.idx[g];
  v = (v >= 0 && v < P.V) ? v : 0;
  T* e = static_cast<T*>(P.L) + v * P.ldL + t;
  *e = from_f32<T>(to_f32(*e) + P.corr[g]);
}

// ------------------------------------------------ student RMSNorm prologue
// Sum over the 256 threads of a block, in every thread (wave sums, then the
// four waves' partials through LDS in a fixed order).
__device__ __forceinline__ float block_sum256(float x, float* red) {
  x = wave_sum(x);
  __syncthreads();  // red is free (a previous call's reads are done)
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// One block per row: y = x * r * gamma with r = rsqrt(sum(x^2) / D + eps),
// in fp32 from the row's 4-element groups, rounded once to T (the reference
// producer's RMSNorm, test/benchmark/src/core.py:13-14, computes the same
// product in the activation dtype).
template <class T>
__global__ __launch_bounds__(256) void k_rmsnorm_fwd(NormParams P) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t t = blockIdx.x;
  const T* x = static_cast<const T*>(P.x) + t * P.H;
  const T* g = static_cast<const T*>(P.gamma);
  T* y = static_cast<T*>(P.y) + t * P.H;
  const int64_t ng = P.H / 4;
  float ss = 0.f;
  for (int64_t c = tid; c < ng; c += 256) {
    float v[4];
    load4(x + c * 4, v, true, 4);
    ss += (v[0] * v[0] + v[1] * v[1]) + (v[2] * v[2] + v[3] * v[3]);
  }
  ss = block_sum256(ss, red);
  const float r = rsqrtf(ss / (float)P.D + P.eps);
  if (tid == 0) P.rstd[t] = r;
  for (int64_t c = tid; c < ng; c += 256) {
    float v[4], w[4];
    load4(x + c * 4, v, true, 4);
    load4(g + c * 4, w, true, 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = v[e] * r * w[e];
    store4(y + c * 4, v, true, 4);
  }
}

// dloss/dgamma_h = sum_t dy[t][h] x[t][h] r_t: one thread per column h and
// token group (blockIdx.y), a sequential sum over the group's tokens into
// gpart[group][h]; then (k_rmsnorm_gacc) the groups summed in order into gacc,
// and on the last chunk the result in T.
template <class T>
__global__ __launch_bounds__(256) void k_rmsnorm_dgamma(NormParams P) {
  // four consecutive columns per thread (one 8-byte load per row for 16-bit
  // types), tokens of the group walked in order
  const int64_t h = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (h >= P.H) return;  // H is a multiple of 4
  const int64_t per = (P.N + P.groups - 1) / P.groups;
  const int64_t t0 = (int64_t)blockIdx.y * per;
  const int64_t t1 = min<int64_t>(P.N, t0 + per);
  const T* dy = static_cast<const T*>(P.dxy);
  const T* x = static_cast<const T*>(P.x);
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int64_t t = t0; t < t1; ++t) {
    float d[4], v[4];
    load4(dy + t * P.H + h, d, true, 4);
    load4(x + t * P.H + h, v, true, 4);
    const float r = P.rstd[t];
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += d[e] * v[e] * r;
  }
  float* o = P.gpart + (int64_t)blockIdx.y * P.H + h;
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = acc[e];
}
// (32 columns per block, 8 group lanes per column: lane l sums groups l,
// l + 8, ... in order, then the 8 lane sums are added in order.)
template <class T>
__global__ __launch_bounds__(256) void k_rmsnorm_gacc(NormParams P) {
  __shared__ float red[8][32];
  const int c = threadIdx.x & 31, gl = threadIdx.x >> 5;
  const int64_t h = (int64_t)blockIdx.x * 32 + c;
  float s = 0.f;
  if (h < P.H) {
#pragma unroll 4
    for (int gi = gl; gi < P.groups; gi += 8) s += P.gpart[(int64_t)gi * P.H + h];
  }
  red[gl][c] = s;
  __syncthreads();
  if (gl != 0 || h >= P.H) return;
  float a = red[0][c];
#pragma unroll
  for (int k = 1; k < 8; ++k) a += red[k][c];
  const float tot = P.first ? a : P.gacc[h] + a;
  P.gacc[h] = tot;
  if (P.gout) static_cast<T*>(P.gout)[h] = from_f32<T>(tot);
}

// dloss/dx = r (gamma . dy) - x r^3 <gamma . dy, x> / D, in place over dy
// (one block per row; two passes over the row).
template <class T>
__global__ __launch_bounds__(256) void k_rmsnorm_bwd(NormParams P) {
  __shared__ float red[4];
  const int tid = threadIdx.x;
  const int64_t t = blockIdx.x;
  const T* x = static_cast<const T*>(P.x) + t * P.H;
  const T* g = static_cast<const T*>(P.gamma);
  T* d = static_cast<T*>(P.dxy) + t * P.H;
  const int64_t ng = P.H / 4;
  float c = 0.f;
  for (int64_t i = tid; i < ng; i += 256) {
    float v[4], w[4], dy[4];
    load4(x + i * 4, v, true, 4);
    load4(g + i * 4, w, true, 4);
    load4(d + i * 4, dy, true, 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) c += w[e] * dy[e] * v[e];
  }
  c = block_sum256(c, red);
  const float r = P.rstd[t];
  const float k = r * r * r * c / (float)P.D;
  for (int64_t i = tid; i < ng; i += 256) {
    float v[4], w[4], dy[4];
    load4(x + i * 4, v, true, 4);
    load4(g + i * 4, w, true, 4);
    load4(d + i * 4, dy, true, 4);
#pragma unroll
    for (int e = 0; e < 4; ++e) dy[e] = r * w[e] * dy[e] - v[e] * k;
    store4(d + i * 4, dy, true, 4);
  }
}

// Materialised path: scan variants with the logits store (phase 0 only).
#define ORDA_SCANST_CASE(T, SV)                                                                  \
  case SV:                                                                                       \
    if constexpr (sizeof(T) == 2) {                                                              \
      if (P.tsrc == TSRC_NONE && P.student_ring) {                                               \
        if constexpr (SV == SV_STUDENT || SV == SV_STUDENT_T)                                    \
          hipLaunchKernelGGL((k_scan16<T, SV, true, TL_STUDENT>), dim3(grid), dim3(kThreads4), 0, s, P); \
        else                                                                                     \
          return hipErrorInvalidValue;                                                           \
        break;                                                                                   \
      }                                                                                          \
      if (P.tsrc == TSRC_L || P.tsrc == TSRC_MEM_RING) {                                         \
        if constexpr (SV == SV_STUDENT || SV == SV_STUDENT_T || SV == SV_POW)                  \
          return hipErrorInvalidValue;                                                           \
        else if (P.tsrc == TSRC_L)                                                               \
          hipLaunchKernelGGL((k_scan4<T, SV, true, TL_FROM_L>), dim3(grid), dim3(kThreads4), 0, s, P); \
        else                                                                                     \
          hipLaunchKernelGGL((k_scan16<T, SV, true, TL_FROM_MEM>), dim3(grid), dim3(kThreads4), 0, s, P); \
        break;                                                                                   \
      }                                                                                          \
      if (scan_on_ring<T>(P)) {                                                                  \
        hipLaunchKernelGGL((k_scan16<T, SV, true>), dim3(grid), dim3(kThreads4), 0, s, P);       \
        break;                                                                                   \
      }                                                                                          \
    }                                                                                            \
    hipLaunchKernelGGL((k_scan<T, SV, true>), dim3(grid), dim3(kThreads), 0, s, P);              \
    break;
#define ORDA_INSTANTIATE_SCAN_STORE(T)                                                     \
  template <> hipError_t launch_scan_store<T>(const FusedParams& P, int grid, hipStream_t s) { \
    if (P.phase != 0) return hipErrorInvalidValue;                                         \
    if ((P.tsrc == TSRC_L || P.tsrc == TSRC_MEM_RING) && (sizeof(T) != 2 || P.H <= 64))    \
      return hipErrorInvalidValue;                                                         \
    if (P.tsrc == TSRC_MEM_RING && P.V % 4 != 0) return hipErrorInvalidValue;              \
    switch (scan_variant_of(P)) {                                                          \
      ORDA_SCANST_CASE(T, SV_STUDENT)                                                      \
      ORDA_SCANST_CASE(T, SV_STUDENT_T)                                                    \
      ORDA_SCANST_CASE(T, SV_TCE_T1)                                                       \
      ORDA_SCANST_CASE(T, SV_TCE)                                                          \
      ORDA_SCANST_CASE(T, SV_LIN_T1)                                                       \
      ORDA_SCANST_CASE(T, SV_LIN)                                                          \
      ORDA_SCANST_CASE(T, SV_POW)                                                          \
      ORDA_SCANST_CASE(T, SV_POW1)                                                         \
      default: return hipErrorInvalidValue;                                                \
    }                                                                                      \
    return hipGetLastError();                                                              \
  }

// fp8 logits: the ring scans with e4m3 operands (tied teacher, precomputed
// logits read by the ring scan, no teacher).
#define ORDA_SCANF8_CASE(T, SV)                                                                  \
  case SV:                                                                                       \
    if (P.tsrc == TSRC_NONE) {                                                                   \
      if constexpr (SV == SV_STUDENT || SV == SV_STUDENT_T)                                      \
        hipLaunchKernelGGL((k_scan4<T, SV, true, TL_STUDENT, true>), dim3(grid), dim3(kThreads4), 0, s, P); \
      else                                                                                       \
        return hipErrorInvalidValue;                                                             \
    } else if (P.tsrc == TSRC_MEM_RING) {                                                        \
      if constexpr (SV == SV_STUDENT || SV == SV_STUDENT_T || SV == SV_POW || SV == SV_POW1)      \
        return hipErrorInvalidValue;                                                             \
      else                                                                                       \
        hipLaunchKernelGGL((k_scan4<T, SV, true, TL_FROM_MEM, true>), dim3(grid), dim3(kThreads4), 0, s, P); \
    } else if (P.tsrc == TSRC_SHARED) {                                                          \
      if constexpr (SV == SV_STUDENT || SV == SV_STUDENT_T)                                      \
        return hipErrorInvalidValue;                                                             \
      else if (!P.ht8 || !P.eT)                                                                  \
        return hipErrorInvalidValue;                                                             \
      else                                                                                       \
        hipLaunchKernelGGL((k_scan4<T, SV, true, TL_NONE, true>), dim3(grid), dim3(kThreads4), 0, s, P); \
    } else {                                                                                     \
      return hipErrorInvalidValue;                                                               \
    }                                                                                            \
    break;
#define ORDA_INSTANTIATE_SCAN_F8(T)                                                        \
  template <> hipError_t launch_scan_store_f8<T>(const FusedParams& P, int grid, hipStream_t s) { \
    if (P.phase != 0 || !P.W8 || !P.hs8 || !P.eW || !P.eS || P.H % 16 != 0 || P.H <= 128) \
      return hipErrorInvalidValue;                                                         \
    if (P.tsrc == TSRC_MEM_RING && P.V % 4 != 0) return hipErrorInvalidValue;              \
    switch (scan_variant_of(P)) {                                                          \
      ORDA_SCANF8_CASE(T, SV_STUDENT)                                                      \
      ORDA_SCANF8_CASE(T, SV_STUDENT_T)                                                    \
      ORDA_SCANF8_CASE(T, SV_TCE_T1)                                                       \
      ORDA_SCANF8_CASE(T, SV_TCE)                                                          \
      ORDA_SCANF8_CASE(T, SV_LIN_T1)                                                       \
      ORDA_SCANF8_CASE(T, SV_LIN)                                                          \
      ORDA_SCANF8_CASE(T, SV_POW)                                                          \
      ORDA_SCANF8_CASE(T, SV_POW1)                                                         \
      default: return hipErrorInvalidValue;                                                \
    }                                                                                      \
    return hipGetLastError();                                                              \
  }

// General GEMM: the (layout, layout, mode) combinations the library uses.
// Persistent grid: one workgroup per CU (a 128 KiB-LDS workgroup fills a CU).
inline int persistent_groups() {
  static int cus = 0;
  if (cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}
template <class T, int LA, int LB, int MODE>
inline void gemm2_go(const GemmParams& P, hipStream_t s) {
  const int64_t total = (int64_t)P.tiles_m * P.tiles_n * P.splits;
  const int grid = (int)(total < persistent_groups() ? total : persistent_groups());
  // the ring engine (four waves, 160 KiB LDS) for the 16-bit K/K and MN/MN
  // GEMMs it covers
  if constexpr (sizeof(T) == 2 && LA == KMAJ && LB == KMAJ && (MODE == GEMM_STORE || MODE == GEMM_ACC_T)) {
    if (P.splits == 1 && P.K > 64) {
      hipLaunchKernelGGL((k_gemm4<T, KMAJ, KMAJ, MODE>), dim3(grid), dim3(kThreads4), 0, s, P);
      return;
    }
  }
  if constexpr (sizeof(T) == 2 && LA == KMAJ && LB == MNMAJ && (MODE == GEMM_STORE || MODE == GEMM_ACC_T)) {
    const int64_t lim = 0x7fffffffll / (int64_t)sizeof(T);
    if (P.splits == 1 && P.K > 64 && !P.B1 && P.b_kval0 * P.ldb < lim) {
      hipLaunchKernelGGL((k_gemm4<T, KMAJ, MNMAJ, MODE>), dim3(grid), dim3(kThreads4), 0, s, P);
      return;
    }
  }
  if constexpr (sizeof(T) == 2 && LA == MNMAJ && LB == MNMAJ && (MODE == GEMM_STORE || MODE == GEMM_SPLIT)) {
    const int64_t lim = 0x7fffffffll / (int64_t)sizeof(T);
    if (P.k_per_split > 64 && P.k_per_split * P.lda < lim && P.k_per_split * P.ldb < lim) {
      hipLaunchKernelGGL((k_gemm4<T, MNMAJ, MNMAJ, MODE>), dim3(grid), dim3(kThreads4), 0, s, P);
      return;
    }
  }
  hipLaunchKernelGGL((k_gemm2<T, LA, LB, MODE>), dim3(grid), dim3(kThreads), 0, s, P);
}
#define ORDA_INSTANTIATE_GEMM2(T)                                                          \
  template <> hipError_t launch_gemm2<T>(const GemmParams& P, hipStream_t s) {             \
    const int key = P.la * 100 + P.lb * 10 + P.mode;                                       \
    switch (key) {                                                                         \
      case KMAJ * 100 + MNMAJ * 10 + GEMM_STORE: gemm2_go<T, KMAJ, MNMAJ, GEMM_STORE>(P, s); break; \
      case KMAJ * 100 + MNMAJ * 10 + GEMM_ACC_T: gemm2_go<T, KMAJ, MNMAJ, GEMM_ACC_T>(P, s); break; \
      case MNMAJ * 100 + MNMAJ * 10 + GEMM_STORE: gemm2_go<T, MNMAJ, MNMAJ, GEMM_STORE>(P, s); break; \
      case MNMAJ * 100 + MNMAJ * 10 + GEMM_SPLIT: gemm2_go<T, MNMAJ, MNMAJ, GEMM_SPLIT>(P, s); break; \
      case KMAJ * 100 + KMAJ * 10 + GEMM_STORE: gemm2_go<T, KMAJ, KMAJ, GEMM_STORE>(P, s); break; \
      case KMAJ * 100 + KMAJ * 10 + GEMM_ACC_T: gemm2_go<T, KMAJ, KMAJ, GEMM_ACC_T>(P, s); break; \
      case MNMAJ * 100 + KMAJ * 10 + GEMM_STORE: gemm2_go<T, MNMAJ, KMAJ, GEMM_STORE>(P, s); break; \
      default: return hipErrorInvalidValue;                                                \
    }                                                                                      \
    return hipGetLastError();                                                              \
  }

// In-place dlogits variants (the divergences of families LIN and POW).
template <class T, int DIV, bool T1, bool NO_T = false>
inline void dlm_go(const DlmParams& P, hipStream_t s) {
  if constexpr (sizeof(T) == 2) {  // (teacher logits in place: 16-bit only)
    if (P.Ltm) {
      const dim3 grid((unsigned)((P.N + kTmTok - 1) / kTmTok), (unsigned)((P.V + kTmRows - 1) / kTmRows));
      hipLaunchKernelGGL((k_dlm_tm<T, DIV, T1>), grid, dim3(256), 0, s, P);
      return;
    }
  }
  const dim3 grid((unsigned)((P.N + 1023) / 1024), (unsigned)((P.V + P.rows_per_block - 1) / P.rows_per_block));
  hipLaunchKernelGGL((k_dlm<T, DIV, T1, NO_T>), grid, dim3(256), 0, s, P);
}
#define ORDA_DLM_CASE(T, D) \
  case D: dlm_go<T, D, false>(P, s); break;
// forward KL / soft-target CE: T = 1 specialised, and the no-teacher variant
// of a top-k teacher (P.no_t; its logits are never read in place)
#define ORDA_DLM_T1_CASE(T, D)                                   \
  if (P.no_t && P.Ltm) return hipErrorInvalidValue;              \
  if (P.no_t) {                                                  \
    if (t1) dlm_go<T, D, true, true>(P, s);                      \
    else dlm_go<T, D, false, true>(P, s);                        \
  } else if (t1) {                                               \
    dlm_go<T, D, true>(P, s);                                    \
  } else {                                                       \
    dlm_go<T, D, false>(P, s);                                   \
  }
#define ORDA_INSTANTIATE_FB(T)                                                             \
  template <> hipError_t launch_quant_f8<T>(const QuantParams& P, hipStream_t s) {         \
    if constexpr (sizeof(T) != 2) {                                                        \
      return hipErrorInvalidValue;                                                         \
    } else {                                                                               \
      if (!P.x || !P.q || !P.e || P.H % 16 != 0) return hipErrorInvalidValue;              \
      if (P.rows <= 0) return hipSuccess;                                                  \
      hipLaunchKernelGGL(k_quant_f8<T>, dim3((unsigned)((P.rows + 3) / 4)), dim3(256), 0, s, P); \
      return hipGetLastError();                                                            \
    }                                                                                      \
  }                                                                                        \
  template <> hipError_t launch_rmsnorm_fwd<T>(const NormParams& P, hipStream_t s) {       \
    if (!P.x || !P.gamma || !P.y || !P.rstd || P.H % 4 != 0 || P.D < 1 || P.D > P.H)       \
      return hipErrorInvalidValue;                                                         \
    if (P.N <= 0) return hipSuccess;                                                       \
    hipLaunchKernelGGL(k_rmsnorm_fwd<T>, dim3((unsigned)P.N), dim3(256), 0, s, P);         \
    return hipGetLastError();                                                              \
  }                                                                                        \
  template <> hipError_t launch_rmsnorm_dgamma<T>(const NormParams& P, hipStream_t s) {    \
    if (!P.x || !P.dxy || !P.rstd || !P.gpart || !P.gacc || P.groups < 1 || P.groups > 65535) \
      return hipErrorInvalidValue;                                                         \
    hipLaunchKernelGGL(k_rmsnorm_dgamma<T>, dim3((unsigned)((P.H + 1023) / 1024), (unsigned)P.groups), \
                       dim3(256), 0, s, P);                                                \
    hipLaunchKernelGGL(k_rmsnorm_gacc<T>, dim3((unsigned)((P.H + 31) / 32)), dim3(256), 0, s, P); \
    return hipGetLastError();                                                              \
  }                                                                                        \
  template <> hipError_t launch_rmsnorm_bwd<T>(const NormParams& P, hipStream_t s) {       \
    if (!P.x || !P.gamma || !P.dxy || !P.rstd || P.H % 4 != 0 || P.D < 1)                  \
      return hipErrorInvalidValue;                                                         \
    if (P.N <= 0) return hipSuccess;                                                       \
    hipLaunchKernelGGL(k_rmsnorm_bwd<T>, dim3((unsigned)P.N), dim3(256), 0, s, P);         \
    return hipGetLastError();                                                              \
  }                                                                                        \
  template <> hipError_t launch_topk_rows<T>(const TopKParams& P, hipStream_t s) {         \
    if (!P.hs || !P.W || !P.idx || !P.lp || !P.labels || !P.mean_scale || !P.lse_sT ||     \
        !P.rowp || !P.rowv || !P.corr || P.k < 1)                                          \
      return hipErrorInvalidValue;                                                         \
    if (P.N <= 0) return hipSuccess;                                                       \
    if (P.H % (16 / (int64_t)sizeof(T)) != 0) return hipErrorInvalidValue;                \
    const int64_t items = P.N * ((P.k + kTopkIds - 1) / kTopkIds);                         \
    hipLaunchKernelGGL(k_topk_logits<T>, dim3((unsigned)((items + 3) / 4)), dim3(256), 0, s, P); \
    hipLaunchKernelGGL(k_topk_rows<T>, dim3((unsigned)((P.N + 3) / 4)), dim3(256), 0, s, P); \
    return hipGetLastError();                                                              \
  }                                                                                        \
  template <> hipError_t launch_topk_scatter<T>(const TopKParams& P, hipStream_t s) {      \
    const int64_t n = P.N * P.k;                                                           \
    if (!P.idx || !P.corr || !P.L) return hipErrorInvalidValue;                            \
    if (n <= 0) return hipSuccess;                                                         \
    hipLaunchKernelGGL(k_topk_scatter<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, P); \
    return hipGetLastError();                                                              \
  }                                                                                        \
  template <> hipError_t launch_dlm<T>(const DlmParams& P, hipStream_t s) {                \
    const bool t1 = P.t_is_one != 0;                                                       \
    if (P.no_t && (P.tgrad || (P.div != -1 && P.div != DIV_FKL && P.div != DIV_SOFT)))     \
      return hipErrorInvalidValue; /* no teacher logits to read */                         \
    if (P.Ltm && (sizeof(T) != 2 || (P.V + kTmRows - 1) / kTmRows > 65535 || P.V % 8 != 0)) \
      return hipErrorInvalidValue; /* grid.y of k_dlm_tm; whole 16-byte teacher pieces */  \
    switch (P.div) {                                                                       \
      case -1: dlm_go<T, -1, true>(P, s); break;                                           \
      case DIV_FKL: ORDA_DLM_T1_CASE(T, DIV_FKL) break;                                    \
      case DIV_SOFT: ORDA_DLM_T1_CASE(T, DIV_SOFT) break;                                  \
      ORDA_DLM_CASE(T, DIV_RKL)                                                            \
      ORDA_DLM_CASE(T, DIV_SYM)                                                            \
      ORDA_DLM_CASE(T, DIV_HELL)                                                           \
      ORDA_DLM_CASE(T, DIV_BHAT)                                                           \
      ORDA_DLM_CASE(T, DIV_RENYI)                                                          \
      ORDA_DLM_CASE(T, DIV_AMARI)                                                          \
      ORDA_DLM_CASE(T, DIV_CHI2)                                                           \
      ORDA_DLM_CASE(T, DIV_L2)                                                             \
      ORDA_DLM_CASE(T, DIV_AB)                                                             \
      ORDA_DLM_CASE(T, DIV_JSD)                                                            \
      ORDA_DLM_CASE(T, DIV_SKEW_F)                                                         \
      ORDA_DLM_CASE(T, DIV_SKEW_R)                                                         \
      ORDA_DLM_CASE(T, DIV_TVD)                                                            \
      default: return hipErrorInvalidValue;                                                \
    }                                                                                      \
    return hipGetLastError();                                                              \
  }                                                                                        \
  template <> hipError_t launch_two<T>(const TwoParams& P, hipStream_t s) {                \
    if (P.n_ranges <= 0 || P.n_ranges > 65535 || P.rows_per_range <= 0) return hipErrorInvalidValue; \
    const dim3 grid((unsigned)((P.N + kTwoTok - 1) / kTwoTok), (unsigned)P.n_ranges);     \
    if (P.Ltm) {                                                                           \
      if (sizeof(T) != 2 || P.rows_per_range % kTmRows != 0 || P.V % 8 != 0)               \
        return hipErrorInvalidValue;                                                       \
      if constexpr (sizeof(T) == 2) switch (P.div) {                                       \
        case DIV_JSD: hipLaunchKernelGGL((k_two_rows_tm<T, DIV_JSD>), grid, dim3(256), 0, s, P); break; \
        case DIV_SKEW_F: hipLaunchKernelGGL((k_two_rows_tm<T, DIV_SKEW_F>), grid, dim3(256), 0, s, P); break; \
        case DIV_SKEW_R: hipLaunchKernelGGL((k_two_rows_tm<T, DIV_SKEW_R>), grid, dim3(256), 0, s, P); break; \
        case DIV_TVD: hipLaunchKernelGGL((k_two_rows_tm<T, DIV_TVD>), grid, dim3(256), 0, s, P); break; \
        case DIV_L2: hipLaunchKernelGGL((k_two_rows_tm<T, DIV_L2>), grid, dim3(256), 0, s, P); break; \
        case DIV_AB: hipLaunchKernelGGL((k_two_rows_tm<T, DIV_AB>), grid, dim3(256), 0, s, P); break; \
        default: return hipErrorInvalidValue;                                              \
      }                                                                                    \
      return hipGetLastError();                                                            \
    }                                                                                      \
    switch (P.div) {                                                                       \
      case DIV_JSD: hipLaunchKernelGGL((k_two_rows<T, DIV_JSD>), grid, dim3(256), 0, s, P); break; \
      case DIV_SKEW_F: hipLaunchKernelGGL((k_two_rows<T, DIV_SKEW_F>), grid, dim3(256), 0, s, P); break; \
      case DIV_SKEW_R: hipLaunchKernelGGL((k_two_rows<T, DIV_SKEW_R>), grid, dim3(256), 0, s, P); break; \
      case DIV_TVD: hipLaunchKernelGGL((k_two_rows<T, DIV_TVD>), grid, dim3(256), 0, s, P); break; \
      case DIV_L2: hipLaunchKernelGGL((k_two_rows<T, DIV_L2>), grid, dim3(256), 0, s, P); break; \
      case DIV_AB: hipLaunchKernelGGL((k_two_rows<T, DIV_AB>), grid, dim3(256), 0, s, P); break; \
      default: return hipErrorInvalidValue;                                                \
    }                                                                                      \
    return hipGetLastError();                                                              \
  }                                                                                        \
  template <>                                                                              \
  hipError_t launch_splitk_reduce<T>(const float* part, int splits, int64_t stride, void* out, int64_t ldo, \
                                     int64_t M, int64_t N, hipStream_t s) {                \
    const int64_t n = M * (N / 4);                                                        \
    hipLaunchKernelGGL(k_splitk_reduce<T>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, part, splits, \
                       stride, static_cast<T*>(out), ldo, M, N);                           \
    return hipGetLastError();                                                              \
  }                                                                                        \
  template <> hipError_t launch_scale<T>(void* x, int64_t n, const float* g, hipStream_t s) { \
    int64_t blocks = (n / 4 + 255) / 256;                                                  \
    if (blocks > 8192) blocks = 8192;                                                      \
    if (blocks < 1) blocks = 1;                                                            \
    hipLaunchKernelGGL(k_scale<T>, dim3((unsigned)blocks), dim3(256), 0, s, static_cast<T*>(x), n, g); \
    return hipGetLastError();                                                              \
  }

#define ORDA_INSTANTIATE_GEMM(T)                                                                     \
  template hipError_t launch_gemm<T>(const GemmParams&, hipStream_t);                                \
  template hipError_t launch_label<T>(const LabelParams&, hipStream_t);                              \
  template hipError_t launch_transpose<T>(const void*, int64_t, void*, int64_t, int64_t, int64_t,    \
                                          hipStream_t);                                              \
  template hipError_t launch_transpose_cast<T>(const void*, int, int64_t, void*, int64_t, int64_t, int64_t, \
                                               hipStream_t);

}  // namespace orda
