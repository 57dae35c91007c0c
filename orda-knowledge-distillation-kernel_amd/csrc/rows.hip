// rows.hip -- per-row merge of partial statistics, the loss reduction, and a
// 2-D zero fill.  These are O(N) kernels; the O(N V H) work is elsewhere.
#include "launch.hpp"
#include "orda_core.hpp"

namespace orda {

// 32 tokens per workgroup, 8 threads per token: thread (slice, token) merges
// the partial states of vocabulary ranges slice, slice + 8, ... in order, and
// the slice-0 thread then merges the 8 slice states in slice order (a fixed
// order: bit-stable), then forms the row losses and the parameters the
// dlogits kernel needs.  The final combination runs in fp64 to limit the
// cancellation in lse_s - lse_t + (cross term).
// x rounded to nearest-even in bf16 (code 1) or fp16 (code 2), as the
// logits stores convert it.
__device__ inline float round_to(float x, int code) {
  return code == 1 ? (float)(bf16)x : (float)(f16)x;
}

constexpr int kMergeSlices = 8;
constexpr int kMergeTok = 32;
__global__ __launch_bounds__(kMergeSlices * kMergeTok) void k_merge(MergeParams P) {
  __shared__ float xch[kMergeSlices - 1][kNStat][kMergeTok];
  __shared__ double xch1[kMergeSlices - 1][2][kMergeTok];
  const int tl = threadIdx.x % kMergeTok, slice = threadIdx.x / kMergeTok;
  const int64_t t = (int64_t)blockIdx.x * kMergeTok + tl;
  const bool live = t < P.N;
  const int64_t N = P.N;

  if (P.phase == 1) {
    double x0 = 0.0, x1 = 0.0;
    if (live)
      for (int vr = slice; vr < P.n_vranges; vr += kMergeSlices) {
        const float* s = P.two_dense ? P.partial + (int64_t)vr * 2 * N + t : P.partial + (int64_t)vr * kNStat * N + 6 * N + t;
        x0 += s[0];
        x1 += s[N];
      }
    if (slice > 0) { xch1[slice - 1][0][tl] = x0; xch1[slice - 1][1][tl] = x1; }
    __syncthreads();
    if (slice > 0 || !live) return;
    for (int k = 0; k < kMergeSlices - 1; ++k) { x0 += xch1[k][0][tl]; x1 += xch1[k][1][tl]; }
    const int64_t y = P.labels[t];
    const bool ignored = (y == P.ignore_index);
    const double T = P.temperature;
    double D = 0.0, c0 = 0.0, c1 = 0.0;
    switch (P.div) {
      case DIV_JSD: D = P.beta * x0 + (1.0 - P.beta) * x1; c1 = x1; break;
      case DIV_SKEW_F: D = x0; c1 = x1; break;
      case DIV_SKEW_R: D = x0; c0 = x0; c1 = x1; break;
      case DIV_L2: D = x0; break;
      case DIV_AB: D = -x0 / ((double)P.alpha * (double)P.beta); break;
      default: D = 0.5 * x0; c1 = x1; break;  // TVD
    }
    if (P.div == DIV_L2 || P.div == DIV_AB) {
      // the dlogits formulas of the power route take the gradient's row
      // constant as exp(c_i) - exp(c_2) (L2: i = 1, sum p_s^2 - sum p_t p_s;
      // AB: i = 0, sum q1 - sum q3): the second pass's x1, split by sign
      const float pos = x1 > 0.0 ? (float)log(x1) : -INFINITY;
      const float neg = x1 < 0.0 ? (float)log(-x1) : -INFINITY;
      P.rowp[4 * N + t] = P.div == DIV_AB ? pos : 0.f;
      P.rowp[5 * N + t] = P.div == DIV_L2 ? pos : 0.f;
      P.rowp[6 * N + t] = neg;
    } else {
      P.rowp[4 * N + t] = (float)c0;
      P.rowp[5 * N + t] = (float)c1;
    }
    P.rowv[2 * P.ldv + t] = ignored ? 0.f : (float)(T * T * D);
    return;
  }

  RowState S;
  state_init_fam(S, P.fam);
  if (live)
    for (int vr = slice; vr < P.n_vranges; vr += kMergeSlices) {
      RowState o;
      const float* s = P.partial + (int64_t)vr * kNStat * N + t;
      float* d = reinterpret_cast<float*>(&o);
#pragma unroll
      for (int f = 0; f < kNStat; ++f) d[f] = s[(int64_t)f * N];
      state_merge(S, o, P.fam, P.t_is_one != 0, P.invT);
    }
  if (slice > 0) {
    const float* d = reinterpret_cast<const float*>(&S);
#pragma unroll
    for (int f = 0; f < kNStat; ++f) xch[slice - 1][f][tl] = d[f];
  }
  __syncthreads();
  if (slice > 0 || !live) return;
  for (int k = 0; k < kMergeSlices - 1; ++k) {
    RowState o;
    float* d = reinterpret_cast<float*>(&o);
#pragma unroll
    for (int f = 0; f < kNStat; ++f) d[f] = xch[k][f][tl];
    state_merge(S, o, P.fam, P.t_is_one != 0, P.invT);
  }
  const int64_t y = P.labels[t];
  const bool ignored = (y == P.ignore_index);
  const double T = P.temperature, invT = P.invT;
  const bool t1 = P.t_is_one != 0;
  const double lse_s = (double)S.ms + log((double)S.ss);
  const double lse_sT = t1 ? lse_s : (double)S.ms * invT + log((double)S.sst);
  double lse_t = 0.0, lse_tT = 0.0;
  if (P.has_t) {
    lse_t = (double)S.mt + log((double)S.st);
    lse_tT = t1 ? lse_t : (double)S.mt * invT + log((double)S.stt);
  }
  const double ce_s = ignored ? 0.0 : lse_s - (double)P.label_x[t];
  const double ce_t = (P.teacher_ce && !ignored) ? lse_t - (double)P.label_x[N + t] : 0.0;

  double D = 0.0, c[4] = {0.0, 0.0, 0.0, 0.0};
  if (P.div_on && P.fam != FAM_TWO) {
    const double sst = t1 ? S.ss : S.sst, stt = t1 ? S.st : S.stt;
    if (P.fam == FAM_LIN) {
      const double fkl = (double)S.x[0] / stt - lse_tT + lse_sT;
      const double rkl = (double)S.x[1] / sst - lse_sT + lse_tT;
      switch (P.div) {
        case DIV_FKL: D = fkl; break;
        case DIV_RKL: D = rkl; c[0] = rkl; break;
        case DIV_SYM: D = fkl + rkl; c[0] = rkl; break;
        default: {  // soft-target CE: lse_s^T - sum p_t z_s
          const double pt_zt = (double)S.x[2] / stt + (double)S.mt * invT;
          D = lse_sT - (pt_zt - (double)S.x[0] / stt);
        } break;
      }
    } else {  // FAM_POW: log P_i = LSE(u_i) - a_i lse_t^T - b_i lse_s^T
      double lp[3] = {0.0, 0.0, 0.0};
#pragma unroll
      for (int i = 0; i < 3; ++i)
        if (i < P.npow)
          lp[i] = (double)S.x[2 * i] + log((double)S.x[2 * i + 1]) - (double)P.pa[i] * lse_tT -
                  (double)P.pb[i] * lse_sT;
      const double a = P.alpha, b = P.beta;
      switch (P.div) {
        case DIV_HELL: D = 1.0 - exp(lp[0]); break;
        case DIV_BHAT: D = -lp[0]; break;
        case DIV_RENYI: D = lp[0] / (a - 1.0); break;
        case DIV_AMARI: D = (1.0 - exp(lp[0])) / (a * (1.0 - a)); break;
        case DIV_CHI2: D = exp(lp[0]) - 1.0; break;
        case DIV_L2: D = exp(lp[0]) + exp(lp[1]) - 2.0 * exp(lp[2]); break;
        default:  // AB
          D = -(exp(lp[0]) - a / (a + b) * exp(lp[1]) - b / (a + b) * exp(lp[2])) / (a * b);
          break;
      }
      // row constants: log P_i, ordered as the dlogits formulas expect
      if (P.div == DIV_L2) { c[0] = lp[0]; c[1] = lp[1]; c[2] = lp[2]; }
      else if (P.div == DIV_AB) { c[0] = lp[0]; c[1] = lp[1]; c[2] = lp[2]; }
      else c[0] = lp[0];
    }
  }
  // Normalisers for the dlogits pass.  When it reads logits stored rounded to
  // 16 bits while lse_* come from the fp32 values, a peaked row's largest
  // logit carries a rounding error d (|d| up to 2^-9 |x| in bf16) that scales
  // its probability by e^d, so the row's probabilities stop summing to one
  // (by up to ~6% at |x| ~ 30).  Adding d * p_max to the normaliser restores
  // the sum to first order; what remains is the error of a softmax over the
  // rounded logits.  The losses keep the fp32 normalisers.
  double g_s = lse_s, g_sT = lse_sT, g_t = lse_t, g_tT = lse_tT;
  if (P.round_s && S.ms > -kInf) {
    const double d = (double)round_to(S.ms, P.round_s) - (double)S.ms;
    g_s += d * exp((double)S.ms - lse_s);
    g_sT = t1 ? g_s : g_sT + d * invT * exp((double)S.ms * invT - lse_sT);
  }
  if (P.round_t && P.has_t && S.mt > -kInf) {
    const double d = (double)round_to(S.mt, P.round_t) - (double)S.mt;
    g_t += d * exp((double)S.mt - lse_t);
    g_tT = t1 ? g_t : g_tT + d * invT * exp((double)S.mt * invT - lse_tT);
  }
  if (P.lse_sT_out) P.lse_sT_out[t] = (float)lse_sT;
  P.rowp[0 * N + t] = (float)g_s;
  P.rowp[1 * N + t] = (float)g_sT;
  P.rowp[2 * N + t] = (float)g_t;
  P.rowp[3 * N + t] = (float)g_tT;
  for (int i = 0; i < 4; ++i) P.rowp[(4 + i) * N + t] = (float)c[i];
  P.rowv[0 * P.ldv + t] = (float)ce_s;
  P.rowv[1 * P.ldv + t] = (float)ce_t;
  P.rowv[2 * P.ldv + t] = (P.div_on && !ignored) ? (float)(T * T * D) : 0.f;
}

// Single workgroup: fixed-order fp64 sums of the row losses, the count of
// non-ignored labels, the mean scale and the weighted loss
// (reference ops/tied_teacher.py:499-516).
__global__ __launch_bounds__(1024) void k_finalize(FinalizeParams P) {
  __shared__ double red[4][1024];
  const int tid = threadIdx.x;
  double s0 = 0.0, s1 = 0.0, s2 = 0.0, cnt = 0.0;
  for (int64_t t = tid; t < P.N; t += 1024) {
    s0 += (double)P.rowv[t];
    s1 += (double)P.rowv[P.N + t];
    s2 += (double)P.rowv[2 * P.N + t];
    cnt += (P.labels[t] != P.ignore_index) ? 1.0 : 0.0;
  }
  red[0][tid] = s0; red[1][tid] = s1; red[2][tid] = s2; red[3][tid] = cnt;
  __syncthreads();
  for (int w = 512; w > 0; w >>= 1) {
    if (tid < w) {
      for (int i = 0; i < 4; ++i) red[i][tid] += red[i][tid + w];
    }
    __syncthreads();
  }
  if (tid == 0) {
    const double count = red[3][0];
    const double denom = count < 1.0 ? 1.0 : count;
    double ce_s = red[0][0], ce_t = red[1][0], kl = red[2][0];
    float mean_scale = 1.0f;
    if (!P.reduction_sum) {
      ce_s /= denom; ce_t /= denom; kl /= denom;
      mean_scale = 1.0f / (float)denom;
    }
    if (!P.teacher_ce) ce_t = 0.0;
    if (!P.div_on) kl = 0.0;
    const double loss = (double)P.w_s * ce_s + (double)P.w_t * ce_t + (double)P.w_kl * kl;
    *P.out_loss = (float)loss;
    *P.out_ce_s = (float)ce_s;
    *P.out_ce_t = (float)ce_t;
    *P.out_kl = (float)kl;
    P.scal[0] = mean_scale;
    P.scal[1] = (float)count;
    P.scal[2] = 1.0f;
  }
}

// Count of non-ignored labels and the mean scale, as k_finalize computes them.
__global__ __launch_bounds__(1024) void k_count(const int64_t* labels, int64_t N, int64_t ignore_index,
                                                int reduction_sum, float* scal) {
  __shared__ double red[1024];
  const int tid = threadIdx.x;
  double cnt = 0.0;
  for (int64_t t = tid; t < N; t += 1024) cnt += (labels[t] != ignore_index) ? 1.0 : 0.0;
  red[tid] = cnt;
  __syncthreads();
  for (int w = 512; w > 0; w >>= 1) {
    if (tid < w) red[tid] += red[tid + w];
    __syncthreads();
  }
  if (tid == 0) {
    const double count = red[0];
    const double denom = count < 1.0 ? 1.0 : count;
    scal[0] = reduction_sum ? 1.0f : 1.0f / (float)denom;
    scal[1] = (float)count;
    scal[2] = 1.0f;
  }
}

__global__ void k_mul_scalars(const float* a, const float* b, float* out) { *out = a[0] * b[0]; }

__global__ void k_zero2d(char* out, int64_t ld_bytes, int64_t R, int64_t c0_bytes, int64_t w_bytes) {
  const int64_t total = R * w_bytes;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / w_bytes, c = i % w_bytes;
    out[r * ld_bytes + c0_bytes + c] = 0;
  }
}

hipError_t launch_merge(const MergeParams& P, hipStream_t s) {
  const int grid = (int)((P.N + kMergeTok - 1) / kMergeTok);
  hipLaunchKernelGGL(k_merge, dim3(grid), dim3(kMergeSlices * kMergeTok), 0, s, P);
  return hipGetLastError();
}

hipError_t launch_finalize(const FinalizeParams& P, hipStream_t s) {
  hipLaunchKernelGGL(k_finalize, dim3(1), dim3(1024), 0, s, P);
  return hipGetLastError();
}

hipError_t launch_count(const int64_t* labels, int64_t N, int64_t ignore_index, int reduction_sum, float* scal,
                        hipStream_t s) {
  hipLaunchKernelGGL(k_count, dim3(1), dim3(1024), 0, s, labels, N, ignore_index, reduction_sum, scal);
  return hipGetLastError();
}
hipError_t launch_mul_scalars(const float* a, const float* b, float* out, hipStream_t s) {
  hipLaunchKernelGGL(k_mul_scalars, dim3(1), dim3(1), 0, s, a, b, out);
  return hipGetLastError();
}
hipError_t launch_zero2d(void* out, int64_t ld, int64_t R, int64_t c0, int64_t c1, int esize, hipStream_t s) {
  if (R <= 0 || c1 <= c0) return hipSuccess;
  const int64_t total = R * (c1 - c0) * esize;
  int grid = (int)((total + 255) / 256);
  if (grid > 4096) grid = 4096;
  hipLaunchKernelGGL(k_zero2d, dim3(grid), dim3(256), 0, s, static_cast<char*>(out), ld * esize, R,
                     c0 * esize, (c1 - c0) * esize);
  return hipGetLastError();
}

}  // namespace orda
