// orda_core.hpp -- device building blocks shared by every kernel of
// liborda_ce.so: element traits, the LDS-staged MFMA main loop (CDNA4,
// gfx950), the XCD-aware workgroup order, and the per-row softmax /
// divergence statistics.
//
// Orientation.  Every GEMM here computes C = A * B^T with both operands
// K-contiguous (row-major [rows x K]).  In the fused loss kernels A is the
// vocabulary weight W [V x H] and B the hidden states [N x H], so the MFMA
// output tile is C[v][t]: one lane owns one token column and 16 vocabulary
// rows per 32x32 block.  Per-token softmax reductions over the vocabulary
// are therefore in-lane, plus one exchange between lane l and lane l^32 and
// one between the two waves that split a tile's 256 vocabulary rows.
//
// Workgroup tile: 256 A rows x 256 B rows, 8 waves (2 per SIMD) arranged
// 2 (A) x 4 (B); each wave owns 128 A rows x 64 B rows = 4 x 2 MFMA blocks
// of 32x32.  B rows come in two 128-row halves; a wave's block 0 is in half 0
// and block 1 in half 1 at the same offset, so for the loss kernels (half 0 =
// student tokens, half 1 = teacher rows of the same tokens) a lane holds the
// student and teacher logits of one token.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace orda {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 512;            // 8 waves of 64, 2 per SIMD
constexpr int kRowBytes = 128;           // bytes of K staged per row per step
constexpr int kLdsRow = kRowBytes + 16;  // padded LDS row: conflict-free b128 reads
constexpr int kLdsTile = 256 * kLdsRow;  // one operand tile
constexpr int kLdsBytes = 4 * kLdsTile;  // double-buffered A and B: 144 KiB

constexpr float kInf = __builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// exp(x) = 2^(x log2 e) on the hardware exp2 (v_exp_f32).
__device__ __forceinline__ float fexp(float x) {
  return __builtin_amdgcn_exp2f(x * kLog2e);
}
// natural log via the hardware log2 (v_log_f32); x > 0.
__device__ __forceinline__ float flog(float x) {
  return __builtin_amdgcn_logf(x) * kLn2;
}
__device__ __forceinline__ float logaddexp(float a, float b) {
  const float m = fmaxf(a, b);
  if (m == -kInf) return -kInf;
  return m + flog(1.0f + fexp(fminf(a, b) - m));
}

// ---------------------------------------------------------------- traits
template <class T> struct Traits;
template <> struct Traits<bf16> {
  using Frag = bf16x8;
  static constexpr int kKStep = 16, kBK = 64;
  __device__ static __forceinline__ f32x16 mma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Traits<f16> {
  using Frag = f16x8;
  static constexpr int kKStep = 16, kBK = 64;
  __device__ static __forceinline__ f32x16 mma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};
template <> struct Traits<float> {
  using Frag = float;
  static constexpr int kKStep = 2, kBK = 32;
  __device__ static __forceinline__ f32x16 mma(Frag a, Frag b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
  }
};

template <class T> __device__ __forceinline__ float to_f32(T x) { return (float)x; }
template <class T> __device__ __forceinline__ T from_f32(float x) { return (T)x; }

// Wave coordinates inside the workgroup tile.
__device__ __forceinline__ int wave_m() { return (threadIdx.x >> 6) >> 2; }  // 0..1
__device__ __forceinline__ int wave_n() { return (threadIdx.x >> 6) & 3; }   // 0..3

// Row (within the wave's 128-row A slice) held by accumulator register r of
// 32x32 block mb for this lane: 8*(r/4) + 4*(lane/32) + r%4 (+ 32*mb).
__device__ __forceinline__ int acc_row(int mb, int r, int lane) {
  return mb * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
}
// First B row of accumulator block nb (0: half 0, 1: half 1) for wave column wn.
__device__ __forceinline__ int acc_col0(int nb, int wn) { return nb * 128 + wn * 32; }

// XCD-aware order.  Workgroup b is dispatched to XCD b % 8; renumber so each
// XCD receives one contiguous run of the logical tile sequence (its L2 then
// sees neighbouring tiles that share operand rows).  Bijective for any count.
__device__ __forceinline__ int xcd_order(int b, int total) {
  const int per = total / 8, extra = total % 8;
  const int x = b % 8, local = b / 8;
  return x * per + min(x, extra) + local;
}

// Grouped 2-D order of a (rows x cols) tile grid: groups of G columns are
// walked column-fastest, so consecutive indices form G x (32 / G) blocks
// and the ~32 workgroups an XCD runs at once share both operands' tiles.
template <int G>
__device__ __forceinline__ void grouped_tile(int t, int rows, int cols, int& row, int& col) {
  const int group = t / (G * rows);
  const int first = group * G;
  const int width = min(cols - first, G);
  const int rem = t % (G * rows);
  col = first + rem % width;
  row = rem / width;
}

// Value of v held by lane (q - j) mod 4 of this lane's quad (DPP quad_perm).
template <int J>
__device__ __forceinline__ float quad_rot(float v) {
  constexpr int ctrl = J == 1 ? 0x93 : J == 2 ? 0x4E : 0x39;  // perm[q] = (q - J) & 3
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), ctrl, 0xF, 0xF, false));
}

// 4 x 4 transpose inside a lane quad: lane q holds x[e] = M[q][e]; on return
// out[k] = M[k][q].
__device__ __forceinline__ void quad_transpose(const float (&x)[4], float (&out)[4]) {
  const int q = threadIdx.x & 3;
#pragma unroll
  for (int k = 0; k < 4; ++k) out[k] = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int si = (q + j) & 3;
    const float send = si == 0 ? x[0] : si == 1 ? x[1] : si == 2 ? x[2] : x[3];
    float recv = send;
    if (j == 1) recv = quad_rot<1>(send);
    if (j == 2) recv = quad_rot<2>(send);
    if (j == 3) recv = quad_rot<3>(send);
    const int di = (q - j) & 3;
#pragma unroll
    for (int k = 0; k < 4; ++k) out[k] = (di == k) ? recv : out[k];
  }
}

// ------------------------------------------------- global -> LDS staging
// A ROWS x 128-byte slab of a row-major [rows x K] operand.  Thread i moves
// 16-byte chunk (i % 8) of rows i/8, i/8 + 64, ...: each row segment is one
// fully used 128-byte line.  Rows >= rows_valid and columns >= K read as 0.
// Contract (checked by the host): the operand base and leading dimension
// are 16-byte aligned and K is a multiple of 16 / sizeof(T), so a chunk is
// either wholly inside or wholly outside [0, K).
template <class T, int ROWS>
struct Stage {
  static constexpr int kRowsPerPass = kThreads / 8;
  static constexpr int kLoads = ROWS / kRowsPerPass;
  static constexpr int kElems = 16 / sizeof(T);
  uint4 v[kLoads];

  __device__ __forceinline__ void load(const T* base, int64_t ld, int64_t rows_valid, int64_t k0, int64_t K) {
    const int tid = threadIdx.x;
    const int64_t kc = k0 + (int64_t)(tid & 7) * kElems;
    const T* p = base + (int64_t)(tid >> 3) * ld + kc;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int r = (tid >> 3) + kRowsPerPass * j;
      v[j] = (r < rows_valid && kc < K)
                 ? *reinterpret_cast<const uint4*>(p + (int64_t)(kRowsPerPass * j) * ld)
                 : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  __device__ __forceinline__ void store(char* lds) const {
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int r = (tid >> 3) + kRowsPerPass * j;
      *reinterpret_cast<uint4*>(lds + r * kLdsRow + (tid & 7) * 16) = v[j];
    }
  }
};

// MFMA operand fragment: lane l supplies row (row0 + l%32) and the K slice
// selected by l/32 of K step ks.
template <class T>
__device__ __forceinline__ typename Traits<T>::Frag frag(const char* tile, int row0, int ks) {
  const int lane = threadIdx.x & 63;
  if constexpr (sizeof(T) == 2) {
    const char* p = tile + (row0 + (lane & 31)) * kLdsRow + ks * 32 + (lane >> 5) * 16;
    return *reinterpret_cast<const typename Traits<T>::Frag*>(p);
  } else {
    const char* p = tile + (row0 + (lane & 31)) * kLdsRow + ks * 8 + (lane >> 5) * 4;
    return *reinterpret_cast<const float*>(p);
  }
}

__device__ __forceinline__ void zero_acc(f32x16 (&acc)[4][2]) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
}

// acc[mb][nb] += A[wm*128 + mb*32 .. +32, :] * Bhalf_nb[wn*32 .. +32, :]^T over K.
// H0/H1 select which 128-row halves of the B tile take part.  A points at the
// tile's first row with a_rows valid rows from there (likewise B0, B1).
// Double-buffered LDS with register prefetch of the next K step (written to
// LDS halfway through the current one) and MFMA fragments read one K
// sub-step ahead; one barrier per K step.
template <class T, bool H0, bool H1>
__device__ __forceinline__ void mainloop(f32x16 (&acc)[4][2], char* lds,
                                         const T* A, int64_t lda, int64_t a_rows,
                                         const T* B0, int64_t ldb0, int64_t b0_rows,
                                         const T* B1, int64_t ldb1, int64_t b1_rows,
                                         int64_t K) {
  using Tr = Traits<T>;
  using Frag = typename Tr::Frag;
  constexpr int BK = Tr::kBK;
  constexpr int KS = BK / Tr::kKStep;
  constexpr int kStoreAt = KS / 2 - 1;
  const int wm = wave_m(), wn = wave_n();
  Stage<T, 256> ga;
  Stage<T, 128> gb0, gb1;
  const int nk = (int)((K + BK - 1) / BK);
  char* const abuf0 = lds;
  char* const bbuf0 = lds + kLdsTile;
  char* const abuf1 = lds + 2 * kLdsTile;
  char* const bbuf1 = lds + 3 * kLdsTile;

  __syncthreads();  // the previous user of LDS is done
  ga.load(A, lda, a_rows, 0, K);
  if (H0) gb0.load(B0, ldb0, b0_rows, 0, K);
  if (H1) gb1.load(B1, ldb1, b1_rows, 0, K);
  ga.store(abuf0);
  if (H0) gb0.store(bbuf0);
  if (H1) gb1.store(bbuf0 + 128 * kLdsRow);
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const bool more = kt + 1 < nk;
    const char* as = (kt & 1) ? abuf1 : abuf0;
    const char* bs = (kt & 1) ? bbuf1 : bbuf0;
    if (more) {
      const int64_t k0 = (int64_t)(kt + 1) * BK;
      ga.load(A, lda, a_rows, k0, K);
      if (H0) gb0.load(B0, ldb0, b0_rows, k0, K);
      if (H1) gb1.load(B1, ldb1, b1_rows, k0, K);
    }
    Frag a[2][4], b[2][2];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) a[0][mb] = frag<T>(as, wm * 128 + mb * 32, 0);
    if (H0) b[0][0] = frag<T>(bs, acc_col0(0, wn), 0);
    if (H1) b[0][1] = frag<T>(bs, acc_col0(1, wn), 0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KS) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) a[cur ^ 1][mb] = frag<T>(as, wm * 128 + mb * 32, ks + 1);
        if (H0) b[cur ^ 1][0] = frag<T>(bs, acc_col0(0, wn), ks + 1);
        if (H1) b[cur ^ 1][1] = frag<T>(bs, acc_col0(1, wn), ks + 1);
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (H0) acc[mb][0] = Tr::mma(a[cur][mb], b[cur][0], acc[mb][0]);
        if (H1) acc[mb][1] = Tr::mma(a[cur][mb], b[cur][1], acc[mb][1]);
      }
      if (ks == kStoreAt && more) {
        char* an = (kt & 1) ? abuf0 : abuf1;
        char* bn = (kt & 1) ? bbuf0 : bbuf1;
        ga.store(an);
        if (H0) gb0.store(bn);
        if (H1) gb1.store(bn + 128 * kLdsRow);
      }
    }
    __syncthreads();
  }
}

// ------------------------------------------------------ row statistics
// Families of per-row state (selected by the divergence).
enum Family { FAM_NONE = 0, FAM_LIN = 1, FAM_POW = 2, FAM_TWO = 3 };

// Divergence codes (same values as enum orda_divergence).
enum Div {
  DIV_FKL = 0, DIV_RKL = 1, DIV_SYM = 2, DIV_SOFT = 3, DIV_HELL = 4, DIV_BHAT = 5,
  DIV_RENYI = 6, DIV_AMARI = 7, DIV_CHI2 = 8, DIV_L2 = 9, DIV_AB = 10, DIV_JSD = 11,
  DIV_SKEW_F = 12, DIV_SKEW_R = 13, DIV_TVD = 14
};

__host__ __device__ inline int div_family(int div) {
  switch (div) {
    case DIV_FKL: case DIV_RKL: case DIV_SYM: case DIV_SOFT: return FAM_LIN;
    case DIV_HELL: case DIV_BHAT: case DIV_RENYI: case DIV_AMARI: case DIV_CHI2:
    case DIV_L2: case DIV_AB: return FAM_POW;
    default: return FAM_TWO;
  }
}

constexpr int kNStat = 12;  // floats of per-row state
constexpr int kNRowP = 8;   // floats of per-row parameters saved for backward

// Online per-row state over a slice of the vocabulary.  With z = x / T:
//   ms, ss : max of x_s and sum exp(x_s - ms)            (CE of the student)
//   mt, st : same for the teacher                         (CE of the teacher)
//   sst,stt: sum exp((x - m) / T)                        (softmax at T)
//   FAM_LIN x0 = sum e_t (z_t - z_s), x1 = sum e_s (z_s - z_t),
//           x2 = sum e_t (z_t - mt / T)     with e = exp((x - m) / T)
//   FAM_POW (x[2i], x[2i+1]) = (max, sum exp(.-max)) of u_i = a_i z_t + b_i z_s
//   FAM_TWO (second pass) x0, x1 = plain sums of normalised-probability terms
struct RowState {
  float ms, ss, mt, st, sst, stt;
  float x[6];
};

__host__ __device__ inline void state_init(RowState& s) {
  s.ms = -__builtin_huge_valf(); s.ss = 0.f;
  s.mt = -__builtin_huge_valf(); s.st = 0.f;
  s.sst = 0.f; s.stt = 0.f;
  for (int i = 0; i < 6; ++i) s.x[i] = 0.f;
}

__device__ __forceinline__ void state_init_fam(RowState& s, int fam) {
  state_init(s);
  if (fam == FAM_POW) { s.x[0] = -kInf; s.x[2] = -kInf; s.x[4] = -kInf; }
}

// Merge b into a (phase 0 state).  t1: temperature is one (sst/stt unused).
__device__ inline void state_merge(RowState& a, const RowState& b, int fam, bool t1, float invT) {
  // student
  if (b.ms != -kInf) {
    if (a.ms == -kInf) {
      a.ms = b.ms; a.ss = b.ss; a.sst = b.sst;
      if (fam == FAM_LIN) a.x[1] = b.x[1];
    } else {
      const float m = fmaxf(a.ms, b.ms);
      const float ca = fexp(a.ms - m), cb = fexp(b.ms - m);
      a.ss = a.ss * ca + b.ss * cb;
      const float caT = t1 ? ca : fexp((a.ms - m) * invT);
      const float cbT = t1 ? cb : fexp((b.ms - m) * invT);
      a.sst = a.sst * caT + b.sst * cbT;
      if (fam == FAM_LIN) a.x[1] = a.x[1] * caT + b.x[1] * cbT;
      a.ms = m;
    }
  }
  // teacher
  if (b.mt != -kInf) {
    if (a.mt == -kInf) {
      a.mt = b.mt; a.st = b.st; a.stt = b.stt;
      if (fam == FAM_LIN) { a.x[0] = b.x[0]; a.x[2] = b.x[2]; }
    } else {
      const float m = fmaxf(a.mt, b.mt);
      const float ca = fexp(a.mt - m), cb = fexp(b.mt - m);
      const float caT = t1 ? ca : fexp((a.mt - m) * invT);
      const float cbT = t1 ? cb : fexp((b.mt - m) * invT);
      if (fam == FAM_LIN) {
        const float sa = t1 ? a.st : a.stt, sb = t1 ? b.st : b.stt;
        const float da = (m - a.mt) * invT, db = (m - b.mt) * invT;
        a.x[0] = a.x[0] * caT + b.x[0] * cbT;
        a.x[2] = caT * (a.x[2] - da * sa) + cbT * (b.x[2] - db * sb);
      }
      a.st = a.st * ca + b.st * cb;
      a.stt = a.stt * caT + b.stt * cbT;
      a.mt = m;
    }
  }
  if (fam == FAM_POW) {
#pragma unroll
    for (int i = 0; i < 3; ++i) {
      const float mb = b.x[2 * i];
      if (mb == -kInf) continue;
      const float ma = a.x[2 * i];
      if (ma == -kInf) { a.x[2 * i] = mb; a.x[2 * i + 1] = b.x[2 * i + 1]; continue; }
      const float m = fmaxf(ma, mb);
      a.x[2 * i + 1] = a.x[2 * i + 1] * fexp(ma - m) + b.x[2 * i + 1] * fexp(mb - m);
      a.x[2 * i] = m;
    }
  }
}

}  // namespace orda
