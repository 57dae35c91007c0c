// orda_core.hpp -- device building blocks shared by every kernel of
// liborda_ce.so: element traits, the two-stage LDS-staged MFMA main loop
// (CDNA4, gfx950; the four-wave ring engine for 16-bit operands is in
// ring4.hpp), the XCD-aware workgroup order, and the per-row softmax /
// divergence statistics.
//
// Orientation.  Every GEMM here computes C = A * B^T; each operand is either
// K-contiguous (row-major [rows x K], "K-major") or MN-contiguous ([K x rows],
// read through transposed LDS reads).  In the fused loss kernels A is the
// vocabulary weight W [V x H] and B the hidden states [N x H], both K-major,
// so the MFMA output tile is C[v][t]: one lane owns one token column and 16
// vocabulary rows per 32x32 block.  Per-token softmax reductions over the
// vocabulary are therefore in-lane, plus one exchange between lane l and
// lane l^32 and one between the waves that split a tile's 256 vocabulary rows.
//
// Two-stage engine tile: 256 A rows x 256 B rows, 8 waves (2 per SIMD)
// arranged 2 (A) x 4 (B); each wave owns 128 A rows x 64 B rows = 4 x 2 MFMA
// blocks of 32x32.  B rows come in two 128-row halves; a wave's block 0 is in
// half 0 and block 1 in half 1 at the same offset, so for the loss kernels
// (half 0 = student tokens, half 1 = teacher rows of the same tokens) a lane
// holds the student and teacher logits of one token.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace orda {

typedef __bf16 bf16;
typedef _Float16 f16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 512;            // 8 waves of 64, 2 per SIMD

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

// Two floats rounded to a 16-bit type, packed low-first in one dword (one
// v_cvt_pk_bf16_f32 / v_cvt_pk_f16_f32 on gfx950).
template <class T>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  typedef float f2v __attribute__((ext_vector_type(2)));
  typedef T t2v __attribute__((ext_vector_type(2)));
  const f2v v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, t2v));
}
// The low / high 16-bit element of a packed dword, as float.
template <class T>
__device__ __forceinline__ float lo16(uint32_t u) {
  return to_f32(__builtin_bit_cast(T, (unsigned short)(u & 0xffffu)));
}
template <class T>
__device__ __forceinline__ float hi16(uint32_t u) {
  return to_f32(__builtin_bit_cast(T, (unsigned short)(u >> 16)));
}

// Wave coordinates inside the workgroup tile (wave-uniform: scalar registers).
__device__ __forceinline__ int wave_m() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) >> 2; }  // 0..1
__device__ __forceinline__ int wave_n() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) & 3; }   // 0..3

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

// Value of the 32-bit v held by lane (quad_perm ctrl) of this lane's quad.
template <int CTRL>
__device__ __forceinline__ uint32_t quad_dpp(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, CTRL, 0xF, 0xF, false);
}

// 4 x 4 transpose of 16-bit values inside a lane quad, in two exchange
// stages (lanes q ^ 2, then q ^ 1) of one packed dword each: lane q holds row
// q of M as p[0] = (M[q][0], M[q][1]), p[1] = (M[q][2], M[q][3]) (low half
// first); on return out[0] = (M[0][q], M[1][q]), out[1] = (M[2][q], M[3][q]).
// Eight VALU instructions (v_perm_b32 byte selects, DPP moves) in place of
// the ~32 of quad_transpose on unpacked floats.
__device__ __forceinline__ void quad_transpose16(const uint32_t (&p)[2], uint32_t (&out)[2]) {
  const int q = threadIdx.x & 3;
  const bool top = q < 2, odd = (q & 1) != 0;
  // stage 1: top lanes keep columns 0-1 and take rows q + 2's; bottom lanes
  // keep columns 2-3 and take rows q - 2's.  Then A = row (q & 1), B = row
  // (q & 1) + 2, both over columns c0, c0 + 1 with c0 = top ? 0 : 2.
  const uint32_t r1 = quad_dpp<0x4E>(top ? p[1] : p[0]);
  const uint32_t a = top ? p[0] : r1, b = top ? r1 : p[1];
  // stage 2: even lanes collect column c0, odd lanes column c0 + 1; each
  // sends the partner the halves it needs (even: A.hi, B.hi; odd: A.lo, B.lo)
  const uint32_t send = __builtin_amdgcn_perm(b, a, odd ? 0x05040100u : 0x07060302u);
  const uint32_t r = quad_dpp<0xB1>(send);
  out[0] = __builtin_amdgcn_perm(r, a, odd ? 0x03020504u : 0x05040100u);  // even (A.lo, R.lo), odd (R.lo, A.hi)
  out[1] = __builtin_amdgcn_perm(r, b, odd ? 0x03020706u : 0x07060100u);  // even (B.lo, R.hi), odd (R.hi, B.hi)
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

// ------------------------------------------- global -> LDS, direct (DMA)
// Operand tiles reach LDS by buffer_load_dwordx4 ... lds: each lane of a wave
// names any 16-byte source, and the 64 chunks land consecutively at the
// wave's LDS base (lane l at +16 l, checked on gfx950 with an in-bounds
// probe).  No VGPRs hold staged data and no ds_write is issued.  A source
// offset past the buffer resource's range writes zeros (same probe): every
// invalid chunk (rows past the operand, K past its end) is sent there, so
// tiles at the edges come out zero-padded.
//
// LDS tiles are unpadded and XOR-swizzled on 16-byte chunks:
//   K-major tile: 256 rows x 128 bytes of K (64 bf16/f16, 32 fp32); logical
//     chunk c of row r sits at chunk c ^ ((r >> 1) & 7): the 16 rows read by
//     16 consecutive lanes of a fragment read hit 16 distinct 16-byte bank
//     groups (two rows per 256-byte bank line).
//   MN-major tile: BK rows of K x 256 elements (512 bytes bf16, 1 KiB fp32);
//     16-bit: chunk c of K row k sits at c ^ ((k & 3) << 2), so the 4 K rows x
//     64 bytes read by a half-wave's transposing reads cover all 64 banks;
//     fp32: c ^ ((k & 1) << 3) for the 2 K rows of a fragment.
// Pipeline (2 stages of A + B, 2 x 64 KiB): the wait for step kt+1 and the
// workgroup barrier sit before the last MFMA sub-step of step kt; after the
// barrier stage kt is free and receives step kt+2, and the first fragments
// of step kt+1 are read during the last sub-step of step kt.
constexpr int kTileBytes = 32768;         // one operand tile of one stage
constexpr int kLdsTile = kTileBytes;
constexpr int kLdsBytes = 4 * kTileBytes;  // 2 stages x (A + B): 128 KiB

constexpr uint32_t kOob = 0x80000000u;  // a source offset past every resource

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_of(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, 0x7fffffff, 0x00020000);
}
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t off, char* lds_wave) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds_wave, 16, off, 0, 0, 0);
}
template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Workgroup barrier without the memory fences of __syncthreads: the caller's
// vmcnt wait covers the DMA; LDS reads of this wave are complete first.
__device__ __forceinline__ void tile_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
}
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }
// A lane-varying value the compiler cannot hoist out of a loop: epilogues
// inside a persistent tile loop recompute their per-lane addresses from it
// instead of keeping dozens of them live across the whole main loop.
__device__ __forceinline__ int opaque_lane() {
  int l = threadIdx.x & 63;
  asm volatile("" : "+v"(l));
  return l;
}

// f(integral_constant<int, I>) for I = B .. E-1, unrolled by construction: a
// loop body too large for the unroller would otherwise index register arrays
// (accumulator blocks) dynamically and demote them to scratch.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
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

__device__ __forceinline__ int kswz(int r) { return (r >> 1) & 7; }

// K-major operand: rows [0, rows) at p (leading dimension ld), K contiguous;
// contract (host-checked): p and ld 16-byte aligned, K a multiple of 16 bytes.
template <class T>
struct KOperand {
  const T* p;
  int64_t ld, rows;
};

// MN-major operand: element (row r, k) at base[k * ld + r].  Rows of K in up
// to two segments: [0, kseg) at p0 (the first kval0 valid), [kseg, K) at p1
// (the first kval1 valid); columns [0, cols) valid, cols rounded up to a
// 16-byte chunk readable.
template <class T>
struct MnOperand {
  const T* p0;
  const T* p1;
  int64_t ld0, ld1, kseg, kval0, kval1, cols;
};

enum Layout { KMAJ = 0, MNMAJ = 1 };

// Per-thread DMA geometry of one K-major tile of 256 rows: 4 chunks per
// thread, chunk i of wave w covers rows (8 i + w) * 8 .. + 8 (i < 2: rows
// 0..127, i >= 2: rows 128..255).  place() fixes the row offsets of one
// output tile (rows past the operand's end get the out-of-range offset);
// issue() then only adds the K step, so a workgroup that moves from tile to
// tile re-places once per tile, not once per step.
template <class T>
struct KDma {
  int cb[4];        // byte offset of the chunk's K slice (logical chunk x 16)
  uint32_t off[4];  // row offset + cb of the current tile, or kOob
  __device__ __forceinline__ static int row_of(int i) {
    return ((i * 8 + wave_id()) * 64 + (int)(threadIdx.x & 63)) >> 3;
  }
  __device__ __forceinline__ void init() {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pslot = (i * 8 + wave_id()) * 64 + (int)(threadIdx.x & 63);
      cb[i] = ((pslot & 7) ^ kswz(pslot >> 3)) * 16;
    }
  }
  // chunks [I0, I1): operand rows valid from tile row row_base up to `rows`
  // of them, leading dimension ld (elements)
  template <int I0, int I1>
  __device__ __forceinline__ void place(int64_t ld, int64_t rows, int row_base) {
#pragma unroll
    for (int i = I0; i < I1; ++i) {
      const int rr = row_of(i) - row_base;
      off[i] = rr < rows ? (uint32_t)rr * (uint32_t)(ld * (int64_t)sizeof(T)) + (uint32_t)cb[i] : kOob;
    }
  }
  // chunks [I0, I1) of K step k0 to `tile`: p is the operand's row
  // `row_base`, K its K extent (elements)
  template <int I0, int I1>
  __device__ __forceinline__ void issue(const T* p, int64_t k0, int64_t K, char* tile) const {
    const int w = wave_id();
    const auto rs = rsrc_of(p + k0);
    const int64_t krem_bytes = (K - k0) * (int64_t)sizeof(T);
#pragma unroll
    for (int i = I0; i < I1; ++i) dma16(rs, cb[i] < krem_bytes ? off[i] : kOob, tile + (i * 8 + w) * 1024);
  }
};

// Per-thread DMA geometry of one MN-major tile (BK rows of K x 256 columns).
template <class T>
struct MnDma {
  static constexpr int kChunks = 256 * (int)sizeof(T) / 16;   // per K row: 32 (16-bit), 64 (fp32)
  static constexpr int kRowsPerInst = 64 / kChunks;           // 2, 1
  int col[4];  // first column of the chunk
  int dk[4];   // K row of the chunk relative to the wave's instruction row (0 or 1)
  __device__ __forceinline__ void init() {
    const int w = wave_id(), l = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int pslot = (i * 8 + w) * 64 + l;
      const int k = pslot / kChunks;
      const int pc = pslot % kChunks;
      const int c = sizeof(T) == 2 ? (pc ^ ((k & 3) << 2)) : (pc ^ ((k & 1) << 3));
      col[i] = c * (16 / (int)sizeof(T));
      dk[i] = k - (i * 8 + w) * kRowsPerInst;
    }
  }
  // K rows [k0, k0 + BK) of the operand, 256 columns from o's column 0
  __device__ __forceinline__ void issue(const MnOperand<T>& o, int64_t k0, char* tile) const {
    const int w = wave_id();
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // the chunk's K row is the same for the whole wave: pick its segment
      const int64_t krow = k0 + (i * 8 + w) * kRowsPerInst;
      const bool seg0 = krow < o.kseg;
      const T* base = seg0 ? o.p0 + krow * o.ld0 : o.p1 + (krow - o.kseg) * o.ld1;
      const uint32_t ldb = (uint32_t)((seg0 ? o.ld0 : o.ld1) * (int64_t)sizeof(T));  // wave-uniform
      const int64_t kval = seg0 ? o.kval0 - krow : o.kval1 - (krow - o.kseg);  // valid rows from krow
      // dk is 0 or 1: a select, not a multiply
      const uint32_t off = (dk[i] < kval && col[i] < o.cols)
                               ? (dk[i] ? ldb : 0u) + (uint32_t)(col[i] * (int)sizeof(T))
                               : kOob;
      dma16(rsrc_of(base), off, tile + (i * 8 + w) * 1024);
    }
  }
};

// MFMA operand fragment from a K-major tile: lane l supplies row row0 + l%32
// and the K slice of sub-step ks selected by l/32.
template <class T>
__device__ __forceinline__ typename Traits<T>::Frag frag(const char* tile, int row0, int ks) {
  const int lane = threadIdx.x & 63;
  const int r = row0 + (lane & 31);
  if constexpr (sizeof(T) == 2) {
    const int c = ks * 2 + (lane >> 5);
    return *reinterpret_cast<const typename Traits<T>::Frag*>(tile + r * 128 + ((c ^ kswz(r)) << 4));
  } else {
    const int k = ks * 2 + (lane >> 5);
    return *reinterpret_cast<const float*>(tile + r * 128 + (((k >> 2) ^ kswz(r)) << 4) + ((k & 3) << 2));
  }
}

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

// ds_read_b64_tr_b16 as inline assembly: the compiler's wait insertion treats
// the builtin as possibly reading LDS still being written by an in-flight
// DMA and puts s_waitcnt vmcnt(0) before it, which would serialise every K
// step on its own prefetch.  The pipeline orders these reads with its own
// waits: the barrier before a stage is read, and lds_wait_tie before the
// fragments are used.
__device__ __forceinline__ s16x4 lds_read_tr16(const char* p) {
  const uint32_t a = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p;
  s16x4 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(v) : "v"(a));
  return v;
}
// The same at LDS byte address a + OFF (OFF an immediate below 65536).
template <int OFF>
__device__ __forceinline__ s16x4 lds_read_tr16_at(uint32_t a) {
  static_assert(OFF >= 0 && OFF < 65536, "ds offset field");
  s16x4 v;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(v) : "v"(a), "i"(OFF));
  return v;
}

// Wait for every LDS read of this wave, then pass x through an empty asm
// so any later use of x is ordered after the wait.
template <class F>
__device__ __forceinline__ void lds_tie(F& x) {
  asm volatile("" : "+v"(x));
}

// MFMA fragment from an MN-major tile: the same operand as frag<T> (lane l:
// row row0 + l%32, K slice 8*(l/32)..+8 of sub-step ks).
// ds_read_b64_tr_b16 works on groups of 16 lanes: lane s of a group supplies
// the address of 4 consecutive 16-bit elements, and lane i of the group
// receives element i%4 of the rows supplied by lanes i/4, i/4+4, i/4+8,
// i/4+12 (checked on gfx950 with an in-bounds probe).  Lane s therefore
// points at K row k0 + s/4, columns m0 + 4*(s%4): lane i gets column m0 + i
// at K rows k0..k0+3.  Group g covers columns 16*(g%2).. and K rows
// 8*(g/2)..; a second read 4 rows further completes the 8-element slice.
template <class T>
__device__ __forceinline__ typename Traits<T>::Frag frag_mn(const char* tile, int row0, int ks) {
  const int lane = threadIdx.x & 63;
  if constexpr (sizeof(T) == 2) {
    const int g = lane >> 4, s = lane & 15;
    const int k = ks * 16 + 8 * (g >> 1) + (s >> 2);
    const int m = row0 + 16 * (g & 1) + 4 * (s & 3);
    const int c = m >> 3, b = (m & 7) * 2;
    const s16x4 lo = lds_read_tr16(tile + k * 512 + ((c ^ ((k & 3) << 2)) << 4) + b);
    const int k4 = k + 4;
    const s16x4 hi = lds_read_tr16(tile + k4 * 512 + ((c ^ ((k4 & 3) << 2)) << 4) + b);
    const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(typename Traits<T>::Frag, both);
  } else {
    const int k = ks * 2 + (lane >> 5);
    const int m = row0 + (lane & 31);
    const int c = m >> 2;
    return *reinterpret_cast<const float*>(tile + k * 1024 + ((c ^ ((k & 1) << 3)) << 4) + ((m & 3) << 2));
  }
}

template <class T, int L>
__device__ __forceinline__ typename Traits<T>::Frag op_frag(const char* tile, int row0, int ks) {
  if constexpr (L == KMAJ) return frag<T>(tile, row0, ks);
  else return frag_mn<T>(tile, row0, ks);
}

template <int N>
__device__ __forceinline__ void wait_dma_steps(int n) {  // n = later steps allowed in flight (0 or 1)
  if (n <= 0) wait_vmem<0>();
  else wait_vmem<N>();
}

// The pipeline shared by every GEMM-shaped kernel.  Loader issue(step, tile)
// sends the A and B chunks of K step `step` to the given stage; H0 / H1
// select which 128-row halves of the B tile take part (the fused loss
// kernels put student tokens in half 0 and the same tokens' teacher rows in
// half 1).  acc[mb][nb] += A[wm*128 + mb*32 ..] x B[nb*128 + wn*32 ..]^T.
//
// pipeline_tiles runs `ntiles` output tiles of `nk` K steps each as one
// flattened sequence of steps: issue(g, stage) loads global step g (tile
// g / nk, K step g % nk; called once per step, in increasing g), and after the last step of each tile epilogue(i,
// acc) consumes the accumulators, which are then cleared for the next tile
// (the last tile's sums are left in acc).  The first stages of
// tile i+1 are loaded while tile i finishes and runs its epilogue, so a
// persistent workgroup pays the pipeline's start-up latency once.  The
// epilogue must not touch LDS (DPP and global memory only).
template <class T, int LA, int LB, bool H0, bool H1, int DMA_PER_STEP, class Issue, class Epi>
__device__ __forceinline__ void pipeline_tiles(f32x16 (&acc)[4][2], char* lds, int ntiles, int nk,
                                               const Issue& issue, const Epi& epilogue) {
  using Tr = Traits<T>;
  using Frag = typename Tr::Frag;
  constexpr int BK = Tr::kBK;
  constexpr int KS = BK / Tr::kKStep;
  static_assert(KS % 2 == 0, "fragment double buffer parity");
  constexpr bool kMN = (LA == MNMAJ || LB == MNMAJ) && sizeof(T) == 2;
  const int wm = wave_m(), wn = wave_n();
  const int total = ntiles * nk;
  if (total <= 0) return;
  auto stage = [&](int step) { return lds + (step & 1) * (2 * kTileBytes); };

  tile_barrier();  // the previous user of LDS is done
  issue(0, stage(0));
  if (total > 1) issue(1, stage(1));
  wait_dma_steps<DMA_PER_STEP>(total > 1 ? 1 : 0);
  tile_barrier();

  Frag a[2][4], b[2][2];
  {
    const char* as = stage(0);
    const char* bs = as + kTileBytes;
#pragma unroll
    for (int mb = 0; mb < 4; ++mb) a[0][mb] = op_frag<T, LA>(as, wm * 128 + mb * 32, 0);
    if (H0) b[0][0] = op_frag<T, LB>(bs, acc_col0(0, wn), 0);
    if (H1) b[0][1] = op_frag<T, LB>(bs, acc_col0(1, wn), 0);
    if constexpr (kMN) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if constexpr (LA == MNMAJ) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) lds_tie(a[0][mb]);
      }
      if constexpr (LB == MNMAJ) {
        if (H0) lds_tie(b[0][0]);
        if (H1) lds_tie(b[0][1]);
      }
    }
  }
  int kt = 0, tile = 0;
  for (int g = 0; g < total; ++g) {
    const char* as = stage(g);
    const char* bs = as + kTileBytes;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int cur = ks & 1;
      if (ks + 1 < KS) {
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) a[cur ^ 1][mb] = op_frag<T, LA>(as, wm * 128 + mb * 32, ks + 1);
        if (H0) b[cur ^ 1][0] = op_frag<T, LB>(bs, acc_col0(0, wn), ks + 1);
        if (H1) b[cur ^ 1][1] = op_frag<T, LB>(bs, acc_col0(1, wn), ks + 1);
      } else if (g + 1 < total) {
        // stage g is fully read (its last fragments are in registers): wait
        // for step g+1, hand stage g to step g+2, prefetch step g+1 -- unless
        // step g+1 starts a new tile: then its fragments are read after the
        // epilogue, so they are not live across it
        wait_dma_steps<DMA_PER_STEP>(0);
        tile_barrier();
        if (g + 2 < total) issue(g + 2, stage(g));
        if (kt + 1 < nk) {
          const char* an = stage(g + 1);
          const char* bn = an + kTileBytes;
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) a[cur ^ 1][mb] = op_frag<T, LA>(an, wm * 128 + mb * 32, 0);
          if (H0) b[cur ^ 1][0] = op_frag<T, LB>(bn, acc_col0(0, wn), 0);
          if (H1) b[cur ^ 1][1] = op_frag<T, LB>(bn, acc_col0(1, wn), 0);
        }
      }
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) {
        if (H0) acc[mb][0] = Tr::mma(a[cur][mb], b[cur][0], acc[mb][0]);
        if (H1) acc[mb][1] = Tr::mma(a[cur][mb], b[cur][1], acc[mb][1]);
      }
      if constexpr (!kMN) {
        if (ks + 1 < KS) {
          // interleave the next sub-step's fragment reads with this
          // sub-step's MFMAs (MFMA, ds_read, MFMA, ...) instead of issuing
          // every read first: the MFMA pipe keeps work while reads queue
          constexpr int kMfma = 4 * ((H0 ? 1 : 0) + (H1 ? 1 : 0));
          constexpr int kReads = 4 + (H0 ? 1 : 0) + (H1 ? 1 : 0);
          constexpr int kPairs = kMfma < kReads ? kMfma : kReads;
#pragma unroll
          for (int q = 0; q < kPairs; ++q) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // one DS read
          }
          if constexpr (kMfma > kPairs) __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kPairs, 0);
          if constexpr (kReads > kPairs) __builtin_amdgcn_sched_group_barrier(0x100, kReads - kPairs, 0);
        }
      }
      if constexpr (kMN) {
        // the next sub-step's transposed fragments came from inline
        // assembly: wait for them after this sub-step's MFMAs are issued
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        if constexpr (LA == MNMAJ) {
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) lds_tie(a[cur ^ 1][mb]);
        }
        if constexpr (LB == MNMAJ) {
          if (H0) lds_tie(b[cur ^ 1][0]);
          if (H1) lds_tie(b[cur ^ 1][1]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    if (++kt == nk) {
      epilogue(tile, acc);
      if (g + 1 < total) zero_acc(acc);  // the last tile's sums stay for the caller
      kt = 0;
      ++tile;
      {
        // first fragments of the next tile (stage g+1 landed before the
        // barrier; after the last tile this reads stale LDS, unused).  Always
        // read, so the old fragments are provably dead across the epilogue.
        const char* an = stage(g + 1);
        const char* bn = an + kTileBytes;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) a[0][mb] = op_frag<T, LA>(an, wm * 128 + mb * 32, 0);
        if (H0) b[0][0] = op_frag<T, LB>(bn, acc_col0(0, wn), 0);
        if (H1) b[0][1] = op_frag<T, LB>(bn, acc_col0(1, wn), 0);
        if constexpr (kMN) {
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          if constexpr (LA == MNMAJ) {
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) lds_tie(a[0][mb]);
          }
          if constexpr (LB == MNMAJ) {
            if (H0) lds_tie(b[0][0]);
            if (H1) lds_tie(b[0][1]);
          }
        }
      }
    }
  }
}

// One output tile of nk = ceil(K / BK) steps (the accumulators keep the result).
template <class T, int LA, int LB, bool H0, bool H1, int DMA_PER_STEP, class Issue>
__device__ __forceinline__ void pipeline(f32x16 (&acc)[4][2], char* lds, int64_t K, const Issue& issue) {
  const int nk = (int)((K + Traits<T>::kBK - 1) / Traits<T>::kBK);
  pipeline_tiles<T, LA, LB, H0, H1, DMA_PER_STEP>(acc, lds, 1, nk, issue, [](int, f32x16 (&)[4][2]) {});
}

// Fused loss tiles: acc[mb][nb] += A[wm*128 + mb*32 ..] x Bnb[wn*32 ..]^T with
// A [a_rows x K] and two separate K-major B halves of 128 rows each.
template <class T, bool H0, bool H1>
__device__ __forceinline__ void mainloop(f32x16 (&acc)[4][2], char* lds,
                                         const T* A, int64_t lda, int64_t a_rows,
                                         const T* B0, int64_t ldb0, int64_t b0_rows,
                                         const T* B1, int64_t ldb1, int64_t b1_rows,
                                         int64_t K) {
  KDma<T> da, db;
  da.init();
  db.init();
  da.template place<0, 4>(lda, a_rows, 0);
  // B chunks i = 0, 1 hold rows 0..127 (half 0), i = 2, 3 rows 128..255 (half 1)
  if (H0) db.template place<0, 2>(ldb0, b0_rows, 0);
  if (H1) db.template place<2, 4>(ldb1, b1_rows, 128);
  constexpr int kDma = 4 + (H0 ? 2 : 0) + (H1 ? 2 : 0);
  auto issue = [&](int step, char* st) {
    const int64_t k0 = (int64_t)step * Traits<T>::kBK;
    da.template issue<0, 4>(A, k0, K, st);
    if (H0) db.template issue<0, 2>(B0, k0, K, st + kTileBytes);
    if (H1) db.template issue<2, 4>(B1, k0, K, st + kTileBytes);
  };
  pipeline<T, KMAJ, KMAJ, H0, H1, kDma>(acc, lds, K, issue);
}

// Issue one K step of a general-GEMM operand: K-major (KOperand, 256 rows
// from p) or MN-major (MnOperand, 256 columns).
template <class T>
__device__ __forceinline__ void place_operand(KDma<T>& d, const KOperand<T>& o) {
  d.template place<0, 4>(o.ld, o.rows, 0);
}
template <class T>
__device__ __forceinline__ void place_operand(MnDma<T>&, const MnOperand<T>&) {}
template <class T>
__device__ __forceinline__ void issue_operand(const KDma<T>& d, const KOperand<T>& o, int64_t k0, int64_t K,
                                              char* tile) {
  d.template issue<0, 4>(o.p, k0, K, tile);
}
template <class T>
__device__ __forceinline__ void issue_operand(const MnDma<T>& d, const MnOperand<T>& o, int64_t k0, int64_t,
                                              char* tile) {
  d.issue(o, k0, tile);
}

// General GEMM tile: A (256 rows) and B (256 rows) each K-major (KOperand)
// or MN-major (MnOperand, 256 columns).
template <class T, int LA, int LB, class OA, class OB>
__device__ __forceinline__ void mainloop_g(f32x16 (&acc)[4][2], char* lds, const OA& A, const OB& B, int64_t K) {
  using DA = typename std::conditional<LA == KMAJ, KDma<T>, MnDma<T>>::type;
  using DB = typename std::conditional<LB == KMAJ, KDma<T>, MnDma<T>>::type;
  DA da;
  DB db;
  da.init();
  db.init();
  place_operand(da, A);
  place_operand(db, B);
  auto issue = [&](int step, char* st) {
    const int64_t k0 = (int64_t)step * Traits<T>::kBK;
    issue_operand(da, A, k0, K, st);
    issue_operand(db, B, k0, K, st + kTileBytes);
  };
  pipeline<T, LA, LB, true, true, 8>(acc, lds, K, issue);
}

// Store 4 consecutive elements (one 8-byte or 16-byte store when full; p is
// then aligned by construction), else the first n.
template <class T>
__device__ __forceinline__ void store4(T* p, const float (&x)[4], bool full, int n) {
  if (full) {
    if constexpr (sizeof(T) == 2) {
      union { T e[4]; uint2 u; } v;
#pragma unroll
      for (int i = 0; i < 4; ++i) v.e[i] = from_f32<T>(x[i]);
      *reinterpret_cast<uint2*>(p) = v.u;
    } else {
      *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (i < n) p[i] = from_f32<T>(x[i]);
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
