// Four-wave ring engine with 16x16x32 MFMAs (bf16 / f16) on gfx950.
//
// The same workgroup (256 threads, 4 waves, output tile 256 x 256, wave tile
// 128 x 128), the same five-slot LDS ring, DMA schedule and tile formats as
// pipeline4; a half step (K = 32) is one 16x16x32 k-step: 8 A and 8 B
// fragments per wave (16 bytes per lane each, the same LDS bytes as the
// 32x32x16 engine) and 8 x 8 MFMAs into 64 four-register accumulators.
// Measured on gfx950 under the socket's power cap, a 16x16x32 stream runs at
// a higher clock than a 32x32x16 one for the same work (fewer accumulator
// register accesses per flop).
//
// Accumulator layout (block acc[mb][nb], element e, lane l): the MFMA
// computes A x B^T (SWAP false) or B x A^T (SWAP true).  Unswapped, e holds A
// row wm * 128 + mb * 16 + 4 (l / 16) + e and B row col16(nb, wn) + l % 16;
// swapped, e holds B row col16(nb, wn) + 4 (l / 16) + e and A row
// wm * 128 + mb * 16 + l % 16 (four consecutive e: four consecutive output
// columns of one row-major C row).
#pragma once
#include "ring4.hpp"

namespace orda {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef f32x4 Acc16[8][8];

__device__ __forceinline__ void zero_acc16(Acc16& acc) {
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[i][j][r] = 0.0f;
}
__device__ __forceinline__ float acc16_get(const f32x4& v, int r) {
  float x;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(v[r]));
  return x;
}
// B row (output column) of block nb: blocks 0..3 in B rows 0..127 (half 0),
// 4..7 in 128..255 (half 1); wave column wn takes 64 rows of each half.
__device__ __forceinline__ int col16(int nb, int wn) { return (nb >> 2) * 128 + wn * 64 + (nb & 3) * 16; }

// One MFMA in place on its accumulator (c += a b^T).  Written as assembly:
// with the builtin, the compiler copies most of the 64 four-register
// accumulators between AGPRs on every half step (~3 register moves per
// MFMA).  Each accumulator is used once per half step, 63 MFMAs after its
// previous use, and the memory clobber keeps the fragment reads and DMAs in
// the program order the half step is written in.
template <class T> struct Mma16;
template <> struct Mma16<bf16> {
  __device__ static __forceinline__ void mma(f32x4& c, const bf16x8& a, const bf16x8& b) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b) : "memory");
  }
};
template <> struct Mma16<f16> {
  __device__ static __forceinline__ void mma(f32x4& c, const f16x8& a, const f16x8& b) {
    asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b) : "memory");
  }
};

// Fragment of half hf (K = 32 from hf * 32) for tile rows row0 + lane % 16:
// lane l holds K elements 8 (l / 16) .. + 7.  K-major: one 16-byte read;
// MN-major: two transposed reads (4 K rows each; waited for and tied by the
// caller).
// MN-major slots: chunk c (8 columns) of K row k at c ^ mn_swz(k).  With
// both operands MN-major (PERM) the swizzle takes k % 8 and a lane's K
// elements are 4 (l / 16) .. + 3 and 16 + 4 (l / 16) .. + 3 (any K order
// serves when both operands use it): the 32 lanes of a transposed read then
// cover 8 consecutive K rows of 16 columns on distinct banks.  Otherwise
// (one operand K-major, whose 16-byte reads give 8 consecutive K) k % 4.
template <bool PERM>
__device__ __forceinline__ int mn_swz(int k) { return PERM ? (k & 7) << 1 : (k & 3) << 2; }

template <class T, int L, bool PERM = false>
__device__ __forceinline__ typename Traits<T>::Frag frag16(const char* tile, int row0, int hf, int lane) {
  if constexpr (L == KMAJ) {
    static_assert(!PERM, "K-major fragments hold 8 consecutive K");
    const int r = row0 + (lane & 15);
    const int c = hf * 4 + (lane >> 4);
    return *reinterpret_cast<const typename Traits<T>::Frag*>(tile + r * 128 + ((c ^ kswz(r)) << 4));
  } else {
    const int g = lane >> 4, s = lane & 15;
    const int k = PERM ? hf * 32 + 4 * g + (s >> 2) : hf * 32 + 8 * g + (s >> 2);
    const int m = row0 + 4 * (s & 3);
    const int c = m >> 3, b = (m & 7) * 2;
    const s16x4 lo = lds_read_tr16(tile + k * 512 + ((c ^ mn_swz<PERM>(k)) << 4) + b);
    const int k4 = PERM ? k + 16 : k + 4;
    const s16x4 hi = lds_read_tr16(tile + k4 * 512 + ((c ^ mn_swz<PERM>(k4)) << 4) + b);
    const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(typename Traits<T>::Frag, both);
  }
}

// pipeline4's contract, with Acc16 accumulators and 16x16x32 MFMAs; the
// epilogue also receives a free 32 KiB ring slot (epilogue(tile, info, acc,
// slot)), which it must leave with a workgroup barrier if it writes it.
template <class T, int LA, int LB, bool H0, bool H1, bool SWAP, class TileInfo, class Opnd, class Epi>
__device__ __forceinline__ void pipeline16(Acc16& acc, char* lds, int ntiles, int64_t K, int64_t lda, int64_t ldb,
                                           const TileInfo& tile_info, const Opnd& opnd, const Epi& epilogue) {
  static_assert(sizeof(T) == 2, "16-bit operands");
  static_assert(LB == KMAJ || (H0 && H1), "an MN-major B has no separate halves");
  using Frag = typename Traits<T>::Frag;
  constexpr bool kTr = LA == MNMAJ || LB == MNMAJ;
  const int w = wave_id(), wm = w >> 1, wn = w & 1;
  const int nk = (int)((K + 63) / 64);
  const int kbytes = (int)(K * (int64_t)sizeof(T));
  if (ntiles <= 0 || nk < 2) return;
  auto mod5 = [](int j) { return j >= kRing ? j - kRing : j; };
  auto slot = [&](int j) { return lds + j * kTileBytes; };
  auto live_b = [](int nb) { return nb < 4 ? H0 : H1; };
  auto live_dma = [](int op, int q) { return op == 0 || LB == MNMAJ || (q < 4 ? H0 : H1); };

  const int lane0 = threadIdx.x & 63;
  const uint32_t krow0 = (uint32_t)(w * 8 + (lane0 >> 3));
  const uint32_t kcb = (uint32_t)(((lane0 & 7) ^ kswz((int)krow0)) * 16);
  constexpr bool kPerm = LA == MNMAJ && LB == MNMAJ;
  const uint32_t mdk = (uint32_t)(2 * w + (lane0 >> 5));
  const int mcol = ((lane0 & 31) ^ mn_swz<kPerm>((int)mdk)) * 8;
  const uint32_t ldbs[2] = {(uint32_t)(lda * (int64_t)sizeof(T)), (uint32_t)(ldb * (int64_t)sizeof(T))};
  struct Step {
    KOp4 o;
    uint32_t ldb, vb, k0;
  };
  auto prep = [&](const KOp4& o, int op, int kd, bool live) {
    Step st;
    st.o = o;
    st.ldb = ldbs[op];
    const bool mn = (op == 0 ? LA : LB) == MNMAJ;
    if (mn) {
      st.k0 = (uint32_t)kd * 64u * st.ldb;
      st.vb = (live && mcol < o.cols) ? mdk * st.ldb + (uint32_t)mcol * (uint32_t)sizeof(T) : kOob;
    } else {
      st.k0 = (uint32_t)kd * 128u;
      const int krem = live ? kbytes - (int)st.k0 : 0;
      st.vb = (int)kcb < krem ? krow0 * st.ldb + kcb : kOob;
    }
    return st;
  };
  auto chunk = [&](const Step& st, int op, int q, char* sb) {
    const bool mn = (op == 0 ? LA : LB) == MNMAJ;
    const int h = mn ? 0 : q >> 2;
    const uint32_t so = (mn ? (uint32_t)q * 8u : (uint32_t)(q & 3) * 32u) * st.ldb + st.k0;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(st.o.r[h], (__attribute__((address_space(3))) void*)(sb + (q * 4 + w) * 1024),
                                             16, st.vb, so, 0, 0);
  };
  // K-major fragment reads (frag16's): lane l reads row l % 16 of a block
  // whose first row is a multiple of 16, so the swizzle kswz(row) depends on
  // l % 16 alone and the lane's byte offset in a block is one value per half
  // (chunk 4 hf + l / 16); the block's offset is then a constant, and a
  // fragment read one add of the slot address and an immediate offset.
  uint32_t koff[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = lane0 & 15;
    koff[h] = (uint32_t)(r * 128 + (((h * 4 + (lane0 >> 4)) ^ kswz(r)) << 4));
  }
  // MN-major fragment reads (frag16's): lane l = 16 g + s reads K rows k and
  // k + dk at columns row0 + 4 (s % 4) .., with k = 32 hf + k0(l).  For row0
  // a multiple of 16 their byte offset in the slot is
  //   32 hf * 512 + k0 * 512 + 8 (s % 4) + ((2 row0) ^ msw),
  // msw = mn_swz(k0) * 16 < 256 (mn_swz sees k % 8, the same for k, k + dk
  // and either half).  A's rows wm * 128 + 16 q give wm * 256 + (32 q ^ msw);
  // B's col16(q, wn) give (2 col16(q, 0)) ^ (msw ^ 128 wn).  So a read is
  // one xor-add of a constant into a per-half base, and the k + dk read an
  // immediate offset of the k read.
  uint32_t mbase = 0, mswa = 0, mswb = 0;
  if constexpr (kTr) {
    const int g = lane0 >> 4, s4 = lane0 & 15;
    const int k0 = (kPerm ? 4 * g : 8 * g) + (s4 >> 2);
    mbase = (uint32_t)(k0 * 512 + 8 * (s4 & 3));
    mswa = (uint32_t)(mn_swz<kPerm>(k0) << 4);
    mswb = mswa ^ (uint32_t)(wn * 128);
  }
  constexpr int kDk = (kPerm ? 16 : 4) * 512;
  auto frag_mn = [&](uint32_t a) __attribute__((always_inline)) {
    const s16x4 lo = lds_read_tr16_at<0>(a);
    const s16x4 hi = lds_read_tr16_at<kDk>(a);
    const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(Frag, both);
  };
  auto lds_addr = [](const char* p) { return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) char*)p; };
  constexpr int kNB = (H0 ? 4 : 0) + (H1 ? 4 : 0);  // live B blocks
  constexpr int kMfmaHalf = 8 * kNB;                // MFMAs per half step

  Frag fa[2][8], fb[2][8];
  auto tie = [&](int buf) {
    if constexpr (kTr) {
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        if constexpr (LA == MNMAJ) lds_tie(fa[buf][x]);
        if constexpr (LB == MNMAJ) {
          if (live_b(x)) lds_tie(fb[buf][x]);
        }
      }
    }
  };
  // One half step: the 8 x kNB / 4 MFMAs of buffer bm, with the fragment
  // reads of the next half step (slots ja, jb, half hf) into buffer br and
  // one operand step's DMA into slot jd between them, in this order per q:
  // A read, MFMA, DMA, MFMA, B read, the rest of q's MFMAs.
  auto half_step = [&](int bm, int br, int ja, int jb, int hf, const Step& st, int op, int jd) {
    char* sb = slot(jd);
    const char* as = slot(ja);
    const char* bs = slot(jb);
    const uint32_t mha = lds_addr(as) + (uint32_t)(hf * 16384 + wm * 256) + mbase;  // MN-major A: half base
    const uint32_t mhb = lds_addr(bs) + (uint32_t)(hf * 16384) + mbase;              // MN-major B
    int n = 0;  // MFMAs issued so far (compile-time after unrolling)
    auto next = [&]() __attribute__((always_inline)) {
      // the n-th live (mb, nb), mb-major
      constexpr int per = kNB;
      const int mb = n / per, x = n % per;
      const int nb = (H0 && H1) ? x : (H0 ? x : x + 4);
      if constexpr (SWAP) Mma16<T>::mma(acc[mb][nb], fb[bm][nb], fa[bm][mb]);
      else Mma16<T>::mma(acc[mb][nb], fa[bm][mb], fb[bm][nb]);
      ++n;
    };
    constexpr int kPerQ = kMfmaHalf / 8;  // MFMAs per group q
    const uint32_t ko = hf ? koff[1] : koff[0];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      int m = 0;  // q's MFMAs issued so far (compile-time)
      auto mm = [&]() __attribute__((always_inline)) {
        if (m < kPerQ) {
          next();
          ++m;
        }
      };
      if constexpr (LA == KMAJ)
        fa[br][q] = *reinterpret_cast<const Frag*>(as + (wm * 128 + q * 16) * 128 + ko);
      else
        fa[br][q] = frag_mn(mha + ((uint32_t)(32 * q) ^ mswa));
      mm();
      if (live_dma(op, q)) chunk(st, op, q, sb);
      mm();
      if (live_b(q)) {
        if constexpr (LB == KMAJ)
          fb[br][q] = *reinterpret_cast<const Frag*>(bs + col16(q, wn) * 128 + ko);
        else
          fb[br][q] = frag_mn(mhb + ((uint32_t)(2 * col16(q, 0)) ^ mswb));
      }
      mm();
#pragma unroll
      for (int i = 0; i < kPerQ; ++i)
        if (i >= m) next();
    }
  };
  auto end_half = [&](int buf_read) {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    tie(buf_read);
  };

  auto cur = tile_info(0);
  auto nxt = tile_info(1);
  {
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int op = 0; op < 2; ++op) {
        const Step st = prep(opnd(cur, op), op, g, true);
        char* sb = slot(2 * g + op);
#pragma unroll
        for (int q = 0; q < 8; ++q)
          if (live_dma(op, q)) chunk(st, op, q, sb);
      }
    constexpr int kStepB = LB == MNMAJ ? 8 : 4 * ((H0 ? 1 : 0) + (H1 ? 1 : 0));  // DMAs of operand B per step
    wait_vmem<8 + kStepB>();
    bar4();
    const int lane = opaque_lane();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      fa[0][q] = frag16<T, LA, kPerm>(slot(0), wm * 128 + q * 16, 0, lane);
      if (live_b(q)) fb[0][q] = frag16<T, LB, kPerm>(slot(1), col16(q, wn), 0, lane);
    }
    end_half(0);
  }

  int j0 = 0;
  for (int tile = 0; tile < ntiles; ++tile) {
    const bool nxt_live = tile + 1 < ntiles;
    for (int kt = 0; kt < nk; ++kt) {
      const bool in_cur = kt + 2 < nk;
      const int kd = in_cur ? kt + 2 : kt + 2 - nk;
      const bool dlive = in_cur || nxt_live;
      const int j1 = mod5(j0 + 1), j2 = mod5(j0 + 2), j3 = mod5(j0 + 3), j4 = mod5(j0 + 4);
      half_step(0, 1, j0, j1, 1, prep(in_cur ? opnd(cur, 0) : opnd(nxt, 0), 0, kd, dlive), 0, j4);
      end_half(1);
      wait_vmem<8>();
      bar4();
      half_step(1, 0, j2, j3, 0, prep(in_cur ? opnd(cur, 1) : opnd(nxt, 1), 1, kd, dlive), 1, j0);
      end_half(0);
      j0 = j2;
    }
    // the last MFMAs' results before the epilogue reads them
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    // (slot mod5(j0 + 4), operand B of the tile's last step, is read by no
    // wave and written by no DMA until the next tile's first step: the
    // epilogue may stage data there)
    epilogue(tile, cur, acc, slot(mod5(j0 + 4)));
    if (nxt_live) {
      zero_acc16(acc);
      cur = nxt;
      nxt = tile_info(tile + 2);
    }
  }
  wait_vmem<0>();
}

}  // namespace orda
