// The four-wave ring engine (ring4.hpp) for fp8 operands: OCP e4m3 bytes,
// both operands K-major, v_mfma_scale_f32_32x32x64_f8f6f4 with one
// power-of-two (E8M0) scale per operand row.
//
// The byte geometry is the 16-bit engine's: a K step is 128 bytes of every
// tile row (here 128 K elements), the same five 32 KiB slots, the same DMA
// chunks and swizzle.  A step is two halves of one 64-K sub-step each: a
// lane's fragment of sub-step ks is the 32 bytes at K bytes 64 ks + 32 (lane
// / 32) of its row (two 16-byte LDS reads), which the MFMA takes as that
// lane's K block for row lane % 32 of the 32-row block.  A and B fragments
// come from the same byte positions, so their products pair up element by
// element whatever order the instruction sums a block's K values in.  Per
// half: 4 A + 4 B fragments (16 reads, as the 16-bit engine's 16 fragments)
// and 16 MFMAs of twice the 16-bit instruction's duration (as its 32), with
// eight 16-byte DMAs per thread.
//
// Scales: the MFMA multiplies a lane's K block of A by 2^(sa - 127) and of B
// by 2^(sb - 127) (sa, sb E8M0 bytes in bits 0..7; op_sel 0).  The lane's A
// row is wm * 128 + mb * 32 + lane % 32 of the tile and its B row
// col4(nb, wn) + lane % 32, so the caller passes the row scales per block:
// TI::sa[mb] (per A tile, from tile_info) and sb[nb] (fixed for the call).
// The accumulators then hold the dequantised dot products directly.
#pragma once
#include "ring4.hpp"

namespace orda {

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ i32x8 cat8(const i32x4& lo, const i32x4& hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// 16-byte piece `part` (0, 1) of the fragment of sub-step ks (0, 1) for tile
// row row0 + lane % 32 of a K-major slot.  (One vector load: split into
// scalar loads, as element-wise packing of a struct type makes the compiler
// do, the reads lose the type information that tells them apart from the
// DMA's writes to LDS, and every read after a DMA waits for all of them.)
__device__ __forceinline__ i32x4 frag8(const char* tile, int row0, int ks, int part, int lane) {
  const int r = row0 + (lane & 31);
  const int c = ks * 4 + (lane >> 5) * 2 + part;
  return *reinterpret_cast<const i32x4*>(tile + r * 128 + ((c ^ kswz(r)) << 4));
}

// pipeline4 (ring4.hpp) with byte operands, both K-major, both B halves live,
// SWAP false (acc[mb][nb] element r: A row wm * 128 + mb * 32 + acc_row, B row
// col4(nb, wn) + lane % 32).  K: bytes per row (a multiple of 16); lda, ldb:
// row pitches in bytes.  TI must have `int sa[4]` (the E8M0 byte of A rows
// wm * 128 + mb * 32 + lane % 32 of the tile); sb[nb] the E8M0 byte of B row
// col4(nb, wn) + lane % 32.
template <class TileInfo, class Opnd, class Epi>
__device__ __forceinline__ void pipeline4_f8(Acc4& acc, char* lds, int ntiles, int64_t K, int64_t lda, int64_t ldb,
                                             const TileInfo& tile_info, const Opnd& opnd, const Epi& epilogue,
                                             const int (&sb)[4]) {
  const int w = wave_id(), wm = w >> 1, wn = w & 1;
  const int nk = (int)((K + 127) / 128);
  const int kbytes = (int)K;
  if (ntiles <= 0 || nk < 2) return;
  auto mod5 = [](int j) { return j >= kRing ? j - kRing : j; };  // j < 10
  auto slot = [&](int j) { return lds + j * kTileBytes; };       // j < 5

  // per-thread DMA geometry (K-major slots, as pipeline4)
  const int lane0 = threadIdx.x & 63;
  const uint32_t krow0 = (uint32_t)(w * 8 + (lane0 >> 3));
  const uint32_t kcb = (uint32_t)(((lane0 & 7) ^ kswz((int)krow0)) * 16);
  const uint32_t ldbs[2] = {(uint32_t)lda, (uint32_t)ldb};
  struct Step {
    KOp4 o;
    uint32_t ldb, vb, k0;
  };
  auto prep = [&](const KOp4& o, int op, int kd, bool live) {
    Step st;
    st.o = o;
    st.ldb = ldbs[op];
    st.k0 = (uint32_t)kd * 128u;
    const int krem = live ? kbytes - (int)st.k0 : 0;
    st.vb = (int)kcb < krem ? krow0 * st.ldb + kcb : kOob;
    return st;
  };
  auto chunk = [&](const Step& st, int q, char* sb_) {
    const int h = q >> 2;
    const uint32_t so = (uint32_t)(q & 3) * 32u * st.ldb + st.k0;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(st.o.r[h], (__attribute__((address_space(3))) void*)(sb_ + (q * 4 + w) * 1024),
                                             16, st.vb, so, 0, 0);
  };

  // frag8's lane offsets, one per (ks, part): row l % 32 of a block whose
  // first row is a multiple of 32 (kswz depends on l % 32 alone)
  uint32_t koff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = (threadIdx.x & 63) & 31;
    koff[i] = (uint32_t)(r * 128 + ((((i >> 1) * 4 + ((threadIdx.x & 63) >> 5) * 2 + (i & 1)) ^ kswz(r)) << 4));
  }
  i32x4 fa[2][4][2], fb[2][4][2];
  // fragment reads of sub-step ks from slots (ja, jb) into buffer buf,
  // interleaved with one operand step's DMA into slot jd: per q, A piece,
  // DMA, B piece
  auto reads_dma = [&](int buf, int ja, int jb, int ks, const Step& st, int jd) {
    char* sbuf = slot(jd);
    const char* as = slot(ja);
    const char* bs = slot(jb);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int x = q & 3, part = q >> 2;
      const uint32_t ko = koff[ks * 2 + part];
      fa[buf][x][part] = *reinterpret_cast<const i32x4*>(as + (wm * 128 + x * 32) * 128 + ko);
      chunk(st, q, sbuf);
      fb[buf][x][part] = *reinterpret_cast<const i32x4*>(bs + col4(x, wn) * 128 + ko);
    }
  };
  int sa[4];
  auto mfma_half = [&](int buf) {
    static_for<0, 4>([&](auto MB) {
      constexpr int mb = decltype(MB)::value;
      static_for<0, 4>([&](auto NB) {
        constexpr int nb = decltype(NB)::value;
        acc[mb][nb] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(
            cat8(fa[buf][mb][0], fa[buf][mb][1]), cat8(fb[buf][nb][0], fb[buf][nb][1]), acc[mb][nb], 0, 0, 0,
            sa[mb], 0, sb[nb]);
      });
    });
  };
  // per q: [A read] M [DMA] M [B read]
  auto schedule = [&]() {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
    }
  };
  auto end_half = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
  };

  auto cur = tile_info(0);
  auto nxt = tile_info(1);
#pragma unroll
  for (int mb = 0; mb < 4; ++mb) sa[mb] = cur.sa[mb];
  // prologue: steps 0 and 1 in flight, step 0 landed, its first sub-step read
  {
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
      for (int op = 0; op < 2; ++op) {
        const Step st = prep(opnd(cur, op), op, g, true);
        char* sbuf = slot(2 * g + op);
#pragma unroll
        for (int q = 0; q < 8; ++q) chunk(st, q, sbuf);
      }
    wait_vmem<16>();  // step 0 landed (A and B of step 1 in flight)
    bar4();
    const int lane = opaque_lane();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int x = q & 3, part = q >> 2;
      fa[0][x][part] = frag8(slot(0), wm * 128 + x * 32, 0, part, lane);
      fb[0][x][part] = frag8(slot(1), col4(x, wn), 0, part, lane);
    }
    end_half();
  }

  int j0 = 0;  // slot of operand A of the current step: (2 g) % 5
  for (int tile = 0; tile < ntiles; ++tile) {
    const bool nxt_live = tile + 1 < ntiles;
    for (int kt = 0; kt < nk; ++kt) {
      const bool in_cur = kt + 2 < nk;
      const int kd = in_cur ? kt + 2 : kt + 2 - nk;
      const bool dlive = in_cur || nxt_live;
      const int j1 = mod5(j0 + 1), j2 = mod5(j0 + 2), j3 = mod5(j0 + 3), j4 = mod5(j0 + 4);
      // half 0: sub-step 1 of step g read, DMA of A(g + 2) into j4, MFMAs of
      // sub-step 0
      reads_dma(1, j0, j1, 1, prep(in_cur ? opnd(cur, 0) : opnd(nxt, 0), 0, kd, dlive), j4);
      mfma_half(0);
      schedule();
      end_half();
      wait_vmem<8>();  // step g + 1 landed (A of step g + 2 may be in flight)
      bar4();
      // half 1: sub-step 0 of step g + 1 read, DMA of B(g + 2) into j0, MFMAs
      // of sub-step 1 of step g
      reads_dma(0, j2, j3, 0, prep(in_cur ? opnd(cur, 1) : opnd(nxt, 1), 1, kd, dlive), j0);
      mfma_half(1);
      schedule();
      end_half();
      j0 = j2;
    }
    epilogue(tile, cur, acc);
    if (nxt_live) {
      zero_acc4(acc);
      cur = nxt;
#pragma unroll
      for (int mb = 0; mb < 4; ++mb) sa[mb] = cur.sa[mb];
      nxt = tile_info(tile + 2);
    }
  }
  wait_vmem<0>();  // the dead steps' DMAs: nothing may land after the waves end
}

}  // namespace orda
