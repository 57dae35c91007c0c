// Four-wave ring engine for 16-bit operands (bf16, f16) on gfx950.
//
// Workgroup: 256 threads = 4 waves, one per SIMD.  Output tile 256 x 256,
// wave tile 128 x 128 = 4 x 4 blocks of 32x32x16 MFMAs whose 256 fp32
// accumulators live in AGPRs (one wave per SIMD may use all 512 registers).
// Compared with eight waves of 128 x 64, each wave reads a third fewer LDS
// bytes per MFMA.
//
// K advances in steps of 64.  A step's two operand tiles (32 KiB each, the
// swizzled layouts of the two-stage engine: K-major 256 rows x 128 B or
// MN-major 64 K rows x 512 B) sit in a ring of five 32 KiB slots: slot j % 5
// holds operand j % 2 of global step j / 2.  A step runs as two halves of
// K = 32:
//   half 0: fragment reads of its own second half, interleaved with the DMA of
//           operand A of step g + 2 (the slot B of step g - 1 used), under the
//           MFMAs of its first half;
//   wait for step g + 1's DMA, barrier;
//   half 1: fragment reads of step g + 1's first half, interleaved with the
//           DMA of operand B of step g + 2 (the slot A of step g used), under
//           the MFMAs of its second half.
// So the loads are spread evenly over the step (eight 16-byte DMAs per thread
// per half), each has one to one and a half steps to land, and every
// fragment read sits between MFMAs.  The reads and DMAs are written in the
// order they should issue (read, DMA, read, ...): the compiler cannot tell the
// LDS slots apart, so it keeps LDS reads and DMA writes in program order, and
// the MFMAs are then placed between them by sched_group_barrier.
//
// The step sequence is flattened over the output tiles a workgroup owns
// (persistent kernels): the next tile's first steps load while the current
// tile finishes, and epilogue(tile, acc) runs after each tile's last step.
#pragma once
#include "orda_core.hpp"

namespace orda {

constexpr int kThreads4 = 256;
constexpr int kRing = 5;
constexpr int kLds4Bytes = kRing * kTileBytes;  // 160 KiB

typedef f32x16 Acc4[4][4];

__device__ __forceinline__ void zero_acc4(Acc4& acc) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
}

// Accumulator element -> VGPR at this point of the program.  Vector ALU
// instructions cannot read AGPRs, so an epilogue needs copies; written as
// volatile assembly (and fenced by the caller per group of four), the copies
// cannot all be hoisted ahead of the first store, which would need 256 VGPRs.
__device__ __forceinline__ float acc_get(const f32x16& v, int r) {
  float x;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(x) : "a"(v[r]));
  return x;
}

// Wave coordinates: rows wm * 128 .. + 127 of A; B row (output column) of
// block nb: blocks 0, 1 in B rows 0..127 (half 0), blocks 2, 3 in 128..255.
__device__ __forceinline__ int w4_m() { return wave_id() >> 1; }
__device__ __forceinline__ int w4_n() { return wave_id() & 1; }
__device__ __forceinline__ int col4(int nb, int wn) { return (nb >> 1) * 128 + wn * 64 + (nb & 1) * 32; }

// One operand tile (256 rows of A or B; K from the tile's first K row/column)
// as buffer resources whose record counts end where the data does, so reads
// past it return zeros.
//  K-major: half h (tile rows h * 128 ..) at r[h], records up to its last
//    valid row; a K step's read of row r, 16 bytes at column byte c, is at
//    r * ldb + c (vector offset) + k0 bytes (scalar offset; the hardware range
//    check covers both, and c + k0 < ldb inside K).
//  MN-major: r[0] at the tile's first column of K row 0, records up to the
//    last valid K row; cols = valid columns (tile rows).
struct KOp4 {
  __amdgpu_buffer_rsrc_t r[2];
  int cols;
};
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_bytes(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc_rows(const void* base, int64_t rows, uint32_t ldb) {
  const int64_t n = rows <= 0 ? 0 : (rows >= 128 ? 128 : rows);
  return rsrc_bytes(base, n * ldb);
}
// K-major: p = the tile's first row (K column 0), rows valid from there, ld
// the row pitch (elements)
template <class T>
__device__ __forceinline__ KOp4 kop4(const T* p, int64_t ld, int64_t rows) {
  KOp4 o;
  const uint32_t ldb = (uint32_t)(ld * (int64_t)sizeof(T));
  o.r[0] = rsrc_rows(p, rows, ldb);
  o.r[1] = rsrc_rows(p + 128 * ld, rows - 128, ldb);
  o.cols = 0;
  return o;
}
// K-major, two halves from separate operands of the same row pitch (a fused
// B: rows 0..127 from p0, rows 128..255 from p1), rows0 / rows1 valid rows.
template <class T>
__device__ __forceinline__ KOp4 kop4_split(const T* p0, int64_t rows0, const T* p1, int64_t rows1, int64_t ld) {
  KOp4 o;
  const uint32_t ldb = (uint32_t)(ld * (int64_t)sizeof(T));
  o.r[0] = rsrc_rows(p0, rows0, ldb);
  o.r[1] = rsrc_rows(p1, rows1, ldb);
  o.cols = 0;
  return o;
}
// MN-major: p = the tile's first column at its first K row, krows valid K
// rows from there (krows * ld * sizeof(T) < 2^31), cols valid columns
template <class T>
__device__ __forceinline__ KOp4 kop4_mn(const T* p, int64_t ld, int64_t krows, int64_t cols) {
  KOp4 o;
  o.r[0] = rsrc_bytes(p, (krows <= 0 ? 0 : krows) * ld * (int64_t)sizeof(T));
  o.r[1] = o.r[0];
  o.cols = (int)(cols <= 0 ? 0 : (cols >= 256 ? 256 : cols));
  return o;
}

// Barrier that no instruction crosses in the scheduler (MFMAs included).
__device__ __forceinline__ void bar4() {
  __builtin_amdgcn_sched_barrier(0);
  tile_barrier();
  __builtin_amdgcn_sched_barrier(0);
}

// Fragment of sub-step ks (0..3) for tile rows row0 + lane % 32: from a
// K-major slot (one 16-byte read) or an MN-major slot (two transposed reads,
// see frag_mn; waited for and tied by the caller).
template <class T, int L>
__device__ __forceinline__ typename Traits<T>::Frag frag4(const char* tile, int row0, int ks, int lane) {
  if constexpr (L == KMAJ) {
    const int r = row0 + (lane & 31);
    const int c = ks * 2 + (lane >> 5);
    return *reinterpret_cast<const typename Traits<T>::Frag*>(tile + r * 128 + ((c ^ kswz(r)) << 4));
  } else {
    const int g = lane >> 4, s = lane & 15;
    const int k = ks * 16 + 8 * (g >> 1) + (s >> 2);
    const int m = row0 + 16 * (g & 1) + 4 * (s & 3);
    const int c = m >> 3, b = (m & 7) * 2;
    const s16x4 lo = lds_read_tr16(tile + k * 512 + ((c ^ ((k & 3) << 2)) << 4) + b);
    const int k4 = k + 4;
    const s16x4 hi = lds_read_tr16(tile + k4 * 512 + ((c ^ ((k4 & 3) << 2)) << 4) + b);
    const s16x8 both = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_bit_cast(typename Traits<T>::Frag, both);
  }
}

// Runs ntiles x nk steps (nk = ceil(K / 64) >= 2).  tile_info(i) -> TI
// describes output tile i (any caller type; called once per tile for the
// tile after the current one, i may equal ntiles); opnd(ti, op) -> KOp4 gives
// operand op (0: A, 1: B) of that tile (selected per step, so it must not
// branch on per-lane values).  K: the K extent (elements; for MN-major
// operands only the step count, their K rows past the data are clipped by the
// record count); lda, ldb: the row pitches (elements).  LA / LB: the operand
// layouts.  epilogue(i, ti, acc) runs after tile i's last step and must not
// touch LDS.  H0 / H1: which halves of B (and which accumulator columns:
// blocks 0, 1 / 2, 3) are live (both for an MN-major B).
//
// Accumulator layout (block acc[mb][nb], element r, lane l): with SWAP false
// the MFMA computes A x B^T, so r holds A row wm * 128 + mb * 32 + acc_row
// (= 8 (r / 4) + 4 (l / 32) + r % 4) and B row col4(nb, wn) + l % 32; with
// SWAP true it computes B x A^T, so r holds B row col4(nb, wn) + acc_row and
// A row wm * 128 + mb * 32 + l % 32 -- four consecutive r are then four
// consecutive output columns of one row-major C row (8-byte stores).
template <class T, int LA, int LB, bool H0, bool H1, bool SWAP, class TileInfo, class Opnd, class Epi>
__device__ __forceinline__ void pipeline4(Acc4& acc, char* lds, int ntiles, int64_t K, int64_t lda, int64_t ldb,
                                          const TileInfo& tile_info, const Opnd& opnd, const Epi& epilogue) {
  static_assert(sizeof(T) == 2, "16-bit operands");
  static_assert(LB == KMAJ || (H0 && H1), "an MN-major B has no separate halves");
  using Tr = Traits<T>;
  using Frag = typename Tr::Frag;
  constexpr bool kTr = LA == MNMAJ || LB == MNMAJ;  // transposed reads: explicit waits
  const int w = wave_id(), wm = w >> 1, wn = w & 1;
  const int nk = (int)((K + 63) / 64);
  const int kbytes = (int)(K * (int64_t)sizeof(T));
  if (ntiles <= 0 || nk < 2) return;
  auto mod5 = [](int j) { return j >= kRing ? j - kRing : j; };  // j < 10
  auto slot = [&](int j) { return lds + j * kTileBytes; };       // j < 5
  auto live_b = [](int nb) { return nb < 2 ? H0 : H1; };
  auto live_dma = [](int op, int q) { return op == 0 || LB == MNMAJ || (q < 4 ? H0 : H1); };

  // Per-thread DMA geometry.  K-major slot: chunk q (0..7) of wave w covers
  // tile row (q % 4) * 32 + w * 8 + lane / 8 of half q / 4, 16 bytes at
  // logical column chunk (lane % 8) ^ swizzle.  MN-major slot: chunk q covers
  // K row 8 q + 2 w + lane / 32, column chunk (lane % 32) ^ swizzle.  Either
  // way the LDS byte is (q * 4 + w) * 1024 + lane * 16 and the swizzle does
  // not depend on q, so the per-thread part of the offset is fixed.
  const int lane0 = threadIdx.x & 63;
  const uint32_t krow0 = (uint32_t)(w * 8 + (lane0 >> 3));                 // K-major: tile row of chunk 0
  const uint32_t kcb = (uint32_t)(((lane0 & 7) ^ kswz((int)krow0)) * 16);  // K-major: column byte
  const uint32_t mdk = (uint32_t)(2 * w + (lane0 >> 5));                   // MN-major: K row of chunk 0
  const int mcol = ((lane0 & 31) ^ (((int)mdk & 3) << 2)) * 8;             // MN-major: column
  const uint32_t ldbs[2] = {(uint32_t)(lda * (int64_t)sizeof(T)), (uint32_t)(ldb * (int64_t)sizeof(T))};
  struct Step {
    KOp4 o;
    uint32_t ldb, vb, k0;
  };
  // one operand step: the thread's vector offset (past every record when its
  // chunk is out of range) and the step's scalar byte offset
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
  // K-major fragment reads (frag4's): lane l reads row l % 32 of a block
  // whose first row is a multiple of 32, so kswz(row) depends on l % 32 alone
  // and the lane's byte offset in a block is one value per sub-step ks
  // (chunk 2 ks + l / 32); a read is then one add of the slot address, with
  // the block's offset an immediate.
  uint32_t koff[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const int r = lane0 & 31;
    koff[ks] = (uint32_t)(r * 128 + (((ks * 2 + (lane0 >> 5)) ^ kswz(r)) << 4));
  }
  constexpr int kNB = (H0 ? 2 : 0) + (H1 ? 2 : 0);  // live B blocks
  constexpr int kMfmaHalf = 2 * 4 * kNB;            // MFMAs per half step

  Frag fa[2][2][4], fb[2][2][4];
  // transposed reads are inline assembly: wait for them and tie the
  // fragments so no use moves above the wait
  auto tie = [&](int buf) {
    if constexpr (kTr) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int x = 0; x < 4; ++x) {
          if constexpr (LA == MNMAJ) lds_tie(fa[buf][h][x]);
          if constexpr (LB == MNMAJ) {
            if (live_b(x)) lds_tie(fb[buf][h][x]);
          }
        }
    }
  };
  // fragment reads of one half step from slots (ja, jb) into buffer buf,
  // interleaved with one operand step's DMA into slot jd (program order per
  // q: A read, DMA, B read)
  auto reads_dma = [&](int buf, int ja, int jb, int hf, const Step& st, int op, int jd) {
    char* sb = slot(jd);
    const char* as = slot(ja);
    const char* bs = slot(jb);
    const int lane = opaque_lane();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int h = q >> 2, x = q & 3, ks = hf * 2 + h;
      if constexpr (LA == KMAJ)
        fa[buf][h][x] = *reinterpret_cast<const Frag*>(as + (wm * 128 + x * 32) * 128 + koff[ks]);
      else
        fa[buf][h][x] = frag4<T, LA>(as, wm * 128 + x * 32, ks, lane);
      if (live_dma(op, q)) chunk(st, op, q, sb);
      if (live_b(x)) {
        if constexpr (LB == KMAJ)
          fb[buf][h][x] = *reinterpret_cast<const Frag*>(bs + col4(x, wn) * 128 + koff[ks]);
        else
          fb[buf][h][x] = frag4<T, LB>(bs, col4(x, wn), ks, lane);
      }
    }
  };
  auto mfma_half = [&](int buf) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int nb = 0; nb < 4; ++nb)
          if (live_b(nb)) {
            if constexpr (SWAP) acc[mb][nb] = Tr::mma(fb[buf][h][nb], fa[buf][h][mb], acc[mb][nb]);
            else acc[mb][nb] = Tr::mma(fa[buf][h][mb], fb[buf][h][nb], acc[mb][nb]);
          }
  };
  // MFMA placement: per q, [A read] M [DMA] M [B read] M.. (transposed reads
  // are assembly, outside the groups: only the MFMAs and DMAs are placed)
  auto schedule = [&](int op) {
    constexpr int kPerQ = kMfmaHalf / 8;  // 4 (both halves of B) or 2
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      if (LA == KMAJ) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (live_dma(op, q)) __builtin_amdgcn_sched_group_barrier(0x010, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if (LB == KMAJ && live_b(q & 3)) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (kPerQ > 2) __builtin_amdgcn_sched_group_barrier(0x008, kPerQ - 2, 0);
    }
  };
  auto end_half = [&](int buf_read) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    tie(buf_read);
    __builtin_amdgcn_sched_barrier(0);
  };

  auto cur = tile_info(0);
  auto nxt = tile_info(1);
  // prologue: steps 0 and 1 (both in tile 0) in flight, step 0 landed, its
  // first half read
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
    constexpr int kStepB = LB == MNMAJ ? 8 : 4 * kNB / 2;  // DMAs of operand B per step
    wait_vmem<8 + kStepB>();                               // step 0 landed
    bar4();
    const int lane = opaque_lane();
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int h = q >> 2, x = q & 3;
      fa[0][h][x] = frag4<T, LA>(slot(0), wm * 128 + x * 32, h, lane);
      if (live_b(x)) fb[0][h][x] = frag4<T, LB>(slot(1), col4(x, wn), h, lane);
    }
    end_half(0);
  }

  int j0 = 0;  // slot of operand A of the current step: (2 g) % 5
  for (int tile = 0; tile < ntiles; ++tile) {
    const bool nxt_live = tile + 1 < ntiles;
    for (int kt = 0; kt < nk; ++kt) {
      // step g + 2: K step kt + 2 of this tile, or of the next one
      const bool in_cur = kt + 2 < nk;
      const int kd = in_cur ? kt + 2 : kt + 2 - nk;
      const bool dlive = in_cur || nxt_live;
      const int j1 = mod5(j0 + 1), j2 = mod5(j0 + 2), j3 = mod5(j0 + 3), j4 = mod5(j0 + 4);
      // half 0: second-half fragments of step g, DMA of A(g + 2) into j4
      reads_dma(1, j0, j1, 1, prep(in_cur ? opnd(cur, 0) : opnd(nxt, 0), 0, kd, dlive), 0, j4);
      mfma_half(0);
      schedule(0);
      end_half(1);
      wait_vmem<8>();  // step g + 1 landed (A of step g + 2 may be in flight)
      bar4();
      // half 1: first-half fragments of step g + 1, DMA of B(g + 2) into j0
      reads_dma(0, j2, j3, 0, prep(in_cur ? opnd(cur, 1) : opnd(nxt, 1), 1, kd, dlive), 1, j0);
      mfma_half(1);
      schedule(1);
      end_half(0);
      j0 = j2;
    }
    // (slot mod5(j0 + 4), operand B of the tile's last step, is read by no
    // wave and written by no DMA until the next tile's first step: the
    // epilogue may stage data there, ending with a workgroup barrier)
    epilogue(tile, cur, acc, slot(mod5(j0 + 4)));
    if (nxt_live) {
      zero_acc4(acc);
      cur = nxt;
      nxt = tile_info(tile + 2);
    }
  }
  wait_vmem<0>();  // the dead steps' DMAs: nothing may land after the waves end
}

}  // namespace orda
