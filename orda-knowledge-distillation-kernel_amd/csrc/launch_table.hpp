// launch_table.hpp -- the gfx950 launch table of the gradients-in-forward
// schedule (host side, read by make_plan in abi.hip).
//
// The reference tunes a Triton (BLOCK_SIZE, num_warps) pair per mode and shape
// (src/orda_ce_kernel/utils/_autotune.py:34-46 DEFAULT_CONFIGS, :255-340
// select_config).  Here the tile is fixed per engine (256 x 256 workgroup
// tiles; the ring engine for 16-bit operands, the two-stage engine for fp32)
// and what is chosen per shape is the launch geometry around it:
//
//   chunk_scale  tokens per chunk = chunk_scale x the requested chunk (the
//                reference's chunk_size); a chunk's logits live in HBM, so
//                this trades grad-W K depth (fewer bf16 read-modify-write
//                passes, fewer per-tile epilogues per token) against memory
//   splits_h     split-K count of the grad-hidden GEMM (contraction over V):
//                the 256 persistent workgroups run tiles x splits items, so
//                it sets how full the last round is
//   scan_groups  workgroups of one chunk's scan (one per CU)
//
// Entries are keyed by (teacher class, dtype, vocabulary, student hidden) and
// were chosen by sweeping on an MI355X (the sweep and its timings are in the
// repository's profiles, launch_table_sweep.md); every other shape takes the
// rule of make_plan in abi.hip (rule_chunk_scale for the chunk scale, the
// round-filling split count), which lands within 1% of the swept best on
// every swept shape that the table lists and keeps the 2 GB budget where one
// can be kept.
#pragma once

#include <stdint.h>

namespace orda {

// How a chunk's teacher logits reach the scan.
enum TeacherClass {
  TC_TIED = 0,     // teacher GEMM inside the scan, sharing W's tiles
  TC_STAGED = 1,   // written to the chunk buffer first (separate / frozen
                   // hidden teachers, precomputed logits not read in place)
  TC_INPLACE = 2,  // precomputed logits read in place (compute dtype, V % 8 == 0)
  TC_OTHER = 3     // no teacher, fp32, power terms with a negative student
                   // exponent over a computed teacher's logits (two-stage
                   // scan)
};

struct LaunchEntry {
  int tclass;
  int dtype;  // ORDA_BF16 / ORDA_F16 / ORDA_F32
  int64_t vocab, hidden;
  int chunk_scale;
  int splits_h;
  int scan_groups;
  const char* evidence;  // the sweep row the entry comes from
};

// dtype: 0 = bf16, 1 = f16 (orda_dtype).
constexpr LaunchEntry kLaunchTable[] = {
    // config 2: tied, N = 8192, H = 4096, V = 128256.  1024-token chunks
    // (2048 would pass the 2 GB memory ceiling); 4 splits: 35.9 ms/step vs
    // 36.0-36.5 for 8-16 and 39.5-42.3 with 512-token chunks
    {TC_TIED, 0, 128256, 4096, 2, 4, 256, "c2: chunk 512 x 2, split 4"},
    // config 3: separate, Hs = 2048 (teacher 4096), V = 128256.  2048-token
    // chunks: 19.2 ms/step at 1.69 GB peak extra (4096-token chunks: 18.75 at
    // 2.82 GB, past the 2 GB the tied config keeps to); 4 splits (8: 19.3,
    // 16: 19.5, more scratch)
    {TC_STAGED, 0, 128256, 2048, 4, 4, 256, "c3: chunk 512 x 4, split 4"},
    // config 4: precomputed logits read in place, H = 4096, V = 128256.
    // 2048-token chunks: 21.7 ms/step vs 23.5-27.2 with 1024; split 2 (4:
    // 21.8, 67 MB more split-K scratch)
    {TC_INPLACE, 0, 128256, 4096, 4, 2, 256, "c4: chunk 512 x 4, split 2"},
    // config 5: tied, N = 32768, H = 5120, V = 152064 (no memory ceiling
    // beyond reporting it).  2048-token chunks, 8 splits (160 tiles x 8 = 5
    // full rounds of 256): 202.0 ms/step, peak extra 3.52 GB, vs 213.6 with
    // 1024-token chunks and 16 splits (2.88 GB); 4 splits 209.4, 16 204.0;
    // 4096-token chunks 197.5 at 5.14 GB
    {TC_TIED, 0, 152064, 5120, 4, 8, 256, "c5: chunk 512 x 4, split 8"},
    // configs 2-5 in fp16 (dlogits unscaled, gradients scaled once at the
    // end).  c2f16: 1024-token chunks, 4 splits: 37.8 ms/step at 1.73 GB
    // (8 splits 37.9, 16 38.4; 512-token chunks 41.7-44.3)
    {TC_TIED, 1, 128256, 4096, 2, 4, 256, "c2f16: chunk 512 x 2, split 4"},
    // c3f16: 2048-token chunks, 4 splits: 20.4 ms/step at 1.69 GB (8 splits
    // 20.55; 4096-token chunks 19.7 at 2.82 GB, past the 2 GB budget)
    {TC_STAGED, 1, 128256, 2048, 4, 4, 256, "c3f16: chunk 512 x 4, split 4"},
    // c4f16: 2048-token chunks, 2 splits: 22.9 ms/step at 1.73 GB (4 splits
    // 23.0 at 1.80 GB, 8 23.2; 1024-token chunks 24.6-28.6)
    {TC_INPLACE, 1, 128256, 4096, 4, 2, 256, "c4f16: chunk 512 x 4, split 2"},
    // c5f16: 2048-token chunks, 8 splits: 205.6 ms/step at 3.52 GB (16
    // splits 207.5, 4 212.4; 1024-token chunks 224.1 at 2.7 GB; 4096-token
    // 200.4 at 5.14 GB)
    {TC_TIED, 1, 152064, 5120, 4, 8, 256, "c5f16: chunk 512 x 4, split 8"},
    // two shapes beyond the benchmark configurations, tied, 8192 tokens.
    // Hidden 8192: the gradients alone take 2.2 GB, so no chunk keeps the
    // 2 GB budget; 2048-token chunks, 2 splits: 65.2 ms/step at 3.49 GB
    // (1024-token chunks 67.8-68.4; 4096-token 65.0 at 4.74 GB)
    {TC_TIED, 0, 128256, 8192, 4, 2, 256, "h8192: chunk 512 x 4, split 2"},
    // Hidden 3584, vocabulary 152064: 1024-token chunks, 9 splits: 38.2
    // ms/step at 1.92 GB (2048-token chunks 36.4-37.1 at 2.5-2.9 GB, past
    // the 2 GB budget; 512-token chunks 42.6-45.6)
    {TC_TIED, 0, 152064, 3584, 2, 9, 256, "h3584: chunk 512 x 2, split 9"},
};
constexpr int kLaunchTableSize = (int)(sizeof(kLaunchTable) / sizeof(kLaunchTable[0]));

// Index of the entry for this shape, or -1.
inline int find_launch_entry(int tclass, int dtype, int64_t vocab, int64_t hidden) {
  for (int i = 0; i < kLaunchTableSize; ++i) {
    const LaunchEntry& e = kLaunchTable[i];
    if (e.tclass == tclass && e.dtype == dtype && e.vocab == vocab && e.hidden == hidden) return i;
  }
  return -1;
}

}  // namespace orda
