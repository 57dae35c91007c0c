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
    // (2048 would pass the 2 GB memory ceiling); 4 splits: 38.7 ms/step vs
    // 38.9-39.3 for 8-16 and 42.5-45.3 with 512-token chunks
    {TC_TIED, 0, 128256, 4096, 2, 4, 256, "c2: chunk 512 x 2, split 4"},
    // config 3: separate, Hs = 2048 (teacher 4096), V = 128256.  2048-token
    // chunks: 20.9 ms/step at 1.69 GB peak extra (4096-token chunks: 20.3 at
    // 2.82 GB, past the 2 GB the tied config keeps to); 4 splits (8, 16
    // within noise, more scratch)
    {TC_STAGED, 0, 128256, 2048, 4, 4, 256, "c3: chunk 512 x 4, split 4"},
    // config 4: precomputed logits read in place, H = 4096, V = 128256.
    // 2048-token chunks: 24.0 ms/step vs 25.8-30.2 with 1024; split 2 = 4
    // within noise, 67 MB less split-K scratch
    {TC_INPLACE, 0, 128256, 4096, 4, 2, 256, "c4: chunk 512 x 4, split 2"},
    // config 5: tied, N = 32768, H = 5120, V = 152064 (no memory ceiling
    // beyond reporting it).  2048-token chunks, 8 splits (160 tiles x 8 = 5
    // full rounds of 256): 216.4 ms/step, peak extra 3.52 GB, vs 229.4 with
    // 1024-token chunks and 16 splits (2.88 GB); 4 splits 224.5, 16 218.2
    {TC_TIED, 0, 152064, 5120, 4, 8, 256, "c5: chunk 512 x 4, split 8"},
    // configs 2-5 in fp16 (dlogits unscaled, gradients scaled once at the
    // end).  c2f16: 1024-token chunks, 4 splits: 39.9 ms/step at 1.73 GB
    // (8 splits 40.2, 16 40.5; 512-token chunks 43.7-47.6)
    {TC_TIED, 1, 128256, 4096, 2, 4, 256, "c2f16: chunk 512 x 2, split 4"},
    // c3f16: 2048-token chunks, 4 splits: 21.4 ms/step at 1.69 GB (8 splits
    // 21.5; 4096-token chunks 21.1 at 2.82 GB, past the 2 GB budget)
    {TC_STAGED, 1, 128256, 2048, 4, 4, 256, "c3f16: chunk 512 x 4, split 4"},
    // c4f16: 2048-token chunks, 2 splits: 24.9 ms/step at 1.73 GB (4 splits
    // equal at 1.80 GB, 8 25.2; 1024-token chunks 26.6-31.7)
    {TC_INPLACE, 1, 128256, 4096, 4, 2, 256, "c4f16: chunk 512 x 4, split 2"},
    // c5f16: 2048-token chunks, 8 splits: 220.0 ms/step at 3.52 GB (16
    // splits 221.7; 1024-token chunks 231.9-259.2 at 2.6-2.9 GB)
    {TC_TIED, 1, 152064, 5120, 4, 8, 256, "c5f16: chunk 512 x 4, split 8"},
    // two shapes beyond the benchmark configurations, tied, 8192 tokens.
    // Hidden 8192: the gradients alone take 2.2 GB, so no chunk keeps the
    // 2 GB budget; 2048-token chunks, 2 splits: 72.1 ms/step at 3.49 GB
    // (1024-token chunks 75.0-75.6, 512-token 82.0-92.2)
    {TC_TIED, 0, 128256, 8192, 4, 2, 256, "h8192: chunk 512 x 4, split 2"},
    // Hidden 3584, vocabulary 152064: 1024-token chunks, 9 splits: 42.5
    // ms/step at 1.92 GB (2048-token chunks 40.1-40.5 at 2.5-2.9 GB, past
    // the 2 GB budget; 512-token chunks 45.9-50.3)
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
