// mfma_rate -- sustained bf16 MFMA throughput on gfx950 for the two MFMA
// shapes the ring engines can use, under the socket's power limit.
//
//   mfma_rate <shape> <source> <seconds>
//     shape   32: v_mfma_f32_32x32x16_bf16, 16: v_mfma_f32_16x16x32_bf16
//     source  reg: operands held in registers (a 64 x 128 wave tile, eight
//                  A and eight B fragments cycled through the MFMAs);
//             lds: operands read from LDS every K = 32 step with 16-byte
//                  reads (a 128 x 128 wave tile, 16 KB per wave per step,
//                  as the ring engines' main loops read)
//
// One workgroup of 4 waves per CU (one wave per SIMD), random bf16 operands
// (|x| in [0.5, 4)), each launch ~50 ms, repeated for <seconds>; prints the
// TFLOP/s of every tenth launch.  Not part of the library: a measurement of
// the hardware that the engine choice rests on.
#include <hip/hip_runtime.h>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#define CK(x)                                                                          \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      printf("%s failed: %s (line %d)\n", #x, hipGetErrorString(e_), __LINE__);       \
      exit(1);                                                                         \
    }                                                                                  \
  } while (0)

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ unsigned short rand_bf16(unsigned& x) {
  x = x * 1664525u + 1013904223u;
  return (unsigned short)(((x >> 16) & 0x807f) | (((x >> 8) % 3 + 126) << 7));
}

// Accumulators stay in place (the compiler's builtin form copies 16x16x32
// accumulators between registers inside loops); every accumulator is used
// again only after all others, far past the MFMA latency.
__device__ __forceinline__ void mma16(f32x4& c, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
}

template <int SHAPE>
__global__ __launch_bounds__(256, 1) void k_reg(int iters, float* out, unsigned seed0) {
  const int lane = threadIdx.x & 63;
  unsigned x = seed0 ^ (blockIdx.x * 977u) ^ (threadIdx.x * 131u);
  bf16x8 a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    s16x8 u, v;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      u[e] = (short)rand_bf16(x);
      v[e] = (short)rand_bf16(x);
    }
    a[i] = __builtin_bit_cast(bf16x8, u);
    b[i] = __builtin_bit_cast(bf16x8, v);
  }
  float s = 0.f;
  if constexpr (SHAPE == 32) {
    f32x16 acc[2][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = (f32x16){};
    for (int it = 0; it < iters; it += 4) {
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int k = 0; k < 2; ++k)
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i + 2 * k], b[j + 4 * k], acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[i][j][r];
  } else {
    f32x4 acc[4][8];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = (f32x4){};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) mma16(acc[i][j], a[i], b[j]);
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) s += acc[i][j][r];
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
  (void)lane;
}

// LDS: two halves of 2 x 256 rows x 64 bytes (A then B); a step reads the
// half it & 1 (so the reads stay in the loop), chunk c of row r at c ^ (r % 4).
template <int SHAPE>
__global__ __launch_bounds__(256, 1) void k_lds(int iters, float* out, unsigned seed0) {
  __shared__ __attribute__((aligned(16))) unsigned short lds[2 * 2 * 256 * 32];
  unsigned x = seed0 ^ (blockIdx.x * 977u) ^ (threadIdx.x * 131u);
  for (int i = threadIdx.x; i < 2 * 2 * 256 * 32; i += 256) lds[i] = rand_bf16(x);
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, wm = w >> 1, wn = w & 1;
  float s = 0.f;
  if constexpr (SHAPE == 32) {
    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = (f32x16){};
    for (int it = 0; it < iters; ++it) {
      const unsigned short* A = lds + (it & 1) * (2 * 256 * 32);
      const unsigned short* B = A + 256 * 32;
      bf16x8 fa[2][4], fb[2][4];
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int ra = wm * 128 + q * 32 + (lane & 31), rb = wn * 128 + q * 32 + (lane & 31);
          const int c = k * 2 + (lane >> 5);
          fa[k][q] = *reinterpret_cast<const bf16x8*>(A + ra * 32 + ((c ^ (ra & 3)) * 8));
          fb[k][q] = *reinterpret_cast<const bf16x8*>(B + rb * 32 + ((c ^ (rb & 3)) * 8));
        }
#pragma unroll
      for (int k = 0; k < 2; ++k)
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[k][i], fb[k][j], acc[i][j], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[i][j][r];
  } else {
    f32x4 acc[8][8];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[i][j] = (f32x4){};
    for (int it = 0; it < iters; ++it) {
      const unsigned short* A = lds + (it & 1) * (2 * 256 * 32);
      const unsigned short* B = A + 256 * 32;
      bf16x8 fa[8], fb[8];
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int ra = wm * 128 + q * 16 + (lane & 15), rb = wn * 128 + q * 16 + (lane & 15);
        const int c = lane >> 4;
        fa[q] = *reinterpret_cast<const bf16x8*>(A + ra * 32 + ((c ^ (ra & 3)) * 8));
        fb[q] = *reinterpret_cast<const bf16x8*>(B + rb * 32 + ((c ^ (rb & 3)) * 8));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) mma16(acc[i][j], fa[i], fb[j]);
    }
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) s += acc[i][j][r];
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

int main(int argc, char** argv) {
  if (argc < 4 || (atoi(argv[1]) != 32 && atoi(argv[1]) != 16) ||
      (strcmp(argv[2], "reg") != 0 && strcmp(argv[2], "lds") != 0)) {
    printf("usage: mfma_rate <32|16> <reg|lds> <seconds>\n");
    return 2;
  }
  const int shape = atoi(argv[1]);
  const bool lds = strcmp(argv[2], "lds") == 0;
  const double seconds = atof(argv[3]);
  hipDeviceProp_t prop;
  CK(hipGetDeviceProperties(&prop, 0));
  const int grid = prop.multiProcessorCount;
  float* out;
  CK(hipMalloc(&out, (size_t)grid * 256 * sizeof(float)));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  // flops per unit of iters: one K = 32 step of the wave tile, 4 waves per CU
  const double tile = lds ? 128.0 * 128.0 : 64.0 * 128.0;
  const double flop_it = tile * 32.0 * 2.0 * 4.0 * grid;
  auto launch = [&](int n) {
    if (lds) {
      if (shape == 32) hipLaunchKernelGGL(k_lds<32>, dim3(grid), dim3(256), 0, 0, n, out, 12345u);
      else hipLaunchKernelGGL(k_lds<16>, dim3(grid), dim3(256), 0, 0, n, out, 12345u);
    } else {
      if (shape == 32) hipLaunchKernelGGL(k_reg<32>, dim3(grid), dim3(256), 0, 0, n, out, 12345u);
      else hipLaunchKernelGGL(k_reg<16>, dim3(grid), dim3(256), 0, 0, n, out, 12345u);
    }
  };
  int iters = 2000;
  launch(iters);
  CK(hipGetLastError());
  CK(hipDeviceSynchronize());
  float ms = 0.f;
  CK(hipEventRecord(e0, 0));
  launch(iters);
  CK(hipEventRecord(e1, 0));
  CK(hipEventSynchronize(e1));
  CK(hipEventElapsedTime(&ms, e0, e1));
  iters = ((int)(iters * 50.0 / ms) + 3) / 4 * 4;
  const int launches = (int)(seconds * 1000.0 / 50.0);
  for (int rep = 0; rep < launches; ++rep) {
    CK(hipEventRecord(e0, 0));
    launch(iters);
    CK(hipEventRecord(e1, 0));
    CK(hipEventSynchronize(e1));
    CK(hipEventElapsedTime(&ms, e0, e1));
    if (rep % 10 == 0 || rep == launches - 1)
      printf("shape %d operands %s launch %3d: %.2f ms  %.1f TFLOP/s\n", shape, argv[2], rep, ms,
             flop_it * iters / (ms * 1e-3) / 1e12);
  }
  CK(hipFree(out));
  return 0;
}
