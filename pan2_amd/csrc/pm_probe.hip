// libpanprobe — ceiling probes for the Newton–Schulz GEMM engine (measurement
// only; bench.py --probe ceiling runs them). Each probe is the engine's inner
// loop with parts taken away, on random bf16 data, so that its rate bounds
// what the full engine can reach on this chip at the clock its power limit
// allows:
//   0  MFMA only: 8 waves per CU, each issuing v_mfma_f32_16x16x32_bf16 on
//      register operands in the engine's 8 x 4 accumulator pattern;
//   1  MFMA + LDS fragment reads + two block barriers per 64-deep unit, as the
//      engine's K loop (8 waves of 128 x 64, two per SIMD), without the
//      global -> LDS copies;
//   2  as 1 with 4 waves of 128 x 128 (one per SIMD, a third fewer LDS bytes
//      per FLOP).
// Every LDS index is reduced modulo the array, and each block writes only its
// own output slots.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void mfma16(f32x4& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Random bf16 pairs in [2^-7, 2) with random mantissas.
__device__ __forceinline__ uint32_t rnd_pair(uint32_t i, uint32_t salt) {
  uint32_t x = i * 2654435761u + salt * 40503u;
  x ^= x >> 13;
  x *= 0x5bd1e995u;
  x ^= x >> 15;
  return (x & 0x3fff3fffu) | 0x3c003c00u;
}

template <int WAVES, int WAVE_COLS, bool LDS_READS>
__global__ __launch_bounds__(WAVES * 64, 1) void probe_kernel(float* out, int units) {
  constexpr int kLdsWords = 128 * 256;  // 128 KiB: one block per CU
  constexpr int kNi = WAVE_COLS / 16;
  __shared__ __attribute__((aligned(16))) uint32_t lds[kLdsWords];
  for (int i = threadIdx.x; i < kLdsWords; i += blockDim.x) lds[i] = rnd_pair(i, blockIdx.x);
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const char* base = (const char*)lds;
  constexpr int kSpan = kLdsWords * 4 - 1024;  // every 16-byte read starts below this
  f32x4 acc[8][kNi];
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < kNi; ++j) acc[i][j] = (f32x4){0, 0, 0, 0};
  bf16x8 af[8], bfr[2][kNi];
  for (int j = 0; j < kNi; ++j) {
    bfr[0][j] = *(const bf16x8*)(base + ((w * 8192 + j * 1024 + lane * 16) % kSpan));
    bfr[1][j] = *(const bf16x8*)(base + ((w * 8192 + (j + kNi) * 1024 + lane * 16) % kSpan));
  }
  for (int j = 0; j < 8; ++j) af[j] = *(const bf16x8*)(base + ((w * 2048 + j * 1024 + lane * 16) % kSpan));
  for (int u = 0; u < units; ++u) {
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const int s = p / 8, mi = p % 8;
      if (LDS_READS) {
        if (p == 12 || p == 14) {
          __builtin_amdgcn_s_waitcnt(0xc07f);
          __builtin_amdgcn_s_barrier();
        }
        af[(p + 2) & 7] = *(const bf16x8*)(base + (((u * 16 + p) * 2048 + w * 512 + lane * 16) % kSpan));
        if (p < kNi) bfr[1][p] = *(const bf16x8*)(base + (((u * 16 + p) * 1024 + w * 256 + lane * 16 + 8192) % kSpan));
        if (p >= 16 - kNi)
          bfr[0][p - 16 + kNi] =
              *(const bf16x8*)(base + (((u * 16 + p) * 1024 + w * 256 + lane * 16 + 4096) % kSpan));
      }
#pragma unroll
      for (int ni = 0; ni < kNi; ++ni) mfma16(acc[mi][ni], af[p & 7], bfr[s][ni]);
      asm volatile("" ::"v"(af[p & 7]), "v"(af[(p + 7) & 7]), "v"(af[(p + 6) & 7]));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  asm volatile("s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7" ::: "memory");
  float sum = 0.0f;
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < kNi; ++j) sum += acc[i][j][0] + acc[i][j][3];
  out[blockIdx.x * blockDim.x + threadIdx.x] = sum;
}

template <int WAVES, int WAVE_COLS, bool LDS_READS>
int run(int blocks, int units, float* out, float* ms, double* flops) {
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return -1;
  hipLaunchKernelGGL((probe_kernel<WAVES, WAVE_COLS, LDS_READS>), dim3(blocks), dim3(WAVES * 64), 0, 0, out, units);
  float best = 1e30f;
  for (int rep = 0; rep < 3; ++rep) {
    hipEventRecord(a, 0);
    hipLaunchKernelGGL((probe_kernel<WAVES, WAVE_COLS, LDS_READS>), dim3(blocks), dim3(WAVES * 64), 0, 0, out,
                       units);
    hipEventRecord(b, 0);
    if (hipEventSynchronize(b) != hipSuccess) return -1;
    float t = 0.0f;
    hipEventElapsedTime(&t, a, b);
    if (t < best) best = t;
  }
  hipEventDestroy(a);
  hipEventDestroy(b);
  *ms = best;
  *flops = (double)blocks * WAVES * units * 16.0 * (WAVE_COLS / 16) * 16384.0;
  return hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

extern "C" {

// Runs probe `which` (0, 1 or 2, see the top of this file) on `blocks` blocks
// (one per CU) for `units` 64-deep units; out must hold blocks * 512 floats.
// Writes the best of three timed launches (ms) and the MFMA FLOPs per launch.
int pp_ceiling(int which, int blocks, int units, float* out, float* ms, double* flops) {
  if (blocks <= 0 || units <= 0 || !out || !ms || !flops) return -1;
  switch (which) {
    case 0: return run<8, 64, false>(blocks, units, out, ms, flops);
    case 1: return run<8, 64, true>(blocks, units, out, ms, flops);
    case 2: return run<4, 128, true>(blocks, units, out, ms, flops);
    default: return -1;
  }
}

}  // extern "C"
