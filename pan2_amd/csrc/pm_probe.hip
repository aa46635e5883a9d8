// libpanprobe — ceiling probes for the Newton–Schulz GEMM engine (measurement
// only; bench.py --probe ceiling runs them). Each probe is the engine's inner
// loop with parts taken away, on random bf16 data, one block per CU, so that
// its rate bounds what the full engine can reach on this chip at the clock its
// power limit allows:
//   0  MFMA only: 8 waves per CU, each issuing v_mfma_f32_16x16x32_bf16 on
//      register operands in the engine's 8 x 4 accumulator pattern;
//   1  MFMA + the engine's LDS fragment reads (ds_read_b128 from per-lane
//      bases plus immediate offsets, as the engine addresses them) + its two
//      block barriers per 64-deep unit (8 waves of 128 x 64, two per SIMD),
//      without the global -> LDS copies;
//   2  as 1 with 4 waves of 128 x 128 (one per SIMD, a third fewer LDS bytes
//      per FLOP);
//   3  as 1 plus the engine's global -> LDS copies (buffer_load_dwordx4 ...
//      lds, 1 KiB each, issued by waves 0..3 at the engine's positions, with
//      its vmcnt waits before the barriers): 64 KiB per unit per CU, unit u of
//      a block reading bytes (64 KiB * u) mod span of its window; block b reads
//      window b mod nwin of the source (nwin = 8 gives each XCD its own window,
//      shared by its 32 CUs as a tile block shares its panels);
//   4  as 0 with v_mfma_f32_32x32x16_bf16 (probe32_kernel).
// Fragment reads stay inside the first 68 KiB of the 128 KiB LDS array, and
// copies fill it as the engine's two-unit ring (4 x 32 KiB); each block writes
// only its own output slots.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void* lds_ptr_t;

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

// One 1 KiB copy: rows of operand op (0 = A, 1 = B) of unit `unit`, copy q (0..31).
__device__ __forceinline__ void probe_copy(__amdgpu_buffer_rsrc_t rs, char* lds, unsigned span, int unit, int op,
                                           int q, int lane) {
  char* dst = lds + ((unit & 1) * 2 + op) * 32768 + q * 1024;
  const unsigned goff = (((unsigned)unit << 16) & (span - 1u)) + op * 32768u + q * 1024u;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(__attribute__((address_space(3))) char*)dst, 16,
                                           lane * 16, goff, 0, 0);
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

template <int WAVES, int WAVE_COLS, bool LDS_READS, bool COPIES>
__global__ __launch_bounds__(WAVES * 64, 1) void probe_kernel(float* out, int units, const char* src, unsigned span,
                                                              int nwin) {
  constexpr int kLdsWords = 128 * 256;  // 128 KiB: one block per CU
  constexpr int kNi = WAVE_COLS / 16;
  __shared__ __attribute__((aligned(1024))) uint32_t lds[kLdsWords];
  for (int i = threadIdx.x; i < kLdsWords; i += blockDim.x) lds[i] = rnd_pair(i, blockIdx.x);
  __syncthreads();
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const char* base = (const char*)lds;
  // A fragments: 16 positions x 2 KiB apart, below 15*2048 + 7*512 + 1024 < 36 KiB;
  // B fragments: 40 KiB + 4 KiB .. 8 KiB + 15 KiB + 7*256 + 1024 < 68 KiB.
  const char* abase = base + w * 512 + lane * 16;
  const char* bbase = base + 40960 + w * 256 + lane * 16;
  f32x4 acc[8][kNi];
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < kNi; ++j) acc[i][j] = (f32x4){0, 0, 0, 0};
  bf16x8 af[8], bfr[2][kNi];
  for (int j = 0; j < kNi; ++j) {
    bfr[0][j] = *(const bf16x8*)(bbase + j * 1024);
    bfr[1][j] = *(const bf16x8*)(bbase + (j + kNi) * 1024);
  }
  for (int j = 0; j < 8; ++j) af[j] = *(const bf16x8*)(abase + j * 2048);
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(src + (size_t)(blockIdx.x % nwin) * span), (short)0, (int)span, 0x00020000);
  const bool copier = COPIES && w < 4;
  const int q0 = w * 8;
  for (int u = 0; u < units; ++u) {
#pragma unroll
    for (int p = 0; p < 16; ++p) {
      const int s = p / 8, mi = p % 8;
      if (LDS_READS) {
        if (p == 12 || p == 14) {
          // the engine's waits: B(u+1) #7 was followed by 6 copies, A(u+1) #7 by 4
          if (COPIES) {
            if (p == 12) wait_vmcnt<6>(); else wait_vmcnt<4>();
          }
          __builtin_amdgcn_s_waitcnt(0xc07f);
          __builtin_amdgcn_s_barrier();
        }
        af[(p + 2) & 7] = *(const bf16x8*)(abase + p * 2048);
        if (p < kNi) bfr[1][p] = *(const bf16x8*)(bbase + p * 1024 + 8192);
        if (p >= 16 - kNi) bfr[0][p - 16 + kNi] = *(const bf16x8*)(bbase + p * 1024 + 4096);
      }
#pragma unroll
      for (int ni = 0; ni < kNi; ++ni) mfma16(acc[mi][ni], af[p & 7], bfr[s][ni]);
      if (copier) {  // the engine's copy positions: A(u+1) #4..7 at 0, 1; B(u+2) at 12..15; A(u+2) #0..3 at 14, 15
        char* l = (char*)lds;
        if (p < 2) {
          probe_copy(rs, l, span, u + 1, 0, q0 + 4 + 2 * p, lane);
          probe_copy(rs, l, span, u + 1, 0, q0 + 5 + 2 * p, lane);
        }
        if (p >= 12) {
          probe_copy(rs, l, span, u + 2, 1, q0 + 2 * (p - 12), lane);
          probe_copy(rs, l, span, u + 2, 1, q0 + 2 * (p - 12) + 1, lane);
        }
        if (p >= 14) {
          probe_copy(rs, l, span, u + 2, 0, q0 + 2 * (p - 14), lane);
          probe_copy(rs, l, span, u + 2, 0, q0 + 2 * (p - 14) + 1, lane);
        }
      }
      asm volatile("" ::"v"(af[p & 7]), "v"(af[(p + 7) & 7]), "v"(af[(p + 6) & 7]));
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  wait_vmcnt<0>();
  asm volatile("s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7" ::: "memory");
  float sum = 0.0f;
  for (int i = 0; i < 8; ++i)
    for (int j = 0; j < kNi; ++j) sum += acc[i][j][0] + acc[i][j][3];
  out[blockIdx.x * blockDim.x + threadIdx.x] = sum;
}

// Probe 4: as probe 0 with v_mfma_f32_32x32x16_bf16, the 128 x 64 wave tile
// as 4 x 2 blocks of 32 x 32 (the same 128 accumulators per lane, in AGPRs):
// a 64-deep unit is 32 MFMAs of twice probe 0's FLOPs, on half the operand
// register reads per FLOP.
typedef float f32x16 __attribute__((ext_vector_type(16)));
__device__ __forceinline__ void mfma32(f32x16& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__global__ __launch_bounds__(512, 1) void probe32_kernel(float* out, int units) {
  const int lane = threadIdx.x & 63;
  bf16x8 af[4], bfr[2];
  for (int i = 0; i < 4; ++i) {
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    const u32x4v v = {rnd_pair(lane * 16 + 4 * i, blockIdx.x), rnd_pair(lane * 16 + 4 * i + 1, blockIdx.x),
                      rnd_pair(lane * 16 + 4 * i + 2, blockIdx.x), rnd_pair(lane * 16 + 4 * i + 3, blockIdx.x)};
    af[i] = __builtin_bit_cast(bf16x8, v);
    if (i < 2) {
      const u32x4v w = {rnd_pair(lane * 16 + 4 * i + 100, blockIdx.x), rnd_pair(lane * 16 + 4 * i + 101, blockIdx.x),
                        rnd_pair(lane * 16 + 4 * i + 102, blockIdx.x), rnd_pair(lane * 16 + 4 * i + 103, blockIdx.x)};
      bfr[i] = __builtin_bit_cast(bf16x8, w);
    }
  }
  f32x16 acc[4][2];
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 2; ++j)
      for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.0f;
  for (int u = 0; u < units; ++u) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) mfma32(acc[i][j], af[i], bfr[j]);
      asm volatile("" ::"v"(af[0]), "v"(af[1]), "v"(af[2]), "v"(af[3]), "v"(bfr[0]), "v"(bfr[1]));
    }
  }
  asm volatile("s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7" ::: "memory");
  float sum = 0.0f;
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 2; ++j) sum += acc[i][j][0] + acc[i][j][15];
  out[blockIdx.x * blockDim.x + threadIdx.x] = sum;
}

int run32(int blocks, int units, float* out, float* ms, double* flops) {
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return -1;
  auto launch = [&]() { hipLaunchKernelGGL(probe32_kernel, dim3(blocks), dim3(512), 0, 0, out, units); };
  launch();
  float best = 1e30f;
  int rc = 0;
  for (int rep = 0; rep < 3 && rc == 0; ++rep) {
    if (hipEventRecord(a, 0) != hipSuccess) rc = -1;
    launch();
    if (hipEventRecord(b, 0) != hipSuccess || hipEventSynchronize(b) != hipSuccess) rc = -1;
    float t = 0.0f;
    if (rc == 0 && hipEventElapsedTime(&t, a, b) != hipSuccess) rc = -1;
    if (rc == 0 && t < best) best = t;
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  *ms = best;
  *flops = (double)blocks * 8 * units * 32.0 * 32768.0;
  return rc == 0 && hipGetLastError() == hipSuccess ? 0 : -1;
}

template <int WAVES, int WAVE_COLS, bool LDS_READS, bool COPIES>
int run(int blocks, int units, float* out, const char* src, unsigned span, int nwin, float* ms, double* flops) {
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return -1;
  auto launch = [&]() {
    hipLaunchKernelGGL((probe_kernel<WAVES, WAVE_COLS, LDS_READS, COPIES>), dim3(blocks), dim3(WAVES * 64), 0, 0,
                       out, units, src, span, nwin);
  };
  launch();
  float best = 1e30f;
  int rc = 0;
  for (int rep = 0; rep < 3 && rc == 0; ++rep) {
    if (hipEventRecord(a, 0) != hipSuccess) rc = -1;
    launch();
    if (hipEventRecord(b, 0) != hipSuccess || hipEventSynchronize(b) != hipSuccess) rc = -1;
    float t = 0.0f;
    if (rc == 0 && hipEventElapsedTime(&t, a, b) != hipSuccess) rc = -1;
    if (rc == 0 && t < best) best = t;
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  *ms = best;
  *flops = (double)blocks * WAVES * units * 16.0 * (WAVE_COLS / 16) * 16384.0;
  return rc == 0 && hipGetLastError() == hipSuccess ? 0 : -1;
}

}  // namespace

extern "C" {

// Runs probe `which` (0..4, see the top of this file and probe32_kernel) on `blocks` blocks (one
// per CU) for `units` 64-deep units; out must hold blocks * 512 floats. Probe
// 3 reads src: nwin windows of span bytes (span a power of two, at least
// 64 KiB; units below 65536). Writes the best of three timed launches (ms) and
// the MFMA FLOPs per launch.
int pp_ceiling(int which, int blocks, int units, float* out, const void* src, unsigned span, int nwin, float* ms,
               double* flops) {
  if (blocks <= 0 || units <= 0 || units >= 65536 || !out || !ms || !flops) return -1;
  const char* s = (const char*)src;
  if (which == 3 && (!s || span < 65536 || (span & (span - 1)) || nwin < 1)) return -1;
  if (which != 3) {
    // unread by probes 0..2, but the resource must still be well formed
    span = 65536;
    nwin = 1;
    if (!s) s = (const char*)out;
  }
  switch (which) {
    case 0: return run<8, 64, false, false>(blocks, units, out, s, span, nwin, ms, flops);
    case 1: return run<8, 64, true, false>(blocks, units, out, s, span, nwin, ms, flops);
    case 2: return run<4, 128, true, false>(blocks, units, out, s, span, nwin, ms, flops);
    case 3: return run<8, 64, true, true>(blocks, units, out, s, span, nwin, ms, flops);
    case 4: return run32(blocks, units, out, ms, flops);
    default: return -1;
  }
}

}  // extern "C"
