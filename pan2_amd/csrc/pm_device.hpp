// Device-side types and kernels of libpanmuon (gfx950 / CDNA4).
//
// The Muon step of one group of matrices is a fixed sequence of grouped
// launches, each walking every matrix of the group:
//   pm_prologue_kernel   momentum update + bf16 X write + per-tile Σx²
//   pm_norm_kernel       per-matrix 1/‖X‖ and 1/‖X‖²
//   pm_ns_gemm_kernel    x ns_steps x {GRAM, POLY, UPDATE|FINAL}
// The GEMM kernel is one bf16 MFMA (v_mfma_f32_16x16x32_bf16) tile engine
// with four epilogues; its operands are read K-contiguous from LDS, except X
// in C = S·X and C = Xᵀ·S, which is read transposed from LDS.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

constexpr int kTile = 256;       // GEMM macro tile, rows and cols
constexpr int kThreads = 256;    // elementwise/prologue blocks: 4 waves of 64 lanes
constexpr int kGemmThreads = 512;  // GEMM blocks: 8 waves, two per SIMD
constexpr int kProTile = 64;     // prologue tile edge

// DT_F16 is accepted by the Adam step only (torch's fused Adam takes fp16
// params and state); the Muon path takes f32 and bf16.
enum DType : int32_t { DT_F32 = 0, DT_BF16 = 1, DT_F16 = 2 };
// GRAM: S[sc] = X Xᵀ. SYMM: S[sc] = alpha·S[sl]·S[sr]ᵀ + beta·S[sd] (symmetric
// result). UPDATE / FINAL: X' = a·X + S[sl]·X (FINAL fused with the param step).
enum Stage : int32_t { ST_GRAM = 0, ST_SYMM = 1, ST_UPDATE = 2, ST_FINAL = 3 };
// Newton–Schulz organisation of a call (pm_hparams.ns_form).
enum NsForm : int32_t { NS_STANDARD = 0, NS_GRAM = 1 };
constexpr int kSquareBufs = 5;  // Mp x Mp bf16 work matrices per matrix (the gram form uses all five)
enum Mode : int32_t { MODE_STEP = 0, MODE_NS = 1 };

// Per-matrix descriptor, resident in the workspace for the duration of a call.
struct MatDesc {
  // caller tensors, param layout rows x cols
  void* param;        // MODE_STEP: parameter (in/out); MODE_NS: bf16 output
  const void* grad;   // MODE_STEP: gradient; MODE_NS: input
  void* mom;          // MODE_STEP: momentum buffer
  int64_t p_ld, g_ld, m_ld;
  int32_t rows, cols;
  int32_t p_dt, g_dt, m_dt;
  int32_t trans;      // rows > cols: X = uᵀ so the short side is contracted
  int32_t M, N;       // short and long side
  int32_t Mp, Np;     // padded to kTile (padding is zero and stays zero)
  float adj_ratio;    // device-lr path: adjusted_lr = lr * adj_ratio
  float neg_lr_host;  // host-lr path: -(lr * adj_ratio), rounded once
  // workspace buffers
  // X and S are in the panel layout of ws_off for large matrices; a small
  // matrix (Mp = 128) keeps X in the layout of sm_x_off
  uint16_t* X[2];     // bf16 Mp x Np (ld Np), ping-pong
  // bf16 Mp x Mp work matrices. Standard form: S[0] = A = X Xᵀ,
  // S[1] = B = b A + c A². Gram form: S[0] = R, S[1] = Z, S[2] = R Z + a R,
  // S[3], S[4] = Q (ping-pong). Unused entries are null.
  uint16_t* S[kSquareBufs];
  float* partials;    // Σx² of each prologue tile
  float* scales;      // [0] = 1/max(‖X‖,eps)², [1] = 1/max(‖X‖,eps)
  int32_t pro_tiles;
  // K-split chunks per tile (k_split) of GRAM, of the symmetric products and
  // of UPDATE / FINAL; 0 or 1: unsplit
  int32_t ks_gram, ks_symm, ks_full;
  int32_t pad_;
  float* kpart;       // fp32 partial tiles of split stages (chunk-major), or null
};

// Layout of the X buffer a prologue launch writes.
enum XLayout : int32_t {
  XL_ROW = 0,    // row-major
  XL_PANEL = 1,  // the panel layout of ws_off (large matrices)
  XL_SMALL = 2,  // the panel layout of a small matrix's X (sm_x_off)
};

struct ProArgs {
  const MatDesc* descs;
  const int32_t* prefix;  // n+1 prefix sums of pro_tiles
  int32_t n;
  int32_t mode;
  float mu;
  int32_t nesterov;
  int32_t layout;         // of X (XLayout)
  int32_t pad_;
};

struct GemmArgs {
  const MatDesc* descs;
  const int32_t* prefix;  // n+1 prefix sums of this stage's tile counts
  int32_t* queues;        // kXcds tile counters of this launch, zero at launch
  int32_t total;          // tiles of this launch (prefix[n])
  int32_t n;
  int32_t stage;
  int32_t cur;            // which X ping-pong buffer holds the current X
  int32_t first;          // iteration 0: fold the Frobenius normalisation
  int32_t mode;
  int32_t sl, sr, sd, sc;  // square-buffer operands: left, right, addend, output
  float a, b, c;           // UPDATE / FINAL: a; SYMM: alpha = c, beta = b
  const float* lr_dev;    // device lr, or null
  float wd;               // weight decay (device-lr path)
  float wdf_host;         // 1 - lr*wd (host-lr path)
};

// Layouts of the GEMM engine's operands and outputs (a template parameter of
// pm_ns_gemm_kernel): bits set for the matrices kept in the panel layout of
// ws_off, the rest row-major. The grouped Muon / Newton–Schulz path keeps all
// of them in the panel layout; pm_gram and pm_gemm_symmetric take the caller's
// row-major matrices.
constexpr int kTiledX = 1;  // X
constexpr int kTiledS = 2;  // the Mp x Mp work matrices
constexpr int kWsLayout = kTiledX | kTiledS;

// ---------------------------------------------------------------- helpers


__device__ __forceinline__ uint16_t f2bf(float f) {
  __bf16 h = (__bf16)f;  // v_cvt_pk_bf16_f32: round to nearest even, NaN kept
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float bf2f(uint16_t u) {
  return __uint_as_float(((uint32_t)u) << 16);
}
__device__ __forceinline__ float load_elem(const void* p, int32_t dt, int64_t i) {
  return dt == DT_F32 ? ((const float*)p)[i] : bf2f(((const uint16_t*)p)[i]);
}
__device__ __forceinline__ void store_elem(void* p, int32_t dt, int64_t i, float v) {
  if (dt == DT_F32) ((float*)p)[i] = v;
  else ((uint16_t*)p)[i] = f2bf(v);
}

// Locate the matrix owning global work item t: prefix[lo] <= t < prefix[lo+1].
template <class P>
__device__ __forceinline__ int find_matrix(P prefix, int n, int t) {
  int lo = 0, hi = n;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (prefix[mid] <= t) lo = mid; else hi = mid;
  }
  return lo;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

}  // namespace pm
