// Small-M path of libpanmuon: matrices whose short side M is at most 128
// (PAN 2's chunked QKV row blocks, [B, 128, N], pan/optim/patch_muon.py:75-142,
// and any other narrow weight). They are padded to Mp = 128 rather than to the
// 256 of the grouped GEMM engine, and a Newton–Schulz pass is two launches:
//
//   pm_small_core_kernel   one block per matrix: R = X Xᵀ (128 x 128, X
//                          streamed through LDS), then the M x M part of the
//                          iteration entirely in LDS, written out as one
//                          128 x 128 matrix S:
//                            standard form: S = B = c R² + b R
//                            gram form: the core steps of one segment of
//                            _gram_newtonschulz_local (pan/optim/patch_muon.py:
//                            320-331): Z = c R² + b R; Q = a I + Z, then
//                            Q Z + a Q; R <- Z (R Z + a R) + a (R Z + a R); S = Q
//   pm_small_apply_kernel  X' = s·(a·X + S X) over 128 x 512 tiles with the
//                          arithmetic of the grouped engine's UPDATE / FINAL
//                          (X', or the fused parameter step). Small matrices
//                          keep X only, no Xᵀ: the apply reads X transposed
//                          from LDS.
//
// This is the counterpart of the reference's fused batched gram-NS
// (pan/optim/muon_triton.py:234-345: the gram and the 128 x 128 iteration in
// one program per matrix, the two Q X applications as batched GEMMs). Every
// product is the grouped engine's, element for element: the same MFMA
// instruction over the same k order (the engine's extra k >= 128 terms of a
// 256-padded matrix are zeros), rounded to bf16 at the same points, with the
// upper triangle stored and mirrored. A small matrix therefore gets the
// result the engine would give it padded to 256.
#pragma once

namespace pm {

constexpr int kSm = 128;              // padded short side of a small matrix
constexpr int kSmRow = kSm * 2;       // 256 B: a row of a 128 x 128 bf16 matrix, or 128 k values
constexpr int kSmMat = kSm * kSmRow;  // 32 KiB: one 128 x 128 bf16 matrix
constexpr int kSmUnit = kSm * 128;    // 16 KiB: 128 rows x 64 k values, one gram unit
constexpr int kSmRing = 8;            // gram units in LDS: 7 in flight while one is read (gram form)
constexpr int kSmRingStd = 4;         // standard form: 64 KiB of ring, two blocks per CU
constexpr int kSmApplyWaves = 8;                     // apply blocks: waves of 128 x 64
constexpr int kSmApplyThreads = 64 * kSmApplyWaves;
constexpr int kSmApplyCols = 64 * kSmApplyWaves;     // columns of X per apply tile: one 1 KiB row
static_assert(kSmApplyCols * 2 == 1024, "an apply tile row is one 1 KiB copy");

struct SmallCoreArgs {
  const MatDesc* descs;
  const float* coeffs;  // (a, b, c) of every Newton–Schulz iteration, on the device
  int32_t it0;          // first iteration of this launch
  int32_t steps;        // gram form: core steps of the segment; 0: standard form, S = c R² + b R
  int32_t cur;          // X slot holding the current X
  int32_t first;        // scale R by 1/‖X‖² (the Frobenius normalisation, folded)
  int32_t so;           // square buffer receiving S
  int32_t pad_;
};

// A buffer resource over [base, base + bytes). Descriptor fields reach
// registers through vector loads (the compiler cannot prove the table
// unclobbered), and a resource built from them would stay in VGPRs, turning
// every buffer load into a waterfall loop; the values are uniform, so
// readfirstlane moves them to SGPRs.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t uniform_rsrc(const uint16_t* base, uint32_t bytes) {
  const uint64_t v = (uint64_t)base;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return panel_rsrc((const uint16_t*)(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(bytes));
}

// A 128 x 128 bf16 matrix in LDS, rows 0..63 in h[0] and 64..127 in h[1]
// (two 16 KiB gram-ring slots). Row r is 256 B and chunk c (16 B, columns
// 8c .. 8c+7) of row r is stored at chunk c ^ (r & 15), so the 16 rows of an
// MFMA operand read of one chunk hit 16 different bank groups. Every access
// below names its half from wave-uniform values.
struct SmMat {
  char* h[2];
};
// chunk c16 of row (64·half + rr)
__device__ __forceinline__ char* sm_at(const SmMat& m, int half, int rr, int c16) {
  return m.h[half] + rr * kSmRow + ((c16 ^ (rr & 15)) << 4);
}
// element (64·half + rr, q)
__device__ __forceinline__ uint16_t* sm_el(const SmMat& m, int half, int rr, int q) {
  return (uint16_t*)(sm_at(m, half, rr, q >> 3) + (q & 7) * 2);
}

__device__ __forceinline__ f32x4 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Stores elements e of v with p0 + e < q: the strict lower part of row q,
// columns p0 .. p0+3 (v[e] is the element at column p0 + e).
__device__ __forceinline__ void store_lower4(uint16_t* dst, u16x4 v, int p0, int q) {
  if (p0 + 3 < q) {
    *(u16x4*)dst = v;
    return;
  }
  if (p0 >= q) return;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (p0 + e < q) dst[e] = v[e];
}

// Finishes a 128 x 128 product of 8 waves, wave w owning rows r0 .. r0+63
// (r0 = 64·(w/4)) and columns c0 .. c0+31 (c0 = 32·(w%4)); acc[i][j] holds
// rows r0 + 16i + 4(lane/16) + 0..3 of column c0 + 16j + lane%16.
// C = alpha·acc + beta·D, rounded to bf16; elements on and above the diagonal
// are stored at (p, q) and (q, p), so C is exactly symmetric. D must be
// symmetric (it is read through its transpose). C may be an operand of the
// product: every wave has read its operands before the first store.
__device__ __forceinline__ void sm_finish(const f32x4 (&acc)[4][2], const SmMat& D, const SmMat& C, float alpha,
                                          float beta, int r0, int c0, int lane) {
#pragma clang fp contract(off)
  const int g = lane >> 4;
  const int rh = r0 >> 6, ch = c0 >> 6, cr = c0 & 63;  // halves and row-in-half base of the wave
  u16x4 o[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int p0 = r0 + 16 * i + 4 * g;
      u16x4 dv = (u16x4){0, 0, 0, 0};
      if (beta != 0.0f) dv = *(const u16x4*)sm_el(D, ch, cr + 16 * j + (lane & 15), p0);  // D[p0..p0+3][q]
#pragma unroll
      for (int r = 0; r < 4; ++r) o[i][j][r] = f2bf(alpha * acc[i][j][r] + beta * bf2f(dv[r]));
    }
  __syncthreads();  // every wave has read its operands and D
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int p0 = r0 + 16 * i + 4 * g, q = c0 + 16 * j + (lane & 15);
      // row p0 + lane%4, columns q&~3 .. +3 (quad_transpose), on and above the diagonal
      const u16x4 t = quad_transpose(o[i][j], lane);
      store_upper4(sm_el(C, rh, 16 * i + 4 * g + (lane & 3), q & ~3), t, q & ~3, p0 + (lane & 3));
      // the mirror: row q, columns p0 .. p0+3, strictly below the diagonal
      store_lower4(sm_el(C, ch, cr + 16 * j + (lane & 15), p0), o[i][j], p0, q);
    }
  __syncthreads();
}

// Waves 4 and 5 own rows 64..127 of columns 0..63: every element of their
// tiles lies below the diagonal, which sm_finish neither stores nor mirrors, so
// they skip the products (fragment reads and MFMAs) and only keep the block's
// barriers.
__device__ __forceinline__ bool sm_idle(int r0, int c0) { return r0 > c0 + 31; }

// C = alpha·L·Rᵀ + beta·D on 128 x 128 LDS matrices (K = 128). Every matrix
// here is symmetric, so L Rᵀ = L R.
__device__ __forceinline__ void sm_product(const SmMat& L, const SmMat& R, const SmMat& D, const SmMat& C, float alpha,
                                           float beta, int wave, int lane) {
  const int r0 = (wave >> 2) * 64, c0 = (wave & 3) * 32;
  const int r16 = lane & 15, g = lane >> 4;
  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  if (!sm_idle(r0, c0)) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {  // k = 32s .. 32s+31: logical chunks 4s .. 4s+3
      bf16x8 a[4], b[2];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = *(const bf16x8*)sm_at(L, r0 >> 6, 16 * i + r16, 4 * s + g);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = *(const bf16x8*)sm_at(R, c0 >> 6, (c0 & 63) + 16 * j + r16, 4 * s + g);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16(a[i], b[j], acc[i][j]);
    }
  }
  sm_finish(acc, D, C, alpha, beta, r0, c0, lane);
}

// Q = Z + a·I on the first m rows (pan/optim/patch_muon.py:321-324: the
// diagonal add in bf16); the padding rows and columns stay zero.
__device__ __forceinline__ void sm_qinit(const SmMat& Z, const SmMat& Q, float a, int m) {
#pragma clang fp contract(off)
  for (int i = threadIdx.x; i < kSm * kSm / 8; i += blockDim.x) {
    const int r = i >> 4, c = i & 15;  // logical chunk c of row r: columns 8c .. 8c+7
    u32x4 v = *(const u32x4*)sm_at(Z, r >> 6, r & 63, c);
    const int e = r - 8 * c;  // the diagonal element's position in the chunk
    if (r < m && e >= 0 && e < 8) {
      const uint32_t w = v[e >> 1];
      const uint16_t z = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
      const uint32_t qv = f2bf(bf2f(z) + a);
      v[e >> 1] = (e & 1) ? ((w & 0xffffu) | (qv << 16)) : ((w & 0xffff0000u) | qv);
    }
    *(u32x4*)sm_at(Q, r >> 6, r & 63, c) = v;
  }
  __syncthreads();
}

// Waits until at most n gram units (two copies each) of this wave are in flight.
__device__ __forceinline__ void wait_units(int n) {
  switch (n) {
    case 6: wait_vmcnt<12>(); break;
    case 5: wait_vmcnt<10>(); break;
    case 4: wait_vmcnt<8>(); break;
    case 3: wait_vmcnt<6>(); break;
    case 2: wait_vmcnt<4>(); break;
    case 1: wait_vmcnt<2>(); break;
    default: wait_vmcnt<0>(); break;
  }
}

// The gram ring: one __shared__ array per slot, so the compiler's LDS-DMA
// tracking sees that reads of one slot do not wait for copies into the others.
struct SmRing {
  char* s[kSmRing];
};

// Unit u of the gram, 64 k values: rows 0..127 of columns 64u .. 64u+63 of X,
// one contiguous 16 KiB block in the panel layout (sm_x_off); 16 copies of
// 1 KiB (8 rows); wave w issues copies 2w and 2w+1. Chunk c of row r is stored
// at chunk c ^ ((r >> 1) & 7), as in the grouped engine.
struct SmCopy {
  __amdgpu_buffer_rsrc_t rsrc;
  int voff[2];  // lane offsets of copies 2w, 2w+1
  int wave;
  __device__ __forceinline__ void operator()(char* dst, int u) const {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int q = 2 * wave + h;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, to_lds(dst + q * 1024), 16, voff[h], u * kSmUnit + q * 1024, 0,
                                               0);
    }
  }
};

// One unit in slot S of a ring of RING slots: wait for it, refill the slot read
// last (unit u-1's) with unit u + RING - 1, accumulate the unit's two k-steps.
// The barrier is a bare s_barrier: __syncthreads' fence would drain every copy
// in flight.
template <int RING, int S>
__device__ __forceinline__ void gram_unit(const SmRing& ring, const SmCopy& copy, int u, int KT, f32x4 (&acc)[4][2],
                                          int r0, int c0, int lane) {
  wait_units(min(RING - 2, KT - 1 - u));  // this wave's copies of unit u have landed
  block_barrier();  // every wave's copies of u have landed; every wave is done with unit u-1
  if (u + RING - 1 < KT) copy(ring.s[(S + RING - 1) % RING], u + RING - 1);
  if (sm_idle(r0, c0)) return;
  const char* src = ring.s[S];
  const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int fo = r16 * 128 + (((4 * s + g) ^ ((r16 >> 1) & 7)) << 4);
    bf16x8 a[4], b[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = *(const bf16x8*)(src + (r0 + 16 * i) * 128 + fo);
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = *(const bf16x8*)(src + (c0 + 16 * j) * 128 + fo);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16(a[i], b[j], acc[i][j]);
  }
}

// One block of 8 waves per small matrix of the group (grid = matrices).
// RING = kSmRing (gram form: R, Z, Q and RZ take the whole ring afterwards,
// one block per CU) or kSmRingStd (standard form, steps == 0: R and B fit in
// four slots, so two blocks share a CU and one's M x M part overlaps the
// other's gram stream).
template <int RING>
__global__ __launch_bounds__(kGemmThreads, kSmRing / RING) void pm_small_core_kernel(SmallCoreArgs args) {
#pragma clang fp contract(off)
  static_assert(RING == kSmRing || RING == kSmRingStd, "ring depth");
  __shared__ __attribute__((aligned(1024))) char g0[kSmUnit];
  __shared__ __attribute__((aligned(1024))) char g1[kSmUnit];
  __shared__ __attribute__((aligned(1024))) char g2[kSmUnit];
  __shared__ __attribute__((aligned(1024))) char g3[kSmUnit];
  SmRing ring;  // (set member by member: an aggregate initialiser of LDS addresses does not compile)
  ring.s[0] = g0; ring.s[1] = g1; ring.s[2] = g2; ring.s[3] = g3;
  // after the gram the ring holds the M x M matrices, two slots each
  SmMat R, Z, Q, RZ;
  R.h[0] = g0; R.h[1] = g1; Z.h[0] = g2; Z.h[1] = g3;
  if constexpr (RING == kSmRing) {
    __shared__ __attribute__((aligned(1024))) char g4[kSmUnit];
    __shared__ __attribute__((aligned(1024))) char g5[kSmUnit];
    __shared__ __attribute__((aligned(1024))) char g6[kSmUnit];
    __shared__ __attribute__((aligned(1024))) char g7[kSmUnit];
    ring.s[4] = g4; ring.s[5] = g5; ring.s[6] = g6; ring.s[7] = g7;
    Q.h[0] = g4; Q.h[1] = g5; RZ.h[0] = g6; RZ.h[1] = g7;
  }

  const MatDesc& d = args.descs[blockIdx.x];
  const int wave = wave_id(), lane = lane_id();
  const int r0 = (wave >> 2) * 64, c0 = (wave & 3) * 32;

  // ---- R = X Xᵀ over k < Np
  const int K = __builtin_amdgcn_readfirstlane(d.Np), KT = K / 64;
  SmCopy copy;
  copy.rsrc = uniform_rsrc(d.X[args.cur], (uint32_t)kSm * K * 2);
  copy.wave = wave;
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // copy q = 2w + h: row 8q + lane/8, stored chunk lane%8
    const int q = 2 * wave + h;
    const int sw = (4 * (q & 1) + (lane >> 4)) & 7;  // ((8q + lane/8) >> 1) & 7
    copy.voff[h] = (lane >> 3) * 128 + (((lane & 7) ^ sw) << 4);
  }
  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < RING - 1; ++i)
    if (i < KT) copy(ring.s[i], i);
  int u = 0;
  for (; u + RING <= KT; u += RING) {
    gram_unit<RING, 0>(ring, copy, u, KT, acc, r0, c0, lane);
    gram_unit<RING, 1>(ring, copy, u + 1, KT, acc, r0, c0, lane);
    gram_unit<RING, 2>(ring, copy, u + 2, KT, acc, r0, c0, lane);
    gram_unit<RING, 3>(ring, copy, u + 3, KT, acc, r0, c0, lane);
    if constexpr (RING == kSmRing) {
      gram_unit<RING, 4>(ring, copy, u + 4, KT, acc, r0, c0, lane);
      gram_unit<RING, 5>(ring, copy, u + 5, KT, acc, r0, c0, lane);
      gram_unit<RING, 6>(ring, copy, u + 6, KT, acc, r0, c0, lane);
      gram_unit<RING, 7>(ring, copy, u + 7, KT, acc, r0, c0, lane);
    }
  }
  if (u < KT) gram_unit<RING, 0>(ring, copy, u, KT, acc, r0, c0, lane);
  if (u + 1 < KT) gram_unit<RING, 1>(ring, copy, u + 1, KT, acc, r0, c0, lane);
  if (u + 2 < KT) gram_unit<RING, 2>(ring, copy, u + 2, KT, acc, r0, c0, lane);
  if constexpr (RING == kSmRing) {
    if (u + 3 < KT) gram_unit<RING, 3>(ring, copy, u + 3, KT, acc, r0, c0, lane);
    if (u + 4 < KT) gram_unit<RING, 4>(ring, copy, u + 4, KT, acc, r0, c0, lane);
    if (u + 5 < KT) gram_unit<RING, 5>(ring, copy, u + 5, KT, acc, r0, c0, lane);
    if (u + 6 < KT) gram_unit<RING, 6>(ring, copy, u + 6, KT, acc, r0, c0, lane);
  }
  // R = s²·X Xᵀ (s² = 1/‖X‖² on the unscaled first X): sm_finish's first
  // barrier also ends every wave's reads of the ring, whose first two slots
  // R overwrites (every copy has landed: the last unit waited for all)
  sm_finish(acc, R, R, args.first ? d.scales[0] : 1.0f, 0.0f, r0, c0, lane);

  // ---- the M x M part of the iteration
  const SmMat* out = &Z;
  if (RING == kSmRingStd || args.steps == 0) {
    const float* k = args.coeffs + 3 * args.it0;
    sm_product(R, R, R, Z, k[2], k[1], wave, lane);  // B = c R R + b R
  } else if constexpr (RING == kSmRing) {
    for (int i = 0; i < args.steps; ++i) {
      const float* k = args.coeffs + 3 * (args.it0 + i);
      const float a = k[0], b = k[1], c = k[2];
      sm_product(R, R, R, Z, c, b, wave, lane);  // Z = c R R + b R
      if (i == 0)
        sm_qinit(Z, Q, a, d.M);  // Q = a I + Z
      else
        sm_product(Q, Z, Q, Q, 1.0f, a, wave, lane);  // Q = Q Z + a Q
      if (i + 1 < args.steps) {
        sm_product(R, Z, R, RZ, 1.0f, a, wave, lane);   // RZ = R Z + a R
        sm_product(Z, RZ, RZ, R, 1.0f, a, wave, lane);  // R = Z RZ + a RZ
      }
    }
    out = &Q;
  }

  // ---- S (row-major 128 x 128) to the workspace
  uint16_t* S = d.S[args.so];
  for (int i = threadIdx.x; i < kSm * kSm / 8; i += blockDim.x) {
    const int r = i >> 4, c = i & 15;
    *(u32x4*)(S + r * kSm + 8 * c) = *(const u32x4*)sm_at(*out, r >> 6, r & 63, c);
  }
}

// Chunk c16 of row r of a flat LDS array of 256-byte rows, swizzled as in SmMat.
__device__ __forceinline__ int sm_off(int r, int c16) { return r * kSmRow + ((c16 ^ (r & 15)) << 4); }

// The X tile of an apply block in LDS, laid out as X is in HBM (sm_x_off):
// kSmApplyCols / 64 units of 64 columns (n), each kSm rows (k) of 128 B.
// Chunk c (16 B, columns 8c .. 8c+7 of the unit) of row k is stored at chunk
// c ^ (2·((k >> 3) & 3)): the transposed fragment reads (16 consecutive
// columns of rows k, k+8, k+16, k+24 in one instruction) then fall in 32
// distinct banks.
constexpr int kSmXUnits = kSmApplyCols / 64;  // units per tile
__device__ __forceinline__ int xt_off(int k, int n) {
  return (n >> 6) * kSmUnit + k * 128 + ((((n >> 3) & 7) ^ (((k >> 3) & 3) << 1)) << 4) + (n & 7) * 2;
}

// Param elements r, c0 .. c0+3 of a small matrix's FINAL: whether the row is
// in bounds, and whether the 4 elements are one aligned vector.
struct Quad4 {
  int r, c0;
  bool in_row, full;
};
template <bool F32P>
__device__ __forceinline__ Quad4 quad4_at(const MatDesc& d, int r, int c0) {
  Quad4 q{r, c0, r < d.rows, false};
  q.full = q.in_row && c0 + 3 < d.cols && (d.p_ld % 4 == 0) && ((uintptr_t)d.param % (F32P ? 16 : 8) == 0);
  return q;
}
// The 4 param elements as stored (2 registers for bf16, 4 for fp32); zeros
// outside the param.
template <bool F32P>
__device__ __forceinline__ typename PickVec<F32P>::type load_param4(const MatDesc& d, const Quad4& q) {
  typedef typename PickVec<F32P>::elem E;
  typedef typename PickVec<F32P>::type V;
  const E* src = (const E*)d.param + (int64_t)q.r * d.p_ld + q.c0;
  if (q.full) return *(const V*)src;
  V v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (q.in_row && q.c0 + e < d.cols) ? src[e] : (E)0;
  return v;
}
template <bool F32P>
__device__ __forceinline__ void store_param4(const MatDesc& d, const Quad4& q, const float (&v)[4]) {
  typedef typename PickVec<F32P>::elem E;
  E* dst = (E*)d.param + (int64_t)q.r * d.p_ld + q.c0;
  if (q.full) {
    typename PickVec<F32P>::type pv;
#pragma unroll
    for (int e = 0; e < 4; ++e) pv[e] = F32P ? (E)v[e] : (E)f2bf(v[e]);
    *(typename PickVec<F32P>::type*)dst = pv;
  } else if (q.in_row) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (q.c0 + e < d.cols) dst[e] = F32P ? (E)v[e] : (E)f2bf(v[e]);
  }
}

// X' = s·(a·X + S X) for one tile of kSmApplyCols columns of a small matrix
// per block (prefix: ceil(Np / kSmApplyCols) tiles per matrix). Small
// matrices keep X only (no Xᵀ): the X tile, 128 contiguous KiB of HBM in the
// panel layout (sm_x_off), is copied into LDS in that layout, and the MFMA's
// B fragments (8 consecutive k of one column) are read from it transposed,
// element by element. Each wave owns a 128 x 64 wave tile. The arithmetic is
// the grouped engine's UPDATE / FINAL (the same MFMA over the same k order,
// the same rounding points), so the result equals the engine's on the
// zero-padded matrix; only the stores differ: X' alone (no Xᵀ copy), and the
// parameter step in param layout for wide and tall matrices alike.
template <int STAGE, int PDT>
__global__ __launch_bounds__(kSmApplyThreads, 1) void pm_small_apply_kernel(GemmArgs args) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(1024))) char sbuf[kSm * kSmRow];       // S, 32 KiB
  __shared__ __attribute__((aligned(1024))) char xbuf[kSmXUnits * kSmUnit];  // X tile, 128 KiB
  const int t = blockIdx.x;
  const int m = find_matrix(args.prefix, args.n, t);
  const MatDesc& d = args.descs[m];
  const int lt = t - args.prefix[m];
  const int w = wave_id(), lane = lane_id();
  const int Np = __builtin_amdgcn_readfirstlane(d.Np);
  const int n0 = lt * kSmApplyCols;
  const int nx = min(kSmApplyCols, Np - n0);  // columns of this tile inside X
  const uint16_t* X = d.X[args.cur];
  {
    // S: copy q moves rows 4q .. 4q+3 (1 KiB); lane l lands at row 4q + l/16,
    // stored chunk l%16, so it loads logical chunk (l%16) ^ ((4q + l/16) & 15)
    const __amdgpu_buffer_rsrc_t rs = uniform_rsrc(d.S[args.sl], (uint32_t)kSm * kSmRow);
    const int row = lane >> 4;
    for (int q = w; q < kSm / 4; q += kSmApplyWaves) {
      const int voff = row * kSmRow + (((lane & 15) ^ ((4 * q + row) & 15)) << 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, to_lds(sbuf + q * 1024), 16, voff, q * 4 * kSmRow, 0, 0);
    }
    // X tile: the tile's units are contiguous in HBM (sm_x_off; n0 is a
    // multiple of 64). Wave w moves unit w, the 64 columns its S X products
    // read: copy i moves rows 8i .. 8i+7 (1 KiB); lane l lands at row 8i + l/8,
    // stored chunk l%8, so it loads logical chunk (l%8) ^ swizzle(row). Units
    // past Np read as zeros (buffer bounds).
    static_assert(kSmXUnits == kSmApplyWaves, "one unit of the X tile per wave");
    const __amdgpu_buffer_rsrc_t rx = uniform_rsrc(X + sm_x_off(0, n0), (uint32_t)(nx / 64) * kSmUnit);
#pragma unroll
    for (int i = 0; i < kSm / 8; ++i) {
      const int k = 8 * i + (lane >> 3);
      const int lc = (lane & 7) ^ (((k >> 3) & 3) << 1);  // logical chunk of row k
      const int voff = 64 * w < nx ? w * kSmUnit + k * 128 + lc * 16 : 0x7fffffff;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, to_lds(xbuf + w * kSmUnit + i * 1024), 16, voff, 0, 0, 0);
    }
  }
  // S is shared: every wave's S copies (issued before its X copies) land
  // before the block barrier. X is not: a wave waits for its own unit only,
  // except in the wide FINAL, whose waves read two units each. Bare barriers:
  // __syncthreads' fence would wait for every copy in flight.
  wait_vmcnt<kSm / 8>();
  block_barrier();
  wait_vmcnt<0>();
  if (STAGE == ST_FINAL && !d.trans) block_barrier();
  const int r16 = lane & 15, g = lane >> 4;
  // the MFMA fragment of X column n for k-step s (k = 32s + 8g .. +7), read
  // transposed from the tile, element by element
  auto xcol = [&](int s, int n) {
    typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
    u16x8 v;
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = *(const uint16_t*)(xbuf + xt_off(32 * s + 8 * g + e, n));
    return __builtin_bit_cast(bf16x8, v);
  };
  f32x4 acc[kMi][kNi];
#pragma unroll
  for (int i = 0; i < kMi; ++i)
#pragma unroll
    for (int j = 0; j < kNi; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  if (STAGE == ST_FINAL && !d.trans) {
    // wide FINAL: the transposed tile X'ᵀ = Xᵀ Sᵀ, whose quads are param rows,
    // finished by the grouped engine's FINAL epilogue. Wave w owns Xᵀ rows
    // (columns n of X) xr .. xr+127, xr = 128(w/2), and S rows 64(w%2) .. +63.
    const int xr = 128 * (w >> 1);
    if (xr >= nx) return;  // past Np: no barrier follows
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      bf16x8 b[kNi];
#pragma unroll
      for (int j = 0; j < kNi; ++j) b[j] = *(const bf16x8*)(sbuf + sm_off(64 * (w & 1) + 16 * j + r16, 4 * s + g));
#pragma unroll
      for (int i = 0; i < kMi; ++i) {
        const bf16x8 a = xcol(s, xr + 16 * i + r16);
#pragma unroll
        for (int j = 0; j < kNi; ++j) acc[i][j] = mfma_bf16(a, b[j], acc[i][j]);
      }
    }
    const int xg = n0 + xr;  // first n of the wave
    TileJob job{};
    job.ti = xg / kTile;
    job.tj = 0;
    const int ew = ((xg % kTile) / kWaveRows) * 4 + (w & 1);  // the engine wave whose quads these are
    if (args.a != 0.0f) {
      // a·X from the tile in LDS rather than from HBM: quad (i, j) is
      // Xᵀ[xr + 16i + 4g .. +3][m], m = 64(w%2) + 16j + lane%16, i.e. 4
      // consecutive columns of X row m; acc = a·x + acc as the engine's epilogue
      // forms it
      const float ca = args.a;
#pragma unroll
      for (int i = 0; i < kMi; ++i)
#pragma unroll
        for (int j = 0; j < kNi; ++j) {
          const u16x4 xq = *(const u16x4*)(xbuf + xt_off(64 * (w & 1) + 16 * j + r16, xr + 16 * i + 4 * g));
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] = ca * bf2f(xq[r]) + acc[i][j][r];
        }
      gemm_epilogue<ST_FINAL, PDT, 0, true>(args, d, job, acc, ew);
    } else {
      gemm_epilogue<ST_FINAL, PDT, 0>(args, d, job, acc, ew);  // a = 0: X is not read
    }
    return;
  }
  // S X: wave w owns columns xr .. xr+63 of the tile (B = X, read transposed), all 128 rows (A = S)
  const int xr = 64 * w;
  if (xr >= nx) return;  // past Np: no barrier follows
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    bf16x8 b[kNi];
#pragma unroll
    for (int j = 0; j < kNi; ++j) b[j] = xcol(s, xr + 16 * j + r16);
#pragma unroll
    for (int i = 0; i < kMi; ++i) {
      const bf16x8 a = *(const bf16x8*)(sbuf + sm_off(16 * i + r16, 4 * s + g));
#pragma unroll
      for (int j = 0; j < kNi; ++j) acc[i][j] = mfma_bf16(a, b[j], acc[i][j]);
    }
  }

  // ---- epilogue: o = bf16(s·(a·X + S X)) at rows p0 .. p0+3 of column q per quad
  const float sc = args.first ? d.scales[1] : 1.0f;
  const float ca = args.a;
  // the o quad of (i, j), in the accumulator layout
  auto quad_o = [&](int i, int j, u16x4& o) {
    const int pr = 16 * i + 4 * g + (lane & 3);
    const int q4 = (xr + 16 * j + r16) & ~3;
    u16x4 xq = (u16x4){0, 0, 0, 0};
    if (ca != 0.0f)  // X[pr][q4 .. q4+3] from the tile, then to the quad layout
      xq = quad_transpose(*(const u16x4*)(xbuf + xt_off(pr, q4)), lane);
#pragma unroll
    for (int r = 0; r < 4; ++r) o[r] = f2bf((ca * bf2f(xq[r]) + acc[i][j][r]) * sc);
  };
  if (STAGE == ST_UPDATE) {
    uint16_t* Xn = d.X[args.cur ^ 1];
#pragma unroll
    for (int i = 0; i < kMi; ++i)
#pragma unroll
      for (int j = 0; j < kNi; ++j) {
        u16x4 o;
        quad_o(i, j, o);
        const int pr = 16 * i + 4 * g + (lane & 3), q4 = (xr + 16 * j + r16) & ~3;
        *(u16x4*)(Xn + sm_x_off(pr, n0 + q4)) = quad_transpose(o, lane);  // row pr, columns q4 .. +3
      }
    return;
  }
  // FINAL of a tall matrix (a wide one returned above): param row n0 + q,
  // columns p0 .. p0+3, o as it is. Param loads go out kBatch rows of quads
  // at a time, before any of them is combined.
  constexpr bool f32p = PDT == DT_F32;
  constexpr int kBatch = f32p ? 2 : 4;
  const bool step = args.mode == MODE_STEP;
  float wdf = 0.0f, neg = 0.0f;
  if (step) {
    if (args.lr_dev) {
      const float lr = *args.lr_dev;
      wdf = 1.0f - lr * args.wd;
      neg = -(lr * d.adj_ratio);
    } else {
      wdf = args.wdf_host;
      neg = d.neg_lr_host;
    }
  }
#pragma unroll
  for (int i0 = 0; i0 < kMi; i0 += kBatch) {
    __builtin_amdgcn_sched_barrier(0);
    typename PickVec<f32p>::type pv[kBatch][kNi];
#pragma unroll
    for (int bi = 0; bi < kBatch; ++bi)
#pragma unroll
      for (int j = 0; j < kNi; ++j) {
        const Quad4 qd = quad4_at<f32p>(d, n0 + xr + 16 * j + r16, 16 * (i0 + bi) + 4 * g);
        if (step) pv[bi][j] = load_param4<f32p>(d, qd);
      }
#pragma unroll
    for (int bi = 0; bi < kBatch; ++bi)
#pragma unroll
      for (int j = 0; j < kNi; ++j) {
        const Quad4 qd = quad4_at<f32p>(d, n0 + xr + 16 * j + r16, 16 * (i0 + bi) + 4 * g);
        u16x4 o;
        quad_o(i0 + bi, j, o);
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float pe = f32p ? (float)pv[bi][j][e] : bf2f((uint16_t)pv[bi][j][e]);
          v[e] = step ? pe * wdf + bf2f(o[e]) * neg : bf2f(o[e]);
        }
        store_param4<f32p>(d, qd, v);
      }
  }
}

}  // namespace pm
