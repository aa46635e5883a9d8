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
//   pm_small_apply_kernel  X' = s·(a·X + S X) with the arithmetic of the
//                          grouped engine's UPDATE / FINAL (X', or the fused
//                          parameter step): one persistent block per CU
//                          streams 64-column units of X (and, for the step,
//                          their param blocks) through an LDS ring across
//                          matrices. The apply reads X transposed from LDS.
//
// With many matrices in a call, the R a core launch starts from is formed by
// the kernel that wrote X instead: the UPDATE apply (its X'), and for the
// first launch pm_small_prologue_kernel, which runs the momentum prologue, the
// norm and the first gram in one pass. The core launches then read R only.
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
constexpr int kSmApplyWaves = 8;      // apply blocks: 8 waves, each 64 rows x 16 columns of a unit
constexpr int kSmApplyThreads = 64 * kSmApplyWaves;
constexpr int kSmApplyCols = 64;      // columns of X per apply work item: one 16 KiB unit

struct SmallCoreArgs {
  const MatDesc* descs;
  const float* coeffs;  // (a, b, c) of every Newton–Schulz iteration, on the device
  int32_t it0;          // first iteration of this launch
  int32_t steps;        // gram form: core steps of the segment; 0: standard form, S = c R² + b R
  int32_t cur;          // X slot holding the current X
  int32_t first;        // scale R by 1/‖X‖² (the Frobenius normalisation, folded)
  int32_t so;           // square buffer receiving S
  int32_t r_in;         // R is already in S[so] (written by the apply that made X): skip the gram
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

// A 128 x 128 bf16 matrix in LDS, rows 0..63 in h0 and 64..127 in h1
// (two 16 KiB gram-ring slots). Row r is 256 B and chunk c (16 B, columns
// 8c .. 8c+7) of row r is stored at chunk c ^ (r & 15), so the 16 rows of an
// MFMA operand read of one chunk hit 16 different bank groups. Every access
// below names its half from wave-uniform values.
struct SmMat {
  char* h0;  // rows 0..63
  char* h1;  // rows 64..127
};
// chunk c16 of row (64·half + rr)
__device__ __forceinline__ char* sm_at(const SmMat& m, int half, int rr, int c16) {
  // a select, not h[half]: a runtime index into the pair would keep it in
  // scratch memory and reload the base from there on every access
  return (half ? m.h1 : m.h0) + rr * kSmRow + ((c16 ^ (rr & 15)) << 4);
}
// element (64·half + rr, q)
__device__ __forceinline__ uint16_t* sm_el(const SmMat& m, int half, int rr, int q) {
  return (uint16_t*)(sm_at(m, half, rr, q >> 3) + (q & 7) * 2);
}

// 16-byte LDS accesses through a pointer the compiler may only know as
// generic (an LDS matrix picked at run time): the cast keeps them ds_
// instructions rather than flat ones, which would also count in vmcnt.
typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
__device__ __forceinline__ u32x4 lds_load16(const char* p) { return *(const lds_u32x4*)(p); }
__device__ __forceinline__ void lds_store16(char* p, u32x4 v) { *(lds_u32x4*)(p) = v; }
// and 16-byte accesses of the workspace, whose pointers come from the
// descriptor table (global_ rather than flat instructions)
typedef __attribute__((address_space(1))) u32x4 glb_u32x4;
__device__ __forceinline__ u32x4 glb_load16(const uint16_t* p) { return *(const glb_u32x4*)(p); }
__device__ __forceinline__ void glb_store16(uint16_t* p, u32x4 v) { *(glb_u32x4*)(p) = v; }

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

// The gram's two k-steps over one unit in LDS (rows 0..127 of 64 k values,
// chunk c of row r stored at chunk c ^ ((r >> 1) & 7)): wave w accumulates rows
// r0 .. r0+63 of columns c0 .. c0+31 of R = X Xᵀ (the layout sm_finish takes).
__device__ __forceinline__ void sm_gram_acc(const char* src, f32x4 (&acc)[4][2], int r0, int c0, int lane) {
  if (sm_idle(r0, c0)) return;
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

// R = bf16(alpha·acc) written row-major (128 x 128) to global memory, through
// the LDS matrix T: elements on and above the diagonal at (p, q) and (q, p),
// as sm_finish writes them with beta = 0 (the same expression, so the same
// bits), then whole rows out with 16-byte stores. Every wave of the block
// calls it: it begins with a barrier (every wave's earlier reads of T's tiles
// have completed: their MFMAs consumed them) and ends with one (every read of T
// is done, so the tiles may be written again). The barriers are bare: a
// __syncthreads fence would also wait for the copies in flight.
__device__ __forceinline__ void sm_gram_store(uint16_t* Rg, const SmMat& T, const f32x4 (&acc)[4][2], int r0, int c0,
                                              int lane, float alpha = 1.0f) {
#pragma clang fp contract(off)
  const int g = lane >> 4;
  const int rh = r0 >> 6, ch = c0 >> 6, cr = c0 & 63;
  const float beta = 0.0f;
  u16x4 o[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[i][j][r] = f2bf(alpha * acc[i][j][r] + beta * bf2f((uint16_t)0));
  block_barrier();
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int p0 = r0 + 16 * i + 4 * g, q = c0 + 16 * j + (lane & 15);
      store_upper4(sm_el(T, rh, 16 * i + 4 * g + (lane & 3), q & ~3), quad_transpose(o[i][j], lane), q & ~3,
                   p0 + (lane & 3));
      store_lower4(sm_el(T, ch, cr + 16 * j + (lane & 15), p0), o[i][j], p0, q);
    }
  wait_lgkmcnt<0>();
  block_barrier();
  for (int i = threadIdx.x; i < kSm * kSm / 8; i += blockDim.x) {
    const int r = i >> 4, c = i & 15;
    glb_store16(Rg + r * kSm + 8 * c, lds_load16(sm_at(T, r >> 6, r & 63, c)));
  }
  wait_lgkmcnt<0>();
  block_barrier();
}

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
  sm_gram_acc(ring.s[S], acc, r0, c0, lane);
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
  R.h0 = g0; R.h1 = g1; Z.h0 = g2; Z.h1 = g3;
  if constexpr (RING == kSmRing) {
    __shared__ __attribute__((aligned(1024))) char g4[kSmUnit];
    __shared__ __attribute__((aligned(1024))) char g5[kSmUnit];
    __shared__ __attribute__((aligned(1024))) char g6[kSmUnit];
    __shared__ __attribute__((aligned(1024))) char g7[kSmUnit];
    ring.s[4] = g4; ring.s[5] = g5; ring.s[6] = g6; ring.s[7] = g7;
    Q.h0 = g4; Q.h1 = g5; RZ.h0 = g6; RZ.h1 = g7;
  }

  const MatDesc& d = args.descs[blockIdx.x];
  const int wave = wave_id(), lane = lane_id();
  const int r0 = (wave >> 2) * 64, c0 = (wave & 3) * 32;

  if (args.r_in) {
    // ---- R from S[so], where the apply that produced X stored it
    const uint16_t* Rg = d.S[args.so];
    for (int i = threadIdx.x; i < kSm * kSm / 8; i += blockDim.x) {
      const int r = i >> 4, c = i & 15;
      lds_store16(sm_at(R, r >> 6, r & 63, c), glb_load16(Rg + r * kSm + 8 * c));
    }
    __syncthreads();
  } else {
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
  }

  // ---- the M x M part of the iteration
  bool out_q = false;  // S = Z (standard form) or Q (gram form)
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
    out_q = true;
  }

  // ---- S (row-major 128 x 128) to the workspace
  uint16_t* S = d.S[args.so];
  for (int i = threadIdx.x; i < kSm * kSm / 8; i += blockDim.x) {
    const int r = i >> 4, c = i & 15;
    const SmMat out{out_q ? Q.h0 : Z.h0, out_q ? Q.h1 : Z.h1};
    glb_store16(S + r * kSm + 8 * c, lds_load16(sm_at(out, r >> 6, r & 63, c)));
  }
}

// ============================================================ prologue + first gram
// Largest prologue partial count per matrix (2 tile rows x 1024 runs: a long
// side of 262144) that pm_small_prologue_kernel keeps in LDS.
constexpr int kSmProParts = 2048;

// The descriptor fields pm_small_prologue_kernel's tile loop reads, loaded
// once into scalar registers: read through the descriptor after the loop's
// stores, they would be reloaded with vector loads every tile.
struct ProMat {
  const void* grad;
  void* mom;
  uint16_t* X;
  int64_t g_ld, m_ld;
  int32_t rows, cols, g_dt, m_dt, trans;
};
__device__ __forceinline__ int32_t uni32(int32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ int64_t uni64(int64_t v) {
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)(uint64_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
  return (int64_t)(((uint64_t)hi << 32) | lo);
}
__device__ __forceinline__ ProMat pro_mat(const MatDesc& d) {
  ProMat q;
  q.grad = (const void*)uni64((int64_t)d.grad);
  q.mom = (void*)uni64((int64_t)d.mom);
  q.X = (uint16_t*)uni64((int64_t)d.X[0]);
  q.g_ld = uni64(d.g_ld);
  q.m_ld = uni64(d.m_ld);
  q.rows = uni32(d.rows);
  q.cols = uni32(d.cols);
  q.g_dt = uni32(d.g_dt);
  q.m_dt = uni32(d.m_dt);
  q.trans = uni32(d.trans);
  return q;
}

// A run of 8 elements' gradient and momentum as loaded (G32 / M32: fp32,
// else bf16), for the runs that take the vector path: pm_small_prologue_kernel
// issues the loads of four runs before the arithmetic of any of them.
template <bool G32, bool M32>
struct ProRaw {
  u32x4 g[G32 ? 2 : 1];
  u32x4 m[M32 ? 2 : 1];
};

// The 16-byte loads pm_prologue_kernel makes for param row pr, columns
// pc .. pc+7 (gvec / mvec: the vector path is allowed and the dtype is the
// template's).
template <bool G32, bool M32>
__device__ __forceinline__ void pro_fetch8(const ProMat& d, bool step, int pr, int pc, bool gvec, bool mvec,
                                           ProRaw<G32, M32>& raw) {
  const bool full = pr < d.rows && d.cols - pc >= 8;
  raw = ProRaw<G32, M32>{};  // defined where the loads are skipped
  // global_ rather than flat loads: a flat load also counts in lgkmcnt, and
  // the compiler then drains every counter before using any of them
  if (full && gvec) {
    const glb_u32x4* p = (const glb_u32x4*)((const char*)d.grad + ((int64_t)pr * d.g_ld + pc) * (G32 ? 4 : 2));
    raw.g[0] = p[0];
    if constexpr (G32) raw.g[1] = p[1];
  }
  if (full && step && mvec) {
    const glb_u32x4* p = (const glb_u32x4*)((const char*)d.mom + ((int64_t)pr * d.m_ld + pc) * (M32 ? 4 : 2));
    raw.m[0] = p[0];
    if constexpr (M32) raw.m[1] = p[1];
  }
}

// 8 floats from a run's raw vector (load8's conversions).
template <bool F32, int N>
__device__ __forceinline__ void pro_unpack8(const u32x4 (&v)[N], float (&x)[8]) {
  if constexpr (F32) {
    // through scalars: this clang's __builtin_bit_cast of a vector element
    // (v[i][e]) reads element 0 whatever e is
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const uint32_t lo = v[0][e], hi = v[N - 1][e];
      x[e] = __builtin_bit_cast(float, lo);
      x[4 + e] = __builtin_bit_cast(float, hi);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      x[2 * e] = bf2f((uint16_t)(v[0][e] & 0xffff));
      x[2 * e + 1] = bf2f((uint16_t)(v[0][e] >> 16));
    }
  }
}

// load_elem / store_elem as global_ accesses (flat ones would make the
// compiler drain every counter at each later wait in the kernel).
__device__ __forceinline__ float load_elem_g(const void* p, int32_t dt, int64_t i) {
  typedef const __attribute__((address_space(1))) float gf;
  typedef const __attribute__((address_space(1))) uint16_t gh;
  return dt == DT_F32 ? ((gf*)p)[i] : bf2f(((gh*)p)[i]);
}
__device__ __forceinline__ void store_elem_g(void* p, int32_t dt, int64_t i, float v) {
  typedef __attribute__((address_space(1))) float gf;
  typedef __attribute__((address_space(1))) uint16_t gh;
  if (dt == DT_F32) ((gf*)p)[i] = v;
  else ((gh*)p)[i] = f2bf(v);
}

// pm_prologue_kernel's arithmetic on one run of 8 elements of param row pr,
// columns pc .. pc+7, with its vector loads already issued into raw
// (pro_fetch8 with the same gvec / mvec); runs off the vector path load
// element by element here. The momentum update is stored back and u (the
// Nesterov blend, or the gradient in MODE_NS) is rounded to bf16 and packed;
// ss accumulates the squares of the rounded values in element order, and
// elements outside the parameter are zeros of X. mvec_any: the caller's
// strides and bases allow the momentum's 16-byte stores, whatever its dtype.
// FAST: the matrix allows the vector path for every run inside it (gvec,
// mvec in MODE_STEP, and a column count that is a multiple of 8), so every
// run is either whole or padding, and raw comes from sm_pro_fetch_buf (zeros
// for padding): no element loads remain.
template <bool FAST, bool G32, bool M32>
__device__ __forceinline__ u32x4 pro_finish8(const ProArgs& args, const ProMat& d, int pr, int pc, bool gvec,
                                             bool mvec, bool mvec_any, const ProRaw<G32, M32>& raw, float& ss) {
#pragma clang fp contract(off)
  const float mu = args.mu, omu = 1.0f - args.mu;
  const bool step = args.mode == MODE_STEP;
  const bool in_row = pr < d.rows;
  const int valid = d.cols - pc;  // elements of the run inside the parameter
  const bool full = in_row && valid >= 8;
  float u[8];
  float g[8];
  // The element loads of the other runs complete inside their branch (the
  // empty asm uses them there): loads still pending at the join would make
  // the vector path wait for every load in flight, the next run's included.
  if (FAST || (full && gvec)) {
    pro_unpack8<G32>(raw.g, g);  // FAST: zeros outside the parameter
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      g[e] = (in_row && e < valid) ? load_elem_g(d.grad, d.g_dt, (int64_t)pr * d.g_ld + pc + e) : 0.0f;
      asm volatile("" : "+v"(g[e]));
    }
  }
  if (step) {
    float m[8];
    const int64_t mo = (int64_t)pr * d.m_ld + pc;
    if (FAST || (full && mvec)) {
      pro_unpack8<M32>(raw.m, m);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        m[e] = (in_row && e < valid) ? load_elem_g(d.mom, d.m_dt, mo + e) : 0.0f;
        asm volatile("" : "+v"(m[e]));
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float nm = mu * m[e] + omu * g[e];
      m[e] = nm;
      u[e] = args.nesterov ? omu * g[e] + mu * nm : nm;
    }
    // store8's stores, the 16-byte ones as global_ stores
    if (in_row && mvec_any && valid >= 8) {
      if (d.m_dt == DT_F32) {
        typedef __attribute__((address_space(1))) f32x4 glb_f32x4;
        glb_f32x4* q = (glb_f32x4*)((float*)d.mom + mo);
        q[0] = (f32x4){m[0], m[1], m[2], m[3]};
        q[1] = (f32x4){m[4], m[5], m[6], m[7]};
      } else {
        u32x4 a;
#pragma unroll
        for (int e = 0; e < 4; ++e) a[e] = (uint32_t)f2bf(m[2 * e]) | ((uint32_t)f2bf(m[2 * e + 1]) << 16);
        *(glb_u32x4*)((uint16_t*)d.mom + mo) = a;
      }
    } else if (!FAST && in_row) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (e < valid) store_elem_g(d.mom, d.m_dt, mo + e, m[e]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) u[e] = g[e];
  }
  u32x4 packed;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint16_t lo = (in_row && 2 * e < valid) ? f2bf(u[2 * e]) : (uint16_t)0;
    const uint16_t hi = (in_row && 2 * e + 1 < valid) ? f2bf(u[2 * e + 1]) : (uint16_t)0;
    const float flo = bf2f(lo), fhi = bf2f(hi);
    ss += flo * flo;
    ss += fhi * fhi;
    packed[e] = (uint32_t)lo | ((uint32_t)hi << 16);
  }
  return packed;
}

// The param origin of tile tj of X rows 64·half .. 64·half+63, and this
// thread's place in it (thread t of the half: rows t/8 and t/8 + 32 of the
// tile, columns 8(t%8) .. +7, as pm_prologue_kernel's thread t). t is rebuilt
// from the lane index at each use, so per-lane offsets are not hoisted out of
// the tile loop (where they would all stay live).
struct ProPos {
  int t, cg, pr0, pc0;
};
__device__ __forceinline__ ProPos sm_pro_pos(const ProMat& d, int tj, int half, int wq) {
  ProPos q;
  q.t = wq * 64 + lane_id();
  q.cg = (q.t & 7) * 8;
  q.pr0 = d.trans ? tj * kProTile : half * kProTile;
  q.pc0 = d.trans ? half * kProTile : tj * kProTile;
  return q;
}

// The loads of half h of tile tj (param row pr0 + t/8 + 32h) into raw.
template <bool G32, bool M32>
__device__ __forceinline__ void sm_pro_fetch(const ProMat& d, bool step, int tj, int h, int half, int wq, bool gvec,
                                             bool mvec, ProRaw<G32, M32>& raw) {
  const ProPos q = sm_pro_pos(d, tj, half, wq);
  pro_fetch8(d, step, q.pr0 + (q.t >> 3) + 32 * h, q.pc0 + q.cg, gvec, mvec, raw);
}

// sm_pro_fetch for a FAST matrix, as buffer loads issued by every lane: a run
// outside the parameter (padding rows or columns) gets an offset beyond the
// resource's range, whose loads return zeros. Loads issued under a branch
// would leave the compiler unsure how many loads follow a register set's,
// and it would then wait for all of them. rg / rm cover the gradient and the
// momentum (extents below 2 GiB).
template <bool G32, bool M32>
__device__ __forceinline__ void sm_pro_fetch_buf(const ProMat& d, bool step, __amdgpu_buffer_rsrc_t rg,
                                                 __amdgpu_buffer_rsrc_t rm, int tj, int h, int half, int wq,
                                                 ProRaw<G32, M32>& raw) {
  const ProPos q = sm_pro_pos(d, tj, half, wq);
  const int pr = q.pr0 + (q.t >> 3) + 32 * h, pc = q.pc0 + q.cg;
  const bool full = pr < d.rows && d.cols - pc >= 8;
  const uint32_t og = full ? (uint32_t)(((int64_t)pr * d.g_ld + pc) * (G32 ? 4 : 2)) : 0x80000000u;
  raw.g[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rg, og, 0, 0));
  if constexpr (G32) raw.g[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rg, og + 16, 0, 0));
  if (step) {
    const uint32_t om = full ? (uint32_t)(((int64_t)pr * d.m_ld + pc) * (M32 ? 4 : 2)) : 0x80000000u;
    raw.m[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rm, om, 0, 0));
    if constexpr (M32) raw.m[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rm, om + 16, 0, 0));
  }
}

// Half h of tile tj (64 columns of X: one gram unit) of a small matrix in a
// pm_small_prologue_kernel block: pm_prologue_kernel's work on the run of 8
// elements its thread t takes in that half of the tile (X rows
// 64·half .. 64·half+63), from the loads in raw; the run's X also goes into
// LDS unit `unit` (the gram's unit layout: row r, chunk c at chunk
// c ^ ((r >> 1) & 7)). ss accumulates the thread's squares as
// pm_prologue_kernel's thread t does (h = 0, then 1, tile by tile).
template <bool FAST, bool G32, bool M32>
__device__ __forceinline__ void sm_pro_run(const ProArgs& args, const ProMat& d, char* unit, int tj, int h, int half,
                                           int wq, bool gvec, bool mvec, bool mvec_any, const ProRaw<G32, M32>& raw,
                                           float& ss) {
  const ProPos q = sm_pro_pos(d, tj, half, wq);
  const int r = (q.t >> 3) + 32 * h;
  const u32x4 packed = pro_finish8<FAST>(args, d, q.pr0 + r, q.pc0 + q.cg, gvec, mvec, mvec_any, raw, ss);
  if (!d.trans) {
    // X row 64·half + r, columns 64·tj + cg .. +7
    const int xr = half * kProTile + r;
    glb_store16(d.X + sm_x_off(xr, tj * kProTile + q.cg), packed);
    lds_store16(unit + xr * 128 + (((q.cg >> 3) ^ ((xr >> 1) & 7)) << 4), packed);
  } else {
    // param row pr0 + r is X column 64·tj + r; its columns cg .. cg+7 are X
    // rows 64·half + cg + e
    typedef __attribute__((address_space(3))) uint16_t lds_u16;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int xr = half * kProTile + q.cg + e;
      const uint16_t v = (uint16_t)(packed[e >> 1] >> (16 * (e & 1)));
      *(lds_u16*)(unit + xr * 128 + (((r >> 3) ^ ((xr >> 1) & 7)) << 4) + (r & 7) * 2) = v;
    }
  }
}

// A transposed tile's X rows out of LDS: thread t of the half writes X row
// 64·half + t/4, columns 64·tj + 16·(t%4) .. +15 (the rows the prologue's
// transposing tile gives pm_prologue_kernel's thread t).
__device__ __forceinline__ void sm_pro_flush_tr(const ProMat& d, const char* unit, int tj, int half, int wq) {
  const int t = wq * 64 + lane_id();
  const int xr = half * kProTile + (t >> 2), rb = (t & 3) * 16;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c8 = (rb >> 3) + h;
    glb_store16(d.X + sm_x_off(xr, tj * kProTile + 8 * c8),
                lds_load16(unit + xr * 128 + ((c8 ^ ((xr >> 1) & 7)) << 4)));
  }
}

// pm_small_prologue_kernel's pass over the tiles of its matrix (the
// prologue, the partial sums and the gram's accumulation, run by run).
template <bool FAST, bool G32, bool M32>
__device__ __forceinline__ void sm_pro_tiles(const ProArgs& args, const ProMat& pm, char (*units)[kSmUnit], float* parts,
                                             float* red, float* partials, f32x4 (&acc)[4][2], int nrun, int half,
                                             int wq, bool gvec, bool mvec, bool mvec_any, __amdgpu_buffer_rsrc_t rg,
                                             __amdgpu_buffer_rsrc_t rm) {
  auto fetch = [&](int tj, int h, ProRaw<G32, M32>& raw) {
    if constexpr (FAST)
      sm_pro_fetch_buf(pm, args.mode == MODE_STEP, rg, rm, tj, h, half, wq, raw);
    else
      sm_pro_fetch(pm, args.mode == MODE_STEP, tj, h, half, wq, gvec, mvec, raw);
  };
  const int wave = 4 * half + wq, lane = lane_id();
  const int r0 = half * 64, c0 = wq * 32;
  const int ntiles = nrun * kProRun;
  // Tiles go in pairs: the four runs of a pair are loaded before any of
  // their arithmetic, so each thread has four loads in flight at once. (The
  // compiler waits for every memory operation before using a load's result
  // whenever stores are pending, so loads issued a run ahead across the
  // previous run's stores gain nothing.)
  float ss = 0.0f;
  for (int tj = 0; tj < ntiles; tj += 2) {
    const int tt = tj & (kProRun - 1), run = tj / kProRun;
    ProRaw<G32, M32> r[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) fetch(tj + (i >> 1), i & 1, r[i]);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      sm_pro_run<FAST>(args, pm, units[tt + (i >> 1)], tj + (i >> 1), i & 1, half, wq, gvec, mvec, mvec_any, r[i], ss);
    if (tt + 2 != kProRun) continue;
    // ---- end of a 256-column run: the prologue block's partial (its waves'
    // sums, then (0 + 1) + (2 + 3)) and the run's four units into the gram
    ss = wave_sum(ss);
    if (lane == 0) red[wave] = ss;
    ss = 0.0f;
    lds_barrier();  // the run's units and sums are in LDS
    if (pm.trans) {
#pragma unroll 1
      for (int u = 0; u < kProRun; ++u) sm_pro_flush_tr(pm, units[u], run * kProRun + u, half, wq);
    }
    if (wq == 0 && lane == 0 && half * nrun + run < kSmProParts) {
      const float* rh = red + 4 * half;
      const float part = (rh[0] + rh[1]) + (rh[2] + rh[3]);
      parts[half * nrun + run] = part;
      partials[half * nrun + run] = part;
    }
    // (the lane index rebuilt for each unit keeps the fragment offsets out of
    // the registers live across the streaming part)
#pragma unroll 1
    for (int u = 0; u < kProRun; ++u) sm_gram_acc(units[u], acc, r0, c0, lane_id());
    lds_barrier();  // every wave is done with the units and the sums
  }

}

// One block of 8 waves per small matrix of the group (grid = matrices): the
// work of pm_prologue_kernel, pm_norm_kernel and the first gram of
// pm_small_core_kernel (R = s²·X Xᵀ, s = 1/‖X‖) in one pass, so the first core
// launch reads R (r_in) instead of X.
// Waves 0-3 and 4-7 run the prologue blocks of X rows 0-63 and 64-127 of each
// 256-column run side by side, thread for thread as pm_prologue_kernel runs
// them (the same elements in the same order, so the momentum, X and the
// partial sums are the same bits); the run's four 64-column units of X also
// go to LDS, where every wave adds its part of X Xᵀ with sm_gram_acc, unit by
// unit in column order as the core kernel's gram does. The partials reduce as
// in pm_norm_kernel, and R = bf16(s²·acc) goes to S[so] as sm_finish would
// round it. The caller keeps pro_tiles <= kSmProParts.
// G32 / M32: the dtypes whose runs take the vector path (fp32 or bf16 grads
// and momentum; a matrix of the other dtype loads element by element).
template <bool G32, bool M32>
__global__ __launch_bounds__(kGemmThreads, 4) void pm_small_prologue_kernel(ProArgs args, float eps, int32_t so) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(1024))) char units[kProRun][kSmUnit];
  __shared__ float parts[kSmProParts];
  __shared__ float red[kGemmThreads / 64];

  const MatDesc& d = args.descs[blockIdx.x];
  const ProMat pm = pro_mat(d);
  const int wave = wave_id(), lane = lane_id();
  const int half = wave >> 2, wq = wave & 3;
  const int r0 = (wave >> 2) * 64, c0 = (wave & 3) * 32;
  const int nrun = uni32(d.Np) / (kProTile * kProRun);
  float* const partials = (float*)uni64((int64_t)d.partials);
  const bool step = args.mode == MODE_STEP;
  const bool mvec_any = step && vec_ok(pm.mom, pm.m_dt, pm.m_ld);
  const bool gvec = vec_ok(pm.grad, pm.g_dt, pm.g_ld) && pm.g_dt == (G32 ? DT_F32 : DT_BF16);
  const bool mvec = mvec_any && pm.m_dt == (M32 ? DT_F32 : DT_BF16);

  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

  // FAST: every run is whole or padding, and the gradient and momentum fit
  // buffer resources (extents below 2 GiB)
  const int64_t gext = ((int64_t)(pm.rows - 1) * pm.g_ld + pm.cols) * (G32 ? 4 : 2);
  const int64_t mext = step ? ((int64_t)(pm.rows - 1) * pm.m_ld + pm.cols) * (M32 ? 4 : 2) : 0;
  const bool fast = gvec && (!step || mvec) && (pm.cols & 7) == 0 && gext < 0x7fff0000 && mext < 0x7fff0000;
  const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc((void*)pm.grad, (short)0, fast ? (int)gext : 0, 0x00020000);
  const __amdgpu_buffer_rsrc_t rm = __builtin_amdgcn_make_buffer_rsrc(pm.mom, (short)0, fast ? (int)mext : 0, 0x00020000);
  if (fast)
    sm_pro_tiles<true, G32, M32>(args, pm, units, parts, red, partials, acc, nrun, half, wq, gvec, mvec, mvec_any, rg, rm);
  else
    sm_pro_tiles<false, G32, M32>(args, pm, units, parts, red, partials, acc, nrun, half, wq, gvec, mvec, mvec_any, rg, rm);

  // ---- the norm: pm_norm_kernel's reduction, by waves 0-3
  float s = 0.0f;
  if (half == 0)
    for (int i = threadIdx.x; i < min(d.pro_tiles, kSmProParts); i += kThreads) s += parts[i];
  s = wave_sum(s);
  if (lane == 0) red[wave] = s;
  lds_barrier();
  const float tot = (red[0] + red[1]) + (red[2] + red[3]);
  float nrm = sqrtf(tot);
  nrm = (nrm != nrm) ? nrm : fmaxf(nrm, eps);
  const float inv = 1.0f / nrm;
  if (threadIdx.x == 0) {
    d.scales[0] = inv * inv;
    d.scales[1] = inv;
  }
  // ---- R = s²·X Xᵀ to S[so], staged in units 0 and 1
  sm_gram_store(d.S[so], SmMat{units[0], units[1]}, acc, r0, c0, lane, inv * inv);
}

// A unit of X in LDS is laid out by xt_off (pm_tiles.hpp): as in HBM
// (sm_x_off), each row's 16-byte chunks permuted by xt_swz.

// The MFMA B fragment of columns n0 .. n0+15 (n0 a multiple of 16) for k =
// k0 .. k0+7 (k0 a multiple of 8) of a unit stored as xt_off lays it out:
// lane 16g + i gets X[k0 + j][n0 + i], j = 0..7. ds_read_b64_tr_b16 gives lane
// 4a + b of each 16-lane group element b of the 8 bytes that lanes a, a+4,
// a+8 and a+12 of the group address (measured on the device), so source lane
// s of the group points at row k0 + 4h + s/4, columns n0 + 4(s%4) .. +3, and
// the two reads (h = 0, 1) return 4 consecutive k each.
__device__ __forceinline__ bf16x8 sm_xcol(const char* xs, int k0, int n0, int r16) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  s16x4 v[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
    v[h] = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (lds_s16x4*)(xs + xt_off(k0 + 4 * h + (r16 >> 2), n0 + 4 * (r16 & 3))));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 w = {v[0][0], v[0][1], v[0][2], v[0][3], v[1][0], v[1][1], v[1][2], v[1][3]};
  return __builtin_bit_cast(bf16x8, w);
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

// ---- the apply: X' = s·(a·X + S X), or the FINAL parameter step, streamed
// unit by unit.
//
// One persistent block per CU walks a contiguous range of the launch's units
// (64 columns of one matrix's X: 16 contiguous KiB in the panel layout;
// prefix: Np / 64 units per matrix), matrix after matrix. The units stream
// through an LDS ring as the core kernel's gram does: while one unit is
// multiplied, the copies of the next kRing - 2 are in flight, so the block's
// loads never stop for its products or stores. FINAL with a parameter step
// copies the unit's param block (128 x 64 param elements) into the same slot.
// S = the matrix's 128 x 128 product from the core kernel; each wave keeps
// the fragments of its 64 rows of S in registers (loaded when the walk enters
// a matrix). Wave w owns rows 64(w%2) .. +63 and columns 16(w/2) .. +15 of
// the unit's S X; a wide FINAL computes the same elements transposed (Xᵀ S,
// whose quads are param rows), a tall one steps param rows directly.
//
// The products are the grouped engine's UPDATE / FINAL element for element
// (the same MFMA over the same k order, bf16 rounding at the same points, the
// same fp32 step), so the result equals the engine's on the zero-padded matrix.
//
// GRAM (UPDATE only): the apply also forms the next iteration's R = X' X'ᵀ,
// which the core kernel would otherwise compute by reading X' back. Each unit's
// X' goes to an LDS tile in the gram ring's layout, and after the next unit's
// barrier every wave adds its two k-steps to the core's accumulators (the same
// MFMAs in the same order, so the same R). Blocks then take whole matrices
// (the gram of one matrix is one chain), and R is written to S[sc] when the
// walk leaves the matrix: S, read into registers on entry, is no longer needed
// by anyone.
template <int STAGE, int PDT>
struct SmApply {
  static constexpr bool kFinal = STAGE == ST_FINAL;
  static constexpr bool kF32 = PDT == DT_F32;
  static constexpr int kEsz = kF32 ? 4 : 2;
  static constexpr int kRing = kFinal ? (kF32 ? 3 : 4) : 8;      // slots
  static constexpr int kPBytes = kFinal ? kSm * 64 * kEsz : 16;  // a unit's param block
  static constexpr int kXCopies = kSmUnit / 1024 / kSmApplyWaves;
  static constexpr int kPCopies = kFinal ? kPBytes / 1024 / kSmApplyWaves : 0;
  static constexpr int kCopies = kXCopies + kPCopies;  // 1 KiB copies per unit and wave
  static constexpr int kStores = 4;                    // vector stores per unit and wave
  // vmcnt while waiting for the r-th unit of the block: the copies of the
  // kRing - 2 units issued after its own, and the stores of the units since
  // (copies are issued right after each unit's barrier, its stores last)
  static constexpr int kWaitMax = (kRing - 2) * kCopies + (kRing - 1) * kStores;
  static_assert(kWaitMax < 64, "vmcnt range");
  static_assert((kRing + (kFinal ? 0 : 2)) * kSmUnit + (kFinal ? kRing * kPBytes : 0) <= 160 * 1024, "LDS");
};

// Waits for the copies of the r-th unit of a block (r counted from 0).
template <class C, int R = 0>
__device__ __forceinline__ void wait_unit(int r) {
  if constexpr (R < C::kRing - 1) {
    if (r == R) {
      wait_vmcnt<(C::kRing - 2) * C::kCopies + R * C::kStores>();
      return;
    }
    wait_unit<C, R + 1>(r);
  } else {
    wait_vmcnt<C::kWaitMax>();
  }
}

// One 16-byte-per-lane LDS-DMA copy, and the buffer stores of the apply's
// param step (functions rather than builtins in the kernel's lambdas, which
// are host-device and must not name target builtins directly).
__device__ __forceinline__ void sm_copy(__amdgpu_buffer_rsrc_t rs, char* dst, int voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, to_lds(dst), 16, voff, 0, 0, 0);
}
__device__ __forceinline__ void sm_store(__amdgpu_buffer_rsrc_t rs, int off, const float (&v)[4]) {
  __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, (f32x4){v[0], v[1], v[2], v[3]}), rs, off, 0, 0);
}
__device__ __forceinline__ void sm_store_bf16(__amdgpu_buffer_rsrc_t rs, int off, const float (&v)[4]) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 pk = {(uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16),
                    (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16)};
  __builtin_amdgcn_raw_buffer_store_b64(pk, rs, off, 0, 0);
}

struct SmSlots {
  char* x[8];
  char* p[4];
};

// Position of a walk over the launch's units: matrix m, its unit lu of nu.
struct SmWalk {
  int m, lu, nu;
};

typedef const __attribute__((address_space(4))) MatDesc* SmDescPtr;
typedef const __attribute__((address_space(4))) int32_t* SmPrefixPtr;

// A unit's param block: rows of RB bytes, chunk c (16 B) of row r stored at
// chunk c ^ (r & 7) (128-byte rows) or c ^ (r & 15) (wider rows).
template <int RB>
__device__ __forceinline__ int pb_off(int r, int byte) {
  constexpr int kSwz = RB == 128 ? 7 : 15;
  return r * RB + ((((byte >> 4) ^ (r & kSwz))) << 4) + (byte & 15);
}

template <int STAGE, int PDT, bool GRAM = false>
__global__ __launch_bounds__(kSmApplyThreads, 1) void pm_small_apply_kernel(GemmArgs args) {
#pragma clang fp contract(off)
  static_assert(!GRAM || STAGE == ST_UPDATE, "the gram of X' is formed by the UPDATE apply");
  typedef SmApply<STAGE, PDT> C;
  constexpr bool kFinal = C::kFinal, kF32 = C::kF32;
  constexpr int kRing = C::kRing, kEsz = C::kEsz;
  typedef typename PickVec<kF32>::type PV;
  typedef typename PickVec<kF32>::elem PE;
  // the ring: one __shared__ array per slot, so the compiler's LDS-DMA
  // tracking sees that reads of one slot do not wait for copies into another
  SmSlots sl = {};
  __shared__ __attribute__((aligned(1024))) char x0[kSmUnit];
  __shared__ __attribute__((aligned(1024))) char x1[kSmUnit];
  __shared__ __attribute__((aligned(1024))) char x2[kSmUnit];
  sl.x[0] = x0; sl.x[1] = x1; sl.x[2] = x2;
  if constexpr (kRing >= 4) {
    __shared__ __attribute__((aligned(1024))) char x3[kSmUnit];
    sl.x[3] = x3;
  }
  if constexpr (kRing == 8) {
    __shared__ __attribute__((aligned(1024))) char x4[kSmUnit];
    __shared__ __attribute__((aligned(1024))) char x5[kSmUnit];
    __shared__ __attribute__((aligned(1024))) char x6[kSmUnit];
    __shared__ __attribute__((aligned(1024))) char x7[kSmUnit];
    sl.x[4] = x4; sl.x[5] = x5; sl.x[6] = x6; sl.x[7] = x7;
  }
  char* gt0 = nullptr;  // GRAM: X' of even / odd units, in the gram ring's layout
  char* gt1 = nullptr;
  if constexpr (GRAM) {
    __shared__ __attribute__((aligned(1024))) char gx0[kSmUnit];
    __shared__ __attribute__((aligned(1024))) char gx1[kSmUnit];
    gt0 = gx0;
    gt1 = gx1;
  }
  if constexpr (kFinal) {
    __shared__ __attribute__((aligned(1024))) char p0[C::kPBytes];
    __shared__ __attribute__((aligned(1024))) char p1[C::kPBytes];
    __shared__ __attribute__((aligned(1024))) char p2[C::kPBytes];
    sl.p[0] = p0; sl.p[1] = p1; sl.p[2] = p2;
    if constexpr (kRing >= 4) {
      __shared__ __attribute__((aligned(1024))) char p3[C::kPBytes];
      sl.p[3] = p3;
    }
  }

  const SmDescPtr descs = (SmDescPtr)args.descs;
  const SmPrefixPtr prefix = (SmPrefixPtr)args.prefix;
  int u0 = (int)((int64_t)blockIdx.x * args.total / gridDim.x);
  int u1 = (int)((int64_t)(blockIdx.x + 1) * args.total / gridDim.x);
  if constexpr (GRAM) {
    // whole matrices: the first matrix starting at or after each even split
    auto bound = [&](int u) {
      const int m = find_matrix(prefix, args.n, u);
      return prefix[m] < u ? prefix[m + 1] : prefix[m];
    };
    u0 = bound(u0);
    u1 = bound(u1);
  }
  if (u0 >= u1) return;
  const int w = wave_id(), lane = lane_id();
  const int r16 = lane & 15, g = lane >> 4;
  const int wr = w & 1, wc = w >> 1;  // rows 64·wr .. +63, columns 16·wc .. +15 of the unit
  const bool step = kFinal && args.mode == MODE_STEP;
  const float ca = args.a;
  float lr = 0.0f;
  if (step && args.lr_dev) lr = *args.lr_dev;

  SmWalk cw;  // the copy walk, kRing - 1 units ahead of the compute walk
  cw.m = find_matrix(prefix, args.n, u0);
  cw.lu = u0 - prefix[cw.m];
  cw.nu = prefix[cw.m + 1] - prefix[cw.m];
  SmWalk kw = cw;
  int cu = u0;  // the unit the copy walk issues next

  // lane offsets of this wave's X copies (copy q = kXCopies·w + h moves rows
  // 8q .. 8q+7 of the unit)
  int xvo[C::kXCopies];
#pragma unroll
  for (int h = 0; h < C::kXCopies; ++h) xvo[h] = xt_copy_src(C::kXCopies * w + h, lane);

  // Issues the copies of the copy walk's unit into slot S (zero-length
  // copies past the block's range, so every unit issues kCopies per wave),
  // then advances the walk.
  auto issue = [&](char* xs, char* ps) {
    const bool live = cu < u1;
    const int m = live ? cw.m : 0;
    auto& d = descs[m];
    const uint16_t* xb = d.X[args.cur] + sm_x_off(0, 64 * cw.lu);
    const __amdgpu_buffer_rsrc_t rx = uniform_rsrc(xb, live ? (uint32_t)kSmUnit : 0u);
#pragma unroll
    for (int h = 0; h < C::kXCopies; ++h) {
      const int q = C::kXCopies * w + h;
      sm_copy(rx, xs + q * 1024, xvo[h]);
    }
    if constexpr (kFinal) {
      // the param block: rows of RB bytes (wide: 128 param rows x 64 columns;
      // tall: 64 param rows x 128 columns), copied only for a step whose
      // param rows are 16-byte aligned (else its units take the masked path)
      const bool wide = !d.trans;
      const int64_t ld = d.p_ld;
      const bool dma = live && step && (ld * kEsz) % 16 == 0 && ((uintptr_t)d.param & 15) == 0;
      const int64_t row0 = wide ? 0 : 64 * (int64_t)cw.lu, col0 = wide ? 64 * (int64_t)cw.lu : 0;
      const PE* pb = (const PE*)d.param + row0 * ld + col0;
      // valid bytes from pb: up to the param's last element
      const int64_t valid = (((int64_t)d.rows - 1 - row0) * ld + d.cols - col0) * kEsz;
      const uint32_t nrec = !dma || valid <= 0 ? 0u : valid >= 0x7fffffff ? 0x7fffffffu : (uint32_t)valid;
      const __amdgpu_buffer_rsrc_t rp = uniform_rsrc((const uint16_t*)pb, nrec);
      const int rb = (wide ? 64 : 128) * kEsz;  // row bytes: 128, 256 or 512
      const int lpr = rb / 16;                   // lanes per row
#pragma unroll
      for (int h = 0; h < C::kPCopies; ++h) {
        const int q = C::kPCopies * w + h;
        const int r = q * (1024 / rb) + lane / lpr, c = lane % lpr;
        const int lc = c ^ (r & (rb == 128 ? 7 : 15));
        const int voff = (int)((int64_t)r * ld * kEsz) + lc * 16;
        sm_copy(rp, ps + q * 1024, voff);
      }
    }
    if (live && ++cw.lu == cw.nu) {
      ++cw.m;
      cw.lu = 0;
      if (cw.m < args.n) cw.nu = prefix[cw.m + 1] - prefix[cw.m];
    }
    ++cu;
  };

  // per-matrix state of the compute walk: this wave's S fragments (rows
  // 64wr + 16i + lane%16, k = 32s + 8g .. +7) and the scalars of the matrix
  bf16x8 sa[4][4];
  float sc = 1.0f, neg = 0.0f;
  auto enter = [&](int m) {
    auto& d = descs[m];
    const uint16_t* S = d.S[args.sl];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int s = 0; s < 4; ++s)
        sa[i][s] = *(const bf16x8*)(S + (64 * wr + 16 * i + r16) * kSm + 32 * s + 8 * g);
    sc = args.first ? d.scales[1] : 1.0f;
    if (step) neg = args.lr_dev ? -(lr * d.adj_ratio) : d.neg_lr_host;
    // the fragments complete in order behind every copy in flight: wait for
    // all of them here, so that no unit after this one waits for them again
    wait_vmcnt<0>();
  };
  const float wdf = step ? (args.lr_dev ? 1.0f - lr * args.wd : args.wdf_host) : 0.0f;

  // GRAM: this wave's part of R (the core's layout), the unit whose X' waits
  // in its LDS tile, and the matrix whose last unit that is (-1: none)
  f32x4 gacc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) gacc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const int gr0 = (w >> 2) * 64, gc0 = (w & 3) * 32;
  bool gpend = false;
  int gfin = -1;
  // adds the waiting unit (in tile gt) to R and, at a matrix's end, writes R
  // to its S[sc]
  auto gram_catch_up = [&](const char* gt) {
    if (!gpend) return;
    sm_gram_acc(gt, gacc, gr0, gc0, lane);
    if (gfin >= 0) {
      sm_gram_store(descs[gfin].S[args.sc], SmMat{gt0, gt1}, gacc, gr0, gc0, lane);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j) gacc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
      gfin = -1;
    }
    gpend = false;
  };

  // prologue: the first kRing - 1 units
#pragma unroll
  for (int s = 0; s < kRing - 1; ++s) issue(sl.x[s], sl.p[s & 3]);
  enter(kw.m);

  // one unit in slot S: wait for its copies, release slot S-1 to the copy
  // walk, multiply, store
  // GRAM: gt receives this unit's X', gp holds unit u-1's. Both are named by
  // the ring slot (kRing is even, so consecutive units alternate tiles), which
  // lets the compiler see that they are not the copies' targets; through a
  // pointer chosen at run time it would wait for every copy in flight before
  // touching them.
  auto unit = [&](char* xs, const char* ps, char* nxs, char* nps, int u, char* gt, const char* gp) {
    wait_unit<C>(u - u0);
    if constexpr (GRAM) wait_lgkmcnt<0>();  // this wave's X' tile writes of unit u-1 are done
    block_barrier();  // every wave's copies of u have landed; every wave is done with unit u-1
    // unit u-1's X' is in its tile (written before the barrier); its gram, and
    // R of a finished matrix, before this unit's copies
    if constexpr (GRAM) gram_catch_up(gp);
    if (kw.lu == kw.nu) {  // the walk enters the next matrix
      ++kw.m;
      kw.lu = 0;
      kw.nu = prefix[kw.m + 1] - prefix[kw.m];
      enter(kw.m);
    }
    issue(nxs, nps);
    auto& d = descs[kw.m];
    const int n0 = 64 * kw.lu;  // the unit's first column of X
    const bool wide = kFinal && !d.trans;
    // the MFMA fragment of X column n = n0 + lane%16 for k-step s (k = 32s +
    // 8g .. +7), read transposed from the unit by two transposed LDS reads
    auto xcol = [&](int s, int n0) { return sm_xcol(xs, 32 * s + 8 * g, n0, r16); };
    f32x4 acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
    if (wide) {
      // Xᵀ S: acc[i] = rows n = 16wc + 4g .. +3 (of Xᵀ) of column m = 64wr + 16i + lane%16
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 xa = xcol(s, 16 * wc);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = mfma_bf16(xa, sa[i][s], acc[i]);
      }
    } else {
      // S X: acc[i] = rows m = 64wr + 16i + 4g .. +3 of column n = 16wc + lane%16
#pragma unroll
      for (int s = 0; s < 4; ++s) {
        const bf16x8 xb = xcol(s, 16 * wc);
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[i] = mfma_bf16(sa[i][s], xb, acc[i]);
      }
    }
    ++kw.lu;
    // ---- the bf16 update o = bf16(s·(a·X + ...)) of quad i, in the accumulator layout
    u16x4 o[4];
    if (wide) {
      // quad i is X[m][n .. n+3] transposed: m = 64wr + 16i + lane%16, n =
      // 16wc + 4g; acc = a·x + acc as the engine's FINAL epilogue forms it
      // (with a = 0 it adds a·0 = +0, which turns a -0 accumulator into +0)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        u16x4 xq = (u16x4){0, 0, 0, 0};
        if (ca != 0.0f) xq = *(const u16x4*)(xs + xt_off(64 * wr + 16 * i + r16, 16 * wc + 4 * g));
#pragma unroll
        for (int e = 0; e < 4; ++e) o[i][e] = f2bf((ca * bf2f(xq[e]) + acc[i][e]) * sc);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // X[pr][q4 .. q4+3] from the unit, then to the quad layout
        const int pr = 64 * wr + 16 * i + 4 * g + (lane & 3), q4 = (16 * wc + r16) & ~3;
        u16x4 xq = (u16x4){0, 0, 0, 0};
        if (ca != 0.0f) xq = quad_transpose(*(const u16x4*)(xs + xt_off(pr, q4)), lane);
#pragma unroll
        for (int e = 0; e < 4; ++e) o[i][e] = f2bf((ca * bf2f(xq[e]) + acc[i][e]) * sc);
      }
    }
    if constexpr (!kFinal) {
      // X' row pr, columns n0 + q4 .. +3
      uint16_t* xn = d.X[args.cur ^ 1] + sm_x_off(0, n0);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pr = 64 * wr + 16 * i + 4 * g + (lane & 3), q4 = (16 * wc + r16) & ~3;
        const u16x4 t = quad_transpose(o[i], lane);
        *(u16x4*)(xn + pr * 64 + q4) = t;
        // GRAM: row pr, columns q4 .. q4+3 of the unit, chunk q4/8 stored at (q4/8) ^ ((pr >> 1) & 7)
        if constexpr (GRAM) *(u16x4*)(gt + pr * 128 + ((((q4 >> 3) ^ ((pr >> 1) & 7))) << 4) + (q4 & 7) * 2) = t;
      }
      if constexpr (GRAM) {
        gpend = true;
        if (kw.lu == kw.nu) gfin = kw.m;
      }
      return;
    }
    // ---- FINAL: quad i is param row pr, columns pc .. pc+3 (relative to the
    // unit's param block): wide pr = 64wr + 16i + lane%16, pc = 16wc + 4g;
    // tall pr = 16wc + lane%16, pc = 64wr + 16i + 4g
    const int64_t ld = d.p_ld;
    const int64_t row0 = wide ? 0 : n0, col0 = wide ? n0 : 0;
    const int rows = d.rows - (int)row0, cols = d.cols - (int)col0;  // of the block, from its corner
    PE* pbase = (PE*)d.param + row0 * ld + col0;
    const bool aligned = ld % 4 == 0 && ((uintptr_t)d.param % sizeof(PV)) == 0 &&
                         (!step || ((ld * kEsz) % 16 == 0 && ((uintptr_t)d.param & 15) == 0));
    const bool regular = aligned && (wide ? cols >= 64 : d.cols % 4 == 0) && (int64_t)kSm * ld * kEsz < 0x7fffffff;
    auto prow = [&](int i) { return wide ? 64 * wr + 16 * i + r16 : 16 * wc + r16; };
    auto pcol = [&](int i) { return wide ? 16 * wc + 4 * g : 64 * wr + 16 * i + 4 * g; };
    auto stepped = [&](int i, const PV& pv, float (&v)[4]) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float pe = kF32 ? (float)pv[e] : bf2f((uint16_t)pv[e]);
        v[e] = step ? pe * wdf + bf2f(o[i][e]) * neg : bf2f(o[i][e]);
      }
    };
    if (regular) {
      // param values from the block in LDS; one buffer store per quad, those
      // outside the param dropped by the buffer's range
      const int64_t valid = ((int64_t)d.rows - 1 - row0) * ld * kEsz + (int64_t)cols * kEsz;
      const uint32_t nrec = valid <= 0 ? 0u : valid >= 0x7fffffff ? 0x7fffffffu : (uint32_t)valid;
      const __amdgpu_buffer_rsrc_t rs = uniform_rsrc((const uint16_t*)pbase, nrec);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = prow(i), c = pcol(i);
        PV pv;
#pragma unroll
        for (int e = 0; e < 4; ++e) pv[e] = 0;
        if (step)
          pv = wide ? *(const PV*)(ps + pb_off<64 * kEsz>(r, c * kEsz)) : *(const PV*)(ps + pb_off<128 * kEsz>(r, c * kEsz));
        float v[4];
        stepped(i, pv, v);
        const bool in = r < rows && c < cols;
        const int off = in ? (int)((int64_t)r * ld * kEsz) + c * kEsz : -16;  // -16: past any range
        if constexpr (kF32)
          sm_store(rs, off, v);
        else
          sm_store_bf16(rs, off, v);
      }
      return;
    }
    // at the param's edges, or rows not 16-byte aligned: element by element
    // from and to the param, then every memory operation of the block is
    // waited for, so the copy waits above stay exact
    const MatDesc& dl = args.descs[kw.m];  // (generic address space for the helpers)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const Quad4 qd = quad4_at<kF32>(dl, (int)row0 + prow(i), (int)col0 + pcol(i));
      PV pv;
#pragma unroll
      for (int e = 0; e < 4; ++e) pv[e] = 0;
      if (step) pv = load_param4<kF32>(dl, qd);
      float v[4];
      stepped(i, pv, v);
      store_param4<kF32>(dl, qd, v);
    }
    wait_vmcnt<0>();
  };

  // slot S holds unit u0 + S (mod kRing); unit S releases slot S - 1 to the copy walk
  static_assert(!GRAM || kRing % 2 == 0, "X' tiles alternate with the ring slots");
#define PM_SM_UNIT(S)                                                                                 \
  unit(sl.x[S], sl.p[(S) & 3], sl.x[((S) + kRing - 1) % kRing], sl.p[(((S) + kRing - 1) % kRing) & 3], u + (S), \
       ((S) & 1) ? gt1 : gt0, ((S) & 1) ? gt0 : gt1)
  for (int u = u0; u < u1; u += kRing) {
    PM_SM_UNIT(0);
    if (u + 1 >= u1) break;
    PM_SM_UNIT(1);
    if (u + 2 >= u1) break;
    PM_SM_UNIT(2);
    if constexpr (kRing >= 4) {
      if (u + 3 >= u1) break;
      PM_SM_UNIT(3);
    }
    if constexpr (kRing == 8) {
      if (u + 4 >= u1) break;
      PM_SM_UNIT(4);
      if (u + 5 >= u1) break;
      PM_SM_UNIT(5);
      if (u + 6 >= u1) break;
      PM_SM_UNIT(6);
      if (u + 7 >= u1) break;
      PM_SM_UNIT(7);
    }
  }
#undef PM_SM_UNIT
  if constexpr (GRAM) {
    wait_lgkmcnt<0>();
    block_barrier();  // every wave's X' of the block's last unit is in its tile
    gram_catch_up(((u1 - 1 - u0) & 1) ? gt1 : gt0);
  }
  wait_vmcnt<0>();  // no copy is still writing this block's LDS when it ends
}

}  // namespace pm
