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
//   pm_small_apply_kernel  X' = s·(a·X + S X) over 128 x 256 tiles through the
//                          grouped engine's UPDATE / FINAL epilogues (X' and
//                          X'ᵀ, or the fused parameter step)
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
constexpr int kSmRing = 8;            // gram units in LDS (the whole 128 KiB)
constexpr int kSmApplyThreads = 256;  // apply blocks: four waves of 128 x 64

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

// 128 x 128 bf16 matrices in LDS: row r is 256 B, and chunk c (16 B, columns
// 8c .. 8c+7) of row r is stored at chunk c ^ (r & 15), so the 16 rows of an
// MFMA operand read of one chunk hit 16 different bank groups.
__device__ __forceinline__ int sm_off(int r, int c16) { return r * kSmRow + ((c16 ^ (r & 15)) << 4); }
__device__ __forceinline__ int sm_elem(int r, int q) { return sm_off(r, q >> 3) + (q & 7) * 2; }

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

// Finishes a 128 x 128 product of 8 waves, wave w owning rows r0 .. r0+63 and
// columns c0 .. c0+31 (acc[i][j]: rows r0 + 16i + 4(lane/16) + 0..3, column
// c0 + 16j + lane%16): C = alpha·acc + beta·D, rounded to bf16, elements on
// and above the diagonal stored at (p, q) and (q, p), so C is exactly
// symmetric. D must be symmetric (it is read through its transpose). C may be
// an operand of the product: every wave has read its operands before the
// first store.
__device__ __forceinline__ void sm_finish(char* lds, const f32x4 (&acc)[4][2], int D, int C, float alpha, float beta,
                                          int r0, int c0, int lane) {
#pragma clang fp contract(off)
  const int g = lane >> 4;
  u16x4 o[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int p0 = r0 + 16 * i + 4 * g, q = c0 + 16 * j + (lane & 15);
      u16x4 dv = (u16x4){0, 0, 0, 0};
      if (beta != 0.0f) dv = *(const u16x4*)(lds + D + sm_elem(q, p0));  // D[p0..p0+3][q]
#pragma unroll
      for (int r = 0; r < 4; ++r) o[i][j][r] = f2bf(alpha * acc[i][j][r] + beta * bf2f(dv[r]));
    }
  __syncthreads();  // every wave has read L, R and D
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int p0 = r0 + 16 * i + 4 * g, q = c0 + 16 * j + (lane & 15);
      // row p0 + lane%4, columns q&~3 .. +3 (quad_transpose), on and above the diagonal
      const u16x4 t = quad_transpose(o[i][j], lane);
      store_upper4((uint16_t*)(lds + C + sm_elem(p0 + (lane & 3), q & ~3)), t, q & ~3, p0 + (lane & 3));
      // the mirror: row q, columns p0 .. p0+3, strictly below the diagonal
      store_lower4((uint16_t*)(lds + C + sm_elem(q, p0)), o[i][j], p0, q);
    }
  __syncthreads();
}

// C = alpha·L·Rᵀ + beta·D on 128 x 128 LDS matrices (K = 128); L, R and D
// are offsets into lds. Every matrix here is symmetric, so L Rᵀ = L R.
__device__ __forceinline__ void sm_product(char* lds, int L, int R, int D, int C, float alpha, float beta,
                                           int wave, int lane) {
  const int r0 = (wave >> 2) * 64, c0 = (wave & 3) * 32;
  const int r16 = lane & 15, g = lane >> 4;
  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {  // k = 32s .. 32s+31: logical chunks 4s .. 4s+3
    bf16x8 a[4], b[2];
#pragma unroll
    for (int i = 0; i < 4; ++i) a[i] = *(const bf16x8*)(lds + L + sm_off(r0 + 16 * i + r16, 4 * s + g));
#pragma unroll
    for (int j = 0; j < 2; ++j) b[j] = *(const bf16x8*)(lds + R + sm_off(c0 + 16 * j + r16, 4 * s + g));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) acc[i][j] = mfma_bf16(a[i], b[j], acc[i][j]);
  }
  sm_finish(lds, acc, D, C, alpha, beta, r0, c0, lane);
}

// Q = Z + a·I on the first m rows (pan/optim/patch_muon.py:321-324: the
// diagonal add in bf16); the padding rows and columns stay zero.
__device__ __forceinline__ void sm_qinit(char* lds, int Z, int Q, float a, int m) {
#pragma clang fp contract(off)
  for (int i = threadIdx.x; i < kSm * kSm / 8; i += blockDim.x) {
    const int r = i >> 4, c = i & 15;  // logical chunk c of row r: columns 8c .. 8c+7
    u32x4 v = *(const u32x4*)(lds + Z + sm_off(r, c));
    const int e = r - 8 * c;  // the diagonal element's position in the chunk
    if (r < m && e >= 0 && e < 8) {
      const uint32_t w = v[e >> 1];
      const uint16_t z = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
      const uint32_t qv = f2bf(bf2f(z) + a);
      v[e >> 1] = (e & 1) ? ((w & 0xffffu) | (qv << 16)) : ((w & 0xffff0000u) | qv);
    }
    *(u32x4*)(lds + Q + sm_off(r, c)) = v;
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

// One block of 8 waves per small matrix of the group (grid = matrices).
__global__ __launch_bounds__(kGemmThreads, 1) void pm_small_core_kernel(SmallCoreArgs args) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(1024))) char lds[4 * kSmMat];
  constexpr int kR = 0, kZ = kSmMat, kQ = 2 * kSmMat, kRZ = 3 * kSmMat;
  static_assert(kSmRing * kSmUnit == 4 * kSmMat, "the gram ring fills the LDS");

  const MatDesc& d = args.descs[blockIdx.x];
  const int wave = wave_id(), lane = lane_id();
  const int r16 = lane & 15, g = lane >> 4;
  const int r0 = (wave >> 2) * 64, c0 = (wave & 3) * 32;

  // ---- R = X Xᵀ over k < Np in units of 64 k values: unit u is rows 0..127,
  // bytes 128u .. 128u+127 of each row of X (ld Np); chunk c of row r of a unit
  // is stored at chunk c ^ ((r >> 1) & 7), as in the grouped engine. A unit is
  // 16 copies of 1 KiB (8 rows); wave w issues copies 2w and 2w+1.
  const uint16_t* X = d.X[args.cur];
  const int K = d.Np, KT = K / 64;
  const __amdgpu_buffer_rsrc_t rsrc = panel_rsrc(X, (uint32_t)kSm * K * 2);
  int voff[2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {  // copy q = 2w + h: rows 8q + lane/8, stored chunk lane%8
    const int q = 2 * wave + h;
    const int sw = (4 * (q & 1) + (lane >> 4)) & 7;  // ((8q + lane/8) >> 1) & 7
    voff[h] = (lane >> 3) * K * 2 + (((lane & 7) ^ sw) << 4);
  }
  auto copy_unit = [&](int u) {
    char* dst = lds + (u % kSmRing) * kSmUnit;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int q = 2 * wave + h;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, to_lds(dst + q * 1024), 16, voff[h], q * 8 * K * 2 + u * 128, 0,
                                               0);
    }
  };
  f32x4 acc[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  for (int u = 0; u < kSmRing - 1 && u < KT; ++u) copy_unit(u);
  for (int u = 0; u < KT; ++u) {
    wait_units(min(kSmRing - 2, KT - 1 - u));  // this wave's copies of unit u have landed
    __syncthreads();  // every wave's copies of u have landed; every wave is done with unit u-1
    if (u + kSmRing - 1 < KT) copy_unit(u + kSmRing - 1);  // into unit u-1's slot
    const char* src = lds + (u % kSmRing) * kSmUnit;
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
  // R = s²·X Xᵀ (s² = 1/‖X‖² on the unscaled first X): sm_finish's first
  // barrier also ends every wave's reads of the ring, which R overwrites
  sm_finish(lds, acc, kR, kR, args.first ? d.scales[0] : 1.0f, 0.0f, r0, c0, lane);

  // ---- the M x M part of the iteration
  int out = kZ;
  if (args.steps == 0) {
    const float* k = args.coeffs + 3 * args.it0;
    sm_product(lds, kR, kR, kR, kZ, k[2], k[1], wave, lane);  // B = c R R + b R
  } else {
    for (int i = 0; i < args.steps; ++i) {
      const float* k = args.coeffs + 3 * (args.it0 + i);
      const float a = k[0], b = k[1], c = k[2];
      sm_product(lds, kR, kR, kR, kZ, c, b, wave, lane);  // Z = c R R + b R
      if (i == 0)
        sm_qinit(lds, kZ, kQ, a, d.M);  // Q = a I + Z
      else
        sm_product(lds, kQ, kZ, kQ, kQ, 1.0f, a, wave, lane);  // Q = Q Z + a Q
      if (i + 1 < args.steps) {
        sm_product(lds, kR, kZ, kR, kRZ, 1.0f, a, wave, lane);   // RZ = R Z + a R
        sm_product(lds, kZ, kRZ, kRZ, kR, 1.0f, a, wave, lane);  // R = Z RZ + a RZ
      }
    }
    out = kQ;
  }

  // ---- S (row-major 128 x 128) to the workspace
  uint16_t* S = d.S[args.so];
  for (int i = threadIdx.x; i < kSm * kSm / 8; i += blockDim.x) {
    const int r = i >> 4, c = i & 15;
    *(u32x4*)(S + r * kSm + 8 * c) = *(const u32x4*)(lds + out + sm_off(r, c));
  }
}

// X' = s·(a·X + S X) for one 128 x 256 tile of a small matrix per block
// (prefix: Np / 256 tiles per matrix). A wide FINAL computes the transposed
// tile X'ᵀ = Xᵀ Sᵀ (256 x 128; S is symmetric), whose quads are param rows, as
// the grouped engine's FINAL does; every other tile is S X. K = 128 is loaded
// whole into LDS; the epilogue is the grouped engine's, each wave standing in
// for one wave of its 2 x 4 grid of 128 x 64 wave tiles.
template <int STAGE, int PDT>
__global__ __launch_bounds__(kSmApplyThreads, 1) void pm_small_apply_kernel(GemmArgs args) {
  __shared__ __attribute__((aligned(1024))) char lds[3 * kSm * kSmRow];  // 96 KiB: 128 + 256 operand rows
  const int t = blockIdx.x;
  const int m = find_matrix(args.prefix, args.n, t);
  const MatDesc& d = args.descs[m];
  const int lt = t - args.prefix[m];
  const int w = wave_id(), lane = lane_id();
  const bool wide_final = STAGE == ST_FINAL && !d.trans;
  // rows of S (128) and rows 256·lt .. 256·lt+255 of Xᵀ (ld 128): 256 B each
  const uint16_t* S = d.S[args.sl];
  const uint16_t* XT = d.XT[args.cur] + (int64_t)lt * kTile * kSm;
  const uint16_t* Lsrc = wide_final ? XT : S;
  const uint16_t* Rsrc = wide_final ? S : XT;
  const int nL = wide_final ? kTile : kSm, nR = wide_final ? kSm : kTile;
  char* lbuf = lds;
  char* rbuf = lds + nL * kSmRow;
  {
    // copy q moves rows 4q .. 4q+3 (1 KiB): lane l lands at row 4q + l/16,
    // stored chunk l%16, so it loads logical chunk (l%16) ^ ((4q + l/16) & 15)
    const __amdgpu_buffer_rsrc_t rl = panel_rsrc(Lsrc, (uint32_t)nL * kSmRow);
    const __amdgpu_buffer_rsrc_t rr = panel_rsrc(Rsrc, (uint32_t)nR * kSmRow);
    const int row = lane >> 4;
    for (int q = w; q < nL / 4; q += kSmApplyThreads / 64) {
      const int voff = row * kSmRow + (((lane & 15) ^ ((4 * q + row) & 15)) << 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, to_lds(lbuf + q * 1024), 16, voff, q * 4 * kSmRow, 0, 0);
    }
    for (int q = w; q < nR / 4; q += kSmApplyThreads / 64) {
      const int voff = row * kSmRow + (((lane & 15) ^ ((4 * q + row) & 15)) << 4);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, to_lds(rbuf + q * 1024), 16, voff, q * 4 * kSmRow, 0, 0);
    }
  }
  wait_vmcnt<0>();
  __syncthreads();
  // waves in a 1 x 4 grid (S X, 128 x 256) or 2 x 2 (wide FINAL, 256 x 128);
  // vw is the wave's index in the engine's 2 x 4 grid
  const int vw = wide_final ? (w >> 1) * 4 + (w & 1) : w;
  const int ar0 = (vw >> 2) * kWaveRows, bc0 = (vw & 3) * kWaveCols;
  const int r16 = lane & 15, g = lane >> 4;
  f32x4 acc[kMi][kNi];
#pragma unroll
  for (int i = 0; i < kMi; ++i)
#pragma unroll
    for (int j = 0; j < kNi; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    bf16x8 b[kNi];
#pragma unroll
    for (int j = 0; j < kNi; ++j) b[j] = *(const bf16x8*)(rbuf + sm_off(bc0 + 16 * j + r16, 4 * s + g));
#pragma unroll
    for (int i = 0; i < kMi; ++i) {
      const bf16x8 a = *(const bf16x8*)(lbuf + sm_off(ar0 + 16 * i + r16, 4 * s + g));
#pragma unroll
      for (int j = 0; j < kNi; ++j) acc[i][j] = mfma_bf16(a, b[j], acc[i][j]);
    }
  }
  TileJob job{};
  job.ti = wide_final ? lt : 0;
  job.tj = wide_final ? 0 : lt;
  gemm_epilogue<STAGE, PDT>(args, d, job, acc, vw);
}

}  // namespace pm
