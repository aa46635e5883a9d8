// Kernels of libpanmuon. Included once, by panmuon.hip.
#pragma once

#include "pm_device.hpp"
#include "pm_tiles.hpp"

namespace pm {

// ============================================================ prologue
//
// 64x64 tiles of the parameter, kProRun consecutive ones per block (tiles
// cover the padded extent; elements outside the parameter become zeros of X).
//   MODE_STEP: buf <- mu*buf + (1-mu)*g;  u <- (1-mu)*g + mu*buf  (nesterov)
//              (pan/optim/muon_triton.py:44-48; fp32 math)
//   MODE_NS:   u <- in
// X gets bf16(u), or bf16(uᵀ) for a tall param (torch casts to bf16 before
// NS, torch/optim/_muon.py:55, and transposes, :56-57), in the layout
// ProArgs.layout names
// and partials[tile] = Σ bf16(u)², the tile's share of ‖X‖² (norm over the
// bf16 tensor, torch/optim/_muon.py:59).
// Each thread moves two runs of 8 consecutive elements of a row: 16-byte
// loads and stores where the row is in range and the caller's strides and
// bases allow, element by element otherwise. A transposed X goes through an
// LDS tile.
constexpr int kProPitch = kProTile + 8;  // LDS row pitch (elements), keeps 16-byte rows aligned
constexpr int kProRun = 4;  // tiles per prologue block, along a tile row (1 and 2 measured slower)
static_assert(kTile % (kProTile * kProRun) == 0, "runs tile the padded long side");

__device__ __forceinline__ void load8(const void* base, int32_t dt, int64_t off, bool vec, bool in_row, int valid,
                                      float (&v)[8]) {
  if (in_row && vec && valid >= 8) {
    if (dt == DT_F32) {
      const f32x4 a = *(const f32x4*)((const float*)base + off);
      const f32x4 b = *(const f32x4*)((const float*)base + off + 4);
#pragma unroll
      for (int e = 0; e < 4; ++e) { v[e] = a[e]; v[4 + e] = b[e]; }
    } else {
      const u32x4 a = *(const u32x4*)((const uint16_t*)base + off);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[2 * e] = bf2f((uint16_t)(a[e] & 0xffff));
        v[2 * e + 1] = bf2f((uint16_t)(a[e] >> 16));
      }
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (in_row && e < valid) ? load_elem(base, dt, off + e) : 0.0f;
}

__device__ __forceinline__ void store8(void* base, int32_t dt, int64_t off, bool vec, int valid, const float (&v)[8]) {
  if (vec && valid >= 8) {
    if (dt == DT_F32) {
      *(f32x4*)((float*)base + off) = (f32x4){v[0], v[1], v[2], v[3]};
      *(f32x4*)((float*)base + off + 4) = (f32x4){v[4], v[5], v[6], v[7]};
    } else {
      u32x4 a;
#pragma unroll
      for (int e = 0; e < 4; ++e) a[e] = (uint32_t)f2bf(v[2 * e]) | ((uint32_t)f2bf(v[2 * e + 1]) << 16);
      *(u32x4*)((uint16_t*)base + off) = a;
    }
    return;
  }
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (e < valid) store_elem(base, dt, off + e, v[e]);
}

__device__ __forceinline__ bool vec_ok(const void* base, int32_t dt, int64_t ld) {
  return (ld % 8 == 0) && ((uintptr_t)base % 16 == 0) && (dt == DT_F32 || dt == DT_BF16);
}

// A barrier that orders LDS accesses only: global loads and stores stay in
// flight across it (__syncthreads would wait for every one of them).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0), vmcnt and expcnt unconstrained (gfx9 encoding)
  __builtin_amdgcn_s_barrier();
}

// One block per kProRun consecutive 64x64 tiles of a tile row of X (tiles
// cover the padded extent; elements outside the parameter become zeros of X).
__global__ __launch_bounds__(kThreads) void pm_prologue_kernel(ProArgs args) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) uint16_t tile[kProTile][kProPitch];
  __shared__ float red[kThreads / 64];

  const int t = blockIdx.x;
  const int mi = find_matrix(args.prefix, args.n, t);
  const MatDesc& d = args.descs[mi];
  const int lt = t - args.prefix[mi];
  const int nrun = d.Np / (kProTile * kProRun);  // runs per tile row
  const int ti = lt / nrun, tj0 = (lt - ti * nrun) * kProRun;  // first tile in X coordinates
  const float mu = args.mu, omu = 1.0f - args.mu;
  const bool step = args.mode == MODE_STEP;
  const bool gvec = vec_ok(d.grad, d.g_dt, d.g_ld);
  const bool mvec = step && vec_ok(d.mom, d.m_dt, d.m_ld);
  // X = u is written in the param's orientation (dst_a); X = uᵀ (a tall
  // param) goes through the LDS tile (dst_b). Only X is kept: the GEMM
  // engine reads it transposed where it needs Xᵀ.
  uint16_t* dst_a = d.trans ? nullptr : d.X[0];
  const int64_t ld_a = d.Np;
  uint16_t* dst_b = d.trans ? d.X[0] : nullptr;
  const int64_t ld_b = d.Np;
  const int layout = args.layout;
  auto x_off = [&](int r, int c, int64_t ld) {
    return layout == XL_SMALL ? sm_x_off(r, c) : ws_off(r, c, ld, layout == XL_PANEL);
  };

  float ss = 0.0f;
  const int cg = (threadIdx.x & 7) * 8;  // first column of this thread's runs
  for (int tt = 0; tt < kProRun; ++tt) {
    const int tj = tj0 + tt;
    const int pr0 = d.trans ? tj * kProTile : ti * kProTile;  // param-layout origin
    const int pc0 = d.trans ? ti * kProTile : tj * kProTile;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int r = (threadIdx.x >> 3) + 32 * h;
      const int pr = pr0 + r, pc = pc0 + cg;
      const bool in_row = pr < d.rows;
      const int valid = d.cols - pc;  // elements of the run inside the parameter
      float u[8];
      float g[8];
      load8(d.grad, d.g_dt, (int64_t)pr * d.g_ld + pc, gvec, in_row, valid, g);
      if (step) {
        float m[8];
        const int64_t mo = (int64_t)pr * d.m_ld + pc;
        load8(d.mom, d.m_dt, mo, mvec, in_row, valid, m);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float nm = mu * m[e] + omu * g[e];
          m[e] = nm;
          u[e] = args.nesterov ? omu * g[e] + mu * nm : nm;
        }
        if (in_row) store8(d.mom, d.m_dt, mo, mvec, valid, m);
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
      if (dst_b) *(u32x4*)&tile[r][cg] = packed;
      if (dst_a) *(u32x4*)(dst_a + x_off(pr, pc, ld_a)) = packed;
    }
    if (dst_b) {
      lds_barrier();
      // other orientation: thread -> column c of the tile, rows 16*(t%4) .. +15
      const int c = threadIdx.x >> 2, rb = (threadIdx.x & 3) * 16;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u32x4 packed;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int r = rb + 8 * h + 2 * e;
          packed[e] = (uint32_t)tile[r][c] | ((uint32_t)tile[r + 1][c] << 16);
        }
        *(u32x4*)(dst_b + x_off(pc0 + c, pr0 + rb + 8 * h, ld_b)) = packed;
      }
      lds_barrier();  // the tile is read before the next run overwrites it
    }
  }

  ss = wave_sum(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) d.partials[lt] = (red[0] + red[1]) + (red[2] + red[3]);
}

// ============================================================ norm
// One block per matrix; fixed-order reduction of the prologue partials.
// torch: X.div_(X.norm().clamp(min=eps)) (torch/optim/_muon.py:59); a NaN
// norm stays NaN (clamp propagates NaN).
__global__ __launch_bounds__(kThreads) void pm_norm_kernel(const MatDesc* descs, float eps) {
  __shared__ float red[kThreads / 64];
  const MatDesc& d = descs[blockIdx.x];
  float s = 0.0f;
  for (int i = threadIdx.x; i < d.pro_tiles; i += kThreads) s += d.partials[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) {
    const float tot = (red[0] + red[1]) + (red[2] + red[3]);
    float nrm = sqrtf(tot);
    nrm = (nrm != nrm) ? nrm : fmaxf(nrm, eps);
    const float inv = 1.0f / nrm;
    d.scales[0] = inv * inv;
    d.scales[1] = inv;
  }
}

// ============================================================ GEMM engine
//
// C[256x256] = L[256xK] · R[256xK]ᵀ, both operands K-contiguous bf16.
// 8 waves (two per SIMD, so one issues MFMAs while the other waits) in a
// 2 x 4 grid, each owning a 128x64 sub-tile as 8 x 4 tiles of
// v_mfma_f32_16x16x32_bf16 (128 fp32 accumulators per lane, held in AGPRs).
//
// K advances in units of 64: a unit is 256 rows x 128 B of each operand
// (32 KiB each), so every row an LDS-DMA load fetches is one whole 128-byte
// cache line. Two units fit in LDS (128 KiB). Global -> LDS copies are
// buffer_load_dwordx4 ... lds: lane l of a load writes 16 B at the
// instruction's LDS base + 16*l, so one instruction fills 8 rows and no VGPRs
// or ds_write instructions are spent on staging. In the panel layout of the
// workspace (ws_off) a unit is one contiguous 32 KiB block, so each copy reads
// 1 KiB of consecutive memory (measured 3-20% faster per stage than 8 rows
// strided by the row pitch, most for long rows). Row chunk c (16 B) is stored
// at chunk c ^ ((row >> 1) & 7): a ds_read_b128 phase (16 lanes, 16
// consecutive rows, one logical chunk) then touches 16 distinct 16-byte bank
// groups of the 64-bank LDS (measured conflict-free).
//
// A unit is 16 MFMA positions of 4 MFMAs (two k-steps of 32). Each operand
// has its own double buffer and its own barrier:
//   B: unit u's k-step-1 fragments are read at positions 0..7, the next
//      unit's k-step-0 fragments at 12..15; the barrier at 12 certifies that
//      every wave's copy of B(u+1) has landed and that no wave still reads
//      B(u), whose buffer then receives B(u+2).
//   A: fragments are read two positions ahead, so the next unit's first two
//      are read at 14, 15; the barrier at 14 (after the read of A(u) at
//      position 13 has returned) certifies A(u+1) landed and A(u) consumed.
// Only waves 0..3 (one per SIMD) issue copies: 8 A and 8 B per unit for unit
// u+2, two per position, B at positions 12..15 and A at 14, 15 of unit u and
// 0, 1 of unit u+1. A copy whose issue the memory pipeline holds back stalls
// only its own wave; the other wave on that SIMD (waves 4..7 never copy)
// keeps the MFMA pipe fed (measured 1.5-2.6% faster than all eight waves
// issuing four copies each). Each copier waits for exactly the loads the
// next barrier needs (vmcnt counts them in issue order).
//
// MFMAs are issued from inline asm with the accumulator tied in place (the
// compiler's own MFMA selection moves accumulators between registers across
// the unrolled loop). An MFMA reads its sources when it executes, after
// issue, so each fragment is kept allocated until 8 more MFMAs (two
// positions) have issued; that is what the hold() calls do. No load can then be assigned a register
// an earlier queued MFMA still has to read.
constexpr int kBK = 64;                        // K depth of one unit
constexpr int kOpBytes = kTile * kBK * 2;      // 32 KiB: one operand of one unit
constexpr int kWaveRows = 128, kWaveCols = 64;
constexpr int kMi = kWaveRows / 16, kNi = kWaveCols / 16;  // 16x16 MFMA tiles per wave
constexpr int kQuads = kMi * kNi;              // accumulator quads per lane
static_assert(kGemmThreads == 512, "the GEMM engine is written for eight waves");

__device__ __forceinline__ __amdgpu_buffer_rsrc_t panel_rsrc(const uint16_t* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ lds_ptr_t to_lds(char* p) {
  return (lds_ptr_t)(__attribute__((address_space(3))) char*)p;
}

// s_waitcnt vmcnt(n) / lgkmcnt(n), leaving the other counters unconstrained
// (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  __builtin_amdgcn_s_waitcnt(15 | (7 << 4) | (N << 8) | (3 << 14));
}

// Block-wide barrier without the release fence of __syncthreads(), which
// would drain every in-flight LDS DMA. Callers wait for exactly the loads they
// need first; the "memory" clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void mfma16(f32x4& acc, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void hold(const bf16x8& v) { asm volatile("" ::"v"(v)); }
__device__ __forceinline__ void hold4(const bf16x8 (&v)[4]) {
  asm volatile("" ::"v"(v[0]), "v"(v[1]), "v"(v[2]), "v"(v[3]));
}

__device__ __forceinline__ void pin8(f32x4 (&x)[kNi], f32x4 (&y)[kNi]) {
  asm volatile("" : "+a"(x[0]), "+a"(x[1]), "+a"(x[2]), "+a"(x[3]), "+a"(y[0]), "+a"(y[1]), "+a"(y[2]), "+a"(y[3]));
}

// One __shared__ array per buffer, so the compiler's LDS-DMA tracking sees
// that reads of one buffer do not depend on copies into the others.
struct Ring {
  char* a[2];
  char* b[2];
};

// An operand is read either by rows (K-contiguous panels: X for GRAM, the
// Mp x Mp work matrices) or transposed (TR below): the right operand of
// C = S·X is X itself, whose rows run along N, not K. A transposed operand's unit is 64 rows (k) x 256 columns, kept in LDS
// as 4 column blocks of 64 x 64 (8 KiB, 128-byte rows); its 32-byte chunk c
// (16 columns) of row k is stored at chunk c ^ tsw(k). Its copy q (0..31) is
// rows 8(q%8) .. +7 of column block q/8: in the panel layout of X (ws_off) 1 KiB
// of consecutive memory, as for a row-read operand.
__device__ __forceinline__ int tsw(int k) { return ((k >> 1) & 1) | (((k >> 3) & 1) << 1); }

struct Engine {
  __amdgpu_buffer_rsrc_t rl, rr;
  int vl_off[2], vr_off[2];  // DMA lane offsets for even / odd loads
  int frag[2];               // fragment lane offset for k-step 0 / 1 (row-read operands)
  int toff[4];               // fragment lane offsets of column chunk 0..3 (transposed right operand)
  int aofs, bofs;            // this wave's first row (bytes) in an A / B unit
  int ql, qr;                // bytes from one 8-row copy of a unit to the next
  int ul, ur;                // bytes from one unit of a panel to the next
  int q0;
  bool copier;               // waves 0..3 issue every copy of the tile
  // transposed right operand: its column blocks in the first 256-row panel of
  // X, and the bytes from one 256-row panel to the next (the buffer resource
  // is rebased per panel so offsets stay small for any extent)
  const uint16_t* tbase;
  int64_t tpanel;
};


__device__ __forceinline__ void dma_a(const Engine& e, char* dst, int unit, int i) {
  const int q = e.q0 + i;
  __builtin_amdgcn_raw_ptr_buffer_load_lds(e.rl, to_lds(dst + q * 1024), 16, e.vl_off[q & 1],
                                           q * e.ql + unit * e.ul, 0, 0);
}
template <bool TR>
__device__ __forceinline__ void dma_b(const Engine& e, char* dst, int unit, int i) {
  const int q = e.q0 + i;
  if (TR) {
    const __amdgpu_buffer_rsrc_t rs = panel_rsrc(
        (const uint16_t*)((const char*)e.tbase + (int64_t)(unit >> 2) * e.tpanel), 4 * kOpBytes);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, to_lds(dst + q * 1024), 16, e.vr_off[q & 1],
                                             (q >> 3) * kOpBytes + (unit & 3) * 8192 + (q & 7) * 1024, 0, 0);
  } else {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(e.rr, to_lds(dst + q * 1024), 16, e.vr_off[q & 1],
                                             q * e.qr + unit * e.ur, 0, 0);
  }
}

// The MFMA fragment (16 rows or columns x 32 k) of a transposed operand: lane
// 16g + i gets the operand's element (k0 + j, column c0 + i), j = 0..7, where
// p addresses this lane's source of the first read. ds_read_b64_tr_b16 gives
// lane 4a + b of each 16-lane group element b of the 8 bytes that lanes a,
// a+4, a+8 and a+12 of the group address, so source lane s points at row
// k0 + 4h + s/4, columns c0 + 4(s%4) .. +3, and the two reads (h = 0, 1, four
// rows = 512 bytes apart) return 4 consecutive k each.
__device__ __forceinline__ bf16x8 tr_frag(const char* p) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 v0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
  const s16x4 v1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + 512));
  typedef short s16x8 __attribute__((ext_vector_type(8)));
  const s16x8 w = {v0[0], v0[1], v0[2], v0[3], v1[0], v1[1], v1[2], v1[3]};
  return __builtin_bit_cast(bf16x8, w);
}

// Fragment j (16-row block of this wave's rows) of k-step s of the left
// operand of unit buffer `buf`, and fragment j (16-column block) of the right.
__device__ __forceinline__ bf16x8 frag_a(const Engine& e, const char* buf, int j, int s) {
  return *(const bf16x8*)(buf + e.aofs + j * 2048 + e.frag[s]);
}
template <bool TR>
__device__ __forceinline__ bf16x8 frag_b(const Engine& e, const char* buf, int j, int s) {
  if (TR) return tr_frag(buf + e.bofs + s * 4096 + e.toff[j]);
  return *(const bf16x8*)(buf + e.bofs + j * 2048 + e.frag[s]);
}

// Unit u in buffer S = u % 2; REL = units after this one (2 or more: steady).
// TR: the right operand is read transposed (two LDS reads a fragment instead
// of one).
template <int S, int REL, bool TR>
__device__ __forceinline__ void gemm_unit(const Ring& ring, int u, const Engine& e, f32x4 (&acc)[kMi][kNi],
                                          bf16x8 (&bf)[2][kNi], bf16x8 (&af)[8]) {
  const char* ca = ring.a[S];
  const char* na = ring.a[S ^ 1];
  const char* cb = ring.b[S];
  const char* nb = ring.b[S ^ 1];
  bf16x8 prev1[kNi];  // previous unit's k-step-1 fragments, still read by queued MFMAs
#pragma unroll
  for (int i = 0; i < kNi; ++i) prev1[i] = bf[1][i];
#pragma unroll
  for (int p = 0; p < 16; ++p) {
    const int s = p / 8, mi = p % 8;
    if (REL >= 1 && p == 12) {
      wait_vmcnt<6>();  // B(u+1) #7 (position 15 of u-1) was followed by A(u+1) #2..#7
      block_barrier();
    }
    if (REL >= 1 && p == 14) {
      if (REL >= 2) wait_vmcnt<4>(); else wait_vmcnt<0>();  // A(u+1) #7 (position 1) was followed by B(u+2) #0..#3
      // the read of A(u) at position 13 has returned: only the B read issued
      // after it (one instruction, two if transposed) may be pending
      wait_lgkmcnt<TR ? 2 : 1>();
      block_barrier();
    }
    if (p + 2 < 16) {
      const int q = p + 2;
      af[q % 8] = frag_a(e, ca, q % 8, q / 8);
      if (p == 13) __builtin_amdgcn_sched_barrier(0);  // the last read of A(u) stays ahead of the B read
    } else if (REL >= 1) {
      const int q = p + 2 - 16;
      af[q % 8] = frag_a(e, na, q, 0);
    }
    // k-step 1's B fragments (used from position 8): one a position, two
    // positions apart when each takes two reads
    if (TR) {
      if (p % 2 == 0 && p < 2 * kNi) bf[1][p / 2] = frag_b<TR>(e, cb, p / 2, 1);
    } else if (p < kNi) {
      bf[1][p] = frag_b<TR>(e, cb, p, 1);
    }
    if (REL >= 1 && p >= 12) bf[0][p - 12] = frag_b<TR>(e, nb, p - 12, 0);
    // odd positions walk the B fragments backwards, so consecutive MFMAs
    // never change both operands (the B fragment is kept across a position
    // change)
#pragma unroll
    for (int i = 0; i < kNi; ++i) {
      const int ni = (p & 1) ? kNi - 1 - i : i;
      mfma16(acc[mi][ni], af[p % 8], bf[s][ni]);
    }
    if (e.copier) {  // waves 0..3: two copies per position
      if (REL >= 1 && p < 2) {
        dma_a(e, ring.a[S ^ 1], u + 1, 4 + 2 * p);
        dma_a(e, ring.a[S ^ 1], u + 1, 5 + 2 * p);
      }
      if (REL >= 2 && p >= 12) {
        dma_b<TR>(e, ring.b[S], u + 2, 2 * (p - 12));
        dma_b<TR>(e, ring.b[S], u + 2, 2 * (p - 12) + 1);
      }
      if (REL >= 2 && p >= 14) {
        dma_a(e, ring.a[S], u + 2, 2 * (p - 14));
        dma_a(e, ring.a[S], u + 2, 2 * (p - 14) + 1);
      }
    }
    // a fragment stays allocated through two positions (8 MFMAs) after its last use
    hold(af[p % 8]);
    hold(af[(p + 7) % 8]);
    hold(af[(p + 6) % 8]);
    if (p <= 2) hold4(prev1);
    if (p >= 8 && p <= 10) hold4(bf[0]);
    __builtin_amdgcn_sched_barrier(0);
  }
}

// Lane index rebuilt from the exec mask inside an asm block with no inputs,
// so neither it nor the per-lane offsets derived from it can be hoisted out of
// the persistent tile loop (where they would stay live through the K loop);
// the wave index lives in an SGPR.
__device__ __forceinline__ int lane_id() {
  int l;
  asm volatile("v_mbcnt_lo_u32_b32 %0, -1, 0\n\tv_mbcnt_hi_u32_b32 %0, -1, %0" : "=v"(l));
  return l;
}
__device__ __forceinline__ int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// Operands and tile of one work item of a stage (decode_tile).
struct TileJob {
  const uint16_t* L;
  const uint16_t* R;
  int ldl, ldr, K;   // K: the item's share of the contraction (a chunk's, when split)
  int ti, tj;
  bool tl, tr;  // L / R in the panel layout
  bool rtr;     // R read transposed (X itself; needs the panel layout)
  int u0;       // first unit (64 k) of the item's K range: a K-split chunk's offset
};

// Operand panels and per-lane addressing of tile (ti, tj). A row-read panel is
// row-major (ld elements a row) or in the panel layout of ws_off (tiled),
// where a unit's 256 rows of 128 bytes are contiguous. A transposed right
// operand is X (panel layout, ld = Np): for tile column tj its columns
// 256tj .. 256tj+255 are the 64-column units 4tj .. 4tj+3 of every 256-row
// panel.
template <bool TR>
__device__ __forceinline__ Engine make_engine(const TileJob& j, int w) {
  const int lane = lane_id();
  Engine e;
  const int ldl = j.ldl, ldr = j.ldr;
  const bool tl = j.tl, tr = j.tr;
  // a K-split chunk starts u0 units into the panels: its bases move there
  // (a unit is 32 KiB of a panel-layout panel, 128 bytes of a row-major row)
  const uint32_t lskip = (uint32_t)j.u0 * (tl ? kOpBytes : kBK * 2);
  const uint32_t rskip = (uint32_t)j.u0 * (tr ? kOpBytes : kBK * 2);
  const uint16_t* Lp = j.L + (int64_t)j.ti * kTile * j.ldl + lskip / 2;
  const uint16_t* Rp = j.R + (int64_t)j.tj * kTile * j.ldr + rskip / 2;
  e.rl = panel_rsrc(Lp, (uint32_t)kTile * ldl * 2 - lskip);
  e.rr = panel_rsrc(Rp, (uint32_t)kTile * ldr * 2 - rskip);
  const int rowl = tl ? kBK * 2 : ldl * 2, rowr = tr ? kBK * 2 : ldr * 2;  // bytes from row to row
  e.ql = 8 * rowl;
  e.qr = 8 * rowr;
  e.ul = tl ? kOpBytes : kBK * 2;
  e.ur = tr ? kOpBytes : kBK * 2;
  // Row-read copy q (0..31) covers rows 8q..8q+7 of a unit. Lane l fills row
  // 8q + l/8 at stored chunk l%8, i.e. logical chunk (l%8) ^ ((row >> 1) & 7).
  // Transposed copy q: lane l fills row k = 8(q%8) + l/8 of column block q/8 at
  // stored 32-byte chunk (l%8)/2, i.e. logical chunk ((l%8)/2) ^ tsw(k), half
  // l%2, and tsw(k) = ((l >> 4) & 1) | 2·(q % 2).
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int sw = (4 * par + (lane >> 4)) & 7;
    const int row_off = (lane >> 3) * 128;
    const int tsw_l = ((lane >> 4) & 1) | (par << 1);
    const int t_off = row_off + ((((((lane & 7) >> 1) ^ tsw_l) << 1) | (lane & 1)) << 4);
    e.vl_off[par] = (lane >> 3) * rowl + (((lane & 7) ^ sw) << 4);
    e.vr_off[par] = TR ? t_off : (lane >> 3) * rowr + (((lane & 7) ^ sw) << 4);
  }
  e.q0 = w * 8;
  e.copier = w < 4;
  // fragment of k-step s: row l%16 of a 16-row block, logical chunk 4s + l/16
  const int r16 = lane & 15, g = lane >> 4;
#pragma unroll
  for (int s = 0; s < 2; ++s) e.frag[s] = r16 * 128 + (((4 * s + g) ^ ((r16 >> 1) & 7)) << 4);
  // transposed fragment reads: source lane r16 of group g reads row
  // 8g + r16/4 (+ 32 per k-step, + 4 for the second read) at columns
  // 16c + 4(r16%4) of its block: chunk c ^ tsw(row), and tsw(row) =
  // ((r16 >> 3) & 1) | 2·(g & 1) for every such row
  const int tsw_f = ((r16 >> 3) & 1) | ((g & 1) << 1);
#pragma unroll
  for (int c = 0; c < 4; ++c) e.toff[c] = (8 * g + (r16 >> 2)) * 128 + ((c ^ tsw_f) << 5) + 8 * (r16 & 3);
  e.aofs = (w >> 2) * kWaveRows * 128;
  e.bofs = TR ? (w & 3) * 8192 : (w & 3) * kWaveCols * 128;
  e.tbase = nullptr;
  e.tpanel = 0;
  if (TR) {
    // X read transposed: unit u is 64 rows of X, so u0 (a multiple of 4)
    // skips u0/4 whole 256-row panels
    e.tpanel = (int64_t)ldr * kTile * 2;
    e.tbase = j.R + (int64_t)j.tj * 4 * (kOpBytes / 2) + (int64_t)(j.u0 >> 2) * (e.tpanel / 2);
  }
  return e;
}

// Copies of unit 0, all of unit 1's B and the first 4 of its A (what a unit -1
// would issue at its positions 12..15); unit 0's positions 0, 1 issue the
// other four. Copier waves only. May be
// issued while the previous tile's epilogue runs: it touches only the LDS
// ring, which the caller has certified free with a barrier.
template <bool TR>
__device__ __forceinline__ void gemm_prefetch(const Engine& e, const Ring& ring) {
  if (!e.copier) return;
#pragma unroll
  for (int i = 0; i < 8; ++i) dma_b<TR>(e, ring.b[0], 0, i);
#pragma unroll
  for (int i = 0; i < 8; ++i) dma_a(e, ring.a[0], 0, i);
#pragma unroll
  for (int i = 0; i < 8; ++i) dma_b<TR>(e, ring.b[1], 1, i);
#pragma unroll
  for (int i = 0; i < 4; ++i) dma_a(e, ring.a[1], 1, i);
}

// Full K loop of one tile whose first copies gemm_prefetch issued. K must be a
// multiple of 256 (padded extents), so the unit count KT = K / 64 is a
// multiple of 4. Every wave waits for all its memory operations first (the
// prefetch, and the previous tile's epilogue stores, which vmcnt also counts),
// so the in-loop counts see only this tile's copies.
template <bool TR>
__device__ __forceinline__ void gemm_run(const Engine& e, int K, const Ring& ring, f32x4 (&acc)[kMi][kNi]) {
#pragma unroll
  for (int i = 0; i < kMi; ++i)
#pragma unroll
    for (int j = 0; j < kNi; ++j) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};
  bf16x8 bf[2][kNi];
  bf16x8 af[8];

  wait_vmcnt<0>();
  wait_lgkmcnt<0>();  // also publishes LDS writes made before this barrier
  block_barrier();
#pragma unroll
  for (int i = 0; i < kNi; ++i) bf[0][i] = frag_b<TR>(e, ring.b[0], i, 0);
  af[0] = frag_a(e, ring.a[0], 0, 0);
  af[1] = frag_a(e, ring.a[0], 1, 0);
  __builtin_amdgcn_sched_barrier(0);

  // KT >= 4, so the steady loop runs at least once; a do-while keeps a single
  // path into the last two units (no zero-trip path with other registers).
  const int KT = K / kBK;
  int u = 0;
  do {
    gemm_unit<0, 2, TR>(ring, u, e, acc, bf, af);
    gemm_unit<1, 2, TR>(ring, u + 1, e, acc, bf, af);
    u += 2;
  } while (u < KT - 2);
  gemm_unit<0, 1, TR>(ring, KT - 2, e, acc, bf, af);
  gemm_unit<1, 0, TR>(ring, KT - 1, e, acc, bf, af);
  // The last MFMAs must have read their sources and retired before those
  // registers are reused and the accumulators read: the padding takes the
  // final accumulators and fragments as operands, so nothing that touches
  // them can be scheduled above it, and it outlasts the MFMA queue.
  asm volatile(
      "s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n"
      "s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7\n s_nop 7"
      : "+a"(acc[7][0]), "+a"(acc[7][1]), "+a"(acc[7][2]), "+a"(acc[7][3]), "+a"(acc[6][0]), "+a"(acc[6][1]),
        "+a"(acc[6][2]), "+a"(acc[6][3])
      : "v"(af[13 % 8]), "v"(af[14 % 8]), "v"(af[15 % 8]), "v"(bf[1][0]), "v"(bf[1][1]), "v"(bf[1][2]), "v"(bf[1][3])
      : "memory");
  // Every accumulator is defined here, in its AGPRs: copies the epilogue makes
  // for VALU work cannot be hoisted into the last units (where the compiler
  // cannot see the asm MFMAs still in flight).
  pin8(acc[0], acc[1]);
  pin8(acc[2], acc[3]);
  pin8(acc[4], acc[5]);
}

// Visits this lane's accumulators as quads: f(i, p0, q, x) gets rows
// p0..p0+3 of column q, i the quad's index. (v_mfma 16x16 layout: lane l,
// register r -> row 4*(l/16) + r, column l%16; pbase / qbase carry the lane
// part.) Indices are compile-time after unrolling, so the accumulators stay
// in registers.
template <class F>
__device__ __forceinline__ void for_each_quad(const f32x4 (&acc)[kMi][kNi], int pbase, int qbase, F&& f) {
#pragma unroll
  for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
    for (int ni = 0; ni < kNi; ++ni) {
      const float x[4] = {acc[mi][ni][0], acc[mi][ni][1], acc[mi][ni][2], acc[mi][ni][3]};
      f(mi * kNi + ni, pbase + mi * 16, qbase + ni * 16, x);
    }
}



// Tiles of one matrix in a stage (upper triangle for the symmetric ones) and
// the stage's K-split chunks per tile (1: unsplit).
template <int STAGE, class D>
__device__ __forceinline__ int stage_tiles(const D& d) {
  const int nt = d.Mp / kTile;
  return (STAGE == ST_GRAM || STAGE == ST_SYMM) ? nt * (nt + 1) / 2 : nt * (d.Np / kTile);
}
template <int STAGE, class D>
__device__ __forceinline__ int stage_split(const D& d) {
  const int ks = STAGE == ST_GRAM ? d.ks_gram : STAGE == ST_SYMM ? d.ks_symm : d.ks_full;
  return ks > 1 ? ks : 1;
}

template <int STAGE, int LAYOUT, bool SPLIT = false, class D>
__device__ __forceinline__ TileJob decode_tile(const D& d, int lt, const GemmArgs& args) {
  TileJob j;
  int P, Q;
  bool sym = false;
  const int cur = args.cur;
  constexpr bool tx = LAYOUT & kTiledX, ts = LAYOUT & kTiledS;
  j.rtr = false;
  if (STAGE == ST_GRAM) {
    j.L = j.R = d.X[cur]; j.ldl = j.ldr = d.Np; j.K = d.Np; P = Q = d.Mp; sym = true;
    j.tl = j.tr = tx;
  } else if (STAGE == ST_SYMM) {
    // S[sl] · S[sr]ᵀ: both operands are read by rows (a symmetric right operand
    // is its own transpose)
    j.L = d.S[args.sl]; j.R = d.S[args.sr]; j.ldl = j.ldr = d.Mp; j.K = d.Mp; P = Q = d.Mp; sym = true;
    j.tl = j.tr = ts;
  } else {
    // UPDATE and FINAL: C (Mp x Np) = S[sl] · X, X read transposed. C is the
    // param of a wide matrix and the param's transpose for a tall one.
    j.L = d.S[args.sl]; j.ldl = d.Mp; j.R = d.X[cur]; j.ldr = d.Np; j.K = d.Mp; P = d.Mp; Q = d.Np;
    j.tl = ts; j.tr = tx; j.rtr = true;
  }
  // SPLIT: work item lt is chunk `chunk` of tile `tile` (chunk-major), its K
  // range the chunk's share of the contraction; otherwise item lt is tile lt
  j.u0 = 0;
  if constexpr (SPLIT) {
    int tile, chunk;
    split_item(lt, stage_tiles<STAGE>(d), tile, chunk);
    j.K /= stage_split<STAGE>(d);
    j.u0 = chunk * (j.K / kBK);
    lt = tile;
  }
  if (sym) {
    sym_tile(lt, P / kTile, j.ti, j.tj);
  } else if (STAGE == ST_UPDATE || STAGE == ST_FINAL) {
    // C = S·X: the large operand is the right one (X's column panels, one per
    // tile column), so the XCDs walk the same few column panels at once.
    // Measured on bench.py --config 5: UPDATE 747.6 -> 737.1 ms per step
    full_tile_cols(lt, P / kTile, Q / kTile, j.ti, j.tj);
  } else {
    full_tile(lt, P / kTile, Q / kTile, j.ti, j.tj);
  }
  return j;
}

// 4x4 transpose of bf16 values across each group of 4 lanes. Lane l holds
// rows 0..3 of column l%4 of a 4x4 block (its accumulator quad); afterwards it
// holds columns 0..3 of row l%4, i.e. 4 consecutive elements of one row of a
// row-major output, stored with one 8-byte store instead of four 2-byte ones.
// Dwords are exchanged with lane l^2 (DPP quad_perm [2,3,0,1]), then 16-bit
// halves with lane l^1 (quad_perm [1,0,3,2]) and reassembled by v_perm_b32.
// All 64 lanes must be active.
__device__ __forceinline__ u16x4 quad_transpose(u16x4 v, int lane) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 d = __builtin_bit_cast(u32x2, v);  // d.x = rows 0,1; d.y = rows 2,3
  const bool low = (lane & 2) == 0;
  const uint32_t recv = (uint32_t)__builtin_amdgcn_mov_dpp((int)(low ? d.y : d.x), 0x4E, 0xF, 0xF, false);
  const uint32_t a0 = low ? d.x : recv;  // rows 2(l/2%2)+{0,1} of column l%2
  const uint32_t a1 = low ? recv : d.y;  // the same rows of column l%2 + 2
  const uint32_t p0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)a0, 0xB1, 0xF, 0xF, false);
  const uint32_t p1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)a1, 0xB1, 0xF, 0xF, false);
  const uint32_t sel = (lane & 1) ? 0x03020706u : 0x05040100u;  // odd: high halves, even: low halves
  const u32x2 o = {__builtin_amdgcn_perm(p0, a0, sel), __builtin_amdgcn_perm(p1, a1, sel)};
  return __builtin_bit_cast(u16x4, o);
}

// Pairs the quads a = (mi, ni) and b = (mi, ni+1) of the transposed output
// Cᵀ[q][p]: lanes of 16-lane rows 0 and 2 end up with 8 consecutive p of a's
// column, rows 1 and 3 with 8 consecutive p of b's column (v_permlane16_swap
// exchanges odd rows of its first operand with even rows of its second), so
// every lane stores 16 contiguous bytes at Cᵀ[q + 16(g&1)][p0 - 4(g&1)],
// g = lane/16. All 64 lanes must be active.
__device__ __forceinline__ u32x4 pair_rows(u16x4 a, u16x4 b) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const u32x2 x = __builtin_bit_cast(u32x2, a), y = __builtin_bit_cast(u32x2, b);
  const auto s0 = __builtin_amdgcn_permlane16_swap(x.x, y.x, false, false);
  const auto s1 = __builtin_amdgcn_permlane16_swap(x.y, y.y, false, false);
  return (u32x4){s0[0], s1[0], s0[1], s1[1]};
}

// Diagonal tiles of a symmetric product whose operands differ: the stores keep
// the elements on and above the diagonal (store_upper4: element e of v is
// column col0 + e of `row`) and mirror the strict upper part (store_lower8:
// element e of v is the output element (p0 + e, q), stored at C[q][p0 + e]),
// so the tile comes out exactly symmetric.
__device__ __forceinline__ void store_upper4(uint16_t* dst, u16x4 v, int col0, int row) {
  if (col0 >= row) {
    *(u16x4*)dst = v;
    return;
  }
  if (col0 + 3 < row) return;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (col0 + e >= row) dst[e] = v[e];
}
__device__ __forceinline__ void store_lower8(uint16_t* dst, u32x4 v, int p0, int q) {
  if (p0 + 7 < q) {
    *(u32x4*)dst = v;
    return;
  }
  if (p0 >= q) return;
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (p0 + e < q) dst[e] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
}

// Loads, for every quad of this lane, the 4 consecutive elements T[q][p0..p0+3]
// of a row-major matrix T (ld elements). Quads (mi, ni) and (mi, ni+1) travel
// together as one 16-byte load in the paired layout of pair_rows, which
// v_permlane16_swap (its own inverse) turns back into the two quads. All
// loads are issued before any swap.
__device__ __forceinline__ void load_quads(u16x4 (&v)[kQuads], const uint16_t* __restrict__ T, int64_t ld,
                                           bool tiled, int pbase, int qbase, int lane) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const int g1 = (lane >> 4) & 1;
  u32x4 w[kQuads / 2];
#pragma unroll
  for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
    for (int ni = 0; ni < kNi; ni += 2)
      w[(mi * kNi + ni) / 2] =
          *(const u32x4*)(T + ws_off(qbase + (ni + g1) * 16, pbase + mi * 16 - 4 * g1, ld, tiled));
#pragma unroll
  for (int k = 0; k < kQuads / 2; ++k) {
    const auto s0 = __builtin_amdgcn_permlane16_swap(w[k].x, w[k].z, false, false);
    const auto s1 = __builtin_amdgcn_permlane16_swap(w[k].y, w[k].w, false, false);
    v[2 * k] = __builtin_bit_cast(u16x4, (u32x2){s0[0], s1[0]});
    v[2 * k + 1] = __builtin_bit_cast(u16x4, (u32x2){s0[1], s1[1]});
  }
}

// Per-wave staging of 16 rows x 128 bytes (2 KiB of LDS) that turns the
// accumulator layout into full-line global stores. A wave's 128 x 64 sub-tile
// is 64 columns wide, one 128-byte line per row in either workspace layout
// (its column runs start at multiples of 64), so each store instruction can
// write 8 whole rows: lane l writes bytes 16(l%8)..16(l%8)+15 of row 8s + l/8.
// The quads land in the slot as they sit in registers; chunk c (16 bytes) of
// staged row r is kept at chunk c ^ swz(r), with the swizzle chosen per
// orientation so that the quad writes hit distinct banks (32-byte runs per row
// for the normal orientation, 16-byte runs for the transposed one); the
// row-order read-back is conflict-free under either. Only the wave itself
// touches its slot, and LDS executes one wave's accesses in order, so no
// barrier is needed between a round's writes and reads or between rounds.
constexpr int kStageBytes = 16 * 128;
__device__ __forceinline__ int swz_norm(int r) { return ((r >> 1) & 3) << 1; }
__device__ __forceinline__ int swz_tr(int r) { return (r >> 1) & 7; }

// Normal orientation: quads o[ni] (rows 4g + r, column 16 ni + lane%16) of
// one 16-row band; after quad_transpose lane l holds row 4g + l%4, columns
// 16 ni + 4 c4 .. + 3 (g = l/16, c4 = (l%16)/4).
__device__ __forceinline__ void stage_band(char* slot, const u16x4 (&o)[kNi], int lane) {
  const int r = 4 * (lane >> 4) + (lane & 3), c4 = (lane & 15) >> 2;
#pragma unroll
  for (int ni = 0; ni < kNi; ++ni) {
    const int c = 2 * ni + (c4 >> 1);
    *(u16x4*)(slot + r * 128 + ((c ^ swz_norm(r)) << 4) + ((c4 & 1) << 3)) = quad_transpose(o[ni], lane);
  }
}

// Transposed orientation: the quads of four consecutive 16-row bands mi at one
// 16-column block ni, staged as 16 rows (columns 16 ni + lane%16 of the tile)
// of 64 elements (rows 16 mi + 4g + r): lane l's quad is 8 consecutive bytes
// of staged row l%16.
__device__ __forceinline__ void stage_block_tr(char* slot, const u16x4 (&o)[4], int lane) {
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = 2 * m + (g >> 1);
    *(u16x4*)(slot + r * 128 + ((c ^ swz_tr(r)) << 4) + ((g & 1) << 3)) = o[m];
  }
}

// Writes the 16 staged rows to memory, row r to row0 + r·step (row0: the
// first element of the block's 64-column run; step: 64 in the panel layout,
// whose 16-row blocks never cross a panel, or ld row-major), 8 whole rows per
// store instruction.
// The stores are buffer stores off a resource for the block (its base is
// wave-uniform, so only a 32-bit offset per lane lives in vector registers).
template <bool TR>
__device__ __forceinline__ void stage_flush(const char* slot, int lane, uint16_t* row0, int step) {
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(row0, (short)0, (15 * step + 64) * 2, 0x00020000);
#pragma unroll
  for (int s = 0; s < 2; ++s) {
    const int r = 8 * s + (lane >> 3), c = lane & 7;
    const u32x4 v = *(const u32x4*)(slot + r * 128 + ((c ^ (TR ? swz_tr(r) : swz_norm(r))) << 4));
    __builtin_amdgcn_raw_buffer_store_b128(v, rs, (r * step + 8 * c) * 2, 0, 0);
  }
}

// Quads T[q][p..p+3] of a wave's band group as full-line loads: round ni
// covers rows q = qw + 16 ni + 0..15 and columns p = p0 .. p0 + 63 (p0 a
// multiple of 64), lane l loading 16 bytes of row 8h + l/8 at column
// p0 + 8 (l % 8) into raw[ni][h]. unstage_quads turns one round into the
// quads of the accumulator layout through the wave's staging slot.
// The 64 rows qw .. qw+63 (qw a multiple of 64) lie in one 256-row panel, so
// in the panel layout they are 64 elements apart, and ld apart row-major.
__device__ __forceinline__ void load_rounds(u32x4 (&raw)[kNi][2], const uint16_t* __restrict__ T, int64_t ld,
                                            bool tiled, int qw, int p0, int lane) {
  const int step = tiled ? 64 : (int)ld;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)(T + ws_off(qw, p0, ld, tiled)), (short)0, (63 * step + 64) * 2, 0x00020000);
  const int v0 = ((lane >> 3) * step + 8 * (lane & 7)) * 2;
#pragma unroll
  for (int ni = 0; ni < kNi; ++ni)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      raw[ni][h] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, v0 + (16 * ni + 8 * h) * step * 2, 0, 0));
}

// Writes round raw[2] to the slot in the transposed staging layout and reads
// back quad m = 0..3 of this lane: T[q][p0 + 16m + 4g .. + 3] for q = the
// round's row lane % 16 (g = lane / 16), the layout stage_block_tr writes.
__device__ __forceinline__ void unstage_quads(char* slot, const u32x4 (&raw)[2], u16x4 (&q)[4], int lane) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = 8 * h + (lane >> 3), c = lane & 7;
    *(u32x4*)(slot + r * 128 + ((c ^ swz_tr(r)) << 4)) = raw[h];
  }
  const int r = lane & 15, g = lane >> 4;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = 2 * m + (g >> 1);
    q[m] = *(const u16x4*)(slot + r * 128 + ((c ^ swz_tr(r)) << 4) + ((g & 1) << 3));
  }
}

// The inverse of stage_band: writes one band's full-line loads raw[2] (16
// rows of 64 columns: lane l holds 16 bytes of row 8h + l/8 at columns
// 8(l%8) .. +7, load_rounds' layout) to the slot in the normal staging layout
// and reads back this lane's quads o[ni] of the band (rows 4g + r, column
// 16 ni + lane%16): quad_transpose is its own inverse.
__device__ __forceinline__ void unstage_band(char* slot, const u32x4 (&raw)[2], u16x4 (&o)[kNi], int lane) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int r = 8 * h + (lane >> 3), c = lane & 7;
    *(u32x4*)(slot + r * 128 + ((c ^ swz_norm(r)) << 4)) = raw[h];
  }
  const int r = 4 * (lane >> 4) + (lane & 3), c4 = (lane & 15) >> 2;
#pragma unroll
  for (int ni = 0; ni < kNi; ++ni) {
    const int c = 2 * ni + (c4 >> 1);
    o[ni] = quad_transpose(*(const u16x4*)(slot + r * 128 + ((c ^ swz_norm(r)) << 4) + ((c4 & 1) << 3)), lane);
  }
}

// load_quads for the band group hb only (bands mi = 4hb .. 4hb+3): v[m * kNi + ni].
__device__ __forceinline__ void load_quads_half(u16x4 (&v)[kQuads / 2], const uint16_t* __restrict__ T, int64_t ld,
                                                bool tiled, int pbase, int qbase, int lane, int hb) {
  typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
  const int g1 = (lane >> 4) & 1;
  u32x4 w[kQuads / 4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int ni = 0; ni < kNi; ni += 2)
      w[(m * kNi + ni) / 2] =
          *(const u32x4*)(T + ws_off(qbase + (ni + g1) * 16, pbase + (4 * hb + m) * 16 - 4 * g1, ld, tiled));
#pragma unroll
  for (int k = 0; k < kQuads / 4; ++k) {
    const auto s0 = __builtin_amdgcn_permlane16_swap(w[k].x, w[k].z, false, false);
    const auto s1 = __builtin_amdgcn_permlane16_swap(w[k].y, w[k].w, false, false);
    v[2 * k] = __builtin_bit_cast(u16x4, (u32x2){s0[0], s1[0]});
    v[2 * k + 1] = __builtin_bit_cast(u16x4, (u32x2){s0[1], s1[1]});
  }
}

// d.scales[i] through the constant address space: a scalar load (the norm
// kernel wrote it in an earlier launch, and a launch starts with its scalar
// cache invalidated), so no vector register holds the address or the value.
template <class D>
__device__ __forceinline__ float scale_of(const D& d, int i) {
  return ((const __attribute__((address_space(4))) float*)d.scales)[i];
}

// Register vector of 4 param elements of the FINAL epilogue.
template <bool F32> struct PickVec { typedef u16x4 type; typedef uint16_t elem; };
template <> struct PickVec<true> { typedef f32x4 type; typedef float elem; };

// Tile counters: the tiles of a launch form kXcds queues, queue x holding the
// virtual indices v = x + kXcds*k in order, each mapped to a tile by
// xcd_remap (a permutation of [0, total)). A block serves the queue of the XCD
// it runs on, so an XCD walks runs of kXcdChunk neighbouring tiles whose
// panels its L2 shares, and takes tiles from the other queues once its own is
// empty, so XCDs that run slower finish no later than the rest. Returns -1
// when every queue is empty. Called by one lane; *home (in LDS, so no register
// stays live across the K loop) is the queue to try first and follows the
// queue that last had work.
__device__ __forceinline__ int grab_tile(int32_t* queues, int total, int* home) {
  const int h = *home;
#pragma unroll 1
  for (int i = 0; i < kXcds; ++i) {
    const int y = (h + i) & (kXcds - 1);
    const int len = total > y ? (total - y + kXcds - 1) / kXcds : 0;
    if (len == 0) continue;
    const int k = __hip_atomic_fetch_add(queues + y, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (k < len) {
      *home = y;
      return xcd_remap(y + kXcds * k, total);
    }
  }
  return -1;
}

__device__ __forceinline__ int xcc_id() {
  return (int)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & (kXcds - 1));  // HW_REG_XCC_ID[3:0]
}

// One Newton–Schulz stage over every matrix of the group.
//   GRAM   S[sc] = s·X Xᵀ          (s = 1/‖X‖² when `first`, folding
//                                   X.div_(norm) of torch/optim/_muon.py:59)
//   SYMM   S[sc] = c·S[sl] S[sr]ᵀ + b·S[sd]
//          standard form: B = c·A A + b·A (torch.addmm(A, A, A, beta=b,
//          alpha=c), :63-65); gram form: the quack gemm_symmetric(_out)
//          products of pan/optim/patch_muon.py:320-331
//   UPDATE X' = s·(a·X + S[sl] X)  (torch.addmm(X, B, X, beta=a), :66; a = 0 is
//                                   the gram form's X <- Q X, :316), written
//                                   as X' (X is read transposed from LDS)
//   FINAL  O = bf16(s·(a·X + S[sl] X)) then p <- p·(1-lr·wd) - lr·adj·O
//          (pan/optim/muon_triton.py:130-131), or O stored (MODE_NS)
// GRAM and SYMM are symmetric: only upper-triangle tiles are computed and
// each off-diagonal tile is also stored transposed. Every result is rounded
// to bf16 where torch rounds it.
// PDT is the param dtype of the FINAL epilogue (one instantiation per dtype
// keeps the epilogue's registers within budget); other stages ignore it.
// slot: this wave's staging slot (kStageBytes of LDS).
template <int STAGE, int PDT, int LAYOUT, class D>
__device__ __forceinline__ void gemm_epilogue(const GemmArgs& args, const D& d, const TileJob& job,
                                              const f32x4 (&acc)[kMi][kNi], int wave, char* slot = nullptr) {
#pragma clang fp contract(off)
  const int cur = args.cur;
  constexpr bool tx = LAYOUT & kTiledX, ts = LAYOUT & kTiledS;
  const int lane = lane_id();
  const int pbase = job.ti * kTile + (wave >> 2) * kWaveRows + 4 * (lane >> 4);
  const int qbase = job.tj * kTile + (wave & 3) * kWaveCols + (lane & 15);

  // Epilogue operands are read as full lines of rows and turned into this
  // lane's quads (4 consecutive output rows p at one column q) through the
  // staging slot, or as quads T[q][p0..p0+3] of a symmetric operand. All
  // loads are issued before any store, so no load waits behind stores in
  // vmcnt order.
  if (STAGE == ST_GRAM || STAGE == ST_SYMM) {
    uint16_t* C = d.S[args.sc];
    const int64_t ldc = d.Mp;
    const float s = (STAGE == ST_GRAM && args.first) ? scale_of(d, 0) : 1.0f;
    const float cb = args.b, cc = args.c;
    const bool mirror = job.ti != job.tj;
    // A diagonal tile of L·Rᵀ with L != R is symmetric only up to rounding:
    // SYMM stores its upper part and mirrors it, so every symmetric product
    // is exactly symmetric (later products read R and the addend through
    // their transposes). A GRAM diagonal tile is bitwise symmetric already
    // (the same products in the same order), and so is SYMM's when L == R
    // (the standard form's A·A, the gram form's R·R): those go through the
    // full-tile stores. SYMM's full tiles always store the mirror too; on such
    // a diagonal tile it writes every element again with the same bits.
    const bool diag = STAGE == ST_SYMM && !mirror && args.sl != args.sr;
    if (ts && !diag) {
      // full tiles: staged full-line stores, normal orientation and (off the
      // diagonal) the mirror, band group by band group; the addend (symmetric,
      // so read from either orientation) a band group at a time
      const int pw = job.ti * kTile + (wave >> 2) * kWaveRows, qw = job.tj * kTile + (wave & 3) * kWaveCols;
      // the addend (symmetric, so read in the transposed orientation) as
      // full-line loads; each band group's loads are issued before the
      // previous group's stores, so no load waits behind stores in vmcnt order
      const bool addend = STAGE == ST_SYMM && cb != 0.0f;
      u32x4 raw[kNi][2];
      if (addend) load_rounds(raw, d.S[args.sd], ldc, ts, qw, pw, lane);
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        u16x4 o[4][kNi];
#pragma unroll
        for (int ni = 0; ni < kNi; ++ni) {
          u16x4 ah[4] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
          if (addend) unstage_quads(slot, raw[ni], ah, lane);
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const int mi = 4 * hb + m;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const float x = acc[mi][ni][r];
              o[m][ni][r] = f2bf((STAGE == ST_GRAM) ? x * s : cc * x + cb * bf2f(ah[m][r]));
            }
          }
        }
        // the second band group's addend is requested before this group's stores
        if (hb == 0 && addend) load_rounds(raw, d.S[args.sd], ldc, ts, qw, pw + 64, lane);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          stage_band(slot, o[m], lane);
          const int p0 = pw + (4 * hb + m) * 16;
          stage_flush<false>(slot, lane, C + ws_off(p0, qw, ldc, ts), ts ? 64 : (int)ldc);
        }
        if (STAGE == ST_SYMM || mirror) {
#pragma unroll
          for (int ni = 0; ni < kNi; ++ni) {
            const u16x4 blk[4] = {o[0][ni], o[1][ni], o[2][ni], o[3][ni]};
            stage_block_tr(slot, blk, lane);
            const int p0 = pw + 64 * hb;
            stage_flush<true>(slot, lane, C + ws_off(qw + 16 * ni, p0, ldc, ts), ts ? 64 : (int)ldc);
          }
        }
      }
      return;
    }
    // diagonal SYMM tiles (masked element stores of the upper part and its
    // mirror), and the row-major outputs of pm_gram / pm_gemm_symmetric
    u16x4 av[kQuads];
    if (STAGE == ST_SYMM && cb != 0.0f) {
      load_quads(av, d.S[args.sd], ldc, ts, pbase, qbase, lane);
    } else {
#pragma unroll
      for (int i = 0; i < kQuads; ++i) av[i] = (u16x4){0, 0, 0, 0};
    }
    const int g1 = (lane >> 4) & 1;
#pragma unroll
    for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
      for (int ni = 0; ni < kNi; ni += 2) {
        const int p0 = pbase + mi * 16;
        u16x4 o[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int i = mi * kNi + ni + h, q = qbase + (ni + h) * 16;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float x = acc[mi][ni + h][r];
            o[h][r] = f2bf((STAGE == ST_GRAM) ? x * s : cc * x + cb * bf2f(av[i][r]));
          }
          const u16x4 t = quad_transpose(o[h], lane);
          uint16_t* dst = C + ws_off(p0 + (lane & 3), q & ~3, ldc, ts);
          if (!diag) {
            *(u16x4*)dst = t;
          } else {
            store_upper4(dst, t, q & ~3, p0 + (lane & 3));
          }
        }
        if (mirror || diag) {
          const int qm = qbase + (ni + g1) * 16, pm = p0 - 4 * g1;
          const u32x4 m = pair_rows(o[0], o[1]);
          if (mirror) {
            *(u32x4*)(C + ws_off(qm, pm, ldc, ts)) = m;
          } else {
            store_lower8(C + ws_off(qm, pm, ldc, ts), m, pm, qm);
          }
        }
      }
    return;
  }

  const float s = args.first ? scale_of(d, 1) : 1.0f;
  const float ca = args.a;
  if (STAGE == ST_UPDATE) {
    uint16_t* Xn = d.X[cur ^ 1];
    const int64_t ldx = d.Np;
    // X[p][q] as full-line loads of X's rows (each band group's loads issued
    // before the previous group's stores), turned into quads through the
    // staging slot; X' goes out through the slot as full lines
    const int pw = job.ti * kTile + (wave >> 2) * kWaveRows, qw = job.tj * kTile + (wave & 3) * kWaveCols;
    u32x4 raw[4][2];
    if (ca != 0.0f) load_rounds(raw, d.X[cur], ldx, tx, pw, qw, lane);
#pragma unroll
    for (int hb = 0; hb < 2; ++hb) {
      u16x4 o[4][kNi];
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        u16x4 xq[kNi] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
        if (ca != 0.0f) unstage_band(slot, raw[m], xq, lane);
        const int mi = 4 * hb + m;
#pragma unroll
        for (int ni = 0; ni < kNi; ++ni)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[m][ni][r] = f2bf((ca * bf2f(xq[ni][r]) + acc[mi][ni][r]) * s);
      }
      // the second band group's X is requested before this group's stores
      if (hb == 0 && ca != 0.0f) load_rounds(raw, d.X[cur], ldx, tx, pw + 64, qw, lane);
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        stage_band(slot, o[m], lane);
        const int p0 = pw + (4 * hb + m) * 16;
        stage_flush<false>(slot, lane, Xn + ws_off(p0, qw, ldx, tx), tx ? 64 : (int)ldx);
      }
    }
    return;
  }

  // ST_FINAL: C = S·X (Mp x Np) holds O = bf16(s·(a·X + S X)) at element
  // (p, q): the param's element (p, q) for a wide param, (q, p) for a tall
  // one. The a·X term is X[p][q], read as full lines of X's rows and turned
  // into quads through the staging slot (or element by element). Then
  // p <- p·(1 - lr·wd) - lr·adj·O in fp32 per element.
  const uint16_t* X = d.X[cur];
  const int64_t ldx = d.Np;
  const bool tall = d.trans;
  const int prow = d.rows, pcol = d.cols;
  const int64_t ldp = d.p_ld;
  float wdf = 0.0f, neg = 0.0f;
  if (args.mode == MODE_STEP) {
    if (args.lr_dev) {
      const float lr = *args.lr_dev;
      wdf = 1.0f - lr * args.wd;
      neg = -(lr * d.adj_ratio);
    } else {
      wdf = args.wdf_host;
      neg = d.neg_lr_host;
    }
  }
  const bool step = args.mode == MODE_STEP;
  const bool ax = ca != 0.0f;
  constexpr bool f32p = PDT == DT_F32;  // MODE_NS launches the bf16 instantiation
  // param update of 8 consecutive bf16 elements (one 16-byte run)
  auto step8 = [&](const u32x4& on, const u32x4& pv) {
    u32x4 out;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      uint16_t o2[2];
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const float onv = bf2f((uint16_t)(on[k] >> (16 * half)));
        const float pe = bf2f((uint16_t)(pv[k] >> (16 * half)));
        o2[half] = f2bf(step ? pe * wdf + onv * neg : onv);
      }
      out[k] = (uint32_t)o2[0] | ((uint32_t)o2[1] << 16);
    }
    return out;
  };
  if (!f32p && slot) {
    // bf16 params: when this wave's 128 x 64 block lies inside the param and
    // rows are 16-byte aligned, O goes through the staging slot and the param
    // is read, stepped and written as full lines (the same fp32 operations
    // per element)
    const int pw = job.ti * kTile + (wave >> 2) * kWaveRows, qw = job.tj * kTile + (wave & 3) * kWaveCols;
    const bool inside = tall ? (qw + kWaveCols <= prow && pw + kWaveRows <= pcol)
                             : (pw + kWaveRows <= prow && qw + kWaveCols <= pcol);
    const bool whole = inside && ldp % 8 == 0 && (uintptr_t)d.param % 16 == 0;
    uint16_t* P = (uint16_t*)d.param;
    if (whole && !tall) {
      // wide: band m (16 param rows) of band group hb is staged as rows and
      // stepped 16 rows x 64 columns at a time
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        __builtin_amdgcn_sched_barrier(0);
        u32x4 xr[4][2];
        if (ax) load_rounds(xr, X, ldx, tx, pw + 64 * hb, qw, lane);
        u32x4 pv[4][2];
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            pv[m][h] = step ? *(const u32x4*)(P + (int64_t)(pw + 64 * hb + 16 * m + 8 * h + (lane >> 3)) * ldp + qw +
                                              8 * (lane & 7))
                            : (u32x4){0, 0, 0, 0};
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          u16x4 xq[kNi] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
          if (ax) unstage_band(slot, xr[m], xq, lane);
          u16x4 o[kNi];
#pragma unroll
          for (int ni = 0; ni < kNi; ++ni)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float a = acc[4 * hb + m][ni][e];
              o[ni][e] = f2bf((ca * bf2f(xq[ni][e]) + a) * s);  // bf16 update
            }
          stage_band(slot, o, lane);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int r = 8 * h + (lane >> 3), c = lane & 7;
            const u32x4 on = *(const u32x4*)(slot + r * 128 + ((c ^ swz_norm(r)) << 4));
            *(u32x4*)(P + (int64_t)(pw + 64 * hb + 16 * m + r) * ldp + qw + 8 * c) = step8(on, pv[m][h]);
          }
        }
      }
      return;
    }
    if (whole) {
      // tall: the param's rows are C's columns; each 16-column block of C (16
      // param rows) is staged transposed and stepped as full lines. The a·X
      // quads of the band group are loaded first as 8-byte pieces of X's rows
      // (row 4g + l%4 of a 16-row band, 4 columns) and turned by
      // quad_transpose.
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        __builtin_amdgcn_sched_barrier(0);
        u16x4 xb[4][kNi];
        const int xrow = pw + 64 * hb + 4 * (lane >> 4) + (lane & 3), xcol = qw + 4 * ((lane & 15) >> 2);
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int ni = 0; ni < kNi; ++ni)
            xb[m][ni] = ax ? *(const u16x4*)(X + ws_off(xrow + 16 * m, xcol + 16 * ni, ldx, tx)) : (u16x4){0, 0, 0, 0};
        u32x4 pv[kNi][2];
#pragma unroll
        for (int ni = 0; ni < kNi; ++ni)
#pragma unroll
          for (int h = 0; h < 2; ++h)
            pv[ni][h] = step ? *(const u32x4*)(P + (int64_t)(qw + 16 * ni + 8 * h + (lane >> 3)) * ldp + pw + 64 * hb +
                                               8 * (lane & 7))
                             : (u32x4){0, 0, 0, 0};
        if (ax) {
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int ni = 0; ni < kNi; ++ni) xb[m][ni] = quad_transpose(xb[m][ni], lane);
        }
#pragma unroll
        for (int ni = 0; ni < kNi; ++ni) {
          u16x4 blk[4];
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const float a = acc[4 * hb + m][ni][e];
              blk[m][e] = f2bf((ca * bf2f(xb[m][ni][e]) + a) * s);  // bf16 update
            }
          stage_block_tr(slot, blk, lane);
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const int r = 8 * h + (lane >> 3), c = lane & 7;
            const u32x4 on = *(const u32x4*)(slot + r * 128 + ((c ^ swz_tr(r)) << 4));
            *(u32x4*)(P + (int64_t)(qw + 16 * ni + r) * ldp + pw + 64 * hb + 8 * c) = step8(on, pv[ni][h]);
          }
        }
      }
      return;
    }
  }
  if (f32p && slot && step) {
    // fp32 params: the same full-line path as bf16 params, each 8-element run
    // of a param row read and written as two 16-byte vectors. Two bands (wide)
    // or two 16-column blocks (tall) at a time, so the param values held in
    // registers stay within budget.
    const int pw = job.ti * kTile + (wave >> 2) * kWaveRows, qw = job.tj * kTile + (wave & 3) * kWaveCols;
    const bool inside = tall ? (qw + kWaveCols <= prow && pw + kWaveRows <= pcol)
                             : (pw + kWaveRows <= prow && qw + kWaveCols <= pcol);
    const bool whole = inside && ldp % 8 == 0 && (uintptr_t)d.param % 16 == 0;
    float* P = (float*)d.param;
    // p <- p·(1 - lr·wd) - lr·adj·O for the 8 elements of O's 16-byte run `on`
    // and the param run p0, p1 at dst (the element path's fp32 operations)
    auto step8f = [&](const u32x4& on, const f32x4& p0, const f32x4& p1, float* dst) {
      f32x4 r0, r1;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const float lo = bf2f((uint16_t)(on[k] & 0xffffu)), hi = bf2f((uint16_t)(on[k] >> 16));
        const float plo = k < 2 ? p0[2 * k] : p1[2 * k - 4], phi = k < 2 ? p0[2 * k + 1] : p1[2 * k - 3];
        const float olo = plo * wdf + lo * neg, ohi = phi * wdf + hi * neg;
        if (k < 2) {
          r0[2 * k] = olo;
          r0[2 * k + 1] = ohi;
        } else {
          r1[2 * k - 4] = olo;
          r1[2 * k - 3] = ohi;
        }
      }
      *(f32x4*)dst = r0;
      *(f32x4*)(dst + 4) = r1;
    };
    if (whole && !tall) {
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        __builtin_amdgcn_sched_barrier(0);
        u32x4 xr[4][2];
        if (ax) load_rounds(xr, X, ldx, tx, pw + 64 * hb, qw, lane);
#pragma unroll
        for (int mh = 0; mh < 2; ++mh) {
          f32x4 pv[2][2][2];
#pragma unroll
          for (int m2 = 0; m2 < 2; ++m2)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float* row =
                  P + (int64_t)(pw + 64 * hb + 16 * (2 * mh + m2) + 8 * h + (lane >> 3)) * ldp + qw + 8 * (lane & 7);
              pv[m2][h][0] = *(const f32x4*)row;
              pv[m2][h][1] = *(const f32x4*)(row + 4);
            }
#pragma unroll
          for (int m2 = 0; m2 < 2; ++m2) {
            const int m = 2 * mh + m2;
            u16x4 xq[kNi] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
            if (ax) unstage_band(slot, xr[m], xq, lane);
            u16x4 o[kNi];
#pragma unroll
            for (int ni = 0; ni < kNi; ++ni)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float a = acc[4 * hb + m][ni][e];
                o[ni][e] = f2bf((ca * bf2f(xq[ni][e]) + a) * s);  // bf16 update
              }
            stage_band(slot, o, lane);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int r = 8 * h + (lane >> 3), c = lane & 7;
              const u32x4 on = *(const u32x4*)(slot + r * 128 + ((c ^ swz_norm(r)) << 4));
              step8f(on, pv[m2][h][0], pv[m2][h][1], P + (int64_t)(pw + 64 * hb + 16 * m + r) * ldp + qw + 8 * c);
            }
          }
        }
      }
      return;
    }
    if (whole) {
      // tall: as for bf16 params, each 16-column block of C (16 param rows)
      // staged transposed
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        __builtin_amdgcn_sched_barrier(0);
        u16x4 xb[4][kNi];
        const int xrow = pw + 64 * hb + 4 * (lane >> 4) + (lane & 3), xcol = qw + 4 * ((lane & 15) >> 2);
#pragma unroll
        for (int m = 0; m < 4; ++m)
#pragma unroll
          for (int ni = 0; ni < kNi; ++ni)
            xb[m][ni] = ax ? *(const u16x4*)(X + ws_off(xrow + 16 * m, xcol + 16 * ni, ldx, tx)) : (u16x4){0, 0, 0, 0};
        if (ax) {
#pragma unroll
          for (int m = 0; m < 4; ++m)
#pragma unroll
            for (int ni = 0; ni < kNi; ++ni) xb[m][ni] = quad_transpose(xb[m][ni], lane);
        }
#pragma unroll
        for (int nh = 0; nh < 2; ++nh) {
          f32x4 pv[2][2][2];
#pragma unroll
          for (int n2 = 0; n2 < 2; ++n2)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const float* row =
                  P + (int64_t)(qw + 16 * (2 * nh + n2) + 8 * h + (lane >> 3)) * ldp + pw + 64 * hb + 8 * (lane & 7);
              pv[n2][h][0] = *(const f32x4*)row;
              pv[n2][h][1] = *(const f32x4*)(row + 4);
            }
#pragma unroll
          for (int n2 = 0; n2 < 2; ++n2) {
            const int ni = 2 * nh + n2;
            u16x4 blk[4];
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const float a = acc[4 * hb + m][ni][e];
                blk[m][e] = f2bf((ca * bf2f(xb[m][ni][e]) + a) * s);  // bf16 update
              }
            stage_block_tr(slot, blk, lane);
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int r = 8 * h + (lane >> 3), c = lane & 7;
              const u32x4 on = *(const u32x4*)(slot + r * 128 + ((c ^ swz_tr(r)) << 4));
              step8f(on, pv[n2][h][0], pv[n2][h][1], P + (int64_t)(qw + 16 * ni + r) * ldp + pw + 64 * hb + 8 * c);
            }
          }
        }
      }
      return;
    }
  }
  // Element path (tiles at a param's edge, unaligned params): quad by quad. A
  // quad is 4 consecutive elements of one param row for a tall param; for a
  // wide one it is turned across each 4-lane group (quad_transpose, every lane
  // active) so that it is too. Loads and stores are 8-byte (bf16) or 16-byte
  // (fp32) vectors where the param's row stride and base allow, else per
  // element. The a·X term comes as full-line loads of X's rows, turned into
  // quads through the staging slot (every lane active) before any lane leaves
  // the band for the param's edge.
  const int vec_align = f32p ? 16 : 8;
  const bool vec = (ldp % 4 == 0) && ((uintptr_t)d.param % vec_align == 0);
  typedef typename PickVec<f32p>::type PV;
  typedef typename PickVec<f32p>::elem E;
  const int qbase_w = job.tj * kTile + (wave & 3) * kWaveCols + 4 * ((lane & 15) >> 2);  // wide: first column
  const int xw_p = job.ti * kTile + (wave >> 2) * kWaveRows, xw_q = job.tj * kTile + (wave & 3) * kWaveCols;
#pragma unroll
  for (int hb = 0; hb < 2; ++hb) {
    u32x4 xr[4][2];
    if (ax && slot) load_rounds(xr, X, ldx, tx, xw_p + 64 * hb, xw_q, lane);
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int mi = 4 * hb + m;
      __builtin_amdgcn_sched_barrier(0);
      u16x4 xq[kNi] = {{0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}, {0, 0, 0, 0}};
      if (ax && slot) unstage_band(slot, xr[m], xq, lane);
#pragma unroll
      for (int ni = 0; ni < kNi; ++ni) {
        const int p0 = pbase + mi * 16, q = qbase + ni * 16;
        u16x4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = !ax ? 0.0f : slot ? bf2f(xq[ni][e]) : bf2f(X[ws_off(p0 + e, q, ldx, tx)]);
          o[e] = f2bf((ca * x + acc[mi][ni][e]) * s);  // bf16 update
        }
        // param row r, columns c0 .. c0+3
        int r = q, c0 = p0;
        if (!tall) {
          o = quad_transpose(o, lane);
          r = pbase + mi * 16 + (lane & 3);  // pbase carries the lane's 4·(lane/16)
          c0 = qbase_w + ni * 16;
        }
        if (r >= prow) continue;
        const E* src = (const E*)d.param + (int64_t)r * ldp + c0;
        PV pv{};
        if (step) {
          if (vec && c0 + 3 < pcol) {
            pv = *(const PV*)src;
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) pv[e] = c0 + e < pcol ? src[e] : (E)0;
          }
        }
        float out[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float on = bf2f(o[e]);
          const float pe = f32p ? (float)pv[e] : bf2f((uint16_t)pv[e]);
          out[e] = step ? pe * wdf + on * neg : on;
        }
        const bool full = vec && c0 + 3 < pcol;
        if (f32p) {
          float* dst = (float*)d.param + (int64_t)r * ldp + c0;
          if (full) {
            *(f32x4*)dst = (f32x4){out[0], out[1], out[2], out[3]};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (c0 + e < pcol) dst[e] = out[e];
          }
        } else {
          uint16_t* dst = (uint16_t*)d.param + (int64_t)r * ldp + c0;
          if (full) {
            *(u16x4*)dst = (u16x4){f2bf(out[0]), f2bf(out[1]), f2bf(out[2]), f2bf(out[3])};
          } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (c0 + e < pcol) dst[e] = f2bf(out[e]);
          }
        }
      }
    }
  }
}

// fp32 partial tiles of a K-split stage: item (chunk c, tile t) of a matrix
// with `tiles` tiles owns 256 KiB at kpart + (c·tiles + t)·65536 floats, as
// [wave][accumulator quad][lane] float4s, so a wave's store of one quad (and
// the reduce's load of it) is 1 KiB of consecutive memory.
__device__ __forceinline__ f32x4* partial_at(float* kpart, int tiles, int tile, int chunk, int wave) {
  return (f32x4*)kpart + (((int64_t)chunk * tiles + tile) * (kGemmThreads / 64) + wave) * (kQuads * 64);
}

// Chunk partial of work item lt (the matrix's item index) of a split stage.
template <int STAGE, class D>
__device__ __forceinline__ void store_partial(const D& d, int lt, const f32x4 (&acc)[kMi][kNi], int wave) {
  typedef __attribute__((address_space(1))) f32x4 glb_f32x4;
  const int tiles = stage_tiles<STAGE>(d);
  int tile, chunk;
  split_item(lt, tiles, tile, chunk);
  glb_f32x4* dst = (glb_f32x4*)partial_at(d.kpart, tiles, tile, chunk, wave) + lane_id();
#pragma unroll
  for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
    for (int ni = 0; ni < kNi; ++ni) dst[(mi * kNi + ni) * 64] = acc[mi][ni];
}

// Persistent GEMM launch: one block per CU (grid = min(tiles, CUs)), each
// taking tiles from the queues until they are empty. The next tile's first
// copies are issued before the current tile's epilogue, so its pipeline
// fills while the epilogue's loads and stores run.
// The next tile index travels through s_tile: lane 0 takes it from the queues
// during the previous epilogue and writes slot slot^1, which the waves read
// after the barrier that ends the following tile's K loop; a slot is
// rewritten only after every wave has passed the barrier that follows its read.
template <int STAGE, int PDT, int LAYOUT, bool SPLIT = false>
__global__ __launch_bounds__(kGemmThreads, 1) void pm_ns_gemm_kernel(GemmArgs args) {
  __shared__ __attribute__((aligned(1024))) char lds_a0[kOpBytes];
  __shared__ __attribute__((aligned(1024))) char lds_a1[kOpBytes];
  __shared__ __attribute__((aligned(1024))) char lds_b0[kOpBytes];
  __shared__ __attribute__((aligned(1024))) char lds_b1[kOpBytes];
  __shared__ __attribute__((aligned(16))) char lds_stage[kGemmThreads / 64][kStageBytes];
  __shared__ int s_tile[2];
  __shared__ int s_home;
  const Ring ring{{lds_a0, lds_a1}, {lds_b0, lds_b1}};

  // The descriptor table does not change during the launch: reading it
  // through the constant address space keeps its loads scalar (SGPRs) even
  // after the epilogue's stores.
  typedef const __attribute__((address_space(4))) MatDesc* DescPtr;
  typedef const __attribute__((address_space(4))) int32_t* PrefixPtr;
  const DescPtr descs = (DescPtr)args.descs;
  const PrefixPtr prefix = (PrefixPtr)args.prefix;
  const int total = args.total;
  const int wave = wave_id();
  if (threadIdx.x == 0) {
    s_home = xcc_id();
    const int t0 = grab_tile(args.queues, total, &s_home);
    s_tile[0] = t0;
    s_tile[1] = t0 >= 0 ? grab_tile(args.queues, total, &s_home) : -1;
  }
  __syncthreads();
  int t = __builtin_amdgcn_readfirstlane(s_tile[0]);
  if (t < 0) return;
  int slot = 1;

  // UPDATE and FINAL read their right operand, X, transposed.
  constexpr bool kXT = STAGE == ST_UPDATE || STAGE == ST_FINAL;
  static_assert(!kXT || (LAYOUT & kTiledX), "X read transposed needs the panel layout");
  auto prefetch = [&](const TileJob& j) { gemm_prefetch<kXT>(make_engine<kXT>(j, wave), ring); };
  int m = find_matrix(prefix, args.n, t);
  TileJob job = decode_tile<STAGE, LAYOUT, SPLIT>(descs[m], t - prefix[m], args);
  prefetch(job);
  for (;;) {
    f32x4 acc[kMi][kNi];
    gemm_run<kXT>(make_engine<kXT>(job, wave), job.K, ring, acc);
    block_barrier();  // every wave is past its last LDS read of this tile
    const int tn = __builtin_amdgcn_readfirstlane(s_tile[slot]);
    int mn = 0;
    TileJob jn{};
    if (tn >= 0) {
      mn = find_matrix(prefix, args.n, tn);
      jn = decode_tile<STAGE, LAYOUT, SPLIT>(descs[mn], tn - prefix[mn], args);
      prefetch(jn);
    }
    const bool leader = wave == 0 && lane_id() == 0;
    int after = -1;
    if (leader && tn >= 0) after = grab_tile(args.queues, total, &s_home);
    if constexpr (SPLIT)
      store_partial<STAGE>(descs[m], t - prefix[m], acc, wave);
    else
      gemm_epilogue<STAGE, PDT, LAYOUT>(args, descs[m], job, acc, wave, lds_stage[wave]);
    if (leader) s_tile[slot ^ 1] = after;
    if (tn < 0) break;
    t = tn;
    m = mn;
    job = jn;
    slot ^= 1;
  }
}

// The second launch of a K-split stage: one single-wave block per (split
// tile, wave sub-tile) of the group (prefix: prefix sums of each matrix's
// split tiles, 0 for an unsplit matrix), so a tile's eight 128 x 64 sub-tiles
// reduce on eight CUs. Each wave adds its accumulators' chunk partials in
// chunk order (((p0 + p1) + p2) + p3, in fp32) and runs the stage's epilogue
// on the sums, exactly as wave w of the unsplit launch runs it on its
// accumulators (an epilogue wave needs no other wave of its block).
template <int STAGE, int PDT, int LAYOUT>
__global__ __launch_bounds__(64) void pm_ns_reduce_kernel(GemmArgs args) {
  __shared__ __attribute__((aligned(16))) char lds_stage[kStageBytes];
  typedef const __attribute__((address_space(4))) MatDesc* DescPtr;
  typedef const __attribute__((address_space(4))) int32_t* PrefixPtr;
  typedef const __attribute__((address_space(1))) f32x4 glb_f32x4;
  const DescPtr descs = (DescPtr)args.descs;
  const PrefixPtr prefix = (PrefixPtr)args.prefix;
  const int t = blockIdx.x / (kGemmThreads / 64), wave = blockIdx.x % (kGemmThreads / 64);
  const int m = find_matrix(prefix, args.n, t);
  const int lane = lane_id();
  const int tile = t - prefix[m];
  const TileJob job = decode_tile<STAGE, LAYOUT>(descs[m], tile, args);  // chunk 0 of the tile
  const int tiles = stage_tiles<STAGE>(descs[m]), split = stage_split<STAGE>(descs[m]);
  float* const kpart = descs[m].kpart;
  // chunk by chunk, each chunk's 32 quads loaded together (one memory
  // latency a chunk), added in chunk order
  f32x4 acc[kMi][kNi];
  {
    const glb_f32x4* p0 = (const glb_f32x4*)partial_at(kpart, tiles, tile, 0, wave) + lane;
#pragma unroll
    for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
      for (int ni = 0; ni < kNi; ++ni) acc[mi][ni] = p0[(mi * kNi + ni) * 64];
  }
#pragma unroll
  for (int c = 1; c < kMaxKSplit; ++c) {
    if (c >= split) break;
    const glb_f32x4* pc = (const glb_f32x4*)partial_at(kpart, tiles, tile, c, wave) + lane;
    f32x4 v[kMi][kNi];
#pragma unroll
    for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
      for (int ni = 0; ni < kNi; ++ni) v[mi][ni] = pc[(mi * kNi + ni) * 64];
#pragma unroll
    for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
      for (int ni = 0; ni < kNi; ++ni) acc[mi][ni] += v[mi][ni];
  }
  gemm_epilogue<STAGE, PDT, LAYOUT>(args, descs[m], job, acc, wave, lds_stage);
}

// ============================================================ gram-form Q init
// Q = Z + a·I for every matrix of the group: the first polynomial of a
// gram-form segment, pan/optim/patch_muon.py:321-324 (Q = Z.clone(), then a
// is added to the diagonal in bf16). Block (x, y) copies the 64-row band x of
// matrix first + y; the padding rows and columns (beyond M) stay zero.
__global__ __launch_bounds__(kThreads) void pm_qinit_kernel(const MatDesc* descs, int32_t first, int32_t sz,
                                                            int32_t sq, float a, int32_t tiled) {
#pragma clang fp contract(off)
  const MatDesc& d = descs[first + blockIdx.y];
  const int r0 = blockIdx.x * kProTile;
  if (r0 >= d.Mp) return;
  const uint16_t* Z = d.S[sz];
  uint16_t* Q = d.S[sq];
  const int runs = d.Mp / 8;  // 16-byte runs per row
  for (int i = threadIdx.x; i < kProTile * runs; i += kThreads) {
    const int r = r0 + i / runs, c0 = (i % runs) * 8;
    u32x4 v = *(const u32x4*)(Z + ws_off(r, c0, d.Mp, tiled));
    const int e = r - c0;  // the diagonal element's place in this run, if any
    if (r < d.M && e >= 0 && e < 8) {
      const uint32_t w = v[e >> 1];
      const uint16_t z = (e & 1) ? (uint16_t)(w >> 16) : (uint16_t)(w & 0xffffu);
      const uint32_t q = f2bf(bf2f(z) + a);
      v[e >> 1] = (e & 1) ? ((w & 0xffffu) | (q << 16)) : ((w & 0xffff0000u) | q);
    }
    *(u32x4*)(Q + ws_off(r, c0, d.Mp, tiled)) = v;
  }
}

// ============================================================ elementwise
// muon_momentum_nesterov (pan/optim/muon_triton.py:25-51), fp32 math.
__global__ __launch_bounds__(kThreads) void pm_momentum_kernel(void* buf, int32_t bdt, const void* grad,
                                                               int32_t gdt, void* upd, int32_t udt,
                                                               int64_t n, float mu, int32_t nesterov) {
#pragma clang fp contract(off)
  const float omu = 1.0f - mu;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float g = load_elem(grad, gdt, i);
    const float m = load_elem(buf, bdt, i);
    const float nm = mu * m + omu * g;
    store_elem(buf, bdt, i, nm);
    store_elem(upd, udt, i, nesterov ? omu * g + mu * nm : nm);
  }
}

// _muon_step_param_{scalar,tensor}_kernel (pan/optim/muon_triton.py:111-161).
__global__ __launch_bounds__(kThreads) void pm_step_kernel(void* param, int32_t pdt, const void* upd,
                                                           int32_t udt, int64_t n, const float* lr_dev,
                                                           float wd, float adj, float wdf_host,
                                                           float neg_host) {
#pragma clang fp contract(off)
  float wdf = wdf_host, neg = neg_host;
  if (lr_dev) {
    const float lr = *lr_dev;
    wdf = 1.0f - lr * wd;
    neg = -(lr * adj);
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float p = load_elem(param, pdt, i);
    const float u = load_elem(upd, udt, i);
    store_elem(param, pdt, i, p * wdf + u * neg);
  }
}

}  // namespace pm
