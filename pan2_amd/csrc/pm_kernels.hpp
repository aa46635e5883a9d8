// Kernels of libpanmuon. Included once, by panmuon.hip.
#pragma once

#include "pm_device.hpp"
#include "pm_tiles.hpp"

namespace pm {

// ============================================================ prologue
//
// One 64x64 tile of X (orientation rows = short side) per block, covering the
// padded Mp x Np extent (tiles outside the parameter write zeros).
//   MODE_STEP: buf <- mu*buf + (1-mu)*g;  u <- (1-mu)*g + mu*buf  (nesterov)
//              (pan/optim/muon_triton.py:44-48; fp32 math)
//   MODE_NS:   u <- in
// X and Xᵀ get bf16(u) (torch casts to bf16 before NS, torch/optim/_muon.py:55)
// and partials[tile] = Σ bf16(u)², the tile's share of ‖X‖² (norm over the
// bf16 tensor, torch/optim/_muon.py:59).
__global__ __launch_bounds__(kThreads) void pm_prologue_kernel(ProArgs args) {
#pragma clang fp contract(off)
  __shared__ uint16_t tile[kProTile][kProTile + 2];
  __shared__ float red[kThreads / 64];

  const int t = blockIdx.x;
  const int mi = find_matrix(args.prefix, args.n, t);
  const MatDesc& d = args.descs[mi];
  const int lt = t - args.prefix[mi];
  const int ntn = d.Np / kProTile;
  const int ti = lt / ntn, tj = lt - ti * ntn;  // tile in X coordinates
  const int pr0 = d.trans ? tj * kProTile : ti * kProTile;  // param-layout origin
  const int pc0 = d.trans ? ti * kProTile : tj * kProTile;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  const float mu = args.mu, omu = 1.0f - args.mu;

  float ss = 0.0f;
#pragma unroll 4
  for (int i = 0; i < kProTile / 4; ++i) {
    const int r = ty + 4 * i;
    const int pr = pr0 + r, pc = pc0 + tx;
    float u = 0.0f;
    if (pr < d.rows && pc < d.cols) {
      const float g = load_elem(d.grad, d.g_dt, (int64_t)pr * d.g_ld + pc);
      if (args.mode == MODE_STEP) {
        const int64_t mo = (int64_t)pr * d.m_ld + pc;
        const float m = load_elem(d.mom, d.m_dt, mo);
        const float nm = mu * m + omu * g;
        store_elem(d.mom, d.m_dt, mo, nm);
        u = args.nesterov ? omu * g + mu * nm : nm;
      } else {
        u = g;
      }
    }
    const uint16_t ub = f2bf(u);
    const float uf = bf2f(ub);
    ss += uf * uf;
    tile[r][tx] = ub;
  }
  __syncthreads();

  // Param-layout copy goes to the buffer whose rows follow the param rows.
  uint16_t* dst_a = d.trans ? d.XT[0] : d.X[0];
  const int64_t ld_a = d.trans ? d.Mp : d.Np;
  uint16_t* dst_b = d.trans ? d.X[0] : d.XT[0];
  const int64_t ld_b = d.trans ? d.Np : d.Mp;
#pragma unroll 4
  for (int i = 0; i < kProTile / 4; ++i) {
    const int r = ty + 4 * i;
    dst_a[(int64_t)(pr0 + r) * ld_a + pc0 + tx] = tile[r][tx];
  }
#pragma unroll 4
  for (int i = 0; i < kProTile / 4; ++i) {
    const int c = ty + 4 * i;
    dst_b[(int64_t)(pc0 + c) * ld_b + pr0 + tx] = tile[tx][c];
  }

  ss = wave_sum(ss);
  if (tx == 0) red[ty] = ss;
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
// 8 waves, two per SIMD, in a 2 (rows) x 4 (cols) grid; each owns a 128x64
// sub-tile = 4x2 MFMA 32x32 tiles (128 fp32 accumulators per lane in AGPRs),
// so the two waves of a SIMD take turns issuing MFMAs while the other one
// waits on memory or the barrier.
//
// Operands stream through a kStages-deep ring of LDS stages, each holding
// kBK = 32 columns of K for both operands (2 x 256 rows x 64 B = 32 KiB).
// Global -> LDS copies are direct (buffer_load_dwordx4 ... lds): lane l of a
// load writes 16 B at the instruction's LDS base + 16*l, so one instruction
// fills 16 rows of 64 B and no VGPRs or ds_write instructions are spent on
// staging. Each wave issues kLoadsPerWave such loads per operand per stage.
//
// LDS rows are 64 B (four 16-byte chunks). Chunk c of row r is stored at
// chunk c ^ ((r >> 2) & 3): a ds_read_b128 phase serves 16 lanes reading 16
// consecutive rows at one chunk, and this spreads them over 16 distinct
// 16-byte bank groups of gfx950's 64-bank LDS (measured conflict-free).
constexpr int kStageBytes = 2 * kTile * kBK * 2;   // 32 KiB
constexpr int kOpBytes = kTile * kBK * 2;          // 16 KiB per operand
constexpr int kWaves = kGemmThreads / 64;          // 8
constexpr int kLoadsPerWave = kOpBytes / 1024 / kWaves;  // per operand, per stage
constexpr int kWaveRows = 128, kWaveCols = 64;     // per-wave sub-tile
constexpr int kMi = kWaveRows / 32, kNi = kWaveCols / 32;
constexpr int kQuads = kMi * kNi * 4;              // accumulator quads per lane

__device__ __forceinline__ __amdgpu_buffer_rsrc_t panel_rsrc(const uint16_t* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ lds_ptr_t to_lds(char* p) {
  return (lds_ptr_t)(__attribute__((address_space(3))) char*)p;
}

// s_waitcnt vmcnt(n), leaving expcnt and lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Block-wide barrier without the release fence of __syncthreads(), which
// would drain every in-flight LDS DMA. Callers wait for exactly the loads they
// need first; the "memory" clobber keeps the compiler from moving LDS
// accesses across it.
__device__ __forceinline__ void block_barrier() { asm volatile("s_barrier" ::: "memory"); }

// One LDS stage per __shared__ array, so the compiler's LDS-DMA tracking
// sees that reads of one stage do not depend on copies into the others.
struct Stages {
  char* s[kStages];
};

// Fragments of one LDS stage (two 16-deep K steps) of this wave's sub-tile.
struct Frags {
  bf16x8 a[2][kMi], b[2][kNi];
};

// Ping-pong schedule. Waves 0-3 (group A, rows 0-127) and 4-7 (group B, rows
// 128-255) put one wave of each group on every SIMD. Every wave runs the same
// program, a sequence of slots closed by block barriers:
//   M(-1) | C(0) | M(0) | C(1) | M(1) | ...
//   C(k): the 16 MFMAs of stage k, with this wave's share of the DMA loads of
//         stage k+3 (into buffer (k-1)%4) issued one per 4 MFMAs
//   M(k): the LDS reads of this wave's fragments of stage k+1
// but group B enters one slot later (one extra barrier up front, A adds one at
// the end), so on every SIMD one wave streams MFMAs while the other reads LDS.
// Issuing the DMA from the compute slot spreads it evenly over time: the
// CU's vector-memory address path (about 55 B/clk measured) stays well below
// saturation and an issue rarely blocks, whereas a burst of DMA issues at the
// start of a memory slot made that slot, and the barrier, wait for it.
// Ordering: stage k is read by A in slot 2k-1 and by B in slot 2k (closed by
// lgkmcnt(0)); A's C(k+1) (slot 2k+2) and B's C(k+1) (slot 2k+3) refill its
// buffer, after both. Each slot ends with this wave's share of the next stage
// anyone reads waited for (k+1 after C(k), k+2 after M(k)). Stage k lives in
// __shared__ array k % 4.
__device__ __forceinline__ void gemm_mainloop(const uint16_t* __restrict__ Lp, int ldl,
                                              const uint16_t* __restrict__ Rp, int ldr,
                                              int K, const Stages& st, f32x16 (&acc)[kMi][kNi]) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: scalar LDS bases
  const int wr = wave >> 2, wc = wave & 3;
  const bool group_b = wr != 0;
  const __amdgpu_buffer_rsrc_t rl = panel_rsrc(Lp, (uint32_t)kTile * ldl * 2);
  const __amdgpu_buffer_rsrc_t rr = panel_rsrc(Rp, (uint32_t)kTile * ldr * 2);
  // Load q (0..15) of an operand covers rows 16q .. 16q+15; this wave issues
  // q = wave*kLoadsPerWave + i. Lane l fills row 16q + l/4, stored chunk l%4,
  // i.e. logical chunk (l%4) ^ ((l/16) & 3).
  const int lchunk = (lane & 3) ^ ((lane >> 4) & 3);
  const int vl_off = (lane >> 2) * ldl * 2 + lchunk * 16;
  const int vr_off = (lane >> 2) * ldr * 2 + lchunk * 16;
  const int q0 = wave * kLoadsPerWave;
  // fragment reads: row rrow of a 32-row block, logical chunk 2*kk + kh
  const int rrow = lane & 31, kh = lane >> 5;
  const int rsw = (rrow >> 2) & 3;
  const int aofs = (wr * kWaveRows + rrow) * 64;
  const int bofs = kOpBytes + (wc * kWaveCols + rrow) * 64;

#pragma unroll
  for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
    for (int ni = 0; ni < kNi; ++ni) acc[mi][ni] = (f32x16){};

  constexpr int kDma = 2 * kLoadsPerWave;  // this wave's loads per stage
  auto issue = [&](char* dst, int kt) {
    const int ko = kt * kBK * 2;
#pragma unroll
    for (int i = 0; i < kLoadsPerWave; ++i) {
      const int q = q0 + i;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rl, to_lds(dst + q * 1024), 16, vl_off, q * 16 * ldl * 2 + ko, 0, 0);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, to_lds(dst + kOpBytes + q * 1024), 16, vr_off,
                                               q * 16 * ldr * 2 + ko, 0, 0);
    }
  };
  auto read = [&](Frags& f, const char* cur) {
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const int sw = ((2 * kk + kh) ^ rsw) << 4;
#pragma unroll
      for (int mi = 0; mi < kMi; ++mi) f.a[kk][mi] = *(const bf16x8*)(cur + aofs + mi * 2048 + sw);
#pragma unroll
      for (int ni = 0; ni < kNi; ++ni) f.b[kk][ni] = *(const bf16x8*)(cur + bofs + ni * 2048 + sw);
    }
  };
  constexpr int kMfma = 0x008, kVmemRead = 0x020;
  constexpr int kMfmas = 2 * kMi * kNi;
  static_assert(kMfmas % kDma == 0, "DMA issues must split the MFMAs evenly");
  // C slot: the stage's MFMAs, with `dst`'s DMA (stage kt) spread among them
  auto compute = [&](const Frags& f, char* dst, int kt, bool refill) {
    __builtin_amdgcn_s_setprio(1);
    if (refill) issue(dst, kt);
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
        for (int ni = 0; ni < kNi; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f.a[kk][mi], f.b[kk][ni], acc[mi][ni], 0, 0, 0);
    if (refill) {
#pragma unroll
      for (int i = 0; i < kDma; ++i) {
        __builtin_amdgcn_sched_group_barrier(kMfma, kMfmas / kDma, 0);
        __builtin_amdgcn_sched_group_barrier(kVmemRead, 1, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_setprio(0);
  };
  // this wave's DMA of a stage landed, with `pending` later stages in flight
  auto wait_loads = [&](int pending) {
    if (pending >= 2) wait_vmcnt<2 * kDma>();
    else if (pending == 1) wait_vmcnt<kDma>();
    else wait_vmcnt<0>();
  };
  auto slot_end = [&]() {
    __builtin_amdgcn_sched_barrier(0);
    block_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };

  // Every caller passes K a multiple of kTile (padded extents), so KT = K / kBK
  // is a multiple of kStages and at least 2 * kStages.
  static_assert(kStages == 4, "one __shared__ array per stage; schedule assumes four");
  const int KT = K / kBK;
  Frags f;

#pragma unroll
  for (int s = 0; s < kStages - 1; ++s) issue(st.s[s], s);
  wait_loads(2);  // stage 0 (stages 1, 2 may stay in flight)
  slot_end();
  if (group_b) slot_end();  // B enters one slot later
  // M(-1): fragments of stage 0; stage 1 landed (this wave's share)
  read(f, st.s[0]);
  __builtin_amdgcn_s_waitcnt(0xC07F);
  wait_loads(1);
  slot_end();

  // Stage k in buffer s = k % 4. `refill`: stage k+3 exists (DMA'd during
  // C(k)); `pend1` / `pend2`: stages allowed in flight after stage k+1 at the
  // end of C(k) / after stage k+2 at the end of M(k); `next` / `next2`: stage
  // k+1 / k+2 exists.
  auto stage = [&](int s, int k, bool refill, int pend1, int pend2, bool next, bool next2) {
    compute(f, st.s[(s + kStages - 1) % kStages], k + kStages - 1, refill);
    if (next) wait_loads(pend1);
    slot_end();
    if (next) {
      read(f, st.s[(s + 1) % kStages]);
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): buffer (k+1)%4 read before it is refilled
    }
    if (next2) wait_loads(pend2);
    slot_end();
  };

  for (int k0 = 0; k0 < KT - kStages; k0 += kStages) {
#pragma unroll
    for (int s = 0; s < kStages; ++s) stage(s, k0 + s, true, 2, 1, true, true);
  }
  const int k0 = KT - kStages;
  // tail: stages issued by the end of C(k) / M(k) run to min(KT-1, k+3)
  stage(0, k0, true, 2, 1, true, true);      // issues KT-1
  stage(1, k0 + 1, false, 1, 0, true, true);
  stage(2, k0 + 2, false, 0, 0, true, false);
  stage(3, k0 + 3, false, 0, 0, false, false);
  if (!group_b) slot_end();  // match B's extra barrier
}

// Visits this lane's accumulators as quads: f(i, p0, q, x) gets rows
// p0..p0+3 of column q, i the quad's index. (v_mfma 32x32 layout: lane l,
// register r -> row 8*(r/4) + 4*(l/32) + r%4, column l%32.) Indices are
// compile-time after unrolling, so the accumulators stay in registers.
template <class F>
__device__ __forceinline__ void for_each_quad(const f32x16 (&acc)[kMi][kNi], int pbase, int qbase, F&& f) {
#pragma unroll
  for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
    for (int ni = 0; ni < kNi; ++ni)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float x[4] = {acc[mi][ni][4 * g], acc[mi][ni][4 * g + 1], acc[mi][ni][4 * g + 2],
                            acc[mi][ni][4 * g + 3]};
        f((mi * kNi + ni) * 4 + g, pbase + mi * 32 + 8 * g, qbase + ni * 32, x);
      }
}

// Loads, for every quad of this lane, the 4 consecutive elements T[q][p0..p0+3]
// of a row-major matrix T (ld elements): 8-byte loads, all issued before use.
__device__ __forceinline__ void load_quads(u16x4 (&v)[kQuads], const uint16_t* __restrict__ T, int64_t ld,
                                           int pbase, int qbase) {
#pragma unroll
  for (int mi = 0; mi < kMi; ++mi)
#pragma unroll
    for (int ni = 0; ni < kNi; ++ni)
#pragma unroll
      for (int g = 0; g < 4; ++g)
        v[(mi * kNi + ni) * 4 + g] =
            *(const u16x4*)(T + (int64_t)(qbase + ni * 32) * ld + pbase + mi * 32 + 8 * g);
}

// Operands and tile of one work item of stage STAGE.
struct TileJob {
  const uint16_t* L;
  const uint16_t* R;
  int ldl, ldr, K;
  int ti, tj;
};

template <int STAGE>
__device__ __forceinline__ TileJob decode_tile(const MatDesc& d, int lt, int cur) {
  TileJob j;
  int P, Q;
  bool sym = false;
  if (STAGE == ST_GRAM) {
    j.L = j.R = d.X[cur]; j.ldl = j.ldr = d.Np; j.K = d.Np; P = Q = d.Mp; sym = true;
  } else if (STAGE == ST_POLY) {
    j.L = j.R = d.A; j.ldl = j.ldr = d.Mp; j.K = d.Mp; P = Q = d.Mp; sym = true;
  } else if (STAGE == ST_UPDATE || !d.trans) {
    // C (Mp x Np) = B · X, X supplied as Xᵀ rows
    j.L = d.B; j.ldl = d.Mp; j.R = d.XT[cur]; j.ldr = d.Mp; j.K = d.Mp; P = d.Mp; Q = d.Np;
  } else {
    // tall FINAL: C (Np x Mp) = Xᵀ · B = (B X)ᵀ, already in param layout
    j.L = d.XT[cur]; j.ldl = d.Mp; j.R = d.B; j.ldr = d.Mp; j.K = d.Mp; P = d.Np; Q = d.Mp;
  }
  if (sym) {
    sym_tile(lt, P / kTile, j.ti, j.tj);
  } else {
    full_tile(lt, P / kTile, Q / kTile, j.ti, j.tj);
  }
  return j;
}

// One Newton–Schulz stage over every matrix of the group.
//   GRAM   A = s·X Xᵀ            (s = 1/‖X‖² at iteration 0, folding
//                                 X.div_(norm) of torch/optim/_muon.py:59)
//   POLY   B = c·A A + b·A        (torch.addmm(A, A, A, beta=b, alpha=c), :63-65)
//   UPDATE X' = s·(a·X + B X)     (torch.addmm(X, B, X, beta=a), :66), written
//                                 as X' and X'ᵀ
//   FINAL  O = bf16(s·(a·X + B X)) then p <- p·(1-lr·wd) - lr·adj·O
//          (pan/optim/muon_triton.py:130-131), or O stored (MODE_NS)
// GRAM and POLY are symmetric: only upper-triangle tiles are computed and
// each off-diagonal tile is also stored transposed. Every result is rounded
// to bf16 where torch rounds it.
template <int STAGE>
__global__ __launch_bounds__(kGemmThreads, 1) void pm_ns_gemm_kernel(GemmArgs args) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(1024))) char lds0[kStageBytes];
  __shared__ __attribute__((aligned(1024))) char lds1[kStageBytes];
  __shared__ __attribute__((aligned(1024))) char lds2[kStageBytes];
  __shared__ __attribute__((aligned(1024))) char lds3[kStageBytes];
  static_assert(kStages == 4, "one __shared__ array per stage");
  const Stages st{{lds0, lds1, lds2, lds3}};

  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int m = find_matrix(args.prefix, args.n, t);
  const MatDesc& d = args.descs[m];
  const int cur = args.cur;
  const TileJob job = decode_tile<STAGE>(d, t - args.prefix[m], cur);

  f32x16 acc[kMi][kNi];
  gemm_mainloop(job.L + (int64_t)job.ti * kTile * job.ldl, job.ldl, job.R + (int64_t)job.tj * kTile * job.ldr,
                job.ldr, job.K, st, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pbase = job.ti * kTile + (wave >> 2) * kWaveRows + 4 * (lane >> 5);
  const int qbase = job.tj * kTile + (wave & 3) * kWaveCols + (lane & 31);

  // Epilogue operands are read as quads T[q][p0..p0+3] from the orientation
  // whose rows run along this lane's 4 consecutive output rows p: A is
  // symmetric, and X / Xᵀ hold the same values transposed. All loads are
  // issued before any store, so no load waits behind stores in vmcnt order.
  if (STAGE == ST_GRAM || STAGE == ST_POLY) {
    uint16_t* C = (STAGE == ST_GRAM) ? d.A : d.B;
    const int64_t ldc = d.Mp;
    const float s = (STAGE == ST_GRAM && args.first) ? d.scales[0] : 1.0f;
    const float cb = args.b, cc = args.c;
    const bool mirror = job.ti != job.tj;
    u16x4 av[kQuads];
    if (STAGE == ST_POLY) load_quads(av, d.A, ldc, pbase, qbase);
    for_each_quad(acc, pbase, qbase, [&](int i, int p0, int q, const float (&x)[4]) {
      u16x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float v = (STAGE == ST_GRAM) ? x[r] * s : cc * x[r] + cb * bf2f(av[i][r]);
        o[r] = f2bf(v);
        C[(int64_t)(p0 + r) * ldc + q] = o[r];
      }
      if (mirror) *(u16x4*)(C + (int64_t)q * ldc + p0) = o;
    });
    return;
  }

  const float s = args.first ? d.scales[1] : 1.0f;
  const float ca = args.a;
  if (STAGE == ST_UPDATE) {
    uint16_t* Xn = d.X[cur ^ 1];
    uint16_t* XTn = d.XT[cur ^ 1];
    const int64_t ldx = d.Np, ldxt = d.Mp;
    u16x4 xv[kQuads];
    load_quads(xv, d.XT[cur], ldxt, pbase, qbase);  // X[p][q] = Xᵀ[q][p]
    for_each_quad(acc, pbase, qbase, [&](int i, int p0, int q, const float (&x)[4]) {
      u16x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        o[r] = f2bf((ca * bf2f(xv[i][r]) + x[r]) * s);
        Xn[(int64_t)(p0 + r) * ldx + q] = o[r];
      }
      *(u16x4*)(XTn + (int64_t)q * ldxt + p0) = o;
    });
    return;
  }

  // ST_FINAL: P rows / Q cols are the param's own rows / cols; the a·X term
  // is X[p][q] (wide) or Xᵀ[p][q] (tall), read from the other orientation.
  // Work goes one 32-row band (16 quads) at a time to bound register use; a
  // band's loads are all issued before its stores.
  const uint16_t* T = d.trans ? d.X[cur] : d.XT[cur];
  const int64_t ldt = d.trans ? d.Np : d.Mp;
  const int rows = d.rows, cols = d.cols;
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
  auto final_bands = [&](auto* P, auto load, auto store, bool step) {
#pragma unroll
    for (int mi = 0; mi < kMi; ++mi) {
      constexpr int kBand = kNi * 4;  // quads per 32-row band
      u16x4 xv[kBand];
      float pv[kBand][4];
#pragma unroll
      for (int j = 0; j < kBand; ++j) {
        const int ni = j >> 2, g = j & 3;
        const int p0 = pbase + mi * 32 + 8 * g, q = qbase + ni * 32;
        xv[j] = *(const u16x4*)(T + (int64_t)q * ldt + p0);
        if (step) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int p = p0 + r;
            pv[j][r] = (p < rows && q < cols) ? load(P + (int64_t)p * ldp + q) : 0.0f;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < kBand; ++j) {
        const int ni = j >> 2, g = j & 3;
        const int p0 = pbase + mi * 32 + 8 * g, q = qbase + ni * 32;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int p = p0 + r;
          const float o = bf2f(f2bf((ca * bf2f(xv[j][r]) + acc[mi][ni][4 * g + r]) * s));
          if (p < rows && q < cols) store(P + (int64_t)p * ldp + q, step ? pv[j][r] * wdf + o * neg : o);
        }
      }
    }
  };
  auto ld_f32 = [](const float* a) { return *a; };
  auto st_f32 = [](float* a, float v) { *a = v; };
  auto ld_bf16 = [](const uint16_t* a) { return bf2f(*a); };
  auto st_bf16 = [](uint16_t* a, float v) { *a = f2bf(v); };
  if (args.mode == MODE_NS) final_bands((uint16_t*)d.param, ld_bf16, st_bf16, false);
  else if (d.p_dt == DT_F32) final_bands((float*)d.param, ld_f32, st_f32, true);
  else final_bands((uint16_t*)d.param, ld_bf16, st_bf16, true);
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

// Copies a by-value chunk of the descriptor table into the workspace.
struct BlobChunk {
  uint32_t w[512];
};
__global__ void pm_upload_kernel(BlobChunk chunk, uint32_t* dst, int nwords) {
  for (int i = threadIdx.x; i < nwords; i += blockDim.x) dst[i] = chunk.w[i];
}

}  // namespace pm
