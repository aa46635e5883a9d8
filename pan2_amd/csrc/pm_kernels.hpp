// Kernels of libpanmuon. Included once, by panmuon.hip.
#pragma once

#include "pm_device.hpp"

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
// 4 waves in a 2x2 grid, each owning 128x128 = 4x4 MFMA 32x32 tiles
// (256 fp32 accumulators per lane, held in AGPRs). K advances 64 at a time
// through a double-buffered LDS stage of 2 x (256x64 + 256x64) bf16 = 128 KiB.
// LDS rows are 128 B; the 16-byte chunk index is XOR-swizzled with (row & 7)
// so the 8 lanes of one ds_read_b128 phase hit 8 distinct chunks.
// Global loads are buffer loads: one per-lane offset VGPR per operand, the
// row-block and K offsets in SGPRs, and reads past the panel return zero.

__device__ __forceinline__ __amdgpu_buffer_rsrc_t panel_rsrc(const uint16_t* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void*)base, (short)0, (int)bytes, 0x00020000);
}

__device__ __forceinline__ void gemm_mainloop(const uint16_t* __restrict__ Lp, int ldl,
                                              const uint16_t* __restrict__ Rp, int ldr,
                                              int K, char* lds, f32x16 (&acc)[4][4]) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int c = tid & 7, r0 = tid >> 3;
  const __amdgpu_buffer_rsrc_t rl = panel_rsrc(Lp, (uint32_t)kTile * ldl * 2);
  const __amdgpu_buffer_rsrc_t rr = panel_rsrc(Rp, (uint32_t)kTile * ldr * 2);
  const int vl_off = r0 * ldl * 2 + c * 16;
  const int vr_off = r0 * ldr * 2 + c * 16;
  const int sl = 32 * ldl * 2, sr = 32 * ldr * 2;  // bytes per 32 rows
  const int wofs = r0 * 128 + ((c ^ (r0 & 7)) << 4);
  const int rrow = lane & 31, kh = lane >> 5;
  const int aofs = (wm * 128 + rrow) * 128;
  const int bofs = 32768 + (wn * 128 + rrow) * 128;

#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = (f32x16){};

  u32x4 vl[8], vr[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    vl[j] = __builtin_amdgcn_raw_buffer_load_b128(rl, vl_off, j * sl, 0);
    vr[j] = __builtin_amdgcn_raw_buffer_load_b128(rr, vr_off, j * sr, 0);
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    *(u32x4*)(lds + wofs + j * 4096) = vl[j];
    *(u32x4*)(lds + 32768 + wofs + j * 4096) = vr[j];
  }
  __syncthreads();

  const int KT = K / kBK;
  for (int kt = 0; kt < KT; ++kt) {
    char* cur = lds + (kt & 1) * 65536;
    char* nxt = lds + ((kt + 1) & 1) * 65536;
    const bool more = kt + 1 < KT;
    if (more) {
      const int ko = (kt + 1) * kBK * 2;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        vl[j] = __builtin_amdgcn_raw_buffer_load_b128(rl, vl_off, j * sl + ko, 0);
        vr[j] = __builtin_amdgcn_raw_buffer_load_b128(rr, vr_off, j * sr + ko, 0);
      }
    }
#pragma unroll
    for (int kk = 0; kk < kBK / 16; ++kk) {
      const int sw = ((2 * kk + kh) ^ (rrow & 7)) << 4;
      bf16x8 a[4], b[4];
#pragma unroll
      for (int mi = 0; mi < 4; ++mi) a[mi] = *(const bf16x8*)(cur + aofs + mi * 4096 + sw);
#pragma unroll
      for (int ni = 0; ni < 4; ++ni) b[ni] = *(const bf16x8*)(cur + bofs + ni * 4096 + sw);
#pragma unroll
      for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
          acc[mi][ni] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[mi], b[ni], acc[mi][ni], 0, 0, 0);
    }
    if (more) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        *(u32x4*)(nxt + wofs + j * 4096) = vl[j];
        *(u32x4*)(nxt + 32768 + wofs + j * 4096) = vr[j];
      }
    }
    __syncthreads();
  }
}

// Visits this lane's accumulators as quads: f(p0, q, x) gets rows p0..p0+3 of
// column q. (v_mfma 32x32 layout: lane l, register r -> row 8*(r/4) +
// 4*(l/32) + r%4, column l%32.) Indices are compile-time after unrolling, so
// the accumulators stay in registers.
template <class F>
__device__ __forceinline__ void for_each_quad(const f32x16 (&acc)[4][4], int pbase, int qbase, F&& f) {
#pragma unroll
  for (int mi = 0; mi < 4; ++mi)
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float x[4] = {acc[mi][ni][4 * g], acc[mi][ni][4 * g + 1], acc[mi][ni][4 * g + 2],
                            acc[mi][ni][4 * g + 3]};
        f(pbase + mi * 32 + 8 * g, qbase + ni * 32, x);
      }
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
    const int nt = P / kTile;
    int rem = lt, i = 0;
    while (rem >= nt - i) { rem -= nt - i; ++i; }
    j.ti = i; j.tj = i + rem;
  } else {
    const int ntq = Q / kTile;
    j.ti = lt / ntq; j.tj = lt - j.ti * ntq;
  }
  (void)P;
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
__global__ __launch_bounds__(kThreads, 1) void pm_ns_gemm_kernel(GemmArgs args) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) char lds[4 * 32768];

  const int t = xcd_remap(blockIdx.x, gridDim.x);
  const int m = find_matrix(args.prefix, args.n, t);
  const MatDesc& d = args.descs[m];
  const int cur = args.cur;
  const TileJob job = decode_tile<STAGE>(d, t - args.prefix[m], cur);

  f32x16 acc[4][4];
  gemm_mainloop(job.L + (int64_t)job.ti * kTile * job.ldl, job.ldl, job.R + (int64_t)job.tj * kTile * job.ldr,
                job.ldr, job.K, lds, acc);

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int pbase = job.ti * kTile + (wave >> 1) * 128 + 4 * (lane >> 5);
  const int qbase = job.tj * kTile + (wave & 1) * 128 + (lane & 31);

  if (STAGE == ST_GRAM || STAGE == ST_POLY) {
    uint16_t* C = (STAGE == ST_GRAM) ? d.A : d.B;
    const uint16_t* A = d.A;
    const int64_t ldc = d.Mp;
    const float s = (STAGE == ST_GRAM && args.first) ? d.scales[0] : 1.0f;
    const float cb = args.b, cc = args.c;
    const bool mirror = job.ti != job.tj;
    for_each_quad(acc, pbase, qbase, [&](int p0, int q, const float (&x)[4]) {
      u16x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t off = (int64_t)(p0 + r) * ldc + q;
        const float v = (STAGE == ST_GRAM) ? x[r] * s : cc * x[r] + cb * bf2f(A[off]);
        o[r] = f2bf(v);
        C[off] = o[r];
      }
      if (mirror) *(u16x4*)(C + (int64_t)q * ldc + p0) = o;
    });
    return;
  }

  const float s = args.first ? d.scales[1] : 1.0f;
  const float ca = args.a;
  if (STAGE == ST_UPDATE) {
    const uint16_t* Xc = d.X[cur];
    uint16_t* Xn = d.X[cur ^ 1];
    uint16_t* XTn = d.XT[cur ^ 1];
    const int64_t ldx = d.Np, ldxt = d.Mp;
    for_each_quad(acc, pbase, qbase, [&](int p0, int q, const float (&x)[4]) {
      u16x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t off = (int64_t)(p0 + r) * ldx + q;
        o[r] = f2bf((ca * bf2f(Xc[off]) + x[r]) * s);
        Xn[off] = o[r];
      }
      *(u16x4*)(XTn + (int64_t)q * ldxt + p0) = o;
    });
    return;
  }

  // ST_FINAL: P rows / Q cols are the param's own rows / cols.
  const uint16_t* Xt = d.trans ? d.XT[cur] : d.X[cur];
  const int64_t ldx = d.trans ? d.Mp : d.Np;
  const int rows = d.rows, cols = d.cols;
  const int64_t ldp = d.p_ld;
  if (args.mode == MODE_NS) {
    uint16_t* out = (uint16_t*)d.param;
    for_each_quad(acc, pbase, qbase, [&](int p0, int q, const float (&x)[4]) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = p0 + r;
        const float v = (ca * bf2f(Xt[(int64_t)p * ldx + q]) + x[r]) * s;
        if (p < rows && q < cols) out[(int64_t)p * ldp + q] = f2bf(v);
      }
    });
    return;
  }
  float wdf, neg;
  if (args.lr_dev) {
    const float lr = *args.lr_dev;
    wdf = 1.0f - lr * args.wd;
    neg = -(lr * d.adj_ratio);
  } else {
    wdf = args.wdf_host;
    neg = d.neg_lr_host;
  }
  if (d.p_dt == DT_F32) {
    float* P = (float*)d.param;
    for_each_quad(acc, pbase, qbase, [&](int p0, int q, const float (&x)[4]) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = p0 + r;
        const float o = bf2f(f2bf((ca * bf2f(Xt[(int64_t)p * ldx + q]) + x[r]) * s));
        if (p < rows && q < cols) {
          const int64_t po = (int64_t)p * ldp + q;
          P[po] = P[po] * wdf + o * neg;
        }
      }
    });
  } else {
    uint16_t* P = (uint16_t*)d.param;
    for_each_quad(acc, pbase, qbase, [&](int p0, int q, const float (&x)[4]) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int p = p0 + r;
        const float o = bf2f(f2bf((ca * bf2f(Xt[(int64_t)p * ldx + q]) + x[r]) * s));
        if (p < rows && q < cols) {
          const int64_t po = (int64_t)p * ldp + q;
          P[po] = f2bf(bf2f(P[po]) * wdf + o * neg);
        }
      }
    });
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

// Copies a by-value chunk of the descriptor table into the workspace.
struct BlobChunk {
  uint32_t w[512];
};
__global__ void pm_upload_kernel(BlobChunk chunk, uint32_t* dst, int nwords) {
  for (int i = threadIdx.x; i < nwords; i += blockDim.x) dst[i] = chunk.w[i];
}

}  // namespace pm
