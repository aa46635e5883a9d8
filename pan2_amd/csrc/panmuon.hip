// libpanmuon — C ABI (include/panmuon.h) over the gfx950 kernels of
// pm_kernels.hpp. Host code only plans workspace, groups matrices, uploads
// the per-call descriptor table and enqueues launches on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/panmuon.h"
#include "pm_kernels.hpp"
#include "pm_small.hpp"
#include "pm_adam.hpp"

using namespace pm;

static_assert(sizeof(MatDesc) % 8 == 0, "descriptor alignment");
// ABI layout, mirrored by the ctypes structures of pan2_amd/_lib.py
static_assert(sizeof(pm_matrix) == 88, "pm_matrix layout");
static_assert(sizeof(pm_ns_matrix) == 56, "pm_ns_matrix layout");
static_assert(sizeof(pm_hparams) == 56, "pm_hparams layout");
static_assert(sizeof(pm_adam_tensor) == 72, "pm_adam_tensor layout");
static_assert(sizeof(pm_adam_hparams) == 48, "pm_adam_hparams layout");

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(PM_EHIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr size_t kAlign = 256;
// Largest extent: a 256-row operand panel of the padded long side spans
// 256 * Np * 2 bytes, which a buffer descriptor's 32-bit size must cover.
constexpr int kMaxExtent = (1 << 23) - kTile;
// Groups of at most 12 GiB: on config 5 (360 matrices) 12 GiB measured
// 0.6% faster per step than 16 GiB and 8 GiB, and 1.1% faster than 32 GiB
// (fewer, larger groups are slower).
constexpr uint64_t kDefaultWorkspaceLimit = 12ull << 30;  // 12 GiB

size_t align_up(size_t x, size_t a = kAlign) { return (x + a - 1) / a * a; }
int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Shape plan of one matrix: orientation and padded extents. A matrix whose
// short side is at most 128 is "small": padded to 128 and run by the
// small-matrix kernels (pm_small.hpp) instead of the grouped GEMM engine.
struct Plan {
  int32_t rows, cols, trans, M, N, Mp, Np;
  bool small;
  int32_t ks_gram, ks_symm, ks_full;  // K-split chunks per tile (split_call), 1: unsplit
  size_t kpart;                       // bytes of fp32 partial tiles (the largest split stage's)
  size_t ws;  // workspace bytes of this matrix (with kpart once split_call has run)
  double flops;
};

// Square Mp x Mp work matrices per matrix: A and B (standard form) or R, Z,
// RZ and two Q (gram form); a small matrix keeps its work matrices in LDS and
// needs one, the S its core launch hands to its apply launch.
int square_bufs(int form, bool small) { return small ? 1 : form == NS_GRAM ? 5 : 2; }

Plan make_plan(int64_t rows, int64_t cols, int form) {
  Plan p{};
  p.rows = (int32_t)rows;
  p.cols = (int32_t)cols;
  p.trans = rows > cols;
  p.M = (int32_t)std::min(rows, cols);
  p.N = (int32_t)std::max(rows, cols);
  p.small = p.M <= kSm;
  p.Mp = p.small ? kSm : (int32_t)round_up(p.M, kTile);
  p.Np = (int32_t)round_up(p.N, kTile);
  const size_t x = align_up((size_t)p.Mp * p.Np * 2);
  const size_t a = align_up((size_t)p.Mp * p.Mp * 2);
  const size_t part = align_up((size_t)(p.Mp / kProTile) * (p.Np / kProTile) * 4);  // (covers every run count)
  // X ping-pong, the square work matrices, the prologue partials; split_call
  // adds the K-split partials
  p.ks_gram = p.ks_symm = p.ks_full = 1;
  p.kpart = 0;
  p.ws = 2 * x + (size_t)square_bufs(form, p.small) * a + part + kAlign;
  const double M = p.M, N = p.N;
  p.flops = M * (M + 1) * N + M * M * (M + 1) + 2 * M * M * N;
  return p;
}

// Iteration at which the gram form applies Q to X and recomputes the gram
// (pan/optim/patch_muon.py:286: reset_iterations = {2} when ns_steps > 2), or -1.
int gram_reset(int steps) { return steps > 2 ? 2 : -1; }

// GEMM launches of one group (an upper bound for the gram form): standard =
// GRAM, POLY and UPDATE/FINAL per iteration; gram = two grams, at most four
// symmetric products per iteration, the apply at the reset and FINAL.
int gemm_launches(const pm_hparams* hp) {
  // x2: a stage over both unsplit and K-split matrices is two GEMM launches
  return 2 * (hp->ns_form == NS_GRAM ? 4 * hp->ns_steps + 4 : 3 * hp->ns_steps);
}

// Descriptor table layout:
//   descs[n] | pro_prefix[n+1] | per stage (GRAM, symmetric products, UPDATE / FINAL) three prefix sums
//   [n+1]: tiles of unsplit matrices, work items (tiles x K-split chunks) of split ones, tiles of split
//   ones (the reduce launch) | queues[launches][kXcds] | coeffs
// The queue counters are uploaded as zeros with the rest of the table, so
// every GEMM launch starts with empty counters without a memset. coeffs holds
// the (a, b, c) of every iteration, which the small-matrix core launch reads.
constexpr int kMaxSteps = 99;
constexpr size_t kCoeffBytes = (3 * kMaxSteps * 4 + kAlign - 1) / kAlign * kAlign;
constexpr int kPrefixArrays = 10;
size_t queue_offset(int n) { return align_up((size_t)n * sizeof(MatDesc)) + kPrefixArrays * align_up((size_t)(n + 1) * 4); }
size_t coeff_offset(int n, int launches) { return queue_offset(n) + align_up((size_t)launches * kXcds * 4); }
size_t table_bytes(int n, int launches) { return coeff_offset(n, launches) + kCoeffBytes; }

// Persistent GEMM grid: one block per CU (the kernel's LDS allows no more),
// never more blocks than tiles.
int gemm_grid(int tiles) {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return std::max(1, std::min(tiles, n));
}

bool valid_dtype(int32_t dt) { return dt == PM_DTYPE_F32 || dt == PM_DTYPE_BF16; }

int check_hparams(const pm_hparams* hp) {
  if (!hp) return fail(PM_EINVAL, "hparams is NULL");
  if (hp->ns_steps < 1 || hp->ns_steps > kMaxSteps)
    return fail(PM_EUNSUPPORTED, "ns_steps must be in [1, %d], got %d", kMaxSteps, hp->ns_steps);
  if (hp->ns_form != PM_NS_STANDARD && hp->ns_form != PM_NS_GRAM)
    return fail(PM_EINVAL, "ns_form must be PM_NS_STANDARD or PM_NS_GRAM, got %d", hp->ns_form);
  if (!(hp->eps >= 0.0f)) return fail(PM_EINVAL, "eps must be >= 0");
  return PM_OK;
}

int check_extent(int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return fail(PM_EINVAL, "matrix extents must be positive, got %lldx%lld",
                                          (long long)rows, (long long)cols);
  // 256 rows of the long side must stay within a 32-bit buffer descriptor
  if (rows > kMaxExtent || cols > kMaxExtent)
    return fail(PM_EUNSUPPORTED, "matrix %lldx%lld: each extent must be at most %d", (long long)rows,
                (long long)cols, kMaxExtent);
  // keeps every per-launch tile count and prefix sum within int32
  if (rows * cols > (1ll << 40))
    return fail(PM_EINVAL, "matrix %lldx%lld is too large", (long long)rows, (long long)cols);
  return PM_OK;
}

// Work item counts of one matrix.
// Prologue blocks of one matrix (kProRun tiles each), one Σx² partial per block.
int32_t pro_tiles(const Plan& p) { return (p.Mp / kProTile) * (p.Np / (kProTile * kProRun)); }
int32_t sym_tiles(const Plan& p) {
  const int32_t nt = p.Mp / kTile;
  return nt * (nt + 1) / 2;
}
int32_t full_tiles(const Plan& p) {
  return p.small ? p.Np / kSmApplyCols : (p.Mp / kTile) * (p.Np / kTile);
}

// One matrix of a call, whatever the entry point.
struct Item {
  Plan plan;
  MatDesc desc;
};

// K-split of a call's engine matrices (k_split in pm_tiles.hpp). A stage
// splits only when all of the call's engine matrices together hold so few of
// its tiles that most of the chip would sit idle; each matrix then cuts its
// tiles into as many chunks as its shape allows within that budget. On a call
// whose tiles fill the chip, the chunks' fp32 partials would cost more than
// the idle CUs they fill (measured: 48 x 2048² runs 8.0 ms unsplit, 15.7 ms
// split). The choice depends on the call only, so a call gives the same bits
// in any workspace grouping and through either step entry point. A matrix
// whose partials would take its workspace past the allocation-free step's
// scratch stays unsplit, so that step takes every matrix it would take
// unsplit. GRAM contracts over Np, the symmetric products and UPDATE / FINAL
// over Mp.
void split_call(std::vector<Item>& items) {
  constexpr size_t kTableRoom = 1u << 20;  // above any one-matrix descriptor table
  int64_t tiles[3] = {0, 0, 0};
  for (const Item& it : items)
    if (!it.plan.small) {
      tiles[0] += sym_tiles(it.plan);
      tiles[1] += sym_tiles(it.plan);
      tiles[2] += full_tiles(it.plan);
    }
  int call[3];
  for (int st = 0; st < 3; ++st) call[st] = (int)std::min<int64_t>(tiles[st], kSplitItems + 1);
  const size_t tile_bytes = (size_t)kTile * kTile * 4;
  for (Item& it : items) {
    Plan& p = it.plan;
    if (p.small) continue;
    p.ks_gram = k_split(p.Mp, call[0], p.Np / 64);
    p.ks_symm = k_split(p.Mp, call[1], p.Mp / 64);
    p.ks_full = k_split(p.Mp, call[2], p.Mp / 64);
    size_t kp = 0;
    if (p.ks_gram > 1) kp = std::max(kp, (size_t)sym_tiles(p) * p.ks_gram * tile_bytes);
    if (p.ks_symm > 1) kp = std::max(kp, (size_t)sym_tiles(p) * p.ks_symm * tile_bytes);
    if (p.ks_full > 1) kp = std::max(kp, (size_t)full_tiles(p) * p.ks_full * tile_bytes);
    if (kp && p.ws + kp + kTableRoom > PM_NOALLOC_SCRATCH_BYTES) {
      p.ks_gram = p.ks_symm = p.ks_full = 1;
      kp = 0;
    }
    p.kpart = kp;
    p.ws += kp;
  }
}

int load_table_by_kernel(const char* src, size_t bytes, char* dst, hipStream_t stream);

// Descriptor uploads go through pinned staging buffers: the host table is
// copied into one, and an asynchronous copy on the caller's stream moves it
// to the workspace, so the host does not wait for the stream. On a stream
// under graph capture the table goes in as kernel arguments instead
// (load_table_by_kernel): a captured copy would read the staging buffer again
// at every replay, after later calls have reused it. A buffer is
// reused once the event recorded after its copy has completed (the smallest
// free one that holds the table, else the largest free one, regrown). The
// pool grows while every buffer is still in flight (calls queued far behind
// the GPU), up to kMaxStaging buffers and kMaxStagingBytes of pinned memory
// per device; a call that finds no free buffer at either limit waits for the
// oldest upload of its device (the lowest sequence number) and reuses that
// buffer. A device's pinned footprint is therefore at most kMaxStagingBytes,
// or its largest single table if that is larger.
struct Staging {
  int device;
  void* host;
  size_t bytes;
  hipEvent_t done;
  uint64_t seq;  // order in which the buffer's current copy was enqueued
};
constexpr size_t kMaxStaging = 1024;
constexpr size_t kMaxStagingBytes = 64ull << 20;
constexpr size_t kStagingMin = 1 << 16;  // smallest buffer (64 KiB)
std::mutex g_stage_mu;
std::vector<Staging> g_stage;
uint64_t g_stage_seq = 0;

int upload(const void* src, size_t bytes, void* dst, hipStream_t stream) {
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(stream, &capture);
  if (e != hipSuccess) return hip_fail(e, "hipStreamIsCapturing");
  if (capture != hipStreamCaptureStatusNone) return load_table_by_kernel((const char*)src, bytes, (char*)dst, stream);
  int dev = 0;
  e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  std::lock_guard<std::mutex> lock(g_stage_mu);
  Staging* s = nullptr;
  size_t mine = 0, mine_bytes = 0, oldest = SIZE_MAX;
  for (size_t i = 0; i < g_stage.size(); ++i) {
    Staging& c = g_stage[i];
    if (c.device != dev) continue;
    ++mine;
    mine_bytes += c.bytes;
    if (oldest == SIZE_MAX || c.seq < g_stage[oldest].seq) oldest = i;
    if (hipEventQuery(c.done) != hipSuccess) continue;  // its copy is still queued
    const bool fits = c.bytes >= bytes, s_fits = s && s->bytes >= bytes;
    if (!s || (fits && (!s_fits || c.bytes < s->bytes)) || (!fits && !s_fits && c.bytes > s->bytes)) s = &c;
  }
  const size_t want = std::max<size_t>(align_up(bytes, kStagingMin), kStagingMin);
  if (!s && mine > 0 && (mine >= kMaxStaging || mine_bytes + want > kMaxStagingBytes)) {
    s = &g_stage[oldest];
    e = hipEventSynchronize(s->done);
    if (e != hipSuccess) return hip_fail(e, "staging event");
  }
  if (!s) {
    Staging c{dev, nullptr, 0, nullptr, 0};
    e = hipEventCreateWithFlags(&c.done, hipEventDisableTiming);
    if (e != hipSuccess) return hip_fail(e, "staging event create");
    g_stage.push_back(c);
    s = &g_stage.back();
  }
  s->seq = ++g_stage_seq;
  if (s->bytes < bytes) {
    if (s->host) {
      e = hipHostFree(s->host);  // its copy has completed
      mine_bytes -= s->bytes;
      s->host = nullptr;
      s->bytes = 0;
      if (e != hipSuccess) return hip_fail(e, "staging free");
    }
    // regrowing past the byte limit: release this device's other idle buffers
    // (their copies have completed) before allocating
    if (mine_bytes + want > kMaxStagingBytes) {
      const uint64_t seq = s->seq;
      for (size_t i = 0; i < g_stage.size();) {
        Staging& c = g_stage[i];
        if (c.device == dev && c.seq != seq && c.host && hipEventQuery(c.done) == hipSuccess) {
          e = hipHostFree(c.host);
          if (e != hipSuccess) return hip_fail(e, "staging free");
          (void)hipEventDestroy(c.done);
          g_stage[i] = g_stage.back();
          g_stage.pop_back();
        } else {
          ++i;
        }
      }
      s = nullptr;
      for (Staging& c : g_stage)
        if (c.seq == seq) s = &c;
      if (!s) return fail(PM_EHIP, "internal: staging buffer lost");
    }
    e = hipHostMalloc(&s->host, want, hipHostMallocDefault);
    if (e != hipSuccess) return hip_fail(e, "staging allocation");
    s->bytes = want;
  }
  std::memcpy(s->host, src, bytes);
  e = hipMemcpyAsync(dst, s->host, bytes, hipMemcpyHostToDevice, stream);
  if (e != hipSuccess) return hip_fail(e, "descriptor upload");
  e = hipEventRecord(s->done, stream);
  return e == hipSuccess ? PM_OK : hip_fail(e, "staging event record");
}

struct Coeff {
  float a, b, c;
};

// ---- opt-in launch timing (pm_timing_enable / pm_timing_read)
struct TimingRec {
  pm_launch_time info;
  hipEvent_t begin, end;
};
// Shared by every thread of the process: `on` is atomic and the rest is
// guarded by `mu`. A record spans from the previous event of the same stream,
// so records of calls that interleave on several streams at once are dropped
// rather than mismeasured; timing is meant for one stream at a time.
struct Timing {
  std::atomic<bool> on{false};
  std::mutex mu;
  std::vector<hipEvent_t> pool;
  std::vector<TimingRec> recs;
  hipEvent_t last = nullptr;
  hipStream_t last_stream = nullptr;
} g_timing;

// Caller holds g_timing.mu.
hipEvent_t timing_event() {
  if (!g_timing.pool.empty()) {
    hipEvent_t e = g_timing.pool.back();
    g_timing.pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

// Marks the start of a timed sequence on `stream`.
void timing_begin(hipStream_t stream) {
  if (!g_timing.on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_timing.mu);
  hipEvent_t e = timing_event();
  if (!e) return;
  if (hipEventRecord(e, stream) != hipSuccess) {
    g_timing.pool.push_back(e);
    return;
  }
  g_timing.last = e;
  g_timing.last_stream = stream;
}

// Records the end of the launch just enqueued on `stream`.
void timing_mark(hipStream_t stream, int kind, int group, int iteration, int nmat, double flops, double bytes) {
  if (!g_timing.on.load(std::memory_order_relaxed)) return;
  std::lock_guard<std::mutex> lock(g_timing.mu);
  if (!g_timing.last || g_timing.last_stream != stream) return;
  hipEvent_t e = timing_event();
  if (!e) return;
  if (hipEventRecord(e, stream) != hipSuccess) {
    g_timing.pool.push_back(e);
    return;
  }
  TimingRec r{};
  r.info.kind = kind;
  r.info.group = group;
  r.info.iteration = iteration;
  r.info.n_matrices = nmat;
  r.info.flops = flops;
  r.info.bytes = bytes;
  r.begin = g_timing.last;
  r.end = e;
  g_timing.recs.push_back(r);
  g_timing.last = e;
}

// Enqueues the GEMM and Q-init launches of one group. Every GEMM launch walks
// all matrices of the group and takes the next set of queue counters.
struct Launcher {
  GemmArgs ga;          // shared fields (descs, n, mode, lr, wd) already set
  // One stage's device prefix sums: work items (tiles x K-split chunks) of the
  // GEMM launch, and split tiles of the reduce launch that follows it
  struct Stage {
    const int32_t* tiles;   // unsplit matrices' tiles
    const int32_t* items;   // split matrices' work items (tiles x chunks)
    const int32_t* split;   // split matrices' tiles
    int32_t tiles_total, items_total, split_total;
  };
  Stage gram_s, sym_s, full_s;
  int32_t* queues;      // kXcds counters per GEMM launch, zero at upload
  int launch = 0, max_launches = 0;
  bool final_f32 = false;
  hipStream_t stream;
  int group, count;
  double f_gram = 0, f_sym = 0, f_upd = 0;  // algorithmic FLOPs per launch kind (timing records)

  int next_queues(GemmArgs& a) {
    if (launch >= max_launches) return fail(PM_EINVAL, "internal: more GEMM launches than planned");
    a.queues = queues + kXcds * launch++;
    return PM_OK;
  }
  // The launches of one stage: the GEMM over unsplit matrices' tiles; then,
  // when some matrix splits this stage, the GEMM over their chunk items
  // (fp32 partials) and the reduce over their tiles. The stage's FLOPs go
  // with its first launch.
  template <int STAGE, int PDT>
  int stage_launch(GemmArgs a, const Stage& st, int kind, int it, double flops, const char* what) {
    if (st.tiles_total > 0) {
      a.prefix = st.tiles;
      a.total = st.tiles_total;
      if (int rc = next_queues(a)) return rc;
      hipLaunchKernelGGL((pm_ns_gemm_kernel<STAGE, PDT, kWsLayout>), dim3(gemm_grid(st.tiles_total)),
                         dim3(kGemmThreads), 0, stream, a);
      timing_mark(stream, kind, group, it, count, flops, 0.0);
      flops = 0.0;
      if (int rc = check(what)) return rc;
    }
    if (st.items_total == 0) return PM_OK;
    a.prefix = st.items;
    a.total = st.items_total;
    if (int rc = next_queues(a)) return rc;
    hipLaunchKernelGGL((pm_ns_gemm_kernel<STAGE, PDT, kWsLayout, true>), dim3(gemm_grid(st.items_total)),
                       dim3(kGemmThreads), 0, stream, a);
    timing_mark(stream, kind, group, it, count, flops, 0.0);
    if (int rc = check(what)) return rc;
    a.prefix = st.split;
    a.total = st.split_total;
    a.queues = nullptr;
    // one single-wave block per (split tile, 128 x 64 sub-tile)
    hipLaunchKernelGGL((pm_ns_reduce_kernel<STAGE, PDT, kWsLayout>), dim3(st.split_total * (kGemmThreads / 64)),
                       dim3(64), 0, stream, a);
    timing_mark(stream, PM_K_REDUCE, group, it, count, 0.0, 0.0);
    return check("K-split reduce launch");
  }
  int gram(int cur, bool first, int sc, int it) {
    GemmArgs a = ga;
    a.stage = ST_GRAM; a.cur = cur; a.first = first; a.sc = sc;
    return stage_launch<ST_GRAM, DT_BF16>(a, gram_s, PM_K_GRAM, it, f_gram, "gram launch");
  }
  // S[sc] = alpha·S[sl]·S[sr]ᵀ + beta·S[sd]
  int symm(int sl, int sr, int sd, int sc, float alpha, float beta, int it) {
    GemmArgs a = ga;
    a.stage = ST_SYMM; a.sl = sl; a.sr = sr; a.sd = sd; a.sc = sc; a.c = alpha; a.b = beta;
    return stage_launch<ST_SYMM, DT_BF16>(a, sym_s, PM_K_POLY, it, f_sym, "symmetric product launch");
  }
  // X' = s·(a·X + S[sl]·X) into the other X slot, or (last) the param step
  int update(int sl, float coef_a, int cur, bool first, bool last, int it) {
    GemmArgs a = ga;
    a.stage = last ? ST_FINAL : ST_UPDATE; a.sl = sl; a.a = coef_a; a.cur = cur; a.first = first;
    const char* what = "Newton-Schulz update launch";
    if (last && final_f32) return stage_launch<ST_FINAL, DT_F32>(a, full_s, PM_K_FINAL, it, f_upd, what);
    if (last) return stage_launch<ST_FINAL, DT_BF16>(a, full_s, PM_K_FINAL, it, f_upd, what);
    return stage_launch<ST_UPDATE, DT_BF16>(a, full_s, PM_K_UPDATE, it, f_upd, what);
  }
  // small matrices: R = X Xᵀ (or, r_in, the R an apply left in S[0]) and the
  // M x M part of `steps` iterations from it0 (steps == 0: the standard form's
  // B) into S[0]
  const float* coeffs = nullptr;  // device (a, b, c) per iteration
  int small_core(int cur, bool first, int it0, int steps, int it, bool r_in = false) {
    const SmallCoreArgs a{ga.descs, coeffs, it0, steps, cur, first, 0, r_in};
    if (steps == 0)  // the standard form's M x M part fits a 4-slot ring: two blocks per CU
      hipLaunchKernelGGL(pm_small_core_kernel<kSmRingStd>, dim3(count), dim3(kGemmThreads), 0, stream, a);
    else
      hipLaunchKernelGGL(pm_small_core_kernel<kSmRing>, dim3(count), dim3(kGemmThreads), 0, stream, a);
    const int products = steps == 0 ? 1 : 4 * steps - 3;
    timing_mark(stream, PM_K_SMALL_CORE, group, it, count, (r_in ? 0.0 : f_gram) + products * f_sym, 0.0);
    return check("small-matrix core launch");
  }
  // small matrices: X' = s·(a·X + S[0]·X), or (last) the param step; gram:
  // also R = X' X'ᵀ into S[0] for the next core launch (r_in)
  int small_apply(float coef_a, int cur, bool first, bool last, int it, bool gram = false) {
    GemmArgs a = ga;
    a.stage = last ? ST_FINAL : ST_UPDATE; a.sl = 0; a.sc = 0; a.a = coef_a; a.cur = cur; a.first = first;
    a.prefix = full_s.tiles; a.total = full_s.tiles_total;
    const dim3 grid(gemm_grid(full_s.tiles_total)), block(kSmApplyThreads);  // persistent: one block per CU
    if (last && final_f32)
      hipLaunchKernelGGL((pm_small_apply_kernel<ST_FINAL, DT_F32>), grid, block, 0, stream, a);
    else if (last)
      hipLaunchKernelGGL((pm_small_apply_kernel<ST_FINAL, DT_BF16>), grid, block, 0, stream, a);
    else if (gram)
      hipLaunchKernelGGL((pm_small_apply_kernel<ST_UPDATE, DT_BF16, true>), grid, block, 0, stream, a);
    else
      hipLaunchKernelGGL((pm_small_apply_kernel<ST_UPDATE, DT_BF16>), grid, block, 0, stream, a);
    timing_mark(stream, last ? PM_K_FINAL : PM_K_UPDATE, group, it, count, f_upd + (gram ? f_gram : 0.0), 0.0);
    return check("small-matrix apply launch");
  }
  int qinit(int sz, int sq, float coef_a, int max_mp, int it) {
    for (int first = 0; first < count; first += 65535)  // gridDim.y limit
      hipLaunchKernelGGL(pm_qinit_kernel, dim3(max_mp / kProTile, std::min(count - first, 65535)), dim3(kThreads), 0,
                         stream, ga.descs, first, sz, sq, coef_a, (int32_t)((kWsLayout & kTiledS) != 0));
    timing_mark(stream, PM_K_QINIT, group, it, count, 0.0, 0.0);
    return check("Q init launch");
  }
  static int check(const char* what) {
    const hipError_t e = hipGetLastError();
    return e == hipSuccess ? PM_OK : hip_fail(e, what);
  }
};

struct Coeffs {
  const pm_hparams* hp;
  Coeff at(int it) const {
    if (hp->coeffs) return Coeff{hp->coeffs[3 * it], hp->coeffs[3 * it + 1], hp->coeffs[3 * it + 2]};
    return Coeff{hp->a, hp->b, hp->c};
  }
};

// Standard quintic (torch/optim/_muon.py:61-66): per iteration A = X Xᵀ,
// B = b A + c A², X <- a X + B X; the last update is fused with the step.
int run_standard(Launcher& L, const pm_hparams* hp) {
  const Coeffs co{hp};
  for (int it = 0; it < hp->ns_steps; ++it) {
    const Coeff k = co.at(it);
    const int cur = it & 1;
    int rc = L.gram(cur, it == 0, /*A*/ 0, it);
    if (!rc) rc = L.symm(0, 0, 0, /*B*/ 1, k.c, k.b, it);
    if (!rc) rc = L.update(/*B*/ 1, k.a, cur, it == 0, it + 1 == hp->ns_steps, it);
    if (rc) return rc;
  }
  return PM_OK;
}

// Gram form of PAN 2 (_gram_newtonschulz_local, pan/optim/patch_muon.py:275-334):
// R = X Xᵀ; per iteration Z = c R R + b R; Q = a I + Z (first of a segment)
// or Q Z + a Q; R <- (aI+Z) R (aI+Z) as RZ = R Z + a R, R = Z RZ + a RZ
// (skipped before a reset and after the last iteration); at the reset
// iteration X <- Q X and R = X Xᵀ again; finally X <- Q X, fused with the step.
// The Frobenius scaling of X is folded as in the standard form: into the first
// gram (s²) and into the first application of Q to the unscaled X (s).
int run_gram(Launcher& L, const pm_hparams* hp, int max_mp) {
  enum { R = 0, Z = 1, RZ = 2, Q0 = 3, Q1 = 4 };
  const Coeffs co{hp};
  const int steps = hp->ns_steps, reset = gram_reset(steps);
  int cur = 0;          // X slot holding the current X
  bool scaled = false;  // has X been scaled by 1/‖X‖ yet?
  int q = -1;           // square buffer holding Q (-1: no Q in this segment)
  int rc = L.gram(cur, true, R, 0);
  for (int it = 0; it < steps && !rc; ++it) {
    const Coeff k = co.at(it);
    if (it == reset) {
      rc = L.update(q, 0.0f, cur, !scaled, false, it);
      cur ^= 1;
      scaled = true;
      if (!rc) rc = L.gram(cur, false, R, it);
      q = -1;
    }
    if (!rc) rc = L.symm(R, R, R, Z, k.c, k.b, it);
    if (rc) break;
    if (q < 0) {
      rc = L.qinit(Z, Q0, k.a, max_mp, it);
      q = Q0;
    } else {
      const int qn = q == Q0 ? Q1 : Q0;
      rc = L.symm(q, Z, q, qn, 1.0f, k.a, it);
      q = qn;
    }
    if (!rc && it + 1 < steps && it + 1 != reset) {
      rc = L.symm(R, Z, R, RZ, 1.0f, k.a, it);
      if (!rc) rc = L.symm(Z, RZ, RZ, R, 1.0f, k.a, it);
    }
  }
  if (!rc) rc = L.update(q, 0.0f, cur, !scaled, true, steps - 1);
  return rc;
}

// Small matrices (pm_small.hpp). Standard form: per iteration one core launch
// (R and B) and one apply. Gram form: one core launch per segment (R, then the
// segment's Z, Q and R updates) and one apply of its Q, the second segment
// starting at the reset iteration on the applied X.
// When the group has many matrices (fused), an apply that is followed by a
// core launch also forms that launch's R from the X' it writes, so the core
// launch reads R (32 KiB a matrix) instead of X' (256 B per column). The fused
// apply gives each block whole matrices, so a group of few long matrices keeps
// the separate gram, which spreads one matrix over many blocks. pro_gram: the
// prologue (pm_small_prologue_kernel) has formed the first R as well.
int run_small(Launcher& L, const pm_hparams* hp, bool fused, bool pro_gram) {
  const int steps = hp->ns_steps;
  if (hp->ns_form != NS_GRAM) {
    const Coeffs co{hp};
    for (int it = 0; it < steps; ++it) {
      const bool r_in = it > 0 ? fused : pro_gram, last = it + 1 == steps;
      int rc = L.small_core(it & 1, it == 0, it, 0, it, r_in);
      if (!rc) rc = L.small_apply(co.at(it).a, it & 1, it == 0, last, it, fused && !last);
      if (rc) return rc;
    }
    return PM_OK;
  }
  const int reset = gram_reset(steps);
  const int seg1 = reset > 0 ? reset : steps;
  int rc = L.small_core(0, true, 0, seg1, 0, pro_gram);
  if (!rc) rc = L.small_apply(0.0f, 0, true, seg1 == steps, seg1 - 1, fused && seg1 < steps);
  if (!rc && seg1 < steps) {
    rc = L.small_core(1, false, seg1, steps - seg1, seg1, fused);
    if (!rc) rc = L.small_apply(0.0f, 1, false, true, steps - 1);
  }
  return rc;
}

// Runs one group: items[0, count) share the workspace `ws` and are all small
// or all not.
// How a group's descriptor table reaches the workspace: an asynchronous copy
// from a pinned staging buffer (upload; kernel arguments under graph
// capture), or kernels that take it as by-value arguments
// (load_table_by_kernel: no staging memory, for pm_muon_step_noalloc).
enum class TablePath { kStaged, kKernelArgs };

int run_group(Item* items, int count, int group, const pm_hparams* hp, int mode, const float* lr_dev,
              double lr_host, char* ws, hipStream_t stream, TablePath path) {
  // plan_groups keeps small and engine matrices in separate groups: the engine's
  // workspace matrices are in the panel layout, small matrices' X row-major
  const bool small = items[0].plan.small;
  for (int i = 1; i < count; ++i)
    if (items[i].plan.small != small) return fail(PM_EINVAL, "internal: a group mixes small and large matrices");
  // The FINAL epilogue is compiled per param dtype; plan_groups keeps a group's
  // params of one dtype (MODE_NS writes bf16).
  for (int i = 1; i < count; ++i)
    if (mode == MODE_STEP && items[i].desc.p_dt != items[0].desc.p_dt)
      return fail(PM_EINVAL, "internal: a group mixes param dtypes");

  const int form = hp->ns_form;
  // Table first, then per-matrix buffers.
  const size_t tb = table_bytes(count, gemm_launches(hp));
  char* cursor = ws + tb;
  std::vector<char> host(tb, 0);
  MatDesc* descs = (MatDesc*)host.data();
  const size_t pstride = align_up((size_t)(count + 1) * 4);
  int32_t* pro = (int32_t*)(host.data() + align_up((size_t)count * sizeof(MatDesc)));
  // per stage: [0] tiles of unsplit matrices, [1] items of split ones, [2] tiles of split ones
  int32_t* pre[3][3];
  for (int st = 0; st < 3; ++st)
    for (int k = 0; k < 3; ++k) pre[st][k] = (int32_t*)((char*)pro + (1 + 3 * st + k) * pstride);
  const int32_t* queues = (const int32_t*)(host.data() + queue_offset(count));  // zeros
  float* coeffs = (float*)(host.data() + coeff_offset(count, gemm_launches(hp)));
  const Coeffs co{hp};
  for (int it = 0; it < hp->ns_steps; ++it) {
    const Coeff k = co.at(it);
    coeffs[3 * it] = k.a;
    coeffs[3 * it + 1] = k.b;
    coeffs[3 * it + 2] = k.c;
  }
  pro[0] = 0;
  for (auto& st : pre)
    for (int32_t* a : st) a[0] = 0;
  int max_mp = 0;
  for (int i = 0; i < count; ++i) {
    Item& it = items[i];
    const Plan& p = it.plan;
    MatDesc& d = it.desc;
    d.rows = p.rows; d.cols = p.cols; d.trans = p.trans;
    d.M = p.M; d.N = p.N; d.Mp = p.Mp; d.Np = p.Np;
    const size_t x = align_up((size_t)p.Mp * p.Np * 2);
    const size_t a = align_up((size_t)p.Mp * p.Mp * 2);
    d.X[0] = (uint16_t*)cursor; cursor += x;
    d.X[1] = (uint16_t*)cursor; cursor += x;
    for (int b = 0; b < kSquareBufs; ++b) {
      d.S[b] = b < square_bufs(form, p.small) ? (uint16_t*)cursor : nullptr;
      if (b < square_bufs(form, p.small)) cursor += a;
    }
    d.partials = (float*)cursor; cursor += align_up((size_t)pro_tiles(p) * 4);
    d.scales = (float*)cursor; cursor += kAlign;
    d.pro_tiles = pro_tiles(p);
    d.ks_gram = p.ks_gram; d.ks_symm = p.ks_symm; d.ks_full = p.ks_full;
    d.kpart = p.kpart ? (float*)cursor : nullptr;
    cursor += p.kpart;
    descs[i] = d;
    pro[i + 1] = pro[i] + pro_tiles(p);
    const int32_t tiles[3] = {sym_tiles(p), sym_tiles(p), full_tiles(p)};
    const int32_t ks[3] = {p.ks_gram, p.ks_symm, p.ks_full};
    for (int st = 0; st < 3; ++st) {
      const bool split = ks[st] > 1;
      pre[st][0][i + 1] = pre[st][0][i] + (split ? 0 : tiles[st]);
      pre[st][1][i + 1] = pre[st][1][i] + (split ? tiles[st] * ks[st] : 0);
      pre[st][2][i + 1] = pre[st][2][i] + (split ? tiles[st] : 0);
    }
    max_mp = std::max(max_mp, p.Mp);
  }
  int rc = path == TablePath::kStaged ? upload(host.data(), tb, ws, stream)
                                      : load_table_by_kernel(host.data(), tb, ws, stream);
  if (rc) return rc;
  timing_begin(stream);

  // Algorithmic work per launch (timing records only).
  double f_gram = 0, f_sym = 0, f_upd = 0, b_pro = 0;
  for (int i = 0; i < count; ++i) {
    const Plan& p = items[i].plan;
    const double M = p.M, N = p.N, elems = M * N;
    f_gram += M * (M + 1) * N;
    f_sym += M * M * (M + 1);
    f_upd += 2 * M * M * N;
    const MatDesc& d = items[i].desc;
    const double gb = d.g_dt == PM_DTYPE_F32 ? 4 : 2;
    const double mb = mode == MODE_STEP ? (d.m_dt == PM_DTYPE_F32 ? 8 : 4) : 0;
    b_pro += elems * (gb + mb + 2);  // grad read, momentum read+write, X bf16 write
  }

  const MatDesc* ddesc = (const MatDesc*)ws;
  const int32_t* dpro = (const int32_t*)(ws + ((char*)pro - host.data()));
  auto dev_ptr = [&](const int32_t* h) { return (const int32_t*)(ws + ((const char*)h - host.data())); };
  int32_t* dqueues = (int32_t*)(ws + ((const char*)queues - host.data()));

  // Small matrices: with many of them the apply takes the fused gram (one
  // matrix per apply block at least, none longer than twice a block's even
  // share of the units), and the prologue forms the first R as well when every
  // matrix's prologue partials fit its LDS.
  bool fused = false, pro_gram = false;
  if (small) {
    int32_t longest = 0, parts = 0;
    for (int i = 0; i < count; ++i) {
      longest = std::max(longest, pre[2][0][i + 1] - pre[2][0][i]);
      parts = std::max(parts, pro[i + 1] - pro[i]);
    }
    const int32_t units = pre[2][0][count];  // small matrices never split
    const int grid = gemm_grid(units);
    fused = count >= grid && (int64_t)longest * grid <= 2 * (int64_t)units;
    pro_gram = fused && parts <= kSmProParts;
  }

  ProArgs pa{ddesc, dpro, count, mode, hp->momentum, hp->nesterov, small ? XL_SMALL : ((kWsLayout & kTiledX) ? XL_PANEL : XL_ROW), 0};
  if (pro_gram) {
    // instantiated for the first matrix's dtypes (a matrix of other dtypes
    // takes the kernel's element-wise loads)
    const bool g32 = items[0].desc.g_dt == PM_DTYPE_F32, m32 = items[0].desc.m_dt == PM_DTYPE_F32;
    const dim3 grid(count), block(kGemmThreads);
    if (g32 && m32)
      hipLaunchKernelGGL((pm_small_prologue_kernel<true, true>), grid, block, 0, stream, pa, hp->eps, 0);
    else if (g32)
      hipLaunchKernelGGL((pm_small_prologue_kernel<true, false>), grid, block, 0, stream, pa, hp->eps, 0);
    else if (m32)
      hipLaunchKernelGGL((pm_small_prologue_kernel<false, true>), grid, block, 0, stream, pa, hp->eps, 0);
    else
      hipLaunchKernelGGL((pm_small_prologue_kernel<false, false>), grid, block, 0, stream, pa, hp->eps, 0);
    timing_mark(stream, PM_K_PROLOGUE, group, -1, count, f_gram, b_pro);
  } else {
    hipLaunchKernelGGL(pm_prologue_kernel, dim3(pro[count]), dim3(kThreads), 0, stream, pa);
    timing_mark(stream, PM_K_PROLOGUE, group, -1, count, 0.0, b_pro);
    hipLaunchKernelGGL(pm_norm_kernel, dim3(count), dim3(kThreads), 0, stream, ddesc, hp->eps);
    timing_mark(stream, PM_K_NORM, group, -1, count, 0.0, 0.0);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return hip_fail(e, "prologue launch");

  Launcher L{};
  L.ga.descs = ddesc;
  L.ga.n = count;
  L.ga.mode = mode;
  L.ga.lr_dev = lr_dev;
  L.ga.wd = (float)hp->weight_decay;
  L.ga.wdf_host = (float)(1.0 - lr_host * (double)hp->weight_decay);
  Launcher::Stage* sts[3] = {&L.gram_s, &L.sym_s, &L.full_s};
  for (int st = 0; st < 3; ++st)
    *sts[st] = Launcher::Stage{dev_ptr(pre[st][0]), dev_ptr(pre[st][1]), dev_ptr(pre[st][2]), pre[st][0][count],
                               pre[st][1][count], pre[st][2][count]};
  L.queues = dqueues;
  L.max_launches = gemm_launches(hp);
  L.final_f32 = mode == MODE_STEP && items[0].desc.p_dt == PM_DTYPE_F32;
  L.stream = stream;
  L.group = group;
  L.count = count;
  L.f_gram = f_gram;
  L.f_sym = f_sym;
  L.f_upd = f_upd;
  L.coeffs = (const float*)(ws + ((char*)coeffs - host.data()));
  if (small) return run_small(L, hp, fused, pro_gram);
  return form == NS_GRAM ? run_gram(L, hp, max_mp) : run_standard(L, hp);
}

// Sorts items (params of one dtype together, small matrices apart, then
// longest tiles first) and packs them into groups [begin, end) whose
// workspace fits ws_bytes. Fails, before anything is enqueued, when a matrix
// does not fit on its own.
int plan_groups(std::vector<Item>& items, const pm_hparams* hp, size_t ws_bytes,
                std::vector<std::pair<size_t, size_t>>& groups) {
  std::stable_sort(items.begin(), items.end(), [](const Item& x, const Item& y) {
    if (x.desc.p_dt != y.desc.p_dt) return x.desc.p_dt < y.desc.p_dt;
    if (x.plan.small != y.plan.small) return y.plan.small;
    return x.plan.Np != y.plan.Np ? x.plan.Np > y.plan.Np : x.plan.Mp > y.plan.Mp;
  });
  groups.clear();
  size_t i = 0;
  while (i < items.size()) {
    size_t j = i, need = 0;
    while (j < items.size()) {
      if (items[j].desc.p_dt != items[i].desc.p_dt) break;  // one param dtype per group
      if (items[j].plan.small != items[i].plan.small) break;  // one kind of kernels per group
      const size_t next = need + items[j].plan.ws;
      if (table_bytes((int)(j - i + 1), gemm_launches(hp)) + next > ws_bytes) break;
      need = next;
      ++j;
    }
    if (j == i)
      return fail(PM_EWORKSPACE, "workspace of %zu bytes cannot hold a %dx%d matrix (needs %zu)", ws_bytes,
                  items[i].plan.rows, items[i].plan.cols, table_bytes(1, gemm_launches(hp)) + items[i].plan.ws);
    groups.emplace_back(i, j);
    i = j;
  }
  return PM_OK;
}

// Plans every group first (so a workspace too small for some matrix fails
// before any momentum or param is touched), then runs the groups in turn on
// the one workspace.
int run_all(std::vector<Item>& items, const pm_hparams* hp, int mode, const float* lr_dev, double lr_host,
            void* workspace, size_t ws_bytes, hipStream_t stream, TablePath path = TablePath::kStaged) {
  if (items.empty()) return PM_OK;
  if (!workspace) return fail(PM_EINVAL, "workspace is NULL");
  if ((uintptr_t)workspace % kAlign) return fail(PM_EINVAL, "workspace must be %zu-byte aligned", kAlign);
  std::vector<std::pair<size_t, size_t>> groups;
  if (int rc = plan_groups(items, hp, ws_bytes, groups)) return rc;
  for (size_t g = 0; g < groups.size(); ++g) {
    const auto [i, j] = groups[g];
    const int rc = run_group(items.data() + i, (int)(j - i), (int)g, hp, mode, lr_dev, lr_host, (char*)workspace,
                             stream, path);
    if (rc) return rc;
  }
  return PM_OK;
}

size_t plan_workspace(const std::vector<Plan>& plans, const pm_hparams* hp) {
  size_t total = 0, largest = 0;
  for (const Plan& p : plans) {
    total += p.ws;
    largest = std::max(largest, p.ws);
  }
  const uint64_t limit = hp->workspace_limit ? hp->workspace_limit : kDefaultWorkspaceLimit;
  const size_t body = std::min<size_t>(total, std::max<size_t>(limit, largest));
  return table_bytes((int)plans.size(), gemm_launches(hp)) + body;
}

int collect_step(const pm_matrix* mats, int n, int form, std::vector<Item>& items) {
  if (n < 0 || (n > 0 && !mats)) return fail(PM_EINVAL, "bad matrix list");
  items.clear();
  items.reserve(n);
  for (int i = 0; i < n; ++i) {
    const pm_matrix& m = mats[i];
    int rc = check_extent(m.rows, m.cols);
    if (rc) return rc;
    if (!m.param || !m.grad || !m.momentum) return fail(PM_EINVAL, "matrix %d: NULL tensor pointer", i);
    if (!valid_dtype(m.param_dtype) || !valid_dtype(m.grad_dtype) || !valid_dtype(m.momentum_dtype))
      return fail(PM_EDTYPE, "matrix %d: dtypes must be f32 or bf16", i);
    if (m.param_ld < m.cols || m.grad_ld < m.cols || m.momentum_ld < m.cols)
      return fail(PM_EINVAL, "matrix %d: row stride smaller than cols", i);
    Item it{};
    it.plan = make_plan(m.rows, m.cols, form);
    MatDesc& d = it.desc;
    d.param = m.param; d.grad = m.grad; d.mom = m.momentum;
    d.p_ld = m.param_ld; d.g_ld = m.grad_ld; d.m_ld = m.momentum_ld;
    d.p_dt = m.param_dtype; d.g_dt = m.grad_dtype; d.m_dt = m.momentum_dtype;
    d.adj_ratio = (float)m.adj_ratio;
    items.push_back(it);
  }
  split_call(items);
  return PM_OK;
}

int collect_ns(const pm_ns_matrix* mats, int n, int form, std::vector<Item>& items) {
  if (n < 0 || (n > 0 && !mats)) return fail(PM_EINVAL, "bad matrix list");
  items.clear();
  items.reserve(n);
  for (int i = 0; i < n; ++i) {
    const pm_ns_matrix& m = mats[i];
    int rc = check_extent(m.rows, m.cols);
    if (rc) return rc;
    if (!m.in || !m.out) return fail(PM_EINVAL, "matrix %d: NULL tensor pointer", i);
    if (!valid_dtype(m.in_dtype)) return fail(PM_EDTYPE, "matrix %d: input dtype must be f32 or bf16", i);
    if (m.in_ld < m.cols || m.out_ld < m.cols) return fail(PM_EINVAL, "matrix %d: row stride smaller than cols", i);
    Item it{};
    it.plan = make_plan(m.rows, m.cols, form);
    MatDesc& d = it.desc;
    d.param = m.out; d.grad = m.in; d.mom = nullptr;
    d.p_ld = m.out_ld; d.g_ld = m.in_ld; d.m_ld = 0;
    d.p_dt = PM_DTYPE_BF16; d.g_dt = m.in_dtype; d.m_dt = PM_DTYPE_F32;
    items.push_back(it);
  }
  split_call(items);
  return PM_OK;
}

int grid_for(int64_t n) {
  const int64_t blocks = (n + kThreads - 1) / kThreads;
  return (int)std::max<int64_t>(1, std::min<int64_t>(blocks, 256 * 64));
}

// ---- the allocation-free step's descriptor tables and scratch

// One launch of pm_table_load_kernel writes kTableChunk bytes of a descriptor
// table that it receives as a kernel argument (the runtime copies kernel
// arguments itself, so no staging memory is involved).
constexpr int kTableChunk = 2048;
struct TableChunk {
  uint32_t* dst;
  uint32_t words;  // 32-bit words of this chunk
  uint32_t pad_;
  uint32_t data[kTableChunk / 4];
};

__global__ __launch_bounds__(kThreads) void pm_table_load_kernel(TableChunk c) {
  for (uint32_t i = threadIdx.x; i < c.words; i += kThreads) c.dst[i] = c.data[i];
}

int load_table_by_kernel(const char* src, size_t bytes, char* dst, hipStream_t stream) {
  if (bytes % 4 || (uintptr_t)dst % 4) return fail(PM_EINVAL, "internal: descriptor table not in 32-bit words");
  for (size_t off = 0; off < bytes; off += kTableChunk) {
    TableChunk c;
    const size_t n = std::min<size_t>(kTableChunk, bytes - off);
    c.dst = (uint32_t*)(dst + off);
    c.words = (uint32_t)(n / 4);
    c.pad_ = 0;
    std::memcpy(c.data, src + off, n);
    hipLaunchKernelGGL(pm_table_load_kernel, dim3(1), dim3(kThreads), 0, stream, c);
  }
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? PM_OK : hip_fail(e, "descriptor table launch");
}

}  // namespace

// Scratch of pm_muon_step_noalloc: the workspace of a step, held by every GPU
// the library runs on until the process ends. Host code never uses this name
// as an address (on the host it is only a handle for the runtime): each
// device's own address comes from hipGetSymbolAddress, once per device.
static __device__ __align__(256) char scratch[PM_NOALLOC_SCRATCH_BYTES];

namespace {

std::mutex g_scratch_mu;
constexpr int kMaxDevices = 64;
char* g_scratch_ptr[kMaxDevices] = {};

// This device's address of `scratch`, looked up on the device's first call.
int scratch_on_device(char** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices) return fail(PM_EUNSUPPORTED, "device %d beyond the first %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    if (!p) return fail(PM_EHIP, "hipGetSymbolAddress(scratch) returned NULL");
    g_scratch_ptr[dev] = (char*)p;
  }
  *out = g_scratch_ptr[dev];
  return PM_OK;
}

}  // namespace

extern "C" {

int pm_abi_version(void) { return PM_ABI_VERSION; }

const char* pm_last_error(void) { return g_err.c_str(); }

size_t pm_workspace_bytes(const pm_matrix* mats, int n, const pm_hparams* hp) {
  if (check_hparams(hp)) return 0;
  std::vector<Item> items;
  if (collect_step(mats, n, hp->ns_form, items)) return 0;
  std::vector<Plan> plans;
  for (auto& it : items) plans.push_back(it.plan);
  return plan_workspace(plans, hp);
}

size_t pm_ns_workspace_bytes(const pm_ns_matrix* mats, int n, const pm_hparams* hp) {
  if (check_hparams(hp)) return 0;
  std::vector<Item> items;
  if (collect_ns(mats, n, hp->ns_form, items)) return 0;
  std::vector<Plan> plans;
  for (auto& it : items) plans.push_back(it.plan);
  return plan_workspace(plans, hp);
}

int pm_muon_step(const pm_matrix* mats, int n, const pm_hparams* hp, const float* lr_dev, double lr_host,
                 void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = check_hparams(hp);
  if (rc) return rc;
  std::vector<Item> items;
  rc = collect_step(mats, n, hp->ns_form, items);
  if (rc) return rc;
  // Items are still in caller order here. The host-lr product stays in double
  // and is rounded once, as the reference passes -adjusted_lr to its kernel.
  for (int i = 0; i < n; ++i) items[i].desc.neg_lr_host = (float)(-(lr_host * mats[i].adj_ratio));
  return run_all(items, hp, MODE_STEP, lr_dev, lr_host, workspace, workspace_bytes, (hipStream_t)stream);
}

int pm_muon_step_noalloc(const pm_matrix* mats, int n, const pm_hparams* hp, const float* lr_dev, double lr_host,
                         void* stream) {
  g_err.clear();
  int rc = check_hparams(hp);
  if (rc) return rc;
  std::vector<Item> items;
  rc = collect_step(mats, n, hp->ns_form, items);
  if (rc) return rc;
  const size_t one = table_bytes(1, gemm_launches(hp));
  for (const Item& it : items)
    if (one + it.plan.ws > PM_NOALLOC_SCRATCH_BYTES)
      return fail(PM_EWORKSPACE,
                  "pm_muon_step_noalloc: a %dx%d matrix needs %zu bytes of scratch; the static scratch holds %zu "
                  "(PM_NOALLOC_SCRATCH_BYTES); use pm_muon_step with a caller workspace",
                  it.plan.rows, it.plan.cols, one + it.plan.ws, (size_t)PM_NOALLOC_SCRATCH_BYTES);
  for (int i = 0; i < n; ++i) items[i].desc.neg_lr_host = (float)(-(lr_host * mats[i].adj_ratio));
  if (items.empty()) return PM_OK;
  char* ws = nullptr;
  rc = scratch_on_device(&ws);
  if (rc) return rc;
  return run_all(items, hp, MODE_STEP, lr_dev, lr_host, ws, PM_NOALLOC_SCRATCH_BYTES, (hipStream_t)stream,
                 TablePath::kKernelArgs);
}

int pm_newton_schulz(const pm_ns_matrix* mats, int n, const pm_hparams* hp, void* workspace,
                     size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = check_hparams(hp);
  if (rc) return rc;
  std::vector<Item> items;
  rc = collect_ns(mats, n, hp->ns_form, items);
  if (rc) return rc;
  return run_all(items, hp, MODE_NS, nullptr, 0.0, workspace, workspace_bytes, (hipStream_t)stream);
}

int pm_momentum_nesterov(void* buf, int32_t buf_dtype, const void* grad, int32_t grad_dtype, void* update,
                         int32_t update_dtype, int64_t n, float momentum, int32_t nesterov, void* stream) {
  g_err.clear();
  if (n < 0) return fail(PM_EINVAL, "negative element count");
  if (n == 0) return PM_OK;
  if (!buf || !grad || !update) return fail(PM_EINVAL, "NULL tensor pointer");
  if (!valid_dtype(buf_dtype) || !valid_dtype(grad_dtype) || !valid_dtype(update_dtype))
    return fail(PM_EDTYPE, "dtypes must be f32 or bf16");
  hipLaunchKernelGGL(pm_momentum_kernel, dim3(grid_for(n)), dim3(kThreads), 0, (hipStream_t)stream, buf,
                     buf_dtype, grad, grad_dtype, update, update_dtype, n, momentum, nesterov);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? PM_OK : hip_fail(e, "momentum launch");
}

int pm_step_param(void* param, int32_t param_dtype, const void* update, int32_t update_dtype, int64_t n,
                  const float* lr_dev, double lr_host, float weight_decay, double adj_ratio, void* stream) {
  g_err.clear();
  if (n < 0) return fail(PM_EINVAL, "negative element count");
  if (n == 0) return PM_OK;
  if (!param || !update) return fail(PM_EINVAL, "NULL tensor pointer");
  if (!valid_dtype(param_dtype) || !valid_dtype(update_dtype)) return fail(PM_EDTYPE, "dtypes must be f32 or bf16");
  const float wdf = (float)(1.0 - lr_host * (double)weight_decay);
  const float neg = (float)(-(lr_host * adj_ratio));
  hipLaunchKernelGGL(pm_step_kernel, dim3(grid_for(n)), dim3(kThreads), 0, (hipStream_t)stream, param,
                     param_dtype, update, update_dtype, n, lr_dev, weight_decay, (float)adj_ratio, wdf, neg);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? PM_OK : hip_fail(e, "step launch");
}

int pm_timing_enable(int on) {
  g_timing.on.store(on != 0, std::memory_order_relaxed);
  return PM_OK;
}

int pm_timing_read(pm_launch_time* out, int max) {
  g_err.clear();
  if (max < 0 || (max > 0 && !out)) return fail(PM_EINVAL, "bad output buffer");
  std::lock_guard<std::mutex> lock(g_timing.mu);
  int n = 0;
  for (TimingRec& r : g_timing.recs) {
    hipError_t e = hipEventSynchronize(r.end);
    if (e != hipSuccess) return hip_fail(e, "timing event");
    float ms = 0.0f;
    e = hipEventElapsedTime(&ms, r.begin, r.end);
    if (e != hipSuccess) return hip_fail(e, "timing elapsed");
    if (n < max) {
      out[n] = r.info;
      out[n].ms = ms;
      ++n;
    }
  }
  // Recycle every distinct event (a record's begin is usually the previous end).
  std::vector<hipEvent_t> used;
  for (TimingRec& r : g_timing.recs) {
    used.push_back(r.begin);
    used.push_back(r.end);
  }
  std::sort(used.begin(), used.end());
  used.erase(std::unique(used.begin(), used.end()), used.end());
  g_timing.pool.insert(g_timing.pool.end(), used.begin(), used.end());
  g_timing.recs.clear();
  g_timing.last = nullptr;
  return n;
}

size_t pm_gram_workspace_bytes(void) { return table_bytes(1, 1); }

int pm_gram(const void* x, int64_t rows, int64_t cols, void* out, void* workspace, size_t workspace_bytes,
            void* stream) {
  g_err.clear();
  int rc = check_extent(rows, cols);
  if (rc) return rc;
  if (!x || !out || !workspace) return fail(PM_EINVAL, "NULL pointer");
  if (rows % kTile || cols % kTile) return fail(PM_EINVAL, "pm_gram needs rows and cols that are multiples of 256");
  if (workspace_bytes < table_bytes(1, 1)) return fail(PM_EWORKSPACE, "workspace too small");
  if ((uintptr_t)workspace % kAlign) return fail(PM_EINVAL, "workspace must be %zu-byte aligned", kAlign);
  std::vector<char> host(table_bytes(1, 1), 0);
  MatDesc* d = (MatDesc*)host.data();
  d->X[0] = (uint16_t*)x;
  d->S[0] = (uint16_t*)out;
  d->Mp = d->M = (int32_t)rows;
  d->Np = d->N = (int32_t)cols;
  d->rows = (int32_t)rows;
  d->cols = (int32_t)cols;
  int32_t* sym = (int32_t*)(host.data() + align_up(sizeof(MatDesc)) + align_up(8));
  const size_t queues_off = queue_offset(1);  // one launch's counters, zeros
  const int32_t nt = (int32_t)(rows / kTile);
  sym[0] = 0;
  sym[1] = nt * (nt + 1) / 2;
  hipStream_t s = (hipStream_t)stream;
  rc = upload(host.data(), host.size(), workspace, s);
  if (rc) return rc;
  GemmArgs ga{};
  ga.descs = (const MatDesc*)workspace;
  ga.prefix = (const int32_t*)((char*)workspace + ((char*)sym - host.data()));
  ga.queues = (int32_t*)((char*)workspace + queues_off);
  ga.total = sym[1];
  ga.n = 1;
  ga.stage = ST_GRAM;
  ga.cur = 0;
  ga.first = 0;
  ga.sc = 0;
  hipLaunchKernelGGL((pm_ns_gemm_kernel<ST_GRAM, DT_BF16, 0>), dim3(gemm_grid(sym[1])), dim3(kGemmThreads), 0, s, ga);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? PM_OK : hip_fail(e, "gram launch");
}

size_t pm_gemm_symmetric_workspace_bytes(void) { return table_bytes(1, 1); }

int pm_gemm_symmetric(const void* left, const void* right, const void* addend, void* out, int64_t m, float alpha,
                      float beta, void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  int rc = check_extent(m, m);
  if (rc) return rc;
  if (!left || !right || !out || !workspace) return fail(PM_EINVAL, "NULL pointer");
  if (beta != 0.0f && !addend) return fail(PM_EINVAL, "addend is NULL but beta != 0");
  if (m % kTile) return fail(PM_EINVAL, "pm_gemm_symmetric needs m to be a multiple of 256");
  if (workspace_bytes < table_bytes(1, 1)) return fail(PM_EWORKSPACE, "workspace too small");
  if ((uintptr_t)workspace % kAlign) return fail(PM_EINVAL, "workspace must be %zu-byte aligned", kAlign);
  std::vector<char> host(table_bytes(1, 1), 0);
  MatDesc* d = (MatDesc*)host.data();
  d->S[0] = (uint16_t*)left;
  d->S[1] = (uint16_t*)right;
  d->S[2] = (uint16_t*)(addend ? addend : left);  // not read when beta == 0
  d->S[3] = (uint16_t*)out;
  d->Mp = d->M = d->Np = d->N = (int32_t)m;
  d->rows = d->cols = (int32_t)m;
  int32_t* sym = (int32_t*)(host.data() + align_up(sizeof(MatDesc)) + align_up(8));
  const size_t queues_off = queue_offset(1);  // one launch's counters, zeros
  const int32_t nt = (int32_t)(m / kTile);
  sym[0] = 0;
  sym[1] = nt * (nt + 1) / 2;
  hipStream_t s = (hipStream_t)stream;
  rc = upload(host.data(), host.size(), workspace, s);
  if (rc) return rc;
  GemmArgs ga{};
  ga.descs = (const MatDesc*)workspace;
  ga.prefix = (const int32_t*)((char*)workspace + ((char*)sym - host.data()));
  ga.queues = (int32_t*)((char*)workspace + queues_off);
  ga.total = sym[1];
  ga.n = 1;
  ga.stage = ST_SYMM;
  ga.sl = 0;
  ga.sr = 1;
  ga.sd = 2;
  ga.sc = 3;
  ga.c = alpha;
  ga.b = beta;
  hipLaunchKernelGGL((pm_ns_gemm_kernel<ST_SYMM, DT_BF16, 0>), dim3(gemm_grid(sym[1])), dim3(kGemmThreads), 0, s, ga);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? PM_OK : hip_fail(e, "symmetric product launch");
}

// Descriptor table of an Adam call: descs[n] | chunk prefix[n+1].
size_t pm_adam_workspace_bytes(int n) {
  if (n < 0) return 0;
  return align_up((size_t)n * sizeof(AdamDesc)) + align_up((size_t)(n + 1) * 4);
}

int pm_adam_step(const pm_adam_tensor* ts, int n, const pm_adam_hparams* hp, const float* lr_dev, double lr_host,
                 const float* grad_scale, const float* found_inf, void* workspace, size_t workspace_bytes,
                 void* stream) {
  g_err.clear();
  if (n < 0 || (n > 0 && !ts)) return fail(PM_EINVAL, "bad tensor list");
  if (!hp) return fail(PM_EINVAL, "hparams is NULL");
  if (n == 0) return PM_OK;
  if (!(hp->beta1 >= 0.0 && hp->beta1 < 1.0) || !(hp->beta2 >= 0.0 && hp->beta2 < 1.0))
    return fail(PM_EINVAL, "betas must be in [0, 1)");
  if (!(hp->eps >= 0.0)) return fail(PM_EINVAL, "eps must be >= 0");
  if (!(hp->weight_decay >= 0.0)) return fail(PM_EINVAL, "weight_decay must be >= 0");
  const size_t need = pm_adam_workspace_bytes(n);
  if (!workspace) return fail(PM_EINVAL, "workspace is NULL");
  if ((uintptr_t)workspace % kAlign) return fail(PM_EINVAL, "workspace must be %zu-byte aligned", kAlign);
  if (workspace_bytes < need) return fail(PM_EWORKSPACE, "workspace of %zu bytes, %zu needed", workspace_bytes, need);
  std::vector<char> host(need, 0);
  AdamDesc* descs = (AdamDesc*)host.data();
  int32_t* prefix = (int32_t*)(host.data() + align_up((size_t)n * sizeof(AdamDesc)));
  prefix[0] = 0;
  for (int i = 0; i < n; ++i) {
    const pm_adam_tensor& t = ts[i];
    if (t.numel < 0) return fail(PM_EINVAL, "tensor %d: negative numel", i);
    if (!t.step) return fail(PM_EINVAL, "tensor %d: NULL step", i);
    if (t.numel > 0 && (!t.param || !t.grad || !t.exp_avg || !t.exp_avg_sq))
      return fail(PM_EINVAL, "tensor %d: NULL tensor pointer", i);
    if (hp->amsgrad && t.numel > 0 && !t.max_exp_avg_sq) return fail(PM_EINVAL, "tensor %d: amsgrad needs max_exp_avg_sq", i);
    auto adam_dtype = [](int32_t dt) { return valid_dtype(dt) || dt == PM_DTYPE_F16; };
    if (!adam_dtype(t.param_dtype) || !adam_dtype(t.grad_dtype) || !adam_dtype(t.exp_avg_dtype) ||
        !adam_dtype(t.exp_avg_sq_dtype))
      return fail(PM_EDTYPE, "tensor %d: dtypes must be f32, bf16 or f16", i);
    const int64_t chunks = (t.numel + kAdamChunk - 1) / kAdamChunk;
    if (prefix[i] + chunks > INT32_MAX) return fail(PM_EINVAL, "too many elements in one call");
    prefix[i + 1] = (int32_t)(prefix[i] + chunks);
    AdamDesc& d = descs[i];
    d.p = t.param; d.g = (void*)t.grad; d.m = t.exp_avg; d.v = t.exp_avg_sq;
    d.vmax = hp->amsgrad ? t.max_exp_avg_sq : nullptr;
    d.step = t.step;
    d.n = t.numel;
    d.p_dt = t.param_dtype; d.g_dt = t.grad_dtype; d.m_dt = t.exp_avg_dtype; d.v_dt = t.exp_avg_sq_dtype;
  }
  hipStream_t s = (hipStream_t)stream;
  int rc = upload(host.data(), need, workspace, s);
  if (rc) return rc;
  const AdamDesc* ddesc = (const AdamDesc*)workspace;
  AdamArgs a{};
  a.descs = ddesc;
  a.prefix = (const int32_t*)((char*)workspace + ((char*)prefix - host.data()));
  a.n = n;
  a.b1d = hp->beta1;
  a.b2d = hp->beta2;
  a.beta2 = (float)hp->beta2;
  a.w1 = (float)(1.0 - hp->beta1);
  a.w2 = (float)(1.0 - hp->beta2);
  a.eps = (float)hp->eps;
  a.wd = (float)hp->weight_decay;
  a.wdd = hp->weight_decay;
  a.amsgrad = hp->amsgrad != 0;
  a.maximize = hp->maximize != 0;
  a.decoupled = hp->decoupled_weight_decay != 0;
  a.lr_dev = lr_dev;
  a.lr_host = lr_host;
  a.grad_scale = grad_scale;
  a.found_inf = found_inf;
  timing_begin(s);
  hipLaunchKernelGGL(pm_adam_count_kernel, dim3((n + kThreads - 1) / kThreads), dim3(kThreads), 0, s, ddesc, n,
                     found_inf);
  if (prefix[n] > 0) hipLaunchKernelGGL(pm_adam_kernel, dim3(prefix[n]), dim3(kThreads), 0, s, a);
  double bytes = 0;
  for (int i = 0; i < n; ++i) {
    const pm_adam_tensor& t = ts[i];
    auto sz = [](int32_t dt) { return dt == PM_DTYPE_F32 ? 4.0 : 2.0; };
    const double per = 2 * sz(t.param_dtype) + sz(t.grad_dtype) + 2 * sz(t.exp_avg_dtype) +
                       (hp->amsgrad ? 4 : 2) * sz(t.exp_avg_sq_dtype);
    bytes += per * (double)t.numel;
  }
  timing_mark(s, PM_K_ADAM, 0, -1, n, 0.0, bytes);
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? PM_OK : hip_fail(e, "adam launch");
}

}  // extern "C"
