// Work-item -> tile decoders of the GEMM stages and the workspace layouts.
// Plain arithmetic, compiled for the device by hipcc and for the host by the
// CPU tests (g++).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define PM_HD __host__ __device__ __forceinline__
#else
#define PM_HD inline
#endif

namespace pm {

// Consecutive work items walk kGroupRows tile rows column by column, so the
// 32 tiles an XCD runs together form a kGroupRows x 8 block that shares
// kGroupRows row panels and 8 column panels in that XCD's L2.
constexpr int kGroupRows = 4;

constexpr int kXcds = 8;       // MI355X: 8 XCDs, blocks dispatched round robin
constexpr int kXcdChunk = 32;  // consecutive tiles handed to one XCD (its 32 CUs)

PM_HD int imin(int a, int b) { return a < b ? a : b; }

// Block b is dispatched to XCD b % 8. Hand each XCD runs of kXcdChunk
// consecutive tiles so tiles that share operand panels share one L2. A
// permutation of [0, nblocks); blocks past the last full 256-block super-block
// keep their index.
PM_HD int xcd_remap(int b, int nblocks) {
  constexpr int per = kXcds * kXcdChunk;
  const int full = (nblocks / per) * per;
  if (b >= full) return b;
  const int w = b % per;
  return (b - w) + (w % kXcds) * kXcdChunk + (w / kXcds);
}

// Rectangular np x nq tile grid; lt in [0, np*nq).
PM_HD void full_tile(int lt, int np, int nq, int& ti, int& tj) {
  const int per_group = kGroupRows * nq;
  const int g = lt / per_group;
  const int g0 = g * kGroupRows;
  const int gm = imin(kGroupRows, np - g0);
  const int r = lt - g * per_group;
  ti = g0 + r % gm;
  tj = r / gm;
}

// The same np x nq grid walked column group by column group: kGroupCols
// columns at a time, and within a column group kGroupRows rows at a time
// (each such block column by column), so the kXcds blocks that run at once go
// down the rows of the same columns. For C = S·X, whose right operand (X's
// 256-column blocks, one per tile column) is the large one, the XCDs then read the same
// few column panels at the same time and the memory-side cache serves the
// repeats: each panel comes from HBM about once instead of once per row group.
constexpr int kGroupCols = 8;

PM_HD void full_tile_cols(int lt, int np, int nq, int& ti, int& tj) {
  const int per_cg = kGroupCols * np;  // tiles of a full column group
  const int cg = lt / per_cg;
  const int c0 = cg * kGroupCols;
  const int cw = imin(kGroupCols, nq - c0);
  const int r = lt - cg * per_cg;
  const int rg = r / (kGroupRows * cw);
  const int g0 = rg * kGroupRows;
  const int gm = imin(kGroupRows, np - g0);
  const int w = r - rg * kGroupRows * cw;
  ti = g0 + w % gm;
  tj = c0 + w / gm;
}

// Upper triangle (ti <= tj) of an nt x nt tile grid, grouped the same way;
// lt in [0, nt*(nt+1)/2).
PM_HD void sym_tile(int lt, int nt, int& ti, int& tj) {
  int rem = lt, g0 = 0, gm = 0;
  for (;; g0 += kGroupRows) {
    gm = imin(kGroupRows, nt - g0);
    const int cnt = gm * (gm + 1) / 2 + (nt - g0 - gm) * gm;
    if (rem < cnt) break;
    rem -= cnt;
  }
  const int tri = gm * (gm + 1) / 2;
  if (rem < tri) {  // columns g0 .. g0+gm-1 hold 1 .. gm tiles of the group
    int c = 0;
    while ((c + 1) * (c + 2) / 2 <= rem) ++c;
    ti = g0 + (rem - c * (c + 1) / 2);
    tj = g0 + c;
  } else {
    rem -= tri;
    ti = g0 + rem % gm;
    tj = g0 + gm + rem / gm;
  }
}

// K-split of one matrix's tiles in one stage: the number of chunks each tile's
// K loop (kt units of 64) is cut into, the chunks' fp32 partial tiles then
// summed in chunk order by a reduce launch. `tiles` is the stage's tile count
// over every engine matrix of the call (the launcher's split_call), so only a
// call that would leave most of the chip idle splits: tiles x chunks stays
// within one wave of 256 CUs. Each chunk keeps at least 16 units (a multiple
// of 4, the K loop's step; measured on a lone 1024 x 4096, chunks of 4 or 8
// units cost as much in partial traffic and the reduce launch as they saved),
// at most 4 chunks, and never below Mp = 512, so a small matrix and its
// 256-padded copy on the engine keep the same arithmetic.
constexpr int kMaxKSplit = 4;
constexpr int kSplitMinMp = 512;
constexpr int kSplitItems = 256;
constexpr int kSplitMinUnits = 16;

PM_HD int k_split(int mp, int tiles, int kt) {
  if (mp < kSplitMinMp || tiles <= 0 || kt % 4) return 1;
  int s = 1;
  while (2 * s <= kMaxKSplit && (kt / 4) % (2 * s) == 0 && kt / (2 * s) >= kSplitMinUnits &&
         tiles * 2 * s <= kSplitItems)
    s *= 2;
  return s;
}

// Work item lt of a matrix whose tiles are split into s chunks: chunk-major,
// so the items an XCD runs together share their chunk's K range.
PM_HD void split_item(int lt, int tiles, int& tile, int& chunk) {
  chunk = lt / tiles;
  tile = lt - chunk * tiles;
}

// Element offset of (r, c) in a workspace matrix with ld columns.
// Row-major: r·ld + c. Panel layout (tiled): the matrix is cut into panels of
// 256 rows (the GEMM tile) and each panel into units of 64 columns; unit
// (r/256, c/64) is a contiguous 32 KiB block of 256 rows of 128 bytes. A panel
// starts where it does row-major (row 256·i), and one unit of a panel is
// exactly what the GEMM engine streams into LDS per K step, so each of its
// 1 KiB copies (8 rows) reads contiguous memory. Needs ld a multiple of 64 and
// rows a multiple of 256 (the engine's padded extents). Runs of up to 8
// elements starting at a multiple of their length stay contiguous in both
// layouts.
PM_HD int64_t ws_off(int r, int c, int64_t ld, bool tiled) {
  if (!tiled) return (int64_t)r * ld + c;
  return ((((int64_t)(r >> 8) * (ld >> 6)) + (c >> 6)) << 14) + ((r & 255) << 6) + (c & 63);
}

// The same layout for a small matrix's X (128 x Np, one panel of 128 rows):
// unit c/64 is a contiguous 16 KiB block of 128 rows of 128 bytes.
PM_HD int64_t sm_x_off(int r, int c) { return ((int64_t)(c >> 6) << 13) + (r << 6) + (c & 63); }

// A unit of a small matrix's X in the apply's LDS ring: its 128 rows (k) of
// 64 columns (n), 128 B each, chunk c (16 B, columns 8c .. 8c+7) of row k
// stored at chunk c ^ xt_swz(k). The LDS serves a 64-lane read 16 lanes at a
// time; the 16 lanes of a transposed fragment read (ds_read_b64_tr_b16)
// address 4 consecutive rows, those of an a·X quad read 4 consecutive rows
// too, and those of the wide FINAL's read 16 consecutive rows: with k bits
// 1, 3 and 1 ^ 2 in the XOR each such group falls in distinct banks. (A XOR
// of k bits 3 and 4 alone put 2 or 4 lanes of a group on one bank: 53% of
// the apply's LDS cycles were bank conflicts.) Byte offset of (k, n):
PM_HD int xt_swz(int k) { return ((k >> 1) & 1) | (((k >> 3) & 1) << 1) | ((((k >> 1) ^ (k >> 2)) & 1) << 2); }
PM_HD int xt_off(int k, int n) { return k * 128 + ((((n >> 3) & 7) ^ xt_swz(k)) << 4) + (n & 7) * 2; }
// The unit's copies into the ring: copy q (0..15) writes its 1 KiB in order,
// lane l filling row k = 8q + l/8 at stored chunk l%8, so it reads the
// unit's (row-major, 128 B a row) bytes at this offset.
PM_HD int xt_copy_src(int q, int lane) {
  const int k = 8 * q + (lane >> 3);
  return k * 128 + (((lane & 7) ^ xt_swz(k)) << 4);
}

}  // namespace pm
