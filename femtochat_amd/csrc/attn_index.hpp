// Index arithmetic shared by the kernels and host-side checks: the grid
// orders that map a workgroup id to its (batch, head, tile) item, and the row
// clamp of the output epilogues.  Plain C++ when built without HIP, so the
// host harness (tests/sanitize/harness.cpp) checks these maps on the CPU.
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define FC_HD __host__ __device__
#else
#define FC_HD
#endif

namespace fc {

FC_HD inline int imin(int a, int b) { return a < b ? a : b; }
FC_HD inline int imax(int a, int b) { return a > b ? a : b; }

// Grid order for (row, tile) work items: all rows' heaviest tiles first
// (rank 0), then the next heaviest, and so on, so the last workgroups
// dispatched are the lightest and no long one starts near the end.  Rows
// are the inner index: the hardware sends workgroup id to XCD id % 8, so a
// row count divisible by 8 keeps each row (and its K/V in L2) on one XCD.
struct GridItem {
  int row, rank;
};
FC_HD inline GridItem heavy_first(int id, int rows) { return {id % rows, id / rows}; }

// (batch, query head) of query-side row r, numbered KV group member outer
// and (batch, KV head) inner: the heads that share a KV head are B*Hkv rows
// apart, on one XCD whenever B*Hkv is divisible by 8.
FC_HD inline void query_row(int r, int B, int Hkv, int group, int& b, int& h) {
  const int bkv = r % (B * Hkv), gi = r / (B * Hkv);
  b = bkv / Hkv;
  h = (bkv - b * Hkv) * group + gi;
}

// Position of item id in a list dealt to the XCDs in contiguous chunks: the
// hardware sends id to XCD id % 8, in increasing id, so XCD x runs list
// entries x*q + min(x, r) onward (q, r = n_items / 8, n_items % 8) in list
// order.
FC_HD inline int xcd_chunk_entry(int id, int n_items) {
  constexpr int X = 8;
  const int x = id % X, s = id / X, q = n_items / X, r = n_items % X;
  return x * q + imin(x, r) + s;
}

// (batch, query head, query tile) of item id in the row-local order, for a
// grid of B*Hkv*group*n_tiles items.  When the B*Hkv (batch, KV head) rows
// divide into 8, each XCD takes B*Hkv/8 whole rows: first their full query
// tiles (tile >= full_from, whose windows the sequence start does not cut),
// row after row, tiles last first, the KV head's group of query heads
// innermost; then their partial tiles, largest tile first, row after row.
// The full tiles all cost the same, so an XCD's workgroups end together and
// the hardware, which starts workgroups in order, finds a free slot for the
// next one at once (mixing partial tiles in left slots empty for
// microseconds); the tiles of a row, and the heads that share its K and V,
// run together on one XCD, whose L2 then serves them.  Otherwise the list runs
// over rows, tiles last first, then heads, in a contiguous part per XCD.
FC_HD inline void local_query_item(int id, int n_items, int n_tiles, int full_from, int B, int Hkv, int group,
                                        int& b, int& h, int& tile) {
  constexpr int X = 8;
  const int rows = B * Hkv;
  int bk, gi;
  if (rows % X == 0) {
    const int x = id % X, s = id / X, rx = rows / X;
    const int per_row = (n_tiles - full_from) * group;  // full items of a row
    const int full = rx * per_row;
    if (s < full) {
      const int r = s / per_row, rem = s - r * per_row;
      tile = n_tiles - 1 - rem / group;
      gi = rem % group;
      bk = x * rx + r;
    } else {
      const int s2 = s - full, per_tile = rx * group;  // partial items of one tile index
      const int k = s2 / per_tile, rem = s2 - k * per_tile;
      tile = full_from - 1 - k;
      bk = x * rx + rem / group;
      gi = rem % group;
    }
  } else {
    const int e = xcd_chunk_entry(id, n_items);
    gi = e % group;
    const int t = e / group;
    tile = n_tiles - 1 - t % n_tiles;
    bk = t / n_tiles;
  }
  b = bk / Hkv;
  h = (bk - b * Hkv) * group + gi;
}

// (batch, query head, query tile) of item id of a query-tile grid taken in a
// work order: order[k] = b * n_tiles + tile names the k-th tile, whose H
// heads are the ids k*H .. k*H + H-1, numbered like query_row's rows of one
// batch row (so the heads that share a KV head are Hkv ids apart).
FC_HD inline void ordered_query_item(int id, const int32_t* order, int n_tiles, int H, int Hkv, int group,
                                          int& b, int& h, int& tile) {
  const int k = id / H, hi = id - k * H;
  const int e = order[k];
  b = e / n_tiles;
  tile = e - b * n_tiles;
  int b0;
  query_row(hi, 1, Hkv, group, b0, h);
}

// First query tile of the row-local order whose queries' windows the
// sequence start does not cut: ceil(left / rows_per_tile), clamped to
// [0, n_tiles].  A window that starts right of its query (left < 0) is never
// cut; C division truncates toward zero, so the quotient alone is negative
// for left <= -rows_per_tile and must be clamped.
FC_HD inline int local_full_from(int n_tiles, int left, int rows_per_tile) {
  return imax(0, imin(n_tiles, (left + rows_per_tile - 1) / rows_per_tile));
}

// Row that an epilogue lane reads the caller's values from when
// accumulating: row q0 + row of the slice, or the slice's last row when that
// is past T (the value is then loaded but not used), so every load stays
// inside the (batch, head) slice whatever T is.
FC_HD inline int epilogue_row(int q0, int row, int T) { return imin(q0 + row, T - 1); }

}  // namespace fc
