// Tile planner shared by the histogram entry points and the engine.
#pragma once
#include "common.hpp"
#include "kernels.hpp"

namespace wgbm {

// --------------------------------------------------------------------------
// tile planner: one workgroup scans segment lengths and splits every segment
// into near-equal tiles that never cross a segment: ceil(len / tile_rows)
// tiles (tiles never exceed tile_rows), or with nearest != 0
// round(len / tile_rows) (at least one, and at most WGBM_MAX_TILE_ROWS rows
// each: a call sized for one workgroup per CU gets exactly that).  No tile is
// a small remainder, so the workgroups of a launch carry even work.  keys:
// either all n_keys (list == nullptr) or the first *n_list entries of
// key_list.  seg: int64 [n_keys+1] (nullptr => a single segment [0, total)).
// --------------------------------------------------------------------------
// (blockDim.x == 1024)
__device__ inline void plan_tiles_body(
    const int64_t* __restrict__ seg, int64_t total_rows, int32_t n_keys,
    const int32_t* __restrict__ key_list, int32_t tile_rows, int32_t nearest,
    int32_t max_tiles, Tile* __restrict__ tiles, int32_t* __restrict__ key_tile_start,
    int32_t* __restrict__ n_tiles) {
  __shared__ int64_t wsum[16];
  __shared__ int64_t sbuf[kScanK * 1024];
  const int nk = n_keys;  // entries of key_list (or keys 0..n_keys-1)
  auto bounds = [&](int i, int& key, int64_t& b0, int64_t& b1) {
    key = key_list ? key_list[i] : i;
    b0 = (key >= 0 && seg) ? seg[key] : 0;
    b1 = key < 0 ? 0 : (seg ? seg[key + 1] : total_rows);
  };
  // segment lengths are below 2^31 (positions are int32): 32-bit divisions
  auto count = [&](int64_t len64) -> int64_t {
    if (len64 <= 0) return 0;
    const uint32_t len = (uint32_t)len64;
    const uint32_t up = (uint32_t)(nearest ? tile_rows / 2 : tile_rows - 1);
    const uint32_t k = (len + up) / (uint32_t)tile_rows;
    static_assert(WGBM_MAX_TILE_ROWS == 1 << 16, "tile row bound");
    const uint32_t kmin = (len + WGBM_MAX_TILE_ROWS - 1) >> 16;
    return k > kmin ? k : kmin;
  };
  // phase 1: exclusive scan of the tile counts -> key_tile_start
  const int64_t total = wgbm_block_scan_tiled(
      nk,
      [&](int i) -> int64_t {
        int key;
        int64_t b0, b1;
        bounds(i, key, b0, b1);
        return key < 0 ? 0 : count(b1 - b0);
      },
      [&](int i, int64_t v) { key_tile_start[i] = (int32_t)v; }, wsum, sbuf);
  const int ntot = total < max_tiles ? (int)total : max_tiles;
  if (threadIdx.x == 0) {
    key_tile_start[nk] = (int32_t)total;
    *n_tiles = ntot;
  }
  __syncthreads();
  // phase 2: every entry writes its own tiles (ids below the tile limit);
  // entries with many tiles are written by the whole workgroup afterwards
  constexpr int kMaxBig = 256, kSmall = 8;
  __shared__ int big[kMaxBig];
  __shared__ int n_big;
  if (threadIdx.x == 0) n_big = 0;
  __syncthreads();
  // tile j of a segment split into nt: q = len / nt rows, the first r = len %
  // nt tiles one more
  auto write_tile = [&](int key, int64_t b0, uint32_t q, uint32_t r, int first, int j) {
    const uint32_t uj = (uint32_t)j;
    Tile tl;
    tl.key = key;
    tl.pad = 0;
    tl.begin = b0 + (int64_t)(uj * q + (uj < r ? uj : r));
    tl.end = tl.begin + (int64_t)(q + (uj < r ? 1u : 0u));
    tiles[first + j] = tl;
  };
  for (int i = threadIdx.x; i < nk; i += blockDim.x) {
    int key;
    int64_t b0, b1;
    bounds(i, key, b0, b1);
    if (key < 0) continue;
    const int first = key_tile_start[i];
    const int nt = key_tile_start[i + 1] - first;
    if (nt > kSmall) {
      const int slot = atomicAdd(&n_big, 1);
      if (slot < kMaxBig) {
        big[slot] = i;
        continue;
      }
    }
    const uint32_t len = (uint32_t)(b1 - b0), q = len / (uint32_t)nt, r = len - q * (uint32_t)nt;
    for (int j = 0; j < nt && first + j < ntot; ++j) write_tile(key, b0, q, r, first, j);
  }
  __syncthreads();
  const int nb = n_big < kMaxBig ? n_big : kMaxBig;
  for (int k = 0; k < nb; ++k) {
    const int i = big[k];
    int key;
    int64_t b0, b1;
    bounds(i, key, b0, b1);
    const int first = key_tile_start[i];
    const int nt = key_tile_start[i + 1] - first;
    const uint32_t len = (uint32_t)(b1 - b0), q = len / (uint32_t)nt, r = len - q * (uint32_t)nt;
    for (int j = threadIdx.x; j < nt && first + j < ntot; j += blockDim.x)
      write_tile(key, b0, q, r, first, j);
  }
}

}  // namespace wgbm
