// Device kernels of the level-wise tree engine (the caller side of the
// histogram / split ops: warpgbm/core.py grow_forest 692-744,
// grow_forest_multiclass 746-818, grow_tree 597-658).
//
// Row bookkeeping.  For a batch of T trees grown together (1 for regression,
// K class trees of one round for softmax), the rows of every live node are
// kept in one position array ORDER, grouped by SEGMENT key
//     key = ((tree * nodes_in_level) + node) * E + era
// and, inside a segment, in ascending row id (the stable partition keeps the
// order of the era-sorted root).  seg[key] .. seg[key+1] bounds a segment.
#include "common.hpp"
#include "engine.hpp"
#include "kernels.hpp"

namespace wgbm {

// ---------------------------------------------------------------------------
// residuals
// ---------------------------------------------------------------------------
// regression: r = y - pred (warpgbm/core.py:719); partial[block] = max |r|
__global__ void residual_regression_kernel(const float* __restrict__ y,
                                           const float* __restrict__ pred, int64_t n,
                                           float* __restrict__ r, uint32_t* __restrict__ partial) {
  uint32_t m = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const float v = y[i] - pred[i];
    r[i] = v;
    const uint32_t b = wgbm_abs_bits(v);
    m = b > m ? b : m;
  }
  m = wgbm_block_max_u32(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

// softmax: p = softmax(F[i, :]); residual_k = -(p_k - onehot_k)
// (warpgbm/core.py:186-214 and :782; metrics.py:12-15).
// partial[k * gridDim.x + block] = max_i |residual_k|
__global__ void residual_softmax_kernel(const float* __restrict__ logits,
                                        const int32_t* __restrict__ label, int64_t n, int32_t K,
                                        float* __restrict__ r /* [K][n] */,
                                        uint32_t* __restrict__ partial) {
  for (int k0 = 0; k0 < K; k0 += 8) {
    // up to 8 class maxima per pass over the rows
    uint32_t m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
      const float* x = logits + i * K;
      const int lab = label[i];
      float mx = x[0];
      for (int k = 1; k < K; ++k) mx = x[k] > mx ? x[k] : mx;
      float s = 0.0f;
      for (int k = 0; k < K; ++k) s = s + wgbm_expf(x[k] - mx);
      for (int kk = 0; kk < 8 && k0 + kk < K; ++kk) {
        const int k = k0 + kk;
        const float p = wgbm_expf(x[k] - mx) / s;
        const float g = p - (k == lab ? 1.0f : 0.0f);
        const float v = -g;
        r[(int64_t)k * n + i] = v;
        const uint32_t b = wgbm_abs_bits(v);
        m[kk] = b > m[kk] ? b : m[kk];
      }
    }
    for (int kk = 0; kk < 8 && k0 + kk < K; ++kk) {
      const uint32_t bm = wgbm_block_max_u32(m[kk]);
      if (threadIdx.x == 0) partial[(int64_t)(k0 + kk) * gridDim.x + blockIdx.x] = bm;
    }
  }
}

// ---------------------------------------------------------------------------
// root setup: every tree starts from the era-sorted order of all rows
// ---------------------------------------------------------------------------
__global__ void root_setup_kernel(const int32_t* __restrict__ root_order, int64_t n,
                                  int32_t T, const int64_t* __restrict__ era_start, int32_t E,
                                  int32_t* __restrict__ order, int64_t* __restrict__ seg,
                                  int32_t* __restrict__ present, int64_t* __restrict__ tot_q,
                                  int64_t* __restrict__ tot_c, unsigned long long* __restrict__ best,
                                  int32_t* __restrict__ agree_max) {
  // root segments, cleared root totals and cleared depth-0 split-pick words
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid < (int64_t)T * n) order[gid] = root_order[gid % n];
  if (gid < (int64_t)T * E) {
    const int t = (int)(gid / E);
    const int e = (int)(gid - (int64_t)t * E);
    seg[gid] = (int64_t)t * n + era_start[e];
    tot_q[gid] = 0;
    tot_c[gid] = 0;
  }
  if (gid == 0) seg[(int64_t)T * E] = (int64_t)T * n;
  if (gid < T) {
    present[gid] = 1;
    best[gid] = 0ull;
    if (agree_max) agree_max[gid] = 0;
  }
}

// sum of quantised residuals and row count per segment (root totals)
__global__ __launch_bounds__(256) void segment_totals_kernel(
    const Tile* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
    const int32_t* __restrict__ order, const float* __restrict__ resid, int64_t n,
    const int32_t* __restrict__ shifts, int32_t keys_per_tree, int64_t* __restrict__ tot_q,
    int64_t* __restrict__ tot_c) {
  const int tile = blockIdx.x;
  if (tile >= *n_tiles) return;
  const Tile tl = tiles[tile];
  const int t = tl.key / keys_per_tree;
  const int s = shifts[t];
  const float* r = resid + (int64_t)t * n;
  int64_t q = 0;
  for (int64_t p = tl.begin + threadIdx.x; p < tl.end; p += blockDim.x)
    q += wgbm_quantise(r[order[p]], s);
  q = wgbm_wave_sum(q);
  __shared__ int64_t sq[4];
  if ((threadIdx.x & 63) == 0) sq[threadIdx.x >> 6] = q;
  __syncthreads();
  if (threadIdx.x == 0) {
    const int64_t tq = sq[0] + sq[1] + sq[2] + sq[3];
    atomicAdd((unsigned long long*)&tot_q[tl.key], (unsigned long long)tq);
    atomicAdd((unsigned long long*)&tot_c[tl.key], (unsigned long long)(tl.end - tl.begin));
  }
}

// ---------------------------------------------------------------------------
// per-level bookkeeping: leaf values and the tree record
//   leaf value = mean of the node's residuals (warpgbm/core.py:599, :614),
//   computed from the exact quantised sum: float(ldexp(Sq, -s) / count)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(64) void level_finish_kernel(
    int32_t depth, int32_t max_depth, int32_t T, int32_t E, int32_t B,
    const int32_t* __restrict__ present, const unsigned long long* __restrict__ best,
    int32_t* __restrict__ split_l, int32_t* __restrict__ split_b,
    const float* __restrict__ split_gain_era, const int32_t* __restrict__ feat_sel,
    const int64_t* __restrict__ tot_q, const int64_t* __restrict__ tot_c,
    const int32_t* __restrict__ shifts, float* __restrict__ leaf_val, TreeRecord rec,
    int64_t* __restrict__ tot_q_next, int64_t* __restrict__ tot_c_next,
    unsigned long long* __restrict__ best_next, int32_t* __restrict__ agree_max_next) {
  // one wave per (tree, node); the eras are spread over the lanes.  The wave
  // also clears the next depth's words of its two children: their per-era
  // totals (accumulated by the partition) and their split-pick words.  With
  // best != null (one era) the packed pick of the split search is decoded here.
  const int nodes = 1 << depth;
  const int tn = blockIdx.x;
  const int lane = threadIdx.x;
  if (tn >= T * nodes) return;
  if (depth < max_depth) {
    const int64_t c0 = (int64_t)2 * tn * E;
    for (int k = lane; k < 2 * E; k += 64) {
      tot_q_next[c0 + k] = 0;
      tot_c_next[c0 + k] = 0;
    }
    if (depth + 1 < max_depth && lane < 2) {
      best_next[2 * tn + lane] = 0ull;
      if (agree_max_next) agree_max_next[2 * tn + lane] = 0;
    }
  }
  int l = -1, b = -1;
  float g1 = 0.0f;
  if (depth < max_depth) {
    if (best) {
      const unsigned long long k = best[tn];
      if (k != 0ull) {
        const int idx = (int)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
        l = idx / (B - 1);
        b = idx - l * (B - 1);
        g1 = gain_from_key((uint32_t)(k >> 32));
      }
      if (lane == 0) {
        split_l[tn] = l;
        split_b[tn] = b;
      }
    } else {
      l = split_l[tn];
      b = split_b[tn];
    }
  }
  const int t = tn / nodes;
  const int node = tn - t * nodes;
  const int64_t h = (int64_t)t * rec.H + (nodes - 1) + node;
  if (!present[tn]) {
    if (lane == 0) {
      rec.feat[h] = -2;
      rec.bin[h] = -1;
      rec.leaf[h] = 0.0f;
      rec.count[h] = 0;
    }
    return;
  }
  int64_t sq = 0, sc = 0;
  for (int e = lane; e < E; e += 64) {
    sq += tot_q[(int64_t)tn * E + e];
    sc += tot_c[(int64_t)tn * E + e];
  }
  for (int o = 32; o > 0; o >>= 1) {
    sq += __shfl_xor(sq, o, 64);
    sc += __shfl_xor(sc, o, 64);
  }
  if (lane == 0) {
    rec.count[h] = sc;
    if (l >= 0) {
      rec.feat[h] = feat_sel[l];
      rec.bin[h] = b;
      rec.leaf[h] = 0.0f;
    } else {
      const float v = (float)(ldexp((double)sq, -shifts[t]) / (double)sc);
      leaf_val[tn] = v;
      rec.feat[h] = -1;
      rec.bin[h] = -1;
      rec.leaf[h] = v;
    }
  }
  if (l >= 0) {
    if (best) {
      if (lane == 0) rec.gain[h] = g1;
    } else {
      for (int e = lane; e < E; e += 64) rec.gain[h * E + e] = split_gain_era[(int64_t)tn * E + e];
    }
  }
}

// ---------------------------------------------------------------------------
// partition, pass 1: per tile, route rows (code <= bin goes left,
// warpgbm/core.py:629), count lefts and accumulate child totals.  Tiles of a
// leaf node instead add lr * leaf to the rows' predictions (core.py:602-605).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void partition_count_kernel(
    const Tile* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
    const int32_t* __restrict__ order, int32_t E, int32_t nodes, int32_t max_split_depth_ok,
    const int32_t* __restrict__ split_l, const int32_t* __restrict__ split_b,
    const int32_t* __restrict__ feat_sel, const int8_t* __restrict__ codes_cm, int64_t n,
    const float* __restrict__ resid, const int32_t* __restrict__ shifts,
    const float* __restrict__ leaf_val, float lr, float* __restrict__ pred, int64_t pstride,
    int64_t pcol, uint8_t* __restrict__ dirbit, int32_t* __restrict__ tile_left,
    int64_t* __restrict__ tot_q_next, int64_t* __restrict__ tot_c_next) {
  const int tile = blockIdx.x;
  if (tile >= *n_tiles) return;
  const Tile tl = tiles[tile];
  const int tn = tl.key / E;
  const int e = tl.key - tn * E;
  const int t = tn / nodes;
  const int node = tn - t * nodes;
  const int l = max_split_depth_ok ? split_l[tn] : -1;
  if (l < 0) {
    const float v = lr * leaf_val[tn];
    float* pc = pred + (int64_t)t * pcol;
    for (int64_t p = tl.begin + threadIdx.x; p < tl.end; p += blockDim.x) {
      const int64_t row = order[p];
      pc[row * pstride] = pc[row * pstride] + v;
    }
    if (threadIdx.x == 0) tile_left[tile] = 0;
    return;
  }
  const int8_t* col = codes_cm + (int64_t)feat_sel[l] * n;
  const int sb = split_b[tn];
  const int s = shifts[t];
  const float* r = resid + (int64_t)t * n;
  int64_t ql = 0, qr = 0;
  int32_t nl = 0, nr = 0;
  for (int64_t p = tl.begin + threadIdx.x; p < tl.end; p += blockDim.x) {
    const int32_t row = order[p];
    const bool right = (int)col[row] > sb;
    dirbit[p] = right ? 1 : 0;
    const int64_t q = wgbm_quantise(r[row], s);
    if (right) {
      qr += q;
      ++nr;
    } else {
      ql += q;
      ++nl;
    }
  }
  ql = wgbm_wave_sum(ql);
  qr = wgbm_wave_sum(qr);
  nl = wgbm_wave_sum(nl);
  nr = wgbm_wave_sum(nr);
  __shared__ int64_t s_ql[4], s_qr[4];
  __shared__ int32_t s_nl[4], s_nr[4];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_ql[w] = ql;
    s_qr[w] = qr;
    s_nl[w] = nl;
    s_nr[w] = nr;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int64_t a = 0, b = 0;
    int32_t c = 0, d = 0;
    for (int k = 0; k < 4; ++k) {
      a += s_ql[k];
      b += s_qr[k];
      c += s_nl[k];
      d += s_nr[k];
    }
    tile_left[tile] = c;
    const int64_t kl = (((int64_t)t * 2 * nodes) + 2 * node) * E + e;
    const int64_t kr = kl + E;
    atomicAdd((unsigned long long*)&tot_q_next[kl], (unsigned long long)a);
    atomicAdd((unsigned long long*)&tot_q_next[kr], (unsigned long long)b);
    atomicAdd((unsigned long long*)&tot_c_next[kl], (unsigned long long)c);
    atomicAdd((unsigned long long*)&tot_c_next[kr], (unsigned long long)d);
  }
}

// ---------------------------------------------------------------------------
// partition, pass 2 (one workgroup of 1024): segment sizes of the next level,
// their offsets, per-tile output bases, next-level presence and the list of
// segments whose histogram is built at the next level (the smaller child of
// every split, warpgbm/core.py:636-643; the other child is parent - child).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void partition_scan_kernel(
    int32_t T, int32_t nodes, int32_t E, const int64_t* __restrict__ seg,
    const Tile* __restrict__ tiles, const int32_t* __restrict__ key_tile_start,
    const int32_t* __restrict__ n_tiles_dev, const int32_t* __restrict__ tile_left,
    const int32_t* __restrict__ split_l, int64_t* __restrict__ Lk,
    int64_t* __restrict__ tile_lbase, int64_t* __restrict__ tile_rbase,
    int64_t* __restrict__ seg_next, int32_t* __restrict__ present_next,
    int32_t* __restrict__ key_list_next) {
  __shared__ int64_t wsum[16];
  __shared__ int64_t sbuf[kScanK * 1024];
  const int n_keys = T * nodes * E;
  const int n_tiles = *n_tiles_dev;
  // phase 1: exclusive scan of the left counts over all tiles (tiles of a
  // segment are consecutive), kept in tile_lbase for now
  const int64_t lefts = wgbm_block_scan_tiled(
      n_tiles, [&](int t) { return (int64_t)tile_left[t]; },
      [&](int t, int64_t v) { tile_lbase[t] = v; }, wsum, sbuf);
  __syncthreads();
  // lefts per segment: difference of the scan at its first tile and the next
  // segment's first tile
  for (int k = threadIdx.x; k < n_keys; k += blockDim.x) {
    const int t0 = key_tile_start[k], t1 = key_tile_start[k + 1];
    const int64_t a = t0 < n_tiles ? tile_lbase[t0] : lefts;
    const int64_t b = t1 < n_tiles ? tile_lbase[t1] : lefts;
    Lk[k] = t1 > t0 ? b - a : 0;
  }
  __syncthreads();
  // phase 2: exclusive scan of next-level segment sizes
  const int nodes2 = 2 * nodes;
  const int n_next = T * nodes2 * E;
  const int64_t total_next = wgbm_block_scan_tiled(
      n_next,
      [&](int k2) -> int64_t {
        const int e = k2 % E;
        const int tc = k2 / E;
        const int t = tc / nodes2;
        const int c = tc - t * nodes2;
        const int tn = t * nodes + (c >> 1);
        if (split_l[tn] < 0) return 0;
        const int k = tn * E + e;
        const int64_t cnt = seg[k + 1] - seg[k];
        return (c & 1) ? cnt - Lk[k] : Lk[k];
      },
      [&](int k2, int64_t v) { seg_next[k2] = v; }, wsum, sbuf);
  if (threadIdx.x == 0) seg_next[n_next] = total_next;
  __syncthreads();
  // phase 3: per-tile output bases (one thread per tile).  The left prefix
  // inside the segment is taken first (into tile_rbase) for every tile, since
  // the bases then overwrite the scan the prefixes are read from.
  for (int tt = threadIdx.x; tt < n_tiles; tt += blockDim.x)
    tile_rbase[tt] = tile_lbase[tt] - tile_lbase[key_tile_start[tiles[tt].key]];
  __syncthreads();
  for (int tt = threadIdx.x; tt < n_tiles; tt += blockDim.x) {
    const Tile tl = tiles[tt];
    const int k = tl.key;
    const int tn = k / E;
    if (split_l[tn] < 0) continue;
    const int e = k - tn * E;
    const int t = tn / nodes;
    const int node = tn - t * nodes;
    const int64_t kl = ((int64_t)t * nodes2 + 2 * node) * E + e;
    const int64_t kr = kl + E;
    const int64_t lpre = tile_rbase[tt];
    const int64_t before = tl.begin - seg[k];
    tile_lbase[tt] = seg_next[kl] + lpre;
    tile_rbase[tt] = seg_next[kr] + (before - lpre);
  }
  // phase 4: presence and the histogram key list of the next level; one wave
  // per (tree, node), the eras spread over its lanes
  const int lane = threadIdx.x & 63;
  for (int tn = threadIdx.x >> 6; tn < T * nodes; tn += blockDim.x >> 6) {
    const bool sp = split_l[tn] >= 0;
    const int t = tn / nodes;
    const int node = tn - t * nodes;
    if (lane == 0) {
      present_next[t * nodes2 + 2 * node] = sp;
      present_next[t * nodes2 + 2 * node + 1] = sp;
    }
    int64_t ls = 0, tot = 0;
    if (sp)
      for (int e = lane; e < E; e += 64) {
        const int k = tn * E + e;
        ls += Lk[k];
        tot += seg[k + 1] - seg[k];
      }
    for (int o = 32; o > 0; o >>= 1) {
      ls += __shfl_xor(ls, o, 64);
      tot += __shfl_xor(tot, o, 64);
    }
    const int side = (ls <= tot - ls) ? 0 : 1;
    for (int e = lane; e < E; e += 64)
      key_list_next[tn * E + e] =
          sp ? (int32_t)(((int64_t)t * nodes2 + 2 * node + side) * E + e) : -1;
  }
}

// ---------------------------------------------------------------------------
// partition, pass 3: stable scatter of the rows of split nodes
__global__ __launch_bounds__(256) void partition_scatter_kernel(
    const Tile* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
    const int32_t* __restrict__ order, int32_t E, const int32_t* __restrict__ split_l,
    const uint8_t* __restrict__ dirbit, const int64_t* __restrict__ tile_lbase,
    const int64_t* __restrict__ tile_rbase, int32_t* __restrict__ order_next) {
  const int tile = blockIdx.x;
  if (tile >= *n_tiles) return;
  const Tile tl = tiles[tile];
  if (split_l[tl.key / E] < 0) return;
  __shared__ int32_t wl[4];
  int64_t lb = tile_lbase[tile], rb = tile_rbase[tile];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int64_t base = tl.begin; base < tl.end; base += blockDim.x) {
    const int64_t p = base + threadIdx.x;
    const bool ok = p < tl.end;
    const bool right = ok && dirbit[p];
    const bool left = ok && !right;
    const unsigned long long ml = __ballot(left);
    const int rank_in_wave = __popcll(ml & __lanemask_lt());
    if (lane == 0) wl[w] = __popcll(ml);
    __syncthreads();
    int pre = 0, tot = 0;
    for (int k = 0; k < 4; ++k) {
      if (k < w) pre += wl[k];
      tot += wl[k];
    }
    const int64_t chunk_n = (tl.end - base) < blockDim.x ? (tl.end - base) : blockDim.x;
    if (ok) {
      const int lrank = pre + rank_in_wave;
      const int64_t idx = p - base;  // position inside the chunk
      if (left)
        order_next[lb + lrank] = order[p];
      else
        order_next[rb + (idx - lrank)] = order[p];
    }
    lb += tot;
    rb += chunk_n - tot;
    __syncthreads();
  }
}

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace wgbm
