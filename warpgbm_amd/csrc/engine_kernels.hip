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
#include "plan.hpp"
#include "split_scan.hpp"

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
constexpr int kSoftmaxRegK = 16;  // classes whose logits a thread holds in registers
__global__ void residual_softmax_kernel(const float* __restrict__ logits /* [K][n] */,
                                        const int32_t* __restrict__ label, int64_t n, int32_t K,
                                        float* __restrict__ r /* [K][n] */,
                                        uint32_t* __restrict__ partial) {
  if (K <= kSoftmaxRegK) {
    // one pass: a row's K logits in registers (fully unrolled: no dynamic
    // register index), max, the exponentials (each computed once, used for
    // the sum and the probability: the same values), every class's
    // residual; then every class's block maximum with one LDS exchange
    uint32_t m[kSoftmaxRegK];
#pragma unroll
    for (int k = 0; k < kSoftmaxRegK; ++k) m[k] = 0u;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
      const float* x = logits + i;
      const int lab = label[i];
      float xr[kSoftmaxRegK];
#pragma unroll
      for (int k = 0; k < kSoftmaxRegK; ++k) xr[k] = x[(k < K ? k : 0) * n];
      float mx = xr[0];
#pragma unroll
      for (int k = 1; k < kSoftmaxRegK; ++k)
        if (k < K) mx = xr[k] > mx ? xr[k] : mx;
      float ex[kSoftmaxRegK];
      float sum = 0.0f;
#pragma unroll
      for (int k = 0; k < kSoftmaxRegK; ++k) {
        ex[k] = k < K ? wgbm_expf(xr[k] - mx) : 0.0f;
        if (k < K) sum = sum + ex[k];
      }
#pragma unroll
      for (int k = 0; k < kSoftmaxRegK; ++k) {
        if (k < K) {
          const float g = ex[k] / sum - (k == lab ? 1.0f : 0.0f);
          const float v = -g;
          r[(int64_t)k * n + i] = v;
          const uint32_t b = wgbm_abs_bits(v);
          m[k] = b > m[k] ? b : m[k];
        }
      }
    }
    __shared__ uint32_t s_m[kSoftmaxRegK][16];  // [class][wave]
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
#pragma unroll
    for (int k = 0; k < kSoftmaxRegK; ++k) {
      if (k < K) {
        const uint32_t wm = wgbm_wave_max_u32(m[k]);
        if ((threadIdx.x & 63) == 0) s_m[k][w] = wm;
      }
    }
    __syncthreads();
    if ((int)threadIdx.x < K) {
      const int k = threadIdx.x;
      uint32_t bm = 0u;
      for (int j = 0; j < nw; ++j) bm = s_m[k][j] > bm ? s_m[k][j] : bm;
      partial[(int64_t)k * gridDim.x + blockIdx.x] = bm;
    }
    return;
  }
  for (int k0 = 0; k0 < K; k0 += 8) {
    // up to 8 class maxima per pass over the rows
    uint32_t m[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
      // the row's K logits, class-major (one coalesced read per class)
      const float* x = logits + i;
      const int lab = label[i];
      float mx = x[0];
      for (int k = 1; k < K; ++k) mx = x[k * n] > mx ? x[k * n] : mx;
      float s = 0.0f;
      for (int k = 0; k < K; ++k) s = s + wgbm_expf(x[k * n] - mx);
      for (int kk = 0; kk < 8 && k0 + kk < K; ++kk) {
        const int k = k0 + kk;
        const float g = wgbm_expf(x[k * n] - mx) / s - (k == lab ? 1.0f : 0.0f);
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
                                  const float* __restrict__ resid, int32_t* __restrict__ order,
                                  int32_t* __restrict__ keyp, float* __restrict__ rpos,
                                  int64_t* __restrict__ seg, int32_t* __restrict__ present,
                                  unsigned long long* __restrict__ best,
                                  int32_t* __restrict__ agree_max,
                                  const int32_t* __restrict__ shifts,
                                  int32_t* __restrict__ node_shift) {
  // root order, segment key and residual of every position, root segments,
  // the roots' histogram shifts (the trees' own) and cleared depth-0
  // split-pick words
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid < (int64_t)T * n) {
    const int64_t t = gid / n, p = gid - t * n;
    const int32_t row = root_order[p];
    order[gid] = row;
    rpos[gid] = resid[t * n + row];
    int lo = 0, hi = E - 1;  // the era e with era_start[e] <= p < era_start[e + 1]
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (era_start[mid] <= p) lo = mid; else hi = mid - 1;
    }
    keyp[gid] = (int32_t)(t * E + lo);
  }
  if (gid < (int64_t)T * E) {
    const int t = (int)(gid / E);
    const int e = (int)(gid - (int64_t)t * E);
    seg[gid] = (int64_t)t * n + era_start[e];
  }
  if (gid == 0) seg[(int64_t)T * E] = (int64_t)T * n;
  if (gid < T) {
    present[gid] = 1;
    // one era: the root's key is its tree; several eras: root_totals_kernel
    // writes every (tree, era) key's own shift
    if (E == 1) node_shift[gid] = shifts[gid];
    best[gid] = 0ull;
    if (agree_max) agree_max[gid] = 0;
  }
}

// One era (E == 1): root_setup_kernel's words, and each tree's root totals
// in the same launch: the exact sums over the tree's rows of the wide
// quantisation q63 = rint(r * 2^s63), s63 = shifts[t] + s63_add, held as
// qh = sum (q63 >> 32) and ql = sum (q63 & (2^32 - 1)) (the words the root
// route + block scan + root_totals_kernel give).  Grid (ceil(n /
// kRootE1Span), T): a workgroup holds kRootE1Span positions of one tree and
// adds its sums to the tree's words with one relaxed atomic each (integer
// sums: any order gives the same words); absmax_finish_kernel cleared them
// and set the row count.  No fence: the next launch sees the sums.
__global__ __launch_bounds__(1024) void root_setup_e1_kernel(
    const int32_t* __restrict__ root_order, int64_t n, int32_t T, const float* __restrict__ resid,
    int32_t* __restrict__ order, int32_t* __restrict__ keyp, float* __restrict__ rpos,
    int64_t* __restrict__ seg, int32_t* __restrict__ present, unsigned long long* __restrict__ best,
    const int32_t* __restrict__ shifts, int32_t s63_add, int32_t* __restrict__ node_shift,
    int64_t* __restrict__ tot_qh, int64_t* __restrict__ tot_ql) {
  constexpr int kThreads = 1024, kWaves = kThreads / 64;
  constexpr int PJ = kRootE1Span / kThreads;  // positions per thread, loads issued together
  __shared__ int64_t s_qh[kWaves], s_ql[kWaves];
  const int t = (int)blockIdx.y;
  const int tid = (int)threadIdx.x;
  const int s63 = shifts[t] + s63_add;
  const int64_t p0 = (int64_t)blockIdx.x * kRootE1Span;
  const int64_t tb = (int64_t)t * n;
  int32_t rows[PJ];
  float rv[PJ];
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int64_t p = p0 + j * kThreads + tid;
    rows[j] = p < n ? root_order[p] : 0;
  }
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int64_t p = p0 + j * kThreads + tid;
    rv[j] = p < n ? resid[tb + rows[j]] : 0.0f;
  }
  int64_t qh = 0, ql = 0;
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int64_t p = p0 + j * kThreads + tid;
    if (p < n) {
      order[tb + p] = rows[j];
      rpos[tb + p] = rv[j];
      keyp[tb + p] = t;
      const int64_t q = (int64_t)rintf(ldexpf(rv[j], s63));
      qh += q >> 32;
      ql += q & 0xffffffffll;
    }
  }
  if (blockIdx.x == 0 && tid == 0) {
    seg[t] = tb;
    if (t == 0) seg[T] = (int64_t)T * n;
    present[t] = 1;
    node_shift[t] = shifts[t];
    best[t] = 0ull;
  }
  qh = wgbm_wave_reduce_add_i64(qh);
  ql = wgbm_wave_reduce_add_i64(ql);
  if ((tid & 63) == 0) {
    s_qh[tid >> 6] = qh;
    s_ql[tid >> 6] = ql;
  }
  __syncthreads();
  if (tid == 0) {
    int64_t a = 0, b = 0;
    for (int k = 0; k < kWaves; ++k) {
      a += s_qh[k];
      b += s_ql[k];
    }
    if (a) atomicAdd((unsigned long long*)(tot_qh + t), (unsigned long long)a);
    if (b) atomicAdd((unsigned long long*)(tot_ql + t), (unsigned long long)b);
  }
}

// ---------------------------------------------------------------------------
// per-level bookkeeping: leaf values and the tree record
//   leaf value = mean of the node's residuals (warpgbm/core.py:599, :614),
//   from the exact sum of the wide quantisation q63 = rint(r * 2^s63),
//   s63 = s + s63_add (|q63| < 2^62), held as qh = sum (q63 >> 32) and
//   ql = sum (q63 & (2^32 - 1)):  H = qh + (ql >> 32), L = ql mod 2^32,
//   leaf = float(ldexp(double(H) * 2^32 + double(L), -s63) / count)
// ---------------------------------------------------------------------------
// The leaf / record step of one (tree, node), by one wave (lane = 0..63).
// have_key: the packed pick of the one-era split search is `key` (the fused
// split kernel's own result); else it is read from best (one era), or the
// era path's split_l / split_b are used.
__device__ inline void finish_node(
    int tn, int lane, int32_t depth, int32_t max_depth, int32_t T, int32_t E, int32_t B,
    const int32_t* __restrict__ present, bool have_key, unsigned long long key,
    const unsigned long long* __restrict__ best, int32_t* __restrict__ split_l,
    int32_t* __restrict__ split_b, const float* __restrict__ split_gain_era,
    const int32_t* __restrict__ feat_sel, const int64_t* __restrict__ tot_qh,
    const int64_t* __restrict__ tot_ql, const int64_t* __restrict__ tot_c,
    const int32_t* __restrict__ shifts, int32_t s63_add, float* __restrict__ leaf_val,
    const TreeRecord& rec, unsigned long long* __restrict__ best_next,
    int32_t* __restrict__ agree_max_next, NodeRoute* __restrict__ nroute) {
  const int nodes = 1 << depth;
  if (depth + 1 < max_depth && lane < 2) {
    best_next[2 * tn + lane] = 0ull;
    if (agree_max_next) agree_max_next[2 * tn + lane] = 0;
  }
  int l = -1, b = -1;
  float g1 = 0.0f;
  const bool one_era_pick = have_key || best;
  if (depth < max_depth) {
    if (one_era_pick) {
      const unsigned long long k = have_key ? key : best[tn];
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
      nroute[tn] = NodeRoute{-2, -1, 0.0f, 0};
    }
    return;
  }
  int64_t sqh = 0, sql = 0, sc = 0;
  {
    // the node's era words, U per lane and round with their loads issued
    // together (an era past the end re-reads the node's first and adds 0)
    constexpr int U = 4;
    const int64_t k0 = (int64_t)tn * E;
    for (int e0 = lane; e0 < E; e0 += U * 64) {
      int64_t a[U], b[U], c[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int e = e0 + u * 64;
        const int64_t k = k0 + (e < E ? e : 0);
        a[u] = tot_qh[k];
        b[u] = tot_ql[k];
        c[u] = tot_c[k];
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const bool in = e0 + u * 64 < E;
        sqh += in ? a[u] : 0;
        sql += in ? b[u] : 0;
        sc += in ? c[u] : 0;
      }
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    sqh += __shfl_xor(sqh, o, 64);
    sql += __shfl_xor(sql, o, 64);
    sc += __shfl_xor(sc, o, 64);
  }
  if (lane == 0) {
    rec.count[h] = sc;
    const int32_t s63 = shifts[t] + s63_add;
    if (l >= 0) {
      const int32_t col = feat_sel[l];
      rec.feat[h] = col;
      rec.bin[h] = b;
      rec.leaf[h] = 0.0f;
      nroute[tn] = NodeRoute{col, b, 0.0f, s63};
    } else {
      const int64_t hi = sqh + (sql >> 32);
      const int64_t lo = sql & 0xffffffffll;
      const double sum = (double)hi * 4294967296.0 + (double)lo;
      const float v = (float)(ldexp(sum, -s63) / (double)sc);
      leaf_val[tn] = v;
      rec.feat[h] = -1;
      rec.bin[h] = -1;
      rec.leaf[h] = v;
      nroute[tn] = NodeRoute{-1, -1, v, s63};
    }
  }
  if (l >= 0) {
    if (one_era_pick) {
      if (lane == 0) rec.gain[h] = g1;
    } else {
      for (int e = lane; e < E; e += 64) rec.gain[h * E + e] = split_gain_era[(int64_t)tn * E + e];
    }
  }
}

__global__ __launch_bounds__(64) void level_finish_kernel(
    int32_t depth, int32_t max_depth, int32_t T, int32_t E, int32_t B,
    const int32_t* __restrict__ present, const unsigned long long* __restrict__ best,
    int32_t* __restrict__ split_l, int32_t* __restrict__ split_b,
    const float* __restrict__ split_gain_era, const int32_t* __restrict__ feat_sel,
    const int64_t* __restrict__ tot_qh, const int64_t* __restrict__ tot_ql,
    const int64_t* __restrict__ tot_c, const int32_t* __restrict__ shifts, int32_t s63_add,
    float* __restrict__ leaf_val, TreeRecord rec,
    unsigned long long* __restrict__ best_next, int32_t* __restrict__ agree_max_next,
    NodeRoute* __restrict__ nroute) {
  // one wave per (tree, node); the eras are spread over the lanes.  The wave
  // also clears the next depth's split-pick words of its two children.  With
  // best != null (one era) the packed pick of the split search is decoded here.
  const int tn = blockIdx.x;
  if (tn >= T * (1 << depth)) return;
  finish_node(tn, threadIdx.x, depth, max_depth, T, E, B, present, false, 0ull, best, split_l,
              split_b, split_gain_era, feat_sel, tot_qh, tot_ql, tot_c, shifts, s63_add,
              leaf_val, rec, best_next, agree_max_next, nroute);
}

// ---------------------------------------------------------------------------
// Partition over position blocks.
//
// Rows stay in the position space [0, T*N) of the whole round: a node that
// does not split (a leaf, or a node under a leaf) keeps its rows where they
// are -- its left child gets all of them, its right child none -- so the
// next level's segments of one parent node cover exactly the parent's
// position range, left child eras first, then right child eras:
//     next key of (tree t, child 2*node + side, era e) = 2*tn*E + side*E + e,
// and the next level's offsets come from a scan over the node's own eras
// (no scan over all segments).  The blocks below are fixed ranges of
// kPartBlock positions, independent of the segment boundaries, so a level
// with many small segments (deep DES levels: 2^d nodes x 500 eras) costs the
// same launches as one with a single segment.
//
// Every position also carries its segment key (keyp) and its row's residual
// (rpos), written by the root setup and by each level's scatter for the next
// level: the kernels of a level read them contiguously instead of gathering
// by row id.
//
// route:   direction of every row of a split node (code <= bin goes left,
//          warpgbm/core.py:629) and leaf update of the rows of a node that
//          stops here (core.py:602-605).  The left rows of every segment and
//          their quantised residual sum are reduced per block in LDS; a
//          segment that lies inside the block stores them to its key's words
//          (own_*), and the block stores those of its first and last segments
//          as block partials (bf_*, bl_*).  Mode 0 counts every row as left
//          (root totals).  There are no global atomics: every word written
//          has one writer.
// block_scan: inclusive prefix P over the blocks of the first-segment
//          partials.  A segment whose positions span blocks b0 < b1 sums to
//          bl[b0] + P[b1] - P[b0]: its part in b0 is b0's last segment and it
//          is the first segment of every block in (b0, b1].
// node_scan: one to four waves per (tree, node): those sums, the next level's segment
//          offsets and child totals (left = the sums, right = the parent's
//          total minus them), the presence of the children and the histogram
//          key list (the smaller child of every split, core.py:636-643).
// scatter: stable destination of every row: left rank in its segment = left
//          rows before it in the block (ballot prefix) - left rows before the
//          segment's start in the block (+ its left rows in earlier blocks,
//          from the same partial sums, when it began in an earlier block).
// ---------------------------------------------------------------------------
__device__ inline void segment_left_sums_at(int64_t k, int64_t s0, int64_t s1,
                                            const PartSums& ps, int64_t& qh, int64_t& ql,
                                            int64_t& n);
__device__ inline void segment_left_sums(int64_t k, const int64_t* __restrict__ seg,
                                         const PartSums& ps, int64_t& qh, int64_t& ql,
                                         int64_t& n) {
  segment_left_sums_at(k, seg[k], seg[k + 1], ps, qh, ql, n);
}
// the same, for segment k at positions [s0, s1)
__device__ inline void segment_left_sums_at(int64_t k, int64_t s0, int64_t s1,
                                            const PartSums& ps, int64_t& qh, int64_t& ql,
                                            int64_t& n) {
  if (s1 <= s0) {
    qh = 0;
    ql = 0;
    n = 0;
    return;
  }
  const int64_t b0 = s0 / kPartBlock, b1 = (s1 - 1) / kPartBlock;
  if (b0 == b1) {
    qh = ps.own_qh[k];
    ql = ps.own_ql[k];
    n = ps.own_n[k];
  } else {
    qh = ps.bl_qh[b0] + ps.P_qh[b1] - ps.P_qh[b0];
    ql = ps.bl_ql[b0] + ps.P_ql[b1] - ps.P_ql[b0];
    n = ps.bl_n[b0] + ps.P_n[b1] - ps.P_n[b0];
  }
}

// Max of the left (ml) and right (mr) residual magnitudes (float bits) of
// the rows of segment k (one era: the node), whose positions are [P0, P1):
// its own words when it lies inside one block, else the last-segment
// partial of its first block and the first-segment partials of the blocks
// after it (the segment is their first segment).  The gthreads threads of a
// group share the blocks; the caller reduces the maximum over the group.
__device__ inline void seg_child_max(int64_t k, int64_t P0, int64_t P1, const PartSums& ps,
                                     int gt, int gthreads, uint32_t& ml, uint32_t& mr) {
  ml = 0;
  mr = 0;
  if (P1 <= P0) return;
  const int64_t b0 = P0 / kPartBlock, b1 = (P1 - 1) / kPartBlock;
  if (b0 == b1) {
    if (gt == 0) {
      ml = ps.own_ml[k];
      mr = ps.own_mr[k];
    }
    return;
  }
  if (gt == 0) {
    ml = ps.bl_ml[b0];
    mr = ps.bl_mr[b0];
  }
  for (int64_t b = b0 + 1 + gt; b <= b1; b += gthreads) {
    const uint32_t l = ps.bf_ml[b], r = ps.bf_mr[b];
    ml = l > ml ? l : ml;
    mr = r > mr ? r : mr;
  }
}

__global__ __launch_bounds__(kPartThreads) void route_kernel(RouteArgs a) {
  // Dynamic LDS (route_lds_bytes): left sums of the block's segments, in the
  // slot of the segment's first position in the block (distinct for
  // distinct non-empty segments; empty segments own no position): s_qn packs
  // the qh sum with the row count (qh_sum * 2^11 + rows: at most kPartBlock
  // < 2^11 rows, |q63 >> 32| <= 2^30 per row), s_ql holds the ql sum.  With
  // a.want_max also the largest |residual| (float bits) of each segment's
  // left and right rows (mode 0: all its rows are "left"), in the same slot:
  // per (node, era) segment, so per node when there is one era.
  extern __shared__ int64_t s_dyn[];
  int64_t* s_qn = s_dyn;
  int64_t* s_ql = s_dyn + kPartBlock;
  uint32_t* s_ml = (uint32_t*)(s_dyn + 2 * kPartBlock);
  uint32_t* s_mr = s_ml + kPartBlock;
  __shared__ int s_wlast[kPartThreads / 64];  // key of each wave's last position
  __shared__ int64_t s_sl;  // start of the block's last segment
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  // Mode 2 (leaf updates only) of several trees takes its blocks in the XCD
  // work order (grid wgbm_xcd_grid(blocks)): each XCD a contiguous range of
  // positions, so a tree's random prediction updates stay in one or two
  // XCDs' L2 instead of pulling the tree's lines into all eight.
  int64_t bx = blockIdx.x;
  if (a.xcd_order) {
    const int64_t nbk = (a.n_pos + kPartBlock - 1) / kPartBlock;
    bx = wgbm_xcd_work(blockIdx.x, nbk);
    if (bx >= nbk) return;  // uniform per workgroup
  }
  const int64_t p0 = bx * kPartBlock;
  const int64_t p1 = p0 + kPartBlock < a.n_pos ? p0 + kPartBlock : a.n_pos;
  const bool sums = a.mode != 2;
  const bool maxes = sums && a.want_max;
  // Thread t owns the PJ consecutive positions pl0 .. pl0 + PJ - 1 of the
  // block (16-byte loads of keys, rows and residuals; rows of one segment
  // are usually combined in registers before the wave reduction).  Issued
  // before the LDS is cleared, so that their latency overlaps it.  A position
  // past the end takes the block's last key (it adds nothing).
  constexpr int PJ = kPartBlock / kPartThreads;
  static_assert(PJ == 4, "four positions per thread");
  typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int pl0 = tid * PJ;
  const int64_t pb = p0 + pl0;
  int key[PJ], slot[PJ], tnv[PJ], lv[PJ];
  int32_t rowv[PJ];
  float rv[PJ];
  bool ok[PJ];
  const bool vec = pb + PJ <= p1 &&
                   (((uintptr_t)a.keyp | (uintptr_t)a.order | (uintptr_t)a.rpos) & 15u) == 0 &&
                   ((uintptr_t)a.dirbit & 3u) == 0;
  if (vec) {
    const i32x4 k4 = *reinterpret_cast<const i32x4*>(a.keyp + pb);
    const i32x4 o4 = *reinterpret_cast<const i32x4*>(a.order + pb);
    f32x4 r4 = {0.0f, 0.0f, 0.0f, 0.0f};
    if (sums) r4 = *reinterpret_cast<const f32x4*>(a.rpos + pb);
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      ok[j] = true;
      key[j] = k4[j];
      rowv[j] = o4[j];
      rv[j] = r4[j];
    }
  } else {
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int64_t p = pb + j;
      ok[j] = p < p1;
      key[j] = a.keyp[ok[j] ? p : p1 - 1];
      rowv[j] = ok[j] ? a.order[p] : 0;
      rv[j] = ok[j] && sums ? a.rpos[p] : 0.0f;
    }
  }
  if (sums) {
    for (int i = tid; i < kPartBlock; i += kPartThreads) {
      s_qn[i] = 0;
      s_ql[i] = 0;
      if (maxes) {
        s_ml[i] = 0u;
        s_mr[i] = 0u;
      }
    }
    if (lane == 63) s_wlast[tid >> 6] = key[PJ - 1];
  }
  wgbm_lds_barrier();  // the LDS words are cleared (the loads stay in flight)
  // Everything a position needs of its segment and node, in one round of
  // independent loads: the segment's bounds and its node's route record.
  // col: -2 the row stays (node absent), -1 leaf update, >= 0 the split's
  // code column.
  bool seg_in[PJ];  // the segment lies inside the block
  int64_t sev[PJ];  // the segment's end
  NodeRoute nr[PJ];
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int64_t sk = a.seg[key[j]], se = a.seg[key[j] + 1];
    sev[j] = se;
    slot[j] = (int)((sk > p0 ? sk : p0) - p0);
    seg_in[j] = sk >= p0 && se <= p1;
    tnv[j] = key[j] / a.E;
    if (sums && pb + j == p1 - 1) s_sl = sk;  // the block's last position: its segment's start
    if (a.mode != 0) nr[j] = a.nroute[tnv[j]];
    lv[j] = (ok[j] && a.mode != 0) ? nr[j].col : -2;
  }
  // Sums go to the LDS slot of the row's segment.  A wave whose rows all lie
  // in one segment (the common case for large segments) reduces them across
  // its lanes first and adds once; otherwise every lane adds its own row.
  auto add_slot = [&](int sl, bool act, int64_t qn, int64_t ql) {
    const uint64_t on = __ballot(act);
    if (on == 0ull) return;
    const int first = __builtin_ctzll(on);  // wave-uniform
    const int s0 = __builtin_amdgcn_readlane(sl, first);
    if (__ballot(act && sl != s0) == 0ull) {
      qn = wgbm_wave_reduce_add_i64(act ? qn : (int64_t)0);
      ql = wgbm_wave_reduce_add_i64(act ? ql : (int64_t)0);
      if (lane == 0) {
        if (qn) atomicAdd((unsigned long long*)&s_qn[s0], (unsigned long long)qn);
        if (ql) atomicAdd((unsigned long long*)&s_ql[s0], (unsigned long long)ql);
      }
    } else if (act) {
      if (qn) atomicAdd((unsigned long long*)&s_qn[sl], (unsigned long long)qn);
      if (ql) atomicAdd((unsigned long long*)&s_ql[sl], (unsigned long long)ql);
    }
  };
  // segment maxima likewise, per segment slot
  auto max_slot = [&](int sl, bool act, uint32_t ml, uint32_t mr) {
    const uint64_t on = __ballot(act);
    if (on == 0ull) return;
    const int first = __builtin_ctzll(on);
    const int s0 = __builtin_amdgcn_readlane(sl, first);
    if (__ballot(act && sl != s0) == 0ull) {
      ml = wgbm_wave_reduce_max_u32(act ? ml : 0u);
      mr = wgbm_wave_reduce_max_u32(act ? mr : 0u);
      if (lane == 0) {
        if (ml) atomicMax(&s_ml[s0], ml);
        if (mr) atomicMax(&s_mr[s0], mr);
      }
    } else if (act) {
      if (ml) atomicMax(&s_ml[sl], ml);
      if (mr) atomicMax(&s_mr[sl], mr);
    }
  };
  // one row's wide quantisation at shift s63, split into (hi word * 2^11 +
  // 1, lo word)
  auto q63_words = [&](float r, int s63, int64_t& qn, int64_t& ql) {
    const int64_t q = (int64_t)rintf(ldexpf(r, s63));
    qn = (q >> 32) * 2048 + 1;
    ql = q & 0xffffffffll;
  };
  // the thread's positions lie in one segment (then also in one node): their
  // sums and maxima are combined here and reduced once per wave, when every
  // thread of the wave can do so
  bool one = true;
#pragma unroll
  for (int j = 1; j < PJ; ++j) one = one && key[j] == key[0];
  const bool wave_one = __ballot(!one) == 0ull;
  uint8_t dirs[PJ];
  int s63v[PJ];  // the wide shift of each position's tree
  if (a.mode == 0) {
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      s63v[j] = a.shifts[tnv[j] / a.nodes] + a.s63_add;
      dirs[j] = ok[j] ? 0 : 2;
    }
  } else {
    int cv[PJ];
#pragma unroll
    for (int j = 0; j < PJ; ++j)
      cv[j] = lv[j] >= 0 ? (int)a.codes_cm[(int64_t)lv[j] * a.n + rowv[j]] : 0;
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int t = tnv[j] / a.nodes;
      uint8_t dir = 2;  // stays in place
      if (lv[j] == -1) {
        // the node is a leaf: add lr * leaf to its rows' predictions
        float* pc = a.pred + (int64_t)t * a.pcol + (int64_t)rowv[j] * a.pstride;
        *pc = *pc + a.lr * nr[j].leaf;
      } else if (lv[j] >= 0) {
        dir = cv[j] > nr[j].bin ? 1 : 0;
      }
      dirs[j] = dir;
      s63v[j] = nr[j].s63;
    }
  }
  if (sums) {
    if (wave_one) {
      int64_t qn = 0, ql = 0;
      bool act = false;
#pragma unroll
      for (int j = 0; j < PJ; ++j) {
        if (dirs[j] == 0) {
          int64_t n1, l1;
          q63_words(rv[j], s63v[j], n1, l1);
          qn += n1;
          ql += l1;
          act = true;
        }
      }
      add_slot(slot[0], act, qn, ql);
    } else {
#pragma unroll
      for (int j = 0; j < PJ; ++j) {
        int64_t n1 = 0, l1 = 0;
        if (dirs[j] == 0) q63_words(rv[j], s63v[j], n1, l1);
        add_slot(slot[j], dirs[j] == 0, n1, l1);
      }
    }
  }
  if (maxes) {
    if (wave_one) {
      uint32_t ml = 0u, mr = 0u;
      bool act = false;
#pragma unroll
      for (int j = 0; j < PJ; ++j) {
        const uint32_t m = wgbm_abs_bits(rv[j]);
        if (dirs[j] == 0) ml = m > ml ? m : ml;
        if (dirs[j] == 1) mr = m > mr ? m : mr;
        act = act || dirs[j] != 2;
      }
      max_slot(slot[0], act, ml, mr);
    } else {
#pragma unroll
      for (int j = 0; j < PJ; ++j) {
        const uint32_t m = wgbm_abs_bits(rv[j]);
        max_slot(slot[j], dirs[j] != 2, dirs[j] == 0 ? m : 0u, dirs[j] == 1 ? m : 0u);
      }
    }
  }
  if (a.mode != 0 && sums) {
    if (vec) {
      const uint32_t w = (uint32_t)dirs[0] | ((uint32_t)dirs[1] << 8) |
                         ((uint32_t)dirs[2] << 16) | ((uint32_t)dirs[3] << 24);
      *reinterpret_cast<uint32_t*>(a.dirbit + pb) = w;  // pb is a multiple of 4
    } else {
#pragma unroll
      for (int j = 0; j < PJ; ++j)
        if (ok[j]) a.dirbit[pb + j] = dirs[j];
    }
  }
  if (!sums) return;  // uniform over the block
  wgbm_lds_barrier();  // the block's sums are in LDS (the stores above need not land)
  // decode a slot's packed word: rows in the low 11 bits, the hi sum above
  auto unpack = [](int64_t qn, int64_t& qh, int32_t& n) {
    n = (int32_t)(qn & 2047);
    qh = qn >> 11;
  };
  // the key of the position before the thread's first: the previous lane's
  // last (lane 0: the previous wave's last; the block's first position has
  // none)
  int prev = __shfl_up(key[PJ - 1], 1, 64);
  if (lane == 0) prev = tid > 0 ? s_wlast[(tid >> 6) - 1] : -1;
  if (a.kw.cnt) {
    // the segments' words (split segments only): stored by the thread of a
    // segment's first position in the block when it lies inside the block;
    // a segment crossing the block's edges (the block's first or last) adds
    // its part with atomics and reserves its rows' place in the children
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int i = pl0 + j;
      const int k = key[j];
      const int kp = j == 0 ? prev : key[j - 1];
      if (!ok[j] || (i > 0 && kp == k) || lv[j] < 0) continue;
      int64_t qh;
      int32_t n;
      unpack(s_qn[i], qh, n);
      const int64_t e_loc = (sev[j] < p1 ? sev[j] : p1) - p0;
      const int32_t nrt = (int32_t)(e_loc - i) - n;
      const unsigned long long packed =
          ((unsigned long long)(uint32_t)n << 32) | (uint32_t)nrt;
      if (seg_in[j]) {
        a.kw.cnt[k] = packed;
        a.kw.qh[k] = qh;
        a.kw.ql[k] = s_ql[i];
        if (maxes) {
          a.kw.ml[k] = s_ml[i];
          a.kw.mr[k] = s_mr[i];
        }
      } else {
        a.res[2 * (int64_t)blockIdx.x + (i == 0 ? 0 : 1)] = atomicAdd(a.kw.cnt + k, packed);
        const int64_t ql = s_ql[i];
        if (qh) atomicAdd((unsigned long long*)(a.kw.qh + k), (unsigned long long)qh);
        if (ql) atomicAdd((unsigned long long*)(a.kw.ql + k), (unsigned long long)ql);
        if (maxes) {
          if (s_ml[i]) atomicMax(a.kw.ml + k, s_ml[i]);
          if (s_mr[i]) atomicMax(a.kw.mr + k, s_mr[i]);
        }
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    // position pl0 + j opens a segment when its key differs from the one
    // before it (the block's first position always does)
    const int i = pl0 + j;
    const int k = key[j];
    const int kp = j == 0 ? prev : key[j - 1];
    if (!ok[j] || (i > 0 && kp == k)) continue;
    if (seg_in[j]) {
      // a segment inside the block: its sums (and maxima) are complete here
      int64_t qh;
      int32_t n;
      unpack(s_qn[i], qh, n);
      a.ps.own_qh[k] = qh;
      a.ps.own_ql[k] = s_ql[i];
      a.ps.own_n[k] = n;
      if (maxes) {
        a.ps.own_ml[k] = s_ml[i];
        a.ps.own_mr[k] = s_mr[i];
      }
    }
  }
  if (tid == 0) {
    // the first and last segments of the block: their sums here
    const int64_t sl = s_sl;
    const int ls = (int)((sl > p0 ? sl : p0) - p0);
    int64_t qh;
    int32_t n;
    unpack(s_qn[0], qh, n);
    a.ps.bf_qh[blockIdx.x] = qh;
    a.ps.bf_ql[blockIdx.x] = s_ql[0];
    a.ps.bf_n[blockIdx.x] = n;
    unpack(s_qn[ls], qh, n);
    a.ps.bl_qh[blockIdx.x] = qh;
    a.ps.bl_ql[blockIdx.x] = s_ql[ls];
    a.ps.bl_n[blockIdx.x] = n;
    if (maxes) {
      // the first and last segments of the block: their maxima here
      a.ps.bf_node[blockIdx.x] = key[0];  // thread 0 holds the block's first position
      a.ps.bf_ml[blockIdx.x] = s_ml[0];
      a.ps.bf_mr[blockIdx.x] = s_mr[0];
      a.ps.bl_ml[blockIdx.x] = s_ml[ls];
      a.ps.bl_mr[blockIdx.x] = s_mr[ls];
    }
  }
}

// LDS copies of the block prefixes (level_scan_e1_kernel, at most
// kScanLdsBlocks blocks)
constexpr int kScanLdsBlocks = 2048;
struct ScanLds {
  int64_t* qh;
  int64_t* ql;
  int64_t* n;
  uint32_t* ml;
  uint32_t* mr;
};

// inclusive prefix over the blocks of the first-segment partials; one
// workgroup of 1024 threads, tiles of 1024 blocks.  The words of the first
// two tiles are loaded before pre() runs (work of the caller that does not
// need the prefixes), later tiles one tile ahead.  Wave totals are scanned
// with DPP over lanes 0..15 and double-buffered by tile parity (one barrier
// per tile); the carries between tiles stay in registers.  With seg_max
// also the segmented inclusive maxima of the first nodes' child maxima:
// pm_l[b] = max of bf_ml over the run of consecutive blocks, ending at b,
// whose first node is bf_node[b] (every such block starts inside that
// node).  With to_lds the prefixes are also left in LDS (nb <=
// kScanLdsBlocks).
struct NoPre {
  __device__ void operator()() const {}
};
template <typename Pre = NoPre>
__device__ inline void block_scan_body(int32_t nb, const PartSums& ps, bool seg_max = false,
                                       bool to_lds = false, ScanLds lds = ScanLds{},
                                       Pre pre = Pre{}) {
  __shared__ int64_t s_wh[2][16], s_wl[2][16], s_wn[2][16];
  __shared__ uint32_t s_mf[2][16], s_ml[2][16], s_mr[2][16];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  // one block's words (blocks past the end: zero, and a run opens there).
  // Loads only: the run test compares the first nodes when the words are
  // used, so that the loads of both tiles are in flight together.
  struct Words {
    int64_t qh, ql;
    int32_t n;  // widened where used (a conversion here would wait for the load)
    uint32_t vl, vr;
    int32_t nd, ndp;  // first node of the block and of the block before
  };
  auto load = [&](int b) {
    Words x{0, 0, 0, 0u, 0u, -1, -2};
    if (b < nb) {
      x.qh = ps.bf_qh[b];
      x.ql = ps.bf_ql[b];
      x.n = ps.bf_n[b];
      if (seg_max) {
        x.vl = ps.bf_ml[b];
        x.vr = ps.bf_mr[b];
        x.nd = ps.bf_node[b];
        x.ndp = b > 0 ? ps.bf_node[b - 1] : -2;
      }
    }
    return x;
  };
  Words nxt = load(t), nxt2 = load(t + 1024);
  pre();
  int64_t ch = 0, cl = 0, cn = 0;  // prefix before the tile (workgroup-uniform)
  uint32_t cml = 0u, cmr = 0u;     // maxima of the run open before the tile
  int par = 0;
  for (int b0 = 0; b0 < nb; b0 += 1024, par ^= 1) {
    const int b = b0 + t;
    const Words cur = nxt;
    nxt = nxt2;
    if (b0 + 2048 < nb) nxt2 = load(b + 2048);
    int64_t qh = wgbm_wave_incl_scan_i64(cur.qh);
    int64_t ql = wgbm_wave_incl_scan_i64(cur.ql);
    int64_t n = wgbm_wave_incl_scan_i64((int64_t)cur.n);
    uint32_t f = cur.nd != cur.ndp ? 1u : 0u, vl = cur.vl, vr = cur.vr;
    if (seg_max) wgbm_wave_segmax_scan(f, vl, vr);
    if (lane == 63) {
      s_wh[par][w] = qh;
      s_wl[par][w] = ql;
      s_wn[par][w] = n;
      s_mf[par][w] = f;
      s_ml[par][w] = vl;
      s_mr[par][w] = vr;
    }
    wgbm_lds_barrier();  // the wave totals are read from LDS only
    // the wave totals scanned over lanes 0..15: lane w - 1 holds waves 0..w-1
    const int src = w > 0 ? w - 1 : 0;
    const int64_t gh = wgbm_row_incl_scan_i64(lane < 16 ? s_wh[par][lane] : 0);
    const int64_t gl = wgbm_row_incl_scan_i64(lane < 16 ? s_wl[par][lane] : 0);
    const int64_t gn = wgbm_row_incl_scan_i64(lane < 16 ? s_wn[par][lane] : 0);
    if (w > 0) {
      qh += wgbm_readlane_i64(gh, src);
      ql += wgbm_readlane_i64(gl, src);
      n += wgbm_readlane_i64(gn, src);
    }
    qh += ch;
    ql += cl;
    n += cn;
    if (b < nb) {
      ps.P_qh[b] = qh;
      ps.P_ql[b] = ql;
      ps.P_n[b] = n;
      if (to_lds) {
        lds.qh[b] = qh;
        lds.ql[b] = ql;
        lds.n[b] = n;
      }
    }
    ch += wgbm_readlane_i64(gh, 15);
    cl += wgbm_readlane_i64(gl, 15);
    cn += wgbm_readlane_i64(gn, 15);
    if (seg_max) {
      uint32_t mf = lane < 16 ? s_mf[par][lane] : 0u;
      uint32_t ma = lane < 16 ? s_ml[par][lane] : 0u;
      uint32_t mb = lane < 16 ? s_mr[par][lane] : 0u;
      wgbm_row_segmax_scan(mf, ma, mb);
      // the open run's maxima before this wave: the tile carry, then waves
      // 0..w-1 (a run opening among them restarts it)
      uint32_t pl = cml, pr = cmr;
      if (w > 0) {
        const uint32_t F = (uint32_t)__builtin_amdgcn_readlane((int)mf, src);
        const uint32_t A = (uint32_t)__builtin_amdgcn_readlane((int)ma, src);
        const uint32_t B = (uint32_t)__builtin_amdgcn_readlane((int)mb, src);
        pl = F ? A : (A > pl ? A : pl);
        pr = F ? B : (B > pr ? B : pr);
      }
      if (!f) {
        vl = pl > vl ? pl : vl;
        vr = pr > vr ? pr : vr;
      }
      if (b < nb) {
        ps.pm_l[b] = vl;
        ps.pm_r[b] = vr;
        if (to_lds) {
          lds.ml[b] = vl;
          lds.mr[b] = vr;
        }
      }
      const uint32_t F = (uint32_t)__builtin_amdgcn_readlane((int)mf, 15);
      const uint32_t A = (uint32_t)__builtin_amdgcn_readlane((int)ma, 15);
      const uint32_t B = (uint32_t)__builtin_amdgcn_readlane((int)mb, 15);
      cml = F ? A : (A > cml ? A : cml);
      cmr = F ? B : (B > cmr ? B : cmr);
    }
  }
  if (to_lds) wgbm_lds_barrier();  // the LDS prefixes are read by other threads
}

__global__ __launch_bounds__(1024) void block_scan_kernel(int32_t nb, PartSums ps) {
  block_scan_body(nb, ps);
}

// root totals of every (tree, era) key: quantised residual sum and rows;
// with key_shift (several eras) also the key's histogram shift from its
// largest |residual| (the root route ran with want_max)
__global__ void root_totals_kernel(int32_t n_keys, const int64_t* __restrict__ seg, PartSums ps,
                                   int64_t* __restrict__ tot_qh, int64_t* __restrict__ tot_ql,
                                   int64_t* __restrict__ tot_c, int32_t qbits,
                                   int32_t* __restrict__ key_shift) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= n_keys) return;
  int64_t qh, ql, n;
  segment_left_sums(k, seg, ps, qh, ql, n);
  tot_qh[k] = qh;
  tot_ql[k] = ql;
  tot_c[k] = n;
  if (key_shift) {
    uint32_t m = 0, unused = 0;
    seg_child_max(k, seg[k], seg[k + 1], ps, 0, 1, m, unused);
    key_shift[k] = key_shift_of(m, qbits);
  }
}

// Several eras: the histogram shifts of one split's two children's segments
// of an era (keys kl, kr of the next level; k the parent's segment), each from
// its own largest |residual| (key_shift_of), and whether both are
// histogrammed: the sibling's segment is parent - child only when the
// parent's and both children's shifts are equal (the subtraction is then
// exact).  A node that does not split has no children: their words are 0.
__device__ inline void era_child_shifts(int64_t k, int64_t kl, int64_t kr, bool sp,
                                        const PartSums& ps, const int64_t* __restrict__ seg,
                                        const LevelNext& nx, const KeyWords& kw, bool& both) {
  int sl = 0, sr = 0;
  both = false;
  if (sp && nx.have_max) {
    uint32_t ml = 0, mr = 0;
    if (kw.cnt) {
      ml = kw.ml[k];
      mr = kw.mr[k];
    } else {
      seg_child_max(k, seg[k], seg[k + 1], ps, 0, 1, ml, mr);
    }
    sl = key_shift_of(ml, nx.qbits);
    sr = key_shift_of(mr, nx.qbits);
    const int sp_k = nx.node_shift[k];
    both = sl != sp_k || sr != sp_k;
  }
  nx.node_shift_next[kl] = sl;
  nx.node_shift_next[kr] = sr;
}

// wpn waves per (tree, node) of the level (1, 2 or 4: the eras are spread
// over the group's lanes); 4 / wpn nodes per workgroup
__global__ __launch_bounds__(256) void node_scan_kernel(
    int32_t T, int32_t nodes, int32_t E, int32_t wpn, int64_t n_pos,
    const int64_t* __restrict__ seg, const int32_t* __restrict__ present,
    const int32_t* __restrict__ split_l, PartSums ps, LevelNext nx, KeyWords kw) {
  const bool kwm = kw.cnt != nullptr;  // uniform: the segments' words are in kw
  __shared__ int64_t s_a[4], s_b[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = wave / wpn, wg = wave - grp * wpn;
  const int tn = blockIdx.x * (4 / wpn) + grp;
  const int gthreads = wpn * 64, gt = wg * 64 + lane;
  // a group past the last node still takes part in the workgroup barriers
  const bool live = tn < T * nodes;
  const bool sp = live && present[tn] && split_l[tn] >= 0;
  const int64_t k0 = (int64_t)tn * E;
  const int64_t base = live ? seg[k0] : 0;
  const int64_t c0 = 2 * k0;  // next keys of the children: c0 + side * E + e
  // left rows of a segment of the node (all of them when it does not split)
  auto left_of = [&](int64_t k, int64_t cnt, int64_t& qh, int64_t& ql) -> int64_t {
    int64_t L = cnt;
    qh = 0;
    ql = 0;
    if (sp && kwm) {
      if (cnt > 0) {
        L = (int64_t)(kw.cnt[k] >> 32);
        qh = kw.qh[k];
        ql = kw.ql[k];
      }
    } else if (sp) {
      segment_left_sums(k, seg, ps, qh, ql, L);
    }
    return L;
  };
  // sum (or max) over the group of one value per wave (every thread gets it)
  auto group_sum = [&](int64_t a, int64_t b, int64_t& ga, int64_t& gb, bool is_max) {
    if (lane == 63) {
      s_a[wave] = a;
      s_b[wave] = b;
    }
    wgbm_lds_barrier();
    ga = 0;
    gb = 0;
    for (int w = grp * wpn; w < (grp + 1) * wpn; ++w) {
      if (is_max) {
        ga = s_a[w] > ga ? s_a[w] : ga;
        gb = s_b[w] > gb ? s_b[w] : gb;
      } else {
        ga += s_a[w];
        gb += s_b[w];
      }
    }
    wgbm_lds_barrier();
  };
  int64_t ltot = 0, tot = 0;
  // With at most NE eras per thread (C4: 500 eras over 256 lanes) the
  // thread's era words are loaded once, in one round per kind of word, and
  // kept for the prefix loop below; else they are loaded in each loop.
  constexpr int NE = 4;
  const bool keep = E <= NE * gthreads;  // uniform
  int64_t eL[NE], eR[NE], eQh[NE], eQl[NE];
  if (live && keep) {
    int64_t s0[NE], s1[NE];
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int e = gt + i * gthreads;
      const int ec = e < E ? e : E - 1;
      s0[i] = seg[k0 + ec];
      s1[i] = seg[k0 + ec + 1];
    }
    // both kinds of left sums of every kept era, loaded in one round
    // (segment_left_sums_at picks one: a segment inside one block has its
    // own words, else its first block's and the block prefix), block
    // indices clamped so that the unused kind stays in bounds
    const int64_t bmax = n_pos > 0 ? (n_pos - 1) / kPartBlock : 0;
    int64_t oq[NE], ol[NE], bq[NE], bl[NE], pq1[NE], pl1[NE], pq0[NE], pl0[NE];
    int32_t on[NE], bn[NE];
    int64_t pn1[NE], pn0[NE];
    if (kwm) {
      // the route's words of each kept era: whole sums, no block prefix
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        const int e = gt + i * gthreads;
        const int64_t k = k0 + (e < E ? e : E - 1);
        const unsigned long long c = kw.cnt[k];
        oq[i] = kw.qh[k];
        ol[i] = kw.ql[k];
        on[i] = (int32_t)(c >> 32);
      }
    }
    if (!kwm) {
#pragma unroll
      for (int i = 0; i < NE; ++i) {
        const int e = gt + i * gthreads;
        const int64_t k = k0 + (e < E ? e : E - 1);
        const int64_t b0 = s0[i] / kPartBlock < bmax ? s0[i] / kPartBlock : bmax;
        const int64_t b1 = s1[i] > s0[i] ? (s1[i] - 1) / kPartBlock : b0;
        oq[i] = ps.own_qh[k];
        ol[i] = ps.own_ql[k];
        on[i] = ps.own_n[k];
        bq[i] = ps.bl_qh[b0];
        bl[i] = ps.bl_ql[b0];
        bn[i] = ps.bl_n[b0];
        pq1[i] = ps.P_qh[b1];
        pl1[i] = ps.P_ql[b1];
        pn1[i] = ps.P_n[b1];
        pq0[i] = ps.P_qh[b0];
        pl0[i] = ps.P_ql[b0];
        pn0[i] = ps.P_n[b0];
      }
    }
#pragma unroll
    for (int i = 0; i < NE; ++i) {
      const int e = gt + i * gthreads;
      const int64_t cnt = e < E ? s1[i] - s0[i] : 0;
      int64_t L = cnt, qh = 0, ql = 0;
      if (sp) {
        if (cnt <= 0) {
          L = 0;
        } else if (kwm || s0[i] / kPartBlock == (s1[i] - 1) / kPartBlock) {
          qh = oq[i];
          ql = ol[i];
          L = on[i];
        } else {
          qh = bq[i] + pq1[i] - pq0[i];
          ql = bl[i] + pl1[i] - pl0[i];
          L = bn[i] + pn1[i] - pn0[i];
        }
      }
      eQh[i] = qh;
      eQl[i] = ql;
      eL[i] = L;
      eR[i] = cnt - L;
      ltot += L;
      tot += cnt;
    }
  } else if (live) {
    for (int e = gt; e < E; e += gthreads) {
      const int64_t cnt = seg[k0 + e + 1] - seg[k0 + e];
      int64_t qh, ql;
      ltot += left_of(k0 + e, cnt, qh, ql);
      tot += cnt;
    }
  }
  ltot = wgbm_wave_incl_scan_i64(ltot);  // inclusive wave scans: lane 63 holds the sums
  tot = wgbm_wave_incl_scan_i64(tot);
  group_sum(ltot, tot, ltot, tot, false);
  const int side = (ltot <= tot - ltot) ? 0 : 1;  // the smaller child gets the histogram
  // One era: the children's histogram shifts from their largest |residual|
  // (node_shift_rule).  Several eras: per (child, era) segment, below.
  int hs = 0, hs_l = 0, hs_r = 0;
  bool both = false;  // both children histogrammed
  if (E == 1) {
    uint32_t ml = 0, mr = 0;
    if (sp && nx.have_max) seg_child_max(tn, base, seg[k0 + E], ps, gt, gthreads, ml, mr);
    ml = wgbm_wave_reduce_max_u32(ml);
    mr = wgbm_wave_reduce_max_u32(mr);
    {
      int64_t gml, gmr;
      group_sum((int64_t)ml, (int64_t)mr, gml, gmr, true);
      ml = (uint32_t)gml;
      mr = (uint32_t)gmr;
    }
    hs = live ? nx.node_shift[tn] : 0;
    hs_l = sp && nx.have_max ? node_shift_rule(ml, hs, nx.qbits) : hs;
    hs_r = sp && nx.have_max ? node_shift_rule(mr, hs, nx.qbits) : hs;
    both = sp && (hs_l != hs || hs_r != hs);
  }
  int64_t carry_l = 0, carry_r = 0;
  for (int e0 = 0, i = 0; e0 < E; e0 += gthreads, ++i) {
    const int e = e0 + gt;
    int64_t L = 0, R = 0, qh = 0, ql = 0;
    if (keep) {
      // the kept words of round i (a fixed-index select: no indexed
      // register access)
#pragma unroll
      for (int j = 0; j < NE; ++j) {
        if (j == i && live) {
          L = eL[j];
          R = eR[j];
          qh = eQh[j];
          ql = eQl[j];
        }
      }
    } else if (live && e < E) {
      const int64_t cnt = seg[k0 + e + 1] - seg[k0 + e];
      L = left_of(k0 + e, cnt, qh, ql);
      R = cnt - L;
    }
    int64_t il = wgbm_wave_incl_scan_i64(L), ir = wgbm_wave_incl_scan_i64(R);
    // earlier waves of the group, and the chunk totals for the carry
    if (lane == 63) {
      s_a[wave] = il;
      s_b[wave] = ir;
    }
    wgbm_lds_barrier();
    int64_t pl = 0, pr = 0, cl = 0, cr = 0;
    for (int w = grp * wpn; w < (grp + 1) * wpn; ++w) {
      if (w < wave) {
        pl += s_a[w];
        pr += s_b[w];
      }
      cl += s_a[w];
      cr += s_b[w];
    }
    wgbm_lds_barrier();
    il += pl;
    ir += pr;
    if (nx.alive_next) {
      // the children's live eras (des_alive_kernel's bits: a segment of at
      // least 2 * mcw rows), one ballot per child and wave: the wave's 64
      // eras are two mask words
      const bool in = live && e < E;
      const uint64_t bl = __ballot(in && !des_segment_dead(L, nx.mcw));
      const uint64_t br = __ballot(in && !des_segment_dead(R, nx.mcw));
      static_assert(kDesEraBlock == 32, "a wave's 64 eras are two mask words");
      const int W = (E + kDesEraBlock - 1) / kDesEraBlock;
      const int w0 = (e0 + wg * 64) / kDesEraBlock;
      if (live && lane == 0 && w0 < W) {
        uint32_t* al = nx.alive_next + (int64_t)(2 * tn) * W;
        uint32_t* ar = al + W;
        al[w0] = (uint32_t)bl;
        ar[w0] = (uint32_t)br;
        if (w0 + 1 < W) {
          al[w0 + 1] = (uint32_t)(bl >> 32);
          ar[w0 + 1] = (uint32_t)(br >> 32);
        }
      }
    }
    if (live && e < E) {
      nx.seg_next[c0 + e] = base + carry_l + il - L;
      nx.seg_next[c0 + E + e] = base + ltot + carry_r + ir - R;
      // child totals (the words of children that do not exist are zero)
      nx.tot_qh_next[c0 + e] = sp ? qh : 0;
      nx.tot_ql_next[c0 + e] = sp ? ql : 0;
      nx.tot_c_next[c0 + e] = sp ? L : 0;
      nx.tot_qh_next[c0 + E + e] = sp ? nx.tot_qh[k0 + e] - qh : 0;
      nx.tot_ql_next[c0 + E + e] = sp ? nx.tot_ql[k0 + e] - ql : 0;
      nx.tot_c_next[c0 + E + e] = sp ? R : 0;
      bool both_e = both;
      if (E > 1) era_child_shifts(k0 + e, c0 + e, c0 + E + e, sp, ps, seg, nx, kw, both_e);
      if (kwm) {
        // read: ready for the next level
        kw.cnt[k0 + e] = 0ull;
        kw.qh[k0 + e] = 0;
        kw.ql[k0 + e] = 0;
        kw.ml[k0 + e] = 0u;
        kw.mr[k0 + e] = 0u;
      }
      nx.key_list_next[2 * (k0 + e)] =
          sp ? (int32_t)(c0 + (both_e ? 0 : side * E) + e) : -1;
      nx.key_list_next[2 * (k0 + e) + 1] = both_e ? (int32_t)(c0 + E + e) : -1;
    }
    carry_l += cl;
    carry_r += cr;
  }
  if (live && gt < 2) {
    nx.present_next[2 * tn + gt] = sp;
    if (E == 1) nx.node_shift_next[2 * tn + gt] = gt == 0 ? hs_l : hs_r;
  }
  if (tn == T * nodes - 1 && gt == 0) nx.seg_next[(int64_t)2 * T * nodes * E] = n_pos;
}

__global__ __launch_bounds__(kPartThreads) void scatter_kernel(
    int64_t n_pos, int32_t E, const int64_t* __restrict__ seg,
    const int64_t* __restrict__ seg_next, const int32_t* __restrict__ keyp,
    const uint8_t* __restrict__ dirbit, PartSums ps, const int32_t* __restrict__ order,
    int32_t* __restrict__ order_next, int32_t* __restrict__ keyp_next,
    const float* __restrict__ rpos, float* __restrict__ rpos_next,
    const unsigned long long* __restrict__ res) {
  constexpr int PJ = kPartBlock / kPartThreads;  // positions per thread (strided)
  constexpr int NW = kPartThreads / 64;
  __shared__ int32_t s_pl[kPartBlock];  // left rows before each block position
  __shared__ int32_t s_c[PJ * NW];      // left rows of each (phase, wave) group
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t p0 = (int64_t)blockIdx.x * kPartBlock;
  uint8_t d[PJ];
  int32_t rowv[PJ], key[PJ], rank[PJ];
  float rr[PJ];
  bool ok[PJ];
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int64_t p = p0 + j * kPartThreads + tid;
    ok[j] = p < n_pos;
    d[j] = ok[j] ? dirbit[p] : 2;
    rowv[j] = ok[j] ? order[p] : 0;
    key[j] = ok[j] ? keyp[p] : 0;
    rr[j] = ok[j] ? rpos[p] : 0.0f;
  }
  // Every global word the positions need is loaded here, ahead of the LDS
  // rank work: the segment bounds and child starts of each position's key,
  // and the left rows of the block's first segment in earlier blocks.
  // Kept in 32 bits relative to the block and the segment: a segment and
  // the node around it hold fewer than 2^31 positions.
  const int kf = keyp[p0];
  const int64_t p1 = p0 + kPartBlock < n_pos ? p0 + kPartBlock : n_pos;
  int32_t sk[PJ], nd[PJ];  // segment start - p0; row's child segment start - segment start
  bool past[PJ];           // (with res) the segment ends past the block
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int k = key[j];
    const int tn = k / E;
    const int64_t kl = (int64_t)2 * tn * E + (k - (int64_t)tn * E);  // left child's key
    const int64_t s_k = seg[k];
    sk[j] = (int32_t)(s_k - p0);
    nd[j] = (int32_t)(seg_next[d[j] == 1 ? kl + E : kl] - s_k);
    past[j] = res ? seg[k + 1] > p1 : false;
  }
  // the block prefix words (without res)
  const int64_t sf = seg[kf];
  const int64_t b0 = (sf < p0 ? sf : p0) / kPartBlock;
  const int64_t bl0 = res ? 0 : ps.bl_n[b0];
  const int64_t pb0 = res ? 0 : ps.P_n[b0];
  const int64_t pprev = !res && blockIdx.x > 0 ? ps.P_n[blockIdx.x - 1] : 0;
  // the route's reserved bases of the block's first and last segments
  const unsigned long long rb0 = res ? res[2 * (int64_t)blockIdx.x] : 0ull;
  const unsigned long long rb1 = res ? res[2 * (int64_t)blockIdx.x + 1] : 0ull;
  // left rows before each position: rank among the wave's lefts plus the
  // lefts of the (phase, wave) groups before it (position order is phase,
  // then wave, then lane)
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const uint64_t m = __ballot(d[j] == 0);
    rank[j] = (int32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    if (lane == 0) s_c[j * NW + w] = __builtin_popcountll(m);
  }
  wgbm_lds_barrier();
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    int pre = 0;
    for (int i = 0; i < j * NW + w; ++i) pre += s_c[i];
    rank[j] += pre;
    s_pl[j * kPartThreads + tid] = rank[j];
  }
  wgbm_lds_barrier();
  // left rows of the block's first segment in earlier blocks
  const int64_t cin = sf < p0 ? bl0 + pprev - pb0 : 0;
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int64_t p = p0 + j * kPartThreads + tid;
    if (!ok[j]) break;
    const int k = key[j];
    const int tn = k / E;
    const int64_t kl = (int64_t)2 * tn * E + (k - (int64_t)tn * E);  // left child's key
    if (d[j] == 2) {
      // a node that does not split: its rows stay, in its left child's segment
      order_next[p] = rowv[j];
      keyp_next[p] = (int32_t)kl;
      rpos_next[p] = rr[j];
      continue;
    }
    const int64_t skj = p0 + sk[j];
    const int s0 = sk[j] > 0 ? sk[j] : 0;  // the segment's first position in the block
    if (res) {
      // ranks in the block's part of the segment, after the part of the
      // blocks that reserved before it (a segment inside the block: none)
      const bool cross = sk[j] < 0 || past[j];
      const unsigned long long base = cross ? (s0 == 0 ? rb0 : rb1) : 0ull;
      const int64_t rlb = (int64_t)rank[j] - s_pl[s0];
      const int64_t csr = skj + nd[j];
      const int64_t dst = d[j] == 0 ? csr + (int64_t)(base >> 32) + rlb
                                    : csr + (int64_t)(base & 0xffffffffull) +
                                          ((p - (p0 + s0)) - rlb);
      order_next[dst] = rowv[j];
      keyp_next[dst] = (int32_t)(d[j] == 0 ? kl : kl + E);
      rpos_next[dst] = rr[j];
      continue;
    }
    const int64_t rl = (int64_t)rank[j] - s_pl[s0] + (sk[j] < 0 ? cin : 0);
    const int64_t cs = skj + nd[j];
    const int64_t dst = d[j] == 0 ? cs + rl : cs + ((p - skj) - rl);
    order_next[dst] = rowv[j];
    keyp_next[dst] = (int32_t)(d[j] == 0 ? kl : kl + E);
    rpos_next[dst] = rr[j];
  }
}

// One-era split level in one pass (E == 1, mode 1, at most
// kPartition1MaxNodes (tree, node)s): every position of a block of 4 NT
// positions (NT threads) is routed (route_kernel's directions, leaf updates, left sums
// and maxima) and placed in the next level's arrays at once.  Its node's
// left rows fill the left child's range from the node's first position
// upwards, its right rows the right child's range from the node's last
// position downwards, so the children's bounds need not be known when a row
// is placed.  A node inside the block takes the block's ranks directly and
// stores its words (kw) plainly; a node that crosses the block's edges --
// only the block's first and last nodes can -- reserves the block's part of
// both ranges with one atomic add on its packed row counts (left * 2^32 +
// right) and adds its sums and maxima with relaxed atomics.  Every sum is
// an exact integer and rows inside a node have no order that any result
// depends on, so the order in which blocks reserve changes no output;
// level_scan_e1_kernel then reads the whole words (and clears them).
// Positions are strided over the threads (position j * NT + tid of the
// block), so that the rows of one child taken by one store
// instruction land on consecutive addresses.  The block's nodes are
// consecutive keys from its first position's key kf: node k's LDS slot is
// k - kf (< n_slots = the level's (tree, node)s).
//
// With leaf_key (the last split level) no position is placed: the next level
// only updates predictions, so each row's child key is written by row
// instead, leaf_key[tree * n + row] (leaf_rows_kernel then reads it in row
// order).
template <int NT>
__global__ __launch_bounds__(NT) void partition_e1_kernel(RouteArgs a, KeyWords kw,
                                                          int32_t n_slots,
                                                          int32_t* __restrict__ order_next,
                                                          int32_t* __restrict__ keyp_next,
                                                          float* __restrict__ rpos_next,
                                                          int32_t* __restrict__ leaf_key) {
  constexpr int PJ = 4;              // positions per thread
  constexpr int PB = PJ * NT;        // positions per block
  constexpr int NW = NT / 64;
  constexpr int kCountBits = 13;     // row counts packed below the hi sums
  static_assert(PB < (1 << kCountBits), "block rows fit the count field");
  // per slot: the left rows' (q63 >> 32) sum * 2^13 + their count (at most
  // PB < 2^13 rows, |q63 >> 32| <= 2^30 per row), the (q63 mod 2^32)
  // sum, both children's max|r|, and the block's lefts before the node's
  // first position (partition1_lds_bytes)
  extern __shared__ int64_t s_dyn[];
  int64_t* s_qn = s_dyn;
  int64_t* s_ql = s_dyn + n_slots;
  uint32_t* s_ml = (uint32_t*)(s_dyn + 2 * n_slots);
  uint32_t* s_mr = s_ml + n_slots;
  int32_t* s_lb = (int32_t*)(s_mr + n_slots);
  __shared__ int32_t s_c[PJ * NW];          // left positions of each (phase, wave) group
  __shared__ unsigned long long s_base[2];  // reserved bases of the first / last node
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t p0 = (int64_t)blockIdx.x * PB;
  const int64_t p1 = p0 + PB < a.n_pos ? p0 + PB : a.n_pos;
  const bool maxes = a.want_max != 0;
  const int kf = a.keyp[p0];
  int key[PJ];
  int32_t rowv[PJ];
  float rv[PJ];
  bool ok[PJ];
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int64_t p = p0 + j * NT + tid;
    ok[j] = p < p1;
    key[j] = a.keyp[ok[j] ? p : p1 - 1];
    rowv[j] = ok[j] ? a.order[p] : 0;
    rv[j] = ok[j] ? a.rpos[p] : 0.0f;
  }
  // the node's bounds and route record (one round of independent loads)
  int64_t sk[PJ], se[PJ];
  NodeRoute nr[PJ];
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    sk[j] = a.seg[key[j]];
    se[j] = a.seg[key[j] + 1];
    nr[j] = a.nroute[key[j]];
  }
  int cv[PJ];
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int col = ok[j] ? nr[j].col : -2;
    cv[j] = col >= 0 ? (int)a.codes_cm[(int64_t)col * a.n + rowv[j]] : 0;
  }
  uint8_t dirs[PJ];  // 0 left, 1 right, 2 stays (the node does not split)
  bool opens[PJ];    // the node's first position in the block
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int col = ok[j] ? nr[j].col : -2;
    uint8_t dir = 2;
    if (col == -1) {
      // the node is a leaf: add lr * leaf to its rows' predictions
      const int t = key[j] / a.nodes;
      float* pc = a.pred + (int64_t)t * a.pcol + (int64_t)rowv[j] * a.pstride;
      *pc = *pc + a.lr * nr[j].leaf;
    } else if (col >= 0) {
      dir = cv[j] > nr[j].bin ? 1 : 0;
    }
    dirs[j] = dir;
    const int64_t first = sk[j] > p0 ? sk[j] : p0;
    opens[j] = ok[j] && dir != 2 && first - p0 == j * NT + tid;
    if (opens[j]) {
      const int sl = key[j] - kf;
      s_qn[sl] = 0;
      s_ql[sl] = 0;
      s_ml[sl] = 0u;
      s_mr[sl] = 0u;
    }
  }
  // left positions before each one: rank among the wave's lefts plus the
  // lefts of the (phase, wave) groups before it
  int32_t rank[PJ];
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const uint64_t m = __ballot(dirs[j] == 0);
    rank[j] = (int32_t)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                                 __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
    if (lane == 0) s_c[j * NW + w] = __builtin_popcountll(m);
  }
  wgbm_lds_barrier();  // group counts and cleared slots
  // sums and maxima per node slot (a wave whose active lanes share a slot
  // reduces first and adds once)
  auto add_slot = [&](int sl, bool act, int64_t qn, int64_t ql, uint32_t ml, uint32_t mr) {
    const uint64_t on = __ballot(act);
    if (on == 0ull) return;
    const int s0 = __builtin_amdgcn_readlane(sl, __builtin_ctzll(on));
    if (__ballot(act && sl != s0) == 0ull) {
      qn = wgbm_wave_reduce_add_i64(act ? qn : (int64_t)0);
      ql = wgbm_wave_reduce_add_i64(act ? ql : (int64_t)0);
      if (maxes) {
        ml = wgbm_wave_reduce_max_u32(act ? ml : 0u);
        mr = wgbm_wave_reduce_max_u32(act ? mr : 0u);
      }
      if (lane == 0) {
        if (qn) atomicAdd((unsigned long long*)&s_qn[s0], (unsigned long long)qn);
        if (ql) atomicAdd((unsigned long long*)&s_ql[s0], (unsigned long long)ql);
        if (ml) atomicMax(&s_ml[s0], ml);
        if (mr) atomicMax(&s_mr[s0], mr);
      }
    } else if (act) {
      if (qn) atomicAdd((unsigned long long*)&s_qn[sl], (unsigned long long)qn);
      if (ql) atomicAdd((unsigned long long*)&s_ql[sl], (unsigned long long)ql);
      if (ml) atomicMax(&s_ml[sl], ml);
      if (mr) atomicMax(&s_mr[sl], mr);
    }
  };
  // the groups' exclusive prefix, scanned by every wave over lanes 0 ..
  // PJ * NW - 1 (at most 64 groups)
  static_assert(PJ * NW <= 64, "one lane per (phase, wave) group");
  const int64_t gcount = lane < PJ * NW ? s_c[lane] : 0;
  const int64_t gexcl = wgbm_wave_incl_scan_i64(gcount) - gcount;
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    rank[j] += (int32_t)wgbm_readlane_i64(gexcl, j * NW + w);
    if (opens[j]) s_lb[key[j] - kf] = rank[j];
    int64_t qn = 0, ql = 0;
    uint32_t ml = 0u, mr = 0u;
    if (dirs[j] == 0) {
      const int64_t q = (int64_t)rintf(ldexpf(rv[j], nr[j].s63));
      qn = (q >> 32) * (1 << kCountBits) + 1;
      ql = q & 0xffffffffll;
    }
    if (maxes) {
      const uint32_t m = wgbm_abs_bits(rv[j]);
      ml = dirs[j] == 0 ? m : 0u;
      mr = dirs[j] == 1 ? m : 0u;
    }
    add_slot(key[j] - kf, dirs[j] != 2, qn, ql, ml, mr);
  }
  wgbm_lds_barrier();  // slot sums, maxima and left bases are complete
  // the node words: the thread of a split node's first position in the
  // block stores them (a node inside the block) or adds them and reserves
  // the block's part of the children's ranges (a node crossing its edges)
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    if (!opens[j]) continue;
    const int k = key[j], sl = k - kf;
    const int64_t qn = s_qn[sl];
    const int32_t nl = (int32_t)(qn & ((1 << kCountBits) - 1));
    const int64_t qh = qn >> kCountBits, ql = s_ql[sl];
    const int64_t b0 = sk[j] > p0 ? sk[j] : p0, b1 = se[j] < p1 ? se[j] : p1;
    const int32_t nrr = (int32_t)(b1 - b0) - nl;
    const unsigned long long packed = ((unsigned long long)(uint32_t)nl << 32) | (uint32_t)nrr;
    if (sk[j] >= p0 && se[j] <= p1) {
      kw.cnt[k] = packed;
      kw.qh[k] = qh;
      kw.ql[k] = ql;
      if (maxes) {
        kw.ml[k] = s_ml[sl];
        kw.mr[k] = s_mr[sl];
      }
    } else {
      s_base[b0 == p0 ? 0 : 1] = atomicAdd(kw.cnt + k, packed);
      if (qh) atomicAdd((unsigned long long*)(kw.qh + k), (unsigned long long)qh);
      if (ql) atomicAdd((unsigned long long*)(kw.ql + k), (unsigned long long)ql);
      if (maxes) {
        if (s_ml[sl]) atomicMax(kw.ml + k, s_ml[sl]);
        if (s_mr[sl]) atomicMax(kw.mr + k, s_mr[sl]);
      }
    }
  }
  wgbm_lds_barrier();  // the reserved bases
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    if (!ok[j]) continue;
    const int64_t p = p0 + j * NT + tid;
    const int kl = 2 * key[j];  // the left child's key (one era)
    if (leaf_key) {
      const int t = key[j] / a.nodes;
      leaf_key[(int64_t)t * a.n + rowv[j]] = kl + (dirs[j] == 1 ? 1 : 0);
      continue;
    }
    if (dirs[j] == 2) {
      // a node that does not split: its rows stay, in its left child's segment
      order_next[p] = rowv[j];
      keyp_next[p] = kl;
      rpos_next[p] = rv[j];
      continue;
    }
    const int64_t b0 = sk[j] > p0 ? sk[j] : p0;
    const bool cross = sk[j] < p0 || se[j] > p1;
    const unsigned long long base = cross ? s_base[b0 == p0 ? 0 : 1] : 0ull;
    const int32_t rl = rank[j] - s_lb[key[j] - kf];  // the node's lefts before p in the block
    int64_t dst;
    if (dirs[j] == 0) {
      dst = sk[j] + (int64_t)(base >> 32) + rl;
    } else {
      const int32_t rr = (int32_t)(p - b0) - rl;  // its rights before p
      dst = se[j] - 1 - (int64_t)(base & 0xffffffffull) - rr;
    }
    // (always inside the node while its words start at zero; the test keeps
    // a broken invariant from writing past it)
    if (dst < sk[j] || dst >= se[j]) continue;
    order_next[dst] = rowv[j];
    keyp_next[dst] = kl + dirs[j];
    rpos_next[dst] = rv[j];
  }
}
template __global__ void partition_e1_kernel<256>(RouteArgs, KeyWords, int32_t, int32_t*,
                                                  int32_t*, float*, int32_t*);
template __global__ void partition_e1_kernel<1024>(RouteArgs, KeyWords, int32_t, int32_t*,
                                                   int32_t*, float*, int32_t*);

// The last level's leaf updates in row order (after partition_e1_kernel
// wrote every row's leaf key): pred[t][row] += lr * leaf of the row's node
// in tree t, as route_kernel's mode 2 does by position.  Four rows per
// thread, their key loads issued together.
__global__ __launch_bounds__(256) void leaf_rows_kernel(const int32_t* __restrict__ leaf_key,
                                                        int64_t n, int32_t T,
                                                        const NodeRoute* __restrict__ nroute,
                                                        float lr, float* __restrict__ pred,
                                                        int64_t pstride, int64_t pcol) {
  constexpr int U = 4;
  const int64_t total = (int64_t)T * n;
  const int64_t i0 = ((int64_t)blockIdx.x * 256) * U + threadIdx.x;
  int32_t k[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = i0 + u * 256;
    k[u] = i < total ? leaf_key[i] : 0;
  }
  NodeRoute nr[U];
#pragma unroll
  for (int u = 0; u < U; ++u) nr[u] = nroute[k[u]];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = i0 + u * 256;
    if (i >= total || nr[u].col != -1) continue;
    const int64_t t = i / n, row = i - t * n;
    float* pc = pred + t * pcol + row * pstride;
    *pc = *pc + lr * nr[u].leaf;
  }
}

// The three steps between route and scatter of a level with few keys (at
// most 64 eras), in one workgroup of 1024 threads: the block prefix, the node
// scan with one wave per node (wave w takes nodes w, w + 16, ...), and the
// tile plan of the next level's histogram (the key pairs of every split, the
// first n_list entries of key_list_next; skipped when n_list is 0).  The
// prefix and the node scan's outputs are read back by the same workgroup
// after a barrier.
__global__ __launch_bounds__(1024) void level_scan_kernel(
    int32_t nb, PartSums ps, int32_t T, int32_t nodes, int32_t E, int64_t n_pos,
    const int64_t* __restrict__ seg, const int32_t* __restrict__ present,
    const int32_t* __restrict__ split_l, LevelNext nx, int32_t n_list, int32_t tile_rows,
    int32_t max_tiles, Tile* __restrict__ tiles, int32_t* __restrict__ key_tile_start,
    int32_t* __restrict__ n_tiles) {
  block_scan_body(nb, ps);
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int tn = wave; tn < T * nodes; tn += 16) {
    const bool sp = present[tn] && split_l[tn] >= 0;
    const int64_t k0 = (int64_t)tn * E;
    const int64_t base = seg[k0];
    const int64_t c0 = 2 * k0;
    // E <= 64: era e on lane e
    int64_t L = 0, R = 0, qh = 0, ql = 0;
    if (lane < E) {
      const int64_t cnt = seg[k0 + lane + 1] - seg[k0 + lane];
      L = cnt;
      if (sp) segment_left_sums(k0 + lane, seg, ps, qh, ql, L);
      R = cnt - L;
    }
    int64_t il = wgbm_wave_incl_scan_i64(L), ir = wgbm_wave_incl_scan_i64(R);
    const int64_t ltot = __shfl(il, 63, 64), rtot = __shfl(ir, 63, 64);
    const int side = (ltot <= rtot) ? 0 : 1;  // the smaller child gets the histogram
    // one era: the children's shifts by node_shift_rule; several eras: per
    // (child, era) segment (era_child_shifts)
    int hs = 0, hs_l = 0, hs_r = 0;
    bool both = false;  // both children histogrammed
    if (E == 1) {
      uint32_t ml = 0, mr = 0;
      if (sp && nx.have_max) seg_child_max(tn, base, seg[k0 + E], ps, lane, 64, ml, mr);
      ml = wgbm_wave_reduce_max_u32(ml);
      mr = wgbm_wave_reduce_max_u32(mr);
      hs = nx.node_shift[tn];
      hs_l = sp && nx.have_max ? node_shift_rule(ml, hs, nx.qbits) : hs;
      hs_r = sp && nx.have_max ? node_shift_rule(mr, hs, nx.qbits) : hs;
      both = sp && (hs_l != hs || hs_r != hs);
    }
    if (lane < E) {
      nx.seg_next[c0 + lane] = base + il - L;
      nx.seg_next[c0 + E + lane] = base + ltot + ir - R;
      // child totals (the words of children that do not exist are zero)
      nx.tot_qh_next[c0 + lane] = sp ? qh : 0;
      nx.tot_ql_next[c0 + lane] = sp ? ql : 0;
      nx.tot_c_next[c0 + lane] = sp ? L : 0;
      nx.tot_qh_next[c0 + E + lane] = sp ? nx.tot_qh[k0 + lane] - qh : 0;
      nx.tot_ql_next[c0 + E + lane] = sp ? nx.tot_ql[k0 + lane] - ql : 0;
      nx.tot_c_next[c0 + E + lane] = sp ? R : 0;
      bool both_e = both;
      if (E > 1)
        era_child_shifts(k0 + lane, c0 + lane, c0 + E + lane, sp, ps, seg, nx, KeyWords{}, both_e);
      nx.key_list_next[2 * (k0 + lane)] =
          sp ? (int32_t)(c0 + (both_e ? 0 : side * E) + lane) : -1;
      nx.key_list_next[2 * (k0 + lane) + 1] = both_e ? (int32_t)(c0 + E + lane) : -1;
    }
    if (lane < 2) {
      nx.present_next[2 * tn + lane] = sp;
      if (E == 1) nx.node_shift_next[2 * tn + lane] = lane == 0 ? hs_l : hs_r;
    }
    if (tn == T * nodes - 1 && lane == 0) nx.seg_next[(int64_t)2 * T * nodes * E] = n_pos;
  }
  if (n_list <= 0) return;  // uniform
  __syncthreads();
  plan_tiles_body(nx.seg_next, 0, n_list, nx.key_list_next, tile_rows, 0, max_tiles, tiles,
                  key_tile_start, n_tiles);
}

// One-era split search fused with the leaf / record step: one lane per
// (node, local feature) scans the node's histogram as split_level_e1_kernel
// does (split.hip); the workgroup's best candidate is the max of the packed
// keys gain_key(gain) << 32 | (0xffffffff - flat index) of its waves.  With
// one workgroup per node that key is the node's pick and the workgroup's
// first wave finishes the node directly; otherwise every workgroup adds its
// key to best[tn] (atomicMax) and counts itself in done[tn], and the last
// one to arrive reads the final pick back and finishes the node (a release
// fence before the count, an acquire fence after; no workgroup waits for
// another).  Saves level_finish_kernel's launch on one-era levels.
template <int BT>
__global__ __launch_bounds__(256) void split_finish_e1_kernel(
    const int64_t* __restrict__ hq, const int32_t* __restrict__ hc, int32_t F, int32_t B_rt,
    int32_t n_sel, int32_t c0, const int32_t* __restrict__ node_shift, float mcw, float eps,
    float min_split_gain, unsigned long long* __restrict__ best, uint32_t* __restrict__ done,
    FinishE1 fa) {
  __shared__ unsigned long long s_key[4];
  __shared__ int s_last;
  const int B = BT > 0 ? BT : B_rt;
  const int bpn = (n_sel + 255) / 256;
  const int tl = blockIdx.x / bpn;  // node within the chunk (histogram index)
  const int tn = c0 + tl;           // node within the level
  const int l = (blockIdx.x - tl * bpn) * 256 + threadIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const bool pres = fa.present[tn] != 0;
  float bg = -__builtin_inff();
  int bi = 0x7fffffff;
  if (pres && l < n_sel) {
    const int s = node_shift[tn];
    const int f = fa.feat_sel[l];
    const int64_t base = ((int64_t)tl * F + f) * B;
    const int64_t* q = hq + base;
    const int32_t* c = hc + base;
    auto emit = [&](int b, float gn, float d) {
      (void)d;
      const int idx = l * (B - 1) + b;
      if (gn > min_split_gain && better(gn, idx, bg, bi)) {
        bg = gn;
        bi = idx;
      }
    };
    if constexpr (BT > 0) {
      float g[BT], h[BT];
#pragma unroll
      for (int b = 0; b < BT; ++b) {
        g[b] = wgbm_dequantise(q[b], s);
        h[b] = (float)c[b];
      }
      scan_bins(
          BT, mcw, eps, [&](int b) { return g[b]; }, [&](int b) { return h[b]; }, emit);
    } else {
      scan_bins(
          B, mcw, eps, [&](int b) { return wgbm_dequantise(q[b], s); },
          [&](int b) { return (float)c[b]; }, emit);
    }
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float og = __shfl_xor(bg, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (better(og, oi, bg, bi)) {
      bg = og;
      bi = oi;
    }
  }
  if (lane == 0)
    s_key[w] = bi != 0x7fffffff ? (((unsigned long long)gain_key(bg) << 32) |
                                   (unsigned long long)(0xffffffffu - (uint32_t)bi))
                                : 0ull;
  wgbm_lds_barrier();
  unsigned long long k = 0ull;
#pragma unroll
  for (int i = 0; i < 4; ++i) k = s_key[i] > k ? s_key[i] : k;
  if (bpn > 1) {
    if (threadIdx.x == 0) {
      if (k) atomicMax(best + tn, k);
      __threadfence();  // the key is visible before the arrival is counted
      const uint32_t prev = atomicAdd(done + tn, 1u);
      const bool last = prev == (uint32_t)(bpn - 1);
      if (last) {
        __threadfence();  // every other workgroup's key is visible
        k = __hip_atomic_load(best + tn, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        done[tn] = 0u;    // ready for the next level
      }
      s_last = last ? 1 : 0;
      s_key[0] = k;
    }
    __syncthreads();
    if (!s_last) return;  // uniform
    k = s_key[0];
  }
  if (w == 0)
    finish_node(tn, lane, fa.depth, fa.max_depth, fa.T, 1, fa.B, fa.present, true, k, nullptr,
                fa.split_l, fa.split_b, nullptr, fa.feat_sel, fa.tot_qh, fa.tot_ql, fa.tot_c,
                fa.shifts, fa.s63_add, fa.leaf_val, fa.rec, fa.best_next, nullptr, fa.nroute);
}

int launch_split_finish_e1(int n_tn, int32_t c0, hipStream_t st, const int64_t* hq,
                           const int32_t* hc, int32_t F, int32_t n_sel,
                           const int32_t* node_shift, float mcw, float eps,
                           float min_split_gain, unsigned long long* best, uint32_t* done,
                           const FinishE1& fa) {
  const dim3 grid((unsigned)(n_tn * ((n_sel + 255) / 256)));
  // a compile-time bin count (every bin loaded before the scan) for the
  // common ones: 10 is the estimator's default, 32 the benchmarks'
#define WGBM_FINISH_E1(BT)                                                                    \
  case BT:                                                                                    \
    hipLaunchKernelGGL(split_finish_e1_kernel<BT>, grid, dim3(256), 0, st, hq, hc, F, fa.B,    \
                       n_sel, c0, node_shift, mcw, eps, min_split_gain, best, done, fa);      \
    break;
  switch (fa.B) {
    WGBM_FINISH_E1(5)
    WGBM_FINISH_E1(8)
    WGBM_FINISH_E1(10)
    WGBM_FINISH_E1(16)
    WGBM_FINISH_E1(32)
    WGBM_FINISH_E1(64)
    default:
      hipLaunchKernelGGL(split_finish_e1_kernel<0>, grid, dim3(256), 0, st, hq, hc, F, fa.B,
                         n_sel, c0, node_shift, mcw, eps, min_split_gain, best, done, fa);
  }
#undef WGBM_FINISH_E1
  WGBM_LAUNCH_CHECK();
  return 0;
}

// The tiles of one list entry: a segment [b0, b0 + len) split into nt tiles
// of len / nt rows, the first len % nt one more (tile ids below ntot).
__device__ inline void write_entry_tiles(int key, int64_t b0, uint32_t len, int first, int nt,
                                         int j0, int dj, int ntot, Tile* __restrict__ tiles) {
  const uint32_t q = len / (uint32_t)nt, r = len - q * (uint32_t)nt;
  for (int j = j0; j < nt && first + j < ntot; j += dj) {
    const uint32_t uj = (uint32_t)j;
    Tile tl;
    tl.key = key;
    tl.pad = 0;
    tl.begin = b0 + (int64_t)(uj * q + (uj < r ? uj : r));
    tl.end = tl.begin + (int64_t)(q + (uj < r ? 1u : 0u));
    tiles[first + j] = tl;
  }
}

// One-era levels (E == 1): a thread per (tree, node).  The node's words
// that do not depend on the block prefix (flags, bounds, its route partials)
// are loaded before the prefix scan, which leaves its prefixes in LDS; the
// node's left / right child maxima come from the segmented block maxima, so
// each node costs a fixed number of loads whatever its size.  The next
// level's list entries are 2 tn (left child) and 2 tn + 1 (right child);
// with at most 1024 nodes their tiles are planned from registers, else from
// the words just written (plan_tiles_body).  Same outputs as
// level_scan_kernel.
__global__ __launch_bounds__(1024) void level_scan_e1_kernel(
    int32_t nb, PartSums ps, KeyWords kw, int32_t n_tn, int64_t n_pos,
    const int64_t* __restrict__ seg, const int32_t* __restrict__ present,
    const int32_t* __restrict__ split_l, LevelNext nx, int32_t plan, int32_t tile_rows,
    int32_t max_tiles, Tile* __restrict__ tiles, int32_t* __restrict__ key_tile_start,
    int32_t* __restrict__ n_tiles) {
  __shared__ int64_t l_qh[kScanLdsBlocks], l_ql[kScanLdsBlocks];
  __shared__ int64_t l_n[kScanLdsBlocks];
  __shared__ uint32_t l_ml[kScanLdsBlocks], l_mr[kScanLdsBlocks];
  const int t = threadIdx.x;
  const bool have_max = nx.have_max != 0;
  const bool one_pass = kw.cnt != nullptr;  // uniform
  // a node's words that do not need the prefix scan: q0 / q1 are its first
  // and last blocks; for a node inside one block its own partials, else the
  // partials of its part of the first block
  struct NodeWords {
    int32_t pr, sl, hs;
    int64_t base, end, tqh, tql;
    int64_t oqh, oql, bqh, bql;  // own partials, and those of the first block
    int32_t on, bn;
    uint32_t oml, omr, bml, bmr;
  };
  // (every load is unconditional and the words are used only after the
  // block scan, so that one round trip brings the flags and bounds and a
  // second the partials, both overlapping the scan)
  auto load_node = [&](int tn) {
    NodeWords x;
    x.pr = present[tn];
    x.sl = split_l[tn];
    x.base = seg[tn];
    x.end = seg[tn + 1];
    x.hs = nx.node_shift[tn];
    x.tqh = nx.tot_qh[tn];
    x.tql = nx.tot_ql[tn];
    x.bqh = x.bql = 0;
    x.bn = 0;
    x.oml = x.omr = x.bml = x.bmr = 0u;
    if (one_pass) {
      // the node's whole left sums (the partition's words), then cleared
      x.on = (int32_t)(kw.cnt[tn] >> 32);
      x.oqh = kw.qh[tn];
      x.oql = kw.ql[tn];
      if (have_max) {
        x.oml = kw.ml[tn];
        x.omr = kw.mr[tn];
      }
      kw.cnt[tn] = 0ull;
      kw.qh[tn] = 0;
      kw.ql[tn] = 0;
      kw.ml[tn] = 0u;
      kw.mr[tn] = 0u;
      return x;
    }
    const int64_t q0 = x.base / kPartBlock;
    const int64_t qb = q0 < nb ? q0 : nb - 1;  // an empty node may start at n_pos
    x.oqh = ps.own_qh[tn];
    x.oql = ps.own_ql[tn];
    x.on = ps.own_n[tn];
    x.bqh = ps.bl_qh[qb];
    x.bql = ps.bl_ql[qb];
    x.bn = ps.bl_n[qb];
    if (have_max) {
      x.oml = ps.own_ml[tn];
      x.omr = ps.own_mr[tn];
      x.bml = ps.bl_ml[qb];
      x.bmr = ps.bl_mr[qb];
    }
    return x;
  };
  NodeWords first{};
  const bool in_lds = nb <= kScanLdsBlocks;
  if (one_pass) {
    if (t < n_tn) first = load_node(t);
  } else {
    // the node's own words load while the block prefixes are scanned
    block_scan_body(nb, ps, have_max, in_lds, ScanLds{l_qh, l_ql, l_n, l_ml, l_mr}, [&]() {
      if (t < n_tn) first = load_node(t);
    });
    if (!in_lds) __syncthreads();  // the prefixes are read back from global memory
  }
  // the entries of this thread's node (when n_tn <= 1024): keys and bounds
  int32_t ka = -1, kb = -1;
  int64_t a0 = 0, a1 = 0, b1 = 0;
  auto finish_node = [&](int tn, const NodeWords& x) {
    const int64_t cnt = x.end - x.base;
    const bool sp = x.pr && x.sl >= 0;
    const int64_t xq0 = x.base / kPartBlock, xq1 = cnt > 0 ? (x.end - 1) / kPartBlock : xq0;
    const bool inside = one_pass || xq0 == xq1;  // (one pass: the node's words are whole)
    const bool use = sp && cnt > 0;
    int64_t L = cnt, qh = 0, ql = 0;
    uint32_t ml = use ? (inside ? x.oml : x.bml) : 0u;
    uint32_t mr = use ? (inside ? x.omr : x.bmr) : 0u;
    if (sp) {
      L = use ? (int64_t)(inside ? x.on : x.bn) : 0;
      qh = use ? (inside ? x.oqh : x.bqh) : 0;
      ql = use ? (inside ? x.oql : x.bql) : 0;
      if (use && !inside) {
        // the first blocks' partials of blocks q0 + 1 .. q1 (all start inside
        // the node), and the maxima of the run of blocks ending at q1
        const int q0 = (int)xq0, q1 = (int)xq1;
        if (in_lds) {
          L += l_n[q1] - l_n[q0];
          qh += l_qh[q1] - l_qh[q0];
          ql += l_ql[q1] - l_ql[q0];
        } else {
          L += ps.P_n[q1] - ps.P_n[q0];
          qh += ps.P_qh[q1] - ps.P_qh[q0];
          ql += ps.P_ql[q1] - ps.P_ql[q0];
        }
        if (have_max) {
          const uint32_t rl = in_lds ? l_ml[q1] : ps.pm_l[q1];
          const uint32_t rr = in_lds ? l_mr[q1] : ps.pm_r[q1];
          ml = rl > ml ? rl : ml;
          mr = rr > mr ? rr : mr;
        }
      }
    }
    const int64_t R = cnt - L;
    const int side = L <= R ? 0 : 1;  // the smaller child gets the histogram
    const int hs = x.hs;
    const int hs_l = sp && have_max ? node_shift_rule(ml, hs, nx.qbits) : hs;
    const int hs_r = sp && have_max ? node_shift_rule(mr, hs, nx.qbits) : hs;
    const bool both = sp && (hs_l != hs || hs_r != hs);  // both children histogrammed
    const int64_t c0 = 2 * (int64_t)tn;
    const int64_t base = x.base;
    nx.seg_next[c0] = base;
    nx.seg_next[c0 + 1] = base + L;
    // child totals (the words of children that do not exist are zero)
    nx.tot_qh_next[c0] = sp ? qh : 0;
    nx.tot_ql_next[c0] = sp ? ql : 0;
    nx.tot_c_next[c0] = sp ? L : 0;
    nx.tot_qh_next[c0 + 1] = sp ? x.tqh - qh : 0;
    nx.tot_ql_next[c0 + 1] = sp ? x.tql - ql : 0;
    nx.tot_c_next[c0 + 1] = sp ? R : 0;
    ka = sp ? (int32_t)(c0 + (both ? 0 : side)) : -1;
    kb = both ? (int32_t)(c0 + 1) : -1;
    nx.key_list_next[c0] = ka;
    nx.key_list_next[c0 + 1] = kb;
    nx.present_next[c0] = sp;
    nx.present_next[c0 + 1] = sp;
    nx.node_shift_next[c0] = hs_l;
    nx.node_shift_next[c0 + 1] = hs_r;
    a0 = base;
    a1 = base + L;
    b1 = x.end;
  };
  if (t < n_tn) finish_node(t, first);
  for (int tn = t + 1024; tn < n_tn; tn += 1024) finish_node(tn, load_node(tn));
  if (t == 0) nx.seg_next[2 * (int64_t)n_tn] = n_pos;
  if (!plan) return;  // uniform
  if (n_tn > 1024) {
    __syncthreads();
    plan_tiles_body(nx.seg_next, 0, 2 * n_tn, nx.key_list_next, tile_rows, 0, max_tiles, tiles,
                    key_tile_start, n_tiles);
    return;
  }
  // tiles per entry (plan_tiles_body's count, rounding up); key c0 spans
  // [a0, a1), key c0 + 1 spans [a1, b1)
  auto count = [&](int32_t key) -> int {
    if (key < 0) return 0;
    const uint32_t len = (uint32_t)((key & 1) ? b1 - a1 : a1 - a0);
    if (len == 0) return 0;
    const uint32_t k = (len + (uint32_t)tile_rows - 1) / (uint32_t)tile_rows;
    static_assert(WGBM_MAX_TILE_ROWS == 1 << 16, "tile row bound");
    const uint32_t kmin = (len + WGBM_MAX_TILE_ROWS - 1) >> 16;
    return (int)(k > kmin ? k : kmin);
  };
  __shared__ int64_t s_wsum[16];
  __shared__ int s_nbig;
  const bool live = t < n_tn;
  const int na = live ? count(ka) : 0, nbt = live ? count(kb) : 0;
  // exclusive scan of the node's tile counts (wave totals through LDS)
  const int lane = t & 63, w = t >> 6;
  const int64_t v = na + nbt;
  const int64_t x = wgbm_wave_incl_scan_i64(v);
  if (lane == 63) s_wsum[w] = x;
  if (t == 0) s_nbig = 0;
  wgbm_lds_barrier();
  const int64_t sw = wgbm_row_incl_scan_i64(lane < 16 ? s_wsum[lane] : 0);
  const int64_t total = wgbm_readlane_i64(sw, 15);
  const int64_t pre = wgbm_readlane_i64(sw, w > 0 ? w - 1 : 0);
  const int64_t ex = (w > 0 ? pre : 0) + x - v;
  const int ntot = total < max_tiles ? (int)total : max_tiles;
  if (live) {
    key_tile_start[2 * t] = (int32_t)ex;
    key_tile_start[2 * t + 1] = (int32_t)(ex + na);
  }
  if (t == 0) {
    key_tile_start[2 * n_tn] = (int32_t)total;
    *n_tiles = ntot;
  }
  // entries with many tiles are written by the whole workgroup afterwards
  constexpr int kMaxBig = 256, kSmall = 8;
  __shared__ int64_t s_b0[kMaxBig];
  __shared__ int s_bkey[kMaxBig], s_blen[kMaxBig], s_bfirst[kMaxBig], s_bnt[kMaxBig];
  for (int s2 = 0; s2 < 2 && live; ++s2) {
    const int32_t key = s2 ? kb : ka;
    const int nt = s2 ? nbt : na;
    if (nt == 0) continue;
    const int64_t e0 = (key & 1) ? a1 : a0, e1 = (key & 1) ? b1 : a1;
    const int first = (int)ex + (s2 ? na : 0);
    if (nt > kSmall) {
      const int slot = atomicAdd(&s_nbig, 1);
      if (slot < kMaxBig) {
        s_b0[slot] = e0;
        s_bkey[slot] = key;
        s_blen[slot] = (int)(e1 - e0);
        s_bfirst[slot] = first;
        s_bnt[slot] = nt;
        continue;
      }
    }
    write_entry_tiles(key, e0, (uint32_t)(e1 - e0), first, nt, 0, 1, ntot, tiles);
  }
  wgbm_lds_barrier();  // the large entries are listed in LDS
  const int nbig = s_nbig < kMaxBig ? s_nbig : kMaxBig;
  for (int k = 0; k < nbig; ++k)
    write_entry_tiles(s_bkey[k], s_b0[k], (uint32_t)s_blen[k], s_bfirst[k], s_bnt[k], t, 1024,
                      ntot, tiles);
}

__global__ void chunk_keys_kernel(const int32_t* __restrict__ present, int32_t E, int32_t n,
                                  int32_t* __restrict__ list) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < (int64_t)n * E) list[i] = present[i / E] ? (int32_t)i : -1;
}

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace wgbm
