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
                                  int32_t* __restrict__ order, int32_t* __restrict__ keyp,
                                  int64_t* __restrict__ seg,
                                  int32_t* __restrict__ present, int64_t* __restrict__ tot_q,
                                  int64_t* __restrict__ tot_c, unsigned long long* __restrict__ best,
                                  int32_t* __restrict__ agree_max) {
  // root order and segment key of every position, root segments, cleared
  // root totals and cleared depth-0 split-pick words
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid < (int64_t)T * n) {
    const int64_t t = gid / n, p = gid - t * n;
    order[gid] = root_order[p];
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
// Every position also carries its segment key (keyp, written by the root
// setup and by each level's scatter for the next level).
//
// route:   direction of every row of a split node (code <= bin goes left,
//          warpgbm/core.py:629), leaf update of the rows of a node that stops
//          here (core.py:602-605), per-(block, segment) left counts and child
//          totals reduced in LDS and added to the segment's words; the key of
//          every position (for the scatter) and the block's first / last
//          segment with its left count (for the carry).  Mode 0 only sums the
//          quantised residuals and rows of every segment (root totals).
// node_scan: one wave per (tree, node): the next level's segment offsets, the
//          presence of the children and the histogram key list (the smaller
//          child of every split, core.py:636-643).
// carry:   per block, the left rows of its first segment in earlier blocks
//          (a segmented scan over the blocks).
// scatter: stable destination of every row: left rank in its segment = left
//          rows before it in the block (block prefix) - left rows before the
//          segment's start in the block (+ the carry when the segment began in
//          an earlier block).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kPartThreads) void route_kernel(RouteArgs a) {
  // per-segment sums of the block, in the slot of the segment's first
  // position in the block (distinct for distinct non-empty segments; empty
  // segments own no position)
  __shared__ int64_t s_ql[kPartBlock], s_qr[kPartBlock];
  __shared__ int32_t s_nl[kPartBlock], s_nr[kPartBlock], s_key[kPartBlock];
  __shared__ int s_k[2];
  const int tid = threadIdx.x;
  const int64_t p0 = (int64_t)blockIdx.x * kPartBlock;
  const int64_t p1 = p0 + kPartBlock < a.n_pos ? p0 + kPartBlock : a.n_pos;
  if (tid == 0) {
    s_k[0] = a.keyp[p0];
    s_k[1] = a.keyp[p1 - 1];
  }
  for (int i = tid; i < kPartBlock; i += kPartThreads) {
    s_ql[i] = 0;
    s_qr[i] = 0;
    s_nl[i] = 0;
    s_nr[i] = 0;
    s_key[i] = -1;
  }
  __syncthreads();
  const int klo = s_k[0], khi = s_k[1];
  // the block's positions, four per thread (strided: coalesced), in phases so
  // that the loads of the four positions are in flight together
  constexpr int PJ = kPartBlock / kPartThreads;
  int key[PJ], slot[PJ], tnv[PJ], lv[PJ];
  int32_t rowv[PJ];
  bool ok[PJ];
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int64_t p = p0 + j * kPartThreads + tid;
    ok[j] = p < p1;
    key[j] = ok[j] ? a.keyp[p] : klo;
    rowv[j] = ok[j] ? a.order[p] : 0;
  }
#pragma unroll
  for (int j = 0; j < PJ; ++j) {
    const int64_t sk = a.seg[key[j]];
    slot[j] = (int)((sk > p0 ? sk : p0) - p0);
    tnv[j] = key[j] / a.E;
    // -2: the row stays (node absent), -1: leaf update, >= 0: split feature
    lv[j] = -2;
    if (ok[j] && a.present[tnv[j]]) lv[j] = a.mode == 1 ? a.split_l[tnv[j]] : -1;
  }
  if (a.mode == 0) {
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      if (!ok[j]) continue;
      const int t = tnv[j] / a.nodes;
      const int64_t q = wgbm_quantise(a.resid[(int64_t)t * a.n + rowv[j]], a.shifts[t]);
      s_key[slot[j]] = key[j];
      atomicAdd((unsigned long long*)&s_ql[slot[j]], (unsigned long long)q);
      atomicAdd(&s_nl[slot[j]], 1);
    }
  } else {
    int cv[PJ];
    float rv[PJ];
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      const int t = tnv[j] / a.nodes;
      cv[j] = 0;
      rv[j] = 0.0f;
      if (lv[j] >= 0) {
        cv[j] = (int)a.codes_cm[(int64_t)a.feat_sel[lv[j]] * a.n + rowv[j]];
        rv[j] = a.resid[(int64_t)t * a.n + rowv[j]];
      }
    }
#pragma unroll
    for (int j = 0; j < PJ; ++j) {
      if (!ok[j]) continue;
      const int64_t p = p0 + j * kPartThreads + tid;
      const int tn = tnv[j];
      const int t = tn / a.nodes;
      uint8_t dir = 2;  // stays in place
      if (lv[j] == -1) {
        // the node is a leaf: add lr * leaf to its rows' predictions
        float* pc = a.pred + (int64_t)t * a.pcol + (int64_t)rowv[j] * a.pstride;
        *pc = *pc + a.lr * a.leaf_val[tn];
      } else if (lv[j] >= 0) {
        const bool right = cv[j] > a.split_b[tn];
        const int64_t q = wgbm_quantise(rv[j], a.shifts[t]);
        dir = right ? 1 : 0;
        s_key[slot[j]] = key[j];
        if (right) {
          atomicAdd((unsigned long long*)&s_qr[slot[j]], (unsigned long long)q);
          atomicAdd(&s_nr[slot[j]], 1);
        } else {
          atomicAdd((unsigned long long*)&s_ql[slot[j]], (unsigned long long)q);
          atomicAdd(&s_nl[slot[j]], 1);
        }
      }
      a.dirbit[p] = dir;
    }
  }
  __syncthreads();
  for (int i = tid; i < kPartBlock; i += kPartThreads) {
    const int k = s_key[i];
    if (k < 0) continue;  // no summed rows start here
    if (a.mode == 0) {
      atomicAdd((unsigned long long*)&a.tot_q[k], (unsigned long long)s_ql[i]);
      atomicAdd((unsigned long long*)&a.tot_c[k], (unsigned long long)(int64_t)s_nl[i]);
      continue;
    }
    const int tn = k / a.E;
    const int e = k - tn * a.E;
    const int64_t kl = (int64_t)2 * tn * a.E + e, kr = kl + a.E;
    atomicAdd((unsigned long long*)&a.Lk[k], (unsigned long long)(int64_t)s_nl[i]);
    if (s_nl[i]) {
      atomicAdd((unsigned long long*)&a.tot_q[kl], (unsigned long long)s_ql[i]);
      atomicAdd((unsigned long long*)&a.tot_c[kl], (unsigned long long)(int64_t)s_nl[i]);
    }
    if (s_nr[i]) {
      atomicAdd((unsigned long long*)&a.tot_q[kr], (unsigned long long)s_qr[i]);
      atomicAdd((unsigned long long*)&a.tot_c[kr], (unsigned long long)(int64_t)s_nr[i]);
    }
  }
  if (a.mode != 0 && tid == 0) {
    // the first and last segments of the block and their left rows here
    const int64_t sl = a.seg[khi];
    a.blk_fk[blockIdx.x] = klo;
    a.blk_fl[blockIdx.x] = s_nl[0];
    a.blk_lk[blockIdx.x] = khi;
    a.blk_ll[blockIdx.x] = s_nl[(int)((sl > p0 ? sl : p0) - p0)];
  }
}

// one wave per (tree, node) of the level; four waves per workgroup
__global__ __launch_bounds__(256) void node_scan_kernel(
    int32_t T, int32_t nodes, int32_t E, int64_t n_pos, const int64_t* __restrict__ seg,
    const int32_t* __restrict__ present, const int32_t* __restrict__ split_l,
    const int64_t* __restrict__ Lk, int64_t* __restrict__ Lk_next,
    int64_t* __restrict__ seg_next, int32_t* __restrict__ present_next,
    int32_t* __restrict__ key_list_next) {
  const int lane = threadIdx.x & 63;
  const int tn = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tn >= T * nodes) return;  // uniform per wave; no workgroup barriers below
  const bool sp = present[tn] && split_l[tn] >= 0;
  const int64_t k0 = (int64_t)tn * E;
  const int64_t base = seg[k0];
  const int64_t c0 = 2 * k0;  // next keys of the children: c0 + side * E + e
  // left rows of the node (all of them when it does not split)
  int64_t ltot = 0, tot = 0;
  for (int e = lane; e < E; e += 64) {
    const int64_t cnt = seg[k0 + e + 1] - seg[k0 + e];
    ltot += sp ? Lk[k0 + e] : cnt;
    tot += cnt;
  }
  for (int o = 32; o > 0; o >>= 1) {
    ltot += __shfl_xor(ltot, o, 64);
    tot += __shfl_xor(tot, o, 64);
  }
  const int side = (ltot <= tot - ltot) ? 0 : 1;  // the smaller child gets the histogram
  int64_t carry_l = 0, carry_r = 0;
  for (int e0 = 0; e0 < E; e0 += 64) {
    const int e = e0 + lane;
    int64_t L = 0, R = 0;
    if (e < E) {
      const int64_t cnt = seg[k0 + e + 1] - seg[k0 + e];
      L = sp ? Lk[k0 + e] : cnt;
      R = cnt - L;
    }
    int64_t il = L, ir = R;  // inclusive wave scans
    for (int o = 1; o < 64; o <<= 1) {
      const int64_t yl = __shfl_up(il, o, 64), yr = __shfl_up(ir, o, 64);
      if (lane >= o) {
        il += yl;
        ir += yr;
      }
    }
    if (e < E) {
      seg_next[c0 + e] = base + carry_l + il - L;
      seg_next[c0 + E + e] = base + ltot + carry_r + ir - R;
      Lk_next[c0 + e] = 0;
      Lk_next[c0 + E + e] = 0;
      key_list_next[k0 + e] = sp ? (int32_t)(c0 + side * E + e) : -1;
    }
    carry_l += __shfl(il, 63, 64);
    carry_r += __shfl(ir, 63, 64);
  }
  if (lane < 2) present_next[2 * tn + lane] = sp;
  if (tn == T * nodes - 1 && lane == 0) seg_next[(int64_t)2 * T * nodes * E] = n_pos;
}

// carry[b] = left rows of block b's first segment in the blocks before b: a
// segmented inclusive scan S of the blocks' last-segment left counts (a run
// continues through blocks that lie inside one segment), read at b - 1.
// One workgroup of 1024 threads, tiles of 1024 blocks.
__global__ __launch_bounds__(1024) void block_carry_kernel(
    int32_t nb, const int32_t* __restrict__ fk, const int32_t* __restrict__ fl,
    const int32_t* __restrict__ lk, const int32_t* __restrict__ ll, int32_t* __restrict__ S,
    int32_t* __restrict__ carry) {
  (void)fl;
  __shared__ int64_t sv[1024];
  __shared__ int sh[1024];
  __shared__ int64_t s_prev;
  const int t = threadIdx.x;
  if (t == 0) s_prev = 0;
  __syncthreads();
  for (int b0 = 0; b0 < nb; b0 += 1024) {
    const int b = b0 + t;
    int64_t v = 0;
    int head = 1;
    if (b < nb) {
      v = ll[b];
      // the run of segment lk[b] continues from b - 1 when block b lies inside
      // that segment and block b - 1 ends in it
      head = !(fk[b] == lk[b] && b > 0 && lk[b - 1] == lk[b]);
    }
    sv[t] = v;
    sh[t] = head;
    __syncthreads();
    for (int o = 1; o < 1024; o <<= 1) {
      int64_t pv = 0;
      int ph = 0;
      if (t >= o) {
        pv = sv[t - o];
        ph = sh[t - o];
      }
      __syncthreads();
      if (t >= o && !sh[t]) {
        sv[t] = sv[t] + pv;
        sh[t] = ph;
      }
      __syncthreads();
    }
    // elements before the tile's first head continue the previous tile's run
    int64_t out = sv[t];
    if (!sh[t]) out += s_prev;
    if (b < nb) S[b] = (int32_t)out;
    __syncthreads();
    if (t == 1023) s_prev = out;
    __syncthreads();
  }
  __syncthreads();
  for (int b = t; b < nb; b += 1024) carry[b] = (b > 0 && lk[b - 1] == fk[b]) ? S[b - 1] : 0;
}

__global__ __launch_bounds__(kPartThreads) void scatter_kernel(
    int64_t n_pos, int32_t E, const int64_t* __restrict__ seg,
    const int64_t* __restrict__ seg_next, const int32_t* __restrict__ keyp,
    const uint8_t* __restrict__ dirbit, const int32_t* __restrict__ carry,
    const int32_t* __restrict__ order, int32_t* __restrict__ order_next,
    int32_t* __restrict__ keyp_next) {
  constexpr int PT = kPartBlock / kPartThreads;  // consecutive positions per thread
  __shared__ int32_t s_pl[kPartBlock + 1];      // left rows before each block position
  __shared__ int32_t s_w[kPartThreads / 64];
  const int tid = threadIdx.x;
  const int64_t p0 = (int64_t)blockIdx.x * kPartBlock;
  const int64_t pb = p0 + (int64_t)tid * PT;
  uint8_t d[PT];
  int cnt = 0;
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    d[j] = pb + j < n_pos ? dirbit[pb + j] : 2;
    cnt += d[j] == 0;
  }
  // exclusive block scan of the per-thread left counts
  const int lane = tid & 63, w = tid >> 6;
  int x = cnt;
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  if (lane == 63) s_w[w] = x;
  __syncthreads();
  int pre = 0;
  for (int k = 0; k < w; ++k) pre += s_w[k];
  int run = pre + x - cnt;
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    s_pl[tid * PT + j] = run;
    run += d[j] == 0;
  }
  __syncthreads();
  const int32_t cin = carry[blockIdx.x];
#pragma unroll
  for (int j = 0; j < PT; ++j) {
    const int64_t p = pb + j;
    if (p >= n_pos) break;
    const int32_t row = order[p];
    const int k = keyp[p];
    const int tn = k / E;
    const int64_t kl = (int64_t)2 * tn * E + (k - (int64_t)tn * E);  // left child's key
    if (d[j] == 2) {
      // a node that does not split: its rows stay, in its left child's segment
      order_next[p] = row;
      keyp_next[p] = (int32_t)kl;
      continue;
    }
    const int64_t sk = seg[k];
    const int64_t s0 = sk > p0 ? sk : p0;
    const int64_t rl = (int64_t)s_pl[tid * PT + j] - s_pl[s0 - p0] + (sk < p0 ? cin : 0);
    const int64_t dst = d[j] == 0 ? seg_next[kl] + rl : seg_next[kl + E] + ((p - sk) - rl);
    order_next[dst] = row;
    keyp_next[dst] = (int32_t)(d[j] == 0 ? kl : kl + E);
  }
}

__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace wgbm
