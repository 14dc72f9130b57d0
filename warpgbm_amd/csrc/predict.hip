// Tree-ensemble inference on int8 bin codes.
//
// Reference (warpgbm/cuda/predict.cu:13-44): thread (row i, tree t) starts at
// node 0 of the flattened table [T, M, 6] = (feature, bin, left, right,
// is_leaf, leaf_value); while !(is_leaf > 0.5): go left if code <= bin;
// at the leaf: atomicAdd(out[i], lr * leaf_value).
//
// Here one lane owns a row (or a (row, class) pair) and adds the trees in tree
// order, so out[i] = ((out[i] + lr*v_0) + lr*v_1) + ... is deterministic; it is
// one of the orders the reference's atomics may produce.  Each product lr*v is
// rounded to float32 before the add, as in the reference.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace wgbm {

// reference table format, walk bounded by M steps (malformed tables cannot
// loop forever; a walk that leaves the table contributes NaN)
// run_if (optional): the walk runs only when *run_if is nonzero (the fallback
// of wgbm_predict_forest's heap path, decided on the device)
__global__ void predict_table_kernel(const int8_t* __restrict__ codes, int64_t n, int64_t F,
                                     const float* __restrict__ table, int64_t T, int64_t M,
                                     float lr, float* __restrict__ out,
                                     const int32_t* __restrict__ run_if) {
  if (run_if && *run_if == 0) return;  // uniform
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int8_t* row = codes + i * F;
  float acc = out[i];
  for (int64_t t = 0; t < T; ++t) {
    const float* tree = table + t * M * 6;
    int64_t node = 0;
    float v = __builtin_nanf("");
    for (int64_t step = 0; step <= M; ++step) {
      const float* nd = tree + node * 6;
      if (nd[4] > 0.5f) {
        v = nd[5];
        break;
      }
      const int feat = (int)nd[0];
      const int sb = (int)nd[1];
      if (feat < 0 || feat >= F) break;
      const int nxt = (int)row[feat] <= sb ? (int)nd[2] : (int)nd[3];
      if (nxt < 0 || nxt >= M) break;
      node = nxt;
    }
    acc = acc + lr * v;
  }
  out[i] = acc;
}

// The reference's flat tables [T, M, 6] as heap tables of depth D (H =
// 2^(D+1) - 1 slots per tree), for wgbm_predict_forest's heap path: one
// thread per (tree, heap node h) walks from node 0 along h's path and
// writes what the flat walk of predict_table_kernel meets there: a leaf
// (feat -1, its value), a split (feature, bin), an absent node (-2, under a
// leaf) or -- where that walk would stop with NaN (a feature outside [0, F),
// a child index outside [0, M)) -- a leaf of value NaN, so the heap walk
// returns the same value.  A split on the last heap level (a deeper tree), a
// negative bin or a feature >= 65536 cannot be held: then *fallback is set
// and the caller's flat walk runs instead.  Bins of 127 and above hold as
// 255: every int8 code is <= such a bin, and every code byte of the native
// copy (127 and 128 included) is <= 255.
__global__ void flat_to_heap_kernel(const float* __restrict__ table, int64_t T, int64_t M,
                                    int64_t F, int32_t D, int32_t* __restrict__ feat,
                                    int32_t* __restrict__ bin, float* __restrict__ leaf,
                                    int32_t* __restrict__ fallback) {
  const int64_t H = (int64_t(2) << D) - 1;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= T * H) return;
  const int64_t t = gid / H;
  const int h = (int)(gid - t * H);
  const float* tree = table + t * M * 6;
  const int d = 31 - __builtin_clz((unsigned)(h + 1));  // depth of heap node h
  int32_t f_out = -2, b_out = 0;
  float v_out = 0.0f;
  int64_t node = 0;
  bool reached = true;
  for (int k = 0; k < d && reached; ++k) {
    const float* nd = tree + node * 6;
    if (nd[4] > 0.5f) {  // a leaf above h: h is absent
      reached = false;
      break;
    }
    const int f = (int)nd[0];
    if (f < 0 || f >= F) {  // the walk stops here (NaN): h is absent
      reached = false;
      break;
    }
    const int right = ((h + 1) >> (d - 1 - k)) & 1;
    const int nxt = right ? (int)nd[3] : (int)nd[2];
    if (nxt < 0 || nxt >= M) {
      // the walk stops (NaN) on this edge: a NaN leaf if it leads to h
      if (k == d - 1) {
        f_out = -1;
        v_out = __builtin_nanf("");
      }
      reached = false;
      break;
    }
    node = nxt;
  }
  if (reached) {
    const float* nd = tree + node * 6;
    if (nd[4] > 0.5f) {
      f_out = -1;
      v_out = nd[5];
    } else {
      const int f = (int)nd[0];
      const int sb = (int)nd[1];
      if (f < 0 || f >= F) {
        f_out = -1;
        v_out = __builtin_nanf("");
      } else if (d == D || sb < 0 || f > 65535) {
        *fallback = 1;
        f_out = -1;
      } else {
        f_out = f;
        b_out = sb < 127 ? sb : 255;
      }
    }
  }
  feat[gid] = f_out;
  bin[gid] = b_out;
  leaf[gid] = v_out;
}

// compact heap tables written by the engine: node h has children 2h+1, 2h+2.
//   feat[t][h] >= 0 split feature, -1 leaf; bin[t][h]; leaf[t][h]
// trees are ordered (round, class); out is [n, K] row-major, pre-initialised.
// codes are native (bytes in [0, B + 1], B = num_bins): the byte B stands for
// a negative code, which goes left at every split (a raw int8 code <= bin
// with bin >= 0), and B + 1 for a code >= B, which goes right; the other
// bytes are the codes themselves.
__global__ void predict_heap_kernel(const int8_t* __restrict__ codes, int64_t n, int64_t S,
                                    int32_t num_bins, const int32_t* __restrict__ feat,
                                    const int32_t* __restrict__ bin,
                                    const float* __restrict__ leaf, int32_t n_rounds, int32_t K,
                                    int32_t H, int32_t max_depth, float lr,
                                    float* __restrict__ out, const int32_t* __restrict__ skip) {
  if (skip && *skip) return;  // uniform: the caller's fallback runs instead
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * K) return;
  const int64_t i = gid / K;
  const int k = (int)(gid - i * K);
  const int8_t* row = codes + i * S;
  float acc = out[gid];
  for (int r = 0; r < n_rounds; ++r) {
    const int64_t t = (int64_t)r * K + k;
    const int32_t* ft = feat + t * H;
    const int32_t* bt = bin + t * H;
    int h = 0;
    for (int d = 0; d < max_depth; ++d) {
      const int f = ft[h];
      if (f < 0) break;
      const int c = (int)(uint8_t)row[f];
      h = 2 * h + ((c <= bt[h] || c == num_bins) ? 1 : 2);
    }
    acc = acc + lr * leaf[t * H + h];
  }
  out[gid] = acc;
}

// Complete-tree tables for the LDS predictors.  Per tree: (2^D - 1) node
// words for the levels above the last, feature << 16 | bin for a split whose
// ancestors are all splits, else (a leaf, an absent node, or any position
// under one) the always-left word 255 (every code byte is <= 255); and 2^D
// last-level values, slot s = lr times the leaf value of the first node on
// the path from the root to heap node 2^D - 1 + s that is not a split (or of
// that node itself), rounded to float32 as the walkers' per-tree products
// are.  A walk then takes exactly D steps with no leaf test and reaches
// the value the heap walk stops at.  Features are clamped into the row
// (S - 1 < 65536), as the walkers clamp them.
__global__ void complete_tables_kernel(const int32_t* __restrict__ feat,
                                       const int32_t* __restrict__ bin,
                                       const float* __restrict__ leaf, int64_t T, int32_t D,
                                       int64_t S, float lr, uint32_t* __restrict__ cnode,
                                       float* __restrict__ cleaf) {
  const int Hi = (1 << D) - 1, L = 1 << D, H = 2 * L - 1;
  const int64_t per = (int64_t)Hi + L;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= T * per) return;
  const int64_t t = gid / per;
  const int j = (int)(gid - t * per);
  const int32_t* ft = feat + t * H;
  if (j < Hi) {
    const int dj = 31 - __builtin_clz((unsigned)(j + 1));  // depth of node j
    bool split = true;
    for (int k = 0; k <= dj && split; ++k) split = ft[((j + 1) >> (dj - k)) - 1] >= 0;
    uint32_t w = 255u;
    if (split) {
      const int64_t f = ft[j] < S ? ft[j] : S - 1;
      w = ((uint32_t)f << 16) | ((uint32_t)bin[t * H + j] & 0xffu);
    }
    cnode[t * Hi + j] = w;
  } else {
    const int sl = j - Hi;
    const int h = Hi + sl;  // heap node at depth D
    int a = h;
    for (int k = 0; k < D; ++k) {
      const int ak = ((h + 1) >> (D - k)) - 1;
      if (ft[ak] < 0) {
        a = ak;
        break;
      }
    }
    cleaf[t * L + sl] = lr * leaf[t * H + a];
  }
}

// Code bytes as the LDS walkers read them: a native byte equal to num_bins (a
// negative code, left at every split) becomes 0, which also goes left at
// every split (split bins are >= 0), so a walk step is one compare: right iff
// code > bin.  bb = num_bins * 0x01010101.
__device__ __forceinline__ uint32_t walk_bytes(uint32_t x, uint32_t bb) {
  const uint32_t t = x ^ bb;  // zero bytes where x has num_bins
  // 0x80 in every byte of t that is not zero (no carries between bytes)
  const uint32_t nz = (((t & 0x7f7f7f7fu) + 0x7f7f7f7fu) | t) & 0x80808080u;
  return x & ((nz >> 7) * 0xffu);
}

// Raw int8 codes (the reference's bin_indices, any value) as the walkers
// read them: a negative code becomes 0, which goes left at every split as the
// reference's signed `code <= bin` sends it (split bins >= 0); 0..127 stay,
// so right iff code > bin as there.
__device__ __forceinline__ uint32_t raw_walk_bytes(uint32_t x) {
  return x & ~(((x >> 7) & 0x01010101u) * 0xffu);
}

// A walk over a complete table held in LDS, stepped by LDS byte address: the
// tree's node words start at `base`, node g (1-based heap index, children 2g
// and 2g + 1) sits at a = base + 4 (g - 1), so the step to child 2g + x is
// a' = 2a + 4 + 4x - base (mod 2^32): one compare, one select, one shift-add
// and the row byte's address per step.
typedef __attribute__((address_space(3))) uint32_t lds_u32_t;
typedef __attribute__((address_space(3))) uint8_t lds_u8_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_u8_t*)p;
}

struct Walk {
  uint32_t a, k0, k1;  // node address; step offsets for left / right
  __device__ __forceinline__ void start(uint32_t base) {
    a = base;
    k0 = 4u - base;
    k1 = 8u - base;
    // opaque to the optimiser, which would otherwise fold the select back into
    // select(4, 8) - base, one more instruction per step
    __asm__("" : "+v"(k0), "+v"(k1));
  }
  // row: LDS address of the row's first code byte
  __device__ __forceinline__ void step(uint32_t row) {
    const uint32_t w = *(const lds_u32_t*)(uintptr_t)a;
    const uint32_t c = *(const lds_u8_t*)(uintptr_t)(row + (w >> 16));
    a = 2u * a + (c > (w & 0xffu) ? k1 : k0);
  }
};

typedef __attribute__((address_space(3))) float lds_f32_t;

// Walks the trees j = j_first, j_first + G, ... (j < n_trees) of one row, NW
// in lock-step, and stores each tree's value at out_a + 4j.  LDS byte
// addresses: row_a = the row's code bytes, nodes_a = tree 0's node words (Hi
// per tree), values_a = tree 0's last-level values (Hi + 1 per tree).  After
// D steps a walk of tree j sits at a = nodes_a + 4 (j Hi + g - 1) with g =
// 2^D + slot, so its value is at a + c0 + 4j, c0 = values_a - nodes_a + 4 -
// 4 (Hi + 1): every address is an add, and the trees' node words advance by
// a uniform stride.  An idle walk (past n_trees, or row_on false) walks tree
// 0 and stores nothing.
template <int NW>
__device__ __forceinline__ void walk_trees(int j_first, int n_trees, int G, bool row_on,
                                           uint32_t row_a, uint32_t nodes_a, uint32_t values_a,
                                           int Hi, int D, uint32_t out_a) {
  const uint32_t hi4 = 4u * (uint32_t)Hi, nstep = hi4 * (uint32_t)G;
  const uint32_t c0 = values_a - nodes_a + 4u - 4u * (uint32_t)(Hi + 1);
  uint32_t nb = nodes_a + hi4 * (uint32_t)j_first;  // node words of tree j0
  for (int j0 = j_first; j0 < n_trees; j0 += NW * G, nb += NW * nstep) {
    Walk wk[NW];
    uint32_t t4[NW];
    bool on[NW];
#pragma unroll
    for (int k = 0; k < NW; ++k) {
      on[k] = row_on && j0 + k * G < n_trees;
      t4[k] = on[k] ? 4u * (uint32_t)(j0 + k * G) : 0u;
      wk[k].start(on[k] ? nb + (uint32_t)k * nstep : nodes_a);
    }
    for (int d = 0; d < D; ++d) {
#pragma unroll
      for (int k = 0; k < NW; ++k) wk[k].step(row_a);
    }
#pragma unroll
    for (int k = 0; k < NW; ++k)
      if (on[k])
        *(lds_f32_t*)(uintptr_t)(out_a + t4[k]) =
            *(const lds_f32_t*)(uintptr_t)(wk[k].a + c0 + t4[k]);
  }
}

// Row-block inference (same results as predict_heap_kernel): a workgroup of
// 1024 threads stages a block of RB rows of codes in LDS (one coalesced read
// of the rows instead of a dependent byte gather per tree level) and walks
// the trees a chunk of TC at a time: the chunk's complete-tree tables
// (complete_tables_kernel) are staged in LDS, every (row, tree) pair of the
// chunk is walked by its own thread (all walks independent: D dependent LDS
// reads each instead of D per tree in sequence), the products lr * leaf (the
// tables hold them) go to an LDS table [row][tree], and one thread per (row,
// class) adds them in tree order.  TC is a multiple of K, so tree t0 + j belongs to class j % K.
//   LDS: rows [RB][S + 4] bytes (a 4-byte pad per row spreads the rows of
//   one wave over the banks), node words [TC][2^D - 1], last-level values
//   [TC][2^D], vals [RB][TC + 1] (odd row stride: no bank conflicts).
constexpr int kPredThreads = 1024;
constexpr int kPredMaxAcc = 4;  // (row, class) accumulators per thread
constexpr int kPredWalks = 2;   // walks a thread advances in lock-step

__global__ __launch_bounds__(kPredThreads) void predict_rows_kernel(
    const int8_t* __restrict__ codes, int64_t n, int64_t S, int32_t num_bins,
    const uint32_t* __restrict__ cnode, const float* __restrict__ cleaf, int32_t n_rounds,
    int32_t K, int32_t max_depth, int32_t RB, int32_t TC, float* __restrict__ out,
    const int32_t* __restrict__ skip) {
  if (skip && *skip) return;  // uniform: the caller's fallback runs instead
  extern __shared__ uint32_t psm[];
  const int Sp = (int)S + 4;
  const int Hi = (1 << max_depth) - 1, L = 1 << max_depth;  // complete-table widths
  uint8_t* rows_s = reinterpret_cast<uint8_t*>(psm);
  uint32_t* nodes_s = psm + (RB * Sp) / 4;
  float* leaves_s = reinterpret_cast<float*>(nodes_s + TC * Hi);
  float* vals_s = leaves_s + TC * L;
  const int64_t row0 = (int64_t)blockIdx.x * RB;
  const int nr = (int)(n - row0 < RB ? n - row0 : RB);
  const int tid = threadIdx.x;
  const uint32_t bb = (uint32_t)num_bins * 0x01010101u;
  // stage the row block: 16-byte global loads, 4-byte LDS stores
  {
    const int q_per_row = (int)(S / 16);
    const int nq = nr * q_per_row;
    for (int q = tid; q < nq; q += kPredThreads) {
      const int r = q / q_per_row, c = q - r * q_per_row;
      typedef uint32_t u4 __attribute__((ext_vector_type(4)));
      const u4 v = __builtin_nontemporal_load(
          reinterpret_cast<const u4*>(codes + (row0 + r) * S) + c);
      uint32_t* dst = reinterpret_cast<uint32_t*>(rows_s + r * Sp + c * 16);
      dst[0] = walk_bytes(v.x, bb);
      dst[1] = walk_bytes(v.y, bb);
      dst[2] = walk_bytes(v.z, bb);
      dst[3] = walk_bytes(v.w, bb);
    }
  }
  // accumulators: pair m*1024 + tid = (row, class) = (p % RB, p / RB)
  float acc[kPredMaxAcc];
#pragma unroll
  for (int m = 0; m < kPredMaxAcc; ++m) {
    const int p = m * kPredThreads + tid;
    const int r = p % RB, k = p / RB;
    acc[m] = (k < K && r < nr) ? out[(row0 + r) * K + k] : 0.0f;
  }
  const int T = n_rounds * K;
  const int G = kPredThreads / RB;  // RB <= 256: G >= 4
  const bool walker = tid < G * RB;
  const int wr = walker ? tid % RB : 0;
  const int wt0 = walker ? tid / RB : 0;
  for (int t0 = 0; t0 < T; t0 += TC) {
    const int tc = T - t0 < TC ? T - t0 : TC;
    __syncthreads();  // rows staged / previous chunk's vals consumed
    for (int i = tid; i < tc * Hi; i += kPredThreads) nodes_s[i] = cnode[(int64_t)t0 * Hi + i];
    for (int i = tid; i < tc * L; i += kPredThreads) leaves_s[i] = cleaf[(int64_t)t0 * L + i];
    __syncthreads();
    // walks: thread w < G * RB owns row wr = w % RB and the chunk's trees
    // wt0, wt0 + G, ... (G = threads / RB row groups, no division per walk),
    // two in lock-step so that the LDS reads of one overlap those of the
    // other; max_depth steps on the complete tables (no leaf test)
    if (walker)
      walk_trees<kPredWalks>(wt0, tc, G, wr < nr, lds_addr(rows_s + wr * Sp), lds_addr(nodes_s),
                             lds_addr(leaves_s), Hi, max_depth, lds_addr(vals_s + wr * (TC + 1)));
    __syncthreads();
    // ordered sums: trees t0 + j of class k are j = k, k + K, ... (t0 % K == 0)
#pragma unroll
    for (int m = 0; m < kPredMaxAcc; ++m) {
      const int p = m * kPredThreads + tid;
      const int r = p % RB, k = p / RB;
      if (k < K && r < nr) {
        float a = acc[m];
        for (int j = k; j < tc; j += K) a = a + vals_s[r * (TC + 1) + j];
        acc[m] = a;
      }
    }
  }
#pragma unroll
  for (int m = 0; m < kPredMaxAcc; ++m) {
    const int p = m * kPredThreads + tid;
    const int r = p % RB, k = p / RB;
    if (k < K && r < nr) out[(row0 + r) * K + k] = acc[m];
  }
}

// ---------------------------------------------------------------------------
// Resident-tree inference, for ensembles whose complete-tree tables fit in
// LDS next to a row block (same results as predict_rows_kernel).  Persistent
// workgroups (one per CU) load every tree once, then stride over blocks of RB
// rows:
//   * the next block's codes are loaded into registers while the current one
//     is walked (QPT 16-byte loads per thread), then stored to the LDS row
//     buffer after the walks;
//   * waves 1..15 walk the (row, tree) pairs of the block, two per thread
//     in lock-step, and write lr * leaf (from the tables) to a per-block value
//     table [RB][T + 1];
//   * wave 0 meanwhile adds the previous block's table to `out` in tree
//     order (one lane per (row, class)), so the ordered sums run beside the
//     walks; the value tables alternate between two buffers.
// ---------------------------------------------------------------------------
constexpr int kResThreads = 1024;
constexpr int kResMaxQ = 4;  // 16-byte row loads per thread and block
constexpr int kResWalks = 2;  // walks a walker thread advances in lock-step

// RAW: the rows are raw int8 codes of stride S (a multiple of 8, read with
// 8-byte loads, twice as many per thread) mapped by raw_walk_bytes, instead
// of native codes (S a multiple of 16) mapped by walk_bytes.
template <bool RAW>
__global__ __launch_bounds__(kResThreads) void predict_resident_kernel(
    const int8_t* __restrict__ codes, int64_t n, int64_t S, int32_t num_bins,
    const uint32_t* __restrict__ cnode, const float* __restrict__ cleaf, int32_t T, int32_t K,
    int32_t max_depth, int32_t RB, float* __restrict__ out,
    const int32_t* __restrict__ skip) {
  if (skip && *skip) return;  // uniform: the caller's fallback runs instead
  extern __shared__ uint32_t psm[];
  const int Sp = (int)S + 4;
  const int TV = T + 1;  // value-table row stride (odd or even, see below)
  const int Hi = (1 << max_depth) - 1, L = 1 << max_depth;  // complete-table widths
  uint32_t* nodes_s = psm;
  float* leaves_s = reinterpret_cast<float*>(nodes_s + T * Hi);
  uint8_t* rows_s = reinterpret_cast<uint8_t*>(leaves_s + T * L);
  float* vals_s = reinterpret_cast<float*>(rows_s + RB * Sp);  // 2 x [RB][TV]
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const uint32_t bb = (uint32_t)num_bins * 0x01010101u;
  for (int i = tid; i < T * Hi; i += kResThreads) nodes_s[i] = cnode[i];
  for (int i = tid; i < T * L; i += kResThreads) leaves_s[i] = cleaf[i];
  const int64_t nblk = (n + RB - 1) / RB;
  constexpr int QW = RAW ? 2 : 4;            // 32-bit words per load
  constexpr int NQ = kResMaxQ * 4 / QW;      // loads per thread and block
  const int qpr = (int)(S / (4 * QW));       // loads per row
  const int nq = RB * qpr;
  typedef uint32_t uq __attribute__((ext_vector_type(QW)));
  uq pre[NQ];
  auto prefetch = [&](int64_t b) {
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int q = u * kResThreads + tid;
      const int r = q / qpr, c = q - r * qpr;
      const int64_t row = b * RB + r;
      pre[u] = uq{};
      if (q < nq && row < n)
        pre[u] = __builtin_nontemporal_load(reinterpret_cast<const uq*>(codes + row * S) + c);
    }
  };
  auto stash = [&]() {
#pragma unroll
    for (int u = 0; u < NQ; ++u) {
      const int q = u * kResThreads + tid;
      if (q < nq) {
        const int r = q / qpr, c = q - r * qpr;
        uint32_t* dst = reinterpret_cast<uint32_t*>(rows_s + r * Sp + c * 4 * QW);
#pragma unroll
        for (int k = 0; k < QW; ++k)
          dst[k] = RAW ? raw_walk_bytes(pre[u][k]) : walk_bytes(pre[u][k], bb);
      }
    }
  };
  // ordered sums of a finished block (wave 0): lane per (row, class)
  auto sums = [&](int64_t b, const float* vt) {
    const int64_t row0 = b * RB;
    const int nr = (int)(n - row0 < RB ? n - row0 : RB);
    for (int p = lane; p < RB * K; p += 64) {
      const int r = p % RB, k = p / RB;
      if (r >= nr) continue;
      float* o = out + (row0 + r) * K + k;
      const float* v = vt + r * TV;
      float a = *o;
      // tree order; eight loads issued ahead of their sequential adds
      int j = k;
      for (; j + 7 * K < T; j += 8 * K) {
        float x[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] = v[j + u * K];
#pragma unroll
        for (int u = 0; u < 8; ++u) a = a + x[u];
      }
      for (; j < T; j += K) a = a + v[j];
      *o = a;
    }
  };
  // walkers (waves 1..15): thread w owns row wr = w % RB of every block and
  // the trees wt0, wt0 + G, ... (G = walkers / RB row groups), so no walk
  // divides; the kWalkers - G * RB threads left over idle
  constexpr int kWalkers = kResThreads - 64;
  const int G = kWalkers / RB;  // RB <= 256: G >= 3
  const int wid = tid - 64;
  const bool walker = wid >= 0 && wid < G * RB;
  const int wr = walker ? wid % RB : 0;
  const int wt0 = walker ? wid / RB : 0;
  int64_t b = blockIdx.x;
  if (b < nblk) prefetch(b);
  int64_t prev = -1;
  for (int it = 0; b < nblk; b += gridDim.x, ++it) {
    stash();
    __syncthreads();  // rows of block b (and the tables) in LDS; last walks done
    if (b + gridDim.x < nblk) prefetch(b + gridDim.x);
    float* vt = vals_s + (it & 1) * RB * TV;
    if (tid < 64) {
      if (prev >= 0) sums(prev, vals_s + ((it & 1) ^ 1) * RB * TV);
    } else if (walker) {
      const int64_t row0 = b * RB;
      const int nr = (int)(n - row0 < RB ? n - row0 : RB);
      walk_trees<kResWalks>(wt0, T, G, wr < nr, lds_addr(rows_s + wr * Sp), lds_addr(nodes_s),
                            lds_addr(leaves_s), Hi, max_depth, lds_addr(vt + wr * TV));
    }
    prev = b;
    __syncthreads();  // the walks are done: the row buffer can be refilled
  }
  if (prev >= 0 && tid < 64) {
    // the last block: its table is the one the last iteration wrote
    int it_last = 0;
    for (int64_t bb = blockIdx.x; bb + gridDim.x < nblk; bb += gridDim.x) ++it_last;
    sums(prev, vals_s + (it_last & 1) * RB * TV);
  }
}

template __global__ void predict_resident_kernel<false>(const int8_t*, int64_t, int64_t, int32_t,
                                                        const uint32_t*, const float*, int32_t,
                                                        int32_t, int32_t, int32_t, float*,
                                                        const int32_t*);
template __global__ void predict_resident_kernel<true>(const int8_t*, int64_t, int64_t, int32_t,
                                                       const uint32_t*, const float*, int32_t,
                                                       int32_t, int32_t, int32_t, float*,
                                                       const int32_t*);

// block shape of predict_resident_kernel: 0 when the trees do not fit (raw:
// rows of raw codes, S a multiple of 8; else native rows, S a multiple of 16)
int predict_resident_plan(int64_t S, int32_t K, int32_t H, int32_t n_rounds, int32_t* RB_out,
                          size_t* lds_out, bool raw) {
  constexpr int64_t kBudget = 150 * 1024;
  const int64_t T = (int64_t)n_rounds * K;
  // complete tables: (H - 1) / 2 node words and (H + 1) / 2 values per tree
  if (S % (raw ? 8 : 16) != 0 || S > (1 << 16) || T * H * 4 > 64 * 1024) return 0;
  const int64_t Sp = S + 4;
  // RB rows: the row buffer, two value tables and at most kResMaxQ loads per thread
  int64_t RB = (kBudget - 4 * T * H) / (Sp + 8 * (T + 1));
  RB = std::min<int64_t>(RB, (int64_t)kResMaxQ * kResThreads * 16 / S);
  RB = std::min<int64_t>(RB, 256);
  if (RB < 8) return 0;
  *RB_out = (int32_t)RB;
  *lds_out = (size_t)(4 * T * H + RB * Sp + 8 * RB * (T + 1));
  return 1;
}

// block shape of predict_rows_kernel: 0 when the trees or rows do not fit
// (then predict_heap_kernel is used)
int predict_rows_plan(int64_t S, int32_t K, int32_t H, int32_t n_rounds, int32_t* RB_out,
                      int32_t* TC_out, size_t* lds_out) {
  constexpr int64_t kBudget = 64 * 1024;
  // complete tables: (H - 1) / 2 node words and (H + 1) / 2 values per tree
  if (S % 16 != 0 || S > (1 << 16) || (int64_t)4 * H * K > 32 * 1024) return 0;
  const int64_t T = (int64_t)n_rounds * K;
  int64_t m = std::max<int64_t>(1, (16 * 1024) / ((int64_t)4 * H * K));
  int64_t TC = std::min<int64_t>(m * K, std::max<int64_t>(K, (T + K - 1) / K * K));
  const int64_t Sp = S + 4;
  int64_t RB = (kBudget - 4 * TC * H) / (Sp + 4 * (TC + 1));
  RB = std::min<int64_t>(RB, 256);
  RB = std::min<int64_t>(RB, (int64_t)kPredMaxAcc * kPredThreads / K);
  if (RB < 16) return 0;
  *RB_out = (int32_t)RB;
  *TC_out = (int32_t)TC;
  *lds_out = (size_t)(RB * Sp + 4 * TC * H + 4 * RB * (TC + 1));
  return 1;
}

// in-place row softmax over K logits: exp(x - max) / sum, sequential in k
__global__ void softmax_rows_kernel(float* __restrict__ x, int64_t n, int32_t K) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float* r = x + i * K;
  float m = r[0];
  for (int k = 1; k < K; ++k) m = r[k] > m ? r[k] : m;
  float s = 0.0f;
  for (int k = 0; k < K; ++k) {
    const float e = wgbm_expf(r[k] - m);
    r[k] = e;
    s = s + e;
  }
  for (int k = 0; k < K; ++k) r[k] = r[k] / s;
}

// ---------------------------------------------------------------------------
// per-era split-gain importance (warpgbm/core.py:624-627): every internal node
// adds its per-era gains to acc[e][feature] with one float32 add per era, the
// nodes in the order the reference visits them.  node / fstart: the gain rows
// of the nodes grouped by feature (group f = node[fstart[f] .. fstart[f+1]),
// in visiting order), so each (feature, era) word is one thread's sequential
// sum and no two threads touch the same word.
// ---------------------------------------------------------------------------
__global__ void importance_add_kernel(float* __restrict__ acc, int32_t F, int32_t E,
                                      const float* __restrict__ gain,
                                      const int64_t* __restrict__ node,
                                      const int64_t* __restrict__ fstart) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)F * E) return;
  const int f = (int)(gid / E), e = (int)(gid - (int64_t)f * E);
  float* w = acc + (int64_t)e * F + f;
  float s = *w;
  const int64_t i1 = fstart[f + 1];
  int64_t i = fstart[f];
  // batches of 16 gathers in flight ahead of their (sequential) adds, the
  // node indices of the next batch loaded with this batch's gains (one
  // memory round trip per batch; a feature can hold thousands of nodes)
  constexpr int U = 16;
  int64_t nx[U];
  if (i + U <= i1) {
#pragma unroll
    for (int u = 0; u < U; ++u) nx[u] = node[i + u];
  }
  for (; i + U <= i1; i += U) {
    float g[U];
#pragma unroll
    for (int u = 0; u < U; ++u) g[u] = gain[nx[u] * E + e];
    if (i + 2 * U <= i1) {
#pragma unroll
      for (int u = 0; u < U; ++u) nx[u] = node[i + U + u];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) s = s + g[u];
  }
  for (; i < i1; ++i) s = s + gain[node[i] * E + e];
  *w = s;
}

}  // namespace wgbm
