// Quantile binning.
//
// Reference binner (warpgbm/cuda/binner.cu:12-25): for one feature column,
//   bin = 0; while (bin < B-1 && x >= edges[bin]) ++bin;
// i.e. the number of leading edges <= x (NaN x -> 0).  With sorted edges this
// is #{j : edges[j] <= x}; the batched kernel uses a branch-free binary search
// for that count, which equals the linear scan whenever the predicate
// x >= edges[j] is monotone in j (sorted, or all-NaN, edges).
//
// Edges (warpgbm/core.py:529-534 calls torch.quantile): for q_j, j = 1..B-1,
// over the ascending column s[0..n-1], d = s[hi] - s[lo]:
//   rank = q_j * (n-1) (float32); lo = floor(rank); hi = ceil(rank); w = rank - lo
//   edge = w < 0.5 ? fma(w, d, s[lo]) : fma(w - 1, d, s[hi])
// (torch's lerp evaluates both branches as single-rounding fused multiply-adds:
// its vectorised CPU kernel by construction and its CUDA kernel through the
// compiler's default contraction), and every edge is NaN when the column holds
// a NaN (NaNs sort last).
#include "common.hpp"
#include "kernels.hpp"

namespace wgbm {

// ---------------------------------------------------------------------------
// reference-compatible single-column binner: literal linear scan
// ---------------------------------------------------------------------------
// bin = the length of the longest prefix of the edges that the value is >=
// (the reference's `while (bin < ne && v >= edges[bin]) ++bin`, any edge
// order, NaN stopping the prefix), for kBinColumnU values per thread.  The
// edges are walked in the same order by every lane (a uniform index: scalar
// loads, eight per wave and step) and each value keeps a running "still in
// the prefix" flag instead of leaving the loop, so no lane waits on a load
// of its own; the walk ends when no value of the wave is still in it.
__global__ __launch_bounds__(256) void bin_column_kernel(const float* __restrict__ x, int64_t n,
                                                         const float* __restrict__ edges,
                                                         int32_t n_edges,
                                                         int8_t* __restrict__ out) {
  constexpr int U = kBinColumnU;
  const int64_t i0 = (int64_t)blockIdx.x * 256 * U + threadIdx.x;
  float v[U];
  int bin[U];
  bool in[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = i0 + (int64_t)u * 256;
    v[u] = i < n ? x[i] : 0.0f;
    bin[u] = 0;
    in[u] = i < n;
  }
  // eight edges per step, their (uniform) loads issued together
  constexpr int EB = 8;
  for (int b0 = 0; b0 < n_edges; b0 += EB) {
    bool any = false;
#pragma unroll
    for (int u = 0; u < U; ++u) any = any || in[u];
    if (__ballot(any) == 0ull) break;  // uniform: every value of the wave has stopped
    float e[EB];
#pragma unroll
    for (int k = 0; k < EB; ++k) e[k] = edges[b0 + k < n_edges ? b0 + k : n_edges - 1];
#pragma unroll
    for (int k = 0; k < EB; ++k) {
      if (b0 + k >= n_edges) break;  // uniform
#pragma unroll
      for (int u = 0; u < U; ++u) {
        in[u] = in[u] && v[u] >= e[k];
        bin[u] += in[u] ? 1 : 0;
      }
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = i0 + (int64_t)u * 256;
    if (i < n) out[i] = (int8_t)bin[u];
  }
}

// #{j < ne : e[j] <= v} for sorted e (branch-free lower bound on the predicate)
// The binner's edge lists in LDS are in breadth-first (Eytzinger) order:
// node p of the complete search tree of 2^k - 1 nodes (k levels, the
// smallest with 2^k - 1 >= ne) holds sorted edge (2j + 1) 2^(k-1-d) - 1,
// d = depth of p, j = p + 1 - 2^d (edges past ne are +inf).  The search
// descends k levels without a branch; every lane of a step reads within one
// level, and feature lists start 1 mod 16 words apart (eytz_stride), so
// the 16 features a wave searches at a time fall in different banks at the
// top levels.  count = #{edges <= v} as count_le: a +inf value also counts
// the +inf padding, hence the clamp to ne; NaN compares false: 0.
__host__ __device__ inline int eytz_levels(int ne) {
  int k = 0;
  while ((1 << k) - 1 < ne) ++k;
  return k;
}
__host__ __device__ inline int eytz_stride(int ne) {
  const int nodes = (1 << eytz_levels(ne)) - 1;
  const int m = nodes > 1 ? nodes : 1;
  return (m - 1 + 15) / 16 * 16 + 1;
}
__device__ inline int eytz_count(const float* e, int k, int ne, float v) {
  uint32_t idx = 0;
  for (int s = 0; s < k; ++s) idx = 2u * idx + 1u + (v >= e[idx] ? 1u : 0u);
  const int c = (int)idx - ((1 << k) - 1);
  return c < ne ? c : ne;
}

__device__ inline int count_le(const float* e, int ne, float v) {
  int lo = 0, len = ne;
  while (len > 0) {
    const int half = len >> 1;
    const bool ge = v >= e[lo + half];
    lo = ge ? lo + half + 1 : lo;
    len = ge ? len - half - 1 : half;
  }
  return lo;
}

// ---------------------------------------------------------------------------
// The row-major code matrix codes_rm [n, S] is this library's own layout
// ("native codes"), read by the histogram kernels and the heap predictor:
// with B = num_bins, every byte is in [0, B + 1]:
//   a code c of a real feature    -> c        if 0 <= c < B
//                                 -> B        if c < 0   (routed left)
//                                 -> B + 1    if c >= B  (routed right)
//   padding bytes F..S-1          -> B + 1.
// Histograms drop both B and B + 1 (the reference skips codes outside
// [0, B): histogram_kernel.cu:41), and a kernel that knows every byte is in
// range needs no clamp.  The column-major copy codes_cm [F, n] keeps the raw
// signed codes (the partition compares them as the reference does,
// core.py:629).
//
// batched binner: X [n, F] row-major float32 (row stride xs floats) ->
//   codes_rm [n, S] (native; the binner's codes are in [0, n_edges] and
//   num_bins = n_edges + 1) and, if non-null, codes_cm [F, n].
// workgroup: 64 features x BT_R rows (the feature tiles of a row block
// consecutive in the XCD work order, so a cache line shared by two tiles is
// fetched once); the edges of its 64 features staged in LDS once.  Thread
// (row group g = t / 16, quad q = t % 16) owns features f0 + 4q .. + 3 of
// rows g, g + 16, ...: one 16-byte load per row when the rows are 16-byte
// aligned (VEC), and the row's four codes stored as one 32-bit word when the
// code rows allow it (rm_words); four rows' loads are issued before they are
// searched.  The column-major copy is transposed through LDS and written as
// 32-bit words of four rows (when n and the pointer allow; bytes otherwise).
// ---------------------------------------------------------------------------
constexpr int BT_F = kBinTileFeats, BT_R = kBinTileRows, BT_U = 4;
static_assert(BT_F == 64 && BT_R == 256, "16 feature quads x 16 row groups per step");

template <bool VEC>
__global__ __launch_bounds__(256) void bin_matrix_kernel(
    const float* __restrict__ X, int64_t n, int32_t F, int64_t xs,
    const float* __restrict__ edges, int32_t n_edges, int8_t* __restrict__ codes_rm, int64_t S,
    int8_t* __restrict__ codes_cm) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  extern __shared__ float sedge[];  // [BT_F][eytz_stride(n_edges)], breadth-first order
  __shared__ __align__(4) int8_t tcode[BT_F][BT_R + 4];
  const int nft = (F + BT_F - 1) / BT_F;
  const int64_t n_work = (n + BT_R - 1) / BT_R * nft;
  const int64_t w = wgbm_xcd_work(blockIdx.x, n_work);
  if (w >= n_work) return;  // uniform over the workgroup
  const int64_t r0 = w / nft * BT_R;
  const int f0 = (int)(w % nft) * BT_F;
  const int tid = threadIdx.x;
  const int ek = eytz_levels(n_edges), es = eytz_stride(n_edges);
  const int enodes = (1 << ek) - 1;
  for (int i = tid; i < BT_F * es; i += blockDim.x) {
    const int fl = i / es;
    const int p = i - fl * es;
    const int f = f0 + fl;
    float val = __builtin_inff();
    if (p < enodes) {
      const int d = 31 - __builtin_clz((unsigned)(p + 1));
      const int j = p + 1 - (1 << d);
      const int si = ((2 * j + 1) << (ek - 1 - d)) - 1;
      if (f < F && si < n_edges) val = edges[(int64_t)f * n_edges + si];
    }
    sedge[i] = val;
  }
  __syncthreads();
  const int q = tid & 15, g = tid >> 4;
  const int fq = f0 + 4 * q;  // first feature of the thread's quad
  const int nvf = F - fq < 4 ? (F - fq > 0 ? F - fq : 0) : 4;  // its real features
  const int8_t pad = (int8_t)(n_edges + 2);                     // num_bins + 1
  const bool rm_words = (S & 3) == 0 && ((uintptr_t)codes_rm & 3) == 0;
  // thread (g, q) bins rows k0 + BT_U g + u (u < BT_U) of its feature quad, so
  // that its codes of one feature for those rows form one 32-bit word of the
  // transposed tile (lanes of a wave then store to distinct banks)
  static_assert(BT_U == 4, "a transposed word holds the codes of four rows");
  for (int k0 = 0; k0 < BT_R; k0 += 16 * BT_U) {
    float v[BT_U][4];
#pragma unroll
    for (int u = 0; u < BT_U; ++u) {
      const int64_t r = r0 + k0 + BT_U * g + u;
#pragma unroll
      for (int c = 0; c < 4; ++c) v[u][c] = 0.0f;
      if (r < n) {
        const float* src = X + r * xs + fq;
        if (VEC && nvf == 4) {
          const f32x4 x4 = *reinterpret_cast<const f32x4*>(src);
          v[u][0] = x4.x;
          v[u][1] = x4.y;
          v[u][2] = x4.z;
          v[u][3] = x4.w;
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (c < nvf) v[u][c] = src[c];
        }
      }
    }
    uint32_t tw[4] = {0u, 0u, 0u, 0u};  // feature c's codes of the thread's rows
#pragma unroll
    for (int u = 0; u < BT_U; ++u) {
      const int k = k0 + BT_U * g + u;
      const int64_t r = r0 + k;
      uint32_t word = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int8_t code =
            c < nvf ? (int8_t)eytz_count(sedge + (4 * q + c) * es, ek, n_edges, v[u][c]) : pad;
        tw[c] |= (uint32_t)(uint8_t)code << (8 * u);
        word |= (uint32_t)(uint8_t)code << (8 * c);
      }
      if (r < n && fq < S) {
        int8_t* dst = codes_rm + r * S + fq;
        if (rm_words && fq + 4 <= S) {
          *reinterpret_cast<uint32_t*>(dst) = word;
        } else {
          for (int c = 0; c < 4 && fq + c < S; ++c) dst[c] = (int8_t)(word >> (8 * c));
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c)
      *reinterpret_cast<uint32_t*>(&tcode[4 * q + c][k0 + BT_U * g]) = tw[c];
  }
  if (!codes_cm) return;  // uniform over the workgroup
  __syncthreads();
  // column-major: lane l of wave wv writes rows r0 + 4l .. 4l + 3 of features
  // wv, wv + 4, ... of the tile
  const int l = tid & 63, wv = tid >> 6;
  const int64_t r = r0 + 4 * l;
  const bool cm_words = (n & 3) == 0 && ((uintptr_t)codes_cm & 3) == 0;
  if (r < n) {
    for (int k = wv; k < BT_F && f0 + k < F; k += 4) {
      int8_t* dst = codes_cm + (int64_t)(f0 + k) * n + r;
      if (cm_words) {  // r + 3 < n: n and r are multiples of 4
        *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(&tcode[k][4 * l]);
      } else {
        for (int c = 0; c < 4 && r + c < n; ++c) dst[c] = tcode[k][4 * l + c];
      }
    }
  }
}
int bin_edge_stride(int32_t n_edges) { return eytz_stride(n_edges); }

template __global__ void bin_matrix_kernel<true>(const float*, int64_t, int32_t, int64_t,
                                                 const float*, int32_t, int8_t*, int64_t, int8_t*);
template __global__ void bin_matrix_kernel<false>(const float*, int64_t, int32_t, int64_t,
                                                  const float*, int32_t, int8_t*, int64_t, int8_t*);

// padding bytes beyond the last 64-feature tile (S > round_up(F, 64))
__global__ void pad_codes_kernel(int8_t* __restrict__ codes_rm, int64_t n, int64_t S,
                                 int32_t from, int8_t value) {
  const int64_t w = S - from;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * w) return;
  const int64_t r = gid / w;
  codes_rm[r * S + from + (gid - r * w)] = value;
}

// pre-binned int8 input [n, F] (row stride xs bytes) -> native row-major
// codes for num_bins B + raw column-major copy.  With over != null, a
// workgroup that copies a value >= B stores 1 there (plain stores of one
// value: no atomics; the flag is cleared before).
__global__ __launch_bounds__(256) void copy_prebinned_kernel(const int8_t* __restrict__ X,
                                                             int64_t n, int32_t F, int64_t xs,
                                                             int8_t* __restrict__ codes_rm,
                                                             int64_t S,
                                                             int8_t* __restrict__ codes_cm,
                                                             int32_t num_bins,
                                                             int32_t* __restrict__ over) {
  __shared__ int8_t tcode[BT_F][BT_R + 4];
  // tiles in the XCD work order, as bin_matrix_kernel
  const int nft = (F + BT_F - 1) / BT_F;
  const int64_t n_work = (n + BT_R - 1) / BT_R * nft;
  const int64_t w = wgbm_xcd_work(blockIdx.x, n_work);
  if (w >= n_work) return;  // uniform over the workgroup
  const int64_t r0 = w / nft * BT_R;
  const int f0 = (int)(w % nft) * BT_F;
  const int tid = threadIdx.x;
  const int fl = tid & 63;
  const int rq = tid >> 6;  // rows rq, rq + 4, ... of the tile
  const int f = f0 + fl;
  int hit = 0;
  const int8_t neg = (int8_t)num_bins, over_b = (int8_t)(num_bins + 1);
  for (int k0 = 0; k0 < BT_R; k0 += 4 * BT_U) {
    int8_t c[BT_U];
#pragma unroll
    for (int u = 0; u < BT_U; ++u) {
      const int64_t r = r0 + k0 + rq + 4 * u;
      c[u] = (r < n && f < F) ? X[r * xs + f] : (int8_t)0;
    }
#pragma unroll
    for (int u = 0; u < BT_U; ++u) {
      const int k = k0 + rq + 4 * u;
      const int64_t r = r0 + k;
      int8_t nat = over_b;  // padding columns: num_bins + 1
      if (r < n && f < F) {
        hit |= (int)c[u] >= num_bins;
        nat = c[u] < 0 ? neg : ((int)c[u] >= num_bins ? over_b : c[u]);
      }
      tcode[fl][k] = c[u];
      if (r < n && f < S) codes_rm[r * S + f] = nat;
    }
  }
  if (over && __syncthreads_or(hit) && tid == 0) over[0] = 1;
  if (!codes_cm) return;  // uniform over the workgroup
  __syncthreads();
  // column-major raw codes: thread t writes row r0 + t of every feature
  const int64_t r = r0 + tid;
  if (r < n) {
    for (int k = 0; k < BT_F && f0 + k < F; ++k)
      codes_cm[(int64_t)(f0 + k) * n + r] = tcode[k][tid];
  }
}

// ---------------------------------------------------------------------------
// quantile edges from ascending-sorted columns sorted[F][n] (NaN last)
// ---------------------------------------------------------------------------
__global__ void quantile_edges_kernel(const float* __restrict__ sorted, int64_t n, int32_t F,
                                      const float* __restrict__ q, int32_t nq,
                                      float* __restrict__ edges) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)F * nq) return;
  const int f = (int)(gid / nq);
  const int j = (int)(gid - (int64_t)f * nq);
  const float* s = sorted + (int64_t)f * n;
  const int64_t last = n - 1;
  const bool has_nan = s[last] != s[last];
  const float rank = has_nan ? (float)last : q[j] * (float)last;
  int64_t lo = (int64_t)rank;
  const float w = rank - (float)lo;
  int64_t hi = (int64_t)ceilf(rank);
  lo = lo < 0 ? 0 : (lo > last ? last : lo);  // q outside [0, 1] stays in bounds
  hi = hi < 0 ? 0 : (hi > last ? last : hi);
  const float a = s[lo], b = s[hi];
  const float d = b - a;
  edges[gid] = w < 0.5f ? fmaf(w, d, a) : fmaf(w - 1.0f, d, b);
}


// ---------------------------------------------------------------------------
// Native quantile edges: the order statistics torch.quantile interpolates
// between, found by radix selection instead of a sort.
//
// keys: order-preserving uint32 encoding of the float32 values, column-major
// [F][n] (NaN -> 0xffffffff, i.e. after +inf, as in torch.sort).  For each
// feature one workgroup selects the ranks lo_j = floor(q_j (n-1)) and
// hi_j = ceil(q_j (n-1)) with four passes over the column, one byte of the
// key per pass: pass 1 histograms the top byte of every key; pass k
// histograms byte k of the keys whose top k-1 bytes equal a target's known
// prefix.  The selected keys are decoded and interpolated exactly as in
// quantile_edges_kernel.
// ---------------------------------------------------------------------------
__device__ inline uint32_t float_to_key(float x) {
  uint32_t u = __float_as_uint(x);
  if (x != x) return 0xffffffffu;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
// the key of a value's bits, the value not a NaN
__device__ inline uint32_t bits_to_key(uint32_t u) {
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline float key_to_float(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// X [n, F] float32 (row stride xs) -> vals [F][ks] (the values' bits; ks >=
// n, a multiple of 4, so every column starts on 16 bytes): a workgroup moves
// 64 features x kTransRows rows in 64 x 64 tiles through LDS, and keeps the
// smallest and largest key of each of its features (a NaN key is the
// largest), merged into kmin / kmax [F] with one atomic per feature.  Loads: 16 threads read
// one row's 64 values as four-value quads (VEC: 16-byte loads, when the
// rows are 16-byte aligned; a quad past the last feature reads its valid
// values one by one); stores: 16 threads write one feature's 64 rows as
// 16-byte quads.
template <bool VEC>
__global__ __launch_bounds__(256) void transpose_values_kernel(const float* __restrict__ X,
                                                               int64_t n, int32_t F, int64_t xs,
                                                               int64_t ks,
                                                               uint32_t* __restrict__ keys,
                                                             uint32_t* __restrict__ kmin,
                                                             uint32_t* __restrict__ kmax) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  __shared__ uint32_t t[64][65];
  __shared__ uint32_t s_mn[16][64], s_mx[16][64];
  // (row block, feature tile) in the XCD work order, feature tiles of a row
  // block consecutive: rows are not line-aligned, and the neighbouring tiles
  // that share a row's lines then read them from the same L2
  const int nft = (F + 63) / 64;
  const int64_t n_work = (n + kTransRows - 1) / kTransRows * nft;
  const int64_t wk = wgbm_xcd_work(blockIdx.x, n_work);
  if (wk >= n_work) return;  // uniform over the workgroup
  const int64_t rb = wk / nft;
  const int f0 = (int)(wk % nft) * 64;
  const int g = threadIdx.x >> 4;  // load: row group; store: feature group
  const int qd = threadIdx.x & 15;  // load: feature quad; store: row quad
  const int fq = f0 + 4 * qd;      // first feature of the load quad
  const int nvf = F - fq < 4 ? (F - fq > 0 ? F - fq : 0) : 4;  // valid features of the quad
  uint32_t mn[4], mx[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    mn[c] = 0xffffffffu;
    mx[c] = 0u;
  }
  for (int64_t r0 = rb * kTransRows; r0 < n && r0 < (rb + 1) * kTransRows; r0 += 64) {
    __syncthreads();  // the previous tile has been written out
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int rr = g + 16 * k;
      const int64_t r = r0 + rr;
      float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      const bool row_ok = r < n;
      if (row_ok) {
        const float* src = X + r * xs + fq;
        if (VEC && nvf == 4) {
          const f32x4 w = *reinterpret_cast<const f32x4*>(src);
          v[0] = w.x;
          v[1] = w.y;
          v[2] = w.z;
          v[3] = w.w;
        } else {
#pragma unroll
          for (int c = 0; c < 4; ++c)
            if (c < nvf) v[c] = src[c];
        }
      }
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        if (row_ok && c < nvf) {
          const uint32_t key = float_to_key(v[c]);
          mn[c] = key < mn[c] ? key : mn[c];
          mx[c] = key > mx[c] ? key : mx[c];
        }
        t[rr][4 * qd + c] = __float_as_uint(v[c]);
      }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int fl = g + 16 * k;  // feature within the tile
      const int f = f0 + fl;
      const int64_t r = r0 + 4 * qd;
      if (f >= F || r >= n) continue;
      uint32_t* dst = keys + (int64_t)f * ks + r;
      if (r + 3 < n) {
        u32x4 w;
        w.x = t[4 * qd + 0][fl];
        w.y = t[4 * qd + 1][fl];
        w.z = t[4 * qd + 2][fl];
        w.w = t[4 * qd + 3][fl];
        *reinterpret_cast<u32x4*>(dst) = w;  // ks and r are multiples of 4
      } else {
        for (int c = 0; r + c < n; ++c) dst[c] = t[4 * qd + c][fl];
      }
    }
  }
  // per-feature extremes: thread (g, qd) holds features fq..fq+3 of row group g
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    s_mn[g][4 * qd + c] = mn[c];
    s_mx[g][4 * qd + c] = mx[c];
  }
  __syncthreads();
  if (threadIdx.x < 64 && f0 + (int)threadIdx.x < F) {
    const int c = threadIdx.x;
    uint32_t a = s_mn[0][c], b = s_mx[0][c];
    for (int w = 1; w < 16; ++w) {
      a = s_mn[w][c] < a ? s_mn[w][c] : a;
      b = s_mx[w][c] > b ? s_mx[w][c] : b;
    }
    atomicMin(&kmin[f0 + c], a);
    atomicMax(&kmax[f0 + c], b);
  }
}
template __global__ void transpose_values_kernel<true>(const float*, int64_t, int32_t, int64_t,
                                                     int64_t, uint32_t*, uint32_t*, uint32_t*);
template __global__ void transpose_values_kernel<false>(const float*, int64_t, int32_t, int64_t,
                                                      int64_t, uint32_t*, uint32_t*, uint32_t*);

constexpr int kSelThreads = 512;
constexpr int kSelMaxTargets = 256;   // 2 * 126 ranks at most (num_bins <= 127)
constexpr int kSelGroup = 32;         // distinct prefixes histogrammed per scan
constexpr int kSelBuckets = 4096;     // value buckets of the first pass

// One workgroup per feature (512 threads, ~37 KB of LDS: four per CU, so a
// 1000-feature matrix runs in one round).  The order statistics at ranks
// floor / ceil(q (n-1)) are found in two scans of the column plus work on a
// small buffer:
//   1. histogram of kSelBuckets value buckets between the column's smallest
//      and largest value, bucket = clamp(int(fma(v, scale, offset))): any
//      function non-decreasing in the value works (each bucket is then a
//      contiguous run of the sorted column), this one costs three VALU
//      operations a value, which is what the scan is bound by;
//   2. the keys of the buckets that hold a target rank are copied to a
//      per-feature buffer (the whole buckets, so a target's rank inside the
//      buffer is the buffer keys of lower buckets plus its rank inside its
//      bucket);
//   3. radix selection (four byte passes) over the buffer.
// A column whose target buckets exceed the buffer (heavy ties, outliers that
// stretch the range, infinities) runs the radix selection over the whole
// column instead; a column holding a NaN gets NaN edges (torch.quantile) and
// a constant column its value.
//
// The columns hold the values' bits (transpose_values_kernel); the buffer and
// the radix selection use the order-preserving keys.  The two column scans
// read 16-byte quads (columns start on 16 bytes: ks is a multiple of 4),
// several per thread in flight.
__global__ __launch_bounds__(kSelThreads) void quantile_select_kernel(
    const uint32_t* __restrict__ keys, int64_t n, int64_t ks, int32_t F,
    const float* __restrict__ q, int32_t nq, float* __restrict__ edges,
    const uint32_t* __restrict__ kmin, const uint32_t* __restrict__ kmax,
    uint32_t* __restrict__ cbuf, int64_t ccap) {
  typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
  __shared__ uint32_t hist[kSelGroup][256];        // 32 KB (also the value buckets)
  __shared__ uint32_t tprefix[kSelMaxTargets];      // known key bits of each target
  __shared__ int64_t trank[kSelMaxTargets];         // rank still to find within the prefix
  __shared__ uint32_t dist[kSelMaxTargets];         // distinct prefixes of this pass (sorted)
  __shared__ uint32_t tbucket[kSelMaxTargets];      // value bucket of each target
  __shared__ uint32_t tfirst[kSelMaxTargets];       // first occurrence of its prefix
  __shared__ uint32_t marked[kSelBuckets / 32];     // buckets copied to the buffer
  __shared__ uint32_t wsum[kSelThreads / 64];
  __shared__ int s_nd;
  __shared__ uint32_t s_tot;
  __shared__ uint32_t s_cnt;
  constexpr int nwaves = kSelThreads / 64;
  const int f = blockIdx.x;
  if (f >= F) return;
  const uint32_t* col = keys + (int64_t)f * ks;
  const u32x4* col4 = reinterpret_cast<const u32x4*>(col);
  const int64_t n4 = n >> 2;  // whole quads; keys [4 * n4, n) are the tail
  uint32_t* cb = cbuf + (int64_t)f * ccap;
  const int nt = 2 * nq;
  const int64_t last = n - 1;
  const int tid = threadIdx.x;
  const uint32_t kmn = kmin[f], kmx = kmax[f];
  float* out = edges + (int64_t)f * nq;
  if (kmx == 0xffffffffu) {  // a NaN anywhere makes every quantile NaN
    for (int j = tid; j < nq; j += kSelThreads) out[j] = __builtin_nanf("");
    return;
  }
  // a constant column: every order statistic is its value (interpolated
  // below like any other, which fixes the sign of a zero as torch does)
  const bool constant = kmn == kmx;
  for (int t = tid; t < nt; t += kSelThreads) tprefix[t] = kmn;
  if (!constant) {
    for (int t = tid; t < nt; t += kSelThreads) {
      const float rank = q[t >> 1] * (float)last;
      int64_t r = (t & 1) ? (int64_t)ceilf(rank) : (int64_t)rank;
      r = r < 0 ? 0 : (r > last ? last : r);
      trank[t] = r;
      tprefix[t] = 0;
    }
    // ---- value buckets
    const float lo = key_to_float(kmn), hi = key_to_float(kmx);
    float scale = (float)kSelBuckets / (hi - lo);
    if (!(scale < __builtin_inff())) scale = 0.0f;  // infinite ends: everything in bucket 0
    const float off = -lo * scale;
    auto bucket = [&](uint32_t bits) -> int {
      // non-decreasing in the value: a correctly rounded fma is monotone in v
      // for scale >= 0, and so is the clamp (fmaxf maps a NaN to 0)
      const float v = __builtin_fmaf(__uint_as_float(bits), scale, off);
      return (int)fminf(fmaxf(v, 0.0f), (float)(kSelBuckets - 1));
    };
    uint32_t* H = &hist[0][0];  // [kSelBuckets]
    for (int i = tid; i < kSelBuckets; i += kSelThreads) H[i] = 0;
    for (int i = tid; i < kSelBuckets / 32; i += kSelThreads) marked[i] = 0;
    if (tid == 0) s_cnt = 0;
    __syncthreads();
    // The column in batches of two 16-byte quads per thread (quads i and
    // i + kSelThreads); two batches alternate so that the next batch's loads
    // are in flight while this one is counted (a thread that loaded, waited
    // and counted left the memory idle half the time).  Quads past the end
    // are not read.
    constexpr int64_t kQ = kSelThreads;
    // quads past the end read the last quad (straight-line loads, so that the
    // wait before a batch covers only its own loads); their keys are not used
    auto ld4 = [&](int64_t i) { return col4[i < n4 ? i : n4 - 1]; };
    auto count4 = [&](const u32x4& k, bool v) {
      if (v) {
        atomicAdd(&H[bucket(k.x)], 1u);
        atomicAdd(&H[bucket(k.y)], 1u);
        atomicAdd(&H[bucket(k.z)], 1u);
        atomicAdd(&H[bucket(k.w)], 1u);
      }
    };
    if (n4 > 0) {
      int64_t i0 = tid;
      u32x4 a0 = ld4(i0), a1 = ld4(i0 + kQ);
      for (; i0 < n4; i0 += 4 * kQ) {
        const int64_t j0 = i0 + 2 * kQ;
        const u32x4 b0 = ld4(j0), b1 = ld4(j0 + kQ);
        count4(a0, true);
        count4(a1, i0 + kQ < n4);
        a0 = ld4(j0 + 2 * kQ);
        a1 = ld4(j0 + 3 * kQ);
        count4(b0, j0 < n4);
        count4(b1, j0 + kQ < n4);
      }
    }
    for (int64_t i = 4 * n4 + tid; i < n; i += kSelThreads) atomicAdd(&H[bucket(col[i])], 1u);
    __syncthreads();
    // exclusive prefix of the buckets, in place: thread t owns buckets
    // [8t, 8t + 8)
    constexpr int per = kSelBuckets / kSelThreads;
    static_assert(per * kSelThreads == kSelBuckets, "buckets per thread");
    auto block_exclusive_scan = [&](uint32_t* a) {
      uint32_t v[per], sum = 0;
#pragma unroll
      for (int k = 0; k < per; ++k) {
        v[k] = a[tid * per + k];
        sum += v[k];
      }
      const int lane = tid & 63, w = tid >> 6;
      uint32_t inc = sum;
      for (int o = 1; o < 64; o <<= 1) {
        const uint32_t y = __shfl_up(inc, o, 64);
        if (lane >= o) inc += y;
      }
      if (lane == 63) wsum[w] = inc;
      __syncthreads();
      uint32_t base = inc - sum;
      for (int k = 0; k < w; ++k) base += wsum[k];
#pragma unroll
      for (int k = 0; k < per; ++k) {
        a[tid * per + k] = base;
        base += v[k];
      }
      __syncthreads();
    };
    // sizes are needed again below: keep them in the buffer-rank scan's input
    uint32_t* C = H;  // exclusive prefix (C[b] = keys in buckets < b)
    uint32_t sz[per];
#pragma unroll
    for (int k = 0; k < per; ++k) sz[k] = H[tid * per + k];
    block_exclusive_scan(C);
    // bucket of every target (last bucket b with C[b] <= rank)
    for (int t = tid; t < nt; t += kSelThreads) {
      const int64_t r = trank[t];
      int a = 0, b = kSelBuckets - 1;
      while (a < b) {
        const int m = (a + b + 1) >> 1;
        if ((int64_t)C[m] <= r) a = m; else b = m - 1;
      }
      tbucket[t] = (uint32_t)a;
      atomicOr(&marked[a >> 5], 1u << (a & 31));
    }
    __syncthreads();
    // buffer ranks: keys of marked buckets below the target's bucket + rank
    // inside the bucket (M = exclusive prefix of the marked buckets' sizes)
    {
      uint32_t* M = &hist[16][0];  // [kSelBuckets] words after C
#pragma unroll
      for (int k = 0; k < per; ++k) {
        const int b = tid * per + k;
        M[b] = ((marked[b >> 5] >> (b & 31)) & 1u) ? sz[k] : 0u;
      }
      __syncthreads();
      if (tid == kSelThreads - 1) {
        uint32_t tl = 0;
        for (int k = 0; k < per; ++k) tl += M[tid * per + k];
        s_tot = tl;  // completed by the scan below
      }
      __syncthreads();
      block_exclusive_scan(M);
      if (tid == kSelThreads - 1) s_tot += M[kSelBuckets - per];
      __syncthreads();
      if ((int64_t)s_tot <= ccap) {
        for (int t = tid; t < nt; t += kSelThreads) {
          const int b = (int)tbucket[t];
          trank[t] = (int64_t)M[b] + (trank[t] - (int64_t)C[b]);
        }
      }
      __syncthreads();
    }
    const uint32_t* src = col;  // what the radix selection scans: the column's
    int64_t ns = n;             // values, or the buffer's keys
    if ((int64_t)s_tot <= ccap) {
      // Batches of two quads per thread (8 keys, double-buffered as in the
      // first scan): a thread marks the keys it keeps, a DPP scan over the
      // wave gives each lane its offset, and one LDS reservation per wave
      // and batch places them (the order inside the buffer is free: the
      // selection below only counts).
      const int lane = tid & 63;
      auto take = [&](uint32_t k) -> uint32_t {
        const int b = bucket(k);
        return (marked[b >> 5] >> (b & 31)) & 1u;
      };
      auto keep8 = [&](const u32x4& x, bool vx, const u32x4& y, bool vy) {
        uint32_t bits = 0;
        if (vx) bits |= take(x.x) | take(x.y) << 1 | take(x.z) << 2 | take(x.w) << 3;
        if (vy) bits |= take(y.x) << 4 | take(y.y) << 5 | take(y.z) << 6 | take(y.w) << 7;
        const int64_t cnt = __builtin_popcount(bits);
        const int64_t inc = wgbm_wave_incl_scan_i64(cnt);
        const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)inc, 63);
        if (tot == 0) return;  // wave-uniform
        uint32_t base = 0;
        if (lane == 63) base = atomicAdd(&s_cnt, tot);
        base = (uint32_t)__builtin_amdgcn_readlane((int)base, 63);
        uint32_t o = base + (uint32_t)(inc - cnt);  // < s_tot <= ccap
        const uint32_t kk[8] = {x.x, x.y, x.z, x.w, y.x, y.y, y.z, y.w};
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if ((bits >> j) & 1u) cb[o++] = bits_to_key(kk[j]);
      };
      if (n4 > 0) {
        // the same trip count for every thread: keep8's wave scan and lane
        // 63's reservation need the whole wave
        u32x4 a0 = ld4(tid), a1 = ld4(tid + kQ);
        for (int64_t q0 = 0; q0 < n4; q0 += 4 * kQ) {
          const int64_t i0 = q0 + tid, j0 = i0 + 2 * kQ;
          const u32x4 b0 = ld4(j0), b1 = ld4(j0 + kQ);
          keep8(a0, i0 < n4, a1, i0 + kQ < n4);
          a0 = ld4(j0 + 2 * kQ);
          a1 = ld4(j0 + 3 * kQ);
          keep8(b0, j0 < n4, b1, j0 + kQ < n4);
        }
      }
      {
        // the tail: fewer than 4 keys, one per thread
        const int64_t i = 4 * n4 + tid;
        const uint32_t k = i < n ? col[i] : 0u;
        const uint32_t bit = (i < n && take(k)) ? 1u : 0u;
        const int64_t inc = wgbm_wave_incl_scan_i64((int64_t)bit);
        const uint32_t tot = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)inc, 63);
        if (tot) {
          uint32_t base = 0;
          if (lane == 63) base = atomicAdd(&s_cnt, tot);
          base = (uint32_t)__builtin_amdgcn_readlane((int)base, 63);
          if (bit) cb[base + (uint32_t)inc - 1u] = bits_to_key(k);
        }
      }
      __syncthreads();
      src = cb;
      ns = (int64_t)s_tot;
    }
    // ---- radix selection over src (ranks in trank are ranks within src)
    // src is read in batches of 8 keys per thread in flight (the column's
    // values are turned into keys here)
    const bool src_vals = src == col;
    auto for_src = [&](auto fn) {
      for (int64_t i0 = tid; i0 < ns; i0 += 8 * kSelThreads) {
        uint32_t k[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          const int64_t i = i0 + u * kSelThreads;
          k[u] = src[i < ns ? i : ns - 1];  // (i0 < ns, so ns >= 1)
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
          if (i0 + u * kSelThreads < ns) fn(src_vals ? bits_to_key(k[u]) : k[u]);
      }
    };
    // a 256-bin row of counts -> inclusive prefix, in place (one wave, 4 bins
    // a lane)
    auto row_prefix = [&](uint32_t* row) {
      const int ln = tid & 63;
      uint32_t v[4];
      uint32_t t = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        t += row[4 * ln + j];
        v[j] = t;
      }
      const uint32_t base = (uint32_t)(wgbm_wave_incl_scan_i64((int64_t)t) - t);
#pragma unroll
      for (int j = 0; j < 4; ++j) row[4 * ln + j] = base + v[j];
    };
    // first bin whose inclusive prefix exceeds r (bins 0..255; 255 when none
    // below does), and r made relative to that bin
    auto pick_bin = [&](const uint32_t* P, int64_t& r) {
      int a = 0, b = 255;
      while (a < b) {
        const int mid = (a + b) >> 1;
        if ((int64_t)P[mid] > r) b = mid; else a = mid + 1;
      }
      if (a > 0) r -= P[a - 1];
      return a;
    };
    for (int i = tid; i < nwaves * 256; i += kSelThreads) (&hist[0][0])[i] = 0;
    __syncthreads();
    {
      const int w = tid >> 6;
      for_src([&](uint32_t k) { atomicAdd(&hist[w][k >> 24], 1u); });
    }
    __syncthreads();
    for (int b = tid; b < 256; b += kSelThreads) {
      uint32_t sum = 0;
      for (int w = 0; w < nwaves; ++w) sum += hist[w][b];
      hist[nwaves][b] = sum;
    }
    __syncthreads();
    if (tid < 64) row_prefix(hist[nwaves]);
    __syncthreads();
    for (int t = tid; t < nt; t += kSelThreads) {
      int64_t r = trank[t];
      const int b = pick_bin(hist[nwaves], r);
      tprefix[t] = (uint32_t)b;
      trank[t] = r;
    }
    __syncthreads();
    // index of prefix pre in the sorted dist[lo..hi] (or where it would be)
    auto find = [&](uint32_t pre, int a, int b) {
      while (a < b) {
        const int mid = (a + b) >> 1;
        if (dist[mid] < pre) a = mid + 1; else b = mid;
      }
      return a;
    };
    // passes 2..4: next byte of the keys that share a target's prefix
    for (int pass = 1; pass < 4; ++pass) {
      const int sh = 32 - 8 * pass;  // prefix = key >> sh
      // sorted distinct prefixes, in parallel (a serial sort on one thread
      // waits on every LDS access behind the other waves' atomics): thread
      // t marks whether it holds the first occurrence of its value, then a
      // first occurrence stores its value at the count of distinct values
      // below it
      if (tid == 0) s_nd = 0;
      if (tid < nt) {
        const uint32_t v = tprefix[tid];
        bool first = true;
        for (int u = 0; u < tid; ++u) first = first && tprefix[u] != v;
        tfirst[tid] = first ? 1u : 0u;
      }
      __syncthreads();
      if (tid < nt && tfirst[tid]) {
        const uint32_t v = tprefix[tid];
        int below = 0;
        for (int u = 0; u < nt; ++u) below += (tfirst[u] && tprefix[u] < v) ? 1 : 0;
        dist[below] = v;
        atomicAdd(&s_nd, 1);
      }
      __syncthreads();
      const int nd = s_nd;
      for (int g0 = 0; g0 < nd; g0 += kSelGroup) {
        const int gn = nd - g0 < kSelGroup ? nd - g0 : kSelGroup;
        for (int i = tid; i < gn * 256; i += kSelThreads) (&hist[0][0])[i] = 0;
        __syncthreads();
        const uint32_t lo_p = dist[g0], hi_p = dist[g0 + gn - 1];
        for_src([&](uint32_t k) {
          const uint32_t pre = k >> sh;
          if (pre < lo_p || pre > hi_p) return;
          const int g = find(pre, g0, g0 + gn - 1);
          if (dist[g] == pre) atomicAdd(&hist[g - g0][(k >> (sh - 8)) & 255u], 1u);
        });
        __syncthreads();
        for (int g = tid >> 6; g < gn; g += nwaves) row_prefix(hist[g]);
        __syncthreads();
        for (int t = tid; t < nt; t += kSelThreads) {
          const uint32_t pre = tprefix[t];
          if (pre < dist[g0] || pre > dist[g0 + gn - 1]) continue;
          const int g = find(pre, g0, g0 + gn - 1);
          int64_t r = trank[t];
          const int b = pick_bin(hist[g - g0], r);
          tprefix[t] = (pre << 8) | (uint32_t)b;
          trank[t] = r;
        }
        __syncthreads();
      }
    }
  }  // !constant
  __syncthreads();
  // interpolate (torch.quantile, linear): see quantile_edges_kernel
  for (int j = tid; j < nq; j += kSelThreads) {
    const float rank = q[j] * (float)last;
    const int64_t lo_r = (int64_t)rank;
    const float w = rank - (float)lo_r;
    const float a = key_to_float(tprefix[2 * j]);
    const float b = key_to_float(tprefix[2 * j + 1]);
    const float d = b - a;
    out[j] = w < 0.5f ? fmaf(w, d, a) : fmaf(w - 1.0f, d, b);
  }
}

}  // namespace wgbm
