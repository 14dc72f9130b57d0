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
__global__ void bin_column_kernel(const float* __restrict__ x, int64_t n,
                                  const float* __restrict__ edges, int32_t n_edges,
                                  int8_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = x[i];
  int b = 0;
  while (b < n_edges && v >= edges[b]) ++b;
  out[i] = (int8_t)b;
}

// #{j < ne : e[j] <= v} for sorted e (branch-free lower bound on the predicate)
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
// workgroup: 64 features x BT_R rows; the edges of its 64 features staged in
// LDS once.  Lane l of every wave owns feature f0 + l (coalesced 256-byte row
// loads, 64-byte code stores); each thread issues the loads of 8 rows before
// it searches them, so several rows are in flight.  The column-major copy is
// transposed through LDS and written as BT_R-byte runs per feature.
// ---------------------------------------------------------------------------
constexpr int BT_F = kBinTileFeats, BT_R = kBinTileRows, BT_U = 8;
static_assert(BT_F == 64 && BT_R == 256, "lane = feature, thread = row of the transposed copy");

__global__ __launch_bounds__(256) void bin_matrix_kernel(
    const float* __restrict__ X, int64_t n, int32_t F, int64_t xs,
    const float* __restrict__ edges, int32_t n_edges, int8_t* __restrict__ codes_rm, int64_t S,
    int8_t* __restrict__ codes_cm) {
  extern __shared__ float sedge[];  // [BT_F][n_edges]
  __shared__ int8_t tcode[BT_F][BT_R + 4];
  const int64_t r0 = (int64_t)blockIdx.x * BT_R;
  const int f0 = blockIdx.y * BT_F;
  const int tid = threadIdx.x;
  for (int i = tid; i < BT_F * n_edges; i += blockDim.x) {
    const int fl = i / n_edges;
    const int f = f0 + fl;
    sedge[i] = f < F ? edges[(int64_t)f * n_edges + (i - fl * n_edges)] : 0.0f;
  }
  __syncthreads();
  const int fl = tid & 63;
  const int rq = tid >> 6;  // rows rq, rq + 4, ... of the tile
  const int f = f0 + fl;
  const float* e = sedge + fl * n_edges;
  const int8_t pad = (int8_t)(n_edges + 2);  // num_bins + 1
  for (int k0 = 0; k0 < BT_R; k0 += 4 * BT_U) {
    float v[BT_U];
#pragma unroll
    for (int u = 0; u < BT_U; ++u) {
      const int64_t r = r0 + k0 + rq + 4 * u;
      v[u] = (r < n && f < F) ? X[r * xs + f] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < BT_U; ++u) {
      const int k = k0 + rq + 4 * u;
      const int64_t r = r0 + k;
      const int8_t c = f < F ? (int8_t)count_le(e, n_edges, v[u]) : pad;
      tcode[fl][k] = c;
      if (r < n && f < S) codes_rm[r * S + f] = c;
    }
  }
  if (!codes_cm) return;  // uniform over the workgroup
  __syncthreads();
  // column-major: thread t writes row r0 + t of every feature of the tile
  const int64_t r = r0 + tid;
  if (r < n) {
    for (int k = 0; k < BT_F && f0 + k < F; ++k)
      codes_cm[(int64_t)(f0 + k) * n + r] = tcode[k][tid];
  }
}

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
  const int64_t r0 = (int64_t)blockIdx.x * BT_R;
  const int f0 = blockIdx.y * BT_F;
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
__device__ inline float key_to_float(uint32_t k) {
  const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// X [n, F] float32 (row stride xs) -> keys [F, n]; 64 x 64 tiles through LDS
__global__ __launch_bounds__(256) void transpose_keys_kernel(const float* __restrict__ X,
                                                             int64_t n, int32_t F, int64_t xs,
                                                             uint32_t* __restrict__ keys) {
  __shared__ uint32_t t[64][65];
  const int64_t r0 = (int64_t)blockIdx.x * 64;
  const int f0 = blockIdx.y * 64;
  const int c = threadIdx.x & 63;
  for (int k = threadIdx.x >> 6; k < 64; k += 4) {
    const int64_t r = r0 + k;
    t[k][c] = (r < n && f0 + c < F) ? float_to_key(X[r * xs + f0 + c]) : 0u;
  }
  __syncthreads();
  for (int k = threadIdx.x >> 6; k < 64; k += 4) {
    const int f = f0 + k;
    const int64_t r = r0 + c;
    if (f < F && r < n) keys[(int64_t)f * n + r] = t[c][k];
  }
}

constexpr int kSelThreads = 1024;
constexpr int kSelMaxTargets = 256;   // 2 * 126 ranks at most (num_bins <= 127)
constexpr int kSelGroup = 48;         // distinct prefixes histogrammed per column pass

__global__ __launch_bounds__(kSelThreads) void quantile_select_kernel(
    const uint32_t* __restrict__ keys, int64_t n, int32_t F, const float* __restrict__ q,
    int32_t nq, float* __restrict__ edges) {
  __shared__ uint32_t hist[kSelGroup][256];        // 48 KB
  __shared__ uint32_t tprefix[kSelMaxTargets];      // known key bits of each target
  __shared__ int64_t trank[kSelMaxTargets];         // rank still to find within the prefix
  __shared__ uint32_t dist[kSelMaxTargets];         // distinct prefixes of this pass (sorted)
  __shared__ int s_nd, s_nan;
  const int f = blockIdx.x;
  if (f >= F) return;
  const uint32_t* col = keys + (int64_t)f * n;
  const int nt = 2 * nq;
  const int64_t last = n - 1;
  for (int t = threadIdx.x; t < nt; t += kSelThreads) {
    const float rank = q[t >> 1] * (float)last;
    int64_t r = (t & 1) ? (int64_t)ceilf(rank) : (int64_t)rank;
    r = r < 0 ? 0 : (r > last ? last : r);
    trank[t] = r;
    tprefix[t] = 0;
  }
  if (threadIdx.x == 0) s_nan = 0;
  // pass 1: histogram of the top byte (per-wave copies in hist rows 0..15)
  for (int i = threadIdx.x; i < 16 * 256; i += kSelThreads) (&hist[0][0])[i] = 0;
  __syncthreads();
  {
    const int w = threadIdx.x >> 6;
    int nan_local = 0;
    for (int64_t i = threadIdx.x; i < n; i += kSelThreads) {
      const uint32_t k = col[i];
      nan_local += k == 0xffffffffu;
      atomicAdd(&hist[w][k >> 24], 1u);
    }
    if (nan_local) atomicAdd(&s_nan, nan_local);
  }
  __syncthreads();
  if (s_nan) {  // torch.quantile: a NaN anywhere makes every quantile NaN
    for (int j = threadIdx.x; j < nq; j += kSelThreads)
      edges[(int64_t)f * nq + j] = __builtin_nanf("");
    return;
  }
  for (int b = threadIdx.x; b < 256; b += kSelThreads) {
    uint32_t s = 0;
    for (int w = 0; w < 16; ++w) s += hist[w][b];
    hist[16][b] = s;
  }
  __syncthreads();
  for (int t = threadIdx.x; t < nt; t += kSelThreads) {
    int64_t r = trank[t];
    int b = 0;
    while (r >= (int64_t)hist[16][b]) r -= hist[16][b++];
    tprefix[t] = (uint32_t)b;
    trank[t] = r;
  }
  __syncthreads();
  // passes 2..4: next byte of the keys that share a target's prefix
  for (int pass = 1; pass < 4; ++pass) {
    const int sh = 32 - 8 * pass;  // prefix = key >> sh
    if (threadIdx.x == 0) {
      // sorted distinct prefixes (insertion sort of <= 252 values)
      int nd = 0;
      for (int t = 0; t < nt; ++t) {
        const uint32_t v = tprefix[t];
        int pos = nd;
        while (pos > 0 && dist[pos - 1] > v) --pos;
        if (pos > 0 && dist[pos - 1] == v) continue;
        for (int m = nd; m > pos; --m) dist[m] = dist[m - 1];
        dist[pos] = v;
        ++nd;
      }
      s_nd = nd;
    }
    __syncthreads();
    const int nd = s_nd;
    for (int g0 = 0; g0 < nd; g0 += kSelGroup) {
      const int gn = nd - g0 < kSelGroup ? nd - g0 : kSelGroup;
      for (int i = threadIdx.x; i < gn * 256; i += kSelThreads) (&hist[0][0])[i] = 0;
      __syncthreads();
      const uint32_t lo_p = dist[g0], hi_p = dist[g0 + gn - 1];
      for (int64_t i = threadIdx.x; i < n; i += kSelThreads) {
        const uint32_t k = col[i];
        const uint32_t pre = k >> sh;
        if (pre < lo_p || pre > hi_p) continue;
        int lo = g0, hi = g0 + gn - 1;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (dist[mid] < pre) lo = mid + 1; else hi = mid;
        }
        if (dist[lo] == pre) atomicAdd(&hist[lo - g0][(k >> (sh - 8)) & 255u], 1u);
      }
      __syncthreads();
      for (int t = threadIdx.x; t < nt; t += kSelThreads) {
        int lo = g0, hi = g0 + gn - 1;
        const uint32_t pre = tprefix[t];
        if (pre < dist[g0] || pre > dist[g0 + gn - 1]) continue;
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if (dist[mid] < pre) lo = mid + 1; else hi = mid;
        }
        int64_t r = trank[t];
        int b = 0;
        while (b < 255 && r >= (int64_t)hist[lo - g0][b]) r -= hist[lo - g0][b++];
        tprefix[t] = (pre << 8) | (uint32_t)b;
        trank[t] = r;
      }
      __syncthreads();
    }
  }
  // interpolate (torch.quantile, linear): see quantile_edges_kernel
  for (int j = threadIdx.x; j < nq; j += kSelThreads) {
    const float rank = q[j] * (float)last;
    const int64_t lo = (int64_t)rank;
    const float w = rank - (float)lo;
    const float a = key_to_float(tprefix[2 * j]);
    const float b = key_to_float(tprefix[2 * j + 1]);
    const float d = b - a;
    edges[(int64_t)f * nq + j] = w < 0.5f ? fmaf(w, d, a) : fmaf(w - 1.0f, d, b);
  }
}

}  // namespace wgbm
