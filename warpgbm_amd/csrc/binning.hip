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
// batched binner: X [n, F] row-major float32 (row stride xs floats) ->
//   codes_rm [n, S] int8 (S >= F; bytes F..S-1 set to -1) and, if non-null,
//   codes_cm [F, n] int8 (column-major, for the row partition).
// workgroup: 64 rows x 64 features; edges of its 64 features staged in LDS.
// ---------------------------------------------------------------------------
constexpr int BT_R = 64, BT_F = 64;

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
  // each thread: feature column fl = tid & 63, rows (tid >> 6) + 4k
  const int fl = tid & 63;
  const int f = f0 + fl;
  for (int k = tid >> 6; k < BT_R; k += 4) {
    const int64_t r = r0 + k;
    int8_t c = -1;
    if (r < n && f < F) {
      const float v = X[r * xs + f];
      c = (int8_t)count_le(sedge + fl * n_edges, n_edges, v);
    }
    tcode[fl][k] = c;
    if (r < n && f < S) codes_rm[r * S + f] = c;  // padding columns get -1
  }
  __syncthreads();
  if (codes_cm) {
    // column-major: thread writes rows (tid & 63) of features (tid >> 6) + 4k
    const int rl = tid & 63;
    const int64_t r = r0 + rl;
    for (int k = tid >> 6; k < BT_F; k += 4) {
      const int ff = f0 + k;
      if (r < n && ff < F) codes_cm[(int64_t)ff * n + r] = tcode[k][rl];
    }
  }
}

// padding bytes beyond the last 64-feature tile (S > round_up(F, 64))
__global__ void pad_codes_kernel(int8_t* __restrict__ codes_rm, int64_t n, int64_t S,
                                 int32_t from) {
  const int64_t w = S - from;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * w) return;
  const int64_t r = gid / w;
  codes_rm[r * S + from + (gid - r * w)] = (int8_t)-1;
}

// pre-binned int8 input [n, F] (row stride xs bytes) -> padded row-major + column-major
__global__ __launch_bounds__(256) void copy_prebinned_kernel(const int8_t* __restrict__ X,
                                                             int64_t n, int32_t F, int64_t xs,
                                                             int8_t* __restrict__ codes_rm,
                                                             int64_t S,
                                                             int8_t* __restrict__ codes_cm) {
  __shared__ int8_t tcode[BT_F][BT_R + 4];
  const int64_t r0 = (int64_t)blockIdx.x * BT_R;
  const int f0 = blockIdx.y * BT_F;
  const int tid = threadIdx.x;
  const int fl = tid & 63;
  const int f = f0 + fl;
  for (int k = tid >> 6; k < BT_R; k += 4) {
    const int64_t r = r0 + k;
    int8_t c = -1;
    if (r < n && f < F) c = X[r * xs + f];
    tcode[fl][k] = c;
    if (r < n && f < S) codes_rm[r * S + f] = c;
  }
  __syncthreads();
  if (codes_cm) {
    const int rl = tid & 63;
    const int64_t r = r0 + rl;
    for (int k = tid >> 6; k < BT_F; k += 4) {
      const int ff = f0 + k;
      if (r < n && ff < F) codes_cm[(int64_t)ff * n + r] = tcode[k][rl];
    }
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

}  // namespace wgbm
