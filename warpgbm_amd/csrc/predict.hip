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
#include "common.hpp"
#include "kernels.hpp"

namespace wgbm {

// reference table format, walk bounded by M steps (malformed tables cannot
// loop forever; a walk that leaves the table contributes NaN)
__global__ void predict_table_kernel(const int8_t* __restrict__ codes, int64_t n, int64_t F,
                                     const float* __restrict__ table, int64_t T, int64_t M,
                                     float lr, float* __restrict__ out) {
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
                                    float* __restrict__ out) {
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

}  // namespace wgbm
