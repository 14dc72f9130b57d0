// Split search: per-era gain / direction scan and Directional Era-Splitting
// (DES) selection.
//
// Per-era scan (warpgbm/cuda/best_split_kernel.cu:25-54), for one (era, feature):
//   Gt = sum_b G[b], Ht = sum_b H[b]                  (sequential, float32)
//   for b in 0 .. B-2 (sequential):
//     GL += G[b]; HL += H[b]; GR = Gt - GL; HR = Ht - HL
//     if HL >= mcw && HR >= mcw:
//        gain = GL^2/(HL+eps) + GR^2/(HR+eps) - Gt^2/(Ht+eps)
//        dir  = GL/(HL+eps) > GR/(HR+eps) ? +1 : -1
//     else gain = 0, dir = 0
// Every lane walks its bins in exactly this order with IEEE float32 ops (the
// library is compiled with -ffp-contract=off), so the gains are bit-identical
// to a sequential float32 evaluation of the same histogram.
//
// DES selection (warpgbm/core.py:577-594):
//   E == 1: crit = gain[0];  mask = crit > min_split_gain
//   E >  1: agree = |mean_e dir|, crit = mean_e gain,
//           mask = (agree == max over all (f, b) of agree) & (crit > min_split_gain)
//   no masked candidate -> leaf; else argmax of crit over masked candidates,
//   first flat index (f * (B-1) + b) on ties.
// Here agree is compared through the exact integer |sum_e dir| (E is common to
// all candidates), and crit = float(sum_e double(gain_e) / E) with the era sum
// taken sequentially in era order.
#include <float.h>
#include "common.hpp"
#include "kernels.hpp"

namespace wgbm {

struct ScanOut {
  float gain;
  float dir;
};

// sequential scan of one (era, feature) histogram; calls emit(b, gain, dir)
template <typename LoadG, typename LoadH, typename Emit>
__device__ inline void scan_bins(int B, float mcw, float eps, LoadG g, LoadH h, Emit emit) {
  float Gt = 0.0f, Ht = 0.0f;
  for (int b = 0; b < B; ++b) {
    Gt = Gt + g(b);
    Ht = Ht + h(b);
  }
  float GL = 0.0f, HL = 0.0f;
  const float tot = (Gt * Gt) / (Ht + eps);
  for (int b = 0; b < B - 1; ++b) {
    GL = GL + g(b);
    HL = HL + h(b);
    const float GR = Gt - GL;
    const float HR = Ht - HL;
    float gain = 0.0f, dir = 0.0f;
    if (HL >= mcw && HR >= mcw) {
      gain = (GL * GL) / (HL + eps) + (GR * GR) / (HR + eps) - tot;
      const float lv = GL / (HL + eps);
      const float rv = GR / (HR + eps);
      dir = lv > rv ? 1.0f : -1.0f;
    }
    emit(b, gain, dir);
  }
}

// ---------------------------------------------------------------------------
// reference-compatible compute_split: one lane per (era, feature)
// ---------------------------------------------------------------------------
__global__ void split_f32_kernel(const float* __restrict__ G, const float* __restrict__ H,
                                 int32_t E, int32_t F, int32_t B, float mcw, float eps,
                                 float* __restrict__ gain_out, float* __restrict__ dir_out) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)E * F) return;
  const float* g = G + gid * B;
  const float* h = H + gid * B;
  float* go = gain_out + gid * (B - 1);
  float* dout = dir_out + gid * (B - 1);
  scan_bins(
      B, mcw, eps, [&](int b) { return g[b]; }, [&](int b) { return h[b]; },
      [&](int b, float gn, float d) {
        go[b] = gn;
        dout[b] = d;
      });
}

// ---------------------------------------------------------------------------
// engine: E == 1, fused scan + selection.
//   hq/hc: [tree][node][F][B] exact sums; feat_sel: local -> global feature
// outputs per (tree, node): split_l (local feature or -1), split_b, best gain
// ---------------------------------------------------------------------------
__device__ inline bool better(float g, int i, float bg, int bi) {
  return g > bg || (g == bg && i < bi);
}

// order-preserving map of float bits to uint32 (and back)
__device__ inline uint32_t gain_key(float g) {
  const uint32_t u = __float_as_uint(g);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline float gain_from_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// One lane per (tree-node, local feature); the node's best candidate is kept
// as a packed key  gain_key(gain) << 32 | (0xffffffff - flat index)  updated
// with a 64-bit atomicMax, so the larger gain wins and, on equal gains, the
// smaller flat index (torch.argmax takes the first).  Integer atomics make
// the result independent of execution order.  best[tn] == 0: no split (every
// real key is nonzero: gain_key(-inf) = 0x007fffff).
__global__ __launch_bounds__(256) void split_level_e1_kernel(
    const int64_t* __restrict__ hq, const int32_t* __restrict__ hc, int32_t F, int32_t B,
    const int32_t* __restrict__ feat_sel, int32_t n_sel, int32_t nodes_in_level,
    const int32_t* __restrict__ present, const int32_t* __restrict__ shifts, float mcw,
    float eps, float min_split_gain, unsigned long long* __restrict__ best) {
  const int blocks_per_node = (n_sel + 255) / 256;
  const int tn = blockIdx.x / blocks_per_node;
  const int l = (blockIdx.x - tn * blocks_per_node) * 256 + threadIdx.x;
  if (!present[tn]) return;  // uniform per workgroup
  const int tree = tn / nodes_in_level;
  const int s = shifts[tree];
  float bg = -__builtin_inff();
  int bi = 0x7fffffff;
  if (l < n_sel) {
    const int f = feat_sel[l];
    const int64_t base = ((int64_t)tn * F + f) * B;
    const int64_t* q = hq + base;
    const int32_t* c = hc + base;
    scan_bins(
        B, mcw, eps, [&](int b) { return wgbm_dequantise(q[b], s); },
        [&](int b) { return (float)c[b]; },
        [&](int b, float gn, float d) {
          (void)d;
          const int idx = l * (B - 1) + b;
          if (gn > min_split_gain && better(gn, idx, bg, bi)) {
            bg = gn;
            bi = idx;
          }
        });
  }
  for (int o = 32; o > 0; o >>= 1) {
    const float og = __shfl_xor(bg, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (better(og, oi, bg, bi)) {
      bg = og;
      bi = oi;
    }
  }
  if ((threadIdx.x & 63) == 0 && bi != 0x7fffffff) {
    const unsigned long long key = ((unsigned long long)gain_key(bg) << 32) |
                                   (unsigned long long)(0xffffffffu - (uint32_t)bi);
    atomicMax(best + tn, key);
  }
}

// decode the packed best keys of a level into (local feature, bin, gain)
__global__ void split_decode_kernel(const unsigned long long* __restrict__ best, int32_t n_tn,
                                    int32_t B, int32_t* __restrict__ split_l,
                                    int32_t* __restrict__ split_b, float* __restrict__ split_gain) {
  const int tn = blockIdx.x * blockDim.x + threadIdx.x;
  if (tn >= n_tn) return;
  const unsigned long long k = best[tn];
  if (k == 0ull) {
    split_l[tn] = -1;
    split_b[tn] = -1;
    return;
  }
  const int idx = (int)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
  split_l[tn] = idx / (B - 1);
  split_b[tn] = idx % (B - 1);
  split_gain[tn] = gain_from_key((uint32_t)(k >> 32));
}

// ---------------------------------------------------------------------------
// engine: E > 1.  (1) per-era scan, one lane per (tree-node, era, local feature)
//   writes gain/dir into [tn][E][n_sel][B-1]
// ---------------------------------------------------------------------------
__global__ void split_level_scan_kernel(const int64_t* __restrict__ hq,
                                        const int32_t* __restrict__ hc, int32_t F, int32_t B,
                                        int32_t E, const int32_t* __restrict__ feat_sel,
                                        int32_t n_sel, int32_t nodes_in_level, int32_t n_tn,
                                        const int32_t* __restrict__ present,
                                        const int32_t* __restrict__ shifts, float mcw, float eps,
                                        float* __restrict__ gain, int8_t* __restrict__ dir) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)n_tn * E * n_sel;
  if (gid >= total) return;
  const int l = (int)(gid % n_sel);
  const int e = (int)((gid / n_sel) % E);
  const int tn = (int)(gid / ((int64_t)n_sel * E));
  if (!present[tn]) return;
  const int s = shifts[tn / nodes_in_level];
  const int f = feat_sel[l];
  const int64_t base = (((int64_t)tn * E + e) * F + f) * B;
  const int64_t* q = hq + base;
  const int32_t* c = hc + base;
  float* go = gain + gid * (B - 1);
  int8_t* dout = dir + gid * (B - 1);
  scan_bins(
      B, mcw, eps, [&](int b) { return wgbm_dequantise(q[b], s); },
      [&](int b) { return (float)c[b]; },
      [&](int b, float gn, float d) {
        go[b] = gn;
        dout[b] = (int8_t)d;
      });
}

// (2) DES selection, one workgroup per (tree, node)
__global__ __launch_bounds__(1024) void des_select_kernel(
    const float* __restrict__ gain, const int8_t* __restrict__ dir, int32_t B, int32_t E,
    int32_t n_sel, const int32_t* __restrict__ present, float min_split_gain,
    int32_t* __restrict__ split_l, int32_t* __restrict__ split_b,
    float* __restrict__ split_gain_era /* [tn][E] */) {
  const int tn = blockIdx.x;
  if (!present[tn]) {
    if (threadIdx.x == 0) {
      split_l[tn] = -1;
      split_b[tn] = -1;
    }
    return;
  }
  const int nb = B - 1;
  const int64_t ncand = (int64_t)n_sel * nb;
  const float* g0 = gain + (int64_t)tn * E * ncand;
  const int8_t* d0 = dir + (int64_t)tn * E * ncand;
  __shared__ int red_i[16];
  __shared__ float red_g[16];
  __shared__ int s_max_agree;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, nw = blockDim.x >> 6;

  // pass 1: max over all candidates of |sum_e dir|
  int amax = 0;
  for (int64_t c = threadIdx.x; c < ncand; c += blockDim.x) {
    int ds = 0;
    for (int e = 0; e < E; ++e) ds += d0[(int64_t)e * ncand + c];
    ds = ds < 0 ? -ds : ds;
    amax = ds > amax ? ds : amax;
  }
  for (int o = 32; o > 0; o >>= 1) {
    const int y = __shfl_xor(amax, o, 64);
    amax = y > amax ? y : amax;
  }
  if (lane == 0) red_i[w] = amax;
  __syncthreads();
  if (threadIdx.x == 0) {
    int m = 0;
    for (int k = 0; k < nw; ++k) m = red_i[k] > m ? red_i[k] : m;
    s_max_agree = m;
  }
  __syncthreads();
  const int max_agree = s_max_agree;
  __syncthreads();

  // pass 2: argmax of crit over candidates with agree == max and crit > msg
  float bg = -__builtin_inff();
  int bi = 0x7fffffff;
  for (int64_t c = threadIdx.x; c < ncand; c += blockDim.x) {
    int ds = 0;
    for (int e = 0; e < E; ++e) ds += d0[(int64_t)e * ncand + c];
    ds = ds < 0 ? -ds : ds;
    if (ds != max_agree) continue;
    double acc = 0.0;
    for (int e = 0; e < E; ++e) acc += (double)g0[(int64_t)e * ncand + c];
    const float crit = (float)(acc / (double)E);
    if (crit > min_split_gain && better(crit, (int)c, bg, bi)) {
      bg = crit;
      bi = (int)c;
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
  if (lane == 0) {
    red_g[w] = bg;
    red_i[w] = bi;
  }
  __syncthreads();
  __shared__ int s_best;
  if (threadIdx.x == 0) {
    for (int k = 1; k < nw; ++k)
      if (better(red_g[k], red_i[k], bg, bi)) {
        bg = red_g[k];
        bi = red_i[k];
      }
    s_best = bi;
    if (bi == 0x7fffffff) {
      split_l[tn] = -1;
      split_b[tn] = -1;
    } else {
      split_l[tn] = bi / nb;
      split_b[tn] = bi % nb;
    }
  }
  __syncthreads();
  const int best = s_best;
  if (best != 0x7fffffff)
    for (int e = threadIdx.x; e < E; e += blockDim.x)
      split_gain_era[(int64_t)tn * E + e] = g0[(int64_t)e * ncand + best];
}

}  // namespace wgbm
