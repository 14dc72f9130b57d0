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

#include <algorithm>
#include "common.hpp"
#include "kernels.hpp"
#include "split_scan.hpp"

namespace wgbm {

// ---------------------------------------------------------------------------
// reference-compatible compute_split: one lane per (era, feature)
// ---------------------------------------------------------------------------
// BT > 0: B known at compile time, and every bin of the thread's (era,
// feature) is loaded before the scan (one memory round trip; with the bin
// count known only at run time the scan's sequential sums wait for each
// bin's load in turn)
template <int BT>
__global__ __launch_bounds__(256) void split_f32_kernel(const float* __restrict__ G,
                                                        const float* __restrict__ H, int32_t E,
                                                        int32_t F, int32_t B_rt, float mcw,
                                                        float eps, float* __restrict__ gain_out,
                                                        float* __restrict__ dir_out) {
  const int B = BT > 0 ? BT : B_rt;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)E * F) return;
  const float* g = G + gid * B;
  const float* h = H + gid * B;
  float* go = gain_out + gid * (B - 1);
  float* dout = dir_out + gid * (B - 1);
  auto emit = [&](int b, float gn, float d) {
    go[b] = gn;
    dout[b] = d;
  };
  if constexpr (BT > 0) {
    float gv[BT], hv[BT];
#pragma unroll
    for (int b = 0; b < BT; ++b) {
      gv[b] = g[b];
      hv[b] = h[b];
    }
    scan_bins(
        BT, mcw, eps, [&](int b) { return gv[b]; }, [&](int b) { return hv[b]; }, emit);
  } else {
    scan_bins(
        B, mcw, eps, [&](int b) { return g[b]; }, [&](int b) { return h[b]; }, emit);
  }
}

int launch_split_f32(const float* G, const float* H, int32_t E, int32_t F, int32_t B, float mcw,
                     float eps, float* gain_out, float* dir_out, hipStream_t st) {
  const int64_t n = (int64_t)E * F;
  const dim3 grid((unsigned)((n + 255) / 256)), blk(256);
#define WGBM_SPLIT_F32(BT)                                                                    \
  case BT:                                                                                    \
    hipLaunchKernelGGL(split_f32_kernel<BT>, grid, blk, 0, st, G, H, E, F, B, mcw, eps,        \
                       gain_out, dir_out);                                                    \
    break;
  switch (B) {
    WGBM_SPLIT_F32(2)
    WGBM_SPLIT_F32(3)
    WGBM_SPLIT_F32(4)
    WGBM_SPLIT_F32(5)
    WGBM_SPLIT_F32(6)
    WGBM_SPLIT_F32(7)
    WGBM_SPLIT_F32(8)
    WGBM_SPLIT_F32(10)
    WGBM_SPLIT_F32(16)
    WGBM_SPLIT_F32(32)
    WGBM_SPLIT_F32(64)
    default:
      hipLaunchKernelGGL(split_f32_kernel<0>, grid, blk, 0, st, G, H, E, F, B, mcw, eps,
                         gain_out, dir_out);
  }
#undef WGBM_SPLIT_F32
  WGBM_LAUNCH_CHECK();
  return 0;
}

// ---------------------------------------------------------------------------
// engine: E == 1, fused scan + selection.
//   hq/hc: [tree][node][F][B] exact sums; feat_sel: local -> global feature
// outputs per (tree, node): split_l (local feature or -1), split_b, best gain
// ---------------------------------------------------------------------------

// One lane per (tree-node, local feature); the node's best candidate is kept
// as a packed key  gain_key(gain) << 32 | (0xffffffff - flat index)  updated
// with a 64-bit atomicMax, so the larger gain wins and, on equal gains, the
// smaller flat index (torch.argmax takes the first).  Integer atomics make
// the result independent of execution order.  best[tn] == 0: no split (every
// real key is nonzero: gain_key(-inf) = 0x007fffff).
// BT > 0: B known at compile time, and every bin of the lane's histogram is
// loaded before the scan (one round trip instead of one per bin)
template <int BT>
__global__ __launch_bounds__(256) void split_level_e1_kernel(
    const int64_t* __restrict__ hq, const int32_t* __restrict__ hc, int32_t F, int32_t B_rt,
    const int32_t* __restrict__ feat_sel, int32_t n_sel, int32_t nodes_in_level,
    const int32_t* __restrict__ present, const int32_t* __restrict__ node_shift, float mcw,
    float eps, float min_split_gain, unsigned long long* __restrict__ best) {
  const int B = BT > 0 ? BT : B_rt;
  const int blocks_per_node = (n_sel + 255) / 256;
  const int tn = blockIdx.x / blocks_per_node;
  const int l = (blockIdx.x - tn * blocks_per_node) * 256 + threadIdx.x;
  if (!present[tn]) return;  // uniform per workgroup
  const int s = node_shift[tn];
  float bg = -__builtin_inff();
  int bi = 0x7fffffff;
  if (l < n_sel) {
    const int f = feat_sel[l];
    const int64_t base = ((int64_t)tn * F + f) * B;
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
  if ((threadIdx.x & 63) == 0 && bi != 0x7fffffff) {
    const unsigned long long key = ((unsigned long long)gain_key(bg) << 32) |
                                   (unsigned long long)(0xffffffffu - (uint32_t)bi);
    atomicMax(best + tn, key);
  }
}


// ---------------------------------------------------------------------------
// engine: E > 1, without per-era gain/direction arrays.
//  (1) des_accumulate: one lane per (tree-node, local feature, chunk of up to
//      kDesChunk split bins) walks the eras in order and keeps, per candidate,
//      sum_e double(gain_e) and sum_e dir_e (the per-era values are exactly
//      those of the sequential scan above).  Writes crit = float(sum / E) and
//      agree = |sum dir| per candidate and the node's max agree (atomicMax).
//  (2) des_pick: among candidates with agree == max agree and crit >
//      min_split_gain, the largest crit (first flat index on ties), through a
//      packed 64-bit atomicMax key as in the E == 1 path.
//  (3) des_finish: decodes the pick and recomputes the chosen split's per-era
//      gains for the tree record.
// ---------------------------------------------------------------------------
// wave-level max into *dst when the wave's active lanes share one target;
// otherwise one atomic per lane
__device__ inline void atomic_max_grouped_i32(int32_t* base, int key, bool active, int v) {
  const int k0 = __builtin_amdgcn_readfirstlane(key);
  const bool uniform = __all(!active || key == k0);
  if (uniform) {
    int m = active ? v : -1;
    for (int o = 32; o > 0; o >>= 1) {
      const int y = __shfl_xor(m, o, 64);
      m = y > m ? y : m;
    }
    if ((threadIdx.x & 63) == 0 && m >= 0) atomicMax(base + k0, m);
  } else if (active) {
    atomicMax(base + key, v);
  }
}

__device__ inline void atomic_max_grouped_u64(unsigned long long* base, int key, bool active,
                                              unsigned long long v) {
  const int k0 = __builtin_amdgcn_readfirstlane(key);
  const bool uniform = __all(!active || key == k0);
  if (uniform) {
    unsigned long long m = active ? v : 0ull;
    for (int o = 32; o > 0; o >>= 1) {
      const unsigned long long y = __shfl_xor(m, o, 64);
      m = y > m ? y : m;
    }
    if ((threadIdx.x & 63) == 0 && m != 0ull) atomicMax(base + k0, m);
  } else if (active) {
    atomicMax(base + key, v);
  }
}

__global__ __launch_bounds__(128) void des_accumulate_kernel(
    const int64_t* __restrict__ hq, const int32_t* __restrict__ hc, int32_t F, int32_t B,
    int32_t E, const int32_t* __restrict__ feat_sel, int32_t n_sel, int32_t nodes_in_level,
    int32_t n_tn, const int32_t* __restrict__ present, const int32_t* __restrict__ key_shift,
    float mcw, float eps, float* __restrict__ crit, int32_t* __restrict__ agree,
    int32_t* __restrict__ agree_max) {
  const int nb = B - 1;
  const int nch = (nb + kDesChunk - 1) / kDesChunk;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t total = (int64_t)n_tn * n_sel * nch;
  int tn = 0, l = 0, ch = 0;
  bool active = gid < total;
  if (active) {
    ch = (int)(gid % nch);
    l = (int)((gid / nch) % n_sel);
    tn = (int)(gid / ((int64_t)nch * n_sel));
    active = present[tn] != 0;
  }
  int amax = 0;
  if (active) {
    const int f = feat_sel[l];
    const int b0 = ch * kDesChunk;
    double gs[kDesChunk];
    int ds[kDesChunk];
#pragma unroll
    for (int k = 0; k < kDesChunk; ++k) {
      gs[k] = 0.0;
      ds[k] = 0;
    }
    double bs[kDesChunk];  // current era block's sums
#pragma unroll
    for (int k = 0; k < kDesChunk; ++k) bs[k] = 0.0;
    for (int e = 0; e < E; ++e) {
      const int s = key_shift[(int64_t)tn * E + e];  // the (node, era) segment's shift
      const int64_t base = (((int64_t)tn * E + e) * F + f) * B;
      const int64_t* q = hq + base;
      const int32_t* c = hc + base;
      // the float operations of scan_bins, in the same order
      float Gt = 0.0f, Ht = 0.0f;
      for (int b = 0; b < B; ++b) {
        Gt = Gt + wgbm_dequantise(q[b], s);
        Ht = Ht + (float)c[b];
      }
      const float tot = (Gt * Gt) / (Ht + eps);
      float GL = 0.0f, HL = 0.0f;
      for (int b = 0; b < b0; ++b) {
        GL = GL + wgbm_dequantise(q[b], s);
        HL = HL + (float)c[b];
      }
#pragma unroll
      for (int k = 0; k < kDesChunk; ++k) {
        const int b = b0 + k;
        if (b < nb) {
          GL = GL + wgbm_dequantise(q[b], s);
          HL = HL + (float)c[b];
          const float GR = Gt - GL;
          const float HR = Ht - HL;
          float gain = 0.0f;
          int dir = 0;
          if (HL >= mcw && HR >= mcw) {
            gain = (GL * GL) / (HL + eps) + (GR * GR) / (HR + eps) - tot;
            const float lv = GL / (HL + eps);
            const float rv = GR / (HR + eps);
            dir = lv > rv ? 1 : -1;
          }
          bs[k] += (double)gain;  // era order inside the block
          ds[k] += dir;
        }
      }
      if ((e + 1) % kDesEraBlock == 0 || e + 1 == E) {
#pragma unroll
        for (int k = 0; k < kDesChunk; ++k) {
          gs[k] += bs[k];  // block order
          bs[k] = 0.0;
        }
      }
    }
    const int64_t ncand = (int64_t)n_sel * nb;
#pragma unroll
    for (int k = 0; k < kDesChunk; ++k) {
      const int b = b0 + k;
      if (b < nb) {
        const int64_t o = (int64_t)tn * ncand + (int64_t)l * nb + b;
        crit[o] = (float)(gs[k] / (double)E);
        const int a = ds[k] < 0 ? -ds[k] : ds[k];
        agree[o] = a;
        amax = a > amax ? a : amax;
      }
    }
  }
  atomic_max_grouped_i32(agree_max, tn, active, amax);
}

__global__ __launch_bounds__(256) void des_pick_kernel(
    const float* __restrict__ crit, const int32_t* __restrict__ agree,
    const int32_t* __restrict__ agree_max, const int32_t* __restrict__ present, int32_t n_tn,
    int64_t ncand, float min_split_gain, unsigned long long* __restrict__ best) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  int tn = 0;
  bool ok = gid < (int64_t)n_tn * ncand;
  unsigned long long key = 0ull;
  if (ok) {
    tn = (int)(gid / ncand);
    const int cand = (int)(gid - (int64_t)tn * ncand);
    const float cr = crit[gid];
    ok = present[tn] && agree[gid] == agree_max[tn] && cr > min_split_gain;
    if (ok)
      key = ((unsigned long long)gain_key(cr) << 32) |
            (unsigned long long)(0xffffffffu - (uint32_t)cand);
  }
  atomic_max_grouped_u64(best, tn, ok, key);
}

// one lane per (tree-node, era): split_l / split_b from the pick and the
// chosen split's gain in every era (record gain [tn][E])
__global__ void des_finish_kernel(const unsigned long long* __restrict__ best,
                                  const int64_t* __restrict__ hq, const int32_t* __restrict__ hc,
                                  int32_t F, int32_t B, int32_t E,
                                  const int32_t* __restrict__ feat_sel, int32_t nodes_in_level,
                                  int32_t n_tn, const int32_t* __restrict__ key_shift,
                                  float mcw, float eps, const float* __restrict__ staged,
                                  const int64_t* __restrict__ seg, int32_t n_sel,
                                  int32_t* __restrict__ split_l, int32_t* __restrict__ split_b,
                                  float* __restrict__ split_gain_era) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)n_tn * E) return;
  const int tn = (int)(gid / E);
  const int e = (int)(gid - (int64_t)tn * E);
  const unsigned long long k = best[tn];
  if (k == 0ull) {
    if (e == 0) {
      split_l[tn] = -1;
      split_b[tn] = -1;
    }
    return;
  }
  const int nb = B - 1;
  const int idx = (int)(0xffffffffu - (uint32_t)(k & 0xffffffffull));
  const int l = idx / nb, bsel = idx - (idx / nb) * nb;
  if (e == 0) {
    split_l[tn] = l;
    split_b[tn] = bsel;
  }
  if (staged) {
    // staged per-era gains [tn][E][n_sel][B-1]; none for dead segments
    const int64_t k2 = (int64_t)tn * E + e;
    const int W = (E + kDesEraBlock - 1) / kDesEraBlock;
    split_gain_era[gid] =
        des_segment_dead(seg[k2 + 1] - seg[k2], mcw)
            ? 0.0f
            : staged[des_stage_slot(tn, e, W, ((int64_t)n_sel * nb + 63) / 64, idx)];
    return;
  }
  const int s = key_shift[gid];  // the (node, era) segment's shift
  const int64_t base = (((int64_t)tn * E + e) * F + feat_sel[l]) * B;
  const int64_t* q = hq + base;
  const int32_t* c = hc + base;
  float g_sel = 0.0f;
  scan_bins(
      B, mcw, eps, [&](int b) { return wgbm_dequantise(q[b], s); },
      [&](int b) { return (float)c[b]; },
      [&](int b, float gn, float d) {
        (void)d;
        if (b == bsel) g_sel = gn;
      });
  split_gain_era[gid] = g_sel;
}

// ---------------------------------------------------------------------------
// engine: E > 1 when every (node, era) segment fits one tile (<= 65536 rows):
// per-era gains straight from an LDS histogram, without materialising the
// per-era histograms.
//   des_era: one workgroup per (tree-node, era, chunk of 64*V features) builds
//     the segment's histogram in LDS (packed q * 2^18 + 1 words, lane-owned
//     columns as in the tile histogram) and writes every candidate's gain and
//     direction for that era: staged gain / dir [tn][E][n_sel][B-1].
//   des_combine: crit / agree per candidate from the staged values, the era
//     sum in double in era order (same values and order as des_accumulate).
// ---------------------------------------------------------------------------
constexpr int kDesEraThreads = 256;
constexpr int kDesEraMaxWG = 8192;  // era kernels grid bound (32 workgroups per CU; 4096 and 16384 measured slower)

template <int V, int BT>
__global__ __launch_bounds__(kDesEraThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
void des_era_kernel(
    const int8_t* __restrict__ codes, int64_t stride, int32_t F,
    const float* __restrict__ rpos, const int32_t* __restrict__ key_shift,
    const int32_t* __restrict__ order,
    const int64_t* __restrict__ seg, int32_t E, int32_t n_keys, int32_t nodes_in_level,
    const int32_t* __restrict__ present, const int32_t* __restrict__ local_of, int32_t n_sel,
    int32_t num_bins_rt, float mcw, float eps, float* __restrict__ gain,
    int8_t* __restrict__ dir) {
  extern __shared__ unsigned long long lds[];
  constexpr int CW = kHistSlots * V;
  constexpr int nwaves = kDesEraThreads / 64;
  const int B = BT > 0 ? BT : num_bins_rt;
  const int Bp = B + 1;
  const int nb = B - 1;
  const int n_chunks = (F + CW - 1) / CW;
  const int W = (E + kDesEraBlock - 1) / kDesEraBlock;  // era blocks (staging layout)
  const int slots = gridDim.x / n_chunks;  // workgroups per chunk; keys stride by it
  const int slot = blockIdx.x / n_chunks;
  const int chunk = blockIdx.x - slot * n_chunks;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int f_base = chunk * CW + lane * V;
  // lanes past the last feature re-read the last real feature's bytes (a line
  // the wave fetches anyway); their words are never evaluated
  const int voff = f_base < F ? f_base : (F - 1) / V * V;
  unsigned long long* my = lds + lane;

  // keys slot, slot + slots, ...: every wave classifies 64 of them at a time
  // (one per lane) and the workgroup visits the live ones in order.  A key
  // is skipped when its node is absent or the segment is dead (fewer than
  // 2*min_child_weight rows: no candidate can split it, so every candidate
  // has gain 0 and direction 0 there; des_combine and des_finish account for
  // it without staged values).
  for (int kb = slot; kb < n_keys; kb += 64 * slots) {
    const int kl = kb + lane * slots;
    bool live = false;
    if (kl < n_keys) {
      const int tnl = kl / E;
      live = present[tnl] && !des_segment_dead(seg[kl + 1] - seg[kl], mcw);
    }
    uint64_t todo = __ballot(live);
    while (todo) {
      const int l0 = __builtin_ctzll(todo);
      todo &= todo - 1;
      const int key = kb + l0 * slots;
      const int64_t begin = seg[key];
      const int n = (int)(seg[key + 1] - begin);  // <= 65536 (checked by the engine)
      const int s = key_shift[key];                // the segment's own shift
      for (int i = threadIdx.x; i < V * Bp * kHistSlots; i += kDesEraThreads) lds[i] = 0ull;
      __syncthreads();
      // software pipeline as in the tile histogram: wave w takes the row
      // groups [i, i + U), i = (w + k*nwaves)*U; two register sets alternate
      // so that the loads of the next group are in flight while this one is
      // added; row ids and residuals (stored by position) are vector loads
      // (lane u < U: row u of the group) broadcast with readlane; positions past the end read the
      // segment's last row and add the word 0
      constexpr int U = 8;
      constexpr int step = nwaves * U;
      const int ul = lane & (U - 1);
      struct Group {
        uint32_t c[U];
        float r;
      };
      Group ga, gb;
      int32_t ids = 0;  // lane u < U: order entry u of the next group to issue
      auto load_ids = [&](int i0) { ids = order[begin + (i0 + ul < n ? i0 + ul : n - 1)]; };
      auto issue = [&](Group& g, int i0) {
        int rows[U];
#pragma unroll
        for (int u = 0; u < U; ++u) rows[u] = __builtin_amdgcn_readlane(ids, u);
        g.r = rpos[begin + (i0 + ul < n ? i0 + ul : n - 1)];
        load_ids(i0 + step);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int8_t* src = codes + (int64_t)rows[u] * stride + voff;
          if constexpr (V == 4)
            g.c[u] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(src));
          else if constexpr (V == 2)
            g.c[u] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(src));
          else
            g.c[u] = __builtin_nontemporal_load(reinterpret_cast<const uint8_t*>(src));
        }
      };
      auto add = [&](const Group& g, int i0) {
        const int64_t qv = (int64_t)wgbm_quantise(g.r, s);
        const uint64_t pv = (uint64_t)(qv * (int64_t)(1 << WGBM_CBITS) + 1);
        const uint32_t plo = (uint32_t)pv, phi = (uint32_t)(pv >> 32);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          // readlane returns int: widen through uint32_t (no sign extension)
          const uint64_t wu = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(phi, u) << 32) |
                              (uint64_t)(uint32_t)__builtin_amdgcn_readlane(plo, u);
          const unsigned long long w = i0 + u < n ? (unsigned long long)wu : 0ull;
#pragma unroll
          for (int j = 0; j < V; ++j) {
            uint32_t c = (g.c[u] >> (8 * j)) & 0xffu;
            c = c < (uint32_t)B ? c : (uint32_t)B;  // out-of-range code -> trash bin
            atomicAdd(my + (j * Bp + (int)c) * kHistSlots, w);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      int i = wave * U;
      if (i < n) {
        load_ids(i);
        issue(ga, i);
        while (i + 2 * step < n) {
          issue(gb, i + step);
          add(ga, i);
          issue(ga, i + 2 * step);
          add(gb, i + step);
          i += 2 * step;
        }
        if (i + step < n) {
          issue(gb, i + step);
          add(ga, i);
          add(gb, i + step);
        } else {
          add(ga, i);
        }
      }
      __syncthreads();

      // candidates of this era: thread per feature of the chunk
      for (int fs = threadIdx.x; fs < CW; fs += kDesEraThreads) {
        const int f = chunk * CW + fs;
        if (f >= F) continue;
        const int l = local_of[f];
        if (l < 0) continue;
        const unsigned long long* col = lds + (fs % V) * Bp * kHistSlots + fs / V;
        const int64_t c64 = ((int64_t)n_sel * nb + 63) / 64;
        const int tnk = key / E, ek = key - (key / E) * E;
        scan_bins(
            B, mcw, eps,
            [&](int b) { return wgbm_dequantise((int64_t)col[b * kHistSlots] >> WGBM_CBITS, s); },
            [&](int b) {
              return (float)(int32_t)(col[b * kHistSlots] & (unsigned long long)WGBM_CMASK);
            },
            [&](int b, float gn, float d) {
              const int64_t o = des_stage_slot(tnk, ek, W, c64, (int64_t)l * nb + b);
              gain[o] = gn;
              dir[o] = (int8_t)d;
            });
      }
      __syncthreads();  // before the next key's histogram reuses the LDS
    }
  }
}

// ---------------------------------------------------------------------------
// des_pair: the direct era path for num_bins <= 7 on pair codes, for levels
// whose (node, era) segments are large (the engine picks it by the mean
// segment size; see kDesPairMinRows).
//   Pair codes (made once per engine by pack_pairs_kernel): byte k of a row
//   is c(2k) * (B+1) + c(2k+1) for the features 2k, 2k+1, each code clamped
//   to the trash bin B (a code >= B or negative, and the padding past the
//   last feature); a row of F features takes ceil(F/2) bytes.
//   LDS: per lane (lane-owned columns as in the tile histogram) one
//   (B+1) x (B+1) table per feature pair, indexed by the pair code, so a row
//   costs one LDS add per pair of features instead of one per feature.  A
//   feature's column is its table summed over the partner's codes (all B+1,
//   the trash bin included): the same packed words as a one-feature
//   histogram, since packed words add exactly.
//   A lane covers 2 pairs (4 features, one 16-bit load per row); the
//   workgroup's 64 lanes cover a chunk of 256 features.  Code loads are
//   buffer loads with the row offset in a scalar register (the engine keeps
//   the copy under 4 GiB), so a row costs no vector address arithmetic.
// Outputs and key order as des_era_kernel (staged gain / dir per (key,
// local feature, bin)).  Each key's scan clears the table words it read, so
// the next key starts from zero without a pass of its own.
// The tables (36 KB at B = 5) allow 4 workgroups per CU: per row of a
// small segment fewer bytes are in flight than with the int8 codes' 12 KB
// tables, which is why deep levels keep des_era_kernel.
// ---------------------------------------------------------------------------
constexpr int kDesPairThreads = 512;
constexpr int kDesPairLanePairs = 2;                                 // pairs per lane
constexpr int kDesPairChunk = kHistSlots * 2 * kDesPairLanePairs;  // features per workgroup

template <int BT>
__global__ __launch_bounds__(kDesPairThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
void des_pair_kernel(
    const uint8_t* __restrict__ pcodes, uint32_t pbytes, uint32_t pstride, int32_t F,
    const float* __restrict__ rpos, const int32_t* __restrict__ key_shift,
    const int32_t* __restrict__ order, const int64_t* __restrict__ seg, int32_t E,
    int32_t n_keys, int32_t nodes_in_level, const int32_t* __restrict__ present,
    const int32_t* __restrict__ local_of, int32_t n_sel, float mcw, float eps,
    float* __restrict__ gain, int8_t* __restrict__ dir) {
  static_assert(BT >= 2 && BT <= 7, "pair tables: num_bins in [2, 7]");
  constexpr int Bp = BT + 1, P = Bp * Bp;
  constexpr int LP = kDesPairLanePairs;
  constexpr int CW = kDesPairChunk;
  constexpr int nwaves = kDesPairThreads / 64;
  constexpr int U = 16;  // rows per group
  constexpr int step = nwaves * U;
  constexpr int nb = BT - 1;
  extern __shared__ unsigned long long lds[];
  const int n_chunks = (F + CW - 1) / CW;
  const int W = (E + kDesEraBlock - 1) / kDesEraBlock;  // era blocks (staging layout)
  const int slots = gridDim.x / n_chunks;
  const int slot = blockIdx.x / n_chunks;
  const int chunk = blockIdx.x - slot * n_chunks;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ul = lane & (U - 1);
  const int f_base = chunk * CW + lane * 2 * LP;
  // lanes past the last feature re-read the last real pair word; their
  // words are never evaluated
  const uint32_t voff = (uint32_t)((f_base < F ? f_base : (F - 1) / (2 * LP) * (2 * LP)) / 2);
  // raw buffer over the whole copy: stride 0, pbytes records (loads past
  // them return 0), word 3 = 0x00020000 (DATA_FORMAT 32-bit: untyped buffer
  // loads need a nonzero data format on gfx9-family targets)
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc((void*)pcodes, (short)0, (int)pbytes, 0x00020000);
  // byte address of this lane's word 0 of pair table 0: lane * 8
  const uint32_t lbase = (uint32_t)lane * 8u;

  for (int i = threadIdx.x; i < LP * P * kHistSlots; i += kDesPairThreads) lds[i] = 0ull;
  __syncthreads();

  for (int kb = slot; kb < n_keys; kb += 64 * slots) {
    const int kl = kb + lane * slots;
    bool live = false;
    if (kl < n_keys) live = present[kl / E] && !des_segment_dead(seg[kl + 1] - seg[kl], mcw);
    uint64_t todo = __ballot(live);
    while (todo) {
      const int l0 = __builtin_ctzll(todo);
      todo &= todo - 1;
      const int key = kb + l0 * slots;
      const int64_t begin = seg[key];
      const int n = (int)(seg[key + 1] - begin);  // <= 65536 (checked by the engine)
      const int s = key_shift[key];  // the segment's own shift

      // rows: wave w takes groups [i, i + U), i = (w + k*nwaves)*U; lane
      // u < U loads row u's id and residual; two register sets alternate so
      // that the next group's loads are in flight while one is added;
      // positions past the end read the segment's last row and add the word 0
      struct Group {
        uint32_t c[U];
        int32_t q;  // lane u < U: quantised residual of row u
      };
      int32_t ids = 0;
      auto load_ids = [&](int i0) { ids = order[begin + (i0 + ul < n ? i0 + ul : n - 1)]; };
      auto issue = [&](Group& g, int i0) {
        uint32_t rows[U];
#pragma unroll
        for (int u = 0; u < U; ++u) rows[u] = (uint32_t)__builtin_amdgcn_readlane(ids, u);
        g.q = wgbm_quantise(rpos[begin + (i0 + ul < n ? i0 + ul : n - 1)], s);
        load_ids(i0 + step);
#pragma unroll
        for (int u = 0; u < U; ++u)
          g.c[u] = __builtin_amdgcn_raw_buffer_load_b16(rsrc, voff, rows[u] * pstride, 0);
      };
      auto add = [&](const Group& g, int i0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int64_t qr = __builtin_amdgcn_readlane(g.q, u);
          const unsigned long long w =
              i0 + u < n ? (unsigned long long)(qr * (int64_t)(1 << WGBM_CBITS) + 1) : 0ull;
#pragma unroll
          for (int p = 0; p < LP; ++p) {
            // the pair code is at most P - 1 already (pack_pairs_kernel clamps
            // each code): for the low byte the min lets the byte select be one
            // SDWA instruction, the top byte of the 16-bit load is one byte
            // permute; either way one more instruction adds shift and lane
            static_assert(LP == 2, "one 16-bit code load per row and lane");
            const uint32_t idx = p == 0 ? min(g.c[u] & 0xffu, (uint32_t)(P - 1))
                                        : __builtin_amdgcn_perm(0u, g.c[u], 0x0c0c0c01u);
            const uint32_t addr = (idx << 9) + lbase + (uint32_t)(p * P * kHistSlots * 8);
            atomicAdd(
                reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(lds) + addr), w);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      };
      Group ga, gb;
      int i = wave * U;
      if (i < n) {
        load_ids(i);
        issue(ga, i);
        while (i + 2 * step < n) {
          issue(gb, i + step);
          add(ga, i);
          issue(ga, i + 2 * step);
          add(gb, i + step);
          i += 2 * step;
        }
        if (i + step < n) {
          issue(gb, i + step);
          add(ga, i);
          add(gb, i + step);
        } else {
          add(ga, i);
        }
      }
      __syncthreads();

      // thread per feature pair: one sweep of the pair's table, row by row,
      // clears it and gives the columns of its first feature (row sums,
      // stored back at word (a, 0) of row a < B) and second feature (column
      // sums, stored in the trash row: word (B, b)); both are scanned from
      // there and cleared
      for (int pi = threadIdx.x; pi < CW / 2; pi += kDesPairThreads) {
        const int pl = pi / LP, p = pi % LP;  // lane, pair of the lane
        unsigned long long* t = lds + p * P * kHistSlots + pl;
        unsigned long long c1[BT];
#pragma unroll
        for (int b = 0; b < BT; ++b) c1[b] = 0ull;
#pragma unroll
        for (int a = 0; a < Bp; ++a) {
          unsigned long long row = 0ull;
#pragma unroll
          for (int b = 0; b < Bp; ++b) {
            const unsigned long long w = t[(a * Bp + b) * kHistSlots];
            row += w;
            if (b < BT) c1[b] += w;
            t[(a * Bp + b) * kHistSlots] = 0ull;
          }
          if (a < BT) t[a * Bp * kHistSlots] = row;
          __builtin_amdgcn_sched_barrier(0);  // one row of words live at a time
        }
#pragma unroll
        for (int b = 0; b < BT; ++b) t[(BT * Bp + b) * kHistSlots] = c1[b];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          // column word b of the feature: h = 0 at (b, 0), h = 1 at (B, b)
          unsigned long long* col = t + (h ? BT * Bp * kHistSlots : 0);
          const int cs = (h ? 1 : Bp) * kHistSlots;
          const int f = chunk * CW + pl * 2 * LP + 2 * p + h;
          const int l = f < F ? local_of[f] : -1;
          if (l >= 0) {
            const int64_t c64 = ((int64_t)n_sel * nb + 63) / 64;
            const int tnk = key / E, ek = key - (key / E) * E;
            scan_bins(
                BT, mcw, eps,
                [&](int b) { return wgbm_dequantise((int64_t)col[b * cs] >> WGBM_CBITS, s); },
                [&](int b) {
                  return (float)(int32_t)(col[b * cs] & (unsigned long long)WGBM_CMASK);
                },
                [&](int b, float gn, float d) {
                  const int64_t o = des_stage_slot(tnk, ek, W, c64, (int64_t)l * nb + b);
                  gain[o] = gn;
                  dir[o] = (int8_t)d;
                });
          }
#pragma unroll
          for (int b = 0; b < BT; ++b) col[b * cs] = 0ull;
        }
      }
      __syncthreads();  // the table is zero again for the next key
    }
  }
}

// pair codes for des_pair (num_bins <= 7): thread per (row, 4 output bytes
// = 8 features); byte k of a row = c(2k) * (B+1) + c(2k+1), each code
// clamped to B (a code >= B or negative, and the padding past the last
// feature)
__global__ void pack_pairs_kernel(const int8_t* __restrict__ codes, int64_t stride, int32_t F,
                                  int64_t n, int32_t B, uint8_t* __restrict__ out,
                                  int64_t pstride) {
  const int64_t wpr = pstride / 4;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= n * wpr) return;
  const int64_t row = gid / wpr;
  const int w = (int)(gid - row * wpr);
  const int f0 = w * 8;
  const int8_t* src = codes + row * stride;
  // one 8-byte load where the row holds all 8 (stride % 16 == 0, f0 % 8 == 0)
  uint64_t v = 0;
  if (f0 + 8 <= stride) {
    v = *reinterpret_cast<const uint64_t*>(src + f0);
  } else {
    for (int j = 0; j < 8 && f0 + j < stride; ++j) v |= (uint64_t)(uint8_t)src[f0 + j] << (8 * j);
  }
  uint32_t word = 0;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    uint32_t c[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int j = 2 * k + h;
      uint32_t x = f0 + j < F ? (uint32_t)(v >> (8 * j)) & 0xffu : (uint32_t)B;
      c[h] = x < (uint32_t)B ? x : (uint32_t)B;
    }
    word |= (c[0] * (uint32_t)(B + 1) + c[1]) << (8 * k);
  }
  reinterpret_cast<uint32_t*>(out + row * pstride)[w] = word;
}

// live-era bit masks: bit (e % 32) of alive[tn * W + e / 32] is set when the
// (tn, era e) segment can hold a split (not des_segment_dead); W = ceil(E/32)
// (one mask word per era block)
__global__ void des_alive_kernel(const int64_t* __restrict__ seg, int32_t E, int32_t n_tn,
                                 float mcw, uint32_t* __restrict__ alive) {
  static_assert(kDesEraBlock == 32, "one 32-bit mask word per era block");
  const int W = (E + kDesEraBlock - 1) / kDesEraBlock;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)n_tn * W) return;
  const int tn = (int)(gid / W);
  const int w = (int)(gid - (int64_t)tn * W);
  const int64_t* sg = seg + (int64_t)tn * E;
  // the block's 33 segment offsets, loaded unconditionally (indices clamped
  // to the node's E + 1 offsets) so that the loads are issued together
  int64_t o[kDesEraBlock + 1];
#pragma unroll
  for (int b = 0; b <= kDesEraBlock; ++b) {
    const int e = w * kDesEraBlock + b;
    o[b] = sg[e < E ? e : E];
  }
  uint32_t m = 0;
#pragma unroll
  for (int b = 0; b < kDesEraBlock; ++b) {
    const int e = w * kDesEraBlock + b;
    if (e < E && !des_segment_dead(o[b + 1] - o[b], mcw)) m |= 1u << b;
  }
  alive[gid] = m;
}

// Era sums in the DES order: float64, each block of kDesEraBlock consecutive
// eras summed in era order (des_block_kernel, one lane per (node, block,
// candidate)), then the block sums in block order (des_combine_pick_kernel,
// one lane per (node, candidate)).  Dead segments add gain 0 and direction 0
// (acc + 0.0 == acc exactly): their staged values are never read, and a block
// without a live era is skipped.
__global__ __launch_bounds__(256) void des_block_kernel(
    const float* __restrict__ gain, const int8_t* __restrict__ dir, int32_t E, int32_t n_tn,
    int64_t ncand, const int32_t* __restrict__ present, const uint32_t* __restrict__ alive,
    double* __restrict__ bsum, int8_t* __restrict__ bdir) {
  const int W = (E + kDesEraBlock - 1) / kDesEraBlock;
  const int64_t c64 = (ncand + 63) / 64;
  // thread per (tree-node, block, candidate) with the candidates padded to
  // whole groups of 64: every wave is one (tree-node, block, 64-group)
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (gid >= (int64_t)n_tn * W * c64 * 64) return;  // whole waves
  const int64_t tb = gid / (c64 * 64);  // tn * W + block
  const int64_t c = gid - tb * (c64 * 64);
  const int tn = (int)(tb / W);
  const int blk = (int)(tb - (int64_t)tn * W);
  if (!present[tn]) return;  // wave-uniform
  const uint32_t m = alive[tb];
  if (m == 0) return;
  // this block's 32 eras of the candidate: slots base + 64 * k (block-major
  // staging layout).  The loads go through raw buffer descriptors over the
  // candidate's 64-group of the block (32 x 64 slots): a dead era's load
  // gets an offset past the descriptor's size, which returns 0 without a
  // memory access, so no load is a branch (a predicated load would become a
  // branch with a wait after every load) and dead eras cost no bytes.
  // the wave's 64 candidates are one group (c % 64 == lane): its slot base
  // is wave-uniform (stated to the compiler, which the descriptor needs)
  const int tnu = __builtin_amdgcn_readfirstlane(tn);
  const int blku = __builtin_amdgcn_readfirstlane(blk);
  const int64_t cw = (int64_t)__builtin_amdgcn_readfirstlane((int)(c - c % 64));
  const int64_t g0 = des_stage_slot(tnu, blku * kDesEraBlock, W, c64, cw);
  const uint32_t cl = (uint32_t)(c % 64);
  const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(gain + g0), (short)0, (int)(kDesEraBlock * 64 * sizeof(float)), 0x00020000);
  const __amdgpu_buffer_rsrc_t rd = __builtin_amdgcn_make_buffer_rsrc(
      (void*)(dir + g0), (short)0, (int)(kDesEraBlock * 64), 0x00020000);
  constexpr uint32_t kPast = 0x80000000u;  // beyond either descriptor
  double acc = 0.0;
  int ds = 0;
  constexpr int kHalf = kDesEraBlock / 2;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    float gv[kHalf];
    int dv[kHalf];
#pragma unroll
    for (int k = 0; k < kHalf; ++k) {
      const int kk = h * kHalf + k;
      const bool live = (m >> kk) & 1u;  // implies the era exists
      const uint32_t slot = (uint32_t)kk * 64u + cl;
      gv[k] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(rg, live ? slot * 4u : kPast, 0, 0));
      dv[k] = (int)(int8_t)__builtin_amdgcn_raw_buffer_load_b8(rd, live ? slot : kPast, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // the half's loads are all issued before its adds
#pragma unroll
    for (int k = 0; k < kHalf; ++k) {
      if ((m >> (h * kHalf + k)) & 1u) {  // a live era (it exists)
        acc += (double)gv[k];  // era order
        ds += dv[k];
      }
    }
  }
  if (c < ncand) {  // padding lanes of the last group store nothing
    bsum[tb * ncand + c] = acc;
    bdir[tb * ncand + c] = (int8_t)ds;  // |ds| <= 32: the eras of one block
  }
}

// The block sums, the pick and the record in one launch (the staged era
// path).  bpn = ceil(ncand / 256) workgroups per (tree-node); each thread
// combines its candidate's block sums in block order (crit = float(sum /
// E), agree = |sum of directions|), and each workgroup leaves a summary:
// its largest agreement a_w and, among its candidates with agree == a_w and
// crit > min_split_gain, the packed key of the largest crit (first flat
// index on ties; gain_key(crit) << 32 | ~index, 0 if none).  The node's
// pick is then the largest key among the workgroups whose a_w is the node's
// largest agreement: a candidate qualifies only with agree == max agree,
// and a workgroup holding one has a_w == max agree.  The last workgroup of
// the node to arrive (done[tn], a release fence before the count, an
// acquire fence after; no workgroup waits for another) reads the bpn
// summaries, stores the pick to best[tn], resets done[tn], and writes
// split_l / split_b and the chosen split's staged gain of every era (0 for
// a dead segment), as des_finish_kernel.
__global__ __launch_bounds__(256) void des_combine_pick_kernel(
    const double* __restrict__ bsum, const int8_t* __restrict__ bdir, int32_t E, int32_t n_tn,
    int64_t ncand, const int32_t* __restrict__ present, const uint32_t* __restrict__ alive,
    float min_split_gain, int32_t* __restrict__ wg_agree, unsigned long long* __restrict__ wg_key,
    unsigned long long* __restrict__ best, uint32_t* __restrict__ done,
    const float* __restrict__ staged, const int64_t* __restrict__ seg, float mcw, int32_t nb,
    int32_t n_sel, int32_t* __restrict__ split_l, int32_t* __restrict__ split_b,
    float* __restrict__ split_gain_era) {
  __shared__ int s_a[4];
  __shared__ unsigned long long s_k[4];
  __shared__ int s_last;
  const int W = (E + kDesEraBlock - 1) / kDesEraBlock;
  const int bpn = (int)((ncand + 255) / 256);
  const int tn = blockIdx.x / bpn;
  const int wg = blockIdx.x - tn * bpn;
  const int64_t c = (int64_t)wg * 256 + threadIdx.x;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (!present[tn]) {  // uniform: the node is absent (no split, as des_finish_kernel)
    if (c == 0) {
      split_l[tn] = -1;
      split_b[tn] = -1;
    }
    return;
  }
  const uint32_t* al = alive + (int64_t)tn * W;
  int a = -1;
  float cr = 0.0f;
  if (c < ncand) {
    double acc = 0.0;
    int ds = 0;
    // blocks in groups of 8, the group's loads issued together (a block
    // without a live era was never written: its words are loaded and not
    // added)
    constexpr int G = 8;
    for (int b0 = 0; b0 < W; b0 += G) {
      // a group whose blocks are all dead is skipped (the alive words are
      // the same for the whole workgroup: a uniform branch)
      uint32_t any = 0u;
#pragma unroll
      for (int k = 0; k < G; ++k) any |= b0 + k < W ? al[b0 + k] : 0u;
      if (any == 0u) continue;
      double v[G];
      int dv[G];
#pragma unroll
      for (int k = 0; k < G; ++k) {
        const int bk = b0 + k < W ? b0 + k : W - 1;
        const int64_t o = ((int64_t)tn * W + bk) * ncand + c;
        v[k] = bsum[o];
        dv[k] = (int)bdir[o];
      }
#pragma unroll
      for (int k = 0; k < G; ++k) {
        if (b0 + k < W && al[b0 + k] != 0u) {
          acc += v[k];  // block order
          ds += dv[k];
        }
      }
    }
    cr = (float)(acc / (double)E);
    a = ds < 0 ? -ds : ds;
  }
  // the workgroup's largest agreement
  int am = a;
  for (int off = 32; off > 0; off >>= 1) {
    const int y = __shfl_xor(am, off, 64);
    am = y > am ? y : am;
  }
  if (lane == 0) s_a[w] = am;
  __syncthreads();
  am = s_a[0];
  for (int i = 1; i < 4; ++i) am = s_a[i] > am ? s_a[i] : am;
  // its best candidate at that agreement
  unsigned long long key = 0ull;
  if (c < ncand && a == am && cr > min_split_gain)
    key = ((unsigned long long)gain_key(cr) << 32) |
          (unsigned long long)(0xffffffffu - (uint32_t)c);
  for (int off = 32; off > 0; off >>= 1) {
    const unsigned long long y = __shfl_xor(key, off, 64);
    key = y > key ? y : key;
  }
  if (lane == 0) s_k[w] = key;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long k = s_k[0];
    for (int i = 1; i < 4; ++i) k = s_k[i] > k ? s_k[i] : k;
    const int64_t slot = (int64_t)tn * bpn + wg;
    wg_agree[slot] = am;
    wg_key[slot] = k;
    __threadfence();  // the summary is visible before the arrival is counted
    const uint32_t prev = atomicAdd(done + tn, 1u);
    const bool last = prev == (uint32_t)(bpn - 1);
    if (last) {
      __threadfence();  // every other workgroup's summary is visible
      done[tn] = 0u;    // ready for the next level
    }
    s_last = last ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;  // uniform
  // the node's pick from the bpn summaries (one wave)
  if (w == 0) {
    int ma = -1;
    unsigned long long mk = 0ull;
    for (int i = lane; i < bpn; i += 64) {
      const int ai = __hip_atomic_load(wg_agree + (int64_t)tn * bpn + i, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
      const unsigned long long ki = __hip_atomic_load(wg_key + (int64_t)tn * bpn + i,
                                                      __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (ai > ma) {
        ma = ai;
        mk = ki;
      } else if (ai == ma) {
        mk = ki > mk ? ki : mk;
      }
    }
    for (int off = 32; off > 0; off >>= 1) {
      const int ya = __shfl_xor(ma, off, 64);
      const unsigned long long yk = __shfl_xor(mk, off, 64);
      if (ya > ma) {
        ma = ya;
        mk = yk;
      } else if (ya == ma) {
        mk = yk > mk ? yk : mk;
      }
    }
    if (lane == 0) s_k[0] = mk;
  }
  __syncthreads();
  const unsigned long long pick = s_k[0];
  if (threadIdx.x == 0) best[tn] = pick;
  if (pick == 0ull) {
    if (threadIdx.x == 0) {
      split_l[tn] = -1;
      split_b[tn] = -1;
    }
    return;
  }
  const int idx = (int)(0xffffffffu - (uint32_t)(pick & 0xffffffffull));
  if (threadIdx.x == 0) {
    split_l[tn] = idx / nb;
    split_b[tn] = idx - (idx / nb) * nb;
  }
  // the chosen split's per-era gains (record gain [tn][E]) from the staged
  // values; none for dead segments
  const int64_t c64 = ((int64_t)n_sel * nb + 63) / 64;
  for (int e = threadIdx.x; e < E; e += 256) {
    const int64_t k2 = (int64_t)tn * E + e;
    split_gain_era[k2] = des_segment_dead(seg[k2 + 1] - seg[k2], mcw)
                             ? 0.0f
                             : staged[des_stage_slot(tn, e, W, c64, idx)];
  }
}

// local index of every feature of the round's subset (local_of is -1 elsewhere)
__global__ void local_scatter_kernel(const int32_t* __restrict__ feat_sel, int32_t n_sel,
                                     int32_t F, int32_t* __restrict__ local_of) {
  const int l = blockIdx.x * blockDim.x + threadIdx.x;
  if (l < n_sel) {
    const int f = feat_sel[l];
    if (f >= 0 && f < F) local_of[f] = l;
  }
}

int launch_split_level_e1(int n_tn, hipStream_t st, const int64_t* hq, const int32_t* hc,
                          int32_t F, int32_t B, const int32_t* feat_sel, int32_t n_sel,
                          int32_t nodes_in_level, const int32_t* present,
                          const int32_t* node_shift, float mcw, float eps, float min_split_gain,
                          unsigned long long* best) {
  const dim3 grid((unsigned)(n_tn * ((n_sel + 255) / 256)));
  if (B == 32)
    hipLaunchKernelGGL(split_level_e1_kernel<32>, grid, dim3(256), 0, st, hq, hc, F, B, feat_sel,
                       n_sel, nodes_in_level, present, node_shift, mcw, eps, min_split_gain,
                       best);
  else
    hipLaunchKernelGGL(split_level_e1_kernel<0>, grid, dim3(256), 0, st, hq, hc, F, B, feat_sel,
                       n_sel, nodes_in_level, present, node_shift, mcw, eps, min_split_gain,
                       best);
  WGBM_LAUNCH_CHECK();
  return 0;
}

int launch_des_era(int V, int B, int32_t n_keys, hipStream_t st, const int8_t* codes,
                   int64_t stride, int32_t F, const float* rpos, const int32_t* key_shift,
                   const int32_t* order, const int64_t* seg, int32_t E, int32_t nodes_in_level,
                   const int32_t* present, const int32_t* local_of, int32_t n_sel, float mcw,
                   float eps, float* gain, int8_t* dir, const uint8_t* pcodes, int64_t n_rows,
                   int64_t pstride) {
  if (pcodes) {
    WGBM_REQUIRE(B >= 2 && B <= 7, "launch_des_era: pair codes need num_bins in [2, 7]");
    WGBM_REQUIRE(pstride > 0 && pstride % 8 == 0 && pstride * 2 >= ((F + 15) / 16) * 16,
                 "launch_des_era: bad pair stride %lld", (long long)pstride);
    WGBM_REQUIRE(n_rows * pstride <= (int64_t)0xffffffffll,
                 "launch_des_era: pair codes must stay under 4 GiB");
    const size_t lds = (size_t)kDesPairLanePairs * (B + 1) * (B + 1) * kHistSlots * 8;
    const int n_chunks = (F + kDesPairChunk - 1) / kDesPairChunk;
    const int slots = std::max(1, std::min(n_keys, kDesEraMaxWG / n_chunks));
    const dim3 grid((unsigned)(slots * n_chunks));
    const uint32_t pbytes = (uint32_t)(n_rows * pstride);
#define WGBM_DES_PAIR(BB)                                                                      \
  do {                                                                                         \
    static bool attr = false;                                                                  \
    if (!attr) {                                                                               \
      WGBM_CHECK(hipFuncSetAttribute((const void*)des_pair_kernel<BB>,                          \
                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024)); \
      attr = true;                                                                             \
    }                                                                                          \
    hipLaunchKernelGGL((des_pair_kernel<BB>), grid, dim3(kDesPairThreads), lds, st, pcodes,    \
                       pbytes, (uint32_t)pstride, F, rpos, key_shift, order, seg, E, n_keys,   \
                       nodes_in_level, present, local_of, n_sel, mcw, eps, gain, dir);         \
    WGBM_LAUNCH_CHECK();                                                                       \
    return 0;                                                                                  \
  } while (0)
    switch (B) {
      case 2: WGBM_DES_PAIR(2);
      case 3: WGBM_DES_PAIR(3);
      case 4: WGBM_DES_PAIR(4);
      case 5: WGBM_DES_PAIR(5);
      case 6: WGBM_DES_PAIR(6);
      default: WGBM_DES_PAIR(7);
    }
#undef WGBM_DES_PAIR
  }
  const size_t lds = (size_t)V * (B + 1) * kHistSlots * 8;
  // at most kDesEraMaxWG workgroups; each strides over the keys of its chunk
  const int n_chunks = (F + kHistSlots * V - 1) / (kHistSlots * V);
  const int slots = std::max(1, std::min(n_keys, kDesEraMaxWG / n_chunks));
  const dim3 grid((unsigned)(slots * n_chunks));
#define WGBM_DES_ERA(VV, BB)                                                                   \
  do {                                                                                         \
    static bool attr = false;                                                                  \
    if (!attr) {                                                                               \
      WGBM_CHECK(hipFuncSetAttribute((const void*)des_era_kernel<VV, BB>,                       \
                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024)); \
      attr = true;                                                                             \
    }                                                                                          \
    hipLaunchKernelGGL((des_era_kernel<VV, BB>), grid, dim3(kDesEraThreads), lds, st, codes,   \
                       stride, F, rpos, key_shift, order, seg, E, n_keys,                     \
                       nodes_in_level, present, local_of, n_sel, B, mcw, eps, gain, dir);      \
    WGBM_LAUNCH_CHECK();                                                                       \
    return 0;                                                                                  \
  } while (0)
  if (V == 4 && B == 5) WGBM_DES_ERA(4, 5);
  if (V == 4) WGBM_DES_ERA(4, 0);
  if (V == 2) WGBM_DES_ERA(2, 0);
  if (V == 1) WGBM_DES_ERA(1, 0);
#undef WGBM_DES_ERA
  wgbm_set_error("launch_des_era: bad V=%d", V);
  return WGBM_EINVAL;
}

int launch_pack_pairs(hipStream_t st, const int8_t* codes, int64_t stride, int32_t F, int64_t n,
                      int32_t B, uint8_t* out, int64_t pstride) {
  WGBM_REQUIRE(B >= 2 && B <= 7, "pack_pairs: num_bins must be in [2, 7]");
  WGBM_REQUIRE(pstride > 0 && pstride % 8 == 0 && pstride * 2 >= ((F + 15) / 16) * 16,
               "pack_pairs: bad pair stride %lld", (long long)pstride);
  const int64_t threads = n * (pstride / 4);
  hipLaunchKernelGGL(pack_pairs_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, st,
                     codes, stride, F, n, B, out, pstride);
  WGBM_LAUNCH_CHECK();
  return 0;
}

}  // namespace wgbm
