// The per-feature split scan shared by the split kernels (split.hip) and the
// fused one-era split + leaf step (engine_kernels.hip).
#pragma once
#include <hip/hip_runtime.h>

namespace wgbm {

// A (node, era) segment of n rows where every candidate split has gain 0 and
// direction 0: HL >= mcw && HR >= mcw needs HL + HR >= 2*mcw, and HL + HR
// counts at most the n rows (exact small integers in float).
__device__ inline bool des_segment_dead(int64_t n, float mcw) {
  return (float)n < 2.0f * mcw;
}


struct ScanOut {
  float gain;
  float dir;
};

// sequential scan of one (era, feature) histogram; calls emit(b, gain, dir)
template <typename LoadG, typename LoadH, typename Emit>
__device__ inline void scan_bins(int B, float mcw, float eps, LoadG g, LoadH h, Emit emit) {
  float Gt = 0.0f, Ht = 0.0f;
#pragma unroll
  for (int b = 0; b < B; ++b) {
    Gt = Gt + g(b);
    Ht = Ht + h(b);
  }
  float GL = 0.0f, HL = 0.0f;
  const float tot = (Gt * Gt) / (Ht + eps);
#pragma unroll
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

// candidate order: the larger gain, then the smaller flat index
__device__ inline bool better(float g, int i, float bg, int bi) {
  return g > bg || (g == bg && i < bi);
}

}  // namespace wgbm
