// Shared device/host helpers for the warpgbm_amd HIP kernels (gfx950 / CDNA4).
//
// Arithmetic conventions used by every kernel in this library:
//
// * Histogram sums are EXACT.  A residual r (f32) is quantised once per call
//   (or once per tree in the engine) to an integer q = rint(r * 2^s), where the
//   shift s is chosen from M = max|r| so that |q| <= 2^qbits (qbits <= 28).
//   Because multiplying by a power of two is exact, q carries every bit of r
//   for |r| >= M/16.  Integer sums are associative, so the histogram is
//   independent of the order in which rows are visited (no float atomics).
//   A float sum is produced once, by rounding the exact integer sum:
//       G = (float) ldexp((double) Q, -s)         (|Q| < 2^53, so exact in double)
// * Row counts are exact integers (the reference's "hess" histogram is a row
//   count: histogram_kernel.cu:44 adds 1.0f per row).
// * Inside a workgroup the (q, 1) pair is packed into ONE 64-bit LDS word,
//       P = q * 2^WGBM_CBITS + 1,
//   so a single ds_add_u64 updates both the gradient sum and the count.
//   With at most WGBM_MAX_TILE_ROWS rows per tile the count field never
//   carries into the sum field and the sum never overflows.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define WGBM_CBITS 18
#define WGBM_CMASK ((1ll << WGBM_CBITS) - 1)
#define WGBM_QBITS_MAX 28
#define WGBM_MAX_TILE_ROWS 65536

// 3rd dword of a raw buffer resource descriptor for gfx9-family parts
// (DATA_FORMAT = 32-bit, untyped raw access).
#define WGBM_RSRC_DW3 0x00020000

#define WGBM_CHECK(expr)                                                        \
  do {                                                                          \
    hipError_t _e = (expr);                                                     \
    if (_e != hipSuccess) {                                                     \
      wgbm_set_error("%s:%d: %s -> %s", __FILE__, __LINE__, #expr,              \
                     hipGetErrorString(_e));                                    \
      return (int)_e;                                                           \
    }                                                                           \
  } while (0)

#define WGBM_REQUIRE(cond, ...)                                                 \
  do {                                                                          \
    if (!(cond)) {                                                              \
      wgbm_set_error(__VA_ARGS__);                                              \
      return WGBM_EINVAL;                                                       \
    }                                                                           \
  } while (0)

#define WGBM_LAUNCH_CHECK()                                                     \
  do {                                                                          \
    hipError_t _e = hipGetLastError();                                          \
    if (_e != hipSuccess) {                                                     \
      wgbm_set_error("%s:%d: kernel launch failed: %s", __FILE__, __LINE__,     \
                     hipGetErrorString(_e));                                    \
      return (int)_e;                                                           \
    }                                                                           \
  } while (0)

#ifndef WGBM_EINVAL
#define WGBM_EINVAL 1000
#define WGBM_ENOMEM 1001
#endif

void wgbm_set_error(const char* fmt, ...);

// ---------------------------------------------------------------------------
// quantisation helpers (bit-identical on host and device: only exact ops)
// ---------------------------------------------------------------------------
__host__ __device__ inline int wgbm_shift_from_absmax(float m, int qbits) {
  if (!(m > 0.0f)) return 0;           // all-zero residual: q == 0 for every row
  int e;
  frexpf(m, &e);                       // m = f * 2^e, f in [0.5, 1)  =>  m < 2^e
  return qbits - e;
}

// the shift of a maximum given as float bits: 0 for a non-finite one (a NaN
// or infinite residual; the caller reports it)
__host__ __device__ inline int wgbm_shift_from_bits(uint32_t absmax_bits, int qbits) {
  if (absmax_bits >= 0x7f800000u) return 0;
  float m;
  __builtin_memcpy(&m, &absmax_bits, sizeof m);
  return wgbm_shift_from_absmax(m, qbits);
}

__host__ __device__ inline int32_t wgbm_quantise(float r, int s) {
  return (int32_t)rintf(ldexpf(r, s));
}

__host__ __device__ inline float wgbm_dequantise(int64_t q, int s) {
  return (float)ldexp((double)q, -s);
}

// qbits for a problem with up to n rows: keeps |sum q| < 2^53 so that the
// int64 -> double step of wgbm_dequantise is exact.
__host__ inline int wgbm_qbits_for_rows(int64_t n) {
  int bl = 0;
  while ((int64_t(1) << bl) <= n && bl < 62) ++bl;   // bit length of n
  int q = 52 - bl;
  return q < WGBM_QBITS_MAX ? (q < 8 ? 8 : q) : WGBM_QBITS_MAX;
}

// ---------------------------------------------------------------------------
// device helpers
// ---------------------------------------------------------------------------
__device__ inline __amdgpu_buffer_rsrc_t wgbm_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0,
                                           (int)bytes, WGBM_RSRC_DW3);
}

// A 64-bit word in LDS addressed by an integer byte offset (address space 3).
typedef __attribute__((address_space(3))) unsigned long long wgbm_lds_u64;

// Lane u (0..15) of every row of 16 lanes, broadcast to the whole row (DPP
// row_newbcast): with the same value in lanes u, u+16, u+32, u+48 this is a
// wave-wide broadcast of that value in one VALU instruction.  u must be a
// constant after unrolling.
__device__ __forceinline__ unsigned long long wgbm_row_bcast(unsigned long long v, int u) {
  switch (u) {
#define WGBM_BC(k) \
  case k:          \
    return __builtin_amdgcn_mov_dpp(v, 0x150 + k, 0xf, 0xf, false);
    WGBM_BC(0) WGBM_BC(1) WGBM_BC(2) WGBM_BC(3) WGBM_BC(4) WGBM_BC(5) WGBM_BC(6) WGBM_BC(7)
    WGBM_BC(8) WGBM_BC(9) WGBM_BC(10) WGBM_BC(11) WGBM_BC(12) WGBM_BC(13) WGBM_BC(14) WGBM_BC(15)
#undef WGBM_BC
    default:
      return v;
  }
}

// Wave-wide reductions on DPP moves (VALU; no LDS crossbar traffic): a
// Hillis-Steele scan inside each row of 16 lanes (row_shr 1, 2, 4, 8; lanes
// with no source read 0), then the rows combined with row_bcast:15 (rows 1
// and 3) and row_bcast:31 (rows 2 and 3).  Lane 63 then holds the reduction
// over the wave; it is read out as a wave-uniform value.  0 is the identity
// (sums, and maxima of unsigned values).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ uint32_t wgbm_dpp_u32(uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROWMASK, 0xf, true);
}

__device__ __forceinline__ uint32_t wgbm_wave_reduce_max_u32(uint32_t x) {
#define WGBM_MAXSTEP(C, M)              \
  {                                     \
    const uint32_t y = wgbm_dpp_u32<C, M>(x); \
    x = y > x ? y : x;                  \
  }
  WGBM_MAXSTEP(0x111, 0xf)
  WGBM_MAXSTEP(0x112, 0xf)
  WGBM_MAXSTEP(0x114, 0xf)
  WGBM_MAXSTEP(0x118, 0xf)
  WGBM_MAXSTEP(0x142, 0xa)
  WGBM_MAXSTEP(0x143, 0xc)
#undef WGBM_MAXSTEP
  return (uint32_t)__builtin_amdgcn_readlane((int)x, 63);
}

__device__ __forceinline__ int64_t wgbm_wave_reduce_add_i64(int64_t x) {
#define WGBM_ADDSTEP(C, M)                                                     \
  {                                                                            \
    const uint32_t lo = wgbm_dpp_u32<C, M>((uint32_t)(uint64_t)x);             \
    const uint32_t hi = wgbm_dpp_u32<C, M>((uint32_t)((uint64_t)x >> 32));     \
    x += (int64_t)(((uint64_t)hi << 32) | lo);                                 \
  }
  WGBM_ADDSTEP(0x111, 0xf)
  WGBM_ADDSTEP(0x112, 0xf)
  WGBM_ADDSTEP(0x114, 0xf)
  WGBM_ADDSTEP(0x118, 0xf)
  WGBM_ADDSTEP(0x142, 0xa)
  WGBM_ADDSTEP(0x143, 0xc)
#undef WGBM_ADDSTEP
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)x, 63);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)x >> 32), 63);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// One DPP step of a 64-bit sum: x + (x of the source lane, 0 where none).
template <int CTRL, int ROWMASK>
__device__ __forceinline__ int64_t wgbm_dpp_add_i64(int64_t x) {
  const uint32_t lo = wgbm_dpp_u32<CTRL, ROWMASK>((uint32_t)(uint64_t)x);
  const uint32_t hi = wgbm_dpp_u32<CTRL, ROWMASK>((uint32_t)((uint64_t)x >> 32));
  return x + (int64_t)(((uint64_t)hi << 32) | lo);
}

// Workgroup barrier that orders LDS accesses only: global stores issued
// before it need not have completed (__syncthreads waits for them, a memory
// round trip).  Use it where the threads exchange data through LDS alone.
__device__ __forceinline__ void wgbm_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// A 64-bit value of one lane (lane wave-uniform).
__device__ __forceinline__ int64_t wgbm_readlane_i64(int64_t x, int lane) {
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)x, lane);
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)x >> 32), lane);
  return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Inclusive prefix sum inside each row of 16 lanes (lane 16 r + i: lanes
// 16 r .. 16 r + i).
__device__ __forceinline__ int64_t wgbm_row_incl_scan_i64(int64_t x) {
  x = wgbm_dpp_add_i64<0x111, 0xf>(x);
  x = wgbm_dpp_add_i64<0x112, 0xf>(x);
  x = wgbm_dpp_add_i64<0x114, 0xf>(x);
  x = wgbm_dpp_add_i64<0x118, 0xf>(x);
  return x;
}

// Segmented inclusive maxima over the lanes: (f, a, b) triples, f set where
// a run opens, combined as (f1, a1, b1) . (f2, a2, b2) = (f1 | f2, f2 ? a2 :
// max(a1, a2), f2 ? b2 : max(b1, b2)); a lane with no source reads (0, 0, 0),
// the identity.  The row steps alone scan each row of 16 lanes.
template <int CTRL, int ROWMASK>
__device__ __forceinline__ void wgbm_dpp_segmax_step(uint32_t& f, uint32_t& a, uint32_t& b) {
  const uint32_t yf = wgbm_dpp_u32<CTRL, ROWMASK>(f);
  const uint32_t ya = wgbm_dpp_u32<CTRL, ROWMASK>(a);
  const uint32_t yb = wgbm_dpp_u32<CTRL, ROWMASK>(b);
  if (!f) {
    a = ya > a ? ya : a;
    b = yb > b ? yb : b;
  }
  f |= yf;
}
__device__ __forceinline__ void wgbm_row_segmax_scan(uint32_t& f, uint32_t& a, uint32_t& b) {
  wgbm_dpp_segmax_step<0x111, 0xf>(f, a, b);
  wgbm_dpp_segmax_step<0x112, 0xf>(f, a, b);
  wgbm_dpp_segmax_step<0x114, 0xf>(f, a, b);
  wgbm_dpp_segmax_step<0x118, 0xf>(f, a, b);
}
__device__ __forceinline__ void wgbm_wave_segmax_scan(uint32_t& f, uint32_t& a, uint32_t& b) {
  wgbm_row_segmax_scan(f, a, b);
  wgbm_dpp_segmax_step<0x142, 0xa>(f, a, b);
  wgbm_dpp_segmax_step<0x143, 0xc>(f, a, b);
}

// Inclusive prefix sum over the wave's lanes (lane i: lanes 0..i), the same
// DPP sequence without the read-out.
__device__ __forceinline__ int64_t wgbm_wave_incl_scan_i64(int64_t x) {
#define WGBM_SCANSTEP(C, M)                                                    \
  {                                                                            \
    const uint32_t lo = wgbm_dpp_u32<C, M>((uint32_t)(uint64_t)x);             \
    const uint32_t hi = wgbm_dpp_u32<C, M>((uint32_t)((uint64_t)x >> 32));     \
    x += (int64_t)(((uint64_t)hi << 32) | lo);                                 \
  }
  WGBM_SCANSTEP(0x111, 0xf)
  WGBM_SCANSTEP(0x112, 0xf)
  WGBM_SCANSTEP(0x114, 0xf)
  WGBM_SCANSTEP(0x118, 0xf)
  WGBM_SCANSTEP(0x142, 0xa)
  WGBM_SCANSTEP(0x143, 0xc)
#undef WGBM_SCANSTEP
  return x;
}

// Work order that keeps neighbouring work items on one XCD.  The hardware
// deals consecutive workgroup ids round-robin over the 8 XCDs, each with its
// own L2; work item w = (id % 8) * per + id / 8 (per = ceil(n_work / 8))
// gives every XCD a contiguous run of work items, so tiles that share cache
// lines (the feature tiles of one row block) run on the same L2 at about the
// same time.  Launch wgbm_xcd_grid(n_work) workgroups; ids whose work item
// is >= n_work have nothing to do.
constexpr int kXcds = 8;
__host__ __device__ inline int64_t wgbm_xcd_grid(int64_t n_work) {
  return (n_work + kXcds - 1) / kXcds * kXcds;
}
__device__ inline int64_t wgbm_xcd_work(int64_t id, int64_t n_work) {
  const int64_t per = (n_work + kXcds - 1) / kXcds;
  return (id % kXcds) * per + id / kXcds;
}

// Order-preserving encoding of a non-negative float's magnitude as uint32
// (for atomicMax over |r|).  NaN maps above +inf and is reported as an error.
__device__ inline uint32_t wgbm_abs_bits(float x) { return __float_as_uint(x) & 0x7fffffffu; }

template <typename T>
__device__ inline T wgbm_wave_sum(T v) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ inline uint32_t wgbm_wave_max_u32(uint32_t v) {
  for (int o = 32; o > 0; o >>= 1) {
    uint32_t w = __shfl_xor(v, o, 64);
    v = v > w ? v : w;
  }
  return v;
}

// block-wide max (blockDim.x a multiple of 64, at most 1024); result valid in
// every thread
__device__ inline uint32_t wgbm_block_max_u32(uint32_t v) {
  __shared__ uint32_t s_red[16];
  v = wgbm_wave_max_u32(v);
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) s_red[w] = v;
  __syncthreads();
  uint32_t m = 0;
  for (int k = 0; k < (int)(blockDim.x >> 6); ++k) m = s_red[k] > m ? s_red[k] : m;
  __syncthreads();
  return m;
}

// Deterministic exp for softmax (x <= 0 expected, any finite x accepted).
// Cody-Waite reduction x = k*ln2 + r with a two-part ln2, then the degree-7
// Taylor polynomial of e^r on |r| <= ln2/2 (truncation < 6e-9 relative),
// evaluated in Horner form with explicit fmaf; scaling by 2^k with ldexpf.
// Only IEEE-exact primitives are used, so host and device agree bit for bit.
__host__ __device__ inline float wgbm_expf(float x) {
  if (x != x) return x;
  if (x < -104.0f) return 0.0f;
  if (x > 88.5f) return __builtin_inff();
  const float log2e = 1.44269504088896341f;
  const float ln2_hi = 0.693145751953125f;        // 15 significant bits: k*ln2_hi is exact
  const float ln2_lo = 1.42860682030941723212e-6f;  // ln 2 - ln2_hi
  float k = rintf(x * log2e);
  float r = fmaf(k, -ln2_hi, x);
  r = fmaf(k, -ln2_lo, r);
  float p = 1.0f / 5040.0f;
  p = fmaf(p, r, 1.0f / 720.0f);
  p = fmaf(p, r, 1.0f / 120.0f);
  p = fmaf(p, r, 1.0f / 24.0f);
  p = fmaf(p, r, 1.0f / 6.0f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)k);
}

// ---------------------------------------------------------------------------
// workgroup scans (blockDim.x == 1024, 16 waves)
// ---------------------------------------------------------------------------
// exclusive scan of one value per thread; *total = sum over the workgroup
__device__ inline int64_t wgbm_block_excl_scan(int64_t v, int64_t* wsum /*[16]*/,
                                               int64_t* total) {
  // 1024 threads: the wave totals, scanned over lanes 0..15 of every wave
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t x = wgbm_wave_incl_scan_i64(v);
  if (lane == 63) wsum[w] = x;
  __syncthreads();
  const int64_t s = wgbm_row_incl_scan_i64(lane < 16 ? wsum[lane] : 0);
  const int64_t pre = wgbm_readlane_i64(s, w > 0 ? w - 1 : 0);
  *total = wgbm_readlane_i64(s, 15);
  __syncthreads();
  return (w > 0 ? pre : 0) + x - v;
}

// Exclusive scan of n values get(i) by one workgroup, kScanK * 1024 values
// per step: the step's values are read coalesced into LDS (buf, kScanK *
// 1024 words), every thread scans kScanK consecutive ones, the thread totals
// are scanned across the workgroup, and put(i, prefix) is written coalesced.
// Returns the total.
constexpr int kScanK = 4;
template <typename Get, typename Put>
__device__ inline int64_t wgbm_block_scan_tiled(int n, Get get, Put put, int64_t* wsum,
                                                int64_t* buf) {
  const int t = threadIdx.x;
  constexpr int kStep = kScanK * 1024;
  int64_t carry = 0;
  for (int base = 0; base < n; base += kStep) {
#pragma unroll
    for (int j = 0; j < kScanK; ++j) {
      const int i = base + j * 1024 + t;
      buf[j * 1024 + t] = i < n ? get(i) : 0;
    }
    __syncthreads();
    int64_t run = 0;
#pragma unroll
    for (int m = 0; m < kScanK; ++m) run += buf[t * kScanK + m];
    int64_t tot;
    int64_t ex = carry + wgbm_block_excl_scan(run, wsum, &tot);
#pragma unroll
    for (int m = 0; m < kScanK; ++m) {
      const int64_t v = buf[t * kScanK + m];
      buf[t * kScanK + m] = ex;
      ex += v;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kScanK; ++j) {
      const int i = base + j * 1024 + t;
      if (i < n) put(i, buf[j * 1024 + t]);
    }
    carry += tot;
    __syncthreads();
  }
  return carry;
}
