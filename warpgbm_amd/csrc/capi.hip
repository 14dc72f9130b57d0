// extern "C" boundary of the library (declared in include/warpgbm_amd.h).
#include <algorithm>
#include <mutex>

#include "../../include/warpgbm_amd.h"
#include "common.hpp"
#include "engine.hpp"
#include "kernels.hpp"

const char* wgbm_last_error_impl();

using namespace wgbm;

static inline hipStream_t S(void* s) { return (hipStream_t)s; }
static inline unsigned nblocks(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

constexpr int kMaxDevices = 64;  // devices the no-allocation entry point keeps addresses for
// wgbm_predict_forest takes the heap path from this many trees on
constexpr int64_t kForestHeapMinTrees = 8;

extern "C" {

int wgbm_probe_lds_atomics(int32_t blocks, int32_t iters, double* ops_per_s, void* stream) {
  WGBM_REQUIRE(blocks >= 1 && blocks <= (1 << 16) && iters >= 1 && ops_per_s,
               "probe_lds_atomics: bad arguments");
  return probe_lds_atomics(blocks, iters, ops_per_s, S(stream));
}

int wgbm_probe_hbm_read(const void* buf, int64_t bytes, int32_t iters, double* bytes_per_s,
                        void* stream) {
  WGBM_REQUIRE(buf && bytes >= 16 && ((uintptr_t)buf & 15) == 0 && iters >= 1 && iters <= 1000 &&
                   bytes_per_s,
               "probe_hbm_read: bad arguments (buffer %p, %lld bytes, %d iterations)", buf,
               (long long)bytes, iters);
  return probe_hbm_read(buf, bytes, iters, bytes_per_s, S(stream));
}

const char* wgbm_version(void) { return "warpgbm_amd 0.1.0 (gfx950)"; }
const char* wgbm_last_error(void) { return wgbm_last_error_impl(); }

// ---------------------------------------------------------------------------
// shared histogram pipeline: shift -> (era sort) -> tiles -> partials -> f32
// ---------------------------------------------------------------------------
// Working memory of one call: the library's arena (scratch_get, grows on
// demand), or one fixed buffer carved into 256-byte-aligned pieces (the
// no-allocation entry point).  Every piece is written before it is read.
struct HistScratch {
  hipStream_t st;
  unsigned char* base = nullptr;
  size_t cap = 0, used = 0;
  void* get(size_t bytes, int slot) {
    if (!base) return scratch_get(st, bytes, slot);
    const size_t off = (used + 255) & ~(size_t)255;
    if (off > cap || bytes > cap - off) return nullptr;
    used = off + bytes;
    return base + off;
  }
};

constexpr int kAbsBlocks = 256;  // per-block |residual| maxima of one call, at most

// sizes of one call, shared by the pipeline and the no-allocation size check
struct HistPlan {
  int V = 1, n_chunks = 1, n_abs = 1, n_keys = 1;
  // per_key: several segments (or eras), each quantised at the shift of its
  // own largest |residual|; else one shift for the call
  bool regroup = false, gather_resid = false, per_key = false;
  int64_t R = 1024, max_tiles = 1, tile_words = 0;
};

static HistPlan hist_plan(int32_t n_hist_feats, int32_t num_bins, int64_t n_pos,
                          const int32_t* rows, const int64_t* seg_dev, int32_t n_seg,
                          int32_t num_eras) {
  HistPlan p;
  p.V = hist_pick_v(num_bins, n_hist_feats);
  p.n_chunks = (n_hist_feats + kHistSlots * p.V - 1) / (kHistSlots * p.V);
  // per-block maxima of |residual|: blocks of 1024 threads, at most 256 of
  // them (every wave of the tile kernel reduces them to the shift)
  p.n_abs = (int)std::max<int64_t>(1, std::min<int64_t>(nblocks(n_pos, 1024), kAbsBlocks));
  // a row list without an era regrouping: the residuals are gathered into
  // position order in the same pass, so the tile kernel reads them
  // contiguously instead of one 4-byte gather per row
  p.regroup = !seg_dev && num_eras > 1;
  p.gather_resid = rows && !p.regroup;
  // segments: explicit (seg_dev), by era (sort rows by era), or a single one
  p.n_keys = seg_dev ? n_seg : (p.regroup ? num_eras : 1);
  p.per_key = p.n_keys > 1;
  // tiles: ~1 workgroup per CU over the whole call
  const int64_t tiles_target = std::max<int64_t>(1, kHistTargetWGCall / p.n_chunks);
  int64_t R = (n_pos + tiles_target - 1) / tiles_target;
  p.R = std::min<int64_t>(std::max<int64_t>(R, 1024), WGBM_MAX_TILE_ROWS);
  p.max_tiles = n_pos / p.R + p.n_keys + 1;
  p.tile_words = (int64_t)p.n_chunks * kHistSlots * p.V * num_bins;
  return p;
}

// bytes of the pieces a call without era regrouping or feature selection
// takes (control words, gathered residuals, tiles, tile starts, partials),
// each rounded up to 256 bytes as HistScratch carves them
static size_t hist_scratch_bytes(const HistPlan& p, int64_t n_pos) {
  auto r = [](size_t b) { return (b + 255) & ~(size_t)255; };
  size_t b = r(sizeof(uint32_t) * (64 + kAbsBlocks));
  if (p.gather_resid) b += r(sizeof(float) * (size_t)std::max<int64_t>(n_pos, 1));
  b += r(sizeof(Tile) * (size_t)p.max_tiles);
  b += r(sizeof(int32_t) * ((size_t)p.n_keys + 1));
  b += r(sizeof(unsigned long long) * (size_t)(p.max_tiles * p.tile_words));
  if (p.per_key) b += r(sizeof(uint32_t) * (size_t)p.n_keys);
  return b;
}

// n_hist_feats: code columns histogrammed (feat_idx == nullptr: outputs
// [key][n_hist_feats][B]), or the code columns of a row that feat_idx
// selects from (outputs [key][n_out_feats][B], output o = column
// feat_idx[o]; only the selected columns are histogrammed)
static int histogram_pipeline(const int8_t* codes, int64_t n_rows, int64_t stride,
                              int32_t n_hist_feats, const float* resid, const int32_t* rows,
                              int64_t n_pos, const int64_t* seg_dev, int32_t n_seg,
                              const int32_t* era, int32_t num_eras, const int32_t* feat_idx,
                              int32_t n_out_feats, int32_t num_bins, float* G, float* H,
                              bool native, HistScratch& sc) {
  hipStream_t st = sc.st;
  const bool fsel = feat_idx != nullptr;
  WGBM_REQUIRE(!fsel || (rows && !native), "feature selection needs a row list and raw codes");
  // histogram features: the distinct selected columns, at most this many
  const int32_t width = fsel ? std::min(n_out_feats, n_hist_feats) : n_hist_feats;
  const HistPlan pl = hist_plan(width, num_bins, n_pos, rows, seg_dev, n_seg, num_eras);
  const int V = pl.V, n_chunks = pl.n_chunks, n_abs = pl.n_abs, n_keys = pl.n_keys;
  const bool regroup = pl.regroup;
  const int64_t R = pl.R, max_tiles = pl.max_tiles, tile_words = pl.tile_words;
  // control words and the per-block maxima
  uint32_t* ctl = (uint32_t*)sc.get(sizeof(uint32_t) * (64 + kAbsBlocks), 0);
  WGBM_REQUIRE(ctl, "scratch allocation failed");
  uint32_t* absmax = ctl;
  int32_t* shift = (int32_t*)(ctl + 16);
  int32_t* n_tiles = (int32_t*)(ctl + 32);
  int32_t* n_sel = (int32_t*)(ctl + 48);
  uint32_t* abs_part = ctl + 64;
  float* rpos = nullptr;
  if (pl.gather_resid) {
    rpos = (float*)sc.get(sizeof(float) * std::max<int64_t>(n_pos, 1), 6);
    WGBM_REQUIRE(rpos, "scratch allocation failed");
  }
  Tile* tiles = (Tile*)sc.get(sizeof(Tile) * max_tiles, 3);
  int32_t* kts = (int32_t*)sc.get(sizeof(int32_t) * ((size_t)n_keys + 1), 4);
  const int64_t words = max_tiles * tile_words;
  unsigned long long* part =
      (unsigned long long*)sc.get(sizeof(unsigned long long) * words, 5);
  WGBM_REQUIRE(tiles && kts && part, "scratch allocation failed (%lld words)", (long long)words);
  uint32_t* key_max = nullptr;
  if (pl.per_key) {
    key_max = (uint32_t*)sc.get(sizeof(uint32_t) * (size_t)n_keys, 13);
    WGBM_REQUIRE(key_max, "scratch allocation failed");
  }
  FeatMapArgs fm;
  if (fsel) {
    // mark [n_master], next [n_out], list and head [width], run [n_chunks]
    const size_t ints =
        (size_t)n_hist_feats + (size_t)n_out_feats + 2 * (size_t)width + (size_t)n_chunks;
    int32_t* m = (int32_t*)sc.get(sizeof(int32_t) * ints, 7);
    WGBM_REQUIRE(m, "scratch allocation failed");
    fm.feat_idx = feat_idx;
    fm.n_out = n_out_feats;
    fm.n_master = n_hist_feats;
    fm.V = V;
    fm.n_chunks = n_chunks;
    fm.mark = m;
    fm.next = m + n_hist_feats;
    fm.list = fm.next + n_out_feats;
    fm.head = fm.list + width;
    fm.run = fm.head + width;
    fm.count = n_sel;
  }

  // maxima (+ gathered residuals), the tile plan unless the rows are
  // regrouped by era first, and the feature map: one launch
  const unsigned prep_blocks = (unsigned)(n_abs + (regroup ? 0 : 1) + (fsel ? 1 : 0));
  hipLaunchKernelGGL(hist_prep_kernel, dim3(prep_blocks), dim3(1024), 0, st, resid, rows, n_pos,
                     abs_part, rpos, n_abs, regroup ? 0 : 1, seg_dev, n_keys, (int32_t)R,
                     (int32_t)max_tiles, tiles, kts, n_tiles, fm, key_max);
  WGBM_LAUNCH_CHECK();
  const int32_t* order = rows;
  const int64_t* seg = seg_dev;
  if (regroup) {
    // blocks of about 8192 positions, at most 1024, and at most 2^24 count words
    int64_t nb = std::min<int64_t>(std::max<int64_t>((n_pos + 8191) / 8192, 1), 1024);
    nb = std::max<int64_t>(1, std::min<int64_t>(nb, ((int64_t)1 << 24) / num_eras));
    const int64_t per_block = std::max<int64_t>(1, (n_pos + nb - 1) / nb);
    int32_t* counts = (int32_t*)sc.get(sizeof(int32_t) * (size_t)(num_eras * nb), 1);
    int64_t* era_tot = (int64_t*)sc.get(sizeof(int64_t) * ((size_t)num_eras + 1), 12);
    int32_t* sorted = (int32_t*)sc.get(sizeof(int32_t) * std::max<int64_t>(n_pos, 1), 2);
    WGBM_REQUIRE(counts && era_tot && sorted, "scratch allocation failed");
    hipLaunchKernelGGL(era_block_count_kernel, dim3((unsigned)nb), dim3(1024), 0, st, rows, n_pos,
                       era, num_eras, per_block, counts);
    WGBM_LAUNCH_CHECK();
    hipLaunchKernelGGL(era_row_scan_kernel, dim3((unsigned)((num_eras + 15) / 16)), dim3(1024), 0,
                       st, counts, num_eras, (int32_t)nb, era_tot);
    WGBM_LAUNCH_CHECK();
    hipLaunchKernelGGL(era_start_scan_kernel, dim3(1), dim3(1024), 0, st, era_tot, num_eras);
    WGBM_LAUNCH_CHECK();
    hipLaunchKernelGGL(era_block_scatter_kernel, dim3((unsigned)nb), dim3(1024), 0, st, rows,
                       n_pos, era, num_eras, per_block, (const int32_t*)counts,
                       (const int64_t*)era_tot, sorted);
    WGBM_LAUNCH_CHECK();
    order = sorted;
    seg = era_tot;
    hipLaunchKernelGGL(plan_tiles_kernel, dim3(1), dim3(1024), 0, st, seg, n_pos, n_keys,
                       (const int32_t*)nullptr, (int32_t)R, 1, (int32_t)max_tiles, tiles, kts,
                       n_tiles);
    WGBM_LAUNCH_CHECK();
  }
  const int qbits = wgbm_qbits_for_rows(std::max<int64_t>(n_pos, 1));
  if (pl.per_key) {
    // each key's largest |residual| (its shift) over its tiles' positions
    hipLaunchKernelGGL(hist_key_max_kernel, dim3((unsigned)max_tiles), dim3(256), 0, st, tiles,
                       n_tiles, rpos ? rpos : resid, order, rpos ? 1 : 0, key_max);
    WGBM_LAUNCH_CHECK();
  }
  HistLaunch a;
  a.codes = codes;
  a.n_rows = n_rows;
  a.stride = stride;
  a.n_feats = width;
  a.resid = rpos ? rpos : resid;
  a.resid_by_pos = rpos ? 1 : 0;
  a.resid_tree_stride = 0;
  a.shifts = shift;
  a.order = order;
  a.tiles = tiles;
  a.n_tiles = n_tiles;
  a.keys_per_tree = n_keys;
  a.num_bins = num_bins;
  a.part = part;
  a.V = V;
  a.n_chunks = n_chunks;
  a.max_tiles = (int32_t)max_tiles;
  a.native = native ? 1 : 0;
  a.timer_tag = sc.base ? nullptr : "hist_tiles";  // timers create events: not without allocation
  a.sm.qbits = qbits;
  if (pl.per_key) {
    a.sm.key_max = key_max;
  } else {
    a.sm.partial = abs_part;
    a.sm.n_part = n_abs;
    a.sm.absmax_bits = absmax;
    a.sm.shift = shift;
  }
  if (fsel) {
    a.fs.list = fm.list;
    a.fs.count = n_sel;
    a.fs.run = fm.run;
    a.fs.n_master = n_hist_feats;
  }
  int r = launch_hist_tiles(a, st);
  if (r) return r;
  // tiles per segment (finalize's tile split): the planner's estimate
  const int64_t tiles_per_key = std::max<int64_t>(1, (n_pos + R - 1) / R / std::max(n_keys, 1));
  // straight into the (accumulated) outputs, through the feature map if any
  FeatOut fo;
  if (fsel) {
    fo.head = fm.head;
    fo.next = fm.next;
    fo.count = n_sel;
    fo.run = fm.run;
    fo.n_out = n_out_feats;
  }
  return launch_finalize_f32(tiles_per_key, part, kts, n_keys, n_chunks, V, num_bins, width,
                             pl.per_key ? key_max : absmax, pl.per_key ? 1 : 0, qbits, n_tiles,
                             1, fo, G, H, st);
}

int wgbm_compute_histogram3(const int8_t* bin_indices, int64_t n_rows, int64_t n_feats_master,
                            const float* residuals, const int32_t* sample_indices,
                            int64_t n_samples, const int32_t* feature_indices, int64_t n_feats,
                            const int32_t* era_indices, int32_t num_eras, float* grad_hist,
                            float* hess_hist, int32_t num_bins, int32_t threads_per_block,
                            int32_t rows_per_thread, void* stream) {
  (void)threads_per_block;
  (void)rows_per_thread;
  WGBM_REQUIRE(num_bins >= 1 && num_bins <= 127, "num_bins must be in [1, 127], got %d", num_bins);
  WGBM_REQUIRE(num_eras >= 1, "num_eras must be >= 1");
  WGBM_REQUIRE(n_rows >= 0 && n_feats_master >= 1 && n_feats >= 0 && n_samples >= 0,
               "negative size");
  WGBM_REQUIRE(n_feats_master < (int64_t(1) << 31) && n_feats < (int64_t(1) << 31),
               "too many features");
  WGBM_REQUIRE(n_samples == 0 || (bin_indices && residuals && sample_indices),
               "null input pointer");
  WGBM_REQUIRE(n_feats == 0 || (feature_indices && grad_hist && hess_hist), "null output pointer");
  WGBM_REQUIRE(num_eras == 1 || era_indices, "era_indices required when num_eras > 1");
  if (n_feats == 0 || n_samples == 0) return 0;  // nothing to add
  HistScratch sc{S(stream)};
  return histogram_pipeline(bin_indices, n_rows, n_feats_master, (int32_t)n_feats_master,
                            residuals, sample_indices, n_samples, nullptr, 1, era_indices,
                            num_eras, feature_indices, (int32_t)n_feats, num_bins, grad_hist,
                            hess_hist, false, sc);
}

int wgbm_histogram_segments(const int8_t* codes, int64_t n_rows, int64_t stride, int32_t n_feats,
                            const float* residuals, const int32_t* order, const int64_t* seg,
                            int32_t n_seg, int64_t n_pos, int32_t num_bins, int32_t flags,
                            float* G, float* H, void* stream) {
  WGBM_REQUIRE(num_bins >= 1 && num_bins <= 127, "num_bins must be in [1, 127]");
  WGBM_REQUIRE(n_seg >= 1 && seg && codes && residuals && G && H, "bad segment arguments");
  WGBM_REQUIRE(stride >= n_feats && n_feats >= 1, "stride must be >= n_feats >= 1");
  WGBM_REQUIRE((flags & ~WGBM_CODES_NATIVE) == 0, "unknown histogram flags 0x%x", flags);
  HistScratch sc{S(stream)};
  return histogram_pipeline(codes, n_rows, stride, n_feats, residuals, order, n_pos, seg, n_seg,
                            nullptr, 1, nullptr, n_feats, num_bins, G, H,
                            (flags & WGBM_CODES_NATIVE) != 0, sc);
}

// ---------------------------------------------------------------------------
// wgbm_histogram_segments without allocation: the call's working memory is
// carved from g_noalloc_scratch, a fixed device array every GPU the library
// runs on holds until the process ends.  Its address on each device comes
// from hipGetSymbolAddress, fetched once per device on the first call made
// with that device current; the host name of the array is a stand-in and is
// never passed to a kernel.  Calls that overlap on one GPU share the array
// and race; each call writes every piece before reading it.
// ---------------------------------------------------------------------------
static __device__ __align__(256) unsigned char g_noalloc_scratch[WGBM_NOALLOC_SCRATCH_BYTES];
static std::mutex g_noalloc_mu;
static void* g_noalloc_ptr[kMaxDevices] = {};

static int noalloc_scratch_ptr(unsigned char** out) {
  int dev = 0;
  WGBM_CHECK(hipGetDevice(&dev));
  WGBM_REQUIRE(dev >= 0 && dev < kMaxDevices, "histogram_segments_noalloc: device %d beyond %d",
               dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_noalloc_mu);
  if (!g_noalloc_ptr[dev]) {
    void* p = nullptr;
    WGBM_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(g_noalloc_scratch)));
    WGBM_REQUIRE(p, "histogram_segments_noalloc: no device address for the scratch array");
    g_noalloc_ptr[dev] = p;
  }
  *out = (unsigned char*)g_noalloc_ptr[dev];
  return 0;
}

int wgbm_histogram_segments_noalloc(const int8_t* codes, int64_t n_rows, int64_t stride,
                                    int32_t n_feats, const float* residuals, const int32_t* order,
                                    const int64_t* seg, int32_t n_seg, int64_t n_pos,
                                    int32_t num_bins, int32_t flags, float* G, float* H,
                                    void* stream) {
  WGBM_REQUIRE(num_bins >= 1 && num_bins <= 127, "num_bins must be in [1, 127]");
  WGBM_REQUIRE(n_seg >= 1 && seg && codes && residuals && G && H, "bad segment arguments");
  WGBM_REQUIRE(stride >= n_feats && n_feats >= 1, "stride must be >= n_feats >= 1");
  WGBM_REQUIRE(n_pos >= 0, "n_pos must be >= 0");
  WGBM_REQUIRE((flags & ~WGBM_CODES_NATIVE) == 0, "unknown histogram flags 0x%x", flags);
  const HistPlan pl = hist_plan(n_feats, num_bins, n_pos, order, seg, n_seg, 1);
  const size_t need = hist_scratch_bytes(pl, n_pos);
  WGBM_REQUIRE(need <= (size_t)WGBM_NOALLOC_SCRATCH_BYTES,
               "histogram_segments_noalloc: this call needs %zu bytes of scratch, the fixed "
               "array holds %zu (fewer rows, features or segments per call)",
               need, (size_t)WGBM_NOALLOC_SCRATCH_BYTES);
  HistScratch sc{S(stream)};
  int r = noalloc_scratch_ptr(&sc.base);
  if (r) return r;
  sc.cap = WGBM_NOALLOC_SCRATCH_BYTES;
  return histogram_pipeline(codes, n_rows, stride, n_feats, residuals, order, n_pos, seg, n_seg,
                            nullptr, 1, nullptr, n_feats, num_bins, G, H,
                            (flags & WGBM_CODES_NATIVE) != 0, sc);
}

int wgbm_compute_split(const float* G, const float* H, int32_t num_eras, int32_t n_feats,
                       int32_t num_bins, float min_split_gain, float min_child_samples,
                       float eps, float* per_era_gain, float* per_era_direction,
                       int32_t threads, void* stream) {
  (void)min_split_gain;
  (void)threads;
  WGBM_REQUIRE(num_eras >= 1 && n_feats >= 0 && num_bins >= 2, "bad split shape");
  const int64_t n = (int64_t)num_eras * n_feats;
  if (n == 0) return 0;
  WGBM_REQUIRE(G && H && per_era_gain && per_era_direction, "null pointer");
  return launch_split_f32(G, H, num_eras, n_feats, num_bins, min_child_samples, eps,
                          per_era_gain, per_era_direction, S(stream));
}

int wgbm_custom_cuda_binner(const float* X, int64_t n, const float* bin_edges, int32_t n_edges,
                            int8_t* bin_indices, void* stream) {
  WGBM_REQUIRE(n >= 0 && n_edges >= 0, "negative size");
  if (n == 0) return 0;
  WGBM_REQUIRE(X && bin_indices && (n_edges == 0 || bin_edges), "null pointer");
  hipLaunchKernelGGL(bin_column_kernel, dim3(nblocks(n, 256 * kBinColumnU)), dim3(256), 0,
                     S(stream), X, n, bin_edges, n_edges, bin_indices);
  WGBM_LAUNCH_CHECK();
  return 0;
}

}  // extern "C"

static int predict_heap_impl(const int8_t* codes, int64_t n, int64_t codes_stride,
                             int32_t num_bins, const int32_t* feat, const int32_t* bin,
                             const float* leaf, int32_t n_rounds, int32_t K, int32_t H,
                             int32_t max_depth, float learning_rate, float* out, void* stream,
                             const int32_t* skip) {
  WGBM_REQUIRE(n >= 0 && K >= 1 && n_rounds >= 0 && max_depth >= 0 && max_depth <= 29,
               "bad predict_heap shape");  // heap indices below 2^30: int32
  WGBM_REQUIRE(num_bins >= 2 && num_bins <= 127, "num_bins must be in [2, 127]");
  WGBM_REQUIRE(H == (1 << (max_depth + 1)) - 1, "H must be 2^(max_depth+1)-1");
  if (n == 0) return 0;
  WGBM_REQUIRE(codes && out && (n_rounds == 0 || (feat && bin && leaf)), "null pointer");
  if (n_rounds == 0) return 0;
  int32_t RB = 0, TC = 0;
  size_t lds = 0;
  int dev = 0, n_cu = 0;
  WGBM_CHECK(hipGetDevice(&dev));
  WGBM_CHECK(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
  const bool resident = predict_resident_plan(codes_stride, K, H, n_rounds, &RB, &lds) != 0;
  const bool rows = !resident && predict_rows_plan(codes_stride, K, H, n_rounds, &RB, &TC, &lds);
  uint32_t* cnode = nullptr;
  float* cleaf = nullptr;
  if (resident || rows) {
    // the complete-tree tables the LDS predictors walk (H words per tree)
    const int64_t T = (int64_t)n_rounds * K;
    cnode = (uint32_t*)scratch_get(S(stream), sizeof(uint32_t) * (size_t)(T * H), 13);
    WGBM_REQUIRE(cnode, "scratch allocation failed");
    cleaf = reinterpret_cast<float*>(cnode + T * ((H - 1) / 2));
    const int64_t work = T * H;
    hipLaunchKernelGGL(complete_tables_kernel, dim3(nblocks(work, 256)), dim3(256), 0,
                       S(stream), feat, bin, leaf, T, max_depth, codes_stride, learning_rate,
                       cnode, cleaf);
    WGBM_LAUNCH_CHECK();
  }
  if (resident) {
    static bool attr_r = false;
    if (!attr_r) {
      WGBM_CHECK(hipFuncSetAttribute((const void*)predict_resident_kernel<false>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
      attr_r = true;
    }
    // one persistent workgroup per CU (fewer when there are fewer blocks)
    const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(n_cu, nblocks(n, RB)));
    hipLaunchKernelGGL(predict_resident_kernel<false>, dim3((unsigned)grid), dim3(1024), lds,
                       S(stream), codes, n, codes_stride, num_bins, (const uint32_t*)cnode,
                       (const float*)cleaf, n_rounds * K, K, max_depth, RB, out, skip);
  } else if (rows) {
    static bool attr = false;
    if (!attr) {
      WGBM_CHECK(hipFuncSetAttribute((const void*)predict_rows_kernel,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
      attr = true;
    }
    hipLaunchKernelGGL(predict_rows_kernel, dim3(nblocks(n, RB)), dim3(1024), lds, S(stream),
                       codes, n, codes_stride, num_bins, (const uint32_t*)cnode,
                       (const float*)cleaf, n_rounds, K, max_depth, RB, TC, out, skip);
  } else {
    hipLaunchKernelGGL(predict_heap_kernel, dim3(nblocks(n * K, 256)), dim3(256), 0, S(stream),
                       codes, n, codes_stride, num_bins, feat, bin, leaf, n_rounds, K, H,
                       max_depth, learning_rate, out, skip);
  }
  WGBM_LAUNCH_CHECK();
  return 0;
}

// predict_forest's heap tables walked straight over the raw codes (no native
// copy): rows of stride n_feats (a multiple of 8, 8-byte aligned), the
// resident predictor only.  Returns -1 without launching when that does not
// fit (the caller then copies the codes to the native layout).
static int predict_forest_raw(const int8_t* raw, int64_t n, int64_t n_feats,
                              const int32_t* feat, const int32_t* bin, const float* leaf,
                              int32_t n_trees, int32_t H, int32_t D, float learning_rate,
                              float* out, hipStream_t st, const int32_t* skip) {
  int32_t RB = 0;
  size_t lds = 0;
  if (n_feats % 8 != 0 || ((uintptr_t)raw % 8) != 0 ||
      !predict_resident_plan(n_feats, 1, H, n_trees, &RB, &lds, true))
    return -1;
  int dev = 0, n_cu = 0;
  WGBM_CHECK(hipGetDevice(&dev));
  WGBM_CHECK(hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev));
  uint32_t* cnode = (uint32_t*)scratch_get(st, sizeof(uint32_t) * (size_t)n_trees * H, 13);
  WGBM_REQUIRE(cnode, "scratch allocation failed");
  float* cleaf = reinterpret_cast<float*>(cnode + (int64_t)n_trees * ((H - 1) / 2));
  const int64_t work = (int64_t)n_trees * H;
  hipLaunchKernelGGL(complete_tables_kernel, dim3(nblocks(work, 256)), dim3(256), 0, st, feat,
                     bin, leaf, (int64_t)n_trees, D, n_feats, learning_rate, cnode, cleaf);
  WGBM_LAUNCH_CHECK();
  static bool attr = false;
  if (!attr) {
    WGBM_CHECK(hipFuncSetAttribute((const void*)predict_resident_kernel<true>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    attr = true;
  }
  const int64_t grid = std::max<int64_t>(1, std::min<int64_t>(n_cu, nblocks(n, RB)));
  hipLaunchKernelGGL(predict_resident_kernel<true>, dim3((unsigned)grid), dim3(1024), lds, st,
                     raw, n, n_feats, 127, (const uint32_t*)cnode, (const float*)cleaf, n_trees,
                     1, D, RB, out, skip);
  WGBM_LAUNCH_CHECK();
  return 0;
}

extern "C" {

int wgbm_predict_forest(const int8_t* bin_indices, int64_t n, int64_t n_feats,
                        const float* tree_tensor, int64_t n_trees, int64_t max_nodes,
                        float learning_rate, float* out, void* stream) {
  WGBM_REQUIRE(n >= 0 && n_feats >= 0 && n_trees >= 0 && max_nodes >= 1, "bad predict shape");
  if (n == 0) return 0;
  WGBM_REQUIRE(bin_indices && out && (n_trees == 0 || tree_tensor), "null pointer");
  hipStream_t st = S(stream);
  // Heap path, for enough trees and rows: the flat tables become heap tables
  // of depth D = floor(log2(max_nodes)) - 1 (flatten_tree's max_nodes =
  // 2^(max_depth+1)), walked by the LDS predictors.  Rows of a multiple of 8
  // bytes are read as they are by the resident predictor (a negative code
  // read as 0, which every split sends left); otherwise the codes get a
  // native copy (num_bins 127: a negative code becomes the byte 127, which
  // every split sends left; 127 becomes 128, which every split bin <= 126
  // sends right; the other codes stay).  A
  // table the heap cannot hold sets a device flag: the heap walk is skipped
  // and the flat walk below runs instead; otherwise the flat walk exits.
  int D = 0;
  while ((int64_t(4) << D) <= max_nodes) ++D;  // 2^(D+1) <= max_nodes < 2^(D+2)
  const bool heap_path = n_trees >= kForestHeapMinTrees && n >= 4096 && n_feats >= 1 &&
                         n_feats <= 65535 && max_nodes >= 2 && D <= 12 &&
                         n_trees * ((int64_t(2) << D) - 1) <= (int64_t(1) << 28);
  const int32_t* flag = nullptr;
  if (heap_path) {
    const int64_t H = (int64_t(2) << D) - 1, Sn = (n_feats + 127) / 128 * 128;
    int32_t* fl = (int32_t*)scratch_get(st, sizeof(int32_t) * 64, 14);
    int32_t* feat = (int32_t*)scratch_get(st, sizeof(int32_t) * (size_t)(n_trees * H), 15);
    int32_t* bin = (int32_t*)scratch_get(st, sizeof(int32_t) * (size_t)(n_trees * H), 16);
    float* leaf = (float*)scratch_get(st, sizeof(float) * (size_t)(n_trees * H), 17);
    WGBM_REQUIRE(fl && feat && bin && leaf, "scratch allocation failed");
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, st, fl, (int64_t)1, 0);
    WGBM_LAUNCH_CHECK();
    hipLaunchKernelGGL(flat_to_heap_kernel, dim3(nblocks(n_trees * H, 256)), dim3(256), 0, st,
                       tree_tensor, n_trees, max_nodes, n_feats, (int32_t)D, feat, bin, leaf, fl);
    WGBM_LAUNCH_CHECK();
    // the raw codes walked as they are when the resident predictor can read
    // them; else a native copy for the LDS predictors
    int r = predict_forest_raw(bin_indices, n, n_feats, feat, bin, leaf, (int32_t)n_trees,
                               (int32_t)H, D, learning_rate, out, st, fl);
    if (r > 0) return r;
    if (r < 0) {
      int8_t* nat = (int8_t*)scratch_get(st, (size_t)(n * Sn), 18);
      WGBM_REQUIRE(nat, "scratch allocation failed");
      r = wgbm_copy_prebinned(bin_indices, n, (int32_t)n_feats, n_feats, nat, Sn, nullptr, 127,
                              nullptr, stream);
      if (r) return r;
      r = predict_heap_impl(nat, n, Sn, 127, feat, bin, leaf, (int32_t)n_trees, 1, (int32_t)H, D,
                            learning_rate, out, stream, fl);
      if (r) return r;
    }
    flag = fl;
  }
  hipLaunchKernelGGL(predict_table_kernel, dim3(nblocks(n, 256)), dim3(256), 0, st, bin_indices,
                     n, n_feats, tree_tensor, n_trees, max_nodes, learning_rate, out, flag);
  WGBM_LAUNCH_CHECK();
  return 0;
}

int wgbm_quantile_edges(const float* sorted, int64_t n, int32_t n_feats, const float* q,
                        int32_t nq, float* edges, void* stream) {
  WGBM_REQUIRE(n >= 1 && n_feats >= 0 && nq >= 0, "bad quantile shape");
  WGBM_REQUIRE(n <= (int64_t(1) << 24), "quantile input too large (n > 2^24), as torch.quantile");
  const int64_t tot = (int64_t)n_feats * nq;
  if (tot == 0) return 0;
  WGBM_REQUIRE(sorted && q && edges, "null pointer");
  hipLaunchKernelGGL(quantile_edges_kernel, dim3(nblocks(tot, 256)), dim3(256), 0, S(stream),
                     sorted, n, n_feats, q, nq, edges);
  WGBM_LAUNCH_CHECK();
  return 0;
}

// values of rows [0, rows) of X (row stride x_stride) into the column-major
// key array keys (column f at keys + f * ks; the caller offsets keys by the
// first row), and the columns' extremes into kmin / kmax
static int launch_stage_rows(const float* X, int64_t rows, int32_t fc, int64_t x_stride,
                             uint32_t* keys, int64_t ks, uint32_t* kmin, uint32_t* kmax,
                             hipStream_t st) {
  const dim3 tg((unsigned)wgbm_xcd_grid((int64_t)nblocks(rows, kTransRows) * nblocks(fc, 64)));
  // 16-byte row loads when every row starts on 16 bytes
  const bool vec = ((uintptr_t)X % 16) == 0 && x_stride % 4 == 0;
  if (vec)
    hipLaunchKernelGGL(transpose_values_kernel<true>, tg, dim3(256), 0, st, X, rows, fc, x_stride,
                       ks, keys, kmin, kmax);
  else
    hipLaunchKernelGGL(transpose_values_kernel<false>, tg, dim3(256), 0, st, X, rows, fc,
                       x_stride, ks, keys, kmin, kmax);
  WGBM_LAUNCH_CHECK();
  return 0;
}

// the selection over staged columns (per-feature buffers from the scratch pool)
static int launch_select(const uint32_t* keys, int64_t n, int64_t ks, int32_t fc, const float* q,
                         int32_t nq, float* edges, const uint32_t* kmin, const uint32_t* kmax,
                         hipStream_t st) {
  // per-feature buffer of the keys of the target buckets (a quarter of the
  // column; a column with more falls back to full scans)
  const int64_t ccap = std::max<int64_t>(1024, n / 4);
  uint32_t* cbuf = (uint32_t*)scratch_get(st, sizeof(uint32_t) * (size_t)((int64_t)fc * ccap), 10);
  WGBM_REQUIRE(cbuf, "scratch allocation failed");
  hipLaunchKernelGGL(quantile_select_kernel, dim3(fc), dim3(512), 0, st, keys, n, ks, fc, q, nq,
                     edges, kmin, kmax, cbuf, ccap);
  WGBM_LAUNCH_CHECK();
  return 0;
}

int wgbm_quantile_stage_rows(const float* X, int64_t rows, int32_t n_feats, int64_t x_stride,
                             int64_t row0, uint32_t* cols, int64_t cols_stride, uint32_t* kmin,
                             uint32_t* kmax, void* stream) {
  WGBM_REQUIRE(rows >= 0 && n_feats >= 0 && x_stride >= n_feats && row0 >= 0,
               "bad quantile staging shape");
  WGBM_REQUIRE(row0 % 4 == 0 && cols_stride % 32 == 0 && row0 + rows <= cols_stride,
               "staged rows must start on a multiple of 4 inside the column stride "
               "(a multiple of 32)");
  WGBM_REQUIRE(cols_stride <= (int64_t(1) << 24) + 32, "quantile input too large (n > 2^24)");
  if (rows == 0 || n_feats == 0) return 0;
  WGBM_REQUIRE(X && cols && kmin && kmax, "null pointer");
  return launch_stage_rows(X, rows, n_feats, x_stride, cols + row0, cols_stride, kmin, kmax,
                           S(stream));
}

int wgbm_quantile_edges_staged(const uint32_t* cols, int64_t n, int32_t n_feats,
                               int64_t cols_stride, const uint32_t* kmin, const uint32_t* kmax,
                               const float* q, int32_t nq, float* edges, void* stream) {
  WGBM_REQUIRE(n >= 1 && n_feats >= 0 && nq >= 0 && nq <= 126, "bad quantile shape");
  WGBM_REQUIRE(n <= (int64_t(1) << 24), "quantile input too large (n > 2^24), as torch.quantile");
  WGBM_REQUIRE(cols_stride % 32 == 0 && cols_stride >= n, "bad staged column stride");
  if ((int64_t)n_feats * nq == 0) return 0;
  WGBM_REQUIRE(cols && kmin && kmax && q && edges, "null pointer");
  return launch_select(cols, n, cols_stride, n_feats, q, nq, edges, kmin, kmax, S(stream));
}

int wgbm_quantile_edges_matrix(const float* X, int64_t n, int32_t n_feats, int64_t x_stride,
                               const float* q, int32_t nq, float* edges, void* stream) {
  WGBM_REQUIRE(n >= 1 && n_feats >= 0 && nq >= 0 && nq <= 126 && x_stride >= n_feats,
               "bad quantile shape");
  WGBM_REQUIRE(n <= (int64_t(1) << 24), "quantile input too large (n > 2^24), as torch.quantile");
  if ((int64_t)n_feats * nq == 0) return 0;
  WGBM_REQUIRE(X && q && edges, "null pointer");
  hipStream_t st = S(stream);
  // column-major keys of up to `chunk` features at a time (bounded scratch)
  // (up to 2^30 keys = 4 GiB of scratch: all features of a 1M-row matrix in
  // one launch, so that every CU holds several columns)
  // value columns padded to a multiple of 32 values (128-byte lines; the
  // kernels need 16-byte aligned quads)
  const int64_t ks = (n + 31) / 32 * 32;
  const int64_t chunk = std::max<int64_t>(1, std::min<int64_t>(n_feats, (int64_t(1) << 30) / ks));
  uint32_t* keys = (uint32_t*)scratch_get(st, sizeof(uint32_t) * (size_t)(chunk * ks), 8);
  uint32_t* kmm = (uint32_t*)scratch_get(st, sizeof(uint32_t) * 2 * (size_t)chunk, 11);
  WGBM_REQUIRE(keys && kmm, "scratch allocation failed");
  uint32_t *kmin = kmm, *kmax = kmm + chunk;
  for (int64_t f0 = 0; f0 < n_feats; f0 += chunk) {
    const int32_t fc = (int32_t)std::min<int64_t>(chunk, n_feats - f0);
    if (fill_u32(kmin, fc, 0xffffffffu, st) || fill_u32(kmax, fc, 0u, st)) return WGBM_EINVAL;
    int r = launch_stage_rows(X + f0, n, fc, x_stride, keys, ks, kmin, kmax, st);
    if (r) return r;
    r = launch_select(keys, n, ks, fc, q, nq, edges + f0 * nq, kmin, kmax, st);
    if (r) return r;
  }
  return 0;
}

int wgbm_bin_matrix(const float* X, int64_t n, int32_t n_feats, int64_t x_stride,
                    const float* edges, int32_t n_edges, int8_t* codes_rm, int64_t codes_stride,
                    int8_t* codes_cm, void* stream) {
  WGBM_REQUIRE(n >= 0 && n_feats >= 1 && x_stride >= n_feats && codes_stride >= n_feats,
               "bad bin_matrix shape");
  WGBM_REQUIRE(n_edges >= 0 && n_edges <= 126, "n_edges must be in [0, 126]");
  if (n == 0) return 0;
  WGBM_REQUIRE(X && codes_rm && (n_edges == 0 || edges), "null pointer");
  const size_t lds = sizeof(float) * kBinTileFeats * bin_edge_stride(n_edges);
  const int64_t nft = nblocks(n_feats, kBinTileFeats);
  const dim3 grid((unsigned)wgbm_xcd_grid((int64_t)nblocks(n, kBinTileRows) * nft));
  // 16-byte loads when every row starts on 16 bytes
  if (((uintptr_t)X % 16) == 0 && x_stride % 4 == 0)
    hipLaunchKernelGGL(bin_matrix_kernel<true>, grid, dim3(256), lds, S(stream), X, n, n_feats,
                       x_stride, edges, n_edges, codes_rm, codes_stride, codes_cm);
  else
    hipLaunchKernelGGL(bin_matrix_kernel<false>, grid, dim3(256), lds, S(stream), X, n, n_feats,
                       x_stride, edges, n_edges, codes_rm, codes_stride, codes_cm);
  WGBM_LAUNCH_CHECK();
  const int64_t covered = nft * kBinTileFeats;
  if (codes_stride > covered) {
    const int64_t tot = n * (codes_stride - covered);
    hipLaunchKernelGGL(pad_codes_kernel, dim3(nblocks(tot, 256)), dim3(256), 0, S(stream),
                       codes_rm, n, codes_stride, (int32_t)covered, (int8_t)(n_edges + 2));
    WGBM_LAUNCH_CHECK();
  }
  return 0;
}

int wgbm_copy_prebinned(const int8_t* X, int64_t n, int32_t n_feats, int64_t x_stride,
                        int8_t* codes_rm, int64_t codes_stride, int8_t* codes_cm,
                        int32_t num_bins, int32_t* over_flag, void* stream) {
  WGBM_REQUIRE(n >= 0 && n_feats >= 1 && x_stride >= n_feats && codes_stride >= n_feats,
               "bad copy_prebinned shape");
  WGBM_REQUIRE(num_bins >= 2 && num_bins <= 127, "num_bins must be in [2, 127]");
  if (over_flag) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, S(stream), over_flag, (int64_t)1, 0);
    WGBM_LAUNCH_CHECK();
  }
  if (n == 0) return 0;
  WGBM_REQUIRE(X && codes_rm, "null pointer");
  const int64_t nft = nblocks(n_feats, kBinTileFeats);
  const dim3 grid((unsigned)wgbm_xcd_grid((int64_t)nblocks(n, kBinTileRows) * nft));
  hipLaunchKernelGGL(copy_prebinned_kernel, grid, dim3(256), 0, S(stream), X, n, n_feats,
                     x_stride, codes_rm, codes_stride, codes_cm, num_bins, over_flag);
  WGBM_LAUNCH_CHECK();
  const int64_t covered = nft * kBinTileFeats;
  if (codes_stride > covered) {
    const int64_t tot = n * (codes_stride - covered);
    hipLaunchKernelGGL(pad_codes_kernel, dim3(nblocks(tot, 256)), dim3(256), 0, S(stream),
                       codes_rm, n, codes_stride, (int32_t)covered, (int8_t)(num_bins + 1));
    WGBM_LAUNCH_CHECK();
  }
  return 0;
}

int wgbm_predict_heap(const int8_t* codes, int64_t n, int64_t codes_stride, int32_t num_bins,
                      const int32_t* feat, const int32_t* bin, const float* leaf,
                      int32_t n_rounds, int32_t K, int32_t H, int32_t max_depth,
                      float learning_rate, float* out, void* stream) {
  return predict_heap_impl(codes, n, codes_stride, num_bins, feat, bin, leaf, n_rounds, K, H,
                           max_depth, learning_rate, out, stream, nullptr);
}

int wgbm_softmax_rows(float* x, int64_t n, int32_t K, void* stream) {
  WGBM_REQUIRE(n >= 0 && K >= 1, "bad softmax shape");
  if (n == 0) return 0;
  WGBM_REQUIRE(x, "null pointer");
  hipLaunchKernelGGL(softmax_rows_kernel, dim3(nblocks(n, 256)), dim3(256), 0, S(stream), x, n, K);
  WGBM_LAUNCH_CHECK();
  return 0;
}

int wgbm_importance_add(float* acc, int32_t n_feats, int32_t num_eras, const float* gain,
                        const int64_t* node, const int64_t* feat_start, void* stream) {
  WGBM_REQUIRE(n_feats >= 1 && num_eras >= 1, "bad importance shape");
  WGBM_REQUIRE(acc && feat_start, "null pointer");
  hipLaunchKernelGGL(importance_add_kernel, dim3(nblocks((int64_t)n_feats * num_eras, 256)),
                     dim3(256), 0, S(stream), acc, n_feats, num_eras, gain, node, feat_start);
  WGBM_LAUNCH_CHECK();
  return 0;
}

// ---------------------------------------------------------------------------
// engine
// ---------------------------------------------------------------------------
struct wgbm_engine {
  Engine* e;
};

int wgbm_engine_create(wgbm_engine** out, const wgbm_engine_config* cfg) {
  WGBM_REQUIRE(out && cfg, "null pointer");
  EngineConfig c;
  c.n_rows = cfg->n_rows;
  c.n_feats = cfg->n_feats;
  c.stride = cfg->codes_stride;
  c.num_bins = cfg->num_bins;
  c.num_eras = cfg->num_eras;
  c.max_depth = cfg->max_depth;
  c.n_trees = cfg->n_trees;
  c.objective = cfg->objective;
  c.min_child_weight = cfg->min_child_weight;
  c.min_split_gain = cfg->min_split_gain;
  c.l2_reg = cfg->l2_reg;
  c.learning_rate = cfg->learning_rate;
  c.codes_rm = cfg->codes_rm;
  c.codes_cm = cfg->codes_cm;
  c.root_order = cfg->root_order;
  c.era_start = cfg->era_start;
  c.level_bytes = cfg->level_bytes;
  Engine* e = nullptr;
  int r = engine_create(&e, c);
  if (r) return r;
  *out = new wgbm_engine{e};
  return 0;
}

int wgbm_engine_round(wgbm_engine* eng, const void* target, float* pred, const int32_t* feat_sel,
                      int32_t n_sel, const wgbm_tree_record* rec, void* stream) {
  WGBM_REQUIRE(eng && rec, "null pointer");
  TreeRecord r;
  r.feat = rec->feat;
  r.bin = rec->bin;
  r.leaf = rec->leaf;
  r.count = rec->count;
  r.gain = rec->gain;
  r.H = rec->H;
  WGBM_REQUIRE(r.feat && r.bin && r.leaf && r.count && r.gain, "null record pointer");
  return engine_round(eng->e, target, pred, feat_sel, n_sel, r, S(stream));
}

int wgbm_engine_set_tuning(wgbm_engine* eng, int32_t key, int64_t value) {
  WGBM_REQUIRE(eng, "null engine");
  return engine_set_tuning(eng->e, key, value);
}

void wgbm_engine_destroy(wgbm_engine* eng) {
  if (!eng) return;
  engine_destroy(eng->e);
  delete eng;
}

void wgbm_timer_enable(int32_t mode) { timer_enable(mode); }
int wgbm_timer_read(const char* tag, double* total_ms, int64_t* count) {
  long c = 0;
  int r = timer_read(tag, total_ms, &c);
  *count = c;
  return r;
}
void wgbm_timer_reset(void) { timer_reset(); }
void wgbm_release_scratch(void) { scratch_release_all(); }

}  // extern "C"
