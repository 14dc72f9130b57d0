/*
 * warpgbm_amd -- C ABI of the MI355X (gfx950) hot path of WarpGBM.
 *
 * All pointers are device pointers (HIP global memory) unless stated
 * otherwise; `stream` is a hipStream_t passed as void* (NULL = default
 * stream).  Every call is asynchronous on `stream` and returns 0 on success,
 * a hipError_t value on a HIP failure, or WGBM_EINVAL / WGBM_ENOMEM; the
 * message is available from wgbm_last_error() (thread-local).  Calls never
 * print, and they validate shapes and ranges before launching anything.
 *
 * Arithmetic contract (see the reference semantics cited at each entry):
 *  - histogram gradient sums are exact sums of the residuals quantised to
 *    q = rint(r * 2^s) with a power-of-two scale s chosen from a maximum
 *    |r| M (at most 28 significant bits per value), rounded once to
 *    float32; counts are exact.  Results do not depend on row order or
 *    launch shape.  M is taken per output block: the whole call when it has
 *    one segment and one era, else each segment / each era separately (an
 *    era or segment of small residuals keeps its precision next to another
 *    one's outliers).  Within one such block a bin's error is at most
 *    count * M * 2^-29, so a bin that holds only residuals far below M (e.g.
 *    1e-3 values in the same era as a 1e6 one) can lose them, where the
 *    reference's float32 atomics keep ~24 bits of that bin's own scale.  A
 *    non-finite residual makes its block's sums NaN.
 *  - split gains/directions are bit-identical to a sequential float32 scan.
 *  - predictions add trees in tree order (deterministic).
 */
#ifndef WARPGBM_AMD_H
#define WARPGBM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WGBM_EINVAL 1000
#define WGBM_ENOMEM 1001

/* Library version string. */
const char* wgbm_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char* wgbm_last_error(void);

/* ------------------------------------------------------------------------
 * Reference-compatible operators.  Each replaces one function bound by the
 * reference's pybind module (warpgbm/cuda/node_kernel.cpp:41-47).
 * ------------------------------------------------------------------------ */

/* compute_histogram3 -- replaces launch_histogram_kernel_cuda_configurable
 * (warpgbm/cuda/histogram_kernel.cu:63-104, bound at node_kernel.cpp:43).
 * For each position p < n_samples, row s = sample_indices[p], era
 * e = era_indices[s] (ignored when num_eras == 1), and each output feature
 * f < n_feats with code b = bin_indices[s * n_feats_master + feature_indices[f]]:
 * if 0 <= b < num_bins:  grad_hist[e,f,b] += residual[s];  hess_hist[e,f,b] += 1.
 * grad_hist / hess_hist: float32 [num_eras, n_feats, num_bins], ACCUMULATED
 * into (the caller zeroes them, as the reference's caller does).  Rows whose
 * era is outside [0, num_eras) are skipped, and so are feature indices
 * outside [0, n_feats_master) (their outputs keep their values; the
 * reference reads such codes out of bounds).  Only the selected columns are
 * histogrammed (in any order, repeats allowed).  threads_per_block and
 * rows_per_thread are accepted for signature compatibility and ignored. */
int wgbm_compute_histogram3(const int8_t* bin_indices, int64_t n_rows, int64_t n_feats_master,
                            const float* residuals, const int32_t* sample_indices,
                            int64_t n_samples, const int32_t* feature_indices, int64_t n_feats,
                            const int32_t* era_indices, int32_t num_eras, float* grad_hist,
                            float* hess_hist, int32_t num_bins, int32_t threads_per_block,
                            int32_t rows_per_thread, void* stream);

/* compute_split -- replaces launch_directional_split_kernel
 * (warpgbm/cuda/best_split_kernel.cu:61-88, bound at node_kernel.cpp:42).
 * G, H: float32 [num_eras, n_feats, num_bins]; per_era_gain and
 * per_era_direction: float32 [num_eras, n_feats, num_bins - 1], overwritten.
 * min_split_gain is accepted and unused, as in the reference kernel. */
int wgbm_compute_split(const float* G, const float* H, int32_t num_eras, int32_t n_feats,
                       int32_t num_bins, float min_split_gain, float min_child_samples,
                       float eps, float* per_era_gain, float* per_era_direction,
                       int32_t threads, void* stream);

/* custom_cuda_binner -- replaces launch_bin_column_kernel
 * (warpgbm/cuda/binner.cu:27-52, bound at node_kernel.cpp:44).
 * bin_indices[i] = number of leading edges with X[i] >= edge (NaN -> 0). */
int wgbm_custom_cuda_binner(const float* X, int64_t n, const float* bin_edges, int32_t n_edges,
                            int8_t* bin_indices, void* stream);

/* predict_forest -- replaces predict_with_forest (warpgbm/cuda/predict.cu:48-76,
 * bound at node_kernel.cpp:45).  tree_tensor: float32 [n_trees, max_nodes, 6]
 * rows (feature, bin, left, right, is_leaf, leaf_value) as written by the
 * reference's flatten_tree; out[i] += learning_rate * leaf, trees added in
 * tree order.  A walk that leaves the table contributes NaN. */
int wgbm_predict_forest(const int8_t* bin_indices, int64_t n, int64_t n_feats,
                        const float* tree_tensor, int64_t n_trees, int64_t max_nodes,
                        float learning_rate, float* out, void* stream);

/* ------------------------------------------------------------------------
 * Batched entry points (no single reference counterpart; each batches the
 * per-node / per-feature / per-tree reference calls named in its comment).
 * ------------------------------------------------------------------------ */

/* Native code layout: codes written by wgbm_bin_matrix (num_bins = n_edges
 * + 1) or wgbm_copy_prebinned (for num_bins).  Every byte of every row is in
 * [0, num_bins + 1]: a code c in [0, num_bins) is stored as c, a negative
 * code as num_bins, a code >= num_bins and every padding byte as
 * num_bins + 1.  The column-major copy keeps the raw codes. */
#define WGBM_CODES_NATIVE 1

/* Multi-segment histogram: the positions order[seg[k] .. seg[k+1]) are the
 * rows of segment k (a node; cf. the per-node sample_indices of
 * warpgbm/core.py:551-562).  codes: int8 [n_rows, stride] row-major,
 * features 0..n_feats-1; codes outside [0, num_bins) are skipped.  flags:
 * 0 for any int8 codes, or WGBM_CODES_NATIVE when the codes are in the native
 * layout for this num_bins (a faster kernel that relies on every byte being
 * in [0, num_bins + 1]).  G, H: float32 [n_seg, n_feats, num_bins],
 * accumulated into.  seg is a device int64 array [n_seg + 1]; n_pos is
 * seg[n_seg] (known to the caller). */
int wgbm_histogram_segments(const int8_t* codes, int64_t n_rows, int64_t stride, int32_t n_feats,
                            const float* residuals, const int32_t* order, const int64_t* seg,
                            int32_t n_seg, int64_t n_pos, int32_t num_bins, int32_t flags,
                            float* G, float* H, void* stream);

/* wgbm_histogram_segments that allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same arguments and results as wgbm_histogram_segments; the
 * call's working memory (tile plan, partial histograms, gathered residuals)
 * is a fixed device array of WGBM_NOALLOC_SCRATCH_BYTES that every GPU the
 * library runs on holds until the process ends.  A call needing more (about
 * 4 bytes per row of a row list plus 256 KiB per histogram tile of 1000
 * features at 32 bins; the 1M x 1000 root and 16-node calls need 32 and
 * 40 MiB)
 * returns WGBM_EINVAL with the sizes in wgbm_last_error().  Calls that
 * overlap on one GPU (other streams, other threads) share the array and
 * race: serialise them. */
#define WGBM_NOALLOC_SCRATCH_BYTES (64 * 1024 * 1024)
int wgbm_histogram_segments_noalloc(const int8_t* codes, int64_t n_rows, int64_t stride,
                                    int32_t n_feats, const float* residuals, const int32_t* order,
                                    const int64_t* seg, int32_t n_seg, int64_t n_pos,
                                    int32_t num_bins, int32_t flags, float* G, float* H,
                                    void* stream);

/* Quantile edges (the torch.quantile call of warpgbm/core.py:529-534) from
 * columns already sorted ascending (NaN last): sorted float32 [n_feats, n];
 * q float32 [nq]; edges float32 [n_feats, nq]. */
int wgbm_quantile_edges(const float* sorted, int64_t n, int32_t n_feats, const float* q,
                        int32_t nq, float* edges, void* stream);

/* Quantile edges of every column of X float32 [n, n_feats] (row stride
 * x_stride elements) without sorting: the order statistics torch.quantile
 * interpolates between are found by radix selection (4 passes over an
 * order-preserving key of each column), then interpolated as above.
 * Bit-identical to torch.quantile(X[:, f], q); n <= 2^24. */
int wgbm_quantile_edges_matrix(const float* X, int64_t n, int32_t n_feats, int64_t x_stride,
                               const float* q, int32_t nq, float* edges, void* stream);

/* wgbm_quantile_edges_matrix in two steps, for a matrix that reaches the
 * device in row blocks (the staged upload of warpgbm/core.py:527-534's input,
 * whose torch.quantile call needs the whole column): each block's values are
 * staged as soon as it lands, the edges taken once every row is staged.
 *
 * stage_rows: rows [row0, row0 + rows) of the matrix, X pointing at the first
 * of them (row stride x_stride elements), into the column-major staging array
 * cols uint32 [n_feats][cols_stride] at column offset row0, and the running
 * per-column extremes kmin / kmax uint32 [n_feats] (order-preserving keys;
 * the caller sets them to 0xffffffff / 0 before the first block).  row0 is a
 * multiple of 4; cols_stride is a multiple of 32 and at least the final row
 * count n.  Blocks may be staged in any order, on one stream.
 * edges_staged: the edges of all n staged rows, bit-identical to
 * wgbm_quantile_edges_matrix on the whole matrix.  n <= 2^24. */
int wgbm_quantile_stage_rows(const float* X, int64_t rows, int32_t n_feats, int64_t x_stride,
                             int64_t row0, uint32_t* cols, int64_t cols_stride, uint32_t* kmin,
                             uint32_t* kmax, void* stream);
int wgbm_quantile_edges_staged(const uint32_t* cols, int64_t n, int32_t n_feats,
                               int64_t cols_stride, const uint32_t* kmin, const uint32_t* kmax,
                               const float* q, int32_t nq, float* edges, void* stream);

/* Batched binner (the per-feature loop of warpgbm/core.py:527-538 and
 * 908-913 in one launch).  X float32 [n, n_feats] with row stride x_stride
 * (elements); edges float32 [n_feats, n_edges] sorted per feature.  Writes
 * codes_rm int8 [n, codes_stride] in the native layout for num_bins =
 * n_edges + 1 (codes in [0, n_edges], padding bytes n_edges + 2) and, if
 * codes_cm is not NULL, codes_cm int8 [n_feats, n] (column-major copy). */
int wgbm_bin_matrix(const float* X, int64_t n, int32_t n_feats, int64_t x_stride,
                    const float* edges, int32_t n_edges, int8_t* codes_rm, int64_t codes_stride,
                    int8_t* codes_cm, void* stream);

/* Pre-binned int8 input (warpgbm/core.py:502-505): copy [n, n_feats] with
 * row stride x_stride bytes into the native row-major layout for num_bins
 * (2..127) and the raw column-major copy, as wgbm_bin_matrix.  If over_flag
 * (one int32 on the device) is not NULL it ends as 1 when some value is
 * >= num_bins, else 0: the reference's "every column max < num_bins" test
 * (core.py:501-503) made in the same pass. */
int wgbm_copy_prebinned(const int8_t* X, int64_t n, int32_t n_feats, int64_t x_stride,
                        int8_t* codes_rm, int64_t codes_stride, int8_t* codes_cm,
                        int32_t num_bins, int32_t* over_flag, void* stream);

/* Single-launch ensemble inference over heap-ordered trees (replaces the
 * per-tree launches of warpgbm/core.py:1010-1026 and the single launch of
 * :928-930).  Tree t = round * K + k, node h has children 2h+1 / 2h+2;
 * feat[t*H + h] >= 0 splits on that feature (left if code <= bin), -1 is a
 * leaf with value leaf[t*H + h].  out float32 [n, K] row-major, pre-filled
 * with the initial scores; tree contributions added round by round.  codes:
 * native layout for num_bins (negative codes go left, codes >= num_bins go
 * right, as the raw int8 compare of the reference). */
int wgbm_predict_heap(const int8_t* codes, int64_t n, int64_t codes_stride, int32_t num_bins,
                      const int32_t* feat, const int32_t* bin, const float* leaf,
                      int32_t n_rounds, int32_t K, int32_t H, int32_t max_depth,
                      float learning_rate, float* out, void* stream);

/* In-place row softmax of float32 [n, K] (warpgbm/metrics.py:12-15). */
int wgbm_softmax_rows(float* x, int64_t n, int32_t K, void* stream);

/* Per-era split-gain importance (replaces the per-node .item() loop of
 * warpgbm/core.py:624-627): acc float32 [num_eras, n_feats] (device, in/out)
 * gets acc[e][f] += gain[node[i] * num_eras + e] for i in [feat_start[f],
 * feat_start[f+1]), one float32 add after the other in that order.  gain:
 * float32 rows of num_eras per node; node: int64 gain-row indices grouped by
 * feature, each group in the order the reference visits the nodes (trees in
 * order, nodes depth-first, left first); feat_start: int64 [n_feats + 1]. */
int wgbm_importance_add(float* acc, int32_t n_feats, int32_t num_eras, const float* gain,
                        const int64_t* node, const int64_t* feat_start, void* stream);

/* ------------------------------------------------------------------------
 * Level-wise boosting engine (the caller of the four operators:
 * warpgbm/core.py grow_forest 692-744, grow_forest_multiclass 746-818,
 * grow_tree 597-658).
 * ------------------------------------------------------------------------ */
typedef struct wgbm_engine wgbm_engine;

typedef struct wgbm_engine_config {
  int64_t n_rows;
  int32_t n_feats;
  int64_t codes_stride;       /* multiple of 16, >= n_feats */
  int32_t num_bins;           /* 2..127 */
  int32_t num_eras;
  int32_t max_depth;
  int32_t n_trees;            /* 1 (regression) or K (softmax) */
  int32_t objective;          /* 0 regression, 1 softmax */
  float min_child_weight;
  float min_split_gain;
  float l2_reg;
  float learning_rate;
  const int8_t* codes_rm;     /* [n_rows, codes_stride], native layout */
  const int8_t* codes_cm;     /* [n_feats, n_rows] */
  const int32_t* root_order;  /* [n_rows] row ids sorted by era, ascending inside */
  const int64_t* era_start;   /* [num_eras + 1] */
  /* device bytes for the per-level split buffers (level histograms, staged
   * per-era gains, era-block sums, criteria); 0 = 4 GiB.  A depth with more
   * (tree, node)s than fit is processed in chunks of nodes, each histogrammed
   * directly; the trees do not depend on it.  max_depth is limited only by
   * int32 node and segment numbering (n_trees * 2^max_depth * num_eras <
   * 2^31) and by the device memory of the per-node bookkeeping, which
   * wgbm_engine_create checks against the free memory. */
  int64_t level_bytes;
} wgbm_engine_config;

/* Heap-ordered record of the trees grown in one round; H = 2^(max_depth+1)-1.
 * feat: split feature, -1 leaf, -2 absent; count: rows in the node;
 * gain: per-era gains of the chosen split [n_trees, H, num_eras]. */
typedef struct wgbm_tree_record {
  int32_t* feat;   /* [n_trees, H] */
  int32_t* bin;    /* [n_trees, H] */
  float* leaf;     /* [n_trees, H] */
  int64_t* count;  /* [n_trees, H] */
  float* gain;     /* [n_trees, H, num_eras] */
  int32_t H;
} wgbm_tree_record;

int wgbm_engine_create(wgbm_engine** out, const wgbm_engine_config* cfg);
/* One boosting round.  target: float32 y [n_rows] (regression) or int32
 * labels [n_rows] (softmax); pred: float32 [n_rows] (regression) or
 * class-major [K, n_rows] (softmax: the scores of class k are row k, so each
 * class tree's leaf updates stay inside one row), updated in place;
 * feat_sel: int32 [n_sel] features of this round's trees (colsample_bytree
 * subset, local order). */
int wgbm_engine_round(wgbm_engine* eng, const void* target, float* pred, const int32_t* feat_sel,
                      int32_t n_sel, const wgbm_tree_record* rec, void* stream);
/* Tuning knobs: key 1 = histogram tile rows (0 = automatic); key 2 = codes
 * read by the era path when num_bins <= 7 (0 = the int8 codes, 1 = a
 * pair-code copy, one byte per feature pair; default 1); key 3 = the
 * per-level node scan of one-era fits (1 = a thread per node, default; 0 = a
 * wave per node); key 4 = one-era split search and leaf / record step (1 =
 * one fused launch, default; 0 = two launches); key 5 = the one-era root
 * (1 = its positions and totals in one launch and the root level's
 * histogram tiles planned once per engine, default; 0 = a root partition
 * pass, block scan and totals launch, and a plan per round); key 6 = the
 * one-era split levels' partition (1 = one pass that routes and places every
 * row, each node's children filled from its two ends, on levels of at most
 * 1024 (tree, node)s, default; 0 = route, block prefix and a stable
 * scatter); key 7 = the era levels' partition (1 = the route reserves each
 * (node, era) segment's child ranges and leaves its sums for the node scan,
 * no block prefix, default; 0 = route, block prefix, node scan, scatter).
 * Set before the first round; every setting grows the same trees. */
int wgbm_engine_set_tuning(wgbm_engine* eng, int32_t key, int64_t value);
void wgbm_engine_destroy(wgbm_engine* eng);

/* ------------------------------------------------------------------------
 * Instrumentation: HIP-event timing of selected kernels (tags
 * "hist_tiles", "engine_hist_tiles"; in mode 1 also the engine's era path
 * per depth d: "des_rows_L<d>", the per-era gain kernel, and "des_sums_L<d>",
 * the era sums, pick and finish).  mode 0 off; 1: events recorded on the
 * kernel's stream right before and after its launch; 2: events attached to
 * the kernel's dispatch (hipExtLaunchKernel).  Reading synchronises the
 * events.
 * ------------------------------------------------------------------------ */
void wgbm_timer_enable(int32_t mode);
int wgbm_timer_read(const char* tag, double* total_ms, int64_t* count);
void wgbm_timer_reset(void);
/* Rate of 64-bit LDS atomic adds (per second, whole GPU) in the tile
 * histogram's LDS layout with synthetic bins and no global traffic: the
 * ceiling of the histogram kernel's LDS stage.  Synchronises `stream`. */
int wgbm_probe_lds_atomics(int32_t blocks, int32_t iters, double* ops_per_s, void* stream);
/* Achievable HBM read rate (bytes per second, whole GPU): `iters` launches
 * that each stream the device buffer `buf` (16-byte aligned, `bytes` long;
 * the last bytes % 16 are not read) once with 16-byte loads and no other
 * memory traffic: the practical ceiling of a read-bound kernel.  No
 * counterpart in the reference.  Synchronises `stream`. */
int wgbm_probe_hbm_read(const void* buf, int64_t bytes, int32_t iters, double* bytes_per_s,
                        void* stream);
/* Free the library's scratch buffers (all devices / streams). */
void wgbm_release_scratch(void);

#ifdef __cplusplus
}
#endif

#endif /* WARPGBM_AMD_H */
