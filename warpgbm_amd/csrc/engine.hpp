// Level-wise tree engine (internal C++ interface).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kernels.hpp"

namespace wgbm {

// Tree record in heap order (node h has children 2h+1, 2h+2), per tree of a
// round: H = 2^(max_depth+1) - 1 slots.  feat: global split feature, -1 leaf,
// -2 absent.  gain: per-era split gains [H][E] (importance bookkeeping).
struct TreeRecord {
  int32_t* feat;
  int32_t* bin;
  float* leaf;
  int64_t* count;
  float* gain;
  int32_t H;
};

struct EngineConfig {
  int64_t n_rows;
  int32_t n_feats;
  int64_t stride;          // row stride of codes_rm (bytes)
  int32_t num_bins;
  int32_t num_eras;
  int32_t max_depth;
  int32_t n_trees;         // trees grown together per round (1 or K)
  int32_t objective;       // 0 regression, 1 softmax
  float min_child_weight;
  float min_split_gain;
  float l2_reg;
  float learning_rate;
  const int8_t* codes_rm;  // [n_rows, stride]
  const int8_t* codes_cm;  // [n_feats, n_rows]
  const int32_t* root_order;  // [n_rows] rows sorted by era (ascending row id inside)
  const int64_t* era_start;   // [E + 1]
  int64_t level_bytes;        // per-level split buffers (0: default)
};

struct Engine;
int engine_create(Engine** out, const EngineConfig& cfg);
void engine_destroy(Engine* e);
// One boosting round.  target: float y [n] (regression) or int32 labels
// (softmax).  pred: [n] or [n, K] row-major, updated in place.
int engine_round(Engine* e, const void* target, float* pred, const int32_t* feat_sel,
                 int32_t n_sel, const TreeRecord& rec, hipStream_t st);
int engine_set_tuning(Engine* e, int key, int64_t value);

// kernels (engine_kernels.hip)
__global__ void residual_regression_kernel(const float* y, const float* pred, int64_t n,
                                           float* r, uint32_t* partial);
__global__ void residual_softmax_kernel(const float* logits, const int32_t* label, int64_t n,
                                        int32_t K, float* r, uint32_t* partial);
__global__ void root_setup_kernel(const int32_t* root_order, int64_t n, int32_t T,
                                  const int64_t* era_start, int32_t E, const float* resid,
                                  int32_t* order, int32_t* keyp, float* rpos, int64_t* seg,
                                  int32_t* present, unsigned long long* best, int32_t* agree_max,
                                  const int32_t* shifts, int32_t* node_shift);
constexpr int kRootE1Span = 4096;  // positions per workgroup of root_setup_e1_kernel
__global__ void root_setup_e1_kernel(const int32_t* root_order, int64_t n, int32_t T,
                                     const float* resid, int32_t* order, int32_t* keyp,
                                     float* rpos, int64_t* seg, int32_t* present,
                                     unsigned long long* best, const int32_t* shifts,
                                     int32_t s63_add, int32_t* node_shift, int64_t* tot_qh,
                                     int64_t* tot_ql);
// What the partition needs of a (tree, node) of the level, written by
// level_finish_kernel: col = the split's code column (-1: the node is a
// leaf, -2: absent), bin = the split bin, leaf = the leaf value, s63 = the
// wide leaf-sum shift of the node's tree.  One 16-byte load per position.
struct alignas(16) NodeRoute {
  int32_t col;
  int32_t bin;
  float leaf;
  int32_t s63;
};
__global__ void level_finish_kernel(int32_t depth, int32_t max_depth, int32_t T, int32_t E,
                                    int32_t B, const int32_t* present,
                                    const unsigned long long* best, int32_t* split_l,
                                    int32_t* split_b, const float* split_gain_era,
                                    const int32_t* feat_sel, const int64_t* tot_qh,
                                    const int64_t* tot_ql, const int64_t* tot_c,
                                    const int32_t* shifts, int32_t s63_add,
                                    float* leaf_val, TreeRecord rec,
                                    unsigned long long* best_next, int32_t* agree_max_next,
                                    NodeRoute* nroute);
// partition over position blocks (engine_kernels.hip)
constexpr int kPartBlock = 1024;   // positions per block
constexpr int kPartThreads = 256;
// Per-level left sums of the partition (see route_kernel): words of the
// segments that lie inside one block, the first- and last-segment partials of
// every block and their inclusive prefix over the blocks.  A residual sum is
// two words, qh = sum of (q63 >> 32) and ql = sum of (q63 & (2^32 - 1)), with
// q63 the wide quantisation of the leaf sums (sum q63 = qh * 2^32 + ql).
// Node maxima of |residual| of the left and right rows of every split node
// (float bits), per node: words of nodes inside one block, and the block's
// first- and last-node partials.
struct PartSums {
  int64_t* own_qh;  // [n_keys]
  int64_t* own_ql;
  int32_t* own_n;
  int64_t* bf_qh;  // [nb]
  int64_t* bf_ql;
  int32_t* bf_n;
  int64_t* bl_qh;
  int64_t* bl_ql;
  int32_t* bl_n;
  int64_t* P_qh;
  int64_t* P_ql;
  int64_t* P_n;
  uint32_t* own_ml;  // [keys] left-child max|r| of a segment inside one block
  uint32_t* own_mr;  //        right-child max
  uint32_t* bf_ml;   // [nb] of the block's first segment
  uint32_t* bf_mr;
  uint32_t* bl_ml;   // [nb] of the block's last segment
  uint32_t* bl_mr;
  int32_t* bf_node;  // [nb] segment key of the block's first position (one era: its node)
  uint32_t* pm_l;    // [nb] segmented maxima of bf_ml / bf_mr over runs of
  uint32_t* pm_r;    //      blocks with one first segment (block_scan_body)
};

// A child node keeps its parent's histogram shift unless the shift of its
// own max|r| is at least this much larger (all its residuals below 2^-8 of
// the parent's scale); then it takes its own, and both children of that
// split are histogrammed directly instead of one by subtraction.
constexpr int kNodeShiftStep = 8;
__device__ inline int node_shift_rule(uint32_t absmax_bits, int parent_shift,
                                               int qbits) {
  if (absmax_bits >= 0x7f800000u) return parent_shift;  // inf / NaN residuals
  const int s_own = wgbm_shift_from_absmax(__uint_as_float(absmax_bits), qbits);
  return s_own - parent_shift >= kNodeShiftStep ? s_own : parent_shift;
}
// Several eras: the histogram shift of one (node, era) segment from the
// float bits of its largest |residual| (0 for an empty, all-zero or
// non-finite segment)
__device__ inline int key_shift_of(uint32_t absmax_bits, int qbits) {
  return wgbm_shift_from_bits(absmax_bits, qbits);
}
// Per-segment words of the partitions that reserve child ranges
// (partition_e1_kernel for one era, route_kernel with kw set for several):
// what a split segment's rows add to its children (row counts of both, the
// left rows' wide residual sums, both children's max|r|).  Zero outside a
// level's partition -> scan window: the level's scan reads and clears them.
struct KeyWords {
  unsigned long long* cnt;  // left rows * 2^32 + right rows
  int64_t* qh;              // left rows' sum of (q63 >> 32)
  int64_t* ql;              // left rows' sum of (q63 & (2^32 - 1))
  uint32_t* ml;             // left rows' max|r| (float bits)
  uint32_t* mr;             // right rows' max|r|
};
struct RouteArgs {
  int32_t mode;  // 0 root totals, 1 split level, 2 last level (leaves only)
  int32_t want_max;  // gather each segment's left / right max|r| (the next level's shifts)
  const int64_t* seg;
  int32_t n_keys;
  int64_t n_pos;
  const int32_t* order;
  int32_t E, nodes;
  const int32_t* present;
  const int32_t* split_l;
  const int32_t* split_b;
  const int32_t* feat_sel;
  const int8_t* codes_cm;
  int64_t n;
  const float* rpos;  // residual of every position's row
  const int32_t* shifts;  // per tree
  int32_t s63_add;        // wide leaf-sum shift = shifts[t] + s63_add
  const float* leaf_val;
  const NodeRoute* nroute;  // modes 1, 2: the level's nodes (level_finish_kernel)
  float lr;
  float* pred;
  int64_t pstride, pcol;
  uint8_t* dirbit;
  const int32_t* keyp;  // segment key of every position
  PartSums ps;
  int32_t xcd_order;  // mode 2: blocks in the XCD work order (grid wgbm_xcd_grid)
  // mode 1 with kw.cnt set (several eras): the segments' words go to kw
  // instead of the block partials, a segment crossing the block's edges
  // reserves the block's part of its children's ranges (res[2 b] for the
  // block's first segment, res[2 b + 1] for its last: left * 2^32 + right
  // rows of the segment in earlier-reserving blocks), and no block prefix is
  // needed
  KeyWords kw;
  unsigned long long* res;
};
__global__ void route_kernel(RouteArgs a);
// dynamic LDS of route_kernel: the slot sums, plus the node maxima
inline size_t route_lds_bytes(const RouteArgs& a) {
  if (a.mode == 2) return 0;
  return (size_t)kPartBlock * (16 + (a.want_max ? 8 : 0));
}
__global__ void block_scan_kernel(int32_t nb, PartSums ps);
constexpr int kLevelScanMaxNodes = 64;  // (tree, node)s of a level for level_scan_kernel
// Per split level: the children's segments and totals, their histogram
// shifts (node_shift_rule from the node maxima) and the histogram key list of
// the next level, two entries per (parent, era): the smaller child and -1
// (the sibling by subtraction), or both children when a child's shift
// differs from the parent's.
struct LevelNext {
  const int64_t* tot_qh;
  const int64_t* tot_ql;
  // histogram shifts of this level: one era [T * nodes], several eras per
  // (node, era) key [T * nodes * E]
  const int32_t* node_shift;
  int32_t qbits;
  int32_t have_max;  // the route gathered the children's max|r| (else no shift changes)
  int64_t* seg_next;
  int64_t* tot_qh_next;
  int64_t* tot_ql_next;
  int64_t* tot_c_next;
  int32_t* present_next;
  int32_t* key_list_next;   // [2 * T * nodes * E]
  int32_t* node_shift_next;  // the next level's, indexed likewise
  // node_scan_kernel: the next level's live-era masks (des_alive_kernel's
  // output for the children, [2 * T * nodes][ceil(E / 32)]), or null
  uint32_t* alive_next;
  float mcw;
};
__global__ void level_scan_kernel(int32_t nb, PartSums ps, int32_t T, int32_t nodes, int32_t E,
                                  int64_t n_pos, const int64_t* seg, const int32_t* present,
                                  const int32_t* split_l, LevelNext nx, int32_t n_list,
                                  int32_t tile_rows, int32_t max_tiles, Tile* tiles,
                                  int32_t* key_tile_start, int32_t* n_tiles);
// One-era split levels in one pass: route, rank and place every position
// (route_kernel + scatter_kernel without the block prefix between them), for
// levels of at most kPartition1MaxNodes (tree, node)s.
constexpr int kPartition1MaxNodes = 1024;
// Nodes that span many blocks make the blocks that share them queue on their
// words' atomics: levels whose nodes average more than kPartition1WideSpan
// positions take blocks of 4096 positions (a quarter of the blocks).
constexpr int64_t kPartition1WideSpan = 16 * 1024;
template <int NT>  // threads per block: 4 NT positions
__global__ void partition_e1_kernel(RouteArgs a, KeyWords kw, int32_t n_slots,
                                    int32_t* order_next, int32_t* keyp_next, float* rpos_next,
                                    int32_t* leaf_key);
// the last level's leaf updates by row, from the rows' leaf keys
__global__ void leaf_rows_kernel(const int32_t* leaf_key, int64_t n, int32_t T,
                                 const NodeRoute* nroute, float lr, float* pred, int64_t pstride,
                                 int64_t pcol);
// its dynamic LDS: 28 bytes per (tree, node) slot
inline size_t partition1_lds_bytes(int64_t n_slots) { return (size_t)n_slots * 28; }
// One-era levels: level_scan_kernel's work with a thread per (tree, node),
// up to kLevelScanE1MaxNodes of them, and the next level's tile plan.  With
// kw.cnt set, the children's counts, sums and maxima come from the
// single-pass partition's words (no block prefix; the words are cleared).
constexpr int kLevelScanE1MaxNodes = 2048;
__global__ void level_scan_e1_kernel(int32_t nb, PartSums ps, KeyWords kw, int32_t n_tn,
                                     int64_t n_pos, const int64_t* seg, const int32_t* present,
                                     const int32_t* split_l, LevelNext nx, int32_t plan,
                                     int32_t tile_rows, int32_t max_tiles, Tile* tiles,
                                     int32_t* key_tile_start, int32_t* n_tiles);
__global__ void root_totals_kernel(int32_t n_keys, const int64_t* seg, PartSums ps,
                                   int64_t* tot_qh, int64_t* tot_ql, int64_t* tot_c,
                                   int32_t qbits, int32_t* key_shift);
// with kw.cnt set (several eras): the segments' words come from the route's
// kw words (no block prefix), and are cleared
__global__ void node_scan_kernel(int32_t T, int32_t nodes, int32_t E, int32_t wpn,
                                 int64_t n_pos, const int64_t* seg, const int32_t* present,
                                 const int32_t* split_l, PartSums ps, LevelNext nx, KeyWords kw);
// with res set: the ranks of a segment crossing the block's edges start at
// the route's reserved bases (RouteArgs::res) instead of the block prefix
__global__ void scatter_kernel(int64_t n_pos, int32_t E, const int64_t* seg,
                               const int64_t* seg_next, const int32_t* keyp,
                               const uint8_t* dirbit, PartSums ps, const int32_t* order,
                               int32_t* order_next, int32_t* keyp_next, const float* rpos,
                               float* rpos_next, const unsigned long long* res);
__global__ void fill_i32_kernel(int32_t* p, int64_t n, int32_t v);
// histogram keys of a chunk of n (tree, node)s: list[i] = i when node i / E
// is present, else -1 (keys relative to the chunk's first node)
__global__ void chunk_keys_kernel(const int32_t* present, int32_t E, int32_t n, int32_t* list);

// split kernels (split.hip); node_shift: the histogram shift of every
// (tree, node) of the level, indexed by tree * nodes_in_level + node
// per-era gains and directions of every (era, feature) (the drop-in op;
// split_f32_kernel, a compile-time bin count for common B)
int launch_split_f32(const float* G, const float* H, int32_t E, int32_t F, int32_t B, float mcw,
                     float eps, float* gain_out, float* dir_out, hipStream_t st);
// split_level_e1_kernel over n_tn tree-nodes (a compile-time bin count for B = 32)
int launch_split_level_e1(int n_tn, hipStream_t st, const int64_t* hq, const int32_t* hc,
                          int32_t F, int32_t B, const int32_t* feat_sel, int32_t n_sel,
                          int32_t nodes_in_level, const int32_t* present,
                          const int32_t* node_shift, float mcw, float eps, float min_split_gain,
                          unsigned long long* best);
// What the leaf / record step of a one-era level needs besides the pick
// (level-wide arrays, indexed by the node's index in the level).
struct FinishE1 {
  int32_t depth, max_depth, T, B;
  const int32_t* present;
  int32_t* split_l;
  int32_t* split_b;
  const int32_t* feat_sel;
  const int64_t* tot_qh;
  const int64_t* tot_ql;
  const int64_t* tot_c;
  const int32_t* shifts;
  int32_t s63_add;
  float* leaf_val;
  TreeRecord rec;
  unsigned long long* best_next;
  NodeRoute* nroute;
};
// split_level_e1_kernel fused with the level's leaf / record step (one era):
// nodes c0 .. c0 + n_tn - 1 of the level; hq / hc hold the chunk's nodes from
// 0.  A node searched by several workgroups is finished by the last of them
// (done: per-node arrival counters, zero between launches).
int launch_split_finish_e1(int n_tn, int32_t c0, hipStream_t st, const int64_t* hq,
                           const int32_t* hc, int32_t F, int32_t n_sel,
                           const int32_t* node_shift, float mcw, float eps,
                           float min_split_gain, unsigned long long* best, uint32_t* done,
                           const FinishE1& fa);
__global__ void des_accumulate_kernel(const int64_t* hq, const int32_t* hc, int32_t F, int32_t B,
                                      int32_t E, const int32_t* feat_sel, int32_t n_sel,
                                      int32_t nodes_in_level, int32_t n_tn,
                                      const int32_t* present, const int32_t* node_shift,
                                      float mcw, float eps, float* crit, int32_t* agree,
                                      int32_t* agree_max);
__global__ void des_pick_kernel(const float* crit, const int32_t* agree, const int32_t* agree_max,
                                const int32_t* present, int32_t n_tn, int64_t ncand,
                                float min_split_gain, unsigned long long* best);
__global__ void des_finish_kernel(const unsigned long long* best, const int64_t* hq,
                                  const int32_t* hc, int32_t F, int32_t B, int32_t E,
                                  const int32_t* feat_sel, int32_t nodes_in_level, int32_t n_tn,
                                  const int32_t* node_shift, float mcw, float eps,
                                  const float* staged,
                                  const int64_t* seg, int32_t n_sel, int32_t* split_l,
                                  int32_t* split_b, float* split_gain_era);
__global__ void des_alive_kernel(const int64_t* seg, int32_t E, int32_t n_tn, float mcw,
                                 uint32_t* alive);
__global__ void des_block_kernel(const float* gain, const int8_t* dir, int32_t E, int32_t n_tn,
                                 int64_t ncand, const int32_t* present, const uint32_t* alive,
                                 double* bsum, int8_t* bdir);
__global__ void des_combine_pick_kernel(const double* bsum, const int8_t* bdir, int32_t E,
                                        int32_t n_tn, int64_t ncand, const int32_t* present,
                                        const uint32_t* alive, float min_split_gain,
                                        int32_t* wg_agree, unsigned long long* wg_key,
                                        unsigned long long* best, uint32_t* done,
                                        const float* staged, const int64_t* seg, float mcw,
                                        int32_t nb, int32_t n_sel, int32_t* split_l,
                                        int32_t* split_b, float* split_gain_era);
__global__ void local_scatter_kernel(const int32_t* feat_sel, int32_t n_sel, int32_t F,
                                     int32_t* local_of);
// pcodes: the pair-code copy of the codes (num_bins <= 7; n_rows rows of
// pstride bytes, under 4 GiB) or null for the int8 codes
int launch_des_era(int V, int B, int32_t n_keys, hipStream_t st, const int8_t* codes,
                   int64_t stride, int32_t F, const float* rpos, const int32_t* node_shift,
                   const int32_t* order, const int64_t* seg, int32_t E, int32_t nodes_in_level,
                   const int32_t* present, const int32_t* local_of, int32_t n_sel, float mcw,
                   float eps, float* gain, int8_t* dir, const uint8_t* pcodes, int64_t n_rows,
                   int64_t pstride);
// levels whose mean (node, era) segment holds at least this many rows use
// the pair codes: below it the int8 kernel's smaller LDS tables keep more
// segments (and so more row loads) in flight per CU
constexpr int kDesPairMinRows = 96;
int launch_pack_pairs(hipStream_t st, const int8_t* codes, int64_t stride, int32_t F, int64_t n,
                      int32_t B, uint8_t* out, int64_t pstride);
// row stride of the pair codes: one byte per feature pair, whole 8-byte
// words of 8 pairs, rows 256-byte aligned
inline int64_t pair_stride(int32_t F) { return ((int64_t)(F + 15) / 16 * 8 + 255) / 256 * 256; }


// binning / predict kernels (bin_column_kernel: kBinColumnU values per thread)
__global__ void bin_column_kernel(const float* x, int64_t n, const float* edges,
                                  int32_t n_edges, int8_t* out);
// words per feature of bin_matrix_kernel's LDS edge lists (dynamic LDS =
// 4 * kBinTileFeats * this)
int bin_edge_stride(int32_t n_edges);
template <bool VEC>
__global__ void bin_matrix_kernel(const float* X, int64_t n, int32_t F, int64_t xs,
                                  const float* edges, int32_t n_edges, int8_t* codes_rm,
                                  int64_t S, int8_t* codes_cm);
__global__ void pad_codes_kernel(int8_t* codes_rm, int64_t n, int64_t S, int32_t from,
                                 int8_t value);
__global__ void copy_prebinned_kernel(const int8_t* X, int64_t n, int32_t F, int64_t xs,
                                      int8_t* codes_rm, int64_t S, int8_t* codes_cm,
                                      int32_t num_bins, int32_t* over);
__global__ void quantile_edges_kernel(const float* sorted, int64_t n, int32_t F,
                                      const float* q, int32_t nq, float* edges);
template <bool VEC>
__global__ void transpose_values_kernel(const float* X, int64_t n, int32_t F, int64_t xs,
                                      int64_t ks, uint32_t* keys, uint32_t* kmin,
                                      uint32_t* kmax);
__global__ void quantile_select_kernel(const uint32_t* keys, int64_t n, int64_t ks, int32_t F,
                                       const float* q, int32_t nq, float* edges,
                                       const uint32_t* kmin, const uint32_t* kmax,
                                       uint32_t* cbuf, int64_t ccap);
// skip / run_if (optional, null: none): device flags that switch a kernel
// off (skip nonzero) or on (run_if nonzero), for wgbm_predict_forest
__global__ void predict_table_kernel(const int8_t* codes, int64_t n, int64_t F,
                                     const float* table, int64_t T, int64_t M, float lr,
                                     float* out, const int32_t* run_if);
__global__ void flat_to_heap_kernel(const float* table, int64_t T, int64_t M, int64_t F,
                                    int32_t D, int32_t* feat, int32_t* bin, float* leaf,
                                    int32_t* fallback);
__global__ void predict_heap_kernel(const int8_t* codes, int64_t n, int64_t S, int32_t num_bins,
                                    const int32_t* feat, const int32_t* bin, const float* leaf,
                                    int32_t n_rounds, int32_t K, int32_t H, int32_t max_depth,
                                    float lr, float* out, const int32_t* skip);
__global__ void complete_tables_kernel(const int32_t* feat, const int32_t* bin, const float* leaf,
                                       int64_t T, int32_t D, int64_t S, float lr,
                                       uint32_t* cnode, float* cleaf);
__global__ void predict_rows_kernel(const int8_t* codes, int64_t n, int64_t S, int32_t num_bins,
                                    const uint32_t* cnode, const float* cleaf, int32_t n_rounds,
                                    int32_t K, int32_t max_depth, int32_t RB, int32_t TC,
                                    float* out, const int32_t* skip);
int predict_rows_plan(int64_t S, int32_t K, int32_t H, int32_t n_rounds, int32_t* RB_out,
                      int32_t* TC_out, size_t* lds_out);
template <bool RAW>
__global__ void predict_resident_kernel(const int8_t* codes, int64_t n, int64_t S,
                                        int32_t num_bins, const uint32_t* cnode,
                                        const float* cleaf, int32_t T, int32_t K,
                                        int32_t max_depth, int32_t RB, float* out,
                                        const int32_t* skip);
int predict_resident_plan(int64_t S, int32_t K, int32_t H, int32_t n_rounds, int32_t* RB_out,
                          size_t* lds_out, bool raw = false);
__global__ void softmax_rows_kernel(float* x, int64_t n, int32_t K);
__global__ void importance_add_kernel(float* acc, int32_t F, int32_t E, const float* gain,
                                      const int64_t* node, const int64_t* fstart);

}  // namespace wgbm
