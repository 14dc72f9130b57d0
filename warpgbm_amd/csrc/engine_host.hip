// Level-wise tree engine: host orchestration of one boosting round.
//
// The reference grows each tree depth-first with a host round trip per node
// (warpgbm/core.py:597-658: .item() at :594, :606, :627, boolean-mask
// compaction at :630).  The tree it builds does not depend on the visiting
// order: the residual is fixed for the whole tree (core.py:719) and each
// node's decision depends only on its own rows.  So the engine grows all
// nodes of a depth at once, for all trees of a round (the K class trees of a
// softmax round share their gradients, core.py:772), with every launch queued
// on one stream and no host synchronisation inside a round:
//   residuals -> shifts -> root segments/totals ->
//   for depth d: histograms of the smaller children (+ siblings by
//   subtraction; both children when one takes a finer histogram shift) ->
//   split/DES -> leaf values + record -> partition.
#include <stdio.h>

#include <algorithm>
#include <vector>

#include "common.hpp"
#include "engine.hpp"
#include "kernels.hpp"

namespace wgbm {

constexpr int kResidBlocks = 1024;  // workgroups of the residual kernels

struct Engine {
  EngineConfig c;
  int V = 16, n_chunks = 1, qbits = 28;
  int H = 1;
  // (tree, node)s the per-level split buffers hold: a depth with more is
  // processed in chunks of nodes, each histogrammed directly
  int64_t nc_max = 1;
  bool stored_prev = false;  // hq[previous depth] holds that whole level (for subtraction)
  int64_t hist_tile_rows = 0;  // 0: automatic
  int64_t n_keys_max = 0, max_htiles = 0, nb = 0;
  // buffers
  float* resid = nullptr;
  uint32_t* absmax = nullptr;
  int32_t* shifts = nullptr;
  int32_t* order[2] = {nullptr, nullptr};
  int64_t* seg[2] = {nullptr, nullptr};
  int64_t* totqh[2] = {nullptr, nullptr};  // wide leaf sums, two words (see PartSums)
  int64_t* totql[2] = {nullptr, nullptr};
  int64_t* totc[2] = {nullptr, nullptr};
  int32_t* present[2] = {nullptr, nullptr};
  // histogram shift per (tree, node) with one era, per (tree, node, era)
  // segment key with several eras
  int32_t* node_shift[2] = {nullptr, nullptr};
  int32_t* key_list[2] = {nullptr, nullptr};    // histogram key pairs per (parent, era)
  // partition over position blocks of kPartBlock positions
  uint8_t* dirbit = nullptr;            // [T*N] 0 left, 1 right, 2 stays
  int32_t* keyp[2] = {nullptr, nullptr};  // [T*N] segment key of each position
  float* rpos[2] = {nullptr, nullptr};    // [T*N] residual of each position's row
  PartSums ps{};  // partition's left sums (own words, block partials, prefix)
  Tile* htiles = nullptr;
  int32_t* hkts = nullptr;
  int32_t* hn = nullptr;
  unsigned long long* part = nullptr;
  uint32_t* abs_part = nullptr;
  int64_t part_words = 0;
  int64_t* hq[2] = {nullptr, nullptr};
  int32_t* hc[2] = {nullptr, nullptr};
  float* crit = nullptr;         // E > 1: per-candidate era-mean gain [tn][n_sel*(B-1)]
  int32_t* agree = nullptr;      // E > 1: per-candidate |sum of directions|
  int32_t* agree_max = nullptr;  // E > 1: per-node max agree, two depths (parity)
  // E > 1 with every era <= 65536 rows: per-era gains straight from LDS
  // histograms of every (node, era) segment (no per-era histogram arrays)
  bool des_direct = false;
  float* sgain = nullptr;       // staged per-era gains (des_stage_slot layout)
  int8_t* sdir = nullptr;       // staged per-era directions
  int32_t* wg_agree = nullptr;  // per-workgroup summaries of des_combine_pick_kernel
  unsigned long long* wg_key = nullptr;
  int32_t* local_of = nullptr;  // [F] local index in the round's subset, or -1
  // num_bins <= 7: pair-code copy of codes_rm for the era path (made by the
  // first round); des_codes 0 = read the int8 codes, 1 = pair codes (default)
  uint8_t* pcodes = nullptr;
  int64_t pstride = 0;
  bool pcodes_ready = false;
  int des_codes = 1;
  // one-era levels: 1 = level_scan_e1_kernel (a thread per node), 0 = the
  // wave-per-node kernels
  int lscan_e1 = 1;
  // one-era levels: 1 = split search and leaf / record step fused
  // (split_finish_e1_kernel), 0 = split_level_e1_kernel + level_finish_kernel
  int fuse_finish = 1;
  uint32_t* done = nullptr;  // [T * nodes_max] arrival counters (zero between launches)
  // one era: 1 = the root's words and totals in one launch (root_setup_e1_kernel)
  // and the root level's histogram tiles planned once (the root segments
  // are the same every round); 0 = root_setup + root route + block scan +
  // root totals and a plan per round
  int root_path = 1;
  // one era: 1 = split levels of at most kPartition1MaxNodes (tree, node)s
  // partitioned in one pass (partition_e1_kernel and the level scan over its
  // node words), 0 = route + level scan + scatter
  int part1 = 1;
  KeyWords kw{};  // [n_keys_max] each, zero between levels
  // several eras: 1 = levels scanned by node_scan_kernel reserve their
  // segments' child ranges in the route (kw words, res bases, no block
  // prefix), 0 = route + block prefix + node scan + scatter
  int part_era = 1;
  unsigned long long* res = nullptr;  // [2 nb] reserved bases of the blocks' first / last segments
  Tile* root_tiles = nullptr;     // the root level's tile plan (planned by the first round)
  int32_t* root_kts = nullptr;
  int32_t* root_hn = nullptr;
  int64_t root_tiles_cap = 0;
  bool root_tiles_ready = false;
  uint32_t* alive = nullptr;    // [tn][W] segments that can hold a split, W = ceil(E/32)
  double* bsum = nullptr;       // [tn][W][n_sel*(B-1)] era-block gain sums
  int8_t* bdir = nullptr;       // [tn][W][n_sel*(B-1)] era-block direction sums (|.| <= 32)
  int32_t* split_l = nullptr;
  int32_t* split_b = nullptr;
  NodeRoute* nroute = nullptr;  // [T*nodes] the level's route records
  float* split_gain = nullptr;
  float* leaf_val = nullptr;
  unsigned long long* best = nullptr;  // packed split picks, two depths (parity)
  int64_t pick_stride = 0;             // words per depth in best / agree_max
  std::vector<void*> allocs;
  // one allocation for the buffers sized at creation (hipMalloc and hipFree
  // cost ~5 and ~20 us each here: ~60 buffers took ~1.5 ms per fit)
  char* arena = nullptr;
  size_t arena_size = 0, arena_used = 0;
};

template <typename T>
static int dalloc(Engine* e, T** p, int64_t n) {
  if (n < 1) n = 1;
  // from the engine's arena while it has room (256-byte aligned pieces)
  const size_t bytes = ((size_t)n * sizeof(T) + 255) / 256 * 256;
  if (e->arena && e->arena_used + bytes <= e->arena_size) {
    *p = (T*)(e->arena + e->arena_used);
    e->arena_used += bytes;
    return 0;
  }
  void* q = nullptr;
  hipError_t err = hipMalloc(&q, (size_t)n * sizeof(T));
  if (err != hipSuccess) {
    wgbm_set_error("engine: hipMalloc of %lld bytes failed: %s", (long long)(n * sizeof(T)),
                   hipGetErrorString(err));
    return WGBM_ENOMEM;
  }
  e->allocs.push_back(q);
  *p = (T*)q;
  return 0;
}

#define E_ALLOC(ptr, n)                      \
  do {                                       \
    int _r = dalloc(e, &(ptr), (int64_t)(n)); \
    if (_r) {                                \
      engine_destroy(e);                     \
      return _r;                             \
    }                                        \
  } while (0)

void engine_destroy(Engine* e) {
  if (!e) return;
  for (void* p : e->allocs) (void)hipFree(p);
  delete e;
}

int engine_create(Engine** out, const EngineConfig& cfg) {
  WGBM_REQUIRE(cfg.n_rows > 0 && cfg.n_rows < (int64_t(1) << 31), "engine: n_rows out of range");
  WGBM_REQUIRE(cfg.n_feats > 0, "engine: n_feats must be positive");
  WGBM_REQUIRE(cfg.stride >= cfg.n_feats && cfg.stride % 16 == 0,
               "engine: codes stride must be >= n_feats and a multiple of 16");
  WGBM_REQUIRE(cfg.num_bins >= 2 && cfg.num_bins <= 127, "engine: num_bins must be in [2, 127]");
  WGBM_REQUIRE(cfg.num_eras >= 1, "engine: num_eras must be >= 1");
  WGBM_REQUIRE(cfg.max_depth >= 1 && cfg.max_depth <= 29, "engine: max_depth must be in [1, 29]");
  WGBM_REQUIRE(cfg.n_trees >= 1, "engine: n_trees must be >= 1");
  WGBM_REQUIRE(cfg.num_eras >= 1 &&
                   ((int64_t)cfg.n_trees << cfg.max_depth) * cfg.num_eras < (int64_t(1) << 31),
               "engine: n_trees * 2^max_depth * num_eras = %lld segments exceeds the int32 "
               "segment numbering; reduce max_depth",
               (long long)(((int64_t)cfg.n_trees << cfg.max_depth) * cfg.num_eras));
  WGBM_REQUIRE(cfg.objective == 0 || cfg.objective == 1, "engine: bad objective");
  WGBM_REQUIRE(cfg.objective == 1 || cfg.n_trees == 1, "engine: regression grows one tree per round");
  WGBM_REQUIRE(cfg.codes_rm && cfg.codes_cm && cfg.root_order && cfg.era_start,
               "engine: null input pointer");
  Engine* e = new Engine();
  e->c = cfg;
  const int64_t T = cfg.n_trees, N = cfg.n_rows, E = cfg.num_eras, F = cfg.n_feats,
                B = cfg.num_bins;
  const int D = cfg.max_depth;
  e->V = hist_pick_v(cfg.num_bins, F);
  e->n_chunks = (int)((F + kHistSlots * e->V - 1) / (kHistSlots * e->V));
  e->qbits = wgbm_qbits_for_rows(N);
  e->H = (1 << (D + 1)) - 1;
  const int64_t nodes_max = int64_t(1) << D;
  e->n_keys_max = T * nodes_max * E;
  const int64_t hist_nodes_max = int64_t(1) << (D - 1);  // deepest level with histograms
  E_ALLOC(e->resid, T * N);
  E_ALLOC(e->absmax, T);
  E_ALLOC(e->abs_part, T * kResidBlocks);
  E_ALLOC(e->shifts, T);
  if (E > 1) {
    // the direct era path needs every (node, era) segment to fit one LDS
    // histogram (counts < 2^18 per bin): all eras at most 65536 rows
    std::vector<int64_t> es((size_t)E + 1);
    if (hipMemcpy(es.data(), cfg.era_start, sizeof(int64_t) * (E + 1), hipMemcpyDeviceToHost) !=
        hipSuccess) {
      wgbm_set_error("engine: cannot read era_start");
      engine_destroy(e);
      return WGBM_EINVAL;
    }
    int64_t mx = 0;
    for (int64_t k = 0; k < E; ++k) mx = std::max<int64_t>(mx, es[k + 1] - es[k]);
    e->des_direct = mx <= WGBM_MAX_TILE_ROWS;
  }
  // per-level split buffers for nc_max (tree, node)s: every node of the
  // deepest split level when that fits the budget, else the largest power of
  // two of nodes that does (deeper levels are then processed in chunks)
  const int64_t W = (E + kDesEraBlock - 1) / kDesEraBlock;
  const int64_t per_node =
      e->des_direct ? des_stage_words(1, (int32_t)W, F * (B - 1)) * 5 +
                          W * (4 + F * (B - 1) * 9) + F * (B - 1) * 8
                    : 2 * E * F * B * 12 + (E > 1 ? F * (B - 1) * 8 : 0);
  const int64_t budget = cfg.level_bytes > 0 ? cfg.level_bytes : (int64_t)4 << 30;
  if (T * hist_nodes_max * per_node <= budget) {
    e->nc_max = T * hist_nodes_max;
  } else {
    e->nc_max = 1;
    while (e->nc_max * 2 <= T * hist_nodes_max && e->nc_max * 2 * per_node <= budget)
      e->nc_max *= 2;
  }
  {
    // device memory of the rest, against what is free (a clear error rather
    // than an allocation failure halfway)
    // positions: order, keyp, rpos (two levels each), residual, direction
    // byte; segments: offsets, wide sums and counts (two levels), key pairs,
    // partition words; nodes: flags, shifts, maxima, picks, leaf values and
    // the chosen split's per-era gains; the pair codes; 64 MiB of slack
    const int64_t keys = e->n_keys_max, tn = T * nodes_max;
    const int64_t pcodes = (e->des_direct && B <= 7) ? N * pair_stride((int32_t)F) : 0;
    const int64_t need = e->nc_max * per_node + T * N * 29 + keys * 132 + tn * 76 + tn * E * 4 +
                         pcodes + ((int64_t)64 << 20);
    size_t free_b = 0, total_b = 0;
    if (hipMemGetInfo(&free_b, &total_b) == hipSuccess && (size_t)need > free_b) {
      wgbm_set_error("engine: needs about %.1f GiB of device memory (max_depth=%d, %d eras, "
                     "%lld rows x %d trees), %.1f GiB free; reduce max_depth or the data",
                     need / 1073741824.0, D, (int)E, (long long)N, (int)T,
                     free_b / 1073741824.0);
      engine_destroy(e);
      return WGBM_ENOMEM;
    }
    // the estimate (with its slack) as one arena; without it every buffer
    // is its own allocation
    void* a = nullptr;
    if (hipMalloc(&a, (size_t)need) == hipSuccess) {
      e->allocs.push_back(a);
      e->arena = (char*)a;
      e->arena_size = (size_t)need;
    } else {
      (void)hipGetLastError();
    }
  }
  for (int k = 0; k < 2; ++k) {
    E_ALLOC(e->order[k], T * N);
    E_ALLOC(e->seg[k], e->n_keys_max + 1);
    E_ALLOC(e->totqh[k], e->n_keys_max);
    E_ALLOC(e->totql[k], e->n_keys_max);
    E_ALLOC(e->totc[k], e->n_keys_max);
    E_ALLOC(e->present[k], T * nodes_max);
    E_ALLOC(e->node_shift[k], e->n_keys_max);
    E_ALLOC(e->key_list[k], 2 * e->n_keys_max);
    if (!e->des_direct) {
      E_ALLOC(e->hq[k], e->nc_max * E * F * B);
      E_ALLOC(e->hc[k], e->nc_max * E * F * B);
    }
  }
  if (e->des_direct) {
    E_ALLOC(e->sgain, des_stage_words(e->nc_max, (int32_t)W, F * (B - 1)));
    E_ALLOC(e->sdir, des_stage_words(e->nc_max, (int32_t)W, F * (B - 1)));
    E_ALLOC(e->local_of, F);
    if (B <= 7 && N * pair_stride((int32_t)F) <= (int64_t)0xffffffffll) {
      e->pstride = pair_stride((int32_t)F);
      E_ALLOC(e->pcodes, N * e->pstride);
    }
    E_ALLOC(e->alive, e->nc_max * W);
    E_ALLOC(e->wg_agree, e->nc_max * ((F * (B - 1) + 255) / 256));
    E_ALLOC(e->wg_key, e->nc_max * ((F * (B - 1) + 255) / 256));
    E_ALLOC(e->bsum, e->nc_max * W * F * (B - 1));
    E_ALLOC(e->bdir, e->nc_max * W * F * (B - 1));
  }
  E_ALLOC(e->dirbit, T * N);
  E_ALLOC(e->keyp[0], T * N);
  E_ALLOC(e->keyp[1], T * N);
  E_ALLOC(e->rpos[0], T * N);
  E_ALLOC(e->rpos[1], T * N);
  e->nb = (T * N + kPartBlock - 1) / kPartBlock;
  E_ALLOC(e->ps.own_qh, e->n_keys_max);
  E_ALLOC(e->ps.own_ql, e->n_keys_max);
  E_ALLOC(e->ps.own_n, e->n_keys_max);
  E_ALLOC(e->ps.bf_qh, e->nb);
  E_ALLOC(e->ps.bf_ql, e->nb);
  E_ALLOC(e->ps.bf_n, e->nb);
  E_ALLOC(e->ps.bl_qh, e->nb);
  E_ALLOC(e->ps.bl_ql, e->nb);
  E_ALLOC(e->ps.bl_n, e->nb);
  E_ALLOC(e->ps.P_qh, e->nb);
  E_ALLOC(e->ps.P_ql, e->nb);
  E_ALLOC(e->ps.P_n, e->nb);
  E_ALLOC(e->ps.own_ml, e->n_keys_max);
  E_ALLOC(e->ps.own_mr, e->n_keys_max);
  E_ALLOC(e->ps.bf_ml, e->nb);
  E_ALLOC(e->ps.bf_mr, e->nb);
  E_ALLOC(e->ps.bl_ml, e->nb);
  E_ALLOC(e->ps.bl_mr, e->nb);
  E_ALLOC(e->ps.bf_node, e->nb);
  E_ALLOC(e->ps.pm_l, e->nb);
  E_ALLOC(e->ps.pm_r, e->nb);
  E_ALLOC(e->hkts, e->n_keys_max + 1);
  E_ALLOC(e->hn, 1);
  E_ALLOC(e->kw.cnt, e->n_keys_max);
  E_ALLOC(e->kw.qh, e->n_keys_max);
  E_ALLOC(e->kw.ql, e->n_keys_max);
  E_ALLOC(e->kw.ml, e->n_keys_max);
  E_ALLOC(e->kw.mr, e->n_keys_max);
  if (E > 1) E_ALLOC(e->res, 2 * e->nb);
  if (E > 1) {
    E_ALLOC(e->crit, e->nc_max * F * (B - 1));
    E_ALLOC(e->agree, e->nc_max * F * (B - 1));
    E_ALLOC(e->agree_max, 2 * T * nodes_max);
  }
  E_ALLOC(e->split_l, T * nodes_max);
  E_ALLOC(e->split_b, T * nodes_max);
  E_ALLOC(e->split_gain, T * nodes_max * E);
  E_ALLOC(e->leaf_val, T * nodes_max);
  E_ALLOC(e->nroute, T * nodes_max);
  E_ALLOC(e->best, 2 * T * nodes_max);
  e->pick_stride = T * nodes_max;
  E_ALLOC(e->done, T * nodes_max);
  {
    hipError_t err = hipMemset(e->done, 0, sizeof(uint32_t) * T * nodes_max);
    if (err == hipSuccess) {
      const size_t k = (size_t)e->n_keys_max;
      err = hipMemset(e->kw.cnt, 0, k * sizeof(unsigned long long));
      if (err == hipSuccess) err = hipMemset(e->kw.qh, 0, k * sizeof(int64_t));
      if (err == hipSuccess) err = hipMemset(e->kw.ql, 0, k * sizeof(int64_t));
      if (err == hipSuccess) err = hipMemset(e->kw.ml, 0, k * sizeof(uint32_t));
      if (err == hipSuccess) err = hipMemset(e->kw.mr, 0, k * sizeof(uint32_t));
    }
    if (err != hipSuccess) {
      wgbm_set_error("engine: clearing the arrival counters and node words failed: %s",
                     hipGetErrorString(err));
      engine_destroy(e);
      return (int)err;
    }
  }
  *out = e;
  return 0;
}

int engine_set_tuning(Engine* e, int key, int64_t value) {
  if (key == 1) {
    WGBM_REQUIRE(value == 0 || (value >= 256 && value <= WGBM_MAX_TILE_ROWS),
                 "hist tile rows must be 0 or in [256, %d]", WGBM_MAX_TILE_ROWS);
    e->hist_tile_rows = value;
    e->root_tiles_ready = false;  // the root plan depends on the tile rows
    return 0;
  }
  if (key == 5) {
    WGBM_REQUIRE(value == 0 || value == 1, "one-era root path must be 0 or 1");
    e->root_path = (int)value;
    return 0;
  }
  if (key == 6) {
    WGBM_REQUIRE(value == 0 || value == 1, "one-era single-pass partition must be 0 or 1");
    e->part1 = (int)value;
    return 0;
  }
  if (key == 7) {
    WGBM_REQUIRE(value == 0 || value == 1, "era-level range reservation must be 0 or 1");
    e->part_era = (int)value;
    return 0;
  }
  if (key == 2) {
    WGBM_REQUIRE(value == 0 || value == 1, "era code layout must be 0 or 1");
    e->des_codes = (int)value;
    return 0;
  }
  if (key == 3) {
    WGBM_REQUIRE(value == 0 || value == 1, "one-era level scan must be 0 or 1");
    e->lscan_e1 = (int)value;
    return 0;
  }
  if (key == 4) {
    WGBM_REQUIRE(value == 0 || value == 1, "fused split / leaf step must be 0 or 1");
    e->fuse_finish = (int)value;
    return 0;
  }
  wgbm_set_error("engine_set_tuning: unknown key %d", key);
  return WGBM_EINVAL;
}

// histogram tile rows for a level: enough tiles for ~2 workgroups per CU
static int64_t pick_tile_rows(const Engine* e, int64_t rows_bound) {
  if (e->hist_tile_rows > 0) return e->hist_tile_rows;
  const int64_t target_wg = kHistTargetWG;
  int64_t tiles = std::max<int64_t>(1, target_wg / e->n_chunks);
  int64_t r = (rows_bound + tiles - 1) / tiles;
  r = (r + 255) / 256 * 256;
  return std::min<int64_t>(std::max<int64_t>(r, 1024), WGBM_MAX_TILE_ROWS);
}

static int ensure_partials(Engine* e, int64_t max_tiles) {
  const int64_t words = max_tiles * e->n_chunks * kHistSlots * e->V * e->c.num_bins;
  if (words <= e->part_words) return 0;
  if (e->part) {
    // partial buffers are only reused within the stream; grow after a sync
    WGBM_CHECK(hipDeviceSynchronize());
    for (auto it = e->allocs.begin(); it != e->allocs.end(); ++it)
      if (*it == e->part) {
        (void)hipFree(*it);
        e->allocs.erase(it);
        break;
      }
    e->part = nullptr;
  }
  int r = dalloc(e, &e->part, words);
  if (r) return r;
  e->part_words = words;
  return 0;
}

// room for max_tiles histogram tiles (tile list and partials)
static int ensure_tiles(Engine* e, int64_t max_tiles) {
  int r = ensure_partials(e, max_tiles);
  if (r) return r;
  if (max_tiles > e->max_htiles) {
    if (e->htiles) {
      // tile lists are only reused within the stream; grow after a sync
      WGBM_CHECK(hipDeviceSynchronize());
      for (auto it = e->allocs.begin(); it != e->allocs.end(); ++it)
        if (*it == e->htiles) {
          (void)hipFree(*it);
          e->allocs.erase(it);
          break;
        }
      e->htiles = nullptr;
    }
    r = dalloc(e, &e->htiles, max_tiles);
    if (r) return r;
    e->max_htiles = max_tiles;
  }
  return 0;
}

// histogram tiles of level d (the root, or the key pairs of every split: the
// smaller child, or both children when one takes a finer shift): tile rows,
// the tile bound, and buffers that hold them
struct LevelPlan {
  int32_t n_list = 0;
  int64_t rows_bound = 0, R = 0, max_tiles = 0;
};

static void level_plan_sizes(const Engine* e, int d, LevelPlan* lp) {
  const int64_t T = e->c.n_trees, N = e->c.n_rows, E = e->c.num_eras;
  const int64_t nodes = int64_t(1) << d;
  lp->n_list = (int32_t)(d == 0 ? T * nodes * E : 2 * T * (nodes / 2) * E);
  // tiles are sized for the smaller children (half the rows); the bound
  // holds the rare level where every split histograms both children
  lp->rows_bound = d == 0 ? T * N : (T * N) / 2;
  lp->R = pick_tile_rows(e, lp->rows_bound);
  lp->max_tiles = (T * N) / lp->R + lp->n_list + 1;
}

static int level_plan(Engine* e, int d, LevelPlan* lp) {
  level_plan_sizes(e, d, lp);
  return ensure_tiles(e, lp->max_tiles);
}

// the tile buffers of every whole level a round histograms, sized once before
// the first round's launches: growing them level by level would synchronise
// the device (a buffer in use is freed only after a sync) at each depth
static int presize_levels(Engine* e) {
  if (e->des_direct) return 0;
  int64_t mt = 0;
  for (int d = 0; d < e->c.max_depth; ++d) {
    // levels take the subtraction path while every level so far fits whole
    if (((int64_t)e->c.n_trees << d) > e->nc_max) break;
    LevelPlan lp;
    level_plan_sizes(e, d, &lp);
    mt = std::max(mt, lp.max_tiles);
  }
  return mt > 0 ? ensure_tiles(e, mt) : 0;
}

// histogram tiles of one chunk of a level (n_list keys, the chunk's present
// nodes histogrammed directly; the level split into n_chunk such chunks)
static int chunk_plan(Engine* e, int64_t n_list, int n_chunk, LevelPlan* lp) {
  const int64_t TN = (int64_t)e->c.n_trees * e->c.n_rows;
  lp->n_list = (int32_t)n_list;
  lp->rows_bound = TN;
  lp->R = pick_tile_rows(e, std::max<int64_t>(1, TN / std::max(n_chunk, 1)));
  lp->max_tiles = TN / lp->R + n_list + 1;
  return ensure_tiles(e, lp->max_tiles);
}

static inline unsigned blocks_for(int64_t n, int bs) { return (unsigned)((n + bs - 1) / bs); }

int engine_round(Engine* e, const void* target, float* pred, const int32_t* feat_sel,
                 int32_t n_sel, const TreeRecord& rec, hipStream_t st) {
  const EngineConfig& c = e->c;
  WGBM_REQUIRE(target && pred && feat_sel, "engine_round: null pointer");
  WGBM_REQUIRE(n_sel >= 1 && n_sel <= c.n_feats, "engine_round: n_sel out of range");
  WGBM_REQUIRE(rec.H == e->H, "engine_round: record has H=%d, expected %d", rec.H, e->H);
  const int T = c.n_trees, E = c.num_eras, F = c.n_feats, B = c.num_bins, D = c.max_depth;
  const int64_t N = c.n_rows;
  if (!e->part) {
    const int r = presize_levels(e);
    if (r) return r;
  }

  // residuals and quantisation shifts (per-workgroup maxima, then one
  // workgroup per tree reduces them)
  const int nres = (int)std::max<int64_t>(1, std::min<int64_t>(blocks_for(N, 256), kResidBlocks));
  if (c.objective == 0) {
    hipLaunchKernelGGL(residual_regression_kernel, dim3(nres), dim3(256), 0, st,
                       (const float*)target, pred, N, e->resid, e->abs_part);
  } else {
    hipLaunchKernelGGL(residual_softmax_kernel, dim3(nres), dim3(256), 0, st, pred,
                       (const int32_t*)target, N, T, e->resid, e->abs_part);
  }
  WGBM_LAUNCH_CHECK();
  // one era, fused root: the root totals words are cleared here for the
  // root's atomic sums
  const bool root_e1 = E == 1 && e->root_path;
  hipLaunchKernelGGL(absmax_finish_kernel, dim3(T), dim3(256), 0, st, e->abs_part, nres, e->qbits,
                     e->absmax, e->shifts, root_e1 ? e->totqh[0] : (int64_t*)nullptr,
                     e->totql[0], e->totc[0], N);
  WGBM_LAUNCH_CHECK();

  // root segments and totals
  int cur = 0;
  const int64_t n_pos = (int64_t)T * N;
  if (root_e1) {
    hipLaunchKernelGGL(root_setup_e1_kernel, dim3(blocks_for(N, kRootE1Span), (unsigned)T),
                       dim3(1024), 0,
                       st, c.root_order, N, T, e->resid, e->order[0], e->keyp[0], e->rpos[0],
                       e->seg[0], e->present[0], e->best, e->shifts, 62 - e->qbits,
                       e->node_shift[0], e->totqh[0], e->totql[0]);
  } else {
    hipLaunchKernelGGL(root_setup_kernel,
                       dim3(blocks_for(std::max<int64_t>(n_pos, T * E), 256)), dim3(256), 0, st,
                       c.root_order, N, T, c.era_start, E, e->resid, e->order[0], e->keyp[0],
                       e->rpos[0], e->seg[0], e->present[0], e->best, e->agree_max, e->shifts,
                       e->node_shift[0]);
  }
  WGBM_LAUNCH_CHECK();
  RouteArgs ra{};
  ra.n_pos = n_pos;
  ra.E = E;
  ra.feat_sel = feat_sel;
  ra.codes_cm = c.codes_cm;
  ra.n = N;
  ra.shifts = e->shifts;
  ra.s63_add = 62 - e->qbits;
  ra.leaf_val = e->leaf_val;
  ra.lr = c.learning_rate;
  ra.pred = pred;
  // scores: [N] (one tree per round) or class-major [K][N] (tree t = class t)
  ra.pstride = 1;
  ra.pcol = c.objective == 0 ? 0 : N;
  ra.dirbit = e->dirbit;
  ra.ps = e->ps;
  if (!root_e1) {
    RouteArgs r0 = ra;
    r0.mode = 0;
    r0.seg = e->seg[0];
    r0.n_keys = T * E;
    r0.order = e->order[0];
    r0.keyp = e->keyp[0];
    r0.rpos = e->rpos[0];
    r0.nodes = 1;
    r0.present = e->present[0];
    r0.want_max = E > 1 ? 1 : 0;  // several eras: every root key's own shift
    hipLaunchKernelGGL(route_kernel, dim3((unsigned)e->nb), dim3(kPartThreads),
                       route_lds_bytes(r0), st, r0);
    WGBM_LAUNCH_CHECK();
    hipLaunchKernelGGL(block_scan_kernel, dim3(1), dim3(1024), 0, st, (int32_t)e->nb, e->ps);
    WGBM_LAUNCH_CHECK();
    hipLaunchKernelGGL(root_totals_kernel, dim3(blocks_for((int64_t)T * E, 256)), dim3(256), 0,
                       st, (int32_t)(T * E), e->seg[0], e->ps, e->totqh[0], e->totql[0],
                       e->totc[0], e->qbits, E > 1 ? e->node_shift[0] : (int32_t*)nullptr);
    WGBM_LAUNCH_CHECK();
  }

  if (e->des_direct) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(blocks_for(F, 256)), dim3(256), 0, st, e->local_of,
                       (int64_t)F, -1);
    WGBM_LAUNCH_CHECK();
    hipLaunchKernelGGL(local_scatter_kernel, dim3(blocks_for(n_sel, 256)), dim3(256), 0, st,
                       feat_sel, n_sel, F, e->local_of);
    WGBM_LAUNCH_CHECK();
  }

  const float mcw = c.min_child_weight, eps = c.l2_reg, msg = c.min_split_gain;
  bool planned = false;  // this level's histogram tiles were planned by the previous level
  // the last split level wrote every row's leaf key (keyp[cur] by row):
  // the last level updates predictions in row order (leaf_rows_kernel)
  bool leaf_keys = false;
  bool alive_ready = false;  // this level's live-era masks were written by the previous scan
  for (int d = 0; d <= D; ++d) {
    const int nodes = 1 << d;
    const int n_tn = T * nodes;
    const int n_keys = n_tn * E;
    const int hcur = d & 1, hprev = hcur ^ 1;
    // split-pick words of this depth (cleared by the previous depth's
    // level_finish, or by root_setup at depth 0)
    unsigned long long* best = e->best + hcur * e->pick_stride;
    int32_t* agree_max = e->agree_max ? e->agree_max + hcur * e->pick_stride : nullptr;
    // the (tree, node)s of this depth go through the split buffers whole, or
    // in chunks of nc_max nodes when they do not fit (chunk nodes are
    // histogrammed directly: their parents' histograms are not kept)
    const bool whole = n_tn <= e->nc_max;
    if (d < D && e->des_direct) {
      // ---- E > 1, direct: per-era gains of every (node, era) segment
      const int64_t ncand = (int64_t)n_sel * (B - 1);
      // pair codes for levels of large segments (mean rows per (node, era))
      const bool use_pairs = e->pcodes && e->des_codes == 1 &&
                             N >= (int64_t)kDesPairMinRows * nodes * E;
      if (use_pairs && !e->pcodes_ready) {
        int r = launch_pack_pairs(st, c.codes_rm, c.stride, F, N, B, e->pcodes, e->pstride);
        if (r) return r;
        e->pcodes_ready = true;
      }
      const int64_t W = (E + kDesEraBlock - 1) / kDesEraBlock;
      for (int c0 = 0; c0 < n_tn; c0 += (int)e->nc_max) {
        // nodes [c0, c0 + nc): every node-indexed argument starts at c0
        const int nc = (int)std::min<int64_t>(e->nc_max, n_tn - c0);
        const int64_t k0 = (int64_t)c0 * E;
        // optional event timers (wgbm_timer_enable(1)): the per-era kernel of
        // the level ("des_rows_L<d>") and the era sums, pick and finish
        // ("des_sums_L<d>")
        char tag[32];
        snprintf(tag, sizeof tag, "des_rows_L%d", d);
        void* tm = timer_mode() == 1 ? timer_begin(tag) : nullptr;
        if (tm) WGBM_CHECK(hipEventRecord(timer_start_event(tm), st));
        int r = launch_des_era(e->V, B, nc * E, st, c.codes_rm, c.stride, F, e->rpos[cur],
                               e->node_shift[cur] + k0, e->order[cur], e->seg[cur] + k0, E, nodes,
                               e->present[cur] + c0, e->local_of, n_sel, mcw, eps, e->sgain,
                               e->sdir, use_pairs ? e->pcodes : nullptr, N, e->pstride);
        if (r) return r;
        if (tm) {
          WGBM_CHECK(hipEventRecord(timer_stop_event(tm), st));
          timer_end(tm);
          snprintf(tag, sizeof tag, "des_sums_L%d", d);
          tm = timer_begin(tag);
          if (tm) WGBM_CHECK(hipEventRecord(timer_start_event(tm), st));
        }
        if (!(alive_ready && nc == n_tn)) {
          hipLaunchKernelGGL(des_alive_kernel, dim3(blocks_for((int64_t)nc * W, 256)), dim3(256),
                             0, st, e->seg[cur] + k0, E, nc, mcw, e->alive);
          WGBM_LAUNCH_CHECK();
        }
        hipLaunchKernelGGL(des_block_kernel,
                           dim3(blocks_for((int64_t)nc * W * ((ncand + 63) / 64) * 64, 256)),
                           dim3(256), 0, st, e->sgain, e->sdir, E, nc, ncand,
                           e->present[cur] + c0, e->alive, e->bsum, e->bdir);
        WGBM_LAUNCH_CHECK();
        // block sums in block order, the pick and the record in one launch
        // (the last workgroup of each node picks from the workgroups'
        // summaries and finishes the node)
        hipLaunchKernelGGL(des_combine_pick_kernel,
                           dim3((unsigned)((int64_t)nc * ((ncand + 255) / 256))), dim3(256), 0,
                           st, e->bsum, e->bdir, E, nc, ncand, e->present[cur] + c0, e->alive,
                           msg, e->wg_agree, e->wg_key, best + c0, e->done + c0, e->sgain,
                           e->seg[cur] + k0, mcw, (int32_t)(B - 1), n_sel, e->split_l + c0,
                           e->split_b + c0, e->split_gain + k0);
        WGBM_LAUNCH_CHECK();
        if (tm) {
          WGBM_CHECK(hipEventRecord(timer_stop_event(tm), st));
          timer_end(tm);
        }
      }
    } else if (d < D) {
      // ---- histograms of the computed segments, then split search + DES
      // selection.  Whole level (and the previous one kept): the smaller
      // child of every split, the sibling by subtraction.  Otherwise each
      // chunk's present nodes directly.
      const bool subtract = whole && (d == 0 || e->stored_prev);
      const int n_chunk = subtract ? 1 : (int)((n_tn + e->nc_max - 1) / e->nc_max);
      for (int ch = 0; ch < n_chunk; ++ch) {
        const int c0 = subtract ? 0 : (int)(ch * e->nc_max);
        const int nc = subtract ? n_tn : (int)std::min<int64_t>(e->nc_max, n_tn - c0);
        const int64_t k0 = (int64_t)c0 * E;
        LevelPlan lp;
        int r = subtract ? level_plan(e, d, &lp) : chunk_plan(e, (int64_t)nc * E, n_chunk, &lp);
        if (r) return r;
        const int n_list = lp.n_list;
        const int64_t R = lp.R, max_tiles = lp.max_tiles, rows_bound = lp.rows_bound;
        // keys: the level's pairs (depth > 0), every root key, or the chunk's
        // present nodes (relative to the chunk)
        const int32_t* list = nullptr;
        if (!subtract) {
          hipLaunchKernelGGL(chunk_keys_kernel, dim3(blocks_for((int64_t)nc * E, 256)),
                             dim3(256), 0, st, e->present[cur] + c0, E, nc, e->key_list[cur]);
          WGBM_LAUNCH_CHECK();
          list = e->key_list[cur];
        } else if (d > 0) {
          list = e->key_list[cur];
        }
        // the level's tile plan: the cached root plan, the previous level's
        // (level_scan_kernel), or planned here
        Tile* tl_d = e->htiles;
        int32_t* kts_d = e->hkts;
        int32_t* hn_d = e->hn;
        if (d == 0 && subtract && root_e1) {
          if (!e->root_tiles_ready) {
            if (max_tiles > e->root_tiles_cap) {
              // a larger plan (new tile rows): fresh buffers, the old ones stay
              // allocated until the engine is destroyed (no sync needed)
              e->root_tiles = nullptr;
              e->root_kts = nullptr;
              e->root_hn = nullptr;
              int ra2 = dalloc(e, &e->root_tiles, max_tiles);
              if (!ra2) ra2 = dalloc(e, &e->root_kts, (int64_t)n_list + 1);
              if (!ra2) ra2 = dalloc(e, &e->root_hn, 1);
              if (ra2) return ra2;
              e->root_tiles_cap = max_tiles;
            }
            hipLaunchKernelGGL(plan_tiles_kernel, dim3(1), dim3(1024), 0, st, e->seg[cur],
                               (int64_t)0, n_list, list, (int32_t)R, 0, (int32_t)max_tiles,
                               e->root_tiles, e->root_kts, e->root_hn);
            WGBM_LAUNCH_CHECK();
            e->root_tiles_ready = true;
          }
          tl_d = e->root_tiles;
          kts_d = e->root_kts;
          hn_d = e->root_hn;
        } else if (!(subtract && planned)) {
          hipLaunchKernelGGL(plan_tiles_kernel, dim3(1), dim3(1024), 0, st, e->seg[cur] + k0,
                             (int64_t)0, n_list, list, (int32_t)R, 0, (int32_t)max_tiles,
                             e->htiles, e->hkts, e->hn);
          WGBM_LAUNCH_CHECK();
        }
        HistLaunch a;
        a.codes = c.codes_rm;
        a.n_rows = N;
        a.stride = c.stride;
        a.n_feats = F;
        a.resid = e->rpos[cur];  // residuals in position order (global positions)
        a.resid_by_pos = 1;
        a.resid_tree_stride = 0;
        // quantised with the histogram shift of each tile's key (the (tree,
        // node) with one era, the (tree, node, era) segment with several)
        a.shifts = e->node_shift[cur] + k0;
        a.order = e->order[cur];
        a.tiles = tl_d;
        a.n_tiles = hn_d;
        a.keys_per_tree = 1;
        a.num_bins = B;
        a.part = e->part;
        a.V = e->V;
        a.n_chunks = e->n_chunks;
        a.max_tiles = (int32_t)max_tiles;
        a.native = 1;  // the engine's codes come from the library's binner / pre-binned copy
        a.timer_tag = "engine_hist_tiles";
        r = launch_hist_tiles(a, st);
        if (r) return r;
        const int64_t pairs = (subtract && d > 0) ? n_list / 2 : n_list;
        const int64_t tiles_per_key = std::max<int64_t>(1, rows_bound / R / std::max<int64_t>(pairs, 1));
        r = launch_finalize_level(tiles_per_key, e->part, kts_d, list, n_list, e->n_chunks, e->V,
                                  B, F, E, nodes, subtract ? d : 0, e->hq[hprev], e->hc[hprev],
                                  hn_d, e->hq[hcur], e->hc[hcur], st);
        if (r) return r;
        if (E == 1 && e->fuse_finish) {
          // split search and the level's leaf / record step in one launch
          FinishE1 fa;
          fa.depth = d;
          fa.max_depth = D;
          fa.T = T;
          fa.B = B;
          fa.present = e->present[cur];
          fa.split_l = e->split_l;
          fa.split_b = e->split_b;
          fa.feat_sel = feat_sel;
          fa.tot_qh = e->totqh[cur];
          fa.tot_ql = e->totql[cur];
          fa.tot_c = e->totc[cur];
          fa.shifts = e->shifts;
          fa.s63_add = 62 - e->qbits;
          fa.leaf_val = e->leaf_val;
          fa.rec = rec;
          fa.best_next = e->best + (hcur ^ 1) * e->pick_stride;
          fa.nroute = e->nroute;
          r = launch_split_finish_e1(nc, c0, st, e->hq[hcur], e->hc[hcur], F, n_sel,
                                     e->node_shift[cur], mcw, eps, msg, best, e->done, fa);
          if (r) return r;
        } else if (E == 1) {
          // the pick is decoded by level_finish
          r = launch_split_level_e1(nc, st, e->hq[hcur], e->hc[hcur], F, B, feat_sel, n_sel, nodes,
                                    e->present[cur] + c0, e->node_shift[cur] + c0, mcw, eps, msg,
                                    best + c0);
          if (r) return r;
        } else {
          const int64_t ncand = (int64_t)n_sel * (B - 1);
          const int64_t nacc = (int64_t)nc * n_sel * ((B - 1 + kDesChunk - 1) / kDesChunk);
          hipLaunchKernelGGL(des_accumulate_kernel, dim3(blocks_for(nacc, 128)), dim3(128), 0, st,
                             e->hq[hcur], e->hc[hcur], F, B, E, feat_sel, n_sel, nodes, nc,
                             e->present[cur] + c0, e->node_shift[cur] + k0, mcw, eps, e->crit,
                             e->agree, agree_max + c0);
          WGBM_LAUNCH_CHECK();
          hipLaunchKernelGGL(des_pick_kernel, dim3(blocks_for((int64_t)nc * ncand, 256)),
                             dim3(256), 0, st, e->crit, e->agree, agree_max + c0,
                             e->present[cur] + c0, nc, ncand, msg, best + c0);
          WGBM_LAUNCH_CHECK();
          hipLaunchKernelGGL(des_finish_kernel, dim3(blocks_for((int64_t)nc * E, 256)), dim3(256),
                             0, st, best + c0, e->hq[hcur], e->hc[hcur], F, B, E, feat_sel, nodes,
                             nc, e->node_shift[cur] + k0, mcw, eps, (const float*)nullptr,
                             e->seg[cur] + k0, n_sel, e->split_l + c0, e->split_b + c0,
                             e->split_gain + k0);
          WGBM_LAUNCH_CHECK();
        }
      }
      e->stored_prev = subtract;
    }
    // ---- leaf values, the tree record of this depth, cleared words of the
    // next depth (child totals, split picks)
    const int nxt = cur ^ 1;
    const bool e1_pick = d < D && !e->des_direct && E == 1;
    if (!(e1_pick && e->fuse_finish)) {  // (else done by split_finish_e1_kernel)
      hipLaunchKernelGGL(level_finish_kernel, dim3((unsigned)n_tn), dim3(64), 0, st, d, D, T, E,
                         B, e->present[cur], e1_pick ? (const unsigned long long*)best : nullptr,
                         e->split_l, e->split_b, e->split_gain, feat_sel, e->totqh[cur],
                         e->totql[cur], e->totc[cur], e->shifts, 62 - e->qbits, e->leaf_val, rec,
                         e->best + (hcur ^ 1) * e->pick_stride,
                         e->agree_max ? e->agree_max + (hcur ^ 1) * e->pick_stride : nullptr,
                         e->nroute);
      WGBM_LAUNCH_CHECK();
    }
    // ---- partition (or final leaf update): route every position, then the
    // next level's segments and the stable scatter
    RouteArgs rl = ra;
    rl.mode = d < D ? 1 : 2;
    rl.seg = e->seg[cur];
    rl.n_keys = n_keys;
    rl.order = e->order[cur];
    rl.keyp = e->keyp[cur];
    rl.rpos = e->rpos[cur];
    rl.nodes = nodes;
    rl.present = e->present[cur];
    rl.split_l = e->split_l;
    rl.split_b = e->split_b;
    rl.nroute = e->nroute;
    // the children's max|r| decides their histogram shifts; children at the
    // last depth are leaves and need none
    rl.want_max = d + 1 < D ? 1 : 0;
    // one era: route and place every position in one pass, the level scan
    // then reads the node words
    const bool one_pass =
        d < D && E == 1 && e->lscan_e1 && e->part1 && n_tn <= kPartition1MaxNodes;
    const bool one_wg = E == 1 ? n_tn <= kLevelScanE1MaxNodes
                               : (E <= 64 && n_tn <= kLevelScanMaxNodes);
    // several eras, levels scanned by node_scan_kernel: the route reserves
    // the segments' child ranges and leaves their words in kw (no block
    // prefix launch)
    const bool era_res = d < D && E > 1 && !one_wg && e->part_era;
    if (d == D && leaf_keys) {
      hipLaunchKernelGGL(leaf_rows_kernel, dim3((unsigned)blocks_for(n_pos, 1024)), dim3(256), 0,
                         st, e->keyp[cur], rl.n, T, rl.nroute, rl.lr, rl.pred, rl.pstride,
                         rl.pcol);
    } else if (one_pass) {
      // the last split level writes each row's leaf key instead of placing it
      leaf_keys = d + 1 == D;
      int32_t* lk = leaf_keys ? e->keyp[nxt] : nullptr;
      const size_t lds = partition1_lds_bytes(n_tn);
      if (n_pos > kPartition1WideSpan * n_tn) {
        hipLaunchKernelGGL(partition_e1_kernel<1024>, dim3((unsigned)((n_pos + 4095) / 4096)),
                           dim3(1024), lds, st, rl, e->kw, (int32_t)n_tn, e->order[nxt],
                           e->keyp[nxt], e->rpos[nxt], lk);
      } else {
        hipLaunchKernelGGL(partition_e1_kernel<256>, dim3((unsigned)((n_pos + 1023) / 1024)),
                           dim3(256), lds, st, rl, e->kw, (int32_t)n_tn, e->order[nxt],
                           e->keyp[nxt], e->rpos[nxt], lk);
      }
    } else {
      rl.xcd_order = rl.mode == 2 && T > 1 ? 1 : 0;
      if (era_res) {
        rl.kw = e->kw;
        rl.res = e->res;
      }
      const int64_t grid = rl.xcd_order ? wgbm_xcd_grid(e->nb) : e->nb;
      hipLaunchKernelGGL(route_kernel, dim3((unsigned)grid), dim3(kPartThreads),
                         route_lds_bytes(rl), st, rl);
    }
    WGBM_LAUNCH_CHECK();
    planned = false;
    alive_ready = false;
    LevelNext nx;
    nx.tot_qh = e->totqh[cur];
    nx.tot_ql = e->totql[cur];
    nx.node_shift = e->node_shift[cur];
    nx.qbits = e->qbits;
    nx.have_max = d + 1 < D ? 1 : 0;
    nx.seg_next = e->seg[nxt];
    nx.tot_qh_next = e->totqh[nxt];
    nx.tot_ql_next = e->totql[nxt];
    nx.tot_c_next = e->totc[nxt];
    nx.present_next = e->present[nxt];
    nx.key_list_next = e->key_list[nxt];
    nx.node_shift_next = e->node_shift[nxt];
    // the next era level's live-era masks, when it runs whole: written by
    // node_scan_kernel (no des_alive_kernel launch there)
    const bool next_alive = d + 1 < D && e->des_direct && 2 * (int64_t)n_tn <= e->nc_max;
    nx.alive_next = nullptr;
    nx.mcw = mcw;
    if (d < D && one_wg) {
      // few keys: block prefix, node scan and the next level's tile plan in
      // one workgroup
      LevelPlan lp;
      // the next level's tiles are planned here when it takes the subtraction
      // path (all its nodes fit and this level's histograms are kept)
      const bool next_hist = d + 1 < D && !e->des_direct && 2 * (int64_t)n_tn <= e->nc_max &&
                             e->stored_prev;
      if (next_hist) {
        const int r = level_plan(e, d + 1, &lp);
        if (r) return r;
      }
      if (E == 1 && e->lscan_e1) {
        hipLaunchKernelGGL(level_scan_e1_kernel, dim3(1), dim3(1024), 0, st, (int32_t)e->nb,
                           e->ps, one_pass ? e->kw : KeyWords{}, (int32_t)n_tn, n_pos,
                           e->seg[cur], e->present[cur], e->split_l,
                           nx, next_hist ? 1 : 0, (int32_t)lp.R, (int32_t)lp.max_tiles, e->htiles,
                           e->hkts, e->hn);
        WGBM_LAUNCH_CHECK();
        planned = next_hist;
      } else if (n_tn <= kLevelScanMaxNodes) {
        hipLaunchKernelGGL(level_scan_kernel, dim3(1), dim3(1024), 0, st, (int32_t)e->nb, e->ps,
                           T, nodes, E, n_pos, e->seg[cur], e->present[cur], e->split_l, nx,
                           next_hist ? lp.n_list : 0, (int32_t)lp.R, (int32_t)lp.max_tiles,
                           e->htiles, e->hkts, e->hn);
        WGBM_LAUNCH_CHECK();
        planned = next_hist;
      } else {
        hipLaunchKernelGGL(block_scan_kernel, dim3(1), dim3(1024), 0, st, (int32_t)e->nb, e->ps);
        WGBM_LAUNCH_CHECK();
        nx.alive_next = next_alive ? e->alive : nullptr;
        hipLaunchKernelGGL(node_scan_kernel, dim3(blocks_for((int64_t)n_tn, 4)), dim3(256), 0,
                           st, T, nodes, E, 1, n_pos, e->seg[cur], e->present[cur], e->split_l,
                           e->ps, nx, KeyWords{});
        WGBM_LAUNCH_CHECK();
        alive_ready = next_alive;
      }
    } else if (d < D) {
      if (!era_res) {
        hipLaunchKernelGGL(block_scan_kernel, dim3(1), dim3(1024), 0, st, (int32_t)e->nb, e->ps);
        WGBM_LAUNCH_CHECK();
      }
      const int wpn = E <= 64 ? 1 : (E <= 128 ? 2 : 4);  // waves per node
      nx.alive_next = next_alive ? e->alive : nullptr;
      hipLaunchKernelGGL(node_scan_kernel, dim3(blocks_for((int64_t)n_tn, 4 / wpn)), dim3(256), 0,
                         st, T, nodes, E, wpn, n_pos, e->seg[cur], e->present[cur], e->split_l,
                         e->ps, nx, era_res ? e->kw : KeyWords{});
      WGBM_LAUNCH_CHECK();
      alive_ready = next_alive;
    }
    if (d < D && !one_pass) {
      hipLaunchKernelGGL(scatter_kernel, dim3((unsigned)e->nb), dim3(kPartThreads), 0, st, n_pos,
                         E, e->seg[cur], e->seg[nxt], e->keyp[cur], e->dirbit, e->ps,
                         e->order[cur], e->order[nxt], e->keyp[nxt], e->rpos[cur],
                         e->rpos[nxt], era_res ? (const unsigned long long*)e->res : nullptr);
      WGBM_LAUNCH_CHECK();
    }
    cur = nxt;
  }
  return 0;
}

}  // namespace wgbm
