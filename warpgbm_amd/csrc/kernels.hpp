// Internal (C++) declarations shared by the kernel translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wgbm {

// values per thread of the per-column binner (bin_column_kernel)
constexpr int kBinColumnU = 4;

// A run of row-order positions [begin, end) that all belong to segment `key`.
struct Tile {
  int32_t key;
  int32_t pad;
  int64_t begin;
  int64_t end;
};

enum { kLoadBuffer = 0, kLoadGlobalAligned = 1, kLoadBytes = 2 };

// threads per histogram workgroup (16 waves; two workgroups fit one CU's LDS)
constexpr int kHistThreads = 1024;
// lanes of a histogram row: lane l owns the V features chunk*64*V + l*V + j
constexpr int kHistSlots = 64;
// split candidates (bins) per lane of the era-accumulating DES scan
constexpr int kDesChunk = 8;
// eras per block of the DES era sum (float64: in era order inside a block,
// then block sums in block order); also the width of a live-era mask word
constexpr int kDesEraBlock = 32;
// Staged per-era gains / directions of the direct era path, block-major: for
// (tree-node tn, era e, candidate c = local feature * (B-1) + bin) the slot
// (((tn * W + e / 32) * C64 + c / 64) * 32 + e % 32) * 64 + c % 64, with W =
// ceil(E / 32) era blocks and C64 = ceil(ncand / 64) groups of 64
// candidates: the 32 eras of one block and 64 candidates are 8 KB of
// consecutive floats, which one wave of des_block_kernel reads front to back.
__host__ __device__ inline int64_t des_stage_slot(int64_t tn, int32_t e, int32_t W,
                                                  int64_t c64, int64_t c) {
  return (((tn * W + e / 32) * c64 + c / 64) * 32 + e % 32) * 64 + c % 64;
}
// slots of nc tree-nodes
__host__ __device__ inline int64_t des_stage_words(int64_t nc, int32_t W, int64_t ncand) {
  return nc * W * ((ncand + 63) / 64) * 32 * 64;
}
// cache-policy bits of a buffer load: non-temporal (streamed once), plus
// sc0 for the code stream of the tile histogram (measured faster there)
constexpr int kAuxNT = 2;
constexpr int kAuxStream = 3;
// tile of the binner and the pre-binned copy: rows x features per workgroup
constexpr int kBinTileRows = 256, kBinTileFeats = 64;
// rows per workgroup of the key transpose of the quantile selection
constexpr int kTransRows = 1024;
// histogram workgroups per launch the tile sizes aim for: 2 per CU, in the
// engine and for a single call (measured on C2: the tile kernel takes 191 us
// against 194 us with one workgroup per CU; the finalize reads twice the
// partials, which leaves the whole call's time the same)
constexpr int kHistTargetWG = 512;
constexpr int kHistTargetWGCall = 512;

// The tile kernel's shift from per-block maxima of |residual| (one tree):
// partial == nullptr means the shifts come from the shifts array instead.
struct ShiftFromMax {
  const uint32_t* partial = nullptr;
  int32_t n_part = 0;
  int32_t qbits = 0;
  uint32_t* absmax_bits = nullptr;  // written by workgroup 0
  int32_t* shift = nullptr;
  // per key (partial == nullptr): the float bits of each key's largest
  // |residual| (hist_key_max_kernel); a tile takes its key's shift from them
  const uint32_t* key_max = nullptr;
};

// Feature selection of a histogram call (compute_histogram3's feature
// indices): histogram feature h < *count reads code column list[h] of each
// row (list ascending, distinct).  list == nullptr: feature h is column h.
// Per chunk of 64*V histogram features, run[c] != 0 when every lane's V
// features are an aligned run of V consecutive columns (lane l owns features
// c*64*V + l*V + j, loaded with one V-byte load per row); otherwise lane l
// owns features c*64*V + j*64 + l (V byte loads per row, each covering 64
// consecutive selected columns).
struct FeatSel {
  const int32_t* list = nullptr;
  const int32_t* count = nullptr;
  const int32_t* run = nullptr;
  int32_t n_master = 0;  // code columns per row
};

// Outputs of a selected histogram feature h: head[h] is the first output
// index o (feature_indices[o] == list[h]), next[o] the following one or -1.
// head == nullptr: feature h is output h (f < n_feats).
struct FeatOut {
  const int32_t* head = nullptr;
  const int32_t* next = nullptr;
  const int32_t* count = nullptr;
  const int32_t* run = nullptr;  // lane ownership per chunk, as FeatSel
  int32_t n_out = 0;  // features of the output layout [key][n_out][B]
};

// The map from requested features to histogram features, built on the
// device by one workgroup of the preparation launch: mark [n_master] and
// next [n_out] hold the per-column output lists, list/head [min(n_out,
// n_master)] and *count the distinct requested columns in ascending order,
// run [n_chunks] the lane ownership of each chunk (FeatSel).
struct FeatMapArgs {
  const int32_t* feat_idx = nullptr;  // nullptr: no map
  int32_t n_out = 0;
  int32_t n_master = 0;
  int32_t V = 1;
  int32_t n_chunks = 0;
  int32_t* mark = nullptr;
  int32_t* next = nullptr;
  int32_t* list = nullptr;
  int32_t* head = nullptr;
  int32_t* count = nullptr;
  int32_t* run = nullptr;
};

struct HistLaunch {
  const int8_t* codes;
  int64_t n_rows;
  int64_t stride;
  int32_t n_feats;
  const float* resid;                // residuals [tree][row]
  int64_t resid_tree_stride;
  const int32_t* shifts;             // quantisation shift per tree
  const int32_t* order;
  const Tile* tiles;
  const int32_t* n_tiles;
  int32_t keys_per_tree;
  int32_t num_bins;
  unsigned long long* part;  // packed tile partials (sum * 2^18 + count)
  int32_t V;
  int32_t n_chunks;
  int32_t max_tiles;
  // codes in the native layout (every byte in [0, num_bins + 1], written by
  // the library's binner / pre-binned copy): the kernel needs no clamp
  int32_t native = 0;
  // with order: resid holds the residuals in position order (resid[p] belongs
  // to row order[p]) instead of row order
  int32_t resid_by_pos = 0;
  // timer tag of the tile kernel (nullptr: not timed)
  const char* timer_tag = nullptr;
  ShiftFromMax sm;
  // selected features (fs.list != nullptr: n_feats bounds *fs.count; row
  // order required, raw codes only)
  FeatSel fs;
};

int hist_pick_v(int num_bins, int64_t n_feats);
size_t hist_lds_bytes(int V, int num_bins, bool native);
bool hist_native_ok(int num_bins);
int hist_load_mode(int64_t n_rows, int64_t stride, int V);
int launch_hist_tiles(const HistLaunch& a, hipStream_t st);
int probe_lds_atomics(int32_t blocks, int32_t iters, double* ops_per_s, hipStream_t st);
int probe_hbm_read(const void* buf, int64_t bytes, int32_t iters, double* bytes_per_s,
                   hipStream_t st);

// kernels launched directly from other translation units
// absmax_bits: the call's largest |residual| (float bits; key_stride 0), or
// each key's (key_stride 1); the shift follows from them and qbits
int launch_finalize_f32(int64_t tiles_per_key, const unsigned long long* part,
                        const int32_t* key_tile_start, int32_t n_keys, int32_t n_chunks, int32_t V,
                        int32_t num_bins, int32_t n_feats, const uint32_t* absmax_bits,
                        int32_t key_stride, int32_t qbits, const int32_t* n_tiles,
                        int32_t accumulate, FeatOut fo, float* G, float* H, hipStream_t st);
int launch_finalize_level(int64_t tiles_per_key, const unsigned long long* part,
                          const int32_t* key_tile_start, const int32_t* key_list, int32_t n_list,
                          int32_t n_chunks, int32_t V, int32_t num_bins, int32_t n_feats,
                          int32_t num_eras, int32_t nodes_in_level, int32_t depth,
                          const int64_t* parent_q, const int32_t* parent_c, const int32_t* n_tiles,
                          int64_t* hq, int32_t* hc, hipStream_t st);
__global__ void absmax_finish_kernel(const uint32_t* partial, int32_t n_part, int32_t qbits,
                                     uint32_t* absmax_bits, int32_t* shifts, int64_t* tot_qh,
                                     int64_t* tot_ql, int64_t* tot_c, int64_t n_rows);
__global__ void plan_tiles_kernel(const int64_t* seg, int64_t total, int32_t n_keys,
                                  const int32_t* key_list, int32_t tile_rows, int32_t nearest,
                                  int32_t max_tiles, Tile* tiles, int32_t* key_tile_start,
                                  int32_t* n_tiles);
__global__ void hist_prep_kernel(const float* resid, const int32_t* rows, int64_t n,
                                 uint32_t* partial, float* gathered, int32_t n_part, int32_t plan,
                                 const int64_t* seg, int32_t n_keys, int32_t tile_rows,
                                 int32_t max_tiles, Tile* tiles, int32_t* key_tile_start,
                                 int32_t* n_tiles, FeatMapArgs fm, uint32_t* key_max);
// the largest |residual| (float bits) of every key of a tile plan: one
// workgroup per tile, atomicMax into key_max (cleared by hist_prep_kernel);
// the residual of position p is resid[p] (by_pos), resid[order[p]], or
// resid[p] without an order
__global__ void hist_key_max_kernel(const Tile* tiles, const int32_t* n_tiles, const float* resid,
                                    const int32_t* order, int32_t by_pos, uint32_t* key_max);
// era regrouping of a row list (compute_histogram3 with eras): block counts,
// per-era scans, era starts, block scatter; no device-scope atomics
constexpr int kEraWindow = 8192;  // eras counted per LDS pass
__global__ void era_block_count_kernel(const int32_t* rows, int64_t n, const int32_t* era,
                                       int32_t num_eras, int64_t per_block, int32_t* counts);
__global__ void era_row_scan_kernel(int32_t* counts, int32_t num_eras, int32_t nb,
                                    int64_t* era_tot);
__global__ void era_start_scan_kernel(int64_t* era_tot, int32_t num_eras);
__global__ void era_block_scatter_kernel(const int32_t* rows, int64_t n, const int32_t* era,
                                         int32_t num_eras, int64_t per_block,
                                         const int32_t* offs, const int64_t* seg, int32_t* out);

// generic fills (graph-safe replacement for memset)
__global__ void fill_u32_kernel(uint32_t* p, int64_t n, uint32_t v);
__global__ void fill_u64_kernel(unsigned long long* p, int64_t n, unsigned long long v);
int fill_u32(uint32_t* p, int64_t n, uint32_t v, hipStream_t st);
int fill_u64(void* p, int64_t n, unsigned long long v, hipStream_t st);

// per-device scratch arena owned by the library (grow-only, stream-keyed)
void* scratch_get(hipStream_t st, size_t bytes, int slot);
void scratch_release_all();

// optional HIP-event timers of selected kernels: timer_begin(tag) gives a
// handle (null when timers are off) whose two events the launcher records
// around the launch on its stream (timer_mode() 1) or passes to
// hipExtLaunchKernel (mode 2); timer_end(handle) files the interval
bool timer_enabled();
int timer_mode();
void* timer_begin(const char* tag);
hipEvent_t timer_start_event(void* h);
hipEvent_t timer_stop_event(void* h);
void timer_end(void* h);
void timer_enable(int on);
int timer_read(const char* tag, double* total_ms, long* count);
void timer_reset();

// order-preserving map of float bits to uint32 (and back)
__device__ inline uint32_t gain_key(float g) {
  const uint32_t u = __float_as_uint(g);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ inline float gain_from_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

}  // namespace wgbm
