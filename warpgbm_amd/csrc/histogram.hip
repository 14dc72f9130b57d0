// Histogram building: per (segment, feature, bin) exact residual sums and row counts.
//
// Reference semantics (warpgbm/cuda/histogram_kernel.cu:16-59): for every row
// s of a node and every feature f, with e = era[s] and b = codes[s, feat[f]],
// if 0 <= b < B:  G[e,f,b] += residual[s];  H[e,f,b] += 1.
//
// MI355X design
// * Rows are processed in TILES; every tile lies inside one SEGMENT (a run of
//   the row-order array that shares one histogram: a node, or a (node, era)
//   pair).  One workgroup = one tile x one chunk of 64*V features.
// * Lane l of every wave owns the V consecutive features chunk*64*V + l*V ..
//   + V-1 and reads their codes with one V-byte buffer load per row, so one
//   load instruction covers 64*V contiguous bytes of one row.  A wave works
//   on one row at a time: the row index and its residual are wave-uniform
//   (scalar loads), and the software pipeline keeps U rows of loads in flight
//   per wave.
// * The workgroup histogram lives in LDS as packed 64-bit words
//   (q * 2^18 + 1: exact gradient sum and row count in one ds_add_u64).  Word
//   (j, b, lane) sits at index (j*(B+1) + b)*64 + lane: every lane updates its
//   own column, so the 64 lanes of an atomic never share an address or a
//   bank pair whatever the bin values are (no address or bank conflicts).
//   Bin B is a trash row for out-of-range codes (negative pre-binned codes and
//   features beyond the end of the row), which keeps the inner loop branch-free.
// * Each tile writes its partial histogram (exact int64 sum, int32 count) in
//   the LDS layout; a finalize kernel sums the tiles of a segment (integers, so
//   in any order) and rounds once to float32.
#include <hip/hip_ext.h>

#include "common.hpp"
#include "kernels.hpp"
#include "plan.hpp"

namespace wgbm {

// --------------------------------------------------------------------------
// tile accumulation
// --------------------------------------------------------------------------
// One workgroup (kHistThreads threads) = one tile x one chunk of 64*V features.
// The residuals of the tile's tree t = key / keys_per_tree are
// resid + t*resid_tree_stride, quantised with shifts[t].  BT > 0 fixes
// num_bins at compile time (LDS offsets become immediates).  GATHER: the rows
// of positions p are order[p] (else p); RPOS (with GATHER): the residual of
// position p is resid[p] (a copy already gathered into position order, read
// contiguously) instead of resid[order[p]].
//
// The kernel is bound by the LDS atomic unit (one 64-lane ds_add_u64 per row
// and feature quad) and by the code stream from HBM; everything else is
// arranged to keep both fed: 8 waves per SIMD (two workgroups per CU, at most
// 64 VGPRs), the row offset in the scalar offset of the code load, and a
// branch-free add.
//
// Two LDS layouts, both conflict-free (the lanes of one atomic never share a
// word or a bank pair, whatever the bins are):
// * raw codes (NAT = false): word (j, b, lane) at (j*(B+1) + b)*64 + lane; the
//   bin of a code byte is clamped to the trash bin B (codes outside [0, B)),
//   two VALU per atomic (a byte-select min, a shift-add).
// * native codes (NAT = true, every byte in [0, B+1]): 256-byte LDS rows of
//   32 lane words; lane l writes row j*2H + (l/32)*H + c, H = B + 2, so the
//   row index of a byte c is c + (l/32)*H (one add per loaded dword, no
//   carries: c + H <= 2B + 3 <= 255) and the address (row << 8) | (l%32)*8
//   is a single byte permute of the code dword with the lane offset; rows B
//   and B+1 of each half are the trash rows.  One VALU per atomic.
//
// FS (selected features, raw codes, row order): histogram feature h <
// *fs.count reads code column fs.list[h] (ascending).  A chunk whose lanes
// all own aligned runs of V consecutive columns (fs.run[chunk]: every
// feature selected, or sorted ranges) is loaded as above, lane l owning h =
// chunk*64*V + l*V + j, with one V-byte load per row.  Otherwise lane l owns
// h = chunk*64*V + j*64 + l and loads its V columns with V byte loads per
// row, each instruction covering 64 consecutive selected columns (few cache
// lines); U = 8/V rows per group, so the group's registers match the run
// path's.
template <int V, int MODE, int BT, bool GATHER, bool NAT, bool RPOS, bool FS>
__global__ __launch_bounds__(kHistThreads) __attribute__((amdgpu_waves_per_eu(8, 8)))
void hist_tiles_kernel(
    const int8_t* __restrict__ codes, int64_t n_rows, int64_t stride, int32_t n_feats,
    const float* __restrict__ resid, int64_t resid_tree_stride,
    const int32_t* __restrict__ shifts, const int32_t* __restrict__ order,
    const Tile* __restrict__ tiles, const int32_t* __restrict__ n_tiles, int32_t keys_per_tree,
    int32_t num_bins_rt, unsigned long long* __restrict__ part, ShiftFromMax sm, FeatSel fs) {
  static_assert(!FS || (GATHER && !NAT), "feature selection: row order and raw codes");
  // the only LDS of this kernel: with no static LDS it starts at LDS address
  // 0, so the NAT path can form LDS addresses as plain integers
  extern __shared__ unsigned long long lds[];
  constexpr int CW = kHistSlots * V;  // features per chunk
  const int num_bins = BT > 0 ? BT : num_bins_rt;
  const int n_chunks = (n_feats + CW - 1) / CW;
  // raw codes: (tile, chunk) work items in the XCD work order over the
  // planned tiles, so the chunks of a tile share an XCD and its L2 (a raw
  // row's chunks straddle 128-byte lines that the neighbouring chunk reads
  // too), each XCD with an even share of the planned work.  Native rows are
  // line-aligned: tile-major order, chunks round-robin over the XCDs.
  const int nt = *n_tiles;
  int tile_id, chunk;
  bool have;
  if constexpr (!NAT) {
    const int64_t n_work = (int64_t)nt * n_chunks;
    const int64_t per = (n_work + kXcds - 1) / kXcds;
    const int64_t xid = blockIdx.x;
    const int64_t wk = (xid % kXcds) * per + xid / kXcds;
    have = xid / kXcds < per && wk < n_work;
    tile_id = have ? (int)(wk / n_chunks) : nt;
    chunk = have ? (int)(wk - (int64_t)tile_id * n_chunks) : 0;
  } else {
    tile_id = blockIdx.x / n_chunks;
    chunk = blockIdx.x - tile_id * n_chunks;
    have = tile_id < nt;
  }
  // sm.partial (one tree): every wave reduces the call's per-block maxima of
  // |residual| to the shift itself (no separate launch); workgroup 0, which
  // always exists, stores the maximum and the shift for the finalize
  int s_call = 0;
  if (sm.partial) {
    const int lane0 = threadIdx.x & 63;
    uint32_t m = 0;
    for (int i = lane0; i < sm.n_part; i += 64) {
      const uint32_t v = sm.partial[i];
      m = v > m ? v : m;
    }
    m = wgbm_wave_max_u32(m);
    s_call = m >= 0x7f800000u ? 0 : wgbm_shift_from_absmax(__uint_as_float(m), sm.qbits);
    if (blockIdx.x == 0 && threadIdx.x == 0) {
      *sm.absmax_bits = m;
      *sm.shift = s_call;
    }
  }
  if (!have) return;
  // FS: chunks past the selected features (the grid is sized for the
  // host's bound) have nothing to do; their partials are never read
  const int n_sel = FS ? *fs.count : n_feats;
  if (FS && chunk * CW >= n_sel) return;
  const Tile tl = tiles[tile_id];
  const int Bp = num_bins + 1;
  const int Hn = num_bins + 2;  // NAT: rows per lane half
  const int nent = NAT ? V * 2 * Hn * 32 : V * Bp * kHistSlots;
  for (int i = threadIdx.x; i < nent; i += kHistThreads) lds[i] = 0ull;
  __syncthreads();

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int nwaves = kHistThreads / 64;
  const int f_base = chunk * CW + lane * V;
  const int tree = tl.key / keys_per_tree;
  const float* __restrict__ r_t = resid + (int64_t)tree * resid_tree_stride;
  // Shifts lie in [qbits - 128, qbits + 149] = [-120, 177] (frexp exponent of
  // a finite float32 maximum); negative ones quantise residuals of magnitude
  // 2^qbits and above.  The clamp to a wider range changes no shift: it
  // consumes the loaded value here, so the wait for the (scalar) load happens
  // once before the loop rather than at the top of every iteration, where it
  // would also drain the wave's outstanding LDS atomics (both share one
  // counter).
  const int s_raw = sm.partial   ? __builtin_amdgcn_readfirstlane(s_call)
                    : sm.key_max ? wgbm_shift_from_bits(sm.key_max[tl.key], sm.qbits)
                                 : shifts[tree];
  const int s = s_raw < -160 ? -160 : (s_raw > 255 ? 255 : s_raw);
  const int32_t* __restrict__ ord = GATHER ? order + tl.begin : nullptr;
  const int n = (int)(tl.end - tl.begin);  // a tile has at most 65536 rows
  // A lane past the last feature adds whatever it reads to its own words,
  // which belong to no feature and are never read back; every address stays
  // inside the lane's column (raw codes: out-of-range bytes go to the trash
  // bin; native codes are in range).  It reads nothing new: an out-of-range
  // buffer offset (returns zeros without a memory access), or the last real
  // feature's offset, whose line the wave fetches anyway.
  // FS: the chunk's lane ownership and the lane's code columns (-1 past the
  // selected features).  In a run chunk the V-byte load starts at the lane's
  // first column and may cover unselected columns past the last selected
  // one, whose words belong to histogram features >= n_sel and are never
  // read back.
  int mcol[V];
  bool run_ok = true;
  if constexpr (FS) {
    run_ok = fs.run[chunk] != 0;
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int h = chunk * CW + (run_ok ? lane * V + j : j * kHistSlots + lane);
      mcol[j] = h < n_sel ? fs.list[h] : -1;
    }
  }
  const int n_cols = FS ? fs.n_master : n_feats;  // code columns of a row
  const int lane_col = FS ? mcol[0] : (f_base < n_feats ? f_base : -1);
  const int vlast = (n_cols - 1) / V * V;
  const int voff = lane_col >= 0 ? lane_col : (MODE == kLoadBuffer ? 0x7fffffff : vlast);
  const int n_valid_bytes =
      lane_col >= 0 ? (n_cols - lane_col < V ? n_cols - lane_col : V) : 0;
  const uint32_t rs_bytes = (MODE == kLoadBuffer) ? (uint32_t)(n_rows * stride) : 0u;
  const __amdgpu_buffer_rsrc_t rs = wgbm_rsrc(codes, rs_bytes);
  unsigned long long* my = lds + lane;
  // NAT: lane offset inside a 256-byte row, and the row offset of the lane's
  // half added to every code byte of its dword
  const uint32_t lane_lo8 = (uint32_t)(lane & 31) * 8u;
  const uint32_t half_add =
      (lane >> 5) ? (uint32_t)Hn * (V == 4 ? 0x01010101u : (V == 2 ? 0x0101u : 1u)) : 0u;
  const uint32_t plane_bytes = (uint32_t)(2 * Hn) * 256u;

  // software pipeline: wave w takes the row groups [i, i + U) with
  // i = (w + k*nwaves)*U (tile-relative).  Two register sets alternate: the
  // loads of group k+1 are in flight while group k is added into LDS.  The
  // loop is unrolled twice so that neither set is ever copied (a copy would
  // wait for every outstanding load).  Positions past the tile end (last
  // group only) repeat the tile's last row and add nothing.
  constexpr int U = 8;  // <= 16: the NAT path broadcasts within 16-lane rows
  constexpr int step = nwaves * U;
  struct Group {
    uint32_t c[U];  // codes of rows 0..U-1 of the group (all lanes)
    float r;        // lane l: residual of row l % U
  };
  Group ga, gb;
  const int row0 = (int)tl.begin;  // row ids fit 31 bits (checked by the launcher)
  const int ul = lane & (U - 1);
  // GATHER: lane l holds order[i0 + l % U] of the next group to issue; read
  // one issue ahead so that turning it into scalar row ids never waits
  int32_t ids = 0;
  auto load_ids = [&](int i0) {
    if constexpr (GATHER) {
      const int iu = i0 + ul < n ? i0 + ul : n - 1;
      ids = ord[iu];
    }
  };
  auto issue = [&](Group& g, int i0) {
    int rows[U];
#pragma unroll
    for (int u = 0; u < U; ++u)
      rows[u] = GATHER ? __builtin_amdgcn_readlane(ids, u) : row0 + (i0 + u < n ? i0 + u : n - 1);
    // residuals: one vector load per group (lane l reads row l % U's)
    const int my_pos = row0 + (i0 + ul < n ? i0 + ul : n - 1);
    g.r = r_t[(GATHER && !RPOS) ? ids : my_pos];
    if constexpr (GATHER) load_ids(i0 + step);
#pragma unroll
    for (int u = 0; u < U; ++u) {
      if (MODE == kLoadBuffer) {
        const int so = rows[u] * (int)stride;  // n_rows * stride < 2^31 in this mode
        if constexpr (V == 4)
          g.c[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, voff, so, kAuxStream);
        else if constexpr (V == 2)
          g.c[u] = __builtin_amdgcn_raw_buffer_load_b16(rs, voff, so, kAuxStream);
        else
          g.c[u] = __builtin_amdgcn_raw_buffer_load_b8(rs, voff, so, kAuxStream);
      } else if (MODE == kLoadGlobalAligned) {
        // row stride and chunk offsets are multiples of V bytes: aligned loads
        // that never run past the row (voff + V <= stride)
        const int8_t* src = codes + (int64_t)rows[u] * stride + voff;
        if constexpr (V == 4)
          g.c[u] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(src));
        else if constexpr (V == 2)
          g.c[u] = __builtin_nontemporal_load(reinterpret_cast<const uint16_t*>(src));
        else
          g.c[u] = __builtin_nontemporal_load(reinterpret_cast<const uint8_t*>(src));
      } else {
        // byte loads for unaligned strides; only bytes of real features are read
        const int8_t* src = codes + (int64_t)rows[u] * stride + voff;
        uint32_t w8 = 0;
#pragma unroll
        for (int j = 0; j < V; ++j)
          if (j < n_valid_bytes) w8 |= (uint32_t)(uint8_t)src[j] << (8 * j);
        g.c[u] = w8;
      }
    }
  };
  // branch-free: positions past the tile end add the word 0 (no sum, no
  // count)
  auto add = [&](const Group& g, int i0) {
    // the group's packed words, quantised once (lane l: row l % U)
    const int64_t qv = (int64_t)wgbm_quantise(g.r, s);
    const uint64_t pv = (uint64_t)(qv * (int64_t)(1 << WGBM_CBITS) + 1);
    if constexpr (NAT) {
      const unsigned long long pm = i0 + ul < n ? (unsigned long long)pv : 0ull;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // row u's word in every lane (DPP broadcast of lane u of each row of 16)
        const unsigned long long w = wgbm_row_bcast(pm, u);
        const uint32_t cw = g.c[u] + half_add;
#pragma unroll
        for (int j = 0; j < V; ++j) {
          const uint32_t addr = __builtin_amdgcn_perm(cw, lane_lo8, 0x0c0c0000u | ((4u + j) << 8));
          __hip_atomic_fetch_add((wgbm_lds_u64*)(uintptr_t)(addr + (uint32_t)j * plane_bytes), w,
                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    } else {
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
          // out-of-range code (incl. negative int8, read as >= 128) -> trash bin
          c = c < (uint32_t)num_bins ? c : (uint32_t)num_bins;
          atomicAdd(my + (j * Bp + (int)c) * kHistSlots, w);
        }
        // one row at a time: hoisting the next rows' work above these atomics
        // only raises register pressure (the LDS unit is the bottleneck)
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  // the software pipeline over the wave's row groups (group size UU)
  auto pipeline = [&](auto& a, auto& b, int uu, auto&& first_ids, auto&& iss, auto&& ad) {
    const int stp = nwaves * uu;
    int i = wave * uu;
    if (i < n) {
      first_ids(i);
      iss(a, i);
      // steady state without conditional loads, so that every add waits for
      // exactly its own group (the other group's loads stay in flight)
      while (i + 2 * stp < n) {
        iss(b, i + stp);
        ad(a, i);
        iss(a, i + 2 * stp);
        ad(b, i + stp);
        i += 2 * stp;
      }
      if (i + stp < n) {
        iss(b, i + stp);
        ad(a, i);
        ad(b, i + stp);
      } else {
        ad(a, i);
      }
    }
  };
  if (!FS || run_ok) {
    pipeline(ga, gb, U, load_ids, issue, add);
  } else if constexpr (FS) {
    // per-column byte loads: UG rows per group, V bytes each
    constexpr int UG = 8 / V;
    constexpr int stepg = nwaves * UG;
    struct GroupB {
      uint32_t c[UG][V];  // zero-extended code bytes
      float r;            // lane l: residual of row l % UG
    };
    GroupB ha, hb;
    // buffer mode (row stride a multiple of 4, out-of-range offsets read
    // zeros): the dword that holds the column, the byte taken by a shift;
    // otherwise byte loads
    const int col_fill = MODE == kLoadBuffer ? 0x7ffffffc : fs.list[n_sel - 1];
    int vcol[V];
    uint32_t vsh[V];
#pragma unroll
    for (int j = 0; j < V; ++j) {
      const int cj = mcol[j] >= 0 ? mcol[j] : col_fill;
      vcol[j] = MODE == kLoadBuffer ? (cj & ~3) : cj;
      vsh[j] = MODE == kLoadBuffer ? (uint32_t)(cj & 3) * 8u : 0u;
    }
    const int ug = lane & (UG - 1);
    int32_t idg = 0;
    auto load_idg = [&](int i0) {
      const int iu = i0 + ug < n ? i0 + ug : n - 1;
      idg = ord[iu];
    };
    auto issue_b = [&](GroupB& g, int i0) {
      int rows[UG];
#pragma unroll
      for (int u = 0; u < UG; ++u) rows[u] = __builtin_amdgcn_readlane(idg, u);
      const int my_pos = row0 + (i0 + ug < n ? i0 + ug : n - 1);
      g.r = r_t[RPOS ? my_pos : idg];
      load_idg(i0 + stepg);
#pragma unroll
      for (int u = 0; u < UG; ++u) {
#pragma unroll
        for (int j = 0; j < V; ++j) {
          if (MODE == kLoadBuffer) {
            g.c[u][j] = __builtin_amdgcn_raw_buffer_load_b32(rs, vcol[j], rows[u] * (int)stride,
                                                             kAuxStream);
          } else {
            const uint8_t* src =
                reinterpret_cast<const uint8_t*>(codes) + (int64_t)rows[u] * stride + vcol[j];
            g.c[u][j] = __builtin_nontemporal_load(src);
          }
        }
      }
    };
    auto add_b = [&](const GroupB& g, int i0) {
      const int64_t qv = (int64_t)wgbm_quantise(g.r, s);
      const uint64_t pv = (uint64_t)(qv * (int64_t)(1 << WGBM_CBITS) + 1);
      const uint32_t plo = (uint32_t)pv, phi = (uint32_t)(pv >> 32);
#pragma unroll
      for (int u = 0; u < UG; ++u) {
        const uint64_t wu = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane(phi, u) << 32) |
                            (uint64_t)(uint32_t)__builtin_amdgcn_readlane(plo, u);
        const unsigned long long w = i0 + u < n ? (unsigned long long)wu : 0ull;
#pragma unroll
        for (int j = 0; j < V; ++j) {
          // out-of-range code (incl. negative int8, read as >= 128) -> trash bin
          uint32_t c = (g.c[u][j] >> vsh[j]) & 0xffu;
          c = c < (uint32_t)num_bins ? c : (uint32_t)num_bins;
          atomicAdd(my + (j * Bp + (int)c) * kHistSlots, w);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    pipeline(ha, hb, UG, load_idg, issue_b, add_b);
  }
  __syncthreads();

  // flush in the partial layout part[tile][chunk][j][b][lane] (trash rows
  // dropped); the packed word (sum * 2^18 + count) is stored as is and
  // unpacked by finalize.  Two words (lanes l, l+1 of one (j, b)) per thread
  // and store: 16-byte non-temporal stores (every workgroup flushes at the
  // same time at the end, so the stores should not wait on cache lines)
  const int64_t tile_words = (int64_t)n_chunks * CW * num_bins;
  const int64_t chunk_off = (int64_t)tile_id * tile_words + (int64_t)chunk * CW * num_bins;
  const int npair = V * num_bins * kHistSlots / 2;
  typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
  for (int k2 = threadIdx.x; k2 < npair; k2 += kHistThreads) {
    const int k = 2 * k2;
    const int sl = k & (kHistSlots - 1);  // even: sl and sl + 1 share (j, b) and a lane half
    const int jb = k / kHistSlots;        // j*B + b
    const int j = jb / num_bins;
    const int b = jb - j * num_bins;
    const int src = NAT ? (j * 2 * Hn + (sl >> 5) * Hn + b) * 32 + (sl & 31)
                        : (j * Bp + b) * kHistSlots + sl;
    const u64x2 v = *reinterpret_cast<const u64x2*>(lds + src);
    __builtin_nontemporal_store(v, reinterpret_cast<u64x2*>(part + chunk_off + k));
  }
}

// unpack a packed tile word into (exact sum, count)
__device__ inline void unpack_word(unsigned long long P, int64_t& Q, int64_t& C) {
  // P = q * 2^18 + c with 0 <= c < 2^18: the arithmetic shift is floor(P / 2^18) = q
  C = (int64_t)(P & (unsigned long long)WGBM_CMASK);
  Q = (int64_t)P >> WGBM_CBITS;
}

// partial-layout index i (within one tile) -> (feature, bin)
__device__ inline void part_feature_bin(int i, int V, int num_bins, int& f, int& b) {
  const int per_chunk = kHistSlots * V * num_bins;
  const int chunk = i / per_chunk;
  const int r = i - chunk * per_chunk;
  const int sl = r & (kHistSlots - 1);
  const int jb = r / kHistSlots;
  const int j = jb / num_bins;
  b = jb - j * num_bins;
  f = chunk * kHistSlots * V + sl * V + j;
}

// the same with the lane ownership of selected-feature chunks (run ==
// nullptr or run[chunk] != 0: lane-major as above; else feature chunk*64*V
// + j*64 + lane)
__device__ inline void part_feature_bin_sel(int i, int V, int num_bins,
                                            const int32_t* __restrict__ run, int& f, int& b) {
  const int per_chunk = kHistSlots * V * num_bins;
  const int chunk = i / per_chunk;
  const int r = i - chunk * per_chunk;
  const int sl = r & (kHistSlots - 1);
  const int jb = r / kHistSlots;
  const int j = jb / num_bins;
  b = jb - j * num_bins;
  const bool lane_major = run == nullptr || run[chunk] != 0;
  f = chunk * kHistSlots * V + (lane_major ? sl * V + j : j * kHistSlots + sl);
}

// --------------------------------------------------------------------------
// finalize (f32): for every segment k and every (feature, bin) of the tile
// layout, sum the tiles of k (integers) and write
//   G[k, f, b] (+)= float(sum * 2^-s),  H[k, f, b] (+)= count.
// Threads walk the partials in their memory order, so reads are coalesced.
// accumulate = 0 overwrites (scratch output), 1 adds (reference semantics).
// --------------------------------------------------------------------------
// A workgroup of 256 threads covers FW consecutive partial words of one
// segment; its 256/FW thread groups each sum every (256/FW)-th tile and the
// groups are combined in LDS (integer sums, so the split does not change the
// result).  Few tiles per segment -> wide FW (long coalesced runs, few
// workgroups); many tiles -> narrow FW (more parallel tile reads).
template <int FW>
__device__ inline void finalize_sum(const unsigned long long* __restrict__ part, int64_t tile_words,
                                    int i, bool ok, int t0, int t1, int64_t& Q, int64_t& C) {
  constexpr int SPLIT = 256 / FW;
  __shared__ int64_t sq[SPLIT][FW];
  __shared__ int64_t sc[SPLIT][FW];
  const int w = threadIdx.x % FW;
  const int g = threadIdx.x / FW;
  int64_t q = 0, c = 0;
  if (ok) {
    // four tiles' loads in flight per step (the partials are read once)
    const unsigned long long* __restrict__ p = part + i;
    int t = t0 + g;
    for (; t + 3 * SPLIT < t1; t += 4 * SPLIT) {
      unsigned long long P[4];
#pragma unroll
      for (int u = 0; u < 4; ++u)
        P[u] = __builtin_nontemporal_load(p + (int64_t)(t + u * SPLIT) * tile_words);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        int64_t a, b;
        unpack_word(P[u], a, b);
        q += a;
        c += b;
      }
    }
    for (; t < t1; t += SPLIT) {
      int64_t a, b;
      unpack_word(__builtin_nontemporal_load(p + (int64_t)t * tile_words), a, b);
      q += a;
      c += b;
    }
  }
  sq[g][w] = q;
  sc[g][w] = c;
  wgbm_lds_barrier();
  Q = 0;
  C = 0;
  for (int k = 0; k < SPLIT; ++k) {
    Q += sq[k][w];
    C += sc[k][w];
  }
}

template <int FW>
__global__ __launch_bounds__(256) void hist_finalize_f32_kernel(
    const unsigned long long* __restrict__ part, const int32_t* __restrict__ key_tile_start,
    int32_t n_keys, int32_t n_chunks, int32_t V, int32_t num_bins, int32_t n_feats,
    const uint32_t* __restrict__ absmax_bits, int32_t key_stride, int32_t qbits,
    const int32_t* __restrict__ n_tiles, int32_t accumulate, FeatOut fo, float* __restrict__ G,
    float* __restrict__ H) {
  // tile_words < 2^31 (checked by the launcher)
  const int tile_words = n_chunks * kHistSlots * V * num_bins;
  const int wpk = (tile_words + FW - 1) / FW;  // workgroups per segment
  const int k = (int)blockIdx.x / wpk;
  const int i = ((int)blockIdx.x - k * wpk) * FW + (int)threadIdx.x % FW;
  const int n_hist = fo.head ? *fo.count : n_feats;  // histogram features with outputs
  int f = 0, b = 0;
  bool ok = k < n_keys && i < tile_words;
  if (ok) {
    part_feature_bin_sel(i, V, num_bins, fo.run, f, b);
    ok = f < n_hist;
  }
  int t0 = 0, t1 = 0;
  if (k < n_keys) {
    t0 = key_tile_start[k];
    t1 = key_tile_start[k + 1] < *n_tiles ? key_tile_start[k + 1] : *n_tiles;
  }
  int64_t Q, C;
  finalize_sum<FW>(part, tile_words, i, ok, t0, t1, Q, C);
  if (!ok || threadIdx.x >= FW) return;
  const uint32_t mb = absmax_bits[key_stride ? k : 0];
  const bool bad = mb >= 0x7f800000u;  // non-finite residual seen
  const float g = bad ? __builtin_nanf("") : wgbm_dequantise(Q, wgbm_shift_from_bits(mb, qbits));
  const float h = (float)C;
  const int n_out = fo.head ? fo.n_out : n_feats;
  for (int of = fo.head ? fo.head[f] : f; of >= 0; of = fo.head ? fo.next[of] : -1) {
    const int64_t o = ((int64_t)k * n_out + of) * num_bins + b;
    if (accumulate) {
      G[o] = G[o] + g;
      H[o] = H[o] + h;
    } else {
      G[o] = g;
      H[o] = h;
    }
  }
}

// --------------------------------------------------------------------------
// plane finalize: one workgroup (1024 threads) per (segment, plane), where a
// plane is the B x 64 partial words of one (chunk, j): bins b of the 64
// features chunk*64V + lane*V + j.  Four thread groups sum every fourth tile
// of the segment (each thread 1..16 words of the plane, all their loads of
// one tile in flight together), the groups are combined with LDS integer
// adds into [b][lane] tables padded to 65 words a row, and the workgroup
// then writes the outputs in their [feature][bin] order: 32 threads write the
// B contiguous bins of one feature (coalesced rows, where a word-per-thread
// finalize stores with a stride of V*B words).  Used when there are many
// segments, each with few tiles.
// --------------------------------------------------------------------------
constexpr int kPlaneThreads = 1024;
constexpr int kPlaneGroups = 4;
constexpr int kPlaneMaxBins = 64;  // words per thread: B*64/256 <= 16
constexpr int kPlaneRow = 65;

// MB: the largest num_bins of the instance (register arrays are sized by
// it); PT threads in PG groups (group g sums tiles t0 + g, t0 + g + PG, ...)
template <int MB = kPlaneMaxBins, int PT = kPlaneThreads, int PG = kPlaneGroups>
__device__ inline void plane_sum(const unsigned long long* __restrict__ part, int64_t tile_words,
                                 int plane_off, int num_bins, int t0, int t1,
                                 unsigned long long* sq, unsigned int* sc) {
  const int W = num_bins * kHistSlots;
  for (int i = threadIdx.x; i < num_bins * kPlaneRow; i += PT) {
    sq[i] = 0ull;
    sc[i] = 0u;
  }
  wgbm_lds_barrier();
  const int g = threadIdx.x / (PT / PG);
  const int lt = threadIdx.x % (PT / PG);
  constexpr int kMaxW = MB * kHistSlots / (PT / PG);
  int64_t q[kMaxW];
  int64_t c[kMaxW];
#pragma unroll
  for (int k = 0; k < kMaxW; ++k) q[k] = c[k] = 0;
  for (int t = t0 + g; t < t1; t += PG) {
    const unsigned long long* __restrict__ p = part + (int64_t)t * tile_words + plane_off;
    unsigned long long P[kMaxW];
#pragma unroll
    for (int k = 0; k < kMaxW; ++k) {
      const int w = lt + k * (PT / PG);
      P[k] = w < W ? __builtin_nontemporal_load(p + w) : 0ull;
    }
#pragma unroll
    for (int k = 0; k < kMaxW; ++k) {
      int64_t a, b;
      unpack_word(P[k], a, b);
      q[k] += a;
      c[k] += b;
    }
  }
#pragma unroll
  for (int k = 0; k < kMaxW; ++k) {
    const int w = lt + k * (PT / PG);
    if (w < W && t1 > t0) {
      const int li = (w / kHistSlots) * kPlaneRow + (w % kHistSlots);  // [b][lane]
      atomicAdd(sq + li, (unsigned long long)q[k]);  // two's complement: exact
      atomicAdd(sc + li, (unsigned int)c[k]);
    }
  }
  wgbm_lds_barrier();
}

// G[k, f, b] (+)= float(sum * 2^-s), H[k, f, b] (+)= count
__global__ __launch_bounds__(kPlaneThreads) void hist_finalize_plane_f32_kernel(
    const unsigned long long* __restrict__ part, const int32_t* __restrict__ key_tile_start,
    int32_t n_keys, int32_t n_chunks, int32_t V, int32_t num_bins, int32_t n_feats,
    const uint32_t* __restrict__ absmax_bits, int32_t key_stride, int32_t qbits,
    const int32_t* __restrict__ n_tiles, int32_t accumulate, FeatOut fo, float* __restrict__ G,
    float* __restrict__ H) {
  __shared__ unsigned long long sq[kPlaneMaxBins * kPlaneRow];
  __shared__ unsigned int sc[kPlaneMaxBins * kPlaneRow];
  const int P = n_chunks * V;
  const int k = (int)blockIdx.x / P;
  const int plane = (int)blockIdx.x - k * P;
  if (k >= n_keys) return;  // uniform per workgroup
  const int chunk = plane / V, j = plane - (plane / V) * V;
  const int n_hist = fo.head ? *fo.count : n_feats;  // histogram features with outputs
  if (chunk * kHistSlots * V >= n_hist) return;     // uniform per workgroup
  const int64_t tile_words = (int64_t)n_chunks * kHistSlots * V * num_bins;
  const int t0 = key_tile_start[k];
  const int t1 = key_tile_start[k + 1] < *n_tiles ? key_tile_start[k + 1] : *n_tiles;
  plane_sum(part, tile_words, plane * num_bins * kHistSlots, num_bins, t0, t1, sq, sc);
  const uint32_t mb = absmax_bits[key_stride ? k : 0];
  const bool bad = mb >= 0x7f800000u;  // non-finite residual seen
  const int s = wgbm_shift_from_bits(mb, qbits);
  const int n_out = fo.head ? fo.n_out : n_feats;
  const bool lane_major = fo.run == nullptr || fo.run[chunk] != 0;
  for (int o = threadIdx.x; o < kHistSlots * num_bins; o += kPlaneThreads) {
    const int lane = o / num_bins, b = o - lane * num_bins;
    const int f = chunk * kHistSlots * V + (lane_major ? lane * V + j : j * kHistSlots + lane);
    if (f >= n_hist) continue;
    const int li = b * kPlaneRow + lane;
    const float g = bad ? __builtin_nanf("") : wgbm_dequantise((int64_t)sq[li], s);
    const float h = (float)sc[li];
    for (int of = fo.head ? fo.head[f] : f; of >= 0; of = fo.head ? fo.next[of] : -1) {
      const int64_t out = ((int64_t)k * n_out + of) * num_bins + b;
      if (accumulate) {
        G[out] = G[out] + g;
        H[out] = H[out] + h;
      } else {
        G[out] = g;
        H[out] = h;
      }
    }
  }
}

// the engine's level arrays (exact int64 sums, int32 counts) and the sibling
// as parent - computed child; key layout and list pairs as
// hist_finalize_level_kernel
template <int MB, int PT, int PG>
__global__ __launch_bounds__(PT) void hist_finalize_plane_level_kernel(
    const unsigned long long* __restrict__ part, const int32_t* __restrict__ key_tile_start,
    const int32_t* __restrict__ key_list, int32_t n_list, int32_t n_chunks, int32_t V,
    int32_t num_bins, int32_t n_feats, int32_t num_eras, int32_t nodes_in_level, int32_t depth,
    const int64_t* __restrict__ parent_q, const int32_t* __restrict__ parent_c,
    const int32_t* __restrict__ n_tiles, int64_t* __restrict__ hq, int32_t* __restrict__ hc) {
  __shared__ unsigned long long sq[MB * kPlaneRow];
  __shared__ unsigned int sc[MB * kPlaneRow];
  const int P = n_chunks * V;
  const int kk = (int)blockIdx.x / P;
  const int plane = (int)blockIdx.x - kk * P;
  if (kk >= n_list) return;  // uniform per workgroup
  // the list words in one round of loads (the tile range does not depend on
  // the key), the parent words of a derived sibling with the partials
  const int key = key_list ? key_list[kk] : kk;
  const int pair = depth > 0 ? key_list[kk ^ 1] : 0;
  const int ts0 = key_tile_start[kk], ts1 = key_tile_start[kk + 1], ntl = *n_tiles;
  if (key < 0) return;  // uniform per workgroup
  const int chunk = plane / V, j = plane - (plane / V) * V;
  const int64_t tile_words = (int64_t)n_chunks * kHistSlots * V * num_bins;
  const int64_t per_key = (int64_t)n_feats * num_bins;
  int64_t pkey = 0, skey = 0;
  // the sibling by subtraction unless it is histogrammed itself (the second
  // entry of the list pair)
  const bool derive = depth > 0 && pair < 0;
  if (derive) {
    const int era = key % num_eras;
    const int tn = key / num_eras;
    const int node = tn % nodes_in_level;
    const int tree = tn / nodes_in_level;
    pkey = ((int64_t)tree * (nodes_in_level >> 1) + (node >> 1)) * num_eras + era;
    skey = ((int64_t)tree * nodes_in_level + (node ^ 1)) * num_eras + era;
  }
  // this thread's outputs (o = threadIdx.x + m * kPlaneThreads) and their
  // parent words, loaded with the partials (up to 32 bins; beyond, the
  // registers go to the partial sums and the parents load afterwards)
  constexpr int kOut = MB * kHistSlots / PT;
  constexpr bool kPre = MB <= 32;
  int64_t pq[kOut];
  int32_t pc[kOut];
#pragma unroll
  for (int m = 0; m < kOut; ++m) {
    const int o = threadIdx.x + m * PT;
    const int lane = o / num_bins, b = o - lane * num_bins;
    const int f = chunk * kHistSlots * V + lane * V + j;
    pq[m] = 0;
    pc[m] = 0;
    if (kPre && derive && o < kHistSlots * num_bins && f < n_feats) {
      const int64_t fb = (int64_t)f * num_bins + b;
      pq[m] = parent_q[pkey * per_key + fb];
      pc[m] = parent_c[pkey * per_key + fb];
    }
  }
  const int t0 = ts0;
  const int t1 = ts1 < ntl ? ts1 : ntl;
  plane_sum<MB, PT, PG>(part, tile_words, plane * num_bins * kHistSlots, num_bins, t0, t1, sq, sc);
#pragma unroll
  for (int m = 0; m < kOut; ++m) {
    const int o = threadIdx.x + m * PT;
    if (o >= kHistSlots * num_bins) break;
    const int lane = o / num_bins, b = o - lane * num_bins;
    const int f = chunk * kHistSlots * V + lane * V + j;
    if (f >= n_feats) continue;
    const int li = b * kPlaneRow + lane;
    const int64_t Q = (int64_t)sq[li];
    const int32_t C = (int32_t)sc[li];
    const int64_t fb = (int64_t)f * num_bins + b;
    hq[(int64_t)key * per_key + fb] = Q;
    hc[(int64_t)key * per_key + fb] = C;
    if (derive) {
      const int64_t pqm = kPre ? pq[m] : parent_q[pkey * per_key + fb];
      const int32_t pcm = kPre ? pc[m] : parent_c[pkey * per_key + fb];
      hq[skey * per_key + fb] = pqm - Q;
      hc[skey * per_key + fb] = pcm - C;
    }
  }
}

// --------------------------------------------------------------------------
// finalize for the level-wise engine: exact int64 sums into the level arrays,
// plus the sibling histogram as (parent - computed child), also exact.
//   computed key k = (tree, node, era) with node = 2*parent + side
//   hq/hc layout: [tree][node][era][F][B]
// Below the root the key list holds pairs (entries 2j, 2j + 1): the computed
// child and -1 (its sibling is derived here), or both children (each
// histogrammed at its own shift; nothing is derived).
// --------------------------------------------------------------------------
template <int FW>
__global__ __launch_bounds__(256) void hist_finalize_level_kernel(
    const unsigned long long* __restrict__ part, const int32_t* __restrict__ key_tile_start,
    const int32_t* __restrict__ key_list, int32_t n_list, int32_t n_chunks, int32_t V,
    int32_t num_bins, int32_t n_feats, int32_t num_eras, int32_t nodes_in_level, int32_t depth,
    const int64_t* __restrict__ parent_q, const int32_t* __restrict__ parent_c,
    const int32_t* __restrict__ n_tiles, int64_t* __restrict__ hq, int32_t* __restrict__ hc) {
  // tile_words < 2^31 (checked by the launcher)
  const int tile_words = n_chunks * kHistSlots * V * num_bins;
  const int wpk = (tile_words + FW - 1) / FW;
  const int kk = (int)blockIdx.x / wpk;
  if (kk >= n_list) return;  // uniform per workgroup
  // the list words in one round of loads (the tile range does not depend on
  // the key), the parent words of a derived sibling with the partials
  const int key = key_list ? key_list[kk] : kk;
  const int pair = depth > 0 ? key_list[kk ^ 1] : 0;
  const int ts0 = key_tile_start[kk], ts1 = key_tile_start[kk + 1], ntl = *n_tiles;
  if (key < 0) return;  // uniform per workgroup
  const int i = ((int)blockIdx.x - kk * wpk) * FW + (int)threadIdx.x % FW;
  const bool ok = i < tile_words;
  int f = 0, b = 0;
  if (ok) part_feature_bin(i, V, num_bins, f, b);
  const int64_t per_key = (int64_t)n_feats * num_bins;
  const int64_t fb = (int64_t)f * num_bins + b;
  // the sibling by subtraction unless it is histogrammed itself
  const bool derive = depth > 0 && pair < 0;
  int64_t skey = 0, pq = 0;
  int32_t pc = 0;
  if (derive && ok && threadIdx.x < FW && f < n_feats) {
    // key = ((tree*nodes + node)*E + era)
    const int era = key % num_eras;
    const int tn = key / num_eras;
    const int node = tn % nodes_in_level;
    const int tree = tn / nodes_in_level;
    const int64_t pkey = ((int64_t)tree * (nodes_in_level >> 1) + (node >> 1)) * num_eras + era;
    skey = ((int64_t)tree * nodes_in_level + (node ^ 1)) * num_eras + era;
    pq = parent_q[pkey * per_key + fb];
    pc = parent_c[pkey * per_key + fb];
  }
  const int t0 = ts0;
  const int t1 = ts1 < ntl ? ts1 : ntl;
  int64_t Q, C;
  finalize_sum<FW>(part, tile_words, i, ok, t0, t1, Q, C);
  if (!ok || threadIdx.x >= FW) return;
  if (f >= n_feats) return;
  hq[(int64_t)key * per_key + fb] = Q;
  hc[(int64_t)key * per_key + fb] = (int32_t)C;
  if (derive) {
    hq[skey * per_key + fb] = pq - Q;
    hc[skey * per_key + fb] = pc - (int32_t)C;
  }
}

// one workgroup per independent maximum t: reduce partial[t*n_part ...] and
// turn it into the quantisation shift (0 for an all-zero or non-finite input;
// absmax_bits keeps the raw maximum so a NaN/inf input can be reported).
// With tot_qh, also tree t's root totals words made ready for the root's
// atomic sums (root_setup_e1_kernel): sums 0, count n_rows.
__global__ void absmax_finish_kernel(const uint32_t* __restrict__ partial, int32_t n_part,
                                     int32_t qbits, uint32_t* __restrict__ absmax_bits,
                                     int32_t* __restrict__ shifts, int64_t* __restrict__ tot_qh,
                                     int64_t* __restrict__ tot_ql, int64_t* __restrict__ tot_c,
                                     int64_t n_rows) {
  const int t = blockIdx.x;
  if (tot_qh && threadIdx.x == 0) {
    tot_qh[t] = 0;
    tot_ql[t] = 0;
    tot_c[t] = n_rows;
  }
  uint32_t m = 0;
  for (int i = threadIdx.x; i < n_part; i += blockDim.x) {
    const uint32_t b = partial[(int64_t)t * n_part + i];
    m = b > m ? b : m;
  }
  m = wgbm_block_max_u32(m);
  if (threadIdx.x == 0) {
    absmax_bits[t] = m;
    shifts[t] = m >= 0x7f800000u ? 0 : wgbm_shift_from_absmax(__uint_as_float(m), qbits);
  }
}

// The feature map of a call with feature indices (one workgroup of 1024):
// every requested column f in [0, n_master) gets the list of its outputs
// (mark[f] = first, next[o] = following, -1 ends; indices outside the
// columns have no list and contribute nothing), and the columns that have
// one are numbered in ascending order: list[h] = column, head[h] = its
// first output, *count = how many.
__device__ void feature_map_body(const FeatMapArgs& fm) {
  __shared__ int64_t wsum[16];
  __shared__ int64_t sbuf[kScanK * 1024];
  for (int f = threadIdx.x; f < fm.n_master; f += blockDim.x) fm.mark[f] = -1;
  __syncthreads();
  for (int o = threadIdx.x; o < fm.n_out; o += blockDim.x) {
    const int f = fm.feat_idx[o];
    fm.next[o] = (f >= 0 && f < fm.n_master) ? atomicExch(&fm.mark[f], o) : -1;
  }
  __syncthreads();
  // the exchanged heads live in L2: read them with device-scope loads
  auto head_of = [&](int f) {
    return __hip_atomic_load(&fm.mark[f], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  };
  const int64_t tot = wgbm_block_scan_tiled(
      fm.n_master, [&](int f) -> int64_t { return head_of(f) >= 0 ? 1 : 0; },
      [&](int f, int64_t h) {
        const int m = head_of(f);
        if (m >= 0) {
          fm.list[h] = f;
          fm.head[h] = m;
        }
      },
      wsum, sbuf);
  // lane ownership per chunk: a run chunk needs every lane's selected
  // features to be V consecutive columns starting at a multiple of V (a
  // lane with none, past the end, does not matter)
  const int n_sel = (int)tot;
  for (int c = threadIdx.x; c < fm.n_chunks; c += blockDim.x) fm.run[c] = 1;
  __syncthreads();
  for (int g = threadIdx.x; g < fm.n_chunks * kHistSlots; g += blockDim.x) {
    const int h0 = g * fm.V;
    if (h0 >= n_sel) continue;
    auto col = [&](int h) {
      return __hip_atomic_load(&fm.list[h], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    const int c0 = col(h0);
    bool ok = c0 % fm.V == 0;
    for (int j = 1; j < fm.V && h0 + j < n_sel; ++j) ok = ok && col(h0 + j) == c0 + j;
    if (!ok) fm.run[g / kHistSlots] = 0;
  }
  if (threadIdx.x == 0) *fm.count = n_sel;
}

// One launch for a call's preparation: blocks [0, n_part) write the per-block
// maxima of |residual| (and, with rows, the residuals in position order);
// then, with plan != 0, one block plans the tiles and, with a feature map,
// one block builds it.  The tile kernel turns the maxima into the shift.
__global__ __launch_bounds__(1024) void hist_prep_kernel(
    const float* __restrict__ resid, const int32_t* __restrict__ rows, int64_t n,
    uint32_t* __restrict__ partial, float* __restrict__ gathered, int32_t n_part, int32_t plan,
    const int64_t* __restrict__ seg, int32_t n_keys, int32_t tile_rows, int32_t max_tiles,
    Tile* __restrict__ tiles, int32_t* __restrict__ key_tile_start,
    int32_t* __restrict__ n_tiles, FeatMapArgs fm, uint32_t* __restrict__ key_max) {
  if ((int)blockIdx.x >= n_part) {
    if (plan && (int)blockIdx.x == n_part)
      plan_tiles_body(seg, n, n_keys, nullptr, tile_rows, 1, max_tiles, tiles, key_tile_start,
                      n_tiles);
    else if (fm.feat_idx)
      feature_map_body(fm);
    return;
  }
  if (key_max) {
    // the per-key maxima of hist_key_max_kernel start from zero
    for (int k = blockIdx.x * blockDim.x + threadIdx.x; k < n_keys; k += n_part * blockDim.x)
      key_max[k] = 0u;
  }
  uint32_t m = 0;
  // U positions per thread and round, the row loads, then the residual
  // loads, issued together (a position past the end re-reads the last one
  // and stores nothing)
  constexpr int U = 4;
  const int64_t stride = (int64_t)n_part * blockDim.x;
  for (int64_t i0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i0 < n; i0 += U * stride) {
    int64_t r[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + u * stride;
      r[u] = i < n ? i : n - 1;
    }
    if (rows) {
#pragma unroll
      for (int u = 0; u < U; ++u) r[u] = (int64_t)rows[r[u]];
    }
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = resid[r[u]];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t i = i0 + u * stride;
      if (gathered && i < n) gathered[i] = v[u];
      const uint32_t b = wgbm_abs_bits(v[u]);
      m = b > m ? b : m;
    }
  }
  m = wgbm_block_max_u32(m);
  if (threadIdx.x == 0) partial[blockIdx.x] = m;
}

__global__ __launch_bounds__(256) void hist_key_max_kernel(
    const Tile* __restrict__ tiles, const int32_t* __restrict__ n_tiles,
    const float* __restrict__ resid, const int32_t* __restrict__ order, int32_t by_pos,
    uint32_t* __restrict__ key_max) {
  if ((int)blockIdx.x >= *n_tiles) return;  // uniform per workgroup
  const Tile tl = tiles[blockIdx.x];
  uint32_t m = 0;
  if (tl.end > tl.begin) {
    // U positions per thread and round, their loads issued together (a
    // position past the tile re-reads the tile's last one: no branch, and
    // the maximum is unchanged)
    constexpr int U = 8;
    const int64_t last = tl.end - 1;
    for (int64_t p0 = tl.begin + threadIdx.x; p0 < tl.end; p0 += (int64_t)U * blockDim.x) {
      int64_t r[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int64_t p = p0 + (int64_t)u * blockDim.x;
        r[u] = p < tl.end ? p : last;
      }
      if (!(by_pos || !order)) {
#pragma unroll
        for (int u = 0; u < U; ++u) r[u] = (int64_t)order[r[u]];
      }
      uint32_t b[U];
#pragma unroll
      for (int u = 0; u < U; ++u) b[u] = wgbm_abs_bits(resid[r[u]]);
#pragma unroll
      for (int u = 0; u < U; ++u) m = b[u] > m ? b[u] : m;
    }
  }
  m = wgbm_block_max_u32(m);
  if (threadIdx.x == 0 && m) atomicMax(key_max + tl.key, m);
}

__global__ __launch_bounds__(1024) void plan_tiles_kernel(
    const int64_t* __restrict__ seg, int64_t total_rows, int32_t n_keys,
    const int32_t* __restrict__ key_list, int32_t tile_rows, int32_t nearest,
    int32_t max_tiles, Tile* __restrict__ tiles, int32_t* __restrict__ key_tile_start,
    int32_t* __restrict__ n_tiles) {
  plan_tiles_body(seg, total_rows, n_keys, key_list, tile_rows, nearest, max_tiles, tiles,
                  key_tile_start, n_tiles);
}


// --------------------------------------------------------------------------
// era regrouping for the ABI path: row list -> era-grouped positions.
// Positions are split into nb contiguous blocks of per_block; block b counts
// its rows per era in LDS (kEraWindow eras per pass), the counts [era][block]
// are scanned per era (offsets inside the era) and across eras (era starts),
// and block b scatters its rows from LDS cursors at start[e] + offset[e][b].
// Rows with an era outside [0, num_eras) are dropped.  The order of rows
// inside an era follows LDS atomics (the histogram sums are exact integers,
// so it does not change a result).
// --------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void era_block_count_kernel(
    const int32_t* __restrict__ rows, int64_t n, const int32_t* __restrict__ era,
    int32_t num_eras, int64_t per_block, int32_t* __restrict__ counts) {
  __shared__ uint32_t c[kEraWindow];
  const int nb = gridDim.x;
  const int64_t p0 = (int64_t)blockIdx.x * per_block;
  const int64_t p1 = p0 + per_block < n ? p0 + per_block : n;
  for (int w0 = 0; w0 < num_eras; w0 += kEraWindow) {
    const int wn = num_eras - w0 < kEraWindow ? num_eras - w0 : kEraWindow;
    for (int i = threadIdx.x; i < wn; i += blockDim.x) c[i] = 0u;
    __syncthreads();
    for (int64_t p = p0 + threadIdx.x; p < p1; p += blockDim.x) {
      const int e = era[rows ? rows[p] : (int32_t)p] - w0;
      if ((unsigned)e < (unsigned)wn) atomicAdd(&c[e], 1u);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < wn; i += blockDim.x)
      counts[(int64_t)(w0 + i) * nb + blockIdx.x] = (int32_t)c[i];
    __syncthreads();
  }
}

// one wave per era: counts[e][0..nb) -> exclusive offsets in place, era_tot[e]
// = the era's rows
__global__ __launch_bounds__(1024) void era_row_scan_kernel(int32_t* __restrict__ counts,
                                                            int32_t num_eras, int32_t nb,
                                                            int64_t* __restrict__ era_tot) {
  const int e = (int)blockIdx.x * 16 + (int)(threadIdx.x >> 6);
  if (e >= num_eras) return;
  const int lane = threadIdx.x & 63;
  int32_t* row = counts + (int64_t)e * nb;
  int64_t carry = 0;
  for (int b0 = 0; b0 < nb; b0 += 64) {
    const int b = b0 + lane;
    const int64_t v = b < nb ? row[b] : 0;
    const int64_t inc = wgbm_wave_incl_scan_i64(v);
    if (b < nb) row[b] = (int32_t)(carry + inc - v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(uint64_t)inc, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)((uint64_t)inc >> 32), 63);
    carry += (int64_t)(((uint64_t)hi << 32) | lo);
  }
  if (lane == 0) era_tot[e] = carry;
}

// one workgroup: era_tot[0..E) -> exclusive era starts in place, era_tot[E] =
// the total (the segment bounds of the regrouped positions)
__global__ __launch_bounds__(1024) void era_start_scan_kernel(int64_t* __restrict__ era_tot,
                                                              int32_t num_eras) {
  __shared__ int64_t wsum[16];
  __shared__ int64_t sbuf[kScanK * 1024];
  const int64_t tot = wgbm_block_scan_tiled(
      num_eras, [&](int i) -> int64_t { return era_tot[i]; },
      [&](int i, int64_t v) { era_tot[i] = v; }, wsum, sbuf);
  if (threadIdx.x == 0) era_tot[num_eras] = tot;
}

__global__ __launch_bounds__(1024) void era_block_scatter_kernel(
    const int32_t* __restrict__ rows, int64_t n, const int32_t* __restrict__ era,
    int32_t num_eras, int64_t per_block, const int32_t* __restrict__ offs,
    const int64_t* __restrict__ seg, int32_t* __restrict__ out) {
  __shared__ uint32_t cur[kEraWindow];
  const int nb = gridDim.x;
  const int64_t p0 = (int64_t)blockIdx.x * per_block;
  const int64_t p1 = p0 + per_block < n ? p0 + per_block : n;
  for (int w0 = 0; w0 < num_eras; w0 += kEraWindow) {
    const int wn = num_eras - w0 < kEraWindow ? num_eras - w0 : kEraWindow;
    // positions < 2^31: 32-bit cursors
    for (int i = threadIdx.x; i < wn; i += blockDim.x)
      cur[i] = (uint32_t)(seg[w0 + i] + offs[(int64_t)(w0 + i) * nb + blockIdx.x]);
    __syncthreads();
    for (int64_t p = p0 + threadIdx.x; p < p1; p += blockDim.x) {
      const int32_t r = rows ? rows[p] : (int32_t)p;
      const int e = era[r] - w0;
      if ((unsigned)e < (unsigned)wn) out[atomicAdd(&cur[e], 1u)] = r;
    }
    __syncthreads();
  }
}

// --------------------------------------------------------------------------
__global__ void era_count_kernel(const int32_t* __restrict__ rows, int64_t n,
                                 const int32_t* __restrict__ era, int32_t num_eras,
                                 int64_t* __restrict__ counts) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int e = era[rows ? rows[i] : i];
    if (e >= 0 && e < num_eras) atomicAdd((unsigned long long*)&counts[e], 1ull);
  }
}

__global__ void exclusive_scan_i64_kernel(const int64_t* __restrict__ in, int32_t n,
                                          int64_t* __restrict__ out) {
  // single thread; n is the number of eras (small)
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    int64_t acc = 0;
    for (int i = 0; i < n; ++i) {
      out[i] = acc;
      acc += in[i];
    }
    out[n] = acc;
  }
}

__global__ void era_scatter_kernel(const int32_t* __restrict__ rows, int64_t n,
                                   const int32_t* __restrict__ era, int32_t num_eras,
                                   unsigned long long* __restrict__ cursor,
                                   int32_t* __restrict__ out) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int32_t r = rows ? rows[i] : (int32_t)i;
    const int e = era[r];
    if (e >= 0 && e < num_eras) out[atomicAdd(&cursor[e], 1ull)] = r;
  }
}

// --------------------------------------------------------------------------
// instrumentation: the LDS atomic rate of the tile histogram's layout alone.
// Same LDS words as hist_tiles_kernel<4, *, 32> (4 features per lane, 33 bins,
// 64 lane-owned columns) and the same packed 64-bit adds; every lane cycles
// through 16 precomputed (feature, bin) words, so the loop is the atomics
// alone (no global traffic, no address arithmetic).
// --------------------------------------------------------------------------
__global__ __launch_bounds__(kHistThreads) void lds_atomic_probe_kernel(
    int32_t iters, unsigned long long* __restrict__ sink) {
  extern __shared__ unsigned long long lds[];
  constexpr int V = 4, Bp = 33;
  for (int i = threadIdx.x; i < V * Bp * kHistSlots; i += kHistThreads) lds[i] = 0ull;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  uint32_t h = threadIdx.x * 2654435761u + blockIdx.x * 97u + 1u;
  unsigned long long* addr[16];
#pragma unroll
  for (int k = 0; k < 16; ++k) {
    h ^= h << 13;
    h ^= h >> 17;
    h ^= h << 5;
    addr[k] = lds + lane + ((k & 3) * Bp + (int)(h & 31u)) * kHistSlots;
  }
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 16; ++k) atomicAdd(addr[k], (unsigned long long)(2 * it + 1));
  }
  __syncthreads();
  // keep the result observable
  if (threadIdx.x < 64) sink[blockIdx.x * 64 + threadIdx.x] = lds[threadIdx.x];
}

int probe_lds_atomics(int32_t blocks, int32_t iters, double* ops_per_s, hipStream_t st) {
  const size_t lds = (size_t)4 * 33 * kHistSlots * 8;
  WGBM_CHECK(hipFuncSetAttribute((const void*)lds_atomic_probe_kernel,
                                 hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
  unsigned long long* sink = (unsigned long long*)scratch_get(st, sizeof(unsigned long long) * 64 * (size_t)blocks, 9);
  WGBM_REQUIRE(sink, "scratch allocation failed");
  hipEvent_t a, b;
  WGBM_CHECK(hipEventCreate(&a));
  WGBM_CHECK(hipEventCreate(&b));
  // one untimed launch, then the timed one
  hipLaunchKernelGGL(lds_atomic_probe_kernel, dim3(blocks), dim3(kHistThreads), lds, st, iters, sink);
  WGBM_LAUNCH_CHECK();
  WGBM_CHECK(hipEventRecord(a, st));
  hipLaunchKernelGGL(lds_atomic_probe_kernel, dim3(blocks), dim3(kHistThreads), lds, st, iters, sink);
  WGBM_LAUNCH_CHECK();
  WGBM_CHECK(hipEventRecord(b, st));
  WGBM_CHECK(hipEventSynchronize(b));
  float ms = 0.0f;
  WGBM_CHECK(hipEventElapsedTime(&ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  *ops_per_s = (double)blocks * kHistThreads * iters * 16 / (ms * 1e-3);
  return 0;
}

// --------------------------------------------------------------------------
// instrumentation: the achievable HBM read rate.  Each workgroup streams
// one contiguous 1/kProbeBlocks of a caller's buffer with 16-byte
// non-temporal loads (like the histogram's code loads), four in flight per
// lane, and folds them into one word per lane, stored to a per-workgroup
// sink so the loads stay live.  The buffer is read whole once per launch;
// nothing else touches memory.  Contiguous per-workgroup ranges beat a
// grid-stride walk of the same loads on this GPU (7.0 against 5.8 TB/s on
// 1 GB; probes of 1024-16384 workgroups and 4 or 8 loads per lane).
// --------------------------------------------------------------------------
typedef uint32_t wgbm_u32x4 __attribute__((ext_vector_type(4)));
constexpr int kProbeBlocks = 1024;  // four workgroups of 256 lanes per CU
__global__ __launch_bounds__(256) void hbm_read_probe_kernel(const wgbm_u32x4* __restrict__ src,
                                                             int64_t n16,
                                                             uint32_t* __restrict__ sink) {
  const int64_t per = (n16 + gridDim.x - 1) / gridDim.x;
  const int64_t b0 = (int64_t)blockIdx.x * per;
  const int64_t b1 = b0 + per < n16 ? b0 + per : n16;
  uint32_t acc = 0;
  int64_t i = b0 + threadIdx.x;
  for (; i + 3 * 256 < b1; i += 4 * 256) {
    wgbm_u32x4 v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = __builtin_nontemporal_load(src + i + k * 256);
#pragma unroll
    for (int k = 0; k < 4; ++k) acc ^= v[k].x ^ v[k].y ^ v[k].z ^ v[k].w;
  }
  for (; i < b1; i += 256) {
    const wgbm_u32x4 v = __builtin_nontemporal_load(src + i);
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  sink[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

int probe_hbm_read(const void* buf, int64_t bytes, int32_t iters, double* bytes_per_s,
                   hipStream_t st) {
  const int64_t n16 = bytes / 16;
  constexpr int kBlocks = kProbeBlocks;
  uint32_t* sink = (uint32_t*)scratch_get(st, sizeof(uint32_t) * kBlocks * 256, 9);
  WGBM_REQUIRE(sink, "scratch allocation failed");
  hipEvent_t a, b;
  WGBM_CHECK(hipEventCreate(&a));
  WGBM_CHECK(hipEventCreate(&b));
  // one untimed launch, then `iters` timed ones back to back
  hipLaunchKernelGGL(hbm_read_probe_kernel, dim3(kBlocks), dim3(256), 0, st,
                     (const wgbm_u32x4*)buf, n16, sink);
  WGBM_LAUNCH_CHECK();
  WGBM_CHECK(hipEventRecord(a, st));
  for (int it = 0; it < iters; ++it) {
    hipLaunchKernelGGL(hbm_read_probe_kernel, dim3(kBlocks), dim3(256), 0, st,
                       (const wgbm_u32x4*)buf, n16, sink);
    WGBM_LAUNCH_CHECK();
  }
  WGBM_CHECK(hipEventRecord(b, st));
  WGBM_CHECK(hipEventSynchronize(b));
  float ms = 0.0f;
  WGBM_CHECK(hipEventElapsedTime(&ms, a, b));
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  *bytes_per_s = (double)n16 * 16.0 * iters / (ms * 1e-3);
  return 0;
}

// --------------------------------------------------------------------------
// finalize launchers: words per workgroup from the expected tiles per segment
// --------------------------------------------------------------------------
int fin_words_for(int64_t tiles_per_key) {
  if (tiles_per_key >= 32) return 32;   // 8-way tile split
  if (tiles_per_key >= 16) return 64;   // 4-way
  if (tiles_per_key >= 8) return 128;   // 2-way
  return 256;                           // one group walks all tiles
}

#define WGBM_FIN_DISPATCH(FWV, LAUNCH) \
  switch (FWV) {                       \
    case 32: LAUNCH(32); break;        \
    case 64: LAUNCH(64); break;        \
    case 128: LAUNCH(128); break;      \
    default: LAUNCH(256); break;       \
  }

// plane finalize for many segments with few tiles each (coalesced output rows);
// the word-per-thread kernels otherwise (few segments: their tile split keeps
// enough loads in flight)
static bool use_plane_finalize(int64_t tiles_per_key, int64_t n_keys, int n_chunks, int V,
                               int num_bins) {
  return num_bins <= kPlaneMaxBins && tiles_per_key <= 64 && n_keys * n_chunks * V >= 128;
}

int launch_finalize_f32(int64_t tiles_per_key, const unsigned long long* part,
                        const int32_t* key_tile_start, int32_t n_keys, int32_t n_chunks, int32_t V,
                        int32_t num_bins, int32_t n_feats, const uint32_t* absmax_bits,
                        int32_t key_stride, int32_t qbits, const int32_t* n_tiles,
                        int32_t accumulate, FeatOut fo, float* G, float* H, hipStream_t st) {
  if (use_plane_finalize(tiles_per_key, n_keys, n_chunks, V, num_bins)) {
    const int64_t wg = (int64_t)n_keys * n_chunks * V;
    WGBM_REQUIRE(wg < ((int64_t)1 << 31), "finalize: too many segments");
    hipLaunchKernelGGL(hist_finalize_plane_f32_kernel, dim3((unsigned)wg), dim3(kPlaneThreads), 0,
                       st, part, key_tile_start, n_keys, n_chunks, V, num_bins, n_feats,
                       absmax_bits, key_stride, qbits, n_tiles, accumulate, fo, G, H);
    WGBM_LAUNCH_CHECK();
    return 0;
  }
  const int fw = fin_words_for(tiles_per_key);
  const int64_t tile_words = (int64_t)n_chunks * kHistSlots * V * num_bins;
  WGBM_REQUIRE(tile_words < ((int64_t)1 << 31) &&
                   n_keys * ((tile_words + fw - 1) / fw) < ((int64_t)1 << 31),
               "finalize: too many histogram words");
  const unsigned wg = (unsigned)(n_keys * ((tile_words + fw - 1) / fw));
#define WGBM_L(F)                                                                                 \
  hipLaunchKernelGGL(hist_finalize_f32_kernel<F>, dim3(wg), dim3(256), 0, st, part, key_tile_start, \
                     n_keys, n_chunks, V, num_bins, n_feats, absmax_bits, key_stride, qbits,        \
                     n_tiles, accumulate, fo, G, H)
  WGBM_FIN_DISPATCH(fw, WGBM_L)
#undef WGBM_L
  WGBM_LAUNCH_CHECK();
  return 0;
}

int launch_finalize_level(int64_t tiles_per_key, const unsigned long long* part,
                          const int32_t* key_tile_start, const int32_t* key_list, int32_t n_list,
                          int32_t n_chunks, int32_t V, int32_t num_bins, int32_t n_feats,
                          int32_t num_eras, int32_t nodes_in_level, int32_t depth,
                          const int64_t* parent_q, const int32_t* parent_c, const int32_t* n_tiles,
                          int64_t* hq, int32_t* hc, hipStream_t st) {
  if (use_plane_finalize(tiles_per_key, n_list, n_chunks, V, num_bins)) {
    const int64_t wg = (int64_t)n_list * n_chunks * V;
    WGBM_REQUIRE(wg < ((int64_t)1 << 31), "finalize: too many segments");
    // up to 32 bins: 512 threads in two tile groups (a level's keys have few
    // tiles each; C5: 13.3 us per call against 14.6 with 1024 threads and 15.8
    // with one group)
    if (num_bins <= 32)
      hipLaunchKernelGGL((hist_finalize_plane_level_kernel<32, 512, 2>), dim3((unsigned)wg),
                         dim3(512), 0, st, part, key_tile_start, key_list, n_list, n_chunks, V,
                         num_bins, n_feats, num_eras, nodes_in_level, depth, parent_q, parent_c,
                         n_tiles, hq, hc);
    else
      hipLaunchKernelGGL((hist_finalize_plane_level_kernel<kPlaneMaxBins, kPlaneThreads,
                                                           kPlaneGroups>),
                         dim3((unsigned)wg), dim3(kPlaneThreads), 0, st, part, key_tile_start,
                         key_list, n_list, n_chunks, V, num_bins, n_feats, num_eras,
                         nodes_in_level, depth, parent_q, parent_c, n_tiles, hq, hc);
    WGBM_LAUNCH_CHECK();
    return 0;
  }
  const int fw = fin_words_for(tiles_per_key);
  const int64_t tile_words = (int64_t)n_chunks * kHistSlots * V * num_bins;
  WGBM_REQUIRE(tile_words < ((int64_t)1 << 31) &&
                   n_list * ((tile_words + fw - 1) / fw) < ((int64_t)1 << 31),
               "finalize: too many histogram words");
  const unsigned wg = (unsigned)(n_list * ((tile_words + fw - 1) / fw));
#define WGBM_L(F)                                                                          \
  hipLaunchKernelGGL(hist_finalize_level_kernel<F>, dim3(wg), dim3(256), 0, st, part,        \
                     key_tile_start, key_list, n_list, n_chunks, V, num_bins, n_feats, num_eras, \
                     nodes_in_level, depth, parent_q, parent_c, n_tiles, hq, hc)
  WGBM_FIN_DISPATCH(fw, WGBM_L)
#undef WGBM_L
  WGBM_LAUNCH_CHECK();
  return 0;
}
#undef WGBM_FIN_DISPATCH

// --------------------------------------------------------------------------
// host launch helpers
// --------------------------------------------------------------------------
// features per lane: the largest V in {4, 2, 1} whose LDS histogram
// V*(B+1)*64 words stays within 68 KiB, so that two workgroups fit a CU
int hist_pick_v(int num_bins, int64_t n_feats) {
  const int bp = num_bins + 1;
  int v = 4 * bp <= 136 ? 4 : (2 * bp <= 136 ? 2 : 1);  // num_bins <= 33 / <= 67 / beyond
  // a narrower lane (fewer features per lane) as long as the chunk count
  // stays the same: each row still costs the same load instructions, and
  // the atomics of lanes past the last feature (every lane adds, for a
  // branch-free loop) shrink, e.g. 100 features: 4 -> 2 LDS atomics per row
  auto chunks = [&](int w) { return (n_feats + kHistSlots * w - 1) / (kHistSlots * w); };
  while (v > 1 && chunks(v / 2) == chunks(v)) v /= 2;
  return v;
}

size_t hist_lds_bytes(int V, int num_bins, bool native) {
  if (native) return (size_t)V * 2 * (num_bins + 2) * 256;
  return (size_t)V * (num_bins + 1) * kHistSlots * 8;
}

// the native-code layout needs c + H <= 255 for every byte c <= B + 1
bool hist_native_ok(int num_bins) { return 2 * num_bins + 3 <= 255; }

template <int V, int MODE, int BT, bool GATHER, bool NAT, bool RPOS, bool FS = false>
static int launch_tiles_t(const HistLaunch& a, hipStream_t st) {
  static bool attr_set = false;
  const size_t lds = hist_lds_bytes(V, a.num_bins, NAT);
  if (!attr_set) {
    WGBM_CHECK(hipFuncSetAttribute(
        (const void*)hist_tiles_kernel<V, MODE, BT, GATHER, NAT, RPOS, FS>,
        hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024));
    attr_set = true;
  }
  // raw codes: a multiple of 8 workgroups, so that every XCD's share of the
  // work is covered
  const int64_t n_wg = (int64_t)a.n_chunks * a.max_tiles;
  dim3 grid((unsigned)(NAT ? n_wg : wgbm_xcd_grid(n_wg)));
  void* tm = timer_begin(a.timer_tag);
  const bool marks = tm && timer_mode() == 1;
  if (marks) WGBM_CHECK(hipEventRecord(timer_start_event(tm), st));
  hipExtLaunchKernelGGL((hist_tiles_kernel<V, MODE, BT, GATHER, NAT, RPOS, FS>), grid,
                        dim3(kHistThreads), lds, st, marks ? nullptr : timer_start_event(tm),
                        marks ? nullptr : timer_stop_event(tm), 0, a.codes, a.n_rows, a.stride,
                        a.n_feats, a.resid, a.resid_tree_stride, a.shifts, a.order, a.tiles,
                        a.n_tiles, a.keys_per_tree, a.num_bins, a.part, a.sm, a.fs);
  if (marks) WGBM_CHECK(hipEventRecord(timer_stop_event(tm), st));
  timer_end(tm);
  WGBM_LAUNCH_CHECK();
  return 0;
}

template <int V, int MODE, int BT, bool NAT>
static int launch_tiles_r(const HistLaunch& a, hipStream_t st) {
  if (!a.order) return launch_tiles_t<V, MODE, BT, false, NAT, false>(a, st);
  if constexpr (!NAT) {
    if (a.fs.list)
      return a.resid_by_pos ? launch_tiles_t<V, MODE, BT, true, false, true, true>(a, st)
                            : launch_tiles_t<V, MODE, BT, true, false, false, true>(a, st);
  }
  return a.resid_by_pos ? launch_tiles_t<V, MODE, BT, true, NAT, true>(a, st)
                        : launch_tiles_t<V, MODE, BT, true, NAT, false>(a, st);
}

template <int V, int MODE, int BT>
static int launch_tiles_g(const HistLaunch& a, hipStream_t st) {
  if (a.native && hist_native_ok(a.num_bins)) return launch_tiles_r<V, MODE, BT, true>(a, st);
  return launch_tiles_r<V, MODE, BT, false>(a, st);
}

int hist_load_mode(int64_t n_rows, int64_t stride, int V) {
  if (n_rows * stride < ((int64_t)1 << 31) && stride % 4 == 0) return kLoadBuffer;
  if (stride % V == 0) return kLoadGlobalAligned;
  return kLoadBytes;
}

int launch_hist_tiles(const HistLaunch& a, hipStream_t st) {
  WGBM_REQUIRE(a.n_rows < ((int64_t)1 << 31), "histogram: at most 2^31 - 1 rows");
  WGBM_REQUIRE(!a.fs.list || (a.order && a.fs.count && a.fs.run && !a.native &&
                                a.fs.n_master <= a.stride),
               "histogram: feature selection needs a row list and raw codes");
  const int mode = hist_load_mode(a.n_rows, a.stride, a.V);
  if (a.V == 4 && a.num_bins == 32) {
    if (mode == kLoadBuffer) return launch_tiles_g<4, kLoadBuffer, 32>(a, st);
    if (mode == kLoadGlobalAligned) return launch_tiles_g<4, kLoadGlobalAligned, 32>(a, st);
  }
  if (a.V == 2 && a.num_bins == 32) {
    if (mode == kLoadBuffer) return launch_tiles_g<2, kLoadBuffer, 32>(a, st);
    if (mode == kLoadGlobalAligned) return launch_tiles_g<2, kLoadGlobalAligned, 32>(a, st);
  }
#define WGBM_DISPATCH(VV)                                                      \
  if (a.V == VV) {                                                             \
    if (mode == kLoadBuffer) return launch_tiles_g<VV, kLoadBuffer, 0>(a, st); \
    if (mode == kLoadGlobalAligned)                                            \
      return launch_tiles_g<VV, kLoadGlobalAligned, 0>(a, st);                 \
    return launch_tiles_g<VV, kLoadBytes, 0>(a, st);                           \
  }
  WGBM_DISPATCH(4)
  WGBM_DISPATCH(2)
  WGBM_DISPATCH(1)
#undef WGBM_DISPATCH
  wgbm_set_error("launch_hist_tiles: bad V=%d", a.V);
  return WGBM_EINVAL;
}

}  // namespace wgbm
