// CSC transpose of the gate's per-query block ids into per-block columns.
//
// Restates src/moba/kernels/routing.py:139-301 (count / offsets+order /
// scatter) and routing.py:309-427 (launcher): counts per (row, kv head,
// block), an exclusive scan into col_offsets, a longest-first column order
// (count desc, id asc; the stable argsort of routing.py:548-553), and a
// scatter of (row, query head, slot) triples. Under GQA every query head of
// a group lands in its kv head's columns. The scatter places a column's
// entries in (query head, row) order on every build. It works on windows of
// up to kDetMaxCols (16384) columns, the (cursor, mask) pairs of one window
// filling 128 KiB of LDS: past that many columns the windows run one after
// another, each reading every id again. Only a device that cannot give a
// workgroup that much LDS falls back to per-entry atomic cursors, whose
// order within a column varies from run to run, as the reference's does.
//
// The order pass ranks each column directly -- rank = #columns with a larger
// count, or the same count and a smaller id -- one lane per column against an
// LDS copy of the counts (order_kernel): O(nb^2) work spread over nb lanes,
// ~16M integer compares per head at nb = 4096 (27 us for four heads). From
// 4097 to 16384 columns it sorts (count desc, id asc) keys per (row, kv head)
// in LDS with a bitonic network instead (order_sort_kernel, O(nb log^2 nb)).
#include <mutex>

#include "common.h"


namespace moba {

__global__ void __launch_bounds__(256)
fill_i32_kernel(int32_t* __restrict__ p, int64_t n, int32_t value) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = value;
}

// One lane per (query, slot) entry; grid.y = row * Hq + hq.
template <bool kScatter>
__global__ void __launch_bounds__(256)
count_or_scatter_kernel(const int32_t* __restrict__ block_idx, const int32_t* __restrict__ cu,
                        int64_t S, int64_t rows_per_seq, int64_t h_q, int64_t h_kv,
                        int64_t n_blocks, int slots, int64_t cap,
                        int32_t* __restrict__ col_nnz_or_cursor,
                        const int32_t* __restrict__ col_offsets,
                        int32_t* __restrict__ row_indices, int32_t* __restrict__ head_indices,
                        int32_t* __restrict__ slot_of_pair, int64_t istride) {
  const int64_t rh = blockIdx.y;
  const int64_t r = rh / h_q;
  const int64_t hq = rh % h_q;
  const int64_t hk = hq / (h_q / h_kv);
  const bool packed = cu != nullptr;
  const SeqSpan sp = seq_span(cu, r, S);
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t t = e / slots;
  const int j = static_cast<int>(e % slots);
  if (t >= sp.len) return;
  const int64_t tok = sp.bos + t;
  const int64_t qid = packed ? hq * S + tok : (r * h_q + hq) * S + t;
  const int32_t blk = block_idx[qid * slots + j];
  if (blk < 0 || blk >= n_blocks) return;  // padding, or an id no query can hold
  const int64_t colbase = (r * h_kv + hk) * n_blocks;
  const int32_t within = atomicAdd(&col_nnz_or_cursor[colbase + blk], 1);
  if (kScatter) {
    const int64_t dst = ((r * h_kv + hk) * cap +
                         col_offsets[(r * h_kv + hk) * (n_blocks + 1) + blk] + within) * istride;
    row_indices[dst] = static_cast<int32_t>(packed ? tok : t);
    head_indices[dst] = static_cast<int32_t>(hq);
    slot_of_pair[dst] = j;
  }
}

// Tiled count: tq queries of one (row, query head) per workgroup (a tile,
// tq 256 or kTileQ), kTileT threads each taking up to
// kTileQ / kTileT of them, counted in an LDS histogram over the blocks the
// tile can see and written out as one row of the unit count table (below).
// The LDS histogram keeps the global memory traffic at one row per tile:
// the own block, which every query of a block selects, would otherwise take
// 128 serialised global atomics.
constexpr int kTileQ = 1024;
typedef int32_t i32x3 __attribute__((ext_vector_type(3), aligned(4)));
constexpr int kTileT = 256;

// Queries per tile (a *unit* of the deterministic build is one tile of one
// query head): 1024, or 256 when 1024-query tiles would give fewer than 512
// units. The scatter walks a unit's entries in one serial chain, so a build
// with few units waits on that chain (256 units at [1,64K,4,64]); with more
// units, smaller tiles cost more in count-table traffic (units x columns)
// than they save (measured: 64K 0.088 -> 0.072 ms, 128K no gain).
inline int64_t tile_queries(int64_t batch, int64_t h_q, int64_t rows_per_seq) {
  const int64_t units = batch * h_q * ((rows_per_seq + kTileQ - 1) / kTileQ);
  return units < 512 ? 256 : kTileQ;
}
constexpr int kMaxBins = 16384;

// Columns of the window [lo, lo + width) that queries seeing `nv` blocks can
// hold: [lo, lo + result).
__device__ inline int window_visible(int64_t nv, int64_t n_blocks, int64_t lo, int64_t width) {
  const int64_t hi = nv < n_blocks ? nv : n_blocks;
  const int64_t n = hi - lo;
  return static_cast<int>(n < 0 ? 0 : (n > width ? width : n));
}

// atomicAdd(&bins[blk], 1) for every active lane, with the lanes that share
// the first active lane's id served by one atomic (every query of a block
// selects its own block, so a wave's 64 consecutive queries usually agree
// there).
__device__ inline void bin_add(int32_t* bins, int32_t blk, bool active) {
  const uint64_t act = __ballot(active);
  if (act == 0) return;
  const int lead = __builtin_ctzll(act);
  const int32_t b0 = __shfl(blk, lead);
  const bool same = active && blk == b0;
  const uint64_t m = __ballot(same);
  const int lane = threadIdx.x & 63;
  if (lane == lead) atomicAdd(&bins[b0], __popcll(m));
  if (active && !same) atomicAdd(&bins[blk], 1);
}

// table row (rh * tiles + tile) = the tile's count of every column of the
// window [lo, lo + width), zeros where it sees none; grid (tiles, R * Hq).
__global__ void __launch_bounds__(kTileT)
tile_count_kernel(const int32_t* __restrict__ block_idx, const int32_t* __restrict__ cu,
                  int64_t S, int64_t h_q, int64_t n_blocks, int64_t bs, int slots, int tq,
                  int32_t* __restrict__ table, int64_t lo, int64_t width) {
  extern __shared__ int32_t bins[];  // width counters (dynamic LDS)
  const int64_t rh = blockIdx.y;
  const int64_t r = rh / h_q;
  const int64_t hq = rh % h_q;
  const bool packed = cu != nullptr;
  const SeqSpan sp = seq_span(cu, r, S);
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * tq;
  int32_t* trow = table + (rh * gridDim.x + blockIdx.x) * width;
  if (t0 >= sp.len) {
    for (int64_t b = threadIdx.x; b < width; b += kTileT) trow[b] = 0;
    return;
  }
  const int64_t t_end = t0 + tq < sp.len ? t0 + tq : sp.len;  // this tile's queries: [t0, t_end)
  const int nvis = window_visible((t_end - 1) / bs + 1, n_blocks, lo, width);
  for (int b = threadIdx.x; b < nvis; b += kTileT) bins[b] = 0;
  __syncthreads();
  // Query i of this thread: t0 + threadIdx.x + kTileT * i (a wave's lanes
  // hold consecutive queries).
  constexpr int QPT = kTileQ / kTileT;
  if (slots == 8) {
    // Every id of the thread's queries requested up front (two 16-byte
    // loads per query), then counted.
    int4 ids[QPT][2];
#pragma unroll
    for (int i = 0; i < QPT; ++i) {
      const int64_t t = t0 + threadIdx.x + kTileT * i;
      const int64_t qid = packed ? hq * S + sp.bos + t : (r * h_q + hq) * S + t;
      const bool in = t < t_end;
      const int4* p = reinterpret_cast<const int4*>(block_idx + (in ? qid : 0) * 8);
      ids[i][0] = in ? p[0] : int4{-1, -1, -1, -1};
      ids[i][1] = in ? p[1] : int4{-1, -1, -1, -1};
    }
#pragma unroll
    for (int i = 0; i < QPT; ++i)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int32_t v[4] = {ids[i][h].x, ids[i][h].y, ids[i][h].z, ids[i][h].w};
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int32_t c = v[w] - static_cast<int32_t>(lo);
          bin_add(bins, c, c >= 0 && c < nvis);
        }
      }
  } else {
    for (int i = 0; i < QPT; ++i) {
      const int64_t t = t0 + threadIdx.x + kTileT * i;
      const int64_t qid = packed ? hq * S + sp.bos + t : (r * h_q + hq) * S + t;
      for (int j = 0; j < slots; ++j) {
        const int32_t c = t < t_end ? block_idx[qid * slots + j] - static_cast<int32_t>(lo) : -1;
        bin_add(bins, c, c >= 0 && c < nvis);
      }
    }
  }
  __syncthreads();
  for (int64_t b = threadIdx.x; b < width; b += kTileT) trow[b] = b < nvis ? bins[b] : 0;
}

// ---------------------------------------------------------------------------
// Deterministic column order. Entries of a column are placed by (query head
// within the group, query position), the order of the dense-mask CSC build
// (routing.py:467-561 builds from mask.nonzero(), which walks that order),
// so the index -- and with it the order in which the backward sums a
// column's dK / dV -- is the same on every build.
//
// A unit is one (row, query head, tile of tq queries); the units of one
// (row, kv head) in (query head, tile) order are exactly the column order.
// The count pass writes each unit's per-column counts to a table
// [R, Hq, tiles, nb]; a two-level exclusive scan over the units turns it
// into each unit's first position per column (chunks of units are summed,
// the chunk sums scanned, then each chunk rescanned from its base), and the
// scatter hands out positions inside a unit in entry order.

// Units of (row, kv head) rhk: (r * Hq + hk * G) * tiles + [0, G * tiles).
// kPhase 0: csum[rhk, c, b] = sum of the chunk's counts of column b.
// kPhase 1: table[u, b] = col_offsets[b] + csum[rhk, c, b] + exclusive sum
// of the chunk's earlier units (csum holding chunk bases by then).
template <int kPhase>
__global__ void __launch_bounds__(256)
unit_chunk_kernel(int32_t* __restrict__ table, int32_t* __restrict__ csum,
                  const int32_t* __restrict__ col_offsets, int64_t n_blocks, int64_t h_q,
                  int64_t h_kv, int64_t units, int64_t chunk, int64_t nchunks, int64_t lo,
                  int64_t width) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t c = blockIdx.y;
  const int64_t rhk = blockIdx.z;
  if (b >= width) return;
  const int64_t r = rhk / h_kv, hk = rhk % h_kv;
  const int64_t u0 = (r * h_q + hk * (h_q / h_kv)) * (units / (h_q / h_kv)) + c * chunk;
  const int64_t u1 = c * chunk + chunk < units ? u0 + chunk : u0 + (units - c * chunk);
  int32_t* cs = csum + (rhk * nchunks + c) * width + b;
  if (kPhase == 0) {
    int32_t acc = 0;
#pragma unroll 8
    for (int64_t u = u0; u < u1; ++u) acc += table[u * width + b];
    *cs = acc;
  } else {
    int32_t run = col_offsets[rhk * (n_blocks + 1) + lo + b] + *cs;
#pragma unroll 8
    for (int64_t u = u0; u < u1; ++u) {
      const int32_t v = table[u * width + b];
      table[u * width + b] = run;
      run += v;
    }
  }
}

// csum[rhk, :, b] -> exclusive scan over the chunks; the total is the
// column's count (written to col_nnz unless that is null).
__global__ void __launch_bounds__(256)
chunk_scan_kernel(int32_t* __restrict__ csum, int32_t* __restrict__ col_nnz, int64_t n_blocks,
                  int64_t nchunks, int64_t width) {
  const int64_t b = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t rhk = blockIdx.y;
  if (b >= width) return;
  int32_t run = 0;
#pragma unroll 8
  for (int64_t c = 0; c < nchunks; ++c) {
    int32_t* p = csum + (rhk * nchunks + c) * width + b;
    const int32_t v = *p;
    *p = run;
    run += v;
  }
  if (col_nnz) col_nnz[rhk * n_blocks + b] = run;
}

// One wave per unit. Its entries (query t, slot j) are contiguous in
// block_idx and are taken 64 at a time (a "row" of the unit, lane l holding
// entry 64 u + l). For each row, with i = t minus the row's first query
// (i < 32: a row spans at most 32 queries when slots >= 2; with one slot a
// row goes as two halves of 32):
//   1. every entry (query offset i, column c) ORs bit i into c's LDS mask --
//      an OR, so the result does not depend on the order of the lanes;
//   2. its position is c's cursor plus the number of mask bits below bit i
//      (the row's earlier queries holding c);
//   3. the row's lowest query holding c (the only one with no mask bit below
//      its own) advances c's cursor by the mask's popcount and clears the
//      mask.
// A query holds a column at most once, and a query split between two rows
// holds each column in only one of them, so this places every column's
// entries in query order, on every run.
// Ids are prefetched a stage of kPer rows ahead into registers: a wave's
// global stores share its load counter, so a load waited on between the
// stores would also wait for every store before it.
// Only columns of the window [lo, lo + width) are placed (the table holds
// that window). Dynamic LDS: (cursor, mask) pairs of the window's columns.
constexpr int kPer = 16;
// Columns the deterministic build handles (8 bytes of LDS each).
constexpr int kDetMaxCols = kMaxBins;
constexpr size_t kDetLdsBytes = 8 * static_cast<size_t>(kDetMaxCols);
__global__ void __launch_bounds__(64)
det_scatter_kernel(const int32_t* __restrict__ block_idx, const int32_t* __restrict__ cu,
                   int64_t S, int64_t h_q, int64_t h_kv, int64_t n_blocks, int64_t bs,
                   int slots, int64_t cap, const int32_t* __restrict__ table,
                   int32_t* __restrict__ row_indices, int32_t* __restrict__ head_indices,
                   int32_t* __restrict__ slot_of_pair, int64_t istride, bool records,
                   int tq, int64_t lo, int64_t width) {
  extern __shared__ uint32_t cm[];  // (cursor, mask) per column of the window
  const int64_t tile = blockIdx.x;
  const int64_t rh = blockIdx.y;
  const int64_t unit = rh * gridDim.x + tile;
  const int64_t r = rh / h_q;
  const int64_t hq = rh % h_q;
  const int64_t hk = hq / (h_q / h_kv);
  const bool packed = cu != nullptr;
  const SeqSpan sp = seq_span(cu, r, S);
  const int64_t t0 = tile * tq;
  if (t0 >= sp.len) return;
  const int64_t t1 = t0 + tq < sp.len ? t0 + tq : sp.len;
  const int nvis = window_visible((t1 - 1) / bs + 1, n_blocks, lo, width);
  if (nvis == 0) return;  // no column of the window is visible here
  const int32_t* trow = table + unit * width;
  const int lane = threadIdx.x;
  for (int b0 = 0; b0 < nvis; b0 += 16 * 64) {  // 16 loads in flight per lane
    int32_t v[16];
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int b = b0 + u * 64 + lane;
      v[u] = b < nvis ? trow[b] : 0;
    }
#pragma unroll
    for (int u = 0; u < 16; ++u) {
      const int b = b0 + u * 64 + lane;
      if (b < nvis) {
        cm[2 * b] = static_cast<uint32_t>(v[u]);
        cm[2 * b + 1] = 0u;
      }
    }
  }
  // block_idx row of query t0 of this (row, head); entries run to t1.
  const int64_t q0 = packed ? hq * S + sp.bos + t0 : (r * h_q + hq) * S + t0;
  const int32_t* src = block_idx + q0 * slots;
  const int32_t n_ent = static_cast<int32_t>((t1 - t0) * slots);
  const int64_t ibase = (r * h_kv + hk) * cap;
  const int32_t rbase = static_cast<int32_t>(packed ? sp.bos + t0 : t0);
  // Lane's entry of the current row: query q (from t0), slot j; stepped by
  // 64 entries per row without division.
  int32_t q = lane / slots, j = lane % slots;
  const int32_t dq = 64 / slots, dj = 64 % slots;
  const int halves = slots == 1 ? 2 : 1;
  int32_t cur[kPer], nxt[kPer];
  auto fetch = [&](int32_t* dst, int32_t s0) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int32_t e = s0 + u * 64 + lane;
      dst[u] = e < n_ent ? src[e] : -1;
    }
  };
  fetch(nxt, 0);
  for (int32_t s0 = 0; s0 < n_ent; s0 += kPer * 64) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) cur[u] = nxt[u];
    if (s0 + kPer * 64 < n_ent) fetch(nxt, s0 + kPer * 64);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      if (s0 + u * 64 < n_ent) {
        const int32_t blk = cur[u] - static_cast<int32_t>(lo);  // window column
        const bool valid = blk >= 0 && blk < nvis;
        for (int h = 0; h < halves; ++h) {
          const bool ok = valid && (halves == 1 || (lane >> 5) == h);
          const int32_t qrow = __builtin_amdgcn_readlane(q, h * 32);
          const uint32_t bit = static_cast<uint32_t>(q - qrow);
          const uint32_t lower = (1u << bit) - 1u;
          if (ok)
            __hip_atomic_fetch_or(&cm[2 * blk + 1], 1u << bit, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_WORKGROUP);
          uint32_t c = 0, m = 0;
          if (ok) {
            c = cm[2 * blk];
            m = cm[2 * blk + 1];
          }
          if (ok && (m & lower) == 0u) {
            cm[2 * blk] = c + __popc(m);
            cm[2 * blk + 1] = 0u;
          }
          if (ok) {
            const int32_t pos = static_cast<int32_t>(c) + __popc(m & lower);
            const int64_t dst = (ibase + pos) * istride;
            if (records) {
              *reinterpret_cast<i32x3*>(row_indices + dst) =
                  i32x3{rbase + q, static_cast<int32_t>(hq), j};
            } else {
              row_indices[dst] = rbase + q;
              head_indices[dst] = static_cast<int32_t>(hq);
              slot_of_pair[dst] = j;
            }
          }
        }
      }
      q += dq;
      j += dj;
      if (j >= slots) {
        j -= slots;
        ++q;
      }
    }
  }
}

// Inclusive scan of x over a 1024-thread workgroup (every thread calls it):
// a shuffle scan inside each wave, then each thread adds the totals of the
// waves before its own. `total` receives the sum over the workgroup. wtot
// is 16 ints of LDS, free again when the call returns.
__device__ inline int32_t block_scan_1024(int32_t x, int32_t* wtot, int32_t& total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int32_t y = __shfl_up(x, o);
    if (lane >= o) x += y;
  }
  if (lane == 63) wtot[wave] = x;
  __syncthreads();
  int32_t before = 0, sum = 0;
#pragma unroll
  for (int w = 0; w < 16; ++w) {
    const int32_t t = wtot[w];
    before += w < wave ? t : 0;
    sum += t;
  }
  __syncthreads();
  total = sum;
  return x + before;
}

// Exclusive scan of one (row, kv head)'s counts; one workgroup each.
__global__ void __launch_bounds__(1024)
scan_kernel(const int32_t* __restrict__ col_nnz, int32_t* __restrict__ col_offsets,
            int64_t n_blocks) {
  __shared__ int32_t wtot[16];
  const int64_t rh = blockIdx.x;
  const int32_t* cnt = col_nnz + rh * n_blocks;
  int32_t* off = col_offsets + rh * (n_blocks + 1);
  int32_t carry = 0;
  for (int64_t base = 0; base < n_blocks; base += 1024) {
    const int64_t i = base + threadIdx.x;
    const int32_t x = i < n_blocks ? cnt[i] : 0;
    int32_t total;
    const int32_t inc = block_scan_1024(x, wtot, total);
    if (i < n_blocks) off[i] = carry + inc - x;
    carry += total;
  }
  if (threadIdx.x == 0) off[n_blocks] = carry;
}

// order[rh, rank] = column with that rank under (nnz desc, column asc).
// Eight lanes share one column and split its comparisons, four counts per
// 16-byte LDS read with several reads in flight; their partial ranks meet by
// shuffles.
__global__ void __launch_bounds__(256)
order_kernel(const int32_t* __restrict__ col_nnz, int32_t* __restrict__ order,
             int64_t n_blocks) {
  constexpr int kTile = 4096;
  __shared__ __attribute__((aligned(16))) int32_t tile[kTile];
  const int64_t rh = blockIdx.y;
  const int32_t* cnt = col_nnz + rh * n_blocks;
  const int sub = threadIdx.x & 7;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 8) + (threadIdx.x >> 3);
  const int32_t mine = c < n_blocks ? cnt[c] : 0;
  int rank = 0;
  for (int64_t base = 0; base < n_blocks; base += kTile) {
    const int64_t len = n_blocks - base < kTile ? n_blocks - base : kTile;
    const int64_t len4 = (len + 3) & ~int64_t(3);  // whole 16-byte reads; only these are compared
    __syncthreads();
    // Past the end: -1 (no count is negative, so it is never larger), and
    // ids past every column (never a smaller id with an equal count).
    for (int64_t i = threadIdx.x; i < len4; i += blockDim.x) tile[i] = i < len ? cnt[base + i] : -1;
    __syncthreads();
    if (c < n_blocks) {
      const int4* t4 = reinterpret_cast<const int4*>(tile);
#pragma unroll 4
      for (int i4 = sub; i4 < len4 / 4; i4 += 8) {
        const int4 o = t4[i4];
        const int64_t id = base + 4 * i4;
        rank += (o.x > mine || (o.x == mine && id < c)) ? 1 : 0;
        rank += (o.y > mine || (o.y == mine && id + 1 < c)) ? 1 : 0;
        rank += (o.z > mine || (o.z == mine && id + 2 < c)) ? 1 : 0;
        rank += (o.w > mine || (o.w == mine && id + 3 < c)) ? 1 : 0;
      }
    }
  }
  rank += __shfl_xor(rank, 1);
  rank += __shfl_xor(rank, 2);
  rank += __shfl_xor(rank, 4);
  if (c < n_blocks && sub == 0) order[rh * n_blocks + rank] = static_cast<int32_t>(c);
}

// The same order by sorting: one workgroup per (row, kv head) sorts the
// 64-bit keys (INT32_MAX - count) << 32 | id ascending -- count descending,
// id ascending -- in LDS with a bitonic network over n2 keys (the power of
// two >= n_blocks; the padding keys, all ones, sort last). O(n log^2 n)
// against the rank kernel's O(n^2): 78 barrier-separated passes at
// n_blocks = 4096, each lane comparing two pairs per pass. Dynamic LDS:
// 8 * n2 bytes, so up to n2 = 16384 on a device with 160 KiB.
constexpr int kOrderSortMaxKeys = 16384;
constexpr size_t kOrderSortMaxLds = 8 * static_cast<size_t>(kOrderSortMaxKeys);
__global__ void __launch_bounds__(1024)
order_sort_kernel(const int32_t* __restrict__ col_nnz, int32_t* __restrict__ order,
                  int64_t n_blocks, int n2) {
  extern __shared__ uint64_t okey[];
  const int64_t rh = blockIdx.x;
  const int32_t* cnt = col_nnz + rh * n_blocks;
  const int tid = threadIdx.x;
  for (int i = tid; i < n2; i += 1024)
    okey[i] = i < n_blocks
                  ? (static_cast<uint64_t>(0x7fffffff - cnt[i]) << 32) | static_cast<uint32_t>(i)
                  : ~uint64_t{0};
  __syncthreads();
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < n2 / 2; i += 1024) {
        const int lo = 2 * i - (i & (j - 1));  // pair (lo, lo + j), lo's bit j clear
        const uint64_t x = okey[lo], y = okey[lo + j];
        // Ascending where bit k of lo is clear, descending where it is set.
        if ((x > y) == ((lo & k) == 0)) {
          okey[lo] = y;
          okey[lo + j] = x;
        }
      }
      __syncthreads();
    }
  }
  for (int64_t i = tid; i < n_blocks; i += 1024)
    order[rh * n_blocks + i] = static_cast<int32_t>(okey[i] & 0xffffffffu);
}

// Segment list of one (row, kv head): its columns in `order` (longest first),
// a column of n entries cut into min(max_seg, ceil(n / seg_len)) segments of
// near-equal length (at least one, also when empty). Entry (c, s, nseg, x):
// column (block id) c, segment s of nseg, and x = the segment's slot in the
// dK / dV scratch when nseg > 1 (else -1). split[rh * (cap - n_blocks) + i]
// lists the first segment of every cut column; counts[2 rh] / counts[2 rh + 1]
// hold the numbers of segments and of cut columns. One workgroup per
// (row, kv head); writes past the capacities are dropped (the caller sizes
// them from an upper bound, so none happen).
__global__ void __launch_bounds__(1024)
seg_build_kernel(const int32_t* __restrict__ col_nnz, const int32_t* __restrict__ order,
                 int64_t n_blocks, int64_t seg_len, int max_seg, int32_t* __restrict__ seg,
                 int32_t* __restrict__ split, int32_t* __restrict__ counts, int64_t cap) {
  __shared__ int32_t wtot[16];
  const int64_t rh = blockIdx.x;
  const int64_t extra_cap = cap - n_blocks;
  const int tid = threadIdx.x;
  int32_t carry_seg = 0, carry_scr = 0, carry_split = 0;
  for (int64_t base = 0; base < n_blocks; base += 1024) {
    const int64_t p = base + tid;
    int32_t nseg = 0;
    if (p < n_blocks) {
      const int64_t n = col_nnz[rh * n_blocks + order[rh * n_blocks + p]];
      const int64_t k = (n + seg_len - 1) / seg_len;
      nseg = static_cast<int32_t>(k < 1 ? 1 : (k > max_seg ? max_seg : k));
    }
    const int32_t nscr = nseg > 1 ? nseg : 0;
    int32_t tot_seg, tot_scr, tot_split;
    const int32_t first = carry_seg + block_scan_1024(nseg, wtot, tot_seg) - nseg;
    const int32_t first_scr = carry_scr + block_scan_1024(nscr, wtot, tot_scr) - nscr;
    for (int32_t j = 0; j < nseg; ++j) {
      const int64_t at = first + j;
      if (at < cap) {
        int32_t* e = seg + (rh * cap + at) * 4;
        e[0] = order[rh * n_blocks + p];
        e[1] = j;
        e[2] = nseg;
        e[3] = nscr ? first_scr + j : -1;
      }
    }
    const int32_t nth = block_scan_1024(nscr ? 1 : 0, wtot, tot_split);  // cut columns so far
    if (nscr && carry_split + nth - 1 < extra_cap)
      split[rh * extra_cap + carry_split + nth - 1] = first;
    carry_seg += tot_seg;
    carry_scr += tot_scr;
    carry_split += tot_split;
  }
  if (tid == 0) {
    counts[2 * rh] = carry_seg < cap ? carry_seg : static_cast<int32_t>(cap);
    counts[2 * rh + 1] = carry_split < extra_cap ? carry_split : static_cast<int32_t>(extra_cap);
  }
}

}  // namespace moba

namespace {
// Deterministic-build geometry: units of one (row, kv head) and their chunks.
struct UnitPlan {
  int64_t tiles, units, chunk, nchunks;
};
UnitPlan unit_plan(int64_t rows_per_seq, int64_t h_q, int64_t h_kv, int64_t tq) {
  UnitPlan p;
  p.tiles = moba::cdiv(rows_per_seq, tq);
  p.units = (h_kv > 0 ? h_q / h_kv : 1) * p.tiles;
  p.chunk = moba::cdiv(p.units, 64) > 16 ? moba::cdiv(p.units, 64) : 16;
  p.nchunks = moba::cdiv(p.units, p.chunk);
  return p;
}
// True when det_scatter_kernel (order_sort_kernel) may take `bytes` of
// dynamic LDS on the current device: always up to 64 KiB; beyond that when
// the device's opt-in limit allows it, after raising both kernels' limits
// (to kDetLdsBytes, kOrderSortMaxLds) once per process.
bool det_lds_ok(size_t bytes) {
  if (bytes <= 65536) return true;
  int dev = 0, optin = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&optin, hipDeviceAttributeSharedMemPerBlockOptin, dev) != hipSuccess ||
      static_cast<size_t>(optin) < bytes)
    return false;
  static std::once_flag once;
  static bool raised = false;
  std::call_once(once, [] {
    raised = hipFuncSetAttribute(reinterpret_cast<const void*>(moba::det_scatter_kernel),
                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                 static_cast<int>(moba::kDetLdsBytes)) == hipSuccess &&
             hipFuncSetAttribute(reinterpret_cast<const void*>(moba::order_sort_kernel),
                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                 static_cast<int>(moba::kOrderSortMaxLds)) == hipSuccess;
  });
  return raised;
}
}  // namespace

extern "C" size_t moba_csc_workspace_size(int64_t batch, int64_t rows_per_seq, int64_t h_q,
                                          int64_t h_kv, int64_t n_blocks, int64_t slots) {
  (void)slots;
  // Unit table and chunk sums of one column window. This is never smaller
  // than the atomic cursors of the untiled build (batch * h_kv * n_blocks),
  // which run in the same memory when the device lacks the LDS.
  const UnitPlan p = unit_plan(rows_per_seq, h_q, h_kv, moba::tile_queries(batch, h_q, rows_per_seq));
  const int64_t width = n_blocks < moba::kDetMaxCols ? n_blocks : moba::kDetMaxCols;
  const size_t det = sizeof(int32_t) * static_cast<size_t>(batch * width *
                                                          (h_q * p.tiles + h_kv * p.nchunks));
  const size_t cur = sizeof(int32_t) * static_cast<size_t>(batch * h_kv * n_blocks);
  return det > cur ? det : cur;
}

extern "C" int moba_csc_build(const int32_t* block_idx, int32_t* col_nnz,
                              int32_t* col_offsets, int32_t* row_indices,
                              int32_t* head_indices, int32_t* slot_of_pair,
                              int32_t* order, const int32_t* cu_seqlens, int64_t batch,
                              int64_t seq_len, int64_t max_seqlen, int64_t h_q,
                              int64_t h_kv, int64_t n_blocks, int64_t slots,
                              int64_t index_stride, int32_t* segments, int32_t* seg_split,
                              int32_t* seg_counts, int64_t seg_cap, int64_t seg_len,
                              int64_t max_seg, void* workspace, size_t workspace_bytes,
                              void* stream) {
  using namespace moba;
  Geometry g;
  const int64_t rps = cu_seqlens ? max_seqlen : seq_len;
  int st = make_geometry(&g, batch, seq_len, max_seqlen, h_q, h_kv, 64, n_blocks,
                         n_blocks > 0 ? cdiv(rps, n_blocks) : 1, slots, cu_seqlens);
  if (st) return st;
  if (slots <= 0) return fail(MOBA_ERR_INVALID, "slots must be positive");
  if (index_stride < 1) return fail(MOBA_ERR_INVALID, "index_stride must be positive");
  if (segments && (!seg_split || !seg_counts || seg_cap < n_blocks || seg_len < 1 ||
                   max_seg < 1 || max_seg > 64))
    return fail(MOBA_ERR_INVALID, "segment list: need split / counts, seg_cap >= n_blocks, "
                                  "seg_len >= 1, 1 <= max_seg <= 64");
  if (!block_idx || !col_nnz || !col_offsets || !row_indices || !head_indices ||
      !slot_of_pair || !order)
    return fail(MOBA_ERR_INVALID, "null pointer");
  const size_t need = moba_csc_workspace_size(batch, rps, h_q, h_kv, n_blocks, slots);
  if (!workspace || workspace_bytes < need)
    return fail(MOBA_ERR_WORKSPACE, "csc workspace too small");
  const int64_t cap = g.group * g.rows_per_seq * slots;
  if (cap >= (int64_t(1) << 31))
    return fail(MOBA_ERR_UNSUPPORTED, "column capacity exceeds int32 offsets");
  hipStream_t s = as_stream(stream);
  const bool records = index_stride == 3 && head_indices == row_indices + 1 &&
                       slot_of_pair == row_indices + 2;
  const int64_t ncols = batch * h_kv * n_blocks;
  const unsigned fill_blocks = static_cast<unsigned>(cdiv(ncols, 256) < 4096 ? cdiv(ncols, 256) : 4096);
  // A lower bound on the block size: cdiv(rows, n_blocks) <= block_size, so
  // t / bs_eff never under-counts the blocks a query can see.
  // Columns go in windows of at most kDetMaxCols (the LDS of one scatter).
  const int64_t win = n_blocks < kDetMaxCols ? n_blocks : kDetMaxCols;
  const int64_t n_win = cdiv(n_blocks, win);
  const size_t det_lds = 8 * static_cast<size_t>(win);
  const bool tiled = det_lds_ok(det_lds);
  const int64_t bs_eff = cdiv(g.rows_per_seq, n_blocks);
  const int64_t tq = tile_queries(batch, h_q, g.rows_per_seq);
  const UnitPlan up = unit_plan(g.rows_per_seq, h_q, h_kv, tq);
  const unsigned rhk = static_cast<unsigned>(batch * h_kv);
  dim3 grid(static_cast<unsigned>(cdiv(g.rows_per_seq * slots, 256)),
            static_cast<unsigned>(batch * h_q));
  dim3 tgrid(static_cast<unsigned>(up.tiles), static_cast<unsigned>(batch * h_q));
  int32_t* table = static_cast<int32_t*>(workspace);
  int32_t* csum = table + batch * h_q * up.tiles * win;
  int32_t* cursor = static_cast<int32_t*>(workspace);
  // Deterministic build of the window [lo, lo + width): per-unit counts,
  // scanned into per-unit bases (after col_offsets exist), then placed.
  auto window_counts = [&](int64_t lo, int64_t width, int32_t* nnz) {
    hipLaunchKernelGGL(tile_count_kernel, tgrid, dim3(kTileT),
                       static_cast<unsigned>(sizeof(int32_t) * width), s, block_idx, cu_seqlens,
                       seq_len, h_q, n_blocks, bs_eff, static_cast<int>(slots),
                       static_cast<int>(tq), table, lo, width);
    hipLaunchKernelGGL(unit_chunk_kernel<0>,
                       dim3(static_cast<unsigned>(cdiv(width, 256)),
                            static_cast<unsigned>(up.nchunks), rhk),
                       dim3(256), 0, s, table, csum, nullptr, n_blocks, h_q, h_kv, up.units,
                       up.chunk, up.nchunks, lo, width);
    hipLaunchKernelGGL(chunk_scan_kernel, dim3(static_cast<unsigned>(cdiv(width, 256)), rhk),
                       dim3(256), 0, s, csum, nnz, n_blocks, up.nchunks, width);
  };
  auto window_place = [&](int64_t lo, int64_t width) {
    hipLaunchKernelGGL(unit_chunk_kernel<1>,
                       dim3(static_cast<unsigned>(cdiv(width, 256)),
                            static_cast<unsigned>(up.nchunks), rhk),
                       dim3(256), 0, s, table, csum, col_offsets, n_blocks, h_q, h_kv,
                       up.units, up.chunk, up.nchunks, lo, width);
    hipLaunchKernelGGL(det_scatter_kernel, tgrid, dim3(64),
                       static_cast<unsigned>(8 * width), s, block_idx, cu_seqlens, seq_len, h_q,
                       h_kv, n_blocks, bs_eff, static_cast<int>(slots), cap, table, row_indices,
                       head_indices, slot_of_pair, index_stride, records, static_cast<int>(tq),
                       lo, width);
  };
  if (tiled && n_win == 1) {
    window_counts(0, n_blocks, col_nnz);
  } else {
    // Column counts by atomics (their sums do not depend on the order).
    hipLaunchKernelGGL(fill_i32_kernel, dim3(fill_blocks), dim3(256), 0, s, col_nnz, ncols, 0);
    if (!tiled)
      hipLaunchKernelGGL(fill_i32_kernel, dim3(fill_blocks), dim3(256), 0, s, cursor, ncols, 0);
    hipLaunchKernelGGL(count_or_scatter_kernel<false>, grid, dim3(256), 0, s, block_idx,
                       cu_seqlens, seq_len, g.rows_per_seq, h_q, h_kv, n_blocks,
                       static_cast<int>(slots), cap, col_nnz, nullptr, nullptr, nullptr,
                       nullptr, index_stride);
  }
  hipLaunchKernelGGL(scan_kernel, dim3(rhk), dim3(1024), 0, s, col_nnz, col_offsets, n_blocks);
  int n2 = 1;
  while (n2 < n_blocks) n2 <<= 1;
  // The rank kernel is faster up to 4096 columns (27 vs 36 us for four
  // heads at 4096); its O(nb^2) cost passes the sort's above.
  if (n_blocks > 4096 && n2 <= kOrderSortMaxKeys && det_lds_ok(8 * static_cast<size_t>(n2)))
    hipLaunchKernelGGL(order_sort_kernel, dim3(rhk), dim3(1024), 8 * static_cast<unsigned>(n2), s,
                       col_nnz, order, n_blocks, n2);
  else
    hipLaunchKernelGGL(order_kernel, dim3(static_cast<unsigned>(cdiv(n_blocks, 32)), rhk),
                       dim3(256), 0, s, col_nnz, order, n_blocks);
  if (segments)
    hipLaunchKernelGGL(seg_build_kernel, dim3(rhk), dim3(1024), 0, s, col_nnz, order, n_blocks,
                       seg_len, static_cast<int>(max_seg), segments, seg_split, seg_counts,
                       seg_cap);
  if (tiled && n_win == 1) {
    window_place(0, n_blocks);
  } else if (tiled) {
    // One window after another through the same table; the counts again,
    // now per unit (col_nnz already holds their totals).
    for (int64_t w = 0; w < n_win; ++w) {
      const int64_t lo = w * win;
      const int64_t width = n_blocks - lo < win ? n_blocks - lo : win;
      window_counts(lo, width, nullptr);
      window_place(lo, width);
    }
  } else {
    hipLaunchKernelGGL(count_or_scatter_kernel<true>, grid, dim3(256), 0, s, block_idx,
                       cu_seqlens, seq_len, g.rows_per_seq, h_q, h_kv, n_blocks,
                       static_cast<int>(slots), cap, cursor, col_offsets, row_indices,
                       head_indices, slot_of_pair, index_stride);
  }
  return check_launch("moba_csc_build");
}
