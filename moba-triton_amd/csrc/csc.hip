// CSC transpose of the gate's per-query block ids into per-block columns.
//
// Restates src/moba/kernels/routing.py:139-301 (count / offsets+order /
// scatter) and routing.py:309-427 (launcher): counts per (row, kv head,
// block) with atomics, an exclusive scan into col_offsets, a longest-first
// column order (count desc, id asc; the stable argsort of routing.py:548-553),
// and an atomic-cursor scatter of (row, query head, slot) triples. Under GQA
// every query head of a group lands in its kv head's columns.
//
// The order pass ranks each column directly -- rank = #columns with a larger
// count, or the same count and a smaller id -- one lane per column against an
// LDS copy of the counts. It is O(nb^2) work spread over nb lanes; at
// nb = 4096 that is ~16M integer compares per head, a few microseconds.
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

// Workgroup-aggregated variant: kTileQ queries of one (row, query head) per
// workgroup, kTileT threads each taking kTileQ / kTileT of them. Selections
// are first counted in an LDS histogram over the blocks this tile can see,
// so the global counter of each block is touched once per workgroup -- the
// own block, which every query of a block selects, would otherwise take 128
// serialised global atomics, and a past block picked by several queries of
// the tile takes one. Those per-(tile, block) atomics bound both passes, so
// the tile is large. The scatter pass reserves each block's range with one
// global atomic and hands out positions from LDS.
constexpr int kTileQ = 1024;
typedef int32_t i32x3 __attribute__((ext_vector_type(3), aligned(4)));
constexpr int kTileT = 256;
constexpr int kMaxBins = 16384;

// atomicAdd(&bins[blk], 1) for every active lane, with the lanes that share
// the first active lane's id served by one atomic (every query of a block
// selects its own block, so a wave's 64 consecutive queries usually agree
// there); returns the old value plus the lane's rank among them.
__device__ inline int32_t bin_add(int32_t* bins, int32_t blk, bool active) {
  const uint64_t act = __ballot(active);
  if (act == 0) return 0;
  const int lead = __builtin_ctzll(act);
  const int32_t b0 = __shfl(blk, lead);
  const bool same = active && blk == b0;
  const uint64_t m = __ballot(same);
  const int lane = threadIdx.x & 63;
  const int32_t rank = __popcll(m & ((uint64_t(1) << lane) - 1));
  int32_t base = 0;
  if (lane == lead) base = atomicAdd(&bins[b0], __popcll(m));
  base = __shfl(base, lead);
  if (same) return base + rank;
  return active ? atomicAdd(&bins[blk], 1) : 0;
}

template <bool kScatter>
__global__ void __launch_bounds__(kTileT)
tile_count_or_scatter_kernel(const int32_t* __restrict__ block_idx,
                             const int32_t* __restrict__ cu, int64_t S, int64_t h_q,
                             int64_t h_kv, int64_t n_blocks, int64_t bs, int slots,
                             int64_t cap, int32_t* __restrict__ col_nnz_or_cursor,
                             const int32_t* __restrict__ col_offsets,
                             int32_t* __restrict__ row_indices,
                             int32_t* __restrict__ head_indices,
                             int32_t* __restrict__ slot_of_pair, int64_t istride,
                             bool records) {
  __shared__ int32_t bins[kMaxBins];
  const int64_t rh = blockIdx.y;
  const int64_t r = rh / h_q;
  const int64_t hq = rh % h_q;
  const int64_t hk = hq / (h_q / h_kv);
  const bool packed = cu != nullptr;
  const SeqSpan sp = seq_span(cu, r, S);
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * kTileQ;
  if (t0 >= sp.len) return;
  const int64_t t_last = (t0 + kTileQ < sp.len ? t0 + kTileQ : sp.len) - 1;
  const int64_t nv = t_last / bs + 1;  // blocks any query here can select
  const int nvis = static_cast<int>(nv < n_blocks ? nv : n_blocks);
  for (int b = threadIdx.x; b < nvis; b += kTileT) bins[b] = 0;
  __syncthreads();
  // Query i of this thread: t0 + threadIdx.x + kTileT * i (a wave's lanes
  // hold consecutive queries).
  auto query = [&](int i, int64_t& t, int64_t& tok, int64_t& qid) {
    t = t0 + threadIdx.x + kTileT * i;
    tok = sp.bos + t;
    qid = packed ? hq * S + tok : (r * h_q + hq) * S + t;
    return t < sp.len;
  };
  for (int i = 0; i < kTileQ / kTileT; ++i) {
    int64_t t, tok, qid;
    const bool live = query(i, t, tok, qid);
    for (int j = 0; j < slots; ++j) {
      const int32_t blk = live ? block_idx[qid * slots + j] : -1;
      bin_add(bins, blk, blk >= 0 && blk < nvis);
    }
  }
  __syncthreads();
  const int64_t colbase = (r * h_kv + hk) * n_blocks;
  const int64_t obase = (r * h_kv + hk) * (n_blocks + 1);
  for (int b = threadIdx.x; b < nvis; b += kTileT) {
    const int32_t n = bins[b];
    if (n > 0) {
      const int32_t base = atomicAdd(&col_nnz_or_cursor[colbase + b], n);
      // The scatter hands out positions from the column's start directly.
      if (kScatter) bins[b] = col_offsets[obase + b] + base;
    }
  }
  if (!kScatter) return;
  __syncthreads();
  const int64_t ibase = (r * h_kv + hk) * cap;
  for (int i = 0; i < kTileQ / kTileT; ++i) {
    int64_t t, tok, qid;
    const bool live = query(i, t, tok, qid);
    for (int j = 0; j < slots; ++j) {
      const int32_t blk = live ? block_idx[qid * slots + j] : -1;
      const bool ok = blk >= 0 && blk < nvis;
      const int32_t pos = bin_add(bins, blk, ok);
      if (!ok) continue;
      const int64_t dst = (ibase + pos) * istride;
      const int32_t rv = static_cast<int32_t>(packed ? tok : t);
      if (records) {  // (row, head, slot) adjacent: one 12-byte store
        *reinterpret_cast<i32x3*>(row_indices + dst) = i32x3{rv, static_cast<int32_t>(hq), j};
      } else {
        row_indices[dst] = rv;
        head_indices[dst] = static_cast<int32_t>(hq);
        slot_of_pair[dst] = j;
      }
    }
  }
}

// Exclusive scan of one (row, kv head)'s counts; one workgroup each.
__global__ void __launch_bounds__(1024)
scan_kernel(const int32_t* __restrict__ col_nnz, int32_t* __restrict__ col_offsets,
            int64_t n_blocks) {
  __shared__ int32_t buf[1024];
  const int64_t rh = blockIdx.x;
  const int32_t* cnt = col_nnz + rh * n_blocks;
  int32_t* off = col_offsets + rh * (n_blocks + 1);
  int32_t carry = 0;
  for (int64_t base = 0; base < n_blocks; base += 1024) {
    const int64_t i = base + threadIdx.x;
    const int32_t x = i < n_blocks ? cnt[i] : 0;
    buf[threadIdx.x] = x;
    __syncthreads();
    for (int s = 1; s < 1024; s <<= 1) {
      int32_t y = threadIdx.x >= s ? buf[threadIdx.x - s] : 0;
      __syncthreads();
      buf[threadIdx.x] += y;
      __syncthreads();
    }
    if (i < n_blocks) off[i] = carry + buf[threadIdx.x] - x;
    const int32_t total = buf[1023];
    __syncthreads();
    carry += total;
  }
  if (threadIdx.x == 0) off[n_blocks] = carry;
}

// order[rh, rank] = column with that rank under (nnz desc, column asc).
// Eight lanes share one column and split its comparisons; their partial
// ranks meet by shuffles.
__global__ void __launch_bounds__(256)
order_kernel(const int32_t* __restrict__ col_nnz, int32_t* __restrict__ order,
             int64_t n_blocks) {
  __shared__ int32_t tile[4096];
  const int64_t rh = blockIdx.y;
  const int32_t* cnt = col_nnz + rh * n_blocks;
  const int sub = threadIdx.x & 7;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * (blockDim.x / 8) + (threadIdx.x >> 3);
  const int32_t mine = c < n_blocks ? cnt[c] : 0;
  int rank = 0;
  for (int64_t base = 0; base < n_blocks; base += 4096) {
    const int64_t len = n_blocks - base < 4096 ? n_blocks - base : 4096;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < len; i += blockDim.x) tile[i] = cnt[base + i];
    __syncthreads();
    if (c < n_blocks) {
      for (int64_t i = sub; i < len; i += 8) {
        const int32_t o = tile[i];
        const int64_t id = base + i;
        rank += (o > mine || (o == mine && id < c)) ? 1 : 0;
      }
    }
  }
  rank += __shfl_xor(rank, 1);
  rank += __shfl_xor(rank, 2);
  rank += __shfl_xor(rank, 4);
  if (c < n_blocks && sub == 0) order[rh * n_blocks + rank] = static_cast<int32_t>(c);
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
  __shared__ int32_t sa[1024], sb[1024];
  const int64_t rh = blockIdx.x;
  const int tid = threadIdx.x;
  const int64_t extra_cap = cap - n_blocks;
  // Inclusive scan of sa (and sb) over the workgroup.
  auto scan = [&](bool both) {
    for (int w = 1; w < 1024; w <<= 1) {
      const int32_t x = tid >= w ? sa[tid - w] : 0;
      const int32_t y = both && tid >= w ? sb[tid - w] : 0;
      __syncthreads();
      sa[tid] += x;
      if (both) sb[tid] += y;
      __syncthreads();
    }
  };
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
    sa[tid] = nseg;
    sb[tid] = nscr;
    __syncthreads();
    scan(true);
    const int32_t first = carry_seg + sa[tid] - nseg;
    const int32_t first_scr = carry_scr + sb[tid] - nscr;
    const int32_t tot_seg = sa[1023], tot_scr = sb[1023];
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
    __syncthreads();  // every thread has read the scans
    sa[tid] = nscr ? 1 : 0;
    __syncthreads();
    scan(false);
    if (nscr && carry_split + sa[tid] - 1 < extra_cap)
      split[rh * extra_cap + carry_split + sa[tid] - 1] = first;
    const int32_t tot_split = sa[1023];
    __syncthreads();
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

extern "C" size_t moba_csc_workspace_size(int64_t batch, int64_t seq_len, int64_t h_q,
                                          int64_t h_kv, int64_t n_blocks, int64_t slots) {
  (void)seq_len; (void)h_q; (void)slots;
  return sizeof(int32_t) * static_cast<size_t>(batch * h_kv * n_blocks);
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
  const size_t need = moba_csc_workspace_size(batch, seq_len, h_q, h_kv, n_blocks, slots);
  if (!workspace || workspace_bytes < need)
    return fail(MOBA_ERR_WORKSPACE, "csc workspace too small");
  const int64_t cap = g.group * g.rows_per_seq * slots;
  if (cap >= (int64_t(1) << 31))
    return fail(MOBA_ERR_UNSUPPORTED, "column capacity exceeds int32 offsets");
  hipStream_t s = as_stream(stream);
  int32_t* cursor = static_cast<int32_t*>(workspace);
  const bool records = index_stride == 3 && head_indices == row_indices + 1 &&
                       slot_of_pair == row_indices + 2;
  const int64_t ncols = batch * h_kv * n_blocks;
  const unsigned fill_blocks = static_cast<unsigned>(cdiv(ncols, 256) < 4096 ? cdiv(ncols, 256) : 4096);
  hipLaunchKernelGGL(fill_i32_kernel, dim3(fill_blocks), dim3(256), 0, s, col_nnz, ncols, 0);
  hipLaunchKernelGGL(fill_i32_kernel, dim3(fill_blocks), dim3(256), 0, s, cursor, ncols, 0);
  // A lower bound on the block size: cdiv(rows, n_blocks) <= block_size, so
  // t / bs_eff never under-counts the blocks a query can see.
  const bool tiled = n_blocks <= kMaxBins;
  const int64_t bs_eff = cdiv(g.rows_per_seq, n_blocks);
  dim3 grid(static_cast<unsigned>(cdiv(g.rows_per_seq * slots, 256)),
            static_cast<unsigned>(batch * h_q));
  dim3 tgrid(static_cast<unsigned>(cdiv(g.rows_per_seq, kTileQ)),
             static_cast<unsigned>(batch * h_q));
  if (tiled)
    hipLaunchKernelGGL(tile_count_or_scatter_kernel<false>, tgrid, dim3(kTileT), 0, s,
                       block_idx, cu_seqlens, seq_len, h_q, h_kv, n_blocks, bs_eff,
                       static_cast<int>(slots), cap, col_nnz, nullptr, nullptr, nullptr,
                       nullptr, index_stride, false);
  else
    hipLaunchKernelGGL(count_or_scatter_kernel<false>, grid, dim3(256), 0, s, block_idx,
                       cu_seqlens, seq_len, g.rows_per_seq, h_q, h_kv, n_blocks,
                       static_cast<int>(slots), cap, col_nnz, nullptr, nullptr, nullptr,
                       nullptr, index_stride);
  hipLaunchKernelGGL(scan_kernel, dim3(static_cast<unsigned>(batch * h_kv)), dim3(1024), 0, s,
                     col_nnz, col_offsets, n_blocks);
  hipLaunchKernelGGL(order_kernel,
                     dim3(static_cast<unsigned>(cdiv(n_blocks, 32)),
                          static_cast<unsigned>(batch * h_kv)),
                     dim3(256), 0, s, col_nnz, order, n_blocks);
  if (segments)
    hipLaunchKernelGGL(seg_build_kernel, dim3(static_cast<unsigned>(batch * h_kv)), dim3(1024),
                       0, s, col_nnz, order, n_blocks, seg_len, static_cast<int>(max_seg),
                       segments, seg_split, seg_counts, seg_cap);
  if (tiled)
    hipLaunchKernelGGL(tile_count_or_scatter_kernel<true>, tgrid, dim3(kTileT), 0, s,
                       block_idx, cu_seqlens, seq_len, h_q, h_kv, n_blocks, bs_eff,
                       static_cast<int>(slots), cap, cursor, col_offsets, row_indices,
                       head_indices, slot_of_pair, index_stride, records);
  else
    hipLaunchKernelGGL(count_or_scatter_kernel<true>, grid, dim3(256), 0, s, block_idx,
                       cu_seqlens, seq_len, g.rows_per_seq, h_q, h_kv, n_blocks,
                       static_cast<int>(slots), cap, cursor, col_offsets, row_indices,
                       head_indices, slot_of_pair, index_stride);
  return check_launch("moba_csc_build");
}
