// Shared arguments and addressing of the KV-block-major attention kernels.
#pragma once

#include "common.h"

namespace moba {

// Everything a KV-block-major kernel needs, passed by value.
struct AttnArgs {
  const void* q;
  const void* k;
  const void* v;
  const void* dout;       // backward only
  const float* lse_delta; // backward only: (lse in log2 units, delta) per row
  const int32_t* col_nnz;
  const int32_t* col_offsets;
  const int32_t* row_indices;
  const int32_t* head_indices;
  const int32_t* slot_of_pair;
  int64_t istride;  // elements between consecutive entries of the three index arrays
  const int32_t* order;
  const int32_t* cu;
  float* part_ml;         // forward only: (m, l) per (row, slot)
  void* part_acc;         // forward: acc partials; backward: dq partials
  void* dk;               // backward only
  void* dv;               // backward only
  int dkv_f32;            // backward: dK / dV stored as float32, not the input dtype
  int64_t S;              // padded S, or packed token count T
  int64_t h_q, h_kv, D, n_blocks, bs, slots, cap;
  int causal;
  float scale_log2;       // D^-1/2 * log2(e)
  float scale;            // D^-1/2
  // Segment list (4 ints per entry: block, segment, segments of the column,
  // scratch slot) or null for one workgroup per whole column.
  const int32_t* seg;
  const int32_t* seg_split;   // first segment of every cut column
  const int32_t* seg_counts;  // per (row, kv head): segments, cut columns
  int64_t seg_cap;            // entries per (row, kv head)
  float* seg_scratch;         // backward: fp32 dK / dV of cut columns' segments
  int64_t scratch_cap;        // scratch slots per (row, kv head)
  int tile_keys;              // FMA attend: keys staged per tile when a block's K / V
                              // exceed LDS (0: the whole block at once)
};

// Per-column context resolved from (program column position, row * h_kv).
struct Column {
  int64_t r, hk;
  int64_t blk;
  int32_t n;       // entries in the column (segment)
  int32_t nseg;    // segments the column is cut into (1: whole)
  int32_t scratch; // scratch slot of this segment when nseg > 1
  bool skip;       // a program past the segment list: nothing to do
  int64_t lo;      // offset of the column in the index arrays (incl. row base)
  int64_t key0;    // first key position, in the frame row_indices use
  int64_t key_end; // one past the last valid key position, same frame
  int64_t tok0;    // global token index of key0 (addresses K / V)
};

__device__ inline Column resolve_column(const AttnArgs& a, int64_t x, int64_t rh) {
  // One return path, every field computed on both: an early return here
  // leaves the struct in scratch memory, read back inside the kernels' loops.
  Column c;
  c.r = rh / a.h_kv;
  c.hk = rh % a.h_kv;
  int64_t s = 0;
  c.nseg = 1;
  c.scratch = -1;
  c.skip = false;
  if (a.seg) {
    // Past the list: entry 0 (every column has one) with nothing to do.
    c.skip = x >= a.seg_counts[2 * rh];
    const int32_t* e = a.seg + (rh * a.seg_cap + (c.skip ? 0 : x)) * 4;
    c.blk = e[0];
    s = e[1];
    c.nseg = e[2];
    c.scratch = e[3];
  } else {
    c.blk = a.order[rh * a.n_blocks + x];
  }
  const int64_t n_all = a.col_nnz[rh * a.n_blocks + c.blk];
  const int64_t e0 = n_all * s / c.nseg, e1 = n_all * (s + 1) / c.nseg;
  c.n = c.skip ? 0 : static_cast<int32_t>(e1 - e0);
  c.lo = rh * a.cap + a.col_offsets[rh * (a.n_blocks + 1) + c.blk] + e0;
  // A column past its sequence's last block (packed sequences shorter than
  // max_seqlen; n_blocks above cdiv(S, bs)) holds no keys: key_end = key0,
  // and key0 / tok0 may then lie past the tensor, so no kernel may address
  // K or V of such a column.
  if (a.cu) {
    const int64_t bos = a.cu[c.r], eos = a.cu[c.r + 1];
    c.key0 = bos + c.blk * a.bs;                     // packed: global tokens
    c.key_end = c.key0 + a.bs < eos ? c.key0 + a.bs : eos;
    c.tok0 = c.key0;
  } else {
    c.key0 = c.blk * a.bs;                           // padded: local positions
    c.key_end = c.key0 + a.bs < a.S ? c.key0 + a.bs : a.S;
    c.tok0 = c.r * a.S + c.key0;
  }
  if (c.key_end < c.key0) c.key_end = c.key0;
  return c;
}

// Token-major element offset of (query row value, head) for this column's row.
__device__ inline int64_t q_offset(const AttnArgs& a, const Column& c, int32_t row, int32_t head) {
  const int64_t tok = a.cu ? row : c.r * a.S + row;
  return (tok * a.h_q + head) * a.D;
}

// Head-major row of (query, head) in [R * Hq, S] partial / lse buffers.
__device__ inline int64_t part_row(const AttnArgs& a, const Column& c, int32_t row, int32_t head) {
  return a.cu ? static_cast<int64_t>(head) * a.S + row : (c.r * a.h_q + head) * a.S + row;
}

// Kernel launchers implemented per file; each returns MOBA_ERR_UNSUPPORTED
// when its fast path does not cover the configuration.
int attend_mfma(const AttnArgs& a, int dtype, int acc_dtype, int64_t n_cols, hipStream_t st);
int bwd_mfma(const AttnArgs& a, int dtype, int acc_dtype, int64_t n_cols, hipStream_t st);

}  // namespace moba
