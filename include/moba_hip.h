/*
 * moba_hip.h -- C ABI of the MI355X (gfx950) MoBA block-sparse attention
 * library `libmoba_hip.so`.
 *
 * One entry point per stage of the reference's hot path
 * (ZuricZ/moba-triton, paths relative to the reference root):
 *
 *   pool -> gate -> CSC transpose -> KV-block-major attend -> LSE merge
 *   delta -> KV-block-major backward (dK, dV, per-slot dQ) -> dQ reduce
 *
 * Conventions (same as the reference, src/moba/gqa.py:55-62):
 *   - API tensors are token-major [B, S, H, D] (packed: [1, T, H, D]).
 *   - Internal buffers are head-major: kbar [R, Hkv, nb, D], block ids
 *     [B, Hq, S, slots], partials [B, Hq, S, slots(, D)], lse/delta
 *     [B, Hq, S]. R = B, or the sequence count when packed.
 *   - All pointers are device pointers allocated by the caller; nothing in
 *     this library allocates device memory. Scratch comes in through the
 *     `workspace` arguments, sized by the *_workspace_size queries.
 *   - Every call is asynchronous on `stream` (a hipStream_t, NULL = default
 *     stream) and never synchronises with the host.
 *   - Return value: MOBA_OK or an error code; moba_last_error() gives the
 *     message of the last failure on the calling thread. Shape / config
 *     errors are MOBA_ERR_INVALID (the Python layer raises ValueError, as
 *     the reference's _validate does, src/moba/kernels/moba_fwd.py:733-780);
 *     unsupported dtype / head_dim combinations are MOBA_ERR_UNSUPPORTED.
 *   - cu_seqlens (int32 [n_seq + 1], device) selects packed mode when
 *     non-NULL; then `batch` is the sequence count, `seq_len` the packed
 *     token count T, and `max_seqlen` the longest sequence.
 */
#ifndef MOBA_HIP_H_
#define MOBA_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum moba_status {
  MOBA_OK = 0,
  MOBA_ERR_INVALID = 1,
  MOBA_ERR_UNSUPPORTED = 2,
  MOBA_ERR_LAUNCH = 3,
  MOBA_ERR_WORKSPACE = 4
};

enum moba_dtype { MOBA_BF16 = 0, MOBA_FP16 = 1, MOBA_FP32 = 2 };

/* Library identity. moba_abi_version() is 6: (m, l) and (lse, delta) travel
 * as 8-byte pairs, the CSC index arrays take an element stride, the CSC
 * build can emit a segment list that attend and backward take, its
 * workspace is sized by rows per sequence, and moba_bwd takes the dK / dV
 * dtype (version 1 took separate statistics arrays; 2 had no index stride;
 * 3 no segments; 4 sized the CSC workspace by seq_len and ordered column
 * entries by atomic cursors; 5 wrote dK / dV in the input dtype only). */
int moba_abi_version(void);
const char* moba_last_error(void);
const char* moba_status_string(int status);

/*
 * Block means of K: kbar[r, h, n, :] = dtype( dtype(sum) / occupancy ).
 * Replaces pool_blocks (src/moba/kernels/pooling.py:103-163) and its kernel
 * (pooling.py:26-96). The block sum is exact (float64), then rounded to
 * float32 and to the input dtype before the divide; the quotient is rounded
 * to the input dtype. A short tail block divides by its real count.
 * k: [B, S, Hkv, D]; kbar: [R, Hkv, n_blocks, D]. Packed: blocks never
 * cross sequence boundaries and rows beyond a sequence's own block count are
 * written as zeros.
 */
int moba_pool(const void* k, void* kbar, const int32_t* cu_seqlens,
              int64_t batch, int64_t seq_len, int64_t max_seqlen,
              int64_t h_kv, int64_t head_dim, int64_t n_blocks,
              int64_t block_size, int dtype, void* stream);

/*
 * Gate: per query, the own block (if `always_current`) plus the top `take`
 * strictly-past blocks by q . kbar (unscaled), ranked by (score desc, block
 * id asc), score = exact dot rounded to float32 then to the input dtype.
 * Emits ids ascending, -1 padded: block_idx [B, Hq, S, slots] int32.
 * Replaces gate_select (src/moba/kernels/gating.py:343-448) and gate_kernel
 * (gating.py:93-335); selection semantics of src/moba/naive.py:64-146.
 * Under GQA query head g reads kbar head g / (Hq / Hkv).
 */
size_t moba_gate_workspace_size(int64_t batch, int64_t seq_len, int64_t h_q);
int moba_gate(const void* q, const void* kbar, int32_t* block_idx,
              const int32_t* cu_seqlens, int64_t batch, int64_t seq_len,
              int64_t max_seqlen, int64_t h_q, int64_t h_kv,
              int64_t head_dim, int64_t n_blocks, int64_t block_size,
              int64_t slots, int64_t take, int always_current, int dtype,
              void* workspace, size_t workspace_bytes, void* stream);

/*
 * Second stage of the opt-in hierarchical gate (never the default): for
 * each query, the strictly-past blocks inside the super-blocks listed in
 * super_idx [B, Hq, S, super_slots] (ascending super-block ids, -1 padded,
 * as moba_gate emits them when run over super-block representatives with
 * block size block_size * group), ranked by the gate's score and tie rule;
 * the best `take` plus the own block (if always_current) go to block_idx
 * [B, Hq, S, slots], ascending, -1 padded. super_slots * group <= 512;
 * padded input only. The scheme is the coarse-to-fine selection the
 * reference measured in docs/gate-hierarchical-measurements.md (no kernel
 * there); the first stage is moba_pool over the block representatives and
 * moba_gate over the result.
 */
int moba_gate_refine(const void* q, const void* kbar, const int32_t* super_idx,
                     int32_t* block_idx, int64_t batch, int64_t seq_len, int64_t h_q,
                     int64_t h_kv, int64_t head_dim, int64_t n_blocks, int64_t block_size,
                     int64_t group, int64_t super_slots, int64_t slots, int64_t take,
                     int always_current, int dtype, void* stream);

/*
 * moba_gate without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). No counterpart in the reference.
 * Same arguments, semantics and output as moba_gate; its scratch (queue
 * counter, kbar norms, one 8-byte queue entry and one 8-byte fallback-list
 * entry per query) is a static device array of about 33 MiB that each GPU the library runs on holds until the
 * process ends. Limits: batch * h_q * rows_per_seq <=
 * MOBA_GATE_STATIC_MAX_QUERIES and batch * h_q <= MOBA_GATE_STATIC_MAX_NORMS
 * (rows_per_seq = seq_len, or max_seqlen when packed); larger calls return
 * MOBA_ERR_WORKSPACE. The call allocates nothing. Every call on one GPU
 * shares that GPU's array (the call clears what must start at zero), so
 * calls that overlap in time on one GPU (different streams, or host
 * threads) race; serialise them. `stream` must belong to the current
 * device.
 */
#define MOBA_GATE_STATIC_MAX_QUERIES 2097152
#define MOBA_GATE_STATIC_MAX_NORMS 4096
int moba_gate_noalloc(const void* q, const void* kbar, int32_t* block_idx,
                      const int32_t* cu_seqlens, int64_t batch, int64_t seq_len,
                      int64_t max_seqlen, int64_t h_q, int64_t h_kv,
                      int64_t head_dim, int64_t n_blocks, int64_t block_size,
                      int64_t slots, int64_t take, int always_current, int dtype,
                      void* stream);

/*
 * CSC transpose of block_idx into per-(row, kv head, block) columns:
 * col_nnz [R, Hkv, nb], col_offsets [R, Hkv, nb + 1] (exclusive prefix
 * sum), row_indices / head_indices / slot_of_pair [R, Hkv, cap] with
 * cap = (Hq / Hkv) * rows_per_seq * slots, order [R, Hkv, nb] (column ids by
 * count desc, id asc). Each (query, slot) pair appears exactly once. A
 * column's entries are in (query head, row) order -- the order of the
 * dense-mask builder, routing.py:467-561 -- on every build, so the
 * backward's dK / dV sums are bitwise reproducible. Columns are placed in
 * windows of 16384 (each window re-reads block_idx). Only on a device that
 * cannot give one workgroup 128 KiB of LDS do entries claim positions by
 * atomic cursors, their order inside a column then being unspecified (as in
 * the reference's scatter, routing.py:35-52).
 * row_indices hold packed token indices when cu_seqlens is given.
 * Ids outside [0, n_blocks), and ids past the last block a query of the
 * same 1024-query tile can see, are ignored like the -1 padding (moba_gate
 * never writes them; the guard keeps a bad caller buffer from addressing
 * memory).
 * Entry i of the three index arrays is element i * index_stride of each:
 * index_stride 1 for three separate arrays, 3 for one array of (row, head,
 * slot) records passed as base, base + 1, base + 2 (one record per entry
 * keeps each scattered entry in one memory sector).
 * Segment list (optional; segments == NULL skips it): each (row, kv head)'s
 * columns in `order`, a column of n entries cut into min(max_seg,
 * ceil(n / seg_len)) segments of near-equal length, so one long column is
 * worked on by several programs. segments [R, Hkv, seg_cap, 4] int32 holds
 * (block, segment, segments of the column, scratch slot or -1); seg_split
 * [R, Hkv, seg_cap - nb] the first segment of every cut column; seg_counts
 * [R, Hkv, 2] the numbers of segments and of cut columns. seg_cap must be at
 * least nb + ceil((Hq/Hkv) * rows_per_seq * slots / seg_len).
 * Replaces build_csc_from_indices (src/moba/kernels/routing.py:309-427)
 * and its three kernels (routing.py:139-301); CSCIndex fields of
 * routing.py:73-130.
 */
/* Workspace of moba_csc_build in bytes; rows_per_seq is seq_len, or
 * max_seqlen when packed. With W = min(nb, 16384) it holds a count table of
 * R * Hq * ceil(rows_per_seq / 1024) * W int32 plus chunk sums of
 * R * Hkv * W * (at most 64) int32 (never less than R * Hkv * nb int32, the
 * atomic cursors of the fallback). */
size_t moba_csc_workspace_size(int64_t batch, int64_t rows_per_seq, int64_t h_q,
                               int64_t h_kv, int64_t n_blocks,
                               int64_t slots);
int moba_csc_build(const int32_t* block_idx, int32_t* col_nnz,
                   int32_t* col_offsets, int32_t* row_indices,
                   int32_t* head_indices, int32_t* slot_of_pair,
                   int32_t* order, const int32_t* cu_seqlens, int64_t batch,
                   int64_t seq_len, int64_t max_seqlen, int64_t h_q,
                   int64_t h_kv, int64_t n_blocks, int64_t slots,
                   int64_t index_stride, int32_t* segments, int32_t* seg_split,
                   int32_t* seg_counts, int64_t seg_cap, int64_t seg_len,
                   int64_t max_seg, void* workspace, size_t workspace_bytes,
                   void* stream);

/*
 * KV-block-major attend: for every column, the keys of that block against
 * every query that selected it; writes per-slot un-normalised partials
 * m (row max of q.k * D^-1/2 * log2 e, log2 units), l (sum of exp2) and
 * part_acc (sum of exp2 * v, in acc_dtype). m and l of a slot travel as
 * one 8-byte pair: part_ml [B, Hq, S, slots, 2] fp32 = (m, l); part_acc
 * [B, Hq, S, slots, D]. Unwritten slots keep m = -inf, which this call sets
 * before the kernel runs. The index arrays and index_stride are those of
 * moba_csc_build; with its segment list (segments != NULL) each segment is
 * one program, else each column.
 * Replaces attend_partials (src/moba/kernels/moba_fwd.py:566-665) and
 * moba_fwd_kernel (moba_fwd.py:230-425).
 */
int moba_attend(const void* q, const void* k, const void* v,
                const int32_t* col_nnz, const int32_t* col_offsets,
                const int32_t* row_indices, const int32_t* head_indices,
                const int32_t* slot_of_pair, const int32_t* order,
                float* part_ml, void* part_acc,
                const int32_t* cu_seqlens, int64_t batch, int64_t seq_len,
                int64_t max_seqlen, int64_t h_q, int64_t h_kv,
                int64_t head_dim, int64_t n_blocks, int64_t block_size,
                int64_t slots, int64_t index_cap, int64_t index_stride,
                const int32_t* segments, const int32_t* seg_split,
                const int32_t* seg_counts, int64_t seg_cap,
                int causal, int dtype, int acc_dtype, void* stream);

/*
 * LSE merge of the per-slot partials: out [B, S, Hq, D] (out_dtype) and,
 * when lse != NULL, lse [B, Hq, S] fp32 in log2 units. part_ml: the (m, l)
 * pairs moba_attend writes. Slots with m = -inf are skipped even if their
 * l / acc hold NaN.
 * Replaces combine_partials (src/moba/kernels/moba_fwd.py:668-725) and
 * moba_combine_kernel (moba_fwd.py:429-521).
 */
int moba_combine(const float* part_ml,
                 const void* part_acc, void* out, float* lse, int64_t batch,
                 int64_t seq_len, int64_t h_q, int64_t head_dim,
                 int64_t slots, int acc_dtype, int out_dtype, void* stream);

/*
 * delta = rowsum(dO * O) per (b, head, token). With lse == NULL, delta is
 * [B, Hq, S] fp32; otherwise it receives the (lse, delta) pairs moba_bwd
 * reads, [B, Hq, S, 2] fp32, lse copied from lse [B, Hq, S]. Replaces
 * compute_delta (src/moba/kernels/moba_bwd.py:454-470, kernel
 * moba_bwd.py:135-160).
 */
int moba_bwd_delta(const void* out, const void* dout, const float* lse,
                   float* delta, int64_t batch, int64_t seq_len, int64_t h_q,
                   int64_t head_dim, int dtype, void* stream);

/*
 * KV-block-major backward: dK, dV [B, S, Hkv, D] (dkv_dtype: the input
 * dtype, or MOBA_FP32 for the unrounded float32 sums, which a caller that
 * adds the dK / dV of several calls -- query-head subsets of one kv head --
 * rounds once at the end; every key written, zero for unselected blocks)
 * and one dQ partial per (query, slot):
 * dq_part [B, Hq, S, slots, D] (acc_dtype). Replaces the kernel launch in
 * moba_backward (src/moba/kernels/moba_bwd.py:506-579; kernel
 * moba_bwd.py:216-394). lse_delta: the (lse, delta) pairs moba_bwd_delta
 * writes, lse in log2 units as moba_combine writes it. The index arrays and
 * index_stride are those of moba_csc_build. With its segment list, the
 * segments of a cut column leave float32 dK / dV sums in seg_scratch
 * ([R, Hkv, scratch_cap, 2, bs, D] float32, scratch_cap >= 2 * (seg_cap -
 * nb)), which this call then adds in segment order into dK / dV.
 */
int moba_bwd(const void* q, const void* k, const void* v, const void* dout,
             const float* lse_delta, const int32_t* col_nnz,
             const int32_t* col_offsets, const int32_t* row_indices,
             const int32_t* head_indices, const int32_t* slot_of_pair,
             const int32_t* order, void* dk, void* dv, void* dq_part,
             const int32_t* cu_seqlens, int64_t batch, int64_t seq_len,
             int64_t max_seqlen, int64_t h_q, int64_t h_kv, int64_t head_dim,
             int64_t n_blocks, int64_t block_size, int64_t slots,
             int64_t index_cap, int64_t index_stride, const int32_t* segments,
             const int32_t* seg_split, const int32_t* seg_counts, int64_t seg_cap,
             float* seg_scratch, int64_t scratch_cap, int causal, int dtype,
             int acc_dtype, int dkv_dtype, void* stream);

/*
 * dQ [B, S, Hq, D] = sum over written slots of dq_part, gated by the
 * forward's m written-marker: slot j of row r reads part_m[(r * slots + j)
 * * m_stride] (m_stride 2 for the pairs of moba_attend, 1 for a plain m
 * array). Replaces reduce_dq (src/moba/kernels/moba_bwd.py:473-503, kernel
 * moba_bwd.py:398-446).
 */
int moba_dq_reduce(const void* dq_part, const float* part_m, int64_t m_stride, void* dq,
                   int64_t batch, int64_t seq_len, int64_t h_q,
                   int64_t head_dim, int64_t slots, int acc_dtype,
                   int out_dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MOBA_HIP_H_ */
