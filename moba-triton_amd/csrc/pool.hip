// Block mean-pooling of keys: kbar[r, h, n, :].
//
// Restates src/moba/kernels/pooling.py:26-96 (launcher :103-163) with the
// oracle's rounding: the block sum is formed in float64 (exact for any
// realistic input), rounded to float32 and to the storage dtype, divided by
// the real occupancy in float32 and rounded again.
//
// One workgroup per (block, row * kv head); one lane per feature column.
// Lanes of a wave read consecutive features of one token row, so every load
// instruction is a contiguous 128-256 byte segment; the 128 rows of a block
// are walked sequentially. The whole pass reads K once (HBM-bound, tiny).
#include "common.h"

namespace moba {

// TS threads per (row, kv head, block, 8-feature chunk). Each walks every
// TS-th token of the block with one 16-byte load per token (eight lanes
// read each key row whole) and accumulates the features in float64; the TS
// partial sums then meet by shuffles. For 16-bit inputs (8- or 11-bit
// significands, at most 128 terms) every partial and total float64 sum is
// exact whenever the block's values span less than 2^38 in magnitude, so
// the split changes nothing there; float32 inputs use TS = 1 (token order,
// like the oracle). The total is rounded once to float32 and to the dtype,
// then divided by the block's real occupancy.
template <typename T, int TS>
__global__ void __launch_bounds__(256)
pool_kernel(const T* __restrict__ k, T* __restrict__ kbar,
            const int32_t* __restrict__ cu, int64_t S, int64_t h_kv,
            int64_t D, int64_t n_blocks, int64_t bs, int64_t n_items) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t cpr = D / 8;                 // 8-feature chunks per row
  const int ts = static_cast<int>(gid % TS); // token phase (adjacent lanes)
  const int64_t lin = gid / TS;
  const int64_t item = lin / cpr;            // (r * h_kv + h) * n_blocks + blk
  const bool ok = item < n_items;
  const int64_t it = ok ? item : 0;
  const int64_t d0 = (lin % cpr) * 8;
  const int64_t blk = it % n_blocks;
  const int64_t rh = it / n_blocks;
  const int64_t r = rh / h_kv, h = rh % h_kv;
  const SeqSpan sp = seq_span(cu, r, S);
  const int64_t lo = blk * bs;
  const int64_t hi = lo + bs < sp.len ? lo + bs : sp.len;
  double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  if (ok && lo < sp.len) {
    const T* src = k + ((sp.bos + lo + ts) * h_kv + h) * D + d0;
    // Unrolled, so a lane keeps several rows in flight; non-temporal, since
    // every row of K is read once here.
#pragma unroll 8
    for (int64_t t = lo + ts; t < hi; t += TS, src += TS * h_kv * D) {
      T x[8];
      if constexpr (sizeof(T) == 2) {
        typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
        *reinterpret_cast<u32x4_nt*>(x) =
            __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(src));
      } else {
        reinterpret_cast<uint4*>(x)[0] = reinterpret_cast<const uint4*>(src)[0];
        reinterpret_cast<uint4*>(x)[1] = reinterpret_cast<const uint4*>(src)[1];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += static_cast<double>(Elem<T>::load(x, i));
    }
  }
#pragma unroll
  for (int off = TS / 2; off > 0; off >>= 1)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += __shfl_xor(acc[i], off);
  if (!ok || ts != 0) return;
  T* dst = kbar + item * D + d0;
  if (lo >= sp.len) {  // a padded block slot of a short sequence: zeros
#pragma unroll
    for (int i = 0; i < 8; ++i) Elem<T>::store(dst, i, 0.f);
    return;
  }
  const float count = static_cast<float>(hi - lo);
#pragma unroll
  for (int i = 0; i < 8; ++i)
    Elem<T>::store(dst, i, Elem<T>::round(static_cast<float>(acc[i])) / count);
}

// Same semantics for head_dim not a multiple of 8: one workgroup per block,
// threads over the features.
template <typename T>
__global__ void __launch_bounds__(256)
pool_any_kernel(const T* __restrict__ k, T* __restrict__ kbar,
                const int32_t* __restrict__ cu, int64_t S, int64_t h_kv,
                int64_t D, int64_t n_blocks, int64_t bs) {
  const int64_t blk = blockIdx.x;
  const int64_t r = blockIdx.y / h_kv;
  const int64_t h = blockIdx.y % h_kv;
  const SeqSpan sp = seq_span(cu, r, S);
  const int64_t lo = blk * bs;
  if (lo >= sp.len) {
    for (int64_t d = threadIdx.x; d < D; d += blockDim.x)
      Elem<T>::store(kbar, ((r * h_kv + h) * n_blocks + blk) * D + d, 0.f);
    return;
  }
  const int64_t hi = lo + bs < sp.len ? lo + bs : sp.len;
  for (int64_t d = threadIdx.x; d < D; d += blockDim.x) {
    double acc = 0.0;
    for (int64_t t = lo; t < hi; ++t)
      acc += static_cast<double>(Elem<T>::load(k, ((sp.bos + t) * h_kv + h) * D + d));
    float sum = Elem<T>::round(static_cast<float>(acc));
    float mean = sum / static_cast<float>(hi - lo);
    Elem<T>::store(kbar, ((r * h_kv + h) * n_blocks + blk) * D + d, mean);
  }
}

}  // namespace moba

extern "C" int moba_pool(const void* k, void* kbar, const int32_t* cu_seqlens,
                         int64_t batch, int64_t seq_len, int64_t max_seqlen,
                         int64_t h_kv, int64_t head_dim, int64_t n_blocks,
                         int64_t block_size, int dtype, void* stream) {
  using namespace moba;
  Geometry g;
  int st = make_geometry(&g, batch, seq_len, max_seqlen, h_kv, h_kv, head_dim,
                         n_blocks, block_size, 0, cu_seqlens);
  if (st) return st;
  if (!k || !kbar) return fail(MOBA_ERR_INVALID, "null pointer");
  return MOBA_DISPATCH_DTYPE(dtype, T, [&] {
    if (head_dim % 8 == 0) {
      const int64_t n_items = g.rows * h_kv * n_blocks;
      constexpr int TS = sizeof(T) == 2 ? 4 : 1;
      hipLaunchKernelGGL((pool_kernel<T, TS>),
                         dim3(static_cast<unsigned>(cdiv(n_items * (head_dim / 8) * TS, 256))),
                         dim3(256), 0, as_stream(stream), static_cast<const T*>(k),
                         static_cast<T*>(kbar), cu_seqlens, seq_len, h_kv, head_dim, n_blocks,
                         block_size, n_items);
    } else {
      dim3 grid(static_cast<unsigned>(n_blocks), static_cast<unsigned>(g.rows * h_kv));
      const int threads = head_dim < 256 ? static_cast<int>(head_dim) : 256;
      hipLaunchKernelGGL(pool_any_kernel<T>, grid, dim3(threads), 0, as_stream(stream),
                         static_cast<const T*>(k), static_cast<T*>(kbar), cu_seqlens,
                         seq_len, h_kv, head_dim, n_blocks, block_size);
    }
    return check_launch("moba_pool");
  });
}
