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

// One thread per (row, kv head, block, 8-feature chunk): it walks the
// block's tokens in order with one 16-byte load per token (the eight lanes
// of a block read each key row whole), accumulating every feature exactly
// in float64 in token order, then rounds once to float32 and to the dtype
// and divides by the block's real occupancy.
template <typename T>
__global__ void __launch_bounds__(256)
pool_kernel(const T* __restrict__ k, T* __restrict__ kbar,
            const int32_t* __restrict__ cu, int64_t S, int64_t h_kv,
            int64_t D, int64_t n_blocks, int64_t bs, int64_t n_items) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t cpr = D / 8;                 // 8-feature chunks per row
  const int64_t item = gid / cpr;            // (r * h_kv + h) * n_blocks + blk
  if (item >= n_items) return;
  const int64_t d0 = (gid % cpr) * 8;
  const int64_t blk = item % n_blocks;
  const int64_t rh = item / n_blocks;
  const int64_t r = rh / h_kv, h = rh % h_kv;
  const SeqSpan sp = seq_span(cu, r, S);
  T* dst = kbar + item * D + d0;
  const int64_t lo = blk * bs;
  if (lo >= sp.len) {  // a padded block slot of a short sequence: zeros
#pragma unroll
    for (int i = 0; i < 8; ++i) Elem<T>::store(dst, i, 0.f);
    return;
  }
  const int64_t hi = lo + bs < sp.len ? lo + bs : sp.len;
  double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  const T* src = k + ((sp.bos + lo) * h_kv + h) * D + d0;
  for (int64_t t = lo; t < hi; ++t, src += h_kv * D) {
    T x[8];
    if constexpr (sizeof(T) == 2) {
      *reinterpret_cast<uint4*>(x) = *reinterpret_cast<const uint4*>(src);
    } else {
      reinterpret_cast<uint4*>(x)[0] = reinterpret_cast<const uint4*>(src)[0];
      reinterpret_cast<uint4*>(x)[1] = reinterpret_cast<const uint4*>(src)[1];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] += static_cast<double>(Elem<T>::load(x, i));
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
      hipLaunchKernelGGL(pool_kernel<T>, dim3(static_cast<unsigned>(cdiv(n_items * (head_dim / 8), 256))),
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
