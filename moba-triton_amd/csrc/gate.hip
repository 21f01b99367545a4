// MoBA gate: per query, the top `take` strictly-past blocks by q . kbar.
//
// Semantics: src/moba/naive.py:64-146 (ranking by score desc, block id asc,
// i.e. the stable descending argsort of naive.py:124-127; -inf leftovers
// dropped; own block forced when always_current), emitted ascending with -1
// padding as src/moba/kernels/gating.py:300-335 does. The score is the exact
// dot product rounded once to float32 and once to the input dtype.
//
// Kernels:
//
// * gate_mfma_kernel (bf16 / fp16, the product path). A workgroup of four
//   waves owns 128 consecutive queries of one (row, query head); a wave owns
//   32, two lanes per query, each holding half of the query's features as
//   the MFMA B operand. Block representatives (kbar) stream through LDS in
//   stages of 64 rows; v_mfma_f32_32x32x16 scores a 32-block x 32-query
//   tile per wave with the query on the lane axis, so each lane holds 16
//   approximate float32 scores of its query per 32-block chunk and the
//   bookkeeping never crosses lanes.
//   - Pass 1 (every chunk once) keeps, per lane, the K largest maxima of
//     its 4-block groups as keys that carry the group id and an LDS slot
//     in their low mantissa bits, and each kept group's four scores in
//     that slot. The take-th largest of the pair's kept maxima is the
//     take-th best of a subset of the query's candidates, hence a lower
//     bound on L (the take-th best of all); theta lies just below the
//     scores that can round to the key R(bound - w) or above (every
//     selected key is at least that).
//   - Decide: |approx - exact| <= E with E = D 2^-22 |q| max|kbar| (twice
//     what D float32 additions, each rounding by at most one ulp, can
//     lose) plus the denormal terms, so a score's key (the exact score
//     rounded to float32 and to the dtype) lies in [R(a - w), R(a + w)], w
//     being E widened by float32 rounding. The candidates (scores >= theta
//     of the kept groups) are compacted per lane; those with a single possible
//     key are ranked by it, those straddling a rounding boundary and not
//     below the take-th lower key bound are rescored exactly (float64
//     partial dots of the two lanes, rounded like the oracle). The result
//     stands when everything left out (groups that left the list, scores
//     below theta, candidates beyond the buffers) has a key bound strictly
//     below the take-th selected key.
//   - Unsettled queries go, with their theta, to lists per (row, query
//     head, position bucket) for the fallback kernel.
//
// * gate_fallback_kernel: tiles of 128 such queries stream every chunk up
//   to the tile's horizon, with pass 1's group tracking, but the groups
//   rank by (largest key any of their scores can have, group id): a group
//   that left the list then ranks below the one that left last, so many
//   equal keys at the boundary (keys sharing a large common component)
//   settle by id, as the oracle breaks ties, instead of going to the
//   queue; the decision is the first kernel's on those groups. Where the
//   group ids do not fit the keys' low bits, the tiles append every score
//   above the lane's threshold to a per-lane LDS buffer instead, folded
//   into lists of the M best by (largest key, id).
//   The work follows the number of unsettled queries, not the number of
//   workgroups holding one. A list's last tile of at most 32 queries runs
//   in a split launch instead: its four waves take the same queries and a
//   quarter of the chunks each, and wave 0 merges their keyed lists, so a
//   lone late tile does not stream alone at one wave per SIMD.
//
//   A query that settles nowhere (more straddling candidates than the
//   buffers hold, constructed ties, inf / NaN input) is queued; it is
//   never guessed.
//
// * gate_queue_kernel: one workgroup of eight waves per queued query,
//   exact scores for every candidate, lists merged across each wave and
//   then across the waves.
//
// * gate_exact_kernel (fp32, take > 16 or unsupported shapes). One thread
//   per query, exact float64 scores for every candidate, streaming top-T in
//   registers.
#include "common.h"

#include <mutex>

namespace moba {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16-byte chunk

// Unsettled queries of gate_mfma_kernel wait for gate_fallback_kernel in
// lists per (row, query head, position bucket): (t, theta bits) pairs, cap
// entries per list (a bucket holds cap consecutive positions).
// A float rounded to T, to nearest even: bf16 takes the hardware conversion
// (v_cvt_pk_bf16_f32: round to nearest even, denormals kept, NaN quiet;
// equal to float_to_bf16 on all 2^32 inputs, in two instructions). Exact
// scores, computed in double, round through Elem<T>::round instead: given
// the cast of a double to float and then to __bf16, the compiler rounds the
// double to bf16 once, which is not the key (float first, then bf16).
template <typename T> __device__ inline float key_round(float v) { return Elem<T>::round(v); }
template <> __device__ inline float key_round<bf16_t>(float v) {
  return static_cast<float>(static_cast<__bf16>(v));
}

constexpr int kFbBuckets = 16;
struct FbLists {
  int2* list;
  int* count;
  int64_t cap;
};

// Workspace layout (bytes), each part starting on a 256-byte boundary:
// counters (int 0: queued queries, int 1: tiles the fallback kernel ran);
// max |kbar| per (row, kv head); the queue of query ids (int64 each, one per
// query); the fallback list lengths (int per (row, query head, bucket));
// the fallback lists ((t, theta) int2 entries, a bucket's positions each).
struct GateWs {
  int* counter;
  float* kbar_norm;
  int64_t* queue;
  int* fb_count;
  int2* fb_list;
  int64_t fb_cap;  // entries per fallback list
  size_t bytes;    // total size of the layout
};

static size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

// norms: (row, kv head) pairs; pairs: (row, query head) pairs.
static GateWs gate_ws(void* base, int64_t norms, int64_t pairs, int64_t rows_per_seq) {
  // A null base only sizes the layout.
  char* p = static_cast<char*>(base);
  auto at = [&](size_t off) { return p ? p + off : nullptr; };
  GateWs w;
  const int64_t fb_cap = (rows_per_seq + kFbBuckets - 1) / kFbBuckets;
  size_t o = 256;
  w.counter = reinterpret_cast<int*>(p);
  w.kbar_norm = reinterpret_cast<float*>(at(o));
  o += align256(sizeof(float) * norms);
  w.queue = reinterpret_cast<int64_t*>(at(o));
  o += align256(sizeof(int64_t) * pairs * rows_per_seq);
  w.fb_count = reinterpret_cast<int*>(at(o));
  o += align256(sizeof(int) * pairs * kFbBuckets);
  w.fb_list = reinterpret_cast<int2*>(at(o));
  o += sizeof(int2) * pairs * kFbBuckets * fb_cap;
  w.fb_cap = fb_cap;
  w.bytes = o;
  return w;
}

// ---------------------------------------------------------------------------
// Prologue: max |kbar_j| per (row, kv head), as float bits (non-negative, so
// unsigned order is value order and NaN, the largest pattern, survives).
// gate_init_kernel clears the maxima and the queue counter; gate_prep_kernel
// gives each block of kbar a thread and folds the maxima in with atomicMax.
// ---------------------------------------------------------------------------
__global__ void __launch_bounds__(256)
gate_init_kernel(unsigned* __restrict__ norm_bits, int64_t n, int* __restrict__ counter,
                 int* __restrict__ fb_count, int64_t n_fb) {
  for (int64_t i = threadIdx.x; i < n; i += blockDim.x) norm_bits[i] = 0u;
  for (int64_t i = threadIdx.x; i < n_fb; i += blockDim.x) fb_count[i] = 0;
  if (threadIdx.x < 2) counter[threadIdx.x] = 0;
}

template <typename T>
__global__ void __launch_bounds__(256)
gate_prep_kernel(const T* __restrict__ kbar, const int32_t* __restrict__ cu,
                 int64_t S, int64_t h_kv, int64_t n_blocks, int64_t D, int64_t bs,
                 unsigned* __restrict__ norm_bits) {
  // Eight lanes per block of kbar, each summing every eighth feature; the
  // partial sums meet by shuffles (the bound these norms feed carries a
  // 1e-4 relative slack, far above any float summation order's effect).
  // A grid-stride loop over the blocks, the maximum taken within the
  // workgroup, then one device atomic per workgroup (a few per row instead
  // of one per wave, which serialised on the row's word).
  __shared__ unsigned s_best[4];
  const int64_t rh = blockIdx.y;
  const int sub = static_cast<int>(threadIdx.x & 7);
  // Only the blocks a sequence owns hold data; the tail of a packed kbar row
  // is never read by the gate.
  const SeqSpan sp = seq_span(cu, rh / h_kv, S);
  const int64_t owned = (sp.len + bs - 1) / bs < n_blocks ? (sp.len + bs - 1) / bs : n_blocks;
  unsigned best = 0u;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * (blockDim.x >> 3);
  // Every lane of an 8-lane group runs the same trips, so the shuffles below
  // see all eight.
  for (int64_t j = (static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x) >> 3;
       j - (threadIdx.x >> 3) < owned; j += stride) {
    float ss = 0.f;
    if (j < owned) {
      const T* row = kbar + (rh * n_blocks + j) * D;
      for (int64_t d = sub; d < D; d += 8) {
        const float x = Elem<T>::load(row, d);
        ss = fmaf(x, x, ss);
      }
    }
    ss += __shfl_xor(ss, 1);
    ss += __shfl_xor(ss, 2);
    ss += __shfl_xor(ss, 4);
    if (j < owned) best = max(best, f2u(sqrtf(ss)) & 0x7fffffffu);  // drop the sign of a NaN
  }
  for (int off = 32; off > 0; off >>= 1) best = max(best, static_cast<unsigned>(__shfl_xor(static_cast<int>(best), off)));
  if ((threadIdx.x & 63) == 0) s_best[threadIdx.x >> 6] = best;
  __syncthreads();
  if (threadIdx.x == 0) {
    best = max(max(s_best[0], s_best[1]), max(s_best[2], s_best[3]));
    if (best != 0u) atomicMax(norm_bits + rh, best);
  }
}

// ---------------------------------------------------------------------------
// Exact scoring helpers.
// ---------------------------------------------------------------------------
template <typename T>
__device__ inline float exact_score(const T* __restrict__ q, const T* __restrict__ kb, int D) {
  // Products of two bf16/fp16/fp32 values are exact in float64, and so is
  // the sum for any realistic input; it is rounded once to float32 and once
  // to the storage dtype, like the oracle's scores.
  double acc = 0.0;
  if constexpr (sizeof(T) == 2) {
    for (int d0 = 0; d0 < D; d0 += 8) {
      const uint4 qa = *reinterpret_cast<const uint4*>(q + d0);
      const uint4 ka = *reinterpret_cast<const uint4*>(kb + d0);
      const T* qe = reinterpret_cast<const T*>(&qa);
      const T* ke = reinterpret_cast<const T*>(&ka);
#pragma unroll
      for (int i = 0; i < 8; ++i)
        acc += static_cast<double>(Elem<T>::load(qe, i)) * static_cast<double>(Elem<T>::load(ke, i));
    }
  } else {
    for (int d = 0; d < D; ++d)
      acc += static_cast<double>(Elem<T>::load(q, d)) * static_cast<double>(Elem<T>::load(kb, d));
  }
  return Elem<T>::round(static_cast<float>(acc));
}

// (s, j) ranks before (v, i) under (score desc, id asc).
__device__ inline bool ranks_before(float s, int j, float v, int i) {
  return s > v || (s == v && j < i);
}

// Inserts (s, j) into a list sorted by (score desc, id asc); the last entry
// falls off. Entries with score -inf / NaN never enter.
// Branch-free: every step selects, so a wave never splits over the list.
template <int M>
__device__ inline void insert_exact(float (&val)[M], int (&idx)[M], float s, int j) {
  bool carry = false;
#pragma unroll
  for (int p = 0; p < M; ++p) {
    const bool take = carry || ranks_before(s, j, val[p], idx[p]);
    const float tv = val[p];
    const int ti = idx[p];
    val[p] = take ? s : tv;
    idx[p] = take ? j : ti;
    s = take ? tv : s;
    j = take ? ti : j;
    carry = take;
  }
}

// val / idx <- the best M of its union with pv / pi (both sorted by (score
// desc, id asc), ids disjoint), sorted: the better of val[p] and pv[M-1-p]
// for every p are the best M of the union, in an order that falls then
// rises (bitonic), which log2(M) half-cleaner stages sort. M is a power of
// two.
template <int M>
__device__ inline void merge_top(float (&val)[M], int (&idx)[M], const float (&pv)[M],
                                 const int (&pi)[M]) {
  static_assert((M & (M - 1)) == 0, "bitonic merge needs a power of two");
#pragma unroll
  for (int p = 0; p < M; ++p)
    if (ranks_before(pv[M - 1 - p], pi[M - 1 - p], val[p], idx[p])) {
      val[p] = pv[M - 1 - p];
      idx[p] = pi[M - 1 - p];
    }
#pragma unroll
  for (int st = M / 2; st > 0; st >>= 1)
#pragma unroll
    for (int p = 0; p < M; ++p)
      if ((p & st) == 0 && ranks_before(val[p + st], idx[p + st], val[p], idx[p])) {
        const float tv = val[p];
        const int ti = idx[p];
        val[p] = val[p + st];
        idx[p] = idx[p + st];
        val[p + st] = tv;
        idx[p + st] = ti;
      }
}

// k-th largest (1-based, k <= M) of the union of two lists sorted in
// descending order: max over i of min(A[i-1], B[k-i-1]), an entry past either
// end counting as +inf. -inf when the union holds fewer than k finite values.
template <int M>
__device__ inline float kth_of_union(const float (&A)[M], const float (&B)[M], int k) {
  float best = -INFINITY;
#pragma unroll
  for (int i = 0; i <= M; ++i) {
    if (i > k) break;
    const float a = i == 0 ? INFINITY : A[i - 1];
    const int jb = k - i;
    float b = INFINITY;
#pragma unroll
    for (int u = 0; u < M; ++u) b = (u == jb - 1) ? B[u] : b;
    if (jb > M) b = -INFINITY;
    best = fmaxf(best, fminf(a, b));
  }
  return best;
}

// Emits own block + selected ids ascending, -1 padded, into `out[0..slots)`.
template <int M>
__device__ inline void emit_sorted(int (&sel)[M], int n_sel, int own, bool cur,
                                   int32_t* __restrict__ out, int slots) {
  // Selected ids are distinct and all < own, so the own block goes last.
  // Sort the first n_sel ascending (small insertion sort, static indices).
#pragma unroll
  for (int a = 1; a < M; ++a) {
#pragma unroll
    for (int b = a; b > 0; --b) {
      if (b < n_sel && a < n_sel) {
        int x = sel[b - 1], y = sel[b];
        bool sw = x > y;
        sel[b - 1] = sw ? y : x;
        sel[b] = sw ? x : y;
      }
    }
  }
  int w = 0;
#pragma unroll
  for (int a = 0; a < M; ++a)
    if (a < n_sel && w < slots) out[w++] = sel[a];
  if (cur && w < slots) out[w++] = own;
  for (; w < slots; ++w) out[w] = -1;
}

// Head-major index of query (r, hq, token) in [R*Hq, S] buffers.
__device__ inline int64_t hm_query(bool packed, int64_t r, int64_t hq, int64_t h_q,
                                   int64_t S, int64_t tok_global, int64_t t_local) {
  return packed ? hq * S + tok_global : (r * h_q + hq) * S + t_local;
}

// ---------------------------------------------------------------------------
// Exact kernel: one thread per query (or per queued query).
// ---------------------------------------------------------------------------
template <typename T, int TMAX>
__global__ void __launch_bounds__(128)
gate_exact_kernel(const T* __restrict__ q, const T* __restrict__ kbar,
                  int32_t* __restrict__ out, const int32_t* __restrict__ cu,
                  int64_t S, int64_t rows_per_seq, int64_t h_q, int64_t h_kv,
                  int D, int64_t n_blocks, int bs, int take, int cur, int slots,
                  const int64_t* __restrict__ queue, const int* __restrict__ queue_len) {
  const int64_t group = h_q / h_kv;
  const bool packed = cu != nullptr;
  int64_t total;
  if (queue) total = *queue_len;
  else total = static_cast<int64_t>(gridDim.y) * rows_per_seq;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x * (queue ? gridDim.y : 1);
  int64_t first = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (queue) first += static_cast<int64_t>(blockIdx.y) * gridDim.x * blockDim.x;
  for (int64_t item = first; item < total; item += stride) {
    int64_t r, hq, t;
    if (queue) {
      int64_t code = queue[item];  // (r * h_q + hq) * rows_per_seq + t
      t = code % rows_per_seq;
      int64_t rh = code / rows_per_seq;
      r = rh / h_q;
      hq = rh % h_q;
    } else {
      int64_t rh = blockIdx.y;
      r = rh / h_q;
      hq = rh % h_q;
      t = item;
      if (t >= rows_per_seq) break;
    }
    SeqSpan sp = seq_span(cu, r, S);
    if (t >= sp.len) continue;
    const int64_t tok = sp.bos + t;
    const T* qrow = q + (tok * h_q + hq) * D;
    const T* kb = kbar + (r * h_kv + hq / group) * n_blocks * D;
    const int own = static_cast<int>(t / bs);
    float val[TMAX];
    int idx[TMAX];
#pragma unroll
    for (int p = 0; p < TMAX; ++p) { val[p] = -INFINITY; idx[p] = 0x7fffffff; }
    if (take > 0) {
      for (int j = 0; j < own; ++j) {
        float s = exact_score(qrow, kb + static_cast<int64_t>(j) * D, D);
        if (!(s > val[take - 1 < TMAX ? take - 1 : TMAX - 1])) {
          // cheap reject: cannot beat the current T-th best (ties lose to
          // the earlier, lower id)
          continue;
        }
        insert_exact<TMAX>(val, idx, s, j);
      }
    }
    int n_sel = 0;
#pragma unroll
    for (int p = 0; p < TMAX; ++p)
      if (p < take && val[p] > -INFINITY) n_sel = p + 1;
    int32_t* o = out + hm_query(packed, r, hq, h_q, S, tok, t) * slots;
    emit_sorted<TMAX>(idx, n_sel, own, cur != 0, o, slots);
  }
}

// ---------------------------------------------------------------------------
// Queue kernel: one workgroup of kQueueWaves waves per queued query. The
// lanes split the query's candidates, each keeps an exact top-T list, the
// lists merge with a butterfly over each wave, and wave 0 merges the waves'
// lists through LDS. Queries reach the queue when the MFMA kernel's evidence
// cannot settle them: a few dozen for random-walk or offset keys at 512K,
// by the thousands for constructed ties. With a few, the kernel is the
// gate's tail: one wave per query (the earlier layout) scanned a late
// query's ~4096 blocks alone for ~86 us. Each lane requests the rows of U
// blocks before it scores any of them (float64 products and sum, as
// exact_score), with the query row in registers.
// ---------------------------------------------------------------------------
constexpr int kQueueWaves = 8;

template <typename T, int TMAX, int D>
__global__ void __launch_bounds__(64 * kQueueWaves)
gate_queue_kernel(const T* __restrict__ q, const T* __restrict__ kbar,
                  int32_t* __restrict__ out, const int32_t* __restrict__ cu,
                  int64_t S, int64_t rows_per_seq, int64_t h_q, int64_t h_kv,
                  int64_t n_blocks, int bs, int take, int cur, int slots,
                  const int64_t* __restrict__ queue, const int* __restrict__ queue_len) {
  constexpr int U = 256 / D;  // rows in flight per lane
  constexpr int C = D / 8;     // 16-byte chunks per row
  constexpr int NL = 64 * kQueueWaves;  // lanes per query
  __shared__ float s_val[kQueueWaves][TMAX];
  __shared__ int s_idx[kQueueWaves][TMAX];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tid = threadIdx.x;
  const int64_t total = *queue_len;  // uniform: every wave runs the same items
  const bool packed = cu != nullptr;
  for (int64_t item = blockIdx.x; item < total; item += gridDim.x) {
    const int64_t code = queue[item];  // (r * h_q + hq) * rows_per_seq + t
    const int64_t t = code % rows_per_seq;
    const int64_t rh = code / rows_per_seq;
    const int64_t r = rh / h_q, hq = rh % h_q;
    const SeqSpan sp = seq_span(cu, r, S);
    const int64_t tok = sp.bos + t;
    const T* qrow = q + (tok * h_q + hq) * D;
    const T* kb = kbar + (r * h_kv + hq / (h_q / h_kv)) * n_blocks * D;
    const int own = static_cast<int>(t / bs);
    float val[TMAX];
    int idx[TMAX];
#pragma unroll
    for (int p = 0; p < TMAX; ++p) { val[p] = -INFINITY; idx[p] = 0x7fffffff; }
    if constexpr (Elem<T>::kCode == MOBA_FP16) {
      // fp16's software conversion needs the registers: one candidate at a
      // time per lane.
      for (int j = tid; j < own; j += NL) {
        const float sc = exact_score(qrow, kb + static_cast<int64_t>(j) * D, D);
        if (ranks_before(sc, j, val[take - 1], idx[take - 1])) insert_exact<TMAX>(val, idx, sc, j);
      }
    } else {
      uint4 qv[C];
#pragma unroll
      for (int c = 0; c < C; ++c) qv[c] = *reinterpret_cast<const uint4*>(qrow + 8 * c);
      for (int j0 = tid; j0 < own; j0 += U * NL) {
        uint4 kv[U][C];
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int j = j0 + u * NL;
          const T* krow = kb + static_cast<int64_t>(j < own ? j : 0) * D;
#pragma unroll
          for (int c = 0; c < C; ++c) kv[u][c] = *reinterpret_cast<const uint4*>(krow + 8 * c);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int j = j0 + u * NL;
          double acc = 0.0;
#pragma unroll
          for (int c = 0; c < C; ++c) {
            // Opaque to the compiler, so the row's float64 conversions stay
            // in the loop (hoisted, they would take 2 * D registers).
            uint4 qc = qv[c];
            asm volatile("" : "+v"(qc.x), "+v"(qc.y), "+v"(qc.z), "+v"(qc.w));
            const T* qe = reinterpret_cast<const T*>(&qc);
            const T* ke = reinterpret_cast<const T*>(&kv[u][c]);
#pragma unroll
            for (int i = 0; i < 8; ++i)
              acc += static_cast<double>(Elem<T>::load(qe, i)) * static_cast<double>(Elem<T>::load(ke, i));
          }
          const float sc = Elem<T>::round(static_cast<float>(acc));
          if (j < own && ranks_before(sc, j, val[take - 1], idx[take - 1]))
            insert_exact<TMAX>(val, idx, sc, j);
        }
      }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      float pv[TMAX];
      int pi[TMAX];
#pragma unroll
      for (int p = 0; p < TMAX; ++p) {
        pv[p] = __shfl_xor(val[p], off);
        pi[p] = __shfl_xor(idx[p], off);
      }
      merge_top<TMAX>(val, idx, pv, pi);
    }
    // Every lane of a wave holds the wave's list; wave 0 merges the others'.
    if (lane == 0) {
#pragma unroll
      for (int p = 0; p < TMAX; ++p) {
        s_val[wave][p] = val[p];
        s_idx[wave][p] = idx[p];
      }
    }
    __syncthreads();
    if (wave == 0) {
      for (int w = 1; w < kQueueWaves; ++w) {
        float pv[TMAX];
        int pi[TMAX];
#pragma unroll
        for (int p = 0; p < TMAX; ++p) {
          pv[p] = s_val[w][p];
          pi[p] = s_idx[w][p];
        }
        merge_top<TMAX>(val, idx, pv, pi);
      }
      if (lane == 0) {
        int n_sel = 0;
#pragma unroll
        for (int p = 0; p < TMAX; ++p)
          if (p < take && val[p] > -INFINITY) n_sel = p + 1;
        emit_sorted<TMAX>(idx, n_sel, own, cur != 0,
                          out + hm_query(packed, r, hq, h_q, S, tok, t) * slots, slots);
      }
    }
    __syncthreads();  // the lists of this item are read before the next is written
  }
}

// ---------------------------------------------------------------------------
// MFMA kernel (bf16 / fp16).
// ---------------------------------------------------------------------------
template <typename T> struct MfmaOps;
template <> struct MfmaOps<bf16_t> {
  typedef bf16x8_t vec;
  __device__ static floatx16_t mfma(vec a, vec b, floatx16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static constexpr float kMaxFinite = 3.0e38f;
  // Largest magnitude the MFMA may flush as a denormal input.
  static constexpr float kDenorm = 1.2e-38f;
};
template <> struct MfmaOps<f16_t> {
  typedef f16x8_t vec;
  __device__ static floatx16_t mfma(vec a, vec b, floatx16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static constexpr float kMaxFinite = 60000.f;  // beyond: fp16 rounds to inf
  static constexpr float kDenorm = 6.2e-5f;     // fp16 subnormals are below 2^-14
};

// The next value of T's format below v (v itself a finite value of it).
template <typename T> __device__ inline float key_below(float v);
template <> __device__ inline float key_below<bf16_t>(float v) {
  const uint16_t b = float_to_bf16(v);
  return bf16_to_float(v > 0.f ? b - 1 : (v < 0.f ? b + 1 : 0x8001));
}
template <> __device__ inline float key_below<f16_t>(float v) {
  const uint16_t b = float_to_f16(v);
  return f16_to_float(v > 0.f ? b - 1 : (v < 0.f ? b + 1 : 0x8001));
}

// Inserts (x, j) with the largest key k it can have into a list sorted by
// (key desc, id asc); the last entry falls off. The entry shifted down at
// each step is compared under the same order (ids break equal keys).
template <int M>
__device__ inline void insert_keyed(float (&key)[M], float (&val)[M], int (&idx)[M], float k,
                                    float x, int j) {
#pragma unroll
  for (int p = 0; p < M; ++p) {
    const bool gt = k > key[p] || (k == key[p] && j < idx[p]);
    const float nk = gt ? k : key[p];
    const float nv = gt ? x : val[p];
    const int ni = gt ? j : idx[p];
    k = gt ? key[p] : k;
    x = gt ? val[p] : x;
    j = gt ? idx[p] : j;
    key[p] = nk;
    val[p] = nv;
    idx[p] = ni;
  }
}

template <typename V>
__device__ inline V load_vec16(const void* p) {
  uint4 u = *reinterpret_cast<const uint4*>(p);
  return __builtin_bit_cast(V, u);
}

// +inf in a register the compiler cannot see through: a med3 against it
// stays one instruction (against the constant the compiler turns it into a
// max that canonicalises both operands first, three instructions).
__device__ inline float opaque_inf() {
  float inf = INFINITY;
  asm volatile("" : "+v"(inf));
  return inf;
}

// Inserts x into a list of values sorted descending; the smallest falls off.
// New entry p is the median of old entries p - 1, p and x; `inf` is +inf
// (from opaque_inf, made once outside the caller's loop).
template <int K>
__device__ inline void insert_value(float (&l)[K], float x, float inf) {
#pragma unroll
  for (int p = K - 1; p > 0; --p) l[p] = __builtin_amdgcn_fmed3f(l[p - 1], l[p], x);
  l[0] = __builtin_amdgcn_fmed3f(l[0], x, inf);  // max, without canonicalising
}

// One tile of 32 * WAVES queries of one (row, query head): the queries
// t0 .. t0 + 32 WAVES - 1 (first kernel, FB false), or entries e0 .. of a
// fallback list (FB true; `ent` is the list, n_ent its length).
// Low mantissa bits that are zero in every float holding a value of T.
template <typename T> __host__ __device__ constexpr int gate_key_bits() {
  return Elem<T>::kCode == MOBA_BF16 ? 16 : 13;
}
// Whether the group ids and LDS slots of every tile fit those bits: a tile
// ranks at most n_blocks blocks, in 32-block chunks of 16 / GB groups.
template <typename T, int K, int GB> static bool gate_keyed_fits(int64_t n_blocks) {
  const int64_t max_gid = (n_blocks + 31) / 32 * (16 / GB) - 1;
  int bits = 0;
  while ((int64_t{1} << bits) <= max_gid) ++bits;
  const int slot_bits = K == 8 ? 3 : (K == 16 ? 4 : 5);
  return slot_bits + bits <= gate_key_bits<T>();
}

// FBM: 0 for the first kernel; for the fallback kernel 1 (groups tracked
// by (key, id), as long as the group ids fit the keys' low bits), 2 (every
// score above the threshold appended to lists) or 3 (as 1, for a tile of at
// most 32 queries: every wave takes the same queries and a quarter of the
// chunks, and wave 0 merges the four lists and decides).
template <typename T, int D, int M, int K, int CAP, int WAVES, int GB, int FBM>
__device__ __forceinline__ void gate_tile(
    const T* __restrict__ q, const T* __restrict__ kbar, int32_t* __restrict__ out,
    const int32_t* __restrict__ cu, int64_t S, int64_t h_q, int64_t h_kv, int64_t n_blocks,
    int bs, int take, int cur, int slots, const float* __restrict__ kbar_norm,
    int64_t* __restrict__ queue, int* __restrict__ queue_len, int64_t rows_per_seq,
    int64_t rh, int64_t first, const FbLists& fb, const int2* __restrict__ ent, int n_ent) {
  using Ops = MfmaOps<T>;
  using V = typename Ops::vec;
  constexpr bool FB = FBM != 0;
  constexpr bool SPLIT = FBM == 3;
  constexpr int KSTEPS = D / 16;
  constexpr int KROW = D + 8;                      // staged kbar row stride (elements)
  constexpr int NT = WAVES * 64;
  constexpr int SR = 64;                           // kbar rows per LDS stage (two chunks)
  constexpr int KCH = (SR * D / 8 + NT - 1) / NT;  // 16-byte chunks per thread per stage
  // Per-wave LDS area. Pass 1 keeps there the four scores of each of the
  // lane's K tracked groups (one float4 per (slot, lane)); the fallback
  // pass 2 reuses the same bytes for its append buffers (CAP scores and CAP
  // ids per lane), and the decision for its uncertain ids.
  static_assert((K & (K - 1)) == 0 && K >= 8, "K is a power of two, at least 8");
  constexpr int SLOT_BITS = K == 8 ? 3 : (K == 16 ? 4 : 5);
  static_assert(GB == 4 || GB == 8, "groups of 4 or 8 blocks");
  constexpr int GPC = 16 / GB;                     // groups per lane and chunk
  constexpr int REC_BYTES = K * 64 * GB * 4;
  constexpr int BUF_BYTES = CAP * 64 * 6;
  constexpr int WAVE_BYTES = REC_BYTES > BUF_BYTES ? REC_BYTES : BUF_BYTES;
  __shared__ __attribute__((aligned(16))) unsigned char s_wave[WAVES][WAVE_BYTES];
  __shared__ __attribute__((aligned(16))) uint16_t s_kb[2][SR * KROW];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int half = lane >> 5;
  const int col = lane & 31;
  const bool packed = cu != nullptr;

  const int64_t r = rh / h_q;
  const int64_t hq = rh % h_q;
  const int64_t hk = hq / (h_q / h_kv);
  const SeqSpan sp = seq_span(cu, r, S);
  int64_t t;
  bool live;
  int own;
  int hz;  // blocks any query of the workgroup may rank: [0, hz)
  float theta_in = -INFINITY;
  if constexpr (!FB) {
    if (first >= sp.len) return;  // uniform over the workgroup
    t = first + wave * 32 + col;
    live = t < sp.len;
    own = live ? static_cast<int>(t / bs) : 0;
    const int64_t last_wg = (first + 32 * WAVES - 1 < sp.len ? first + 32 * WAVES - 1 : sp.len - 1);
    hz = static_cast<int>(last_wg / bs);
  } else {
    // Queries of one list in no particular order: the horizon is the
    // largest own block of the tile.
    __shared__ int s_hz;
    const int64_t e = first + (SPLIT ? 0 : wave * 32) + col;
    live = e < n_ent;
    const int2 en = live ? ent[e] : make_int2(0, 0);
    t = en.x;
    theta_in = __int_as_float(en.y);
    own = live ? static_cast<int>(t / bs) : 0;
    int m = own;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = max(m, __shfl_xor(m, off));
    if (tid == 0) s_hz = 0;
    __syncthreads();
    if (lane == 0) atomicMax(&s_hz, m);
    __syncthreads();
    hz = s_hz;
    if (tid == 0) atomicAdd(queue_len + 1, 1);  // fallback tiles, for tests
  }
  const T* kb = kbar + (r * h_kv + hk) * n_blocks * D;
  const int64_t tok = sp.bos + (live ? t : 0);
  const T* qrow = q + (tok * h_q + hq) * D;

  // B operand: this lane's query, features 16c + 8*half + [0, 8). The two
  // lanes of a query hold complementary halves of it.
  V bq[KSTEPS];
#pragma unroll
  for (int c = 0; c < KSTEPS; ++c) {
    if (live) bq[c] = load_vec16<V>(qrow + 16 * c + 8 * half);
    else bq[c] = V{};
  }
  // The query half again, from memory: keeps bq out of the registers live
  // across pass 1 where it is needed only later (rescoring, fallback pass).
  auto reload_q = [&](V (&dst)[KSTEPS]) {
    const T* qr = qrow;
    asm volatile("" : "+v"(qr));
#pragma unroll
    for (int c = 0; c < KSTEPS; ++c)
      dst[c] = live ? load_vec16<V>(qr + 16 * c + 8 * half) : V{};
  };
  // Error band of this query: E >= |approx - exact| for every candidate.
  float qn = 0.f;
#pragma unroll
  for (int c = 0; c < KSTEPS; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float x = static_cast<float>(bq[c][i]);
      qn += x * x;
    }
  qn += __shfl_xor(qn, 32);
  // Accumulation error, plus what flushing denormal operands could drop:
  // each flushed factor is below kDenorm, so the lost products sum to at
  // most kDenorm (sum |kbar_i| + sum |q_i|) <= kDenorm sqrt(D) (|kbar| + |q|).
  // The products of 16-bit inputs are exact in float32; the D of them reach
  // the result through at most D float32 additions, in any order, each
  // rounding by at most one ulp (2^-23 relative, truncation included) of a
  // partial sum no larger than sum |q_i kbar_i| <= |q| |kbar|. So
  // |approx - exact| <= D 2^-23 |q| |kbar|; E takes twice that.
  const float qnorm = sqrtf(qn) * 1.0001f;
  // Slack for the float sum of squares and sqrtf (a few ulp).
  const float knorm = kbar_norm[r * h_kv + hk] * 1.0001f + 1e-30f;
  // The last term covers float32 denormal products or partial sums the
  // matrix core may flush: at most 2^-126 each, D + 1 of them.
  const float E = qnorm * knorm * (D * 0x1p-22f) + Ops::kDenorm * sqrtf(D) * (qnorm + knorm) +
                  (D + 1) * 1.2e-38f;
  // E widened by the float32 rounding of a -+ E (2.4e-7 > 2^-22).
  auto widen = [&](float a) { return E * 1.001f + fabsf(a) * 2.4e-7f; };

  const int n_chunks = (take > 0 && hz > 0) ? (hz + 31) / 32 : 0;
  const int n_stages = (n_chunks + 1) / 2;
  // kbar rows are staged in LDS by the whole workgroup, 64 rows (two chunks
  // of 32) per stage. Rows past the horizon are clamped to a valid row;
  // their scores are masked (every such block is >= own for every query
  // here). Stage st waits in register slot st % 2 (loaded two stages ahead)
  // until it is stored to LDS buffer st % 2.
  u32x4 kr0[KCH], kr1[KCH];
  auto kload = [&](u32x4 (&r)[KCH], int st) {
#pragma unroll
    for (int u = 0; u < KCH; ++u) {
      const int i = tid + u * NT;
      if (i < SR * D / 8) {
        const int blk = min(st * SR + i / (D / 8), hz - 1);
        r[u] = *reinterpret_cast<const u32x4*>(kb + static_cast<int64_t>(blk) * D +
                                              (i % (D / 8)) * 8);
      }
    }
  };
  auto kstore = [&](const u32x4 (&r)[KCH], int buf) {
#pragma unroll
    for (int u = 0; u < KCH; ++u) {
      const int i = tid + u * NT;
      if (i < SR * D / 8)
        *reinterpret_cast<u32x4*>(&s_kb[buf][(i / (D / 8)) * KROW + (i % (D / 8)) * 8]) = r[u];
    }
  };

  // --- Pass 1: every chunk once. Each lane keeps the K largest maxima of
  // its 4-block groups, and the four scores of each kept group in LDS. The
  // take-th largest of the union of the two lanes' kept maxima is the
  // take-th best of a subset of the query's candidates, so it is <= L (the
  // take-th best of all of them); every candidate that can matter then has
  // a key >= R(that value - w) and a score >= theta. The kept groups then
  // hold every such candidate unless the largest group maximum that left
  // the list reaches theta (then the decision below counts it as a bound).
  // Lane 0 of the wave holds its smallest query, so its own block bounds
  // every lane's: chunks entirely below it need no causal mask.
  int own_min;
  if constexpr (!FB) {
    own_min = __builtin_amdgcn_readfirstlane(own);
  } else {
    int m = live ? own : 0x7fffffff;
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = min(m, __shfl_xor(m, off));
    own_min = m;
  }
  float theta = theta_in;
  auto stream_chunks = [&](auto&& body) {
    // step(st): score both chunks of stage st (two independent MFMA chains
    // over one A-operand buffer), move stage st + 1 from `next` into LDS,
    // and request stage st + 2 into the slot stage st came from (`freed`).
    auto step = [&](int st, const u32x4 (&next)[KCH], u32x4 (&freed)[KCH]) {
      if (st >= n_stages) return;
      const uint16_t* arow = &s_kb[st & 1][col * KROW + 8 * half];
      // All A operands of the stage are requested before the first MFMA.
      V ka[2][KSTEPS];
#pragma unroll
      for (int c = 0; c < KSTEPS; ++c) {
        ka[0][c] = load_vec16<V>(arow + 16 * c);
        ka[1][c] = load_vec16<V>(arow + 32 * KROW + 16 * c);
      }
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
      floatx16_t a0 = {}, a1 = {};
#pragma unroll
      for (int c = 0; c < KSTEPS; ++c) {
        a0 = Ops::mfma(ka[0][c], bq[c], a0);
        a1 = Ops::mfma(ka[1][c], bq[c], a1);
      }
      // a?[v] scores block 32 ch + 8(v/4) + 4 half + v%4
      const int c0 = 2 * st;
      body(c0, a0, c0 * 32 + 32 <= own_min);
      if (c0 + 1 < n_chunks) body(c0 + 1, a1, c0 * 32 + 64 <= own_min);
      if (st + 1 < n_stages) kstore(next, (st + 1) & 1);
      if (st + 2 < n_stages) kload(freed, st + 2);
      __syncthreads();
    };
    kload(kr0, 0);
    if (n_stages > 1) kload(kr1, 1);
    kstore(kr0, 0);
    __syncthreads();
    for (int st = 0; st < n_stages; st += 2) {
      step(st, kr1, kr0);
      step(st + 1, kr0, kr1);
    }
  };
  // SPLIT: wave w scores chunks w, w + WAVES, ... of the same queries, its
  // A operands loaded straight from kbar (no staging, no barriers), three
  // chunks in flight.
  auto split_stream = [&](auto&& body) {
    auto aload = [&](V (&dst)[KSTEPS], int ch) {
      const int blk = min(32 * ch + col, hz - 1);
      const T* row = kb + static_cast<int64_t>(blk) * D + 8 * half;
#pragma unroll
      for (int c = 0; c < KSTEPS; ++c) dst[c] = load_vec16<V>(row + 16 * c);
    };
    // step(c): score chunk c from `cur`, after requesting chunk c + 2 WAVES
    // into `freed` (the buffer chunk c - WAVES was scored from).
    // Inlined, so that the three buffers stay in registers.
    auto step = [&](int c, const V (&cur)[KSTEPS], V (&freed)[KSTEPS]) __attribute__((always_inline)) {
      if (c >= n_chunks) return;
      if (c + 2 * WAVES < n_chunks) aload(freed, c + 2 * WAVES);
      floatx16_t acc = {};
#pragma unroll
      for (int k = 0; k < KSTEPS; ++k) acc = Ops::mfma(cur[k], bq[k], acc);
      body(c, acc, c * 32 + 32 <= own_min);
    };
    V a0[KSTEPS], a1[KSTEPS], a2[KSTEPS];
    if (wave < n_chunks) aload(a0, wave);
    if (wave + WAVES < n_chunks) aload(a1, wave + WAVES);
    for (int c = wave; c < n_chunks; c += 3 * WAVES) {
      step(c, a0, a2);
      step(c + WAVES, a1, a0);
      step(c + 2 * WAVES, a2, a1);
    }
  };
  // Group keys. A group is four consecutive blocks of one lane (lane half h
  // holds the groups with (block >> 2) & 1 == h), numbered gid = block >> 3
  // within the lane. A key is the group's maximum score with its low
  // mantissa bits replaced by (gid << SLOT_BITS | slot): float order of the
  // keys is the order of the maxima up to that truncation, and the key
  // names both the group and the LDS slot holding its four scores.
  const int max_gid = n_chunks > 0 ? n_chunks * GPC - 1 : 0;
  const int gid_bits = max_gid > 0 ? 32 - __clz(max_gid) : 0;
  const uint32_t low_mask = (1u << (SLOT_BITS + gid_bits)) - 1u;
  // The key's value range: [lo, hi] holds the maximum it was made from.
  // Keys at or below -3e38 (masked groups, empty slots) mean "none".
  auto key_lo = [&](float k) {
    const uint32_t u = __float_as_uint(k);
    const float f = __uint_as_float((u >> 31) ? (u | low_mask) : (u & ~low_mask));
    return f <= -3.0e38f ? -INFINITY : f;
  };
  auto key_hi = [&](float k) {
    const uint32_t u = __float_as_uint(k);
    const float f = __uint_as_float((u >> 31) ? (u & ~low_mask) : (u | low_mask));
    return f <= -3.0e38f ? -INFINITY : f;
  };
  // [K][GB / 4][64] float4: a group's scores in order, four per float4.
  float4* srec = reinterpret_cast<float4*>(&s_wave[wave][0]) + lane;
  float gk[K];
  // Largest key that left the list (or never entered it): every group not
  // in the list has its maximum <= key_hi(ev).
  float ev = -INFINITY;
  // The fallback kernel ranks groups by (largest key any of their scores
  // can have, group id asc): the key R(max + w) as a float, whose low
  // mantissa bits (16 for bf16, 13 for fp16) are zero, carries in them the
  // group id (rising for negative keys, falling for positive ones, so that
  // a lower id ranks first either way) and the LDS slot. Float order is
  // then exactly that ranking. Where the ids may not fit
  // (gate_keyed_fits), the host launches FBM = 2, which appends scores.
  const bool keyed = (FBM == 1 || SPLIT) && SLOT_BITS + gid_bits <= gate_key_bits<T>();
  auto keyed_gid = [&](float k) {
    const uint32_t u = __float_as_uint(k);
    const int g = static_cast<int>((u & low_mask) >> SLOT_BITS);
    return (u >> 31) ? g : max_gid - g;
  };
  auto keyed_val = [&](float k) {
    const float f = __uint_as_float(__float_as_uint(k) & ~low_mask);
    return f <= -3.0e38f ? -INFINITY : f;
  };
  if ((!FB || keyed) && n_chunks > 0) {
    const float empty = -INFINITY;
#pragma unroll
    for (int p = 0; p < K; ++p) {
      gk[p] = __uint_as_float((0xff7fffffu & ~low_mask) | static_cast<uint32_t>(p));
#pragma unroll
      for (int h = 0; h < GB / 4; ++h)
        srec[(p * (GB / 4) + h) * 64] = make_float4(empty, empty, empty, empty);
    }
    // Element w of group gid scores block gid 2GB + 8 (w / 4) + 4 half + w % 4.
    const float pinf = opaque_inf();
    auto track = [&](const float (&x)[GB], int gid) {
      // Clamped to -FLT_MAX so that replacing low bits keeps it a number.
      float mx = -3.4028235e38f;
#pragma unroll
      for (int w = 0; w < GB; ++w) mx = fmaxf(mx, x[w]);
      const float old = gk[K - 1];
      const uint32_t slot = __float_as_uint(old) & (K - 1);
      float key;
      if constexpr (FB) {
        // + 0: a key of -0 ranks as +0 (they are equal keys). Clamped to
        // -+0x1.fep127, whose low 16 bits are zero, so that the low bits
        // keep it a number (a masked group: "none").
        const float kr = fminf(fmaxf(key_round<T>(mx + widen(mx)) + 0.f, -0x1.fep127f), 0x1.fep127f);
        const uint32_t g = kr < 0.f ? static_cast<uint32_t>(gid) : static_cast<uint32_t>(max_gid - gid);
        key = __uint_as_float(__float_as_uint(kr) | (g << SLOT_BITS) | slot);
      } else {
        const uint32_t low = slot | (static_cast<uint32_t>(gid) << SLOT_BITS);
        key = __uint_as_float((__float_as_uint(mx) & ~low_mask) | low);
      }
      ev = __builtin_amdgcn_fmed3f(ev, old, key);  // ev <= old always
      // The key enters the list iff it beats the last entry, whose slot
      // it takes over.
      if (key > old) {
#pragma unroll
        for (int h = 0; h < GB / 4; ++h)
          srec[(slot * (GB / 4) + h) * 64] =
              make_float4(x[4 * h], x[4 * h + 1], x[4 * h + 2], x[4 * h + 3]);
      }
      insert_value<K>(gk, key, pinf);
    };
    auto chunk = [&](int ch, const floatx16_t& acc, bool full) {
      if (full) {
#pragma unroll
        for (int g = 0; g < GPC; ++g) {
          float x[GB];
#pragma unroll
          for (int w = 0; w < GB; ++w) x[w] = acc[GB * g + w];
          track(x, ch * GPC + g);
        }
      } else {
#pragma unroll
        for (int g = 0; g < GPC; ++g) {
          const int gid = ch * GPC + g;
          float x[GB];
#pragma unroll
          for (int w = 0; w < GB; ++w)
            x[w] = gid * 2 * GB + 8 * (w >> 2) + 4 * half + (w & 3) < own ? acc[GB * g + w]
                                                                         : -INFINITY;
          track(x, gid);
        }
      }
    };
    if constexpr (SPLIT) {
      split_stream(chunk);
      // Wave 0 takes the K best groups of the four waves' lists by (key,
      // id), their records moved to its own slots 0 .. K - 1; every group
      // left out ranks at or below the largest key that left a list (ev).
      float* mk = reinterpret_cast<float*>(&s_kb[0][0]);  // [WAVES][K + 1][64]
      static_assert(WAVES * (K + 1) * 64 * 4 <= sizeof(s_kb), "merge area");
#pragma unroll
      for (int p = 0; p < K; ++p) mk[(wave * (K + 1) + p) * 64 + lane] = gk[p];
      mk[(wave * (K + 1) + K) * 64 + lane] = ev;
      __syncthreads();
      if (wave != 0) return;
      int src[K];  // record of each entry: wave * K + slot
#pragma unroll
      for (int p = 0; p < K; ++p) src[p] = static_cast<int>(__float_as_uint(gk[p]) & (K - 1));
      for (int w = 1; w < WAVES; ++w) {
        ev = fmaxf(ev, mk[(w * (K + 1) + K) * 64 + lane]);
#pragma unroll
        for (int p = 0; p < K; ++p) {
          float k = mk[(w * (K + 1) + p) * 64 + lane];
          int si = w * K + static_cast<int>(__float_as_uint(k) & (K - 1));
          ev = fmaxf(ev, fminf(gk[K - 1], k));  // what this insertion drops
#pragma unroll
          for (int u = 0; u < K; ++u) {
            const bool gt = k > gk[u];
            const float nk = gt ? k : gk[u];
            const int ns = gt ? si : src[u];
            k = gt ? gk[u] : k;
            si = gt ? src[u] : si;
            gk[u] = nk;
            src[u] = ns;
          }
        }
      }
      // (u32x4, not float4: an array of HIP's float4 struct stays in memory.)
      static_assert(GB == 4, "one 16-byte record per group");
      u32x4 rec[K];
      const u32x4* recs = reinterpret_cast<const u32x4*>(&s_wave[0][0]) + lane;
      constexpr int kWaveRecs = sizeof(s_wave[0]) / 16;
#pragma unroll
      for (int p = 0; p < K; ++p) rec[p] = recs[(src[p] / K) * kWaveRecs + (src[p] % K) * 64];
#pragma unroll
      for (int p = 0; p < K; ++p) {
        reinterpret_cast<u32x4*>(srec)[p * 64] = rec[p];
        gk[p] = __uint_as_float((__float_as_uint(gk[p]) & ~static_cast<uint32_t>(K - 1)) | p);
      }
    } else {
      stream_chunks(chunk);
    }
    if constexpr (!FB) {  // the fallback kernel keeps the first kernel's theta
    float lo[K], plo[K];
#pragma unroll
    for (int p = 0; p < K; ++p) {
      lo[p] = key_lo(gk[p]);
      plo[p] = __shfl_xor(lo[p], 32);
    }
    // The take-th largest of the union of the two lanes' group maxima (each
    // from a distinct block) is <= L, the take-th best score of the query.
    const float tau = kth_of_union<K>(lo, plo, take);
    // Keys of the take-th best and above are >= kt0 = R(tau - w); scores
    // below the midpoint between kt0 and the key under it (less a margin
    // of two widths) round below kt0 and cannot be needed.
    if (tau > -INFINITY) {
      const float kt0 = key_round<T>(tau - widen(tau));
      const float mid = 0.5f * (kt0 + key_below<T>(kt0));
      theta = nextafterf(mid - 2.f * widen(mid), -INFINITY);
    }
    }
  }
  // Collection threshold: a > thr0 is a >= theta.
  const float thr0 = theta > -INFINITY ? nextafterf(theta, -INFINITY) : -INFINITY;

  // Lists of the fallback pass: the lane's M best candidates by (largest
  // key the score can have, id asc), approximate scores beside them.
  float lk[M], lv[M];  // lk: fallback kernel only
  int li[M];
  auto clear_lists = [&]() {
#pragma unroll
    for (int p = 0; p < M; ++p) { lv[p] = -INFINITY; li[p] = 0x7fffffff; }
    if constexpr (FB) {
#pragma unroll
      for (int p = 0; p < M; ++p) lk[p] = -INFINITY;
    }
  };
  float rej_mine = -INFINITY;

  float* sv = reinterpret_cast<float*>(&s_wave[wave][0]) + lane;  // [CAP][64]
  uint16_t* si = reinterpret_cast<uint16_t*>(&s_wave[wave][CAP * 64 * 4]) + lane;

  // --- Merge the two half-lists of this query and decide. -----------------
  // A query's ranking key is its exact score rounded to float32 and then to
  // the storage dtype (ties broken by the lower id). Every approximate
  // score a carries |a - exact| <= E, so its key lies in
  // [R(a - w), R(a + w)] (R: that rounding, monotone; w: E widened by the
  // float32 rounding of a -+ E). Keys are coarse (one dtype ulp is far
  // wider than E), so most intervals are a single key: those candidates
  // are ranked as they are, and only the ones whose interval straddles a
  // rounding boundary are rescored exactly. Scores below theta have keys
  // below every selected key; what a full list left out ranks below its
  // last entry, so the result stands when each lane's last entry ranks at
  // or below the take-th selected (equal keys: ids asc). Many equal keys
  // at the boundary thus settle by id, as the oracle breaks the tie.
  constexpr int TS = M <= 12 ? 8 : 16;  // most past blocks one query selects
  float fv[TS];
  int fi[TS];
  uint32_t* su = reinterpret_cast<uint32_t*>(sv);
  // The fallback kernel's lists rank by (largest key, id), so equal keys at
  // the boundary settle by id.
  auto decide_keyed = [&]() -> bool {
    // Everything a lane's full list left out ranks below its last entry
    // (key rk, id rid) in (key desc, id asc) order: an entry that fell off
    // ranked below the entry then last, and a score that was never
    // appended could not reach a key above rk, with an id past the list's.
    const bool full = lk[M - 1] > -INFINITY;
    const float rk_m = full ? lk[M - 1] : -INFINITY;
    const int rid_m = full ? li[M - 1] : 0x7fffffff;
    const float rk_p = __shfl_xor(rk_m, 32);
    const int rid_p = __shfl_xor(rid_m, 32);
    float pk[M], pv[M];
    int pi[M];
#pragma unroll
    for (int p = 0; p < M; ++p) {
      pk[p] = __shfl_xor(lk[p], 32);
      pv[p] = __shfl_xor(lv[p], 32);
      pi[p] = __shfl_xor(li[p], 32);
    }
    // q or kbar carries inf / NaN, or a score could round to an infinite key.
    bool ok = !(take > 0) || (qnorm * knorm < Ops::kMaxFinite);
#pragma unroll
    for (int p = 0; p < TS; ++p) { fv[p] = -INFINITY; fi[p] = 0x7fffffff; }
    if (ok && take > 0 && live) {
      // Lk: the take-th largest lower key bound of the union; a candidate
      // whose largest key is below it ranks below `take` others.
      float kl[TS];
#pragma unroll
      for (int p = 0; p < TS; ++p) kl[p] = -INFINITY;
      auto lower = [&](float x) { return x > -INFINITY ? key_round<T>(x - widen(x)) : -INFINITY; };
      const float kinf = opaque_inf();
#pragma unroll
      for (int p = 0; p < M; ++p) insert_value<TS>(kl, lower(half == 0 ? lv[p] : pv[p]), kinf);
#pragma unroll
      for (int p = 0; p < M; ++p) insert_value<TS>(kl, lower(half == 0 ? pv[p] : lv[p]), kinf);
      float Lk = -INFINITY;
#pragma unroll
      for (int p = 0; p < TS; ++p) Lk = p == take - 1 ? kl[p] : Lk;
      // The candidates that can still rank in the top `take`, with exact keys,
      // in (key desc, id asc) order. Both lanes walk the union in the same
      // order (half 0's list first) and reach identical lists; uncertain ids
      // wait in the lane's candidate buffer and are rescored (float64) by the
      // two lanes together, each forming the partial dot over the features it
      // holds.
      int nu = 0;
      auto visit = [&](float x, int j) {
        if (!(x > -INFINITY)) return;
        const float w = widen(x);
        const float khi = key_round<T>(x + w);
        if (khi < Lk) return;
        const float klo = key_round<T>(x - w);
        if (klo == khi) {
          insert_exact<TS>(fv, fi, klo, j);
        } else {
          if (nu < CAP) su[nu * 64] = static_cast<uint32_t>(j);
          ++nu;
        }
      };
#pragma unroll
      for (int p = 0; p < M; ++p) visit(half == 0 ? lv[p] : pv[p], half == 0 ? li[p] : pi[p]);
#pragma unroll
      for (int p = 0; p < M; ++p) visit(half == 0 ? pv[p] : lv[p], half == 0 ? pi[p] : li[p]);
      if (nu > CAP) ok = false;  // more straddling candidates than the buffer holds
      constexpr int R = 2;
      V qv[KSTEPS];
      if (nu > 0) reload_q(qv);
#pragma unroll 1
      for (int u0 = 0; ok && u0 < nu; u0 += R) {
        int jr[R];
        V kv[R][KSTEPS];
#pragma unroll
        for (int r = 0; r < R; ++r) {
          jr[r] = u0 + r < nu ? static_cast<int>(su[(u0 + r) * 64]) : 0;
          jr[r] = jr[r] < hz ? jr[r] : 0;  // ids come from this lane's lists; a guard
          const T* krow = kb + static_cast<int64_t>(jr[r]) * D + 8 * half;
#pragma unroll
          for (int c = 0; c < KSTEPS; ++c) kv[r][c] = load_vec16<V>(krow + 16 * c);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
          double part = 0.0;
#pragma unroll
          for (int c = 0; c < KSTEPS; ++c)
#pragma unroll
            for (int i = 0; i < 8; ++i)
              part += static_cast<double>(static_cast<float>(qv[c][i])) *
                      static_cast<double>(static_cast<float>(kv[r][c][i]));
          part += __shfl_xor(part, 32);
          const float sc = Elem<T>::round(static_cast<float>(part));
          if (u0 + r < nu && sc > -INFINITY) insert_exact<TS>(fv, fi, sc, jr[r]);
        }
      }
      float kt = -INFINITY;
      int it = 0x7fffffff;
#pragma unroll
      for (int p = 0; p < TS; ++p) {
        kt = p == take - 1 ? fv[p] : kt;
        it = p == take - 1 ? fi[p] : it;
      }
      // Scores below theta have keys below every selected key.
      if (theta > -INFINITY && !(kt > key_round<T>(theta + widen(theta)))) ok = false;
      // What the lists left out must rank below the take-th selected.
      if (rk_m > kt || (rk_m == kt && rid_m < it)) ok = false;
      if (rk_p > kt || (rk_p == kt && rid_p < it)) ok = false;
    }
    return ok;
  };

  // --- Decide from the tracked groups. ------------------------------------
  // Candidates: the scores >= theta of every tracked group whose maximum
  // may reach theta. Left out: scores below theta, and the groups that
  // left the list or never entered it (maxima <= key_hi(ev)). Each lane
  // ranks its own candidates by exact key where the key interval is one
  // key, the two lanes' lists are merged, and candidates whose interval
  // straddles a rounding boundary are rescored exactly by both lanes (each
  // forms the float64 partial dot over its feature half) and inserted by
  // both, so the pair ends with identical lists.
  bool ok = !(take > 0) || (qnorm * knorm < Ops::kMaxFinite);
#pragma unroll
  for (int p = 0; p < TS; ++p) { fv[p] = -INFINITY; fi[p] = 0x7fffffff; }
  // Lower key bounds of every candidate (the exact key where known), the
  // TS largest, descending.
  float kl[TS];
#pragma unroll
  for (int p = 0; p < TS; ++p) kl[p] = -INFINITY;
  // The lane's candidates are first compacted into the kbar staging area
  // (idle after pass 1; every wave is past its last barrier), C per lane,
  // plus one entry that takes the writes of non-candidates once C are held;
  // then only those are ranked. An entry is the score with its low IB bits
  // replaced by its place among the kept groups' scores (p * GB + w), from
  // which the block id follows; the decision widens its error band by that
  // truncation (less than 2^(IB - 23) |score|).
  constexpr int IB = SLOT_BITS + (GB == 4 ? 2 : 3);
  constexpr uint32_t IMASK = (1u << IB) - 1u;
  constexpr int CB = (2 * SR * KROW * 2) / (WAVES * 64 * 4) - 1;
  constexpr int C = CB < 24 ? CB : 24;
  static_assert(C >= 4, "candidate buffer");
  float* cbuf = reinterpret_cast<float*>(&s_kb[0][0]) + wave * (C + 1) * 64 + lane;
  // The kept groups' keys, stored over the records once these are compacted.
  float* gks = reinterpret_cast<float*>(&s_wave[wave][0]) + lane;
  uint32_t* su_c = reinterpret_cast<uint32_t*>(cbuf);
  auto widen_c = [&](float a) { return widen(a) + fabsf(a) * ldexpf(1.f, IB - 22); };
  int cn = 0;
  // Largest candidate score that found the buffer full (groups come in
  // key order, so those are from the lane's lowest-ranked groups): a bound
  // like key_hi(ev) on what the lists leave out.
  float drop_max = -INFINITY;
  int ns = 0;  // straddling candidates held
  // Candidate e: its (truncated) score, block id and key interval.
  auto cand = [&](int e, float& x, int& jx, float& klo, float& khi) {
    x = cbuf[e * 64];
    const uint32_t ix = __float_as_uint(x) & IMASK;
    // Block id from the kept group's key, read back from LDS (one read in
    // place of a select over the K registers).
    const uint32_t gu = __float_as_uint(gks[((ix >> 2) / (GB / 4)) * 64]);
    const int hh = static_cast<int>(ix >> 2) % (GB / 4);
    const int gx = FB ? keyed_gid(__uint_as_float(gu)) : static_cast<int>((gu & low_mask) >> SLOT_BITS);
    jx = gx * 2 * GB + 8 * hh + 4 * half + static_cast<int>(ix & 3);
    const float wd = widen_c(x);
    klo = key_round<T>(x - wd);
    khi = key_round<T>(x + wd);
  };
  if ((!FB || keyed) && n_chunks > 0 && live && take > 0) {
#pragma unroll
    for (int p = 0; p < K; ++p) {
      // Keyed: every group in the list (its scores are filtered below).
      if (FB ? keyed_val(gk[p]) > -INFINITY : key_hi(gk[p]) >= theta) {
        const uint32_t u = __float_as_uint(gk[p]);
#pragma unroll
        for (int h = 0; h < GB / 4; ++h) {
          const float4 r4 = srec[((u & (K - 1)) * (GB / 4) + h) * 64];
          const float x[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            // Written at the next free entry; only a candidate advances it.
            cbuf[min(cn, C) * 64] = __uint_as_float(
                (__float_as_uint(x[w]) & ~IMASK) | static_cast<uint32_t>((p * (GB / 4) + h) * 4 + w));
            drop_max = fmaxf(drop_max, (x[w] > thr0 && cn >= C) ? x[w] : -INFINITY);
            cn += x[w] > thr0 ? 1 : 0;
          }
        }
      }
    }
#pragma unroll
    for (int p = 0; p < K; ++p) gks[p * 64] = gk[p];
    // Straddlers move to the front of the buffer (in place: the write
    // index never passes the read index); ns of them.
    const int ce = min(cn, C);
    const float kinf = opaque_inf();
    for (int e = 0; e < ce; ++e) {
      float x, klo, khi;
      int jx;
      cand(e, x, jx, klo, khi);
      insert_value<TS>(kl, klo, kinf);
      if (klo == khi) {
        insert_exact<TS>(fv, fi, klo, jx);
      } else {
        cbuf[ns * 64] = x;
        ++ns;
      }
    }
    rej_mine = FB ? drop_max : fmaxf(key_hi(ev), drop_max);
  }
  if (!FB || keyed) {
    float pv[TS];
    int pi[TS];
#pragma unroll
    for (int p = 0; p < TS; ++p) {
      pv[p] = __shfl_xor(fv[p], 32);
      pi[p] = __shfl_xor(fi[p], 32);
    }
    merge_top<TS>(fv, fi, pv, pi);
    // kappa: the take-th largest lower key bound of all candidates of the
    // query. A straddler (key interval over a rounding boundary) whose
    // largest possible key is below kappa ranks below `take` other
    // candidates and is left out; the others are rescored. The pair walks
    // both lanes' straddlers in step; a step where no lane of the wave
    // holds one that reaches kappa costs no loads.
    float pkl[TS];
#pragma unroll
    for (int p = 0; p < TS; ++p) pkl[p] = __shfl_xor(kl[p], 32);
    const float kappa = take > 0 ? kth_of_union<TS>(kl, pkl, take) : -INFINITY;
    // The straddlers that reach kappa, as block ids at the front of the
    // buffer (in place: entry nr is written after entry e >= nr is read).
    int nr = 0;
    for (int e = 0; e < ns; ++e) {
      float x, klo, khi;
      int jx;
      cand(e, x, jx, klo, khi);
      if (!(khi < kappa)) {
        su_c[nr * 64] = static_cast<uint32_t>(jx);
        ++nr;
      }
    }
    const int nr_pair = max(nr, __shfl_xor(nr, 32));
    V qv[KSTEPS];
    if (__any(ok && nr_pair > 0)) reload_q(qv);
#pragma unroll 1
    for (int e = 0; ok && e < nr_pair; ++e) {
      const int jm = e < nr ? static_cast<int>(su_c[e * 64]) : -1;
      const int jp = __shfl_xor(jm, 32);
      V kv[2][KSTEPS];
      const int j2[2] = {jm, jp};
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const int jr = (j2[r] >= 0 && j2[r] < hz) ? j2[r] : 0;  // a guard
        const T* krow = kb + static_cast<int64_t>(jr) * D + 8 * half;
#pragma unroll
        for (int c = 0; c < KSTEPS; ++c) kv[r][c] = load_vec16<V>(krow + 16 * c);
      }
      double part[2] = {0.0, 0.0};
#pragma unroll
      for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < KSTEPS; ++c)
#pragma unroll
          for (int i = 0; i < 8; ++i)
            part[r] += static_cast<double>(static_cast<float>(qv[c][i])) *
                       static_cast<double>(static_cast<float>(kv[r][c][i]));
      // Mine: my half plus the partner's half of my id (its second part).
      const double tm = part[0] + __shfl_xor(part[1], 32);
      const double tp = __shfl_xor(tm, 32);
      const float sm = Elem<T>::round(static_cast<float>(tm));
      const float sp = Elem<T>::round(static_cast<float>(tp));
      if (jm >= 0 && sm > -INFINITY) insert_exact<TS>(fv, fi, sm, jm);
      if (jp >= 0 && sp > -INFINITY) insert_exact<TS>(fv, fi, sp, jp);
    }
    const float rej = fmaxf(rej_mine, __shfl_xor(rej_mine, 32));
    const float U = fmaxf(rej, theta);
    if (!FB && ok && take > 0 && live && U > -INFINITY) {
      const float Uk = key_round<T>(U + widen(U));
      float kt = -INFINITY;
#pragma unroll
      for (int p = 0; p < TS; ++p) kt = p == take - 1 ? fv[p] : kt;
      if (!(kt > Uk)) ok = false;
    }
    if (FB && ok && take > 0 && live) {
      // Scores below theta and candidates that found the buffer full have
      // keys at most R(U + w(U)). A group that left a lane's list ranks at
      // or below that lane's ev by (key, group id): its scores' keys are at
      // most ev's key, and where equal to it, its blocks have ids at or
      // above ev's group's lowest block.
      float kt = -INFINITY;
      int it = 0x7fffffff;
#pragma unroll
      for (int p = 0; p < TS; ++p) {
        kt = p == take - 1 ? fv[p] : kt;
        it = p == take - 1 ? fi[p] : it;
      }
      if (U > -INFINITY && !(kt > key_round<T>(U + widen(U)))) ok = false;
      const float evk = keyed_val(ev);
      const int ev_lo = evk > -INFINITY ? keyed_gid(ev) * 2 * GB + 4 * half : 0x7fffffff;
      const bool mine = !(evk > kt) && !(evk == kt && ev_lo <= it);
      // Both lanes of the pair take part in the shuffle (no short circuit).
      const bool partner = __shfl_xor(mine ? 1 : 0, 32) != 0;
      if (!(mine && partner)) ok = false;
    }
  }

  // --- Appending fallback (FBM 2: group ids too wide for keyed groups):
  // stream every chunk again. Each score above the lane's threshold (rare:
  // theta sits about one key below L) is appended, with its block id, to
  // the lane's LDS buffer; a buffer that may overflow on the next chunk is
  // folded into the lane's list of its M best by (largest key, id), and the
  // threshold rises to the last entry's score.
  if ((FBM == 1 || SPLIT) && !keyed) ok = false;  // not launched so: a guard
  if (FBM == 2 && n_chunks > 0) {
    clear_lists();
    float thr = thr0;
    int cnt = 0;
    auto fold = [&]() {
      for (int e = 0; e < cnt; ++e) {
        const float x = sv[e * 64];
        insert_keyed<M>(lk, lv, li, key_round<T>(x + widen(x)), x, si[e * 64]);
      }
      cnt = 0;
      // A full list takes a later score only if it can beat the last entry.
      // By (key, id): x + w(x) and the rounding rise with x, so x <= the
      // last entry's score cannot reach a larger key, and a later id loses
      // a tie.
      if (lv[M - 1] > -INFINITY) thr = fmaxf(thr0, lv[M - 1]);
    };
    // Scores go in groups of four consecutive blocks. A group is skipped
    // when no lane's group maximum beats its threshold (one wave-wide
    // ballot); otherwise each score is written at the lane's next free entry
    // and only a score that beats the threshold advances it (no per-score
    // branch). The fold below keeps 16 free entries for every chunk.
    // The four compares go straight to wave masks; a lane almost never
    // holds two scores of one group above its threshold, so when no lane
    // does (scalar test on the masks) each lane appends its one hit, if
    // any, as a single entry.
    auto append4 = [&](const float (&x)[4], uint32_t id0) {
      const bool h0 = x[0] > thr, h1 = x[1] > thr, h2 = x[2] > thr, h3 = x[3] > thr;
      const uint64_t b0 = __ballot(h0), b1 = __ballot(h1), b2 = __ballot(h2), b3 = __ballot(h3);
      if ((b0 | b1 | b2 | b3) == 0) return;
      if (((b0 & (b1 | b2 | b3)) | (b1 & (b2 | b3)) | (b2 & b3)) == 0) {
        float v = h1 ? x[1] : x[0];
        v = h2 ? x[2] : v;
        v = h3 ? x[3] : v;
        uint32_t w = h1 ? 1u : 0u;
        w = h2 ? 2u : w;
        w = h3 ? 3u : w;
        sv[cnt * 64] = v;
        si[cnt * 64] = static_cast<uint16_t>(id0 + w);
        cnt += (h0 || h1 || h2 || h3) ? 1 : 0;
      } else {
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          sv[cnt * 64] = x[w];
          si[cnt * 64] = static_cast<uint16_t>(id0 + w);
          cnt += x[w] > thr ? 1 : 0;
        }
      }
    };
    stream_chunks([&](int ch, const floatx16_t& acc, bool full) {
      const uint32_t base = static_cast<uint32_t>(ch * 32 + 4 * half);
      if (full) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float x[4] = {acc[4 * g], acc[4 * g + 1], acc[4 * g + 2], acc[4 * g + 3]};
          append4(x, base + 8 * g);
        }
      } else {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const uint32_t id0 = base + 8 * g;
          float x[4];
#pragma unroll
          for (int w = 0; w < 4; ++w)
            x[w] = static_cast<int>(id0 + w) < own ? acc[4 * g + w] : -INFINITY;
          append4(x, id0);
        }
      }
      if (__any(cnt > CAP - 16)) fold();
    });
    fold();
    ok = decide_keyed();
  }

  if (!live || half != 0) return;
  const int64_t qid = hm_query(packed, r, hq, h_q, S, tok, t);
  if (!ok) {
    if (!FB && n_chunks > 0) {
      // The fallback kernel streams again for the queries that need it.
      // The lanes here that share the first one's list take their places
      // with one atomic (the order within a list does not matter).
      const int64_t li = rh * kFbBuckets + t / fb.cap;
      const uint64_t act = __ballot(1);
      const int lead = __builtin_ffsll(static_cast<long long>(act)) - 1;
      const bool same = li == __shfl(li, lead);
      const uint64_t ms = __ballot(same);
      int e;
      if (same) {
        int base = 0;
        if (lane == lead) base = atomicAdd(fb.count + li, __popcll(ms));
        e = __shfl(base, lead) + __popcll(ms & ((1ull << lane) - 1));
      } else {
        e = atomicAdd(fb.count + li, 1);
      }
      fb.list[li * fb.cap + e] = make_int2(static_cast<int>(t), __float_as_int(theta));
    } else {
      const int slot = atomicAdd(queue_len, 1);
      queue[slot] = (r * h_q + hq) * rows_per_seq + t;
    }
    return;
  }
  int n_sel = 0;
  int sel[TS];
#pragma unroll
  for (int p = 0; p < TS; ++p) {
    const bool in = p < take && fv[p] > -INFINITY;
    sel[p] = in ? fi[p] : 0x7fffffff;
    n_sel += in ? 1 : 0;
  }
  emit_sorted<TS>(sel, n_sel, own, cur != 0, out + qid * slots, slots);
}

// First kernel: one tile per workgroup, tiles numbered from the end so the
// longest ones start first.
template <typename T, int D, int M, int K, int CAP, int WAVES, int GB>
__global__ void __launch_bounds__(WAVES * 64, M <= 12 ? (D == 64 ? 3 : 2) : 1)
gate_mfma_kernel(const T* __restrict__ q, const T* __restrict__ kbar,
                 int32_t* __restrict__ out, const int32_t* __restrict__ cu,
                 int64_t S, int64_t h_q, int64_t h_kv, int64_t n_blocks, int bs,
                 int take, int cur, int slots, const float* __restrict__ kbar_norm,
                 int64_t* __restrict__ queue, int* __restrict__ queue_len,
                 int64_t rows_per_seq, FbLists fb) {
  const int64_t n_tiles = (rows_per_seq + 32 * WAVES - 1) / (32 * WAVES);
  const int64_t tile = n_tiles - 1 - blockIdx.x;
  gate_tile<T, D, M, K, CAP, WAVES, GB, 0>(q, kbar, out, cu, S, h_q, h_kv, n_blocks, bs,
                                               take, cur, slots, kbar_norm, queue, queue_len,
                                               rows_per_seq, blockIdx.y, tile * 32 * WAVES, fb,
                                               nullptr, 0);
}

// Fallback kernel: the unsettled queries of one (row, query head, position
// bucket) list per grid row, 32 * WAVES per tile, the workgroups of a row
// striding over its tiles. The work is proportional to the unsettled
// queries, not to the tiles that hold one.
template <typename T, int D, int M, int K, int CAP, int WAVES, int GB, int FBM>
__global__ void __launch_bounds__(WAVES * 64, M <= 12 ? (D == 64 ? 3 : 2) : 1)
gate_fallback_kernel(const T* __restrict__ q, const T* __restrict__ kbar,
                     int32_t* __restrict__ out, const int32_t* __restrict__ cu,
                     int64_t S, int64_t h_q, int64_t h_kv, int64_t n_blocks, int bs,
                     int take, int cur, int slots, const float* __restrict__ kbar_norm,
                     int64_t* __restrict__ queue, int* __restrict__ queue_len,
                     int64_t rows_per_seq, FbLists fb, int split_tail) {
  // Grid rows run the last position bucket (the longest streams) of every
  // (row, query head) first, down to bucket 0, so the long tiles start first.
  const int64_t n_rh = gridDim.y / kFbBuckets;
  const int64_t li = (blockIdx.y % n_rh) * kFbBuckets + (kFbBuckets - 1 - blockIdx.y / n_rh);
  const int n = fb.count[li];
  const int2* ent = fb.list + li * fb.cap;
  // A last tile of at most 32 queries goes to the split kernel (FBM 3), when
  // it runs: its four waves share the chunks instead of one wave holding
  // every query.
  constexpr int TQ = 32 * WAVES;
  const int tail = n % TQ;
  const bool split = split_tail && tail > 0 && tail <= 32;
  if constexpr (FBM == 3) {
    if (!split || blockIdx.x != 0) return;  // uniform
    gate_tile<T, D, M, K, CAP, WAVES, GB, FBM>(q, kbar, out, cu, S, h_q, h_kv, n_blocks, bs,
                                                take, cur, slots, kbar_norm, queue, queue_len,
                                                rows_per_seq, li / kFbBuckets, n - tail, fb, ent,
                                                n);
    return;
  }
  const int n_full = split ? n - tail : n;
  for (int64_t e0 = static_cast<int64_t>(blockIdx.x) * TQ; e0 < n_full;
       e0 += static_cast<int64_t>(gridDim.x) * TQ) {
    __syncthreads();  // the previous tile's LDS reads are done
    gate_tile<T, D, M, K, CAP, WAVES, GB, FBM>(q, kbar, out, cu, S, h_q, h_kv, n_blocks, bs,
                                                take, cur, slots, kbar_norm, queue, queue_len,
                                                rows_per_seq, li / kFbBuckets, e0, fb, ent, n);
  }
}

// ---------------------------------------------------------------------------
// Hierarchical refinement (opt-in): one wave per query. The candidates are
// the strictly-past blocks inside the super-blocks the super-block gate
// opened for the query (`sup`: ascending super-block ids, -1 padded, the
// query's own super-block among them); each lane scores up to LMAX of them
// exactly, keeps them sorted by (score desc, id asc), and `take` rounds of a
// wave-wide arg-max pick the best. Scores follow the gate's definition:
// the exact dot product rounded to float32 and to the input dtype.
// ---------------------------------------------------------------------------
template <typename T, int LMAX, int TMAX>
__global__ void __launch_bounds__(256)
gate_refine_kernel(const T* __restrict__ q, const T* __restrict__ kbar,
                   const int32_t* __restrict__ sup, int32_t* __restrict__ out,
                   int64_t S, int64_t h_q, int64_t h_kv, int D, int64_t n_blocks, int bs,
                   int group, int sup_slots, int take, int cur, int slots) {
  const int lane = threadIdx.x & 63;
  const int64_t rh = blockIdx.y;
  const int64_t r = rh / h_q, hq = rh % h_q;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= S) return;  // uniform over the wave
  const int own = static_cast<int>(t / bs);
  const T* qrow = q + ((r * S + t) * h_q + hq) * D;
  const T* kb = kbar + (r * h_kv + hq / (h_q / h_kv)) * n_blocks * D;
  const int32_t* sp = sup + (rh * S + t) * sup_slots;
  float val[LMAX];
  int idx[LMAX];
#pragma unroll
  for (int p = 0; p < LMAX; ++p) { val[p] = -INFINITY; idx[p] = 0x7fffffff; }
  const int n_cand = sup_slots * group;
#pragma unroll
  for (int u = 0; u < LMAX; ++u) {
    const int c = lane + 64 * u;
    if (c >= n_cand) break;
    const int sb = sp[c / group];
    if (sb < 0 || sb > (n_blocks - 1) / group) continue;  // no block (and no overflow)
    const int j = sb * group + c % group;
    if (j >= own || j >= n_blocks) continue;
    insert_exact<LMAX>(val, idx, exact_score(qrow, kb + static_cast<int64_t>(j) * D, D), j);
  }
  int sel[TMAX];
  int n_sel = 0;
  for (int round = 0; round < take; ++round) {
    // Wave-wide best of the lanes' heads under (score desc, id asc).
    float bv = val[0];
    int bi = idx[0];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(bv, off);
      const int oi = __shfl_xor(bi, off);
      if (ranks_before(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (!(bv > -INFINITY)) break;  // no candidate left (uniform)
    if (idx[0] == bi) {            // the owner drops its head
#pragma unroll
      for (int p = 0; p + 1 < LMAX; ++p) { val[p] = val[p + 1]; idx[p] = idx[p + 1]; }
      val[LMAX - 1] = -INFINITY;
      idx[LMAX - 1] = 0x7fffffff;
    }
#pragma unroll
    for (int p = 0; p < TMAX; ++p) if (p == n_sel) sel[p] = bi;
    ++n_sel;
  }
  if (lane != 0) return;
#pragma unroll
  for (int p = 0; p < TMAX; ++p) if (p >= n_sel) sel[p] = 0x7fffffff;
  emit_sorted<TMAX>(sel, n_sel, own, cur != 0, out + (rh * S + t) * slots, slots);
}

// ---------------------------------------------------------------------------
// Host launchers.
// ---------------------------------------------------------------------------
template <typename T, int TMAX>
static int launch_exact(const void* q, const void* kbar, int32_t* out,
                        const int32_t* cu, const Geometry& g, int take, int cur,
                        const int64_t* queue, const int* queue_len, hipStream_t st) {
  if (queue) {
    dim3 grid(512, 1);
    hipLaunchKernelGGL((gate_exact_kernel<T, TMAX>), grid, dim3(128), 0, st,
                       static_cast<const T*>(q), static_cast<const T*>(kbar), out, cu,
                       g.seq_len, g.rows_per_seq, g.h_q, g.h_kv,
                       static_cast<int>(g.head_dim), g.n_blocks,
                       static_cast<int>(g.block_size), take, cur,
                       static_cast<int>(g.slots), queue, queue_len);
  } else {
    dim3 grid(static_cast<unsigned>(cdiv(g.rows_per_seq, 128)),
              static_cast<unsigned>(g.rows * g.h_q));
    hipLaunchKernelGGL((gate_exact_kernel<T, TMAX>), grid, dim3(128), 0, st,
                       static_cast<const T*>(q), static_cast<const T*>(kbar), out, cu,
                       g.seq_len, g.rows_per_seq, g.h_q, g.h_kv,
                       static_cast<int>(g.head_dim), g.n_blocks,
                       static_cast<int>(g.block_size), take, cur,
                       static_cast<int>(g.slots), nullptr, nullptr);
  }
  return check_launch("moba_gate (exact)");
}

template <typename T>
static int dispatch_exact(const void* q, const void* kbar, int32_t* out,
                          const int32_t* cu, const Geometry& g, int take, int cur,
                          const int64_t* queue, const int* queue_len, hipStream_t st) {
  if (take <= 8) return launch_exact<T, 8>(q, kbar, out, cu, g, take, cur, queue, queue_len, st);
  if (take <= 16) return launch_exact<T, 16>(q, kbar, out, cu, g, take, cur, queue, queue_len, st);
  if (take <= 32) return launch_exact<T, 32>(q, kbar, out, cu, g, take, cur, queue, queue_len, st);
  if (take <= 64) return launch_exact<T, 64>(q, kbar, out, cu, g, take, cur, queue, queue_len, st);
  if (take <= 128) return launch_exact<T, 128>(q, kbar, out, cu, g, take, cur, queue, queue_len, st);
  return fail(MOBA_ERR_UNSUPPORTED, "gate supports at most 128 past blocks per query");
}

template <typename T, int D, int M>
static int launch_mfma(const void* q, const void* kbar, int32_t* out, const int32_t* cu,
                       const Geometry& g, int take, int cur, const GateWs& ws,
                       hipStream_t st) {
  // Groups of 4 blocks, 4 waves (3 workgroups per CU at head_dim 64).
  // Groups of 8 at 8 waves per workgroup (2 per SIMD, the records need
  // twice the LDS) ran pass 1 no faster and the decision slower.
  constexpr int GB = 4;
  constexpr int WAVES = 4;
  // Per-lane candidate buffer: one chunk's 16 scores beyond the fold
  // trigger (cnt > CAP - 16); also holds the uncertain ids of the decision.
  constexpr int CAP = M + 8;
  // Groups tracked per lane (2K >= take). With 8, a query on i.i.d. keys
  // finds its candidates outside the kept groups about once in 4e4.
  constexpr int K = M <= 12 ? 8 : 16;
  const FbLists fb{ws.fb_list, ws.fb_count, ws.fb_cap};
  dim3 grid(static_cast<unsigned>(cdiv(g.rows_per_seq, 32 * WAVES)),
            static_cast<unsigned>(g.rows * g.h_q));
  hipLaunchKernelGGL((gate_mfma_kernel<T, D, M, K, CAP, WAVES, GB>), grid, dim3(64 * WAVES), 0, st,
                     static_cast<const T*>(q), static_cast<const T*>(kbar), out, cu,
                     g.seq_len, g.h_q, g.h_kv, g.n_blocks, static_cast<int>(g.block_size),
                     take, cur, static_cast<int>(g.slots), ws.kbar_norm, ws.queue,
                     ws.counter, g.rows_per_seq, fb);
  int rc = check_launch("moba_gate (mfma)");
  if (rc) return rc;
  // Up to 32 workgroups per list, each striding over the list's tiles; a
  // workgroup past its list's length exits at once.
  const int64_t per_list = cdiv(ws.fb_cap, 32 * WAVES) < 32 ? cdiv(ws.fb_cap, 32 * WAVES) : 32;
  dim3 fgrid(static_cast<unsigned>(per_list), static_cast<unsigned>(g.rows * g.h_q * kFbBuckets));
  // Keyed groups: lists' last tiles of at most 32 queries (all of them on
  // i.i.d. keys, where a few queries per list are unsettled) go to the
  // split kernel, one workgroup per list.
  const int split_tail = gate_keyed_fits<T, K, GB>(g.n_blocks) ? 1 : 0;
  auto fallback = [&](auto kern) {
    hipLaunchKernelGGL(kern, fgrid, dim3(64 * WAVES), 0, st, static_cast<const T*>(q),
                       static_cast<const T*>(kbar), out, cu, g.seq_len, g.h_q, g.h_kv,
                       g.n_blocks, static_cast<int>(g.block_size), take, cur,
                       static_cast<int>(g.slots), ws.kbar_norm, ws.queue, ws.counter,
                       g.rows_per_seq, fb, split_tail);
  };
  if (split_tail) {
    fallback(gate_fallback_kernel<T, D, M, K, CAP, WAVES, GB, 1>);
    fgrid.x = 1;
    fallback(gate_fallback_kernel<T, D, M, K, CAP, WAVES, GB, 3>);
  } else {
    fallback(gate_fallback_kernel<T, D, M, K, CAP, WAVES, GB, 2>);
  }
  return check_launch("moba_gate (fallback)");
}

template <typename T>
static int run_gate(const void* q, const void* kbar, int32_t* out, const int32_t* cu,
                    const Geometry& g, int take, int cur, void* workspace,
                    size_t ws_bytes, hipStream_t st) {
  if constexpr (Elem<T>::kCode == MOBA_FP32) {
    (void)workspace; (void)ws_bytes;
    return dispatch_exact<T>(q, kbar, out, cu, g, take, cur, nullptr, nullptr, st);
  } else {
  // Block ids travel through LDS as 16 bits in the MFMA kernel.
  const bool mfma_ok = (g.head_dim == 64 || g.head_dim == 128) && take <= 16 &&
                       g.n_blocks <= 65535;
  if (!mfma_ok) return dispatch_exact<T>(q, kbar, out, cu, g, take, cur, nullptr, nullptr, st);
  GateWs ws = gate_ws(workspace, g.rows * g.h_kv, g.rows * g.h_q, g.rows_per_seq);
  if (!workspace || ws_bytes < moba_gate_workspace_size(g.rows, g.rows_per_seq, g.h_q) ||
      ws_bytes < ws.bytes)
    return fail(MOBA_ERR_WORKSPACE, "gate workspace too small");
  unsigned* norm_bits = reinterpret_cast<unsigned*>(ws.kbar_norm);
  hipLaunchKernelGGL(gate_init_kernel, dim3(1), dim3(256), 0, st, norm_bits,
                     g.rows * g.h_kv, ws.counter, ws.fb_count, g.rows * g.h_q * kFbBuckets);
  hipLaunchKernelGGL(gate_prep_kernel<T>,
                     dim3(static_cast<unsigned>(cdiv(g.n_blocks * 8, 256) < 16 ? cdiv(g.n_blocks * 8, 256) : 16),
                          static_cast<unsigned>(g.rows * g.h_kv)),
                     dim3(256), 0, st, static_cast<const T*>(kbar), cu, g.seq_len,
                     g.h_kv, g.n_blocks, g.head_dim, g.block_size, norm_bits);
  int rc = check_launch("moba_gate (prep)");
  if (rc) return rc;
  if (g.head_dim == 64) {
    rc = take <= 8 ? launch_mfma<T, 64, 12>(q, kbar, out, cu, g, take, cur, ws, st)
                   : launch_mfma<T, 64, 20>(q, kbar, out, cu, g, take, cur, ws, st);
  } else {
    rc = take <= 8 ? launch_mfma<T, 128, 12>(q, kbar, out, cu, g, take, cur, ws, st)
                   : launch_mfma<T, 128, 20>(q, kbar, out, cu, g, take, cur, ws, st);
  }
  if (rc) return rc;
  // Queries whose approximate evidence was insufficient: exact rescoring,
  // one workgroup per query.
  auto queue_launch = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(1024), dim3(64 * kQueueWaves), 0, st, static_cast<const T*>(q),
                       static_cast<const T*>(kbar), out, cu, g.seq_len, g.rows_per_seq, g.h_q,
                       g.h_kv, g.n_blocks, static_cast<int>(g.block_size), take, cur,
                       static_cast<int>(g.slots), ws.queue, ws.counter);
  };
  if (g.head_dim == 64)
    take <= 8 ? queue_launch(gate_queue_kernel<T, 8, 64>) : queue_launch(gate_queue_kernel<T, 16, 64>);
  else
    take <= 8 ? queue_launch(gate_queue_kernel<T, 8, 128>) : queue_launch(gate_queue_kernel<T, 16, 128>);
  return check_launch("moba_gate (queue)");
  }
}

}  // namespace moba

extern "C" size_t moba_gate_workspace_size(int64_t batch, int64_t seq_len, int64_t h_q) {
  // The layout of moba::gate_ws with the norms bounded by batch * h_q.
  return moba::gate_ws(nullptr, batch * h_q, batch * h_q, seq_len).bytes;
}

// ---------------------------------------------------------------------------
// No-allocation variant: the gate's scratch (queue counter, kbar norms,
// queue) lives in a file-scope device array instead of a caller workspace.
// Each device holds its own copy at its own address; host code takes that
// address once per device with hipGetSymbolAddress and never uses the
// array's name (on the host the name is a stand-in, not a device address).
// ---------------------------------------------------------------------------
namespace moba {

// The gate_ws layout at its largest: norms and fallback lengths for
// MOBA_GATE_STATIC_MAX_NORMS pairs, queue entries for the queries, and
// fallback lists rounded up to whole buckets (at most kFbBuckets - 1 spare
// entries per pair).
constexpr size_t kStaticBytes =
    256 + sizeof(float) * MOBA_GATE_STATIC_MAX_NORMS +
    sizeof(int64_t) * size_t(MOBA_GATE_STATIC_MAX_QUERIES) + 256 +
    sizeof(int) * kFbBuckets * size_t(MOBA_GATE_STATIC_MAX_NORMS) + 256 +
    sizeof(int2) * (size_t(MOBA_GATE_STATIC_MAX_QUERIES) +
                    size_t(kFbBuckets - 1) * MOBA_GATE_STATIC_MAX_NORMS);

static __device__ __align__(256) unsigned char scratch[kStaticBytes];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices];

// Address of the current device's copy of `scratch`, taken on the first
// call on that device.
static int static_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return fail(MOBA_ERR_LAUNCH, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return fail(MOBA_ERR_UNSUPPORTED, "device ordinal beyond the static scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(MOBA_ERR_LAUNCH,
                  std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MOBA_OK;
}

}  // namespace moba

extern "C" int moba_gate_noalloc(const void* q, const void* kbar, int32_t* block_idx,
                                 const int32_t* cu_seqlens, int64_t batch,
                                 int64_t seq_len, int64_t max_seqlen, int64_t h_q,
                                 int64_t h_kv, int64_t head_dim, int64_t n_blocks,
                                 int64_t block_size, int64_t slots, int64_t take,
                                 int always_current, int dtype, void* stream) {
  using namespace moba;
  Geometry g;
  int st = make_geometry(&g, batch, seq_len, max_seqlen, h_q, h_kv, head_dim, n_blocks,
                         block_size, slots, cu_seqlens);
  if (st) return st;
  const int64_t queries = g.rows * g.h_q * g.rows_per_seq;
  if (queries > MOBA_GATE_STATIC_MAX_QUERIES)
    return fail(MOBA_ERR_WORKSPACE,
                "moba_gate_noalloc: " + std::to_string(queries) +
                    " query rows (batch * h_q * rows per sequence) exceed the static "
                    "scratch limit of " + std::to_string(MOBA_GATE_STATIC_MAX_QUERIES));
  if (g.rows * g.h_q > MOBA_GATE_STATIC_MAX_NORMS ||
      moba_gate_workspace_size(g.rows, g.rows_per_seq, g.h_q) > kStaticBytes)
    return fail(MOBA_ERR_WORKSPACE,
                "moba_gate_noalloc: " + std::to_string(g.rows * g.h_q) +
                    " (row, query head) pairs exceed the static scratch limit of " +
                    std::to_string(MOBA_GATE_STATIC_MAX_NORMS));
  void* ws = nullptr;
  st = static_scratch(&ws);
  if (st) return st;
  return moba_gate(q, kbar, block_idx, cu_seqlens, batch, seq_len, max_seqlen, h_q, h_kv,
                   head_dim, n_blocks, block_size, slots, take, always_current, dtype, ws,
                   kStaticBytes, stream);
}

extern "C" int moba_gate(const void* q, const void* kbar, int32_t* block_idx,
                         const int32_t* cu_seqlens, int64_t batch, int64_t seq_len,
                         int64_t max_seqlen, int64_t h_q, int64_t h_kv,
                         int64_t head_dim, int64_t n_blocks, int64_t block_size,
                         int64_t slots, int64_t take, int always_current, int dtype,
                         void* workspace, size_t workspace_bytes, void* stream) {
  using namespace moba;
  Geometry g;
  int st = make_geometry(&g, batch, seq_len, max_seqlen, h_q, h_kv, head_dim, n_blocks,
                         block_size, slots, cu_seqlens);
  if (st) return st;
  if (!q || !kbar || !block_idx) return fail(MOBA_ERR_INVALID, "null pointer");
  if (take < 0 || slots < take + (always_current ? 1 : 0))
    return fail(MOBA_ERR_INVALID, "slots must hold take (+1 with the own block)");
  if (head_dim % 8 != 0)
    return fail(MOBA_ERR_UNSUPPORTED, "head_dim must be a multiple of 8");
  if (g.rows_per_seq >= (int64_t(1) << 31) / 2)
    return fail(MOBA_ERR_UNSUPPORTED, "sequence too long for int32 block ids");
  return MOBA_DISPATCH_DTYPE(dtype, T, [&] {
    return run_gate<T>(q, kbar, block_idx, cu_seqlens, g, static_cast<int>(take),
                       always_current ? 1 : 0, workspace, workspace_bytes,
                       as_stream(stream));
  });
}

// ---------------------------------------------------------------------------
// Hierarchical gate, second stage (opt-in).
// ---------------------------------------------------------------------------
namespace moba {

template <typename T>
static int launch_refine(const void* q, const void* kbar, const int32_t* sup, int32_t* out,
                         const Geometry& g, int group, int sup_slots, int take, int cur,
                         hipStream_t st) {
  const int n_cand = sup_slots * group;
  dim3 grid(static_cast<unsigned>(cdiv(g.seq_len, 4)), static_cast<unsigned>(g.rows * g.h_q));
  const int D = static_cast<int>(g.head_dim), bs = static_cast<int>(g.block_size);
  const int slots = static_cast<int>(g.slots);
#define MOBA_REFINE(L, TM)                                                                 \
  hipLaunchKernelGGL((gate_refine_kernel<T, L, TM>), grid, dim3(256), 0, st,              \
                     static_cast<const T*>(q), static_cast<const T*>(kbar), sup, out,      \
                     g.seq_len, g.h_q, g.h_kv, D, g.n_blocks, bs, group, sup_slots, take,  \
                     cur, slots)
  if (take > 16) return fail(MOBA_ERR_UNSUPPORTED, "moba_gate_refine: at most 16 past blocks");
  if (n_cand <= 64) {
    MOBA_REFINE(1, 16);
  } else if (n_cand <= 128) {
    MOBA_REFINE(2, 16);
  } else if (n_cand <= 256) {
    MOBA_REFINE(4, 16);
  } else if (n_cand <= 512) {
    MOBA_REFINE(8, 16);
  } else {
    return fail(MOBA_ERR_UNSUPPORTED,
                "moba_gate_refine: (opened + 1) * group must be at most 512 candidates");
  }
#undef MOBA_REFINE
  return check_launch("moba_gate_refine");
}

}  // namespace moba

extern "C" int moba_gate_refine(const void* q, const void* kbar, const int32_t* super_idx,
                                int32_t* block_idx, int64_t batch, int64_t seq_len,
                                int64_t h_q, int64_t h_kv, int64_t head_dim, int64_t n_blocks,
                                int64_t block_size, int64_t group, int64_t super_slots,
                                int64_t slots, int64_t take, int always_current, int dtype,
                                void* stream) {
  using namespace moba;
  Geometry g;
  int st = make_geometry(&g, batch, seq_len, seq_len, h_q, h_kv, head_dim, n_blocks,
                         block_size, slots, nullptr);
  if (st) return st;
  if (!q || !kbar || !super_idx || !block_idx) return fail(MOBA_ERR_INVALID, "null pointer");
  if (group <= 0 || super_slots <= 0)
    return fail(MOBA_ERR_INVALID, "moba_gate_refine: group and super_slots must be positive");
  if (take < 0 || slots < take + (always_current ? 1 : 0))
    return fail(MOBA_ERR_INVALID, "slots must hold take (+1 with the own block)");
  if (super_slots * group > 512)
    return fail(MOBA_ERR_UNSUPPORTED,
                "moba_gate_refine: super_slots * group must be at most 512 candidates");
  if (head_dim % 8 != 0) return fail(MOBA_ERR_UNSUPPORTED, "head_dim must be a multiple of 8");
  return MOBA_DISPATCH_DTYPE(dtype, T, [&] {
    return launch_refine<T>(q, kbar, super_idx, block_idx, g, static_cast<int>(group),
                            static_cast<int>(super_slots), static_cast<int>(take),
                            always_current ? 1 : 0, as_stream(stream));
  });
}
