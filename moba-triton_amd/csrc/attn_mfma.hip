// bf16 / fp16 MFMA kernels of the KV-block-major attention (gfx950).
//
// Forward (attend_mfma_kernel): one workgroup per (KV block, row * kv head),
// four waves (eight when one workgroup fills a CU's LDS). The block's K (row-major) and V (transposed, key order
// permuted per 16-key slice) are staged once in LDS. Each wave then takes
// groups of 32 column entries and runs, with v_mfma_f32_32x32x16:
//
//   S^T[key][q] = K . Q^T        (M = keys, N = queries, K = head_dim)
//   O^T[d][q]   = V^T . P^T      (M = head_dim, N = queries, K = keys)
//
// With the query on the N axis, every lane holds one query's scores, so the
// row max / sum need one cross-lane step (lane ^ 32) and P^T feeds the second
// MFMA straight from registers: the C layout of S^T gives lane-half h the
// keys 16j + 4h + {0..3, 8..11} of K-step j, and V^T is stored with each
// 16-key slice permuted so those eight keys are contiguous (one 16-byte LDS
// read per operand). Q rows are gathered from HBM directly into the B
// operand (each lane one 16-byte chunk of one query row).
//
// Semantics: src/moba/kernels/moba_fwd.py:230-425 -- additive tail / causal
// masks, m = max(q.k * D^-1/2 * log2 e), p = exp2(s - m) rounded to the
// input dtype for the PV product, l = sum p (float32; at head_dim >= 128
// the sum of the rounded p, on the matrix cores), partials stored at the
// query's fixed slot.
#include <type_traits>

#include "attn_common.h"

namespace moba {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));  // 16-byte chunk

template <typename T> struct Mfma;
template <> struct Mfma<bf16_t> {
  typedef bf16x8_t vec;
  typedef __bf16 scalar;
  __device__ static floatx16_t mma(vec a, vec b, floatx16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <> struct Mfma<f16_t> {
  typedef f16x8_t vec;
  typedef _Float16 scalar;
  __device__ static floatx16_t mma(vec a, vec b, floatx16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <typename V>
__device__ inline V ld16(const void* p) {
  return __builtin_bit_cast(V, *reinterpret_cast<const uint4*>(p));
}

// Transposing LDS read (ds_read_b64_tr_b16): within each group of 16 lanes,
// lane i receives element i % 4 of the 8-byte chunks that lanes i / 4,
// 4 + i / 4, 8 + i / 4 and 12 + i / 4 address. Two of them give one 8-wide
// MFMA operand whose elements run along the rows of a row-major tile.
typedef short v4i16_t __attribute__((ext_vector_type(4)));
template <typename V>
__device__ inline V ld_tr2(const uint16_t* p0, const uint16_t* p1) {
  typedef __attribute__((address_space(3))) v4i16_t lds_v4i16;
  const v4i16_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p0));
  const v4i16_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16*)(p1));
  typedef short v8i16_t __attribute__((ext_vector_type(8)));
  const v8i16_t v = {lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
  return __builtin_bit_cast(V, v);
}

// Four consecutive elements in one store (8 bytes for 16-bit types).
template <typename A>
__device__ inline void store4(A* p, float x0, float x1, float x2, float x3);
// Round to nearest even by the hardware conversions (v_cvt_pk_bf16_f32,
// v_cvt_f16_f32): the same results as the integer rounding of common.h for
// every finite input, without its per-value branches.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
template <>
__device__ inline void store4<bf16_t>(bf16_t* p, float x0, float x1, float x2, float x3) {
  uint2 u;
  u.x = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{x0, x1}, bf16x2_t));
  u.y = __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{x2, x3}, bf16x2_t));
  *reinterpret_cast<uint2*>(p) = u;
}
template <>
__device__ inline void store4<f16_t>(f16_t* p, float x0, float x1, float x2, float x3) {
  uint2 u;
  u.x = __builtin_bit_cast(uint32_t, f16x2_t{static_cast<_Float16>(x0), static_cast<_Float16>(x1)});
  u.y = __builtin_bit_cast(uint32_t, f16x2_t{static_cast<_Float16>(x2), static_cast<_Float16>(x3)});
  *reinterpret_cast<uint2*>(p) = u;
}
template <>
__device__ inline void store4<float>(float* p, float x0, float x1, float x2, float x3) {
  *reinterpret_cast<float4*>(p) = make_float4(x0, x1, x2, x3);
}

// Position of key offset o (within a 16-key slice) in the permuted layout:
// lane-half h = bit 2 of o owns positions [8h, 8h + 8).
__device__ inline int perm16(int o) { return ((o >> 2) & 1) * 8 + (o >> 3) * 4 + (o & 3); }

// Waves per attend workgroup. Each wave works through its own 32-entry
// groups, so the count only sets how many waves share one K / V^T tile: 4
// where two workgroups fit a CU's LDS, 8 where one workgroup fills it (so
// a CU still runs 2 waves per SIMD).
__host__ __device__ constexpr int attend_waves(int D, int BS) { return D * BS > 8192 ? 8 : 4; }

template <typename T, typename A, int D, int BS>
__global__ void __launch_bounds__(64 * attend_waves(D, BS), (D * BS > 8192) ? 1 : 2)
attend_mfma_kernel(AttnArgs a) {
  using M = Mfma<T>;
  using V8 = typename M::vec;
  constexpr int KS = D + 8;    // K row stride in LDS (elements): 16-byte aligned, staggered banks
  constexpr int VS = BS + 8;   // V^T row stride
  constexpr int KT = BS / 32;  // key tiles of 32
  constexpr int DT = D / 32;   // head_dim tiles of 32
  constexpr int RQ = D / 8;    // 16-byte chunks per row
  constexpr int CH = 32 * RQ / 64;  // 16-byte chunks per lane per 32-row tile
  constexpr bool kWide = sizeof(A) == 2;  // 16-bit partials go out through LDS as rows
  // Row sums on the matrix cores at D >= 128, where the P.V stage keeps
  // them least busy relative to the softmax VALU work (measured: 2.5 %
  // faster at D = 128, 2 % slower at D = 64).
  constexpr bool kOnesSum = D >= 128;
  __shared__ __attribute__((aligned(16))) uint16_t Ks[BS * KS];
  __shared__ __attribute__((aligned(16))) uint16_t Vt[D * VS];
  // Per wave: the group's Q rows on the way in, its partial rows on the way out.
  constexpr int NWV = attend_waves(D, BS);
  constexpr int NT = 64 * NWV;
  __shared__ __attribute__((aligned(16))) uint16_t Rw[NWV][32 * KS];

  const Column c = resolve_column(a, blockIdx.x, blockIdx.y);
  if (c.n == 0) return;
  const int tid = threadIdx.x;
  const uint16_t* K = static_cast<const uint16_t*>(a.k);
  const uint16_t* Vg = static_cast<const uint16_t*>(a.v);
  const uint16_t* Q = static_cast<const uint16_t*>(a.q);

  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int h = lane >> 5;
  const int col = lane & 31;
  uint16_t* rw = Rw[wave];
  A* acc_out = static_cast<A*>(a.part_acc);

  // Rows move in whole 16-byte chunks: lane i of the wave carries chunk
  // i % RQ of rows i / RQ + (64 / RQ) u, so every load / store instruction
  // covers complete rows. Two-stage pipeline: while group g is computed the
  // Q rows of group g + 1 and the index entries of group g + 2 are in flight.
  // Lane col holds the entries of query g + col; slot < 0 marks a dead lane.
  auto load_idx = [&](int32_t g, int32_t& r, int32_t& hd, int32_t& sl) {
    // Unconditional loads (clamped entry) keep the wait counts static.
    const int32_t e = g + col;
    const int64_t i = c.lo + (e < c.n ? e : c.n - 1);
    r = a.row_indices[i * a.istride];
    hd = a.head_indices[i * a.istride];
    sl = e < c.n ? a.slot_of_pair[i * a.istride] : -1;
  };
  u32x4 nq[CH];
  auto q_off = [&](int32_t r, int32_t hd, int32_t sl) -> int64_t {
    return sl >= 0 ? q_offset(a, c, r, hd) : -1;
  };
  auto fetch = [&](int64_t off) {
    // Unconditional: a dead entry reads row 0; its lanes' results are never
    // stored, and every MFMA column (query) is independent of the others.
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int64_t o = __shfl(off, lane / RQ + (64 / RQ) * u);
      nq[u] = *reinterpret_cast<const u32x4*>(Q + (o >= 0 ? o : 0) + (lane % RQ) * 8);
    }
  };
  // Column start: the first group's index entries and every K / V chunk of
  // the block are requested together, the first group's Q rows as soon as
  // its entries are in, and only then are K and V^T (permuted keys) written
  // to LDS -- one memory round trip before the first group, not several.
  constexpr int KVN = BS * D / 8 / NT;  // 16-byte K (and V) chunks per thread
  static_assert(BS * D / 8 % NT == 0, "K / V chunks must tile the workgroup");
  int32_t cr, chd, csl, nr, nhd, nsl;
  load_idx(wave * 32, cr, chd, csl);
  u32x4 kc[KVN], vc[KVN];
#pragma unroll
  for (int u = 0; u < KVN; ++u) {
    const int i = tid + u * NT;
    const int key = i / (D / 8);
    const int d8 = (i % (D / 8)) * 8;
    const int kk = c.key0 + key < c.key_end ? key : 0;  // tail keys: a valid row, zeroed below
    const int64_t off = ((c.tok0 + kk) * a.h_kv + c.hk) * D + d8;
    kc[u] = *reinterpret_cast<const u32x4*>(K + off);
    vc[u] = *reinterpret_cast<const u32x4*>(Vg + off);
  }
  fetch(q_off(cr, chd, csl));
  load_idx(wave * 32 + NWV * 32, nr, nhd, nsl);
#pragma unroll
  for (int u = 0; u < KVN; ++u) {
    const int i = tid + u * NT;
    const int key = i / (D / 8);
    const int d8 = (i % (D / 8)) * 8;
    const bool kin = c.key0 + key < c.key_end;
    const u32x4 kv = kin ? kc[u] : u32x4{0, 0, 0, 0};
    const u32x4 vv = kin ? vc[u] : u32x4{0, 0, 0, 0};
    *reinterpret_cast<u32x4*>(&Ks[key * KS + d8]) = kv;
    const uint16_t* ve = reinterpret_cast<const uint16_t*>(&vv);
    const int kp = (key & ~15) + perm16(key & 15);
#pragma unroll
    for (int w = 0; w < 8; ++w) Vt[(d8 + w) * VS + kp] = ve[w];
  }
  __syncthreads();
  auto stage_q = [&]() {
#pragma unroll
    for (int u = 0; u < CH; ++u)
      *reinterpret_cast<u32x4*>(&rw[(lane / RQ + (64 / RQ) * u) * KS + (lane % RQ) * 8]) = nq[u];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };
  stage_q();
  int64_t noff = q_off(nr, nhd, nsl);

  for (int32_t g0 = wave * 32; g0 < c.n; g0 += NWV * 32) {
    const bool live = csl >= 0;
    const int32_t row = cr;
    const int32_t head = chd;
    const int32_t slot = csl;
    // B operand: this lane's query, features 16k + 8h + [0, 8).
    V8 bq[D / 16];
#pragma unroll
    for (int k = 0; k < D / 16; ++k) bq[k] = ld16<V8>(&rw[col * KS + 16 * k + 8 * h]);
    if (g0 + NWV * 32 < c.n) fetch(noff);
    cr = nr;
    chd = nhd;
    csl = nsl;
    load_idx(g0 + 2 * NWV * 32, nr, nhd, nsl);

    // S^T tiles: the KT chains interleave (independent MFMAs back to back),
    // each K-step's operands read together.
    floatx16_t s[KT];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) s[kt] = floatx16_t{};
#pragma unroll
    for (int k = 0; k < D / 16; ++k) {
      V8 ka[KT];
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) ka[kt] = ld16<V8>(&Ks[(kt * 32 + col) * KS + 8 * h + 16 * k]);
#pragma unroll
      for (int kt = 0; kt < KT; ++kt) s[kt] = M::mma(ka[kt], bq[k], s[kt]);
    }

    // Masks, row max and sum. s[kt][v] is key 32kt + 8(v/4) + 4h + v%4.
    // Key / row positions relative to the block start fit in 32 bits.
    const int key_lim = static_cast<int>(c.key_end - c.key0);
    const int64_t rrel = static_cast<int64_t>(row) - c.key0;
    const int row_lim = !a.causal ? BS : (rrel < 0 ? -1 : (rrel >= BS ? BS : static_cast<int>(rrel)));
    const int lim = live ? min(key_lim - 1, row_lim) : -1;  // last visible key
    float m = -INFINITY, l = 0.f;
    if (__all(!live || lim == BS - 1)) {
      // Every key of the block is visible to every live query of the group
      // (a full, strictly past block): no masks; the scale folds into one
      // fma before the exp2 (scale > 0, so the max commutes with it).
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) m = fmaxf(m, s[kt][v]);
      m = fmaxf(m, __shfl_xor(m, 32)) * a.scale_log2;
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[kt][v], a.scale_log2, -m));
          s[kt][v] = p;
          if constexpr (!kOnesSum) l += p;
        }
    } else {
      // Same arithmetic as above on the visible keys (so a query's result
      // never depends on which queries share its group): hidden keys become
      // -inf once, and exp2 takes them to 0 (the masks are not kept alive
      // across both loops).
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const int key = kt * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
          s[kt][v] = key <= lim ? s[kt][v] : -INFINITY;
          m = fmaxf(m, s[kt][v]);
        }
      m = fmaxf(m, __shfl_xor(m, 32)) * a.scale_log2;
      const float mz = m > -INFINITY ? m : 0.f;  // no visible key: every p is 0
#pragma unroll
      for (int kt = 0; kt < KT; ++kt)
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[kt][v], a.scale_log2, -mz));
          s[kt][v] = p;
          if constexpr (!kOnesSum) l += p;
        }
    }
    if constexpr (!kOnesSum) l += __shfl_xor(l, 32);

    // O^T = V^T . P^T; K-step j takes registers 8(j%2)..+8 of tile j/2.
    floatx16_t o[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) o[dt] = floatx16_t{};
    // kOnesSum: the row sum as one more MFMA chain, a tile of ones against
    // the same P^T operand (every row of it is the sum of this lane's
    // query's rounded weights, exactly the weights that multiply V).
    floatx16_t lt = floatx16_t{};
    V8 ones;
#pragma unroll
    for (int u = 0; u < 8; ++u) ones[u] = static_cast<typename M::scalar>(1.0f);
#pragma unroll
    for (int j = 0; j < BS / 16; ++j) {
      V8 bp;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        bp[u] = static_cast<typename M::scalar>(s[j >> 1][8 * (j & 1) + u]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
        o[dt] = M::mma(ld16<V8>(&Vt[(dt * 32 + col) * VS + 16 * j + 8 * h]), bp, o[dt]);
      if constexpr (kOnesSum) lt = M::mma(ones, bp, lt);
    }
    if constexpr (kOnesSum) l = lt[0];

    const int64_t dst = live ? part_row(a, c, row, head) * a.slots + slot : -1;
    const bool more = g0 + NWV * 32 < c.n;
    // o[dt][v] is feature 32dt + 8(v/4) + 4h + v%4 of this lane's query.
    // Stores go out after the next group's rows are staged, so the wait for
    // those rows never includes them.
    if constexpr (kWide) {
      // Through LDS: four consecutive features per (dt, v/4) into the row of
      // this lane's query, then whole rows out.
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          store4<A>(reinterpret_cast<A*>(&rw[col * KS + dt * 32 + 8 * q4 + 4 * h]),
                    o[dt][4 * q4], o[dt][4 * q4 + 1], o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      u32x4 ov[CH];
#pragma unroll
      for (int u = 0; u < CH; ++u)
        ov[u] = *reinterpret_cast<const u32x4*>(&rw[(lane / RQ + (64 / RQ) * u) * KS + (lane % RQ) * 8]);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      if (more) stage_q();
      noff = q_off(nr, nhd, nsl);  // waits for the index loads, before any store
      if (live && h == 0) {
        *reinterpret_cast<float2*>(a.part_ml + 2 * dst) = make_float2(m, l);
      }
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        const int64_t rd = __shfl(dst, lane / RQ + (64 / RQ) * u);
        // Non-temporal: each partial row is read once, by the merge.
        if (rd >= 0)
          __builtin_nontemporal_store(ov[u], reinterpret_cast<u32x4*>(acc_out + rd * D + (lane % RQ) * 8));
      }
    } else {
      if (more) stage_q();
      noff = q_off(nr, nhd, nsl);
      if (live) {
        if (h == 0) {
          *reinterpret_cast<float2*>(a.part_ml + 2 * dst) = make_float2(m, l);
        }
        A* base = acc_out + dst * D + 4 * h;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            store4<A>(base + dt * 32 + 8 * q4, o[dt][4 * q4], o[dt][4 * q4 + 1],
                      o[dt][4 * q4 + 2], o[dt][4 * q4 + 3]);
      }
    }
  }
}

template <typename T, typename A, int D, int BS>
static int launch_attend(const AttnArgs& a, int64_t n_cols, hipStream_t st) {
  dim3 grid(static_cast<unsigned>(a.seg ? a.seg_cap : a.n_blocks), static_cast<unsigned>(n_cols));
  hipLaunchKernelGGL((attend_mfma_kernel<T, A, D, BS>), grid, dim3(64 * attend_waves(D, BS)), 0, st, a);
  return check_launch("moba_attend (mfma)");
}

template <typename T, typename A>
static int attend_dispatch(const AttnArgs& a, int64_t n_cols, hipStream_t st) {
  if (a.D == 64) {
    if (a.bs == 128) return launch_attend<T, A, 64, 128>(a, n_cols, st);
    if (a.bs == 64) return launch_attend<T, A, 64, 64>(a, n_cols, st);
    if (a.bs == 32) return launch_attend<T, A, 64, 32>(a, n_cols, st);
  } else if (a.D == 128) {
    if (a.bs == 128) return launch_attend<T, A, 128, 128>(a, n_cols, st);
    if (a.bs == 64) return launch_attend<T, A, 128, 64>(a, n_cols, st);
    if (a.bs == 32) return launch_attend<T, A, 128, 32>(a, n_cols, st);
  }
  return MOBA_ERR_UNSUPPORTED;
}

int attend_mfma(const AttnArgs& a, int dtype, int acc_dtype, int64_t n_cols, hipStream_t st) {
  if (dtype == MOBA_BF16) {
    if (acc_dtype == MOBA_BF16) return attend_dispatch<bf16_t, bf16_t>(a, n_cols, st);
    if (acc_dtype == MOBA_FP32) return attend_dispatch<bf16_t, float>(a, n_cols, st);
  } else if (dtype == MOBA_FP16) {
    if (acc_dtype == MOBA_FP16) return attend_dispatch<f16_t, f16_t>(a, n_cols, st);
    if (acc_dtype == MOBA_FP32) return attend_dispatch<f16_t, float>(a, n_cols, st);
  }
  return MOBA_ERR_UNSUPPORTED;
}

// ---------------------------------------------------------------------------
// Backward (bwd_mfma_kernel): one workgroup per (KV block, row * kv head),
// one wave per 32 keys of the block. The workgroup owns its keys' dK / dV
// for the whole column (registers, stored once: no atomics), and walks the
// column in steps of 64 entries. Per step, with the step's Q / dO rows
// staged in LDS (row-major; the transposed operands come from transposing
// reads, ds_read_b64_tr_b16):
//
//   S[q][key]   = Q . K^T,   dP[q][key] = dO . V^T      (lane <-> key)
//   P = exp2(S * scale log2e - lse),  dS = P (dP - delta)
//   dV^T[d][key] += dO^T . P,   dK^T[d][key] += Q^T . dS  (P, dS straight
//                                                         from registers)
//   dQ^T[d][q]   = K^T . dS^T over all keys of the block, via dS^T rows
//                  ([key][q], 8-byte writes) in LDS
//
// and writes one dQ partial per (query, slot) -- summed over the whole block
// inside the workgroup, so the partial buffer is [.., slots, D], not
// slots x sub-tiles. Semantics: src/moba/kernels/moba_bwd.py:216-394.
// ---------------------------------------------------------------------------
// Piece permutation of a Q / dO tile row (bwd_mfma_kernel at head_dim 64):
// bits 1-3 of the row, reversed. Rows 2i and 2i + 1 share it; the eight
// even (odd) rows of 16 consecutive ones take eight distinct values, and
// rows 4a, 4a + 1 and 4a + 2, 4a + 3 differ in bit 2, which moves a
// 64-byte run of four pieces to the other half of the row.
__device__ constexpr int bq_swz(int row) {
  return (((row >> 1) & 1) << 2) | ((row >> 1) & 2) | ((row >> 3) & 1);
}

template <typename T, typename A, int D, int BS, int NQ, int ST>
__global__ void __launch_bounds__(BS * 2 * ST, (D == 64 && BS == 128) ? 2 : 1)
bwd_mfma_kernel(AttnArgs a) {
  using M = Mfma<T>;
  using V8 = typename M::vec;
  using Sc = typename M::scalar;
  // NQ: queries per step (64; 32 at head_dim 128 with blocks under 128 keys)
  constexpr int QT = NQ / 32;   // query tiles of 32
  constexpr int NW = BS / 32;   // waves per stream: 32 keys each
  constexpr int NT = NW * 64;   // threads per stream
  constexpr int NTA = NT * ST;  // threads
  // ST = 2: two streams of waves walk alternate steps of the column against
  // the same keys, each with its own rows, dS^T and dK / dV sums (added at
  // the end). K and V then sit row-major in LDS instead of in each lane's
  // registers (S / dP read their B operands from there, dQ its K^T operand
  // by transposing reads), which keeps a wave within 256 registers so a CU
  // runs two of them per SIMD.
  constexpr bool kKV = ST > 1;
  constexpr int DT = D / 32;
  constexpr int RS = D + 8;     // row stride of [key|q][d] tiles
  // Q / dO tiles at head_dim 64 with one stream: unpadded 128-byte rows
  // whose 16-byte pieces are permuted by bq_swz (qx below). The S / dP row
  // reads (16 lanes: 16 consecutive rows, one piece each) and the
  // transposing reads (32 lanes: 4 consecutive rows x 4 pieces) then meet
  // 16 distinct 4-bank groups per 16 lanes; with the padded stride the
  // transposing reads folded rows r and r + 2 onto the same banks. Each
  // lane's addresses stay loop-invariant.
  constexpr bool kSwz = D == 64 && !kKV;
  constexpr int QRS = kSwz ? D : RS;  // row stride of the Q / dO tiles
  auto qx = [](int row, int e) {      // element offset of (row, feature e)
    return kSwz ? row * QRS + ((((e >> 3) ^ bq_swz(row)) << 3) | (e & 7)) : row * QRS + e;
  };
  constexpr int KTS = BS + 8;   // row stride of K^T ([d][key])
  // Row stride of dS^T ([key][q]): 34 banks, so the 32 keys of a wave's
  // 8-byte dS writes land on distinct bank pairs (NQ + 8 paired keys c and
  // c + 16; measured 2% faster at 512K).
  constexpr int QS2 = NQ + 4;
  // K^T ([d][key]) for one stream, or K and V ([key][d]) for two.
  __shared__ __attribute__((aligned(16))) uint16_t Kl[kKV ? 2 * BS * RS : D * KTS];
  // Per stream: Q rows, dO rows, dS^T. One array, so that the float32
  // hand-over of dK / dV between the streams can reuse all of it.
  constexpr int kRows = 2 * NQ * QRS + BS * QS2;
  __shared__ __attribute__((aligned(16))) uint16_t Sm[ST * kRows];
  __shared__ __attribute__((aligned(16))) float s_lse_[ST][NQ];
  __shared__ __attribute__((aligned(16))) float s_delta_[ST][NQ];
  __shared__ __attribute__((aligned(16))) int s_lim_[ST][NQ];
  // dQ destinations by step parity: the stores of step g read them after the
  // dS barrier, while step g + 1's are already being staged.
  __shared__ int64_t s_dst_[ST][2][NQ];
  // dQ tiles per wave ([q][d], 32 x 32, row stride DQS) on their way out as
  // 16-byte chunks; private to the wave, so only a wave barrier orders them.
  constexpr int TPW = DT * (NQ / 32) / (BS / 32);
  constexpr int DQS = 40;
  __shared__ __attribute__((aligned(16))) uint16_t DQs_[sizeof(A) == 2 ? ST * (BS / 32) * TPW * 32 * DQS : 8];
  static_assert((NQ * QRS * 2) % 16 == 0 && (kRows * 2) % 16 == 0, "16-byte aligned carving");

  const Column c = resolve_column(a, blockIdx.x, blockIdx.y);
  if (c.skip) return;  // past the segment list (uniform)
  const int tid = threadIdx.x;
  const uint16_t* Kg = static_cast<const uint16_t*>(a.k);
  const uint16_t* Vg = static_cast<const uint16_t*>(a.v);
  const uint16_t* Qg = static_cast<const uint16_t*>(a.q);
  const uint16_t* Og = static_cast<const uint16_t*>(a.dout);
  const int key_lim = static_cast<int>(c.key_end - c.key0);
  // No keys (a column past its sequence): no query selects it and there is
  // no dK / dV to write; its K / V rows would lie past the tensor.
  if (key_lim <= 0) return;  // uniform

  const int lane = tid & 63;
  const int stream = kKV ? tid / NT : 0;
  const int stid = kKV ? tid % NT : tid;  // thread index within the stream
  const int wave = stid >> 6;
  uint16_t* Qs = Sm + stream * kRows;
  uint16_t* Os = Qs + NQ * QRS;
  uint16_t* DSt = Os + NQ * QRS;
  uint16_t* Kt = Kl;          // one stream
  uint16_t* Ks = Kl;          // two streams
  uint16_t* Vs = kKV ? Kl + BS * RS : Kl;  // (unused with one stream)
  float* s_lse = s_lse_[stream];
  float* s_delta = s_delta_[stream];
  int* s_lim = s_lim_[stream];
  const int h = lane >> 5;
  const int col = lane & 31;
  const int mykey = wave * 32 + col;  // the key this lane holds in S / dP / dV / dK
  floatx16_t dv[DT], dk[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) { dv[dt] = floatx16_t{}; dk[dt] = floatx16_t{}; }
  A* dq_out = static_cast<A*>(a.part_acc);

  // Entry pipeline. A thread of the stream's first wave tracks entry
  // stid % NQ of a step (lanes past NQ duplicate it); its loads are
  // unconditional within the loop: while step g is computed, the Q / dO
  // rows and lse / delta of step g + 1 and the index entries of step g + 2
  // are in flight; everything is waited for once, after the step's dQ.
  constexpr int CH = NQ * D / 8 / NT;  // 16-byte chunks per thread per tensor
  static_assert(NQ * D / 8 % NT == 0, "row chunks must tile the workgroup");
  const int qi = stid % NQ;
  const int32_t last = c.n > 0 ? c.n - 1 : 0;
  int32_t i_row = 0, i_head = 0, i_slot = 0;    // raw entry, step g + 2
  bool i_live = false;
  // Only the first wave of a stream (threads stid < 64 >= NQ) loads the
  // index entries and row statistics, derives them and stages them; the
  // other waves read what it staged.
  const bool idx_wave = stid < 64;
  auto load_idx = [&](int32_t g) {
    if (!idx_wave) return;  // wave-uniform
    const int32_t e = g + qi;
    const int64_t i = c.lo + (e < c.n ? e : last);
    i_row = a.row_indices[i * a.istride];
    i_head = a.head_indices[i * a.istride];
    // Raw: the entry's liveness is applied in derive(), after the wait;
    // a select here would wait for the load right away.
    i_slot = a.slot_of_pair[i * a.istride];
    i_live = e < c.n;
  };
  int64_t n_pr = 0, n_dst = -1;                 // derived, step g + 1
  int n_lim = -1;
  __shared__ int64_t s_qoff_[ST][NQ];
  int64_t* s_qoff = s_qoff_[stream];
  // derive() runs in every wave (on constants outside the first), so the
  // loads above are consumed on every path and never waited for later.
  auto derive = [&]() {
    const bool ok = i_live;
    const int64_t pr = part_row(a, c, i_row, i_head);
    const int64_t rrel = static_cast<int64_t>(i_row) - c.key0;
    const int row_lim = !a.causal ? BS : (rrel < 0 ? -1 : (rrel >= BS ? BS : static_cast<int>(rrel)));
    n_pr = ok ? pr : 0;
    n_dst = ok ? pr * a.slots + i_slot : -1;
    n_lim = ok ? min(key_lim - 1, row_lim) : -1;
    if (stid < NQ) s_qoff[stid] = ok ? q_offset(a, c, i_row, i_head) : -1;
  };
  u32x4 pq[CH], po[CH];
  bool pv[CH];  // chunk belongs to a live entry (zeroed when staged)
  float n_lse = 0.f, n_dl = 0.f;
  auto fetch = [&]() {  // step g + 1: rows via s_qoff, lse / delta via n_pr
    if (idx_wave) {
      const float2 ld = *reinterpret_cast<const float2*>(a.lse_delta + 2 * n_pr);
      n_lse = ld.x;
      n_dl = ld.y;
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int i = stid + u * NT;
      const int64_t o = s_qoff[i / (D / 8)];
      const int64_t off = (o >= 0 ? o : 0) + (i % (D / 8)) * 8;
      pq[u] = *reinterpret_cast<const u32x4*>(Qg + off);
      po[u] = *reinterpret_cast<const u32x4*>(Og + off);
      pv[u] = o >= 0;
    }
  };
  int c_lim = -1;
  int64_t c_dst = -1;
  float c_lse = 0.f, c_dl = 0.f;
  // Column start: step 0's index entries, the block's K chunks for K^T in
  // LDS (for dQ) and this lane's K and V rows (the B operands of S and dP
  // for the whole column) are requested together; step 0's rows as soon as
  // its entries are in; then K^T is written. Loads are unconditional: keys
  // past the block's end read a valid row (K^T zeroes them; their S and dP
  // are masked and their dK / dV never stored).
  constexpr int KTN = BS * D / 8 / NTA;  // 16-byte K (and V) chunks per thread
  static_assert(BS * D / 8 % NTA == 0, "K chunks must tile the workgroup");
  if (c.n > 0) load_idx(stream * NQ);
  u32x4 ktc[KTN], vtc[kKV ? KTN : 1];
#pragma unroll
  for (int u = 0; u < KTN; ++u) {
    const int i = tid + u * NTA;
    const int key = i / (D / 8);
    const int d8 = (i % (D / 8)) * 8;
    const int64_t off = ((c.tok0 + (key < key_lim ? key : 0)) * a.h_kv + c.hk) * D + d8;
    ktc[u] = *reinterpret_cast<const u32x4*>(Kg + off);
    if constexpr (kKV) vtc[u] = *reinterpret_cast<const u32x4*>(Vg + off);
  }
  V8 kb[kKV ? 1 : D / 16], vb[kKV ? 1 : D / 16];
  if constexpr (!kKV) {
    const int64_t off = ((c.tok0 + (mykey < key_lim ? mykey : 0)) * a.h_kv + c.hk) * D + 8 * h;
#pragma unroll
    for (int k = 0; k < D / 16; ++k) {
      kb[k] = ld16<V8>(Kg + off + 16 * k);
      vb[k] = ld16<V8>(Vg + off + 16 * k);
    }
  }
  if (c.n > 0) {
    derive();
    __syncthreads();
    fetch();
    load_idx(stream * NQ + ST * NQ);
  }
#pragma unroll
  for (int u = 0; u < KTN; ++u) {
    const int i = tid + u * NTA;
    const int key = i / (D / 8);
    const int d8 = (i % (D / 8)) * 8;
    const u32x4 kv = key < key_lim ? ktc[u] : u32x4{0, 0, 0, 0};
    if constexpr (kKV) {
      *reinterpret_cast<u32x4*>(&Ks[key * RS + d8]) = kv;
      *reinterpret_cast<u32x4*>(&Vs[key * RS + d8]) = key < key_lim ? vtc[u] : u32x4{0, 0, 0, 0};
    } else {
      const uint16_t* ke = reinterpret_cast<const uint16_t*>(&kv);
#pragma unroll
      for (int w = 0; w < 8; ++w) Kt[(d8 + w) * KTS + key] = ke[w];
    }
  }
  if (c.n > 0) {
    c_lim = n_lim; c_dst = n_dst; c_lse = n_lse; c_dl = n_dl;
    derive();  // s_qoff now describes step 1; every thread read step 0's above
  }
  // Stages one step: its limits, row statistics, dQ destinations (parity
  // par) and its Q / dO rows, row-major (the dV / dK products read them
  // transposed). A dead step (act false) gets zero rows and no entries.
  auto stage = [&](bool act, int par) {
    if (stid < NQ) {
      s_lim[stid] = act ? c_lim : -1;
      s_lse[stid] = c_lse;
      s_delta[stid] = c_dl;
      s_dst_[stream][par][stid] = act ? c_dst : -1;
    }
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const int i = stid + u * NT;
      const int q = i / (D / 8);
      const int d8 = (i % (D / 8)) * 8;
      *reinterpret_cast<u32x4*>(&Qs[qx(q, d8)]) = pv[u] && act ? pq[u] : u32x4{0, 0, 0, 0};
      *reinterpret_cast<u32x4*>(&Os[qx(q, d8)]) = pv[u] && act ? po[u] : u32x4{0, 0, 0, 0};
    }
  };
  // vmcnt(0): the K / V operands and the prologue loads are all resident, so
  // the loop's wait counts start from an empty queue on every path.
  __builtin_amdgcn_s_waitcnt(0x0f70);
  if (c.n > 0) stage(stream * NQ < c.n, 0);

  // Every stream runs the same number of iterations (the barriers are
  // shared); a stream past the column's end runs a dead step: zero rows,
  // every entry hidden, nothing stored. Two workgroup barriers per step:
  // the first makes the step's staging visible (and orders the previous
  // step's dQ reads of dS^T before this step's dS writes), the second makes
  // dS visible and frees Qs / Os, which the next step is then staged into
  // while this step's dQ is formed.
  int par = 0;
  for (int32_t base = 0; base < c.n; base += ST * NQ, par ^= 1) {
    const int32_t g0 = base + stream * NQ;
    __syncthreads();
    const int64_t* s_dst = s_dst_[stream][par];
    // Every entry of the step sees the whole block (a strictly past, full
    // block) or is dead: the causal masks can go. A dead entry's Q and dO
    // rows are zero, so it adds nothing to dK / dV either way, and its dQ is
    // never stored. Each wave reads the same NQ limits, so the vote is
    // uniform over the workgroup.
    const bool all_visible = __all(lane >= NQ || s_lim[lane < NQ ? lane : 0] == BS - 1 ||
                                   s_lim[lane < NQ ? lane : 0] < 0);
    const bool more = g0 + ST * NQ < c.n;
    // Unconditional (past the column's end they read valid, clamped rows
    // and are never used): loads issued under a condition that the
    // consuming derive() below repeats leave the compiler's wait analysis
    // a path on which they are still pending at the next step, and it then
    // waits there for every store in flight.
    fetch();
    load_idx(g0 + 2 * ST * NQ);

    // S and dP for this wave's 32 keys and each 32-query tile; lane <->
    // key, register v <-> query 32 qt + 8(v/4) + 4h + v%4.
#pragma unroll
    for (int qt = 0; qt < QT; ++qt) {
      floatx16_t sacc = floatx16_t{}, pacc = floatx16_t{};
#pragma unroll
      for (int k = 0; k < D / 16; ++k) {
        const int qo = qx(qt * 32 + col, 16 * k + 8 * h);
        if constexpr (kKV) {
          sacc = M::mma(ld16<V8>(&Qs[qo]), ld16<V8>(&Ks[mykey * RS + 16 * k + 8 * h]), sacc);
          pacc = M::mma(ld16<V8>(&Os[qo]), ld16<V8>(&Vs[mykey * RS + 16 * k + 8 * h]), pacc);
        } else {
          sacc = M::mma(ld16<V8>(&Qs[qo]), kb[k], sacc);
          pacc = M::mma(ld16<V8>(&Os[qo]), vb[k], pacc);
        }
      }
      V8 pb[2], db[2];  // P and dS as B operands, K-steps over queries
      auto softmax = [&](auto masked) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {  // queries 32qt + 8g + 4h + [0, 4)
        const int q0 = qt * 32 + 8 * g + 4 * h;
        int limv[4] = {BS, BS, BS, BS};
        if constexpr (decltype(masked)::value) {
          const int4 lim4 = *reinterpret_cast<const int4*>(&s_lim[q0]);
          limv[0] = lim4.x; limv[1] = lim4.y; limv[2] = lim4.z; limv[3] = lim4.w;
        }
        const float4 lse4 = *reinterpret_cast<const float4*>(&s_lse[q0]);
        const float4 dl4 = *reinterpret_cast<const float4*>(&s_delta[q0]);
        const float lsev[4] = {lse4.x, lse4.y, lse4.z, lse4.w};
        const float dlv[4] = {dl4.x, dl4.y, dl4.z, dl4.w};
        float dsf[4];  // this key's dS of the four queries: one 8-byte row piece
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int v = 4 * g + w;
          const float x = (!decltype(masked)::value || mykey <= limv[w])
                              ? sacc[v] * a.scale_log2 - lsev[w] : -INFINITY;
          const float p = __builtin_amdgcn_exp2f(x);
          const float ds = p * (pacc[v] - dlv[w]);
          pb[v >> 3][v & 7] = static_cast<Sc>(p);
          db[v >> 3][v & 7] = static_cast<Sc>(ds);
          dsf[w] = ds;
        }
        typedef Sc sc4_t __attribute__((ext_vector_type(4)));
        typedef float f32x4_t __attribute__((ext_vector_type(4)));
        *reinterpret_cast<uint2*>(&DSt[mykey * QS2 + q0]) = __builtin_bit_cast(
            uint2, __builtin_convertvector(f32x4_t{dsf[0], dsf[1], dsf[2], dsf[3]}, sc4_t));
      }
      };
      if (all_visible) softmax(std::false_type{});
      else softmax(std::true_type{});
      // dV^T += dO^T . P and dK^T += Q^T . dS. The A operands are dO / Q
      // read transposed: lane (group g = lane / 16, r = lane % 16) addresses
      // row 32qt + 16j + 8m + 4h + r / 4, features 32dt + 16(g % 2) + 4(r % 4)
      // + [0, 4) for half m of the operand, so lane (col, h) receives
      // feature 32dt + col of the queries 32qt + 16j + 8m + 4h + [0, 4) --
      // the queries of its P / dS B operand elements 4m .. 4m + 3.
      const int tr_row = 4 * h + ((lane & 15) >> 2);
      const int tr_col = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          const int o0 = qx(qt * 32 + 16 * j + tr_row, dt * 32 + tr_col);
          const int o1 = qx(qt * 32 + 16 * j + tr_row + 8, dt * 32 + tr_col);
          dv[dt] = M::mma(ld_tr2<V8>(&Os[o0], &Os[o1]), pb[j], dv[dt]);
          dk[dt] = M::mma(ld_tr2<V8>(&Qs[o0], &Qs[o1]), db[j], dk[dt]);
        }
      }
    }
    __syncthreads();  // dS of every wave visible; Qs / Os free

    // dQ^T[d][q] over all BS keys; (feature tile, query tile) pairs spread
    // over the waves.
    static_assert(DT * QT % NW == 0, "dQ tiles must spread evenly over the waves");
    // B operand (dS^T, keys 16j + 8h + [0, 8) of query 32qt + col) read
    // transposed from the [key][q] rows: lane (g, r) addresses key
    // 16j + 8h + 4m + r / 4, queries 32qt + 16(g % 2) + 4(r % 4) + [0, 4).
    const int tr_key = 8 * h + ((lane & 15) >> 2);
    const int tr_q = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
    floatx16_t dq[TPW];
#pragma unroll
    for (int t = 0; t < TPW; ++t) {
      const int tt = wave + t * NW;
      const int dt = tt % DT, qt = tt / DT;
      dq[t] = floatx16_t{};
#pragma unroll
      for (int j = 0; j < BS / 16; ++j) {
        if constexpr (kKV) {
          // Both operands by transposing reads with the dV / dK pattern:
          // lane (col, h) holds, at K slots 8h + 4m + [0, 4), the keys
          // 16j + 8m + 4h + [0, 4) -- of feature 32dt + col of K (A) and of
          // query 32qt + col of dS (B).
          const int kr = 16 * j + 4 * h + ((lane & 15) >> 2);
          const int c4 = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);
          dq[t] = M::mma(ld_tr2<V8>(&Ks[kr * RS + dt * 32 + c4], &Ks[(kr + 8) * RS + dt * 32 + c4]),
                         ld_tr2<V8>(&DSt[kr * QS2 + qt * 32 + c4], &DSt[(kr + 8) * QS2 + qt * 32 + c4]),
                         dq[t]);
        } else {
          dq[t] = M::mma(ld16<V8>(&Kt[(dt * 32 + col) * KTS + 16 * j + 8 * h]),
                         ld_tr2<V8>(&DSt[(16 * j + tr_key) * QS2 + qt * 32 + tr_q],
                                    &DSt[(16 * j + 4 + tr_key) * QS2 + qt * 32 + tr_q]),
                         dq[t]);
        }
      }
    }
    // dq[t][v] is feature 32dt + 8(v/4) + 4h + v%4 of query 32qt + col.
    const bool next = base + ST * NQ < c.n;  // uniform: the loop runs again
    if constexpr (sizeof(A) == 2) {
      // dQ through this wave's LDS tiles, read back as 16-byte chunks.
      uint16_t* dqs = DQs_ + ((stream * NW + wave) * TPW) * 32 * DQS;
#pragma unroll
      for (int t = 0; t < TPW; ++t)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4)
          store4<A>(reinterpret_cast<A*>(&dqs[(t * 32 + col) * DQS + 8 * q4 + 4 * h]),
                    dq[t][4 * q4] * a.scale, dq[t][4 * q4 + 1] * a.scale,
                    dq[t][4 * q4 + 2] * a.scale, dq[t][4 * q4 + 3] * a.scale);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      u32x4 val[TPW][2];
      int64_t dst[TPW][2];
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int qt = (wave + t * NW) / DT;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int ci = lane + 64 * u;
          val[t][u] = *reinterpret_cast<const u32x4*>(&dqs[(t * 32 + (ci >> 2)) * DQS + (ci & 3) * 8]);
          dst[t][u] = s_dst[qt * 32 + (ci >> 2)];
        }
      }
      // Keep the next step's index arithmetic (which waits for the loads in
      // flight) behind this step's dQ work.
      __builtin_amdgcn_sched_barrier(0);
      c_lim = n_lim; c_dst = n_dst; c_lse = n_lse; c_dl = n_dl;
      derive();  // waits for every load in flight
      if (next) stage(more, par ^ 1);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int dt = (wave + t * NW) % DT;
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int d8 = dt * 32 + ((lane + 64 * u) & 3) * 8;
          if (dst[t][u] >= 0) *reinterpret_cast<u32x4*>(dq_out + dst[t][u] * D + d8) = val[t][u];
        }
      }
    } else {
      int64_t dst[TPW];
#pragma unroll
      for (int t = 0; t < TPW; ++t) dst[t] = s_dst[((wave + t * NW) / DT) * 32 + col];
      // Keep the next step's index arithmetic (which waits for the loads in
      // flight) behind this step's dQ work.
      __builtin_amdgcn_sched_barrier(0);
      c_lim = n_lim; c_dst = n_dst; c_lse = n_lse; c_dl = n_dl;
      derive();  // waits for every load in flight
      if (next) stage(more, par ^ 1);
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int tt = wave + t * NW;
        const int dt = tt % DT;
        if (dst[t] >= 0) {
          A* base = dq_out + dst[t] * D + dt * 32 + 4 * h;
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            store4<A>(base + 8 * q4, dq[t][4 * q4] * a.scale, dq[t][4 * q4 + 1] * a.scale,
                      dq[t][4 * q4 + 2] * a.scale, dq[t][4 * q4 + 3] * a.scale);
        }
      }
    }
  }

  if constexpr (kKV) {
    // Stream 1 hands its float32 sums to stream 0 through the K / V LDS
    // (free once every step is done), dK then dV; slot (dt, q4, wave, lane)
    // holds four consecutive floats.
    float4* xb = reinterpret_cast<float4*>(Kl);
    static_assert(DT * 4 * NW * 64 * 16 <= sizeof(Kl), "dK / dV hand-over fits the K / V LDS");
    auto hand_over = [&](floatx16_t (&acc)[DT]) {
      __syncthreads();  // the previous use of this LDS is complete
      if (stream == 1) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4)
            xb[((dt * 4 + q4) * NW + wave) * 64 + lane] =
                make_float4(acc[dt][4 * q4], acc[dt][4 * q4 + 1], acc[dt][4 * q4 + 2], acc[dt][4 * q4 + 3]);
      }
      __syncthreads();
      if (stream == 0) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const float4 o = xb[((dt * 4 + q4) * NW + wave) * 64 + lane];
            acc[dt][4 * q4] += o.x;
            acc[dt][4 * q4 + 1] += o.y;
            acc[dt][4 * q4 + 2] += o.z;
            acc[dt][4 * q4 + 3] += o.w;
          }
      }
    };
    hand_over(dk);
    hand_over(dv);
    if (stream != 0) return;
  }
  // dK, dV of this lane's key: register v is feature 32dt + 8(v/4) + 4h + v%4.
  // A segment of a cut column leaves its float32 sums in its scratch slot
  // ([2][BS][D]: dK scaled, dV); the finishing pass adds the column's
  // segments in order.
  if (c.nseg > 1) {
    if (mykey < key_lim) {
      float* sk = a.seg_scratch +
                  (static_cast<int64_t>(blockIdx.y) * a.scratch_cap + c.scratch) * 2 * BS * D +
                  mykey * D + 4 * h;
      float* sv = sk + BS * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          store4<float>(sk + dt * 32 + 8 * q4, dk[dt][4 * q4] * a.scale,
                        dk[dt][4 * q4 + 1] * a.scale, dk[dt][4 * q4 + 2] * a.scale,
                        dk[dt][4 * q4 + 3] * a.scale);
          store4<float>(sv + dt * 32 + 8 * q4, dv[dt][4 * q4], dv[dt][4 * q4 + 1],
                        dv[dt][4 * q4 + 2], dv[dt][4 * q4 + 3]);
        }
    }
    return;
  }
  if (mykey < key_lim) {
    const int64_t off = ((c.tok0 + mykey) * a.h_kv + c.hk) * D + 4 * h;
    auto store_kv = [&](auto* dK, auto* dV) {
      using E = std::remove_pointer_t<decltype(dK)>;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          store4<E>(dK + dt * 32 + 8 * q4, dk[dt][4 * q4] * a.scale, dk[dt][4 * q4 + 1] * a.scale,
                    dk[dt][4 * q4 + 2] * a.scale, dk[dt][4 * q4 + 3] * a.scale);
          store4<E>(dV + dt * 32 + 8 * q4, dv[dt][4 * q4], dv[dt][4 * q4 + 1],
                    dv[dt][4 * q4 + 2], dv[dt][4 * q4 + 3]);
        }
    };
    if (a.dkv_f32)  // uniform: float32 sums for a caller that adds several calls
      store_kv(static_cast<float*>(a.dk) + off, static_cast<float*>(a.dv) + off);
    else
      store_kv(static_cast<T*>(a.dk) + off, static_cast<T*>(a.dv) + off);
  }
}

template <typename T, typename A, int D, int BS>
static int launch_bwd(const AttnArgs& a, int64_t n_cols, hipStream_t st) {
  // 64 queries per step at head_dim 64, 32 at 128 (wider steps spill). At
  // head_dim 128 with 128-key blocks, two streams of 4 waves share the keys
  // (K / V in LDS): 8 waves, 2 per SIMD, in 125 KiB of LDS.
  constexpr int ST = (D == 128 && BS == 128) ? 2 : 1;
  constexpr int NQ = D == 128 ? 32 : 64;
  dim3 grid(static_cast<unsigned>(a.seg ? a.seg_cap : a.n_blocks), static_cast<unsigned>(n_cols));
  hipLaunchKernelGGL((bwd_mfma_kernel<T, A, D, BS, NQ, ST>), grid, dim3(BS * 2 * ST), 0, st, a);
  return check_launch("moba_bwd (mfma)");
}

template <typename T, typename A>
static int bwd_dispatch(const AttnArgs& a, int64_t n_cols, hipStream_t st) {
  if (a.D == 64) {
    if (a.bs == 128) return launch_bwd<T, A, 64, 128>(a, n_cols, st);
    if (a.bs == 64) return launch_bwd<T, A, 64, 64>(a, n_cols, st);
    if (a.bs == 32) return launch_bwd<T, A, 64, 32>(a, n_cols, st);
  } else if (a.D == 128) {
    if (a.bs == 128) return launch_bwd<T, A, 128, 128>(a, n_cols, st);
    if (a.bs == 64) return launch_bwd<T, A, 128, 64>(a, n_cols, st);
    if (a.bs == 32) return launch_bwd<T, A, 128, 32>(a, n_cols, st);
  }
  return MOBA_ERR_UNSUPPORTED;
}

int bwd_mfma(const AttnArgs& a, int dtype, int acc_dtype, int64_t n_cols, hipStream_t st) {
  if (dtype == MOBA_BF16) {
    if (acc_dtype == MOBA_BF16) return bwd_dispatch<bf16_t, bf16_t>(a, n_cols, st);
    if (acc_dtype == MOBA_FP32) return bwd_dispatch<bf16_t, float>(a, n_cols, st);
  } else if (dtype == MOBA_FP16) {
    if (acc_dtype == MOBA_FP16) return bwd_dispatch<f16_t, f16_t>(a, n_cols, st);
    if (acc_dtype == MOBA_FP32) return bwd_dispatch<f16_t, float>(a, n_cols, st);
  }
  return MOBA_ERR_UNSUPPORTED;
}

}  // namespace moba
