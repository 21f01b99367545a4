// KV-block-major attention, forward and backward, in plain float32 FMA.
//
// This file holds the C ABI entry points of the attention stages and the
// general kernels behind them: every dtype (the float32 path always runs
// here), head_dim a power of two from 8 to 1024. A block whose keys and
// values do not fit in LDS at once is staged in tiles of keys, with the
// same arithmetic in the same order. The bf16 / fp16 MFMA kernels (attn_mfma.hip) take the shapes they
// cover and report MOBA_ERR_UNSUPPORTED otherwise, which routes here.
//
// Semantics restated:
//   attend : src/moba/kernels/moba_fwd.py:230-425 -- per column, queries x
//            the block's keys, additive tail / causal masks, m = row max of
//            q.k * D^-1/2 * log2 e, p = exp2(s - m), l = sum p, acc = p V,
//            stored at the query's fixed slot.
//   combine: moba_fwd.py:429-521 -- two passes over the slots, skipping slots
//            whose m is -inf, out = acc / l, lse = m_g + log2 l.
//   delta  : src/moba/kernels/moba_bwd.py:135-160.
//   bwd    : moba_bwd.py:216-394 -- p = exp2(s - lse), dv += p^T dO,
//            ds = p (dO V^T - delta), dk += ds^T Q D^-1/2, dq = ds K D^-1/2.
//   reduce : moba_bwd.py:398-446 -- sum of written slots.
//
// Work per column is split into groups of E entries; everything a group
// touches is staged in LDS as float32 so each product is formed once.
#include "attn_common.h"

#include <type_traits>

namespace moba {

constexpr int kE = 16;    // entries per group, forward kernel

__device__ inline float neg_inf() { return -INFINITY; }

// ---------------------------------------------------------------------------
// Forward attend.
// ---------------------------------------------------------------------------
// TILED: the block's keys, then its values, pass through LDS a tile of
// a.tile_keys at a time (head_dim above 256, or blocks too large for LDS);
// each thread then keeps the sums of its (entry, feature) elements, at most
// OWN of them, in registers across the tiles. Otherwise the whole block
// stays in LDS. Both form every score, max, sum and product in the same
// order, so their results are identical.
template <typename T, typename A, bool TILED, int OWN>
__global__ void __launch_bounds__(256)
attend_simple_kernel(AttnArgs a) {
  extern __shared__ float smem[];
  const int64_t D = a.D, bs = a.bs;
  const int64_t KT = TILED ? a.tile_keys : bs;
  // The block's keys and values stay in the input type (16-bit types take
  // half the LDS, so a 128-key block of head_dim 256 fits whole).
  T* Ks = reinterpret_cast<T*>(smem);      // [KT][D]
  T* Vs = TILED ? Ks : Ks + bs * D;        // [bs][D] (TILED: the same tile)
  float* Qs = reinterpret_cast<float*>(Ks + (TILED ? KT : 2 * bs) * D);  // [kE][D]
  float* Ss = Qs + kE * D;          // [kE][bs]
  float* Ms = Ss + kE * bs;         // [kE]
  float* Ls = Ms + kE;              // [kE]
  int* Rs = reinterpret_cast<int*>(Ls + kE);  // rows
  int* Hs = Rs + kE;                          // heads
  int* Zs = Hs + kE;                          // slots

  const Column c = resolve_column(a, blockIdx.x, blockIdx.y);
  if (c.n == 0) return;
  const T* K = static_cast<const T*>(a.k);
  const T* V = static_cast<const T*>(a.v);
  const T* Q = static_cast<const T*>(a.q);
  // Keys kt0 .. kt0 + KT - 1 of `src` into `dst` (zero past the block).
  auto stage = [&](T* dst, const T* src, int64_t kt0) {
    for (int64_t i = threadIdx.x; i < KT * D; i += blockDim.x) {
      const int64_t j = kt0 + i / D, d = i % D;
      const bool ok = j < bs && c.key0 + j < c.key_end;
      dst[i] = ok ? src[((c.tok0 + j) * a.h_kv + c.hk) * D + d] : T{};
    }
  };
  if constexpr (!TILED) {
    stage(Ks, K, 0);
    stage(Vs, V, 0);
  }
  for (int32_t e0 = 0; e0 < c.n; e0 += kE) {
    __syncthreads();
    if (threadIdx.x < kE) {
      const int32_t e = e0 + threadIdx.x;
      const bool live = e < c.n;
      Rs[threadIdx.x] = live ? a.row_indices[(c.lo + e) * a.istride] : -1;
      Hs[threadIdx.x] = live ? a.head_indices[(c.lo + e) * a.istride] : 0;
      Zs[threadIdx.x] = live ? a.slot_of_pair[(c.lo + e) * a.istride] : 0;
    }
    __syncthreads();
    for (int64_t i = threadIdx.x; i < kE * D; i += blockDim.x) {
      const int e = static_cast<int>(i / D);
      const int64_t d = i % D;
      Qs[i] = Rs[e] >= 0 ? Elem<T>::load(Q, q_offset(a, c, Rs[e], Hs[e]) + d) : 0.f;
    }
    __syncthreads();
    for (int64_t kt0 = 0; kt0 < bs; kt0 += KT) {
      if constexpr (TILED) {
        stage(Ks, K, kt0);
        __syncthreads();
      }
      for (int64_t i = threadIdx.x; i < kE * KT; i += blockDim.x) {
        const int e = static_cast<int>(i / KT);
        const int64_t jt = i % KT, j = kt0 + jt;
        if (j >= bs) continue;
        const int64_t kpos = c.key0 + j;
        float s = 0.f;
        for (int64_t d = 0; d < D; ++d) s = fmaf(Qs[e * D + d], Elem<T>::load(Ks, jt * D + d), s);
        s *= a.scale_log2;
        const bool ok = kpos < c.key_end && (!a.causal || kpos <= Rs[e]);
        Ss[e * bs + j] = ok ? s : neg_inf();
      }
      __syncthreads();
    }
    if (threadIdx.x < kE) {
      const int e = threadIdx.x;
      float m = neg_inf();
      for (int64_t j = 0; j < bs; ++j) m = fmaxf(m, Ss[e * bs + j]);
      float l = 0.f;
      for (int64_t j = 0; j < bs; ++j) {
        const float p = Ss[e * bs + j] > neg_inf() ? exp2f(Ss[e * bs + j] - m) : 0.f;
        Ss[e * bs + j] = p;
        l += p;
      }
      Ms[e] = m;
      Ls[e] = l;
      if (Rs[e] >= 0) {
        const int64_t dst = part_row(a, c, Rs[e], Hs[e]) * a.slots + Zs[e];
        *reinterpret_cast<float2*>(a.part_ml + 2 * dst) = make_float2(m, l);
      }
    }
    __syncthreads();
    A* acc_out = static_cast<A*>(a.part_acc);
    if constexpr (!TILED) {
      for (int64_t i = threadIdx.x; i < kE * D; i += blockDim.x) {
        const int e = static_cast<int>(i / D);
        const int64_t d = i % D;
        if (Rs[e] < 0) continue;
        float acc = 0.f;
        for (int64_t j = 0; j < bs; ++j) acc = fmaf(Ss[e * bs + j], Elem<T>::load(Vs, j * D + d), acc);
        const int64_t dst = part_row(a, c, Rs[e], Hs[e]) * a.slots + Zs[e];
        Elem<A>::store(acc_out, dst * D + d, acc);
      }
    } else {
      // Element i = threadIdx.x + 256 u of the group's [kE][D] outputs (kE * D
      // is a multiple of 256 at the head_dims that take this path).
      const int own = static_cast<int>(kE * D / 256);
      float acc[OWN];
#pragma unroll
      for (int u = 0; u < OWN; ++u) acc[u] = 0.f;
      for (int64_t kt0 = 0; kt0 < bs; kt0 += KT) {
        __syncthreads();  // the previous tile (or the keys) fully read
        stage(Vs, V, kt0);
        __syncthreads();
        const int64_t kn = kt0 + KT < bs ? KT : bs - kt0;
#pragma unroll
        for (int u = 0; u < OWN; ++u) {
          if (u < own) {
            const int64_t i = threadIdx.x + 256 * static_cast<int64_t>(u);
            const int e = static_cast<int>(i / D);
            const int64_t d = i % D;
            float x = acc[u];
            for (int64_t jt = 0; jt < kn; ++jt)
              x = fmaf(Ss[e * bs + kt0 + jt], Elem<T>::load(Vs, jt * D + d), x);
            acc[u] = x;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < OWN; ++u) {
        const int64_t i = threadIdx.x + 256 * static_cast<int64_t>(u);
        const int e = static_cast<int>(i / D);
        const int64_t d = i % D;
        if (u < own && Rs[e] >= 0) {
          const int64_t dst = part_row(a, c, Rs[e], Hs[e]) * a.slots + Zs[e];
          Elem<A>::store(acc_out, dst * D + d, acc[u]);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Backward: dK / dV per key tile, one program per (column, key tile).
// ---------------------------------------------------------------------------
// KT keys per tile, BE entries per group; the tile sizes shrink with
// head_dim so the float32 tiles fit in LDS.
template <typename T, int MAXD, int kKT, int kBE>
__global__ void __launch_bounds__(256)
bwd_dkdv_simple_kernel(AttnArgs a) {
  extern __shared__ float smem[];
  const int64_t D = a.D;
  float* Kt = smem;                 // [kKT][D]
  float* Vt = Kt + kKT * D;         // [kKT][D]
  float* Qs = Vt + kKT * D;         // [kBE][D]
  float* Os = Qs + kBE * D;         // [kBE][D]  (dO)
  float* Ps = Os + kBE * D;         // [kBE][kKT]
  float* Gs = Ps + kBE * kKT;       // [kBE][kKT] (dS)
  float* Lse = Gs + kBE * kKT;      // [kBE]
  float* Dl = Lse + kBE;            // [kBE]
  int* Rs = reinterpret_cast<int*>(Dl + kBE);
  int* Hs = Rs + kBE;

  const int64_t tiles = (a.bs + kKT - 1) / kKT;
  const Column c = resolve_column(a, blockIdx.x / tiles, blockIdx.y);
  const int64_t kt0 = (blockIdx.x % tiles) * kKT;
  const T* K = static_cast<const T*>(a.k);
  const T* V = static_cast<const T*>(a.v);
  const T* Q = static_cast<const T*>(a.q);
  const T* dO = static_cast<const T*>(a.dout);
  for (int64_t i = threadIdx.x; i < kKT * D; i += blockDim.x) {
    const int64_t j = i / D, d = i % D;
    const bool ok = kt0 + j < a.bs && c.key0 + kt0 + j < c.key_end;
    const int64_t off = ((c.tok0 + kt0 + j) * a.h_kv + c.hk) * D + d;
    Kt[i] = ok ? Elem<T>::load(K, off) : 0.f;
    Vt[i] = ok ? Elem<T>::load(V, off) : 0.f;
  }
  // Accumulators for the (key, feature) elements this thread owns. dK / dV
  // sum over every query of the column (thousands at long sequences): the
  // float32 path accumulates in float64 so the sum's rounding stays far
  // below its 1e-5 bar; the 16-bit paths round to 8 or 11 bits anyway.
  using Acc = typename std::conditional<sizeof(T) == 4, double, float>::type;
  constexpr int kMaxOwn = (kKT * MAXD) / 256;
  Acc dk[kMaxOwn], dv[kMaxOwn];
#pragma unroll
  for (int u = 0; u < kMaxOwn; ++u) { dk[u] = 0; dv[u] = 0; }
  const int own = static_cast<int>((kKT * D) / 256);
  for (int32_t e0 = 0; e0 < c.n; e0 += kBE) {
    __syncthreads();
    if (threadIdx.x < kBE) {
      const int32_t e = e0 + threadIdx.x;
      const bool live = e < c.n;
      const int32_t row = live ? a.row_indices[(c.lo + e) * a.istride] : -1;
      const int32_t head = live ? a.head_indices[(c.lo + e) * a.istride] : 0;
      Rs[threadIdx.x] = row;
      Hs[threadIdx.x] = head;
      Lse[threadIdx.x] = live ? a.lse_delta[2 * part_row(a, c, row, head)] : 0.f;
      Dl[threadIdx.x] = live ? a.lse_delta[2 * part_row(a, c, row, head) + 1] : 0.f;
    }
    __syncthreads();
    for (int64_t i = threadIdx.x; i < kBE * D; i += blockDim.x) {
      const int e = static_cast<int>(i / D);
      const int64_t d = i % D;
      const bool live = Rs[e] >= 0;
      const int64_t off = live ? q_offset(a, c, Rs[e], Hs[e]) + d : 0;
      Qs[i] = live ? Elem<T>::load(Q, off) : 0.f;
      Os[i] = live ? Elem<T>::load(dO, off) : 0.f;
    }
    __syncthreads();
    for (int64_t i = threadIdx.x; i < kBE * kKT; i += blockDim.x) {
      const int e = static_cast<int>(i / kKT);
      const int64_t j = i % kKT;
      const int64_t kpos = c.key0 + kt0 + j;
      float s = 0.f, dp = 0.f;
      for (int64_t d = 0; d < D; ++d) {
        s = fmaf(Qs[e * D + d], Kt[j * D + d], s);
        dp = fmaf(Os[e * D + d], Vt[j * D + d], dp);
      }
      const bool ok = Rs[e] >= 0 && kt0 + j < a.bs && kpos < c.key_end &&
                      (!a.causal || kpos <= Rs[e]);
      const float p = ok ? exp2f(s * a.scale_log2 - Lse[e]) : 0.f;
      Ps[i] = p;
      Gs[i] = p * (dp - Dl[e]);
    }
    __syncthreads();
    for (int u = 0; u < own; ++u) {
      const int64_t i = threadIdx.x + static_cast<int64_t>(u) * blockDim.x;
      const int64_t j = i / D, d = i % D;
      Acc adk = dk[u], adv = dv[u];
      for (int e = 0; e < kBE; ++e) {
        adv += static_cast<Acc>(Ps[e * kKT + j]) * static_cast<Acc>(Os[e * D + d]);
        adk += static_cast<Acc>(Gs[e * kKT + j]) * static_cast<Acc>(Qs[e * D + d]);
      }
      dk[u] = adk;
      dv[u] = adv;
    }
  }
  for (int u = 0; u < own; ++u) {
    const int64_t i = threadIdx.x + static_cast<int64_t>(u) * blockDim.x;
    const int64_t j = i / D, d = i % D;
    if (kt0 + j >= a.bs || c.key0 + kt0 + j >= c.key_end) continue;
    const int64_t off = ((c.tok0 + kt0 + j) * a.h_kv + c.hk) * D + d;
    const float gk = static_cast<float>(dk[u] * static_cast<Acc>(a.scale));
    const float gv = static_cast<float>(dv[u]);
    if (a.dkv_f32) {
      static_cast<float*>(a.dk)[off] = gk;
      static_cast<float*>(a.dv)[off] = gv;
    } else {
      Elem<T>::store(static_cast<T*>(a.dk), off, gk);
      Elem<T>::store(static_cast<T*>(a.dv), off, gv);
    }
  }
}

// ---------------------------------------------------------------------------
// Backward: per-slot dQ partials, one program per column.
// ---------------------------------------------------------------------------
// kKT keys per tile, kE entries per group, as the dK / dV kernel.
template <typename T, typename A, int MAXD, int kKT, int kE>
__global__ void __launch_bounds__(256)
bwd_dq_simple_kernel(AttnArgs a) {
  extern __shared__ float smem[];
  const int64_t D = a.D;
  float* Kt = smem;                 // [kKT][D]
  float* Vt = Kt + kKT * D;         // [kKT][D]
  float* Qs = Vt + kKT * D;         // [kE][D]
  float* Os = Qs + kE * D;          // [kE][D]
  float* Gs = Os + kE * D;          // [kE][kKT]
  float* Lse = Gs + kE * kKT;       // [kE]
  float* Dl = Lse + kE;             // [kE]
  int* Rs = reinterpret_cast<int*>(Dl + kE);
  int* Hs = Rs + kE;
  int* Zs = Hs + kE;

  const Column c = resolve_column(a, blockIdx.x, blockIdx.y);
  if (c.n == 0) return;
  const T* K = static_cast<const T*>(a.k);
  const T* V = static_cast<const T*>(a.v);
  const T* Q = static_cast<const T*>(a.q);
  const T* dO = static_cast<const T*>(a.dout);
  A* out = static_cast<A*>(a.part_acc);
  constexpr int kMaxOwn = (kE * MAXD) / 256;
  const int own = static_cast<int>((kE * D) / 256);
  for (int32_t e0 = 0; e0 < c.n; e0 += kE) {
    __syncthreads();
    if (threadIdx.x < kE) {
      const int32_t e = e0 + threadIdx.x;
      const bool live = e < c.n;
      const int32_t row = live ? a.row_indices[(c.lo + e) * a.istride] : -1;
      const int32_t head = live ? a.head_indices[(c.lo + e) * a.istride] : 0;
      Rs[threadIdx.x] = row;
      Hs[threadIdx.x] = head;
      Zs[threadIdx.x] = live ? a.slot_of_pair[(c.lo + e) * a.istride] : 0;
      Lse[threadIdx.x] = live ? a.lse_delta[2 * part_row(a, c, row, head)] : 0.f;
      Dl[threadIdx.x] = live ? a.lse_delta[2 * part_row(a, c, row, head) + 1] : 0.f;
    }
    __syncthreads();
    for (int64_t i = threadIdx.x; i < kE * D; i += blockDim.x) {
      const int e = static_cast<int>(i / D);
      const int64_t d = i % D;
      const bool live = Rs[e] >= 0;
      const int64_t off = live ? q_offset(a, c, Rs[e], Hs[e]) + d : 0;
      Qs[i] = live ? Elem<T>::load(Q, off) : 0.f;
      Os[i] = live ? Elem<T>::load(dO, off) : 0.f;
    }
    float dq[kMaxOwn];
#pragma unroll
    for (int u = 0; u < kMaxOwn; ++u) dq[u] = 0.f;
    for (int64_t kt0 = 0; kt0 < a.bs; kt0 += kKT) {
      __syncthreads();
      for (int64_t i = threadIdx.x; i < kKT * D; i += blockDim.x) {
        const int64_t j = i / D, d = i % D;
        const bool ok = kt0 + j < a.bs && c.key0 + kt0 + j < c.key_end;
        const int64_t off = ((c.tok0 + kt0 + j) * a.h_kv + c.hk) * D + d;
        Kt[i] = ok ? Elem<T>::load(K, off) : 0.f;
        Vt[i] = ok ? Elem<T>::load(V, off) : 0.f;
      }
      __syncthreads();
      for (int64_t i = threadIdx.x; i < kE * kKT; i += blockDim.x) {
        const int e = static_cast<int>(i / kKT);
        const int64_t j = i % kKT;
        const int64_t kpos = c.key0 + kt0 + j;
        float s = 0.f, dp = 0.f;
        for (int64_t d = 0; d < D; ++d) {
          s = fmaf(Qs[e * D + d], Kt[j * D + d], s);
          dp = fmaf(Os[e * D + d], Vt[j * D + d], dp);
        }
        const bool ok = Rs[e] >= 0 && kt0 + j < a.bs && kpos < c.key_end &&
                        (!a.causal || kpos <= Rs[e]);
        const float p = ok ? exp2f(s * a.scale_log2 - Lse[e]) : 0.f;
        Gs[i] = p * (dp - Dl[e]);
      }
      __syncthreads();
      for (int u = 0; u < own; ++u) {
        const int64_t i = threadIdx.x + static_cast<int64_t>(u) * blockDim.x;
        const int e = static_cast<int>(i / D);
        const int64_t d = i % D;
        float acc = dq[u];
        for (int64_t j = 0; j < kKT; ++j) acc = fmaf(Gs[e * kKT + j], Kt[j * D + d], acc);
        dq[u] = acc;
      }
    }
    for (int u = 0; u < own; ++u) {
      const int64_t i = threadIdx.x + static_cast<int64_t>(u) * blockDim.x;
      const int e = static_cast<int>(i / D);
      const int64_t d = i % D;
      if (Rs[e] < 0) continue;
      const int64_t dst = part_row(a, c, Rs[e], Hs[e]) * a.slots + Zs[e];
      Elem<A>::store(out, dst * D + d, dq[u] * a.scale);
    }
  }
}

// ---------------------------------------------------------------------------
// Row-wise passes: combine, delta, dq reduce.
// ---------------------------------------------------------------------------
// Eight consecutive elements as floats / from floats (16-byte accesses for
// 16-bit types). The partial rows are streamed once, so the 16-bit loads
// and stores are non-temporal (they do not displace reused lines from the
// caches; combine and dQ reduce took 11-14% off at the 512K workload).
template <typename A>
__device__ inline void load8(const A* p, float (&x)[8]) {
  typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
  const u32x4_nt w = __builtin_nontemporal_load(reinterpret_cast<const u32x4_nt*>(p));
  const uint4 u = __builtin_bit_cast(uint4, w);
  const uint16_t* e = reinterpret_cast<const uint16_t*>(&u);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = Elem<A>::load(reinterpret_cast<const A*>(e), i);
}
template <>
__device__ inline void load8<float>(const float* p, float (&x)[8]) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
// 16-bit stores round to nearest even by the hardware conversions
// (v_cvt_pk_bf16_f32, v_cvt_f16_f32): the integer rounding of common.h for
// every finite input, without its per-value branches.
template <typename A>
__device__ inline void store8(A* p, const float (&x)[8]);
template <>
__device__ inline void store8<bf16_t>(bf16_t* p, const float (&x)[8]) {
  typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
  typedef float f32x8_t __attribute__((ext_vector_type(8)));
  typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
  const f32x8_t v = {x[0], x[1], x[2], x[3], x[4], x[5], x[6], x[7]};
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_nt, __builtin_convertvector(v, bf16x8_t)),
                              reinterpret_cast<u32x4_nt*>(p));
}
template <>
__device__ inline void store8<f16_t>(f16_t* p, const float (&x)[8]) {
  typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
  typedef unsigned int u32x4_nt __attribute__((ext_vector_type(4)));
  f16x8_t h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = static_cast<_Float16>(x[i]);
  __builtin_nontemporal_store(__builtin_bit_cast(u32x4_nt, h), reinterpret_cast<u32x4_nt*>(p));
}
template <>
__device__ inline void store8<float>(float* p, const float (&x)[8]) {
  *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(x[4], x[5], x[6], x[7]);
}

// One lane per (query, 8 features). Two passes over the slots, as in the
// reference merge: the global max, then the rescaled sums.
// One lane per (query, 8 features). K > 0 fixes the slot count at compile
// time: every slot's partial row is then requested before the first is
// used (the addresses are valid whether or not the slot was written, and an
// unwritten slot's values are selected away, never multiplied in), so a lane
// keeps K loads in flight. K = 0 loops over `slots` at run time.
template <typename A, typename O, int K>
__global__ void __launch_bounds__(256)
combine_kernel(const float* __restrict__ part_ml, const A* __restrict__ part_acc, O* __restrict__ out, float* __restrict__ lse,
               int64_t n_rows, int64_t S, int64_t h_q, int64_t D, int64_t slots) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per_row = D / 8;
  const int64_t row = gid / per_row;     // head-major (b * Hq + h) * S + t
  const int64_t d0 = (gid % per_row) * 8;
  if (row >= n_rows) return;
  const float* ml = part_ml + row * slots * 2;  // (m, l) per slot
  float m_g = -INFINITY;
  float ls = 0.f;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if constexpr (K > 0) {
    float2 st[K];
    float x[K][8];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      {
        typedef float f32x2_nt __attribute__((ext_vector_type(2)));
        const f32x2_nt t = __builtin_nontemporal_load(reinterpret_cast<const f32x2_nt*>(ml + 2 * j));
        st[j] = make_float2(t[0], t[1]);
      }
      load8<A>(part_acc + (row * K + j) * D + d0, x[j]);
    }
#pragma unroll
    for (int j = 0; j < K; ++j) m_g = fmaxf(m_g, st[j].x);
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const bool ok = st[j].x > -INFINITY;
      const float w = ok ? exp2f(st[j].x - m_g) : 0.f;
      ls += ok ? st[j].y * w : 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += (ok ? x[j][i] : 0.f) * w;
    }
  } else {
    for (int64_t j = 0; j < slots; ++j) m_g = fmaxf(m_g, ml[2 * j]);
    for (int64_t j = 0; j < slots; ++j) {
      const float mi = ml[2 * j];
      if (mi > -INFINITY) {
        const float w = exp2f(mi - m_g);
        ls += ml[2 * j + 1] * w;
        float x[8];
        load8<A>(part_acc + (row * slots + j) * D + d0, x);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += x[i] * w;
      }
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = acc[i] / ls;  // l == 0 (index bug) -> NaN, loudly
  const int64_t bh = row / S, t = row % S;
  const int64_t b = bh / h_q, h = bh % h_q;
  store8<O>(out + ((b * S + t) * h_q + h) * D + d0, acc);
  if (lse && d0 == 0) lse[row] = m_g + log2f(ls);
}

// delta[row] = sum_d O[row, d] * dO[row, d]. L lanes own one token-major
// row (C chunks of 8 features each, one vector load per tensor and chunk),
// so a wave streams 64 / L whole rows per instruction; the L partial sums
// meet by shuffles.
template <typename T, int L, int C>
__global__ void __launch_bounds__(256)
delta_kernel(const T* __restrict__ o, const T* __restrict__ dout, const float* __restrict__ lse,
             float* __restrict__ delta, int64_t n_rows, int64_t S, int64_t h_q) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t row = gid / L;  // token-major: (b * S + t) * h_q + h
  const int sub = static_cast<int>(gid % L);
  float acc = 0.f;
  if (row < n_rows) {
#pragma unroll
    for (int ch = 0; ch < C; ++ch) {
      float x[8], y[8];
      load8<T>(o + row * (8 * L * C) + 8 * (sub + L * ch), x);
      load8<T>(dout + row * (8 * L * C) + 8 * (sub + L * ch), y);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc = fmaf(x[i], y[i], acc);
    }
  }
#pragma unroll
  for (int w = L / 2; w > 0; w >>= 1) acc += __shfl_xor(acc, w);
  if (row < n_rows && sub == 0) {
    const int64_t h = row % h_q, bt = row / h_q;
    const int64_t hm = (bt / S * h_q + h) * S + bt % S;
    if (lse) *reinterpret_cast<float2*>(delta + 2 * hm) = make_float2(lse[hm], acc);
    else delta[hm] = acc;
  }
}

// One lane per (query, 8 features); a slot counts only if the forward wrote
// it (part_m > -inf), so unwritten dq partials never reach the sum. K as in
// combine_kernel: with K > 0 every slot's row is requested up front (and an
// unwritten slot's values selected away); K = 0 loops at run time and
// reads only the written slots.
template <typename A, typename O, int K>
__global__ void __launch_bounds__(256)
dq_reduce_kernel(const A* __restrict__ dq_part, const float* __restrict__ part_m,
                 int64_t m_stride, O* __restrict__ dq, int64_t n_rows, int64_t S,
                 int64_t h_q, int64_t D, int64_t slots) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t per_row = D / 8;
  const int64_t row = gid / per_row;
  const int64_t d0 = (gid % per_row) * 8;
  if (row >= n_rows) return;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  if constexpr (K > 0) {
    float mk[K];
    float x[K][8];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      mk[j] = __builtin_nontemporal_load(part_m + (row * K + j) * m_stride);
      load8<A>(dq_part + (row * K + j) * D + d0, x[j]);
    }
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const bool ok = mk[j] > -INFINITY;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[i] += ok ? x[j][i] : 0.f;
    }
  } else {
    for (int64_t j = 0; j < slots; ++j)
      if (part_m[(row * slots + j) * m_stride] > -INFINITY) {
        float x[8];
        load8<A>(dq_part + (row * slots + j) * D + d0, x);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] += x[i];
      }
  }
  const int64_t bh = row / S, t = row % S;
  const int64_t b = bh / h_q, h = bh % h_q;
  store8<O>(dq + ((b * S + t) * h_q + h) * D + d0, acc);
}

// dK / dV of the cut columns: the column's segments' float32 sums (scratch
// slots x .. x + nseg - 1, [2][BS][D] each) added in segment order, written
// in the input dtype. One workgroup per cut column of a (row, kv head).
template <typename T>
__global__ void __launch_bounds__(256)
seg_finish_kernel(AttnArgs a) {
  const int64_t rh = blockIdx.y;
  const int64_t extra_cap = a.seg_cap - a.n_blocks;
  if (static_cast<int64_t>(blockIdx.x) >= a.seg_counts[2 * rh + 1]) return;
  const int32_t first = a.seg_split[rh * extra_cap + blockIdx.x];
  const Column c = resolve_column(a, first, rh);
  const int64_t bsd = a.bs * a.D;
  const float* base = a.seg_scratch + (rh * a.scratch_cap + c.scratch) * 2 * bsd;
  const int key_lim = static_cast<int>(c.key_end - c.key0);
  T* dK = static_cast<T*>(a.dk);
  T* dV = static_cast<T*>(a.dv);
  // Thread -> (key, four features): D / 4 threads per key row (the MFMA
  // backward, the only producer of segments, has D of 64 or 128).
  const int v4 = static_cast<int>(a.D / 4);
  const int per = static_cast<int>(blockDim.x) / v4;
  const int c4 = static_cast<int>(threadIdx.x) % v4;
  for (int key = static_cast<int>(threadIdx.x) / v4; key < key_lim; key += per) {
    const int64_t i = static_cast<int64_t>(key) * a.D + 4 * c4;
    float4 sk = make_float4(0.f, 0.f, 0.f, 0.f), sv = sk;
    for (int j = 0; j < c.nseg; ++j) {
      const float4 x = *reinterpret_cast<const float4*>(base + j * 2 * bsd + i);
      const float4 y = *reinterpret_cast<const float4*>(base + j * 2 * bsd + bsd + i);
      sk.x += x.x; sk.y += x.y; sk.z += x.z; sk.w += x.w;
      sv.x += y.x; sv.y += y.y; sv.z += y.z; sv.w += y.w;
    }
    const int64_t off = ((c.tok0 + key) * a.h_kv + c.hk) * a.D + 4 * c4;
    if (a.dkv_f32) {
      *reinterpret_cast<float4*>(static_cast<float*>(a.dk) + off) = sk;
      *reinterpret_cast<float4*>(static_cast<float*>(a.dv) + off) = sv;
      continue;
    }
    Elem<T>::store(dK, off, sk.x); Elem<T>::store(dK, off + 1, sk.y);
    Elem<T>::store(dK, off + 2, sk.z); Elem<T>::store(dK, off + 3, sk.w);
    Elem<T>::store(dV, off, sv.x); Elem<T>::store(dV, off + 1, sv.y);
    Elem<T>::store(dV, off + 2, sv.z); Elem<T>::store(dV, off + 3, sv.w);
  }
}

__global__ void __launch_bounds__(256)
fill_f32_kernel(float* __restrict__ p, int64_t n, float value) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x)
    p[i] = value;
}

// ---------------------------------------------------------------------------
// Host side.
// ---------------------------------------------------------------------------
static int prepare_attn(AttnArgs* a, Geometry* g, const void* q, const void* k,
                        const void* v, const int32_t* col_nnz, const int32_t* col_offsets,
                        const int32_t* row_indices, const int32_t* head_indices,
                        const int32_t* slot_of_pair, const int32_t* order,
                        const int32_t* cu, int64_t batch, int64_t seq_len,
                        int64_t max_seqlen, int64_t h_q, int64_t h_kv, int64_t head_dim,
                        int64_t n_blocks, int64_t block_size, int64_t slots,
                        int64_t index_cap, int64_t index_stride, int causal) {
  int st = make_geometry(g, batch, seq_len, max_seqlen, h_q, h_kv, head_dim, n_blocks,
                         block_size, slots, cu);
  if (st) return st;
  if (!q || !k || !v || !col_nnz || !col_offsets || !row_indices || !head_indices ||
      !slot_of_pair || !order)
    return fail(MOBA_ERR_INVALID, "null pointer");
  if (slots <= 0) return fail(MOBA_ERR_INVALID, "slots must be positive");
  if (index_cap < g->group * g->rows_per_seq * slots)
    return fail(MOBA_ERR_INVALID, "index capacity below group * rows * slots");
  if (index_stride < 1) return fail(MOBA_ERR_INVALID, "index_stride must be positive");
  if (head_dim & (head_dim - 1))
    return fail(MOBA_ERR_UNSUPPORTED, "head_dim must be a power of two");
  *a = AttnArgs{};
  a->q = q; a->k = k; a->v = v;
  a->col_nnz = col_nnz; a->col_offsets = col_offsets; a->row_indices = row_indices;
  a->head_indices = head_indices; a->slot_of_pair = slot_of_pair; a->order = order;
  a->istride = index_stride;
  a->cu = cu;
  a->S = seq_len; a->h_q = h_q; a->h_kv = h_kv; a->D = head_dim; a->n_blocks = n_blocks;
  a->bs = block_size; a->slots = slots; a->cap = index_cap; a->causal = causal ? 1 : 0;
  a->scale = 1.0f / sqrtf(static_cast<float>(head_dim));
  a->scale_log2 = a->scale * 1.4426950408889634f;
  return MOBA_OK;
}

// Segment list of moba_csc_build (null: one program per whole column).
static int set_segments(AttnArgs* a, const int32_t* segments, const int32_t* seg_split,
                        const int32_t* seg_counts, int64_t seg_cap) {
  if (!segments) return MOBA_OK;
  if (!seg_split || !seg_counts || seg_cap < a->n_blocks)
    return fail(MOBA_ERR_INVALID, "segment list: need split / counts and seg_cap >= n_blocks");
  a->seg = segments;
  a->seg_split = seg_split;
  a->seg_counts = seg_counts;
  a->seg_cap = seg_cap;
  return MOBA_OK;
}

// The FMA kernels take head_dim 8..1024 (a power of two).
static bool simple_shape_ok(const Geometry& g) {
  return g.head_dim <= 1024 && g.head_dim >= 8;
}

template <typename K>
static int set_lds(K kernel, size_t bytes) {
  if (bytes > 160 * 1024) return fail(MOBA_ERR_UNSUPPORTED, "tile exceeds LDS");
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize,
                                     static_cast<int>(bytes));
  if (e != hipSuccess) return fail(MOBA_ERR_LAUNCH, hipGetErrorString(e));
  return MOBA_OK;
}

#define MOBA_DISPATCH_ACC(code, A, ...)                                   \
  [&]() -> int {                                                          \
    switch (code) {                                                       \
      case MOBA_BF16: { using A = ::moba::bf16_t; return __VA_ARGS__(); } \
      case MOBA_FP16: { using A = ::moba::f16_t; return __VA_ARGS__(); }  \
      case MOBA_FP32: { using A = float; return __VA_ARGS__(); }          \
      default:                                                            \
        return ::moba::fail(MOBA_ERR_UNSUPPORTED, "unknown dtype code");  \
    }                                                                     \
  }()

}  // namespace moba

extern "C" int moba_attend(const void* q, const void* k, const void* v,
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
                           int causal, int dtype, int acc_dtype, void* stream) {
  using namespace moba;
  AttnArgs a;
  Geometry g;
  int st = prepare_attn(&a, &g, q, k, v, col_nnz, col_offsets, row_indices, head_indices,
                        slot_of_pair, order, cu_seqlens, batch, seq_len, max_seqlen, h_q,
                        h_kv, head_dim, n_blocks, block_size, slots, index_cap,
                        index_stride, causal);
  if (st) return st;
  if (!part_ml || !part_acc) return fail(MOBA_ERR_INVALID, "null partials");
  a.part_ml = part_ml; a.part_acc = part_acc;
  st = set_segments(&a, segments, seg_split, seg_counts, seg_cap);
  if (st) return st;
  hipStream_t s = as_stream(stream);
  // Unwritten slots must read as m = -inf: the marker combine and dq reduce
  // rely on. The (m, l) pairs are cleared whole; l / acc of such slots are
  // never read.
  const int64_t n_m = (g.packed ? 1 : batch) * h_q * seq_len * slots * 2;
  hipLaunchKernelGGL(fill_f32_kernel, dim3(static_cast<unsigned>(cdiv(n_m, 256) < 8192 ? cdiv(n_m, 256) : 8192)),
                     dim3(256), 0, s, part_ml, n_m, -INFINITY);
  st = check_launch("moba_attend (fill)");
  if (st) return st;
  st = attend_mfma(a, dtype, acc_dtype, batch * h_kv, s);
  if (st != MOBA_ERR_UNSUPPORTED) return st;
  a.seg = nullptr;  // the FMA kernels take whole columns
  if (!simple_shape_ok(g))
    return fail(MOBA_ERR_UNSUPPORTED, "attend: head_dim must be in [8, 1024]");
  const size_t esize = dtype == MOBA_FP32 ? 4 : 2;
  constexpr size_t kLds = 160 * 1024;
  // Queries, scores and row statistics of a group; then the block's keys
  // and values whole, or tiles of keys when they do not fit.
  const size_t fixed = sizeof(float) * (kE * head_dim + kE * block_size + 2 * kE) +
                       sizeof(int) * 3 * kE;
  const size_t whole = fixed + esize * 2 * block_size * head_dim;
  int64_t kt = 0;
  if (whole > kLds) {
    for (kt = 1; kt * 2 <= block_size && fixed + esize * 2 * kt * head_dim <= kLds;) kt *= 2;
    if (fixed + esize * kt * head_dim > kLds)
      return fail(MOBA_ERR_UNSUPPORTED,
                  "attend: a group's queries and scores exceed LDS (4 * 16 * (head_dim + "
                  "block_size) bytes above about 160 KiB)");
  }
  a.tile_keys = static_cast<int>(kt);
  const size_t lds = kt ? fixed + esize * kt * head_dim : whole;
  dim3 grid(static_cast<unsigned>(n_blocks), static_cast<unsigned>(batch * h_kv));
  return MOBA_DISPATCH_DTYPE(dtype, T, [&] {
    return MOBA_DISPATCH_ACC(acc_dtype, A, [&] {
      auto go = [&](auto kernel) {
        int rc = set_lds(kernel, lds);
        if (rc) return rc;
        hipLaunchKernelGGL(kernel, grid, dim3(256), lds, s, a);
        return check_launch("moba_attend");
      };
      if (!kt) return go(attend_simple_kernel<T, A, false, 1>);
      if (head_dim <= 256) return go(attend_simple_kernel<T, A, true, 16>);
      if (head_dim <= 512) return go(attend_simple_kernel<T, A, true, 32>);
      return go(attend_simple_kernel<T, A, true, 64>);
    });
  });
}

extern "C" int moba_combine(const float* part_ml, const void* part_acc,
                            void* out, float* lse, int64_t batch, int64_t seq_len,
                            int64_t h_q, int64_t head_dim, int64_t slots, int acc_dtype,
                            int out_dtype, void* stream) {
  using namespace moba;
  if (batch <= 0 || seq_len <= 0 || h_q <= 0 || head_dim <= 0 || slots <= 0)
    return fail(MOBA_ERR_INVALID, "non-positive shape argument");
  if (!part_ml || !part_acc || !out) return fail(MOBA_ERR_INVALID, "null pointer");
  if (head_dim % 8) return fail(MOBA_ERR_UNSUPPORTED, "head_dim must be a multiple of 8");
  const int64_t n_rows = batch * h_q * seq_len;
  dim3 grid(static_cast<unsigned>(cdiv(n_rows * (head_dim / 8), 256)));
  return MOBA_DISPATCH_ACC(acc_dtype, A, [&] {
    return MOBA_DISPATCH_DTYPE(out_dtype, O, [&] {
      auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, as_stream(stream), part_ml,
                           static_cast<const A*>(part_acc), static_cast<O*>(out), lse, n_rows,
                           seq_len, h_q, head_dim, slots);
      };
      if (slots == 8) go(combine_kernel<A, O, 8>);
      else if (slots == 16) go(combine_kernel<A, O, 16>);
      else go(combine_kernel<A, O, 0>);
      return check_launch("moba_combine");
    });
  });
}

extern "C" int moba_bwd_delta(const void* out, const void* dout, const float* lse,
                              float* delta, int64_t batch, int64_t seq_len, int64_t h_q,
                              int64_t head_dim, int dtype, void* stream) {
  using namespace moba;
  if (batch <= 0 || seq_len <= 0 || h_q <= 0 || head_dim <= 0)
    return fail(MOBA_ERR_INVALID, "non-positive shape argument");
  if (!out || !dout || !delta) return fail(MOBA_ERR_INVALID, "null pointer");
  const int64_t n_rows = batch * h_q * seq_len;
  const int64_t chunks = head_dim / 8;
  if (head_dim % 8 != 0 || chunks > 128 || (chunks & (chunks - 1)) != 0)
    return fail(MOBA_ERR_UNSUPPORTED, "delta: head_dim must be 8 times a power of two <= 1024");
  const int64_t lanes = chunks < 64 ? chunks : 64;  // a row spans at most one wave
  dim3 grid(static_cast<unsigned>(cdiv(n_rows * lanes, 256)));
  return MOBA_DISPATCH_DTYPE(dtype, T, [&] {
    auto go = [&](auto lanes_c) {
      constexpr int Lc = decltype(lanes_c)::value;
      if (Lc == 64 && chunks == 128)
        hipLaunchKernelGGL((delta_kernel<T, 64, 2>), grid, dim3(256), 0, as_stream(stream),
                           static_cast<const T*>(out), static_cast<const T*>(dout), lse,
                           delta, n_rows, seq_len, h_q);
      else
        hipLaunchKernelGGL((delta_kernel<T, Lc, 1>), grid, dim3(256), 0, as_stream(stream),
                           static_cast<const T*>(out), static_cast<const T*>(dout), lse,
                           delta, n_rows, seq_len, h_q);
    };
    switch (lanes) {
      case 1: go(std::integral_constant<int, 1>{}); break;
      case 2: go(std::integral_constant<int, 2>{}); break;
      case 4: go(std::integral_constant<int, 4>{}); break;
      case 8: go(std::integral_constant<int, 8>{}); break;
      case 16: go(std::integral_constant<int, 16>{}); break;
      case 32: go(std::integral_constant<int, 32>{}); break;
      default: go(std::integral_constant<int, 64>{}); break;
    }
    return check_launch("moba_bwd_delta");
  });
}

extern "C" int moba_bwd(const void* q, const void* k, const void* v, const void* dout,
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
                        int acc_dtype, int dkv_dtype, void* stream) {
  using namespace moba;
  AttnArgs a;
  Geometry g;
  int st = prepare_attn(&a, &g, q, k, v, col_nnz, col_offsets, row_indices, head_indices,
                        slot_of_pair, order, cu_seqlens, batch, seq_len, max_seqlen, h_q,
                        h_kv, head_dim, n_blocks, block_size, slots, index_cap,
                        index_stride, causal);
  if (st) return st;
  if (!dout || !lse_delta || !dk || !dv || !dq_part)
    return fail(MOBA_ERR_INVALID, "null pointer");
  a.dout = dout; a.lse_delta = lse_delta; a.dk = dk; a.dv = dv; a.part_acc = dq_part;
  if (dkv_dtype != dtype && dkv_dtype != MOBA_FP32)
    return fail(MOBA_ERR_INVALID, "dkv_dtype must be the input dtype or float32");
  a.dkv_f32 = dkv_dtype == MOBA_FP32 && dtype != MOBA_FP32;
  st = set_segments(&a, segments, seg_split, seg_counts, seg_cap);
  if (st) return st;
  if (a.seg) {
    if (!seg_scratch || scratch_cap < 2 * (seg_cap - n_blocks))
      return fail(MOBA_ERR_INVALID, "segment scratch: need scratch_cap >= 2 * (seg_cap - n_blocks)");
    a.seg_scratch = seg_scratch;
    a.scratch_cap = scratch_cap;
  }
  hipStream_t s = as_stream(stream);
  st = bwd_mfma(a, dtype, acc_dtype, batch * h_kv, s);
  if (st == MOBA_OK && a.seg && seg_cap > n_blocks) {
    dim3 fgrid(static_cast<unsigned>(seg_cap - n_blocks), static_cast<unsigned>(batch * h_kv));
    st = MOBA_DISPATCH_DTYPE(dtype, T, [&] {
      hipLaunchKernelGGL(seg_finish_kernel<T>, fgrid, dim3(256), 0, s, a);
      return check_launch("moba_bwd (cut columns)");
    });
  }
  if (st != MOBA_ERR_UNSUPPORTED) return st;
  a.seg = nullptr;  // the FMA kernels take whole columns
  if (head_dim > 1024 || head_dim < 8)
    return fail(MOBA_ERR_UNSUPPORTED, "backward: head_dim must be in [8, 1024]");
  // Keys per tile and entries per group of the two kernels: float32 tiles
  // of K, V, Q and dO must fit in LDS, so they shrink with head_dim.
  const int kt_kv = head_dim <= 256 ? 32 : (head_dim <= 512 ? 16 : 8);
  const int be_kv = kt_kv;
  const int kt_q = kt_kv;
  const int e_q = head_dim <= 256 ? 16 : 8;
  const int64_t tiles = cdiv(block_size, kt_kv);
  const size_t lds_kv = sizeof(float) * (2 * kt_kv * head_dim + 2 * be_kv * head_dim +
                                         2 * be_kv * kt_kv + 2 * be_kv) + sizeof(int) * 2 * be_kv;
  const size_t lds_q = sizeof(float) * (2 * kt_q * head_dim + 2 * e_q * head_dim +
                                        e_q * kt_q + 2 * e_q) + sizeof(int) * 3 * e_q;
  return MOBA_DISPATCH_DTYPE(dtype, T, [&] {
    return MOBA_DISPATCH_ACC(acc_dtype, A, [&] {
      auto run = [&](auto dkdv_kernel, auto dq_kernel) {
        int rc = set_lds(dkdv_kernel, lds_kv);
        if (rc) return rc;
        rc = set_lds(dq_kernel, lds_q);
        if (rc) return rc;
        hipLaunchKernelGGL(dkdv_kernel,
                           dim3(static_cast<unsigned>(n_blocks * tiles),
                                static_cast<unsigned>(batch * h_kv)),
                           dim3(256), lds_kv, s, a);
        rc = check_launch("moba_bwd (dk/dv)");
        if (rc) return rc;
        hipLaunchKernelGGL(dq_kernel,
                           dim3(static_cast<unsigned>(n_blocks), static_cast<unsigned>(batch * h_kv)),
                           dim3(256), lds_q, s, a);
        return check_launch("moba_bwd (dq)");
      };
      if (head_dim <= 128)
        return run(bwd_dkdv_simple_kernel<T, 128, 32, 32>, bwd_dq_simple_kernel<T, A, 128, 32, 16>);
      if (head_dim <= 256)
        return run(bwd_dkdv_simple_kernel<T, 256, 32, 32>, bwd_dq_simple_kernel<T, A, 256, 32, 16>);
      if (head_dim <= 512)
        return run(bwd_dkdv_simple_kernel<T, 512, 16, 16>, bwd_dq_simple_kernel<T, A, 512, 16, 8>);
      return run(bwd_dkdv_simple_kernel<T, 1024, 8, 8>, bwd_dq_simple_kernel<T, A, 1024, 8, 8>);
    });
  });
}

extern "C" int moba_dq_reduce(const void* dq_part, const float* part_m, int64_t m_stride,
                              void* dq,
                              int64_t batch, int64_t seq_len, int64_t h_q, int64_t head_dim,
                              int64_t slots, int acc_dtype, int out_dtype, void* stream) {
  using namespace moba;
  if (batch <= 0 || seq_len <= 0 || h_q <= 0 || head_dim <= 0 || slots <= 0)
    return fail(MOBA_ERR_INVALID, "non-positive shape argument");
  if (!dq_part || !part_m || !dq) return fail(MOBA_ERR_INVALID, "null pointer");
  if (m_stride < 1) return fail(MOBA_ERR_INVALID, "m_stride must be positive");
  if (head_dim % 8) return fail(MOBA_ERR_UNSUPPORTED, "head_dim must be a multiple of 8");
  const int64_t n_rows = batch * h_q * seq_len;
  dim3 grid(static_cast<unsigned>(cdiv(n_rows * (head_dim / 8), 256)));
  return MOBA_DISPATCH_ACC(acc_dtype, A, [&] {
    return MOBA_DISPATCH_DTYPE(out_dtype, O, [&] {
      auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, dim3(256), 0, as_stream(stream),
                           static_cast<const A*>(dq_part), part_m, m_stride,
                           static_cast<O*>(dq), n_rows, seq_len, h_q, head_dim, slots);
      };
      if (slots == 8) go(dq_reduce_kernel<A, O, 8>);
      else if (slots == 16) go(dq_reduce_kernel<A, O, 16>);
      else go(dq_reduce_kernel<A, O, 0>);
      return check_launch("moba_dq_reduce");
    });
  });
}
