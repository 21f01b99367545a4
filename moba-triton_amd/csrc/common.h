// Shared device/host helpers for the MoBA gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "moba_hip.h"

namespace moba {

__host__ __device__ inline uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ inline float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// ---------------------------------------------------------------------------
// Element types. Storage is raw bits; arithmetic is float.
// ---------------------------------------------------------------------------

struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

__host__ __device__ inline float bf16_to_float(uint16_t b) {
  return u2f(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even float -> bf16 (NaN kept quiet).
__host__ __device__ inline uint16_t float_to_bf16(float f) {
  uint32_t u = f2u(f);
  if ((u & 0x7f800000u) == 0x7f800000u) {
    if (u & 0x007fffffu) u |= 0x00400000u;
    return static_cast<uint16_t>(u >> 16);
  }
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

// IEEE binary16 <-> float in integer arithmetic, so the result never depends
// on the wave's denormal mode (fp16 subnormals are common in pooled means).
__host__ __device__ inline float f16_to_float(uint16_t h) {
  const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  if (e == 0) {
    // m * 2^-24 is a normal float: exact in any denormal mode.
    const float v = static_cast<float>(m) * 5.9604644775390625e-8f;
    return u2f(f2u(v) | sign);
  }
  if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

// Round-to-nearest-even float -> binary16 (overflow to inf, NaN kept quiet).
__host__ __device__ inline uint16_t float_to_f16(float f) {
  const uint32_t u = f2u(f);
  const uint16_t sign = static_cast<uint16_t>((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00u;            // NaN
  if (a >= 0x477ff000u) return sign | 0x7c00u;           // >= 65520 -> inf
  if (a >= 0x38800000u) {                                // normal range
    uint32_t r = a - 0x38000000u;                        // rebias 127 -> 15
    r += 0xfffu + ((r >> 13) & 1u);
    return sign | static_cast<uint16_t>(r >> 13);
  }
  if (a < 0x33000000u) return sign;                      // below 2^-25: zero
  const uint32_t e = a >> 23;                            // subnormal result
  const uint32_t m = (a & 0x7fffffu) | 0x800000u;
  const uint32_t shift = 126u - e;                       // in [14, 24]
  uint32_t q = m >> shift;
  const uint32_t rem = m & ((1u << shift) - 1u);
  const uint32_t half = 1u << (shift - 1u);
  if (rem > half || (rem == half && (q & 1u))) ++q;
  return sign | static_cast<uint16_t>(q);
}

template <typename T> struct Elem;
template <> struct Elem<bf16_t> {
  static constexpr int kCode = MOBA_BF16;
  __device__ static float load(const bf16_t* p, int64_t i) { return bf16_to_float(p[i].bits); }
  __device__ static void store(bf16_t* p, int64_t i, float v) { p[i].bits = float_to_bf16(v); }
  __device__ static float round(float v) { return bf16_to_float(float_to_bf16(v)); }
};
template <> struct Elem<f16_t> {
  static constexpr int kCode = MOBA_FP16;
  __device__ static float load(const f16_t* p, int64_t i) { return f16_to_float(p[i].bits); }
  __device__ static void store(f16_t* p, int64_t i, float v) { p[i].bits = float_to_f16(v); }
  __device__ static float round(float v) { return f16_to_float(float_to_f16(v)); }
};
template <> struct Elem<float> {
  static constexpr int kCode = MOBA_FP32;
  __device__ static float load(const float* p, int64_t i) { return p[i]; }
  __device__ static void store(float* p, int64_t i, float v) { p[i] = v; }
  __device__ static float round(float v) { return v; }
};

// ---------------------------------------------------------------------------
// Host-side error plumbing.
// ---------------------------------------------------------------------------

void set_error(const std::string& msg);
int fail(int status, const std::string& msg);
int check_launch(const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Geometry shared by every stage. `rows` is the batch (padded) or the
// sequence count (packed); `rows_per_seq` is S (padded) or max_seqlen.
struct Geometry {
  int64_t rows;
  int64_t seq_len;       // S, or packed token count T
  int64_t rows_per_seq;  // S, or max_seqlen
  int64_t h_q, h_kv, group, head_dim, n_blocks, block_size, slots;
  bool packed;
};

int make_geometry(Geometry* g, int64_t batch, int64_t seq_len,
                  int64_t max_seqlen, int64_t h_q, int64_t h_kv,
                  int64_t head_dim, int64_t n_blocks, int64_t block_size,
                  int64_t slots, const int32_t* cu_seqlens);

// Device view of where a sequence lives. Padded: sequence r is batch row r,
// tokens [r*S, r*S + S). Packed: tokens [cu[r], cu[r+1]).
struct SeqSpan {
  int64_t bos;  // first token (global token index)
  int64_t len;
};

__device__ inline SeqSpan seq_span(const int32_t* cu, int64_t r, int64_t S) {
  SeqSpan s;
  if (cu) {
    s.bos = cu[r];
    s.len = static_cast<int64_t>(cu[r + 1]) - s.bos;
  } else {
    s.bos = r * S;
    s.len = S;
  }
  return s;
}

}  // namespace moba

// Dispatch on a runtime dtype code to a template taking the element type.
#define MOBA_DISPATCH_DTYPE(code, T, ...)                                  \
  [&]() -> int {                                                          \
    switch (code) {                                                       \
      case MOBA_BF16: { using T = ::moba::bf16_t; return __VA_ARGS__(); } \
      case MOBA_FP16: { using T = ::moba::f16_t; return __VA_ARGS__(); }  \
      case MOBA_FP32: { using T = float; return __VA_ARGS__(); }          \
      default:                                                            \
        return ::moba::fail(MOBA_ERR_UNSUPPORTED, "unknown dtype code");  \
    }                                                                     \
  }()
