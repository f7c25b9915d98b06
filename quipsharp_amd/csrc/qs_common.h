// Shared definitions for the gfx950 QuIP# kernels: status plumbing, the two
// codebook tables (generated at compile time into __constant__ memory), and
// small device helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/quipsharp_hip.h"

namespace qs {

// ----------------------------------------------------------------------------
// status
// ----------------------------------------------------------------------------
void set_error(const char* fmt, ...);
int hip_status(hipError_t e, const char* what);

#define QS_REQUIRE(cond, ...)                                 \
  do {                                                        \
    if (!(cond)) {                                            \
      ::qs::set_error(__VA_ARGS__);                           \
      return QS_ERR_INVALID;                                  \
    }                                                         \
  } while (0)

#define QS_SUPPORTED(cond, ...)                               \
  do {                                                        \
    if (!(cond)) {                                            \
      ::qs::set_error(__VA_ARGS__);                           \
      return QS_ERR_UNSUPPORTED;                              \
    }                                                         \
  } while (0)

#define QS_HIP(expr)                                          \
  do {                                                        \
    hipError_t e_ = (expr);                                   \
    if (e_ != hipSuccess) return ::qs::hip_status(e_, #expr); \
  } while (0)

#define QS_LAUNCHED(name)                                     \
  do {                                                        \
    hipError_t e_ = hipGetLastError();                        \
    if (e_ != hipSuccess) return ::qs::hip_status(e_, name);  \
  } while (0)

inline hipStream_t as_stream(qs_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// ----------------------------------------------------------------------------
// Codebook tables, built by constexpr code so that no initialisation call is
// needed on any device.
//
// E8P abs table (quipsharp/codebooks/e8p.py:64-89): rows 0..226 are every abs
// pattern over {1/2,3/2,5/2,7/2}^8 with squared norm <= 10 in ascending
// lexicographic order; rows 227..255 are the 29 norm^2 = 12 padding rows of the
// QuIP# paper (Appendix C.1) in the reference's order; finally each row whose
// coordinate sum is odd has its last coordinate negated.
// ----------------------------------------------------------------------------
struct Table8 {
  float v[256][8];
};

namespace detail {
// k[i] is the half-integer index (value k + 1/2); budget bounds sum k(k+1).
constexpr void e8p_enum(Table8& t, int& n, int pos, int budget, int* k) {
  if (pos == 8) {
    for (int i = 0; i < 8; ++i) t.v[n][i] = (float)k[i] + 0.5f;
    ++n;
    return;
  }
  for (int v = 0; v < 4; ++v) {
    int c = v * (v + 1);
    if (c > budget) break;
    k[pos] = v;
    e8p_enum(t, n, pos + 1, budget - c, k);
  }
}
// Padding rows, each digit a numerator over 2.
constexpr const char* kPad29[29] = {
    "31113333", "13113333", "11313333", "11133333", "33313311", "33313131",
    "33311331", "33313113", "33311313", "33311133", "33133311", "33133131",
    "33131331", "33133113", "33131313", "33131133", "31333311", "31333131",
    "31331331", "31333113", "31331313", "13331133", "13333311", "13333131",
    "13331331", "13333113", "13331313", "11331333", "33113331"};

// Integer / half-integer shells of E8 in itertools.product order (last
// coordinate fastest).  vals are doubled integers (value = vals/2).
constexpr void e8_shell(Table8& t, int& n, int cap, const int* vals, int nv, int pos,
                        int norm4_left, int sum2, int* cur) {
  if (n >= cap) return;
  if (pos == 8) {
    if (norm4_left != 0) return;
    if ((sum2 / 2) % 2 != 0) return;  // coordinate sum must be even
    for (int i = 0; i < 8; ++i) t.v[n][i] = (float)cur[i] * 0.5f;
    ++n;
    return;
  }
  for (int j = 0; j < nv && n < cap; ++j) {
    int v = vals[j];
    int sq = v * v;
    if (sq > norm4_left) continue;
    cur[pos] = v;
    e8_shell(t, n, cap, vals, nv, pos + 1, norm4_left - sq, sum2 + v, cur);
  }
}
}  // namespace detail

constexpr Table8 make_e8p_table() {
  Table8 t{};
  int n = 0;
  int k[8] = {};
  detail::e8p_enum(t, n, 0, 8, k);
  for (int r = 0; r < 29; ++r, ++n)
    for (int i = 0; i < 8; ++i) t.v[n][i] = (float)(detail::kPad29[r][i] - '0') * 0.5f;
  for (int r = 0; r < 256; ++r) {
    int s2 = 0;
    for (int i = 0; i < 8; ++i) s2 += (int)(t.v[r][i] * 2.0f);
    if ((s2 / 2) % 2 != 0) t.v[r][7] = -t.v[r][7];
  }
  return t;
}

// E8 one-bit table (quipsharp/codebooks/e8_1bit.py:26-70): zero, the 112
// integer and 128 half-integer norm^2 = 2 vectors, then the first 15 integer
// norm^2 = 4 vectors, each group in cartesian-product order.
constexpr Table8 make_e81_table() {
  Table8 t{};
  int n = 1;  // row 0 stays zero
  int cur[8] = {};
  const int ints1[3] = {-2, 0, 2};                  // {-1,0,1} doubled
  const int halves[4] = {-3, -1, 1, 3};             // {-3/2,...,3/2} doubled
  const int ints2[5] = {-4, -2, 0, 2, 4};           // {-2,...,2} doubled
  detail::e8_shell(t, n, 256, ints1, 3, 0, 8, 0, cur);   // norm^2 2 -> doubled norm 8
  detail::e8_shell(t, n, 256, halves, 4, 0, 8, 0, cur);
  int cap = n + 15;
  detail::e8_shell(t, n, cap, ints2, 5, 0, 16, 0, cur);  // norm^2 4 -> 16
  return t;
}

// fp16 bit pattern of a float that fp16 represents exactly (zero or normal).
constexpr uint16_t f16_bits_exact(float f) {
  const uint16_t sign = f < 0.0f ? 0x8000 : 0;
  float a = f < 0.0f ? -f : f;
  if (a == 0.0f) return sign;
  int e = 0;
  while (a >= 2.0f) a *= 0.5f, ++e;
  while (a < 1.0f) a *= 2.0f, --e;
  return (uint16_t)(sign | ((e + 15) << 10) | (int)((a - 1.0f) * 1024.0f));
}

// A Table8 as fp16 pairs: w[r][i] holds elements 2i (low half) and 2i + 1.
struct Table8h {
  uint32_t w[256][4];
};

constexpr Table8h pack_table_f16(const Table8& t) {
  Table8h h{};
  for (int r = 0; r < 256; ++r)
    for (int i = 0; i < 4; ++i)
      h.w[r][i] = (uint32_t)f16_bits_exact(t.v[r][2 * i]) | ((uint32_t)f16_bits_exact(t.v[r][2 * i + 1]) << 16);
  return h;
}

constexpr Table8 kE8PHost = make_e8p_table();
constexpr Table8 kE81Host = make_e81_table();

// ----------------------------------------------------------------------------
// device helpers
// ----------------------------------------------------------------------------
__device__ __forceinline__ float load_as_float(const void* p, int dtype, int64_t i) {
  if (dtype == QS_DTYPE_F32) return static_cast<const float*>(p)[i];
  if (dtype == QS_DTYPE_F16) return (float)static_cast<const _Float16*>(p)[i];
  uint32_t b = (uint32_t) static_cast<const uint16_t*>(p)[i] << 16;  // bf16
  return __uint_as_float(b);
}

// Round-to-nearest-even fp32 -> bf16, NaN kept quiet: (u + 0x7FFF + lsb) >> 16
// of the bits u, and (u >> 16) | 0x40 for a NaN.  gfx950's conversion
// instruction (v_cvt_pk_bf16_f32) gives exactly these bits for every one of
// the 2^32 fp32 inputs (checked exhaustively on the device), in one
// instruction for two values instead of six or seven integer operations per
// value.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
// Two values: lo in bits 0-15, hi in bits 16-31.
__device__ __forceinline__ uint32_t f32x2_to_bf16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

__device__ __forceinline__ void store_from_float(void* p, int dtype, int64_t i, float v) {
  if (dtype == QS_DTYPE_F32) static_cast<float*>(p)[i] = v;
  else if (dtype == QS_DTYPE_F16) static_cast<_Float16*>(p)[i] = (_Float16)v;
  else static_cast<uint16_t*>(p)[i] = f32_to_bf16(v);
}

inline int dtype_bytes(int dtype) { return dtype == QS_DTYPE_F32 ? 4 : 2; }

}  // namespace qs
