// Device building blocks shared by the forward kernels on the chunk scheme:
// the one-launch kernel (qs_linear_fused.hip) and the batched input /
// decode-matvec / output kernels (qs_linear_batched.hip).  Work-groups are
// 16 waves of 64 lanes (1024 threads).
#pragma once

#include "qs_chunk_dev.h"
#include "qs_slots.h"
#include "qs_tags.h"

namespace qs {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

namespace {
// E8P abs table and E8 one-bit table rows as fp16 pairs (Table8h).
__constant__ Table8h kE8Ph = pack_table_f16(make_e8p_table());
__constant__ Table8h kE81h = pack_table_f16(make_e81_table());
}  // namespace

constexpr int kFwdThreads = 1024;

// ---------------------------------------------------------------------------
// Signed half-codeword LUTs, one byte per value
// ---------------------------------------------------------------------------
// Every E8P value is +-(k + 1/2), k < 4, whose fp16 pattern has a zero low
// byte, so a LUT entry holds the four high bytes of a half codeword and
// v_perm_b32 rebuilds the fp16 pairs.  (Against 8-byte fp16 entries this
// halves the LDS bytes per lookup for four v_perm_b32 per code, which
// measured faster: the decode loop is bound by LDS and VALU issue together.)
constexpr bool e8p_low_bytes_zero() {
  for (int r = 0; r < 256; ++r)
    for (int i = 0; i < 8; ++i)
      if (f16_bits_exact(kE8PHost.v[r][i]) & 0xFF) return false;
  return true;
}
static_assert(e8p_low_bytes_zero(), "E8P values are fp16 high bytes only");

// fp16 pairs (values 0,1 and 2,3) from the four high bytes of a LUT entry.
__device__ __forceinline__ uint32_t lut_pair_lo(uint32_t e) { return __builtin_amdgcn_perm(0u, e, 0x010C000Cu); }
__device__ __forceinline__ uint32_t lut_pair_hi(uint32_t e) { return __builtin_amdgcn_perm(0u, e, 0x030C020Cu); }

// 32-bit LDS word at byte address a.  The kernels that use the LUTs have no
// static LDS, so their dynamic LDS starts at address 0 (the launchers check
// this) and a LUT offset is the LDS address itself.
typedef const __attribute__((address_space(3))) uint32_t* lds_u32_ptr;
__device__ __forceinline__ uint32_t lds_word(uint32_t a) { return *reinterpret_cast<lds_u32_ptr>((size_t)a); }

// The two 4096-entry LUTs (hi: words 0..4095, lo: 4096..8191), built at
// compile time; kernels copy them into LDS at address 0.  Entry e of hi:
// abs row e & 255, flip nibble H = e >> 8 = (f1 f2 f3 q), f0 = q^f1^f2^f3;
// of lo: abs row (e >> 3) & 255 (+128 for odd e >> 10), f4..f6 = e & 7,
// q = e >> 11, coordinate 7 flipped by q^f4^f5^f6.  A sign flip of value v
// is bit 7 of byte v (mod 4).
struct LutWords {
  uint32_t w[8192];
};
constexpr uint32_t high_bytes(uint32_t a, uint32_t b) {  // bytes 1, 3 of a, then of b
  return ((a >> 8) & 0xFFu) | ((a >> 16) & 0xFF00u) | (((b >> 8) & 0xFFu) << 16) | ((b >> 24) << 24);
}
constexpr LutWords make_luts(const Table8h& t) {
  LutWords L{};
  for (uint32_t e = 0; e < 4096; ++e) {
    const uint32_t H = e >> 8;
    const uint32_t f1 = (H >> 3) & 1, f2 = (H >> 2) & 1, f3 = (H >> 1) & 1;
    const uint32_t f0 = (H & 1) ^ f1 ^ f2 ^ f3;
    L.w[e] = high_bytes(t.w[e & 255][0], t.w[e & 255][1]) ^ ((f0 << 7) | (f1 << 15) | (f2 << 23) | (f3 << 31));
    const uint32_t lt = e & 1023, k = e >> 10;
    const uint32_t f4 = (lt >> 2) & 1, f5 = (lt >> 1) & 1, f6 = lt & 1;
    const uint32_t f7 = (k >> 1) ^ f4 ^ f5 ^ f6;
    const uint32_t r = ((lt >> 3) + ((k & 1) ? 128u : 0u)) & 255;
    L.w[4096 + e] = high_bytes(t.w[r][2], t.w[r][3]) ^ ((f4 << 7) | (f5 << 15) | (f6 << 23)) ^ (f7 << 31);
  }
  return L;
}
namespace {
__device__ const LutWords kLuts = make_luts(pack_table_f16(make_e8p_table()));
}  // namespace
// Thread tid's share of the LUTs in a work-group of NT threads: 16-byte
// words tid + NT k (loads issued by load_luts, stored by store_luts into LDS
// at address 0 once they are needed).
template <int NT>
struct LutCopy {
  static_assert(NT >= 256 && 2048 % NT == 0, "LUT copy: 2048 16-byte words over the work-group");
  uint4 v[2048 / NT];
};
template <int NT>
__device__ __forceinline__ void load_luts(int tid, LutCopy<NT>& r) {
  const uint4* src = reinterpret_cast<const uint4*>(kLuts.w);
#pragma unroll
  for (int k = 0; k < 2048 / NT; ++k) r.v[k] = src[tid + NT * k];
}
template <int NT>
__device__ __forceinline__ void store_luts(char* lds_base, int tid, const LutCopy<NT>& r) {
  uint4* dst = reinterpret_cast<uint4*>(lds_base);
#pragma unroll
  for (int k = 0; k < 2048 / NT; ++k) dst[tid + NT * k] = r.v[k];
}

// MFMA A operand (8 fp16 values) of code word c (c odd: the upper 16 bits of
// wv) from the LUTs at LDS addresses off_hi / off_lo.
__device__ __forceinline__ half8 decode_code(uint32_t wv, int c, uint32_t off_hi, uint32_t off_lo) {
  const uint32_t ha = (c & 1) ? ((wv >> 18) & 0x3FFCu) : ((wv >> 2) & 0x3FFCu);
  const uint32_t la = (c & 1) ? ((wv >> 15) & 0x3FFCu) : ((wv << 1) & 0x3FFCu);
  const uint32_t hv = lds_word(off_hi + ha);
  const uint32_t lv = lds_word(off_lo + la);
  return __builtin_bit_cast(half8, make_uint4(lut_pair_lo(hv), lut_pair_hi(hv), lut_pair_lo(lv), lut_pair_hi(lv)));
}

// The two LUT words of code word c (c odd: the upper 16 bits of wv), and the
// MFMA A operand built from them, split so that a tile's 16 LDS reads can be
// issued together before the first operand is built.
__device__ __forceinline__ void code_lut_words(uint32_t wv, int c, uint32_t off_hi, uint32_t off_lo, uint32_t& hv,
                                               uint32_t& lv) {
  const uint32_t ha = (c & 1) ? ((wv >> 18) & 0x3FFCu) : ((wv >> 2) & 0x3FFCu);
  const uint32_t la = (c & 1) ? ((wv >> 15) & 0x3FFCu) : ((wv << 1) & 0x3FFCu);
  hv = lds_word(off_hi + ha);
  lv = lds_word(off_lo + la);
}
__device__ __forceinline__ half8 code_operand(uint32_t hv, uint32_t lv) {
  return __builtin_bit_cast(half8, make_uint4(lut_pair_lo(hv), lut_pair_hi(hv), lut_pair_lo(lv), lut_pair_hi(lv)));
}

// fp16 shift operand of a tile: 1.0 where a code's shift bit is set.
__device__ __forceinline__ half8 shift_operand(const uint32_t (&wd)[4]) {
  return __builtin_bit_cast(half8, make_uint4((wd[0] & 0x10001u) * 0x3C00u, (wd[1] & 0x10001u) * 0x3C00u,
                                              (wd[2] & 0x10001u) * 0x3C00u, (wd[3] & 0x10001u) * 0x3C00u));
}

// ---------------------------------------------------------------------------
// Activation chunks
// ---------------------------------------------------------------------------
struct XSource {
  const void* x;
  int dtype;
  int vec;  // rows of 4 elements can be loaded as one 8- or 16-byte word
  int64_t ldx;
  int S;    // chunks of 256
  int sbits;  // sv holds packed sign bits (QS_SIGNS_BITS), not fp32 values
};

// x times the sign of bit k of b (set: -1), as a sign-bit flip: the same
// value as x * -1.0f / x * 1.0f.
__device__ __forceinline__ float flip_by_bit(float x, uint32_t b, int k) {
  return __uint_as_float(__float_as_uint(x) ^ (((b >> k) & 1u) << 31));
}

// One chunk's four activations t = 4 lane .. 4 lane + 3 of batch row b as
// loaded (the words of x and of sv), so that loads can be issued ahead of
// their use.  Sign bits: the word of elements i0 .. i0 + 3, kept raw in s.x
// and applied by finish_chunk.
__device__ __forceinline__ void load_chunk_raw(const XSource& X, const float* sv, int b, int c, int lane, uint4& v,
                                               float4& s) {
  const int i0 = 256 * c + 4 * lane;
  if (X.sbits) s.x = __uint_as_float(reinterpret_cast<const uint32_t*>(sv)[i0 >> 5]);
  else s = *reinterpret_cast<const float4*>(sv + i0);
  const int64_t xi = (int64_t)b * X.ldx + i0;
  if (X.vec && X.dtype == QS_DTYPE_F32) {
    v = *reinterpret_cast<const uint4*>(static_cast<const float*>(X.x) + xi);
  } else if (X.vec) {
    const uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(X.x) + xi);
    v = make_uint4(t.x, t.y, 0, 0);
  } else {
    v = make_uint4(__float_as_uint(load_as_float(X.x, X.dtype, xi)), __float_as_uint(load_as_float(X.x, X.dtype, xi + 1)),
                   __float_as_uint(load_as_float(X.x, X.dtype, xi + 2)),
                   __float_as_uint(load_as_float(X.x, X.dtype, xi + 3)));
  }
}

// The four activations times sv, as fp32.
__device__ __forceinline__ void finish_chunk(const XSource& X, const uint4& t, const float4& s, int lane,
                                             float (&o)[4]) {
  float x0, x1, x2, x3;
  if (X.vec && X.dtype == QS_DTYPE_BF16) {
    x0 = __uint_as_float(t.x << 16), x1 = __uint_as_float(t.x & 0xFFFF0000u);
    x2 = __uint_as_float(t.y << 16), x3 = __uint_as_float(t.y & 0xFFFF0000u);
  } else if (X.vec && X.dtype == QS_DTYPE_F16) {
    x0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.x & 0xFFFFu));
    x1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.x >> 16));
    x2 = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.y & 0xFFFFu));
    x3 = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.y >> 16));
  } else {
    x0 = __uint_as_float(t.x), x1 = __uint_as_float(t.y), x2 = __uint_as_float(t.z), x3 = __uint_as_float(t.w);
  }
  if (X.sbits) {
    const uint32_t b = __float_as_uint(s.x) >> (4 * (lane & 7));
    o[0] = flip_by_bit(x0, b, 0);
    o[1] = flip_by_bit(x1, b, 1);
    o[2] = flip_by_bit(x2, b, 2);
    o[3] = flip_by_bit(x3, b, 3);
  } else {
    o[0] = x0 * s.x;
    o[1] = x1 * s.y;
    o[2] = x2 * s.z;
    o[3] = x3 * s.w;
  }
}

// Activation chunks c = w + 16 u of batch row b (CPW: chunks per wave the
// caller holds, S <= 16 CPW), as loaded.
template <int CPW = kCPW>
struct XRawT {
  uint4 v[CPW];
  float4 s[CPW];
};
using XRaw = XRawT<>;
template <int CPW>
__device__ __forceinline__ void load_x_raw(const XSource& X, const float* sv, int b, int w, int lane,
                                           XRawT<CPW>& r) {
#pragma unroll
  for (int u = 0; u < CPW; ++u) {
    const int c = w + kWaves * u;
    r.v[u] = make_uint4(0, 0, 0, 0);
    r.s[u] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c < X.S) load_chunk_raw(X, sv, b, c, lane, r.v[u], r.s[u]);
  }
}

// Activation chunks (times sv), chunk c = w + 16 u, as element t = 4 lane + j.
template <int CPW>
__device__ __forceinline__ void finish_x(const XSource& X, const XRawT<CPW>& r, int w, int lane,
                                         float (&v)[CPW][4]) {
#pragma unroll
  for (int u = 0; u < CPW; ++u) {
    const int c = w + kWaves * u;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[u][j] = 0.0f;
    if (c < X.S) finish_chunk(X, r.v[u], r.s[u], lane, v[u]);
  }
}

template <int CPW>
__device__ __forceinline__ void load_x(const XSource& X, const float* sv, int b, int w, int lane,
                                       float (&v)[CPW][4]) {
  XRawT<CPW> r;
  load_x_raw(X, sv, b, w, lane, r);
  finish_x(X, r, w, lane, v);
}

// Chunks held as element t = 4 lane + j (the layout of load_x).
template <int CPW>
__device__ __forceinline__ void store_chunks(float* Y, int S, int w, int lane, const float (&v)[CPW][4]) {
#pragma unroll
  for (int u = 0; u < CPW; ++u) {
    const int c = w + kWaves * u;
    if (c < S)
      *reinterpret_cast<float4*>(Y + c * kYStride + 4 * lane) = make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
  }
}

// Chunks held as element t = lane + 64 j (the layout of load_partials).
template <int CPW>
__device__ __forceinline__ void store_chunks_lanes(float* Y, int S, int w, int lane, const float (&v)[CPW][4]) {
#pragma unroll
  for (int u = 0; u < CPW; ++u) {
    const int c = w + kWaves * u;
    if (c < S) {
#pragma unroll
      for (int j = 0; j < 4; ++j) Y[c * kYStride + lane + 64 * j] = v[u][j];
    }
  }
}


// 2^e with |x2_i| <= ||x|| 2^-e < 2^14 for the fp16 operand of a row of
// squared norm norm2 (e = 0 for a zero or non-finite norm).
__device__ __forceinline__ int operand_exponent(float norm2) {
  int e = 0;
  if (norm2 > 0.0f && norm2 < INFINITY) {
    int ex;
    frexpf(sqrtf(norm2) * 1.0001f, &ex);
    e = ex - 14;
  }
  return e;
}

// ---------------------------------------------------------------------------
// Chunk stage on the matrix cores
// ---------------------------------------------------------------------------
// For 16 rows of a chunk matrix M (bf16 hi / lo rows of kMStride in LDS, zero
// past the S chunks) and chunk rows Z in LDS (kYStride floats), lane (q, r16)
// of a wave owning column t accumulates acc[j] = sum_c M[row0 + 4 q + j][c]
// Z[c][t] over k-steps of 32 chunks.  Both operands are split into bf16
// hi + lo and multiplied as hi*hi + hi*lo (+ lo*hi when M has a low part),
// fp32 accumulate: ~16 significant bits per product.
constexpr int kMStride = 72;                 // bf16 per row (16-byte aligned rows)
constexpr int kMRows = 48, kMCols = 64;      // a full chunk matrix, S <= 48
constexpr int kMBytes = kMRows * kMStride * 2;  // one of hi / lo
static_assert(kMRows >= kMaxS && kMCols >= kMaxS, "M covers every chunk count");
static_assert(kMRows * kMCols == 3 * kFwdThreads && kCPW == 3, "three M entries / output rows per thread");

// Two floats as bf16 pairs: the truncated high parts and the (truncated)
// remainders.
__device__ __forceinline__ void split_bf2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
  const uint32_t ha = ua & 0xFFFF0000u, hb = ub & 0xFFFF0000u;
  const uint32_t la = __float_as_uint(a - __uint_as_float(ha)), lb = __float_as_uint(b - __uint_as_float(hb));
  hi = (ha >> 16) | hb;
  lo = (la >> 16) | (lb & 0xFFFF0000u);
}

struct ZOperand {
  bf16x8 h, l;  // Z[c][t], c = 32 kb + 8 q + i
};

__device__ __forceinline__ ZOperand z_operand(const float* Z, int S, int t, int q, int kb) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c0 = 32 * kb + 8 * q + 2 * i;
    const float z0 = c0 < S ? Z[c0 * kYStride + t] : 0.0f;
    const float z1 = c0 + 1 < S ? Z[(c0 + 1) * kYStride + t] : 0.0f;
    split_bf2(z0, z1, h[i], l[i]);
  }
  return ZOperand{__builtin_bit_cast(bf16x8, make_uint4(h[0], h[1], h[2], h[3])),
                  __builtin_bit_cast(bf16x8, make_uint4(l[0], l[1], l[2], l[3]))};
}

// acc += M[row0 + r16][32 kb + 8 q ..] x z (the k-step kb of a tile).
__device__ __forceinline__ floatx4 mstage_step(floatx4 acc, const uint16_t* Mh, const uint16_t* Ml, int row0,
                                               const ZOperand& z, int kb, bool m_lo, int q, int r16) {
  const int off = (row0 + r16) * kMStride + 32 * kb + 8 * q;
  const bf16x8 ah = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(Mh + off));
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, z.h, acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, z.l, acc, 0, 0, 0);
  if (m_lo) {
    const bf16x8 al = __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(Ml + off));
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, z.h, acc, 0, 0, 0);
  }
  return acc;
}

// The K entries of a full chunk matrix M = K_p (x) H_{2^lsh} (S x S) that
// thread tid writes (entries e = tid + 1024 i, row e / 64, column e % 64);
// loads only, so they can be issued ahead of other loads.
__device__ __forceinline__ void mmat_load(float (&kv)[3], int S, int lsh, int p, const float* K, int tid) {
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int e = tid + kFwdThreads * i, r = e / kMCols, c = e % kMCols;
    kv[i] = 1.0f;
    if (p > 1) kv[i] = K[(r < S && c < S) ? (r >> lsh) * p + (c >> lsh) : 0];
  }
}

// Writes those entries (times the Hadamard signs, zero outside S x S) as
// bf16 hi / lo.
__device__ __forceinline__ void mmat_store(const float (&kv)[3], int S, int lsh, uint16_t* Mh, uint16_t* Ml,
                                           int tid) {
  const int hm = (1 << lsh) - 1;
#pragma unroll
  for (int i = 0; i < 3; ++i) {
    const int e = tid + kFwdThreads * i, r = e / kMCols, c = e % kMCols;
    float v = (r < S && c < S) ? kv[i] : 0.0f;
    if (__builtin_popcount(r & c & hm) & 1) v = -v;
    uint32_t hi, lo;
    split_bf2(v, 0.0f, hi, lo);
    Mh[r * kMStride + c] = (uint16_t)hi;
    Ml[r * kMStride + c] = (uint16_t)lo;
  }
}

// ---------------------------------------------------------------------------
// Output side
// ---------------------------------------------------------------------------
constexpr int kMaxSG = (kMaxS + kWaves - 1) / kWaves;  // column groups of the partial sums

// Partial sums y1p[g][b][.] of batch row b (B rows per group), summed over
// the SG column groups, for the chunks c = w + 16 u < Sm of this wave, as
// element t = lane + 64 j (each load instruction reads 256 contiguous bytes).
// Every load is issued before the first one is used.  ATOMIC: agent-scope
// loads (partials written by other work-groups of the same launch).  (The
// 256-point transform is the same for any assignment of the index bits to
// lanes and registers.)
template <int G = kMaxSG, int CPW = kCPW>
struct PRaw {
  float v[G][CPW][4];
};
template <bool ATOMIC, int G, int CPW>
__device__ __forceinline__ void load_partials_raw(const float* y1p, int m, int Sm, int SG, int B, int b, int w,
                                                  int lane, PRaw<G, CPW>& r) {
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      const int c = w + kWaves * u;
#pragma unroll
      for (int j = 0; j < 4; ++j) r.v[g][u][j] = 0.0f;
      if (g < SG && c < Sm) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float* src = y1p + partial_index(g, B, b, m, chunk_elem(c, lane, j));
          r.v[g][u][j] = ATOMIC ? __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *src;
        }
      }
    }
}
template <int G, int CPW>
__device__ __forceinline__ void sum_partials(const PRaw<G, CPW>& r, float (&zv)[CPW][4]) {
#pragma unroll
  for (int u = 0; u < CPW; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float v = r.v[0][u][j];
#pragma unroll
      for (int g = 1; g < G; ++g) v += r.v[g][u][j];
      zv[u][j] = v;
    }
}
// The same sum for any number of groups, one group at a time (groups in
// ascending order, as sum_partials adds them).
template <int CPW>
__device__ __forceinline__ void sum_partials_loop(const float* y1p, int m, int Sm, int SG, int B, int b, int w,
                                                  int lane, float (&zv)[CPW][4]) {
#pragma unroll
  for (int u = 0; u < CPW; ++u)
#pragma unroll
    for (int j = 0; j < 4; ++j) zv[u][j] = 0.0f;
  for (int g = 0; g < SG; ++g)
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      const int c = w + kWaves * u;
      if (c < Sm) {
        float t[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = y1p[partial_index(g, B, b, m, chunk_elem(c, lane, j))];
#pragma unroll
        for (int j = 0; j < 4; ++j) zv[u][j] = g == 0 ? t[j] : zv[u][j] + t[j];
      }
    }
}

template <bool ATOMIC>
__device__ __forceinline__ void load_partials(const float* y1p, int m, int Sm, int SG, int B, int b, int w,
                                              int lane, float (&zv)[kCPW][4]) {
  PRaw<kMaxSG> r;
  load_partials_raw<ATOMIC, kMaxSG>(y1p, m, Sm, SG, B, b, w, lane, r);
  sum_partials(r, zv);
}

// Tagged partial sums.  Each work-group of a one-launch forward writes its
// partial sums as 64-bit slots {fp32 value (low word), launch tag (high
// word)} with one agent-scope store each, and the tail work-groups poll the
// slots until every one carries this launch's tag: no completion counter, no
// wait for the stores to complete before signalling.  The tag (qs_tags.h)
// holds a launch counter and the job's index g in the launch, so a slot can
// only match the launch that wrote it: other jobs' tags differ in g, earlier
// launches of job index g in the counter (slots left from 2^20 - 1 launches
// earlier are cleared when the counter wraps: finish_tagged_launch), and any
// other data left in the workspace would have to be a NaN.  The counter
// continues the workspace's epoch word of job index g (zero: no launch yet);
// the tail work-groups store the tag as the new epoch once every slot they
// poll has been read.
__device__ __forceinline__ unsigned long long tagged(float v, uint32_t tag) {
  return ((unsigned long long)tag << 32) | __float_as_uint(v);
}

// Bound on the polling rounds (each one a device-scope load round trip,
// about a microsecond): a slot still missing after it reads as NaN, so a
// failure shows in the output instead of keeping the GPU busy.
constexpr int kMaxPolls = 1 << 20;

// End of a tail work-group of a tagged launch, called by every thread once
// every slot the work-group polls has been read: stores the tag as the epoch
// (all the tail work-groups store the same value) and, on the launch with the
// last counter value, clears the job's tags from the workspace (the counter
// wrap, qs_tags.h).  `flag` is one int of LDS that is free by now.
__device__ __forceinline__ void finish_tagged_launch(unsigned* epoch, uint32_t tag, int g, const TagWs ws, int* flag) {
  const int tid = threadIdx.x;
  if (tid == 0) {
    __hip_atomic_store(epoch, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (wrap_reset_launch(tag)) __hip_atomic_store(ws.wrap, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!wrap_launch(tag)) return;  // uniform over the work-group
  __syncthreads();                // every wave has read its slots (and LDS)
  if (tid == 0) {
    const unsigned done = __hip_atomic_fetch_add(ws.wrap, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) + 1u;
    const bool last = done == (unsigned)ws.ntail;
    if (last) __hip_atomic_store(ws.wrap, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  if (!*flag) return;
  // every work-group of the job has finished with the workspace: no slot of
  // this launch is in flight, and other jobs' slots hold other tags
  const int nt = (int)blockDim.x;
  for (unsigned long long i = kWsHeaderWords + tid; i < ws.words; i += 4ull * nt) {
    unsigned long long v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const unsigned long long e = i + (unsigned long long)k * nt;
      v[k] = e < ws.words ? __hip_atomic_load(ws.base + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0ull;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const unsigned long long e = i + (unsigned long long)k * nt;
      if (e < ws.words && slot_of_job(v[k], g))
        __hip_atomic_store(ws.base + e, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// Polling the tagged partial sums of batch row b for the chunks
// c = w + 16 u < Sm of this wave (element t = lane + 64 j, as
// load_partials_raw), summed over the SG groups in ascending order once every
// slot holds `tag`.  One group at a time (4 CPW slots per lane in flight;
// issuing four groups together measured slower).
// poll_issue only issues the first group's loads, so that loads issued after
// it share its round trip; poll_finish waits, reloads the slots that do not
// carry the tag yet, and moves on to the next group.
template <int CPW>
struct PollState {
  unsigned long long v[CPW][4];
};
template <int CPW>
__device__ __forceinline__ void poll_load(const unsigned long long* y1t, int m, int Sm, int B, int b, int g, int w,
                                          int lane, uint32_t tag, PollState<CPW>& p, bool only_missing) {
  const unsigned long long fill = tagged(0.0f, tag);  // chunks past Sm: present, zero
#pragma unroll
  for (int u = 0; u < CPW; ++u) {
    const int c = w + kWaves * u;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned long long* src = y1t + partial_index(g, B, b, m, chunk_elem(c, lane, j));
      if (only_missing) {
        if ((uint32_t)(p.v[u][j] >> 32) != tag)
          p.v[u][j] = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      } else {
        p.v[u][j] = c < Sm ? __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : fill;
      }
    }
  }
}
template <int CPW>
__device__ __forceinline__ void poll_issue(const unsigned long long* y1t, int m, int Sm, int B, int b, int w,
                                           int lane, uint32_t tag, PollState<CPW>& p) {
  poll_load(y1t, m, Sm, B, b, 0, w, lane, tag, p, false);
}
template <int CPW>
__device__ __forceinline__ void poll_finish(const unsigned long long* y1t, int m, int Sm, int SG, int B, int b,
                                            int w, int lane, uint32_t tag, PollState<CPW>& p, float (&zv)[CPW][4]) {
  for (int g = 0; g < SG; ++g) {
    if (g > 0) poll_load(y1t, m, Sm, B, b, g, w, lane, tag, p, false);
    for (int round = 0;; ++round) {
      bool ok = true;
#pragma unroll
      for (int u = 0; u < CPW; ++u)
#pragma unroll
        for (int j = 0; j < 4; ++j) ok = ok && (uint32_t)(p.v[u][j] >> 32) == tag;
      if (ok) break;
      if (round == kMaxPolls) {
#pragma unroll
        for (int u = 0; u < CPW; ++u)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if ((uint32_t)(p.v[u][j] >> 32) != tag) p.v[u][j] = tagged(__builtin_nanf(""), tag);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      poll_load(y1t, m, Sm, B, b, g, w, lane, tag, p, true);
    }
#pragma unroll
    for (int u = 0; u < CPW; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x = __uint_as_float((uint32_t)p.v[u][j]);
        zv[u][j] = g == 0 ? x : zv[u][j] + x;
      }
  }
}

// su entry i for the output stage: the fp32 value, or with sign bits the raw
// word holding bit i (kept as float bits; applied by apply_su at the end).
// Code bytes read once: nontemporal loads (16 or 8 bytes).  The forward
// kernels stream every code tile once; with this hint the Llama-2-7B step
// measured 3.6 % faster at batch 1, 2.2 % at 16 rows, 1.6 % at 64 and 0.9 %
// at 512, and the 3-bit Llama-3-8B step 3.2 % at batch 1 and 3.4 % at 16 rows.
typedef unsigned int u32x4nt __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2nt __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ld_nt_u4(const void* p) {
  const u32x4nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x4nt*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ld_nt_u2(const void* p) {
  const u32x2nt v = __builtin_nontemporal_load(reinterpret_cast<const u32x2nt*>(p));
  return make_uint2(v.x, v.y);
}

// Element i of a buffer as a 32-bit byte offset from its (uniform) base: the
// address is the scalar base plus one 32-bit vector register, instead of a
// 64-bit vector address per element (which the compiler would otherwise keep
// live, and spill, across the tail's polling loop).
template <class T>
__device__ __forceinline__ const T& at_off(const T* base, uint32_t i) {
  return *reinterpret_cast<const T*>(reinterpret_cast<const char*>(base) + i * (uint32_t)sizeof(T));
}
template <class T>
__device__ __forceinline__ T& at_off(T* base, uint32_t i) {
  return *reinterpret_cast<T*>(reinterpret_cast<char*>(base) + i * (uint32_t)sizeof(T));
}

__device__ __forceinline__ float load_su(const float* su, int sbits, int i) {
  return sbits ? __uint_as_float(at_off(reinterpret_cast<const uint32_t*>(su), (uint32_t)i >> 5))
               : at_off(su, (uint32_t)i);
}
__device__ __forceinline__ float apply_su(float v, float suo, int sbits, int i) {
  return sbits ? flip_by_bit(v, __float_as_uint(suo), i & 31) : v * suo;
}

// Output values out[a][j] to y[base + idx[a][j]] (idx < 0: no output), one
// dtype dispatch for all of them.
template <int NA>
__device__ __forceinline__ void store_outputs(void* y, int dtype, int64_t base, const int (&idx)[NA][4],
                                              const float (&out)[NA][4]) {
  if (dtype == QS_DTYPE_F32) {
    float* p = static_cast<float*>(y) + base;
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (idx[a][j] >= 0) at_off(p, (uint32_t)idx[a][j]) = out[a][j];
  } else if (dtype == QS_DTYPE_F16) {
    _Float16* p = static_cast<_Float16*>(y) + base;
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (idx[a][j] >= 0) at_off(p, (uint32_t)idx[a][j]) = (_Float16)out[a][j];
  } else {
    uint16_t* p = static_cast<uint16_t*>(y) + base;
#pragma unroll
    for (int a = 0; a < NA; ++a)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (idx[a][j] >= 0) at_off(p, (uint32_t)idx[a][j]) = f32_to_bf16(out[a][j]);
  }
}

}  // namespace qs
