// Quantized-linear forward on gfx950 (quipsharp/quantize.py:116-124 and
// quipsharp/checkpoint.py:141-146):
//
//   y = su (.) T_m( layer_scale * W_hat @ T_n(sv (.) x) ) + bias,
//   W_hat[r] = s0 * E8P(code0[r]) (+ s1 * E81(code1[r]))
//
// Three launches:
//   xin_kernel      one work-group per batch row: sv-scaling and T_n in LDS,
//                   then fp16 activations (per-row power-of-two scaled) and the
//                   per-8-column sums used for the +-1/4 shift term.
//   mv_tiled_kernel the HBM-bound part.  Codes stream once from HBM in
//                   16-row x 32-code tiles (one 16-byte load per lane); each
//                   code is turned into eight fp16 weights by two 8-byte reads
//                   from 4096-entry LDS tables (coordinates 0..3 and 4..7, signs
//                   folded in) and fed to v_mfma_f32_16x16x32_f16 with the
//                   activations as the 16-column operand (one column per batch
//                   row).  The +-1/4 shifts become one more MFMA per tile:
//                   sum_g shift_bit_g * S_g, S_g the sum of x over group g.
//   yout_kernel     one work-group per batch row: sums the column-group
//                   partials, scales, T_m in LDS, su, bias, output dtype.
#include <cmath>

#include "qs_rht_dev.h"

namespace qs {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__constant__ Table8 kE8P = make_e8p_table();
__constant__ Table8 kE81 = make_e81_table();

constexpr int kRowThreads = 1024;
constexpr int kMaxLen = 32768;
constexpr int kMaxTileBatch = 16;   // MFMA N dimension
constexpr int kMaxWaves = 16;

size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct WsLayout {
  size_t x2h, sg, xtot, xmul, x2, y1p, total;
  int S, SG, W;
};

WsLayout ws_layout(int64_t m, int64_t n, int64_t batch, int layout) {
  WsLayout L{};
  const int64_t B = batch < kMaxTileBatch ? batch : kMaxTileBatch;
  size_t off = 0;
  if (layout == QS_LAYOUT_TILED) {
    L.S = (int)(n / 256);
    L.SG = (L.S + kMaxWaves - 1) / kMaxWaves;
    L.W = (L.S + L.SG - 1) / L.SG;
    L.x2h = off; off = align256(off + (size_t)B * n * 2);
    L.sg = off; off = align256(off + (size_t)B * (n / 8) * 2);
    L.xtot = off; off = align256(off + (size_t)B * 4);
    L.xmul = off; off = align256(off + (size_t)B * 4);
  } else {
    L.S = 0;
    L.SG = 1;
    L.W = 0;
    L.x2 = off; off = align256(off + (size_t)B * n * 4);
  }
  L.y1p = off; off = align256(off + (size_t)L.SG * B * m * 4);
  L.total = off;
  return L;
}

int cu_count() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int c = 0;
    if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
    cached[dev] = c;
  }
  return cached[dev];
}

// ---------------------------------------------------------------------------
// input transform
// ---------------------------------------------------------------------------
struct XinArgs {
  const void* x;
  int x_dtype;
  int64_t ldx;
  int n, L, p;
  const float* K;
  float scale;
  const float* sv;
  int tiled;
  _Float16* x2h;
  _Float16* sg;
  float* xtot;
  float* xmul;
  float* x2;
};

__device__ float block_reduce_max(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) r = fmaxf(r, red[i]);
  __syncthreads();
  return r;
}

// Deterministic block sum: per-wave tree, then waves in order.
__device__ float block_reduce_sum(float v, float* red) {
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) r += red[i];
  __syncthreads();
  return r;
}

__global__ __launch_bounds__(kRowThreads) void xin_kernel(XinArgs A) {
  extern __shared__ float buf[];
  __shared__ float red[kRowThreads / 64];
  const int64_t b = blockIdx.x;
  for (int i = threadIdx.x; i < A.n; i += blockDim.x)
    buf[i] = load_as_float(A.x, A.x_dtype, b * A.ldx + i) * A.sv[i];
  __syncthreads();
  lds_rht(buf, A.n, A.L, A.p, A.K, A.scale);
  if (!A.tiled) {
    for (int i = threadIdx.x; i < A.n; i += blockDim.x) A.x2[b * A.n + i] = buf[i];
    return;
  }
  float amax = 0.0f;
  for (int i = threadIdx.x; i < A.n; i += blockDim.x) amax = fmaxf(amax, fabsf(buf[i]));
  amax = block_reduce_max(amax, red);
  int e = 0;
  if (amax > 0.0f && amax < INFINITY) {
    int ex;
    frexpf(amax, &ex);  // amax < 2^ex
    e = ex - 14;        // scaled maximum in [2^13, 2^14)
  }
  for (int i = threadIdx.x; i < A.n; i += blockDim.x)
    A.x2h[b * A.n + i] = (_Float16)ldexpf(buf[i], -e);
  const int T = A.n / 8;
  float part = 0.0f;
  for (int g = threadIdx.x; g < T; g += blockDim.x) {
    float s = ldexpf(buf[8 * g], -e);
#pragma unroll
    for (int i = 1; i < 8; ++i) s = s + ldexpf(buf[8 * g + i], -e);
    const _Float16 h = (_Float16)s;
    A.sg[b * T + g] = h;
    part += (float)h;
  }
  const float tot = block_reduce_sum(part, red);
  if (threadIdx.x == 0) {
    A.xtot[b] = tot;
    A.xmul[b] = ldexpf(1.0f, e);
  }
}

// ---------------------------------------------------------------------------
// decode-matvec, tiled layout, matrix cores
// ---------------------------------------------------------------------------
struct MvArgs {
  const uint16_t* codes0;
  const uint8_t* codes1;
  const _Float16* x2h;
  const _Float16* sg;
  float* y1p;
  int m, n, B, S, SG, W;
  float s0, s1;
};

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

template <bool HAS2>
__global__ __launch_bounds__(kMaxWaves * 64) void mv_tiled_kernel(MvArgs A) {
  __shared__ uint2 lut_hi[4096];
  __shared__ uint2 lut_lo[4096];
  __shared__ uint4 lut1[HAS2 ? 256 : 1];
  __shared__ float red[kMaxWaves][16][kMaxTileBatch];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  const int RB = A.m >> 4;
  const int nitems = RB * A.SG;
  const int T = A.n >> 3;

  // Signed half-codeword tables.  hi[H*256 + a]: coordinates 0..3 of row a,
  // H = (f1 f2 f3 q); lo[q*2048 + a*8 + f]: coordinates 4..7, f = (f4 f5 f6),
  // coordinate 7 flipped by q^f4^f5^f6.
  for (int e = threadIdx.x; e < 4096; e += blockDim.x) {
    {
      const int H = e >> 8, a = e & 255;
      const int f1 = (H >> 3) & 1, f2 = (H >> 2) & 1, f3 = (H >> 1) & 1, qq = H & 1;
      const int f0 = qq ^ f1 ^ f2 ^ f3;
      const float c0 = f0 ? -kE8P.v[a][0] : kE8P.v[a][0];
      const float c1 = f1 ? -kE8P.v[a][1] : kE8P.v[a][1];
      const float c2 = f2 ? -kE8P.v[a][2] : kE8P.v[a][2];
      const float c3 = f3 ? -kE8P.v[a][3] : kE8P.v[a][3];
      lut_hi[e] = make_uint2(pack_h2(c0, c1), pack_h2(c2, c3));
    }
    {
      const int qq = e >> 11, a = (e >> 3) & 255, f = e & 7;
      const int f4 = (f >> 2) & 1, f5 = (f >> 1) & 1, f6 = f & 1;
      const int f7 = qq ^ f4 ^ f5 ^ f6;
      const float c4 = f4 ? -kE8P.v[a][4] : kE8P.v[a][4];
      const float c5 = f5 ? -kE8P.v[a][5] : kE8P.v[a][5];
      const float c6 = f6 ? -kE8P.v[a][6] : kE8P.v[a][6];
      const float c7 = f7 ? -kE8P.v[a][7] : kE8P.v[a][7];
      lut_lo[e] = make_uint2(pack_h2(c4, c5), pack_h2(c6, c7));
    }
  }
  if (HAS2) {
    for (int e = threadIdx.x; e < 256; e += blockDim.x)
      lut1[e] = make_uint4(pack_h2(kE81.v[e][0], kE81.v[e][1]), pack_h2(kE81.v[e][2], kE81.v[e][3]),
                           pack_h2(kE81.v[e][4], kE81.v[e][5]), pack_h2(kE81.v[e][6], kE81.v[e][7]));
  }
  __syncthreads();

  const half8 hzero = {0, 0, 0, 0, 0, 0, 0, 0};
  int cur_sg = -1;
  half8 xb[8];
  half8 xs = hzero;
#pragma unroll
  for (int c = 0; c < 8; ++c) xb[c] = hzero;

  for (int it = blockIdx.x; it < nitems; it += gridDim.x) {
    const int sg = it / RB, rb = it - sg * RB;
    const int sl = sg * A.W + w;
    const bool active = sl < A.S;
    if (sg != cur_sg) {
      cur_sg = sg;
      const bool have = active && r16 < A.B;
      const _Float16* xrow = A.x2h + (size_t)r16 * A.n + (size_t)256 * sl + 64 * q;
#pragma unroll
      for (int c = 0; c < 8; ++c) xb[c] = have ? *reinterpret_cast<const half8*>(xrow + 8 * c) : hzero;
      xs = have ? *reinterpret_cast<const half8*>(A.sg + (size_t)r16 * T + 32 * sl + 8 * q) : hzero;
    }
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    floatx4 accs = {0.f, 0.f, 0.f, 0.f};
    floatx4 acc2 = {0.f, 0.f, 0.f, 0.f};
    if (active) {
      const size_t tile = ((size_t)rb * A.S + sl) * 64 + lane;
      const uint4 cw = *reinterpret_cast<const uint4*>(A.codes0 + tile * 8);
      uint2 cw1 = make_uint2(0, 0);
      if (HAS2) cw1 = *reinterpret_cast<const uint2*>(A.codes1 + tile * 8);
      const uint32_t wd[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t wv = wd[c >> 1];
        const uint32_t ha = (c & 1) ? ((wv >> 17) & 0x7FF8u) : ((wv >> 1) & 0x7FF8u);
        const uint32_t la = (c & 1) ? ((wv >> 14) & 0x7FF8u) : ((wv << 2) & 0x7FF8u);
        const uint2 hv = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(lut_hi) + ha);
        const uint2 lv = *reinterpret_cast<const uint2*>(reinterpret_cast<const char*>(lut_lo) + la);
        const half8 av = __builtin_bit_cast(half8, make_uint4(hv.x, hv.y, lv.x, lv.y));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, xb[c], acc, 0, 0, 0);
        if (HAS2) {
          const uint32_t idx = ((c < 4 ? cw1.x : cw1.y) >> (8 * (c & 3))) & 0xFFu;
          const half8 a2 = __builtin_bit_cast(half8, lut1[idx]);
          acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, xb[c], acc2, 0, 0, 0);
        }
      }
      const half8 ash = __builtin_bit_cast(
          half8, make_uint4((wd[0] & 0x10001u) * 0x3C00u, (wd[1] & 0x10001u) * 0x3C00u,
                            (wd[2] & 0x10001u) * 0x3C00u, (wd[3] & 0x10001u) * 0x3C00u));
      accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(ash, xs, accs, 0, 0, 0);
    }
    // lane holds rows 4q..4q+3 of the tile for batch column r16
    if (r16 < A.B) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = A.s0 * (acc[j] + 0.5f * accs[j]);
        if (HAS2) v = v + A.s1 * acc2[j];
        red[w][4 * q + j][r16] = active ? v : 0.0f;
      }
    }
    __syncthreads();
    const int nw = A.S - sg * A.W < A.W ? A.S - sg * A.W : A.W;
    for (int u = threadIdx.x; u < 16 * A.B; u += blockDim.x) {
      const int row = u / A.B, bc = u - row * A.B;
      float s = red[0][row][bc];
      for (int ww = 1; ww < nw; ++ww) s += red[ww][row][bc];
      A.y1p[((size_t)sg * A.B + bc) * A.m + rb * 16 + row] = s;
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// decode-matvec, row-major layout (any m, n % 8 == 0), fp32 vector units
// ---------------------------------------------------------------------------
struct MvgArgs {
  const uint16_t* codes0;
  const void* codes1;  // uint16 (E8P) or uint8 (E8 1-bit) row-major
  int kind1;
  const float* x2;
  float* y1p;
  int m, n, B;
  float s0, s1;
};

__device__ __forceinline__ void decode_e8p_f32(uint32_t c, float v[8]) {
  const int a = (c >> 8) & 0xFF;
  uint32_t par = 0;
  const float sh = (c & 1) ? 0.25f : -0.25f;
#pragma unroll
  for (int i = 0; i < 7; ++i) {
    const uint32_t f = (c >> (7 - i)) & 1;
    par ^= f;
    const float t = kE8P.v[a][i];
    v[i] = (f ? -t : t) + sh;
  }
  const float t7 = kE8P.v[a][7];
  v[7] = (par ? -t7 : t7) + sh;
}

__global__ __launch_bounds__(256) void mv_generic_kernel(MvgArgs A) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= A.m) return;
  const int T = A.n >> 3;
  float acc[kMaxTileBatch];
#pragma unroll
  for (int b = 0; b < kMaxTileBatch; ++b) acc[b] = 0.0f;
  for (int t = lane; t < T; t += 64) {
    float v[8];
    decode_e8p_f32(A.codes0[r * T + t], v);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = A.s0 * v[i];
    if (A.codes1) {
      float v2[8];
      if (A.kind1 == QS_STAGE_E8P) {
        decode_e8p_f32(static_cast<const uint16_t*>(A.codes1)[r * T + t], v2);
      } else {
        const int idx = static_cast<const uint8_t*>(A.codes1)[r * T + t];
#pragma unroll
        for (int i = 0; i < 8; ++i) v2[i] = kE81.v[idx][i];
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = __builtin_fmaf(A.s1, v2[i], v[i]);
    }
#pragma unroll
    for (int b = 0; b < kMaxTileBatch; ++b) {
      if (b < A.B) {
        const float* xr = A.x2 + (int64_t)b * A.n + 8 * t;
        float s = acc[b];
#pragma unroll
        for (int i = 0; i < 8; ++i) s = __builtin_fmaf(v[i], xr[i], s);
        acc[b] = s;
      }
    }
  }
#pragma unroll
  for (int b = 0; b < kMaxTileBatch; ++b) {
    if (b < A.B) {
      float s = acc[b];
      for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o);
      if (lane == 0) A.y1p[(int64_t)b * A.m + r] = s;
    }
  }
}

// ---------------------------------------------------------------------------
// output transform
// ---------------------------------------------------------------------------
struct YoutArgs {
  const float* y1p;
  int SG, B, m, L, p;
  const float* K;
  float scale;
  const float* xtot;  // NULL on the row-major path
  const float* xmul;
  float s0, layer_scale;
  const float* su;
  const float* bias;
  void* y;
  int y_dtype;
  int64_t ldy;
};

__global__ __launch_bounds__(kRowThreads) void yout_kernel(YoutArgs A) {
  extern __shared__ float buf[];
  const int b = blockIdx.x;
  const float shift = A.xtot ? -0.25f * A.s0 * A.xtot[b] : 0.0f;
  const float mul = A.layer_scale * (A.xmul ? A.xmul[b] : 1.0f);
  for (int i = threadIdx.x; i < A.m; i += blockDim.x) {
    float s = A.y1p[(size_t)b * A.m + i];
    for (int g = 1; g < A.SG; ++g) s += A.y1p[((size_t)g * A.B + b) * A.m + i];
    buf[i] = (s + shift) * mul;
  }
  __syncthreads();
  lds_rht(buf, A.m, A.L, A.p, A.K, A.scale);
  for (int i = threadIdx.x; i < A.m; i += blockDim.x) {
    float v = buf[i] * A.su[i];
    if (A.bias) v = v + A.bias[i];
    store_from_float(A.y, A.y_dtype, (int64_t)b * A.ldy + i, v);
  }
}

// Raises a kernel's dynamic-LDS limit when needed (remembers the largest value
// set per kernel; a benign race at worst repeats the call).
int set_lds(const void* fn, size_t bytes, int* done) {
  if (bytes > 65536 && (int)bytes > *done) {
    QS_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    *done = (int)bytes;
  }
  return QS_OK;
}
int g_xin_lds = 0, g_yout_lds = 0;

int check_transform(int64_t len, int p, const float* K, const char* which) {
  QS_REQUIRE(p >= 1 && (p & 1) && p <= QS_MAX_KRON, "%s: kron factor must be odd in [1, %d]", which, QS_MAX_KRON);
  QS_REQUIRE(len % p == 0, "%s: length %lld not divisible by %d", which, (long long)len, p);
  const int64_t L = len / p;
  QS_REQUIRE((L & (L - 1)) == 0, "%s: length / kron factor must be a power of two", which);
  QS_REQUIRE(p == 1 || K, "%s: kron matrix required", which);
  QS_REQUIRE(len <= kMaxLen, "%s: length %lld exceeds %d", which, (long long)len, kMaxLen);
  return QS_OK;
}

}  // namespace
}  // namespace qs

using namespace qs;

extern "C" size_t qs_linear_workspace_bytes(int64_t m, int64_t n, int64_t batch, int layout) {
  if (m <= 0 || n <= 0 || batch <= 0) return 0;
  return ws_layout(m, n, batch, layout).total;
}

extern "C" int qs_linear_forward(const void* x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int64_t m,
                                 const void* codes0, const void* codes1, int kind1, int layout, const float* sv,
                                 const float* su, int kron_pn, const float* kron_n, int kron_pm,
                                 const float* kron_m, float s0, float s1, float layer_scale, const float* bias,
                                 void* y, int y_dtype, int64_t ldy, void* workspace, size_t workspace_bytes,
                                 qs_stream_t stream) {
  QS_REQUIRE(batch >= 0 && n > 0 && m > 0 && n % 8 == 0, "bad shape batch=%lld n=%lld m=%lld", (long long)batch,
             (long long)n, (long long)m);
  QS_REQUIRE(x_dtype >= QS_DTYPE_F32 && x_dtype <= QS_DTYPE_BF16 && y_dtype >= QS_DTYPE_F32 &&
                 y_dtype <= QS_DTYPE_BF16,
             "bad dtype");
  QS_REQUIRE(layout == QS_LAYOUT_TILED || layout == QS_LAYOUT_ROWMAJOR, "bad layout");
  if (batch == 0) return QS_OK;
  QS_REQUIRE(x && y && codes0 && sv && su && workspace, "null pointer");
  QS_REQUIRE(ldx >= n && ldy >= m, "row strides too small");
  int rc = check_transform(n, kron_pn, kron_n, "input");
  if (rc) return rc;
  rc = check_transform(m, kron_pm, kron_m, "output");
  if (rc) return rc;
  if (layout == QS_LAYOUT_TILED)
    QS_REQUIRE(m % 16 == 0 && n % 256 == 0, "tiled layout needs m %% 16 == 0 and n %% 256 == 0");
  QS_REQUIRE(!codes1 || kind1 == QS_STAGE_E8_1BIT || (kind1 == QS_STAGE_E8P && layout == QS_LAYOUT_ROWMAJOR),
             "second stage must be E8 1-bit (or E8P on the row-major layout)");
  const WsLayout W = ws_layout(m, n, batch, layout);
  QS_REQUIRE(workspace_bytes >= W.total, "workspace too small: %zu < %zu", workspace_bytes, W.total);
  QS_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "workspace must be 256-byte aligned");
  if (layout == QS_LAYOUT_TILED)
    QS_REQUIRE((reinterpret_cast<uintptr_t>(codes0) & 15) == 0 &&
                   (!codes1 || (reinterpret_cast<uintptr_t>(codes1) & 7) == 0),
               "packed codes must be 16-byte aligned");

  hipStream_t s = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  const int Ln = (int)(n / kron_pn), Lm = (int)(m / kron_pm);
  rc = set_lds((const void*)xin_kernel, (size_t)n * 4, &g_xin_lds);
  if (rc) return rc;
  rc = set_lds((const void*)yout_kernel, (size_t)m * 4, &g_yout_lds);
  if (rc) return rc;

  for (int64_t b0 = 0; b0 < batch; b0 += kMaxTileBatch) {
    const int B = (int)(batch - b0 < kMaxTileBatch ? batch - b0 : kMaxTileBatch);
    const char* xb = static_cast<const char*>(x) + (size_t)b0 * ldx * dtype_bytes(x_dtype);
    char* yb = static_cast<char*>(y) + (size_t)b0 * ldy * dtype_bytes(y_dtype);

    XinArgs XA{};
    XA.x = xb;
    XA.x_dtype = x_dtype;
    XA.ldx = ldx;
    XA.n = (int)n;
    XA.L = Ln;
    XA.p = kron_pn;
    XA.K = kron_n;
    XA.scale = inv_sqrt_len(Ln);
    XA.sv = sv;
    XA.tiled = layout == QS_LAYOUT_TILED;
    XA.x2h = reinterpret_cast<_Float16*>(ws + W.x2h);
    XA.sg = reinterpret_cast<_Float16*>(ws + W.sg);
    XA.xtot = reinterpret_cast<float*>(ws + W.xtot);
    XA.xmul = reinterpret_cast<float*>(ws + W.xmul);
    XA.x2 = reinterpret_cast<float*>(ws + W.x2);
    hipLaunchKernelGGL(xin_kernel, dim3(B), dim3(kRowThreads), (size_t)n * 4, s, XA);
    QS_LAUNCHED("xin_kernel");

    float* y1p = reinterpret_cast<float*>(ws + W.y1p);
    if (layout == QS_LAYOUT_TILED) {
      MvArgs MA{};
      MA.codes0 = static_cast<const uint16_t*>(codes0);
      MA.codes1 = static_cast<const uint8_t*>(codes1);
      MA.x2h = XA.x2h;
      MA.sg = XA.sg;
      MA.y1p = y1p;
      MA.m = (int)m;
      MA.n = (int)n;
      MA.B = B;
      MA.S = W.S;
      MA.SG = W.SG;
      MA.W = W.W;
      MA.s0 = s0;
      MA.s1 = s1;
      const int items = (int)(m / 16) * W.SG;
      const int grid = items < cu_count() ? items : cu_count();
      if (codes1)
        hipLaunchKernelGGL(mv_tiled_kernel<true>, dim3(grid), dim3(W.W * 64), 0, s, MA);
      else
        hipLaunchKernelGGL(mv_tiled_kernel<false>, dim3(grid), dim3(W.W * 64), 0, s, MA);
      QS_LAUNCHED("mv_tiled_kernel");
    } else {
      MvgArgs GA{};
      GA.codes0 = static_cast<const uint16_t*>(codes0);
      GA.codes1 = codes1;
      GA.kind1 = kind1;
      GA.x2 = XA.x2;
      GA.y1p = y1p;
      GA.m = (int)m;
      GA.n = (int)n;
      GA.B = B;
      GA.s0 = s0;
      GA.s1 = s1;
      hipLaunchKernelGGL(mv_generic_kernel, dim3((unsigned)((m + 3) / 4)), dim3(256), 0, s, GA);
      QS_LAUNCHED("mv_generic_kernel");
    }

    YoutArgs YA{};
    YA.y1p = y1p;
    YA.SG = W.SG;
    YA.B = B;
    YA.m = (int)m;
    YA.L = Lm;
    YA.p = kron_pm;
    YA.K = kron_m;
    YA.scale = inv_sqrt_len(Lm);
    YA.xtot = layout == QS_LAYOUT_TILED ? XA.xtot : nullptr;
    YA.xmul = layout == QS_LAYOUT_TILED ? XA.xmul : nullptr;
    YA.s0 = s0;
    YA.layer_scale = layer_scale;
    YA.su = su;
    YA.bias = bias;
    YA.y = yb;
    YA.y_dtype = y_dtype;
    YA.ldy = ldy;
    hipLaunchKernelGGL(yout_kernel, dim3(B), dim3(kRowThreads), (size_t)m * 4, s, YA);
    QS_LAUNCHED("yout_kernel");
  }
  return QS_OK;
}
