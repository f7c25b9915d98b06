// Quantized-linear forward on gfx950 (quipsharp/quantize.py:116-124 and
// quipsharp/checkpoint.py:141-146):
//
//   y = su (.) T_m( layer_scale * W_hat @ T_n(sv (.) x) ) + bias,
//   W_hat[r] = s0 * E8P(code0[r]) (+ s1 * E81(code1[r]))
//
// This file holds the entry points (qs_linear_forward, qs_linear_forward_group,
// qs_decode_matvec), the workspace layout, and the kernels for the shapes the
// chunk-scheme kernels do not take: the LDS-radix row transforms xin_kernel /
// yout_kernel (any n, m up to 32768; the input or output side of a pass whose
// n or m is outside both the per-row chunk kernels' 12288 and the 16-chunk
// work-group kernels of qs_linear_big.hip, and the transform-free calls),
// yout_chunk_kernel, and the row-major
// decode-matvec of the generic code layout (mv_generic_kernel).  Which path a
// call takes: one launch for 1-2 rows (qs_linear_fused.hip), passes of 16
// rows through the batched decode-matvec (qs_linear_batched.hip), the wide
// GEMM from kWideMinBatch rows (qs_linear_wide.hip).
#include <atomic>
#include <cmath>

#include <hip/hip_ext.h>

#include "qs_chunk_dev.h"
#include "qs_linear_dev.h"
#include "qs_slots.h"

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

constexpr int kMaxParts = 16;  // work-groups per batch row for odd-factor transforms

struct WsLayout {
  size_t x2h, sg, xtot, xmul, x2, y1p, y1t, h2t, y1bt, total;
  int S, SG, W;    // chunks, slice groups and slices per group of the decode-matvec
  FusedPlan fused;  // the one-launch kernel's (its partial sums: fused.SG groups)
  bool wide;
};

// From this many activation rows on (more than one 16-row pass), the tiled
// forward runs the wide GEMM (qs_linear_wide.hip: each code decoded once per
// up to 256 activation rows, every decoded fragment feeding several MFMAs)
// instead of decoding the codes once per 16 rows.  Measured at 17..48 rows
// on the 7B shapes: 24 rows 23 / 34 / 35 us wide against 36 / 47 / 50 us in
// two 16-row passes (4096x4096, 11008x4096, 4096x11008).
constexpr int64_t kWideMinBatch = 17;

// Work-groups per batch row of the input / output transform: the odd-factor
// stage is split over up to 16 of them (each computes L/G columns).
int parts_for(int64_t len, int p) {
  if (p == 1) return 1;
  const int64_t L = len / p;
  int64_t g = L / 8;
  if (g > kMaxParts) g = kMaxParts;
  return g < 1 ? 1 : (int)g;
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

// The first 256 bytes of every workspace hold the epoch words of the kernels
// with tagged partial sums (per job index, the tag of the last such launch;
// zero before the first call) and their wrap words (qs_tags.h).  With the
// tiled layout the next regions hold the one-launch kernel's tagged partial
// sums (8 bytes per slot, up to two rows) and tagged chunk transforms (its
// two-level output transform), and the last region the 16-row
// decode-matvec's tagged partial sums; each is written by its kernel only, so
// a slot can only carry a tag of an earlier launch of the same workspace, and
// those of 2^20 - 1 launches earlier are cleared when the counter wraps.
WsLayout ws_layout(int64_t m, int64_t n, int64_t batch, int layout) {
  WsLayout L{};
  L.wide = layout == QS_LAYOUT_TILED && batch >= kWideMinBatch;
  const int64_t B = L.wide ? batch : batch < kMaxTileBatch ? batch : kMaxTileBatch;
  size_t off = 256;
  if (layout == QS_LAYOUT_TILED) {
    L.S = (int)(n / 256);
    L.SG = (L.S + kMaxWaves - 1) / kMaxWaves;
    L.W = (L.S + L.SG - 1) / L.SG;
    L.fused = fused_plan(L.S);
    L.y1t = off; off = align256(off + fused_slot_count(L.fused.SG, m) * 8);
    L.h2t = off; off = align256(off + h2_slot_count(m) * 8);
    const size_t xrows = (size_t)(B + 15) / 16 * 16;  // fragment-major rows: 16s
    L.x2h = off; off = align256(off + xrows * n * 2);
    L.sg = off; off = align256(off + xrows * (n / 8) * 2);
    L.xtot = off; off = align256(off + (size_t)B * kMaxParts * 4);
    L.xmul = off; off = align256(off + (size_t)B * 4);
  } else {
    L.S = 0;
    L.SG = 1;
    L.W = 0;
    L.fused = FusedPlan{1, 0, 1};
    L.x2 = off; off = align256(off + (size_t)B * n * 4);
  }
  if (L.wide) {
    // partial groups of the wide GEMM, or the 16-row passes of the
    // decode-matvec (which also takes this layout)
    const int g0 = wide_splits(m, n, B, cu_count(), false), g1 = wide_splits(m, n, B, cu_count(), true);
    const size_t a = (size_t)(g0 > g1 ? g0 : g1) * B, b = (size_t)L.SG * kMaxTileBatch;
    L.y1p = off; off = align256(off + (a > b ? a : b) * m * 4);
  } else {
    const int sgp = L.SG > L.fused.SG ? L.SG : L.fused.SG;
    L.y1p = off; off = align256(off + (size_t)sgp * B * m * 4);
    if (layout == QS_LAYOUT_TILED) {
      // tagged partial sums of the 16-row decode-matvec that applies the
      // output transform itself (written by no other kernel; only for m on
      // the chunk scheme, bm_tail_eligible)
      L.y1bt = off;
      if (m <= kMaxN) off = align256(off + batched_slot_count(L.SG, B, m) * 8);
    }
  }
  L.total = off;
  return L;
}


// ---------------------------------------------------------------------------
// input transform
// ---------------------------------------------------------------------------
struct XinArgs {
  const void* x;
  int x_dtype;
  int64_t ldx;
  int n, logL, p, G;
  const float* K;
  float scale;
  const float* sv;     // NULL with identity
  int tiled;
  int identity;        // no transform: x2 = x (decode-matvec only)
  _Float16* x2h;
  _Float16* sg;
  float* xtot;  // [B][kMaxParts] partial sums of the rounded group sums
  float* xmul;
  float* x2;
  int frag;     // x2h and sg fragment-major (wide GEMM operands; sg / 4)
};

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

// x2 = T_n(sv (.) x) for one batch row (grid = batch * G).  Tiled path: the
// row is scaled by 2^-e, e from the row's L2 norm (an upper bound of every
// transformed element), and written as fp16 together with the fp16 sums of
// each 8-column group; each of the G work-groups of a row writes the groups
// of its share of the columns b.
__global__ __launch_bounds__(kRowThreads) void xin_kernel(XinArgs A) {
  extern __shared__ float sm[];
  __shared__ float red[kRowThreads / 64];
  float* buf = sm;
  float* Ks = sm + padded_len(A.n);
  const int64_t b = blockIdx.x / A.G;
  const int part = blockIdx.x - (int)(b * A.G);
  const int tid = threadIdx.x, nthr = blockDim.x;
  float ss = 0.0f;
  for (int i = tid; i < A.n; i += nthr) {
    const float v = load_as_float(A.x, A.x_dtype, b * A.ldx + i) * (A.sv ? A.sv[i] : 1.0f);
    buf[pad_idx(i)] = v;
    ss = __builtin_fmaf(v, v, ss);
  }
  if (A.p > 1)
    for (int i = tid; i < A.p * A.p; i += nthr) Ks[i] = A.K[i];
  const float norm2 = block_reduce_sum(ss, red);  // ends with a barrier
  if (!A.identity) lds_fwht(buf, A.n, A.logL, tid, nthr);
  // segment length of the odd-factor stage (the whole row without a transform)
  const int L = A.identity ? A.n : 1 << A.logL;
  if (!A.tiled) {
    if (A.p == 1) {
      for (int i = tid; i < A.n; i += nthr) A.x2[b * A.n + i] = buf[pad_idx(i)] * A.scale;
    } else {
      for (int i = tid; i < A.n; i += nthr) buf[pad_idx(i)] = buf[pad_idx(i)] * A.scale;
      __syncthreads();
      const int cw = L / A.G;
      float* x2 = A.x2 + b * A.n;
      kron_cols(buf, Ks, A.p, A.logL, part * cw, (part + 1) * cw, tid, nthr,
                [&](int a, int c, float v) { x2[(a << A.logL) + c] = v; });
    }
    return;
  }
  int e = 0;
  if (norm2 > 0.0f && norm2 < INFINITY) {
    int ex;
    frexpf(sqrtf(norm2) * 1.0001f, &ex);  // |x2_i| <= ||x|| < 2^ex
    e = ex - 14;
  }
  const float mul = ldexpf(A.scale, -e);
  const int cw = L / A.G;          // columns of this work-group (multiple of 8)
  const int units = A.p * (cw >> 3);
  const int T = A.n >> 3;
  float part_sum = 0.0f;
  for (int u = tid; u < units; u += nthr) {
    const int a = u / (cw >> 3);
    const int c0 = part * cw + ((u - a * (cw >> 3)) << 3);
    float v[8];
    if (A.p == 1) {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = buf[pad_idx(c0 + k)] * mul;
    } else {
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = 0.0f;
      const float* Kr = Ks + a * A.p;
      for (int c = 0; c < A.p; ++c) {
        const float kv = Kr[c];
#pragma unroll
        for (int k = 0; k < 8; ++k) v[k] = __builtin_fmaf(kv, buf[pad_idx(c * L + c0 + k)], v[k]);
      }
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = v[k] * mul;
    }
    const int i0 = a * L + c0;
    _Float16 h[8];
    float gsum = v[0];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      h[k] = (_Float16)v[k];
      if (k) gsum = gsum + v[k];
    }
    const size_t xo = A.frag ? frag_index(b, i0, A.n >> 8) : (size_t)(b * A.n + i0);
    *reinterpret_cast<uint4*>(A.x2h + xo) = __builtin_bit_cast(uint4, h);
    const _Float16 hs = (_Float16)gsum;
    if (A.frag)
      A.sg[sg_frag_index(b, i0 >> 3, A.n >> 8)] = hs * (_Float16)0.25f;
    else
      A.sg[b * T + (i0 >> 3)] = hs;
    part_sum += (float)hs;
  }
  const float tot = block_reduce_sum(part_sum, red);
  if (tid == 0) {
    A.xtot[b * kMaxParts + part] = tot;
    if (part == 0) A.xmul[b] = ldexpf(1.0f, e);
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
  int SG, B, m, logL, p, G;
  int identity;  // no transform: y = layer_scale * y1 (+ bias); su NULL
  const float* K;
  float scale;
  const float* xtot;  // [B][kMaxParts] or NULL on the row-major path
  int xparts;
  const float* xmul;
  float s0, layer_scale;
  const float* su;
  const float* bias;
  void* y;
  int y_dtype;
  int64_t ldy;
};

// y = su (.) T_m(layer_scale * 2^e * (sum of partials - s0 X / 4)) + bias for
// one batch row (grid = batch * G; with an odd factor each work-group
// transforms the whole row and writes its share of the columns).
__global__ __launch_bounds__(kRowThreads) void yout_kernel(YoutArgs A) {
  extern __shared__ float sm[];
  float* buf = sm;
  float* Ks = sm + padded_len(A.m);
  const int b = blockIdx.x / A.G;
  const int part = blockIdx.x - b * A.G;
  const int tid = threadIdx.x, nthr = blockDim.x;
  float xt = 0.0f;
  if (A.xtot)
    for (int j = 0; j < A.xparts; ++j) xt += A.xtot[b * kMaxParts + j];
  const float shift = -0.25f * A.s0 * xt;
  const float mul = A.layer_scale * (A.xmul ? A.xmul[b] : 1.0f);
  for (int i = tid; i < A.m; i += nthr) {
    float s = A.y1p[(size_t)b * A.m + i];
    for (int g = 1; g < A.SG; ++g) s += A.y1p[((size_t)g * A.B + b) * A.m + i];
    buf[pad_idx(i)] = (s + shift) * mul;
  }
  if (A.p > 1)
    for (int i = tid; i < A.p * A.p; i += nthr) Ks[i] = A.K[i];
  __syncthreads();
  if (!A.identity) lds_fwht(buf, A.m, A.logL, tid, nthr);
  if (A.p == 1) {
    for (int i = tid; i < A.m; i += nthr) {
      float v = buf[pad_idx(i)] * A.scale * (A.su ? A.su[i] : 1.0f);
      if (A.bias) v = v + A.bias[i];
      store_from_float(A.y, A.y_dtype, (int64_t)b * A.ldy + i, v);
    }
    return;
  }
  for (int i = tid; i < A.m; i += nthr) buf[pad_idx(i)] = buf[pad_idx(i)] * A.scale;
  __syncthreads();
  const int cw = (1 << A.logL) / A.G;
  kron_cols(buf, Ks, A.p, A.logL, part * cw, (part + 1) * cw, tid, nthr, [&](int a, int c, float v) {
    const int i = (a << A.logL) + c;
    v = v * A.su[i];
    if (A.bias) v = v + A.bias[i];
    store_from_float(A.y, A.y_dtype, (int64_t)b * A.ldy + i, v);
  });
}

// The same output transform with the chunk scheme: one work-group per (batch
// row, output chunk a of 256).  Every work-group sums the partials of all
// chunks and runs their 256-point transforms (a few hundred VALU cycles per
// wave, repeated in each work-group), then forms its own chunk row of
// M = K_p (x) H_{L/256}: y[256 a + t] = sum_c M[a][c] Y[c][t].
// Floats of the chunk buffer: the chunks, and at least the 1024 partial sums
// of the final reduction that reuse it.
__host__ __device__ inline int yc_rows_floats(int Sm) { return Sm * kYStride > 1024 ? Sm * kYStride : 1024; }

struct YcArgs {
  const float* y1p;
  int SG, B, m, Sm, lsh, p;
  const float* K;
  float scale;
  const float* xtot;  // [B][kMaxParts] or NULL
  int xparts;
  const float* xmul;  // [B] or NULL
  float s0, layer_scale;
  const float* su;
  const float* bias;
  void* y;
  int y_dtype;
  int64_t ldy;
};

// Up to QS_MAX_GROUP output transforms in one launch; job g owns the
// work-groups [wg0[g], wg0[g] + B * Sm_g).
struct YcGroup {
  int njobs;
  int wg0[QS_MAX_GROUP];
  YcArgs job[QS_MAX_GROUP];
};

__global__ __launch_bounds__(kRowThreads) void yout_chunk_kernel(YcGroup G) {
  extern __shared__ __attribute__((aligned(16))) float smc[];
  int g = 0;
#pragma unroll
  for (int k = 1; k < QS_MAX_GROUP; ++k)
    if (k < G.njobs && (int)blockIdx.x >= G.wg0[k]) g = k;
  const YcArgs& A = G.job[g];
  const int lb = (int)blockIdx.x - G.wg0[g];
  float* Y = smc;                                   // Sm x kYStride, at least 1024 floats
  float* Ks = smc + yc_rows_floats(A.Sm);           // p x p
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int b = lb / A.Sm, a = lb - b * A.Sm;
  const LaneX lx = lane_x_init();
  float xt = 0.0f;
  if (A.xtot)
    for (int j = 0; j < A.xparts; ++j) xt += A.xtot[b * kMaxParts + j];
  const float shift = -0.25f * A.s0 * xt;
  if (A.p > 1)
    for (int i = tid; i < A.p * A.p; i += kRowThreads) Ks[i] = A.K[i];
  // output element of thread tid < 256 (loads issued early)
  const int io = 256 * a + (tid & 255);
  const float su_o = A.su[io];
  const float bias_o = A.bias ? A.bias[io] : 0.0f;
  float zv[kCPW][4];
#pragma unroll
  for (int u = 0; u < kCPW; ++u) {
    const int c = w + kWaves * u;
#pragma unroll
    for (int j = 0; j < 4; ++j) zv[u][j] = 0.0f;
    if (c < A.Sm) {
      for (int g = 0; g < A.SG; ++g) {
        const float4 v =
            *reinterpret_cast<const float4*>(A.y1p + ((size_t)g * A.B + b) * A.m + 256 * c + 4 * lane);
        zv[u][0] += v.x;
        zv[u][1] += v.y;
        zv[u][2] += v.z;
        zv[u][3] += v.w;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) zv[u][j] += shift;
    }
  }
  h256_chunks(zv, A.Sm, lane, lx);
#pragma unroll
  for (int u = 0; u < kCPW; ++u) {
    const int c = w + kWaves * u;
    if (c < A.Sm)
      *reinterpret_cast<float4*>(Y + c * kYStride + 4 * lane) = make_float4(zv[u][0], zv[u][1], zv[u][2], zv[u][3]);
  }
  __syncthreads();
  // four threads per output column t (one per wave quarter), each over the
  // chunks c = part (mod 4); partial sums meet in LDS
  {
    const int t = tid & 255, part = tid >> 8;
    float acc = 0.0f;
    for (int c = part; c < A.Sm; c += 4) acc = __builtin_fmaf(mmat(a, c, A.lsh, A.p, Ks), Y[c * kYStride + t], acc);
    __syncthreads();  // Y row 0 is reused for the partial sums
    if (part > 0) Y[part * 256 + t] = acc;
    __syncthreads();
    if (part == 0) {
      for (int k = 1; k < 4; ++k) acc += Y[k * 256 + t];
      const float mul = A.scale * A.layer_scale * (A.xmul ? A.xmul[b] : 1.0f);
      store_from_float(A.y, A.y_dtype, (int64_t)b * A.ldy + io, acc * mul * su_o + bias_o);
    }
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

// Fills one job of yout_chunk_kernel (m a multiple of 256, m <= kMaxN,
// m / p >= 256).
YcArgs yc_args(const float* y1p, int SG, int B, int64_t m, int p, const float* K, const float* xtot, int xparts,
               const float* xmul, float s0, float layer_scale, const float* su, const float* bias, void* y,
               int y_dtype, int64_t ldy) {
  YcArgs A{};
  A.y1p = y1p;
  A.SG = SG;
  A.B = B;
  A.m = (int)m;
  A.Sm = (int)(m / 256);
  A.lsh = log2_exact(m / p / 256);
  A.p = p;
  A.K = K;
  A.scale = inv_sqrt_len(m / p);
  A.xtot = xtot;
  A.xparts = xparts;
  A.xmul = xmul;
  A.s0 = s0;
  A.layer_scale = layer_scale;
  A.su = su;
  A.bias = bias;
  A.y = y;
  A.y_dtype = y_dtype;
  A.ldy = ldy;
  return A;
}

int launch_yout_chunk_group(int count, const YcArgs* jobs, hipStream_t s) {
  YcGroup G{};
  G.njobs = count;
  int wg = 0;
  size_t lds = 0;
  for (int g = 0; g < count; ++g) {
    G.job[g] = jobs[g];
    G.wg0[g] = wg;
    wg += jobs[g].B * jobs[g].Sm;
    const size_t need = ((size_t)yc_rows_floats(jobs[g].Sm) + (size_t)jobs[g].p * jobs[g].p) * 4;
    if (need > lds) lds = need;
  }
  QS_REQUIRE(lds <= 65536, "chunk output transform: %zu bytes of LDS", lds);
  hipLaunchKernelGGL(yout_chunk_kernel, dim3((unsigned)wg), dim3(kRowThreads), lds, s, G);
  QS_LAUNCHED("yout_chunk_kernel");
  return QS_OK;
}

int launch_yout_chunk(const float* y1p, int SG, int B, int64_t m, int p, const float* K, const float* xtot,
                      int xparts, const float* xmul, float s0, float layer_scale, const float* su,
                      const float* bias, void* y, int y_dtype, int64_t ldy, hipStream_t s) {
  const YcArgs A = yc_args(y1p, SG, B, m, p, K, xtot, xparts, xmul, s0, layer_scale, su, bias, y, y_dtype, ldy);
  return launch_yout_chunk_group(1, &A, s);
}

// Output transform with the older whole-row kernel (outputs the chunk scheme
// does not cover: m not a multiple of 256, or larger than kMaxN).
int launch_yout_rows(const float* y1p, int SG, int B, int64_t m, int p, const float* K, const float* xtot,
                     int xparts, const float* xmul, float s0, float layer_scale, const float* su, const float* bias,
                     void* y, int y_dtype, int64_t ldy, hipStream_t s, bool identity = false) {
  const int L = identity ? 1 : (int)(m / p);
  const size_t lds = ((size_t)padded_len((int)m) + (size_t)p * p) * 4;
  const int G = identity ? 1 : parts_for(m, p);
  int rc = set_lds((const void*)yout_kernel, lds, &g_yout_lds);
  if (rc) return rc;
  YoutArgs YA{};
  YA.y1p = y1p;
  YA.SG = SG;
  YA.B = B;
  YA.m = (int)m;
  YA.logL = log2_exact(L);
  YA.p = p;
  YA.G = G;
  YA.K = K;
  YA.scale = identity ? 1.0f : inv_sqrt_len(L);
  YA.identity = identity;
  YA.xtot = xtot;
  YA.xparts = xparts;
  YA.xmul = xmul;
  YA.s0 = s0;
  YA.layer_scale = layer_scale;
  YA.su = su;
  YA.bias = bias;
  YA.y = y;
  YA.y_dtype = y_dtype;
  YA.ldy = ldy;
  hipLaunchKernelGGL(yout_kernel, dim3((unsigned)(B * G)), dim3(kRowThreads), lds, s, YA);
  QS_LAUNCHED("yout_kernel");
  return QS_OK;
}

// Input transform of B rows with the LDS-radix kernel (any n the transforms
// allow): fp16 operand rows x2h (fragment-major with frag), group sums sg,
// the rows' 2^e in xmul, partial group-sum totals in xtot.
int launch_xin_rows(const void* x, int x_dtype, int64_t ldx, int64_t B, int64_t n, int p, const float* K,
                    const float* sv, _Float16* x2h, _Float16* sg, float* xtot, float* xmul, int frag, hipStream_t s,
                    bool identity = false) {
  const size_t xin_lds = ((size_t)padded_len((int)n) + (size_t)p * p) * 4;
  const int G = identity ? 1 : parts_for(n, p);
  int rc = set_lds((const void*)xin_kernel, xin_lds, &g_xin_lds);
  if (rc) return rc;
  const int L = identity ? 1 : (int)(n / p);
  XinArgs XA{};
  XA.x = x;
  XA.x_dtype = x_dtype;
  XA.ldx = ldx;
  XA.n = (int)n;
  XA.logL = log2_exact(L);
  XA.p = p;
  XA.G = G;
  XA.K = K;
  XA.scale = identity ? 1.0f : inv_sqrt_len(L);
  XA.sv = sv;
  XA.identity = identity;
  XA.tiled = 1;
  XA.x2h = x2h;
  XA.sg = sg;
  XA.xtot = xtot;
  XA.xmul = xmul;
  XA.x2 = nullptr;
  XA.frag = frag;
  hipLaunchKernelGGL(xin_kernel, dim3((unsigned)(B * G)), dim3(kRowThreads), xin_lds, s, XA);
  QS_LAUNCHED("xin_kernel");
  return QS_OK;
}

int check_transform(int64_t len, int p, const float* K, const char* which) {
  QS_REQUIRE(p >= 1 && (p & 1) && p <= QS_MAX_KRON, "%s: kron factor must be odd in [1, %d]", which, QS_MAX_KRON);
  QS_REQUIRE(len % p == 0, "%s: length %lld not divisible by %d", which, (long long)len, p);
  const int64_t L = len / p;
  QS_REQUIRE((L & (L - 1)) == 0, "%s: length / kron factor must be a power of two", which);
  QS_REQUIRE(p == 1 || K, "%s: kron matrix required", which);
  QS_REQUIRE(len <= kMaxLen, "%s: length %lld exceeds %d", which, (long long)len, kMaxLen);
  return QS_OK;
}

// Spins until the wall clock (100 MHz on gfx9-class parts) has advanced by
// `ticks`, sleeping between reads; the iteration cap bounds the kernel even if
// the clock misbehaves.
__global__ void busy_wait_kernel(uint64_t ticks, uint64_t max_iters) {
  const uint64_t t0 = wall_clock64();
  for (uint64_t it = 0; it < max_iters; ++it) {
    if (wall_clock64() - t0 >= ticks) break;
    __builtin_amdgcn_s_sleep(32);
  }
}

}  // namespace
}  // namespace qs

using namespace qs;

// The wide-batch path (tiled codes, kWideMinBatch rows or more): input
// transform of every row into the fragment-major fp16 operand, the GEMM with
// the decode in its loop on the matrix cores (qs_linear_wide.hip), output
// transform of every row.  The chunk-scheme row kernels take the n and m they
// cover, the LDS-radix kernels the rest.
static int forward_wide(const void* x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int64_t m,
                        const void* codes0, const void* codes1, const float* sv, const float* su, int kron_pn,
                        const float* kron_n, int kron_pm, const float* kron_m, float s0, float s1, float layer_scale,
                        const float* bias, void* y, int y_dtype, int64_t ldy, char* ws, const WsLayout& W,
                        void* mv_begin, void* mv_end, hipStream_t s, int sbits) {
  QS_REQUIRE(batch <= (int64_t)1 << 30, "wide forward: at most 2^30 rows");
  BatchedPass P{};
  P.x = x;
  P.x_dtype = x_dtype;
  P.ldx = ldx;
  P.B = (int)batch;
  P.n = n;
  P.m = m;
  P.pn = kron_pn;
  P.pm = kron_pm;
  P.Kn = kron_n;
  P.Km = kron_m;
  P.sv = sv;
  P.su = su;
  P.layer_scale = layer_scale;
  P.bias = bias;
  P.y = y;
  P.y_dtype = y_dtype;
  P.ldy = ldy;
  P.SG = 1;
  P.ncu = cu_count();
  P.x2h = reinterpret_cast<_Float16*>(ws + W.x2h);
  P.sg = reinterpret_cast<_Float16*>(ws + W.sg);
  P.xmul = reinterpret_cast<float*>(ws + W.xmul);
  P.y1p = reinterpret_cast<float*>(ws + W.y1p);
  P.frag = 1;
  P.sbits = sbits;
  int rc = QS_OK;
  const bool sv_aligned = (reinterpret_cast<uintptr_t>(sv) & (sbits ? 3 : 15)) == 0;
  if (chunk_transform_fits(n, kron_pn) && sv_aligned)
    rc = launch_bx_rows(P, s);
  else if (big_input_fits(n, kron_pn, x_dtype) && sv_aligned && fused_x_aligned(x, x_dtype, ldx))
    rc = launch_bx_big(P, s);
  else
    rc = launch_xin_rows(x, x_dtype, ldx, batch, n, kron_pn, kron_n, sv, P.x2h, P.sg, reinterpret_cast<float*>(ws + W.xtot),
                         P.xmul, P.frag, s);
  if (rc) return rc;

  if (mv_begin) QS_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(mv_begin), s));
  WideMfma F{};
  F.codes0 = codes0;
  F.codes1 = codes1;
  F.m = m;
  F.n = n;
  F.B = (int)batch;
  F.s0 = s0;
  F.s1 = s1;
  F.x2f = P.x2h;
  F.sgf = P.sg;
  F.y1p = P.y1p;
  F.SGk = wide_splits(m, n, batch, cu_count(), codes1 != nullptr);
  rc = launch_linear_wide_mfma(F, s);
  if (rc) return rc;
  if (mv_end) QS_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(mv_end), s));
  // partial groups summed by the output kernels; the +-1/4 shifts are in y1
  P.SG = F.SGk;
  if (chunk_transform_fits(m, kron_pm)) return launch_by_rows(P, s);
  if (big_transform_fits(m, kron_pm)) return launch_by_big(&P, 1, s);
  return launch_yout_rows(P.y1p, F.SGk, (int)batch, m, kron_pm, kron_m, nullptr, 0, P.xmul, s0, layer_scale, su, bias,
                          y, y_dtype, ldy, s);
}

// The batched path (and the decode-matvec without transforms): per block of
// up to 16 batch rows, input transform -> decode-matvec -> output transform.
static int forward_batched(const void* x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int64_t m,
                    const void* codes0, const void* codes1, int kind1, int layout, const float* sv, const float* su,
                    int kron_pn, const float* kron_n, int kron_pm, const float* kron_m, float s0, float s1,
                    float layer_scale, const float* bias, void* y, int y_dtype, int64_t ldy, char* ws,
                    size_t ws_bytes, const WsLayout& W, void* mv_begin, void* mv_end, hipStream_t s, bool identity,
                    int sbits = 0) {
  int rc = QS_OK;
  if (!identity && W.wide)
    return forward_wide(x, x_dtype, ldx, batch, n, m, codes0, codes1, sv, su, kron_pn, kron_n, kron_pm, kron_m, s0, s1,
                        layer_scale, bias, y, y_dtype, ldy, ws, W, mv_begin, mv_end, s, sbits);
  if (layout == QS_LAYOUT_TILED) {
    // passes of up to 16 rows: input transform, decode-matvec on all 16 MFMA
    // columns, output transform (qs_linear_batched.hip); an n or m outside
    // the chunk scheme takes the LDS-radix row kernel for that side
    const bool sv_aligned = (reinterpret_cast<uintptr_t>(sv) & (sbits ? 3 : 15)) == 0;
    for (int64_t b0 = 0; b0 < batch; b0 += kMaxTileBatch) {
      BatchedPass P{};
      P.B = (int)(batch - b0 < kMaxTileBatch ? batch - b0 : kMaxTileBatch);
      P.x = static_cast<const char*>(x) + (size_t)b0 * ldx * dtype_bytes(x_dtype);
      P.x_dtype = x_dtype;
      P.ldx = ldx;
      P.n = n;
      P.m = m;
      P.pn = kron_pn;
      P.pm = kron_pm;
      P.Kn = kron_n;
      P.Km = kron_m;
      P.sv = sv;
      P.su = su;
      P.codes0 = codes0;
      P.codes1 = codes1;
      P.s0 = s0;
      P.s1 = s1;
      P.layer_scale = layer_scale;
      P.bias = bias;
      P.y = static_cast<char*>(y) + (size_t)b0 * ldy * dtype_bytes(y_dtype);
      P.y_dtype = y_dtype;
      P.ldy = ldy;
      P.S = W.S;
      P.SG = W.SG;
      P.W = W.W;
      P.ncu = cu_count();
      P.x2h = reinterpret_cast<_Float16*>(ws + W.x2h);
      P.sg = reinterpret_cast<_Float16*>(ws + W.sg);
      P.xmul = reinterpret_cast<float*>(ws + W.xmul);
      P.y1p = reinterpret_cast<float*>(ws + W.y1p);
      P.frag = 1;
      P.sbits = sbits;
      hipEvent_t ev0 = b0 == 0 ? reinterpret_cast<hipEvent_t>(mv_begin) : nullptr;
      hipEvent_t ev1 = b0 + kMaxTileBatch >= batch ? reinterpret_cast<hipEvent_t>(mv_end) : nullptr;
      if (!identity && batched_eligible(n, kron_pn, m, kron_pm) && sv_aligned) {
        P.y1t = reinterpret_cast<unsigned long long*>(ws + W.y1bt);  // output transform in the decode-matvec
        P.epoch = reinterpret_cast<unsigned*>(ws);
        P.tw = tag_ws(ws, ws_bytes, 0);
        rc = launch_linear_batched(P, s, ev0, ev1);
      } else {
        if (!identity && chunk_transform_fits(n, kron_pn) && sv_aligned)
          rc = launch_bx_rows(P, s);
        else if (!identity && big_input_fits(n, kron_pn, x_dtype) && sv_aligned &&
                 fused_x_aligned(P.x, x_dtype, ldx))
          rc = launch_bx_big(P, s);
        else
          rc = launch_xin_rows(P.x, x_dtype, ldx, P.B, n, kron_pn, kron_n, sv, P.x2h, P.sg,
                               reinterpret_cast<float*>(ws + W.xtot), P.xmul, P.frag, s, identity);
        // m on the chunk scheme: the decode-matvec applies the output
        // transform itself where it can (tagged slots), whatever n
        bool tail = false;
        if (!identity && chunk_transform_fits(m, kron_pm)) {
          P.y1t = reinterpret_cast<unsigned long long*>(ws + W.y1bt);
          P.epoch = reinterpret_cast<unsigned*>(ws);
          P.tw = tag_ws(ws, ws_bytes, 0);
        }
        if (!rc) rc = launch_bm(P, s, ev0, ev1, &tail);
        if (!rc && tail) {
          // done in the decode-matvec
        } else if (!rc && !identity && chunk_transform_fits(m, kron_pm))
          rc = launch_by_rows(P, s);
        else if (!rc && !identity && big_transform_fits(m, kron_pm))
          rc = launch_by_big(&P, 1, s);
        else if (!rc)
          rc = launch_yout_rows(P.y1p, P.SG, P.B, m, kron_pm, kron_m, nullptr, 0, P.xmul, s0, layer_scale, su, bias,
                                P.y, y_dtype, ldy, s, identity);
      }
      if (rc) return rc;
    }
    return QS_OK;
  }
  // row-major (generic) code layout: fp32 operand rows, vector-unit decode-matvec
  const int Ln = identity ? 1 : (int)(n / kron_pn);
  const size_t xin_lds = ((size_t)padded_len((int)n) + (size_t)kron_pn * kron_pn) * 4;
  const int Gx = identity ? 1 : parts_for(n, kron_pn);
  rc = set_lds((const void*)xin_kernel, xin_lds, &g_xin_lds);
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
    XA.logL = log2_exact(Ln);
    XA.p = kron_pn;
    XA.G = Gx;
    XA.K = kron_n;
    XA.scale = identity ? 1.0f : inv_sqrt_len(Ln);
    XA.sv = sv;
    XA.identity = identity;
    XA.tiled = 0;
    XA.x2 = reinterpret_cast<float*>(ws + W.x2);
    hipLaunchKernelGGL(xin_kernel, dim3(B * Gx), dim3(kRowThreads), xin_lds, s, XA);
    QS_LAUNCHED("xin_kernel");

    float* y1p = reinterpret_cast<float*>(ws + W.y1p);
    hipEvent_t ev0 = b0 == 0 ? reinterpret_cast<hipEvent_t>(mv_begin) : nullptr;
    hipEvent_t ev1 = b0 + kMaxTileBatch >= batch ? reinterpret_cast<hipEvent_t>(mv_end) : nullptr;
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
    hipExtLaunchKernelGGL(mv_generic_kernel, dim3((unsigned)((m + 3) / 4)), dim3(256), 0, s, ev0, ev1, 0, GA);
    QS_LAUNCHED("mv_generic_kernel");
    rc = launch_yout_rows(y1p, W.SG, B, m, kron_pm, kron_m, nullptr, 0, nullptr, s0, layer_scale, su, bias, yb,
                          y_dtype, ldy, s, identity);
    if (rc) return rc;
  }
  return QS_OK;
}


extern "C" int qs_busy_wait(int64_t nanoseconds, qs_stream_t stream) {
  QS_REQUIRE(nanoseconds >= 0 && nanoseconds <= 1000000000ll, "busy wait must be in [0, 1 s]");
  int dev = 0, khz = 0;
  QS_HIP(hipGetDevice(&dev));
  QS_HIP(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev));
  if (khz <= 0) khz = 100000;
  const uint64_t ticks = (uint64_t)((double)nanoseconds * khz / 1e6);
  // a sleep of 32 units is at least ~0.8 us, so ns/100 iterations outlast the wait
  const uint64_t max_iters = (uint64_t)nanoseconds / 100 + 1000;
  hipLaunchKernelGGL(busy_wait_kernel, dim3(1), dim3(64), 0, as_stream(stream), ticks, max_iters);
  QS_LAUNCHED("busy_wait_kernel");
  return QS_OK;
}

extern "C" size_t qs_linear_workspace_bytes(int64_t m, int64_t n, int64_t batch, int layout) {
  if (m <= 0 || n <= 0 || batch <= 0) return 0;
  return ws_layout(m, n, batch, layout).total;
}

extern "C" int qs_linear_forward(const void* x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int64_t m,
                                 const void* codes0, const void* codes1, int kind1, int layout, const float* sv,
                                 const float* su, int kron_pn, const float* kron_n, int kron_pm,
                                 const float* kron_m, float s0, float s1, float layer_scale, const float* bias,
                                 void* y, int y_dtype, int64_t ldy, void* workspace, size_t workspace_bytes,
                                 void* mv_begin, void* mv_end, qs_stream_t stream) {
  QS_REQUIRE(batch >= 0 && n > 0 && m > 0 && n % 8 == 0, "bad shape batch=%lld n=%lld m=%lld", (long long)batch,
             (long long)n, (long long)m);
  QS_REQUIRE(x_dtype >= QS_DTYPE_F32 && x_dtype <= QS_DTYPE_BF16 && y_dtype >= QS_DTYPE_F32 &&
                 y_dtype <= QS_DTYPE_BF16,
             "bad dtype");
  const int sbits = (layout & QS_SIGNS_BITS) ? 1 : 0;
  layout &= ~QS_SIGNS_BITS;
  QS_REQUIRE(layout == QS_LAYOUT_TILED || layout == QS_LAYOUT_ROWMAJOR, "bad layout");
  if (batch == 0) return QS_OK;
  QS_REQUIRE(x && y && codes0 && sv && su && workspace, "null pointer");
  QS_REQUIRE(ldx >= n && ldy >= m, "row strides too small");
  int rc = check_transform(n, kron_pn, kron_n, "input");
  if (rc) return rc;
  rc = check_transform(m, kron_pm, kron_m, "output");
  if (rc) return rc;
  if (sbits) {
    // every kernel of the chunk scheme reads sign bits; beyond it, the
    // one-launch kernel with its output transform in the launch
    const bool one = layout == QS_LAYOUT_TILED && fused_eligible(batch, n, x_dtype, kron_pn) &&
                     fused_x_aligned(x, x_dtype, ldx) && fused_output_in_kernel(m, kron_pm);
    QS_SUPPORTED(one || (layout == QS_LAYOUT_TILED && chunk_transform_fits(n, kron_pn) &&
                         chunk_transform_fits(m, kron_pm)),
                 "packed sign bits need the tiled layout with n and m on the chunk scheme, or a one-launch "
                 "call (1-2 aligned rows, m and n up to 32768) (got m %lld, n %lld, %lld rows)",
                 (long long)m, (long long)n, (long long)batch);
    QS_REQUIRE((reinterpret_cast<uintptr_t>(sv) & 3) == 0 && (reinterpret_cast<uintptr_t>(su) & 3) == 0,
               "packed sign bits must be 4-byte aligned");
  }
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
  if (layout == QS_LAYOUT_TILED && fused_eligible(batch, n, x_dtype, kron_pn) && fused_x_aligned(x, x_dtype, ldx) &&
      (reinterpret_cast<uintptr_t>(sv) & (sbits ? 3 : 15)) == 0) {
    FusedJobDesc d{};
    d.codes0 = codes0;
    d.codes1 = codes1;
    d.m = m;
    d.sv = sv;
    d.su = su;
    d.pm = kron_pm;
    d.Km = kron_m;
    d.s0 = s0;
    d.s1 = s1;
    d.layer_scale = layer_scale;
    d.bias = bias;
    d.y = y;
    d.ldy = ldy;
    d.epoch = reinterpret_cast<unsigned*>(ws);
    d.tw = tag_ws(ws, workspace_bytes, 0);
    d.xmul = reinterpret_cast<float*>(ws + W.xmul);
    d.y1p = reinterpret_cast<float*>(ws + W.y1p);
    d.y1t = reinterpret_cast<unsigned long long*>(ws + W.y1t);
    d.h2t = reinterpret_cast<unsigned long long*>(ws + W.h2t);
    rc = launch_linear_fused(x, x_dtype, ldx, (int)batch, (int)n, kron_pn, kron_n, y_dtype, sbits, 1, &d, W.S, W.fused,
                             cu_count(), s, reinterpret_cast<hipEvent_t>(mv_begin),
                             reinterpret_cast<hipEvent_t>(mv_end));
    if (rc) return rc;
    if (fused_output_in_kernel(m, kron_pm)) return QS_OK;
    // the output kernels below read su as m fp32 values
    QS_REQUIRE(!sbits, "packed sign bits reached an fp32-sign output path (m %lld)", (long long)m);
    if (chunk_transform_fits(m, kron_pm))
      return launch_yout_chunk(d.y1p, W.fused.SG, (int)batch, m, kron_pm, kron_m, nullptr, 0, d.xmul, s0, layer_scale,
                               su, bias, y, y_dtype, ldy, s);
    return launch_yout_rows(d.y1p, W.fused.SG, (int)batch, m, kron_pm, kron_m, nullptr, 0, d.xmul, s0, layer_scale, su,
                            bias, y, y_dtype, ldy, s);
  }
  return forward_batched(x, x_dtype, ldx, batch, n, m, codes0, codes1, kind1, layout, sv, su, kron_pn, kron_n,
                         kron_pm, kron_m, s0, s1, layer_scale, bias, y, y_dtype, ldy, ws, workspace_bytes, W, mv_begin,
                         mv_end, s, false, sbits);
}

// ---------------------------------------------------------------------------
// Allocation-free forward: the workspace lives in a file-scope device array
// ---------------------------------------------------------------------------
// `scratch` is part of the library's code object: each GPU the library runs
// on holds one copy (QS_NOALLOC_SCRATCH_BYTES) from load until the process
// ends, zero-filled at load.  Host code never passes the array's name to a
// kernel (on the host it only names a stand-in): the device address comes
// from hipGetSymbolAddress, looked up once per device with that device
// current, and only that address is used.
static __device__ __align__(256) char scratch[QS_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// Device address of `scratch` on the current device.
int scratch_address(void** out) {
  int dev = 0;
  QS_HIP(hipGetDevice(&dev));
  QS_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (!p) {
    QS_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    QS_REQUIRE(p != nullptr, "no device address for the scratch array");
    g_scratch_ptr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  return QS_OK;
}
}  // namespace

extern "C" int qs_linear_forward_noalloc(const void* x, int x_dtype, int64_t ldx, int64_t batch, int64_t n,
                                         int64_t m, const void* codes0, const void* codes1, int kind1, int layout,
                                         const float* sv, const float* su, int kron_pn, const float* kron_n,
                                         int kron_pm, const float* kron_m, float s0, float s1, float layer_scale,
                                         const float* bias, void* y, int y_dtype, int64_t ldy, qs_stream_t stream) {
  QS_REQUIRE(batch >= 0 && n > 0 && m > 0, "bad shape batch=%lld n=%lld m=%lld", (long long)batch, (long long)n,
             (long long)m);
  const int lay = layout & ~QS_SIGNS_BITS;
  QS_REQUIRE(lay == QS_LAYOUT_TILED || lay == QS_LAYOUT_ROWMAJOR, "bad layout");
  if (batch == 0) return QS_OK;
  const size_t need = ws_layout(m, n, batch, lay).total;
  QS_SUPPORTED(need <= QS_NOALLOC_SCRATCH_BYTES,
               "qs_linear_forward_noalloc: m %lld, n %lld, %lld rows need %zu bytes of scratch; the "
               "allocation-free forward has %zu (use qs_linear_forward with a workspace)",
               (long long)m, (long long)n, (long long)batch, need, (size_t)QS_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc) return rc;
  return qs_linear_forward(x, x_dtype, ldx, batch, n, m, codes0, codes1, kind1, layout, sv, su, kron_pn, kron_n,
                           kron_pm, kron_m, s0, s1, layer_scale, bias, y, y_dtype, ldy, ws,
                           QS_NOALLOC_SCRATCH_BYTES, nullptr, nullptr, stream);
}

// Grouped workspace.  A 256-byte header holding the one-launch kernel's
// epoch word of each job index (job g at byte 4 g; a single-linear call uses
// the word of job 0, at offset 0 of its own layout too), then one block per
// job for the one-launch kernel (1-2 rows) at offsets that do not depend on
// the call's row count: [tagged partial sums of up to two rows | tagged chunk
// transforms of up to two rows | row multipliers | fp32 partial sums of up to
// two rows (output transform in a separate kernel)]; then one ws_layout
// region per job for the kernels of wider calls.  The tags carry the job
// index and a per-index launch counter, so calls with other job lists (or
// single calls) sharing the workspace cannot leave slots that pass for this
// call's.
struct FusedBlock {
  size_t y1t, h2t, xmul, y1p, total;  // offsets within the job's block
};
constexpr size_t kGroupHeader = 256;
FusedBlock fused_block(int64_t m, int64_t n) {
  const WsLayout W = ws_layout(m, n, 2, QS_LAYOUT_TILED);
  FusedBlock F{};
  F.y1t = 0;
  F.h2t = F.y1t + align256(fused_slot_count(W.fused.SG, m) * 8);
  F.xmul = F.h2t + align256(h2_slot_count(m) * 8);
  F.y1p = F.xmul + 256;
  F.total = F.y1p + align256((size_t)W.fused.SG * 2 * (size_t)m * 4);
  return F;
}
template <class M>
size_t group_prefix_bytes(int count, int64_t n, M m_of) {
  size_t total = kGroupHeader;
  for (int g = 0; g < count; ++g) total += fused_block(m_of(g), n).total;
  return total;
}

// Grouped forward for three or more rows: the input transforms of all the
// linears in one launch, their decode-matvecs in one launch (16-row pass) or
// one wide GEMM each (kWideMinBatch rows and more; above 128 rows one GEMM
// for linears of one shape whose tiles fit one round over the CUs), and their
// output transforms in one launch (a linear whose m is outside the chunk
// scheme: the whole-row output kernel).  Bit-identical to one
// qs_linear_forward per linear, except a shared GEMM: its slice groups are the
// group's, so the outputs equal separate calls up to the fp32 summation order.
static int forward_group_rows(const void* x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int kron_pn,
                              const float* kron_n, int count, const qs_linear_job* jobs, int y_dtype, char* ws,
                              size_t ws_bytes, void* mv_begin, void* mv_end, hipStream_t s, int sbits,
                              const FusedPre* pre) {
  const bool wide = batch >= kWideMinBatch;
  BatchedPass P[QS_MAX_GROUP];
  size_t off = group_prefix_bytes(count, n, [&](int g) { return jobs[g].m; });
  for (int g = 0; g < count; ++g) {
    const qs_linear_job& j = jobs[g];
    const WsLayout W = ws_layout(j.m, n, batch, QS_LAYOUT_TILED);
    BatchedPass& Q = P[g];
    Q = BatchedPass{};
    Q.x = x;
    Q.x_dtype = x_dtype;
    Q.ldx = ldx;
    Q.B = (int)batch;
    Q.n = n;
    Q.m = j.m;
    Q.pn = kron_pn;
    Q.pm = j.kron_pm;
    Q.Kn = kron_n;
    Q.Km = j.kron_m;
    Q.sv = j.sv;
    Q.su = j.su;
    Q.codes0 = j.codes0;
    Q.codes1 = j.codes1;
    Q.s0 = j.s0;
    Q.s1 = j.s1;
    Q.layer_scale = j.layer_scale;
    Q.bias = j.bias;
    Q.y = j.y;
    Q.y_dtype = y_dtype;
    Q.ldy = j.ldy;
    Q.S = W.S;
    Q.SG = W.SG;
    Q.W = W.W;
    Q.ncu = cu_count();
    Q.x2h = reinterpret_cast<_Float16*>(ws + off + W.x2h);
    Q.sg = reinterpret_cast<_Float16*>(ws + off + W.sg);
    Q.xmul = reinterpret_cast<float*>(ws + off + W.xmul);
    Q.y1p = reinterpret_cast<float*>(ws + off + W.y1p);
    Q.frag = 1;
    Q.sbits = sbits;
    if (!wide) {
      Q.y1t = reinterpret_cast<unsigned long long*>(ws + off + W.y1bt);
      Q.epoch = reinterpret_cast<unsigned*>(ws) + g;
      Q.tw = tag_ws(ws, ws_bytes, g);
    }
    off += W.total;
  }
  int rc = launch_bx_group(P, count, s, pre);
  if (rc) return rc;
  if (wide) {
    if (mv_begin) QS_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(mv_begin), s));
    // linears of one shape whose tiles fit one round over the CUs: one GEMM
    // launch with the slice groups chosen for the group
    bool one_shape = true;
    for (int g = 0; g < count; ++g) one_shape = one_shape && P[g].m == P[0].m && P[g].codes1 == nullptr;
    const int gsk = one_shape ? wide_group_splits(P[0].m, n, batch, count, cu_count()) : 0;
    WideMfma F[QS_MAX_GROUP];
    for (int g = 0; g < count; ++g) {
      F[g] = WideMfma{};
      F[g].codes0 = P[g].codes0;
      F[g].codes1 = P[g].codes1;
      F[g].m = P[g].m;
      F[g].n = n;
      F[g].B = (int)batch;
      F[g].s0 = P[g].s0;
      F[g].s1 = P[g].s1;
      F[g].x2f = P[g].x2h;
      F[g].sgf = P[g].sg;
      F[g].y1p = P[g].y1p;
      F[g].SGk = gsk ? gsk : wide_splits(P[g].m, n, batch, cu_count(), P[g].codes1 != nullptr);
      if (!gsk) {
        rc = launch_linear_wide_mfma(F[g], s);
        if (rc) return rc;
      }
      P[g].SG = F[g].SGk;  // partial groups summed by the output kernels
    }
    if (gsk) {
      rc = launch_linear_wide_group(F, count, s);
      if (rc) return rc;
    }
    if (mv_end) QS_HIP(hipEventRecord(reinterpret_cast<hipEvent_t>(mv_end), s));
  } else {
    bool tail = false;
    rc = launch_bm_group(P, count, s, reinterpret_cast<hipEvent_t>(mv_begin), reinterpret_cast<hipEvent_t>(mv_end),
                         &tail);
    if (rc) return rc;
    if (tail) return QS_OK;  // the decode-matvec applied the output transforms
  }
  // output transforms: the chunk-scheme ones in one launch, those up to
  // 32768 in another, the others one by one
  BatchedPass Pc[QS_MAX_GROUP], Pb[QS_MAX_GROUP];
  int nc = 0, nb = 0;
  for (int g = 0; g < count; ++g) {
    if (chunk_transform_fits(P[g].m, P[g].pm)) {
      Pc[nc++] = P[g];
      continue;
    }
    if (big_transform_fits(P[g].m, P[g].pm)) {
      Pb[nb++] = P[g];
      continue;
    }
    rc = launch_yout_rows(P[g].y1p, P[g].SG, (int)batch, P[g].m, P[g].pm, P[g].Km, nullptr, 0, P[g].xmul, P[g].s0,
                          P[g].layer_scale, P[g].su, P[g].bias, P[g].y, y_dtype, P[g].ldy, s);
    if (rc) return rc;
  }
  if (nb) {
    rc = launch_by_big(Pb, nb, s);
    if (rc) return rc;
  }
  return nc ? launch_by_group(Pc, nc, s) : QS_OK;
}

extern "C" size_t qs_linear_group_workspace_bytes(int64_t n, int64_t batch, int count, const int64_t* ms) {
  if (n <= 0 || batch <= 0 || count < 1 || count > QS_MAX_GROUP || !ms) return 0;
  for (int g = 0; g < count; ++g)
    if (ms[g] <= 0) return 0;
  size_t total = group_prefix_bytes(count, n, [&](int g) { return ms[g]; });
  for (int g = 0; g < count; ++g) total += ws_layout(ms[g], n, batch, QS_LAYOUT_TILED).total;
  return total;
}

static int forward_group_impl(const void* x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int kron_pn,
                              const float* kron_n, int count, const qs_linear_job* jobs, int y_dtype,
                              void* workspace, size_t workspace_bytes, void* mv_begin, void* mv_end,
                              qs_stream_t stream, const FusedPre* pre) {
  QS_REQUIRE(count >= 1 && count <= QS_MAX_GROUP, "count must be in [1, %d]", QS_MAX_GROUP);
  QS_REQUIRE(jobs && x && workspace, "null pointer");
  QS_REQUIRE(x_dtype >= QS_DTYPE_F32 && x_dtype <= QS_DTYPE_BF16 && y_dtype >= QS_DTYPE_F32 &&
                 y_dtype <= QS_DTYPE_BF16,
             "bad dtype");
  QS_REQUIRE(batch >= 0 && n > 0 && ldx >= n, "bad shape batch=%lld n=%lld", (long long)batch, (long long)n);
  if (batch == 0) return QS_OK;
  int rc = check_transform(n, kron_pn, kron_n, "input");
  if (rc) return rc;
  const bool one_launch = fused_eligible(batch, n, x_dtype, kron_pn) && fused_x_aligned(x, x_dtype, ldx);
  QS_REQUIRE(n % 256 == 0 && n / kron_pn >= 256,
             "grouped forward needs n a multiple of 256 with n / kron_pn >= 256 (got n %lld)", (long long)n);
  if (pre)
    QS_SUPPORTED(one_launch || (batch >= 3 && batch <= 16 && chunk_transform_fits(n, kron_pn)),
                 "a pre-operation runs in one-launch calls (1-2 rows) and in 3-16 row calls on the chunk scheme "
                 "(batch %lld, n %lld)",
                 (long long)batch, (long long)n);
  QS_REQUIRE((reinterpret_cast<uintptr_t>(workspace) & 255) == 0, "workspace must be 256-byte aligned");
  size_t need = 0;
  for (int g = 0; g < count; ++g) {
    const qs_linear_job& j = jobs[g];
    QS_REQUIRE(j.codes0 && j.su && j.sv && j.y, "job %d: null pointer", g);
    QS_REQUIRE(j.m > 0 && j.m % 16 == 0 && j.ldy >= j.m, "job %d: bad m %lld / ldy", g, (long long)j.m);
    rc = check_transform(j.m, j.kron_pm, j.kron_m, "output");
    if (rc) return rc;
    QS_REQUIRE((j.sign_bits != 0) == (jobs[0].sign_bits != 0), "all jobs need the same sign format");
    QS_REQUIRE((reinterpret_cast<uintptr_t>(j.codes0) & 15) == 0 &&
                   (!j.codes1 || (reinterpret_cast<uintptr_t>(j.codes1) & 7) == 0) &&
                   (reinterpret_cast<uintptr_t>(j.sv) & (j.sign_bits ? 3 : 15)) == 0 &&
                   (reinterpret_cast<uintptr_t>(j.su) & 3) == 0,
               "job %d: packed codes and sv must be 16-byte aligned (4 bytes for sign bits)", g);
    if (j.sign_bits)
      QS_SUPPORTED(one_launch ? fused_output_in_kernel(j.m, j.kron_pm)
                              : chunk_transform_fits(n, kron_pn) && chunk_transform_fits(j.m, j.kron_pm),
                   "job %d: packed sign bits need m and n on the chunk scheme, or a one-launch call (got m %lld)",
                   g, (long long)j.m);
    QS_REQUIRE((j.codes1 != nullptr) == (jobs[0].codes1 != nullptr), "all jobs need the same number of stages");
    need += ws_layout(j.m, n, batch, QS_LAYOUT_TILED).total;
  }
  need += group_prefix_bytes(count, n, [&](int g) { return jobs[g].m; });
  QS_REQUIRE(workspace_bytes >= need, "workspace too small: %zu < %zu", workspace_bytes, need);
  hipStream_t s = as_stream(stream);
  char* ws = static_cast<char*>(workspace);
  if (!one_launch && chunk_transform_fits(n, kron_pn))
    return forward_group_rows(x, x_dtype, ldx, batch, n, kron_pn, kron_n, count, jobs, y_dtype, ws, workspace_bytes,
                              mv_begin, mv_end, s, jobs[0].sign_bits ? 1 : 0, pre);
  if (!one_launch) {
    // n outside the chunk scheme of the multi-row kernels: one forward per
    // linear, one after the other on the stream, each with the whole
    // workspace (so that its tags continue the workspace's epoch of job 0)
    for (int g = 0; g < count; ++g) {
      const qs_linear_job& j = jobs[g];
      rc = qs_linear_forward(x, x_dtype, ldx, batch, n, j.m, j.codes0, j.codes1, QS_STAGE_E8_1BIT,
                             QS_LAYOUT_TILED | (j.sign_bits ? QS_SIGNS_BITS : 0), j.sv, j.su, kron_pn, kron_n,
                             j.kron_pm, j.kron_m, j.s0, j.s1, j.layer_scale, j.bias, j.y, y_dtype, j.ldy, workspace,
                             workspace_bytes, g == 0 ? mv_begin : nullptr, g == count - 1 ? mv_end : nullptr, stream);
      if (rc) return rc;
    }
    return QS_OK;
  }
  FusedJobDesc d[QS_MAX_GROUP];
  const WsLayout W0 = ws_layout(jobs[0].m, n, batch, QS_LAYOUT_TILED);
  size_t off = kGroupHeader;  // the job's block
  for (int g = 0; g < count; ++g) {
    const qs_linear_job& j = jobs[g];
    const FusedBlock F = fused_block(j.m, n);
    d[g] = FusedJobDesc{};
    d[g].codes0 = j.codes0;
    d[g].codes1 = j.codes1;
    d[g].m = j.m;
    d[g].sv = j.sv;
    d[g].su = j.su;
    d[g].pm = j.kron_pm;
    d[g].Km = j.kron_m;
    d[g].s0 = j.s0;
    d[g].s1 = j.s1;
    d[g].layer_scale = j.layer_scale;
    d[g].bias = j.bias;
    d[g].y = j.y;
    d[g].ldy = j.ldy;
    d[g].epoch = reinterpret_cast<unsigned*>(ws) + g;
    d[g].tw = tag_ws(ws, workspace_bytes, g);
    d[g].xmul = reinterpret_cast<float*>(ws + off + F.xmul);
    d[g].y1p = reinterpret_cast<float*>(ws + off + F.y1p);
    d[g].y1t = reinterpret_cast<unsigned long long*>(ws + off + F.y1t);
    d[g].h2t = reinterpret_cast<unsigned long long*>(ws + off + F.h2t);
    off += F.total;
  }
  rc = launch_linear_fused(x, x_dtype, ldx, (int)batch, (int)n, kron_pn, kron_n, y_dtype, jobs[0].sign_bits ? 1 : 0,
                           count, d, W0.S, W0.fused, cu_count(), s, reinterpret_cast<hipEvent_t>(mv_begin),
                           reinterpret_cast<hipEvent_t>(mv_end), pre);
  if (rc) return rc;
  // outputs the kernel did not finish: chunked ones in one launch, others per job
  YcArgs yc[QS_MAX_GROUP];
  int nyc = 0;
  for (int g = 0; g < count; ++g) {
    const qs_linear_job& j = jobs[g];
    if (fused_output_in_kernel(j.m, j.kron_pm)) continue;
    // the output kernels below read su as m fp32 values
    QS_REQUIRE(!j.sign_bits, "job %d: packed sign bits reached an fp32-sign output path (m %lld)", g, (long long)j.m);
    if (chunk_transform_fits(j.m, j.kron_pm)) {
      yc[nyc++] = yc_args(d[g].y1p, W0.fused.SG, (int)batch, j.m, j.kron_pm, j.kron_m, nullptr, 0, d[g].xmul, j.s0,
                          j.layer_scale, j.su, j.bias, j.y, y_dtype, j.ldy);
    } else {
      rc = launch_yout_rows(d[g].y1p, W0.fused.SG, (int)batch, j.m, j.kron_pm, j.kron_m, nullptr, 0, d[g].xmul, j.s0,
                            j.layer_scale, j.su, j.bias, j.y, y_dtype, j.ldy, s);
      if (rc) return rc;
    }
  }
  if (nyc) return launch_yout_chunk_group(nyc, yc, s);
  return QS_OK;
}

extern "C" int qs_linear_forward_group(const void* x, int x_dtype, int64_t ldx, int64_t batch, int64_t n,
                                       int kron_pn, const float* kron_n, int count, const qs_linear_job* jobs,
                                       int y_dtype, void* workspace, size_t workspace_bytes, void* mv_begin,
                                       void* mv_end, qs_stream_t stream) {
  return forward_group_impl(x, x_dtype, ldx, batch, n, kron_pn, kron_n, count, jobs, y_dtype, workspace,
                            workspace_bytes, mv_begin, mv_end, stream, nullptr);
}

// [a, a + abytes) and [b, b + bbytes) share a byte
static bool overlaps(const void* a, size_t abytes, const void* b, size_t bbytes) {
  const uintptr_t pa = reinterpret_cast<uintptr_t>(a), pb = reinterpret_cast<uintptr_t>(b);
  return pa < pb + bbytes && pb < pa + abytes;
}

extern "C" int qs_linear_forward_group_pre(const void* x, int64_t ldx, int64_t batch, int64_t n, int kron_pn,
                                           const float* kron_n, int count, const qs_linear_job* jobs,
                                           const qs_preop* pre, int y_dtype, void* workspace,
                                           size_t workspace_bytes, qs_stream_t stream) {
  QS_REQUIRE(pre && x, "null pointer");
  QS_REQUIRE(pre->kind == QS_PREOP_RMSNORM, "bad pre-operation kind %d", pre->kind);
  QS_REQUIRE(batch >= 0 && n > 0 && ldx >= n, "bad shape batch=%lld n=%lld", (long long)batch, (long long)n);
  if (batch == 0) return QS_OK;
  QS_REQUIRE(pre->weight != nullptr, "RMSNorm pre-operation: null weight");
  QS_REQUIRE(!pre->x2 || pre->ldx2 >= n, "pre-operation: ldx2 %lld < n", (long long)pre->ldx2);
  QS_REQUIRE(!pre->h_out || pre->ldo >= n, "pre-operation: ldo %lld < n", (long long)pre->ldo);
  auto a8 = [](const void* p, int64_t ld) { return (reinterpret_cast<uintptr_t>(p) & 7) == 0 && ld % 4 == 0; };
  QS_SUPPORTED(((batch <= 2 && n % 256 == 0 && n / 256 <= 64) ||
                (batch >= 3 && batch <= 16 && chunk_transform_fits(n, kron_pn))) &&
                   a8(x, ldx) && (!pre->x2 || a8(pre->x2, pre->ldx2)) &&
                   (reinterpret_cast<uintptr_t>(pre->weight) & 7) == 0 && (!pre->h_out || a8(pre->h_out, pre->ldo)),
               "pre-operation: 1-2 rows with n a multiple of 256 up to 16384, or 3-16 rows with n on the chunk "
               "scheme (up to 12288), 8-byte aligned rows (got batch %lld, n %lld)",
               (long long)batch, (long long)n);
  if (pre->h_out) {
    const size_t out_bytes = (size_t)((batch - 1) * pre->ldo + n) * 2;
    QS_REQUIRE(!overlaps(pre->h_out, out_bytes, x, (size_t)((batch - 1) * ldx + n) * 2) &&
                   (!pre->x2 || !overlaps(pre->h_out, out_bytes, pre->x2, (size_t)((batch - 1) * pre->ldx2 + n) * 2)),
               "pre-operation: h_out overlaps x or x2 (every work-group reads them while one writes h_out)");
  }
  FusedPre fp{pre->kind, pre->x2, pre->ldx2, pre->weight, pre->h_out, pre->ldo, pre->eps};
  return forward_group_impl(x, QS_DTYPE_BF16, ldx, batch, n, kron_pn, kron_n, count, jobs, y_dtype, workspace,
                            workspace_bytes, nullptr, nullptr, stream, &fp);
}

extern "C" int qs_decode_matvec(const void* x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int64_t m,
                                const void* codes0, const void* codes1, int kind1, int layout, float s0, float s1,
                                float layer_scale, void* y, int y_dtype, int64_t ldy, void* workspace,
                                size_t workspace_bytes, qs_stream_t stream) {
  QS_REQUIRE(batch >= 0 && n > 0 && m > 0 && n % 8 == 0, "bad shape batch=%lld n=%lld m=%lld", (long long)batch,
             (long long)n, (long long)m);
  QS_REQUIRE(x_dtype >= QS_DTYPE_F32 && x_dtype <= QS_DTYPE_BF16 && y_dtype >= QS_DTYPE_F32 &&
                 y_dtype <= QS_DTYPE_BF16,
             "bad dtype");
  QS_REQUIRE(layout == QS_LAYOUT_TILED || layout == QS_LAYOUT_ROWMAJOR, "bad layout");
  if (batch == 0) return QS_OK;
  QS_REQUIRE(x && y && codes0 && workspace, "null pointer");
  QS_REQUIRE(ldx >= n && ldy >= m, "row strides too small");
  QS_REQUIRE(n <= kMaxLen && m <= kMaxLen, "dims exceed %d", kMaxLen);
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
  return forward_batched(x, x_dtype, ldx, batch, n, m, codes0, codes1, kind1, layout, nullptr, nullptr, 1, nullptr, 1,
                         nullptr, s0, s1, layer_scale, nullptr, y, y_dtype, ldy, static_cast<char*>(workspace),
                         workspace_bytes, W, nullptr, nullptr, as_stream(stream), true);
}
