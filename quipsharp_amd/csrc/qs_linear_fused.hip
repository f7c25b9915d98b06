// One-launch quantized-linear forward for decode-size batches (B <= 2,
// n <= 12288), the path QuantizedLinear.forward takes at generation time
// (quipsharp/checkpoint.py:141-146 -> quipsharp/quantize.py:116-124).
//
// Transforms.  A length-n transform T_n = K_p (x) H_L (n = p L, L = 2^k >= 256)
// is split as T_n = M (x) H_256 over the index i = 256 c + t: a 256-point
// Walsh-Hadamard inside each chunk c (one wave, four values per lane, two
// stages in registers and six across lanes with DPP / swizzle exchanges, no
// barrier), then the S x S matrix M = K_p (x) H_{L/256} (S = n / 256 <= 48)
// across chunks, as fp32 16x16x4 MFMAs over 16-column tiles.  Entries of M are
// generated on the fly (Hadamard signs from a popcount, K from LDS).
//
// Work-group j owns one slice group (up to 16 slices of 256 input columns,
// one per wave) and a strided set of 16-row blocks, so each wave's activation
// operand stays in registers for the whole launch.  Per work-group:
//   1. issue the table and activation loads, build the signed half-codeword
//      LDS tables; the first code tiles are requested once the activations
//      have arrived;
//   2. input transform (every work-group; only its own slices' rows of M):
//      chunks -> LDS, MFMA over M rows of this group, fp16 operand per wave
//      scaled by 2^-e (e from the row norm) plus the per-group sums for the
//      +-1/4 shift term, whose -1/4 sum_g S_g part is folded in per slice;
//   3. per row block: 8 MFMAs (+1 for the shift, +8 for an E8 1-bit second
//      stage), a cross-wave tree reduction in LDS (double-buffered, one
//      barrier), partial sums to the workspace as write-through stores;
//   4. completion: the stores are waited for, then one atomic per work-group
//      on a counter; the last work-group reads the partials (write-through
//      loads), applies S_u T_m(.) + bias with the same chunk/MFMA scheme and
//      resets the counter.  This is done for pure Walsh-Hadamard outputs
//      (m a power of two, 256 <= m <= 8192); outputs with an odd factor run
//      the chunk output kernel instead, one work-group per output chunk
//      (qs_linear.hip), which spreads the K_p stage over many CUs.
//
// Cross-work-group visibility.  Partial sums are written with agent-scope
// relaxed atomic stores and read with agent-scope relaxed atomic loads, which
// on gfx950 are write-through / read-through at the device coherence point
// (no per-XCD L2 copy is involved), and every work-group waits for its own
// stores to complete (s_waitcnt) before its counter increment.  This avoids
// an L2 write-back per wave that a device-scope fence would cost.
#include <hip/hip_ext.h>

#include "qs_chunk_dev.h"

namespace qs {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__constant__ Table8 kE8P = make_e8p_table();
__constant__ Table8 kE81 = make_e81_table();

constexpr int kThreads = 1024;
constexpr int kMaxB = 2;
constexpr int kPrefetch = 4;
constexpr int kXStride = 264;               // halves per slice row of the fp16 operand buffer

struct FusedArgs {
  const void* x;
  int x_dtype;
  int x_vec;  // rows of 4 elements can be loaded as one 8- or 16-byte word
  int64_t ldx;
  int B;
  int n, Sn, lsh_n, pn;
  const float* Kn;
  float scale_n;
  const float* sv;
  const uint16_t* codes0;
  const uint8_t* codes1;
  int m, S, SG, W, Gr;
  float s0, s1;
  float* y1p;          // [SG][B][m]
  unsigned* counter;   // zero between launches
  float* xmul;         // [B] 2^e per batch row (for a separate output kernel)
  int out_in_kernel;
  int Sm, lsh_m, pm;
  const float* Km;
  float scale_m, layer_scale;
  const float* su;
  const float* bias;
  void* y;
  int y_dtype;
  int64_t ldy;
};

// LDS layout (bytes).  The half-codeword table staging area aliases the
// operand buffer (it is dead before the first operand write); the output
// transform of the last work-group reuses the K and Y regions.
constexpr int kOffHi = 0;                                   // 4096 x uint2
constexpr int kOffLo = 32768;                               // 4096 x uint2
constexpr int kOffLut1 = 65536;                             // 256 x uint4
constexpr int kOffRed = kOffLut1 + 4096;                    // 2 x 16 x 16 x kMaxB floats
constexpr int kOffK = kOffRed + 2 * kWaves * 16 * kMaxB * 4;  // p x p floats (p <= 64)
constexpr int kOffXH = kOffK + QS_MAX_KRON * QS_MAX_KRON * 4;  // kMaxB x 16 x kXStride halves
constexpr int kOffTab = kOffXH;                             // 256 x uint4 (table staging)
constexpr int kOffY = kOffXH + kMaxB * 16 * kXStride * 2;   // kMaxS x kYStride floats
constexpr int kLdsBytes = kOffY + kMaxS * kYStride * 4;
static_assert(kLdsBytes <= 160 * 1024 - 128, "LDS budget");
static_assert(kMaxB * 16 * kXStride * 2 >= 4096, "table staging fits the operand buffer");

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Activation chunks of batch row b (times sv), chunk c = w + 16 u.
__device__ __forceinline__ void load_x(const FusedArgs& A, int b, int w, int lane, float (&v)[kCPW][4]) {
#pragma unroll
  for (int u = 0; u < kCPW; ++u) {
    const int c = w + kWaves * u;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[u][j] = 0.0f;
    if (c < A.Sn) {
      const int i0 = 256 * c + 4 * lane;
      const float4 s = *reinterpret_cast<const float4*>(A.sv + i0);
      const int64_t xi = (int64_t)b * A.ldx + i0;
      float x0, x1, x2, x3;
      if (A.x_vec && A.x_dtype == QS_DTYPE_F32) {
        const float4 t = *reinterpret_cast<const float4*>(static_cast<const float*>(A.x) + xi);
        x0 = t.x, x1 = t.y, x2 = t.z, x3 = t.w;
      } else if (A.x_vec) {
        const uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(A.x) + xi);
        if (A.x_dtype == QS_DTYPE_BF16) {
          x0 = __uint_as_float(t.x << 16), x1 = __uint_as_float(t.x & 0xFFFF0000u);
          x2 = __uint_as_float(t.y << 16), x3 = __uint_as_float(t.y & 0xFFFF0000u);
        } else {
          x0 = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.x & 0xFFFFu));
          x1 = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.x >> 16));
          x2 = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.y & 0xFFFFu));
          x3 = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.y >> 16));
        }
      } else {
        x0 = load_as_float(A.x, A.x_dtype, xi);
        x1 = load_as_float(A.x, A.x_dtype, xi + 1);
        x2 = load_as_float(A.x, A.x_dtype, xi + 2);
        x3 = load_as_float(A.x, A.x_dtype, xi + 3);
      }
      v[u][0] = x0 * s.x;
      v[u][1] = x1 * s.y;
      v[u][2] = x2 * s.z;
      v[u][3] = x3 * s.w;
    }
  }
}

__device__ __forceinline__ void store_chunks(float* Y, int S, int w, int lane, const float (&v)[kCPW][4]) {
#pragma unroll
  for (int u = 0; u < kCPW; ++u) {
    const int c = w + kWaves * u;
    if (c < S)
      *reinterpret_cast<float4*>(Y + c * kYStride + 4 * lane) = make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
  }
}

template <bool HAS2>
__global__ __launch_bounds__(kThreads) void linear_fused_kernel(FusedArgs A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint2* lut_hi = reinterpret_cast<uint2*>(lds + kOffHi);
  uint2* lut_lo = reinterpret_cast<uint2*>(lds + kOffLo);
  uint4* lut1 = reinterpret_cast<uint4*>(lds + kOffLut1);
  uint4* tab16 = reinterpret_cast<uint4*>(lds + kOffTab);
  float* red = reinterpret_cast<float*>(lds + kOffRed);
  float* Ks = reinterpret_cast<float*>(lds + kOffK);
  _Float16* XH = reinterpret_cast<_Float16*>(lds + kOffXH);
  float* Y = reinterpret_cast<float*>(lds + kOffY);
  __shared__ float wsum[kWaves];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  const int RB = A.m >> 4;
  const int sg = blockIdx.x / A.Gr, jr = blockIdx.x - sg * A.Gr;
  const int sl = sg * A.W + w;
  const bool active = w < A.W && sl < A.S;
  const LaneX lx = lane_x_init();

  // 1. loads, in the order they are needed: tables, K, activations, codes
  float trow[8], t1row[8];
  if (tid < 256) {
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      trow[k] = kE8P.v[tid][k];
      if (HAS2) t1row[k] = kE81.v[tid][k];
    }
  }
  float kv[4];
  const int pp = A.pn * A.pn;
#pragma unroll
  for (int k = 0; k < 4; ++k) kv[k] = (A.pn > 1 && tid + kThreads * k < pp) ? A.Kn[tid + kThreads * k] : 0.0f;
  float xv[kCPW][4];
  load_x(A, 0, w, lane, xv);
  uint4 pre[kPrefetch];
  uint2 pre1[kPrefetch];
  if (tid < 256) {
    tab16[tid] = make_uint4(pack_h2(trow[0], trow[1]), pack_h2(trow[2], trow[3]), pack_h2(trow[4], trow[5]),
                            pack_h2(trow[6], trow[7]));
    if (HAS2)
      lut1[tid] = make_uint4(pack_h2(t1row[0], t1row[1]), pack_h2(t1row[2], t1row[3]),
                             pack_h2(t1row[4], t1row[5]), pack_h2(t1row[6], t1row[7]));
  }
#pragma unroll
  for (int k = 0; k < 4; ++k)
    if (A.pn > 1 && tid + kThreads * k < pp) Ks[tid + kThreads * k] = kv[k];
  __syncthreads();
  {
    // LUT entries e = tid + 1024 k.  hi: abs row e & 255 = tid & 255 and flip
    // nibble H = e >> 8 = (tid >> 8) + 4 k.  lo: abs row (e >> 3) & 255 (two
    // rows, k even / odd), f4..f6 from e & 7 = tid & 7, q = e >> 11 = k >> 1.
    const uint4 th = tab16[tid & 255];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t H = (uint32_t)(tid >> 8) + 4u * k;
      const uint32_t f1 = (H >> 3) & 1, f2 = (H >> 2) & 1, f3 = (H >> 1) & 1;
      const uint32_t f0 = (H & 1) ^ f1 ^ f2 ^ f3;
      lut_hi[tid + kThreads * k] = make_uint2(th.x ^ ((f0 << 15) | (f1 << 31)), th.y ^ ((f2 << 15) | (f3 << 31)));
    }
    const uint32_t f4 = (tid >> 2) & 1, f5 = (tid >> 1) & 1, f6 = tid & 1;
    const uint32_t m45 = (f4 << 15) | (f5 << 31), p456 = f4 ^ f5 ^ f6;
    const uint4 ta = tab16[(tid >> 3) & 255], tb = tab16[((tid >> 3) + 128) & 255];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint4 t = (k & 1) ? tb : ta;
      const uint32_t f7 = (uint32_t)(k >> 1) ^ p456;
      lut_lo[tid + kThreads * k] = make_uint2(t.z ^ m45, t.w ^ ((f6 << 15) | (f7 << 31)));
    }
  }

  // 2. input transform, one batch row at a time, into fp16 operand rows
  float emul0 = 1.0f, emul1 = 1.0f;  // 2^e of batch rows 0 and 1
  const int kt_n = (A.Sn + 3) >> 2;
  for (int b = 0; b < A.B; ++b) {
    if (b > 0) load_x(A, b, w, lane, xv);
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kCPW; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) ss = __builtin_fmaf(xv[u][j], xv[u][j], ss);
    for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o);
    if (lane == 0) wsum[w] = ss;
    h256_chunks(xv, A.Sn, lane, lx);
    if (b == 0) {
      // first code tiles (issued once the activations are in, so the
      // activation loads do not queue behind them)
#pragma unroll
      for (int k = 0; k < kPrefetch; ++k) {
        const int rb = jr + k * A.Gr;
        pre[k] = make_uint4(0, 0, 0, 0);
        pre1[k] = make_uint2(0, 0);
        if (active && rb < RB) {
          const size_t tile = ((size_t)rb * A.S + sl) * 64 + lane;
          pre[k] = *reinterpret_cast<const uint4*>(A.codes0 + tile * 8);
          if (HAS2) pre1[k] = *reinterpret_cast<const uint2*>(A.codes1 + tile * 8);
        }
      }
    }
    if (b > 0) __syncthreads();  // the previous row's MFMAs have read Y
    store_chunks(Y, A.Sn, w, lane, xv);
    __syncthreads();  // chunks, norms (and, the first time, the LUTs) complete
    float norm2 = 0.0f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) norm2 += wsum[i];
    int e = 0;
    if (norm2 > 0.0f && norm2 < INFINITY) {
      int ex;
      frexpf(sqrtf(norm2) * 1.0001f, &ex);  // |x2_i| <= ||x|| < 2^ex
      e = ex - 14;
    }
    if (b == 0) emul0 = ldexpf(1.0f, e);
    else emul1 = ldexpf(1.0f, e);
    const float mul = ldexpf(A.scale_n, -e);
    // rows of M for this group's slices, columns 16w..16w+15
    const int r = sg * A.W + r16;
    const bool rv = r16 < A.W && r < A.Sn;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int t = 0; t < kt_n; ++t) {
      const int c = 4 * t + q;
      const float av = (rv && c < A.Sn) ? mmat(r, c, A.lsh_n, A.pn, Ks) : 0.0f;
      const float bv = c < A.Sn ? Y[c * kYStride + 16 * w + r16] : 0.0f;
      acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) XH[(b * 16 + 4 * q + j) * kXStride + 16 * w + r16] = (_Float16)(acc[j] * mul);
  }
  __syncthreads();  // operand rows complete
  // MFMA operand of lane (q, b = r16): columns 64q..64q+63 of this wave's slice
  const half8 hzero = {0, 0, 0, 0, 0, 0, 0, 0};
  half8 xb[8];
  half8 xs = hzero;
  float slice_shift = 0.0f;  // sum_g S_g over the lane's 64 columns, batch row r16
#pragma unroll
  for (int c = 0; c < 8; ++c) xb[c] = hzero;
  if (active && r16 < A.B) {
    _Float16 sh[8];
    const _Float16* row = XH + (r16 * 16 + w) * kXStride + 64 * q;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const half8 hv = *reinterpret_cast<const half8*>(row + 8 * c);
      xb[c] = hv;
      const float g01 = (float)hv[0] + (float)hv[1], g23 = (float)hv[2] + (float)hv[3];
      const float g45 = (float)hv[4] + (float)hv[5], g67 = (float)hv[6] + (float)hv[7];
      sh[c] = (_Float16)((g01 + g23) + (g45 + g67));
      slice_shift += (float)sh[c];
    }
    xs = __builtin_bit_cast(half8, sh);
  }
  // slice total of S_g over the four q-lanes of batch row r16
  slice_shift += __shfl_xor(slice_shift, 16);
  slice_shift += __shfl_xor(slice_shift, 32);
  if (blockIdx.x == 0 && tid < A.B) A.xmul[tid] = tid == 0 ? emul0 : emul1;

  // 3. row blocks
  const int nw = A.S - sg * A.W < A.W ? A.S - sg * A.W : A.W;
  int k = 0;  // iteration count: selects the reduction buffer
  for (int rb = jr; rb < RB; rb += A.Gr, ++k) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    floatx4 accs = {0.f, 0.f, 0.f, 0.f};
    floatx4 acc2 = {0.f, 0.f, 0.f, 0.f};
    uint4 cw = pre[0];
    uint2 cw1 = pre1[0];
#pragma unroll
    for (int j = 0; j + 1 < kPrefetch; ++j) {
      pre[j] = pre[j + 1];
      pre1[j] = pre1[j + 1];
    }
    {
      // keep kPrefetch tiles in flight
      const int rbn = rb + kPrefetch * A.Gr;
      pre[kPrefetch - 1] = make_uint4(0, 0, 0, 0);
      pre1[kPrefetch - 1] = make_uint2(0, 0);
      if (active && rbn < RB) {
        const size_t tile = ((size_t)rbn * A.S + sl) * 64 + lane;
        pre[kPrefetch - 1] = *reinterpret_cast<const uint4*>(A.codes0 + tile * 8);
        if (HAS2) pre1[kPrefetch - 1] = *reinterpret_cast<const uint2*>(A.codes1 + tile * 8);
      }
    }
    if (active) {
      const uint32_t wd[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const uint32_t wv = wd[c >> 1];
        const uint32_t ha = (c & 1) ? ((wv >> 17) & 0x7FF8u) : ((wv >> 1) & 0x7FF8u);
        const uint32_t la = (c & 1) ? ((wv >> 14) & 0x7FF8u) : ((wv << 2) & 0x7FF8u);
        const uint2 hv = *reinterpret_cast<const uint2*>(lds + kOffHi + ha);
        const uint2 lv = *reinterpret_cast<const uint2*>(lds + kOffLo + la);
        const half8 av = __builtin_bit_cast(half8, make_uint4(hv.x, hv.y, lv.x, lv.y));
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, xb[c], acc, 0, 0, 0);
        if (HAS2) {
          const uint32_t idx = ((c < 4 ? cw1.x : cw1.y) >> (8 * (c & 3))) & 0xFFu;
          acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, lut1[idx]), xb[c], acc2, 0, 0,
                                                          0);
        }
      }
      const half8 ash = __builtin_bit_cast(
          half8, make_uint4((wd[0] & 0x10001u) * 0x3C00u, (wd[1] & 0x10001u) * 0x3C00u,
                            (wd[2] & 0x10001u) * 0x3C00u, (wd[3] & 0x10001u) * 0x3C00u));
      accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(ash, xs, accs, 0, 0, 0);
    }
    // partial of this slice for rows 4q..4q+3, batch column r16
    float* rbuf = red + (k & 1) * (kWaves * 16 * kMaxB);
    if (r16 < A.B) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = A.s0 * (acc[j] + 0.5f * accs[j] - 0.25f * slice_shift);
        if (HAS2) v = v + A.s1 * acc2[j];
        rbuf[(w * 16 + 4 * q + j) * kMaxB + r16] = active ? v : 0.0f;
      }
    }
    __syncthreads();
    // tree sum over the waves: thread (o, ww), o = row*B + b
    {
      const int o = tid >> 4, ww = tid & 15;
      float v = 0.0f;
      if (o < 16 * A.B && ww < nw) v = rbuf[(ww * 16 + o / A.B) * kMaxB + (o % A.B)];
      v += __shfl_xor(v, 1);
      v += __shfl_xor(v, 2);
      v += __shfl_xor(v, 4);
      v += __shfl_xor(v, 8);
      if (o < 16 * A.B && ww == 0) {
        const int row = o / A.B, bc = o % A.B;
        __hip_atomic_store(&A.y1p[((size_t)sg * A.B + bc) * A.m + rb * 16 + row], v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }

  // 4. completion: the last work-group applies the output transform
  if (!A.out_in_kernel) return;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial-sum stores have completed
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(A.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
  __syncthreads();
  if (!s_last) return;
  {
    float* Km = Ks;  // the input K is dead
    const int ppm = A.pm * A.pm;
    if (A.pm > 1)
      for (int i = tid; i < ppm; i += kThreads) Km[i] = A.Km[i];
    const int kt_m = (A.Sm + 3) >> 2;
    const int rt_m = (A.Sm + 15) >> 4;
    // this lane's outputs: rows 16u + 4q + j of column 16w + r16 (row = chunk of 256)
    float suv[kCPW][4], biv[kCPW][4];
#pragma unroll
    for (int u = 0; u < kCPW; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 16 * u + 4 * q + j;
        const int i = 256 * r + 16 * w + r16;
        const bool ok = r < A.Sm;
        suv[u][j] = ok ? A.su[i] : 0.0f;
        biv[u][j] = (ok && A.bias) ? A.bias[i] : 0.0f;
      }
    for (int b = 0; b < A.B; ++b) {
      float zv[kCPW][4];
#pragma unroll
      for (int u = 0; u < kCPW; ++u) {
        const int c = w + kWaves * u;
#pragma unroll
        for (int j = 0; j < 4; ++j) zv[u][j] = 0.0f;
        if (c < A.Sm) {
          for (int g = 0; g < A.SG; ++g) {
            const float* src = A.y1p + ((size_t)g * A.B + b) * A.m + 256 * c + 4 * lane;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              zv[u][j] += __hip_atomic_load(src + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
      h256_chunks(zv, A.Sm, lane, lx);
      store_chunks(Y, A.Sm, w, lane, zv);
      __syncthreads();  // chunks (and Km) complete
      const float mul = A.scale_m * A.layer_scale * (b == 0 ? emul0 : emul1);
      // wave w: output columns 16w..16w+15 of every row tile
      floatx4 acc[kCPW];
#pragma unroll
      for (int u = 0; u < kCPW; ++u) acc[u] = floatx4{0.f, 0.f, 0.f, 0.f};
      for (int t = 0; t < kt_m; ++t) {
        const int c = 4 * t + q;
        const float bv = c < A.Sm ? Y[c * kYStride + 16 * w + r16] : 0.0f;
#pragma unroll
        for (int u = 0; u < kCPW; ++u) {
          if (u < rt_m) {
            const int r = 16 * u + r16;
            const float av = (r < A.Sm && c < A.Sm) ? mmat(r, c, A.lsh_m, A.pm, Km) : 0.0f;
            acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, bv, acc[u], 0, 0, 0);
          }
        }
      }
#pragma unroll
      for (int u = 0; u < kCPW; ++u) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 16 * u + 4 * q + j;
          if (r < A.Sm)
            store_from_float(A.y, A.y_dtype, (int64_t)b * A.ldy + 256 * r + 16 * w + r16,
                             acc[u][j] * mul * suv[u][j] + biv[u][j]);
        }
      }
      __syncthreads();  // Y is rewritten by the next batch row
    }
  }
  if (tid == 0) __hip_atomic_store(A.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// Host launcher used by qs_linear_forward (qs_linear.hip).
int launch_linear_fused(const void* x, int x_dtype, int64_t ldx, int B, int n, int m, const void* codes0,
                        const void* codes1, const float* sv, const float* su, int pn, const float* Kn, int pm,
                        const float* Km, float s0, float s1, float layer_scale, const float* bias, void* y,
                        int y_dtype, int64_t ldy, unsigned* counter, float* xmul, float* y1p, int S, int SG, int W,
                        int ncu, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop, bool* out_done) {
  FusedArgs A{};
  A.x = x;
  A.x_dtype = x_dtype;
  {
    const uintptr_t align = x_dtype == QS_DTYPE_F32 ? 16 : 8;
    A.x_vec = (reinterpret_cast<uintptr_t>(x) % align) == 0 && ldx % 4 == 0;
  }
  A.ldx = ldx;
  A.B = B;
  A.n = n;
  A.Sn = n / 256;
  A.lsh_n = log2_exact(n / pn / 256);
  A.pn = pn;
  A.Kn = Kn;
  A.scale_n = inv_sqrt_len(n / pn);
  A.sv = sv;
  A.codes0 = static_cast<const uint16_t*>(codes0);
  A.codes1 = static_cast<const uint8_t*>(codes1);
  A.m = m;
  A.S = S;
  A.SG = SG;
  A.W = W;
  const int RB = m / 16;
  int Gr = ncu / SG;
  if (Gr < 1) Gr = 1;
  if (Gr > RB) Gr = RB;
  A.Gr = Gr;
  A.s0 = s0;
  A.s1 = s1;
  A.y1p = y1p;
  A.counter = counter;
  A.xmul = xmul;
  // in-kernel output for pure Walsh-Hadamard outputs; an odd factor runs the
  // chunk output kernel with one work-group per output chunk instead
  A.out_in_kernel = pm == 1 && chunk_transform_fits(m, pm);
  if (A.out_in_kernel) {
    A.Sm = m / 256;
    A.lsh_m = log2_exact(m / pm / 256);
  }
  A.pm = pm;
  A.Km = Km;
  A.scale_m = inv_sqrt_len(m / pm);
  A.layer_scale = layer_scale;
  A.su = su;
  A.bias = bias;
  A.y = y;
  A.y_dtype = y_dtype;
  A.ldy = ldy;
  static int attr_done = 0;
  if (!attr_done) {
    QS_HIP(hipFuncSetAttribute((const void*)linear_fused_kernel<false>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes));
    QS_HIP(hipFuncSetAttribute((const void*)linear_fused_kernel<true>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes));
    attr_done = 1;
  }
  const unsigned grid = (unsigned)(SG * Gr);
  if (codes1)
    hipExtLaunchKernelGGL(linear_fused_kernel<true>, dim3(grid), dim3(kThreads), kLdsBytes, stream, ev_start, ev_stop,
                          0, A);
  else
    hipExtLaunchKernelGGL(linear_fused_kernel<false>, dim3(grid), dim3(kThreads), kLdsBytes, stream, ev_start,
                          ev_stop, 0, A);
  QS_LAUNCHED("linear_fused_kernel");
  *out_done = A.out_in_kernel != 0;
  return QS_OK;
}

bool fused_eligible(int64_t batch, int64_t n, int64_t m, int pn) {
  (void)m;
  return batch >= 1 && batch <= kMaxB && chunk_transform_fits(n, pn);
}

}  // namespace qs
