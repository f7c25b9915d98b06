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
//   1. issue the activation loads, then the abs-table and K loads; the first
//      code tiles are requested once the activations have arrived, and the
//      signed half-codeword LDS tables are built after the input transform
//      (off its critical path);
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
#include "qs_linear_dev.h"

namespace qs {
namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

__constant__ Table8 kE8P = make_e8p_table();
__constant__ Table8 kE81 = make_e81_table();

constexpr int kThreads = 1024;
constexpr int kMaxB = 2;
constexpr int kPrefetch = 4;
constexpr int kMaxJobs = QS_MAX_GROUP;
constexpr int kXStride = 264;               // halves per slice row of the fp16 operand buffer

// One linear of a launch.  Linears in one launch share the input x (and n);
// each has its own codes, signs, scales, output and workspace region.
struct FusedJob {
  const float* sv;
  const uint16_t* codes0;
  const uint8_t* codes1;
  int m, Gr, wg0;      // rows; row-block stride; first work-group of this linear
  float s0, s1;
  float* y1p;          // [SG][B][m]
  unsigned* counter;   // zero between launches
  float* xmul;         // [B] 2^e per batch row (for a separate output kernel)
  int out_in_kernel;
  int Sm, lsh_m;
  float scale_m, layer_scale;
  const float* su;
  const float* bias;
  void* y;
  int64_t ldy;
};

struct FusedArgs {
  const void* x;
  int x_dtype;
  int x_vec;  // rows of 4 elements can be loaded as one 8- or 16-byte word
  int64_t ldx;
  int B;
  int n, Sn, lsh_n, pn;
  const float* Kn;
  float scale_n;
  int S, SG, W;
  int y_dtype;
  int njobs;
  FusedJob job[kMaxJobs];
};

// LDS layout (bytes).  The abs-table staging area aliases the reduction
// buffer (the table is dead before the first row block); the output
// transform of the last work-group reuses the Y region.
constexpr int kOffHi = 0;                                   // 4096 x uint2
constexpr int kOffLo = 32768;                               // 4096 x uint2
constexpr int kOffLut1 = 65536;                             // 256 x uint4
constexpr int kOffRed = kOffLut1 + 4096;                    // 2 x 16 x 16 x kMaxB floats
constexpr int kOffK = kOffRed + 2 * kWaves * 16 * kMaxB * 4;  // p x p floats (p <= 64)
constexpr int kOffTab = kOffRed;                            // 256 x uint4 (table staging, before the row blocks)
constexpr int kOffXH = kOffK + QS_MAX_KRON * QS_MAX_KRON * 4;  // kMaxB x 16 x kXStride halves
constexpr int kOffXS = kOffXH + kMaxB * 16 * kXStride * 2;  // kMaxB x 16 x 32 halves (group sums)
constexpr int kOffY = kOffXS + kMaxB * 16 * 32 * 2;          // kMaxS x kYStride floats
constexpr int kLdsBytes = kOffY + kMaxS * kYStride * 4;
static_assert(kLdsBytes <= 160 * 1024 - 128, "LDS budget");
static_assert(2 * kWaves * 16 * kMaxB * 4 >= 4096, "table staging fits the reduction buffer");

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
  _Float16 a = (_Float16)lo, b = (_Float16)hi;
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Activation chunks of batch row b (times sv), chunk c = w + 16 u.
__device__ __forceinline__ void load_x(const FusedArgs& A, const float* sv, int b, int w, int lane,
                                       float (&v)[kCPW][4]) {
#pragma unroll
  for (int u = 0; u < kCPW; ++u) {
    const int c = w + kWaves * u;
#pragma unroll
    for (int j = 0; j < 4; ++j) v[u][j] = 0.0f;
    if (c < A.Sn) {
      const int i0 = 256 * c + 4 * lane;
      const float4 s = *reinterpret_cast<const float4*>(sv + i0);
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
  _Float16* XS = reinterpret_cast<_Float16*>(lds + kOffXS);
  float* Y = reinterpret_cast<float*>(lds + kOffY);
  __shared__ float wsum[kWaves];
  __shared__ int s_last;

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  int g = 0;
#pragma unroll
  for (int k = 1; k < kMaxJobs; ++k)
    if (k < A.njobs && (int)blockIdx.x >= A.job[k].wg0) g = k;
  const FusedJob& J = A.job[g];
  const int lb = (int)blockIdx.x - J.wg0;  // work-group index within this linear
  const int RB = J.m >> 4;
  const int sg = lb / J.Gr, jr = lb - sg * J.Gr;
  const int sl = sg * A.W + w;
  const bool active = w < A.W && sl < A.S;
  const LaneX lx = lane_x_init();

  // 1. loads: the activations first (the transform waits for them), then the
  //    abs table and K; the code tiles once the activations are in
  float xv[kCPW][4];
  load_x(A, J.sv, 0, w, lane, xv);
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
  uint4 pre[kPrefetch];
  uint2 pre1[kPrefetch];

  // 2. input transform, one batch row at a time, into fp16 operand rows
  float emul0 = 1.0f, emul1 = 1.0f;  // 2^e of batch rows 0 and 1
  for (int b = 0; b < A.B; ++b) {
    if (b > 0) load_x(A, J.sv, b, w, lane, xv);
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
        const int rb = jr + k * J.Gr;
        pre[k] = make_uint4(0, 0, 0, 0);
        pre1[k] = make_uint2(0, 0);
        if (active && rb < RB) {
          const size_t tile = ((size_t)rb * A.S + sl) * 64 + lane;
          pre[k] = *reinterpret_cast<const uint4*>(J.codes0 + tile * 8);
          if (HAS2) pre1[k] = *reinterpret_cast<const uint2*>(J.codes1 + tile * 8);
        }
      }
      // table staging and K (read after the barrier below)
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
    }
    if (b > 0) __syncthreads();  // the previous row's reads of Y are done
    store_chunks(Y, A.Sn, w, lane, xv);
    __syncthreads();  // chunks, norms (and, the first time, the staged table and K) complete
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
    // this wave's slice row of M . Y: X2[sl][4 lane + j] = sum_c M[sl][c] Y[c][4 lane + j]
    // (M[sl][c] is the same for the whole wave), as fp16 into the wave's own
    // operand row
    if (active) {
      const float4 a = mrow_times_chunks(Y, A.Sn, sl, A.lsh_n, A.pn, Ks, lane);
      const _Float16 h0 = (_Float16)(a.x * mul), h1 = (_Float16)(a.y * mul);
      const _Float16 h2 = (_Float16)(a.z * mul), h3 = (_Float16)(a.w * mul);
      const uint2 hv = make_uint2((uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16),
                                  (uint32_t)__builtin_bit_cast(uint16_t, h2) | ((uint32_t)__builtin_bit_cast(uint16_t, h3) << 16));
      *reinterpret_cast<uint2*>(XH + (b * 16 + w) * kXStride + 4 * lane) = hv;
      // group sums of the fp16 values: group t / 8 spans lanes 2g and 2g + 1
      const float s4 = ((float)h0 + (float)h1) + ((float)h2 + (float)h3);
      const float s8 = s4 + lane_xor<1>(s4, lx);
      if ((lane & 1) == 0) XS[(b * 16 + w) * 32 + (lane >> 1)] = (_Float16)s8;
    }
  }
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
  __syncthreads();  // LUTs and operand rows complete; the table staging area is free again
  // MFMA operand of lane (q, b = r16): columns 64q..64q+63 of this wave's slice
  const half8 hzero = {0, 0, 0, 0, 0, 0, 0, 0};
  half8 xb[8];
  half8 xs = hzero;
  float slice_shift = 0.0f;  // sum_g S_g over the lane's 64 columns, batch row r16
#pragma unroll
  for (int c = 0; c < 8; ++c) xb[c] = hzero;
  if (active && r16 < A.B) {
    const _Float16* row = XH + (r16 * 16 + w) * kXStride + 64 * q;
#pragma unroll
    for (int c = 0; c < 8; ++c) xb[c] = *reinterpret_cast<const half8*>(row + 8 * c);
    xs = *reinterpret_cast<const half8*>(XS + (r16 * 16 + w) * 32 + 8 * q);
#pragma unroll
    for (int c = 0; c < 8; ++c) slice_shift += (float)xs[c];
  }
  // slice total of S_g over the four q-lanes of batch row r16
  slice_shift += __shfl_xor(slice_shift, 16);
  slice_shift += __shfl_xor(slice_shift, 32);
  if (lb == 0 && tid < A.B) J.xmul[tid] = tid == 0 ? emul0 : emul1;

  // 3. row blocks
  const int nw = A.S - sg * A.W < A.W ? A.S - sg * A.W : A.W;
  int k = 0;  // iteration count: selects the reduction buffer
  for (int rb = jr; rb < RB; rb += J.Gr, ++k) {
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
      const int rbn = rb + kPrefetch * J.Gr;
      pre[kPrefetch - 1] = make_uint4(0, 0, 0, 0);
      pre1[kPrefetch - 1] = make_uint2(0, 0);
      if (active && rbn < RB) {
        const size_t tile = ((size_t)rbn * A.S + sl) * 64 + lane;
        pre[kPrefetch - 1] = *reinterpret_cast<const uint4*>(J.codes0 + tile * 8);
        if (HAS2) pre1[kPrefetch - 1] = *reinterpret_cast<const uint2*>(J.codes1 + tile * 8);
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
        float v = J.s0 * (acc[j] + 0.5f * accs[j] - 0.25f * slice_shift);
        if (HAS2) v = v + J.s1 * acc2[j];
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
        __hip_atomic_store(&J.y1p[((size_t)sg * A.B + bc) * J.m + rb * 16 + row], v, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  }

  // 4. completion: the last work-group applies the output transform
  if (!J.out_in_kernel) return;
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial-sum stores have completed
  __syncthreads();
  if (tid == 0)
    s_last = __hip_atomic_fetch_add(J.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
             (unsigned)(J.Gr * A.SG - 1);
  __syncthreads();
  if (!s_last) return;
  {
    // this lane's outputs: rows r = w + 16u (chunks of 256), columns 4 lane + j
    float suv[kCPW][4], biv[kCPW][4];
#pragma unroll
    for (int u = 0; u < kCPW; ++u) {
      const int r = w + kWaves * u;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 256 * r + 4 * lane + j;
        const bool ok = r < J.Sm;
        suv[u][j] = ok ? J.su[i] : 0.0f;
        biv[u][j] = (ok && J.bias) ? J.bias[i] : 0.0f;
      }
    }
    for (int b = 0; b < A.B; ++b) {
      float zv[kCPW][4];
#pragma unroll
      for (int u = 0; u < kCPW; ++u) {
        const int c = w + kWaves * u;
#pragma unroll
        for (int j = 0; j < 4; ++j) zv[u][j] = 0.0f;
        if (c < J.Sm) {
          for (int g = 0; g < A.SG; ++g) {
            const float* src = J.y1p + ((size_t)g * A.B + b) * J.m + 256 * c + 4 * lane;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              zv[u][j] += __hip_atomic_load(src + j, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
      }
      h256_chunks(zv, J.Sm, lane, lx);
      if (b > 0) __syncthreads();  // the previous row's reads of Y are done
      store_chunks(Y, J.Sm, w, lane, zv);
      __syncthreads();  // chunks complete
      const float mul = J.scale_m * J.layer_scale * (b == 0 ? emul0 : emul1);
#pragma unroll
      for (int u = 0; u < kCPW; ++u) {
        const int r = w + kWaves * u;
        if (r < J.Sm) {
          const float4 av = mrow_times_chunks(Y, J.Sm, r, J.lsh_m, 1, nullptr, lane);
          const float a[4] = {av.x, av.y, av.z, av.w};
#pragma unroll
          for (int j = 0; j < 4; ++j)
            store_from_float(J.y, A.y_dtype, (int64_t)b * J.ldy + 256 * r + 4 * lane + j,
                             a[j] * mul * suv[u][j] + biv[u][j]);
        }
      }
    }
  }
  if (tid == 0) __hip_atomic_store(J.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// Host launcher used by qs_linear_forward and qs_linear_forward_group
// (qs_linear.hip).  The CUs are shared between the linears in proportion to
// their rows; each linear's work-groups form a contiguous block of the grid.
int launch_linear_fused(const void* x, int x_dtype, int64_t ldx, int B, int n, int pn, const float* Kn, int y_dtype,
                        int count, const FusedJobDesc* jobs, int S, int SG, int W, int ncu, hipStream_t stream,
                        hipEvent_t ev_start, hipEvent_t ev_stop) {
  QS_REQUIRE(count >= 1 && count <= kMaxJobs, "1..%d linears per launch", kMaxJobs);
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
  A.S = S;
  A.SG = SG;
  A.W = W;
  A.y_dtype = y_dtype;
  A.njobs = count;
  int64_t mtot = 0;
  for (int g = 0; g < count; ++g) mtot += jobs[g].m;
  const bool has2 = jobs[0].codes1 != nullptr;
  int wg = 0;
  for (int g = 0; g < count; ++g) {
    const FusedJobDesc& d = jobs[g];
    QS_REQUIRE((d.codes1 != nullptr) == has2, "all linears of a launch need the same number of stages");
    FusedJob& J = A.job[g];
    J.sv = d.sv;
    J.codes0 = static_cast<const uint16_t*>(d.codes0);
    J.codes1 = static_cast<const uint8_t*>(d.codes1);
    J.m = (int)d.m;
    const int RB = (int)(d.m / 16);
    int Gr = (int)((double)ncu / SG * (double)d.m / (double)mtot);
    if (Gr < 1) Gr = 1;
    if (Gr > RB) Gr = RB;
    J.Gr = Gr;
    J.wg0 = wg;
    wg += Gr * SG;
    J.s0 = d.s0;
    J.s1 = d.s1;
    J.y1p = d.y1p;
    J.counter = d.counter;
    J.xmul = d.xmul;
    J.out_in_kernel = d.pm == 1 && chunk_transform_fits(d.m, d.pm);
    if (J.out_in_kernel) {
      J.Sm = (int)(d.m / 256);
      J.lsh_m = log2_exact(d.m / 256);
    }
    J.scale_m = inv_sqrt_len(d.m / d.pm);
    J.layer_scale = d.layer_scale;
    J.su = d.su;
    J.bias = d.bias;
    J.y = d.y;
    J.ldy = d.ldy;
  }
  static int attr_done = 0;
  if (!attr_done) {
    QS_HIP(hipFuncSetAttribute((const void*)linear_fused_kernel<false>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes));
    QS_HIP(hipFuncSetAttribute((const void*)linear_fused_kernel<true>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes));
    attr_done = 1;
  }
  if (has2)
    hipExtLaunchKernelGGL(linear_fused_kernel<true>, dim3((unsigned)wg), dim3(kThreads), kLdsBytes, stream, ev_start,
                          ev_stop, 0, A);
  else
    hipExtLaunchKernelGGL(linear_fused_kernel<false>, dim3((unsigned)wg), dim3(kThreads), kLdsBytes, stream,
                          ev_start, ev_stop, 0, A);
  QS_LAUNCHED("linear_fused_kernel");
  return QS_OK;
}

bool fused_output_in_kernel(int64_t m, int pm) { return pm == 1 && chunk_transform_fits(m, pm); }

bool fused_eligible(int64_t batch, int64_t n, int64_t m, int pn) {
  (void)m;
  return batch >= 1 && batch <= kMaxB && chunk_transform_fits(n, pn);
}

}  // namespace qs
