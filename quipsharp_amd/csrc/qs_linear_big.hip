// Per-row input and output transforms of the multi-row forward (3 or more
// rows: the 16-row passes and the wide GEMM) for lengths beyond the per-row
// chunk kernels' 12288, up to 32768: the Llama-3-8B (14336), Qwen2.5-7B
// (18944) and Qwen3-32B (25600) MLP widths.  Both split T_n = M (x) H_256
// (M = K_p (x) H_{L/256}, S = n / 256 <= 128 chunks) over work-groups of 16
// chunks each, so a row's transform is spread over ceil(S / 16) CUs.
//
//  * bx_big_kernel (input, work-group = (row b, slices 16 k .. 16 k + 15)):
//    the row times sv into a bf16 chunk table XR[t][c] in LDS (exact for bf16
//    activations; fp16 / fp32 add a plane of remainders, n <= 16384), the 16
//    slice rows sum_c M[s][c] x_c on the matrix cores (bf16 hi / lo, fp32
//    accumulate), then per slice (one wave) the 256-point transform and the
//    fragment-major fp16 operand and group sums the decode-matvec reads.
//  * by_big_kernel (output, work-group = (row b, output chunks 16 k .. 16 k +
//    15)): the slice groups' partial sums of every chunk (chunk rows in LDS),
//    its 16 rows of M . z on the matrix cores, then per output chunk (one
//    wave) the 256-point transform, scale, su and bias -- M first, as in the
//    input kernel, so that a work-group transforms its own 16 chunks rather
//    than all S of the row.
// Both replace the LDS-radix row kernels (xin_kernel, yout_kernel) for these
// lengths (Qwen3-32B at 8 rows: 26 and 21 us per launch).
#include "qs_forward_dev.h"
#include "qs_linear_dev.h"

namespace qs {
namespace {

constexpr int kThreads = kFwdThreads;
constexpr int kBigMaxS = 128;                   // chunks (length <= 32768)
constexpr int kMStr = kBigMaxS + 8;             // bf16 per row of 16 M rows (16-byte aligned rows)
constexpr int kZStr = 260;                      // floats per slice row

__device__ __forceinline__ void split_bf(float a, float b, uint32_t& hi, uint32_t& lo) {
  const uint32_t ua = __float_as_uint(a), ub = __float_as_uint(b);
  const uint32_t ha = ua & 0xFFFF0000u, hb = ub & 0xFFFF0000u;
  const uint32_t la = __float_as_uint(a - __uint_as_float(ha)), lb = __float_as_uint(b - __uint_as_float(hb));
  hi = (ha >> 16) | hb;
  lo = (la >> 16) | (lb & 0xFFFF0000u);
}
__device__ __forceinline__ bf16x8 ld_bf16x8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

// Rows rr < 16 of M (row 16 k + rr of K_p (x) H_{2^lsh}; zero past S and
// past Spad columns), bf16 hi / lo with kMStr per row.
__device__ __forceinline__ void build_m_rows(uint16_t* Mh, uint16_t* Ml, int k, int S, int Spad, int lsh, int p,
                                             const float* K, int tid) {
  for (int e = tid; e < 16 * Spad; e += kThreads) {
    const int rr = e / Spad, c = e - rr * Spad;
    const int r = 16 * k + rr;
    float v = 0.0f;
    if (r < S && c < S) v = mmat(r, c, lsh, p, K);
    uint32_t hi, lo;
    split_bf(v, 0.0f, hi, lo);
    Mh[rr * kMStr + c] = (uint16_t)hi;
    Ml[rr * kMStr + c] = (uint16_t)lo;
  }
}

// ---------------------------------------------------------------------------
// input transform
// ---------------------------------------------------------------------------
struct BxBigArgs {
  const void* x;
  int64_t ldx;
  int B, n, S, lsh_n, pn, ngrp;  // rows, length, chunks, log2 (L / 256), odd factor, slice groups of 16
  const float* Kn;
  float scale_n;
  const float* sv;
  _Float16* x2h;  // operand (fragment-major when frag)
  _Float16* sg;   // group sums (fragment-major / 4 when frag)
  float* xmul;    // [B] 2^e
  int frag;
};
// LDS: chunk table (bf16: one plane of 128 chunks; fp16 / fp32: two planes
// of 64), 16 M rows (hi, lo), 16 slice rows, row-norm parts.
constexpr int kBxXR = 0;
constexpr int kBxXRBytes = 256 * (kBigMaxS + 8) * 2;
static_assert(2 * 256 * (kBigMaxS / 2 + 8) * 2 <= kBxXRBytes + 4096, "two planes of 64 chunks");
constexpr int kBxMh = kBxXR + 2 * 256 * (kBigMaxS / 2 + 8) * 2;
constexpr int kBxMl = kBxMh + 16 * kMStr * 2;
constexpr int kBxZ = kBxMl + 16 * kMStr * 2;
constexpr int kBxMisc = kBxZ + 16 * kZStr * 4;
constexpr int kBxLds = kBxMisc + 16 * 4;
static_assert(kBxXRBytes <= kBxMh && kBxLds <= 160 * 1024, "bx_big LDS");

// XT: 0 bf16, 1 fp16, 2 fp32 activations; SB: sv is packed sign bits.
template <int XT, bool SB>
__global__ __launch_bounds__(kThreads) void bx_big_kernel(BxBigArgs A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint16_t* XR0 = reinterpret_cast<uint16_t*>(lds + kBxXR);
  uint16_t* Mh = reinterpret_cast<uint16_t*>(lds + kBxMh);
  uint16_t* Ml = reinterpret_cast<uint16_t*>(lds + kBxMl);
  float* Z = reinterpret_cast<float*>(lds + kBxZ);
  float* wsum = reinterpret_cast<float*>(lds + kBxMisc);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, q = lane >> 4, r16 = lane & 15;
  const LaneX lx = lane_x_init();
  const int b = (int)blockIdx.x / A.ngrp, k = (int)blockIdx.x - b * A.ngrp;
  const int S = A.S, Spad = (S + 31) & ~31, xrs = Spad + 8;
  uint16_t* XR1 = XR0 + 256 * xrs;

  // 1. the row times sv into the chunk table: thread (w, lane) takes chunks
  //    c0 .. c0 + 3 (c0 = 64 round + 4 w) at columns 4 lane .. 4 lane + 3
  float ss = 0.0f;
  for (int c0 = 4 * w; c0 < Spad; c0 += 64) {
    float v[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = c0 + i;
#pragma unroll
      for (int u = 0; u < 4; ++u) v[i][u] = 0.0f;
      if (c < S) {
        const int i0 = 256 * c + 4 * lane;
        const int64_t xi = (int64_t)b * A.ldx + i0;
        float xv[4];
        if constexpr (XT == 2) {
          const float4 t = *reinterpret_cast<const float4*>(static_cast<const float*>(A.x) + xi);
          xv[0] = t.x, xv[1] = t.y, xv[2] = t.z, xv[3] = t.w;
        } else {
          const uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(A.x) + xi);
          if constexpr (XT == 0) {
            xv[0] = __uint_as_float(t.x << 16), xv[1] = __uint_as_float(t.x & 0xFFFF0000u);
            xv[2] = __uint_as_float(t.y << 16), xv[3] = __uint_as_float(t.y & 0xFFFF0000u);
          } else {
            xv[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.x & 0xFFFFu));
            xv[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.x >> 16));
            xv[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.y & 0xFFFFu));
            xv[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(t.y >> 16));
          }
        }
        if constexpr (SB) {
          const uint32_t bits = reinterpret_cast<const uint32_t*>(A.sv)[i0 >> 5] >> (4 * (lane & 7));
#pragma unroll
          for (int u = 0; u < 4; ++u) v[i][u] = flip_by_bit(xv[u], bits, u);
        } else {
          const float4 s4 = *reinterpret_cast<const float4*>(A.sv + i0);
          v[i][0] = xv[0] * s4.x, v[i][1] = xv[1] * s4.y, v[i][2] = xv[2] * s4.z, v[i][3] = xv[3] * s4.w;
        }
      }
    }
#pragma unroll
    for (int pr = 0; pr < 2; ++pr)
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float a = v[2 * pr][u], c = v[2 * pr + 1][u];
        ss = __builtin_fmaf(a, a, ss);
        ss = __builtin_fmaf(c, c, ss);
        uint32_t hi, lo;
        split_bf(a, c, hi, lo);
        const int off = (4 * lane + u) * xrs + c0 + 2 * pr;
        *reinterpret_cast<uint32_t*>(XR0 + off) = hi;
        if constexpr (XT != 0) *reinterpret_cast<uint32_t*>(XR1 + off) = lo;
      }
  }
  ss = wave_sum(ss, lx);
  if (lane == 0) wsum[w] = ss;
  // 2. this work-group's 16 rows of M
  build_m_rows(Mh, Ml, k, S, Spad, A.lsh_n, A.pn, A.Kn, tid);
  __syncthreads();  // chunk table, M rows and norm parts complete
  float norm2 = 0.0f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) norm2 += wsum[i];
  const int e = operand_exponent(norm2);
  const float mul = ldexpf(A.scale_n, -e);
  if (k == 0 && tid == 0) A.xmul[b] = ldexpf(1.0f, e);
  // 3. slice rows z_s = sum_c M[s][c] x_c: wave w takes columns t = 16 w + r16
  {
    const int t = 16 * w + r16;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < (Spad >> 5); ++kb) {
      const int k0 = 32 * kb + 8 * q;
      const bf16x8 xh = ld_bf16x8(XR0 + t * xrs + k0);
      const bf16x8 ah = ld_bf16x8(Mh + r16 * kMStr + k0);
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, xh, acc, 0, 0, 0);
      if (A.pn > 1) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ld_bf16x8(Ml + r16 * kMStr + k0), xh, acc, 0, 0, 0);
      if constexpr (XT != 0)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, ld_bf16x8(XR1 + t * xrs + k0), acc, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) Z[(4 * q + j) * kZStr + t] = acc[j];
  }
  __syncthreads();  // slice rows complete
  // 4. slice s = 16 k + w: 256-point transform, fp16 operand (t = 4 lane + u)
  //    and the sums of its 8-column groups (lane pairs)
  const int s = 16 * k + w;
  if (s < S) {
    const float4 z4 = *reinterpret_cast<const float4*>(Z + w * kZStr + 4 * lane);
    float v[1][4] = {{z4.x, z4.y, z4.z, z4.w}};
    h256<1>(v, lane, lx);
    _Float16 h[4];
    float hs = 0.0f;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      h[u] = (_Float16)(v[0][u] * mul);
      hs += (float)h[u];
    }
    hs += lane_xor<1>(hs, lx);
    const int t0 = 4 * lane;
    const size_t xi = A.frag ? frag_index(b, 256 * s + t0, S) : (size_t)b * A.n + 256 * s + t0;
    *reinterpret_cast<uint2*>(A.x2h + xi) =
        make_uint2((uint32_t)__builtin_bit_cast(uint16_t, h[0]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[1]) << 16),
                   (uint32_t)__builtin_bit_cast(uint16_t, h[2]) | ((uint32_t)__builtin_bit_cast(uint16_t, h[3]) << 16));
    if ((lane & 1) == 0) {
      const int G = 32 * s + (t0 >> 3);
      const size_t si = A.frag ? sg_frag_index(b, G, S) : (size_t)b * (A.n / 8) + G;
      A.sg[si] = A.frag ? (_Float16)hs * (_Float16)0.25f : (_Float16)hs;
    }
  }
}

// ---------------------------------------------------------------------------
// output transform
// ---------------------------------------------------------------------------
struct ByBigJob {
  const float* y1p;    // [SG][B][m] partial sums
  int SG, m, Sm, lsh_m, pm, ngrp, wg0;
  const float* Km;
  float scale_m, layer_scale;
  const float* xmul;   // [B]
  const float* su;
  const float* bias;
  void* y;
  int64_t ldy;
};
struct ByBigArgs {
  int B, y_dtype, njobs;
  ByBigJob job[QS_MAX_GROUP];
};
constexpr int kByCPW = kBigMaxS / kWaves;  // chunks per wave (8)
constexpr int kByY = 0;                     // chunk rows, kYStride floats each
constexpr int kByMh = kByY + kBigMaxS * kYStride * 4;
constexpr int kByMl = kByMh + 16 * kMStr * 2;
constexpr int kByLds = kByMl + 16 * kMStr * 2;
static_assert(kByLds <= 160 * 1024, "by_big LDS");

template <bool SB>
__global__ __launch_bounds__(kThreads) void by_big_kernel(ByBigArgs A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  float* Y = reinterpret_cast<float*>(lds + kByY);
  uint16_t* Mh = reinterpret_cast<uint16_t*>(lds + kByMh);
  uint16_t* Ml = reinterpret_cast<uint16_t*>(lds + kByMl);
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, q = lane >> 4, r16 = lane & 15;
  const LaneX lx = lane_x_init();
  int g = 0;
#pragma unroll
  for (int j = 1; j < QS_MAX_GROUP; ++j)
    if (j < A.njobs && (int)blockIdx.x >= A.job[j].wg0) g = j;
  const ByBigJob& J = A.job[g];
  const int lb = (int)blockIdx.x - J.wg0;
  const int b = lb / J.ngrp, k = lb - b * J.ngrp;
  const int Sm = J.Sm, Spad = (Sm + 31) & ~31;
  // wave w finishes output chunk r = 16 k + w (elements t = lane + 64 j):
  // its su and bias (no bias: a dummy load from the partial sums, at least m
  // floats, never used -- the bias term is selected, not multiplied by 0)
  const int r = 16 * k + w;
  const float* const bsrc = J.bias ? J.bias : J.y1p;
  const bool has_bias = J.bias != nullptr;
  int oidx[1][4];
  float suo[4], bio[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = lane + 64 * j;
    oidx[0][j] = r < Sm ? out_elem(r, t) : -1;
    const int ii = r < Sm ? out_elem(r, t) : 0;
    suo[j] = load_su(J.su, SB, ii);
    bio[j] = bsrc[ii];
  }
  // 1. z_c = the sum over the slice groups of chunk c, chunks c = w + 16 u
  //    (element t = lane + 64 j), into the chunk rows
  {
    float zv[kByCPW][4];
    sum_partials_loop<kByCPW>(J.y1p, J.m, Sm, J.SG, A.B, b, w, lane, zv);
    store_chunks_lanes<kByCPW>(Y, Sm, w, lane, zv);
  }
  // 2. this work-group's 16 rows of M
  build_m_rows(Mh, Ml, k, Sm, Spad, J.lsh_m, J.pm, J.Km, tid);
  __syncthreads();
  // 3. rows 16 k .. 16 k + 15 of M . z, column t = 16 w + r16
  floatx4 acc = {0.f, 0.f, 0.f, 0.f};
  const int tc = 16 * w + r16;
  for (int kb = 0; kb < (Spad >> 5); ++kb) {
    const ZOperand z = z_operand(Y, Sm, tc, q, kb);
    const int off = r16 * kMStr + 32 * kb + 8 * q;
    const bf16x8 ah = ld_bf16x8(Mh + off);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, z.h, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, z.l, acc, 0, 0, 0);
    if (J.pm > 1) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ld_bf16x8(Ml + off), z.h, acc, 0, 0, 0);
  }
  __syncthreads();  // every wave has read the chunk rows
  // 4. the 16 rows into the first 16 chunk rows; wave w then applies the
  //    256-point transform to row w (output chunk r), scale, su and bias
#pragma unroll
  for (int j = 0; j < 4; ++j) Y[(4 * q + j) * kYStride + tc] = acc[j];
  __syncthreads();
  if (r >= Sm) return;  // no barrier follows
  float v[1][4];
#pragma unroll
  for (int j = 0; j < 4; ++j) v[0][j] = Y[w * kYStride + lane + 64 * j];
  h256<1>(v, lane, lx);
  const float mul = J.scale_m * J.layer_scale * J.xmul[b];
  float out[1][4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    out[0][j] = apply_su(v[0][j] * mul, suo[j], SB, oidx[0][j]) + (has_bias ? bio[j] : 0.0f);
  store_outputs(J.y, A.y_dtype, (int64_t)b * J.ldy, oidx, out);
}

int big_lds(const void* fn, size_t bytes, int* done) {
  if (!*done) {
    hipFuncAttributes fa{};
    QS_HIP(hipFuncGetAttributes(&fa, fn));
    QS_REQUIRE(fa.sharedSizeBytes == 0, "per-row transform kernels must not use static LDS");
    QS_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    *done = 1;
  }
  return QS_OK;
}
template <int XT, bool SB>
int launch_bx_big_v(const BxBigArgs& A, unsigned grid, hipStream_t s) {
  static int done = 0;
  const int rc = big_lds((const void*)bx_big_kernel<XT, SB>, kBxLds, &done);
  if (rc) return rc;
  hipLaunchKernelGGL((bx_big_kernel<XT, SB>), dim3(grid), dim3(kThreads), kBxLds, s, A);
  QS_LAUNCHED("bx_big_kernel");
  return QS_OK;
}
template <bool SB>
int launch_by_big_v(const ByBigArgs& A, unsigned grid, hipStream_t s) {
  static int done = 0;
  const int rc = big_lds((const void*)by_big_kernel<SB>, kByLds, &done);
  if (rc) return rc;
  hipLaunchKernelGGL((by_big_kernel<SB>), dim3(grid), dim3(kThreads), kByLds, s, A);
  QS_LAUNCHED("by_big_kernel");
  return QS_OK;
}

}  // namespace

bool big_transform_fits(int64_t len, int p) {
  return len % 256 == 0 && len / 256 <= kBigMaxS && len / p >= 256 && p >= 1 && p <= QS_MAX_KRON;
}
bool big_input_fits(int64_t n, int p, int x_dtype) {
  return big_transform_fits(n, p) && (x_dtype == QS_DTYPE_BF16 || n / 256 <= kBigMaxS / 2);
}

int launch_bx_big(const BatchedPass& P, hipStream_t stream) {
  QS_REQUIRE(big_input_fits(P.n, P.pn, P.x_dtype) && P.B >= 1, "input transform: n %lld (p %d, dtype %d)",
             (long long)P.n, P.pn, P.x_dtype);
  QS_REQUIRE((reinterpret_cast<uintptr_t>(P.x) & (P.x_dtype == QS_DTYPE_F32 ? 15 : 7)) == 0 && P.ldx % 4 == 0,
             "input transform: x rows must be 8-byte (fp32: 16-byte) aligned");
  QS_REQUIRE((reinterpret_cast<uintptr_t>(P.sv) & (P.sbits ? 3 : 15)) == 0, "input transform: sv alignment");
  BxBigArgs A{};
  A.x = P.x;
  A.ldx = P.ldx;
  A.B = P.B;
  A.n = (int)P.n;
  A.S = (int)(P.n / 256);
  A.pn = P.pn;
  A.lsh_n = log2_exact(P.n / P.pn / 256);
  A.ngrp = (A.S + 15) / 16;
  A.Kn = P.Kn;
  A.scale_n = inv_sqrt_len(P.n / P.pn);
  A.sv = P.sv;
  A.x2h = P.x2h;
  A.sg = P.sg;
  A.xmul = P.xmul;
  A.frag = P.frag;
  const int64_t grid = (int64_t)P.B * A.ngrp;
  QS_REQUIRE(grid <= 0x7FFFFFFF, "input transform: %lld work-groups", (long long)grid);
  const int xt = P.x_dtype == QS_DTYPE_BF16 ? 0 : P.x_dtype == QS_DTYPE_F16 ? 1 : 2;
  const unsigned gr = (unsigned)grid;
  if (P.sbits) {
    return xt == 0 ? launch_bx_big_v<0, true>(A, gr, stream) : xt == 1 ? launch_bx_big_v<1, true>(A, gr, stream)
                                                                        : launch_bx_big_v<2, true>(A, gr, stream);
  }
  return xt == 0 ? launch_bx_big_v<0, false>(A, gr, stream) : xt == 1 ? launch_bx_big_v<1, false>(A, gr, stream)
                                                                       : launch_bx_big_v<2, false>(A, gr, stream);
}

int launch_by_big(const BatchedPass* P, int count, hipStream_t stream) {
  QS_REQUIRE(count >= 1 && count <= QS_MAX_GROUP, "output transform: 1..%d linears", QS_MAX_GROUP);
  ByBigArgs A{};
  A.B = P[0].B;
  A.y_dtype = P[0].y_dtype;
  A.njobs = count;
  int64_t wg = 0;
  for (int g = 0; g < count; ++g) {
    const BatchedPass& Q = P[g];
    QS_REQUIRE(big_transform_fits(Q.m, Q.pm) && Q.B == A.B && Q.y_dtype == A.y_dtype && Q.sbits == P[0].sbits,
               "output transform: m %lld (p %d) or mixed rows / dtype / sign format", (long long)Q.m, Q.pm);
    ByBigJob& J = A.job[g];
    J.y1p = Q.y1p;
    J.SG = Q.SG;
    J.m = (int)Q.m;
    J.Sm = (int)(Q.m / 256);
    J.pm = Q.pm;
    J.lsh_m = log2_exact(Q.m / Q.pm / 256);
    J.ngrp = (J.Sm + 15) / 16;
    J.wg0 = (int)wg;
    J.Km = Q.Km;
    J.scale_m = inv_sqrt_len(Q.m / Q.pm);
    J.layer_scale = Q.layer_scale;
    J.xmul = Q.xmul;
    J.su = Q.su;
    J.bias = Q.bias;
    J.y = Q.y;
    J.ldy = Q.ldy;
    wg += (int64_t)Q.B * J.ngrp;
  }
  QS_REQUIRE(wg <= 0x7FFFFFFF, "output transform: %lld work-groups", (long long)wg);
  return P[0].sbits ? launch_by_big_v<true>(A, (unsigned)wg, stream) : launch_by_big_v<false>(A, (unsigned)wg, stream);
}

}  // namespace qs
