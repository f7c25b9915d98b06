// Wide-batch quantized-linear forward (prefill: 32 or more activation rows
// per call), the path QuantizedLinear.forward takes for a long prompt
// (quipsharp/checkpoint.py:141-146 -> quipsharp/quantize.py:116-124: the
// reference decodes the whole weight and multiplies densely).  With many
// rows the contraction is a real GEMM, so the codes are decoded once per call
// into exact fp16 weights and multiplied by a library GEMM on the matrix
// cores:
//   dq_kernel   codes (tiled layout) -> W_hat rows in fp16: every E8P value
//               +-(k + 1/2) +- 1/4 and every E8 1-bit value is exact in fp16,
//               so the dense weights are the codebook values themselves
//               (the layer scales stay in the GEMM's alpha);
//   rocBLAS     Y1^T[rows][B] = alpha W_hat[rows][n] X2^T (fp16 x fp16 ->
//               fp32, MFMA); a second E8 1-bit stage accumulates with
//               beta = 1.
// The input and output transforms around it are the per-row kernels of the
// batched path (qs_linear_batched.hip) or, outside the chunk scheme, the
// LDS-radix kernels of qs_linear.hip.
#include <mutex>

#include <rocblas/rocblas.h>

#include "qs_forward_dev.h"
#include "qs_linear_dev.h"

namespace qs {
namespace {

constexpr int kThreads = kFwdThreads;
constexpr int kDqOffHi = 0;                // 4096 x uint32 LUT entries
constexpr int kDqOffLo = 16384;
constexpr int kDqOffLut1 = 32768;          // 256 x uint4 (E8 1-bit rows, fp16)
constexpr int kDqOffTab = kDqOffLut1 + 4096;  // 256 x uint4 (abs table staging)
constexpr int kDqLds = kDqOffTab + 4096;

struct DqArgs {
  const uint16_t* codes0;
  const uint8_t* codes1;
  int S;           // slices of 256 columns
  int rb0, nrb;    // first row block and row blocks of this chunk
  int n;
  _Float16* w;     // [nrb * 16][n]
  _Float16* w2;    // [nrb * 16][n] (second stage) or null
};

// One 1 KiB code tile (16 rows x 256 columns) per wave per step; lane
// (q, r16) writes row r16, columns 64 q .. 64 q + 63 of its slice.
template <bool HAS2>
__global__ __launch_bounds__(kThreads) void dq_kernel(DqArgs A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint32_t* lut_hi = reinterpret_cast<uint32_t*>(lds + kDqOffHi);
  uint32_t* lut_lo = reinterpret_cast<uint32_t*>(lds + kDqOffLo);
  uint4* lut1 = reinterpret_cast<uint4*>(lds + kDqOffLut1);
  uint4* tab16 = reinterpret_cast<uint4*>(lds + kDqOffTab);
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  if (tid < 256) {
    tab16[tid] = *reinterpret_cast<const uint4*>(kE8Ph.w[tid]);
    if (HAS2) lut1[tid] = *reinterpret_cast<const uint4*>(kE81h.w[tid]);
  }
  __syncthreads();
  fill_luts(tab16, lut_hi, lut_lo, tid);
  __syncthreads();
  const _Float16 qv = (_Float16)0.25f;
  const half8 quarter = {qv, qv, qv, qv, qv, qv, qv, qv};
  const int ntiles = A.nrb * A.S;
  for (int t = (int)blockIdx.x * kWaves + w; t < ntiles; t += (int)gridDim.x * kWaves) {
    const int rbl = t / A.S, sl = t - rbl * A.S;
    const size_t tile = ((size_t)(A.rb0 + rbl) * A.S + sl) * 64 + lane;
    const uint4 cw = *reinterpret_cast<const uint4*>(A.codes0 + tile * 8);
    uint2 cw1 = make_uint2(0, 0);
    if (HAS2) cw1 = *reinterpret_cast<const uint2*>(A.codes1 + tile * 8);
    const uint32_t wd[4] = {cw.x, cw.y, cw.z, cw.w};
    const size_t o = (size_t)(16 * rbl + r16) * A.n + 256 * sl + 64 * q;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const half8 v = decode_code(wd[c >> 1], c, kDqOffHi, kDqOffLo);
      const bool up = (wd[c >> 1] >> (16 * (c & 1))) & 1u;  // shift +1/4 (else -1/4)
      const half8 vs = up ? v + quarter : v - quarter;      // exact in fp16
      *reinterpret_cast<half8*>(A.w + o + 8 * c) = vs;
      if (HAS2) {
        const uint32_t idx = ((c < 4 ? cw1.x : cw1.y) >> (8 * (c & 3))) & 0xFFu;
        *reinterpret_cast<uint4*>(A.w2 + o + 8 * c) = lut1[idx];
      }
    }
  }
}

std::mutex g_blas_mu;
rocblas_handle g_blas[64] = {};

int blas_handle(rocblas_handle* h) {
  int dev = 0;
  QS_HIP(hipGetDevice(&dev));
  QS_REQUIRE(dev >= 0 && dev < 64, "device index %d", dev);
  if (!g_blas[dev]) {
    rocblas_handle nh = nullptr;
    QS_REQUIRE(rocblas_create_handle(&nh) == rocblas_status_success, "rocblas_create_handle failed");
    // same result on every call: no split-K solutions that accumulate with atomics
    QS_REQUIRE(rocblas_set_atomics_mode(nh, rocblas_atomics_not_allowed) == rocblas_status_success,
               "rocblas_set_atomics_mode failed");
    g_blas[dev] = nh;
  }
  *h = g_blas[dev];
  return QS_OK;
}

int lds_attr_done[2] = {0, 0};

}  // namespace

int64_t wide_chunk_rows(int64_t m, int64_t n) {
  int64_t r = (kWideChunkElems / n) / 256 * 256;
  if (r < 16) r = 16;
  if (r > m) r = m;
  return r;
}

int launch_linear_wide_gemm(const WideGemm& G, hipStream_t stream) {
  QS_REQUIRE(G.m % 16 == 0 && G.n % 256 == 0 && G.B >= 1, "wide GEMM: m %% 16, n %% 256");
  const bool has2 = G.codes1 != nullptr;
  const void* kfn = has2 ? (const void*)dq_kernel<true> : (const void*)dq_kernel<false>;
  if (!lds_attr_done[has2]) {
    hipFuncAttributes fa{};
    QS_HIP(hipFuncGetAttributes(&fa, kfn));
    QS_REQUIRE(fa.sharedSizeBytes == 0, "dq_kernel must not use static LDS");
    QS_HIP(hipFuncSetAttribute(kfn, hipFuncAttributeMaxDynamicSharedMemorySize, kDqLds));
    lds_attr_done[has2] = 1;
  }
  std::lock_guard<std::mutex> lock(g_blas_mu);
  rocblas_handle h = nullptr;
  int rc = blas_handle(&h);
  if (rc) return rc;
  QS_REQUIRE(rocblas_set_stream(h, stream) == rocblas_status_success, "rocblas_set_stream failed");
  const int64_t R = wide_chunk_rows(G.m, G.n);
  for (int64_t r0 = 0; r0 < G.m; r0 += R) {
    const int64_t rows = G.m - r0 < R ? G.m - r0 : R;
    DqArgs D{};
    D.codes0 = static_cast<const uint16_t*>(G.codes0);
    D.codes1 = static_cast<const uint8_t*>(G.codes1);
    D.S = (int)(G.n / 256);
    D.rb0 = (int)(r0 / 16);
    D.nrb = (int)(rows / 16);
    D.n = (int)G.n;
    D.w = G.wbuf;
    D.w2 = G.wbuf2;
    const int64_t tiles = (rows / 16) * D.S;
    int64_t grid = (tiles + kWaves - 1) / kWaves;
    if (grid > 4 * G.ncu) grid = 4 * G.ncu;
    if (has2)
      hipLaunchKernelGGL(dq_kernel<true>, dim3((unsigned)grid), dim3(kThreads), kDqLds, stream, D);
    else
      hipLaunchKernelGGL(dq_kernel<false>, dim3((unsigned)grid), dim3(kThreads), kDqLds, stream, D);
    QS_LAUNCHED("dq_kernel");
    // Row-major Y1[B][m] is column-major Y1^T (m x B, ldc = m); its rows
    // r0 .. r0 + rows are op(A) op(B) with A the fp16 chunk (row-major
    // rows x n = column-major n x rows, lda = n, transposed) and B the fp16
    // operand X2 (row-major B x n = column-major n x B, ldb = n).
    const float beta0 = 0.0f, beta1 = 1.0f;
    float* c = G.y1 + r0;
    rocblas_status st = rocblas_gemm_ex(
        h, rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)rows, (rocblas_int)G.B,
        (rocblas_int)G.n, &G.s0, G.wbuf, rocblas_datatype_f16_r, (rocblas_int)G.n, G.x2h, rocblas_datatype_f16_r,
        (rocblas_int)G.n, &beta0, c, rocblas_datatype_f32_r, (rocblas_int)G.m, c, rocblas_datatype_f32_r,
        (rocblas_int)G.m, rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
    QS_REQUIRE(st == rocblas_status_success, "rocblas_gemm_ex failed (%d)", (int)st);
    if (has2) {
      st = rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, (rocblas_int)rows,
                           (rocblas_int)G.B, (rocblas_int)G.n, &G.s1, G.wbuf2, rocblas_datatype_f16_r,
                           (rocblas_int)G.n, G.x2h, rocblas_datatype_f16_r, (rocblas_int)G.n, &beta1, c,
                           rocblas_datatype_f32_r, (rocblas_int)G.m, c, rocblas_datatype_f32_r, (rocblas_int)G.m,
                           rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
      QS_REQUIRE(st == rocblas_status_success, "rocblas_gemm_ex failed (%d)", (int)st);
    }
  }
  return QS_OK;
}

}  // namespace qs
