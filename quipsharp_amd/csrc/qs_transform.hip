// Randomized Hadamard transform along one axis of a [outer][n][inner] fp32
// tensor: the quantize-time incoherence transforms of quipsharp/incoherence.py
// (W_hat = H_m (S_u W S_v) H_n, H_hat = H_n (S_v H S_v) H_n, their inverses,
// and transform_input/transform_output).  The Walsh-Hadamard part is bit-exact
// with quipsharp/hadamard.py:17-40.
//
//  inner == 1 : one work-group per row, the whole row staged in LDS.
//  inner  > 1 : radix-64 passes over tiles of 64 axis elements x 64 inner
//               columns (256-byte row segments), then the odd-factor pass.
#include <cmath>

#include "qs_rht_dev.h"

namespace qs {
namespace {

constexpr int kRowThreads = 1024;
constexpr int kMaxRowLen = 32768;  // 128 KiB of LDS
constexpr int kTileR = 64;          // axis elements per column-pass tile
constexpr int kTileC = 64;          // inner columns per column-pass tile

struct RowArgs {
  const float* in;
  float* out;
  int n, logL, p, G;
  const float* K;
  const float* pre;
  const float* post;
  float scale;
};

// One work-group per (row, column share): the whole row is staged in LDS and
// transformed; with an odd factor each of the G work-groups of a row computes
// the K stage for L/G of the columns b and writes those outputs.
__global__ __launch_bounds__(kRowThreads) void rht_rows_kernel(RowArgs A) {
  extern __shared__ float sm[];
  float* buf = sm;
  float* Ks = sm + padded_len(A.n);
  const int64_t row = blockIdx.x / A.G;
  const int part = blockIdx.x - (int)(row * A.G);
  const int tid = threadIdx.x, nthr = blockDim.x;
  const float* src = A.in + row * A.n;
  for (int i = tid; i < A.n; i += nthr) {
    float v = src[i];
    if (A.pre) v = v * A.pre[i];
    buf[pad_idx(i)] = v;
  }
  if (A.p > 1)
    for (int i = tid; i < A.p * A.p; i += nthr) Ks[i] = A.K[i];
  __syncthreads();
  lds_fwht(buf, A.n, A.logL, tid, nthr);
  float* dst = A.out + row * A.n;
  if (A.p == 1) {
    for (int i = tid; i < A.n; i += nthr) {
      float v = buf[pad_idx(i)] * A.scale;
      if (A.post) v = v * A.post[i];
      dst[i] = v;
    }
    return;
  }
  for (int i = tid; i < A.n; i += nthr) buf[pad_idx(i)] = buf[pad_idx(i)] * A.scale;
  __syncthreads();
  const int L = 1 << A.logL;
  const int cw = L / A.G;
  const float* post = A.post;
  kron_cols(buf, Ks, A.p, A.logL, part * cw, (part + 1) * cw, tid, nthr, [&](int a, int b, float v) {
    const int i = (a << A.logL) + b;
    if (post) v = v * post[i];
    dst[i] = v;
  });
}

// One radix pass of Walsh-Hadamard stages h0, 2*h0, ..., h0*(R/2) on the axis.
struct ColArgs {
  const float* in;
  float* out;
  int64_t outer, n, inner;
  int L;         // length of the Walsh-Hadamard part (n = p*L)
  int h0;        // first stage of this pass
  int R;         // elements per butterfly group (2^stages of this pass)
  const float* pre_axis;
  const float* pre_inner;
  const float* post_axis;
  float scale;   // applied when != 0 (last Walsh-Hadamard pass)
};

__global__ __launch_bounds__(256) void rht_cols_pass_kernel(ColArgs A) {
  __shared__ float tile[kTileR][kTileC + 1];
  // group id -> (o, a, blk, off): elements a*L + blk*h0*R + off + h0*j
  const int64_t groups_per_seg = A.L / A.R;
  int64_t g = blockIdx.x;
  const int64_t o = g / ((A.n / A.L) * groups_per_seg);
  g -= o * ((A.n / A.L) * groups_per_seg);
  const int64_t a = g / groups_per_seg;
  const int64_t gi = g - a * groups_per_seg;
  const int64_t blk = gi / A.h0, off = gi - blk * A.h0;
  const int64_t base_i = a * A.L + blk * (int64_t)A.h0 * A.R + off;
  const int64_t c0 = (int64_t)blockIdx.y * kTileC;
  const int tc = threadIdx.x & (kTileC - 1);
  const int tr = threadIdx.x / kTileC;  // 0..3
  const int64_t c = c0 + tc;
  const bool cvalid = c < A.inner;
  for (int j = tr; j < A.R; j += 256 / kTileC) {
    const int64_t i = base_i + (int64_t)A.h0 * j;
    float v = 0.0f;
    if (cvalid) {
      v = A.in[(o * A.n + i) * A.inner + c];
      if (A.pre_axis) v = v * A.pre_axis[i];
      if (A.pre_inner) v = v * A.pre_inner[c];
    }
    tile[j][tc] = v;
  }
  __syncthreads();
  for (int h = 1; h < A.R; h <<= 1) {
    // R/2 butterflies per column, 4 rows of threads
    for (int t = tr; t < A.R / 2; t += 256 / kTileC) {
      const int b = t / h, of = t - b * h;
      const int j = b * 2 * h + of;
      const float x = tile[j][tc], y = tile[j + h][tc];
      tile[j][tc] = x + y;
      tile[j + h][tc] = x - y;
    }
    __syncthreads();
  }
  for (int j = tr; j < A.R; j += 256 / kTileC) {
    const int64_t i = base_i + (int64_t)A.h0 * j;
    float v = tile[j][tc];
    if (A.scale != 0.0f) v = v * A.scale;
    if (A.post_axis) v = v * A.post_axis[i];
    if (cvalid) A.out[(o * A.n + i) * A.inner + c] = v;
  }
}

// Odd-factor pass: for each (o, b, c): out[a] = sum_a' K[a][a'] in[a'], a = 0..p-1.
struct KronColArgs {
  const float* in;
  float* out;
  int64_t outer, n, inner;
  int L, p;
  const float* K;
  const float* post_axis;
};

__global__ __launch_bounds__(256) void rht_cols_kron_kernel(KronColArgs A) {
  __shared__ float tile[QS_MAX_KRON][kTileC];
  const int64_t o = blockIdx.x / A.L;
  const int64_t b = blockIdx.x - o * A.L;
  const int64_t c0 = (int64_t)blockIdx.y * kTileC;
  const int tc = threadIdx.x & (kTileC - 1);
  const int tr = threadIdx.x / kTileC;
  const int64_t c = c0 + tc;
  const bool cvalid = c < A.inner;
  for (int a = tr; a < A.p; a += 256 / kTileC)
    tile[a][tc] = cvalid ? A.in[(o * A.n + a * A.L + b) * A.inner + c] : 0.0f;
  __syncthreads();
  for (int a = tr; a < A.p; a += 256 / kTileC) {
    float s = 0.0f;
    for (int k = 0; k < A.p; ++k) s = __builtin_fmaf(A.K[a * A.p + k], tile[k][tc], s);
    const int64_t i = a * A.L + b;
    if (A.post_axis) s = s * A.post_axis[i];
    if (cvalid) A.out[(o * A.n + i) * A.inner + c] = s;
  }
}

}  // namespace
}  // namespace qs

using namespace qs;

extern "C" int qs_rht_f32(const float* in, float* out, int64_t outer, int64_t n, int64_t inner,
                          const float* pre_axis, const float* pre_inner, const float* post_axis, int kron_p,
                          const float* kron_mat, qs_stream_t stream) {
  QS_REQUIRE(outer >= 0 && n >= 1 && inner >= 1, "bad shape outer=%lld n=%lld inner=%lld", (long long)outer,
             (long long)n, (long long)inner);
  QS_REQUIRE(kron_p >= 1 && (kron_p & 1) && kron_p <= QS_MAX_KRON, "kron_p must be odd in [1, %d]", QS_MAX_KRON);
  QS_REQUIRE(n % kron_p == 0, "n=%lld is not divisible by kron_p=%d", (long long)n, kron_p);
  const int64_t L = n / kron_p;
  QS_REQUIRE((L & (L - 1)) == 0, "n / kron_p must be a power of two (n=%lld, p=%d)", (long long)n, kron_p);
  QS_REQUIRE(kron_p == 1 || kron_mat, "kron_mat is required when kron_p > 1");
  QS_REQUIRE(in && out, "null pointer");
  if (outer == 0) return QS_OK;
  hipStream_t s = as_stream(stream);
  const float scale = inv_sqrt_len(L);
  if (inner == 1) {
    QS_REQUIRE(n <= kMaxRowLen, "row transform supports n <= %d (got %lld)", kMaxRowLen, (long long)n);
    // Work-groups of one row read the whole row: split the odd-factor stage over
    // several of them only when the output does not overwrite the input.
    const int G = (kron_p > 1 && in != out) ? (L / 8 < 16 ? (int)(L / 8 > 0 ? L / 8 : 1) : 16) : 1;
    QS_REQUIRE(outer * G < (1ll << 31), "too many rows");
    const size_t lds = ((size_t)padded_len((int)n) + (kron_p > 1 ? (size_t)kron_p * kron_p : 0)) * sizeof(float);
    if (lds > 65536)
      QS_HIP(hipFuncSetAttribute((const void*)rht_rows_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)lds));
    RowArgs A{in, out, (int)n, log2_exact(L), kron_p, G, kron_mat, pre_axis, post_axis, scale};
    hipLaunchKernelGGL(rht_rows_kernel, dim3((unsigned)(outer * G)), dim3(kRowThreads), lds, s, A);
    QS_LAUNCHED("rht_rows_kernel");
    return QS_OK;
  }
  // column passes
  int logL = 0;
  while ((1ll << logL) < L) ++logL;
  const int64_t ctiles = (inner + kTileC - 1) / kTileC;
  QS_REQUIRE(ctiles < 65536, "inner too large");
  const float* src = in;
  int done = 0;
  bool first = true;  // logL == 0 still runs one pass (R = 1) to apply signs
  do {
    const int bits = logL - done < 6 ? logL - done : 6;
    const int R = 1 << bits;
    const int h0 = 1 << done;
    const bool last = done + bits >= logL;
    ColArgs A{};
    A.in = src;
    A.out = out;
    A.outer = outer;
    A.n = n;
    A.inner = inner;
    A.L = (int)L;
    A.h0 = h0;
    A.R = R;
    A.pre_axis = first ? pre_axis : nullptr;
    A.pre_inner = first ? pre_inner : nullptr;
    A.post_axis = (last && kron_p == 1) ? post_axis : nullptr;
    A.scale = last ? scale : 0.0f;
    const int64_t groups = outer * kron_p * (L / R);
    QS_REQUIRE(groups < (1ll << 31), "too many groups");
    hipLaunchKernelGGL(rht_cols_pass_kernel, dim3((unsigned)groups, (unsigned)ctiles), dim3(256), 0, s, A);
    QS_LAUNCHED("rht_cols_pass_kernel");
    src = out;
    first = false;
    done += bits;
  } while (done < logL);
  if (kron_p > 1) {
    KronColArgs K{out, out, outer, n, inner, (int)L, kron_p, kron_mat, post_axis};
    const int64_t groups = outer * L;
    QS_REQUIRE(groups < (1ll << 31), "too many groups");
    hipLaunchKernelGGL(rht_cols_kron_kernel, dim3((unsigned)groups, (unsigned)ctiles), dim3(256), 0, s, K);
    QS_LAUNCHED("rht_cols_kron_kernel");
  }
  return QS_OK;
}
