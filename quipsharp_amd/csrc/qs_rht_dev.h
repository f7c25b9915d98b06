// In-LDS randomized-Hadamard building blocks shared by the transform and the
// forward kernels.  A length-n vector (n = p * L, L = 2^k, p odd) is indexed
// i = a*L + b.  T_n applies the Sylvester Walsh-Hadamard stages over b (h = 1,
// 2, 4, ..., exactly the butterfly order of quipsharp/hadamard.py:37-43), the
// scale fl(L^-1/2), and then, when p > 1, the p x p orthogonal matrix K over a.
#pragma once

#include "qs_common.h"

namespace qs {

// Walsh-Hadamard stages over the low log2(L) index bits of buf[0..n), all
// threads of the block participating.  Ends with a barrier.
__device__ __forceinline__ void lds_fwht_stages(float* buf, int n, int L) {
  const int half = n >> 1;
  for (int h = 1; h < L; h <<= 1) {
    for (int t = threadIdx.x; t < half; t += blockDim.x) {
      // t enumerates the n/2 butterflies of this stage
      const int blk = t / h, off = t - blk * h;
      const int i = blk * 2 * h + off;
      const float a = buf[i], b = buf[i + h];
      buf[i] = a + b;
      buf[i + h] = a - b;
    }
    __syncthreads();
  }
}

// buf[i] *= scale, then the K stage over a when p > 1.  Ends with a barrier.
// K is p x p fp32, row-major, in global memory.
__device__ __forceinline__ void lds_scale_kron(float* buf, int n, int L, int p, const float* K, float scale) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) buf[i] = buf[i] * scale;
  __syncthreads();
  if (p <= 1) return;
  // Work unit = (column b, share of <= 16 outputs a).  All reads of an
  // iteration complete before its writes (barrier), so the update is in place.
  const int parts = (p + 15) / 16;
  const int per = (p + parts - 1) / parts;
  const int cols = (int)blockDim.x / parts > 0 ? (int)blockDim.x / parts : 1;
  for (int b0 = 0; b0 < L; b0 += cols) {
    const int t = threadIdx.x;
    const int part = t / cols;
    const int b = b0 + t % cols;
    const bool active = part < parts && b < L;
    const int a0 = part * per;
    const int a1 = a0 + per < p ? a0 + per : p;
    float acc[16];
    if (active) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        if (a0 + j < a1) {
          const float* Kr = K + (a0 + j) * p;
          float s = 0.0f;
          for (int c = 0; c < p; ++c) s = __builtin_fmaf(Kr[c], buf[c * L + b], s);
          acc[j] = s;
        }
      }
    }
    __syncthreads();
    if (active) {
#pragma unroll
      for (int j = 0; j < 16; ++j)
        if (a0 + j < a1) buf[(a0 + j) * L + b] = acc[j];
    }
    __syncthreads();
  }
}

// Full T_n in place.  scale must be fl(L^-1/2).
__device__ __forceinline__ void lds_rht(float* buf, int n, int L, int p, const float* K, float scale) {
  lds_fwht_stages(buf, n, L);
  lds_scale_kron(buf, n, L, p, K, scale);
}

// fl(L ** -0.5) computed like Python's float power, then rounded to fp32.
inline float inv_sqrt_len(int64_t L) { return (float)__builtin_pow((double)L, -0.5); }

}  // namespace qs
