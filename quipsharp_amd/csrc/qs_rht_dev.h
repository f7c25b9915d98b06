// In-LDS randomized-Hadamard building blocks shared by the transform and the
// forward kernels.  A length-n vector (n = p * L, L = 2^k, p odd) is indexed
// i = a*L + b.  T_n applies the Sylvester Walsh-Hadamard stages over b (h = 1,
// 2, 4, ..., exactly the butterfly order of quipsharp/hadamard.py:37-43), the
// scale fl(L^-1/2), and then, when p > 1, the p x p orthogonal matrix K over a.
//
// The Walsh-Hadamard stages run in rounds of up to four: each thread loads the
// 16 elements of one butterfly group (stride h0) from LDS, applies the round's
// stages in registers in ascending order, and writes them back -- one barrier
// per round instead of one per stage.  LDS arrays are padded by one float per
// 32 (pad_idx) so the strided group loads do not pile onto one bank.
#pragma once

#include "qs_common.h"

namespace qs {

__device__ __forceinline__ int pad_idx(int i) { return i + (i >> 5); }
__host__ __device__ constexpr int padded_len(int n) { return n + (n >> 5) + 1; }

template <int BITS>
__device__ __forceinline__ void fwht_round(float* buf, int n, int logL, int logh0, int tid, int nthr) {
  constexpr int R = 1 << BITS;
  const int L = 1 << logL;
  const int groups_per_seg = L >> BITS;
  const int ngroups = (n >> logL) * groups_per_seg;
  const int h0 = 1 << logh0;
  for (int g = tid; g < ngroups; g += nthr) {
    const int a = g >> (logL - BITS);
    const int gi = g & (groups_per_seg - 1);
    const int blk = gi >> logh0, off = gi & (h0 - 1);
    const int base = (a << logL) + (blk << (logh0 + BITS)) + off;
    float v[R];
#pragma unroll
    for (int j = 0; j < R; ++j) v[j] = buf[pad_idx(base + (j << logh0))];
#pragma unroll
    for (int s = 0; s < BITS; ++s) {
      const int hh = 1 << s;
#pragma unroll
      for (int j = 0; j < R; ++j) {
        if ((j & hh) == 0) {
          const float x = v[j], y = v[j + hh];
          v[j] = x + y;
          v[j + hh] = x - y;
        }
      }
    }
#pragma unroll
    for (int j = 0; j < R; ++j) buf[pad_idx(base + (j << logh0))] = v[j];
  }
}

// All Walsh-Hadamard stages over the low logL index bits of the padded buffer
// (threads tid < nthr of the block participate; every thread of the block
// must call this, it contains barriers).  The radix adapts so that every
// participating thread owns about one butterfly group per round: a 4096-point
// transform on 1024 threads runs six radix-4 rounds.  Ends with a barrier.
__device__ __forceinline__ void lds_fwht(float* buf, int n, int logL, int tid, int nthr) {
  int per = n / nthr;  // elements per thread
  int rb = 2;
  while (rb < 4 && (2 << rb) <= per) ++rb;  // radix 4, 8 or 16
  int done = 0;
  while (done < logL) {
    const int bits = logL - done >= rb ? rb : logL - done;
    if (bits == 4) fwht_round<4>(buf, n, logL, done, tid, nthr);
    else if (bits == 3) fwht_round<3>(buf, n, logL, done, tid, nthr);
    else if (bits == 2) fwht_round<2>(buf, n, logL, done, tid, nthr);
    else fwht_round<1>(buf, n, logL, done, tid, nthr);
    done += bits;
    __syncthreads();
  }
}

// out[a][b] = sum_c K[a][c] * in[c][b] for columns b in [b0, b1), all a < p,
// reading the padded buffer `in` and writing `out(a, b)` through a functor.
// K is p x p fp32 in LDS.  No barrier.
template <class Out>
__device__ __forceinline__ void kron_cols(const float* in, const float* K, int p, int logL, int b0, int b1,
                                          int tid, int nthr, Out out) {
  const int cols = b1 - b0;
  const int total = p * cols;
  for (int u = tid; u < total; u += nthr) {
    const int a = u / cols;
    const int b = b0 + (u - a * cols);
    const float* Kr = K + a * p;
    float s = 0.0f;
    for (int c = 0; c < p; ++c) s = __builtin_fmaf(Kr[c], in[pad_idx((c << logL) + b)], s);
    out(a, b, s);
  }
}

// fl(L ** -0.5) computed like Python's float power, then rounded to fp32.
inline float inv_sqrt_len(int64_t L) { return (float)__builtin_pow((double)L, -0.5); }

inline int log2_exact(int64_t v) {
  int k = 0;
  while ((1ll << k) < v) ++k;
  return k;
}

}  // namespace qs
