// Pre-operations on bf16 activation rows with one arithmetic wherever they
// run: RMSNorm with the residual add (transformers' Qwen3RMSNorm after
// `hidden_states = residual + hidden_states`: h' = bf16(x + delta),
// x' = bf16(weight * bf16(h' * rs)), rs = 1 / sqrt(mean(h'^2) + eps)) where
// the one-launch forward loads its input (qs_linear_fused.hip) and in the
// standalone decode-step kernel (qs_decoder.hip) and the multi-row input
// transform (qs_linear_batched.hip, through rms_row_scale), and SiLU(gate) *
// up (x' = bf16(bf16(silu(g)) * u)) in the standalone kernel.
// Layout: the activation quads of the forward's loader -- thread (w, lane) of
// a 1024-thread work-group holds chunks c0 + i (i < 4, c0 = 64 round + 4 w)
// at columns 4 lane + u (u < 4) as two bf16 pairs per chunk.  The sum of
// squares is taken in one order (per thread chunk by chunk, pair by pair,
// low element first, fused multiply-adds; the second round after the first;
// then wave_sum; then the 16 waves in order), so a norm in the loader equals
// qs_dec_rmsnorm's bit for bit.
#pragma once

#include "qs_chunk_dev.h"

namespace qs {

__device__ __forceinline__ float bf16_lo(uint32_t p) { return __uint_as_float(p << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t p) { return __uint_as_float(p & 0xFFFF0000u); }
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) { return f32x2_to_bf16x2(lo, hi); }
__device__ __forceinline__ float round_bf16(float f) { return __uint_as_float((uint32_t)f32_to_bf16(f) << 16); }

// h' = bf16(x + delta) of one bf16 pair.
__device__ __forceinline__ uint32_t rms_pair_resid(uint32_t h, uint32_t d) {
  return bf16_pair(bf16_lo(h) + bf16_lo(d), bf16_hi(h) + bf16_hi(d));
}

// x' = bf16(weight * bf16(h' * rs)) of one bf16 pair.
__device__ __forceinline__ uint32_t rms_pair_apply(uint32_t h, uint32_t wt, float rs) {
  const float lo = round_bf16(bf16_lo(h) * rs), hi = round_bf16(bf16_hi(h) * rs);
  return bf16_pair(bf16_lo(wt) * lo, bf16_hi(wt) * hi);
}

// h' = bf16(x + delta) in place (x itself without a delta); returns the sum
// of h'^2 over the quad.
__device__ __forceinline__ float rms_quad_resid(uint32_t (&h)[4][2], const uint32_t (&d)[4][2], bool has_delta) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if (has_delta) h[i][k] = rms_pair_resid(h[i][k], d[i][k]);
      const float lo = bf16_lo(h[i][k]), hi = bf16_hi(h[i][k]);
      ss = __builtin_fmaf(lo, lo, ss);
      ss = __builtin_fmaf(hi, hi, ss);
    }
  return ss;
}

// rs from the row's sum of squares over n elements.
__device__ __forceinline__ float rms_scale(float ss, int n, float eps) { return 1.0f / sqrtf(ss / (float)n + eps); }

// x' = bf16(weight * bf16(h' * rs)) in place.
__device__ __forceinline__ void rms_quad_apply(uint32_t (&h)[4][2], const uint32_t (&wt)[4][2], float rs) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int k = 0; k < 2; ++k) h[i][k] = rms_pair_apply(h[i][k], wt[i][k], rs);
}

// rs of one bf16 row of n (a multiple of 256, at most 16384) with the
// residual delta (may be null), for a work-group that holds the row in
// another layout: thread (w, lane) of the 1024 reads its quad (chunks
// 4 w + i, i < 4, columns 4 lane + u) of h and delta (in memory or LDS; a
// null delta with h' itself), and the sum runs in the order above -- the
// same rs as rmsnorm_kernel's for the row.  wsum: kWaves
// floats of LDS that no other thread reads meanwhile; one barrier inside.
__device__ __forceinline__ float rms_row_scale(const uint16_t* h, const uint16_t* d, int n, float eps, int w,
                                               int lane, LaneX lx, float* wsum) {
  const int S = n / 256;
  uint32_t hv[4][2], dv[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int c = 4 * w + i, e = 256 * c + 4 * lane;
    uint2 a = make_uint2(0, 0), b = make_uint2(0, 0);
    if (c < S) {
      a = *reinterpret_cast<const uint2*>(h + e);
      if (d) b = *reinterpret_cast<const uint2*>(d + e);
    }
    hv[i][0] = a.x, hv[i][1] = a.y;
    dv[i][0] = b.x, dv[i][1] = b.y;
  }
  float ss = rms_quad_resid(hv, dv, d != nullptr);
  ss = wave_sum(ss, lx);
  if (lane == 0) wsum[w] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) tot += wsum[i];
  return rms_scale(tot, n, eps);
}

// bf16(silu(g)) (transformers' SiLU on a bf16 tensor).
__device__ __forceinline__ float silu_bf16(float g) { return round_bf16(g / (1.0f + __expf(-g))); }

}  // namespace qs
