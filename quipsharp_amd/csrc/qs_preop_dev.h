// Pre-operations on bf16 activation rows with one arithmetic wherever they
// run: RMSNorm with the residual add (transformers' Qwen3RMSNorm after
// `hidden_states = residual + hidden_states`: h' = bf16(x + delta),
// x' = bf16(weight * bf16(h' * rs)), rs = 1 / sqrt(mean(h'^2) + eps)) where
// the one-launch forward loads its input (qs_linear_fused.hip) and in the
// standalone decode-step kernel (qs_decoder.hip), and SiLU(gate) * up
// (x' = bf16(bf16(silu(g)) * u)) in the standalone kernel.
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
__device__ __forceinline__ uint32_t bf16_pair(float lo, float hi) {
  return (uint32_t)f32_to_bf16(lo) | ((uint32_t)f32_to_bf16(hi) << 16);
}
__device__ __forceinline__ float round_bf16(float f) { return __uint_as_float((uint32_t)f32_to_bf16(f) << 16); }

// h' = bf16(x + delta) in place (x itself without a delta); returns the sum
// of h'^2 over the quad.
__device__ __forceinline__ float rms_quad_resid(uint32_t (&h)[4][2], const uint32_t (&d)[4][2], bool has_delta) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      if (has_delta) h[i][k] = bf16_pair(bf16_lo(h[i][k]) + bf16_lo(d[i][k]), bf16_hi(h[i][k]) + bf16_hi(d[i][k]));
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
    for (int k = 0; k < 2; ++k) {
      const float lo = round_bf16(bf16_lo(h[i][k]) * rs), hi = round_bf16(bf16_hi(h[i][k]) * rs);
      h[i][k] = bf16_pair(bf16_lo(wt[i][k]) * lo, bf16_hi(wt[i][k]) * hi);
    }
}

// bf16(silu(g)) (transformers' SiLU on a bf16 tensor).
__device__ __forceinline__ float silu_bf16(float g) { return round_bf16(g / (1.0f + __expf(-g))); }

}  // namespace qs
