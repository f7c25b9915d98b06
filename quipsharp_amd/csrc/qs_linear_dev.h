// Host-side interface between the forward launchers (qs_linear.hip) and the
// one-launch kernel (qs_linear_fused.hip).
#pragma once

#include "qs_common.h"

namespace qs {

// One linear of a one-launch forward; all linears of a launch share x and n.
struct FusedJobDesc {
  const void* codes0;   // packed E8P codes (tiled layout)
  const void* codes1;   // packed E8 1-bit codes or NULL
  int64_t m;
  const float* sv;
  const float* su;
  int pm;               // odd factor of m (output transform)
  const float* Km;      // pm x pm K factor of the output transform (pm > 1)
  float s0, s1, layer_scale;
  const float* bias;
  void* y;
  int64_t ldy;
  unsigned* counter;    // workspace: completion counter (zero between calls)
  float* xmul;          // workspace: [B] activation scales
  float* y1p;           // workspace: [SG][B][m] partial sums
};

int launch_linear_fused(const void* x, int x_dtype, int64_t ldx, int B, int n, int pn, const float* Kn, int y_dtype,
                        int count, const FusedJobDesc* jobs, int S, int SG, int W, int ncu, hipStream_t stream,
                        hipEvent_t ev_start, hipEvent_t ev_stop);
bool fused_eligible(int64_t batch, int64_t n, int64_t m, int pn);
bool fused_output_in_kernel(int64_t m, int pm);

}  // namespace qs
