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

// One pass (up to 16 rows) of the batched forward (qs_linear_batched.hip):
// input transform, decode-matvec and output transform launches.
struct BatchedPass {
  const void* x;
  int x_dtype;
  int64_t ldx;
  int B;                 // rows in this pass, 1..16
  int64_t n, m;
  int pn, pm;            // odd factors of n and m
  const float* Kn;
  const float* Km;
  const float* sv;
  const float* su;
  const void* codes0;    // tiled layout
  const void* codes1;    // E8 1-bit second stage or NULL
  float s0, s1, layer_scale;
  const float* bias;
  void* y;
  int y_dtype;
  int64_t ldy;
  int S, SG, W, ncu;     // slices, slice groups, waves per group, CUs
  _Float16* x2h;         // workspace: [B][n] fp16 operand
  _Float16* sg;          // workspace: [B][n / 8] group sums
  float* xmul;           // workspace: [B]
  float* y1p;            // workspace: [SG][B][m]
};
bool batched_eligible(int64_t n, int pn, int64_t m, int pm);
int launch_linear_batched(const BatchedPass& P, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop);
// The per-row input / output transform kernels of a pass on their own, for
// any number of rows P.B (the output reads P.SG partial groups of P.B rows).
int launch_bx_rows(const BatchedPass& P, hipStream_t stream);
int launch_by_rows(const BatchedPass& P, hipStream_t stream);

// Wide-batch GEMM (qs_linear_wide.hip): decode m x n codes into fp16 chunks
// of wide_chunk_rows() rows and multiply by the fp16 operand on the matrix
// cores, y1[B][m] = s0 X2 W0^T (+ s1 X2 W1^T).
constexpr int64_t kWideChunkElems = (int64_t)16 << 20;  // fp16 elements per dequantized chunk
struct WideGemm {
  const void* codes0;
  const void* codes1;
  int64_t m, n;
  int B;
  float s0, s1;
  const _Float16* x2h;   // [B][n]
  float* y1;             // [B][m]
  _Float16* wbuf;        // workspace: one chunk of stage-0 weights
  _Float16* wbuf2;       // workspace: one chunk of stage-1 weights (codes1)
  int ncu;
};
int64_t wide_chunk_rows(int64_t m, int64_t n);
int launch_linear_wide_gemm(const WideGemm& G, hipStream_t stream);

}  // namespace qs
