// Host-side interface between the forward launchers (qs_linear.hip) and the
// one-launch kernel (qs_linear_fused.hip).
#pragma once

#include "qs_common.h"
#include "qs_tags.h"

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
  unsigned* epoch;      // workspace: tag of the last launch's partial sums (zero before the first call)
  TagWs tw;             // workspace: wrap word and extent (tag_ws; ntail set by the launcher)
  float* xmul;          // workspace: [B] activation scales
  float* y1p;           // workspace: [SG][B][m] fp32 partial sums (output transform in a separate kernel)
  unsigned long long* y1t;  // workspace: [SG][B][m] tagged partial sums (output transform in the kernel)
  unsigned long long* h2t;  // workspace: [B][m] tagged chunk transforms (output transform in two levels)
};

// How the one-launch kernel splits S chunks over a 16-wave work-group: SG
// slice groups of W slices, each slice taken by P waves (row-block phases),
// W P <= 16, P in {1, 2, 4}.
struct FusedPlan {
  int SG, W, P;
};
FusedPlan fused_plan(int S);
// A pre-operation on the bf16 input rows of a one-launch forward
// (qs_preop_dev.h; the fields of qs_preop, include/quipsharp_hip.h).
struct FusedPre {
  int kind;             // QS_PREOP_RMSNORM
  const void* x2;       // the residual delta (or NULL)
  int64_t ldx2;
  const void* weight;   // norm weights [n]
  void* h_out;          // x + delta [B][ldo] (or NULL)
  int64_t ldo;
  float eps;
};
int launch_linear_fused(const void* x, int x_dtype, int64_t ldx, int B, int n, int pn, const float* Kn, int y_dtype,
                        int sbits, int count, const FusedJobDesc* jobs, int S, const FusedPlan& plan, int ncu,
                        hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop, const FusedPre* pre = nullptr);
bool fused_eligible(int64_t batch, int64_t n, int x_dtype, int pn);
bool fused_x_aligned(const void* x, int x_dtype, int64_t ldx);
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
  _Float16* x2h;         // workspace: [B][n] fp16 operand (fragment-major with frag)
  _Float16* sg;          // workspace: [B][n / 8] group sums (fragment-major / 4 with frag)
  int sbits;             // sv and su are packed sign bits (QS_SIGNS_BITS)
  int frag;              // input transform writes x2h and sg fragment-major (the order the decode-matvec
                         // and the wide GEMM read; the decode-matvec requires it)
  float* xmul;           // workspace: [B]
  float* y1p;            // workspace: [SG][B][m]
  unsigned long long* y1t;  // workspace: [SG][B][m] tagged slots, or null: with them the decode-matvec
                            // applies the output transform itself (bm_tail_eligible)
  unsigned* epoch;       // the epoch word of the linear's tags (with y1t)
  TagWs tw;              // the linear's wrap word and the workspace (tag_ws; with y1t)
};
bool batched_eligible(int64_t n, int pn, int64_t m, int pm);
// The decode-matvec of these linears may also apply their output transforms
// (one launch fewer per pass; launch_bm / launch_bm_group report it in
// tail_done) when every one has tagged slots (y1t, epoch), at most 16 rows, m
// on the chunk scheme, and they share the output dtype and sign format.
bool bm_tail_eligible(const BatchedPass* P, int count);
int launch_linear_batched(const BatchedPass& P, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop);
// The per-row input / output transform kernels of a pass on their own, for
// any number of rows P.B (the output reads P.SG partial groups of P.B rows).
int launch_bx_rows(const BatchedPass& P, hipStream_t stream);
int launch_by_rows(const BatchedPass& P, hipStream_t stream);
// Input transforms of several linears of one x (each its own sv, x2h, sg,
// xmul) in one launch, bit-identical to one launch_bx_rows per linear.
int launch_bx_group(const BatchedPass* P, int count, hipStream_t stream, const FusedPre* pre = nullptr);
// The decode-matvec of a pass on its own (any n; operand in x2h / sg,
// fragment-major, 16 rows), y1p[SG][B][m].
int launch_bm(const BatchedPass& P, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop,
              bool* tail_done = nullptr);
// The same for several linears of one operand (shared x2h, sg, n, B, slice
// grouping, stages) in one launch: the work-groups are dealt to the linears in
// proportion to their rows.  Bit-identical to one launch per linear.
int launch_bm_group(const BatchedPass* P, int count, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop,
                    bool* tail_done = nullptr);
// Output transforms of several linears (shared B, xmul and output dtype; each
// its own P[j].SG partial groups) in one launch, bit-identical to one
// launch_by_rows per linear.
int launch_by_group(const BatchedPass* P, int count, hipStream_t stream);

// Per-row transforms for lengths past the chunk kernels' 12288, up to 32768
// (qs_linear_big.hip): work-groups of 16 slices (input) or 16 output chunks
// (output) per row.  big_input_fits also checks the activation dtype (fp16 /
// fp32 rows: n <= 16384).  launch_bx_big writes the pass's operand (x2h, sg,
// xmul) for P.B rows; launch_by_big applies the output transforms of up to
// QS_MAX_GROUP linears (shared rows, output dtype and sign format) from their
// P[g].SG partial groups.
bool big_transform_fits(int64_t len, int p);
bool big_input_fits(int64_t n, int p, int x_dtype);
int launch_bx_big(const BatchedPass& P, hipStream_t stream);
int launch_by_big(const BatchedPass* P, int count, hipStream_t stream);

// Fragment-major fp16 operand of the wide GEMM: row b, columns k .. k + 7 (k
// a multiple of 8) are one 16-byte word, words ordered by [b / 16][k / 256]
// [(k / 8) % 8][(k % 256) / 64][b % 16], so that the 64 lanes of a wave read
// the B operand of one 16 x 16 x 32 MFMA step (16 rows, 32 columns in the
// order the code tiles decode them) as 1 KiB of consecutive bytes.  Rows are
// padded to a multiple of 16.  Returns the element index of (b, k).
__host__ __device__ inline size_t frag_index(int64_t b, int64_t k, int S) {
  const int64_t t = k & 255;
  return (size_t)(((((b >> 4) * S + (k >> 8)) * 8 + ((t >> 3) & 7)) * 64 + (t >> 6) * 16 + (b & 15)) * 8 + (t & 7));
}

// Fragment-major group sums of the same operand, divided by 4: the sums of
// row b over the 8-column groups G .. G + 7 of a 64-column quarter (G a
// multiple of 8) are one 16-byte word, ordered [b / 16][G / 32][(G / 8) % 4]
// [b % 16] -- the B operand of the MFMA that adds the codes' +-1/4 shifts.
// Returns the element index of (b, G).
__host__ __device__ inline size_t sg_frag_index(int64_t b, int64_t G, int S) {
  return (size_t)((((((b >> 4) * S + (G >> 5)) * 4 + ((G >> 3) & 3)) * 16 + (b & 15)) * 8) + (G & 7));
}

// Wide-batch GEMM with the decode in the loop (qs_linear_wide.hip): y1p[g]
// [B][m] = s0 X2 W0^T (+ s1 X2 W1^T) over the g-th of SGk groups of 256-column
// slices, X2 fragment-major.
// Slice groups of the wide GEMM (partial sums summed by the output kernels).
constexpr int kWideMaxGroups = 8;
struct WideMfma {
  const void* codes0;
  const void* codes1;
  int64_t m, n;
  int B;
  float s0, s1;
  const _Float16* x2f;
  const _Float16* sgf;   // group sums / 4, fragment-major
  float* y1p;            // [SGk][B][m]
  int SGk;
};
// Slice groups for (m, n, B): as many as keep the work-groups within one
// round over the CUs (a partial second round costs more than the split
// saves: 11008 x 4096 at 512 rows, 172 tiles, runs 3.7 % faster over the
// step as 1 group than as 2), at most the output kernel's partial-group
// limit.
int wide_splits(int64_t m, int64_t n, int64_t B, int ncu, bool has2);
// Linears of one shape (m, n, B) with one stage above 128 rows whose tiles
// together fit one round over the CUs share one producer / consumer GEMM
// launch (launch_linear_wide_group), with the slice groups chosen for the
// whole group (fewer than each would take alone, so their outputs equal
// separate calls up to the fp32 summation order).  Returns those slice
// groups, or 0 when the linears take one launch each.
int wide_group_splits(int64_t m, int64_t n, int64_t B, int count, int ncu);
int launch_linear_wide_group(const WideMfma* G, int count, hipStream_t stream);
int launch_linear_wide_mfma(const WideMfma& G, hipStream_t stream);


}  // namespace qs
