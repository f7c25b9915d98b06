// Workspace indices of the forward kernels' partial sums and of the
// operands their output transforms poll, and the sizes of the regions that
// hold them.  The kernels (qs_forward_dev.h, qs_linear_fused.hip,
// qs_linear_batched.hip, qs_linear_big.hip) and the workspace layout
// (qs_linear.hip) call these functions, and a host check compiled without HIP
// enumerates them under the kernels' guards against the region sizes.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "qs_tags.h"  // QS_HD

namespace qs {

// Partial sums (fp32, or tagged 64-bit slots) laid out [SG][B][m]: slice
// group g, batch row b of B, output element e.
QS_HD inline size_t partial_index(int g, int B, int b, int m, int e) { return ((size_t)g * B + b) * m + e; }

// Output element t = lane + 64 j of the 256-element chunk c (the layout in
// which the polls and partial-sum loads hold a chunk: each load of a wave
// reads 64 consecutive elements).
QS_HD inline int chunk_elem(int c, int lane, int j) { return 256 * c + lane + 64 * j; }

// Output element `row` of the 16-row block rb (the reduction stores of the
// decode loops).
QS_HD inline int block_elem(int rb, int row) { return 16 * rb + row; }

// Chunk transforms of the two-level output transform, laid out [B][m]:
// batch row b, output element e.
QS_HD inline size_t h2_index(int b, int m, int e) { return (size_t)b * m + e; }

// Column 16 g + tt of chunk c (the level-2 polls: column group g < 16).
QS_HD inline int column_elem(int c, int g, int tt) { return 256 * c + 16 * g + tt; }

// Output element of output-stage row r (the chunk) and column t < 256.
QS_HD inline int out_elem(int r, int t) { return 256 * r + t; }

// Region sizes, in slots: the one-launch kernel's tagged partial sums (up to
// two rows) and its chunk transforms, and the 16-row decode-matvec's tagged
// partial sums.
QS_HD inline size_t fused_slot_count(int SG, int64_t m) { return (size_t)SG * 2 * (size_t)m; }
QS_HD inline size_t h2_slot_count(int64_t m) { return (size_t)2 * (size_t)m; }
QS_HD inline size_t batched_slot_count(int SG, int64_t B, int64_t m) { return (size_t)SG * (size_t)B * (size_t)m; }

}  // namespace qs
