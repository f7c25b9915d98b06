// Wide-batch quantized-linear forward (prefill: 17 or more activation rows
// per call), the path QuantizedLinear.forward takes for a long prompt
// (quipsharp/checkpoint.py:141-146 -> quipsharp/quantize.py:116-124: the
// reference decodes the whole weight and multiplies densely).  With many
// rows the contraction is a real GEMM: wg_kernel decodes the codes inside
// its K loop (byte LUTs in LDS, exactly as the narrow kernels) and feeds
// every decoded fragment to several 16 x 16 x 32 fp16 MFMAs; the codes' +-1/4
// shifts are one extra MFMA per slice against the operand's group sums.  The
// input and output transforms around it are the per-row kernels of the
// batched path (qs_linear_batched.hip) or, outside the chunk scheme, the
// LDS-radix kernels of qs_linear.hip, writing the fragment-major operand.
#include "qs_forward_dev.h"
#include "qs_linear_dev.h"

namespace qs {
namespace {

constexpr int kDqOffHi = 0;                // 4096 x uint32 LUT entries
constexpr int kDqOffLo = 16384;
constexpr int kDqOffLut1 = 32768;          // 256 x uint4 (E8 1-bit rows, fp16)

// ---------------------------------------------------------------------------
// Decode in the GEMM loop
// ---------------------------------------------------------------------------
// Work-group: 4 waves, 128 weight rows (8 code tiles of 16 rows) x 128
// activation rows; wave w multiplies all 128 weight rows by activation rows
// 32 w .. 32 w + 31 (two 16-row MFMA column tiles), so every decoded A
// fragment feeds two MFMAs (four with a second stage) and every B fragment
// (1 KiB, one coalesced load from the fragment-major operand) eight.  The
// code tiles of a slice are copied into LDS once per work-group (double
// buffered, one barrier per slice); every wave decodes all of them itself
// (VALU work that overlaps the matrix cores) rather than sharing decoded
// fragments through LDS.
constexpr int kWgThreads = 256;
constexpr int kWgRowTiles = 8;     // 16-row code tiles per work-group
constexpr int kWgWaves = kWgThreads / 64;
// 16-row activation tiles per wave (CT): four (64 activation rows per wave,
// 256 per work-group) for wide batches, two with a second stage (whose
// accumulators take the registers), and fewer for short batches so that no
// wave multiplies tiles past the last row.  Wave w of work-group column ct
// takes tiles 4 CT ct + w + 4 t, t < CT.
inline int wg_ct(int64_t B, bool has2) {
  const int64_t nbt = (B + 15) / 16;
  const int ct = nbt <= kWgWaves ? 1 : nbt <= 2 * kWgWaves ? 2 : 4;
  return has2 && ct > 2 ? 2 : ct;
}
constexpr int kWgRows = 16 * kWgRowTiles;
constexpr int kWgCodeBuf = kWgRowTiles * 1024;           // code bytes of one slice
constexpr int kWgOffCodes = kDqOffLut1 + 4096;           // 2 slices (the table staging before them)
constexpr int kWgOffCodes1 = kWgOffCodes + 2 * kWgCodeBuf;  // 2 slices of second-stage bytes
constexpr int kWgLds = kWgOffCodes1 + kWgCodeBuf;
constexpr int kWgRing = 4;         // B fragments in flight per wave (steps of 32 columns)
constexpr int kWgAhead = 3;        // steps between a B load and its use
static_assert(kWgLds <= 65536, "LDS budget");
constexpr int kWgCopies = kWgCodeBuf / (16 * kWgThreads);  // 16-byte code copies per thread and slice
static_assert(kWgCopies >= 1 && kWgCopies <= 2 && kWgCopies * 16 * kWgThreads == kWgCodeBuf, "code copy");
static_assert(kWgThreads >= 256 && kFwdThreads % kWgThreads == 0, "table staging and LUT fill");

struct WgArgs {
  const uint16_t* codes0;
  const uint8_t* codes1;
  const _Float16* x2f;
  const _Float16* sgf;
  float* y1p;
  int m, B, S, RB;     // RB: 16-row blocks
  int nrt, nct;        // work-group tiles along the weight rows / activation rows
  int SGk, spg;        // slice groups, slices per group
  float s0, s1;
};

template <bool HAS2, int kWgColTiles>
__global__ __launch_bounds__(kWgThreads) void wg_kernel(WgArgs A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint32_t* lut_hi = reinterpret_cast<uint32_t*>(lds + kDqOffHi);
  uint32_t* lut_lo = reinterpret_cast<uint32_t*>(lds + kDqOffLo);
  uint4* lut1 = reinterpret_cast<uint4*>(lds + kDqOffLut1);
  uint4* tab16 = reinterpret_cast<uint4*>(lds + kWgOffCodes);  // staging, before the first code tiles
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15;

  // Tiles are ordered weight-row tiles fastest, then activation tiles, then
  // slice groups, and dealt to the XCDs in contiguous runs: work-group i runs
  // on XCD i % 8, so tile (i % 8) * ceil(T / 8) + i / 8 keeps each XCD's L2 on
  // a few activation columns and slice groups (the grid is rounded up to a
  // multiple of 8; the surplus work-groups exit at once).
  const int T = A.nrt * A.nct * A.SGk;
  const int per = (T + 7) >> 3;
  int bid = ((int)blockIdx.x & 7) * per + ((int)blockIdx.x >> 3);
  if (bid >= T) return;
  const int rt = bid % A.nrt;
  bid /= A.nrt;
  const int ct = bid % A.nct;
  const int g = bid / A.nct;
  const int s_begin = g * A.spg;
  const int s_end = s_begin + A.spg < A.S ? s_begin + A.spg : A.S;
  const int s_last = s_end > s_begin ? s_end - 1 : (A.S - 1);  // an empty group reads, never uses, slice S - 1

  // Global bytes of a slice's code tiles: thread tid copies bytes 16 tid
  // (and 16 tid + 16 kWgThreads) of the 8 KiB (tile = byte / 1024), threads
  // below 256 byte 16 tid of the 4 KiB second stage (tile = byte / 512).  Row
  // blocks past the end read the last one (decoded, never stored).
  auto tile_of = [&](int i, int s) -> size_t {
    int rb = rt * kWgRowTiles + i;
    rb = rb < A.RB ? rb : A.RB - 1;
    s = s < s_last ? s : s_last;
    return (size_t)rb * A.S + s;
  };
  struct CodeCopy {
    uint4 c0, c1, c2;  // bytes 16 tid, 16 (tid + kWgThreads) of the codes; 16 tid of the second stage
  };
  auto load_codes = [&](int s) -> CodeCopy {
    CodeCopy r;
    const int b0 = 16 * tid, b1 = 16 * (tid + kWgThreads);
    const char* c0 = reinterpret_cast<const char*>(A.codes0);
    r.c0 = *reinterpret_cast<const uint4*>(c0 + tile_of(b0 >> 10, s) * 1024 + (b0 & 1023));
    r.c1 = kWgCopies > 1 ? *reinterpret_cast<const uint4*>(c0 + tile_of(b1 >> 10, s) * 1024 + (b1 & 1023))
                         : make_uint4(0, 0, 0, 0);
    r.c2 = HAS2 && tid < 256
               ? *reinterpret_cast<const uint4*>(A.codes1 + tile_of(b0 >> 9, s) * 512 + (b0 & 511))
               : make_uint4(0, 0, 0, 0);
    return r;
  };
  auto store_codes = [&](int p, const CodeCopy& r) {
    *reinterpret_cast<uint4*>(lds + kWgOffCodes + p * kWgCodeBuf + 16 * tid) = r.c0;
    if (kWgCopies > 1) *reinterpret_cast<uint4*>(lds + kWgOffCodes + p * kWgCodeBuf + 16 * (tid + kWgThreads)) = r.c1;
    if (HAS2 && tid < 256) *reinterpret_cast<uint4*>(lds + kWgOffCodes1 + p * (kWgCodeBuf / 2) + 16 * tid) = r.c2;
  };

  // activation tiles of this wave (clamped to the last one: computed, never stored)
  const int nbt = (A.B + 15) >> 4;
  const _Float16* xb[kWgColTiles];
  const _Float16* sb[kWgColTiles];
#pragma unroll
  for (int t = 0; t < kWgColTiles; ++t) {
    int c = kWgWaves * kWgColTiles * ct + w + kWgWaves * t;
    c = c < nbt ? c : nbt - 1;
    xb[t] = A.x2f + (size_t)c * A.S * 8 * 512 + 8 * lane;  // + (s * 8 + step) * 512 halves
    sb[t] = A.sgf + (size_t)c * A.S * 512 + 8 * lane;      // + s * 512 halves
  }
  half8 bring[kWgRing][kWgColTiles];
  auto load_b = [&](int s, int step, half8 (&dst)[kWgColTiles]) {
    s = s < s_last ? s : s_last;
#pragma unroll
    for (int t = 0; t < kWgColTiles; ++t)
      dst[t] = *reinterpret_cast<const half8*>(xb[t] + ((size_t)s * 8 + step) * 512);
  };

  // a wave with no activation tile of its own only helps copy the codes
  // (with four tiles per wave, chosen for long batches, every wave but those
  // of a ragged last column has work: no branch)
  const bool wave_on = kWgColTiles == 4 || kWgWaves * kWgColTiles * ct + w < nbt;
  CodeCopy gc = load_codes(s_begin);
  if (wave_on) {
#pragma unroll
    for (int k = 0; k < kWgAhead; ++k) load_b(s_begin, k, bring[k]);
  }
  if (tid < 256) {
    tab16[tid] = *reinterpret_cast<const uint4*>(kE8Ph.w[tid]);
    if (HAS2) lut1[tid] = *reinterpret_cast<const uint4*>(kE81h.w[tid]);
  }
  __syncthreads();
#pragma unroll
  for (int r = 0; r < kFwdThreads / kWgThreads; ++r) fill_luts(tab16, lut_hi, lut_lo, tid + kWgThreads * r);
  __syncthreads();
  store_codes(0, gc);
  __syncthreads();

  floatx4 acc[kWgRowTiles][kWgColTiles];
  floatx4 acc2[kWgRowTiles][kWgColTiles];
#pragma unroll
  for (int i = 0; i < kWgRowTiles; ++i)
#pragma unroll
    for (int t = 0; t < kWgColTiles; ++t) {
      acc[i][t] = floatx4{0.f, 0.f, 0.f, 0.f};
      acc2[i][t] = floatx4{0.f, 0.f, 0.f, 0.f};
    }

  for (int s = s_begin; s < s_end; ++s) {
    const int p = (s - s_begin) & 1;
    uint4 cw[kWgRowTiles];
    uint2 cw1[kWgRowTiles];
#pragma unroll
    for (int i = 0; i < kWgRowTiles; ++i) {
      cw[i] = *reinterpret_cast<const uint4*>(lds + kWgOffCodes + p * kWgCodeBuf + 1024 * i + 16 * lane);
      if (HAS2)
        cw1[i] = *reinterpret_cast<const uint2*>(lds + kWgOffCodes1 + p * (kWgCodeBuf / 2) + 512 * i + 8 * lane);
    }
    gc = load_codes(s + 1);  // the next slice's tiles, stored after this slice
    if (wave_on) {
    half8 sgs[kWgColTiles];  // group sums / 4 of this slice, used after its 8 steps
#pragma unroll
    for (int t = 0; t < kWgColTiles; ++t) sgs[t] = *reinterpret_cast<const half8*>(sb[t] + (size_t)s * 512);

    auto word = [&](int i, int c) -> uint32_t {
      return c < 2 ? cw[i].x : c < 4 ? cw[i].y : c < 6 ? cw[i].z : cw[i].w;
    };
    // LUT words of step c + 1 are read while the MFMAs of step c run, and the
    // fp16 A fragments of step c + 1 are built between them, so neither the
    // LDS latency nor the decode VALU work stalls the matrix cores.
    uint32_t hv[kWgRowTiles], lv[kWgRowTiles];
    half8 l1[2][kWgRowTiles];
    auto read_luts = [&](int c) {
#pragma unroll
      for (int i = 0; i < kWgRowTiles; ++i) {
        const uint32_t v = word(i, c);
        const uint32_t ha = (c & 1) ? ((v >> 18) & 0x3FFCu) : ((v >> 2) & 0x3FFCu);
        const uint32_t la = (c & 1) ? ((v >> 15) & 0x3FFCu) : ((v << 1) & 0x3FFCu);
        hv[i] = lds_word(kDqOffHi + ha);
        lv[i] = lds_word(kDqOffLo + la);
        if (HAS2) {
          const uint32_t idx = ((c < 4 ? cw1[i].x : cw1[i].y) >> (8 * (c & 3))) & 0xFFu;
          l1[c & 1][i] = __builtin_bit_cast(half8, lut1[idx]);
        }
      }
    };
    // E8P value +-(k + 1/2); the code's +-1/4 shift is added per slice below
    auto build = [&](int i, int c) -> half8 {
      return __builtin_bit_cast(half8, make_uint4(lut_pair_lo(hv[i]), lut_pair_hi(hv[i]), lut_pair_lo(lv[i]),
                                                  lut_pair_hi(lv[i])));
    };
    half8 a[2][kWgRowTiles];
    read_luts(0);
#pragma unroll
    for (int i = 0; i < kWgRowTiles; ++i) a[0][i] = build(i, 0);
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      // B fragments of step c + kWgAhead (into the ring slot step c - 1 freed)
      {
        const int cn = c + kWgAhead;
        load_b(cn < 8 ? s : s + 1, cn & 7, bring[cn % kWgRing]);
      }
      if (c < 7) read_luts(c + 1);
      const half8(&bf)[kWgColTiles] = bring[c % kWgRing];
#pragma unroll
      for (int i = 0; i < kWgRowTiles; ++i) {
#pragma unroll
        for (int t = 0; t < kWgColTiles; ++t)
          acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[c & 1][i], bf[t], acc[i][t], 0, 0, 0);
        if (HAS2) {
#pragma unroll
          for (int t = 0; t < kWgColTiles; ++t)
            acc2[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(l1[c & 1][i], bf[t], acc2[i][t], 0, 0, 0);
        }
        if (c < 7) a[(c + 1) & 1][i] = build(i, c + 1);
      }
    }
    // shifts: +-1 per code (its shift bit) times the group sums / 4 -- one
    // MFMA per tile pair for the slice's 8 steps
#pragma unroll
    for (int i = 0; i < kWgRowTiles; ++i) {
      const uint32_t wd[4] = {cw[i].x, cw[i].y, cw[i].z, cw[i].w};
      uint32_t sh[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) sh[k] = 0xBC00BC00u ^ ((wd[k] & 0x10001u) * 0x8000u);
      const half8 so = __builtin_bit_cast(half8, make_uint4(sh[0], sh[1], sh[2], sh[3]));
#pragma unroll
      for (int t = 0; t < kWgColTiles; ++t)
        acc[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(so, sgs[t], acc[i][t], 0, 0, 0);
    }
    }  // wave_on
    store_codes(p ^ 1, gc);
    __syncthreads();
  }

  // lane (q, r16) holds weight rows 4 q .. 4 q + 3 of tile i for activation
  // row r16 of tile t: four consecutive outputs
#pragma unroll
  for (int t = 0; t < kWgColTiles; ++t) {
    const int b = (kWgWaves * kWgColTiles * ct + w + kWgWaves * t) * 16 + r16;
    if (b >= A.B) continue;
    float* yrow = A.y1p + ((size_t)g * A.B + b) * A.m;
#pragma unroll
    for (int i = 0; i < kWgRowTiles; ++i) {
      const int rb = rt * kWgRowTiles + i;
      if (rb >= A.RB) continue;
      floatx4 v;
#pragma unroll
      for (int j = 0; j < 4; ++j) v[j] = HAS2 ? A.s0 * acc[i][t][j] + A.s1 * acc2[i][t][j] : A.s0 * acc[i][t][j];
      *reinterpret_cast<floatx4*>(yrow + rb * 16 + 4 * q) = v;
    }
  }
}

template <bool HAS2, int CT>
int launch_wg(const WgArgs& A, unsigned grid, hipStream_t stream) {
  static int done = 0;
  if (!done) {
    hipFuncAttributes fa{};
    QS_HIP(hipFuncGetAttributes(&fa, (const void*)wg_kernel<HAS2, CT>));
    QS_REQUIRE(fa.sharedSizeBytes == 0, "wg_kernel must not use static LDS");
    done = 1;
  }
  hipLaunchKernelGGL((wg_kernel<HAS2, CT>), dim3(grid), dim3(kWgThreads), kWgLds, stream, A);
  QS_LAUNCHED("wg_kernel");
  return QS_OK;
}


}  // namespace

int wide_splits(int64_t m, int64_t n, int64_t B, int ncu, bool has2) {
  const int64_t cols = 16 * kWgWaves * wg_ct(B, has2);
  const int64_t tiles = ((m / 16 + kWgRowTiles - 1) / kWgRowTiles) * ((B + cols - 1) / cols);
  const int64_t S = n / 256;
  int64_t g = 1;
  while (g < kWideMaxGroups && g < S && tiles * g < ncu) ++g;
  return (int)g;
}

int launch_linear_wide_mfma(const WideMfma& G, hipStream_t stream) {
  QS_REQUIRE(G.m % 16 == 0 && G.n % 256 == 0 && G.B >= 1, "wide GEMM: m %% 16, n %% 256");
  QS_REQUIRE(G.SGk >= 1 && G.SGk <= kWideMaxGroups, "wide GEMM: 1..%d slice groups", kWideMaxGroups);
  QS_REQUIRE(G.m * G.n / 4 < ((int64_t)1 << 40), "wide GEMM: codes too large");
  const bool has2 = G.codes1 != nullptr;
  const int CT = wg_ct(G.B, has2);
  WgArgs A{};
  A.codes0 = static_cast<const uint16_t*>(G.codes0);
  A.codes1 = static_cast<const uint8_t*>(G.codes1);
  A.x2f = G.x2f;
  A.sgf = G.sgf;
  A.y1p = G.y1p;
  A.m = (int)G.m;
  A.B = G.B;
  A.S = (int)(G.n / 256);
  A.RB = (int)(G.m / 16);
  A.nrt = (A.RB + kWgRowTiles - 1) / kWgRowTiles;
  A.nct = (G.B + 16 * kWgWaves * CT - 1) / (16 * kWgWaves * CT);
  A.SGk = G.SGk;
  A.spg = (A.S + G.SGk - 1) / G.SGk;
  A.s0 = G.s0;
  A.s1 = G.s1;
  const int64_t tiles = (int64_t)A.nrt * A.nct * A.SGk;
  QS_REQUIRE(tiles < ((int64_t)1 << 30), "wide GEMM: grid too large");
  const int64_t grid = (tiles + 7) / 8 * 8;  // XCD-contiguous tile order (see wg_kernel)
  const unsigned g = (unsigned)grid;
  if (has2) return CT == 1 ? launch_wg<true, 1>(A, g, stream) : launch_wg<true, 2>(A, g, stream);
  return CT == 1 ? launch_wg<false, 1>(A, g, stream)
                 : CT == 2 ? launch_wg<false, 2>(A, g, stream) : launch_wg<false, 4>(A, g, stream);
}

}  // namespace qs
