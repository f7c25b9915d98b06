// Wide-batch quantized-linear forward (prefill: 17 or more activation rows
// per call), the path QuantizedLinear.forward takes for a long prompt
// (quipsharp/checkpoint.py:141-146 -> quipsharp/quantize.py:116-124: the
// reference decodes the whole weight and multiplies densely).  With many
// rows the contraction is a real GEMM: wg_kernel decodes the codes inside
// its K loop (byte LUTs in LDS, exactly as the narrow kernels) and feeds
// every decoded fragment to several 16 x 16 x 32 fp16 MFMAs; the codes' +-1/4
// shifts are one extra MFMA per slice against the operand's group sums.
// Single-stage calls of more than 128 rows take wp_kernel instead, which
// splits decoding and multiplying between the waves of a work-group.  The
// input and output transforms around it are the per-row kernels of the
// batched path (qs_linear_batched.hip) or, outside the chunk scheme, the
// LDS-radix kernels of qs_linear.hip, writing the fragment-major operand.
#include <type_traits>

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
constexpr int kWgOffCodes = kDqOffLut1 + 4096;           // 2 slices
constexpr int kWgOffCodes1 = kWgOffCodes + 2 * kWgCodeBuf;  // 2 slices of second-stage bytes
constexpr int kWgLds = kWgOffCodes1 + kWgCodeBuf;
constexpr int kWgRing = 4;         // B fragments in flight per wave (steps of 32 columns)
constexpr int kWgAhead = 3;        // steps between a B load and its use
static_assert(kWgLds <= 65536, "LDS budget");
constexpr int kWgCopies = kWgCodeBuf / (16 * kWgThreads);  // 16-byte code copies per thread and slice
static_assert(kWgCopies >= 1 && kWgCopies <= 2 && kWgCopies * 16 * kWgThreads == kWgCodeBuf, "code copy");
static_assert(kWgThreads >= 256, "E8 one-bit table rows: one per thread of the first 256");

// One linear of a wp_kernel launch: linears of one shape (m, n, rows) that
// read their own operands share a launch, job j taking tiles j T1 .. (j + 1)
// T1 - 1 of the grid's tile order (T1 = nrt nct SGk).
struct WpJob {
  const uint16_t* codes0;
  const _Float16* x2f;
  float* y1p;
  float s0;
};

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
  int njobs;           // wp_kernel: linears of the launch (job[0]: the fields above)
  WpJob job[QS_MAX_GROUP];
};

template <bool HAS2, int kWgColTiles>
__global__ __launch_bounds__(kWgThreads) void wg_kernel(WgArgs A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint4* lut1 = reinterpret_cast<uint4*>(lds + kDqOffLut1);
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
    r.c0 = ld_nt_u4(c0 + tile_of(b0 >> 10, s) * 1024 + (b0 & 1023));
    r.c1 = kWgCopies > 1 ? ld_nt_u4(c0 + tile_of(b1 >> 10, s) * 1024 + (b1 & 1023)) : make_uint4(0, 0, 0, 0);
    r.c2 = HAS2 && tid < 256 ? ld_nt_u4(A.codes1 + tile_of(b0 >> 9, s) * 512 + (b0 & 511)) : make_uint4(0, 0, 0, 0);
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
  {
    LutCopy<kWgThreads> lc;
    load_luts(tid, lc);
    uint4 t1 = make_uint4(0, 0, 0, 0);
    if (HAS2 && tid < 256) t1 = *reinterpret_cast<const uint4*>(kE81h.w[tid]);
    store_luts(lds, tid, lc);
    if (HAS2 && tid < 256) lut1[tid] = t1;
  }
  store_codes(0, gc);
  __syncthreads();  // LUTs and the first slice's code tiles complete

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


// ---------------------------------------------------------------------------
// Producer / consumer variant for long single-stage batches
// ---------------------------------------------------------------------------
// The wave that feeds the matrix cores should issue nothing but MFMAs and
// their operand loads: VALU work issued by that wave is not hidden behind its
// MFMAs.  So a work-group of 8 waves splits the roles, one of each per SIMD:
// decode waves 4..7 turn the codes of 32 weight rows each into fp16 A
// fragments (E8P value plus the code's +-1/4 shift, exact in fp16) in the
// 32x32x16 MFMA layout, one half slice (128 columns) at a time into a double
// buffer in LDS; MFMA waves 0..3 each multiply all 128 weight rows by 64
// activation rows with v_mfma_f32_32x32x16_f16 (4 x 2 accumulator tiles),
// reading the A fragments from LDS and the B fragments from the
// fragment-major operand through a register ring.  One barrier per half
// slice hands the buffers over.  The tile order, slice groups and partial
// sums are wg_kernel's (with 256 activation rows per work-group).
//
// A fragment (R, k) of a half slice (R: 32-row weight tile, k: 16-column
// step) is 64 lanes x 8 fp16: lane l holds row 32 R + l % 32, columns
// 16 k + 8 (l / 32) .. + 7, i.e. one code.  Code (tile i, lane (q, r16),
// step c = 4 h + cc) of the packed layout holds row 16 i + r16, columns
// 32 c + 8 q: fragment (i / 2, 2 cc + q / 2), lane 16 (i % 2) + r16 + 32 (q % 2).
constexpr int kWpThreads = 512;
constexpr int kWpMfmaWaves = 4;
constexpr int kWpOffA = 32768;                  // after the byte LUTs
constexpr int kWpABuf = 32 * 1024;              // 4 x 8 fragments of 1 KiB
constexpr int kWpLds = kWpOffA + 2 * kWpABuf;
constexpr int kWpRing = 8;                      // B fragment steps in flight per MFMA wave (one half slice)
static_assert(kWpLds <= 160 * 1024, "LDS budget");
static_assert(kWpMfmaWaves * 32 * 528 <= kWpLds, "output staging fits");
typedef float floatx16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(kWpThreads) void wp_kernel(WgArgs A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);

  // tile order as wg_kernel (XCD-contiguous runs), job after job
  const int T1 = A.nrt * A.nct * A.SGk;
  const int T = A.njobs * T1;
  const int per = (T + 7) >> 3;
  int bid = ((int)blockIdx.x & 7) * per + ((int)blockIdx.x >> 3);
  if (bid >= T) return;
  int jj = 0;
#pragma unroll
  for (int k = 1; k < QS_MAX_GROUP; ++k)
    if (k < A.njobs && bid >= k * T1) jj = k;
  const WpJob& J = A.job[jj];
  bid -= jj * T1;
  const int rt = bid % A.nrt;
  bid /= A.nrt;
  const int ct = bid % A.nct;
  const int g = bid / A.nct;
  const int s_begin = g * A.spg;
  const int s_end = s_begin + A.spg < A.S ? s_begin + A.spg : A.S;
  const int s_last = s_end > s_begin ? s_end - 1 : (A.S - 1);

  // every wave issues its first global loads (code words, B fragments), then
  // copies its share of the LUTs into LDS
  auto build_luts = [&]() {
    LutCopy<kWpThreads> lc;
    load_luts(tid, lc);
    store_luts(lds, tid, lc);
    __syncthreads();  // LUTs complete
  };

  const int nsl = s_end > s_begin ? s_end - s_begin : 0;  // slices of this work-group
  using H0 = std::integral_constant<int, 0>;
  using H1 = std::integral_constant<int, 1>;
  if (w >= kWpMfmaWaves) {
    // ---------------- decode waves ----------------
    const int d = w - kWpMfmaWaves;  // weight rows 32 d .. 32 d + 31: code tiles 2 d, 2 d + 1
    const int q = lane >> 4, r16 = lane & 15;
    // code words are read once per work-group (nontemporal loads)
    auto words = [&](int ii, int s) -> uint4 {
      int rb = rt * 8 + 2 * d + ii;
      rb = rb < A.RB ? rb : A.RB - 1;  // past the end: the last row block (decoded, never stored)
      s = s < s_last ? s : s_last;
      return ld_nt_u4(reinterpret_cast<const char*>(J.codes0) + ((size_t)rb * A.S + s) * 1024 + 16 * lane);
    };
    // half h of the slice whose code words are c0 / c1 into buffer h
    auto decode_half = [&](auto hc, const uint4& c0, const uint4& c1) {
      constexpr int h = decltype(hc)::value;
      char* buf = lds + kWpOffA + h * kWpABuf;
#pragma unroll
      for (int ii = 0; ii < 2; ++ii) {
        const uint4& cw = ii ? c1 : c0;
        // the two code words of steps 4 h .. 4 h + 3
        const uint32_t wd[2] = {h ? cw.z : cw.x, h ? cw.w : cw.y};
        uint32_t hv[4], lv[4];
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) code_lut_words(wd[cc >> 1], cc & 1, kDqOffHi, kDqOffLo, hv[cc], lv[cc]);
#pragma unroll
        for (int cc = 0; cc < 4; ++cc) {
          const uint32_t sh = (wd[cc >> 1] >> (16 * (cc & 1))) & 1u;  // shift bit: +1/4 set, -1/4 clear
          half8 v = code_operand(hv[cc], lv[cc]);
          v = v + (sh ? (_Float16)0.25f : (_Float16)-0.25f);
          const int kk = 2 * cc + (q >> 1);
          const int l = 16 * ii + r16 + 32 * (q & 1);
          *reinterpret_cast<half8*>(buf + ((d * 8 + kk) * 64 + l) * 16) = v;
        }
      }
    };
    uint4 c0 = words(0, s_begin), c1 = words(1, s_begin);
    build_luts();
    if (nsl > 0) decode_half(H0{}, c0, c1);
    __syncthreads();
    for (int sl = 0; sl < nsl; ++sl) {
      const uint4 n0 = words(0, s_begin + sl + 1), n1 = words(1, s_begin + sl + 1);  // next slice, in flight
      decode_half(H1{}, c0, c1);  // while the MFMA waves take half 0
      __syncthreads();
      c0 = n0;
      c1 = n1;
      if (sl + 1 < nsl) decode_half(H0{}, c0, c1);  // while they take half 1
      __syncthreads();
    }
    return;
  }

  // ---------------- MFMA waves ----------------
  const int nbt = (A.B + 15) >> 4;  // 16-row fragments of the operand
  const int row0 = (kWpMfmaWaves * ct + w) * 64;  // this wave's activation rows row0 .. row0 + 63
  // B fragment (t, slice s, half h, step k): lane l reads activation row row0 + 32 t + l % 32,
  // columns 128 h + 16 k + 8 (l / 32) of the slice; fragment-major operand: 16-row fragment
  // c16, 32-column step st of slice s at ((c16 S + s) 8 + st) 512 halves, lane' = q' 16 + r16'
  // at 8 lane' halves, q' = 2 (k % 2) + l / 32
  const _Float16* xrow[2];
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const int r = row0 + 32 * t + (lane & 31);
    int c16 = r >> 4;
    c16 = c16 < nbt ? c16 : nbt - 1;  // rows past the batch: computed, never stored
    xrow[t] = J.x2f + (size_t)c16 * A.S * 8 * 512 + 8 * ((lane >> 5) * 16 + (r & 15));
  }
  // slices past the work-group's last are clamped to it: those loads are in
  // bounds and never used, so every load is unconditional
  auto load_b = [&](int s, int h, int k, half8 (&dst)[2]) {
    s = s < s_last ? s : s_last;
    const size_t off = ((size_t)s * 8 + 4 * h + (k >> 1)) * 512 + 8 * 16 * 2 * (k & 1);
#pragma unroll
    for (int t = 0; t < 2; ++t) dst[t] = *reinterpret_cast<const half8*>(xrow[t] + off);
  };
  auto a_frag = [&](int h, int R, int k) {
    return *reinterpret_cast<const half8*>(lds + kWpOffA + h * kWpABuf + ((R * 8 + k) * 64 + lane) * 16);
  };
  floatx16 acc[4][2];
#pragma unroll
  for (int R = 0; R < 4; ++R)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc[R][t] = floatx16{};
  // ring entry k holds step k of the half slice being multiplied; step k of
  // the next half slice (slice sn, half hn) replaces it once its MFMAs are
  // issued, one half slice of MFMAs ahead of its use.  The scheduling
  // barriers keep that order (and the ring in the same registers across the
  // loop): each step reads the next step's A fragments from LDS, issues its
  // 8 MFMAs, then its 2 ring loads.
  half8 ring[kWpRing][2];
  auto mfma_half = [&](auto hc, int sn, int hn) {
    constexpr int h = decltype(hc)::value;
    half8 a[2][4];
#pragma unroll
    for (int R = 0; R < 4; ++R) a[0][R] = a_frag(h, R, 0);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (k < 7) {
#pragma unroll
        for (int R = 0; R < 4; ++R) a[(k + 1) & 1][R] = a_frag(h, R, k + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int R = 0; R < 4; ++R)
#pragma unroll
        for (int t = 0; t < 2; ++t)
          acc[R][t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[k & 1][R], ring[k][t], acc[R][t], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      load_b(sn, hn, k, ring[k]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  const bool wave_on = row0 < A.B;
  if (wave_on) {
#pragma unroll
    for (int k = 0; k < kWpRing; ++k) {
      load_b(s_begin, 0, k, ring[k]);  // in the order the loop issues them
      __builtin_amdgcn_sched_barrier(0);
    }
    build_luts();
    __syncthreads();  // the first half slice's fragments are in buffer 0
    for (int sl = 0; sl < nsl; ++sl) {
      const int s = s_begin + sl;
      mfma_half(H0{}, s, 1);
      __syncthreads();  // buffer 0 free; half 1 complete
      mfma_half(H1{}, s + 1, 0);
      __syncthreads();  // buffer 1 free; the next slice's half 0 complete
    }
  } else {
    // no activation rows: only the barriers that hand the buffers over
    build_luts();
    __syncthreads();
    for (int sl = 0; sl < nsl; ++sl) {
      __syncthreads();
      __syncthreads();
    }
    return;
  }
  // lane l, accumulator v of tile (R, t): weight row 32 R + 8 (v / 4) + 4 (l / 32) + v % 4,
  // activation row row0 + 32 t + l % 32; four consecutive weight rows per float4.
  // The tiles go out through LDS (each MFMA wave its own 32 x 528-byte area
  // in the LUT and fragment space, free after the last barrier), so that each
  // store instruction writes two activation rows' 512 contiguous bytes
  // instead of 32 rows' 32 bytes (2 % of the 512-row step).
  char* stg = lds + w * (32 * 528);
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int R = 0; R < 4; ++R)
#pragma unroll
      for (int vg = 0; vg < 4; ++vg) {
        floatx4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = J.s0 * acc[R][t][4 * vg + e];
        *reinterpret_cast<floatx4*>(stg + (lane & 31) * 528 + (32 * R + 8 * vg + 4 * (lane >> 5)) * 4) = v;
      }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
    const int row = rt * 128 + 4 * (lane & 31);
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      const int r = 2 * k + (lane >> 5);
      const int b = row0 + 32 * t + r;
      const floatx4 v = *reinterpret_cast<const floatx4*>(stg + r * 528 + (lane & 31) * 16);
      if (b < A.B && row < A.m) *reinterpret_cast<floatx4*>(J.y1p + ((size_t)g * A.B + b) * A.m + row) = v;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);
    __builtin_amdgcn_wave_barrier();
  }
}

int launch_wp(const WgArgs& A, unsigned grid, hipStream_t stream) {
  static int done = 0;
  if (!done) {
    hipFuncAttributes fa{};
    QS_HIP(hipFuncGetAttributes(&fa, (const void*)wp_kernel));
    QS_REQUIRE(fa.sharedSizeBytes == 0, "wp_kernel must not use static LDS");
    QS_HIP(hipFuncSetAttribute((const void*)wp_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, kWpLds));
    done = 1;
  }
  hipLaunchKernelGGL(wp_kernel, dim3(grid), dim3(kWpThreads), kWpLds, stream, A);
  QS_LAUNCHED("wp_kernel");
  return QS_OK;
}

}  // namespace

int wide_splits(int64_t m, int64_t n, int64_t B, int ncu, bool has2) {
  const int64_t cols = 16 * kWgWaves * wg_ct(B, has2);
  const int64_t tiles = ((m / 16 + kWgRowTiles - 1) / kWgRowTiles) * ((B + cols - 1) / cols);
  const int64_t S = n / 256;
  int64_t g = 1;  // as many groups as fit in one round of work-groups
  while (g < kWideMaxGroups && g < S && tiles * (g + 1) <= ncu) ++g;
  return (int)g;
}

int wide_group_splits(int64_t m, int64_t n, int64_t B, int count, int ncu) {
  if (count < 2 || wg_ct(B, false) != 4) return 0;
  const int64_t cols = 16 * kWgWaves * 4;
  const int64_t tiles = ((m / 16 + kWgRowTiles - 1) / kWgRowTiles) * ((B + cols - 1) / cols) * count;
  if (tiles > ncu) return 0;
  const int64_t S = n / 256;
  int64_t g = 1;
  while (g < kWideMaxGroups && g < S && tiles * (g + 1) <= ncu) ++g;
  return (int)g;
}

namespace {
WgArgs wide_args(const WideMfma& G) {
  const int CT = wg_ct(G.B, G.codes1 != nullptr);
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
  A.njobs = 1;
  A.job[0] = WpJob{A.codes0, A.x2f, A.y1p, A.s0};
  return A;
}
int check_wide(const WideMfma& G) {
  QS_REQUIRE(G.m % 16 == 0 && G.n % 256 == 0 && G.B >= 1, "wide GEMM: m %% 16, n %% 256");
  QS_REQUIRE(G.SGk >= 1 && G.SGk <= kWideMaxGroups, "wide GEMM: 1..%d slice groups", kWideMaxGroups);
  QS_REQUIRE(G.m * G.n / 4 < ((int64_t)1 << 40), "wide GEMM: codes too large");
  return QS_OK;
}
}  // namespace

int launch_linear_wide_mfma(const WideMfma& G, hipStream_t stream) {
  int rc = check_wide(G);
  if (rc) return rc;
  const bool has2 = G.codes1 != nullptr;
  const int CT = wg_ct(G.B, has2);
  const WgArgs A = wide_args(G);
  const int64_t tiles = (int64_t)A.nrt * A.nct * A.SGk;
  QS_REQUIRE(tiles < ((int64_t)1 << 30), "wide GEMM: grid too large");
  const int64_t grid = (tiles + 7) / 8 * 8;  // XCD-contiguous tile order (see wg_kernel)
  const unsigned g = (unsigned)grid;
  if (has2) return CT == 1 ? launch_wg<true, 1>(A, g, stream) : launch_wg<true, 2>(A, g, stream);
  if (CT == 4) return launch_wp(A, g, stream);  // 256 activation rows per work-group, as wp_kernel's
  return CT == 1 ? launch_wg<false, 1>(A, g, stream)
                 : CT == 2 ? launch_wg<false, 2>(A, g, stream) : launch_wg<false, 4>(A, g, stream);
}

int launch_linear_wide_group(const WideMfma* G, int count, hipStream_t stream) {
  QS_REQUIRE(count >= 1 && count <= QS_MAX_GROUP, "wide GEMM group: 1..%d linears", QS_MAX_GROUP);
  for (int j = 0; j < count; ++j) {
    const int rc = check_wide(G[j]);
    if (rc) return rc;
    QS_REQUIRE(G[j].m == G[0].m && G[j].n == G[0].n && G[j].B == G[0].B && G[j].SGk == G[0].SGk &&
                   G[j].codes1 == nullptr && wg_ct(G[j].B, false) == 4,
               "wide GEMM group: one shape, one stage, more than %d rows", 16 * kWgWaves * 2);
  }
  WgArgs A = wide_args(G[0]);
  A.njobs = count;
  for (int j = 0; j < count; ++j)
    A.job[j] = WpJob{static_cast<const uint16_t*>(G[j].codes0), G[j].x2f, G[j].y1p, G[j].s0};
  const int64_t tiles = (int64_t)A.nrt * A.nct * A.SGk * count;
  QS_REQUIRE(tiles < ((int64_t)1 << 30), "wide GEMM: grid too large");
  return launch_wp(A, (unsigned)((tiles + 7) / 8 * 8), stream);
}

}  // namespace qs
