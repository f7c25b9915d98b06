// One-launch quantized-linear forward for decode-size batches (B <= 2,
// n, m <= 32768 on the chunk scheme; n <= 16384 for fp16 / fp32 activations),
// the path QuantizedLinear.forward takes at generation time
// (quipsharp/checkpoint.py:141-146 -> quipsharp/quantize.py:116-124).
//
// Transforms.  A length-n transform T_n = K_p (x) H_L (n = p L, L = 2^k >= 256)
// is split as T_n = M (x) H_256 over the index i = 256 c + t, with the S x S
// chunk matrix M = K_p (x) H_{L/256} (S = n / 256 <= 128) applied on the
// matrix cores (bf16 hi + lo operands, fp32 accumulate) and the 256-point
// Walsh-Hadamard inside a chunk by one wave (four values per lane, two
// stages in registers and six across lanes with DPP / permlane exchanges).
//
// Work-group j owns one slice group (W <= 16 slices of 256 input columns)
// and a strided set of 16-row blocks, so each wave's activation operand stays
// in registers for the whole launch.  Each slice is taken by P = 1, 2 or 4
// waves that split the row blocks (phases), so that W P waves of the 16 have
// work (fused_plan: 20 chunks run as 5 groups of 4 slices x 4 phases rather
// than 2 groups of 10 slices with 6 waves idle).  Per work-group:
//   1. issue the activation loads, then the decode LUTs (built at compile
//      time, copied into LDS) and K;
//   2. input transform (every work-group, only its own slices), chunk
//      combination first: activations times sv -> chunk table (bf16) ->
//      slice rows sum_c M[s][c] x_c on the matrix cores -> per slice (one
//      wave) the 256-point transform -> fp16 operand row scaled by 2^-e (e
//      from the row norm) plus the per-group sums for the +-1/4 shift term,
//      whose -1/4 sum_g S_g part is folded in per slice; the first code
//      tiles are requested once the chunk table is complete;
//   3. per row block: 8 MFMAs (+1 for the shift, +8 for an E8 1-bit second
//      stage) into one of 8 LDS slots; every 8 row blocks (and after the
//      last) the slots are reduced across the waves and the partial sums go
//      out as 64-bit slots {value, launch tag}, one agent-scope store each;
//   4. completion: tail work-groups poll the slots until every one they need
//      carries this launch's tag and apply S_u T_m(.) + bias: for m <= 4096
//      the job's first work-group alone (256-point transforms, then M); for
//      larger m in two levels, chunk transforms spread over the job's first
//      ceil(m / 4096) work-groups (one chunk per wave, results as tagged
//      slots), then M over 16 column groups of 16 (one work-group each).
//      The tail work-groups then store the tag as the workspace's new epoch.
//
// Cross-work-group visibility.  Slots are written with agent-scope relaxed
// atomic stores and read with agent-scope relaxed atomic loads, which on
// gfx950 are write-through / read-through at the device coherence point (no
// per-XCD L2 copy is involved).  A 64-bit atomic store makes value and tag
// visible together, so the reader needs no counter and the writers no wait
// for their stores to complete (that wait plus a counter round trip cost
// ~3 us per launch).  A work-group only waits for work-groups that wait for
// nothing, or (second level) for those, so no cycle of waits exists; the
// launch progresses as long as the work-groups that poll (at most 16 per
// linear) leave a CU free for the others, and every poll is bounded
// (kMaxPolls, NaN outputs if exceeded).
#include <hip/hip_ext.h>

#include <type_traits>

#include "qs_forward_dev.h"
#include "qs_linear_dev.h"
#include "qs_preop_dev.h"

namespace qs {
namespace {


constexpr int kThreads = kFwdThreads;
constexpr int kMaxB = 2;
constexpr int kPrefetch = 2;  // code tiles in flight per wave (deeper rings measured slower)
constexpr int kMaxJobs = QS_MAX_GROUP;
constexpr int kXStride = 264;               // halves per slice row of the fp16 operand buffer
constexpr int kMaxSF = 128;                 // chunks of 256 (n, m <= 32768; n <= 16384 for fp16 / fp32 x)

// One linear of a launch.  Linears in one launch share the input x (and n);
// each has its own codes, signs, scales, output and workspace region.
struct FusedJob {
  const float* sv;
  const uint16_t* codes0;
  const uint8_t* codes1;
  int m, Gr, wg0;      // rows; row-block stride; first work-group of this linear
  float s0, s1;
  int ntail;           // tail work-groups (output transform here; fills the alignment gap before y1p)
  float* y1p;          // [SG][B][m] fp32 partials (output transform in a separate kernel)
  unsigned long long* y1t;  // [SG][B][m] tagged partials (output transform here)
  unsigned long long* h2t;  // [B][m] tagged chunk transforms (two-level output transform)
  unsigned* epoch;     // tag of the last launch (zero before the first)
  float* xmul;         // [B] 2^e per batch row (for a separate output kernel)
  int out_in_kernel;
  int Sm, lsh_m, pm;
  const float* Km;     // pm x pm (pm > 1)
  float scale_m, layer_scale;
  const float* su;
  const float* bias;
  void* y;
  int64_t ldy;
};

struct FusedArgs {
  const void* x;
  int x_dtype;
  int64_t ldx;
  int B;
  int n, Sn, lsh_n, pn;
  const float* Kn;
  float scale_n;
  int S, SG, W, P, lgP;  // chunks, slice groups, slices per group, row-block phases (W P <= 16), log2 P
  int y_dtype;
  int sbits;  // su, sv of every job are packed sign bits
  int njobs;
  FusedJob job[kMaxJobs];
  // the workspace (its tags are cleared when a job's counter wraps); after
  // the jobs so that their fields keep the offsets the kernel loads them from
  unsigned long long* ws;
  unsigned long long ws_words;
  // pre-operation on the input rows (XT 3: RMSNorm of x + x2 with weight nw,
  // h' to h_out by work-group 0), qs_preop_dev.h
  const uint16_t* x2;
  int64_t ldx2;
  const uint16_t* nw;
  uint16_t* h_out;
  int64_t ldo;
  float eps;
};

// LDS layout (bytes).  The slice rows of the input transform alias the
// reduction buffer (both are dead before the first row block); the output
// transform reuses everything.
constexpr int kOffHi = 0;                                   // 4096 x uint32 (four fp16 high bytes)
constexpr int kOffLo = 16384;                               // 4096 x uint32
constexpr int kOffLut1 = 32768;                             // 256 x uint4
constexpr int kRedSlots = 8;                                // row blocks reduced together
constexpr int kRedSlot = kWaves * 16 * kMaxB;               // floats per slot: [wave][row][batch]
constexpr int kZStride = 260;                               // floats per slice row (rows 16 banks apart)
constexpr int kRedBytes = kRedSlots * kRedSlot * 4 > 16 * kZStride * 4 ? kRedSlots * kRedSlot * 4 : 16 * kZStride * 4;
constexpr int kOffRed = kOffLut1 + 4096;                    // kRedSlots x kRedSlot floats
constexpr int kOffZ = kOffRed;                              // 16 x kZStride floats (slice rows)
constexpr int kMinStride = kMaxSF + 8;                      // bf16 per row of the input chunk matrix
constexpr int kOffMin = kOffRed + kRedBytes;                // 2 x 16 x kMinStride bf16 (hi, lo)
constexpr int kOffXH = kOffMin + 2 * 16 * kMinStride * 2;   // kMaxB x 16 x kXStride halves
constexpr int kOffXS = kOffXH + kMaxB * 16 * kXStride * 2;  // kMaxB x 16 x 32 halves (group sums)
constexpr int kOffMisc = kOffXS + kMaxB * 16 * 32 * 2;      // row norms (16 floats; 16 more for a norm pre-op)
constexpr int kOffXR = kOffMisc + 128;                      // chunk table (bf16, one or two planes)
constexpr int kXRBytes = 2 * 256 * (kMaxSF / 2 + 8) * 2;    // two planes of 64 chunks
static_assert(256 * (kMaxSF + 8) * 2 <= kXRBytes, "one plane of kMaxSF chunks fits");
constexpr int kLdsBytes = kOffXR + kXRBytes;
static_assert(kLdsBytes <= 160 * 1024 - 128, "LDS budget");
static_assert(kOffMin % 16 == 0 && kOffXR % 16 == 0 && kOffZ % 16 == 0, "16-byte aligned regions");
// Output transform in one work-group (m <= 4096): the chunk matrix M as bf16
// hi / lo at address 0 (48 x 64, zero-padded), the chunks in the chunk
// table's place.
constexpr int kOffMh = 0;
constexpr int kOffMl = kOffMh + kMBytes;
constexpr int kOffY1 = kOffXR;
static_assert(kOffMl + kMBytes <= kOffXR && kOffY1 + 16 * kYStride * 4 <= kLdsBytes, "one-group output fits");
// Output transform in two levels (m > 4096): all of M (rows padded to 16,
// columns to 32; bf16 hi / lo) at address 0, the staged columns of h of
// both batch rows (hi / lo) in the chunk table's place.
constexpr int kOffM2 = 0;
constexpr int kL2Groups = 16;                               // column groups of 16
static_assert(2 * kMaxSF * kMinStride * 2 <= kOffXR, "M of kMaxSF chunks fits below the chunk table");
constexpr int kOffHB = kOffXR;
static_assert(kOffHB + 2 * kMaxB * 16 * kMinStride * 2 <= kLdsBytes, "staged columns fit");
static_assert(kRedSlots * 16 * 8 == kThreads, "one reduction pass: 8 / (P B) threads per output, P B <= 8");

// Activation quads of the input transform: thread (w, lane) holds chunks
// c = c0 + i (i < 4, c0 = 64 round + 4 w) of one batch row at columns
// t = 4 lane + u (u < 4), as loaded: x words (XT: 0 bf16, 1 fp16, 2 fp32;
// rows of x 8- / 16-byte aligned) and sv (fp32, or with SB the word of sign
// bits).  A thread holds one quad at a time, so a chunk table of more than
// 64 chunks takes a second round of loads.
// XT 3: bf16 rows with the RMSNorm pre-operation (qs_preop_dev.h): v2 holds
// the residual delta's words and nw the norm weights; after the
// pre-operation v holds the bf16 operand.
template <int XT, bool SB>
struct XQuad {
  uint32_t v[4][XT == 2 ? 4 : 2];
  uint32_t s[4][SB ? 1 : 4];
  uint32_t v2[4][2];
  uint32_t nw[4][2];
};
template <int XT, bool SB>
__device__ __forceinline__ void load_x_quad(const void* x, int64_t ldx, const float* sv, int S, int b, int c0,
                                            int lane, XQuad<XT, SB>& r, const uint16_t* x2 = nullptr,
                                            int64_t ldx2 = 0, const uint16_t* nw = nullptr) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int k = 0; k < (XT == 2 ? 4 : 2); ++k) r.v[i][k] = 0;
#pragma unroll
    for (int k = 0; k < (SB ? 1 : 4); ++k) r.s[i][k] = 0;
#pragma unroll
    for (int k = 0; k < 2; ++k) r.v2[i][k] = r.nw[i][k] = 0;
    const int c = c0 + i;
    if (c < S) {
      if constexpr (XT >= 3) {
        const int e = 256 * c + 4 * lane;
        if (x2) {
          const uint2 t = *reinterpret_cast<const uint2*>(x2 + (int64_t)b * ldx2 + e);
          r.v2[i][0] = t.x, r.v2[i][1] = t.y;
        }
        if constexpr (XT == 3) {
          const uint2 t = *reinterpret_cast<const uint2*>(nw + e);
          r.nw[i][0] = t.x, r.nw[i][1] = t.y;
        }
      }
      const int i0 = 256 * c + 4 * lane;
      if constexpr (SB) {
        r.s[i][0] = reinterpret_cast<const uint32_t*>(sv)[i0 >> 5];
      } else {
        const uint4 t = *reinterpret_cast<const uint4*>(sv + i0);
        r.s[i][0] = t.x, r.s[i][1] = t.y, r.s[i][2] = t.z, r.s[i][3] = t.w;
      }
      const int64_t xi = (int64_t)b * ldx + i0;
      if constexpr (XT == 2) {
        const uint4 t = *reinterpret_cast<const uint4*>(static_cast<const float*>(x) + xi);
        r.v[i][0] = t.x, r.v[i][1] = t.y, r.v[i][2] = t.z, r.v[i][3] = t.w;
      } else {
        const uint2 t = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(x) + xi);
        r.v[i][0] = t.x, r.v[i][1] = t.y;
      }
    }
  }
}
// Chunk i of the quad times sv, as fp32 (zero past the S chunks: the loads
// left zeros).
template <int XT, bool SB>
__device__ __forceinline__ void finish_quad_chunk(const XQuad<XT, SB>& r, int i, int lane, float (&o)[4]) {
  float xv[4];
  if constexpr (XT == 0 || XT >= 3) {
    xv[0] = __uint_as_float(r.v[i][0] << 16), xv[1] = __uint_as_float(r.v[i][0] & 0xFFFF0000u);
    xv[2] = __uint_as_float(r.v[i][1] << 16), xv[3] = __uint_as_float(r.v[i][1] & 0xFFFF0000u);
  } else if constexpr (XT == 1) {
    xv[0] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.v[i][0] & 0xFFFFu));
    xv[1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.v[i][0] >> 16));
    xv[2] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.v[i][1] & 0xFFFFu));
    xv[3] = (float)__builtin_bit_cast(_Float16, (uint16_t)(r.v[i][1] >> 16));
  } else {
#pragma unroll
    for (int u = 0; u < 4; ++u) xv[u] = __uint_as_float(r.v[i][u]);
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    if constexpr (SB) o[u] = flip_by_bit(xv[u], r.s[i][0] >> (4 * (lane & 7)), u);
    else o[u] = xv[u] * __uint_as_float(r.s[i][u]);
  }
}
// The quad into the chunk table XR[t][c] (xrs halves per column t), one
// chunk pair at a time: the truncated bf16 high parts, and (fp16 / fp32
// activations) the truncated remainders into the second plane XR1.  Returns
// the quad's sum of squares.
template <int XT, bool SB>
__device__ __forceinline__ float store_quad(const XQuad<XT, SB>& r, uint16_t* XR0, uint16_t* XR1, int xrs, int c0,
                                            int lane, bool store) {
  float ss = 0.0f;
#pragma unroll
  for (int p = 0; p < 2; ++p) {
    float a[4], c[4];
    finish_quad_chunk(r, 2 * p, lane, a);
    finish_quad_chunk(r, 2 * p + 1, lane, c);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      ss = __builtin_fmaf(a[u], a[u], ss);
      ss = __builtin_fmaf(c[u], c[u], ss);
      uint32_t h, l;
      split_bf2(a[u], c[u], h, l);
      const int off = (4 * lane + u) * xrs + c0 + 2 * p;
      if (store) {
        *reinterpret_cast<uint32_t*>(XR0 + off) = h;
        if constexpr (XT == 1 || XT == 2) *reinterpret_cast<uint32_t*>(XR1 + off) = l;
      }
    }
  }
  return ss;
}
__device__ __forceinline__ bf16x8 lds_bf16x8(const uint16_t* p) {
  return __builtin_bit_cast(bf16x8, *reinterpret_cast<const uint4*>(p));
}

// Level 1 of the two-level output transform: h_c of batch row b as tagged
// slots h2t[b][256 c + t], element t = lane + 64 j.
__device__ __forceinline__ void store_h2(unsigned long long* h2t, int b, int m, int c, int lane, uint32_t tag,
                                         const float (&z)[1][4]) {
#pragma unroll
  for (int j = 0; j < 4; ++j)
    __hip_atomic_store(h2t + h2_index(b, m, chunk_elem(c, lane, j)), tagged(z[0][j], tag), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
// Level 2: h[c][16 g + tt] of both batch rows, v = tid + 1024 k -> (c, tt) =
// (v / 16, v % 16), polled until every slot carries the tag (bounded: NaN
// for a slot still missing after kMaxPolls rounds); zero for c >= Sm.
__device__ __forceinline__ void poll_columns(const unsigned long long* h2t, int m, int Sm, int B, int g, int tid,
                                             uint32_t tag, float (&hv)[kMaxB][2]) {
  const unsigned long long fill = tagged(0.0f, tag);
  unsigned long long p[kMaxB][2];
  auto load = [&](bool only_missing) {
#pragma unroll
    for (int b = 0; b < kMaxB; ++b)
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int v = tid + kThreads * k, c = v >> 4, tt = v & 15;
        const unsigned long long* src = h2t + h2_index(b, m, column_elem(c, g, tt));
        if (only_missing) {
          if ((uint32_t)(p[b][k] >> 32) != tag)
            p[b][k] = __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
          p[b][k] = (b < B && c < Sm) ? __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : fill;
        }
      }
  };
  load(false);
  for (int round = 0;; ++round) {
    bool ok = true;
#pragma unroll
    for (int b = 0; b < kMaxB; ++b)
#pragma unroll
      for (int k = 0; k < 2; ++k) ok = ok && (uint32_t)(p[b][k] >> 32) == tag;
    if (ok) break;
    if (round == kMaxPolls) {
#pragma unroll
      for (int b = 0; b < kMaxB; ++b)
#pragma unroll
        for (int k = 0; k < 2; ++k)
          if ((uint32_t)(p[b][k] >> 32) != tag) p[b][k] = tagged(__builtin_nanf(""), tag);
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    load(true);
  }
#pragma unroll
  for (int b = 0; b < kMaxB; ++b)
#pragma unroll
    for (int k = 0; k < 2; ++k) hv[b][k] = __uint_as_float((uint32_t)p[b][k]);
}

template <bool HAS2, bool SB, int XT>
__global__ __launch_bounds__(kThreads) void linear_fused_kernel(FusedArgs A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint4* lut1 = reinterpret_cast<uint4*>(lds + kOffLut1);
  float* red = reinterpret_cast<float*>(lds + kOffRed);
  uint16_t* MinH = reinterpret_cast<uint16_t*>(lds + kOffMin);
  uint16_t* MinL = MinH + 16 * kMinStride;
  _Float16* XH = reinterpret_cast<_Float16*>(lds + kOffXH);
  _Float16* XS = reinterpret_cast<_Float16*>(lds + kOffXS);
  float* Z = reinterpret_cast<float*>(lds + kOffZ);
  float* wsum = reinterpret_cast<float*>(lds + kOffMisc);
  uint16_t* XR0 = reinterpret_cast<uint16_t*>(lds + kOffXR);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, in a scalar register
  const int q = lane >> 4, r16 = lane & 15;
  int g = 0;
#pragma unroll
  for (int k = 1; k < kMaxJobs; ++k)
    if (k < A.njobs && (int)blockIdx.x >= A.job[k].wg0) g = k;
  const FusedJob& J = A.job[g];
  const int lb = (int)blockIdx.x - J.wg0;  // work-group index within this linear
  const int RB = J.m >> 4;
  const int sg = lb / J.Gr, jr = lb - sg * J.Gr;
  // wave w = ph W + wsl takes slice wsl of the group and the row blocks of
  // phase ph: at step i, row block jr + (P i + ph) Gr
  const int ph = w / A.W, wsl = w - ph * A.W;
  const int sl = sg * A.W + wsl;
  const bool active = ph < A.P && sl < A.S;
  auto own_rb = [&](int i) { return jr + (A.P * i + ph) * J.Gr; };
  const LaneX lx = lane_x_init();

  // 1. loads: the first activation quad (the transform waits for it), then
  //    the decode LUTs (32 bytes per thread, stored into LDS before the first
  //    barrier), this wave's row of K and its first code tiles; the rest of
  //    the code tiles once the activations are in the chunk table, the
  //    launch tag after the transform.
  LutCopy<kThreads> lutw;
  uint4 t1row = make_uint4(0, 0, 0, 0);  // E8 one-bit table row (fp16)
  // this wave's row of the input chunk matrix (slice sl): K at columns
  // c = lane, lane + 64 (unconditional loads; sv is a dummy source without K)
  float mk[2];
  auto load_mk = [&]() {
    const float* ksrc = A.pn > 1 ? A.Kn : J.sv;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int c = lane + 64 * h;
      const int ki = (A.pn > 1 && active && c < A.Sn) ? (sl >> A.lsh_n) * A.pn + (c >> A.lsh_n) : 0;
      mk[h] = at_off(ksrc, (uint32_t)ki);
    }
  };
  // Code tiles stream through a ring of kPrefetch registers, refilled as
  // they are consumed.  The loads are unconditional (a tile past the end or
  // of an idle wave reads tile 0 instead) and the ring is unrolled, so the
  // compiler waits for exactly the tile in use, never for the whole ring.
  uint4 pre[kPrefetch];
  uint2 pre1[kPrefetch] = {};
  // byte offset of this lane's 16 code bytes of row block rb; past the end,
  // the work-group's own last row block again (an L2 hit, and spread over the
  // chip: every wave of every work-group clamping to one tile made that tile's
  // cache lines a hot spot), and the last slice for an idle wave.  jr < Gr <=
  // RB, so rb_last is a valid row block; m n / 4 < 2^32 bytes of codes.
  const int rb_last = jr + ((RB - 1 - jr) / J.Gr) * J.Gr;
  const uint32_t slc = (uint32_t)(sl < A.S ? sl : A.S - 1);
  auto code_off = [&](int rb) -> uint32_t {
    const uint32_t r = (uint32_t)(rb < RB ? rb : rb_last);
    return (r * (uint32_t)A.S + slc) * 1024u + 16u * lane;
  };

  // tag of this launch's partial sums, read by every work-group before it
  // stores any slot; the epoch only changes after every slot of the launch
  // has been read
  uint32_t epoch = 0;
  // ring entries k0 .. k1 - 1: the first kEarlyTiles are requested before the
  // input transform (they arrive while it runs), the rest once the chunk
  // table is complete (requesting the whole ring early measured slower)
  auto prefetch_codes = [&](int k0, int k1) {
#pragma unroll
    for (int k = 0; k < kPrefetch; ++k) {
      if (k < k0 || k >= k1) continue;
      const uint32_t off = code_off(own_rb(k));
      pre[k] = ld_nt_u4(reinterpret_cast<const char*>(J.codes0) + off);
      if (HAS2) pre1[k] = ld_nt_u2(J.codes1 + off / 2);
    }
  };
  constexpr int kEarlyTiles = 1;
  float emul0 = 1.0f, emul1 = 1.0f;  // 2^e of batch rows 0 and 1
  // This wave's fp16 operand row of batch row b (slice values t = 4 lane + u
  // times mul), and the per-group sums for the +-1/4 shift term (group t / 8).
  auto store_operand_row = [&](const int b, const float (&v)[4], const float mul) {
    uint32_t hw[2];
    float hs = 0.0f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const _Float16 h0 = (_Float16)(v[2 * k] * mul), h1 = (_Float16)(v[2 * k + 1] * mul);
      hs += (float)h0;
      hs += (float)h1;
      hw[k] = (uint32_t)__builtin_bit_cast(uint16_t, h0) | ((uint32_t)__builtin_bit_cast(uint16_t, h1) << 16);
    }
    *reinterpret_cast<uint2*>(XH + (b * 16 + w) * kXStride + 4 * lane) = make_uint2(hw[0], hw[1]);
    hs += lane_xor<1>(hs, lx);  // lane pairs
    if ((lane & 1) == 0) XS[(b * 16 + w) * 32 + (lane >> 1)] = (_Float16)hs;
  };

  XQuad<XT, SB> xr;
  load_x_quad(A.x, A.ldx, J.sv, A.Sn, 0, 4 * w, lane, xr, A.x2, A.ldx2, A.nw);
  load_luts(tid, lutw);
  if (HAS2 && tid < 256) t1row = *reinterpret_cast<const uint4*>(kE81h.w[tid]);
  load_mk();
  prefetch_codes(0, kEarlyTiles);
  // 2. input transform, one batch row at a time, chunk combination first:
  //    T_n = M (x) H_256 = (I (x) H_256)(M (x) I).  The activation chunks go
  //    into the chunk table XR[t][c] as bf16 (exact for bf16 activations
  //    times signs; fp16 / fp32 activations add a plane of low parts); the
  //    slice rows z_s = sum_c M[sl][c] x_c of this work-group come out of the
  //    matrix cores (wave w: columns t = 16 w + r16 of all 16 rows), and wave
  //    w applies the 256-point transform to its own slice row and writes it
  //    as its fp16 operand row (plus the per-group sums for the +-1/4 shift
  //    term).
  const int Spad = (A.Sn + 31) & ~31;  // chunks padded to the matrix cores' k-steps of 32
  const int xrs = Spad + 8;            // halves per column of the chunk table
  uint16_t* XR1 = XR0 + 256 * xrs;
  // one batch row; called once per row rather than looped, so that no
  // activation registers are carried from one row to the next
  auto input_row = [&](const int b) {
    // quads inside the padded range are stored (zeros past the S chunks);
    // the first quad of row 0 was loaded at the start
    if (b > 0) load_x_quad(A.x, A.ldx, J.sv, A.Sn, b, 4 * w, lane, xr, A.x2, A.ldx2, A.nw);
    // a wave whose quad lies past the row's chunks holds zeros, and past the
    // padded chunk table stores nothing: it skips that arithmetic (a
    // wave-uniform branch; its sums stay +0, added in the same order)
    const bool row_quad = 4 * w < A.Sn, table_quad = 4 * w < Spad;
    float ss;
    if constexpr (XT == 3) {
      // the norm needs the whole row before the chunk table (one quad: n <=
      // 16384, checked on the host)
      const bool has_delta = A.x2 != nullptr;
      float ssn = row_quad ? rms_quad_resid(xr.v, xr.v2, has_delta) : 0.0f;
      ssn = wave_sum(ssn, lx);
      if (lane == 0) wsum[kWaves + w] = ssn;
      if (b == 0) {
        // the LUTs at the first barrier, as without a pre-operation (their
        // registers are not kept across the norm)
        store_luts(lds, tid, lutw);
        if (HAS2 && tid < 256) lut1[tid] = t1row;
      }
      __syncthreads();  // the row's sums of squares
      float tot = 0.0f;
#pragma unroll
      for (int i = 0; i < kWaves; ++i) tot += wsum[kWaves + i];
      const float rs = rms_scale(tot, A.n, A.eps);
      if (blockIdx.x == 0 && A.h_out) {  // the residual stream h', once
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int c = 4 * w + i;
          if (c < A.Sn)
            *reinterpret_cast<uint2*>(A.h_out + (int64_t)b * A.ldo + 256 * c + 4 * lane) =
                make_uint2(xr.v[i][0], xr.v[i][1]);
        }
      }
      if (row_quad) rms_quad_apply(xr.v, xr.nw, rs);
      ss = table_quad ? store_quad(xr, XR0, XR1, xrs, 4 * w, lane, true) : 0.0f;
    } else {
      ss = table_quad ? store_quad(xr, XR0, XR1, xrs, 4 * w, lane, true) : 0.0f;
      if (64 + 4 * w < Spad) {
        XQuad<XT, SB> x2;
        load_x_quad(A.x, A.ldx, J.sv, A.Sn, b, 64 + 4 * w, lane, x2);
        ss += store_quad(x2, XR0, XR1, xrs, 64 + 4 * w, lane, true);
      }
    }
    ss = wave_sum(ss, lx);
    if (lane == 0) wsum[w] = ss;
    if (b == 0) {
      // row w of M = K_p (x) H_{2^lsh} (hi / lo), zero past the S chunks and
      // for idle waves
      const int hm = (1 << A.lsh_n) - 1;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int c = lane + 64 * h;
        if (c < Spad) {
          float v = (active && c < A.Sn) ? (A.pn > 1 ? mk[h] : 1.0f) : 0.0f;
          if (__builtin_popcount(sl & c & hm) & 1) v = -v;
          uint32_t hi, lo;
          split_bf2(v, 0.0f, hi, lo);
          MinH[w * kMinStride + c] = (uint16_t)hi;
          MinL[w * kMinStride + c] = (uint16_t)lo;
        }
      }
    }
    if (b == 0 && XT != 3) {
      store_luts(lds, tid, lutw);
      if (HAS2 && tid < 256) lut1[tid] = t1row;
    }
    __syncthreads();  // chunk table, norms (and, the first time, M and the LUTs) complete
    if (b == 0) prefetch_codes(kEarlyTiles, kPrefetch);
    float norm2 = 0.0f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) norm2 += wsum[i];
    const int e = operand_exponent(norm2);
    if (b == 0) emul0 = ldexpf(1.0f, e);
    else emul1 = ldexpf(1.0f, e);
    const float mul = ldexpf(A.scale_n, -e);
    {
      const int t = 16 * w + r16;
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int kb = 0; kb < (Spad >> 5); ++kb) {
        const int k0 = 32 * kb + 8 * q;
        const bf16x8 xh = lds_bf16x8(XR0 + t * xrs + k0);
        const bf16x8 ah = lds_bf16x8(MinH + r16 * kMinStride + k0);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, xh, acc, 0, 0, 0);
        if (A.pn > 1)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lds_bf16x8(MinL + r16 * kMinStride + k0), xh, acc, 0, 0, 0);
        if constexpr (XT == 1 || XT == 2)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, lds_bf16x8(XR1 + t * xrs + k0), acc, 0, 0, 0);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) Z[(4 * q + j) * kZStride + t] = acc[j];
    }
    __syncthreads();  // slice rows complete (the chunk table and the norms are free again)
    // the waves of the other phases hold the same slices as phase 0's: they
    // read phase 0's operand rows; waves past the last slice read none (a
    // wave-uniform branch)
    if (ph == 0 && sl < A.S) {
      const float4 z4 = *reinterpret_cast<const float4*>(Z + w * kZStride + 4 * lane);
      float v[1][4] = {{z4.x, z4.y, z4.z, z4.w}};
      h256<1>(v, lane, lx);
      store_operand_row(b, v[0], mul);
    }
    };
  input_row(0);
  if (A.B > 1) input_row(1);
  __syncthreads();  // slice rows read (their LDS becomes the reduction slots)
  // the launch tag's epoch: read once the input transform is done (reading it
  // earlier measured slower); sv is a dummy source for a linear whose output
  // transform runs in another kernel
  epoch = __hip_atomic_load(J.out_in_kernel ? J.epoch : reinterpret_cast<unsigned*>(const_cast<float*>(J.sv)),
                            __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // MFMA operand of lane (q, b = r16): columns 64q..64q+63 of this wave's
  // slice (the operand rows of the phase-0 wave of the slice, wave wsl)
  const half8 hzero = {0, 0, 0, 0, 0, 0, 0, 0};
  half8 xb[8];
  half8 xs = hzero;
  float slice_shift = 0.0f;  // sum_g S_g over the lane's 64 columns, batch row r16
#pragma unroll
  for (int c = 0; c < 8; ++c) xb[c] = hzero;
  if (active && r16 < A.B) {
    const _Float16* row = XH + (r16 * 16 + wsl) * kXStride + 64 * q;
#pragma unroll
    for (int c = 0; c < 8; ++c) xb[c] = *reinterpret_cast<const half8*>(row + 8 * c);
    xs = *reinterpret_cast<const half8*>(XS + (r16 * 16 + wsl) * 32 + 8 * q);
#pragma unroll
    for (int c = 0; c < 8; ++c) slice_shift += (float)xs[c];
  }
  // slice total of S_g over the four q-lanes of batch row r16
  slice_shift += lane_xor<16>(slice_shift, lx);
  slice_shift += lane_xor<32>(slice_shift, lx);
  if (lb == 0 && tid < A.B) J.xmul[tid] = tid == 0 ? emul0 : emul1;

  const uint32_t tag = J.out_in_kernel ? next_tag(epoch, g) : 0u;

  // 3. row blocks, in steps of P (one per phase)
  const int nw = A.S - sg * A.W < A.W ? A.S - sg * A.W : A.W;
  const int stride = A.P * J.Gr;  // row blocks per step
  int k = 0;  // steps done: selects the reduction slot
  for (int i0 = 0; jr + i0 * stride < RB; i0 += kPrefetch) {
#pragma unroll
  for (int u = 0; u < kPrefetch; ++u) {
    // every ring step runs (the ring registers are never copied); a step
    // past the last row block only refills its entry
    const int step = i0 + u;
    const bool step_valid = jr + step * stride < RB;  // the work-group has row blocks at this step
    const int rb = own_rb(step);
    const bool valid = rb < RB;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    floatx4 accs = {0.f, 0.f, 0.f, 0.f};
    floatx4 acc2 = {0.f, 0.f, 0.f, 0.f};
    const uint4 cw = pre[u];
    const uint2 cw1 = pre1[u];
    if (valid) {
      // (idle waves decode tile 0 with a zero operand; their results are
      // not stored)
      // all of the tile's LUT reads first (one LDS round trip per tile, not
      // one per code), then the MFMAs, alternating between two accumulators
      // so that consecutive MFMAs do not wait for each other
      const uint32_t wd[4] = {cw.x, cw.y, cw.z, cw.w};
      uint32_t hv[8], lv[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) code_lut_words(wd[c >> 1], c, kOffHi, kOffLo, hv[c], lv[c]);
      floatx4 acc_b = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const half8 av = code_operand(hv[c], lv[c]);
        if (c & 1) acc_b = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, xb[c], acc_b, 0, 0, 0);
        else acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, xb[c], acc, 0, 0, 0);
        if constexpr (HAS2) {
          const uint32_t idx = ((c < 4 ? cw1.x : cw1.y) >> (8 * (c & 3))) & 0xFFu;
          acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, lut1[idx]), xb[c], acc2, 0, 0,
                                                          0);
        }
      }
      accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(shift_operand(wd), xs, accs, 0, 0, 0);
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[j] += acc_b[j];
    }
    {
      // refill this ring entry (its tile is consumed) with the tile
      // kPrefetch steps ahead
      const uint32_t off = code_off(own_rb(step + kPrefetch));
      pre[u] = ld_nt_u4(reinterpret_cast<const char*>(J.codes0) + off);
      if (HAS2) pre1[u] = ld_nt_u2(J.codes1 + off / 2);
    }
    // partial of this slice for rows 4q..4q+3, batch column r16, into this
    // step's slot; the slots are reduced across the waves every kRedSlots
    // steps (and after the last), so the waves decode without a barrier per
    // row block
    const int slot = k % kRedSlots;
    float* rbuf = red + slot * kRedSlot;
    if (valid && r16 < A.B) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = J.s0 * (acc[j] + 0.5f * accs[j] - 0.25f * slice_shift);
        if (HAS2) v = v + J.s1 * acc2[j];
        rbuf[(w * 16 + 4 * q + j) * kMaxB + r16] = active ? v : 0.0f;
      }
    }
    if (step_valid && (slot == kRedSlots - 1 || jr + (step + 1) * stride >= RB)) {
      __syncthreads();
      // output o = ((s P + p) 16 + row) B + b of slot s <= slot, phase p,
      // summed over the phase's waves by tpo threads (waves part, part +
      // tpo, ...), then across them; tpo depends on B and P only, so every
      // output is summed in the same order whatever the number of steps
      // pending
      // (P and B are powers of two: shifts, not divisions)
      const int lgb = A.B - 1, lgpb = A.lgP + lgb;  // log2 B, log2 (P B)
      const int nout = (slot + 1) << (4 + lgpb);
      const int tpo = 8 >> lgpb;  // kThreads / (kRedSlots * 16 * P * B)
      const int o = tid >> (3 - lgpb), part = tid & (tpo - 1);
      float v = 0.0f;
      int s = 0, p = 0, row = 0, bc = 0;
      if (o < nout) {
        s = o >> (4 + lgpb);
        const int rr = o & ((16 << lgpb) - 1);
        p = rr >> (4 + lgb);
        const int r2 = rr & ((16 << lgb) - 1);
        row = r2 >> lgb;
        bc = r2 & lgb;
        for (int ww = part; ww < nw; ww += tpo)
          v += red[s * kRedSlot + ((p * A.W + ww) * 16 + row) * kMaxB + bc];
      }
      if (tpo >= 2) v += lane_xor<1>(v, lx);
      if (tpo >= 4) v += lane_xor<2>(v, lx);
      if (tpo == 8) v += lane_xor<4>(v, lx);
      const int rbs = jr + (A.P * (step - (slot - s)) + p) * J.Gr;  // row block of slot s, phase p
      if (o < nout && part == 0 && rbs < RB) {
        const size_t idx = partial_index(sg, A.B, bc, J.m, block_elem(rbs, row));
        if (J.out_in_kernel)
          __hip_atomic_store(&J.y1t[idx], tagged(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          J.y1p[idx] = v;  // read by a separate output kernel after this one
      }
      __syncthreads();  // the slots are free again
    }
    k += step_valid;
  }
  }

  // 4. completion: the tail work-groups of the job wait for every tagged
  //    partial sum of this launch and apply the output transform
  if (!J.out_in_kernel) return;
  if (J.Sm <= kWaves) {
    // m <= 4096: the job's first work-group, one output chunk per wave,
    // 256-point transforms first
    if (lb != 0) return;
    constexpr int OC = 1;
    float* Y1 = reinterpret_cast<float*>(lds + kOffY1);
    // Output chunk stage on the matrix cores (mstage_tile): lane (q, r16) of
    // wave w produces column t = 16 w + r16 of rows r = 16 a + 4 q + j.
    const int Sm = J.Sm;
    const int t = 16 * w + r16;
    // Loads: the K entries of M (odd factor), su and bias, then the first
    // partial-sum slots (su and bias before the slots measured slightly
    // faster), all in flight together (unconditional loads from valid
    // addresses, selected where they are used: a load under a branch is
    // waited for at the branch's end).
    float kmv[3];
    mmat_load(kmv, Sm, J.lsh_m, J.pm, J.Km, tid);
    float suo[OC][4], bio[OC][4];
    // no bias: a dummy load from the partial-sum slots (at least m floats;
    // su may be m / 32 words of sign bits), never used: the bias term is
    // selected, not multiplied by 0, so a non-finite dummy cannot reach the
    // output
    const float* const bsrc = J.bias ? J.bias : reinterpret_cast<const float*>(J.y1t);
    const bool has_bias = J.bias != nullptr;
    auto load_su_bias = [&]() {
#pragma unroll
      for (int a = 0; a < OC; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 16 * a + 4 * q + j;
          const int ii = r < Sm ? out_elem(r, t) : 0;
          suo[a][j] = load_su(J.su, SB, ii);
          bio[a][j] = at_off(bsrc, (uint32_t)ii);
        }
    };
    // M = K_p (x) H_{2^lsh_m} as bf16 hi / lo, zero-padded to 48 x 64
    uint16_t* Mh = reinterpret_cast<uint16_t*>(lds + kOffMh);
    uint16_t* Ml = reinterpret_cast<uint16_t*>(lds + kOffMl);
    void* const yp = J.y;
    const int64_t ldy = J.ldy;
    const int ydt = A.y_dtype;
    const float mul0 = J.scale_m * J.layer_scale;
    const int nrt = (Sm + 15) >> 4, nkb = (Sm + 31) >> 5;
    // one batch row (B <= 2); called once per row rather than looped, so that
    // no address arithmetic is hoisted out of a loop and kept live (and
    // spilled) across the polling
    auto row = [&](const int b) {
      PollState<OC> ps;
      if (b == 0) load_su_bias();
      poll_issue(J.y1t, J.m, Sm, A.B, b, w, lane, tag, ps);
      if (b == 0) mmat_store(kmv, Sm, J.lsh_m, Mh, Ml, tid);  // waits for the K loads only
      float zv[OC][4];
      poll_finish(J.y1t, J.m, Sm, A.SG, A.B, b, w, lane, tag, ps, zv);
      h256_chunks(zv, Sm, lane, lx);
      if (b > 0) __syncthreads();  // the previous row's reads of Y1 are done
      store_chunks_lanes(Y1, Sm, w, lane, zv);
      __syncthreads();  // chunks (and, the first time, M) complete
      const float mul = mul0 * (b == 0 ? emul0 : emul1);
      floatx4 acc[OC];
#pragma unroll
      for (int a = 0; a < OC; ++a) acc[a] = floatx4{0.f, 0.f, 0.f, 0.f};
      for (int kb = 0; kb < nkb; ++kb) {
        const ZOperand z = z_operand(Y1, Sm, t, q, kb);
#pragma unroll
        for (int a = 0; a < OC; ++a)
          if (a < nrt) acc[a] = mstage_step(acc[a], Mh, Ml, 16 * a, z, kb, J.pm > 1, q, r16);
      }
      float out[OC][4];
      int oidx[OC][4];  // output element of out[a][j] (-1: none)
#pragma unroll
      for (int a = 0; a < OC; ++a)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 16 * a + 4 * q + j;
          oidx[a][j] = r < Sm ? out_elem(r, t) : -1;
          out[a][j] = apply_su(acc[a][j] * mul, suo[a][j], SB, oidx[a][j]) + (has_bias ? bio[a][j] : 0.0f);
        }
      store_outputs(yp, ydt, (int64_t)b * ldy, oidx, out);
    };
    row(0);
    if (A.B > 1) row(1);  } else {
    // m > 4096 (S_m = m / 256 chunks): the output transform in two levels,
    // each spread over the job's first work-groups.
    //  1. chunk c = 16 j + w goes to wave w of work-group j < ceil(S_m / 16):
    //     it polls the chunk's partial sums, sums the slice groups, applies
    //     the 256-point transform and stores h_c as tagged slots (h2t);
    //  2. column group g (16 columns) goes to work-group g < 16: it polls
    //     h[c][16 g .. 16 g + 15] of every chunk, stages it as bf16 hi / lo,
    //     and wave a < ceil(S_m / 16) computes rows 16 a .. 16 a + 15 of
    //     M . h on the matrix cores, scales them, applies su and bias and
    //     stores them.
    // Level 1 only waits for work-groups that never wait; level 2 only for
    // level 1, which every work-group does before its level 2.
    const int Sm = J.Sm;
    const int nl1 = (Sm + 15) >> 4;
    const int nwg = J.Gr * A.SG;  // work-groups of this linear (>= 1)
    if (lb >= kL2Groups) return;
    for (int cg = lb; cg < nl1; cg += nwg) {
      const int c = 16 * cg + w;
      if (c < Sm) {
        PollState<1> p0, p1;
        poll_issue(J.y1t, J.m, Sm, A.B, 0, c, lane, tag, p0);
        if (A.B > 1) poll_issue(J.y1t, J.m, Sm, A.B, 1, c, lane, tag, p1);
        float z[1][4];
        poll_finish(J.y1t, J.m, Sm, A.SG, A.B, 0, c, lane, tag, p0, z);
        h256<1>(z, lane, lx);
        store_h2(J.h2t, 0, J.m, c, lane, tag, z);
        if (A.B > 1) {
          poll_finish(J.y1t, J.m, Sm, A.SG, A.B, 1, c, lane, tag, p1, z);
          h256<1>(z, lane, lx);
          store_h2(J.h2t, 1, J.m, c, lane, tag, z);
        }
      }
    }
    const int Smpad = (Sm + 31) & ~31;
    const int ms = Smpad + 8;  // halves per row of M and per staged column
    const int rows = 16 * nl1;
    uint16_t* M2h = reinterpret_cast<uint16_t*>(lds + kOffM2);
    uint16_t* M2l = M2h + rows * ms;
    uint16_t* HBh = reinterpret_cast<uint16_t*>(lds + kOffHB);  // [b][tt][c]
    uint16_t* HBl = HBh + kMaxB * 16 * ms;
    const bool m_lo = J.pm > 1;
    const float mul0 = J.scale_m * J.layer_scale;
    // no bias: a dummy load from the partial-sum slots (at least m floats),
    // never used (the bias term is selected, not multiplied by 0)
    const float* const bsrc = J.bias ? J.bias : reinterpret_cast<const float*>(J.y1t);
    const bool has_bias = J.bias != nullptr;
    {
      // M = K_p (x) H_{2^lsh_m} over the rows < 16 ceil(S_m / 16) and columns
      // < S_m padded to 32 in use: entry e = tid + 1024 i at (e >> LCS,
      // e & (2^LCS - 1)), a row stride of 32, 64 or 128 columns (S_m <= 32:
      // at most 32 rows, one entry per thread; <= 64: 64 rows, four; else
      // sixteen) (K loads first, unconditional: su is a dummy source without K)
      const float* ksrc = m_lo ? J.Km : J.su;
      const int hm = (1 << J.lsh_m) - 1;
      auto build_m = [&](auto lcs, auto ni) {
        constexpr int LCS = decltype(lcs)::value, NI = decltype(ni)::value;
        // rows in use <= S_m padded to 32 <= 2^LCS
        static_assert((1 << (2 * LCS)) <= NI * kThreads, "entries cover the rows in use");
        float kv[NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int e = tid + kThreads * i, r = e >> LCS, c = e & ((1 << LCS) - 1);
          const int ki = (m_lo && r < Sm && c < Sm) ? (r >> J.lsh_m) * J.pm + (c >> J.lsh_m) : 0;
          kv[i] = at_off(ksrc, (uint32_t)ki);
        }
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          const int e = tid + kThreads * i, r = e >> LCS, c = e & ((1 << LCS) - 1);
          if (r < rows && c < Smpad) {
            float v = (r < Sm && c < Sm) ? (m_lo ? kv[i] : 1.0f) : 0.0f;
            if (__builtin_popcount(r & c & hm) & 1) v = -v;
            uint32_t hi, lo;
            split_bf2(v, 0.0f, hi, lo);
            M2h[r * ms + c] = (uint16_t)hi;
            M2l[r * ms + c] = (uint16_t)lo;
          }
        }
      };
      using std::integral_constant;
      if (Smpad <= 32) build_m(integral_constant<int, 5>{}, integral_constant<int, 1>{});
      else if (Smpad <= 64) build_m(integral_constant<int, 6>{}, integral_constant<int, 4>{});
      else build_m(integral_constant<int, 7>{}, integral_constant<int, 16>{});
    }
    for (int g2 = lb; g2 < kL2Groups; g2 += nwg) {
      const int t = 16 * g2 + r16;  // this lane's output column
      // su and bias of this lane's outputs (rows 16 w + 4 q + j), before the poll
      float suo[4], bio[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 16 * w + 4 * q + j;
        const int i = (w < nl1 && r < Sm) ? out_elem(r, t) : 0;
        suo[j] = load_su(J.su, SB, i);
        bio[j] = at_off(bsrc, (uint32_t)i);
      }
      float hv[kMaxB][2];
      poll_columns(J.h2t, J.m, Sm, A.B, g2, tid, tag, hv);
      if (g2 != lb) __syncthreads();  // the previous group's reads of the staged columns are done
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int v = tid + kThreads * k, c = v >> 4, tt = v & 15;
        if (c < Smpad) {
#pragma unroll
          for (int b = 0; b < kMaxB; ++b) {
            uint32_t hi, lo;
            split_bf2(hv[b][k], 0.0f, hi, lo);
            HBh[(b * 16 + tt) * ms + c] = (uint16_t)hi;
            HBl[(b * 16 + tt) * ms + c] = (uint16_t)lo;
          }
        }
      }
      __syncthreads();  // M (the first time) and the staged columns complete
      if (w < nl1) {
        auto row = [&](const int b) {
          floatx4 acc = {0.f, 0.f, 0.f, 0.f};
          for (int kb = 0; kb < (Smpad >> 5); ++kb) {
            const int k0 = 32 * kb + 8 * q;
            const bf16x8 ah = lds_bf16x8(M2h + (16 * w + r16) * ms + k0);
            const bf16x8 bh = lds_bf16x8(HBh + (b * 16 + r16) * ms + k0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, acc, 0, 0, 0);
            acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, lds_bf16x8(HBl + (b * 16 + r16) * ms + k0), acc, 0,
                                                          0, 0);
            if (m_lo)
              acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lds_bf16x8(M2l + (16 * w + r16) * ms + k0), bh, acc, 0,
                                                            0, 0);
          }
          const float mul = mul0 * (b == 0 ? emul0 : emul1);
          float out[1][4];
          int oidx[1][4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 16 * w + 4 * q + j;
            oidx[0][j] = r < Sm ? out_elem(r, t) : -1;
            out[0][j] = apply_su(acc[j] * mul, suo[j], SB, oidx[0][j]) + (has_bias ? bio[j] : 0.0f);
          }
          store_outputs(J.y, A.y_dtype, (int64_t)b * J.ldy, oidx, out);
        };
        row(0);
        if (A.B > 1) row(1);
      }
    }
  }
  // every slot this work-group polls has been read: the next launch's tag
  // follows this one
  finish_tagged_launch(J.epoch, tag, g, TagWs{J.epoch + kWrapWord, A.ws, A.ws_words, J.ntail},
                       reinterpret_cast<int*>(lds));
}

}  // namespace

// Host launcher used by qs_linear_forward and qs_linear_forward_group
// (qs_linear.hip).  The CUs are shared between the linears in proportion to
// their rows; each linear's work-groups form a contiguous block of the grid.
namespace {
template <bool HAS2, bool SB, int XT>
int launch_fused_variant(const FusedArgs& A, int wg, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop) {
  static int attr_done = 0;
  if (!attr_done) {
    hipFuncAttributes fa{};
    QS_HIP(hipFuncGetAttributes(&fa, (const void*)linear_fused_kernel<HAS2, SB, XT>));
    QS_REQUIRE(fa.sharedSizeBytes == 0, "linear_fused_kernel: static LDS would move the LUT off address 0");
    QS_HIP(hipFuncSetAttribute((const void*)linear_fused_kernel<HAS2, SB, XT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               kLdsBytes));
    attr_done = 1;
  }
  hipExtLaunchKernelGGL((linear_fused_kernel<HAS2, SB, XT>), dim3((unsigned)wg), dim3(kThreads), kLdsBytes, stream,
                        ev_start, ev_stop, 0, A);
  QS_LAUNCHED("linear_fused_kernel");
  return QS_OK;
}
}  // namespace

// Slice groups first as few as fit (W = ceil(S / SG) <= 16), then more of
// them where P phases then keep a tenth more of the 16 waves busy (S = 20:
// 5 groups of 4 slices x 4 phases, all 16 waves, against 2 groups of 10).
FusedPlan fused_plan(int S) {
  const int base = (S + kWaves - 1) / kWaves;
  FusedPlan best{0, 0, 0};
  double best_eff = 0.0;
  for (int sg = base; sg <= 2 * base + 3 && sg <= S; ++sg) {
    const int w = (S + sg - 1) / sg;
    const int fit = kWaves / w;
    const int p = fit >= 4 ? 4 : fit >= 2 ? 2 : 1;
    const double eff = (double)S * p / (double)(kWaves * sg);  // busy share of the waves
    if (best.SG == 0 || eff > best_eff + 0.1) {
      best = FusedPlan{sg, w, p};
      best_eff = eff;
    }
  }
  return best;
}

int launch_linear_fused(const void* x, int x_dtype, int64_t ldx, int B, int n, int pn, const float* Kn, int y_dtype,
                        int sbits, int count, const FusedJobDesc* jobs, int S, const FusedPlan& plan, int ncu,
                        hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop, const FusedPre* pre) {
  const int SG = plan.SG, W = plan.W, P = plan.P;
  QS_REQUIRE(count >= 1 && count <= kMaxJobs, "1..%d linears per launch", kMaxJobs);
  QS_REQUIRE(fused_eligible(B, n, x_dtype, pn) && SG * W >= S && W * P <= kWaves && (P == 1 || P == 2 || P == 4) &&
                 P * B <= 8,
             "one-launch forward: B %d, n %d (dtype %d) outside its shapes", B, n, x_dtype);
  FusedArgs A{};
  A.x = x;
  A.x_dtype = x_dtype;
  QS_REQUIRE(fused_x_aligned(x, x_dtype, ldx), "one-launch forward: x rows must be 8-byte (fp32: 16-byte) aligned");
  A.ldx = ldx;
  A.B = B;
  A.n = n;
  A.Sn = n / 256;
  A.lsh_n = log2_exact(n / pn / 256);
  A.pn = pn;
  A.Kn = Kn;
  A.scale_n = inv_sqrt_len(n / pn);
  A.S = S;
  A.SG = SG;
  A.W = W;
  A.P = P;
  A.lgP = P == 4 ? 2 : P == 2 ? 1 : 0;
  A.y_dtype = y_dtype;
  A.sbits = sbits;
  A.njobs = count;
  int64_t mtot = 0;
  for (int g = 0; g < count; ++g) mtot += jobs[g].m;
  const bool has2 = jobs[0].codes1 != nullptr;
  int wg = 0;
  for (int g = 0; g < count; ++g) {
    const FusedJobDesc& d = jobs[g];
    QS_REQUIRE((d.codes1 != nullptr) == has2, "all linears of a launch need the same number of stages");
    FusedJob& J = A.job[g];
    J.sv = d.sv;
    J.codes0 = static_cast<const uint16_t*>(d.codes0);
    J.codes1 = static_cast<const uint8_t*>(d.codes1);
    J.m = (int)d.m;
    const int RB = (int)(d.m / 16);
    int Gr = (int)((double)ncu / SG * (double)d.m / (double)mtot);
    if (Gr < 1) Gr = 1;
    if (Gr > RB) Gr = RB;
    J.Gr = Gr;
    J.wg0 = wg;
    wg += Gr * SG;
    J.s0 = d.s0;
    J.s1 = d.s1;
    J.y1p = d.y1p;
    J.y1t = d.y1t;
    J.epoch = d.epoch;
    J.xmul = d.xmul;
    J.h2t = d.h2t;
    J.out_in_kernel = fused_output_in_kernel(d.m, d.pm);
    if (J.out_in_kernel) {
      J.Sm = (int)(d.m / 256);
      J.lsh_m = log2_exact(d.m / d.pm / 256);
      // tail work-groups: the first one (m <= 4096), else the first
      // kL2Groups (or all, if fewer)
      J.ntail = J.Sm <= kWaves ? 1 : (Gr * SG < kL2Groups ? Gr * SG : kL2Groups);
      // the wrap word sits kWrapWord words past the epoch word, in one
      // workspace for every job of the launch
      QS_REQUIRE(d.tw.wrap == d.epoch + kWrapWord && d.tw.base && d.tw.words > kWsHeaderWords,
                 "job %d: no workspace for the tags", g);
      QS_REQUIRE(!A.ws || (A.ws == d.tw.base && A.ws_words == d.tw.words), "job %d: another workspace", g);
      A.ws = d.tw.base;
      A.ws_words = d.tw.words;
    }
    J.pm = d.pm;
    J.Km = d.Km;
    J.scale_m = inv_sqrt_len(d.m / d.pm);
    J.layer_scale = d.layer_scale;
    J.su = d.su;
    J.bias = d.bias;
    J.y = d.y;
    J.ldy = d.ldy;
  }
  int xt = x_dtype == QS_DTYPE_BF16 ? 0 : x_dtype == QS_DTYPE_F16 ? 1 : 2;
  if (pre) {
    QS_REQUIRE(x_dtype == QS_DTYPE_BF16 && pre->kind == QS_PREOP_RMSNORM,
               "one-launch forward: the norm pre-operation needs bf16 rows");
    xt = 3;
    A.x2 = static_cast<const uint16_t*>(pre->x2);
    A.ldx2 = pre->ldx2;
    A.nw = static_cast<const uint16_t*>(pre->weight);
    A.h_out = static_cast<uint16_t*>(pre->h_out);
    A.ldo = pre->ldo;
    A.eps = pre->eps;
  }
#define QS_FUSED_XT(H, SBITS)                                                          \
  (xt == 0 ? launch_fused_variant<H, SBITS, 0>(A, wg, stream, ev_start, ev_stop)      \
   : xt == 1 ? launch_fused_variant<H, SBITS, 1>(A, wg, stream, ev_start, ev_stop)    \
   : xt == 2 ? launch_fused_variant<H, SBITS, 2>(A, wg, stream, ev_start, ev_stop)    \
             : launch_fused_variant<H, SBITS, 3>(A, wg, stream, ev_start, ev_stop))
  if (has2) return sbits ? QS_FUSED_XT(true, true) : QS_FUSED_XT(true, false);
  return sbits ? QS_FUSED_XT(false, true) : QS_FUSED_XT(false, false);
#undef QS_FUSED_XT
}

bool fused_output_in_kernel(int64_t m, int pm) { return m % 256 == 0 && m / 256 <= kMaxSF && m / pm >= 256; }

bool fused_x_aligned(const void* x, int x_dtype, int64_t ldx) {
  const uintptr_t align = x_dtype == QS_DTYPE_F32 ? 16 : 8;
  return (reinterpret_cast<uintptr_t>(x) % align) == 0 && ldx % 4 == 0;
}

bool fused_eligible(int64_t batch, int64_t n, int x_dtype, int pn) {
  const int64_t smax = x_dtype == QS_DTYPE_BF16 ? kMaxSF : kMaxSF / 2;
  return batch >= 1 && batch <= kMaxB && n % 256 == 0 && n / 256 <= smax && n / pn >= 256;
}

}  // namespace qs
