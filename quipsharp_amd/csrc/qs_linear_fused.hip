// One-launch quantized-linear forward for decode-size batches (B <= 2,
// n <= 12288), the path QuantizedLinear.forward takes at generation time
// (quipsharp/checkpoint.py:141-146 -> quipsharp/quantize.py:116-124).
//
// Transforms.  A length-n transform T_n = K_p (x) H_L (n = p L, L = 2^k >= 256)
// is split as T_n = M (x) H_256 over the index i = 256 c + t: a 256-point
// Walsh-Hadamard inside each chunk c (one wave, four values per lane, two
// stages in registers and six across lanes with DPP / permlane exchanges, no
// barrier), then the S x S matrix M = K_p (x) H_{L/256} (S = n / 256 <= 48)
// across chunks on the matrix cores (bf16 hi + lo operands, fp32 accumulate).
//
// Work-group j owns one slice group (up to 16 slices of 256 input columns,
// one per wave) and a strided set of 16-row blocks, so each wave's activation
// operand stays in registers for the whole launch.  Per work-group:
//   1. issue the activation loads, then the abs-table and K loads; the first
//      code tiles are requested once the activations have arrived, and the
//      byte-per-value half-codeword LUTs are built after the input transform;
//   2. input transform (every work-group; only its own 16 rows of M): chunks
//      -> LDS, chunk stage, fp16 operand rows scaled by 2^-e (e from the row
//      norm) plus the per-group sums for the +-1/4 shift term, whose
//      -1/4 sum_g S_g part is folded in per slice;
//   3. per row block: 8 MFMAs (+1 for the shift, +8 for an E8 1-bit second
//      stage) into one of 8 LDS slots; every 8 row blocks (and after the
//      last) the slots are reduced across the waves and the partial sums go
//      to the workspace as write-through stores;
//   4. completion: the partial sums go out as 64-bit slots {value, launch
//      tag}, one agent-scope store each, and the work-group is done; the
//      job's first work-group, after its own row blocks, polls the slots until
//      every one carries this launch's tag, then applies S_u T_m(.) + bias
//      with the same chunk scheme (every m of the scheme: m = p 2^k, 256 | m,
//      m <= 12288) and stores the tag as the workspace's new epoch.
//
// Cross-work-group visibility.  Slots are written with agent-scope relaxed
// atomic stores and read with agent-scope relaxed atomic loads, which on
// gfx950 are write-through / read-through at the device coherence point (no
// per-XCD L2 copy is involved).  A 64-bit atomic store makes value and tag
// visible together, so the reader needs no counter and the writers no wait
// for their stores to complete (that wait plus a counter round trip cost
// ~3 us per launch).  Only the polling work-group ever waits, and only for
// work-groups that never wait themselves, so the launch cannot deadlock
// whatever order its work-groups are dispatched in; the poll is bounded
// (kMaxPolls, NaN outputs if exceeded).
#include <hip/hip_ext.h>

#include "qs_forward_dev.h"
#include "qs_linear_dev.h"

namespace qs {
namespace {


constexpr int kThreads = kFwdThreads;
constexpr int kMaxB = 2;
constexpr int kPrefetch = 4;
constexpr int kMaxJobs = QS_MAX_GROUP;
constexpr int kXStride = 264;               // halves per slice row of the fp16 operand buffer

// One linear of a launch.  Linears in one launch share the input x (and n);
// each has its own codes, signs, scales, output and workspace region.
struct FusedJob {
  const float* sv;
  const uint16_t* codes0;
  const uint8_t* codes1;
  int m, Gr, wg0;      // rows; row-block stride; first work-group of this linear
  float s0, s1;
  float* y1p;          // [SG][B][m] fp32 partials (output transform in a separate kernel)
  unsigned long long* y1t;  // [SG][B][m] tagged partials (output transform here)
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
  int x_vec;  // rows of 4 elements can be loaded as one 8- or 16-byte word
  int64_t ldx;
  int B;
  int n, Sn, lsh_n, pn;
  const float* Kn;
  float scale_n;
  int S, SG, W;
  int y_dtype;
  int sbits;  // su, sv of every job are packed sign bits
  int njobs;
  FusedJob job[kMaxJobs];
};

// LDS layout (bytes).  The abs-table staging area aliases the reduction
// buffer (the table is dead before the first row block); the output
// transform of the last work-group reuses the LUT and Y regions.
constexpr int kOffHi = 0;                                   // 4096 x uint32 (four fp16 high bytes)
constexpr int kOffLo = 16384;                               // 4096 x uint32
constexpr int kOffLut1 = 32768;                             // 256 x uint4
constexpr int kRedSlots = 8;                                // row blocks reduced together
constexpr int kRedSlot = kWaves * 16 * kMaxB;               // floats per slot: [wave][row][batch]
constexpr int kOffRed = kOffLut1 + 4096;                    // kRedSlots x kRedSlot floats
constexpr int kOffMin = kOffRed + kRedSlots * kRedSlot * 4;  // 2 x 16 x kMStride bf16: input chunk stage (hi, lo)
constexpr int kOffTab = kOffRed;                            // 256 x uint4 (table staging, before the row blocks)
constexpr int kOffXH = kOffMin + 2 * 16 * kMStride * 2;     // kMaxB x 16 x kXStride halves
constexpr int kOffXS = kOffXH + kMaxB * 16 * kXStride * 2;  // kMaxB x 16 x 32 halves (group sums)
constexpr int kOffY = kOffXS + kMaxB * 16 * 32 * 2;          // kMaxS x kYStride floats
constexpr int kOffMisc = kOffY + kMaxS * kYStride * 4;      // row norms (16 floats), last-group flag
constexpr int kLdsBytes = kOffMisc + 128;
static_assert(kLdsBytes <= 160 * 1024 - 128, "LDS budget");
// Output chunk stage (last work-group, the LUTs are dead): the chunk matrix
// M as bf16 hi / lo parts, rows and columns padded with zeros.
constexpr int kOffMh = 0;
constexpr int kOffMl = kOffMh + kMBytes;
static_assert(kOffMl + kMBytes <= kOffLut1, "M fits the LUT region");
// Split output transform (m > 4096): one 16-chunk tile of M . Y1 per
// work-group, staged here for the per-chunk 256-point transforms (the LUT,
// table and reduction regions are dead by then; Y is untouched).
constexpr int kOffZ2 = 16384;
static_assert(kOffZ2 >= kOffMl + kMBytes && kOffZ2 + 16 * kYStride * 4 <= kOffY, "tile stage fits below Y");
static_assert(kRedSlots * kRedSlot * 4 >= 4096, "table staging fits the reduction buffer");
static_assert(kRedSlots * 16 * kMaxB * 4 == kThreads && kRedSlots * 16 * 8 == kThreads,
              "one reduction pass: 8 threads per output at B = 1, 4 at B = 2");


// OCPW: output side.  1 (m <= 4096): the job's first work-group applies the
// whole output transform, 256-point transforms first.  3 (m <= 12288): the
// output transform is split over the job's first ceil(m / 4096) work-groups,
// M first (see the completion section).
template <bool HAS2, bool SB, int OCPW>
__global__ __launch_bounds__(kThreads) void linear_fused_kernel(FusedArgs A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint32_t* lut_hi = reinterpret_cast<uint32_t*>(lds + kOffHi);
  uint32_t* lut_lo = reinterpret_cast<uint32_t*>(lds + kOffLo);
  uint4* lut1 = reinterpret_cast<uint4*>(lds + kOffLut1);
  uint4* tab16 = reinterpret_cast<uint4*>(lds + kOffTab);
  float* red = reinterpret_cast<float*>(lds + kOffRed);
  uint16_t* MinH = reinterpret_cast<uint16_t*>(lds + kOffMin);
  uint16_t* MinL = MinH + 16 * kMStride;
  _Float16* XH = reinterpret_cast<_Float16*>(lds + kOffXH);
  _Float16* XS = reinterpret_cast<_Float16*>(lds + kOffXS);
  float* Y = reinterpret_cast<float*>(lds + kOffY);
  float* wsum = reinterpret_cast<float*>(lds + kOffMisc);

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
  const int sl = sg * A.W + w;
  const bool active = w < A.W && sl < A.S;
  const LaneX lx = lane_x_init();

  // 1. loads: the activations first (the transform waits for them), then the
  //    abs table and K; the code tiles once the activations are in, then the
  //    launch tag.  (The table staging below waits for every load issued so
  //    far: the compiler cannot count the activation loads' conditional paths,
  //    so issuing the table first would only delay the activations, and the
  //    tag, read from the device coherence point, would delay the staging.)
  const XSource X{A.x, A.x_dtype, A.x_vec, A.ldx, A.Sn, SB ? 1 : 0};
  XRaw xr;
  load_x_raw(X, J.sv, 0, w, lane, xr);
  uint4 trow = make_uint4(0, 0, 0, 0), t1row = make_uint4(0, 0, 0, 0);  // fp16 table rows
  if (tid < 256) {
    trow = *reinterpret_cast<const uint4*>(kE8Ph.w[tid]);
    if (HAS2) t1row = *reinterpret_cast<const uint4*>(kE81h.w[tid]);
  }
  // this wave's row of the input chunk stage: M[sl][c] for c = lane (Sn <= 48)
  const bool m_ok = active && lane < A.Sn;
  float mk = 1.0f;
  if (A.pn > 1 && m_ok) mk = A.Kn[(sl >> A.lsh_n) * A.pn + (lane >> A.lsh_n)];
  if (tid < 256) {
    tab16[tid] = trow;
    if (HAS2) lut1[tid] = t1row;
  }
  __syncthreads();  // staged table complete
  fill_luts(tab16, lut_hi, lut_lo, tid);
  float xv[kCPW][4];
  finish_x(X, xr, w, lane, xv);
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

  // tag of this launch's partial sums, read (below, after the first code
  // tiles) by every work-group before it stores any slot; the epoch only
  // changes after every slot of the launch has been read
  uint32_t epoch = 0;

  // 2. input transform, one batch row at a time, into fp16 operand rows
  float emul0 = 1.0f, emul1 = 1.0f;  // 2^e of batch rows 0 and 1
  for (int b = 0; b < A.B; ++b) {
    if (b > 0) load_x(X, J.sv, b, w, lane, xv);
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < kCPW; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) ss = __builtin_fmaf(xv[u][j], xv[u][j], ss);
    ss = wave_sum(ss, lx);
    if (lane == 0) wsum[w] = ss;
    h256_chunks(xv, A.Sn, lane, lx);
    if (b == 0) {
      // K (read after the barrier below), before the code loads are issued
      // so these stores do not wait for them
      {
        const int hm = (1 << A.lsh_n) - 1;
        const float v = m_ok ? ((__builtin_popcount(sl & lane & hm) & 1) ? -mk : mk) : 0.0f;
        uint32_t hi, lo;
        split_bf2(v, 0.0f, hi, lo);
        MinH[w * kMStride + lane] = (uint16_t)hi;
        MinL[w * kMStride + lane] = (uint16_t)lo;
      }
      // first code tiles (issued once the activations are in, so the
      // activation loads do not queue behind them)
#pragma unroll
      for (int k = 0; k < kPrefetch; ++k) {
        const uint32_t off = code_off(jr + k * J.Gr);
        pre[k] = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(J.codes0) + off);
        if (HAS2) pre1[k] = *reinterpret_cast<const uint2*>(J.codes1 + off / 2);
      }
      if (J.out_in_kernel) epoch = __hip_atomic_load(J.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (b > 0) __syncthreads();  // the previous row's reads of Y are done
    store_chunks(Y, A.Sn, w, lane, xv);
    __syncthreads();  // chunks, norms (and, the first time, the staged table and K) complete
    float norm2 = 0.0f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) norm2 += wsum[i];
    const int e = operand_exponent(norm2);
    if (b == 0) emul0 = ldexpf(1.0f, e);
    else emul1 = ldexpf(1.0f, e);
    const float mul = ldexpf(A.scale_n, -e);
    // chunk stage for this group's 16 slice rows: X2[s][t] = sum_c
    // M[sg W + s][c] Y[c][t]; wave w computes columns t = 16 w + r16, rows
    // s = 4 q + j, and writes them as fp16 operand rows
    {
      const int t = 16 * w + r16;
      floatx4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int kb = 0; kb < ((A.Sn + 31) >> 5); ++kb)
        acc = mstage_step(acc, MinH, MinL, 0, z_operand(Y, A.Sn, t, q, kb), kb, A.pn > 1, q, r16);
      float hs[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const _Float16 h = (_Float16)(acc[j] * mul);
        XH[(b * 16 + 4 * q + j) * kXStride + t] = h;
        hs[j] = (float)h;
      }
      // group sums of the fp16 values, group t / 8: lanes r16 & 7 = 0..7
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        hs[j] += lane_xor<1>(hs[j], lx);
        hs[j] += lane_xor<2>(hs[j], lx);
        hs[j] += lane_xor<4>(hs[j], lx);
      }
      if ((r16 & 7) == 0) {
#pragma unroll
        for (int j = 0; j < 4; ++j) XS[(b * 16 + 4 * q + j) * 32 + (t >> 3)] = (_Float16)hs[j];
      }
    }
  }
  __syncthreads();  // operand rows complete
  // MFMA operand of lane (q, b = r16): columns 64q..64q+63 of this wave's slice
  const half8 hzero = {0, 0, 0, 0, 0, 0, 0, 0};
  half8 xb[8];
  half8 xs = hzero;
  float slice_shift = 0.0f;  // sum_g S_g over the lane's 64 columns, batch row r16
#pragma unroll
  for (int c = 0; c < 8; ++c) xb[c] = hzero;
  if (active && r16 < A.B) {
    const _Float16* row = XH + (r16 * 16 + w) * kXStride + 64 * q;
#pragma unroll
    for (int c = 0; c < 8; ++c) xb[c] = *reinterpret_cast<const half8*>(row + 8 * c);
    xs = *reinterpret_cast<const half8*>(XS + (r16 * 16 + w) * 32 + 8 * q);
#pragma unroll
    for (int c = 0; c < 8; ++c) slice_shift += (float)xs[c];
  }
  // slice total of S_g over the four q-lanes of batch row r16
  slice_shift += lane_xor<16>(slice_shift, lx);
  slice_shift += lane_xor<32>(slice_shift, lx);
  if (lb == 0 && tid < A.B) J.xmul[tid] = tid == 0 ? emul0 : emul1;

  const uint32_t tag = J.out_in_kernel ? next_tag(epoch) : 0u;

  // 3. row blocks
  const int nw = A.S - sg * A.W < A.W ? A.S - sg * A.W : A.W;
  int k = 0;  // row blocks done: selects the reduction slot
  for (int rb0 = jr; rb0 < RB; rb0 += kPrefetch * J.Gr) {
#pragma unroll
  for (int u = 0; u < kPrefetch; ++u) {
    // every ring step runs (the ring registers are never copied); a step
    // past the last row block only refills its entry
    const int rb = rb0 + u * J.Gr;
    const bool valid = rb < RB;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    floatx4 accs = {0.f, 0.f, 0.f, 0.f};
    floatx4 acc2 = {0.f, 0.f, 0.f, 0.f};
    const uint4 cw = pre[u];
    const uint2 cw1 = pre1[u];
    if (valid) {
      // (idle waves decode tile 0 with a zero operand; their results are
      // not stored)
      const uint32_t wd[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const half8 av = decode_code(wd[c >> 1], c, kOffHi, kOffLo);
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, xb[c], acc, 0, 0, 0);
        if (HAS2) {
          const uint32_t idx = ((c < 4 ? cw1.x : cw1.y) >> (8 * (c & 3))) & 0xFFu;
          acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, lut1[idx]), xb[c], acc2, 0, 0,
                                                          0);
        }
      }
      accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(shift_operand(wd), xs, accs, 0, 0, 0);
    }
    {
      // refill this ring entry (its tile is consumed) with the tile
      // kPrefetch row blocks ahead
      const uint32_t off = code_off(rb + kPrefetch * J.Gr);
      pre[u] = *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(J.codes0) + off);
      if (HAS2) pre1[u] = *reinterpret_cast<const uint2*>(J.codes1 + off / 2);
    }
    // partial of this slice for rows 4q..4q+3, batch column r16, into this
    // row block's slot; the slots are reduced across the waves every
    // kRedSlots row blocks (and after the last), so the waves decode without
    // a barrier per row block
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
    if (valid && (slot == kRedSlots - 1 || rb + J.Gr >= RB)) {
      __syncthreads();
      // output o = (s * 16 + row) * B + b of slot s <= slot, summed over the
      // waves by tpo threads (waves part, part + tpo, ...), then across them;
      // tpo depends on B only, so every output is summed in the same order
      // whatever the number of row blocks pending
      const int nout = (slot + 1) * 16 * A.B;
      const int tpo = A.B == 1 ? 8 : 4;  // kThreads / (kRedSlots * 16 * B)
      const int o = tid / tpo, part = tid - o * tpo;
      float v = 0.0f;
      int s = 0, row = 0, bc = 0;
      if (o < nout) {
        s = o / (16 * A.B);
        const int rr = o - s * 16 * A.B;
        row = rr / A.B;
        bc = rr - row * A.B;
        for (int ww = part; ww < nw; ww += tpo) v += red[s * kRedSlot + (ww * 16 + row) * kMaxB + bc];
      }
      v += lane_xor<1>(v, lx);
      v += lane_xor<2>(v, lx);
      if (tpo == 8) v += lane_xor<4>(v, lx);
      if (o < nout && part == 0) {
        const int rbs = rb - (slot - s) * J.Gr;  // row block of slot s
        const size_t idx = ((size_t)sg * A.B + bc) * J.m + rbs * 16 + row;
        if (J.out_in_kernel)
          __hip_atomic_store(&J.y1t[idx], tagged(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          J.y1p[idx] = v;  // read by a separate output kernel after this one
      }
      __syncthreads();  // the slots are free again
    }
    k += valid;
  }
  }

  // 4. completion: the tail work-group(s) of the job wait for every tagged
  //    partial sum of this launch and apply the output transform
  if (!J.out_in_kernel) return;
  if (OCPW == 1 || J.Sm <= kWaves) {
    // m <= 4096, in either instantiation (a linear's output does not depend
    // on the others of its group): the job's first work-group, one output
    // chunk per wave, 256-point transforms first
    if (lb != 0) return;
    constexpr int OC = 1;
    // Output chunk stage on the matrix cores (mstage_tile): lane (q, r16) of
    // wave w produces column t = 16 w + r16 of rows r = 16 a + 4 q + j.
    const int Sm = J.Sm;
    const int t = 16 * w + r16;
    // Loads, in the order they are waited for: the K entries of M (odd
    // factor), the first partial-sum slots, su and bias, all in flight
    // together (unconditional loads from valid addresses, selected where they
    // are used: a load under a branch is waited for at the branch's end).
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
          const int ii = r < Sm ? 256 * r + t : 0;
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
      poll_issue(J.y1t, J.m, Sm, A.B, b, w, lane, tag, ps);
      if (b == 0) {
        load_su_bias();
        mmat_store(kmv, Sm, J.lsh_m, Mh, Ml, tid);  // waits for the K loads only
      }
      float zv[OC][4];
      poll_finish(J.y1t, J.m, Sm, A.SG, A.B, b, w, lane, tag, ps, zv);
      h256_chunks(zv, Sm, lane, lx);
      if (b > 0) __syncthreads();  // the previous row's reads of Y are done
      store_chunks_lanes(Y, Sm, w, lane, zv);
      __syncthreads();  // chunks (and, the first time, M) complete
      const float mul = mul0 * (b == 0 ? emul0 : emul1);
      floatx4 acc[OC];
#pragma unroll
      for (int a = 0; a < OC; ++a) acc[a] = floatx4{0.f, 0.f, 0.f, 0.f};
      for (int kb = 0; kb < nkb; ++kb) {
        const ZOperand z = z_operand(Y, Sm, t, q, kb);
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
          oidx[a][j] = r < Sm ? 256 * r + t : -1;
          out[a][j] = apply_su(acc[a][j] * mul, suo[a][j], SB, oidx[a][j]) + (has_bias ? bio[a][j] : 0.0f);
        }
      store_outputs(yp, ydt, (int64_t)b * ldy, oidx, out);
    };
    row(0);
    if (A.B > 1) row(1);
  } else if constexpr (OCPW > 1) {
    // T_m = M (x) H_256 = (I (x) H_256)(M (x) I): output chunk r is
    // H_256(z_r) with z_r = sum_c M[r][c] y1_c.  Work-group lb < ntile of the
    // job takes the 16-chunk tile lb (tiles lb + nwg, ... when the job has
    // fewer work-groups than tiles): it polls every slot of y1, stages the
    // chunks in LDS, computes its tile of M . Y1 on the matrix cores (wave w:
    // columns t = 16 w + r16), stages it, and each wave transforms output
    // chunk r = 16 tile + w and stores it.  Each tail work-group transforms
    // one chunk per wave instead of one work-group transforming all of them.
    const int Sm = J.Sm;
    const int ntile = (Sm + 15) >> 4;
    const int nwg = J.Gr * A.SG;
    if (lb >= ntile) return;
    const int t = 16 * w + r16;
    float* Z2 = reinterpret_cast<float*>(lds + kOffZ2);
    uint16_t* Mh = reinterpret_cast<uint16_t*>(lds + kOffMh);
    uint16_t* Ml = reinterpret_cast<uint16_t*>(lds + kOffMl);
    float kmv[3];
    mmat_load(kmv, Sm, J.lsh_m, J.pm, J.Km, tid);
    const float* const bsrc = J.bias ? J.bias : reinterpret_cast<const float*>(J.y1t);  // dummy: never used
    const bool has_bias = J.bias != nullptr;
    const float mul0 = J.scale_m * J.layer_scale;
    const int nkb = (Sm + 31) >> 5;
    bool first = true;
    for (int tile = lb; tile < ntile; tile += nwg) {
      const int r = 16 * tile + w;  // this wave's output chunk
      const bool rv = r < Sm;
      // su and bias of the wave's output elements 256 r + lane + 64 j
      // (issued before the polling; dummy element 0 for r >= Sm)
      float suo[4], bio[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = rv ? 256 * r + lane + 64 * j : 0;
        suo[j] = load_su(J.su, SB, i);
        bio[j] = at_off(bsrc, (uint32_t)i);
      }
      auto row = [&](const int b) {
        PollState<kCPW> ps;
        poll_issue(J.y1t, J.m, Sm, A.B, b, w, lane, tag, ps);
        if (first) mmat_store(kmv, Sm, J.lsh_m, Mh, Ml, tid);  // waits for the K loads only
        float zv[kCPW][4];
        poll_finish(J.y1t, J.m, Sm, A.SG, A.B, b, w, lane, tag, ps, zv);
        if (!first) __syncthreads();  // the previous tile's / row's reads of Y and Z2 are done
        first = false;
        store_chunks_lanes(Y, Sm, w, lane, zv);
        __syncthreads();  // chunks of y1 (and, the first time, M) complete
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        for (int kb = 0; kb < nkb; ++kb)
          acc = mstage_step(acc, Mh, Ml, 16 * tile, z_operand(Y, Sm, t, q, kb), kb, J.pm > 1, q, r16);
#pragma unroll
        for (int j = 0; j < 4; ++j) Z2[(4 * q + j) * kYStride + t] = acc[j];
        __syncthreads();  // the tile of M . Y1 is complete
        if (rv) {
          float v[1][4];
#pragma unroll
          for (int j = 0; j < 4; ++j) v[0][j] = Z2[w * kYStride + lane + 64 * j];
          h256<1>(v, lane, lx);
          const float mul = mul0 * (b == 0 ? emul0 : emul1);
          float out[1][4];
          int oidx[1][4];
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            oidx[0][j] = 256 * r + lane + 64 * j;
            out[0][j] = apply_su(v[0][j] * mul, suo[j], SB, oidx[0][j]) + (has_bias ? bio[j] : 0.0f);
          }
          store_outputs(J.y, A.y_dtype, (int64_t)b * J.ldy, oidx, out);
        }
      };
      row(0);
      if (A.B > 1) row(1);
    }
  }
  // every slot of this launch has been read (by this work-group; any tail
  // work-group may store it, all store the same): the next launch's tag
  // follows this one
  if (tid == 0) __hip_atomic_store(J.epoch, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// Host launcher used by qs_linear_forward and qs_linear_forward_group
// (qs_linear.hip).  The CUs are shared between the linears in proportion to
// their rows; each linear's work-groups form a contiguous block of the grid.
namespace {
template <bool HAS2, bool SB, int OCPW>
int launch_fused_variant(const FusedArgs& A, int wg, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop) {
  static int attr_done = 0;
  if (!attr_done) {
    hipFuncAttributes fa{};
    QS_HIP(hipFuncGetAttributes(&fa, (const void*)linear_fused_kernel<HAS2, SB, OCPW>));
    QS_REQUIRE(fa.sharedSizeBytes == 0, "linear_fused_kernel: static LDS would move the LUT off address 0");
    QS_HIP(hipFuncSetAttribute((const void*)linear_fused_kernel<HAS2, SB, OCPW>, hipFuncAttributeMaxDynamicSharedMemorySize,
                               kLdsBytes));
    attr_done = 1;
  }
  hipExtLaunchKernelGGL((linear_fused_kernel<HAS2, SB, OCPW>), dim3((unsigned)wg), dim3(kThreads), kLdsBytes, stream,
                        ev_start, ev_stop, 0, A);
  QS_LAUNCHED("linear_fused_kernel");
  return QS_OK;
}
}  // namespace

int launch_linear_fused(const void* x, int x_dtype, int64_t ldx, int B, int n, int pn, const float* Kn, int y_dtype,
                        int sbits, int count, const FusedJobDesc* jobs, int S, int SG, int W, int ncu, hipStream_t stream,
                        hipEvent_t ev_start, hipEvent_t ev_stop) {
  QS_REQUIRE(count >= 1 && count <= kMaxJobs, "1..%d linears per launch", kMaxJobs);
  FusedArgs A{};
  A.x = x;
  A.x_dtype = x_dtype;
  {
    const uintptr_t align = x_dtype == QS_DTYPE_F32 ? 16 : 8;
    A.x_vec = (reinterpret_cast<uintptr_t>(x) % align) == 0 && ldx % 4 == 0;
  }
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
    J.out_in_kernel = chunk_transform_fits(d.m, d.pm);
    if (J.out_in_kernel) {
      J.Sm = (int)(d.m / 256);
      J.lsh_m = log2_exact(d.m / d.pm / 256);
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
  // output chunks per wave of the widest in-kernel output transform
  int sm_max = 0;
  for (int g = 0; g < count; ++g)
    if (A.job[g].out_in_kernel && A.job[g].Sm > sm_max) sm_max = A.job[g].Sm;
  if (sm_max <= kWaves) {
    if (has2) return sbits ? launch_fused_variant<true, true, 1>(A, wg, stream, ev_start, ev_stop)
                           : launch_fused_variant<true, false, 1>(A, wg, stream, ev_start, ev_stop);
    return sbits ? launch_fused_variant<false, true, 1>(A, wg, stream, ev_start, ev_stop)
                 : launch_fused_variant<false, false, 1>(A, wg, stream, ev_start, ev_stop);
  }
  if (has2) return sbits ? launch_fused_variant<true, true, kCPW>(A, wg, stream, ev_start, ev_stop)
                         : launch_fused_variant<true, false, kCPW>(A, wg, stream, ev_start, ev_stop);
  return sbits ? launch_fused_variant<false, true, kCPW>(A, wg, stream, ev_start, ev_stop)
               : launch_fused_variant<false, false, kCPW>(A, wg, stream, ev_start, ev_stop);
}

bool fused_output_in_kernel(int64_t m, int pm) { return chunk_transform_fits(m, pm); }

bool fused_eligible(int64_t batch, int64_t n, int64_t m, int pn) {
  (void)m;
  return batch >= 1 && batch <= kMaxB && chunk_transform_fits(n, pn);
}

}  // namespace qs
