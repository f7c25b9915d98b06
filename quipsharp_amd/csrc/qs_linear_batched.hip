// Quantized-linear forward for batches of 3..16 rows per pass (prefill
// chunks, batched decode), the path QuantizedLinear.forward takes for more
// than two activation rows (quipsharp/checkpoint.py:141-146 ->
// quipsharp/quantize.py:116-124), on the chunk scheme of qs_chunk_dev.h.
// Two launches per pass (three where the output transform cannot run in the
// decode-matvec):
//   bx_kernel  input transform, one work-group per batch row: activation
//              chunks times S_v, 256-point transforms in registers, the chunk
//              stage on the matrix cores, fp16 operand (scaled by 2^-e from the
//              row norm) and its group sums to the workspace, both in the
//              fragment-major order the MFMA B operand is read in;
//   bm_kernel  decode-matvec: work-group j owns one slice group (one 256-column
//              slice per wave) and a strided set of 16-row blocks; each wave's
//              operand (16 batch rows of its slice) stays in registers, codes
//              stream through a 2-tile prefetch ring, the byte-per-value LUTs
//              feed 16x16x32 MFMAs with all 16 batch columns in use, and the
//              per-wave partials are reduced across the waves every four row
//              blocks into the workspace, as tagged slots when the kernel also
//              applies the output transform (work-group b < B of each linear,
//              after its own row blocks, polls row b's slots and runs
//              by_kernel's row body on them);
//   by_kernel  output transform, one work-group per batch row: partial sums,
//              256-point transforms, chunk stage on the matrix cores,
//              S_u (.) * scales + bias (the wide path, and passes whose
//              decode-matvec cannot take it: bm_tail_eligible).
// Each kernel takes a table of up to QS_MAX_GROUP linears that read the same
// x (their work-groups side by side in one grid), so a group of linears is
// two or three launches in all; bx_kernel and by_kernel also serve the wide
// path and are instantiated for 1, 2 or 3 chunks of 256 per wave.
#include <hip/hip_ext.h>

#include "qs_forward_dev.h"
#include "qs_linear_dev.h"
#include "qs_preop_dev.h"

namespace qs {
namespace {

constexpr int kThreads = kFwdThreads;
constexpr int kTB = 16;  // batch rows per pass (the MFMA N dimension)
constexpr int kPrefetch = 2;  // code tiles in flight per wave (deeper rings measured slower)

// ---------------------------------------------------------------------------
// input transform
// ---------------------------------------------------------------------------
// One linear of an input-transform launch (its own signs and operand); the
// linears of a launch share x, n and the transform.
struct BxJob {
  const float* sv;
  _Float16* x2h;  // [B][n] fp16 operand, index 256 slice + t
  _Float16* sg;   // [B][n / 8] sums of 8 consecutive operand values
  float* xmul;    // [B] 2^e
};

struct BxArgs {
  const void* x;
  int x_dtype, x_vec;
  int64_t ldx;
  int B;          // rows
  int n, Sn, lsh_n, pn;
  const float* Kn;
  float scale_n;
  int frag;       // x2h and sg fragment-major (wide GEMM operands; sg / 4)
  int sbits;      // sv of every linear is packed sign bits
  int per;        // work-groups per linear: linear blockIdx / per
  BxJob job[QS_MAX_GROUP];
  // RMSNorm pre-operation (PRE kernels): x is the residual stream h (bf16
  // rows, 8-byte loads), the linears read bf16(nw * bf16(h' * rs)) of
  // h' = bf16(h + x2) (x2 may be null), and the first linear's work-groups
  // write h' to h_out (may be null)
  const uint16_t* x2;
  int64_t ldx2;
  const uint16_t* nw;
  uint16_t* h_out;
  int64_t ldo;
  float eps;
};

// LDS of the per-row transform kernels holding CPW chunks per wave (S <= 16
// CPW): the chunk rows, then the chunk matrix M as bf16 hi / lo, then the row
// norm parts.  One chunk per wave (n <= 4096) keeps the registers and LDS of
// a work-group small enough for two per CU.
template <int CPW>
struct RowLds {
  static constexpr int kY = 0;
  static constexpr int kMh = kY + 16 * CPW * kYStride * 4;
  static constexpr int kMl = kMh + kMBytes;
  static constexpr int kMisc = kMl + kMBytes;
  static constexpr int kPre = kMisc + 4 * kWaves;  // the pre-operation's wave sums
  static constexpr int kTotal = kPre + 4 * kWaves;
};
static_assert(16 * kCPW >= kMaxS, "chunk rows");
inline int chunks_per_wave(int64_t S) { return S <= kWaves ? 1 : S <= 2 * kWaves ? 2 : 3; }

// Rows b = lb, lb + per, ... of linear blockIdx / per (lb = blockIdx % per):
// the next row's activations are loaded while this row is transformed.
// PRE: each row is first put through the RMSNorm pre-operation -- h' formed
// in this kernel's layout and staged in LDS, its rs taken from there in
// rmsnorm_kernel's layout and order (rms_row_scale), then x' formed element
// by element in this kernel's layout -- so the operand equals that of
// qs_dec_rmsnorm followed by the plain kernel, bit for bit.
template <int CPW, bool SB, bool PRE>
__global__ __launch_bounds__(kThreads) void bx_kernel(BxArgs A) {
  using L = RowLds<CPW>;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  float* Y = reinterpret_cast<float*>(lds + L::kY);
  uint16_t* Mh = reinterpret_cast<uint16_t*>(lds + L::kMh);
  uint16_t* Ml = reinterpret_cast<uint16_t*>(lds + L::kMl);
  float* wsum = reinterpret_cast<float*>(lds + L::kMisc);
  float* pre_wsum = reinterpret_cast<float*>(lds + L::kPre);
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  const LaneX lx = lane_x_init();
  const XSource X{A.x, A.x_dtype, A.x_vec, A.ldx, A.Sn, SB ? 1 : 0};
  const int stride = A.per;
  const int g = (int)blockIdx.x / A.per, lb = (int)blockIdx.x - g * A.per;
  const BxJob& J = A.job[g];

  XRawT<CPW> xr;
  load_x_raw(X, J.sv, lb, w, lane, xr);
  // PRE: the residual delta of row b (with up to two chunks per wave loaded
  // with the row's h, ahead of its use; with three, at the row's start, which
  // keeps the registers from spilling) and the norm weights of this thread's
  // quads
  constexpr bool kEarlyDelta = CPW <= 2;
  auto load_delta = [&](int b, uint2 (&dst)[CPW]) {
#pragma unroll
    for (int u = 0; u < CPW; ++u) {
      const int c = w + kWaves * u;
      dst[u] = PRE && A.x2 && c < A.Sn ? *reinterpret_cast<const uint2*>(A.x2 + (int64_t)b * A.ldx2 + 256 * c + 4 * lane)
                                       : make_uint2(0, 0);
    }
  };
  uint2 dq_next[CPW];
  if (kEarlyDelta && lb < A.B) load_delta(lb, dq_next);
  uint2 nwq[CPW];
#pragma unroll
  for (int u = 0; u < CPW; ++u) {
    const int c = w + kWaves * u;
    nwq[u] = PRE && c < A.Sn ? *reinterpret_cast<const uint2*>(A.nw + 256 * c + 4 * lane) : make_uint2(0, 0);
  }
  {
    float kmv[3];
    mmat_load(kmv, A.Sn, A.lsh_n, A.pn, A.Kn, tid);
    mmat_store(kmv, A.Sn, A.lsh_n, Mh, Ml, tid);
  }
  for (int b = lb; b < A.B; b += stride) {
    float xv[CPW][4];
    if constexpr (PRE) {
      const bool has_delta = A.x2 != nullptr;
      uint2 dq[CPW];
      if constexpr (kEarlyDelta) {
#pragma unroll
        for (int u = 0; u < CPW; ++u) dq[u] = dq_next[u];
      } else {
        const uint16_t* drow = A.x2 ? A.x2 + (int64_t)b * A.ldx2 : nullptr;
#pragma unroll
        for (int u = 0; u < CPW; ++u) {
          const int c = w + kWaves * u;
          dq[u] = drow && c < A.Sn ? *reinterpret_cast<const uint2*>(drow + 256 * c + 4 * lane) : make_uint2(0, 0);
        }
      }
      // h' = bf16(h + delta) in this kernel's layout, staged as a bf16 row in
      // the chunk rows' region (rewritten only after the norm), so that rs is
      // taken in rmsnorm_kernel's layout and order from LDS rather than from
      // a second read of the row in memory
      uint16_t* hs = reinterpret_cast<uint16_t*>(lds + L::kY);
      uint32_t hpv[CPW][2];
#pragma unroll
      for (int u = 0; u < CPW; ++u) {
        const int c = w + kWaves * u;
        hpv[u][0] = xr.v[u].x;  // h as loaded
        hpv[u][1] = xr.v[u].y;
        if (has_delta) {
          hpv[u][0] = rms_pair_resid(hpv[u][0], dq[u].x);
          hpv[u][1] = rms_pair_resid(hpv[u][1], dq[u].y);
        }
        if (c < A.Sn) *reinterpret_cast<uint2*>(hs + 256 * c + 4 * lane) = make_uint2(hpv[u][0], hpv[u][1]);
      }
      __syncthreads();  // the staged row is complete
      const float rs = rms_row_scale(hs, nullptr, A.n, A.eps, w, lane, lx, pre_wsum);
#pragma unroll
      for (int u = 0; u < CPW; ++u) {
        const int c = w + kWaves * u;
        const uint32_t hp[2] = {hpv[u][0], hpv[u][1]};
        if (g == 0 && A.h_out && c < A.Sn)
          *reinterpret_cast<uint2*>(A.h_out + (int64_t)b * A.ldo + 256 * c + 4 * lane) = make_uint2(hp[0], hp[1]);
        const uint4 xq = make_uint4(rms_pair_apply(hp[0], nwq[u].x, rs), rms_pair_apply(hp[1], nwq[u].y, rs), 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) xv[u][j] = 0.0f;
        if (c < A.Sn) finish_chunk(X, xq, xr.s[u], lane, xv[u]);
      }
    } else {
      finish_x(X, xr, w, lane, xv);
    }
    if (b + stride < A.B) {  // the next row
      load_x_raw(X, J.sv, b + stride, w, lane, xr);
      if constexpr (PRE && kEarlyDelta) load_delta(b + stride, dq_next);
    }
    float ss = 0.0f;
#pragma unroll
    for (int u = 0; u < CPW; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) ss = __builtin_fmaf(xv[u][j], xv[u][j], ss);
    ss = wave_sum(ss, lx);
    if (lane == 0) wsum[w] = ss;
    h256_chunks(xv, A.Sn, lane, lx);
    store_chunks(Y, A.Sn, w, lane, xv);
    __syncthreads();
    float norm2 = 0.0f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) norm2 += wsum[i];
    const int e = operand_exponent(norm2);
    const float mul = ldexpf(A.scale_n, -e);
    if (tid == 0) J.xmul[b] = ldexpf(1.0f, e);

    // chunk stage: operand row (slice) s = 16 a + 4 q + j, column t = 16 w + r16
    const int t = 16 * w + r16;
    const int nrt = (A.Sn + 15) >> 4, nkb = (A.Sn + 31) >> 5;
    floatx4 acc[CPW];
#pragma unroll
    for (int a = 0; a < CPW; ++a) acc[a] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < nkb; ++kb) {
      const ZOperand z = z_operand(Y, A.Sn, t, q, kb);
#pragma unroll
      for (int a = 0; a < CPW; ++a)
        if (a < nrt) acc[a] = mstage_step(acc[a], Mh, Ml, 16 * a, z, kb, A.pn > 1, q, r16);
    }
    // destinations: natural rows, or the fragment-major operand whose index
    // is a row part plus a column part (frag_index, sg_frag_index)
    _Float16* xrow = J.x2h + (A.frag ? frag_index(b, 0, A.Sn) : (size_t)b * A.n);
    _Float16* srow = J.sg + (A.frag ? sg_frag_index(b, 0, A.Sn) : (size_t)b * (A.n / 8));
    const int xcol = A.frag ? ((t >> 3) & 7) * 512 + (t >> 6) * 128 + (t & 7) : t;     // + 4096 s (frag) / 256 s
    const int scol = A.frag ? ((t >> 6) & 3) * 128 + ((t >> 3) & 7) : (t >> 3);        // + 512 s (frag) / 32 s
    const int xs = A.frag ? 4096 : 256, ss_ = A.frag ? 512 : 32;
    const _Float16 sgmul = A.frag ? (_Float16)0.25f : (_Float16)1.0f;
#pragma unroll
    for (int a = 0; a < CPW; ++a) {
      if (a < nrt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int s = 16 * a + 4 * q + j;
          const _Float16 h = (_Float16)(acc[a][j] * mul);
          // sum of the 8 fp16 values of group t / 8 (lanes r16 & 7 = 0..7)
          float hs = (float)h;
          hs += lane_xor<1>(hs, lx);
          hs += lane_xor<2>(hs, lx);
          hs += lane_xor<4>(hs, lx);
          if (s < A.Sn) {
            xrow[xs * s + xcol] = h;
            if ((r16 & 7) == 0) srow[ss_ * s + scol] = (_Float16)hs * sgmul;
          }
        }
      }
    }
    __syncthreads();  // Y and wsum are rewritten for the next row
  }
}

// ---------------------------------------------------------------------------
// decode-matvec
// ---------------------------------------------------------------------------
// One linear of a decode-matvec launch; the linears of a launch share n and
// the batch rows, and split the grid: work-groups wg0 .. wg0 + Gr SG - 1 are
// this linear's.
struct BmJob {
  const uint16_t* codes0;
  const uint8_t* codes1;
  const _Float16* x2h;  // fragment-major operand of this linear (16 rows)
  const _Float16* sg;
  float* y1p;  // [SG][B][m] partial sums for a separate output kernel
  int m, Gr, wg0;
  float s0, s1;
  // output transform in this kernel (the tail instantiations): tagged
  // partial sums [SG][B][m], the epoch word of the job, and by_kernel's
  // per-linear arguments
  unsigned long long* y1t;
  unsigned* epoch;
  const float* xmul;
  int Sm, lsh_m, pm;
  const float* Km;
  float scale_m, layer_scale;
  const float* su;
  const float* bias;
  void* y;
  int64_t ldy;
};

struct BmArgs {
  int n, B, S, SG, W;
  int lgBp, lgtpo;  // log2 of B rounded up to a power of two, log2 of the threads per output of the
                    // reduction (2^lgtpo kBmSlots 16 2^lgBp <= 1024)
  int y_dtype;      // tail instantiations: output dtype
  int njobs;
  BmJob job[QS_MAX_GROUP];
  // tail instantiations: the workspace (its tags are cleared when a job's
  // counter wraps); after the jobs so that their fields keep their offsets
  unsigned long long* ws;
  unsigned long long ws_words;
};

constexpr int kBmSlots = 4;                  // row blocks reduced together (2: 0.6 % slower at 16 rows)
constexpr int kBmSlot = kWaves * 16 * kTB;   // floats per slot: [wave][row][batch]
constexpr int kBmOffHi = 0;                  // 4096 x uint32 (four fp16 high bytes)
constexpr int kBmOffLo = 16384;              // 4096 x uint32
constexpr int kBmOffLut1 = 32768;            // 256 x uint4
constexpr int kBmOffRed = kBmOffLut1 + 4096; // kBmSlots x kBmSlot floats
constexpr int kBmLds = kBmOffRed + kBmSlots * kBmSlot * 4;
static_assert(kBmLds <= 160 * 1024, "LDS budget");

// OC > 0: the output transform runs in this kernel as well (OC output
// chunks per wave, SB: su as packed sign bits).  The partial sums go out as
// tagged 64-bit slots (as in the one-launch kernel, qs_forward_dev.h), and
// work-group b < B of each linear, once its own row blocks are done, polls
// batch row b's slots (every work-group of the linear writes every row's) and
// applies by_kernel's output transform to that row: the same sums in the
// same order, so the outputs are bit-identical to bm_kernel + by_kernel.  The
// grid is at most one work-group per CU, so every polled work-group runs; a
// poll is bounded (NaN outputs if a slot never arrives).
template <bool HAS2, int OC, bool SB>
__global__ __launch_bounds__(kThreads) void bm_kernel(BmArgs A) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  uint4* lut1 = reinterpret_cast<uint4*>(lds + kBmOffLut1);
  float* red = reinterpret_cast<float*>(lds + kBmOffRed);

  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  int g = 0;
#pragma unroll
  for (int k = 1; k < QS_MAX_GROUP; ++k)
    if (k < A.njobs && (int)blockIdx.x >= A.job[k].wg0) g = k;
  const BmJob& J = A.job[g];
  const int RB = J.m >> 4;
  const int lb = (int)blockIdx.x - J.wg0;  // work-group index within this linear
  const int sg = lb / J.Gr, jr = lb - sg * J.Gr;
  const int sl = sg * A.W + w;
  const bool active = w < A.W && sl < A.S;
  const LaneX lx = lane_x_init();

  // All global loads here are unconditional (an idle lane reads a valid
  // address it does not use), so the compiler waits for exactly the data in
  // use: first the LUTs, then the operand, then the code tiles.
  LutCopy<kThreads> lutw;
  load_luts(tid, lutw);
  uint4 t1row = make_uint4(0, 0, 0, 0);
  if (HAS2) t1row = *reinterpret_cast<const uint4*>(kE81h.w[tid & 255]);
  // operand of lane (q, b = r16), fragment-major (frag_index): columns
  // 256 sl + 64 q + 8 c .. + 7 of row r16 are the 16 bytes of lane l = 16 q +
  // r16 in fragment c of slice sl, so each of the wave's loads reads one run
  // of consecutive bytes; then the quarter-sums of its eight groups of 8
  // (sg_frag_index).  Lanes of rows b >= B read row 0 again (no extra bytes;
  // the padding rows are never written) and, like idle waves, compute values
  // that are never stored.
  const size_t sla = active ? (size_t)sl : 0;
  const int lrow = 16 * q + (r16 < A.B ? r16 : 0);
  const _Float16* xfrag = J.x2h + sla * 4096 + 8 * lrow;
  half8 xb[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) xb[c] = *reinterpret_cast<const half8*>(xfrag + 512 * c);
  const half8 xs = *reinterpret_cast<const half8*>(J.sg + sla * 512 + 8 * lrow);
  // code tiles stream through a ring of kPrefetch registers (see the row
  // loop).  Byte offset of this lane's 16 code bytes of row block rb; past
  // the end, the work-group's own last row block again, and for an idle
  // wave the group's first slice, the tile wave 0 of this work-group reads
  // at the same time (an L2 hit; a slice index past the group's own would
  // fetch another group's tiles, on another XCD's L2); m n / 4 < 2^32 bytes
  // of codes
  const int rb_last = jr + ((RB - 1 - jr) / J.Gr) * J.Gr;
  const int sl0 = sg * A.W < A.S ? sg * A.W : A.S - 1;
  const uint32_t slc = (uint32_t)(active ? sl : sl0);
  auto code_off = [&](int rb) -> uint32_t {
    const uint32_t r = (uint32_t)(rb < RB ? rb : rb_last);
    return (r * (uint32_t)A.S + slc) * 1024u + 16u * lane;
  };
  uint4 pre[kPrefetch];
  uint2 pre1[kPrefetch] = {};
#pragma unroll
  for (int k = 0; k < kPrefetch; ++k) {
    const uint32_t off = code_off(jr + k * J.Gr);
    pre[k] = ld_nt_u4(reinterpret_cast<const char*>(J.codes0) + off);
    if (HAS2) pre1[k] = ld_nt_u2(J.codes1 + off / 2);
  }
  store_luts(lds, tid, lutw);
  if (HAS2 && tid < 256) lut1[tid] = t1row;
  __syncthreads();
  // tag of this launch's partial sums (tail instantiations); the epoch only
  // changes once a tail work-group has read every slot of its row
  uint32_t tag = 0;
  if constexpr (OC > 0) tag = next_tag(__hip_atomic_load(J.epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT), g);

  float slice_shift = 0.0f;  // sum_g S_g / 4 over the slice, batch row r16
#pragma unroll
  for (int c = 0; c < 8; ++c) slice_shift += (float)xs[c];
  slice_shift += lane_xor<16>(slice_shift, lx);
  slice_shift += lane_xor<32>(slice_shift, lx);

  const int nw = A.S - sg * A.W < A.W ? A.S - sg * A.W : A.W;
  // The ring is unrolled and every step runs (a step past the last row
  // block only refills its entry), so its registers are never copied and
  // each step waits for its own tile only; an entry is refilled once its
  // tile is decoded.
  int k = 0;  // row blocks done: selects the reduction slot
  for (int rb0 = jr; rb0 < RB; rb0 += kPrefetch * J.Gr) {
#pragma unroll
  for (int u = 0; u < kPrefetch; ++u) {
    const int rb = rb0 + u * J.Gr;
    const bool valid = rb < RB;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    floatx4 accs = {0.f, 0.f, 0.f, 0.f};
    floatx4 acc2 = {0.f, 0.f, 0.f, 0.f};
    const uint4 cw = pre[u];
    const uint2 cw1 = pre1[u];
    if (valid && active) {
      // (idle waves skip the decode, a wave-uniform branch: they hold no
      // slice, and their LUT reads would take LDS cycles from the others)
      const uint32_t wd[4] = {cw.x, cw.y, cw.z, cw.w};
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(decode_code(wd[c >> 1], c, kBmOffHi, kBmOffLo), xb[c], acc, 0,
                                                     0, 0);
        if (HAS2) {
          const uint32_t idx = ((c < 4 ? cw1.x : cw1.y) >> (8 * (c & 3))) & 0xFFu;
          acc2 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8, lut1[idx]), xb[c], acc2, 0, 0,
                                                          0);
        }
      }
      accs = __builtin_amdgcn_mfma_f32_16x16x32_f16(shift_operand(wd), xs, accs, 0, 0, 0);
    }
    {
      const uint32_t off = code_off(rb + kPrefetch * J.Gr);
      pre[u] = ld_nt_u4(reinterpret_cast<const char*>(J.codes0) + off);
      if (HAS2) pre1[u] = ld_nt_u2(J.codes1 + off / 2);
    }
    // lane holds rows 4q..4q+3 of the tile for batch column r16
    const int slot = k % kBmSlots;
    float* rbuf = red + slot * kBmSlot;
    if (valid) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float v = J.s0 * (acc[j] + 2.0f * accs[j] - slice_shift);
        if (HAS2) v = v + J.s1 * acc2[j];
        rbuf[(w * 16 + 4 * q + j) * kTB + r16] = active ? v : 0.0f;
      }
    }
    if (valid && (slot == kBmSlots - 1 || rb + J.Gr >= RB)) {
      __syncthreads();
      // output o = (s * 16 + row) * Bp + b of slot s <= slot (Bp: B rounded
      // up to a power of two, so that every index is a shift; columns b >= B
      // are skipped), summed over the waves by tpo threads (waves part, part
      // + tpo, ...), then across them; tpo depends on B only (a fixed
      // summation order per output)
      const int lgBp = A.lgBp, lgt = A.lgtpo;
      const int nout = (slot + 1) << (4 + lgBp);
      const int tpo = 1 << lgt;
      const int o = tid >> lgt, part = tid & (tpo - 1);
      float v = 0.0f;
      int s = 0, row = 0, bc = 0;
      if (o < nout) {
        s = o >> (4 + lgBp);
        const int rr = o & ((16 << lgBp) - 1);
        row = rr >> lgBp;
        bc = rr & ((1 << lgBp) - 1);
        if (bc < A.B)
          for (int ww = part; ww < nw; ww += tpo) v += red[s * kBmSlot + (ww * 16 + row) * kTB + bc];
      }
      if (tpo >= 2) v += lane_xor<1>(v, lx);
      if (tpo >= 4) v += lane_xor<2>(v, lx);
      if (tpo >= 8) v += lane_xor<4>(v, lx);
      if (tpo >= 16) v += lane_xor<8>(v, lx);
      if (o < nout && part == 0 && bc < A.B) {
        const int rbs = rb - (slot - s) * J.Gr;  // row block of slot s
        const size_t idx = partial_index(sg, A.B, bc, J.m, block_elem(rbs, row));
        if constexpr (OC > 0)
          __hip_atomic_store(&J.y1t[idx], tagged(v, tag), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        else
          J.y1p[idx] = v;
      }
      __syncthreads();  // the slots are free again
    }
    k += valid;
  }
  }
  if constexpr (OC > 0) {
    // output transform of batch row lb (by_kernel's, on polled slots)
    if (lb >= A.B) return;
    const int b = lb;
    using L = RowLds<OC>;
    __syncthreads();  // the LUT and reduction space becomes the row's chunk rows and M
    float* Y = reinterpret_cast<float*>(lds + L::kY);
    uint16_t* Mh = reinterpret_cast<uint16_t*>(lds + L::kMh);
    uint16_t* Ml = reinterpret_cast<uint16_t*>(lds + L::kMl);
    const int Sm = J.Sm;
    const int t = 16 * w + r16;
    float kmv[3];
    mmat_load(kmv, Sm, J.lsh_m, J.pm, J.Km, tid);
    int oidx[OC][4];
    float suo[OC][4], bio[OC][4];
    // no bias: a dummy load from the slots (at least m entries), selected
    // away rather than multiplied by 0
    const float* const bsrc = J.bias ? J.bias : reinterpret_cast<const float*>(J.y1t);
    const bool has_bias = J.bias != nullptr;
#pragma unroll
    for (int a = 0; a < OC; ++a)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 16 * a + 4 * q + j;
        oidx[a][j] = r < Sm ? out_elem(r, t) : -1;
        const int ii = oidx[a][j] >= 0 ? oidx[a][j] : 0;
        suo[a][j] = load_su(J.su, SB, ii);
        bio[a][j] = at_off(bsrc, (uint32_t)ii);
      }
    const float xm = J.xmul[b];
    PollState<OC> ps;
    poll_issue(J.y1t, J.m, Sm, A.B, b, w, lane, tag, ps);
    mmat_store(kmv, Sm, J.lsh_m, Mh, Ml, tid);
    float zv[OC][4];
    poll_finish(J.y1t, J.m, Sm, A.SG, A.B, b, w, lane, tag, ps, zv);
    const float mul = J.scale_m * J.layer_scale * xm;
    h256_chunks(zv, Sm, lane, lx);
    store_chunks_lanes(Y, Sm, w, lane, zv);
    __syncthreads();  // chunk rows and M complete
    const int nrt = (Sm + 15) >> 4, nkb = (Sm + 31) >> 5;
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
#pragma unroll
    for (int a = 0; a < OC; ++a)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        out[a][j] = apply_su(acc[a][j] * mul, suo[a][j], SB, oidx[a][j]) + (has_bias ? bio[a][j] : 0.0f);
    store_outputs(J.y, A.y_dtype, (int64_t)b * J.ldy, oidx, out);
    // every slot of row b has been read, so every work-group of the linear has
    // read the epoch: the next launch's tag follows this one
    finish_tagged_launch(J.epoch, tag, g, TagWs{J.epoch + kWrapWord, A.ws, A.ws_words, A.B},
                         reinterpret_cast<int*>(lds));  // the tails: work-groups b < B
  }
}

// ---------------------------------------------------------------------------
// output transform
// ---------------------------------------------------------------------------
// One linear of an output-transform launch: work-groups wg0 .. wg0 + grid - 1
// walk its rows.  The linears of a launch share B and the output dtype.
struct ByJob {
  const float* y1p;  // [SG][B][m]
  const float* xmul; // [B]
  int SG, m, Sm, lsh_m, pm, wg0, grid;
  const float* Km;
  float scale_m, layer_scale;
  const float* su;
  const float* bias;
  void* y;
  int64_t ldy;
};

struct ByArgs {
  int B;
  int y_dtype;
  int sbits;  // su of every linear is packed sign bits
  int njobs;
  ByJob job[QS_MAX_GROUP];
};

// Rows b = lb, lb + grid, ... of the linear whose work-groups include this
// one (lb its index among them); su, bias and M are loaded once.  With one
// partial group (G == 1) the next row's partial sums are loaded while this
// row is transformed (with up to kMaxSG or 4 they would not fit the registers
// alongside su and bias, and are loaded per row, all groups at once); G == 0
// sums any number of groups one at a time.  A linear with fewer groups than G
// adds zeros.  CPW: chunks per wave, as bx_kernel.
template <int G, int CPW, bool SB>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(CPW == 1 ? 8 : 1)))
void by_kernel(ByArgs A) {
  using L = RowLds<CPW>;
  extern __shared__ __attribute__((aligned(16))) char lds[];
  float* Y = reinterpret_cast<float*>(lds + L::kY);
  uint16_t* Mh = reinterpret_cast<uint16_t*>(lds + L::kMh);
  uint16_t* Ml = reinterpret_cast<uint16_t*>(lds + L::kMl);
  const int tid = threadIdx.x;
  const int lane = tid & 63, w = tid >> 6;
  const int q = lane >> 4, r16 = lane & 15;
  int g = 0;
#pragma unroll
  for (int k = 1; k < QS_MAX_GROUP; ++k)
    if (k < A.njobs && (int)blockIdx.x >= A.job[k].wg0) g = k;
  const ByJob& J = A.job[g];
  const int lb = (int)blockIdx.x - J.wg0;
  const int Sm = J.Sm;
  const int t = 16 * w + r16;
  const LaneX lx = lane_x_init();
  const int stride = J.grid;

  // loads in the order they are waited for: K entries of M, partial sums,
  // su and bias (unconditional loads from valid addresses)
  float kmv[3];
  mmat_load(kmv, Sm, J.lsh_m, J.pm, J.Km, tid);
  PRaw<1, CPW> pr;
  if constexpr (G == 1) load_partials_raw<false, 1>(J.y1p, J.m, Sm, J.SG, A.B, lb, w, lane, pr);
  // output element of out[a][j] (-1: none), recomputed where it is used
  auto out_index = [&](int a, int j) {
    const int r = 16 * a + 4 * q + j;
    return r < Sm ? out_elem(r, t) : -1;
  };
  float suo[CPW][4], bio[CPW][4];
  // no bias: a dummy load from the partial sums (at least m floats; su may
  // be m / 32 words of sign bits), never used: the bias term is selected,
  // not multiplied by 0, so a non-finite dummy cannot reach the output
  const float* const bsrc = J.bias ? J.bias : J.y1p;
  const bool has_bias = J.bias != nullptr;
#pragma unroll
  for (int a = 0; a < CPW; ++a)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int oi = out_index(a, j);
      const int ii = oi >= 0 ? oi : 0;
      suo[a][j] = load_su(J.su, SB, ii);
      bio[a][j] = bsrc[ii];
    }
  mmat_store(kmv, Sm, J.lsh_m, Mh, Ml, tid);
  for (int b = lb; b < A.B; b += stride) {
    float zv[CPW][4];
    if constexpr (G == 1) {
      sum_partials(pr, zv);
      if (b + stride < A.B) load_partials_raw<false, 1>(J.y1p, J.m, Sm, J.SG, A.B, b + stride, w, lane, pr);
    } else if constexpr (G == 0) {
      sum_partials_loop(J.y1p, J.m, Sm, J.SG, A.B, b, w, lane, zv);
    } else {
      PRaw<G, CPW> pg;
      load_partials_raw<false, G>(J.y1p, J.m, Sm, J.SG, A.B, b, w, lane, pg);
      sum_partials(pg, zv);
    }
    const float mul = J.scale_m * J.layer_scale * J.xmul[b];
    h256_chunks(zv, Sm, lane, lx);
    store_chunks_lanes(Y, Sm, w, lane, zv);
    __syncthreads();
    const int nrt = (Sm + 15) >> 4, nkb = (Sm + 31) >> 5;
    floatx4 acc[CPW];
#pragma unroll
    for (int a = 0; a < CPW; ++a) acc[a] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int kb = 0; kb < nkb; ++kb) {
      const ZOperand z = z_operand(Y, Sm, t, q, kb);
#pragma unroll
      for (int a = 0; a < CPW; ++a)
        if (a < nrt) acc[a] = mstage_step(acc[a], Mh, Ml, 16 * a, z, kb, J.pm > 1, q, r16);
    }
    float out[CPW][4];
    int oidx[CPW][4];
#pragma unroll
    for (int a = 0; a < CPW; ++a)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        oidx[a][j] = out_index(a, j);
        out[a][j] = apply_su(acc[a][j] * mul, suo[a][j], SB, oidx[a][j]) + (has_bias ? bio[a][j] : 0.0f);
      }
    store_outputs(J.y, A.y_dtype, (int64_t)b * J.ldy, oidx, out);
    __syncthreads();  // Y is rewritten for the next row
  }
}

int lds_checked(const void* fn, size_t bytes, int* done) {
  if (!*done) {
    hipFuncAttributes fa{};
    QS_HIP(hipFuncGetAttributes(&fa, fn));
    QS_REQUIRE(fa.sharedSizeBytes == 0, "batched forward kernels must not use static LDS");
    QS_HIP(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes));
    *done = 1;
  }
  return QS_OK;
}

}  // namespace

bool batched_eligible(int64_t n, int pn, int64_t m, int pm) {
  return chunk_transform_fits(n, pn) && chunk_transform_fits(m, pm);
}

namespace {

// Work-groups of a per-row kernel: one per row up to one per CU, or two with
// one chunk per wave, whose registers and LDS let two 1024-thread work-groups
// share a CU (each walks its rows with the next row's loads in flight).  A
// launch for several linears passes its share of the CUs.
constexpr int kRowWgsPerCu1 = 2;
inline int row_wgs_per_cu(int cpw) { return cpw == 1 ? kRowWgsPerCu1 : 1; }
unsigned row_grid(int B, int ncu) {
  const int cap = ncu > 0 ? ncu : 256;
  return (unsigned)(B < cap ? B : cap);
}

template <bool HAS2, int OC, bool SB>
int launch_bm_v(const BmArgs& M, unsigned grid, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop) {
  static int done = 0;
  const int rc = lds_checked((const void*)bm_kernel<HAS2, OC, SB>, kBmLds, &done);
  if (rc) return rc;
  hipExtLaunchKernelGGL((bm_kernel<HAS2, OC, SB>), dim3(grid), dim3(kThreads), kBmLds, stream, ev_start, ev_stop, 0, M);
  QS_LAUNCHED("bm_kernel");
  return QS_OK;
}
template <bool HAS2>
int launch_bm_h(const BmArgs& M, int oc, bool sb, unsigned grid, hipStream_t stream, hipEvent_t ev_start,
                hipEvent_t ev_stop) {
  switch (oc) {
    case 0: return launch_bm_v<HAS2, 0, false>(M, grid, stream, ev_start, ev_stop);
    case 1: return sb ? launch_bm_v<HAS2, 1, true>(M, grid, stream, ev_start, ev_stop)
                      : launch_bm_v<HAS2, 1, false>(M, grid, stream, ev_start, ev_stop);
    case 2: return sb ? launch_bm_v<HAS2, 2, true>(M, grid, stream, ev_start, ev_stop)
                      : launch_bm_v<HAS2, 2, false>(M, grid, stream, ev_start, ev_stop);
    default: return sb ? launch_bm_v<HAS2, 3, true>(M, grid, stream, ev_start, ev_stop)
                       : launch_bm_v<HAS2, 3, false>(M, grid, stream, ev_start, ev_stop);
  }
}

template <int CPW, bool SB, bool PRE>
int launch_bx_cs(const BxArgs& X, unsigned grid, hipStream_t stream) {
  static int done = 0;
  const int rc = lds_checked((const void*)bx_kernel<CPW, SB, PRE>, RowLds<CPW>::kTotal, &done);
  if (rc) return rc;
  hipLaunchKernelGGL((bx_kernel<CPW, SB, PRE>), dim3(grid), dim3(kThreads), RowLds<CPW>::kTotal, stream, X);
  QS_LAUNCHED("bx_kernel");
  return QS_OK;
}

template <int G, int CPW, bool SB>
int launch_by_gc(const ByArgs& Y, unsigned grid, hipStream_t stream) {
  static int done = 0;
  const int rc = lds_checked((const void*)by_kernel<G, CPW, SB>, RowLds<CPW>::kTotal, &done);
  if (rc) return rc;
  hipLaunchKernelGGL((by_kernel<G, CPW, SB>), dim3(grid), dim3(kThreads), RowLds<CPW>::kTotal, stream, Y);
  QS_LAUNCHED("by_kernel");
  return QS_OK;
}

// With one partial group the next row's sums are prefetched (by_kernel<1>);
// up to 3 or 4 groups are loaded together; more, one group at a time.
template <int CPW, bool SB>
int launch_by_cs(const ByArgs& Y, unsigned grid, int maxsg, hipStream_t stream) {
  if (maxsg == 1) return launch_by_gc<1, CPW, SB>(Y, grid, stream);
  if (maxsg <= kMaxSG) return launch_by_gc<kMaxSG, CPW, SB>(Y, grid, stream);
  if (maxsg <= 4) return launch_by_gc<4, CPW, SB>(Y, grid, stream);
  return launch_by_gc<0, CPW, SB>(Y, grid, stream);
}
template <int CPW>
int launch_bx_cpw(const BxArgs& X, unsigned grid, bool pre, hipStream_t stream) {
  if (pre)
    return X.sbits ? launch_bx_cs<CPW, true, true>(X, grid, stream) : launch_bx_cs<CPW, false, true>(X, grid, stream);
  return X.sbits ? launch_bx_cs<CPW, true, false>(X, grid, stream) : launch_bx_cs<CPW, false, false>(X, grid, stream);
}
template <int CPW>
int launch_by_cpw(const ByArgs& Y, unsigned grid, int maxsg, hipStream_t stream) {
  return Y.sbits ? launch_by_cs<CPW, true>(Y, grid, maxsg, stream) : launch_by_cs<CPW, false>(Y, grid, maxsg, stream);
}

}  // namespace

int launch_bx_group(const BatchedPass* P, int count, hipStream_t stream, const FusedPre* pre) {
  QS_REQUIRE(count >= 1 && count <= QS_MAX_GROUP, "input transform: 1..%d linears", QS_MAX_GROUP);
  const BatchedPass& P0 = P[0];
  QS_REQUIRE(chunk_transform_fits(P0.n, P0.pn), "input transform: n outside the chunk scheme");
  BxArgs X{};
  X.x = P0.x;
  X.x_dtype = P0.x_dtype;
  {
    const uintptr_t align = P0.x_dtype == QS_DTYPE_F32 ? 16 : 8;
    X.x_vec = (reinterpret_cast<uintptr_t>(P0.x) % align) == 0 && P0.ldx % 4 == 0;
  }
  X.ldx = P0.ldx;
  X.B = P0.B;
  X.n = (int)P0.n;
  X.Sn = (int)(P0.n / 256);
  X.lsh_n = log2_exact((int)(P0.n / P0.pn / 256));
  X.pn = P0.pn;
  X.Kn = P0.Kn;
  X.scale_n = inv_sqrt_len((int)(P0.n / P0.pn));
  X.frag = P0.frag;
  X.sbits = P0.sbits;
  const int cpw = chunks_per_wave(X.Sn);
  X.per = (int)row_grid(P0.B, P0.ncu * row_wgs_per_cu(cpw) / count);
  for (int j = 0; j < count; ++j) {
    const BatchedPass& Q = P[j];
    QS_REQUIRE(Q.x == P0.x && Q.x_dtype == P0.x_dtype && Q.ldx == P0.ldx && Q.B == P0.B && Q.n == P0.n &&
                   Q.pn == P0.pn && Q.Kn == P0.Kn && Q.frag == P0.frag && Q.sbits == P0.sbits,
               "input transform: linears of one launch share x and its transform");
    X.job[j] = BxJob{Q.sv, Q.x2h, Q.sg, Q.xmul};
  }
  if (pre) {
    QS_REQUIRE(pre->kind == QS_PREOP_RMSNORM && X.x_dtype == QS_DTYPE_BF16 && X.x_vec && pre->weight &&
                   X.n <= 16384,
               "input transform: the RMSNorm pre-operation needs bf16 rows loaded 8 bytes at a time");
    X.x2 = static_cast<const uint16_t*>(pre->x2);
    X.ldx2 = pre->ldx2;
    X.nw = static_cast<const uint16_t*>(pre->weight);
    X.h_out = static_cast<uint16_t*>(pre->h_out);
    X.ldo = pre->ldo;
    X.eps = pre->eps;
  }
  const unsigned grid = (unsigned)(X.per * count);
  switch (cpw) {
    case 1: return launch_bx_cpw<1>(X, grid, pre != nullptr, stream);
    case 2: return launch_bx_cpw<2>(X, grid, pre != nullptr, stream);
    default: return launch_bx_cpw<3>(X, grid, pre != nullptr, stream);
  }
}

int launch_bx_rows(const BatchedPass& P, hipStream_t stream) { return launch_bx_group(&P, 1, stream, nullptr); }

int launch_by_group(const BatchedPass* P, int count, hipStream_t stream) {
  QS_REQUIRE(count >= 1 && count <= QS_MAX_GROUP, "output transform: 1..%d linears", QS_MAX_GROUP);
  ByArgs Y{};
  Y.B = P[0].B;
  Y.y_dtype = P[0].y_dtype;
  Y.sbits = P[0].sbits;
  Y.njobs = count;
  int maxsg = 1, cpw = 1;
  for (int j = 0; j < count; ++j)
    if (chunks_per_wave(P[j].m / 256) > cpw) cpw = chunks_per_wave(P[j].m / 256);
  const unsigned per = row_grid(P[0].B, P[0].ncu * row_wgs_per_cu(cpw) / count);
  for (int j = 0; j < count; ++j) {
    const BatchedPass& Q = P[j];
    QS_REQUIRE(chunk_transform_fits(Q.m, Q.pm), "output transform: m outside the chunk scheme");
    QS_REQUIRE(Q.SG >= 1 && Q.SG <= kWideMaxGroups, "output transform: 1..%d partial groups", kWideMaxGroups);
    QS_REQUIRE(Q.B == Y.B && Q.y_dtype == Y.y_dtype && Q.sbits == Y.sbits,
               "output transform: linears of one launch share rows, dtype and sign format");
    ByJob& J = Y.job[j];
    J.y1p = Q.y1p;
    J.xmul = Q.xmul;
    J.SG = Q.SG;
    J.m = (int)Q.m;
    J.Sm = (int)(Q.m / 256);
    J.lsh_m = log2_exact((int)(Q.m / Q.pm / 256));
    J.pm = Q.pm;
    J.wg0 = (int)per * j;
    J.grid = (int)per;
    J.Km = Q.Km;
    J.scale_m = inv_sqrt_len((int)(Q.m / Q.pm));
    J.layer_scale = Q.layer_scale;
    J.su = Q.su;
    J.bias = Q.bias;
    J.y = Q.y;
    J.ldy = Q.ldy;
    if (Q.SG > maxsg) maxsg = Q.SG;
  }
  const unsigned grid = per * (unsigned)count;
  switch (cpw) {
    case 1: return launch_by_cpw<1>(Y, grid, maxsg, stream);
    case 2: return launch_by_cpw<2>(Y, grid, maxsg, stream);
    default: return launch_by_cpw<3>(Y, grid, maxsg, stream);
  }
}

int launch_by_rows(const BatchedPass& P, hipStream_t stream) { return launch_by_group(&P, 1, stream); }

int launch_bm_group(const BatchedPass* P, int count, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop,
                    bool* tail_done) {
  QS_REQUIRE(count >= 1 && count <= QS_MAX_GROUP, "decode-matvec: 1..%d linears", QS_MAX_GROUP);
  const BatchedPass& P0 = P[0];
  QS_REQUIRE(P0.B >= 1 && P0.B <= kTB, "batched pass: 1..%d rows", kTB);
  QS_REQUIRE(P0.n % 256 == 0 && P0.S == (int)(P0.n / 256) && P0.SG >= 1 && P0.W >= 1 && P0.W <= kWaves &&
                 P0.SG * P0.W >= P0.S,
             "decode-matvec: bad slice grouping");
  BmArgs M{};
  M.n = (int)P0.n;
  M.B = P0.B;
  M.S = P0.S;
  M.SG = P0.SG;
  M.W = P0.W;
  M.njobs = count;
  M.lgBp = 0;
  while ((1 << M.lgBp) < P0.B) ++M.lgBp;
  M.lgtpo = 4;
  while (M.lgtpo > 0 && (kBmSlots * 16 << (M.lgtpo + M.lgBp)) > kThreads) --M.lgtpo;
  // work-groups per slice group: one per CU over all the linears, dealt in
  // proportion to their row blocks (at least one, at most one per row block)
  int budget = P0.ncu / P0.SG;
  if (budget < 1) budget = 1;
  int64_t rb_total = 0;
  for (int j = 0; j < count; ++j) rb_total += P[j].m / 16;
  int wg = 0;
  for (int j = 0; j < count; ++j) {
    const BatchedPass& Q = P[j];
    QS_REQUIRE(Q.m % 16 == 0 && Q.n == P0.n && Q.B == P0.B && (Q.codes1 != nullptr) == (P0.codes1 != nullptr),
               "decode-matvec: linears of one launch share n, rows and stages");
    QS_REQUIRE(Q.frag, "decode-matvec: the operand must be fragment-major");
    BmJob& J = M.job[j];
    const int RB = (int)(Q.m / 16);
    int64_t gr = (int64_t)budget * RB / rb_total;
    if (gr < 1) gr = 1;
    if (gr > RB) gr = RB;
    J.codes0 = static_cast<const uint16_t*>(Q.codes0);
    J.codes1 = static_cast<const uint8_t*>(Q.codes1);
    J.x2h = Q.x2h;
    J.sg = Q.sg;
    J.y1p = Q.y1p;
    J.m = (int)Q.m;
    J.Gr = (int)gr;
    J.wg0 = wg;
    J.s0 = Q.s0;
    J.s1 = Q.s1;
    wg += J.Gr * P0.SG;
  }
  // output transforms in this launch when every linear provides tagged
  // partial-sum slots (bm_tail_eligible) and has a work-group per row
  // (work-group b < B of each linear transforms row b), the grid fitting the
  // CUs
  bool tail = bm_tail_eligible(P, count) && wg <= (P0.ncu > 0 ? P0.ncu : 256);
  for (int j = 0; j < count; ++j) tail = tail && M.job[j].Gr * P0.SG >= P0.B;
  if (tail_done) *tail_done = tail;
  int oc = 0;
  if (tail) {
    M.y_dtype = P0.y_dtype;
    for (int j = 0; j < count; ++j) {
      const BatchedPass& Q = P[j];
      BmJob& J = M.job[j];
      J.y1t = Q.y1t;
      J.epoch = Q.epoch;
      // the wrap word sits kWrapWord words past the epoch word, in one
      // workspace for every linear of the launch
      QS_REQUIRE(Q.tw.wrap == Q.epoch + kWrapWord, "linear %d: wrap word not beside the epoch", j);
      QS_REQUIRE(j == 0 || (Q.tw.base == M.ws && Q.tw.words == M.ws_words), "linear %d: another workspace", j);
      M.ws = Q.tw.base;
      M.ws_words = Q.tw.words;
      J.xmul = Q.xmul;
      J.Sm = (int)(Q.m / 256);
      J.lsh_m = log2_exact((int)(Q.m / Q.pm / 256));
      J.pm = Q.pm;
      J.Km = Q.Km;
      J.scale_m = inv_sqrt_len((int)(Q.m / Q.pm));
      J.layer_scale = Q.layer_scale;
      J.su = Q.su;
      J.bias = Q.bias;
      J.y = Q.y;
      J.ldy = Q.ldy;
      const int c = chunks_per_wave(J.Sm);
      if (c > oc) oc = c;
    }
  }
  const unsigned grid = (unsigned)wg;
  return P0.codes1 ? launch_bm_h<true>(M, oc, P0.sbits != 0, grid, stream, ev_start, ev_stop)
                   : launch_bm_h<false>(M, oc, P0.sbits != 0, grid, stream, ev_start, ev_stop);
}

bool bm_tail_eligible(const BatchedPass* P, int count) {
  for (int j = 0; j < count; ++j)
    if (!P[j].y1t || !P[j].epoch || !P[j].tw.wrap || !P[j].tw.base || P[j].tw.words <= kWsHeaderWords ||
        P[j].B > kTB || !chunk_transform_fits(P[j].m, P[j].pm) ||
        P[j].y_dtype != P[0].y_dtype || P[j].sbits != P[0].sbits)
      return false;
  return count >= 1;
}

int launch_bm(const BatchedPass& P, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop, bool* tail_done) {
  return launch_bm_group(&P, 1, stream, ev_start, ev_stop, tail_done);
}

int launch_linear_batched(const BatchedPass& P, hipStream_t stream, hipEvent_t ev_start, hipEvent_t ev_stop) {
  QS_REQUIRE(P.B >= 1 && P.B <= kTB, "batched pass: 1..%d rows", kTB);
  QS_REQUIRE(batched_eligible(P.n, P.pn, P.m, P.pm), "batched pass: shapes outside the chunk scheme");
  int rc = launch_bx_rows(P, stream);
  bool tail = false;
  if (!rc) rc = launch_bm(P, stream, ev_start, ev_stop, &tail);
  if (!rc && !tail) rc = launch_by_rows(P, stream);  // else done inside the decode-matvec
  return rc;
}

}  // namespace qs
