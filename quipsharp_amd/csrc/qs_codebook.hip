// E8P / E8 1-bit / residual-VQ encode and decode on gfx950, plus the fused
// BlockLDLQ rounding step and the code repacker for the forward kernels.
//
// Bit-exactness: the encoder reproduces the reference's fp32 CPU arithmetic
// (quipsharp/codebooks/e8p.py:104-162): every product, difference and square
// is a separately rounded IEEE operation (this file is compiled with
// -ffp-contract=off), the eight squares are summed left to right, flips are
// strict "< 0", the parity repair goes to the first coordinate of least
// |product|, and the winner is the lexicographic minimum of
// (distance, shift bit, table row).
#include "qs_common.h"

namespace qs {
namespace {

__constant__ Table8 kE8P = make_e8p_table();
__constant__ Table8 kE81 = make_e81_table();

constexpr int kWaves = 16;          // waves per encode work-group
constexpr int kVecPerBlock = 64;    // one vector per lane
constexpr int64_t kWaveEncodeMax = 32768;  // up to this many vectors: one vector per wave
constexpr int kVecWaves = 4;  // waves (vectors or rows) per work-group of the one-vector-per-wave kernels
                              // (small work-groups: a wave may use up to 512 registers, no spills)

struct StageCfg {
  int n;
  int kind[QS_MAX_STAGES];
  float scale[QS_MAX_STAGES];
};

struct EncodeArgs {
  // target = base (+ delta (@ dinv))
  const float* base;
  int64_t ldbase;
  const float* delta;  // [nvec][8] or NULL
  const float* dinv;   // [8][8] or NULL
  // outputs
  float* vals;
  int64_t ldvals;
  const float* w;      // residual output: resid = w - vals
  int64_t ldw;
  float* resid;
  int64_t ldresid;
  void* codes;
  int code_bytes;
  int64_t code_stage_stride;
  int64_t code_stride;
  int64_t nvec;
  float in_div, out_mul;
  StageCfg st;
};

__device__ __forceinline__ void store_code(void* codes, int code_bytes, int64_t off, uint32_t c) {
  if (code_bytes == 2) static_cast<uint16_t*>(codes)[off] = (uint16_t)c;
  else if (code_bytes == 4) static_cast<int32_t*>(codes)[off] = (int32_t)c;
  else static_cast<int64_t*>(codes)[off] = (int64_t)c;
}

__device__ __forceinline__ uint32_t load_code(const void* codes, int code_bytes, int64_t off) {
  if (code_bytes == 2) return static_cast<const uint16_t*>(codes)[off];
  if (code_bytes == 4) return (uint32_t) static_cast<const int32_t*>(codes)[off];
  return (uint32_t) static_cast<const int64_t*>(codes)[off];
}

// Distance of the shifted input (|xs| = a, parity bit `odd` for this row) to
// the best even-parity signing of table row t (absolute values T).
__device__ __forceinline__ float e8p_row_d2(const float a[8], const float T[8], bool odd) {
  float sq[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float d = a[i] - T[i];
    sq[i] = d * d;
  }
  if (odd) {
    float best = a[0] * T[0];
    int j = 0;
#pragma unroll
    for (int i = 1; i < 8; ++i) {
      float p = a[i] * T[i];
      if (p < best) { best = p; j = i; }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (i == j) {
        float d = a[i] + T[i];
        sq[i] = d * d;
      }
    }
  }
  float d2 = sq[0];
#pragma unroll
  for (int i = 1; i < 8; ++i) d2 = d2 + sq[i];
  return d2;
}

// Packs the code of table row r at shift bit sb for input x (e8p.py:116-123,
// 165-171) and writes the decoded codeword to q.
__device__ __forceinline__ uint32_t e8p_finish(const float x[8], int sb, int r, float q[8]) {
  float xs[8], prod[8];
  int flip[8];
  int pc = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    xs[i] = sb == 0 ? x[i] + 0.25f : x[i] - 0.25f;
    prod[i] = xs[i] * kE8P.v[r][i];
    flip[i] = prod[i] < 0.0f;
    pc += flip[i];
  }
  if (pc & 1) {
    float best = fabsf(prod[0]);
    int j = 0;
#pragma unroll
    for (int i = 1; i < 8; ++i) {
      float p = fabsf(prod[i]);
      if (p < best) { best = p; j = i; }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (i == j) flip[i] ^= 1;
  }
  uint32_t sign7 = 0;
#pragma unroll
  for (int i = 0; i < 7; ++i) sign7 |= (uint32_t)flip[i] << (6 - i);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float t = kE8P.v[r][i];
    float v = flip[i] ? -t : t;
    q[i] = sb == 0 ? v - 0.25f : v + 0.25f;
  }
  return ((uint32_t)r << 8) | (sign7 << 1) | (uint32_t)sb;
}

// res += dl . dinv (dinv 8 x 8, row-major), or res += dl without dinv (one
// arithmetic for every rounding step).
__device__ __forceinline__ void add_delta(float (&res)[8], const float (&dl)[8], const float* dinv) {
  if (dinv) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float acc = dl[0] * dinv[i];
#pragma unroll
      for (int j = 1; j < 8; ++j) acc = __builtin_fmaf(dl[j], dinv[j * 8 + i], acc);
      res[i] = res[i] + acc;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) res[i] = res[i] + dl[i];
  }
}

// The target of vector vv: base (+ delta, or + delta . dinv), divided by
// in_div (one arithmetic for both encode kernels).
__device__ __forceinline__ void encode_target(const EncodeArgs& A, int64_t vv, float (&res)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) res[i] = A.base[vv * A.ldbase + i];
  if (A.delta) {
    float dl[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) dl[i] = A.delta[vv * 8 + i];
    add_delta(res, dl, A.dinv);
  }
  if (A.in_div != 1.0f) {
#pragma unroll
    for (int i = 0; i < 8; ++i) res[i] = res[i] / A.in_div;
  }
}

// Key of E8P table row r at shift bit sb for the shifted magnitudes a and
// the parities p_pos / p_neg: (distance, shift bit, row), ordered as the
// lexicographic minimum.
__device__ __forceinline__ unsigned long long e8p_key(const float a[8], bool p_pos, bool p_neg, int sb, int r) {
  float T[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) T[i] = fabsf(kE8P.v[r][i]);
  const bool odd = kE8P.v[r][7] < 0.0f ? p_neg : p_pos;
  const float d2 = e8p_row_d2(a, T, odd);
  return ((unsigned long long)__float_as_uint(d2) << 9) | ((unsigned)sb << 8) | (unsigned)r;
}
// Key of E8 one-bit table row r for x: (distance, row).
__device__ __forceinline__ unsigned long long e81_key(const float x[8], int r) {
  float d2 = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float d = x[i] - kE81.v[r][i];
    float sq = d * d;
    d2 = i == 0 ? sq : d2 + sq;
  }
  return ((unsigned long long)__float_as_uint(d2) << 8) | (unsigned)r;
}
// |x + 1/4| (sb 0) or |x - 1/4| (sb 1) and the parities of the signings.
__device__ __forceinline__ void e8p_shifted(const float x[8], int sb, float a[8], bool& p_pos, bool& p_neg) {
  uint32_t sx = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float xs = sb == 0 ? x[i] + 0.25f : x[i] - 0.25f;
    a[i] = fabsf(xs);
    sx ^= __float_as_uint(xs) >> 31;
  }
  const bool z7 = (sb == 0 ? x[7] + 0.25f : x[7] - 0.25f) == 0.0f;
  p_pos = sx & 1;
  p_neg = p_pos ^ !z7;
}

// One vector per lane; wave w evaluates table rows 16 w .. 16 w + 15 and the
// waves' least keys meet in LDS.  The body is written out here rather than
// through the helpers of the one-vector-per-wave kernels below (the same
// arithmetic): built from them it took 90 SGPRs instead of 74 and ran
// ~25 % slower on a 2^21-vector call.
__global__ __launch_bounds__(kWaves * 64) void rvq_encode_kernel(EncodeArgs A) {
  __shared__ unsigned long long keys[2][kWaves][64];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t v = (int64_t)blockIdx.x * kVecPerBlock + lane;
  const bool valid = v < A.nvec;
  const int64_t vv = valid ? v : 0;

  // target (identical in every wave)
  float res[8], tot[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) res[i] = A.base[vv * A.ldbase + i];
  if (A.delta) {
    float dl[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) dl[i] = A.delta[vv * 8 + i];
    if (A.dinv) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float acc = dl[0] * A.dinv[i];
#pragma unroll
        for (int j = 1; j < 8; ++j) acc = __builtin_fmaf(dl[j], A.dinv[j * 8 + i], acc);
        res[i] = res[i] + acc;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) res[i] = res[i] + dl[i];
    }
  }
  if (A.in_div != 1.0f) {
#pragma unroll
    for (int i = 0; i < 8; ++i) res[i] = res[i] / A.in_div;
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) tot[i] = 0.0f;

  for (int s = 0; s < A.st.n; ++s) {
    const float sc = A.st.scale[s];
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = res[i] / sc;
    unsigned long long best;
    if (A.st.kind[s] == QS_STAGE_E8P) {
      best = ~0ull;
      for (int sb = 0; sb < 2; ++sb) {
        float a[8];
        uint32_t sx = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float xs = sb == 0 ? x[i] + 0.25f : x[i] - 0.25f;
          a[i] = fabsf(xs);
          sx ^= __float_as_uint(xs) >> 31;
        }
        const bool z7 = (sb == 0 ? x[7] + 0.25f : x[7] - 0.25f) == 0.0f;
        const bool p_pos = sx & 1;
        const bool p_neg = p_pos ^ !z7;
        for (int rr = 0; rr < 256 / kWaves; ++rr) {
          const int r = wave * (256 / kWaves) + rr;
          float T[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) T[i] = fabsf(kE8P.v[r][i]);
          const bool odd = kE8P.v[r][7] < 0.0f ? p_neg : p_pos;
          const float d2 = e8p_row_d2(a, T, odd);
          const unsigned long long key =
              ((unsigned long long)__float_as_uint(d2) << 9) | ((unsigned)sb << 8) | (unsigned)r;
          if (key < best) best = key;
        }
      }
    } else {
      best = ~0ull;
      for (int rr = 0; rr < 256 / kWaves; ++rr) {
        const int r = wave * (256 / kWaves) + rr;
        float d2 = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          float d = x[i] - kE81.v[r][i];
          float sq = d * d;
          d2 = i == 0 ? sq : d2 + sq;
        }
        const unsigned long long key = ((unsigned long long)__float_as_uint(d2) << 8) | (unsigned)r;
        if (key < best) best = key;
      }
    }
    keys[s & 1][wave][lane] = best;
    __syncthreads();
    unsigned long long win = keys[s & 1][0][lane];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) {
      unsigned long long k2 = keys[s & 1][w][lane];
      win = k2 < win ? k2 : win;
    }
    float q[8];
    uint32_t code;
    if (A.st.kind[s] == QS_STAGE_E8P) {
      const int r = (int)(win & 0xFF);
      const int sb = (int)((win >> 8) & 1);
      code = e8p_finish(x, sb, r, q);
    } else {
      const int r = (int)(win & 0xFF);
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = kE81.v[r][i];
      code = (uint32_t)r;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float qs = q[i] * sc;
      tot[i] = tot[i] + qs;
      res[i] = res[i] - qs;
    }
    if (wave == 0 && valid && A.codes)
      store_code(A.codes, A.code_bytes, s * A.code_stage_stride + v * A.code_stride, code);
  }
  if (A.out_mul != 1.0f) {
#pragma unroll
    for (int i = 0; i < 8; ++i) tot[i] = tot[i] * A.out_mul;
  }
  if (wave == 0 && valid) {
    if (A.vals) {
#pragma unroll
      for (int i = 0; i < 8; ++i) A.vals[v * A.ldvals + i] = tot[i];
    }
    if (A.resid) {
#pragma unroll
      for (int i = 0; i < 8; ++i) A.resid[v * A.ldresid + i] = A.w[v * A.ldw + i] - tot[i];
    }
  }
}

// Least 64-bit key over the wave.
__device__ __forceinline__ unsigned long long wave_min_key(unsigned long long k) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const unsigned lo = __shfl_xor((unsigned)k, off), hi = __shfl_xor((unsigned)(k >> 32), off);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    k = o < k ? o : k;
  }
  return k;
}

// The stages of the target res (the same in every lane of the wave) on one
// wave: lane l evaluates table rows l + 64 k (k < 4) at both shifts and the
// wave takes the least key -- rvq_encode_kernel's keys and minimum, so its
// codes and values.  tot = the sum of the stage values; res is left as the
// residual; lane 0 stores the code of stage s at codes + s stage_stride + off.
__device__ __forceinline__ void wave_encode(const StageCfg& st, float (&res)[8], float (&tot)[8], int lane,
                                            void* codes, int code_bytes, int64_t stage_stride, int64_t off) {
#pragma unroll
  for (int i = 0; i < 8; ++i) tot[i] = 0.0f;
  for (int s = 0; s < st.n; ++s) {
    const float sc = st.scale[s];
    float x[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) x[i] = res[i] / sc;
    unsigned long long best = ~0ull;
    if (st.kind[s] == QS_STAGE_E8P) {
      for (int sb = 0; sb < 2; ++sb) {
        float a[8];
        bool p_pos, p_neg;
        e8p_shifted(x, sb, a, p_pos, p_neg);
        // two table rows per iteration: their loads overlap (4096-row
        // refinement chunk 2.3 % faster than one row per iteration; all four
        // at once took 147 registers, too many for four waves per SIMD)
#pragma unroll 2
        for (int k = 0; k < 256 / 64; ++k) {
          const unsigned long long key = e8p_key(a, p_pos, p_neg, sb, lane + 64 * k);
          if (key < best) best = key;
        }
      }
    } else {
#pragma unroll 2
      for (int k = 0; k < 256 / 64; ++k) {
        const unsigned long long key = e81_key(x, lane + 64 * k);
        if (key < best) best = key;
      }
    }
    const unsigned long long win = wave_min_key(best);
    float q[8];
    uint32_t code;
    if (st.kind[s] == QS_STAGE_E8P) {
      code = e8p_finish(x, (int)((win >> 8) & 1), (int)(win & 0xFF), q);
    } else {
      const int r = (int)(win & 0xFF);
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = kE81.v[r][i];
      code = (uint32_t)r;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float qs = q[i] * sc;
      tot[i] = tot[i] + qs;
      res[i] = res[i] - qs;
    }
    if (lane == 0 && codes) store_code(codes, code_bytes, s * stage_stride + off, code);
  }
}

// rvq_encode_kernel for short calls (the BlockLDLQ rounding step encodes one
// 8-column block of m rows): one vector per wave (wave_encode), so a step of
// 4096 rows runs 4096 waves instead of 64 work-groups of one vector per lane.
__global__ __launch_bounds__(kVecWaves * 64) void rvq_encode_wave_kernel(EncodeArgs A) {
  const int lane = threadIdx.x & 63;
  const int64_t v = (int64_t)blockIdx.x * kVecWaves + (threadIdx.x >> 6);
  if (v >= A.nvec) return;  // wave-uniform (the kernel has no barrier)
  float res[8], tot[8];
  encode_target(A, v, res);
  wave_encode(A.st, res, tot, lane, A.codes, A.code_bytes, A.code_stage_stride, v * A.code_stride);
  if (A.out_mul != 1.0f) {
#pragma unroll
    for (int i = 0; i < 8; ++i) tot[i] = tot[i] * A.out_mul;
  }
  if (lane == 0) {
    if (A.vals) {
#pragma unroll
      for (int i = 0; i < 8; ++i) A.vals[v * A.ldvals + i] = tot[i];
    }
    if (A.resid) {
#pragma unroll
      for (int i = 0; i < 8; ++i) A.resid[v * A.ldresid + i] = A.w[v * A.ldw + i] - tot[i];
    }
  }
}

// A chunk of blocks c0 .. c0 + nb - 1 of the BlockLDLQ refinement pass, the
// blocks in descending order, one row per wave: for block k
//   delta = p[row][8 (k - c0) ..] + E[row][chunk columns] . H[chunk rows][block k]
//   target = wq[row][block k] + delta . dinv[k]
// then the stages (wave_encode), wq and E of block k rewritten.  The chunk's
// columns of E stay in registers (lane l: columns l and l + 64 of the chunk).
constexpr int kChunkBlocks = 16;  // blocks per chunk (8 * 16 = 128 columns: two per lane)
struct ChunkArgs {
  const float* w;
  int64_t ldw;
  float* wq;
  int64_t ldwq;
  float* e;
  int64_t lde;
  const float* p;  // [m][8 nb]: the product of E with H's block columns outside the chunk
  int64_t ldp;
  const float* h;  // H's rows of the chunk (row c0 8 of H), ldh per row
  int64_t ldh;
  const float* dinv;  // [T][8][8]
  int c0, nb;
  int64_t m;
  void* codes;
  int code_bytes;
  int64_t code_stage_stride, code_stride;
  StageCfg st;
};
__global__ __launch_bounds__(kVecWaves * 64) void ldlq_chunk_kernel(ChunkArgs A) {
  const int lane = threadIdx.x & 63;
  const int64_t v = (int64_t)blockIdx.x * kVecWaves + (threadIdx.x >> 6);
  if (v >= A.m) return;  // wave-uniform (the kernel has no barrier)
  const int wc = 8 * A.nb;
  float ec[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int c = lane + 64 * i;
    ec[i] = c < wc ? A.e[v * A.lde + 8 * A.c0 + c] : 0.0f;
  }
  for (int kk = A.nb - 1; kk >= 0; --kk) {
    const int k = A.c0 + kk;
    float part[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) part[j] = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      // rows past the chunk load row 0 and are selected away (no load under a branch)
      const int c = lane + 64 * i;
      const float* hr = A.h + (int64_t)(c < wc ? c : 0) * A.ldh + 8 * k;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const float f = __builtin_fmaf(ec[i], hr[j], part[j]);
        part[j] = c < wc ? f : part[j];
      }
    }
    float dl[8], res[8], tot[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      float t = part[j];
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) t = t + __shfl_xor(t, off);  // the same sum in every lane
      dl[j] = A.p[v * A.ldp + 8 * kk + j] + t;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) res[i] = A.wq[v * A.ldwq + 8 * k + i];
    add_delta(res, dl, A.dinv + 64 * k);
    wave_encode(A.st, res, tot, lane, A.codes, A.code_bytes, A.code_stage_stride, v * A.code_stride + k);
    float r8[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) r8[i] = A.w[v * A.ldw + 8 * k + i] - tot[i];
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        A.wq[v * A.ldwq + 8 * k + i] = tot[i];
        A.e[v * A.lde + 8 * k + i] = r8[i];
      }
    }
    // block k's new E into the lanes that hold its columns
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int cb = lane + 64 * i - 8 * kk;
      float nv = r8[0];
#pragma unroll
      for (int t = 1; t < 8; ++t) nv = cb == t ? r8[t] : nv;
      if (cb >= 0 && cb < 8) ec[i] = nv;
    }
  }
}

int launch_encode(EncodeArgs& A, hipStream_t stream) {
  if (A.nvec == 0) return QS_OK;
  if (A.nvec <= kWaveEncodeMax) {
    const int64_t blocks = (A.nvec + kVecWaves - 1) / kVecWaves;
    hipLaunchKernelGGL(rvq_encode_wave_kernel, dim3((unsigned)blocks), dim3(kVecWaves * 64), 0, stream, A);
    QS_LAUNCHED("rvq_encode_wave_kernel");
    return QS_OK;
  }
  const int64_t blocks = (A.nvec + kVecPerBlock - 1) / kVecPerBlock;
  QS_REQUIRE(blocks < (1ll << 31), "too many vectors: %lld", (long long)A.nvec);
  hipLaunchKernelGGL(rvq_encode_kernel, dim3((unsigned)blocks), dim3(kWaves * 64), 0, stream, A);
  QS_LAUNCHED("rvq_encode_kernel");
  return QS_OK;
}

int fill_stages(StageCfg& st, int nstages, const int* kinds, const float* scales) {
  QS_REQUIRE(nstages >= 1 && nstages <= QS_MAX_STAGES, "nstages must be in [1, %d], got %d",
             QS_MAX_STAGES, nstages);
  QS_REQUIRE(kinds && scales, "kinds and scales must be host arrays");
  st.n = nstages;
  for (int s = 0; s < nstages; ++s) {
    QS_REQUIRE(kinds[s] == QS_STAGE_E8P || kinds[s] == QS_STAGE_E8_1BIT, "bad stage kind %d", kinds[s]);
    QS_REQUIRE(scales[s] != 0.0f, "stage scale must be non-zero");
    st.kind[s] = kinds[s];
    st.scale[s] = scales[s];
  }
  return QS_OK;
}

// ---------------------------------------------------------------------------
// decode
// ---------------------------------------------------------------------------
struct DecodeArgs {
  const void* codes;
  int code_bytes;
  int64_t stage_stride;
  int64_t nvec;
  StageCfg st;
  float out_scale;
  float* out;
};

__device__ __forceinline__ void e8p_decode(uint32_t c, float v[8]) {
  const int a = (c >> 8) & 0xFF;
  uint32_t par = 0;
  const float sh = (c & 1) ? 0.25f : -0.25f;
#pragma unroll
  for (int i = 0; i < 7; ++i) {
    uint32_t f = (c >> (7 - i)) & 1;
    par ^= f;
    float t = kE8P.v[a][i];
    v[i] = (f ? -t : t) + sh;
  }
  float t7 = kE8P.v[a][7];
  v[7] = (par ? -t7 : t7) + sh;
}

__global__ __launch_bounds__(256) void rvq_decode_kernel(DecodeArgs A) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= A.nvec) return;
  float tot[8];
  for (int s = 0; s < A.st.n; ++s) {
    uint32_t c = load_code(A.codes, A.code_bytes, s * A.stage_stride + k);
    float v[8];
    if (A.st.kind[s] == QS_STAGE_E8P) {
      e8p_decode(c & 0xFFFF, v);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) v[i] = kE81.v[c & 0xFF][i];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float vs = v[i] * A.st.scale[s];
      tot[i] = s == 0 ? vs : tot[i] + vs;
    }
  }
  float4* o = reinterpret_cast<float4*>(A.out + k * 8);
  o[0] = make_float4(tot[0] * A.out_scale, tot[1] * A.out_scale, tot[2] * A.out_scale, tot[3] * A.out_scale);
  o[1] = make_float4(tot[4] * A.out_scale, tot[5] * A.out_scale, tot[6] * A.out_scale, tot[7] * A.out_scale);
}

// ---------------------------------------------------------------------------
// repack for the forward kernels
// ---------------------------------------------------------------------------
// Kernel form of an E8P code: [f1 f2 f3 q | abs_idx | f4 f5 f6 | shift], where
// f_i is the flip of coordinate i and q = f0^f1^f2^f3.  Then (e >> 4) indexes
// the table of signed coordinates 0..3 and ((e >> 1) & 0xFFF) the table of
// signed coordinates 4..7 (coordinate 7's flip is q^f4^f5^f6, the parity of
// the seven stored flips).
__device__ __forceinline__ uint32_t kernel_form(uint32_t c) {
  const uint32_t a = (c >> 8) & 0xFF;
  const uint32_t f0 = (c >> 7) & 1, f1 = (c >> 6) & 1, f2 = (c >> 5) & 1, f3 = (c >> 4) & 1;
  const uint32_t f4 = (c >> 3) & 1, f5 = (c >> 2) & 1, f6 = (c >> 1) & 1, sh = c & 1;
  const uint32_t q = f0 ^ f1 ^ f2 ^ f3;
  return (f1 << 15) | (f2 << 14) | (f3 << 13) | (q << 12) | (a << 4) | (f4 << 3) | (f5 << 2) |
         (f6 << 1) | sh;
}

struct PackArgs {
  const void* codes;
  int code_bytes;
  int64_t m, T;
  int kind;
  int layout;
  void* out;
};

__global__ __launch_bounds__(256) void pack_kernel(PackArgs A) {
  const int64_t k = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (k >= A.m * A.T) return;
  const int64_t r = k / A.T, t = k % A.T;
  uint32_t c = load_code(A.codes, A.code_bytes, k);
  int64_t o = k;
  if (A.layout == QS_LAYOUT_TILED) {
    const int64_t S = A.T / 32;
    const int64_t rb = r >> 4, rr = r & 15, sl = t >> 5, tt = t & 31;
    const int64_t lane = (tt >> 3) * 16 + rr;
    o = ((rb * S + sl) * 64 + lane) * 8 + (tt & 7);
  }
  if (A.kind == QS_STAGE_E8P) {
    static_cast<uint16_t*>(A.out)[o] =
        (uint16_t)(A.layout == QS_LAYOUT_TILED ? kernel_form(c & 0xFFFF) : (c & 0xFFFF));
  } else {
    static_cast<uint8_t*>(A.out)[o] = (uint8_t)(c & 0xFF);
  }
}

__global__ __launch_bounds__(256) void div_kernel(const float* in, float* out, int64_t n, float d) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i < n) out[i] = in[i] / d;
}

}  // namespace
}  // namespace qs

using namespace qs;

extern "C" int qs_div_f32(const float* in, float* out, int64_t count, float divisor, qs_stream_t stream) {
  QS_REQUIRE(count >= 0, "count must be >= 0");
  QS_REQUIRE(divisor != 0.0f, "divisor must be non-zero");
  if (count == 0) return QS_OK;
  QS_REQUIRE(in && out, "null pointer");
  QS_REQUIRE((count + 255) / 256 < (1ll << 31), "count too large");
  hipLaunchKernelGGL(div_kernel, dim3((unsigned)((count + 255) / 256)), dim3(256), 0, as_stream(stream), in, out,
                     count, divisor);
  QS_LAUNCHED("div_kernel");
  return QS_OK;
}

extern "C" int qs_e8p_abs_table(float* out_host) {
  QS_REQUIRE(out_host, "null output");
  for (int r = 0; r < 256; ++r)
    for (int i = 0; i < 8; ++i) out_host[r * 8 + i] = kE8PHost.v[r][i];
  return QS_OK;
}

extern "C" int qs_e81_table(float* out_host) {
  QS_REQUIRE(out_host, "null output");
  for (int r = 0; r < 256; ++r)
    for (int i = 0; i < 8; ++i) out_host[r * 8 + i] = kE81Host.v[r][i];
  return QS_OK;
}

extern "C" int qs_rvq_encode(const float* x, int64_t ldx, int64_t nvec, int nstages, const int* kinds,
                             const float* scales, float in_div, float out_mul, float* vals, int64_t ldv,
                             void* codes, int code_bytes, int64_t code_stage_stride, int64_t code_stride,
                             qs_stream_t stream) {
  QS_REQUIRE(nvec >= 0, "nvec must be >= 0");
  QS_REQUIRE(nvec == 0 || x, "null input");
  QS_REQUIRE(ldx >= 8 && (!vals || ldv >= 8), "row strides must be >= 8");
  QS_REQUIRE(!codes || code_bytes == 2 || code_bytes == 4 || code_bytes == 8, "code_bytes must be 2, 4 or 8");
  EncodeArgs A{};
  int rc = fill_stages(A.st, nstages, kinds, scales);
  if (rc) return rc;
  A.base = x;
  A.ldbase = ldx;
  A.vals = vals;
  A.ldvals = ldv;
  A.codes = codes;
  A.code_bytes = code_bytes;
  A.code_stage_stride = code_stage_stride;
  A.code_stride = code_stride;
  A.nvec = nvec;
  A.in_div = in_div;
  A.out_mul = out_mul;
  QS_REQUIRE(in_div != 0.0f, "in_div must be non-zero");
  return launch_encode(A, as_stream(stream));
}

extern "C" int qs_ldlq_step(const float* base, int64_t ldbase, const float* delta, const float* dinv,
                            const float* w, int64_t ldw, float* wq, int64_t ldwq, float* resid,
                            int64_t ldresid, int64_t m, int nstages, const int* kinds, const float* scales,
                            void* codes, int code_bytes, int64_t code_stage_stride, int64_t code_stride,
                            qs_stream_t stream) {
  QS_REQUIRE(m >= 0, "m must be >= 0");
  QS_REQUIRE(m == 0 || (base && delta && wq), "base, delta and wq are required");
  QS_REQUIRE(!resid || w, "resid needs w");
  QS_REQUIRE(ldbase >= 8 && ldwq >= 8 && (!resid || (ldw >= 8 && ldresid >= 8)), "row strides must be >= 8");
  QS_REQUIRE(!codes || code_bytes == 2 || code_bytes == 4 || code_bytes == 8, "code_bytes must be 2, 4 or 8");
  EncodeArgs A{};
  int rc = fill_stages(A.st, nstages, kinds, scales);
  if (rc) return rc;
  A.base = base;
  A.ldbase = ldbase;
  A.delta = delta;
  A.dinv = dinv;
  A.vals = wq;
  A.ldvals = ldwq;
  A.w = w;
  A.ldw = ldw;
  A.resid = resid;
  A.ldresid = ldresid;
  A.codes = codes;
  A.code_bytes = code_bytes;
  A.code_stage_stride = code_stage_stride;
  A.code_stride = code_stride;
  A.nvec = m;
  A.in_div = 1.0f;
  A.out_mul = 1.0f;
  return launch_encode(A, as_stream(stream));
}

extern "C" int qs_ldlq_chunk(const float* w, int64_t ldw, float* wq, int64_t ldwq, float* e, int64_t lde,
                             const float* p, int64_t ldp, const float* h, int64_t ldh, const float* dinv, int c0,
                             int nb, int64_t m, int nstages, const int* kinds, const float* scales, void* codes,
                             int code_bytes, int64_t code_stage_stride, int64_t code_stride, qs_stream_t stream) {
  QS_REQUIRE(m >= 0 && nb >= 1 && nb <= kChunkBlocks && c0 >= 0, "m %lld, nb %d (1..%d), c0 %d", (long long)m, nb,
             kChunkBlocks, c0);
  QS_REQUIRE(m == 0 || (w && wq && e && p && h && dinv), "w, wq, e, p, h and dinv are required");
  QS_REQUIRE(ldw >= 8 * (c0 + nb) && ldwq >= 8 * (c0 + nb) && lde >= 8 * (c0 + nb) && ldp >= 8 * nb &&
                 ldh >= 8 * (c0 + nb),
             "row strides too small");
  QS_REQUIRE(!codes || code_bytes == 2 || code_bytes == 4 || code_bytes == 8, "code_bytes must be 2, 4 or 8");
  ChunkArgs A{};
  int rc = fill_stages(A.st, nstages, kinds, scales);
  if (rc) return rc;
  if (m == 0) return QS_OK;
  QS_REQUIRE((m + kVecWaves - 1) / kVecWaves < (1ll << 31), "m too large: %lld", (long long)m);
  A.w = w;
  A.ldw = ldw;
  A.wq = wq;
  A.ldwq = ldwq;
  A.e = e;
  A.lde = lde;
  A.p = p;
  A.ldp = ldp;
  A.h = h;
  A.ldh = ldh;
  A.dinv = dinv;
  A.c0 = c0;
  A.nb = nb;
  A.m = m;
  A.codes = codes;
  A.code_bytes = code_bytes;
  A.code_stage_stride = code_stage_stride;
  A.code_stride = code_stride;
  hipLaunchKernelGGL(ldlq_chunk_kernel, dim3((unsigned)((m + kVecWaves - 1) / kVecWaves)), dim3(kVecWaves * 64), 0,
                     as_stream(stream), A);
  QS_LAUNCHED("ldlq_chunk_kernel");
  return QS_OK;
}

extern "C" int qs_rvq_decode(const void* codes, int code_bytes, int64_t code_stage_stride, int64_t nvec,
                             int nstages, const int* kinds, const float* scales, float out_scale, float* out,
                             qs_stream_t stream) {
  QS_REQUIRE(nvec >= 0, "nvec must be >= 0");
  QS_REQUIRE(nvec == 0 || (codes && out), "null pointer");
  QS_REQUIRE(code_bytes == 2 || code_bytes == 4 || code_bytes == 8, "code_bytes must be 2, 4 or 8");
  QS_REQUIRE((reinterpret_cast<uintptr_t>(out) & 15) == 0, "out must be 16-byte aligned");
  DecodeArgs A{};
  int rc = fill_stages(A.st, nstages, kinds, scales);
  if (rc) return rc;
  A.codes = codes;
  A.code_bytes = code_bytes;
  A.stage_stride = code_stage_stride;
  A.nvec = nvec;
  A.out_scale = out_scale;
  A.out = out;
  if (nvec == 0) return QS_OK;
  hipLaunchKernelGGL(rvq_decode_kernel, dim3((unsigned)((nvec + 255) / 256)), dim3(256), 0, as_stream(stream), A);
  QS_LAUNCHED("rvq_decode_kernel");
  return QS_OK;
}

extern "C" int qs_pack_codes(const void* codes, int code_bytes, int64_t m, int64_t n, int stage_kind,
                             int layout, void* out, qs_stream_t stream) {
  QS_REQUIRE(m >= 0 && n >= 0 && n % 8 == 0, "n must be a multiple of 8");
  QS_REQUIRE(code_bytes == 2 || code_bytes == 4 || code_bytes == 8, "code_bytes must be 2, 4 or 8");
  QS_REQUIRE(stage_kind == QS_STAGE_E8P || stage_kind == QS_STAGE_E8_1BIT, "bad stage kind");
  QS_REQUIRE(layout == QS_LAYOUT_ROWMAJOR || layout == QS_LAYOUT_TILED, "bad layout");
  if (layout == QS_LAYOUT_TILED)
    QS_REQUIRE(m % 16 == 0 && n % 256 == 0, "tiled layout needs m %% 16 == 0 and n %% 256 == 0 (m=%lld n=%lld)",
               (long long)m, (long long)n);
  const int64_t total = m * (n / 8);
  if (total == 0) return QS_OK;
  QS_REQUIRE(codes && out, "null pointer");
  PackArgs A{codes, code_bytes, m, n / 8, stage_kind, layout, out};
  hipLaunchKernelGGL(pack_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, as_stream(stream), A);
  QS_LAUNCHED("pack_kernel");
  return QS_OK;
}
