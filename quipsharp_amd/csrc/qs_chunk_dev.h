// Chunked transform building blocks shared by the forward kernels.
//
// A length-n transform T_n = K_p (x) H_L (n = p L, L = 2^k >= 256) is split
// as T_n = M (x) H_256 over the index i = 256 c + t: a 256-point
// Walsh-Hadamard inside each chunk c (one wave, four values per lane, two
// stages in registers and six across lanes with DPP / permlane exchanges, no
// barrier), then the S x S matrix M = K_p (x) H_{L/256} (S = n / 256) across
// chunks.  Entries of M are generated on the fly: Hadamard signs from a
// popcount, K from LDS.  Work-groups are 16 waves; a wave holds up to three
// chunks (S <= 48, n <= 12288).
#pragma once

#include "qs_rht_dev.h"

namespace qs {

constexpr int kWaves = 16;
constexpr int kMaxN = 12288;
constexpr int kMaxS = kMaxN / 256;    // chunks of 256
constexpr int kCPW = kMaxS / kWaves;  // chunks per wave (3)
constexpr int kYStride = 272;         // floats per chunk row in LDS (consecutive rows 16 banks apart)

// Lane exchanges for the butterflies, all on the VALU: DPP within rows of 16
// lanes, v_permlane16/32_swap across rows.  The swaps return two values (the
// two operands after the swap); which one holds lane ^ 16 (lane ^ 32) is
// found once per thread by swapping the lane ids themselves.
struct LaneX {
  bool pick16, pick32;
};

__device__ __forceinline__ LaneX lane_x_init() {
  const unsigned l = __lane_id();
  const auto r16 = __builtin_amdgcn_permlane16_swap(l, l, false, false);
  const auto r32 = __builtin_amdgcn_permlane32_swap(l, l, false, false);
  return LaneX{r16[0] == (l ^ 16u), r32[0] == (l ^ 32u)};
}

// Value of lane (lane ^ MASK).
template <int MASK>
__device__ __forceinline__ float lane_xor(float v, LaneX lx) {
  const int iv = __builtin_bit_cast(int, v);
  int r;
  if constexpr (MASK == 1) {
    r = __builtin_amdgcn_update_dpp(0, iv, 0xB1, 0xF, 0xF, false);  // quad_perm [1,0,3,2]
  } else if constexpr (MASK == 2) {
    r = __builtin_amdgcn_update_dpp(0, iv, 0x4E, 0xF, 0xF, false);  // quad_perm [2,3,0,1]
  } else if constexpr (MASK == 4) {
    // row_half_mirror (i ^ 7 within 8 lanes), then quad_perm [3,2,1,0] (i ^ 3)
    const int t = __builtin_amdgcn_update_dpp(0, iv, 0x141, 0xF, 0xF, false);
    r = __builtin_amdgcn_update_dpp(0, t, 0x1B, 0xF, 0xF, false);
  } else if constexpr (MASK == 8) {
    r = __builtin_amdgcn_update_dpp(0, iv, 0x128, 0xF, 0xF, false);  // row_ror:8
  } else if constexpr (MASK == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap((unsigned)iv, (unsigned)iv, false, false);
    r = (int)(lx.pick16 ? p[0] : p[1]);
  } else {
    static_assert(MASK == 32, "lane mask");
    const auto p = __builtin_amdgcn_permlane32_swap((unsigned)iv, (unsigned)iv, false, false);
    r = (int)(lx.pick32 ? p[0] : p[1]);
  }
  return __builtin_bit_cast(float, r);
}

// Sum of a float over the 64 lanes of a wave (DPP / permlane exchanges).
__device__ __forceinline__ float wave_sum(float v, LaneX lx) {
  v += lane_xor<32>(v, lx);
  v += lane_xor<16>(v, lx);
  v += lane_xor<8>(v, lx);
  v += lane_xor<4>(v, lx);
  v += lane_xor<2>(v, lx);
  v += lane_xor<1>(v, lx);
  return v;
}

// Butterfly across lanes: the lane with the bit clear keeps a + b, its
// partner a - b (exact: fma with +-1).
template <int MASK, int NC>
__device__ __forceinline__ void lane_stage(float (*v)[4], int lane, LaneX lx) {
  const float sgn = (lane & MASK) ? -1.0f : 1.0f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float o = lane_xor<MASK>(v[c][j], lx);
      v[c][j] = __builtin_fmaf(sgn, v[c][j], o);
    }
}

// Unnormalised 256-point Walsh-Hadamard of each of NC chunks held as element
// t = 4 * lane + j in v[c][j].
template <int NC>
__device__ __forceinline__ void h256(float (*v)[4], int lane, LaneX lx) {
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const float a0 = v[c][0] + v[c][1], a1 = v[c][0] - v[c][1];
    const float a2 = v[c][2] + v[c][3], a3 = v[c][2] - v[c][3];
    v[c][0] = a0 + a2;
    v[c][2] = a0 - a2;
    v[c][1] = a1 + a3;
    v[c][3] = a1 - a3;
  }
  lane_stage<1, NC>(v, lane, lx);
  lane_stage<2, NC>(v, lane, lx);
  lane_stage<4, NC>(v, lane, lx);
  lane_stage<8, NC>(v, lane, lx);
  lane_stage<16, NC>(v, lane, lx);
  lane_stage<32, NC>(v, lane, lx);
}

// h256 over the chunks a wave holds (one for S <= 16, else up to CPW).
template <int CPW>
__device__ __forceinline__ void h256_chunks(float (&v)[CPW][4], int S, int lane, LaneX lx) {
  if constexpr (CPW == 1) {
    h256<1>(v, lane, lx);
  } else {
    if (S <= kWaves) h256<1>(v, lane, lx);
    else h256<CPW>(v, lane, lx);
  }
}


// Entry (r, c) of M = K_p (x) H_{2^lsh}: chunk index r = a * 2^lsh + h.
__device__ __forceinline__ float mmat(int r, int c, int lsh, int p, const float* Ks) {
  const int hm = (1 << lsh) - 1;
  float v = (__builtin_popcount(r & c & hm) & 1) ? -1.0f : 1.0f;
  if (p > 1) v *= Ks[(r >> lsh) * p + (c >> lsh)];
  return v;
}

// Row r of M . Y for the four columns 4 lane .. 4 lane + 3: sum over the S
// chunks c of M[r][c] Y[c][4 lane + j].  r is the same for the whole wave, so
// the coefficients are scalars: the Hadamard sign from a scalar popcount and
// the K factor read once per lane (K[r's a][lane], p <= 64) and broadcast with
// readlane.  Four chunks per step, loads first.
__device__ __forceinline__ float4 mrow_times_chunks(const float* Y, int S, int r, int lsh, int p, const float* Ks,
                                                    int lane) {
  r = __builtin_amdgcn_readfirstlane(r);
  const int hm = (1 << lsh) - 1;
  const float krow = (p > 1 && lane < p) ? Ks[(r >> lsh) * p + lane] : 1.0f;
  float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int c0 = 0; c0 < S; c0 += 4) {
    float4 yv[4];
    float cf[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int c = c0 + k < S ? c0 + k : S - 1;
      yv[k] = *reinterpret_cast<const float4*>(Y + c * kYStride + 4 * lane);
      float v = (__builtin_popcount(r & c & hm) & 1) ? -1.0f : 1.0f;
      if (p > 1)
        v *= __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, krow), c >> lsh));
      cf[k] = c0 + k < S ? v : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      acc.x = __builtin_fmaf(cf[k], yv[k].x, acc.x);
      acc.y = __builtin_fmaf(cf[k], yv[k].y, acc.y);
      acc.z = __builtin_fmaf(cf[k], yv[k].z, acc.z);
      acc.w = __builtin_fmaf(cf[k], yv[k].w, acc.w);
    }
  }
  return acc;
}

// True when a length-len transform with odd factor p fits the chunk scheme.
inline bool chunk_transform_fits(int64_t len, int p) {
  return len % 256 == 0 && len <= kMaxN && (len / p) >= 256;
}

}  // namespace qs
