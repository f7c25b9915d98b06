// Decode-step kernels of the greedy-decode harness: everything a Qwen3-style
// decoder layer does around its quantized linears for one new token per
// batch row, so that a step is a short chain of launches (per layer: norm,
// q/k/v, q/k norm + rotary + cache write, attention, combine, o, norm,
// gate/up, SiLU * up, down) instead of the ~50 small framework kernels of
// transformers' modules.  The arithmetic follows transformers'
// Qwen3RMSNorm, apply_rotary_pos_emb and SiLU MLP on bf16 tensors (each
// framework op rounds to bf16; so do these kernels, at the same points);
// attention keeps the scores and the softmax in fp32 with bf16 probabilities
// into the value product (fp32 accumulate), over the filled cache prefix only.
//
// All row counts, head counts and lengths are checked on the host; the
// position is read on the device (one int64 shared by every batch row), so a
// captured step replays for any position below the cache length.
#include "qs_preop_dev.h"

namespace qs {
namespace {

typedef __bf16 bf16x8v __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
__device__ __forceinline__ float rbf(float f) { return bf(f32_to_bf16(f)); }  // round through bf16

// h_out = h + delta (bf16 add; h_out may be h); x = weight * bf16(h_out *
// rsqrt(mean(h_out^2) + eps)) (transformers' Qwen3RMSNorm.forward).  One
// 1024-thread work-group per row in the activation-quad layout of the
// one-launch forward's loader, with its order of the sum of squares
// (qs_preop_dev.h), so a norm there equals this kernel's bit for bit; each
// element is read and written by one thread, so h_out may alias h.
__global__ __launch_bounds__(1024) void rmsnorm_kernel(const uint16_t* h, const uint16_t* delta, uint16_t* h_out,
                                                       const uint16_t* weight, uint16_t* x, int dim, int64_t ld,
                                                       float eps) {
  __shared__ float wsum[kWaves];
  const LaneX lx = lane_x_init();
  const int64_t r = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63;
  const int S = (dim + 255) / 256;
  const bool two = S > 64;
  uint32_t hv[2][4][2], dv[2][4][2], wv[2][4][2];
#pragma unroll
  for (int rr = 0; rr < 2; ++rr)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 64 * rr + 4 * w + i, e = 256 * c + 4 * lane;
      const bool valid = (rr == 0 || two) && c < S && e < dim;
      uint2 a = make_uint2(0, 0), d = make_uint2(0, 0), wt = make_uint2(0, 0);
      if (valid) {
        a = *reinterpret_cast<const uint2*>(h + r * ld + e);
        if (delta) d = *reinterpret_cast<const uint2*>(delta + r * ld + e);
        wt = *reinterpret_cast<const uint2*>(weight + e);
      }
      hv[rr][i][0] = a.x, hv[rr][i][1] = a.y;
      dv[rr][i][0] = d.x, dv[rr][i][1] = d.y;
      wv[rr][i][0] = wt.x, wv[rr][i][1] = wt.y;
    }
  const bool has_delta = delta != nullptr;
  float ss = rms_quad_resid(hv[0], dv[0], has_delta);
  if (two) ss += rms_quad_resid(hv[1], dv[1], has_delta);
  ss = wave_sum(ss, lx);
  if (lane == 0) wsum[w] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int i = 0; i < kWaves; ++i) tot += wsum[i];
  const float rs = rms_scale(tot, dim, eps);
#pragma unroll
  for (int rr = 0; rr < 2; ++rr) {
    if (rr == 1 && !two) break;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 64 * rr + 4 * w + i, e = 256 * c + 4 * lane;
      if (has_delta && c < S && e < dim)
        *reinterpret_cast<uint2*>(h_out + r * ld + e) = make_uint2(hv[rr][i][0], hv[rr][i][1]);
    }
    rms_quad_apply(hv[rr], wv[rr], rs);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int c = 64 * rr + 4 * w + i, e = 256 * c + 4 * lane;
      if (c < S && e < dim) *reinterpret_cast<uint2*>(x + r * ld + e) = make_uint2(hv[rr][i][0], hv[rr][i][1]);
    }
  }
}

// cos and sin of the rotary embedding at one position, dims l and l + 64.
struct Rot {
  float c0, c1, s0, s1;
};

__device__ __forceinline__ Rot load_rot(const uint16_t* cos_r, const uint16_t* sin_r, int l) {
  return Rot{bf(cos_r[l]), bf(cos_r[l + 64]), bf(sin_r[l]), bf(sin_r[l + 64])};
}

// q_norm / k_norm (RMSNorm over the head dim) and the rotary embedding of
// one 128-wide head, one wave: lane l holds dims l and l + 64 (x0, x1; the
// pair rotate_half mixes) and the norm weights there (w0, w1); o0 / o1 the
// bf16 results.  The sum of squares is a lane-local fma then a fixed
// butterfly, so every kernel that calls this gets the same bits.
__device__ __forceinline__ void norm_rope(float x0, float x1, float w0, float w1, const Rot& r, float eps, LaneX lx,
                                          uint16_t& o0, uint16_t& o1) {
  float ss = __builtin_fmaf(x1, x1, x0 * x0);
  ss += lane_xor<32>(ss, lx);
  ss += lane_xor<16>(ss, lx);
  ss += lane_xor<8>(ss, lx);
  ss += lane_xor<4>(ss, lx);
  ss += lane_xor<2>(ss, lx);
  ss += lane_xor<1>(ss, lx);
  const float rs = 1.0f / sqrtf(__builtin_fmaf(ss, 1.0f / 128.0f, eps));
  const float y0 = rbf(w0 * rbf(x0 * rs)), y1 = rbf(w1 * rbf(x1 * rs));
  // q * cos + rotate_half(q) * sin, rotate_half(q) = (-q[64:], q[:64])
  o0 = f32_to_bf16(rbf(y0 * r.c0) + (-rbf(y1 * r.s0)));
  o1 = f32_to_bf16(rbf(y1 * r.c1) + rbf(y0 * r.s1));
}

// One wave per head of one row: q heads get q_norm and the rotary embedding
// (into q_out), k heads k_norm and the rotary embedding (into the key cache
// at the position), v heads go to the value cache unchanged.
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                                                           const uint16_t* qw, const uint16_t* kw,
                                                           const uint16_t* cos_t, const uint16_t* sin_t,
                                                           const int64_t* pos_p, uint16_t* q_out, uint16_t* kc,
                                                           uint16_t* vc, int nh, int nkv, int64_t max_len,
                                                           float eps) {
  const LaneX lx = lane_x_init();
  const int b = blockIdx.x;
  const int hh = blockIdx.y * 4 + (threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  if (hh >= nh + 2 * nkv) return;
  const int64_t pos = *pos_p;
  if (pos >= max_len) return;  // a position past the cache (a caller's error) writes nothing
  if (hh >= nh + nkv) {  // value head: copy into the cache
    const int g = hh - nh - nkv;
    const uint16_t* src = v + ((int64_t)b * nkv + g) * 128;
    uint16_t* dst = vc + (((int64_t)b * nkv + g) * max_len + pos) * 128;
    dst[l] = src[l];
    dst[l + 64] = src[l + 64];
    return;
  }
  const bool isq = hh < nh;
  const int g = isq ? hh : hh - nh;
  const uint16_t* src = isq ? q + ((int64_t)b * nh + g) * 128 : k + ((int64_t)b * nkv + g) * 128;
  const uint16_t* w = isq ? qw : kw;
  uint16_t o0, o1;
  norm_rope(bf(src[l]), bf(src[l + 64]), bf(w[l]), bf(w[l + 64]), load_rot(cos_t + pos * 128, sin_t + pos * 128, l),
            eps, lx, o0, o1);
  uint16_t* dst = isq ? q_out + ((int64_t)b * nh + g) * 128 : kc + (((int64_t)b * nkv + g) * max_len + pos) * 128;
  dst[l] = o0;
  dst[l + 64] = o1;
}

// Inputs of the q/k norm + rotary step when the attention split does it.
struct RopeIn {
  const uint16_t *k, *v, *qw, *kw, *cos_t, *sin_t;
  float eps;
};

constexpr int kSplit = 64;     // cache positions per attention work-group
constexpr int kQStride = 136;  // bf16 per row of the staged queries / probabilities (rows 16 banks apart)
constexpr int kPartFloats = 16 * 2 + 16 * 128;  // per (row, kv head, split): max, sum, unnormalised output

// One work-group (4 waves) per (split of 64 cache positions, kv head, row):
// scores of the G <= 16 query heads that share the kv head against the
// split's keys on the matrix cores (bf16 16x16x32, rows past G zero), masked
// past the filled length, split-local softmax in fp32, then the probabilities
// (bf16) times the split's values on the matrix cores.  Writes the split's
// per-head max, sum and unnormalised output for attn_combine_kernel.
// ROPE: q holds the raw query heads; each work-group forms the normed,
// rotated queries of its kv group itself, and the split that holds the new
// position (the only one that reads it) forms its key and takes its value,
// uses both from LDS and stores them into the caches at its end, so
// qk_norm_rope_kernel's launch is not needed.
template <bool ROPE>
__global__ __launch_bounds__(256) void attn_split_kernel(const uint16_t* q, uint16_t* kc, uint16_t* vc,
                                                         const int64_t* pos_p, float* part, int nh, int nkv,
                                                         int64_t max_len, int nsplit, float scale, RopeIn ri) {
  __shared__ __attribute__((aligned(16))) uint16_t Qs[16 * kQStride];
  __shared__ __attribute__((aligned(16))) uint16_t Ps[16 * kQStride];
  __shared__ float red[2][4][16];
  const int s = blockIdx.x, g = blockIdx.y, b = blockIdx.z;
  const int64_t len = *pos_p + 1;
  const int64_t p0 = (int64_t)s * kSplit;
  // the combine reads only the filled splits; a position past the cache
  // (a caller's error) writes nothing
  if (p0 >= len || len > max_len) return;
  const int G = nh / nkv;
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, qd = lane >> 4, r16 = lane & 15;
  const LaneX lx = lane_x_init();
  // the split's keys and values are requested first: they depend only on the
  // position, and arrive while the queries are staged
  const uint16_t* kbase = kc + ((int64_t)b * nkv + g) * max_len * 128;
  const uint16_t* vbase = vc + ((int64_t)b * nkv + g) * max_len * 128;
  // scores: wave w, positions p0 + 16 w + r16 (column r16 of the tile)
  int64_t pk = p0 + 16 * w + r16;
  const bool pvalid = pk < len;
  if (!pvalid) pk = len - 1;  // a valid row, masked below
  uint4 kg[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) kg[ks] = *reinterpret_cast<const uint4*>(kbase + pk * 128 + 32 * ks + 8 * qd);
  // values: wave w, dims 32 w + 16 dt + r16, positions p0 + 32 ks + 8 qd + 2 i
  // (+1), clamped into the filled prefix (probability 0 there; any finite
  // cached row)
  uint32_t vg[2][2][4][2];
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = 32 * w + 16 * dt + r16;
        int64_t pa = p0 + 32 * ks + 8 * qd + 2 * i, pb = pa + 1;
        pa = pa < len ? pa : len - 1;
        pb = pb < len ? pb : len - 1;
        vg[dt][ks][i][0] = vbase[pa * 128 + d];
        vg[dt][ks][i][1] = vbase[pb * 128 + d];
      }
  __shared__ __attribute__((aligned(16))) uint16_t Kn[ROPE ? 128 : 8], Vn[ROPE ? 128 : 8];
  const int64_t pos = len - 1;
  const bool own = ROPE && pos < p0 + kSplit;  // the split holds the new position
  const int64_t kv_src = ((int64_t)b * nkv + g) * 128;
  uint16_t kn0 = 0, kn1 = 0;  // wave 0 of the owning split: the new key at lane, lane + 64
  if constexpr (ROPE) {
    // every load first: the wave's query rows w + 4 i (row 0 again past G),
    // the weights, the rotary row, and the new key (wave 0) and value (wave 1)
    float xq[4][2];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = w + 4 * i;
      const uint16_t* src = q + ((int64_t)b * nh + g * G + (row < G ? row : 0)) * 128;
      xq[i][0] = bf(src[lane]);
      xq[i][1] = bf(src[lane + 64]);
    }
    const Rot rot = load_rot(ri.cos_t + pos * 128, ri.sin_t + pos * 128, lane);
    const float qw0 = bf(ri.qw[lane]), qw1 = bf(ri.qw[lane + 64]);
    const float xk0 = bf(ri.k[kv_src + lane]), xk1 = bf(ri.k[kv_src + lane + 64]);
    const float kw0 = bf(ri.kw[lane]), kw1 = bf(ri.kw[lane + 64]);
    if (own && w == 1) {
      Vn[lane] = ri.v[kv_src + lane];
      Vn[lane + 64] = ri.v[kv_src + lane + 64];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int row = w + 4 * i;
      uint16_t o0 = 0, o1 = 0;
      if (row < G) norm_rope(xq[i][0], xq[i][1], qw0, qw1, rot, ri.eps, lx, o0, o1);
      Qs[row * kQStride + lane] = o0;
      Qs[row * kQStride + lane + 64] = o1;
    }
    if (own && w == 0) {
      norm_rope(xk0, xk1, kw0, kw1, rot, ri.eps, lx, kn0, kn1);
      Kn[lane] = kn0;
      Kn[lane + 64] = kn1;
    }
  } else {
    // queries of heads g G .. g G + G - 1: 16 rows x 128, 8 bf16 per thread
    const int row = tid >> 4, c8 = (tid & 15) * 8;
    uint4 val = make_uint4(0, 0, 0, 0);
    if (row < G) val = *reinterpret_cast<const uint4*>(q + (((int64_t)b * nh + g * G + row) * 128 + c8));
    *reinterpret_cast<uint4*>(Qs + row * kQStride + c8) = val;
  }
  __syncthreads();
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const bf16x8v a = __builtin_bit_cast(bf16x8v, *reinterpret_cast<const uint4*>(Qs + r16 * kQStride + 32 * ks + 8 * qd));
    uint4 kb = kg[ks];
    if constexpr (ROPE) {
      // the new position from LDS (its cache row is written at the end)
      const uint4 kl = *reinterpret_cast<const uint4*>(Kn + 32 * ks + 8 * qd);
      if (pk == pos) kb = kl;
    }
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8v, kb), acc, 0, 0, 0);
  }
  // acc[j]: head 4 qd + j, position p0 + 16 w + r16
  float sc[4], mx[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sc[j] = pvalid ? acc[j] * scale : -INFINITY;
    float m = sc[j];
    m = fmaxf(m, lane_xor<8>(m, lx));
    m = fmaxf(m, lane_xor<4>(m, lx));
    m = fmaxf(m, lane_xor<2>(m, lx));
    m = fmaxf(m, lane_xor<1>(m, lx));
    mx[j] = m;
  }
  if (r16 == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) red[0][w][4 * qd + j] = mx[j];
  }
  __syncthreads();
  float ps[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int h = 4 * qd + j;
    const float m = fmaxf(fmaxf(red[0][0][h], red[0][1][h]), fmaxf(red[0][2][h], red[0][3][h]));
    mx[j] = m;
    const float e = pvalid ? __expf(sc[j] - m) : 0.0f;
    const uint16_t eb = f32_to_bf16(e);
    Ps[h * kQStride + 16 * w + r16] = eb;
    float t = bf(eb);  // the sum of the probabilities the value product uses
    t += lane_xor<8>(t, lx);
    t += lane_xor<4>(t, lx);
    t += lane_xor<2>(t, lx);
    t += lane_xor<1>(t, lx);
    ps[j] = t;
  }
  if (r16 == 0) {
#pragma unroll
    for (int j = 0; j < 4; ++j) red[1][w][4 * qd + j] = ps[j];
  }
  __syncthreads();
  float* out = part + (((int64_t)b * nkv + g) * nsplit + s) * kPartFloats;
  if (tid < 16) {
    out[tid] = fmaxf(fmaxf(red[0][0][tid], red[0][1][tid]), fmaxf(red[0][2][tid], red[0][3][tid]));
    out[16 + tid] = (red[1][0][tid] + red[1][1][tid]) + (red[1][2][tid] + red[1][3][tid]);
  }
  // values: wave w, dims 32 w .. 32 w + 31 (two tiles of 16), positions in two k-steps of 32
  // (loaded at the start)
#pragma unroll
  for (int dt = 0; dt < 2; ++dt) {
    const int d = 32 * w + 16 * dt + r16;
    const uint32_t vn = ROPE ? Vn[d] : 0u;  // the new position's value at d
    f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const bf16x8v a = __builtin_bit_cast(bf16x8v, *reinterpret_cast<const uint4*>(Ps + r16 * kQStride + 32 * ks + 8 * qd));
      uint32_t vb[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        uint32_t va = vg[dt][ks][i][0], vv = vg[dt][ks][i][1];
        if constexpr (ROPE) {
          // the positions the loads used (clamped like them): the new one
          // takes its value from LDS, a select of loaded values
          int64_t pa = p0 + 32 * ks + 8 * qd + 2 * i, pb = pa + 1;
          pa = pa < len ? pa : len - 1;
          pb = pb < len ? pb : len - 1;
          va = pa == pos ? vn : va;
          vv = pb == pos ? vn : vv;
        }
        vb[i] = va | (vv << 16);
      }
      o = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8v, make_uint4(vb[0], vb[1], vb[2], vb[3])),
                                                  o, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) out[32 + (4 * qd + j) * 128 + d] = o[j];
  }
  if (own && w < 2) {  // the new position into the caches for the next steps
    uint16_t* dst = (w == 0 ? kc : vc) + (((int64_t)b * nkv + g) * max_len + pos) * 128;
    dst[lane] = w == 0 ? kn0 : Vn[lane];
    dst[lane + 64] = w == 0 ? kn1 : Vn[lane + 64];
  }
}

// Output of head h (row b): the splits' outputs rescaled to the common max,
// summed, divided by the summed probabilities; bf16 into [row][head * 128].
__global__ __launch_bounds__(128) void attn_combine_kernel(const float* part, const int64_t* pos_p, uint16_t* out,
                                                           int nh, int nkv, int nsplit, int64_t ldo, int64_t max_len) {
  const int b = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int G = nh / nkv, g = h / G, hl = h - g * G;
  const int64_t len = *pos_p + 1;
  if (len > max_len) return;  // a position past the cache (a caller's error)
  const int ns = (int)((len + kSplit - 1) / kSplit);
  const float* base = part + ((int64_t)b * nkv + g) * nsplit * kPartFloats;
  // the loads of four splits go out together (the same sums in split order)
  float M = -INFINITY;
#pragma unroll 4
  for (int s = 0; s < ns; ++s) M = fmaxf(M, base[s * kPartFloats + hl]);
  float L = 0.0f, O = 0.0f;
#pragma unroll 4
  for (int s = 0; s < ns; ++s) {
    const float* p = base + s * kPartFloats;
    const float f = __expf(p[hl] - M);
    L += f * p[16 + hl];
    O += f * p[32 + hl * 128 + d];
  }
  out[(int64_t)b * ldo + h * 128 + d] = f32_to_bf16(O / L);
}

// act = bf16(silu(gate)) * up, each op rounded to bf16 (act_fn(gate) * up).
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* gt, const uint16_t* up, uint16_t* out,
                                                       int64_t m, int64_t ldg, int64_t ldu, int64_t ldo) {
  const int64_t r = blockIdx.y;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 2;
  if (i >= m) return;
  const uint32_t a = *reinterpret_cast<const uint32_t*>(gt + r * ldg + i);
  const uint32_t u = *reinterpret_cast<const uint32_t*>(up + r * ldu + i);
  float gv[2] = {bf((uint16_t)(a & 0xFFFF)), bf((uint16_t)(a >> 16))};
  float uv[2] = {bf((uint16_t)(u & 0xFFFF)), bf((uint16_t)(u >> 16))};
  uint32_t o = 0;
#pragma unroll
  for (int k = 0; k < 2; ++k) o |= (uint32_t)f32_to_bf16(silu_bf16(gv[k]) * uv[k]) << (16 * k);
  *reinterpret_cast<uint32_t*>(out + r * ldo + i) = o;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace qs

using namespace qs;

extern "C" int qs_dec_rmsnorm(const void* h, const void* delta, void* h_out, const void* weight, void* x,
                              int64_t rows, int64_t dim, int64_t ld, float eps, qs_stream_t stream) {
  QS_REQUIRE(h && weight && x && rows >= 1 && rows <= 65535 && dim >= 8 && dim % 8 == 0 && dim <= 32768 &&
                 ld >= dim && ld % 8 == 0,
             "qs_dec_rmsnorm: rows %lld, dim %lld (multiple of 8, at most 32768), ld %lld", (long long)rows,
             (long long)dim, (long long)ld);
  QS_REQUIRE(!delta || h_out, "qs_dec_rmsnorm: a residual delta needs h_out");
  QS_REQUIRE(aligned16(h) && aligned16(weight) && aligned16(x) && (!delta || (aligned16(delta) && aligned16(h_out))),
             "qs_dec_rmsnorm: buffers must be 16-byte aligned");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(1024), 0, as_stream(stream),
                     static_cast<const uint16_t*>(h), static_cast<const uint16_t*>(delta), static_cast<uint16_t*>(h_out),
                     static_cast<const uint16_t*>(weight), static_cast<uint16_t*>(x), (int)dim, ld, eps);
  QS_LAUNCHED("rmsnorm_kernel");
  return QS_OK;
}

extern "C" int qs_dec_qk_norm_rope(const void* q, const void* k, const void* v, const void* q_norm_w,
                                   const void* k_norm_w, const void* cos_table, const void* sin_table,
                                   const int64_t* pos, void* q_out, void* k_cache, void* v_cache, int64_t rows, int nh,
                                   int nkv, int head_dim, int64_t max_len, float eps, qs_stream_t stream) {
  QS_REQUIRE(q && k && v && q_norm_w && k_norm_w && cos_table && sin_table && pos && q_out && k_cache && v_cache,
             "qs_dec_qk_norm_rope: null pointer");
  QS_SUPPORTED(head_dim == 128, "qs_dec_qk_norm_rope: head_dim %d (128 only)", head_dim);
  QS_REQUIRE(rows >= 1 && rows <= 65535 && nh >= 1 && nkv >= 1 && nh % nkv == 0 && max_len >= 1,
             "qs_dec_qk_norm_rope: rows %lld, heads %d / %d, cache length %lld", (long long)rows, nh, nkv,
             (long long)max_len);
  hipLaunchKernelGGL(qk_norm_rope_kernel, dim3((unsigned)rows, (unsigned)((nh + 2 * nkv + 3) / 4)), dim3(256), 0,
                     as_stream(stream), static_cast<const uint16_t*>(q), static_cast<const uint16_t*>(k),
                     static_cast<const uint16_t*>(v), static_cast<const uint16_t*>(q_norm_w),
                     static_cast<const uint16_t*>(k_norm_w), static_cast<const uint16_t*>(cos_table),
                     static_cast<const uint16_t*>(sin_table), pos, static_cast<uint16_t*>(q_out),
                     static_cast<uint16_t*>(k_cache), static_cast<uint16_t*>(v_cache), nh, nkv, max_len, eps);
  QS_LAUNCHED("qk_norm_rope_kernel");
  return QS_OK;
}

extern "C" int64_t qs_dec_attention_workspace_bytes(int64_t rows, int nkv, int64_t max_len) {
  const int64_t ns = (max_len + kSplit - 1) / kSplit;
  return rows * nkv * ns * kPartFloats * (int64_t)sizeof(float);
}

namespace {
int attention_checks(const char* fn, int64_t ldo, int64_t workspace_bytes, int64_t rows, int nh, int nkv,
                     int head_dim, int64_t max_len) {
  QS_SUPPORTED(head_dim == 128, "%s: head_dim %d (128 only)", fn, head_dim);
  QS_REQUIRE(rows >= 1 && rows <= 65535 && nh >= 1 && nkv >= 1 && nh % nkv == 0 && nh / nkv <= 16 && max_len >= 1 &&
                 ldo >= (int64_t)nh * 128,
             "%s: rows %lld, heads %d / %d (at most 16 per kv head), cache length %lld, ldo %lld", fn,
             (long long)rows, nh, nkv, (long long)max_len, (long long)ldo);
  QS_REQUIRE(workspace_bytes >= qs_dec_attention_workspace_bytes(rows, nkv, max_len),
             "%s: workspace of %lld bytes, %lld needed", fn, (long long)workspace_bytes,
             (long long)qs_dec_attention_workspace_bytes(rows, nkv, max_len));
  QS_REQUIRE((max_len + kSplit - 1) / kSplit <= 65535, "%s: cache length %lld", fn, (long long)max_len);
  return QS_OK;
}

template <bool ROPE>
int launch_attention(const void* q, void* k_cache, void* v_cache, const int64_t* pos, void* out, int64_t ldo,
                     void* workspace, int64_t rows, int nh, int nkv, int64_t max_len, float scale, const RopeIn& ri,
                     qs_stream_t stream) {
  const int ns = (int)((max_len + kSplit - 1) / kSplit);
  hipLaunchKernelGGL(attn_split_kernel<ROPE>, dim3((unsigned)ns, (unsigned)nkv, (unsigned)rows), dim3(256), 0,
                     as_stream(stream), static_cast<const uint16_t*>(q), static_cast<uint16_t*>(k_cache),
                     static_cast<uint16_t*>(v_cache), pos, static_cast<float*>(workspace), nh, nkv, max_len, ns,
                     scale, ri);
  QS_LAUNCHED("attn_split_kernel");
  hipLaunchKernelGGL(attn_combine_kernel, dim3((unsigned)rows, (unsigned)nh), dim3(128), 0, as_stream(stream),
                     static_cast<const float*>(workspace), pos, static_cast<uint16_t*>(out), nh, nkv, ns, ldo,
                     max_len);
  QS_LAUNCHED("attn_combine_kernel");
  return QS_OK;
}
}  // namespace

extern "C" int qs_dec_attention(const void* q, const void* k_cache, const void* v_cache, const int64_t* pos, void* out,
                                int64_t ldo, void* workspace, int64_t workspace_bytes, int64_t rows, int nh, int nkv,
                                int head_dim, int64_t max_len, float scale, qs_stream_t stream) {
  QS_REQUIRE(q && k_cache && v_cache && pos && out && workspace, "qs_dec_attention: null pointer");
  const int rc = attention_checks("qs_dec_attention", ldo, workspace_bytes, rows, nh, nkv, head_dim, max_len);
  if (rc != QS_OK) return rc;
  QS_REQUIRE(aligned16(q) && aligned16(k_cache), "qs_dec_attention: q and the key cache must be 16-byte aligned");
  // the plain variant only reads the caches
  return launch_attention<false>(q, const_cast<void*>(k_cache), const_cast<void*>(v_cache), pos, out, ldo, workspace,
                                 rows, nh, nkv, max_len, scale, RopeIn{}, stream);
}

extern "C" int qs_dec_attention_rope(const void* q, const void* k, const void* v, const void* q_norm_w,
                                     const void* k_norm_w, const void* cos_table, const void* sin_table,
                                     const int64_t* pos, void* k_cache, void* v_cache, void* out, int64_t ldo,
                                     void* workspace, int64_t workspace_bytes, int64_t rows, int nh, int nkv,
                                     int head_dim, int64_t max_len, float eps, float scale, qs_stream_t stream) {
  QS_REQUIRE(q && k && v && q_norm_w && k_norm_w && cos_table && sin_table && pos && k_cache && v_cache && out &&
                 workspace,
             "qs_dec_attention_rope: null pointer");
  const int rc = attention_checks("qs_dec_attention_rope", ldo, workspace_bytes, rows, nh, nkv, head_dim, max_len);
  if (rc != QS_OK) return rc;
  QS_REQUIRE(aligned16(k_cache), "qs_dec_attention_rope: the key cache must be 16-byte aligned");
  const RopeIn ri{static_cast<const uint16_t*>(k),        static_cast<const uint16_t*>(v),
                  static_cast<const uint16_t*>(q_norm_w), static_cast<const uint16_t*>(k_norm_w),
                  static_cast<const uint16_t*>(cos_table), static_cast<const uint16_t*>(sin_table), eps};
  return launch_attention<true>(q, k_cache, v_cache, pos, out, ldo, workspace, rows, nh, nkv, max_len, scale, ri,
                                stream);
}

extern "C" int qs_dec_silu_mul(const void* gate, const void* up, void* out, int64_t rows, int64_t m, int64_t ldg,
                               int64_t ldu, int64_t ldo, qs_stream_t stream) {
  QS_REQUIRE(gate && up && out && rows >= 1 && rows <= 65535 && m >= 2 && m % 2 == 0 && ldg >= m && ldu >= m &&
                 ldo >= m && ldg % 2 == 0 && ldu % 2 == 0 && ldo % 2 == 0,
             "qs_dec_silu_mul: rows %lld, m %lld (even)", (long long)rows, (long long)m);
  QS_REQUIRE(((reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up) | reinterpret_cast<uintptr_t>(out)) &
              3) == 0,
             "qs_dec_silu_mul: buffers must be 4-byte aligned");
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((m / 2 + 255) / 256), (unsigned)rows), dim3(256), 0,
                     as_stream(stream), static_cast<const uint16_t*>(gate), static_cast<const uint16_t*>(up),
                     static_cast<uint16_t*>(out), m, ldg, ldu, ldo);
  QS_LAUNCHED("silu_mul_kernel");
  return QS_OK;
}
