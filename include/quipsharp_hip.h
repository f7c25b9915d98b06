/*
 * quipsharp_hip.h -- C ABI of libquipsharp_hip.so, the MI355X (gfx950) kernels
 * behind the quipsharp_amd Python package.
 *
 * Conventions
 *   - Every pointer argument is a device pointer unless stated otherwise;
 *     tensors are dense with the strides given in elements.
 *   - Every entry point enqueues work on `stream` (a hipStream_t; NULL is the
 *     default stream) and returns without synchronising.  Entry points are
 *     reentrant: the library keeps no mutable global state besides the
 *     per-thread error string.
 *   - Return value: QS_OK, or an error code with a message available from
 *     qs_last_error() on the calling thread.  Argument errors are detected on
 *     the host before anything is launched.
 *   - No entry point allocates memory; callers pass workspaces.
 *
 * Reference: numbersletter/quipsharp (pure PyTorch).  Each entry point names
 * the reference function(s) whose computation it performs.
 */
#ifndef QUIPSHARP_HIP_H
#define QUIPSHARP_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef void *qs_stream_t;

enum {
  QS_OK = 0,
  QS_ERR_INVALID = 1,     /* bad argument (shape, stride, dtype, null pointer) */
  QS_ERR_HIP = 2,         /* the HIP runtime reported an error */
  QS_ERR_UNSUPPORTED = 3  /* valid request outside what these kernels implement */
};

enum { QS_STAGE_E8P = 0, QS_STAGE_E8_1BIT = 1 };          /* residual-VQ stage codebooks */
enum { QS_DTYPE_F32 = 0, QS_DTYPE_F16 = 1, QS_DTYPE_BF16 = 2 };
enum { QS_LAYOUT_ROWMAJOR = 0, QS_LAYOUT_TILED = 1 };     /* packed-code layouts */
/* Flag OR'd into qs_linear_forward's layout (QS_LAYOUT_TILED only): su and sv
 * point to packed sign bits instead of fp32 vectors -- uint32 words, bit
 * (i % 32) of word i / 32 set for element i = -1, clear for +1 -- a 32nd of
 * the bytes every work-group of the transforms reads.  Accepted when n and m
 * are both on the chunk scheme (multiples of 256, at most 12288, length / odd
 * factor >= 256), or for a call the one-launch kernel covers with its output
 * transform in the launch (1-2 rows, x rows 8-byte aligned -- 16-byte for
 * fp32 -- with a row stride that is a multiple of 4, m and n multiples of
 * 256 up to 32768, n up to 16384 for fp16 / fp32 x); QS_ERR_UNSUPPORTED
 * otherwise. */
#define QS_SIGNS_BITS 0x100

#define QS_ABI_VERSION 1
#define QS_MAX_STAGES 4
#define QS_MAX_KRON 64 /* largest odd factor of a Kronecker transform */
#define QS_MAX_GROUP 4 /* linears per qs_linear_forward_group call */

/* Message of the last failed call on this thread ("" if none). */
const char *qs_last_error(void);
int qs_abi_version(void);

/* Host copies of the device codebook tables, 256 x 8 fp32 each (host pointer).
 * quipsharp/codebooks/e8p.py:84-89 build_abs_table;
 * quipsharp/codebooks/e8_1bit.py:66-70 build_table. */
int qs_e8p_abs_table(float *out_host);
int qs_e81_table(float *out_host);

/* ---------------------------------------------------------------------------
 * Codebook encode / decode
 * ------------------------------------------------------------------------- */

/* Residual-VQ nearest-codeword encode of nvec 8-vectors, bit-exact with the
 * reference's fp32 CPU arithmetic (ties resolved the same way).
 *   quipsharp/rvq.py:69-80 rvq_quantize, with stage codebooks
 *   quipsharp/codebooks/e8p.py:104-171 (E8PCodebook.quantize) and
 *   quipsharp/codebooks/e8_1bit.py:80-83 (E8OneBitCodebook.quantize).
 * A single stage of scale 1.0 is exactly E8PCodebook.quantize /
 * E8OneBitCodebook.quantize.  The input is first divided by in_div and the
 * summed output multiplied by out_mul (IEEE fp32; 1.0 leaves values
 * unchanged), which is ``codebook.quantize(x / s)`` followed by ``vals * s``
 * of the scale sweep quipsharp/rvq.py:28-37.
 *   x      [nvec][ldx] fp32 (first 8 of each row used)
 *   kinds, scales: host arrays of nstages (1..QS_MAX_STAGES) entries
 *   vals   [nvec][ldv] fp32 output, the summed dequantized approximation (may be NULL)
 *   codes  output, element (s, k) at codes + s*code_stage_stride + k*code_stride,
 *          code_bytes 2 (int16/uint16), 4 (int32) or 8 (int64); may be NULL. */
int qs_rvq_encode(const float *x, int64_t ldx, int64_t nvec, int nstages, const int *kinds,
                  const float *scales, float in_div, float out_mul, float *vals, int64_t ldv,
                  void *codes, int code_bytes, int64_t code_stage_stride, int64_t code_stride,
                  qs_stream_t stream);

/* out[i] = in[i] / divisor, IEEE fp32 (torch's CPU ``tensor / float``,
 * e.g. quipsharp/quantize.py:85 ``what / layer_scale``).  out may equal in. */
int qs_div_f32(const float *in, float *out, int64_t count, float divisor, qs_stream_t stream);

/* Decode: out[k][0..7] = (sum_s fl(Q_s(code_s,k) * scales[s])) * out_scale,
 * every product and sum rounded as in quipsharp/rvq.py:83-88 followed by the
 * ``* layer.scale`` of quipsharp/quantize.py:113.  Codes are read as unsigned
 * 16-bit values (E8P) or 8-bit values (E8 1-bit) of width code_bytes. */
int qs_rvq_decode(const void *codes, int code_bytes, int64_t code_stage_stride, int64_t nvec,
                  int nstages, const int *kinds, const float *scales, float out_scale,
                  float *out, qs_stream_t stream);

/* One BlockLDLQ rounding step on block column k, fused:
 *   target = base + delta            (dinv == NULL, base pass, ldlq.py:126-128)
 *   target = base + delta @ dinv     (dinv = 8x8 fp32, refinement, ldlq.py:136-138)
 *   q      = rvq_quantize(target)    (the codebook callback, quantize.py:90-93)
 *   wq[r][0..7] = q ; resid[r][0..7] = w[r][0..7] - q  (resid may be NULL)
 *   codes  written like qs_rvq_encode.
 * base, w, wq, resid are row-strided views (ld* elements per row) of m rows;
 * delta is [m][8] contiguous.  base may alias wq. */
int qs_ldlq_step(const float *base, int64_t ldbase, const float *delta, const float *dinv,
                 const float *w, int64_t ldw, float *wq, int64_t ldwq, float *resid,
                 int64_t ldresid, int64_t m, int nstages, const int *kinds, const float *scales,
                 void *codes, int code_bytes, int64_t code_stage_stride, int64_t code_stride,
                 qs_stream_t stream);

/* A chunk of nb <= 16 blocks c0 .. c0 + nb - 1 of the BlockLDLQ refinement
 * pass (ldlq.py:132-139), in descending block order, all in one launch: for
 * each row r and block k
 *   delta  = p[r][8 (k - c0) .. + 7] + sum_{c < 8 nb} e[r][8 c0 + c] * h[c][8 k .. 8 k + 7]
 *   target = wq[r][8 k ..] + delta @ dinv[k]          (dinv: [T][8][8] fp32)
 *   then as qs_ldlq_step: wq[r][8 k ..] = q, e[r][8 k ..] = w[r][8 k ..] - q, codes.
 * w, wq, e, p are row-strided views of m rows (e is the error W - Wq, its
 * chunk columns read as the pass leaves them); h points at row 8 c0 of H (ldh
 * per row); p holds the product of E with H's block columns of the chunk
 * over the columns outside the chunk (E @ H[:, chunk] - E[:, chunk] @
 * H[chunk, chunk], taken at the chunk's start).  No counterpart in the
 * reference, which forms E @ H[:, block] for each block: the library's
 * BlockLDLQ reads E once per chunk of blocks, and launches once per chunk.
 * Codes agree with qs_ldlq_step's except where the reassociated fp32 sums
 * move a near-tie. */
int qs_ldlq_chunk(const float *w, int64_t ldw, float *wq, int64_t ldwq, float *e, int64_t lde, const float *p,
                  int64_t ldp, const float *h, int64_t ldh, const float *dinv, int c0, int nb, int64_t m,
                  int nstages, const int *kinds, const float *scales, void *codes, int code_bytes,
                  int64_t code_stage_stride, int64_t code_stride, qs_stream_t stream);

/* ---------------------------------------------------------------------------
 * Randomized Hadamard transform
 * ------------------------------------------------------------------------- */

/* out = post_axis (.) T_n( pre_axis (.) pre_inner (.) in ) along the middle axis
 * of in viewed as [outer][n][inner] (fp32, contiguous; out may equal in).
 *   kron_p == 1 : T_n is the orthonormal Sylvester Walsh-Hadamard transform,
 *                 bit-exact with quipsharp/hadamard.py:17-40 fwht (stages
 *                 h = 1,2,4,... then * fl(n^-1/2)); n a power of two.
 *   kron_p  > 1 : n = kron_p * 2^k with kron_p odd; T_n = K (x) H_{2^k}, the
 *                 Walsh-Hadamard stages first, then the kron_p x kron_p
 *                 orthogonal symmetric matrix kron_mat (device, fp32, row-major)
 *                 along the outer index.  New transform kind for dims the
 *                 reference routes to RFFT (quipsharp/incoherence.py:115-131).
 * pre_axis/post_axis: length n, pre_inner: length inner; any may be NULL.
 * Signs used by incoherence_process (quipsharp/incoherence.py:48-71),
 * reconstruct_* (:74-83) and transform_input/output (:86-93). */
int qs_rht_f32(const float *in, float *out, int64_t outer, int64_t n, int64_t inner,
               const float *pre_axis, const float *pre_inner, const float *post_axis, int kron_p,
               const float *kron_mat, qs_stream_t stream);

/* ---------------------------------------------------------------------------
 * Quantized linear forward (quipsharp/quantize.py:116-124 linear_forward,
 * quipsharp/checkpoint.py:141-146 QuantizedLinear.forward)
 * ------------------------------------------------------------------------- */

/* Repack reference-layout codes (int16/int32/int64 [m][T], T = n/8, one stage)
 * into the kernel layout.  QS_LAYOUT_TILED needs m % 16 == 0 and n % 256 == 0:
 * tiles of 16 rows x 32 codes, each code re-encoded so both halves of the
 * codeword index a 4096-entry table directly.  stage_kind selects E8P
 * (16-bit output) or E8 1-bit (8-bit output).  QS_LAYOUT_ROWMAJOR keeps the
 * order and writes the low 16 (8) bits. */
int qs_pack_codes(const void *codes, int code_bytes, int64_t m, int64_t n, int stage_kind,
                  int layout, void *out, qs_stream_t stream);

/* Workspace bytes needed by qs_linear_forward for this shape and batch. */
size_t qs_linear_workspace_bytes(int64_t m, int64_t n, int64_t batch, int layout);

/* y = su (.) T_m( layer_scale * W_hat @ T_n(sv (.) x) ) + bias for batch rows,
 * with W_hat decoded on the fly from packed codes:
 *   W_hat[r] = s0 * E8P(codes0[r]) (+ s1 * E8_1bit(codes1[r]) when codes1 != NULL)
 *   x      [batch][ldx] in x_dtype, y [batch][ldy] in y_dtype
 *   codes0 packed E8P codes; codes1 packed second-stage codes or NULL, of kind
 *          kind1 (QS_STAGE_E8_1BIT, or QS_STAGE_E8P on the row-major layout)
 *   sv [n], su [m] fp32 sign vectors (packed bits with QS_SIGNS_BITS in
 *          layout); kron_* as in qs_rht_f32 (p = 1: FWHT)
 *   bias [m] fp32 or NULL
 * Activations enter the matrix cores as fp16 (per-row power-of-two scaled),
 * decoded weights are exact in fp16, accumulation is fp32.
 * The workspace must be zero before its first use (its first 256 bytes hold
 * the epoch: the tag of the one-launch kernel's last partial sums, which each
 * call advances, and the count of the launch that clears old tags from the
 * whole workspace once every 2^20 - 1 calls); calls that may run concurrently
 * need separate workspaces.
 * mv_begin / mv_end: optional hipEvent_t attached to the start of the first
 * and the end of the last decode-matvec kernel (hipExtLaunchKernelGGL start /
 * stop events, so the interval is kernel execution only; NULL: none). */
int qs_linear_forward(const void *x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int64_t m,
                      const void *codes0, const void *codes1, int kind1, int layout, const float *sv,
                      const float *su, int kron_pn, const float *kron_n, int kron_pm,
                      const float *kron_m, float s0, float s1, float layer_scale,
                      const float *bias, void *y, int y_dtype, int64_t ldy, void *workspace,
                      size_t workspace_bytes, void *mv_begin, void *mv_end, qs_stream_t stream);

/* The forward of qs_linear_forward without a workspace argument, for callers
 * that cannot allocate one (code under HIP graph capture, tight serving loops,
 * harnesses that forbid hipMalloc).  No counterpart in the reference.
 * The workspace is a device array in the library's code object, one copy of
 * QS_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; this entry
 * point calls no hipMalloc / hipFree.  Shapes whose workspace
 * (qs_linear_workspace_bytes) exceeds it return QS_ERR_UNSUPPORTED before
 * anything is launched.  Every shape with m, n <= 32768 fits at 1..128 rows;
 * wide prefill batches (256 rows and more) of most shapes do not (11008 x
 * 4096 at 4096 rows needs 219 MB).  Every call on one GPU shares that
 * GPU's array: calls that may overlap on one GPU (other streams, other host
 * threads) race and must be serialised by the caller.  The array is zero when
 * loaded; every call advances the epoch in its first 256 bytes.
 * Outputs are bit-identical to qs_linear_forward on the same inputs. */
#define QS_NOALLOC_SCRATCH_BYTES ((size_t)32 << 20)
int qs_linear_forward_noalloc(const void *x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int64_t m,
                              const void *codes0, const void *codes1, int kind1, int layout, const float *sv,
                              const float *su, int kron_pn, const float *kron_n, int kron_pm,
                              const float *kron_m, float s0, float s1, float layer_scale,
                              const float *bias, void *y, int y_dtype, int64_t ldy, qs_stream_t stream);

/* y = layer_scale * W_hat @ x for batch rows, no transforms: the decode-matvec
 * alone, for inputs already in the transformed basis (the reference's RFFT
 * layers, whose transforms run as FFTs: quipsharp/rfft.py:37-60 around
 * quipsharp/quantize.py:123).  Arguments as in qs_linear_forward (no signs,
 * no bias); n, m <= 32768. */
int qs_decode_matvec(const void *x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int64_t m,
                     const void *codes0, const void *codes1, int kind1, int layout, float s0, float s1,
                     float layer_scale, void *y, int y_dtype, int64_t ldy, void *workspace,
                     size_t workspace_bytes, qs_stream_t stream);

/* One linear of a grouped forward (all linears of a group share x and n). */
typedef struct qs_linear_job {
  const void *codes0;   /* packed E8P codes, QS_LAYOUT_TILED */
  const void *codes1;   /* packed E8 1-bit codes or NULL (the same for every job of a call) */
  int64_t m;
  const float *su, *sv; /* [m], [n] fp32 signs */
  int kron_pm;          /* odd factor of m; kron_m its p x p matrix (NULL when 1) */
  const float *kron_m;
  float s0, s1, layer_scale;
  const float *bias;    /* [m] fp32 or NULL */
  void *y;              /* [batch][ldy] in the call's y_dtype */
  int64_t ldy;
  int sign_bits;        /* nonzero: su and sv are packed sign bits (see QS_SIGNS_BITS); the same for every job */
} qs_linear_job;

/* Workspace bytes for qs_linear_forward_group: ms[count] output sizes. */
size_t qs_linear_group_workspace_bytes(int64_t n, int64_t batch, int count, const int64_t *ms);

/* Several linears that read the same input x in one launch: for each job,
 * y_j = su_j (.) T_m( layer_scale_j * W_hat_j @ T_n(sv_j (.) x) ) + bias_j, the
 * same as qs_linear_forward per job, with the GPU's work-groups shared between
 * the jobs in proportion to m, so their latency chains overlap (q/k/v and
 * gate/up of a decoder layer).  No counterpart in the reference, whose
 * QuantizedLinear.forward (quipsharp/checkpoint.py:141-146) is one linear per
 * call; callers that own several linears of one input use it.
 * At 1-2 rows the group is one launch (n up to 32768; 16384 for fp16 / fp32
 * x); from 3 rows with n <= 12288 each stage of the path (input transforms,
 * decode-matvecs, output transforms; up to 16 rows the decode-matvec launch
 * also applies the output transforms) is one launch for the whole group,
 * except the wide GEMM (17 rows and more), one launch per job; otherwise one
 * qs_linear_forward per job.  Every output is bit-identical to
 * qs_linear_forward of that job, with one exception: above 128 rows, jobs of
 * one shape (m, one stage) whose GEMM tiles together fit one round over the
 * CUs share one wide GEMM launch whose K range is split for the whole group
 * (fewer splits than a job alone), so their outputs equal qs_linear_forward's
 * up to the order of the fp32 partial sums.
 * Requirements: 1 <= count <= QS_MAX_GROUP, tiled layout, n a multiple of 256
 * with n / kron_pn >= 256, codes1 NULL for all jobs or for none.  The workspace (zero before first use, see qs_linear_forward) holds
 * one region per job.  mv_begin / mv_end bracket the decode-matvec launch (or
 * the wide GEMM launches) as in qs_linear_forward. */
int qs_linear_forward_group(const void *x, int x_dtype, int64_t ldx, int64_t batch, int64_t n, int kron_pn,
                            const float *kron_n, int count, const qs_linear_job *jobs, int y_dtype,
                            void *workspace, size_t workspace_bytes, void *mv_begin, void *mv_end,
                            qs_stream_t stream);

/* A pre-operation on the bf16 input rows of a grouped one-launch forward:
 * QS_PREOP_RMSNORM: h' = x + x2 (bf16 add; x itself when x2 is NULL), input =
 * bf16(weight * bf16(h' * rsqrt(mean(h'^2) + eps))) (transformers' residual
 * add and Qwen3RMSNorm), h' written to h_out when it is not NULL.  The
 * results equal qs_dec_rmsnorm followed by qs_linear_forward_group bit for
 * bit. */
enum { QS_PREOP_RMSNORM = 1 };
typedef struct qs_preop {
  int kind;
  const void *x2;      /* residual delta [batch][ldx2] or NULL */
  int64_t ldx2;
  const void *weight;  /* norm weights [n] bf16 */
  void *h_out;         /* h' [batch][ldo] or NULL; must not overlap x or x2 */
  int64_t ldo;
  float eps;
} qs_preop;

/* qs_linear_forward_group on the rows the pre-operation makes of x (bf16),
 * in its launches: no counterpart in the reference (its decoder runs the
 * norm as a framework kernel before each QuantizedLinear.forward,
 * scripts/eval_ppl.py:41-65); for decode loops that would otherwise launch it
 * on its own.  1-2 rows with n a multiple of 256 up to 16384 (inside the
 * one-launch kernel: every work-group redoes the norm, so it pays at one
 * row), or 3-16 rows with n on the multi-row chunk scheme -- a multiple of
 * 256 up to 12288 with n / kron_pn >= 256 -- (inside the input-transform
 * launch, one work-group per row and linear); rows of x, x2 and h_out 8-byte
 * aligned with strides that are multiples of 4, weight 8-byte aligned;
 * anything else returns QS_ERR_UNSUPPORTED (the caller runs the norm on its
 * own).  Outputs and h_out bit-identical to qs_dec_rmsnorm followed by
 * qs_linear_forward_group. */
int qs_linear_forward_group_pre(const void *x, int64_t ldx, int64_t batch, int64_t n, int kron_pn,
                                const float *kron_n, int count, const qs_linear_job *jobs, const qs_preop *pre,
                                int y_dtype, void *workspace, size_t workspace_bytes, qs_stream_t stream);

/* Measurement helper: enqueue a kernel that keeps `stream` busy for about
 * `nanoseconds` (bounded; at most 1 s), so that work enqueued after it runs
 * back to back on the GPU while the host is still submitting. */
int qs_busy_wait(int64_t nanoseconds, qs_stream_t stream);

/* ---------------------------------------------------------------------------
 * Decode-step kernels of the greedy-decode harness (a Qwen3-style decoder
 * around QuantizedLinear layers, one new token per batch row).  No
 * counterpart in the reference, whose evaluation runs transformers' modules
 * around QuantizedLinear.forward (scripts/eval_ppl.py:41-65); these do the
 * same arithmetic as transformers' Qwen3RMSNorm, apply_rotary_pos_emb, the
 * attention over the cache and act_fn(gate) * up, in a few launches per
 * layer.  Tensors are bf16 (uint16 bits) unless stated; `pos` is a device
 * int64, the position of the new token (the same for every row); the kernels
 * that read it write nothing when it is max_len or more.
 * --------------------------------------------------------------------------- */

/* h_out = h + delta (bf16 add; skipped when delta is NULL, then h_out is
 * unused; h_out may alias h), x = weight * bf16(h' * rsqrt(mean(h'^2) + eps))
 * for each of `rows` rows of `dim` (a multiple of 8, at most 32768) with row
 * stride ld; 16-byte aligned buffers.  The sum of squares is taken in the
 * order of the RMSNorm pre-operation of qs_linear_forward_group_pre, so the
 * two give the same rows bit for bit. */
int qs_dec_rmsnorm(const void *h, const void *delta, void *h_out, const void *weight, void *x, int64_t rows,
                   int64_t dim, int64_t ld, float eps, qs_stream_t stream);

/* Per row: q heads [rows][nh][128] get q_norm (RMSNorm over the head dim)
 * then the rotary embedding cos_table / sin_table [max_len][128] at `pos`,
 * into q_out [rows][nh][128]; k heads [rows][nkv][128] get k_norm and the
 * rotary embedding, into k_cache [rows][nkv][max_len][128] at `pos`; v heads
 * are copied into v_cache at `pos`.  head_dim 128. */
int qs_dec_qk_norm_rope(const void *q, const void *k, const void *v, const void *q_norm_w, const void *k_norm_w,
                        const void *cos_table, const void *sin_table, const int64_t *pos, void *q_out,
                        void *k_cache, void *v_cache, int64_t rows, int nh, int nkv, int head_dim, int64_t max_len,
                        float eps, qs_stream_t stream);

/* Attention of the new token over cache positions 0 .. pos: out[row][h * 128
 * + d] (row stride ldo) = softmax(scale q_h . k) . v over the kv head h / (nh /
 * nkv) (at most 16 query heads per kv head), in splits of 64 positions (fp32
 * scores and softmax, bf16 probabilities, fp32 accumulate) combined in a
 * second launch.  workspace: qs_dec_attention_workspace_bytes bytes. */
int64_t qs_dec_attention_workspace_bytes(int64_t rows, int nkv, int64_t max_len);
int qs_dec_attention(const void *q, const void *k_cache, const void *v_cache, const int64_t *pos, void *out,
                     int64_t ldo, void *workspace, int64_t workspace_bytes, int64_t rows, int nh, int nkv,
                     int head_dim, int64_t max_len, float scale, qs_stream_t stream);

/* qs_dec_qk_norm_rope followed by qs_dec_attention in the attention's
 * launches: q, k, v are the raw heads ([rows][nh][128], [rows][nkv][128]);
 * each split forms the normed, rotated queries of its kv group, and the split
 * holding `pos` writes that position's key (normed, rotated) and value into
 * the caches before it reads them.  Same bits as the two calls, without the
 * normed queries in memory. */
int qs_dec_attention_rope(const void *q, const void *k, const void *v, const void *q_norm_w, const void *k_norm_w,
                          const void *cos_table, const void *sin_table, const int64_t *pos, void *k_cache,
                          void *v_cache, void *out, int64_t ldo, void *workspace, int64_t workspace_bytes,
                          int64_t rows, int nh, int nkv, int head_dim, int64_t max_len, float eps, float scale,
                          qs_stream_t stream);

/* out = bf16(silu(gate)) * up (each op rounded to bf16), rows x m (even). */
int qs_dec_silu_mul(const void *gate, const void *up, void *out, int64_t rows, int64_t m, int64_t ldg, int64_t ldu,
                    int64_t ldo, qs_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* QUIPSHARP_HIP_H */
