/*
 * CPU oracle for the QuIP# quantize/dequantize hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, only to compare results
 * against it or to time it as the CPU baseline.
 * The product path (quipsharp_amd) never calls it.
 *
 * Every routine restates the scalar fp32 semantics of the reference's torch
 * code, one IEEE operation at a time, and is compiled with -ffp-contract=off
 * so that no multiply-add is fused.  Citations are to numbersletter/quipsharp.
 *
 * Parity pinning (how each routine is checked, see tests/test_oracle_*.py):
 *   qso_e8p_abs_table   closed form + known answers (227/256 rows, even sums,
 *                       unique, the Appendix C.2 row) + golden table
 *   qso_e81_table       240-vector shell, 256 unique rows + golden table
 *   qso_e8p_decode      paper worked example, lattice membership, golden codes
 *   qso_e8p_encode      golden codes from the reference, brute-force optimality
 *                       over all 65,536 codewords, greedy-vs-128-pattern check
 *   qso_e81_encode      golden indices, brute force (it is brute force)
 *   qso_rvq_encode      golden 3-bit / 4-bit codes
 *   qso_fwht            golden outputs (bit-exact), dense Sylvester matrix
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define DIM 8

/* ------------------------------------------------------------------------ */
/* E8P abs table.  quipsharp/codebooks/e8p.py:64-89                          */
/* ------------------------------------------------------------------------ */

/* The 29 norm^2 = 12 padding rows of Appendix C.1, listed as numerators over
 * 2 (each digit is 1 or 3), in the order of e8p.py:31-61. */
static const char *k_pad29[29] = {
    "31113333", "13113333", "11313333", "11133333", "33313311", "33313131",
    "33311331", "33313113", "33311313", "33311133", "33133311", "33133131",
    "33131331", "33133113", "33131313", "33131133", "31333311", "31333131",
    "31331331", "31333113", "31331313", "13331133", "13333311", "13333131",
    "13331331", "13333113", "13331313", "11331333", "33113331"};

/* Fills out[256*8].  Rows 0..226: every abs pattern over {1/2,3/2,5/2,7/2}^8
 * with squared norm <= 10 (any abs pattern of half-integers has an even-sum
 * signing, so the D8-hat filter of e8p.py:69 keeps all of them), in ascending
 * lexicographic order, which is the order torch.unique(dim=0) returns
 * (e8p.py:72).  Rows 227..255: the padding rows (e8p.py:87).  Finally every
 * row whose coordinate sum is odd has its last coordinate negated
 * (e8p.py:75-81).  Returns the number of enumerated rows (227). */
int qso_e8p_abs_table(float *out) {
    int nrow = 0;
    for (int code = 0; code < (1 << 16); ++code) {
        int k[DIM];
        int s = 0;
        for (int i = 0; i < DIM; ++i) {
            k[i] = (code >> (2 * (DIM - 1 - i))) & 3; /* coordinate 0 most significant */
            s += k[i] * (k[i] + 1);                     /* (k+1/2)^2 = k(k+1) + 1/4 */
        }
        if (s + 2 > 10) continue;
        for (int i = 0; i < DIM; ++i) out[nrow * DIM + i] = (float)k[i] + 0.5f;
        ++nrow;
    }
    int enumerated = nrow;
    for (int r = 0; r < 29; ++r, ++nrow)
        for (int i = 0; i < DIM; ++i) out[nrow * DIM + i] = (float)(k_pad29[r][i] - '0') * 0.5f;
    for (int r = 0; r < nrow; ++r) {
        double sum = 0.0;
        for (int i = 0; i < DIM; ++i) sum += out[r * DIM + i];
        long isum = (long)llround(sum);
        if (isum % 2 != 0) out[r * DIM + DIM - 1] = -out[r * DIM + DIM - 1];
    }
    return enumerated;
}

/* ------------------------------------------------------------------------ */
/* E8 1-bit table.  quipsharp/codebooks/e8_1bit.py:26-70                     */
/* ------------------------------------------------------------------------ */

/* Enumerates base^8 tuples of vals[] in itertools.product / cartesian_prod
 * order (last coordinate fastest) and keeps those with the given squared norm
 * and an even coordinate sum.  Writes at most `cap` rows. */
static int shell(const float *vals, int nv, float norm_sq, float *out, int cap) {
    int total = 1;
    for (int i = 0; i < DIM; ++i) total *= nv;
    int n = 0;
    for (int idx = 0; idx < total && n < cap; ++idx) {
        float v[DIM];
        int rem = idx;
        for (int i = DIM - 1; i >= 0; --i) { v[i] = vals[rem % nv]; rem /= nv; }
        double nsq = 0.0, sum = 0.0;
        for (int i = 0; i < DIM; ++i) { nsq += (double)v[i] * v[i]; sum += v[i]; }
        if (nsq != norm_sq) continue;
        if (fmod(sum, 2.0) != 0.0) continue; /* sum is an integer here */
        memcpy(out + n * DIM, v, sizeof v);
        ++n;
    }
    return n;
}

/* out[256*8]: zero row, 112 integer norm^2=2 rows, 128 half-integer norm^2=2
 * rows, then the first 15 integer norm^2=4 rows. */
int qso_e81_table(float *out) {
    const float ints1[3] = {-1.f, 0.f, 1.f};          /* arange(-1, 2)       */
    const float halves2[4] = {-1.5f, -0.5f, 0.5f, 1.5f}; /* arange(-2, 2)+1/2 */
    const float ints2[5] = {-2.f, -1.f, 0.f, 1.f, 2.f};  /* arange(-2, 3)     */
    memset(out, 0, DIM * sizeof(float));
    int n = 1;
    n += shell(ints1, 3, 2.0f, out + n * DIM, 256 - n);
    n += shell(halves2, 4, 2.0f, out + n * DIM, 256 - n);
    n += shell(ints2, 5, 4.0f, out + n * DIM, 15);
    return n;
}

/* ------------------------------------------------------------------------ */
/* E8P decode.  quipsharp/codebooks/e8p.py:92-101, 174-180                   */
/* ------------------------------------------------------------------------ */

/* code = [abs_idx:8][sign bit of coord 0..6 at bits 7..1][shift:1]; the sign
 * of coord 7 is the parity of bits 7..1; shift 1 -> +1/4, 0 -> -1/4. */
static void e8p_decode_one(uint32_t code, const float *tab, float *v) {
    uint32_t a = (code >> 8) & 0xFF;
    uint32_t par = 0;
    for (int i = 0; i < 7; ++i) {
        uint32_t f = (code >> (7 - i)) & 1;
        par ^= f;
        v[i] = f ? -tab[a * DIM + i] : tab[a * DIM + i];
    }
    v[7] = par ? -tab[a * DIM + 7] : tab[a * DIM + 7];
    float sh = (code & 1) ? 0.25f : -0.25f;
    for (int i = 0; i < DIM; ++i) v[i] = v[i] + sh;
}

void qso_e8p_decode(const int64_t *codes, int64_t n, const float *tab, float *out) {
    for (int64_t k = 0; k < n; ++k) e8p_decode_one((uint32_t)(codes[k] & 0xFFFF), tab, out + k * DIM);
}

/* ------------------------------------------------------------------------ */
/* E8P encode.  quipsharp/codebooks/e8p.py:104-162, 165-171                  */
/* ------------------------------------------------------------------------ */

/* One table row against the shifted input xs (e8p.py:116-127): products,
 * strict-negative flips, parity repair at the first coordinate of least
 * |product|, then the squared distance summed left to right. */
static float row_dist(const float *xs, const float *row, int *flip_out) {
    float prod[DIM];
    int flip[DIM];
    int pc = 0;
    for (int i = 0; i < DIM; ++i) {
        prod[i] = xs[i] * row[i];
        flip[i] = prod[i] < 0.0f;
        pc += flip[i];
    }
    if (pc & 1) {
        int j = 0;
        float best = fabsf(prod[0]);
        for (int i = 1; i < DIM; ++i) {
            float a = fabsf(prod[i]);
            if (a < best) { best = a; j = i; }
        }
        flip[j] ^= 1;
    }
    float d2 = 0.0f;
    for (int i = 0; i < DIM; ++i) {
        float v = flip[i] ? -row[i] : row[i];
        float diff = xs[i] - v;
        float sq = diff * diff;
        d2 = (i == 0) ? sq : d2 + sq;
    }
    if (flip_out) memcpy(flip_out, flip, sizeof flip);
    return d2;
}

/* Encodes n 8-vectors.  codes[k] gets the packed 16-bit code, vals (if not
 * NULL) the decoded codeword.  The winner is the lexicographic minimum of
 * (d2, shift_bit, abs_idx): first-index argmin per shift (e8p.py:143-144),
 * the +1/4 search (shift bit 0) winning ties (e8p.py:156). */
void qso_e8p_encode(const float *x, int64_t n, const float *tab, int64_t *codes, float *vals) {
    for (int64_t k = 0; k < n; ++k) {
        const float *xk = x + k * DIM;
        float best_d2[2];
        int best_r[2];
        for (int sb = 0; sb < 2; ++sb) {
            float xs[DIM];
            for (int i = 0; i < DIM; ++i) xs[i] = sb == 0 ? xk[i] + 0.25f : xk[i] - 0.25f;
            best_r[sb] = 0;
            best_d2[sb] = row_dist(xs, tab, NULL);
            for (int r = 1; r < 256; ++r) {
                float d2 = row_dist(xs, tab + r * DIM, NULL);
                if (d2 < best_d2[sb]) { best_d2[sb] = d2; best_r[sb] = r; }
            }
        }
        int sb = best_d2[0] <= best_d2[1] ? 0 : 1;
        float xs[DIM];
        for (int i = 0; i < DIM; ++i) xs[i] = sb == 0 ? xk[i] + 0.25f : xk[i] - 0.25f;
        int flip[DIM];
        row_dist(xs, tab + best_r[sb] * DIM, flip);
        uint32_t sign7 = 0;
        for (int i = 0; i < 7; ++i) sign7 |= (uint32_t)flip[i] << (6 - i);
        codes[k] = ((int64_t)best_r[sb] << 8) | (int64_t)(sign7 << 1) | sb;
        if (vals) {
            for (int i = 0; i < DIM; ++i) {
                float v = flip[i] ? -tab[best_r[sb] * DIM + i] : tab[best_r[sb] * DIM + i];
                vals[k * DIM + i] = sb == 0 ? v - 0.25f : v + 0.25f;
            }
        }
    }
}

/* Squared distance of x to every one of the 65,536 decoded codewords, in
 * double precision: the brute-force optimality check of the encoder. */
void qso_e8p_bruteforce_d2(const float *x, int64_t n, const float *tab, double *best_d2_out) {
    float *all = (float *)malloc((size_t)65536 * DIM * sizeof(float));
    for (uint32_t c = 0; c < 65536; ++c) e8p_decode_one(c, tab, all + (size_t)c * DIM);
    for (int64_t k = 0; k < n; ++k) {
        double best = INFINITY;
        for (uint32_t c = 0; c < 65536; ++c) {
            double d = 0.0;
            for (int i = 0; i < DIM; ++i) {
                double t = (double)x[k * DIM + i] - all[(size_t)c * DIM + i];
                d += t * t;
            }
            if (d < best) best = d;
        }
        best_d2_out[k] = best;
    }
    free(all);
}

/* ------------------------------------------------------------------------ */
/* E8 1-bit encode.  quipsharp/codebooks/e8_1bit.py:80-83                    */
/* ------------------------------------------------------------------------ */

void qso_e81_encode(const float *x, int64_t n, const float *tab, int64_t *idx, float *vals) {
    for (int64_t k = 0; k < n; ++k) {
        const float *xk = x + k * DIM;
        int best_r = 0;
        float best = 0.0f;
        for (int r = 0; r < 256; ++r) {
            float d2 = 0.0f;
            for (int i = 0; i < DIM; ++i) {
                float diff = xk[i] - tab[r * DIM + i];
                float sq = diff * diff;
                d2 = (i == 0) ? sq : d2 + sq;
            }
            if (r == 0 || d2 < best) { best = d2; best_r = r; }
        }
        idx[k] = best_r;
        if (vals) memcpy(vals + k * DIM, tab + best_r * DIM, DIM * sizeof(float));
    }
}

/* ------------------------------------------------------------------------ */
/* Residual VQ.  quipsharp/rvq.py:69-88                                      */
/* ------------------------------------------------------------------------ */

/* kinds[s]: 0 = E8P (code in [0,65536)), 1 = E8 1-bit (code in [0,256)).
 * codes is [nstages][n].  Per stage: q = Q(residual / scale) (IEEE fp32
 * division), total += q*scale, residual -= q*scale, every op rounded. */
void qso_rvq_encode(const float *x, int64_t n, int nstages, const int *kinds, const float *scales,
                    const float *e8p_tab, const float *e81_tab, int64_t *codes, float *total_out) {
    for (int64_t k = 0; k < n; ++k) {
        float res[DIM], tot[DIM];
        memcpy(res, x + k * DIM, sizeof res);
        for (int i = 0; i < DIM; ++i) tot[i] = 0.0f;
        for (int s = 0; s < nstages; ++s) {
            float in[DIM], q[DIM];
            int64_t c;
            for (int i = 0; i < DIM; ++i) in[i] = res[i] / scales[s];
            if (kinds[s] == 0) qso_e8p_encode(in, 1, e8p_tab, &c, q);
            else qso_e81_encode(in, 1, e81_tab, &c, q);
            codes[(int64_t)s * n + k] = c;
            for (int i = 0; i < DIM; ++i) {
                float qs = q[i] * scales[s];
                tot[i] = tot[i] + qs;
                res[i] = res[i] - qs;
            }
        }
        if (total_out) memcpy(total_out + k * DIM, tot, sizeof tot);
    }
}

/* Dequantize as quipsharp/rvq.py:83-88 then quipsharp/quantize.py:107-113:
 * total = v0*s0; total = total + v1*s1; ...; out = total * layer_scale. */
void qso_rvq_decode(const int64_t *codes, int64_t n, int nstages, const int *kinds, const float *scales,
                    float layer_scale, const float *e8p_tab, const float *e81_tab, float *out) {
    for (int64_t k = 0; k < n; ++k) {
        float tot[DIM];
        for (int s = 0; s < nstages; ++s) {
            float v[DIM];
            int64_t c = codes[(int64_t)s * n + k];
            if (kinds[s] == 0) e8p_decode_one((uint32_t)(c & 0xFFFF), e8p_tab, v);
            else memcpy(v, e81_tab + (c & 0xFF) * DIM, sizeof v);
            for (int i = 0; i < DIM; ++i) {
                float vs = v[i] * scales[s];
                tot[i] = s == 0 ? vs : tot[i] + vs;
            }
        }
        for (int i = 0; i < DIM; ++i) out[k * DIM + i] = tot[i] * layer_scale;
    }
}

/* ------------------------------------------------------------------------ */
/* Walsh-Hadamard transform.  quipsharp/hadamard.py:17-40                    */
/* ------------------------------------------------------------------------ */

/* In place along the middle axis of x viewed as [outer][n][inner]: stages
 * h = 1, 2, 4, ... pair (i, i+h) inside each 2h block as (a+b, a-b), then
 * every element is multiplied by float(n ** -0.5). */
void qso_fwht(float *x, int64_t outer, int64_t n, int64_t inner) {
    float sc = (float)pow((double)n, -0.5);
    for (int64_t o = 0; o < outer; ++o) {
        for (int64_t c = 0; c < inner; ++c) {
            float *p = x + o * n * inner + c;
            for (int64_t h = 1; h < n; h *= 2)
                for (int64_t b = 0; b < n; b += 2 * h)
                    for (int64_t i = b; i < b + h; ++i) {
                        float a = p[i * inner], d = p[(i + h) * inner];
                        p[i * inner] = a + d;
                        p[(i + h) * inner] = a - d;
                    }
            for (int64_t i = 0; i < n; ++i) p[i * inner] = p[i * inner] * sc;
        }
    }
}
