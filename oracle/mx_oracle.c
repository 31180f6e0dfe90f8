/*
 * CPU oracle: a plain-C restatement of the reference quantized matmul `mx_gemm`
 * (app/native/src/mx_gemm.c:123-194). TEST INFRASTRUCTURE ONLY: tests, the smoke check and the
 * CPU-baseline leg of bench.py load it as a checker; the product never links it.
 *
 * Semantics restated (file:line into the reference):
 *   - Q8_K activation quantization per 256 values (mx_common.c:42-69): amax, iscale = 127/amax,
 *     q = clamp(lrintf(x*iscale), +-127), bsums over 16, d = amax/127; an all-zero block is zero.
 *   - Q4_K block dot (mx_dot_k_ssse3.c:109-157): sumi = sum_s sc_s * sum(u*q8) over sub-blocks of
 *     32, summ = sum over the 16 bsums of min_{s/2} * bsum; sumf += y.d * (d*sumi - dmin*summ).
 *   - Q6_K block dot (mx_dot_k_ssse3.c:167-209): sumi = sum_s sc_s * sum((u-32)*q8) over
 *     sub-blocks of 16; sumf += y.d * d * sumi.
 *   - Q8_0 (mx_dot_q8_0.c:5-22): per 256 values, block_sum += d_k * sum(qs*q8) over the eight
 *     32-value blocks; sumf += y.d * block_sum.
 *   - IQ4_XS on raw fp32 activations, no Q8_K (mx_dot_f32.c:32-58):
 *     acc += x[j]*(dl*K[lo]) + x[j+16]*(dl*K[hi]) sequentially.
 *   - every output row is the sequential fold over blocks 0..nb-1 (mx_gemm.c:158-167).
 *
 * The fp32 fold points are written with explicit fmaf() where an FMA-contracting compiler fuses
 * the reference expression (x86-64 gcc with FMA, the reference's -march=native default), and
 * the file is compiled with -ffp-contract=off, so these results do not depend on the host:
 *     Q4_K: T = fmaf(d, sumi, -(dmin*summ)); acc = fmaf(y.d, T, acc)
 *     Q6_K: acc = fmaf(y.d*d, sumi, acc)
 *     Q8_0: block_sum = fmaf(d_k, acc_k, block_sum); acc = fmaf(y.d, block_sum, acc)
 *     IQ4_XS: acc += fmaf(x[j], dl*K[lo], x[j+16]*(dl*K[hi]))  (the reference's sequential chain)
 * With these, the results equal the reference C built with gcc's default contraction bit for bit
 * (checked in tests/test_oracle_vs_reference.py). The integer sums are exact, so the K-quant and
 * Q8_0 order is also what the GPU kernels reproduce bit for bit; IQ4_XS's long sequential fp32
 * chain cannot be parallelised bit-exactly, so GPU results for it are compared within tolerance.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QK 256
#define T_Q8_0 8
#define T_Q4_K 12
#define T_Q6_K 14
#define T_IQ4_XS 23

static const float GRID_IQ4[16] = {-127.f, -104.f, -83.f, -65.f, -49.f, -35.f, -22.f, -10.f,
                                   1.f,    13.f,   25.f,  38.f,  53.f,  69.f,  89.f,  113.f};

/* IEEE half at p (little endian) widened exactly: subnormals are mant * 2^-24. */
static float half_at(const uint8_t *p) {
    const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
    const uint32_t sign = (h >> 15) & 1u, exp = (h >> 10) & 0x1Fu, mant = h & 0x3FFu;
    float v;
    if (exp == 0) {
        v = ldexpf((float)mant, -24);
    } else if (exp == 31) {
        uint32_t bits = 0x7F800000u | (mant << 13);
        memcpy(&v, &bits, 4);
    } else {
        uint32_t bits = ((exp + 112u) << 23) | (mant << 13);
        memcpy(&v, &bits, 4);
    }
    return sign ? -v : v;
}

/* Q4_K scale/min pair j of the 12 packed bytes (app/gguf/dequant/kquants.py:10-23). */
static void k4_pair(const uint8_t *s, int j, int *sc, int *mn) {
    if (j < 4) {
        *sc = s[j] & 63;
        *mn = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

/* Unsigned 6-bit code u = q + 32 of Q6_K element e (kquants.py:138-159). */
static int q6_code(const uint8_t *blk, int e) {
    const int h = e / 128, g = (e % 128) / 32, l = e % 32;
    const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
    const int low = (g & 1) ? ql[32 + l] : ql[l];
    const int nib = (g & 2) ? (low >> 4) : (low & 15);
    return nib | (((qh[l] >> (2 * g)) & 3) << 4);
}

void mxo_quantize_q8_k(const float *x, int8_t *q, float *d, int16_t *bsums, int n_rows, int k) {
    const int nb = k / QK;
    for (int r = 0; r < n_rows; ++r) {
        for (int b = 0; b < nb; ++b) {
            const float *xb = x + (size_t)r * k + (size_t)b * QK;
            int8_t *qb = q + (size_t)r * k + (size_t)b * QK;
            int16_t *sb = bsums + ((size_t)r * nb + b) * 16;
            float amax = 0.0f;
            for (int j = 0; j < QK; ++j) {
                const float a = fabsf(xb[j]);
                if (a > amax) amax = a;
            }
            if (amax == 0.0f) {
                memset(qb, 0, QK);
                memset(sb, 0, 16 * sizeof(int16_t));
                d[(size_t)r * nb + b] = 0.0f;
                continue;
            }
            const float iscale = 127.0f / amax;
            for (int j = 0; j < QK; ++j) {
                long v = lrintf(xb[j] * iscale);
                qb[j] = (int8_t)(v > 127 ? 127 : (v < -127 ? -127 : v));
            }
            for (int s = 0; s < 16; ++s) {
                int sum = 0;
                for (int l = 0; l < 16; ++l) sum += qb[16 * s + l];
                sb[s] = (int16_t)sum;
            }
            d[(size_t)r * nb + b] = amax / 127.0f;
        }
    }
}

typedef struct {
    const int8_t *q;      /* K values */
    const float *d;       /* nb scales */
    const int16_t *bsums; /* nb * 16 */
} act_row;

static float dot_q4_k(const uint8_t *row, act_row a, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = row + (size_t)b * 144;
        const uint8_t *qs = blk + 16;
        const int8_t *q8 = a.q + (size_t)b * QK;
        int sc[8], mn[8];
        for (int j = 0; j < 8; ++j) k4_pair(blk + 4, j, &sc[j], &mn[j]);
        int32_t sumi = 0, summ = 0;
        for (int c = 0; c < 4; ++c) {
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; ++l) {
                lo += (qs[32 * c + l] & 15) * q8[64 * c + l];
                hi += (qs[32 * c + l] >> 4) * q8[64 * c + 32 + l];
            }
            sumi += sc[2 * c] * lo + sc[2 * c + 1] * hi;
        }
        for (int s = 0; s < 16; ++s) summ += mn[s / 2] * a.bsums[b * 16 + s];
        const float t = half_at(blk + 2) * (float)summ;
        const float blockv = fmaf(half_at(blk), (float)sumi, -t);
        acc = fmaf(a.d[b], blockv, acc);
    }
    return acc;
}

static float dot_q6_k(const uint8_t *row, act_row a, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = row + (size_t)b * 210;
        const int8_t *sc = (const int8_t *)(blk + 192);
        const int8_t *q8 = a.q + (size_t)b * QK;
        int32_t sumi = 0;
        for (int s = 0; s < 16; ++s) {
            int32_t p = 0;
            for (int l = 0; l < 16; ++l) p += (q6_code(blk, 16 * s + l) - 32) * q8[16 * s + l];
            sumi += sc[s] * p;
        }
        acc = fmaf(a.d[b] * half_at(blk + 208), (float)sumi, acc);
    }
    return acc;
}

static float dot_q8_0(const uint8_t *row, act_row a, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; ++b) {
        float block_sum = 0.0f;
        for (int k = 0; k < 8; ++k) {
            const uint8_t *blk = row + (size_t)(b * 8 + k) * 34;
            const int8_t *qs = (const int8_t *)(blk + 2);
            const int8_t *q8 = a.q + (size_t)b * QK + 32 * k;
            int32_t p = 0;
            for (int l = 0; l < 32; ++l) p += qs[l] * q8[l];
            block_sum = fmaf(half_at(blk), (float)p, block_sum);
        }
        acc = fmaf(a.d[b], block_sum, acc);
    }
    return acc;
}

static float dot_iq4_xs(const uint8_t *row, const float *x, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; ++b) {
        const uint8_t *blk = row + (size_t)b * 136;
        const float d = half_at(blk);
        const int sh = blk[2] | (blk[3] << 8);
        for (int ib = 0; ib < 8; ++ib) {
            const int ls = ((blk[4 + ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
            const float dl = d * (float)(ls - 32);
            const uint8_t *q = blk + 8 + 16 * ib;
            const float *xo = x + (size_t)b * QK + 32 * ib;
            for (int j = 0; j < 16; ++j) {
                const float wl = dl * GRID_IQ4[q[j] & 15];
                const float wh = dl * GRID_IQ4[q[j] >> 4];
                acc += fmaf(xo[j], wl, xo[16 + j] * wh);
            }
        }
    }
    return acc;
}

static size_t row_bytes(int type, int k) {
    switch (type) {
    case T_Q8_0: return (size_t)(k / 32) * 34;
    case T_Q4_K: return (size_t)(k / QK) * 144;
    case T_Q6_K: return (size_t)(k / QK) * 210;
    case T_IQ4_XS: return (size_t)(k / QK) * 136;
    default: return 0;
    }
}

int mxo_supports(int type, int k) {
    return row_bytes(type, k) != 0 && k > 0 && k % QK == 0;
}

/* y (n_tokens, out) = x (n_tokens, in) @ W.T; 0 ok, -1 unsupported, -2 out of memory. */
int mxo_gemm(int type, const uint8_t *w, const float *x, float *y, int n_tokens, int out_f,
             int in_f, int n_threads) {
    if (!mxo_supports(type, in_f)) return -1;
    const size_t rb = row_bytes(type, in_f);
    const int nb = in_f / QK;
    if (type == T_IQ4_XS) {
#pragma omp parallel for schedule(static) num_threads(n_threads)
        for (int o = 0; o < out_f; ++o)
            for (int t = 0; t < n_tokens; ++t)
                y[(size_t)t * out_f + o] = dot_iq4_xs(w + (size_t)o * rb, x + (size_t)t * in_f, nb);
        return 0;
    }
    int8_t *q = malloc((size_t)n_tokens * in_f);
    float *d = malloc((size_t)n_tokens * nb * sizeof(float));
    int16_t *bs = malloc((size_t)n_tokens * nb * 16 * sizeof(int16_t));
    if (!q || !d || !bs) {
        free(q), free(d), free(bs);
        return -2;
    }
    mxo_quantize_q8_k(x, q, d, bs, n_tokens, in_f);
#pragma omp parallel for schedule(static) num_threads(n_threads)
    for (int o = 0; o < out_f; ++o) {
        const uint8_t *row = w + (size_t)o * rb;
        for (int t = 0; t < n_tokens; ++t) {
            act_row a = {q + (size_t)t * in_f, d + (size_t)t * nb, bs + (size_t)t * nb * 16};
            float v = type == T_Q4_K ? dot_q4_k(row, a, nb)
                      : type == T_Q6_K ? dot_q6_k(row, a, nb)
                                       : dot_q8_0(row, a, nb);
            y[(size_t)t * out_f + o] = v;
        }
    }
    free(q), free(d), free(bs);
    return 0;
}

/* Flat fp32 values of n_blocks packed blocks, in the numpy restatement's rounding order. */
int mxo_dequantize(int type, const uint8_t *blocks, long n_blocks, float *out) {
    for (long i = 0; i < n_blocks; ++i) {
        switch (type) {
        case T_Q8_0: {
            const uint8_t *b = blocks + i * 34;
            const float d = half_at(b);
            for (int l = 0; l < 32; ++l) out[i * 32 + l] = (float)(int8_t)b[2 + l] * d;
            break;
        }
        case T_Q4_K: {
            const uint8_t *b = blocks + i * 144;
            const float d = half_at(b), dmin = half_at(b + 2);
            for (int c = 0; c < 4; ++c)
                for (int h = 0; h < 2; ++h) {
                    int sc, mn;
                    k4_pair(b + 4, 2 * c + h, &sc, &mn);
                    const float ds = d * (float)sc, dm = dmin * (float)mn;
                    for (int l = 0; l < 32; ++l) {
                        const int u = h ? (b[16 + 32 * c + l] >> 4) : (b[16 + 32 * c + l] & 15);
                        out[i * QK + 64 * c + 32 * h + l] = ds * (float)u - dm;
                    }
                }
            break;
        }
        case T_Q6_K: {
            const uint8_t *b = blocks + i * 210;
            const float d = half_at(b + 208);
            for (int e = 0; e < QK; ++e) {
                const float ds = d * (float)(int8_t)b[192 + e / 16];
                out[i * QK + e] = ds * ((float)q6_code(b, e) - 32.0f);
            }
            break;
        }
        case T_IQ4_XS: {
            const uint8_t *b = blocks + i * 136;
            const float d = half_at(b);
            const int sh = b[2] | (b[3] << 8);
            for (int ib = 0; ib < 8; ++ib) {
                const int ls =
                    ((b[4 + ib / 2] >> (4 * (ib % 2))) & 15) | (((sh >> (2 * ib)) & 3) << 4);
                const float dl = d * (float)(ls - 32);
                for (int j = 0; j < 16; ++j) {
                    out[i * QK + 32 * ib + j] = dl * GRID_IQ4[b[8 + 16 * ib + j] & 15];
                    out[i * QK + 32 * ib + 16 + j] = dl * GRID_IQ4[b[8 + 16 * ib + j] >> 4];
                }
            }
            break;
        }
        default: return -1;
        }
    }
    return 0;
}
