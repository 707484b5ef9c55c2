/*
 * q6k_oracle.c -- CPU restatement of the Q6_K x Q8_1 arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  The oracle for the HIP Q6_K path.  Only
 * tests/, the smoke entry point and the benchmark's CPU-baseline leg may load
 * it; the product library never links, loads or calls anything in this file.
 *
 * As for Q4_K, the arithmetic lives in llama.cpp b7389 / ggml 0.9.4, which the
 * reference calls into but does not vendor.  The reference itself holds the
 * Q6_K x Q8_1 dot product (kernels/vecdotq.cuh:576-600, :867-891) and its
 * dispatch (kernels/mmvq.cu:600-605); the quantiser and block type are
 * ggml's (quantize_row_q6_K_ref, block_q6_K), restated from its published
 * algorithm.
 *
 * Pinning (tests/test_oracle_q6K.py):
 *   orc_gemv_q6K_q8_1    against a numpy decode that follows the loops of
 *                        ggml's dequantize_row_q6_K (a second, independent
 *                        statement of the byte/bit layout): exact int32 group
 *                        sums and the f64 dot, at the extremes q in {0, 63},
 *                        q8 in {-127, 127}, scales in {-128, 127}
 *   orc_dequantize_q6_K  the same numpy decode, bit for bit
 *   orc_q6K_fit_block /
 *   orc_quantize_q6_K    stage 1 against a numpy argmax over ggml's 19
 *                        candidate scales with f64 objectives (agreement away
 *                        from near-ties; planted rdelta/weight/nstep mistakes
 *                        fail); int8 scales nearest to -128 * fit / max; every
 *                        value on the nearest level; all-zero blocks;
 *                        exact-grid blocks round-trip bit for bit
 *
 *   orc_vec_dot_q6_K_q8_K_scalar / _avx2 (ggml's CPU dot, the CPU baseline
 *                        for Q6_K): against the f64 dot of the dequantised
 *                        weights and the dequantised Q8_K activation, and the
 *                        threaded product against the Q8_1 path to the
 *                        activation-quantisation error
 *                        (tests/test_oracle_cpu_baseline.py); bit-exactness
 *                        with ggml is unpinned (ggml is not available)
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <immintrin.h>

#define ORC_QK_K 256
#define ORC_Q6K_BYTES 210 /* ql[128], qh[64], scales[16] (int8), d (fp16) */
#define ORC_Q81_BYTES 36
#define ORC_Q8K_BYTES 292 /* float d + int8 qs[256] + int16 bsums[16] */
#define ORC_GROUP_MAX_EPS 1e-15f

/* from q4k_oracle.c */
uint16_t orc_f32_to_f16(float f);
float orc_f16_to_f32(uint16_t h);
int orc_nearest_int(float v);

static inline int orc_clamp(int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); }

/* make_qx_quants(n, nmax, x, L, rmse_type = 1, qw = NULL): fit of x to
 * scale * l, l in [-nmax, nmax - 1], weights x^2; the inverse scale -nmax/x_m
 * (x_m the value of largest magnitude) and 18 neighbours -(nmax + 0.1 k)/x_m,
 * k = +-1..+-9, keeping the best sum(w x l)^2 / sum(w l^2).  Writes l + nmax.
 * ggml's rdelta = 0.1, nstep = 9 and weights x^2 (weight_mode 0) are
 * arguments so that the tests can plant a wrong one (weight_mode 1: |x|). */
static float orc_make_qx_quants(int n, int nmax, const float *x, int8_t *L, float rdelta, int nstep,
                                int weight_mode) {
    float amax = 0.0f, xm = 0.0f;
    for (int i = 0; i < n; ++i) {
        const float ax = fabsf(x[i]);
        if (ax > amax) {
            amax = ax;
            xm = x[i];
        }
    }
    if (amax < ORC_GROUP_MAX_EPS) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        return 0.0f;
    }
    float iscale = (float)(-nmax) / xm;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < n; ++i) {
        const int l = orc_clamp(orc_nearest_int(iscale * x[i]), -nmax, nmax - 1);
        L[i] = (int8_t)(l + nmax);
        const float w = weight_mode == 1 ? fabsf(x[i]) : x[i] * x[i];
        sumlx += w * x[i] * l;
        suml2 += w * l * l;
    }
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int is = -nstep; is <= nstep; ++is) {
        if (is == 0) continue;
        iscale = -(nmax + rdelta * is) / xm;
        sumlx = suml2 = 0.0f;
        for (int i = 0; i < n; ++i) {
            const int l = orc_clamp(orc_nearest_int(iscale * x[i]), -nmax, nmax - 1);
            const float w = weight_mode == 1 ? fabsf(x[i]) : x[i] * x[i];
            sumlx += w * x[i] * l;
            suml2 += w * l * l;
        }
        if (suml2 > 0.0f && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < n; ++i)
                L[i] = (int8_t)(nmax + orc_clamp(orc_nearest_int(iscale * x[i]), -nmax, nmax - 1));
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

/* Stage 1 of quantize_row_q6_K_ref for one 256-value block: the
 * make_qx_quants fit (nmax 32) of each 16-value group, giving its scale and
 * levels L (l + 32).  ggml's parameters: rdelta 0.1, nstep 9, weight_mode 0. */
void orc_q6K_fit_block(const float *x, float rdelta, int nstep, int weight_mode, float scales[16],
                       int8_t L[256]) {
    for (int ib = 0; ib < 16; ++ib)
        scales[ib] = orc_make_qx_quants(16, 32, x + 16 * ib, L + 16 * ib, rdelta, nstep, weight_mode);
}

/* quantize_row_q6_K_ref: k floats (k % 256 == 0) -> k/256 blocks of 210 B. */
void orc_quantize_q6_K(const float *x, uint8_t *y, int64_t k) {
    const int64_t nb = k / ORC_QK_K;
    int8_t L[ORC_QK_K];
    float scales[16];
    for (int64_t i = 0; i < nb; ++i, x += ORC_QK_K, y += ORC_Q6K_BYTES) {
        float max_scale = 0.0f, max_abs = 0.0f;
        orc_q6K_fit_block(x, 0.1f, 9, 0, scales, L);
        for (int ib = 0; ib < 16; ++ib) {
            const float s = scales[ib];
            if (fabsf(s) > max_abs) {
                max_abs = fabsf(s);
                max_scale = s;
            }
        }
        if (max_abs < ORC_GROUP_MAX_EPS) {
            memset(y, 0, ORC_Q6K_BYTES);
            continue;
        }
        const float iscale = -128.0f / max_scale;
        const uint16_t dh = orc_f32_to_f16(1.0f / iscale);
        int8_t *sc = (int8_t *)(y + 192);
        for (int ib = 0; ib < 16; ++ib) {
            const int v = orc_nearest_int(iscale * scales[ib]);
            sc[ib] = (int8_t)(v < 127 ? v : 127);
        }
        for (int j = 0; j < 16; ++j) {
            const float d = orc_f16_to_f32(dh) * sc[j];
            if (!d) continue;
            for (int ii = 0; ii < 16; ++ii)
                L[16 * j + ii] = (int8_t)(orc_clamp(orc_nearest_int(x[16 * j + ii] / d), -32, 31) + 32);
        }
        uint8_t *ql = y, *qh = y + 128;
        for (int j = 0; j < ORC_QK_K; j += 128, ql += 64, qh += 32) {
            for (int l = 0; l < 32; ++l) {
                const uint8_t q1 = (uint8_t)(L[j + l] & 0xf), q2 = (uint8_t)(L[j + l + 32] & 0xf);
                const uint8_t q3 = (uint8_t)(L[j + l + 64] & 0xf), q4 = (uint8_t)(L[j + l + 96] & 0xf);
                ql[l] = (uint8_t)(q1 | (q3 << 4));
                ql[l + 32] = (uint8_t)(q2 | (q4 << 4));
                qh[l] = (uint8_t)((L[j + l] >> 4) | ((L[j + l + 32] >> 4) << 2) | ((L[j + l + 64] >> 4) << 4) |
                                  ((L[j + l + 96] >> 4) << 6));
            }
        }
        y[208] = (uint8_t)(dh & 0xff);
        y[209] = (uint8_t)(dh >> 8);
    }
}

/* dequantize_row_q6_K: w = d * scales[e/16] * (q - 32). */
void orc_dequantize_q6_K(const uint8_t *y, float *x, int64_t k) {
    const int64_t nb = k / ORC_QK_K;
    for (int64_t i = 0; i < nb; ++i, y += ORC_Q6K_BYTES, x += ORC_QK_K) {
        const float d = orc_f16_to_f32((uint16_t)(y[208] | (y[209] << 8)));
        const uint8_t *ql = y, *qh = y + 128;
        const int8_t *sc = (const int8_t *)(y + 192);
        float *o = x;
        for (int h = 0; h < 2; ++h, ql += 64, qh += 32, sc += 8, o += 128) {
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int q1 = ((ql[l] & 0xf) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = ((ql[l + 32] & 0xf) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = ((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = ((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                o[l] = d * sc[is] * q1;
                o[l + 32] = d * sc[is + 2] * q2;
                o[l + 64] = d * sc[is + 4] * q3;
                o[l + 96] = d * sc[is + 6] * q4;
            }
        }
    }
}

static inline int32_t orc_ld_i32_le(const uint8_t *p) {
    int32_t v;
    memcpy(&v, p, 4);
    return v;
}

/* sum over the four signed bytes of a*b */
static inline int32_t orc_dp4a6(int32_t a, int32_t b, int32_t c) {
    for (int i = 0; i < 4; ++i) c += (int32_t)(int8_t)(a >> (8 * i)) * (int32_t)(int8_t)(b >> (8 * i));
    return c;
}

/* per-byte a - b with signed saturation (__vsubss4) */
static inline int32_t orc_vsubss4(int32_t a, int32_t b) {
    uint32_t r = 0;
    for (int i = 0; i < 4; ++i) {
        int v = (int)(int8_t)(a >> (8 * i)) - (int)(int8_t)(b >> (8 * i));
        v = v < -128 ? -128 : (v > 127 ? 127 : v);
        r |= (uint32_t)(uint8_t)(int8_t)v << (8 * i);
    }
    return (int32_t)r;
}

/*
 * y[c*ld + r] for r < M, c < N, following kernels/vecdotq.cuh:867-891 and
 * :580-600 for every (block kb, iqs = 0..31) -- QI6_K = 32, QR6_K = 2,
 * QI8_1 = 8 -- and kernels/mmvq.cu:236-256 for the accumulation over the
 * blocks of a row.
 *   w:   M rows of K/256 blocks, row stride row_stride bytes
 *   q8:  N columns of Q8_1 blocks, column stride stride_col_y blocks
 * Outputs (each optional):
 *   y64[c*M + r]              the result in double precision
 *   l1[c*M + r]               sum of |d * d8 * sc * S_g| over the groups (error scale)
 *   s16[(c*M + r)*(K/16) + g] int32 sum over 16-weight group g of (q - 32) * q8
 * Returns the number of (iqs, i) pairs whose scale index differs from the
 * 16-weight group their q8 values belong to (0: the two index formulas of
 * the reference agree).
 */
static int64_t orc_gemv_q6K_rows(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride, const uint8_t *q8,
                                 int64_t N, int64_t stride_col_y, int64_t r0, int64_t r1, double *y64, double *l1,
                                 int32_t *s16) {
    const int64_t nb = K / ORC_QK_K, ng = K / 16;
    int64_t mismatches = 0;
    for (int64_t c = 0; c < N; ++c) {
        const uint8_t *yc = q8 + c * stride_col_y * ORC_Q81_BYTES;
        for (int64_t r = r0; r < r1; ++r) {
            const uint8_t *wr = w + r * row_stride;
            double acc = 0.0, acc_l1 = 0.0;
            for (int64_t kb = 0; kb < nb; ++kb) {
                const uint8_t *blk = wr + kb * ORC_Q6K_BYTES;
                const uint8_t *ql = blk, *qh = blk + 128;
                const int8_t *scales = (const int8_t *)(blk + 192);
                const double d = orc_f16_to_f32((uint16_t)(blk[208] | (blk[209] << 8)));
                int32_t sg[16] = {0};
                int sc_of[16];
                for (int g = 0; g < 16; ++g) sc_of[g] = scales[g];
                for (int iqs = 0; iqs < 32; ++iqs) {
                    const int bq8_offset = 2 * 2 * (iqs / 16) + (iqs % 16) / 8;
                    const int scale_offset = 8 * (iqs / 16) + (iqs % 16) / 4;
                    const int vh_shift = 2 * ((iqs % 16) / 8);
                    const int32_t vl = orc_ld_i32_le(ql + 4 * iqs);
                    const int32_t vh = (int32_t)((uint32_t)orc_ld_i32_le(qh + 4 * (8 * (iqs / 16) + iqs % 8)) >> vh_shift);
                    for (int i = 0; i < 2; ++i) {
                        const int sidx = scale_offset + 4 * i;
                        const int32_t vil = (vl >> (4 * i)) & 0x0f0f0f0f;
                        const int32_t vih = ((vh >> (4 * i)) << 4) & 0x30303030;
                        const int32_t vi = orc_vsubss4(vil | vih, 0x20202020);
                        const int b8 = bq8_offset + 2 * i;
                        const int32_t u = orc_ld_i32_le(yc + (kb * 8 + b8) * ORC_Q81_BYTES + 4 + 4 * (iqs % 8));
                        const int g = 2 * b8 + (iqs % 8) / 4;  /* 16-weight group of these q8 */
                        if (g != sidx) ++mismatches;
                        sg[g] += orc_dp4a6(vi, u, 0);
                    }
                }
                for (int g = 0; g < 16; ++g) {
                    const uint8_t *b8 = yc + (kb * 8 + g / 2) * ORC_Q81_BYTES;
                    const double d8 = orc_f16_to_f32((uint16_t)(b8[0] | (b8[1] << 8)));
                    const double t = d * d8 * (double)sc_of[g] * (double)sg[g];
                    acc += t;
                    acc_l1 += fabs(t);
                    if (s16) s16[(c * M + r) * ng + kb * 16 + g] = sg[g];
                }
            }
            if (y64) y64[c * M + r] = acc;
            if (l1) l1[c * M + r] = acc_l1;
        }
    }
    return mismatches;
}

int64_t orc_gemv_q6K_q8_1(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride, const uint8_t *q8,
                          int64_t N, int64_t stride_col_y, double *y64, double *l1, int32_t *s16) {
    return orc_gemv_q6K_rows(w, M, K, row_stride, q8, N, stride_col_y, 0, M, y64, l1, s16);
}

/* The same with the rows split over nthreads threads (contiguous ranges);
 * returns the summed mismatch count. */
typedef struct {
    const uint8_t *w, *q8;
    int64_t M, K, row_stride, N, stride_col_y, r0, r1;
    double *y64, *l1;
    int32_t *s16;
    int64_t mismatches;
} orc_q6_task;

static void *orc_gemv_q6K_task(void *arg) {
    orc_q6_task *t = (orc_q6_task *)arg;
    t->mismatches = orc_gemv_q6K_rows(t->w, t->M, t->K, t->row_stride, t->q8, t->N, t->stride_col_y, t->r0,
                                      t->r1, t->y64, t->l1, t->s16);
    return NULL;
}

int64_t orc_gemv_q6K_q8_1_mt(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride, const uint8_t *q8,
                             int64_t N, int64_t stride_col_y, double *y64, double *l1, int32_t *s16,
                             int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > M) nthreads = M > 0 ? (int)M : 1;
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    orc_q6_task *task = (orc_q6_task *)malloc(sizeof(orc_q6_task) * (size_t)nthreads);
    for (int i = 0; i < nthreads; ++i) {
        orc_q6_task t = {w, q8, M, K, row_stride, N, stride_col_y, M * i / nthreads, M * (i + 1) / nthreads,
                         y64, l1, s16, 0};
        task[i] = t;
        if (i > 0) pthread_create(&th[i], NULL, orc_gemv_q6K_task, &task[i]);
    }
    orc_gemv_q6K_task(&task[0]);
    int64_t mism = task[0].mismatches;
    for (int i = 1; i < nthreads; ++i) {
        pthread_join(th[i], NULL);
        mism += task[i].mismatches;
    }
    free(th);
    free(task);
    return mism;
}

/* ------------------------------------------------------------------------ */
/* ggml's CPU dot for Q6_K (the CPU baseline of the Q6_K configs)           */
/* ------------------------------------------------------------------------ */

/* The 256 weights of a block as q - 32 in [-32, 31], in weight order (the
 * layout dequantize_row_q6_K reads: half h, l in [0, 32): weights 128h + l,
 * +32, +64, +96 from ql[64h + l] low, ql[64h + 32 + l] low, ql[64h + l] high,
 * ql[64h + 32 + l] high and qh[32h + l] bits 0-1, 2-3, 4-5, 6-7). */
static void orc_q6_values(const uint8_t *x, int8_t a[ORC_QK_K]) {
    const uint8_t *ql = x, *qh = x + 128;
    for (int h = 0; h < 2; ++h) {
        for (int l = 0; l < 32; ++l) {
            const int lo0 = ql[64 * h + l], lo1 = ql[64 * h + 32 + l], hb = qh[32 * h + l];
            a[128 * h + l] = (int8_t)(((lo0 & 0x0f) | ((hb & 3) << 4)) - 32);
            a[128 * h + 32 + l] = (int8_t)(((lo1 & 0x0f) | (((hb >> 2) & 3) << 4)) - 32);
            a[128 * h + 64 + l] = (int8_t)(((lo0 >> 4) | (((hb >> 4) & 3) << 4)) - 32);
            a[128 * h + 96 + l] = (int8_t)(((lo1 >> 4) | (((hb >> 6) & 3) << 4)) - 32);
        }
    }
}

/* ggml_vec_dot_q6_K_q8_K, portable form: per block, eight int32 lanes (lane l
 * takes elements 8t + l of every 8-element slice) accumulate scale * q8 * w
 * over the 16 scale groups; each block's lanes are scaled by d_w * d_y and
 * summed per lane in float, the lanes added at the end. */
float orc_vec_dot_q6_K_q8_K_scalar(int64_t n, const uint8_t *x, const uint8_t *y) {
    const int64_t nb = n / ORC_QK_K;
    float sums[8] = {0};
    for (int64_t i = 0; i < nb; ++i, x += ORC_Q6K_BYTES, y += ORC_Q8K_BYTES) {
        float dy;
        memcpy(&dy, y, 4);
        const int8_t *q8 = (const int8_t *)(y + 4);
        const int8_t *sc = (const int8_t *)(x + 192);
        int8_t a[ORC_QK_K];
        orc_q6_values(x, a);
        int32_t lanes[8] = {0};
        for (int g = 0; g < 16; ++g)
            for (int t = 0; t < 2; ++t)
                for (int l = 0; l < 8; ++l) {
                    const int e = 16 * g + 8 * t + l;
                    lanes[l] += sc[g] * ((int32_t)q8[e] * (int32_t)a[e]);
                }
        const float d = orc_f16_to_f32((uint16_t)(x[208] | (x[209] << 8))) * dy;
        for (int l = 0; l < 8; ++l) sums[l] += d * lanes[l];
    }
    float sumf = 0;
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* The AVX2 form (ggml-cpu's x86 path): per half block the four 32-weight runs
 * are assembled as unsigned 6-bit values, multiplied with the q8 as u8*s8 pair
 * products (maddubs), corrected by 32 * (pair sums of q8) and scaled by the
 * 16-bit scales of their two scale groups (madd) into eight int32 lanes; the
 * lanes are scaled per block by d_w * d_y in a float vector, reduced at the
 * end. */
__attribute__((target("avx2,fma,f16c")))
float orc_vec_dot_q6_K_q8_K_avx2(int64_t n, const uint8_t *x, const uint8_t *y) {
    const int64_t nb = n / ORC_QK_K;
    const __m256i m4 = _mm256_set1_epi8(0x0f), m3 = _mm256_set1_epi8(3), k32 = _mm256_set1_epi8(32);
    __m256 acc = _mm256_setzero_ps();
    for (int64_t i = 0; i < nb; ++i, x += ORC_Q6K_BYTES, y += ORC_Q8K_BYTES) {
        float dy;
        memcpy(&dy, y, 4);
        const float d = dy * _cvtsh_ss((unsigned short)(x[208] | (x[209] << 8)));
        const int8_t *sc = (const int8_t *)(x + 192);
        const int8_t *q8 = (const int8_t *)(y + 4);
        __m256i sumi = _mm256_setzero_si256();
        for (int h = 0; h < 2; ++h) {
            const __m256i lo0 = _mm256_loadu_si256((const __m256i *)(x + 64 * h));
            const __m256i lo1 = _mm256_loadu_si256((const __m256i *)(x + 64 * h + 32));
            const __m256i hb = _mm256_loadu_si256((const __m256i *)(x + 128 + 32 * h));
            __m256i w[4];
            w[0] = _mm256_or_si256(_mm256_and_si256(lo0, m4), _mm256_slli_epi16(_mm256_and_si256(hb, m3), 4));
            w[1] = _mm256_or_si256(_mm256_and_si256(lo1, m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 2), m3), 4));
            w[2] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(lo0, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 4), m3), 4));
            w[3] = _mm256_or_si256(_mm256_and_si256(_mm256_srli_epi16(lo1, 4), m4),
                                   _mm256_slli_epi16(_mm256_and_si256(_mm256_srli_epi16(hb, 6), m3), 4));
            for (int r = 0; r < 4; ++r) {
                const __m256i yv = _mm256_loadu_si256((const __m256i *)(q8 + 128 * h + 32 * r));
                const __m256i p = _mm256_sub_epi16(_mm256_maddubs_epi16(w[r], yv), _mm256_maddubs_epi16(k32, yv));
                /* scale groups 8h + 2r (pairs 0..7) and 8h + 2r + 1 (pairs 8..15) */
                const __m256i s16 = _mm256_setr_m128i(_mm_set1_epi16(sc[8 * h + 2 * r]),
                                                      _mm_set1_epi16(sc[8 * h + 2 * r + 1]));
                sumi = _mm256_add_epi32(sumi, _mm256_madd_epi16(s16, p));
            }
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    __m128 h4 = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    h4 = _mm_add_ps(h4, _mm_movehl_ps(h4, h4));
    h4 = _mm_add_ss(h4, _mm_movehdup_ps(h4));
    return _mm_cvtss_f32(h4);
}
