/*
 * q4k_oracle.c -- CPU restatement of the Q4_K x Q8 arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the oracle the tests compare the HIP
 * product path against, and the CPU baseline that the benchmark times beside it.  Only tests/, the smoke
 * entry point and the benchmark's CPU-baseline leg may load it; the product
 * library never links, loads or calls anything in this file.
 *
 * The arithmetic lives in llama.cpp b7389 / ggml 0.9.4, which the reference
 * calls into but does not vendor (version pinned by the reference's capture
 * metadata, profiling/upstream_run.sqlite).  Each function names the reference
 * file:line it follows, or the upstream function it restates from ggml's
 * published algorithm.
 *
 * Pinning (see tests/test_oracle_*.py):
 *   orc_f16_*                 exhaustive against numpy float16
 *   orc_nearest_int           against numpy.rint over the valid range
 *   orc_scale_min_k4 /
 *   orc_vecdot_scale_pair     exhaustive agreement of two independent unpackers
 *                             + pack/unpack identity over all 64x64 (sc, m)
 *   orc_quantize_q8_1         invariants (|q|<=127, amax -> +-127, zero blocks,
 *                             |x-d*q| <= d/2, exact multiples round-trip) and
 *                             exact ties rounding away from zero (roundf)
 *   orc_gemv_q4K_q8_1         brute force: naive dequantised f64 dot (numpy) and
 *                             nibble-by-position integer sums (numpy)
 *   orc_q4K_fit_block /
 *   orc_quantize_q4_K         stage 1 against a numpy walk over ggml's candidate
 *                             scales with f64 fits (agreement away from near-ties;
 *                             planted rdelta/rmin/weight/nstep mistakes fail);
 *                             stages 2-3 nearest-field and nearest-level
 *                             properties; exact-grid blocks round-trip bit for bit
 *   orc_quantize_q8_K         signed-max rule (x_max -> -127, first on ties),
 *                             bsums, error bound
 *   orc_vec_dot_q4_K_q8_K_*   scalar vs AVX2 agreement, error bound against the
 *                             f64 dequantised product; the f32 summation order
 *                             of ggml's own AVX2 code: parity unpinned
 *
 * Build: oracle/Makefile (gcc, -ffp-contract=off so float expressions are
 * evaluated exactly as written).
 */
#define _GNU_SOURCE
#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>
#include <immintrin.h>

#define ORC_QK_K 256
#define ORC_QK8_1 32
#define ORC_Q4K_BYTES 144 /* kernels/2pack.cu:6 */
#define ORC_Q81_BYTES 36  /* kernels/2pack.cu:7 */
#define ORC_Q8K_BYTES 292 /* float d + int8 qs[256] + int16 bsums[16] */

/* ------------------------------------------------------------------------ */
/* fp16 <-> fp32 (IEEE binary16, round-to-nearest-even)                      */
/* ------------------------------------------------------------------------ */

uint16_t orc_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) { /* NaN: keep it quiet, keep top payload bits */
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) { /* >= 65520 (and inf) rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x38800000u) { /* normal half range: |f| >= 2^-14 */
        const uint32_t exp_h = (ax >> 23) - 112u;
        const uint32_t mant = ax & 0x7fffffu;
        uint32_t h = (exp_h << 10) | (mant >> 13);
        const uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) { /* < 2^-25: rounds to zero (2^-25 itself ties to even 0) */
        return (uint16_t)sign;
    }
    /* subnormal half: value = m * 2^(e-150), unit 2^-24 -> shift by 126-e */
    const uint32_t e = ax >> 23;
    const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    const uint32_t shift = 126u - e;
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1u);
    const uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t m = h & 0x3ffu;
    uint32_t x;
    float f;
    if (e == 0) {
        f = (float)m * 5.9604644775390625e-08f; /* m * 2^-24, exact */
        memcpy(&x, &f, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7f800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    memcpy(&f, &x, 4);
    return f;
}

void orc_f32_to_f16_array(const float *x, uint16_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f32_to_f16(x[i]);
}

void orc_f16_to_f32_array(const uint16_t *x, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_f16_to_f32(x[i]);
}

/* ggml-quants.c nearest_int: round-half-to-even through the 1.5*2^23 bias,
 * valid for |v| <= 2^22 - 1. */
int orc_nearest_int(float v) {
    const float t = v + 12582912.0f;
    int32_t i;
    memcpy(&i, &t, 4);
    return (i & 0x007fffff) - 0x00400000;
}

void orc_nearest_int_array(const float *x, int32_t *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_nearest_int(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Q4_K 6-bit scale / min fields                                            */
/* ------------------------------------------------------------------------ */

/* ggml-quants.c get_scale_min_k4: sub-block s in 0..7 of the 12 scale bytes.
 * s < 4 : sc = b[s] & 63,               m = b[s+4] & 63
 * s >= 4: sc = lo4(b[s+4]) | hi2(b[s-4]), m = hi4(b[s+4]) | hi2(b[s]) */
void orc_scale_min_k4(int s, const uint8_t *b, uint8_t *sc, uint8_t *m) {
    if (s < 4) {
        *sc = b[s] & 63;
        *m = b[s + 4] & 63;
    } else {
        *sc = (uint8_t)((b[s + 4] & 0x0f) | ((b[s - 4] >> 6) << 4));
        *m = (uint8_t)((b[s + 4] >> 4) | ((b[s] >> 6) << 4));
    }
}

/* kernels/vecdotq.cuh:796-807: the GPU vec-dot reads the scale bytes as
 * little-endian uint16 pairs and unpacks the (sc, m) of sub-blocks 2j and
 * 2j+1 at once.  out = {sc[2j], sc[2j+1], m[2j], m[2j+1]}. */
void orc_vecdot_scale_pair(int j, const uint8_t *b, uint8_t out[4]) {
    uint16_t w[6];
    for (int i = 0; i < 6; ++i) w[i] = (uint16_t)(b[2 * i] | (b[2 * i + 1] << 8));
    uint16_t scp, mp;
    if (j < 2) {
        scp = w[j] & 0x3f3f;
        mp = w[j + 2] & 0x3f3f;
    } else {
        scp = (uint16_t)((w[j + 2] & 0x0f0f) | ((w[j - 2] & 0xc0c0) >> 2));
        mp = (uint16_t)(((w[j + 2] >> 4) & 0x0f0f) | ((w[j] & 0xc0c0) >> 2));
    }
    out[0] = (uint8_t)(scp & 0xff);
    out[1] = (uint8_t)(scp >> 8);
    out[2] = (uint8_t)(mp & 0xff);
    out[3] = (uint8_t)(mp >> 8);
}

/* Packs 8 (sc, m) pairs of 6 bits into the 12 scale bytes; the layout that
 * quantize_row_q4_K_ref writes (ggml-quants.c). */
void orc_pack_scales_k4(const uint8_t *sc, const uint8_t *m, uint8_t *b) {
    memset(b, 0, 12);
    for (int s = 0; s < 8; ++s) {
        const uint8_t ls = sc[s] & 63, lm = m[s] & 63;
        if (s < 4) {
            b[s] = ls;
            b[s + 4] = lm;
        } else {
            b[s + 4] = (uint8_t)((ls & 0x0f) | ((lm & 0x0f) << 4));
            b[s - 4] |= (uint8_t)((ls >> 4) << 6);
            b[s] |= (uint8_t)((lm >> 4) << 6);
        }
    }
}

/* Exhaustive cross-check of the two unpackers: for every sub-block s, every
 * value of the (up to four) bytes it reads is enumerated in 3-byte slices.
 * Returns the number of disagreements. */
int64_t orc_selftest_scale_unpack(void) {
    int64_t bad = 0;
    uint8_t b[12], out[4], sc, m;
    for (int s = 0; s < 8; ++s) {
        const int j = s / 2, lohi = s & 1;
        /* bytes read by s: s<4: b[s], b[s+4]; s>=4: b[s+4], b[s-4], b[s] */
        int idx[3];
        int nidx;
        if (s < 4) {
            idx[0] = s; idx[1] = s + 4; nidx = 2;
        } else {
            idx[0] = s + 4; idx[1] = s - 4; idx[2] = s; nidx = 3;
        }
        const uint32_t lim = nidx == 2 ? (1u << 16) : (1u << 24);
        for (uint32_t v = 0; v < lim; ++v) {
            /* fill the remaining bytes with a pattern that changes with v */
            for (int i = 0; i < 12; ++i) b[i] = (uint8_t)(0xA5u ^ (v * 131u + (uint32_t)i * 29u));
            for (int i = 0; i < nidx; ++i) b[idx[i]] = (uint8_t)(v >> (8 * i));
            orc_scale_min_k4(s, b, &sc, &m);
            orc_vecdot_scale_pair(j, b, out);
            if (out[lohi] != sc || out[2 + lohi] != m) bad++;
        }
    }
    return bad;
}

/* The GPU quantiser computes d = amax/127 without a division instruction:
 * q0 = amax*RN(1/127), r = fma(-q0, 127, amax) (exact), d = fma(r, RN(1/127), q0).
 * Counts the float bit patterns lo, lo+stride, ... < hi (non-negative finite
 * floats: hi <= 0x7f800000) where that differs from the IEEE quotient
 * amax / 127.0f that ggml-cuda's quantize_q8_1 computes.  stride = 1 over
 * [0, 0x7f800000) is the exhaustive check. */
int64_t orc_check_div127(uint32_t lo, uint32_t hi, uint32_t stride) {
    const float rcp = (float)(1.0 / 127.0);
    int64_t bad = 0;
    if (stride == 0) stride = 1;
    for (uint64_t u = lo; u < hi; u += stride) {
        const uint32_t bits = (uint32_t)u;
        float a;
        memcpy(&a, &bits, 4);
        const float ref = a / 127.0f;
        const float q0 = a * rcp;
        const float r = fmaf(-q0, 127.0f, a);
        const float q1 = fmaf(r, rcp, q0);
        if (memcmp(&q1, &ref, 4) != 0) bad++;
    }
    return bad;
}

/* pack -> unpack identity for all 64x64 (sc, m) at every sub-block position */
int64_t orc_selftest_scale_pack(void) {
    int64_t bad = 0;
    uint8_t scv[8], mv[8], b[12], sc, m;
    for (int s = 0; s < 8; ++s) {
        for (int a = 0; a < 64; ++a) {
            for (int c = 0; c < 64; ++c) {
                for (int t = 0; t < 8; ++t) {
                    scv[t] = (uint8_t)((t * 23 + a + c) & 63);
                    mv[t] = (uint8_t)((t * 41 + 3 * a + c) & 63);
                }
                scv[s] = (uint8_t)a;
                mv[s] = (uint8_t)c;
                orc_pack_scales_k4(scv, mv, b);
                for (int t = 0; t < 8; ++t) {
                    orc_scale_min_k4(t, b, &sc, &m);
                    if (sc != scv[t] || m != mv[t]) bad++;
                }
            }
        }
    }
    return bad;
}

/* ------------------------------------------------------------------------ */
/* Q4_K weight quantiser (restates ggml-quants.c quantize_row_q4_K_ref)      */
/* ------------------------------------------------------------------------ */

/* make_qkx2_quants(n, nmax, x, weights, L, &min, Laux, rmin, rdelta, nstep,
 * use_mad=false): weighted least-squares fit of x ~ scale*L + min with L in
 * [0, nmax], min <= 0, trying nstep+1 candidate inverse scales.  Returns the
 * scale and stores -min. */
static float orc_make_qkx2_quants(int n, int nmax, const float *x, const float *w, uint8_t *L,
                                  float *neg_min, uint8_t *Laux, float rmin, float rdelta,
                                  int nstep) {
    float lo = x[0], hi = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < lo) lo = x[i];
        if (x[i] > hi) hi = x[i];
        sum_w += w[i];
        sum_x += w[i] * x[i];
    }
    if (lo > 0) lo = 0;
    if (hi == lo) {
        for (int i = 0; i < n; ++i) L[i] = 0;
        *neg_min = -lo;
        return 0.0f;
    }
    float iscale = nmax / (hi - lo);
    float scale = 1 / iscale;
    float best = 0;
    for (int i = 0; i < n; ++i) {
        int l = orc_nearest_int(iscale * (x[i] - lo));
        l = l < 0 ? 0 : (l > nmax ? nmax : l);
        L[i] = (uint8_t)l;
        float diff = scale * L[i] + lo - x[i];
        diff = diff * diff;
        best += w[i] * diff;
    }
    if (nstep < 1) {
        *neg_min = -lo;
        return scale;
    }
    for (int is = 0; is <= nstep; ++is) {
        iscale = (rmin + rdelta * is + nmax) / (hi - lo);
        float sum_l = 0, sum_l2 = 0, sum_xl = 0;
        for (int i = 0; i < n; ++i) {
            int l = orc_nearest_int(iscale * (x[i] - lo));
            l = l < 0 ? 0 : (l > nmax ? nmax : l);
            Laux[i] = (uint8_t)l;
            sum_l += w[i] * l;
            sum_l2 += w[i] * l * l;
            sum_xl += w[i] * l * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0) {
                this_min = 0;
                this_scale = sum_xl / sum_l2;
            }
            float cur = 0;
            for (int i = 0; i < n; ++i) {
                float diff = this_scale * Laux[i] + this_min - x[i];
                diff = diff * diff;
                cur += w[i] * diff;
            }
            if (cur < best) {
                for (int i = 0; i < n; ++i) L[i] = Laux[i];
                best = cur;
                scale = this_scale;
                lo = this_min;
            }
        }
    }
    *neg_min = -lo;
    return scale;
}

/* Stage 1 of quantize_row_q4_K_ref for one 256-value block: the
 * make_qkx2_quants fit of each 32-value sub-block, giving its scale, its
 * -min and its levels L.  ggml's parameters are rmin = -1, rdelta = 0.1,
 * nstep = 20 and the weights sqrt(mean(x^2)) + |x| (weight_mode 0); the
 * parameters are arguments so that the tests can plant a wrong one (weight_mode
 * 1: x^2) and see their brute-force check of the fit fail. */
void orc_q4K_fit_block(const float *x, float rmin, float rdelta, int nstep, int weight_mode,
                       float scales[8], float mins[8], uint8_t L[256]) {
    uint8_t Laux[32];
    float w[32];
    for (int s = 0; s < 8; ++s) {
        const float *xs = x + 32 * s;
        float sum_x2 = 0;
        for (int l = 0; l < 32; ++l) sum_x2 += xs[l] * xs[l];
        const float av_x = sqrtf(sum_x2 / 32);
        for (int l = 0; l < 32; ++l) w[l] = weight_mode == 1 ? xs[l] * xs[l] : av_x + fabsf(xs[l]);
        scales[s] = orc_make_qkx2_quants(32, 15, xs, w, L + 32 * s, &mins[s], Laux, rmin, rdelta, nstep);
    }
}

/* quantize_row_q4_K_ref: k floats (k % 256 == 0) -> k/256 blocks of 144 B. */
void orc_quantize_q4_K(const float *x, uint8_t *y, int64_t k) {
    const int64_t nb = k / ORC_QK_K;
    uint8_t L[ORC_QK_K];
    float mins[8], scales[8];
    for (int64_t i = 0; i < nb; ++i, x += ORC_QK_K, y += ORC_Q4K_BYTES) {
        float max_scale = 0, max_min = 0;
        orc_q4K_fit_block(x, -1.0f, 0.1f, 20, 0, scales, mins, L);
        for (int s = 0; s < 8; ++s) {
            if (scales[s] > max_scale) max_scale = scales[s];
            if (mins[s] > max_min) max_min = mins[s];
        }
        const float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
        const float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
        uint8_t ls[8], lm[8];
        for (int s = 0; s < 8; ++s) {
            int a = orc_nearest_int(inv_scale * scales[s]);
            int b = orc_nearest_int(inv_min * mins[s]);
            /* ggml stores the rounded value in a uint8_t before MIN(63, .) */
            uint8_t ua = (uint8_t)a, ub = (uint8_t)b;
            ls[s] = ua > 63 ? 63 : ua;
            lm[s] = ub > 63 ? 63 : ub;
        }
        uint8_t *sb = y + 4;
        orc_pack_scales_k4(ls, lm, sb);
        const uint16_t dh = orc_f32_to_f16(max_scale / 63.0f);
        const uint16_t mh = orc_f32_to_f16(max_min / 63.0f);
        y[0] = (uint8_t)(dh & 0xff); y[1] = (uint8_t)(dh >> 8);
        y[2] = (uint8_t)(mh & 0xff); y[3] = (uint8_t)(mh >> 8);
        for (int s = 0; s < 8; ++s) {
            uint8_t sc, m;
            orc_scale_min_k4(s, sb, &sc, &m);
            const float d = orc_f16_to_f32(dh) * sc;
            if (!d) continue;
            const float dm = orc_f16_to_f32(mh) * m;
            for (int l = 0; l < 32; ++l) {
                int q = orc_nearest_int((x[32 * s + l] + dm) / d);
                L[32 * s + l] = (uint8_t)(q < 0 ? 0 : (q > 15 ? 15 : q));
            }
        }
        uint8_t *qs = y + 16;
        for (int c = 0; c < 4; ++c)
            for (int l = 0; l < 32; ++l)
                qs[32 * c + l] = (uint8_t)(L[64 * c + l] | (L[64 * c + 32 + l] << 4));
    }
}

/* dequantize_row_q4_K: w = d*sc*q - dmin*m per sub-block */
void orc_dequantize_q4_K(const uint8_t *y, float *x, int64_t k) {
    const int64_t nb = k / ORC_QK_K;
    for (int64_t i = 0; i < nb; ++i, y += ORC_Q4K_BYTES, x += ORC_QK_K) {
        const float d = orc_f16_to_f32((uint16_t)(y[0] | (y[1] << 8)));
        const float mn = orc_f16_to_f32((uint16_t)(y[2] | (y[3] << 8)));
        const uint8_t *qs = y + 16;
        for (int s = 0; s < 8; ++s) {
            uint8_t sc, m;
            orc_scale_min_k4(s, y + 4, &sc, &m);
            const float d1 = d * sc, m1 = mn * m;
            const int c = s / 2, hi = s & 1;
            for (int l = 0; l < 32; ++l) {
                const int q = hi ? (qs[32 * c + l] >> 4) : (qs[32 * c + l] & 0x0f);
                x[32 * s + l] = d1 * q - m1;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Q8_1 activation quantiser (ggml-cuda quantize_q8_1, called at             */
/* kernels/mmvq.cu:728-735)                                                  */
/* ------------------------------------------------------------------------ */

/* One column of k floats -> k_padded/32 blocks of 36 B.  Elements at index
 * >= k are zero (the padding to MATRIX_ROW_PADDING=512, kernels/mmvq.cu:728).
 * Per block: amax via max, sum via the 32-lane butterfly tree of
 * warp_reduce_sum (lane 0 adds its partner at distance 16, 8, 4, 2, 1);
 * d = amax/127, q = amax == 0 ? 0 : roundf(x/d), ds = (half(d), half(sum)). */
void orc_quantize_q8_1(const float *x, int64_t k, int64_t k_padded, uint8_t *y) {
    const int64_t nb = k_padded / ORC_QK8_1;
    for (int64_t b = 0; b < nb; ++b, y += ORC_Q81_BYTES) {
        float v[32], t[32];
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const int64_t e = 32 * b + i;
            v[i] = e < k ? x[e] : 0.0f;
            t[i] = v[i];
            const float a = fabsf(v[i]);
            if (a > amax) amax = a;
        }
        for (int off = 16; off > 0; off >>= 1)
            for (int i = 0; i < off; ++i) t[i] = t[i] + t[i + off];
        const float sum = t[0];
        const float d = amax / 127;
        for (int i = 0; i < 32; ++i) {
            const int q = amax == 0.0f ? 0 : (int)roundf(v[i] / d);
            y[4 + i] = (uint8_t)(int8_t)q;
        }
        const uint16_t dh = orc_f32_to_f16(d), sh = orc_f32_to_f16(sum);
        y[0] = (uint8_t)(dh & 0xff); y[1] = (uint8_t)(dh >> 8);
        y[2] = (uint8_t)(sh & 0xff); y[3] = (uint8_t)(sh >> 8);
    }
}

/* N columns with column stride ldx floats -> N * k_padded/32 blocks */
void orc_quantize_q8_1_cols(const float *x, int64_t k, int64_t ldx, int64_t ncols, int64_t k_padded,
                            uint8_t *y) {
    for (int64_t c = 0; c < ncols; ++c)
        orc_quantize_q8_1(x + c * ldx, k, k_padded, y + c * (k_padded / ORC_QK8_1) * ORC_Q81_BYTES);
}

/* ------------------------------------------------------------------------ */
/* Q4_K x Q8_1 GEMV with the vec-dot's structure                             */
/* ------------------------------------------------------------------------ */

static inline int32_t orc_ld_i32(const uint8_t *p) {
    int32_t v;
    memcpy(&v, p, 4);
    return v;
}

/* sum over the four signed bytes of a*b (ggml_cuda_dp4a) */
static inline int32_t orc_dp4a(int32_t a, int32_t b, int32_t c) {
    for (int i = 0; i < 4; ++i) c += (int32_t)(int8_t)(a >> (8 * i)) * (int32_t)(int8_t)(b >> (8 * i));
    return c;
}

/*
 * y[c*ld_dst + r] for r < M, c < N, following kernels/vecdotq.cuh:775-819 and
 * :457-483 for every (block kb, iqs = 0,2,..,30) and kernels/mmvq.cu:236-256
 * for the accumulation over blocks of a row.
 *   w:   M rows of K/256 blocks, row stride row_stride bytes
 *   q8:  N columns of Q8_1 blocks, column stride stride_col_y blocks
 * Outputs (each optional):
 *   y64[c*M + r]             the result in double precision
 *   l1[c*M + r]              sum of |term| over the per-sub-block terms
 *                            d*d8*sc*S_qq and dmin*d8*m*S_q (error scale)
 *   sqq[(c*M + r)*(K/32)+s]  int32 sum over the sub-block of q4*q8
 *   sq[c*(K/32) + s]         int32 sum over the sub-block of q8
 */
/* Rows [r0, r1) of orc_gemv_q4K_q8_1 (outputs indexed as there); sq is
 * written by the range that holds row 0. */
static void orc_gemv_q4K_rows(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride, const uint8_t *q8,
                              int64_t N, int64_t stride_col_y, int64_t r0, int64_t r1, double *y64, double *l1,
                              int32_t *sqq, int32_t *sq) {
    const int64_t nb = K / ORC_QK_K, ns = K / 32;
    for (int64_t c = 0; c < N; ++c) {
        const uint8_t *yc = q8 + c * stride_col_y * ORC_Q81_BYTES;
        for (int64_t r = r0; r < r1; ++r) {
            const uint8_t *wr = w + r * row_stride;
            double acc = 0.0, acc_l1 = 0.0;
            for (int64_t kb = 0; kb < nb; ++kb) {
                const uint8_t *blk = wr + kb * ORC_Q4K_BYTES;
                const double d = orc_f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
                const double dmin = orc_f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
                const uint8_t *qs = blk + 16;
                /* per sub-block integer sums, collected from the 16 (iqs) lanes */
                int32_t s_qq[8] = {0}, s_q[8] = {0};
                uint8_t scm[8][2];
                for (int t = 0; t < 16; ++t) { /* iqs = 2t */
                    const int bq8_offset = 2 * (t / 4);
                    const uint8_t *q4 = qs + 16 * bq8_offset + 4 * (t % 4);
                    const int32_t v0 = orc_ld_i32(q4), v1 = orc_ld_i32(q4 + 16);
                    uint8_t pair[4];
                    orc_vecdot_scale_pair(bq8_offset / 2, blk + 4, pair);
                    for (int i = 0; i < 2; ++i) {
                        const uint8_t *b8 = yc + (kb * 8 + bq8_offset + i) * ORC_Q81_BYTES;
                        const int32_t u0 = orc_ld_i32(b8 + 4 + 4 * (t % 4));
                        const int32_t u1 = orc_ld_i32(b8 + 4 + 4 * (t % 4) + 16);
                        const int32_t v0i = (v0 >> (4 * i)) & 0x0f0f0f0f;
                        const int32_t v1i = (v1 >> (4 * i)) & 0x0f0f0f0f;
                        const int32_t dot1 = orc_dp4a(v1i, u1, orc_dp4a(v0i, u0, 0));
                        const int32_t dot2 = orc_dp4a(0x01010101, u1, orc_dp4a(0x01010101, u0, 0));
                        s_qq[bq8_offset + i] += dot1;
                        s_q[bq8_offset + i] += dot2;
                        scm[bq8_offset + i][0] = pair[i];
                        scm[bq8_offset + i][1] = pair[2 + i];
                    }
                }
                for (int s = 0; s < 8; ++s) {
                    const uint8_t *b8 = yc + (kb * 8 + s) * ORC_Q81_BYTES;
                    const double d8 = orc_f16_to_f32((uint16_t)(b8[0] | (b8[1] << 8)));
                    const double tq = d * d8 * (double)scm[s][0] * (double)s_qq[s];
                    const double tm = dmin * d8 * (double)scm[s][1] * (double)s_q[s];
                    acc += tq - tm;
                    acc_l1 += fabs(tq) + fabs(tm);
                    if (sqq) sqq[(c * M + r) * ns + kb * 8 + s] = s_qq[s];
                    if (sq && r == 0) sq[c * ns + kb * 8 + s] = s_q[s];
                }
            }
            if (y64) y64[c * M + r] = acc;
            if (l1) l1[c * M + r] = acc_l1;
        }
    }
}

void orc_gemv_q4K_q8_1(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride,
                       const uint8_t *q8, int64_t N, int64_t stride_col_y,
                       double *y64, double *l1, int32_t *sqq, int32_t *sq) {
    orc_gemv_q4K_rows(w, M, K, row_stride, q8, N, stride_col_y, 0, M, y64, l1, sqq, sq);
}

/* The same with the rows split over nthreads threads (contiguous ranges). */
typedef struct {
    const uint8_t *w, *q8;
    int64_t M, K, row_stride, N, stride_col_y, r0, r1;
    double *y64, *l1;
    int32_t *sqq, *sq;
} orc_gemv_task;

static void *orc_gemv_q4K_task(void *arg) {
    orc_gemv_task *t = (orc_gemv_task *)arg;
    orc_gemv_q4K_rows(t->w, t->M, t->K, t->row_stride, t->q8, t->N, t->stride_col_y, t->r0, t->r1, t->y64,
                      t->l1, t->sqq, t->sq);
    return NULL;
}

void orc_gemv_q4K_q8_1_mt(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride, const uint8_t *q8,
                          int64_t N, int64_t stride_col_y, double *y64, double *l1, int32_t *sqq, int32_t *sq,
                          int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if (nthreads > M) nthreads = M > 0 ? (int)M : 1;
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    orc_gemv_task *task = (orc_gemv_task *)malloc(sizeof(orc_gemv_task) * (size_t)nthreads);
    for (int i = 0; i < nthreads; ++i) {
        orc_gemv_task t = {w, q8, M, K, row_stride, N, stride_col_y, M * i / nthreads, M * (i + 1) / nthreads,
                           y64, l1, sqq, sq};
        task[i] = t;
        if (i > 0) pthread_create(&th[i], NULL, orc_gemv_q4K_task, &task[i]);
    }
    orc_gemv_q4K_task(&task[0]);
    for (int i = 1; i < nthreads; ++i) pthread_join(th[i], NULL);
    free(th);
    free(task);
}

/* ------------------------------------------------------------------------ */
/* ggml CPU path: Q8_K activations and ggml_vec_dot_q4_K_q8_K                */
/* ------------------------------------------------------------------------ */

/* quantize_row_q8_K_ref: per 256 values, the signed value of largest
 * magnitude fixes iscale = -127/max; q = min(127, nearest_int(iscale*x));
 * d = 1/iscale; bsums[j] = sum of q over 16-element group j. */
void orc_quantize_q8_K(const float *x, uint8_t *y, int64_t k) {
    const int64_t nb = k / ORC_QK_K;
    for (int64_t i = 0; i < nb; ++i, x += ORC_QK_K, y += ORC_Q8K_BYTES) {
        float mx = 0, amax = 0;
        for (int j = 0; j < ORC_QK_K; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) { amax = ax; mx = x[j]; }
        }
        int8_t *qs = (int8_t *)(y + 4);
        int16_t bs[16];
        if (!amax) {
            const float z = 0.0f;
            memcpy(y, &z, 4);
            memset(qs, 0, ORC_QK_K);
            memset(bs, 0, sizeof(bs));
            memcpy(y + 4 + ORC_QK_K, bs, sizeof(bs));
            continue;
        }
        const float iscale = -127.0f / mx;
        for (int j = 0; j < ORC_QK_K; ++j) {
            const int v = orc_nearest_int(iscale * x[j]);
            qs[j] = (int8_t)(v > 127 ? 127 : v);
        }
        for (int g = 0; g < 16; ++g) {
            int s = 0;
            for (int l = 0; l < 16; ++l) s += qs[16 * g + l];
            bs[g] = (int16_t)s;
        }
        memcpy(y + 4 + ORC_QK_K, bs, sizeof(bs));
        const float d = 1 / iscale;
        memcpy(y, &d, 4);
    }
}

/* the 12 scale bytes -> 8 scales (sc[0..7]) and 8 mins (m[0..7]) as bytes */
static inline void orc_unpack_k4_all(const uint8_t *b, uint8_t sc[8], uint8_t m[8]) {
    for (int s = 0; s < 8; ++s) orc_scale_min_k4(s, b, &sc[s], &m[s]);
}

/* ggml_vec_dot_q4_K_q8_K, portable form: eight int32 lanes (lane l takes
 * elements 8t+l of every 32-wide sub-block's 8-element slices) scaled per block
 * by d_w*d_y and summed in float, the min term subtracted per block. */
float orc_vec_dot_q4_K_q8_K_scalar(int64_t n, const uint8_t *x, const uint8_t *y) {
    const int64_t nb = n / ORC_QK_K;
    float sums[8] = {0};
    float sumf = 0;
    for (int64_t i = 0; i < nb; ++i, x += ORC_Q4K_BYTES, y += ORC_Q8K_BYTES) {
        float dy;
        memcpy(&dy, y, 4);
        const int8_t *q8 = (const int8_t *)(y + 4);
        int16_t bs[16];
        memcpy(bs, y + 4 + ORC_QK_K, sizeof(bs));
        uint8_t sc[8], m[8];
        orc_unpack_k4_all(x + 4, sc, m);
        int8_t a[ORC_QK_K];
        const uint8_t *qs = x + 16;
        for (int c = 0; c < 4; ++c) {
            for (int l = 0; l < 32; ++l) {
                a[64 * c + l] = (int8_t)(qs[32 * c + l] & 0x0f);
                a[64 * c + 32 + l] = (int8_t)(qs[32 * c + l] >> 4);
            }
        }
        int32_t summ = 0;
        for (int g = 0; g < 16; ++g) summ += bs[g] * m[g / 2];
        int32_t lanes[8] = {0};
        for (int s = 0; s < 8; ++s) {
            for (int t = 0; t < 4; ++t) {
                for (int l = 0; l < 8; ++l) {
                    const int e = 32 * s + 8 * t + l;
                    lanes[l] += sc[s] * ((int32_t)q8[e] * (int32_t)a[e]);
                }
            }
        }
        const float d = orc_f16_to_f32((uint16_t)(x[0] | (x[1] << 8))) * dy;
        for (int l = 0; l < 8; ++l) sums[l] += d * lanes[l];
        const float dmin = orc_f16_to_f32((uint16_t)(x[2] | (x[3] << 8))) * dy;
        sumf -= dmin * summ;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* The AVX2 form of the same dot (ggml-cpu/arch/x86/quants.c path): per block
 * the 4 chunks of 64 weights go through u8*s8 pair products (maddubs) and
 * 16-bit scale products (madd) into eight int32 lanes; the min term is an
 * int32x4 madd of the mins with the pairwise-added bsums; both accumulate in
 * float vectors across blocks and are reduced at the end. */
__attribute__((target("avx2,fma,f16c")))
float orc_vec_dot_q4_K_q8_K_avx2(int64_t n, const uint8_t *x, const uint8_t *y) {
    const int64_t nb = n / ORC_QK_K;
    const __m256i nib = _mm256_set1_epi8(0x0f);
    __m256 acc = _mm256_setzero_ps();
    __m128 acc_m = _mm_setzero_ps();
    for (int64_t i = 0; i < nb; ++i, x += ORC_Q4K_BYTES, y += ORC_Q8K_BYTES) {
        float dy;
        memcpy(&dy, y, 4);
        const float dw = _cvtsh_ss((unsigned short)(x[0] | (x[1] << 8)));
        const float mw = _cvtsh_ss((unsigned short)(x[2] | (x[3] << 8)));
        const float d = dy * dw;
        const float neg_dmin = -dy * mw;
        uint8_t sc[8], m[8];
        orc_unpack_k4_all(x + 4, sc, m);
        /* mins: 8 x int16 times (bsums[2s] + bsums[2s+1]) paired into int32x4 */
        const __m128i mins16 = _mm_cvtepu8_epi16(_mm_loadl_epi64((const __m128i *)m));
        const __m256i bs = _mm256_loadu_si256((const __m256i *)(y + 4 + ORC_QK_K));
        const __m128i bs32 = _mm_hadd_epi16(_mm256_castsi256_si128(bs), _mm256_extracti128_si256(bs, 1));
        const __m128i mprod = _mm_madd_epi16(mins16, bs32);
        acc_m = _mm_fmadd_ps(_mm_set1_ps(neg_dmin), _mm_cvtepi32_ps(mprod), acc_m);
        const uint8_t *qs = x + 16;
        const int8_t *q8 = (const int8_t *)(y + 4);
        __m256i sumi = _mm256_setzero_si256();
        for (int c = 0; c < 4; ++c) {
            const __m256i bits = _mm256_loadu_si256((const __m256i *)(qs + 32 * c));
            const __m256i lo = _mm256_and_si256(bits, nib);
            const __m256i hi = _mm256_and_si256(_mm256_srli_epi16(bits, 4), nib);
            const __m256i y_lo = _mm256_loadu_si256((const __m256i *)(q8 + 64 * c));
            const __m256i y_hi = _mm256_loadu_si256((const __m256i *)(q8 + 64 * c + 32));
            const __m256i p_lo = _mm256_madd_epi16(_mm256_set1_epi16((short)sc[2 * c]),
                                                   _mm256_maddubs_epi16(lo, y_lo));
            const __m256i p_hi = _mm256_madd_epi16(_mm256_set1_epi16((short)sc[2 * c + 1]),
                                                   _mm256_maddubs_epi16(hi, y_hi));
            sumi = _mm256_add_epi32(sumi, _mm256_add_epi32(p_lo, p_hi));
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(d), _mm256_cvtepi32_ps(sumi), acc);
    }
    acc_m = _mm_add_ps(acc_m, _mm_movehl_ps(acc_m, acc_m));
    acc_m = _mm_add_ss(acc_m, _mm_movehdup_ps(acc_m));
    __m128 h = _mm_add_ps(_mm256_castps256_ps128(acc), _mm256_extractf128_ps(acc, 1));
    h = _mm_add_ps(h, _mm_movehl_ps(h, h));
    h = _mm_add_ss(h, _mm_movehdup_ps(h));
    return _mm_cvtss_f32(h) + _mm_cvtss_f32(acc_m);
}

int orc_cpu_has_avx2(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma") ? 1 : 0;
}

/* ------------------------------------------------------------------------ */
/* threaded mul_mat (ggml_compute_forward_mul_mat shape of work)            */
/* ------------------------------------------------------------------------ */

typedef struct {
    const uint8_t *w;
    int64_t M, K, row_stride;
    const float *x;
    int64_t N, ldx;
    uint8_t *yq; /* N * (K/256) Q8_K blocks */
    float *dst;
    int64_t ld_dst;
    int use_avx2;
    int q6; /* weights are block_q6_K (vec_dot_q6_K_q8_K) */
    int nthreads;
    atomic_long next_chunk;
    pthread_barrier_t bar;
    int quantize;
} orc_mm_job;

typedef struct {
    orc_mm_job *job;
    int ith;
} orc_mm_arg;

/* CPUs the threads of orc_cpu_mul_mat_q4_K are pinned to (thread t on
 * cpus[t % n]); n = 0: not pinned. */
static int orc_pin_cpus[1024];
static int orc_pin_n = 0;

void orc_set_pin_cpus(const int *cpus, int n) {
    if (n < 0) n = 0;
    if (n > 1024) n = 1024;
    for (int i = 0; i < n; ++i) orc_pin_cpus[i] = cpus[i];
    orc_pin_n = n;
}

static void orc_pin_self(int t) {
    if (orc_pin_n == 0) return;
    cpu_set_t set;
    CPU_ZERO(&set);
    CPU_SET(orc_pin_cpus[t % orc_pin_n], &set);
    pthread_setaffinity_np(pthread_self(), sizeof(set), &set);
}

#define ORC_ROW_CHUNK 16

/* q6k_oracle.c */
float orc_vec_dot_q6_K_q8_K_scalar(int64_t n, const uint8_t *x, const uint8_t *y);
float orc_vec_dot_q6_K_q8_K_avx2(int64_t n, const uint8_t *x, const uint8_t *y);

static void *orc_mm_worker(void *p) {
    orc_mm_arg *a = (orc_mm_arg *)p;
    orc_mm_job *j = a->job;
    if (a->ith > 0) orc_pin_self(a->ith);
    const int64_t nbk = j->K / ORC_QK_K;
    /* 1. activations -> Q8_K, columns spread over threads */
    if (j->quantize) {
        for (int64_t c = a->ith; c < j->N; c += j->nthreads)
            orc_quantize_q8_K(j->x + c * j->ldx, j->yq + c * nbk * ORC_Q8K_BYTES, j->K);
    }
    pthread_barrier_wait(&j->bar);
    /* 2. output rows in chunks of 16, handed out through an atomic counter */
    const int64_t nchunks = (j->M + ORC_ROW_CHUNK - 1) / ORC_ROW_CHUNK;
    for (;;) {
        const int64_t ch = atomic_fetch_add(&j->next_chunk, 1);
        if (ch >= nchunks) break;
        const int64_t r0 = ch * ORC_ROW_CHUNK;
        const int64_t r1 = r0 + ORC_ROW_CHUNK < j->M ? r0 + ORC_ROW_CHUNK : j->M;
        for (int64_t c = 0; c < j->N; ++c) {
            const uint8_t *yc = j->yq + c * nbk * ORC_Q8K_BYTES;
            for (int64_t r = r0; r < r1; ++r) {
                const uint8_t *wr = j->w + r * j->row_stride;
                j->dst[c * j->ld_dst + r] =
                    j->q6 ? (j->use_avx2 ? orc_vec_dot_q6_K_q8_K_avx2(j->K, wr, yc)
                                         : orc_vec_dot_q6_K_q8_K_scalar(j->K, wr, yc))
                          : (j->use_avx2 ? orc_vec_dot_q4_K_q8_K_avx2(j->K, wr, yc)
                                         : orc_vec_dot_q4_K_q8_K_scalar(j->K, wr, yc));
            }
        }
    }
    return NULL;
}

/* dst[c*ld_dst + r] = dot(W row r, Q8_K(x column c)).  yq is caller scratch of
 * N*(K/256)*292 bytes; with quantize == 0 it must already hold Q8_K(x).
 * isa: 0 scalar, 1 AVX2 (falls back to scalar when the CPU lacks it).
 * Returns the ISA used. */
static int orc_cpu_mul_mat(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride, const float *x,
                           int64_t N, int64_t ldx, uint8_t *yq, float *dst, int64_t ld_dst,
                           int nthreads, int isa, int quantize, int q6) {
    if (nthreads < 1) nthreads = 1;
    orc_mm_job job;
    job.q6 = q6;
    job.w = w; job.M = M; job.K = K; job.row_stride = row_stride;
    job.x = x; job.N = N; job.ldx = ldx; job.yq = yq; job.dst = dst; job.ld_dst = ld_dst;
    job.use_avx2 = (isa == 1) && orc_cpu_has_avx2();
    job.nthreads = nthreads;
    job.quantize = quantize;
    atomic_init(&job.next_chunk, 0);
    pthread_barrier_init(&job.bar, NULL, (unsigned)nthreads);
    /* the calling thread works as thread 0: pinned for the call, then
     * restored */
    cpu_set_t saved;
    const int restore = orc_pin_n > 0 && pthread_getaffinity_np(pthread_self(), sizeof(saved), &saved) == 0;
    orc_pin_self(0);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    orc_mm_arg *args = (orc_mm_arg *)malloc(sizeof(orc_mm_arg) * (size_t)nthreads);
    for (int t = 0; t < nthreads; ++t) {
        args[t].job = &job;
        args[t].ith = t;
        if (t > 0) pthread_create(&th[t], NULL, orc_mm_worker, &args[t]);
    }
    orc_mm_worker(&args[0]);
    for (int t = 1; t < nthreads; ++t) pthread_join(th[t], NULL);
    if (restore) pthread_setaffinity_np(pthread_self(), sizeof(saved), &saved);
    pthread_barrier_destroy(&job.bar);
    free(th);
    free(args);
    return job.use_avx2;
}

int orc_cpu_mul_mat_q4_K(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride, const float *x,
                         int64_t N, int64_t ldx, uint8_t *yq, float *dst, int64_t ld_dst,
                         int nthreads, int isa, int quantize) {
    return orc_cpu_mul_mat(w, M, K, row_stride, x, N, ldx, yq, dst, ld_dst, nthreads, isa, quantize, 0);
}

/* The same for block_q6_K weights (vec_dot_q6_K_q8_K). */
int orc_cpu_mul_mat_q6_K(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride, const float *x,
                         int64_t N, int64_t ldx, uint8_t *yq, float *dst, int64_t ld_dst,
                         int nthreads, int isa, int quantize) {
    return orc_cpu_mul_mat(w, M, K, row_stride, x, N, ldx, yq, dst, ld_dst, nthreads, isa, quantize, 1);
}

/* Times `reps` calls of orc_cpu_mul_mat_q4_K (q6: orc_cpu_mul_mat_q6_K) and
 * writes each call's wall time in seconds into t[0..reps). */
static void orc_time_cpu_mul_mat(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride,
                                 const float *x, int64_t N, int64_t ldx, uint8_t *yq, float *dst,
                                 int64_t ld_dst, int nthreads, int isa, int quantize, int reps,
                                 double *t, int q6) {
    for (int i = 0; i < reps; ++i) {
        struct timespec a, b;
        clock_gettime(CLOCK_MONOTONIC, &a);
        orc_cpu_mul_mat(w, M, K, row_stride, x, N, ldx, yq, dst, ld_dst, nthreads, isa, quantize, q6);
        clock_gettime(CLOCK_MONOTONIC, &b);
        t[i] = (double)(b.tv_sec - a.tv_sec) + 1e-9 * (double)(b.tv_nsec - a.tv_nsec);
    }
}

void orc_time_cpu_mul_mat_q4_K(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride,
                               const float *x, int64_t N, int64_t ldx, uint8_t *yq, float *dst,
                               int64_t ld_dst, int nthreads, int isa, int quantize, int reps,
                               double *t) {
    orc_time_cpu_mul_mat(w, M, K, row_stride, x, N, ldx, yq, dst, ld_dst, nthreads, isa, quantize, reps, t, 0);
}

void orc_time_cpu_mul_mat_q6_K(const uint8_t *w, int64_t M, int64_t K, int64_t row_stride,
                               const float *x, int64_t N, int64_t ldx, uint8_t *yq, float *dst,
                               int64_t ld_dst, int nthreads, int isa, int quantize, int reps,
                               double *t) {
    orc_time_cpu_mul_mat(w, M, K, row_stride, x, N, ldx, yq, dst, ld_dst, nthreads, isa, quantize, reps, t, 1);
}

/* ------------------------------------------------------------------------ */
/* threaded Q4_K quantisation of many rows (fixture / input generation)     */
/* ------------------------------------------------------------------------ */

typedef struct {
    const float *x;
    uint8_t *y;
    int64_t nrows, K;
    atomic_long next;
} orc_q_job;

static void *orc_q_worker(void *p) {
    orc_q_job *j = (orc_q_job *)p;
    const int64_t rb = (j->K / ORC_QK_K) * ORC_Q4K_BYTES;
    for (;;) {
        const int64_t r0 = atomic_fetch_add(&j->next, 64);
        if (r0 >= j->nrows) break;
        const int64_t r1 = r0 + 64 < j->nrows ? r0 + 64 : j->nrows;
        for (int64_t r = r0; r < r1; ++r) orc_quantize_q4_K(j->x + r * j->K, j->y + r * rb, j->K);
    }
    return NULL;
}

void orc_quantize_q4_K_rows(const float *x, uint8_t *y, int64_t nrows, int64_t K, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    orc_q_job job;
    job.x = x; job.y = y; job.nrows = nrows; job.K = K;
    atomic_init(&job.next, 0);
    pthread_t *th = (pthread_t *)malloc(sizeof(pthread_t) * (size_t)nthreads);
    for (int t = 1; t < nthreads; ++t) pthread_create(&th[t], NULL, orc_q_worker, &job);
    orc_q_worker(&job);
    for (int t = 1; t < nthreads; ++t) pthread_join(th[t], NULL);
    free(th);
}
