// q4k_quantize_host.cpp -- host F32 -> Q4_K and Q6_K weight quantisers.
//
// Produce the weight formats the GEMVs consume, with the arithmetic of
// ggml's quantize_row_q4_K_ref and quantize_row_q6_K_ref (ggml-quants.c; the
// reference consumes their output and does not vendor them).
//
// Q4_K, per 256-value super-block:
//   1. each 32-value sub-block gets a weighted least-squares fit
//      x ~ scale*L + min, L in [0,15], min <= 0 (weights sqrt(mean x^2)+|x|,
//      21 candidate inverse scales (15 + -1 + 0.1*k)/(max-min));
//   2. scales and -mins are quantised to 6 bits against the block maxima,
//      d = fp16(max_scale/63), dmin = fp16(max_min/63);
//   3. every value is re-quantised against the fp16 (d*sc, dmin*m) it will be
//      decoded with, and the nibbles are packed 32 low + 32 high per 32 bytes.
// Q6_K, per 256-value super-block:
//   1. each 16-value group gets a fit x ~ scale*l, l in [-32, 31], weighted by
//      x^2, over 19 candidate inverse scales -(32 + 0.1*k)/x_m (k = -9..9,
//      x_m the value of largest magnitude), keeping the best by sum(wxl)^2/sum(wl^2);
//   2. the group scales are quantised to int8 against the one of largest
//      magnitude s_m: iscale = -128/s_m, sc = min(127, round(iscale*scale)),
//      d = fp16(1/iscale);
//   3. every value is re-quantised against fp16(d)*sc, and l + 32 is split
//      into ql (low nibbles) and qh (2-bit fields).
// Built with -ffp-contract=off: every float expression rounds as written,
// which the byte-for-byte agreement with ggml's reference code relies on.
#include <cmath>
#include <cstdint>
#include <cstring>
#include <thread>
#include <vector>
#include <atomic>

#include "../../include/q4k_gemv.h"

namespace {

constexpr int kSub = 32;
constexpr int kBlock = 256;
constexpr int kBytes = 144;

inline int round_half_even(float v) {
    // 1.5 * 2^23 bias: the float adder rounds to nearest-even at integer
    // granularity; valid for |v| < 2^22.
    float t = v + 12582912.0f;
    int32_t bits;
    std::memcpy(&bits, &t, sizeof bits);
    return (bits & 0x007fffff) - 0x00400000;
}

inline uint16_t to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, sizeof x);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) {
        uint32_t h = ((ax >> 23) - 112u) << 10 | ((ax & 0x7fffffu) >> 13);
        const uint32_t rem = ax & 0x1fffu;
        h += (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ? 1u : 0u;
        return (uint16_t)(sign | h);
    }
    if (ax < 0x33000000u) return (uint16_t)sign;
    const uint32_t shift = 126u - (ax >> 23);
    const uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t h = mant >> shift;
    const uint32_t rem = mant & ((1u << shift) - 1u);
    const uint32_t halfway = 1u << (shift - 1u);
    h += (rem > halfway || (rem == halfway && (h & 1u))) ? 1u : 0u;
    return (uint16_t)(sign | h);
}

inline float from_half(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        float f = (float)m * 5.9604644775390625e-08f;
        return sign ? -f : f;
    }
    uint32_t x = e == 31 ? (sign | 0x7f800000u | (m << 13)) : (sign | ((e + 112u) << 23) | (m << 13));
    float f;
    std::memcpy(&f, &x, sizeof f);
    return f;
}

inline uint8_t clamp15(int v) { return (uint8_t)(v < 0 ? 0 : (v > 15 ? 15 : v)); }

// Weighted fit of one sub-block; returns the scale, writes -min and levels.
float fit_subblock(const float *x, const float *w, uint8_t *levels, float *neg_min) {
    float lo = x[0], hi = x[0], sw = w[0], sx = w[0] * x[0];
    for (int i = 1; i < kSub; ++i) {
        lo = x[i] < lo ? x[i] : lo;
        hi = x[i] > hi ? x[i] : hi;
        sw += w[i];
        sx += w[i] * x[i];
    }
    if (lo > 0) lo = 0;
    if (hi == lo) {
        std::memset(levels, 0, kSub);
        *neg_min = -lo;
        return 0.0f;
    }
    float inv = 15 / (hi - lo);
    float scale = 1 / inv;
    float best = 0;
    for (int i = 0; i < kSub; ++i) {
        levels[i] = clamp15(round_half_even(inv * (x[i] - lo)));
        float e = scale * levels[i] + lo - x[i];
        best += w[i] * (e * e);
    }
    uint8_t trial[kSub];
    for (int step = 0; step <= 20; ++step) {
        inv = (-1.0f + 0.1f * step + 15) / (hi - lo);
        float sl = 0, sl2 = 0, sxl = 0;
        for (int i = 0; i < kSub; ++i) {
            const int l = clamp15(round_half_even(inv * (x[i] - lo)));
            trial[i] = (uint8_t)l;
            sl += w[i] * l;
            sl2 += w[i] * l * l;
            sxl += w[i] * l * x[i];
        }
        const float det = sw * sl2 - sl * sl;
        if (!(det > 0)) continue;
        float s = (sw * sxl - sx * sl) / det;
        float mn = (sl2 * sx - sl * sxl) / det;
        if (mn > 0) {
            mn = 0;
            s = sxl / sl2;
        }
        float err = 0;
        for (int i = 0; i < kSub; ++i) {
            float e = s * trial[i] + mn - x[i];
            err += w[i] * (e * e);
        }
        if (err < best) {
            std::memcpy(levels, trial, kSub);
            best = err;
            scale = s;
            lo = mn;
        }
    }
    *neg_min = -lo;
    return scale;
}

// (sc, m) of sub-block s from the 12 packed bytes
inline void scale_min(int s, const uint8_t *b, uint8_t &sc, uint8_t &m) {
    if (s < 4) {
        sc = b[s] & 63;
        m = b[s + 4] & 63;
    } else {
        sc = (uint8_t)((b[s + 4] & 0x0f) | ((b[s - 4] >> 6) << 4));
        m = (uint8_t)((b[s + 4] >> 4) | ((b[s] >> 6) << 4));
    }
}

void quantize_block(const float *x, uint8_t *out) {
    uint8_t levels[kBlock];
    float scales[8], mins[8], w[kSub];
    float max_scale = 0, max_min = 0;
    for (int s = 0; s < 8; ++s) {
        const float *xs = x + kSub * s;
        float sum2 = 0;
        for (int i = 0; i < kSub; ++i) sum2 += xs[i] * xs[i];
        const float rms = std::sqrt(sum2 / kSub);
        for (int i = 0; i < kSub; ++i) w[i] = rms + std::fabs(xs[i]);
        scales[s] = fit_subblock(xs, w, levels + kSub * s, &mins[s]);
        if (scales[s] > max_scale) max_scale = scales[s];
        if (mins[s] > max_min) max_min = mins[s];
    }
    const float inv_scale = max_scale > 0 ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0 ? 63.0f / max_min : 0.0f;
    uint8_t *sb = out + 4;
    std::memset(sb, 0, 12);
    for (int s = 0; s < 8; ++s) {
        uint8_t ls = (uint8_t)round_half_even(inv_scale * scales[s]);
        uint8_t lm = (uint8_t)round_half_even(inv_min * mins[s]);
        ls = ls > 63 ? 63 : ls;
        lm = lm > 63 ? 63 : lm;
        if (s < 4) {
            sb[s] = ls;
            sb[s + 4] = lm;
        } else {
            sb[s + 4] = (uint8_t)((ls & 0x0f) | ((lm & 0x0f) << 4));
            sb[s - 4] |= (uint8_t)((ls >> 4) << 6);
            sb[s] |= (uint8_t)((lm >> 4) << 6);
        }
    }
    const uint16_t dh = to_half(max_scale / 63.0f), mh = to_half(max_min / 63.0f);
    std::memcpy(out, &dh, 2);
    std::memcpy(out + 2, &mh, 2);
    const float dd = from_half(dh), dm = from_half(mh);
    for (int s = 0; s < 8; ++s) {
        uint8_t sc, m;
        scale_min(s, sb, sc, m);
        const float d = dd * sc;
        if (!d) continue;
        const float off = dm * m;
        for (int i = 0; i < kSub; ++i) levels[kSub * s + i] = clamp15(round_half_even((x[kSub * s + i] + off) / d));
    }
    uint8_t *qs = out + 16;
    for (int c = 0; c < 4; ++c)
        for (int i = 0; i < 32; ++i)
            qs[32 * c + i] = (uint8_t)(levels[64 * c + i] | (levels[64 * c + 32 + i] << 4));
}

// ---------------------------------------------------------------- Q6_K ----

constexpr int kQ6Bytes = 210;
constexpr float kGroupEps = 1e-15f;  // ggml's GROUP_MAX_EPS

inline int clamp_q6(int v) { return v < -32 ? -32 : (v > 31 ? 31 : v); }

// Fit of one 16-value group (ggml's make_qx_quants with nmax 32, weights
// x^2): returns the scale and writes the levels l + 32.
float fit_group16(const float *x, int8_t *levels) {
    float amax = 0.0f, xm = 0.0f;
    for (int i = 0; i < 16; ++i) {
        const float ax = std::fabs(x[i]);
        if (ax > amax) {
            amax = ax;
            xm = x[i];
        }
    }
    if (amax < kGroupEps) {
        for (int i = 0; i < 16; ++i) levels[i] = 0;
        return 0.0f;
    }
    float iscale = -32.0f / xm;
    float sumlx = 0.0f, suml2 = 0.0f;
    for (int i = 0; i < 16; ++i) {
        const int l = clamp_q6(round_half_even(iscale * x[i]));
        levels[i] = (int8_t)(l + 32);
        const float w = x[i] * x[i];
        sumlx += w * x[i] * (float)l;
        suml2 += w * (float)l * (float)l;
    }
    float scale = suml2 != 0.0f ? sumlx / suml2 : 0.0f;
    float best = scale * sumlx;
    for (int k = -9; k <= 9; ++k) {
        if (k == 0) continue;
        iscale = -(32.0f + 0.1f * (float)k) / xm;
        sumlx = suml2 = 0.0f;
        for (int i = 0; i < 16; ++i) {
            const int l = clamp_q6(round_half_even(iscale * x[i]));
            const float w = x[i] * x[i];
            sumlx += w * x[i] * (float)l;
            suml2 += w * (float)l * (float)l;
        }
        if (suml2 > 0.0f && sumlx * sumlx > best * suml2) {
            for (int i = 0; i < 16; ++i) levels[i] = (int8_t)(clamp_q6(round_half_even(iscale * x[i])) + 32);
            scale = sumlx / suml2;
            best = scale * sumlx;
        }
    }
    return scale;
}

void quantize_block_q6(const float *x, uint8_t *out) {
    int8_t levels[kBlock];
    float scales[16];
    float max_scale = 0.0f, max_abs = 0.0f;
    for (int g = 0; g < 16; ++g) {
        scales[g] = fit_group16(x + 16 * g, levels + 16 * g);
        const float a = std::fabs(scales[g]);
        if (a > max_abs) {
            max_abs = a;
            max_scale = scales[g];
        }
    }
    if (max_abs < kGroupEps) {
        std::memset(out, 0, kQ6Bytes);
        return;
    }
    const float iscale = -128.0f / max_scale;
    const uint16_t dh = to_half(1.0f / iscale);
    int8_t *sc = reinterpret_cast<int8_t *>(out + 192);
    for (int g = 0; g < 16; ++g) {
        const int v = round_half_even(iscale * scales[g]);
        sc[g] = (int8_t)(v < 127 ? v : 127);
    }
    const float d = from_half(dh);
    for (int g = 0; g < 16; ++g) {
        const float dg = d * (float)sc[g];
        if (dg == 0.0f) continue;
        for (int i = 0; i < 16; ++i)
            levels[16 * g + i] = (int8_t)(clamp_q6(round_half_even(x[16 * g + i] / dg)) + 32);
    }
    uint8_t *ql = out, *qh = out + 128;
    for (int h = 0; h < 2; ++h) {
        const int8_t *L = levels + 128 * h;
        for (int l = 0; l < 32; ++l) {
            ql[64 * h + l] = (uint8_t)((L[l] & 0xf) | ((L[l + 64] & 0xf) << 4));
            ql[64 * h + 32 + l] = (uint8_t)((L[l + 32] & 0xf) | ((L[l + 96] & 0xf) << 4));
            qh[32 * h + l] = (uint8_t)((L[l] >> 4) | ((L[l + 32] >> 4) << 2) | ((L[l + 64] >> 4) << 4) |
                                       ((L[l + 96] >> 4) << 6));
        }
    }
    out[208] = (uint8_t)(dh & 0xff);
    out[209] = (uint8_t)(dh >> 8);
}

// nrows x n_per_row floats -> blocks of `bytes` each, on up to nthreads threads.
int quantize_rows(const float *src, void *dst, int64_t nrows, int64_t n_per_row, int nthreads, int bytes,
                  void (*block_fn)(const float *, uint8_t *)) {
    if (nrows < 0 || n_per_row <= 0 || n_per_row % kBlock != 0) return Q4K_EINVAL;
    if (nrows == 0) return Q4K_OK;
    if (!src || !dst) return Q4K_EINVAL;
    const int64_t total = nrows * (n_per_row / kBlock);
    uint8_t *out = static_cast<uint8_t *>(dst);
    if (nthreads < 1) nthreads = 1;
    std::atomic<int64_t> next{0};
    auto work = [&]() {
        constexpr int64_t chunk = 256;
        for (;;) {
            const int64_t b0 = next.fetch_add(chunk);
            if (b0 >= total) break;
            const int64_t b1 = b0 + chunk < total ? b0 + chunk : total;
            for (int64_t b = b0; b < b1; ++b) block_fn(src + b * kBlock, out + b * bytes);
        }
    };
    std::vector<std::thread> pool;
    for (int t = 1; t < nthreads; ++t) pool.emplace_back(work);
    work();
    for (auto &t : pool) t.join();
    return Q4K_OK;
}

}  // namespace

extern "C" int q4k_quantize_rows_q4_K(const float *src, void *dst, int64_t nrows, int64_t n_per_row,
                                      int nthreads) {
    return quantize_rows(src, dst, nrows, n_per_row, nthreads, kBytes, quantize_block);
}

extern "C" int q4k_quantize_rows_q6_K(const float *src, void *dst, int64_t nrows, int64_t n_per_row,
                                      int nthreads) {
    return quantize_rows(src, dst, nrows, n_per_row, nthreads, kQ6Bytes, quantize_block_q6);
}
