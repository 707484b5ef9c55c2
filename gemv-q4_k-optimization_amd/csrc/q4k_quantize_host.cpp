// q4k_quantize_host.cpp -- host F32 -> Q4_K weight quantiser.
//
// Produces the weight format the GEMV consumes, with the arithmetic of ggml's
// quantize_row_q4_K_ref (ggml-quants.c; the reference consumes its output and
// does not vendor it).  Per 256-value super-block:
//   1. each 32-value sub-block gets a weighted least-squares fit
//      x ~ scale*L + min, L in [0,15], min <= 0 (weights sqrt(mean x^2)+|x|,
//      21 candidate inverse scales (15 + -1 + 0.1*k)/(max-min));
//   2. scales and -mins are quantised to 6 bits against the block maxima,
//      d = fp16(max_scale/63), dmin = fp16(max_min/63);
//   3. every value is re-quantised against the fp16 (d*sc, dmin*m) it will be
//      decoded with, and the nibbles are packed 32 low + 32 high per 32 bytes.
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

}  // namespace

extern "C" int q4k_quantize_rows_q4_K(const float *src, void *dst, int64_t nrows, int64_t n_per_row,
                                      int nthreads) {
    if (nrows < 0 || n_per_row <= 0 || n_per_row % kBlock != 0) return Q4K_EINVAL;
    if (nrows == 0) return Q4K_OK;
    if (!src || !dst) return Q4K_EINVAL;
    const int64_t nb = n_per_row / kBlock;
    const int64_t total = nrows * nb;
    uint8_t *out = static_cast<uint8_t *>(dst);
    if (nthreads < 1) nthreads = 1;
    std::atomic<int64_t> next{0};
    auto work = [&]() {
        constexpr int64_t chunk = 256;
        for (;;) {
            const int64_t b0 = next.fetch_add(chunk);
            if (b0 >= total) break;
            const int64_t b1 = b0 + chunk < total ? b0 + chunk : total;
            for (int64_t b = b0; b < b1; ++b) quantize_block(src + b * kBlock, out + b * kBytes);
        }
    };
    std::vector<std::thread> pool;
    for (int t = 1; t < nthreads; ++t) pool.emplace_back(work);
    work();
    for (auto &t : pool) t.join();
    return Q4K_OK;
}
