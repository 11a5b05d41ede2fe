/*
 * thq_oracle.c — scalar CPU restatement of the reference's GGUF quantized
 * matmul path.  TEST INFRASTRUCTURE ONLY (the checker, never the product).
 *
 * Built with -ffp-contract=off so that every f32 expression rounds exactly as
 * written (Rust, which candle is written in, never contracts a*b+c).
 *
 * [ext] = candle-core 0.11.0 (engine/Cargo.lock:253-256), file
 * src/quantized/k_quants.rs and src/quantized/utils.rs, not present in the
 * reference tree; restated from the published GGML block formats.
 */
#include "thq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ */
/* scalar conversions                                                   */
/* ------------------------------------------------------------------ */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float o_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return u2f(sign);
        /* subnormal: man * 2^-24, exact in f32 */
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    if (exp == 31) return u2f(sign | 0x7f800000u | (man << 13));
    return u2f(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t o_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {                       /* inf / nan */
        if (ax == 0x7f800000u) return sign | 0x7c00u;
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    }
    if (ax >= 0x477ff000u) return sign | 0x7c00u;   /* rounds to >= 65520 -> inf */
    if (ax < 0x38800000u) {                        /* result subnormal or zero */
        if (ax < 0x33000000u) return sign;         /* < 2^-25: rounds to 0 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126u - e;                 /* 14..24 */
        uint32_t q = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t e = (ax >> 23) - 112u;
    uint32_t m = ax & 0x7fffffu;
    uint32_t q = (e << 10) | (m >> 13);
    uint32_t rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float o_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t o_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x0040u); /* quiet nan */
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

float o_bf16_round(float f) { return o_bf16_to_f32(o_f32_to_bf16(f)); }

/* ------------------------------------------------------------------ */
/* synthetic inputs                                                     */
/* ------------------------------------------------------------------ */

static inline uint64_t splitmix64(uint64_t* s) {
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* Stream `stream` of seed `seed`: state = seed ^ (stream * 0xD1B54A32D192ED03).
 * Pairs of uniforms in (0, 1] -> Box-Muller in f64 -> sigma * z -> f32. */
void o_randn(uint64_t seed, uint64_t stream, float sigma, float* out, size_t n) {
    uint64_t s = seed ^ (stream * 0xD1B54A32D192ED03ull);
    const double two_pi = 6.283185307179586476925286766559;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
        double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
        double r = sqrt(-2.0 * log(u1));
        out[i] = (float)((double)sigma * r * cos(two_pi * u2));
        if (i + 1 < n) out[i + 1] = (float)((double)sigma * r * sin(two_pi * u2));
    }
}

/* ------------------------------------------------------------------ */
/* block formats                                                        */
/* ------------------------------------------------------------------ */

size_t o_row_bytes(int type, int64_t k) {
    if (type == O_TYPE_Q8_0) return (size_t)(k / OQK8_0) * O_Q8_0_BYTES;
    if (type == O_TYPE_Q4_K) return (size_t)(k / OQK_K) * O_Q4_K_BYTES;
    if (type == O_TYPE_Q6_K) return (size_t)(k / OQK_K) * O_Q6_K_BYTES;
    return 0;
}

static inline uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void wr16(uint8_t* p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* Rust's f32::round: half away from zero (C roundf has the same rule). */
static inline float rust_round(float v) { return roundf(v); }

/* [ext] candle utils.rs nearest_int: v.round() as i32 (Rust saturating cast). */
static inline int nearest_int(float v) {
    float r = rust_round(v);
    if (r != r) return 0;
    if (r >= 2147483647.0f) return 2147483647;
    if (r <= -2147483648.0f) return (-2147483647 - 1);
    return (int)r;
}

/* Rust `as i8` of an f32: saturating, NaN -> 0. */
static inline int8_t f32_as_i8(float v) {
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int8_t)v;
}

/* [ext] BlockQ8_0::from_float: amax = max|x|; d = amax / 127 (f32);
 * id = d != 0 ? 1/d : 0; qs = round(x * id) as i8; block.d = f16(d). */
void o_quantize_q8_0(const float* x, uint8_t* blocks, int64_t k) {
    for (int64_t b = 0; b < k / OQK8_0; ++b) {
        const float* xs = x + b * OQK8_0;
        uint8_t* blk = blocks + b * O_Q8_0_BYTES;
        float amax = 0.0f;
        for (int i = 0; i < OQK8_0; ++i) {
            float a = fabsf(xs[i]);
            amax = (a > amax || amax != amax) ? a : amax; /* f32::max */
        }
        float d = amax / 127.0f;
        float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        wr16(blk, o_f32_to_f16(d));
        for (int i = 0; i < OQK8_0; ++i) blk[2 + i] = (uint8_t)f32_as_i8(rust_round(xs[i] * id));
    }
}

/* [ext] BlockQ8_0::to_float: y = q as f32 * f32(d). */
void o_dequantize_q8_0(const uint8_t* blocks, float* y, int64_t k) {
    for (int64_t b = 0; b < k / OQK8_0; ++b) {
        const uint8_t* blk = blocks + b * O_Q8_0_BYTES;
        float d = o_f16_to_f32(rd16(blk));
        for (int i = 0; i < OQK8_0; ++i) y[b * OQK8_0 + i] = (float)(int8_t)blk[2 + i] * d;
    }
}

/* [ext] BlockQ6K::to_float (GGML's dequantize_row_q6_K): per 128-element
 * half n of a superblock (ql += 64n, qh += 32n, sc += 8n) and l = 0..31,
 * is = l / 16:
 *   y[l]      = d * sc[is]     * ((ql[l]      & 0xF) | ((qh[l] >> 0) & 3) << 4) - 32)
 *   y[l + 32] = d * sc[is + 2] * ((ql[l + 32] & 0xF) | ((qh[l] >> 2) & 3) << 4) - 32)
 *   y[l + 64] = d * sc[is + 4] * ((ql[l]      >> 4) | ((qh[l] >> 4) & 3) << 4) - 32)
 *   y[l + 96] = d * sc[is + 6] * ((ql[l + 32] >> 4) | ((qh[l] >> 6) & 3) << 4) - 32)
 * with the products evaluated left to right in f32 (d * sc first). */
void o_dequantize_q6_k(const uint8_t* blocks, float* y, int64_t k) {
    for (int64_t b = 0; b < k / OQK_K; ++b) {
        const uint8_t* blk = blocks + b * O_Q6_K_BYTES;
        const float d = o_f16_to_f32(rd16(blk + 208));
        float* yb = y + b * OQK_K;
        for (int n = 0; n < 2; ++n) {
            const uint8_t* ql = blk + 64 * n;
            const uint8_t* qh = blk + 128 + 32 * n;
            const int8_t* sc = (const int8_t*)(blk + 192 + 8 * n);
            float* yy = yb + 128 * n;
            for (int l = 0; l < 32; ++l) {
                const int is = l / 16;
                const int q1 = (int)((ql[l] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                const int q2 = (int)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                const int q3 = (int)((ql[l] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                const int q4 = (int)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                yy[l] = d * (float)sc[is] * (float)q1;
                yy[l + 32] = d * (float)sc[is + 2] * (float)q2;
                yy[l + 64] = d * (float)sc[is + 4] * (float)q3;
                yy[l + 96] = d * (float)sc[is + 6] * (float)q4;
            }
        }
    }
}

/* [ext] k_quants.rs get_scale_min_k4 (GGML's 6-bit scale/min packing). */
void o_get_scale_min_k4(int j, const uint8_t* q, uint8_t* sc, uint8_t* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* [ext] utils.rs make_qkx1_quants(nmax, ntry, x) -> (scale, -min):
 * min/max by total order, min clamped to <= 0, iscale = nmax/(max-min),
 * up to ntry refinement passes of (least-squares scale, mean-residual min),
 * stopping early when no level changed. */
void o_make_qkx1_quants(int nmax, int ntry, const float* x, int n, float* scale_out, float* min_out,
                        uint8_t* levels) {
    uint8_t l[256];
    memset(l, 0, sizeof(l));
    if (levels) memset(levels, 0, (size_t)n);
    float mn = x[0], mx = x[0];
    for (int i = 1; i < n; ++i) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
    }
    if (mx == mn) { *scale_out = 0.0f; *min_out = 0.0f; return; }
    float min = mn < 0.0f ? mn : 0.0f;
    float iscale = (float)nmax / (mx - min);
    float scale = 1.0f / iscale;
    for (int it = 0; it < ntry; ++it) {
        float sumlx = 0.0f;
        int suml2 = 0;
        int did_change = 0;
        for (int i = 0; i < n; ++i) {
            int li = nearest_int(iscale * (x[i] - min));
            if (li < 0) li = 0;
            if (li > nmax) li = nmax;
            if ((uint8_t)li != l[i]) { l[i] = (uint8_t)li; did_change = 1; }
            sumlx += (x[i] - min) * (float)li;
            suml2 += li * li;
        }
        scale = sumlx / (float)suml2;
        float sum = 0.0f;
        for (int i = 0; i < n; ++i) sum += x[i] - scale * (float)l[i];
        min = sum / (float)n;
        if (min > 0.0f) min = 0.0f;
        iscale = 1.0f / scale;
        if (!did_change) break;
    }
    *scale_out = scale;
    *min_out = -min;
    if (levels) memcpy(levels, l, (size_t)n);
}

/* [ext] BlockQ4K::from_float: per 32-sub-block make_qkx1_quants(15, 5);
 * 6-bit quantize scales and mins against their maxima (63/max), pack with
 * the k4 layout; d = f16(max_scale/63), dmin = f16(max_min/63); then
 * requantize every weight against the stored (d*sc, dmin*m). */
void o_quantize_q4_k(const float* x, uint8_t* blocks, int64_t k) {
    for (int64_t b = 0; b < k / OQK_K; ++b) {
        const float* xs = x + b * OQK_K;
        uint8_t* blk = blocks + b * O_Q4_K_BYTES;
        uint8_t* sc = blk + 4;
        uint8_t* qs = blk + 16;
        float scales[8], mins[8];
        for (int j = 0; j < 8; ++j) o_make_qkx1_quants(15, 5, xs + 32 * j, 32, &scales[j], &mins[j], NULL);
        float max_scale = 0.0f, max_min = 0.0f;
        for (int j = 0; j < 8; ++j) {
            max_scale = (scales[j] > max_scale || max_scale != max_scale) ? scales[j] : max_scale;
            max_min = (mins[j] > max_min || max_min != max_min) ? mins[j] : max_min;
        }
        float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
        float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
        memset(sc, 0, 12);
        for (int j = 0; j < 8; ++j) {
            int lsi = nearest_int(inv_scale * scales[j]);
            int lmi = nearest_int(inv_min * mins[j]);
            uint8_t ls = (uint8_t)(lsi < 63 ? lsi : 63);
            uint8_t lm = (uint8_t)(lmi < 63 ? lmi : 63);
            if (j < 4) {
                sc[j] = ls;
                sc[j + 4] = lm;
            } else {
                sc[j + 4] = (uint8_t)((ls & 0xF) | ((lm & 0xF) << 4));
                sc[j - 4] |= (uint8_t)((ls >> 4) << 6);
                sc[j] |= (uint8_t)((lm >> 4) << 6);
            }
        }
        uint16_t dh = o_f32_to_f16(max_scale / 63.0f);
        uint16_t mh = o_f32_to_f16(max_min / 63.0f);
        wr16(blk, dh);
        wr16(blk + 2, mh);
        uint8_t L[OQK_K];
        memset(L, 0, sizeof(L));
        for (int j = 0; j < 8; ++j) {
            uint8_t s, m;
            o_get_scale_min_k4(j, sc, &s, &m);
            float d = o_f16_to_f32(dh) * (float)s;
            if (d != 0.0f) {
                float dm = o_f16_to_f32(mh) * (float)m;
                for (int ii = 0; ii < 32; ++ii) {
                    int lv = nearest_int((xs[32 * j + ii] + dm) / d);
                    if (lv < 0) lv = 0;
                    if (lv > 15) lv = 15;
                    L[32 * j + ii] = (uint8_t)lv;
                }
            }
        }
        for (int j = 0; j < OQK_K; j += 64)
            for (int l = 0; l < 32; ++l) qs[(j / 64) * 32 + l] = (uint8_t)(L[j + l] | (L[j + l + 32] << 4));
    }
}

/* [ext] BlockQ4K::to_float: per 64-chunk j the two sub-blocks (2j, 2j+1):
 * d1 = d*sc, m1 = dmin*m; y = d1*(q&0xF) - m1 and y = d2*(q>>4) - m2. */
void o_dequantize_q4_k(const uint8_t* blocks, float* y, int64_t k) {
    for (int64_t b = 0; b < k / OQK_K; ++b) {
        const uint8_t* blk = blocks + b * O_Q4_K_BYTES;
        float d = o_f16_to_f32(rd16(blk));
        float dmin = o_f16_to_f32(rd16(blk + 2));
        const uint8_t* sc = blk + 4;
        const uint8_t* q = blk + 16;
        float* yb = y + b * OQK_K;
        int is = 0;
        for (int j = 0; j < OQK_K; j += 64) {
            uint8_t s, m;
            o_get_scale_min_k4(is, sc, &s, &m);
            float d1 = d * (float)s, m1 = dmin * (float)m;
            o_get_scale_min_k4(is + 1, sc, &s, &m);
            float d2 = d * (float)s, m2 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) yb[j + l] = d1 * (float)(q[l] & 0xF) - m1;
            for (int l = 0; l < 32; ++l) yb[j + 32 + l] = d2 * (float)(q[l] >> 4) - m2;
            q += 32;
            is += 2;
        }
    }
}

/* [ext] BlockQ8K::from_float: signed element of largest magnitude `max`
 * (first one wins on equal |x|), iscale = -128/max,
 * qs = min(round(iscale*x), 127) as i8, bsums over 16, d = 1/iscale.
 * Layout: f32 d, i8 qs[256], i16 bsums[16]. */
void o_quantize_q8_k(const float* x, uint8_t* blocks, int64_t k) {
    for (int64_t b = 0; b < k / OQK_K; ++b) {
        const float* xs = x + b * OQK_K;
        uint8_t* blk = blocks + b * O_Q8_K_BYTES;
        int8_t* qs = (int8_t*)(blk + 4);
        float max = 0.0f, amax = 0.0f;
        for (int i = 0; i < OQK_K; ++i) {
            if (amax < fabsf(xs[i])) { amax = fabsf(xs[i]); max = xs[i]; }
        }
        float d;
        if (amax == 0.0f) {
            d = 0.0f;
            memset(qs, 0, OQK_K);
        } else {
            float iscale = -128.0f / max;
            for (int i = 0; i < OQK_K; ++i) {
                float v = rust_round(iscale * xs[i]);
                qs[i] = f32_as_i8(v < 127.0f ? v : 127.0f);
            }
            d = 1.0f / iscale;
        }
        memcpy(blk, &d, 4);
        for (int j = 0; j < 16; ++j) {
            int s = 0;
            for (int i = 0; i < 16; ++i) s += qs[16 * j + i];
            int16_t s16 = (int16_t)s;
            memcpy(blk + 4 + OQK_K + 2 * j, &s16, 2);
        }
    }
}

/* ------------------------------------------------------------------ */
/* dot products                                                         */
/* ------------------------------------------------------------------ */

/* [ext] BlockQ8_0::vec_dot_unopt: sumf += (sum_i as f32) * f32(dw) * f32(dx). */
float o_vec_dot_q8_0_q8_0(int64_t k, const uint8_t* w, const uint8_t* x) {
    float sumf = 0.0f;
    for (int64_t b = 0; b < k / OQK8_0; ++b) {
        const uint8_t* wb = w + b * O_Q8_0_BYTES;
        const uint8_t* xb = x + b * O_Q8_0_BYTES;
        int32_t s = 0;
        for (int i = 0; i < OQK8_0; ++i) s += (int32_t)(int8_t)wb[2 + i] * (int32_t)(int8_t)xb[2 + i];
        sumf += (float)s * o_f16_to_f32(rd16(wb)) * o_f16_to_f32(rd16(xb));
    }
    return sumf;
}

/* [ext] BlockQ4K::vec_dot_unopt with BlockQ8K (GGML reference order):
 * per superblock: aux32[8] += scale_j * q8*q4 in lanes of 8, sumi = sum
 * bsums*mins; sums[l] += (d_w*d_x) * aux32[l]; sumf -= (dmin_w*d_x) * sumi;
 * result = sumf + sum(sums). */
float o_vec_dot_q4_k_q8_k(int64_t k, const uint8_t* w, const uint8_t* x) {
    float sums[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    float sumf = 0.0f;
    for (int64_t b = 0; b < k / OQK_K; ++b) {
        const uint8_t* wb = w + b * O_Q4_K_BYTES;
        const uint8_t* xb = x + b * O_Q8_K_BYTES;
        const uint8_t* q4 = wb + 16;
        const int8_t* q8 = (const int8_t*)(xb + 4);
        int8_t a[OQK_K];
        for (int j = 0; j < 4; ++j) {
            for (int l = 0; l < 32; ++l) a[64 * j + l] = (int8_t)(q4[32 * j + l] & 0xF);
            for (int l = 0; l < 32; ++l) a[64 * j + 32 + l] = (int8_t)(q4[32 * j + l] >> 4);
        }
        uint8_t scales[8], mins[8];
        for (int j = 0; j < 8; ++j) o_get_scale_min_k4(j, wb + 4, &scales[j], &mins[j]);
        int32_t sumi = 0;
        for (int j = 0; j < 16; ++j) {
            int16_t bs;
            memcpy(&bs, xb + 4 + OQK_K + 2 * j, 2);
            sumi += (int32_t)bs * (int32_t)mins[j / 2];
        }
        int32_t aux32[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        int off = 0;
        for (int j = 0; j < 8; ++j) {
            int32_t scale = scales[j];
            for (int r = 0; r < 4; ++r) {
                for (int l = 0; l < 8; ++l) aux32[l] += scale * (int32_t)((int16_t)q8[off + l] * (int16_t)a[off + l]);
                off += 8;
            }
        }
        float dx;
        memcpy(&dx, xb, 4);
        float d = o_f16_to_f32(rd16(wb)) * dx;
        for (int l = 0; l < 8; ++l) sums[l] += d * (float)aux32[l];
        float dmin = o_f16_to_f32(rd16(wb + 2)) * dx;
        sumf -= dmin * (float)sumi;
    }
    for (int l = 0; l < 8; ++l) sumf += sums[l];
    return sumf;
}

/* ------------------------------------------------------------------ */
/* whole-matrix helpers                                                 */
/* ------------------------------------------------------------------ */

static int block_of(int type) {
    return type == O_TYPE_Q8_0 ? OQK8_0 : (type == O_TYPE_Q4_K || type == O_TYPE_Q6_K) ? OQK_K : 0;
}
static void dequant_row(int type, const uint8_t* b, float* y, int64_t k) {
    if (type == O_TYPE_Q8_0) o_dequantize_q8_0(b, y, k);
    else if (type == O_TYPE_Q4_K) o_dequantize_q4_k(b, y, k);
    else o_dequantize_q6_k(b, y, k);
}

int o_quantize(int type, const float* w, int64_t n, int64_t k, uint8_t* out) {
    int bs = block_of(type);
    if (!bs || k % bs || type == O_TYPE_Q6_K) return -1;  /* no Q6_K quantizer: files carry Q6_K */
    size_t rb = o_row_bytes(type, k);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        if (type == O_TYPE_Q8_0) o_quantize_q8_0(w + r * k, out + r * rb, k);
        else o_quantize_q4_k(w + r * k, out + r * rb, k);
    }
    return 0;
}

int o_dequantize(int type, const uint8_t* blocks, int64_t n, int64_t k, float* out) {
    int bs = block_of(type);
    if (!bs || k % bs) return -1;
    size_t rb = o_row_bytes(type, k);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < n; ++r) {
        dequant_row(type, blocks + r * rb, out + r * k, k);
    }
    return 0;
}

/* [ext] k_quants::matmul((m,k,n), lhs, rhs_t, dst): quantize each lhs row to
 * VecDotType, then every (row, col) is T::vec_dot(k, rhs_col, lhs_row)
 * (candle splits the columns over rayon; the split does not change values).
 * Mode 0 replaces this with the exact dequantized weight and an f64 sum. */
int o_matmul(int type, int mode, const uint8_t* w, int64_t n, int64_t k, const float* x, int64_t m,
             float* y, int threads) {
    int bs = block_of(type);
    if (!bs || k % bs) return -1;
#ifdef _OPENMP
    int nt = threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
#endif
    size_t rb = o_row_bytes(type, k);
    if (mode == 0) {
#pragma omp parallel num_threads(nt)
        {
            float* wrow = (float*)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(static)
            for (int64_t c = 0; c < n; ++c) {
                dequant_row(type, w + c * rb, wrow, k);
                for (int64_t r = 0; r < m; ++r) {
                    const float* xr = x + r * k;
                    double acc = 0.0;
                    for (int64_t i = 0; i < k; ++i) acc += (double)xr[i] * (double)wrow[i];
                    y[r * n + c] = (float)acc;
                }
            }
            free(wrow);
        }
        return 0;
    }
    if (mode != 1 || type == O_TYPE_Q6_K) return -1;  /* Q8ACT is restated for Q8_0 / Q4_K */
    size_t xrb = type == O_TYPE_Q8_0 ? (size_t)(k / OQK8_0) * O_Q8_0_BYTES : (size_t)(k / OQK_K) * O_Q8_K_BYTES;
    uint8_t* xq = (uint8_t*)malloc(xrb * (size_t)(m > 0 ? m : 1));
    for (int64_t r = 0; r < m; ++r) {
        if (type == O_TYPE_Q8_0) o_quantize_q8_0(x + r * k, xq + r * xrb, k);
        else o_quantize_q8_k(x + r * k, xq + r * xrb, k);
    }
    for (int64_t r = 0; r < m; ++r) {
#pragma omp parallel for schedule(static) num_threads(nt)
        for (int64_t c = 0; c < n; ++c) {
            y[r * n + c] = type == O_TYPE_Q8_0 ? o_vec_dot_q8_0_q8_0(k, w + c * rb, xq + r * xrb)
                                               : o_vec_dot_q4_k_q8_k(k, w + c * rb, xq + r * xrb);
        }
    }
    free(xq);
    return 0;
}

/* ------------------------------------------------------------------ */
/* epilogues / consumers                                                */
/* ------------------------------------------------------------------ */

/* engine/src/qwen35.rs:7002-7007 (test expectation) and
 * engine/src/quant_kernel.rs:2922-2926 (kernel): g, u rounded to bf16,
 * value = g / (1 + e^-g) * u in f32, output bf16. */
void o_gate_up_silu(const float* y_gu, int64_t m, int64_t h, uint16_t* out) {
    for (int64_t r = 0; r < m; ++r) {
        for (int64_t i = 0; i < h; ++i) {
            float g = o_bf16_round(y_gu[r * 2 * h + i]);
            float u = o_bf16_round(y_gu[r * 2 * h + h + i]);
            float v = g / (1.0f + expf(-g)) * u;
            out[r * h + i] = o_f32_to_bf16(v);
        }
    }
}

/* engine/src/engine.rs:1891-1898 greedy_argmax: best = (0, -inf); strict '>'. */
uint32_t o_argmax(const float* v, int64_t n) {
    uint32_t bi = 0;
    float bv = -INFINITY;
    for (int64_t i = 0; i < n; ++i) {
        if (v[i] > bv) { bv = v[i]; bi = (uint32_t)i; }
    }
    return bi;
}

void o_argmax_rows(const float* v, int64_t m, int64_t n, uint32_t* idx) {
    for (int64_t r = 0; r < m; ++r) idx[r] = o_argmax(v + r * n, n);
}

/* engine/src/sample_kernel.rs key (:163-169): NaN ranks as -inf, -0.0 as +0.0. */
static float topk_key(float v) {
    if (v != v) return -INFINITY;
    return v + 0.0f;
}

typedef struct { float key; uint32_t id; } o_kv;

static int kv_cmp(const void* a, const void* b) {
    const o_kv* x = (const o_kv*)a;
    const o_kv* y = (const o_kv*)b;
    if (x->key != y->key) return x->key > y->key ? -1 : 1;  /* key desc */
    return x->id < y->id ? -1 : (x->id > y->id);            /* then id asc */
}

/* sorted_row_dist's candidate order (engine/src/sample_kernel.rs:326-337):
 * the first k of the row sorted by (key desc, id asc), keys reported as
 * key(v); slots past n are (-inf, 0xFFFFFFFF) as ts_topk leaves them. */
void o_topk_rows(const float* v, int64_t m, int64_t n, int k, float* vals, uint32_t* idx) {
    o_kv* buf = (o_kv*)malloc(sizeof(o_kv) * (size_t)(n > 0 ? n : 1));
    for (int64_t r = 0; r < m; ++r) {
        for (int64_t i = 0; i < n; ++i) {
            buf[i].key = topk_key(v[r * n + i]);
            buf[i].id = (uint32_t)i;
        }
        qsort(buf, (size_t)n, sizeof(o_kv), kv_cmp);
        for (int j = 0; j < k; ++j) {
            vals[r * k + j] = j < n ? buf[j].key : -INFINITY;
            idx[r * k + j] = j < n ? buf[j].id : 0xFFFFFFFFu;
        }
    }
    free(buf);
}

int o_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
