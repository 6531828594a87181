/*
 * CPU oracle for the PocketLM quantized-decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker: it is loaded by tests/,
 * by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, never by the
 * product library (pocketlm_amd/), which has no CPU fallback.
 *
 * Each function restates the reference algorithm, in plain C, with the loop
 * nest and fp32 accumulation order of the reference kernel it follows, so that
 * its outputs can be compared bit for bit with a build of the reference
 * sources (oracle/_ref) and with the golden vectors under tests/golden.
 * Reference paths are relative to the PocketLM source tree.
 *
 * Build flags matter: -ffp-contract=off keeps "a += b * c" as a rounded
 * multiply followed by a rounded add, which is what the reference's scalar
 * loops compute (MSVC does not contract).  The row8 GEMV is the one place the
 * reference uses a fused multiply-add (_mm256_fmadd_ps) and it is written with
 * fmaf() here.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define ORC_API __attribute__((visibility("default")))

static inline float bits_to_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

static inline uint32_t f32_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    return u;
}

/* ------------------------------------------------------------------------- */
/* e4m3fn decoding                                                            */
/* ------------------------------------------------------------------------- */

/*
 * Value of an OCP e4m3fn byte.  nan_code selects what the two NaN encodings
 * (0x7F, 0xFF) decode to:
 *   0 -> +0.0  (GEMV/MLP kernels: src/pcketlm/native/fp8_linear.cpp:19-36,
 *               fp8_linear_avx512.cpp:9-26 and its bit decoder 67-88)
 *   1 -> NaN with f32 bits 0x7FF00000 / 0xFFF00000 by sign
 *               (dequant kernels: src/pcketlm/native/fp8_dequant.cpp:10-30)
 * Normal bytes are (-1)^s * (1 + m/8) * 2^(e-7); e == 0 gives m * 2^-9.
 */
static float e4m3_value(uint8_t byte, int nan_code) {
    const int negative = (byte & 0x80u) != 0;
    const int e = (byte >> 3) & 0xF;
    const int m = byte & 0x7;
    float mag;
    if (e == 0xF && m == 0x7) {
        if (nan_code == 0) {
            return 0.0f;
        }
        return bits_to_f32(negative ? 0xFFF00000u : 0x7FF00000u);
    }
    if (e == 0) {
        mag = ldexpf((float)m, -9);
    } else {
        mag = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    }
    return negative ? -mag : mag;
}

static float g_lut_linear[256];
static float g_lut_dequant[256];

__attribute__((constructor)) static void build_luts(void) {
    for (int i = 0; i < 256; ++i) {
        g_lut_linear[i] = e4m3_value((uint8_t)i, 0);
        g_lut_dequant[i] = e4m3_value((uint8_t)i, 1);
    }
}

ORC_API float orc_e4m3_linear(uint8_t byte) { return g_lut_linear[byte]; }
ORC_API float orc_e4m3_dequant(uint8_t byte) { return g_lut_dequant[byte]; }

/* ------------------------------------------------------------------------- */
/* half / bfloat16 conversions                                                */
/* ------------------------------------------------------------------------- */

/*
 * fp16 -> fp32, exact (src/pcketlm/native/q4_dequant.cpp:10-40 in software,
 * F16C _mm_cvtph_ps in fp16_packed_gemv.cpp:13-17).  NaN payloads are kept.
 */
ORC_API float orc_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 0) {
        if (m == 0) {
            return bits_to_f32(sign);
        }
        /* subnormal half: m * 2^-24, exact in f32 */
        float v = ldexpf((float)m, -24);
        return sign ? -v : v;
    }
    if (e == 0x1F) {
        return bits_to_f32(sign | 0x7F800000u | (m << 13));
    }
    return bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/*
 * fp32 -> fp16 with round-to-nearest-even, restating the software converter
 * of src/pcketlm/native/q4_dequant.cpp:42-90.  For finite inputs and
 * infinities this equals the x86 F16C conversion; for NaN it returns
 * sign | 0x7C00 | payload>>13 | 1 (the software converter's choice).
 */
ORC_API uint16_t orc_f32_to_f16_sw(float value) {
    const uint32_t bits = f32_to_bits(value);
    const uint32_t sign = (bits >> 16) & 0x8000u;
    uint32_t mant = bits & 0x7FFFFFu;
    int exp = (int)((bits >> 23) & 0xFFu);
    if (exp == 255) {
        return (uint16_t)(mant == 0 ? (sign | 0x7C00u) : (sign | 0x7C00u | (mant >> 13) | 1u));
    }
    exp = exp - 127 + 15;
    if (exp >= 31) {
        return (uint16_t)(sign | 0x7C00u);
    }
    if (exp <= 0) {
        if (exp < -10) {
            return (uint16_t)sign;
        }
        /* result is a half subnormal (or rounds up to the smallest normal) */
        mant |= 0x800000u;
        const uint32_t shift = (uint32_t)(14 - exp);
        uint32_t q = mant >> shift;
        const uint32_t half_bit = (mant >> (shift - 1)) & 1u;
        const uint32_t rest = mant & ((1u << (shift - 1)) - 1u);
        if (half_bit && (rest || (q & 1u))) {
            ++q;
        }
        return (uint16_t)(sign | q);
    }
    uint32_t he = (uint32_t)exp << 10;
    uint32_t hm = mant >> 13;
    const uint32_t tail = mant & 0x1FFFu;
    if (tail > 0x1000u || (tail == 0x1000u && (hm & 1u))) {
        ++hm;
        if (hm == 0x400u) {
            hm = 0;
            he += 0x400u;
            if (he >= 0x7C00u) {
                return (uint16_t)(sign | 0x7C00u);
            }
        }
    }
    return (uint16_t)(sign | he | hm);
}

/*
 * fp32 -> fp16 as the x86 F16C instruction (vcvtps2ph, RNE) computes it:
 * identical to the software converter except that a NaN keeps its upper
 * payload bits and gets the quiet bit: sign | 0x7E00 | payload>>13.  This is
 * the converter of src/pcketlm/native/fp8_dequant.cpp:81-106 and of the
 * AVX2 Q4 path q4_dequant.cpp:130-152.
 */
ORC_API uint16_t orc_f32_to_f16_hw(float value) {
    const uint32_t bits = f32_to_bits(value);
    if ((bits & 0x7F800000u) == 0x7F800000u && (bits & 0x7FFFFFu) != 0) {
        return (uint16_t)(((bits >> 16) & 0x8000u) | 0x7E00u | ((bits & 0x7FFFFFu) >> 13));
    }
    return orc_f32_to_f16_sw(value);
}

/*
 * fp32 -> bf16, round-to-nearest-even by adding 0x7FFF + lsb; every NaN maps
 * to 0xFFFF (src/pcketlm/native/fp8_dequant.cpp:108-117).
 */
ORC_API uint16_t orc_f32_to_bf16(float value) {
    if (isnan(value)) {
        return 0xFFFFu;
    }
    const uint32_t bits = f32_to_bits(value);
    const uint32_t lsb = (bits >> 16) & 1u;
    return (uint16_t)((bits + 0x7FFFu + lsb) >> 16);
}

static inline float bf16_to_f32(uint16_t v) { return bits_to_f32((uint32_t)v << 16); }

/* ------------------------------------------------------------------------- */
/* FP8 block-scaled GEMV family (src/pcketlm/native/fp8_linear.cpp)           */
/* ------------------------------------------------------------------------- */

/*
 * One row of a 128x128 block-scaled e4m3 weight dotted with one fp32 row:
 * for each 128-column scale block, a plain fp32 sum of hidden*w (multiply,
 * then add), then acc += block_sum * scale.  This is the per-(row, b)
 * arithmetic of every kernel in fp8_linear.cpp (e.g. 103-112, 74-88,
 * 535-549); the batch-reuse nests compute exactly the same operations in a
 * different loop order, which is why they are bit-exact to the default nest.
 */
static float fp8_row_dot(const uint8_t* wrow, const float* srow, const float* x,
                         int64_t cols, int64_t scale_cols) {
    float acc = 0.0f;
    for (int64_t sc = 0; sc < scale_cols; ++sc) {
        const int64_t c0 = sc * 128;
        const int64_t c1 = c0 + 128 < cols ? c0 + 128 : cols;
        float blk = 0.0f;
        for (int64_t c = c0; c < c1; ++c) {
            blk += x[c] * g_lut_linear[wrow[c]];
        }
        acc += blk * srow[sc];
    }
    return acc;
}

static float silu_mul(float gate, float up) {
    /* fp8_linear.cpp:279-280: gate / (1 + exp(-gate)) * up, in fp32 */
    const float s = gate / (1.0f + expf(-gate));
    return s * up;
}

/* fp8_linear.cpp:50-117 (fp8_e4m3_block_linear_f32); batch_reuse selects the
 * 68-94 nest (weights read once per row for all batch rows). */
ORC_API int orc_fp8_linear(const uint8_t* w, const float* s, const float* x, float* out,
                           int64_t batch, int64_t rows, int64_t cols, int64_t scale_cols,
                           int batch_reuse) {
    if (!w || !s || !x || !out) return -1;
    if (batch <= 0 || rows <= 0 || cols <= 0 || scale_cols <= 0) return -2;
    if (batch_reuse && batch > 1 && batch <= 64) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < rows; ++r) {
            const uint8_t* wrow = w + r * cols;
            const float* srow = s + (r / 128) * scale_cols;
            float acc[64] = {0.0f};
            for (int64_t sc = 0; sc < scale_cols; ++sc) {
                const int64_t c0 = sc * 128;
                const int64_t c1 = c0 + 128 < cols ? c0 + 128 : cols;
                float blk[64] = {0.0f};
                for (int64_t c = c0; c < c1; ++c) {
                    const float wv = g_lut_linear[wrow[c]];
                    for (int64_t b = 0; b < batch; ++b) blk[b] += x[b * cols + c] * wv;
                }
                for (int64_t b = 0; b < batch; ++b) acc[b] += blk[b] * srow[sc];
            }
            for (int64_t b = 0; b < batch; ++b) out[b * rows + r] = acc[b];
        }
        return 0;
    }
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t r = 0; r < rows; ++r) {
            out[b * rows + r] = fp8_row_dot(w + r * cols, s + (r / 128) * scale_cols,
                                            x + b * cols, cols, scale_cols);
        }
    }
    return 0;
}

/* fp8_linear.cpp:119-210 (fp8_e4m3_block_dual_linear_f32) */
ORC_API int orc_fp8_dual_linear(const uint8_t* wa, const float* sa, const uint8_t* wb,
                                const float* sb, const float* x, float* out_a, float* out_b,
                                int64_t batch, int64_t rows, int64_t cols, int64_t scale_cols) {
    if (!wa || !sa || !wb || !sb || !x || !out_a || !out_b) return -1;
    if (batch <= 0 || rows <= 0 || cols <= 0 || scale_cols <= 0) return -2;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t r = 0; r < rows; ++r) {
            const int64_t so = (r / 128) * scale_cols;
            out_a[b * rows + r] = fp8_row_dot(wa + r * cols, sa + so, x + b * cols, cols, scale_cols);
            out_b[b * rows + r] = fp8_row_dot(wb + r * cols, sb + so, x + b * cols, cols, scale_cols);
        }
    }
    return 0;
}

/*
 * Gate/up phase of one SwiGLU expert for one batch row: act[row] =
 * silu(gate_row . x) * (up_row . x)  (fp8_linear.cpp:310-335, 514-552).
 */
static void mlp_gate_up(const uint8_t* g, const float* gs, const uint8_t* u, const float* us,
                        const float* x, float* act, int64_t inter, int64_t hid, int64_t gsc) {
    for (int64_t r = 0; r < inter; ++r) {
        const int64_t so = (r / 128) * gsc;
        const float ga = fp8_row_dot(g + r * hid, gs + so, x, hid, gsc);
        const float ua = fp8_row_dot(u + r * hid, us + so, x, hid, gsc);
        act[r] = silu_mul(ga, ua);
    }
}

/* fp8_linear.cpp:212-362 (fp8_e4m3_block_mlp_f32); also the arithmetic of
 * the AVX-512 twin fp8_linear_avx512.cpp:157-250, whose lane-ordered sums are
 * bit-exact to it. */
ORC_API int orc_fp8_mlp(const uint8_t* g, const float* gs, const uint8_t* u, const float* us,
                        const uint8_t* d, const float* ds, const float* x, float* out,
                        int64_t batch, int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!g || !gs || !u || !us || !d || !ds || !x || !out) return -1;
    if (batch <= 0 || inter <= 0 || hid <= 0 || gsc <= 0 || dsc <= 0) return -2;
    float* act = (float*)malloc((size_t)(batch * inter) * sizeof(float));
    if (!act) return -3;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t r = 0; r < inter; ++r) {
            const int64_t so = (r / 128) * gsc;
            const float ga = fp8_row_dot(g + r * hid, gs + so, x + b * hid, hid, gsc);
            const float ua = fp8_row_dot(u + r * hid, us + so, x + b * hid, hid, gsc);
            act[b * inter + r] = silu_mul(ga, ua);
        }
    }
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t h = 0; h < hid; ++h) {
            out[b * hid + h] = fp8_row_dot(d + h * inter, ds + (h / 128) * dsc, act + b * inter,
                                           inter, dsc);
        }
    }
    free(act);
    return 0;
}

#define PTR(arr, e) ((const void*)(uintptr_t)(arr)[e])

/* fp8_linear.cpp:364-473 (fp8_e4m3_block_mlp_many_f32): out [E, batch, hid] */
ORC_API int orc_fp8_mlp_many(const uint64_t* gp, const uint64_t* gsp, const uint64_t* up,
                             const uint64_t* usp, const uint64_t* dp, const uint64_t* dsp,
                             const float* x, float* out, int64_t experts, int64_t batch,
                             int64_t inter, int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !x || !out) return -1;
    if (experts <= 0 || batch <= 0 || inter <= 0 || hid <= 0 || gsc <= 0 || dsc <= 0) return -2;
    float* act = (float*)malloc((size_t)(experts * batch * inter) * sizeof(float));
    if (!act) return -3;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t e = 0; e < experts; ++e) {
        for (int64_t b = 0; b < batch; ++b) {
            const uint8_t* g = PTR(gp, e);
            const float* gs = PTR(gsp, e);
            const uint8_t* u = PTR(up, e);
            const float* us = PTR(usp, e);
            if (!g || !gs || !u || !us) continue;
            mlp_gate_up(g, gs, u, us, x + b * hid, act + (e * batch + b) * inter, inter, hid, gsc);
        }
    }
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t e = 0; e < experts; ++e) {
        for (int64_t b = 0; b < batch; ++b) {
            const uint8_t* d = PTR(dp, e);
            const float* ds = PTR(dsp, e);
            if (!d || !ds) continue;
            for (int64_t h = 0; h < hid; ++h) {
                out[(e * batch + b) * hid + h] = fp8_row_dot(
                    d + h * inter, ds + (h / 128) * dsc, act + (e * batch + b) * inter, inter, dsc);
            }
        }
    }
    free(act);
    return 0;
}

/*
 * Shared core of the weighted MoE kernels.  route_of(e, b) is the route
 * weight of expert e for batch row b; zero_skip reproduces the row-weighted
 * kernel's skipping of (e, b) pairs whose weight is exactly 0.
 * Phase 1: fp8_linear.cpp:514-554; phase 2 (per output element, experts in
 * order, routed += route * expert_acc): 556-585 and 794-827.
 */
static int weighted_core(const uint64_t* gp, const uint64_t* gsp, const uint64_t* up,
                         const uint64_t* usp, const uint64_t* dp, const uint64_t* dsp,
                         const float* x, const float* route, int route_per_row, int zero_skip,
                         float* out, int64_t experts, int64_t batch, int64_t inter, int64_t hid,
                         int64_t gsc, int64_t dsc) {
    float* act = (float*)calloc((size_t)(experts * batch * inter), sizeof(float));
    if (!act) return -3;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t e = 0; e < experts; ++e) {
        for (int64_t b = 0; b < batch; ++b) {
            const float rw = route_per_row ? route[e * batch + b] : route[e];
            if (zero_skip && rw == 0.0f) continue;
            const uint8_t* g = PTR(gp, e);
            const float* gs = PTR(gsp, e);
            const uint8_t* u = PTR(up, e);
            const float* us = PTR(usp, e);
            if (!g || !gs || !u || !us) continue; /* activation stays 0 */
            mlp_gate_up(g, gs, u, us, x + b * hid, act + (e * batch + b) * inter, inter, hid, gsc);
        }
    }
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t h = 0; h < hid; ++h) {
            float routed = 0.0f;
            for (int64_t e = 0; e < experts; ++e) {
                const float rw = route_per_row ? route[e * batch + b] : route[e];
                if (zero_skip && rw == 0.0f) continue;
                const uint8_t* d = PTR(dp, e);
                const float* ds = PTR(dsp, e);
                if (!d || !ds) continue;
                const float ea = fp8_row_dot(d + h * inter, ds + (h / 128) * dsc,
                                             act + (e * batch + b) * inter, inter, dsc);
                routed += rw * ea;
            }
            out[b * hid + h] = routed;
        }
    }
    free(act);
    return 0;
}

/* fp8_linear.cpp:475-589 (fp8_e4m3_block_mlp_many_weighted_f32); the
 * AVX-512 twin fp8_linear_avx512.cpp:252-371 is bit-exact to it.
 * route_weights has one entry per expert. */
ORC_API int orc_fp8_mlp_many_weighted(const uint64_t* gp, const uint64_t* gsp, const uint64_t* up,
                                      const uint64_t* usp, const uint64_t* dp,
                                      const uint64_t* dsp, const float* x, const float* route,
                                      float* out, int64_t experts, int64_t batch, int64_t inter,
                                      int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !x || !route || !out) return -1;
    if (experts <= 0 || batch <= 0 || inter <= 0 || hid <= 0 || gsc <= 0 || dsc <= 0) return -2;
    return weighted_core(gp, gsp, up, usp, dp, dsp, x, route, 0, 0, out, experts, batch, inter,
                         hid, gsc, dsc);
}

/* fp8_linear.cpp:591-831 (fp8_e4m3_block_mlp_many_row_weighted_f32):
 * route_weights is [E, batch]; pairs with weight 0 are skipped. */
ORC_API int orc_fp8_mlp_many_row_weighted(const uint64_t* gp, const uint64_t* gsp,
                                          const uint64_t* up, const uint64_t* usp,
                                          const uint64_t* dp, const uint64_t* dsp, const float* x,
                                          const float* route, float* out, int64_t experts,
                                          int64_t batch, int64_t inter, int64_t hid, int64_t gsc,
                                          int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !x || !route || !out) return -1;
    if (experts <= 0 || batch <= 0 || inter <= 0 || hid <= 0 || gsc <= 0 || dsc <= 0) return -2;
    return weighted_core(gp, gsp, up, usp, dp, dsp, x, route, 1, 1, out, experts, batch, inter,
                         hid, gsc, dsc);
}

/* fp8_linear.cpp:833-980 (fp8_e4m3_block_mlp_many_pair_weighted_f32):
 * per-pair expert outputs, then out[b, h] = sum over pairs of row b, in pair
 * order, of weight * pair_output. */
ORC_API int orc_fp8_mlp_many_pair_weighted(const uint64_t* gp, const uint64_t* gsp,
                                           const uint64_t* up, const uint64_t* usp,
                                           const uint64_t* dp, const uint64_t* dsp, const float* x,
                                           const int64_t* pitem, const int64_t* prow,
                                           const float* pw, float* out, int64_t experts,
                                           int64_t pairs, int64_t batch, int64_t inter,
                                           int64_t hid, int64_t gsc, int64_t dsc) {
    if (!gp || !gsp || !up || !usp || !dp || !dsp || !x || !pitem || !prow || !pw || !out)
        return -1;
    if (experts <= 0 || pairs < 0 || batch <= 0 || inter <= 0 || hid <= 0 || gsc <= 0 || dsc <= 0)
        return -2;
    for (int64_t i = 0; i < batch * hid; ++i) out[i] = 0.0f;
    if (pairs == 0) return 0;
    for (int64_t p = 0; p < pairs; ++p) {
        if (pitem[p] < 0 || pitem[p] >= experts || prow[p] < 0 || prow[p] >= batch) return -4;
    }
    float* act = (float*)calloc((size_t)(pairs * inter), sizeof(float));
    float* pout = (float*)calloc((size_t)(pairs * hid), sizeof(float));
    if (!act || !pout) {
        free(act);
        free(pout);
        return -3;
    }
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < pairs; ++p) {
        const int64_t e = pitem[p];
        const uint8_t* g = PTR(gp, e);
        const float* gs = PTR(gsp, e);
        const uint8_t* u = PTR(up, e);
        const float* us = PTR(usp, e);
        if (!g || !gs || !u || !us) continue;
        mlp_gate_up(g, gs, u, us, x + prow[p] * hid, act + p * inter, inter, hid, gsc);
    }
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < pairs; ++p) {
        const int64_t e = pitem[p];
        const uint8_t* d = PTR(dp, e);
        const float* ds = PTR(dsp, e);
        if (!d || !ds) continue;
        for (int64_t h = 0; h < hid; ++h) {
            pout[p * hid + h] =
                fp8_row_dot(d + h * inter, ds + (h / 128) * dsc, act + p * inter, inter, dsc);
        }
    }
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t b = 0; b < batch; ++b) {
        for (int64_t h = 0; h < hid; ++h) {
            float acc = 0.0f;
            for (int64_t p = 0; p < pairs; ++p) {
                if (prow[p] == b) acc += pw[p] * pout[p * hid + h];
            }
            out[b * hid + h] = acc;
        }
    }
    free(act);
    free(pout);
    return 0;
}

/* ds_forward.cpp:337-367 / 866-873: out[i] = sum_e route[e] * outputs[e][i] */
ORC_API int orc_ds_moe_combine(const float* outputs, const float* route, int64_t selected,
                               int64_t batch, int64_t hid, float* out) {
    if (!outputs || !route || !out) return 1;
    if (selected <= 0 || batch <= 0 || hid <= 0) return 2;
    const int64_t width = batch * hid;
    for (int64_t i = 0; i < width; ++i) {
        float acc = 0.0f;
        for (int64_t e = 0; e < selected; ++e) acc += route[e] * outputs[e * width + i];
        out[i] = acc;
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* FP8 dequant (src/pcketlm/native/fp8_dequant.cpp, fp8_source.py:812-858)    */
/* ------------------------------------------------------------------------- */

/*
 * out_code: 0 = fp16 (fp8_dequant.cpp:119-164, F16C rounding),
 *           1 = bf16 (fp8_dequant.cpp:166-204),
 *           2 = fp32 (the torch branch of dequantize_fp8_block_scaled,
 *               fp8_source.py:852-858: decode, then one fp32 multiply).
 * In every case the fp32 product dec(byte) * scale is formed first.
 */
ORC_API int orc_fp8_dequant(const uint8_t* w, const float* s, void* out, int64_t rows,
                            int64_t cols, int64_t scale_cols, int out_code) {
    if (!w || !s || !out) return -1;
    if (rows <= 0 || cols <= 0 || scale_cols <= 0) return -2;
    if (scale_cols != (cols + 127) / 128) return -3;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) {
        const float* srow = s + (r / 128) * scale_cols;
        for (int64_t c = 0; c < cols; ++c) {
            const float v = g_lut_dequant[w[r * cols + c]] * srow[c / 128];
            if (out_code == 0) {
                ((uint16_t*)out)[r * cols + c] = orc_f32_to_f16_hw(v);
            } else if (out_code == 1) {
                ((uint16_t*)out)[r * cols + c] = orc_f32_to_bf16(v);
            } else {
                ((float*)out)[r * cols + c] = v;
            }
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Q4 (src/pcketlm/native/q4_dequant.cpp, model_import/q4_quantize.py)       */
/* ------------------------------------------------------------------------- */

static inline int q4_at(const uint8_t* packed, int64_t idx) {
    const uint8_t byte = packed[idx >> 1];
    const int nib = (idx & 1) ? (byte >> 4) : (byte & 0xF);
    return nib >= 8 ? nib - 16 : nib;
}

/*
 * q4_dequant.cpp:171-208: out[c*cs+i] = fp16(q * f32(scale[c])).  The product
 * is exact in fp32.  The reference converts with F16C inside its 16-value
 * AVX2 blocks (taken when the channel's first value index is even) and with
 * its software converter for the tail; the two differ only for NaN, and this
 * restatement reproduces which one each element gets.
 */
ORC_API void orc_q4_dequant_f16(const uint8_t* packed, const uint16_t* scales, uint16_t* out,
                                int64_t channels, int64_t cs) {
#pragma omp parallel for schedule(static)
    for (int64_t c = 0; c < channels; ++c) {
        const float sc = orc_f16_to_f32(scales[c]);
        const int64_t off = c * cs;
        int64_t vec_end = 0;
        if ((off & 1) == 0) vec_end = (cs / 16) * 16;
        for (int64_t i = 0; i < cs; ++i) {
            const float v = (float)q4_at(packed, off + i) * sc;
            out[off + i] = i < vec_end ? orc_f32_to_f16_hw(v) : orc_f32_to_f16_sw(v);
        }
    }
}

/*
 * One Q4 row dotted with an fp32 vector in the lane order of
 * q4_dot_row_avx2 (q4_dequant.cpp:314-355): two 8-lane accumulators over
 * 16-value steps, each term (q*scale)*x rounded as multiply then add; then
 * (acc0 + acc1) reduced as (l0+l4 + l1+l5) + (l2+l6 + l3+l7) the way
 * hsum256_ps (305-312) does; then the scalar tail.  The reference reads the
 * packed bytes at value_index/2, which is only right when value_index is
 * even; for odd row offsets this restatement indexes nibbles correctly
 * (the semantics of q4_dot_row_scalar, 288-303) instead of reproducing that
 * misread.
 */
static float q4_row_dot(const uint8_t* packed, const uint16_t* scales, int64_t row, int64_t n,
                        const float* x) {
    const float sc = orc_f16_to_f32(scales[row]);
    const int64_t off = row * n;
    float a0[8] = {0}, a1[8] = {0};
    int64_t i = 0;
    for (; i + 15 < n; i += 16) {
        for (int l = 0; l < 8; ++l) {
            const float q0 = (float)q4_at(packed, off + i + l) * sc;
            const float q1 = (float)q4_at(packed, off + i + 8 + l) * sc;
            a0[l] = a0[l] + q0 * x[i + l];
            a1[l] = a1[l] + q1 * x[i + 8 + l];
        }
    }
    float v[8];
    for (int l = 0; l < 8; ++l) v[l] = a0[l] + a1[l];
    /* low128 + high128, then two horizontal adds */
    const float t0 = v[0] + v[4], t1 = v[1] + v[5], t2 = v[2] + v[6], t3 = v[3] + v[7];
    float sum = (t0 + t1) + (t2 + t3);
    for (; i < n; ++i) sum += (float)q4_at(packed, off + i) * sc * x[i];
    return sum;
}

/* q4_dequant.cpp:357-476 (q4_moe_selected_forward_u16): one token, S
 * selected Q4 SwiGLU experts, route-weighted sum, fp16 output. */
ORC_API int orc_q4_moe_selected(const uint16_t* hidden, const uint8_t** gp, const uint16_t** gsp,
                                const uint8_t** upp, const uint16_t** usp, const uint8_t** dp,
                                const uint16_t** dsp, const float* route, uint16_t* out,
                                int64_t hid, int64_t inter, int64_t selected) {
    if (!hidden || !gp || !gsp || !upp || !usp || !dp || !dsp || !route || !out || hid <= 0 ||
        inter <= 0 || selected <= 0)
        return 1;
    for (int64_t e = 0; e < selected; ++e) {
        if (!gp[e] || !gsp[e] || !upp[e] || !usp[e] || !dp[e] || !dsp[e]) return 3;
    }
    float* hf = (float*)malloc((size_t)hid * sizeof(float));
    float* comb = (float*)calloc((size_t)hid, sizeof(float));
    float* gate = (float*)malloc((size_t)inter * sizeof(float));
    float* upv = (float*)malloc((size_t)inter * sizeof(float));
    float* act = (float*)malloc((size_t)inter * sizeof(float));
    if (!hf || !comb || !gate || !upv || !act) {
        free(hf); free(comb); free(gate); free(upv); free(act);
        return 2;
    }
    for (int64_t i = 0; i < hid; ++i) hf[i] = orc_f16_to_f32(hidden[i]);
    for (int64_t e = 0; e < selected; ++e) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < inter; ++r) {
            gate[r] = q4_row_dot(gp[e], gsp[e], r, hid, hf);
            upv[r] = q4_row_dot(upp[e], usp[e], r, hid, hf);
        }
        for (int64_t r = 0; r < inter; ++r) act[r] = silu_mul(gate[r], upv[r]);
        const float rw = route[e];
#pragma omp parallel for schedule(static)
        for (int64_t h = 0; h < hid; ++h) comb[h] += rw * q4_row_dot(dp[e], dsp[e], h, inter, act);
    }
    for (int64_t i = 0; i < hid; ++i) out[i] = orc_f32_to_f16_sw(comb[i]);
    free(hf); free(comb); free(gate); free(upv); free(act);
    return 0;
}

/* One Q4 matrix times one fp32 vector, y[r] = q4_row_dot(...): the per-row
 * dot of q4_moe_selected_forward_u16, exposed on its own. */
ORC_API int orc_q4_gemv(const uint8_t* packed, const uint16_t* scales, const float* x, float* y,
                        int64_t rows, int64_t cols) {
    if (!packed || !scales || !x || !y) return 1;
    if (rows <= 0 || cols <= 0) return 2;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; ++r) y[r] = q4_row_dot(packed, scales, r, cols, x);
    return 0;
}

/* ------------------------------------------------------------------------- */
/* row8 (src/pcketlm/native/fp16_packed_gemv.cpp)                            */
/* ------------------------------------------------------------------------- */

/* fp16_packed_gemv.cpp:52-77: packed[blk][col][lane] = W[8*blk+lane][col],
 * rows past the end zero. */
ORC_API int orc_pack_rows8(const uint16_t* w, uint16_t* packed, int64_t rows, int64_t cols) {
    if (!w || !packed) return 1;
    if (rows < 0 || cols < 0) return 2;
    const int64_t blocks = (rows + 7) / 8;
    for (int64_t blk = 0; blk < blocks; ++blk) {
        for (int64_t c = 0; c < cols; ++c) {
            for (int64_t l = 0; l < 8; ++l) {
                const int64_t r = blk * 8 + l;
                packed[(blk * cols + c) * 8 + l] = r < rows ? w[r * cols + c] : 0;
            }
        }
    }
    return 0;
}

/* fp16_packed_gemv.cpp:79-116: per 8-row block, acc[lane] = fma(x[k],
 * W[lane][k], acc[lane]) over k in order; hidden and weights share one
 * dtype (0 fp16, 1 bf16).  bias (may be NULL) is added after the dot, as in
 * fp16_kv_cache.cpp:117-148. */
ORC_API int orc_packed_gemv_rows8(const uint16_t* hidden, const uint16_t* packed, float* out,
                                  int64_t rows, int64_t cols, int dtype_code,
                                  const uint16_t* bias) {
    if (!hidden || !packed || !out) return 1;
    if (rows < 0 || cols < 0 || (dtype_code != 0 && dtype_code != 1)) return 2;
    const int64_t blocks = (rows + 7) / 8;
#pragma omp parallel for schedule(static)
    for (int64_t blk = 0; blk < blocks; ++blk) {
        float acc[8] = {0};
        const uint16_t* wb = packed + blk * cols * 8;
        for (int64_t c = 0; c < cols; ++c) {
            const float h = dtype_code ? bf16_to_f32(hidden[c]) : orc_f16_to_f32(hidden[c]);
            for (int l = 0; l < 8; ++l) {
                const uint16_t wv = wb[c * 8 + l];
                acc[l] = fmaf(h, dtype_code ? bf16_to_f32(wv) : orc_f16_to_f32(wv), acc[l]);
            }
        }
        for (int l = 0; l < 8; ++l) {
            const int64_t r = blk * 8 + l;
            if (r < rows) {
                float bv = 0.0f;
                if (bias) bv = dtype_code ? bf16_to_f32(bias[r]) : orc_f16_to_f32(bias[r]);
                out[r] = bias ? acc[l] + bv : acc[l];
            }
        }
    }
    return 0;
}

/*
 * fp32-activation row8 GEMV of the dense decode's o and down projections
 * (packed_rows8_gemv_float_hidden, src/pcketlm/native/fp16_kv_cache.cpp:146-174):
 * per 8-row block one fused multiply-add chain over the columns in order,
 * hidden[c] broadcast, no bias.
 */
ORC_API int orc_packed_gemv_rows8_f32_hidden(const float* hidden, const uint16_t* packed, float* out,
                                             int64_t rows, int64_t cols, int dtype_code) {
    if (!hidden || !packed || !out) return 1;
    if (rows < 0 || cols < 0 || (dtype_code != 0 && dtype_code != 1)) return 2;
    const int64_t blocks = (rows + 7) / 8;
#pragma omp parallel for schedule(static)
    for (int64_t blk = 0; blk < blocks; ++blk) {
        float acc[8] = {0};
        const uint16_t* wb = packed + blk * cols * 8;
        for (int64_t c = 0; c < cols; ++c) {
            const float h = hidden[c];
            for (int l = 0; l < 8; ++l) {
                const uint16_t wv = wb[c * 8 + l];
                acc[l] = fmaf(h, dtype_code ? bf16_to_f32(wv) : orc_f16_to_f32(wv), acc[l]);
            }
        }
        for (int l = 0; l < 8; ++l) {
            const int64_t r = blk * 8 + l;
            if (r < rows) out[r] = acc[l];
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------- */
/* Softmax top-k router (src/pcketlm/native/ds_forward.cpp:879-955)          */
/* ------------------------------------------------------------------------- */

ORC_API int orc_router_topk_u16(const uint16_t* hidden, const uint16_t* router, int64_t hid,
                                int64_t experts, int64_t k, int64_t dtype_code, int64_t* ids,
                                float* weights) {
    if (!hidden || !router || !ids || !weights) return 1;
    if (hid <= 0 || experts <= 0 || k <= 0 || k > experts) return 2;
    float* sc = (float*)malloc((size_t)experts * sizeof(float));
    int64_t* order = (int64_t*)malloc((size_t)experts * sizeof(int64_t));
    if (!sc || !order) {
        free(sc); free(order);
        return 2;
    }
    for (int64_t e = 0; e < experts; ++e) {
        float acc = 0.0f;
        for (int64_t c = 0; c < hid; ++c) {
            const float a = dtype_code == 1 ? bf16_to_f32(hidden[c]) : orc_f16_to_f32(hidden[c]);
            const uint16_t wv = router[e * hid + c];
            const float b = dtype_code == 1 ? bf16_to_f32(wv) : orc_f16_to_f32(wv);
            acc += a * b;
        }
        sc[e] = acc;
    }
    float mx = sc[0];
    for (int64_t e = 1; e < experts; ++e) mx = sc[e] > mx ? sc[e] : mx;
    double denom = 0.0;
    for (int64_t e = 0; e < experts; ++e) {
        sc[e] = expf(sc[e] - mx);
        denom += (double)sc[e];
    }
    if (denom <= 0.0) {
        free(sc); free(order);
        return 3;
    }
    for (int64_t e = 0; e < experts; ++e) sc[e] = (float)((double)sc[e] / denom);
    /* selection of the k best: larger score first, lower id on ties */
    for (int64_t e = 0; e < experts; ++e) order[e] = e;
    for (int64_t i = 0; i < k; ++i) {
        int64_t best = i;
        for (int64_t j = i + 1; j < experts; ++j) {
            const float sj = sc[order[j]], sb = sc[order[best]];
            if (sj > sb || (sj == sb && order[j] < order[best])) best = j;
        }
        const int64_t t = order[i];
        order[i] = order[best];
        order[best] = t;
    }
    double sel = 0.0;
    for (int64_t i = 0; i < k; ++i) sel += (double)sc[order[i]];
    if (sel <= 0.0) {
        free(sc); free(order);
        return 4;
    }
    for (int64_t i = 0; i < k; ++i) {
        ids[i] = order[i];
        weights[i] = (float)((double)sc[order[i]] / sel);
    }
    free(sc);
    free(order);
    return 0;
}

ORC_API int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
