/*
 * oracle.c -- CPU restatement of the reference's quantized mat-vec hot path.
 *
 * TEST INFRASTRUCTURE ONLY (see oracle.h): the checker for the HIP library,
 * never part of it. Built with -ffp-contract=off so that every `a*b + c` below
 * is two IEEE roundings; explicit fmaf() is used exactly where the compiled
 * reference fuses (its _mm256_fmadd_ps calls, and the scalar accumulations g++
 * contracts under its default -ffp-contract=fast).
 *
 * Reference paths cited as file:line relative to the reference repository.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

static const uint64_t k_iq2xs_grid[512] = {
#include "iq2xs_grid.inc"
};
static const uint64_t k_iq2s_grid[1024] = {
#include "iq2s_grid.inc"
};
static const uint32_t k_iq3s_grid[512] = {
#include "iq3s_grid.inc"
};
static const uint32_t k_iq3xxs_grid[256] = {
#include "iq3xxs_grid.inc"
};

uint32_t oc_type_size(int type) {
    /* src/cpp/core/GGUFLoader.cpp:64 (ggmlTypeSize); pinned by
     * unit_tests/DequantizeTest.cpp:570 (Q4_K=144, IQ3_XXS=98). */
    switch (type) {
        case OC_TYPE_Q8_0: return 34;
        case OC_TYPE_Q2_K: return 84;
        case OC_TYPE_Q3_K: return 110;
        case OC_TYPE_Q4_K: return 144;
        case OC_TYPE_Q5_K: return 176;
        case OC_TYPE_Q6_K: return 210;
        case OC_TYPE_IQ3_XXS: return 98;
        case OC_TYPE_IQ3_S: return 110;
        case OC_TYPE_IQ2_S: return 82;
        case OC_TYPE_IQ2_XS: return 74;
        case OC_TYPE_IQ4_XS: return 136;
        case OC_TYPE_IQ4_NL: return 18;
        case OC_TYPE_Q5_0: return 22;
        default: return 0;
    }
}

uint32_t oc_block_size(int type) {
    return type == OC_TYPE_Q8_0 || type == OC_TYPE_IQ4_NL || type == OC_TYPE_Q5_0 ? 32u : (oc_type_size(type) ? 256u : 0u);
}

/* ---- fp16 <-> fp32 -------------------------------------------------------- */

/* include/GGMLDequantize.hpp:89-141 (halfToFloat): exact IEEE widening with
 * subnormal normalisation. */
float oc_half_to_float(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) & 1u;
    uint32_t exp = (uint32_t)(h >> 10) & 0x1Fu;
    uint32_t mant = (uint32_t)h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign << 31;
        } else {
            int shift = 0;
            while ((mant & 0x400u) == 0) {
                mant <<= 1;
                ++shift;
            }
            mant &= 0x3FFu;
            bits = (sign << 31) | ((uint32_t)(113 - shift) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = (sign << 31) | (0xFFu << 23) | (mant << 13);
    } else {
        bits = (sign << 31) | ((exp + 112u) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* include/GGMLDequantize.hpp:61-87 (floatToHalf): TRUNCATES the mantissa (no
 * rounding), saturates exponents above 15 to inf, flushes below 2^-24. */
uint16_t oc_float_to_half(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    uint32_t sign = (b >> 31) & 1u;
    int32_t exp = (int32_t)((b >> 23) & 0xFFu) - 127;
    uint32_t mant = b & 0x7FFFFFu;
    uint32_t h;
    if (exp > 15) {
        h = (sign << 15) | (0x1Fu << 10) | (mant != 0 ? 0x200u : 0u);
    } else if (exp > -14) {
        h = (sign << 15) | ((uint32_t)(exp + 15) << 10) | (mant >> 13);
    } else if (exp > -24) {
        mant = (mant | 0x800000u) >> (14 - exp);
        h = (sign << 15) | (mant >> 13);
    } else {
        h = sign << 15;
    }
    return (uint16_t)h;
}

/* IEEE fp32 -> fp16, round to nearest even (used by this build's own
 * encoders; the reference's floatToHalf truncates and flushes every value below
 * 2^-13 to zero because its subnormal branch also takes exponent -14). */
static uint16_t f2h_rne(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | 0x7C00u | (ax > 0x7F800000u ? 0x200u : 0u));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) {
        float a;
        memcpy(&a, &ax, 4);
        return (uint16_t)(sign | (uint32_t)lrintf(a * 16777216.0f));
    }
    uint32_t h = ((((ax >> 23) - 112u)) << 10) | ((ax & 0x7FFFFFu) >> 13);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
}

static float h2f_at(const uint8_t *p) {
    uint16_t h;
    memcpy(&h, p, 2);
    return oc_half_to_float(h);
}

/* ---- activation quantizers ------------------------------------------------- */

/* Signed value of the FIRST element with the largest |x| (strict '>' scan). */
static float first_abs_max(const float *x, uint32_t n, float *amax_out) {
    float amax = 0.0f, maxv = 0.0f;
    for (uint32_t j = 0; j < n; ++j) {
        float ax = fabsf(x[j]);
        if (ax > amax) {
            amax = ax;
            maxv = x[j];
        }
    }
    *amax_out = amax;
    return maxv;
}

static int8_t quant_one(float iscale, float v) {
    long q = lrintf(iscale * v);
    return (int8_t)(q < 127 ? q : 127);
}

/* include/GGMLDequantize.hpp:2769-2807 (quantizeQ8K). */
void oc_quantize_q8k(const float *x, uint32_t n, int8_t *qs, float *d, int16_t *bsums) {
    for (uint32_t b = 0; b < n / 256; ++b) {
        const float *xb = x + (size_t)b * 256;
        int8_t *q = qs + (size_t)b * 256;
        float amax;
        float maxv = first_abs_max(xb, 256, &amax);
        if (amax == 0.0f) {
            d[b] = 0.0f;
            memset(q, 0, 256);
            memset(bsums + (size_t)b * 16, 0, 32);
            continue;
        }
        const float iscale = -127.0f / maxv;
        for (uint32_t j = 0; j < 256; ++j) q[j] = quant_one(iscale, xb[j]);
        for (uint32_t g = 0; g < 16; ++g) {
            int s = 0;
            for (uint32_t i = 0; i < 16; ++i) s += q[g * 16 + i];
            bsums[(size_t)b * 16 + g] = (int16_t)s;
        }
        d[b] = 1.0f / iscale;
    }
}

/* src/cpp/core/SIMDMatMulVecAVX2.cpp:4296-4326 (per-call Q8_0 activation
 * quantization inside matMulVecBatchQ8_0_Q8K_AVX2): same rule as quantizeQ8K
 * on 32-element blocks, fp32 scale, no bsums. */
void oc_quantize_q8_0_act(const float *x, uint32_t n, int8_t *qs, float *d) {
    for (uint32_t b = 0; b < n / 32; ++b) {
        const float *xb = x + (size_t)b * 32;
        int8_t *q = qs + (size_t)b * 32;
        float amax;
        float maxv = first_abs_max(xb, 32, &amax);
        if (amax == 0.0f) {
            d[b] = 0.0f;
            memset(q, 0, 32);
            continue;
        }
        const float iscale = -127.0f / maxv;
        for (uint32_t j = 0; j < 32; ++j) q[j] = quant_one(iscale, xb[j]);
        d[b] = 1.0f / iscale;
    }
}

/* ---- block decoders ---------------------------------------------------------- */

/* Q4_K 6-bit scale/min unpack: include/GGMLDequantize.hpp:444-453
 * (getScaleMin, ggml get_scale_min_k4 order). */
static void q4k_scale_min(const uint8_t *s, int j, uint8_t *sc, uint8_t *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (uint8_t)((s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4));
        *m = (uint8_t)((s[j + 4] >> 4) | ((s[j] >> 6) << 4));
    }
}

/* Q6_K raw 6-bit value (0..63) of element e of a block:
 * include/GGMLDequantize.hpp:503-527. */
/* Q5_K 5-bit value of weight l of sub-block g (include/GGMLDequantize.hpp:
 * 392-402; the byte layout of SIMDMatMulVecAVX2.cpp:3890-3903): qs at 48,
 * qh at 16. */
static int q5k_value(const uint8_t *blk, int g, int l) {
    const int c = g >> 1, h = g & 1;
    const uint8_t *qs = blk + 48, *qh = blk + 16;
    return ((qs[32 * c + l] >> (4 * h)) & 0xF) | (((qh[l] >> (2 * c + h)) & 1) << 4);
}

/* Q2_K (84 B: scales[16] at 0 -- low nibble scale, high nibble min per 16
 * weights --, qs[64] at 16, d at 80, dmin at 82): 2-bit value of element
 * e = 128h + 32t + l, bits 2t of qs[32h + l] (include/GGMLDequantize.hpp:
 * 550-590). */
static int q2k_value(const uint8_t *blk, int e) {
    const int h = e >> 7, t = (e >> 5) & 3, l = e & 31;
    return (blk[16 + 32 * h + l] >> (2 * t)) & 3;
}

/* Q3_K (110 B: hmask[32] at 0, qs[64] at 32, 12 scale bytes at 96, d at
 * 108): the 16 6-bit scales as unpacked by include/GGMLDequantize.hpp:612-630
 * (kmask1/kmask2 on three little-endian words), returned minus 32. */
static void q3k_scales(const uint8_t *blk, int sc[16]) {
    uint32_t aux[4];
    memcpy(aux, blk + 96, 12);
    const uint32_t km1 = 0x03030303u, km2 = 0x0f0f0f0fu, tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & km2) | (((tmp >> 4) & km1) << 4);
    aux[3] = ((aux[1] >> 4) & km2) | (((tmp >> 6) & km1) << 4);
    aux[0] = (aux[0] & km2) | (((tmp >> 0) & km1) << 4);
    aux[1] = (aux[1] & km2) | (((tmp >> 2) & km1) << 4);
    const int8_t *b = (const int8_t *)aux;
    for (int i = 0; i < 16; ++i) sc[i] = b[i] - 32;
}

/* Q3_K signed value (-4..3) of element e = 128n + 32j + l: 2 bits of
 * qs[32n + l] at 2j, minus 4 unless bit 4n+j of hmask[l] is set
 * (include/GGMLDequantize.hpp:632-648); its scale is sc[e/16]. */
static int q3k_value(const uint8_t *blk, int e) {
    const int n = e >> 7, j = (e >> 5) & 3, l = e & 31;
    const int q2 = (blk[32 + 32 * n + l] >> (2 * j)) & 3;
    return q2 - (((blk[l] >> (4 * n + j)) & 1) ? 0 : 4);
}

static int q6k_raw(const uint8_t *blk, int e) {
    const int half = e >> 7, r = e & 127, quad = r >> 5, l = r & 31;
    const uint8_t *ql = blk + 64 * half;
    const uint8_t *qh = blk + 128 + 32 * half;
    int lo = (quad & 1) ? ql[l + 32] : ql[l];
    lo = (quad & 2) ? (lo >> 4) : (lo & 0xF);
    int hi = (qh[l] >> (2 * quad)) & 3;
    return lo | (hi << 4);
}

/* IQ3_XXS signed integer weight (grid magnitude with sign) of element e:
 * include/GGMLDequantize.hpp:1135-1161 and the sign table :671-674
 * (ksigns_iq2xs[i] = i | parity(i) << 7). Returns the integer value; the
 * per-32 scale is (2*ls+1) (dot form :2064) or d*(0.5+ls)*0.5 (float form). */
static int iq3_signed(const uint8_t *blk, int e, int *ls_out) {
    const uint8_t *qs = blk + 2;
    const uint8_t *sas = blk + 2 + 64;
    const int ib32 = e >> 5, r = e & 31, l = r >> 3, j = r & 7;
    uint32_t aux;
    memcpy(&aux, sas + 4 * ib32, 4);
    const uint32_t idx7 = (aux >> (7 * l)) & 127u;
    const uint32_t signs = idx7 | ((uint32_t)__builtin_parity(idx7) << 7);
    const uint8_t gi = qs[8 * ib32 + 2 * l + (j >> 2)];
    const int mag = (int)((k_iq3xxs_grid[gi] >> (8 * (j & 3))) & 0xFFu);
    *ls_out = (int)(aux >> 28);
    return (signs >> j) & 1u ? -mag : mag;
}

/* IQ3_S (110 B: d, qs[64] at 2, qh[8] at 66, signs[32] at 74, scales[4] at
 * 106) signed integer weight of element e = 32ib + 8l + j: grid entry
 * qs[8ib + 2l + (j>=4)] with bit 8 from qh[ib] bit 2l (+1 for j>=4), byte
 * j&3, negated by bit j of signs[4ib + l]; per-32 scale 2*ls+1 with ls the
 * nibble ib&1 of scales[ib/2] (include/GGMLDequantize.hpp:1164-1212,
 * :2102-2145). */
static int iq3s_signed(const uint8_t *blk, int e, int *ls_out) {
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7, hi = j >> 2;
    const uint8_t *qs = blk + 2, *qh = blk + 66, *signs = blk + 74, *scales = blk + 106;
    const int idx = qs[8 * ib + 2 * l + hi] | ((qh[ib] << ((hi ? 7 : 8) - 2 * l)) & 256);
    const int mag = (int)((k_iq3s_grid[idx] >> (8 * (j & 3))) & 0xFFu);
    *ls_out = (scales[ib >> 1] >> (4 * (ib & 1))) & 15;
    return (signs[4 * ib + l] >> j) & 1 ? -mag : mag;
}

/* IQ2_S (82 B: d, qs[32] at 2, signs[32] at 34, qh[8] at 66, scales[8] at
 * 74) signed integer weight of element e = 32ib + 8l + j: byte j of codebook
 * entry qs[4ib + l] | ((qh[ib] << (8 - 2l)) & 0x300), negated by bit j of
 * signs[4ib + l]; scale nibble (l >= 2) of scales[ib]
 * (include/GGMLDequantize.hpp:1215-1242, :2028-2057). */
static int iq2s_signed(const uint8_t *blk, int e, int *ls_out) {
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    const uint8_t *qs = blk + 2, *signs = blk + 34, *qh = blk + 66, *scales = blk + 74;
    const int idx = qs[4 * ib + l] | ((qh[ib] << (8 - 2 * l)) & 0x300);
    const int mag = (int)((k_iq2s_grid[idx] >> (8 * j)) & 0xFFu);
    *ls_out = (scales[ib] >> (4 * (l >> 1))) & 15;
    return (signs[4 * ib + l] >> j) & 1 ? -mag : mag;
}

/* IQ4_XS (136 B: d at 0, scales_h (16 bits) at 2, scales_l[4] at 4, qs[128]
 * at 8): element 32ib + j is kvalues_iq4nl[nibble] with the low nibble of
 * qs[16ib + j] for j < 16 and the high nibble of qs[16ib + j - 16] above;
 * sub-block scale ls - 32 with ls = scales_l nibble ib | scales_h bits 2ib
 * << 4 (include/GGMLDequantize.hpp:1044-1080, table :55-57). */
static const int8_t k_kvalues_iq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                           1, 13, 25, 38, 53, 69, 89, 113};
static int iq4xs_value(const uint8_t *blk, int e) {
    const int ib = e >> 5, j = e & 31;
    const uint8_t q = blk[8 + 16 * ib + (j & 15)];
    return k_kvalues_iq4nl[j < 16 ? (q & 0xF) : (q >> 4)];
}
static int iq4xs_scale(const uint8_t *blk, int ib) {
    const int sh = blk[2] | (blk[3] << 8);
    return (((blk[4 + ib / 2] >> (4 * (ib % 2))) & 0xF) | (((sh >> (2 * ib)) & 3) << 4)) - 32;
}

/* IQ2_XS (74 B: d, qs16[32] at 2 -- bits 0-8 codebook index, bits 9-15 a
 * 7-bit sign index whose 8th sign is its parity --, scales[8] at 66) float
 * weight of element e = 32ib + 8l + j: dl * grid byte j * sign with dl =
 * (d * (0.5 + ls)) * 0.25, ls the nibble (l >= 2) of scales[ib]
 * (include/GGMLDequantize.hpp:1245-1271, the same arithmetic in the block
 * dot :1901-1927). */
static float iq2xs_weight(const uint8_t *blk, int e) {
    const int ib = e >> 5, l = (e >> 3) & 3, j = e & 7;
    uint16_t q;
    memcpy(&q, blk + 2 + 2 * (4 * ib + l), 2);
    const uint32_t si = q >> 9;
    const uint32_t signs = si | ((uint32_t)__builtin_parity(si) << 7);
    const int ls = (blk[66 + ib] >> (4 * (l >> 1))) & 15;
    const float dl = h2f_at(blk) * (0.5f + (float)ls) * 0.25f;
    const float g = (float)((k_iq2xs_grid[q & 511] >> (8 * j)) & 0xFFu);
    return dl * g * ((signs >> j) & 1 ? -1.0f : 1.0f);
}

/* Q5_0 (22 B: d, qh (32 bits) at 2, qs[16] at 6): element j < 16 is the low
 * nibble of qs[j] with bit j of qh as bit 4, element j + 16 the high nibble
 * with bit j + 16; value q - 16 (include/GGMLDequantize.hpp:163-185). */
static int q50_value(const uint8_t *blk, int e) {
    const uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) | ((uint32_t)blk[5] << 24);
    const uint8_t q = blk[6 + (e & 15)];
    return (int)(((e < 16 ? q & 0xF : q >> 4) | (((qh >> e) & 1u) << 4))) - 16;
}

int oc_dequant_row(int type, const uint8_t *w, uint32_t n, float *out) {
    const uint32_t bs = oc_block_size(type), ts = oc_type_size(type);
    if (bs == 0 || n % bs) return -1;
    for (uint32_t b = 0; b < n / bs; ++b) {
        const uint8_t *blk = w + (size_t)b * ts;
        float *y = out + (size_t)b * bs;
        if (type == OC_TYPE_Q5_0) {
            /* include/GGMLDequantize.hpp:163-185: y = d * (q5 - 16) */
            const float d = h2f_at(blk);
            for (int e = 0; e < 32; ++e) y[e] = d * (float)q50_value(blk, e);
        } else if (type == OC_TYPE_IQ4_NL) {
            /* include/GGMLDequantize.hpp:1304-1312: y[j] = d * kvalues[low
             * nibble of qs[j]], y[j+16] = d * kvalues[high nibble] */
            const float d = h2f_at(blk);
            for (int j = 0; j < 16; ++j) {
                y[j] = d * (float)k_kvalues_iq4nl[blk[2 + j] & 0xF];
                y[j + 16] = d * (float)k_kvalues_iq4nl[blk[2 + j] >> 4];
            }
        } else if (type == OC_TYPE_Q8_0) {
            /* include/GGMLDequantize.hpp:243-250 */
            const float d = h2f_at(blk);
            for (int i = 0; i < 32; ++i) y[i] = (float)(int8_t)blk[2 + i] * d;
        } else if (type == OC_TYPE_Q4_K) {
            /* include/GGMLDequantize.hpp:436-477 */
            const float d = h2f_at(blk), dmin = h2f_at(blk + 2);
            for (int g = 0; g < 8; ++g) {
                uint8_t sc, m;
                q4k_scale_min(blk + 4, g, &sc, &m);
                const float d1 = d * (float)sc, m1 = dmin * (float)m;
                const uint8_t *q = blk + 16 + 32 * (g >> 1);
                for (int l = 0; l < 32; ++l) {
                    const int v = (g & 1) ? (q[l] >> 4) : (q[l] & 0xF);
                    y[32 * g + l] = d1 * (float)v - m1;
                }
            }
        } else if (type == OC_TYPE_Q5_K) {
            /* include/GGMLDequantize.hpp:346-411: sub-block g = 2c + h of chunk
             * c: q5 = (qs[32c+l] >> 4h & 15) | (qh[l] bit 2c+h) << 4 (the same
             * 32 qh bytes serve every chunk), y = d1 * q5 - m1. */
            const float d = h2f_at(blk), dmin = h2f_at(blk + 2);
            for (int g = 0; g < 8; ++g) {
                uint8_t sc, m;
                q4k_scale_min(blk + 4, g, &sc, &m);
                const float d1 = d * (float)sc, m1 = dmin * (float)m;
                for (int l = 0; l < 32; ++l) y[32 * g + l] = d1 * (float)q5k_value(blk, g, l) - m1;
            }
        } else if (type == OC_TYPE_Q2_K) {
            /* include/GGMLDequantize.hpp:550-590: dl = d * sc, ml = dmin * m per
             * 16, y = dl * q - ml. */
            const float d = h2f_at(blk + 80), dmin = h2f_at(blk + 82);
            for (int e = 0; e < 256; ++e) {
                const uint8_t sc = blk[e >> 4];
                const float dl = d * (float)(sc & 0xF), ml = dmin * (float)(sc >> 4);
                y[e] = dl * (float)q2k_value(blk, e) - ml;
            }
        } else if (type == OC_TYPE_Q3_K) {
            /* include/GGMLDequantize.hpp:612-648: dl = d * (sc - 32) per 16,
             * y = dl * q with q = q2 - (hmask bit ? 0 : 4). */
            const float d = h2f_at(blk + 108);
            int sc[16];
            q3k_scales(blk, sc);
            for (int e = 0; e < 256; ++e) y[e] = (d * (float)sc[e >> 4]) * (float)q3k_value(blk, e);
        } else if (type == OC_TYPE_Q6_K) {
            /* include/GGMLDequantize.hpp:503-527: y = d * sc * q, evaluated
             * left to right as (d*sc)*q with q = raw-32. */
            const float d = h2f_at(blk + 208);
            const int8_t *sc = (const int8_t *)(blk + 192);
            for (int e = 0; e < 256; ++e) {
                const int q = q6k_raw(blk, e) - 32;
                y[e] = d * (float)sc[e >> 4] * (float)q;
            }
        } else if (type == OC_TYPE_IQ2_XS) {
            for (int e = 0; e < 256; ++e) y[e] = iq2xs_weight(blk, e);
        } else if (type == OC_TYPE_IQ4_XS) {
            /* dl = d * (ls - 32) per 32, y = dl * kvalues (:1044-1080) */
            const float d = h2f_at(blk);
            for (int e = 0; e < 256; ++e) y[e] = d * (float)iq4xs_scale(blk, e >> 5) * (float)iq4xs_value(blk, e);
        } else if (type == OC_TYPE_IQ2_S) {
            /* include/GGMLDequantize.hpp:1215-1242: db = (d * (0.5 + ls)) *
             * 0.25, y = (db * grid) * sign. */
            const float d = h2f_at(blk);
            for (int e = 0; e < 256; ++e) {
                int ls;
                const int v = iq2s_signed(blk, e, &ls);
                const float db = d * (0.5f + (float)ls) * 0.25f;
                const float mag = (float)(v < 0 ? -v : v);
                y[e] = db * mag * (v < 0 ? -1.0f : 1.0f);
            }
        } else if (type == OC_TYPE_IQ3_S) {
            /* include/GGMLDequantize.hpp:1164-1212: y = (db * grid) * sign,
             * db = d * (1 + 2*ls). */
            const float d = h2f_at(blk);
            for (int e = 0; e < 256; ++e) {
                int ls;
                const int v = iq3s_signed(blk, e, &ls);
                const float db = d * (1.0f + 2.0f * (float)ls);
                const float mag = (float)(v < 0 ? -v : v);
                y[e] = db * mag * (v < 0 ? -1.0f : 1.0f);
            }
        } else {
            /* include/GGMLDequantize.hpp:1135-1161:
             * y = db * grid * sign, db = d * (0.5 + ls) * 0.5. */
            const float d = h2f_at(blk);
            for (int e = 0; e < 256; ++e) {
                int ls;
                const int v = iq3_signed(blk, e, &ls);
                const float db = d * (0.5f + (float)ls) * 0.5f;
                const float mag = (float)(v < 0 ? -v : v);
                y[e] = db * mag * (v < 0 ? -1.0f : 1.0f);
            }
        }
    }
    return 0;
}

/* ---- per-block integer dots --------------------------------------------------- */

/* Q4_K sub-block integer sums s32q[i] = sum_32 nibble * q8 (the maddubs/madd
 * chain of src/cpp/core/SIMDMatMulVecAVX2.cpp:3690-3702). */
static void q4k_subsums(const uint8_t *blk, const int8_t *xq, int32_t s[8]) {
    const uint8_t *qs = blk + 16;
    for (int i = 0; i < 8; ++i) {
        int32_t acc = 0;
        const uint8_t *q = qs + 32 * (i >> 1);
        for (int l = 0; l < 32; ++l) {
            const int v = (i & 1) ? (q[l] >> 4) : (q[l] & 0xF);
            acc += v * xq[32 * i + l];
        }
        s[i] = acc;
    }
}

/* Q5_K sub-block integer sums s32q[i] = sum_32 q5 * q8 (the maddubs/madd
 * chain of src/cpp/core/SIMDMatMulVecAVX2.cpp:3924-3933). */
static void q5k_subsums(const uint8_t *blk, const int8_t *xq, int32_t s[8]) {
    for (int i = 0; i < 8; ++i) {
        int32_t acc = 0;
        for (int l = 0; l < 32; ++l) acc += q5k_value(blk, i, l) * xq[32 * i + l];
        s[i] = acc;
    }
}

/* Q6_K block integer sum_g sc[g] * sum_16 (raw - 32) * q8: the exact integer
 * that matMulVecBatchQ6K_Q8K_AVX2's blockDot scales by d*d8
 * (src/cpp/core/SIMDMatMulVecAVX2.cpp:4636-4667, -32 folded via bsums). */
static int32_t q6k_isum(const uint8_t *blk, const int8_t *xq) {
    const int8_t *sc = (const int8_t *)(blk + 192);
    int32_t tot = 0;
    for (int g = 0; g < 16; ++g) {
        int32_t s = 0;
        for (int i = 0; i < 16; ++i) s += (q6k_raw(blk, 16 * g + i) - 32) * xq[16 * g + i];
        tot += (int32_t)sc[g] * s;
    }
    return tot;
}

/* Q2_K block integers: out[0] = sum_g sc_g * sum_16 q*q8 (main), out[1] =
 * sum_g m_g * bsum_g (min), the two exact sums of the compact kernel's
 * blockDot (src/cpp/core/SIMDMatMulVecAVX2.cpp:4995-5020). */
static void q2k_isums(const uint8_t *blk, const int8_t *xq, const int16_t *bsums, int32_t out[2]) {
    int32_t mainI = 0, minI = 0;
    for (int g = 0; g < 16; ++g) {
        int32_t s = 0;
        for (int i = 0; i < 16; ++i) s += q2k_value(blk, 16 * g + i) * xq[16 * g + i];
        mainI += (blk[g] & 0xF) * s;
        minI += (blk[g] >> 4) * bsums[g];
    }
    out[0] = mainI;
    out[1] = minI;
}

/* Q3_K block integer sum_g (sc[g]-32) * sum_16 q * q8 with q in -4..3: the
 * exact integer behind matMulVecBatchQ3K_Q8K_AVX2's blockDot
 * (src/cpp/core/SIMDMatMulVecAVX2.cpp:3480-3520: w' = q + 4 in the dots and
 * -4 * sum (sc-32) * bsum folded back). */
static int32_t q3k_isum(const uint8_t *blk, const int8_t *xq) {
    int sc[16];
    q3k_scales(blk, sc);
    int32_t tot = 0;
    for (int g = 0; g < 16; ++g) {
        int32_t s = 0;
        for (int i = 0; i < 16; ++i) s += q3k_value(blk, 16 * g + i) * xq[16 * g + i];
        tot += sc[g] * s;
    }
    return tot;
}

/* IQ3_XXS block integer bsum = sum_ib32 (2*ls+1) * sum_32 grid*sign*q8:
 * include/GGMLDequantize.hpp:2064-2097 (dotProductIQ3_XXS_Q8K). */
static int32_t iq3_isum(const uint8_t *blk, const int8_t *xq) {
    int32_t bsum = 0;
    for (int ib = 0; ib < 8; ++ib) {
        int32_t sumi = 0;
        int ls = 0;
        for (int r = 0; r < 32; ++r) sumi += iq3_signed(blk, 32 * ib + r, &ls) * xq[32 * ib + r];
        bsum += sumi * (2 * ls + 1);
    }
    return bsum;
}

/* IQ3_S block integer bsum = sum_ib32 (2*ls+1) * sum_32 grid*sign*q8:
 * include/GGMLDequantize.hpp:2102-2145 (dotProductIQ3_S_Q8K). */
static int32_t iq3s_isum(const uint8_t *blk, const int8_t *xq) {
    int32_t bsum = 0;
    for (int ib = 0; ib < 8; ++ib) {
        int32_t sumi = 0;
        int ls = 0;
        for (int r = 0; r < 32; ++r) sumi += iq3s_signed(blk, 32 * ib + r, &ls) * xq[32 * ib + r];
        bsum += sumi * (2 * ls + 1);
    }
    return bsum;
}

/* IQ2_S block integer bsum = sum_ib32 (1+2*ls1) * sum_16 + (1+2*ls2) * sum_16
 * of grid*sign*q8: include/GGMLDequantize.hpp:2028-2057 (dotProductIQ2_S_Q8K). */
static int32_t iq2s_isum(const uint8_t *blk, const int8_t *xq) {
    int32_t bsum = 0;
    for (int ib = 0; ib < 8; ++ib)
        for (int h = 0; h < 2; ++h) {
            int32_t sumi = 0;
            int ls = 0;
            for (int r = 0; r < 16; ++r) sumi += iq2s_signed(blk, 32 * ib + 16 * h + r, &ls) * xq[32 * ib + 16 * h + r];
            bsum += (1 + 2 * ls) * sumi;
        }
    return bsum;
}

/* IQ4_XS per-32 integer sums s[ib] = sum_32 kvalues*q8, the exact int32 of
 * the reference's maddubs/madd reduction (|w|, |x| <= 127: no int16
 * saturation; SIMDMatMulVecAVX2.cpp:4090-4101). */
static void iq4xs_subsums(const uint8_t *blk, const int8_t *xq, int32_t s[8]) {
    for (int ib = 0; ib < 8; ++ib) {
        int32_t t = 0;
        for (int j = 0; j < 32; ++j) t += iq4xs_value(blk, 32 * ib + j) * xq[32 * ib + j];
        s[ib] = t;
    }
}

/* IQ4_XS block integer sum_ib (ls_ib - 32) * s[ib] (the GPU test hook's value). */
static int32_t iq4xs_isum(const uint8_t *blk, const int8_t *xq) {
    int32_t s[8], tot = 0;
    iq4xs_subsums(blk, xq, s);
    for (int ib = 0; ib < 8; ++ib) tot += iq4xs_scale(blk, ib) * s[ib];
    return tot;
}

/* Q8_0 block sum_32 w*q8, the true integer product (the reference kernel's
 * sum, src/cpp/core/SIMDMatMulVecAVX2.cpp:4346-4356, equals it whenever no
 * weight byte is -128). */
static int32_t q80_isum(const uint8_t *blk, const int8_t *xq) {
    int32_t s = 0;
    for (int i = 0; i < 32; ++i) s += (int8_t)blk[2 + i] * xq[i];
    return s;
}

typedef struct {
    int8_t *qs;
    float *d;
    int16_t *bsums;
} act_t;

static int quantize_acts(int type, const float *X, uint32_t S, uint32_t cols, act_t *a) {
    a->qs = (int8_t *)malloc((size_t)S * cols);
    a->d = (float *)malloc(sizeof(float) * ((size_t)S * cols / 32 + 1));
    a->bsums = (int16_t *)malloc(sizeof(int16_t) * ((size_t)S * cols / 16 + 1));
    if (!a->qs || !a->d || !a->bsums) return -1;
    for (uint32_t s = 0; s < S; ++s) {
        if (type == OC_TYPE_Q8_0)
            oc_quantize_q8_0_act(X + (size_t)s * cols, cols, a->qs + (size_t)s * cols,
                                 a->d + (size_t)s * (cols / 32));
        else
            oc_quantize_q8k(X + (size_t)s * cols, cols, a->qs + (size_t)s * cols,
                            a->d + (size_t)s * (cols / 256), a->bsums + (size_t)s * (cols / 16));
    }
    return 0;
}

static void free_acts(act_t *a) {
    free(a->qs);
    free(a->d);
    free(a->bsums);
}

static int shape_ok(int type, uint32_t cols) {
    const uint32_t bs = oc_block_size(type);
    return bs != 0 && cols != 0 && cols % bs == 0;
}

int oc_block_isums(int type, const uint8_t *W, const float *X, uint32_t S,
                   uint32_t rows, uint32_t cols, int32_t *isums) {
    if (!shape_ok(type, cols) || type == OC_TYPE_IQ2_XS || type == OC_TYPE_IQ4_NL || type == OC_TYPE_Q5_0) return -1;  /* float paths: no integer sums */
    act_t a;
    if (quantize_acts(type, X, S, cols, &a)) return -1;
    const uint32_t bs = oc_block_size(type), ts = oc_type_size(type), nb = cols / bs;
    const uint32_t k = (type == OC_TYPE_Q4_K || type == OC_TYPE_Q5_K) ? 8 : type == OC_TYPE_Q2_K ? 2 : 1;
    for (uint32_t s = 0; s < S; ++s)
        for (uint32_t r = 0; r < rows; ++r)
            for (uint32_t b = 0; b < nb; ++b) {
                const uint8_t *blk = W + ((size_t)r * nb + b) * ts;
                const int8_t *xq = a.qs + (size_t)s * cols + (size_t)b * bs;
                int32_t *o = isums + (((size_t)s * rows + r) * nb + b) * k;
                switch (type) {
                    case OC_TYPE_Q4_K: q4k_subsums(blk, xq, o); break;
                    case OC_TYPE_Q5_K: q5k_subsums(blk, xq, o); break;
                    case OC_TYPE_Q3_K: o[0] = q3k_isum(blk, xq); break;
                    case OC_TYPE_Q2_K:
                        q2k_isums(blk, xq, a.bsums + (size_t)s * (cols / 16) + (size_t)b * 16, o);
                        break;
                    case OC_TYPE_Q6_K: o[0] = q6k_isum(blk, xq); break;
                    case OC_TYPE_IQ3_XXS: o[0] = iq3_isum(blk, xq); break;
                    case OC_TYPE_IQ3_S: o[0] = iq3s_isum(blk, xq); break;
                    case OC_TYPE_IQ2_S: o[0] = iq2s_isum(blk, xq); break;
                    case OC_TYPE_IQ4_XS: o[0] = iq4xs_isum(blk, xq); break;
                    default: o[0] = q80_isum(blk, xq); break;
                }
            }
    free_acts(&a);
    return 0;
}

/* ---- row kernels with the reference float evaluation order ---------------- */

/* src/cpp/core/SIMDMatMulVecAVX2.cpp:3649-3715 (seqLen==1 row path; the batch
 * path :3719-3830 has the same per-block math and block-order accumulation).
 * The three accumulations `x += a*b` are fused multiply-adds: g++ compiles C++
 * with -ffp-contract=fast, and with -mfma it contracts them (verified by the
 * bit-exact golden vectors from the compiled reference). */
static float row_q4k(const uint8_t *rp, uint32_t nb, const act_t *a, size_t qoff, size_t doff,
                     size_t boff) {
    float sum = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = rp + (size_t)b * 144;
        const float d = h2f_at(blk), dmin = h2f_at(blk + 2);
        int32_t s32[8];
        q4k_subsums(blk, a->qs + qoff + (size_t)b * 256, s32);
        const int16_t *bsums = a->bsums + boff + (size_t)b * 16;
        float mainS = 0.0f, minS = 0.0f;
        for (int i = 0; i < 8; ++i) {
            uint8_t sc, m;
            q4k_scale_min(blk + 4, i, &sc, &m);
            const float ds = d * (float)sc;
            const float mn = dmin * (float)m;
            mainS = fmaf(ds, (float)s32[i], mainS);
            minS = fmaf(mn, (float)(bsums[2 * i] + bsums[2 * i + 1]), minS);
        }
        sum = fmaf(a->d[doff + b], mainS - minS, sum);
    }
    return sum;
}

/* src/cpp/core/SIMDMatMulVecAVX2.cpp:3842-3955 (matMulVecBatchQ5K_Q8K_AVX2):
 * per block ds = d*sc, mn = dmin*m; mainS += ds*s32, minS += mn*pairsum,
 * acc += d8*(mainS - minS), accumulated over blocks in order; the three
 * accumulations contract to fused multiply-adds as in the Q4_K kernel. */
static float row_q5k(const uint8_t *rp, uint32_t nb, const act_t *a, size_t qoff, size_t doff,
                     size_t boff) {
    float sum = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = rp + (size_t)b * 176;
        const float d = h2f_at(blk), dmin = h2f_at(blk + 2);
        int32_t s32[8];
        q5k_subsums(blk, a->qs + qoff + (size_t)b * 256, s32);
        const int16_t *bsums = a->bsums + boff + (size_t)b * 16;
        float mainS = 0.0f, minS = 0.0f;
        for (int i = 0; i < 8; ++i) {
            uint8_t sc, m;
            q4k_scale_min(blk + 4, i, &sc, &m);
            mainS = fmaf(d * (float)sc, (float)s32[i], mainS);
        }
        for (int i = 0; i < 8; ++i) {
            uint8_t sc, m;
            q4k_scale_min(blk + 4, i, &sc, &m);
            minS = fmaf(dmin * (float)m, (float)(bsums[2 * i] + bsums[2 * i + 1]), minS);
        }
        sum = fmaf(a->d[doff + b], mainS - minS, sum);
    }
    return sum;
}

/* AVX2 horizontal float sum used by the reference store paths:
 * lo+hi, then two _mm_hadd_ps (SIMDMatMulVecAVX2.cpp:4353-4356, 4729-4735). */
static float hsum8(const float v[8]) {
    const float s0 = v[0] + v[4], s1 = v[1] + v[5], s2 = v[2] + v[6], s3 = v[3] + v[7];
    return (s0 + s1) + (s2 + s3);
}

/* Product w*x as the reference Q8_0 kernel forms it: |x| * sign(w, x) through
 * _mm256_sign_epi8 / _mm256_maddubs_epi16 (SIMDMatMulVecAVX2.cpp:4348-4351).
 * sign_epi8 cannot negate -128, so w = -128 with x < 0 contributes -128*|x|
 * instead of +128*|x|. Encoders never emit -128 (they clamp to +-127); the
 * true product is what oc_block_isums reports. */
static int32_t q80_maddubs_product(int8_t w, int8_t x) {
    if (x == 0) return 0;
    const int ax = x < 0 ? -x : x;
    const int8_t ws = x < 0 ? (int8_t)(uint8_t)(0u - (uint8_t)w) : w;
    return ax * ws;
}

/* src/cpp/core/SIMDMatMulVecAVX2.cpp:4239-4383 (matMulVecBatchQ8_0_Q8K_AVX2):
 * per block, 8 int32 lanes of 4-byte partial dots scaled by d*d8 in fp32,
 * horizontally summed, added to a scalar accumulator; blocks with d8 == 0 are
 * skipped. */
static float row_q80(const uint8_t *rp, uint32_t nb, const act_t *a, size_t qoff, size_t doff) {
    float acc = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = rp + (size_t)b * 34;
        const float d = h2f_at(blk);
        const float d8 = a->d[doff + b];
        if (d8 == 0.0f) continue;
        const int8_t *xq = a->qs + qoff + (size_t)b * 32;
        const float dd8 = d * d8;
        float v[8];
        for (int j = 0; j < 8; ++j) {
            int32_t s = 0;
            for (int k = 0; k < 4; ++k) s += q80_maddubs_product((int8_t)blk[2 + 4 * j + k], xq[4 * j + k]);
            v[j] = dd8 * (float)s;
        }
        acc += hsum8(v);
    }
    return acc;
}

/* src/cpp/core/SIMDMatMulVecAVX2.cpp:4410-4743 (matMulVecBatchQ6K_Q8K_AVX2):
 * blockDot keeps 8 float lanes: lane j starts at (-32*d*d8) * (sc[2j]*bsum[2j] +
 * sc[2j+1]*bsum[2j+1]); each 128-element chunk adds fma(d*d8, sumi_j, acc_j),
 * where sumi_j = sum over the chunk's 4 sub-blocks of the scale for lane j's
 * 16-half times the 4-byte partial dot of bytes 4j..4j+3. Blocks are summed
 * lane-wise and the 8 lanes are horizontally summed once per row. */
static float row_q6k(const uint8_t *rp, uint32_t nb, const act_t *a, size_t qoff, size_t doff,
                     size_t boff) {
    float racc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = rp + (size_t)b * 210;
        const float d = h2f_at(blk + 208);
        const int8_t *sc = (const int8_t *)(blk + 192);
        const float d8 = a->d[doff + b];
        const int8_t *xq = a->qs + qoff + (size_t)b * 256;
        const int16_t *bsums = a->bsums + boff + (size_t)b * 16;
        const float c0 = -32.0f * d * d8;
        const float dd8 = d * d8;
        float acc[8];
        for (int j = 0; j < 8; ++j) {
            const int32_t bp = (int32_t)sc[2 * j] * bsums[2 * j] + (int32_t)sc[2 * j + 1] * bsums[2 * j + 1];
            acc[j] = c0 * (float)bp;
        }
        for (int chunk = 0; chunk < 2; ++chunk) {
            int32_t sumi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int sub = 0; sub < 4; ++sub) {
                const int idx = chunk * 4 + sub;
                for (int j = 0; j < 8; ++j) {
                    int32_t p = 0;
                    for (int k = 0; k < 4; ++k) {
                        const int e = 32 * idx + 4 * j + k;
                        p += q6k_raw(blk, e) * xq[e];
                    }
                    sumi[j] += (int32_t)sc[2 * idx + (j >= 4)] * p;
                }
            }
            for (int j = 0; j < 8; ++j) acc[j] = fmaf(dd8, (float)sumi[j], acc[j]);
        }
        for (int j = 0; j < 8; ++j) racc[j] = racc[j] + acc[j];
    }
    return hsum8(racc);
}

/* src/cpp/core/SIMDMatMulVecAVX2.cpp:4757-5050
 * (matMulVecBatchQ2K_Compact_Q8K_AVX2): 8 lanes per block. Lane j: min term
 * (-dmin*d8) * (m[2j]*bs[2j] + m[2j+1]*bs[2j+1]) (one rounding: an fma with
 * 0); acc from 0 gets fma(dq*d8, sumi_j) per chunk, sumi_j summing over the
 * chunk's 4 sub-blocks idx sc[2idx + (j>=4)] * sum_4 q*q8 over elements
 * 32idx + 4j..; the block adds acc + minTerm lane-wise into the row
 * accumulator; the 8 lanes reduce as ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)). */
static float row_q2k(const uint8_t *rp, uint32_t nb, const act_t *a, size_t qoff, size_t doff,
                     size_t boff) {
    float racc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = rp + (size_t)b * 84;
        const float dq = h2f_at(blk + 80), ndmin = -h2f_at(blk + 82);
        const float d8 = a->d[doff + b];
        const int8_t *xq = a->qs + qoff + (size_t)b * 256;
        const int16_t *bsums = a->bsums + boff + (size_t)b * 16;
        const float cm = ndmin * d8, dd8 = dq * d8;
        float minT[8], acc[8];
        for (int j = 0; j < 8; ++j) {
            const int32_t prod = (int32_t)(blk[2 * j] >> 4) * bsums[2 * j] + (int32_t)(blk[2 * j + 1] >> 4) * bsums[2 * j + 1];
            minT[j] = cm * (float)prod;
            acc[j] = 0.0f;
        }
        for (int chunk = 0; chunk < 2; ++chunk) {
            int32_t sumi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int sub = 0; sub < 4; ++sub) {
                const int idx = chunk * 4 + sub;
                for (int j = 0; j < 8; ++j) {
                    int32_t p = 0;
                    for (int k = 0; k < 4; ++k) {
                        const int e = 32 * idx + 4 * j + k;
                        p += q2k_value(blk, e) * xq[e];
                    }
                    sumi[j] += (int32_t)(blk[2 * idx + (j >= 4)] & 0xF) * p;
                }
            }
            for (int j = 0; j < 8; ++j) acc[j] = fmaf(dd8, (float)sumi[j], acc[j]);
        }
        for (int j = 0; j < 8; ++j) racc[j] = racc[j] + (acc[j] + minT[j]);
    }
    return hsum8(racc);
}

/* src/cpp/core/SIMDMatMulVecAVX2.cpp:3220-3560 (matMulVecBatchQ3K_Q8K_AVX2):
 * the same 8-lane structure as the Q6_K kernel. Per block, lane j starts at
 * c0 * (s[2j]*bs[2j] + s[2j+1]*bs[2j+1]) with c0 = (-4*dq)*d8 and s = sc-32;
 * per chunk, lane j adds fma(dq*d8, sumi_j) where sumi_j sums, over the 4
 * sub-blocks idx of the chunk, s[2idx + (j>=4)] * sum_4 w'*q8 over elements
 * 32idx + 4j.. (w' = q + 4, 0..7); lanes add into the row accumulator, then
 * the 8 lanes are reduced as ((a0+a4)+(a1+a5)) + ((a2+a6)+(a3+a7)). */
static float row_q3k(const uint8_t *rp, uint32_t nb, const act_t *a, size_t qoff, size_t doff,
                     size_t boff) {
    float racc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = rp + (size_t)b * 110;
        const float dq = h2f_at(blk + 108);
        int sc[16];
        q3k_scales(blk, sc);
        const float d8 = a->d[doff + b];
        const int8_t *xq = a->qs + qoff + (size_t)b * 256;
        const int16_t *bsums = a->bsums + boff + (size_t)b * 16;
        const float c0 = -4.0f * dq * d8;
        const float dd8 = dq * d8;
        float acc[8];
        for (int j = 0; j < 8; ++j) {
            const int32_t bp = (int32_t)sc[2 * j] * bsums[2 * j] + (int32_t)sc[2 * j + 1] * bsums[2 * j + 1];
            acc[j] = c0 * (float)bp;
        }
        for (int chunk = 0; chunk < 2; ++chunk) {
            int32_t sumi[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            for (int sub = 0; sub < 4; ++sub) {
                const int idx = chunk * 4 + sub;
                for (int j = 0; j < 8; ++j) {
                    int32_t p = 0;
                    for (int k = 0; k < 4; ++k) {
                        const int e = 32 * idx + 4 * j + k;
                        p += (q3k_value(blk, e) + 4) * xq[e];
                    }
                    sumi[j] += (int32_t)sc[2 * idx + (j >= 4)] * p;
                }
            }
            for (int j = 0; j < 8; ++j) acc[j] = fmaf(dd8, (float)sumi[j], acc[j]);
        }
        for (int j = 0; j < 8; ++j) racc[j] = racc[j] + acc[j];
    }
    return hsum8(racc);
}

/* include/GGMLDequantize.hpp:2231-2269 (matMulVecBatchQ8K) with the IQ3_XXS
 * block dot :2064-2097 and the row scale 0.25 (:2148-2159). */
static float row_iq3(const uint8_t *rp, uint32_t nb, const act_t *a, size_t qoff, size_t doff) {
    float sumf = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = rp + (size_t)b * 98;
        const float d = h2f_at(blk) * a->d[doff + b];
        const int32_t bsum = iq3_isum(blk, a->qs + qoff + (size_t)b * 256);
        sumf += d * (float)bsum;
    }
    return 0.25f * sumf;
}

/* include/GGMLDequantize.hpp:2231-2269 (matMulVecBatchQ8K) with the IQ3_S
 * block dot :2102-2145 (d = d_w * d8, d * bsum) and the row scale 1
 * (:2148-2159). */
static float row_iq3s(const uint8_t *rp, uint32_t nb, const act_t *a, size_t qoff, size_t doff) {
    float sumf = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = rp + (size_t)b * 110;
        const float d = h2f_at(blk) * a->d[doff + b];
        const int32_t bsum = iq3s_isum(blk, a->qs + qoff + (size_t)b * 256);
        sumf += d * (float)bsum;
    }
    return 1.0f * sumf;
}

/* The IQ2_S row: the same loop with the block dot :2028-2057 and the row
 * scale 0.125 (:2148-2159). */
static float row_iq2s(const uint8_t *rp, uint32_t nb, const act_t *a, size_t qoff, size_t doff) {
    float sumf = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = rp + (size_t)b * 82;
        const float d = h2f_at(blk) * a->d[doff + b];
        const int32_t bsum = iq2s_isum(blk, a->qs + qoff + (size_t)b * 256);
        sumf += d * (float)bsum;
    }
    return 0.125f * sumf;
}

/* src/cpp/core/SIMDMatMulVecAVX2.cpp:3988-4119 (matMulVecBatchIQ4XS_Q8K_AVX2):
 * per block dl[ib] = d * (float)(ls - 32); mainS from 0 accumulates dl[ib] *
 * (float)s[ib] over ib; acc += d8 * mainS over blocks in order. Both
 * accumulations contract to fused multiply-adds (g++ -ffp-contract=fast with
 * -mfma, as the Q4_K kernel). */
static float row_iq4xs(const uint8_t *rp, uint32_t nb, const act_t *a, size_t qoff, size_t doff) {
    float acc = 0.0f;
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t *blk = rp + (size_t)b * 136;
        const float d = h2f_at(blk);
        int32_t s[8];
        iq4xs_subsums(blk, a->qs + qoff + (size_t)b * 256, s);
        float mainS = 0.0f;
        for (int ib = 0; ib < 8; ++ib) mainS = fmaf(d * (float)iq4xs_scale(blk, ib), (float)s[ib], mainS);
        acc = fmaf(a->d[doff + b], mainS, acc);
    }
    return acc;
}

/* IQ2_XS: no activation quantization. Block dot = float(sum_e double(x_e) *
 * double(w_e)) (dotProductIQ2_XS, include/GGMLDequantize.hpp:1901-1927); row =
 * float(sum_b double(block dot)) (matMulVecFused, :2449-2461). The double
 * products of two floats are exact, so fused or not they round the same. */
static void matmul_iq2xs(const uint8_t *W, const float *X, uint32_t S, uint32_t rows, uint32_t cols,
                         float *out) {
    const uint32_t nb = cols / 256;
    for (uint32_t s = 0; s < S; ++s)
        for (uint32_t r = 0; r < rows; ++r) {
            double dot = 0.0;
            for (uint32_t b = 0; b < nb; ++b) {
                const uint8_t *blk = W + ((size_t)r * nb + b) * 74;
                const float *x = X + (size_t)s * cols + (size_t)b * 256;
                double bd = 0.0;
                for (int e = 0; e < 256; ++e) bd += (double)x[e] * (double)iq2xs_weight(blk, e);
                dot += (double)(float)bd;
            }
            out[(size_t)s * rows + r] = (float)dot;
        }
}

/* Q5_0: no activation quantization. Block dot = (float)(sum over j < 16 of
 * double(x_j) * v_j then double(x_{j+16}) * v_{j+16}, in that order) * d
 * (dotProductQ5_0, include/GGMLDequantize.hpp:1820-1836); row = float(sum_b
 * double(block dot)) (matMulVecFused, :2449-2461). */
static void matmul_q50(const uint8_t *W, const float *X, uint32_t S, uint32_t rows, uint32_t cols, float *out) {
    const uint32_t nb = cols / 32;
    for (uint32_t s = 0; s < S; ++s)
        for (uint32_t r = 0; r < rows; ++r) {
            double dot = 0.0;
            for (uint32_t b = 0; b < nb; ++b) {
                const uint8_t *blk = W + ((size_t)r * nb + b) * 22;
                const float *x = X + (size_t)s * cols + (size_t)b * 32;
                double bd = 0.0;
                for (int j = 0; j < 16; ++j) {
                    bd += (double)x[j] * q50_value(blk, j);
                    bd += (double)x[j + 16] * q50_value(blk, j + 16);
                }
                dot += (double)((float)bd * h2f_at(blk));
            }
            out[(size_t)s * rows + r] = (float)dot;
        }
}

/* IQ4_NL: no activation quantization (src/cpp/core/SIMDMatMulVecAVX2.cpp:
 * 4126-4200, matMulVecBatchIQ4NL_Q8K_AVX2, dots fp32 x). Per 32-block, lane l
 * of 8 forms fma(w3, x[24+l], fma(w2, x[16+l], fma(w1, x[8+l], w0 * x[l])))
 * with w_k = kvalues of element 8k + l; the lanes reduce as ((v0+v4) +
 * (v1+v5)) + ((v2+v6) + (v3+v7)) (lo+hi, then two hadd); the row accumulator
 * from 0 takes fma(d, sum, acc) block by block (contracted `acc += d * sum`). */
static void matmul_iq4nl(const uint8_t *W, const float *X, uint32_t S, uint32_t rows, uint32_t cols,
                         float *out) {
    const uint32_t nb = cols / 32;
    for (uint32_t s = 0; s < S; ++s)
        for (uint32_t r = 0; r < rows; ++r) {
            float acc = 0.0f;
            for (uint32_t b = 0; b < nb; ++b) {
                const uint8_t *blk = W + ((size_t)r * nb + b) * 18;
                const float *x = X + (size_t)s * cols + (size_t)b * 32;
                float w[32], v[8];
                for (int j = 0; j < 16; ++j) {
                    w[j] = (float)k_kvalues_iq4nl[blk[2 + j] & 0xF];
                    w[j + 16] = (float)k_kvalues_iq4nl[blk[2 + j] >> 4];
                }
                for (int l = 0; l < 8; ++l) {
                    float t = w[l] * x[l];
                    t = fmaf(w[8 + l], x[8 + l], t);
                    t = fmaf(w[16 + l], x[16 + l], t);
                    v[l] = fmaf(w[24 + l], x[24 + l], t);
                }
                const float sum = hsum8(v);
                acc = fmaf(h2f_at(blk), sum, acc);
            }
            out[(size_t)s * rows + r] = acc;
        }
}

int oc_matmul(int type, const uint8_t *W, const float *X, uint32_t S, uint32_t rows,
              uint32_t cols, float *out) {
    if (!shape_ok(type, cols)) return -1;
    if (type == OC_TYPE_IQ2_XS) {
        matmul_iq2xs(W, X, S, rows, cols, out);
        return 0;
    }
    if (type == OC_TYPE_IQ4_NL) {
        matmul_iq4nl(W, X, S, rows, cols, out);
        return 0;
    }
    if (type == OC_TYPE_Q5_0) {
        matmul_q50(W, X, S, rows, cols, out);
        return 0;
    }
    act_t a;
    if (quantize_acts(type, X, S, cols, &a)) return -1;
    const uint32_t bs = oc_block_size(type), ts = oc_type_size(type), nb = cols / bs;
    for (uint32_t s = 0; s < S; ++s) {
        const size_t qoff = (size_t)s * cols;
        const size_t doff = (size_t)s * (cols / bs);
        const size_t boff = (size_t)s * (cols / 16);
        for (uint32_t r = 0; r < rows; ++r) {
            const uint8_t *rp = W + (size_t)r * nb * ts;
            float v;
            switch (type) {
                case OC_TYPE_Q4_K: v = row_q4k(rp, nb, &a, qoff, doff, boff); break;
                case OC_TYPE_Q5_K: v = row_q5k(rp, nb, &a, qoff, doff, boff); break;
                case OC_TYPE_Q3_K: v = row_q3k(rp, nb, &a, qoff, doff, boff); break;
                case OC_TYPE_Q2_K: v = row_q2k(rp, nb, &a, qoff, doff, boff); break;
                case OC_TYPE_Q6_K: v = row_q6k(rp, nb, &a, qoff, doff, boff); break;
                case OC_TYPE_IQ3_XXS: v = row_iq3(rp, nb, &a, qoff, doff); break;
                case OC_TYPE_IQ3_S: v = row_iq3s(rp, nb, &a, qoff, doff); break;
                case OC_TYPE_IQ2_S: v = row_iq2s(rp, nb, &a, qoff, doff); break;
                case OC_TYPE_IQ4_XS: v = row_iq4xs(rp, nb, &a, qoff, doff); break;
                default: v = row_q80(rp, nb, &a, qoff, doff); break;
            }
            out[(size_t)s * rows + r] = v;
        }
    }
    free_acts(&a);
    return 0;
}

/* ---- weight encoders ----------------------------------------------------------- */

/* src/cpp/core/GGMLQuantize.cpp:47-95 (quantizeQ4KBlock): per 32-group affine
 * fit scale=(max-min)/15, min=-min (clamped at 0 by starting the scan at 0),
 * 6-bit sub-scales against fp16 super-scales maxScale/63 and maxMin/63, packed
 * in get_scale_min_k4 order (GGMLQuantize.cpp:37-45). */
void oc_encode_q4k_block(const float *x, uint8_t *out) {
    float scale[8], minv[8];
    uint8_t q[256];
    float maxScale = 0.0f, maxMin = 0.0f;
    for (int g = 0; g < 8; ++g) {
        const float *xp = x + 32 * g;
        float mn = 0.0f, mx = 0.0f;
        for (int i = 0; i < 32; ++i) {
            mn = xp[i] < mn ? xp[i] : mn;
            mx = mx < xp[i] ? xp[i] : mx;
        }
        const float sc = (mx - mn) / 15.0f;
        scale[g] = sc;
        minv[g] = -mn;
        maxScale = maxScale < sc ? sc : maxScale;
        maxMin = maxMin < minv[g] ? minv[g] : maxMin;
        for (int i = 0; i < 32; ++i) {
            int v = sc > 1e-30f ? (int)lrintf((xp[i] - mn) / sc) : 0;
            v = v < 0 ? 0 : (v > 15 ? 15 : v);
            q[32 * g + i] = (uint8_t)v;
        }
    }
    const uint16_t hd = maxScale > 0.0f ? oc_float_to_half(maxScale / 63.0f) : 0;
    const uint16_t hdm = maxMin > 0.0f ? oc_float_to_half(maxMin / 63.0f) : 0;
    const float d = oc_half_to_float(hd), dm = oc_half_to_float(hdm);
    uint8_t sc6[8], m6[8];
    for (int g = 0; g < 8; ++g) {
        int s = d > 1e-30f ? (int)lrintf(scale[g] / d) : 0;
        int m = dm > 1e-30f ? (int)lrintf(minv[g] / dm) : 0;
        sc6[g] = (uint8_t)(s < 0 ? 0 : (s > 63 ? 63 : s));
        m6[g] = (uint8_t)(m < 0 ? 0 : (m > 63 ? 63 : m));
    }
    memcpy(out, &hd, 2);
    memcpy(out + 2, &hdm, 2);
    for (int j = 0; j < 4; ++j) {
        out[4 + j] = (uint8_t)(sc6[j] | ((sc6[j + 4] >> 4) << 6));
        out[4 + j + 4] = (uint8_t)(m6[j] | ((m6[j + 4] >> 4) << 6));
        out[4 + j + 8] = (uint8_t)((sc6[j + 4] & 0x0F) | ((m6[j + 4] & 0x0F) << 4));
    }
    uint8_t *qs = out + 16;
    memset(qs, 0, 128);
    for (int g = 0; g < 8; ++g)
        for (int i = 0; i < 32; ++i) qs[32 * (g >> 1) + i] |= (uint8_t)(q[32 * g + i] << (4 * (g & 1)));
}

/* Q8_0 weight encoder (the reference ships none; BASELINE config #1 defines it):
 * d = max|w|/127 stored as fp16 (round to nearest even), q = round to
 * nearest even of w / d_fp16,
 * clamped to [-127, 127]. */
void oc_encode_q8_0_block(const float *x, uint8_t *out) {
    float amax = 0.0f;
    for (int i = 0; i < 32; ++i) amax = fabsf(x[i]) > amax ? fabsf(x[i]) : amax;
    const uint16_t hd = f2h_rne(amax / 127.0f);
    const float d = oc_half_to_float(hd);
    memcpy(out, &hd, 2);
    for (int i = 0; i < 32; ++i) {
        long q = d > 0.0f ? lrintf(x[i] / d) : 0;
        q = q < -127 ? -127 : (q > 127 ? 127 : q);
        out[2 + i] = (uint8_t)(int8_t)q;
    }
}

/* Q5_K weight encoder (the reference ships none; this build defines it, in
 * the shape of the Q4_K one, src/cpp/core/GGMLQuantize.cpp:47-95): per
 * 32-group affine fit scale = (max-min)/31, min = -min (the scan starts at 0);
 * 6-bit sub-scales and mins against fp16 super-scales maxScale/63, maxMin/63
 * (round to nearest even); q = clamp(rne((x + m6*dmin) / (sc6*d)), 0, 31)
 * against the stored scales, packed as include/GGMLDequantize.hpp:346-411
 * reads them. */
void oc_encode_q5k_block(const float *x, uint8_t *out) {
    float scale[8], minv[8];
    float maxScale = 0.0f, maxMin = 0.0f;
    for (int g = 0; g < 8; ++g) {
        const float *xp = x + 32 * g;
        float mn = 0.0f, mx = 0.0f;
        for (int i = 0; i < 32; ++i) {
            mn = xp[i] < mn ? xp[i] : mn;
            mx = mx < xp[i] ? xp[i] : mx;
        }
        scale[g] = (mx - mn) / 31.0f;
        minv[g] = -mn;
        maxScale = maxScale < scale[g] ? scale[g] : maxScale;
        maxMin = maxMin < minv[g] ? minv[g] : maxMin;
    }
    const uint16_t hd = maxScale > 0.0f ? f2h_rne(maxScale / 63.0f) : 0;
    const uint16_t hdm = maxMin > 0.0f ? f2h_rne(maxMin / 63.0f) : 0;
    const float d = oc_half_to_float(hd), dm = oc_half_to_float(hdm);
    uint8_t sc6[8], m6[8];
    for (int g = 0; g < 8; ++g) {
        int sv = d > 0.0f ? (int)lrintf(scale[g] / d) : 0;
        int mv = dm > 0.0f ? (int)lrintf(minv[g] / dm) : 0;
        sc6[g] = (uint8_t)(sv < 0 ? 0 : (sv > 63 ? 63 : sv));
        m6[g] = (uint8_t)(mv < 0 ? 0 : (mv > 63 ? 63 : mv));
    }
    memcpy(out, &hd, 2);
    memcpy(out + 2, &hdm, 2);
    for (int j = 0; j < 4; ++j) {
        out[4 + j] = (uint8_t)(sc6[j] | ((sc6[j + 4] >> 4) << 6));
        out[4 + j + 4] = (uint8_t)(m6[j] | ((m6[j + 4] >> 4) << 6));
        out[4 + j + 8] = (uint8_t)((sc6[j + 4] & 0x0F) | ((m6[j + 4] & 0x0F) << 4));
    }
    uint8_t *qh = out + 16, *qs = out + 48;
    memset(qh, 0, 32);
    memset(qs, 0, 128);
    for (int g = 0; g < 8; ++g) {
        const float es = d * (float)sc6[g], em = dm * (float)m6[g];
        const int c = g >> 1, h = g & 1;
        for (int l = 0; l < 32; ++l) {
            int v = es > 0.0f ? (int)lrintf((x[32 * g + l] + em) / es) : 0;
            v = v < 0 ? 0 : (v > 31 ? 31 : v);
            qs[32 * c + l] |= (uint8_t)((v & 15) << (4 * h));
            qh[l] |= (uint8_t)((v >> 4) << (2 * c + h));
        }
    }
}

/* Q2_K weight encoder (the reference ships none; this build defines it).
 * Per 16: mn = min(0, min x), mx = max(0, max x), scale (mx-mn)/3, min -mn.
 * Block: d = max scale / 15 and dmin = max min / 15 as fp16 (RNE); 4-bit
 * sc = clamp(rne(scale/d), 0, 15), m = clamp(rne(min/dmin), 0, 15); weights
 * q = clamp(rne((x + dmin_fp16*m) / (d_fp16*sc)), 0, 3), packed as the
 * decoder include/GGMLDequantize.hpp:550-590 reads them. */
void oc_encode_q2k_block(const float *x, uint8_t *out) {
    float scale[16], minv[16], maxScale = 0.0f, maxMin = 0.0f;
    for (int g = 0; g < 16; ++g) {
        float mn = 0.0f, mx = 0.0f;
        for (int i = 0; i < 16; ++i) {
            mn = x[16 * g + i] < mn ? x[16 * g + i] : mn;
            mx = mx < x[16 * g + i] ? x[16 * g + i] : mx;
        }
        scale[g] = (mx - mn) / 3.0f;
        minv[g] = -mn;
        maxScale = maxScale < scale[g] ? scale[g] : maxScale;
        maxMin = maxMin < minv[g] ? minv[g] : maxMin;
    }
    memset(out, 0, 84);
    const uint16_t hd = maxScale > 0.0f ? f2h_rne(maxScale / 15.0f) : 0;
    const uint16_t hm = maxMin > 0.0f ? f2h_rne(maxMin / 15.0f) : 0;
    memcpy(out + 80, &hd, 2);
    memcpy(out + 82, &hm, 2);
    const float d = oc_half_to_float(hd), dm = oc_half_to_float(hm);
    for (int g = 0; g < 16; ++g) {
        int sv = d > 0.0f ? (int)lrintf(scale[g] / d) : 0;
        int mv = dm > 0.0f ? (int)lrintf(minv[g] / dm) : 0;
        sv = sv < 0 ? 0 : (sv > 15 ? 15 : sv);
        mv = mv < 0 ? 0 : (mv > 15 ? 15 : mv);
        out[g] = (uint8_t)(sv | (mv << 4));
        const float es = d * (float)sv, em = dm * (float)mv;
        for (int i = 0; i < 16; ++i) {
            const int e = 16 * g + i;
            int q = es > 0.0f ? (int)lrintf((x[e] + em) / es) : 0;
            q = q < 0 ? 0 : (q > 3 ? 3 : q);
            const int h = e >> 7, t = (e >> 5) & 3, l = e & 31;
            out[16 + 32 * h + l] |= (uint8_t)(q << (2 * t));
        }
    }
}

/* Q3_K weight encoder (the reference ships none; this build defines it).
 * Per 16-group: signed first-abs-max m, group scale m/-4 (m maps to -4).
 * Block: signed first-abs-max of the group scales M, iscale = -32/M, 6-bit
 * signed scales s = clamp(rne(iscale*scale), -32, 31) stored as s+32, d =
 * 1/iscale as fp16 (RNE). Weights q = clamp(rne(x / (d_fp16*s)), -4, 3),
 * stored as q+4: 2 low bits in qs, the third bit in hmask, laid out as the
 * decoder include/GGMLDequantize.hpp:612-648 reads them. */
void oc_encode_q3k_block(const float *x, uint8_t *out) {
    float gs[16];
    for (int g = 0; g < 16; ++g) {
        float amax;
        const float m = first_abs_max(x + 16 * g, 16, &amax);
        gs[g] = amax == 0.0f ? 0.0f : m / -4.0f;
    }
    float amaxs;
    const float M = first_abs_max(gs, 16, &amaxs);
    memset(out, 0, 110);
    int s6[16], L[256];
    if (amaxs == 0.0f) {
        for (int g = 0; g < 16; ++g) s6[g] = 32;
        for (int e = 0; e < 256; ++e) L[e] = 4;
    } else {
        const float iscale = -32.0f / M;
        for (int g = 0; g < 16; ++g) {
            int v = (int)lrintf(iscale * gs[g]);
            v = v < -32 ? -32 : (v > 31 ? 31 : v);
            s6[g] = v + 32;
        }
        const uint16_t hd = f2h_rne(1.0f / iscale);
        memcpy(out + 108, &hd, 2);
        const float dh = oc_half_to_float(hd);
        for (int e = 0; e < 256; ++e) {
            const float dg = dh * (float)(s6[e >> 4] - 32);
            int q = dg != 0.0f ? (int)lrintf(x[e] / dg) : 0;
            q = q < -4 ? -4 : (q > 3 ? 3 : q);
            L[e] = q + 4;
        }
    }
    for (int i = 0; i < 4; ++i) {
        out[96 + i] = (uint8_t)((s6[i] & 15) | ((s6[8 + i] & 15) << 4));
        out[100 + i] = (uint8_t)((s6[4 + i] & 15) | ((s6[12 + i] & 15) << 4));
        out[104 + i] = (uint8_t)((s6[i] >> 4) | ((s6[4 + i] >> 4) << 2) | ((s6[8 + i] >> 4) << 4) |
                                 ((s6[12 + i] >> 4) << 6));
    }
    for (int e = 0; e < 256; ++e) {
        const int n = e >> 7, j = (e >> 5) & 3, l = e & 31;
        out[32 + 32 * n + l] |= (uint8_t)((L[e] & 3) << (2 * j));
        out[l] |= (uint8_t)((L[e] >> 2) << (4 * n + j));
    }
}

/* Q6_K weight encoder (the reference ships none; this build defines it).
 * Per 16-group: signed first-abs-max m, group scale m/-32. Block: signed
 * first-abs-max of the group scales M, iscale = -128/M, sc = min(127,
 * rne(iscale*scale)), d = 1/iscale stored as fp16 (RNE). Weights:
 * q = clamp(rne(x / (d_fp16*sc)), -32, 31) + 32, packed as the decoder
 * include/GGMLDequantize.hpp:503-527 reads them. */
void oc_encode_q6k_block(const float *x, uint8_t *out) {
    float gs[16];
    for (int g = 0; g < 16; ++g) {
        float amax;
        const float m = first_abs_max(x + 16 * g, 16, &amax);
        gs[g] = amax == 0.0f ? 0.0f : m / -32.0f;
    }
    float amaxs;
    const float M = first_abs_max(gs, 16, &amaxs);
    memset(out, 0, 210);
    uint8_t L[256];
    if (amaxs == 0.0f) {
        for (int e = 0; e < 256; ++e) L[e] = 32;
    } else {
        const float iscale = -128.0f / M;
        int8_t *sc = (int8_t *)(out + 192);
        for (int g = 0; g < 16; ++g) {
            long v = lrintf(iscale * gs[g]);
            sc[g] = (int8_t)(v > 127 ? 127 : v);
        }
        const uint16_t hd = f2h_rne(1.0f / iscale);
        memcpy(out + 208, &hd, 2);
        const float dh = oc_half_to_float(hd);
        for (int e = 0; e < 256; ++e) {
            const float dg = dh * (float)sc[e >> 4];
            long q = dg != 0.0f ? lrintf(x[e] / dg) : 0;
            q = q < -32 ? -32 : (q > 31 ? 31 : q);
            L[e] = (uint8_t)(q + 32);
        }
    }
    for (int half = 0; half < 2; ++half) {
        uint8_t *ql = out + 64 * half;
        uint8_t *qh = out + 128 + 32 * half;
        const uint8_t *Lh = L + 128 * half;
        for (int l = 0; l < 32; ++l) {
            const int q1 = Lh[l], q2 = Lh[l + 32], q3 = Lh[l + 64], q4 = Lh[l + 96];
            ql[l] = (uint8_t)((q1 & 0xF) | ((q3 & 0xF) << 4));
            ql[l + 32] = (uint8_t)((q2 & 0xF) | ((q4 & 0xF) << 4));
            qh[l] = (uint8_t)((q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6));
        }
    }
}

/* IQ3_XXS weight encoder (the reference ships none; this build defines it).
 * Per 32-chunk c: s_c = max|x| / 62 (62 = largest grid magnitude). Block:
 * d = max_c s_c / 7.75 stored as fp16 (RNE); ls_c = clamp(rne(s_c /
 * (0.5*d) - 0.5), 0, 15); db = d*(0.5+ls)*0.5 (the decoder's expression).
 * Signs per 8: the negative elements, with the smallest-|x| (first) element's
 * sign flipped when the count is odd (the format stores 7 sign bits and
 * implies the 8th by even parity). Magnitudes per 4: the grid entry with the
 * least sum of squared differences to |x|/db (first on ties), sums formed in
 * index order without FMA. */
/* IQ3_S weight encoder (the reference ships none; this build defines it).
 * Per 32: s = max|x|/15; d = max s / 31 (fp16 RNE); ls = clamp(rne((s/d -
 * 1)/2), 0, 15), db = d*(1+2ls); per weight the sign bit (x < 0); per 4 the
 * grid entry (of 512) nearest |x|/db in squared error (first wins), its
 * bit 8 in qh, as the decoder include/GGMLDequantize.hpp:1164-1212 reads. */
void oc_encode_iq3s_block(const float *x, uint8_t *out) {
    float sc[8], smax = 0.0f;
    for (int c = 0; c < 8; ++c) {
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fabsf(x[32 * c + i]) > amax ? fabsf(x[32 * c + i]) : amax;
        sc[c] = amax / 15.0f;
        smax = sc[c] > smax ? sc[c] : smax;
    }
    memset(out, 0, 110);
    const uint16_t hd = f2h_rne(smax / 31.0f);
    const float d = oc_half_to_float(hd);
    if (d == 0.0f) return;
    memcpy(out, &hd, 2);
    uint8_t *qs = out + 2, *qh = out + 66, *signs = out + 74, *scales = out + 106;
    for (int c = 0; c < 8; ++c) {
        int ls = (int)lrintf((sc[c] / d - 1.0f) / 2.0f);
        ls = ls < 0 ? 0 : (ls > 15 ? 15 : ls);
        scales[c >> 1] |= (uint8_t)(ls << (4 * (c & 1)));
        const float db = d * (1.0f + 2.0f * (float)ls);
        for (int l = 0; l < 4; ++l) {
            const float *xv = x + 32 * c + 8 * l;
            for (int j = 0; j < 8; ++j)
                if (xv[j] < 0.0f) signs[4 * c + l] |= (uint8_t)(1u << j);
            for (int h = 0; h < 2; ++h) {
                float t[4];
                for (int j = 0; j < 4; ++j) t[j] = fabsf(xv[4 * h + j]) / db;
                int best = 0;
                float berr = 0.0f;
                for (int gi = 0; gi < 512; ++gi) {
                    float err = 0.0f;
                    for (int j = 0; j < 4; ++j) {
                        const float diff = (float)((k_iq3s_grid[gi] >> (8 * j)) & 0xFFu) - t[j];
                        err = err + diff * diff;
                    }
                    if (gi == 0 || err < berr) {
                        berr = err;
                        best = gi;
                    }
                }
                qs[8 * c + 2 * l + h] = (uint8_t)(best & 255);
                qh[c] |= (uint8_t)((best >> 8) << (2 * l + h));
            }
        }
    }
}

/* IQ2_S weight encoder (the reference ships none; this build defines it).
 * Per 16 (half of a 32-run): s = max|x|/43; d = 8 * max s / 31 (fp16 RNE);
 * ls = clamp(rne((8s/d - 1)/2), 0, 15), db = (d*(0.5+ls))*0.25; a sign bit
 * per weight; per 8 the codebook entry (of 1024) nearest |x|/db in squared
 * error (first wins), index bits 8-9 in qh, as the decoder
 * include/GGMLDequantize.hpp:1215-1242 reads them. */
void oc_encode_iq2s_block(const float *x, uint8_t *out) {
    float sc[16], smax = 0.0f;
    for (int c = 0; c < 16; ++c) {
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i) amax = fabsf(x[16 * c + i]) > amax ? fabsf(x[16 * c + i]) : amax;
        sc[c] = amax / 43.0f;
        smax = sc[c] > smax ? sc[c] : smax;
    }
    memset(out, 0, 82);
    const uint16_t hd = f2h_rne(8.0f * smax / 31.0f);
    const float d = oc_half_to_float(hd);
    if (d == 0.0f) return;
    memcpy(out, &hd, 2);
    uint8_t *qs = out + 2, *signs = out + 34, *qh = out + 66, *scales = out + 74;
    for (int c = 0; c < 16; ++c) {
        const int ib = c >> 1, h = c & 1;
        int ls = (int)lrintf((8.0f * sc[c] / d - 1.0f) / 2.0f);
        ls = ls < 0 ? 0 : (ls > 15 ? 15 : ls);
        scales[ib] |= (uint8_t)(ls << (4 * h));
        const float db = d * (0.5f + (float)ls) * 0.25f;
        for (int q = 0; q < 2; ++q) {
            const int l = 2 * h + q;
            const float *xv = x + 32 * ib + 8 * l;
            float t[8];
            for (int j = 0; j < 8; ++j) {
                if (xv[j] < 0.0f) signs[4 * ib + l] |= (uint8_t)(1u << j);
                t[j] = fabsf(xv[j]) / db;
            }
            int best = 0;
            float berr = 0.0f;
            for (int gi = 0; gi < 1024; ++gi) {
                float err = 0.0f;
                for (int j = 0; j < 8; ++j) {
                    const float diff = (float)((k_iq2s_grid[gi] >> (8 * j)) & 0xFFu) - t[j];
                    err = err + diff * diff;
                }
                if (gi == 0 || err < berr) {
                    berr = err;
                    best = gi;
                }
            }
            qs[4 * ib + l] = (uint8_t)(best & 255);
            qh[ib] |= (uint8_t)((best >> 8) << (2 * l));
        }
    }
}

/* IQ4_XS weight encoder (the reference ships none; this build defines it).
 * Per 32: s = m / -127 with m the first element of largest |x| (it maps to
 * kvalues[0]). Block: d = M / -32 (fp16 RNE) with M the first s of largest
 * |s|; ls - 32 = clamp(rne(s / d), -32, 31); dl = d * (ls - 32); per weight
 * the table entry n minimising (dl * kvalues[n] - x)^2 (first wins), packed
 * as the decoder include/GGMLDequantize.hpp:1044-1080 reads it. */
void oc_encode_iq4xs_block(const float *x, uint8_t *out) {
    float sc[8], smax = 0.0f;
    for (int c = 0; c < 8; ++c) {
        float m = 0.0f;
        for (int i = 0; i < 32; ++i) m = fabsf(x[32 * c + i]) > fabsf(m) ? x[32 * c + i] : m;
        sc[c] = m / -127.0f;
        smax = fabsf(sc[c]) > fabsf(smax) ? sc[c] : smax;
    }
    memset(out, 0, 136);
    const uint16_t hd = f2h_rne(smax / -32.0f);
    const float d = oc_half_to_float(hd);
    if (d == 0.0f || d != d) return;
    memcpy(out, &hd, 2);
    uint16_t sh = 0;
    for (int c = 0; c < 8; ++c) {
        int l = (int)rintf(sc[c] / d);
        l = l < -32 ? -32 : (l > 31 ? 31 : l);
        const int ls = l + 32;
        out[4 + c / 2] |= (uint8_t)((ls & 15) << (4 * (c % 2)));
        sh |= (uint16_t)((ls >> 4) << (2 * c));
        const float dl = d * (float)l;
        for (int j = 0; j < 32; ++j) {
            int best = 0;
            float berr = 0.0f;
            for (int n = 0; n < 16; ++n) {
                const float diff = dl * (float)k_kvalues_iq4nl[n] - x[32 * c + j];
                const float err = diff * diff;
                if (n == 0 || err < berr) {
                    berr = err;
                    best = n;
                }
            }
            out[8 + 16 * c + (j & 15)] |= (uint8_t)(j < 16 ? best : best << 4);
        }
    }
    memcpy(out + 2, &sh, 2);
}

/* Q5_0 weight encoder (the reference ships none; this build defines it): d =
 * m / -16 (fp16 RNE) with m the first element of largest |x|; q =
 * clamp(rne(x / d) + 16, 0, 31), packed as the decoder
 * include/GGMLDequantize.hpp:163-185 reads it. */
void oc_encode_q50_block(const float *x, uint8_t *out) {
    float m = 0.0f;
    for (int i = 0; i < 32; ++i) m = fabsf(x[i]) > fabsf(m) ? x[i] : m;
    memset(out, 0, 22);
    const uint16_t hd = f2h_rne(m / -16.0f);
    const float d = oc_half_to_float(hd);
    if (d == 0.0f || d != d) return;
    memcpy(out, &hd, 2);
    uint32_t qh = 0;
    for (int j = 0; j < 32; ++j) {
        int q = (int)rintf(x[j] / d) + 16;
        q = q < 0 ? 0 : (q > 31 ? 31 : q);
        out[6 + (j & 15)] |= (uint8_t)(j < 16 ? (q & 15) : (q & 15) << 4);
        qh |= (uint32_t)(q >> 4) << j;
    }
    memcpy(out + 2, &qh, 4);
}

/* IQ4_NL weight encoder (the reference ships none; this build defines it):
 * d = m / -127 (fp16 RNE) with m the first element of largest |x|; per weight
 * the table entry minimising (d * kvalues[n] - x)^2 (first wins), packed as
 * the decoder include/GGMLDequantize.hpp:1304-1312 reads it. */
void oc_encode_iq4nl_block(const float *x, uint8_t *out) {
    float m = 0.0f;
    for (int i = 0; i < 32; ++i) m = fabsf(x[i]) > fabsf(m) ? x[i] : m;
    memset(out, 0, 18);
    const uint16_t hd = f2h_rne(m / -127.0f);
    const float d = oc_half_to_float(hd);
    if (d == 0.0f || d != d) return;
    memcpy(out, &hd, 2);
    for (int j = 0; j < 32; ++j) {
        int best = 0;
        float berr = 0.0f;
        for (int n = 0; n < 16; ++n) {
            const float diff = d * (float)k_kvalues_iq4nl[n] - x[j];
            const float err = diff * diff;
            if (n == 0 || err < berr) {
                berr = err;
                best = n;
            }
        }
        out[2 + (j & 15)] |= (uint8_t)(j < 16 ? best : best << 4);
    }
}

/* IQ2_XS weight encoder (the reference ships none; this build defines it).
 * Scales as IQ2_S (per 16: s = max|x|/43, d = 8 max s / 31 fp16 RNE, ls =
 * clamp(rne((8s/d - 1)/2), 0, 15)); per 8: the negative signs with the
 * smallest-|x| one flipped on odd count (the format implies even parity) and
 * the codebook entry (of 512) nearest |x|/db in squared error (first wins);
 * qs16 = index | (signs & 127) << 9, as include/GGMLDequantize.hpp:1245-1271
 * reads them. */
void oc_encode_iq2xs_block(const float *x, uint8_t *out) {
    float sc[16], smax = 0.0f;
    for (int c = 0; c < 16; ++c) {
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i) amax = fabsf(x[16 * c + i]) > amax ? fabsf(x[16 * c + i]) : amax;
        sc[c] = amax / 43.0f;
        smax = sc[c] > smax ? sc[c] : smax;
    }
    memset(out, 0, 74);
    const uint16_t hd = f2h_rne(8.0f * smax / 31.0f);
    const float d = oc_half_to_float(hd);
    if (d == 0.0f) return;
    memcpy(out, &hd, 2);
    for (int c = 0; c < 16; ++c) {
        const int ib = c >> 1, h = c & 1;
        int ls = (int)lrintf((8.0f * sc[c] / d - 1.0f) / 2.0f);
        ls = ls < 0 ? 0 : (ls > 15 ? 15 : ls);
        out[66 + ib] |= (uint8_t)(ls << (4 * h));
        const float db = d * (0.5f + (float)ls) * 0.25f;
        for (int q = 0; q < 2; ++q) {
            const int l = 2 * h + q;
            const float *xv = x + 32 * ib + 8 * l;
            uint32_t neg = 0;
            int minj = 0;
            float t[8];
            for (int j = 0; j < 8; ++j) {
                if (xv[j] < 0.0f) neg |= 1u << j;
                if (fabsf(xv[j]) < fabsf(xv[minj])) minj = j;
                t[j] = fabsf(xv[j]) / db;
            }
            if (__builtin_popcount(neg) & 1) neg ^= 1u << minj;
            int best = 0;
            float berr = 0.0f;
            for (int gi = 0; gi < 512; ++gi) {
                float err = 0.0f;
                for (int j = 0; j < 8; ++j) {
                    const float diff = (float)((k_iq2xs_grid[gi] >> (8 * j)) & 0xFFu) - t[j];
                    err = err + diff * diff;
                }
                if (gi == 0 || err < berr) {
                    berr = err;
                    best = gi;
                }
            }
            const uint16_t qv = (uint16_t)(best | ((neg & 127u) << 9));
            memcpy(out + 2 + 2 * (4 * ib + l), &qv, 2);
        }
    }
}

void oc_encode_iq3xxs_block(const float *x, uint8_t *out) {
    float sc[8], smax = 0.0f;
    for (int c = 0; c < 8; ++c) {
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) amax = fabsf(x[32 * c + i]) > amax ? fabsf(x[32 * c + i]) : amax;
        sc[c] = amax / 62.0f;
        smax = sc[c] > smax ? sc[c] : smax;
    }
    memset(out, 0, 98);
    const uint16_t hd = f2h_rne(smax / 7.75f);
    const float d = oc_half_to_float(hd);
    if (d == 0.0f) return;
    memcpy(out, &hd, 2);
    uint8_t *qs = out + 2;
    uint8_t *sas = out + 66;
    for (int c = 0; c < 8; ++c) {
        long lsl = lrintf(sc[c] / (0.5f * d) - 0.5f);
        const int ls = lsl < 0 ? 0 : (lsl > 15 ? 15 : (int)lsl);
        const float db = d * (0.5f + (float)ls) * 0.5f;
        uint32_t aux = (uint32_t)ls << 28;
        for (int l = 0; l < 4; ++l) {
            const float *xv = x + 32 * c + 8 * l;
            uint32_t neg = 0;
            int minj = 0;
            for (int j = 0; j < 8; ++j) {
                if (xv[j] < 0.0f) neg |= 1u << j;
                if (fabsf(xv[j]) < fabsf(xv[minj])) minj = j;
            }
            if (__builtin_parity(neg)) neg ^= 1u << minj;
            aux |= (neg & 127u) << (7 * l);
            for (int h = 0; h < 2; ++h) {
                float t[4];
                for (int j = 0; j < 4; ++j) t[j] = fabsf(xv[4 * h + j]) / db;
                int best = 0;
                float berr = 0.0f;
                for (int gi = 0; gi < 256; ++gi) {
                    float err = 0.0f;
                    for (int j = 0; j < 4; ++j) {
                        const float diff = (float)((k_iq3xxs_grid[gi] >> (8 * j)) & 0xFFu) - t[j];
                        err = err + diff * diff;
                    }
                    if (gi == 0 || err < berr) {
                        berr = err;
                        best = gi;
                    }
                }
                qs[8 * c + 2 * l + h] = (uint8_t)best;
            }
        }
        memcpy(sas + 4 * c, &aux, 4);
    }
}

int oc_encode_rows(int type, const float *x, uint32_t rows, uint32_t cols, uint8_t *out) {
    if (!shape_ok(type, cols)) return -1;
    const uint32_t bs = oc_block_size(type), ts = oc_type_size(type);
    const size_t nblk = (size_t)rows * (cols / bs);
    for (size_t i = 0; i < nblk; ++i) {
        const float *xb = x + i * bs;
        uint8_t *o = out + i * ts;
        switch (type) {
            case OC_TYPE_Q8_0: oc_encode_q8_0_block(xb, o); break;
            case OC_TYPE_Q4_K: oc_encode_q4k_block(xb, o); break;
            case OC_TYPE_Q5_K: oc_encode_q5k_block(xb, o); break;
            case OC_TYPE_Q3_K: oc_encode_q3k_block(xb, o); break;
            case OC_TYPE_Q2_K: oc_encode_q2k_block(xb, o); break;
            case OC_TYPE_Q6_K: oc_encode_q6k_block(xb, o); break;
            case OC_TYPE_IQ3_S: oc_encode_iq3s_block(xb, o); break;
            case OC_TYPE_IQ2_S: oc_encode_iq2s_block(xb, o); break;
            case OC_TYPE_IQ2_XS: oc_encode_iq2xs_block(xb, o); break;
            case OC_TYPE_IQ4_XS: oc_encode_iq4xs_block(xb, o); break;
            case OC_TYPE_IQ4_NL: oc_encode_iq4nl_block(xb, o); break;
            case OC_TYPE_Q5_0: oc_encode_q50_block(xb, o); break;
            default: oc_encode_iq3xxs_block(xb, o); break;
        }
    }
    return 0;
}

/* ---- MoE expert FFN ----------------------------------------------------------- */

/* src/cpp/core/ModelMoE.cpp:660-672 (the math statement) with the per-expert
 * path :566-600 and the rank-order reduction :990-1002: per (token s, rank r):
 * g = Wg[e] x, u = Wu[e] x (Q4_K mat-vec, Q8_K activations), h = g/(1+exp(-g))*u,
 * down = Wd[e] h (Q8_K quantization of h), partial = wg*down; out[s] starts at
 * 0 and adds partial for r = 0..K-1 in order. */
int oc_moe_ffn(const float *x, const int32_t *ids, const float *wts, uint32_t S, uint32_t K,
               const uint8_t *wg, const uint8_t *wu, const uint8_t *wd, uint32_t E, uint32_t H,
               uint32_t FF, float *out) {
    if (H % 256 || FF % 256) return -1;
    const size_t gBytes = (size_t)FF * (H / 256) * 144;
    const size_t dBytes = (size_t)H * (FF / 256) * 144;
    float *g = (float *)malloc(sizeof(float) * FF);
    float *u = (float *)malloc(sizeof(float) * FF);
    float *dn = (float *)malloc(sizeof(float) * H);
    if (!g || !u || !dn) return -1;
    for (uint32_t s = 0; s < S; ++s) {
        float *o = out + (size_t)s * H;
        for (uint32_t i = 0; i < H; ++i) o[i] = 0.0f;
        for (uint32_t r = 0; r < K; ++r) {
            const int32_t e = ids[(size_t)s * K + r];
            if (e < 0 || (uint32_t)e >= E) continue;
            const float *xs = x + (size_t)s * H;
            oc_matmul(OC_TYPE_Q4_K, wg + (size_t)e * gBytes, xs, 1, FF, H, g);
            oc_matmul(OC_TYPE_Q4_K, wu + (size_t)e * gBytes, xs, 1, FF, H, u);
            for (uint32_t i = 0; i < FF; ++i) g[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
            oc_matmul(OC_TYPE_Q4_K, wd + (size_t)e * dBytes, g, 1, H, FF, dn);
            const float w = wts[(size_t)s * K + r];
            for (uint32_t i = 0; i < H; ++i) o[i] += w * dn[i];
        }
    }
    free(g);
    free(u);
    free(dn);
    return 0;
}

/* ---- MoE router (F32 router matrix, softmax, top-k, renormalisation) ---- */

/* src/cpp/core/SIMDMatMulVecAVX2.cpp:2982-3090 (matMulVecBatchF32_AVX2, the
 * qwen35moe router logits, ModelMoE.cpp:372-386): per (token, row) 32 fp32
 * FMA lanes (four 8-wide chains) over the first floor(cols/32)*32 columns in
 * steps of 32, the remaining whole 8-column groups into chain 0, the fixed
 * horizontal tree (chains 0+1 and 2+3, their sum, halves, two pairwise adds),
 * then the cols % 8 tail added serially (contracted into an FMA as g++
 * compiles `v += x * w` there). out[S][rows]. */
void oc_matmul_f32(const float *W, const float *X, uint32_t S, uint32_t rows, uint32_t cols, float *out) {
    const uint32_t vec = cols / 8 * 8, tail = cols & 7u;
    for (uint32_t s = 0; s < S; ++s) {
        const float *x = X + (size_t)s * cols;
        for (uint32_t r = 0; r < rows; ++r) {
            const float *w = W + (size_t)r * cols;
            float acc[4][8];
            memset(acc, 0, sizeof acc);
            uint32_t i = 0;
            for (; i + 31 < vec; i += 32)
                for (int c = 0; c < 4; ++c)
                    for (int l = 0; l < 8; ++l) acc[c][l] = fmaf(x[i + 8 * c + l], w[i + 8 * c + l], acc[c][l]);
            for (; i + 7 < vec; i += 8)
                for (int l = 0; l < 8; ++l) acc[0][l] = fmaf(x[i + l], w[i + l], acc[0][l]);
            float sv[8];
            for (int l = 0; l < 8; ++l) sv[l] = (acc[0][l] + acc[1][l]) + (acc[2][l] + acc[3][l]);
            float t[4];
            for (int l = 0; l < 4; ++l) t[l] = sv[l] + sv[l + 4];
            float v = (t[0] + t[1]) + (t[2] + t[3]);
            for (uint32_t k = 0; k < tail; ++k) v = fmaf(x[vec + k], w[vec + k], v);
            out[(size_t)s * rows + r] = v;
        }
    }
}

/* One (probability, expert) entry of the router's ranking. */
typedef struct {
    float p;
    uint32_t e;
} oc_scored;

/* The ranking's order: a before b when a.p > b.p (the comparator of
 * ModelMoE.cpp:402-405). */
static int oc_before(const oc_scored *a, const oc_scored *b) { return a->p > b->p; }

/* The selection of ModelMoE.cpp:402-405 is std::partial_sort(begin,
 * begin + k, end, cmp), which leaves equal probabilities in an order the
 * library's algorithm fixes: a binary heap over the first k entries whose
 * top is the entry every other one is "before" (the smallest probability),
 * each later entry that is strictly before the top replacing it, and a final
 * heap sort. The next three functions are those heap steps as the GNU C++
 * library (the reference's toolchain) performs them: a sift-down that moves
 * the hole to a leaf along the child that is not before its sibling, then a
 * sift-up of the value; the tie order of the result depends on exactly these
 * moves. */
static void oc_heap_push_up(oc_scored *h, size_t hole, size_t top, oc_scored v) {
    size_t parent = (hole - 1) / 2;
    while (hole > top && oc_before(&h[parent], &v)) {
        h[hole] = h[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    h[hole] = v;
}

static void oc_heap_adjust(oc_scored *h, size_t hole, size_t len, oc_scored v) {
    const size_t top = hole;
    size_t child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (oc_before(&h[child], &h[child - 1])) child--;
        h[hole] = h[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        h[hole] = h[child - 1];
        hole = child - 1;
    }
    oc_heap_push_up(h, hole, top, v);
}

/* h[0..k) <- the k first entries of a[0..n) in the order std::partial_sort
 * leaves them (a is permuted as the library permutes it). */
static void oc_partial_sort(oc_scored *a, size_t k, size_t n) {
    if (k == 0) return;
    if (k > 1)
        for (size_t parent = (k - 2) / 2;; --parent) {
            oc_heap_adjust(a, parent, k, a[parent]);
            if (parent == 0) break;
        }
    for (size_t i = k; i < n; ++i)
        if (oc_before(&a[i], &a[0])) {
            const oc_scored v = a[i];
            a[i] = a[0];
            oc_heap_adjust(a, 0, k, v);
        }
    for (size_t last = k; last > 1;) {
        --last;
        const oc_scored v = a[last];
        a[last] = a[0];
        oc_heap_adjust(a, 0, last, v);
    }
}

/* src/cpp/core/ModelMoE.cpp:387-424 (computeQwen35MoERouterOnly, from the
 * logits on): per token, maxL = max logit; probs[e] = (float)exp((double)
 * logit - maxL) summed in double in expert order; invSum = (float)(1/sum);
 * probs *= invSum in float; the top k by the partial_sort above; wsum = the
 * double sum of the k probabilities in rank order, clamped below at
 * 6.103515625e-5; ids[s][r] = expert, wts[s][r] = p / (float)wsum. */
int oc_moe_route(const float *logits, uint32_t S, uint32_t E, uint32_t K, int32_t *ids, float *wts) {
    if (E == 0 || K == 0 || K > E) return -1;
    oc_scored *sc = (oc_scored *)malloc(sizeof(oc_scored) * E);
    float *probs = (float *)malloc(sizeof(float) * E);
    if (!sc || !probs) return -1;
    for (uint32_t s = 0; s < S; ++s) {
        const float *l = logits + (size_t)s * E;
        float maxL = -INFINITY;
        for (uint32_t e = 0; e < E; ++e) maxL = l[e] > maxL ? l[e] : maxL;
        double sum = 0.0;
        for (uint32_t e = 0; e < E; ++e) {
            probs[e] = (float)exp((double)l[e] - (double)maxL);
            sum += (double)probs[e];
        }
        const float inv = (float)(1.0 / sum);
        for (uint32_t e = 0; e < E; ++e) {
            probs[e] = probs[e] * inv;
            sc[e].p = probs[e];
            sc[e].e = e;
        }
        oc_partial_sort(sc, K, E);
        double wsum = 0.0;
        for (uint32_t r = 0; r < K; ++r) wsum += (double)sc[r].p;
        const float wc = (float)(wsum > 6.103515625e-5 ? wsum : 6.103515625e-5);
        for (uint32_t r = 0; r < K; ++r) {
            ids[(size_t)s * K + r] = (int32_t)sc[r].e;
            wts[(size_t)s * K + r] = sc[r].p / wc;
        }
    }
    free(sc);
    free(probs);
    return 0;
}
