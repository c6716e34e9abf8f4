/*
 * ssdq_oracle.c — CPU oracle for the ssd-llm quantized compute path.
 *
 * TEST INFRASTRUCTURE ONLY (see ssdq_oracle.h). Restates the reference's Rust
 * CPU functions op for op. Build with -ffp-contract=off and without
 * -ffast-math: Rust never fuses a*b+c, so neither may this file.
 *
 * Checks that pin this restatement (reference known-answer tests, closed
 * forms, an independent encoder round trip, exhaustive f16 widening, double
 * brute force) live in tests/test_oracle.py.
 */
#include "ssdq_oracle.h"

#include "../ssd-llm_amd/csrc/iq_grids.h" /* IQ2 / IQ3 lattice code books */

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

size_t ssdo_block_size(int dtype) {
    /* src/model/gguf.rs:87-105 */
    switch (dtype) {
        case SSDO_F32: case SSDO_F16: case SSDO_BF16: return 1;
        case SSDO_Q4_0: case SSDO_Q8_0: case SSDO_IQ4_NL: return 32;
        case SSDO_Q2_K: case SSDO_Q3_K: case SSDO_Q4_K: case SSDO_Q5_K: case SSDO_Q6_K:
        case SSDO_Q8_K: case SSDO_IQ4_XS: case SSDO_IQ2_XXS: case SSDO_IQ2_XS: case SSDO_IQ3_XXS:
        case SSDO_IQ3_S: return 256;
        default: return 0;
    }
}

size_t ssdo_type_size(int dtype) {
    /* src/model/gguf.rs:108-135 */
    switch (dtype) {
        case SSDO_F32: return 4;
        case SSDO_F16: case SSDO_BF16: return 2;
        case SSDO_Q4_0: return 18;                      /* 2 + 32/2 */
        case SSDO_Q8_0: return 34;                      /* 2 + 32 */
        case SSDO_Q4_K: return 2 + 2 + 12 + 256 / 2;    /* 144 */
        case SSDO_Q6_K: return 256 / 2 + 256 / 4 + 256 / 16 + 2; /* 210 */
        case SSDO_Q2_K: return 2 + 2 + 16 + 64;         /* 84 */
        case SSDO_Q3_K: return 256 / 8 + 256 / 4 + 12 + 2; /* 110: the block matvec_q3_k_cpu
                                  reads (compute.rs:798); gguf.rs:127 writes 256/8*3 (174) */
        case SSDO_Q5_K: return 2 + 2 + 12 + 256 / 8 + 256 / 2; /* 176 */
        case SSDO_Q8_K: return 4 + 256 + 16 * 2;        /* 292 */
        case SSDO_IQ4_NL: return 2 + 16;                /* 18 */
        case SSDO_IQ4_XS: return 2 + 2 + 128 + 16;      /* 148 */
        case SSDO_IQ2_XXS: return 2 + 256 / 8 * 2;      /* 66 */
        case SSDO_IQ2_XS: return 2 + 256 / 8 * 2 + 256 / 32; /* 74 */
        case SSDO_IQ3_XXS: return 2 + 3 * 256 / 8;      /* 98 */
        case SSDO_IQ3_S: return 2 + 64 + 8 + 32 + 4;    /* 110 */
        default: return 0;
    }
}

/* IEEE-754 binary16 -> binary32 widening (exact). This is what
 * half::f16::to_f32 computes for f16_to_f32, src/metal/compute.rs:2243-2246:
 * subnormals are normalised, infinities kept, NaNs quieted with the payload
 * shifted into the top of the f32 mantissa. */
float ssdo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    uint32_t bits;
    if (e == 0x1Fu) {
        bits = sign | 0x7F800000u | (m << 13);
        if (m) bits |= 0x00400000u;
    } else if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {
            int p = 31 - __builtin_clz(m); /* leading one: value = 2^(p-24) * 1.f */
            bits = sign | ((uint32_t)(p + 103) << 23) | ((m << (23 - p)) & 0x7FFFFFu);
        }
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void ssdo_f16_to_f32_array(const uint16_t* h, size_t n, float* out) {
    for (size_t i = 0; i < n; i++) out[i] = ssdo_f16_to_f32(h[i]);
}

float ssdo_bf16_to_f32(uint16_t h) {
    /* f32::from_bits((h as u32) << 16), src/ssd/streamer.rs:108-114 */
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static inline float le_f16(const uint8_t* p) {
    return ssdo_f16_to_f32((uint16_t)(p[0] | ((uint16_t)p[1] << 8)));
}

/* ---------------------------------------------------------------- dequant */

void ssdo_dequant_q8_0(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    /* src/ssd/streamer.rs:128-150: element = (i8 as f32) * scale */
    const size_t bs = 32, bb = 34;
    size_t n_blocks = n_elements / bs, written = 0;
    for (size_t i = 0; i < n_blocks; i++) {
        size_t s = i * bb;
        if (s + bb > data_len) break;
        float scale = le_f16(data + s);
        for (size_t j = 0; j < bs; j++) out[written++] = (float)(int8_t)data[s + 2 + j] * scale;
    }
    for (; written < n_elements; written++) out[written] = 0.0f; /* output.resize(n, 0.0) */
}

void ssdo_dequant_q4_0(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    /* src/ssd/streamer.rs:153-178: element 2j from the low nibble of qs[j],
     * 2j+1 from the high nibble, both minus 8, times scale */
    const size_t bs = 32, bb = 18;
    size_t n_blocks = n_elements / bs, written = 0;
    for (size_t i = 0; i < n_blocks; i++) {
        size_t s = i * bb;
        if (s + bb > data_len) break;
        float scale = le_f16(data + s);
        for (size_t j = 0; j < 16; j++) {
            uint8_t byte = data[s + 2 + j];
            int lo = (int)(byte & 0x0F) - 8;
            int hi = (int)((byte >> 4) & 0x0F) - 8;
            out[written++] = (float)lo * scale;
            out[written++] = (float)hi * scale;
        }
    }
    for (; written < n_elements; written++) out[written] = 0.0f;
}

void ssdo_dequant_q6_k(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    /* src/ssd/streamer.rs:182-220: ql[128] @0, qh[64] @128, scales i8[16] @192,
     * d f16 @208; element = (d * scale) * q, q = (hi2<<4 | lo4) - 32 */
    const size_t bs = 256, bb = 210;
    size_t n_blocks = n_elements / bs, written = 0;
    for (size_t i = 0; i < n_blocks; i++) {
        size_t s = i * bb;
        if (s + bb > data_len) break;
        const uint8_t* ql = data + s;
        const uint8_t* qh = data + s + 128;
        const uint8_t* sc = data + s + 192;
        float d = le_f16(data + s + 208);
        for (size_t j = 0; j < 256; j++) {
            uint8_t qlb = ql[j / 2];
            unsigned lo4 = (j % 2 == 0) ? (qlb & 0x0Fu) : (unsigned)(qlb >> 4);
            unsigned hi2 = (qh[j / 4] >> ((j % 4) * 2)) & 0x03u;
            int q = (int)(lo4 | (hi2 << 4)) - 32;
            float scale = (float)(int8_t)sc[j / 16];
            out[written++] = d * scale * (float)q;
        }
    }
    for (; written < n_elements; written++) out[written] = 0.0f;
}

/* The 6-bit scale/min of sub-block sb as matvec_q4_k_cpu unpacks them,
 * src/metal/compute.rs:724-731 (note: for sb>=4 the bits taken from sc[sb-4]
 * and sc[sb] land in the LOW two bits). */
static inline void q4k_scale_min(const uint8_t* sc, unsigned sb, unsigned* s, unsigned* m) {
    if (sb < 4) {
        *s = sc[sb] & 0x3Fu;
        *m = sc[sb + 4] & 0x3Fu;
    } else {
        unsigned si = sb - 4;
        *s = (unsigned)(sc[si] >> 6) | ((unsigned)(sc[sb + 4] & 0x0F) << 2);
        *m = (unsigned)(sc[sb] >> 6) | ((unsigned)(sc[sb + 4] >> 4) << 2);
    }
}

void ssdo_dequant_q4_k(const uint8_t* data, size_t data_len, size_t n_elements, float* out) {
    /* Element values of matvec_q4_k_cpu, src/metal/compute.rs:716-744:
     * d f16 @0, dmin f16 @2, sc[12] @4, qs[128] @16;
     * v = (d*s)*q - dmin*m, with q the low/high nibble of qs[sb*16+j]
     * for elements sb*32+2j / sb*32+2j+1. */
    const size_t bs = 256, bb = 144;
    size_t n_blocks = n_elements / bs, written = 0;
    for (size_t i = 0; i < n_blocks; i++) {
        size_t s0 = i * bb;
        if (s0 + bb > data_len) break;
        float d = le_f16(data + s0);
        float dmin = le_f16(data + s0 + 2);
        const uint8_t* sc = data + s0 + 4;
        const uint8_t* qs = data + s0 + 16;
        for (unsigned sb = 0; sb < 8; sb++) {
            unsigned s, m;
            q4k_scale_min(sc, sb, &s, &m);
            float scale = d * (float)s;
            float min_val = dmin * (float)m;
            for (unsigned j = 0; j < 16; j++) {
                uint8_t b = qs[sb * 16 + j];
                out[written++] = scale * (float)(b & 0x0F) - min_val;
                out[written++] = scale * (float)((b >> 4) & 0x0F) - min_val;
            }
        }
    }
    for (; written < n_elements; written++) out[written] = 0.0f;
}

int ssdo_dequantize_to_f32(int dtype, const uint8_t* data, size_t data_len, size_t n_elements,
                           float* out) {
    /* src/ssd/streamer.rs:93-125 (Q4_K added: its values per compute.rs:716-744) */
    switch (dtype) {
        case SSDO_F32:
            memcpy(out, data, n_elements * 4);
            return 0;
        case SSDO_F16:
            for (size_t i = 0; i < n_elements; i++) out[i] = le_f16(data + 2 * i);
            return 0;
        case SSDO_BF16:
            for (size_t i = 0; i < n_elements; i++)
                out[i] = ssdo_bf16_to_f32((uint16_t)(data[2 * i] | (data[2 * i + 1] << 8)));
            return 0;
        case SSDO_Q8_0: ssdo_dequant_q8_0(data, data_len, n_elements, out); return 0;
        case SSDO_Q4_0: ssdo_dequant_q4_0(data, data_len, n_elements, out); return 0;
        case SSDO_Q6_K: ssdo_dequant_q6_k(data, data_len, n_elements, out); return 0;
        case SSDO_Q4_K: ssdo_dequant_q4_k(data, data_len, n_elements, out); return 0;
        default:
            for (size_t i = 0; i < n_elements; i++) out[i] = 0.0f;
            return 1;
    }
}

/* ----------------------------------------------------------------- matvec */

static void mv_q4_0(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                    float* y) {
    /* src/metal/compute.rs:680-704 */
    const size_t bs = 32, bb = 18, bpr = in_dim / bs;
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * bpr * bb;
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            size_t boff = row_off + b * bb;
            float scale = le_f16(w + boff);
            size_t xb = b * bs;
            for (size_t j = 0; j < 16; j++) {
                uint8_t byte = w[boff + 2 + j];
                int lo = (int)(byte & 0x0F) - 8;
                int hi = (int)((byte >> 4) & 0x0F) - 8;
                sum += scale * (float)lo * x[xb + j * 2];
                sum += scale * (float)hi * x[xb + j * 2 + 1];
            }
        }
        y[row] = sum;
    }
}

static void mv_q4_k(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                    float* y) {
    /* src/metal/compute.rs:707-750 */
    const size_t bs = 256, bb = 144, bpr = in_dim / bs;
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * bpr * bb;
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            size_t boff = row_off + b * bb;
            float d = le_f16(w + boff);
            float dmin = le_f16(w + boff + 2);
            const uint8_t* sc = w + boff + 4;
            const uint8_t* qs = w + boff + 16;
            size_t xb = b * bs;
            for (unsigned sb = 0; sb < 8; sb++) {
                unsigned s, m;
                q4k_scale_min(sc, sb, &s, &m);
                float scale = d * (float)s;
                float min_val = dmin * (float)m;
                size_t qo = sb * 16;
                for (size_t j = 0; j < 16; j++) {
                    uint8_t bv = qs[qo + j];
                    float v0 = scale * (float)(bv & 0x0F) - min_val;
                    float v1 = scale * (float)((bv >> 4) & 0x0F) - min_val;
                    size_t xi = xb + sb * 32 + j * 2;
                    sum += v0 * x[xi] + v1 * x[xi + 1];
                }
            }
        }
        y[row] = sum;
    }
}

static void mv_q6_k(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                    float* y) {
    /* src/metal/compute.rs:753-791 */
    const size_t bs = 256, bb = 210, bpr = in_dim / bs;
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * bpr * bb;
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            size_t boff = row_off + b * bb;
            const uint8_t* ql = w + boff;
            const uint8_t* qh = w + boff + 128;
            const uint8_t* scales = w + boff + 192;
            float d = le_f16(w + boff + 208);
            size_t xb = b * bs;
            for (size_t sb = 0; sb < 16; sb++) {
                float sc = d * (float)(int8_t)scales[sb];
                for (size_t j = 0; j < 16; j++) {
                    size_t idx = sb * 16 + j;
                    uint8_t qlb = ql[idx / 2];
                    unsigned low4 = (idx & 1) ? ((qlb >> 4) & 0x0Fu) : (qlb & 0x0Fu);
                    unsigned high2 = (qh[idx / 4] >> ((idx % 4) * 2)) & 0x03u;
                    int q = (int)((high2 << 4) | low4) - 32;
                    sum += sc * (float)q * x[xb + idx];
                }
            }
        }
        y[row] = sum;
    }
}

static void mv_q8_0(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                    float* y) {
    /* src/metal/compute.rs:904-925 */
    const size_t bs = 32, bb = 34, bpr = in_dim / bs;
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * bpr * bb;
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            size_t boff = row_off + b * bb;
            float scale = le_f16(w + boff);
            size_t xb = b * bs;
            for (size_t j = 0; j < 32; j++) {
                int8_t val = (int8_t)w[boff + 2 + j];
                sum += scale * (float)val * x[xb + j];
            }
        }
        y[row] = sum;
    }
}

/* The reference's other matvec types (compute.rs:796-1077, 2256-2285). Each
 * keeps the reference's block layout, element order and expression order. */

static void mv_q3_k(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                    float* y) {
    /* src/metal/compute.rs:796-840: hmask[32] @0, qs[64] @32, sc[12] @96, d f16 @108 */
    const size_t bs = 256, bb = 110, bpr = in_dim / bs;
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * bpr * bb;
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            size_t boff = row_off + b * bb;
            const uint8_t* hmask = w + boff;
            const uint8_t* qs = w + boff + 32;
            const uint8_t* sc = w + boff + 96;
            float d = le_f16(w + boff + 108);
            size_t xb = b * bs;
            for (size_t sb = 0; sb < 16; sb++) {
                unsigned low4 = (sc[sb / 2] >> ((sb & 1) * 4)) & 0x0Fu;
                unsigned hi2 = (sc[8 + sb / 4] >> ((sb % 4) * 2)) & 0x03u;
                int scale_val = (int)(low4 | (hi2 << 4));
                if (scale_val >= 32) scale_val -= 64;
                float sc_f = d * (float)scale_val;
                for (size_t j = 0; j < 16; j++) {
                    size_t idx = sb * 16 + j;
                    unsigned low2 = (qs[idx / 4] >> ((idx % 4) * 2)) & 0x03u;
                    unsigned hbit = (hmask[idx / 8] >> (idx % 8)) & 1u;
                    int q = (int)(low2 | (hbit << 2)) - 4;
                    sum += sc_f * (float)q * x[xb + idx];
                }
            }
        }
        y[row] = sum;
    }
}

static void mv_q5_k(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                    float* y) {
    /* src/metal/compute.rs:845-902: d @0, dmin @2, sc[12] @4 (Q4_K packing),
     * qh[32] @16, ql[128] @48 */
    const size_t bs = 256, bb = 176, bpr = in_dim / bs;
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * bpr * bb;
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            size_t boff = row_off + b * bb;
            float d = le_f16(w + boff);
            float dmin = le_f16(w + boff + 2);
            const uint8_t* sc = w + boff + 4;
            const uint8_t* qh = w + boff + 16;
            const uint8_t* ql = w + boff + 48;
            size_t xb = b * bs;
            for (unsigned sb = 0; sb < 8; sb++) {
                unsigned s, m;
                q4k_scale_min(sc, sb, &s, &m);
                float scale = d * (float)s;
                float min_val = dmin * (float)m;
                size_t qs_off = sb * 16;
                for (size_t j = 0; j < 16; j++) {
                    size_t idx0 = sb * 32 + j * 2, idx1 = idx0 + 1;
                    uint8_t bv = ql[qs_off + j];
                    unsigned low0 = bv & 0x0Fu, low1 = (bv >> 4) & 0x0Fu;
                    unsigned hbit0 = (qh[idx0 / 8] >> (idx0 % 8)) & 1u;
                    unsigned hbit1 = (qh[idx1 / 8] >> (idx1 % 8)) & 1u;
                    float v0 = scale * (float)(low0 | (hbit0 << 4)) - min_val;
                    float v1 = scale * (float)(low1 | (hbit1 << 4)) - min_val;
                    sum += v0 * x[xb + idx0] + v1 * x[xb + idx1];
                }
            }
        }
        y[row] = sum;
    }
}

static void mv_q2_k(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                    float* y) {
    /* src/metal/compute.rs:930-966: d @0, dmin @2, sc[16] @4 (low nibble scale,
     * high nibble min), qs[64] @20 (2 bits, 4 per byte) */
    const size_t bs = 256, bb = 84, bpr = in_dim / bs;
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * bpr * bb;
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            size_t boff = row_off + b * bb;
            float d = le_f16(w + boff);
            float dmin = le_f16(w + boff + 2);
            const uint8_t* sc = w + boff + 4;
            const uint8_t* qs = w + boff + 20;
            size_t xb = b * bs;
            for (size_t sb = 0; sb < 16; sb++) {
                float scale = d * (float)(sc[sb] & 0x0F);
                float min_val = dmin * (float)((sc[sb] >> 4) & 0x0F);
                for (size_t j = 0; j < 16; j++) {
                    size_t idx = sb * 16 + j;
                    float q = (float)((qs[idx / 4] >> ((idx % 4) * 2)) & 0x03);
                    sum += (scale * q - min_val) * x[xb + idx];
                }
            }
        }
        y[row] = sum;
    }
}

static inline float le_f32(const uint8_t* p) {
    uint32_t bits = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) |
                    ((uint32_t)p[3] << 24);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static void mv_q8_k(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                    float* y) {
    /* src/metal/compute.rs:971-993: d f32 @0, int8 qs[256] @4, bsums unused */
    const size_t bs = 256, bb = 292, bpr = in_dim / bs;
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * bpr * bb;
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            size_t boff = row_off + b * bb;
            float d = le_f32(w + boff);
            size_t xb = b * bs;
            for (size_t j = 0; j < 256; j++) sum += d * (float)(int8_t)w[boff + 4 + j] * x[xb + j];
        }
        y[row] = sum;
    }
}

/* IQ4_NL non-linear code book, src/metal/compute.rs:997-999 (a format constant) */
static const int8_t kIq4nl[16] = {-127, -104, -83, -65, -49, -35, -22, -10,
                                  1,    13,   25,  38,  53,  69,  89,  113};

static void mv_iq4_nl(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                      float* y) {
    /* src/metal/compute.rs:1004-1028: d f16 @0, qs[16] @2, elements 2j / 2j+1
     * from the low / high nibble of qs[j] through the code book */
    const size_t bs = 32, bb = 18, bpr = in_dim / bs;
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * bpr * bb;
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            size_t boff = row_off + b * bb;
            float d = le_f16(w + boff);
            size_t xb = b * bs;
            for (size_t j = 0; j < 16; j++) {
                uint8_t bv = w[boff + 2 + j];
                sum += d * (float)kIq4nl[bv & 0x0F] * x[xb + 2 * j];
                sum += d * (float)kIq4nl[(bv >> 4) & 0x0F] * x[xb + 2 * j + 1];
            }
        }
        y[row] = sum;
    }
}

static void mv_iq4_xs(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                      float* y) {
    /* src/metal/compute.rs:1034-1077: d f16 @0, scales_h u16 @2, scales_l u16[8]
     * @4 (sub-block sb: nibble sb%2 of word sb/2), qs[128] @20; scale =
     * (sl | sh << 4) - 32 */
    const size_t bs = 256, bb = 148, bpr = in_dim / bs;
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * bpr * bb;
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            size_t boff = row_off + b * bb;
            float d = le_f16(w + boff);
            unsigned scales_h = (unsigned)w[boff + 2] | ((unsigned)w[boff + 3] << 8);
            for (size_t sb = 0; sb < 8; sb++) {
                size_t sl_idx = sb / 2;
                unsigned sl_word = (unsigned)w[boff + 4 + sl_idx * 2] |
                                   ((unsigned)w[boff + 5 + sl_idx * 2] << 8);
                int sl = (sb % 2 == 0) ? (int)(sl_word & 0x0F) : (int)((sl_word >> 4) & 0x0F);
                int sh = (int)((scales_h >> (2 * sb)) & 0x03);
                float scale = (float)(sl | (sh << 4)) - 32.0f;
                size_t qs_off = boff + 20 + sb * 16;
                size_t xb = b * bs + sb * 32;
                for (size_t j = 0; j < 16; j++) {
                    uint8_t bv = w[qs_off + j];
                    sum += d * scale * (float)kIq4nl[bv & 0x0F] * x[xb + 2 * j];
                    sum += d * scale * (float)kIq4nl[(bv >> 4) & 0x0F] * x[xb + 2 * j + 1];
                }
            }
        }
        y[row] = sum;
    }
}

static void mv_f16(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                   float* y) {
    /* src/metal/compute.rs:2272-2285 */
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * in_dim * 2;
        float sum = 0.0f;
        for (size_t col = 0; col < in_dim; col++) sum += le_f16(w + row_off + col * 2) * x[col];
        y[row] = sum;
    }
}

static void mv_bf16(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                    float* y) {
    /* src/metal/compute.rs:2249-2269 */
    for (size_t row = r0; row < r1; row++) {
        size_t row_off = row * in_dim * 2;
        float sum = 0.0f;
        for (size_t col = 0; col < in_dim; col++) {
            const uint8_t* p = w + row_off + col * 2;
            sum += ssdo_bf16_to_f32((uint16_t)(p[0] | ((uint16_t)p[1] << 8))) * x[col];
        }
        y[row] = sum;
    }
}

/* KSIGNS_IQ2XS (compute.rs:1964-1973): the 7-bit index with bit 7 set to its
 * parity, so every mask has an even number of negative signs */
static inline unsigned ksigns(unsigned i) { return i | ((unsigned)(__builtin_popcount(i) & 1) << 7); }
static inline float sgn(unsigned mask, unsigned j) { return (mask >> j) & 1u ? -1.0f : 1.0f; }
static inline unsigned le_u32(const uint8_t* p) {
    return (unsigned)p[0] | ((unsigned)p[1] << 8) | ((unsigned)p[2] << 16) | ((unsigned)p[3] << 24);
}
static inline unsigned gbyte(uint64_t v, unsigned j) { return (unsigned)(v >> (8 * j)) & 0xFFu; }

/* Element values of one 256-element block of the IQ2 / IQ3 types, as the
 * matvecs below form them before the multiply by x (one product per element,
 * in the reference's operand order db * grid * sign). */
static void iq_block_elements(int dtype, const uint8_t* p, float* e) {
    float d = le_f16(p);
    for (unsigned ib32 = 0; ib32 < 8; ib32++) {
        float* o = e + ib32 * 32;
        if (dtype == SSDO_IQ2_XXS) { /* compute.rs:2137-2182 */
            const uint8_t* g = p + 2 + ib32 * 8;
            unsigned a0 = le_u32(g), a1 = le_u32(g + 4);
            float db = d * (0.5f + (float)(a1 >> 28)) * 0.25f;
            for (unsigned l = 0; l < 4; l++) {
                uint64_t gr = ssdq_iq2xxs_grid[(a0 >> (8 * l)) & 0xFF];
                unsigned sg = ksigns((a1 >> (7 * l)) & 127);
                for (unsigned j = 0; j < 8; j++) o[l * 8 + j] = db * (float)gbyte(gr, j) * sgn(sg, j);
            }
        } else if (dtype == SSDO_IQ2_XS) { /* compute.rs:2192-2238 */
            unsigned sbyte = p[2 + 64 + ib32 / 2];
            unsigned nib = (ib32 % 2 == 0) ? (sbyte & 0x0F) : (sbyte >> 4);
            float db = d * (0.5f + (float)nib) * 0.25f;
            for (unsigned l = 0; l < 4; l++) {
                const uint8_t* q = p + 2 + (ib32 * 4 + l) * 2;
                unsigned qv = (unsigned)q[0] | ((unsigned)q[1] << 8);
                uint64_t gr = ssdq_iq2xs_grid[qv & 511];
                unsigned sg = ksigns(qv >> 9);
                for (unsigned j = 0; j < 8; j++) o[l * 8 + j] = db * (float)gbyte(gr, j) * sgn(sg, j);
            }
        } else if (dtype == SSDO_IQ3_XXS) { /* compute.rs:1983-2034 */
            unsigned aux = le_u32(p + 2 + 64 + ib32 * 4);
            float db = d * (0.5f + (float)(aux >> 28)) * 0.5f;
            for (unsigned l = 0; l < 4; l++) {
                unsigned sg = ksigns((aux >> (7 * l)) & 127);
                uint32_t g1 = ssdq_iq3xxs_grid[p[2 + ib32 * 8 + 2 * l]];
                uint32_t g2 = ssdq_iq3xxs_grid[p[2 + ib32 * 8 + 2 * l + 1]];
                for (unsigned j = 0; j < 4; j++) {
                    o[l * 8 + j] = db * (float)gbyte(g1, j) * sgn(sg, j);
                    o[l * 8 + j + 4] = db * (float)gbyte(g2, j) * sgn(sg, j + 4);
                }
            }
        } else { /* SSDO_IQ3_S, compute.rs:2042-2128 */
            unsigned sbyte = p[2 + 64 + 8 + 32 + ib32 / 2];
            float db = d * (float)(1 + 2 * (int)((ib32 % 2 == 0) ? (sbyte & 0x0F) : (sbyte >> 4)));
            unsigned qh = p[2 + 64 + ib32];
            for (unsigned l = 0; l < 4; l++) {
                unsigned i1 = p[2 + ib32 * 8 + 2 * l] | ((qh << (8 - 2 * l)) & 256);
                unsigned i2 = p[2 + ib32 * 8 + 2 * l + 1] | ((qh << (7 - 2 * l)) & 256);
                uint32_t g1 = ssdq_iq3s_grid[i1], g2 = ssdq_iq3s_grid[i2];
                unsigned sg = p[2 + 64 + 8 + ib32 * 4 + l];
                for (unsigned j = 0; j < 4; j++) {
                    o[l * 8 + j] = db * (float)gbyte(g1, j) * sgn(sg, j);
                    o[l * 8 + j + 4] = db * (float)gbyte(g2, j) * sgn(sg, j + 4);
                }
            }
        }
    }
}

/* The four IQ2 / IQ3 matvecs: the serial sum of element * x (sum += db * grid *
 * sign * x, compute.rs:1983-2238), in the reference's order: element order for
 * IQ2, and j, j+4 alternating within each group of 8 for IQ3 (its two grid
 * words are consumed together). */
/* GCC's -O3 tree vectorizer was seen to change the result of the alternating
 * IQ3 sum below (a serial fp32 chain it may not reorder; correct at -O2 and
 * with -fno-tree-vectorize), so this function is built without it. */
__attribute__((optimize("no-tree-vectorize")))
static void mv_iq_lattice(int dtype, const uint8_t* w, const float* x, size_t r0, size_t r1, size_t in_dim,
                          float* y) {
    const size_t bb = ssdo_type_size(dtype), bpr = in_dim / 256;
    float e[256];
    for (size_t row = r0; row < r1; row++) {
        float sum = 0.0f;
        for (size_t b = 0; b < bpr; b++) {
            iq_block_elements(dtype, w + (row * bpr + b) * bb, e);
            if (dtype == SSDO_IQ3_XXS || dtype == SSDO_IQ3_S) {
                for (size_t g8 = 0; g8 < 256; g8 += 8)
                    for (size_t j = 0; j < 4; j++) {
                        sum += e[g8 + j] * x[b * 256 + g8 + j];
                        sum += e[g8 + j + 4] * x[b * 256 + g8 + j + 4];
                    }
            } else {
                for (size_t j = 0; j < 256; j++) sum += e[j] * x[b * 256 + j];
            }
        }
        y[row] = sum;
    }
}
static void mv_iq2_xxs(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t k, float* y) {
    mv_iq_lattice(SSDO_IQ2_XXS, w, x, r0, r1, k, y);
}
static void mv_iq2_xs(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t k, float* y) {
    mv_iq_lattice(SSDO_IQ2_XS, w, x, r0, r1, k, y);
}
static void mv_iq3_xxs(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t k, float* y) {
    mv_iq_lattice(SSDO_IQ3_XXS, w, x, r0, r1, k, y);
}
static void mv_iq3_s(const uint8_t* w, const float* x, size_t r0, size_t r1, size_t k, float* y) {
    mv_iq_lattice(SSDO_IQ3_S, w, x, r0, r1, k, y);
}

typedef void (*mv_fn)(const uint8_t*, const float*, size_t, size_t, size_t, float*);

static mv_fn pick_mv(int dtype) {
    /* matvec_quantized_cpu dispatch, src/metal/compute.rs:648-677 */
    switch (dtype) {
        case SSDO_Q4_0: return mv_q4_0;
        case SSDO_Q4_K: return mv_q4_k;
        case SSDO_Q6_K: return mv_q6_k;
        case SSDO_Q8_0: return mv_q8_0;
        case SSDO_Q3_K: return mv_q3_k;
        case SSDO_Q5_K: return mv_q5_k;
        case SSDO_Q2_K: return mv_q2_k;
        case SSDO_Q8_K: return mv_q8_k;
        case SSDO_IQ4_NL: return mv_iq4_nl;
        case SSDO_IQ4_XS: return mv_iq4_xs;
        case SSDO_BF16: return mv_bf16;
        case SSDO_F16: return mv_f16;
        case SSDO_IQ2_XXS: return mv_iq2_xxs;
        case SSDO_IQ2_XS: return mv_iq2_xs;
        case SSDO_IQ3_XXS: return mv_iq3_xxs;
        case SSDO_IQ3_S: return mv_iq3_s;
        default: return NULL;
    }
}

int ssdo_matvec_quantized(const uint8_t* w, const float* x, size_t out_dim, size_t in_dim,
                          int dtype, float* y) {
    mv_fn f = pick_mv(dtype);
    if (!f) {
        for (size_t i = 0; i < out_dim; i++) y[i] = 0.0f; /* compute.rs:672-675 */
        return 1;
    }
    f(w, x, 0, out_dim, in_dim, y);
    return 0;
}

typedef struct {
    mv_fn f;
    const uint8_t* w;
    const float* x;
    size_t r0, r1, in_dim;
    float* y;
} mv_job;

static void* mv_worker(void* p) {
    mv_job* j = (mv_job*)p;
    j->f(j->w, j->x, j->r0, j->r1, j->in_dim, j->y);
    return NULL;
}

int ssdo_matvec_quantized_mt(const uint8_t* w, const float* x, size_t out_dim, size_t in_dim,
                             int dtype, float* y, int nthreads) {
    /* Row shards like src/inference/tensor_parallel.rs:45-96 */
    mv_fn f = pick_mv(dtype);
    if (!f) return ssdo_matvec_quantized(w, x, out_dim, in_dim, dtype, y);
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > out_dim) nthreads = (int)(out_dim ? out_dim : 1);
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    mv_job* jobs = (mv_job*)calloc((size_t)nthreads, sizeof(mv_job));
    size_t chunk = (out_dim + (size_t)nthreads - 1) / (size_t)nthreads;
    for (int t = 0; t < nthreads; t++) {
        size_t r0 = (size_t)t * chunk, r1 = r0 + chunk;
        if (r0 > out_dim) r0 = out_dim;
        if (r1 > out_dim) r1 = out_dim;
        jobs[t] = (mv_job){f, w, x, r0, r1, in_dim, y};
        pthread_create(&th[t], NULL, mv_worker, &jobs[t]);
    }
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
    return 0;
}

/* Element values of one row as the matvec functions above form them before the
 * multiply by x (for the exact sums; the dequant path covers the other types). */
static void row_elements(int dtype, const uint8_t* r, size_t row_bytes, size_t k, float* e) {
    size_t bpr = k / 256;
    switch (dtype) {
        case SSDO_Q3_K:
            for (size_t b = 0; b < bpr; b++) {
                const uint8_t* p = r + b * 110;
                float d = le_f16(p + 108);
                for (size_t sb = 0; sb < 16; sb++) {
                    unsigned low4 = (p[96 + sb / 2] >> ((sb & 1) * 4)) & 0x0Fu;
                    unsigned hi2 = (p[104 + sb / 4] >> ((sb % 4) * 2)) & 0x03u;
                    int sv = (int)(low4 | (hi2 << 4));
                    if (sv >= 32) sv -= 64;
                    float sc_f = d * (float)sv;
                    for (size_t j = 0; j < 16; j++) {
                        size_t idx = sb * 16 + j;
                        unsigned low2 = (p[32 + idx / 4] >> ((idx % 4) * 2)) & 0x03u;
                        unsigned hbit = (p[idx / 8] >> (idx % 8)) & 1u;
                        e[b * 256 + idx] = sc_f * (float)((int)(low2 | (hbit << 2)) - 4);
                    }
                }
            }
            return;
        case SSDO_Q5_K:
            for (size_t b = 0; b < bpr; b++) {
                const uint8_t* p = r + b * 176;
                float d = le_f16(p), dmin = le_f16(p + 2);
                for (unsigned sb = 0; sb < 8; sb++) {
                    unsigned sv, mv;
                    q4k_scale_min(p + 4, sb, &sv, &mv);
                    float scale = d * (float)sv, min_val = dmin * (float)mv;
                    for (size_t j = 0; j < 32; j++) {
                        size_t idx = sb * 32 + j;
                        uint8_t bv = p[48 + sb * 16 + j / 2];
                        unsigned lo = (j & 1) ? ((bv >> 4) & 0x0Fu) : (bv & 0x0Fu);
                        unsigned hb = (p[16 + idx / 8] >> (idx % 8)) & 1u;
                        e[b * 256 + idx] = scale * (float)(lo | (hb << 4)) - min_val;
                    }
                }
            }
            return;
        case SSDO_Q2_K:
            for (size_t b = 0; b < bpr; b++) {
                const uint8_t* p = r + b * 84;
                float d = le_f16(p), dmin = le_f16(p + 2);
                for (size_t sb = 0; sb < 16; sb++) {
                    float scale = d * (float)(p[4 + sb] & 0x0F);
                    float min_val = dmin * (float)((p[4 + sb] >> 4) & 0x0F);
                    for (size_t j = 0; j < 16; j++) {
                        size_t idx = sb * 16 + j;
                        float q = (float)((p[20 + idx / 4] >> ((idx % 4) * 2)) & 0x03);
                        e[b * 256 + idx] = scale * q - min_val;
                    }
                }
            }
            return;
        case SSDO_Q8_K:
            for (size_t b = 0; b < bpr; b++) {
                float d = le_f32(r + b * 292);
                for (size_t j = 0; j < 256; j++) e[b * 256 + j] = d * (float)(int8_t)r[b * 292 + 4 + j];
            }
            return;
        case SSDO_IQ4_NL:
            for (size_t b = 0; b < k / 32; b++) {
                const uint8_t* p = r + b * 18;
                float d = le_f16(p);
                for (size_t j = 0; j < 16; j++) {
                    e[b * 32 + 2 * j] = d * (float)kIq4nl[p[2 + j] & 0x0F];
                    e[b * 32 + 2 * j + 1] = d * (float)kIq4nl[(p[2 + j] >> 4) & 0x0F];
                }
            }
            return;
        case SSDO_IQ4_XS:
            for (size_t b = 0; b < bpr; b++) {
                const uint8_t* p = r + b * 148;
                float d = le_f16(p);
                unsigned sh_all = (unsigned)p[2] | ((unsigned)p[3] << 8);
                for (size_t sb = 0; sb < 8; sb++) {
                    unsigned slw = (unsigned)p[4 + (sb / 2) * 2] | ((unsigned)p[5 + (sb / 2) * 2] << 8);
                    int sl = (sb % 2 == 0) ? (int)(slw & 0x0F) : (int)((slw >> 4) & 0x0F);
                    int sh = (int)((sh_all >> (2 * sb)) & 0x03);
                    float scale = (float)(sl | (sh << 4)) - 32.0f;
                    for (size_t j = 0; j < 16; j++) {
                        uint8_t bv = p[20 + sb * 16 + j];
                        e[b * 256 + sb * 32 + 2 * j] = d * scale * (float)kIq4nl[bv & 0x0F];
                        e[b * 256 + sb * 32 + 2 * j + 1] = d * scale * (float)kIq4nl[(bv >> 4) & 0x0F];
                    }
                }
            }
            return;
        case SSDO_IQ2_XXS: case SSDO_IQ2_XS: case SSDO_IQ3_XXS: case SSDO_IQ3_S:
            for (size_t b = 0; b < bpr; b++) iq_block_elements(dtype, r + b * ssdo_type_size(dtype), e + b * 256);
            return;
        default:
            ssdo_dequantize_to_f32(dtype, r, row_bytes, k, e);
    }
}

int ssdo_matvec_elements(const uint8_t* w, size_t out_dim, size_t in_dim, int dtype, float* e) {
    size_t bs = ssdo_block_size(dtype), tb = ssdo_type_size(dtype);
    if (!pick_mv(dtype)) return 1;
    size_t bpr = in_dim / bs, k = bpr * bs, row_bytes = bpr * tb;
    for (size_t r = 0; r < out_dim; r++) row_elements(dtype, w + r * row_bytes, row_bytes, k, e + r * k);
    return 0;
}

int ssdo_matvec_exact(const uint8_t* w, const float* x, size_t out_dim, size_t in_dim, int dtype,
                      double* y) {
    size_t bs = ssdo_block_size(dtype), tb = ssdo_type_size(dtype);
    if (!pick_mv(dtype)) {
        for (size_t i = 0; i < out_dim; i++) y[i] = 0.0;
        return 1;
    }
    size_t bpr = in_dim / bs, k = bpr * bs, row_bytes = bpr * tb;
    float* e = (float*)malloc(k * sizeof(float));
    for (size_t r = 0; r < out_dim; r++) {
        row_elements(dtype, w + r * row_bytes, row_bytes, k, e);
        double s = 0.0;
        for (size_t i = 0; i < k; i++) s += (double)e[i] * (double)x[i];
        y[r] = s;
    }
    free(e);
    return 0;
}

/* ---------------------------------------------------------------- INT8 KV */

void ssdo_quantize_rows_int8(const float* data, size_t n_rows, size_t dim, int8_t* codes,
                             float* scales) {
    /* src/ssd/block_swap.rs:36-60 (== quantized_kv_cache.rs:23-41) */
    for (size_t row = 0; row < n_rows; row++) {
        const float* r = data + row * dim;
        int8_t* c = codes + row * dim;
        float absmax = 0.0f;
        for (size_t i = 0; i < dim; i++) absmax = fmaxf(absmax, fabsf(r[i])); /* f32::max ignores NaN */
        if (absmax == 0.0f) {
            scales[row] = 0.0f;
            memset(c, 0, dim);
            continue;
        }
        float inv_scale = 127.0f / absmax;
        scales[row] = absmax / 127.0f;
        for (size_t i = 0; i < dim; i++) {
            float t = roundf(r[i] * inv_scale); /* f32::round: half away from zero */
            if (isnan(t)) {
                c[i] = 0; /* `as i8` saturates, NaN -> 0 */
            } else {
                if (t < -127.0f) t = -127.0f;
                if (t > 127.0f) t = 127.0f;
                c[i] = (int8_t)t;
            }
        }
    }
}

void ssdo_dequantize_rows_int8(const int8_t* codes, const float* scales, size_t n_rows,
                               size_t dim, float* out) {
    /* src/ssd/block_swap.rs:63-74 */
    for (size_t row = 0; row < n_rows; row++)
        for (size_t i = 0; i < dim; i++)
            out[row * dim + i] = (float)codes[row * dim + i] * scales[row];
}

/* -------------------------------------------------------------- attention */

/* One head of the online-softmax loop, src/inference/flash_attention.rs:76-139.
 * k_at / v_at produce the f32 key/value head vectors for a position. */
typedef struct {
    /* flattened f32 KV */
    const float* k;
    const float* v;
    size_t stride; /* n_head_kv*head_dim */
    /* paged int8 KV */
    const int8_t* kc;
    const float* ks;
    const int8_t* vc;
    const float* vs;
    const int32_t* table;
    size_t block_size;
    int paged;
} kv_src;

static void kv_fetch(const kv_src* s, size_t pos, size_t kv_h, size_t head_dim, float* kh,
                     float* vh) {
    if (!s->paged) {
        const float* kp = s->k + pos * s->stride + kv_h * head_dim;
        const float* vp = s->v + pos * s->stride + kv_h * head_dim;
        memcpy(kh, kp, head_dim * 4);
        memcpy(vh, vp, head_dim * 4);
        return;
    }
    /* physical_block_for_position, src/inference/paged_attention.rs:113-123 */
    size_t logical = pos / s->block_size, slot = pos % s->block_size;
    size_t phys = (size_t)s->table[logical];
    size_t row = phys * s->block_size + slot;
    /* PhysicalBlock layout [block_size, kv_dim], key_at offset
     * slot*kv_dim + kv_head*head_dim (paged_attention.rs:34-35, 72-76) */
    const int8_t* kc = s->kc + row * s->stride + kv_h * head_dim;
    const int8_t* vc = s->vc + row * s->stride + kv_h * head_dim;
    float ksc = s->ks[row], vsc = s->vs[row];
    /* QuantizedVec::dequantize_into, quantized_kv_cache.rs:49-53 */
    for (size_t d = 0; d < head_dim; d++) {
        kh[d] = (float)kc[d] * ksc;
        vh[d] = (float)vc[d] * vsc;
    }
}

static void attend_head(const float* qh, const kv_src* src, size_t kv_h, size_t head_dim,
                        size_t p0, size_t p1, float* out, float* kh, float* vh, float* acc) {
    float scale = 1.0f / sqrtf((float)head_dim); /* flash_attention.rs:70 */
    float running_max = -INFINITY, running_sum = 0.0f;
    for (size_t d = 0; d < head_dim; d++) acc[d] = 0.0f;
    size_t chunks = head_dim / 4, rem = head_dim % 4;
    for (size_t pos = p0; pos < p1; pos++) {
        kv_fetch(src, pos, kv_h, head_dim, kh, vh);
        float dot = 0.0f;
        for (size_t c = 0; c < chunks; c++) { /* 4-wide partial dot, flash_attention.rs:93-104 */
            size_t b = c * 4;
            dot += qh[b] * kh[b] + qh[b + 1] * kh[b + 1] + qh[b + 2] * kh[b + 2] +
                   qh[b + 3] * kh[b + 3];
        }
        for (size_t i = chunks * 4; i < chunks * 4 + rem; i++) dot += qh[i] * kh[i];
        float score = dot * scale;
        if (score > running_max) { /* flash_attention.rs:110-118 */
            float correction = expf(running_max - score);
            running_sum *= correction;
            for (size_t d = 0; d < head_dim; d++) acc[d] *= correction;
            running_max = score;
        }
        float weight = expf(score - running_max);
        running_sum += weight;
        for (size_t d = 0; d < head_dim; d++) acc[d] += weight * vh[d];
    }
    if (running_sum > 0.0f) { /* flash_attention.rs:128-137 */
        float inv_sum = 1.0f / running_sum;
        for (size_t d = 0; d < head_dim; d++) out[d] = acc[d] * inv_sum;
    } else {
        for (size_t d = 0; d < head_dim; d++) out[d] = 0.0f;
    }
}

void ssdo_flash_attention_f32(const float* q, const float* k, const float* v, size_t n_head,
                              size_t n_head_kv, size_t head_dim, size_t seq_len,
                              size_t window_start, size_t window_end, float* out) {
    kv_src src;
    memset(&src, 0, sizeof src);
    src.k = k;
    src.v = v;
    src.stride = n_head_kv * head_dim;
    size_t group = n_head_kv ? n_head / n_head_kv : 0;
    if (group < 1) group = 1; /* (n_head / n_head_kv).max(1), flash_attention.rs:71 */
    size_t end = window_end < seq_len ? window_end : seq_len;
    float* scratch = (float*)malloc(3 * head_dim * sizeof(float));
    for (size_t h = 0; h < n_head; h++)
        attend_head(q + h * head_dim, &src, h / group, head_dim, window_start, end,
                    out + h * head_dim, scratch, scratch + head_dim, scratch + 2 * head_dim);
    free(scratch);
}

typedef struct {
    const float* q;
    kv_src base;
    const int32_t* block_tables;
    const int32_t* ctx_lens;
    size_t n_head, group, head_dim, max_blocks;
    size_t u0, u1; /* units = seq*n_head + h */
    float* out;
    const int32_t* win_lo; /* optional per-sequence window (NULL: 0 / no bound) */
    const int32_t* win_hi;
} attn_job;

static void* attn_worker(void* p) {
    attn_job* j = (attn_job*)p;
    float* scratch = (float*)malloc(3 * j->head_dim * sizeof(float));
    for (size_t u = j->u0; u < j->u1; u++) {
        size_t s = u / j->n_head, h = u % j->n_head;
        kv_src src = j->base;
        src.table = j->block_tables + s * j->max_blocks;
        size_t ctx = j->ctx_lens[s] > 0 ? (size_t)j->ctx_lens[s] : 0;
        /* flash_attention_windowed, flash_attention.rs:176 and 187:
         * positions window_start .. min(window_end, seq_len), empty when the
         * start is past the end (attend_head then writes zeros) */
        size_t p0 = 0, p1 = ctx;
        if (j->win_lo && j->win_lo[s] > 0) p0 = (size_t)j->win_lo[s];
        if (j->win_hi) p1 = j->win_hi[s] > 0 ? ((size_t)j->win_hi[s] < ctx ? (size_t)j->win_hi[s] : ctx) : 0;
        if (p0 > p1) p0 = p1;
        attend_head(j->q + u * j->head_dim, &src, h / j->group, j->head_dim, p0, p1,
                    j->out + u * j->head_dim, scratch, scratch + j->head_dim,
                    scratch + 2 * j->head_dim);
    }
    free(scratch);
    return NULL;
}

void ssdo_paged_attention_int8_window_mt(const float* q, const int8_t* k_codes, const float* k_scales,
                                         const int8_t* v_codes, const float* v_scales,
                                         const int32_t* block_tables, const int32_t* ctx_lens,
                                         const int32_t* window_starts, const int32_t* window_ends,
                                         size_t n_seq, size_t n_head, size_t n_head_kv, size_t head_dim,
                                         size_t block_size, size_t max_blocks_per_seq, float* out,
                                         int nthreads) {
    kv_src base;
    memset(&base, 0, sizeof base);
    base.paged = 1;
    base.kc = k_codes;
    base.ks = k_scales;
    base.vc = v_codes;
    base.vs = v_scales;
    base.stride = n_head_kv * head_dim;
    base.block_size = block_size;
    size_t group = n_head_kv ? n_head / n_head_kv : 0;
    if (group < 1) group = 1;
    size_t units = n_seq * n_head;
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > units) nthreads = (int)(units ? units : 1);
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    attn_job* jobs = (attn_job*)calloc((size_t)nthreads, sizeof(attn_job));
    size_t chunk = (units + (size_t)nthreads - 1) / (size_t)nthreads;
    for (int t = 0; t < nthreads; t++) {
        size_t u0 = (size_t)t * chunk, u1 = u0 + chunk;
        if (u0 > units) u0 = units;
        if (u1 > units) u1 = units;
        jobs[t] = (attn_job){q, base, block_tables, ctx_lens, n_head, group, head_dim,
                             max_blocks_per_seq, u0, u1, out, window_starts, window_ends};
        if (nthreads == 1)
            attn_worker(&jobs[t]);
        else
            pthread_create(&th[t], NULL, attn_worker, &jobs[t]);
    }
    if (nthreads > 1)
        for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

void ssdo_paged_attention_int8_mt(const float* q, const int8_t* k_codes, const float* k_scales,
                                  const int8_t* v_codes, const float* v_scales,
                                  const int32_t* block_tables, const int32_t* ctx_lens,
                                  size_t n_seq, size_t n_head, size_t n_head_kv, size_t head_dim,
                                  size_t block_size, size_t max_blocks_per_seq, float* out,
                                  int nthreads) {
    ssdo_paged_attention_int8_window_mt(q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens,
                                        NULL, NULL, n_seq, n_head, n_head_kv, head_dim, block_size,
                                        max_blocks_per_seq, out, nthreads);
}

void ssdo_paged_attention_int8(const float* q, const int8_t* k_codes, const float* k_scales,
                               const int8_t* v_codes, const float* v_scales,
                               const int32_t* block_tables, const int32_t* ctx_lens,
                               size_t n_seq, size_t n_head, size_t n_head_kv, size_t head_dim,
                               size_t block_size, size_t max_blocks_per_seq, float* out) {
    ssdo_paged_attention_int8_mt(q, k_codes, k_scales, v_codes, v_scales, block_tables, ctx_lens,
                                 n_seq, n_head, n_head_kv, head_dim, block_size,
                                 max_blocks_per_seq, out, 1);
}

/* -------------------------------------------------------------------- GEMM */

typedef struct {
    const uint8_t* w;
    const uint16_t* x;
    size_t N, K, t0, t1;
    float* y;
    double* yd;
} gemm_job;

static void* gemm_worker(void* p) {
    gemm_job* j = (gemm_job*)p;
    float* xf = (float*)malloc(j->K * sizeof(float));
    for (size_t t = j->t0; t < j->t1; t++) {
        for (size_t i = 0; i < j->K; i++) xf[i] = ssdo_bf16_to_f32(j->x[t * j->K + i]);
        if (j->y)
            mv_q4_k(j->w, xf, 0, j->N, j->K, j->y + t * j->N);
        else
            ssdo_matvec_exact(j->w, xf, j->N, j->K, SSDO_Q4_K, j->yd + t * j->N);
    }
    free(xf);
    return NULL;
}

static void gemm_run(const uint8_t* w, const uint16_t* x, size_t M, size_t N, size_t K, float* y,
                     double* yd, int nthreads) {
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > M) nthreads = (int)(M ? M : 1);
    pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
    gemm_job* jobs = (gemm_job*)calloc((size_t)nthreads, sizeof(gemm_job));
    size_t chunk = (M + (size_t)nthreads - 1) / (size_t)nthreads;
    for (int t = 0; t < nthreads; t++) {
        size_t t0 = (size_t)t * chunk, t1 = t0 + chunk;
        if (t0 > M) t0 = M;
        if (t1 > M) t1 = M;
        jobs[t] = (gemm_job){w, x, N, K, t0, t1, y, yd};
        pthread_create(&th[t], NULL, gemm_worker, &jobs[t]);
    }
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    free(th);
    free(jobs);
}

void ssdo_gemm_q4k_bf16(const uint8_t* w, const uint16_t* x, size_t M, size_t N, size_t K,
                        float* y, int nthreads) {
    gemm_run(w, x, M, N, K, y, NULL, nthreads);
}

void ssdo_gemm_q4k_bf16_exact(const uint8_t* w, const uint16_t* x, size_t M, size_t N, size_t K,
                              double* y, int nthreads) {
    gemm_run(w, x, M, N, K, NULL, y, nthreads);
}

/* ------------------------------------------------- decode-layer f32 ops */

void ssdo_rope_multi_head(float* x, size_t len, size_t head_dim, size_t n_heads, size_t position,
                          float theta_base) {
    /* rope_f32_multi_head, src/metal/compute.rs:482-507 (f32 powf / sin_cos
     * are libm's on this platform, as for the reference's Rust build) */
    size_t half_dim = head_dim / 2;
    for (size_t h = 0; h < n_heads; h++) {
        size_t base = h * head_dim;
        for (size_t i = 0; i < half_dim; i++) {
            float freq = 1.0f / powf(theta_base, 2.0f * (float)i / (float)head_dim);
            float angle = (float)position * freq;
            float sin_val = sinf(angle), cos_val = cosf(angle);
            size_t idx0 = base + i * 2, idx1 = idx0 + 1;
            if (idx1 < len) {
                float x0 = x[idx0], x1 = x[idx1];
                x[idx0] = x0 * cos_val - x1 * sin_val;
                x[idx1] = x0 * sin_val + x1 * cos_val;
            }
        }
    }
}

void ssdo_silu(float* x, size_t n) {
    /* silu_f32, src/metal/compute.rs:641-645 */
    for (size_t i = 0; i < n; i++) x[i] = x[i] / (1.0f + expf(-x[i]));
}

static float sum_sq(const float* x, size_t n) {
    float s = 0.0f; /* Iterator::sum: a serial fold from 0 */
    for (size_t i = 0; i < n; i++) s += x[i] * x[i];
    return s;
}

void ssdo_rmsnorm(float* x, const float* w, size_t n, float eps) {
    /* rmsnorm_f32_fast_scalar, src/metal/compute.rs:580-589: x *= inv_rms * w */
    float inv_rms = 1.0f / sqrtf(sum_sq(x, n) / (float)n + eps);
    for (size_t i = 0; i < n; i++) x[i] *= inv_rms * w[i];
}

void ssdo_fused_post_attn_norm(float* hidden, const float* attn, const float* w, size_t n,
                               float eps, float* out) {
    /* fused_post_attn_norm_f32_cpu, src/metal/compute.rs:536-555:
     * hidden += attn; out = hidden * inv_rms * w */
    for (size_t i = 0; i < n; i++) hidden[i] += attn[i];
    float inv_rms = 1.0f / sqrtf(sum_sq(hidden, n) / (float)n + eps);
    for (size_t i = 0; i < n; i++) out[i] = hidden[i] * inv_rms * w[i];
}

int ssdo_fused_rmsnorm_linear(int dtype, const uint8_t* w, const float* x, const float* norm_w,
                              size_t vocab, size_t n_embd, float* y) {
    /* fused_rmsnorm_linear_f32_cpu, src/metal/compute.rs:557-578, with the
     * projection through matvec_quantized_cpu: eps is fixed at 1e-5 there */
    float inv_rms = 1.0f / sqrtf(sum_sq(x, n_embd) / (float)n_embd + 1e-5f);
    float* xn = (float*)malloc((n_embd ? n_embd : 1) * sizeof(float));
    for (size_t i = 0; i < n_embd; i++) xn[i] = x[i] * inv_rms * norm_w[i];
    int rc = ssdo_matvec_quantized(w, xn, vocab, n_embd, dtype, y);
    free(xn);
    return rc;
}

/* ------------------------------------------------ INT8 KV swap slots */

size_t ssdo_kv_slot_bytes(size_t block_size, size_t kv_dim) {
    /* SwapFile::with_quant_mode, Int8 (src/ssd/block_swap.rs:148-170):
     * keys + values i8, one f32 scale per key row and per value row, num_filled u32 */
    return block_size * kv_dim * 2 + block_size * 2 * 4 + 4;
}

void ssdo_kv_swap_write(const float* keys, const float* values, size_t block_size, size_t kv_dim,
                        uint32_t num_filled, uint8_t* slot) {
    /* SwapFile::write_block, Int8 (block_swap.rs:187-252): quantize_vectors_int8
     * of keys and of values (rows of kv_dim), then codes K, codes V, scales K,
     * scales V, num_filled little-endian */
    size_t n = block_size * kv_dim;
    int8_t* kc = (int8_t*)slot;
    int8_t* vc = (int8_t*)(slot + n);
    float* ks = (float*)malloc(block_size * sizeof(float));
    float* vs = (float*)malloc(block_size * sizeof(float));
    ssdo_quantize_rows_int8(keys, block_size, kv_dim, kc, ks);
    ssdo_quantize_rows_int8(values, block_size, kv_dim, vc, vs);
    memcpy(slot + 2 * n, ks, block_size * 4);
    memcpy(slot + 2 * n + block_size * 4, vs, block_size * 4);
    for (int i = 0; i < 4; i++) slot[2 * n + block_size * 8 + i] = (uint8_t)(num_filled >> (8 * i));
    free(ks);
    free(vs);
}

void ssdo_kv_swap_read(const uint8_t* slot, size_t block_size, size_t kv_dim, float* keys, float* values,
                       uint32_t* num_filled) {
    /* SwapFile::read_block, Int8 (block_swap.rs:283-370): dequantize_vectors_int8 */
    size_t n = block_size * kv_dim;
    float* ks = (float*)malloc(block_size * sizeof(float));
    float* vs = (float*)malloc(block_size * sizeof(float));
    memcpy(ks, slot + 2 * n, block_size * 4);
    memcpy(vs, slot + 2 * n + block_size * 4, block_size * 4);
    ssdo_dequantize_rows_int8((const int8_t*)slot, ks, block_size, kv_dim, keys);
    ssdo_dequantize_rows_int8((const int8_t*)(slot + n), vs, block_size, kv_dim, values);
    const uint8_t* p = slot + 2 * n + block_size * 8;
    *num_filled = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    free(ks);
    free(vs);
}
