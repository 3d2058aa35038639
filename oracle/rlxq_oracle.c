/*
 * rlxq_oracle.c -- CPU restatement of rlx-models' quantized-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY (see rlxq_oracle.h).  Built with
 * -ffp-contract=off so that every multiply-add below rounds exactly where the
 * restated reference code rounds; explicit fmaf() marks the places where the
 * reference itself calls f32::mul_add.
 */
#include "rlxq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define QK 32
#define QKK 256 /* Q4_K super-block */

/* ------------------------------------------------------------------------ */
/* Scalar conversions                                                        */
/* ------------------------------------------------------------------------ */

static uint32_t f2u(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    return u;
}
static float u2f(uint32_t u) {
    float v;
    memcpy(&v, &u, 4);
    return v;
}

/* IEEE binary32 -> binary16, round to nearest even, with subnormals, the
 * conversion `half::f16::from_f32` performs (the reference writes every GGUF
 * scale through it, e.g. crates/rlx-flint/src/quant.rs:91). */
uint16_t orc_f32_to_f16(float v) {
    uint32_t x = f2u(v);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) {
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    uint32_t e = ax >> 23;
    int he = (int)e - 127 + 15;
    if (he >= 1) {
        uint32_t m = ax & 0x7fffffu;
        uint32_t h = ((uint32_t)he << 10) | (m >> 13);
        uint32_t rem = m & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        if (h >= 0x7c00u) h = 0x7c00u;
        return (uint16_t)(sign | h);
    }
    int shift = 126 - (int)e;
    if (shift > 24) return (uint16_t)sign;
    uint32_t m = (ax & 0x7fffffu) | 0x800000u;
    uint32_t h = m >> shift;
    uint32_t rem = m & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu;
    uint32_t m = h & 0x3ffu;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        if (m == 0) return u2f(sign);
        /* subnormal: m * 2^-24, exact in f32 */
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* f32 -> bf16, round to nearest even, NaN kept quiet (`half::bf16::from_f32`,
 * crates/rlx-diffusiongemma/tests/real_layer_precision.rs:89-92). */
uint16_t orc_f32_to_bf16(float v) {
    uint32_t x = f2u(v);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

/* bf16 -> f32 is a 16-bit shift (crates/rlx-moshi/src/mlx_dequant.rs:79-81). */
float orc_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

void orc_f32_to_f16_n(const float* s, int64_t n, uint16_t* d) {
    for (int64_t i = 0; i < n; i++) d[i] = orc_f32_to_f16(s[i]);
}
void orc_f16_to_f32_n(const uint16_t* s, int64_t n, float* d) {
    for (int64_t i = 0; i < n; i++) d[i] = orc_f16_to_f32(s[i]);
}
void orc_f32_to_bf16_n(const float* s, int64_t n, uint16_t* d) {
    for (int64_t i = 0; i < n; i++) d[i] = orc_f32_to_bf16(s[i]);
}
void orc_bf16_to_f32_n(const uint16_t* s, int64_t n, float* d) {
    for (int64_t i = 0; i < n; i++) d[i] = orc_bf16_to_f32(s[i]);
}

static float rd_f16(const uint8_t* p) { return orc_f16_to_f32((uint16_t)(p[0] | (p[1] << 8))); }
static void wr_f16(uint8_t* p, float v) {
    uint16_t h = orc_f32_to_f16(v);
    p[0] = (uint8_t)(h & 0xff);
    p[1] = (uint8_t)(h >> 8);
}

/* ------------------------------------------------------------------------ */
/* GGUF legacy block codecs                                                  */
/* ------------------------------------------------------------------------ */

/* Block sizes: Q8_0 = f16 d + 32 x i8 (crates/rlx-flint/src/quant.rs:72-77),
 * Q4_0 = f16 d + 16 nibble bytes (same lines), Q4_1 = f16 d + f16 m + 16
 * nibble bytes (GGML block_q4_1; QuantScheme::GgufQ4_1,
 * crates/rlx-models-core/src/weight_loader.rs:508). */
int64_t orc_block_bytes(int scheme) {
    switch (scheme) {
        case ORC_GGUF_Q8_0: return 2 + QK;
        case ORC_GGUF_Q4_0: return 2 + QK / 2;
        case ORC_GGUF_Q4_1: return 4 + QK / 2;
        case ORC_GGUF_Q4_K: return 2 + 2 + 12 + QKK / 2;
        case ORC_GGUF_Q6_K: return QKK / 2 + QKK / 4 + QKK / 16 + 2;
        case ORC_GGUF_Q5_K: return 2 + 2 + 12 + QKK / 8 + QKK / 2;
        case ORC_GGUF_Q3_K: return QKK / 8 + QKK / 4 + 12 + 2;
        case ORC_GGUF_Q2_K: return QKK / 16 + QKK / 4 + 2 + 2;
        case ORC_GGUF_Q8_K: return 4 + QKK + 2 * (QKK / 16);
        default: return -1;
    }
}

static int is_kquant(int scheme) {
    return scheme == ORC_GGUF_Q4_K || scheme == ORC_GGUF_Q6_K || scheme == ORC_GGUF_Q5_K ||
           scheme == ORC_GGUF_Q3_K || scheme == ORC_GGUF_Q2_K || scheme == ORC_GGUF_Q8_K;
}

int64_t orc_block_len(int scheme) { return is_kquant(scheme) ? QKK : QK; }

int64_t orc_row_bytes(int scheme, int64_t k) {
    int64_t bb = orc_block_bytes(scheme), len = orc_block_len(scheme);
    if (bb < 0 || k % len) return -1;
    return k / len * bb;
}

/* Rust `f32::round`: half away from zero (C roundf). */
static float rnd_away(float v) { return roundf(v); }

/* Q8_0 encoder: crates/rlx-flint/src/quant.rs:86-95. */
static void quant_q8_0_block(const float* x, uint8_t* out) {
    float amax = 0.f;
    for (int i = 0; i < QK; i++) {
        float a = fabsf(x[i]);
        if (a > amax) amax = a;
    }
    float d = amax / 127.0f;
    float inv = d == 0.0f ? 0.0f : 1.0f / d;
    wr_f16(out, d);
    for (int i = 0; i < QK; i++) {
        float q = rnd_away(x[i] * inv);
        if (q < -127.f) q = -127.f;
        if (q > 127.f) q = 127.f;
        out[2 + i] = (uint8_t)(int8_t)q;
    }
}

/* Q4_0 encoder: crates/rlx-flint/src/quant.rs:97-110 (signed extreme, d =
 * max / -8, q = (v*inv + 8.5) truncated, clamped to 0..15). */
static void quant_q4_0_block(const float* x, uint8_t* out) {
    float mx = 0.f;
    for (int i = 0; i < QK; i++)
        if (fabsf(x[i]) > fabsf(mx)) mx = x[i];
    float d = mx / -8.0f;
    float inv = d == 0.0f ? 0.0f : 1.0f / d;
    wr_f16(out, d);
    for (int j = 0; j < QK / 2; j++) {
        float a = x[j] * inv + 8.5f, b = x[j + QK / 2] * inv + 8.5f;
        int qa = (int)a, qb = (int)b; /* truncation toward zero, as `as i32` */
        qa = qa < 0 ? 0 : (qa > 15 ? 15 : qa);
        qb = qb < 0 ? 0 : (qb > 15 ? 15 : qb);
        out[2 + j] = (uint8_t)(qa | (qb << 4));
    }
}

/* Q4_1 encoder: min/max rule of
 * crates/rlx-diffusiongemma/tests/real_layer_precision.rs:129-146 (d = (max -
 * min) / 15, q = floor((x - min)*id + 0.5) clamped to 15), stored as GGML
 * block_q4_1: f16 d, f16 min, byte j = q[j] | q[j+16] << 4. */
static void quant_q4_1_block(const float* x, uint8_t* out) {
    float mn = INFINITY, mx = -INFINITY;
    for (int i = 0; i < QK; i++) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
    }
    float d = (mx - mn) / 15.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    wr_f16(out, d);
    wr_f16(out + 2, mn);
    for (int j = 0; j < QK / 2; j++) {
        int qa = (int)floorf((x[j] - mn) * id + 0.5f);
        int qb = (int)floorf((x[j + QK / 2] - mn) * id + 0.5f);
        qa = qa < 0 ? 0 : (qa > 15 ? 15 : qa);
        qb = qb < 0 ? 0 : (qb > 15 ? 15 : qb);
        out[4 + j] = (uint8_t)(qa | (qb << 4));
    }
}

int orc_quantize(int scheme, const float* src, int64_t n, uint8_t* dst) {
    int64_t bb = orc_block_bytes(scheme);
    if (bb < 0 || n % QK || is_kquant(scheme)) return -1;  /* no K-quant encoders */
    for (int64_t b = 0; b < n / QK; b++) {
        const float* x = src + b * QK;
        uint8_t* o = dst + b * bb;
        if (scheme == ORC_GGUF_Q8_0) quant_q8_0_block(x, o);
        else if (scheme == ORC_GGUF_Q4_0) quant_q4_0_block(x, o);
        else quant_q4_1_block(x, o);
    }
    return 0;
}

/* Dequantize one block into 32 floats.
 *  Q8_0: w = d * q (crates/rlx-flint/src/quant.rs:124-127);
 *  Q4_0: w[j] = d*((b&15)-8), w[j+16] = d*((b>>4)-8) (quant.rs:128-135);
 *  Q4_1: w = d*q + m (GGML dequantize_row_q4_1; every product d*q is exact
 *        in f32, so the one rounding is on the add). */
static void dequant_block(int scheme, const uint8_t* b, float* o) {
    float d = rd_f16(b);
    if (scheme == ORC_GGUF_Q8_0) {
        for (int i = 0; i < QK; i++) o[i] = d * (float)(int8_t)b[2 + i];
    } else if (scheme == ORC_GGUF_Q4_0) {
        for (int j = 0; j < QK / 2; j++) {
            o[j] = d * (float)((int)(b[2 + j] & 0x0f) - 8);
            o[j + QK / 2] = d * (float)((int)(b[2 + j] >> 4) - 8);
        }
    } else {
        float m = rd_f16(b + 2);
        for (int j = 0; j < QK / 2; j++) {
            o[j] = d * (float)(b[4 + j] & 0x0f) + m;
            o[j + QK / 2] = d * (float)(b[4 + j] >> 4) + m;
        }
    }
}

/* GGUF Q4_K (GGML block_q4_K; QuantScheme::GgufQ4K, decoded by the absent
 * rlx_gguf::dequant_q4_k): 256 weights in 144 bytes -- f16 d, f16 dmin, 12
 * bytes packing eight 6-bit (scale, min) pairs, then 128 nibble bytes.  Byte
 * j of the 32-byte group g holds weight 64g + j (low nibble, sub-block 2g)
 * and weight 64g + 32 + j (high nibble, sub-block 2g + 1).  Sub-block s has
 * scale sc and min mn taken from the 12 packed bytes q as
 *   s < 4: sc = q[s] & 63,                       mn = q[s + 4] & 63;
 *   s >= 4: sc = (q[s + 4] & 15) | (q[s - 4] >> 6) << 4,
 *           mn = (q[s + 4] >> 4) | (q[s] >> 6) << 4;
 * and w = (d * sc) * code - (dmin * mn): each product rounded to f32, then
 * the subtraction rounded (no fused multiply-add). */
void orc_q4k_scale_min(const uint8_t* q, int s, int* sc, int* mn) {
    if (s < 4) {
        *sc = q[s] & 63;
        *mn = q[s + 4] & 63;
    } else {
        *sc = (q[s + 4] & 15) | ((q[s - 4] >> 6) << 4);
        *mn = (q[s + 4] >> 4) | ((q[s] >> 6) << 4);
    }
}

static void dequant_q4k_block(const uint8_t* b, float* o) {
    const float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t* sc12 = b + 4;
    const uint8_t* qs = b + 16;
    for (int g = 0; g < 4; g++) {
        for (int h = 0; h < 2; h++) {
            int sc, mn;
            orc_q4k_scale_min(sc12, 2 * g + h, &sc, &mn);
            const float d1 = d * (float)sc, m1 = dmin * (float)mn;
            for (int j = 0; j < 32; j++) {
                const int code = h == 0 ? (qs[32 * g + j] & 15) : (qs[32 * g + j] >> 4);
                const float prod = d1 * (float)code;
                o[64 * g + 32 * h + j] = prod - m1;
            }
        }
    }
}

/* GGUF Q6_K (GGML block_q6_K; QuantScheme::GgufQ6K, decoded by the absent
 * rlx_gguf::dequant_q6_k): 256 weights in 210 bytes -- ql[128] (low 4 bits
 * of each 6-bit code), qh[64] (high 2 bits), int8 scales[16] (one per 16
 * weights), f16 d.  In half h (weights 128h..128h+127; ql + 64h, qh + 32h,
 * scales + 8h), for l < 32 and j < 4, weight 128h + 32j + l has
 *   code = (ql[64h + l + 32 (j & 1)] >> 4 (j >> 1)) & 15
 *          | ((qh[32h + l] >> 2j) & 3) << 4,
 *   scale = scales[8h + 2j + l / 16],
 * and w = (d * scale) * (code - 32), each product rounded to f32 in that
 * order (d * scale is exact). */
static void dequant_q6k_block(const uint8_t* b, float* o) {
    const uint8_t* ql = b;
    const uint8_t* qh = b + 128;
    const int8_t* sc = (const int8_t*)(b + 192);
    const float d = rd_f16(b + 208);
    for (int h = 0; h < 2; h++)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 32; l++) {
                const int lo = (ql[64 * h + l + 32 * (j & 1)] >> (4 * (j >> 1))) & 15;
                const int hi = (qh[32 * h + l] >> (2 * j)) & 3;
                const float ds = d * (float)sc[8 * h + 2 * j + l / 16];
                o[128 * h + 32 * j + l] = ds * (float)((lo | (hi << 4)) - 32);
            }
}

/* GGUF Q5_K (GGML block_q5_K; QuantScheme::GgufQ5K, decoded by the absent
 * rlx_gguf::dequant_q5_k): 256 weights in 176 bytes -- f16 d, f16 dmin, the
 * 12 scale/min bytes of Q4_K, qh[32], qs[128].  Group g (weights
 * 64g..64g+63) reads qs[32g..32g+31]; weight 64g + 32h + l has
 *   code = (qs[32g + l] >> 4h) & 15 | ((qh[l] >> (2g + h)) & 1) << 4,
 * sub-block s = 2g + h, and w = (d * sc) * code - (dmin * mn) as for Q4_K. */
static void dequant_q5k_block(const uint8_t* b, float* o) {
    const float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t* sc12 = b + 4;
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    for (int g = 0; g < 4; g++)
        for (int h = 0; h < 2; h++) {
            int sc, mn;
            orc_q4k_scale_min(sc12, 2 * g + h, &sc, &mn);
            const float d1 = d * (float)sc, m1 = dmin * (float)mn;
            for (int l = 0; l < 32; l++) {
                const int code = ((qs[32 * g + l] >> (4 * h)) & 15) | (((qh[l] >> (2 * g + h)) & 1) << 4);
                const float prod = d1 * (float)code;
                o[64 * g + 32 * h + l] = prod - m1;
            }
        }
}

/* GGUF Q3_K (GGML block_q3_K; QuantScheme::GgufQ3K, absent
 * rlx_gguf::dequant_q3_k): 256 weights in 110 bytes -- hmask[32], qs[64]
 * (2-bit codes), 12 bytes packing sixteen 6-bit scales, f16 d.  Scale s
 * (16 weights each) from the 12 bytes q:
 *   s < 4:  q[s] & 15       | ((q[8 + s] >> 0) & 3) << 4
 *   s < 8:  q[s] & 15       | ((q[4 + s] >> 2) & 3) << 4      (q[s], s = 4..7)
 *   s < 12: q[s - 8] >> 4   | ((q[s] >> 4) & 3) << 4          (q[8 + (s - 8)])
 *   else:   q[s - 8] >> 4   | ((q[s - 4] >> 6) & 3) << 4      (q[8 + (s - 12)])
 * In half n (weights 128n..128n+127; qs + 32n) and quarter j, weight
 * 128n + 32j + 16i + l (i, l < 16) has
 *   code = (qs[32n + 16i + l] >> 2j) & 3, minus 4 unless bit 4n + j of
 *   hmask[16i + l] is set,
 *   scale = scale[8n + 2j + i] - 32,
 * and w = (d * scale) * code, each product rounded to f32 (d * scale exact). */
int orc_q3k_scale(const uint8_t* q, int s) {
    if (s < 4) return (q[s] & 15) | (((q[8 + s] >> 0) & 3) << 4);
    if (s < 8) return (q[s] & 15) | (((q[4 + s] >> 2) & 3) << 4);
    if (s < 12) return (q[s - 8] >> 4) | (((q[s] >> 4) & 3) << 4);
    return (q[s - 8] >> 4) | (((q[s - 4] >> 6) & 3) << 4);
}

static void dequant_q3k_block(const uint8_t* b, float* o) {
    const uint8_t* hm = b;
    const uint8_t* qs = b + 32;
    const uint8_t* sc12 = b + 96;
    const float d = rd_f16(b + 108);
    for (int n = 0; n < 2; n++)
        for (int j = 0; j < 4; j++)
            for (int i = 0; i < 2; i++) {
                const float dl = d * (float)(orc_q3k_scale(sc12, 8 * n + 2 * j + i) - 32);
                for (int l = 0; l < 16; l++) {
                    const int lo = (qs[32 * n + 16 * i + l] >> (2 * j)) & 3;
                    const int hi = (hm[16 * i + l] >> (4 * n + j)) & 1;
                    o[128 * n + 32 * j + 16 * i + l] = dl * (float)(lo - (hi ? 0 : 4));
                }
            }
}

/* GGUF Q2_K (GGML block_q2_K; QuantScheme::GgufQ2K, absent
 * rlx_gguf::dequant_q2_k): 256 weights in 84 bytes -- scales[16] (low
 * nibble scale, high nibble min, per 16 weights), qs[64] (2-bit codes), f16
 * d, f16 dmin.  Weight 128n + 32j + 16i + l has
 *   code = (qs[32n + 16i + l] >> 2j) & 3, byte c = scales[8n + 2j + i],
 * and w = (d * (c & 15)) * code - (dmin * (c >> 4)), each product rounded
 * to f32, then the subtraction. */
static void dequant_q2k_block(const uint8_t* b, float* o) {
    const uint8_t* sc = b;
    const uint8_t* qs = b + 16;
    const float d = rd_f16(b + 80), dmin = rd_f16(b + 82);
    for (int n = 0; n < 2; n++)
        for (int j = 0; j < 4; j++)
            for (int i = 0; i < 2; i++) {
                const int c = sc[8 * n + 2 * j + i];
                const float dl = d * (float)(c & 15), ml = dmin * (float)(c >> 4);
                for (int l = 0; l < 16; l++) {
                    const int code = (qs[32 * n + 16 * i + l] >> (2 * j)) & 3;
                    const float prod = dl * (float)code;
                    o[128 * n + 32 * j + 16 * i + l] = prod - ml;
                }
            }
}

/* GGUF Q8_K (GGML block_q8_K; QuantScheme::GgufQ8K, absent
 * rlx_gguf::dequant_q8_k): 256 weights in 292 bytes -- f32 d, int8 qs[256],
 * int16 bsums[16] (sums of 16 codes, not needed to decode); w = d * q. */
static void dequant_q8k_block(const uint8_t* b, float* o) {
    float d;
    memcpy(&d, b, 4);
    const int8_t* qs = (const int8_t*)(b + 4);
    for (int l = 0; l < 256; l++) o[l] = d * (float)qs[l];
}

int orc_dequantize(int scheme, const uint8_t* src, int64_t n, float* dst) {
    int64_t bb = orc_block_bytes(scheme), len = orc_block_len(scheme);
    if (bb < 0 || n % len) return -1;
    for (int64_t b = 0; b < n / len; b++) {
        const uint8_t* s = src + b * bb;
        float* o = dst + b * len;
        switch (scheme) {
            case ORC_GGUF_Q6_K: dequant_q6k_block(s, o); break;
            case ORC_GGUF_Q4_K: dequant_q4k_block(s, o); break;
            case ORC_GGUF_Q5_K: dequant_q5k_block(s, o); break;
            case ORC_GGUF_Q3_K: dequant_q3k_block(s, o); break;
            case ORC_GGUF_Q2_K: dequant_q2k_block(s, o); break;
            case ORC_GGUF_Q8_K: dequant_q8k_block(s, o); break;
            default: dequant_block(scheme, s, o);
        }
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* MLX affine                                                                */
/* ------------------------------------------------------------------------ */

/* pack_codes, crates/rlx-laguna/src/mlx_affine.rs:272-288: `bits`-wide codes
 * LSB-first, 32/bits per u32, contiguous per row. */
int orc_mlx_pack(const uint32_t* codes, int64_t rows, int64_t cols, int bits,
                 uint32_t* dst) {
    if (bits != 4 && bits != 8) return -1;
    int per = 32 / bits;
    if (cols % per) return -1;
    uint32_t mask = (1u << bits) - 1u;
    int64_t wpr = cols / per;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t w = 0; w < wpr; w++) {
            uint32_t word = 0;
            for (int j = 0; j < per; j++)
                word |= (codes[r * cols + w * per + j] & mask) << (j * bits);
            dst[r * wpr + w] = word;
        }
    return 0;
}

/* dequantize_affine, crates/rlx-moshi/src/mlx_dequant.rs:12-76: code s of a
 * word sits at bits [s*bits, (s+1)*bits); w = scale*code + bias (a multiply
 * rounded, then an add rounded -- no fused multiply-add). */
int orc_mlx_dequantize(const uint32_t* wq, const float* scales,
                       const float* biases, int64_t rows, int64_t cols,
                       int bits, int group, float* dst) {
    if (bits != 4 && bits != 8) return -1;
    if (group <= 0 || cols % group) return -1;
    int per = 32 / bits;
    if (cols % per) return -1;
    uint32_t mask = (1u << bits) - 1u;
    int64_t wpr = cols / per, ng = cols / group;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t c = 0; c < cols; c++) {
            uint32_t word = wq[r * wpr + c / per];
            float code = (float)((word >> ((c % per) * bits)) & mask);
            int64_t g = c / group;
            float prod = scales[r * ng + g] * code;
            dst[r * cols + c] = prod + biases[r * ng + g];
        }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Dense matmul                                                              */
/* ------------------------------------------------------------------------ */

/* y = x . W^T with W [n, k] row-major (host_matmul_t,
 * crates/rlx-unlimited-ocr/tests/quant_parity_backends.rs:74-86), evaluated
 * on the dequantized weights in double. */
int orc_matmul_f64(int scheme, const float* x, const uint8_t* w, int64_t m,
                   int64_t k, int64_t n, double* y) {
    int64_t rb = orc_row_bytes(scheme, k);
    if (rb < 0) return -1;
    float* row = (float*)malloc(sizeof(float) * (size_t)k);
    if (!row) return -2;
    for (int64_t j = 0; j < n; j++) {
        orc_dequantize(scheme, w + j * rb, k, row);
        for (int64_t r = 0; r < m; r++) {
            double acc = 0.0;
            const float* xr = x + r * k;
            for (int64_t i = 0; i < k; i++) acc += (double)xr[i] * (double)row[i];
            y[r * n + j] = acc;
        }
    }
    free(row);
    return 0;
}

/* One output element in the reference's block-dot order.
 * Q8_0: crates/rlx-flint/src/quant.rs:250-268; Q4_0: quant.rs:272-292.
 * Q4_1 has no in-tree restatement; it uses the Q4_0 loop shape with the
 * unsigned code and adds m * sum(x) for the block. */
static float dot_refl(int scheme, const float* x, const uint8_t* row, int64_t k) {
    int64_t bb = orc_block_bytes(scheme);
    float sum = 0.f;
    for (int64_t b = 0; b < k / QK; b++) {
        const float* xs = x + b * QK;
        const uint8_t* blk = row + b * bb;
        float d = rd_f16(blk);
        if (scheme == ORC_GGUF_Q8_0) {
            float acc[8] = {0};
            for (int l = 0; l < QK / 8; l++)
                for (int i = 0; i < 8; i++)
                    acc[i] = fmaf(xs[l * 8 + i], (float)(int8_t)blk[2 + l * 8 + i], acc[i]);
            float s = 0.f;
            for (int i = 0; i < 8; i++) s += acc[i];
            sum = fmaf(d, s, sum);
        } else if (scheme == ORC_GGUF_Q4_0) {
            float acc[16] = {0};
            for (int j = 0; j < QK / 2; j++) {
                int lo = (blk[2 + j] & 0x0f) - 8, hi = (blk[2 + j] >> 4) - 8;
                acc[j] = fmaf(xs[j], (float)lo, acc[j]);
                acc[j] = fmaf(xs[j + QK / 2], (float)hi, acc[j]);
            }
            float s = 0.f;
            for (int i = 0; i < 16; i++) s += acc[i];
            sum = fmaf(d, s, sum);
        } else {
            float mm = rd_f16(blk + 2);
            float acc[16] = {0};
            float xsum = 0.f;
            for (int j = 0; j < QK / 2; j++) {
                int lo = blk[4 + j] & 0x0f, hi = blk[4 + j] >> 4;
                acc[j] = fmaf(xs[j], (float)lo, acc[j]);
                acc[j] = fmaf(xs[j + QK / 2], (float)hi, acc[j]);
            }
            for (int i = 0; i < QK; i++) xsum += xs[i];
            float s = 0.f;
            for (int i = 0; i < 16; i++) s += acc[i];
            sum = fmaf(d, s, sum);
            sum = fmaf(mm, xsum, sum);
        }
    }
    return sum;
}

int orc_matmul_refl(int scheme, const float* x, const uint8_t* w, int64_t m,
                    int64_t k, int64_t n, float* y) {
    if (is_kquant(scheme)) return -1;  /* reference-order loop: legacy blocks only */
    int64_t rb = orc_row_bytes(scheme, k);
    if (rb < 0) return -1;
    for (int64_t r = 0; r < m; r++)
        for (int64_t j = 0; j < n; j++) y[r * n + j] = dot_refl(scheme, x + r * k, w + j * rb, k);
    return 0;
}

/* Output rows split over threads like gguf_matmul_bt_parallel's rayon
 * partition (call site crates/rlx-laguna/src/packed_forward.rs:226-241). */
int orc_matmul_refl_par(int scheme, const float* x, const uint8_t* w,
                        int64_t m, int64_t k, int64_t n, float* y,
                        int nthreads) {
    if (is_kquant(scheme)) return -1;
    int64_t rb = orc_row_bytes(scheme, k);
    if (rb < 0) return -1;
#ifdef _OPENMP
    if (nthreads <= 0) nthreads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(nthreads)
#endif
    for (int64_t j = 0; j < n; j++)
        for (int64_t r = 0; r < m; r++) y[r * n + j] = dot_refl(scheme, x + r * k, w + j * rb, k);
    (void)nthreads;
    return 0;
}

int orc_mlx_matmul_f64(const float* x, const uint32_t* wq, const float* scales,
                       const float* biases, int64_t m, int64_t k, int64_t n,
                       int bits, int group, double* y) {
    float* wd = (float*)malloc(sizeof(float) * (size_t)(n * k));
    if (!wd) return -2;
    int rc = orc_mlx_dequantize(wq, scales, biases, n, k, bits, group, wd);
    if (rc) {
        free(wd);
        return rc;
    }
    for (int64_t r = 0; r < m; r++)
        for (int64_t j = 0; j < n; j++) {
            double acc = 0.0;
            for (int64_t i = 0; i < k; i++) acc += (double)x[r * k + i] * (double)wd[j * k + i];
            y[r * n + j] = acc;
        }
    free(wd);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Grouped experts and MoE                                                   */
/* ------------------------------------------------------------------------ */

/* crates/rlx-unlimited-ocr/tests/quant_parity_backends.rs:268-281: expert e
 * is bank rows e*N..(e+1)*N; row r uses expert e[r]. */
int orc_grouped_matmul_f64(int scheme, const float* x, const uint8_t* bank,
                           const float* expert_idx, int64_t rows, int64_t k,
                           int64_t n, int64_t num_experts, double* y) {
    int64_t rb = orc_row_bytes(scheme, k);
    if (rb < 0) return -1;
    for (int64_t r = 0; r < rows; r++) {
        float ef = expert_idx[r];
        int64_t e = (int64_t)ef;
        if (!(ef >= 0.f) || e >= num_experts || (float)e != ef) return -3;
        int rc = orc_matmul_f64(scheme, x + r * k, bank + e * n * rb, 1, k, n, y + r * n);
        if (rc) return rc;
    }
    return 0;
}

/* topk_softmax, crates/rlx-unlimited-ocr/src/nn.rs:371-379 (softmax, sort by
 * probability descending, keep k); optional renormalisation of the kept
 * probabilities, crates/rlx-models-core/src/standard_decoder.rs:12657-12661. */
int orc_topk_softmax(const float* logits, int64_t rows, int64_t e, int64_t k,
                     int renorm, int32_t* ids, float* probs) {
    if (k <= 0 || k > e) return -1;
    float* p = (float*)malloc(sizeof(float) * (size_t)e);
    unsigned char* used = (unsigned char*)malloc((size_t)e);
    if (!p || !used) {
        free(p);
        free(used);
        return -2;
    }
    for (int64_t r = 0; r < rows; r++) {
        const float* l = logits + r * e;
        float mx = -INFINITY;
        for (int64_t i = 0; i < e; i++)
            if (l[i] > mx) mx = l[i];
        float s = 0.f;
        for (int64_t i = 0; i < e; i++) {
            p[i] = expf(l[i] - mx);
            s += p[i];
        }
        for (int64_t i = 0; i < e; i++) p[i] /= s;
        memset(used, 0, (size_t)e);
        float kept = 0.f;
        for (int64_t j = 0; j < k; j++) {
            int64_t best = -1;
            for (int64_t i = 0; i < e; i++)
                if (!used[i] && (best < 0 || p[i] > p[best])) best = i;
            used[best] = 1;
            ids[r * k + j] = (int32_t)best;
            probs[r * k + j] = p[best];
            kept += p[best];
        }
        if (renorm)
            for (int64_t j = 0; j < k; j++) probs[r * k + j] /= kept;
    }
    free(p);
    free(used);
    return 0;
}

/* quant_parity_backends.rs:360-373: for each (row, slot) the expert's
 * product, weighted by its probability, accumulated over the slots. */
int orc_moe_f64(int scheme, const float* x, const uint8_t* bank,
                const int32_t* ids, const float* probs, int64_t rows,
                int64_t topk, int64_t k, int64_t n, int64_t num_experts,
                double* y) {
    int64_t rb = orc_row_bytes(scheme, k);
    if (rb < 0) return -1;
    double* tmp = (double*)malloc(sizeof(double) * (size_t)n);
    if (!tmp) return -2;
    for (int64_t i = 0; i < rows * n; i++) y[i] = 0.0;
    for (int64_t r = 0; r < rows; r++)
        for (int64_t j = 0; j < topk; j++) {
            int32_t e = ids[r * topk + j];
            if (e < 0 || e >= num_experts) {
                free(tmp);
                return -3;
            }
            orc_matmul_f64(scheme, x + r * k, bank + (int64_t)e * n * rb, 1, k, n, tmp);
            double pr = probs[r * topk + j];
            for (int64_t c = 0; c < n; c++) y[r * n + c] += pr * tmp[c];
        }
    free(tmp);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* int8                                                                      */
/* ------------------------------------------------------------------------ */

int orc_quantize_act_int8(const float* x, int64_t rows, int64_t cols,
                          int8_t* q, float* scales) {
    for (int64_t r = 0; r < rows; r++) {
        const float* row = x + r * cols;
        float amax = 0.f;
        for (int64_t c = 0; c < cols; c++) {
            float a = fabsf(row[c]);
            if (a > amax) amax = a;
        }
        float s = amax > 0.f ? amax / 127.0f : 1.0f;
        float inv = 1.0f / s;
        for (int64_t c = 0; c < cols; c++) {
            float v = rnd_away(row[c] * inv);
            if (v < -127.f) v = -127.f;
            if (v > 127.f) v = 127.f;
            q[r * cols + c] = (int8_t)v;
        }
        scales[r] = s;
    }
    return 0;
}

int orc_quantize_int8_col(const float* w, int64_t k, int64_t n, int8_t* q,
                          float* scales) {
    for (int64_t c = 0; c < n; c++) {
        float amax = 0.f;
        for (int64_t r = 0; r < k; r++) {
            float a = fabsf(w[r * n + c]);
            if (a > amax) amax = a;
        }
        float s = amax > 0.f ? amax / 127.0f : 1.0f;
        scales[c] = s;
        for (int64_t r = 0; r < k; r++) {
            float v = rnd_away(w[r * n + c] / s);
            if (v < -127.f) v = -127.f;
            if (v > 127.f) v = 127.f;
            q[r * n + c] = (int8_t)v;
        }
    }
    return 0;
}

/* y = acc * sx[m] * sw[n], acc the exact int32 dot; the two scale products
 * are applied as (acc * sx) * sw in f32. */
int orc_w8a8_matmul(const int8_t* qx, const float* sx, const int8_t* qw,
                    const float* sw, int64_t m, int64_t k, int64_t n,
                    float* y) {
    for (int64_t r = 0; r < m; r++)
        for (int64_t c = 0; c < n; c++) {
            int64_t acc = 0;
            for (int64_t i = 0; i < k; i++) acc += (int64_t)qx[r * k + i] * (int64_t)qw[i * n + c];
            y[r * n + c] = ((float)acc * sx[r]) * sw[c];
        }
    return 0;
}

int orc_int8_block_matmul_f64(const float* x, const int8_t* wq,
                              const float* scale, const float* zp, int64_t m,
                              int64_t k, int64_t n, double* y) {
    for (int64_t r = 0; r < m; r++)
        for (int64_t c = 0; c < n; c++) {
            double acc = 0.0;
            for (int64_t i = 0; i < k; i++) {
                float wv = ((float)wq[i * n + c] - zp[c]) * scale[c];
                acc += (double)x[r * k + i] * (double)wv;
            }
            y[r * n + c] = acc;
        }
    return 0;
}
