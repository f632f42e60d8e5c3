// Seeded synthetic weights and activations for the MoE block.
//
// The benchmark configurations draw their inputs from stated distributions
// (x ~ N(0,1); router ~ N(0,0.02); IQ4_NL codes uniform 0..15 with fp16 scales
// |N(0,1)|*0.02; Q8 shared expert int8 ~ U[-127,127] with fp16 scale 0.0005).
// Every value here is a pure function of (seed, tensor, layer, index), built
// only from integer operations and correctly rounded double-precision
// add/mul/div/fma/sqrt, so the CPU checker and the GPU fill kernels produce
// identical bytes.  Generator pieces, all public methods:
//   * counter-based stream: the SplitMix64 output function (Steele, Lea and
//     Flood 2014; constants of Stafford's "Mix13") over key + (i+1)*golden;
//   * N(0,1): Box-Muller on two 32-bit uniforms of one draw;
//   * ln: exponent split plus the atanh series ln m = 2 atanh((m-1)/(m+1));
//   * cos(2*pi*t): quadrant reduction in turns plus Taylor series to degree 22.
// float -> fp16 conversion is round-to-nearest-even, written out in integer ops.
#pragma once
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "qe_format.h"

#ifdef __HIPCC__
#define QE_HD __host__ __device__ static inline
#else
#define QE_HD static inline
#endif

enum qe_tensor_id {
    QE_T_CODES = 1,   /* NL4 code bytes of the routed experts */
    QE_T_SCALES = 2,  /* fp16 block scales of the routed experts */
    QE_T_ROUTER = 3,  /* router rows 0..255 and the shared-gate row 256 */
    QE_T_SH_GU = 4,   /* shared expert gate|up int8 */
    QE_T_SH_DN = 5,   /* shared expert down int8 */
    QE_T_X = 6,       /* input activations */
    QE_T_PERM = 7,    /* Zipf rank permutation of the router bias */
};

QE_HD uint64_t qe_mix64(uint64_t z) {
    z ^= z >> 30;
    z *= 0xBF58476D1CE4E5B9ull;
    z ^= z >> 27;
    z *= 0x94D049BB133111EBull;
    z ^= z >> 31;
    return z;
}
QE_HD uint64_t qe_stream_key(uint64_t seed, uint32_t tensor, uint32_t layer, uint32_t sub) {
    const uint64_t stream = ((uint64_t)tensor << 56) ^ ((uint64_t)layer << 32) ^ (uint64_t)sub;
    return qe_mix64(seed ^ qe_mix64(stream + 0x9E3779B97F4A7C15ull));
}
QE_HD uint64_t qe_draw(uint64_t key, uint64_t i) {
    return qe_mix64(key + (i + 1) * 0x9E3779B97F4A7C15ull);
}

QE_HD double qe_bits_to_f64(uint64_t b) { double d; memcpy(&d, &b, 8); return d; }
QE_HD uint64_t qe_f64_to_bits(double d) { uint64_t b; memcpy(&b, &d, 8); return b; }
QE_HD float qe_bits_to_f32(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
QE_HD uint32_t qe_f32_to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

/* Natural log for u in (0, 1] (normal doubles only). */
QE_HD double qe_log_unit(double u) {
    uint64_t b = qe_f64_to_bits(u);
    int e = (int)((b >> 52) & 0x7ff) - 1023;
    double m = qe_bits_to_f64((b & 0x000FFFFFFFFFFFFFull) | 0x3FF0000000000000ull); /* [1,2) */
    if (m > 1.4142135623730951) { m = m * 0.5; e += 1; }
    const double f = (m - 1.0) / (m + 1.0); /* |f| <= 0.1716 */
    const double s = f * f;
    double p = 1.0 / 25.0;
    p = fma(p, s, 1.0 / 23.0);
    p = fma(p, s, 1.0 / 21.0);
    p = fma(p, s, 1.0 / 19.0);
    p = fma(p, s, 1.0 / 17.0);
    p = fma(p, s, 1.0 / 15.0);
    p = fma(p, s, 1.0 / 13.0);
    p = fma(p, s, 1.0 / 11.0);
    p = fma(p, s, 1.0 / 9.0);
    p = fma(p, s, 1.0 / 7.0);
    p = fma(p, s, 1.0 / 5.0);
    p = fma(p, s, 1.0 / 3.0);
    p = fma(p, s, 1.0);
    const double lnm = (2.0 * f) * p;
    const double de = (double)e;
    /* ln 2 split so that e*LN2_HI is exact for |e| < 2^11 */
    return fma(de, 6.93147180369123816490e-01, fma(de, 1.90821492927058770002e-10, lnm));
}

/* cos(2*pi*t) for t in [0, 1). */
QE_HD double qe_cos_turns(double t) {
    const double t4 = t * 4.0;
    const int q = (int)t4;
    const double r = t4 - (double)q;            /* exact, [0,1) */
    const double th = r * 1.5707963267948966;   /* [0, pi/2) */
    const double x = th * th;
    double c = 1.0 / 1124000727777607680000.0;  /* 1/22! */
    c = fma(c, -x, 1.0 / 2432902008176640000.0); /* 1/20! */
    c = fma(c, -x, 1.0 / 6402373705728000.0);    /* 1/18! */
    c = fma(c, -x, 1.0 / 20922789888000.0);      /* 1/16! */
    c = fma(c, -x, 1.0 / 87178291200.0);         /* 1/14! */
    c = fma(c, -x, 1.0 / 479001600.0);           /* 1/12! */
    c = fma(c, -x, 1.0 / 3628800.0);             /* 1/10! */
    c = fma(c, -x, 1.0 / 40320.0);               /* 1/8!  */
    c = fma(c, -x, 1.0 / 720.0);                 /* 1/6!  */
    c = fma(c, -x, 1.0 / 24.0);                  /* 1/4!  */
    c = fma(c, -x, 1.0 / 2.0);                   /* 1/2!  */
    c = fma(c, -x, 1.0);
    double s = 1.0 / 51090942171709440000.0;     /* 1/21! */
    s = fma(s, -x, 1.0 / 121645100408832000.0);  /* 1/19! */
    s = fma(s, -x, 1.0 / 355687428096000.0);     /* 1/17! */
    s = fma(s, -x, 1.0 / 1307674368000.0);       /* 1/15! */
    s = fma(s, -x, 1.0 / 6227020800.0);          /* 1/13! */
    s = fma(s, -x, 1.0 / 39916800.0);            /* 1/11! */
    s = fma(s, -x, 1.0 / 362880.0);              /* 1/9!  */
    s = fma(s, -x, 1.0 / 5040.0);                /* 1/7!  */
    s = fma(s, -x, 1.0 / 120.0);                 /* 1/5!  */
    s = fma(s, -x, 1.0 / 6.0);                   /* 1/3!  */
    s = fma(s, -x, 1.0);
    s = s * th;
    /* cos(q*pi/2 + th) by quadrant */
    switch (q & 3) {
        case 0: return c;
        case 1: return -s;
        case 2: return -c;
        default: return s;
    }
}

/* One N(0,1) sample per index (Box-Muller, cosine branch). */
QE_HD double qe_normal(uint64_t key, uint64_t i) {
    const uint64_t d = qe_draw(key, i);
    const double u1 = ((double)(d >> 32) + 1.0) * (1.0 / 4294967296.0); /* (0,1] */
    const double u2 = (double)(d & 0xffffffffu) * (1.0 / 4294967296.0); /* [0,1) */
    return sqrt(-2.0 * qe_log_unit(u1)) * qe_cos_turns(u2);
}

/* float -> IEEE binary16, round to nearest even. */
QE_HD uint16_t qe_f32_to_f16(float f) {
    const uint32_t x = qe_f32_to_bits(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) return (uint16_t)(sign | (ax > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 */
    if (ax < 0x38800000u) {                                   /* < 2^-14: subnormal or zero */
        const int e = (int)(ax >> 23);
        if (e == 0) return (uint16_t)sign;
        const int shift = 126 - e; /* >= 14 */
        if (shift > 25) return (uint16_t)sign;
        const uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t k = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (k & 1u))) ++k;
        return (uint16_t)(sign | k);
    }
    uint32_t r = ax - 0x38000000u;
    r += 0xfffu + ((r >> 13) & 1u);
    return (uint16_t)(sign | (r >> 13));
}
QE_HD float qe_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1f, m = (uint32_t)h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24, exact in float */
        const float v = (float)m * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    if (e == 31) return qe_bits_to_f32(sign | 0x7f800000u | (m << 13));
    return qe_bits_to_f32(sign | ((e + 112u) << 23) | (m << 13));
}

/* ---------------- tensors ---------------- */

/* 8 bytes of a routed expert blob (pack layout) at byte offset 8*w, 0 <= w < EXPERT_BYTES/8. */
QE_HD uint64_t qe_synth_expert_word(uint64_t seed, int layer, int expert, uint64_t w) {
    const uint64_t o = 8 * w;
    uint64_t code_idx, scale_idx;
    int is_code;
    if (o < QE_EXPERT_DOWN_OFF) {
        const uint64_t row = o / QE_GU_ROW_BYTES, c = o % QE_GU_ROW_BYTES; /* row 0..1023 (gate|up) */
        is_code = c < QE_D / 2;
        code_idx = row * (QE_D / 16) + c / 8;
        scale_idx = row * (QE_D / QE_BLK) + (c - QE_D / 2) / 2;
    } else {
        const uint64_t od = o - QE_EXPERT_DOWN_OFF;
        const uint64_t row = od / QE_DN_ROW_BYTES, c = od % QE_DN_ROW_BYTES;
        is_code = c < QE_FF_EXP / 2;
        code_idx = 2ull * QE_FF_EXP * (QE_D / 16) + row * (QE_FF_EXP / 16) + c / 8;
        scale_idx = 2ull * QE_FF_EXP * (QE_D / QE_BLK) + row * (QE_FF_EXP / QE_BLK) + (c - QE_FF_EXP / 2) / 2;
    }
    if (is_code) return qe_draw(qe_stream_key(seed, QE_T_CODES, (uint32_t)layer, (uint32_t)expert), code_idx);
    const uint64_t key = qe_stream_key(seed, QE_T_SCALES, (uint32_t)layer, (uint32_t)expert);
    uint64_t out = 0;
    for (int j = 0; j < 4; ++j) {
        const double z = qe_normal(key, scale_idx + (uint64_t)j);
        const uint16_t h = qe_f32_to_f16((float)(fabs(z) * 0.02));
        out |= (uint64_t)h << (16 * j);
    }
    return out;
}

/* Router weight: rows 0..255 = W_r, row 256 = shared-expert gate vector W_g; N(0, 0.02). */
QE_HD float qe_synth_router(uint64_t seed, int layer, int row, int col) {
    const uint64_t key = qe_stream_key(seed, QE_T_ROUTER, (uint32_t)layer, 0);
    return (float)(0.02 * qe_normal(key, (uint64_t)row * QE_D + (uint64_t)col));
}

/* int8 ~ U[-127,127] by multiply-shift of the high 32 bits. */
QE_HD int8_t qe_synth_q8_value(uint64_t key, uint64_t i) {
    const uint64_t d = qe_draw(key, i);
    return (int8_t)((int)(((d >> 32) * 255ull) >> 32) - 127);
}

/* 8 bytes of a Q8 matrix (rows x cols, row = int8[cols] then fp16[cols/32]) at byte 8*w. */
QE_HD uint64_t qe_synth_q8_word(uint64_t seed, int layer, uint32_t tensor, int cols, uint64_t w) {
    const uint64_t rb = (uint64_t)cols + (uint64_t)cols / QE_BLK * 2;
    const uint64_t o = 8 * w, row = o / rb, c = o % rb;
    if (c >= (uint64_t)cols) {
        const uint64_t h = qe_f32_to_f16(0.0005f);
        return h | (h << 16) | (h << 32) | (h << 48);
    }
    const uint64_t key = qe_stream_key(seed, tensor, (uint32_t)layer, 0);
    uint64_t out = 0;
    for (int j = 0; j < 8; ++j)
        out |= (uint64_t)(uint8_t)qe_synth_q8_value(key, row * (uint64_t)cols + c + (uint64_t)j) << (8 * j);
    return out;
}

/* Zipf router bias (host only): b_e = -s * ln(rank_e), ranks 1..256 under a
 * seeded Fisher-Yates permutation; the Zipf normaliser cancels in softmax/top-k. */
static inline void qe_synth_zipf_bias(uint64_t seed, int layer, double s, float *out) {
    int perm[QE_N_EXPERT];
    for (int i = 0; i < QE_N_EXPERT; ++i) perm[i] = i + 1;
    const uint64_t key = qe_stream_key(seed, QE_T_PERM, (uint32_t)layer, 0);
    for (int i = QE_N_EXPERT - 1; i > 0; --i) {
        const int j = (int)(((qe_draw(key, (uint64_t)i) >> 32) * (uint64_t)(i + 1)) >> 32);
        const int t = perm[i]; perm[i] = perm[j]; perm[j] = t;
    }
    for (int e = 0; e < QE_N_EXPERT; ++e) {
        /* ln(r) = ln(r/256) + 8 ln 2, with r/256 in (0,1] exact */
        const double lr = qe_log_unit((double)perm[e] / 256.0) + 8.0 * 0.69314718055994530942;
        out[e] = (float)(-s * lr);
    }
}

/* Input activation element i of activation set `inst`: N(0,1). */
QE_HD float qe_synth_x(uint64_t seed, int inst, uint64_t i) {
    const uint64_t key = qe_stream_key(seed, QE_T_X, 0, (uint32_t)inst);
    return (float)qe_normal(key, i);
}
