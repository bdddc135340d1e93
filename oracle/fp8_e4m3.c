/*
 * CPU oracle: OCP FP8 E4M3 ("fn": bias 7, max 448, no infinities, NaN =
 * S.1111.111) conversion and the FP8 KV scale rule.  TEST INFRASTRUCTURE
 * ONLY (see oracle/__init__.py).
 *
 * The encoder is written as a nearest-value search over the format's value
 * set, not as bit manipulation, so that it is independent of the device
 * kernel's formulation:
 *   - the 127 non-negative finite codes are ordered by value;
 *   - a magnitude is rounded to the nearest code, ties to the code with an
 *     even mantissa (round-to-nearest-even, OCP FP8 spec section 5);
 *   - 480 (the value that code 0x7F would have if it were finite) bounds the
 *     top interval: magnitudes above 464 round up to 0x7F, the NaN code, as
 *     torch's float8_e4m3fn cast does (the cast the reference uses at
 *     compiler/quantize/fp8_kv_cache.py:89), and NaN/inf give 0x7F;
 *   - the sign bit is copied (so -0.0 -> 0x80, -NaN -> 0xFF).
 *
 * Scale rule (compiler/quantize/fp8_kv_cache.py:81-86):
 *   amax = max|x| ; scale = 1.0 if amax == 0 else max(amax / 448, 1e-12)
 * in float32, with IEEE division.  Build without -ffast-math.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <string.h>

static float g_values[129]; /* value of code i (0..126), g_values[127] = 480 */
static int g_ready = 0;

static float bits_to_f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

static uint32_t f_to_bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}

/* Value of an e4m3fn code from the format definition. */
float oracle_e4m3_to_f32(uint8_t code) {
    const int s = code >> 7, e = (code >> 3) & 15, m = code & 7;
    float v;
    if (e == 15 && m == 7) return s ? -NAN : NAN;
    if (e == 0)
        v = ldexpf((float)m, -9); /* subnormal: m/8 * 2^(1-7) */
    else
        v = ldexpf(1.0f + (float)m / 8.0f, e - 7);
    return s ? -v : v;
}

static void init_values(void) {
    if (g_ready) return;
    for (int i = 0; i < 127; ++i) g_values[i] = oracle_e4m3_to_f32((uint8_t)i);
    g_values[127] = 480.0f;
    g_ready = 1;
}

uint8_t oracle_e4m3_from_f32(float x) {
    init_values();
    const uint8_t sign = (f_to_bits(x) >> 24) & 0x80;
    const float a = fabsf(x);
    if (isnan(x) || a >= 480.0f) return (uint8_t)(0x7F | sign);
    /* largest i with g_values[i] <= a (g_values is increasing) */
    int lo = 0, hi = 127;
    while (hi - lo > 1) {
        const int mid = (lo + hi) / 2;
        if (g_values[mid] <= a)
            lo = mid;
        else
            hi = mid;
    }
    int code;
    if (g_values[lo] == a) {
        code = lo;
    } else {
        /* a lies strictly between g_values[lo] and g_values[lo + 1] */
        const double dlo = (double)a - (double)g_values[lo];
        const double dhi = (double)g_values[lo + 1] - (double)a;
        if (dlo < dhi)
            code = lo;
        else if (dhi < dlo)
            code = lo + 1;
        else
            code = (lo & 1) ? lo + 1 : lo; /* tie: even mantissa */
    }
    return (uint8_t)(code | sign);
}

void oracle_e4m3_encode(const float* x, uint8_t* out, size_t n) {
    init_values();
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; ++i) out[i] = oracle_e4m3_from_f32(x[i]);
}

/* Encodes the float whose bit pattern is start + i, for i < count. */
void oracle_e4m3_encode_bits(uint32_t start, uint64_t count, uint8_t* out) {
    init_values();
#pragma omp parallel for schedule(static)
    for (uint64_t i = 0; i < count; ++i) out[i] = oracle_e4m3_from_f32(bits_to_f((uint32_t)(start + i)));
}

void oracle_e4m3_decode(const uint8_t* codes, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_e4m3_to_f32(codes[i]);
}

/* amax -> scale (float32). */
float oracle_fp8_scale_from_amax(float amax) {
    if (amax == 0.0f) return 1.0f;
    volatile float s = amax / 448.0f;
    if (s < 1e-12f) s = 1e-12f; /* NaN compares false and stays NaN */
    return s;
}

float oracle_fp8_amax(const float* x, size_t n) {
    float m = 0.0f;
    for (size_t i = 0; i < n; ++i) {
        const float a = fabsf(x[i]);
        if (isnan(a)) return a;
        if (a > m) m = a;
    }
    return m;
}

/* codes = e4m3(x / scale) */
void oracle_fp8_quantize(const float* x, size_t n, float scale, uint8_t* out) {
    init_values();
    for (size_t i = 0; i < n; ++i) {
        volatile float q = x[i] / scale;
        out[i] = oracle_e4m3_from_f32(q);
    }
}

/* out = f32(code) * scale */
void oracle_fp8_dequantize(const uint8_t* codes, size_t n, float scale, float* out) {
    for (size_t i = 0; i < n; ++i) out[i] = oracle_e4m3_to_f32(codes[i]) * scale;
}
