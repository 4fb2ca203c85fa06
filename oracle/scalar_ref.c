/*
 * scalar_ref.c -- independent scalar restatement of the eager quantizers.
 * TEST INFRASTRUCTURE ONLY (built by oracle/build_ref.py, loaded by tests/ via ctypes).
 *
 * Purpose: pin oracle/eager_ref.py (the torch restatement of the reference eager
 * backend) with a second implementation that shares none of its rounding code.
 * Every narrowing conversion here is a brute-force nearest-value search over the
 * target format's finite values, ties to the code with an even last bit, done in
 * double precision (exact for these formats).  No bit tricks, no magic numbers.
 *
 * Eager arithmetic restated (reference backends/eager/quantization.py):
 *   per-tensor FP8 41-55, NVFP4 block 137-158, MXFP8 block 292-318.
 * Compile with -ffp-contract=off -fno-fast-math so each float operation rounds once.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float f_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* value of an E4M3FN code (0x7F/0xFF NaN) */
double ref_e4m3_value(int c) {
    int s = c & 0x80, e = (c >> 3) & 15, m = c & 7;
    double v = e ? ldexp(1.0 + m / 8.0, e - 7) : ldexp(m / 8.0, -6);
    if ((c & 0x7f) == 0x7f) return NAN;
    return s ? -v : v;
}

double ref_e5m2_value(int c) {
    int s = c & 0x80, e = (c >> 2) & 31, m = c & 3;
    if (e == 31) return m ? NAN : (s ? -INFINITY : INFINITY);
    double v = e ? ldexp(1.0 + m / 4.0, e - 15) : ldexp(m / 4.0, -14);
    return s ? -v : v;
}

double ref_e2m1_value(int c) {
    static const double mag[8] = {0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0};
    return (c & 8) ? -mag[c & 7] : mag[c & 7];
}

/* nearest code among positive codes [0, maxcode] of |x|, ties to even code */
static int nearest_code(double ax, int maxcode, double (*val)(int)) {
    int best = 0;
    double bd = fabs(ax - val(0));
    for (int c = 1; c <= maxcode; ++c) {
        double d = fabs(ax - val(c));
        if (d < bd || (d == bd && (c & 1) == 0)) { bd = d; best = c; }
    }
    return best;
}

/* x already clamped to [-448, 448] or NaN.  A NaN keeps its sign: 0x7F | sign, the
 * rule of torch's c10 fp32 -> Float8_e4m3fn / Float8_e5m2 conversion. */
int ref_f32_to_e4m3(float x) {
    if (isnan(x)) return signbit(x) ? 0xff : 0x7f;
    int c = nearest_code(fabs((double)x), 0x7e, ref_e4m3_value);
    return (signbit(x) ? 0x80 : 0) | c;
}

int ref_f32_to_e5m2(float x) {
    if (isnan(x)) return signbit(x) ? 0xff : 0x7f;
    int c = nearest_code(fabs((double)x), 0x7b, ref_e5m2_value);
    return (signbit(x) ? 0x80 : 0) | c;
}

/* x already clamped to [-6, 6]; sign kept (including -0) */
int ref_f32_to_e2m1(float x) {
    int c = nearest_code(fabs((double)x), 7, ref_e2m1_value);
    return (signbit(x) ? 8 : 0) | c;
}

/* bf16 round-to-nearest-even of a finite float, by comparing the two neighbours */
uint16_t ref_f32_to_bf16(float x) {
    uint32_t u = bits_of(x);
    if (isnan(x)) return (uint16_t)((u >> 16) | 0x40);
    uint32_t lo = u & 0xffff0000u;          /* truncation toward zero */
    uint32_t hi = lo + 0x10000u;            /* next bf16 away from zero */
    double dx = fabs((double)x), dlo = fabs((double)f_from_bits(lo)), dhi = fabs((double)f_from_bits(hi));
    double a = dx - dlo, b = dhi - dx;
    if (a < b) return (uint16_t)(lo >> 16);
    if (b < a) return (uint16_t)(hi >> 16);
    return (uint16_t)((((lo >> 16) & 1) == 0 ? lo : hi) >> 16);
}

float ref_bf16_value(uint16_t h) { return f_from_bits((uint32_t)h << 16); }

/* bf16 narrowing in torch's vectorised CPU kernels (x86 vec256/vec512 cvtfp32_bf16):
 * round to nearest even, and every NaN becomes 0xFFFF. */
uint16_t ref_vec_f32_to_bf16(float x) {
    if (isnan(x)) return 0xffff;
    return ref_f32_to_bf16(x);
}

/* ---- per-tensor FP8 on bf16 input (quantization.py:53-55), as eager's vectorised
 * loop computes it: the bf16 product is narrowed by ref_vec_f32_to_bf16, so every NaN
 * product encodes as 0xFF.  (r is a one-element tensor, narrowed by c10::BFloat16.) */
void ref_quantize_fp8_bf16(const uint16_t* x, int64_t n, float scale, int e5m2, uint8_t* out) {
    float r = ref_bf16_value(ref_f32_to_bf16(1.0f / scale));
    float lim = e5m2 ? 57344.0f : 448.0f;
    for (int64_t i = 0; i < n; ++i) {
        float t = ref_bf16_value(ref_vec_f32_to_bf16(ref_bf16_value(x[i]) * r));
        if (t > lim) t = lim;
        if (t < -lim) t = -lim;
        out[i] = (uint8_t)(e5m2 ? ref_f32_to_e5m2(t) : ref_f32_to_e4m3(t));
    }
}

/* ---- MXFP8 on one row of bf16, nblk blocks of 32 (quantization.py:292-318);
 * scale exponents (logical, unswizzled) into e[nblk], codes into q[32*nblk].
 * ceil(log2 s) is found exactly: s = m * 2^k with m in [0.5, 1) (frexp), so
 * ceil(log2 s) = k - 1 when m == 0.5 and k otherwise. */
void ref_quantize_mxfp8_row_bf16(const uint16_t* x, int64_t nblk, uint8_t* e, uint8_t* q) {
    for (int64_t b = 0; b < nblk; ++b) {
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            float v = fabsf(ref_bf16_value(x[32 * b + i]));
            if (v > amax || isnan(v)) amax = v;
        }
        float s = amax / 448.0f;
        if (s < ldexpf(1.0f, -127)) s = ldexpf(1.0f, -127);
        int k;
        double m = frexp((double)s, &k);
        int ex = (m == 0.5 ? k - 1 : k) + 127;
        if (!isfinite(s)) ex = 0; /* float->int of +-inf/NaN on x86 gives INT_MIN */
        if (ex < 0) ex = 0;
        if (ex > 254) ex = 254;
        float S = ex == 0 ? 0.0f : ldexpf(1.0f, ex - 127);
        int zero = amax == 0.0f;
        e[b] = zero ? 0 : (uint8_t)ex;
        for (int i = 0; i < 32; ++i) {
            float v = zero ? 0.0f : ref_bf16_value(x[32 * b + i]) / S;
            if (v > 448.0f) v = 448.0f;
            if (v < -448.0f) v = -448.0f;
            q[32 * b + i] = (uint8_t)ref_f32_to_e4m3(v);
        }
    }
}

/* ---- NVFP4 on one row of bf16, nblk blocks of 16 (quantization.py:137-158);
 * E4M3 scale bytes into s[nblk], unpacked E2M1 codes into c[16*nblk]. */
void ref_quantize_nvfp4_row_bf16(const uint16_t* x, int64_t nblk, float g, uint8_t* s, uint8_t* c) {
    for (int64_t b = 0; b < nblk; ++b) {
        float amax = 0.0f;
        for (int i = 0; i < 16; ++i) {
            float v = fabsf(ref_bf16_value(x[16 * b + i]));
            if (v > amax) amax = v;
        }
        float cs = (amax / 6.0f) / g;
        if (cs > 448.0f) cs = 448.0f;
        int s8 = ref_f32_to_e4m3(cs);
        s[b] = (uint8_t)s8;
        float T = g * (float)ref_e4m3_value(s8);
        for (int i = 0; i < 16; ++i) {
            float v = T == 0.0f ? 0.0f : ref_bf16_value(x[16 * b + i]) / T;
            if (v > 6.0f) v = 6.0f;
            if (v < -6.0f) v = -6.0f;
            c[16 * b + i] = (uint8_t)ref_f32_to_e2m1(v);
        }
    }
}

/* ---- 16-bit float formats by value (out code 1 = f16, 2 = bf16) */
static double ref_value16(int code, unsigned h) {
    double v;
    if (code == 2) {
        v = (double)f_from_bits((uint32_t)(h & 0x7fff) << 16);
    } else {
        int e = (h >> 10) & 31, m = h & 1023;
        if (e == 31) v = m ? NAN : INFINITY;
        else v = e ? ldexp(1.0 + m / 1024.0, e - 15) : ldexp(m / 1024.0, -14);
    }
    return (h & 0x8000) ? -v : v;
}

/* nearest 16-bit code to v, ties to the even code: binary search over the positive
 * finite codes, whose values increase with the code, then the nearer of the two that
 * bracket |v|.  Past the largest finite value the next binade's first value stands for
 * infinity: |v| at or above the midpoint between the two rounds to inf (the largest
 * finite code is odd, so the tie goes to inf as well). */
static unsigned ref_round16(int code, double v) {
    unsigned lo = 0, hi = code == 2 ? 0x7f7f : 0x7bff;
    double a = fabs(v);
    double top = ref_value16(code, hi), past = code == 2 ? ldexp(1.0, 128) : ldexp(1.0, 16);
    if (a >= (top + past) / 2) return (signbit(v) ? 0x8000u : 0u) | (hi + 1);
    while (hi - lo > 1) {
        unsigned mid = (lo + hi) / 2;
        if (ref_value16(code, mid) <= a) lo = mid; else hi = mid;
    }
    double dl = a - ref_value16(code, lo), dh = ref_value16(code, hi) - a;
    unsigned c = (dl < dh || (dl == dh && (lo & 1) == 0)) ? lo : hi;
    return (signbit(v) ? 0x8000u : 0u) | c;
}

/* nearest fp32 to a double that is exact in double precision (products of two floats),
 * ties to even, by comparing the float neighbours of a first guess */
static float ref_nearest_f32(double p) {
    float c = (float)p, best = c;
    double bd = fabs(p - (double)c);
    float cand[2] = {nextafterf(c, -INFINITY), nextafterf(c, INFINITY)};
    for (int i = 0; i < 2; ++i) {
        double d = fabs(p - (double)cand[i]);
        if (d < bd || (d == bd && (bits_of(cand[i]) & 1u) == 0)) { bd = d; best = cand[i]; }
    }
    return best;
}

/* RN32(1/d): the float c nearest 1/d, i.e. with the smallest |c*d - 1| (c*d is exact) */
static float ref_recip_f32(float d) {
    float c = (float)(1.0 / (double)d), best = c;
    double bd = fabs((double)c * d - 1.0);
    float cand[2] = {nextafterf(c, -INFINITY), nextafterf(c, INFINITY)};
    for (int i = 0; i < 2; ++i) {
        double e = fabs((double)cand[i] * d - 1.0);
        if (e < bd || (e == bd && (bits_of(cand[i]) & 1u) == 0)) { bd = e; best = cand[i]; }
    }
    return best;
}

/* ---- the layouts' default scale, torch.amax(x.abs()) / divisor on a GPU tensor
 * (tensor/fp8.py:56-61, tensor/nvfp4.py:64-69): amax * RN32(1/divisor) rounded to fp32,
 * then to x's dtype (in_code 0 = f32, 1 = f16, 2 = bf16); returned widened to fp32. */
float ref_default_scale(float amax, float divisor, int in_code) {
    float p = ref_nearest_f32((double)amax * (double)ref_recip_f32(divisor));
    if (in_code == 0) return p;
    return (float)ref_value16(in_code, ref_round16(in_code, (double)p));
}

/* ---- one dequantized NVFP4 element (quantization.py:208-214): the block total
 * g.to(out) * s8.to(out) and the product with the E2M1 value are each rounded to the
 * output dtype (out_code 0 = f32, 1 = f16, 2 = bf16). */
float ref_dequantize_nvfp4_value(int code4, int s8, float g, int out_code) {
    double e = ref_e2m1_value(code4), s = ref_e4m3_value(s8);
    if (out_code == 0) {
        float t = ref_nearest_f32((double)g * s);
        return ref_nearest_f32(e * (double)t);
    }
    double gt = ref_value16(out_code, ref_round16(out_code, (double)g));
    double t = ref_value16(out_code, ref_round16(out_code, gt * s));
    return (float)ref_value16(out_code, ref_round16(out_code, e * t));
}
