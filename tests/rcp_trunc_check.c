// Exhaustive check of the INT8 dispatcher quantiser's division-free form:
//   code(RN(x / s)) == code(RN(x * r_up)),  r_up = RN(RN(1/s) * (1 + 2^-21)),
// for every finite fp16 amax >= 0, its scale s = fp16(RN(amax * f32(1/127)))
// (the reference's a_scale, EE/python/kernels.py:336-337), and every fp16 x with
// |x| <= amax; code() is the truncating int32 cast keeping the low byte
// (kernels.py:338).  Exit status 0 iff no pair differs.  Built and run by
// tests/test_quant_rcp_exhaustive.py (gcc, OpenMP, SSE binary32 arithmetic).
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
static float h2f(uint16_t h) {
    uint32_t s = (h >> 15) & 1, e = (h >> 10) & 31, m = h & 1023, u;
    if (e == 0) { if (!m) u = s << 31; else { float f = ldexpf((float)m, -24); return s ? -f : f; } }
    else if (e == 31) u = (s << 31) | 0x7f800000u | (m << 13);
    else u = (s << 31) | ((e + 112) << 23) | (m << 13);
    float f; memcpy(&f, &u, 4); return f;
}
static uint16_t f2h(float f) {  // RNE
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return sign | 0x7e00u;
    if (ax >= 0x477ff000u) return sign | 0x7c00u;
    if (ax < 0x38800000u) {  // subnormal / zero
        float a; memcpy(&a, &ax, 4);
        float q = a * 16777216.0f;  // exact scaling by 2^24
        uint32_t r = (uint32_t)nearbyintf(q);
        return sign | (uint16_t)r;
    }
    uint32_t e = (ax >> 23) - 112, m = ax & 0x7fffffu;
    uint32_t r = (e << 10) | (m >> 13), rem = m & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (r & 1))) r++;
    return sign | (uint16_t)r;
}
static int code(float q) {
    int32_t iv;
    if (fabsf(q) < 2147483648.0f) iv = (int32_t)q;
    else if (q != q) iv = 0;
    else iv = q > 0 ? 0x7fffffff : (int32_t)0x80000000;
    return iv & 0xff;
}
int main(void) {
    volatile float one = 1.0f, inv127v = 1.0f / 127.0f, bias = 1.0f + ldexpf(1.0f, -21);
    const float inv127 = inv127v;
    long long bad = 0, total = 0;
#pragma omp parallel for reduction(+ : bad, total) schedule(dynamic, 64)
    for (int ah = 0; ah < 0x7c00; ++ah) {                   // every finite non-negative fp16 amax
        const float amax = h2f((uint16_t)ah);
        const float s = h2f(f2h(amax * inv127));
        const float r_up = (one / s) * bias;
        for (int xh = 0; xh < 0x10000; ++xh) {
            const float x = h2f((uint16_t)xh);
            if (!(fabsf(x) <= amax)) continue;
            ++total;
            if (code(x / s) != code(x * r_up)) {
                if (bad < 5) printf("mismatch amax=%g s=%g x=%g q=%.9g q'=%.9g\n", amax, s, x, x / s, x * r_up);
                ++bad;
            }
        }
    }
    printf("pairs %lld mismatches %lld\n", total, bad);
    return bad != 0;
}
