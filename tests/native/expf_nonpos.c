// ggml_v_expf as i2s_device.h computes it (src/ops.c:342-379), the
// general form against the NONPOS one the softmax uses: same bits for every x
// with the sign bit set (a stride through them; argv[1]: the stride) and for
// a sample of the NaNs.

#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float gen(float x) {
    const float r = 0x1.8p23f;
    const float z = fmaf(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = fmaf(-n, 0x1.7f7d1cp-20f, fmaf(-n, 0x1.62e4p-1f, x));
    const uint32_t e = f2u(z) << 23;
    const float k = u2f(e + f2u(1.0f));
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u, fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)), u, 0x1.ffffecp-1f * b);
    const uint32_t g = n <= 0.0f ? 0x82000000u : 0u;
    const float s1 = u2f(g + 0x7f000000u);
    const float s2 = u2f(e - g);
    const float in_range = fmaf(j, k, k), scaled = fmaf(s2, j, s2) * s1, extreme = s1 * s1;
    return !(fabsf(n) > 126.0f) ? in_range : (fabsf(n) > 192.0f ? extreme : scaled);
}
static float spec(float x) {
    const float r = 0x1.8p23f;
    const float z = fmaf(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = fmaf(-n, 0x1.7f7d1cp-20f, fmaf(-n, 0x1.62e4p-1f, x));
    const uint32_t e = f2u(z) << 23;
    const float k = u2f(e + f2u(1.0f));
    const float u = b * b;
    const float j = fmaf(fmaf(fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u, fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)), u, 0x1.ffffecp-1f * b);
    const float s1 = u2f(0x82000000u + 0x7f000000u);
    const float s2 = u2f(e - 0x82000000u);
    const float in_range = fmaf(j, k, k), scaled = fmaf(s2, j, s2) * s1, extreme = s1 * s1;
    return !(fabsf(n) > 126.0f) ? in_range : (fabsf(n) > 192.0f ? extreme : scaled);
}
int main(int argc, char **argv) {
    const uint64_t stride = argc > 1 ? strtoull(argv[1], NULL, 10) : 1;
    uint64_t bad = 0, n = 0;
    for (uint64_t i = 0x80000000ull; i <= 0xFFFFFFFFull; i += stride) {
        const float x = u2f((uint32_t) i);
        const uint32_t a = f2u(gen(x)), c = f2u(spec(x));
        ++n;
        if (a != c && !(isnan(u2f(a)) && isnan(u2f(c)))) { if (bad < 5) printf("x=%08x gen=%08x spec=%08x\n", (uint32_t) i, a, c); ++bad; }
    }
    for (uint32_t m = 1; m < 0x800000u; m += 97) {     // positive NaNs (a sample)
        const float x = u2f(0x7f800000u | m);
        if (f2u(gen(x)) != f2u(spec(x)) && !(isnan(gen(x)) && isnan(spec(x)))) ++bad;
    }
    printf("%llu inputs, %llu differ\n", (unsigned long long) n, (unsigned long long) bad);
    return bad != 0;
}
