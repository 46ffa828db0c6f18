/* Exhaustive host check of the identities the activation quantizers use instead of IEEE
 * division and of the reference's rounding steps (test infrastructure; the fp16 conversions come
 * from the oracle, which restates qwen_moe_hp.c:70-86).  Prints three mismatch counts:
 *   div127: RN(a * RN(1/127)) corrected by one FMA vs a / 127.0f, every a in [1e-6, FLT_MAX];
 *   f16:    the quantizers' fp16 truncation of d vs f16_to_f32(f32_to_f16(d)), every d > 0;
 *   round:  (bits(v + 1.5 * 2^23) - bits(1.5 * 2^23)) vs lrintf(v), every v in [-128, 128]. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include "x100_oracle.h"

static float fb(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bf(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

int main(void)
{
    const volatile float c127 = 127.0f;
    const float c = 1.0f / c127;
    unsigned long long bad_div = 0, bad_f16 = 0, bad_round = 0;
    for (uint32_t u = bf(1e-6f);; u++) {
        const float a = fb(u);
        const float q0 = a * c;
        const float r = fmaf(-q0, 127.0f, a);
        bad_div += bf(fmaf(r, c, q0)) != bf(a / c127);
        if (u == 0x7f7fffffu) break;
    }
    for (uint32_t u = 1;; u++) {
        const float d = fb(u);
        const float nrm = fb(bf(d) & 0xffffe000u);
        const float sub = truncf(d * 0x1p24f) * 0x1p-24f;
        float t = d >= 0x1p-14f ? nrm : sub;
        t = d >= 65536.0f ? INFINITY : t;
        bad_f16 += bf(t) != bf(orc_f16_to_f32(orc_f32_to_f16(d)));
        if (u == 0x7f7fffffu) break;
    }
    const float rnd = 0x1.8p23f;
    for (uint32_t u = 0; u <= bf(128.0f); u++)
        for (int sgn = 0; sgn < 2; sgn++) {
            const float v = sgn ? -fb(u) : fb(u);
            const int q = (int)(bf(v + rnd) - bf(rnd));
            bad_round += q != (int)lrintf(v);
        }
    printf("%llu %llu %llu\n", bad_div, bad_f16, bad_round);
    return 0;
}
