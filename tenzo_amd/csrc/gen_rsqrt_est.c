/* Generates the reciprocal-square-root estimate table of rsqrt_est.h.
 *
 * The reference builds TenzoEngine.cpp with -ffast-math, under which GCC
 * evaluates rms_norm_raw's 1.0f / std::sqrt(a) (TenzoEngine.cpp:154) as the
 * x86 estimate RSQRTSS(a) refined by one Newton step. RSQRTSS is a table
 * lookup whose contents are not specified by the ISA. On the Intel host where
 * the reference was built and its goldens written, its result depends only on
 * the parity of the exponent and the top 10 mantissa bits of a, and scales
 * exactly with the exponent: rsqrtss(4a) == rsqrtss(a) / 2. So 2 x 1024 values,
 * taken for a in [0.5, 2), reproduce it for every positive normal a.
 *
 *   gcc -O2 -msse gen_rsqrt_est.c -o gen && ./gen table > rsqrt_est_table.inc
 *   ./gen check < rsqrt_est_table.inc   # every positive normal float, this host
 *
 * "check" reads a table (the hex words of the .inc file) and compares the
 * table lookup with this host's RSQRTSS over all 2^31 - 2^24 positive normal
 * floats; it prints the mismatch count (0 on the hosts the table was taken
 * from). Built and run only on x86-64 hosts; the table itself is plain data.
 */
#include <immintrin.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static uint32_t rsqrtss_bits(uint32_t a) {
    float f, r;
    uint32_t o;
    memcpy(&f, &a, 4);
    r = _mm_cvtss_f32(_mm_rsqrt_ss(_mm_set_ss(f)));
    memcpy(&o, &r, 4);
    return o;
}

/* entry (odd, m10): a = 2^(odd ? 0 : -1) * (1 + m10 / 1024) */
static uint32_t entry_input(int odd, int m10) {
    return ((uint32_t)(odd ? 127 : 126) << 23) | ((uint32_t)m10 << 13);
}

static uint32_t lookup(const uint32_t* tab, uint32_t a) {
    const uint32_t e = a >> 23, odd = e & 1u, e0 = odd ? 127u : 126u;
    const uint32_t t = tab[odd * 1024u + ((a >> 13) & 1023u)];
    /* e - e0 is even; the estimate's exponent moves by half of it */
    return (uint32_t)((int32_t)t - (((int32_t)e - (int32_t)e0) / 2) * (1 << 23));
}

int main(int argc, char** argv) {
    if (argc > 1 && strcmp(argv[1], "check") == 0) {
        static uint32_t tab[2048];
        for (int i = 0; i < 2048; ++i)
            if (scanf(" 0x%x ,", &tab[i]) != 1) {
                fprintf(stderr, "table entry %d unreadable\n", i);
                return 2;
            }
        unsigned long long bad = 0;
        for (uint32_t a = 1u << 23; a < 0x7f800000u; ++a)
            if (lookup(tab, a) != rsqrtss_bits(a)) ++bad;
        printf("%llu\n", bad);
        return bad != 0;
    }
    for (int i = 0; i < 2048; ++i)
        printf("0x%08x,%s", rsqrtss_bits(entry_input(i >> 10, i & 1023)),
               (i & 7) == 7 ? "\n" : " ");
    return 0;
}
