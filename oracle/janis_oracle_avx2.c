/*
 * janis_oracle_avx2.c -- TEST INFRASTRUCTURE ONLY (see janis_oracle.h).
 *
 * The per-output-channel AVX2+FMA kernel of cpu/qmv_amd64.s:28-81 written
 * with compiler intrinsics (a restatement, not the reference's assembly): one
 * u32 word broadcast to 8 lanes, lane l shifted right by 4*l and masked to its
 * nibble, converted to fp32; fused sumXQ += q*x and unfused sumX += x per
 * word; two fused folds per group (scale, then bias); the 8 lanes reduced as
 * lo4+hi4 followed by two horizontal pair-adds. This file is compiled with
 * -mavx2 -mfma; callers check or_have_avx2_fma() before using it.
 */
#include <immintrin.h>
#include <math.h>

#include "janis_oracle.h"

int or_have_avx2_fma(void) {
    __builtin_cpu_init();
    return __builtin_cpu_supports("avx2") && __builtin_cpu_supports("fma");
}

float or_qchannel4_avx2(const uint32_t *w, const float *x, const float *s, const float *b,
                        int groups, int words_per_group) {
    if (!or_have_avx2_fma()) return NAN;
    const __m256i shifts = _mm256_setr_epi32(0, 4, 8, 12, 16, 20, 24, 28);
    const __m256i nib = _mm256_set1_epi32(0xF);
    __m256 acc = _mm256_setzero_ps();
    for (int g = 0; g < groups; g++) {
        __m256 sxq = _mm256_setzero_ps();
        __m256 sx = _mm256_setzero_ps();
        for (int wc = 0; wc < words_per_group; wc++) {
            const __m256i word = _mm256_set1_epi32((int)*w++);
            const __m256i codes = _mm256_and_si256(_mm256_srlv_epi32(word, shifts), nib);
            const __m256 q = _mm256_cvtepi32_ps(codes);
            const __m256 xv = _mm256_loadu_ps(x);
            x += 8;
            sxq = _mm256_fmadd_ps(q, xv, sxq);
            sx = _mm256_add_ps(sx, xv);
        }
        acc = _mm256_fmadd_ps(_mm256_set1_ps(s[g]), sxq, acc);
        acc = _mm256_fmadd_ps(_mm256_set1_ps(b[g]), sx, acc);
    }
    __m128 lo = _mm256_castps256_ps128(acc);
    const __m128 hi = _mm256_extractf128_ps(acc, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_hadd_ps(lo, lo);
    lo = _mm_hadd_ps(lo, lo);
    return _mm_cvtss_f32(lo);
}
