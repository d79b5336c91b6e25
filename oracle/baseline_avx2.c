/*
 * baseline_avx2.c — AVX2/FMA/F16C row kernels used as the host-CPU baseline.
 * TEST/BENCH INFRASTRUCTURE ONLY (bench.py's cpu_baseline leg).
 *
 * The per-row structure follows the reference's fused dequant-dot kernels:
 * widen int8 (or nibbles) to int32, convert to fp32, scale, FMA against the
 * fp32 activation and reduce with one horizontal sum per row
 * (src/kernels/quant.cpp:150-194 for Q8_0, :210-304 for Q4_K), called once
 * per output row like the matvec loops of src/kernels/matvec.cpp:62-142.
 * Rows are shared among OpenMP threads (omp_set_num_threads picks 1 for the
 * reference's single-threaded configuration).
 */
#include <immintrin.h>
#include <stdint.h>
#include <stddef.h>
#include <omp.h>

static inline float hsum256(__m256 v) {
    __m128 s = _mm_add_ps(_mm256_extractf128_ps(v, 1), _mm256_castps256_ps128(v));
    s = _mm_hadd_ps(s, s);
    s = _mm_hadd_ps(s, s);
    return _mm_cvtss_f32(s);
}

static inline float row_q8_0(const uint8_t* row, uint32_t nb, const float* x) {
    __m256 acc = _mm256_setzero_ps();
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t* bp = row + 34 * (size_t)b;
        uint16_t dh = (uint16_t)(bp[0] | (bp[1] << 8));
        __m256 sv = _mm256_set1_ps(_cvtsh_ss(dh));
        const int8_t* qs = (const int8_t*)(bp + 2);
        for (int c = 0; c < 4; ++c) {
            __m128i q8 = _mm_loadl_epi64((const __m128i*)(qs + 8 * c));
            __m256 wf = _mm256_mul_ps(_mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(q8)), sv);
            acc = _mm256_fmadd_ps(wf, _mm256_loadu_ps(x + 32 * b + 8 * c), acc);
        }
    }
    return hsum256(acc);
}

static inline void scale_min(const uint8_t* q, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0F) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

static inline float row_q4_K(const uint8_t* row, uint32_t nb, const float* x) {
    __m256 acc = _mm256_setzero_ps();
    const __m128i m4 = _mm_set1_epi8(0x0F);
    for (uint32_t b = 0; b < nb; ++b) {
        const uint8_t* bp = row + 144 * (size_t)b;
        float d = _cvtsh_ss((uint16_t)(bp[0] | (bp[1] << 8)));
        float dmin = _cvtsh_ss((uint16_t)(bp[2] | (bp[3] << 8)));
        const uint8_t* sc = bp + 4;
        const uint8_t* qs = bp + 16;
        const float* xb = x + 256 * (size_t)b;
        for (int blk = 0; blk < 4; ++blk) {
            int s0, m0, s1, m1;
            scale_min(sc, 2 * blk, &s0, &m0);
            scale_min(sc, 2 * blk + 1, &s1, &m1);
            __m256 rs0 = _mm256_set1_ps(d * s0), nm0 = _mm256_set1_ps(-dmin * m0);
            __m256 rs1 = _mm256_set1_ps(d * s1), nm1 = _mm256_set1_ps(-dmin * m1);
            __m128i r0 = _mm_loadu_si128((const __m128i*)(qs + 32 * blk));
            __m128i r1 = _mm_loadu_si128((const __m128i*)(qs + 32 * blk + 16));
            __m128i lo0 = _mm_and_si128(r0, m4), lo1 = _mm_and_si128(r1, m4);
            __m128i hi0 = _mm_and_si128(_mm_srli_epi16(r0, 4), m4), hi1 = _mm_and_si128(_mm_srli_epi16(r1, 4), m4);
            const __m128i parts[4] = {lo0, lo1, hi0, hi1};
            for (int p = 0; p < 4; ++p) {
                __m256 rs = (p & 1) ? rs1 : rs0, nm = (p & 1) ? nm1 : nm0;
                const float* xp = xb + 64 * blk + 16 * p;
                __m256 w0 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(parts[p])), rs, nm);
                acc = _mm256_fmadd_ps(w0, _mm256_loadu_ps(xp), acc);
                __m256 w1 = _mm256_fmadd_ps(_mm256_cvtepi32_ps(_mm256_cvtepu8_epi32(_mm_srli_si128(parts[p], 8))), rs, nm);
                acc = _mm256_fmadd_ps(w1, _mm256_loadu_ps(xp + 8), acc);
            }
        }
    }
    return hsum256(acc);
}

void ob_matvec_q8_0_avx2(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K) {
    const uint8_t* base = (const uint8_t*)blocks;
    uint32_t nb = K / 32;
#pragma omp parallel for schedule(static)
    for (uint32_t m = 0; m < M; ++m) y[m] += row_q8_0(base + (size_t)m * nb * 34, nb, x);
}

void ob_matvec_q4_K_avx2(const void* blocks, const float* x, float* y, uint32_t M, uint32_t K) {
    const uint8_t* base = (const uint8_t*)blocks;
    uint32_t nb = K / 256;
#pragma omp parallel for schedule(static)
    for (uint32_t m = 0; m < M; ++m) y[m] += row_q4_K(base + (size_t)m * nb * 144, nb, x);
}

void ob_set_threads(int n) { omp_set_num_threads(n); }
int ob_max_threads(void) { return omp_get_max_threads(); }
