/*
 * C restatement of the reference's centered RNS GEMM pipeline, for CPU-side
 * checking at medium sizes and for the CPU baseline timing.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ and by bench.py's cpu_baseline
 * leg through ctypes; never linked into the shipped library.
 *
 * Follows, step for step:
 *   encode     src/rns_llm/reference.py:32-40  (centered residues, int8)
 *   GEMM       csrc/rns_cuda.cu:478-523        (per-channel int8 x int8 -> int32)
 *   reduce     csrc/rns_cuda.cu:52-67          (canonical residue of int32)
 *   Garner     csrc/rns_cuda.cu:380-414        (mixed radix, pairwise inverses)
 *   correction csrc/rns_cuda.cu:409-412        (x > P/2 -> x - P)
 * Pinned against the NumPy oracle and the exact int64 product in
 * tests/test_oracle.py.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static int64_t mod_pos(int64_t v, int64_t m) {
    int64_t r = v % m;
    return r < 0 ? r + m : r;
}

static int inv_mod(int a, int m) {
    /* extended Euclid; a and m coprime */
    int64_t t = 0, nt = 1, r = m, nr = mod_pos(a, m);
    while (nr != 0) {
        int64_t q = r / nr, tmp;
        tmp = t - q * nt; t = nt; nt = tmp;
        tmp = r - q * nr; r = nr; nr = tmp;
    }
    return (int)mod_pos(t, m);
}

/* values [n] (int8) -> out [R][n] centered residues */
void oracle_encode_centered_i8(const int8_t *values, int64_t n,
                               const int32_t *moduli, int channels,
                               int8_t *out) {
    for (int c = 0; c < channels; ++c) {
        const int m = moduli[c];
        for (int64_t i = 0; i < n; ++i) {
            int64_t r = mod_pos(values[i], m);
            if (r > m / 2) r -= m;
            out[(int64_t)c * n + i] = (int8_t)r;
        }
    }
}

/*
 * a [M][K] int8, b [K][N] int8 (row-major), out [M][N] int64.
 * Returns 0 on success, -1 on bad arguments or allocation failure.
 */
int oracle_rns_matmul_centered(const int8_t *a, const int8_t *b, int M, int K,
                               int N, const int32_t *moduli, int channels,
                               int64_t *out) {
    if (M < 0 || K <= 0 || N < 0 || channels < 1 || channels > 16) return -1;
    int8_t *ar = (int8_t *)malloc((size_t)channels * M * K);
    int8_t *bt = (int8_t *)malloc((size_t)channels * N * K); /* [R][N][K] */
    int8_t *tmp = (int8_t *)malloc((size_t)channels * K * N);
    int32_t *canon = (int32_t *)malloc(sizeof(int32_t) * (size_t)channels * M * N);
    if (!ar || !bt || !tmp || !canon) {
        free(ar); free(bt); free(tmp); free(canon);
        return -1;
    }
    oracle_encode_centered_i8(a, (int64_t)M * K, moduli, channels, ar);
    oracle_encode_centered_i8(b, (int64_t)K * N, moduli, channels, tmp);
    for (int c = 0; c < channels; ++c)
        for (int k = 0; k < K; ++k)
            for (int n = 0; n < N; ++n)
                bt[((size_t)c * N + n) * K + k] = tmp[((size_t)c * K + k) * N + n];

    for (int c = 0; c < channels; ++c) {
        const int m = moduli[c];
        const int8_t *ac = ar + (size_t)c * M * K;
        const int8_t *bc = bt + (size_t)c * N * K;
#pragma omp parallel for schedule(static)
        for (int i = 0; i < M; ++i) {
            for (int j = 0; j < N; ++j) {
                int32_t acc = 0;
                const int8_t *x = ac + (size_t)i * K;
                const int8_t *y = bc + (size_t)j * K;
                for (int k = 0; k < K; ++k) acc += (int32_t)x[k] * (int32_t)y[k];
                canon[((size_t)c * M + i) * N + j] = (int32_t)mod_pos(acc, m);
            }
        }
    }

    /* Garner with pairwise inverses inv[j][i] = m_j^-1 mod m_i, j < i */
    int inv[16][16];
    for (int i = 0; i < channels; ++i)
        for (int j = 0; j < i; ++j) inv[j][i] = inv_mod(moduli[j], moduli[i]);
    int64_t big_p = 1;
    for (int c = 0; c < channels; ++c) big_p *= moduli[c];

#pragma omp parallel for schedule(static)
    for (int64_t e = 0; e < (int64_t)M * N; ++e) {
        int64_t d[16];
        for (int i = 0; i < channels; ++i) {
            int64_t v = canon[(size_t)i * M * N + e];
            for (int j = 0; j < i; ++j) v = mod_pos((v - d[j]) * inv[j][i], moduli[i]);
            d[i] = v;
        }
        int64_t x = 0, radix = 1;
        for (int i = 0; i < channels; ++i) {
            x += d[i] * radix;
            radix *= moduli[i];
        }
        if (x > big_p / 2) x -= big_p;
        out[e] = x;
    }
    free(ar); free(bt); free(tmp); free(canon);
    return 0;
}
