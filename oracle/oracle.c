/*
 * CPU oracle for the q4 weight path. TEST INFRASTRUCTURE ONLY: see oracle.h.
 * Built with -O2 -ffp-contract=off (oracle/Makefile).
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#define GAMMA 0x9e3779b97f4a7c15ULL

/* src/bench/rng.rs:20-25: add gamma, then two xor-shift-multiply rounds. */
uint64_t or_splitmix_mix(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

uint64_t or_splitmix_next(uint64_t *state) {
    *state += GAMMA;
    return or_splitmix_mix(*state);
}

uint64_t or_splitmix_at(uint64_t seed, uint64_t index) {
    return or_splitmix_mix(seed + (index + 1) * GAMMA);
}

/* src/bench/rng.rs:27-42. rejected = ((2^64-1) % bound + 1) % bound draws
 * at the top of the range are refused so the remainder is unbiased; at
 * most 64 draws are tried. */
int or_splitmix_below(uint64_t *state, uint32_t bound, uint32_t *out) {
    if (bound == 0) return -1;
    const uint64_t bnd = bound;
    const uint64_t rejected = ((UINT64_MAX % bnd) + 1) % bnd;
    const uint64_t max_accepted = UINT64_MAX - rejected;
    for (int i = 0; i < 64; ++i) {
        uint64_t draw = or_splitmix_next(state);
        if (draw <= max_accepted) {
            *out = (uint32_t)(draw % bnd);
            return 0;
        }
    }
    return -1;
}

double or_unit(uint64_t draw) { return (double)(draw >> 40) * (1.0 / 16777216.0); }

double or_normal(uint64_t d0, uint64_t d1) {
    double u1 = (double)((d0 >> 40) + 1) * (1.0 / 16777216.0);
    double u2 = or_unit(d1);
    return sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
}

/* src/metal/kernels/common.metal:29-31 */
float or_bf16_to_f32(uint16_t bits) {
    uint32_t w = (uint32_t)bits << 16;
    float f;
    memcpy(&f, &w, 4);
    return f;
}

/* src/metal/kernels/common.metal:37-43: NaN keeps its top bits and is
 * made quiet; everything else rounds to nearest, ties to even. */
uint16_t or_bf16_from_f32(float value) {
    uint32_t bits;
    memcpy(&bits, &value, 4);
    if (value != value) return (uint16_t)((bits >> 16) | 0x0040u);
    return (uint16_t)((bits + 0x7FFFu + ((bits >> 16) & 1u)) >> 16);
}

uint32_t or_q4_get(const uint32_t *wq, int64_t k, int64_t row, int64_t col) {
    uint32_t word = wq[row * (k / 8) + col / 8];
    return (word >> (4 * (col % 8))) & 0xFu;
}

void or_q4_pack(const uint8_t *q, int64_t rows, int64_t k, uint32_t *wq) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t w = 0; w < k / 8; ++w) {
            uint32_t word = 0;
            for (int j = 0; j < 8; ++j) word |= (uint32_t)(q[r * k + w * 8 + j] & 0xF) << (4 * j);
            wq[r * (k / 8) + w] = word;
        }
}

void or_q4_unpack(const uint32_t *wq, int64_t rows, int64_t k, uint8_t *q) {
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < k; ++c) q[r * k + c] = (uint8_t)or_q4_get(wq, k, r, c);
}

/* Product rounded, then sum rounded (the reference's mul-then-add order).
 * f32(s) * q is exact whenever it is finite (8-bit significand times a 4-bit
 * integer), so an FMA gives the same bits except when the product overflows. */
float or_q4_dequant_one(uint16_t s, uint32_t q, uint16_t b) {
    float prod = or_bf16_to_f32(s) * (float)q;
    return prod + or_bf16_to_f32(b);
}

void or_q4_dequant_f32(const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                       int64_t rows, int64_t k, int64_t group, float *out) {
    const int64_t groups = k / group;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < k; ++c) {
            int64_t g = r * groups + c / group;
            out[r * k + c] = or_q4_dequant_one(s[g], or_q4_get(wq, k, r, c), b[g]);
        }
}

void or_q4_dequant_bf16(const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                        int64_t rows, int64_t k, int64_t group, uint16_t *out) {
    const int64_t groups = k / group;
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < k; ++c) {
            int64_t g = r * groups + c / group;
            out[r * k + c] = or_bf16_from_f32(or_q4_dequant_one(s[g], or_q4_get(wq, k, r, c), b[g]));
        }
}

/* src/metal/kernels/index_select.metal:11-29 over the dequantised table. */
void or_q4_embed(const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                 int64_t rows, int64_t k, int64_t group,
                 const uint32_t *ids, int64_t n_ids, uint16_t *out) {
    const int64_t groups = k / group;
    for (int64_t i = 0; i < n_ids; ++i) {
        uint16_t *dst = out + i * k;
        if ((int64_t)ids[i] >= rows) {
            for (int64_t c = 0; c < k; ++c) dst[c] = or_bf16_from_f32(0.0f);
            continue;
        }
        int64_t r = ids[i];
        for (int64_t c = 0; c < k; ++c) {
            int64_t g = r * groups + c / group;
            dst[c] = or_bf16_from_f32(or_q4_dequant_one(s[g], or_q4_get(wq, k, r, c), b[g]));
        }
    }
}

/* src/metal/kernels/matmul.metal:42-64: one fp32 accumulator per output,
 * k ascending, product then add. */
void or_matmul_f32(const float *lhs, int64_t m, int64_t k, int64_t lhs_ld,
                   const float *rhs_t, int64_t n, float *out) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            float acc = 0.0f;
            for (int64_t t = 0; t < k; ++t) {
                float p = lhs[i * lhs_ld + t] * rhs_t[j * k + t];
                acc = acc + p;
            }
            out[i * n + j] = acc;
        }
}

struct linear_job {
    const uint16_t *x;
    int64_t m, k, x_ld;
    const uint32_t *wq;
    const uint16_t *s, *b;
    int64_t n, group, n0, n1;
    float *y_f32;
    uint16_t *y_bf16;
};

static void *linear_rows(void *arg) {
    struct linear_job *jb = (struct linear_job *)arg;
    const int64_t k = jb->k, groups = k / jb->group;
    float *xf = (float *)malloc(sizeof(float) * (size_t)(jb->m * k));
    float *w = (float *)malloc(sizeof(float) * (size_t)k);
    if (!xf || !w) {
        free(xf);
        free(w);
        return (void *)1;
    }
    for (int64_t i = 0; i < jb->m; ++i)
        for (int64_t t = 0; t < k; ++t) xf[i * k + t] = or_bf16_to_f32(jb->x[i * jb->x_ld + t]);
    for (int64_t r = jb->n0; r < jb->n1; ++r) {
        /* dequantise one weight row into fp32, then accumulate in k order */
        const uint32_t *row = jb->wq + r * (k / 8);
        for (int64_t t = 0; t < k; ++t) {
            int64_t g = r * groups + t / jb->group;
            uint32_t q = (row[t / 8] >> (4 * (t % 8))) & 0xFu;
            w[t] = or_q4_dequant_one(jb->s[g], q, jb->b[g]);
        }
        for (int64_t i = 0; i < jb->m; ++i) {
            const float *xr = xf + i * k;
            float acc = 0.0f;
            for (int64_t t = 0; t < k; ++t) {
                float p = xr[t] * w[t];
                acc = acc + p;
            }
            if (jb->y_f32) jb->y_f32[i * jb->n + r] = acc;
            if (jb->y_bf16) jb->y_bf16[i * jb->n + r] = or_bf16_from_f32(acc);
        }
    }
    free(xf);
    free(w);
    return NULL;
}

void or_q4_linear(const uint16_t *x, int64_t m, int64_t k, int64_t x_ld,
                  const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                  int64_t n, int64_t group, float *y_f32, uint16_t *y_bf16,
                  int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    if (threads > n) threads = (int)(n > 0 ? n : 1);
    struct linear_job jobs[256];
    pthread_t tids[256];
    for (int t = 0; t < threads; ++t) {
        struct linear_job jb = {x, m, k, x_ld, wq, s, b, n, group,
                                n * t / threads, n * (t + 1) / threads, y_f32, y_bf16};
        jobs[t] = jb;
    }
    if (threads == 1) {
        linear_rows(&jobs[0]);
        return;
    }
    for (int t = 0; t < threads; ++t) pthread_create(&tids[t], NULL, linear_rows, &jobs[t]);
    for (int t = 0; t < threads; ++t) pthread_join(tids[t], NULL);
}

void or_gen_q4(uint64_t seed, int64_t rows, int64_t k, int64_t group,
               uint32_t *wq, uint16_t *s, uint16_t *b) {
    const int64_t words = rows * (k / 8);
    const int64_t word_draws = (words + 1) / 2;
    const int64_t ngroups = rows * (k / group);
    for (int64_t i = 0; i < word_draws; ++i) {
        uint64_t d = or_splitmix_at(seed, (uint64_t)i);
        wq[2 * i] = (uint32_t)d;
        if (2 * i + 1 < words) wq[2 * i + 1] = (uint32_t)(d >> 32);
    }
    for (int64_t g = 0; g < ngroups; ++g) {
        double u = or_unit(or_splitmix_at(seed, (uint64_t)(word_draws + g)));
        s[g] = or_bf16_from_f32((float)(0.004 + 0.016 * u));
    }
    const int64_t base = word_draws + ngroups;
    for (int64_t g = 0; g < ngroups; ++g) {
        double z = or_normal(or_splitmix_at(seed, (uint64_t)(base + 2 * g)),
                             or_splitmix_at(seed, (uint64_t)(base + 2 * g + 1)));
        double bias = -8.0 * (double)or_bf16_to_f32(s[g]) + 1e-3 * z;
        b[g] = or_bf16_from_f32((float)bias);
    }
}

void or_gen_bf16_normal(uint64_t seed, int64_t count, uint16_t *out) {
    for (int64_t i = 0; i < count; ++i) {
        double z = or_normal(or_splitmix_at(seed, (uint64_t)(2 * i)),
                             or_splitmix_at(seed, (uint64_t)(2 * i + 1)));
        out[i] = or_bf16_from_f32((float)z);
    }
}

int or_gen_token_ids(uint64_t seed, int64_t count, uint32_t vocab, uint32_t *out) {
    uint64_t state = seed;
    for (int64_t i = 0; i < count; ++i)
        if (or_splitmix_below(&state, vocab, &out[i]) != 0) return -1;
    return 0;
}
