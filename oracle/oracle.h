/*
 * CPU oracle for the q4 weight path. TEST INFRASTRUCTURE ONLY.
 *
 * This is the checker: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. The product path
 * (libfoundry_hip.so) never links, calls or falls back to it.
 *
 * It restates the reference's arithmetic for the path it replaces:
 *   - SplitMix64 and `below`           src/bench/rng.rs:13-43
 *   - bf16 decode / RNE encode         src/metal/kernels/common.metal:29-43
 *   - row gather, out-of-range -> 0    src/metal/kernels/index_select.metal:11-29
 *   - fp32 matmul, sequential k        src/metal/kernels/matmul.metal:29-65
 *   - Linear = x . W^T                 src/nn/linear.rs:22-35
 * and adds the q4 arithmetic, which the reference does not have. Its format
 * (group 64 along K, 8 little-endian nibbles per u32, bf16 scale and bias,
 * w = s*q + b) comes from the task's configuration. No reference test pins
 * the q4 part; it is pinned by closed forms, invariants and brute force
 * (see tests/test_oracle.py).
 *
 * Every float function is compiled with -ffp-contract=off so a*b+c is two
 * roundings, as written.
 */
#ifndef FOUNDRY_ORACLE_H
#define FOUNDRY_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- SplitMix64 (src/bench/rng.rs:13-25) ---- */
uint64_t or_splitmix_next(uint64_t *state);
/* src/bench/rng.rs:27-42: rejection sampling, at most 64 draws.
 * Returns 0 and writes *out on success, -1 if bound == 0 or every draw
 * was rejected. */
int or_splitmix_below(uint64_t *state, uint32_t bound, uint32_t *out);
/* The mixing function alone: output of the draw whose state is `z`. */
uint64_t or_splitmix_mix(uint64_t z);
/* Draw number `index` (0-based) of a stream seeded with `seed`, without
 * stepping through the earlier ones: state = seed + (index+1)*gamma. */
uint64_t or_splitmix_at(uint64_t seed, uint64_t index);

/* ---- Seeded float draws (this build's definition; the reference has none).
 * u(d)  = (d >> 40) * 2^-24                       in [0, 1)
 * n(d0, d1) = sqrt(-2 ln u1) * cos(2 pi u2),  u1 = ((d0 >> 40) + 1) * 2^-24,
 *                                             u2 = u(d1)                   */
double or_unit(uint64_t draw);
double or_normal(uint64_t d0, uint64_t d1);

/* ---- bf16 codec (src/metal/kernels/common.metal:29-43) ---- */
float or_bf16_to_f32(uint16_t bits);
uint16_t or_bf16_from_f32(float value);

/* ---- q4 format ----
 * Packed weights wq: u32[rows, k/8]. Element j of a row is nibble j%8
 * (bits 4*(j%8) .. +3) of word j/8. Scales s and biases b: bf16[rows, k/g].
 * Dequantised value (fp32): w = f32(s) * q + f32(b). */
uint32_t or_q4_get(const uint32_t *wq, int64_t k, int64_t row, int64_t col);
void or_q4_pack(const uint8_t *q, int64_t rows, int64_t k, uint32_t *wq);
void or_q4_unpack(const uint32_t *wq, int64_t rows, int64_t k, uint8_t *q);
float or_q4_dequant_one(uint16_t s, uint32_t q, uint16_t b);
/* Materialised bf16 table: out[r, j] = RNE(w[r, j]). */
void or_q4_dequant_bf16(const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                        int64_t rows, int64_t k, int64_t group, uint16_t *out);
void or_q4_dequant_f32(const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                       int64_t rows, int64_t k, int64_t group, float *out);

/* q4 embedding gather: out[i, :] = RNE(w[ids[i], :]), or zeros when
 * ids[i] >= rows (src/metal/kernels/index_select.metal:23-26). */
void or_q4_embed(const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                 int64_t rows, int64_t k, int64_t group,
                 const uint32_t *ids, int64_t n_ids, uint16_t *out);

/* Generic fp32 matmul in matmul_tiled's order: for each output,
 * acc = 0; for k ascending: acc = acc + lhs[m,k] * rhs_t[n,k].
 * lhs: f32[m, k] (row stride lhs_ld), rhs_t: f32[n, k] (the weight, i.e.
 * the transposed right operand of src/nn/linear.rs:27). */
void or_matmul_f32(const float *lhs, int64_t m, int64_t k, int64_t lhs_ld,
                   const float *rhs_t, int64_t n, float *out);

/* q4 Linear with the reference arithmetic: x bf16[m, k] (row stride x_ld),
 * dequantised fp32 weights, sequential fp32 accumulation, and
 * y_bf16 = RNE(acc). Either output pointer may be NULL. Rows of the weight
 * are split over `threads` std-C threads (1 = scalar). */
void or_q4_linear(const uint16_t *x, int64_t m, int64_t k, int64_t x_ld,
                  const uint32_t *wq, const uint16_t *s, const uint16_t *b,
                  int64_t n, int64_t group, float *y_f32, uint16_t *y_bf16,
                  int threads);

/* ---- Synthetic inputs (the task's config distributions) ----
 * Draw order from one stream seeded with `seed`:
 *   words:  ceil(rows*k/8 / 2) draws; word 2i = low 32 bits of draw i,
 *           word 2i+1 = high 32 bits      (16 uniform nibbles per draw)
 *   scales: rows*k/g draws; s = RNE(0.004 + 0.016 * u(d))
 *   biases: 2*rows*k/g draws; b = RNE(f32(-8 * s + 1e-3 * n(d0, d1)))   */
void or_gen_q4(uint64_t seed, int64_t rows, int64_t k, int64_t group,
               uint32_t *wq, uint16_t *s, uint16_t *b);
/* x = RNE(f32(n(d0, d1))), two draws per element. */
void or_gen_bf16_normal(uint64_t seed, int64_t count, uint16_t *out);
/* Token ids as the reference draws them: `below(vocab)` per id
 * (src/bench/mod.rs:233-241). Returns 0, or -1 on a failed draw. */
int or_gen_token_ids(uint64_t seed, int64_t count, uint32_t vocab, uint32_t *out);

#ifdef __cplusplus
}
#endif

#endif
