/*
 * w4a16_oracle.c -- CPU restatement of the reference's W4A16 hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the parity tests, the
 * smoke check and bench.py's cpu_baseline leg compare the HIP library
 * against.  The product path (libw4a16.so) never links, loads or calls it.
 *
 * What it restates (reference = TheCause/gemma4-zml-probe):
 *   pack     compressed-tensors pack_to_int32(q, num_bits=4), as called at
 *            scripts/57_w4_unpack_fixture.py:39; format fixed by
 *            zml_runner/w4.zig:4-10 (nibble j of word w = column 8w+j,
 *            stores q+8, unsigned) and docs/W4_RESULTS.md:28-37.
 *   unpack   unpackW4, zml_runner/w4.zig:33-45: logical shift by 4j, AND 0xF,
 *            minus 8 (an arithmetic shift would be wrong when bit 31 is set).
 *   dequant  dequantW4, zml_runner/w4.zig:47-54 (== dequant_manual,
 *            scripts/63_u_dequant_export.py:83-89): q converted to bf16
 *            (exact), times the group-32 bf16 scale, bf16 x bf16 -> bf16 with
 *            round-to-nearest-even.  The fp32 product of a 4-bit integer and
 *            an 8-bit-significand scale is exact, so the bf16 result is
 *            RNE_bf16(float(q) * float(s)).  NaN results (NaN or infinite
 *            scales only) become the canonical quiet NaN 0x7FC0.  The libraries
 *            in play disagree on NaN bit patterns (torch's scalar path gives
 *            0x7FC0, its vectorised path 0xFFFF, Eigen/XLA keeps the sign), so
 *            tests compare NaN against NaN by position, everything else by bits.
 *   linear   G3.forward, zml_runner/gemma4_w4gate.zig:288-292, and the
 *            fixture oracle scripts/58_w4_gemm_oracle.py:29:
 *            y = x.f32 @ dequant(pk, sc).f32^T, fp32 accumulate
 *            (dotPrec with fam = null, zml_runner/engine.zig:530-533).
 *            A float64-accumulate variant gives the error-bound reference.
 *
 * Pinning (what checks this file, so that it is not trusted on its own):
 *   tests/test_oracle.py checks pack/unpack against hand-derived known
 *   answers and an independent little-endian byte-view formulation, the
 *   bit-31 case and the one-nibble corruption of the reference's W1 gate;
 *   dequant exhaustively against torch's bf16 multiply over every q and every
 *   bf16 scale pattern; linear against float64 with a gamma_K error bound,
 *   one-hot / zero-scale / constant-q closed forms and torch's fp32 matmul.
 *
 * Parity unpinned: (1) pack's equality with compressed-tensors 0.17.1
 * pack_to_int32 is pinned by the documented closed form only (the library
 * is not installed here); (2) the reference's own W3 fixed points
 * (fixtures/w4_gemm_manifest.json:4-18) need the E2B-W4 checkpoint, which is
 * absent, so linear values are pinned by the bounds above, not by them.
 */
#include <stdint.h>
#include <string.h>
#include <math.h>

#define W4_GROUP 32

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* float -> bf16, round to nearest even; NaN -> 0x7FC0. */
static inline uint16_t f32_to_bf16_rne(float f) {
    uint32_t u;
    memcpy(&u, &f, sizeof u);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0;
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

uint16_t oracle_f32_to_bf16(float f) { return f32_to_bf16_rne(f); }
float oracle_bf16_to_f32(uint16_t h) { return bf16_to_f32(h); }

/* bf16(q) * bf16(s) -> bf16 (RNE).  w4.zig:49-52. */
uint16_t oracle_dequant_one(int32_t q, uint16_t s_bits) {
    return f32_to_bf16_rne((float)q * bf16_to_f32(s_bits));
}

/* pack_to_int32: q int8 [N, K] in [-8, 7] -> pk int32 [N, K/8].
 * Returns 0, or -1 if K % 8 != 0 or a value lies outside [-8, 7]. */
int oracle_pack(const int8_t *q, int32_t *pk, int64_t N, int64_t K) {
    if (K % 8 != 0) return -1;
    const int64_t W = K / 8;
    for (int64_t n = 0; n < N; ++n) {
        for (int64_t w = 0; w < W; ++w) {
            uint32_t word = 0;
            for (int j = 0; j < 8; ++j) {
                int v = q[n * K + 8 * w + j];
                if (v < -8 || v > 7) return -1;
                word |= (uint32_t)(v + 8) << (4 * j);
            }
            memcpy(&pk[n * W + w], &word, sizeof word);
        }
    }
    return 0;
}

/* unpackW4: pk int32 [N, K/8] -> q int8 [N, K].  Logical shift (w4.zig:38-39). */
int oracle_unpack(const int32_t *pk, int8_t *q, int64_t N, int64_t K) {
    if (K % 8 != 0) return -1;
    const int64_t W = K / 8;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t w = 0; w < W; ++w) {
            uint32_t word = (uint32_t)pk[n * W + w];
            for (int j = 0; j < 8; ++j)
                q[n * K + 8 * w + j] = (int8_t)((int32_t)((word >> (4 * j)) & 0xFu) - 8);
        }
    return 0;
}

/* dequantW4: pk [N, K/8] + sc bf16 [N, K/group] -> w bf16 [N, K]. */
int oracle_dequant(const int32_t *pk, const uint16_t *sc, uint16_t *w,
                   int64_t N, int64_t K, int64_t group) {
    if (group <= 0 || group % 8 != 0 || K % group != 0) return -1;
    const int64_t W = K / 8, G = K / group;
    for (int64_t n = 0; n < N; ++n)
        for (int64_t k = 0; k < K; ++k) {
            uint32_t word = (uint32_t)pk[n * W + k / 8];
            int32_t qv = (int32_t)((word >> (4 * (k % 8))) & 0xFu) - 8;
            w[n * K + k] = oracle_dequant_one(qv, sc[n * G + k / group]);
        }
    return 0;
}

/* y[m, n] = sum_k f32(x[m, k]) * f32(w[n, k]), k ascending, fp32 accumulate.
 * x bf16 [M, K], w bf16 [N, K] (already dequantized), y f32 [M, N]. */
void oracle_matmul_bf16_f32(const uint16_t *x, const uint16_t *w, float *y,
                            int64_t M, int64_t N, int64_t K) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float acc = 0.0f;
            const uint16_t *xr = x + m * K, *wr = w + n * K;
            for (int64_t k = 0; k < K; ++k) acc += bf16_to_f32(xr[k]) * bf16_to_f32(wr[k]);
            y[m * N + n] = acc;
        }
}

/* Same contraction, float64 accumulate; also returns sum_k |x||w| per output
 * (the magnitude that bounds the fp32 rounding error). */
void oracle_matmul_bf16_f64(const uint16_t *x, const uint16_t *w, double *y, double *absdot,
                            int64_t M, int64_t N, int64_t K) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            double acc = 0.0, mag = 0.0;
            const uint16_t *xr = x + m * K, *wr = w + n * K;
            for (int64_t k = 0; k < K; ++k) {
                double p = (double)bf16_to_f32(xr[k]) * (double)bf16_to_f32(wr[k]);
                acc += p;
                mag += fabs(p);
            }
            y[m * N + n] = acc;
            if (absdot) absdot[m * N + n] = mag;
        }
}

/* f32 activations (the engine's compute dtype, dotPrec fam = null with an f32
 * lhs, engine.zig:531-532): y = sum_k x[m, k] * f32(w[n, k]), fp32 and f64. */
void oracle_matmul_f32x_f32(const float *x, const uint16_t *w, float *y,
                            int64_t M, int64_t N, int64_t K) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            float acc = 0.0f;
            const float *xr = x + m * K;
            const uint16_t *wr = w + n * K;
            for (int64_t k = 0; k < K; ++k) acc += xr[k] * bf16_to_f32(wr[k]);
            y[m * N + n] = acc;
        }
}

void oracle_matmul_f32x_f64(const float *x, const uint16_t *w, double *y, double *absdot,
                            int64_t M, int64_t N, int64_t K) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t m = 0; m < M; ++m)
        for (int64_t n = 0; n < N; ++n) {
            double acc = 0.0, mag = 0.0;
            const float *xr = x + m * K;
            const uint16_t *wr = w + n * K;
            for (int64_t k = 0; k < K; ++k) {
                double p = (double)xr[k] * (double)bf16_to_f32(wr[k]);
                acc += p;
                mag += fabs(p);
            }
            y[m * N + n] = acc;
            if (absdot) absdot[m * N + n] = mag;
        }
}

/* The reference flow end to end: dequant (bit-exact bf16) then fp32 dot.
 * wbuf is caller scratch of N*K uint16. */
int oracle_linear(const uint16_t *x, const int32_t *pk, const uint16_t *sc, float *y,
                  uint16_t *wbuf, int64_t M, int64_t N, int64_t K, int64_t group) {
    int rc = oracle_dequant(pk, sc, wbuf, N, K, group);
    if (rc) return rc;
    oracle_matmul_bf16_f32(x, wbuf, y, M, N, K);
    return 0;
}

/* f32 -> bf16 RNE over an array (the bf16 output flavour, y_dtype = BF16). */
void oracle_round_bf16(const float *src, uint16_t *dst, int64_t n) {
    for (int64_t i = 0; i < n; ++i) dst[i] = f32_to_bf16_rne(src[i]);
}
