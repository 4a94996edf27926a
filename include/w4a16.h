/*
 * w4a16.h -- C ABI of the MI355X (gfx950) W4A16 library, libw4a16.so.
 *
 * Drop-in for the quantized hot path of TheCause/gemma4-zml-probe: the
 * `dequantW4` brick (zml_runner/w4.zig:33-54) and the decode matmul that
 * consumes its output (`dotPrec`, zml_runner/engine.zig:530-533), fused as
 * one call per linear.  In the reference these are ZML graph-construction
 * functions traced into one XLA executable; here each becomes one
 * stream-ordered call into hand-written HIP kernels.
 *
 * Weight format (compressed-tensors "pack-quantized", w4a16, symmetric;
 * zml_runner/w4.zig:4-10, docs/W4_RESULTS.md:28-37):
 *   pk  int32  [N, K/8]      nibble j of word w is column 8w+j, little
 *                            endian within the word; the nibble stores q+8
 *                            (unsigned), q in [-8, 7].
 *   sc  bf16   [N, K/group]  one scale per `group` consecutive columns along
 *                            K (the input dimension); group is 32 in every
 *                            checkpoint the reference loads.
 *   dequantized weight w[n][k] = RNE_bf16(q[n][k] * sc[n][k / group]).
 * Row-major everywhere.  bf16 values are passed as uint16_t bit patterns, the
 * way the reference's gates compare them (zml_runner/gemma4_w4gate.zig:98-111).
 *
 * Conventions
 *   - Every entry point returns W4A16_OK (0) or a negative w4a16_status and
 *     never aborts; w4a16_last_error() gives a thread-local message.
 *   - `stream` is a hipStream_t passed as void* (NULL = the default stream).
 *     Calls are stream-ordered and asynchronous: no implicit device sync, no
 *     host callbacks.  Stateless and reentrant; safe to call from several
 *     host threads on different streams.
 *   - The caller owns every device buffer.  No entry point allocates device
 *     memory.  w4a16_linear takes caller-provided workspace where a shape
 *     needs it, or where it makes a faster route possible (see
 *     w4a16_workspace_size).
 *   - Device pointers must be 16-byte aligned (pk, sc, x, y, q, w, workspace).
 *     Row strides are the dense ones implied by the shapes; K % group == 0
 *     and group % 32 == 0 are required.
 *   - M == 0 or N == 0 is a no-op; K == 0 writes zeros to y.
 */
#ifndef W4A16_H
#define W4A16_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define W4A16_ABI_VERSION 1

typedef enum w4a16_status {
    W4A16_OK = 0,
    W4A16_EINVAL_SHAPE = -1, /* negative dims, K % group, K % 8, size overflow   */
    W4A16_EINVAL_PTR = -2,   /* null or misaligned pointer                        */
    W4A16_EINVAL_ARG = -3,   /* unknown dtype / flag, unsupported group size      */
    W4A16_EWORKSPACE = -4,   /* workspace missing or smaller than required      */
    W4A16_EHIP = -5          /* HIP launch / runtime error (detail in last_error) */
} w4a16_status;

/* Element types of x and y. */
enum {
    W4A16_DTYPE_BF16 = 0,
    W4A16_DTYPE_F32 = 1
};

/* Library version (== W4A16_ABI_VERSION of the build). */
int w4a16_version(void);

/* Thread-local text of the last error raised on this host thread ("" if none). */
const char *w4a16_last_error(void);

/*
 * unpackW4 (zml_runner/w4.zig:33-45; exposed there for the W1 gate,
 * zml_runner/gemma4_w4gate.zig:44-48): pk int32 [N, K/8] -> q int8 [N, K],
 * q = ((word >> 4j) & 0xF) - 8 with a logical shift.  Bit-exact.
 */
int w4a16_unpack(const int32_t *pk, int8_t *q, int64_t N, int64_t K, void *stream);

/*
 * dequantW4 (zml_runner/w4.zig:47-54) == W4Lin.toW (w4.zig:28-30) without the
 * retag: pk [N, K/8] + sc bf16 [N, K/group] -> w bf16 [N, K],
 * w = RNE_bf16(q * s) (bf16 x bf16 -> bf16, NaN -> 0x7FC0).  Bit-exact.
 */
int w4a16_dequant(const int32_t *pk, const uint16_t *sc, uint16_t *w,
                  int64_t N, int64_t K, int32_t group, void *stream);

/*
 * Bytes of device workspace w4a16_linear can use for (M, N, K, x_dtype).
 * x_dtype = W4A16_DTYPE_F32: 6 * M * K bytes (rounded up to 256) to hold the
 * three bf16 terms of x, required; above M = 4 plus 12 * M * N bytes (rounded up to
 * 256) and the bf16 split-K part for 3M rows, optional: given all of it, the three
 * planes run as 3M rows of bf16 x through the bf16 routes and their results are
 * added in plane order (deterministic); with only the first part, one generic kernel
 * reads the three planes.  Both meet the same fp32 bound.  (At M <= 4 the decode
 * GEMV splits x itself.)
 * x_dtype = W4A16_DTYPE_BF16: nothing is required.  On shapes whose one-pass
 * kernel cannot fill the GPU (K % 64 == 0, and: 64 < M <= 128, or up to 256
 * with K <= 8192, with K % 256 == 0 while the skinny kernel's grid of
 * ceil(M / 64) * ceil(N / 64) workgroups is at most 128; other rows above
 * M = 64 with fewer than 240 workgroups of 256 x 128, and N <= 8192 up to
 * M = 128; or N < 16384 and:
 * 16 < M <= 64; 4 < M <= 16 beyond the 16-row decode GEMV with K >= 8192 or
 * N < 8192; M <= 4 with K % 256 == 0 and x beyond the decode GEMV's 64 KiB of
 * LDS; with K % 256 == 0 at M <= 64 only while the skinny kernel's one-pass grid
 * has at most 128 workgroups -- the 12B q/k/v/o rows at M > 16, down at M >= 3 up
 * to M = 1024, E2B
 * down at M = 16) it is the size of kq f32 partial planes, kq * M * N * 4 bytes
 * rounded up to 256 with 2 <= kq <= 64 K parts; given at least that much, the
 * call splits K across workgroups and adds the parts in a second launch in a
 * fixed order (deterministic).  With less, or NULL, it takes the one-pass route;
 * both meet the same fp32 bound.  0 otherwise.
 */
size_t w4a16_workspace_size(int64_t M, int64_t N, int64_t K, int32_t x_dtype);

/*
 * The fused unit: y[M, N] = x[M, K] . dequantW4(pk, sc)^T, i.e. G3.forward
 * (zml_runner/gemma4_w4gate.zig:288-292) and every dotPrec site that consumes
 * a W4Lin (zml_runner/engine.zig:552,571,583,649,653,659,661,723 through
 * W4Lin.toW, zml_runner/w4.zig:28-30).  Replaces "x.dot(lin.toW())".
 *
 * Numerics: each weight is rounded exactly as dequantW4 rounds it
 * (RNE_bf16(q * s)); products with x are exact and accumulate in fp32, as in
 * dotPrec with fam = null (engine.zig:531-532).  Only the summation order
 * differs from the reference.
 * Scale range: the in-register dequant is exact for 2^-126 <= |s| < 2^117 and
 * s = +-0, which holds for every scale a quantizer writes (max|w| / 7.5 of a
 * finite bf16 row group).  Outside it the fused kernels may differ from
 * w4a16_dequant followed by a dot: a subnormal scale may be flushed to zero (its
 * group's weights count as 0), and from |s| >= 2^117 the expansion's fp32
 * intermediates ((1024 + n) * s in the decode GEMV, (128 + n) * s elsewhere) may
 * overflow, so such scales (and +-inf / NaN ones) can give +-inf or NaN outputs.  w4a16_dequant is exact for every bit
 * pattern.  The same holds for w4a16_linear_group and w4a16_gate_up_gelu.
 *   x_dtype  W4A16_DTYPE_BF16 or W4A16_DTYPE_F32 (the
 *            engine's f32 activations; carried exactly as a sum of three bf16
 *            terms, so no precision is lost before the fp32 accumulate).
 *   y_dtype  W4A16_DTYPE_F32 (fam = null flow) or W4A16_DTYPE_BF16 (the fp32
 *            result rounded to nearest even once, as the bf16 dot of the
 *            fam = bf16 flow).
 *   flags    must be 0.
 *   workspace / ws_bytes  f32 x: at least the x-planes part of
 *            w4a16_workspace_size, W4A16_EWORKSPACE otherwise; bf16 x: optional
 *            (NULL / 0 allowed), the split-K route when ws_bytes reaches
 *            w4a16_workspace_size(M, N, K, x_dtype).
 */
int w4a16_linear(const void *x, int32_t x_dtype,
                 const int32_t *pk, const uint16_t *sc,
                 void *y, int32_t y_dtype,
                 int64_t M, int64_t N, int64_t K, int32_t group,
                 int32_t flags, void *workspace, size_t ws_bytes, void *stream);

/*
 * w4a16_linear without a workspace argument, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  No counterpart in the reference (its dequant temporaries
 * live in the XLA arena).  It allocates nothing and calls no allocating routine:
 * the f32-activation planes and the split-K partial sums that w4a16_linear keeps in
 * the caller's workspace go to a static device array of 8 MiB per GPU, held until
 * the process ends (its address is looked up once per device, on the first call
 * with that device current).  Same results as w4a16_linear given an 8 MiB
 * workspace: f32 x needs 6 * M * K <= 8 MiB (rounded up to 256), else
 * W4A16_EWORKSPACE before any HIP call; bf16 x takes the split-K route when its
 * partials fit, else the one-pass route.  Every call on one GPU shares that array:
 * calls that overlap on one GPU (different streams without ordering between them)
 * race.  The stream must belong to the current device.
 */
int w4a16_linear_noalloc(const void *x, int32_t x_dtype,
                         const int32_t *pk, const uint16_t *sc,
                         void *y, int32_t y_dtype,
                         int64_t M, int64_t N, int64_t K, int32_t group,
                         int32_t flags, void *stream);

/*
 * Several linears that read the same activations, y_j[M, N_j] = x[M, K] .
 * dequantW4(pk_j, sc_j)^T for j < n (1 <= n <= 4): q, k and v of a layer, which all
 * take the normed hidden h0 (zml_runner/engine.zig:552,571,583).  Each y_j is
 * exactly what w4a16_linear gives for that weight; at decode (M <= 16) the n
 * linears run as one launch when every one of them would take the same decode
 * GEMV plan on its own (the 12B and E2B q/k/v shapes do), otherwise one launch
 * each.  pk, sc, y and N are
 * host arrays of n entries; every weight has K columns and the same group.
 * Workspace as w4a16_linear: f32 x needs w4a16_workspace_size(M, 0, K, x_dtype);
 * with bf16 x, optional, each member that runs as its own launch takes the
 * split-K route when ws_bytes reaches w4a16_workspace_size(M, N_j, K, x_dtype)
 * (pass the largest over the members for all of them).
 */
int w4a16_linear_group(const void *x, int32_t x_dtype, int32_t n,
                       const int32_t *const *pk, const uint16_t *const *sc,
                       void *const *y, const int64_t *N, int32_t y_dtype,
                       int64_t M, int64_t K, int32_t group,
                       int32_t flags, void *workspace, size_t ws_bytes, void *stream);

/* Flags of w4a16_gate_up_gelu. */
enum {
    /* g and u rounded to bf16 before the activation: the dot outputs of dotPrec
     * with fam = bf16 (engine.zig:531, a.convert(bf16).dot(..).convert(compute)). */
    W4A16_GATE_UP_BF16_DOTS = 1
};

/*
 * Bytes of device workspace w4a16_gate_up_gelu can use for (M, F, K, x_dtype).
 * Required: the f32-activation x planes of w4a16_workspace_size, plus
 * 2 * 4 * M * F bytes for f32 g and u on shapes that no fused kernel takes
 * (then g and u make a round trip through the workspace).  That second part is
 * 0 when a fused kernel takes the shape: bf16 x with K % 256 == 0 (any M) or
 * with M > 64 and K % 64 == 0 (every Gemma gate/up shape: K = 1536 or 3840);
 * f32 x in the decode GEMV (M <= 4, K % 256 == 0, within its LDS and register
 * limits).  Optional, added on top: bf16 x takes the split-K route of
 * w4a16_linear (same shape rules) over the 16 * ceil(F / 8) interleaved
 * gate/up rows when that row count is below 16384 (E2B: F = 6144 at M > 16),
 * with the activation applied when the parts are added; f32 x above M = 4 (the
 * unfused route) takes g and u each as w4a16_linear does with the optional part of
 * w4a16_workspace_size(M, F, K, x_dtype), here the room after g and u.
 */
size_t w4a16_gate_up_workspace_size(int64_t M, int64_t F, int64_t K, int32_t x_dtype);

/*
 * The front half of Gemma's MLP at engine.zig:653, both W4 linears and the
 * activation in one call:
 *     h[M, F] = gelu(x . Wg^T) * (x . Wu^T),
 *     Wg = dequantW4(pk_gate, sc_gate), Wu = dequantW4(pk_up, sc_up), both [F, K],
 *     gelu(g) = 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3)))  (ZML Tensor.gelu,
 *     the gelu_pytorch_tanh of the checkpoint config).
 * Replaces "dotPrec(xff, gate_proj).gelu().mul(dotPrec(xff, up_proj))"; h then
 * feeds down_proj through w4a16_linear.  g and u are exactly the two results
 * w4a16_linear would produce in fp32 (same rounding of the weights, fp32
 * accumulate); the activation and the product are evaluated in fp32.  On the
 * fused shapes g and u never leave the registers: one launch reads x, both
 * weights and writes h.
 *   x_dtype   as w4a16_linear.
 *   h_dtype   W4A16_DTYPE_F32 (compute = f32) or W4A16_DTYPE_BF16 (h rounded
 *             once to nearest even).
 *   flags     0 or W4A16_GATE_UP_BF16_DOTS.
 *   group     shared by both weights.
 *   workspace / ws_bytes  at least the required part of
 *             w4a16_gate_up_workspace_size (W4A16_EWORKSPACE otherwise); the
 *             split-K route when it reaches the whole size.
 */
int w4a16_gate_up_gelu(const void *x, int32_t x_dtype,
                       const int32_t *pk_gate, const uint16_t *sc_gate,
                       const int32_t *pk_up, const uint16_t *sc_up,
                       void *h, int32_t h_dtype,
                       int64_t M, int64_t F, int64_t K, int32_t group,
                       int32_t flags, void *workspace, size_t ws_bytes, void *stream);

/*
 * Bytes of device workspace w4a16_lm_head needs: the f32-activation split of
 * w4a16_workspace_size (x_dtype F32, K > 0) plus 8 * M * ceil(V / S) * topk bytes
 * of top-k candidates, S = 1024 when ceil(V / 1024) * topk <= 4096 and 4096
 * otherwise (0 when topk is 0), rounded up to 256.  The candidate part does not
 * depend on K: at K == 0 the logits are zeros and the top-k still runs.
 */
size_t w4a16_lm_head_workspace_size(int64_t M, int64_t V, int64_t K, int32_t x_dtype, int32_t topk);

/*
 * The lm_head of the decode step (zml_runner/engine.zig:765-766) and its topK
 * (zml_runner/gemma4_g12auto.zig:1532):
 *     raw[M, V]    = x[M, K] . embed[V, K]^T   (the tied bf16 embedding, f32 accumulate:
 *                                               dotPrec(prec.head, compute, ...) with fam = null)
 *     logits[M, V] = cap * tanh(raw / cap)     (softcapPrec, engine.zig:193-195; cap = 0: raw)
 *     top_values[M, topk], top_indices[M, topk]: the topk largest logits of each row,
 *                    descending; equal values in ascending index order; NaN counts as larger
 *                    than +inf.  NaN logits are written as the quiet NaN 0x7FC00000.
 *   x_dtype   W4A16_DTYPE_BF16 or W4A16_DTYPE_F32 (carried exactly, as in w4a16_linear).
 *   embed     bf16 [V, K], row-major; K % 32 == 0 and K <= 8192 (W4A16_EINVAL_SHAPE otherwise).
 *   logits    f32 [M, V] output (the step returns it alongside the top-k).
 *   topk      0..64 with topk <= V and ceil(V / 4096) * topk <= 4096; 0 skips the top-k
 *             (top_values / top_indices may then be NULL).
 * The kernels read embed once per launch of up to 16 rows of x at K = 3840 (5 with
 * f32 x): the decode head (M = 1) and a batch of up to 16 sequences in one pass.
 */
int w4a16_lm_head(const void *x, int32_t x_dtype, const uint16_t *embed, float *logits,
                  int64_t M, int64_t V, int64_t K, float softcap, int32_t topk,
                  float *top_values, int32_t *top_indices,
                  void *workspace, size_t ws_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* W4A16_H */
