// w4a16_launch.h -- internal launcher interface between the C ABI
// (w4a16_abi.cpp) and the kernels (w4a16_kernels.hip).  Not installed.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Launch bound of linear_kernel<MT, NT>: register-heavier variants get fewer
// threads per workgroup so that the compiler may use more VGPRs per lane.
#define W4_MAXT(MT_, NT_) (((MT_) * (NT_)) <= 2 ? 1024 : 512)

struct W4Plan {
  int mt;      // 16-row m-tiles per workgroup (1..4)
  int grid_m;  // workgroups along M
  int grid_n;  // workgroups along N (16 rows each)
  int waves;   // waves per workgroup, splitting K
};

W4Plan w4l_plan(int64_t M, int64_t N, int64_t K, int nterms);

// Gate/up pair of the fused MLP front half (engine.zig:653): the launch's pk/sc
// are the gate weight, these the up weight, both [F, K]; the output is
// h[M, F] = gelu_tanh(g) * u.  Kernels that take one run over 16 * ceil(F / 8)
// virtual rows (8 gate rows, then the 8 matching up rows, per 16-row tile).
struct W4Pair {
  const int32_t* pk_up;
  const uint16_t* sc_up;
  int64_t F;
  int bf16_dots;  // round g and u to bf16 before gelu
};

// Decode GEMV path (M <= 4, x planes fit in 64 KiB of LDS).
bool w4l_gemv_ok(int64_t M, int64_t K, int nterms);
// 4 < M <= 16 through the same GEMV kernel (bf16 x, small N); w4l_gemv takes it.
bool w4l_gemv16_ok(int64_t M, int64_t N, int64_t K, int nterms);
int w4l_gemv_waves(int64_t N, int64_t K);
// The straight-line decode GEMV (4-row epilogue) takes (M, N, K, nterms).
bool w4l_gemv_fast_ok(int64_t M, int64_t N, int64_t K, int nterms);
// With a pair, only the straight-line plans are used (hipErrorInvalidValue when
// neither holds) and N is ignored.
// xf: f32 x [M][K] read by the GEMV itself (its three bf16 planes staged per wave; x_planes
// and nterms are then ignored) where w4l_gemv_f32x_ok holds (hipErrorInvalidValue otherwise).
hipError_t w4l_gemv(const uint16_t* x_planes, int nterms, const int32_t* pk, const uint16_t* sc,
                    void* y, int y_f32, int64_t M, int64_t N, int64_t K, int32_t group,
                    hipStream_t st, const W4Pair* pair = nullptr, const float* xf = nullptr);
// The decode GEMV takes f32 x directly (N = the pair's virtual rows 16 * ceil(F / 8) with pair).
bool w4l_gemv_f32x_ok(int64_t M, int64_t N, int64_t K, int32_t group, bool pair);
// f32 x better served by its planes run as 3M rows of bf16 x (M > 4, or planes beyond the
// decode GEMV's 64 KB at M >= 2, or no decode plan)
bool w4l_f32x_rows(int64_t M, int64_t N, int64_t K);

// Skinny / prefill path (M > 4, bf16 x, K % 256 == 0).
bool w4l_skinny_ok(int64_t M, int64_t K, int nterms);
// kq > 1 splits K into kq parts (K / 256 divisible by kq) with f32 partials
// part[kq][M][N] (virtual rows in pair mode) and a finalize launch.
hipError_t w4l_skinny(const uint16_t* x, const int32_t* pk, const uint16_t* sc, void* y, int y_f32,
                      int64_t M, int64_t N, int64_t K, int32_t group, hipStream_t st,
                      const W4Pair* pair = nullptr, int kq = 1, float* part = nullptr);

// Prefill path (M > 64, bf16 x, K % 64 == 0).
bool w4l_prefill_ok(int64_t M, int64_t K, int nterms);
hipError_t w4l_prefill(const uint16_t* x, const int32_t* pk, const uint16_t* sc, void* y, int y_f32,
                       int64_t M, int64_t N, int64_t K, int32_t group, hipStream_t st,
                       const W4Pair* pair = nullptr);

// Weight group: n <= 4 linears [N_j, K] that read the same x (q, k, v), one
// launch of the straight-line GEMV when w4l_group_fused (every member would run that
// GEMV with the same plan on its own, so each y_j equals w4l_linear's bit for bit);
// otherwise the caller runs w4l_linear per weight.
bool w4l_group_fused(int64_t M, int n, const int64_t* N, int64_t K, int nterms);
// y[m][n] = (y3[0][m][n] + y3[1][m][n]) + y3[2][m][n] for y3 [3][M][N] f32 (the three bf16
// planes of f32 x run as 3M rows), f32 or bf16 (RNE) out.
hipError_t w4l_add_planes(const float* y3, int64_t M, int64_t N, void* y, int y_f32, hipStream_t st);

// xf: f32 x read by the GEMV itself (as w4l_gemv), where w4l_group_f32x_ok holds.
hipError_t w4l_gemv_group(const uint16_t* x_planes, int nterms, int n, const int32_t* const* pk,
                          const uint16_t* const* sc, void* const* y, const int64_t* N, int y_f32, int64_t M, int64_t K,
                          int32_t group, hipStream_t st, const float* xf = nullptr);
bool w4l_group_f32x_ok(int64_t M, int n, const int64_t* N, int64_t K, int32_t group);

// Fused gate/up + gelu * mul: true when one of the three kernels above takes
// (M, F, K, nterms) in pair mode; w4l_gate_up launches it.  Otherwise the
// caller composes two w4l_linear calls into f32 g, u and w4l_gelu_mul.
bool w4l_gate_up_fused(int64_t M, int64_t F, int64_t K, int nterms);
hipError_t w4l_gate_up(const uint16_t* x_planes, int nterms, const int32_t* pk_gate, const uint16_t* sc_gate,
                       const W4Pair& pair, void* h, int h_f32, int64_t M, int64_t K, int32_t group,
                       hipStream_t st);
hipError_t w4l_gelu_mul(const float* g, const float* u, void* h, int h_f32, int bf16_dots, int64_t n,
                        hipStream_t st);

// Static device scratch of w4a16_linear_noalloc (w4a16_scratch.hip): W4L_SCRATCH_BYTES
// bytes per GPU, whose address on the current device this returns (looked up once
// per device).
#define W4L_SCRATCH_BYTES (8u << 20)
hipError_t w4l_scratch(void** ptr);

hipError_t w4l_unpack(const int32_t* pk, int8_t* q, int64_t nwords, hipStream_t st);
hipError_t w4l_dequant(const int32_t* pk, const uint16_t* sc, uint16_t* w, int64_t N, int64_t K,
                       int32_t group, hipStream_t st);
hipError_t w4l_split3(const float* x, uint16_t* out, int64_t n, hipStream_t st);
hipError_t w4l_fill_zero(void* p, int64_t bytes, hipStream_t st);
hipError_t w4l_linear(const uint16_t* x_planes, int nterms, const int32_t* pk, const uint16_t* sc,
                      void* y, int y_f32, int64_t M, int64_t N, int64_t K, int32_t group,
                      hipStream_t st);
// Split-K route (bf16 x, M <= 64, shapes whose one-pass grid is small): bytes of f32 partial
// sums it needs (0 when the shape does not take it) and the launch (main kernel
// + finalize); with pair set, N is ignored and the output is h [M, F].
size_t w4l_splitk_bytes(int64_t M, int64_t N, int64_t K, int nterms);
hipError_t w4l_splitk(const uint16_t* x, const int32_t* pk, const uint16_t* sc, void* y, int y_f32, int64_t M,
                      int64_t N, int64_t K, int32_t group, hipStream_t st, const W4Pair* pair, float* part);

// lm_head (w4a16_head.hip): f32 logits of a bf16 [V, K] embedding with the
// softcap applied, for up to w4l_head_rows(K, nterms) rows of x per launch
// (0 when K is not a multiple of 32), and the deterministic top-k over them
// (w4l_topk_parts(V, k) * k candidate keys of scratch per row).
int w4l_head_rows(int64_t K, int nterms);
// x_planes: nterms planes of [M][K] bf16, xplane halves apart
hipError_t w4l_head_logits(const uint16_t* x_planes, int64_t xplane, int nterms, const uint16_t* e, float* logits,
                           int64_t M, int64_t V, int64_t K, float cap, hipStream_t st);
int64_t w4l_topk_parts(int64_t V, int k);
hipError_t w4l_topk(const float* logits, int64_t M, int64_t V, int k, uint64_t* cand, float* values,
                    int32_t* indices, hipStream_t st);
