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

// Decode GEMV path (M <= 4, x planes fit in 64 KiB of LDS).
bool w4l_gemv_ok(int64_t M, int64_t K, int nterms);
int w4l_gemv_waves(int64_t N, int64_t K);
bool w4l_gemv_stream_plan(int64_t M, int64_t N, int64_t K, int nterms, int* w, int* nst, int* cpw, int* xpt);
bool w4l_gemv_fast_plan(int64_t M, int64_t N, int64_t K, int nterms, int* nst, int* waves, int* xpt, int* tpw);
hipError_t w4l_gemv(const uint16_t* x_planes, int nterms, const int32_t* pk, const uint16_t* sc,
                    void* y, int y_f32, int64_t M, int64_t N, int64_t K, int32_t group,
                    hipStream_t st);

// Skinny / prefill path (M > 4, bf16 x, K % 256 == 0).
bool w4l_skinny_ok(int64_t M, int64_t K, int nterms);
hipError_t w4l_skinny(const uint16_t* x, const int32_t* pk, const uint16_t* sc, void* y, int y_f32,
                      int64_t M, int64_t N, int64_t K, int32_t group, hipStream_t st);

// Prefill path (M > 64, bf16 x, K % 64 == 0).
bool w4l_prefill_ok(int64_t M, int64_t K, int nterms);
hipError_t w4l_prefill(const uint16_t* x, const int32_t* pk, const uint16_t* sc, void* y, int y_f32,
                       int64_t M, int64_t N, int64_t K, int32_t group, hipStream_t st);

hipError_t w4l_unpack(const int32_t* pk, int8_t* q, int64_t nwords, hipStream_t st);
hipError_t w4l_dequant(const int32_t* pk, const uint16_t* sc, uint16_t* w, int64_t N, int64_t K,
                       int32_t group, hipStream_t st);
hipError_t w4l_split3(const float* x, uint16_t* out, int64_t n, hipStream_t st);
hipError_t w4l_fill_zero(void* p, int64_t bytes, hipStream_t st);
hipError_t w4l_linear(const uint16_t* x_planes, int nterms, const int32_t* pk, const uint16_t* sc,
                      void* y, int y_f32, int64_t M, int64_t N, int64_t K, int32_t group,
                      hipStream_t st);
