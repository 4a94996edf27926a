// w4a16_abi.cpp -- the C ABI declared in include/w4a16.h.
//
// Validates every argument on the host before any HIP call (so the error
// paths are testable without a GPU), records a thread-local message, and
// dispatches to the gfx950 kernels in w4a16_kernels.hip.  Nothing here
// allocates device memory.
//
// Boundary it replaces: the ZML graph functions unpackW4 / dequantW4
// (zml_runner/w4.zig:33-54) and the dotPrec contraction that consumes the
// dequantized weight (zml_runner/engine.zig:530-533), fused per linear as in
// G3.forward (zml_runner/gemma4_w4gate.zig:288-292).  In the reference a
// shape or tag mismatch is a compile-time error of the traced graph
// (zml_runner/w4.zig:116-117); here it is a negative status code.

#include "../../include/w4a16.h"

#include <hip/hip_runtime.h>

#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "w4a16_launch.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof g_err, fmt, ap);
  va_end(ap);
  return code;
}

void clear_err() { g_err[0] = '\0'; }

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_ptr(const void* p, const char* name, const char* fn) {
  if (p == nullptr) return fail(W4A16_EINVAL_PTR, "%s: %s is NULL", fn, name);
  if (!aligned16(p)) return fail(W4A16_EINVAL_PTR, "%s: %s is not 16-byte aligned", fn, name);
  return W4A16_OK;
}

int hip_status(hipError_t e, const char* fn) {
  if (e == hipSuccess) return W4A16_OK;
  return fail(W4A16_EHIP, "%s: HIP error %d (%s)", fn, (int)e, hipGetErrorString(e));
}

// Shared shape checks: dims in [0, INT_MAX], K % 8 (and % group when given).
int check_dims(const char* fn, int64_t M, int64_t N, int64_t K) {
  if (M < 0 || N < 0 || K < 0)
    return fail(W4A16_EINVAL_SHAPE, "%s: negative dimension (M=%lld N=%lld K=%lld)", fn,
                (long long)M, (long long)N, (long long)K);
  if (M > INT_MAX || N > INT_MAX || K > INT_MAX)
    return fail(W4A16_EINVAL_SHAPE, "%s: dimension above INT_MAX", fn);
  if (K % 8 != 0) return fail(W4A16_EINVAL_SHAPE, "%s: K=%lld is not a multiple of 8", fn, (long long)K);
  return W4A16_OK;
}

int check_group(const char* fn, int64_t K, int32_t group) {
  if (group < 32 || group % 32 != 0)
    return fail(W4A16_EINVAL_ARG, "%s: group=%d must be a positive multiple of 32", fn, (int)group);
  if (K % group != 0)
    return fail(W4A16_EINVAL_SHAPE, "%s: K=%lld is not a multiple of group=%d", fn, (long long)K,
                (int)group);
  return W4A16_OK;
}

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

}  // namespace

extern "C" {

int w4a16_version(void) { return W4A16_ABI_VERSION; }

const char* w4a16_last_error(void) { return g_err; }

int w4a16_unpack(const int32_t* pk, int8_t* q, int64_t N, int64_t K, void* stream) {
  static const char* fn = "w4a16_unpack";
  clear_err();
  int rc = check_dims(fn, 0, N, K);
  if (rc) return rc;
  if (N == 0 || K == 0) return W4A16_OK;
  if ((rc = check_ptr(pk, "pk", fn)) || (rc = check_ptr(q, "q", fn))) return rc;
  return hip_status(w4l_unpack(pk, q, N * (K / 8), static_cast<hipStream_t>(stream)), fn);
}

int w4a16_dequant(const int32_t* pk, const uint16_t* sc, uint16_t* w, int64_t N, int64_t K,
                  int32_t group, void* stream) {
  static const char* fn = "w4a16_dequant";
  clear_err();
  int rc = check_dims(fn, 0, N, K);
  if (rc) return rc;
  if ((rc = check_group(fn, K, group))) return rc;
  if (N == 0 || K == 0) return W4A16_OK;
  if ((rc = check_ptr(pk, "pk", fn)) || (rc = check_ptr(sc, "sc", fn)) || (rc = check_ptr(w, "w", fn)))
    return rc;
  return hip_status(w4l_dequant(pk, sc, w, N, K, group, static_cast<hipStream_t>(stream)), fn);
}

namespace {
// f32 activations: their three bf16 planes (required workspace)
size_t x_split_bytes(int64_t M, int64_t K, int32_t x_dtype) {
  if (M <= 0 || K <= 0 || x_dtype != W4A16_DTYPE_F32) return 0;
  return round_up((size_t)(3 * 2) * (size_t)M * (size_t)K, 256);
}
// f32 activations above M = 4 (or with planes too wide for the decode GEMV): the three
// planes' results when the planes run as 3M rows of bf16 x through the bf16 routes
// (optional; without it the three-plane kernels)
// (then, for the 3M rows, the split-K partial sums where the bf16 route splits K)
size_t f32_rows_bytes(int64_t M, int64_t N, int64_t K, int32_t x_dtype) {
  if (M <= 0 || N <= 0 || K <= 0 || x_dtype != W4A16_DTYPE_F32 || M > INT_MAX / 3 || !w4l_f32x_rows(M, N, K))
    return 0;
  return round_up((size_t)12 * (size_t)M * (size_t)N, 256) + round_up(w4l_splitk_bytes(3 * M, N, K, 1), 256);
}
// bf16 activations, 4 < M <= 64: the split-K partial sums (optional workspace;
// without it the call takes the one-pass skinny route)
size_t splitk_bytes(int64_t M, int64_t N, int64_t K, int32_t x_dtype) {
  if (M <= 0 || N <= 0 || K <= 0 || x_dtype != W4A16_DTYPE_BF16) return 0;
  return round_up(w4l_splitk_bytes(M, N, K, 1), 256);
}
}  // namespace

size_t w4a16_workspace_size(int64_t M, int64_t N, int64_t K, int32_t x_dtype) {
  return x_split_bytes(M, K, x_dtype) + f32_rows_bytes(M, N, K, x_dtype) + splitk_bytes(M, N, K, x_dtype);
}

namespace {
// f32 x at M > 4 given the planes and f32_rows_bytes of workspace: the planes as 3M rows of
// bf16 x through the bf16 routes into y3, then the three results added in plane order
hipError_t f32_rows_linear(const uint16_t* planes, const int32_t* pk, const uint16_t* sc, void* y, int y_f32,
                           int64_t M, int64_t N, int64_t K, int32_t group, float* y3, hipStream_t st) {
  const size_t y3_bytes = round_up((size_t)12 * (size_t)M * (size_t)N, 256);
  hipError_t e = w4l_splitk_bytes(3 * M, N, K, 1)
                     ? w4l_splitk(planes, pk, sc, y3, 1, 3 * M, N, K, group, st, nullptr,
                                  reinterpret_cast<float*>(reinterpret_cast<char*>(y3) + y3_bytes))
                     : w4l_linear(planes, 1, pk, sc, y3, 1, 3 * M, N, K, group, st);
  if (e != hipSuccess) return e;
  return w4l_add_planes(y3, M, N, y, y_f32, st);
}
}  // namespace

namespace {
// argument checks shared by w4a16_linear and w4a16_linear_noalloc (no HIP call)
int linear_args(const char* fn, int32_t x_dtype, int32_t y_dtype, int64_t M, int64_t N, int64_t K, int32_t group,
                int32_t flags) {
  int rc = check_dims(fn, M, N, K);
  if (rc) return rc;
  if ((rc = check_group(fn, K, group))) return rc;
  if (x_dtype != W4A16_DTYPE_BF16 && x_dtype != W4A16_DTYPE_F32)
    return fail(W4A16_EINVAL_ARG, "%s: unknown x_dtype %d", fn, (int)x_dtype);
  if (y_dtype != W4A16_DTYPE_BF16 && y_dtype != W4A16_DTYPE_F32)
    return fail(W4A16_EINVAL_ARG, "%s: unknown y_dtype %d", fn, (int)y_dtype);
  if (flags != 0) return fail(W4A16_EINVAL_ARG, "%s: unknown flags 0x%x", fn, (unsigned)flags);
  return W4A16_OK;
}
}  // namespace

int w4a16_linear(const void* x, int32_t x_dtype, const int32_t* pk, const uint16_t* sc, void* y,
                 int32_t y_dtype, int64_t M, int64_t N, int64_t K, int32_t group, int32_t flags,
                 void* workspace, size_t ws_bytes, void* stream) {
  static const char* fn = "w4a16_linear";
  clear_err();
  int rc = linear_args(fn, x_dtype, y_dtype, M, N, K, group, flags);
  if (rc) return rc;
  if (M == 0 || N == 0) return W4A16_OK;
  if ((rc = check_ptr(y, "y", fn))) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int y_f32 = y_dtype == W4A16_DTYPE_F32;
  if (K == 0) return hip_status(w4l_fill_zero(y, M * N * (y_f32 ? 4 : 2), st), fn);
  if ((rc = check_ptr(x, "x", fn)) || (rc = check_ptr(pk, "pk", fn)) || (rc = check_ptr(sc, "sc", fn)))
    return rc;

  const uint16_t* planes = static_cast<const uint16_t*>(x);
  int nterms = 1;
  if (x_dtype == W4A16_DTYPE_F32) {
    const size_t need = x_split_bytes(M, K, x_dtype);
    if (workspace == nullptr || ws_bytes < need)
      return fail(W4A16_EWORKSPACE, "%s: f32 activations need %zu bytes of workspace, got %zu", fn,
                  need, workspace ? ws_bytes : (size_t)0);
    if ((rc = check_ptr(workspace, "workspace", fn))) return rc;
    // the decode GEMV splits f32 x into its three bf16 planes itself (one launch, the
    // same planes); other routes take the planes from the workspace
    if (w4l_gemv_f32x_ok(M, N, K, group, false))
      return hip_status(w4l_gemv(nullptr, 3, pk, sc, y, y_f32, M, N, K, group, st, nullptr,
                                 static_cast<const float*>(x)),
                        fn);
    uint16_t* split = static_cast<uint16_t*>(workspace);
    if ((rc = hip_status(w4l_split3(static_cast<const float*>(x), split, M * K, st), fn))) return rc;
    const size_t rows = f32_rows_bytes(M, N, K, x_dtype);
    if (rows && ws_bytes >= need + rows)
      return hip_status(f32_rows_linear(split, pk, sc, y, y_f32, M, N, K, group,
                                        reinterpret_cast<float*>(static_cast<char*>(workspace) + need), st),
                        fn);
    planes = split;
    nterms = 3;
  } else if (workspace != nullptr && !aligned16(workspace)) {
    return fail(W4A16_EINVAL_PTR, "%s: workspace is not 16-byte aligned", fn);
  } else if (workspace != nullptr) {
    const size_t sk = splitk_bytes(M, N, K, x_dtype);
    if (sk && ws_bytes >= sk)
      return hip_status(w4l_splitk(planes, pk, sc, y, y_f32, M, N, K, group, st, nullptr,
                                   static_cast<float*>(workspace)),
                        fn);
  }
  return hip_status(w4l_linear(planes, nterms, pk, sc, y, y_f32, M, N, K, group, st), fn);
}

int w4a16_linear_noalloc(const void* x, int32_t x_dtype, const int32_t* pk, const uint16_t* sc, void* y,
                         int32_t y_dtype, int64_t M, int64_t N, int64_t K, int32_t group, int32_t flags,
                         void* stream) {
  static const char* fn = "w4a16_linear_noalloc";
  clear_err();
  int rc = linear_args(fn, x_dtype, y_dtype, M, N, K, group, flags);
  if (rc) return rc;
  if (M == 0 || N == 0) return W4A16_OK;
  if ((rc = check_ptr(y, "y", fn))) return rc;
  if (K > 0 && ((rc = check_ptr(x, "x", fn)) || (rc = check_ptr(pk, "pk", fn)) || (rc = check_ptr(sc, "sc", fn))))
    return rc;
  const size_t need = x_split_bytes(M, K, x_dtype);
  if (need > W4L_SCRATCH_BYTES)
    return fail(W4A16_EWORKSPACE, "%s: f32 activations need %zu bytes of scratch, beyond its %u-byte maximum", fn,
                need, (unsigned)W4L_SCRATCH_BYTES);
  void* scratch = nullptr;
  if ((rc = hip_status(w4l_scratch(&scratch), fn))) return rc;
  // the same routes as w4a16_linear given a W4L_SCRATCH_BYTES workspace: the f32 planes,
  // or the split-K partials when they fit (else the one-pass route)
  rc = w4a16_linear(x, x_dtype, pk, sc, y, y_dtype, M, N, K, group, flags, scratch, W4L_SCRATCH_BYTES, stream);
  if (rc) {
    char msg[sizeof g_err];
    snprintf(msg, sizeof msg, "%s", g_err);
    return fail(rc, "%s: %s", fn, msg);
  }
  return W4A16_OK;
}

int w4a16_linear_group(const void* x, int32_t x_dtype, int32_t n, const int32_t* const* pk,
                       const uint16_t* const* sc, void* const* y, const int64_t* N, int32_t y_dtype, int64_t M,
                       int64_t K, int32_t group, int32_t flags, void* workspace, size_t ws_bytes, void* stream) {
  static const char* fn = "w4a16_linear_group";
  clear_err();
  if (n < 1 || n > 4) return fail(W4A16_EINVAL_ARG, "%s: n=%d outside 1..4", fn, (int)n);
  if (pk == nullptr || sc == nullptr || y == nullptr || N == nullptr)
    return fail(W4A16_EINVAL_PTR, "%s: pk, sc, y and N must be arrays of n entries", fn);
  int rc;
  for (int j = 0; j < n; ++j)
    if ((rc = check_dims(fn, M, N[j], K))) return rc;
  if ((rc = check_group(fn, K, group))) return rc;
  if (x_dtype != W4A16_DTYPE_BF16 && x_dtype != W4A16_DTYPE_F32)
    return fail(W4A16_EINVAL_ARG, "%s: unknown x_dtype %d", fn, (int)x_dtype);
  if (y_dtype != W4A16_DTYPE_BF16 && y_dtype != W4A16_DTYPE_F32)
    return fail(W4A16_EINVAL_ARG, "%s: unknown y_dtype %d", fn, (int)y_dtype);
  if (flags != 0) return fail(W4A16_EINVAL_ARG, "%s: unknown flags 0x%x", fn, (unsigned)flags);
  if (M == 0) return W4A16_OK;
  for (int j = 0; j < n; ++j)
    if (N[j] && (rc = check_ptr(y[j], "y[j]", fn))) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int y_f32 = y_dtype == W4A16_DTYPE_F32;
  if (K == 0) {
    for (int j = 0; j < n; ++j)
      if (N[j] && (rc = hip_status(w4l_fill_zero(y[j], M * N[j] * (y_f32 ? 4 : 2), st), fn))) return rc;
    return W4A16_OK;
  }
  if ((rc = check_ptr(x, "x", fn))) return rc;
  for (int j = 0; j < n; ++j)
    if (N[j] && ((rc = check_ptr(pk[j], "pk[j]", fn)) || (rc = check_ptr(sc[j], "sc[j]", fn)))) return rc;
  const uint16_t* planes = static_cast<const uint16_t*>(x);
  int nterms = 1;
  if (x_dtype == W4A16_DTYPE_F32) {
    const size_t need = x_split_bytes(M, K, x_dtype);
    if (workspace == nullptr || ws_bytes < need)
      return fail(W4A16_EWORKSPACE, "%s: f32 activations need %zu bytes of workspace, got %zu", fn, need,
                  workspace ? ws_bytes : (size_t)0);
    if ((rc = check_ptr(workspace, "workspace", fn))) return rc;
    if (w4l_group_f32x_ok(M, n, N, K, group))
      return hip_status(w4l_gemv_group(nullptr, 3, n, pk, sc, y, N, y_f32, M, K, group, st,
                                       static_cast<const float*>(x)),
                        fn);
    uint16_t* split = static_cast<uint16_t*>(workspace);
    if ((rc = hip_status(w4l_split3(static_cast<const float*>(x), split, M * K, st), fn))) return rc;
    planes = split;
    nterms = 3;
  } else if (workspace != nullptr && !aligned16(workspace)) {
    return fail(W4A16_EINVAL_PTR, "%s: workspace is not 16-byte aligned", fn);
  }
  // (a member that w4a16_linear would run as 3M rows of planes runs that way here too,
  // so every y_j stays w4a16_linear's bit for bit)
  bool rows_any = false;
  for (int j = 0; j < n && nterms == 3; ++j) {
    const size_t rows = f32_rows_bytes(M, N[j], K, x_dtype);
    rows_any = rows_any || (rows && ws_bytes >= x_split_bytes(M, K, x_dtype) + rows);
  }
  if (!rows_any && w4l_group_fused(M, n, N, K, nterms))
    return hip_status(w4l_gemv_group(planes, nterms, n, pk, sc, y, N, y_f32, M, K, group, st), fn);
  // one launch each; with bf16 x and enough workspace a member takes the split-K
  // route as w4a16_linear would (the members run in stream order, so they share
  // the workspace one after another)
  const size_t planes_bytes = x_split_bytes(M, K, x_dtype);
  for (int j = 0; j < n; ++j) {
    if (!N[j]) continue;
    const size_t sk = nterms == 1 && workspace != nullptr ? splitk_bytes(M, N[j], K, x_dtype) : 0;
    const size_t rows = nterms == 3 ? f32_rows_bytes(M, N[j], K, x_dtype) : 0;
    if (rows && ws_bytes >= planes_bytes + rows)
      rc = hip_status(f32_rows_linear(planes, pk[j], sc[j], y[j], y_f32, M, N[j], K, group,
                                      reinterpret_cast<float*>(static_cast<char*>(workspace) + planes_bytes), st),
                      fn);
    else if (sk && ws_bytes >= sk)
      rc = hip_status(w4l_splitk(planes, pk[j], sc[j], y[j], y_f32, M, N[j], K, group, st, nullptr,
                                 static_cast<float*>(workspace)),
                      fn);
    else
      rc = hip_status(w4l_linear(planes, nterms, pk[j], sc[j], y[j], y_f32, M, N[j], K, group, st), fn);
    if (rc) return rc;
  }
  return W4A16_OK;
}

namespace {
// workspace a gate/up call cannot do without: the x planes (f32 x) and, for
// shapes no fused kernel takes, f32 g and u
size_t gate_up_required(int64_t M, int64_t F, int64_t K, int32_t x_dtype) {
  if (M <= 0 || F <= 0 || K <= 0) return 0;
  const size_t split = x_split_bytes(M, K, x_dtype);
  const int nterms = x_dtype == W4A16_DTYPE_F32 ? 3 : 1;
  if (w4l_gate_up_fused(M, F, K, nterms)) return split;
  return split + 2 * round_up((size_t)4 * (size_t)M * (size_t)F, 256);  // f32 g, then u
}
// optional: the split-K partial sums over the 16 * ceil(F / 8) virtual rows
size_t gate_up_splitk(int64_t M, int64_t F, int64_t K, int32_t x_dtype) {
  if (M <= 0 || F <= 0 || K <= 0 || F > INT_MAX / 2 - 16) return 0;
  return splitk_bytes(M, 16 * ((F + 7) / 8), K, x_dtype);
}
}  // namespace

size_t w4a16_gate_up_workspace_size(int64_t M, int64_t F, int64_t K, int32_t x_dtype) {
  // (f32 x above M = 4: the unfused route's optional room for the planes run as 3M rows)
  const int nterms = x_dtype == W4A16_DTYPE_F32 ? 3 : 1;
  const size_t rows = M > 0 && F > 0 && K > 0 && !w4l_gate_up_fused(M, F, K, nterms) ? f32_rows_bytes(M, F, K, x_dtype) : 0;
  return gate_up_required(M, F, K, x_dtype) + gate_up_splitk(M, F, K, x_dtype) + rows;
}

int w4a16_gate_up_gelu(const void* x, int32_t x_dtype, const int32_t* pk_gate, const uint16_t* sc_gate,
                       const int32_t* pk_up, const uint16_t* sc_up, void* h, int32_t h_dtype, int64_t M,
                       int64_t F, int64_t K, int32_t group, int32_t flags, void* workspace, size_t ws_bytes,
                       void* stream) {
  static const char* fn = "w4a16_gate_up_gelu";
  clear_err();
  int rc = check_dims(fn, M, F, K);
  if (rc) return rc;
  // the fused launch runs over 16 * ceil(F / 8) virtual rows
  if (F > INT_MAX / 2 - 16) return fail(W4A16_EINVAL_SHAPE, "%s: F=%lld is too large", fn, (long long)F);
  if ((rc = check_group(fn, K, group))) return rc;
  if (x_dtype != W4A16_DTYPE_BF16 && x_dtype != W4A16_DTYPE_F32)
    return fail(W4A16_EINVAL_ARG, "%s: unknown x_dtype %d", fn, (int)x_dtype);
  if (h_dtype != W4A16_DTYPE_BF16 && h_dtype != W4A16_DTYPE_F32)
    return fail(W4A16_EINVAL_ARG, "%s: unknown h_dtype %d", fn, (int)h_dtype);
  if (flags & ~W4A16_GATE_UP_BF16_DOTS) return fail(W4A16_EINVAL_ARG, "%s: unknown flags 0x%x", fn, (unsigned)flags);
  if (M == 0 || F == 0) return W4A16_OK;
  if ((rc = check_ptr(h, "h", fn))) return rc;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const int h_f32 = h_dtype == W4A16_DTYPE_F32;
  // K == 0: g = u = 0 and gelu(0) * 0 = 0
  if (K == 0) return hip_status(w4l_fill_zero(h, M * F * (h_f32 ? 4 : 2), st), fn);
  if ((rc = check_ptr(x, "x", fn)) || (rc = check_ptr(pk_gate, "pk_gate", fn)) ||
      (rc = check_ptr(sc_gate, "sc_gate", fn)) || (rc = check_ptr(pk_up, "pk_up", fn)) ||
      (rc = check_ptr(sc_up, "sc_up", fn)))
    return rc;
  const size_t need = gate_up_required(M, F, K, x_dtype);
  if (need) {
    if (workspace == nullptr || ws_bytes < need)
      return fail(W4A16_EWORKSPACE, "%s: this shape needs %zu bytes of workspace, got %zu", fn, need,
                  workspace ? ws_bytes : (size_t)0);
    if ((rc = check_ptr(workspace, "workspace", fn))) return rc;
  } else if (workspace != nullptr && !aligned16(workspace)) {
    return fail(W4A16_EINVAL_PTR, "%s: workspace is not 16-byte aligned", fn);
  }

  const uint16_t* planes = static_cast<const uint16_t*>(x);
  int nterms = 1;
  char* ws = static_cast<char*>(workspace);
  W4Pair pair;
  pair.pk_up = pk_up;
  pair.sc_up = sc_up;
  pair.F = F;
  pair.bf16_dots = (flags & W4A16_GATE_UP_BF16_DOTS) ? 1 : 0;
  if (x_dtype == W4A16_DTYPE_F32) {
    if (w4l_gemv_f32x_ok(M, 16 * ((F + 7) / 8), K, group, true))
      return hip_status(w4l_gemv(nullptr, 3, pk_gate, sc_gate, h, h_f32, M, 0, K, group, st, &pair,
                                 static_cast<const float*>(x)),
                        fn);
    uint16_t* split = reinterpret_cast<uint16_t*>(ws);
    if ((rc = hip_status(w4l_split3(static_cast<const float*>(x), split, M * K, st), fn))) return rc;
    planes = split;
    nterms = 3;
    ws += x_split_bytes(M, K, x_dtype);
  }
  const size_t sk = gate_up_splitk(M, F, K, x_dtype);
  if (sk && workspace != nullptr && ws_bytes >= sk)
    return hip_status(w4l_splitk(planes, pk_gate, sc_gate, h, h_f32, M, 0, K, group, st, &pair,
                                 reinterpret_cast<float*>(ws)),
                      fn);
  if (w4l_gate_up_fused(M, F, K, nterms))
    return hip_status(w4l_gate_up(planes, nterms, pk_gate, sc_gate, pair, h, h_f32, M, K, group, st), fn);
  // unfused route: g and u in f32 through the workspace, then the activation
  const size_t gu = round_up((size_t)4 * (size_t)M * (size_t)F, 256);
  float* g = reinterpret_cast<float*>(ws);
  float* u = reinterpret_cast<float*>(ws + gu);
  // f32 x above M = 4 with the optional room after g and u: each of them as w4a16_linear
  // computes it from the planes run as 3M rows
  char* rows_ws = ws + 2 * gu;
  const size_t rows = nterms == 3 ? f32_rows_bytes(M, F, K, x_dtype) : 0;
  if (rows && ws_bytes >= (size_t)(rows_ws - static_cast<char*>(workspace)) + rows) {
    float* y3 = reinterpret_cast<float*>(rows_ws);
    if ((rc = hip_status(f32_rows_linear(planes, pk_gate, sc_gate, g, 1, M, F, K, group, y3, st), fn))) return rc;
    if ((rc = hip_status(f32_rows_linear(planes, pk_up, sc_up, u, 1, M, F, K, group, y3, st), fn))) return rc;
    return hip_status(w4l_gelu_mul(g, u, h, h_f32, pair.bf16_dots, M * F, st), fn);
  }
  if ((rc = hip_status(w4l_linear(planes, nterms, pk_gate, sc_gate, g, 1, M, F, K, group, st), fn))) return rc;
  if ((rc = hip_status(w4l_linear(planes, nterms, pk_up, sc_up, u, 1, M, F, K, group, st), fn))) return rc;
  return hip_status(w4l_gelu_mul(g, u, h, h_f32, pair.bf16_dots, M * F, st), fn);
}

size_t w4a16_lm_head_workspace_size(int64_t M, int64_t V, int64_t K, int32_t x_dtype, int32_t topk) {
  // the x planes need K > 0; the top-k candidates do not depend on K (at K == 0 the
  // logits are zeros and the top-k still runs over them)
  if (M <= 0 || V <= 0 || K < 0) return 0;
  const size_t split = x_split_bytes(M, K, x_dtype);
  if (topk <= 0) return split;
  return split + round_up((size_t)8 * (size_t)M * (size_t)w4l_topk_parts(V, topk) * (size_t)topk, 256);
}

int w4a16_lm_head(const void* x, int32_t x_dtype, const uint16_t* embed, float* logits, int64_t M, int64_t V,
                  int64_t K, float softcap, int32_t topk, float* top_values, int32_t* top_indices, void* workspace,
                  size_t ws_bytes, void* stream) {
  static const char* fn = "w4a16_lm_head";
  clear_err();
  int rc = check_dims(fn, M, V, K);
  if (rc) return rc;
  if (K % 32 != 0) return fail(W4A16_EINVAL_SHAPE, "%s: K=%lld is not a multiple of 32", fn, (long long)K);
  if (x_dtype != W4A16_DTYPE_BF16 && x_dtype != W4A16_DTYPE_F32)
    return fail(W4A16_EINVAL_ARG, "%s: unknown x_dtype %d", fn, (int)x_dtype);
  if (!(softcap >= 0.0f) || softcap > 3.0e38f)
    return fail(W4A16_EINVAL_ARG, "%s: softcap must be finite and >= 0 (0 = none)", fn);
  if (topk < 0 || topk > 64) return fail(W4A16_EINVAL_ARG, "%s: topk=%d outside 0..64", fn, (int)topk);
  if (topk > V) return fail(W4A16_EINVAL_ARG, "%s: topk=%d > V=%lld", fn, (int)topk, (long long)V);
  if (topk && ((V + 4095) / 4096) * topk > 4096)
    return fail(W4A16_EINVAL_ARG, "%s: ceil(V / 4096) * topk = %lld exceeds 4096", fn,
                (long long)(((V + 4095) / 4096) * topk));
  if (M == 0 || V == 0) return W4A16_OK;
  if ((rc = check_ptr(logits, "logits", fn))) return rc;
  if (topk && ((rc = check_ptr(top_values, "top_values", fn)) || (rc = check_ptr(top_indices, "top_indices", fn))))
    return rc;
  const size_t need = w4a16_lm_head_workspace_size(M, V, K, x_dtype, topk);
  if (need) {
    if (workspace == nullptr || ws_bytes < need)
      return fail(W4A16_EWORKSPACE, "%s: needs %zu bytes of workspace, got %zu", fn, need,
                  workspace ? ws_bytes : (size_t)0);
    if ((rc = check_ptr(workspace, "workspace", fn))) return rc;
  } else if (workspace != nullptr && !aligned16(workspace)) {
    return fail(W4A16_EINVAL_PTR, "%s: workspace is not 16-byte aligned", fn);
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (K == 0) {
    // raw = 0, softcap(0) = 0
    if ((rc = hip_status(w4l_fill_zero(logits, M * V * 4, st), fn))) return rc;
  } else {
    if ((rc = check_ptr(x, "x", fn)) || (rc = check_ptr(embed, "embed", fn))) return rc;
    const uint16_t* planes = static_cast<const uint16_t*>(x);
    int nterms = 1;
    if (x_dtype == W4A16_DTYPE_F32) {
      uint16_t* split = static_cast<uint16_t*>(workspace);
      if ((rc = hip_status(w4l_split3(static_cast<const float*>(x), split, M * K, st), fn))) return rc;
      planes = split;
      nterms = 3;
    }
    const int mc = w4l_head_rows(K, nterms);
    if (mc == 0) return fail(W4A16_EINVAL_SHAPE, "%s: K=%lld has no launch plan", fn, (long long)K);
    // chunks of mc rows: rows [m0, m0 + mc) of each plane (planes are M * K halves apart)
    for (int64_t m0 = 0; m0 < M; m0 += mc) {
      const int64_t mm = M - m0 < mc ? M - m0 : mc;
      if ((rc = hip_status(w4l_head_logits(planes + m0 * K, M * K, nterms, embed, logits + m0 * V, mm, V, K, softcap,
                                           st), fn)))
        return rc;
    }
  }
  if (topk == 0) return W4A16_OK;
  uint64_t* cand = reinterpret_cast<uint64_t*>(static_cast<char*>(workspace) + x_split_bytes(M, K, x_dtype));
  return hip_status(w4l_topk(logits, M, V, topk, cand, top_values, top_indices, st), fn);
}

}  // extern "C"
