// w4a16_head.hip -- gfx950 kernels of the lm_head: logits, softcap and top-k.
//
// Reference semantics (TheCause/gemma4-zml-probe):
//   raw    = dotPrec(prec.head, compute, last_hidden, embed_tokens, .d)   zml_runner/engine.zig:765
//            (the tied embedding, bf16 [V, K], against f32 or bf16 activations, f32 accumulate)
//   logits = softcapPrec: raw.scale(1/cap).tanh().scale(cap)              zml_runner/engine.zig:193-195,766
//   t5     = logits.topK(.{ .voc = .voc }, TOP_K, .{})                      zml_runner/gemma4_g12auto.zig:1532
//
// Logits (M <= 4): one workgroup per 16-row tile of the embedding, its waves
// splitting K.  A lane's 16-byte load is 8 consecutive bf16 of one row, which
// is exactly its part of the B operand of v_mfma_f32_16x16x32_bf16, so the
// weights go from the load straight into the MFMA.  x sits in LDS; the waves'
// partial sums meet in LDS in a fixed order; the epilogue applies the softcap
// and writes f32 logits.  Every weight load is issued before the first MFMA.
//
// Top-k: keys k = (order(value) << 32) | ~index, where order() maps f32 bits to
// an unsigned total order (-inf < ... < -0 < +0 < ... < +inf < NaN; every NaN is
// taken as the canonical +NaN, which the logits epilogue also writes).
// Larger key = larger value, and among equal values the smaller index.  Round r
// of a block selects the largest key below the key selected in round r-1, so k
// rounds give the k best in order with no per-thread sorting state.
// topk_partial_kernel reduces slices of 1024 (or 4096) logits to k candidates each;
// topk_merge_kernel reduces the candidates of a row to its k results.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include "w4a16_device.h"
#include "w4a16_launch.h"

namespace w4k {

struct HeadArgs {
  const uint16_t* x;  // NT bf16 planes of [M][K], xplane halves apart
  int64_t xplane;
  const uint16_t* e;  // [V][K] bf16
  float* logits;      // [M][V] f32
  int M, V, K;
  float cap;          // softcap; 0 = none
  // runs of 32-column steps: the first wrem waves take wbase + 1 steps, the others
  // wbase (wrem = 0 when the waves split K evenly)
  int wbase, wrem;
};

// NT: bf16 planes of x (1, or 3 for f32 x).  NST: the longest run of 32-column steps
// of a wave.  XPT: x vectors (16 B) per thread.  Waves = blockDim.x / 64; wave w covers
// steps [s0, s0 + cnt) with cnt = wbase + (w < wrem) and s0 = w * wbase + min(w, wrem),
// so the runs tile K / 32 steps in order; a run one step short loads its last step
// twice and skips the duplicate's MFMAs (a wave-uniform branch).  MR: rows of x the
// epilogue covers, 4 or 16 (the MFMA's A operand holds 16 rows either way).
template <int NT, int NST, int XPT, int MR = 4>
__global__ void __launch_bounds__(1024) head_logits_kernel(HeadArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int r = lane & 15, c = lane >> 4;

  // x loads first (every load unconditional, index clamped), then the weights;
  // LDS holds the NT planes back to back
  const int pv = (a.M * a.K) >> 3;  // 16-byte vectors per plane
  const int nvec = NT * pv;
  const uint4* xsrc = reinterpret_cast<const uint4*>(a.x);
  uint4 xv[XPT];
  int xi[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    xi[i] = min((int)threadIdx.x + i * (int)blockDim.x, nvec - 1);
    const int t = NT == 1 ? 0 : xi[i] / pv;
    xv[i] = xsrc[t * (a.xplane >> 3) + (xi[i] - t * pv)];
  }
  const int cnt = a.wbase + (wave < a.wrem ? 1 : 0);
  const int s0 = wave * a.wbase + min(wave, a.wrem);
  const int n = min((int)blockIdx.x * 16 + r, a.V - 1);
  const uint16_t* erow = a.e + (int64_t)n * a.K + s0 * 32 + 8 * c;
  uint4 wv[NST];
#pragma unroll
  for (int i = 0; i < NST; ++i) wv[i] = *reinterpret_cast<const uint4*>(erow + 32 * (i < NST - 1 ? i : min(i, cnt - 1)));

  uint4* xdst = reinterpret_cast<uint4*>(lds);
#pragma unroll
  for (int i = 0; i < XPT; ++i) xdst[xi[i]] = xv[i];
  __syncthreads();

  // A: lane (r, c) holds x[m = r][8c .. 8c+7] of the step (rows past M repeat M-1)
  const int plane = a.M * a.K;
  const uint16_t* xrow = lds + min(r, a.M - 1) * a.K + s0 * 32 + 8 * c;
  floatx4 acc[1] = {floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
  for (int i = 0; i < NST; ++i) {
    if (i < NST - 1 || i < cnt) {
      const bf16x8 b = __builtin_bit_cast(bf16x8, wv[i]);
#pragma unroll
      for (int t = 0; t < NT; ++t) mfma_acc(acc[0], *reinterpret_cast<const bf16x8*>(xrow + t * plane + 32 * i), b);
    }
  }
  mfma_drain<1>(acc);

  // D: lane (n = r, c) holds D[m = 4c + i][n]; MR = 4 keeps c == 0 only
  float* red = reinterpret_cast<float*>(lds + NT * plane);  // [waves][MR][16]
  if (MR == 16 || c == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * MR + (MR == 16 ? 4 * c : 0) + i) * 16 + r] = acc[0][i];
  }
  __syncthreads();
  for (int t = (int)threadIdx.x; t < 16 * MR; t += (int)blockDim.x) {
    const int m = t >> 4, rr = t & 15;
    const int nout = (int)blockIdx.x * 16 + rr;
    if (m < a.M && nout < a.V) {
      float v = 0.f;
      for (int w = 0; w < nwaves; ++w) v += red[(w * MR + m) * 16 + rr];
      // softcap as the reference orders it: scale by 1/cap, tanh, scale by cap
      if (a.cap > 0.f) v = tanhf(v * (1.0f / a.cap)) * a.cap;
      // NaN (a NaN weight or activation) as the canonical quiet NaN: the sign of a
      // computed NaN is not defined, and the top-k ranks NaN by its bits
      if (v != v) v = __uint_as_float(0x7fc00000u);
      a.logits[(int64_t)m * a.V + nout] = v;
    }
  }
}

// The same logits with a tile loop: each workgroup stages x once and walks
// `per` consecutive 16-row tiles, the loads of tile t+1 in flight while tile t
// computes (two register buffers, every load unconditional with the tile index
// clamped so the wait counts stay exact).  x is then read from L2 once per
// workgroup instead of once per tile: 16384 tiles re-reading a 123 KB x (16
// rows at K = 3840) is 2 GB, as much as the embedding.
template <int NT, int NST, int XPT, int MR>
__global__ void __launch_bounds__(1024) head_loop_kernel(HeadArgs a, int per) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int r = lane & 15, c = lane >> 4;
  const int ntiles = (a.V + 15) >> 4;
  const int t0 = (int)blockIdx.x * per;
  const int tend = min(t0 + per, ntiles);

  const int pv = (a.M * a.K) >> 3;
  const int nvec = NT * pv;
  const uint4* xsrc = reinterpret_cast<const uint4*>(a.x);
  uint4 xv[XPT];
  int xi[XPT];
#pragma unroll
  for (int i = 0; i < XPT; ++i) {
    xi[i] = min((int)threadIdx.x + i * (int)blockDim.x, nvec - 1);
    const int t = NT == 1 ? 0 : xi[i] / pv;
    xv[i] = xsrc[t * (a.xplane >> 3) + (xi[i] - t * pv)];
  }
  const int cnt = a.wbase + (wave < a.wrem ? 1 : 0);
  const int s0 = wave * a.wbase + min(wave, a.wrem);
  uint4 wv[2][NST];
  auto wload = [&](auto b_c, int tile) __attribute__((always_inline)) {
    constexpr int b = decltype(b_c)::value;
    const int n = min(min(tile, tend - 1) * 16 + r, a.V - 1);
    const uint16_t* erow = a.e + (int64_t)n * a.K + s0 * 32 + 8 * c;
#pragma unroll
    for (int i = 0; i < NST; ++i)
      wv[b][i] = *reinterpret_cast<const uint4*>(erow + 32 * (i < NST - 1 ? i : min(i, cnt - 1)));
  };
  wload(std::integral_constant<int, 0>{}, t0);
  uint4* xdst = reinterpret_cast<uint4*>(lds);
#pragma unroll
  for (int i = 0; i < XPT; ++i) xdst[xi[i]] = xv[i];
  __syncthreads();

  const int plane = a.M * a.K;
  const uint16_t* xrow = lds + min(r, a.M - 1) * a.K + s0 * 32 + 8 * c;
  float* red = reinterpret_cast<float*>(lds + NT * plane);  // [waves][MR][16]
  auto compute = [&](auto b_c, int tile) __attribute__((always_inline)) {
    constexpr int b = decltype(b_c)::value;
    floatx4 acc[1] = {floatx4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      if (i < NST - 1 || i < cnt) {
        const bf16x8 w = __builtin_bit_cast(bf16x8, wv[b][i]);
#pragma unroll
        for (int t = 0; t < NT; ++t) mfma_acc(acc[0], *reinterpret_cast<const bf16x8*>(xrow + t * plane + 32 * i), w);
      }
    }
    mfma_drain<1>(acc);
    if (MR == 16 || c == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) red[(wave * MR + (MR == 16 ? 4 * c : 0) + i) * 16 + r] = acc[0][i];
    }
    __syncthreads();
    for (int t = (int)threadIdx.x; t < 16 * MR; t += (int)blockDim.x) {
      const int m = t >> 4, rr = t & 15;
      const int nout = tile * 16 + rr;
      if (tile < tend && m < a.M && nout < a.V) {
        float v = 0.f;
        for (int w = 0; w < nwaves; ++w) v += red[(w * MR + m) * 16 + rr];
        if (a.cap > 0.f) v = tanhf(v * (1.0f / a.cap)) * a.cap;
        if (v != v) v = __uint_as_float(0x7fc00000u);
        a.logits[(int64_t)m * a.V + nout] = v;
      }
    }
    __syncthreads();  // red is rewritten by the next tile
  };
  for (int t = t0; t < tend; t += 2) {
    wload(std::integral_constant<int, 1>{}, t + 1);
    compute(std::integral_constant<int, 0>{}, t);
    wload(std::integral_constant<int, 0>{}, t + 2);
    compute(std::integral_constant<int, 1>{}, t + 1);
  }
}

// ---------------------------------------------------------------- top-k
__device__ __forceinline__ uint32_t order_bits(float v) {
  const uint32_t u = __float_as_uint(v);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float order_value(uint32_t o) {
  return __uint_as_float((o & 0x80000000u) ? (o & 0x7fffffffu) : ~o);
}
__device__ __forceinline__ uint64_t topk_key(float v, uint32_t index) {
  if (v != v) v = __uint_as_float(0x7fc00000u);  // every NaN ranks as +NaN, above +inf
  return ((uint64_t)order_bits(v) << 32) | (uint64_t)(~index);
}

constexpr int TOPK_THREADS = 256;
constexpr int TOPK_PER_THREAD = 16;                               // keys held per thread (merge)
constexpr int TOPK_SLICE = TOPK_THREADS * TOPK_PER_THREAD;        // 4096: candidates per merge
constexpr int TOPK_SMALL = 4;                                     // keys per thread of a 1024-logit slice

// Largest key of the block among each thread's `best` (0 = none); all threads get it.
__device__ __forceinline__ uint64_t block_max_key(uint64_t best, uint64_t* sh) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const uint32_t lo = __shfl_xor((uint32_t)best, o, 64), hi = __shfl_xor((uint32_t)(best >> 32), o, 64);
    const uint64_t other = ((uint64_t)hi << 32) | lo;
    best = other > best ? other : best;
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) sh[wave] = best;
  __syncthreads();
  uint64_t m = sh[0];
#pragma unroll
  for (int w = 1; w < TOPK_THREADS / 64; ++w) m = sh[w] > m ? sh[w] : m;
  __syncthreads();  // sh is reused by the next round
  return m;
}

// k rounds over the keys a thread holds: round r writes the r-th largest key of
// the block (0 when fewer than r + 1 keys exist) to out[r].
template <int PER>
__device__ __forceinline__ void select_rounds(const uint64_t (&keys)[PER], int k, uint64_t* out, uint64_t* sh) {
  uint64_t last = 0;
  bool first = true;
  for (int rd = 0; rd < k; ++rd) {
    uint64_t best = 0;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if ((first || keys[i] < last) && keys[i] > best) best = keys[i];
    const uint64_t win = block_max_key(best, sh);
    if (threadIdx.x == 0) out[rd] = win;
    last = win;
    first = false;
  }
}

// grid (ceil(V / (256 * PER)), M): block p of row m writes the k best keys of its
// slice of 256 * PER logits to cand[m][p][0..k).
template <int PER>
__global__ void __launch_bounds__(TOPK_THREADS) topk_partial_kernel(const float* __restrict__ logits, int V, int k,
                                                                    uint64_t* __restrict__ cand) {
  __shared__ uint64_t sh[TOPK_THREADS / 64];
  const int p = blockIdx.x, m = blockIdx.y;
  const float* row = logits + (int64_t)m * V;
  uint64_t keys[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int idx = p * (TOPK_THREADS * PER) + i * TOPK_THREADS + (int)threadIdx.x;
    keys[i] = idx < V ? topk_key(row[idx], (uint32_t)idx) : 0;
  }
  select_rounds<PER>(keys, k, cand + ((int64_t)m * gridDim.x + p) * k, sh);
}

// grid (M): merges the nparts * k candidate keys of row m into values / indices.
__global__ void __launch_bounds__(TOPK_THREADS) topk_merge_kernel(const uint64_t* __restrict__ cand, int ncand, int k,
                                                                  float* __restrict__ values,
                                                                  int32_t* __restrict__ indices) {
  __shared__ uint64_t sh[TOPK_THREADS / 64];
  __shared__ uint64_t res[64];
  const int m = blockIdx.x;
  const uint64_t* c = cand + (int64_t)m * ncand;
  uint64_t keys[TOPK_PER_THREAD];
#pragma unroll
  for (int i = 0; i < TOPK_PER_THREAD; ++i) {
    const int j = i * TOPK_THREADS + (int)threadIdx.x;
    keys[i] = j < ncand ? c[j] : 0;
  }
  select_rounds<TOPK_PER_THREAD>(keys, k, res, sh);
  __syncthreads();
  if ((int)threadIdx.x < k) {
    const uint64_t key = res[threadIdx.x];
    values[(int64_t)m * k + threadIdx.x] = order_value((uint32_t)(key >> 32));
    indices[(int64_t)m * k + threadIdx.x] = (int32_t)(~(uint32_t)key);
  }
}

}  // namespace w4k

// ---------------------------------------------------------------- launchers

// Where no even split exists (a step count with no divisor pair within 16 x 16, e.g.
// 37 steps at K = 1184): runs of at most nst = ceil(steps / 16) steps over
// ceil(steps / nst) waves (<= 16), up to 256 steps (K <= 8192).
static bool head_plan_runs(int64_t steps, int* nst, int* waves) {
  if (steps < 1 || steps > 256) return false;
  *nst = (int)((steps + 15) / 16);
  *waves = (int)((steps + *nst - 1) / *nst);
  return true;
}

// Steps per wave for K / 32 steps: the divisor <= 16 that gives the wave count
// closest to 8 (at most 16 waves); else uneven runs.
static bool head_plan(int64_t K, int* nst, int* waves) {
  if (K % 32 != 0) return false;
  const int64_t steps = K / 32;
  int best = 0;
  for (int d = 1; d <= 16; ++d) {
    if (steps % d != 0 || steps / d > 16) continue;
    if (!best || llabs(steps / d - 8) < llabs(steps / best - 8)) best = d;
  }
  if (!best) return head_plan_runs(steps, nst, waves);
  *nst = best;
  *waves = (int)(steps / best);
  return true;
}

// More rows per launch (5..16) use the MR = 16 epilogue and the plan with the
// most waves (<= 16), so that each thread stages <= 8 x vectors; x then takes
// up to 160 KB of LDS.  Uneven runs where no even split exists.
static bool head_plan16(int64_t K, int* nst, int* waves) {
  if (K % 32 != 0) return false;
  const int64_t steps = K / 32;
  for (int d = 1; d <= 16; ++d)
    if (steps % d == 0 && steps / d <= 16) {
      *nst = d;
      *waves = (int)(steps / d);
      return true;
    }
  return head_plan_runs(steps, nst, waves);
}
static bool head_fits(int64_t K, int nterms, int mc, int waves, int mr) {
  const int64_t xbytes = (int64_t)nterms * mc * K * 2;
  const int64_t xpt = ((int64_t)nterms * mc * K / 8 + 64 * waves - 1) / (64 * waves);
  return xbytes + (int64_t)waves * mr * 16 * 4 <= (mr == 4 ? 65536 : 160 * 1024) && xpt <= 8;
}

int w4l_head_rows(int64_t K, int nterms) {
  int nst, waves;
  if (head_plan16(K, &nst, &waves))
    for (int mc = 16; mc > 4; --mc)
      if (head_fits(K, nterms, mc, waves, 16)) return mc;
  if (!head_plan(K, &nst, &waves)) return 0;
  for (int mc = 4; mc >= 1; --mc)
    if (head_fits(K, nterms, mc, waves, 4)) return mc;
  return 0;
}

hipError_t w4l_head_logits(const uint16_t* x_planes, int64_t xplane, int nterms, const uint16_t* e, float* logits,
                           int64_t M, int64_t V, int64_t K, float cap, hipStream_t st) {
  // the 4-row form where it fits (M <= 4), else the 16-row form
  int nst = 0, waves = 0, mr = 0;
  if (M >= 1 && M <= 4 && head_plan(K, &nst, &waves) && head_fits(K, nterms, (int)M, waves, 4)) mr = 4;
  else if (M >= 1 && M <= 16 && head_plan16(K, &nst, &waves) && head_fits(K, nterms, (int)M, waves, 16)) mr = 16;
  if (!mr) return hipErrorInvalidValue;
  w4k::HeadArgs a{};
  a.x = x_planes;
  a.xplane = xplane;
  a.e = e;
  a.logits = logits;
  a.M = (int)M;
  a.V = (int)V;
  a.K = (int)K;
  a.cap = cap;
  a.wbase = (int)(K / 32 / waves);
  a.wrem = (int)(K / 32 % waves);
  if ((K / 32 + waves - 1) / waves != nst) return hipErrorInvalidValue;
  const int64_t nvec = (int64_t)nterms * M * K / 8;
  const int64_t per = (nvec + 64 * waves - 1) / (64 * waves);
  int xpt = 1;
  while (xpt < per) xpt *= 2;
  if (xpt > 8) return hipErrorInvalidValue;
  const size_t lds = (size_t)nterms * M * K * 2 + (size_t)waves * mr * 16 * 4;
  hipError_t err = hipSuccess;
  // 16-row form: the tile loop, ~1 workgroup per CU (2 when x fits in 64 KB)
  // each walking `per` tiles (at M = 16, V = 262144: 539 -> 415 us).  The 4-row
  // form keeps one workgroup per tile, which measured faster there (M = 1: 322
  // against 350 us).
  if (mr == 16) {
    const int64_t ntiles = (V + 15) / 16;
    const int64_t nwg = lds > 65536 ? 256 : 512;
    const int per = (int)((ntiles + nwg - 1) / nwg);
    const dim3 grid((unsigned)((ntiles + per - 1) / per)), block(64 * waves);
#define W4_HL(NT_, NST_, XPT_)                                                                       \
  do {                                                                                               \
    auto k = w4k::head_loop_kernel<NT_, NST_, XPT_, 16>;                                              \
    if (lds > 65536 &&                                                                               \
        (err = hipFuncSetAttribute(reinterpret_cast<const void*>(k),                                 \
                                   hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024)) != hipSuccess) \
      return err;                                                                                    \
    hipLaunchKernelGGL(k, grid, block, lds, st, a, per);                                             \
  } while (0)
#define W4_HL_X(NT_, NST_)                  \
  switch (xpt) {                            \
    case 1: W4_HL(NT_, NST_, 1); break;     \
    case 2: W4_HL(NT_, NST_, 2); break;     \
    case 4: W4_HL(NT_, NST_, 4); break;     \
    default: W4_HL(NT_, NST_, 8); break;    \
  }
#define W4_HL_N(NT_)                                                                 \
  switch (nst) {                                                                     \
    case 1: W4_HL_X(NT_, 1); break;   case 2: W4_HL_X(NT_, 2); break;                \
    case 3: W4_HL_X(NT_, 3); break;   case 4: W4_HL_X(NT_, 4); break;                \
    case 5: W4_HL_X(NT_, 5); break;   case 6: W4_HL_X(NT_, 6); break;                \
    case 7: W4_HL_X(NT_, 7); break;   case 8: W4_HL_X(NT_, 8); break;                \
    case 9: W4_HL_X(NT_, 9); break;   case 10: W4_HL_X(NT_, 10); break;              \
    case 11: W4_HL_X(NT_, 11); break; case 12: W4_HL_X(NT_, 12); break;              \
    case 13: W4_HL_X(NT_, 13); break; case 14: W4_HL_X(NT_, 14); break;              \
    case 15: W4_HL_X(NT_, 15); break; default: W4_HL_X(NT_, 16); break;              \
  }
    if (nterms == 1) { W4_HL_N(1) } else { W4_HL_N(3) }
#undef W4_HL_N
#undef W4_HL_X
#undef W4_HL
    return hipGetLastError();
  }
  const dim3 grid((unsigned)((V + 15) / 16)), block(64 * waves);
#define W4_HEAD(NT_, NST_, XPT_)                                                                      \
  do {                                                                                                \
    if (mr == 16) {                                                                                   \
      auto k = w4k::head_logits_kernel<NT_, NST_, XPT_, 16>;                                          \
      if (lds > 65536 &&                                                                              \
          (err = hipFuncSetAttribute(reinterpret_cast<const void*>(k),                                \
                                     hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024)) != hipSuccess) \
        return err;                                                                                   \
      hipLaunchKernelGGL(k, grid, block, lds, st, a);                                                 \
    } else {                                                                                          \
      hipLaunchKernelGGL((w4k::head_logits_kernel<NT_, NST_, XPT_>), grid, block, lds, st, a);        \
    }                                                                                                 \
  } while (0)
#define W4_HEAD_X(NT_, NST_)                  \
  switch (xpt) {                              \
    case 1: W4_HEAD(NT_, NST_, 1); break;     \
    case 2: W4_HEAD(NT_, NST_, 2); break;     \
    case 4: W4_HEAD(NT_, NST_, 4); break;     \
    default: W4_HEAD(NT_, NST_, 8); break;    \
  }
#define W4_HEAD_N(NT_)                                                                   \
  switch (nst) {                                                                         \
    case 1: W4_HEAD_X(NT_, 1); break;   case 2: W4_HEAD_X(NT_, 2); break;                \
    case 3: W4_HEAD_X(NT_, 3); break;   case 4: W4_HEAD_X(NT_, 4); break;                \
    case 5: W4_HEAD_X(NT_, 5); break;   case 6: W4_HEAD_X(NT_, 6); break;                \
    case 7: W4_HEAD_X(NT_, 7); break;   case 8: W4_HEAD_X(NT_, 8); break;                \
    case 9: W4_HEAD_X(NT_, 9); break;   case 10: W4_HEAD_X(NT_, 10); break;              \
    case 11: W4_HEAD_X(NT_, 11); break; case 12: W4_HEAD_X(NT_, 12); break;              \
    case 13: W4_HEAD_X(NT_, 13); break; case 14: W4_HEAD_X(NT_, 14); break;              \
    case 15: W4_HEAD_X(NT_, 15); break; default: W4_HEAD_X(NT_, 16); break;              \
  }
  if (nterms == 1) { W4_HEAD_N(1) } else { W4_HEAD_N(3) }
#undef W4_HEAD_N
#undef W4_HEAD_X
#undef W4_HEAD
  return hipGetLastError();
}

// Slices of 1024 logits (more blocks in flight) while their candidates fit one
// merge block, else slices of 4096.
static int64_t topk_slice(int64_t V, int k) {
  const int64_t small = w4k::TOPK_THREADS * w4k::TOPK_SMALL;
  return ((V + small - 1) / small) * k <= w4k::TOPK_SLICE ? small : w4k::TOPK_SLICE;
}

int64_t w4l_topk_parts(int64_t V, int k) {
  const int64_t s = topk_slice(V, k);
  return (V + s - 1) / s;
}

hipError_t w4l_topk(const float* logits, int64_t M, int64_t V, int k, uint64_t* cand, float* values,
                    int32_t* indices, hipStream_t st) {
  const int64_t parts = w4l_topk_parts(V, k);
  if (k < 1 || k > 64 || parts * k > w4k::TOPK_SLICE) return hipErrorInvalidValue;
  if (topk_slice(V, k) == w4k::TOPK_SLICE)
    hipLaunchKernelGGL(w4k::topk_partial_kernel<w4k::TOPK_PER_THREAD>, dim3((unsigned)parts, (unsigned)M),
                       dim3(w4k::TOPK_THREADS), 0, st, logits, (int)V, k, cand);
  else
    hipLaunchKernelGGL(w4k::topk_partial_kernel<w4k::TOPK_SMALL>, dim3((unsigned)parts, (unsigned)M),
                       dim3(w4k::TOPK_THREADS), 0, st, logits, (int)V, k, cand);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(w4k::topk_merge_kernel, dim3((unsigned)M), dim3(w4k::TOPK_THREADS), 0, st, cand,
                     (int)(parts * k), k, values, indices);
  return hipGetLastError();
}
