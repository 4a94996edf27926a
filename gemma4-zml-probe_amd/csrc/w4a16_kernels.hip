// w4a16_kernels.hip -- gfx950 kernels of the W4A16 path.
//
// Reference semantics (TheCause/gemma4-zml-probe):
//   unpackW4   zml_runner/w4.zig:33-45   (logical shift, AND 0xF, minus 8)
//   dequantW4  zml_runner/w4.zig:47-54   (bf16(q) * bf16 scale -> bf16, RNE)
//   linear     zml_runner/gemma4_w4gate.zig:288-292, zml_runner/engine.zig:530-533
//              (x.f32 . dequant(pk, sc).f32, fp32 accumulate)
//
// Linear design (every M): a wave owns 16 output rows n and a range of K.
// Each lane loads one 16-byte chunk of packed weights per step (32 nibbles =
// one scale group of one row) and expands it in registers straight into the
// B operand of v_mfma_f32_16x16x32_bf16 -- no LDS staging of weights.  The
// expansion of 8 nibbles costs 19 VALU ops (dequant8 below).  Each weight
// enters the MFMA rounded exactly as the reference rounds it, and the products
// with bf16 x are exact with fp32 accumulation.
// Activations form the A operand (16 rows of x per m-tile; rows >= M are 0).
// Waves of one workgroup split K and are reduced through LDS in fixed order.

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>

#include <atomic>
#include <type_traits>

#include "w4a16_device.h"

namespace w4k {


constexpr int KSTEP = 128;  // K covered by one wave per step (4 lane groups x 32)

// ---------------------------------------------------------------- bf16 helpers

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}

// float -> bf16 bits, round to nearest even, NaN -> 0x7FC0 (same rule as the
// oracle and torch's float->bf16 conversion).
__device__ __forceinline__ uint32_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return ((u & 0x7fffffffu) > 0x7f800000u) ? 0x7fc0u : r;
}

// ---------------------------------------------------------------- gate/up pairs
// Gemma's MLP front half (zml_runner/engine.zig:653): h = gelu(x . Wg^T) * (x . Wu^T).
// The linear kernels run it as one launch over a virtual weight of 16 * ceil(F / 8)
// rows in which every aligned 16-row tile holds 8 gate rows and the 8 matching up
// rows: virtual row v is row ((v >> 4) << 3) | (v & 7) of gate (v & 8 == 0) or of
// up (v & 8 != 0).  Each kernel's 16-row weight tile sits on 16 consecutive lanes
// (lane & 15 == v & 15), so the up value of a gate row is one lane-xor-8 away and
// the product is formed in registers before the only store.

// Row pointers of virtual row v (clamped into range; rows past the end are
// recomputed and not stored).  pair_f == 0: plain linear, row min(v, N - 1).
__device__ __forceinline__ void weight_row(const uint32_t* pk, const uint16_t* sc, const uint32_t* pk2,
                                           const uint16_t* sc2, int pair_f, int v, int N, int K,
                                           int groups_per_row, const uint32_t*& pkrow,
                                           const uint16_t*& scrow) {
  int n = min(v, N - 1);
  if (pair_f) {
    n = min(((v >> 4) << 3) | (v & 7), pair_f - 1);
    if (v & 8) {
      pk = pk2;
      sc = sc2;
    }
  }
  pkrow = pk + (int64_t)n * (K >> 3);
  scrow = sc + (int64_t)n * groups_per_row;
}

// gelu with the tanh approximation, as ZML's Tensor.gelu (gelu_pytorch_tanh):
// 0.5 g (1 + tanh(z)), z = sqrt(2/pi) (g + 0.044715 g^3), in fp32.  Evaluated
// through the identity 0.5 (1 + tanh(z)) = 1 / (1 + exp(-2 z)): no cancellation
// where tanh(z) is near -1, and branch-free (the epilogues that call it are
// fully unrolled over the accumulator registers).  exp(-2z) = 2^(-2z log2 e) on
// v_exp_f32; overflow to +inf gives -0 for very negative g, as the tanh form.
__device__ __forceinline__ float gelu_tanh(float g) {
  const float z = 0.7978845608028654f * (g + 0.044715f * g * g * g);
  const float e = __builtin_amdgcn_exp2f(-2.8853900817779268f * z);  // -2 log2(e) z
  return g * __builtin_amdgcn_rcpf(1.0f + e);  // v_rcp_f32: 1 ulp
}

// Compile-time loop: f(integral_constant<int, I>) for I in [B, E).  Expands
// fully whatever the unroller's thresholds, so register arrays indexed by I
// stay in registers.
template <int B, int E, class Fn>
__device__ __forceinline__ void static_for(Fn&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// h = gelu(g) * u; with bf16_dots, g and u are first rounded to bf16 (the dot
// outputs of dotPrec with fam = bf16, engine.zig:531).
__device__ __forceinline__ void store_gelu_mul(void* y, int y_f32, int bf16_dots, int64_t idx, float g,
                                               float u) {
  if (bf16_dots) {
    g = bf16_bits_to_f32(f32_to_bf16_rne(g));
    u = bf16_bits_to_f32(f32_to_bf16_rne(u));
  }
  const float h = gelu_tanh(g) * u;
  if (y_f32) reinterpret_cast<float*>(y)[idx] = h;
  else reinterpret_cast<uint16_t*>(y)[idx] = (uint16_t)f32_to_bf16_rne(h);
}

// Value of lane (lane ^ 8): DPP row_ror:8 within each row of 16 lanes.  Every
// lane of the row must be active.
__device__ __forceinline__ float lane_xor8(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xf, 0xf, false));
}

// ---------------------------------------------------------------- in-register dequant
// 8 nibbles of one packed word -> 8 bf16 weights RNE(q * s) in column order,
// laid out as one MFMA B operand (4 VGPRs, pairs (w0,w1) .. (w6,w7)).
//   p_j = (w >> 4j) & 0x000F000F | 0x43004300  bf16 pair (128 + n_j, 128 + n_{j+4})
//   d   = v_dot2_f32_bf16(p_j, (s, 0) | (0, s), -136 s) = (n - 8) * s, exact in fp32
//   r   = v_cvt_pk_bf16_f32(d_a, d_b)           RNE to bf16: dequantW4's rounding
// 19 VALU instructions.  The sequence is one asm block because the compiler's
// hazard recognizer cannot see inside inline asm, and gfx950 does not
// interlock a DOT result read by another VALU instruction (3 wait states):
// all dots are issued before the first conversion, so every conversion reads
// a dot result at least 3 instructions old.  The VALU -> MFMA wait states are
// issued by mfma_acc.  Twelve temporaries: the shifts land in the pair
// registers and each conversion overwrites its first dot result, which keeps
// the decode kernels at <= 80 VGPRs (six waves per SIMD).
// kM = 0x000F000F and kO = 0x43004300 come in VGPRs (VOP3 takes no literals).
__device__ __forceinline__ bf16x8 dequant8(uint32_t w, uint32_t slo, uint32_t shi, float c,
                                           uint32_t kM, uint32_t kO) {
  uint32_t p0, p1, p2, p3, d0, d1, d2, d3, d4, d5, d6, d7;
  // v_bitop3_b32 with truth table 0xEA computes (a & b) | c.
  asm("v_bitop3_b32 %[p0], %[w], %[km], %[ko] bitop3:0xea\n\t"
      "v_lshrrev_b32 %[p1], 4, %[w]\n\t"
      "v_lshrrev_b32 %[p2], 8, %[w]\n\t"
      "v_lshrrev_b32 %[p3], 12, %[w]\n\t"
      "v_bitop3_b32 %[p1], %[p1], %[km], %[ko] bitop3:0xea\n\t"
      "v_bitop3_b32 %[p2], %[p2], %[km], %[ko] bitop3:0xea\n\t"
      "v_bitop3_b32 %[p3], %[p3], %[km], %[ko] bitop3:0xea\n\t"
      "v_dot2_f32_bf16 %[d0], %[p0], %[slo], %[c]\n\t"
      "v_dot2_f32_bf16 %[d1], %[p1], %[slo], %[c]\n\t"
      "v_dot2_f32_bf16 %[d2], %[p2], %[slo], %[c]\n\t"
      "v_dot2_f32_bf16 %[d3], %[p3], %[slo], %[c]\n\t"
      "v_dot2_f32_bf16 %[d4], %[p0], %[shi], %[c]\n\t"
      "v_dot2_f32_bf16 %[d5], %[p1], %[shi], %[c]\n\t"
      "v_dot2_f32_bf16 %[d6], %[p2], %[shi], %[c]\n\t"
      "v_dot2_f32_bf16 %[d7], %[p3], %[shi], %[c]\n\t"
      "v_cvt_pk_bf16_f32 %[d0], %[d0], %[d1]\n\t"
      "v_cvt_pk_bf16_f32 %[d2], %[d2], %[d3]\n\t"
      "v_cvt_pk_bf16_f32 %[d4], %[d4], %[d5]\n\t"
      "v_cvt_pk_bf16_f32 %[d6], %[d6], %[d7]"
      : [p0] "=&v"(p0), [p1] "=&v"(p1), [p2] "=&v"(p2), [p3] "=&v"(p3),
        [d0] "=&v"(d0), [d1] "=&v"(d1), [d2] "=&v"(d2), [d3] "=&v"(d3),
        [d4] "=&v"(d4), [d5] "=&v"(d5), [d6] "=&v"(d6), [d7] "=&v"(d7)
      : [w] "v"(w), [slo] "v"(slo), [shi] "v"(shi), [c] "v"(c), [km] "v"(kM), [ko] "v"(kO));
  u32x4 r;
  r[0] = d0;
  r[1] = d2;
  r[2] = d4;
  r[3] = d6;
  return __builtin_bit_cast(bf16x8, r);
}

// 8 nibbles -> the same 8 bf16 weights RNE(q * s), written in C so that the
// compiler schedules it and tracks every hazard (used by the decode GEMV).
// Nibbles become f16 values placed by one v_bitop3 per pair:
//   h0 = (w & 0x000F000F) | 0x64006400 = (1024 + n0, 1024 + n4)
//   h1 = (w & 0x00F000F0) | 0x64006400 = (1024 + 16 n1, 1024 + 16 n5)
//   h2, h3: the same on w >> 8 (n2, n6 and n3, n7).
// v_fma_mix_f32 widens the selected f16 half exactly and computes
//   (1024 + n) s - 1032 s = (n - 8) s   or   (1024 + 16 n) (s / 16) - 72 s = (n - 8) s
// in one rounding of an exact result (both are integer multiples of s with at most
// 12 significant bits), and v_cvt_pk_bf16_f32 rounds pairs to bf16 (RNE):
// dequantW4's rounding.  Exact for 2^-126 <= |s| < 2^117 (1039 |s| stays finite;
// below 2^-122, s / 16 is an fp32 denormal, which the kernels keep) and s = +-0;
// 17 VALU instructions per 8 weights, 12 of them at half rate, against 19 (12 at
// half rate) for dequant8.
struct MixScale {
  float s, c1, s16, c2;  // s, -1032 s, s / 16, -72 s
};
__device__ __forceinline__ MixScale mix_scale(uint32_t sbits) {
  const float s = __uint_as_float(sbits << 16);
  return MixScale{s, -1032.0f * s, s * 0.0625f, -72.0f * s};
}
// (a & m) | o as one full-rate v_bitop3_b32 (the compiler would emit an and + an or
// with literals, or the half-rate v_and_or_b32); m and o come in VGPRs.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
  uint32_t r;
  asm("v_bitop3_b32 %0, %1, %2, %3 bitop3:0xea" : "=v"(r) : "v"(a), "v"(m), "v"(o));
  return r;
}
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  typedef float f2 __attribute__((ext_vector_type(2)));
  typedef __bf16 b2 __attribute__((ext_vector_type(2)));
  const f2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, b2));
}
struct MixMasks {
  uint32_t m0, m1, o;  // 0x000F000F, 0x00F000F0, 0x64006400, held in VGPRs
};
__device__ __forceinline__ MixMasks mix_masks() {
  MixMasks k{0x000F000Fu, 0x00F000F0u, 0x64006400u};
  asm volatile("" : "+v"(k.m0), "+v"(k.m1), "+v"(k.o));
  return k;
}
__device__ __forceinline__ bf16x8 dequant8_mix(uint32_t w, const MixScale& S, const MixMasks& k) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const uint32_t w8 = w >> 8;
  const h2 h0 = __builtin_bit_cast(h2, and_or(w, k.m0, k.o));
  const h2 h1 = __builtin_bit_cast(h2, and_or(w, k.m1, k.o));
  const h2 h2v = __builtin_bit_cast(h2, and_or(w8, k.m0, k.o));
  const h2 h3 = __builtin_bit_cast(h2, and_or(w8, k.m1, k.o));
  const float q0 = __builtin_fmaf((float)h0.x, S.s, S.c1), q4 = __builtin_fmaf((float)h0.y, S.s, S.c1);
  const float q1 = __builtin_fmaf((float)h1.x, S.s16, S.c2), q5 = __builtin_fmaf((float)h1.y, S.s16, S.c2);
  const float q2 = __builtin_fmaf((float)h2v.x, S.s, S.c1), q6 = __builtin_fmaf((float)h2v.y, S.s, S.c1);
  const float q3 = __builtin_fmaf((float)h3.x, S.s16, S.c2), q7 = __builtin_fmaf((float)h3.y, S.s16, S.c2);
  u32x4 r;
  r[0] = pack_bf16x2(q0, q1);
  r[1] = pack_bf16x2(q2, q3);
  r[2] = pack_bf16x2(q4, q5);
  r[3] = pack_bf16x2(q6, q7);
  return __builtin_bit_cast(bf16x8, r);
}

// ================================================================ unpack, dequant
// Flat over packed words: word i holds weights 8i .. 8i+7 of the [N, K] matrix (rows
// are K/8 whole words).  One word per lane per unit, U units per thread 256 words
// apart, so every load instruction reads 256 consecutive words and every store writes
// one contiguous block (2 KiB of int8 q, 4 KiB of bf16 w per 256 lanes); U = 4 keeps
// four words in flight per lane on large matrices.  (The first form, one thread per
// 32-column chunk with 16-byte stores 64 bytes apart and a 64-bit division per chunk,
// ran dequant at 3.4-3.7 TB/s on 12B-sized matrices; this form at 5.8-6.1.)
template <int U>
__global__ void __launch_bounds__(256) unpack_kernel(const uint32_t* __restrict__ pk,
                                                     int8_t* __restrict__ q, int64_t nwords) {
  const int64_t base = (int64_t)blockIdx.x * (256 * U) + threadIdx.x;
  uint32_t wd[U];
#pragma unroll
  for (int u = 0; u < U; ++u) wd[u] = pk[min(base + 256 * u, nwords - 1)];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + 256 * u;
    // n - 8 is the nibble n ^ 8 read as a signed 4-bit number
    const uint32_t t = wd[u] ^ 0x88888888u;
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lo |= ((uint32_t)((int32_t)(t << (28 - 4 * j)) >> 28) & 0xFFu) << (8 * j);
      hi |= ((uint32_t)((int32_t)(t << (12 - 4 * j)) >> 28) & 0xFFu) << (8 * j);
    }
    if (i < nwords) reinterpret_cast<uint2*>(q)[i] = make_uint2(lo, hi);
  }
}

// Bit-exact RNE_bf16(float(q) * s).  Word i's scale is sc[i / (group / 8)] for every
// row: K % group == 0 starts each row on a group boundary, so the flat word index
// divided by the words per group is the flat scale index (a shift when group / 8 is a
// power of two, shift < 0 otherwise).
template <int U>
__global__ void __launch_bounds__(256) dequant_kernel(const uint32_t* __restrict__ pk,
                                                      const uint16_t* __restrict__ sc,
                                                      uint16_t* __restrict__ w, int64_t nwords,
                                                      int64_t words_per_group, int shift) {
  const int64_t base = (int64_t)blockIdx.x * (256 * U) + threadIdx.x;
  uint32_t wd[U];
  float s[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = min(base + 256 * u, nwords - 1);
    wd[u] = pk[i];
    s[u] = bf16_bits_to_f32(sc[shift >= 0 ? (i >> shift) : (i / words_per_group)]);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t i = base + 256 * u;
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float a = (float)((int)((wd[u] >> (8 * j)) & 0xFu) - 8) * s[u];
      const float b = (float)((int)((wd[u] >> (8 * j + 4)) & 0xFu) - 8) * s[u];
      o[j] = f32_to_bf16_rne(a) | (f32_to_bf16_rne(b) << 16);
    }
    if (i < nwords) reinterpret_cast<uint4*>(w)[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ================================================================ f32 x split
// x f32 [M, K] -> three bf16 planes [3][M][K] with x = t0 + t1 + t2 exactly:
// t0, t1 take the top 8 significand bits of x and of the remainder (bit
// truncation), t2 the remaining <= 8 bits.  A non-finite x goes whole into t0
// (+-inf, or the quiet NaN 0x7FC0) with t1 = t2 = +0, so the dot sees exactly
// the f32 dot's +-inf * w and NaN * w (inf - inf in the split would make NaN).
// The three bf16 terms of an f32 value u (bits), low 16 bits of h0, h1, h2: h0 its top
// half (truncation), h1 the top half of the remainder, h2 the rest rounded to bf16 (RNE);
// h0 + h1 + h2 = v exactly for finite v.  A non-finite v keeps its top half (a NaN as
// the canonical quiet NaN 0x7fc0) and two zero terms.
__device__ __forceinline__ void split3_terms(uint32_t u, uint32_t& h0, uint32_t& h1, uint32_t& h2) {
  const float v = __uint_as_float(u);
  const float t0 = __uint_as_float(u & 0xffff0000u);
  const float r1 = v - t0;
  const float t1 = __uint_as_float(__float_as_uint(r1) & 0xffff0000u);
  const float r2 = r1 - t1;
  const bool nf = (u & 0x7f800000u) == 0x7f800000u;
  h0 = nf && (u & 0x007fffffu) ? 0x7fc0u : (u >> 16);
  h1 = nf ? 0u : (__float_as_uint(t1) >> 16);
  h2 = nf ? 0u : f32_to_bf16_rne(r2);
}

__global__ void __launch_bounds__(256) split3_kernel(const float* __restrict__ x,
                                                     uint16_t* __restrict__ out, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    uint32_t h0, h1, h2;
    split3_terms(__float_as_uint(x[i]), h0, h1, h2);
    out[i] = (uint16_t)h0;
    out[n + i] = (uint16_t)h1;
    out[2 * n + i] = (uint16_t)h2;
  }
}

// ================================================================ linear
struct LinearArgs {
  const uint16_t* x;   // [NT][M][K] bf16 planes
  const uint32_t* pk;  // [N][K/8]
  const uint16_t* sc;  // [N][K/group]
  void* y;             // [M][N] bf16 or f32
  int M, N, K;
  int group_chunks;    // group / 32
  int groups_per_row;  // K / group
  int y_f32;
  int64_t x_plane;     // M * K
};

// MT: 16-row m-tiles per workgroup (1..4).  NT: number of bf16 x planes (1 or 3).
// MAXT: launch bound (threads); smaller for the register-heavier variants.
template <int MT, int NT, int MAXT>
__global__ void __launch_bounds__(MAXT) linear_kernel(LinearArgs a) {
  extern __shared__ float red[];  // [waves][MT][4][64] partials
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int nwaves = blockDim.x >> 6;
  const int r = lane & 15;  // row within the 16-row tile (n for B, m for A)
  const int c = lane >> 4;  // lane group: which 32-column chunk of the step
  const int n0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * (16 * MT);

  const int steps = (a.K + KSTEP - 1) / KSTEP;
  const int s_begin = (int)(((int64_t)steps * wave) / nwaves);
  const int s_end = (int)(((int64_t)steps * (wave + 1)) / nwaves);

  const int nrow = min(n0 + r, a.N - 1);  // clamped: loads stay in bounds
  const int kwords = a.K >> 3;
  const uint32_t* pkrow = a.pk + (int64_t)nrow * kwords;
  const uint16_t* scrow = a.sc + (int64_t)nrow * a.groups_per_row;
  const int ngroups32 = a.K >> 5;

  uint32_t kM = 0x000F000Fu, kO = 0x43004300u;
  asm volatile("" : "+v"(kM), "+v"(kO));

  floatx4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int s = s_begin; s < s_end; ++s) {
    const int g = s * 4 + c;  // 32-column chunk index of this lane
    const bool valid = g < ngroups32;
    uint4 wv = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
    uint32_t sb = 0;
    if (valid) {
      wv = *reinterpret_cast<const uint4*>(pkrow + g * 4);
      sb = scrow[g / a.group_chunks];
    }
    const float cneg = -136.0f * bf16_bits_to_f32(sb);
    const uint32_t wj[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // A operands: lane (r, c) holds x[m][32g + 8j .. +7] for m = m0 + 16 mt + r
      bf16x8 xa[NT][MT];
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          const int m = m0 + 16 * mt + r;
          uint4 v = make_uint4(0, 0, 0, 0);
          if (valid && m < a.M)
            v = *reinterpret_cast<const uint4*>(a.x + t * a.x_plane + (int64_t)m * a.K + g * 32 + 8 * j);
          xa[t][mt] = __builtin_bit_cast(bf16x8, v);
        }
      const bf16x8 b = dequant8(wj[j], sb, sb << 16, cneg, kM, kO);
#pragma unroll
      for (int t = 0; t < NT; ++t)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          mfma_acc(acc[mt], xa[t][mt], b);
    }
    mfma_drain<MT>(acc);
  }

  // D layout: lane (n = lane & 15, c = lane >> 4) holds D[m = 4c + i][n], i = 0..3.
  if (nwaves > 1) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) red[((wave * MT + mt) * 4 + i) * 64 + lane] = acc[mt][i];
    __syncthreads();
    const int per_wave = MT * 4 * 64;
    for (int e = threadIdx.x; e < per_wave; e += blockDim.x) {
      float v = 0.f;
      for (int w = 0; w < nwaves; ++w) v += red[w * per_wave + e];
      const int l = e & 63, i = (e >> 6) & 3, mt = e >> 8;
      const int m = m0 + 16 * mt + 4 * (l >> 4) + i;
      const int n = n0 + (l & 15);
      if (m < a.M && n < a.N) {
        if (a.y_f32) reinterpret_cast<float*>(a.y)[(int64_t)m * a.N + n] = v;
        else reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.N + n] = (uint16_t)f32_to_bf16_rne(v);
      }
    }
  } else {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * mt + 4 * c + i;
        const int n = n0 + r;
        if (m < a.M && n < a.N) {
          if (a.y_f32) reinterpret_cast<float*>(a.y)[(int64_t)m * a.N + n] = acc[mt][i];
          else reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.N + n] = (uint16_t)f32_to_bf16_rne(acc[mt][i]);
        }
      }
  }
}

// ================================================================ GEMV (decode, M <= 4)
// One workgroup per 16 output rows; its W waves split K.  A "step" covers
// 256 columns: lane (r = row, c = lane group) loads VPL = 2 consecutive
// 16-byte packed vectors of its row (64 nibbles = 2 scale groups) and the two
// bf16 scales as one 32-bit word, so each row is read 128 contiguous bytes at
// a time.  A wave issues the loads of all its steps (<= SPW) before anything
// else; while they arrive the workgroup copies x (M rows, whole K, <= 64 KiB
// minus the reduction area) into LDS.  A operands are then read from LDS with
// every lane of a 16-lane group reading the same row (rows >= M duplicate row
// M-1 and are discarded), so no lane needs a zero fill.  The waves' partial
// tiles are summed in LDS in wave order (deterministic).
constexpr int VPL = 2;                  // 16-byte vectors per lane per step
constexpr int GSTEP = 128 * VPL;        // columns per step
constexpr int SPW = 4;                  // steps a wave keeps in flight

struct GemvArgs {
  const uint16_t* x;  // [NT][M][K] bf16 planes
  const uint32_t* pk;
  const uint16_t* sc;
  void* y;
  int M, N, K;
  int group_chunks;    // group / 32
  int groups_per_row;  // K / group
  int y_f32;
  int steps;           // ceil(K / GSTEP)
  // gemv_fast_kernel: steps of GSTEP columns per wave within one K segment; the
  // first wrem waves of a workgroup take wbase + 1 steps, the others wbase
  int wbase, wrem;
  // gemv_fast_kernel: tiles of the launch, and the grid size: workgroup b takes tiles b,
  // b + gstride, ... (kept next to wbase and wrem, so that all of them arrive in the
  // kernel's first batch of argument loads)
  int ntiles, gstride, waves;  // (waves = blockDim.x / 64)
  // gate/up pair mode (gemv_fast_kernel only): pk/sc are gate, pk2/sc2 up,
  // pair_f = F real rows each (0 = plain linear), N = 16 * ceil(F / 8).
  const uint32_t* pk2;
  const uint16_t* sc2;
  int pair_f;
  int bf16_dots;
  // weight group (gemv_fast_kernel, TPW = 1): nmat > 1 linears that share x;
  // matrix j owns tiles [tile0[j], tile0[j + 1]) of the grid.
  int nmat;
  // (host only) x holds f32 x [M][K], staged by the XF instances
  int xf;
  const uint32_t* gpk[4];
  const uint16_t* gsc[4];
  void* gy[4];
  int gN[4];
  int tile0[4];
};

// Matrix of a weight group that owns tile t (uniform across the workgroup);
// selects rather than indexing, so the arguments stay in scalar registers.
struct GroupSel {
  const uint32_t* pk;
  const uint16_t* sc;
  void* y;
  int N;
  int tile0;
};
// Branch-free, so that every kernel argument arrives in one batch of scalar loads
// (a branch here puts the group's arguments behind a second round trip, which
// delays the first weight load of every wave): every candidate is read and pinned
// in SGPRs first, then the tile's matrix is picked with scalar selects.
__device__ __forceinline__ GroupSel group_select(const GemvArgs& a, int t) {
  uint64_t p[4], q[4], y[4];
  int n[4], t0[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    p[k] = reinterpret_cast<uint64_t>(a.gpk[k]);
    q[k] = reinterpret_cast<uint64_t>(a.gsc[k]);
    y[k] = reinterpret_cast<uint64_t>(a.gy[k]);
    n[k] = a.gN[k];
    t0[k] = a.tile0[k];
    asm volatile("" : "+s"(p[k]), "+s"(q[k]), "+s"(y[k]), "+s"(n[k]), "+s"(t0[k]));
  }
  uint64_t p1 = reinterpret_cast<uint64_t>(a.pk), q1 = reinterpret_cast<uint64_t>(a.sc),
           y1 = reinterpret_cast<uint64_t>(a.y);
  int n1 = a.N, nm = a.nmat;
  asm volatile("" : "+s"(p1), "+s"(q1), "+s"(y1), "+s"(n1), "+s"(nm));
  const int j = (nm > 1 && t >= t0[1]) + (nm > 2 && t >= t0[2]) + (nm > 3 && t >= t0[3]);
  const bool grp = nm > 1;
  GroupSel g;
  g.pk = reinterpret_cast<const uint32_t*>(grp ? (j == 0 ? p[0] : j == 1 ? p[1] : j == 2 ? p[2] : p[3]) : p1);
  g.sc = reinterpret_cast<const uint16_t*>(grp ? (j == 0 ? q[0] : j == 1 ? q[1] : j == 2 ? q[2] : q[3]) : q1);
  g.y = reinterpret_cast<void*>(grp ? (j == 0 ? y[0] : j == 1 ? y[1] : j == 2 ? y[2] : y[3]) : y1);
  g.N = grp ? (j == 0 ? n[0] : j == 1 ? n[1] : j == 2 ? n[2] : n[3]) : n1;
  g.tile0 = grp ? (j == 0 ? t0[0] : j == 1 ? t0[1] : j == 2 ? t0[2] : t0[3]) : 0;
  return g;
}

// NT: bf16 x planes (1, or 3 for f32 x).  KFULL: K % GSTEP == 0 (no partial
// step).  G32: group == 32 (scale index == 32-column chunk index).
template <int NT, bool KFULL, bool G32>
__global__ void __launch_bounds__(1024) gemv_kernel(GemvArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int lane = threadIdx.x & 63;
  // wave-uniform (SGPR) so that the step guards below are scalar branches
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = blockDim.x >> 6;
  const int r = lane & 15;
  const int c = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int ng32 = a.K >> 5;
  const int s_begin = (a.steps * wave) / nwaves;
  const int s_end = (a.steps * (wave + 1)) / nwaves;

  const int nrow = min(n0 + r, a.N - 1);
  const uint32_t* pkrow = a.pk + (int64_t)nrow * (a.K >> 3);
  const uint16_t* scrow = a.sc + (int64_t)nrow * a.groups_per_row;

  uint4 wv[SPW][VPL];
  uint32_t sv[SPW];  // two bf16 scales (low half: first vector's group)
  int ch = s_begin;
  int cnt = min(SPW, s_end - ch);
  // chunk index (32 columns) of vector v of step s for this lane
  auto chunk = [&](int s, int v) { return (s * 4 + c) * VPL + v; };
  auto load_steps = [&](int base, int n) {
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      if (i < n) {
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          int g = chunk(base + i, v);
          if (!KFULL) g = min(g, ng32 - 1);
          wv[i][v] = *reinterpret_cast<const uint4*>(pkrow + 4 * g);
        }
        if (G32 && KFULL) {
          sv[i] = *reinterpret_cast<const uint32_t*>(scrow + chunk(base + i, 0));
        } else {
          int g0 = chunk(base + i, 0), g1 = chunk(base + i, 1);
          if (!KFULL) { g0 = min(g0, ng32 - 1); g1 = min(g1, ng32 - 1); }
          const uint32_t s0 = scrow[G32 ? g0 : g0 / a.group_chunks];
          const uint32_t s1 = scrow[G32 ? g1 : g1 / a.group_chunks];
          sv[i] = s0 | (s1 << 16);
        }
      }
    }
  };
  load_steps(ch, cnt);

  // stage x (all planes, rows, columns) into LDS
  {
    const int nvec = (NT * a.M * a.K) >> 3;  // 16-byte vectors
    const uint4* src = reinterpret_cast<const uint4*>(a.x);
    uint4* dst = reinterpret_cast<uint4*>(lds);
    for (int v = threadIdx.x; v < nvec; v += blockDim.x) dst[v] = src[v];
  }
  __syncthreads();

  uint32_t kM = 0x000F000Fu, kO = 0x43004300u;
  asm volatile("" : "+v"(kM), "+v"(kO));
  floatx4 acc[1] = {floatx4{0.f, 0.f, 0.f, 0.f}};
  const int mrow = min(r, a.M - 1);
  const int plane = a.M * a.K;
  const uint16_t* xrow = lds + mrow * a.K;

  while (cnt > 0) {
#pragma unroll
    for (int i = 0; i < SPW; ++i) {
      if (i < cnt) {
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          int g = chunk(ch + i, v);
          uint32_t slo = v == 0 ? (sv[i] & 0xffffu) : (sv[i] >> 16);
          if (!KFULL) {
            if (g >= ng32) slo = 0;  // past K: weights become exact zeros
            g = min(g, ng32 - 1);
          }
          const uint32_t shi = slo << 16;
          const float cneg = -136.0f * __uint_as_float(shi);
          const uint16_t* xr = xrow + 32 * g;
          const uint32_t wj[4] = {wv[i][v].x, wv[i][v].y, wv[i][v].z, wv[i][v].w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bf16x8 bb = dequant8(wj[j], slo, shi, cneg, kM, kO);
#pragma unroll
            for (int t = 0; t < NT; ++t)
              mfma_acc(acc[0], *reinterpret_cast<const bf16x8*>(xr + t * plane + 8 * j), bb);
          }
        }
      }
    }
    mfma_drain<1>(acc);
    ch += SPW;
    cnt = min(SPW, s_end - ch);
    if (cnt > 0) load_steps(ch, cnt);
  }

  // rows m < M <= 4 live in lanes 0..15 (c == 0), acc[m]
  float* red = reinterpret_cast<float*>(lds + NT * plane);
  if (c == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * 4 + i) * 16 + r] = acc[0][i];
  }
  __syncthreads();
  if ((int)threadIdx.x < 16 * a.M) {
    const int m = threadIdx.x >> 4, rr = threadIdx.x & 15;
    float v = 0.f;
    for (int w = 0; w < nwaves; ++w) v += red[(w * 4 + m) * 16 + rr];
    const int n = n0 + rr;
    if (n < a.N) {
      if (a.y_f32) reinterpret_cast<float*>(a.y)[(int64_t)m * a.N + n] = v;
      else reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.N + n] = (uint16_t)f32_to_bf16_rne(v);
    }
  }
}

// ---------------------------------------------------------------- GEMV, straight-line variant
// Same lane layout as gemv_kernel, for K a multiple of GSTEP * S.  A workgroup covers
// one tile of R = 16 / S rows of W; its waves split each of the S K segments of the
// tile's rows into runs of steps (wbase + 1 steps for the first wrem waves, wbase for
// the others; NST = the longer run, a compile-time bound).  LOOP: a grid of at most
// one round of workgroups walks the tiles (b, b + gstride, ...), see below.
//
// K segments (S = 2, M = 1 only): the MFMA's 16 B-operand columns are R rows x S
// segments of K -- lane r holds row r % R in segment r / R -- and its A operand row r
// (r < S) holds x of segment r, so D[s][n] for n in segment s is that segment's partial
// sum; the S partials of a row meet in registers (DPP) before the cross-wave sum.  A
// tile then spans half as many rows, so a shape with few rows of W gets twice the
// workgroups and waves.
//
// Every load is issued up front, unconditionally (indices clamped) and in a fixed
// order held by scheduling barriers: this thread's x vectors, then the scales of
// the wave's NST steps, then its weights step by step.  vmcnt is an in-order
// per-wave counter, so each step then waits only for its own loads, and x is
// written to LDS as soon as it lands while the weights are still in flight.  A wave
// with a run one step shorter than NST loads its last step twice and skips the
// duplicate's compute (a wave-uniform branch).  Each lane reads a step's weights and
// scales at constant offsets from one row pointer (no per-load address arithmetic,
// so no address registers crowd out the data).
// XW: each wave stages only its own K ranges of x (NT planes x M rows x S segments x
// NST * 256 columns, XPT vectors per lane) at their places in the [NT][M][K] LDS
// image and reads nothing else, so it starts computing without waiting for the other
// waves; otherwise the workgroup stages all of x (XPT vectors per thread) behind one
// barrier.
// Weights are expanded with dequant8_mix.  Tiles past N (odd tile counts) are
// not written.
// MR: rows of x the epilogue covers, 4 (M <= 4) or 16 (M <= 16; the MFMA's A
// operand holds 16 rows of x either way, rows past M repeat row M-1).
// PLAIN: one matrix, no gate/up pair (a.pk, a.sc, a.y, a.N only): the kernel then
// reads none of the group or pair arguments, whose selection the compiler turns into
// branches with late scalar loads that delay every wave's first weight load.
// S = 2 needs NT = 1, MR = 4, XW, M = 1 and no gate/up pair (checked on the host): a
// single weight (PLAIN) or a weight group, whose tiles are then 8-row tiles too.
template <int NT, int NST, int XPT, bool G32, int MR, bool XW, bool PLAIN = false, int S = 1, bool LOOP = false,
          bool XF = false>
__global__ void __launch_bounds__(1024) gemv_fast_kernel(GemvArgs a) {
  static_assert(S == 1 || (S == 2 && NT == 1 && MR == 4 && XW), "K segments: the bf16 M = 1 form only");
  // Wave priority: high until every load of the wave is issued (a wave that has just
  // started then gets its requests out ahead of the dequant of the waves already
  // computing), lowest while it computes, raised again for the epilogue so that a
  // finished workgroup frees its slots for the next one (12B gate/up: 1-5 % faster).
  __builtin_amdgcn_s_setprio(3);
  constexpr int R = 16 / S;  // W rows per tile
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int nwaves = a.waves;  // blockDim.x / 64, from the first batch of argument loads
  const int r = lane & 15;
  const int c = lane >> 4;
  const int seg = r / R, rr = r % R;  // B column r: row rr of the tile, K segment seg
  // this wave's run of steps in every segment: [s0, s0 + cnt), cnt = NST or NST - 1
  const int cnt = a.wbase + (wave < a.wrem ? 1 : 0);
  const int s0 = wave * a.wbase + min(wave, a.wrem);
  const int K = a.K;
  const int KS = (int)((unsigned)K / S);  // columns per segment
  const int plane = a.M * K;
  // LOOP (one weight or a gate/up pair, group-32 scales, bf16 x, the 4-row epilogue):
  // workgroup b takes tiles b, b + gstride, ... of a grid the host caps at one round; the
  // next tile's loads go out before the current tile's epilogue and x is staged once.
  // Otherwise one tile per workgroup.
  static_assert(!LOOP || (G32 && S == 1 && MR == 4 && XW), "tile loop: the 4-row group-32 form");
  // XF: a.x holds f32 x [M][K] (not bf16 planes); each wave loads its share of it and writes
  // the three bf16 terms of every value (as split3_kernel computes them) into the NT = 3
  // planes of its LDS image, so no separate split launch precedes the GEMV.  XPT then counts
  // 8-column vectors of f32 x per lane (two 16-byte loads each).
  static_assert(!XF || (NT == 3 && XW && S == 1), "f32 x staging: the per-wave three-plane form");
  const int T = a.ntiles;  // (gridDim.x is a.gstride)

  // 1. x loads, first (they need nothing but x's address; x is the same for every tile)
  typedef __attribute__((address_space(1))) const u32x4 g_u4;
  typedef __attribute__((address_space(1))) const uint32_t g_u32;
  const u32x4* xsrc = reinterpret_cast<const u32x4*>(a.x);
  int xi[XPT];
  if (XW) {
    // vector v of the wave's share: (plane t, row m) = v / (S * NST * 32), then segment
    // (v / (NST * 32)) % S, then column vector s0 * 32 + u of that segment, u = v % (NST * 32)
    // clamped to the run's cnt * 32 vectors
    // (unsigned: divisions by the powers of two become shifts; with S = 2, M = NT = 1)
    constexpr unsigned per_seg = NST * 32;
    // (XF: the column vectors of the M rows of f32 x, each feeding all three planes)
    const unsigned nv = S == 2 ? S * per_seg : (XF ? 1 : NT) * (unsigned)a.M * S * per_seg;
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      const unsigned v = min((unsigned)(lane + 64 * i), nv - 1);
      const unsigned pm = S == 2 ? 0u : v / (S * per_seg), sv_ = (v / per_seg) % S;
      const unsigned u = min(v % per_seg, (unsigned)(cnt * 32 - 1));
      xi[i] = (int)(pm * ((unsigned)K >> 3) + sv_ * ((unsigned)KS >> 3) + (unsigned)s0 * 32 + u);
    }
  } else {
    const int nvec = (NT * plane) >> 3;
#pragma unroll
    for (int i = 0; i < XPT; ++i) xi[i] = min((int)threadIdx.x + i * 64 * nwaves, nvec - 1);
  }
  u32x4 xv[XF ? 2 * XPT : XPT];
  if constexpr (XF) {
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      xv[2 * i] = xsrc[2 * xi[i]];
      xv[2 * i + 1] = xsrc[2 * xi[i] + 1];
    }
  } else {
#pragma unroll
    for (int i = 0; i < XPT; ++i) xv[i] = xsrc[xi[i]];
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. scales, then 3. weights, of this wave's NST steps of tile t (the last one clamped
  // into the run: a short run loads its last step twice).  The tile's matrix (a weight
  // group's member, or the single weight) and row pointers are formed first and pinned
  // in VGPRs as global-memory pointers, so that the compiler forms no address between
  // the loads.
  const int pair_f = PLAIN ? 0 : a.pair_f;
  const int cb = seg * (KS >> 5) + s0 * 8 + c * 2;  // first 32-column chunk of the lane's run
  auto step_of = [&](int i) { return i < NST - 1 ? i : min(i, cnt - 1); };
  GroupSel gs;
  int bt;                // tile index within its matrix
  uint32_t sv[NST];      // two bf16 scales (low half: the step's first vector)
  u32x4 wv[NST][VPL];
  auto issue = [&](int t) __attribute__((always_inline)) {
    gs = (PLAIN || LOOP) ? GroupSel{a.pk, a.sc, a.y, a.N, 0} : group_select(a, t);
    bt = t - gs.tile0;
    const int tile = min(bt, (gs.N + R - 1) / R - 1);
    const uint32_t* pkrow;
    const uint16_t* scrow;
    weight_row(gs.pk, gs.sc, a.pk2, a.sc2, pair_f, tile * R + rr, gs.N, K, a.groups_per_row, pkrow, scrow);
    g_u4* wb = (g_u4*)(reinterpret_cast<const u32x4*>(pkrow) + cb);
    g_u32* sb = (g_u32*)(reinterpret_cast<const uint32_t*>(scrow) + (cb >> 1));
    asm volatile("" : "+v"(wb), "+v"(sb));
    __builtin_amdgcn_sched_barrier(0);
    if (G32) {
#pragma unroll
      for (int i = 0; i < NST; ++i) sv[i] = sb[4 * step_of(i)];
    } else {
#pragma unroll
      for (int i = 0; i < NST; ++i) {
        const int g0 = cb + 8 * step_of(i);
        sv[i] = (uint32_t)scrow[g0 / a.group_chunks] | ((uint32_t)scrow[(g0 + 1) / a.group_chunks] << 16);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      wv[i][0] = wb[8 * step_of(i)];
      wv[i][1] = wb[8 * step_of(i) + 1];
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  int t = (int)blockIdx.x;
  issue(t);
  __builtin_amdgcn_s_setprio(0);

  // 4. x -> LDS ([NT][M][K] halves); with XW a wave reads only what it wrote, and a
  // wave's LDS accesses complete in order, so no barrier is needed
  u32x4* xdst = reinterpret_cast<u32x4*>(lds);
  if constexpr (XF) {
    const int pv = plane >> 3;  // 16-byte vectors per plane
#pragma unroll
    for (int i = 0; i < XPT; ++i) {
      u32x4 t0, t1, t2;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        uint32_t h0[2], h1[2], h2[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) split3_terms(xv[2 * i + (e >> 1)][2 * (e & 1) + q], h0[q], h1[q], h2[q]);
        t0[e] = h0[0] | (h0[1] << 16);
        t1[e] = h1[0] | (h1[1] << 16);
        t2[e] = h2[0] | (h2[1] << 16);
      }
      xdst[xi[i]] = t0;
      xdst[pv + xi[i]] = t1;
      xdst[2 * pv + xi[i]] = t2;
    }
  } else {
#pragma unroll
    for (int i = 0; i < XPT; ++i) xdst[xi[i]] = xv[i];
  }
  if (!XW) __syncthreads();

  const MixMasks km = mix_masks();
  // A row r: x row r (S = 1, rows past M repeat row M - 1) or x segment r (S = 2)
  const uint16_t* xrow = S == 1 ? lds + min(r, a.M - 1) * K : lds + (r < S ? r : 0) * KS;
  // partial sums [2][waves][MR][16]: consecutive tiles of a workgroup use alternate halves
  float* red = reinterpret_cast<float*>(lds + NT * plane);
  for (int it = 0;; ++it) {
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < NST; ++i) {
      if (i < NST - 1 || i < cnt) {
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
          const MixScale Sc = mix_scale(v == 0 ? (sv[i] & 0xffffu) : (sv[i] >> 16));
          const uint16_t* xr = xrow + 32 * ((s0 + i) * 8 + c * 2 + v);
          const uint32_t wj[4] = {wv[i][v][0], wv[i][v][1], wv[i][v][2], wv[i][v][3]};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const bf16x8 bb = dequant8_mix(wj[j], Sc, km);
#pragma unroll
            for (int q = 0; q < NT; ++q)
              acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(*reinterpret_cast<const bf16x8*>(xr + q * plane + 8 * j),
                                                            bb, acc, 0, 0, 0);
          }
        }
      }
    }
    // this tile's output; the next tile's loads go out before its epilogue
    const GroupSel go = gs;
    const int bo = bt;
    const int tn = t + a.gstride;
    if (LOOP && tn < T) {
      __builtin_amdgcn_s_setprio(3);
      issue(tn);
      __builtin_amdgcn_s_setprio(0);
    }

    // D: lane (r, c) holds rows m = 4c + i of column r; MR = 4 keeps c == 0 only.  With
    // K segments, column r's sum is D[seg][r]: select it, then add the two segments of
    // row rr (lanes rr and rr + 8, one DPP rotation apart).
    float* rb = red + (it & 1) * nwaves * MR * 16;
    if (S == 2) {
      float v = seg == 0 ? acc[0] : acc[1];
      v += lane_xor8(v);
      if (c == 0) rb[(wave * MR) * 16 + r] = v;
    } else if (MR == 16 || c == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) rb[(wave * MR + (MR == 16 ? 4 * c : 0) + i) * 16 + r] = acc[i];
    }
    // (the other half was last read before the previous barrier, so one barrier per tile
    // orders both the writes above and their reads below)
    __builtin_amdgcn_s_setprio(2);
    __syncthreads();
    const int N = go.N;
    for (int e = (int)threadIdx.x; e < 16 * MR; e += 64 * nwaves) {
      const int m = e >> 4, ro = e & 15;
      const int n = bo * R + ro;
      if (pair_f) {
        // gate row ro < 8 of the tile and its up row ro + 8
        const int f = (bo << 3) + ro;
        if (ro < 8 && m < a.M && f < pair_f) {
          float g = 0.f, u = 0.f;
          for (int w = 0; w < nwaves; ++w) {
            g += rb[(w * MR + m) * 16 + ro];
            u += rb[(w * MR + m) * 16 + ro + 8];
          }
          store_gelu_mul(a.y, a.y_f32, a.bf16_dots, (int64_t)m * pair_f + f, g, u);
        }
      } else if (m < a.M && ro < R && n < N) {
        float v = 0.f;
        for (int w = 0; w < nwaves; ++w) v += rb[(w * MR + m) * 16 + ro];
        if (a.y_f32) reinterpret_cast<float*>(go.y)[(int64_t)m * N + n] = v;
        else reinterpret_cast<uint16_t*>(go.y)[(int64_t)m * N + n] = (uint16_t)f32_to_bf16_rne(v);
      }
    }
    if (!LOOP || tn >= T) break;
    t = tn;
    __builtin_amdgcn_s_setprio(0);
  }
}

// ---------------------------------------------------------------- skinny / prefill linear
// M > 4, bf16 x, K % 256 == 0.  A workgroup of 4 waves owns 64 rows of W (16 per
// wave) and 16*MT rows of x, and walks K in chunks of 256 columns.  Per chunk:
//   - x[16*MT][256] is staged in LDS (double buffered; the global loads of the
//     chunk after next are issued two chunks ahead, into a register ring),
//   - each wave expands its 16 rows x 256 columns of W once in registers and
//     feeds every 16x32 weight fragment to MT MFMAs (one per 16 rows of x),
//   - weights are prefetched P chunks ahead in a register ring.
// Every load is unconditional (chunk index clamped to the last chunk), and the
// main loop is unrolled by P so that the ring slots are compile-time registers;
// together these keep the compiler's wait counts exact.  Rows of x past M
// duplicate row M-1 and rows of W past N duplicate row N-1; neither is stored.
// Grid: (ceil(N/64), ceil(M/(16*MT))); large M re-expands W once per 16*MT rows.
struct SkinnyArgs {
  const uint16_t* x;  // [M][K] bf16
  const uint32_t* pk;
  const uint16_t* sc;
  void* y;
  int M, N, K;
  int group_chunks;    // group / 32
  int groups_per_row;  // K / group
  int y_f32;
  int nk;              // chunks of 256 columns per K part (K / 256 / kq)
  // gate/up pair mode, as GemvArgs
  const uint32_t* pk2;
  const uint16_t* sc2;
  int pair_f;
  int bf16_dots;
  // K split (grid.z = kq parts of nk chunks): kq > 1 writes f32 partial sums
  // part[kq][M][N] (N in virtual rows in pair mode) for splitk_finalize_kernel
  int kq;
  float* part;
};

// Weight prefetch depth (chunks); even, for the two-slot x ring.  Four x blocks (MT = 4,
// M = 49..64) take 2: with a wave waiting on its x staging (an in-order vmcnt wait that
// also covers every earlier weight load) the deeper ring only adds registers (12B gate/up
// at M = 64: 30.1 -> 28.9 us in the lab; 8 slots were 8-10 % slower at every M).
template <int MT>
constexpr int sk_prefetch() { return MT == 4 ? 2 : 4; }

// NW waves of 16 W rows per workgroup (4 or 8): 8 halves the x traffic from L2
// (x is staged once per 16 * NW rows of W).
template <int MT, bool G32, int NW = 4>
__global__ void __launch_bounds__(64 * NW) skinny_kernel(SkinnyArgs a) {
  constexpr int NTH = 64 * NW;
  constexpr int P = sk_prefetch<MT>();
  // x rows of 256 halves as 4 groups of 64 (one lane group c each), every group padded
  // to 72 halves and every row to 304: the A-fragment reads (16 rows, lane groups
  // 144 B apart) are then free of LDS bank conflicts (measured on gfx950: a 16-byte
  // row pad with groups 128 B apart reads 18 % slower), and every (v, j) read is an
  // immediate offset from one address per lane.
  constexpr int XG = 72, XROW = 304;
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][16 * MT][XROW];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, c = lane >> 4;
  const int m0 = blockIdx.y * (16 * MT);
  const int kb = (int)blockIdx.z * a.nk;  // first chunk of this K part
  const uint32_t* pkrow;
  const uint16_t* scrow;
  weight_row(a.pk, a.sc, a.pk2, a.sc2, a.pair_f, (int)blockIdx.x * (16 * NW) + 16 * wave + r, a.N, a.K,
             a.groups_per_row, pkrow, scrow);

  // weight ring: chunk k -> slot k % P; lane (r, c) holds the 32-column chunks
  // 8k + 2c and 8k + 2c + 1 of its row (two 16-byte vectors) and their scales.
  uint4 wv[P][2];
  uint32_t sv[P];
  auto wload = [&](auto slot_c, int k) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    const int g0 = ((kb + k) * 4 + c) * 2;
    wv[slot][0] = *reinterpret_cast<const uint4*>(pkrow + 4 * g0);
    wv[slot][1] = *reinterpret_cast<const uint4*>(pkrow + 4 * g0 + 4);
    if (G32) sv[slot] = *reinterpret_cast<const uint32_t*>(scrow + g0);
    else sv[slot] = (uint32_t)scrow[g0 / a.group_chunks] | ((uint32_t)scrow[(g0 + 1) / a.group_chunks] << 16);
  };

  // x staging: thread t moves vectors t + 256 i (i < 2*MT) of the [16*MT][256] chunk.
  // The register ring is an ext_vector value (not an array) so that it never lives
  // in scratch memory.
  constexpr int XV = 512 * MT / NTH;
  typedef uint32_t xvec_t __attribute__((ext_vector_type(4 * XV)));
  auto xload = [&](xvec_t& xr, int k) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int v = (int)threadIdx.x + NTH * i;
      const int row = v >> 5, col = (v & 31) * 8;
      const int m = min(m0 + row, a.M - 1);
      const u32x4 t = *reinterpret_cast<const u32x4*>(a.x + (int64_t)m * a.K + (kb + k) * 256 + col);
      xr[4 * i] = t[0];
      xr[4 * i + 1] = t[1];
      xr[4 * i + 2] = t[2];
      xr[4 * i + 3] = t[3];
    }
  };
  auto xstore = [&](const xvec_t& xr, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int v = (int)threadIdx.x + NTH * i;
      const int row = v >> 5, col = (v & 31) * 8;
      *reinterpret_cast<u32x4*>(&xs[buf][row][(col >> 6) * XG + (col & 63)]) =
          u32x4{xr[4 * i], xr[4 * i + 1], xr[4 * i + 2], xr[4 * i + 3]};
    }
  };

  // prologue: x chunk 0 -> LDS buffer 0, x chunk 1 -> register slot 1, weights 0..P-1
  xvec_t xreg0, xreg1;
  xload(xreg0, 0);
  xload(xreg1, min(1, a.nk - 1));
  static_for<0, P>([&](auto i_c) __attribute__((always_inline)) {
    wload(i_c, min((int)decltype(i_c)::value, a.nk - 1));
  });
  xstore(xreg0, 0);
  __syncthreads();

  const MixMasks km = mix_masks();
  floatx4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Weights expanded with dequant8_mix (written in C: the compiler sees every hazard,
  // so the MFMAs are the builtin and need no drain).  Against the asm v_dot2 form
  // (19 VALU per 8 weights) it measured 4-7 % faster at M = 16..64 (12B gate/up).
  auto compute = [&](auto slot_c, int buf) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
#pragma unroll
    for (int v = 0; v < 2; ++v) {
      const MixScale S = mix_scale(v == 0 ? (sv[slot] & 0xffffu) : (sv[slot] >> 16));
      // every A fragment of this half-chunk first: one LDS round trip
      bf16x8 xa[4][MT];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          xa[j][mt] = *reinterpret_cast<const bf16x8*>(&xs[buf][16 * mt + r][c * XG + v * 32 + 8 * j]);
      __builtin_amdgcn_sched_barrier(0);
      const uint32_t wj[4] = {wv[slot][v].x, wv[slot][v].y, wv[slot][v].z, wv[slot][v].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const bf16x8 bb = dequant8_mix(wj[j], S, km);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[j][mt], bb, acc[mt], 0, 0, 0);
      }
    }
  };

  // chunk k: x of chunk k+2 into register slot k%2 (chunk k left it last
  // iteration), compute from LDS buffer k%2, weights of chunk k+P into slot k%P,
  // x of chunk k+1 (register slot (k+1)%2) into LDS buffer (k+1)%2, barrier.
  auto iter = [&](int k, auto slot_c) __attribute__((always_inline)) {
    constexpr int p = decltype(slot_c)::value;
    if constexpr (p % 2 == 0) xload(xreg0, min(k + 2, a.nk - 1));
    else xload(xreg1, min(k + 2, a.nk - 1));
    compute(slot_c, k & 1);
    wload(slot_c, min(k + P, a.nk - 1));
    if constexpr (p % 2 == 0) xstore(xreg1, (k + 1) & 1);
    else xstore(xreg0, (k + 1) & 1);
    __syncthreads();
  };
  int k = 0;
  for (; k + P <= a.nk; k += P)
    static_for<0, P>([&](auto i_c) __attribute__((always_inline)) { iter(k + decltype(i_c)::value, i_c); });
  static_for<0, P - 1>([&](auto i_c) __attribute__((always_inline)) {
    if (k + decltype(i_c)::value < a.nk) iter(k + decltype(i_c)::value, i_c);
  });

  // D layout: lane (n = r, c) holds D[m = 4c + i][n]
  const int nout = (int)blockIdx.x * (16 * NW) + 16 * wave + r;
  if (a.kq > 1) {
    if (nout < a.N) {
      float* pp = a.part + (int64_t)blockIdx.z * a.M * a.N + nout;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = m0 + 16 * mt + 4 * c + i;
          if (m < a.M) pp[(int64_t)m * a.N] = acc[mt][i];
        }
    }
  } else if (a.pair_f) {
    // Lanes r and r ^ 8 hold gate and up of row f for the same m; per pair of
    // rows m, m + 1 the gate lane finishes m and the up lane m + 1 (all lanes
    // active here).
    const int f = ((nout >> 4) << 3) | (r & 7);
    const int up = (r >> 3) & 1;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; i += 2) {
        const float p0 = lane_xor8(acc[mt][i]), p1 = lane_xor8(acc[mt][i + 1]);
        const float g = up ? p1 : acc[mt][i];
        const float u = up ? acc[mt][i + 1] : p0;
        const int m = m0 + 16 * mt + 4 * c + i + up;
        if (f < a.pair_f && m < a.M) store_gelu_mul(a.y, a.y_f32, a.bf16_dots, (int64_t)m * a.pair_f + f, g, u);
      }
  } else if (nout < a.N) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = m0 + 16 * mt + 4 * c + i;
        if (m < a.M) {
          const float v = acc[mt][i];
          if (a.y_f32) reinterpret_cast<float*>(a.y)[(int64_t)m * a.N + nout] = v;
          else reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.N + nout] = (uint16_t)f32_to_bf16_rne(v);
        }
      }
  }
}

// ---------------------------------------------------------------- prefill linear (M > 64)
// bf16 x, K % 64 == 0.  v_mfma_f32_32x32x16_bf16 with the accumulators in AGPRs.
// A workgroup of 4 waves owns 256 rows of x (staged in LDS, 64 columns per step,
// double buffered, global loads two steps ahead) and 4 * 32 * TN rows of W; each
// wave expands its 32 * TN rows of W per step in registers and feeds every
// 16x32 weight fragment to 8 MFMAs (one per 32 rows of x), so each weight is
// expanded once per 256 rows of x.
// Lane layouts (checked on the GPU): A lane l holds A[l % 32][8 (l / 32) + i],
// B lane l holds B[8 (l / 32) + i][l % 32], D lane l value e holds
// D[8 (e / 4) + 4 (l / 32) + e % 4][l % 32].  Lane (n, h) of a W block loads the
// 32 columns [64 s + 32 h, +32) of its row; word j of them feeds MFMA j, whose
// reduction index kk = 8 h + i is column 64 s + 32 h + 8 j + i, and the A
// fragment is read from the same columns of x.
// Workgroup b takes the x block b % mblk and the W block b / mblk: consecutive
// workgroups (placed on different XCDs) share a W block, and an XCD keeps the
// same x rows while it walks W.
__device__ __forceinline__ void mfma32_acc(floatx16& acc, const bf16x8& a, const bf16x8& b) {
  asm("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

struct PrefillArgs {
  const uint16_t* x;  // [M][K] bf16
  const uint32_t* pk;
  const uint16_t* sc;
  void* y;
  int M, N, K;
  int group_chunks;
  int groups_per_row;
  int y_f32;
  int ns;    // steps (64 KS columns each) per K part
  int mblk;  // ceil(M / BM)
  // split K across workgroups: kq parts of ns steps each; part q of every
  // output tile goes to part[q][M][N] (f32), which splitk_finalize_kernel sums
  int kq;
  float* part;
  // gate/up pair mode, as GemvArgs
  const uint32_t* pk2;
  const uint16_t* sc2;
  int pair_f;
  int bf16_dots;
};

// Small M (the skinny regime) uses WS waves of W rows and a K split KS: a step
// covers 64*KS columns, wave (wsub, kh) takes the kh-th 64 of them for its
// 32*TN rows, and the KS partial sums meet in LDS at the end.  That keeps
// enough waves in flight when a 64-row x tile leaves few workgroups, while
// each A fragment still feeds a 32x32x16 MFMA (half the LDS reads per weight
// of the 16x16x32 form).
template <int TN, int P, bool G32, int MB = 8, int WS = 4, int KS = 1>  // MB: 32-row blocks of x per workgroup
__global__ void __launch_bounds__(64 * WS * KS) prefill_kernel(PrefillArgs a) {
  constexpr int NTH = 64 * WS * KS;
  constexpr int BM = 32 * MB;
  constexpr int BN = WS * 32 * TN;
  constexpr int XPAD = 8;
  __shared__ __attribute__((aligned(16))) uint16_t xs[2][KS][BM][64 + XPAD];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wsub = wave % WS, kh = wave / WS;
  const int l32 = lane & 31, h = lane >> 5;
  // workgroup b: K part b % kq (consecutive workgroups, on different XCDs, share
  // the W tile), then x block, then W tile
  const int kpart = (int)blockIdx.x % a.kq;
  const int bt = (int)blockIdx.x / a.kq;
  const int m0 = (bt % a.mblk) * BM;
  const int nw0 = (bt / a.mblk) * BN + wsub * 32 * TN;
  const int sbase = kpart * a.ns;  // first step of this part

  const uint32_t* pkrow[TN];
  const uint16_t* scrow[TN];
#pragma unroll
  for (int t = 0; t < TN; ++t)
    weight_row(a.pk, a.sc, a.pk2, a.sc2, a.pair_f, nw0 + 32 * t + l32, a.N, a.K, a.groups_per_row, pkrow[t],
               scrow[t]);
  uint4 wv[P][TN];
  uint32_t sv[P][TN];
  auto wload = [&](auto slot_c, int s) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      const int g = 2 * ((sbase + s) * KS + kh) + h;
      wv[slot][t] = *reinterpret_cast<const uint4*>(pkrow[t] + 4 * g);
      sv[slot][t] = scrow[t][G32 ? g : g / a.group_chunks];
    }
  };
  // 16-byte vectors of the [BM][64 KS] step per thread; vector v is row
  // v / (8 KS), columns 8 (v % (8 KS)) .. +8 of the step, LDS tile (v % (8 KS)) / 8
  constexpr int XV = BM * 8 * KS / NTH;
  static_assert(XV >= 1 && XV * NTH == BM * 8 * KS, "x step must split evenly over the threads");
  typedef uint32_t xvec_t __attribute__((ext_vector_type(4 * XV)));
  auto xload = [&](xvec_t& xr, int s) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int v = (int)threadIdx.x + NTH * i;
      const int row = v / (8 * KS), col = (v % (8 * KS)) * 8;
      const int m = min(m0 + row, a.M - 1);
      const u32x4 t = *reinterpret_cast<const u32x4*>(a.x + (int64_t)m * a.K + (sbase + s) * 64 * KS + col);
      xr[4 * i] = t[0];
      xr[4 * i + 1] = t[1];
      xr[4 * i + 2] = t[2];
      xr[4 * i + 3] = t[3];
    }
  };
  auto xstore = [&](const xvec_t& xr, int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < XV; ++i) {
      const int v = (int)threadIdx.x + NTH * i;
      const int row = v / (8 * KS), u = v % (8 * KS);
      *reinterpret_cast<u32x4*>(&xs[buf][u >> 3][row][(u & 7) * 8]) =
          u32x4{xr[4 * i], xr[4 * i + 1], xr[4 * i + 2], xr[4 * i + 3]};
    }
  };

  xvec_t xreg0, xreg1;
  xload(xreg0, 0);
  xload(xreg1, min(1, a.ns - 1));
  static_for<0, P>([&](auto i_c) __attribute__((always_inline)) {
    wload(i_c, min((int)decltype(i_c)::value, a.ns - 1));
  });
  xstore(xreg0, 0);
  __syncthreads();

  uint32_t kM = 0x000F000Fu, kO = 0x43004300u;
  asm volatile("" : "+v"(kM), "+v"(kO));
  floatx16 acc[MB][TN];
#pragma unroll
  for (int i = 0; i < MB; ++i)
#pragma unroll
    for (int t = 0; t < TN; ++t) acc[i][t] = floatx16{};

  auto compute = [&](auto slot_c, int buf) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    uint32_t shi[TN];
    float cn[TN];
#pragma unroll
    for (int t = 0; t < TN; ++t) {
      shi[t] = sv[slot][t] << 16;
      cn[t] = -136.0f * __uint_as_float(shi[t]);
    }
    bf16x8 xa[2][MB];
#pragma unroll
    for (int i = 0; i < MB; ++i) xa[0][i] = *reinterpret_cast<const bf16x8*>(&xs[buf][kh][32 * i + l32][32 * h]);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // A fragments of step j+1 go out before the MFMAs of step j; the scheduling
      // barriers keep the compiler from sinking them next to their uses (it does
      // not know the asm MFMAs' latency and would serialize load -> wait -> MFMA).
      if (j < 3) {
#pragma unroll
        for (int i = 0; i < MB; ++i)
          xa[(j + 1) & 1][i] = *reinterpret_cast<const bf16x8*>(&xs[buf][kh][32 * i + l32][32 * h + 8 * (j + 1)]);
      }
      __builtin_amdgcn_sched_barrier(0);
      bf16x8 bb[TN];
#pragma unroll
      for (int t = 0; t < TN; ++t) {
        const uint32_t w = j == 0 ? wv[slot][t].x : j == 1 ? wv[slot][t].y : j == 2 ? wv[slot][t].z : wv[slot][t].w;
        bb[t] = dequant8(w, sv[slot][t], shi[t], cn[t], kM, kO);
      }
#pragma unroll
      for (int i = 0; i < MB; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t) mfma32_acc(acc[i][t], xa[j & 1][i], bb[t]);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  auto iter = [&](int s, auto slot_c) __attribute__((always_inline)) {
    constexpr int p = decltype(slot_c)::value;
    if constexpr (p % 2 == 0) xload(xreg0, min(s + 2, a.ns - 1));
    else xload(xreg1, min(s + 2, a.ns - 1));
    compute(slot_c, s & 1);
    wload(slot_c, min(s + P, a.ns - 1));
    if constexpr (p % 2 == 0) xstore(xreg1, (s + 1) & 1);
    else xstore(xreg0, (s + 1) & 1);
    __syncthreads();
  };
  static_assert(P % 2 == 0, "the unrolled ring alternates the two x register slots");
  int s = 0;
  for (; s + P <= a.ns; s += P)
    static_for<0, P>([&](auto i_c) __attribute__((always_inline)) { iter(s + decltype(i_c)::value, i_c); });
  static_for<0, P - 1>([&](auto i_c) __attribute__((always_inline)) {
    if (s + decltype(i_c)::value < a.ns) iter(s + decltype(i_c)::value, i_c);
  });
  // the last MFMAs must finish before their AGPRs are read (16-pass MFMA: >= 18 wait states)
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

  if constexpr (KS > 1) {
    // waves kh > 0 hand their partial sums to kh = 0 through the x tiles (idle:
    // every iteration ended with a barrier)
    constexpr int NE = MB * TN * 16;
    static_assert((KS - 1) * WS * NE * 64 * 4 <= (int)sizeof(xs), "reduction buffer fits in the x tiles");
    float* red = reinterpret_cast<float*>(&xs[0][0][0][0]);
    auto at = [&](int q, int e) { return ((q * WS + wsub) * NE + e) * 64 + lane; };
    if (kh > 0) {
      static_for<0, MB>([&](auto i_c) __attribute__((always_inline)) {
        static_for<0, TN>([&](auto t_c) __attribute__((always_inline)) {
          constexpr int i = decltype(i_c)::value, t = decltype(t_c)::value;
#pragma unroll
          for (int e = 0; e < 16; ++e) red[at(kh - 1, (i * TN + t) * 16 + e)] = acc[i][t][e];
        });
      });
    }
    __syncthreads();
    if (kh > 0) return;
    static_for<0, MB>([&](auto i_c) __attribute__((always_inline)) {
      static_for<0, TN>([&](auto t_c) __attribute__((always_inline)) {
        constexpr int i = decltype(i_c)::value, t = decltype(t_c)::value;
#pragma unroll
        for (int q = 0; q < KS - 1; ++q)
#pragma unroll
          for (int e = 0; e < 16; ++e) acc[i][t][e] += red[at(q, (i * TN + t) * 16 + e)];
      });
    });
  }

  if (a.kq > 1) {
    // split K: this part's sums, every row m < M of every row n < N (the pair
    // layout is resolved by the finalize kernel)
    static_for<0, TN>([&](auto t_c) __attribute__((always_inline)) {
      constexpr int t = decltype(t_c)::value;
      const int n = nw0 + 32 * t + l32;
      if (n < a.N) {
        float* pp = a.part + (int64_t)kpart * a.M * a.N + n;
        static_for<0, MB>([&](auto i_c) __attribute__((always_inline)) {
          constexpr int i = decltype(i_c)::value;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int m = m0 + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
            if (m < a.M) pp[(int64_t)m * a.N] = acc[i][t][e];
          }
        });
      }
    });
    return;
  }

  static_for<0, TN>([&](auto t_c) __attribute__((always_inline)) {
    constexpr int t = decltype(t_c)::value;
    const int n = nw0 + 32 * t + l32;
    if (a.pair_f) {
      // Lanes l and l ^ 8 hold gate and up of row f for the same m.  Per pair of
      // values e, e + 1 (rows m, m + 1) the gate lane finishes row m and the up
      // lane row m + 1, so each lane evaluates one activation per pair (all
      // lanes active here).
      const int f = ((n >> 4) << 3) | (l32 & 7);
      const int up = (l32 >> 3) & 1;
      static_for<0, MB>([&](auto i_c) __attribute__((always_inline)) {
        constexpr int i = decltype(i_c)::value;
        static_for<0, 8>([&](auto e_c) __attribute__((always_inline)) {
          constexpr int e = 2 * decltype(e_c)::value;
          const float p0 = lane_xor8(acc[i][t][e]), p1 = lane_xor8(acc[i][t][e + 1]);
          const float g = up ? p1 : acc[i][t][e];
          const float u = up ? acc[i][t][e + 1] : p0;
          const int m = m0 + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3) + up;
          if (f < a.pair_f && m < a.M) store_gelu_mul(a.y, a.y_f32, a.bf16_dots, (int64_t)m * a.pair_f + f, g, u);
        });
      });
    } else if (n < a.N) {
      static_for<0, MB>([&](auto i_c) __attribute__((always_inline)) {
        constexpr int i = decltype(i_c)::value;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = m0 + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
          if (m < a.M) {
            const float v = acc[i][t][e];
            if (a.y_f32) reinterpret_cast<float*>(a.y)[(int64_t)m * a.N + n] = v;
            else reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.N + n] = (uint16_t)f32_to_bf16_rne(v);
          }
        }
      });
    }
  });
}

// ---------------------------------------------------------------- prefill, W expanded into LDS
// M > 64, bf16 x, K % 64 == 0.  A workgroup of 8 waves (two per SIMD) owns 256
// rows of x and 256 rows of W and walks K in steps of 64 columns.  Per step every
// thread expands one 16-byte packed vector (32 weights of one W row, one scale
// group of 32), loaded P steps ahead, into the step's bf16 W tile in LDS, and the
// x tile is staged beside it; both tiles are double buffered.  Wave (wm, wn)
// multiplies x rows 128 wm .. +128 by W rows 64 wn .. +64 as 4 x 2 MFMA tiles of
// 32x32, reading A and B fragments from LDS (rows of 72 halves: both read
// patterns are conflict-free).  Each weight is still expanded once per 256 rows
// of x, and each SIMD has a second wave to issue while one waits.
template <bool G32, int TN = 2>  // TN: W blocks of 32 rows per wave, 128 * TN W rows per workgroup
__global__ void __launch_bounds__(512) prefill_lds_kernel(PrefillArgs a) {
  constexpr int P = 4;          // packed-weight ring depth (steps)
  constexpr int RS = 72;        // LDS row stride (halves)
  constexpr int TILE = 256 * RS;
  constexpr int BN = 128 * TN;
  constexpr int WTILE = BN * RS;
  constexpr int WPT = 2 * TN;       // packed words (8 weights each) a thread expands per step
  constexpr int PPR = 8 / WPT;      // threads per W row
  extern __shared__ __attribute__((aligned(16))) uint16_t lds[];  // xs[2][256][RS] then ws[2][BN][RS]
  uint16_t* const xs = lds;
  uint16_t* const ws = lds + 2 * TILE;
  const int tid = (int)threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, h = lane >> 5;
  // workgroup b: K part b % kq (kq = 1 without a split), then x block, then W block
  const int kpart = (int)blockIdx.x % a.kq;
  const int bt = (int)blockIdx.x / a.kq;
  const int m0 = (bt % a.mblk) * 256;
  const int n0 = (bt / a.mblk) * BN;
  const int ns = a.ns;               // steps of this part
  const int sbase = kpart * a.ns;    // its first step

  // expansion: thread -> W row wr of the tile, its part wh (8 * WPT columns) of the step
  const int wr = tid / PPR, wh = tid % PPR;
  const uint32_t* pkrow;
  const uint16_t* scrow;
  weight_row(a.pk, a.sc, a.pk2, a.sc2, a.pair_f, n0 + wr, a.N, a.K, a.groups_per_row, pkrow, scrow);
  uint32_t wv[P][WPT];
  uint32_t sv[P];
  auto wload = [&](auto slot_c, int s) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    const int w0 = 8 * (sbase + s) + WPT * wh;  // first packed word (column 8 * w0)
    const int g = w0 >> 2;            // its 32-column scale group
    if constexpr (WPT == 4) {
      const uint4 t = *reinterpret_cast<const uint4*>(pkrow + w0);
      wv[slot][0] = t.x; wv[slot][1] = t.y; wv[slot][2] = t.z; wv[slot][3] = t.w;
    } else {
      const uint2 t = *reinterpret_cast<const uint2*>(pkrow + w0);
      wv[slot][0] = t.x; wv[slot][1] = t.y;
    }
    sv[slot] = scrow[G32 ? g : g / a.group_chunks];
  };
  const MixMasks km = mix_masks();
  auto expand = [&](auto slot_c, int buf) __attribute__((always_inline)) {
    constexpr int slot = decltype(slot_c)::value;
    const MixScale S = mix_scale(sv[slot] & 0xffffu);
    uint16_t* dst = ws + buf * WTILE + wr * RS + 8 * WPT * wh;
#pragma unroll
    for (int j = 0; j < WPT; ++j)
      *reinterpret_cast<bf16x8*>(dst + 8 * j) = dequant8_mix(wv[slot][j], S, km);
  };
  // x tile [256][64]: vector v = tid + 512 i is row v / 8, columns 8 (v % 8) .. +8
  u32x4 xr[4];
  auto xload = [&](int s) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 512 * i;
      const int m = min(m0 + (v >> 3), a.M - 1);
      xr[i] = *reinterpret_cast<const u32x4*>(a.x + (int64_t)m * a.K + 64 * (sbase + s) + 8 * (v & 7));
    }
  };
  auto xstore = [&](int buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int v = tid + 512 * i;
      *reinterpret_cast<u32x4*>(xs + buf * TILE + (v >> 3) * RS + 8 * (v & 7)) = xr[i];
    }
  };

  floatx16 acc[4][TN];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < TN; ++t) acc[i][t] = floatx16{};
  auto compute = [&](int buf) __attribute__((always_inline)) {
    const uint16_t* xb = xs + buf * TILE + (128 * wm + l32) * RS + 32 * h;
    const uint16_t* wb = ws + buf * WTILE + (32 * TN * wn + l32) * RS + 32 * h;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bf16x8 av[4], bv[TN];
#pragma unroll
      for (int i = 0; i < 4; ++i) av[i] = *reinterpret_cast<const bf16x8*>(xb + 32 * i * RS + 8 * j);
#pragma unroll
      for (int t = 0; t < TN; ++t) bv[t] = *reinterpret_cast<const bf16x8*>(wb + 32 * t * RS + 8 * j);
      // TN = 2: builtin MFMAs (the expansion is C code, so the compiler sees every hazard
      // and schedules the fragment reads around the MFMAs), 4 % faster than the asm form
      // on 12B gate/up at M = 512 and 2048 with bit-identical output; TN = 1 measured
      // 9-19 % slower with them (12B down at M = 256 and 2048) and keeps the asm form.
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int t = 0; t < TN; ++t) {
          if constexpr (TN == 2) acc[i][t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av[i], bv[t], acc[i][t], 0, 0, 0);
          else mfma32_acc(acc[i][t], av[i], bv[t]);
        }
    }
  };

  // prologue: packed steps 0..P-1 (slot k = step k), step 0 expanded and slot 0
  // refilled with step P, x of step 0 staged
  static_for<0, P>([&](auto i_c) __attribute__((always_inline)) {
    wload(i_c, min((int)decltype(i_c)::value, ns - 1));
  });
  xload(0);
  expand(std::integral_constant<int, 0>{}, 0);
  wload(std::integral_constant<int, 0>{}, min(P, ns - 1));
  xstore(0);
  __syncthreads();
  // step s (ring slot (s + 1) % P holds step s + 1): x of step s + 1 into registers,
  // the MFMAs of step s, step s + 1 expanded into the other W buffer and its slot
  // refilled with step s + 1 + P, x of step s + 1 into the other x buffer, barrier
  auto iter = [&](int s, auto i_c) __attribute__((always_inline)) {
    constexpr int i = decltype(i_c)::value;
    xload(min(s + 1, ns - 1));
    compute(s & 1);
    expand(std::integral_constant<int, (i + 1) % P>{}, (s + 1) & 1);
    wload(std::integral_constant<int, (i + 1) % P>{}, min(s + 1 + P, ns - 1));
    xstore((s + 1) & 1);
    __syncthreads();
  };
  int s = 0;
  for (; s + P <= ns; s += P)
    static_for<0, P>([&](auto i_c) __attribute__((always_inline)) { iter(s + decltype(i_c)::value, i_c); });
  static_for<0, P - 1>([&](auto i_c) __attribute__((always_inline)) {
    if (s + decltype(i_c)::value < ns) iter(s + decltype(i_c)::value, i_c);
  });
  // asm MFMAs (TN = 1) must finish before their AGPRs are read (16-pass MFMA: >= 18 wait states)
  if constexpr (TN != 2) asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");

  const int mb0 = m0 + 128 * wm;
  if (a.kq > 1) {
    // split K: this part's sums for every row m < M of every row n < N (the pair
    // layout is resolved by the finalize kernel)
    static_for<0, TN>([&](auto t_c) __attribute__((always_inline)) {
      constexpr int t = decltype(t_c)::value;
      const int n = n0 + 32 * TN * wn + 32 * t + l32;
      if (n < a.N) {
        float* pp = a.part + (int64_t)kpart * a.M * a.N + n;
        static_for<0, 4>([&](auto i_c) __attribute__((always_inline)) {
          constexpr int i = decltype(i_c)::value;
#pragma unroll
          for (int e = 0; e < 16; ++e) {
            const int m = mb0 + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
            if (m < a.M) pp[(int64_t)m * a.N] = acc[i][t][e];
          }
        });
      }
    });
    return;
  }
  static_for<0, TN>([&](auto t_c) __attribute__((always_inline)) {
    constexpr int t = decltype(t_c)::value;
    const int n = n0 + 32 * TN * wn + 32 * t + l32;
    if (a.pair_f) {
      // lanes l and l ^ 8 hold gate and up of row f for the same m (as prefill_kernel)
      const int f = ((n >> 4) << 3) | (l32 & 7);
      const int up = (l32 >> 3) & 1;
      static_for<0, 4>([&](auto i_c) __attribute__((always_inline)) {
        constexpr int i = decltype(i_c)::value;
        static_for<0, 8>([&](auto e_c) __attribute__((always_inline)) {
          constexpr int e = 2 * decltype(e_c)::value;
          const float p0 = lane_xor8(acc[i][t][e]), p1 = lane_xor8(acc[i][t][e + 1]);
          const float g = up ? p1 : acc[i][t][e];
          const float u = up ? acc[i][t][e + 1] : p0;
          const int m = mb0 + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3) + up;
          if (f < a.pair_f && m < a.M) store_gelu_mul(a.y, a.y_f32, a.bf16_dots, (int64_t)m * a.pair_f + f, g, u);
        });
      });
    } else if (n < a.N) {
      static_for<0, 4>([&](auto i_c) __attribute__((always_inline)) {
        constexpr int i = decltype(i_c)::value;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
          const int m = mb0 + 32 * i + 8 * (e >> 2) + 4 * h + (e & 3);
          if (m < a.M) {
            const float v = acc[i][t][e];
            if (a.y_f32) reinterpret_cast<float*>(a.y)[(int64_t)m * a.N + n] = v;
            else reinterpret_cast<uint16_t*>(a.y)[(int64_t)m * a.N + n] = (uint16_t)f32_to_bf16_rne(v);
          }
        }
      });
    }
  });
}

// Split-K combine: y[m][n] = sum over q < kq of part[q][m][n] (f32 or bf16 out),
// or in gate/up pair mode (pair_f = F) h[m][f] = gelu(g) * u with g and u the
// sums of virtual rows ((f >> 3) << 4) | (f & 7) and that | 8.  The parts are
// added in q order, so the result does not depend on scheduling.
__global__ void __launch_bounds__(256) splitk_finalize_kernel(const float* __restrict__ part, int kq, int M, int N,
                                                              void* y, int y_f32, int pair_f, int bf16_dots) {
  const int cols = pair_f ? pair_f : N;
  const int64_t total = (int64_t)M * cols;
  const int64_t plane = (int64_t)M * N;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  if ((cols & 3) == 0 && (N & 3) == 0) {
    // four consecutive outputs per thread (16-byte loads; in pair mode four
    // consecutive f map to four consecutive virtual rows of the same tile)
    for (int64_t i4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i4 < total / 4; i4 += stride) {
      const int64_t i = 4 * i4;
      const int m = (int)(i / cols), col = (int)(i % cols);
      const int vc = pair_f ? (((col >> 3) << 4) | (col & 7)) : col;
      const float4* pv = reinterpret_cast<const float4*>(part + (int64_t)m * N + vc);
      float4 g = pv[0], u = make_float4(0.f, 0.f, 0.f, 0.f);
      if (pair_f) u = pv[2];  // + 8 floats
      // parts in batches of FB: the batch's loads are issued together (indices
      // clamped in bounds), then added in q order
      constexpr int FB = 8;
      for (int q0 = 1; q0 < kq; q0 += FB) {
        float4 t[FB], w[FB];
#pragma unroll
        for (int i = 0; i < FB; ++i) {
          const int64_t o = (int64_t)min(q0 + i, kq - 1) * (plane / 4);
          t[i] = pv[o];
          if (pair_f) w[i] = pv[o + 2];
        }
#pragma unroll
        for (int i = 0; i < FB; ++i) {
          if (q0 + i < kq) {
            g.x += t[i].x; g.y += t[i].y; g.z += t[i].z; g.w += t[i].w;
            if (pair_f) { u.x += w[i].x; u.y += w[i].y; u.z += w[i].z; u.w += w[i].w; }
          }
        }
      }
      if (pair_f) {
        store_gelu_mul(y, y_f32, bf16_dots, i, g.x, u.x);
        store_gelu_mul(y, y_f32, bf16_dots, i + 1, g.y, u.y);
        store_gelu_mul(y, y_f32, bf16_dots, i + 2, g.z, u.z);
        store_gelu_mul(y, y_f32, bf16_dots, i + 3, g.w, u.w);
      } else if (y_f32) {
        reinterpret_cast<float4*>(y)[i4] = g;
      } else {
        const uint32_t lo = f32_to_bf16_rne(g.x) | (f32_to_bf16_rne(g.y) << 16);
        const uint32_t hi = f32_to_bf16_rne(g.z) | (f32_to_bf16_rne(g.w) << 16);
        reinterpret_cast<uint2*>(y)[i4] = make_uint2(lo, hi);
      }
    }
    return;
  }
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int m = (int)(i / cols), col = (int)(i % cols);
    if (pair_f) {
      const int vg = ((col >> 3) << 4) | (col & 7);
      const float* pg = part + (int64_t)m * N + vg;
      float g = 0.f, u = 0.f;
      for (int q = 0; q < kq; ++q) {
        g += pg[q * plane];
        u += pg[q * plane + 8];
      }
      store_gelu_mul(y, y_f32, bf16_dots, i, g, u);
    } else {
      const float* pv = part + (int64_t)m * N + col;
      float v = 0.f;
      for (int q = 0; q < kq; ++q) v += pv[q * plane];
      if (y_f32) reinterpret_cast<float*>(y)[i] = v;
      else reinterpret_cast<uint16_t*>(y)[i] = (uint16_t)f32_to_bf16_rne(v);
    }
  }
}

// h = gelu(g) * u elementwise over f32 g, u: the combine step of the unfused
// gate/up route (shapes no pair-mode kernel takes).
__global__ void __launch_bounds__(256) gelu_mul_kernel(const float* __restrict__ g, const float* __restrict__ u,
                                                       void* h, int h_f32, int bf16_dots, int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    store_gelu_mul(h, h_f32, bf16_dots, i, g[i], u[i]);
}

// K == 0: y = 0 (a kernel rather than a memset, so callers may capture it in a graph).
__global__ void __launch_bounds__(256) fill_zero_kernel(uint16_t* __restrict__ p, int64_t nhalves) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nhalves; i += stride) p[i] = 0;
}

}  // namespace w4k

// ---------------------------------------------------------------- launchers
// Called by the C ABI (w4a16_abi.cpp) after argument validation.

#include "w4a16_launch.h"

namespace {
int grid_for(int64_t work, int block) {
  int64_t g = (work + block - 1) / block;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}
}  // namespace

// Four words per thread once there are enough words for ~1024 workgroups of them;
// below that one word per thread (more workgroups on small matrices: a 2048 x 1536
// dequant took 3.6 us at U = 1 against 4.0 at U = 4).
constexpr int64_t kWordsPerThreadMin = 1ll << 20;

hipError_t w4l_unpack(const int32_t* pk, int8_t* q, int64_t nwords, hipStream_t st) {
  const uint32_t* p = reinterpret_cast<const uint32_t*>(pk);
  if (nwords >= kWordsPerThreadMin)
    hipLaunchKernelGGL(w4k::unpack_kernel<4>, dim3((unsigned)((nwords + 1023) / 1024)), dim3(256), 0, st, p, q,
                       nwords);
  else
    hipLaunchKernelGGL(w4k::unpack_kernel<1>, dim3((unsigned)((nwords + 255) / 256)), dim3(256), 0, st, p, q,
                       nwords);
  return hipGetLastError();
}

hipError_t w4l_dequant(const int32_t* pk, const uint16_t* sc, uint16_t* w, int64_t N, int64_t K,
                       int32_t group, hipStream_t st) {
  const int64_t nwords = N * (K / 8);
  const int64_t wpg = group / 8;
  const int shift = (wpg & (wpg - 1)) == 0 ? __builtin_ctzll((unsigned long long)wpg) : -1;
  const uint32_t* p = reinterpret_cast<const uint32_t*>(pk);
  if (nwords >= kWordsPerThreadMin)
    hipLaunchKernelGGL(w4k::dequant_kernel<4>, dim3((unsigned)((nwords + 1023) / 1024)), dim3(256), 0, st, p, sc,
                       w, nwords, wpg, shift);
  else
    hipLaunchKernelGGL(w4k::dequant_kernel<1>, dim3((unsigned)((nwords + 255) / 256)), dim3(256), 0, st, p, sc,
                       w, nwords, wpg, shift);
  return hipGetLastError();
}

hipError_t w4l_split3(const float* x, uint16_t* out, int64_t n, hipStream_t st) {
  const int block = 256;
  hipLaunchKernelGGL(w4k::split3_kernel, dim3(grid_for(n, block)), dim3(block), 0, st, x, out, n);
  return hipGetLastError();
}

hipError_t w4l_fill_zero(void* p, int64_t bytes, hipStream_t st) {
  const int block = 256;
  const int64_t nhalves = bytes / 2;
  hipLaunchKernelGGL(w4k::fill_zero_kernel, dim3(grid_for(nhalves, block)), dim3(block), 0, st,
                     reinterpret_cast<uint16_t*>(p), nhalves);
  return hipGetLastError();
}


// ---------------------------------------------------------------- decode GEMV plans
namespace {
struct GemvPlan {
  int nst;    // longest run of GSTEP-column steps per wave (compile-time bound)
  int waves;  // waves per workgroup; they split each K segment's steps into runs
  int xpt;    // x vectors per lane (per-wave staging) or per thread (workgroup staging)
  bool xw;    // each wave stages only its own K range of x
  int s;      // K segments per tile (1, or 2: 8-row tiles, M = 1 plain form only)
  int tiles;  // workgroups (tiles of 16 / s rows)
};
// About ten resident waves per SIMD on 256 CUs: a grid of at most this many waves
// issues every load in its first round.
constexpr int64_t GEMV_ONE_ROUND_WAVES = 10240;

int pow2_at_least(int64_t v) {
  int p = 1;
  while (p < v) p *= 2;
  return p;
}

bool nst_instanced(int nst) { return (nst >= 1 && nst <= 6) || nst == 8; }

// M <= 4 (the 4-row epilogue), bf16 or f32 x: runs of two steps per wave, and where
// that leaves fewer than 8192 waves (one round of eight waves per SIMD on 256 CUs),
// more and shorter runs up to 16 waves per workgroup; K in two segments (8-row tiles)
// where M = 1, x is bf16, K allows and the caller takes the plain form.  Measured
// against the uniform-run plans that preceded it (lab sweep over every segment count,
// waves per workgroup and run length on the 12B and E2B rows at M = 1, us): 12B gate/up
// 30720 x 3840 15.0 -> 13.6 (runs 2,..,2,1 over 8 waves; 3-step runs 14.6, 4-step runs
// 14.5, more than 8 waves 15.8-18.6), down 3840 x 15360 9.9 -> 9.1 (two segments, 16
// waves; one segment 9.4, four segments 9.8), q,k,v 8192 x 3840 5.9 -> 5.8, E2B down
// 1536 x 6144 5.3 -> 4.1, E2B double-wide down 1536 x 12288 7.6 -> 5.2, E2B gate/up
// 12288 x 1536 4.9 -> 4.8 and 24576 x 1536 6.8 -> 6.3; q 4096 x 3840 and o 3840 x 4096
// unchanged (4.5).  A/B of the product on one box: 12B gate/up at M = 2 / 4 16.1 / 19.3 ->
// 15.0 / 17.7, with f32 x at M = 1 / 2 23.1 / 27.1 -> 20.4 / 24.2; down, q and E2B rows
// at M = 2..4 unchanged.  The 16-row form (mr = 16, bf16 x, runs of at most 2 steps)
// uses the same rule: E2B down at M = 8 7.7 -> 7.2 us, the other rows it serves unchanged.
// (Through this form at M = 5..16, 12B gate/up measured 13-110 % slower than the skinny
// kernel: every 16-row tile re-reads x from L2; the 40 MiB rule of w4l_gemv16_ok holds.)
bool gemv_plan_runs(int64_t M, int64_t N, int64_t K, int nterms, int mr, bool allow_s2, GemvPlan* out) {
  const int s = allow_s2 && M == 1 && nterms == 1 && K % (2 * w4k::GSTEP) == 0 ? 2 : 1;
  const int64_t steps = K / (w4k::GSTEP * s), tiles = (N + 16 / s - 1) / (16 / s);
  if (steps < 1) return false;
  int64_t nw = (steps + 1) / 2;
  if (nw > 16) nw = 16;
  if (tiles * nw < 8192) {
    int64_t want = (8192 + tiles - 1) / tiles;
    if (want > 16) want = 16;
    if (want > steps) want = steps;
    if (want > nw) nw = want;
  }
  const int nst = (int)((steps + nw - 1) / nw);
  if (!nst_instanced(nst) || (nterms == 3 && nst > 5) || (mr == 16 && nst > 2)) return false;
  const int64_t nv = (int64_t)nterms * M * s * nst * 32;  // x vectors per wave
  if (nv > 64 * 8) return false;
  if ((int64_t)nterms * M * K * 2 + nw * mr * 16 * 4 * 2 > 160 * 1024) return false;
  *out = GemvPlan{nst, (int)nw, pow2_at_least((nv + 63) / 64), true, s, (int)tiles};
  return true;
}

// Straight-line GEMV plan for the 4-row (mr = 4, M <= 4) or 16-row (mr = 16,
// 4 < M <= 16, bf16 x) epilogue.  The 4-row form: gemv_plan_runs where it holds.  Otherwise
// per-wave x staging when a wave's share of x,
// nterms * M * nst * 256 columns, takes at most 8 vectors per lane; then the fewest
// steps per wave (the most waves, up to 16 per workgroup) whose grid of
// tiles * waves stays within one round, else the fewest waves.
// Otherwise (f32 x or 16 rows beyond that share) the workgroup stages all of x behind
// a barrier: the first nst of {5, 2, 4, 1, 3, 6} (4-row form) or the smallest of 1..6
// (16-row form) with at most 16 waves and 8 vectors per thread.  Every wave of these
// plans runs the same number of steps.
bool gemv_plan(int64_t M, int64_t N, int64_t K, int nterms, int mr, GemvPlan* out, bool allow_s2 = false) {
  if (K % w4k::GSTEP != 0 || M < 1 || N <= 0 || K > (1 << 20)) return false;
  if (mr == 4 ? M > 4 : (M > 16 || nterms != 1)) return false;
  if (mr == 4 || nterms == 1) {
    if (allow_s2 && gemv_plan_runs(M, N, K, nterms, mr, true, out)) return true;
    if (gemv_plan_runs(M, N, K, nterms, mr, false, out)) return true;
  }
  const int64_t steps = K / w4k::GSTEP, tiles = (N + 15) / 16;
  const int64_t lds_x = (int64_t)nterms * M * K * 2;
  static const int cand[] = {1, 2, 3, 4, 5, 6, 8};
  bool have = false;
  GemvPlan best{};
  for (int nst : cand) {
    if (steps % nst != 0 || steps / nst > 16) continue;
    if (nterms == 3 && nst > 5) continue;  // the f32-x instances
    if (mr == 16 && nst != 1) continue;    // the 16-row per-wave instances
    const int64_t nv = (int64_t)nterms * M * nst * 32;
    if (nv > 64 * 8) continue;
    const int waves = (int)(steps / nst);
    if (lds_x + (int64_t)waves * mr * 16 * 4 * 2 > 160 * 1024) continue;
    best = GemvPlan{nst, waves, pow2_at_least((nv + 63) / 64), true, 1, (int)tiles};
    have = true;
    if (tiles * waves <= GEMV_ONE_ROUND_WAVES) break;
  }
  if (have) {
    *out = best;
    return true;
  }
  if (nterms == 1 && mr == 4) return false;  // callers take the 16-row or skinny route
  static const int pref4[] = {5, 2, 4, 1, 3, 6};
  static const int pref16[] = {1, 2, 3, 4, 5, 6};
  for (int k = 0; k < 6; ++k) {
    const int nst = mr == 4 ? pref4[k] : pref16[k];
    if (steps % nst != 0 || steps / nst > 16) continue;
    const int waves = (int)(steps / nst);
    const int64_t nvec = (int64_t)nterms * M * K / 8;
    const int64_t per = (nvec + 64 * waves - 1) / (64 * waves);
    if (per > 8) continue;
    if (lds_x + (int64_t)waves * mr * 16 * 4 * 2 > 160 * 1024) continue;
    *out = GemvPlan{nst, waves, pow2_at_least(per), false, 1, (int)tiles};
    return true;
  }
  return false;
}
}  // namespace

// M <= 16 through the 16-row GEMV (for M <= 4 where the 4-row plan does not
// hold) when its plan holds and every 16-row tile
// re-reading x from L2 stays under 40 MiB:
// measured on the 12B and E2B rows, the GEMV wins 1.2-1.9x below that (q, k/v, o,
// E2B) and the skinny kernel, whose workgroups share x over 64-128 rows, wins
// above it (12B gate/up, full-layer q at M = 16).
bool w4l_gemv16_ok(int64_t M, int64_t N, int64_t K, int nterms) {
  GemvPlan p;
  if (!gemv_plan(M, N, K, nterms, 16, &p)) return false;
  const int64_t max_bytes = 40ll << 20;
  return (N + 15) / 16 * M * K * 2 <= max_bytes;
}

// x planes in LDS up to 64 KB per workgroup; f32 x (three planes) up to the 160 KB of a CU,
// where the alternative is the generic kernel (12B down at M = 1: 92 KB of planes)
bool w4l_gemv_ok(int64_t M, int64_t K, int nterms) {
  const int64_t lim = nterms == 3 ? 160 * 1024 : 65536;
  return M >= 1 && M <= 4 && (int64_t)nterms * M * K * 2 + 16 * 4 * 16 * 4 <= lim;
}

bool w4l_gemv_fast_ok(int64_t M, int64_t N, int64_t K, int nterms) {
  GemvPlan p;
  return w4l_gemv_ok(M, K, nterms) && gemv_plan(M, N, K, nterms, 4, &p);
}

// f32 x whose three planes take more than 64 KB of LDS at M >= 2 (one workgroup per CU)
// over more 16-row tiles than the CUs: the planes run as 3M rows of bf16 x instead (12B
// gate/up at M = 3, 4: 26.2 / 32.1 -> 23.1 / 23.5 us; q at M = 4, 256 tiles, stays)
static bool f32x_wide(int64_t M, int64_t N, int64_t K) {
  return M >= 2 && (int64_t)6 * M * K + 16 * 4 * 16 * 4 > 65536 && (N + 15) / 16 > 256;
}
static bool f32x_direct(int64_t M, int64_t N, int64_t K, int32_t group, bool pair);
bool w4l_f32x_rows(int64_t M, int64_t N, int64_t K) {
  return M > 4 || f32x_wide(M, N, K) || !f32x_direct(M, N, K, 32, false);
}

// f32 x straight into the decode GEMV (no split launch): the 4-row plan with per-wave
// staging of three planes, group-32 scales, at most four 8-column vectors of f32 x per lane
static bool f32x_plan_ok(const GemvPlan& p, int64_t M) {
  return p.xw && p.s == 1 && M * p.nst * 32 <= 4 * 64;
}
static bool f32x_direct(int64_t M, int64_t N, int64_t K, int32_t group, bool pair) {
  GemvPlan p;
  if (group != 32 || !w4l_gemv_ok(M, K, 3)) return false;
  if (pair && !gemv_plan(M, N, K, 3, 4, &p)) return false;
  if (!pair && !gemv_plan(M, N, K, 3, 4, &p, true)) return false;
  return f32x_plan_ok(p, M);
}
bool w4l_gemv_f32x_ok(int64_t M, int64_t N, int64_t K, int32_t group, bool pair) {
  return f32x_direct(M, N, K, group, pair) && !f32x_wide(M, N, K);
}

int w4l_gemv_waves(int64_t N, int64_t K) {
  const int64_t steps = (K + w4k::GSTEP - 1) / w4k::GSTEP;
  int64_t w = (steps + w4k::SPW - 1) / w4k::SPW;  // every wave holds <= SPW steps
  if (w > 16) w = 16;
  if (w < 1) w = 1;
  (void)N;
  return (int)w;
}

// Workgroups of `block` threads and `lds` bytes that one CU holds at once for kernel k
// (the occupancy query, remembered per thread for the last kernel, size and LDS asked).
static hipError_t resident_blocks(const void* k, int block, size_t lds, int* out) {
  struct Last {
    const void* k;
    int block;
    size_t lds;
    int n;
  };
  static thread_local Last last{nullptr, 0, 0, 0};
  if (last.k == k && last.block == block && last.lds == lds) {
    *out = last.n;
    return hipSuccess;
  }
  int n = 0;
  const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, k, block, lds);
  if (e != hipSuccess) return e;
  last = Last{k, block, lds, n};
  *out = n;
  return hipSuccess;
}

// CUs of the current device (remembered per device).
static int device_cus() {
  static std::atomic<int> cus[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cus[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cus[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// LDS above 64 KB per workgroup needs the kernel's attribute raised once.
template <class Kern>
static hipError_t allow_big_lds(Kern k, size_t lds) {
  if (lds <= 64 * 1024) return hipSuccess;
  return hipFuncSetAttribute(reinterpret_cast<const void*>(k), hipFuncAttributeMaxDynamicSharedMemorySize,
                             160 * 1024);
}

template <int NT, int NST, int XPT, int MR, bool XW, int S = 1, bool XF = false>
static hipError_t gemv_fast_one(const w4k::GemvArgs& a, dim3 grid, dim3 block, size_t lds, bool g32,
                                hipStream_t st) {
  if constexpr (XF) {
    // f32 x staged by the GEMV itself (group-32 scales only; a weight group, a single
    // weight or a gate/up pair, all of which read x through the same staging)
    if (!g32) return hipErrorInvalidValue;
    auto kf = w4k::gemv_fast_kernel<NT, NST, XPT, true, MR, XW, false, 1, false, true>;
    if (a.nmat <= 1) {
      auto kl = w4k::gemv_fast_kernel<NT, NST, XPT, true, MR, XW, false, 1, true, true>;
      int per_cu = 0;
      hipError_t e = allow_big_lds(kl, lds);
      if (e != hipSuccess) return e;
      e = resident_blocks(reinterpret_cast<const void*>(kl), (int)block.x, lds, &per_cu);
      if (e != hipSuccess) return e;
      const int64_t cap = (int64_t)per_cu * device_cus();
      if (cap > 0 && (int64_t)grid.x > cap) {
        w4k::GemvArgs b = a;
        b.gstride = (int)cap;
        hipLaunchKernelGGL(kl, dim3((unsigned)cap), block, lds, st, b);
        return hipGetLastError();
      }
    }
    hipError_t e = allow_big_lds(kf, lds);
    if (e != hipSuccess) return e;
    w4k::GemvArgs b = a;
    b.gstride = (int)grid.x;
    hipLaunchKernelGGL(kf, grid, block, lds, st, b);
    return hipGetLastError();
  }
  // the plain single-matrix form for bf16 x with per-wave staging and the 4-row epilogue;
  // K segments (S = 2) in that form or for a weight group (no gate/up pair), at M = 1
  constexpr bool PL = NT == 1 && MR == 4 && XW;
  constexpr int S2 = PL ? S : 1;
  const bool plain = PL && a.nmat <= 1 && a.pair_f == 0;
  if (S != 1 && !(PL && a.pair_f == 0 && a.M == 1)) return hipErrorInvalidValue;
  auto k = plain ? (g32 ? w4k::gemv_fast_kernel<NT, NST, XPT, true, MR, XW, PL, S2>
                        : w4k::gemv_fast_kernel<NT, NST, XPT, false, MR, XW, PL, S2>)
                 : (g32 ? w4k::gemv_fast_kernel<NT, NST, XPT, true, MR, XW, false, S2>
                        : w4k::gemv_fast_kernel<NT, NST, XPT, false, MR, XW, false, S2>);
  // The tile loop (one weight or a gate/up pair, group-32 scales, bf16 x at M >= 3 or
  // f32 x at any M, more tiles than one round of workgroups holds): the workgroups that
  // fit on the device at once walk the tiles, each issuing its next tile's loads before
  // the current tile's epilogue and staging x once, instead of a second round of
  // workgroups that starts only as first-round slots free (12B gate/up at M = 4: 19.4 ->
  // 16.7 us; f32 x at M = 2: -7 %).  With bf16 x at M = 1 and 2 it measured 1-8 % slower
  // (the loop's code costs more than the shorter x staging and the missing second round
  // save), and so does a one-round grid.
  if constexpr (MR == 4 && XW && S2 == 1) {
    if (a.nmat <= 1 && g32 && (NT == 3 || a.M >= 3)) {
      // (one instance for the single weight and the gate/up pair: pair_f decides)
      auto kl = w4k::gemv_fast_kernel<NT, NST, XPT, true, MR, XW, false, 1, true>;
      int per_cu = 0;
      hipError_t e = allow_big_lds(kl, lds);
      if (e != hipSuccess) return e;
      e = resident_blocks(reinterpret_cast<const void*>(kl), (int)block.x, lds, &per_cu);
      if (e != hipSuccess) return e;
      const int64_t cap = (int64_t)per_cu * device_cus();
      if (cap > 0 && (int64_t)grid.x > cap) {
        w4k::GemvArgs b = a;
        b.gstride = (int)cap;
        hipLaunchKernelGGL(kl, dim3((unsigned)cap), block, lds, st, b);
        return hipGetLastError();
      }
    }
  }
  hipError_t e = allow_big_lds(k, lds);
  if (e != hipSuccess) return e;
  w4k::GemvArgs b = a;
  b.gstride = (int)grid.x;
  hipLaunchKernelGGL(k, grid, block, lds, st, b);
  return hipGetLastError();
}

// Launch of gemv_fast_kernel for a filled GemvArgs and a plan (instances: bf16 x with
// per-wave staging, steps 1..6 and 8; f32 x per wave up to 5 steps, or the workgroup
// form; the 16-row epilogue per wave at 1 step, or the workgroup form).
static hipError_t gemv_fast_launch(const w4k::GemvArgs& a0, int nterms, int mr, const GemvPlan& p, int nblocks,
                                   bool g32, hipStream_t st) {
  // runs of steps: every K segment's steps over the plan's waves (at least one step each)
  w4k::GemvArgs a = a0;
  const int steps = a.K / (w4k::GSTEP * p.s);
  if (p.waves < 1 || p.waves > steps || (steps + p.waves - 1) / p.waves != p.nst) return hipErrorInvalidValue;
  a.wbase = steps / p.waves;
  a.wrem = steps % p.waves;
  a.ntiles = nblocks;
  a.waves = p.waves;
  // x, then two halves of partial sums (alternate tiles of a workgroup)
  const size_t lds = (size_t)nterms * a.M * a.K * 2 + (size_t)p.waves * mr * 16 * 4 * 2;
  const dim3 grid((unsigned)nblocks), block(64 * p.waves);
#define W4_GFS(NT_, NST_, MR_, XW_, S_)                                                           \
  switch (p.xpt) {                                                                                \
    case 1: return gemv_fast_one<NT_, NST_, 1, MR_, XW_, S_>(a, grid, block, lds, g32, st);       \
    case 2: return gemv_fast_one<NT_, NST_, 2, MR_, XW_, S_>(a, grid, block, lds, g32, st);       \
    case 4: return gemv_fast_one<NT_, NST_, 4, MR_, XW_, S_>(a, grid, block, lds, g32, st);       \
    case 8: return gemv_fast_one<NT_, NST_, 8, MR_, XW_, S_>(a, grid, block, lds, g32, st);       \
    default: return hipErrorInvalidValue;                                                         \
  }
#define W4_GF(NT_, NST_, MR_, XW_) W4_GFS(NT_, NST_, MR_, XW_, 1)
#define W4_GF6(NT_, MR_, XW_)                     \
  switch (p.nst) {                                \
    case 1: W4_GF(NT_, 1, MR_, XW_)               \
    case 2: W4_GF(NT_, 2, MR_, XW_)               \
    case 3: W4_GF(NT_, 3, MR_, XW_)               \
    case 4: W4_GF(NT_, 4, MR_, XW_)               \
    case 5: W4_GF(NT_, 5, MR_, XW_)               \
    case 6: W4_GF(NT_, 6, MR_, XW_)               \
    default: return hipErrorInvalidValue;         \
  }
  if (mr == 4 && nterms == 1 && p.xw && p.s == 2) {
    switch (p.nst) {
      case 1: W4_GFS(1, 1, 4, true, 2)
      case 2: W4_GFS(1, 2, 4, true, 2)
      case 3: W4_GFS(1, 3, 4, true, 2)
      case 4: W4_GFS(1, 4, 4, true, 2)
      case 5: W4_GFS(1, 5, 4, true, 2)
      case 6: W4_GFS(1, 6, 4, true, 2)
      case 8: W4_GFS(1, 8, 4, true, 2)
      default: return hipErrorInvalidValue;
    }
  }
  if (p.s != 1) return hipErrorInvalidValue;
  if (mr == 4 && nterms == 1 && p.xw) {
    switch (p.nst) {
      case 1: W4_GF(1, 1, 4, true)
      case 2: W4_GF(1, 2, 4, true)
      case 3: W4_GF(1, 3, 4, true)
      case 4: W4_GF(1, 4, 4, true)
      case 5: W4_GF(1, 5, 4, true)
      case 6: W4_GF(1, 6, 4, true)
      case 8: W4_GF(1, 8, 4, true)
      default: return hipErrorInvalidValue;
    }
  }
  if (mr == 4 && nterms == 3 && p.xw && a.xf) {
    // f32 x staged in the kernel: XPT counts 8-column vectors of f32 x per lane
    const int xpt = pow2_at_least(((int64_t)a.M * p.nst * 32 + 63) / 64);
#define W4_GFX(NST_)                                                                              \
  switch (xpt) {                                                                                  \
    case 1: return gemv_fast_one<3, NST_, 1, 4, true, 1, true>(a, grid, block, lds, g32, st);     \
    case 2: return gemv_fast_one<3, NST_, 2, 4, true, 1, true>(a, grid, block, lds, g32, st);     \
    case 4: return gemv_fast_one<3, NST_, 4, 4, true, 1, true>(a, grid, block, lds, g32, st);     \
    default: return hipErrorInvalidValue;                                                         \
  }
    switch (p.nst) {
      case 1: W4_GFX(1)
      case 2: W4_GFX(2)
      case 3: W4_GFX(3)
      case 4: W4_GFX(4)
      case 5: W4_GFX(5)
      default: return hipErrorInvalidValue;
    }
#undef W4_GFX
  }
  if (a.xf) return hipErrorInvalidValue;
  if (mr == 4 && nterms == 3 && p.xw) {
    switch (p.nst) {
      case 1: W4_GF(3, 1, 4, true)
      case 2: W4_GF(3, 2, 4, true)
      case 3: W4_GF(3, 3, 4, true)
      case 4: W4_GF(3, 4, 4, true)
      case 5: W4_GF(3, 5, 4, true)
      default: return hipErrorInvalidValue;
    }
  }
  if (mr == 4 && nterms == 3) W4_GF6(3, 4, false)
  if (mr == 16 && nterms == 1 && p.xw) {
    switch (p.nst) {
      case 1: W4_GF(1, 1, 16, true)
      case 2: W4_GF(1, 2, 16, true)
      default: return hipErrorInvalidValue;
    }
  }
  if (mr == 16 && nterms == 1) W4_GF6(1, 16, false)
#undef W4_GF6
#undef W4_GF
#undef W4_GFS
  return hipErrorInvalidValue;
}

// Epilogue rows (4 or 16) and plan of the straight-line GEMV for N rows: the 4-row form
// where its plan holds, else the 16-row form (M <= 16, bf16 x); 0 when neither holds.
// K segments (8-row tiles) except for a gate/up pair.
static int gemv_fast_plan(int64_t M, int64_t N, int64_t K, int nterms, bool pair, GemvPlan* p) {
  if (w4l_gemv_ok(M, K, nterms) && gemv_plan(M, N, K, nterms, 4, p, !pair)) return 4;
  if (gemv_plan(M, N, K, nterms, 16, p)) return 16;
  return 0;
}

hipError_t w4l_gemv(const uint16_t* x_planes, int nterms, const int32_t* pk, const uint16_t* sc,
                    void* y, int y_f32, int64_t M, int64_t N, int64_t K, int32_t group,
                    hipStream_t st, const W4Pair* pair, const float* xf) {
  if (pair) N = 16 * ((pair->F + 7) / 8);
  GemvPlan p;
  const int mr = gemv_fast_plan(M, N, K, xf ? 3 : nterms, pair != nullptr, &p);
  w4k::GemvArgs a{};
  a.x = x_planes;
  if (xf) {
    if (!(mr == 4 && p.xw && group == 32)) return hipErrorInvalidValue;
    a.x = reinterpret_cast<const uint16_t*>(xf);
    a.xf = 1;
    nterms = 3;
  }
  a.pk = reinterpret_cast<const uint32_t*>(pk);
  a.sc = sc;
  a.y = y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.group_chunks = group / 32;
  a.groups_per_row = (int)(K / group);
  a.y_f32 = y_f32;
  if (pair) {
    a.pk2 = reinterpret_cast<const uint32_t*>(pair->pk_up);
    a.sc2 = pair->sc_up;
    a.pair_f = (int)pair->F;
    a.bf16_dots = pair->bf16_dots;
  }
  if (mr) {
    a.steps = (int)(K / w4k::GSTEP);
    return gemv_fast_launch(a, nterms, mr, p, p.tiles, group == 32, st);
  }
  if (pair) return hipErrorInvalidValue;
  a.steps = (int)((K + w4k::GSTEP - 1) / w4k::GSTEP);
  const int waves = w4l_gemv_waves(N, K);
  const size_t lds = (size_t)nterms * M * K * 2 + (size_t)waves * 4 * 16 * 4;
  const dim3 grid((unsigned)((N + 15) / 16)), block(64 * waves);
  const bool kfull = (K % w4k::GSTEP) == 0, g32 = group == 32;
#define W4_GEMV(NT_, KF_, G_) \
  hipLaunchKernelGGL((w4k::gemv_kernel<NT_, KF_, G_>), grid, block, lds, st, a)
  if (nterms == 1) {
    if (kfull) { if (g32) W4_GEMV(1, true, true); else W4_GEMV(1, true, false); }
    else { if (g32) W4_GEMV(1, false, true); else W4_GEMV(1, false, false); }
  } else {
    if (kfull) { if (g32) W4_GEMV(3, true, true); else W4_GEMV(3, true, false); }
    else { if (g32) W4_GEMV(3, false, true); else W4_GEMV(3, false, false); }
  }
#undef W4_GEMV
  return hipGetLastError();
}

W4Plan w4l_plan(int64_t M, int64_t N, int64_t K, int nterms) {
  W4Plan p{};
  const int64_t mtiles = (M + 15) / 16;
  p.mt = (int)(mtiles < 4 ? mtiles : 4);
  if (p.mt < 1) p.mt = 1;
  p.grid_m = (int)((M + 16 * p.mt - 1) / (16 * p.mt));
  p.grid_n = (int)((N + 15) / 16);
  const int64_t steps = (K + w4k::KSTEP - 1) / w4k::KSTEP;
  const int64_t wgs = (int64_t)p.grid_n * p.grid_m;
  const int maxw = W4_MAXT(p.mt, nterms) / 64;
  int64_t waves = (4096 + wgs - 1) / wgs;  // aim at ~4 waves per SIMD on 256 CUs
  if (waves > maxw) waves = maxw;
  if (waves > steps) waves = steps;
  if (waves < 1) waves = 1;
  p.waves = (int)waves;
  return p;
}

static hipError_t splitk_finalize_launch(const float* part, int kq, int64_t M, int64_t Nv, void* y, int y_f32,
                                         const W4Pair* pair, hipStream_t st);

bool w4l_skinny_ok(int64_t M, int64_t K, int nterms) {
  return nterms == 1 && M > 4 && K % 256 == 0;
}

hipError_t w4l_skinny(const uint16_t* x, const int32_t* pk, const uint16_t* sc, void* y, int y_f32,
                      int64_t M, int64_t N, int64_t K, int32_t group, hipStream_t st, const W4Pair* pair, int kq,
                      float* part) {
  if (kq < 1 || (K / 256) % kq != 0 || (kq > 1 && !part)) return hipErrorInvalidValue;
  w4k::SkinnyArgs a{};
  if (pair) {
    N = 16 * ((pair->F + 7) / 8);
    a.pk2 = reinterpret_cast<const uint32_t*>(pair->pk_up);
    a.sc2 = pair->sc_up;
    a.pair_f = (int)pair->F;
    a.bf16_dots = pair->bf16_dots;
  }
  a.x = x;
  a.pk = reinterpret_cast<const uint32_t*>(pk);
  a.sc = sc;
  a.y = y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.group_chunks = group / 32;
  a.groups_per_row = (int)(K / group);
  a.y_f32 = y_f32;
  a.nk = (int)(K / 256 / kq);
  a.kq = kq;
  a.part = part;
  const int mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
  // Eight waves (128 W rows) per workgroup when that still gives >= 240
  // workgroups: x is then re-read from L2 half as often (12B gate/up, M = 64:
  // 36.6 -> 30.7 us; M = 16 / 32: 22.0 / 26.6 -> 19.8 / 23.1).  Smaller N keeps
  // four waves so the grid still fills the GPU.
  const int nw = ((N + 127) / 128) * ((M + 16 * mt - 1) / (16 * mt)) * kq >= 240 ? 8 : 4;
  const dim3 grid((unsigned)((N + 16 * nw - 1) / (16 * nw)), (unsigned)((M + 16 * mt - 1) / (16 * mt)),
                  (unsigned)kq),
      block(64 * nw);
  const bool g32 = group == 32;
#define W4_SK(MT_, NW_)                                                                               \
  do {                                                                                                \
    if (g32) hipLaunchKernelGGL((w4k::skinny_kernel<MT_, true, NW_>), grid, block, 0, st, a);        \
    else hipLaunchKernelGGL((w4k::skinny_kernel<MT_, false, NW_>), grid, block, 0, st, a);           \
  } while (0)
#define W4_SK_N(MT_)       \
  do {                     \
    if (nw == 8) W4_SK(MT_, 8); \
    else W4_SK(MT_, 4);    \
  } while (0)
  if (mt == 1) W4_SK_N(1);
  else if (mt == 2) W4_SK_N(2);
  else W4_SK_N(4);
#undef W4_SK_N
#undef W4_SK
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || kq == 1) return e;
  return splitk_finalize_launch(part, kq, M, N, y, y_f32, pair, st);
}

bool w4l_prefill_ok(int64_t M, int64_t K, int nterms) {
  return nterms == 1 && M > 64 && K % 64 == 0;
}

// Launch of prefill_lds_kernel for filled PrefillArgs (mblk in 256-row x blocks,
// ns steps per K part, kq parts): 128 * tn W rows per workgroup.
static hipError_t prefill_lds_launch(const w4k::PrefillArgs& a, int tn, bool g32, hipStream_t st) {
  const int bn = 128 * tn;
  const size_t lds = (size_t)(2 * 256 + 2 * bn) * 72 * 2;
  const dim3 grid((unsigned)((((int64_t)a.N + bn - 1) / bn) * a.mblk * a.kq)), block(512);
  auto k = tn == 2 ? (g32 ? w4k::prefill_lds_kernel<true, 2> : w4k::prefill_lds_kernel<false, 2>)
                   : (g32 ? w4k::prefill_lds_kernel<true, 1> : w4k::prefill_lds_kernel<false, 1>);
  hipError_t e = allow_big_lds(k, lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k, grid, block, lds, st, a);
  return hipGetLastError();
}

hipError_t w4l_prefill(const uint16_t* x, const int32_t* pk, const uint16_t* sc, void* y, int y_f32,
                       int64_t M, int64_t N, int64_t K, int32_t group, hipStream_t st, const W4Pair* pair) {
  w4k::PrefillArgs a{};
  if (pair) {
    N = 16 * ((pair->F + 7) / 8);
    a.pk2 = reinterpret_cast<const uint32_t*>(pair->pk_up);
    a.sc2 = pair->sc_up;
    a.pair_f = (int)pair->F;
    a.bf16_dots = pair->bf16_dots;
  }
  a.x = x;
  a.pk = reinterpret_cast<const uint32_t*>(pk);
  a.sc = sc;
  a.y = y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.group_chunks = group / 32;
  a.groups_per_row = (int)(K / group);
  a.y_f32 = y_f32;
  a.ns = (int)(K / 64);
  a.kq = 1;
  // x rows per workgroup: 128 / 256 (MB = 4 / 8 blocks of 32; M > 64 here), the
  // smallest that holds M, so M <= 128 pays no MFMAs on padding rows
  if (M <= 64) return hipErrorInvalidValue;
  const int mb = M <= 128 ? 4 : 8;
  a.mblk = (int)((M + 32 * mb - 1) / (32 * mb));
  // W expanded into LDS, 8 waves (two per SIMD): 256 x 256 tiles when they still
  // give >= 240 workgroups, else 256 x 128.  Measured on the 12B / E2B shapes, us,
  // against the one-wave-per-SIMD kernel below: 256 x 256 gate/up at M = 512 /
  // 1024 / 2048 / 4096 167 / 327 / 536 / 1066 -> 133 / 257 / 510 / 1019, down at
  // M = 4096 569 -> 457; 256 x 128 down at M = 1024 / 2048 287 / 293 -> 249 / 279,
  // full-layer o 163 -> 152, E2B down 124 -> 105 (the 256 x 256 tile gives those
  // 60-120 workgroups and took 224-416).
  const int lds_tn = ((N + 255) / 256) * a.mblk >= 240 ? 2 : 1;
  if (mb == 8) return prefill_lds_launch(a, lds_tn, group == 32, st);
  // 64 < M <= 128: the one-wave kernel over 128-row x tiles
  const int bn = 128;
  const dim3 grid((unsigned)(((N + bn - 1) / bn) * a.mblk)), block(256);
  const bool g32 = group == 32;
#define W4_PF(TN_, P_, MB_)                                                                         \
  do {                                                                                              \
    if (g32) hipLaunchKernelGGL((w4k::prefill_kernel<TN_, P_, true, MB_>), grid, block, 0, st, a);  \
    else hipLaunchKernelGGL((w4k::prefill_kernel<TN_, P_, false, MB_>), grid, block, 0, st, a);     \
  } while (0)
  W4_PF(1, 4, 4);
#undef W4_PF
  return hipGetLastError();
}

// Upper bound of the rows above 64 that the skinny kernel takes in several
// 64-row x blocks.
static int64_t skinny_mid_max() { return 256; }

// Split-K plan (bf16 x) for the shapes whose one-pass grid cannot fill the GPU.
// Above M = 64: the skinny form up to M = 128 when K % 256 == 0, and up to 256
// when also K <= 8192 (else one pass); the LDS prefill form beyond (comments in
// the branch).  Up to M = 64, N < 16384:
//  - M <= 4 when x is too large for the decode GEMV's LDS (12B down at M = 3..4:
//    21.3 -> 15.5 us), skinny form only;
//  - 4 < M <= 16 when the 16-row GEMV does not take the shape (it is faster
//    where it does: 12B q/k/v/o, E2B rows at M = 8 / 16) and K >= 8192 or
//    N < 8192, i.e. the one-pass skinny grid (N / 64 workgroups) is under half
//    the CUs (E2B down at M = 16: 16.7 -> 9.9 us; 12B full-layer q, N = 8192,
//    stays one-pass);
//  - 16 < M <= 64.
// Two forms:
//  - skinny (K % 256 == 0): the skinny kernel over kq parts of K, kq the largest
//    divisor of K / 256 (<= 64) that keeps ceil(N / 64) * (x blocks) * kq <= 256
//    workgroups (one per CU).  Measured on the 12B shapes, us: down M = 8 / 16 /
//    32 / 64 23.2 / 23.7 / 23.8 / 27.5 -> 15.5 / 15.9 / 18.5 / 25.3; q, o, k/v at
//    M = 32 15.4, 12.6, 12.7 -> 10.2, 10.3, 9.6 and at M = 64 20.2, 21.6, 17.3 ->
//    13.4, 13.3, 11.4 (each against the prefill form).
//  - prefill (K % 256 != 0, M > 4): workgroups of WS waves x 32 W rows (256 rows for
//    M > 32, 128 for M <= 32; x blocks of 64 / 32 rows) and kq parts, the
//    smallest divisor of K / 64 (<= 16) that gives >= 240 workgroups, else the
//    largest.
// Both cost kq f32 partial planes and one finalize pass.  The plan, and so the
// workspace size, is a function of (M, N, K) only.
namespace {
enum SplitForm { SPLIT_SKINNY, SPLIT_PF32, SPLIT_LDS };
struct SplitPlan {
  SplitForm form;
  int kq;
  int ws, mb;  // 32x32 form
};
bool splitk_plan(int64_t M, int64_t N, int64_t K, int nterms, SplitPlan* p) {
  if (nterms != 1 || M < 1 || K % 64 != 0 || N <= 0) return false;
  if (M > 64) {
    // 64 < M <= 128: the skinny kernel in two 64-row x blocks over K parts (one
    // workgroup per CU at most), else one pass; faster than the LDS form on every
    // row measured (M = 65: 12B down 42.4 -> 40.7 us, E2B down 27.2 -> 20.9,
    // K = 3840 / N = 1024: 14.7 -> 10.3; where no part count fits, the one-pass
    // skinny kernel: N = 8192, 28.7 -> 21.3)
    // 128 < M <= 256 (three or four x blocks) only for K <= 8192: 3840 -> 1024 /
    // 4096 at M = 160 17.8 / 26.1 -> 11.2 / 21.4 us, E2B down 23.7 -> 17.0, but
    // 12B down 48.8 against 72.5 and the E2B model projection (K = 15360) 30.8
    // against 41.6 at M = 256, where the LDS form splits K into more parts
    const bool sk = K % 256 == 0 && M <= skinny_mid_max() && (M <= 128 || K <= 8192);
    if (sk) {
      const int64_t nk = K / 256;
      const int64_t per_part = ((N + 63) / 64) * ((M + 63) / 64);
      int q = 0;
      for (int c = 2; c <= nk && c <= 64; ++c)
        if (nk % c == 0 && per_part * c <= 256) q = c;
      if (q < 2) return false;
      *p = SplitPlan{SPLIT_SKINNY, q, 0, 0};
      return true;
    }
    // the other rows: prefill_lds_kernel with 256 x 128 tiles over kq K
    // parts when its one-pass grid is under 240 workgroups (N <= 8192 at M <= 128):
    // the largest divisor of K / 64 (<= 16) that keeps the grid within 256
    // workgroups, one per CU (its LDS holds one workgroup per CU: q at M = 128 took
    // 24.6 us with 192 workgroups against 31.9 with 320)
    const int64_t grid = ((N + 127) / 128) * ((M + 255) / 256);
    if (grid >= 240) return false;
    // up to 128 rows the one-pass kernel's 128-row x tiles waste no MFMAs, and with
    // 96 workgroups it stays ahead (E2B gate/up rows at M = 128: 24.0 against 36.9;
    // with 64, full-layer q, the split wins: 32.3 against 49.8)
    if (M <= 128 && N > 8192) return false;
    const int64_t steps = K / 64;
    int q = 0;
    for (int c = 16; !q && c >= 2; --c)
      if (steps % c == 0 && grid * c <= 256) q = c;
    if (q < 2) return false;
    *p = SplitPlan{SPLIT_LDS, q, 0, 0};
    return true;
  }
  if (N >= 16384) return false;
  if (M <= 4 && (w4l_gemv_ok(M, K, nterms) || K % 256 != 0)) return false;
  if (M > 4 && M <= 16 && (w4l_gemv16_ok(M, N, K, nterms) || (K < 8192 && N >= 8192))) return false;
  if (K % 256 == 0) {
    const int64_t nk = K / 256;
    const int64_t mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
    const int64_t per_part = ((N + 63) / 64) * ((M + 16 * mt - 1) / (16 * mt));
    int q = 0;
    for (int c = 2; c <= nk && c <= 64; ++c)
      if (nk % c == 0 && per_part * c <= 256) q = c;
    if (q >= 2) {
      *p = SplitPlan{SPLIT_SKINNY, q, 0, 0};
      return true;
    }
    // no part count within 256 workgroups: the one-pass grid already has > 128,
    // and the 32x32 form below is slower there (E2B gate/up rows at M = 17 / 32 /
    // 64: 14.2 / 15.6 / 24.4 us against 8.0 / 8.4 / 11.8 one-pass)
    return false;
  }
  const int mb = M <= 32 ? 1 : 2;
  const int ws = mb == 2 ? 8 : 4;
  const int64_t tiles = (N + 32 * ws - 1) / (32 * ws);
  const int64_t steps = K / 64;
  int q = 0;
  for (int c = 2; !q && c <= 16; ++c)
    if (steps % c == 0 && tiles * c >= 240) q = c;
  if (!q) {
    for (int c = 16; c >= 2 && !q; --c)
      if (steps % c == 0) q = c;
  }
  if (q < 2 || M <= 4) return false;
  *p = SplitPlan{SPLIT_PF32, q, ws, mb};
  return true;
}
}  // namespace

// Sum of the kq partial planes part[kq][M][Nv] into y (gate/up: gelu(g) * u).
static hipError_t splitk_finalize_launch(const float* part, int kq, int64_t M, int64_t Nv, void* y, int y_f32,
                                         const W4Pair* pair, hipStream_t st) {
  const int64_t cols = pair ? pair->F : Nv;
  const int64_t outs = (cols % 4 == 0 && Nv % 4 == 0) ? M * cols / 4 : M * cols;  // threads (4 outputs each when aligned)
  const int block_f = 256;
  hipLaunchKernelGGL(w4k::splitk_finalize_kernel, dim3(grid_for(outs, block_f)), dim3(block_f), 0, st, part, kq,
                     (int)M, (int)Nv, y, y_f32, pair ? (int)pair->F : 0, pair ? pair->bf16_dots : 0);
  return hipGetLastError();
}

hipError_t w4l_add_planes(const float* y3, int64_t M, int64_t N, void* y, int y_f32, hipStream_t st) {
  return splitk_finalize_launch(y3, 3, M, N, y, y_f32, nullptr, st);
}

size_t w4l_splitk_bytes(int64_t M, int64_t N, int64_t K, int nterms) {
  SplitPlan p;
  if (!splitk_plan(M, N, K, nterms, &p)) return 0;
  return (size_t)p.kq * (size_t)M * (size_t)N * sizeof(float);
}

hipError_t w4l_splitk(const uint16_t* x, const int32_t* pk, const uint16_t* sc, void* y, int y_f32, int64_t M,
                      int64_t N, int64_t K, int32_t group, hipStream_t st, const W4Pair* pair, float* part) {
  const int64_t Nv = pair ? 16 * ((pair->F + 7) / 8) : N;
  SplitPlan p;
  if (!splitk_plan(M, Nv, K, 1, &p)) return hipErrorInvalidValue;
  if (p.form == SPLIT_SKINNY) return w4l_skinny(x, pk, sc, y, y_f32, M, N, K, group, st, pair, p.kq, part);
  const int kq = p.kq, ws = p.ws, mb = p.mb;
  w4k::PrefillArgs a{};
  if (pair) {
    a.pk2 = reinterpret_cast<const uint32_t*>(pair->pk_up);
    a.sc2 = pair->sc_up;
    a.pair_f = (int)pair->F;
    a.bf16_dots = pair->bf16_dots;
  }
  a.x = x;
  a.pk = reinterpret_cast<const uint32_t*>(pk);
  a.sc = sc;
  a.y = y;
  a.M = (int)M;
  a.N = (int)Nv;
  a.K = (int)K;
  a.group_chunks = group / 32;
  a.groups_per_row = (int)(K / group);
  a.y_f32 = y_f32;
  a.ns = (int)(K / 64 / kq);
  a.kq = kq;
  a.part = part;
  if (p.form == SPLIT_LDS) {
    a.mblk = (int)((M + 255) / 256);
    hipError_t e = prefill_lds_launch(a, 1, group == 32, st);
    if (e != hipSuccess) return e;
    return splitk_finalize_launch(part, kq, M, Nv, y, y_f32, pair, st);
  }
  a.mblk = (int)((M + 32 * mb - 1) / (32 * mb));
  const int bn = 32 * ws;
  const dim3 grid((unsigned)(((Nv + bn - 1) / bn) * a.mblk * kq)), block(64 * ws);
  const bool g32 = group == 32;
#define W4_SKQ(MB_, WS_)                                                                                   \
  do {                                                                                                     \
    if (g32) hipLaunchKernelGGL((w4k::prefill_kernel<1, 4, true, MB_, WS_, 1>), grid, block, 0, st, a);   \
    else hipLaunchKernelGGL((w4k::prefill_kernel<1, 4, false, MB_, WS_, 1>), grid, block, 0, st, a);      \
  } while (0)
  if (mb == 2) W4_SKQ(2, 8);
  else W4_SKQ(1, 4);
#undef W4_SKQ
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  return splitk_finalize_launch(part, kq, M, Nv, y, y_f32, pair, st);
}

// 64 < M <= 256 where the prefill kernel's 128-wide tiles give fewer than 240
// workgroups: the skinny kernel in two to four 64-row x blocks (the later ones
// read W mostly from the MALL), 2.2-2.4x faster one-pass up to M = 128 (12B down
// at M = 65: 168 -> 71 us, q: 47 -> 21, E2B gate/up: 21 -> 16) and ahead of the
// LDS kernel's 256-row tiles above (E2B gate/up at M = 160 / 256: 30.4 / 32.6 ->
// 26.0 / 27.3).  The 12B gate/up pair (240 tiles) stays on the prefill kernels
// (48 against 55 us at M = 65, a tie at 160-256).
static bool skinny_mid(int64_t M, int64_t N, int64_t K, int nterms) {
  return M > 64 && M <= skinny_mid_max() && (N + 127) / 128 < 240 && w4l_skinny_ok(M, K, nterms);
}

hipError_t w4l_linear(const uint16_t* x_planes, int nterms, const int32_t* pk, const uint16_t* sc,
                      void* y, int y_f32, int64_t M, int64_t N, int64_t K, int32_t group,
                      hipStream_t st) {
  if (w4l_gemv_fast_ok(M, N, K, nterms)) return w4l_gemv(x_planes, nterms, pk, sc, y, y_f32, M, N, K, group, st);
  if (w4l_gemv16_ok(M, N, K, nterms)) return w4l_gemv(x_planes, nterms, pk, sc, y, y_f32, M, N, K, group, st);
  // M <= 4 beyond both GEMV plans (12B gate/up rows at M = 4): the skinny kernel,
  // 23.5 -> 19 us against the generic GEMV below
  if (M <= 4 && nterms == 1 && K % 256 == 0) return w4l_skinny(x_planes, pk, sc, y, y_f32, M, N, K, group, st);
  if (w4l_gemv_ok(M, K, nterms)) return w4l_gemv(x_planes, nterms, pk, sc, y, y_f32, M, N, K, group, st);
  if (skinny_mid(M, N, K, nterms)) return w4l_skinny(x_planes, pk, sc, y, y_f32, M, N, K, group, st);
  if (w4l_prefill_ok(M, K, nterms)) return w4l_prefill(x_planes, pk, sc, y, y_f32, M, N, K, group, st);
  if (w4l_skinny_ok(M, K, nterms)) return w4l_skinny(x_planes, pk, sc, y, y_f32, M, N, K, group, st);
  const W4Plan p = w4l_plan(M, N, K, nterms);
  w4k::LinearArgs a{};
  a.x = x_planes;
  a.pk = reinterpret_cast<const uint32_t*>(pk);
  a.sc = sc;
  a.y = y;
  a.M = (int)M;
  a.N = (int)N;
  a.K = (int)K;
  a.group_chunks = group / 32;
  a.groups_per_row = (int)(K / group);
  a.y_f32 = y_f32;
  a.x_plane = M * K;
  const dim3 grid(p.grid_n, p.grid_m);
  const dim3 block(64 * p.waves);
  const size_t lds = p.waves > 1 ? (size_t)p.waves * p.mt * 4 * 64 * sizeof(float) : 0;
#define W4_LAUNCH(MT_, NT_) \
  hipLaunchKernelGGL((w4k::linear_kernel<MT_, NT_, W4_MAXT(MT_, NT_)>), grid, block, lds, st, a)
  if (nterms == 1) {
    switch (p.mt) {
      case 1: W4_LAUNCH(1, 1); break;
      case 2: W4_LAUNCH(2, 1); break;
      case 3: W4_LAUNCH(3, 1); break;
      default: W4_LAUNCH(4, 1); break;
    }
  } else {
    switch (p.mt) {
      case 1: W4_LAUNCH(1, 3); break;
      case 2: W4_LAUNCH(2, 3); break;
      case 3: W4_LAUNCH(3, 3); break;
      default: W4_LAUNCH(4, 3); break;
    }
  }
#undef W4_LAUNCH
  return hipGetLastError();
}

namespace {
enum PairRoute { PAIR_NONE, PAIR_GEMV, PAIR_PREFILL, PAIR_SKINNY };

// Kernel of the fused gate/up launch, in the order of w4l_linear; the skinny
// kernel also takes decode shapes the straight-line GEMV plan cannot hold (its
// x rows past M repeat row M - 1 and are not stored).
PairRoute pair_route(int64_t M, int64_t F, int64_t K, int nterms) {
  if (w4l_gemv_fast_ok(M, 16 * ((F + 7) / 8), K, nterms)) return PAIR_GEMV;
  if (w4l_gemv16_ok(M, 16 * ((F + 7) / 8), K, nterms)) return PAIR_GEMV;
  if (skinny_mid(M, 16 * ((F + 7) / 8), K, nterms)) return PAIR_SKINNY;
  if (w4l_prefill_ok(M, K, nterms)) return PAIR_PREFILL;
  if (nterms == 1 && K % 256 == 0) return PAIR_SKINNY;
  return PAIR_NONE;
}
}  // namespace

bool w4l_gate_up_fused(int64_t M, int64_t F, int64_t K, int nterms) {
  return pair_route(M, F, K, nterms) != PAIR_NONE;
}

hipError_t w4l_gate_up(const uint16_t* x_planes, int nterms, const int32_t* pk_gate, const uint16_t* sc_gate,
                       const W4Pair& pair, void* h, int h_f32, int64_t M, int64_t K, int32_t group,
                       hipStream_t st) {
  switch (pair_route(M, pair.F, K, nterms)) {
    case PAIR_GEMV: return w4l_gemv(x_planes, nterms, pk_gate, sc_gate, h, h_f32, M, 0, K, group, st, &pair);
    case PAIR_PREFILL: return w4l_prefill(x_planes, pk_gate, sc_gate, h, h_f32, M, 0, K, group, st, &pair);
    case PAIR_SKINNY: return w4l_skinny(x_planes, pk_gate, sc_gate, h, h_f32, M, 0, K, group, st, &pair);
    default: return hipErrorInvalidValue;
  }
}

hipError_t w4l_gelu_mul(const float* g, const float* u, void* h, int h_f32, int bf16_dots, int64_t n,
                        hipStream_t st) {
  const int block = 256;
  hipLaunchKernelGGL(w4k::gelu_mul_kernel, dim3(grid_for(n, block)), dim3(block), 0, st, g, u, h, h_f32, bf16_dots,
                     n);
  return hipGetLastError();
}

// The plan every member of a weight group gets from w4l_linear on its own, when they all
// run the straight-line GEMV with the same plan: one launch then gives each y_j exactly
// the single call's result (same tiles per row, same runs of steps, same summation
// order).  Returns the epilogue rows (0: no common plan, so one launch per member).
static int group_common_plan(int64_t M, int n, const int64_t* N, int64_t K, int nterms, GemvPlan* p) {
  int mr = 0;
  for (int j = 0; j < n; ++j) {
    if (!N[j]) continue;
    // w4l_linear's first two routes are the ones that reach this GEMV
    if (!w4l_gemv_fast_ok(M, N[j], K, nterms) && !w4l_gemv16_ok(M, N[j], K, nterms)) return 0;
    GemvPlan q;
    const int m = gemv_fast_plan(M, N[j], K, nterms, false, &q);
    if (!m) return 0;
    if (!mr) {
      mr = m;
      *p = q;
    } else if (m != mr || q.s != p->s || q.waves != p->waves || q.nst != p->nst || q.xpt != p->xpt || q.xw != p->xw) {
      return 0;
    }
  }
  return mr;
}

bool w4l_group_fused(int64_t M, int n, const int64_t* N, int64_t K, int nterms) {
  int64_t ntot = 0;
  for (int j = 0; j < n; ++j) ntot += 16 * ((N[j] + 15) / 16);
  const bool fits = (M <= 4 && w4l_gemv_fast_ok(M, ntot, K, nterms)) || w4l_gemv16_ok(M, ntot, K, nterms);
  GemvPlan p;
  return fits && group_common_plan(M, n, N, K, nterms, &p) != 0;
}

bool w4l_group_f32x_ok(int64_t M, int n, const int64_t* N, int64_t K, int32_t group) {
  GemvPlan p;
  int64_t ntot = 0;
  for (int j = 0; j < n; ++j) ntot += N[j];
  return group == 32 && !f32x_wide(M, ntot, K) && w4l_group_fused(M, n, N, K, 3) &&
         group_common_plan(M, n, N, K, 3, &p) == 4 && f32x_plan_ok(p, M);
}

hipError_t w4l_gemv_group(const uint16_t* x_planes, int nterms, int n, const int32_t* const* pk,
                          const uint16_t* const* sc, void* const* y, const int64_t* N, int y_f32, int64_t M, int64_t K,
                          int32_t group, hipStream_t st, const float* xf) {
  if (n < 1 || n > 4) return hipErrorInvalidValue;
  if (xf) nterms = 3;
  GemvPlan p;
  const int mr = group_common_plan(M, n, N, K, nterms, &p);
  if (!mr) return hipErrorInvalidValue;
  const int R = 16 / p.s;  // W rows per tile
  w4k::GemvArgs a{};
  a.x = x_planes;
  if (xf) {
    if (!(mr == 4 && p.xw && group == 32)) return hipErrorInvalidValue;
    a.x = reinterpret_cast<const uint16_t*>(xf);
    a.xf = 1;
  }
  a.M = (int)M;
  a.K = (int)K;
  a.group_chunks = group / 32;
  a.groups_per_row = (int)(K / group);
  a.y_f32 = y_f32;
  a.steps = (int)(K / w4k::GSTEP);
  a.nmat = n;
  int64_t tiles = 0;
  for (int j = 0; j < n; ++j) {
    a.gpk[j] = reinterpret_cast<const uint32_t*>(pk[j]);
    a.gsc[j] = sc[j];
    a.gy[j] = y[j];
    a.gN[j] = (int)N[j];
    a.tile0[j] = (int)tiles;
    tiles += (N[j] + R - 1) / R;
  }
  // a matrix with N = 0 owns no tiles; the single-matrix fields stay those of matrix 0
  a.pk = a.gpk[0];
  a.sc = a.gsc[0];
  a.y = a.gy[0];
  a.N = a.gN[0];
  if (tiles == 0) return hipSuccess;
  return gemv_fast_launch(a, nterms, mr, p, (int)tiles, group == 32, st);
}
