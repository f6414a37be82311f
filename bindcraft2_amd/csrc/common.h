// Shared device/host helpers for the gfx950 (CDNA4) trunk kernels.
//
// Everything here is written for wave64 and the gfx950 MFMA set; there is no
// other target.  IEEE binary16 (h16) is the storage type of every MFMA
// operand, f32 the type of every accumulation, residual carry, softmax
// statistic and of the one product without a range bound (the triangle
// multiplication's contraction output).
//
// Why binary16 and not bf16: the trunk's MFMA operands are either bounded by
// construction (LayerNorm outputs, projections of them, softmax
// probabilities, sigmoid gates, weights) or backward cotangents, which every
// module multiplies by a power-of-two scale s (s * max|cotangent| in (8, 16],
// ct_scale in kernels.h) before they are rounded and divides out in the f32
// epilogue that ends the module.  So the 5 exponent bits suffice, and the 3
// extra significand bits make each rounding 8x finer at the same MFMA rate
// and conversion cost (v_cvt_pk_f16_f32).  Over a 48-block stack the bf16
// roundings compound to a few percent of the input gradient in L2.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

namespace bc2n {

typedef _Float16 h16;
typedef _Float16 h16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 h16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float LN_EPS = 1e-5f;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
// AF2's attention clip (accel.py LOGIT_CLIP) and mask bias magnitude.
constexpr float LOGIT_CLIP = 1e8f;
constexpr float MASK_BIAS = 1e9f;

__device__ __forceinline__ float h2f(h16 v) { return (float)v; }
__device__ __forceinline__ h16 f2h(float v) { return (h16)v; }
// Round to binary16, saturating at the largest finite value instead of going
// to infinity: for backward tensors, where an exact-model value that is huge
// but finite (the LayerNorm backward of an all-zero masked row) is later
// multiplied by a zero mask; inf * 0 would be NaN, 65504 * 0 is 0.
__device__ __forceinline__ h16 f2h_sat(float v) {
  return (h16)__builtin_amdgcn_fmed3f(v, -65504.f, 65504.f);
}

// 1/(1+e^-x) with the hardware reciprocal (v_rcp_f32, 1 ulp) instead of an
// IEEE division: the results feed binary16 operands or f32 sums far coarser than
// that.  exp(-x) = 2^(-x log2 e).
__device__ __forceinline__ float sigmoidf_(float x) {
  return __builtin_amdgcn_rcpf(1.f + __builtin_amdgcn_exp2f(-x * 1.4426950408889634f));
}

// Workgroups are handed to the 8 XCDs round-robin (workgroup b runs on XCD
// b % 8) and every XCD has its own L2.  A kernel launched on xcd_grid(G)
// workgroups that takes its logical index from xcd_block(G) gives each XCD
// one contiguous range of the logical order, so workgroups that share
// operands (neighbours in that order) share an L2.  Indices >= G are padding
// and must exit before any barrier.
constexpr int NUM_XCD = 8;
__host__ __device__ inline long xcd_per(long G) { return (G + NUM_XCD - 1) / NUM_XCD; }
inline unsigned xcd_grid(long G) { return (unsigned)(xcd_per(G) * NUM_XCD); }
__device__ __forceinline__ long xcd_block(long G) {
  const long b = blockIdx.x;
  return (b % NUM_XCD) * xcd_per(G) + b / NUM_XCD;
}

// D += A(16x32) * B(32x16), binary16 operands, f32 accumulation.
// Lane l: A row l%16, B column l%16, 8 K-slots per lane; D lane l holds
// column l%16, rows 4*(l/16)+r.  The K-slot -> k mapping is the same for A
// and B, so any bijection of the 32 k values over (lane group, element) that
// is applied identically to both operands yields the exact product.
__device__ __forceinline__ f32x4 mfma16x16x32(h16x8 a, h16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// DPP lane moves (gfx9 encodings): a VALU operand read from another lane of
// the same 16-lane row, no LDS round trip.
constexpr int DPP_QUAD_1032 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_2301 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// Reductions over aligned groups of W lanes (every lane of the group gets the
// result).  Within a 16-lane row they are DPP steps: pairs, quads, the
// half-row mirror (lane i <-> 7-i) and the row mirror (i <-> 15-i), each of
// which pairs a partial with the complementary one; beyond 16 lanes, xor
// shuffles.  Groups must be wholly active or wholly inactive.
template <int W, class Op>
__device__ __forceinline__ float group_reduce(float v, Op op) {
  static_assert(W >= 1 && W <= 64 && (W & (W - 1)) == 0, "W: power of two <= 64");
  if constexpr (W >= 2) v = op(v, dpp_mov<DPP_QUAD_1032>(v));
  if constexpr (W >= 4) v = op(v, dpp_mov<DPP_QUAD_2301>(v));
  if constexpr (W >= 8) v = op(v, dpp_mov<DPP_ROW_HALF_MIRROR>(v));
  if constexpr (W >= 16) v = op(v, dpp_mov<DPP_ROW_MIRROR>(v));
  if constexpr (W >= 32) v = op(v, __shfl_xor(v, 16, 64));
  if constexpr (W >= 64) v = op(v, __shfl_xor(v, 32, 64));
  return v;
}
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  return group_reduce<W>(v, [](float a, float b) { return a + b; });
}
template <int W>
__device__ __forceinline__ float group_max(float v) {
  return group_reduce<W>(v, [](float a, float b) { return fmaxf(a, b); });
}

// Row of an N x N grid read in transposed order: row m of the transposed
// view is row (m % nt) * nt + m / nt of the stored one (nt <= 0: identity).
__device__ __forceinline__ long ln_src_row(long m, int nt) {
  if (nt <= 0) return m;
  const long p = m / nt, q = m % nt;
  return q * nt + p;
}

// 16-byte vector load/store of 8 binary16 values.
__device__ __forceinline__ h16x8 ld8(const h16* p) {
  return *reinterpret_cast<const h16x8*>(p);
}
__device__ __forceinline__ void st8(h16* p, h16x8 v) {
  *reinterpret_cast<h16x8*>(p) = v;
}

// ---------------------------------------------------------------------------
// JAX threefry2x32-20 (Salmon et al. 2011, Random123), the block cipher under
// jax.random; used for dropout masks that equal jax.random.bernoulli's.
__host__ __device__ __forceinline__ uint32_t rotl32(uint32_t v, int d) {
  return (v << d) | (v >> (32 - d));
}

__host__ __device__ __forceinline__ void threefry2x32(uint32_t k0, uint32_t k1,
                                                      uint32_t& x0,
                                                      uint32_t& x1) {
  const uint32_t k2 = k0 ^ k1 ^ 0x1BD11BDAu;
  const uint32_t ks[3] = {k0, k1, k2};
  x0 += k0;
  x1 += k1;
#pragma unroll
  for (int g = 0; g < 5; ++g) {
    const int r0 = (g & 1) ? 17 : 13, r1 = (g & 1) ? 29 : 15;
    const int r2 = (g & 1) ? 16 : 26, r3 = (g & 1) ? 24 : 6;
    x0 += x1; x1 = rotl32(x1, r0); x1 ^= x0;
    x0 += x1; x1 = rotl32(x1, r1); x1 ^= x0;
    x0 += x1; x1 = rotl32(x1, r2); x1 ^= x0;
    x0 += x1; x1 = rotl32(x1, r3); x1 ^= x0;
    x0 += ks[(g + 1) % 3];
    x1 += ks[(g + 2) % 3] + (uint32_t)(g + 1);
  }
}

// jax.random.uniform(key, shape, float32) element `idx` (partitionable
// counters: element i is enciphered as the pair (hi32(i), lo32(i)); the two
// output words are XORed to one 32-bit draw; 23 mantissa bits make a float in
// [1,2) from which 1 is subtracted).
__host__ __device__ __forceinline__ float jax_uniform01(uint32_t k0, uint32_t k1,
                                                        uint64_t idx) {
  uint32_t x0 = (uint32_t)(idx >> 32), x1 = (uint32_t)(idx & 0xffffffffu);
  threefry2x32(k0, k1, x0, x1);
  const uint32_t bits = x0 ^ x1;
  const uint32_t fb = (bits >> 9) | 0x3F800000u;
  float f;
  __builtin_memcpy(&f, &fb, 4);
  return f - 1.0f;
}

}  // namespace bc2n
