// MFMA issue-rate probe: the matrix-core ceiling the contraction kernels'
// MFMA fractions are quoted against, measured with the instruction forms the
// kernels use.  Each wave runs CH independent accumulator chains of one MFMA
// form for `iters` rounds from register operands only (no memory traffic in
// the loop), then writes one float a lane so nothing is dead code.
#include "common.h"
#include "kernels.h"
#include "runtime.h"

namespace bc2n {
namespace {

constexpr int CH = 8;  // independent chains a wave: hides the MFMA latency

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// FORM 0: v_mfma_f32_16x16x32_f16 (16384 FLOP), 1: v_mfma_f32_16x16x16_f16
// (8192), 2: v_mfma_f32_32x32x16_f16 (32768), 3: v_mfma_f32_16x16x32_bf16
// (16384).
template <int FORM>
__global__ __launch_bounds__(256) void mfma_rate_kernel(int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  h16x8 a, b;
  bf16x8 ab, bb;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (h16)(0.001f * (float)((lane + e) & 7));
    b[e] = (h16)(0.002f * (float)((lane * 3 + e) & 7));
    ab[e] = (__bf16)(0.001f * (float)((lane + e) & 7));
    bb[e] = (__bf16)(0.002f * (float)((lane * 3 + e) & 7));
  }
  constexpr int W = FORM == 2 ? 16 : 4;  // accumulator floats a lane
  typedef float accv __attribute__((ext_vector_type(W)));
  // distinct starting values, so no two chains are the same computation
  accv acc[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < W; ++e) acc[c][e] = (float)(lane * CH * W + c * W + e);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if constexpr (FORM == 0) {
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
      } else if constexpr (FORM == 1) {
        h16x4 a4 = {a[0], a[1], a[2], a[3]}, b4 = {b[4], b[5], b[6], b[7]};
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(a4, b4, acc[c], 0, 0, 0);
      } else if constexpr (FORM == 2) {
        acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, acc[c], 0, 0, 0);
      } else {
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ab, bb, acc[c], 0, 0, 0);
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c)
#pragma unroll
    for (int e = 0; e < W; ++e) s += acc[c][e];
  out[(long)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace

double probe_mfma_rate(hipStream_t st, int form, int blocks, int iters, float* out) {
  if (blocks <= 0 || iters <= 0 || !out) throw std::runtime_error("mfma probe: bad arguments");
  const dim3 g(blocks), t(256);
  switch (form) {
    case 0: hipLaunchKernelGGL(mfma_rate_kernel<0>, g, t, 0, st, iters, out); break;
    case 1: hipLaunchKernelGGL(mfma_rate_kernel<1>, g, t, 0, st, iters, out); break;
    case 2: hipLaunchKernelGGL(mfma_rate_kernel<2>, g, t, 0, st, iters, out); break;
    case 3: hipLaunchKernelGGL(mfma_rate_kernel<3>, g, t, 0, st, iters, out); break;
    default: throw std::runtime_error("mfma probe: form must be 0..3");
  }
  BC2N_HIP(hipGetLastError());
  const double per = form == 1 ? 8192.0 : form == 2 ? 32768.0 : 16384.0;
  return per * CH * (double)iters * 4.0 * (double)blocks;  // 4 waves a block
}

}  // namespace bc2n
