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

template <int FORM>  // 0: v_mfma_f32_16x16x32_f16 (16384 FLOP), 1: _16x16x16f16 (8192)
__global__ __launch_bounds__(256) void mfma_rate_kernel(int iters, float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  h16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (h16)(0.001f * (float)((lane + e) & 7));
    b[e] = (h16)(0.002f * (float)((lane * 3 + e) & 7));
  }
  f32x4 acc[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) acc[c] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      if constexpr (FORM == 0) {
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[c], 0, 0, 0);
      } else {
        h16x4 a4 = {a[0], a[1], a[2], a[3]}, b4 = {b[4], b[5], b[6], b[7]};
        acc[c] = __builtin_amdgcn_mfma_f32_16x16x16f16(a4, b4, acc[c], 0, 0, 0);
      }
    }
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) s += acc[c][0] + acc[c][1] + acc[c][2] + acc[c][3];
  out[(long)blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace

double probe_mfma_rate(hipStream_t st, int form, int blocks, int iters, float* out) {
  if (blocks <= 0 || iters <= 0 || !out) throw std::runtime_error("mfma probe: bad arguments");
  if (form == 0)
    hipLaunchKernelGGL(mfma_rate_kernel<0>, dim3(blocks), dim3(256), 0, st, iters, out);
  else if (form == 1)
    hipLaunchKernelGGL(mfma_rate_kernel<1>, dim3(blocks), dim3(256), 0, st, iters, out);
  else
    throw std::runtime_error("mfma probe: form must be 0 (16x16x32 f16) or 1 (16x16x16 f16)");
  BC2N_HIP(hipGetLastError());
  const double per = form == 0 ? 16384.0 : 8192.0;
  return per * CH * (double)iters * 4.0 * (double)blocks;  // 4 waves a block
}

}  // namespace bc2n
