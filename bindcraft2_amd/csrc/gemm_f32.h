// Batched, strided f32 GEMM on gfx950 MFMA (v_mfma_f32_16x16x4_f32), for the
// structure module, which AF2 runs in float32 throughout (the point and
// rigid projections ask for Precision.HIGHEST; a frame is a rotation whose
// orthogonality h16 would not keep).  Shapes there are N-sized (N <= 512
// residues, K <= 2112), so the kernel favours generality: any strides for
// A, B and C, any M/N/K, and a fused epilogue
//
//   C = ((alpha * A B + bias[n]) -> relu? ) * gate? + add? (+ beta * C)
//
// where `gate` is an elementwise multiplier in C's layout (a dropout table or
// a relu-derivative mask: gate > 0 keeps, as `gate_is_mask`), `add` an
// elementwise addend in C's layout (a residual).
//
// Tile 64x64 per workgroup of 256 threads (4 waves, 32x32 each = 2x2 MFMA
// tiles), K in steps of 16 staged through LDS as [k][m] / [k][n] so a lane's
// MFMA operand read (row l%16 at k l/16) is one conflict-free LDS word.
#pragma once
#include <algorithm>
#include <mutex>
#include <stdexcept>

#include "common.h"
#include "runtime.h"

namespace bc2n {

struct GemmF32 {
  int M = 0, N = 0, K = 0, batch = 1;
  const float* A = nullptr; long a_sm = 0, a_sk = 0, a_sb = 0;
  const float* B = nullptr; long b_sk = 0, b_sn = 0, b_sb = 0;
  float* C = nullptr; long c_sm = 0, c_sn = 0, c_sb = 0;
  const float* bias = nullptr;  // [N]
  const float* gate = nullptr;  // C layout
  const float* add = nullptr;   // C layout
  float alpha = 1.f, beta = 0.f;
  bool relu = false, gate_is_mask = false;
  // split-K (set by gemm_f32): ksplit > 1 workgroups per tile each sum one
  // K range into part[s][b][m][n]; a second kernel adds them and applies the
  // epilogue
  int ksplit = 1, kchunk = 0;
  float* part = nullptr;
};

namespace gf32 {
constexpr int BM = 64, BN = 64, BK = 32, LDS_LD = BM + 4;
}

// internal linkage: the header is included by several translation units
static __global__ __launch_bounds__(256) void gemm_f32_kernel(GemmF32 g) {
  using namespace gf32;
  __shared__ float As[BK][LDS_LD];
  __shared__ float Bs[BK][LDS_LD];
  const int tiles_n = (g.N + BN - 1) / BN;
  const int tiles = ((g.M + BM - 1) / BM) * tiles_n;
  const long G = (long)tiles * g.batch * g.ksplit;
  const long bid0 = xcd_block(G);
  if (bid0 >= G) return;
  const int ks = (int)(bid0 % g.ksplit);
  const long bid = bid0 / g.ksplit;
  const int kbeg = ks * g.kchunk, kend = g.ksplit > 1 ? min(g.K, kbeg + g.kchunk) : g.K;
  const int b = (int)(bid / tiles), t = (int)(bid % tiles);
  const int m0 = (t / tiles_n) * BM, n0 = (t % tiles_n) * BN;
  const float* A = g.A + (long)b * g.a_sb;
  const float* B = g.B + (long)b * g.b_sb;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // load mapping: the unit-stride index runs fastest across threads
  const bool a_kfast = (g.a_sk == 1), b_nfast = (g.b_sn == 1) || (g.b_sk != 1);
  f32x4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The next K step's elements are loaded into registers while the current
  // step multiplies out of LDS, so a step waits for memory only once.
  constexpr int NA = (BM * BK) / 256, NB = (BN * BK) / 256;
  float ra[NA], rb[NB];
  auto gload = [&](int k0) {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int e = tid + 256 * i;
      int m, k;
      if (a_kfast) { k = e % BK; m = e / BK; } else { m = e % BM; k = e / BM; }
      const int gm = m0 + m, gk = k0 + k;
      ra[i] = (gm < g.M && gk < kend) ? A[gm * g.a_sm + gk * g.a_sk] : 0.f;
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int e = tid + 256 * i;
      int n, k;
      if (b_nfast) { n = e % BN; k = e / BN; } else { k = e % BK; n = e / BK; }
      const int gn = n0 + n, gk = k0 + k;
      rb[i] = (gn < g.N && gk < kend) ? B[gk * g.b_sk + gn * g.b_sn] : 0.f;
    }
  };
  auto sstore = [&]() {
#pragma unroll
    for (int i = 0; i < NA; ++i) {
      const int e = tid + 256 * i;
      int m, k;
      if (a_kfast) { k = e % BK; m = e / BK; } else { m = e % BM; k = e / BM; }
      As[k][m] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
      const int e = tid + 256 * i;
      int n, k;
      if (b_nfast) { n = e % BN; k = e / BN; } else { k = e % BK; n = e / BK; }
      Bs[k][n] = rb[i];
    }
  };
  if (kbeg < kend) gload(kbeg);
  for (int k0 = kbeg; k0 < kend; k0 += BK) {
    sstore();
    __syncthreads();
    if (k0 + BK < kend) gload(k0 + BK);
#pragma unroll
    for (int kk = 0; kk < BK; kk += 4) {
      const int kr = kk + (lane >> 4);
      float av[2], bv[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) av[i] = As[kr][wm * 32 + i * 16 + (lane & 15)];
#pragma unroll
      for (int j = 0; j < 2; ++j) bv[j] = Bs[kr][wn * 32 + j * 16 + (lane & 15)];
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av[i], bv[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }

  if (g.ksplit > 1) {
    float* P = g.part + ((long)ks * g.batch + b) * g.M * g.N;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int n = n0 + wn * 32 + j * 16 + (lane & 15);
        if (n >= g.N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
          if (m < g.M) P[(long)m * g.N + n] = acc[i][j][r];
        }
      }
    return;
  }
  float* C = g.C + (long)b * g.c_sb;
  const float* gate = g.gate ? g.gate + (long)b * g.c_sb : nullptr;
  const float* add = g.add ? g.add + (long)b * g.c_sb : nullptr;
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int n = n0 + wn * 32 + j * 16 + (lane & 15);
      if (n >= g.N) continue;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int m = m0 + wm * 32 + i * 16 + 4 * (lane >> 4) + r;
        if (m >= g.M) continue;
        const long o = (long)m * g.c_sm + (long)n * g.c_sn;
        float v = g.alpha * acc[i][j][r];
        if (g.bias) v += g.bias[n];
        if (g.relu) v = fmaxf(v, 0.f);
        if (gate) v = g.gate_is_mask ? (gate[o] > 0.f ? v : 0.f) : v * gate[o];
        if (add) v += add[o];
        if (g.beta != 0.f) v += g.beta * C[o];
        C[o] = v;
      }
    }
}

// Sum of the split-K partials, then the epilogue of gemm_f32_kernel.
static __global__ __launch_bounds__(256) void gemm_f32_splitk_reduce(GemmF32 g) {
  const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long MN = (long)g.M * g.N;
  if (e >= MN * g.batch) return;
  const int b = (int)(e / MN);
  const int m = (int)((e % MN) / g.N), n = (int)(e % g.N);
  float v = 0.f;
  for (int s = 0; s < g.ksplit; ++s) v += g.part[((long)s * g.batch + b) * MN + (long)m * g.N + n];
  const long o = (long)b * g.c_sb + (long)m * g.c_sm + (long)n * g.c_sn;
  v *= g.alpha;
  if (g.bias) v += g.bias[n];
  if (g.relu) v = fmaxf(v, 0.f);
  if (g.gate) v = g.gate_is_mask ? (g.gate[o] > 0.f ? v : 0.f) : v * g.gate[o];
  if (g.add) v += g.add[o];
  if (g.beta != 0.f) v += g.beta * g.C[o];
  g.C[o] = v;
}

// Split-K partial buffer, grow-only, one per process (the arena is in use by
// the callers while they launch these GEMMs).
inline Arena& gemm_f32_scratch() {
  static Arena a;
  return a;
}

inline void gemm_f32(hipStream_t st, const GemmF32& g_in, const char* name = "gemm_f32") {
  GemmF32 g = g_in;
  if (g.M <= 0 || g.N <= 0 || g.K <= 0 || g.batch <= 0) throw std::runtime_error("gemm_f32: empty shape");
  if (!g.A || !g.B || !g.C) throw std::runtime_error("gemm_f32: missing operand");
  const long tiles = (long)((g.M + gf32::BM - 1) / gf32::BM) * ((g.N + gf32::BN - 1) / gf32::BN);
  KTimed kt(name, st);
  // Few tiles and a long K (the structure module's N-row products, e.g. the
  // IPA output projection, 224 x 384 over K = 2112, is 24 tiles): split K so
  // that about one workgroup per CU works, each over >= 128 of K.
  const long want = device_cus();
  int split = 1;
  if (tiles * g.batch < want / 2 && g.K >= 256) {
    split = (int)std::min<long>((want + tiles * g.batch - 1) / (tiles * g.batch), g.K / 128);
    split = std::max(split, 1);
  }
  if (split == 1) {
    g.ksplit = 1; g.kchunk = g.K;
    hipLaunchKernelGGL(gemm_f32_kernel, dim3(xcd_grid(tiles * g.batch)), dim3(256), 0, st, g);
    return;
  }
  const int chunk = ((g.K + split - 1) / split + gf32::BK - 1) / gf32::BK * gf32::BK;
  split = (g.K + chunk - 1) / chunk;
  Arena& ar = gemm_f32_scratch();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  const size_t elems = (size_t)split * g.batch * g.M * g.N;
  ar.reset(st, elems * 4 + 256);
  g.part = ar.take_n<float>(elems);
  g.ksplit = split; g.kchunk = chunk;
  hipLaunchKernelGGL(gemm_f32_kernel, dim3(xcd_grid(tiles * g.batch * split)), dim3(256), 0, st, g);
  const long n = (long)g.M * g.N * g.batch;
  hipLaunchKernelGGL(gemm_f32_splitk_reduce, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g);
}

// Row-major helpers: C[M,N] = A[M,K] . B[K,N] (or B^T given as [N,K]).
inline GemmF32 gemm_rows(int M, int N, int K, const float* A, const float* B, float* C,
                         bool b_transposed = false) {
  GemmF32 g;
  g.M = M; g.N = N; g.K = K;
  g.A = A; g.a_sm = K; g.a_sk = 1;
  g.B = B;
  if (b_transposed) { g.b_sk = 1; g.b_sn = K; } else { g.b_sk = N; g.b_sn = 1; }
  g.C = C; g.c_sm = N; g.c_sn = 1;
  return g;
}

}  // namespace bc2n
