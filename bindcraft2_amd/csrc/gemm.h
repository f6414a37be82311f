// LDS-tiled bf16 MFMA GEMM for gfx950 with fused, caller-supplied epilogues.
//
//   C_b[m, n] = sum_k A_b[m, k] * B_b[n, k]        (f32 accumulation)
//
// A and B are each either K-contiguous (row-major [rows][K]) or
// row-contiguous (stored [K][rows]); the tile loader transposes the second
// form on its way into LDS, so the MFMA fragments are always read the same
// way.  A 256-thread workgroup (4 waves, 2x2) owns a BM x BN tile; each wave
// owns (BM/2) x (BN/2) as a grid of 16x16 MFMA tiles fed by
// v_mfma_f32_16x16x32_bf16.  K is walked in BK steps with two LDS buffers and
// a register prefetch of the next step's tile.
//
// The epilogue is called once per (batch, output row, lane column) with the
// lane's TN accumulator values, which sit 16 columns apart.  Epilogues that
// need two logically paired columns (a projection and its gate) get them in
// one call by ordering the weight rows so the pair lands 16 columns apart.
#pragma once
#include "common.h"
#include "runtime.h"
#include <stdexcept>
#include <string>

namespace bc2n {

struct GemmArgs {
  int M = 0, N = 0, K = 0, batch = 1;
  const bf16* A = nullptr;
  long a_sm = 0, a_sk = 0, a_sb = 0;  // element strides; a_sm==1 or a_sk==1
  const bf16* B = nullptr;
  long b_sn = 0, b_sk = 0, b_sb = 0;  // element strides; b_sn==1 or b_sk==1
};

template <int BM, int BN, int BK, bool AK, bool BKC, class Epi>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g, Epi epi) {
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int LDK = BK + 8;
  constexpr int A_CH = BM * BK / 8 / 256;
  constexpr int B_CH = BN * BK / 8 / 256;
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) bf16 As[2][BM * LDK];
  __shared__ __attribute__((aligned(16))) bf16 Bs[2][BN * LDK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int tiles_n = (g.N + BN - 1) / BN;
  const int m0 = (blockIdx.x / tiles_n) * BM;
  const int n0 = (blockIdx.x % tiles_n) * BN;
  const int b = blockIdx.z;
  const bf16* __restrict__ A = g.A + (long)b * g.a_sb;
  const bf16* __restrict__ B = g.B + (long)b * g.b_sb;
  const int M = g.M, N = g.N;

  bf16x8 ra[A_CH], rb[B_CH];
  const bf16x8 zero8 = {};

  auto gload = [&](int k0) {
#pragma unroll
    for (int p = 0; p < A_CH; ++p) {
      const int c = tid + 256 * p;
      if constexpr (AK) {
        const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        const int m = m0 + row;
        ra[p] = (m < M) ? ld8(A + (long)m * g.a_sm + k0 + kc) : zero8;
      } else {
        const int k = c / (BM / 8), mc = (c % (BM / 8)) * 8;
        const int m = m0 + mc;
        ra[p] = (m < M) ? ld8(A + (long)(k0 + k) * g.a_sk + m) : zero8;
      }
    }
#pragma unroll
    for (int p = 0; p < B_CH; ++p) {
      const int c = tid + 256 * p;
      if constexpr (BKC) {
        const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        const int n = n0 + row;
        rb[p] = (n < N) ? ld8(B + (long)n * g.b_sn + k0 + kc) : zero8;
      } else {
        const int k = c / (BN / 8), nc = (c % (BN / 8)) * 8;
        const int n = n0 + nc;
        rb[p] = (n < N) ? ld8(B + (long)(k0 + k) * g.b_sk + n) : zero8;
      }
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int p = 0; p < A_CH; ++p) {
      const int c = tid + 256 * p;
      if constexpr (AK) {
        const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        st8(&As[buf][row * LDK + kc], ra[p]);
      } else {
        const int k = c / (BM / 8), mc = (c % (BM / 8)) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) As[buf][(mc + e) * LDK + k] = ra[p][e];
      }
    }
#pragma unroll
    for (int p = 0; p < B_CH; ++p) {
      const int c = tid + 256 * p;
      if constexpr (BKC) {
        const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        st8(&Bs[buf][row * LDK + kc], rb[p]);
      } else {
        const int k = c / (BN / 8), nc = (c % (BN / 8)) * 8;
#pragma unroll
        for (int e = 0; e < 8; ++e) Bs[buf][(nc + e) * LDK + k] = rb[p][e];
      }
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = g.K / BK;
  gload(0);
  sstore(0);
  __syncthreads();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = ld8(&As[buf][(wm * WM + i * 16 + fr) * LDK + kk * 32 + fk]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfr[j] = ld8(&Bs[buf][(wn * WN + j * 16 + fr) * LDK + kk * 32 + fk]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j]);
    }
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  const int ncol = n0 + wn * WN + fr;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int m = m0 + wm * WM + i * 16 + (lane >> 4) * 4 + r;
      if (m >= M) continue;
      float v[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) v[j] = acc[i][j][r];
      epi.template apply<TN>(b, m, ncol, v);
    }
  }
}

inline void gemm_check(bool ok, const char* what) {
  if (!ok) throw std::runtime_error(std::string("bc2n gemm: ") + what);
}

// Launch with tile BM x BN; picks the loader form from the strides and BK
// from K.  Shapes are validated here, on the host, before any launch.
template <int BM, int BN, class Epi>
void gemm(hipStream_t st, const GemmArgs& g, const Epi& epi, const char* name = "gemm") {
  gemm_check(g.M > 0 && g.N > 0 && g.K > 0 && g.batch > 0, "empty shape");
  gemm_check(g.K % 32 == 0, "K must be a multiple of 32");
  const bool ak = (g.a_sk == 1), bk = (g.b_sk == 1);
  gemm_check(ak || g.a_sm == 1, "A needs a unit stride");
  gemm_check(bk || g.b_sn == 1, "B needs a unit stride");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  gemm_check(al16(g.A) && al16(g.B), "operands must be 16-byte aligned");
  if (ak) gemm_check(g.a_sm % 8 == 0, "A row stride must be a multiple of 8");
  else gemm_check(g.a_sk % 8 == 0 && g.M % 8 == 0, "A(T) stride/M must be multiples of 8");
  if (bk) gemm_check(g.b_sn % 8 == 0, "B row stride must be a multiple of 8");
  else gemm_check(g.b_sk % 8 == 0 && g.N % 8 == 0, "B(T) stride/N must be multiples of 8");
  gemm_check(g.batch == 1 || (g.a_sb % 8 == 0 && g.b_sb % 8 == 0), "batch strides");
  const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  dim3 grid(tiles, 1, g.batch), block(256);
  const bool k64 = (g.K % 64 == 0);
  KTimed kt(name, st);
#define BC2N_GEMM_LAUNCH(BKV, AKV, BKCV) \
  hipLaunchKernelGGL((gemm_kernel<BM, BN, BKV, AKV, BKCV, Epi>), grid, block, 0, st, g, epi)
  if (k64) {
    if (ak && bk) BC2N_GEMM_LAUNCH(64, true, true);
    else if (ak) BC2N_GEMM_LAUNCH(64, true, false);
    else if (bk) BC2N_GEMM_LAUNCH(64, false, true);
    else BC2N_GEMM_LAUNCH(64, false, false);
  } else {
    if (ak && bk) BC2N_GEMM_LAUNCH(32, true, true);
    else if (ak) BC2N_GEMM_LAUNCH(32, true, false);
    else if (bk) BC2N_GEMM_LAUNCH(32, false, true);
    else BC2N_GEMM_LAUNCH(32, false, false);
  }
#undef BC2N_GEMM_LAUNCH
}

// ---------------------------------------------------------------- epilogues

// C[b][m][n] = act(acc + bias[n]) (+= existing when ACC), OutT in {float, bf16}.
template <class OutT, bool RELU = false, bool ACC = false>
struct EpiStore {
  OutT* C;
  long ldc, sb;
  const float* bias;  // may be null
  int N;
  template <int TN>
  __device__ __forceinline__ void apply(int b, int m, int n, const float (&v)[TN]) const {
    OutT* row = C + (long)b * sb + (long)m * ldc;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int c = n + 16 * j;
      if (c >= N) continue;
      float x = v[j] + (bias ? bias[c] : 0.f);
      if (RELU) x = fmaxf(x, 0.f);
      if (ACC) x += (float)row[c];
      row[c] = (OutT)x;
    }
  }
};

// Transposed store: C[b][n][m] (channel-major planes), bf16 or f32.
template <class OutT>
struct EpiStoreT {
  OutT* C;
  long ldc, sb;  // plane stride (per n) and batch stride
  int N;
  template <int TN>
  __device__ __forceinline__ void apply(int b, int m, int n, const float (&v)[TN]) const {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int c = n + 16 * j;
      if (c >= N) continue;
      C[(long)b * sb + (long)c * ldc + m] = (OutT)v[j];
    }
  }
};

// dH = acc * (H > 0): backward through a ReLU whose output H is kept (bf16).
struct EpiReluMask {
  bf16* C;
  const bf16* H;
  long ldc;
  int N;
  template <int TN>
  __device__ __forceinline__ void apply(int, int m, int n, const float (&v)[TN]) const {
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int c = n + 16 * j;
      if (c >= N) continue;
      const long o = (long)m * ldc + c;
      C[o] = (float)H[o] > 0.f ? (bf16)v[j] : (bf16)0.f;
    }
  }
};

}  // namespace bc2n
