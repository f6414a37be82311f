// A LayerNorm over C = 128 fused with the product that consumes it: a
// workgroup LayerNorms 48 rows (xn, mean, rstd and optional pair-bias heads
// written as the unfused LayerNorm writes them), keeps the binary16 rows in
// LDS and multiplies them by an nout x 128 weight matrix 128 output columns
// at a time (fragments read straight from memory in b_frags_k128 order,
// prefetched a chunk ahead), each chunk's accumulators staged through LDS for
// the epilogue's row mode (8 columns of a row) or column mode (8 rows of a
// column, channel-major outputs).  Saves xn's write-then-read and the GEMM's
// per-tile operand staging.
#pragma once
#include "gemm.h"
#include "kernels.h"

namespace bc2n {
namespace lnproj {
// An epilogue whose column calls each handle a pair of columns (c and c + 16
// of every 32-column block: a projection and its gate) says kColPairs; the
// column loop then visits only the first of each pair, so no lane idles.
template <class E, class = void>
struct col_pairs : std::false_type {};
template <class E>
struct col_pairs<E, std::void_t<decltype(E::kColPairs)>> : std::bool_constant<E::kColPairs> {};

constexpr int C = 128, RT = 3, BM = 16 * RT, LDX = C + 8, LDT = 128 + 4;

struct Args {
  long M;
  int nt, bn, nout;  // nt: transposed read (ending node) when > 0; bn = N; nout = 4HD
  const float* x;
  const float *g, *b, *wb;  // LayerNorm scale, offset; bias weights [C][H]
  float bscale;
  h16* xn;  // LayerNorm output (written when not null); the input rows when LN = false
  float *mean, *rstd;
  h16* bias;  // [H][M] binary16 in score-fragment order
  const h16* W;  // [nout][C] in b_frags_k128 order
};

// LN = false: no LayerNorm; the binary16 rows are read from a.xn as they are.
// CM: the input is channel-major ([C][M], trimul's contraction output) and
// the LayerNorm is the centre norm's (ln_fwd_cm: eight lanes a row with 16
// consecutive channels each, the same sums in the same order), no xn.
template <int H, bool FAST, class Epi, bool LN = true, bool CM = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void kernel(Args a,
                                                                                           Epi epi) {
  __shared__ __align__(16) h16 xs[BM * LDX];
  __shared__ __align__(16) float T[BM * LDT];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, l16 = lane & 15;
  const long M = a.M, m0 = (long)blockIdx.x * BM;
  const int nch = a.nout / 128;
  h16x8 bf[4][2];
  auto load_b = [&](int j) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) bf[ks][jj] = b_frag_k128(a.W, j, w, jj, ks, lane);
  };
  if constexpr (!LN) {
    const int lr = lane >> 4, c0 = l16 * 8;
    h16x8 ob[RT];
#pragma unroll
    for (int p = 0; p < RT; ++p) {
      const long m = min(m0 + p * 16 + w * 4 + lr, M - 1);  // rows past M: in bounds, zeroed below
      ob[p] = ld8(a.xn + m * C + c0);
    }
    load_b(0);
#pragma unroll
    for (int p = 0; p < RT; ++p) {
      const int r = p * 16 + w * 4 + lr;
      st8(xs + r * LDX + c0, m0 + r < M ? ob[p] : h16x8{});
    }
  } else if constexpr (CM) {
    // the [C][BM] tile through T (rows past M read as zero), then the rows
    static_assert(H == 0 && BM % 4 == 0, "centre norm: no bias heads");
    load_b(0);
    for (int i = tid; i < C * (BM / 4); i += 256) {
      const int c = i / (BM / 4), q = (i % (BM / 4)) * 4;
      const long m = m0 + q;
      float4 v4 = make_float4(0.f, 0.f, 0.f, 0.f);
      if (m < M) v4 = *reinterpret_cast<const float4*>(a.x + (long)c * M + m);  // M % 4 == 0
      T[(q + 0) * LDT + c] = v4.x;
      T[(q + 1) * LDT + c] = v4.y;
      T[(q + 2) * LDT + c] = v4.z;
      T[(q + 3) * LDT + c] = v4.w;
    }
    __syncthreads();
    constexpr int P = 8, CPL = C / P;  // lanes and channels a row
#pragma unroll
    for (int rb = 0; rb < BM; rb += 256 / P) {
      const int r = rb + tid / P, part = tid % P;
      if (r < BM) {  // whole 8-lane groups
        const long m = m0 + r;
        float v[CPL];
        float s = 0.f, s2 = 0.f;
#pragma unroll
        for (int e = 0; e < CPL; ++e) {
          v[e] = T[r * LDT + part * CPL + e];
          s += v[e];
          s2 += v[e] * v[e];
        }
        s = group_sum<P>(s);
        const float mu = s / C;
        float var;
        if (FAST) {
          var = group_sum<P>(s2) / C - mu * mu;
        } else {
          float d2 = 0.f;
#pragma unroll
          for (int e = 0; e < CPL; ++e) { const float d = v[e] - mu; d2 += d * d; }
          var = group_sum<P>(d2) / C;
        }
        const float rs = rsqrtf(var + LN_EPS);
#pragma unroll
        for (int e0 = 0; e0 < CPL; e0 += 8) {
          h16x8 ob;
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const int c = part * CPL + e0 + e;
            ob[e] = (h16)((v[e0 + e] - mu) * rs * a.g[c] + a.b[c]);
          }
          st8(xs + r * LDX + part * CPL + e0, m < M ? ob : h16x8{});
        }
        if (part == 0 && m < M) {
          a.mean[m] = mu;
          a.rstd[m] = rs;
        }
      }
    }
  } else {
    const int lr = lane >> 4, c0 = l16 * 8;
    float v[RT][8];
#pragma unroll
    for (int p = 0; p < RT; ++p) {
      const long m = min(m0 + p * 16 + w * 4 + lr, M - 1);  // rows past M: in bounds, unused
      ld_f8(a.x + ln_src_row(m, a.nt) * C + c0, v[p]);
    }
    float gm[8], bt[8], wv[8][H > 0 ? H : 1];
    ld_f8(a.g + c0, gm);
    ld_f8(a.b + c0, bt);
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int h = 0; h < H; ++h) wv[e][h] = a.wb[(c0 + e) * H + h];
    load_b(0);
#pragma unroll
    for (int p = 0; p < RT; ++p) {
      const int r = p * 16 + w * 4 + lr;
      const long m = m0 + r;
      float s = 0.f, s2 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        s += v[p][e];
        s2 += v[p][e] * v[p][e];
      }
      const float mu = group_sum<16>(s) / C;
      float var;
      if constexpr (FAST) {
        var = group_sum<16>(s2) / C - mu * mu;
      } else {
        float d2 = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = v[p][e] - mu;
          d2 += d * d;
        }
        var = group_sum<16>(d2) / C;
      }
      const float rs = rsqrtf(var + LN_EPS);
      float o[8];
      h16x8 ob;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        o[e] = (v[p][e] - mu) * rs * gm[e] + bt[e];
        ob[e] = (h16)o[e];
      }
      float mine = 0.f;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        float q = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) q += o[e] * wv[e][h];
        q = group_sum<16>(q);
        if (l16 == h) mine = q;
      }
      if (m < M) {
        if (a.xn) st8(a.xn + m * C + c0, ob);
        if (l16 == 0) {
          a.mean[m] = mu;
          a.rstd[m] = rs;
        }
        if (H > 0 && l16 < H)
          a.bias[bias_frag_index(l16, (int)(m / a.bn), (int)(m % a.bn), a.bn)] = (h16)(mine * a.bscale);
      } else {
        ob = h16x8{};
      }
      st8(xs + r * LDX + c0, ob);
    }
  }
  __syncthreads();
  const int g = lane >> 4;
#pragma unroll 1
  for (int j = 0; j < nch; ++j) {
    f32x4 acc[RT][2];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) acc[i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      h16x8 af[RT];
#pragma unroll
      for (int i = 0; i < RT; ++i) af[i] = ld8(xs + (i * 16 + l16) * LDX + ks * 32 + 8 * g);
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) acc[i][jj] = mfma16x16x32(af[i], bf[ks][jj], acc[i][jj]);
    }
    // unconditional (the last chunk reloads its own): a load under a branch
    // leaves the in-order memory counter unknown at the join
    load_b(min(j + 1, nch - 1));
    __syncthreads();  // the previous chunk's epilogue is done with T
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          T[(i * 16 + 4 * g + r) * LDT + 32 * w + 16 * jj + l16] = acc[i][jj][r];
    __syncthreads();
    bool colm = false;
    if constexpr (Epi::kHasCol) colm = epi.col_mode(j * 128);
    if (colm) {
      // 8 consecutive rows of one column a call (channel-major outputs),
      // columns fastest (M and BM are multiples of 8)
      constexpr int CV = col_pairs<Epi>::value ? 64 : 128;  // columns visited
      for (int it = tid; it < CV * (BM / 8); it += 256) {
        const int cv = it % CV, rg = it / CV;
        const int c = col_pairs<Epi>::value ? (cv >> 4) * 32 + (cv & 15) : cv;
        const long m = m0 + rg * 8;
        if (m >= M) continue;
        const float* tp = T + (rg * 8) * LDT + c;
        float vv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) vv[e] = tp[e * LDT];
        epi.col(0, (int)m, j * 128 + c, vv, tp, LDT);
      }
    } else {
      for (int it = tid; it < BM * 16; it += 256) {
        const int r = it >> 4, c8 = (it & 15) * 8;
        const long m = m0 + r;
        if (m >= M) continue;
        float vv[8];
        ld_f8(T + r * LDT + c8, vv);
        epi.row(0, (int)m, j * 128 + c8, vv);
      }
    }
  }
}

// H = 0 (no bias heads) or 4; FAST: the one-pass variance.
template <int H, bool FAST, class Epi>
void launch(hipStream_t st, const Args& a, const Epi& epi) {
  static_assert(H == 0 || H == 4, "bias heads 0 or 4");
  if (a.M <= 0 || a.M % 8 != 0 || a.nout % 128 != 0 || (H > 0 && (long)a.bn * a.bn != a.M))
    throw std::runtime_error("LayerNorm-projection: shape");
  const dim3 grid((unsigned)((a.M + BM - 1) / BM));
  hipLaunchKernelGGL((kernel<H, FAST, Epi>), grid, dim3(256), 0, st, a, epi);
}
// The centre norm of a channel-major input (a.x = [C][M] f32, the statistics
// to a.mean / a.rstd) fused with the product; FAST: the one-pass variance.
template <bool FAST, class Epi>
void launch_cm(hipStream_t st, const Args& a, const Epi& epi) {
  if (a.M <= 0 || a.M % 8 != 0 || a.nout % 128 != 0 || !a.x || !a.W || !a.mean || !a.rstd)
    throw std::runtime_error("centre-norm projection: shape");
  const dim3 grid((unsigned)((a.M + BM - 1) / BM));
  hipLaunchKernelGGL((kernel<0, FAST, Epi, true, true>), grid, dim3(256), 0, st, a, epi);
}
// The same product without the LayerNorm: rows = a.xn (binary16 [M][128]).
template <class Epi>
void launch_rows(hipStream_t st, const Args& a, const Epi& epi) {
  if (a.M <= 0 || a.M % 8 != 0 || a.nout % 128 != 0 || !a.xn || !a.W)
    throw std::runtime_error("row projection: shape");
  const dim3 grid((unsigned)((a.M + BM - 1) / BM));
  hipLaunchKernelGGL((kernel<0, false, Epi, false>), grid, dim3(256), 0, st, a, epi);
}
}  // namespace lnproj
}  // namespace bc2n
