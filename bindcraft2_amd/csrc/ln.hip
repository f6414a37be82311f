// LayerNorm forward/backward over the channel axis, bandwidth kernels.
//
// A row of C channels is held by C/8 consecutive lanes, 8 channels each, so a
// 256-thread block normalises 2048/C rows with no LDS and no block barrier;
// both reductions are butterflies inside the lane group.  Variance is either
// two-pass (mean of squared deviations; haiku's default) or the "fast" form
// E[x^2]-E[x]^2 that AF2's fused triangle multiplication asks for.
//
// Options used by the trunk:
//  * transposed read: output row (p,q) normalises input row (q,p) of an
//    N x N grid -- the "ending node"/"per column" orientation without a copy;
//  * fused pair-bias projection: bias[h][row] = sum_c y[c] * W[c][h] from the
//    f32 normalised row (triangle attention / MSA row attention bias);
//  * channel-major input (trimul's centre norm), staged through LDS.
#include "kernels.h"

namespace bc2n {

template <int C>
struct LnGeom {
  static constexpr int TPR = C / 8;         // lanes per row
  static constexpr int RPB = 256 / TPR;     // rows per block
};

template <class T>
__device__ __forceinline__ void load8f(const T* p, float (&v)[8]);
template <>
__device__ __forceinline__ void load8f<float>(const float* p, float (&v)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
template <>
__device__ __forceinline__ void load8f<h16>(const h16* p, float (&v)[8]) {
  const h16x8 a = ld8(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (float)a[e];
}


template <int H>
__device__ __forceinline__ void load_w(const float* __restrict__ wb, int c0, float (&w)[8][H]) {
  const float4* p = reinterpret_cast<const float4*>(wb + c0 * H);
#pragma unroll
  for (int i = 0; i < 2 * H; ++i) {
    const float4 q = p[i];
    const float f[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) w[(4 * i + k) / H][(4 * i + k) % H] = f[k];
  }
}

// H = 0: plain LayerNorm.  H in {4, 8}: also the pair-bias projection
// bias_scale * sum_c y[m][c] W[c][h], from the f32 row, written in the
// attention kernels' score-fragment order (bias_frag_index, grid side bn).
// A lane group handles U rows (RPB apart): all U rows are loaded before the
// first is reduced, and gamma, beta and the projection slice are read once
// per U rows.
template <int C, bool FAST, class InT, int H, int U>
__global__ __launch_bounds__(256) void ln_fwd_kernel(
    const InT* __restrict__ x, long M, int nt, const float* __restrict__ gamma,
    const float* __restrict__ beta, h16* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out,
    const float* __restrict__ wb, h16* __restrict__ bias_out, float bias_scale, int bn) {
  using G = LnGeom<C>;
  const int t = threadIdx.x;
  const long mb = (long)blockIdx.x * (U * G::RPB) + t / G::TPR;
  const int gl = t % G::TPR;
  const int c0 = gl * 8;
  if (mb >= M) return;  // whole lane groups exit together
  float v[U][8];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long m = mb + (long)u * G::RPB;
    if (m < M) load8f<InT>(x + ln_src_row(m, nt) * C + c0, v[u]);
  }
  float gm[8], bt[8];
  load8f<float>(gamma + c0, gm);
  load8f<float>(beta + c0, bt);
  float w[8][H > 0 ? H : 1];
  if constexpr (H > 0) load_w<H>(wb, c0, w);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long m = mb + (long)u * G::RPB;
    if (m >= M) break;  // uniform over the lane group
    float s = 0.f, s2 = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) { s += v[u][e]; s2 += v[u][e] * v[u][e]; }
    s = group_sum<G::TPR>(s);
    const float mu = s / C;
    float var;
    if (FAST) {
      s2 = group_sum<G::TPR>(s2);
      var = s2 / C - mu * mu;
    } else {
      float d2 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) { const float d = v[u][e] - mu; d2 += d * d; }
      var = group_sum<G::TPR>(d2) / C;
    }
    const float r = rsqrtf(var + LN_EPS);
    float o[8];
    h16x8 ob;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o[e] = (v[u][e] - mu) * r * gm[e] + bt[e];
      ob[e] = (h16)o[e];
    }
    if (y) st8(y + m * C + c0, ob);
    if (gl == 0) {
      if (mean_out) mean_out[m] = mu;
      if (rstd_out) rstd_out[m] = r;
    }
    if constexpr (H > 0) {
      static_assert(H <= G::TPR, "one lane per head writes");
      float mine = 0.f;
#pragma unroll
      for (int h = 0; h < H; ++h) {
        float p = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) p += o[e] * w[e][h];
        p = group_sum<G::TPR>(p);
        if (gl == h) mine = p;
      }
      if (gl < H) bias_out[bias_frag_index(gl, (int)(m / bn), (int)(m % bn), bn)] = (h16)(mine * bias_scale);
    }
  }
}

// The LayerNorm + pair-bias projection of C = 128 rows with no normalised
// output (the MSA row attention's pair bias, 8 heads), in the MFMA operand
// layout: a wave takes 16 rows, lane l row l & 15 and channels
// 32 ks + 8 (l >> 4) + e (ks < 4, e < 8) -- its A fragments of the
// 16 x 128 x 16 product with the weights (heads padded to 16 columns), so
// the statistics need two xor exchanges and the H dot products are four
// v_mfma_f32_16x16x32_f16 instead of H lane-group reductions.  The
// LayerNorm's scale and offset are folded into the weights on the host
// (ln_bias_frags): bias = sum_c xhat_c (gamma_c W_ch) + sum_c beta_c W_ch,
// with xhat in binary16 (as every other projection of the trunk) and the
// second sum a per-head constant, so a lane reads four 16-byte fragments
// and one constant.  Result lane l holds head l & 15 of rows 4 (l >> 4) + r,
// r < 4: four consecutive bias_frag_index slots, one 8-byte store.
template <bool FAST>
__global__ __launch_bounds__(256) void ln_bias16_kernel(
    const float* __restrict__ x, long M, float* __restrict__ mean_out,
    float* __restrict__ rstd_out, const h16* __restrict__ wfrag, const float* __restrict__ wconst,
    int H, h16* __restrict__ bias_out, float bias_scale, int bn) {
  constexpr int C = 128;
  const int lane = threadIdx.x & 63;
  const long m0 = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 16;
  if (m0 >= M) return;  // M % 16 == 0: whole waves
  const int r = lane & 15, kg = lane >> 4;
  float v[4][8];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) load8f<float>(x + (m0 + r) * C + ks * 32 + kg * 8, v[ks]);
  h16x8 bf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) bf[ks] = ld8(wfrag + (ks * 64 + lane) * 8);
  const float wc = wconst[r];
  auto quad_sum = [](float a) {
    a += __shfl_xor(a, 16, 64);
    return a + __shfl_xor(a, 32, 64);
  };
  float s = 0.f, s2 = 0.f;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      s += v[ks][e];
      s2 += v[ks][e] * v[ks][e];
    }
  const float mu = quad_sum(s) / C;
  float var;
  if constexpr (FAST) {
    var = quad_sum(s2) / C - mu * mu;
  } else {
    float d2 = 0.f;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float d = v[ks][e] - mu;
        d2 += d * d;
      }
    var = quad_sum(d2) / C;
  }
  const float rs = rsqrtf(var + LN_EPS);
  if (kg == 0) {
    if (mean_out) mean_out[m0 + r] = mu;
    if (rstd_out) rstd_out[m0 + r] = rs;
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    h16x8 af;
#pragma unroll
    for (int e = 0; e < 8; ++e) af[e] = (h16)((v[ks][e] - mu) * rs);
    acc = mfma16x16x32(af, bf[ks], acc);
  }
  if (r < H) {
    // rows m0 + 4 kg + i: query q, keys k0 + i (k0 % 4 == 0, one 16-key tile)
    const long m = m0 + 4 * kg;
    const int q = (int)(m / bn), k0 = (int)(m % bn);
    h16x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (h16)((acc[i] + wc) * bias_scale);
    *reinterpret_cast<h16x4*>(bias_out + bias_frag_index(r, q, k0, bn)) = o;
  }
}

// Its backward with the residual add, dx[m] += LN'(gs * sum_h dbias[h][m]
// W[c][h]) (C = 128, H <= 16), the bias term as an f32 MFMA product in the
// forward's row-per-lane layout: the transposed product
// G^T[c][m] = sum_h (gamma_c W_ch) dbias[h][m], one 16-channel block at a
// time (v_mfma_f32_16x16x4_f32, K = 4 heads a step, A fragments pre-arranged
// on the host by ln_bias_bwd_frags), leaves lane l with row m0 + (l & 15) and
// channels 16 cb + 4 (l >> 4) + i (cb < 8, i < 4): the row sums of the
// LayerNorm backward are two xor exchanges, and x and dx move in 16-byte
// pieces.  Exact f32 arithmetic throughout.  With amax_part, the
// workgroup's max |dx| of its 64 rows goes to amax_part[blockIdx.x] (the
// partial maxima of the next cotangent scale, saving that pass its read).
__global__ __launch_bounds__(256) void ln_bias16_bwd_kernel(
    const float* __restrict__ x, long M, const float* __restrict__ mean,
    const float* __restrict__ rstd, const float* __restrict__ afrag, int H,
    const float* __restrict__ dbias, float* __restrict__ dx, const float* __restrict__ gmul,
    float* __restrict__ amax_part) {
  constexpr int C = 128;
  const int lane = threadIdx.x & 63;
  // M % 64 == 0 and the grid is exact (host): every wave has its 16 rows
  const long m0 = ((long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 16;
  const int r = lane & 15, kg = lane >> 4;
  const long row = (m0 + r) * C + 4 * kg;
  float4 xv[8], dr[8];
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) {
    xv[cb] = *reinterpret_cast<const float4*>(x + row + 16 * cb);
    dr[cb] = *reinterpret_cast<const float4*>(dx + row + 16 * cb);
  }
  const float mu = mean[m0 + r], rs = rstd[m0 + r];
  const float gs = gmul ? *gmul : 1.f;
  const int T = (H + 3) / 4;
  float bv[4];
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    const int h = 4 * t + kg;
    bv[t] = (t < T && h < H) ? dbias[(long)h * M + m0 + r] : 0.f;
  }
  f32x4 g[8];
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) {
    g[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
      if (t < T)
        g[cb] = __builtin_amdgcn_mfma_f32_16x16x4f32(afrag[(t * 8 + cb) * 64 + lane], bv[t], g[cb],
                                                     0, 0, 0);
  }
  float sg = 0.f, sgx = 0.f;
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) {
    const float xs[4] = {xv[cb].x, xv[cb].y, xv[cb].z, xv[cb].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      g[cb][i] *= gs;
      sg += g[cb][i];
      sgx += g[cb][i] * ((xs[i] - mu) * rs);
    }
  }
  auto quad_sum = [](float a) {
    a += __shfl_xor(a, 16, 64);
    return a + __shfl_xor(a, 32, 64);
  };
  sg = quad_sum(sg) * (1.f / C);
  sgx = quad_sum(sgx) * (1.f / C);
  float am = 0.f;
#pragma unroll
  for (int cb = 0; cb < 8; ++cb) {
    const float xs[4] = {xv[cb].x, xv[cb].y, xv[cb].z, xv[cb].w};
    float o[4] = {dr[cb].x, dr[cb].y, dr[cb].z, dr[cb].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[i] += rs * (g[cb][i] - sg - ((xs[i] - mu) * rs) * sgx);
      am = fmaxf(am, fabsf(o[i]));
    }
    *reinterpret_cast<float4*>(dx + row + 16 * cb) = make_float4(o[0], o[1], o[2], o[3]);
  }
  if (amax_part) {  // the same maximum as amax_part_kernel's (fmaxf of |dx|)
    am = group_max<64>(am);
    __shared__ float red[4];
    if (lane == 0) red[threadIdx.x >> 6] = am;
    __syncthreads();
    if (threadIdx.x == 0)
      amax_part[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  }
}

// dx[src(m)] = (ACC ? res[src(m)] : 0) + LN'(gs * (dy[m] + sum_h dbias[h][m] W[c][h]))
// (dy may be null; res = dres, or dx itself when dres is null; gs = *gmul,
// the inverse cotangent scale of the module, or 1 when gmul is null); U rows
// per lane group, as the forward.
template <int C, class InT, bool ACC, int H, int U>
__global__ __launch_bounds__(256) void ln_bwd_kernel(
    const float* __restrict__ dy, const InT* __restrict__ x, long M, int nt,
    const float* __restrict__ gamma, const float* __restrict__ mean,
    const float* __restrict__ rstd, float* __restrict__ dx,
    const float* __restrict__ dbias, const float* __restrict__ wb, const float* dres,
    const float* __restrict__ gmul) {
  using G = LnGeom<C>;
  const int t = threadIdx.x;
  const long mb = (long)blockIdx.x * (U * G::RPB) + t / G::TPR;
  const float* res = dres ? dres : dx;  // the residual cotangent ACC adds
  const int c0 = (t % G::TPR) * 8;
  if (mb >= M) return;
  float xv[U][8], g[U][8], ov[U][8], mu[U], r[U];
  float db[U][H > 0 ? H : 1];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long m = mb + (long)u * G::RPB;
    if (m >= M) continue;
    const long src = ln_src_row(m, nt);
    load8f<InT>(x + src * C + c0, xv[u]);
    if (dy) {
      load8f<float>(dy + m * C + c0, g[u]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) g[u][e] = 0.f;
    }
    if (ACC) load8f<float>(res + src * C + c0, ov[u]);
    mu[u] = mean[m];
    r[u] = rstd[m];
    if constexpr (H > 0) {
#pragma unroll
      for (int h = 0; h < H; ++h) db[u][h] = dbias[(long)h * M + m];
    }
  }
  float gm[8];
  load8f<float>(gamma + c0, gm);
  if (gmul) {
    const float gs = *gmul;
#pragma unroll
    for (int e = 0; e < 8; ++e) gm[e] *= gs;
  }
  float w[8][H > 0 ? H : 1];
  if constexpr (H > 0) load_w<H>(wb, c0, w);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const long m = mb + (long)u * G::RPB;
    if (m >= M) break;
    if constexpr (H > 0) {
#pragma unroll
      for (int h = 0; h < H; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) g[u][e] += db[u][h] * w[e][h];
    }
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xv[u][e] = (xv[u][e] - mu[u]) * r[u];
      g[u][e] *= gm[e];
      sg += g[u][e];
      sgx += g[u][e] * xv[u][e];
    }
    sg = group_sum<G::TPR>(sg) / C;
    sgx = group_sum<G::TPR>(sgx) / C;
    float* out = dx + ln_src_row(m, nt) * C + c0;
    float res[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      res[e] = r[u] * (g[u][e] - sg - xv[u][e] * sgx);
      if (ACC) res[e] += ov[u][e];
    }
    reinterpret_cast<float4*>(out)[0] = make_float4(res[0], res[1], res[2], res[3]);
    reinterpret_cast<float4*>(out)[1] = make_float4(res[4], res[5], res[6], res[7]);
  }
}

// Channel-major input: x is [C][M] (one plane per channel).  A block of
// LNCM_R rows stages the [C][LNCM_R] tile through LDS (4-wide loads along m)
// and then normalises it 256/LNCM_R lanes per row; the output is row-major
// [M][C] h16.
// Requires M % 4 == 0.
// 4 consecutive m of channel plane c (x is [C][M], float or h16)
__device__ __forceinline__ float4 cm_load4(const float* x, long idx) {
  return *reinterpret_cast<const float4*>(x + idx);
}
__device__ __forceinline__ float4 cm_load4(const h16* x, long idx) {
  const h16x4 v = *reinterpret_cast<const h16x4*>(x + idx);
  return make_float4((float)v[0], (float)v[1], (float)v[2], (float)v[3]);
}

// Rows per workgroup of the channel-major kernels (256 threads, 256/R lanes a row).
constexpr int LNCM_R = 32;
static_assert(64 / (256 / LNCM_R) >= 8, "the 64-channel kernels store 8 channels a lane");

template <int C, bool FAST, class InT>
__global__ __launch_bounds__(256) void ln_fwd_cm_kernel(
    const InT* __restrict__ x, long M, const float* __restrict__ gamma,
    const float* __restrict__ beta, h16* __restrict__ y,
    float* __restrict__ mean_out, float* __restrict__ rstd_out) {
  constexpr int R = LNCM_R;
  __shared__ float tile[R][C + 1];
  const int t = threadIdx.x;
  const long m0 = (long)blockIdx.x * R;
  for (int i = t; i < C * (R / 4); i += 256) {
    const int c = i / (R / 4), q = (i % (R / 4)) * 4;
    const long m = m0 + q;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (m < M) v = cm_load4(x, (long)c * M + m);
    tile[q + 0][c] = v.x;
    tile[q + 1][c] = v.y;
    tile[q + 2][c] = v.z;
    tile[q + 3][c] = v.w;
  }
  __syncthreads();
  constexpr int P = 256 / R, CPL = C / P;  // lanes and channels per row
  const int r = t / P, part = t % P;
  const long m = m0 + r;
  float v[CPL];
  float s = 0.f, s2 = 0.f;
#pragma unroll
  for (int e = 0; e < CPL; ++e) {
    v[e] = tile[r][part * CPL + e];
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
  if (m < M) {
#pragma unroll
    for (int e0 = 0; e0 < CPL; e0 += 8) {
      h16x8 ob;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int c = part * CPL + e0 + e;
        ob[e] = (h16)((v[e0 + e] - mu) * rs * gamma[c] + beta[c]);
      }
      st8(y + m * C + part * CPL + e0, ob);
    }
    if (part == 0) { mean_out[m] = mu; rstd_out[m] = rs; }
  }
}

// Backward of the channel-major norm: dy row-major [M][C] f32, x channel-major
// [C][M] f32; writes dx channel-major [C][M] as h16 (a GEMM operand).
template <int C, class InT>
__global__ __launch_bounds__(256) void ln_bwd_cm_kernel(
    const float* __restrict__ dy, const InT* __restrict__ x, long M,
    const float* __restrict__ gamma, const float* __restrict__ mean,
    const float* __restrict__ rstd, h16* __restrict__ dx) {
  constexpr int R = LNCM_R;
  __shared__ float tile[R][C + 1];
  const int t = threadIdx.x;
  const long m0 = (long)blockIdx.x * R;
  for (int i = t; i < C * (R / 4); i += 256) {
    const int c = i / (R / 4), q = (i % (R / 4)) * 4;
    const long m = m0 + q;
    float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
    if (m < M) v = cm_load4(x, (long)c * M + m);
    tile[q + 0][c] = v.x;
    tile[q + 1][c] = v.y;
    tile[q + 2][c] = v.z;
    tile[q + 3][c] = v.w;
  }
  __syncthreads();
  constexpr int P = 256 / R, CPL = C / P;  // lanes and channels per row
  const int r = t / P, part = t % P;
  const long m = m0 + r;
  const bool live = m < M;
  const float mu = live ? mean[m] : 0.f, rs = live ? rstd[m] : 0.f;
  float xh[CPL], g[CPL];
  float sg = 0.f, sgx = 0.f;
#pragma unroll
  for (int e0 = 0; e0 < CPL; e0 += 4) {
    float4 d = make_float4(0.f, 0.f, 0.f, 0.f);
    if (live) d = *reinterpret_cast<const float4*>(dy + m * C + part * CPL + e0);
    const float dv[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int e = e0 + k, c = part * CPL + e;
      xh[e] = (tile[r][c] - mu) * rs;
      g[e] = dv[k] * gamma[c];
      sg += g[e];
      sgx += g[e] * xh[e];
    }
  }
  sg = group_sum<P>(sg) / C;
  sgx = group_sum<P>(sgx) / C;
  __syncthreads();
#pragma unroll
  for (int e = 0; e < CPL; ++e) {
    const int c = part * CPL + e;
    tile[r][c] = rs * (g[e] - sg - xh[e] * sgx);
  }
  __syncthreads();
  for (int i = t; i < C * (R / 4); i += 256) {
    const int c = i / (R / 4), q = (i % (R / 4)) * 4;
    const long mm = m0 + q;
    if (mm < M) {
      h16x4 o;
      o[0] = f2h_sat(tile[q + 0][c]);
      o[1] = f2h_sat(tile[q + 1][c]);
      o[2] = f2h_sat(tile[q + 2][c]);
      o[3] = f2h_sat(tile[q + 3][c]);
      *reinterpret_cast<h16x4*>(dx + (long)c * M + mm) = o;
    }
  }
}

// ------------------------------------------------------------------ launchers

// Rows per lane group of the row-major kernels: several only where a bias
// projection (weights in registers, H sums per row) is amortised over them;
// a plain row keeps the register count, and so the occupancy, low.
template <int H>
constexpr int ln_rows() { return H > 0 ? 4 : 1; }

template <int C, int H>
static void ln_fwd_launch(hipStream_t st, const float* x, long M, int nt, const float* gamma,
                          const float* beta, h16* y, float* mean, float* rstd, bool fast,
                          const float* wb, h16* bias_out, float bs, int bn) {
  constexpr int U = ln_rows<H>();
  const int grid = (int)((M + U * LnGeom<C>::RPB - 1) / (U * LnGeom<C>::RPB));
  if (fast)
    hipLaunchKernelGGL((ln_fwd_kernel<C, true, float, H, U>), dim3(grid), dim3(256), 0, st, x, M,
                       nt, gamma, beta, y, mean, rstd, wb, bias_out, bs, bn);
  else
    hipLaunchKernelGGL((ln_fwd_kernel<C, false, float, H, U>), dim3(grid), dim3(256), 0, st, x, M,
                       nt, gamma, beta, y, mean, rstd, wb, bias_out, bs, bn);
}

template <int C>
static void ln_fwd_dispatch(hipStream_t st, const float* x, long M, int nt, const float* gamma,
                            const float* beta, h16* y, float* mean, float* rstd, bool fast, int H,
                            const float* wb, h16* bias_out, float bs, int bn) {
  switch (H) {
    case 0: ln_fwd_launch<C, 0>(st, x, M, nt, gamma, beta, y, mean, rstd, fast, wb, bias_out, bs, bn); break;
    case 4: ln_fwd_launch<C, 4>(st, x, M, nt, gamma, beta, y, mean, rstd, fast, wb, bias_out, bs, bn); break;
    case 8: ln_fwd_launch<C, 8>(st, x, M, nt, gamma, beta, y, mean, rstd, fast, wb, bias_out, bs, bn); break;
    default: throw std::runtime_error("ln_fwd: bias heads must be 0, 4 or 8");
  }
}

void ln_fwd_f32(hipStream_t st, const float* x, long M, int C, int nt,
                const float* gamma, const float* beta, h16* y, float* mean,
                float* rstd, bool fast, int H, const float* wb, h16* bias_out,
                float bs) {
  int bn = 0;  // side of the N x N grid of the pair bias
  if (H > 0) {
    while ((long)(bn + 1) * (bn + 1) <= M) ++bn;
    if ((long)bn * bn != M || bn % 32 != 0)
      throw std::runtime_error("ln_fwd: the pair bias needs M = N*N with N % 32 == 0");
  }
  switch (C) {
    case 64: ln_fwd_dispatch<64>(st, x, M, nt, gamma, beta, y, mean, rstd, fast, H, wb, bias_out, bs, bn); break;
    case 128: ln_fwd_dispatch<128>(st, x, M, nt, gamma, beta, y, mean, rstd, fast, H, wb, bias_out, bs, bn); break;
    case 256: ln_fwd_dispatch<256>(st, x, M, nt, gamma, beta, y, mean, rstd, fast, H, wb, bias_out, bs, bn); break;
    default: throw std::runtime_error("ln_fwd: unsupported channel count");
  }
}

std::vector<h16> ln_bias_frags(const float* gamma, const float* wb, int H) {
  if (H <= 0 || H > 16) throw std::runtime_error("ln_bias_frags: 1 to 16 heads");
  std::vector<h16> f(4 * 64 * 8);
  for (int ks = 0; ks < 4; ++ks)
    for (int l = 0; l < 64; ++l)
      for (int e = 0; e < 8; ++e) {
        const int c = ks * 32 + 8 * (l >> 4) + e, h = l & 15;
        f[(ks * 64 + l) * 8 + e] = h < H ? (h16)(gamma[c] * wb[c * H + h]) : (h16)0.f;
      }
  return f;
}

std::vector<float> ln_bias_const(const float* beta, const float* wb, int H) {
  if (H <= 0 || H > 16) throw std::runtime_error("ln_bias_const: 1 to 16 heads");
  std::vector<float> b(16, 0.f);
  for (int h = 0; h < H; ++h) {
    double t = 0.0;
    for (int c = 0; c < 128; ++c) t += (double)beta[c] * wb[c * H + h];
    b[h] = (float)t;
  }
  return b;
}

std::vector<float> ln_bias_bwd_frags(const float* gamma, const float* wb, int H) {
  if (H <= 0 || H > 16) throw std::runtime_error("ln_bias_bwd_frags: 1 to 16 heads");
  std::vector<float> f(4 * 8 * 64, 0.f);
  for (int t = 0; t < 4; ++t)
    for (int cb = 0; cb < 8; ++cb)
      for (int l = 0; l < 64; ++l) {
        const int c = 16 * cb + (l & 15), h = 4 * t + (l >> 4);
        if (h < H) f[(t * 8 + cb) * 64 + l] = gamma[c] * wb[c * H + h];
      }
  return f;
}

long ln_pair_bias_bwd_f32(hipStream_t st, const float* x, long M, const float* mean,
                          const float* rstd, const float* afrag, int H, const float* dbias,
                          float* dx, const float* gmul, float* amax_part, long amax_cap) {
  if (M <= 0 || M % 64 != 0 || H <= 0 || H > 16 || !x || !mean || !rstd || !afrag || !dbias || !dx)
    throw std::runtime_error("ln_pair_bias_bwd: M % 64 == 0, 1 to 16 heads");
  const long grid = M / 64;
  if (grid > amax_cap) amax_part = nullptr;
  hipLaunchKernelGGL(ln_bias16_bwd_kernel, dim3((unsigned)grid), dim3(256), 0, st, x, M, mean, rstd,
                     afrag, H, dbias, dx, gmul, amax_part);
  return amax_part ? grid : 0;
}

void ln_pair_bias_f32(hipStream_t st, const float* x, long M, bool fast, float* mean, float* rstd,
                      const h16* wfrag, const float* wconst, int H, h16* bias_out, float bs) {
  int bn = 0;
  while ((long)(bn + 1) * (bn + 1) <= M) ++bn;
  if ((long)bn * bn != M || bn % 32 != 0 || H <= 0 || H > 16 || !x || !wfrag || !wconst || !bias_out)
    throw std::runtime_error("ln_pair_bias: M = N*N with N % 32 == 0, 1 to 16 heads");
  const unsigned grid = (unsigned)((M / 16 + 3) / 4);
  if (fast)
    hipLaunchKernelGGL(ln_bias16_kernel<true>, dim3(grid), dim3(256), 0, st, x, M, mean, rstd,
                       wfrag, wconst, H, bias_out, bs, bn);
  else
    hipLaunchKernelGGL(ln_bias16_kernel<false>, dim3(grid), dim3(256), 0, st, x, M, mean, rstd,
                       wfrag, wconst, H, bias_out, bs, bn);
}

template <int C, int H>
static void ln_bwd_launch(hipStream_t st, const float* dy, const float* x, long M, int nt,
                          const float* gamma, const float* mean, const float* rstd, float* dx,
                          bool acc, const float* dbias, const float* wb, const float* dres,
                          const float* gmul) {
  constexpr int U = ln_rows<H>();
  const int grid = (int)((M + U * LnGeom<C>::RPB - 1) / (U * LnGeom<C>::RPB));
  if (acc)
    hipLaunchKernelGGL((ln_bwd_kernel<C, float, true, H, U>), dim3(grid), dim3(256), 0, st, dy, x,
                       M, nt, gamma, mean, rstd, dx, dbias, wb, dres, gmul);
  else
    hipLaunchKernelGGL((ln_bwd_kernel<C, float, false, H, U>), dim3(grid), dim3(256), 0, st, dy, x,
                       M, nt, gamma, mean, rstd, dx, dbias, wb, dres, gmul);
}

template <int C>
static void ln_bwd_dispatch(hipStream_t st, const float* dy, const float* x, long M, int nt,
                            const float* gamma, const float* mean, const float* rstd, float* dx,
                            bool acc, int H, const float* dbias, const float* wb, const float* dres,
                            const float* gmul) {
  switch (H) {
    case 0: ln_bwd_launch<C, 0>(st, dy, x, M, nt, gamma, mean, rstd, dx, acc, dbias, wb, dres, gmul); break;
    case 4: ln_bwd_launch<C, 4>(st, dy, x, M, nt, gamma, mean, rstd, dx, acc, dbias, wb, dres, gmul); break;
    case 8: ln_bwd_launch<C, 8>(st, dy, x, M, nt, gamma, mean, rstd, dx, acc, dbias, wb, dres, gmul); break;
    default: throw std::runtime_error("ln_bwd: bias heads must be 0, 4 or 8");
  }
}

void ln_bwd_f32(hipStream_t st, const float* dy, const float* x, long M, int C,
                int nt, const float* gamma, const float* mean, const float* rstd,
                float* dx, bool acc, int H, const float* dbias, const float* wb,
                const float* dres, const float* gmul) {
  switch (C) {
    case 64: ln_bwd_dispatch<64>(st, dy, x, M, nt, gamma, mean, rstd, dx, acc, H, dbias, wb, dres, gmul); break;
    case 128: ln_bwd_dispatch<128>(st, dy, x, M, nt, gamma, mean, rstd, dx, acc, H, dbias, wb, dres, gmul); break;
    case 256: ln_bwd_dispatch<256>(st, dy, x, M, nt, gamma, mean, rstd, dx, acc, H, dbias, wb, dres, gmul); break;
    default: throw std::runtime_error("ln_bwd: unsupported channel count");
  }
}

template <class InT>
static void ln_fwd_cm_t(hipStream_t st, const InT* x, long M, int C, const float* gamma,
                        const float* beta, h16* y, float* mean, float* rstd, bool fast) {
  if (M % 4 != 0) throw std::runtime_error("ln_fwd_cm: M must be a multiple of 4");
  const int grid = (int)((M + LNCM_R - 1) / LNCM_R);
#define BC2N_LNCM(CV, FV) \
  hipLaunchKernelGGL((ln_fwd_cm_kernel<CV, FV, InT>), dim3(grid), dim3(256), 0, st, x, M, gamma, beta, y, mean, rstd)
  if (C == 128) {
    if (fast) BC2N_LNCM(128, true); else BC2N_LNCM(128, false);
  } else if (C == 64) {
    if (fast) BC2N_LNCM(64, true); else BC2N_LNCM(64, false);
  } else {
    throw std::runtime_error("ln_fwd_cm: unsupported channel count");
  }
#undef BC2N_LNCM
}
void ln_fwd_cm(hipStream_t st, const float* x, long M, int C, const float* gamma,
               const float* beta, h16* y, float* mean, float* rstd, bool fast) {
  ln_fwd_cm_t(st, x, M, C, gamma, beta, y, mean, rstd, fast);
}
void ln_fwd_cm(hipStream_t st, const h16* x, long M, int C, const float* gamma,
               const float* beta, h16* y, float* mean, float* rstd, bool fast) {
  ln_fwd_cm_t(st, x, M, C, gamma, beta, y, mean, rstd, fast);
}

template <class InT>
static void ln_bwd_cm_t(hipStream_t st, const float* dy, const InT* x, long M, int C,
                        const float* gamma, const float* mean, const float* rstd, h16* dx) {
  if (M % 4 != 0) throw std::runtime_error("ln_bwd_cm: M must be a multiple of 4");
  const int grid = (int)((M + LNCM_R - 1) / LNCM_R);
  if (C == 128) hipLaunchKernelGGL((ln_bwd_cm_kernel<128, InT>), dim3(grid), dim3(256), 0, st, dy, x, M, gamma, mean, rstd, dx);
  else if (C == 64) hipLaunchKernelGGL((ln_bwd_cm_kernel<64, InT>), dim3(grid), dim3(256), 0, st, dy, x, M, gamma, mean, rstd, dx);
  else throw std::runtime_error("ln_bwd_cm: unsupported channel count");
}
void ln_bwd_cm(hipStream_t st, const float* dy, const float* x, long M, int C,
               const float* gamma, const float* mean, const float* rstd, h16* dx) {
  ln_bwd_cm_t(st, dy, x, M, C, gamma, mean, rstd, dx);
}
void ln_bwd_cm(hipStream_t st, const float* dy, const h16* x, long M, int C,
               const float* gamma, const float* mean, const float* rstd, h16* dx) {
  ln_bwd_cm_t(st, dy, x, M, C, gamma, mean, rstd, dx);
}

// ------------------------------------------------- f32 rows, any width
// f32 in, f32 out, one wave per row (two-pass variance): the structure
// module and the small MSA modules, where rows are few or short.
__global__ void ln_f32_rows_fwd_kernel(const float* __restrict__ x, long M, int C,
                                   const float* __restrict__ g, const float* __restrict__ b,
                                   float* __restrict__ y, float* __restrict__ mean,
                                   float* __restrict__ rstd) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const float* xr = x + row * C;
  float s = 0.f;
  for (int c = lane; c < C; c += 64) s += xr[c];
  s = group_sum<64>(s);
  const float mu = s / C;
  float v = 0.f;
  for (int c = lane; c < C; c += 64) { const float d = xr[c] - mu; v += d * d; }
  v = group_sum<64>(v);
  const float r = rsqrtf(v / C + LN_EPS);
  for (int c = lane; c < C; c += 64) y[row * C + c] = (xr[c] - mu) * r * g[c] + b[c];
  if (lane == 0) { mean[row] = mu; rstd[row] = r; }
}

// dx = r * (g*dy - mean(g*dy) - xhat * mean(g*dy*xhat)); dx may alias dy.
__global__ void ln_f32_rows_bwd_kernel(const float* dy, const float* __restrict__ x,
                                   long M, int C, const float* __restrict__ g,
                                   const float* __restrict__ mean, const float* __restrict__ rstd,
                                   float* dx) {
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (row >= M) return;
  const float mu = mean[row], r = rstd[row];
  float s1 = 0.f, s2 = 0.f;
  for (int c = lane; c < C; c += 64) {
    const float gd = g[c] * dy[row * C + c];
    s1 += gd;
    s2 += gd * (x[row * C + c] - mu) * r;
  }
  s1 = group_sum<64>(s1) / C;
  s2 = group_sum<64>(s2) / C;
  for (int c = lane; c < C; c += 64) {
    const float xh = (x[row * C + c] - mu) * r;
    dx[row * C + c] = r * (g[c] * dy[row * C + c] - s1 - xh * s2);
  }
}

void ln_f32_rows_fwd(hipStream_t st, const float* x, long M, int C, const float* g, const float* b,
                 float* y, float* mean, float* rstd) {
  hipLaunchKernelGGL(ln_f32_rows_fwd_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, st, x, M, C,
                     g, b, y, mean, rstd);
}
void ln_f32_rows_bwd(hipStream_t st, const float* dy, const float* x, long M, int C, const float* g,
                 const float* mean, const float* rstd, float* dx) {
  hipLaunchKernelGGL(ln_f32_rows_bwd_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, st, dy, x, M,
                     C, g, mean, rstd, dx);
}

}  // namespace bc2n
