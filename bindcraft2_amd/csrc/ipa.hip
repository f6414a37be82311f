// The structure module's fold iterations: invariant point attention (IPA),
// the transition and the quaternion rigid update, forward and backward, in
// f32 as AF2 runs them.
//
// Reference: bindcraft/af/alphafold/model/folding_multimer.py:188-371
// (InvariantPointAttention), :374-474 (FoldIteration, without the
// sidechain), :476-548 (generate_monomer_rigids: LN + initial projection,
// identity frames, LN(pair), a scan over `depth` iterations sharing one set
// of weights, per-iteration keys split(key, depth)); geometry/
// rotation_matrix.py:117-140 (from_quaternion), rigid_matrix_vector.py:37-55
// (compose, apply, apply_inverse).  The reference keeps gradient through
// the rotation between iterations (its stop_gradient is commented out,
// folding_multimer.py:467), and so does this.
//
// Layouts (N residues, H = 12 heads):
//   rigid  [N][12]       R row-major (9) then t (3)
//   P      [N][1152]     the six projections of act, one GEMM:
//                        q_s 0..191 | k_s ..383 | v_s ..575 (head*16 + c) |
//                        q_pt ..719 | k_pt ..863 (head*12 + [x4 y4 z4]) |
//                        v_pt ..1151 (head*24 + [x8 y8 z8])
//   qpk    [N][H][32]    [q_s/4 (16) | global q points (p*3+xyz, 12) | 1 | 0 0 0]
//   kpk    [N][H][32]    [k_s (16)   | global k points (12)           | 1 | 0 0 0]
//   vpk    [N][H][40]    [v_s (16)   | global v points (p*3+xyz, 24)]
//   b2d    [H][N][N]     Linear(LN(pair)) -> H; the same for every iteration
//   attn   [H][N][N]     softmax over keys
//   final  [N][2112]     [scalar 192 | x 96 | y 96 | z 96 | norm 96 | pair 1536]
// The trailing 1 of qpk/kpk makes the backward's GEMMs against them also
// produce the row / column sums of dlogit that the point term needs.
#include "gemm_f32.h"
#include "kernels.h"
#include "modules.h"

namespace bc2n {

namespace {

constexpr int CS = 384, CZ = 128, H = 12, SQK = 16, PQK = 4, SV = 16, PV = 8;
constexpr int PROJ = 3 * H * SQK + 2 * H * PQK * 3 + H * PV * 3;  // 1152
constexpr int OFF_QS = 0, OFF_KS = H * SQK, OFF_VS = 2 * H * SQK;
constexpr int OFF_QP = 3 * H * SQK, OFF_KP = OFF_QP + H * PQK * 3, OFF_VP = OFF_KP + H * PQK * 3;
constexpr int FIN = H * SV + 4 * H * PV + H * CZ;  // 2112
constexpr int FIN_X = H * SV, FIN_Y = FIN_X + H * PV, FIN_Z = FIN_Y + H * PV,
              FIN_NORM = FIN_Z + H * PV, FIN_PAIR = FIN_NORM + H * PV;
constexpr int QKW = 32, VW = 40;
constexpr float LOGIT_W = 0.57735026918962576f;  // sqrt(1/3): three logit terms
constexpr float SCALAR_W = 0.25f;                 // sqrt(1/16)
constexpr float DIST_EPS2 = 1e-16f;               // (1e-8)^2, Vec3Array.norm clip
constexpr float QUAT_EPS = 1e-6f;
constexpr float POSITION_SCALE = 20.f;            // config.py:595 (multimer)
constexpr int MAXN = 1024;

static_assert(PROJ == 1152 && FIN == 2112, "IPA widths");

// ---------------------------------------------------------- small helpers
__device__ __forceinline__ void rot_apply(const float* R, const float* p, float* o) {
#pragma unroll
  for (int i = 0; i < 3; ++i) o[i] = R[i * 3] * p[0] + R[i * 3 + 1] * p[1] + R[i * 3 + 2] * p[2];
}
__device__ __forceinline__ void rot_apply_t(const float* R, const float* p, float* o) {
#pragma unroll
  for (int i = 0; i < 3; ++i) o[i] = R[i] * p[0] + R[3 + i] * p[1] + R[6 + i] * p[2];
}

// elementwise: y = (a + b) * tbl   (tbl may be null)
__global__ void add_scale_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                 const float* __restrict__ tbl, long n, float* __restrict__ y) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float v = a[i] + b[i];
  y[i] = tbl ? v * tbl[i] : v;
}
// y = x * tbl (tbl may be null; y may alias x)
__global__ void scale_kernel(const float* x, const float* __restrict__ tbl, long n, float* y) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  y[i] = tbl ? x[i] * tbl[i] : x[i];
}
void add_scale(hipStream_t st, const float* a, const float* b, const float* tbl, long n, float* y) {
  hipLaunchKernelGGL(add_scale_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, b, tbl, n, y);
}
void scale(hipStream_t st, const float* x, const float* tbl, long n, float* y) {
  hipLaunchKernelGGL(scale_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, tbl, n, y);
}

// ----------------------------------------------------------------- points
// One thread per (residue, head): global points R l + t of the q, k, v point
// projections, packed with the scalar parts (qpk, kpk, vpk).
__global__ void ipa_points_kernel(const float* __restrict__ P, const float* __restrict__ rig,
                                  int N, float* __restrict__ qpk, float* __restrict__ kpk,
                                  float* __restrict__ vpk) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N * H) return;
  const int n = i / H, h = i % H;
  const float* R = rig + n * 12;
  const float* t = R + 9;
  const float* p = P + (long)n * PROJ;
  float* q = qpk + (long)i * QKW;
  float* k = kpk + (long)i * QKW;
  float* v = vpk + (long)i * VW;
  for (int c = 0; c < SQK; ++c) {
    q[c] = SCALAR_W * p[OFF_QS + h * SQK + c];
    k[c] = p[OFF_KS + h * SQK + c];
  }
  for (int c = 0; c < SV; ++c) v[c] = p[OFF_VS + h * SV + c];
  for (int pt = 0; pt < PQK; ++pt) {
    float l[3], g[3];
#pragma unroll
    for (int x = 0; x < 3; ++x) l[x] = p[OFF_QP + h * 3 * PQK + x * PQK + pt];
    rot_apply(R, l, g);
#pragma unroll
    for (int x = 0; x < 3; ++x) q[SQK + pt * 3 + x] = g[x] + t[x];
#pragma unroll
    for (int x = 0; x < 3; ++x) l[x] = p[OFF_KP + h * 3 * PQK + x * PQK + pt];
    rot_apply(R, l, g);
#pragma unroll
    for (int x = 0; x < 3; ++x) k[SQK + pt * 3 + x] = g[x] + t[x];
  }
  for (int pt = 0; pt < PV; ++pt) {
    float l[3], g[3];
#pragma unroll
    for (int x = 0; x < 3; ++x) l[x] = p[OFF_VP + h * 3 * PV + x * PV + pt];
    rot_apply(R, l, g);
#pragma unroll
    for (int x = 0; x < 3; ++x) v[SV + pt * 3 + x] = g[x] + t[x];
  }
  q[28] = 1.f; q[29] = q[30] = q[31] = 0.f;
  k[28] = 1.f; k[29] = k[30] = k[31] = 0.f;
}

// ----------------------------------------------------------------- logits
// One wave per (head, query): logits over the keys (lane-strided), softmax.
template <int NJ>
__global__ __launch_bounds__(256) void ipa_logits_kernel(
    const float* __restrict__ qpk, const float* __restrict__ kpk, const float* __restrict__ b2d,
    const float* __restrict__ mask, const float* __restrict__ pw, int N,
    float* __restrict__ attn) {
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wid >= H * N) return;
  const int h = wid / N, q = wid % N;
  const float* qv = qpk + ((long)q * H + h) * QKW;
  float qr[28];
#pragma unroll
  for (int c = 0; c < 28; ++c) qr[c] = qv[c];
  const float w = pw[h], mq = mask[q];
  float lg[NJ];
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int k = lane + 64 * j;
    lg[j] = -INFINITY;
    if (k < N) {
      const float* kv = kpk + ((long)k * H + h) * QKW;
      float s = 0.f, d2 = 0.f;
#pragma unroll
      for (int c = 0; c < SQK; ++c) s += qr[c] * kv[c];
#pragma unroll
      for (int c = SQK; c < 28; ++c) { const float d = qr[c] - kv[c]; d2 += d * d; }
      // the mask term 1e5 (1 - m_q m_k): for a masked query it is the same
      // on every key, which the softmax ignores, so it is left out there --
      // in f32 it would round the row's logits to ~4e-3
      const float l = s - 0.5f * w * d2 + b2d[((long)h * N + q) * N + k] -
                      (mq != 0.f ? 1e5f * (1.f - mq * mask[k]) : 0.f);
      lg[j] = l * LOGIT_W;
      mx = fmaxf(mx, lg[j]);
    }
  }
  mx = group_max<64>(mx);
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int k = lane + 64 * j;
    lg[j] = k < N ? __expf(lg[j] - mx) : 0.f;
    sum += lg[j];
  }
  sum = group_sum<64>(sum);
  const float inv = 1.f / sum;
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const int k = lane + 64 * j;
    if (k < N) attn[((long)h * N + q) * N + k] = lg[j] * inv;
  }
}

// ---------------------------------------------------------------- readout
// One workgroup per query: scalar and point readouts (pairs (h, j<40)), the
// pair readout (thread = channel x half of the heads), then the points to
// the query's local frame and their norms.
template <int MN>  // the attention row's capacity: 512, or 1024 for longer N
__global__ __launch_bounds__(256) void ipa_readout_kernel(
    const float* __restrict__ attn, const float* __restrict__ vpk,
    const float* __restrict__ act2d, const float* __restrict__ rig, int N,
    float* __restrict__ fin) {
  __shared__ float at[H][MN];
  __shared__ float r40[H][VW];
  const int q = blockIdx.x, t = threadIdx.x;
  for (int i = t; i < H * N; i += 256) at[i / N][i % N] = attn[((long)(i / N) * N + q) * N + i % N];
  __syncthreads();
  for (int pr = t; pr < H * VW; pr += 256) {
    const int h = pr / VW, j = pr % VW;
    float s = 0.f;
    for (int k = 0; k < N; ++k) s += at[h][k] * vpk[((long)k * H + h) * VW + j];
    r40[h][j] = s;
  }
  {
    const int c = t & 127, h0 = (t >> 7) * 6;
    float acc[6] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const float* a2 = act2d + (long)q * N * CZ + c;
    for (int k = 0; k < N; ++k) {
      const float a = a2[(long)k * CZ];
#pragma unroll
      for (int j = 0; j < 6; ++j) acc[j] += at[h0 + j][k] * a;
    }
#pragma unroll
    for (int j = 0; j < 6; ++j) fin[(long)q * FIN + FIN_PAIR + (h0 + j) * CZ + c] = acc[j];
  }
  __syncthreads();
  float* f = fin + (long)q * FIN;
  if (t < H * SV) f[t] = r40[t / SV][t % SV];
  if (t < H * PV) {
    const int h = t / PV, p = t % PV;
    const float* R = rig + q * 12;
    float d[3], l[3];
#pragma unroll
    for (int x = 0; x < 3; ++x) d[x] = r40[h][SV + p * 3 + x] - R[9 + x];
    rot_apply_t(R, d, l);
    f[FIN_X + t] = l[0];
    f[FIN_Y + t] = l[1];
    f[FIN_Z + t] = l[2];
    f[FIN_NORM + t] = sqrtf(fmaxf(l[0] * l[0] + l[1] * l[1] + l[2] * l[2], DIST_EPS2));
  }
}

// ------------------------------------------------------- readout backward
// One workgroup per query.  From dfinal: the readouts' gradients (dres,
// written for the value GEMM), the query frame's gradient from the local
// conversion (added to drig[q]), d attn, the softmax backward (dlogit,
// scaled by sqrt(1/3), also accumulated into db2d_sum), and the pair
// readout's contribution to d LN(pair)[q] (added to dact2d[q]).
template <int MN>
__global__ __launch_bounds__(256) void ipa_readout_bwd_kernel(
    const float* __restrict__ dfin, const float* __restrict__ fin,
    const float* __restrict__ attn, const float* __restrict__ vpk,
    const float* __restrict__ act2d, const float* __restrict__ rig, int N,
    float* __restrict__ dres, float* __restrict__ drig, float* __restrict__ dlogit,
    float* __restrict__ db2d_sum, float* __restrict__ dact2d) {
  __shared__ float at[H][MN];
  __shared__ float da[H][MN];
  __shared__ float d40[H][VW];
  __shared__ float dp[H][CZ];
  __shared__ float rg[H * PV][12];
  __shared__ float sh[H];
  const int q = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const float* df = dfin + (long)q * FIN;
  const float* R = rig + q * 12;
  for (int i = t; i < H * N; i += 256) at[i / N][i % N] = attn[((long)(i / N) * N + q) * N + i % N];
  for (int i = t; i < H * CZ; i += 256) dp[i / CZ][i % CZ] = df[FIN_PAIR + i];
  if (t < H * SV) d40[t / SV][t % SV] = df[t];
  if (t < H * PV) {
    const int h = t / PV, p = t % PV;
    const float* f = fin + (long)q * FIN;
    const float l[3] = {f[FIN_X + t], f[FIN_Y + t], f[FIN_Z + t]};
    const float nrm = f[FIN_NORM + t];
    const float n2 = l[0] * l[0] + l[1] * l[1] + l[2] * l[2];
    const float dn = df[FIN_NORM + t];
    float dl[3] = {df[FIN_X + t], df[FIN_Y + t], df[FIN_Z + t]};
    if (n2 > DIST_EPS2) {
#pragma unroll
      for (int x = 0; x < 3; ++x) dl[x] += dn * l[x] / nrm;
    }
    // l = R^T (g - t):  dg = R dl,  dt -= dg,  dR[j][i] += dl_i (R l)_j
    float dg[3], gl[3];
    rot_apply(R, dl, dg);
    rot_apply(R, l, gl);
#pragma unroll
    for (int x = 0; x < 3; ++x) d40[h][SV + p * 3 + x] = dg[x];
#pragma unroll
    for (int j = 0; j < 3; ++j)
#pragma unroll
      for (int i = 0; i < 3; ++i) rg[t][j * 3 + i] = dl[i] * gl[j];
#pragma unroll
    for (int x = 0; x < 3; ++x) rg[t][9 + x] = -dg[x];
  }
  __syncthreads();
  if (t < 12) {
    float s = 0.f;
    for (int i = 0; i < H * PV; ++i) s += rg[i][t];
    drig[q * 12 + t] += s;
  }
  for (int i = t; i < H * VW; i += 256) dres[(long)q * H * VW + i] = d40[i / VW][i % VW];
  // d attn[h][k]: value readouts + pair readout
  for (int k = t; k < N; k += 256) {
    float acc[H];
    const float* vk = vpk + (long)k * H * VW;
#pragma unroll
    for (int h = 0; h < H; ++h) {
      float s = 0.f;
      for (int j = 0; j < VW; ++j) s += d40[h][j] * vk[h * VW + j];
      acc[h] = s;
    }
    const float4* a2 = reinterpret_cast<const float4*>(act2d + ((long)q * N + k) * CZ);
    for (int c4 = 0; c4 < CZ / 4; ++c4) {
      const float4 a = a2[c4];
#pragma unroll
      for (int h = 0; h < H; ++h)
        acc[h] += dp[h][c4 * 4] * a.x + dp[h][c4 * 4 + 1] * a.y + dp[h][c4 * 4 + 2] * a.z +
                  dp[h][c4 * 4 + 3] * a.w;
    }
#pragma unroll
    for (int h = 0; h < H; ++h) da[h][k] = acc[h];
  }
  __syncthreads();
  for (int h = wave; h < H; h += 4) {
    float s = 0.f;
    for (int k = lane; k < N; k += 64) s += at[h][k] * da[h][k];
    s = group_sum<64>(s);
    if (lane == 0) sh[h] = s;
  }
  __syncthreads();
  for (int i = t; i < H * N; i += 256) {
    const int h = i / N, k = i % N;
    const long o = ((long)h * N + q) * N + k;
    const float d = at[h][k] * (da[h][k] - sh[h]) * LOGIT_W;
    dlogit[o] = d;
    db2d_sum[o] += d;
  }
  // d LN(pair)[q][k][c] += sum_h attn[h][q][k] * dres_pair[q][h][c]
  {
    const int c = t & 127;
    for (int k = t >> 7; k < N; k += 2) {
      float s = 0.f;
#pragma unroll
      for (int h = 0; h < H; ++h) s += at[h][k] * dp[h][c];
      dact2d[((long)q * N + k) * CZ + c] += s;
    }
  }
}

// -------------------------------------------------------- points backward
// One thread per residue: gradients of the six projections (dP) from the
// logit GEMMs (T1 = dlogit . kpk, T2 = dlogit^T . qpk) and the value GEMM
// (dvpk), and the frame's gradient from the local -> global conversion.
__global__ void ipa_points_bwd_kernel(const float* __restrict__ T1, const float* __restrict__ T2,
                                      const float* __restrict__ dvpk, const float* __restrict__ qpk,
                                      const float* __restrict__ kpk, const float* __restrict__ vpk,
                                      const float* __restrict__ rig, const float* __restrict__ pw,
                                      int N, float* __restrict__ dP, float* __restrict__ drig) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const float* R = rig + n * 12;
  const float* t = R + 9;
  float* d = dP + (long)n * PROJ;
  float dR[9] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, dt[3] = {0.f, 0.f, 0.f};
  // g = R l + t:  dl = R^T dg,  dR[i][j] += dg_i l_j,  dt += dg
  auto point = [&](const float* g, const float* dg, float* dl) {
    float gm[3], l[3];
#pragma unroll
    for (int x = 0; x < 3; ++x) gm[x] = g[x] - t[x];
    rot_apply_t(R, gm, l);
    rot_apply_t(R, dg, dl);
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
      for (int j = 0; j < 3; ++j) dR[i * 3 + j] += dg[i] * l[j];
      dt[i] += dg[i];
    }
  };
  for (int h = 0; h < H; ++h) {
    const long i = (long)n * H + h;
    const float* t1 = T1 + i * QKW;
    const float* t2 = T2 + i * QKW;
    const float* dv = dvpk + i * VW;
    const float* qv = qpk + i * QKW;
    const float* kv = kpk + i * QKW;
    const float* vv = vpk + i * VW;
    for (int c = 0; c < SQK; ++c) {
      d[OFF_QS + h * SQK + c] = SCALAR_W * t1[c];
      d[OFF_KS + h * SQK + c] = t2[c];
    }
    for (int c = 0; c < SV; ++c) d[OFF_VS + h * SV + c] = dv[c];
    const float w = pw[h], rs = t1[28], cs = t2[28];
    for (int p = 0; p < PQK; ++p) {
      float dg[3], dl[3];
#pragma unroll
      for (int x = 0; x < 3; ++x) dg[x] = -w * (qv[SQK + p * 3 + x] * rs - t1[SQK + p * 3 + x]);
      point(qv + SQK + p * 3, dg, dl);
#pragma unroll
      for (int x = 0; x < 3; ++x) d[OFF_QP + h * 3 * PQK + x * PQK + p] = dl[x];
#pragma unroll
      for (int x = 0; x < 3; ++x) dg[x] = -w * (kv[SQK + p * 3 + x] * cs - t2[SQK + p * 3 + x]);
      point(kv + SQK + p * 3, dg, dl);
#pragma unroll
      for (int x = 0; x < 3; ++x) d[OFF_KP + h * 3 * PQK + x * PQK + p] = dl[x];
    }
    for (int p = 0; p < PV; ++p) {
      float dg[3], dl[3];
#pragma unroll
      for (int x = 0; x < 3; ++x) dg[x] = dv[SV + p * 3 + x];
      point(vv + SV + p * 3, dg, dl);
#pragma unroll
      for (int x = 0; x < 3; ++x) d[OFF_VP + h * 3 * PV + x * PV + p] = dl[x];
    }
  }
  float* o = drig + n * 12;
#pragma unroll
  for (int i = 0; i < 9; ++i) o[i] += dR[i];
#pragma unroll
  for (int i = 0; i < 3; ++i) o[9 + i] += dt[i];
}

// ------------------------------------------------------------ rigid update
// rigid' = rigid @ (R_u(1, x, y, z normalised), t_u); traj = [R' | 20 t'].
__device__ __forceinline__ void quat_rot(const float* f, float* Ru, float* qn, float* inv_out) {
  float w = 1.f, x = f[0], y = f[1], z = f[2];
  const float inv = rsqrtf(fmaxf(QUAT_EPS, w * w + x * x + y * y + z * z));
  w *= inv; x *= inv; y *= inv; z *= inv;
  Ru[0] = 1.f - 2.f * (y * y + z * z); Ru[1] = 2.f * (x * y - w * z); Ru[2] = 2.f * (x * z + w * y);
  Ru[3] = 2.f * (x * y + w * z); Ru[4] = 1.f - 2.f * (x * x + z * z); Ru[5] = 2.f * (y * z - w * x);
  Ru[6] = 2.f * (x * z - w * y); Ru[7] = 2.f * (y * z + w * x); Ru[8] = 1.f - 2.f * (x * x + y * y);
  qn[0] = w; qn[1] = x; qn[2] = y; qn[3] = z;
  *inv_out = inv;
}

__global__ void rigid_update_kernel(const float* __restrict__ flat, const float* __restrict__ rin,
                                    int N, float* __restrict__ rout, float* __restrict__ traj) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const float* f = flat + n * 6;
  const float* R = rin + n * 12;
  float Ru[9], qn[4], inv;
  quat_rot(f, Ru, qn, &inv);
  float o[12];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      o[i * 3 + j] = R[i * 3] * Ru[j] + R[i * 3 + 1] * Ru[3 + j] + R[i * 3 + 2] * Ru[6 + j];
  float tu[3] = {f[3], f[4], f[5]}, rt[3];
  rot_apply(R, tu, rt);
#pragma unroll
  for (int i = 0; i < 3; ++i) o[9 + i] = rt[i] + R[9 + i];
#pragma unroll
  for (int i = 0; i < 12; ++i) rout[n * 12 + i] = o[i];
  float* tr = traj + n * 12;  // [3][4]
#pragma unroll
  for (int i = 0; i < 3; ++i) {
#pragma unroll
    for (int j = 0; j < 3; ++j) tr[i * 4 + j] = o[i * 3 + j];
    tr[i * 4 + 3] = POSITION_SCALE * o[9 + i];
  }
}

// From the cotangent of rigid' (drout, plus the trajectory's) to dflat and
// the input rigid's gradient (written, not added).
__global__ void rigid_update_bwd_kernel(const float* __restrict__ flat, const float* __restrict__ rin,
                                        const float* __restrict__ drout,
                                        const float* __restrict__ dtraj, int N,
                                        float* __restrict__ dflat, float* __restrict__ drin) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  const float* f = flat + n * 6;
  const float* R = rin + n * 12;
  float Ru[9], qn[4], inv;
  quat_rot(f, Ru, qn, &inv);
  float dRo[9], dto[3];
#pragma unroll
  for (int i = 0; i < 9; ++i) dRo[i] = drout ? drout[n * 12 + i] : 0.f;
#pragma unroll
  for (int i = 0; i < 3; ++i) dto[i] = drout ? drout[n * 12 + 9 + i] : 0.f;
  if (dtraj) {
    const float* tr = dtraj + n * 12;
#pragma unroll
    for (int i = 0; i < 3; ++i) {
#pragma unroll
      for (int j = 0; j < 3; ++j) dRo[i * 3 + j] += tr[i * 4 + j];
      dto[i] += POSITION_SCALE * tr[i * 4 + 3];
    }
  }
  // R' = R Ru, t' = R tu + t
  const float tu[3] = {f[3], f[4], f[5]};
  float G[9], dtu[3];
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      G[i * 3 + j] = R[i] * dRo[j] + R[3 + i] * dRo[3 + j] + R[6 + i] * dRo[6 + j];  // R^T dR'
  rot_apply_t(R, dto, dtu);
  float* o = drin + n * 12;
#pragma unroll
  for (int i = 0; i < 3; ++i)
#pragma unroll
    for (int j = 0; j < 3; ++j)
      o[i * 3 + j] = dRo[i * 3] * Ru[j * 3] + dRo[i * 3 + 1] * Ru[j * 3 + 1] +
                     dRo[i * 3 + 2] * Ru[j * 3 + 2] + dto[i] * tu[j];  // dR' Ru^T + dt' tu^T
#pragma unroll
  for (int i = 0; i < 3; ++i) o[9 + i] = dto[i];
  // d(normalised quaternion) from G = dRu
  const float w = qn[0], x = qn[1], y = qn[2], z = qn[3];
  const float dw = 2.f * (-z * G[1] + y * G[2] + z * G[3] - x * G[5] - y * G[6] + x * G[7]);
  const float dx = 2.f * (y * G[1] + z * G[2] + y * G[3] - 2.f * x * G[4] - w * G[5] + z * G[6] +
                          w * G[7] - 2.f * x * G[8]);
  const float dy = 2.f * (-2.f * y * G[0] + x * G[1] + w * G[2] + x * G[3] + z * G[5] - w * G[6] +
                          z * G[7] - 2.f * y * G[8]);
  const float dz = 2.f * (-2.f * z * G[0] - w * G[1] + x * G[2] + w * G[3] - 2.f * z * G[4] +
                          y * G[5] + x * G[6] + y * G[7]);
  // qn = q * inv, inv = rsqrt(max(eps, |q|^2)), q = (1, f0, f1, f2)
  const float raw2 = 1.f + f[0] * f[0] + f[1] * f[1] + f[2] * f[2];
  const float dot = w * dw + x * dx + y * dy + z * dz;  // qn . dqn
  const float cl = raw2 > QUAT_EPS ? 1.f : 0.f;         // the clip has no slope
  float* df = dflat + n * 6;
  df[0] = inv * (dx - cl * x * dot);
  df[1] = inv * (dy - cl * y * dot);
  df[2] = inv * (dz - cl * z * dot);
  df[3] = dtu[0];
  df[4] = dtu[1];
  df[5] = dtu[2];
}

// d LN(pair)[m][c] += sum_h db2d_sum[h][m] * w2d[c][h]
__global__ void b2d_bwd_kernel(const float* __restrict__ db2d, const float* __restrict__ w2d,
                               long M, float* __restrict__ dact2d) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * CZ) return;
  const long m = i / CZ;
  const int c = (int)(i % CZ);
  float s = 0.f;
#pragma unroll
  for (int h = 0; h < H; ++h) s += db2d[(long)h * M + m] * w2d[c * H + h];
  dact2d[i] += s;
}

// keys[(it*2 + j)*2 + {0,1}] = split(split(key, depth)[it], 3)[1 + j]
__global__ void fold_keys_kernel(const uint32_t* __restrict__ key, int depth,
                                 uint32_t* __restrict__ out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  for (int it = 0; it < depth; ++it) {
    uint32_t a0 = 0u, a1 = (uint32_t)it;
    threefry2x32(key[0], key[1], a0, a1);
    for (int j = 0; j < 2; ++j) {
      uint32_t b0 = 0u, b1 = (uint32_t)(1 + j);
      threefry2x32(a0, a1, b0, b1);
      out[(it * 2 + j) * 2] = b0;
      out[(it * 2 + j) * 2 + 1] = b1;
    }
  }
}

}  // namespace

// ---------------------------------------------------------------- weights
FoldW fold_weights(WeightStore& ws) {
  FoldW w;
  const std::string P = "param/", F = P + "fold_iteration/", I = F + "invariant_point_attention/";
  auto need_shape = [&](const std::string& n, size_t count) {
    const HostTensor& t = ws.host(n);
    if (t.data.size() != count) throw std::runtime_error("fold: " + n + " has the wrong size");
  };
  need_shape(I + "output_projection/weights", (size_t)FIN * CS);
  need_shape(F + "quat_rigid/rigid/weights", (size_t)CS * 6);
  w.ln_s_g = ws.f32(P + "single_layer_norm/scale");
  w.ln_s_b = ws.f32(P + "single_layer_norm/offset");
  w.wi = ws.f32(P + "initial_projection/weights");
  w.bi = ws.f32(P + "initial_projection/bias");
  w.ln_z_g = ws.f32(P + "pair_layer_norm/scale");
  w.ln_z_b = ws.f32(P + "pair_layer_norm/offset");
  const char* names[6] = {"q_scalar_projection", "k_scalar_projection", "v_scalar_projection",
                          "q_point_projection/point_projection",
                          "k_point_projection/point_projection",
                          "v_point_projection/point_projection"};
  const int width[6] = {H * SQK, H * SQK, H * SV, H * PQK * 3, H * PQK * 3, H * PV * 3};
  w.wcat = ws.derived<float>("fold.wcat", [&] {
    std::vector<float> c((size_t)CS * PROJ, 0.f);
    int off = 0;
    for (int m = 0; m < 6; ++m) {
      const HostTensor& t = ws.host(I + names[m] + "/weights");
      if (t.data.size() != (size_t)CS * width[m]) throw std::runtime_error("fold: projection size");
      for (int r = 0; r < CS; ++r)
        for (int j = 0; j < width[m]; ++j) c[(size_t)r * PROJ + off + j] = t.data[(size_t)r * width[m] + j];
      off += width[m];
    }
    return c;
  });
  w.bcat = ws.derived<float>("fold.bcat", [&] {
    std::vector<float> c(PROJ, 0.f);
    int off = 0;
    for (int m = 0; m < 6; ++m) {
      const std::string bn = I + names[m] + "/bias";  // the scalar biases may be absent (zero)
      if (ws.has(bn)) {
        const HostTensor& t = ws.host(bn);
        if (t.data.size() != (size_t)width[m]) throw std::runtime_error("fold: " + bn + " has the wrong size");
        for (int j = 0; j < width[m]; ++j) c[off + j] = t.data[j];
      }
      off += width[m];
    }
    return c;
  });
  w.w2d = ws.f32(I + "attention_2d/weights");
  w.b2d = ws.f32(I + "attention_2d/bias");
  w.wo = ws.f32(I + "output_projection/weights");
  w.bo = ws.f32(I + "output_projection/bias");
  w.pw = ws.derived<float>("fold.point_weights", [&] {
    // sqrt(1 / (P_qk * 9/2)) * softplus(raw), softplus = logaddexp(x, 0)
    const HostTensor& t = ws.host(I + "trainable_point_weights");
    std::vector<float> o(H);
    for (int h = 0; h < H; ++h) {
      const double x = t.data[h];
      const double sp = x > 0 ? x + std::log1p(std::exp(-x)) : std::log1p(std::exp(x));
      o[h] = (float)(std::sqrt(1.0 / (PQK * 4.5)) * sp);
    }
    return o;
  });
  w.ln1_g = ws.f32(F + "attention_layer_norm/scale");
  w.ln1_b = ws.f32(F + "attention_layer_norm/offset");
  w.ln2_g = ws.f32(F + "transition_layer_norm/scale");
  w.ln2_b = ws.f32(F + "transition_layer_norm/offset");
  const char* tn[3] = {"transition", "transition_1", "transition_2"};
  for (int i = 0; i < 3; ++i) {
    w.wt[i] = ws.f32(F + tn[i] + "/weights");
    w.bt[i] = ws.f32(F + tn[i] + "/bias");
  }
  w.wq = ws.f32(F + "quat_rigid/rigid/weights");
  w.bq = ws.f32(F + "quat_rigid/rigid/bias");
  return w;
}

// --------------------------------------------------------------- save-set
namespace {
template <class A>
struct FoldIterSave {
  float *rig, *qpk, *kpk, *vpk, *attn, *fin, *x1, *m1, *r1, *t1, *t2, *x3, *m3, *r3, *flat;
  FoldIterSave(A& a, int N) {
    rig = a.template take<float>((size_t)N * 12);
    qpk = a.template take<float>((size_t)N * H * QKW);
    kpk = a.template take<float>((size_t)N * H * QKW);
    vpk = a.template take<float>((size_t)N * H * VW);
    attn = a.template take<float>((size_t)H * N * N);
    fin = a.template take<float>((size_t)N * FIN);
    x1 = a.template take<float>((size_t)N * CS);
    m1 = a.template take<float>(N);
    r1 = a.template take<float>(N);
    t1 = a.template take<float>((size_t)N * CS);
    t2 = a.template take<float>((size_t)N * CS);
    x3 = a.template take<float>((size_t)N * CS);
    m3 = a.template take<float>(N);
    r3 = a.template take<float>(N);
    flat = a.template take<float>((size_t)N * 6);
  }
};
template <class A>
struct FoldSave {
  float *sm, *sr, *act2d, *zm, *zr, *b2d, *tbl;
  uint32_t* keys;
  size_t iter0 = 0, per_iter = 0;
  FoldSave(A& a, int N, int depth) {
    sm = a.template take<float>(N);
    sr = a.template take<float>(N);
    act2d = a.template take<float>((size_t)N * N * CZ);
    zm = a.template take<float>((size_t)N * N);
    zr = a.template take<float>((size_t)N * N);
    b2d = a.template take<float>((size_t)H * N * N);
    tbl = a.template take<float>((size_t)depth * 2 * N * CS);
    keys = a.template take<uint32_t>((size_t)depth * 4);
  }
};
}  // namespace

size_t fold_save_bytes(int N, int depth) {
  Sizer s;
  FoldSave<Sizer> g(s, N, depth);
  const size_t head = s.off;
  Sizer it;
  FoldIterSave<Sizer> one(it, N);
  return head + (size_t)depth * it.off;
}

static void fold_check(int N, int depth) {
  if (N <= 0 || N > MAXN) throw std::runtime_error("fold: N must be in 1..1024");
  if (depth <= 0) throw std::runtime_error("fold: depth must be positive");
}

static FoldIterSave<Carver> iter_save(void* save, int N, int depth, int it) {
  Sizer s;
  FoldSave<Sizer> g(s, N, depth);
  Sizer one;
  FoldIterSave<Sizer> o(one, N);
  Carver c(reinterpret_cast<char*>(save) + s.off + (size_t)it * one.off);
  return FoldIterSave<Carver>(c, N);
}

template <int NJ>
static void launch_logits(hipStream_t st, const float* qpk, const float* kpk, const float* b2d,
                          const float* mask, const float* pw, int N, float* attn) {
  hipLaunchKernelGGL((ipa_logits_kernel<NJ>), dim3((unsigned)((H * N + 3) / 4)), dim3(256), 0, st,
                     qpk, kpk, b2d, mask, pw, N, attn);
}

// ------------------------------------------------------------------ forward

// rigid frames [N][12] (rotation row-major, then translation) set to the identity
__global__ void ident_frames_kernel(float* __restrict__ r, int N) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= N * 12) return;
  const int k = e % 12;
  r[e] = (k == 0 || k == 4 || k == 8) ? 1.f : 0.f;
}

// Initial frames from atom positions (folding_multimer.py:508-515 with
// initial_atom_pos; all_atom_multimer.py:943-966 and
// geometry/rotation_matrix.py:79-99): R's columns are e0 = unit(C - CA),
// e1 = unit((N - CA) minus its e0 part), e2 = e0 x e1, each unit() clipping
// the norm at 1e-6 (an all-zero row gives the zero matrix, as in the
// multimer model); t = CA / position_scale.  pos: atom37 [N][37][3].
__global__ void ref_frames_kernel(const float* __restrict__ pos, int N, float* __restrict__ r) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const float* p = pos + (long)i * 37 * 3;
  float e0[3], e1[3];
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    e0[k] = p[2 * 3 + k] - p[1 * 3 + k];
    e1[k] = p[0 * 3 + k] - p[1 * 3 + k];
  }
  const float n0 = sqrtf(fmaxf(e0[0] * e0[0] + e0[1] * e0[1] + e0[2] * e0[2], 1e-12f));
#pragma unroll
  for (int k = 0; k < 3; ++k) e0[k] /= n0;
  const float c = e1[0] * e0[0] + e1[1] * e0[1] + e1[2] * e0[2];
#pragma unroll
  for (int k = 0; k < 3; ++k) e1[k] -= c * e0[k];
  const float n1 = sqrtf(fmaxf(e1[0] * e1[0] + e1[1] * e1[1] + e1[2] * e1[2], 1e-12f));
#pragma unroll
  for (int k = 0; k < 3; ++k) e1[k] /= n1;
  const float e2[3] = {e0[1] * e1[2] - e0[2] * e1[1], e0[2] * e1[0] - e0[0] * e1[2],
                       e0[0] * e1[1] - e0[1] * e1[0]};
  float* o = r + (long)i * 12;
#pragma unroll
  for (int k = 0; k < 3; ++k) {
    o[k * 3 + 0] = e0[k];
    o[k * 3 + 1] = e1[k];
    o[k * 3 + 2] = e2[k];
    o[9 + k] = p[1 * 3 + k] * (1.f / POSITION_SCALE);
  }
}

void fold_fwd(hipStream_t st, const FoldW& w, int N, int depth, const float* single,
              const float* pair, const float* mask, const uint32_t* key, const uint32_t* enabled,
              bool dropout, float* act_out, float* traj, void* save, const float* init_pos37) {
  fold_check(N, depth);
  nonnull(single, "fold single"); nonnull(pair, "fold pair"); nonnull(mask, "fold mask");
  nonnull(act_out, "fold act_out"); nonnull(traj, "fold traj"); nonnull(save, "fold save");
  Carver cv(save);
  FoldSave<Carver> sv(cv, N, depth);
  const long M2 = (long)N * N;
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  Sizer need;
  need.take<float>((size_t)N * PROJ);
  for (int i = 0; i < 5; ++i) need.take<float>((size_t)N * CS);
  need.take<float>((size_t)N * 12 * 2);
  ar.reset(st, need.off);
  float* P = ar.take_n<float>((size_t)N * PROJ);
  float* act = ar.take_n<float>((size_t)N * CS);
  float* a0 = ar.take_n<float>((size_t)N * CS);
  float* ipo = ar.take_n<float>((size_t)N * CS);
  float* a2 = ar.take_n<float>((size_t)N * CS);
  float* a4 = ar.take_n<float>((size_t)N * CS);
  float* rigA = ar.take_n<float>((size_t)N * 12);
  float* rigB = ar.take_n<float>((size_t)N * 12);

  if (dropout) {
    if (!key) throw std::runtime_error("fold: dropout needs a key");
    hipLaunchKernelGGL(fold_keys_kernel, dim3(1), dim3(64), 0, st, key, depth, sv.keys);
    for (int it = 0; it < depth; ++it)
      for (int j = 0; j < 2; ++j)
        dropout_table_dev(st, sv.tbl + ((size_t)it * 2 + j) * N * CS, N, CS,
                          sv.keys + (it * 2 + j) * 2, enabled, 1.0f - 0.1f);
  }
  {
    KTimed kt("fold.prologue", st);
    ln_f32_rows_fwd(st, single, N, CS, w.ln_s_g, w.ln_s_b, a0, sv.sm, sv.sr);
    GemmF32 g = gemm_rows(N, CS, CS, a0, w.wi, act);
    g.bias = w.bi;
    gemm_f32(st, g, "fold.gemm_init");
    ln_f32_rows_fwd(st, pair, M2, CZ, w.ln_z_g, w.ln_z_b, sv.act2d, sv.zm, sv.zr);
    // b2d[h][m] = act2d[m] . w2d[:, h] + b[h]
    GemmF32 b = gemm_rows((int)M2, H, CZ, sv.act2d, w.w2d, sv.b2d);
    b.c_sm = 1; b.c_sn = M2;
    b.bias = w.b2d;
    gemm_f32(st, b, "fold.gemm_b2d");
    // identity frames (or those of the given atoms), written on the device
    // (no host copy, no stream sync)
    if (init_pos37)
      hipLaunchKernelGGL(ref_frames_kernel, dim3((N + 127) / 128), dim3(128), 0, st, init_pos37, N,
                         rigA);
    else
      hipLaunchKernelGGL(ident_frames_kernel, dim3((N * 12 + 255) / 256), dim3(256), 0, st, rigA,
                         N);
  }
  const int NJ = (N + 63) / 64;
  for (int it = 0; it < depth; ++it) {
    FoldIterSave<Carver> s = iter_save(save, N, depth, it);
    const float* tb1 = dropout ? sv.tbl + ((size_t)it * 2) * N * CS : nullptr;
    const float* tb2 = dropout ? sv.tbl + ((size_t)it * 2 + 1) * N * CS : nullptr;
    BC2N_HIP(hipMemcpyAsync(s.rig, rigA, (size_t)N * 12 * 4, hipMemcpyDeviceToDevice, st));
    {
      KTimed kt("fold.ipa", st);
      GemmF32 g = gemm_rows(N, PROJ, CS, act, w.wcat, P);
      g.bias = w.bcat;
      gemm_f32(st, g, "fold.gemm_proj");
      hipLaunchKernelGGL(ipa_points_kernel, dim3((N * H + 127) / 128), dim3(128), 0, st, P, s.rig,
                         N, s.qpk, s.kpk, s.vpk);
      switch (NJ) {
        case 1: launch_logits<1>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
        case 2: launch_logits<2>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
        case 3: launch_logits<3>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
        case 4: launch_logits<4>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
        case 5: launch_logits<5>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
        case 6: launch_logits<6>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
        case 7: launch_logits<7>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
        case 8: launch_logits<8>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
        case 9: case 10: launch_logits<10>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
        case 11: case 12: launch_logits<12>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
        default: launch_logits<16>(st, s.qpk, s.kpk, sv.b2d, mask, w.pw, N, s.attn); break;
      }
      if (N <= 512)
        hipLaunchKernelGGL(ipa_readout_kernel<512>, dim3(N), dim3(256), 0, st, s.attn, s.vpk,
                           sv.act2d, s.rig, N, s.fin);
      else
        hipLaunchKernelGGL(ipa_readout_kernel<MAXN>, dim3(N), dim3(256), 0, st, s.attn, s.vpk,
                           sv.act2d, s.rig, N, s.fin);
      GemmF32 o = gemm_rows(N, CS, FIN, s.fin, w.wo, ipo);
      o.bias = w.bo;
      gemm_f32(st, o, "fold.gemm_out");
    }
    {
      KTimed kt("fold.transition", st);
      add_scale(st, act, ipo, tb1, (long)N * CS, s.x1);
      ln_f32_rows_fwd(st, s.x1, N, CS, w.ln1_g, w.ln1_b, a2, s.m1, s.r1);
      GemmF32 g1 = gemm_rows(N, CS, CS, a2, w.wt[0], s.t1);
      g1.bias = w.bt[0]; g1.relu = true;
      gemm_f32(st, g1, "fold.gemm_t1");
      GemmF32 g2 = gemm_rows(N, CS, CS, s.t1, w.wt[1], s.t2);
      g2.bias = w.bt[1]; g2.relu = true;
      gemm_f32(st, g2, "fold.gemm_t2");
      // x3 = (t2 W3 + b3 + a2) * tbl2
      GemmF32 g3 = gemm_rows(N, CS, CS, s.t2, w.wt[2], s.x3);
      g3.bias = w.bt[2]; g3.add = a2;
      gemm_f32(st, g3, "fold.gemm_t3");
      scale(st, s.x3, tb2, (long)N * CS, s.x3);
      ln_f32_rows_fwd(st, s.x3, N, CS, w.ln2_g, w.ln2_b, a4, s.m3, s.r3);
      GemmF32 gq = gemm_rows(N, 6, CS, a4, w.wq, s.flat);
      gq.bias = w.bq;
      gemm_f32(st, gq, "fold.gemm_quat");
      hipLaunchKernelGGL(rigid_update_kernel, dim3((N + 127) / 128), dim3(128), 0, st, s.flat,
                         s.rig, N, rigB, traj + (size_t)it * N * 12);
    }
    std::swap(rigA, rigB);
    std::swap(act, a4);
  }
  BC2N_HIP(hipMemcpyAsync(act_out, act, (size_t)N * CS * 4, hipMemcpyDeviceToDevice, st));
}

// ----------------------------------------------------------------- backward
void fold_bwd(hipStream_t st, const FoldW& w, int N, int depth, const float* single,
              const float* pair, const float* mask, bool dropout, const void* save,
              const float* d_act, const float* d_traj, float* dsingle, float* dpair) {
  fold_check(N, depth);
  nonnull(single, "fold single"); nonnull(pair, "fold pair"); nonnull(mask, "fold mask");
  nonnull(save, "fold save"); nonnull(dsingle, "fold dsingle"); nonnull(dpair, "fold dpair");
  (void)mask;
  Carver cv(const_cast<void*>(save));
  FoldSave<Carver> sv(cv, N, depth);
  const long M2 = (long)N * N;
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  Sizer need;
  need.take<float>((size_t)N * FIN);      // dfin
  need.take<float>((size_t)N * H * VW);   // dres
  need.take<float>((size_t)N * H * VW);   // dvpk
  need.take<float>((size_t)H * N * N);    // dlogit
  need.take<float>((size_t)H * N * N);    // db2d_sum
  need.take<float>((size_t)N * H * QKW);  // T1
  need.take<float>((size_t)N * H * QKW);  // T2
  need.take<float>((size_t)N * PROJ);     // dP
  for (int i = 0; i < 6; ++i) need.take<float>((size_t)N * CS);
  need.take<float>((size_t)N * 12 * 2);
  need.take<float>((size_t)N * 6);
  ar.reset(st, need.off);
  float* dfin = ar.take_n<float>((size_t)N * FIN);
  float* dres = ar.take_n<float>((size_t)N * H * VW);
  float* dvpk = ar.take_n<float>((size_t)N * H * VW);
  float* dlog = ar.take_n<float>((size_t)H * N * N);
  float* db2d = ar.take_n<float>((size_t)H * N * N);
  float* T1 = ar.take_n<float>((size_t)N * H * QKW);
  float* T2 = ar.take_n<float>((size_t)N * H * QKW);
  float* dP = ar.take_n<float>((size_t)N * PROJ);
  float* da = ar.take_n<float>((size_t)N * CS);    // d act at the iteration output
  float* dx = ar.take_n<float>((size_t)N * CS);
  float* dt2 = ar.take_n<float>((size_t)N * CS);
  float* dt1 = ar.take_n<float>((size_t)N * CS);
  float* da2 = ar.take_n<float>((size_t)N * CS);
  float* dnext = ar.take_n<float>((size_t)N * CS);
  float* drA = ar.take_n<float>((size_t)N * 12);
  float* drB = ar.take_n<float>((size_t)N * 12);
  float* dflat = ar.take_n<float>((size_t)N * 6);
  // d LN(pair) accumulates in dpair, then the LN backward runs in place
  zero_f32(st, dpair, (long)M2 * CZ);
  zero_f32(st, db2d, (long)H * M2);
  if (d_act) BC2N_HIP(hipMemcpyAsync(da, d_act, (size_t)N * CS * 4, hipMemcpyDeviceToDevice, st));
  else zero_f32(st, da, (long)N * CS);
  zero_f32(st, drA, (long)N * 12);  // d rigid' of the last iteration

  for (int it = depth - 1; it >= 0; --it) {
    FoldIterSave<Carver> s = iter_save(const_cast<void*>(save), N, depth, it);
    const float* tb1 = dropout ? sv.tbl + ((size_t)it * 2) * N * CS : nullptr;
    const float* tb2 = dropout ? sv.tbl + ((size_t)it * 2 + 1) * N * CS : nullptr;
    {
      KTimed kt("fold.transition_bwd", st);
      hipLaunchKernelGGL(rigid_update_bwd_kernel, dim3((N + 127) / 128), dim3(128), 0, st, s.flat,
                         s.rig, drA, d_traj ? d_traj + (size_t)it * N * 12 : nullptr, N, dflat,
                         drB);
      // da4 += dflat Wq^T
      GemmF32 gq = gemm_rows(N, CS, 6, dflat, w.wq, da, true);
      gq.beta = 1.f;
      gemm_f32(st, gq, "fold.gemm_quat_dx");
      ln_f32_rows_bwd(st, da, s.x3, N, CS, w.ln2_g, s.m3, s.r3, dx);  // dx3
      scale(st, dx, tb2, (long)N * CS, dx);                       // da3
      // dt2 = (da3 W3^T) * [t2 > 0]
      GemmF32 g3 = gemm_rows(N, CS, CS, dx, w.wt[2], dt2, true);
      g3.gate = s.t2; g3.gate_is_mask = true;
      gemm_f32(st, g3, "fold.gemm_t3_dx");
      GemmF32 g2 = gemm_rows(N, CS, CS, dt2, w.wt[1], dt1, true);
      g2.gate = s.t1; g2.gate_is_mask = true;
      gemm_f32(st, g2, "fold.gemm_t2_dx");
      // da2 = dt1 W1^T + da3
      GemmF32 g1 = gemm_rows(N, CS, CS, dt1, w.wt[0], da2, true);
      g1.add = dx;
      gemm_f32(st, g1, "fold.gemm_t1_dx");
      ln_f32_rows_bwd(st, da2, s.x1, N, CS, w.ln1_g, s.m1, s.r1, dx);  // dx1
      scale(st, dx, tb1, (long)N * CS, dx);                       // da1 = d act_in (residual) = d ipa
    }
    {
      KTimed kt("fold.ipa_bwd", st);
      GemmF32 go = gemm_rows(N, FIN, CS, dx, w.wo, dfin, true);
      gemm_f32(st, go, "fold.gemm_out_dx");
      if (N <= 512)
        hipLaunchKernelGGL(ipa_readout_bwd_kernel<512>, dim3(N), dim3(256), 0, st, dfin, s.fin,
                           s.attn, s.vpk, sv.act2d, s.rig, N, dres, drB, dlog, db2d, dpair);
      else
        hipLaunchKernelGGL(ipa_readout_bwd_kernel<MAXN>, dim3(N), dim3(256), 0, st, dfin, s.fin,
                           s.attn, s.vpk, sv.act2d, s.rig, N, dres, drB, dlog, db2d, dpair);
      // dvpk[k][h][j] = sum_q attn[h][q][k] dres[q][h][j]
      GemmF32 gv;
      gv.M = N; gv.N = VW; gv.K = N; gv.batch = H;
      gv.A = s.attn; gv.a_sm = 1; gv.a_sk = N; gv.a_sb = M2;
      gv.B = dres; gv.b_sk = H * VW; gv.b_sn = 1; gv.b_sb = VW;
      gv.C = dvpk; gv.c_sm = H * VW; gv.c_sn = 1; gv.c_sb = VW;
      gemm_f32(st, gv, "fold.gemm_dv");
      // T1[q][h] = sum_k dlogit[h][q][k] kpk[k][h];  T2[k][h] = sum_q dlogit[h][q][k] qpk[q][h]
      GemmF32 g1;
      g1.M = N; g1.N = QKW; g1.K = N; g1.batch = H;
      g1.A = dlog; g1.a_sm = N; g1.a_sk = 1; g1.a_sb = M2;
      g1.B = s.kpk; g1.b_sk = H * QKW; g1.b_sn = 1; g1.b_sb = QKW;
      g1.C = T1; g1.c_sm = H * QKW; g1.c_sn = 1; g1.c_sb = QKW;
      gemm_f32(st, g1, "fold.gemm_dq");
      GemmF32 g2 = g1;
      g2.A = dlog; g2.a_sm = 1; g2.a_sk = N;
      g2.B = s.qpk;
      g2.C = T2;
      gemm_f32(st, g2, "fold.gemm_dk");
      hipLaunchKernelGGL(ipa_points_bwd_kernel, dim3((N + 63) / 64), dim3(64), 0, st, T1, T2, dvpk,
                         s.qpk, s.kpk, s.vpk, s.rig, w.pw, N, dP, drB);
      // d act_in = da1 + dP Wcat^T
      GemmF32 gp = gemm_rows(N, CS, PROJ, dP, w.wcat, dnext, true);
      gp.add = dx;
      gemm_f32(st, gp, "fold.gemm_proj_dx");
    }
    std::swap(da, dnext);
    std::swap(drA, drB);
  }
  {
    KTimed kt("fold.prologue_bwd", st);
    // act = Linear(LN(single)):  d LN(single) = da Wi^T
    GemmF32 g = gemm_rows(N, CS, CS, da, w.wi, dx, true);
    gemm_f32(st, g, "fold.gemm_init_dx");
    ln_f32_rows_bwd(st, dx, single, N, CS, w.ln_s_g, sv.sm, sv.sr, dsingle);
    hipLaunchKernelGGL(b2d_bwd_kernel, dim3((unsigned)((M2 * CZ + 255) / 256)), dim3(256), 0, st,
                       db2d, w.w2d, M2, dpair);
    ln_f32_rows_bwd(st, dpair, pair, M2, CZ, w.ln_z_g, sv.zm, sv.zr, dpair);
  }
}

}  // namespace bc2n
