// MSA column global attention (the extra-MSA stack's column module), forward
// and backward, f32.
//
// Reference: bindcraft/af/alphafold/model/modules.py:619-672
// (MSAColumnGlobalAttention: per residue column, LayerNorm, then
// GlobalAttention over the sequences) and :403-497 (GlobalAttention: one
// masked-mean query per column and head, a single shared key/value head,
// softmax over the sequences with bias 1e9 (mask - 1), per-sequence sigmoid
// gates, output projection); utils.py mask_mean (eps 1e-10).
//
// The module is tiny next to the pair track (N_extra x N x 64), so it runs in
// f32: the projections are f32 MFMA GEMMs over all S*N rows at once
//   kvg = LN(msa) [Wk | Wv | Wg] + [0 | 0 | bg]      [S*N][DK + DV + H*DV]
//   out = msa + tbl * ((sigmoid(G) * wa[col]) Wo + bo)
// and the per-column softmax over the sequences is one workgroup per column.
#include "gemm_f32.h"
#include "kernels.h"
#include "modules.h"

namespace bc2n {

namespace {

// per column j: masked-mean query, q = qavg Wq / sqrt(DK), weights over the
// sequences w[j][h][s] (softmax), weighted average wa[j][h][dv]
__global__ __launch_bounds__(256) void glob_attn_fwd_kernel(
    const float* __restrict__ xn, const float* __restrict__ kvg, const float* __restrict__ mask,
    const float* __restrict__ wq, int S, int N, int C, int H, int DK, int DV,
    float* __restrict__ q_out, float* __restrict__ w, float* __restrict__ wa) {
  __shared__ float qa[256], qs[256], hm[16], hs[16];
  const int j = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int ld = DK + DV + H * DV;
  if (t < C) {
    float s = 0.f, ms = 0.f;
    for (int r = 0; r < S; ++r) {
      const float m = mask[(long)r * N + j];
      s += m * xn[((long)r * N + j) * C + t];
      ms += m;
    }
    qa[t] = s / (ms + 1e-10f);
  }
  __syncthreads();
  const float sc = rsqrtf((float)DK);
  if (t < H * DK) {
    float s = 0.f;
    for (int c = 0; c < C; ++c) s += qa[c] * wq[c * H * DK + t];
    qs[t] = s * sc;
    q_out[(long)j * H * DK + t] = qs[t];
  }
  __syncthreads();
  float* wj = w + (long)j * H * S;
  for (int i = t; i < H * S; i += 256) {
    const int h = i / S, r = i % S;
    const float* k = kvg + ((long)r * N + j) * ld;
    float l = 0.f;
    for (int d = 0; d < DK; ++d) l += qs[h * DK + d] * k[d];
    wj[i] = l + 1e9f * (mask[(long)r * N + j] - 1.f);
  }
  __syncthreads();
  for (int h = wave; h < H; h += 4) {
    float mx = -INFINITY;
    for (int r = lane; r < S; r += 64) mx = fmaxf(mx, wj[h * S + r]);
    mx = group_max<64>(mx);
    float s = 0.f;
    for (int r = lane; r < S; r += 64) s += __expf(wj[h * S + r] - mx);
    s = group_sum<64>(s);
    if (lane == 0) { hm[h] = mx; hs[h] = s; }
  }
  __syncthreads();
  for (int i = t; i < H * S; i += 256) {
    const int h = i / S;
    wj[i] = __expf(wj[i] - hm[h]) / hs[h];
  }
  __syncthreads();
  if (t < H * DV) {
    const int h = t / DV, d = t % DV;
    float s = 0.f;
    for (int r = 0; r < S; ++r) s += wj[h * S + r] * kvg[((long)r * N + j) * ld + DK + d];
    wa[(long)j * H * DV + t] = s;
  }
}

// Y[row][hv] = sigmoid(G[row][hv]) * wa[col][hv]
__global__ void glob_gate_kernel(const float* __restrict__ kvg, const float* __restrict__ wa,
                                 long rows, int N, int DK, int DV, int HV,
                                 float* __restrict__ Y) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * HV) return;
  const long row = i / HV;
  const int hv = (int)(i % HV);
  const int j = (int)(row % N);
  const int ld = DK + DV + HV;
  Y[i] = sigmoidf_(kvg[row * ld + DK + DV + hv]) * wa[(long)j * HV + hv];
}

// per column j: dwa = sum_s dY sigmoid(G); dG = dY wa s(1-s) (into dkvg)
__global__ __launch_bounds__(256) void glob_gate_bwd_kernel(
    const float* __restrict__ dY, const float* __restrict__ kvg, const float* __restrict__ wa,
    int S, int N, int DK, int DV, int HV, float* __restrict__ dwa, float* __restrict__ dkvg) {
  const int j = blockIdx.x, t = threadIdx.x;
  const int ld = DK + DV + HV;
  if (t >= HV) return;
  const float a = wa[(long)j * HV + t];
  float s = 0.f;
  for (int r = 0; r < S; ++r) {
    const long row = (long)r * N + j;
    const float g = sigmoidf_(kvg[row * ld + DK + DV + t]);
    const float d = dY[row * HV + t];
    s += d * g;
    dkvg[row * ld + DK + DV + t] = d * a * g * (1.f - g);
  }
  dwa[(long)j * HV + t] = s;
}

// per column j: softmax backward and the key / value / query gradients;
// dkvg[.][0:DK] = dk, [DK:DK+DV] = dv; dqavg[j][c] (before the mask mean)
__global__ __launch_bounds__(256) void glob_attn_bwd_kernel(
    const float* __restrict__ kvg, const float* __restrict__ w, const float* __restrict__ q,
    const float* __restrict__ dwa, const float* __restrict__ wq, int S, int N, int C, int H,
    int DK, int DV, float* __restrict__ dl, float* __restrict__ dkvg,
    float* __restrict__ dqavg) {
  __shared__ float qs[256], da[256], dq[256], sh[16];
  const int j = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int HV = H * DV, ld = DK + DV + HV;
  if (t < H * DK) qs[t] = q[(long)j * H * DK + t];
  if (t < HV) da[t] = dwa[(long)j * HV + t];
  __syncthreads();
  const float* wj = w + (long)j * H * S;
  float* dj = dl + (long)j * H * S;
  // dv[s][d] = sum_h w[h][s] dwa[h][d];  dw[h][s] = dwa[h] . v[s]
  for (int i = t; i < S * DV; i += 256) {
    const int r = i / DV, d = i % DV;
    float s = 0.f;
    for (int h = 0; h < H; ++h) s += wj[h * S + r] * da[h * DV + d];
    dkvg[((long)r * N + j) * ld + DK + d] = s;
  }
  for (int i = t; i < H * S; i += 256) {
    const int h = i / S, r = i % S;
    const float* v = kvg + ((long)r * N + j) * ld + DK;
    float s = 0.f;
    for (int d = 0; d < DV; ++d) s += da[h * DV + d] * v[d];
    dj[i] = s;
  }
  __syncthreads();
  for (int h = wave; h < H; h += 4) {
    float s = 0.f;
    for (int r = lane; r < S; r += 64) s += wj[h * S + r] * dj[h * S + r];
    s = group_sum<64>(s);
    if (lane == 0) sh[h] = s;
  }
  __syncthreads();
  for (int i = t; i < H * S; i += 256) dj[i] = wj[i] * (dj[i] - sh[i / S]);
  __syncthreads();
  // dq[h][d] = sum_s dlogit[h][s] k[s][d];  dk[s][d] = sum_h dlogit[h][s] q[h][d]
  if (t < H * DK) {
    const int h = t / DK, d = t % DK;
    float s = 0.f;
    for (int r = 0; r < S; ++r) s += dj[h * S + r] * kvg[((long)r * N + j) * ld + d];
    dq[t] = s;
  }
  for (int i = t; i < S * DK; i += 256) {
    const int r = i / DK, d = i % DK;
    float s = 0.f;
    for (int h = 0; h < H; ++h) s += dj[h * S + r] * qs[h * DK + d];
    dkvg[((long)r * N + j) * ld + d] = s;
  }
  __syncthreads();
  const float sc = rsqrtf((float)DK);
  if (t < C) {
    float s = 0.f;
    for (int o = 0; o < H * DK; ++o) s += dq[o] * wq[t * H * DK + o];
    dqavg[(long)j * C + t] = s * sc;
  }
}

// dxn[s][j][c] += mask[s][j] dqavg[j][c] / (sum_s mask[s][j] + 1e-10)
__global__ void glob_qavg_bwd_kernel(const float* __restrict__ dqavg, const float* __restrict__ mask,
                                     int S, int N, int C, float* __restrict__ dxn) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)S * N * C) return;
  const long row = i / C;
  const int c = (int)(i % C), j = (int)(row % N);
  float ms = 0.f;
  for (int r = 0; r < S; ++r) ms += mask[(long)r * N + j];
  dxn[i] += mask[row] * dqavg[(long)j * C + c] / (ms + 1e-10f);
}

__global__ void mul_rows_kernel(const float* __restrict__ a, const float* __restrict__ b, long n,
                                float* __restrict__ y) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = a[i] * b[i];
}

__global__ void add_rows_kernel(const float* __restrict__ a, const float* __restrict__ b, long n,
                                float* __restrict__ y) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = a[i] + b[i];
}

template <class A>
struct GlobSave {
  float *xn, *lm, *lr, *kvg, *q, *w, *wa;
  GlobSave(A& a, int S, int N, int C, int H, int DK, int DV) {
    const size_t R = (size_t)S * N;
    xn = a.template take<float>(R * C);
    lm = a.template take<float>(R);
    lr = a.template take<float>(R);
    kvg = a.template take<float>(R * (DK + DV + H * DV));
    q = a.template take<float>((size_t)N * H * DK);
    w = a.template take<float>((size_t)N * H * S);
    wa = a.template take<float>((size_t)N * H * DV);
  }
};

}  // namespace

MsaGlobW msaglobal_weights(WeightStore& ws, const std::string& P) {
  MsaGlobW w;
  const HostTensor& q = ws.host(P + "attention/query_w");  // [C, H, DK]
  const HostTensor& v = ws.host(P + "attention/value_w");  // [C, DV]
  if (q.shape.size() != 3 || v.shape.size() != 2) throw std::runtime_error("msa global: weight ranks");
  w.C = q.shape[0]; w.H = q.shape[1]; w.DK = q.shape[2]; w.DV = v.shape[1];
  if (w.C > 256 || w.H > 16 || w.H * w.DK > 256 || w.H * w.DV > 256)
    throw std::runtime_error("msa global: widths beyond this kernel's limits");
  const int C = w.C, H = w.H, DK = w.DK, DV = w.DV, W = DK + DV + H * DV;
  w.ln_g = ws.f32(P + "query_norm/scale");
  w.ln_b = ws.f32(P + "query_norm/offset");
  w.wq = ws.f32(P + "attention/query_w");
  w.wcat = ws.derived<float>("msaglobal.wcat:" + P, [&] {
    const HostTensor& k = ws.host(P + "attention/key_w");
    const HostTensor& g = ws.host(P + "attention/gating_w");
    std::vector<float> c((size_t)C * W);
    for (int r = 0; r < C; ++r) {
      for (int d = 0; d < DK; ++d) c[(size_t)r * W + d] = k.data[(size_t)r * DK + d];
      for (int d = 0; d < DV; ++d) c[(size_t)r * W + DK + d] = v.data[(size_t)r * DV + d];
      for (int o = 0; o < H * DV; ++o) c[(size_t)r * W + DK + DV + o] = g.data[(size_t)r * H * DV + o];
    }
    return c;
  });
  w.bcat = ws.derived<float>("msaglobal.bcat:" + P, [&] {
    const HostTensor& gb = ws.host(P + "attention/gating_b");
    std::vector<float> c(W, 0.f);
    for (int o = 0; o < H * DV; ++o) c[DK + DV + o] = gb.data[o];
    return c;
  });
  w.wo = ws.f32(P + "attention/output_w");  // [H, DV, C] = [H*DV][C]
  w.bo = ws.f32(P + "attention/output_b");
  return w;
}

size_t msaglobal_save_bytes(const MsaGlobW& w, int S, int N) {
  Sizer s;
  GlobSave<Sizer> g(s, S, N, w.C, w.H, w.DK, w.DV);
  return s.off;
}

void msaglobal_fwd(hipStream_t st, const MsaGlobW& w, int S, int N, const float* msa_in,
                   const float* msa_mask, const float* tbl, float* msa_out, void* save) {
  nonnull(msa_in, "msa global msa_in"); nonnull(msa_mask, "msa global mask");
  nonnull(msa_out, "msa global out"); nonnull(save, "msa global save");
  if (S <= 0 || N <= 0) throw std::runtime_error("msa global: empty shape");
  const int C = w.C, H = w.H, DK = w.DK, DV = w.DV, HV = H * DV, W = DK + DV + HV;
  const long R = (long)S * N;
  Carver cv(save);
  GlobSave<Carver> sv(cv, S, N, C, H, DK, DV);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)R * HV * 4 + 256);
  float* Y = ar.take_n<float>((size_t)R * HV);
  KTimed kt("msaglobal.fwd", st);
  ln_f32_rows_fwd(st, msa_in, R, C, w.ln_g, w.ln_b, sv.xn, sv.lm, sv.lr);
  GemmF32 g = gemm_rows((int)R, W, C, sv.xn, w.wcat, sv.kvg);
  g.bias = w.bcat;
  gemm_f32(st, g, "msaglobal.gemm_kvg");
  hipLaunchKernelGGL(glob_attn_fwd_kernel, dim3(N), dim3(256), 0, st, sv.xn, sv.kvg, msa_mask,
                     w.wq, S, N, C, H, DK, DV, sv.q, sv.w, sv.wa);
  hipLaunchKernelGGL(glob_gate_kernel, dim3((unsigned)((R * HV + 255) / 256)), dim3(256), 0, st,
                     sv.kvg, sv.wa, R, N, DK, DV, HV, Y);
  GemmF32 o = gemm_rows((int)R, C, HV, Y, w.wo, msa_out);
  o.bias = w.bo; o.gate = tbl; o.add = msa_in;
  gemm_f32(st, o, "msaglobal.gemm_out");
}

void msaglobal_bwd(hipStream_t st, const MsaGlobW& w, int S, int N, const float* msa_in,
                   const float* msa_mask, const float* tbl, const void* save,
                   const float* dmsa_out, float* dmsa_in) {
  nonnull(msa_in, "msa global msa_in"); nonnull(msa_mask, "msa global mask");
  nonnull(save, "msa global save"); nonnull(dmsa_out, "msa global dout");
  nonnull(dmsa_in, "msa global din");
  const int C = w.C, H = w.H, DK = w.DK, DV = w.DV, HV = H * DV, W = DK + DV + HV;
  const long R = (long)S * N;
  Carver cv(const_cast<void*>(save));
  GlobSave<Carver> sv(cv, S, N, C, H, DK, DV);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  Sizer need;
  need.take<float>((size_t)R * C);       // d update (after the table)
  need.take<float>((size_t)R * HV);      // dY
  need.take<float>((size_t)R * W);       // dkvg
  need.take<float>((size_t)N * HV);      // dwa
  need.take<float>((size_t)N * H * S);   // dlogit
  need.take<float>((size_t)N * C);       // dqavg
  need.take<float>((size_t)R * C);       // dxn
  ar.reset(st, need.off);
  float* du = ar.take_n<float>((size_t)R * C);
  float* dY = ar.take_n<float>((size_t)R * HV);
  float* dkvg = ar.take_n<float>((size_t)R * W);
  float* dwa = ar.take_n<float>((size_t)N * HV);
  float* dlg = ar.take_n<float>((size_t)N * H * S);
  float* dqa = ar.take_n<float>((size_t)N * C);
  float* dxn = ar.take_n<float>((size_t)R * C);
  KTimed kt("msaglobal.bwd", st);
  // the update's cotangent: dmsa_out * tbl (the residual passes dmsa_out on)
  const float* dup = dmsa_out;
  if (tbl) {
    hipLaunchKernelGGL(mul_rows_kernel, dim3((unsigned)((R * C + 255) / 256)), dim3(256), 0, st,
                       dmsa_out, tbl, R * C, du);
    dup = du;
  }
  GemmF32 gy = gemm_rows((int)R, HV, C, dup, w.wo, dY, true);
  gemm_f32(st, gy, "msaglobal.gemm_dY");
  hipLaunchKernelGGL(glob_gate_bwd_kernel, dim3(N), dim3(256), 0, st, dY, sv.kvg, sv.wa, S, N, DK,
                     DV, HV, dwa, dkvg);
  hipLaunchKernelGGL(glob_attn_bwd_kernel, dim3(N), dim3(256), 0, st, sv.kvg, sv.w, sv.q, dwa,
                     w.wq, S, N, C, H, DK, DV, dlg, dkvg, dqa);
  GemmF32 gx = gemm_rows((int)R, C, W, dkvg, w.wcat, dxn, true);
  gemm_f32(st, gx, "msaglobal.gemm_dx");
  hipLaunchKernelGGL(glob_qavg_bwd_kernel, dim3((unsigned)((R * C + 255) / 256)), dim3(256), 0, st,
                     dqa, msa_mask, S, N, C, dxn);
  ln_f32_rows_bwd(st, dxn, msa_in, R, C, w.ln_g, sv.lm, sv.lr, dxn);
  hipLaunchKernelGGL(add_rows_kernel, dim3((unsigned)((R * C + 255) / 256)), dim3(256), 0, st,
                     dmsa_out, dxn, R * C, dmsa_in);
}

}  // namespace bc2n
