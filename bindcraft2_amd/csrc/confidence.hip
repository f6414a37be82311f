// Confidence metrics from the head logits (alphafold_prediction_metrics):
//
//   plddt[i]  = sum_b softmax(lddt[i])_b (b + 1/2) / 50
//   E[i,j]    = sum_b softmax(pae[i,j])_b c_b,  c_b = 0.5 b + 0.25 (breaks
//               linspace(0, 31, 63) + half a step, the catch-all bin appended)
//   pae       = (E + E^T) / 2
//   T[i,j]    = sum_b softmax(pae[i,j])_b t_b,  t_b = 1 / (1 + c_b^2 / d0^2),
//               d0 = 1.24 (max(sum seq_mask, 19) - 15)^(1/3) - 1.8
//   per[i]    = sum_j T[i,j] m_ij w_ij / (1e-8 + sum_j w_ij),  w_ij = m_ij s_i s_j
//               (m = 1 for pTM; asym_i != asym_j for ipTM)
//   ptm, iptm = max_i per[i] s_i;  iptm_per_residue = per (ipTM's)
//   expres_ca = sigmoid(expres[i, CA])
//
// One pass over the [N, N, 64] PAE logits gives both expectations (16 lanes
// per pair, 4 bins a lane, DPP reductions); a workgroup per row forms the
// per-alignment sums and the symmetrised PAE.  The backward recomputes the
// softmax and routes every cotangent to the logits in one more pass:
//   d pae[i,j,b] = p_b ((c_b - E) (g_pae[i,j] + g_pae[j,i]) / 2 + (t_b - T) g_T[i,j])
// with g_T[i,j] from pTM (its max routes to one row), ipTM and its
// per-residue vector; the masks' normalisation is a constant.
// Reference: bindcraft/af2.py:197-219 (alphafold_prediction_metrics),
// bindcraft/af/alphafold/common/confidence.py:53-68, :113-176
// (bin centres, predicted_tm_score); native/confidence.cuh.
#include "confidence.h"

#include "common.h"
#include "runtime.h"

namespace bc2n {

namespace {

constexpr int PB = CONF_PBINS, LB = CONF_LBINS, CA = 1;

template <class A>
struct ConfSave {
  float *err, *tm, *tab, *per_p, *den_p, *den_a;
  int* best;
  ConfSave(A& c, int N) {
    const size_t NN = (size_t)N * N;
    err = c.template take<float>(NN);
    tm = c.template take<float>(NN);
    tab = c.template take<float>(2 * PB);  // centres, tm_bin
    per_p = c.template take<float>(N);
    den_p = c.template take<float>(N);
    den_a = c.template take<float>(N);
    best = c.template take<int>(2);
  }
};

// the two bin tables; d0 from the runtime residue weights
__global__ void conf_tables_kernel(const float* __restrict__ smask, int N, float* __restrict__ tab) {
  const int t = threadIdx.x;  // one wave
  float s = 0.f;
  for (int i = t; i < N; i += 64) s += smask[i];
  s = group_sum<64>(s);
  const float d0 = 1.24f * cbrtf(fmaxf(s, 19.f) - 15.f) - 1.8f;
  const float step = 31.f / (float)(PB - 2);
  const float c = step * (float)t + 0.5f * step;
  tab[t] = c;
  tab[PB + t] = 1.f / (1.f + (c * c) / (d0 * d0));
}

// softmax over a pair's 64 bins held 4 per lane by a 16-lane group:
// probabilities into e[], returns 1/z
__device__ __forceinline__ float pair_softmax(const float* __restrict__ L, int l, float (&e)[4]) {
  const float4 v = *reinterpret_cast<const float4*>(L + 4 * l);
  e[0] = v.x; e[1] = v.y; e[2] = v.z; e[3] = v.w;
  const float m = group_max<16>(fmaxf(fmaxf(e[0], e[1]), fmaxf(e[2], e[3])));
  float z = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    e[k] = __expf(e[k] - m);
    z += e[k];
  }
  return 1.f / group_sum<16>(z);
}

__global__ __launch_bounds__(256) void conf_pair_kernel(const float* __restrict__ pae_l, long NN,
                                                        const float* __restrict__ tab,
                                                        float* __restrict__ err,
                                                        float* __restrict__ tm) {
  const int l = threadIdx.x & 15;
  const long p0 = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  const long p = p0 < NN ? p0 : NN - 1;  // whole groups stay active
  float e[4];
  const float inv = pair_softmax(pae_l + p * PB, l, e);
  float ye = 0.f, yt = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    ye += e[k] * tab[4 * l + k];
    yt += e[k] * tab[PB + 4 * l + k];
  }
  ye = group_sum<16>(ye) * inv;
  yt = group_sum<16>(yt) * inv;
  if (l == 0 && p0 < NN) {
    err[p0] = ye;
    tm[p0] = yt;
  }
}

__global__ __launch_bounds__(64) void conf_rows_kernel(const float* __restrict__ err,
                                                       const float* __restrict__ tm,
                                                       const float* __restrict__ smask,
                                                       const int32_t* __restrict__ asym, int N,
                                                       float* __restrict__ pae,
                                                       float* __restrict__ per_p,
                                                       float* __restrict__ den_p,
                                                       float* __restrict__ per_a,
                                                       float* __restrict__ den_a) {
  const int i = blockIdx.x, t = threadIdx.x;
  const float si = smask[i];
  const int ai = asym[i];
  float np_ = 0.f, dp = 0.f, na = 0.f, da = 0.f;
  for (int j = t; j < N; j += 64) {
    const long q = (long)i * N + j;
    const float w = si * smask[j], T = tm[q];
    np_ += T * w;
    dp += w;
    if (asym[j] != ai) {
      na += T * w;
      da += w;
    }
    pae[q] = 0.5f * (err[q] + err[(long)j * N + i]);
  }
  np_ = group_sum<64>(np_);
  dp = group_sum<64>(dp);
  na = group_sum<64>(na);
  da = group_sum<64>(da);
  if (t == 0) {
    per_p[i] = np_ / (1e-8f + dp);
    den_p[i] = dp;
    per_a[i] = na / (1e-8f + da);
    den_a[i] = da;
  }
}

// max_i v[i] s[i] and its first index, over one wave
__device__ __forceinline__ void wave_argmax(const float* __restrict__ v, const float* __restrict__ s,
                                            int N, float& best, int& idx) {
  const int t = threadIdx.x;
  float b = -INFINITY;
  int bi = N;
  for (int i = t; i < N; i += 64) {
    const float x = v[i] * s[i];
    if (x > b) {
      b = x;
      bi = i;
    }
  }
  best = group_max<64>(b);
  const float cand = b == best ? (float)bi : (float)N;
  idx = (int)-group_max<64>(-cand);  // smallest index reaching the max
}

__global__ __launch_bounds__(64) void conf_max_kernel(const float* __restrict__ per_p,
                                                      const float* __restrict__ per_a,
                                                      const float* __restrict__ smask, int N,
                                                      float* __restrict__ ptm,
                                                      float* __restrict__ iptm,
                                                      int* __restrict__ best) {
  float bp, ba;
  int ip, ia;
  wave_argmax(per_p, smask, N, bp, ip);
  wave_argmax(per_a, smask, N, ba, ia);
  if (threadIdx.x == 0) {
    *ptm = bp;
    *iptm = ba;
    best[0] = ip;
    best[1] = ia;
  }
}

__global__ void conf_res_kernel(const float* __restrict__ lddt_l, const float* __restrict__ expres_l,
                                int N, float* __restrict__ plddt, float* __restrict__ expres_ca) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const float* L = lddt_l + (long)i * LB;
  float m = -INFINITY;
  for (int b = 0; b < LB; ++b) m = fmaxf(m, L[b]);
  float z = 0.f, y = 0.f;
  for (int b = 0; b < LB; ++b) {
    const float e = __expf(L[b] - m);
    z += e;
    y += e * ((float)b + 0.5f) * (1.f / LB);
  }
  plddt[i] = y / z;
  expres_ca[i] = 1.f / (1.f + __expf(-expres_l[(long)i * CONF_EXPRES + CA]));
}

__global__ void conf_res_bwd_kernel(const float* __restrict__ lddt_l,
                                    const float* __restrict__ expres_l,
                                    const float* __restrict__ g_plddt,
                                    const float* __restrict__ g_expres, int N,
                                    float* __restrict__ d_lddt, float* __restrict__ d_expres) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const float* L = lddt_l + (long)i * LB;
  float* D = d_lddt + (long)i * LB;
  const float g = g_plddt ? g_plddt[i] : 0.f;
  float m = -INFINITY;
  for (int b = 0; b < LB; ++b) m = fmaxf(m, L[b]);
  float z = 0.f, y = 0.f;
  for (int b = 0; b < LB; ++b) {
    const float e = __expf(L[b] - m);
    z += e;
    y += e * ((float)b + 0.5f) * (1.f / LB);
  }
  const float inv = 1.f / z;
  y *= inv;
  for (int b = 0; b < LB; ++b)
    D[b] = __expf(L[b] - m) * inv * (((float)b + 0.5f) * (1.f / LB) - y) * g;
  float* E = d_expres + (long)i * CONF_EXPRES;
  for (int k = 0; k < CONF_EXPRES; ++k) E[k] = 0.f;
  const float s = 1.f / (1.f + __expf(-expres_l[(long)i * CONF_EXPRES + CA]));
  E[CA] = s * (1.f - s) * (g_expres ? g_expres[i] : 0.f);
}

struct PairBwdArgs {
  const float *pae_l, *tab, *smask, *den_p, *den_a;
  const int32_t* asym;
  const int* best;
  const float *g_pae, *g_ptm, *g_iptm, *g_iptm_pr;
  float* d_pae;
  int N;
};

__global__ __launch_bounds__(256) void conf_pair_bwd_kernel(PairBwdArgs a) {
  const int l = threadIdx.x & 15, N = a.N;
  const long NN = (long)N * N;
  const long p0 = (long)blockIdx.x * 16 + (threadIdx.x >> 4);
  const long p = p0 < NN ? p0 : NN - 1;
  const int i = (int)(p / N), j = (int)(p % N);
  float e[4];
  const float inv = pair_softmax(a.pae_l + p * PB, l, e);
  float c[4], t[4], ye = 0.f, yt = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    e[k] *= inv;
    c[k] = a.tab[4 * l + k];
    t[k] = a.tab[PB + 4 * l + k];
    ye += e[k] * c[k];
    yt += e[k] * t[k];
  }
  ye = group_sum<16>(ye);
  yt = group_sum<16>(yt);
  const float ge = a.g_pae ? 0.5f * (a.g_pae[p] + a.g_pae[(long)j * N + i]) : 0.f;
  const float w = a.smask[i] * a.smask[j];
  float gt = 0.f;
  if (a.g_ptm && i == a.best[0]) gt += a.g_ptm[0] * a.smask[i] * w / (1e-8f + a.den_p[i]);
  if (a.asym[i] != a.asym[j]) {
    float gi = a.g_iptm_pr ? a.g_iptm_pr[i] : 0.f;
    if (a.g_iptm && i == a.best[1]) gi += a.g_iptm[0] * a.smask[i];
    gt += gi * w / (1e-8f + a.den_a[i]);
  }
  if (p0 < NN) {
    float4 o;
    o.x = e[0] * ((c[0] - ye) * ge + (t[0] - yt) * gt);
    o.y = e[1] * ((c[1] - ye) * ge + (t[1] - yt) * gt);
    o.z = e[2] * ((c[2] - ye) * ge + (t[2] - yt) * gt);
    o.w = e[3] * ((c[3] - ye) * ge + (t[3] - yt) * gt);
    *reinterpret_cast<float4*>(a.d_pae + p0 * PB + 4 * l) = o;
  }
}

void conf_check(int N, const float* pae_l) {
  if (N <= 0) throw std::runtime_error("confidence: N must be positive");
  if (((uintptr_t)pae_l & 15) != 0) throw std::runtime_error("confidence: pae logits must be 16-byte aligned");
}

}  // namespace

size_t confidence_save_bytes(int N) {
  Sizer s;
  ConfSave<Sizer> plan(s, N);
  (void)plan;
  return s.off;
}

void confidence_fwd(hipStream_t st, const float* lddt_l, const float* pae_l, const float* expres_l,
                    const float* seq_mask, const int32_t* asym, int N, float* plddt, float* pae,
                    float* ptm, float* iptm, float* iptm_pr, float* expres_ca, void* save) {
  conf_check(N, pae_l);
  Carver cv(save);
  ConfSave<Carver> sv(cv, N);
  const long NN = (long)N * N;
  KTimed kt("confidence", st);
  hipLaunchKernelGGL(conf_tables_kernel, dim3(1), dim3(64), 0, st, seq_mask, N, sv.tab);
  hipLaunchKernelGGL(conf_pair_kernel, dim3((unsigned)((NN + 15) / 16)), dim3(256), 0, st, pae_l,
                     NN, sv.tab, sv.err, sv.tm);
  hipLaunchKernelGGL(conf_rows_kernel, dim3(N), dim3(64), 0, st, sv.err, sv.tm, seq_mask, asym, N,
                     pae, sv.per_p, sv.den_p, iptm_pr, sv.den_a);
  hipLaunchKernelGGL(conf_max_kernel, dim3(1), dim3(64), 0, st, sv.per_p, iptm_pr, seq_mask, N, ptm,
                     iptm, sv.best);
  hipLaunchKernelGGL(conf_res_kernel, dim3((N + 127) / 128), dim3(128), 0, st, lddt_l, expres_l, N,
                     plddt, expres_ca);
}

void confidence_bwd(hipStream_t st, const float* lddt_l, const float* pae_l, const float* expres_l,
                    const float* seq_mask, const int32_t* asym, int N, const void* save,
                    const float* g_plddt, const float* g_pae, const float* g_ptm,
                    const float* g_iptm, const float* g_iptm_pr, const float* g_expres,
                    float* d_lddt, float* d_pae, float* d_expres) {
  conf_check(N, pae_l);
  Carver cv(const_cast<void*>(save));
  ConfSave<Carver> sv(cv, N);
  const long NN = (long)N * N;
  KTimed kt("confidence.bwd", st);
  hipLaunchKernelGGL(conf_res_bwd_kernel, dim3((N + 127) / 128), dim3(128), 0, st, lddt_l, expres_l,
                     g_plddt, g_expres, N, d_lddt, d_expres);
  PairBwdArgs a{pae_l, sv.tab, seq_mask, sv.den_p, sv.den_a, asym, sv.best,
                g_pae, g_ptm, g_iptm, g_iptm_pr, d_pae, N};
  hipLaunchKernelGGL(conf_pair_bwd_kernel, dim3((unsigned)((NN + 15) / 16)), dim3(256), 0, st, a);
}

}  // namespace bc2n
