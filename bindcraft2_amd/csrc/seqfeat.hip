// Design sequence features and the trunk inputs built from them.
//
//   k       = logit_scale / temperature
//   p       = softmax(k * logits + bias)            (bias per amino acid, may be absent)
//   blended = logits, zero where the acid is omitted (logit <= omitted_half)
//   f       = sw * p + (1 - sw) * blended
//   feat    = ohw * onehot(argmax p) + (1 - ohw) * f
//   prof    = onehot(argmax p)                       (the same with ohw = 1)
//
// The one-hot is straight-through: forward it is the hard one-hot, backward
// the identity on p.  So both outputs reach the logits through the one
// softmax, with weight cf = ohw + (1 - ohw) sw for feat and 1 for prof, and
// feat also through the linear path with weight (1 - ohw)(1 - sw) where the
// acid is not omitted:
//
//   g_p      = cf * d_feat + d_prof
//   d_logits = k * p * (g_p - <p, g_p>) + (1 - ohw)(1 - sw) * d_feat * [not omitted]
//
// A residue not flagged DESIGN passes its logits through both outputs, so
// its d_logits = d_feat + d_prof.
// Reference: bindcraft/sequence_optimization.py:33-52 (sequence_features_from_logits,
// straight_through_one_hot, omitted_amino_acid_mask), bindcraft/af2.py:99-104
// (prepare_design_sequence_features), bindcraft/af2.py:187-192 (target_feat,
// msa_feat and aatype of alphafold_input_features); native/seqfeat.cuh
// (seqFeatK / seqFeatBwdK).
#include "seqfeat.h"

#include "runtime.h"

namespace bc2n {

namespace {

constexpr int A = SEQ_A;

__device__ __forceinline__ SeqScalars pick(SeqScalars s, const float* sc4) {
  if (sc4) {
    s.sw = sc4[0];
    s.ohw = sc4[1];
    s.temp = sc4[2];
    s.ls = sc4[3];
  }
  return s;
}

// p (softmax of k * logits + bias) into pr; returns the first index of the maximum
__device__ __forceinline__ int seq_softmax(const float* L, const float* bias, float k, float (&pr)[A]) {
  float m = -INFINITY;
#pragma unroll
  for (int a = 0; a < A; ++a) {
    pr[a] = L[a] * k + (bias ? bias[a] : 0.f);
    m = fmaxf(m, pr[a]);
  }
  float z = 0.f;
#pragma unroll
  for (int a = 0; a < A; ++a) {
    pr[a] = __expf(pr[a] - m);
    z += pr[a];
  }
  const float inv = 1.f / z;
  int amax = 0;
  float pmax = -1.f;
#pragma unroll
  for (int a = 0; a < A; ++a) {
    pr[a] *= inv;
    if (pr[a] > pmax) {
      pmax = pr[a];
      amax = a;
    }
  }
  return amax;
}

__global__ void seqfeat_kernel(const float* __restrict__ logits, const uint8_t* __restrict__ flags,
                               const float* __restrict__ bias, SeqScalars s_,
                               const float* __restrict__ sc4, float omitted_half, int N,
                               float* __restrict__ feat, float* __restrict__ prof) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const float* L = logits + (long)i * A;
  float* F = feat + (long)i * A;
  float* P = prof + (long)i * A;
  if (!(flags[i] & 1u)) {
#pragma unroll
    for (int a = 0; a < A; ++a) F[a] = P[a] = L[a];
    return;
  }
  const SeqScalars s = pick(s_, sc4);
  float pr[A];
  const int amax = seq_softmax(L, bias, s.ls / s.temp, pr);
#pragma unroll
  for (int a = 0; a < A; ++a) {
    const float blended = L[a] <= omitted_half ? 0.f : L[a];
    const float f = s.sw * pr[a] + (1.f - s.sw) * blended;
    const float oh = a == amax ? 1.f : 0.f;
    F[a] = s.ohw * oh + (1.f - s.ohw) * f;
    P[a] = oh;
  }
}

__global__ void seqfeat_bwd_kernel(const float* __restrict__ logits,
                                   const uint8_t* __restrict__ flags,
                                   const float* __restrict__ bias, SeqScalars s_,
                                   const float* __restrict__ sc4, float omitted_half, int N,
                                   const float* __restrict__ d_feat,
                                   const float* __restrict__ d_prof,
                                   float* __restrict__ d_logits) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const float* L = logits + (long)i * A;
  const float* gf = d_feat + (long)i * A;
  const float* gp = d_prof + (long)i * A;
  float* out = d_logits + (long)i * A;
  if (!(flags[i] & 1u)) {
#pragma unroll
    for (int a = 0; a < A; ++a) out[a] = gf[a] + gp[a];
    return;
  }
  const SeqScalars s = pick(s_, sc4);
  const float k = s.ls / s.temp;
  float pr[A];
  seq_softmax(L, bias, k, pr);
  const float cf = s.ohw + (1.f - s.ohw) * s.sw;
  const float lin = (1.f - s.ohw) * (1.f - s.sw);
  float g[A], dot = 0.f;
#pragma unroll
  for (int a = 0; a < A; ++a) {
    g[a] = cf * gf[a] + gp[a];
    dot += pr[a] * g[a];
  }
#pragma unroll
  for (int a = 0; a < A; ++a) {
    float d = k * pr[a] * (g[a] - dot);
    if (L[a] > omitted_half) d += lin * gf[a];
    out[a] = d;
  }
}

__global__ void design_inputs_kernel(const float* __restrict__ feat, const float* __restrict__ prof,
                                     int N, float* __restrict__ tf, float* __restrict__ mf,
                                     float* __restrict__ aatype) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const float* F = feat + (long)i * A;
  const float* P = prof + (long)i * A;
  float* T = tf + (long)i * (A + 1);
  float* Mf = mf + (long)i * 49;
  int amax = 0;
  float best = -INFINITY;
#pragma unroll
  for (int a = 0; a < A; ++a) {
    const float f = F[a];
    if (f > best) {
      best = f;
      amax = a;
    }
    T[a] = f;
    Mf[a] = f;
    Mf[25 + a] = P[a];
  }
  T[A] = 0.f;
#pragma unroll
  for (int c = 20; c < 25; ++c) Mf[c] = 0.f;
#pragma unroll
  for (int c = 45; c < 49; ++c) Mf[c] = 0.f;
  aatype[i] = (float)amax;
}

__global__ void design_inputs_bwd_kernel(const float* __restrict__ dtf, const float* __restrict__ dmf,
                                         int N, float* __restrict__ d_feat,
                                         float* __restrict__ d_prof) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
#pragma unroll
  for (int a = 0; a < A; ++a) {
    d_feat[(long)i * A + a] = dtf[(long)i * (A + 1) + a] + dmf[(long)i * 49 + a];
    d_prof[(long)i * A + a] = dmf[(long)i * 49 + 25 + a];
  }
}

unsigned blocks(int N) { return (unsigned)((N + 127) / 128); }

}  // namespace

void seqfeat_fwd(hipStream_t st, const float* logits, const uint8_t* flags, const float* bias,
                 SeqScalars s, const float* sc4, float omitted_half, int N, float* feat,
                 float* prof) {
  if (N <= 0) return;
  KTimed kt("seqfeat", st);
  hipLaunchKernelGGL(seqfeat_kernel, dim3(blocks(N)), dim3(128), 0, st, logits, flags, bias, s, sc4,
                     omitted_half, N, feat, prof);
}

void seqfeat_bwd(hipStream_t st, const float* logits, const uint8_t* flags, const float* bias,
                 SeqScalars s, const float* sc4, float omitted_half, int N, const float* d_feat,
                 const float* d_prof, float* d_logits) {
  if (N <= 0) return;
  KTimed kt("seqfeat.bwd", st);
  hipLaunchKernelGGL(seqfeat_bwd_kernel, dim3(blocks(N)), dim3(128), 0, st, logits, flags, bias, s,
                     sc4, omitted_half, N, d_feat, d_prof, d_logits);
}

void design_inputs_fwd(hipStream_t st, const float* feat, const float* prof, int N, float* tf,
                       float* mf, float* aatype) {
  if (N <= 0) return;
  hipLaunchKernelGGL(design_inputs_kernel, dim3(blocks(N)), dim3(128), 0, st, feat, prof, N, tf, mf,
                     aatype);
}

void design_inputs_bwd(hipStream_t st, const float* dtf, const float* dmf, int N, float* d_feat,
                       float* d_prof) {
  if (N <= 0) return;
  hipLaunchKernelGGL(design_inputs_bwd_kernel, dim3(blocks(N)), dim3(128), 0, st, dtf, dmf, N,
                     d_feat, d_prof);
}

}  // namespace bc2n
