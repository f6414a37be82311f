// Post-trunk step: fold iterations, the last iteration's sidechain and the
// four heads, forward and backward, all f32 (the reference's
// StructureHeadsFwd/Bwd handlers, native/ffi.cu:530-639 / 1009-1044).
//
//   act, traj      = fold iterations (ipa.hip)
//   initial_act    = LN(single)                           single_layer_norm
//   atom14         = sidechain(traj[-1] = [R | 20 t], act, initial_act, aatype)
//   distogram      = h + h^T,  h = pair . Wd + bd         (symmetrised)
//   pae            = pair . Wp + bp                        (not symmetrised)
//   plddt          = relu(relu(LN(act) W0 + b0) W1 + b1) Wl + bl
//   expres         = single . We + be
//
// Sidechain (folding_multimer.py:950-1040, all_atom_multimer.py:370-468):
//   a0 = relu(act) Wi0 + bi0 + relu(initial_act) Wi1 + bi1
//   a_{b+1} = a_b + relu(relu(a_b) W1_b + b1_b) W2_b + b2_b     (b = 0, 1)
//   (sin, cos) of 7 torsions = l2-normalised pairs of relu(a2) Wa + ba
//   frames: F_g = (D_g X(torsion g), d_g) from the residue's default frames,
//   chi2..chi4 chained on the previous chi frame, mapped by [R | 20 t];
//   atom k = its group's frame applied to its literature position, masked.
// One thread per residue does the frame algebra and, in the backward, its
// exact reverse (the rotations and the l2 normalisation included).
// Weights: the post-trunk directory (bindcraft/af/native.py:339-444) plus
// its residue tables const/default_frame, atom14_to_group, atom14_lit_pos,
// atom14_mask (:432-440).
#include "heads.h"

#include "gemm_f32.h"
#include "kernels.h"

#include <algorithm>

namespace bc2n {

namespace {

constexpr int CS = 384, CZ = 128, SC = 128, NANG = 14, NA = SH_ATOMS;
constexpr int PL = 128;

template <class A>
struct ShSave {
  void* fold;
  float *traj, *act, *init, *imean, *irstd;
  float *a[3], *rh[2], *un;                  // sidechain
  float *lmean, *lrstd, *r0, *r1;            // pLDDT head
  float *d_act, *d_init, *d_traj;            // backward scratch
  ShSave(A& c, int N, int depth) {
    fold = c.template take<char>(fold_save_bytes(N, depth));
    traj = c.template take<float>((size_t)depth * N * 12);
    act = c.template take<float>((size_t)N * CS);
    init = c.template take<float>((size_t)N * CS);
    imean = c.template take<float>(N);
    irstd = c.template take<float>(N);
    for (int i = 0; i < 3; ++i) a[i] = c.template take<float>((size_t)N * SC);
    for (int i = 0; i < 2; ++i) rh[i] = c.template take<float>((size_t)N * SC);
    un = c.template take<float>((size_t)N * NANG);
    lmean = c.template take<float>(N);
    lrstd = c.template take<float>(N);
    r0 = c.template take<float>((size_t)N * PL);
    r1 = c.template take<float>((size_t)N * PL);
    d_act = c.template take<float>((size_t)N * CS);
    d_init = c.template take<float>((size_t)N * CS);
    d_traj = c.template take<float>((size_t)depth * N * 12);
  }
};

// ---------------------------------------------------------------- elementwise
__global__ void relu_kernel(const float* __restrict__ x, long n, float* __restrict__ y) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = fmaxf(x[i], 0.f);
}
void relu(hipStream_t st, const float* x, long n, float* y) {
  hipLaunchKernelGGL(relu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n, y);
}
__global__ void add_kernel(float* __restrict__ y, const float* __restrict__ x, long n) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] += x[i];
}
void add_into(hipStream_t st, float* y, const float* x, long n) {
  hipLaunchKernelGGL(add_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y, x, n);
}

// o[i][j][c] = h[i][j][c] + h[j][i][c], 64 channels, float4 per thread
__global__ void symmetrise_kernel(const float* __restrict__ h, float* __restrict__ o, int N) {
  const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (long)N * N * 16) return;
  const int c4 = (int)(e & 15);
  const long ij = e >> 4;
  const int i = (int)(ij / N), j = (int)(ij % N);
  const float4 a = reinterpret_cast<const float4*>(h + ij * 64)[c4];
  const float4 b = reinterpret_cast<const float4*>(h + ((long)j * N + i) * 64)[c4];
  reinterpret_cast<float4*>(o + ij * 64)[c4] = make_float4(a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w);
}
void symmetrise(hipStream_t st, const float* h, float* o, int N) {
  const long n = (long)N * N * 16;
  hipLaunchKernelGGL(symmetrise_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, h, o, N);
}

// ------------------------------------------------------------- frame algebra
struct Rig {
  float R[9], t[3];
};
__device__ __forceinline__ void compose(const Rig& a, const Rig& b, Rig& o) {
#pragma unroll
  for (int i = 0; i < 3; ++i) {
#pragma unroll
    for (int j = 0; j < 3; ++j)
      o.R[i * 3 + j] = a.R[i * 3] * b.R[j] + a.R[i * 3 + 1] * b.R[3 + j] + a.R[i * 3 + 2] * b.R[6 + j];
    o.t[i] = a.R[i * 3] * b.t[0] + a.R[i * 3 + 1] * b.t[1] + a.R[i * 3 + 2] * b.t[2] + a.t[i];
  }
}
// Reverse of o = a . b: da += do.R b.R^T + do.t b.t^T (rotation), da.t += do.t,
// db.R += a.R^T do.R, db.t += a.R^T do.t.
__device__ __forceinline__ void compose_bwd(const Rig& a, const Rig& b, const Rig& d, Rig& da, Rig& db) {
#pragma unroll
  for (int i = 0; i < 3; ++i) {
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      da.R[i * 3 + j] += d.R[i * 3] * b.R[j * 3] + d.R[i * 3 + 1] * b.R[j * 3 + 1] +
                         d.R[i * 3 + 2] * b.R[j * 3 + 2] + d.t[i] * b.t[j];
      db.R[i * 3 + j] += a.R[i] * d.R[j] + a.R[3 + i] * d.R[3 + j] + a.R[6 + i] * d.R[6 + j];
    }
    da.t[i] += d.t[i];
    db.t[i] += a.R[i] * d.t[0] + a.R[3 + i] * d.t[1] + a.R[6 + i] * d.t[2];
  }
}
__device__ __forceinline__ void zero(Rig& r) {
#pragma unroll
  for (int i = 0; i < 9; ++i) r.R[i] = 0.f;
#pragma unroll
  for (int i = 0; i < 3; ++i) r.t[i] = 0.f;
}

constexpr float ANG_EPS = 1e-12f;

// Per residue: the 8 frames F_g (default frame composed with the torsion
// rotation about x), their chained-to-backbone forms B_g and the (s, c) pairs.
struct SideFrames {
  Rig F[8], B[8], BB;
  float s[8], c[8], nrm[8];
  int a;
};
__device__ void side_frames(const float* un, const float* trj, const float* aatype,
                            const ResTables& tab, int n, SideFrames& f) {
  f.a = min(max((int)aatype[n], 0), 20);
  const float* D = tab.frame + (long)f.a * 8 * 16;
  f.s[0] = 0.f; f.c[0] = 1.f; f.nrm[0] = 1.f;
  for (int g = 1; g < 8; ++g) {
    const float us = un[n * NANG + 2 * (g - 1)], uc = un[n * NANG + 2 * (g - 1) + 1];
    f.nrm[g] = sqrtf(fmaxf(us * us + uc * uc, ANG_EPS));
    f.s[g] = us / f.nrm[g];
    f.c[g] = uc / f.nrm[g];
  }
  for (int g = 0; g < 8; ++g) {
    const float* d = D + g * 16;
    // (D X)[:, 0] = D[:, 0]; [:, 1] = c D[:, 1] + s D[:, 2]; [:, 2] = -s D[:, 1] + c D[:, 2]
    for (int i = 0; i < 3; ++i) {
      f.F[g].R[i * 3] = d[i * 4];
      f.F[g].R[i * 3 + 1] = f.c[g] * d[i * 4 + 1] + f.s[g] * d[i * 4 + 2];
      f.F[g].R[i * 3 + 2] = -f.s[g] * d[i * 4 + 1] + f.c[g] * d[i * 4 + 2];
      f.F[g].t[i] = d[i * 4 + 3];
    }
  }
  for (int g = 0; g < 5; ++g) f.B[g] = f.F[g];
  for (int g = 5; g < 8; ++g) compose(f.B[g - 1], f.F[g], f.B[g]);
  for (int i = 0; i < 3; ++i) {
    for (int j = 0; j < 3; ++j) f.BB.R[i * 3 + j] = trj[n * 12 + i * 4 + j];
    f.BB.t[i] = trj[n * 12 + i * 4 + 3];
  }
}

__global__ void side_atoms_kernel(const float* __restrict__ un, const float* __restrict__ trj,
                                  const float* __restrict__ aatype, ResTables tab, int N,
                                  float* __restrict__ atom14) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  SideFrames f;
  side_frames(un, trj, aatype, tab, n, f);
  Rig G[8];
  for (int g = 0; g < 8; ++g) compose(f.BB, f.B[g], G[g]);
  for (int k = 0; k < NA; ++k) {
    const int g = min(max((int)tab.group[f.a * NA + k], 0), 7);
    const float m = tab.mask[f.a * NA + k];
    const float* l = tab.lit + (f.a * NA + k) * 3;
    for (int i = 0; i < 3; ++i)
      atom14[((long)n * NA + k) * 3 + i] =
          m * (G[g].R[i * 3] * l[0] + G[g].R[i * 3 + 1] * l[1] + G[g].R[i * 3 + 2] * l[2] + G[g].t[i]);
  }
}

// d(atom14) -> d(unnormalised angles) [N][14] and d[R | 20 t] [N][12]
__global__ void side_atoms_bwd_kernel(const float* __restrict__ un, const float* __restrict__ trj,
                                      const float* __restrict__ aatype, ResTables tab, int N,
                                      const float* __restrict__ datom, float* __restrict__ dun,
                                      float* __restrict__ dtrj) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  SideFrames f;
  side_frames(un, trj, aatype, tab, n, f);
  Rig dG[8], dB[8], dBB, dummy;
  for (int g = 0; g < 8; ++g) { zero(dG[g]); zero(dB[g]); }
  zero(dBB);
  for (int k = 0; k < NA; ++k) {
    const int g = min(max((int)tab.group[f.a * NA + k], 0), 7);
    const float m = tab.mask[f.a * NA + k];
    const float* l = tab.lit + (f.a * NA + k) * 3;
    for (int i = 0; i < 3; ++i) {
      const float dp = m * datom[((long)n * NA + k) * 3 + i];
      for (int j = 0; j < 3; ++j) dG[g].R[i * 3 + j] += dp * l[j];
      dG[g].t[i] += dp;
    }
  }
  // G_g = BB . B_g
  for (int g = 0; g < 8; ++g) compose_bwd(f.BB, f.B[g], dG[g], dBB, dB[g]);
  // B_g = B_{g-1} . F_g for g = 7, 6, 5 (B_4 = F_4); the F translations are constants
  Rig dF[8];
  for (int g = 0; g < 8; ++g) zero(dF[g]);
  for (int g = 7; g >= 5; --g) compose_bwd(f.B[g - 1], f.F[g], dB[g], dB[g - 1], dF[g]);
  for (int g = 1; g < 5; ++g)
    for (int i = 0; i < 9; ++i) dF[g].R[i] += dB[g].R[i];
  (void)dummy;
  // F_g.R = D_g X(s, c):  dX = D^T dF.R;  ds = dX[2][1] - dX[1][2], dc = dX[1][1] + dX[2][2]
  const float* D = tab.frame + (long)f.a * 8 * 16;
  for (int g = 1; g < 8; ++g) {
    const float* d = D + g * 16;
    float dX[9];
    for (int i = 0; i < 3; ++i)
      for (int j = 0; j < 3; ++j)
        dX[i * 3 + j] = d[i] * dF[g].R[j] + d[4 + i] * dF[g].R[3 + j] + d[8 + i] * dF[g].R[6 + j];
    const float ds = dX[7] - dX[5], dc = dX[4] + dX[8];
    // (s, c) = u / max(|u|, sqrt eps): du = (dn - n (n . dn)) / |u| above the floor
    const float us = un[n * NANG + 2 * (g - 1)], uc = un[n * NANG + 2 * (g - 1) + 1];
    const bool live = us * us + uc * uc > ANG_EPS;
    const float dot = live ? f.s[g] * ds + f.c[g] * dc : 0.f;
    dun[n * NANG + 2 * (g - 1)] = (ds - f.s[g] * dot) / f.nrm[g];
    dun[n * NANG + 2 * (g - 1) + 1] = (dc - f.c[g] * dot) / f.nrm[g];
  }
  for (int i = 0; i < 3; ++i) {
    for (int j = 0; j < 3; ++j) dtrj[n * 12 + i * 4 + j] = dBB.R[i * 3 + j];
    dtrj[n * 12 + i * 4 + 3] = dBB.t[i];
  }
}

const float* need_f32(WeightStore& ws, const std::string& name, size_t count) {
  const HostTensor& t = ws.host(name);
  if (t.data.size() != count) throw std::runtime_error("structure heads: " + name + " has the wrong size");
  return ws.f32(name);
}

void sh_check(int N, int depth) {
  if (N <= 0 || N > 1024) throw std::runtime_error("structure heads: N must be in 1..1024");
  if (depth <= 0) throw std::runtime_error("structure heads: depth must be positive");
}

}  // namespace

StructHeadsW structheads_weights(WeightStore& ws) {
  StructHeadsW w;
  w.fold = fold_weights(ws);
  const std::string P = "param/", S = P + "fold_iteration/rigid_sidechain/";
  w.sc.wi0 = need_f32(ws, S + "input_projection/weights", (size_t)CS * SC);
  w.sc.bi0 = need_f32(ws, S + "input_projection/bias", SC);
  w.sc.wi1 = need_f32(ws, S + "input_projection_1/weights", (size_t)CS * SC);
  w.sc.bi1 = need_f32(ws, S + "input_projection_1/bias", SC);
  for (int b = 0; b < 2; ++b) {
    const std::string sfx = b ? "_1" : "";
    w.sc.wr1[b] = need_f32(ws, S + "resblock1" + sfx + "/weights", (size_t)SC * SC);
    w.sc.br1[b] = need_f32(ws, S + "resblock1" + sfx + "/bias", SC);
    w.sc.wr2[b] = need_f32(ws, S + "resblock2" + sfx + "/weights", (size_t)SC * SC);
    w.sc.br2[b] = need_f32(ws, S + "resblock2" + sfx + "/bias", SC);
  }
  w.sc.wa = need_f32(ws, S + "unnormalized_angles/weights", (size_t)SC * NANG);
  w.sc.ba = need_f32(ws, S + "unnormalized_angles/bias", NANG);
  w.hd.wdg = need_f32(ws, P + "distogram_head/half_logits/weights", (size_t)CZ * SH_DGRAM);
  w.hd.bdg = need_f32(ws, P + "distogram_head/half_logits/bias", SH_DGRAM);
  w.hd.wpae = need_f32(ws, P + "predicted_aligned_error_head/logits/weights", (size_t)CZ * SH_PAE);
  w.hd.bpae = need_f32(ws, P + "predicted_aligned_error_head/logits/bias", SH_PAE);
  const std::string L = P + "predicted_lddt_head/";
  w.hd.ln_g = need_f32(ws, L + "input_layer_norm/scale", CS);
  w.hd.ln_b = need_f32(ws, L + "input_layer_norm/offset", CS);
  w.hd.w0 = need_f32(ws, L + "act_0/weights", (size_t)CS * PL);
  w.hd.b0 = need_f32(ws, L + "act_0/bias", PL);
  w.hd.w1 = need_f32(ws, L + "act_1/weights", (size_t)PL * PL);
  w.hd.b1 = need_f32(ws, L + "act_1/bias", PL);
  w.hd.wl = need_f32(ws, L + "logits/weights", (size_t)PL * SH_PLDDT);
  w.hd.bl = need_f32(ws, L + "logits/bias", SH_PLDDT);
  w.hd.wer = need_f32(ws, P + "experimentally_resolved_head/logits/weights", (size_t)CS * SH_EXPRES);
  w.hd.ber = need_f32(ws, P + "experimentally_resolved_head/logits/bias", SH_EXPRES);
  w.tab.frame = need_f32(ws, "const/default_frame", 21 * 8 * 16);
  w.tab.group = need_f32(ws, "const/atom14_to_group", 21 * NA);
  w.tab.lit = need_f32(ws, "const/atom14_lit_pos", 21 * NA * 3);
  w.tab.mask = need_f32(ws, "const/atom14_mask", 21 * NA);
  return w;
}

size_t structheads_save_bytes(int N, int depth) {
  Sizer s;
  ShSave<Sizer> plan(s, N, depth);
  (void)plan;
  return s.off;
}

void structheads_fwd(hipStream_t st, const StructHeadsW& w, int N, int depth, const float* single,
                     const float* pair, const float* mask, const float* aatype,
                     const uint32_t* key, const uint32_t* enabled, bool dropout, float* atom14,
                     float* dgram, float* pae, float* plddt, float* expres, void* save,
                     const float* init_pos37) {
  sh_check(N, depth);
  nonnull(single, "structure heads single"); nonnull(pair, "structure heads pair");
  nonnull(mask, "structure heads mask"); nonnull(aatype, "structure heads aatype");
  nonnull(atom14, "structure heads atom14"); nonnull(dgram, "structure heads distogram");
  nonnull(pae, "structure heads pae"); nonnull(plddt, "structure heads plddt");
  nonnull(expres, "structure heads expres"); nonnull(save, "structure heads save");
  if ((uintptr_t)dgram & 15) throw std::runtime_error("structure heads: distogram must be 16-byte aligned");
  Carver cv(save);
  ShSave<Carver> sv(cv, N, depth);
  const long M2 = (long)N * N;
  fold_fwd(st, w.fold, N, depth, single, pair, mask, key, enabled, dropout, sv.act, sv.traj,
           sv.fold, init_pos37);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)M2 * SH_DGRAM * 4 + (size_t)N * (3 * CS + 2 * SC) * 4 + 4096);
  float* h = ar.take_n<float>((size_t)M2 * SH_DGRAM);
  float* ra = ar.take_n<float>((size_t)N * CS);
  float* ri = ar.take_n<float>((size_t)N * CS);
  float* y0 = ar.take_n<float>((size_t)N * CS);
  float* rb = ar.take_n<float>((size_t)N * SC);
  {
    KTimed kt("sidechain.fwd", st);
    ln_f32_rows_fwd(st, single, N, CS, w.fold.ln_s_g, w.fold.ln_s_b, sv.init, sv.imean, sv.irstd);
    relu(st, sv.act, (long)N * CS, ra);
    relu(st, sv.init, (long)N * CS, ri);
    GemmF32 g0 = gemm_rows(N, SC, CS, ra, w.sc.wi0, sv.a[0]);
    g0.bias = w.sc.bi0;
    gemm_f32(st, g0, "sidechain.gemm_in0");
    GemmF32 g1 = gemm_rows(N, SC, CS, ri, w.sc.wi1, sv.a[0]);
    g1.bias = w.sc.bi1; g1.beta = 1.f;
    gemm_f32(st, g1, "sidechain.gemm_in1");
    for (int b = 0; b < 2; ++b) {
      relu(st, sv.a[b], (long)N * SC, rb);
      GemmF32 r1 = gemm_rows(N, SC, SC, rb, w.sc.wr1[b], sv.rh[b]);
      r1.bias = w.sc.br1[b]; r1.relu = true;
      gemm_f32(st, r1, "sidechain.gemm_res1");
      GemmF32 r2 = gemm_rows(N, SC, SC, sv.rh[b], w.sc.wr2[b], sv.a[b + 1]);
      r2.bias = w.sc.br2[b]; r2.add = sv.a[b];
      gemm_f32(st, r2, "sidechain.gemm_res2");
    }
    relu(st, sv.a[2], (long)N * SC, rb);
    GemmF32 ga = gemm_rows(N, NANG, SC, rb, w.sc.wa, sv.un);
    ga.bias = w.sc.ba;
    gemm_f32(st, ga, "sidechain.gemm_angles");
    hipLaunchKernelGGL(side_atoms_kernel, dim3((N + 63) / 64), dim3(64), 0, st, sv.un,
                       sv.traj + (size_t)(depth - 1) * N * 12, aatype, w.tab, N, atom14);
  }
  KTimed kt("heads.fwd", st);
  GemmF32 gd = gemm_rows((int)M2, SH_DGRAM, CZ, pair, w.hd.wdg, h);
  gd.bias = w.hd.bdg;
  gemm_f32(st, gd, "heads.gemm_distogram");
  symmetrise(st, h, dgram, N);
  GemmF32 gp = gemm_rows((int)M2, SH_PAE, CZ, pair, w.hd.wpae, pae);
  gp.bias = w.hd.bpae;
  gemm_f32(st, gp, "heads.gemm_pae");
  ln_f32_rows_fwd(st, sv.act, N, CS, w.hd.ln_g, w.hd.ln_b, y0, sv.lmean, sv.lrstd);
  GemmF32 p0 = gemm_rows(N, PL, CS, y0, w.hd.w0, sv.r0);
  p0.bias = w.hd.b0; p0.relu = true;
  gemm_f32(st, p0, "heads.gemm_plddt0");
  GemmF32 p1 = gemm_rows(N, PL, PL, sv.r0, w.hd.w1, sv.r1);
  p1.bias = w.hd.b1; p1.relu = true;
  gemm_f32(st, p1, "heads.gemm_plddt1");
  GemmF32 pl = gemm_rows(N, SH_PLDDT, PL, sv.r1, w.hd.wl, plddt);
  pl.bias = w.hd.bl;
  gemm_f32(st, pl, "heads.gemm_plddt");
  GemmF32 ge = gemm_rows(N, SH_EXPRES, CS, single, w.hd.wer, expres);
  ge.bias = w.hd.ber;
  gemm_f32(st, ge, "heads.gemm_expres");
}

void structheads_bwd(hipStream_t st, const StructHeadsW& w, int N, int depth, const float* single,
                     const float* pair, const float* mask, const float* aatype, bool dropout,
                     const void* save_c, const float* datom, const float* ddgram, const float* dpae,
                     const float* dplddt, const float* dexpres, float* dsingle, float* dpair) {
  sh_check(N, depth);
  nonnull(single, "structure heads single"); nonnull(pair, "structure heads pair");
  nonnull(mask, "structure heads mask"); nonnull(aatype, "structure heads aatype");
  nonnull(save_c, "structure heads save"); nonnull(dsingle, "structure heads dsingle");
  nonnull(dpair, "structure heads dpair");
  if (ddgram && ((uintptr_t)ddgram & 15)) throw std::runtime_error("structure heads: d(distogram) must be 16-byte aligned");
  // the save buffer's tail is the backward's scratch (d act, d initial act,
  // d traj survive the fold backward, which resets the scratch arena)
  void* save = const_cast<void*>(save_c);
  Carver cv(save);
  ShSave<Carver> sv(cv, N, depth);
  const long M2 = (long)N * N;
  {
    Arena& ar = arena();
    std::lock_guard<std::recursive_mutex> lk(ar.lock());
    ar.reset(st, (size_t)N * (3 * PL + 3 * SC + CS + NANG) * 4 + 4096);
    float* t0 = ar.take_n<float>((size_t)N * PL);
    float* t1 = ar.take_n<float>((size_t)N * PL);
    float* dy = ar.take_n<float>((size_t)N * CS);
    float* da = ar.take_n<float>((size_t)N * SC);
    float* db = ar.take_n<float>((size_t)N * SC);
    float* dh = ar.take_n<float>((size_t)N * SC);
    float* dun = ar.take_n<float>((size_t)N * NANG);
    // pLDDT head -> d act
    if (dplddt) {
      KTimed kt("heads.plddt_bwd", st);
      GemmF32 g = gemm_rows(N, PL, SH_PLDDT, dplddt, w.hd.wl, t1, true);
      g.gate = sv.r1; g.gate_is_mask = true;
      gemm_f32(st, g, "heads.gemm_plddt_dx");
      GemmF32 g1 = gemm_rows(N, PL, PL, t1, w.hd.w1, t0, true);
      g1.gate = sv.r0; g1.gate_is_mask = true;
      gemm_f32(st, g1, "heads.gemm_plddt1_dx");
      GemmF32 g0 = gemm_rows(N, CS, PL, t0, w.hd.w0, dy, true);
      gemm_f32(st, g0, "heads.gemm_plddt0_dx");
      ln_f32_rows_bwd(st, dy, sv.act, N, CS, w.hd.ln_g, sv.lmean, sv.lrstd, sv.d_act);
    } else {
      zero_f32(st, sv.d_act, (long)N * CS);
    }
    // sidechain -> d act, d initial act, d traj[-1]
    if (datom) {
      KTimed kt("sidechain.bwd", st);
      zero_f32(st, sv.d_traj, (long)(depth - 1) * N * 12);
      const float* trj = sv.traj + (size_t)(depth - 1) * N * 12;
      hipLaunchKernelGGL(side_atoms_bwd_kernel, dim3((N + 63) / 64), dim3(64), 0, st, sv.un, trj,
                         aatype, w.tab, N, datom, dun, sv.d_traj + (size_t)(depth - 1) * N * 12);
      GemmF32 g = gemm_rows(N, SC, NANG, dun, w.sc.wa, da, true);
      g.gate = sv.a[2]; g.gate_is_mask = true;
      gemm_f32(st, g, "sidechain.gemm_angles_dx");
      for (int b = 1; b >= 0; --b) {
        // da_b = da_{b+1} + ((da_{b+1} W2^T) * [h > 0]) W1^T * [a_b > 0]
        GemmF32 g2 = gemm_rows(N, SC, SC, da, w.sc.wr2[b], dh, true);
        g2.gate = sv.rh[b]; g2.gate_is_mask = true;
        gemm_f32(st, g2, "sidechain.gemm_res2_dx");
        GemmF32 g1 = gemm_rows(N, SC, SC, dh, w.sc.wr1[b], db, true);
        g1.gate = sv.a[b]; g1.gate_is_mask = true; g1.add = da;
        gemm_f32(st, g1, "sidechain.gemm_res1_dx");
        std::swap(da, db);
      }
      GemmF32 gi0 = gemm_rows(N, CS, SC, da, w.sc.wi0, sv.d_act, true);
      gi0.gate = sv.act; gi0.gate_is_mask = true; gi0.beta = 1.f;
      gemm_f32(st, gi0, "sidechain.gemm_in0_dx");
      GemmF32 gi1 = gemm_rows(N, CS, SC, da, w.sc.wi1, sv.d_init, true);
      gi1.gate = sv.init; gi1.gate_is_mask = true;
      gemm_f32(st, gi1, "sidechain.gemm_in1_dx");
    }
  }
  fold_bwd(st, w.fold, N, depth, single, pair, mask, dropout, sv.fold, sv.d_act,
           datom ? sv.d_traj : nullptr, dsingle, dpair);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)M2 * SH_DGRAM * 4 + (size_t)N * CS * 4 + 4096);
  float* dhs = ar.take_n<float>((size_t)M2 * SH_DGRAM);
  float* tmp = ar.take_n<float>((size_t)N * CS);
  KTimed kt("heads.bwd", st);
  if (datom) {
    // initial_act = LN(single): its LayerNorm backward, added to d single
    ln_f32_rows_bwd(st, sv.d_init, single, N, CS, w.fold.ln_s_g, sv.imean, sv.irstd, tmp);
    add_into(st, dsingle, tmp, (long)N * CS);
  }
  if (dexpres) {
    GemmF32 g = gemm_rows(N, CS, SH_EXPRES, dexpres, w.hd.wer, dsingle, true);
    g.beta = 1.f;
    gemm_f32(st, g, "heads.gemm_expres_dx");
  }
  if (ddgram) {
    symmetrise(st, ddgram, dhs, N);
    GemmF32 g = gemm_rows((int)M2, CZ, SH_DGRAM, dhs, w.hd.wdg, dpair, true);
    g.beta = 1.f;
    gemm_f32(st, g, "heads.gemm_distogram_dx");
  }
  if (dpae) {
    GemmF32 g = gemm_rows((int)M2, CZ, SH_PAE, dpae, w.hd.wpae, dpair, true);
    g.beta = 1.f;
    gemm_f32(st, g, "heads.gemm_pae_dx");
  }
}

}  // namespace bc2n
