// Outer product mean, forward and backward, reassociated so that nothing of
// size N*N*O*O is ever formed:
//   R'[s,j,(c,f)] = sum_e right[s,j,e] W[c,e,f]          (small GEMM)
//   out[i,(j,f)]  = sum_(s,c) left[s,i,c] R'[s,j,c,f]      (one GEMM, K = S*O)
//   pair[i,j,f]  += (out + b[f]) / (1e-3 + sum_s mask[s,i] mask[s,j])
// Backward: d_act = dout * 1/(eps + norm);
//   dleft  = d_act . R'^T  (split over K, summed in a fixed order)
//   dR'    = left^T . d_act
//   dright = dR' . W^T     (split over K)
//   d(xn)  = [dleft|dright]*mask . [Wl|Wr]^T ; LayerNorm backward into dmsa.
// Reference: modules.py:1128-1212 (OuterProductMean); the reassociation is
// the one native/opm.cuh:7-24 describes (native/README.md:577-606).
#include "gemm.h"
#include "modules.h"

namespace bc2n {

namespace {

// lr = (acc + b) * mask -> left_t [N][S][O] and right [S*N][O] (h16)
struct EpiOpmLR : EpiRows {
  h16 *left_t, *right;
  const float *b, *mask;
  int S, N, O;
  EpiOpmLR(h16* l, h16* r, const float* bb, const float* mk, int s, int n, int o)
      : left_t(l), right(r), b(bb), mask(mk), S(s), N(n), O(o) {}
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const int s = m / N, r = m % N;
    const float mk = mask[m];
    float bb[8], x[8];
    ld_f8(b + n, bb);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (v[e] + bb[e]) * mk;
    if (n < O) st_h8f(left_t + ((long)r * S + s) * O + n, x);
    else st_h8f(right + (long)m * O + (n - O), x);
  }
};

// R'[(s,j)][(c,f)] -> Rp[(j,f)][(s,c)]  (the main GEMM's K-contiguous B)
struct EpiOpmR : EpiRows {
  h16* rp;
  int S, N, O, C;
  EpiOpmR(h16* r, int s, int n, int o, int c) : rp(r), S(s), N(n), O(o), C(c) {}
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const int s = m / N, jj = m % N;
    const int c = n / C, f0 = n % C;  // 8 columns share c (C % 8 == 0)
#pragma unroll
    for (int e = 0; e < 8; ++e) rp[(((long)jj * C + f0 + e) * S + s) * O + c] = (h16)v[e];
  }
};

// pair_out[i][j][f] = pair_in + tbl[j][f] * (acc + b[f]) * normf[i][j]
struct EpiOpmOut : EpiRows {
  const float* in;
  float* out;
  const float *b, *normf, *tbl;
  int N, C;
  EpiOpmOut(const float* i, float* o, const float* bb, const float* nf, const float* t, int n, int c)
      : in(i), out(o), b(bb), normf(nf), tbl(t), N(n), C(c) {}
  __device__ __forceinline__ void row(int, int i, int n, const float (&v)[8]) const {
    const int jj = n / C, f0 = n % C;
    const float nf = normf[(long)i * N + jj];
    float bb[8], x[8], r[8];
    ld_f8(b + f0, bb);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (v[e] + bb[e]) * nf;
    if (tbl) {
      float tt[8];
      ld_f8(tbl + (long)jj * C + f0, tt);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= tt[e];
    }
    const long o = (long)i * N * C + n;
    ld_f8(in + o, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] += x[e];
    st_f8(out + o, r);
  }
};

// dR'[(s,c)][(j,f)] -> dRp2[(s,j)][(c,f)] (h16)
struct EpiOpmDR : EpiRows {
  h16* d;
  int S, N, O, C;
  EpiOpmDR(h16* dd, int s, int n, int o, int c) : d(dd), S(s), N(n), O(o), C(c) {}
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const int s = m / O, c = m % O;
    const int jj = n / C, f0 = n % C;
    st_h8f(d + ((long)s * N + jj) * O * C + (long)c * C + f0, v);
  }
};

__global__ void opm_norm_kernel(const float* __restrict__ mask, int S, int N,
                                float* __restrict__ normf) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)N * N) return;
  const int i = (int)(idx / N), j = (int)(idx % N);
  float s = 0.f;
  for (int r = 0; r < S; ++r) s += mask[(long)r * N + i] * mask[(long)r * N + j];
  normf[idx] = 1.f / (1e-3f + s);
}

// d_act[i][(j,f)] = h16(s * dout * tbl[j][f] * normf[i][j]), s = sc[0] (the
// cotangent scale)
// 8 consecutive channels a thread (C % 8 == 0): 16-byte store, 32-bit index
// math (N * N * C < 2^31 for N <= 1024, C <= 128)
__global__ void opm_dact_kernel(const float* __restrict__ dout, const float* __restrict__ tbl,
                                const float* __restrict__ normf, int N, int C,
                                const float* __restrict__ sc, h16* __restrict__ dact) {
  const int v = blockIdx.x * blockDim.x + threadIdx.x;  // 8-channel group
  const int c8 = C / 8;
  if (v >= N * N * c8) return;
  const int ij = v / c8, f = (v - ij * c8) * 8;
  const float s = normf[ij] * sc[0];
  const float4* d4 = reinterpret_cast<const float4*>(dout + (long)ij * C + f);
  const float4 a = d4[0], b = d4[1];
  float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  if (tbl) {
    const float4* t4 = reinterpret_cast<const float4*>(tbl + (long)(ij % N) * C + f);
    const float4 ta = t4[0], tb = t4[1];
    const float t[8] = {ta.x, ta.y, ta.z, ta.w, tb.x, tb.y, tb.z, tb.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] *= t[e];
  }
  h16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = f2h_sat(x[e] * s);
  st8(dact + (long)ij * C + f, o);
}

// dlr[(s,r)][col0 + c] = mask[s][r] * sum_chunk part[chunk][row(r,s)][c]
// left:  part rows are residues r, columns (s,c);   right: rows (s,r), cols c
__global__ void opm_reduce_kernel(const float* __restrict__ part, int nch, long chunk_stride,
                                  int rows, int cols, const float* __restrict__ mask, int S, int N,
                                  int O, bool left, h16* __restrict__ dlr) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (long)rows * cols) return;
  // eight partials loaded at a time (in flight together), added in chunk order
  float s = 0.f;
  int ch = 0;
  for (; ch + 8 <= nch; ch += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = part[(long)(ch + u) * chunk_stride + idx];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; ch < nch; ++ch) s += part[(long)ch * chunk_stride + idx];
  const int row = (int)(idx / cols), col = (int)(idx % cols);
  int sr, r, c;
  if (left) { r = row; sr = col / O; c = col % O; }
  else { sr = row / N; r = row % N; c = col; }
  const long m = (long)sr * N + r;
  dlr[m * 2 * O + (left ? 0 : O) + c] = f2h_sat(s * mask[m]);
}

template <class A>
struct OpmSave {
  float *mean, *rstd, *normf;
  h16 *left_t, *rp;
  OpmSave(A& a, int S, int N, int O, int C) {
    mean = a.template take<float>((size_t)S * N);
    rstd = a.template take<float>((size_t)S * N);
    normf = a.template take<float>((size_t)N * N);
    left_t = a.template take<h16>((size_t)N * S * O);
    rp = a.template take<h16>((size_t)N * C * S * O);
  }
};

}  // namespace

OpmW opm_weights(WeightStore& ws, const std::string& P) {
  OpmW w;
  const HostTensor& lw = ws.host(P + "left_projection/weights");  // [Cm, O]
  const HostTensor& rw = ws.host(P + "right_projection/weights");
  const HostTensor& ow = ws.host(P + "output_w");                 // [O, O, C]
  w.Cm = lw.shape[0];
  w.O = lw.shape[1];
  w.C = ow.shape[2];
  const int Cm = w.Cm, O = w.O, C = w.C;
  w.ln_g = ws.f32(P + "layer_norm_input/scale");
  w.ln_b = ws.f32(P + "layer_norm_input/offset");
  w.bo = ws.f32(P + "output_b");
  w.blr = ws.derived<float>("opm.blr:" + P, [&] {
    std::vector<float> b(2 * O);
    const HostTensor& lb = ws.host(P + "left_projection/bias");
    const HostTensor& rb = ws.host(P + "right_projection/bias");
    for (int e = 0; e < O; ++e) { b[e] = lb.data[e]; b[O + e] = rb.data[e]; }
    return b;
  });
  auto wlr = [&]() {
    std::vector<float> c((size_t)Cm * 2 * O);
    for (int r = 0; r < Cm; ++r)
      for (int e = 0; e < O; ++e) {
        c[(size_t)r * 2 * O + e] = lw.data[(size_t)r * O + e];
        c[(size_t)r * 2 * O + O + e] = rw.data[(size_t)r * O + e];
      }
    return c;
  };
  w.wlr = ws.derived<h16>("opm.wlr:" + P, [&] { return to_h16(wlr()); });
  w.wlr_t = ws.derived<h16>("opm.wlr_t:" + P, [&] {
    std::vector<float> c = wlr();
    return transpose_h16(c.data(), Cm, 2 * O);
  });
  // wt[(c,f)][e] = W[c,e,f]; wt2[e][(c,f)] = W[c,e,f]
  w.wt = ws.derived<h16>("opm.wt:" + P, [&] {
    std::vector<h16> t((size_t)O * C * O);
    for (int c = 0; c < O; ++c)
      for (int e = 0; e < O; ++e)
        for (int f = 0; f < C; ++f)
          t[((size_t)c * C + f) * O + e] = (h16)ow.data[((size_t)c * O + e) * C + f];
    return t;
  });
  w.wt2 = ws.derived<h16>("opm.wt2:" + P, [&] {
    std::vector<h16> t((size_t)O * O * C);
    for (int c = 0; c < O; ++c)
      for (int e = 0; e < O; ++e)
        for (int f = 0; f < C; ++f)
          t[(size_t)e * O * C + (size_t)c * C + f] = (h16)ow.data[((size_t)c * O + e) * C + f];
    return t;
  });
  return w;
}

size_t opm_save_bytes(int S, int N, int O, int C) {
  Sizer s;
  OpmSave<Sizer> p(s, S, N, O, C);
  (void)p;
  return s.off;
}

// The MSA half of the forward: LayerNorm, the mask norm and the left / right
// projections, all into the save-set; nothing here reads the pair, so a
// stack can issue it as soon as the MSA input exists.
void opm_fwd_msa(hipStream_t st, const OpmW& w, int S, int N, const float* msa,
                 const float* msa_mask, void* save) {
  nonnull(msa, "opm msa"); nonnull(msa_mask, "opm mask"); nonnull(save, "opm save");
  const int Cm = w.Cm, O = w.O, C = w.C;
  if ((S * O) % 32 != 0 || N % 32 != 0) throw std::runtime_error("opm: S*O and N must be multiples of 32");
  const long R = (long)S * N;
  Carver cv(save);
  OpmSave<Carver> sv(cv, S, N, O, C);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)R * Cm * 2 + (size_t)R * O * 2 + 1024);
  h16* xn = ar.take_n<h16>((size_t)R * Cm);
  h16* right = ar.take_n<h16>((size_t)R * O);
  {
    KTimed kt("opm.ln", st);
    ln_fwd_f32(st, msa, R, Cm, 0, w.ln_g, w.ln_b, xn, sv.mean, sv.rstd, false, 0, nullptr, nullptr);
    const long nn = (long)N * N;
    hipLaunchKernelGGL(opm_norm_kernel, dim3((unsigned)((nn + 255) / 256)), dim3(256), 0, st,
                       msa_mask, S, N, sv.normf);
  }
  GemmArgs g1;
  g1.M = (int)R; g1.N = 2 * O; g1.K = Cm;
  g1.A = xn; g1.a_sm = Cm; g1.a_sk = 1;
  g1.B = w.wlr_t; g1.b_sn = Cm; g1.b_sk = 1;
  gemm<64, 64>(st, g1, EpiOpmLR(sv.left_t, right, w.blr, msa_mask, S, N, O), "opm.gemm_lr");
  GemmArgs g2;
  g2.M = (int)R; g2.N = O * C; g2.K = O;
  g2.A = right; g2.a_sm = O; g2.a_sk = 1;
  g2.B = w.wt; g2.b_sn = O; g2.b_sk = 1;
  gemm<64, 64>(st, g2, EpiOpmR(sv.rp, S, N, O, C), "opm.gemm_r");
}

// The pair half: the outer product of the saved projections, normalised,
// added to the pair.
void opm_fwd_pair(hipStream_t st, const OpmW& w, int S, int N, const float* pair_in,
                  const float* tbl, float* pair_out, void* save) {
  nonnull(pair_in, "opm pair"); nonnull(pair_out, "opm out"); nonnull(save, "opm save");
  const int O = w.O, C = w.C;
  Carver cv(save);
  OpmSave<Carver> sv(cv, S, N, O, C);
  GemmArgs g3;
  g3.M = N; g3.N = N * C; g3.K = S * O;
  g3.A = sv.left_t; g3.a_sm = (long)S * O; g3.a_sk = 1;
  g3.B = sv.rp; g3.b_sn = (long)S * O; g3.b_sk = 1;
  gemm<128, 128>(st, g3, EpiOpmOut(pair_in, pair_out, w.bo, sv.normf, tbl, N, C), "opm.gemm_out");
}

void opm_fwd(hipStream_t st, const OpmW& w, int S, int N, const float* msa, const float* msa_mask,
             const float* pair_in, const float* tbl, float* pair_out, void* save) {
  opm_fwd_msa(st, w, S, N, msa, msa_mask, save);
  opm_fwd_pair(st, w, S, N, pair_in, tbl, pair_out, save);
}

void opm_bwd(hipStream_t st, const OpmW& w, int S, int N, const float* msa, const float* msa_mask,
             const float* tbl, const void* save, const float* dpair, const float* dmsa_out,
             float* dmsa_in, const float* sc) {
  nonnull(msa, "opm msa"); nonnull(msa_mask, "opm mask"); nonnull(save, "opm save");
  nonnull(dpair, "opm dpair"); nonnull(dmsa_out, "opm dout"); nonnull(dmsa_in, "opm din");
  const int Cm = w.Cm, O = w.O, C = w.C;
  const long R = (long)S * N, NC = (long)N * C;
  Carver cv(const_cast<void*>(save));
  OpmSave<Carver> sv(cv, S, N, O, C);
  // split-K plans: dleft over the N*C axis in chunks of 2 residues (256),
  // dright over the O*C axis in chunks of 256 -- chains of four 64-deep K
  // steps, and enough workgroups (N/2 x 4 and 16 x 4 at N = 224) to cover the
  // latency; the ordered reduce adds the chunks
  const int kc1 = 2 * C, nch1 = (int)((NC + kc1 - 1) / kc1);
  const int kc2 = 256, nch2 = (O * C + kc2 - 1) / kc2;
  if (NC % kc1 != 0 || (O * C) % kc2 != 0) throw std::runtime_error("opm: unsupported split");
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  sc = module_scale(st, sc, dpair, (long)N * NC);
  Sizer need;
  need.take<h16>((size_t)N * NC);
  need.take<float>((size_t)nch1 * N * S * O);
  need.take<h16>((size_t)R * O * C);
  need.take<float>((size_t)nch2 * R * O);
  need.take<h16>((size_t)R * 2 * O);
  need.take<float>((size_t)R * Cm);
  ar.reset(st, need.off);
  h16* dact = ar.take_n<h16>((size_t)N * NC);
  float* p1 = ar.take_n<float>((size_t)nch1 * N * S * O);
  h16* drp = ar.take_n<h16>((size_t)R * O * C);
  float* p2 = ar.take_n<float>((size_t)nch2 * R * O);
  h16* dlr = ar.take_n<h16>((size_t)R * 2 * O);
  float* dxn = ar.take_n<float>((size_t)R * Cm);
  {
    KTimed kt("opm.dact", st);
    if (C % 8 != 0) throw std::runtime_error("opm: C must be a multiple of 8");
    const long n = (long)N * NC / 8;
    hipLaunchKernelGGL(opm_dact_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, dpair,
                       tbl, sv.normf, N, C, sc, dact);
  }
  {  // dleft partials: [chunk][i][(s,c)]
    GemmArgs g;
    g.M = N; g.N = S * O; g.K = kc1; g.batch = nch1;
    g.A = dact; g.a_sm = NC; g.a_sk = 1; g.a_sb = kc1;
    g.B = sv.rp; g.b_sn = 1; g.b_sk = (long)S * O; g.b_sb = (long)kc1 * S * O;
    gemm<64, 64>(st, g, EpiStore<float>{p1, (long)S * O, (long)N * S * O, nullptr, S * O},
                 "opm.gemm_dleft");
    KTimed kt("opm.reduce", st);
    const long n = (long)N * S * O;
    hipLaunchKernelGGL(opm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p1,
                       nch1, n, N, S * O, msa_mask, S, N, O, true, dlr);
  }
  {  // dR' = left^T . d_act -> [(s,j)][(c,f)]
    GemmArgs g;
    g.M = S * O; g.N = (int)NC; g.K = N;
    g.A = sv.left_t; g.a_sm = 1; g.a_sk = (long)S * O;
    g.B = dact; g.b_sn = 1; g.b_sk = NC;
    gemm<64, 64>(st, g, EpiOpmDR(drp, S, N, O, C), "opm.gemm_drp");
  }
  {  // dright partials: [chunk][(s,j)][e]
    GemmArgs g;
    g.M = (int)R; g.N = O; g.K = kc2; g.batch = nch2;
    g.A = drp; g.a_sm = (long)O * C; g.a_sk = 1; g.a_sb = kc2;
    g.B = w.wt2; g.b_sn = (long)O * C; g.b_sk = 1; g.b_sb = kc2;
    gemm<64, 64>(st, g, EpiStore<float>{p2, O, R * O, nullptr, O}, "opm.gemm_dright");
    KTimed kt("opm.reduce", st);
    const long n = R * O;
    hipLaunchKernelGGL(opm_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p2,
                       nch2, n, (int)R, O, msa_mask, S, N, O, false, dlr);
  }
  GemmArgs g5;
  g5.M = (int)R; g5.N = Cm; g5.K = 2 * O;
  g5.A = dlr; g5.a_sm = 2 * O; g5.a_sk = 1;
  g5.B = w.wlr; g5.b_sn = 2 * O; g5.b_sk = 1;
  gemm<128, 128>(st, g5, EpiStore<float>{dxn, Cm, 0, nullptr, Cm}, "opm.gemm_dx");
  KTimed kt("opm.ln_bwd", st);
  ln_bwd_f32(st, dxn, msa, R, Cm, 0, w.ln_g, sv.mean, sv.rstd, dmsa_in, true, 0, nullptr, nullptr,
             dmsa_out, sc + 1);
}

}  // namespace bc2n
