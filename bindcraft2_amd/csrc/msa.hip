// MSA row attention with pair bias and MSA column attention, fwd + bwd.
//
// Row attention (H=8, D=32 over the N residues of each of the S rows):
//   LN(msa) -> xn;  LN(pair) fused with the [C_z -> H] bias projection;
//   GEMM qkvg; flash attention (rows = S, mask = msa_mask[s][k]); GEMM out +
//   residual (+ shared per-row dropout).  The backward returns both d(msa)
//   and d(pair) (through the bias projection and the pair LN).
// Column attention (H=8, D=32 over the S rows of each residue): same
//   projections; the S x S attention per (residue, head) is tiny (S <= 32)
//   and runs one wave per (residue, head) in registers.
// Reference: modules.py:500-563 (MSARowAttentionWithPairBias), :566-616
// (MSAColumnAttention); native/msarow.cuh:208-441, native/msacol.cuh:247-361.
#include "gemm.h"
#include "modules.h"
#include <cmath>

namespace bc2n {

namespace {

// Gated-attention weights shared by the row and column modules:
// [Wq|Wk|Wv|Wg] (C_in x 4HD) in both orientations, gate bias, output.
void attn_weights(WeightStore& ws, const std::string& P, AttnW& w) {
  const HostTensor& qw = ws.host(P + "attention/query_w");
  w.Cin = qw.shape[0];
  w.H = qw.shape[1];
  w.D = qw.shape[2];
  const int C = w.Cin, HD = w.H * w.D;
  const HostTensor& ow = ws.host(P + "attention/output_w");  // [H, D, Cout]
  w.Cout = ow.shape[2];
  const char* parts[4] = {"attention/query_w", "attention/key_w", "attention/value_w",
                          "attention/gating_w"};
  auto cat = [&]() {
    std::vector<float> c((size_t)C * 4 * HD);
    for (int p = 0; p < 4; ++p) {
      const HostTensor& t = ws.host(P + parts[p]);
      for (int r = 0; r < C; ++r)
        for (int j = 0; j < HD; ++j) c[(size_t)r * 4 * HD + p * HD + j] = t.data[(size_t)r * HD + j];
    }
    return c;
  };
  w.wqkvg = ws.derived<h16>("attn.wqkvg:" + P, [&] { return to_h16(cat()); });
  w.wqkvg_t = ws.derived<h16>("attn.wqkvg_t:" + P, [&] {
    std::vector<float> c = cat();
    return transpose_h16(c.data(), C, 4 * HD);
  });
  w.bqkvg = ws.derived<float>("attn.bqkvg:" + P, [&] {
    std::vector<float> b((size_t)4 * HD, 0.f);
    const HostTensor& gb = ws.host(P + "attention/gating_b");
    for (int j = 0; j < HD; ++j) b[3 * HD + j] = gb.data[j];
    return b;
  });
  w.wo = ws.derived<h16>("attn.wo:" + P, [&] { return to_h16(ow.data); });
  w.wo_t = ws.derived<h16>("attn.wo_t:" + P, [&] { return transpose_h16(ow.data.data(), HD, w.Cout); });
  w.bo = ws.f32(P + "attention/output_b");
  w.ln_g = ws.f32(P + "query_norm/scale");
  w.ln_b = ws.f32(P + "query_norm/offset");
}

// ------------------------------------------------- small-S column attention
// One wave per (residue j, head h); lane s_q < S owns one query row over all
// S keys (S <= 32).  q already carries D^-1/2 (no log2 scale here: scores
// are in natural units, clipped as the reference does); the mask of key row
// s is msa_mask[s][j].
constexpr int SA_D = 32;

__global__ __launch_bounds__(64) void small_attn_fwd_kernel(
    const h16* __restrict__ qkvg, long ld, int S, int N, int H,
    const float* __restrict__ mask, h16* __restrict__ o, h16* __restrict__ og, long ldo,
    float* __restrict__ lse) {
  const int j = blockIdx.x / H, h = blockIdx.x % H;
  const int lane = threadIdx.x;
  const int HD = H * SA_D;
  // every lane handles one query row (lane < S) over all keys
  if (lane >= S) return;
  const int sq = lane;
  const h16* q = qkvg + ((long)sq * N + j) * ld + h * SA_D;
  float qv[SA_D];
#pragma unroll
  for (int d = 0; d < SA_D; ++d) qv[d] = (float)q[d];
  float mx = -INFINITY;
  float sc[32];
  for (int sk = 0; sk < S; ++sk) {
    const h16* k = qkvg + ((long)sk * N + j) * ld + HD + h * SA_D;
    float s = 0.f;
#pragma unroll
    for (int d = 0; d < SA_D; ++d) s += qv[d] * (float)k[d];
    const float mb = MASK_BIAS * (mask[(long)sk * N + j] - 1.f);
    s = fminf(fmaxf(s + mb, -LOGIT_CLIP), LOGIT_CLIP);
    sc[sk] = s;
    mx = fmaxf(mx, s);
  }
  float sum = 0.f;
  for (int sk = 0; sk < S; ++sk) {
    sc[sk] = __expf(sc[sk] - mx);
    sum += sc[sk];
  }
  const float inv = 1.f / sum;
  float acc[SA_D];
#pragma unroll
  for (int d = 0; d < SA_D; ++d) acc[d] = 0.f;
  for (int sk = 0; sk < S; ++sk) {
    const h16* v = qkvg + ((long)sk * N + j) * ld + 2 * HD + h * SA_D;
    const float p = sc[sk] * inv;
#pragma unroll
    for (int d = 0; d < SA_D; ++d) acc[d] += p * (float)v[d];
  }
  const long row = (long)sq * N + j;
  const h16* g = qkvg + row * ld + 3 * HD + h * SA_D;
#pragma unroll
  for (int d = 0; d < SA_D; ++d) {
    o[row * ldo + h * SA_D + d] = (h16)acc[d];
    og[row * ldo + h * SA_D + d] = (h16)(acc[d] * sigmoidf_((float)g[d]));
  }
  lse[((long)j * H + h) * S + sq] = mx + __logf(sum);
}

// S = 1 (one sequence: the design step's MSA).  The softmax over one key is
// exactly 1 (exp(s - s) = 1), so o = v and the general kernels' arithmetic
// reduces to the lines below, bit for bit; one thread per (residue, head)
// instead of a 64-lane wave with one live lane.  The score is still formed
// (same order of products) for the saved lse.
__global__ __launch_bounds__(256) void small_attn1_fwd_kernel(
    const h16* __restrict__ qkvg, long ld, int N, int H, const float* __restrict__ mask,
    h16* __restrict__ o, h16* __restrict__ og, long ldo, float* __restrict__ lse) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * H) return;
  const int j = t / H, h = t % H;
  const int HD = H * SA_D;
  const h16* q = qkvg + (long)j * ld + h * SA_D;
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < SA_D / 8; ++c) {
    const h16x8 qa = ld8(q + 8 * c), ka = ld8(q + HD + 8 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) s += (float)qa[e] * (float)ka[e];
  }
  s = fminf(fmaxf(s + MASK_BIAS * (mask[j] - 1.f), -LOGIT_CLIP), LOGIT_CLIP);
#pragma unroll
  for (int c = 0; c < SA_D / 8; ++c) {
    const h16x8 v = ld8(q + 2 * HD + 8 * c), g = ld8(q + 3 * HD + 8 * c);
    h16x8 ov, gv;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float a = (float)v[e];
      ov[e] = (h16)a;
      gv[e] = (h16)(a * sigmoidf_((float)g[e]));
    }
    st8(o + (long)j * ldo + h * SA_D + 8 * c, ov);
    st8(og + (long)j * ldo + h * SA_D + 8 * c, gv);
  }
  lse[t] = s + __logf(1.f);
}

// dS = p (dP - Dsum) is exactly 0 at S = 1 (o = v, so dP and Dsum are the same
// products summed in the same order): dq = dk = 0, dv = dO.
__global__ __launch_bounds__(256) void small_attn1_bwd_kernel(
    const h16* __restrict__ qkvg, long ld, int N, int H, const h16* __restrict__ o,
    const h16* __restrict__ dog, long ldo, h16* __restrict__ dqkvg) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * H * (SA_D / 8)) return;
  const int c = t % (SA_D / 8), jh = t / (SA_D / 8);  // 8 channels of one (residue, head)
  const int j = jh / H, h = jh % H;
  const int HD = H * SA_D;
  const long orow = (long)j * ldo + h * SA_D + 8 * c;
  const h16x8 g = ld8(qkvg + (long)j * ld + 3 * HD + h * SA_D + 8 * c);
  const h16x8 dg = ld8(dog + orow), ov = ld8(o + orow);
  h16x8 dgate, dv;
  const h16x8 zero = {};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sg = sigmoidf_((float)g[e]);
    const float dgo = (float)dg[e];
    dgate[e] = f2h_sat(dgo * (float)ov[e] * sg * (1.f - sg));
    dv[e] = f2h_sat(dgo * sg);
  }
  h16* dq = dqkvg + (long)j * ld + h * SA_D + 8 * c;
  st8(dq, zero);
  st8(dq + HD, zero);
  st8(dq + 2 * HD, dv);
  st8(dq + 3 * HD, dgate);
}

// Backward, same decomposition; lane = query row.  dK/dV sums over queries
// go through LDS atomics of the one wave that owns the (j,h) pair.
__global__ __launch_bounds__(64) void small_attn_bwd_kernel(
    const h16* __restrict__ qkvg, long ld, int S, int N, int H,
    const float* __restrict__ mask, const h16* __restrict__ o, const h16* __restrict__ dog,
    long ldo, float qscale, h16* __restrict__ dqkvg) {
  __shared__ float dk_s[32][SA_D + 1];
  __shared__ float dv_s[32][SA_D + 1];
  const int j = blockIdx.x / H, h = blockIdx.x % H;
  const int lane = threadIdx.x;
  const int HD = H * SA_D;
  for (int i = lane; i < 32 * (SA_D + 1); i += 64) {
    (&dk_s[0][0])[i] = 0.f;
    (&dv_s[0][0])[i] = 0.f;
  }
  __syncthreads();
  if (lane < S) {
    const int sq = lane;
    const long row = (long)sq * N + j;
    const h16* q = qkvg + row * ld + h * SA_D;
    const h16* g = qkvg + row * ld + 3 * HD + h * SA_D;
    float qv[SA_D], dO[SA_D];
    float Dsum = 0.f;
#pragma unroll
    for (int d = 0; d < SA_D; ++d) {
      qv[d] = (float)q[d];
      const float sg = sigmoidf_((float)g[d]);
      const float dgo = (float)dog[row * ldo + h * SA_D + d];
      const float ov = (float)o[row * ldo + h * SA_D + d];
      dO[d] = dgo * sg;
      Dsum += dO[d] * ov;
      dqkvg[row * ld + 3 * HD + h * SA_D + d] = f2h_sat(dgo * ov * sg * (1.f - sg));
    }
    // softmax recomputed in full (S is small): exact even for a fully masked
    // column, where every clipped logit is -1e8 and f32 cannot carry an lse
    float sc[32], mx = -INFINITY;
    bool live[32];
    for (int sk = 0; sk < S; ++sk) {
      const h16* k = qkvg + ((long)sk * N + j) * ld + HD + h * SA_D;
      float s = 0.f;
#pragma unroll
      for (int d = 0; d < SA_D; ++d) s += qv[d] * (float)k[d];
      const float raw = s + MASK_BIAS * (mask[(long)sk * N + j] - 1.f);
      live[sk] = raw > -LOGIT_CLIP && raw < LOGIT_CLIP;
      sc[sk] = fminf(fmaxf(raw, -LOGIT_CLIP), LOGIT_CLIP);
      mx = fmaxf(mx, sc[sk]);
    }
    float sum = 0.f;
    for (int sk = 0; sk < S; ++sk) {
      sc[sk] = __expf(sc[sk] - mx);
      sum += sc[sk];
    }
    const float inv = 1.f / sum;
    float dq[SA_D];
#pragma unroll
    for (int d = 0; d < SA_D; ++d) dq[d] = 0.f;
    for (int sk = 0; sk < S; ++sk) {
      const long krow = (long)sk * N + j;
      const h16* k = qkvg + krow * ld + HD + h * SA_D;
      const h16* v = qkvg + krow * ld + 2 * HD + h * SA_D;
      float dp = 0.f;
#pragma unroll
      for (int d = 0; d < SA_D; ++d) dp += dO[d] * (float)v[d];
      const float p = sc[sk] * inv;
      const float ds = live[sk] ? p * (dp - Dsum) : 0.f;
#pragma unroll
      for (int d = 0; d < SA_D; ++d) {
        dq[d] += ds * (float)k[d];
        atomicAdd(&dk_s[sk][d], ds * qv[d]);
        atomicAdd(&dv_s[sk][d], p * dO[d]);
      }
    }
#pragma unroll
    for (int d = 0; d < SA_D; ++d) dqkvg[row * ld + h * SA_D + d] = f2h_sat(dq[d] * qscale);
  }
  __syncthreads();
  for (int i = lane; i < S * SA_D; i += 64) {
    const int sk = i / SA_D, d = i % SA_D;
    const long krow = (long)sk * N + j;
    // q was scaled by qscale: dK (unscaled k) = sum ds * q_scaled
    dqkvg[krow * ld + HD + h * SA_D + d] = f2h_sat(dk_s[sk][d]);
    dqkvg[krow * ld + 2 * HD + h * SA_D + d] = f2h_sat(dv_s[sk][d]);
  }
}

template <class A>
struct MsaRowSave {
  float *mean, *rstd, *pmean, *prstd, *lse;
  h16* bias;
  h16 *qkvg, *o;
  MsaRowSave(A& a, int S, int N, int Cm, int H) {
    const size_t R = (size_t)S * N, M = (size_t)N * N;
    mean = a.template take<float>(R);
    rstd = a.template take<float>(R);
    pmean = a.template take<float>(M);
    prstd = a.template take<float>(M);
    bias = a.template take<h16>((size_t)H * M);
    lse = a.template take<float>((size_t)S * H * N);
    qkvg = a.template take<h16>(R * 4 * Cm);
    o = a.template take<h16>(R * Cm);
  }
};

template <class A>
struct MsaColSave {
  float *mean, *rstd, *lse;
  h16 *qkvg, *o;
  MsaColSave(A& a, int S, int N, int Cm, int H) {
    const size_t R = (size_t)S * N;
    mean = a.template take<float>(R);
    rstd = a.template take<float>(R);
    lse = a.template take<float>((size_t)N * H * S);
    qkvg = a.template take<h16>(R * 4 * Cm);
    o = a.template take<h16>(R * Cm);
  }
};

void qkvg_gemm(hipStream_t st, const AttnW& w, long rows, const h16* xn, h16* qkvg, float qscale,
               const char* name) {
  const int HD = w.H * w.D;
  GemmArgs g;
  g.M = (int)rows; g.N = 4 * HD; g.K = w.Cin;
  g.A = xn; g.a_sm = w.Cin; g.a_sk = 1;
  g.B = w.wqkvg_t; g.b_sn = w.Cin; g.b_sk = 1;
  gemm<128, 128>(st, g, EpiScaledCols(qkvg, 4L * HD, w.bqkvg, qscale, HD), name);
}

void out_gemm(hipStream_t st, const AttnW& w, long rows, const h16* og, const float* in,
              float* out, const float* tbl, int nt, const char* name) {
  const int HD = w.H * w.D;
  GemmArgs g;
  g.M = (int)rows; g.N = w.Cout; g.K = HD;
  g.A = og; g.a_sm = HD; g.a_sk = 1;
  g.B = w.wo_t; g.b_sn = HD; g.b_sk = 1;
  gemm<128, 128>(st, g, EpiResidualRows(in, out, w.bo, tbl, nt, w.Cout, false), name);
}

// d(og) = (s * tbl * dout) . Wo^T, the dropout table and the cotangent scale
// s = *sc applied as A is loaded, with epilogue `epi`; after the attention
// backward, d(xn) = dqkvg . Wcat^T
template <class Epi>
void dout_gemm(hipStream_t st, const AttnW& w, long rows, const float* dout, const float* tbl,
               int nt, const Epi& epi, const char* name, const float* sc) {
  const int HD = w.H * w.D;
  GemmArgs g;
  g.M = (int)rows; g.N = HD; g.K = w.Cout;
  g.a_sm = w.Cout; g.a_sk = 1;
  g.B = w.wo; g.b_sn = w.Cout; g.b_sk = 1;
  gemm<128, 128>(st, g, epi, name, ALoadScaledRows{dout, tbl, nt, w.Cout, false, sc});
}

void dx_gemm(hipStream_t st, const AttnW& w, long rows, const h16* dqkvg, float* dxn,
             const char* name) {
  const int HD = w.H * w.D;
  GemmArgs g;
  g.M = (int)rows; g.N = w.Cin; g.K = 4 * HD;
  g.A = dqkvg; g.a_sm = 4L * HD; g.a_sk = 1;
  g.B = w.wqkvg; g.b_sn = 4L * HD; g.b_sk = 1;
  gemm<128, 128>(st, g, EpiStore<float>{dxn, w.Cin, 0, nullptr, w.Cin}, name);
}

}  // namespace

MsaRowW msarow_weights(WeightStore& ws, const std::string& P) {
  MsaRowW w;
  attn_weights(ws, P, w.a);
  w.pn_g = ws.f32(P + "feat_2d_norm/scale");
  w.pn_b = ws.f32(P + "feat_2d_norm/offset");
  w.w2d = ws.f32(P + "feat_2d_weights");
  w.Cz = ws.host(P + "feat_2d_weights").shape[0];
  const int H = w.a.H;
  if (w.Cz == 128 && H > 0 && H <= 16) {
    const HostTensor& g = ws.host(P + "feat_2d_norm/scale");
    const HostTensor& b = ws.host(P + "feat_2d_norm/offset");
    const HostTensor& wt = ws.host(P + "feat_2d_weights");  // [Cz][H]
    w.pb_frag = ws.derived<h16>("msarow.pb_frag:" + P,
                                [&] { return ln_bias_frags(g.data.data(), wt.data.data(), H); });
    w.pb_const = ws.derived<float>("msarow.pb_const:" + P,
                                   [&] { return ln_bias_const(b.data.data(), wt.data.data(), H); });
    w.pb_bwd_frag = ws.derived<float>(
        "msarow.pb_bwd_frag:" + P, [&] { return ln_bias_bwd_frags(g.data.data(), wt.data.data(), H); });
  }
  return w;
}

MsaColW msacol_weights(WeightStore& ws, const std::string& P) {
  MsaColW w;
  attn_weights(ws, P, w.a);
  return w;
}

size_t msarow_save_bytes(int S, int N, int Cm, int H) {
  Sizer s;
  MsaRowSave<Sizer> p(s, S, N, Cm, H);
  (void)p;
  return s.off;
}

size_t msacol_save_bytes(int S, int N, int Cm, int H) {
  Sizer s;
  MsaColSave<Sizer> p(s, S, N, Cm, H);
  (void)p;
  return s.off;
}

void msarow_fwd(hipStream_t st, const MsaRowW& w, int S, int N, const float* msa_in,
                const float* msa_mask, const float* pair, const float* tbl, float* msa_out,
                void* save) {
  nonnull(msa_in, "msarow msa"); nonnull(msa_mask, "msarow mask"); nonnull(pair, "msarow pair");
  nonnull(msa_out, "msarow out"); nonnull(save, "msarow save");
  const AttnW& a = w.a;
  if (a.D != 32 || a.Cin != a.Cout || a.H * a.D != a.Cin)
    throw std::runtime_error("msarow: unsupported widths");
  if (N % 32 != 0) throw std::runtime_error("msarow: N must be a multiple of 32");
  const int Cm = a.Cin, H = a.H, HD = H * a.D;
  const long R = (long)S * N, M = (long)N * N;
  Carver cv(save);
  MsaRowSave<Carver> sv(cv, S, N, Cm, H);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)R * Cm * 2 + (size_t)R * HD * 2 + 1024);
  h16* xn = ar.take_n<h16>((size_t)R * Cm);
  h16* og = ar.take_n<h16>((size_t)R * HD);
  {
    KTimed kt("msarow.ln", st);
    ln_fwd_f32(st, msa_in, R, Cm, 0, a.ln_g, a.ln_b, xn, sv.mean, sv.rstd, false, 0, nullptr,
               nullptr);
    if (w.pb_frag)
      ln_pair_bias_f32(st, pair, M, false, sv.pmean, sv.prstd, w.pb_frag, w.pb_const, H, sv.bias,
                       LOG2E);
    else
      ln_fwd_f32(st, pair, M, w.Cz, 0, w.pn_g, w.pn_b, nullptr, sv.pmean, sv.prstd, false, H,
                 w.w2d, sv.bias, LOG2E);
  }
  qkvg_gemm(st, a, R, xn, sv.qkvg, LOG2E / std::sqrt((float)a.D), "msarow.gemm_qkvg");
  AttnArgs at;
  at.R = S; at.H = H; at.N = N; at.D = a.D;
  at.qkvg = sv.qkvg; at.ld = 4L * HD;
  at.mask = msa_mask; at.mask_sr = N; at.mask_sk = 1;
  at.bias = sv.bias;
  at.o = sv.o; at.og = og; at.ldo = HD;
  at.lse = sv.lse;
  at.site = 1;
  attn_fwd(st, at);
  out_gemm(st, a, R, og, msa_in, msa_out, tbl, N, "msarow.gemm_out");
}

// Everything of the backward but the pair term: dmsa_in, and the gradient of
// the pair bias [H][N][N] left in the calling lane's arena (the returned
// pointer, valid until that arena's next call).  sc must be given.
const float* msarow_bwd_msa(hipStream_t st, const MsaRowW& w, int S, int N, const float* msa_in,
                            const float* msa_mask, const float* tbl, const void* save,
                            const float* dmsa_out, float* dmsa_in, const float* sc) {
  nonnull(msa_in, "msarow msa"); nonnull(msa_mask, "msarow mask");
  nonnull(save, "msarow save"); nonnull(dmsa_out, "msarow dout"); nonnull(dmsa_in, "msarow din");
  nonnull(sc, "msarow scale");
  const AttnW& a = w.a;
  const int Cm = a.Cin, H = a.H, HD = H * a.D;
  const long R = (long)S * N, M = (long)N * N;
  Carver cv(const_cast<void*>(save));
  MsaRowSave<Carver> sv(cv, S, N, Cm, H);
  AttnBwdArgs b;
  b.rows_per_chunk = attn_rows_per_chunk(S, N, H, a.D);
  const int nch = attn_bwd_nchunk(S, b.rows_per_chunk);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  sc = module_scale(st, sc, dmsa_out, R * Cm);
  Sizer need;
  need.take<h16>((size_t)R * HD);
  need.take<float>((size_t)S * H * N);
  need.take<h16>((size_t)R * 4 * HD);
  need.take<float>((size_t)nch * H * M);
  need.take<float>((size_t)H * M);
  need.take<float>((size_t)R * Cm);
  ar.reset(st, need.off);
  b.dO = ar.take_n<h16>((size_t)R * HD);
  b.nDsum = ar.take_n<float>((size_t)S * H * N);
  b.dqkvg = ar.take_n<h16>((size_t)R * 4 * HD);
  b.dbias_part = ar.take_n<float>((size_t)nch * H * M);
  b.dbias = ar.take_n<float>((size_t)H * M);
  float* dxn = ar.take_n<float>((size_t)R * Cm);
  EpiGateBwd eg;
  eg.qkvg = sv.qkvg; eg.ld = 4L * HD; eg.o = sv.o; eg.dO = b.dO; eg.dqkvg = b.dqkvg;
  eg.nDsum = b.nDsum; eg.HD = HD; eg.H = H; eg.D = a.D; eg.Ntok = N;
  dout_gemm(st, a, R, dmsa_out, tbl, N, eg, "msarow.gemm_dout", sc);
  b.gate_done = true;
  AttnArgs& at = b.f;
  at.R = S; at.H = H; at.N = N; at.D = a.D;
  at.qkvg = sv.qkvg; at.ld = 4L * HD;
  at.mask = msa_mask; at.mask_sr = N; at.mask_sk = 1;
  at.bias = sv.bias;
  at.o = sv.o; at.og = nullptr; at.ldo = HD;
  at.lse = sv.lse;
  at.site = 1;
  b.scale = 1.f / std::sqrt((float)a.D);
  attn_bwd(st, b);
  dx_gemm(st, a, R, b.dqkvg, dxn, "msarow.gemm_dx");
  KTimed kt("msarow.ln_bwd", st);
  ln_bwd_f32(st, dxn, msa_in, R, Cm, 0, a.ln_g, sv.mean, sv.rstd, dmsa_in, true, 0, nullptr,
             nullptr, dmsa_out, sc + 1);
  return b.dbias;
}

// The pair term: dpair += the pair LayerNorm's backward of the bias
// projection's gradient (the only way the pair enters the row attention).
long msarow_bwd_pair(hipStream_t st, const MsaRowW& w, int S, int N, const float* pair,
                     const void* save, const float* dbias, float* dpair, const float* sc,
                     float* amax_part) {
  nonnull(pair, "msarow pair"); nonnull(save, "msarow save"); nonnull(dbias, "msarow dbias");
  nonnull(dpair, "msarow dpair");
  const AttnW& a = w.a;
  const int Cm = a.Cin, H = a.H;
  const long M = (long)N * N;
  Carver cv(const_cast<void*>(save));
  MsaRowSave<Carver> sv(cv, S, N, Cm, H);
  KTimed kt("msarow.ln_bwd_pair", st);
  if (w.pb_bwd_frag)
    return ln_pair_bias_bwd_f32(st, pair, M, sv.pmean, sv.prstd, w.pb_bwd_frag, H, dbias, dpair,
                                sc + 1, amax_part, amax_part ? CT_FUSED : 0);
  ln_bwd_f32(st, nullptr, pair, M, w.Cz, 0, w.pn_g, sv.pmean, sv.prstd, dpair, true, H, dbias,
             w.w2d, nullptr, sc + 1);
  return 0;
}

long msarow_bwd(hipStream_t st, const MsaRowW& w, int S, int N, const float* msa_in,
                const float* msa_mask, const float* pair, const float* tbl, const void* save,
                const float* dmsa_out, float* dmsa_in, float* dpair, const float* sc,
                float* amax_part) {
  nonnull(pair, "msarow pair"); nonnull(dpair, "msarow dpair");
  nonnull(dmsa_out, "msarow dout");
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  sc = module_scale(st, sc, dmsa_out, (long)S * N * w.a.Cin);
  const float* dbias = msarow_bwd_msa(st, w, S, N, msa_in, msa_mask, tbl, save, dmsa_out, dmsa_in,
                                      sc);
  return msarow_bwd_pair(st, w, S, N, pair, save, dbias, dpair, sc, amax_part);
}

void msacol_fwd(hipStream_t st, const MsaColW& w, int S, int N, const float* msa_in,
                const float* msa_mask, const float* tbl, float* msa_out, void* save) {
  nonnull(msa_in, "msacol msa"); nonnull(msa_mask, "msacol mask"); nonnull(msa_out, "msacol out");
  nonnull(save, "msacol save");
  const AttnW& a = w.a;
  if (a.D != 32 || S > 32) throw std::runtime_error("msacol: D must be 32 and S <= 32");
  const int Cm = a.Cin, H = a.H, HD = H * a.D;
  const long R = (long)S * N;
  Carver cv(save);
  MsaColSave<Carver> sv(cv, S, N, Cm, H);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)R * Cm * 2 + (size_t)R * HD * 2 + 1024);
  h16* xn = ar.take_n<h16>((size_t)R * Cm);
  h16* og = ar.take_n<h16>((size_t)R * HD);
  {
    KTimed kt("msacol.ln", st);
    ln_fwd_f32(st, msa_in, R, Cm, 0, a.ln_g, a.ln_b, xn, sv.mean, sv.rstd, false, 0, nullptr,
               nullptr);
  }
  qkvg_gemm(st, a, R, xn, sv.qkvg, 1.f / std::sqrt((float)a.D), "msacol.gemm_qkvg");
  {
    KTimed kt("msacol.attn", st);
    if (S == 1)
      hipLaunchKernelGGL(small_attn1_fwd_kernel, dim3((N * H + 255) / 256), dim3(256), 0, st,
                         sv.qkvg, 4L * HD, N, H, msa_mask, sv.o, og, (long)HD, sv.lse);
    else
      hipLaunchKernelGGL(small_attn_fwd_kernel, dim3(N * H), dim3(64), 0, st, sv.qkvg, 4L * HD, S,
                         N, H, msa_mask, sv.o, og, (long)HD, sv.lse);
  }
  out_gemm(st, a, R, og, msa_in, msa_out, tbl, N, "msacol.gemm_out");
}

void msacol_bwd(hipStream_t st, const MsaColW& w, int S, int N, const float* msa_in,
                const float* msa_mask, const float* tbl, const void* save,
                const float* dmsa_out, float* dmsa_in, const float* sc) {
  nonnull(msa_in, "msacol msa"); nonnull(msa_mask, "msacol mask"); nonnull(save, "msacol save");
  nonnull(dmsa_out, "msacol dout"); nonnull(dmsa_in, "msacol din");
  const AttnW& a = w.a;
  const int Cm = a.Cin, H = a.H, HD = H * a.D;
  const long R = (long)S * N;
  Carver cv(const_cast<void*>(save));
  MsaColSave<Carver> sv(cv, S, N, Cm, H);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  sc = module_scale(st, sc, dmsa_out, R * Cm);
  Sizer need;
  need.take<h16>((size_t)R * HD);
  need.take<h16>((size_t)R * 4 * HD);
  need.take<float>((size_t)R * Cm);
  ar.reset(st, need.off);
  h16* dog = ar.take_n<h16>((size_t)R * HD);
  h16* dqkvg = ar.take_n<h16>((size_t)R * 4 * HD);
  float* dxn = ar.take_n<float>((size_t)R * Cm);
  dout_gemm(st, a, R, dmsa_out, tbl, N, EpiStore<h16>{dog, HD, 0, nullptr, HD}, "msacol.gemm_dout",
            sc);
  {
    KTimed kt("msacol.attn_bwd", st);
    if (S == 1)
      hipLaunchKernelGGL(small_attn1_bwd_kernel, dim3((N * H * 4 + 255) / 256), dim3(256), 0, st,
                         sv.qkvg, 4L * HD, N, H, sv.o, dog, (long)HD, dqkvg);
    else
      hipLaunchKernelGGL(small_attn_bwd_kernel, dim3(N * H), dim3(64), 0, st, sv.qkvg, 4L * HD, S,
                         N, H, msa_mask, sv.o, dog, (long)HD, 1.f / std::sqrt((float)a.D), dqkvg);
  }
  dx_gemm(st, a, R, dqkvg, dxn, "msacol.gemm_dx");
  KTimed kt("msacol.ln_bwd", st);
  ln_bwd_f32(st, dxn, msa_in, R, Cm, 0, a.ln_g, sv.mean, sv.rstd, dmsa_in, true, 0, nullptr,
             nullptr, dmsa_out, sc + 1);
}

}  // namespace bc2n
