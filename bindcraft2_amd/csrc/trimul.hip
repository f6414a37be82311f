// Triangle multiplication (outgoing 'ikc,jkc->ijc' / incoming 'kjc,kic->ijc'),
// AF2's fused-projection form, forward and backward.
//
// Forward:
//   LN (fast variance) -> xn bf16
//   GEMM xn . Wcat  (Wcat = [proj|gate] channel pairs interleaved in 16-wide
//        blocks, then gating_linear), fused epilogue:
//          a = mask * proj * sigmoid(gate)   -> left/right planes [I][N*N] bf16
//          g_out = sigmoid(gating_linear)  -> [M][C] bf16
//        (xn is kept; the backward recomputes the proj/gate pre-activations)
//   batched MFMA GEMM over the I channels (plane layouts pick out/in)  -> T f32
//   centre LN (fast variance) reading the channel-major T            -> Tn bf16
//   GEMM Tn . Wo + bo, fused: o kept, out = in + tbl * (o * g_out)
// Backward: the exact reverse with the contraction's two transposed GEMMs; the
// projection's gradient comes from a GEMM that recomputes the pre-activations
// from xn and turns them, with d(left|right), into the [proj|gate] columns of
// d(cat) in its epilogue.
// Reference: modules.py:1044-1088 (_fused_triangle_multiplication), :909-919
// (fast-variance LN); native/trimul_body.cuh:1183-1796 (TriMul).
#include "gemm.h"
#include "modules.h"

namespace bc2n {

namespace {

// GEMM column of projection channel ch (0..2I) and of its gate.
__host__ __device__ inline int col_proj(int ch) { return (ch / 16) * 32 + ch % 16; }
__host__ __device__ inline int col_gate(int ch) { return (ch / 16) * 32 + 16 + ch % 16; }

// Projection epilogue.  Tiles of the [proj|gate] columns (n0 < 4I) run in
// column mode: the thread of a proj column reads its gate column (16 to the
// right, same tile) from LDS and writes 8 consecutive m of the channel-major
// planes: a = mask * proj * sigmoid(gate) into left/right.  Tiles of
// gating_linear columns run in row mode: g_out[m][c] = sigmoid(acc + b).
struct EpiTrimulProj {
  static constexpr bool kHasCol = true;
  bf16 *left, *right;   // [I][M]
  bf16* gout;           // [M][C]
  const float *bp, *bg, *bgl, *mask;
  long M;
  int I, C;
  __device__ __forceinline__ bool col_mode(int n0) const { return n0 < 4 * I; }
  __device__ __forceinline__ void col(int, int m, int n, const float (&v)[8], const float* tp,
                                      int ldt) const {
    if ((n & 31) >= 16) return;  // gate column: done by its projection column
    const int ch = (n >> 5) * 16 + (n & 15);
    const float bpv = bp[ch], bgv = bg[ch];
    float mk[8];
    ld_f8(mask + m, mk);
    float pv[8], gv[8], av[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pv[e] = v[e] + bpv;
      gv[e] = tp[e * ldt + 16] + bgv;
      av[e] = mk[e] * pv[e] * sigmoidf_(gv[e]);
    }
    if (ch < I) st_b8f(left + (long)ch * M + m, av);
    else st_b8f(right + (long)(ch - I) * M + m, av);
  }
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const int c = n - 4 * I;
    if (c < 0 || c >= C) return;
    float bb[8], x[8];
    ld_f8(bgl + c, bb);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = sigmoidf_(v[e] + bb[e]);
    st_b8f(gout + (long)m * C + c, x);
  }
};

// o = acc + bo (kept, bf16); out[m] = in[m] + tbl[(m%nt)*C+c] * o * g_out
struct EpiTrimulOut : EpiRows {
  const float* in;
  float* out;
  const float* bo;
  const bf16* gout;
  bf16* osave;
  const float* tbl;
  int nt, C;
  EpiTrimulOut(const float* i, float* o, const float* b, const bf16* g, bf16* os, const float* t,
               int n, int c)
      : in(i), out(o), bo(b), gout(g), osave(os), tbl(t), nt(n), C(c) {}
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const long o = (long)m * C + n;
    float bb[8], ov[8], gv[8], r[8];
    ld_f8(bo + n, bb);
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] = v[e] + bb[e];
    st_b8f(osave + o, ov);
    ld_b8f(gout + o, gv);
#pragma unroll
    for (int e = 0; e < 8; ++e) gv[e] *= ov[e];
    if (tbl) {
      float tt[8];
      ld_f8(tbl + (long)(m % nt) * C + n, tt);
#pragma unroll
      for (int e = 0; e < 8; ++e) gv[e] *= tt[e];
    }
    ld_f8(in + o, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] += gv[e];
    st_f8(out + o, r);
  }
};

template <class A>
struct TriMulSave {
  float *mean, *rstd, *cmean, *crstd, *T;
  bf16 *xn, *left, *right, *gout, *osave;
  TriMulSave(A& a, int N, int C, int I) {
    const size_t M = (size_t)N * N;
    mean = a.template take<float>(M);
    rstd = a.template take<float>(M);
    cmean = a.template take<float>(M);
    crstd = a.template take<float>(M);
    T = a.template take<float>(M * I);
    xn = a.template take<bf16>(M * C);
    left = a.template take<bf16>(M * I);
    right = a.template take<bf16>(M * I);
    gout = a.template take<bf16>(M * C);
    osave = a.template take<bf16>(M * C);
  }
};

// Backward of the projection, as the epilogue of the GEMM xn . Wcat[:, :4I]
// that recomputes the [proj|gate] pre-activations.  Column pass: the thread of
// a proj column takes its gate column (16 to the right) from the staged tile
// and d(left|right) for 8 consecutive m (channel-major), and rewrites both
// columns of the tile with
//   dproj = da * mask * s,  dgate = da * mask * p * s(1-s),  s = sigmoid(gate);
// row pass: the rewritten tile goes to the row-major d(cat) columns.
struct EpiTrimulProjBwd {
  static constexpr bool kHasCol = true;
  static constexpr bool kTwoPhase = true;
  const bf16 *dl, *dr;  // [I][M]
  const float *bp, *bg, *mask;
  bf16* dcat;           // [M][ldcat]
  long M;
  int I, ldcat;
  __device__ __forceinline__ bool col_mode(int) const { return true; }
  __device__ __forceinline__ void col(int, int m, int n, const float (&v)[8], float* tp,
                                      int ldt) const {
    if ((n & 31) >= 16) return;  // gate column: done by its projection column
    const int ch = (n >> 5) * 16 + (n & 15);
    const float bpv = bp[ch], bgv = bg[ch];
    float mk[8], da[8];
    ld_f8(mask + m, mk);
    ld_b8f((ch < I ? dl + (long)ch * M : dr + (long)(ch - I) * M) + m, da);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pv = v[e] + bpv;
      const float sg = sigmoidf_(tp[e * ldt + 16] + bgv);
      const float a = da[e] * mk[e];
      tp[e * ldt] = a * sg;
      tp[e * ldt + 16] = a * pv * sg * (1.f - sg);
    }
  }
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    st_b8f(dcat + (long)m * ldcat + n, v);
  }
};

// A loader of the output-projection backward GEMM: d = tbl*dout;
// A = d*g_out (the GEMM operand) and, as a side output,
// dcat[m][off + c] = d * o * g(1-g)   (gating_linear pre-activation grad).
struct ALoadTrimulOut {
  static constexpr bool kDirect = false;
  static constexpr bool kSide = true;
  const float* dout;
  const float* tbl;
  const bf16* gout;
  const bf16* osave;
  bf16* dcat;
  int C, ldcat, off, nt;
  __device__ __forceinline__ bf16x8 operator()(int, int m, int k) const {
    const long i = (long)m * C + k;
    float d[8], gv[8], ov[8];
    ld_f8(dout + i, d);
    if (tbl) {
      float t[8];
      ld_f8(tbl + (long)(m % nt) * C + k, t);
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] *= t[e];
    }
    ld_b8f(gout + i, gv);
    ld_b8f(osave + i, ov);
    bf16x8 a, dc;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = (bf16)(d[e] * gv[e]);
      dc[e] = (bf16)(d[e] * ov[e] * gv[e] * (1.f - gv[e]));
    }
    st8(dcat + (long)m * ldcat + off + k, dc);
    return a;
  }
};

}  // namespace

TriMulW trimul_weights(WeightStore& ws, const std::string& P) {
  TriMulW w;
  const HostTensor& pw = ws.host(P + "projection/weights");  // [C, 2I]
  w.C = pw.shape[0];
  w.I = pw.shape[1] / 2;
  const int C = w.C, I = w.I, NC = 4 * I + C;
  if (I % 16 != 0 || C % 64 != 0) throw std::runtime_error("trimul: widths must be multiples of 16/64");
  w.ln_g = ws.f32(P + "left_norm_input/scale");
  w.ln_b = ws.f32(P + "left_norm_input/offset");
  w.cn_g = ws.f32(P + "center_norm/scale");
  w.cn_b = ws.f32(P + "center_norm/offset");
  w.bp = ws.f32(P + "projection/bias");
  w.bg = ws.f32(P + "gate/bias");
  w.bgl = ws.f32(P + "gating_linear/bias");
  w.bo = ws.f32(P + "output_projection/bias");
  // Wcat [C][NC] in GEMM column order
  auto cat = [&]() {
    const HostTensor& gw = ws.host(P + "gate/weights");
    const HostTensor& lw = ws.host(P + "gating_linear/weights");
    std::vector<float> c((size_t)C * NC);
    for (int r = 0; r < C; ++r) {
      for (int ch = 0; ch < 2 * I; ++ch) {
        c[(size_t)r * NC + col_proj(ch)] = pw.data[(size_t)r * 2 * I + ch];
        c[(size_t)r * NC + col_gate(ch)] = gw.data[(size_t)r * 2 * I + ch];
      }
      for (int j = 0; j < C; ++j) c[(size_t)r * NC + 4 * I + j] = lw.data[(size_t)r * C + j];
    }
    return c;
  };
  w.wcat = ws.derived<bf16>("trimul.wcat:" + P, [&] { return to_bf16(cat()); });
  w.wcat_t = ws.derived<bf16>("trimul.wcat_t:" + P, [&] {
    std::vector<float> c = cat();
    return transpose_bf16(c.data(), C, NC);
  });
  const HostTensor& ow = ws.host(P + "output_projection/weights");  // [I, C]
  w.wo = ws.derived<bf16>("trimul.wo:" + P, [&] { return to_bf16(ow.data); });
  w.wo_t = ws.derived<bf16>("trimul.wo_t:" + P, [&] { return transpose_bf16(ow.data.data(), I, C); });
  return w;
}

size_t trimul_save_bytes(int N, int C, int I) {
  Sizer s;
  TriMulSave<Sizer> plan(s, N, C, I);
  (void)plan;
  return s.off;
}

static void trimul_check(int N) {
  if (N <= 0 || N % 32 != 0) throw std::runtime_error("trimul: N must be a positive multiple of 32");
}

// One batched contraction (operands described by `g`, one channel plane per
// batch entry): the dedicated kernel for N <= 256, the tiled GEMM beyond.
template <class OutT>
static void contract(hipStream_t st, const GemmArgs& g, OutT* C, const char* name) {
  {
    KTimed kt(name, st);
    float* cf = nullptr;
    bf16* cb = nullptr;
    if constexpr (sizeof(OutT) == 4) cf = C;
    else cb = C;
    if (trimul_contract(st, g.M, g.batch, g.A, g.a_sk == 1, g.B, g.b_sk == 1, cf, cb)) return;
  }
  gemm<64, 64>(st, g, EpiStore<OutT>{C, g.N, (long)g.M * g.N, nullptr, g.N}, name);
}

// Contraction operand layouts for one channel plane (row-major N x N).
static void contraction_fwd(hipStream_t st, bool outgoing, int N, int I, const bf16* L,
                            const bf16* R, float* T) {
  const long M = (long)N * N;
  GemmArgs g;
  g.M = N; g.N = N; g.K = N; g.batch = I;
  if (outgoing) {  // T[i][j] = sum_k L[i][k] R[j][k]
    g.A = L; g.a_sm = N; g.a_sk = 1;
    g.B = R; g.b_sn = N; g.b_sk = 1;
  } else {         // T[i][j] = sum_k R[k][i] L[k][j]
    g.A = R; g.a_sm = 1; g.a_sk = N;
    g.B = L; g.b_sn = 1; g.b_sk = N;
  }
  g.a_sb = M; g.b_sb = M;
  contract<float>(st, g, T, "trimul.contract_fwd");
}

void trimul_fwd(hipStream_t st, const TriMulW& w, bool outgoing, int N, const float* pair_in,
                const float* mask, const float* tbl, float* pair_out, void* save) {
  trimul_check(N);
  nonnull(pair_in, "trimul pair_in"); nonnull(mask, "trimul mask");
  nonnull(pair_out, "trimul pair_out"); nonnull(save, "trimul save");
  const int C = w.C, I = w.I, NC = 4 * I + C;
  const long M = (long)N * N;
  Carver cv(save);
  TriMulSave<Carver> sv(cv, N, C, I);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)M * I * 2 + 1024);
  bf16* xn = sv.xn;
  bf16* tn = ar.take_n<bf16>((size_t)M * I);
  {
    KTimed kt("trimul.ln_fwd", st);
    ln_fwd_f32(st, pair_in, M, C, 0, w.ln_g, w.ln_b, xn, sv.mean, sv.rstd, true, 0, nullptr,
               nullptr);
  }
  GemmArgs g1;
  g1.M = (int)M; g1.N = NC; g1.K = C;
  g1.A = xn; g1.a_sm = C; g1.a_sk = 1;
  g1.B = w.wcat_t; g1.b_sn = C; g1.b_sk = 1;
  gemm<128, 128>(st, g1,
                 EpiTrimulProj{sv.left, sv.right, sv.gout, w.bp, w.bg, w.bgl, mask, M, I, C},
                 "trimul.gemm_proj");
  contraction_fwd(st, outgoing, N, I, sv.left, sv.right, sv.T);
  {
    KTimed kt("trimul.ln_center", st);
    ln_fwd_cm(st, sv.T, M, I, w.cn_g, w.cn_b, tn, sv.cmean, sv.crstd, true);
  }
  GemmArgs g2;
  g2.M = (int)M; g2.N = C; g2.K = I;
  g2.A = tn; g2.a_sm = I; g2.a_sk = 1;
  g2.B = w.wo_t; g2.b_sn = I; g2.b_sk = 1;
  gemm<128, 128>(st, g2, EpiTrimulOut(pair_in, pair_out, w.bo, sv.gout, sv.osave, tbl, N, C),
                 "trimul.gemm_out");
}

void trimul_bwd(hipStream_t st, const TriMulW& w, bool outgoing, int N, const float* pair_in,
                const float* mask, const float* tbl, const void* save, const float* dout,
                float* din) {
  trimul_check(N);
  nonnull(pair_in, "trimul pair_in"); nonnull(mask, "trimul mask"); nonnull(save, "trimul save");
  nonnull(dout, "trimul dout"); nonnull(din, "trimul din");
  const int C = w.C, I = w.I, NC = 4 * I + C;
  const long M = (long)N * N;
  Carver cv(const_cast<void*>(save));
  TriMulSave<Carver> sv(cv, N, C, I);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  Sizer need;
  need.take<bf16>((size_t)M * NC);  // dcat
  need.take<float>((size_t)M * I);  // dTn
  need.take<bf16>((size_t)M * I);   // dT
  need.take<bf16>((size_t)M * I);   // dL
  need.take<bf16>((size_t)M * I);   // dR
  if (C != 128) need.take<float>((size_t)M * C);  // dxn (C = 128: fused LayerNorm backward)
  ar.reset(st, need.off);
  bf16* dcat = ar.take_n<bf16>((size_t)M * NC);
  float* dtn = ar.take_n<float>((size_t)M * I);
  bf16* dT = ar.take_n<bf16>((size_t)M * I);
  bf16* dL = ar.take_n<bf16>((size_t)M * I);
  bf16* dR = ar.take_n<bf16>((size_t)M * I);
  float* dxn = C != 128 ? ar.take_n<float>((size_t)M * C) : nullptr;

  // d(tn) = (tbl*dout*g_out) . Wo^T, the operand built as the GEMM loads it;
  // the loader also writes the gating_linear columns of dcat
  GemmArgs g1;
  g1.M = (int)M; g1.N = I; g1.K = C;
  g1.a_sm = C; g1.a_sk = 1;
  g1.B = w.wo; g1.b_sn = C; g1.b_sk = 1;
  gemm<128, 128>(st, g1, EpiStore<float>{dtn, I, 0, nullptr, I}, "trimul.gemm_dout",
                 ALoadTrimulOut{dout, tbl, sv.gout, sv.osave, dcat, C, NC, 4 * I, N});
  {
    KTimed kt("trimul.ln_center_bwd", st);
    ln_bwd_cm(st, dtn, sv.T, M, I, w.cn_g, sv.cmean, sv.crstd, dT);
  }
  {
    GemmArgs a, b;
    a.M = N; a.N = N; a.K = N; a.batch = I; a.a_sb = M; a.b_sb = M;
    b = a;
    if (outgoing) {
      // dL[i][k] = sum_j dT[i][j] R[j][k]
      a.A = dT; a.a_sm = N; a.a_sk = 1;
      a.B = sv.right; a.b_sn = 1; a.b_sk = N;
      // dR[j][k] = sum_i dT[i][j] L[i][k]
      b.A = dT; b.a_sm = 1; b.a_sk = N;
      b.B = sv.left; b.b_sn = 1; b.b_sk = N;
    } else {
      // dL[k][j] = sum_i R[k][i] dT[i][j]
      a.A = sv.right; a.a_sm = N; a.a_sk = 1;
      a.B = dT; a.b_sn = 1; a.b_sk = N;
      // dR[k][i] = sum_j L[k][j] dT[i][j]
      b.A = sv.left; b.a_sm = N; b.a_sk = 1;
      b.B = dT; b.b_sn = N; b.b_sk = 1;
    }
    contract<bf16>(st, a, dL, "trimul.contract_bwd");
    contract<bf16>(st, b, dR, "trimul.contract_bwd");
  }
  {
    GemmArgs g;
    g.M = (int)M; g.N = 4 * I; g.K = C;
    g.A = sv.xn; g.a_sm = C; g.a_sk = 1;
    g.B = w.wcat_t; g.b_sn = C; g.b_sk = 1;
    gemm<128, 128>(st, g, EpiTrimulProjBwd{dL, dR, w.bp, w.bg, mask, dcat, M, I, NC},
                   "trimul.proj_bwd");
  }
  GemmArgs g2;
  g2.M = (int)M; g2.N = C; g2.K = NC;
  g2.A = dcat; g2.a_sm = NC; g2.a_sk = 1;
  g2.B = w.wcat; g2.b_sn = NC; g2.b_sk = 1;
  if (C == 128) {
    // the input LayerNorm's backward and the residual add in the epilogue
    gemm<128, 128>(st, g2, EpiLnBwd<0>(pair_in, w.ln_g, sv.mean, sv.rstd, dout, din, M, 0),
                   "trimul.gemm_dx_ln");
    return;
  }
  gemm<128, 128>(st, g2, EpiStore<float>{dxn, C, 0, nullptr, C}, "trimul.gemm_dx");
  if (din != dout)
    BC2N_HIP(hipMemcpyAsync(din, dout, (size_t)M * C * 4, hipMemcpyDeviceToDevice, st));
  KTimed kt("trimul.ln_bwd", st);
  ln_bwd_f32(st, dxn, pair_in, M, C, 0, w.ln_g, sv.mean, sv.rstd, din, true, 0, nullptr, nullptr);
}

}  // namespace bc2n
