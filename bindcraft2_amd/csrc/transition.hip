// Transition (pair and MSA), forward and backward.
//   LN -> GEMM (C -> F*C) + bias + relu (the hidden's ReLU mask kept, a bit
//      an element; the hidden itself is scratch)
//      -> GEMM (F*C -> C) + bias, fused residual (+ shared dropout table)
// Backward: dh = ((tbl*dout) . W2^T) * (h > 0), the dropout scale applied as
// the GEMM loads A; dxn = dh . W1^T; LN backward accumulated into din.
//
// The backward's ReLU mask is h > 0, and every pre-activation that rounding
// moves across zero flips a mask entry against the exact model: with bf16
// operands about 0.1% of them flip, 4-5% of d(hidden) in L2; the binary16
// operands flip 8x fewer.
// Reference: modules.py:252-305 (Transition); native/transition.cuh:313-675.
#include "gemm.h"
#include "modules.h"

namespace bc2n {

namespace {

template <class A>
struct TransSave {
  float *mean, *rstd;
  uint8_t* hbits;  // bit n of row m: relu(xn . W1 + b1)[m][n] > 0
  TransSave(A& a, long rows, int C, int F) {
    mean = a.template take<float>(rows);
    rstd = a.template take<float>(rows);
    hbits = a.template take<uint8_t>((size_t)rows * C * F / 8);
  }
};

}  // namespace

TransW transition_weights(WeightStore& ws, const std::string& P) {
  TransW w;
  const HostTensor& w1 = ws.host(P + "transition1/weights");  // [C, F*C]
  w.C = w1.shape[0];
  w.F = w1.shape[1] / w.C;
  const int C = w.C, H = w.C * w.F;
  w.ln_g = ws.f32(P + "input_layer_norm/scale");
  w.ln_b = ws.f32(P + "input_layer_norm/offset");
  w.b1 = ws.f32(P + "transition1/bias");
  w.b2 = ws.f32(P + "transition2/bias");
  const HostTensor& w2 = ws.host(P + "transition2/weights");  // [F*C, C]
  w.w1 = ws.derived<h16>("trans.w1:" + P, [&] { return to_h16(w1.data); });
  w.w1_t = ws.derived<h16>("trans.w1_t:" + P, [&] { return transpose_h16(w1.data.data(), C, H); });
  w.w2 = ws.derived<h16>("trans.w2:" + P, [&] { return to_h16(w2.data); });
  w.w2_t = ws.derived<h16>("trans.w2_t:" + P, [&] { return transpose_h16(w2.data.data(), H, C); });
  return w;
}

size_t transition_save_bytes(long rows, int C, int F) {
  Sizer s;
  TransSave<Sizer> plan(s, rows, C, F);
  (void)plan;
  return s.off;
}

void transition_fwd(hipStream_t st, const TransW& w, long rows, int nt, const float* act_in,
                    const float* tbl, float* act_out, void* save) {
  nonnull(act_in, "transition act"); nonnull(act_out, "transition out"); nonnull(save, "transition save");
  const int C = w.C, H = w.C * w.F;
  Carver cv(save);
  TransSave<Carver> sv(cv, rows, C, w.F);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  Sizer need;
  need.take<h16>((size_t)rows * C);
  need.take<h16>((size_t)rows * H);
  ar.reset(st, need.off);
  h16* xn = ar.take_n<h16>((size_t)rows * C);
  h16* hid = ar.take_n<h16>((size_t)rows * H);
  {
    KTimed kt(BC2N_TN(C, "trans.ln_fwd"), st);
    ln_fwd_f32(st, act_in, rows, C, 0, w.ln_g, w.ln_b, xn, sv.mean, sv.rstd, false, 0, nullptr,
               nullptr);
  }
  GemmArgs g1;
  g1.M = (int)rows; g1.N = H; g1.K = C;
  g1.A = xn; g1.a_sm = C; g1.a_sk = 1;
  g1.B = w.w1_t; g1.b_sn = C; g1.b_sk = 1;
  gemm<128, 128>(st, g1, EpiReluBits(hid, sv.hbits, H, w.b1), BC2N_TN(C, "trans.gemm1"));
  GemmArgs g2;
  g2.M = (int)rows; g2.N = C; g2.K = H;
  g2.A = hid; g2.a_sm = H; g2.a_sk = 1;
  g2.B = w.w2_t; g2.b_sn = H; g2.b_sk = 1;
  gemm<128, 128>(st, g2, EpiResidualRows(act_in, act_out, w.b2, tbl, nt, C, false), BC2N_TN(C, "trans.gemm2"));
}

void transition_bwd(hipStream_t st, const TransW& w, long rows, int nt, const float* act_in,
                    const float* tbl, const void* save, const float* dout, float* din,
                    const float* sc) {
  nonnull(act_in, "transition act"); nonnull(save, "transition save");
  nonnull(dout, "transition dout"); nonnull(din, "transition din");
  const int C = w.C, H = w.C * w.F;
  Carver cv(const_cast<void*>(save));
  TransSave<Carver> sv(cv, rows, C, w.F);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  sc = module_scale(st, sc, dout, rows * C);
  Sizer need;
  need.take<h16>((size_t)rows * H);
  need.take<float>((size_t)rows * C);
  ar.reset(st, need.off);
  h16* dh = ar.take_n<h16>((size_t)rows * H);
  float* dxn = ar.take_n<float>((size_t)rows * C);
  // dH = ((tbl * dout) . W2^T) * (H > 0), the dropout scale applied as A is loaded
  GemmArgs g1;
  g1.M = (int)rows; g1.N = H; g1.K = C;
  g1.a_sm = C; g1.a_sk = 1;
  g1.B = w.w2; g1.b_sn = C; g1.b_sk = 1;
  gemm<128, 128>(st, g1, EpiReluMaskBits<h16>(dh, sv.hbits, H), BC2N_TN(C, "trans.gemm_dh"),
                 ALoadScaledRows{dout, tbl, nt, C, false, sc});
  GemmArgs g2;
  g2.M = (int)rows; g2.N = C; g2.K = H;
  g2.A = dh; g2.a_sm = H; g2.a_sk = 1;
  g2.B = w.w1; g2.b_sn = H; g2.b_sk = 1;
  if (C == 128) {
    // the input LayerNorm's backward and the residual add in the epilogue
    gemm<128, 128>(st, g2,
                   EpiLnBwd<0>(act_in, w.ln_g, sv.mean, sv.rstd, dout, din, rows, 0, nullptr,
                               nullptr, sc + 1),
                   BC2N_TN(C, "trans.gemm_dx_ln"));
    return;
  }
  gemm<128, 128>(st, g2, EpiStore<float>{dxn, C, 0, nullptr, C}, BC2N_TN(C, "trans.gemm_dx"));
  KTimed kt(BC2N_TN(C, "trans.ln_bwd"), st);
  ln_bwd_f32(st, dxn, act_in, rows, C, 0, w.ln_g, sv.mean, sv.rstd, din, true, 0, nullptr, nullptr,
             dout, sc + 1);
}

}  // namespace bc2n
