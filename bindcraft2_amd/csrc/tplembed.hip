// Template embedding, forward and backward, for one template whose eight
// constant feature projections the caller has already summed into act_const
// (the reference's TemplateEmbeddingFwd/Bwd handlers, native/ffi.cu
// TeFwdImpl/TeBwdImpl, over modules_multimer.py:704-1005):
//
//   q   = LN(query)                    query_embedding_norm, C = 128, two-pass
//   act = act_const + q . W8 + b8      template_pair_embedding_8, 128 -> 64
//   act = template pair stack (act)    `depth` TemplateEmbeddingIterations
//   y   = LN(act)                      output_layer_norm, 64
//   out = relu(y) . Wo + bo            output_linear, 64 -> 128 (num_templates = 1)
//
// The backward replays nothing: the save-set holds the stack's own save-set,
// both LayerNorms' statistics, the stack output and y.  act_const is a
// constant of the design step and gets no gradient.
#include "evoformer.h"
#include "gemm.h"
#include "tplembed.h"

namespace bc2n {

namespace {

constexpr int CQ = 128;  // query / output channels
constexpr int CT = 64;   // template stack channels

template <class A>
struct TplEmbedSave {
  float *qmean, *qrstd, *omean, *orstd, *act2;
  h16* y;
  void* stack;
  TplEmbedSave(A& a, int N, size_t stack_bytes) {
    const size_t M = (size_t)N * N;
    qmean = a.template take<float>(M);
    qrstd = a.template take<float>(M);
    omean = a.template take<float>(M);
    orstd = a.template take<float>(M);
    act2 = a.template take<float>(M * CT);
    y = a.template take<h16>(M * CT);
    stack = a.template take<char>(stack_bytes);
  }
};

}  // namespace

TplEmbedW tplembed_weights(WeightStore& ws, int depth) {
  TplEmbedW w;
  const std::string P = "param/";
  const HostTensor& w8 = ws.host(P + "template_pair_embedding_8/weights");  // [128, 64]
  const HostTensor& wo = ws.host(P + "output_linear/weights");              // [64, 128]
  if (w8.shape != std::vector<int>{CQ, CT} || wo.shape != std::vector<int>{CT, CQ})
    throw std::runtime_error("tplembed: template_pair_embedding_8 must be [128,64], "
                             "output_linear [64,128]");
  w.qn_g = ws.f32(P + "query_embedding_norm/scale");
  w.qn_b = ws.f32(P + "query_embedding_norm/offset");
  w.b8 = ws.f32(P + "template_pair_embedding_8/bias");
  w.on_g = ws.f32(P + "output_layer_norm/scale");
  w.on_b = ws.f32(P + "output_layer_norm/offset");
  w.bo = ws.f32(P + "output_linear/bias");
  w.w8 = ws.derived<h16>("tplembed.w8", [&] { return to_h16(w8.data); });
  w.w8_t = ws.derived<h16>("tplembed.w8_t", [&] { return transpose_h16(w8.data.data(), CQ, CT); });
  w.wo = ws.derived<h16>("tplembed.wo", [&] { return to_h16(wo.data); });
  w.wo_t = ws.derived<h16>("tplembed.wo_t", [&] { return transpose_h16(wo.data.data(), CT, CQ); });
  w.stack = stack_weights(ws, depth, StackKind::TEMPLATE);
  w.depth = depth;
  return w;
}

size_t tplembed_save_bytes(const TplEmbedW& w, int N) {
  Sizer s;
  TplEmbedSave<Sizer> plan(s, N, stack_save_bytes(w.stack, N, 1, w.depth));
  (void)plan;
  return s.off;
}

static void tplembed_check(int N) {
  if (N <= 0 || N % 32 != 0) throw std::runtime_error("tplembed: N must be a positive multiple of 32");
}

void tplembed_fwd(hipStream_t st, const TplEmbedW& w, int N, const float* query,
                  const float* act_const, const float* pmask, const uint32_t* key,
                  const uint32_t* enabled, bool dropout, float* out, void* save) {
  tplembed_check(N);
  nonnull(query, "tplembed query"); nonnull(act_const, "tplembed act_const");
  nonnull(pmask, "tplembed pair_mask"); nonnull(out, "tplembed out"); nonnull(save, "tplembed save");
  if (out == query || out == act_const) throw std::runtime_error("tplembed: out must not alias an input");
  const long M = (long)N * N;
  Carver cv(save);
  TplEmbedSave<Carver> sv(cv, N, stack_save_bytes(w.stack, N, 1, w.depth));
  // The stack's input is staged in `out` (M x 64 of its M x 128 floats),
  // which is written only by the last GEMM: the stack's modules reuse the
  // scratch arena, so nothing the stack reads may live there.
  float* act = out;
  {
    Arena& ar = arena();
    std::lock_guard<std::recursive_mutex> lk(ar.lock());
    ar.reset(st, (size_t)M * CQ * 2 + 1024);
    h16* qn = ar.take_n<h16>((size_t)M * CQ);
    {
      KTimed kt("tplembed.ln_query", st);
      ln_fwd_f32(st, query, M, CQ, 0, w.qn_g, w.qn_b, qn, sv.qmean, sv.qrstd, false, 0, nullptr,
                 nullptr);
    }
    // act = act_const + qn . W8 + b8
    GemmArgs g;
    g.M = (int)M; g.N = CT; g.K = CQ;
    g.A = qn; g.a_sm = CQ; g.a_sk = 1;
    g.B = w.w8_t; g.b_sn = CQ; g.b_sk = 1;
    gemm<128, 128>(st, g, EpiResidualRows(act_const, act, w.b8, nullptr, N, CT, false),
                   "tplembed.gemm_proj");
  }
  stack_fwd(st, w.stack, N, 1, w.depth, act, nullptr, pmask, nullptr, key, enabled, dropout,
            sv.act2, nullptr, sv.stack);
  {
    KTimed kt("tplembed.ln_out", st);
    ln_fwd_f32(st, sv.act2, M, CT, 0, w.on_g, w.on_b, sv.y, sv.omean, sv.orstd, false, 0, nullptr,
               nullptr);
  }
  // out = relu(y) . Wo + bo
  GemmArgs g;
  g.M = (int)M; g.N = CQ; g.K = CT;
  g.a_sm = CT; g.a_sk = 1;
  g.B = w.wo_t; g.b_sn = CT; g.b_sk = 1;
  gemm<128, 128>(st, g, EpiStore<float>{out, CQ, 0, w.bo, CQ}, "tplembed.gemm_out",
                 ALoadRelu16{sv.y, CT});
}

void tplembed_bwd(hipStream_t st, const TplEmbedW& w, int N, const float* query,
                  const float* pmask, bool dropout, const void* save, const float* dout,
                  float* dquery) {
  tplembed_check(N);
  nonnull(query, "tplembed query"); nonnull(pmask, "tplembed pair_mask");
  nonnull(save, "tplembed save"); nonnull(dout, "tplembed dout"); nonnull(dquery, "tplembed dquery");
  if (dquery == dout || dquery == query) throw std::runtime_error("tplembed: dquery must not alias an input");
  const long M = (long)N * N;
  Carver cv(const_cast<void*>(save));
  TplEmbedSave<Carver> sv(cv, N, stack_save_bytes(w.stack, N, 1, w.depth));
  // The stack's cotangent is staged in `dquery` (M x 64 of its M x 128
  // floats), written only by the last LayerNorm backward, for the same
  // reason as the forward's staging.
  float* dact = dquery;
  {
    Arena& ar = arena();
    std::lock_guard<std::recursive_mutex> lk(ar.lock());
    ar.reset(st, (size_t)M * CT * 4 + 1024);
    float* dy = ar.take_n<float>((size_t)M * CT);
    // d(y) = (s dout . Wo^T) * (y > 0), s the cotangent scale of dout
    float* sc = ct_scale_slot(3);
    ct_scale(st, dout, M * CQ, sc);
    GemmArgs g;
    g.M = (int)M; g.N = CT; g.K = CQ;
    g.a_sm = CQ; g.a_sk = 1;
    g.B = w.wo; g.b_sn = CQ; g.b_sk = 1;
    gemm<128, 128>(st, g, EpiReluMask<float>(dy, sv.y, CT), "tplembed.gemm_dout",
                   ALoadScaledRows{dout, nullptr, N, CQ, false, sc});
    KTimed kt("tplembed.ln_out_bwd", st);
    ln_bwd_f32(st, dy, sv.act2, M, CT, 0, w.on_g, sv.omean, sv.orstd, dact, false, 0, nullptr,
               nullptr, nullptr, sc + 1);
  }
  stack_bwd(st, w.stack, N, 1, w.depth, pmask, nullptr, dropout, sv.stack, dact, nullptr, dact,
            nullptr);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)M * CQ * 4 + 1024);
  float* dq = ar.take_n<float>((size_t)M * CQ);
  // d(q) = d(act) . W8^T (scaled by the cotangent scale of d(act)), then the
  // query LayerNorm's backward, which divides it out
  float* sc = ct_scale_slot(3);
  ct_scale(st, dact, M * CT, sc);
  GemmArgs g;
  g.M = (int)M; g.N = CQ; g.K = CT;
  g.a_sm = CT; g.a_sk = 1;
  g.B = w.w8; g.b_sn = CT; g.b_sk = 1;
  gemm<128, 128>(st, g, EpiStore<float>{dq, CQ, 0, nullptr, CQ}, "tplembed.gemm_dq",
                 ALoadScaledRows{dact, nullptr, N, CT, false, sc});
  KTimed kt("tplembed.ln_query_bwd", st);
  ln_bwd_f32(st, dq, query, M, CQ, 0, w.qn_g, sv.qmean, sv.qrstd, dquery, false, 0, nullptr,
             nullptr, nullptr, sc + 1);
}

}  // namespace bc2n
