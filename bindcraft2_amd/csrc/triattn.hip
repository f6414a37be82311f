// Triangle attention (starting / ending node), forward and backward.
//
// Forward, in the module's frame (the transposed pair for the ending node):
//   LN (two-pass) + fused pair-bias projection  -> xn h16, bias[H][M] (log2 e)
//   GEMM xn . [Wq|Wk|Wv|Wg]  (q scaled by D^-1/2 log2 e, +gating_b)  -> qkvg
//   flash attention (mask per row/key, bias per head)               -> o, og, lse
//   GEMM og . Wo + bo, fused residual + shared dropout (+ transposed write)
// Backward replays nothing: the save-set holds LN stats, bias, qkvg, o, lse.
// It runs on the cotangent times the module's scale s (ct_scale): loaded so
// by the first GEMM, divided out by the LayerNorm backward that ends it.
//   GEMM (tbl * dout) . Wo^T, the scale applied as A is loaded (transposed
//        read for the ending node), epilogue through the gate -> dO, dG, Dsum
//   attention backward                    -> dq|dk|dv, d(bias)
//   GEMM dqkvg . [Wq|Wk|Wv|Wg]^T          -> d(xn)
//   LN backward (+ d(bias) . W2d^T) accumulated into din
// Reference: modules.py:675-734 (TriangleAttention), :313-400 (Attention),
// accel.py:13-24 (logit clip); native/triattn_body.cuh:647-1488 (TriAttn).
#include "gemm.h"
#include "lnproj.h"
#include "modules.h"
#include <cmath>
#include <mutex>
#include <string>

namespace bc2n {

namespace {

template <class A>
struct TriAttnSave {
  float *mean, *rstd, *lse;
  h16* bias;
  h16 *qkvg, *o;
  TriAttnSave(A& a, int N, int C, int H) {
    const size_t M = (size_t)N * N;
    mean = a.template take<float>(M);
    rstd = a.template take<float>(M);
    bias = a.template take<h16>((size_t)H * M);
    lse = a.template take<float>((size_t)H * M);
    qkvg = a.template take<h16>(M * 4 * C);
    o = a.template take<h16>(M * C);
  }
};

}  // namespace

TriAttnW triattn_weights(WeightStore& ws, const std::string& P) {
  TriAttnW w;
  const HostTensor& qw = ws.host(P + "attention/query_w");
  if (qw.shape.size() != 3) throw std::runtime_error("triattn: query_w must be [C,H,D]");
  w.C = qw.shape[0];
  w.H = qw.shape[1];
  w.D = qw.shape[2];
  const int C = w.C, HD = w.H * w.D;
  if (HD != C) throw std::runtime_error("triattn: H*D must equal C");
  w.ln_g = ws.f32(P + "query_norm/scale");
  w.ln_b = ws.f32(P + "query_norm/offset");
  w.w2d = ws.f32(P + "feat_2d_weights");
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
  w.wqkvg = ws.derived<h16>("triattn.wqkvg:" + P, [&] { return to_h16(cat()); });
  w.wqkvg_t = ws.derived<h16>("triattn.wqkvg_t:" + P, [&] {
    std::vector<float> c = cat();
    return transpose_h16(c.data(), C, 4 * HD);
  });
  if (C == 128 && w.H == 4 && (4 * HD) % 128 == 0) {
    w.wqkvg_frag = ws.derived<h16>("triattn.wqkvg_frag:" + P, [&] {
      const std::vector<float> c = cat();  // [C][4HD]
      return b_frags_k128(4 * HD, [&](int n, int k) { return c[(size_t)k * 4 * HD + n]; });
    });
  }
  w.bqkvg = ws.derived<float>("triattn.bqkvg:" + P, [&] {
    std::vector<float> b((size_t)4 * HD, 0.f);
    const HostTensor& gb = ws.host(P + "attention/gating_b");
    for (int j = 0; j < HD; ++j) b[3 * HD + j] = gb.data[j];
    return b;
  });
  const HostTensor& ow = ws.host(P + "attention/output_w");  // [H,D,C]
  w.wo = ws.derived<h16>("triattn.wo:" + P, [&] { return to_h16(ow.data); });
  w.wo_t = ws.derived<h16>("triattn.wo_t:" + P, [&] { return transpose_h16(ow.data.data(), HD, C); });
  w.bo = ws.f32(P + "attention/output_b");
  if (C == 128 && HD == 128) {
    w.wo_frag = ws.derived<h16>("triattn.wo_frag:" + P, [&] {
      return b_frags_k128(C, [&](int n, int k) { return ow.data[(size_t)k * C + n]; });
    });
  }
  return w;
}

size_t triattn_save_bytes(int N, int C, int H) {
  Sizer s;
  TriAttnSave<Sizer> plan(s, N, C, H);
  (void)plan;
  return s.off;
}

static void triattn_check(const TriAttnW& w, int N) {
  if (N <= 0 || N % 32 != 0) throw std::runtime_error("triattn: N must be a positive multiple of 32");
  if (w.D != 32 && w.D != 16) throw std::runtime_error("triattn: head width 16 or 32 only");
}


// The forward with its scratch (xn [M][C], og [M][HD], binary16) supplied.
static void triattn_fwd_with(hipStream_t st, const TriAttnW& w, bool per_column, int N,
                             const float* pair_in, const float* mask, const float* tbl,
                             float* pair_out, void* save, h16* xn, h16* og) {
  const int C = w.C, H = w.H, HD = w.H * w.D;
  const long M = (long)N * N;
  Carver cv(save);
  TriAttnSave<Carver> sv(cv, N, C, H);
  const float qscale = LOG2E / std::sqrt((float)w.D);
  if (w.wqkvg_frag) {
    lnproj::Args la{};
    la.M = M; la.nt = per_column ? N : 0; la.bn = N; la.nout = 4 * HD;
    la.x = pair_in; la.g = w.ln_g; la.b = w.ln_b; la.wb = w.w2d; la.bscale = LOG2E;
    // xn stays on chip: the backward's LayerNorm term reads pair_in, mean and rstd
    la.xn = nullptr; la.mean = sv.mean; la.rstd = sv.rstd; la.bias = sv.bias; la.W = w.wqkvg_frag;
    KTimed kt(BC2N_TN(C, "triattn.ln_qkvg"), st);
    if (H != 4) throw std::runtime_error("triattn: the fused LayerNorm-projection takes 4 bias heads");
    lnproj::launch<4, false>(st, la, EpiScaledCols(sv.qkvg, 4L * HD, w.bqkvg, qscale, HD));
  } else {
    {
      KTimed kt(BC2N_TN(C, "triattn.ln_fwd"), st);
      ln_fwd_f32(st, pair_in, M, C, per_column ? N : 0, w.ln_g, w.ln_b, xn, sv.mean, sv.rstd,
                 false, H, w.w2d, sv.bias, LOG2E);
    }
    GemmArgs g1;
    g1.M = (int)M; g1.N = 4 * HD; g1.K = C;
    g1.A = xn; g1.a_sm = C; g1.a_sk = 1;
    g1.B = w.wqkvg_t; g1.b_sn = C; g1.b_sk = 1;
    gemm<128, 128>(st, g1, EpiScaledCols(sv.qkvg, 4L * HD, w.bqkvg, qscale, HD),
                   BC2N_TN(C, "triattn.gemm_qkvg"));
  }

  AttnArgs a;
  a.R = N; a.H = H; a.N = N; a.D = w.D;
  a.qkvg = sv.qkvg; a.ld = 4L * HD;
  a.mask = mask;
  a.mask_sr = per_column ? 1 : N;
  a.mask_sk = per_column ? N : 1;
  a.bias = sv.bias;
  a.o = sv.o; a.og = og; a.ldo = HD;
  a.lse = sv.lse;
  attn_fwd(st, a);

  const EpiResidualRows res(pair_in, pair_out, w.bo, tbl, N, C, per_column);
  if (w.wo_frag) {
    lnproj::Args la{};
    la.M = M; la.nout = C; la.xn = og; la.W = w.wo_frag;
    KTimed kt(BC2N_TN(C, "triattn.gemm_out"), st);
    lnproj::launch_rows(st, la, res);
    return;
  }
  GemmArgs g2;
  g2.M = (int)M; g2.N = C; g2.K = HD;
  g2.A = og; g2.a_sm = HD; g2.a_sk = 1;
  g2.B = w.wo_t; g2.b_sn = HD; g2.b_sk = 1;
  gemm<128, 128>(st, g2, res, BC2N_TN(C, "triattn.gemm_out"));
}

void triattn_fwd(hipStream_t st, const TriAttnW& w, bool per_column, int N,
                 const float* pair_in, const float* mask, const float* tbl,
                 float* pair_out, void* save) {
  triattn_check(w, N);
  nonnull(pair_in, "triattn pair_in"); nonnull(mask, "triattn mask");
  nonnull(pair_out, "triattn pair_out"); nonnull(save, "triattn save");
  const int C = w.C, HD = w.H * w.D;
  const long M = (long)N * N;
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)M * C * 2 + (size_t)M * HD * 2 + 1024);
  h16* xn = ar.take_n<h16>((size_t)M * C);
  h16* og = ar.take_n<h16>((size_t)M * HD);
  triattn_fwd_with(st, w, per_column, N, pair_in, mask, tbl, pair_out, save, xn, og);
}

// ------------------------------------------------- the allocation-free variant
// Its scratch (xn and og of triattn_fwd_with) is this file-scope device
// array: one copy per GPU, allocated with the code object, held until the
// process ends.  Host code never passes `scratch` itself (its host-side name
// is a stand-in, not a device address): the first call on each device looks
// up the device address with hipGetSymbolAddress and keeps it per device.
// Calls on one GPU share the array, so calls that overlap on one GPU race.
static __device__ __align__(256) unsigned char scratch[TRIATTN_NOALLOC_SCRATCH_BYTES];

static void* scratch_ptr() {
  static std::mutex mu;
  static void* per_dev[64] = {};
  int dev = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) throw std::runtime_error("triattn noalloc: device index out of range");
  std::lock_guard<std::mutex> lk(mu);
  if (!per_dev[dev]) {
    void* p = nullptr;
    hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
    per_dev[dev] = p;
  }
  return per_dev[dev];
}

void triattn_fwd_noalloc(hipStream_t st, const TriAttnW& w, bool per_column, int N,
                         const float* pair_in, const float* mask, const float* tbl,
                         float* pair_out, void* save) {
  triattn_check(w, N);
  nonnull(pair_in, "triattn pair_in"); nonnull(mask, "triattn mask");
  nonnull(pair_out, "triattn pair_out"); nonnull(save, "triattn save");
  const int C = w.C, HD = w.H * w.D;
  const size_t M = (size_t)N * N;
  const size_t xn_bytes = (M * C * sizeof(h16) + 255) & ~size_t(255);
  if (xn_bytes + M * HD * sizeof(h16) > TRIATTN_NOALLOC_SCRATCH_BYTES)
    throw std::invalid_argument(
        "triattn_fwd_noalloc: N = " + std::to_string(N) + " needs " +
        std::to_string(xn_bytes + M * HD * sizeof(h16)) + " bytes of scratch; the static scratch holds " +
        std::to_string(TRIATTN_NOALLOC_SCRATCH_BYTES) + " (N <= 256 at C = 128)");
  char* base = static_cast<char*>(scratch_ptr());
  h16* xn = reinterpret_cast<h16*>(base);
  h16* og = reinterpret_cast<h16*>(base + xn_bytes);
  triattn_fwd_with(st, w, per_column, N, pair_in, mask, tbl, pair_out, save, xn, og);
}

void triattn_bwd(hipStream_t st, const TriAttnW& w, bool per_column, int N,
                 const float* pair_in, const float* mask, const float* tbl,
                 const void* save, const float* dout, float* din, const float* sc) {
  triattn_check(w, N);
  nonnull(pair_in, "triattn pair_in"); nonnull(mask, "triattn mask"); nonnull(save, "triattn save");
  nonnull(dout, "triattn dout"); nonnull(din, "triattn din");
  const int C = w.C, H = w.H, HD = w.H * w.D;
  const long M = (long)N * N;
  Carver cv(const_cast<void*>(save));
  TriAttnSave<Carver> sv(cv, N, C, H);
  AttnBwdArgs b;
  b.rows_per_chunk = attn_rows_per_chunk(N, N, H, w.D);
  const int nch = attn_bwd_nchunk(N, b.rows_per_chunk);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  sc = module_scale(st, sc, dout, M * C);
  Sizer need;
  need.take<h16>((size_t)M * HD);           // dO
  need.take<float>((size_t)H * M);           // Dsum
  need.take<h16>((size_t)M * 4 * HD);       // dqkvg
  need.take<float>((size_t)nch * H * M);     // dbias partials
  need.take<float>((size_t)H * M);           // dbias
  need.take<float>((size_t)M * C);           // dxn
  ar.reset(st, need.off);
  b.dO = ar.take_n<h16>((size_t)M * HD);
  b.nDsum = ar.take_n<float>((size_t)H * M);
  b.dqkvg = ar.take_n<h16>((size_t)M * 4 * HD);
  b.dbias_part = ar.take_n<float>((size_t)nch * H * M);
  b.dbias = ar.take_n<float>((size_t)H * M);
  float* dxn = ar.take_n<float>((size_t)M * C);

  // d(og) = (tbl * dout) . Wo^T, the dropout scale applied as A is loaded;
  // the epilogue continues through the gate (dO, dG, Dsum)
  GemmArgs g1;
  g1.M = (int)M; g1.N = HD; g1.K = C;
  g1.a_sm = C; g1.a_sk = 1;
  g1.B = w.wo; g1.b_sn = C; g1.b_sk = 1;
  EpiGateBwd eg;
  eg.qkvg = sv.qkvg; eg.ld = 4L * HD; eg.o = sv.o; eg.dO = b.dO; eg.dqkvg = b.dqkvg;
  eg.nDsum = b.nDsum; eg.HD = HD; eg.H = H; eg.D = w.D; eg.Ntok = N;
  // 64-row tiles: with N = K = 128 a 128-row grid leaves most workgroup
  // slots empty (392 workgroups at 224 tokens); the 128 x 128 B operand is
  // cheap to re-read
  gemm<64, 128>(st, g1, eg, BC2N_TN(C, "triattn.gemm_dout"), ALoadScaledRows{dout, tbl, N, C, per_column, sc});
  b.gate_done = true;

  AttnArgs& a = b.f;
  a.R = N; a.H = H; a.N = N; a.D = w.D;
  a.qkvg = sv.qkvg; a.ld = 4L * HD;
  a.mask = mask;
  a.mask_sr = per_column ? 1 : N;
  a.mask_sk = per_column ? N : 1;
  a.bias = sv.bias;
  a.o = sv.o; a.og = nullptr; a.ldo = HD;
  a.lse = sv.lse;
  b.scale = 1.f / std::sqrt((float)w.D);
  b.dbias_deferred = C == 128 && H == 4;  // the dX product's epilogue adds the partials
  attn_bwd(st, b);

  GemmArgs g2;
  g2.M = (int)M; g2.N = C; g2.K = 4 * HD;
  g2.A = b.dqkvg; g2.a_sm = 4L * HD; g2.a_sk = 1;
  g2.B = w.wqkvg; g2.b_sn = 4L * HD; g2.b_sk = 1;
  if (C == 128 && H == 4) {
    // the input LayerNorm's backward (with the pair-bias projection's term,
    // its per-chunk partials added in the epilogue: attn_bwd launched no
    // reduction) and the residual add in the epilogue
    const float* dbp = nch == 1 ? b.dbias : b.dbias_part;
    gemm<128, 128>(st, g2,
                   EpiLnBwd<4>(pair_in, w.ln_g, sv.mean, sv.rstd, dout, din, M, per_column ? N : 0,
                               dbp, w.w2d, sc + 1, nch),
                   BC2N_TN(C, "triattn.gemm_dx_ln"));
    return;
  }
  gemm<128, 128>(st, g2, EpiStore<float>{dxn, C, 0, nullptr, C}, BC2N_TN(C, "triattn.gemm_dx"));

  KTimed kt(BC2N_TN(C, "triattn.ln_bwd"), st);
  ln_bwd_f32(st, dxn, pair_in, M, C, per_column ? N : 0, w.ln_g, sv.mean, sv.rstd, din, true,
             H, b.dbias, w.w2d, dout, sc + 1);
}

}  // namespace bc2n
