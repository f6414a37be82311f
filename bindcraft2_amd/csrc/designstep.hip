// The trunk of one design step in one call, forward and backward (the
// reference's fused NativeDesignStep, native/ffi.cu:1691-2178 over
// native/design_step.cuh, restricted to the differentiable trunk: features
// in, structure-module outputs out, losses left to the caller; `recycles`
// forward-only passes ahead of the differentiated one):
//
//   msa0, pair0 = embedder(target_feat, msa_feat, ids)         (embed.hip)
//   pair0 += recycle terms, msa0[0] += recycle term            (previous pass, or constants)
//   pair1 = pair0 + template_embedding(pair0, act_const)        (tplembed.hip; skipped without act_const)
//   pair2 = extra-MSA stack, pair only (its MSA mask is zero)   (evoformer.hip)
//   msa3, pair3 = main stack (msa0, pair2)
//   single = msa3[0] . W + b                                    single_activations, f32
//   outputs = structure module + heads (single, pair3)          (heads.hip)
//
// (modules_multimer.py:441-700 and the structure module / heads of
// AlphaFoldIteration.)  The backward runs the chain in reverse to
// d(target_feat) and d(msa_feat).  Every intermediate lives in the caller's
// save buffer, so the two calls share nothing else.
#include "designstep.h"

#include "gemm_f32.h"

namespace bc2n {

namespace {

constexpr int CM = 256, CZ = 128, CS = 384;

// Every save buffer opens with a 256-byte header that the forward writes:
// hdr[0] a magic word naming the layout, hdr[1] the optional parts it
// computed.  The backward refuses a buffer whose parts differ from the ones
// it is asked to differentiate, instead of reading memory never written.
constexpr uint32_t DS_MAGIC = 0xBC2D0001u, SEQ_MAGIC = 0xBC2D0002u;
constexpr uint32_t HAS_TEMPLATE = 1u, HAS_CONFIDENCE = 2u, HAS_ATOM37 = 4u, HAS_ROW = 8u;

__global__ void hdr_set_kernel(uint32_t* h, uint32_t magic, uint32_t flags) {
  if (threadIdx.x == 0) {
    h[0] = magic;
    h[1] = flags;
  }
}

void hdr_set(hipStream_t st, uint32_t* h, uint32_t magic, uint32_t flags) {
  hipLaunchKernelGGL(hdr_set_kernel, dim3(1), dim3(64), 0, st, h, magic, flags);
}

// The header's flags, after the forward that wrote them has finished (this
// waits for the stream).  Under graph capture nothing can be read back, so
// the check is skipped there and -1 returned.
long hdr_flags(hipStream_t st, const uint32_t* h, uint32_t magic, const char* what) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  BC2N_HIP(hipStreamIsCapturing(st, &cs));
  if (cs != hipStreamCaptureStatusNone) return -1;
  uint32_t v[2] = {0, 0};
  BC2N_HIP(hipMemcpyAsync(v, h, sizeof v, hipMemcpyDeviceToHost, st));
  BC2N_HIP(hipStreamSynchronize(st));
  if (v[0] != magic)
    throw std::invalid_argument(std::string(what) +
                                ": the save buffer was not written by this step's forward");
  return v[1];
}

void hdr_require(long flags, uint32_t bit, bool want, const char* what) {
  if (flags < 0 || ((flags & bit) != 0) == want) return;
  throw std::invalid_argument(std::string(what) + (want ? ": the backward asks for " : ": the backward omits ") +
                              (bit == HAS_TEMPLATE    ? "the template embedding"
                               : bit == HAS_ATOM37 ? "the atom37 positions"
                               : bit == HAS_ROW    ? "the template's MSA row"
                                                   : "the confidence metrics") +
                              (want ? ", which the forward did not compute" : ", which the forward computed"));
}

template <class A>
struct DsSave {
  uint32_t* hdr;
  void *tpl, *extra, *main, *sh;
  float *pmask, *mmask, *msa0, *pair0, *tplo, *pair1, *pair2, *msa3, *pair3, *single;
  float *dpair, *dq, *dmsa, *dsingle;
  DsSave(A& c, const DesignStepW& w, int N, int S) {
    const size_t M = (size_t)N * N;
    hdr = c.template take<uint32_t>(64);
    tpl = c.template take<char>(tplembed_save_bytes(w.tpl, N));
    extra = c.template take<char>(stack_save_bytes(w.extra, N, 1, w.d_extra));
    main = c.template take<char>(stack_save_bytes(w.main, N, S, w.d_main));
    sh = c.template take<char>(structheads_save_bytes(N, w.d_fold));
    pmask = c.template take<float>(M);
    mmask = c.template take<float>((size_t)S * N);
    msa0 = c.template take<float>((size_t)S * N * CM);
    pair0 = c.template take<float>(M * CZ);
    tplo = c.template take<float>(M * CZ);
    pair1 = c.template take<float>(M * CZ);
    pair2 = c.template take<float>(M * CZ);
    msa3 = c.template take<float>((size_t)S * N * CM);
    pair3 = c.template take<float>(M * CZ);
    single = c.template take<float>((size_t)N * CS);
    dpair = c.template take<float>(M * CZ);
    dq = c.template take<float>(M * CZ);
    dmsa = c.template take<float>((size_t)S * N * CM);
    dsingle = c.template take<float>((size_t)N * CS);
    rpb = c.template take<float>((size_t)N * 4);
    rpair = c.template take<float>(M * CZ);
    rmsa0 = c.template take<float>((size_t)N * CM);
    rpos = c.template take<float>((size_t)N * 37 * 3);
    rposm = c.template take<float>((size_t)N * 37);
  }
  float *rpb, *rpair, *rmsa0;  // the previous pass's pseudo-beta [N][3(+1)], pair, msa[0]
  float *rpos, *rposm;         // and its atom37 positions (and their mask)
};

// pmask[i][j] = m[i] m[j]; mmask[s][n] = m[n]
__global__ void masks_kernel(const float* __restrict__ m, int N, int S, float* __restrict__ pm,
                             float* __restrict__ mm) {
  const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < (long)N * N) pm[e] = m[e / N] * m[e % N];
  if (e < (long)S * N) mm[e] = m[e % N];
}

// y = a + b elementwise (y may alias a or b)
__global__ void add2_kernel(const float* a, const float* b, long n, float* y) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] = a[i] + b[i];
}
void add2(hipStream_t st, const float* a, const float* b, long n, float* y) {
  hipLaunchKernelGGL(add2_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, b, n, y);
}

// ------------------------------------------------------------- recycling
// The embedder's three recycle terms (modules_multimer.py:487-507):
//   pair  += prev_pos_linear(dgram(pseudo_beta(prev atoms))) + LN_pair(prev pair)
//   msa[0] += LN_msa(prev msa[0])
// The distogram (modules.py:1215-1238) is one-hot in 15 bins between the
// squared lower breaks 3.25 + 1.25 b (b = 0..14; exact in f32), strict on
// both sides, the last bin open to 1e8: at most one bin is set, so the
// Linear is the bias plus one weight row.  LayerNorms: eps 1e-5, two-pass.
constexpr int RBINS = 15;

// First pass: the previous state is zero, so the terms are constants -- the
// Linear's bias (a zero distance lies in no bin) and the two norms' offsets
// (a LayerNorm of a zero vector is its offset).
__global__ void recycle_first_kernel(float* __restrict__ pair, float* __restrict__ msa0, long M,
                                     int N, const float* __restrict__ bpp,
                                     const float* __restrict__ o_pair,
                                     const float* __restrict__ o_msa) {
  const long e = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e < M * CZ) {
    const int c = (int)(e % CZ);
    pair[e] += bpp[c] + o_pair[c];
  } else if (e < M * CZ + (long)N * CM) {
    const long f = e - M * CZ;
    msa0[f] += o_msa[f % CM];
  }
}

// One wave per pair row (i, j): 2 channels per lane.
__global__ __launch_bounds__(256) void recycle_pair_kernel(
    float* __restrict__ pair, const float* __restrict__ prev_pair, const float* __restrict__ pb,
    int N, const float* __restrict__ wpp, const float* __restrict__ bpp,
    const float* __restrict__ s_pair, const float* __restrict__ o_pair) {
  const long m = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (m >= (long)N * N) return;
  const int i = (int)(m / N), j = (int)(m % N);
  float d2 = 0.f;
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float d = pb[i * 4 + c] - pb[j * 4 + c];
    d2 += d * d;
  }
  int bin = -1;
#pragma unroll
  for (int b = 0; b < RBINS; ++b) {
    const float lo = 3.25f + 1.25f * (float)b;
    const float hi = 3.25f + 1.25f * (float)(b + 1);
    if (d2 > lo * lo && (b == RBINS - 1 ? d2 < 1e8f : d2 < hi * hi)) bin = b;
  }
  const float* x = prev_pair + m * CZ;
  const float x0 = x[lane], x1 = x[lane + 64];
  float sum = x0 + x1;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  const float mean = sum * (1.f / CZ);
  float var = (x0 - mean) * (x0 - mean) + (x1 - mean) * (x1 - mean);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) var += __shfl_xor(var, o, 64);
  const float rstd = rsqrtf(var * (1.f / CZ) + 1e-5f);
  float* y = pair + m * CZ;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int c = lane + 64 * h;
    const float xv = h ? x1 : x0;
    const float lin = bpp[c] + (bin >= 0 ? wpp[bin * CZ + c] : 0.f);
    y[c] += lin + (xv - mean) * rstd * s_pair[c] + o_pair[c];
  }
}

// One wave per residue: msa[0][i] += LN_msa(prev msa[0][i]), 4 channels per lane.
__global__ __launch_bounds__(256) void recycle_msa_kernel(float* __restrict__ msa0,
                                                          const float* __restrict__ prev, int N,
                                                          const float* __restrict__ s_msa,
                                                          const float* __restrict__ o_msa) {
  const int i = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (i >= N) return;
  const float* x = prev + (long)i * CM;
  float v[4], sum = 0.f;
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    v[h] = x[lane + 64 * h];
    sum += v[h];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) sum += __shfl_xor(sum, o, 64);
  const float mean = sum * (1.f / CM);
  float var = 0.f;
#pragma unroll
  for (int h = 0; h < 4; ++h) var += (v[h] - mean) * (v[h] - mean);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) var += __shfl_xor(var, o, 64);
  const float rstd = rsqrtf(var * (1.f / CM) + 1e-5f);
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const int c = lane + 64 * h;
    msa0[(long)i * CM + c] += (v[h] - mean) * rstd * s_msa[c] + o_msa[c];
  }
}

// pseudo_beta_fn (modules.py:1249-1264): CB, or CA for glycine (aatype 7),
// read from atom14 (CA slot 1, CB slot 4); stored with stride 4.
__global__ void pseudo_beta_kernel(const float* __restrict__ aatype,
                                   const float* __restrict__ atom14, int N,
                                   float* __restrict__ pb) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const int slot = (int)aatype[i] == 7 ? 1 : 4;
#pragma unroll
  for (int c = 0; c < 3; ++c) pb[i * 4 + c] = atom14[((long)i * 14 + slot) * 3 + c];
  pb[i * 4 + 3] = 0.f;
}

void ds_check(const DesignStepW& w, int N, int S) {
  // the composed step is parity-tested to L = 224 (its parts to 1024)
  if (N <= 0 || N % 32 != 0 || N > 768)
    throw std::runtime_error("design step: N must be a positive multiple of 32, at most 768");
  if (S <= 0) throw std::runtime_error("design step: S must be positive");
  if (w.d_tpl <= 0 || w.d_extra <= 0 || w.d_main <= 0 || w.d_fold <= 0)
    throw std::runtime_error("design step: depths must be positive");
}

}  // namespace

void recycle_terms(hipStream_t st, const RecycleW& r, int N, const float* aatype,
                   const float* prev_atom14, const float* prev_pair, const float* prev_msa0,
                   float* pair, float* msa0) {
  if (N <= 0) throw std::invalid_argument("recycle terms: N must be positive");
  nonnull(pair, "recycle terms pair"); nonnull(msa0, "recycle terms msa0");
  const long M = (long)N * N;
  if (!prev_atom14) {
    const long n = M * CZ + (long)N * CM;
    hipLaunchKernelGGL(recycle_first_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       pair, msa0, M, N, r.bpp, r.o_pair, r.o_msa);
    return;
  }
  nonnull(aatype, "recycle terms aatype"); nonnull(prev_pair, "recycle terms prev_pair");
  nonnull(prev_msa0, "recycle terms prev_msa0");
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)N * 16 + 256);
  float* pb = ar.take_n<float>((size_t)N * 4);
  hipLaunchKernelGGL(pseudo_beta_kernel, dim3((unsigned)((N + 127) / 128)), dim3(128), 0, st,
                     aatype, prev_atom14, N, pb);
  hipLaunchKernelGGL(recycle_pair_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, st, pair,
                     prev_pair, pb, N, r.wpp, r.bpp, r.s_pair, r.o_pair);
  hipLaunchKernelGGL(recycle_msa_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st, msa0,
                     prev_msa0, N, r.s_msa, r.o_msa);
}

size_t design_step_save_bytes(const DesignStepW& w, int N, int S) {
  Sizer s;
  DsSave<Sizer> plan(s, w, N, S);
  (void)plan;
  return s.off;
}

__global__ void atom37_kernel(const float* __restrict__ atom14, const float* __restrict__ aatype,
                              const float* __restrict__ seq_mask,
                              const float* __restrict__ a37_14,
                              const float* __restrict__ a37_mask, int N,
                              float* __restrict__ atom37, float* __restrict__ mask37);

void design_step_fwd(hipStream_t st, const DesignStepW& w, int N, int S, const float* tf,
                     const float* mf, const float* ri, const float* ai, const float* ei,
                     const float* si, const int32_t* offset, const float* seq_mask,
                     const float* act_const, const float* aatype, const uint32_t* seeds,
                     bool dropout, int recycles, float* atom14, float* dgram, float* pae,
                     float* plddt, float* expres, void* save, const float* row,
                     const float* row_mask, const float* init_pos37) {
  const int SM = S + (row ? 1 : 0);  // the main stack's msa rows
  ds_check(w, N, SM);
  nonnull(seq_mask, "design step seq_mask"); nonnull(save, "design step save");
  nonnull(aatype, "design step aatype");
  if (row) nonnull(row_mask, "design step row mask");
  if (dropout) nonnull(seeds, "design step seeds");
  if (recycles < 0 || recycles > 64) throw std::invalid_argument("design step: recycles must be in [0, 64]");
  if (init_pos37 && recycles > 0 && (!w.a37_14 || !w.a37_mask))
    throw std::invalid_argument("design step: initial atom positions with recycling need "
                                "const/atom37_to_atom14 and const/atom37_mask in the structure "
                                "module's directory");
  Carver cv(save);
  DsSave<Carver> sv(cv, w, N, SM);
  const long M = (long)N * N;
  hdr_set(st, sv.hdr, DS_MAGIC, (act_const ? HAS_TEMPLATE : 0u) | (row ? HAS_ROW : 0u));
  {
    const long n = std::max(M, (long)SM * N);
    hipLaunchKernelGGL(masks_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, seq_mask,
                       N, SM, sv.pmask, sv.mmask);
  }
  if (row) {
    // the constant row after the embedder's S rows (embed_fwd writes those only)
    BC2N_HIP(hipMemcpyAsync(sv.msa0 + (size_t)S * N * CM, row, (size_t)N * CM * 4,
                            hipMemcpyDeviceToDevice, st));
    BC2N_HIP(hipMemcpyAsync(sv.mmask + (size_t)S * N, row_mask, (size_t)N * 4,
                            hipMemcpyDeviceToDevice, st));
  }
  for (int pass = 0; pass <= recycles; ++pass) {
    // forward-only passes keep no save-sets: their stacks run detached
    const bool last = pass == recycles;
    const uint32_t* sp = dropout ? seeds + 12 * pass : nullptr;
    auto key = [&](int i) { return sp ? sp + 3 * i : nullptr; };
    auto enabled = [&](int i) { return sp ? sp + 3 * i + 2 : nullptr; };
    embed_fwd(st, w.emb, N, S, tf, mf, ri, ai, ei, si, offset, sv.msa0, sv.pair0);
    {
      KTimed kt("design.recycle_terms", st);
      if (pass == 0) {
        const long n = M * CZ + (long)N * CM;
        hipLaunchKernelGGL(recycle_first_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           st, sv.pair0, sv.msa0, M, N, w.rec.bpp, w.rec.o_pair, w.rec.o_msa);
      } else {
        hipLaunchKernelGGL(recycle_pair_kernel, dim3((unsigned)((M + 3) / 4)), dim3(256), 0, st,
                           sv.pair0, sv.rpair, sv.rpb, N, w.rec.wpp, w.rec.bpp, w.rec.s_pair,
                           w.rec.o_pair);
        hipLaunchKernelGGL(recycle_msa_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, st,
                           sv.msa0, sv.rmsa0, N, w.rec.s_msa, w.rec.o_msa);
      }
    }
    const float* pair = sv.pair0;
    if (act_const) {
      tplembed_fwd(st, w.tpl, N, sv.pair0, act_const, sv.pmask, key(0), enabled(0), dropout,
                   sv.tplo, sv.tpl);
      add2(st, sv.pair0, sv.tplo, M * CZ, sv.pair1);
      pair = sv.pair1;
    }
    stack_fwd(st, w.extra, N, 1, w.d_extra, pair, nullptr, sv.pmask, nullptr, key(1), enabled(1),
              dropout, sv.pair2, nullptr, sv.extra, !last);
    stack_fwd(st, w.main, N, SM, w.d_main, sv.pair2, sv.msa0, sv.pmask, sv.mmask, key(2),
              enabled(2), dropout, sv.pair3, sv.msa3, sv.main, !last);
    GemmF32 g = gemm_rows(N, CS, CM, sv.msa3, w.wsa, sv.single);
    g.bias = w.bsa;
    gemm_f32(st, g, "design.gemm_single");
    // the first pass starts from the given atoms, later ones from the
    // previous pass's (native/design_step.cuh:1112-1114)
    const float* init = init_pos37 ? (pass == 0 ? init_pos37 : sv.rpos) : nullptr;
    structheads_fwd(st, w.sh, N, w.d_fold, sv.single, sv.pair3, seq_mask, aatype, key(3),
                    enabled(3), dropout, atom14, dgram, pae, plddt, expres, sv.sh, init);
    if (!last) {
      // what the next pass's recycle terms read (under stop_gradient)
      hipLaunchKernelGGL(pseudo_beta_kernel, dim3((unsigned)((N + 127) / 128)), dim3(128), 0, st,
                         aatype, atom14, N, sv.rpb);
      if (init_pos37)
        hipLaunchKernelGGL(atom37_kernel, dim3((unsigned)((N * 37 + 255) / 256)), dim3(256), 0, st,
                           atom14, aatype, seq_mask, w.a37_14, w.a37_mask, N, sv.rpos, sv.rposm);
      BC2N_HIP(hipMemcpyAsync(sv.rpair, sv.pair3, (size_t)M * CZ * 4, hipMemcpyDeviceToDevice, st));
      BC2N_HIP(hipMemcpyAsync(sv.rmsa0, sv.msa3, (size_t)N * CM * 4, hipMemcpyDeviceToDevice, st));
    }
  }
}

void design_step_bwd(hipStream_t st, const DesignStepW& w, int N, int S, const float* tf,
                     const float* seq_mask, bool with_template, const float* aatype,
                     bool dropout, void* save, const float* datom, const float* ddgram,
                     const float* dpae, const float* dplddt, const float* dexpres, float* dtf,
                     float* dmf, bool row) {
  const int SM = S + (row ? 1 : 0);
  ds_check(w, N, SM);
  nonnull(seq_mask, "design step seq_mask"); nonnull(save, "design step save");
  Carver cv(save);
  DsSave<Carver> sv(cv, w, N, SM);
  const long M = (long)N * N;
  const long ds_flags = hdr_flags(st, sv.hdr, DS_MAGIC, "design step");
  hdr_require(ds_flags, HAS_TEMPLATE, with_template, "design step");
  hdr_require(ds_flags, HAS_ROW, row, "design step");
  structheads_bwd(st, w.sh, N, w.d_fold, sv.single, sv.pair3, seq_mask, aatype, dropout, sv.sh,
                  datom, ddgram, dpae, dplddt, dexpres, sv.dsingle, sv.dpair);
  // d msa3: row 0 from the single projection, the other rows zero
  zero_f32(st, sv.dmsa, (long)SM * N * CM);
  GemmF32 g = gemm_rows(N, CM, CS, sv.dsingle, w.wsa, sv.dmsa, true);
  gemm_f32(st, g, "design.gemm_single_dx");
  // the stacks accumulate in place: d pair3 -> d pair2 -> d pair1, d msa3 -> d msa0
  stack_bwd(st, w.main, N, SM, w.d_main, sv.pmask, sv.mmask, dropout, sv.main, sv.dpair, sv.dmsa,
            sv.dpair, sv.dmsa);
  stack_bwd(st, w.extra, N, 1, w.d_extra, sv.pmask, nullptr, dropout, sv.extra, sv.dpair, nullptr,
            sv.dpair, nullptr);
  if (with_template) {
    // pair1 = pair0 + template(pair0): d pair0 = d pair1 + d query
    tplembed_bwd(st, w.tpl, N, sv.pair0, sv.pmask, dropout, sv.tpl, sv.dpair, sv.dq);
    add2(st, sv.dpair, sv.dq, M * CZ, sv.dpair);
  }
  embed_bwd(st, w.emb, N, S, sv.dmsa, sv.dpair, tf, dtf, dmf);
}

namespace {

// The sequence front's buffers, carved ahead of the step's own save-set.
template <class A>
struct SeqExtra {
  uint32_t* hdr;
  float *feat, *prof, *tf, *mf, *aatype, *dtf, *dmf, *dfeat, *dprof;
  SeqExtra(A& c, int N) {
    hdr = c.template take<uint32_t>(64);
    feat = c.template take<float>((size_t)N * SEQ_A);
    prof = c.template take<float>((size_t)N * SEQ_A);
    tf = c.template take<float>((size_t)N * (SEQ_A + 1));
    mf = c.template take<float>((size_t)N * 49);
    aatype = c.template take<float>(N);
    dtf = c.template take<float>((size_t)N * (SEQ_A + 1));
    dmf = c.template take<float>((size_t)N * 49);
    dfeat = c.template take<float>((size_t)N * SEQ_A);
    dprof = c.template take<float>((size_t)N * SEQ_A);
    conf = c.template take<char>(confidence_save_bytes(N));
    dl = c.template take<float>((size_t)N * CONF_LBINS);
    dp = c.template take<float>((size_t)N * N * CONF_PBINS);
    de = c.template take<float>((size_t)N * CONF_EXPRES);
    ll = c.template take<float>((size_t)N * CONF_LBINS);
    pl = c.template take<float>((size_t)N * N * CONF_PBINS);
    el = c.template take<float>((size_t)N * CONF_EXPRES);
    kab = c.template take<float>(64);
    d14 = c.template take<float>((size_t)N * 14 * 3);
    row = c.template take<float>((size_t)N * CM);
    rmask = c.template take<float>(N);
    smask = c.template take<float>(N);
    fl = c.template take<uint8_t>(N);
    dd = c.template take<float>((size_t)N * N * CONF_PBINS);
    cc = c.template take<float>((size_t)3 * N + (size_t)N * N);
    off = c.template take<int32_t>((size_t)N * N);
  }
  int32_t* off;  // the cyclic sequence offsets [N][N]
  float *row, *rmask;  // the template's MSA row [N][256] and its mask
  // with a runtime length: seq_mask and flags with the padding rows zeroed,
  // and the padding-masked distogram and confidence cotangents
  float* smask;
  uint8_t* fl;
  float *dd, *cc;
  float* kab;  // the superposition: R [3][3], centres of the prediction and template
  float* d14;  // the atom14 cotangent with the atom37 one folded in
  char* conf;
  float *dl, *dp, *de;  // head-logit cotangents with the confidence terms added
  float *ll, *pl, *el;  // the head logits the confidence metrics were computed from
};

// y += a + b, either may be null (zero)
__global__ void add_opt_kernel(const float* a, const float* b, long n, float* y) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) y[i] += (a ? a[i] : 0.f) + (b ? b[i] : 0.f);  // y already holds one term
}
void add_into(hipStream_t st, const float* a, const float* b, long n, float* y) {
  hipLaunchKernelGGL(add_opt_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a, b, n, y);
}

}  // namespace

// ------------------------------------------------------ atom37 + alignment
constexpr int A37 = 37, CA37 = 1;
constexpr uint8_t F_DESIGN = 1u, F_TEMPLATE = 2u, F_CYCLIC = 64u;  // bindcraft/protein.py:42-51

// atom37[i][a] = atom14[i][a37_14[aat][a]] * ex, ex = a37_mask[aat][a] * seq_mask[i]
__global__ void atom37_kernel(const float* __restrict__ atom14, const float* __restrict__ aatype,
                              const float* __restrict__ seq_mask,
                              const float* __restrict__ a37_14,
                              const float* __restrict__ a37_mask, int N,
                              float* __restrict__ atom37, float* __restrict__ mask37) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= N * A37) return;
  const int i = e / A37, a = e % A37;
  const int aat = min(max((int)aatype[i], 0), 20);
  const float ex = a37_mask[aat * A37 + a] * (seq_mask[i] != 0.f ? 1.f : 0.f);
  const int j = (int)a37_14[aat * A37 + a];
#pragma unroll
  for (int c = 0; c < 3; ++c) atom37[(long)e * 3 + c] = atom14[((long)i * 14 + j) * 3 + c] * ex;
  mask37[e] = ex;
}

// The 3x3 SVD by one-sided Jacobi (Hestenes; Golub & Van Loan 8.6.3): rotate
// column pairs of A until orthogonal, accumulating the rotations in V; the
// column norms are the singular values and the normalised columns U.
__device__ void svd3(const double (&H)[3][3], double (&U)[3][3], double (&S)[3], double (&V)[3][3]) {
  double A[3][3];
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) {
      A[i][j] = H[i][j];
      V[i][j] = i == j ? 1.0 : 0.0;
    }
  for (int sweep = 0; sweep < 30; ++sweep) {
    double off = 0.0;
    for (int p = 0; p < 2; ++p)
      for (int q = p + 1; q < 3; ++q) {
        double al = 0, be = 0, ga = 0;
        for (int i = 0; i < 3; ++i) {
          al += A[i][p] * A[i][p];
          be += A[i][q] * A[i][q];
          ga += A[i][p] * A[i][q];
        }
        if (ga == 0.0 || fabs(ga) <= 1e-15 * sqrt(al * be)) continue;
        off = fmax(off, fabs(ga) / sqrt(al * be));
        const double z = (be - al) / (2.0 * ga);
        const double t = (z >= 0 ? 1.0 : -1.0) / (fabs(z) + sqrt(1.0 + z * z));
        const double c = 1.0 / sqrt(1.0 + t * t), s = c * t;
        for (int i = 0; i < 3; ++i) {
          const double ap = A[i][p], aq = A[i][q];
          A[i][p] = c * ap - s * aq;
          A[i][q] = s * ap + c * aq;
          const double vp = V[i][p], vq = V[i][q];
          V[i][p] = c * vp - s * vq;
          V[i][q] = s * vp + c * vq;
        }
      }
    if (off < 1e-15) break;
  }
  for (int j = 0; j < 3; ++j) {
    double n = 0;
    for (int i = 0; i < 3; ++i) n += A[i][j] * A[i][j];
    S[j] = sqrt(n);
  }
  // descending singular values (the determinant fix acts on the smallest)
  for (int a = 0; a < 2; ++a)
    for (int b = a + 1; b < 3; ++b)
      if (S[b] > S[a]) {
        double t = S[a]; S[a] = S[b]; S[b] = t;
        for (int i = 0; i < 3; ++i) {
          t = A[i][a]; A[i][a] = A[i][b]; A[i][b] = t;
          t = V[i][a]; V[i][a] = V[i][b]; V[i][b] = t;
        }
      }
  for (int j = 0; j < 3; ++j)
    for (int i = 0; i < 3; ++i) U[i][j] = S[j] > 0 ? A[i][j] / S[j] : 0.0;
  // a vanishing smallest singular value leaves its left vector free: complete
  // U to an orthonormal basis (its sign is absorbed by the determinant fix)
  if (!(S[2] > 1e-12 * fmax(S[0], 1e-300))) {
    U[0][2] = U[1][0] * U[2][1] - U[2][0] * U[1][1];
    U[1][2] = U[2][0] * U[0][1] - U[0][0] * U[2][1];
    U[2][2] = U[0][0] * U[1][1] - U[1][0] * U[0][1];
  }
}

// One workgroup: weighted centres and covariance of the CA atoms (f64), the
// SVD and the rotation R = V diag(1, 1, sign det(V U^T)) U^T; kab = R, xc, yc.
__global__ __launch_bounds__(256) void kabsch_kernel(const float* __restrict__ atom37,
                                                     const float* __restrict__ tpl37,
                                                     const float* __restrict__ tplm37,
                                                     const uint8_t* __restrict__ flags, int N,
                                                     float* __restrict__ kab) {
  __shared__ double red[256][10];
  const int tid = threadIdx.x;
  auto weight = [&](int i) -> double {
    const bool t = (flags[i] & F_TEMPLATE) && !(flags[i] & F_DESIGN);
    return t && tplm37[(long)i * A37 + CA37] > 0.f ? 1.0 : 0.0;
  };
  double acc[10] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
  for (int i = tid; i < N; i += 256) {
    const double w = weight(i);
    acc[0] += w;
    for (int c = 0; c < 3; ++c) {
      acc[1 + c] += w * atom37[((long)i * A37 + CA37) * 3 + c];
      acc[4 + c] += w * tpl37[((long)i * A37 + CA37) * 3 + c];
    }
  }
  auto reduce = [&](int n) {
    for (int k = 0; k < n; ++k) red[tid][k] = acc[k];
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
      if (tid < o)
        for (int k = 0; k < n; ++k) red[tid][k] += red[tid + o][k];
      __syncthreads();
    }
    for (int k = 0; k < n; ++k) acc[k] = red[0][k];
    __syncthreads();
  };
  reduce(7);
  const double ws = acc[0], inv = 1.0 / (ws + 1e-8);
  double xc[3], yc[3];
  for (int c = 0; c < 3; ++c) {
    xc[c] = acc[1 + c] * inv;
    yc[c] = acc[4 + c] * inv;
  }
  for (int k = 0; k < 9; ++k) acc[k] = 0;
  for (int i = tid; i < N; i += 256) {
    const double w = weight(i);
    if (w == 0.0) continue;
    double p[3], q[3];
    for (int c = 0; c < 3; ++c) {
      p[c] = atom37[((long)i * A37 + CA37) * 3 + c] - xc[c];
      q[c] = tpl37[((long)i * A37 + CA37) * 3 + c] - yc[c];
    }
    for (int a = 0; a < 3; ++a)
      for (int b = 0; b < 3; ++b) acc[a * 3 + b] += w * p[a] * q[b];
  }
  reduce(9);
  if (tid != 0) return;
  double H[3][3], U[3][3], S[3], V[3][3];
  for (int a = 0; a < 3; ++a)
    for (int b = 0; b < 3; ++b) H[a][b] = ws > 0 ? acc[a * 3 + b] : (a == b ? 1.0 : 0.0);
  svd3(H, U, S, V);
  double M[3][3];  // V U^T
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j) M[i][j] = V[i][0] * U[j][0] + V[i][1] * U[j][1] + V[i][2] * U[j][2];
  const double det = M[0][0] * (M[1][1] * M[2][2] - M[1][2] * M[2][1]) -
                     M[0][1] * (M[1][0] * M[2][2] - M[1][2] * M[2][0]) +
                     M[0][2] * (M[1][0] * M[2][1] - M[1][1] * M[2][0]);
  const double d = det >= 0 ? 1.0 : -1.0;
  for (int i = 0; i < 3; ++i)
    for (int j = 0; j < 3; ++j)
      kab[i * 3 + j] = (float)(V[i][0] * U[j][0] + V[i][1] * U[j][1] + d * V[i][2] * U[j][2]);
  for (int c = 0; c < 3; ++c) {
    kab[9 + c] = (float)xc[c];
    kab[12 + c] = (float)yc[c];
  }
}

// kab = the identity and zero centres (no alignment)
__global__ void kabsch_identity_kernel(float* kab) {
  const int t = threadIdx.x;
  if (t < 15) kab[t] = t < 9 ? (t % 4 == 0 ? 1.f : 0.f) : 0.f;
}

// atom37 = ((atom37 - xc) R^T + yc) * ex, in place (the xc, R of the CA atoms)
__global__ void align_apply_kernel(float* __restrict__ atom37, const float* __restrict__ mask37,
                                   const float* __restrict__ kab, int N) {
  const int e = blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= N * A37) return;
  float x[3];
#pragma unroll
  for (int c = 0; c < 3; ++c) x[c] = atom37[(long)e * 3 + c] - kab[9 + c];
  const float ex = mask37[e];
#pragma unroll
  for (int c = 0; c < 3; ++c) {
    const float y = kab[c * 3 + 0] * x[0] + kab[c * 3 + 1] * x[1] + kab[c * 3 + 2] * x[2] + kab[12 + c];
    atom37[(long)e * 3 + c] = y * ex;
  }
}

// d14 = d_atom14 (or 0) + the gather's transpose of (ex * d37 . R), one
// residue per thread (a fixed order over its 37 slots)
__global__ void atom37_bwd_kernel(const float* __restrict__ datom14, const float* __restrict__ d37,
                                  const float* __restrict__ aatype, const float* __restrict__ seq_mask,
                                  const float* __restrict__ a37_14,
                                  const float* __restrict__ a37_mask,
                                  const float* __restrict__ kab, int N, float* __restrict__ d14) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  float g[14][3];
#pragma unroll
  for (int j = 0; j < 14; ++j)
#pragma unroll
    for (int c = 0; c < 3; ++c) g[j][c] = datom14 ? datom14[((long)i * 14 + j) * 3 + c] : 0.f;
  const int aat = min(max((int)aatype[i], 0), 20);
  const bool on = seq_mask[i] != 0.f;
  for (int a = 0; a < A37; ++a) {
    const float ex = on ? a37_mask[aat * A37 + a] : 0.f;
    if (ex == 0.f) continue;
    const int j = (int)a37_14[aat * A37 + a];
    const float* d = d37 + ((long)i * A37 + a) * 3;
    // both masks (the gather's and the alignment's) scale the cotangent
    float r[3];
#pragma unroll
    for (int k = 0; k < 3; ++k)
      r[k] = (d[0] * kab[0 * 3 + k] + d[1] * kab[1 * 3 + k] + d[2] * kab[2 * 3 + k]) * ex * ex;
#pragma unroll
    for (int jj = 0; jj < 14; ++jj)
      if (jj == j)
#pragma unroll
        for (int k = 0; k < 3; ++k) g[jj][k] += r[k];
  }
#pragma unroll
  for (int j = 0; j < 14; ++j)
#pragma unroll
    for (int c = 0; c < 3; ++c) d14[((long)i * 14 + j) * 3 + c] = g[j][c];
}

// The template's MSA row, one workgroup per residue (modules_multimer.py:
// 1080-1137; the template arrays as bindcraft/af2.py:153-160 builds them
// from the input atoms): features one_hot(t, 22) with t = aatype on TEMPLATE
// residues, else 21 (the gap), then for the 4 chi angles sin m, cos m, m
// (atoms chi_idx[t], m = chi_mask[t] times all four present; t = 21 reads
// the unknown type's row 20), then relu(f . W1 + b1) . W2 + b2; the row's
// mask is m of chi 1.  Dihedral as geometry/vector.py:187-212.
__global__ __launch_bounds__(256) void template_row_kernel(
    const float* __restrict__ aatype, const uint8_t* __restrict__ flags,
    const float* __restrict__ ridx, float flex, const float* __restrict__ tpl37,
    const float* __restrict__ tplm37, const float* __restrict__ chi_idx,
    const float* __restrict__ chi_mask, const float* __restrict__ w1, const float* __restrict__ b1,
    const float* __restrict__ w2, const float* __restrict__ b2, float* __restrict__ row,
    float* __restrict__ rmask) {
  __shared__ float f[34];
  __shared__ float hid[CM];
  const int i = blockIdx.x, t = threadIdx.x;
  const bool tres = (flags[i] & F_TEMPLATE) != 0;
  // target flexibility (bindcraft/af2.py:150-157): a template residue, not
  // designed, whose index i has floor((i + 1) f) > floor(i f) (f32, as JAX)
  // is a gap; its chi features vanish with the gap's all-zero chi mask
  const bool flexible = tres && flex > 0.f && !(flags[i] & F_DESIGN) &&
                        floorf((ridx[i] + 1.f) * flex) > floorf(ridx[i] * flex);
  const int aat = (tres && !flexible) ? min(max((int)aatype[i], 0), 20) : 21;
  const int g = min(aat, 20);
  if (t < 22) f[t] = t == aat ? 1.f : 0.f;
  if (t < 4) {
    float p[4][3], m = chi_mask[g * 4 + t];
    for (int k = 0; k < 4; ++k) {
      const int a = (int)chi_idx[(g * 4 + t) * 4 + k];
      const long o = (long)i * A37 + a;
      m *= tres ? tplm37[o] : 0.f;
      for (int c = 0; c < 3; ++c) p[k][c] = tres ? tpl37[o * 3 + c] : 0.f;
    }
    float v1[3], v2[3], v3[3];
    for (int c = 0; c < 3; ++c) {
      v1[c] = p[0][c] - p[1][c];
      v2[c] = p[1][c] - p[2][c];
      v3[c] = p[3][c] - p[2][c];
    }
    auto cross = [](const float* x, const float* y, float* o) {
      o[0] = x[1] * y[2] - x[2] * y[1];
      o[1] = x[2] * y[0] - x[0] * y[2];
      o[2] = x[0] * y[1] - x[1] * y[0];
    };
    float c1[3], c2[3], c3[3];
    cross(v1, v2, c1);
    cross(v3, v2, c2);
    cross(c2, c1, c3);
    const float v2n = sqrtf(fmaxf(v2[0] * v2[0] + v2[1] * v2[1] + v2[2] * v2[2], 1e-12f));
    const float ang = atan2f(c3[0] * v2[0] + c3[1] * v2[1] + c3[2] * v2[2],
                             v2n * (c1[0] * c2[0] + c1[1] * c2[1] + c1[2] * c2[2]));
    f[22 + t] = sinf(ang) * m;
    f[26 + t] = cosf(ang) * m;
    f[30 + t] = m;
  }
  __syncthreads();
  float h = b1[t];
  for (int k = 0; k < 34; ++k) h += f[k] * w1[k * CM + t];
  hid[t] = fmaxf(h, 0.f);
  __syncthreads();
  float o = b2[t];
  for (int j = 0; j < CM; ++j) o += hid[j] * w2[j * CM + t];
  row[(long)i * CM + t] = o;
  if (t == 0) rmask[i] = f[30];
}

namespace {

// Cyclic sequence offsets (bindcraft/af2.py:174-185): off[i][j] = r_i - r_j,
// except between two unmasked CYCLIC residues of one chain, whose offset is
// the ring distance min(|d|, L - |d|) with d's sign (L = the chain's unmasked
// residue count); mode 1 ('direction') and 2 ('neighbours') negate it where
// the short way round is the other way, mode 2 then saturates beyond 2 at
// +-32.  One wave per row i: it first counts its chain's length.
__global__ __launch_bounds__(64) void cyclic_offsets_kernel(
    const float* __restrict__ ridx, const float* __restrict__ asym,
    const uint8_t* __restrict__ flags, const float* __restrict__ smask, int N, int mode,
    int32_t* __restrict__ off) {
  const int i = blockIdx.x, lane = threadIdx.x;
  const float ai = asym[i];
  float len = 0.f;
  for (int j = lane; j < N; j += 64) len += asym[j] == ai ? smask[j] : 0.f;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) len += __shfl_xor(len, o, 64);
  const bool ci = (flags[i] & F_CYCLIC) && smask[i] != 0.f;
  for (int j = lane; j < N; j += 64) {
    const int d = (int)ridx[i] - (int)ridx[j];
    int v = d;
    if (ci && asym[j] == ai && (flags[j] & F_CYCLIC) && smask[j] != 0.f) {
      const float ad = (float)abs(d);
      float cd = fminf(ad, len - ad);
      if (mode >= 1 && cd < ad) cd = -cd;
      if (mode == 2 && fabsf(cd) > 2.f) cd = cd > 0.f ? 32.f : -32.f;
      v = (int)(cd * (float)((d > 0) - (d < 0)));
    }
    off[(long)i * N + j] = v;
  }
}

// The runtime length: rows i >= *n of the caller's [N]-row buffers are
// padding.  smask = seq_mask and fl = flags on real rows, 0 on padding, so
// every mask the step derives (pair and MSA masks, the template row, the
// Kabsch selection, the confidence residue weights) leaves the padding out.
__global__ void pad_rows_kernel(const float* __restrict__ seq_mask,
                                const uint8_t* __restrict__ flags, const int32_t* __restrict__ n,
                                int N, float* __restrict__ smask, uint8_t* __restrict__ fl) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= N) return;
  const bool real = i < *n;
  smask[i] = real ? seq_mask[i] : 0.f;
  fl[i] = real ? flags[i] : (uint8_t)0;
}

// y = a where the entry's row (and, for a pair array, its column) is real,
// 0 on padding; with acc, y += that instead.  [N][K] (pair false) or
// [N][N][K] arrays; a == nullptr reads as zeros; a == y masks in place.
__global__ void pad_mask_kernel(const float* a, long total, int N, int K, bool pair,
                                const int32_t* __restrict__ n, bool acc, float* y) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= total) return;
  const int nn = *n;
  const long row = idx / K;  // i (row arrays) or i * N + j (pair arrays)
  const bool real = pair ? (row / N < nn && row % N < nn) : row < nn;
  const float v = (real && a) ? a[idx] : 0.f;
  y[idx] = acc ? y[idx] + v : v;
}

void pad_mask(hipStream_t st, const float* a, int N, int K, bool pair, const int32_t* n, bool acc,
              float* y) {
  if (!y) return;
  const long total = (long)N * (pair ? N : 1) * K;
  hipLaunchKernelGGL(pad_mask_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a,
                     total, N, K, pair, n, acc, y);
}

}  // namespace

size_t design_step_seq_save_bytes(const DesignStepW& w, int N) {
  Sizer s;
  SeqExtra<Sizer> x(s, N);
  (void)x;
  // room for the template's MSA row: the main stack runs two rows then
  return s.off + design_step_save_bytes(w, N, 2);
}

void design_step_seq_fwd(hipStream_t st, const DesignStepW& w, int N, const int32_t* nlen,
                         const float* logits, const uint8_t* flags_in, const float* bias,
                         const float* sc4, float omitted_half, const float* ri, const float* ai,
                         const float* ei, const float* si, const int32_t* offset,
                         const float* seq_mask_in, const float* act_const, const uint32_t* seeds,
                         bool dropout, int recycles, int cyclic_mode, float flexibility,
                         float* atom14, float* dgram, float* pae, float* plddt, float* expres,
                         const AtomsOut& atoms, const ConfOut& conf, void* save) {
  ds_check(w, N, 1);
  // the reference's attribute: bits 0-1 the offset mode, bit 2 the initial
  // atom positions; -1 here takes `offset` as given
  if (cyclic_mode < -1 || cyclic_mode > 6 || (cyclic_mode >= 0 && (cyclic_mode & 3) == 3))
    throw std::invalid_argument("design step: cyclic_mode must be -1 (offset as given) or an offset "
                                "mode 0, 1, 2 plus 4 for the initial atom positions");
  const bool init_pos = cyclic_mode >= 0 && (cyclic_mode & 4);
  if (init_pos && !atoms.tpl37)
    throw std::invalid_argument("design step: the initial atom positions are the atoms operand "
                                "(tpl_atoms37), which is missing");
  if (!(flexibility >= 0.f)) throw std::invalid_argument("design step: flexibility must be >= 0");
  nonnull(logits, "design step logits"); nonnull(flags_in, "design step flags");
  nonnull(sc4, "design step scalars"); nonnull(save, "design step save");
  nonnull(seq_mask_in, "design step seq_mask");
  Carver cv(save);
  SeqExtra<Carver> x(cv, N);
  // a runtime length masks the padding rows out of seq_mask and flags; every
  // mask downstream derives from these two
  const float* seq_mask = seq_mask_in;
  const uint8_t* flags = flags_in;
  if (nlen) {
    hipLaunchKernelGGL(pad_rows_kernel, dim3((unsigned)((N + 127) / 128)), dim3(128), 0, st,
                       seq_mask_in, flags_in, nlen, N, x.smask, x.fl);
    seq_mask = x.smask;
    flags = x.fl;
  }
  if (atoms.atom37) {
    if (!w.a37_14 || !w.a37_mask)
      throw std::invalid_argument("design step: atom37 outputs need const/atom37_to_atom14 and "
                                  "const/atom37_mask in the structure module's directory");
    nonnull(atoms.mask37, "design step atom37 mask");
  }
  if (atoms.tpl37) nonnull(atoms.tplm37, "design step template atom mask");
  // A template embedding adds the template's MSA row whenever its weights
  // are there (modules_multimer.py:608-617 adds it with every template), so
  // the backward knows the row from with_template alone.
  const bool row = act_const && w.trow.ok();
  if (row && !atoms.tpl37)
    throw std::invalid_argument("design step: the template's MSA row needs the template's atoms "
                                "(tpl_atoms37, tpl_mask37)");
  hdr_set(st, x.hdr, SEQ_MAGIC,
          (conf.plddt ? HAS_CONFIDENCE : 0u) | (atoms.atom37 ? HAS_ATOM37 : 0u) |
              (row ? HAS_ROW : 0u));
  seqfeat_fwd(st, logits, flags, bias, SeqScalars{}, sc4, omitted_half, N, x.feat, x.prof);
  design_inputs_fwd(st, x.feat, x.prof, N, x.tf, x.mf, x.aatype);
  if (row) {
    KTimed kt("design.template_row", st);
    hipLaunchKernelGGL(template_row_kernel, dim3((unsigned)N), dim3(CM), 0, st, x.aatype, flags,
                       ri, flexibility, atoms.tpl37, atoms.tplm37, w.trow.chi_idx,
                       w.trow.chi_mask, w.trow.w1, w.trow.b1, w.trow.w2, w.trow.b2, x.row,
                       x.rmask);
  }
  if (cyclic_mode >= 0) {
    // the offset feature the embedder reads, built here (bindcraft/af2.py:193)
    hipLaunchKernelGGL(cyclic_offsets_kernel, dim3((unsigned)N), dim3(64), 0, st, ri, ai, flags,
                       seq_mask, N, cyclic_mode & 3, x.off);
    offset = x.off;
  }
  design_step_fwd(st, w, N, 1, x.tf, x.mf, ri, ai, ei, si, offset, seq_mask, act_const, x.aatype,
                  seeds, dropout, recycles, atom14, dgram, pae, plddt, expres, cv.p + cv.off,
                  row ? x.row : nullptr, row ? x.rmask : nullptr,
                  init_pos ? atoms.tpl37 : nullptr);
  if (atoms.atom37) {
    KTimed kt("design.atom37", st);
    hipLaunchKernelGGL(atom37_kernel, dim3((unsigned)((N * A37 + 255) / 256)), dim3(256), 0, st,
                       atom14, x.aatype, seq_mask, w.a37_14, w.a37_mask, N, atoms.atom37,
                       atoms.mask37);
    if (atoms.tpl37) {
      hipLaunchKernelGGL(kabsch_kernel, dim3(1), dim3(256), 0, st, atoms.atom37, atoms.tpl37,
                         atoms.tplm37, flags, N, x.kab);
      hipLaunchKernelGGL(align_apply_kernel, dim3((unsigned)((N * A37 + 255) / 256)), dim3(256), 0,
                         st, atoms.atom37, atoms.mask37, x.kab, N);
    } else {
      hipLaunchKernelGGL(kabsch_identity_kernel, dim3(1), dim3(64), 0, st, x.kab);
    }
  }
  if (conf.plddt) {
    nonnull(conf.asym, "design step interface asym");
    confidence_fwd(st, plddt, pae, expres, seq_mask, conf.asym, N, conf.plddt, conf.pae, conf.ptm,
                   conf.iptm, conf.iptm_pr, conf.expres_ca, x.conf);
    // the backward reads the logits from the save buffer, not the caller's outputs
    BC2N_HIP(hipMemcpyAsync(x.ll, plddt, (size_t)N * CONF_LBINS * 4, hipMemcpyDeviceToDevice, st));
    BC2N_HIP(hipMemcpyAsync(x.pl, pae, (size_t)N * N * CONF_PBINS * 4, hipMemcpyDeviceToDevice, st));
    BC2N_HIP(hipMemcpyAsync(x.el, expres, (size_t)N * CONF_EXPRES * 4, hipMemcpyDeviceToDevice, st));
  }
  if (nlen) {
    // the padding's outputs are zero (the metrics' backward keeps its own copies)
    KTimed kt("design.pad_outputs", st);
    pad_mask(st, atom14, N, 14 * 3, false, nlen, false, atom14);
    pad_mask(st, dgram, N, CONF_PBINS, true, nlen, false, dgram);
    pad_mask(st, pae, N, CONF_PBINS, true, nlen, false, pae);
    pad_mask(st, plddt, N, CONF_LBINS, false, nlen, false, plddt);
    pad_mask(st, expres, N, CONF_EXPRES, false, nlen, false, expres);
    pad_mask(st, atoms.atom37, N, A37 * 3, false, nlen, false, atoms.atom37);
    pad_mask(st, atoms.mask37, N, A37, false, nlen, false, atoms.mask37);
    pad_mask(st, conf.plddt, N, 1, false, nlen, false, conf.plddt);
    pad_mask(st, conf.pae, N, 1, true, nlen, false, conf.pae);
    pad_mask(st, conf.iptm_pr, N, 1, false, nlen, false, conf.iptm_pr);
    pad_mask(st, conf.expres_ca, N, 1, false, nlen, false, conf.expres_ca);
  }
}

void design_step_seq_bwd(hipStream_t st, const DesignStepW& w, int N, const int32_t* nlen,
                         const float* logits, const uint8_t* flags_in, const float* bias,
                         const float* sc4, float omitted_half, const float* seq_mask_in,
                         bool with_template, bool dropout, void* save, const float* datom,
                         const float* ddgram, const float* dpae, const float* dplddt,
                         const float* dexpres, const float* datom37, const ConfCt& conf_in,
                         float* d_logits) {
  ds_check(w, N, 1);
  nonnull(logits, "design step logits"); nonnull(flags_in, "design step flags");
  nonnull(sc4, "design step scalars"); nonnull(save, "design step save");
  nonnull(d_logits, "design step d_logits"); nonnull(seq_mask_in, "design step seq_mask");
  Carver cv(save);
  SeqExtra<Carver> x(cv, N);
  // confidence cotangents need the forward's metrics; leaving them out is allowed
  const long seq_flags = hdr_flags(st, x.hdr, SEQ_MAGIC, "design step");
  if (conf_in.any()) hdr_require(seq_flags, HAS_CONFIDENCE, true, "design step");
  if (datom37) hdr_require(seq_flags, HAS_ATOM37, true, "design step");
  const float* seq_mask = seq_mask_in;
  const uint8_t* flags = flags_in;
  ConfCt conf = conf_in;
  if (nlen) {
    // the forward's masks again, and every cotangent with its padding zeroed:
    // a query at a padding position still attends to real keys, so a nonzero
    // cotangent there would reach the real rows
    KTimed kt("design.pad_cotangents", st);
    hipLaunchKernelGGL(pad_rows_kernel, dim3((unsigned)((N + 127) / 128)), dim3(128), 0, st,
                       seq_mask_in, flags_in, nlen, N, x.smask, x.fl);
    seq_mask = x.smask;
    flags = x.fl;
    float* c0 = x.cc;  // [N] plddt, [N][N] pae, [N] per-residue ipTM, [N] expres-CA
    float* c1 = c0 + N;
    float* c2 = c1 + (size_t)N * N;
    float* c3 = c2 + N;
    if (conf.plddt) pad_mask(st, conf.plddt, N, 1, false, nlen, false, c0), conf.plddt = c0;
    if (conf.pae) pad_mask(st, conf.pae, N, 1, true, nlen, false, c1), conf.pae = c1;
    if (conf.iptm_pr) pad_mask(st, conf.iptm_pr, N, 1, false, nlen, false, c2), conf.iptm_pr = c2;
    if (conf.expres_ca)
      pad_mask(st, conf.expres_ca, N, 1, false, nlen, false, c3), conf.expres_ca = c3;
    if (ddgram) pad_mask(st, ddgram, N, CONF_PBINS, true, nlen, false, x.dd), ddgram = x.dd;
  }
  if (datom37) {
    KTimed kt("design.atom37_bwd", st);
    hipLaunchKernelGGL(atom37_bwd_kernel, dim3((unsigned)((N + 63) / 64)), dim3(64), 0, st, datom,
                       datom37, x.aatype, seq_mask, w.a37_14, w.a37_mask, x.kab, N, x.d14);
    datom = x.d14;
  }
  if (nlen && datom) {
    // per residue, so masking the sum masks both terms
    pad_mask(st, datom, N, 14 * 3, false, nlen, false, x.d14);
    datom = x.d14;
  }
  if (conf.any()) {
    // the confidence metrics' backward over the logits the forward kept (confidence requested there)
    nonnull(conf.asym, "design step interface asym");
    confidence_bwd(st, x.ll, x.pl, x.el, seq_mask, conf.asym, N, x.conf, conf.plddt,
                   conf.pae, conf.ptm, conf.iptm, conf.iptm_pr, conf.expres_ca, x.dl, x.dp, x.de);
    if (nlen) {
      pad_mask(st, dplddt, N, CONF_LBINS, false, nlen, true, x.dl);
      pad_mask(st, dpae, N, CONF_PBINS, true, nlen, true, x.dp);
      pad_mask(st, dexpres, N, CONF_EXPRES, false, nlen, true, x.de);
    } else {
      add_into(st, dplddt, nullptr, (long)N * CONF_LBINS, x.dl);
      add_into(st, dpae, nullptr, (long)N * N * CONF_PBINS, x.dp);
      add_into(st, dexpres, nullptr, (long)N * CONF_EXPRES, x.de);
    }
    dplddt = x.dl;
    dpae = x.dp;
    dexpres = x.de;
  } else if (nlen) {
    if (dplddt) pad_mask(st, dplddt, N, CONF_LBINS, false, nlen, false, x.dl), dplddt = x.dl;
    if (dpae) pad_mask(st, dpae, N, CONF_PBINS, true, nlen, false, x.dp), dpae = x.dp;
    if (dexpres) pad_mask(st, dexpres, N, CONF_EXPRES, false, nlen, false, x.de), dexpres = x.de;
  }
  // the inner step's header checks the template embedding, then the row
  const bool row = with_template && w.trow.ok();
  design_step_bwd(st, w, N, 1, x.tf, seq_mask, with_template, x.aatype, dropout, cv.p + cv.off,
                  datom, ddgram, dpae, dplddt, dexpres, x.dtf, x.dmf, row);
  design_inputs_bwd(st, x.dtf, x.dmf, N, x.dfeat, x.dprof);
  seqfeat_bwd(st, logits, flags, bias, SeqScalars{}, sc4, omitted_half, N, x.dfeat, x.dprof,
              d_logits);
  if (nlen) pad_mask(st, d_logits, N, 20, false, nlen, false, d_logits);
}

}  // namespace bc2n
