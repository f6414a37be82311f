// Evoformer block and stack, forward and backward, with JAX-exact dropout.
//
// Block order (modules.py:1278-1391, outer_product_mean.first=True):
//   pair += OPM(msa)               msa += RowAttn(msa, pair)
//   msa  += ColAttn(msa)           msa += MsaTransition(msa)
//   pair += TriMulOut, TriMulIn, TriAttnStart, TriAttnEnd, PairTransition
// each wrapped in dropout_wrapper with the shared per-row/per-column mask of
// its config (config.py:386-460).  pair_only blocks (the extra-MSA stack with
// its MSA mask all zero, native/block.cuh:79-91) reduce the MSA side to OPM's
// constant output_b/1e-3 and skip the MSA modules.
//
// The stack keeps every block's carries and module save-sets (no replay):
// 288 GB of HBM holds them at the lengths the configs use.  Dropout keys are
// derived on the device from the stack key by JAX's split chain
// (modules_multimer.py:622-641), turned into shared-mask tables once per
// forward and kept in the save-set, so the backward applies the identical
// masks and a reseed is a new value in the seed operand, not a recompile.
#include "evoformer.h"

namespace bc2n {

namespace {

// module indices of a block's 9 dropout keys (modules.py:1308-1390 order)
enum { K_OPM = 0, K_ROW, K_COL, K_MTR, K_TMO, K_TMI, K_TAS, K_TAE, K_PTR };
// ... and of the template iteration's 5 (modules_multimer.py:1039-1075)
enum { T_TMO = 0, T_TMI, T_TAS, T_TAE, T_PTR };

size_t al256(size_t n) { return (n + 255) & ~size_t(255); }

struct Layout {
  int N = 0, S = 0, Cz = 0, Cm = 0, depth = 0;
  bool pair_only = false, tpl = false;
  // a detached forward (no backward follows): one block region reused by
  // every block and two carry slots used in turn, instead of the save-set
  bool detached = false;
  // the replay tier: every block's input carries and one block region; the
  // backward runs each block's forward again into that region first
  bool replay = false;
  size_t opm = 0, row = 0, col = 0, mtr = 0, tmo = 0, tmi = 0, tas = 0, tae = 0, ptr = 0;
  size_t pair_bytes = 0, msa_bytes = 0, block_bytes = 0;
  size_t tbl_per_block = 0;  // floats
  // offsets of the save-set regions
  size_t off_carry_p = 0, off_carry_m = 0, off_msa_in = 0, off_pair_in = 0, off_scr = 0,
         off_tbl = 0, off_keys = 0, total = 0;
};

// Which save-set a stack keeps: 0 = by size (the replay tier when the full
// one would take more than 60% of the device's memory), 1 = always the full
// one, 2 = always the replay tier.  Process-wide; the forward and its
// backward must see the same policy (bc2n_set_save_policy).
int g_save_policy = 0;

size_t device_total_bytes() {
  static size_t cache[64] = {};
  int dev = 0;
  BC2N_HIP(hipGetDevice(&dev));
  if (dev < 0 || dev >= 64) throw std::runtime_error("stack: device index out of range");
  if (!cache[dev]) {
    size_t fr = 0, tot = 0;
    BC2N_HIP(hipMemGetInfo(&fr, &tot));
    cache[dev] = tot;
  }
  return cache[dev];
}

bool use_replay(size_t full_bytes) {
  if (g_save_policy == 1) return false;
  if (g_save_policy == 2) return true;
  return full_bytes > device_total_bytes() / 10 * 6;
}

Layout layout(const StackW& w, int N, int S, int depth, bool detached = false) {
  Layout L;
  L.N = N; L.S = S; L.depth = depth; L.pair_only = w.pair_only; L.detached = detached;
  L.tpl = (w.kind == StackKind::TEMPLATE);
  const BlockW& b = w.blocks[0];
  L.Cz = b.tmo.C;
  L.Cm = w.pair_only ? 0 : b.row.a.Cin;
  const long M = (long)N * N;
  L.tmo = trimul_save_bytes(N, b.tmo.C, b.tmo.I);
  L.tmi = trimul_save_bytes(N, b.tmi.C, b.tmi.I);
  L.tas = triattn_save_bytes(N, b.tas.C, b.tas.H);
  L.tae = triattn_save_bytes(N, b.tae.C, b.tae.H);
  L.ptr = transition_save_bytes(M, b.ptr.C, b.ptr.F);
  if (!w.pair_only) {
    L.opm = opm_save_bytes(S, N, b.opm.O, b.opm.C);
    L.row = msarow_save_bytes(S, N, b.row.a.Cin, b.row.a.H);
    L.col = msacol_save_bytes(S, N, b.col.a.Cin, b.col.a.H);
    L.mtr = transition_save_bytes((long)S * N, b.mtr.C, b.mtr.F);
  }
  L.pair_bytes = al256((size_t)M * L.Cz * 4);
  L.msa_bytes = w.pair_only ? 0 : al256((size_t)S * N * L.Cm * 4);
  // per block: module save-sets + the pair after opm, tmo, tmi, tas, tae and
  // the msa after row and col attention
  L.block_bytes = L.opm + L.row + L.col + L.mtr + L.tmo + L.tmi + L.tas + L.tae + L.ptr +
                  5 * L.pair_bytes + 2 * L.msa_bytes;
  L.tbl_per_block = (size_t)N * L.Cm + 4 * (size_t)N * L.Cz;
  auto place = [&](bool replay) {
    L.replay = replay;
    const size_t regions = (detached || replay) ? 1 : (size_t)depth;
    const size_t carries = detached ? 2 : (size_t)depth - 1;
    L.off_carry_p = regions * L.block_bytes;
    L.off_carry_m = L.off_carry_p + carries * L.pair_bytes;
    // the stack's msa input, kept for the backward of block 0
    L.off_msa_in = L.off_carry_m + carries * L.msa_bytes;
    // the template iteration's first module reads the block input itself, and
    // a replayed block 0 reads both inputs: the stack's pair input is kept
    L.off_pair_in = L.off_msa_in + (detached ? 0 : L.msa_bytes);
    L.off_scr = L.off_pair_in + ((L.tpl || replay) && !detached ? L.pair_bytes : 0);
    // the replayed last block's outputs land here (the caller's are not given)
    L.off_tbl = L.off_scr + (replay ? L.pair_bytes + L.msa_bytes : 0);
    L.off_keys = L.off_tbl + al256((size_t)depth * L.tbl_per_block * 4);
    L.total = L.off_keys + al256((size_t)depth * 9 * 2 * 4);
  };
  place(false);
  if (!detached && use_replay(L.total)) place(true);
  (void)K_OPM; (void)K_COL; (void)K_MTR; (void)K_PTR; (void)T_PTR;
  return L;
}

struct BlockPtrs {
  char *opm, *row, *col, *mtr, *tmo, *tmi, *tas, *tae, *ptr;
  float *p1, *p2, *p3, *p4, *p5;  // pair after opm, tmo, tmi, tas, tae
  float *m1, *m2;                 // msa after row, col
};

BlockPtrs carve(const Layout& L, char* base) {
  BlockPtrs p{};
  char* c = base;
  auto take = [&](size_t n) { char* r = c; c += n; return r; };
  p.opm = take(L.opm); p.row = take(L.row); p.col = take(L.col); p.mtr = take(L.mtr);
  p.tmo = take(L.tmo); p.tmi = take(L.tmi); p.tas = take(L.tas); p.tae = take(L.tae);
  p.ptr = take(L.ptr);
  p.p1 = reinterpret_cast<float*>(take(L.pair_bytes));
  p.p2 = reinterpret_cast<float*>(take(L.pair_bytes));
  p.p3 = reinterpret_cast<float*>(take(L.pair_bytes));
  p.p4 = reinterpret_cast<float*>(take(L.pair_bytes));
  p.p5 = reinterpret_cast<float*>(take(L.pair_bytes));
  p.m1 = reinterpret_cast<float*>(take(L.msa_bytes));
  p.m2 = reinterpret_cast<float*>(take(L.msa_bytes));
  return p;
}

// pair_out = pair_in + c with the per-channel constant c = output_b / 1e-3
// (OPM of a fully masked MSA: left = right = 0, norm = 0).  OPM's dropout
// rate is 0, and its backward on the pair is the identity.
__global__ void add_const_kernel(const float* __restrict__ in, float* __restrict__ out,
                                 const float* __restrict__ b, long M, int C) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * C) return;
  out[i] = in[i] + b[i % C] / 1e-3f;
}

struct Tables {
  const float* base = nullptr;
  const Layout* L = nullptr;
  const float* row(int b) const { return base ? base + b * L->tbl_per_block : nullptr; }
  const float* pair(int b, int k) const {
    return base ? base + b * L->tbl_per_block + (size_t)L->N * L->Cm + (size_t)k * L->N * L->Cz
                : nullptr;
  }
};

struct Frame {
  const float *pin, *min;
  float *pout, *mout;
};

Frame frame(const Layout& L, char* save, int b, const float* pair, const float* msa,
            float* pair_out, float* msa_out) {
  Frame f;
  // carry k = output of block k; a detached forward alternates two slots
  auto slot = [&](int k) { return (size_t)(L.detached ? k % 2 : k); };
  auto cp = [&](int k) { return reinterpret_cast<float*>(save + L.off_carry_p + slot(k) * L.pair_bytes); };
  auto cm = [&](int k) { return reinterpret_cast<float*>(save + L.off_carry_m + slot(k) * L.msa_bytes); };
  // pair == nullptr: the backward, which reads block 0's input from the save-set
  f.pin = b == 0 ? (pair ? pair : (L.tpl ? reinterpret_cast<float*>(save + L.off_pair_in) : nullptr))
                 : cp(b - 1);
  f.pout = b == L.depth - 1 ? pair_out : cp(b);
  if (L.pair_only) {
    f.min = msa;
    f.mout = nullptr;
  } else {
    // msa == nullptr: the backward, which reads block 0's input from the save-set
    f.min = b == 0 ? (msa ? msa : reinterpret_cast<float*>(save + L.off_msa_in)) : cm(b - 1);
    f.mout = b == L.depth - 1 ? msa_out : cm(b);
  }
  return f;
}

// ------------------------------------------------------------ two streams
// With the MSA overlap on (msa_overlap(), the default), a block's MSA side
// runs on the side stream (lane 1, its own arena) beside the pair track:
//
//  forward   main: OPM's pair half, then the pair track
//            side: row attention (reads p1 only), column attention, MSA
//                  transition, then the NEXT block's OPM MSA half (LayerNorm
//                  and projections of this block's msa output)
//  backward  side: the later block's deferred OPM backward, then this
//                  block's MSA transition and column attention backward and
//                  the row attention's backward up to its pair-bias gradient
//            main: the pair track's backward, then (join) the row attention's
//                  pair term; this block's OPM backward is deferred to the
//                  side stream, beside the earlier block's pair track
//
// The deferred OPM backward reads this block's pair cotangent while the
// earlier block's pair track writes its own, so the stack alternates two pair
// cotangent buffers; it finishes (on the side stream, in order) before the
// earlier block's bias gradient, which main waits for before touching the
// buffer again.  Every kernel computes what it computes on one stream, so
// the results are bit-identical to the single-stream order.

struct FwdPipe {
  bool on = false;
  hipStream_t ms = nullptr;
  bool prepped = false;  // this block's OPM MSA half was issued by the block before
  // the next block's OPM MSA half, issued by this block (null: none)
  const OpmW* next_opm = nullptr;
  char* next_opm_save = nullptr;
};

struct OpmPending {
  bool on = false;
  const OpmW* w = nullptr;
  const float* min = nullptr;
  const char* save = nullptr;
  const float* dpair = nullptr;
  const float* sp = nullptr;
};

struct BwdPipe {
  bool on = false;
  bool defer_opm = false;  // false: each block's OPM backward before the next block (replay tier)
  hipStream_t ms = nullptr;
  OpmPending opm;
  // partial maxima of the last block's pair cotangent output amax_of, left
  // in the pair lane's ct_fused_parts() by its last writer (amax_np of them)
  long amax_np = 0;
  const float* amax_of = nullptr;
};

namespace {
void issue_opm_bwd(hipStream_t ms, const OpmPending& o, int S, int N, const float* mmask,
                   float* dmsa) {
  opm_bwd(ms, *o.w, S, N, o.min, mmask, nullptr, o.save, o.dpair, dmsa, dmsa, o.sp);
}
}  // namespace

void block_fwd(hipStream_t st, const BlockW& B, const Layout& L, int b, const Tables& t,
               const Frame& f, const float* pmask, const float* mmask, char* save,
               const FwdPipe* pipe = nullptr) {
  BlockPtrs p = carve(L, save);
  const int N = L.N, S = L.S;
  const long M = (long)N * N;
  // the template iteration starts at the triangle multiplications
  const float* p1 = L.tpl ? f.pin : p.p1;
  const bool msa_side = !L.tpl && !L.pair_only;
  const bool two = msa_side && pipe && pipe->on;
  if (L.tpl) {
  } else if (L.pair_only) {
    KTimed kt("block.opm_const", st);
    hipLaunchKernelGGL(add_const_kernel, dim3((unsigned)((M * L.Cz + 255) / 256)), dim3(256), 0,
                       st, f.pin, p.p1, B.opm_b, M, L.Cz);
  } else if (!two) {
    opm_fwd(st, B.opm, S, N, f.min, mmask, f.pin, nullptr, p.p1, p.opm);
    msarow_fwd(st, B.row, S, N, f.min, mmask, p.p1, t.row(b), p.m1, p.row);
    msacol_fwd(st, B.col, S, N, p.m1, mmask, nullptr, p.m2, p.col);
    transition_fwd(st, B.mtr, (long)S * N, N, p.m2, nullptr, f.mout, p.mtr);
  } else {
    hipStream_t ms = pipe->ms;
    if (pipe->prepped) stream_wait(st, ms);  // this block's OPM MSA half, the last MSA side
    else opm_fwd_msa(st, B.opm, S, N, f.min, mmask, p.opm);
    opm_fwd_pair(st, B.opm, S, N, f.pin, nullptr, p.p1, p.opm);
    stream_wait(ms, st);
    LaneGuard lg(1);
    msarow_fwd(ms, B.row, S, N, f.min, mmask, p.p1, t.row(b), p.m1, p.row);
    msacol_fwd(ms, B.col, S, N, p.m1, mmask, nullptr, p.m2, p.col);
    transition_fwd(ms, B.mtr, (long)S * N, N, p.m2, nullptr, f.mout, p.mtr);
    if (pipe->next_opm) opm_fwd_msa(ms, *pipe->next_opm, S, N, f.mout, mmask, pipe->next_opm_save);
  }
  trimul_fwd(st, B.tmo, true, N, p1, pmask, t.pair(b, 0), p.p2, p.tmo);
  trimul_fwd(st, B.tmi, false, N, p.p2, pmask, t.pair(b, 1), p.p3, p.tmi);
  triattn_fwd(st, B.tas, false, N, p.p3, pmask, t.pair(b, 2), p.p4, p.tas);
  triattn_fwd(st, B.tae, true, N, p.p4, pmask, t.pair(b, 3), p.p5, p.tae);
  transition_fwd(st, B.ptr, M, N, p.p5, nullptr, f.pout, p.ptr);
}

// dp_in: the cotangent of the block's pair output; dp_out (== dp_in on one
// stream) receives that of its pair input.  dmsa: the msa cotangent, in place.
void block_bwd(hipStream_t st, const BlockW& B, const Layout& L, int b, const Tables& t,
               const Frame& f, const float* pmask, const float* mmask, char* save,
               const float* dp_in, float* dp_out, float* dmsa, BwdPipe* pipe = nullptr) {
  BlockPtrs p = carve(L, save);
  const int N = L.N, S = L.S;
  const long M = (long)N * N;
  const bool msa_side = !L.tpl && !L.pair_only;
  const bool two = msa_side && pipe && pipe->on;
  // one cotangent scale per carry and block (the modules' own would cost a
  // max-reduction each); within a block the pair cotangent grows by a few
  // tens of percent, far inside binary16's headroom over the scaled maximum
  float* sm = msa_side ? ct_scale_slot(2) : nullptr;
  const float* dbias = nullptr;
  if (two) {
    hipStream_t ms = pipe->ms;
    stream_wait(ms, st);
    LaneGuard lg(1);
    if (pipe->opm.on) {
      issue_opm_bwd(ms, pipe->opm, S, N, mmask, dmsa);
      pipe->opm.on = false;
    }
    {
      KTimed kt("block.ct_scale", ms);
      ct_scale(ms, dmsa, (long)S * N * L.Cm, sm);
    }
    transition_bwd(ms, B.mtr, (long)S * N, N, p.m2, nullptr, p.mtr, dmsa, dmsa, sm);
    msacol_bwd(ms, B.col, S, N, p.m1, mmask, nullptr, p.col, dmsa, dmsa, sm);
    dbias = msarow_bwd_msa(ms, B.row, S, N, f.min, mmask, t.row(b), p.row, dmsa, dmsa, sm);
  }
  // the pair scale alternates two slots a block when the OPM backward that
  // reads it is deferred past the next block's ct_scale
  float* sp = ct_scale_slot(two ? 4 + (b & 1) : 1);
  {
    KTimed kt("block.ct_scale", st);
    if (pipe && pipe->amax_np > 0 && pipe->amax_of == dp_in)
      ct_scale_parts(st, ct_fused_parts(), pipe->amax_np, sp);
    else
      ct_scale(st, dp_in, M * L.Cz, sp);
    if (pipe) pipe->amax_np = 0;
  }
  transition_bwd(st, B.ptr, M, N, p.p5, nullptr, p.ptr, dp_in, dp_out, sp);
  triattn_bwd(st, B.tae, true, N, p.p4, pmask, t.pair(b, 3), p.tae, dp_out, dp_out, sp);
  triattn_bwd(st, B.tas, false, N, p.p3, pmask, t.pair(b, 2), p.tas, dp_out, dp_out, sp);
  trimul_bwd(st, B.tmi, false, N, p.p2, pmask, t.pair(b, 1), p.tmi, dp_out, dp_out, sp);
  trimul_bwd(st, B.tmo, true, N, L.tpl ? f.pin : p.p1, pmask, t.pair(b, 0), p.tmo, dp_out, dp_out,
             sp);
  if (!msa_side) return;
  if (!two) {
    {
      KTimed kt("block.ct_scale", st);
      ct_scale(st, dmsa, (long)S * N * L.Cm, sm);
    }
    transition_bwd(st, B.mtr, (long)S * N, N, p.m2, nullptr, p.mtr, dmsa, dmsa, sm);
    msacol_bwd(st, B.col, S, N, p.m1, mmask, nullptr, p.col, dmsa, dmsa, sm);
    // the row attention's pair term is the block's last write of dp_out: its
    // partial maxima serve the next block's pair scale
    const long np = msarow_bwd(st, B.row, S, N, f.min, mmask, p.p1, t.row(b), p.row, dmsa, dmsa,
                               dp_out, sm, pipe ? ct_fused_parts() : nullptr);
    if (pipe) {
      pipe->amax_np = np;
      pipe->amax_of = dp_out;
    }
    opm_bwd(st, B.opm, S, N, f.min, mmask, nullptr, p.opm, dp_out, dmsa, dmsa, sp);
    return;
  }
  stream_wait(st, pipe->ms);  // the pair-bias gradient (and the MSA side so far)
  // the block's last write of dp_out (the OPM backward only reads it)
  pipe->amax_np = msarow_bwd_pair(st, B.row, S, N, p.p1, p.row, dbias, dp_out, sm, ct_fused_parts());
  pipe->amax_of = dp_out;
  pipe->opm = OpmPending{true, &B.opm, f.min, p.opm, dp_out, sp};
  if (!pipe->defer_opm) {
    hipStream_t ms = pipe->ms;
    stream_wait(ms, st);
    LaneGuard lg(1);
    issue_opm_bwd(ms, pipe->opm, S, N, mmask, dmsa);
    pipe->opm.on = false;
    stream_wait(st, ms);
  }
}

void stack_check(const StackW& w, int N, int S, int depth) {
  if (depth <= 0 || depth > (int)w.blocks.size()) throw std::runtime_error("stack: bad depth");
  if (N <= 0 || N % 32 != 0) throw std::runtime_error("stack: N must be a positive multiple of 32");
  if (!w.pair_only && (S <= 0 || S > 32)) throw std::runtime_error("stack: S must be in 1..32");
}

}  // namespace

BlockW block_weights(WeightStore& ws, const std::string& P, StackKind kind) {
  const bool pair_only = kind != StackKind::EVO;
  BlockW b;
  b.tmo = trimul_weights(ws, P + "triangle_multiplication_outgoing/");
  b.tmi = trimul_weights(ws, P + "triangle_multiplication_incoming/");
  b.tas = triattn_weights(ws, P + "triangle_attention_starting_node/");
  b.tae = triattn_weights(ws, P + "triangle_attention_ending_node/");
  b.ptr = transition_weights(ws, P + "pair_transition/");
  if (kind != StackKind::TEMPLATE) b.opm_b = ws.f32(P + "outer_product_mean/output_b");
  if (!pair_only) {
    b.opm = opm_weights(ws, P + "outer_product_mean/");
    b.row = msarow_weights(ws, P + "msa_row_attention_with_pair_bias/");
    b.col = msacol_weights(ws, P + "msa_column_attention/");
    b.mtr = transition_weights(ws, P + "msa_transition/");
  }
  return b;
}

StackW stack_weights(WeightStore& ws, int depth, StackKind kind, const std::string& root) {
  StackW s;
  s.kind = kind;
  s.pair_only = kind != StackKind::EVO;
  for (int b = 0; b < depth; ++b)
    s.blocks.push_back(block_weights(ws, root + "block" + std::to_string(b) + "/", kind));
  return s;
}

size_t stack_save_bytes(const StackW& w, int N, int S, int depth) {
  stack_check(w, N, S, depth);
  return layout(w, N, S, depth).total;
}

size_t stack_detached_bytes(const StackW& w, int N, int S, int depth) {
  stack_check(w, N, S, depth);
  return layout(w, N, S, depth, true).total;
}

void stack_fwd(hipStream_t st, const StackW& w, int N, int S, int depth, const float* pair,
               const float* msa, const float* pmask, const float* mmask, const uint32_t* key,
               const uint32_t* enabled, bool dropout, float* pair_out, float* msa_out,
               void* save, bool detached) {
  stack_check(w, N, S, depth);
  const Layout L = layout(w, N, S, depth, detached);
  char* sv = reinterpret_cast<char*>(save);
  Tables t;
  t.L = &L;
  if (dropout) {
    if (!key) throw std::runtime_error("stack: dropout needs a key");
    float* tbl = reinterpret_cast<float*>(sv + L.off_tbl);
    uint32_t* keys = reinterpret_cast<uint32_t*>(sv + L.off_keys);
    KTimed kt("stack.dropout_tables", st);
    const int nk = L.tpl ? 5 : 9;
    stack_keys(st, key, depth, keys, nk);
    const int pm_evo[4] = {K_TMO, K_TMI, K_TAS, K_TAE};
    const int pm_tpl[4] = {T_TMO, T_TMI, T_TAS, T_TAE};
    const int* pm = L.tpl ? pm_tpl : pm_evo;
    const int pk[4] = {pm[0], pm[1], pm[2], pm[3]};
    stack_dropout_tables(st, tbl, (long)L.tbl_per_block, N, L.Cm, L.Cz, depth, nk, !L.pair_only,
                         K_ROW, pk, keys, enabled);
    t.base = tbl;
  }
  if (!L.pair_only && !detached)
    BC2N_HIP(hipMemcpyAsync(sv + L.off_msa_in, msa, (size_t)S * N * L.Cm * 4,
                            hipMemcpyDeviceToDevice, st));
  if ((L.tpl || L.replay) && !detached)
    BC2N_HIP(hipMemcpyAsync(sv + L.off_pair_in, pair, (size_t)N * N * L.Cz * 4,
                            hipMemcpyDeviceToDevice, st));
  const bool one_region = detached || L.replay;
  auto region = [&](int b) { return sv + (one_region ? 0 : (size_t)b * L.block_bytes); };
  FwdPipe pipe;
  pipe.on = !L.tpl && !L.pair_only && msa_overlap();
  if (pipe.on) pipe.ms = side_stream();
  for (int b = 0; b < depth; ++b) {
    pipe.prepped = b > 0;
    pipe.next_opm = b + 1 < depth ? &w.blocks[b + 1].opm : nullptr;
    pipe.next_opm_save = b + 1 < depth ? carve(L, region(b + 1)).opm : nullptr;
    block_fwd(st, w.blocks[b], L, b, t, frame(L, sv, b, pair, msa, pair_out, msa_out), pmask,
              mmask, region(b), &pipe);
  }
  if (pipe.on) stream_wait(st, pipe.ms);  // the last block's MSA output
}

void stack_bwd(hipStream_t st, const StackW& w, int N, int S, int depth, const float* pmask,
               const float* mmask, bool dropout, const void* save, const float* ct_pair,
               const float* ct_msa, float* dpair, float* dmsa) {
  stack_check(w, N, S, depth);
  const Layout L = layout(w, N, S, depth);
  char* sv = const_cast<char*>(reinterpret_cast<const char*>(save));
  Tables t;
  t.L = &L;
  if (dropout) t.base = reinterpret_cast<const float*>(sv + L.off_tbl);
  const long M = (long)N * N;
  BwdPipe pipe;
  pipe.on = !L.tpl && !L.pair_only && msa_overlap();
  pipe.defer_opm = !L.replay;  // the replay tier's next forward reuses the block region
  if (pipe.on) pipe.ms = side_stream();
  // two streams: block b's pair cotangent input dp(b + 1), output dp(b), with
  // dp(0) = dpair; one stream: dpair throughout
  const size_t pb = (size_t)M * L.Cz * 4;
  float* alt = pipe.on ? stack_pair_scratch(pb) : nullptr;
  auto dp = [&](int k) { return (!pipe.on || k % 2 == 0) ? dpair : alt; };
  if (dp(depth) != ct_pair)
    BC2N_HIP(hipMemcpyAsync(dp(depth), ct_pair, pb, hipMemcpyDeviceToDevice, st));
  if (!L.pair_only && dmsa != ct_msa)
    BC2N_HIP(hipMemcpyAsync(dmsa, ct_msa, (size_t)S * N * L.Cm * 4, hipMemcpyDeviceToDevice, st));
  auto finish = [&] {
    if (!pipe.on) return;
    if (pipe.opm.on) {
      stream_wait(pipe.ms, st);
      LaneGuard lg(1);
      issue_opm_bwd(pipe.ms, pipe.opm, S, N, mmask, dmsa);
      pipe.opm.on = false;
    }
    stream_wait(st, pipe.ms);
  };
  if (L.replay) {
    // each block's forward again from its kept inputs, into the one region,
    // then its backward (the recomputed carries are the same bits)
    const float* pin0 = reinterpret_cast<const float*>(sv + L.off_pair_in);
    const float* min0 = reinterpret_cast<const float*>(sv + L.off_msa_in);
    float* scr_p = reinterpret_cast<float*>(sv + L.off_scr);
    float* scr_m = L.pair_only ? nullptr : reinterpret_cast<float*>(sv + L.off_scr + L.pair_bytes);
    for (int b = depth - 1; b >= 0; --b) {
      {
        KTimed kt("stack.replay", st);
        block_fwd(st, w.blocks[b], L, b, t,
                  frame(L, sv, b, b == 0 ? pin0 : nullptr, b == 0 ? min0 : nullptr, scr_p, scr_m),
                  pmask, mmask, sv);
      }
      Frame f = frame(L, sv, b, b == 0 ? pin0 : nullptr, b == 0 ? min0 : nullptr, nullptr, nullptr);
      block_bwd(st, w.blocks[b], L, b, t, f, pmask, mmask, sv, dp(b + 1), dp(b), dmsa, &pipe);
    }
    finish();
    return;
  }
  for (int b = depth - 1; b >= 0; --b)
    block_bwd(st, w.blocks[b], L, b, t, frame(L, sv, b, nullptr, nullptr, nullptr, nullptr),
              pmask, mmask, sv + (size_t)b * L.block_bytes, dp(b + 1), dp(b), dmsa, &pipe);
  finish();
}

int set_save_policy(int p) {
  if (p < 0 || p > 2) return -1;
  const int old = g_save_policy;
  g_save_policy = p;
  return old;
}

bool stack_replays(const StackW& w, int N, int S, int depth) {
  stack_check(w, N, S, depth);
  return layout(w, N, S, depth).replay;
}

}  // namespace bc2n
