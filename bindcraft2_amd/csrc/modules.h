// Trunk modules: AF2 layers as sequences of gfx950 kernels.  Each module has
// a forward that writes `pair_out = pair_in + dropout(module(pair_in))` and
// fills a caller-owned save-set, and a backward that consumes the save-set
// and adds the module's input cotangent to the residual cotangent.  Scratch
// comes from the process arena; nothing is allocated inside a call once the
// arena has grown to the call's plan.
//
// Every backward takes `sc`, the device pair {s, 1/s} of its cotangent scale
// (ct_scale in kernels.h): its incoming cotangent is multiplied by s where it
// is first rounded to binary16, and 1/s is applied in the f32 epilogue that
// writes the module's input cotangent.  A caller running many modules on one
// cotangent (the stack, per block) computes it once; sc = nullptr makes the
// module compute its own from its incoming cotangent.
#pragma once
#include "runtime.h"
#include "kernels.h"

namespace bc2n {

// The scale a backward uses: the caller's, or one computed now from the n
// floats of the module's incoming cotangent into the module slot.
inline const float* module_scale(hipStream_t st, const float* sc, const float* dout, long n) {
  if (sc) return sc;
  float* s = ct_scale_slot(0);
  ct_scale(st, dout, n, s);
  return s;
}

// ---------------------------------------------------------- triangle attention
// modules.py TriangleAttention (+ Attention with pair bias and gating).
struct TriAttnW {
  int C = 0, H = 0, D = 0;
  const float *ln_g = nullptr, *ln_b = nullptr, *w2d = nullptr;  // w2d [C][H]
  const float* bqkvg = nullptr;  // [4HD]: zeros for q,k,v; gating_b for g
  const h16* wqkvg_t = nullptr; // [4HD][C]
  const h16* wqkvg_frag = nullptr;  // C = 128: wqkvg_t in b_frags_k128 order
  const h16* wo_frag = nullptr;     // C = HD = 128: wo_t in b_frags_k128 order
  const h16* wqkvg = nullptr;   // [C][4HD]
  const h16* wo_t = nullptr;    // [C][HD]
  const h16* wo = nullptr;      // [HD][C]
  const float* bo = nullptr;     // [C]
};
TriAttnW triattn_weights(WeightStore& ws, const std::string& prefix);

size_t triattn_save_bytes(int N, int C, int H);
// per_column = "ending node" (the module runs on the transposed pair).
void triattn_fwd(hipStream_t st, const TriAttnW& w, bool per_column, int N,
                 const float* pair_in, const float* mask, const float* tbl,
                 float* pair_out, void* save);
// triattn_fwd without any allocation: its scratch is a static device array
// of TRIATTN_NOALLOC_SCRATCH_BYTES (N <= 256 at C = 128); larger N throw
// std::invalid_argument before any launch.  Calls overlapping on one GPU race.
constexpr size_t TRIATTN_NOALLOC_SCRATCH_BYTES = 2ull * 256 * 256 * 128 * 2;
void triattn_fwd_noalloc(hipStream_t st, const TriAttnW& w, bool per_column, int N,
                         const float* pair_in, const float* mask, const float* tbl,
                         float* pair_out, void* save);
void triattn_bwd(hipStream_t st, const TriAttnW& w, bool per_column, int N,
                 const float* pair_in, const float* mask, const float* tbl,
                 const void* save, const float* dout, float* din, const float* sc = nullptr);

// ------------------------------------------------------ triangle multiplication
// modules.py:1044-1088 (fused projection weights).
struct TriMulW {
  int C = 0, I = 0;
  const float *ln_g = nullptr, *ln_b = nullptr, *cn_g = nullptr, *cn_b = nullptr;
  const float *bp = nullptr, *bg = nullptr, *bgl = nullptr, *bo = nullptr;
  const h16* wcat = nullptr;    // [C][4I+C]  (GEMM column order)
  const h16* wcat_t = nullptr;  // [4I+C][C]
  const h16* wcat_frag = nullptr;  // C = 128: wcat_t in b_frags_k128 order
  const h16* wo_frag = nullptr;    // C = I = 128: wo_t in b_frags_k128 order
  // the same two matrices with k permuted within each 32-block (tail_kperm):
  // the backward tail reads a lane's 8 MFMA k-slots as one 16-byte LDS read
  const h16* wcat_k = nullptr;
  const h16* wcat_tk = nullptr;
  const h16* wo = nullptr;      // [I][C]
  const h16* wo_t = nullptr;    // [C][I]
};
TriMulW trimul_weights(WeightStore& ws, const std::string& prefix);
size_t trimul_save_bytes(int N, int C, int I);
void trimul_fwd(hipStream_t st, const TriMulW& w, bool outgoing, int N, const float* pair_in,
                const float* mask, const float* tbl, float* pair_out, void* save);
void trimul_bwd(hipStream_t st, const TriMulW& w, bool outgoing, int N, const float* pair_in,
                const float* mask, const float* tbl, const void* save, const float* dout,
                float* din, const float* sc = nullptr);

// ----------------------------------------------------------------- transition
// modules.py:252-305; pair (rows = N*N) and MSA (rows = S*N) alike.  `nt` is
// the residue count: the shared dropout table row of act row m is m % nt.
struct TransW {
  int C = 0, F = 0;
  const float *ln_g = nullptr, *ln_b = nullptr, *b1 = nullptr, *b2 = nullptr;
  const h16 *w1 = nullptr, *w1_t = nullptr, *w2 = nullptr, *w2_t = nullptr;
  // C = 128, F = 4: both products' B operands in MFMA fragment order, per
  // direction (forward W1^T / W2^T, backward W2 / W1)
  const h16 *frag1_f = nullptr, *frag2_f = nullptr, *frag1_b = nullptr, *frag2_b = nullptr;
};
TransW transition_weights(WeightStore& ws, const std::string& prefix);
size_t transition_save_bytes(long rows, int C, int F);
void transition_fwd(hipStream_t st, const TransW& w, long rows, int nt, const float* act_in,
                    const float* tbl, float* act_out, void* save);
void transition_bwd(hipStream_t st, const TransW& w, long rows, int nt, const float* act_in,
                    const float* tbl, const void* save, const float* dout, float* din,
                    const float* sc = nullptr);

// ------------------------------------------------------------- MSA attention
struct AttnW {
  int Cin = 0, Cout = 0, H = 0, D = 0;
  const float *ln_g = nullptr, *ln_b = nullptr, *bqkvg = nullptr, *bo = nullptr;
  const h16 *wqkvg = nullptr, *wqkvg_t = nullptr, *wo = nullptr, *wo_t = nullptr;
};
struct MsaRowW {
  AttnW a;
  int Cz = 0;
  const float *pn_g = nullptr, *pn_b = nullptr, *w2d = nullptr;
  // the bias projection with the pair LayerNorm folded in (Cz = 128)
  const h16* pb_frag = nullptr;
  const float* pb_const = nullptr;
  const float* pb_bwd_frag = nullptr;
};
struct MsaColW {
  AttnW a;
};
MsaRowW msarow_weights(WeightStore& ws, const std::string& prefix);
MsaColW msacol_weights(WeightStore& ws, const std::string& prefix);
size_t msarow_save_bytes(int S, int N, int Cm, int H);
size_t msacol_save_bytes(int S, int N, int Cm, int H);
void msarow_fwd(hipStream_t st, const MsaRowW& w, int S, int N, const float* msa_in,
                const float* msa_mask, const float* pair, const float* tbl, float* msa_out,
                void* save);
// dpair is accumulated (+=), dmsa_in = dmsa_out + J^T(...)
// With amax_part (room for CT_FUSED floats, the calling lane's
// ct_fused_parts()): also the partial maxima of the final dpair for
// ct_scale_parts; returns their count (0: none written).
long msarow_bwd(hipStream_t st, const MsaRowW& w, int S, int N, const float* msa_in,
                const float* msa_mask, const float* pair, const float* tbl, const void* save,
                const float* dmsa_out, float* dmsa_in, float* dpair, const float* sc = nullptr,
                float* amax_part = nullptr);
// msarow_bwd in two halves: everything but the pair term (returns the pair
// bias gradient [H][N][N], in the calling lane's arena until its next call;
// sc required), then dpair += the pair LayerNorm's backward of it.
const float* msarow_bwd_msa(hipStream_t st, const MsaRowW& w, int S, int N, const float* msa_in,
                            const float* msa_mask, const float* tbl, const void* save,
                            const float* dmsa_out, float* dmsa_in, const float* sc);
long msarow_bwd_pair(hipStream_t st, const MsaRowW& w, int S, int N, const float* pair,
                     const void* save, const float* dbias, float* dpair, const float* sc,
                     float* amax_part = nullptr);
void msacol_fwd(hipStream_t st, const MsaColW& w, int S, int N, const float* msa_in,
                const float* msa_mask, const float* tbl, float* msa_out, void* save);
void msacol_bwd(hipStream_t st, const MsaColW& w, int S, int N, const float* msa_in,
                const float* msa_mask, const float* tbl, const void* save,
                const float* dmsa_out, float* dmsa_in, const float* sc = nullptr);

// ---------------------------------------------- MSA column global attention
struct MsaGlobW {
  int C = 0, H = 0, DK = 0, DV = 0;
  const float *ln_g = nullptr, *ln_b = nullptr, *wq = nullptr, *wcat = nullptr, *bcat = nullptr;
  const float *wo = nullptr, *bo = nullptr;
};
MsaGlobW msaglobal_weights(WeightStore& ws, const std::string& prefix);
size_t msaglobal_save_bytes(const MsaGlobW& w, int S, int N);
void msaglobal_fwd(hipStream_t st, const MsaGlobW& w, int S, int N, const float* msa_in,
                   const float* msa_mask, const float* tbl, float* msa_out, void* save);
void msaglobal_bwd(hipStream_t st, const MsaGlobW& w, int S, int N, const float* msa_in,
                   const float* msa_mask, const float* tbl, const void* save,
                   const float* dmsa_out, float* dmsa_in);

// --------------------------------------------------------- outer product mean
struct OpmW {
  int Cm = 0, O = 0, C = 0;
  const float *ln_g = nullptr, *ln_b = nullptr, *blr = nullptr, *bo = nullptr;
  const h16 *wlr = nullptr, *wlr_t = nullptr, *wt = nullptr, *wt2 = nullptr;
};
OpmW opm_weights(WeightStore& ws, const std::string& prefix);
size_t opm_save_bytes(int S, int N, int O, int C);
void opm_fwd(hipStream_t st, const OpmW& w, int S, int N, const float* msa, const float* msa_mask,
             const float* pair_in, const float* tbl, float* pair_out, void* save);
// opm_fwd in two halves: the MSA one (LayerNorm, mask norm, left / right
// projections into the save-set; reads no pair) and the pair one (the outer
// product of the saved projections added to the pair).
void opm_fwd_msa(hipStream_t st, const OpmW& w, int S, int N, const float* msa,
                 const float* msa_mask, void* save);
void opm_fwd_pair(hipStream_t st, const OpmW& w, int S, int N, const float* pair_in,
                  const float* tbl, float* pair_out, void* save);
// dmsa_in = dmsa_out + J^T(tbl * dpair)
void opm_bwd(hipStream_t st, const OpmW& w, int S, int N, const float* msa, const float* msa_mask,
             const float* tbl, const void* save, const float* dpair, const float* dmsa_out,
             float* dmsa_in, const float* sc = nullptr);

// ------------------------------------------- structure module fold iterations
// Weights of generate_monomer_rigids + FoldIteration (without the sidechain),
// all f32 (folding_multimer.py:188-548); the iterations share one set.
struct FoldW {
  const float *ln_s_g = nullptr, *ln_s_b = nullptr, *wi = nullptr, *bi = nullptr;
  const float *ln_z_g = nullptr, *ln_z_b = nullptr;
  const float *wcat = nullptr, *bcat = nullptr;  // six projections [384][1152]
  const float *w2d = nullptr, *b2d = nullptr, *wo = nullptr, *bo = nullptr, *pw = nullptr;
  const float *ln1_g = nullptr, *ln1_b = nullptr, *ln2_g = nullptr, *ln2_b = nullptr;
  const float *wt[3] = {nullptr, nullptr, nullptr}, *bt[3] = {nullptr, nullptr, nullptr};
  const float *wq = nullptr, *bq = nullptr;
};
FoldW fold_weights(WeightStore& ws);
size_t fold_save_bytes(int N, int depth);
// act_out [N][384]; traj [depth][N][3][4] = [R | 20 t] after each iteration.
// init_pos37 (atom37 [N][37][3]) or null: the first frames are those of its
// N, CA, C atoms instead of the identity (the model's initial_atom_pos).
void fold_fwd(hipStream_t st, const FoldW& w, int N, int depth, const float* single,
              const float* pair, const float* mask, const uint32_t* key, const uint32_t* enabled,
              bool dropout, float* act_out, float* traj, void* save,
              const float* init_pos37 = nullptr);
// d_act / d_traj may be null (zero cotangent)
void fold_bwd(hipStream_t st, const FoldW& w, int N, int depth, const float* single,
              const float* pair, const float* mask, bool dropout, const void* save,
              const float* d_act, const float* d_traj, float* dsingle, float* dpair);

}  // namespace bc2n
