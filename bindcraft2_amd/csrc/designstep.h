// The trunk of one design step in one call: embedder, template embedding,
// extra-MSA stack (pair only), main stack, single projection, structure
// module and heads, forward and backward to the input features.
#pragma once
#include "embed.h"
#include "heads.h"
#include "confidence.h"
#include "seqfeat.h"
#include "tplembed.h"

namespace bc2n {

// The embedder's three recycle terms (modules_multimer.py:487-507).
struct RecycleW {
  const float *wpp = nullptr, *bpp = nullptr;      // prev_pos_linear [15][128], [128]
  const float *s_msa = nullptr, *o_msa = nullptr;  // prev_msa_first_row_norm [256]
  const float *s_pair = nullptr, *o_pair = nullptr;  // prev_pair_norm [128]
};

// The template's MSA row (modules_multimer.py:1080-1137): Linears from the
// embedder's directory, chi tables (const/chi_atom_indices [21][4][4],
// const/chi_angles_mask [21][4]) from the structure module's; null if absent.
struct TplRowW {
  const float *w1 = nullptr, *b1 = nullptr;  // template_single_embedding [34][256], [256]
  const float *w2 = nullptr, *b2 = nullptr;  // template_projection [256][256], [256]
  const float *chi_idx = nullptr, *chi_mask = nullptr;
  bool ok() const { return w1 && b1 && w2 && b2 && chi_idx && chi_mask; }
};

struct DesignStepW {
  EmbedW emb;
  RecycleW rec;
  TplRowW trow;
  const float *wsa = nullptr, *bsa = nullptr;  // single_activations [256][384], [384]
  TplEmbedW tpl;
  StackW extra, main;
  StructHeadsW sh;
  // the atom37 gather (residx_atom37_to_atom14, atom37_mask [21][37]); null
  // when the structure module's directory holds no such tables
  const float *a37_14 = nullptr, *a37_mask = nullptr;
  int d_tpl = 0, d_extra = 0, d_main = 0, d_fold = 0;
};

// pair [N][N][128] += the pair recycle term, msa0 [N][256] += the msa[0] term,
// of the previous pass's atoms (atom14 [N][14][3], pseudo-beta by aatype),
// pair and msa[0]; prev_atom14 null = the first pass (a zero state).
void recycle_terms(hipStream_t st, const RecycleW& r, int N, const float* aatype,
                   const float* prev_atom14, const float* prev_pair, const float* prev_msa0,
                   float* pair, float* msa0);

// Every pass adds the embedder's recycle terms of the previous pass's atoms,
// pair and msa[0] (all zero before the first).  `recycles` forward-only
// passes run before the differentiated one (bindcraft/af2.py:195-202); the
// outputs are the last pass's.  Seeds: u32[recycles + 1][4][3] on the
// device, per pass one (k0, k1, enabled) JAX key per stack in the order
// template, extra, main, structure module.
size_t design_step_save_bytes(const DesignStepW& w, int N, int S);
void design_step_fwd(hipStream_t st, const DesignStepW& w, int N, int S, const float* tf,
                     const float* mf, const float* ri, const float* ai, const float* ei,
                     const float* si, const int32_t* offset, const float* seq_mask,
                     const float* act_const, const float* aatype, const uint32_t* seeds,
                     bool dropout, int recycles, float* atom14, float* dgram, float* pae,
                     float* plddt, float* expres, void* save, const float* row = nullptr,
                     const float* row_mask = nullptr, const float* init_pos37 = nullptr);
// init_pos37 (atom37 [N][37][3]) or null: the structure module of the first
// pass starts from these atoms' frames (the model's initial_atom_pos), each
// later pass from the previous pass's atom37 positions (needs the atom37
// tables).
// row [N][256] / row_mask [N]: a constant MSA row appended after the
// embedder's S rows (the template's, modules_multimer.py:608-617); the main
// stack then runs S + 1 rows and `save` must hold design_step_save_bytes(S + 1).
// Cotangents may be null (zero) -> d target_feat [N][21], d msa_feat [S][N][49];
// `row` says whether the forward appended one.
void design_step_bwd(hipStream_t st, const DesignStepW& w, int N, int S, const float* tf,
                     const float* seq_mask, bool with_template, const float* aatype,
                     bool dropout, void* save, const float* datom, const float* ddgram,
                     const float* dpae, const float* dplddt, const float* dexpres, float* dtf,
                     float* dmf, bool row = false);

// The same step from the designed sequence logits [N][20] (one MSA row):
// sequence features and profile (seqfeat.h) -> target_feat, msa_feat and
// aatype -> the step above; the backward returns d logits.  `sc4` is the
// device buffer of the four design scalars (softmax_weight, one_hot_weight,
// temperature, logit_scale); `bias` [20] may be null.
// The confidence metrics of the step's head logits (confidence.h), computed
// when `plddt` is set; their cotangents join the logits' in the backward.
struct ConfOut {
  const int32_t* asym = nullptr;  // interface chain ids [N]
  float *plddt = nullptr, *pae = nullptr, *ptm = nullptr, *iptm = nullptr, *iptm_pr = nullptr,
        *expres_ca = nullptr;
};
struct ConfCt {
  const int32_t* asym = nullptr;
  const float *plddt = nullptr, *pae = nullptr, *ptm = nullptr, *iptm = nullptr,
              *iptm_pr = nullptr, *expres_ca = nullptr;
  bool any() const { return plddt || pae || ptm || iptm || iptm_pr || expres_ca; }
};
// The reference step's atoms (native/design_step.cuh:77-80, 1162-1168): the
// atom14 prediction gathered to atom37 (times restype_atom37_mask[aatype] *
// seq_mask) and, given the template's atoms, superposed on them by a Kabsch
// of the CA atoms of the TEMPLATE-and-not-DESIGN residues (flags bits 1, 0;
// bindcraft/af2.py:89-97, bindcraft/protein.py:75-83).  Its cotangent joins
// the atom14 one in the backward (the rotation is under stop_gradient).
struct AtomsOut {
  const float* tpl37 = nullptr;   // template atoms [N][37][3], or null (no alignment)
  const float* tplm37 = nullptr;  // their mask [N][37]
  float* atom37 = nullptr;        // [N][37][3], or null (no atom37 output)
  float* mask37 = nullptr;        // [N][37]
};
size_t design_step_seq_save_bytes(const DesignStepW& w, int N);
// nlen: the runtime length on the device (rows >= *nlen are padding), or
// null for all N rows.
void design_step_seq_fwd(hipStream_t st, const DesignStepW& w, int N, const int32_t* nlen,
                         const float* logits, const uint8_t* flags, const float* bias, const float* sc4,
                         float omitted_half, const float* ri, const float* ai, const float* ei,
                         const float* si, const int32_t* offset, const float* seq_mask,
                         const float* act_const, const uint32_t* seeds, bool dropout,
                         int recycles, int cyclic_mode, float flexibility, float* atom14, float* dgram, float* pae, float* plddt,
                         float* expres, const AtomsOut& atoms, const ConfOut& conf, void* save);
void design_step_seq_bwd(hipStream_t st, const DesignStepW& w, int N, const int32_t* nlen,
                         const float* logits, const uint8_t* flags, const float* bias, const float* sc4,
                         float omitted_half, const float* seq_mask, bool with_template,
                         bool dropout, void* save, const float* datom, const float* ddgram,
                         const float* dpae, const float* dplddt, const float* dexpres,
                         const float* datom37, const ConfCt& conf, float* d_logits);

}  // namespace bc2n
