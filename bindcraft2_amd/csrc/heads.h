// The post-trunk step around the fold iterations: the last iteration's
// sidechain (torsions -> rigid-group frames -> atom14 positions) and the four
// heads, forward and backward, f32.
#pragma once
#include "modules.h"

namespace bc2n {

// MultiRigidSidechain under fold_iteration/rigid_sidechain/ (128 channels,
// two residual blocks, 7 torsions).
struct SideW {
  const float *wi0 = nullptr, *bi0 = nullptr, *wi1 = nullptr, *bi1 = nullptr;
  const float *wr1[2] = {nullptr, nullptr}, *br1[2] = {nullptr, nullptr};
  const float *wr2[2] = {nullptr, nullptr}, *br2[2] = {nullptr, nullptr};
  const float *wa = nullptr, *ba = nullptr;
};
// distogram (half_logits), predicted aligned error, pLDDT, experimentally resolved
struct HeadsW {
  const float *wdg = nullptr, *bdg = nullptr, *wpae = nullptr, *bpae = nullptr;
  const float *ln_g = nullptr, *ln_b = nullptr, *w0 = nullptr, *b0 = nullptr;
  const float *w1 = nullptr, *b1 = nullptr, *wl = nullptr, *bl = nullptr;
  const float *wer = nullptr, *ber = nullptr;
};
// residue tables (const/...): default frames [21][8][4][4], atom -> group
// [21][14], literature positions [21][14][3], atom mask [21][14]
struct ResTables {
  const float *frame = nullptr, *group = nullptr, *lit = nullptr, *mask = nullptr;
};
struct StructHeadsW {
  FoldW fold;
  SideW sc;
  HeadsW hd;
  ResTables tab;
};

constexpr int SH_ATOMS = 14, SH_DGRAM = 64, SH_PAE = 64, SH_PLDDT = 50, SH_EXPRES = 37;

StructHeadsW structheads_weights(WeightStore& ws);
size_t structheads_save_bytes(int N, int depth);
// single [N][384], pair [N][N][128], mask [N], aatype [N] (f32 residue types,
// clamped to 0..20) -> atom14 [N][14][3], distogram [N][N][64], pae [N][N][64],
// plddt [N][50], expres [N][37]; key/enabled as for fold_fwd.
void structheads_fwd(hipStream_t st, const StructHeadsW& w, int N, int depth, const float* single,
                     const float* pair, const float* mask, const float* aatype,
                     const uint32_t* key, const uint32_t* enabled, bool dropout, float* atom14,
                     float* dgram, float* pae, float* plddt, float* expres, void* save,
                     const float* init_pos37 = nullptr);
// Cotangents may be null (zero) -> dsingle [N][384], dpair [N][N][128].
void structheads_bwd(hipStream_t st, const StructHeadsW& w, int N, int depth, const float* single,
                     const float* pair, const float* mask, const float* aatype, bool dropout,
                     const void* save, const float* datom, const float* ddgram, const float* dpae,
                     const float* dplddt, const float* dexpres, float* dsingle, float* dpair);

}  // namespace bc2n
