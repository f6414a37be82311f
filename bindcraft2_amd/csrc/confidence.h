// Confidence metrics of one prediction from the head logits: pLDDT, the
// symmetrised PAE, pTM, ipTM with its per-residue vector, and the
// experimentally-resolved CA probability; forward and backward.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace bc2n {

constexpr int CONF_LBINS = 50;  // predicted_lddt bins
constexpr int CONF_PBINS = 64;  // predicted_aligned_error bins
constexpr int CONF_EXPRES = 37;

// Bytes of the buffer the forward fills and the backward reads.
size_t confidence_save_bytes(int N);

// plddt_logits [N][50], pae_logits [N][N][64], expres_logits [N][37],
// seq_mask [N], asym [N] (interface chain ids) -> plddt [N], pae [N][N],
// ptm [1], iptm [1], iptm_pr [N], expres_ca [N].
void confidence_fwd(hipStream_t st, const float* lddt_l, const float* pae_l, const float* expres_l,
                    const float* seq_mask, const int32_t* asym, int N, float* plddt, float* pae,
                    float* ptm, float* iptm, float* iptm_pr, float* expres_ca, void* save);
// Cotangents may be null (zero); g_ptm and g_iptm are device scalars.
void confidence_bwd(hipStream_t st, const float* lddt_l, const float* pae_l, const float* expres_l,
                    const float* seq_mask, const int32_t* asym, int N, const void* save,
                    const float* g_plddt, const float* g_pae, const float* g_ptm,
                    const float* g_iptm, const float* g_iptm_pr, const float* g_expres,
                    float* d_lddt, float* d_pae, float* d_expres);

}  // namespace bc2n
