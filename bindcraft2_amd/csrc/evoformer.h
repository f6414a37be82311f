// Evoformer block / stack (host orchestration over the module kernels).
#pragma once
#include "modules.h"
#include <vector>

namespace bc2n {

struct BlockW {
  OpmW opm;
  MsaRowW row;
  MsaColW col;
  TransW mtr;
  TriMulW tmo, tmi;
  TriAttnW tas, tae;
  TransW ptr;
  const float* opm_b = nullptr;  // outer_product_mean/output_b (pair_only constant)
};

// EVO: full Evoformer blocks.  PAIR_ONLY: the extra-MSA specialisation
// (OPM constant + pair modules).  TEMPLATE: TemplateEmbeddingIteration
// (modules_multimer.py:1008-1077: tmo, tmi, tas, tae, transition).
enum class StackKind { EVO, PAIR_ONLY, TEMPLATE };

struct StackW {
  StackKind kind = StackKind::EVO;
  bool pair_only = false;  // no MSA track (PAIR_ONLY or TEMPLATE)
  std::vector<BlockW> blocks;
};

BlockW block_weights(WeightStore& ws, const std::string& prefix, StackKind kind);
// Blocks param/block0 .. param/block{depth-1} of a weights directory.
StackW stack_weights(WeightStore& ws, int depth, StackKind kind,
                     const std::string& root = "param/");

// Bytes of the save-set a forward with these shapes writes and the backward
// reads: every block's carries and module save-sets and the dropout tables,
// or, in the replay tier, every block's input carries and one block's module
// save-sets (the backward runs each block's forward again first).
size_t stack_save_bytes(const StackW& w, int N, int S, int depth);

// The save policy of every stack in the process: 0 = by size (the replay
// tier when the full save-set would take more than 60% of the device's
// memory), 1 = always full, 2 = always the replay tier.  Returns the
// previous policy (-1 for a bad value).  A forward and its backward must run
// under the same policy.
int set_save_policy(int policy);
// Whether a stack of these shapes keeps the replay tier under the policy.
bool stack_replays(const StackW& w, int N, int S, int depth);

// Bytes of a detached forward's scratch (detached = true below): one
// block's module save-sets, two carries of each track, the dropout tables.
size_t stack_detached_bytes(const StackW& w, int N, int S, int depth);

// Forward of `depth` blocks.  key = stack key (2 x u32, device), enabled =
// device u32 flag (may be null = on); dropout=false skips every mask.
// detached: no backward will follow (a recycling or inference pass); `save`
// is then stack_detached_bytes of scratch, reused block after block.
void stack_fwd(hipStream_t st, const StackW& w, int N, int S, int depth, const float* pair,
               const float* msa, const float* pmask, const float* mmask, const uint32_t* key,
               const uint32_t* enabled, bool dropout, float* pair_out, float* msa_out,
               void* save, bool detached = false);
// Backward: cotangents of the stack outputs in, of the stack inputs out.
// Everything else it needs (inputs, carries, dropout tables) is in `save`.
void stack_bwd(hipStream_t st, const StackW& w, int N, int S, int depth, const float* pmask,
               const float* mmask, bool dropout, const void* save, const float* ct_pair,
               const float* ct_msa, float* dpair, float* dmsa);

}  // namespace bc2n
