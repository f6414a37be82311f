/*
 * bc2n -- MI355X-native AlphaFold2 trunk for BindCraft2, C ABI.
 *
 * Every entry point is plain C: device pointers, sizes, an opaque HIP stream
 * (hipStream_t passed as void*; NULL = the null stream) and an int status
 * (0 = success; otherwise call bc2n_last_error() for the message).  Nothing
 * here exits the process.  All work of one call is enqueued on `stream`; no
 * call synchronises the host unless its scratch arena has to grow.
 *
 * Weights are not arguments: as in the reference, they come from a weights
 * directory (manifest.txt + raw little-endian f32 files, names
 * "param/block{b}/<module path>/<param>") loaded once per process.
 *
 * Calls are serialised by one process-wide lock and share one scratch arena
 * and one weight cache, so a process drives one GPU (the reference runs one
 * design worker process per GPU).  Calls may use different streams: each
 * call records an event on its stream after its last launch and a call on
 * another stream first waits for it, so calls run one after another as on
 * one stream (under graph capture only the capturing stream orders a call).
 * Calls from several host threads must not overlap.
 *
 * Lengths: N (residues) must be a multiple of 32 -- the reference's caller
 * pads to 32 outside the custom VJP (bindcraft/af/native.py:950-972).
 */
#ifndef BC2N_H
#define BC2N_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Message of the last failed call on this thread ("" if none). */
const char* bc2n_last_error(void);
/* ABI version of this library. */
int bc2n_abi_version(void);

/* ------------------------------------------------------------------------
 * Module entry points: one AF2 layer wrapped in dropout_wrapper
 * (reference: bindcraft/af/alphafold/model/modules.py:46-76), i.e.
 *     pair_out = pair + drop_tbl * module(pair)
 * and its VJP
 *     dpair_in = dpair_out + J^T (drop_tbl * dpair_out).
 * `prefix` names the module inside the weights directory, e.g.
 * "param/block0/triangle_attention_starting_node/".  `drop_tbl` is the
 * shared-dropout scale table [N][C] (1/keep or 0; see bc2n_dropout_table) or
 * NULL for no dropout.  `save` is a caller-owned device buffer of
 * bc2n_*_save_bytes() bytes written by the forward and read by the backward.
 * pair_out must not alias pair (the backward reads the module input);
 * dpair_in may alias dpair_out.
 * ---------------------------------------------------------------------- */

/* Triangle attention, starting node (per_column=0) or ending node
 * (per_column=1).  pair f32 [N,N,C], pair_mask f32 [N,N] (binary).
 * Replaces native/triattn_body.cuh TriAttn::forward (:1090) / backward
 * (:1228); semantics of modules.py:675-734. */
size_t bc2n_triattn_save_bytes(int N, int C, int H);
int bc2n_triattn_fwd(void* stream, const char* weights_dir, const char* prefix,
                     int per_column, int N, const float* pair,
                     const float* pair_mask, const float* drop_tbl,
                     float* pair_out, void* save);
int bc2n_triattn_bwd(void* stream, const char* weights_dir, const char* prefix,
                     int per_column, int N, const float* pair,
                     const float* pair_mask, const float* drop_tbl,
                     const void* save, const float* dpair_out, float* dpair_in);
/* bc2n_triattn_fwd that allocates nothing.  No counterpart in the reference:
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * operands and results as bc2n_triattn_fwd (bit for bit); its scratch is a
 * static 32 MiB device array per GPU, so N <= 256 at C = 128 (a larger N
 * returns an error before any launch).  The weights must already be
 * resident: call bc2n_triattn_fwd once with the same weights_dir/prefix
 * first, else an error is returned.  Calls that overlap on one GPU share
 * the array and race; serialise them (one stream). */
int bc2n_triattn_fwd_noalloc(void* stream, const char* weights_dir, const char* prefix,
                             int per_column, int N, const float* pair,
                             const float* pair_mask, const float* drop_tbl,
                             float* pair_out, void* save);

/* Triangle multiplication, outgoing (outgoing=1, 'ikc,jkc->ijc') or incoming
 * (outgoing=0, 'kjc,kic->ijc'), AF2's fused-projection form with
 * fast-variance LayerNorms.  pair f32 [N,N,C]; pair_out must not alias pair.
 * Replaces native/trimul_body.cuh TriMul::forward (:1572) / backward
 * (:1680); semantics of modules.py:1044-1088. */
size_t bc2n_trimul_save_bytes(int N, int C, int I);
int bc2n_trimul_fwd(void* stream, const char* weights_dir, const char* prefix,
                    int outgoing, int N, const float* pair,
                    const float* pair_mask, const float* drop_tbl,
                    float* pair_out, void* save);
int bc2n_trimul_bwd(void* stream, const char* weights_dir, const char* prefix,
                    int outgoing, int N, const float* pair,
                    const float* pair_mask, const float* drop_tbl,
                    const void* save, const float* dpair_out, float* dpair_in);

/* Transition (pair or MSA): act f32 [B, N, C] as rows = B*N; the shared
 * dropout table row of act row m is m % N.  AF2 passes a mask it does not
 * use; none is taken here.  Replaces native/transition.cuh Trans::forward
 * (:569) / backward (:619); semantics of modules.py:252-305. */
size_t bc2n_transition_save_bytes(long rows, int C, int factor);
int bc2n_transition_fwd(void* stream, const char* weights_dir, const char* prefix,
                        long rows, int N, const float* act, const float* drop_tbl,
                        float* act_out, void* save);
int bc2n_transition_bwd(void* stream, const char* weights_dir, const char* prefix,
                        long rows, int N, const float* act, const float* drop_tbl,
                        const void* save, const float* dact_out, float* dact_in);

/* Outer product mean added into the pair: msa f32 [S,N,Cm], msa_mask f32
 * [S,N], pair f32 [N,N,C].  The backward returns the MSA cotangent:
 * dmsa_in = dmsa_out + J^T(drop_tbl * dpair) (the pair's own cotangent passes
 * through the residual unchanged).  Replaces native/opm.cuh Opm::forward
 * (:271) / backward (:293); semantics of modules.py:1128-1212. */
size_t bc2n_opm_save_bytes(int S, int N, int O, int C);
int bc2n_opm_fwd(void* stream, const char* weights_dir, const char* prefix, int S,
                 int N, const float* msa, const float* msa_mask, const float* pair,
                 const float* drop_tbl, float* pair_out, void* save);
int bc2n_opm_bwd(void* stream, const char* weights_dir, const char* prefix, int S,
                 int N, const float* msa, const float* msa_mask,
                 const float* drop_tbl, const void* save, const float* dpair,
                 const float* dmsa_out, float* dmsa_in);

/* MSA row attention with pair bias: msa [S,N,Cm], msa_mask [S,N], pair
 * [N,N,Cz].  The backward also accumulates (+=) the pair cotangent of the
 * bias path into dpair.  Replaces native/msarow.cuh MsaRow::forward (:363) /
 * backward (:385); semantics of modules.py:500-563. */
size_t bc2n_msarow_save_bytes(int S, int N, int Cm, int H);
int bc2n_msarow_fwd(void* stream, const char* weights_dir, const char* prefix,
                    int S, int N, const float* msa, const float* msa_mask,
                    const float* pair, const float* drop_tbl, float* msa_out,
                    void* save);
int bc2n_msarow_bwd(void* stream, const char* weights_dir, const char* prefix,
                    int S, int N, const float* msa, const float* msa_mask,
                    const float* pair, const float* drop_tbl, const void* save,
                    const float* dmsa_out, float* dmsa_in, float* dpair);

/* MSA column attention (S <= 32).  Replaces native/msacol.cuh
 * MsaCol (:247-361); semantics of modules.py:566-616. */
size_t bc2n_msacol_save_bytes(int S, int N, int Cm, int H);
int bc2n_msacol_fwd(void* stream, const char* weights_dir, const char* prefix,
                    int S, int N, const float* msa, const float* msa_mask,
                    const float* drop_tbl, float* msa_out, void* save);
int bc2n_msacol_bwd(void* stream, const char* weights_dir, const char* prefix,
                    int S, int N, const float* msa, const float* msa_mask,
                    const float* drop_tbl, const void* save,
                    const float* dmsa_out, float* dmsa_in);

/* MSA column global attention, f32 (the extra-MSA stack's column module;
 * modules.py:619-672 over GlobalAttention :403-497).  The reference runs it
 * in JAX only: its native extra stack is the pair-only specialisation
 * (native/block.cuh:79-91), so this has no native counterpart.  Widths from
 * the weights (attention/query_w [C, H, DK], value_w [C, DV]).  The save-set
 * size depends on the weights, hence weights_dir / prefix. */
size_t bc2n_msaglobal_save_bytes(const char* weights_dir, const char* prefix, int S, int N);
int bc2n_msaglobal_fwd(void* stream, const char* weights_dir, const char* prefix,
                       int S, int N, const float* msa, const float* msa_mask,
                       const float* drop_tbl, float* msa_out, void* save);
int bc2n_msaglobal_bwd(void* stream, const char* weights_dir, const char* prefix,
                       int S, int N, const float* msa, const float* msa_mask,
                       const float* drop_tbl, const void* save,
                       const float* dmsa_out, float* dmsa_in);

/* ------------------------------------------------------------------------
 * The Evoformer stack: the drop-in for the reference's XLA FFI pair
 * NativeEvoformerFwd / NativeEvoformerBwd (native/ffi.cu:942-982, impl
 * FwdImpl :183-331, BwdImpl :333-371), same operands and attributes:
 *   fwd(pair f32[N,N,128], msa f32[S,N,Cm], pair_mask f32[N,N],
 *       msa_mask f32[S,N], seed u32[seed_len]; depth, save, pair_only,
 *       own_save, opm_first, dropout, weights_dir)
 *     -> (pair_out, msa_out, psave, msave)
 *   bwd(ct_pair, ct_msa, pair_mask, msa_mask, psave, msave, seed; depth,
 *       pair_only, own_save, opm_first, dropout, weights_dir) -> (dpair, dmsa)
 * Shapes cross as N, S, Cm.  psave is one opaque byte buffer of
 * bc2n_evoformer_save_bytes() (every block's carries and module save-sets:
 * the backward replays nothing); msave is accepted and unused (may be NULL).
 * save=0 is a detached forward (no backward follows: a recycling or
 * inference pass): psave is not written (may be NULL) and the library uses
 * bc2n_evoformer_detached_bytes() of its own scratch, one block's worth
 * reused block after block.  own_save=1 uses a library-owned save-set.
 * seed: seed_len=3 -> [k0, k1, enabled] with (k0,k1) = key_data of the
 * stack's JAX key: dropout masks are bit-identical to jax.random.bernoulli
 * through AF2's key chain.  seed_len=2 -> the reference's [bits, enabled]
 * operand (modules_multimer.py:660-667), taken as PRNGKey(bits).
 * opm_first must be 1 (AF2-multimer, config.py:414).  pair_only=1 is the
 * reference's extra-MSA specialisation (MSA mask all zero: OPM adds
 * output_b/1e-3, the MSA modules are skipped, msa passes through).
 * ---------------------------------------------------------------------- */
size_t bc2n_evoformer_save_bytes(const char* weights_dir, int N, int S,
                                 int64_t depth, int64_t pair_only);
/* Scratch bytes of a detached (save=0) forward: one block's module
 * save-sets, two carries of each track and the dropout tables. */
size_t bc2n_evoformer_detached_bytes(const char* weights_dir, int N, int S,
                                     int64_t depth, int64_t pair_only);
/* The save-set tier of every stack in the process (the evoformer and
 * template stacks here, and those inside the template embedding and the
 * design step): 0 = by size (the default: the full save-set, whose backward
 * replays nothing, unless it would take more than 60% of the device's
 * memory -- e.g. the 48-block stack beyond L ~ 600 on a 288 GB MI355X --
 * then the replay tier), 1 = always full, 2 = always the replay tier: every
 * block's input carries and one block's module save-sets, the backward
 * running each block's forward again before its backward (the reference's
 * replay/remat tiers, native/stack.cuh:775-798, priced the same way: about
 * one more forward).  The *_save_bytes functions, forwards and backwards
 * all follow it, so a forward and its backward must see the same policy.
 * Returns the previous policy, or -1 for a bad value. */
int bc2n_set_save_policy(int policy);
/* Process-wide: whether the Evoformer stacks run the MSA side of each block
 * (forward: row and column attention, the MSA transition and the next
 * block's outer-product-mean MSA half; backward: the transition, column
 * attention, row attention up to its bias gradient and the outer product
 * mean) on a library-owned second stream (non-blocking, default priority)
 * beside the pair track, ordered by events and joined back to the caller's
 * stream before the call returns (1, the default), or everything on the
 * caller's stream (0).  Results are bit-identical either way.  No reference
 * counterpart (the reference's trunk is single-stream).  Returns the
 * previous setting. */
int bc2n_set_msa_overlap(int on);
/* 1 if a stack of these shapes keeps the replay tier under the policy, 0 if
 * the full save-set, -1 on error. */
int bc2n_evoformer_replays(const char* weights_dir, int N, int S, int64_t depth,
                           int64_t pair_only);
/* The number of bf16 [N,N,128] slots that hold the save-set, for a caller
 * that declares psave in the reference's shape bf16[slots,N,N,128]
 * (replaces native_save_slots_probe(depth, n), native/ffi.cu:1684-1689,
 * whose Python twin is _save_slots, bindcraft/af/native.py:1250-1272; the
 * save-set here also depends on the widths in weights_dir, S and pair_only).
 * -1 on error. */
int bc2n_save_slots_probe(const char* weights_dir, int depth, int N, int S,
                          int pair_only);
/* Preallocation before the first call (the reference calls these at trace
 * time, before XLA allocates): upload the weights and grow every scratch
 * buffer the component's calls at these shapes use (and, for the stack, its
 * detached-forward scratch), so that no later call at these shapes
 * allocates.  0 on success; prints what it took to stderr.  Replace
 * native_stack_prealloc, native_tplstack_prealloc, native_sm_prealloc and
 * native_tplembed_prealloc (native/ffi.cu:835-937; callers
 * bindcraft/af/native.py:1279-1407), same signatures. */
int bc2n_stack_prealloc(int N, int S, int depth, const char* weights_dir, int pair_only,
                        int opm_first, int dropout);
int bc2n_tplstack_prealloc(int N, int depth, const char* weights_dir);
int bc2n_sm_prealloc(int N, int depth, const char* weights_dir);
int bc2n_tplembed_prealloc(int N, int depth, const char* weights_dir);
int bc2n_evoformer_fwd(void* stream, const float* pair, const float* msa,
                       const float* pair_mask, const float* msa_mask,
                       const uint32_t* seed, int seed_len, int N, int S, int Cm,
                       int64_t depth, int64_t save, int64_t pair_only,
                       int64_t own_save, int64_t opm_first, int64_t dropout,
                       const char* weights_dir, float* pair_out, float* msa_out,
                       void* psave, void* msave);
int bc2n_evoformer_bwd(void* stream, const float* ct_pair, const float* ct_msa,
                       const float* pair_mask, const float* msa_mask,
                       const void* psave, const void* msave,
                       const uint32_t* seed, int seed_len, int N, int S, int Cm,
                       int64_t depth, int64_t pair_only, int64_t own_save,
                       int64_t opm_first, int64_t dropout,
                       const char* weights_dir, float* dpair, float* dmsa);

/* ------------------------------------------------------------------------
 * The template pair stack: the drop-in for TemplatePairStackFwd / Bwd
 * (native/ffi.cu:983-1008, impl TplFwdImpl :403-430, TplBwdImpl :432-456):
 *   fwd(pair f32[N,N,64], pair_mask f32[N,N], seed; depth, dropout,
 *       weights_dir) -> (out f32[N,N,64], save)
 *   bwd(ct f32[N,N,64], pair_mask, save, seed; ...) -> dpair
 * Blocks are TemplateEmbeddingIteration (modules_multimer.py:1008-1077:
 * tmo, tmi, tas, tae at C=64 with 4 heads of 16, transition x2), dropout
 * keys split(sub, 20)[1..5].  save holds bc2n_tplstack_save_bytes() bytes;
 * seed as for the Evoformer stack.
 * ---------------------------------------------------------------------- */
size_t bc2n_tplstack_save_bytes(const char* weights_dir, int N, int64_t depth);
int bc2n_tplstack_fwd(void* stream, const float* pair, const float* pair_mask,
                      const uint32_t* seed, int seed_len, int N, int64_t depth,
                      int64_t dropout, const char* weights_dir, float* out,
                      void* save);
int bc2n_tplstack_bwd(void* stream, const float* ct, const float* pair_mask,
                      const void* save, const uint32_t* seed, int seed_len, int N,
                      int64_t depth, int64_t dropout, const char* weights_dir,
                      float* dpair);

/* ------------------------------------------------------------------------
 * Template embedding, one template (the reference's TemplateEmbeddingFwd /
 * TemplateEmbeddingBwd custom calls, native/ffi.cu:1072-1098 (handlers
 * TeFwdImpl / TeBwdImpl :766-803), called from bindcraft/af/native.py:
 * 1049-1128 for modules_multimer.py:704-1005).  Replaces:
 *   fwd(query f32[N,N,128], act_const f32[N,N,64], pair_mask f32[N,N],
 *       seed; depth, dropout, weights_dir) -> (out f32[N,N,128], save)
 *   bwd(ct f32[N,N,128], query, act_const, pair_mask, save, seed; ...)
 *       -> dquery f32[N,N,128]
 * act_const is the caller's sum of the eight constant template-feature
 * projections; out = output_linear(relu(output_layer_norm(stack(act_const +
 * template_pair_embedding_8(query_embedding_norm(query)))))).  The weights
 * directory holds param/query_embedding_norm, template_pair_embedding_8,
 * output_layer_norm, output_linear and the stack's param/block{b}/...
 * save holds bc2n_tplembed_save_bytes() bytes (the backward replays no
 * forward); seed as for the stacks.  act_const gets no gradient and is
 * accepted by the backward for the reference's operand list only.  out
 * (dquery) must not alias an input: it is used as staging before it is
 * written.
 * ---------------------------------------------------------------------- */
size_t bc2n_tplembed_save_bytes(const char* weights_dir, int N, int64_t depth);
int bc2n_tplembed_fwd(void* stream, const float* query, const float* act_const,
                      const float* pair_mask, const uint32_t* seed, int seed_len,
                      int N, int64_t depth, int64_t dropout,
                      const char* weights_dir, float* out, void* save);
int bc2n_tplembed_bwd(void* stream, const float* ct, const float* query,
                      const float* act_const, const float* pair_mask,
                      const void* save, const uint32_t* seed, int seed_len, int N,
                      int64_t depth, int64_t dropout, const char* weights_dir,
                      float* dquery);

/* ------------------------------------------------------------------------
 * Input embedder, multimer (the reference's EmbedderFwd / EmbedderBwd custom
 * calls, native/ffi.cu:1046-1071 (handlers EmbFwdImpl / EmbBwdImpl :682-729)
 * over native/embed.cuh:54-372, called from bindcraft/af/native.py:573-622
 * for modules_multimer.py:358-483).  Replaces:
 *   fwd(target_feat f32[N,21], msa_feat f32[S,N,49], residue_index f32[N],
 *       asym_id f32[N], entity_id f32[N], sym_id f32[N]; weights_dir)
 *       -> (msa f32[S,N,256], pair f32[N,N,128])
 *   bwd(dmsa f32[S,N,256], dpair f32[N,N,128], target_feat; weights_dir)
 *       -> (dtarget_feat f32[N,21], dmsa_feat f32[S,N,49])
 * target_feat is already padded to 21 columns.  msa = preprocess_1d(tf)
 * (zeroed on rows whose target_feat sums to zero) + preprocess_msa(msa_feat);
 * pair = left_single(tf)[:,None] + right_single(tf)[None] + the relative
 * encoding (max_relative_idx 32, max_relative_chain 2, chain-relative).
 * offset, i32[N,N] or NULL, is the optional batch['offset'] feature
 * (modules_multimer.py:384-388) that replaces residue_index[i] -
 * residue_index[j] when present.  No save-set; the id features get no
 * gradient.  Weights under param/{preprocess_1d, preprocess_msa,
 * left_single, right_single}/ and position_activations under param/ or
 * param/evoformer/~_relative_encoding/ (native.py:529-570).
 * ---------------------------------------------------------------------- */
int bc2n_embedder_fwd(void* stream, const float* target_feat, const float* msa_feat,
                      const float* residue_index, const float* asym_id,
                      const float* entity_id, const float* sym_id,
                      const int32_t* offset, int N, int S, const char* weights_dir,
                      float* msa, float* pair);
int bc2n_embedder_bwd(void* stream, const float* dmsa, const float* dpair,
                      const float* target_feat, int N, int S,
                      const char* weights_dir, float* dtarget_feat,
                      float* dmsa_feat);

/* ------------------------------------------------------------------------
 * Structure module fold iterations (the IPA step of the post-trunk
 * StructureHeadsFwd/Bwd handlers, native/ffi.cu:1009-1044, up to and
 * excluding the sidechain; native/foldit.cuh:141-440, ipa.cuh:507-842,
 * quatrigid.cuh:172-250).  Replaces:
 *   fwd(single f32[N,384], pair f32[N,N,128], seq_mask f32[N], seed; depth,
 *       dropout, weights_dir) -> (act f32[N,384], traj f32[depth,N,3,4], save)
 *   bwd(d_act, d_traj, single, pair, seq_mask, save; ...) -> (dsingle, dpair)
 * following folding_multimer.py:476-548 (generate_monomer_rigids without
 * initial_atom_pos): act = initial_projection(LN(single)), identity frames,
 * act_2d = LN(pair), then `depth` FoldIterations (:374-474) sharing one set
 * of weights, iteration i keyed by split(key, depth)[i] (dropout 0.1 with
 * keys split(k_i, 3)[1], [2]).  traj[i] = [R | 20 t] after iteration i
 * (StructureModule 'traj', position_scale 20).  All f32.  Weights in the
 * post-trunk manifest naming of bindcraft/af/native.py:339-444.  N <= 1024.
 * d_act / d_traj may be NULL (zero cotangent).  seed as for the stacks.
 * ---------------------------------------------------------------------- */
size_t bc2n_fold_save_bytes(const char* weights_dir, int N, int64_t depth);
int bc2n_fold_fwd(void* stream, const float* single, const float* pair,
                  const float* seq_mask, const uint32_t* seed, int seed_len, int N,
                  int64_t depth, int64_t dropout, const char* weights_dir,
                  float* act, float* traj, void* save);
int bc2n_fold_bwd(void* stream, const float* d_act, const float* d_traj,
                  const float* single, const float* pair, const float* seq_mask,
                  const void* save, int N, int64_t depth, int64_t dropout,
                  const char* weights_dir, float* dsingle, float* dpair);

/* ------------------------------------------------------------------------
 * Structure module and heads (the reference's StructureHeadsFwd /
 * StructureHeadsBwd custom calls, native/ffi.cu:1009-1044 (handlers
 * SmFwdImpl / SmBwdImpl :530-639) over native/structmod.cuh,
 * sidechain.cuh, atom14.cuh, heads.cuh; runner bindcraft/af/native.py
 * _make_post_runner).  Replaces:
 *   fwd(single f32[N,384], pair f32[N,N,128], seq_mask f32[N], aatype f32[N],
 *       seed; depth, weights_dir)
 *       -> (atom14 f32[N,14,3], distogram f32[N,N,64], pae f32[N,N,64],
 *           plddt f32[N,50], expres f32[N,37])
 *   bwd(single, pair, seq_mask, aatype, d_atom14, d_distogram, d_pae,
 *       d_plddt, d_expres, seed; ...) -> (dsingle, dpair)
 * = the fold iterations (as bc2n_fold_*), the last iteration's sidechain
 * (folding_multimer.py:950-1040: torsions, rigid-group frames, atom14
 * positions from the residue tables const/default_frame, atom14_to_group,
 * atom14_lit_pos, atom14_mask of the weights directory) and the distogram
 * (symmetrised), predicted-aligned-error, pLDDT and experimentally-resolved
 * heads (modules.py:777-1120).  All f32.  aatype holds residue types 0..20
 * (clamped).  save holds bc2n_structure_heads_save_bytes() bytes; unlike the
 * reference's, the backward replays nothing, and it uses the save buffer's
 * tail as scratch (so save is writable in both calls).  Cotangents may be
 * NULL (zero).  seed as for the stacks.  N <= 1024.
 * ---------------------------------------------------------------------- */
size_t bc2n_structure_heads_save_bytes(const char* weights_dir, int N, int64_t depth);
int bc2n_structure_heads_fwd(void* stream, const float* single, const float* pair,
                             const float* seq_mask, const float* aatype,
                             const uint32_t* seed, int seed_len, int N, int64_t depth,
                             int64_t dropout, const char* weights_dir, float* atom14,
                             float* distogram, float* pae, float* plddt, float* expres,
                             void* save);
int bc2n_structure_heads_bwd(void* stream, const float* single, const float* pair,
                             const float* seq_mask, const float* aatype,
                             const float* d_atom14, const float* d_distogram,
                             const float* d_pae, const float* d_plddt,
                             const float* d_expres, void* save, int N, int64_t depth,
                             int64_t dropout, const char* weights_dir, float* dsingle,
                             float* dpair);

/* ------------------------------------------------------------------------
 * The trunk of one design step in one call (a reduced form of the
 * reference's NativeDesignStep custom call, native/ffi.cu:1691-2178, runner
 * bindcraft/af/native_step.py: features in, structure-module outputs out;
 * the sequence parametrisation, confidence metrics and losses stay with the
 * caller).  fwd:
 *   (target_feat f32[N,21], msa_feat f32[S,N,49], residue_index, asym_id,
 *    entity_id, sym_id f32[N], offset i32[N,N] or NULL, seq_mask f32[N],
 *    act_const f32[N,N,64] or NULL (no template), aatype f32[N],
 *    seeds u32[recycles+1][4][3] = per pass the (k0, k1, enabled) keys of the
 *    template, extra, main and structure-module stacks; depths, dropout,
 *    recycles, five weights directories)
 *   -> (atom14 f32[N,14,3], distogram, pae f32[N,N,64], plddt f32[N,50],
 *       expres f32[N,37]) and save
 * = bc2n_embedder plus the three recycle terms (modules_multimer.py:
 * 487-507; their weights prev_pos_linear, prev_msa_first_row_norm and
 * prev_pair_norm in the embedder's directory), + bc2n_tplembed on that
 * pair, bc2n_evoformer pair-only (extra MSA mask zero), bc2n_evoformer
 * (main), single = msa[0] . single_activations (from the embedder's
 * directory), bc2n_structure_heads (modules_multimer.py:441-700).
 * `recycles` forward-only passes run first (bindcraft/af2.py:195-202; the
 * reference's design default is 1, settings/core/default.json:38), each
 * feeding its atoms' pseudo-beta, pair and msa[0] to the next pass's recycle
 * terms; the first pass's terms are the constants of a zero state.  The
 * outputs and the save-set are the last pass's.  bwd: the five
 * cotangents (any may be NULL) -> d_target_feat f32[N,21], d_msa_feat
 * f32[S,N,49].  N is a runtime value (a multiple of 32, at most 768): one
 * set of weights serves every length.  save holds
 * bc2n_design_step_save_bytes() bytes and is written by both calls.
 * ---------------------------------------------------------------------- */
size_t bc2n_design_step_save_bytes(const char* emb_dir, const char* tpl_dir,
                                   const char* extra_dir, const char* main_dir,
                                   const char* post_dir, int N, int S, int64_t d_tpl,
                                   int64_t d_extra, int64_t d_main, int64_t d_fold);
int bc2n_design_step_fwd(void* stream, const float* target_feat, const float* msa_feat,
                         const float* residue_index, const float* asym_id,
                         const float* entity_id, const float* sym_id, const int32_t* offset,
                         const float* seq_mask, const float* act_const, const float* aatype,
                         const uint32_t* seeds, int N, int S, int64_t d_tpl, int64_t d_extra,
                         int64_t d_main, int64_t d_fold, int64_t dropout, int64_t recycles,
                         const char* emb_dir, const char* tpl_dir, const char* extra_dir,
                         const char* main_dir, const char* post_dir, float* atom14,
                         float* distogram, float* pae, float* plddt, float* expres, void* save);
int bc2n_design_step_bwd(void* stream, const float* target_feat, const float* seq_mask,
                         const float* aatype, int64_t with_template, const float* d_atom14,
                         const float* d_distogram, const float* d_pae, const float* d_plddt,
                         const float* d_expres, void* save, int N, int S, int64_t d_tpl,
                         int64_t d_extra, int64_t d_main, int64_t d_fold, int64_t dropout,
                         const char* emb_dir, const char* tpl_dir, const char* extra_dir,
                         const char* main_dir, const char* post_dir, float* d_target_feat,
                         float* d_msa_feat);

/* ------------------------------------------------------------------------
 * Design sequence features: replaces GlueSeqFeat / GlueSeqFeatBwd
 * (native/ffi.cu:1105-1118 SeqFeatImpl, :1213-1227 GlueBwdImpl over
 * native/seqfeat.cuh).  logits f32[N,20], flags u8[N] (bit 0 = designed),
 * aa_bias f32[20] or NULL, the four design scalars (softmax_weight,
 * one_hot_weight, temperature, logit_scale) as values or, when `scalars` is
 * non-NULL, from that device buffer f32[4] in the same order; omitted_half =
 * the logit at or below which an acid counts as omitted (-5000 in BindCraft)
 *   -> feat, prof f32[N,20] (bindcraft/af2.py:99-104 over
 *      bindcraft/sequence_optimization.py:33-52; the one-hot is
 *      straight-through).
 * bwd: d_feat, d_prof f32[N,20] -> d_logits f32[N,20].
 * ---------------------------------------------------------------------- */
int bc2n_seqfeat_fwd(void* stream, const float* logits, const uint8_t* flags, const float* aa_bias,
                     float softmax_weight, float one_hot_weight, float temperature,
                     float logit_scale, float omitted_half, const float* scalars, int N,
                     float* feat, float* prof);
int bc2n_seqfeat_bwd(void* stream, const float* logits, const uint8_t* flags, const float* aa_bias,
                     const float* d_feat, const float* d_prof, float softmax_weight,
                     float one_hot_weight, float temperature, float logit_scale,
                     float omitted_half, const float* scalars, int N, float* d_logits);

/* ------------------------------------------------------------------------
 * The trunk inputs of the sequence features: the target_feat, msa_feat and
 * aatype entries of alphafold_input_features (bindcraft/af2.py:187-192;
 * native/inputfeat.cuh).  feat, prof f32[N,20] -> target_feat f32[N,21]
 * (feat and a zero column), msa_feat f32[1,N,49] (feat in channels 0..19,
 * prof in 25..44), aatype f32[N] = argmax(feat).  bwd: d_target_feat,
 * d_msa_feat -> d_feat, d_prof.
 * ---------------------------------------------------------------------- */
int bc2n_design_inputs_fwd(void* stream, const float* feat, const float* prof, int N,
                           float* target_feat, float* msa_feat, float* aatype);
int bc2n_design_inputs_bwd(void* stream, const float* d_target_feat, const float* d_msa_feat,
                           int N, float* d_feat, float* d_prof);

/* ------------------------------------------------------------------------
 * The one-call design step from the designed logits: the front of the
 * reference's NativeDesignStep (native/design_step.cuh seqfeat -> inputfeat
 * -> embed ..., native/ffi.cu:1691-2178) ahead of bc2n_design_step_fwd with
 * one MSA row.  logits f32[N,20], flags u8[N], aa_bias f32[20] or NULL,
 * scalars f32[4] on the device (softmax_weight, one_hot_weight, temperature,
 * logit_scale), omitted_half; the rest as bc2n_design_step_fwd without
 * target_feat, msa_feat, aatype (derived) and S (1).  When conf_plddt is
 * non-NULL the step also returns the confidence metrics of its head logits
 * (as bc2n_confidence_fwd: plddt, pae f32[N,N], ptm, iptm, iptm_per_residue,
 * expres_ca; interface_asym i32[N]), the reference step's Outputs.  When
 * atom37 is non-NULL the step also returns the prediction's atom37 positions
 * f32[N,37,3] and their exists mask f32[N,37] (the atom14 positions gathered
 * by residx_atom37_to_atom14 times restype_atom37_mask[aatype] * seq_mask,
 * tables const/atom37_to_atom14 and const/atom37_mask in post_dir); given
 * the template's atoms tpl_atoms37 f32[N,37,3] and mask f32[N,37] they are
 * superposed on them, as the reference step's atoms are
 * (native/design_step.cuh:1162-1168): a Kabsch of the CA atoms of the
 * residues flagged TEMPLATE and not DESIGN (flags bits 1, 0;
 * bindcraft/af2.py:89-97, bindcraft/protein.py:75-83), its rotation under
 * stop_gradient.  With a template embedding (act_const) and the template
 * row's weights present (template_single_embedding, template_projection in
 * emb_dir; const/chi_atom_indices, const/chi_angles_mask in post_dir) the
 * template's MSA row joins the main stack, as modules_multimer.py:608-617
 * adds it (the reference's S = 2): its features are the one-hot of aatype
 * on TEMPLATE residues (21 elsewhere) and the template's chi angles from
 * tpl_atoms37 / tpl_mask37, which are then required (template_embedding_1d,
 * modules_multimer.py:1080-1137; bindcraft/af2.py:153-160).
 * bwd: the five head cotangents, the atom37 one and those of
 * the confidence metrics (any may be NULL; the atom37 and confidence ones
 * need a forward that computed them) -> d_logits f32[N,20].  save holds
 * bc2n_design_step_seq_save_bytes() bytes.
 * cyclic_mode: -1 takes `offset` as given (NULL: residue_index
 * differences); 0 'distance', 1 'direction', 2 'neighbours' build the
 * offset feature on the device from residue_index, asym_id, flags (bit 6 =
 * CYCLIC) and seq_mask as bc2's cyclic_sequence_offsets does
 * (bindcraft/af2.py:174-185, :193; the reference's cyclic_mode attribute,
 * native/inputfeat.cuh offsetK), ignoring `offset`.  flexibility: the
 * reference's target flexibility f (>= 0; 0 = off): a TEMPLATE residue not
 * designed whose residue_index i has floor((i + 1) f) > floor(i f) is a gap
 * of the template row (bindcraft/af2.py:150-157).  cyclic_mode + 4 (the
 * reference's bit 2, bc2's large_complex_initialization; needs an offset
 * mode and tpl_atoms37): the first pass's structure module starts from the
 * frames of tpl_atoms37's N, CA, C (an all-zero residue: the zero matrix, as
 * the multimer model's), each recycle pass from the previous pass's atom37
 * positions (folding_multimer.py:508-515, native/design_step.cuh:1112-1114).
 * RUNTIME LENGTH (the reference's `n`, native/design_step.cuh:10-19,
 * :42-58): n is NULL (all N rows real) or an i32 scalar in device memory,
 * 1 <= *n <= N, read by the kernels and never by the host, so one set of
 * buffers sized N (the bucket) serves every length up to it.  Rows i >= *n
 * of every input are padding (any finite values): seq_mask and flags are
 * zeroed there before any mask is derived, the padding's outputs are
 * written as zeros, and in the backward the padding's cotangents are
 * zeroed before use and its d_logits rows are zero.  Pass the same n to
 * both calls.
 * ---------------------------------------------------------------------- */
size_t bc2n_design_step_seq_save_bytes(const char* emb_dir, const char* tpl_dir,
                                       const char* extra_dir, const char* main_dir,
                                       const char* post_dir, int N, int64_t d_tpl,
                                       int64_t d_extra, int64_t d_main, int64_t d_fold);
int bc2n_design_step_seq_fwd(void* stream, const float* logits, const uint8_t* flags,
                             const float* aa_bias, const float* scalars, float omitted_half,
                             const float* residue_index, const float* asym_id,
                             const float* entity_id, const float* sym_id, const int32_t* offset,
                             const float* seq_mask, const float* act_const,
                             const uint32_t* seeds, int N, const int32_t* n, int64_t d_tpl,
                             int64_t d_extra, int64_t d_main, int64_t d_fold, int64_t dropout,
                             int64_t recycles, int64_t cyclic_mode, float flexibility,
                             const char* emb_dir, const char* tpl_dir,
                             const char* extra_dir, const char* main_dir, const char* post_dir,
                             float* atom14, float* distogram, float* pae, float* plddt,
                             float* expres, const float* tpl_atoms37, const float* tpl_mask37,
                             float* atom37,
                             float* atom37_mask, const int32_t* interface_asym,
                             float* conf_plddt, float* conf_pae, float* ptm, float* iptm,
                             float* iptm_per_residue, float* expres_ca, void* save);
int bc2n_design_step_seq_bwd(void* stream, const float* logits, const uint8_t* flags,
                             const float* aa_bias, const float* scalars, float omitted_half,
                             const float* seq_mask, int64_t with_template,
                             const float* d_atom14, const float* d_distogram, const float* d_pae,
                             const float* d_plddt, const float* d_expres, const float* d_atom37,
                             const int32_t* interface_asym, const float* d_conf_plddt,
                             const float* d_conf_pae, const float* d_ptm, const float* d_iptm,
                             const float* d_iptm_per_residue, const float* d_expres_ca, void* save,
                             int N, const int32_t* n, int64_t d_tpl, int64_t d_extra, int64_t d_main, int64_t d_fold,
                             int64_t dropout, const char* emb_dir, const char* tpl_dir,
                             const char* extra_dir, const char* main_dir, const char* post_dir,
                             float* d_logits);

/* ------------------------------------------------------------------------
 * Confidence metrics: replaces Confidence / ConfidenceBwd (native/ffi.cu:
 * 1120-1159 ConfidenceImpl, :1227-1252 ConfBwdImpl over native/confidence.cuh).
 * plddt_logits f32[N,50], pae_logits f32[N,N,64] (16-byte aligned),
 * expres_logits f32[N,37] (the structure heads' outputs), seq_mask f32[N],
 * interface_asym i32[N] -> plddt f32[N], pae f32[N,N] (symmetrised), ptm
 * f32[1], iptm f32[1], iptm_per_residue f32[N], expres_ca f32[N]
 * (bindcraft/af2.py:197-219 with AF2's predicted_tm_score; the bin tables,
 * including d0 of the runtime residue weights, are built on the device).
 * save holds bc2n_confidence_save_bytes(N) bytes, written by fwd, read by bwd.
 * bwd: cotangents of the six outputs (any may be NULL; d_ptm and d_iptm are
 * device scalars; pTM/ipTM route through their max to one row, as the
 * reference's tmBwdK does) -> d_plddt_logits, d_pae_logits, d_expres_logits.
 * ---------------------------------------------------------------------- */
size_t bc2n_confidence_save_bytes(int N);
int bc2n_confidence_fwd(void* stream, const float* plddt_logits, const float* pae_logits,
                        const float* expres_logits, const float* seq_mask,
                        const int32_t* interface_asym, int N, float* plddt, float* pae,
                        float* ptm, float* iptm, float* iptm_per_residue, float* expres_ca,
                        void* save);
int bc2n_confidence_bwd(void* stream, const float* plddt_logits, const float* pae_logits,
                        const float* expres_logits, const float* seq_mask,
                        const int32_t* interface_asym, const void* save, const float* d_plddt,
                        const float* d_pae, const float* d_ptm, const float* d_iptm,
                        const float* d_iptm_per_residue, const float* d_expres_ca, int N,
                        float* d_plddt_logits, float* d_pae_logits, float* d_expres_logits);

/* ------------------------------------------------------------------------
 * Dropout with JAX's own bits.  tbl[b*C+c] = keep/keep_rate where
 * keep = jax.random.bernoulli(key, keep_rate, (B, C)), keep_rate =
 * float32(1) - float32(rate); key = (k0, k1) = jax.random.key_data(key).
 * Reference semantics: modules.py:37-44 (apply_dropout).
 * ---------------------------------------------------------------------- */
int bc2n_dropout_table(void* stream, float* tbl, int B, int C, uint32_t k0,
                       uint32_t k1, float rate);
/* keep bits (uint8 0/1) of jax.random.bernoulli(key, 1-rate, (n,)). */
int bc2n_bernoulli_bits(void* stream, uint8_t* out, long n, uint32_t k0,
                        uint32_t k1, float rate);
/* Per-module dropout keys of an Evoformer stack, derived on the device from
 * the stack key seed[0..1] (modules_multimer.py:622-641, modules.py:1308):
 * out[(layer*9 + module)*2 + {0,1}]. */
int bc2n_stack_keys(void* stream, const uint32_t* seed, int depth, uint32_t* out);

/* ------------------------------------------------------------------------
 * Per-kernel device timing (the reference's BLK_PROF/PROF_STEP counterpart,
 * native/common.cuh:842-900): when enabled each kernel launch is bracketed
 * by a HIP event pair on its stream.  bc2n_prof_read synchronises, writes
 * up to `cap` (name, total ms, launch count) entries -- names as
 * NUL-terminated strings at names + i*name_len -- clears the records and
 * returns the entry count (-1 on error).
 * ---------------------------------------------------------------------- */
int bc2n_prof_enable(int on);
/* Time only the launches named `name` (NULL: every launch). */
int bc2n_prof_filter(const char* name);
int bc2n_prof_read(char* names, int name_len, double* ms, int* counts, int cap);

/* ------------------------------------------------------------------------
 * Kernel probes (test hooks; no reference counterpart beyond the module
 * gates of native/*.cu).
 * ---------------------------------------------------------------------- */
/* C[M,N] = A[M,K] . B[N,K]^T, IEEE binary16 (uint16 bits) in, f32 out. */
int bc2n_probe_gemm(void* stream, int M, int N, int K, const uint16_t* A,
                    const uint16_t* B, float* C);
/* MFMA issue rate: `blocks` workgroups of 4 waves, each wave 8 independent
 * accumulator chains of `iters` MFMAs from registers (form 0:
 * v_mfma_f32_16x16x32_f16, 1: v_mfma_f32_16x16x16_f16, 2:
 * v_mfma_f32_32x32x16_f16, 3: v_mfma_f32_16x16x32_bf16); out f32[blocks*256].
 * Returns the FLOPs launched, or -1 on a bad argument (bc2n_last_error()). */
double bc2n_probe_mfma(void* stream, int form, int blocks, int iters, float* out);
/* Batched f32 GEMM with element strides (the structure module's GEMM):
 * C[b][m][n] = sum_k A[b*a_sb + m*a_sm + k*a_sk] * B[b*b_sb + k*b_sk + n*b_sn]. */
int bc2n_probe_gemm_f32(void* stream, int M, int N, int K, int batch, const float* A,
                        long a_sm, long a_sk, long a_sb, const float* B, long b_sk,
                        long b_sn, long b_sb, float* C, long c_sm, long c_sn, long c_sb);
/* The design step's recycle terms, in place (modules_multimer.py:487-507):
 * pair f32[N,N,128] += prev_pos_linear(dgram(pseudo_beta(prev_atom14, aatype)))
 * + prev_pair_norm(prev_pair), msa0 f32[N,256] +=
 * prev_msa_first_row_norm(prev_msa0); weights from emb_dir.  prev_atom14
 * NULL = the first pass (bias and offsets only). */
int bc2n_probe_recycle(void* stream, int N, const char* emb_dir, const float* aatype,
                       const float* prev_atom14, const float* prev_pair, const float* prev_msa0,
                       float* pair, float* msa0);
/* y = LN(x) over C channels, binary16 out + mean/rstd. fast = E[x^2]-E[x]^2. */
int bc2n_probe_layernorm(void* stream, long M, int C, const float* x,
                         const float* gamma, const float* beta, int fast,
                         uint16_t* y, float* mean, float* rstd);

#ifdef __cplusplus
}
#endif
#endif /* BC2N_H */
