"""Random-init AF2 trunk parameters and the weights-manifest writer.

Parameter names and shapes are those of the AF2 multimer Evoformer haiku
modules (bindcraft/af/alphafold/model/modules.py), flattened into the
manifest naming the reference's native loader reads,
``param/block{b}/<module>/<sub>/<param>`` (bindcraft/af/native.py:171-226).
The manifest format is kept identical on purpose so a directory written by
the reference's ``weights_from_params`` loads here unchanged: one line
``name file ndim d0 d1 ...`` per tensor, raw little-endian float32 files.
"""
import math
import os

import numpy as np

# AF2 multimer widths (config.py:386-460)
C_Z, C_M, C_E, C_T = 128, 256, 64, 64


def _shapes_attention(c_in, h, d, c_out, gating=True):
    s = {
        "attention/query_w": (c_in, h, d),
        "attention/key_w": (c_in, h, d),
        "attention/value_w": (c_in, h, d),
        "attention/output_w": (h, d, c_out),
        "attention/output_b": (c_out,),
    }
    if gating:
        s["attention/gating_w"] = (c_in, h, d)
        s["attention/gating_b"] = (h, d)
    return s


def module_shapes(c_z=C_Z, c_m=C_M, tri_heads=4, trimul_hidden=None, opm_c=32,
                  row_heads=8, col_heads=8):
    """{module: {param: shape}} of one EvoformerIteration."""
    ti = trimul_hidden or c_z
    sh = {}
    for n in ("triangle_attention_starting_node", "triangle_attention_ending_node"):
        s = {"query_norm/scale": (c_z,), "query_norm/offset": (c_z,),
             "feat_2d_weights": (c_z, tri_heads)}
        s.update(_shapes_attention(c_z, tri_heads, c_z // tri_heads, c_z))
        sh[n] = s
    for n in ("triangle_multiplication_outgoing", "triangle_multiplication_incoming"):
        sh[n] = {
            "left_norm_input/scale": (c_z,), "left_norm_input/offset": (c_z,),
            "projection/weights": (c_z, 2 * ti), "projection/bias": (2 * ti,),
            "gate/weights": (c_z, 2 * ti), "gate/bias": (2 * ti,),
            "center_norm/scale": (ti,), "center_norm/offset": (ti,),
            "output_projection/weights": (ti, c_z), "output_projection/bias": (c_z,),
            "gating_linear/weights": (c_z, c_z), "gating_linear/bias": (c_z,),
        }
    for n, c in (("pair_transition", c_z), ("msa_transition", c_m)):
        sh[n] = {"input_layer_norm/scale": (c,), "input_layer_norm/offset": (c,),
                 "transition1/weights": (c, 4 * c), "transition1/bias": (4 * c,),
                 "transition2/weights": (4 * c, c), "transition2/bias": (c,)}
    sh["outer_product_mean"] = {
        "layer_norm_input/scale": (c_m,), "layer_norm_input/offset": (c_m,),
        "left_projection/weights": (c_m, opm_c), "left_projection/bias": (opm_c,),
        "right_projection/weights": (c_m, opm_c), "right_projection/bias": (opm_c,),
        "output_w": (opm_c, opm_c, c_z), "output_b": (c_z,),
    }
    s = {"query_norm/scale": (c_m,), "query_norm/offset": (c_m,),
         "feat_2d_norm/scale": (c_z,), "feat_2d_norm/offset": (c_z,),
         "feat_2d_weights": (c_z, row_heads)}
    s.update(_shapes_attention(c_m, row_heads, c_m // row_heads, c_m))
    sh["msa_row_attention_with_pair_bias"] = s
    s = {"query_norm/scale": (c_m,), "query_norm/offset": (c_m,)}
    s.update(_shapes_attention(c_m, col_heads, c_m // col_heads, c_m))
    sh["msa_column_attention"] = s
    return sh


def _fan_in(pname, shape):
    if pname.endswith("output_w") and len(shape) == 3 and not pname.startswith("output_w"):
        return shape[0] * shape[1]      # attention output [H, D, C]
    if pname == "output_w":
        return shape[0] * shape[1]      # OPM [c, e, f]
    return shape[0]


def init_module(shapes, rng, gates="zero", ln="identity"):
    """LeCun-normal weights (std 1/sqrt(fan_in)), zero biases.  gates='zero'
    gives AF2's gate init (weights 0, bias 1); gates='random' draws them like
    any weight (bias N(0,1)) so the gate paths carry signal in tests.
    ln='identity' -> scale 1, offset 0; 'random' -> 1+N(0,.1), N(0,.1)."""
    out = {}
    for pname, shape in shapes.items():
        leaf = pname.split("/")[-1]
        is_gate = ("gating" in pname) or pname.startswith("gate/")
        if leaf == "scale":
            v = np.ones(shape) if ln == "identity" else 1.0 + 0.1 * rng.standard_normal(shape)
        elif leaf == "offset":
            v = np.zeros(shape) if ln == "identity" else 0.1 * rng.standard_normal(shape)
        elif leaf in ("bias", "output_b", "gating_b"):
            if is_gate:
                v = np.ones(shape) if gates == "zero" else rng.standard_normal(shape)
            else:
                v = np.zeros(shape) if gates == "zero" else 0.1 * rng.standard_normal(shape)
        else:
            if is_gate and gates == "zero":
                v = np.zeros(shape)
            else:
                v = rng.standard_normal(shape) / np.sqrt(_fan_in(pname, shape))
        out[pname] = np.asarray(v, np.float32)
    return out


TEMPLATE_MODULES = ("triangle_multiplication_outgoing", "triangle_multiplication_incoming",
                    "triangle_attention_starting_node", "triangle_attention_ending_node",
                    "pair_transition")


def init_template_block_params(block, rng, gates="zero", ln="identity"):
    """One TemplateEmbeddingIteration (c_t=64, 4 heads, trimul hidden 64,
    transition factor 2 -- config.py template_pair_stack)."""
    sh = module_shapes(c_z=C_T, tri_heads=4, trimul_hidden=64)
    sh["pair_transition"] = {"input_layer_norm/scale": (C_T,), "input_layer_norm/offset": (C_T,),
                             "transition1/weights": (C_T, 2 * C_T), "transition1/bias": (2 * C_T,),
                             "transition2/weights": (2 * C_T, C_T), "transition2/bias": (C_T,)}
    out = {}
    for mod in TEMPLATE_MODULES:
        for pname, arr in init_module(sh[mod], rng, gates, ln).items():
            out[f"param/block{block}/{mod}/{pname}"] = arr
    return out


def template_embedding_shapes(c_z=C_Z, c_t=C_T):
    """The template embedding's own weights around the stack
    (modules_multimer.py:704-1005; names as under param/ in the reference's
    template-embedding weights directory)."""
    return {"query_embedding_norm/scale": (c_z,), "query_embedding_norm/offset": (c_z,),
            "template_pair_embedding_8/weights": (c_z, c_t), "template_pair_embedding_8/bias": (c_t,),
            "output_layer_norm/scale": (c_t,), "output_layer_norm/offset": (c_t,),
            "output_linear/weights": (c_t, c_z), "output_linear/bias": (c_z,)}


def init_template_embedding_params(depth, rng, gates="zero", ln="identity"):
    """Weights directory contents of a template embedding with `depth` stack
    blocks."""
    out = {}
    for b in range(depth):
        out.update(init_template_block_params(b, rng, gates, ln))
    for pname, arr in init_module(template_embedding_shapes(), rng, gates, ln).items():
        out[f"param/{pname}"] = arr
    return out


def embedder_shapes(c_m=C_M, c_z=C_Z):
    """The multimer embedder's input Linears (modules_multimer.py:441-483;
    names as under param/ in the reference's embedder weights directory,
    bindcraft/af/native.py:529-570): target_feat 21 wide, msa_feat 49,
    73 relative-position features."""
    return {"preprocess_1d/weights": (21, c_m), "preprocess_1d/bias": (c_m,),
            "preprocess_msa/weights": (49, c_m), "preprocess_msa/bias": (c_m,),
            "left_single/weights": (21, c_z), "left_single/bias": (c_z,),
            "right_single/weights": (21, c_z), "right_single/bias": (c_z,),
            "position_activations/weights": (73, c_z), "position_activations/bias": (c_z,)}


def recycle_shapes(c_m=C_M, c_z=C_Z, bins=15):
    """The embedder's three recycle terms (modules_multimer.py:487-507; in
    the embedder's weights directory, bindcraft/af/native.py:515-527):
    prev_pos_linear over the 15-bin distogram of the previous pseudo-beta
    positions, and the LayerNorms of the previous msa[0] and pair."""
    return {"prev_pos_linear/weights": (bins, c_z), "prev_pos_linear/bias": (c_z,),
            "prev_msa_first_row_norm/scale": (c_m,), "prev_msa_first_row_norm/offset": (c_m,),
            "prev_pair_norm/scale": (c_z,), "prev_pair_norm/offset": (c_z,)}


def template_row_shapes(c_m=C_M, nfeat=34):
    """template_embedding_1d's two Linears (modules_multimer.py:1080-1137):
    the template's MSA row from 34 features (one-hot template aatype 22,
    sin/cos/mask of 4 chi angles); in the embedder's weights directory
    (bindcraft/af/native.py:521-524)."""
    return {"template_single_embedding/weights": (nfeat, c_m),
            "template_single_embedding/bias": (c_m,),
            "template_projection/weights": (c_m, c_m), "template_projection/bias": (c_m,)}


def single_activations_shapes(c_m=C_M, c_s=384):
    """single_activations (modules_multimer.py EmbeddingsAndEvoformer: the
    single representation from the main stack's msa[0]); it ships in the
    embedder's weights directory (bindcraft/af/native.py:515-527)."""
    return {"single_activations/weights": (c_m, c_s), "single_activations/bias": (c_s,)}


def init_embedder_params(rng, scoped=False):
    """Weights directory contents of the embedder (with single_activations);
    `scoped` puts
    position_activations under evoformer/~_relative_encoding/ as haiku's
    method scope (and the checkpoint) does."""
    out = {}
    for name, shape in {**embedder_shapes(), **single_activations_shapes(),
                        **recycle_shapes(), **template_row_shapes()}.items():
        fan_in = shape[0] if len(shape) == 2 else 1
        arr = rng.standard_normal(shape) / math.sqrt(fan_in)
        if len(shape) == 1:
            arr = 0.1 * rng.standard_normal(shape)
        if scoped and name.startswith("position_activations/"):
            name = "evoformer/~_relative_encoding/" + name
        out[f"param/{name}"] = arr.astype(np.float32)
    return out


def global_attention_shapes(c=C_E, heads=8):
    """MSAColumnGlobalAttention of the extra-MSA stack (modules.py:403-497,
    619-672; config.py extra_msa: 8 heads, key/value dim c)."""
    d = c // heads
    return {"query_norm/scale": (c,), "query_norm/offset": (c,),
            "attention/query_w": (c, heads, d), "attention/key_w": (c, d),
            "attention/value_w": (c, d), "attention/gating_w": (c, heads, d),
            "attention/gating_b": (heads, d), "attention/output_w": (heads, d, c),
            "attention/output_b": (c,)}


def init_block_params(block, rng, modules=None, gates="zero", ln="identity", **shape_kw):
    """Flat {manifest name: array} for one Evoformer block."""
    sh = module_shapes(**shape_kw)
    out = {}
    for mod, shapes in sh.items():
        if modules is not None and mod not in modules:
            continue
        for pname, arr in init_module(shapes, rng, gates, ln).items():
            out[f"param/block{block}/{mod}/{pname}"] = arr
    return out


# The pair-track modules of an extra-MSA block in its pair-only form (the
# outer product mean kept for its output_b, which the fully masked extra MSA
# turns into a constant pair update).
PAIR_ONLY_MODULES = ("outer_product_mean", "triangle_multiplication_outgoing",
                     "triangle_multiplication_incoming", "triangle_attention_starting_node",
                     "triangle_attention_ending_node", "pair_transition")


def init_trunk_params(rng, depth=48, extra_depth=4, tpl_depth=2, gates="zero", ln="identity"):
    """The design-step trunk of BASELINE configs[3]/[4] with random weights:
    `depth` Evoformer blocks (c_m=256, c_z=128), `extra_depth` pair-only
    extra-MSA blocks and `tpl_depth` template pair blocks (c_t=64), LeCun-normal
    weights with AF2's gate init.  Returns three flat manifest dicts (main,
    extra, template), drawn in that order from `rng`."""
    evo = {}
    for blk in range(depth):
        evo.update(init_block_params(blk, rng, gates=gates, ln=ln))
    extra = {}
    for blk in range(extra_depth):
        extra.update(init_block_params(blk, rng, gates=gates, ln=ln, modules=PAIR_ONLY_MODULES))
    tpl = {}
    for blk in range(tpl_depth):
        tpl.update(init_template_block_params(blk, rng, gates=gates, ln=ln))
    return evo, extra, tpl


# AF2 multimer structure module (folding_multimer.py, config.py:578-600):
# single width 384, 12 heads, 16 scalar / 4 point qk, 16 scalar / 8 point v.
C_S, IPA_H = 384, 12


def fold_shapes(c_s=C_S, c_z=C_Z, h=IPA_H, sqk=16, pqk=4, sv=16, pv=8):
    """{param: shape} of the post-trunk weights the fold iterations use, in
    the naming of bindcraft/af/native.py:339-444 (post_weights_from_params):
    no block index -- the iterations share one set."""
    ipa = "fold_iteration/invariant_point_attention/"
    sh = {
        "single_layer_norm/scale": (c_s,), "single_layer_norm/offset": (c_s,),
        "initial_projection/weights": (c_s, c_s), "initial_projection/bias": (c_s,),
        "pair_layer_norm/scale": (c_z,), "pair_layer_norm/offset": (c_z,),
        ipa + "trainable_point_weights": (h,),
        ipa + "q_scalar_projection/weights": (c_s, h, sqk), ipa + "q_scalar_projection/bias": (h * sqk,),
        ipa + "k_scalar_projection/weights": (c_s, h, sqk), ipa + "k_scalar_projection/bias": (h * sqk,),
        ipa + "v_scalar_projection/weights": (c_s, h, sv), ipa + "v_scalar_projection/bias": (h * sv,),
        ipa + "q_point_projection/point_projection/weights": (c_s, h, 3 * pqk),
        ipa + "q_point_projection/point_projection/bias": (h, 3 * pqk),
        ipa + "k_point_projection/point_projection/weights": (c_s, h, 3 * pqk),
        ipa + "k_point_projection/point_projection/bias": (h, 3 * pqk),
        ipa + "v_point_projection/point_projection/weights": (c_s, h, 3 * pv),
        ipa + "v_point_projection/point_projection/bias": (h, 3 * pv),
        ipa + "attention_2d/weights": (c_z, h), ipa + "attention_2d/bias": (h,),
        ipa + "output_projection/weights": (h * sv + 4 * h * pv + h * c_z, c_s),
        ipa + "output_projection/bias": (c_s,),
        "fold_iteration/attention_layer_norm/scale": (c_s,),
        "fold_iteration/attention_layer_norm/offset": (c_s,),
        "fold_iteration/transition_layer_norm/scale": (c_s,),
        "fold_iteration/transition_layer_norm/offset": (c_s,),
        "fold_iteration/quat_rigid/rigid/weights": (c_s, 6),
        "fold_iteration/quat_rigid/rigid/bias": (6,),
    }
    for t in ("transition", "transition_1", "transition_2"):
        sh[f"fold_iteration/{t}/weights"] = (c_s, c_s)
        sh[f"fold_iteration/{t}/bias"] = (c_s,)
    return sh


def init_fold_params(rng, final="random", ln="identity"):
    """Flat {manifest name: array} of the fold iterations.  final='zero' is
    AF2's zero init of the last layers (output projection, last transition,
    quat_rigid); 'random' draws them (small) so every path carries signal in
    tests.  trainable_point_weights start at softplus^-1(1) = log(e - 1)."""
    out = {}
    zero_last = ("output_projection", "transition_2/", "quat_rigid")
    for pname, shape in fold_shapes().items():
        leaf = pname.split("/")[-1]
        if leaf == "trainable_point_weights":
            v = np.full(shape, np.log(np.e - 1.0)) + (0.1 * rng.standard_normal(shape)
                                                       if final == "random" else 0.0)
        elif leaf == "scale":
            v = np.ones(shape) if ln == "identity" else 1.0 + 0.1 * rng.standard_normal(shape)
        elif leaf == "offset":
            v = np.zeros(shape) if ln == "identity" else 0.1 * rng.standard_normal(shape)
        elif leaf == "bias":
            v = np.zeros(shape) if final == "zero" else 0.1 * rng.standard_normal(shape)
        else:
            last = any(z in pname for z in zero_last)
            if last and final == "zero":
                v = np.zeros(shape)
            else:
                scale = 0.1 if (last and "quat_rigid" in pname) else 1.0
                v = scale * rng.standard_normal(shape) / np.sqrt(shape[0])
        out[f"param/{pname}"] = np.asarray(v, np.float32)
    return out


def sidechain_shapes(c_s=C_S, c=128):
    """MultiRigidSidechain of the fold iteration (folding_multimer.py:950-1040,
    config.py sidechain: num_channel 128, 2 residual blocks), under
    fold_iteration/rigid_sidechain/."""
    sh = {"input_projection/weights": (c_s, c), "input_projection/bias": (c,),
          "input_projection_1/weights": (c_s, c), "input_projection_1/bias": (c,),
          "unnormalized_angles/weights": (c, 14), "unnormalized_angles/bias": (14,)}
    for sfx in ("", "_1"):
        for r in ("resblock1", "resblock2"):
            sh[f"{r}{sfx}/weights"] = (c, c)
            sh[f"{r}{sfx}/bias"] = (c,)
    return {f"fold_iteration/rigid_sidechain/{k}": v for k, v in sh.items()}


def heads_shapes(c_s=C_S, c_z=C_Z):
    """The four heads (modules.py:777-1120; config.py heads: 64 distogram
    bins, 64 aligned-error bins, pLDDT 128 channels x 50 bins, 37
    experimentally-resolved logits)."""
    return {"distogram_head/half_logits/weights": (c_z, 64),
            "distogram_head/half_logits/bias": (64,),
            "predicted_aligned_error_head/logits/weights": (c_z, 64),
            "predicted_aligned_error_head/logits/bias": (64,),
            "predicted_lddt_head/input_layer_norm/scale": (c_s,),
            "predicted_lddt_head/input_layer_norm/offset": (c_s,),
            "predicted_lddt_head/act_0/weights": (c_s, 128),
            "predicted_lddt_head/act_0/bias": (128,),
            "predicted_lddt_head/act_1/weights": (128, 128),
            "predicted_lddt_head/act_1/bias": (128,),
            "predicted_lddt_head/logits/weights": (128, 50),
            "predicted_lddt_head/logits/bias": (50,),
            "experimentally_resolved_head/logits/weights": (c_s, 37),
            "experimentally_resolved_head/logits/bias": (37,)}


def init_structure_heads_params(rng, final="random", ln="identity"):
    """The post-trunk weights directory: fold iterations, sidechain, heads
    (LeCun-normal weights, small random biases unless final == 'zero')."""
    out = init_fold_params(rng, final=final, ln=ln)
    for name, shape in {**sidechain_shapes(), **heads_shapes()}.items():
        leaf = name.split("/")[-1]
        if leaf == "scale":
            v = np.ones(shape) if ln == "identity" else 1.0 + 0.1 * rng.standard_normal(shape)
        elif leaf == "offset":
            v = np.zeros(shape) if ln == "identity" else 0.1 * rng.standard_normal(shape)
        elif leaf == "bias":
            v = np.zeros(shape) if final == "zero" else 0.1 * rng.standard_normal(shape)
            if final != "zero" and "unnormalized_angles" in name:
                # cos components +2: every (sin, cos) torsion vector keeps a norm
                # well away from 0, as trained weights give, so its normalisation
                # does not amplify upstream rounding (a random head can put one
                # near 0, where the angle's direction is ill-conditioned)
                v[1::2] += 2.0
        else:
            v = rng.standard_normal(shape) / np.sqrt(shape[0])
        out[f"param/{name}"] = np.asarray(v, np.float32)
    return out


def init_residue_tables(rng):
    """Random residue tables of the shapes the structure module reads
    (const/default_frame [21,8,4,4] rigid 4x4 frames, const/atom14_to_group
    [21,14], const/atom14_lit_pos [21,14,3], const/atom14_mask [21,14]) and
    the design step's atom37 gather (const/atom37_to_atom14 [21,37],
    const/atom37_mask [21,37]).  Both are table-driven, so random tables
    exercise every path; the real ones come from the model's
    residue_constants."""
    q = rng.standard_normal((21, 8, 4))
    q /= np.linalg.norm(q, axis=-1, keepdims=True)
    w, x, y, z = q[..., 0], q[..., 1], q[..., 2], q[..., 3]
    R = np.stack([1 - 2 * (y * y + z * z), 2 * (x * y - w * z), 2 * (x * z + w * y),
                  2 * (x * y + w * z), 1 - 2 * (x * x + z * z), 2 * (y * z - w * x),
                  2 * (x * z - w * y), 2 * (y * z + w * x), 1 - 2 * (x * x + y * y)],
                 -1).reshape(21, 8, 3, 3)
    fr = np.zeros((21, 8, 4, 4))
    fr[..., :3, :3] = R
    fr[..., :3, 3] = 1.5 * rng.standard_normal((21, 8, 3))
    fr[..., 3, 3] = 1.0
    fr[:, 0] = np.eye(4)  # the backbone group is the backbone frame
    out = {"default_frame": fr.astype(np.float32),
           "atom14_to_group": rng.integers(0, 8, (21, 14)).astype(np.float32),
           "atom14_lit_pos": (1.5 * rng.standard_normal((21, 14, 3))).astype(np.float32),
           "atom14_mask": (rng.random((21, 14)) < 0.8).astype(np.float32)}
    # the atom37 gather of the design step's outputs: every atom37 slot reads
    # one atom14 slot (CA always slot 1, as in residue_constants)
    a37 = rng.integers(0, 14, (21, 37))
    a37[:, :3] = [0, 1, 2]  # N, CA, C: atom14 slots 0-2 and present, as in every real type
    m37 = (rng.random((21, 37)) < 0.5).astype(np.float32)
    m37[:, :3] = 1.0
    out["atom37_to_atom14"] = a37.astype(np.float32)
    out["atom37_mask"] = m37
    # the template row's chi angles: four distinct atom37 slots per chi (as
    # the real table has; a repeated atom makes the dihedral 0/0), and which
    # chis each residue type has (the unknown type, row 20, has none)
    out["chi_atom_indices"] = rng.random((21, 4, 37)).argsort(-1)[..., :4].astype(np.float32)
    cm = (rng.random((21, 4)) < 0.7).astype(np.float32)
    cm[20] = 0.0
    out["chi_angles_mask"] = cm
    return out


def residue_tables_from(rc):
    """The residue tables from a residue_constants module (alphafold.common),
    in the layout the weights directory stores (const/...): the structure
    module's four and the atom37 gather's two."""
    # residx_atom37_to_atom14 per restype (the make_atom14_masks tables):
    # restypes order, UNK all zeros
    a37 = np.zeros((21, 37), np.float32)
    for r, rt in enumerate(rc.restypes):
        for j, name in enumerate(rc.restype_name_to_atom14_names[rc.restype_1to3[rt]]):
            if name:
                a37[r, rc.atom_order[name]] = j
    # all_atom_multimer.get_chi_atom_indices: restypes order, UNK all zeros
    chi = np.zeros((21, 4, 4), np.float32)
    for r, rt in enumerate(rc.restypes):
        for c, atoms in enumerate(rc.chi_angles_atoms[rc.restype_1to3[rt]]):
            chi[r, c] = [rc.atom_order[a] for a in atoms]
    return {"default_frame": np.asarray(rc.restype_rigid_group_default_frame, np.float32),
            "atom14_to_group": np.asarray(rc.restype_atom14_to_rigid_group, np.float32),
            "atom14_lit_pos": np.asarray(rc.restype_atom14_rigid_group_positions, np.float32),
            "atom14_mask": np.asarray(rc.restype_atom14_mask, np.float32),
            "atom37_to_atom14": a37,
            "atom37_mask": np.asarray(rc.restype_atom37_mask, np.float32),
            "chi_atom_indices": chi,
            "chi_angles_mask": np.asarray(list(rc.chi_angles_mask) + [[0.0] * 4], np.float32)}


def write_manifest(out_dir, params):
    """Write {name: array} as a weights directory (manifest.txt + .f32)."""
    os.makedirs(out_dir, exist_ok=True)
    with open(os.path.join(out_dir, "manifest.txt"), "w") as fh:
        for name in sorted(params):
            arr = np.ascontiguousarray(params[name], dtype=np.float32)
            fn = name.replace("/", "__") + ".f32"
            arr.tofile(os.path.join(out_dir, fn))
            fh.write(f"{name} {fn} {arr.ndim} {' '.join(str(x) for x in arr.shape)}\n")
    return out_dir


def read_manifest(in_dir):
    """Inverse of write_manifest (numpy only; nothing is unpickled)."""
    out = {}
    with open(os.path.join(in_dir, "manifest.txt")) as fh:
        for line in fh:
            parts = line.split()
            if not parts:
                continue
            name, fn, nd = parts[0], parts[1], int(parts[2])
            shape = tuple(int(x) for x in parts[3:3 + nd])
            out[name] = np.fromfile(os.path.join(in_dir, fn), dtype="<f4").reshape(shape)
    return out
