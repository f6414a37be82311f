"""AF2 parameter trees -> the library's weights directories.

The library reads its weights from a directory: ``manifest.txt`` with one
line ``name file ndim d0 d1 ...`` per tensor and one raw little-endian f32
file per tensor.  The names are the haiku module paths of the AF2 multimer
model below a per-component scope, with the layer-stack axis spelled as a
block index: ``param/block{b}/<module path>/<param>`` for the stacks,
``param/<module path>/<param>`` for the rest.  This is the format and naming
of bindcraft/af/native.py:171-226 (weights_from_params), 264-323
(tplembed_weights_from_params), 339-444 (post_weights_from_params) and
529-570 (embed_weights_from_params), so directories written by either side
load in both.

A parameter tree here is haiku's: ``{module path: {param name: array}}``,
stacked modules carrying the block axis first.  ``load_params_npz`` reads an
AF2 ``.npz`` checkpoint into one (keys ``scope//name``, read with numpy's
pickle-free loader); ``init_af2_params`` draws a random one of the multimer
architecture.  Directories are cached on the content of the arrays (a hash of
names and leading bytes), never on a model name.
"""
import hashlib
import os
import tempfile

import numpy as np

from . import params as P

IT = "alphafold/alphafold_iteration"
EVO = f"{IT}/evoformer"
MAIN = f"{EVO}/evoformer_iteration"
EXTRA = f"{EVO}/extra_msa_stack"
TPE = f"{EVO}/template_embedding"
TEMPLATE_STACK = f"{TPE}/single_template_embedding/template_embedding_iteration"
STRUCTURE = f"{IT}/structure_module"
HEADS = ("distogram_head", "predicted_aligned_error_head", "predicted_lddt_head",
         "experimentally_resolved_head")
EMBED_LEAVES = ("preprocess_1d", "preprocess_msa", "left_single", "right_single",
                "position_activations")
# the one-call design step reads these: the single projection, the template
# row's two Linears and the three recycle terms (bindcraft/af/native.py:521-524
# lists them with the embedder's)
EMBED_OPTIONAL = ("single_activations", "prev_pos_linear", "prev_msa_first_row_norm",
                  "prev_pair_norm", "template_single_embedding", "template_projection")
IPA_HEADS = 12


# ------------------------------------------------------------------ reading

def load_params_npz(path):
    """An AF2 checkpoint (``params_model_*.npz``: flat ``scope//name`` keys)
    as a haiku tree.  numpy's loader runs with allow_pickle=False."""
    tree = {}
    with np.load(path, allow_pickle=False) as z:
        for key in z.files:
            scope, name = key.split("//", 1)
            tree.setdefault(scope, {})[name] = np.asarray(z[key])
    return tree


def save_params_npz(path, tree):
    """Inverse of load_params_npz."""
    flat = {f"{scope}//{name}": np.asarray(v) for scope, d in tree.items() for name, v in d.items()}
    np.savez(path, **flat)


def fuse_trimul_projections(tree):
    """Older checkpoints keep a triangle multiplication's left/right
    projections and gates as separate Linears (and name its norms
    layer_norm_input / center_layer_norm); the library takes the fused form
    (modules.py:1044-1088: one `projection` and one `gate` whose output halves
    are left then right, `left_norm_input`, `center_norm`).  Returns a new tree;
    only scopes whose parent is a triangle_multiplication_* module change (the
    outer product mean also has left/right_projection and layer_norm_input)."""
    out = {}
    pending = {}
    for scope, d in tree.items():
        parent, _, leaf = scope.rpartition("/")
        if not parent.rpartition("/")[2].startswith("triangle_multiplication_"):
            out[scope] = d
            continue
        if leaf == "layer_norm_input":
            out[f"{parent}/left_norm_input"] = d
        elif leaf == "center_layer_norm":
            out[f"{parent}/center_norm"] = d
        elif leaf in ("left_projection", "right_projection", "left_gate", "right_gate"):
            pending[scope] = d
        else:
            out[scope] = d
    for scope, d in pending.items():
        parent, _, leaf = scope.rpartition("/")
        if not leaf.startswith("left_"):
            continue
        kind = leaf[len("left_"):]
        right = pending.get(f"{parent}/right_{kind}")
        if right is None:
            raise KeyError(f"{scope} has no right_{kind} partner")
        out[f"{parent}/{kind}"] = {k: np.concatenate([np.asarray(v), np.asarray(right[k])], -1)
                                   for k, v in d.items()}
    return out


# ------------------------------------------------------------------ writing

def write_dir(flat, out_dir=None, tag="bc2n"):
    """Write {manifest name: array} as a weights directory.  Without out_dir
    the directory is ``<tmp>/<tag>_<content hash>`` and an existing one is
    reused as is."""
    flat = {k: np.ascontiguousarray(np.asarray(v, np.float32)) for k, v in flat.items()}
    if out_dir is None:
        h = hashlib.sha1()
        for k in sorted(flat):
            h.update(k.encode())
            h.update(str(flat[k].shape).encode())
            h.update(flat[k].tobytes()[:4096])
        out_dir = os.path.join(tempfile.gettempdir(), f"{tag}_{h.hexdigest()[:16]}")
        if os.path.exists(os.path.join(out_dir, "manifest.txt")):
            return out_dir
    return P.write_manifest(out_dir, flat)


def _scoped(tree, prefix):
    mods = {k: v for k, v in tree.items() if k == prefix or k.startswith(prefix + "/")}
    if not mods:
        raise KeyError(f"no {prefix}* in these params")
    return mods


def stack_flat(tree, prefix=MAIN, depth=None):
    """{param/block{b}/<path>/<param>: array} of a layer stack under `prefix`
    (the stacked axis first); depth defaults to the shortest stacked axis."""
    tree = fuse_trimul_projections(tree)
    mods = _scoped(tree, prefix)
    if depth is None:
        depth = min(int(np.asarray(a).shape[0]) for d in mods.values() for a in d.values())
    flat = {}
    for mod, d in mods.items():
        path = mod[len(prefix) + 1:]
        for pname, v in d.items():
            w = np.asarray(v, np.float32)
            if w.shape[0] < depth:
                raise ValueError(f"{mod}/{pname}: {w.shape[0]} blocks < depth {depth}")
            for b in range(depth):
                key = f"param/block{b}/{path}/{pname}" if path else f"param/block{b}/{pname}"
                flat[key] = w[b]
    return flat


def stack_weights_from_params(tree, out_dir=None, depth=None, prefix=MAIN):
    """The directory of a layer stack: the main Evoformer stack (MAIN), the
    extra-MSA stack (EXTRA) or the template pair stack (TEMPLATE_STACK)."""
    return write_dir(stack_flat(tree, prefix, depth), out_dir, "bc2n_stack")


def tplembed_flat(tree):
    """The template embedding: its stack's blocks plus the modules around it
    (query_embedding_norm, template_pair_embedding_0..8, output_layer_norm
    under single_template_embedding/, output_linear one scope up)."""
    flat = stack_flat(tree, TEMPLATE_STACK)
    around = {f"{TPE}/single_template_embedding/query_embedding_norm": "query_embedding_norm",
              f"{TPE}/single_template_embedding/output_layer_norm": "output_layer_norm",
              f"{TPE}/output_linear": "output_linear"}
    around.update({f"{TPE}/single_template_embedding/template_pair_embedding_{i}":
                   f"template_pair_embedding_{i}" for i in range(9)})
    for scope, leaf in around.items():
        if scope not in tree:
            if leaf.startswith("template_pair_embedding_") and leaf != "template_pair_embedding_8":
                continue  # the constant eight are the caller's (act_const)
            raise KeyError(f"template embedding: no {scope} in these params")
        for pname, v in tree[scope].items():
            flat[f"param/{leaf}/{pname}"] = np.asarray(v, np.float32)
    return flat


def tplembed_weights_from_params(tree, out_dir=None):
    return write_dir(tplembed_flat(tree), out_dir, "bc2n_tpe")


def embed_flat(tree):
    """The embedder's five Linears, matched on the leaf of the module path:
    position_activations sits under evoformer/~_relative_encoding/ (haiku's
    method scope), its siblings directly under evoformer/."""
    flat = {}
    for mod, d in tree.items():
        if not mod.startswith(EVO + "/"):
            continue
        leaf = mod.rpartition("/")[2]
        if leaf not in EMBED_LEAVES + EMBED_OPTIONAL:
            continue
        for pname, v in d.items():
            flat[f"param/{leaf}/{pname}"] = np.asarray(v, np.float32)
    missing = [l for l in EMBED_LEAVES if f"param/{l}/weights" not in flat]
    if missing:
        raise KeyError(f"embedder: no {', '.join(missing)} in these params")
    if flat["param/preprocess_1d/weights"].shape[0] != 21:
        raise ValueError("embedder: preprocess_1d must be 21 wide (the multimer model)")
    return flat


def embed_weights_from_params(tree, out_dir=None):
    return write_dir(embed_flat(tree), out_dir, "bc2n_emb")


def _monomer_ipa_to_multimer(flat):
    """A monomer IPA keeps q/kv scalar projections as [C, H*per] Linears and
    the point projections as [C, 3*H*P] (x block, y block, z block, each head
    by point); the multimer form is per projection [C, H, per] and, for points,
    [C, H, 3*P] (per head: x points, y points, z points).  k and v share the
    monomer's kv Linears (k first).  Biases follow their weights."""
    ipa = "param/fold_iteration/invariant_point_attention/"
    H = IPA_HEADS
    for src, parts in (("q_scalar", (("q_scalar_projection", 16),)),
                       ("kv_scalar", (("k_scalar_projection", 16), ("v_scalar_projection", 16)))):
        if f"{ipa}{src}/weights" not in flat:
            continue
        w, b = flat.pop(f"{ipa}{src}/weights"), flat.pop(f"{ipa}{src}/bias")
        c = w.shape[0]
        w, b = w.reshape(c, H, -1), b.reshape(H, -1)
        o = 0
        for dst, n in parts:
            flat[f"{ipa}{dst}/weights"] = w[:, :, o:o + n]
            flat[f"{ipa}{dst}/bias"] = b[:, o:o + n].reshape(-1)
            o += n
    for src, parts in (("q_point_local", (("q_point_projection", 4),)),
                       ("kv_point_local", (("k_point_projection", 4), ("v_point_projection", 8)))):
        if f"{ipa}{src}/weights" not in flat:
            continue
        w, b = flat.pop(f"{ipa}{src}/weights"), flat.pop(f"{ipa}{src}/bias")
        c = w.shape[0]
        w = w.reshape(c, 3, H, -1).transpose(0, 2, 1, 3)   # [C, H, xyz, points]
        b = b.reshape(3, H, -1).transpose(1, 0, 2)
        o = 0
        for dst, n in parts:
            flat[f"{ipa}{dst}/point_projection/weights"] = w[:, :, :, o:o + n].reshape(c, H, 3 * n)
            flat[f"{ipa}{dst}/point_projection/bias"] = b[:, :, o:o + n].reshape(H, 3 * n)
            o += n
    au, qr = "param/fold_iteration/affine_update/", "param/fold_iteration/quat_rigid/rigid/"
    if f"{au}weights" in flat:
        flat[f"{qr}weights"] = flat.pop(f"{au}weights")
        flat[f"{qr}bias"] = flat.pop(f"{au}bias")


def post_flat(tree):
    """Structure module and heads: ``param/<path below structure_module or
    below alphafold_iteration for a head>/<param>``, no block index (the fold
    iterations share one set).  A monomer IPA is rewritten to the multimer
    layout, and the q/k/v scalar projections, built with biases that no
    checkpoint carries (trained at zero), get zero biases."""
    flat = {}
    for mod, d in tree.items():
        if mod == STRUCTURE or mod.startswith(STRUCTURE + "/"):
            path = mod[len(STRUCTURE) + 1:]
        elif mod.startswith(IT + "/") and mod[len(IT) + 1:].split("/")[0] in HEADS:
            path = mod[len(IT) + 1:]
        else:
            continue
        for pname, v in d.items():
            flat[f"param/{path}/{pname}" if path else f"param/{pname}"] = np.asarray(v, np.float32)
    if not flat:
        raise KeyError("no structure_module or head parameters in these params")
    _monomer_ipa_to_multimer(flat)
    for m in ("q_scalar_projection", "k_scalar_projection", "v_scalar_projection"):
        wk = f"param/fold_iteration/invariant_point_attention/{m}/weights"
        bk = wk[:-len("weights")] + "bias"
        if wk in flat and bk not in flat:
            flat[bk] = np.zeros(int(np.prod(flat[wk].shape[1:])), np.float32)
    return flat


def post_weights_from_params(tree, out_dir=None, tables=None):
    """The post-trunk directory; `tables` (params.residue_tables_from(the
    model's residue_constants), or any dict of the arrays) adds the residue
    tables the sidechain reads (const/default_frame, const/atom14_to_group,
    const/atom14_lit_pos, const/atom14_mask) and, where the dict has them,
    the design step's atom37 (const/atom37_to_atom14, const/atom37_mask) and
    template-row chi tables (const/chi_atom_indices, const/chi_angles_mask)."""
    flat = post_flat(tree)
    if tables is not None:
        for k in ("default_frame", "atom14_to_group", "atom14_lit_pos", "atom14_mask"):
            flat[f"const/{k}"] = np.asarray(tables[k], np.float32)
        for k in ("atom37_to_atom14", "atom37_mask", "chi_atom_indices", "chi_angles_mask"):
            if k in tables:
                flat[f"const/{k}"] = np.asarray(tables[k], np.float32)
    return write_dir(flat, out_dir, "bc2n_post")


# ------------------------------------------------------------- random trees

def _unflatten(flat, prefix, stacked_from=None):
    """{"<module>/<path>/<param>": array} -> haiku scopes below `prefix`."""
    tree = {}
    for name, v in flat.items():
        path, _, pname = name.rpartition("/")
        tree.setdefault(f"{prefix}/{path}" if path else prefix, {})[pname] = v
    return tree


def _stack(block_dicts):
    keys = block_dicts[0].keys()
    return {k: np.stack([d[k] for d in block_dicts]) for k in keys}


def init_af2_params(rng, num_blocks=48, extra_blocks=4, template_blocks=2, gates="zero",
                    ln="identity"):
    """A random haiku tree of the AF2 multimer architecture (config.py:386-600)
    for every part the library runs: the main stack, the extra-MSA stack
    (c_e = 64, global column attention), the template embedding with its
    stack, the embedder, the structure module with its sidechain, and the
    four heads.  Weights are LeCun normal;
    gates/ln as for params.init_module."""
    tree = {}

    def stack(prefix, n, shapes):
        blocks = []
        for _ in range(n):
            d = {}
            for mod, sh in shapes.items():
                for pname, arr in P.init_module(sh, rng, gates, ln).items():
                    d[f"{mod}/{pname}"] = arr
            blocks.append(d)
        if n:
            tree.update(_unflatten(_stack(blocks), prefix))

    stack(MAIN, num_blocks, P.module_shapes())
    ex = P.module_shapes(c_m=P.C_E)
    ex.pop("msa_column_attention")
    ex["msa_column_global_attention"] = P.global_attention_shapes(P.C_E)
    stack(EXTRA, extra_blocks, ex)
    tsh = P.module_shapes(c_z=P.C_T, tri_heads=4, trimul_hidden=64)
    tsh["pair_transition"] = {"input_layer_norm/scale": (P.C_T,),
                              "input_layer_norm/offset": (P.C_T,),
                              "transition1/weights": (P.C_T, 2 * P.C_T),
                              "transition1/bias": (2 * P.C_T,),
                              "transition2/weights": (2 * P.C_T, P.C_T),
                              "transition2/bias": (P.C_T,)}
    stack(TEMPLATE_STACK, template_blocks, {m: tsh[m] for m in P.TEMPLATE_MODULES})

    around = P.init_module(P.template_embedding_shapes(), rng, gates, ln)
    for pname, arr in around.items():
        mod, _, leaf = pname.rpartition("/")
        scope = f"{TPE}/{mod}" if mod == "output_linear" else f"{TPE}/single_template_embedding/{mod}"
        tree.setdefault(scope, {})[leaf] = arr
    # the constant eight (modules_multimer.py:867-925): dgram 39, the pseudo-
    # beta mask, aatype one-hots 22 (two), unit vector x, y, z, backbone mask
    const_in = {0: (39,), 1: (), 2: (22,), 3: (22,), 4: (), 5: (), 6: (), 7: ()}
    for i, din in const_in.items():
        w = rng.standard_normal(din + (P.C_T,)) / np.sqrt(din[0] if din else 1)
        tree[f"{TPE}/single_template_embedding/template_pair_embedding_{i}"] = {
            "weights": w.astype(np.float32), "bias": np.zeros(P.C_T, np.float32)}

    for name, arr in P.init_embedder_params(rng, scoped=True).items():
        path, _, leaf = name[len("param/"):].rpartition("/")
        tree.setdefault(f"{EVO}/{path}", {})[leaf] = arr

    for name, arr in P.init_structure_heads_params(
            rng, final="zero" if gates == "zero" else "random", ln=ln).items():
        path, _, leaf = name[len("param/"):].rpartition("/")
        root = IT if path.split("/")[0] in HEADS else STRUCTURE
        tree.setdefault(f"{root}/{path}", {})[leaf] = arr
    return tree
