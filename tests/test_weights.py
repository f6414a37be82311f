"""AF2 parameter trees -> weights directories (bindcraft2_amd/weights.py, the
restatement of bindcraft/af/native.py:171-226, 264-323, 339-444, 529-570).
CPU only: names, shapes and values of every directory the library reads,
the fused-trimul and monomer-IPA rewrites against per-element formulas, the
npz loader and the content-keyed cache."""
import os

import numpy as np
import pytest

from bindcraft2_amd import params as P
from bindcraft2_amd import weights as W


@pytest.fixture(scope="module")
def tree():
    return W.init_af2_params(np.random.default_rng(0), num_blocks=2, extra_blocks=1,
                             template_blocks=2, gates="random", ln="random")


def _names_shapes(flat):
    return {k: tuple(np.shape(v)) for k, v in flat.items()}


def test_main_stack_names_shapes_values(tree):
    flat = W.stack_flat(tree, W.MAIN)
    want = {}
    for b in range(2):
        want.update(P.init_block_params(b, np.random.default_rng(1)))
    assert _names_shapes(flat) == _names_shapes(want)
    scope = f"{W.MAIN}/triangle_multiplication_outgoing/projection"
    np.testing.assert_array_equal(
        flat["param/block1/triangle_multiplication_outgoing/projection/weights"],
        tree[scope]["weights"][1])


def test_extra_and_template_stacks(tree):
    ex = W.stack_flat(tree, W.EXTRA)
    sh = P.module_shapes(c_m=P.C_E)
    sh.pop("msa_column_attention")
    sh["msa_column_global_attention"] = P.global_attention_shapes(P.C_E)
    want = {f"param/block0/{m}/{p}": s for m, d in sh.items() for p, s in d.items()}
    assert _names_shapes(ex) == want
    tp = W.stack_flat(tree, W.TEMPLATE_STACK)
    want = {}
    for b in range(2):
        want.update(P.init_template_block_params(b, np.random.default_rng(1)))
    assert _names_shapes(tp) == _names_shapes(want)
    with pytest.raises(ValueError):
        W.stack_flat(tree, W.TEMPLATE_STACK, depth=3)


def test_template_embedding_embedder_post(tree):
    te = W.tplembed_flat(tree)
    for name, shape in P.template_embedding_shapes().items():
        assert te[f"param/{name}"].shape == shape
    assert te["param/template_pair_embedding_0/weights"].shape == (39, 64)
    assert te["param/template_pair_embedding_1/weights"].shape == (64,)
    assert "param/block1/pair_transition/transition1/weights" in te
    em = W.embed_flat(tree)
    want = {**P.embedder_shapes(), **P.single_activations_shapes(), **P.recycle_shapes(),
            **P.template_row_shapes()}
    assert _names_shapes(em) == {f"param/{k}": v for k, v in want.items()}
    po = W.post_flat(tree)
    want = {**P.fold_shapes(), **P.sidechain_shapes(), **P.heads_shapes()}
    assert _names_shapes(po) == {f"param/{k}": v for k, v in want.items()}


def test_post_zero_scalar_biases(tree):
    t = {k: dict(v) for k, v in tree.items()}
    for m in ("q", "k", "v"):
        del t[f"{W.STRUCTURE}/fold_iteration/invariant_point_attention/{m}_scalar_projection"]["bias"]
    po = W.post_flat(t)
    for m in ("q", "k", "v"):
        b = po[f"param/fold_iteration/invariant_point_attention/{m}_scalar_projection/bias"]
        assert b.shape == (192,) and not b.any()


def test_fuse_trimul_projections_leaves_opm():
    rng = np.random.default_rng(2)
    base = f"{W.MAIN}/triangle_multiplication_incoming"
    lw, rw = rng.standard_normal((3, 128, 5)), rng.standard_normal((3, 128, 5))
    lb, rb = rng.standard_normal((3, 5)), rng.standard_normal((3, 5))
    opm = {"weights": rng.standard_normal((3, 256, 32)), "bias": rng.standard_normal((3, 32))}
    t = {f"{base}/left_projection": {"weights": lw, "bias": lb},
         f"{base}/right_projection": {"weights": rw, "bias": rb},
         f"{base}/left_gate": {"weights": lw + 1, "bias": lb + 1},
         f"{base}/right_gate": {"weights": rw + 1, "bias": rb + 1},
         f"{base}/layer_norm_input": {"scale": np.ones((3, 128))},
         f"{base}/center_layer_norm": {"scale": np.ones((3, 5))},
         f"{W.MAIN}/outer_product_mean/left_projection": opm,
         f"{W.MAIN}/outer_product_mean/layer_norm_input": {"scale": np.ones((3, 256))}}
    f = W.fuse_trimul_projections(t)
    pw = f[f"{base}/projection"]["weights"]
    assert pw.shape == (3, 128, 10)
    for j in range(10):  # output column j: left's j for j < 5, right's j - 5 after
        src = lw[..., j] if j < 5 else rw[..., j - 5]
        np.testing.assert_array_equal(pw[..., j], src)
    np.testing.assert_array_equal(f[f"{base}/gate"]["bias"][:, 7], rb[:, 2] + 1)
    assert f"{base}/left_norm_input" in f and f"{base}/center_norm" in f
    assert f[f"{W.MAIN}/outer_product_mean/left_projection"] is opm
    assert f"{W.MAIN}/outer_product_mean/layer_norm_input" in f


def test_monomer_ipa_rewrite_per_element():
    """Monomer q_point_local output index a*H*P + h*P + p (coordinate a of
    point p of head h, modules.py's split into x, y, z blocks) must land at
    multimer [h][a*P + p]; kv_scalar output h*32 + j is k's j < 16, v's
    j - 16 after."""
    rng = np.random.default_rng(3)
    H, C = 12, 384
    ipa = f"{W.STRUCTURE}/fold_iteration/invariant_point_attention"
    qp = rng.standard_normal((C, 3 * H * 4)).astype(np.float32)
    kvp = rng.standard_normal((C, 3 * H * 12)).astype(np.float32)
    kvs = rng.standard_normal((C, H * 32)).astype(np.float32)
    t = {f"{ipa}/q_point_local": {"weights": qp, "bias": qp[0]},
         f"{ipa}/kv_point_local": {"weights": kvp, "bias": kvp[1]},
         f"{ipa}/kv_scalar": {"weights": kvs, "bias": kvs[2]},
         f"{W.STRUCTURE}/fold_iteration/affine_update": {"weights": np.ones((C, 6)),
                                                        "bias": np.zeros(6)}}
    po = W.post_flat(t)
    q = po["param/fold_iteration/invariant_point_attention/q_point_projection/point_projection/weights"]
    k = po["param/fold_iteration/invariant_point_attention/k_point_projection/point_projection/weights"]
    v = po["param/fold_iteration/invariant_point_attention/v_point_projection/point_projection/bias"]
    for h in range(H):
        for a in range(3):
            for p in range(4):
                assert q[5, h, a * 4 + p] == qp[5, a * H * 4 + h * 4 + p]
                assert k[7, h, a * 4 + p] == kvp[7, a * H * 12 + h * 12 + p]
            for p in range(8):
                assert v[h, a * 8 + p] == kvp[1, a * H * 12 + h * 12 + 4 + p]
    ks = po["param/fold_iteration/invariant_point_attention/k_scalar_projection/weights"]
    vs = po["param/fold_iteration/invariant_point_attention/v_scalar_projection/bias"]
    assert ks[9, 3, 5] == kvs[9, 3 * 32 + 5]
    assert vs[4 * 16 + 2] == kvs[2, 4 * 32 + 16 + 2]
    assert "param/fold_iteration/quat_rigid/rigid/weights" in po


def test_npz_round_trip_and_cache(tree, tmp_path):
    path = os.path.join(tmp_path, "params_model_test.npz")
    W.save_params_npz(path, tree)
    back = W.load_params_npz(path)
    assert back.keys() == tree.keys()
    for scope in tree:
        for k in tree[scope]:
            np.testing.assert_array_equal(back[scope][k], tree[scope][k])
    d1 = W.embed_weights_from_params(back)
    d2 = W.embed_weights_from_params(tree)
    assert d1 == d2
    got = P.read_manifest(d1)
    for k, v in W.embed_flat(tree).items():
        np.testing.assert_array_equal(got[k], v)
    out = W.stack_weights_from_params(tree, out_dir=os.path.join(tmp_path, "main"))
    assert len(P.read_manifest(out)) == len(W.stack_flat(tree))
