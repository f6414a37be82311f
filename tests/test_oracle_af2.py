"""Pins oracle/af2.py against closed forms, invariants and finite differences."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import params as bparams
from oracle import af2

DT = torch.float64


def _block(rng, mods=None, gates="random", ln="random", **kw):
    return bparams.init_block_params(0, rng, modules=mods, gates=gates, ln=ln, **kw)


def test_layer_norm_matches_torch():
    rng = np.random.default_rng(0)
    x = torch.as_tensor(rng.standard_normal((7, 128)) * 3 + 1, dtype=DT)
    g = torch.as_tensor(rng.standard_normal(128), dtype=DT)
    b = torch.as_tensor(rng.standard_normal(128), dtype=DT)
    ref = torch.nn.functional.layer_norm(x, (128,), g, b, eps=1e-5)
    torch.testing.assert_close(af2.layer_norm(x, g, b), ref, rtol=1e-12, atol=1e-12)
    # fast variance is the same function in exact arithmetic
    torch.testing.assert_close(af2.layer_norm(x, g, b, fast=True), ref, rtol=1e-9, atol=1e-9)


def _loop_attention(q_data, bias, nb, P):
    """Pure-Python loops over (b, q, h): softmax(q.k/sqrt(d) + bias) v."""
    qw, kw, vw = P("attention/query_w"), P("attention/key_w"), P("attention/value_w")
    B, Q, A = q_data.shape
    H, D = qw.shape[1], qw.shape[2]
    out = torch.zeros(B, Q, H, D, dtype=DT)
    for b in range(B):
        for i in range(Q):
            for h in range(H):
                q = sum(q_data[b, i, a] * qw[a, h] for a in range(A)) / D ** 0.5
                logits = []
                for j in range(Q):
                    k = sum(q_data[b, j, a] * kw[a, h] for a in range(A))
                    lg = float(torch.dot(q, k)) + float(bias[b, 0, 0, j]) + float(nb[h, i, j])
                    logits.append(min(max(lg, -1e8), 1e8))
                m = max(logits)
                w = [np.exp(x - m) for x in logits]
                s = sum(w)
                acc = torch.zeros(D, dtype=DT)
                for j in range(Q):
                    v = sum(q_data[b, j, a] * vw[a, h] for a in range(A))
                    acc += w[j] / s * v
                g = torch.sigmoid(sum(q_data[b, i, a] * P("attention/gating_w")[a, h]
                                      for a in range(A)) + P("attention/gating_b")[h])
                out[b, i, h] = acc * g
    return torch.einsum("bqhc,hco->bqo", out, P("attention/output_w")) + P("attention/output_b")


def test_attention_matches_loops():
    rng = np.random.default_rng(1)
    shapes = bparams.module_shapes(c_z=8, tri_heads=2)["triangle_attention_starting_node"]
    prm = {f"x/{k}": v for k, v in bparams.init_module(shapes, rng, "random", "random").items()}
    P = af2.Params(prm, "x/")
    q = torch.as_tensor(rng.standard_normal((2, 5, 8)), dtype=DT)
    mask = torch.ones(2, 5, dtype=DT)
    mask[1, 3] = 0
    bias = (1e9 * (mask - 1))[:, None, None, :]
    nb = torch.as_tensor(rng.standard_normal((2, 5, 5)), dtype=DT)
    torch.testing.assert_close(af2.attention(q, q, bias, nb, P), _loop_attention(q, bias, nb, P),
                               rtol=1e-10, atol=1e-10)


def test_fully_masked_row_attends_uniformly():
    rng = np.random.default_rng(2)
    shapes = bparams.module_shapes(c_z=8, tri_heads=2)["triangle_attention_starting_node"]
    prm = {f"x/{k}": v for k, v in bparams.init_module(shapes, rng, "random", "random").items()}
    P = af2.Params(prm, "x/")
    q = torch.as_tensor(rng.standard_normal((1, 6, 8)), dtype=DT)
    bias = torch.full((1, 1, 1, 6), -1e9, dtype=DT)
    out = af2.attention(q, q, bias, None, P)
    v = torch.einsum("bka,ahc->bkhc", q, P("attention/value_w")).mean(1, keepdim=True)
    g = torch.sigmoid(torch.einsum("bqc,chv->bqhv", q, P("attention/gating_w")) + P("attention/gating_b"))
    ref = torch.einsum("bqhc,hco->bqo", v * g, P("attention/output_w")) + P("attention/output_b")
    torch.testing.assert_close(out, ref, rtol=1e-10, atol=1e-10)


def test_ending_node_is_starting_node_on_transpose():
    rng = np.random.default_rng(3)
    prm = _block(rng, ["triangle_attention_starting_node"], c_z=16, tri_heads=2)
    P = af2.Params(prm, "param/block0/triangle_attention_starting_node/")
    pair = torch.as_tensor(rng.standard_normal((6, 6, 16)), dtype=DT)
    mask = torch.as_tensor((rng.random((6, 6)) > 0.2).astype(np.float64))
    end = af2.triangle_attention(pair, mask, P, per_column=True)
    start_t = af2.triangle_attention(pair.transpose(0, 1), mask.T, P, per_column=False)
    torch.testing.assert_close(end, start_t.transpose(0, 1), rtol=1e-12, atol=1e-12)


def test_incoming_is_outgoing_on_transpose():
    rng = np.random.default_rng(4)
    prm = _block(rng, ["triangle_multiplication_outgoing"], c_z=16, trimul_hidden=8)
    P = af2.Params(prm, "param/block0/triangle_multiplication_outgoing/")
    pair = torch.as_tensor(rng.standard_normal((7, 7, 16)), dtype=DT)
    mask = torch.as_tensor((rng.random((7, 7)) > 0.2).astype(np.float64))
    inc = af2.triangle_multiplication(pair, mask, P, outgoing=False)
    out_t = af2.triangle_multiplication(pair.transpose(0, 1), mask.T, P, outgoing=True)
    torch.testing.assert_close(inc, out_t.transpose(0, 1), rtol=1e-10, atol=1e-10)


def test_trimul_contraction_direct_sum():
    """outgoing T[i,j,c] = sum_k a[i,k,c] b[j,k,c] checked by explicit loops."""
    rng = np.random.default_rng(5)
    prm = _block(rng, ["triangle_multiplication_outgoing"], c_z=8, trimul_hidden=4)
    P = af2.Params(prm, "param/block0/triangle_multiplication_outgoing/")
    pair = torch.as_tensor(rng.standard_normal((5, 5, 8)), dtype=DT)
    mask = torch.ones(5, 5, dtype=DT)
    x = af2.layer_norm(pair, P("left_norm_input/scale"), P("left_norm_input/offset"), fast=True)
    proj = af2.linear(x, P.sub("projection/")) * torch.sigmoid(af2.linear(x, P.sub("gate/")))
    a, b = proj[..., :4], proj[..., 4:]
    T = torch.zeros(5, 5, 4, dtype=DT)
    for i in range(5):
        for j in range(5):
            for k in range(5):
                T[i, j] += a[i, k] * b[j, k]
    T = af2.layer_norm(T, P("center_norm/scale"), P("center_norm/offset"), fast=True)
    ref = af2.linear(T, P.sub("output_projection/")) * torch.sigmoid(af2.linear(x, P.sub("gating_linear/")))
    torch.testing.assert_close(af2.triangle_multiplication(pair, mask, P, True), ref, rtol=1e-10, atol=1e-10)


def test_opm_direct_sum_and_masked_constant():
    rng = np.random.default_rng(6)
    prm = _block(rng, ["outer_product_mean"], c_z=8, c_m=12, opm_c=3)
    P = af2.Params(prm, "param/block0/outer_product_mean/")
    msa = torch.as_tensor(rng.standard_normal((2, 4, 12)), dtype=DT)
    mask = torch.as_tensor([[1, 1, 0, 1], [1, 0, 1, 1]], dtype=DT)
    out = af2.outer_product_mean(msa, mask, P)
    x = af2.layer_norm(msa, P("layer_norm_input/scale"), P("layer_norm_input/offset"))
    L = mask[..., None] * af2.linear(x, P.sub("left_projection/"))
    R = mask[..., None] * af2.linear(x, P.sub("right_projection/"))
    W, bo = P("output_w"), P("output_b")
    ref = torch.zeros(4, 4, 8, dtype=DT)
    for i in range(4):
        for j in range(4):
            acc = torch.zeros(8, dtype=DT)
            for s in range(2):
                for c in range(3):
                    for e in range(3):
                        acc += L[s, i, c] * R[s, j, e] * W[c, e]
            norm = float((mask[:, i] * mask[:, j]).sum())
            ref[i, j] = (acc + bo) / (1e-3 + norm)
    torch.testing.assert_close(out, ref, rtol=1e-10, atol=1e-10)
    zero = af2.outer_product_mean(msa, torch.zeros_like(mask), P)
    torch.testing.assert_close(zero, (bo / 1e-3).expand(4, 4, 8), rtol=1e-12, atol=1e-12)


def test_column_attention_single_row_closed_form():
    rng = np.random.default_rng(7)
    prm = _block(rng, ["msa_column_attention"], c_m=16, col_heads=2)
    P = af2.Params(prm, "param/block0/msa_column_attention/")
    msa = torch.as_tensor(rng.standard_normal((1, 5, 16)), dtype=DT)
    mask = torch.ones(1, 5, dtype=DT)
    out = af2.msa_column_attention(msa, mask, P)
    x = af2.layer_norm(msa, P("query_norm/scale"), P("query_norm/offset"))
    v = torch.einsum("bka,ahc->bkhc", x, P("attention/value_w"))
    g = torch.sigmoid(torch.einsum("bqc,chv->bqhv", x, P("attention/gating_w")) + P("attention/gating_b"))
    ref = torch.einsum("bqhc,hco->bqo", v * g, P("attention/output_w")) + P("attention/output_b")
    torch.testing.assert_close(out, ref, rtol=1e-10, atol=1e-10)


def test_dropout_wrapper_rate_zero_and_table():
    from oracle import jax_prng as J
    rng = np.random.default_rng(8)
    t = torch.as_tensor(rng.standard_normal((4, 6, 3)), dtype=DT)
    key = J.prng_key(9)
    assert torch.equal(af2.apply_dropout(t, key, 0.0, 0), t)
    out = af2.apply_dropout(t, key, 0.25, 0)
    tbl = torch.as_tensor(af2.dropout_table(key, 0.25, 6, 3), dtype=DT)
    torch.testing.assert_close(out, t * tbl[None], rtol=1e-6, atol=0)
    keep = J.bernoulli(key, J.keep_rate(0.25), (1, 6, 3))
    assert np.array_equal((tbl.numpy() > 0), keep[0])


@pytest.mark.parametrize("per_column", [False, True])
def test_triangle_attention_grad_finite_differences(per_column):
    rng = np.random.default_rng(10)
    prm = _block(rng, ["triangle_attention_starting_node"], c_z=8, tri_heads=2)
    P = af2.Params(prm, "param/block0/triangle_attention_starting_node/")
    pair = torch.tensor(rng.standard_normal((4, 4, 8)), dtype=DT, requires_grad=True)
    mask = torch.as_tensor((rng.random((4, 4)) > 0.25).astype(np.float64))
    w = torch.as_tensor(rng.standard_normal((4, 4, 8)), dtype=DT)
    f = lambda x: (af2.triangle_attention(x, mask, P, per_column) * w).sum()
    (g,) = torch.autograd.grad(f(pair), pair)
    eps = 1e-6
    with torch.no_grad():
        for idx in [(0, 1, 2), (3, 2, 7), (2, 0, 0), (1, 3, 5)]:
            e = torch.zeros_like(pair)
            e[idx] = eps
            fd = (f(pair + e) - f(pair - e)) / (2 * eps)
            assert abs(fd.item() - g[idx].item()) < 1e-6 * max(1.0, abs(fd.item()))


@pytest.mark.parametrize("per_column", [False, True])
def test_triangle_attention_chunked_vjp(per_column):
    """The row-chunked VJP (for lengths whose whole graph does not fit) equals
    autograd of the unchunked module times the dropout table, value and
    gradient, with chunks that do not divide N and a masked residue."""
    rng = np.random.default_rng(12)
    n = 11
    prm = _block(rng, ["triangle_attention_starting_node"], c_z=8, tri_heads=2)
    P = af2.Params(prm, "param/block0/triangle_attention_starting_node/")
    pair = torch.tensor(rng.standard_normal((n, n, 8)), dtype=DT, requires_grad=True)
    m = np.ones(n)
    m[4] = 0
    mask = torch.as_tensor(np.outer(m, m))
    tbl = torch.as_tensor((rng.random((n, 8)) > 0.25) / 0.75)
    dout = torch.as_tensor(rng.standard_normal((n, n, 8)), dtype=DT)
    sc = tbl[:, None] if per_column else tbl[None]
    ref = af2.triangle_attention(pair, mask, P, per_column) * sc
    (g,) = torch.autograd.grad(ref, pair, dout)
    for rows in (3, 4, n):
        d, gc = af2.triangle_attention_vjp(pair, mask, P, per_column, dout, tbl, rows=rows)
        torch.testing.assert_close(d, ref.detach(), rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(gc, g, rtol=1e-11, atol=1e-12)


def test_evoformer_block_runs_and_is_identity_for_zero_outputs():
    """All output layers zero => the block is the identity (sanity only)."""
    rng = np.random.default_rng(11)
    prm = bparams.init_block_params(0, rng, c_z=16, c_m=16, tri_heads=2, trimul_hidden=8,
                                    opm_c=4, row_heads=2, col_heads=2)
    for k in list(prm):
        if k.endswith(("output_w", "output_b", "output_projection/weights",
                       "output_projection/bias", "transition2/weights", "transition2/bias")):
            prm[k] = np.zeros_like(prm[k])
    msa = torch.as_tensor(rng.standard_normal((1, 6, 16)), dtype=DT)
    pair = torch.as_tensor(rng.standard_normal((6, 6, 16)), dtype=DT)
    m2, p2 = af2.evoformer_iteration(msa, pair, torch.ones(1, 6, dtype=DT), torch.ones(6, 6, dtype=DT),
                                     prm, "param/block0/", None, False)
    torch.testing.assert_close(m2, msa)
    torch.testing.assert_close(p2, pair)


# ------------------------------------------------------- structure module oracle
def _fold_params(seed=0):
    return bparams.init_fold_params(np.random.default_rng(seed), final="random", ln="random")


def test_quat_to_rot_is_a_rotation_and_matches_scipy():
    """rotation_matrix.py:117-140 against scipy's quaternion convention
    (scalar last) and orthonormality / det +1."""
    from scipy.spatial.transform import Rotation
    rng = np.random.default_rng(3)
    q = rng.standard_normal((20, 4))
    R = af2.quat_to_rot(*[torch.tensor(q[:, i]) for i in range(4)]).numpy()
    ref = Rotation.from_quat(q[:, [1, 2, 3, 0]]).as_matrix()
    assert np.abs(R - ref).max() < 1e-12
    assert np.abs(R @ R.transpose(0, 2, 1) - np.eye(3)).max() < 1e-12
    assert np.abs(np.linalg.det(R) - 1).max() < 1e-12


def test_ipa_invariant_under_global_rigid_motion():
    """IPA's defining property: moving every frame by one global rigid
    transform (R -> G R, t -> G t + g) leaves the output unchanged.  A
    transposed rotation in the point projection or the local readout breaks
    it."""
    prm = _fold_params(1)
    p = af2.Params(prm, "param/fold_iteration/invariant_point_attention/")
    rng = np.random.default_rng(4)
    n = 12
    act = torch.tensor(rng.standard_normal((n, 384)))
    a2d = torch.tensor(rng.standard_normal((n, n, 128)))
    mask = torch.ones(n, dtype=torch.float64)
    mask[3] = 0
    q = torch.tensor(rng.standard_normal((n, 4)))
    R = af2.quat_to_rot(q[:, 0], q[:, 1], q[:, 2], q[:, 3])
    t = torch.tensor(rng.standard_normal((n, 3)))
    o1 = af2.invariant_point_attention(act, a2d, mask, R, t, p)
    G = af2.quat_to_rot(*torch.tensor(rng.standard_normal(4)))
    g = torch.tensor(rng.standard_normal(3))
    o2 = af2.invariant_point_attention(act, a2d, mask, G @ R, t @ G.T + g, p)
    assert (o1 - o2).abs().max() < 1e-10 * o1.abs().max()
    # and it is not trivially constant in the frames: move one residue
    t3 = t.clone()
    t3[0] += 1.0
    o3 = af2.invariant_point_attention(act, a2d, mask, R, t3, p)
    assert (o1 - o3).abs().max() > 1e-3


def test_fold_grad_finite_differences():
    """fp64 autograd of the fold (frames carried across 2 iterations, no
    stop_gradient) against central differences on single and pair."""
    prm = _fold_params(2)
    rng = np.random.default_rng(5)
    n = 4
    s = torch.tensor(rng.standard_normal((n, 384)), requires_grad=True)
    z = torch.tensor(rng.standard_normal((n, n, 128)), requires_grad=True)
    m = torch.ones(n, dtype=torch.float64)
    w_act = torch.tensor(rng.standard_normal((n, 384)))
    w_traj = torch.tensor(rng.standard_normal((2, n, 3, 4)))

    def f(s_, z_):
        act, traj = af2.fold(s_, z_, m, prm, 2, None, False)
        return (act * w_act).sum() + (traj * w_traj).sum()

    gs, gz = torch.autograd.grad(f(s, z), (s, z))
    eps = 1e-6
    for (x, gx, idx) in ((s, gs, (1, 7)), (s, gs, (3, 300)), (z, gz, (0, 2, 5)), (z, gz, (3, 1, 100))):
        xp = x.detach().clone(); xp[idx] += eps
        xm = x.detach().clone(); xm[idx] -= eps
        fp = f(xp, z.detach()) if x is s else f(s.detach(), xp)
        fm = f(xm, z.detach()) if x is s else f(s.detach(), xm)
        fd = ((fp - fm) / (2 * eps)).item()
        assert abs(fd - gx[idx].item()) <= 1e-5 * max(1.0, abs(fd)), (idx, fd, gx[idx].item())


def _two_chain_ids(n1, n2, same_entity):
    ri = np.concatenate([np.arange(n1), np.arange(n2) + 3]).astype(np.float32)
    ai = np.concatenate([np.full(n1, 1), np.full(n2, 2)]).astype(np.float32)
    ei = np.concatenate([np.full(n1, 1), np.full(n2, 1 if same_entity else 2)]).astype(np.float32)
    si = np.concatenate([np.full(n1, 1), np.full(n2, 2 if same_entity else 1)]).astype(np.float32)
    return ri, ai, ei, si


@pytest.mark.parametrize("same_entity,use_offset", [(True, False), (False, False), (True, True)])
def test_relative_encoding_is_the_row_gather(same_entity, use_offset):
    """The one-hot concatenation times position_activations equals, per (i,j),
    W[rel] + [same entity] W[66] + W[67 + chain] + b with the bins written out
    by hand (the gather form of native/embed.cuh:58-103)."""
    rng = np.random.default_rng(11)
    prm = bparams.init_embedder_params(rng)
    W = prm["param/position_activations/weights"].astype(np.float64)
    b = prm["param/position_activations/bias"].astype(np.float64)
    ri, ai, ei, si = _two_chain_ids(40, 9, same_entity)
    ri[20:] += 50  # offsets beyond +-32 inside chain 1
    n = ri.shape[0]
    off = rng.integers(-40, 41, (n, n)).astype(np.int32) if use_offset else None
    got = af2.relative_encoding(ri, ai, ei, si, af2.Params(prm, "param/position_activations/"),
                                off).numpy()
    for i in range(n):
        for j in range(n):
            o = int(off[i, j]) if use_offset else int(ri[i]) - int(ri[j])
            rel = min(max(o + 32, 0), 64) if ai[i] == ai[j] else 65
            chain = min(max(int(si[i]) - int(si[j]) + 2, 0), 4) if ei[i] == ei[j] else 5
            want = W[rel] + (W[66] if ei[i] == ei[j] else 0) + W[67 + chain] + b
            np.testing.assert_allclose(got[i, j], want, rtol=0, atol=1e-12)
    # the bins the cases above must visit
    if not use_offset:
        assert (np.abs(ri[:20, None] - ri[None, 20:40]) > 32).all()


def test_embedder_structure_and_feature_mask():
    """msa[s,n] - preprocess_msa(mf)[s,n] is the same for every s and zero on
    a padded (all-zero) target_feat row; pair - relpos splits into a row term
    plus a column term; the gradients are the row/column sums and the S-sum
    (finite differences on a tiny case pin the autograd)."""
    rng = np.random.default_rng(12)
    prm = bparams.init_embedder_params(rng, scoped=True)
    n, s = 6, 3
    tf = np.zeros((n, 21))
    tf[:, :20] = rng.dirichlet(np.ones(20), n)
    tf[4] = 0.0  # padded residue
    mf = rng.standard_normal((s, n, 49))
    ri, ai, ei, si = _two_chain_ids(4, 2, False)
    T = lambda a: torch.tensor(a, dtype=torch.float64, requires_grad=True)
    tft, mft = T(tf), T(mf)
    msa, pair = af2.embedder(tft, mft, ri, ai, ei, si, prm)
    P = af2.Params(prm, "param/")
    premsa = af2.linear(torch.as_tensor(mf), P.sub("preprocess_msa/"))
    d = (msa - premsa).detach()
    assert torch.allclose(d, d[:1].expand_as(d), atol=1e-12)
    assert torch.count_nonzero(d[:, 4]) == 0 and torch.count_nonzero(d[:, 3]) > 0
    rel = af2.relative_encoding(ri, ai, ei, si, af2.Params(
        prm, "param/evoformer/~_relative_encoding/position_activations/"))
    q = (pair - rel).detach()
    assert torch.allclose(q, q[:, :1] + q[:1, :] - q[:1, :1], atol=1e-12)
    # gradient against central differences
    dm, dp = rng.standard_normal((s, n, 256)), rng.standard_normal((n, n, 128))
    loss = (msa * torch.as_tensor(dm)).sum() + (pair * torch.as_tensor(dp)).sum()
    gtf, gmf = torch.autograd.grad(loss, (tft, mft))

    def f(tf_, mf_):
        a, p = af2.embedder(torch.as_tensor(tf_), torch.as_tensor(mf_), ri, ai, ei, si, prm)
        return float((a * torch.as_tensor(dm)).sum() + (p * torch.as_tensor(dp)).sum())

    h = 1e-6
    for (i, k) in [(0, 3), (3, 20), (5, 7)]:
        e = np.zeros_like(tf); e[i, k] = h
        fd = (f(tf + e, mf) - f(tf - e, mf)) / (2 * h)
        assert abs(fd - gtf[i, k].item()) <= 1e-5 * max(1.0, abs(fd))
    for (t, i, k) in [(0, 0, 0), (2, 5, 48)]:
        e = np.zeros_like(mf); e[t, i, k] = h
        fd = (f(tf, mf + e) - f(tf, mf - e)) / (2 * h)
        assert abs(fd - gmf[t, i, k].item()) <= 1e-5 * max(1.0, abs(fd))


def _h4(R, t):
    m = np.eye(4)
    m[:3, :3], m[:3, 3] = R, t
    return m


def _xrot4(s, c):
    m = np.eye(4)
    m[1, 1], m[1, 2], m[2, 1], m[2, 2] = c, -s, s, c
    return m


def test_torsion_frames_and_atom14_against_homogeneous_products():
    """The 8 global frames equal products of 4x4 homogeneous matrices
    T_bb D_g X_g (chi2..4 chained: T_bb D4 X4 D5 X5 ...), and every atom is
    its group's frame applied to its literature position, masked."""
    rng = np.random.default_rng(31)
    tables = bparams.init_residue_tables(rng)
    n = 5
    aat = torch.as_tensor(rng.integers(0, 21, n))
    q, _ = np.linalg.qr(rng.standard_normal((n, 3, 3)))
    R = torch.as_tensor(q * np.sign(np.linalg.det(q))[:, None, None])
    t = torch.as_tensor(rng.standard_normal((n, 3)))
    ang = rng.standard_normal((n, 7, 2))
    ang /= np.linalg.norm(ang, axis=-1, keepdims=True)
    GR, Gt = af2.torsion_angles_to_frames(aat, R, t, torch.as_tensor(ang), tables)
    pos = af2.frames_to_atom14(aat, GR, Gt, tables).numpy()
    for i in range(n):
        a = int(aat[i])
        D = tables["default_frame"][a].astype(np.float64)
        X = [np.eye(4)] + [_xrot4(ang[i, g, 0], ang[i, g, 1]) for g in range(7)]
        T = _h4(R[i].numpy(), t[i].numpy())
        want = [T @ D[g] @ X[g] for g in range(5)]
        chain = D[4] @ X[4]
        for g in (5, 6, 7):
            chain = chain @ D[g] @ X[g]
            want.append(T @ chain)
        for g in range(8):
            np.testing.assert_allclose(GR[i, g].numpy(), want[g][:3, :3], atol=1e-12)
            np.testing.assert_allclose(Gt[i, g].numpy(), want[g][:3, 3], atol=1e-12)
        for k in range(14):
            g = int(tables["atom14_to_group"][a, k])
            lit = np.append(tables["atom14_lit_pos"][a, k].astype(np.float64), 1.0)
            p = (want[g] @ lit)[:3] * tables["atom14_mask"][a, k]
            np.testing.assert_allclose(pos[i, k], p, atol=1e-12)


def test_sidechain_rigid_equivariance_and_angle_scale():
    """A global rigid motion of the backbone frames moves every atom with it
    (a transposed rotation anywhere breaks this), and scaling the
    unnormalised angles changes nothing (they are l2-normalised)."""
    rng = np.random.default_rng(32)
    tables = bparams.init_residue_tables(rng)
    prm = bparams.init_structure_heads_params(rng)
    n = 6
    aat = torch.as_tensor(rng.integers(0, 21, n))
    q, _ = np.linalg.qr(rng.standard_normal((n, 3, 3)))
    R = torch.as_tensor(q * np.sign(np.linalg.det(q))[:, None, None])
    t = torch.as_tensor(rng.standard_normal((n, 3)))
    act = torch.as_tensor(rng.standard_normal((n, 384)))
    init = torch.as_tensor(rng.standard_normal((n, 384)))
    p = af2.Params(prm, "param/fold_iteration/rigid_sidechain/")
    pos = af2.multi_rigid_sidechain(R, t, act, init, aat, p, tables)
    Q, _ = np.linalg.qr(rng.standard_normal((3, 3)))
    Q = torch.as_tensor(Q * np.sign(np.linalg.det(Q)))
    u = torch.as_tensor(rng.standard_normal(3))
    pos2 = af2.multi_rigid_sidechain(Q @ R, (Q @ t[..., None])[..., 0] + u, act, init, aat, p, tables)
    mask = torch.as_tensor(tables["atom14_mask"], dtype=torch.float64)[aat][..., None]
    moved = ((Q @ pos[..., None])[..., 0] + u) * mask
    assert torch.allclose(pos2, moved, atol=1e-10)
    prm3 = dict(prm)
    for k in ("weights", "bias"):
        nm = f"param/fold_iteration/rigid_sidechain/unnormalized_angles/{k}"
        prm3[nm] = 3.0 * prm[nm]
    pos3 = af2.multi_rigid_sidechain(R, t, act, init, aat,
                                     af2.Params(prm3, "param/fold_iteration/rigid_sidechain/"), tables)
    assert torch.allclose(pos3, pos, atol=1e-10)


def test_structure_heads_symmetry_and_finite_differences():
    rng = np.random.default_rng(33)
    tables = bparams.init_residue_tables(rng)
    prm = bparams.init_structure_heads_params(rng, ln="random")
    n, depth = 5, 2
    single = rng.standard_normal((n, 384))
    pair = rng.standard_normal((n, n, 128))
    mask = np.ones(n)
    aat = rng.integers(0, 21, n).astype(np.float32)
    outs = af2.structure_heads(torch.as_tensor(single), torch.as_tensor(pair), torch.as_tensor(mask),
                               aat, prm, depth, None, False, tables)
    dgram, pae = outs[1], outs[2]
    assert torch.allclose(dgram, dgram.transpose(0, 1))
    assert not torch.allclose(pae, pae.transpose(0, 1))
    cts = [rng.standard_normal(tuple(o.shape)) for o in outs]

    def f(s_, z_):
        o = af2.structure_heads(torch.as_tensor(s_), torch.as_tensor(z_), torch.as_tensor(mask), aat,
                                prm, depth, None, False, tables)
        return sum(float((a * torch.as_tensor(c)).sum()) for a, c in zip(o, cts))

    s_t = torch.tensor(single, requires_grad=True)
    z_t = torch.tensor(pair, requires_grad=True)
    o = af2.structure_heads(s_t, z_t, torch.as_tensor(mask), aat, prm, depth, None, False, tables)
    loss = sum((a * torch.as_tensor(c)).sum() for a, c in zip(o, cts))
    gs, gz = torch.autograd.grad(loss, (s_t, z_t))
    h = 1e-6
    for (i, k) in [(0, 0), (3, 200)]:
        e = np.zeros_like(single); e[i, k] = h
        fd = (f(single + e, pair) - f(single - e, pair)) / (2 * h)
        assert abs(fd - gs[i, k].item()) <= 1e-5 * max(1.0, abs(fd))
    for (i, j, k) in [(0, 1, 5), (4, 2, 127)]:
        e = np.zeros_like(pair); e[i, j, k] = h
        fd = (f(single, pair + e) - f(single, pair - e)) / (2 * h)
        assert abs(fd - gz[i, j, k].item()) <= 1e-5 * max(1.0, abs(fd))


# ------------------------------------------------------------- global attention
def _global_params(rng, c=8, heads=2):
    shapes = bparams.global_attention_shapes(c, heads)
    return {f"x/{k}": v for k, v in bparams.init_module(shapes, rng, "random", "random").items()}


def _loop_global_attention(x, mask, P):
    """modules.py:403-497 written out as loops over (column, head, key): the
    masked-mean query (utils.py:61-86 with a [.., 1] mask: broadcast factor 1),
    one query per head, shared single-head keys and values, softmax over the
    sequences, then per query row the head-wise sigmoid gate and the output
    projection."""
    qw, kw, vw = P("attention/query_w"), P("attention/key_w"), P("attention/value_w")
    gw, gb = P("attention/gating_w"), P("attention/gating_b")
    ow, ob = P("attention/output_w"), P("attention/output_b")
    B, K, A = x.shape
    H, D = qw.shape[1], qw.shape[2]
    out = torch.zeros(B, K, ow.shape[-1], dtype=DT)
    for b in range(B):
        msum = sum(float(mask[b, k]) for k in range(K))
        qa = [sum(float(mask[b, k]) * float(x[b, k, a]) for k in range(K)) / (msum + 1e-10)
              for a in range(A)]
        keys = [[sum(float(x[b, k, a]) * float(kw[a, c]) for a in range(A)) for c in range(D)]
                for k in range(K)]
        vals = [[sum(float(x[b, k, a]) * float(vw[a, c]) for a in range(A)) for c in range(D)]
                for k in range(K)]
        wa = []
        for h in range(H):
            q = [sum(qa[a] * float(qw[a, h, c]) for a in range(A)) / D ** 0.5 for c in range(D)]
            lg = [sum(q[c] * keys[k][c] for c in range(D)) + 1e9 * (float(mask[b, k]) - 1.0)
                  for k in range(K)]
            m = max(lg)
            w = [np.exp(v - m) for v in lg]
            s = sum(w)
            wa.append([sum(w[k] / s * vals[k][c] for k in range(K)) for c in range(D)])
        for i in range(K):
            for o in range(ow.shape[-1]):
                acc = float(ob[o])
                for h in range(H):
                    for c in range(D):
                        g = sum(float(x[b, i, a]) * float(gw[a, h, c]) for a in range(A)) + float(gb[h, c])
                        acc += wa[h][c] / (1.0 + np.exp(-g)) * float(ow[h, c, o])
                out[b, i, o] = acc
    return out


def test_global_attention_matches_loops():
    rng = np.random.default_rng(21)
    P = af2.Params(_global_params(rng), "x/")
    x = torch.as_tensor(rng.standard_normal((3, 5, 8)), dtype=DT)
    mask = torch.ones(3, 5, dtype=DT)
    mask[0, 1] = mask[2, 0] = mask[2, 4] = 0
    got = af2.global_attention(x, x, mask[..., None], P)
    torch.testing.assert_close(got, _loop_global_attention(x, mask, P), rtol=1e-10, atol=1e-10)


def _gated_output(x, v, P):
    """sum_h (v . sigmoid(gate_h(x))) W_o[h] + b_o for one value vector per head."""
    g = torch.sigmoid(torch.einsum("bqc,chv->bqhv", x, P("attention/gating_w")) + P("attention/gating_b"))
    return torch.einsum("bqhc,hco->bqo", v * g, P("attention/output_w")) + P("attention/output_b")


@pytest.mark.parametrize("masked", [False, True])
def test_global_attention_single_sequence_closed_form(masked):
    """One sequence: the softmax over one key is 1 whatever its mask, so every
    head reads the one value row."""
    rng = np.random.default_rng(22)
    P = af2.Params(_global_params(rng), "x/")
    x = torch.as_tensor(rng.standard_normal((4, 1, 8)), dtype=DT)
    mask = torch.full((4, 1), 0.0 if masked else 1.0, dtype=DT)
    v = torch.einsum("bka,ac->bkc", x, P("attention/value_w"))[:, :, None]  # [B,1,1,D]
    torch.testing.assert_close(af2.global_attention(x, x, mask[..., None], P), _gated_output(x, v, P),
                               rtol=1e-12, atol=1e-12)


def test_global_attention_fully_masked_column_is_uniform():
    """All sequences masked: the masked-mean query is 0, so every logit is the
    same -1e9 and the weights are uniform: each head reads the mean value."""
    rng = np.random.default_rng(23)
    P = af2.Params(_global_params(rng), "x/")
    x = torch.as_tensor(rng.standard_normal((2, 6, 8)), dtype=DT)
    mask = torch.zeros(2, 6, dtype=DT)
    v = torch.einsum("bka,ac->bkc", x, P("attention/value_w")).mean(1)[:, None, None]
    torch.testing.assert_close(af2.global_attention(x, x, mask[..., None], P), _gated_output(x, v, P),
                               rtol=1e-12, atol=1e-12)


def test_pair_only_iteration_is_the_extra_block_at_zero_mask():
    """The pair-only block equals the full extra-MSA EvoformerIteration (MSA
    row attention, global column attention, MSA transition, outer product
    mean on a c_e MSA) on an all-zero extra-MSA mask, dropout on."""
    from oracle import jax_prng as J
    rng = np.random.default_rng(24)
    kw = dict(c_z=16, c_m=8, tri_heads=2, trimul_hidden=8, opm_c=4, row_heads=2, col_heads=2)
    sh = bparams.module_shapes(**kw)
    sh.pop("msa_column_attention")
    sh["msa_column_global_attention"] = bparams.global_attention_shapes(8, 2)
    prm = {}
    for mod, shapes in sh.items():
        for pname, arr in bparams.init_module(shapes, rng, "random", "random").items():
            prm[f"param/block0/{mod}/{pname}"] = arr
    prm["param/block0/outer_product_mean/output_b"] *= 1e-3
    pair = torch.as_tensor(rng.standard_normal((7, 7, 16)), dtype=DT)
    msa = torch.as_tensor(rng.standard_normal((3, 7, 8)), dtype=DT)
    pmask = torch.as_tensor((rng.random((7, 7)) > 0.2).astype(np.float64))
    key = J.prng_key(5)
    _, full = af2.evoformer_iteration(msa, pair, torch.zeros(3, 7, dtype=DT), pmask, prm,
                                      "param/block0/", key, True, is_extra_msa=True)
    got = af2.pair_only_iteration(pair, pmask, prm, "param/block0/", key, True)
    torch.testing.assert_close(got, full, rtol=1e-12, atol=1e-12)
    # and the dropout is live: a different key changes the result
    other = af2.pair_only_iteration(pair, pmask, prm, "param/block0/", J.prng_key(6), True)
    assert not torch.allclose(other, full)


def test_block_recompute_is_exact():
    """Per-block recompute (activation checkpointing of the stack blocks)
    gives autograd's values and gradients to rounding."""
    from oracle import jax_prng as J
    rng = np.random.default_rng(13)
    prm = {}
    for b in range(2):
        prm.update(bparams.init_block_params(b, rng, c_z=16, c_m=16, tri_heads=2,
                                             trimul_hidden=8, gates="random", ln="random"))
    n, s = 6, 2
    pair = torch.tensor(rng.standard_normal((n, n, 16)), dtype=DT, requires_grad=True)
    msa = torch.tensor(rng.standard_normal((s, n, 16)), dtype=DT, requires_grad=True)
    mm = torch.ones(s, n, dtype=DT)
    pm = torch.ones(n, n, dtype=DT)
    key = J.prng_key(5)
    cts = (torch.as_tensor(rng.standard_normal((s, n, 16))), torch.as_tensor(rng.standard_normal((n, n, 16))))

    def run():
        out = af2.evoformer_stack(msa, pair, mm, pm, prm, 2, key, True)
        return [o.detach() for o in out] + list(torch.autograd.grad(out, (msa, pair), cts))

    ref = run()
    with af2.block_recompute():
        got = run()
    for a, b in zip(got, ref):
        torch.testing.assert_close(a, b, rtol=1e-12, atol=1e-12)
