"""The library run from an AF2 multimer parameter tree through the
weights-directory writers (bindcraft2_amd/weights.py, the restatement of
bindcraft/af/native.py:171-570): every component's directory is written from
one haiku-style tree, loaded by the library, and each component's forward is
checked against the oracle on the same directory read back."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as P, weights as W
from oracle import af2
from tests.helpers import assert_act, random_mask

pytestmark = pytest.mark.gpu
D = torch.float64


@pytest.fixture(scope="module")
def tree():
    return W.init_af2_params(np.random.default_rng(21), num_blocks=1, extra_blocks=1,
                             template_blocks=1, gates="random", ln="random")


def test_tree_main_stack_and_template_embedding(cuda, tree, tmp_path):
    n, s = 32, 2
    rng = np.random.default_rng(22)
    T = lambda a: torch.as_tensor(a, device=cuda)
    main = W.stack_weights_from_params(tree, str(tmp_path / "main"), prefix=W.MAIN)
    prm = P.read_manifest(main)
    pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    msa = rng.standard_normal((s, n, 256)).astype(np.float32)
    pmask, m1 = random_mask(n, 0.1, rng)
    mmask = np.tile(m1, (s, 1)).astype(np.float32)
    po, mo, _ = ops.EvoformerStack(main, 1).forward(T(pair), T(msa), T(pmask), T(mmask), None,
                                                    dropout=False)
    torch.cuda.synchronize()
    x, y = torch.as_tensor(pair, dtype=D), torch.as_tensor(msa, dtype=D)
    rm, rp = af2.evoformer_stack(y, x, torch.as_tensor(mmask, dtype=D),
                                 torch.as_tensor(pmask, dtype=D), prm, 1, None, False)
    print("main pair", assert_act(po.cpu().double() - x, rp - x, what="pair"))
    print("main msa", assert_act(mo.cpu().double() - y, rm - y, what="msa"))

    tpe = W.tplembed_weights_from_params(tree, str(tmp_path / "tpe"))
    prm = P.read_manifest(tpe)
    query = rng.standard_normal((n, n, 128)).astype(np.float32)
    act_const = rng.standard_normal((n, n, 64)).astype(np.float32)
    out, _ = ops.TemplateEmbedding(tpe, 1).forward(T(query), T(act_const), T(pmask), None,
                                                   dropout=False)
    torch.cuda.synchronize()
    ref = af2.template_embedding(torch.as_tensor(query, dtype=D), torch.as_tensor(act_const, dtype=D),
                                 torch.as_tensor(pmask, dtype=D), prm, 1, None, False)
    print("template embedding", assert_act(out.cpu().double(), ref, what="tplembed"))


def test_tree_embedder_and_fold(cuda, tree, tmp_path):
    n = 40
    rng = np.random.default_rng(23)
    T = lambda a: torch.as_tensor(a, device=cuda)
    emb = W.embed_weights_from_params(tree, str(tmp_path / "emb"))
    prm = P.read_manifest(emb)
    assert "param/evoformer/~_relative_encoding/position_activations/weights" not in prm
    tf = np.zeros((n, 21), np.float32)
    tf[:, :20] = rng.dirichlet(np.ones(20), n)
    mf = rng.standard_normal((1, n, 49)).astype(np.float32)
    ids = [np.concatenate([np.arange(25), np.arange(15)]).astype(np.float32),
           np.repeat([1, 2], [25, 15]).astype(np.float32), np.ones(n, np.float32),
           np.repeat([1, 2], [25, 15]).astype(np.float32)]
    msa, pair = ops.Embedder(emb).forward(T(tf), T(mf), *map(T, ids))
    torch.cuda.synchronize()
    rmsa, rpair = af2.embedder(torch.as_tensor(tf, dtype=D), torch.as_tensor(mf, dtype=D), *ids, prm)
    print("embedder msa", assert_act(msa.cpu().double(), rmsa, 1e-5, "msa"))
    print("embedder pair", assert_act(pair.cpu().double(), rpair, 1e-5, "pair"))

    tables = P.init_residue_tables(rng)
    post = W.post_weights_from_params(tree, str(tmp_path / "post"), tables=tables)
    prm = P.read_manifest(post)
    single = rng.standard_normal((n, 384)).astype(np.float32)
    z = rng.standard_normal((n, n, 128)).astype(np.float32)
    mask = np.ones(n, np.float32)
    act, traj, _ = ops.Fold(post, 2).forward(T(single), T(z), T(mask), None, dropout=False)
    torch.cuda.synchronize()
    ract, rtraj = af2.fold(torch.as_tensor(single, dtype=D), torch.as_tensor(z, dtype=D),
                           torch.as_tensor(mask, dtype=D), prm, 2, None, False)
    print("fold act", assert_act(act.cpu().double(), ract, 1e-3, "act"))
    print("fold traj", assert_act(traj.cpu().double(), rtraj, 1e-3, "traj"))
    aat = rng.integers(0, 21, n).astype(np.float32)
    outs, _ = ops.StructureHeads(post, 2).forward(T(single), T(z), T(mask), T(aat), None,
                                                  dropout=False)
    torch.cuda.synchronize()
    ref = af2.structure_heads(torch.as_tensor(single, dtype=D), torch.as_tensor(z, dtype=D),
                              torch.as_tensor(mask, dtype=D), aat, prm, 2, None, False, tables)
    for name, o, r in zip(("atom14", "distogram", "pae", "plddt", "expres"), outs, ref):
        print("structure heads", name, assert_act(o.cpu().double(), r, 1e-3, name))
