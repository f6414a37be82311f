"""GPU parity of the design-sequence front (bc2n_seqfeat_*, bc2n_design_inputs_*,
bc2n_design_step_seq_*) against the oracle's sequence_features,
design_inputs and design_step_seq (bindcraft/af2.py:99-104, :187-192 over
bindcraft/sequence_optimization.py:33-52).

The features are f32 arithmetic on 20 values per residue: forward and
gradient within 1e-5 relative of the fp64 oracle.  The one-call step takes
the design-step bars (tests/test_gpu_design_step.py), absolute: outputs
relL2 and normwise max error <= 2e-2 and cosine >= 0.9999 (pTM/ipTM:
relative error), d(logits) cosine >= 0.999 and relL2 <= 5e-2."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import metrics, weights_dir
from tests.test_gpu_design_step import _extra_params

pytestmark = pytest.mark.gpu
D = torch.float64


def _inputs(n, rng, with_bias):
    x = rng.standard_normal((n, 20)).astype(np.float32)
    flags = np.ones(n, np.uint8)
    flags[n // 2:] = 0  # a target chain: its one-hot sequence passes through
    x[n // 2:] = np.eye(20, dtype=np.float32)[rng.integers(0, 20, n - n // 2)]
    x[1, 4] = x[3, 17] = -1e4  # omitted acids
    bias = (0.5 * rng.standard_normal(20)).astype(np.float32) if with_bias else None
    return x, flags, bias


@pytest.mark.parametrize("scalars,with_bias,device_scalars", [
    ((1.0, 0.0, 1.0, 1.0), False, False),
    ((0.7, 0.3, 1.3, 2.0), True, False),
    ((0.0, 0.0, 1.0, 1.0), False, True),
    ((0.5, 1.0, 0.01, 1.0), True, True),
])
def test_seqfeat_parity(cuda, scalars, with_bias, device_scalars):
    print(f"seqfeat scalars={scalars} bias={with_bias} device={device_scalars}", flush=True)
    rng = np.random.default_rng(int(100 * sum(scalars)) + with_bias)
    n = 75
    x, flags, bias = _inputs(n, rng, with_bias)
    gf = rng.standard_normal((n, 20)).astype(np.float32)
    gp = rng.standard_normal((n, 20)).astype(np.float32)
    T = lambda a: None if a is None else torch.as_tensor(a, device=cuda)
    sc = torch.tensor(scalars, dtype=torch.float32, device=cuda) if device_scalars else scalars
    op = ops.SeqFeat(sc, aa_bias=T(bias))
    feat, prof = op.forward(T(x), T(flags))
    dlog = op.backward(T(x), T(flags), T(gf), T(gp))
    torch.cuda.synchronize()

    t = torch.tensor(x, dtype=D, requires_grad=True)
    rf, rp = af2.sequence_features(t, flags, *scalars,
                                   bias=None if bias is None else torch.tensor(bias, dtype=D))
    (rg,) = torch.autograd.grad((rf * torch.tensor(gf, dtype=D)).sum()
                                + (rp * torch.tensor(gp, dtype=D)).sum(), t)
    for name, g, r in (("feat", feat, rf.detach()), ("prof", prof, rp.detach()), ("d_logits", dlog, rg)):
        g = g.cpu().double()
        err = ((g - r).norm() / r.norm().clamp_min(1e-30)).item()
        print(f"  {name}: rel {err:.2e}")
        assert err <= 1e-5, name


def test_design_inputs_parity(cuda):
    rng = np.random.default_rng(7)
    n = 40
    feat = rng.standard_normal((n, 20)).astype(np.float32)
    prof = rng.standard_normal((n, 20)).astype(np.float32)
    T = lambda a: torch.as_tensor(a, device=cuda)
    tf, mf, aat = ops.design_inputs(T(feat), T(prof))
    dtf = rng.standard_normal((n, 21)).astype(np.float32)
    dmf = rng.standard_normal((1, n, 49)).astype(np.float32)
    dfeat, dprof = ops.design_inputs_backward(T(dtf), T(dmf))
    torch.cuda.synchronize()
    rtf, rmf, raat = af2.design_inputs(torch.tensor(feat, dtype=D), torch.tensor(prof, dtype=D))
    np.testing.assert_array_equal(tf.cpu().numpy(), rtf.numpy().astype(np.float32))
    np.testing.assert_array_equal(mf.cpu().numpy(), rmf.numpy().astype(np.float32))
    np.testing.assert_array_equal(aat.cpu().numpy(), raat)
    np.testing.assert_array_equal(dfeat.cpu().numpy(), dtf[:, :20] + dmf[0, :, :20])
    np.testing.assert_array_equal(dprof.cpu().numpy(), dmf[0, :, 25:45])


@pytest.mark.parametrize("with_template,dropout", [(False, False), (True, True)])
def test_design_step_seq_parity(cuda, with_template, dropout):
    n = 32
    print(f"design step from logits n={n} template={with_template} dropout={dropout}", flush=True)
    depths = {"tpl": 1, "extra": 1, "main": 1, "fold": 2}
    rng = np.random.default_rng(9100 + int(with_template) + 2 * int(dropout))
    prm = {"emb": bparams.init_embedder_params(rng),
           "tpl": bparams.init_template_embedding_params(depths["tpl"], rng, gates="random",
                                                         ln="random"),
           "extra": _extra_params(depths["extra"], rng),
           "main": bparams.init_block_params(0, rng, gates="random", ln="random"),
           "post": bparams.init_structure_heads_params(rng, final="random", ln="random")}
    tables = bparams.init_residue_tables(rng)
    prm["post"].update({f"const/{k}": v for k, v in tables.items()})
    tag = f"seq_{int(with_template)}_{int(dropout)}"
    dirs = [weights_dir(prm[k], f"dss_{k}_{tag}") for k in ("emb", "tpl", "extra", "main", "post")]

    x, flags, bias = _inputs(n, rng, True)
    flags[n // 2:] |= 2  # the target chain is the template (its MSA row's chi angles)
    tpl37 = (3 * rng.standard_normal((n, 37, 3))).astype(np.float32)
    tplm37 = (rng.random((n, 37)) < 0.9).astype(np.float32)
    scalars = (0.8, 0.25, 1.2, 1.5)
    cut = n // 2 + 3
    ids = [np.concatenate([np.arange(cut), np.arange(n - cut)]).astype(np.float32),
           np.repeat([1, 2], [cut, n - cut]).astype(np.float32),
           np.repeat([1, 2], [cut, n - cut]).astype(np.float32), np.ones(n, np.float32)]
    seq_mask = np.ones(n, np.float32)
    seq_mask[rng.choice(n, 2, replace=False)] = 0.0
    act_const = (0.5 * rng.standard_normal((n, n, 64))).astype(np.float32) if with_template else None
    emsa = rng.standard_normal((1, n, 64))
    keys = {k: J.prng_key(400 + i) for i, k in enumerate(("tpl", "extra", "main", "fold"))}
    seeds = torch.tensor([[int(keys[k][0]), int(keys[k][1]), 1]
                          for k in ("tpl", "extra", "main", "fold")], dtype=torch.int64)
    shapes = ((n, 14, 3), (n, n, 64), (n, n, 64), (n, 50), (n, 37),
              (n,), (n, n), (1,), (1,), (n,), (n,))  # + the confidence metrics
    cts = [rng.standard_normal(sh).astype(np.float32) for sh in shapes]
    iasym = ids[1].astype(np.int32)

    t = torch.tensor(x, dtype=D, requires_grad=True)
    ref = af2.design_step_seq(t, flags, scalars, ids, None, torch.as_tensor(seq_mask, dtype=D),
                              None if act_const is None else torch.as_tensor(act_const, dtype=D),
                              torch.as_tensor(emsa, dtype=D), prm, depths,
                              keys if dropout else {k: None for k in keys}, dropout, tables,
                              bias=torch.tensor(bias, dtype=D),
                              tpl_atoms37=tpl37 if with_template else None,
                              tpl_mask37=tplm37 if with_template else None)
    ref = list(ref[:5]) + list(af2.confidence(ref[3], ref[2], ref[4],
                                              torch.as_tensor(seq_mask, dtype=D), iasym))
    loss = sum((r * torch.as_tensor(c, dtype=D)).sum() for r, c in zip(ref, cts))
    ref = [r.detach() for r in ref] + list(torch.autograd.grad(loss, (t,)))

    T = lambda a: None if a is None else torch.as_tensor(a, device=cuda)
    step = ops.DesignStepSeq(*dirs, depths=(depths["tpl"], depths["extra"], depths["main"],
                                            depths["fold"]))
    sc = torch.tensor(scalars, dtype=torch.float32, device=cuda)
    outs, save, conf = step.forward(T(x), T(flags), sc, [T(v) for v in ids], T(seq_mask),
                                    aa_bias=T(bias), act_const=T(act_const),
                                    seeds=seeds.to(torch.uint32).to(cuda), dropout=dropout,
                                    interface_asym=T(iasym),
                                    tpl_atoms37=T(tpl37) if with_template else None,
                                    tpl_mask37=T(tplm37) if with_template else None)[:3]
    dlog = step.backward([T(c) for c in cts[:5]], T(x), T(flags), sc, T(seq_mask), save,
                         aa_bias=T(bias), with_template=with_template, dropout=dropout,
                         interface_asym=T(iasym), conf_cts=[T(c) for c in cts[5:]])
    torch.cuda.synchronize()

    names = ("atom14", "distogram", "pae", "plddt", "expres", "conf plddt", "conf pae", "ptm",
             "iptm", "iptm_per_residue", "expres_ca", "d logits")
    last = len(names) - 1
    for i, (name, g, r) in enumerate(zip(names, list(outs) + list(conf) + [dlog], ref)):
        m = metrics(g.cpu().double(), r)
        print(f"  {name}", m)
        if i in (7, 8):  # scalars: relative error only
            assert m["rel_l2"] <= 2e-2, name
        elif i < last:
            assert m["rel_l2"] <= 2e-2 and m["max_rel"] <= 2e-2 and m["cos"] >= 0.9999, name
        else:
            assert m["cos"] >= 0.999 and m["rel_l2"] <= 5e-2, name


def test_design_step_save_flags(cuda):
    """The backward refuses a save buffer whose optional parts (template
    embedding, confidence metrics) differ from the ones it is asked to
    differentiate, and one no forward wrote."""
    from bindcraft2_amd import NativeError
    n = 32
    print(f"design step save-buffer flags n={n}", flush=True)
    depths = {"tpl": 1, "extra": 1, "main": 1, "fold": 1}
    rng = np.random.default_rng(9200)
    prm = {"emb": bparams.init_embedder_params(rng),
           "tpl": bparams.init_template_embedding_params(depths["tpl"], rng),
           "extra": _extra_params(depths["extra"], rng),
           "main": bparams.init_block_params(0, rng),
           "post": bparams.init_structure_heads_params(rng)}
    prm["post"].update({f"const/{k}": v for k, v in bparams.init_residue_tables(rng).items()})
    dirs = [weights_dir(prm[k], f"dsf_{k}") for k in ("emb", "tpl", "extra", "main", "post")]
    T = lambda a: None if a is None else torch.as_tensor(a, device=cuda)
    x, flags, _ = _inputs(n, rng, False)
    ids = [np.arange(n, dtype=np.float32), np.repeat([1, 2], n // 2).astype(np.float32),
           np.repeat([1, 2], n // 2).astype(np.float32), np.ones(n, np.float32)]
    seq_mask = np.ones(n, np.float32)
    sc = torch.tensor((1.0, 0.0, 1.0, 1.0), dtype=torch.float32, device=cuda)
    step = ops.DesignStepSeq(*dirs, depths=tuple(depths[k] for k in ("tpl", "extra", "main", "fold")))
    shapes = ((n, 14, 3), (n, n, 64), (n, n, 64), (n, 50), (n, 37))
    cts = [T(rng.standard_normal(sh).astype(np.float32)) for sh in shapes]
    conf_cts = [T(np.ones(n, np.float32))] + [None] * 5
    iasym = T(ids[1].astype(np.int32))
    args = (T(x), T(flags), sc, T(seq_mask))

    # forward with neither template nor confidence
    _, save = step.forward(T(x), T(flags), sc, [T(v) for v in ids], T(seq_mask), dropout=False)
    with pytest.raises(NativeError, match="template embedding, which the forward did not"):
        step.backward(cts, *args, save, with_template=True, dropout=False)
    with pytest.raises(NativeError, match="confidence metrics, which the forward did not"):
        step.backward(cts, *args, save, with_template=False, dropout=False,
                      interface_asym=iasym, conf_cts=conf_cts)
    with pytest.raises(NativeError, match="atom37 positions, which the forward did not"):
        step.backward(cts, *args, save, with_template=False, dropout=False,
                      d_atom37=T(np.ones((n, 37, 3), np.float32)))
    d_ok = step.backward(cts, *args, save, with_template=False, dropout=False)

    # forward with both: leaving the template out of the backward is refused,
    # leaving the confidence cotangents out is allowed
    act_const = T((0.5 * rng.standard_normal((n, n, 64))).astype(np.float32))
    tpl37 = T((3 * rng.standard_normal((n, 37, 3))).astype(np.float32))
    _, save2, _, _ = step.forward(T(x), T(flags), sc, [T(v) for v in ids], T(seq_mask),
                                  act_const=act_const, dropout=False, interface_asym=iasym,
                                  tpl_atoms37=tpl37, tpl_mask37=torch.ones(n, 37, device=cuda))
    with pytest.raises(NativeError, match="omits the template"):
        step.backward(cts, *args, save2, with_template=False, dropout=False)
    d2 = step.backward(cts, *args, save2, with_template=True, dropout=False)

    # a buffer no forward wrote
    blank = torch.zeros_like(save)
    with pytest.raises(NativeError, match="not written by this step's forward"):
        step.backward(cts, *args, blank, with_template=False, dropout=False)
    torch.cuda.synchronize()
    assert torch.isfinite(d_ok).all() and torch.isfinite(d2).all()


@pytest.mark.parametrize("align", [False, True])
def test_design_step_seq_atom37(cuda, align):
    """The step's atom37 output (gathered, masked) and its superposition on
    the template's CA atoms (bindcraft/af2.py:89-97), with an atom37
    cotangent in the loss, one recycle pass first.  Bars as the step's
    (outputs relL2/max <= 2e-2, cos >= 0.9999; d(logits) cos >= 0.999,
    relL2 <= 5e-2); the exists mask exactly."""
    n, recycles = 32, 1
    print(f"design step atom37 n={n} align={align} recycles={recycles}", flush=True)
    depths = {"tpl": 1, "extra": 1, "main": 1, "fold": 2}
    rng = np.random.default_rng(9300 + int(align))
    prm = {"emb": bparams.init_embedder_params(rng),
           "tpl": bparams.init_template_embedding_params(depths["tpl"], rng, gates="random",
                                                         ln="random"),
           "extra": _extra_params(depths["extra"], rng),
           "main": bparams.init_block_params(0, rng, gates="random", ln="random"),
           "post": bparams.init_structure_heads_params(rng, final="random", ln="random")}
    prm["emb"]["param/prev_pos_linear/weights"] *= 1e-3  # see test_gpu_design_step.py
    tables = bparams.init_residue_tables(rng)
    prm["post"].update({f"const/{k}": v for k, v in tables.items()})
    dirs = [weights_dir(prm[k], f"dsa_{k}_{int(align)}") for k in ("emb", "tpl", "extra", "main",
                                                                    "post")]
    x, flags, bias = _inputs(n, rng, False)
    flags[n // 2:] |= 2  # the target chain is the template
    scalars = (0.9, 0.1, 1.0, 1.0)
    ids = [np.arange(n, dtype=np.float32), np.repeat([1, 2], n // 2).astype(np.float32),
           np.repeat([1, 2], n // 2).astype(np.float32), np.ones(n, np.float32)]
    seq_mask = np.ones(n, np.float32)
    seq_mask[3] = 0.0
    emsa = rng.standard_normal((1, n, 64))
    stacks = ("tpl", "extra", "main", "fold")
    keys = [{k: None for k in stacks}] * (recycles + 1)
    tpl37 = (8 * rng.standard_normal((n, 37, 3))).astype(np.float32)
    tplm37 = (rng.random((n, 37)) < 0.8).astype(np.float32)
    tplm37[n // 2 + 1, 1] = 0.0  # a template residue without its CA is not aligned on
    shapes = ((n, 14, 3), (n, n, 64), (n, n, 64), (n, 50), (n, 37))
    cts = [rng.standard_normal(sh).astype(np.float32) for sh in shapes]
    ct37 = rng.standard_normal((n, 37, 3)).astype(np.float32)

    t = torch.tensor(x, dtype=D, requires_grad=True)
    # with the alignment, a template embedding too: its MSA row joins the stack
    act_const = (0.5 * rng.standard_normal((n, n, 64))).astype(np.float32) if align else None
    ref = af2.design_step_seq(t, flags, scalars, ids, None, torch.as_tensor(seq_mask, dtype=D),
                              None if act_const is None else torch.as_tensor(act_const, dtype=D),
                              torch.as_tensor(emsa, dtype=D), prm, depths, keys, False,
                              tables, recycles=recycles,
                              tpl_atoms37=tpl37 if align else None,
                              tpl_mask37=tplm37 if align else None)
    if not align:  # the gather alone: the oracle's atom37 of its atom14
        a37, ex = af2.atom14_to_atom37(ref[0], af2.design_inputs(*af2.sequence_features(
            t, flags, *scalars))[2], torch.as_tensor(seq_mask, dtype=D), tables)
        ref = tuple(ref) + (a37, ex)
    loss = sum((r * torch.as_tensor(c, dtype=D)).sum() for r, c in zip(ref[:5], cts))
    loss = loss + (ref[5] * torch.as_tensor(ct37, dtype=D)).sum()
    (dref,) = torch.autograd.grad(loss, (t,))

    T = lambda a: None if a is None else torch.as_tensor(a, device=cuda)
    step = ops.DesignStepSeq(*dirs, depths=tuple(depths[k] for k in stacks))
    sc = torch.tensor(scalars, dtype=torch.float32, device=cuda)
    outs, save, _, (g37, gm37) = step.forward(
        T(x), T(flags), sc, [T(v) for v in ids], T(seq_mask), act_const=T(act_const),
        dropout=False, recycles=recycles, atom37=True, tpl_atoms37=T(tpl37) if align else None,
        tpl_mask37=T(tplm37) if align else None)
    dlog = step.backward([T(c) for c in cts], T(x), T(flags), sc, T(seq_mask), save,
                         with_template=align, dropout=False, d_atom37=T(ct37))
    torch.cuda.synchronize()
    assert torch.equal(gm37.cpu().double(), ref[6].detach()), "atom37 exists mask"
    for name, g, r in (("atom14", outs[0], ref[0]), ("atom37", g37, ref[5])):
        m = metrics(g.cpu().double(), r.detach())
        print(f"  {name}", m)
        assert m["rel_l2"] <= 2e-2 and m["max_rel"] <= 2e-2 and m["cos"] >= 0.9999, name
    m = metrics(dlog.cpu().double(), dref)
    print("  d logits", m)
    assert m["cos"] >= 0.999 and m["rel_l2"] <= 5e-2


def test_design_step_seq_runtime_length(cuda):
    """The runtime length (the reference's `n`, native/design_step.cuh:10-19):
    buffers sized for a bucket of 64 rows, the length 45 in device memory.
    The 19 padding rows hold junk -- random logits, DESIGN and TEMPLATE
    flags, seq_mask 1, template atoms, and random cotangents on every
    padding row and column -- which must not reach the 45 real rows.  The
    real rows are held to the step's bars against the oracle run on the 45
    residues alone (template row, dropout with JAX keys, one recycle,
    confidence metrics, atom37 aligned); every padding output and padding
    d(logits) row is exactly zero.  The length equal to the bucket gives the
    same bits as no length at all."""
    nb, n, recycles = 64, 45, 1
    print(f"design step runtime length bucket={nb} n={n} recycles={recycles}", flush=True)
    depths = {"tpl": 1, "extra": 1, "main": 1, "fold": 2}
    rng = np.random.default_rng(9400)
    prm = {"emb": bparams.init_embedder_params(rng),
           "tpl": bparams.init_template_embedding_params(depths["tpl"], rng, gates="random",
                                                         ln="random"),
           "extra": _extra_params(depths["extra"], rng),
           "main": bparams.init_block_params(0, rng, gates="random", ln="random"),
           "post": bparams.init_structure_heads_params(rng, final="random", ln="random")}
    prm["emb"]["param/prev_pos_linear/weights"] *= 1e-3  # see test_gpu_design_step.py
    tables = bparams.init_residue_tables(rng)
    prm["post"].update({f"const/{k}": v for k, v in tables.items()})
    dirs = [weights_dir(prm[k], f"dsl_{k}") for k in ("emb", "tpl", "extra", "main", "post")]
    stacks = ("tpl", "extra", "main", "fold")

    # the bucket's inputs: real rows first, junk after
    x, flags, bias = _inputs(nb, rng, True)
    flags[n // 2:n] |= 2  # the real target chain is the template
    flags[n:] = rng.integers(0, 4, nb - n).astype(np.uint8)
    x[n:] = 3 * rng.standard_normal((nb - n, 20)).astype(np.float32)
    cut = 20
    ids = [np.concatenate([np.arange(cut), np.arange(n - cut), 100 + np.arange(nb - n)]),
           np.concatenate([np.repeat([1, 2], [cut, n - cut]), np.full(nb - n, 3)]),
           np.concatenate([np.repeat([1, 2], [cut, n - cut]), np.full(nb - n, 3)]),
           np.ones(nb)]
    ids = [v.astype(np.float32) for v in ids]
    # every real row unmasked: a masked real residue's attention rows are
    # fully masked, which the f32 model (and the GPU) turns uniform while the
    # fp64 oracle keeps the logit differences (1e9 absorbs them only in f32)
    seq_mask = np.ones(nb, np.float32)
    iasym = ids[1].astype(np.int32)
    tpl37 = (8 * rng.standard_normal((nb, 37, 3))).astype(np.float32)
    tplm37 = (rng.random((nb, 37)) < 0.8).astype(np.float32)
    act_const = (0.5 * rng.standard_normal((nb, nb, 64))).astype(np.float32)
    scalars = (0.8, 0.25, 1.2, 1.5)
    keys = [{k: J.prng_key(700 + 10 * p + i) for i, k in enumerate(stacks)}
            for p in range(recycles + 1)]
    seeds = torch.tensor([[int(kp[k][0]), int(kp[k][1]), 1] for kp in keys for k in stacks],
                         dtype=torch.int64)
    shapes = ((nb, 14, 3), (nb, nb, 64), (nb, nb, 64), (nb, 50), (nb, 37))
    cts = [rng.standard_normal(sh).astype(np.float32) for sh in shapes]
    ct37 = rng.standard_normal((nb, 37, 3)).astype(np.float32)
    conf_cts = [rng.standard_normal(sh).astype(np.float32) for sh in ((nb,), (nb, nb), (1,), (1,),
                                                                      (nb,), (nb,))]

    # the oracle on the 45 real residues
    r1, r2 = slice(0, n), (slice(0, n), slice(0, n))
    t = torch.tensor(x[:n], dtype=D, requires_grad=True)
    sm = torch.as_tensor(seq_mask[:n], dtype=D)
    ref = af2.design_step_seq(t, flags[:n], scalars, [v[:n] for v in ids], None, sm,
                              torch.as_tensor(act_const[r2], dtype=D),
                              torch.as_tensor(rng.standard_normal((1, n, 64)), dtype=D), prm,
                              depths, keys, True, tables, bias=torch.tensor(bias, dtype=D),
                              recycles=recycles, tpl_atoms37=tpl37[:n], tpl_mask37=tplm37[:n])
    conf = af2.confidence(ref[3], ref[2], ref[4], sm, iasym[:n])
    real = [(ref[0], cts[0][r1]), (ref[1], cts[1][r2]), (ref[2], cts[2][r2]),
            (ref[3], cts[3][r1]), (ref[4], cts[4][r1]), (ref[5], ct37[r1])]
    real += [(c, ct[r2] if c.dim() == 2 else ct[r1] if c.numel() == n else ct)
             for c, ct in zip(conf, conf_cts)]
    loss = sum((r * torch.as_tensor(c, dtype=D)).sum() for r, c in real)
    (dref,) = torch.autograd.grad(loss, (t,))

    T = lambda a: None if a is None else torch.as_tensor(a, device=cuda)
    step = ops.DesignStepSeq(*dirs, depths=tuple(depths[k] for k in stacks))
    sc = torch.tensor(scalars, dtype=torch.float32, device=cuda)
    length = torch.tensor([n], dtype=torch.int32, device=cuda)
    common = dict(aa_bias=T(bias), act_const=T(act_const), seeds=seeds.to(torch.uint32).to(cuda),
                  dropout=True, interface_asym=T(iasym), recycles=recycles,
                  tpl_atoms37=T(tpl37), tpl_mask37=T(tplm37))
    outs, save, gconf, (g37, gm37) = step.forward(T(x), T(flags), sc, [T(v) for v in ids],
                                                  T(seq_mask), length=length, **common)
    dlog = step.backward([T(c) for c in cts], T(x), T(flags), sc, T(seq_mask), save,
                         aa_bias=T(bias), with_template=True, dropout=True,
                         interface_asym=T(iasym), conf_cts=[T(c) for c in conf_cts],
                         d_atom37=T(ct37), length=length)
    torch.cuda.synchronize()

    names = ("atom14", "distogram", "pae", "plddt", "expres", "atom37", "conf plddt", "conf pae",
             "ptm", "iptm", "iptm_per_residue", "expres_ca")
    gots = list(outs) + [g37] + list(gconf)
    refs = list(ref[:6]) + list(conf)
    for name, g, r in zip(names, gots, refs):
        g = g.cpu().double()
        pair = g.dim() >= 2 and g.shape[0] == nb and g.shape[1] == nb
        gr = g[r2] if pair else g[r1] if g.shape[0] == nb else g
        m = metrics(gr, r.detach())
        print(f"  {name}", m)
        if name in ("ptm", "iptm"):
            assert m["rel_l2"] <= 2e-2, name
        else:
            assert m["rel_l2"] <= 2e-2 and m["max_rel"] <= 2e-2 and m["cos"] >= 0.9999, name
        if g.shape[0] == nb:  # the padding is written as zeros
            assert not g[n:].any(), name
            if pair:
                assert not g[:, n:].any(), name
    assert not gm37.cpu()[n:].any()
    m = metrics(dlog.cpu().double()[:n], dref)
    print("  d logits", m)
    assert m["cos"] >= 0.999 and m["rel_l2"] <= 5e-2
    assert not dlog.cpu()[n:].any(), "padding d(logits)"

    # the bucket's own length gives the bits of no length at all
    full = torch.tensor([nb], dtype=torch.int32, device=cuda)
    a = step.forward(T(x), T(flags), sc, [T(v) for v in ids], T(seq_mask), length=full,
                     **common)[0]
    b = step.forward(T(x), T(flags), sc, [T(v) for v in ids], T(seq_mask), **common)[0]
    torch.cuda.synchronize()
    for u, v in zip(a, b):
        assert torch.equal(u, v)


@pytest.mark.parametrize("mode,flex", [("direction", 0.5), ("neighbours", 0.25),
                                       ("distance", 0.0)])
def test_design_step_seq_cyclic_flexible(cuda, mode, flex):
    """Cyclic offsets built on the device (bindcraft/af2.py:174-185, the
    reference's cyclic_mode) for a cyclic designed chain, and the target
    flexibility's gaps in the template row (af2.py:150-157), against the
    oracle at the step's bars; the oracle without the two features is far
    from the GPU result, so both are exercised."""
    n, nb = 64, 24  # a 24-residue cyclic binder, a 40-residue template target
    print(f"design step cyclic mode={mode} flexibility={flex} n={n}", flush=True)
    depths = {"tpl": 1, "extra": 1, "main": 1, "fold": 2}
    rng = np.random.default_rng(9500 + int(100 * flex))
    prm = {"emb": bparams.init_embedder_params(rng),
           "tpl": bparams.init_template_embedding_params(depths["tpl"], rng, gates="random",
                                                         ln="random"),
           "extra": _extra_params(depths["extra"], rng),
           "main": bparams.init_block_params(0, rng, gates="random", ln="random"),
           "post": bparams.init_structure_heads_params(rng, final="random", ln="random")}
    tables = bparams.init_residue_tables(rng)
    prm["post"].update({f"const/{k}": v for k, v in tables.items()})
    dirs = [weights_dir(prm[k], f"dsc_{k}_{mode}") for k in ("emb", "tpl", "extra", "main", "post")]
    stacks = ("tpl", "extra", "main", "fold")
    x = rng.standard_normal((n, 20)).astype(np.float32)
    x[nb:] = np.eye(20, dtype=np.float32)[rng.integers(0, 20, n - nb)]
    flags = np.zeros(n, np.uint8)
    flags[:nb] = 1 | af2.CYCLIC
    flags[nb:] = 2
    ids = [np.concatenate([np.arange(nb), 100 + np.arange(n - nb)]),
           np.repeat([1, 2], [nb, n - nb]), np.repeat([1, 2], [nb, n - nb]), np.ones(n)]
    ids = [v.astype(np.float32) for v in ids]
    seq_mask = np.ones(n, np.float32)
    iasym = ids[1].astype(np.int32)
    tpl37 = (8 * rng.standard_normal((n, 37, 3))).astype(np.float32)
    tplm37 = (rng.random((n, 37)) < 0.9).astype(np.float32)
    act_const = (0.5 * rng.standard_normal((n, n, 64))).astype(np.float32)
    scalars = (0.8, 0.25, 1.2, 1.5)
    keys = {k: J.prng_key(800 + i) for i, k in enumerate(stacks)}
    seeds = torch.tensor([[int(keys[k][0]), int(keys[k][1]), 1] for k in stacks],
                         dtype=torch.int64)
    shapes = ((n, 14, 3), (n, n, 64), (n, n, 64), (n, 50), (n, 37))
    cts = [rng.standard_normal(sh).astype(np.float32) for sh in shapes]
    emsa = torch.as_tensor(rng.standard_normal((1, n, 64)), dtype=D)

    def oracle(cyclic, fl, grad):
        t = torch.tensor(x, dtype=D, requires_grad=grad)
        r = af2.design_step_seq(t, flags, scalars, ids, None, torch.as_tensor(seq_mask, dtype=D),
                                torch.as_tensor(act_const, dtype=D), emsa, prm, depths, keys,
                                True, tables, tpl_atoms37=tpl37, tpl_mask37=tplm37,
                                cyclic_mode=cyclic, flexibility=fl)
        if not grad:
            return r, None
        loss = sum((a * torch.as_tensor(c, dtype=D)).sum() for a, c in zip(r[:5], cts))
        return r, torch.autograd.grad(loss, (t,))[0]

    ref, dref = oracle(mode, flex, True)
    plain, _ = oracle(None, 0.0, False)

    T = lambda a: None if a is None else torch.as_tensor(a, device=cuda)
    step = ops.DesignStepSeq(*dirs, depths=tuple(depths[k] for k in stacks))
    sc = torch.tensor(scalars, dtype=torch.float32, device=cuda)
    outs, save, _, _ = step.forward(T(x), T(flags), sc, [T(v) for v in ids], T(seq_mask),
                                    act_const=T(act_const), seeds=seeds.to(torch.uint32).to(cuda),
                                    dropout=True, interface_asym=T(iasym), tpl_atoms37=T(tpl37),
                                    tpl_mask37=T(tplm37), cyclic_mode=mode, flexibility=flex)
    dlog = step.backward([T(c) for c in cts], T(x), T(flags), sc, T(seq_mask), save,
                         with_template=True, dropout=True)
    torch.cuda.synchronize()
    for name, g, r, p in zip(("atom14", "distogram", "pae", "plddt", "expres"), outs, ref, plain):
        m = metrics(g.cpu().double(), r.detach())
        away = metrics(g.cpu().double(), p.detach())
        print(f"  {name}", m, "| without the features: rel", away["rel_l2"])
        assert m["rel_l2"] <= 2e-2 and m["max_rel"] <= 2e-2 and m["cos"] >= 0.9999, name
        if name == "distogram":  # the offsets change the pair, the row the msa
            assert away["rel_l2"] > 10 * m["rel_l2"], "the features were not exercised"
    m = metrics(dlog.cpu().double(), dref)
    print("  d logits", m)
    assert m["cos"] >= 0.999 and m["rel_l2"] <= 5e-2


@pytest.mark.parametrize("recycles", [0, 1])
def test_design_step_seq_initial_atom_pos(cuda, recycles):
    """The initial atom positions (bit 2 of the reference's cyclic_mode,
    bc2's large_complex_initialization): the structure module's first frames
    are those of the atoms operand's N, CA, C (all-zero binder rows: the zero
    matrix, as the multimer model's), a recycle pass's those of the previous
    pass's atom37 positions; against the oracle at the step's bars, and far
    from the oracle that starts from the identity."""
    n, nb = 64, 24
    print(f"design step initial atom positions n={n} recycles={recycles}", flush=True)
    depths = {"tpl": 1, "extra": 1, "main": 1, "fold": 2}
    rng = np.random.default_rng(9600 + recycles)
    prm = {"emb": bparams.init_embedder_params(rng),
           "tpl": bparams.init_template_embedding_params(depths["tpl"], rng, gates="random",
                                                         ln="random"),
           "extra": _extra_params(depths["extra"], rng),
           "main": bparams.init_block_params(0, rng, gates="random", ln="random"),
           "post": bparams.init_structure_heads_params(rng, final="random", ln="random")}
    prm["emb"]["param/prev_pos_linear/weights"] *= 1e-3  # see test_gpu_design_step.py
    tables = bparams.init_residue_tables(rng)
    prm["post"].update({f"const/{k}": v for k, v in tables.items()})
    dirs = [weights_dir(prm[k], f"dsi_{k}_{recycles}") for k in ("emb", "tpl", "extra", "main",
                                                                 "post")]
    stacks = ("tpl", "extra", "main", "fold")
    x = rng.standard_normal((n, 20)).astype(np.float32)
    x[nb:] = np.eye(20, dtype=np.float32)[rng.integers(0, 20, n - nb)]
    flags = np.zeros(n, np.uint8)
    flags[:nb] = 1
    flags[nb:] = 2
    ids = [np.concatenate([np.arange(nb), np.arange(n - nb)]), np.repeat([1, 2], [nb, n - nb]),
           np.repeat([1, 2], [nb, n - nb]), np.ones(n)]
    ids = [v.astype(np.float32) for v in ids]
    seq_mask = np.ones(n, np.float32)
    tpl37 = (8 * rng.standard_normal((n, 37, 3))).astype(np.float32)
    tpl37[:nb] = 0.0  # the binder has no atoms yet
    tplm37 = (rng.random((n, 37)) < 0.9).astype(np.float32)
    tplm37[:nb] = 0.0
    act_const = (0.5 * rng.standard_normal((n, n, 64))).astype(np.float32)
    scalars = (0.8, 0.25, 1.2, 1.5)
    keys = [{k: J.prng_key(900 + 10 * p + i) for i, k in enumerate(stacks)}
            for p in range(recycles + 1)]
    seeds = torch.tensor([[int(kp[k][0]), int(kp[k][1]), 1] for kp in keys for k in stacks],
                         dtype=torch.int64)
    shapes = ((n, 14, 3), (n, n, 64), (n, n, 64), (n, 50), (n, 37))
    cts = [rng.standard_normal(sh).astype(np.float32) for sh in shapes]
    emsa = torch.as_tensor(rng.standard_normal((1, n, 64)), dtype=D)

    def oracle(init, grad):
        t = torch.tensor(x, dtype=D, requires_grad=grad)
        r = af2.design_step_seq(t, flags, scalars, ids, None, torch.as_tensor(seq_mask, dtype=D),
                                torch.as_tensor(act_const, dtype=D), emsa, prm, depths, keys,
                                True, tables, recycles=recycles, tpl_atoms37=tpl37,
                                tpl_mask37=tplm37, cyclic_mode="direction",
                                initial_atom_pos=init)
        if not grad:
            return r, None
        loss = sum((a * torch.as_tensor(c, dtype=D)).sum() for a, c in zip(r[:5], cts))
        return r, torch.autograd.grad(loss, (t,))[0]

    ref, dref = oracle(True, True)
    plain, _ = oracle(False, False)

    T = lambda a: None if a is None else torch.as_tensor(a, device=cuda)
    step = ops.DesignStepSeq(*dirs, depths=tuple(depths[k] for k in stacks))
    sc = torch.tensor(scalars, dtype=torch.float32, device=cuda)
    outs, save, _ = step.forward(T(x), T(flags), sc, [T(v) for v in ids], T(seq_mask),
                                 act_const=T(act_const), seeds=seeds.to(torch.uint32).to(cuda),
                                 dropout=True, recycles=recycles, tpl_atoms37=T(tpl37),
                                 tpl_mask37=T(tplm37), cyclic_mode="direction",
                                 initial_atom_pos=True)[:3]
    dlog = step.backward([T(c) for c in cts], T(x), T(flags), sc, T(seq_mask), save,
                         with_template=True, dropout=True)
    torch.cuda.synchronize()
    for name, g, r, p in zip(("atom14", "distogram", "pae", "plddt", "expres"), outs, ref, plain):
        m = metrics(g.cpu().double(), r.detach())
        away = metrics(g.cpu().double(), p.detach())
        print(f"  {name}", m, "| from the identity: rel", away["rel_l2"])
        assert m["rel_l2"] <= 2e-2 and m["max_rel"] <= 2e-2 and m["cos"] >= 0.9999, name
        if name == "atom14":
            assert away["rel_l2"] > 10 * m["rel_l2"], "the initial positions were not exercised"
    m = metrics(dlog.cpu().double(), dref)
    print("  d logits", m)
    assert m["cos"] >= 0.999 and m["rel_l2"] <= 5e-2
