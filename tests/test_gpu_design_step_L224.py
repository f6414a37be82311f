"""GPU parity of the one-call design step (bc2n_design_step_seq_*) at the size
and setup bench.py times it (`design_step_ms`, configs[3]): L = 224 (160
target + 64 designed residues), depths 2 / 4 / 48 / 8 (template stack,
extra stack, main stack, fold), the template's MSA row in the main stack
(S = 2), dropout on with JAX keys, 10% of residues masked, confidence
metrics, atom37 aligned on the template, one forward-only recycle pass, and
the backward to d(logits); weights drawn as bench.py draws them (the AF2
tree through the weights writers, full-strength prev_pos_linear).

The oracle is oracle.af2.design_step_seq in f32 with per-block recompute
(oracle.af2.block_recompute), run on the host's cores.

Recycling: the recycle pass hands its atoms to the next pass through the
distogram of their pseudo-beta positions (15 bins, a step function), so a
pair whose positions straddle a bin edge by less than the trunk's rounding
takes another bin.  The test counts those flips between the kernels' and the
oracle's first-pass atoms, prints the count and bounds it; the end-to-end
comparison then feeds the oracle's second pass the kernels' own first-pass
atoms (the bins the kernels used), so the outputs and d(logits) are held to
the north star's bars without the flips in them.  The kernels' first-pass
atoms come from the same step run with no recycle pass: a detached forward
gives the bits of a saving one (tests/test_gpu_boundary.py)."""
import os
import tempfile
import time

import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams, weights as W
from oracle import af2, jax_prng as J
from tests.helpers import metrics

pytestmark = pytest.mark.gpu
F = torch.float32
STACKS = ("tpl", "extra", "main", "fold")
DEPTHS = {"tpl": 2, "extra": 4, "main": 48, "fold": 8}


def _say(*a):
    print(*a, flush=True)


@pytest.mark.timeout(1800)
def test_design_step_seq_L224(cuda):
    n, recycles, t0 = 224, 1, time.time()
    nt = n - 64
    _say(f"design step from logits L={n} depths={DEPTHS} S=2 dropout=on recycles={recycles}")
    rng = np.random.default_rng(224)
    tree = W.init_af2_params(rng, num_blocks=48, extra_blocks=4, template_blocks=2)
    tables = bparams.init_residue_tables(rng)
    root = tempfile.mkdtemp(prefix="bc2n_ds224_")
    dirs = [W.embed_weights_from_params(tree, os.path.join(root, "emb")),
            W.tplembed_weights_from_params(tree, os.path.join(root, "tpl")),
            W.stack_weights_from_params(tree, os.path.join(root, "extra"), prefix=W.EXTRA),
            W.stack_weights_from_params(tree, os.path.join(root, "main"), prefix=W.MAIN),
            W.post_weights_from_params(tree, os.path.join(root, "post"), tables=tables)]
    prm = {k: bparams.read_manifest(d) for k, d in zip(("emb", "tpl", "extra", "main", "post"),
                                                         dirs)}
    del tree

    m1 = np.ones(n, np.float32)
    m1[rng.choice(n, int(round(0.1 * n)), replace=False)] = 0
    logits = (0.5 * rng.standard_normal((n, 20))).astype(np.float32)
    logits[:nt] = np.eye(20, dtype=np.float32)[rng.integers(0, 20, nt)]
    flags = np.zeros(n, np.uint8)
    flags[nt:] = 1  # the binder is designed
    flags[:nt] = 2  # the target is the template: its MSA row joins the stack (S = 2)
    scalars = (1.0, 0.0, 1.0, 1.0)
    chain = (np.arange(n) >= nt).astype(np.float32)
    ids = [np.arange(n, dtype=np.float32), chain + 1, chain + 1, np.ones(n, np.float32)]
    iasym = chain.astype(np.int32)
    act_const = (0.1 * rng.standard_normal((n, n, 64))).astype(np.float32)
    tpl37 = (8.0 * rng.standard_normal((n, 37, 3))).astype(np.float32)
    tplm37 = np.ones((n, 37), np.float32)
    emsa = rng.standard_normal((1, n, 64)).astype(np.float32)
    keys = [{k: J.prng_key(11 + 4 * p + i) for i, k in enumerate(STACKS)}
            for p in range(recycles + 1)]
    seeds = torch.tensor([[int(keys[p][k][0]), int(keys[p][k][1]), 1]
                          for p in range(recycles + 1) for k in STACKS], dtype=torch.int64)
    seeds = seeds.to(torch.uint32).to(cuda)
    shapes = ((n, 14, 3), (n, n, 64), (n, n, 64), (n, 50), (n, 37),
              (n,), (n, n), (1,), (1,), (n,), (n,))
    cts = [rng.standard_normal(sh).astype(np.float32) for sh in shapes]
    ct37 = rng.standard_normal((n, 37, 3)).astype(np.float32)

    T = lambda a: None if a is None else torch.as_tensor(a, device=cuda)
    step = ops.DesignStepSeq(*dirs, depths=tuple(DEPTHS[k] for k in STACKS))
    sc = T(np.array(scalars, np.float32))
    args = (T(logits), T(flags), sc, [T(v) for v in ids], T(m1))
    kw = dict(act_const=T(act_const), interface_asym=T(iasym), atom37=True, tpl_atoms37=T(tpl37),
              tpl_mask37=T(tplm37))
    # the kernels' first-pass atoms: the step with no recycle pass, pass-0 keys
    outs0 = step.forward(*args, seeds=seeds[:4].contiguous(), recycles=0, **kw)[0]
    gpu_atoms0 = outs0[0].cpu().double()
    outs, save, conf, (g37, gm37) = step.forward(*args, seeds=seeds, recycles=recycles, **kw)
    dlog = step.backward([T(c) for c in cts[:5]], T(logits), T(flags), sc, T(m1), save,
                         interface_asym=T(iasym), conf_cts=[T(c) for c in cts[5:]],
                         d_atom37=T(ct37))
    torch.cuda.synchronize()
    got = [t.cpu().double() for t in list(outs) + list(conf) + [g37, dlog]]
    del save
    torch.cuda.empty_cache()
    _say(f"  gpu done {time.time() - t0:.0f}s")

    flips = {}

    def feed_gpu_atoms(p, atoms):
        aat = af2.design_inputs(*af2.sequence_features(
            torch.as_tensor(logits, dtype=torch.float64), flags, *scalars))[2]
        pair_ok = torch.as_tensor(m1, dtype=torch.float64)
        pair_ok = (pair_ok[:, None] * pair_ok[None]) > 0
        bins = lambda a: af2.dgram_from_positions(
            af2.pseudo_beta_atom14(aat, torch.as_tensor(a, dtype=torch.float64)))
        flips["n"] = int(((bins(atoms) != bins(gpu_atoms0)).any(-1) & pair_ok).sum())
        flips["atoms"] = metrics(gpu_atoms0, atoms.double())
        _say(f"  oracle pass {p} done {time.time() - t0:.0f}s; first-pass atoms "
             f"{flips['atoms']}; distogram bins that differ: {flips['n']} of {int(pair_ok.sum())} "
             "live pairs")
        return gpu_atoms0

    t = torch.tensor(logits, dtype=F, requires_grad=True)
    with af2.block_recompute():
        ref = af2.design_step_seq(t, flags, scalars, ids, None, torch.as_tensor(m1, dtype=F),
                                  torch.as_tensor(act_const), torch.as_tensor(emsa), prm, DEPTHS,
                                  keys, True, tables, recycles=recycles, tpl_atoms37=tpl37,
                                  tpl_mask37=tplm37, dtype=F, on_pass=feed_gpu_atoms)
        ref = list(ref)
        conf_ref = af2.confidence(ref[3], ref[2], ref[4], torch.as_tensor(m1, dtype=F), iasym)
        outs_ref = ref[:5] + list(conf_ref) + [ref[5]]
        loss = sum((r * torch.as_tensor(c, dtype=F)).sum() for r, c in zip(outs_ref[:11], cts))
        loss = loss + (ref[5] * torch.as_tensor(ct37)).sum()
        _say(f"  oracle forward done {time.time() - t0:.0f}s")
        (dref,) = torch.autograd.grad(loss, (t,))
    _say(f"  oracle backward done {time.time() - t0:.0f}s")

    assert torch.equal(gm37.cpu().double(), ref[6].detach().double()), "atom37 exists mask"
    names = ("atom14", "distogram", "pae", "plddt", "expres", "conf plddt", "conf pae", "ptm",
             "iptm", "iptm_per_residue", "expres_ca", "atom37 aligned", "d logits")
    refs = [r.detach().double() for r in outs_ref] + [dref.double()]
    bad = []
    for i, (name, g, r) in enumerate(zip(names, got, refs)):
        m = metrics(g, r)
        _say(f"  {name}", m)
        if name in ("ptm", "iptm"):  # scalars: relative error only
            ok = m["rel_l2"] <= 2e-2
        elif name == "d logits":
            ok = m["cos"] >= 0.999 and m["rel_l2"] <= 5e-2
        else:
            ok = m["rel_l2"] <= 2e-2 and m["max_rel"] <= 2e-2 and m["cos"] >= 0.9999
        if not ok:
            bad.append(name)
    # a flip needs |d| within the rounding of a bin edge: a wrong atom, bin
    # edge or glycine rule moves most of the 15-bin histogram instead
    live = int((m1 > 0).sum()) ** 2
    assert flips["n"] <= 0.02 * live, f"{flips['n']} distogram bins differ"
    # the first pass's atoms (one trunk pass and the structure module) at the
    # activation bar; the recycled pass compounds two passes' roundings
    fa = flips["atoms"]
    assert fa["max_rel"] <= 2e-2 and fa["rel_l2"] <= 2e-2 and fa["cos"] >= 0.9999, fa
    assert not bad, f"outside the bars: {bad}"
    _say(f"  total {time.time() - t0:.0f}s")
