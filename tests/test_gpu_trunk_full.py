"""GPU parity of the whole design-step trunk at the benchmark's size, and of
the L=512 trunk of the large-complex configuration, against the fp32 oracle
on the host's cores.

configs[3] (the benchmarked workload, bench.py's default step with the same
weights): the 2-block template pair stack (c_t=64), the 4-block extra-MSA
stack in its pair-only form and the 48-block Evoformer stack at L=224, S=1,
forward and backward, dropout on (JAX keys), 10% of residues masked.  The
stacks are chained as the design step chains them: extra -> main on the
pair, the template stack on its own activations; the backward runs main ->
extra.  The oracle is the reference's JAX trunk restated in oracle/af2.py,
run in fp32 with per-block recompute (tests/trunk_ref.py).

the same chain at L=512 with 8 main-stack blocks, and a 2-block
Evoformer stack at L=512 on its own (the 8-iteration fold at L=512 is in
test_gpu_fold.py, the single modules at L=512 in test_gpu_triattn.py and
test_gpu_trimul.py).

Bars (north star): activations relL2 and max|d|/max|ref| <= 2e-2; gradient
cosine >= 0.999."""
import time

import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests import trunk_ref as R
from tests.helpers import assert_act, assert_grad, metrics, random_mask, weights_dir

pytestmark = pytest.mark.gpu
F = torch.float32


def _say(*a):
    print(*a, flush=True)


def _t(a, dev):
    return torch.as_tensor(a, device=dev)


def _trunk_case(cuda, n, depth, seed):
    t0 = time.time()
    _say(f"trunk {depth}+4+2 blocks n={n} s=1 dropout=on mask=0.1")
    # the benchmark's draws: residue mask, then the three stacks' weights
    rng = np.random.default_rng(seed)
    m1 = np.ones(n, np.float32)
    m1[rng.choice(n, int(round(0.1 * n)), replace=False)] = 0
    evo, extra, tpl = bparams.init_trunk_params(rng, depth=depth)
    pmask = np.outer(m1, m1).astype(np.float32)
    mmask = m1[None].copy()
    emask = np.zeros((1, n), np.float32)
    g = np.random.default_rng(1)
    pair0 = g.standard_normal((n, n, 128)).astype(np.float32)
    msa0 = g.standard_normal((1, n, 256)).astype(np.float32)
    emsa0 = g.standard_normal((1, n, 64)).astype(np.float32)
    tpl0 = g.standard_normal((n, n, 64)).astype(np.float32)
    ct_pair = g.standard_normal((n, n, 128)).astype(np.float32)
    ct_msa = g.standard_normal((1, n, 256)).astype(np.float32)
    ct_tpl = g.standard_normal((n, n, 64)).astype(np.float32)
    keys = [J.prng_key(11 + i) for i in range(3)]  # template, extra, main

    main = ops.EvoformerStack(weights_dir(evo, f"full_main_{n}_{depth}"), depth)
    xst = ops.EvoformerStack(weights_dir(extra, f"full_extra_{n}"), 4, pair_only=True, c_m=64)
    tst = ops.TemplatePairStack(weights_dir(tpl, f"full_tpl_{n}"), 2)
    T = lambda a: _t(a, cuda)
    seeds = [ops.seed_tensor(k, True, cuda) for k in keys]
    to, s_t = tst.forward(T(tpl0), T(pmask), seeds[0])
    pe, _, s_e = xst.forward(T(pair0), T(emsa0), T(pmask), T(emask), seeds[1])
    pm, mm, s_m = main.forward(pe, T(msa0), T(pmask), T(mmask), seeds[2])
    dpe, dmsa = main.backward(T(ct_pair), T(ct_msa), T(pmask), T(mmask), s_m, seeds[2])
    dpair, _ = xst.backward(dpe, torch.zeros(1, n, 64, device=cuda), T(pmask), T(emask), s_e,
                            seeds[1])
    dtpl = tst.backward(T(ct_tpl), T(pmask), s_t, seeds[0])
    torch.cuda.synchronize()
    got = {k: v.cpu().double() for k, v in dict(to=to, pe=pe, pm=pm, mm=mm, dpair=dpair,
                                                 dmsa=dmsa, dtpl=dtpl).items()}
    del s_t, s_e, s_m
    torch.cuda.empty_cache()
    _say(f"  gpu done {time.time() - t0:.0f}s")

    pm_t, mm_t = torch.as_tensor(pmask), torch.as_tensor(mmask)
    bt = R.template_block(tpl, pm_t, True, F)
    be = R.pair_only_block(extra, pm_t, True, F)
    bm = R.evoformer_block(evo, pm_t, mm_t, True, F)
    kt, ke, km = (af2.stack_block_keys(k, d) for k, d in zip(keys, (2, 4, depth)))
    xt = R.stack_forward(bt, (torch.as_tensor(tpl0),), kt)
    r_to = xt[-1][0]
    (r_dtpl,) = R.stack_backward(bt, xt, kt, (torch.as_tensor(ct_tpl),))
    xe = R.stack_forward(be, (torch.as_tensor(pair0),), ke)
    r_pe = xe[-1][0]
    xm = R.stack_forward(bm, (torch.as_tensor(msa0), r_pe), km)
    r_mm, r_pm = xm[-1]
    _say(f"  oracle forward done {time.time() - t0:.0f}s")
    r_dmsa, r_dpe = R.stack_backward(
        bm, xm, km, (torch.as_tensor(ct_msa), torch.as_tensor(ct_pair)),
        progress=lambda b: b % 8 == 0 and _say(f"  oracle backward at block {b} "
                                               f"{time.time() - t0:.0f}s"))
    (r_dpair,) = R.stack_backward(be, xe, ke, (r_dpe,))

    d = lambda a: torch.as_tensor(a).double()
    P0, M0, T0 = d(pair0), d(msa0), d(tpl0)
    _say("  template out", assert_act(got["to"] - T0, d(r_to) - T0, what="template out"))
    _say("  extra pair", assert_act(got["pe"] - P0, d(r_pe) - P0, what="extra pair"))
    _say("  trunk pair", assert_act(got["pm"] - P0, d(r_pm) - P0, what="trunk pair"))
    _say("  trunk msa", assert_act(got["mm"] - M0, d(r_mm) - M0, what="trunk msa"))
    _say("  d pair", assert_grad(got["dpair"], d(r_dpair), what="dpair"))
    _say("  d msa", assert_grad(got["dmsa"], d(r_dmsa), what="dmsa"))
    _say("  d template", assert_grad(got["dtpl"], d(r_dtpl), what="dtpl"))
    _say(f"  total {time.time() - t0:.0f}s")


@pytest.mark.timeout(1500)
def test_trunk_full_depth_L224(cuda):
    _trunk_case(cuda, 224, 48, 0)


@pytest.mark.timeout(1500)
def test_trunk_L512_depth8(cuda):
    """configs[4]'s trunk structure at L=512 (template 2, extra 4, main 8
    blocks), chained as at L=224: the stacks' hand-offs and eight main
    blocks of accumulated rounding at the large-complex length."""
    _trunk_case(cuda, 512, 8, 5120)


@pytest.mark.timeout(900)
def test_stack_L512_depth2(cuda):
    n, depth, t0 = 512, 2, time.time()
    _say(f"stack L={n} depth={depth} s=1 dropout=on mask=0.1")
    rng = np.random.default_rng(512)
    m1 = np.ones(n, np.float32)
    m1[rng.choice(n, int(round(0.1 * n)), replace=False)] = 0
    evo, _, _ = bparams.init_trunk_params(rng, depth=depth, extra_depth=0, tpl_depth=0)
    pmask = np.outer(m1, m1).astype(np.float32)
    mmask = m1[None].copy()
    pair0 = rng.standard_normal((n, n, 128)).astype(np.float32)
    msa0 = rng.standard_normal((1, n, 256)).astype(np.float32)
    ct_pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    ct_msa = rng.standard_normal((1, n, 256)).astype(np.float32)
    key = J.prng_key(4000)

    st = ops.EvoformerStack(weights_dir(evo, "stack512"), depth)
    T = lambda a: _t(a, cuda)
    seed = ops.seed_tensor(key, True, cuda)
    pm, mm, save = st.forward(T(pair0), T(msa0), T(pmask), T(mmask), seed)
    dp, dm = st.backward(T(ct_pair), T(ct_msa), T(pmask), T(mmask), save, seed)
    torch.cuda.synchronize()
    got = [x.cpu().double() for x in (pm, mm, dp, dm)]
    del save
    torch.cuda.empty_cache()
    _say(f"  gpu done {time.time() - t0:.0f}s")

    bm = R.evoformer_block(evo, torch.as_tensor(pmask), torch.as_tensor(mmask), True, F)
    km = af2.stack_block_keys(key, depth)
    xm = R.stack_forward(bm, (torch.as_tensor(msa0), torch.as_tensor(pair0)), km)
    r_mm, r_pm = xm[-1]
    r_dm, r_dp = R.stack_backward(bm, xm, km, (torch.as_tensor(ct_msa), torch.as_tensor(ct_pair)))
    d = lambda a: torch.as_tensor(a).double()
    _say("  pair", assert_act(got[0] - d(pair0), d(r_pm) - d(pair0), what="pair"))
    _say("  msa", assert_act(got[1] - d(msa0), d(r_mm) - d(msa0), what="msa"))
    _say("  d pair", assert_grad(got[2], d(r_dp), what="dpair"))
    _say("  d msa", assert_grad(got[3], d(r_dm), what="dmsa"))
    _say(f"  total {time.time() - t0:.0f}s")
