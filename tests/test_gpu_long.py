"""GPU tests of the long-length path: the stacks' replay save tier and a
stack past L = 512.

The replay tier keeps every block's input carries and one block's module
save-sets; the backward runs each block's forward again into that region
before the block's backward (the role of the reference's replay/remat tiers,
native/stack.cuh:775-798).  It must give the full tier's bits exactly: the
recompute runs the same deterministic kernels on the same inputs with the
same dropout tables.  At L = 768 -- beyond the no-replay save-set one GPU
holds for 48 blocks (about 325 GB) -- a depth-2 stack under the replay tier
is held to the north-star bars against the fp32 oracle; it runs the
eight-wave dK/dV kernel of N > 512.  The single modules at 768 are in
test_gpu_triattn.py, test_gpu_trimul.py and test_gpu_fold.py."""
import time

import numpy as np
import pytest
import torch

from bindcraft2_amd import lib, ops, params as bparams
from oracle import af2, jax_prng as J
from tests import trunk_ref as R
from tests.helpers import assert_act, assert_grad, weights_dir

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)


@pytest.mark.parametrize("kind", ["evoformer", "pair_only", "template"])
def test_replay_tier_gives_the_full_tiers_bits(cuda, kind):
    n, depth = 64, 3
    _say(f"replay tier {kind} n={n} depth={depth}")
    rng = np.random.default_rng(77)
    evo, extra, tpl = bparams.init_trunk_params(rng, depth=depth, extra_depth=depth,
                                                tpl_depth=depth)
    m1 = np.ones(n, np.float32)
    m1[rng.choice(n, 6, replace=False)] = 0
    T = lambda a: torch.as_tensor(a, device=cuda)
    pmask = T(np.outer(m1, m1).astype(np.float32))
    seed = ops.seed_tensor(J.prng_key(31), True, cuda)
    s = 2 if kind == "evoformer" else 1
    c = {"evoformer": 128, "pair_only": 128, "template": 64}[kind]
    cm = {"evoformer": 256, "pair_only": 64, "template": 0}[kind]
    pair = T(rng.standard_normal((n, n, c)).astype(np.float32))
    ct = T(rng.standard_normal((n, n, c)).astype(np.float32))
    msa = T(rng.standard_normal((s, n, max(cm, 1))).astype(np.float32))
    ct_msa = T(rng.standard_normal((s, n, max(cm, 1))).astype(np.float32))
    mmask = T(np.repeat(m1[None], s, 0) if kind == "evoformer" else np.zeros((1, n), np.float32))
    if kind == "template":
        st = ops.TemplatePairStack(weights_dir(tpl, f"rp_tpl"), depth)
    else:
        st = ops.EvoformerStack(weights_dir(evo if kind == "evoformer" else extra, f"rp_{kind}"),
                                depth, pair_only=kind == "pair_only", c_m=cm)

    def run(policy):
        with ops.save_policy(policy):
            if kind == "template":
                out, save = st.forward(pair, pmask, seed)
                d = st.backward(ct, pmask, save, seed)
                res, nbytes = (out, d), save.numel()
            else:
                po, mo, save = st.forward(pair, msa, pmask, mmask, seed)
                dp, dm = st.backward(ct, ct_msa, pmask, mmask, save, seed)
                res, nbytes = (po, mo, dp, dm), save.numel()
                if kind == "evoformer":
                    flag = lib().bc2n_evoformer_replays(st.dir, n, s, depth, 0)
                    assert flag == (1 if policy == "replay" else 0), flag
            torch.cuda.synchronize()
            return [r.clone() for r in res], nbytes

    full, b_full = run("full")
    replay, b_replay = run("replay")
    _say(f"  save-set {b_full / 1e6:.1f} MB full, {b_replay / 1e6:.1f} MB replay")
    assert b_replay < b_full
    for a, b in zip(full, replay):
        assert torch.equal(a, b)


@pytest.mark.timeout(1500)
def test_stack_L768_replay_depth2(cuda):
    n, depth, t0 = 768, 2, time.time()
    _say(f"stack L={n} depth={depth} s=1 dropout=on mask=0.1, replay tier")
    rng = np.random.default_rng(768)
    m1 = np.ones(n, np.float32)
    m1[rng.choice(n, int(round(0.1 * n)), replace=False)] = 0
    evo, _, _ = bparams.init_trunk_params(rng, depth=depth, extra_depth=0, tpl_depth=0)
    pmask = np.outer(m1, m1).astype(np.float32)
    mmask = m1[None].copy()
    pair0 = rng.standard_normal((n, n, 128)).astype(np.float32)
    msa0 = rng.standard_normal((1, n, 256)).astype(np.float32)
    ct_pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    ct_msa = rng.standard_normal((1, n, 256)).astype(np.float32)
    key = J.prng_key(7680)

    st = ops.EvoformerStack(weights_dir(evo, "stack768"), depth)
    T = lambda a: torch.as_tensor(a, device=cuda)
    seed = ops.seed_tensor(key, True, cuda)
    with ops.save_policy("replay"):
        assert lib().bc2n_evoformer_replays(st.dir, n, 1, depth, 0) == 1
        pm, mm, save = st.forward(T(pair0), T(msa0), T(pmask), T(mmask), seed)
        dp, dm = st.backward(T(ct_pair), T(ct_msa), T(pmask), T(mmask), save, seed)
    torch.cuda.synchronize()
    got = [x.cpu().double() for x in (pm, mm, dp, dm)]
    del save
    torch.cuda.empty_cache()
    _say(f"  gpu done {time.time() - t0:.0f}s")

    bm = R.evoformer_block(evo, torch.as_tensor(pmask), torch.as_tensor(mmask), True,
                           torch.float32)
    km = af2.stack_block_keys(key, depth)
    xm = R.stack_forward(bm, (torch.as_tensor(msa0), torch.as_tensor(pair0)), km)
    _say(f"  oracle forward done {time.time() - t0:.0f}s")
    r_mm, r_pm = xm[-1]
    r_dm, r_dp = R.stack_backward(bm, xm, km, (torch.as_tensor(ct_msa), torch.as_tensor(ct_pair)),
                                  progress=lambda b: _say(f"  oracle backward at block {b} "
                                                          f"{time.time() - t0:.0f}s"))
    d = lambda a: torch.as_tensor(a).double()
    _say("  pair", assert_act(got[0] - d(pair0), d(r_pm) - d(pair0), what="pair"))
    _say("  msa", assert_act(got[1] - d(msa0), d(r_mm) - d(msa0), what="msa"))
    _say("  d pair", assert_grad(got[2], d(r_dp), what="dpair"))
    _say("  d msa", assert_grad(got[3], d(r_dm), what="dmsa"))
    _say(f"  total {time.time() - t0:.0f}s")
