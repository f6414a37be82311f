"""GPU parity of the Evoformer stack (the native_evoformer_fwd/bwd drop-in)
against the fp64 oracle stack: same weights, inputs, masks and JAX stack key,
dropout on, gradients w.r.t. both the pair and the MSA input."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import assert_act, assert_grad, metrics, random_mask, weights_dir

pytestmark = pytest.mark.gpu
D = torch.float64


def _params(depth, rng, pair_only=False):
    prm = {}
    for b in range(depth):
        prm.update(bparams.init_block_params(b, rng, gates="random", ln="random"))
    return prm


@pytest.mark.parametrize("depth,n,s,dropout", [(1, 32, 1, False), (2, 32, 2, True),
                                               (2, 64, 1, True)])
def test_stack_parity(cuda, depth, n, s, dropout):
    print(f"stack depth={depth} n={n} s={s} dropout={dropout}", flush=True)
    rng = np.random.default_rng(depth * 1000 + n + s)
    prm = _params(depth, rng)
    wdir = weights_dir(prm, f"stack_{depth}_{n}_{s}")
    pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    msa = rng.standard_normal((s, n, 256)).astype(np.float32)
    pmask, m1 = random_mask(n, 0.1, rng)
    mmask = np.tile(m1, (s, 1)).astype(np.float32)
    ct_pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    ct_msa = rng.standard_normal((s, n, 256)).astype(np.float32)
    key = J.prng_key(777 + n)

    st = ops.EvoformerStack(wdir, depth)
    T = lambda a: torch.as_tensor(a, device=cuda)
    seed = ops.seed_tensor(key, enabled=True, device=cuda)
    po, mo, save = st.forward(T(pair), T(msa), T(pmask), T(mmask), seed, dropout=dropout)
    dp, dm = st.backward(T(ct_pair), T(ct_msa), T(pmask), T(mmask), save, seed, dropout=dropout)
    torch.cuda.synchronize()

    x = torch.tensor(pair, dtype=D, requires_grad=True)
    y = torch.tensor(msa, dtype=D, requires_grad=True)
    rm, rp = af2.evoformer_stack(y, x, torch.as_tensor(mmask, dtype=D), torch.as_tensor(pmask, dtype=D),
                                 prm, depth, key if dropout else None, dropout)
    gx, gy = torch.autograd.grad((rp, rm), (x, y), (torch.as_tensor(ct_pair, dtype=D),
                                                    torch.as_tensor(ct_msa, dtype=D)))
    print(" pair delta", assert_act((po.cpu().double() - x.detach()), rp.detach() - x.detach(), what="pair"))
    print(" msa delta", assert_act((mo.cpu().double() - y.detach()), rm.detach() - y.detach(), what="msa"))
    print(" dpair", assert_grad(dp.cpu().double(), gx, what="dpair"))
    print(" dmsa", assert_grad(dm.cpu().double(), gy, what="dmsa"))


def test_stack_dropout_is_keyed(cuda):
    """Same key -> identical output; different key or disabled flag -> different."""
    n, s, depth = 32, 1, 1
    rng = np.random.default_rng(5)
    prm = _params(depth, rng)
    wdir = weights_dir(prm, "stack_keyed")
    T = lambda a: torch.as_tensor(a, device=cuda)
    pair = T(rng.standard_normal((n, n, 128)).astype(np.float32))
    msa = T(rng.standard_normal((s, n, 256)).astype(np.float32))
    pm, mm = T(np.ones((n, n), np.float32)), T(np.ones((s, n), np.float32))
    st = ops.EvoformerStack(wdir, depth)
    a = st.forward(pair, msa, pm, mm, ops.seed_tensor(J.prng_key(1), True, cuda))[0].clone()
    b = st.forward(pair, msa, pm, mm, ops.seed_tensor(J.prng_key(1), True, cuda))[0].clone()
    c = st.forward(pair, msa, pm, mm, ops.seed_tensor(J.prng_key(2), True, cuda))[0].clone()
    d = st.forward(pair, msa, pm, mm, ops.seed_tensor(J.prng_key(1), False, cuda))[0].clone()
    e = st.forward(pair, msa, pm, mm, None, dropout=False)[0].clone()
    assert torch.equal(a, b)
    assert not torch.equal(a, c)
    assert not torch.equal(a, d)
    assert torch.equal(d, e)


@pytest.mark.parametrize("n,s,depth,policy", [(64, 2, 2, "full"), (224, 1, 3, "full"),
                                              (96, 2, 2, "replay")])
def test_stack_msa_overlap_bit_identical(cuda, n, s, depth, policy):
    """The MSA side of each block on the library's second stream (the
    default) gives exactly the bits of the single-stream order, forward and
    backward, under both save tiers."""
    print(f"stack msa overlap n={n} s={s} depth={depth} policy={policy}", flush=True)
    rng = np.random.default_rng(8800 + n)
    prm = _params(depth, rng)
    st = ops.EvoformerStack(weights_dir(prm, f"overlap_{n}_{s}_{policy}"), depth)
    T = lambda a: torch.as_tensor(a, device=cuda)
    pmask, m1 = random_mask(n, 0.1, rng)
    pmask, mmask = T(pmask), T(np.tile(m1, (s, 1)).astype(np.float32))
    pair = T(rng.standard_normal((n, n, 128)).astype(np.float32))
    msa = T(rng.standard_normal((s, n, 256)).astype(np.float32))
    ct_p, ct_m = torch.randn_like(pair), torch.randn_like(msa)
    seed = ops.seed_tensor(J.prng_key(31), True, cuda)
    res = []
    with ops.save_policy(policy):
        for on in (False, True, True):
            with ops.msa_overlap(on):
                po, mo, sv = st.forward(pair, msa, pmask, mmask, seed)
                dp, dm = st.backward(ct_p, ct_m, pmask, mmask, sv, seed)
                res.append([t.clone() for t in (po, mo, dp, dm)])
    torch.cuda.synchronize()
    for r in res[1:]:
        for a, b in zip(res[0], r):
            assert torch.equal(a, b)
