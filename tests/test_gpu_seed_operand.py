"""The reference caller's own seed operand, u32[2] = [bits, enabled]
(modules_multimer.py:591-592, :660-667, :778-779: jax.random.bits of the
stack's subkey and the traced use_dropout), through the three stack entry
points that take it (bc2n_evoformer_*, bc2n_tplstack_*, bc2n_tplembed_*).

The library keys a stack given [bits, enabled] with PRNGKey(bits) = (0, bits)
(threefry_seed of a 32-bit seed).  Checked against the fp64 oracle keyed by
that key; bit-equal to the same stack called with the 3-word operand
[0, bits, enabled]; and [bits, 0] (use_dropout traced off) bit-equal to the
call with dropout off."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import assert_act, assert_grad, random_mask, weights_dir

pytestmark = pytest.mark.gpu
D = torch.float64
BITS = 0x9E3779B9  # above 2^31: the word is taken unsigned


def _seeds(dev):
    two = ops.bits_seed_tensor(BITS, True, dev)
    assert two.numel() == 2 and two.dtype == torch.uint32
    three = ops.seed_tensor(J.prng_key(BITS), True, dev)  # (0, bits, 1)
    off = ops.bits_seed_tensor(BITS, False, dev)
    return two, three, off


def test_evoformer_bits_seed(cuda):
    n, s, depth = 32, 2, 1
    print(f"evoformer [bits, enabled] seed n={n} s={s} depth={depth}", flush=True)
    rng = np.random.default_rng(61)
    prm = bparams.init_block_params(0, rng, gates="random", ln="random")
    st = ops.EvoformerStack(weights_dir(prm, "seed2_evo"), depth)
    pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    msa = rng.standard_normal((s, n, 256)).astype(np.float32)
    pmask, m1 = random_mask(n, 0.1, rng)
    mmask = np.tile(m1, (s, 1)).astype(np.float32)
    ct_pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    ct_msa = rng.standard_normal((s, n, 256)).astype(np.float32)
    T = lambda a: torch.as_tensor(a, device=cuda)
    two, three, off = _seeds(cuda)
    res = {}
    for name, seed, drop in (("two", two, True), ("three", three, True), ("off", off, True),
                             ("nodrop", None, False)):
        po, mo, sv = st.forward(T(pair), T(msa), T(pmask), T(mmask), seed, dropout=drop)
        dp, dm = st.backward(T(ct_pair), T(ct_msa), T(pmask), T(mmask), sv, seed, dropout=drop)
        res[name] = [t.clone() for t in (po, mo, dp, dm)]
    torch.cuda.synchronize()
    for a, b in zip(res["two"], res["three"]):
        assert torch.equal(a, b), "[bits, 1] differs from [0, bits, 1]"
    for a, b in zip(res["off"], res["nodrop"]):
        assert torch.equal(a, b), "[bits, 0] differs from dropout off"
    assert not torch.equal(res["two"][0], res["nodrop"][0])

    x = torch.tensor(pair, dtype=D, requires_grad=True)
    y = torch.tensor(msa, dtype=D, requires_grad=True)
    rm, rp = af2.evoformer_stack(y, x, torch.as_tensor(mmask, dtype=D),
                                 torch.as_tensor(pmask, dtype=D), prm, depth, J.prng_key(BITS),
                                 True)
    gx, gy = torch.autograd.grad((rp, rm), (x, y), (torch.as_tensor(ct_pair, dtype=D),
                                                    torch.as_tensor(ct_msa, dtype=D)))
    po, mo, dp, dm = (t.cpu().double() for t in res["two"])
    print(" pair", assert_act(po - x.detach(), rp.detach() - x.detach(), what="pair"))
    print(" msa", assert_act(mo - y.detach(), rm.detach() - y.detach(), what="msa"))
    print(" dpair", assert_grad(dp, gx, what="dpair"))
    print(" dmsa", assert_grad(dm, gy, what="dmsa"))


def test_template_stack_bits_seed(cuda):
    n, depth = 32, 1
    print(f"template stack [bits, enabled] seed n={n} depth={depth}", flush=True)
    rng = np.random.default_rng(62)
    prm = bparams.init_template_block_params(0, rng, gates="random", ln="random")
    st = ops.TemplatePairStack(weights_dir(prm, "seed2_tpl"), depth)
    pair = rng.standard_normal((n, n, 64)).astype(np.float32)
    mask, _ = random_mask(n, 0.1, rng)
    ct = rng.standard_normal((n, n, 64)).astype(np.float32)
    T = lambda a: torch.as_tensor(a, device=cuda)
    two, three, off = _seeds(cuda)
    res = {}
    for name, seed, drop in (("two", two, True), ("three", three, True), ("off", off, True),
                             ("nodrop", None, False)):
        out, sv = st.forward(T(pair), T(mask), seed, dropout=drop)
        dp = st.backward(T(ct), T(mask), sv, seed, dropout=drop)
        res[name] = [out.clone(), dp.clone()]
    torch.cuda.synchronize()
    for a, b in zip(res["two"], res["three"]):
        assert torch.equal(a, b), "[bits, 1] differs from [0, bits, 1]"
    for a, b in zip(res["off"], res["nodrop"]):
        assert torch.equal(a, b), "[bits, 0] differs from dropout off"
    assert not torch.equal(res["two"][0], res["nodrop"][0])

    x = torch.tensor(pair, dtype=D, requires_grad=True)
    ref = af2.template_stack(x, torch.as_tensor(mask, dtype=D), prm, depth, J.prng_key(BITS), True)
    (g,) = torch.autograd.grad(ref, x, torch.as_tensor(ct, dtype=D))
    out, dp = (t.cpu().double() for t in res["two"])
    print(" out", assert_act(out - x.detach(), ref.detach() - x.detach(), what="delta"))
    print(" dpair", assert_grad(dp, g, what="dpair"))


def test_template_embedding_bits_seed(cuda):
    n, depth = 32, 1
    print(f"template embedding [bits, enabled] seed n={n} depth={depth}", flush=True)
    rng = np.random.default_rng(63)
    prm = bparams.init_template_embedding_params(depth, rng, gates="random", ln="random")
    # keep the relu away from its hinge (see test_gpu_tplembed.py)
    prm["param/output_layer_norm/offset"] = prm["param/output_layer_norm/offset"] + np.float32(5.0)
    te = ops.TemplateEmbedding(weights_dir(prm, "seed2_tpe"), depth)
    query = rng.standard_normal((n, n, 128)).astype(np.float32)
    act_const = rng.standard_normal((n, n, 64)).astype(np.float32)
    mask, _ = random_mask(n, 0.1, rng)
    ct = rng.standard_normal((n, n, 128)).astype(np.float32)
    T = lambda a: torch.as_tensor(a, device=cuda)
    two, three, off = _seeds(cuda)
    res = {}
    for name, seed, drop in (("two", two, True), ("three", three, True), ("off", off, True),
                             ("nodrop", None, False)):
        out, sv = te.forward(T(query), T(act_const), T(mask), seed, dropout=drop)
        dq = te.backward(T(ct), T(query), T(act_const), T(mask), sv, seed, dropout=drop)
        res[name] = [out.clone(), dq.clone()]
    torch.cuda.synchronize()
    for a, b in zip(res["two"], res["three"]):
        assert torch.equal(a, b), "[bits, 1] differs from [0, bits, 1]"
    for a, b in zip(res["off"], res["nodrop"]):
        assert torch.equal(a, b), "[bits, 0] differs from dropout off"
    assert not torch.equal(res["two"][0], res["nodrop"][0])

    x = torch.tensor(query, dtype=D, requires_grad=True)
    ref = af2.template_embedding(x, torch.as_tensor(act_const, dtype=D), torch.as_tensor(mask, dtype=D),
                                 prm, depth, J.prng_key(BITS), True)
    (g,) = torch.autograd.grad(ref, x, torch.as_tensor(ct, dtype=D))
    out, dq = (t.cpu().double() for t in res["two"])
    print(" out", assert_act(out, ref.detach(), what="out"))
    print(" dquery", assert_grad(dq, g, what="dquery"))
