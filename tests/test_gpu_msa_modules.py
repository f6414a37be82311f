"""GPU parity of the transition, outer product mean and MSA row/column
attention modules (fwd + bwd) through the C ABI against the fp64 oracle."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import assert_act, assert_grad, random_mask, weights_dir

pytestmark = pytest.mark.gpu
D = torch.float64


def _t(a, dev):
    return torch.as_tensor(np.ascontiguousarray(a), device=dev)


@pytest.mark.parametrize("kind,b,n", [("pair_transition", 32, 32), ("pair_transition", 64, 64),
                                      ("msa_transition", 1, 64), ("msa_transition", 3, 32)])
def test_transition(cuda, kind, b, n):
    print(f"transition {kind} b={b} n={n}", flush=True)
    rng = np.random.default_rng(b * 100 + n)
    prm = bparams.init_block_params(0, rng, modules=[kind], gates="random", ln="random")
    wdir = weights_dir(prm, f"tr_{kind}_{b}_{n}")
    c = 128 if kind == "pair_transition" else 256
    act = rng.standard_normal((b, n, c)).astype(np.float32)
    dout = rng.standard_normal((b, n, c)).astype(np.float32)
    mod = ops.Transition(wdir, f"param/block0/{kind}/", c)
    ta, td = _t(act, cuda), _t(dout, cuda)
    out, save = mod.forward(ta)
    din = mod.backward(ta, None, save, td)
    P = af2.Params(prm, f"param/block0/{kind}/")
    x = torch.tensor(act, dtype=D, requires_grad=True)
    ref = af2.transition(x, None, P)
    (g,) = torch.autograd.grad(ref, x, torch.as_tensor(dout, dtype=D))
    print(assert_act((out - ta).cpu().double(), ref.detach(), what="delta"),
          assert_grad((din - td).cpu().double(), g, what="dact"))


@pytest.mark.parametrize("b,n", [(5, 20), (3, 50)])
def test_pair_transition_ragged_rows_with_dropout_table(cuda, b, n):
    """Row counts that are not a multiple of the fused kernel's 64-row tile,
    and the shared dropout table (row m takes table row m % n) on both the
    residual add and the cotangent."""
    print(f"pair transition + dropout table b={b} n={n}", flush=True)
    rng = np.random.default_rng(7 * b + n)
    prm = bparams.init_block_params(0, rng, modules=["pair_transition"], gates="random",
                                    ln="random")
    wdir = weights_dir(prm, f"trd_{b}_{n}")
    act = rng.standard_normal((b, n, 128)).astype(np.float32)
    dout = rng.standard_normal((b, n, 128)).astype(np.float32)
    tbl = ((rng.random((n, 128)) > 0.25) / 0.75).astype(np.float32)
    mod = ops.Transition(wdir, "param/block0/pair_transition/", 128)
    ta, td, tt = _t(act, cuda), _t(dout, cuda), _t(tbl, cuda)
    out, save = mod.forward(ta, tt)
    din = mod.backward(ta, tt, save, td)
    P = af2.Params(prm, "param/block0/pair_transition/")
    x = torch.tensor(act, dtype=D, requires_grad=True)
    ref = torch.as_tensor(tbl, dtype=D)[None] * af2.transition(x, None, P)
    (g,) = torch.autograd.grad(ref, x, torch.as_tensor(dout, dtype=D))
    print(assert_act((out - ta).cpu().double(), ref.detach(), what="delta"),
          assert_grad((din - td).cpu().double(), g, what="dact"))


@pytest.mark.parametrize("s,n,mfrac", [(1, 32, 0.0), (1, 64, 0.1), (3, 32, 0.2)])
def test_outer_product_mean(cuda, s, n, mfrac):
    print(f"opm s={s} n={n}", flush=True)
    rng = np.random.default_rng(s * 10 + n)
    prm = bparams.init_block_params(0, rng, modules=["outer_product_mean"], gates="random", ln="random")
    wdir = weights_dir(prm, f"opm_{s}_{n}")
    msa = rng.standard_normal((s, n, 256)).astype(np.float32)
    mask = (rng.random((s, n)) > mfrac).astype(np.float32)
    pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    dpair = rng.standard_normal((n, n, 128)).astype(np.float32)
    mod = ops.OuterProductMean(wdir, "param/block0/outer_product_mean/")
    tm, tk, tp, td = _t(msa, cuda), _t(mask, cuda), _t(pair, cuda), _t(dpair, cuda)
    out, save = mod.forward(tm, tk, tp)
    dmsa = mod.backward(tm, tk, None, save, td)
    P = af2.Params(prm, "param/block0/outer_product_mean/")
    x = torch.tensor(msa, dtype=D, requires_grad=True)
    ref = af2.outer_product_mean(x, torch.as_tensor(mask, dtype=D), P)
    (g,) = torch.autograd.grad(ref, x, torch.as_tensor(dpair, dtype=D))
    print(assert_act((out - tp).cpu().double(), ref.detach(), what="delta"),
          assert_grad(dmsa.cpu().double(), g, what="dmsa"))


@pytest.mark.parametrize("s,n,mfrac,drop", [(1, 32, 0.0, False), (1, 64, 0.1, True),
                                            (2, 64, 0.1, True)])
def test_msa_row_attention(cuda, s, n, mfrac, drop):
    print(f"msarow s={s} n={n}", flush=True)
    name = "msa_row_attention_with_pair_bias"
    rng = np.random.default_rng(s * 7 + n)
    prm = bparams.init_block_params(0, rng, modules=[name], gates="random", ln="random")
    wdir = weights_dir(prm, f"row_{s}_{n}")
    msa = rng.standard_normal((s, n, 256)).astype(np.float32)
    _, m1 = random_mask(n, mfrac, rng)
    mask = np.tile(m1, (s, 1)).astype(np.float32)
    pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    dout = rng.standard_normal((s, n, 256)).astype(np.float32)
    tbl = af2.dropout_table(J.prng_key(n + s), 0.15, n, 256) if drop else None
    mod = ops.MSARowAttentionWithPairBias(wdir, f"param/block0/{name}/")
    tm, tk, tp, td = _t(msa, cuda), _t(mask, cuda), _t(pair, cuda), _t(dout, cuda)
    tt = _t(tbl, cuda) if drop else None
    out, save = mod.forward(tm, tk, tp, tt)
    din, dpair = mod.backward(tm, tk, tp, tt, save, td)
    P = af2.Params(prm, f"param/block0/{name}/")
    x = torch.tensor(msa, dtype=D, requires_grad=True)
    z = torch.tensor(pair, dtype=D, requires_grad=True)
    ref = af2.msa_row_attention(x, torch.as_tensor(mask, dtype=D), z, P)
    if drop:
        ref = ref * torch.as_tensor(tbl, dtype=D)[None]
    gx, gz = torch.autograd.grad(ref, (x, z), torch.as_tensor(dout, dtype=D))
    print(assert_act((out - tm).cpu().double(), ref.detach(), what="delta"),
          assert_grad((din - td).cpu().double(), gx, what="dmsa"),
          assert_grad(dpair.cpu().double(), gz, what="dpair"))


@pytest.mark.parametrize("s,n", [(1, 32), (2, 32), (5, 64)])
def test_msa_column_attention(cuda, s, n):
    print(f"msacol s={s} n={n}", flush=True)
    name = "msa_column_attention"
    rng = np.random.default_rng(s * 3 + n)
    prm = bparams.init_block_params(0, rng, modules=[name], gates="random", ln="random")
    wdir = weights_dir(prm, f"col_{s}_{n}")
    msa = rng.standard_normal((s, n, 256)).astype(np.float32)
    mask = (rng.random((s, n)) > 0.2).astype(np.float32)
    mask[:, 3] = 0.0  # a fully masked column
    dout = rng.standard_normal((s, n, 256)).astype(np.float32)
    mod = ops.MSAColumnAttention(wdir, f"param/block0/{name}/")
    tm, tk, td = _t(msa, cuda), _t(mask, cuda), _t(dout, cuda)
    out, save = mod.forward(tm, tk)
    din = mod.backward(tm, tk, None, save, td)
    P = af2.Params(prm, f"param/block0/{name}/")
    x = torch.tensor(msa, dtype=D, requires_grad=True)
    ref = af2.msa_column_attention(x, torch.as_tensor(mask, dtype=D), P)
    (g,) = torch.autograd.grad(ref, x, torch.as_tensor(dout, dtype=D))
    print(assert_act((out - tm).cpu().double(), ref.detach(), what="delta"),
          assert_grad((din - td).cpu().double(), g, what="dmsa"))


@pytest.mark.parametrize("s,n,mfrac", [(1, 32, 0.0), (5, 64, 0.2), (40, 32, 0.3)])
def test_msa_column_global_attention(cuda, s, n, mfrac):
    """The extra-MSA column module (modules.py:619-672), f32 end to end,
    with some fully masked columns."""
    print(f"msa global s={s} n={n} mask={mfrac}", flush=True)
    rng = np.random.default_rng(s * 31 + n)
    name = "msa_column_global_attention"
    prm = {f"param/block0/{name}/{k}": v for k, v in
           bparams.init_module(bparams.global_attention_shapes(), rng, gates="random",
                               ln="random").items()}
    wdir = weights_dir(prm, f"glob_{s}_{n}")
    msa = rng.standard_normal((s, n, 64)).astype(np.float32)
    mask = (rng.random((s, n)) > mfrac).astype(np.float32)
    mask[:, 3] = 0.0  # a fully masked column attends uniformly
    dout = rng.standard_normal((s, n, 64)).astype(np.float32)
    mod = ops.MSAColumnGlobalAttention(wdir, f"param/block0/{name}/")
    tm, tk, td = _t(msa, cuda), _t(mask, cuda), _t(dout, cuda)
    out, save = mod.forward(tm, tk)
    din = mod.backward(tm, tk, None, save, td)
    P = af2.Params(prm, f"param/block0/{name}/")
    x = torch.tensor(msa, dtype=D, requires_grad=True)
    ref = af2.msa_column_global_attention(x, torch.as_tensor(mask, dtype=D), P)
    (g,) = torch.autograd.grad(ref, x, torch.as_tensor(dout, dtype=D))
    ma = assert_act((out - tm).cpu().double(), ref.detach(), tol=1e-4, what="delta")
    mg = assert_grad((din - td).cpu().double(), g, cos=0.99999, what="dmsa")
    print(ma, mg)
