"""The per-block-recompute stack runner (tests/trunk_ref.py) equals autograd
through the oracle's whole stack (CPU, small widths, dropout on)."""
import numpy as np
import torch

from bindcraft2_amd import params as bparams
from oracle import af2, jax_prng as J
from tests import trunk_ref as R

DT = torch.float64
KW = dict(c_z=16, c_m=8, tri_heads=2, trimul_hidden=8, opm_c=4, row_heads=2, col_heads=2)


def test_recompute_stack_equals_whole_stack_autograd():
    rng = np.random.default_rng(31)
    depth, n, s = 3, 6, 2
    prm = {}
    for b in range(depth):
        prm.update(bparams.init_block_params(b, rng, gates="random", ln="random", **KW))
    pair = torch.as_tensor(rng.standard_normal((n, n, 16)), dtype=DT)
    msa = torch.as_tensor(rng.standard_normal((s, n, 8)), dtype=DT)
    pm = torch.as_tensor((rng.random((n, n)) > 0.2).astype(np.float64))
    mm = torch.as_tensor((rng.random((s, n)) > 0.2).astype(np.float64))
    ct_p = torch.as_tensor(rng.standard_normal((n, n, 16)), dtype=DT)
    ct_m = torch.as_tensor(rng.standard_normal((s, n, 8)), dtype=DT)
    key = J.prng_key(9)

    x, y = pair.clone().requires_grad_(True), msa.clone().requires_grad_(True)
    rm, rp = af2.evoformer_stack(y, x, mm, pm, prm, depth, key, True)
    gx, gy = torch.autograd.grad((rp, rm), (x, y), (ct_p, ct_m))

    blk = R.evoformer_block(prm, pm, mm, True, DT)
    keys = af2.stack_block_keys(key, depth)
    xs = R.stack_forward(blk, (msa, pair), keys)
    om, op = xs[-1]
    dm, dp = R.stack_backward(blk, xs, keys, (ct_m, ct_p))
    torch.testing.assert_close(op, rp.detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(om, rm.detach(), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(dp, gx, rtol=1e-10, atol=1e-10)
    torch.testing.assert_close(dm, gy, rtol=1e-10, atol=1e-10)
