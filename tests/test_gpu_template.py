"""GPU parity of the template pair stack (C=64, D=16 flash attention) with
JAX-exact dropout against the fp64 oracle (modules_multimer.py:1008-1077)."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import assert_act, assert_grad, random_mask, weights_dir

pytestmark = pytest.mark.gpu
D = torch.float64


@pytest.mark.parametrize("depth,n,dropout", [(1, 32, False), (2, 64, True)])
def test_template_stack_parity(cuda, depth, n, dropout):
    print(f"template depth={depth} n={n} dropout={dropout}", flush=True)
    rng = np.random.default_rng(depth * 10 + n)
    prm = {}
    for b in range(depth):
        prm.update(bparams.init_template_block_params(b, rng, gates="random", ln="random"))
    wdir = weights_dir(prm, f"tpl_{depth}_{n}")
    pair = rng.standard_normal((n, n, 64)).astype(np.float32)
    mask, _ = random_mask(n, 0.1, rng)
    ct = rng.standard_normal((n, n, 64)).astype(np.float32)
    key = J.prng_key(31 + n)
    T = lambda a: torch.as_tensor(a, device=cuda)
    st = ops.TemplatePairStack(wdir, depth)
    seed = ops.seed_tensor(key, True, cuda)
    out, save = st.forward(T(pair), T(mask), seed, dropout=dropout)
    dp = st.backward(T(ct), T(mask), save, seed, dropout=dropout)
    torch.cuda.synchronize()
    x = torch.tensor(pair, dtype=D, requires_grad=True)
    ref = af2.template_stack(x, torch.as_tensor(mask, dtype=D), prm, depth, key if dropout else None,
                             dropout)
    (g,) = torch.autograd.grad(ref, x, torch.as_tensor(ct, dtype=D))
    print(" out", assert_act(out.cpu().double() - x.detach(), ref.detach() - x.detach(), what="delta"))
    print(" dpair", assert_grad(dp.cpu().double(), g, what="dpair"))
