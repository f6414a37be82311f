"""GPU parity of the template embedding (the TemplateEmbeddingFwd/Bwd
drop-in: query LayerNorm and projection added to the constant features,
template pair stack, output LayerNorm, relu, output linear) against the fp64
oracle (modules_multimer.py:704-1005), dropout on with the JAX stack key;
the gradient reaches the query only (act_const is a constant)."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import assert_act, assert_grad, random_mask, weights_dir

pytestmark = pytest.mark.gpu
D = torch.float64


# The relu acts on LN(stack output), so every element the kernels' rounding
# moves across zero flips its whole gradient term.  `hinge=False` shifts
# output_layer_norm's offset by +5 so that no element lies near the hinge
# (the composite gradient alone); `hinge=True` keeps the hinge live.  With
# binary16 operands the stack's output is ~5e-4 (relative) from the fp64
# oracle and both cases are held to the north star's cosine bar (measured:
# 0.99995+ strict, 0.99965 live).
@pytest.mark.parametrize("depth,n,dropout,hinge", [(1, 32, False, False), (2, 64, True, False),
                                                   (2, 96, True, False), (2, 64, True, True)])
def test_template_embedding_parity(cuda, depth, n, dropout, hinge):
    print(f"template embedding depth={depth} n={n} dropout={dropout} hinge={hinge}", flush=True)
    rng = np.random.default_rng(7000 + depth * 10 + n)
    prm = bparams.init_template_embedding_params(depth, rng, gates="random", ln="random")
    if not hinge:
        prm["param/output_layer_norm/offset"] = prm["param/output_layer_norm/offset"] + np.float32(5.0)
        wtag = "strict"
    else:
        wtag = "hinge"
    wdir = weights_dir(prm, f"tplembed_{depth}_{n}_{wtag}")
    query = rng.standard_normal((n, n, 128)).astype(np.float32)
    act_const = rng.standard_normal((n, n, 64)).astype(np.float32)
    mask, _ = random_mask(n, 0.1, rng)
    ct = rng.standard_normal((n, n, 128)).astype(np.float32)
    key = J.prng_key(51 + n)
    T = lambda a: torch.as_tensor(a, device=cuda)
    te = ops.TemplateEmbedding(wdir, depth)
    seed = ops.seed_tensor(key, True, cuda)
    out, save = te.forward(T(query), T(act_const), T(mask), seed, dropout=dropout)
    dq = te.backward(T(ct), T(query), T(act_const), T(mask), save, seed, dropout=dropout)
    torch.cuda.synchronize()
    x = torch.tensor(query, dtype=D, requires_grad=True)
    ref = af2.template_embedding(x, torch.as_tensor(act_const, dtype=D), torch.as_tensor(mask, dtype=D),
                                 prm, depth, key if dropout else None, dropout)
    (g,) = torch.autograd.grad(ref, x, torch.as_tensor(ct, dtype=D))
    print(" out", assert_act(out.cpu().double(), ref.detach(), what="out"))
    print(" dquery", assert_grad(dq.cpu().double(), g, what="dquery"))
