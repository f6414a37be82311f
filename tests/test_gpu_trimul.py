"""GPU parity of the fused triangle multiplication (outgoing/incoming),
forward and backward, through the C ABI against the fp64 oracle
(modules.py:1044-1088 + dropout_wrapper)."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import assert_act, assert_grad, random_mask, weights_dir

pytestmark = pytest.mark.gpu

NAMES = {True: "triangle_multiplication_outgoing", False: "triangle_multiplication_incoming"}


def _oracle(prm, outgoing, pair, mask, tbl, dout):
    dt = torch.float64 if pair.shape[0] < 512 else torch.float32
    P = af2.Params(prm, f"param/block0/{NAMES[outgoing]}/", dt)
    x = torch.tensor(pair, dtype=dt, requires_grad=True)
    delta = af2.triangle_multiplication(x, torch.as_tensor(mask, dtype=dt), P, outgoing)
    if tbl is not None:
        delta = delta * torch.as_tensor(tbl, dtype=dt)[None]
    (g,) = torch.autograd.grad(delta, x, torch.as_tensor(dout, dtype=dt))
    return delta.detach().double(), g.double()


@pytest.mark.parametrize("n,outgoing,drop,mask_frac", [
    (32, True, False, 0.0), (32, False, False, 0.0),
    (64, True, True, 0.1), (64, False, True, 0.1), (96, False, True, 0.2),
    (224, True, True, 0.1), (224, False, True, 0.1), (288, True, True, 0.1),
    # the large complex of BASELINE configs[4]
    (512, True, True, 0.1), (512, False, True, 0.1),
    (768, True, True, 0.1),
])
def test_trimul_fwd_bwd_parity(cuda, n, outgoing, drop, mask_frac):
    print(f"trimul n={n} outgoing={outgoing} drop={drop} mask={mask_frac}", flush=True)
    rng = np.random.default_rng(n + int(outgoing))
    prm = bparams.init_block_params(0, rng, modules=[NAMES[outgoing]], gates="random", ln="random")
    wdir = weights_dir(prm, f"tm{int(outgoing)}_{n}")
    pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    mask, _ = random_mask(n, mask_frac, rng)
    dout = rng.standard_normal((n, n, 128)).astype(np.float32)
    tbl = af2.dropout_table(J.prng_key(n), 0.25, n, 128) if drop else None
    mod = ops.TriangleMultiplication(wdir, f"param/block0/{NAMES[outgoing]}/", outgoing)
    tp, tm = torch.as_tensor(pair, device=cuda), torch.as_tensor(mask, device=cuda)
    tt = torch.as_tensor(tbl, device=cuda) if tbl is not None else None
    dd = torch.as_tensor(dout, device=cuda)
    out, save = mod.forward(tp, tm, tt)
    din = mod.backward(tp, tm, tt, save, dd)
    torch.cuda.synchronize()
    ref_delta, ref_grad = _oracle(prm, outgoing, pair, mask, tbl, dout)
    ma = assert_act((out - tp).cpu().double(), ref_delta, what="delta")
    mg = assert_grad((din - dd).cpu().double(), ref_grad, what="dpair")
    print("  fwd", ma, "\n  bwd", mg)
