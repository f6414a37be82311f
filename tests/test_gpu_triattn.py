"""GPU parity of triangle attention (starting/ending node), forward and
backward, through the C ABI against the fp64 oracle (modules.py:675-734 +
dropout_wrapper) on the same seeded inputs, weights and JAX dropout keys."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops, params as bparams
from oracle import af2, jax_prng as J
from tests.helpers import assert_act, assert_grad, metrics, random_mask, weights_dir

pytestmark = pytest.mark.gpu

NAMES = {False: "triangle_attention_starting_node", True: "triangle_attention_ending_node"}


def _case(n, per_column, seed, drop, mask_frac):
    rng = np.random.default_rng(seed)
    prm = bparams.init_block_params(0, rng, modules=[NAMES[per_column]], gates="random",
                                    ln="random")
    wdir = weights_dir(prm, f"ta{int(per_column)}_{n}_{seed}")
    pair = rng.standard_normal((n, n, 128)).astype(np.float32)
    mask, _ = random_mask(n, mask_frac, rng)
    dout = rng.standard_normal((n, n, 128)).astype(np.float32)
    key = J.prng_key(seed + 100)
    tbl = af2.dropout_table(key, 0.25, n, 128) if drop else None
    return prm, wdir, pair, mask, dout, tbl


def _oracle(prm, per_column, pair, mask, tbl, dout):
    # fp64, or fp32 from L=512 (the [L,H,L,L] logits then take 4 GB per copy);
    # past 768 the VJP row chunk by row chunk (17 GB a copy at L=1024)
    dt = torch.float64 if pair.shape[0] < 512 else torch.float32
    P = af2.Params(prm, f"param/block0/{NAMES[per_column]}/", dt)
    if pair.shape[0] > 768:
        delta, g = af2.triangle_attention_vjp(
            torch.as_tensor(pair, dtype=dt), torch.as_tensor(mask, dtype=dt), P, per_column,
            torch.as_tensor(dout, dtype=dt), None if tbl is None else torch.as_tensor(tbl, dtype=dt),
            rows=32)
        return delta.double(), g.double()
    x = torch.tensor(pair, dtype=dt, requires_grad=True)
    m = torch.as_tensor(mask, dtype=dt)
    delta = af2.triangle_attention(x, m, P, per_column)
    if tbl is not None:
        t = torch.as_tensor(tbl, dtype=dt)
        delta = delta * (t[None] if not per_column else t[:, None])
    (g,) = torch.autograd.grad(delta, x, torch.as_tensor(dout, dtype=dt))
    return delta.detach().double(), g.double()


@pytest.mark.parametrize("n,per_column,drop,mask_frac", [
    (32, False, False, 0.0), (32, True, False, 0.0),
    (64, False, True, 0.1), (64, True, True, 0.1),
    (96, True, True, 0.25),
    # the benchmark length, and lengths past one 256-key chunk (chunked
    # keys with an online rescale; four query groups in dK/dV)
    (224, False, True, 0.1), (224, True, True, 0.1), (288, True, True, 0.1),
    (320, False, True, 0.25),
    # the large complex of BASELINE configs[4]
    (512, False, True, 0.1), (512, True, True, 0.1),
    # past 512: 24 key blocks, eight-wave dK/dV (the long-length path)
    (768, False, True, 0.1), (768, True, True, 0.1),
    # the longest lengths the entry points take: eight query groups x one
    # key tile in dK/dV, a partial last key chunk at 800
    (800, False, True, 0.1), (800, True, True, 0.1), (1024, False, True, 0.1),
    (1024, True, True, 0.1),
])
def test_triattn_fwd_bwd_parity(cuda, n, per_column, drop, mask_frac):
    print(f"triattn n={n} per_column={per_column} drop={drop} mask={mask_frac}", flush=True)
    prm, wdir, pair, mask, dout, tbl = _case(n, per_column, 7 + n, drop, mask_frac)
    mod = ops.TriangleAttention(wdir, f"param/block0/{NAMES[per_column]}/", per_column)
    tp = torch.as_tensor(pair, device=cuda)
    tm = torch.as_tensor(mask, device=cuda)
    tt = torch.as_tensor(tbl, device=cuda) if tbl is not None else None
    out, save = mod.forward(tp, tm, tt)
    dd = torch.as_tensor(dout, device=cuda)
    din = mod.backward(tp, tm, tt, save, dd)
    torch.cuda.synchronize()
    ref_delta, ref_grad = _oracle(prm, per_column, pair, mask, tbl, dout)
    got_delta = (out - tp).cpu().double()
    got_grad = (din - dd).cpu().double()
    ma = assert_act(got_delta, ref_delta, what="delta")
    mg = assert_grad(got_grad, ref_grad, what="dpair")
    print("  fwd", ma, "\n  bwd", mg)
    assert mg["rel_l2"] < 5e-2


@pytest.mark.parametrize("n", [64, 288])
def test_triattn_fully_masked_rows(cuda, n):
    """Padding residues: rows with every key masked attend uniformly."""
    print(f"triattn fully masked rows n={n}", flush=True)
    prm, wdir, pair, _, dout, _ = _case(n, False, 3, False, 0.0)
    m = np.ones(n, np.float32)
    m[-7:] = 0.0
    mask = np.outer(m, m).astype(np.float32)
    mod = ops.TriangleAttention(wdir, "param/block0/triangle_attention_starting_node/", False)
    tp = torch.as_tensor(pair, device=cuda)
    out, save = mod.forward(tp, torch.as_tensor(mask, device=cuda))
    din = mod.backward(tp, torch.as_tensor(mask, device=cuda), None, save, torch.as_tensor(dout, device=cuda))
    ref_delta, ref_grad = _oracle(prm, False, pair, mask, None, dout)
    assert_act((out - tp).cpu().double(), ref_delta, what="delta")
    assert_grad((din - torch.as_tensor(dout, device=cuda)).cpu().double(), ref_grad, what="dpair")


def test_triattn_deterministic(cuda):
    n = 64
    prm, wdir, pair, mask, dout, tbl = _case(n, True, 5, True, 0.1)
    mod = ops.TriangleAttention(wdir, "param/block0/triangle_attention_ending_node/", True)
    tp = torch.as_tensor(pair, device=cuda)
    tm = torch.as_tensor(mask, device=cuda)
    tt = torch.as_tensor(tbl, device=cuda)
    dd = torch.as_tensor(dout, device=cuda)
    r = []
    for _ in range(2):
        out, save = mod.forward(tp, tm, tt)
        r.append((out.clone(), mod.backward(tp, tm, tt, save, dd).clone()))
    assert torch.equal(r[0][0], r[1][0]) and torch.equal(r[0][1], r[1][1])
