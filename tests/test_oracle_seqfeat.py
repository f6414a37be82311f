"""Pins of the oracle's design-sequence features (oracle/af2.py
sequence_features, design_inputs) by what the mathematics fixes: the
softmax limit against scipy, the linear limit, the pass-through of
undesigned residues, the straight-through one-hot's forward value and its
gradient against the closed-form softmax Jacobian, finite differences of
the smooth case, and the msa_feat channel layout."""
import numpy as np
import pytest
import scipy.special
import torch

from oracle import af2

D = torch.float64


def _logits(n, rng, omitted=()):
    x = rng.standard_normal((n, 20))
    for i, a in omitted:
        x[i, a] = af2.OMITTED_AMINO_ACID_LOGIT
    return x


def test_softmax_limit_and_profile():
    rng = np.random.default_rng(1)
    x = _logits(9, rng)
    bias = rng.standard_normal(20)
    k = 2.0 / 0.7
    f, p = af2.sequence_features(torch.tensor(x, dtype=D), np.ones(9, np.uint8), 1.0, 0.0, 0.7, 2.0,
                                 bias=torch.tensor(bias, dtype=D))
    ref = scipy.special.softmax(x * k + bias, axis=-1)
    np.testing.assert_allclose(f.numpy(), ref, rtol=1e-12, atol=1e-14)
    np.testing.assert_array_equal(p.numpy(), np.eye(20)[ref.argmax(-1)])


def test_linear_limit_zeroes_omitted_and_passthrough():
    rng = np.random.default_rng(2)
    x = _logits(7, rng, omitted=[(0, 3), (4, 11)])
    flags = np.array([1, 1, 0, 1, 1, 0, 1], np.uint8)
    f, p = af2.sequence_features(torch.tensor(x, dtype=D), flags, 0.0, 0.0, 1.0, 1.0)
    want = np.where(x <= -5000.0, 0.0, x)
    want[flags == 0] = x[flags == 0]
    np.testing.assert_array_equal(f.numpy(), want)
    np.testing.assert_array_equal(p.numpy()[flags == 0], x[flags == 0])


def test_straight_through_value_and_gradient():
    rng = np.random.default_rng(3)
    x = _logits(5, rng)
    g = rng.standard_normal((5, 20))
    t = torch.tensor(x, dtype=D, requires_grad=True)
    f, _ = af2.sequence_features(t, np.ones(5, np.uint8), 0.4, 1.0, 1.3, 0.9)
    p = scipy.special.softmax(x * 0.9 / 1.3, axis=-1)
    # forward: the hard one-hot (up to the rounding of (1 - p) + p)
    np.testing.assert_allclose(f.detach().numpy(), np.eye(20)[p.argmax(-1)], atol=1e-15)
    # backward: identity on p, so the softmax Jacobian k p (g - <p, g>)
    (grad,) = torch.autograd.grad((f * torch.tensor(g, dtype=D)).sum(), t)
    k = 0.9 / 1.3
    want = k * p * (g - (p * g).sum(-1, keepdims=True))
    np.testing.assert_allclose(grad.numpy(), want, rtol=1e-12, atol=1e-14)


def test_smooth_case_finite_differences():
    rng = np.random.default_rng(4)
    x = torch.tensor(_logits(4, rng), dtype=D, requires_grad=True)
    bias = torch.tensor(rng.standard_normal(20), dtype=D)
    flags = np.array([1, 0, 1, 1], np.uint8)
    fn = lambda t: sum(af2.sequence_features(t, flags, 0.6, 0.0, 0.8, 1.7, bias=bias)[:1])
    assert torch.autograd.gradcheck(fn, (x,), eps=1e-6, atol=1e-8)


def test_design_inputs_layout():
    rng = np.random.default_rng(5)
    feat = torch.tensor(rng.standard_normal((6, 20)), dtype=D)
    prof = torch.tensor(rng.standard_normal((6, 20)), dtype=D)
    tf, mf, aat = af2.design_inputs(feat, prof)
    assert tf.shape == (6, 21) and mf.shape == (1, 6, 49)
    np.testing.assert_array_equal(tf[:, :20].numpy(), feat.numpy())
    assert (tf[:, 20] == 0).all()
    want = np.zeros((6, 49))
    want[:, 0:20], want[:, 25:45] = feat.numpy(), prof.numpy()
    np.testing.assert_array_equal(mf[0].numpy(), want)
    np.testing.assert_array_equal(aat, feat.numpy().argmax(-1))
