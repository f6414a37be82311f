"""GPU parity of the building-block kernels (GEMM, LayerNorm, dropout bits)
through the C ABI against the oracle / a float reference of the same op."""
import numpy as np
import pytest
import torch

from bindcraft2_amd import ops
from oracle import jax_prng as J

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("m,n,k", [(128, 128, 64), (200, 96, 32), (50176 // 49, 512, 128),
                                   (333, 640, 224), (64, 16, 1024),
                                   # few tiles and a long K: split over K, partials
                                   # added in slice order by the epilogue pass
                                   (224, 256, 1024), (96, 512, 512)])
def test_gemm_matches_fp32(cuda, m, n, k):
    print(f"gemm m={m} n={n} k={k}", flush=True)
    g = torch.Generator().manual_seed(m * 7 + n)
    a = torch.randn(m, k, generator=g).to(torch.float16)
    b = torch.randn(n, k, generator=g).to(torch.float16)
    ref = a.double() @ b.double().T
    got = ops.probe_gemm(a.to(cuda), b.to(cuda)).cpu().double()
    err = (got - ref).abs().max() / ref.abs().max()
    assert err < 1e-5, err


@pytest.mark.parametrize("c,fast", [(128, False), (128, True), (256, False), (64, True)])
def test_layernorm_matches_fp64(cuda, c, fast):
    print(f"layernorm c={c} fast={fast}", flush=True)
    g = torch.Generator().manual_seed(c)
    x = torch.randn(1000, c, generator=g) * 2 + 0.5
    gamma = torch.randn(c, generator=g)
    beta = torch.randn(c, generator=g)
    ref = torch.nn.functional.layer_norm(x.double(), (c,), gamma.double(), beta.double(), eps=1e-5)
    y, mean, rstd = ops.probe_layernorm(x.to(cuda), gamma.to(cuda), beta.to(cuda), fast)
    err = (y.cpu().double() - ref).abs().max() / ref.abs().max()
    assert err < 1e-3, err  # binary16 output rounding (2^-11 relative)
    torch.testing.assert_close(mean.cpu().double(), x.double().mean(1), rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("rate", [0.25, 0.15])
def test_dropout_bits_equal_jax_bernoulli(cuda, rate):
    print(f"bernoulli rate={rate}", flush=True)
    for seed in (0, 1, 12345):
        key = J.prng_key(seed)
        n = 224 * 128
        got = ops.bernoulli_bits(n, key, rate).cpu().numpy().astype(bool)
        ref = J.bernoulli(key, J.keep_rate(rate), (n,))
        assert np.array_equal(got, ref)
        tbl = ops.dropout_table(224, 128, key, rate).cpu().numpy()
        assert np.array_equal(tbl > 0, ref.reshape(224, 128))
        np.testing.assert_array_equal(tbl[tbl > 0], np.float32(1.0) / J.keep_rate(rate))


def test_stack_keys_equal_jax_chain(cuda):
    key = J.prng_key(2024)
    got = ops.stack_keys(key, 5).cpu().numpy().astype(np.uint64)
    ref = J.stack_module_keys(key, 5)
    for l in range(5):
        for m in range(9):
            assert (int(got[l, m, 0]), int(got[l, m, 1])) == (int(ref[l][m][0]), int(ref[l][m][1]))
