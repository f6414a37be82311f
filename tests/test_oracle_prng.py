"""Pins oracle/jax_prng.py (the restatement of jax.random used for dropout)."""
import ctypes
import os

import numpy as np
import pytest

from oracle import jax_prng as J

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libjaxrandom_ref.so")

# Threefry-2x32-20 known-answer vectors (Random123 kat_vectors; the same three
# JAX's random_test.py testThreefry2x32 checks): (key, counter) -> output.
KAT = [
    ((0x00000000, 0x00000000), (0x00000000, 0x00000000), (0x6B200159, 0x99BA4EFE)),
    ((0xFFFFFFFF, 0xFFFFFFFF), (0xFFFFFFFF, 0xFFFFFFFF), (0x1CB996FC, 0xBB002BE7)),
    ((0x13198A2E, 0x03707344), (0x243F6A88, 0x85A308D3), (0xC4923A9C, 0x483DF7A0)),
]


@pytest.mark.parametrize("key,ctr,out", KAT)
def test_threefry_kat(key, ctr, out):
    x0, x1 = J.threefry2x32(key[0], key[1], np.uint32(ctr[0]), np.uint32(ctr[1]))
    assert (int(x0), int(x1)) == out


def _ref():
    if not os.path.exists(REF_LIB):
        pytest.skip("oracle/_ref not built (needs /root/reference; built by build())")
    L = ctypes.CDLL(REF_LIB)
    u32 = ctypes.c_uint32
    L.ref_threefry2x32.argtypes = [u32, u32, ctypes.POINTER(u32), ctypes.POINTER(u32)]
    L.ref_split.argtypes = [u32, u32, ctypes.c_int, ctypes.POINTER(u32)]
    L.ref_fold_in.argtypes = [u32, u32, ctypes.c_uint64, ctypes.POINTER(u32)]
    L.ref_random_bits_scalar.argtypes = [u32, u32]
    L.ref_random_bits_scalar.restype = u32
    L.ref_prng_key.argtypes = [ctypes.c_uint64, ctypes.POINTER(u32)]
    return L


def test_threefry_matches_reference_build():
    L = _ref()
    rng = np.random.default_rng(0)
    for _ in range(200):
        k0, k1, c0, c1 = (int(v) for v in rng.integers(0, 2**32, 4, dtype=np.uint64))
        a, b = ctypes.c_uint32(c0), ctypes.c_uint32(c1)
        L.ref_threefry2x32(k0, k1, ctypes.byref(a), ctypes.byref(b))
        x0, x1 = J.threefry2x32(k0, k1, np.uint32(c0), np.uint32(c1))
        assert (int(x0), int(x1)) == (a.value, b.value)


def test_split_fold_in_bits_match_reference_build():
    L = _ref()
    for seed in (0, 1, 42, 2**33 + 5):
        buf = (ctypes.c_uint32 * 2)()
        L.ref_prng_key(seed, buf)
        key = J.prng_key(seed)
        assert (int(key[0]), int(key[1])) == (buf[0], buf[1])
        for n in (2, 3, 10):
            out = (ctypes.c_uint32 * (2 * n))()
            L.ref_split(int(key[0]), int(key[1]), n, out)
            ks = J.split(key, n)
            assert [(int(a), int(b)) for a, b in ks] == [(out[2 * i], out[2 * i + 1]) for i in range(n)]
        fo = (ctypes.c_uint32 * 2)()
        L.ref_fold_in(int(key[0]), int(key[1]), 7, fo)
        f = J.fold_in(key, 7)
        assert (int(f[0]), int(f[1])) == (fo[0], fo[1])
        # element 0 of random_bits is the scalar draw
        assert int(J.random_bits(key, (4,))[0]) == L.ref_random_bits_scalar(int(key[0]), int(key[1]))


def test_uniform_closed_form():
    key = J.prng_key(3)
    bits = J.random_bits(key, (1000,))
    u = J.uniform(key, (1000,))
    # exact: u = (bits >> 9) * 2^-23, in [0, 1)
    np.testing.assert_array_equal(u.astype(np.float64), (bits >> 9).astype(np.float64) * 2.0**-23)
    assert u.min() >= 0.0 and u.max() < 1.0


def test_bernoulli_rate():
    key = J.prng_key(11)
    keep = J.bernoulli(key, J.keep_rate(0.25), (200000,))
    assert abs(keep.mean() - 0.75) < 0.005
    assert J.keep_rate(0.25) == np.float32(0.75)
    # 1 - float32(0.15) rounds (tie to even) to 0.85000002384...
    assert J.keep_rate(0.15) == np.float32(14260634 * 2.0**-24)


def test_random_bits_partitionable_counters():
    """Element i of a (B, C) draw is enciphered from the counter (0, i)."""
    key = (np.uint32(0x1234), np.uint32(0xABCD))
    b = J.random_bits(key, (3, 5))
    for i in range(15):
        x0, x1 = J.threefry2x32(key[0], key[1], np.uint32(0), np.uint32(i))
        assert int(b.reshape(-1)[i]) == int(x0 ^ x1)


def test_stack_keys_chain():
    key = J.prng_key(5)
    ks = J.stack_module_keys(key, 3)
    carry = key
    for layer in range(3):
        carry2, sub = J.split(carry, 2)
        sub10 = J.split(sub, 10)
        assert ks[layer] == sub10[1:]
        carry = carry2
