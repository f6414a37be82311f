"""CPU restatement of the parts of jax.random that AF2's dropout draws from.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py as the checker.  The product never routes
through this module.

Semantics restated (JAX with ``jax_threefry_partitionable=True``, the default
of the JAX the reference pins, pyproject.toml:6 ``jax>=0.11``):

* threefry2x32-20 (Salmon et al., SC'11; Random123), key schedule with the
  0x1BD11BDA parity word, rotations (13,15,26,6 | 17,29,16,24), key injection
  after every 4 rounds -- same as the reference's own pin,
  native/jaxrandom.cuh:46-64.
* split(key, n): key i = threefry(key, counter (0, i))      (jaxrandom.cuh:86-97)
* fold_in(key, d): threefry(key, (hi32(d), lo32(d)))         (jaxrandom.cuh:101-110)
* random_bits(key, 32, shape): element i (row-major) is threefry(key,
  (hi32(i), lo32(i))) with the two words XORed            (jaxrandom.cuh:71-74, 114-118)
* uniform(key, shape, f32) = bitcast((bits >> 9) | 0x3F800000) - 1
* bernoulli(key, p, shape) = uniform(key, shape) < p
  (used by apply_dropout, bindcraft/af/alphafold/model/modules.py:37-44).

Pinned by tests/test_oracle_prng.py against the Random123/JAX threefry
known-answer vectors and against oracle/_ref (a build of the reference's
jaxrandom.cuh).  uniform/bernoulli float construction is pinned by its
closed form (exact float, monotone in the bits, mean of the draws) only:
parity unpinned against JAX itself (jax is absent here).
"""
import numpy as np

_ROT = ((13, 15, 26, 6), (17, 29, 16, 24))
_M32 = np.uint64(0xFFFFFFFF)


def _rotl(x, d):
    return ((x << np.uint32(d)) | (x >> np.uint32(32 - d))).astype(np.uint32)


def threefry2x32(k0, k1, x0, x1):
    """Vectorised threefry2x32-20 over uint32 arrays x0, x1 (broadcast)."""
    with np.errstate(over="ignore"):
        k0 = np.uint32(k0)
        k1 = np.uint32(k1)
        k2 = np.uint32(k0 ^ k1 ^ np.uint32(0x1BD11BDA))
        ks = (k0, k1, k2)
        x0 = np.asarray(x0, np.uint32) + k0
        x1 = np.asarray(x1, np.uint32) + k1
        for g in range(5):
            for r in _ROT[g % 2]:
                x0 = (x0 + x1).astype(np.uint32)
                x1 = _rotl(x1, r)
                x1 = x1 ^ x0
            x0 = (x0 + ks[(g + 1) % 3]).astype(np.uint32)
            x1 = (x1 + ks[(g + 2) % 3] + np.uint32(g + 1)).astype(np.uint32)
    return x0.astype(np.uint32), x1.astype(np.uint32)


def prng_key(seed):
    """jax.random.PRNGKey(seed) for a non-negative int seed (threefry_seed)."""
    seed = int(seed)
    return (np.uint32((seed >> 32) & 0xFFFFFFFF), np.uint32(seed & 0xFFFFFFFF))


def split(key, n=2):
    """jax.random.split(key, n) -> list of n (k0, k1) pairs."""
    i = np.arange(n, dtype=np.uint64)
    x0, x1 = threefry2x32(key[0], key[1], (i >> np.uint64(32)).astype(np.uint32),
                          (i & _M32).astype(np.uint32))
    return [(np.uint32(a), np.uint32(b)) for a, b in zip(x0, x1)]


def fold_in(key, data):
    d = prng_key(data)
    x0, x1 = threefry2x32(key[0], key[1], d[0], d[1])
    return (np.uint32(x0), np.uint32(x1))


def random_bits(key, shape):
    """jax.random.bits(key, shape, uint32)."""
    n = int(np.prod(shape, dtype=np.int64)) if len(shape) else 1
    i = np.arange(n, dtype=np.uint64)
    x0, x1 = threefry2x32(key[0], key[1], (i >> np.uint64(32)).astype(np.uint32),
                          (i & _M32).astype(np.uint32))
    return (x0 ^ x1).reshape(shape)


def uniform(key, shape):
    """jax.random.uniform(key, shape, float32) on [0, 1)."""
    bits = random_bits(key, shape)
    fb = (bits >> np.uint32(9)) | np.uint32(0x3F800000)
    return fb.view(np.float32) - np.float32(1.0)


def bernoulli(key, p, shape):
    """jax.random.bernoulli(key, p, shape) with p a float32 scalar."""
    return uniform(key, shape) < np.float32(p)


def keep_rate(rate):
    """float32(1) - float32(rate): the keep probability apply_dropout uses."""
    return np.float32(1.0) - np.float32(rate)


def stack_module_keys(stack_key, depth, n_modules=9):
    """Per-module keys of an Evoformer stack (modules_multimer.py:622-641):
    per layer (carry, sub) = split(carry); the block splits sub into 10 and
    hands keys[1..9] to its modules (modules.py:1308-1309)."""
    out = []
    carry = stack_key
    for _ in range(depth):
        carry, sub = split(carry, 2)
        ks = split(sub, 10)
        out.append(ks[1:1 + n_modules])
    return out
