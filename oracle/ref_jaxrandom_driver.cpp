// C entry points over the reference's own JAX PRNG pin
// (/root/reference/native/jaxrandom.cuh, compiled from where it lies by
// oracle/build_ref.sh into oracle/_ref/).  Test infrastructure only: used to
// check oracle/jax_prng.py; never linked into the product.
#include <stddef.h>
#include <cstdint>
#include <vector>
#include "jaxrandom.cuh"

extern "C" {

void ref_threefry2x32(uint32_t k0, uint32_t k1, uint32_t* x0, uint32_t* x1) {
  jrandom::threefry2x32(k0, k1, *x0, *x1);
}

void ref_split(uint32_t k0, uint32_t k1, int n, uint32_t* out) {
  jrandom::Key k;
  k.a = k0;
  k.b = k1;
  std::vector<jrandom::Key> ks = jrandom::split(k, n);
  for (int i = 0; i < n; ++i) {
    out[2 * i] = ks[i].a;
    out[2 * i + 1] = ks[i].b;
  }
}

void ref_fold_in(uint32_t k0, uint32_t k1, uint64_t d, uint32_t* out) {
  jrandom::Key k;
  k.a = k0;
  k.b = k1;
  jrandom::Key r = jrandom::foldIn(k, d);
  out[0] = r.a;
  out[1] = r.b;
}

uint32_t ref_random_bits_scalar(uint32_t k0, uint32_t k1) {
  jrandom::Key k;
  k.a = k0;
  k.b = k1;
  return jrandom::randomBits(k);
}

void ref_prng_key(uint64_t seed, uint32_t* out) {
  jrandom::Key k = jrandom::prngKey(seed);
  out[0] = k.a;
  out[1] = k.b;
}

}  // extern "C"
