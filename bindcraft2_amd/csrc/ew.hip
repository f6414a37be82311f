// Small elementwise kernels: dropout tables from JAX keys, the JAX key chain of
// the Evoformer stack, residual/dropout glue of the backward passes, and the
// backward's cotangent scales.
#include "kernels.h"
#include "runtime.h"

#include <algorithm>
#include <mutex>

namespace bc2n {

// -------------------------------------------------------- cotangent scales
// {s, 1/s} slots and the partial maxima of ct_scale live in file-scope device
// arrays (one copy per GPU, resolved per device by hipGetSymbolAddress), so
// computing a scale allocates nothing.  Each work lane has its own partials
// (the two lanes' scales are computed on two streams at once); the slots are
// assigned per carry by the callers.
namespace {
constexpr int CT_SLOTS = 8;
constexpr int CT_PART = 512;  // partial-maximum blocks (grid of the first pass)
__device__ __align__(256) float g_ct_slots[CT_SLOTS * 2];
__device__ __align__(256) float g_ct_part[NUM_LANES * CT_PART];
__device__ __align__(256) float g_ct_fused[NUM_LANES * CT_FUSED];

struct CtPtrs {
  float* slots = nullptr;
  float* part = nullptr;
  float* fused = nullptr;
};
CtPtrs ct_ptrs() {
  static std::mutex mu;
  static CtPtrs per_dev[64];
  int dev = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) throw std::runtime_error("ct_scale: device index out of range");
  std::lock_guard<std::mutex> lk(mu);
  CtPtrs& p = per_dev[dev];
  if (!p.slots) {
    void *a = nullptr, *b = nullptr, *c = nullptr;
    hip_check(hipGetSymbolAddress(&a, HIP_SYMBOL(g_ct_slots)), "hipGetSymbolAddress(slots)");
    hip_check(hipGetSymbolAddress(&b, HIP_SYMBOL(g_ct_part)), "hipGetSymbolAddress(part)");
    hip_check(hipGetSymbolAddress(&c, HIP_SYMBOL(g_ct_fused)), "hipGetSymbolAddress(fused)");
    p.slots = static_cast<float*>(a);
    p.part = static_cast<float*>(b);
    p.fused = static_cast<float*>(c);
  }
  return p;
}
}  // namespace

// part[block] = max |x| over a grid-stride range (4 floats a load); x and n
// are 16-byte aligned / a multiple of 4 (checked on the host).
__global__ __launch_bounds__(256) void amax_part_kernel(const float* __restrict__ x, long n4,
                                                        float* __restrict__ part) {
  __shared__ float red[4];
  float m = 0.f;
  const float4* x4 = reinterpret_cast<const float4*>(x);
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n4; i += (long)gridDim.x * 256) {
    const float4 v = x4[i];
    m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
  }
  m = group_max<64>(m);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0) part[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// sc = {s, 1/s}: s = 2^(4 - e) for max|x| in (2^(e-1), 2^e], so s*max|x| is
// in (8, 16]; s = 1 when x is all zero or its maximum is not finite.
// One workgroup of 256; four independent loads a thread in flight (up to
// CT_FUSED partials).
__global__ __launch_bounds__(256) void amax_final_kernel(const float* __restrict__ part, int np,
                                                         float* __restrict__ sc) {
  float m4[4] = {0.f, 0.f, 0.f, 0.f};
  for (int i = threadIdx.x; i < np; i += 1024) {
#pragma unroll
    for (int u = 0; u < 4; ++u)
      if (i + 256 * u < np) m4[u] = fmaxf(m4[u], part[i + 256 * u]);
  }
  float m = group_max<64>(fmaxf(fmaxf(m4[0], m4[1]), fmaxf(m4[2], m4[3])));
  __shared__ float red[4];
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  if (threadIdx.x == 0) {
    float s = 1.f;
    if (m > 0.f && m <= 3.0e38f) {
      int e = 0;
      (void)frexpf(m, &e);
      s = ldexpf(1.f, max(-100, min(100, 4 - e)));
    }
    sc[0] = s;
    sc[1] = 1.f / s;
  }
}

float* ct_scale_slot(int k) {
  if (k < 0 || k >= CT_SLOTS) throw std::runtime_error("ct_scale: slot out of range");
  return ct_ptrs().slots + 2 * k;
}

void ct_scale(hipStream_t st, const float* x, long n, float* sc) {
  if (x == nullptr || n <= 0 || n % 4 != 0 || ((uintptr_t)x & 15))
    throw std::runtime_error("ct_scale: x must be 16-byte aligned with n a positive multiple of 4");
  const CtPtrs p = ct_ptrs();
  const long n4 = n / 4;
  const int blocks = (int)std::min<long>(CT_PART, (n4 + 255) / 256);
  float* part = p.part + (size_t)lane() * CT_PART;
  hipLaunchKernelGGL(amax_part_kernel, dim3(blocks), dim3(256), 0, st, x, n4, part);
  hipLaunchKernelGGL(amax_final_kernel, dim3(1), dim3(256), 0, st, part, blocks, sc);
}

float* ct_fused_parts() { return ct_ptrs().fused + (size_t)lane() * CT_FUSED; }

void ct_scale_parts(hipStream_t st, const float* part, long np, float* sc) {
  if (!part || !sc || np <= 0 || np > CT_FUSED)
    throw std::runtime_error("ct_scale_parts: 1 to CT_FUSED partial maxima");
  hipLaunchKernelGGL(amax_final_kernel, dim3(1), dim3(256), 0, st, part, (int)np, sc);
}

// ----------------------------------------------------------------- zero fill
// A kernel, not hipMemsetAsync: memset nodes in a captured HIP graph have
// given wrong results on replays after the first.
__global__ void zero_f32_kernel(float* __restrict__ p, long n) {
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (long)gridDim.x * blockDim.x)
    p[i] = 0.f;
}

void zero_f32(hipStream_t st, float* p, long n) {
  if (n <= 0) return;
  const long blocks = std::min<long>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(zero_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, st, p, n);
}

// -------------------------------------------------------------- dropout
// tbl[b*C+c] = keep ? 1/keep_rate : 0 where keep = uniform(key, (B,C)) < keep_rate
// and the key (k0,k1) / enable flag are read on the device.
__global__ void dropout_table_kernel(float* __restrict__ tbl, int B, int C,
                                     const uint32_t* __restrict__ key,
                                     const uint32_t* __restrict__ enabled,
                                     float keep_rate) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)B * C) return;
  const bool on = enabled == nullptr || enabled[0] != 0u;
  if (!on) { tbl[i] = 1.f; return; }
  const float u = jax_uniform01(key[0], key[1], (uint64_t)i);
  tbl[i] = (u < keep_rate) ? 1.f / keep_rate : 0.f;
}

void dropout_table_dev(hipStream_t st, float* tbl, int B, int C,
                       const uint32_t* key, const uint32_t* enabled, float keep_rate) {
  const long n = (long)B * C;
  hipLaunchKernelGGL(dropout_table_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     tbl, B, C, key, enabled, keep_rate);
}

// Every dropout table of a stack in one launch: per block, the MSA row
// attention's [N][Cm] table (when msa_row) and the four pair modules' [N][Cz]
// tables, at the same offsets and from the same keys as one
// dropout_table_dev call each.
__global__ void stack_dropout_tables_kernel(float* __restrict__ tbl, long per_block, int N, int Cm,
                                            int Cz, int depth, int nk, int msa_row, int row_key,
                                            int4 pair_keys, const uint32_t* __restrict__ keys,
                                            const uint32_t* __restrict__ enabled) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const long row_n = msa_row ? (long)N * Cm : 0, pn = (long)N * Cz;
  const long per = row_n + 4 * pn;
  if (i >= per * depth) return;
  const int b = (int)(i / per);
  long r = i % per, off, e;
  int kidx;
  float keep;
  if (r < row_n) {
    kidx = row_key;
    e = off = r;
    keep = 1.0f - 0.15f;
  } else {
    r -= row_n;
    const int k = (int)(r / pn);
    e = r % pn;
    kidx = k == 0 ? pair_keys.x : k == 1 ? pair_keys.y : k == 2 ? pair_keys.z : pair_keys.w;
    off = (long)N * Cm + k * pn + e;
    keep = 1.0f - 0.25f;
  }
  float* dst = tbl + b * per_block + off;
  const bool on = enabled == nullptr || enabled[0] != 0u;
  if (!on) { *dst = 1.f; return; }
  const uint32_t* key = keys + ((long)b * nk + kidx) * 2;
  const float u = jax_uniform01(key[0], key[1], (uint64_t)e);
  *dst = (u < keep) ? 1.f / keep : 0.f;
}

void stack_dropout_tables(hipStream_t st, float* tbl, long per_block, int N, int Cm, int Cz,
                          int depth, int nk, bool msa_row, int row_key, const int (&pair_keys)[4],
                          const uint32_t* keys, const uint32_t* enabled) {
  const long n = ((msa_row ? (long)N * Cm : 0) + 4L * N * Cz) * depth;
  hipLaunchKernelGGL(stack_dropout_tables_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     st, tbl, per_block, N, Cm, Cz, depth, nk, msa_row ? 1 : 0, row_key,
                     make_int4(pair_keys[0], pair_keys[1], pair_keys[2], pair_keys[3]), keys,
                     enabled);
}

__global__ void dropout_table_host_key_kernel(float* __restrict__ tbl, int B, int C,
                                              uint32_t k0, uint32_t k1, float keep_rate) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (long)B * C) return;
  const float u = jax_uniform01(k0, k1, (uint64_t)i);
  tbl[i] = (u < keep_rate) ? 1.f / keep_rate : 0.f;
}

void dropout_table(hipStream_t st, float* tbl, int B, int C, uint32_t k0,
                   uint32_t k1, float keep_rate) {
  const long n = (long)B * C;
  hipLaunchKernelGGL(dropout_table_host_key_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256),
                     0, st, tbl, B, C, k0, k1, keep_rate);
}

// Raw keep bits (1 keep, 0 drop) of jax.random.bernoulli(key, keep_rate, (n,)).
__global__ void bernoulli_bits_kernel(uint8_t* __restrict__ out, long n, uint32_t k0,
                                      uint32_t k1, float keep_rate) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  out[i] = jax_uniform01(k0, k1, (uint64_t)i) < keep_rate ? 1 : 0;
}

void bernoulli_bits(hipStream_t st, uint8_t* out, long n, uint32_t k0, uint32_t k1,
                    float keep_rate) {
  hipLaunchKernelGGL(bernoulli_bits_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                     out, n, k0, k1, keep_rate);
}

// -------------------------------------------------------------- key chain
// A layer_stack's per-module keys: for each layer, (carry, sub) =
// split(carry); the block splits `sub` into n_split and hands keys
// 1..n_used to its modules in order -- (10, 9) for the Evoformer
// (modules_multimer.py:622-641, modules.py:1308-1309), (20, 5) for the
// template pair stack (modules_multimer.py:957-966, :1036-1037).
// out[(layer*n_used + module)*2 + {0,1}].
// jax.random.split (partitionable): key i = threefry(key, counter (0, i)).
__device__ __host__ inline void split_key(uint32_t k0, uint32_t k1, int i,
                                          uint32_t* o0, uint32_t* o1) {
  uint32_t x0 = 0u, x1 = (uint32_t)i;
  threefry2x32(k0, k1, x0, x1);
  *o0 = x0;
  *o1 = x1;
}

__global__ void stack_keys_kernel(const uint32_t* __restrict__ seed, int depth, int n_used,
                                  uint32_t* __restrict__ out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  uint32_t c0 = seed[0], c1 = seed[1];
  for (int l = 0; l < depth; ++l) {
    uint32_t s0, s1, n0, n1;
    split_key(c0, c1, 1, &s0, &s1);
    split_key(c0, c1, 0, &n0, &n1);
    for (int m = 0; m < n_used; ++m) {
      uint32_t a, b;
      split_key(s0, s1, m + 1, &a, &b);
      out[(l * n_used + m) * 2 + 0] = a;
      out[(l * n_used + m) * 2 + 1] = b;
    }
    c0 = n0;
    c1 = n1;
  }
}

// jax.random.PRNGKey(bits) = (0, bits) for the reference's 2-word seed
// operand [bits, enabled] (modules_multimer.py:660-667).
__global__ void key_from_bits_kernel(const uint32_t* __restrict__ seed, uint32_t* __restrict__ out) {
  if (threadIdx.x == 0) {
    out[0] = 0u;
    out[1] = seed[0];
  }
}

void key_from_bits(hipStream_t st, const uint32_t* seed, uint32_t* out) {
  hipLaunchKernelGGL(key_from_bits_kernel, dim3(1), dim3(64), 0, st, seed, out);
}

void stack_keys(hipStream_t st, const uint32_t* seed, int depth, uint32_t* out, int n_used) {
  hipLaunchKernelGGL(stack_keys_kernel, dim3(1), dim3(64), 0, st, seed, depth, n_used, out);
}

}  // namespace bc2n
