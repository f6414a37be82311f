// Host-side launchers of the non-template kernels (defined in *.hip files).
#pragma once
#include "common.h"
#include <stdexcept>

namespace bc2n {

// ---------------------------------------------------------------- LayerNorm
// Pair-bias layout shared by its producer (ln_fwd_f32 with H > 0) and the
// attention kernels, "score-fragment order": bias (h, q, k) of an N x N grid
// (N % 32 == 0) sits in the 2 KB block of (head h, 16-query tile q/16,
// 32-key block k/32), at lane ((k%16)/4)*16 + q%16, element ((k%32)/16)*4 +
// k%4 -- the 8 floats one lane of a score MFMA's accumulator takes for the
// block, so a wave reads a block as two contiguous 1 KB vectors (in [h][q][k]
// order every 16-byte lane read was a separate cache line).  Stored as
// binary16 (the reference's flash kernels take an f16 bias as well): a lane
// reads its 8 values of a block as one 16-byte vector.
__host__ __device__ __forceinline__ long bias_frag_index(int h, int q, int k, int N) {
  const int lane = ((k & 15) >> 2) * 16 + (q & 15);
  const int e = ((k & 31) >> 4) * 4 + (k & 3);
  return ((((long)h * (N >> 4) + (q >> 4)) * (N >> 5) + (k >> 5)) << 9) + lane * 8 + e;
}
// The 8 values of lane `lane` for (head h, query tile qt, key block kb).
__host__ __device__ __forceinline__ const h16* bias_frag_block(const h16* bias, int h, int qt,
                                                               int kb, int N, int lane) {
  return bias + ((((long)h * (N >> 4) + qt) * (N >> 5) + kb) << 9) + lane * 8;
}

// y[m] = LN(x[src(m)]) with src(m) = m, or (q*nt+p) for m = p*nt+q when nt>0.
// When H>0, M = N*N for an N x N grid (N % 32 == 0) and the pair bias
// bias_scale * sum_c LN(x)[m][c] * wb[c*H+h] of m = q*N+k is written at
// bias_out[bias_frag_index(h, q, k, N)].
void ln_fwd_f32(hipStream_t st, const float* x, long M, int C, int nt,
                const float* gamma, const float* beta, h16* y, float* mean,
                float* rstd, bool fast, int H, const float* wb, h16* bias_out,
                float bias_scale = 1.f);
// The pair bias of ln_fwd_f32 (C = 128, no normalised output) with the
// LayerNorm's scale and offset folded into the weights: wfrag =
// ln_bias_frags(gamma, wb, H) (binary16 MFMA fragments of gamma_c wb[c][h]),
// wconst = ln_bias_const(beta, wb, H) (sum_c beta_c wb[c][h], 16 floats).
std::vector<h16> ln_bias_frags(const float* gamma, const float* wb, int H);
std::vector<float> ln_bias_const(const float* beta, const float* wb, int H);
void ln_pair_bias_f32(hipStream_t st, const float* x, long M, bool fast, float* mean, float* rstd,
                      const h16* wfrag, const float* wconst, int H, h16* bias_out, float bias_scale);
// Its backward, accumulated: dx[m] += LN'(gs * sum_h dbias[h*M+m] wb[c][h])
// (gs = *gmul, 1 if null), afrag = ln_bias_bwd_frags(gamma, wb, H) (f32),
// M % 64 == 0.  With amax_part (room for amax_cap floats) the partial maxima
// of |dx| for ct_scale_parts, one a 64 rows; returns their count (0: none
// written, the grid exceeds amax_cap).
std::vector<float> ln_bias_bwd_frags(const float* gamma, const float* wb, int H);
long ln_pair_bias_bwd_f32(hipStream_t st, const float* x, long M, const float* mean,
                          const float* rstd, const float* afrag, int H, const float* dbias,
                          float* dx, const float* gmul, float* amax_part = nullptr,
                          long amax_cap = 0);
// dx[src(m)] (+)= LN-backward(gs * (dy[m] + sum_h dbias[h*M+m] * wb[c*H+h])).
// acc: dx = res + LN'(...) with res = dres, or dx itself when dres is null.
// gs = *gmul (device scalar: a module's inverse cotangent scale), 1 if null.
void ln_bwd_f32(hipStream_t st, const float* dy, const float* x, long M, int C,
                int nt, const float* gamma, const float* mean, const float* rstd,
                float* dx, bool acc, int H, const float* dbias, const float* wb,
                const float* dres = nullptr, const float* gmul = nullptr);
// Channel-major ([C][M]) input forms used by the triangle multiplication.
void ln_fwd_cm(hipStream_t st, const float* x, long M, int C, const float* gamma,
               const float* beta, h16* y, float* mean, float* rstd, bool fast);
void ln_fwd_cm(hipStream_t st, const h16* x, long M, int C, const float* gamma,
               const float* beta, h16* y, float* mean, float* rstd, bool fast);
void ln_bwd_cm(hipStream_t st, const float* dy, const float* x, long M, int C,
               const float* gamma, const float* mean, const float* rstd, h16* dx);
void ln_bwd_cm(hipStream_t st, const float* dy, const h16* x, long M, int C,
               const float* gamma, const float* mean, const float* rstd, h16* dx);

// ---------------------------------------------------------------- attention
// Gated multi-head attention over R independent rows of N tokens, H heads of
// width D, keys = queries = the N tokens of the row (AF2 Attention with a
// per-(row,key) mask and an optional per-head [H][N][N] bias shared by rows).
struct AttnArgs {
  int R = 0, H = 0, N = 0, D = 32;
  // q|k|v|g for token t = r*N+i live in row t of `qkvg` (row stride ld):
  // q at column h*D (pre-scaled by D^-1/2 * log2 e), k at H*D+h*D,
  // v at 2*H*D+h*D, gate pre-activation at 3*H*D+h*D.
  const h16* qkvg = nullptr;
  long ld = 0;
  const float* mask = nullptr;  // mask[r*mask_sr + k*mask_sk], binary 0/1
  long mask_sr = 0, mask_sk = 0;
  const h16* bias = nullptr;  // [H][N][N] binary16, log2 domain, score-fragment order, or null
  h16* o = nullptr;            // ungated output [R*N][H*D]
  h16* og = nullptr;           // sigmoid(g) * o   [R*N][H*D]
  long ldo = 0;
  float* lse = nullptr;         // [R][H][N], log2 domain
  // launch-site tag for the per-kernel timer: 0 triangle attention, 1 MSA
  // row attention (the template stack's D=16 launches are told apart by D)
  int site = 0;
};
void attn_fwd(hipStream_t st, const AttnArgs& a);

struct AttnBwdArgs {
  AttnArgs f;                  // forward operands (o, lse read back)
  const h16* dog = nullptr;   // upstream gradient of og [R*N][H*D]
  h16* dO = nullptr;          // scratch: dL/do [R*N][H*D]
  float* nDsum = nullptr;      // scratch: [R][H][N] -rowsum(dO*o) (negated: the
                               // dP - Dsum accumulators start from it as stored)
  h16* dqkvg = nullptr;       // out: dq|dk|dv|dg with the layout of qkvg
  float* dbias_part = nullptr; // scratch: [nchunk][H][N][N]
  float* dbias = nullptr;      // out: [H][N][N] (natural units), or null
  float scale = 1.f;           // D^-1/2 (q scaling applied in the forward)
  int rows_per_chunk = 8;
  // dO, nDsum and the gate gradient already written by the caller (the
  // d(og) GEMM's EpiGateBwd epilogue); dog is then not read
  bool gate_done = false;
  // the caller adds the attn_bwd_nchunk partials itself (in chunk order, as
  // the reduction would): no reduction launch; with one chunk the partial is
  // dbias itself
  bool dbias_deferred = false;
};
void attn_bwd(hipStream_t st, const AttnBwdArgs& a);
int attn_bwd_nchunk(int R, int rows_per_chunk);
int attn_rows_per_chunk(int R, int N, int H, int D);

// f32 LayerNorm over rows of any width (one wave per row); dx may alias dy.
void ln_f32_rows_fwd(hipStream_t st, const float* x, long M, int C, const float* g,
                     const float* b, float* y, float* mean, float* rstd);
void ln_f32_rows_bwd(hipStream_t st, const float* dy, const float* x, long M, int C,
                     const float* g, const float* mean, const float* rstd, float* dx);

// ------------------------------------------------- triangle multiplication
// C_c[m][n] = sum_k A_c[m][k] B_c[n][k] for c < channels, N x N planes at
// stride N*N; an operand plane is K-contiguous ((r, k) at r*N + k) or k-major
// ((r, k) at k*N + r).  Writes Cf (f32) if non-null, else Cb (h16).  Returns
// false (and launches nothing) when N is outside the kernel's range
// (N % 32 != 0 or N > 256).
bool trimul_contract(hipStream_t st, int N, int channels, const h16* A, bool a_kcontig,
                     const h16* B, bool b_kcontig, float* Cf, h16* Cb);

// p[0..n) = 0 by a kernel (graph-capture safe, unlike hipMemsetAsync).
void zero_f32(hipStream_t st, float* p, long n);

// ------------------------------------------------------- cotangent scales
// The backward rounds cotangents to binary16 after multiplying them by a
// power-of-two scale s and divides s out in the f32 epilogue that ends the
// module (the backward is linear in the cotangent, so this is exact up to the
// rounding it is for).  ct_scale writes sc[0] = s, sc[1] = 1/s with
// s * max|x| in (8, 16] (s = 1 for an all-zero x); x: n floats, 16-byte
// aligned, n % 4 == 0.  sc must be device memory; ct_scale_slot(k) is one of
// the library's 8 two-float slots on the current device (0: a module's own
// scale; 1, 2: the stack's per-block pair and MSA scales; 3: the template
// embedding).  No allocation.
void ct_scale(hipStream_t st, const float* x, long n, float* sc);
float* ct_scale_slot(int k);
// The same scale from partial maxima a producing kernel wrote (np of them at
// ct_fused_parts()): the final reduction alone.  ct_fused_parts is the
// calling lane's region of CT_FUSED floats (file-scope device memory).
constexpr long CT_FUSED = 16384;
float* ct_fused_parts();
void ct_scale_parts(hipStream_t st, const float* part, long np, float* sc);

// ---------------------------------------------------------------- dropout
// Shared-dropout keep/scale table for one module: tbl[b*C+c] = keep/keep_rate
// (0 where dropped), with keep = jax.random.uniform(key,(B,C)) < keep_rate.
void dropout_table(hipStream_t st, float* tbl, int B, int C, uint32_t k0,
                   uint32_t k1, float keep_rate);
// Same with the key (2 x u32) and the enable flag (u32, may be null) in device
// memory; a disabled flag gives an all-ones table (rate 0).
void dropout_table_dev(hipStream_t st, float* tbl, int B, int C,
                       const uint32_t* key, const uint32_t* enabled, float keep_rate);
// All of a stack's dropout tables in one launch (see ew.hip).
void stack_dropout_tables(hipStream_t st, float* tbl, long per_block, int N, int Cm, int Cz,
                          int depth, int nk, bool msa_row, int row_key, const int (&pair_keys)[4],
                          const uint32_t* keys, const uint32_t* enabled);
// out[i] = jax.random.bernoulli(key, keep_rate, (n,))[i].
void bernoulli_bits(hipStream_t st, uint8_t* out, long n, uint32_t k0, uint32_t k1,
                    float keep_rate);
// Per-module keys of a `depth`-layer stack from the stack key seed[0..1]:
// out[(layer*n_used+module)*2 + {0,1}] = split(sub_layer)[1 + module]
// (n_used = 9: Evoformer; 5: template pair stack).
void stack_keys(hipStream_t st, const uint32_t* seed, int depth, uint32_t* out,
                int n_used = 9);
// out[0..1] = (0, seed[0]): PRNGKey of a 32-bit seed word, on the device.
void key_from_bits(hipStream_t st, const uint32_t* seed, uint32_t* out);

// MFMA issue-rate probe (probe.hip): `blocks` workgroups of 4 waves, each
// wave 8 independent chains of `iters` MFMAs of one form (0: 16x16x32 f16,
// 1: 16x16x16 f16, 2: 32x32x16 f16, 3: 16x16x32 bf16) on register operands;
// out holds blocks*256 floats.
// Returns the FLOPs the launch executes.
double probe_mfma_rate(hipStream_t st, int form, int blocks, int iters, float* out);

}  // namespace bc2n
