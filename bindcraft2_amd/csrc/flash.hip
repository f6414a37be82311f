// Flash attention forward/backward for AF2's gated attention with pair bias,
// written for wave64 and gfx950 MFMA, head width D = 32 (Evoformer) or 16
// (template stack).
//
// Every product is arranged so that the lane -> query (or lane -> key)
// assignment of the MFMA result is the one the next MFMA needs as its B
// operand, so probabilities never leave registers:
//
//   forward / dQ:  S^T = K Q^T       -> lane l owns query l%16, 8 keys
//                  O^T += V^T P^T    (B operand = those 8 probabilities)
//                  dQ^T += K^T dS^T
//   dK/dV:         S = Q K^T         -> lane l owns key l%16, 8 queries
//                  dV^T += dO^T P,   dK^T += Q^T dS
//
// The contraction over the head width uses v_mfma_f32_16x16x32_bf16 (D=32)
// or v_mfma_f32_16x16x16_bf16 (D=16); the contraction over 32 keys (or 32
// queries) always uses the x32 form.  For that second product the 8 K-slots
// of lane group g=l/16 are mapped to positions {4g..4g+3, 16+4g..16+4g+3}
// of the 32-block, for both operands; the first product's result already
// sits in exactly that order.
//
// Scores are kept in the log2 domain: q is pre-scaled by D^-1/2 * log2(e)
// and the pair bias by log2(e) upstream, so a score is one MFMA plus one add.
// A masked key takes one shared constant score, as AF2's
// clip(-1e9 + x, -1e8, 1e8) gives every masked key the same -1e8: a fully
// masked row attends uniformly, partially masked rows give masked keys zero
// weight, and masked keys carry no gradient (the clip's derivative is 0).
// The constant is -2^13 rather than -1e8*log2(e): only score differences
// matter, 2^13 log2-units (5678 natural units) is far beyond any unmasked
// logit, and at that magnitude f32 still resolves the row's log-sum-exp
// (lse = -2^13 + log2 N) to ~1e-3, so the backward's exp2(s - lse) = 1/N on a
// fully masked row is exact to bf16 precision.
//
// The bias gradient (a sum over rows) is accumulated in registers over a
// chunk of rows and written once per chunk; a second pass adds the chunks in
// a fixed order, so the result is deterministic (no float atomics anywhere).
#include "kernels.h"
#include "runtime.h"

namespace bc2n {

constexpr float NEG_LOGIT = -8192.0f;

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// 8 bf16 from two runs of 4 contiguous elements (positions p and p+16).
__device__ __forceinline__ bf16x8 ld_slots(const bf16* p) {
  const bf16x4 a = *reinterpret_cast<const bf16x4*>(p);
  const bf16x4 b = *reinterpret_cast<const bf16x4*>(p + 16);
  bf16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// Operand fragment of the head-width contraction for lane group g.
template <int D>
struct HFrag;
template <>
struct HFrag<32> {
  bf16x8 v;
  __device__ __forceinline__ void load(const bf16* row, int g) { v = ld8(row + 8 * g); }
  __device__ __forceinline__ static f32x4 mma(const HFrag& a, const HFrag& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a.v, b.v, c, 0, 0, 0);
  }
};
template <>
struct HFrag<16> {
  bf16x4 v;
  __device__ __forceinline__ void load(const bf16* row, int g) {
    v = *reinterpret_cast<const bf16x4*>(row + 4 * g);
  }
  __device__ __forceinline__ static f32x4 mma(const HFrag& a, const HFrag& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a.v, b.v, c, 0, 0, 0);
  }
};

// ------------------------------------------------------------------ forward
// Workgroup = (row r, head h, 64 queries); 4 waves x 16 queries.  The row's
// K (row-major) and V (transposed) for head h are staged once in LDS.
template <int D>
__global__ __launch_bounds__(256) void attn_fwd_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  constexpr int DT = D / 16;
  const int N = a.N, H = a.H;
  const int KLD = D + 8, VLD = N + 8;
  bf16* Ks = reinterpret_cast<bf16*>(smem_raw);          // [N][KLD]
  bf16* Vt = Ks + N * KLD;                               // [D][VLD]
  float* Ms = reinterpret_cast<float*>(Vt + D * VLD);    // [N]

  const int nqb = (N + 63) / 64;
  const int qb = blockIdx.x % nqb;
  const int h = (blockIdx.x / nqb) % H;
  const int r = blockIdx.x / (nqb * H);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long tok0 = (long)r * N;
  const bf16* Kg = a.qkvg + tok0 * a.ld + H * D + h * D;
  const bf16* Vg = a.qkvg + tok0 * a.ld + 2 * H * D + h * D;
  for (int c = tid; c < N * (D / 8); c += 256) {
    const int k = c / (D / 8), dc = (c % (D / 8)) * 8;
    st8(&Ks[k * KLD + dc], ld8(Kg + (long)k * a.ld + dc));
    const bf16x8 v = ld8(Vg + (long)k * a.ld + dc);
#pragma unroll
    for (int e = 0; e < 8; ++e) Vt[(dc + e) * VLD + k] = v[e];
  }
  for (int k = tid; k < N; k += 256) Ms[k] = a.mask[r * a.mask_sr + k * a.mask_sk];
  __syncthreads();

  const int q0 = qb * 64 + wave * 16;
  if (q0 >= N) return;  // no barrier follows
  const int lq = lane & 15, g = lane >> 4;
  const int q = q0 + lq;
  HFrag<D> qf;
  qf.load(a.qkvg + (tok0 + q) * a.ld + h * D, g);
  const float* brow = a.bias ? a.bias + ((long)h * N + q) * N : nullptr;

  float mrun = -INFINITY, lrun = 0.f;
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = z4;
  for (int kb = 0; kb < N; kb += 32) {
    float sv[8];
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      HFrag<D> kf;
      kf.load(&Ks[(kb + kh * 16 + lq) * KLD], g);
      const f32x4 s = HFrag<D>::mma(kf, qf, z4);
      const int key0 = kb + kh * 16 + 4 * g;
      float4 bb = brow ? *reinterpret_cast<const float4*>(brow + key0)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 mm = *reinterpret_cast<const float4*>(Ms + key0);
      sv[kh * 4 + 0] = mm.x != 0.f ? s[0] + bb.x : NEG_LOGIT;
      sv[kh * 4 + 1] = mm.y != 0.f ? s[1] + bb.y : NEG_LOGIT;
      sv[kh * 4 + 2] = mm.z != 0.f ? s[2] + bb.z : NEG_LOGIT;
      sv[kh * 4 + 3] = mm.w != 0.f ? s[3] + bb.w : NEG_LOGIT;
    }
    float bm = sv[0];
#pragma unroll
    for (int e = 1; e < 8; ++e) bm = fmaxf(bm, sv[e]);
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mnew = fmaxf(mrun, bm);
    const float alpha = fast_exp2(mrun - mnew);
    bf16x8 pf;
    float ps = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float p = fast_exp2(sv[e] - mnew);
      ps += p;
      pf[e] = (bf16)p;
    }
    lrun = lrun * alpha + ps;
    mrun = mnew;
#pragma unroll
    for (int dh = 0; dh < DT; ++dh) {
      acc[dh] *= alpha;
      const bf16x8 vf = ld_slots(&Vt[(dh * 16 + lq) * VLD + kb + 4 * g]);
      acc[dh] = mfma16x16x32(vf, pf, acc[dh]);
    }
  }
  lrun += __shfl_xor(lrun, 16, 64);
  lrun += __shfl_xor(lrun, 32, 64);
  const float inv = 1.f / lrun;
  const long orow = (tok0 + q) * a.ldo + h * D;
  const bf16* grow = a.qkvg + (tok0 + q) * a.ld + 3 * H * D + h * D;
#pragma unroll
  for (int dh = 0; dh < DT; ++dh) {
    const int d0 = dh * 16 + 4 * g;
    const bf16x4 gv = *reinterpret_cast<const bf16x4*>(grow + d0);
    bf16x4 ov, gov;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float o = acc[dh][i] * inv;
      ov[i] = (bf16)o;
      gov[i] = (bf16)(o * sigmoidf_((float)gv[i]));
    }
    *reinterpret_cast<bf16x4*>(a.o + orow + d0) = ov;
    *reinterpret_cast<bf16x4*>(a.og + orow + d0) = gov;
  }
  if (g == 0) a.lse[((long)r * H + h) * N + q] = mrun + __log2f(lrun);
}

// ------------------------------------------------------- backward: gate + D
// dO = dog * sigmoid(g); dG = dog * o * s(1-s); Dsum = sum_d dO * o.
// D/8 lanes per (token, head), 8 channels each.
template <int D>
__global__ __launch_bounds__(256) void attn_gate_bwd_kernel(AttnBwdArgs b) {
  constexpr int LPH = D / 8;
  const AttnArgs& a = b.f;
  const long idx = (long)blockIdx.x * (256 / LPH) + threadIdx.x / LPH;
  const int part = threadIdx.x % LPH;
  const long total = (long)a.R * a.N * a.H;
  if (idx >= total) return;
  const int h = (int)(idx % a.H);
  const long tok = idx / a.H;
  const int HD = a.H * D;
  const int c0 = h * D + part * 8;
  const bf16x8 gv = ld8(a.qkvg + tok * a.ld + 3 * HD + c0);
  const bf16x8 ov = ld8(a.o + tok * a.ldo + c0);
  const bf16x8 dv = ld8(b.dog + tok * a.ldo + c0);
  bf16x8 dov, dgv;
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sg = sigmoidf_((float)gv[e]);
    const float o = (float)ov[e], d = (float)dv[e];
    const float dO = d * sg;
    dov[e] = (bf16)dO;
    dgv[e] = (bf16)(d * o * sg * (1.f - sg));
    s += dO * o;
  }
  st8(b.dO + tok * a.ldo + c0, dov);
  st8(b.dqkvg + tok * a.ld + 3 * HD + c0, dgv);
  s = group_sum<LPH>(s);
  if (part == 0) {
    const long r = tok / a.N, q = tok % a.N;
    b.Dsum[(r * a.H + h) * a.N + q] = s;
  }
}

// ----------------------------------------------------------- backward: dQ
// Same decomposition as the forward: (row, head, 64 queries), 4 waves.
template <int D>
__global__ __launch_bounds__(256) void attn_bwd_dq_kernel(AttnBwdArgs b) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  constexpr int DT = D / 16;
  const AttnArgs& a = b.f;
  const int N = a.N, H = a.H;
  const int KLD = D + 8, TLD = N + 8;
  bf16* Ks = reinterpret_cast<bf16*>(smem_raw);   // [N][KLD]
  bf16* Vs = Ks + N * KLD;                        // [N][KLD]
  bf16* Kt = Vs + N * KLD;                        // [D][TLD]
  float* Ms = reinterpret_cast<float*>(Kt + D * TLD);

  const int nqb = (N + 63) / 64;
  const int qb = blockIdx.x % nqb;
  const int h = (blockIdx.x / nqb) % H;
  const int r = blockIdx.x / (nqb * H);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long tok0 = (long)r * N;
  const bf16* Kg = a.qkvg + tok0 * a.ld + H * D + h * D;
  const bf16* Vg = a.qkvg + tok0 * a.ld + 2 * H * D + h * D;
  for (int c = tid; c < N * (D / 8); c += 256) {
    const int k = c / (D / 8), dc = (c % (D / 8)) * 8;
    const bf16x8 kv = ld8(Kg + (long)k * a.ld + dc);
    st8(&Ks[k * KLD + dc], kv);
    st8(&Vs[k * KLD + dc], ld8(Vg + (long)k * a.ld + dc));
#pragma unroll
    for (int e = 0; e < 8; ++e) Kt[(dc + e) * TLD + k] = kv[e];
  }
  for (int k = tid; k < N; k += 256) Ms[k] = a.mask[r * a.mask_sr + k * a.mask_sk];
  __syncthreads();

  const int q0 = qb * 64 + wave * 16;
  if (q0 >= N) return;
  const int lq = lane & 15, g = lane >> 4;
  const int q = q0 + lq;
  HFrag<D> qf, dof;
  qf.load(a.qkvg + (tok0 + q) * a.ld + h * D, g);
  dof.load(b.dO + (tok0 + q) * a.ldo + h * D, g);
  const float lse = a.lse[((long)r * H + h) * N + q];
  const float Dq = b.Dsum[((long)r * H + h) * N + q];
  const float* brow = a.bias ? a.bias + ((long)h * N + q) * N : nullptr;
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = z4;
  for (int kb = 0; kb < N; kb += 32) {
    bf16x8 dsf;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const int krow = (kb + kh * 16 + lq) * KLD;
      HFrag<D> kf, vf;
      kf.load(&Ks[krow], g);
      vf.load(&Vs[krow], g);
      const f32x4 s = HFrag<D>::mma(kf, qf, z4);
      const f32x4 dp = HFrag<D>::mma(vf, dof, z4);
      const int key0 = kb + kh * 16 + 4 * g;
      float4 bb = brow ? *reinterpret_cast<const float4*>(brow + key0)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
      const float4 mm = *reinterpret_cast<const float4*>(Ms + key0);
      const float bv[4] = {bb.x, bb.y, bb.z, bb.w};
      const float mv[4] = {mm.x, mm.y, mm.z, mm.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = fast_exp2(s[i] + bv[i] - lse);
        dsf[kh * 4 + i] = (bf16)(mv[i] != 0.f ? p * (dp[i] - Dq) : 0.f);
      }
    }
#pragma unroll
    for (int dh = 0; dh < DT; ++dh) {
      const bf16x8 kt = ld_slots(&Kt[(dh * 16 + lq) * TLD + kb + 4 * g]);
      acc[dh] = mfma16x16x32(kt, dsf, acc[dh]);
    }
  }
  bf16* out = b.dqkvg + (tok0 + q) * a.ld + h * D;
#pragma unroll
  for (int dh = 0; dh < DT; ++dh) {
    bf16x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (bf16)(acc[dh][i] * b.scale);
    *reinterpret_cast<bf16x4*>(out + dh * 16 + 4 * g) = v;
  }
}

// ------------------------------------------------------ backward: dK, dV, dB
// Workgroup = (head h, 32 keys, chunk of rows), 4 waves: wave w owns key
// tile w&1 (16 keys) and the 32-query blocks ib with ib%2 == w>>1, so the
// bias-gradient tile it keeps in registers is ceil(N/64) x 8 floats per lane.
// Per row, Q^T and dO^T (head h) are staged in LDS; the two query halves'
// dK/dV partials are combined through LDS before the write.  NQ_MAX bounds N.
template <int D, int NQ_MAX>
__global__ __launch_bounds__(256) void attn_bwd_dkv_kernel(AttnBwdArgs b) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  constexpr int DT = D / 16;
  constexpr int NB = (NQ_MAX / 32 + 1) / 2;  // query blocks per wave
  const AttnArgs& a = b.f;
  const int N = a.N, H = a.H;
  const int TLD = N + 8;
  bf16* Qt = reinterpret_cast<bf16*>(smem_raw);         // [D][TLD]
  bf16* Dt = Qt + D * TLD;                              // [D][TLD]
  float* Ls = reinterpret_cast<float*>(Dt + D * TLD);   // [N] lse
  float* Ds = Ls + N;                                   // [N] Dsum
  float* Xs = Ds + N;                                   // [2 tiles][K,V][DT*4][64]

  const int nkb = (N + 31) / 32;
  const int kb32 = blockIdx.x % nkb;
  const int h = (blockIdx.x / nkb) % H;
  const int ch = blockIdx.x / (nkb * H);
  const int r0 = ch * b.rows_per_chunk;
  const int r1 = min(a.R, r0 + b.rows_per_chunk);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int kt_ = wave & 1, half = wave >> 1;
  const int lk = lane & 15, g = lane >> 4;
  const int k = kb32 * 32 + kt_ * 16 + lk;
  const int nqblk = N / 32;
  float dbias[NB][8];
#pragma unroll
  for (int i = 0; i < NB; ++i)
#pragma unroll
    for (int e = 0; e < 8; ++e) dbias[i][e] = 0.f;
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  const long HD = (long)H * D;
  float* xk = Xs + (kt_ * 2 + 0) * DT * 4 * 64;
  float* xv = Xs + (kt_ * 2 + 1) * DT * 4 * 64;

  for (int r = r0; r < r1; ++r) {
    const long tok0 = (long)r * N;
    __syncthreads();  // previous row's LDS readers are done
    for (int c = tid; c < N * (D / 8); c += 256) {
      const int qq = c / (D / 8), dc = (c % (D / 8)) * 8;
      const bf16x8 qv = ld8(a.qkvg + (tok0 + qq) * a.ld + h * D + dc);
      const bf16x8 dv = ld8(b.dO + (tok0 + qq) * a.ldo + h * D + dc);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        Qt[(dc + e) * TLD + qq] = qv[e];
        Dt[(dc + e) * TLD + qq] = dv[e];
      }
    }
    for (int qq = tid; qq < N; qq += 256) {
      Ls[qq] = a.lse[((long)r * H + h) * N + qq];
      Ds[qq] = b.Dsum[((long)r * H + h) * N + qq];
    }
    __syncthreads();
    HFrag<D> kf, vf;
    kf.load(a.qkvg + (tok0 + k) * a.ld + HD + h * D, g);
    vf.load(a.qkvg + (tok0 + k) * a.ld + 2 * HD + h * D, g);
    const bool mk = a.mask[r * a.mask_sr + k * a.mask_sk] != 0.f;
    f32x4 accK[DT], accV[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i) { accK[i] = z4; accV[i] = z4; }
#pragma unroll
    for (int ib = 0; ib < NB; ++ib) {
      const int blk = ib * 2 + half;
      if (blk >= nqblk) break;
      const int qb = blk * 32;
      bf16x8 pf, dsf;
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        const long qrow = tok0 + qb + qh * 16 + lk;
        HFrag<D> qa, da;
        qa.load(a.qkvg + qrow * a.ld + h * D, g);
        da.load(b.dO + qrow * a.ldo + h * D, g);
        const f32x4 s = HFrag<D>::mma(qa, kf, z4);
        const f32x4 dp = HFrag<D>::mma(da, vf, z4);
        const int qi0 = qb + qh * 16 + 4 * g;
        const float4 lv = *reinterpret_cast<const float4*>(Ls + qi0);
        const float4 dv = *reinterpret_cast<const float4*>(Ds + qi0);
        const float lsv[4] = {lv.x, lv.y, lv.z, lv.w};
        const float dsv[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float bb = a.bias ? a.bias[((long)h * N + qi0 + i) * N + k] : 0.f;
          const float sc = mk ? s[i] + bb : NEG_LOGIT;
          const float p = fast_exp2(sc - lsv[i]);
          const float ds = mk ? p * (dp[i] - dsv[i]) : 0.f;
          pf[qh * 4 + i] = (bf16)p;
          dsf[qh * 4 + i] = (bf16)ds;
          dbias[ib][qh * 4 + i] += ds;
        }
      }
#pragma unroll
      for (int dh = 0; dh < DT; ++dh) {
        const bf16x8 dot = ld_slots(&Dt[(dh * 16 + lk) * TLD + qb + 4 * g]);
        accV[dh] = mfma16x16x32(dot, pf, accV[dh]);
        const bf16x8 qt = ld_slots(&Qt[(dh * 16 + lk) * TLD + qb + 4 * g]);
        accK[dh] = mfma16x16x32(qt, dsf, accK[dh]);
      }
    }
    // combine the two query halves: half 1 parks its partials in LDS
    if (half == 1) {
#pragma unroll
      for (int dh = 0; dh < DT; ++dh)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xk[(dh * 4 + i) * 64 + lane] = accK[dh][i];
          xv[(dh * 4 + i) * 64 + lane] = accV[dh][i];
        }
    }
    __syncthreads();
    if (half == 0) {
      // dK (w.r.t. the unscaled k) = sum_q dS * q_scaled / log2(e)
      bf16* dk = b.dqkvg + (tok0 + k) * a.ld + HD + h * D;
      bf16* dvp = b.dqkvg + (tok0 + k) * a.ld + 2 * HD + h * D;
#pragma unroll
      for (int dh = 0; dh < DT; ++dh) {
        bf16x4 kv, vv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          kv[i] = (bf16)((accK[dh][i] + xk[(dh * 4 + i) * 64 + lane]) * (1.f / LOG2E));
          vv[i] = (bf16)(accV[dh][i] + xv[(dh * 4 + i) * 64 + lane]);
        }
        *reinterpret_cast<bf16x4*>(dk + dh * 16 + 4 * g) = kv;
        *reinterpret_cast<bf16x4*>(dvp + dh * 16 + 4 * g) = vv;
      }
    }
  }
  if (b.dbias_part == nullptr) return;
  float* part = b.dbias_part + (((long)ch * H + h) * N) * N;
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {
    const int blk = ib * 2 + half;
    if (blk >= nqblk) break;
    const int qb = blk * 32;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int qi = qb + (e / 4) * 16 + 4 * g + (e % 4);
      part[(long)qi * N + k] = dbias[ib][e];
    }
  }
}

__global__ void attn_dbias_reduce_kernel(const float* __restrict__ part, int nch,
                                         long n, float* __restrict__ out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  float s = 0.f;
  for (int c = 0; c < nch; ++c) s += part[(long)c * n + i];
  out[i] = s;
}

// ------------------------------------------------------------------ launchers

int attn_bwd_nchunk(int R, int rows_per_chunk) {
  return (R + rows_per_chunk - 1) / rows_per_chunk;
}

static void attn_check(const AttnArgs& a) {
  if (a.D != 32 && a.D != 16) throw std::runtime_error("attention: head width must be 16 or 32");
  if (a.N <= 0 || a.N % 32 != 0) throw std::runtime_error("attention: N must be a positive multiple of 32");
  if (a.N > 256) throw std::runtime_error("attention: N > 256 not supported yet");
  if (a.ld % 8 != 0 || a.ldo % 8 != 0) throw std::runtime_error("attention: row strides must be multiples of 8");
  if (!a.qkvg || !a.mask || !a.lse || !a.o) throw std::runtime_error("attention: missing operand");
}

template <int D>
static void attn_fwd_t(hipStream_t st, const AttnArgs& a) {
  const int nqb = (a.N + 63) / 64;
  const size_t lds = (size_t)a.N * (D + 8) * 2 + (size_t)D * (a.N + 8) * 2 + (size_t)a.N * 4;
  KTimed kt("attn_fwd", st);
  hipLaunchKernelGGL((attn_fwd_kernel<D>), dim3(a.R * a.H * nqb), dim3(256), lds, st, a);
}

void attn_fwd(hipStream_t st, const AttnArgs& a) {
  attn_check(a);
  if (!a.og) throw std::runtime_error("attention: missing gated output");
  if (a.D == 32) attn_fwd_t<32>(st, a);
  else attn_fwd_t<16>(st, a);
}

template <int D>
static void attn_bwd_t(hipStream_t st, const AttnBwdArgs& b) {
  const AttnArgs& a = b.f;
  const long tot = (long)a.R * a.N * a.H;
  {
    KTimed kt("attn_gate_bwd", st);
    const long per = 256 / (D / 8);
    hipLaunchKernelGGL((attn_gate_bwd_kernel<D>), dim3((unsigned)((tot + per - 1) / per)),
                       dim3(256), 0, st, b);
  }
  const int nqb = (a.N + 63) / 64;
  const size_t lds_q = (size_t)a.N * (D + 8) * 2 * 2 + (size_t)D * (a.N + 8) * 2 + (size_t)a.N * 4;
  {
    KTimed kt("attn_bwd_dq", st);
    hipLaunchKernelGGL((attn_bwd_dq_kernel<D>), dim3(a.R * a.H * nqb), dim3(256), lds_q, st, b);
  }
  const int nch = attn_bwd_nchunk(a.R, b.rows_per_chunk);
  const int nkb = (a.N + 31) / 32;
  const size_t lds_k = (size_t)D * (a.N + 8) * 2 * 2 + (size_t)a.N * 4 * 2 +
                       (size_t)2 * 2 * (D / 16) * 4 * 64 * 4;
  {
    KTimed kt("attn_bwd_dkv", st);
    hipLaunchKernelGGL((attn_bwd_dkv_kernel<D, 256>), dim3(nch * a.H * nkb), dim3(256), lds_k, st,
                       b);
  }
  if (b.dbias && a.bias) {
    if (!b.dbias_part) throw std::runtime_error("attention bwd: missing dbias scratch");
    const long n = (long)a.H * a.N * a.N;
    KTimed kt("attn_dbias_reduce", st);
    hipLaunchKernelGGL(attn_dbias_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       b.dbias_part, nch, n, b.dbias);
  }
}

void attn_bwd(hipStream_t st, const AttnBwdArgs& b) {
  attn_check(b.f);
  if (!b.dog || !b.dO || !b.Dsum || !b.dqkvg) throw std::runtime_error("attention bwd: missing operand");
  if (b.f.D == 32) attn_bwd_t<32>(st, b);
  else attn_bwd_t<16>(st, b);
}

}  // namespace bc2n
