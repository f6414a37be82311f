// Triangle multiplication (outgoing 'ikc,jkc->ijc' / incoming 'kjc,kic->ijc'),
// AF2's fused-projection form, forward and backward.
//
// Forward:
//   LN (fast variance) -> xn h16
//   GEMM xn . Wcat  (Wcat = [proj|gate] channel pairs interleaved in 16-wide
//        blocks, then gating_linear), fused epilogue:
//          a = mask * proj * sigmoid(gate)   -> left/right planes [I][N*N] h16
//          g_out = sigmoid(gating_linear)  -> [M][C] h16
//        (xn is kept; the backward recomputes the proj/gate pre-activations)
//   batched MFMA GEMM over the I channels (plane layouts pick out/in)  -> T f32
//     (kept in f32: a sum of N products has no range bound binary16 holds)
//   centre LN (fast variance) reading the channel-major T            -> Tn h16
//   GEMM Tn . Wo + bo, fused: o kept, out = in + tbl * (o * g_out)
// Backward: the exact reverse with the contraction's two transposed GEMMs; the
// projection's gradient comes from a GEMM that recomputes the pre-activations
// from xn and turns them, with d(left|right), into the [proj|gate] columns of
// d(cat) in its epilogue.  The backward runs on the cotangent times the
// module's scale s (ct_scale), applied as the output projection's backward
// loads it and divided out by the input LayerNorm's backward at the end.
// Reference: modules.py:1044-1088 (_fused_triangle_multiplication), :909-919
// (fast-variance LN); native/trimul_body.cuh:1183-1796 (TriMul).
#include "gemm.h"
#include "lnproj.h"
#include "modules.h"

namespace bc2n {

namespace {

// GEMM column of projection channel ch (0..2I) and of its gate.
__host__ __device__ inline int col_proj(int ch) { return (ch / 16) * 32 + ch % 16; }
__host__ __device__ inline int col_gate(int ch) { return (ch / 16) * 32 + 16 + ch % 16; }

// Projection epilogue.  Tiles of the [proj|gate] columns (n0 < 4I) run in
// column mode: the thread of a proj column reads its gate column (16 to the
// right, same tile) from LDS and writes 8 consecutive m of the channel-major
// planes: a = mask * proj * sigmoid(gate) into left/right.  Tiles of
// gating_linear columns run in row mode: g_out[m][c] = sigmoid(acc + b).
struct EpiTrimulProj {
  static constexpr bool kHasCol = true;
  static constexpr bool kColPairs = true;  // col() of column c also does its gate c + 16
  h16 *left, *right;   // [I][M]
  h16* gout;           // [M][C]
  const float *bp, *bg, *bgl, *mask;
  long M;
  int I, C;
  __device__ __forceinline__ bool col_mode(int n0) const { return n0 < 4 * I; }
  __device__ __forceinline__ void col(int, int m, int n, const float (&v)[8], const float* tp,
                                      int ldt) const {
    if ((n & 31) >= 16) return;  // gate column: done by its projection column
    const int ch = (n >> 5) * 16 + (n & 15);
    const float bpv = bp[ch], bgv = bg[ch];
    float mk[8];
    ld_f8(mask + m, mk);
    float pv[8], gv[8], av[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pv[e] = v[e] + bpv;
      gv[e] = tp[e * ldt + 16] + bgv;
      av[e] = mk[e] * pv[e] * sigmoidf_(gv[e]);
    }
    if (ch < I) st_h8f(left + (long)ch * M + m, av);
    else st_h8f(right + (long)(ch - I) * M + m, av);
  }
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const int c = n - 4 * I;
    if (c < 0 || c >= C) return;
    float bb[8], x[8];
    ld_f8(bgl + c, bb);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = sigmoidf_(v[e] + bb[e]);
    st_h8f(gout + (long)m * C + c, x);
  }
};

// o = acc + bo (kept, h16); out[m] = in[m] + tbl[(m%nt)*C+c] * o * g_out
struct EpiTrimulOut : EpiRows {
  const float* in;
  float* out;
  const float* bo;
  const h16* gout;
  h16* osave;
  const float* tbl;
  int nt, C;
  EpiTrimulOut(const float* i, float* o, const float* b, const h16* g, h16* os, const float* t,
               int n, int c)
      : in(i), out(o), bo(b), gout(g), osave(os), tbl(t), nt(n), C(c) {}
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const long o = (long)m * C + n;
    float bb[8], ov[8], gv[8], r[8];
    ld_f8(bo + n, bb);
#pragma unroll
    for (int e = 0; e < 8; ++e) ov[e] = v[e] + bb[e];
    st_h8f(osave + o, ov);
    ld_h8f(gout + o, gv);
#pragma unroll
    for (int e = 0; e < 8; ++e) gv[e] *= ov[e];
    if (tbl) {
      float tt[8];
      ld_f8(tbl + (long)(m % nt) * C + n, tt);
#pragma unroll
      for (int e = 0; e < 8; ++e) gv[e] *= tt[e];
    }
    ld_f8(in + o, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] += gv[e];
    st_f8(out + o, r);
  }
};

template <class A>
struct TriMulSave {
  float *mean, *rstd, *cmean, *crstd, *T;
  h16 *xn, *left, *right, *gout, *osave;
  TriMulSave(A& a, int N, int C, int I) {
    const size_t M = (size_t)N * N;
    mean = a.template take<float>(M);
    rstd = a.template take<float>(M);
    cmean = a.template take<float>(M);
    crstd = a.template take<float>(M);
    T = a.template take<float>(M * I);
    xn = a.template take<h16>(M * C);
    left = a.template take<h16>(M * I);
    right = a.template take<h16>(M * I);
    gout = a.template take<h16>(M * C);
    osave = a.template take<h16>(M * C);
  }
};

// Backward of the projection, as the epilogue of the GEMM xn . Wcat[:, :4I]
// that recomputes the [proj|gate] pre-activations.  Column pass: the thread of
// a proj column takes its gate column (16 to the right) from the staged tile
// and d(left|right) for 8 consecutive m (channel-major), and rewrites both
// columns of the tile with
//   dproj = da * mask * s,  dgate = da * mask * p * s(1-s),  s = sigmoid(gate);
// row pass: the rewritten tile goes to the row-major d(cat) columns.
struct EpiTrimulProjBwd {
  static constexpr bool kHasCol = true;
  static constexpr bool kTwoPhase = true;
  const h16 *dl, *dr;  // [I][M]
  const float *bp, *bg, *mask;
  h16* dcat;           // [M][ldcat]
  long M;
  int I, ldcat;
  __device__ __forceinline__ bool col_mode(int) const { return true; }
  __device__ __forceinline__ void col(int, int m, int n, const float (&v)[8], float* tp,
                                      int ldt) const {
    if ((n & 31) >= 16) return;  // gate column: done by its projection column
    const int ch = (n >> 5) * 16 + (n & 15);
    const float bpv = bp[ch], bgv = bg[ch];
    float mk[8], da[8];
    ld_f8(mask + m, mk);
    ld_h8f((ch < I ? dl + (long)ch * M : dr + (long)(ch - I) * M) + m, da);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float pv = v[e] + bpv;
      const float sg = sigmoidf_(tp[e * ldt + 16] + bgv);
      const float a = da[e] * mk[e];
      tp[e * ldt] = a * sg;
      tp[e * ldt + 16] = a * pv * sg * (1.f - sg);
    }
  }
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    st_h8f(dcat + (long)m * ldcat + n, v);
  }
};

// A loader of the output-projection backward GEMM: d = s*tbl*dout (s = *mul,
// the cotangent scale); A = d*g_out (the GEMM operand) and, as a side output,
// dcat[m][off + c] = d * o * g(1-g)   (gating_linear pre-activation grad).
struct ALoadTrimulOut {
  static constexpr bool kDirect = false;
  static constexpr bool kSide = true;
  const float* dout;
  const float* tbl;
  const h16* gout;
  const h16* osave;
  h16* dcat;
  int C, ldcat, off, nt;
  const float* mul;
  __device__ __forceinline__ h16x8 operator()(int, int m, int k) const {
    const long i = (long)m * C + k;
    float d[8], gv[8], ov[8];
    ld_f8(dout + i, d);
    const float sm = *mul;
    if (tbl) {
      float t[8];
      ld_f8(tbl + (long)(m % nt) * C + k, t);
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] *= t[e] * sm;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) d[e] *= sm;
    }
    ld_h8f(gout + i, gv);
    ld_h8f(osave + i, ov);
    h16x8 a, dc;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[e] = f2h_sat(d[e] * gv[e]);
      dc[e] = f2h_sat(d[e] * ov[e] * gv[e] * (1.f - gv[e]));
    }
    st8(dcat + (long)m * ldcat + off + k, dc);
    return a;
  }
};

// The centre LayerNorm's backward fused into the d(tn) product as its
// row-block epilogue (I = 128): each staged half tile of d(tn) rows is the dy
// of ln_bwd_cm, normalised with the same arithmetic in the same order (eight
// lanes a row, 16 consecutive channels each, the x values read from the
// channel-major T), and written channel-major in binary16 through the tile,
// so d(tn) never reaches memory.
struct EpiCmLnBwd : EpiRows {
  static constexpr bool kRowBlock = true;
  // four waves a SIMD: the 64-row grid (784 workgroups at 224 tokens) in one
  // round of 1024 slots (three would leave 16 workgroups for a second round)
  static constexpr int kMinWaves = 4;
  static constexpr int C = 128, P = 8, CPL = C / P;
  const float *x, *gamma, *mean, *rstd;  // x: channel-major [C][M]
  h16* dx;                               // channel-major [C][M]
  long M;
  static constexpr int WMP = 256 / P;  // rows a pass: one (of eight lanes) a thread
  __device__ __forceinline__ void row(int, int, int, const float (&)[8]) const {}
  template <int WM>
  __device__ __forceinline__ void block(int, long mb, const float* T, int ldt, int tid) const {
    static_assert(WM == WMP, "one 32-row pass a call");
    float* Tw = const_cast<float*>(T);  // the kernel's own staging tile
    {
      const int r = tid / P, part = tid % P;
      const long m = mb + r;
      const bool live = m < M;
      const float mu = live ? mean[m] : 0.f, rs = live ? rstd[m] : 0.f;
      float xv[CPL];
#pragma unroll
      for (int e = 0; e < CPL; ++e) xv[e] = live ? x[(long)(part * CPL + e) * M + m] : 0.f;
      float xh[CPL], g[CPL];
      float sg = 0.f, sgx = 0.f;
#pragma unroll
      for (int e0 = 0; e0 < CPL; e0 += 4) {
        float4 d = make_float4(0.f, 0.f, 0.f, 0.f);
        if (live) d = *reinterpret_cast<const float4*>(T + r * ldt + part * CPL + e0);
        const float dv[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int e = e0 + k, c = part * CPL + e;
          xh[e] = (xv[e] - mu) * rs;
          g[e] = dv[k] * gamma[c];
          sg += g[e];
          sgx += g[e] * xh[e];
        }
      }
      sg = group_sum<P>(sg) / C;
      sgx = group_sum<P>(sgx) / C;
      // each thread rewrites exactly the 16 values it read
#pragma unroll
      for (int e = 0; e < CPL; ++e) {
        const int c = part * CPL + e;
        Tw[r * ldt + c] = rs * (g[e] - sg - xh[e] * sgx);
      }
    }
    __syncthreads();
    for (int i = tid; i < C * (WM / 4); i += 256) {
      const int c = i / (WM / 4), q = (i % (WM / 4)) * 4;
      const long mm = mb + q;
      if (mm < M) {
        h16x4 o;
        o[0] = f2h_sat(T[(q + 0) * ldt + c]);
        o[1] = f2h_sat(T[(q + 1) * ldt + c]);
        o[2] = f2h_sat(T[(q + 2) * ldt + c]);
        o[3] = f2h_sat(T[(q + 3) * ldt + c]);
        *reinterpret_cast<h16x4*>(dx + (long)c * M + mm) = o;
      }
    }
  }
};

// ---------------------------------------------------------------------------
// The backward's tail in one kernel (C = I = 128):
//
//   P   = xn . Wcat[:, :4I]                    (recompute, K = C)
//   d(cat)[:, :4I] from P, d(left|right), mask (the EpiTrimulProjBwd formulas)
//   dy  = d(cat) . Wcat^T                      (K = 4I + C; the last C columns
//                                               of d(cat) come from memory)
//   din = dout + LN'(dy)                       (the input LayerNorm's backward)
//
// d(cat)'s [proj|gate] columns never leave registers: GEMM1 runs transposed
// (the weights as the first MFMA operand), so a lane ends with row m = l%16 and
// 4 consecutive columns 4g..4g+3 of a 16-column block.  The proj block and its
// gate block (16 columns to the right) land in the same lane positions, so the
// epilogue pairs them in registers, and the 8 values {proj 4g..4g+3, gate
// 4g..4g+3} of a 32-column block are exactly one k-slot set of a 32-deep MFMA
// step of GEMM2 -- the same slot order that its weights are read in.  GEMM2
// also runs transposed, so each lane holds 32 channels (16j + 4g + r) of its
// row for the LayerNorm's row sums (completed across the 4 lanes of the row).
//
// Workgroup: 128 rows, 4 waves of 32 rows (two 16-row tiles).  The weights
// stream through LDS in 10 chunks (8 of 64 GEMM1 columns, with the matching
// 64 rows of GEMM2's K, and 2 chunks of the gating_linear K), double-buffered
// with a register prefetch of the next chunk.
namespace tail {
constexpr int C = 128, I = 128, NC = 4 * I + C;
constexpr int RT = 2;                     // 16-row tiles per wave
constexpr int BM = 64 * RT;               // rows per workgroup (4 waves)
constexpr int CH = 64;                    // GEMM1 columns (= GEMM2 k) per chunk
constexpr int NPG = 4 * I / CH;           // [proj|gate] chunks
constexpr int NCHUNK = NPG + C / CH;      // + gating_linear chunks
// row strides = 8 (mod 64) dwords: the 16-byte fragment reads of 16 rows are
// bank-conflict free
constexpr int LD1 = C + 16;               // B1 chunk: [CH][C] (n rows, k contiguous)
constexpr int LD2 = CH + 16;              // B2 chunk: [C][CH] (c rows, k contiguous)
constexpr int B1E = CH * LD1, B2E = C * LD2;
}  // namespace tail

// 8 h16 of row `row` at k = k0 + {4g..4g+3, 16+4g..16+4g+3} of a
// K-contiguous tile (row stride ld), global or LDS.
__device__ __forceinline__ h16x8 kslots(const h16* T, long ld, long row, int k0, int g) {
  const h16* p = T + row * ld + k0 + 4 * g;
  const h16x4 a = *reinterpret_cast<const h16x4*>(p);
  const h16x4 b = *reinterpret_cast<const h16x4*>(p + 16);
  h16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// The weights' k order in the tail kernel's copies: within each 32-block,
// physical position 8g + e holds logical k = 4g + e (e < 4) and 8g + 4 + e
// holds 16 + 4g + e, so kslots' 8 values are 16 contiguous bytes.
inline int tail_kperm(int p) {
  const int b = p & ~31, g = (p & 31) >> 3, e = p & 7;
  return b + (e < 4 ? 4 * g + e : 16 + 4 * g + e - 4);
}

struct TailArgs {
  const h16* xn;      // [M][C]
  const h16* wcat_t;  // [NC][C], k permuted (tail_kperm)
  const h16* wcat;    // [C][NC], k permuted (tail_kperm)
  const h16 *dl, *dr; // [I][M]
  const h16* dcg;     // [M][C]: d(cat)'s gating_linear columns
  const float *bp, *bg, *mask;
  const float *x, *ln_g, *mean, *rstd, *dres;
  const float* gmul;  // inverse cotangent scale (device scalar)
  float* out;
  long M;
};

__global__ __launch_bounds__(256, 2) void trimul_tail_kernel(TailArgs a) {
  using namespace tail;
  __shared__ __attribute__((aligned(16))) h16 B1s[2 * B1E];
  __shared__ __attribute__((aligned(16))) h16 B2s[2 * B2E];
  // the projection biases, read in the d(cat) formulas from LDS: a global
  // load there would wait (in-order vmcnt) for the next chunk's prefetch
  __shared__ __attribute__((aligned(16))) float Bps[2 * I], Bgs[2 * I];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const long m0 = (long)blockIdx.x * BM + wave * 16 * RT;
  const long M = a.M;

  // ---- chunk staging: 16 KB of B1 and 16 KB of B2 per chunk, 4 + 4 16-byte pieces a thread
  // Chunk s's operands are fetched during chunk s - 1: its weights into
  // p1/p2 (stored to LDS at the end of chunk s - 1), and the lane's own
  // operands into registers -- d(left|right) at its rows and channels (da) for
  // a [proj|gate] chunk, its d(cat) gating fragments (in p1) for the others.
  // The weights are issued first, so waiting for them leaves the rest in flight.
  h16x8 p1[4], p2[4];
  h16 da[RT][2][4];
  auto prefetch = [&](int s) {
    if (s < NPG) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = tid + 256 * q, r = c / (C / 8), k8 = (c % (C / 8)) * 8;
        p1[q] = ld8(a.wcat_t + (long)(s * CH + r) * C + k8);
      }
    }
    const int kb = s < NPG ? s * CH : 4 * I + (s - NPG) * CH;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q, r = c / (CH / 8), k8 = (c % (CH / 8)) * 8;
      p2[q] = ld8(a.wcat + (long)r * NC + kb + k8);
    }
    if (s < NPG) {
      const h16* dsrc = s < NPG / 2 ? a.dl : a.dr;
      const int chb = (s % (NPG / 2)) * 32;  // channel within left or right
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            da[i][q][r] = dsrc[(long)(chb + q * 16 + 4 * g + r) * M + m0 + i * 16 + l16];
    } else {
      const int kc = (s - NPG) * CH;
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int q = 0; q < 2; ++q) p1[2 * i + q] = kslots(a.dcg, C, m0 + i * 16 + l16, kc + q * 32, g);
    }
  };
  auto stash = [&](int s, int buf) {
    if (s < NPG) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int c = tid + 256 * q, r = c / (C / 8), k8 = (c % (C / 8)) * 8;
        st8(B1s + buf * B1E + r * LD1 + k8, p1[q]);
      }
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = tid + 256 * q, r = c / (CH / 8), k8 = (c % (CH / 8)) * 8;
      st8(B2s + buf * B2E + r * LD2 + k8, p2[q]);
    }
  };

  prefetch(0);
  // xn fragments of the wave's two row tiles, all of K, in GEMM1's slot order
  h16x8 xf[RT][C / 32];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int ks = 0; ks < C / 32; ++ks) xf[i][ks] = kslots(a.xn, C, m0 + i * 16 + l16, ks * 32, g);
  float mk[RT];
#pragma unroll
  for (int i = 0; i < RT; ++i) mk[i] = a.mask[m0 + i * 16 + l16];
  if (tid < 2 * I) {
    Bps[tid] = a.bp[tid];
    Bgs[tid] = a.bg[tid];
  }
  stash(0, 0);
  __syncthreads();

  float4 xpre[RT][C / 16];
  f32x4 acc2[RT][C / 16];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int j = 0; j < C / 16; ++j) acc2[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  // fully unrolled: every chunk's registers are fixed at compile time, so the
  // prefetched operands stay in flight until their use (no loop-carried copies)
#pragma unroll
  for (int s = 0; s < NCHUNK; ++s) {
    const int buf = s & 1;
    const h16* b1 = B1s + buf * B1E;
    const h16* b2 = B2s + buf * B2E;
    h16x8 af[RT][2];  // GEMM2 A fragments: [row tile][k-step of this chunk]
    if (s < NPG) {
      // GEMM1: P for 4 column blocks (proj, gate, proj, gate)
      f32x4 acc1[RT][4];
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int t = 0; t < 4; ++t) acc1[i][t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < C / 32; ++ks) {
        h16x8 bfr[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) bfr[t] = ld8(b1 + (t * 16 + l16) * LD1 + ks * 32 + 8 * g);
#pragma unroll
        for (int i = 0; i < RT; ++i)
#pragma unroll
          for (int t = 0; t < 4; ++t)
            acc1[i][t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bfr[t], xf[i][ks], acc1[i][t], 0, 0, 0);
      }
      // epilogue: d(proj) = a * sigmoid(gate), d(gate) = a * proj * s (1 - s), a = d(act) * mask
#pragma unroll
      for (int q = 0; q < 2; ++q) {
        const int ch = s * 32 + q * 16 + 4 * g;  // channel of slot r = ch + r (0..2I)
        float bpv[4], bgv[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) { bpv[r] = Bps[ch + r]; bgv[r] = Bgs[ch + r]; }
#pragma unroll
        for (int i = 0; i < RT; ++i) {
          h16x8 f;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float pv = acc1[i][2 * q][r] + bpv[r];
            const float sg = sigmoidf_(acc1[i][2 * q + 1][r] + bgv[r]);
            const float ad = (float)da[i][q][r] * mk[i];
            f[r] = f2h_sat(ad * sg);
            f[4 + r] = f2h_sat(ad * pv * sg * (1.f - sg));
          }
          af[i][q] = f;
        }
      }
    } else {
      // gating_linear columns of d(cat), fetched during the previous chunk
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int q = 0; q < 2; ++q) af[i][q] = p1[2 * i + q];
    }
    // the next chunk's operands load behind GEMM2 (the weights are
    // L2-resident: every workgroup reads the same 288 KB)
    if (s + 1 < NCHUNK) prefetch(s + 1);
    if (s == NPG) {
      // the LayerNorm tail's x rows, loaded behind the last two chunks (GEMM1
      // is done, so its operand registers are free)
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int j = 0; j < C / 16; ++j)
          xpre[i][j] = *reinterpret_cast<const float4*>(a.x + (m0 + i * 16 + l16) * C + 16 * j + 4 * g);
    }
    // GEMM2: dy[m][c] += d(cat)[m][k] Wcat[c][k] over the chunk's 64 k
#pragma unroll
    for (int q = 0; q < 2; ++q) {
#pragma unroll
      for (int j = 0; j < C / 16; ++j) {
        const h16x8 bfr = ld8(b2 + (j * 16 + l16) * LD2 + q * 32 + 8 * g);
#pragma unroll
        for (int i = 0; i < RT; ++i)
          acc2[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bfr, af[i][q], acc2[i][j], 0, 0, 0);
      }
    }
    if (s + 1 < NCHUNK) stash(s + 1, buf ^ 1);
    __syncthreads();
  }

  // ---- LayerNorm backward + residual: lane has channels 16j + 4g + r of row m
  const float gs = *a.gmul;
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const long m = m0 + i * 16 + l16;
    const float mu = a.mean[m], rs = a.rstd[m];
    float xh[C / 16][4], gg[C / 16][4];
    float sg = 0.f, sgx = 0.f;
#pragma unroll
    for (int j = 0; j < C / 16; ++j) {
      const int c = 16 * j + 4 * g;
      const float4 xv = xpre[i][j];
      const float4 gm = *reinterpret_cast<const float4*>(a.ln_g + c);
      const float xa[4] = {xv.x, xv.y, xv.z, xv.w}, ga[4] = {gm.x, gm.y, gm.z, gm.w};
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        xh[j][r] = (xa[r] - mu) * rs;
        gg[j][r] = acc2[i][j][r] * (ga[r] * gs);
        sg += gg[j][r];
        sgx += gg[j][r] * xh[j][r];
      }
    }
    sg += __shfl_xor(sg, 16, 64);
    sg += __shfl_xor(sg, 32, 64);
    sgx += __shfl_xor(sgx, 16, 64);
    sgx += __shfl_xor(sgx, 32, 64);
    sg *= 1.f / C;
    sgx *= 1.f / C;
#pragma unroll
    for (int j = 0; j < C / 16; ++j) {
      const int c = 16 * j + 4 * g;
      const float4 d = *reinterpret_cast<const float4*>(a.dres + m * C + c);
      float4 o;
      o.x = d.x + rs * (gg[j][0] - sg - xh[j][0] * sgx);
      o.y = d.y + rs * (gg[j][1] - sg - xh[j][1] * sgx);
      o.z = d.z + rs * (gg[j][2] - sg - xh[j][2] * sgx);
      o.w = d.w + rs * (gg[j][3] - sg - xh[j][3] * sgx);
      *reinterpret_cast<float4*>(a.out + m * C + c) = o;
    }
  }
}

}  // namespace

TriMulW trimul_weights(WeightStore& ws, const std::string& P) {
  TriMulW w;
  const HostTensor& pw = ws.host(P + "projection/weights");  // [C, 2I]
  w.C = pw.shape[0];
  w.I = pw.shape[1] / 2;
  const int C = w.C, I = w.I, NC = 4 * I + C;
  if (I % 16 != 0 || C % 64 != 0) throw std::runtime_error("trimul: widths must be multiples of 16/64");
  w.ln_g = ws.f32(P + "left_norm_input/scale");
  w.ln_b = ws.f32(P + "left_norm_input/offset");
  w.cn_g = ws.f32(P + "center_norm/scale");
  w.cn_b = ws.f32(P + "center_norm/offset");
  w.bp = ws.f32(P + "projection/bias");
  w.bg = ws.f32(P + "gate/bias");
  w.bgl = ws.f32(P + "gating_linear/bias");
  w.bo = ws.f32(P + "output_projection/bias");
  // Wcat [C][NC] in GEMM column order
  auto cat = [&]() {
    const HostTensor& gw = ws.host(P + "gate/weights");
    const HostTensor& lw = ws.host(P + "gating_linear/weights");
    std::vector<float> c((size_t)C * NC);
    for (int r = 0; r < C; ++r) {
      for (int ch = 0; ch < 2 * I; ++ch) {
        c[(size_t)r * NC + col_proj(ch)] = pw.data[(size_t)r * 2 * I + ch];
        c[(size_t)r * NC + col_gate(ch)] = gw.data[(size_t)r * 2 * I + ch];
      }
      for (int j = 0; j < C; ++j) c[(size_t)r * NC + 4 * I + j] = lw.data[(size_t)r * C + j];
    }
    return c;
  };
  w.wcat = ws.derived<h16>("trimul.wcat:" + P, [&] { return to_h16(cat()); });
  w.wcat_t = ws.derived<h16>("trimul.wcat_t:" + P, [&] {
    std::vector<float> c = cat();
    return transpose_h16(c.data(), C, NC);
  });
  if (C == 128 && NC % 128 == 0) {
    w.wcat_frag = ws.derived<h16>("trimul.wcat_frag:" + P, [&] {
      const std::vector<float> c = cat();  // [C][NC]
      return b_frags_k128(NC, [&](int n, int k) { return c[(size_t)k * NC + n]; });
    });
  }
  auto kperm_cols = [](std::vector<h16> m, int rows, int cols) {
    std::vector<h16> o(m.size());
    for (int r = 0; r < rows; ++r)
      for (int p = 0; p < cols; ++p) o[(size_t)r * cols + p] = m[(size_t)r * cols + tail_kperm(p)];
    return o;
  };
  w.wcat_k = ws.derived<h16>("trimul.wcat_k:" + P, [&] { return kperm_cols(to_h16(cat()), C, NC); });
  w.wcat_tk = ws.derived<h16>("trimul.wcat_tk:" + P, [&] {
    std::vector<float> c = cat();
    return kperm_cols(transpose_h16(c.data(), C, NC), NC, C);
  });
  const HostTensor& ow = ws.host(P + "output_projection/weights");  // [I, C]
  w.wo = ws.derived<h16>("trimul.wo:" + P, [&] { return to_h16(ow.data); });
  w.wo_t = ws.derived<h16>("trimul.wo_t:" + P, [&] { return transpose_h16(ow.data.data(), I, C); });
  if (C == 128 && I == 128) {
    w.wo_frag = ws.derived<h16>("trimul.wo_frag:" + P, [&] {
      return b_frags_k128(C, [&](int n, int k) { return ow.data[(size_t)k * C + n]; });
    });
  }
  return w;
}

size_t trimul_save_bytes(int N, int C, int I) {
  Sizer s;
  TriMulSave<Sizer> plan(s, N, C, I);
  (void)plan;
  return s.off;
}

static void trimul_check(int N) {
  if (N <= 0 || N % 32 != 0) throw std::runtime_error("trimul: N must be a positive multiple of 32");
}

// One batched contraction (operands described by `g`, one channel plane per
// batch entry): the dedicated kernel for N <= 256, the tiled GEMM beyond, in
// 128 x 128 tiles (64 x 64 tiles read every operand row of a plane from 8
// tiles: 1 GB of L2 traffic per contraction at N = 512).
template <class OutT>
static void contract(hipStream_t st, const GemmArgs& g, OutT* C, const char* name) {
  {
    KTimed kt(name, st);
    float* cf = nullptr;
    h16* cb = nullptr;
    if constexpr (sizeof(OutT) == 4) cf = C;
    else cb = C;
    if (trimul_contract(st, g.M, g.batch, g.A, g.a_sk == 1, g.B, g.b_sk == 1, cf, cb)) return;
  }
  gemm<128, 128>(st, g, EpiStore<OutT>{C, g.N, (long)g.M * g.N, nullptr, g.N}, name);
}

// Contraction operand layouts for one channel plane (row-major N x N).
static void contraction_fwd(hipStream_t st, bool outgoing, int N, int I, const h16* L,
                            const h16* R, float* T) {
  const long M = (long)N * N;
  GemmArgs g;
  g.M = N; g.N = N; g.K = N; g.batch = I;
  if (outgoing) {  // T[i][j] = sum_k L[i][k] R[j][k]
    g.A = L; g.a_sm = N; g.a_sk = 1;
    g.B = R; g.b_sn = N; g.b_sk = 1;
  } else {         // T[i][j] = sum_k R[k][i] L[k][j]
    g.A = R; g.a_sm = 1; g.a_sk = N;
    g.B = L; g.b_sn = 1; g.b_sk = N;
  }
  g.a_sb = M; g.b_sb = M;
  contract<float>(st, g, T, BC2N_TN(I, "trimul.contract_fwd"));
}

void trimul_fwd(hipStream_t st, const TriMulW& w, bool outgoing, int N, const float* pair_in,
                const float* mask, const float* tbl, float* pair_out, void* save) {
  trimul_check(N);
  nonnull(pair_in, "trimul pair_in"); nonnull(mask, "trimul mask");
  nonnull(pair_out, "trimul pair_out"); nonnull(save, "trimul save");
  const int C = w.C, I = w.I, NC = 4 * I + C;
  const long M = (long)N * N;
  Carver cv(save);
  TriMulSave<Carver> sv(cv, N, C, I);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)M * I * 2 + 1024);
  h16* xn = sv.xn;
  h16* tn = ar.take_n<h16>((size_t)M * I);
  const EpiTrimulProj proj{sv.left, sv.right, sv.gout, w.bp, w.bg, w.bgl, mask, M, I, C};
  if (w.wcat_frag) {
    lnproj::Args la{};
    la.M = M; la.nt = 0; la.bn = N; la.nout = NC;
    la.x = pair_in; la.g = w.ln_g; la.b = w.ln_b;
    la.xn = xn; la.mean = sv.mean; la.rstd = sv.rstd; la.W = w.wcat_frag;
    KTimed kt(BC2N_TN(C, "trimul.ln_proj"), st);
    lnproj::launch<0, true>(st, la, proj);
  } else {
    {
      KTimed kt(BC2N_TN(C, "trimul.ln_fwd"), st);
      ln_fwd_f32(st, pair_in, M, C, 0, w.ln_g, w.ln_b, xn, sv.mean, sv.rstd, true, 0, nullptr,
                 nullptr);
    }
    GemmArgs g1;
    g1.M = (int)M; g1.N = NC; g1.K = C;
    g1.A = xn; g1.a_sm = C; g1.a_sk = 1;
    g1.B = w.wcat_t; g1.b_sn = C; g1.b_sk = 1;
    gemm<128, 128>(st, g1, proj, BC2N_TN(C, "trimul.gemm_proj"));
  }
  contraction_fwd(st, outgoing, N, I, sv.left, sv.right, sv.T);
  const EpiTrimulOut out(pair_in, pair_out, w.bo, sv.gout, sv.osave, tbl, N, C);
  if (w.wo_frag && I == lnproj::C) {
    // the centre norm and the output projection in one kernel: the normalised
    // rows stay on chip (the same statistics and binary16 rows as ln_fwd_cm)
    lnproj::Args la{};
    la.M = M; la.nout = C; la.x = sv.T; la.g = w.cn_g; la.b = w.cn_b;
    la.mean = sv.cmean; la.rstd = sv.crstd; la.W = w.wo_frag;
    KTimed kt(BC2N_TN(C, "trimul.ln_out"), st);
    lnproj::launch_cm<true>(st, la, out);
    return;
  }
  {
    KTimed kt(BC2N_TN(C, "trimul.ln_center"), st);
    ln_fwd_cm(st, sv.T, M, I, w.cn_g, w.cn_b, tn, sv.cmean, sv.crstd, true);
  }
  if (w.wo_frag) {
    lnproj::Args la{};
    la.M = M; la.nout = C; la.xn = tn; la.W = w.wo_frag;
    KTimed kt(BC2N_TN(C, "trimul.gemm_out"), st);
    lnproj::launch_rows(st, la, out);
    return;
  }
  GemmArgs g2;
  g2.M = (int)M; g2.N = C; g2.K = I;
  g2.A = tn; g2.a_sm = I; g2.a_sk = 1;
  g2.B = w.wo_t; g2.b_sn = I; g2.b_sk = 1;
  gemm<128, 128>(st, g2, out, BC2N_TN(C, "trimul.gemm_out"));
}

void trimul_bwd(hipStream_t st, const TriMulW& w, bool outgoing, int N, const float* pair_in,
                const float* mask, const float* tbl, const void* save, const float* dout,
                float* din, const float* sc) {
  trimul_check(N);
  nonnull(pair_in, "trimul pair_in"); nonnull(mask, "trimul mask"); nonnull(save, "trimul save");
  nonnull(dout, "trimul dout"); nonnull(din, "trimul din");
  const int C = w.C, I = w.I, NC = 4 * I + C;
  const long M = (long)N * N;
  Carver cv(const_cast<void*>(save));
  TriMulSave<Carver> sv(cv, N, C, I);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  sc = module_scale(st, sc, dout, M * C);
  // C = I = 128: the tail kernel keeps d(cat)'s [proj|gate] columns in
  // registers; only its gating_linear columns ([M][C]) go through memory
  const bool fused = (C == tail::C && I == tail::I && M % tail::BM == 0);
  const int ldcat = fused ? C : NC, off = fused ? 0 : 4 * I;
  Sizer need;
  need.take<h16>((size_t)M * ldcat);  // dcat
  need.take<float>((size_t)M * I);  // dTn
  need.take<h16>((size_t)M * I);   // dT
  need.take<h16>((size_t)M * I);   // dL
  need.take<h16>((size_t)M * I);   // dR
  if (!fused) need.take<float>((size_t)M * C);  // dxn
  ar.reset(st, need.off);
  h16* dcat = ar.take_n<h16>((size_t)M * ldcat);
  float* dtn = ar.take_n<float>((size_t)M * I);
  h16* dT = ar.take_n<h16>((size_t)M * I);
  h16* dL = ar.take_n<h16>((size_t)M * I);
  h16* dR = ar.take_n<h16>((size_t)M * I);
  float* dxn = fused ? nullptr : ar.take_n<float>((size_t)M * C);

  // d(tn) = (tbl*dout*g_out) . Wo^T, the operand built as the GEMM loads it;
  // the loader also writes the gating_linear columns of dcat
  GemmArgs g1;
  g1.M = (int)M; g1.N = I; g1.K = C;
  g1.a_sm = C; g1.a_sk = 1;
  g1.B = w.wo; g1.b_sn = C; g1.b_sk = 1;
  // 64-row tiles: with N = K = 128 a 128-row grid leaves most workgroup
  // slots empty (392 workgroups at 224 tokens); the 128 x 128 B operand is
  // cheap to re-read
  const ALoadTrimulOut aload{dout, tbl, sv.gout, sv.osave, dcat, C, ldcat, off, N, sc};
  if (I == EpiCmLnBwd::C && M % 4 == 0) {
    // the centre norm's backward in the epilogue: dT straight from d(tn)
    EpiCmLnBwd ep;
    ep.x = sv.T; ep.gamma = w.cn_g; ep.mean = sv.cmean; ep.rstd = sv.crstd; ep.dx = dT; ep.M = M;
    gemm<64, 128>(st, g1, ep, BC2N_TN(C, "trimul.gemm_dout_ln"), aload);
  } else {
    gemm<64, 128>(st, g1, EpiStore<float>{dtn, I, 0, nullptr, I}, BC2N_TN(C, "trimul.gemm_dout"),
                  aload);
    KTimed kt(BC2N_TN(C, "trimul.ln_center_bwd"), st);
    ln_bwd_cm(st, dtn, sv.T, M, I, w.cn_g, sv.cmean, sv.crstd, dT);
  }
  {
    GemmArgs a, b;
    a.M = N; a.N = N; a.K = N; a.batch = I; a.a_sb = M; a.b_sb = M;
    b = a;
    if (outgoing) {
      // dL[i][k] = sum_j dT[i][j] R[j][k]
      a.A = dT; a.a_sm = N; a.a_sk = 1;
      a.B = sv.right; a.b_sn = 1; a.b_sk = N;
      // dR[j][k] = sum_i dT[i][j] L[i][k]
      b.A = dT; b.a_sm = 1; b.a_sk = N;
      b.B = sv.left; b.b_sn = 1; b.b_sk = N;
    } else {
      // dL[k][j] = sum_i R[k][i] dT[i][j]
      a.A = sv.right; a.a_sm = N; a.a_sk = 1;
      a.B = dT; a.b_sn = 1; a.b_sk = N;
      // dR[k][i] = sum_j L[k][j] dT[i][j]
      b.A = sv.left; b.a_sm = N; b.a_sk = 1;
      b.B = dT; b.b_sn = N; b.b_sk = 1;
    }
    contract<h16>(st, a, dL, BC2N_TN(C, "trimul.contract_bwd"));
    contract<h16>(st, b, dR, BC2N_TN(C, "trimul.contract_bwd"));
  }
  if (fused) {
    TailArgs t;
    t.xn = sv.xn; t.wcat_t = w.wcat_tk; t.wcat = w.wcat_k;
    t.dl = dL; t.dr = dR; t.dcg = dcat;
    t.bp = w.bp; t.bg = w.bg; t.mask = mask;
    t.x = pair_in; t.ln_g = w.ln_g; t.mean = sv.mean; t.rstd = sv.rstd; t.dres = dout;
    t.gmul = sc + 1;
    t.out = din; t.M = M;
    KTimed kt(BC2N_TN(C, "trimul.tail_bwd"), st);
    hipLaunchKernelGGL(trimul_tail_kernel, dim3((unsigned)(M / tail::BM)), dim3(256), 0, st, t);
    return;
  }
  {
    GemmArgs g;
    g.M = (int)M; g.N = 4 * I; g.K = C;
    g.A = sv.xn; g.a_sm = C; g.a_sk = 1;
    g.B = w.wcat_t; g.b_sn = C; g.b_sk = 1;
    gemm<128, 128>(st, g, EpiTrimulProjBwd{dL, dR, w.bp, w.bg, mask, dcat, M, I, NC},
                   BC2N_TN(C, "trimul.proj_bwd"));
  }
  GemmArgs g2;
  g2.M = (int)M; g2.N = C; g2.K = NC;
  g2.A = dcat; g2.a_sm = NC; g2.a_sk = 1;
  g2.B = w.wcat; g2.b_sn = NC; g2.b_sk = 1;
  if (C == 128) {
    // the input LayerNorm's backward and the residual add in the epilogue
    gemm<128, 128>(st, g2,
                   EpiLnBwd<0>(pair_in, w.ln_g, sv.mean, sv.rstd, dout, din, M, 0, nullptr,
                               nullptr, sc + 1),
                   BC2N_TN(C, "trimul.gemm_dx_ln"));
    return;
  }
  gemm<128, 128>(st, g2, EpiStore<float>{dxn, C, 0, nullptr, C}, BC2N_TN(C, "trimul.gemm_dx"));
  KTimed kt(BC2N_TN(C, "trimul.ln_bwd"), st);
  ln_bwd_f32(st, dxn, pair_in, M, C, 0, w.ln_g, sv.mean, sv.rstd, din, true, 0, nullptr, nullptr,
             dout, sc + 1);
}

}  // namespace bc2n
