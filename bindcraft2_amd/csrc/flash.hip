// Flash attention forward/backward for AF2's gated attention with pair bias,
// written for wave64 and gfx950 MFMA, head width D = 32 (Evoformer) or 16
// (template stack), N <= 256 keys per row.
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
// The contraction over the head width uses v_mfma_f32_16x16x32_f16 (D=32)
// or v_mfma_f32_16x16x16_f16 (D=16); the contraction over 32 keys (or 32
// queries) always uses the x32 form.  For that second product the 8 K-slots
// of lane group g=l/16 are mapped to positions {4g..4g+3, 16+4g..16+4g+3}
// of the 32-block, for both operands; the first product's result already
// sits in exactly that order.  All operands live in LDS row-major (token x
// head width); the second product's transposed operand (V^T, K^T, Q^T, dO^T)
// is read with ds_read_b64_tr_b16, which hands each lane a column of a 4 x 16
// block, so nothing is ever staged transposed.
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
// fully masked row is exact to h16 precision.
//
// The bias gradient (a sum over rows) is accumulated in registers over a
// chunk of rows and written once per chunk; a second pass adds the chunks in
// a fixed order, so the result is deterministic (no float atomics anywhere).
#include <algorithm>
#include <type_traits>

#include "kernels.h"
#include "runtime.h"

namespace bc2n {

constexpr float NEG_LOGIT = -8192.0f;

// Row stride (in h16) of the LDS token x head-width tiles.  gfx950's LDS
// serves a wave's 8-byte transposed read in two 32-lane halves of 256 bytes
// and a 16-byte row read in four; with D = 32 a 96-byte stride puts every
// half-wave's rows on distinct banks for both patterns (80 bytes costs two
// cycles of conflicts per read, measured with SQ_LDS_BANK_CONFLICT).
template <int D>
__host__ __device__ constexpr int lds_ld() { return D == 32 ? 48 : D + 8; }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// Column read of a row-major h16 LDS tile T[row][ld] (ld % 4 == 0):
// returns, for lane l (column c = l%16, group g = l/16), the four values
// T[r0 + 4g + j][c0 + c], j = 0..3.  One ds_read_b64_tr_b16: within each
// 16-lane group, lane m addresses the 8-byte chunk T[r0 + 4g + m/4][c0 + 4(m%4)
// .. +3] and the instruction returns to lane 4a + c element c of the chunks
// of lanes a, a+4, a+8, a+12.
__device__ __forceinline__ h16x4 ld_tr4(const h16* T, int ld, int r0, int c0, int lane) {
  const int g = lane >> 4, m = lane & 15;
  const h16* p = T + (r0 + 4 * g + (m >> 2)) * ld + c0 + 4 * (m & 3);
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p);
  return __builtin_bit_cast(h16x4, v);
}

// x32 operand over a 32-block at row r0 (slots {4g..4g+3, 16+4g..16+4g+3}),
// column c0 + l%16 of a row-major LDS tile.
__device__ __forceinline__ h16x8 ld_tr8(const h16* T, int ld, int r0, int c0, int lane) {
  const h16x4 a = ld_tr4(T, ld, r0, c0, lane);
  const h16x4 b = ld_tr4(T, ld, r0 + 16, c0, lane);
  h16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// Row-major copies of the first `rows` (<= N) rows of two head slices (row
// strides lda, ldb) into LDS tiles [N][lds_ld<D>()], by 256 threads: every 16-byte
// load is issued before the first store, so one memory latency covers the
// whole tile.  The loads and the LDS stores are separate steps, so a kernel
// walking several rows can hold the next row's tiles in registers while it
// computes.
template <int D, int N, int T = 256>
struct RowPair {
  static constexpr int CPR = D / 8;  // 16-byte chunks per row
  static constexpr int IT = (N * CPR + T - 1) / T;
  h16x8 va[IT], vb[IT];
  __device__ __forceinline__ void load(const h16* sA, long lda, const h16* sB, long ldb, int tid,
                                       int rows) {
    const int items = rows * CPR;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + T * i;
      if (c < items) {
        va[i] = ld8(sA + (long)(c / CPR) * lda + (c % CPR) * 8);
        vb[i] = ld8(sB + (long)(c / CPR) * ldb + (c % CPR) * 8);
      }
    }
  }
  __device__ __forceinline__ void store(h16* dA, h16* dB, int tid, int rows) const {
    const int items = rows * CPR;
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int c = tid + T * i;
      if (c < items) {
        st8(&dA[(c / CPR) * lds_ld<D>() + (c % CPR) * 8], va[i]);
        st8(&dB[(c / CPR) * lds_ld<D>() + (c % CPR) * 8], vb[i]);
      }
    }
  }
};

template <int D, int N, int T = 256>
__device__ __forceinline__ void stage_rows2(h16* dA, const h16* sA, long lda, h16* dB,
                                            const h16* sB, long ldb, int tid, int rows = N) {
  RowPair<D, N, T> p;
  p.load(sA, lda, sB, ldb, tid, rows);
  p.store(dA, dB, tid, rows);
}

// Operand fragment of the head-width contraction for lane group g.
template <int D>
struct HFrag;
template <>
struct HFrag<32> {
  h16x8 v;
  __device__ __forceinline__ void load(const h16* row, int g) { v = ld8(row + 8 * g); }
  __device__ __forceinline__ static f32x4 mma(const HFrag& a, const HFrag& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a.v, b.v, c, 0, 0, 0);
  }
};
template <>
struct HFrag<16> {
  h16x4 v;
  __device__ __forceinline__ void load(const h16* row, int g) {
    v = *reinterpret_cast<const h16x4*>(row + 4 * g);
  }
  __device__ __forceinline__ static f32x4 mma(const HFrag& a, const HFrag& b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(a.v, b.v, c, 0, 0, 0);
  }
};

// Logical (row, head, query block) of workgroup `bid` of the per-row
// forward and dQ kernels (N > 256), ordered head pair, tile of 8 rows, query
// block, head in the pair, row in the tile.  The neighbours one XCD runs
// together then share 8 rows' K and V and the pair's pair bias in that XCD's
// L2; the two heads of a pair share every 128-byte line of a token's q, k, v
// and gate slices (64 bytes a head), so each line is fetched once.  (In
// (row, head, query block) order no two workgroups in flight shared a bias
// tile; in head-major order each line was fetched once per head, a head's
// whole pass apart.)
struct RowHeadQb {
  int r, h, qb;
};
__device__ __forceinline__ RowHeadQb row_tile_order(int bid, int R, int H, int nqb) {
  constexpr int T = 8;
  const int per_head = R * nqb;
  const int h0 = 2 * (bid / (2 * per_head));  // first head of the pair
  const int nh = min(2, H - h0);              // heads in the pair (1 for an odd last head)
  int j = bid - h0 * per_head;                // index among the pair's nh * R * nqb
  const int full = (R / T) * T;               // rows in whole tiles
  RowHeadQb o;
  if (j < full * nqb * nh) {
    const int t = j / (T * nqb * nh), w = j - t * (T * nqb * nh);
    o.qb = w / (T * nh);
    const int u = w - o.qb * (T * nh);
    o.h = h0 + u / T;
    o.r = t * T + u % T;
  } else {  // the last R % T rows
    j -= full * nqb * nh;
    const int rem = R - full;
    o.qb = j / (rem * nh);
    const int u = j - o.qb * (rem * nh);
    o.h = h0 + u / rem;
    o.r = full + u % rem;
  }
  return o;
}

// ------------------------------------------------------------------ forward
// Workgroup = (row r, head h, 64 queries); 4 waves x 16 queries; N = 32*NKB
// > 256.  Keys are processed in chunks of 128 (4 blocks of 32) staged in one
// LDS buffer; the next chunk's K and V are loaded into registers while the
// current one computes, so the buffer is small (five workgroups fit a CU)
// and the register budget leaves four waves per SIMD.  A lane keeps its
// query's 32 scores of the chunk (8 keys of every block) in registers.
// Per score: the pair bias is the score MFMA's accumulator, then one fma
// (the key mask), half a max, a subtract, the exponent and half a convert;
// the row sum of the probabilities comes from the P V product itself (one
// more MFMA per block with an all-ones operand), summed over the same h16
// probabilities the numerator uses.  Online softmax across chunks: the
// output accumulator and the row sum are rescaled once per chunk.
template <int D, int NKB, int QW>
__global__ __launch_bounds__(64 * QW) void attn_fwd_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  constexpr int DT = D / 16;
  constexpr int LD = lds_ld<D>();
  constexpr int N = 32 * NKB;  // == a.N (dispatch)
  constexpr int CB = 4;        // key blocks per chunk
  constexpr int CN = 32 * CB;  // keys per chunk
  constexpr int NFULL = NKB / CB, TAIL = NKB % CB;
  constexpr int NCH = NFULL + (TAIL ? 1 : 0);
  const int H = a.H;
  h16* Ks = reinterpret_cast<h16*>(smem_raw);          // [CN][LD]
  h16* Vs = Ks + CN * LD;                               // [CN][LD]
  float* Mm = reinterpret_cast<float*>(Vs + CN * LD);    // [N] 1 / 0 per key
  float* Ma = Mm + N;                                    // [N] 0 / NEG_LOGIT
  constexpr int T = 64 * QW;   // threads; QW waves of 16 queries

  const int nqb = (N + 16 * QW - 1) / (16 * QW);
  const long G = (long)a.R * H * nqb;
  const int bid = (int)xcd_block(G);
  if (bid >= G) return;
  const RowHeadQb ord = row_tile_order(bid, a.R, H, nqb);
  const int qb = ord.qb, h = ord.h, r = ord.r;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const long tok0 = (long)r * N;
  const h16* Kg = a.qkvg + tok0 * a.ld + H * D + h * D;
  const h16* Vg = a.qkvg + tok0 * a.ld + 2 * H * D + h * D;
  RowPair<D, CN, T> nkv;  // the next chunk's K and V rows
  nkv.load(Kg, a.ld, Vg, a.ld, tid, min(CN, N));
  for (int k = tid; k < N; k += T) {
    const bool on = a.mask[r * a.mask_sr + k * a.mask_sk] != 0.f;
    Mm[k] = on ? 1.f : 0.f;
    Ma[k] = on ? 0.f : NEG_LOGIT;
  }

  const int q0 = qb * 16 * QW + wave * 16;
  const bool active = q0 < N;  // idle waves keep to the barriers only
  const int lq = lane & 15, g = lane >> 4;
  const int q = min(q0, N - 16) + lq;  // idle waves read in bounds, store nothing
  HFrag<D> qf;
  qf.load(a.qkvg + (tok0 + q) * a.ld + h * D, g);
  const h16* grow = a.qkvg + (tok0 + q) * a.ld + 3 * H * D + h * D;
  h16x4 gv[DT];
#pragma unroll
  for (int dh = 0; dh < DT; ++dh) gv[dh] = *reinterpret_cast<const h16x4*>(grow + dh * 16 + 4 * g);
  const int qt = q >> 4;  // the wave's 16-query tile (bias blocks; the launcher requires the bias)
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  h16x8 ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (h16)1.f;
  float mx = -INFINITY;  // running maximum (exp2(-inf - m) = 0 rescales nothing)
  f32x4 acc[DT], lacc = z4;
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = z4;

  auto chunk = [&](int c, auto nbc) {
    constexpr int NBC = decltype(nbc)::value;  // key blocks in this chunk
    const int k0 = c * CN;
    // the chunk's pair bias: the score MFMAs' accumulators
    f32x4 sv[NBC][2];
#pragma unroll
    for (int kb = 0; kb < NBC; ++kb) {
      const h16x8 bb = ld8(bias_frag_block(a.bias, h, qt, (k0 >> 5) + kb, N, lane));
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int i = 0; i < 4; ++i) sv[kb][kh][i] = (float)bb[kh * 4 + i];
    }
    __syncthreads();  // the previous chunk's LDS readers are done
    nkv.store(Ks, Vs, tid, NBC * 32);
    __syncthreads();
    // the next chunk's K and V, issued after this chunk's scores (the wait
    // counter retires loads in order: issued earlier, they would hold up
    // the scores' wait for the bias)
    auto prefetch = [&] {
      if (c + 1 < NCH)
        nkv.load(Kg + (long)(k0 + CN) * a.ld, a.ld, Vg + (long)(k0 + CN) * a.ld, a.ld, tid,
                 min(CN, N - k0 - CN));
    };
    float mc = -INFINITY;
    if (active) {
#pragma unroll
      for (int kb = 0; kb < NBC; ++kb) {
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          HFrag<D> kf;
          kf.load(&Ks[(kb * 32 + kh * 16 + lq) * LD], g);
          sv[kb][kh] = HFrag<D>::mma(kf, qf, sv[kb][kh]);  // score + bias
          const int kk = k0 + kb * 32 + kh * 16 + 4 * g;
          const float4 mm = *reinterpret_cast<const float4*>(Mm + kk);
          const float4 ma = *reinterpret_cast<const float4*>(Ma + kk);
          const float mv[4] = {mm.x, mm.y, mm.z, mm.w};
          const float av[4] = {ma.x, ma.y, ma.z, ma.w};
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            // unmasked: s + bias; masked: exactly NEG_LOGIT
            const float x = __builtin_fmaf(sv[kb][kh][i], mv[i], av[i]);
            sv[kb][kh][i] = x;
            mc = fmaxf(mc, x);
          }
        }
      }
    }
    prefetch();
    if (!active) return;
    mc = fmaxf(mc, __shfl_xor(mc, 16, 64));
    mc = fmaxf(mc, __shfl_xor(mc, 32, 64));
    const float mn = fmaxf(mx, mc);
    const float alpha = fast_exp2(mx - mn);
#pragma unroll
    for (int dh = 0; dh < DT; ++dh) acc[dh] *= alpha;
    lacc *= alpha;
    mx = mn;
#pragma unroll
    for (int kb = 0; kb < NBC; ++kb) {
      h16x8 pf;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int i = 0; i < 4; ++i) pf[kh * 4 + i] = (h16)fast_exp2(sv[kb][kh][i] - mx);
#pragma unroll
      for (int dh = 0; dh < DT; ++dh)
        acc[dh] = mfma16x16x32(ld_tr8(Vs, LD, kb * 32, dh * 16, lane), pf, acc[dh]);
      lacc = mfma16x16x32(ones, pf, lacc);  // row sum of the probabilities
    }
  };
  // unrolled, so the wait for each chunk's loads counts only what is in flight
#pragma unroll
  for (int c = 0; c < NFULL; ++c) chunk(c, std::integral_constant<int, CB>());
  if constexpr (TAIL > 0) chunk(NFULL, std::integral_constant<int, TAIL>());

  if (!active) return;
  const float lsum = lacc[0];
  const float inv = __builtin_amdgcn_rcpf(lsum);
  const long orow = (tok0 + q) * a.ldo + h * D;
#pragma unroll
  for (int dh = 0; dh < DT; ++dh) {
    const int d0 = dh * 16 + 4 * g;
    h16x4 ov, gov;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float o = acc[dh][i] * inv;
      ov[i] = (h16)o;
      gov[i] = (h16)(o * sigmoidf_((float)gv[dh][i]));
    }
    *reinterpret_cast<h16x4*>(a.o + orow + d0) = ov;
    *reinterpret_cast<h16x4*>(a.og + orow + d0) = gov;
  }
  if (g == 0) a.lse[((long)r * H + h) * N + q] = mx + __log2f(lsum);
}

// Forward over a chunk of rows, N <= 256 (one key chunk).  Workgroup = (row
// chunk, head h, 64 queries), 4 waves x 16 queries, as attn_fwd_kernel, but
// it walks `rpc` rows: the pair bias of its queries is row-independent, so it
// is read once into registers and enters every row's score MFMA as the
// accumulator (no add per score); the next row's K, V, q, gate and key mask
// are loaded into registers while the current row computes, and only stored
// to LDS at the next row, so no compute waits on them.
template <int D, int NKB>
__global__ __launch_bounds__(256) void attn_fwd_rows_kernel(AttnArgs a, int rpc) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  constexpr int DT = D / 16;
  constexpr int LD = lds_ld<D>();
  constexpr int N = 32 * NKB;  // == a.N (dispatch)
  static_assert(NKB <= 8, "one key chunk");
  constexpr int QR = 64;       // query rows of the workgroup
  const int H = a.H;
  h16* Ks = reinterpret_cast<h16*>(smem_raw);          // [N][LD]
  h16* Vs = Ks + N * LD;                                // [N][LD]
  h16* Qs = Vs + N * LD;                                // [QR][LD]
  h16* Gs = Qs + QR * LD;                               // [QR][LD]
  float* Mm = reinterpret_cast<float*>(Gs + QR * LD);    // [N] 1 / 0 per key
  float* Ma = Mm + N;                                    // [N] 0 / NEG_LOGIT

  const int nqb = (N + QR - 1) / QR;
  const int nch = (a.R + rpc - 1) / rpc;
  const long G = (long)nch * H * nqb;
  const int bid = (int)xcd_block(G);  // (chunk, h, qb): the qb blocks of (chunk, h) share K, V
  if (bid >= G) return;
  const int qb = bid % nqb;
  const int h = (bid / nqb) % H;
  const int ch = bid / (nqb * H);
  const int r0 = ch * rpc, r1 = min(a.R, r0 + rpc);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int q0 = qb * QR + wave * 16;
  const bool active = q0 < N;  // idle waves keep to the barriers only
  const int lq = lane & 15, g = lane >> 4;
  const int q = min(q0, N - 16) + lq;
  const long HD = (long)H * D;

  // pair bias of this lane's query, all N keys, in score-fragment order
  float bsv[NKB][8];
  {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const h16x8 bb = ld8(bias_frag_block(a.bias, h, q >> 4, kb, N, lane));
#pragma unroll
      for (int e = 0; e < 8; ++e) bsv[kb][e] = (float)bb[e];
    }
    // Make the bias resident here: the row loop then never waits on these
    // loads (the wait counter retires in order, so a first use inside the
    // loop would also wait for the prefetch issued before it).
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int e = 0; e < 8; ++e) asm volatile("" ::"v"(bsv[kb][e]));
  }

  // next-row registers: K/V rows, one q or gate chunk, one key's mask
  constexpr int QCH = QR * (D / 8);  // 16-byte chunks of the q (or gate) tile
  static_assert(2 * QCH <= 512, "q and gate: at most two chunks per thread");
  RowPair<D, N> nkv;
  h16x8 nq, ng;
  float nm = 0.f;
  const int qrow = tid / (D / 8), qc = (tid % (D / 8)) * 8;  // tid < QCH
  const int qtok = min(qb * QR + qrow, N - 1);               // rows past N: any in-bounds row
  auto prefetch = [&](int r) {
    const long tok0 = (long)r * N;
    nkv.load(a.qkvg + tok0 * a.ld + HD + h * D, a.ld, a.qkvg + tok0 * a.ld + 2 * HD + h * D, a.ld,
             tid, N);
    if (tid < QCH) {
      const h16* row = a.qkvg + (tok0 + qtok) * a.ld + h * D + qc;
      nq = ld8(row);
      ng = ld8(row + 3 * HD);
    }
    if (tid < N) nm = a.mask[r * a.mask_sr + tid * a.mask_sk];
  };

  prefetch(r0);
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  for (int r = r0; r < r1; ++r) {
    __syncthreads();  // the previous row's LDS readers are done
    nkv.store(Ks, Vs, tid, N);
    if (tid < QCH) {
      st8(&Qs[qrow * LD + qc], nq);
      st8(&Gs[qrow * LD + qc], ng);
    }
    if (tid < N) {
      const bool on = nm != 0.f;
      Mm[tid] = on ? 1.f : 0.f;
      Ma[tid] = on ? 0.f : NEG_LOGIT;
    }
    __syncthreads();
    if (r + 1 < r1) prefetch(r + 1);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the compute
    if (!active) continue;

    HFrag<D> qf;
    qf.load(&Qs[(wave * 16 + lq) * LD], g);
    float sv[NKB][8];
    float mx = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        HFrag<D> kf;
        kf.load(&Ks[(kb * 32 + kh * 16 + lq) * LD], g);
        f32x4 cb;
#pragma unroll
        for (int i = 0; i < 4; ++i) cb[i] = bsv[kb][kh * 4 + i];
        const f32x4 s = HFrag<D>::mma(kf, qf, cb);  // score + bias
        const int kk = kb * 32 + kh * 16 + 4 * g;
        const float4 mm = *reinterpret_cast<const float4*>(Mm + kk);
        const float4 ma = *reinterpret_cast<const float4*>(Ma + kk);
        const float mv[4] = {mm.x, mm.y, mm.z, mm.w};
        const float av[4] = {ma.x, ma.y, ma.z, ma.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          // unmasked: s + bias; masked: exactly NEG_LOGIT
          const float x = __builtin_fmaf(s[i], mv[i], av[i]);
          sv[kb][kh * 4 + i] = x;
          mx = fmaxf(mx, x);
        }
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    float lsum = 0.f;
    f32x4 acc[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i) acc[i] = z4;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      h16x8 pf;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float p = fast_exp2(sv[kb][e] - mx);
        lsum += p;
        pf[e] = (h16)p;
      }
#pragma unroll
      for (int dh = 0; dh < DT; ++dh)
        acc[dh] = mfma16x16x32(ld_tr8(Vs, LD, kb * 32, dh * 16, lane), pf, acc[dh]);
    }
    lsum += __shfl_xor(lsum, 16, 64);
    lsum += __shfl_xor(lsum, 32, 64);
    const float inv = __builtin_amdgcn_rcpf(lsum);
    const long tok0 = (long)r * N;
    const long orow = (tok0 + q) * a.ldo + h * D;
    if (q0 + 16 <= N || lq < N - q0) {
#pragma unroll
      for (int dh = 0; dh < DT; ++dh) {
        const int d0 = dh * 16 + 4 * g;
        const h16x4 gv = *reinterpret_cast<const h16x4*>(&Gs[(wave * 16 + lq) * LD + d0]);
        h16x4 ov, gov;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float o = acc[dh][i] * inv;
          ov[i] = (h16)o;
          gov[i] = (h16)(o * sigmoidf_((float)gv[i]));
        }
        *reinterpret_cast<h16x4*>(a.o + orow + d0) = ov;
        *reinterpret_cast<h16x4*>(a.og + orow + d0) = gov;
      }
      if (g == 0) a.lse[((long)r * H + h) * N + q] = mx + __log2f(lsum);
    }
  }
}

// ------------------------------------------------------- backward: gate + D
// dO = dog * sigmoid(g); dG = dog * o * s(1-s); nDsum = -sum_d dO * o.
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
  const h16x8 gv = ld8(a.qkvg + tok * a.ld + 3 * HD + c0);
  const h16x8 ov = ld8(a.o + tok * a.ldo + c0);
  const h16x8 dv = ld8(b.dog + tok * a.ldo + c0);
  h16x8 dov, dgv;
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float sg = sigmoidf_((float)gv[e]);
    const float o = (float)ov[e], d = (float)dv[e];
    const float dO = d * sg;
    dov[e] = (h16)dO;
    dgv[e] = (h16)(d * o * sg * (1.f - sg));
    s += dO * o;
  }
  st8(b.dO + tok * a.ldo + c0, dov);
  st8(b.dqkvg + tok * a.ld + 3 * HD + c0, dgv);
  s = group_sum<LPH>(s);
  if (part == 0) {
    const long r = tok / a.N, q = tok % a.N;
    b.nDsum[(r * a.H + h) * a.N + q] = -s;
  }
}

// ----------------------------------------------------------- backward: dQ
// Same decomposition as the forward: (row, head, 64 queries), 4 waves, keys
// in chunks of up to 256 staged in LDS.  Per chunk the lane's pair-bias row
// (minus lse, with -inf at masked keys so p = dS = 0 there) is fetched up
// front, all loads in flight at once.
template <int D, int NKB, int QW>
__global__ __launch_bounds__(64 * QW) void attn_bwd_dq_kernel(AttnBwdArgs b) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  constexpr int DT = D / 16;
  constexpr int LD = lds_ld<D>();
  const AttnArgs& a = b.f;
  constexpr int N = 32 * NKB;  // == a.N (dispatch)
  constexpr int CB = NKB < 8 ? NKB : 8;  // key blocks per chunk
  constexpr int NCH = (NKB + CB - 1) / CB;
  constexpr int CN = 32 * CB;
  const int H = a.H;
  h16* Ks = reinterpret_cast<h16*>(smem_raw);   // [CN][LD]
  h16* Vs = Ks + CN * LD;                        // [CN][LD]
  float* Ms = reinterpret_cast<float*>(Vs + CN * LD);  // [N]
  constexpr int T = 64 * QW;   // threads; QW waves of 16 queries

  const int nqb = (N + 16 * QW - 1) / (16 * QW);
  const long G = (long)a.R * H * nqb;
  const int bid = (int)xcd_block(G);
  if (bid >= G) return;
  const RowHeadQb ord = row_tile_order(bid, a.R, H, nqb);
  const int qb = ord.qb, h = ord.h, r = ord.r;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const long tok0 = (long)r * N;
  const h16* Kg = a.qkvg + tok0 * a.ld + H * D + h * D;
  const h16* Vg = a.qkvg + tok0 * a.ld + 2 * H * D + h * D;
  stage_rows2<D, CN, T>(Ks, Kg, a.ld, Vs, Vg, a.ld, tid);
  // additive key mask: a masked key's exponent becomes -inf, so p = dS = 0
  for (int k = tid; k < N; k += T)
    Ms[k] = a.mask[r * a.mask_sr + k * a.mask_sk] != 0.f ? 0.f : -INFINITY;

  const int q0 = qb * 16 * QW + wave * 16;
  const int lq = lane & 15, g = lane >> 4;
  const int q = min(q0, N - 16) + lq;  // idle waves read in bounds, store nothing
  HFrag<D> qf, dof;
  qf.load(a.qkvg + (tok0 + q) * a.ld + h * D, g);
  dof.load(b.dO + (tok0 + q) * a.ldo + h * D, g);
  const float lse = a.lse[((long)r * H + h) * N + q];
  const float nDq = b.nDsum[((long)r * H + h) * N + q];
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  const f32x4 nD = {nDq, nDq, nDq, nDq};
  f32x4 acc[DT];
#pragma unroll
  for (int i = 0; i < DT; ++i) acc[i] = z4;

#pragma unroll
  for (int c = 0; c < NCH; ++c) {
    const int k0c = c * CN;
    float bsv[CB][8];
#pragma unroll
    for (int kb = 0; kb < CB; ++kb) {
      if (c * CB + kb < NKB) {
        const h16x8 bb = ld8(bias_frag_block(a.bias, h, q >> 4, (k0c >> 5) + kb, N, lane));
#pragma unroll
        for (int e = 0; e < 8; ++e) bsv[kb][e] = (float)bb[e] - lse;
      }
    }
    if (c > 0) {
      __syncthreads();  // every wave is done with the previous chunk
      stage_rows2<D, CN, T>(Ks, Kg + (long)k0c * a.ld, a.ld, Vs, Vg + (long)k0c * a.ld, a.ld, tid,
                            min(CN, N - k0c));
    }
    __syncthreads();
    if (NCH == 1 && q0 >= N) return;  // idle wave, no barrier follows
#pragma unroll
    for (int kb = 0; kb < CB; ++kb) {
      if (c * CB + kb < NKB) {
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const float4 mm = *reinterpret_cast<const float4*>(Ms + k0c + kb * 32 + kh * 16 + 4 * g);
          bsv[kb][kh * 4 + 0] += mm.x;
          bsv[kb][kh * 4 + 1] += mm.y;
          bsv[kb][kh * 4 + 2] += mm.z;
          bsv[kb][kh * 4 + 3] += mm.w;
        }
      }
    }
#pragma unroll
    for (int kb = 0; kb < CB; ++kb) {
      if (c * CB + kb < NKB) {
        h16x8 dsf;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const int krow = (kb * 32 + kh * 16 + lq) * LD;
          HFrag<D> kf, vf;
          kf.load(&Ks[krow], g);
          vf.load(&Vs[krow], g);
          f32x4 cs;
#pragma unroll
          for (int i = 0; i < 4; ++i) cs[i] = bsv[kb][kh * 4 + i];
          const f32x4 s = HFrag<D>::mma(kf, qf, cs);    // S + bias - lse
          const f32x4 dp = HFrag<D>::mma(vf, dof, nD);  // dP - Dsum
#pragma unroll
          for (int i = 0; i < 4; ++i) dsf[kh * 4 + i] = (h16)(fast_exp2(s[i]) * dp[i]);
        }
#pragma unroll
        for (int dh = 0; dh < DT; ++dh)
          acc[dh] = mfma16x16x32(ld_tr8(Ks, LD, kb * 32, dh * 16, lane), dsf, acc[dh]);
      }
    }
  }
  if (q0 >= N) return;
  h16* out = b.dqkvg + (tok0 + q) * a.ld + h * D;
#pragma unroll
  for (int dh = 0; dh < DT; ++dh) {
    h16x4 v;
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = (h16)(acc[dh][i] * b.scale);
    *reinterpret_cast<h16x4*>(out + dh * 16 + 4 * g) = v;
  }
}

// dQ over a chunk of rows, N <= 256: the forward's row-chunk structure
// (bias of the workgroup's queries resident in registers across rows, next
// row's K, V, q, dO, lse, Dsum and key mask prefetched into registers while
// the current row computes).
template <int D, int NKB>
__global__ __launch_bounds__(256) void attn_bwd_dq_rows_kernel(AttnBwdArgs b, int rpc) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  constexpr int DT = D / 16;
  constexpr int LD = lds_ld<D>();
  const AttnArgs& a = b.f;
  constexpr int N = 32 * NKB;  // == a.N (dispatch)
  static_assert(NKB <= 8, "one key chunk");
  constexpr int QR = 64;
  const int H = a.H;
  h16* Ks = reinterpret_cast<h16*>(smem_raw);         // [N][LD]
  h16* Vs = Ks + N * LD;                               // [N][LD]
  h16* Qs = Vs + N * LD;                               // [QR][LD]
  h16* Os = Qs + QR * LD;                              // [QR][LD] dO
  float* Ms = reinterpret_cast<float*>(Os + QR * LD);   // [N] 0 / -inf per key
  float* Ls = Ms + N;                                   // [QR] lse
  float* Dl = Ls + QR;                                  // [QR] -Dsum

  const int nqb = (N + QR - 1) / QR;
  const int nch = (a.R + rpc - 1) / rpc;
  const long G = (long)nch * H * nqb;
  const int bid = (int)xcd_block(G);
  if (bid >= G) return;
  const int qb = bid % nqb;
  const int h = (bid / nqb) % H;
  const int ch = bid / (nqb * H);
  const int r0 = ch * rpc, r1 = min(a.R, r0 + rpc);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q0 = qb * QR + wave * 16;
  const bool active = q0 < N;
  const int lq = lane & 15, g = lane >> 4;
  const int q = min(q0, N - 16) + lq;
  const int ql = wave * 16 + lq;  // query row in the staged tiles
  const long HD = (long)H * D;

  float bsv[NKB][8];
  {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      const h16x8 bb = ld8(bias_frag_block(a.bias, h, q >> 4, kb, N, lane));
#pragma unroll
      for (int e = 0; e < 8; ++e) bsv[kb][e] = (float)bb[e];
    }
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
      for (int e = 0; e < 8; ++e) asm volatile("" ::"v"(bsv[kb][e]));
  }

  constexpr int QCH = QR * (D / 8);
  RowPair<D, N> nkv;
  h16x8 nq, no;
  float nm = 0.f, nl = 0.f, nd = 0.f;
  const int qrow = tid / (D / 8), qc = (tid % (D / 8)) * 8;  // tid < QCH
  const int qtok = min(qb * QR + qrow, N - 1);
  const int stok = min(qb * QR + tid, N - 1);                // tid < QR: statistics row
  auto prefetch = [&](int r) {
    const long tok0 = (long)r * N;
    nkv.load(a.qkvg + tok0 * a.ld + HD + h * D, a.ld, a.qkvg + tok0 * a.ld + 2 * HD + h * D, a.ld,
             tid, N);
    if (tid < QCH) {
      nq = ld8(a.qkvg + (tok0 + qtok) * a.ld + h * D + qc);
      no = ld8(b.dO + (tok0 + qtok) * a.ldo + h * D + qc);
    }
    if (tid < N) nm = a.mask[r * a.mask_sr + tid * a.mask_sk];
    if (tid < QR) {
      nl = a.lse[((long)r * H + h) * N + stok];
      nd = b.nDsum[((long)r * H + h) * N + stok];
    }
  };

  prefetch(r0);
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  for (int r = r0; r < r1; ++r) {
    __syncthreads();
    nkv.store(Ks, Vs, tid, N);
    if (tid < QCH) {
      st8(&Qs[qrow * LD + qc], nq);
      st8(&Os[qrow * LD + qc], no);
    }
    // a masked key's exponent becomes -inf, so p = dS = 0
    if (tid < N) Ms[tid] = nm != 0.f ? 0.f : -INFINITY;
    if (tid < QR) {
      Ls[tid] = nl;
      Dl[tid] = nd;
    }
    __syncthreads();
    if (r + 1 < r1) prefetch(r + 1);
    __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the compute
    if (!active) continue;

    HFrag<D> qf, dof;
    qf.load(&Qs[ql * LD], g);
    dof.load(&Os[ql * LD], g);
    const float lse = Ls[ql], nDq = Dl[ql];
    const f32x4 nD = {nDq, nDq, nDq, nDq};
    f32x4 acc[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i) acc[i] = z4;
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb) {
      h16x8 dsf;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        const int krow = (kb * 32 + kh * 16 + lq) * LD;
        HFrag<D> kf, vf;
        kf.load(&Ks[krow], g);
        vf.load(&Vs[krow], g);
        const float4 mm = *reinterpret_cast<const float4*>(Ms + kb * 32 + kh * 16 + 4 * g);
        f32x4 cs;
        cs[0] = bsv[kb][kh * 4 + 0] + (mm.x - lse);
        cs[1] = bsv[kb][kh * 4 + 1] + (mm.y - lse);
        cs[2] = bsv[kb][kh * 4 + 2] + (mm.z - lse);
        cs[3] = bsv[kb][kh * 4 + 3] + (mm.w - lse);
        const f32x4 s = HFrag<D>::mma(kf, qf, cs);    // S + bias - lse
        const f32x4 dp = HFrag<D>::mma(vf, dof, nD);  // dP - Dsum
#pragma unroll
        for (int i = 0; i < 4; ++i) dsf[kh * 4 + i] = (h16)(fast_exp2(s[i]) * dp[i]);
      }
#pragma unroll
      for (int dh = 0; dh < DT; ++dh)
        acc[dh] = mfma16x16x32(ld_tr8(Ks, LD, kb * 32, dh * 16, lane), dsf, acc[dh]);
    }
    if (q0 + 16 <= N || lq < N - q0) {
      h16* out = b.dqkvg + ((long)r * N + q) * a.ld + h * D;
#pragma unroll
      for (int dh = 0; dh < DT; ++dh) {
        h16x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = (h16)(acc[dh][i] * b.scale);
        *reinterpret_cast<h16x4*>(out + dh * 16 + 4 * g) = v;
      }
    }
  }
}

// ------------------------------------------------------ backward: dK, dV, dB
// Workgroup = (chunk of rows, head h, KT*16 keys), 4 waves = KT key tiles x
// QS query groups (KT=2, QS=2 for N <= 256; KT=1, QS=4 beyond).  Wave
// (kt, qs) owns key tile kt and the 32-query blocks blk = ib*QS + qs, so the
// bias-gradient tile it keeps in registers is ceil(N/(32*QS)) x 8 floats per
// lane; the pair bias is row-independent and is read once per workgroup into
// a register tile of the same shape.  Per row, Q and dO (head h) are staged
// in LDS (in chunks of up to 256 rows); the QS query groups' dK/dV partials
// are added through LDS in a fixed order before the write.  N = 32*NQB.
//
// Per score the MFMA accumulators start at (bias - lse) and -Dsum, so
// p = exp2(S) and dS = p * dP' need no further adds.  A masked key gets
// exponent -inf (p = dS = 0) -- exact for a row with any unmasked key, where
// AF2's masked weight exp(-1e8 - lse) underflows to 0.  A fully masked row is
// the uniform distribution (p = 1/N, dS = 0).
//
// W waves per workgroup as QS query groups x KT key tiles: 4 = 2 x 2 up to
// N = 256; 8 beyond, as 4 x 2 up to N = 768 (6 query blocks a wave: 235
// registers) and 8 x 1 past it, so a wave's bias column and bias-gradient
// registers stay within two waves per SIMD (one workgroup per CU).  Every key
// group of a row re-stages the row's Q and dO, so 32 keys a workgroup
// instead of 16 halve that traffic.
template <int D, int NQB, int W, int QS>
__global__ __launch_bounds__(64 * W) void attn_bwd_dkv_kernel(AttnBwdArgs b) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  constexpr int T = 64 * W;              // threads
  constexpr int DT = D / 16;
  constexpr int LD = lds_ld<D>();
  constexpr int N = 32 * NQB;            // == a.N (dispatch)
  static_assert(W % QS == 0, "query groups x key tiles");
  constexpr int KT = W / QS;             // 16-key tiles per workgroup
  constexpr int NB = (NQB + QS - 1) / QS;  // query blocks per wave (at most)
  constexpr int CQB = NQB < 8 ? NQB : 8;   // query blocks per staged chunk
  constexpr int NCH = (NQB + CQB - 1) / CQB;
  constexpr int CN = 32 * CQB;
  static_assert(NCH == 1 || CQB % QS == 0, "chunk must hold whole rounds of query groups");
  const AttnArgs& a = b.f;
  const int H = a.H;
  h16* Qs = reinterpret_cast<h16*>(smem_raw);         // [CN][LD]
  h16* Os = Qs + CN * LD;                              // [CN][LD] dO
  float* Ls = reinterpret_cast<float*>(Os + CN * LD);   // [N] -lse
  float* Ds = Ls + N;                                   // [N] -Dsum
  float* Xs = Ds + N;                                   // [QS-1][KT][K,V][DT*4][64]
  float* Ms = Xs + (QS - 1) * KT * 2 * DT * 4 * 64;     // [N] key mask of the row
  h16* KVs = reinterpret_cast<h16*>(Ms + N);          // [K,V][16*KT][LD] own keys

  constexpr int NKW = N / (16 * KT);  // key groups per (chunk, head)
  const long G = (long)((a.R + b.rows_per_chunk - 1) / b.rows_per_chunk) * H * NKW;
  const int bid = (int)xcd_block(G);  // (chunk, h, kw): the kw groups share Q, dO
  if (bid >= G) return;
  const int kw = bid % NKW;
  const int h = (bid / NKW) % H;
  const int ch = bid / (NKW * H);
  const int r0 = ch * b.rows_per_chunk;
  const int r1 = min(a.R, r0 + b.rows_per_chunk);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int kt_ = wave % KT, qs = (wave / KT) % QS;
  const int lk = lane & 15, g = lane >> 4;
  const int k = kw * 16 * KT + kt_ * 16 + lk;
  const long HD = (long)H * D;

  // bias column k at this wave's queries; bias-gradient accumulators
  float bsl[NB][8], dbias[NB][8];
  const bool hasb = a.bias != nullptr;
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {
    const int qb = (ib * QS + qs) * 32;
    const bool have = hasb && qb < N;  // wave-uniform
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bsl[ib][e] = 0.f;
      dbias[ib][e] = 0.f;
    }
    if (have) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        bsl[ib][e] = (float)a.bias[bias_frag_index(h, qb + (e / 4) * 16 + 4 * g + (e % 4), k, N)];
    }
  }
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};

  // Stage s = (row r0 + s / NCH, chunk s % NCH).  While a stage computes, the
  // next stage's Q/dO tile -- and, at a row's first chunk, the row's -lse,
  // -Dsum, mask and this lane's key/value fragments -- are loaded into
  // registers, so the row loop does not wait on memory at every row.
  constexpr int NPT = (N + T - 1) / T;  // row statistics per thread
  const int nst = (r1 - r0) * NCH;
  // Loaded values are only consumed at the next stage (vmcnt retires loads
  // in order, so any use now would wait for the whole prefetch).
  // The workgroup's own 16*KT keys and values of the row go through LDS too,
  // so no register filled by the prefetch is read before the next stage.
  RowPair<D, CN, T> nxt;
  float nls[NPT], nds[NPT], nmask[NPT];
  constexpr int KCH = 16 * KT * 2 * (D / 8);  // 16-byte chunks of own K and V
  static_assert(KCH <= T, "own keys: one chunk per thread");
  h16x8 nkv;
  const int kvi = tid % (KCH / 2), kvs = tid / (KCH / 2);  // chunk, 0 = K / 1 = V
  const int kvrow = kvi / (D / 8), kvc = (kvi % (D / 8)) * 8;
  auto prefetch = [&](int s) {
    const int r = r0 + s / NCH, c = s % NCH;
    const long tok = (long)r * N + c * CN;
    nxt.load(a.qkvg + tok * a.ld + h * D, a.ld, b.dO + tok * a.ldo + h * D, a.ldo, tid,
             min(CN, N - c * CN));
    if (c == 0) {
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        const int qq = tid + T * i;
        nls[i] = 0.f;
        nds[i] = 0.f;
        nmask[i] = 0.f;
        if (qq < N) {
          nls[i] = a.lse[((long)r * H + h) * N + qq];
          nds[i] = b.nDsum[((long)r * H + h) * N + qq];
          nmask[i] = a.mask[r * a.mask_sr + qq * a.mask_sk];
        }
      }
      if (tid < KCH) {
        const long kt = (long)r * N + kw * 16 * KT + kvrow;
        nkv = ld8(a.qkvg + kt * a.ld + (1 + kvs) * HD + h * D + kvc);
      }
    }
  };

  prefetch(0);
  HFrag<D> kf, vf;
  bool mk = false;
  const int klocal = kt_ * 16 + lk;  // this lane's key among the workgroup's
  float xm = 0.f;
  f32x4 accK[DT], accV[DT];
  for (int s = 0; s < nst; ++s) {
    const int r = r0 + s / NCH, c = s % NCH;
    const long tok0 = (long)r * N;
    __syncthreads();  // the previous stage's LDS readers are done
    nxt.store(Qs, Os, tid, min(CN, N - c * CN));
    if (c == 0) {
      int non = 0;
#pragma unroll
      for (int i = 0; i < NPT; ++i) {
        const int qq = tid + T * i;
        if (qq < N) {
          Ls[qq] = -nls[i];
          Ds[qq] = nds[i];
          Ms[qq] = nmask[i];
        }
        non |= nmask[i] != 0.f;
      }
      if (tid < KCH) st8(&KVs[(kvs * 16 * KT + kvrow) * LD + kvc], nkv);
      const bool live = __syncthreads_or(non);  // the row has an unmasked key
      kf.load(&KVs[klocal * LD], g);
      vf.load(&KVs[(16 * KT + klocal) * LD], g);
      mk = Ms[k] != 0.f;
      // exponent of a masked key: -inf (weight 0) in a live row, -log2 N
      // (weight 1/N) in a fully masked one; either way its dS is 0
      xm = live ? -INFINITY : -__log2f((float)N);
#pragma unroll
      for (int i = 0; i < DT; ++i) { accK[i] = z4; accV[i] = z4; }
    } else {
      __syncthreads();
    }
    if (s + 1 < nst) prefetch(s + 1);

    // One unit = this wave's 16 keys against one 32-query block.  Its LDS
    // operands (row reads, -lse, -Dsum and the transposed reads) are read in
    // one batch; with PF the next unit's batch of the same stage is issued
    // right after this unit's S / dP products, so the reads are in flight
    // during the exponentials and the dV / dK products.  Without PF each
    // batch is read at its unit: five or six units a wave (N = 544..768),
    // whose bias registers leave no room, and the four-wave D = 32 shapes
    // (N <= 256 without a pair bias), whose next-row registers hold a whole
    // row's Q and dO.
    constexpr bool PF = NB <= 4 && (D == 16 || W == 8);
    struct Ops {
      HFrag<D> q[2], o[2];
      h16x8 to[DT], tq[DT];
      float4 l[2], d[2];
    };
    auto load_ops = [&](int ib, Ops& x) __attribute__((always_inline)) {
      const int qb = (ib * QS + qs) * 32, ql = qb - c * CN;
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        x.q[qh].load(&Qs[(ql + qh * 16 + lk) * LD], g);
        x.o[qh].load(&Os[(ql + qh * 16 + lk) * LD], g);
        x.l[qh] = *reinterpret_cast<const float4*>(Ls + qb + qh * 16 + 4 * g);
        x.d[qh] = *reinterpret_cast<const float4*>(Ds + qb + qh * 16 + 4 * g);
      }
#pragma unroll
      for (int dh = 0; dh < DT; ++dh) {
        x.to[dh] = ld_tr8(Os, LD, ql, dh * 16, lane);
        x.tq[dh] = ld_tr8(Qs, LD, ql, dh * 16, lane);
      }
    };
    // this stage's units: ib = ib0 .. (blocks of chunk c; all blocks with one chunk)
    const int ib0 = NCH > 1 ? c * (CQB / QS) : 0;
    Ops cur, nxt;
    if (PF && ib0 < NB && ib0 * QS + qs < NQB) load_ops(ib0, cur);
#pragma unroll
    for (int ib = 0; ib < NB; ++ib) {
      if (NCH > 1 && ib * QS / CQB != c) continue;  // block of another chunk
      const int blk = ib * QS + qs;
      if (blk < NQB) {
        if constexpr (!PF) load_ops(ib, cur);
        h16x8 pf, dsf;
        f32x4 s4[2], dp[2];
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
          f32x4 cs, cd;
          cs[0] = bsl[ib][qh * 4 + 0] + cur.l[qh].x;
          cs[1] = bsl[ib][qh * 4 + 1] + cur.l[qh].y;
          cs[2] = bsl[ib][qh * 4 + 2] + cur.l[qh].z;
          cs[3] = bsl[ib][qh * 4 + 3] + cur.l[qh].w;
          cd[0] = cur.d[qh].x; cd[1] = cur.d[qh].y; cd[2] = cur.d[qh].z; cd[3] = cur.d[qh].w;
          s4[qh] = HFrag<D>::mma(cur.q[qh], kf, cs);  // S + bias - lse
          dp[qh] = HFrag<D>::mma(cur.o[qh], vf, cd);  // dP - Dsum
        }
        // the next unit of this stage (wave-uniform)
        const bool more = PF && ib + 1 < NB && (NCH == 1 || (ib + 1) * QS / CQB == c) &&
                          (ib + 1) * QS + qs < NQB;
        if (more) load_ops(ib + 1, nxt);
#pragma unroll
        for (int qh = 0; qh < 2; ++qh)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float p = fast_exp2(mk ? s4[qh][i] : xm);
            const float ds = mk ? p * dp[qh][i] : 0.f;
            pf[qh * 4 + i] = (h16)p;
            dsf[qh * 4 + i] = (h16)ds;
            dbias[ib][qh * 4 + i] += ds;
          }
#pragma unroll
        for (int dh = 0; dh < DT; ++dh) {
          accV[dh] = mfma16x16x32(cur.to[dh], pf, accV[dh]);
          accK[dh] = mfma16x16x32(cur.tq[dh], dsf, accK[dh]);
        }
        if (more) cur = nxt;
      }
    }
    if (c != NCH - 1) continue;

    // row done: add the query groups' partials (groups 1..QS-1 park theirs
    // in LDS) and write dK, dV
    if (qs > 0) {
      float* x = Xs + ((qs - 1) * KT + kt_) * 2 * DT * 4 * 64;
#pragma unroll
      for (int dh = 0; dh < DT; ++dh)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[(dh * 4 + i) * 64 + lane] = accK[dh][i];
          x[(DT * 4 + dh * 4 + i) * 64 + lane] = accV[dh][i];
        }
    }
    __syncthreads();
    if (qs == 0) {
#pragma unroll
      for (int j = 1; j < QS; ++j) {
        const float* x = Xs + ((j - 1) * KT + kt_) * 2 * DT * 4 * 64;
#pragma unroll
        for (int dh = 0; dh < DT; ++dh)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            accK[dh][i] += x[(dh * 4 + i) * 64 + lane];
            accV[dh][i] += x[(DT * 4 + dh * 4 + i) * 64 + lane];
          }
      }
      // dK (w.r.t. the unscaled k) = sum_q dS * q_scaled / log2(e)
      h16* dk = b.dqkvg + (tok0 + k) * a.ld + HD + h * D;
      h16* dvp = b.dqkvg + (tok0 + k) * a.ld + 2 * HD + h * D;
#pragma unroll
      for (int dh = 0; dh < DT; ++dh) {
        h16x4 kv, vv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          kv[i] = (h16)(accK[dh][i] * (1.f / LOG2E));
          vv[i] = (h16)accV[dh][i];
        }
        *reinterpret_cast<h16x4*>(dk + dh * 16 + 4 * g) = kv;
        *reinterpret_cast<h16x4*>(dvp + dh * 16 + 4 * g) = vv;
      }
    }
  }
  if (b.dbias_part == nullptr) return;
  float* part = b.dbias_part + (((long)ch * H + h) * N) * N;
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {
    const int blk = ib * QS + qs;
    if (blk >= NQB) break;
    const int qb = blk * 32;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int qi = qb + (e / 4) * 16 + 4 * g + (e % 4);
      part[(long)qi * N + k] = dbias[ib][e];
    }
  }
}

// Direct global -> LDS copies (gfx950 global_load_lds_dword / _dwordx4): lane
// i writes its 4 (16) bytes at LDS byte m0 + 4 i (16 i).  Issued as inline
// asm, so the compiler neither counts them nor makes every later LDS read
// wait for them; the kernels that use them retire them with explicit
// vmcnt waits before the barrier that publishes the data.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
  return (unsigned)(size_t)((const __attribute__((address_space(3))) unsigned char*)p);
}
__device__ __forceinline__ void dma16(const void* src, unsigned lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4(const void* src, unsigned lds) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dword %0, off" ::"v"(src), "s"(lds)
               : "memory", "m0");
}
// The same with a uniform 64-bit base (SGPRs) and a per-lane 32-bit byte
// offset: the per-row address update is scalar.
__device__ __forceinline__ void dma16s(unsigned voff, const void* sbase, unsigned lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}
__device__ __forceinline__ void dma4s(unsigned voff, const void* sbase, unsigned lds) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sbase), "s"(lds)
               : "memory", "m0");
}
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 16, "vmcnt");
  __builtin_amdgcn_s_waitcnt(0x0F70 | N);
}

// dK/dV/dBias for D = 32 and N <= 256, the same work split and arithmetic
// as attn_bwd_dkv_kernel, with the row staging rebuilt around the direct
// copies:
//
//  * LDS holds two row buffers.  Each is Q, dO (the row's N tokens) and K, V
//    (the workgroup's 32 keys) as h16 tiles of 64-byte rows, the 16-byte
//    chunk c of tile row t stored at chunk c ^ ((t >> 1) & 3) -- conflict-free
//    for both the row reads (b128) and the transposed reads
//    (ds_read_b64_tr_b16) -- then the row's lse, -Dsum and key mask.  While
//    row s computes from one buffer, the copies of row s+1 fill the other;
//    their addresses are a per-lane offset fixed for the kernel plus a
//    scalar row base.
//  * Nothing else in the row loop reads global memory, and each wave issues
//    the same copies and stores every row (the last row's prefetch re-reads
//    that row), so the wait that opens a row retires exactly its copies and
//    leaves the previous row's dK/dV stores in flight.
//  * The two query groups split the 32-query blocks evenly: with an odd
//    count, each takes one 16-query half of the last block.
//  * Two barriers per row: one after the copies land, one to add the query
//    groups' dK/dV partials.
template <int NQB>
__global__ __launch_bounds__(256, 2) void attn_bwd_dkv_lds_kernel(AttnBwdArgs b) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  constexpr int D = 32, DT = 2;
  constexpr int N = 32 * NQB;            // == a.N (dispatch)
  static_assert(NQB <= 8, "one query chunk");
  constexpr int QS = 2, KT = 2;          // query groups x 16-key tiles per workgroup
  constexpr int FULL = NQB / QS;         // whole blocks per query group
  constexpr bool HALF = NQB % QS != 0;   // plus half of the last block
  constexpr int NB = FULL + (HALF ? 1 : 0);
  constexpr int TILE = N * 64;           // bytes of one [N][32] h16 tile
  constexpr int KVT = 16 * KT * 64;      // bytes of the K (or V) tile
  constexpr int SOFF = 2 * TILE + 2 * KVT;
  constexpr int BUF = SOFF + 3 * N * 4;
  constexpr int JT = N / 16;             // 1 KB copies per Q (dO) tile
  constexpr int NCP = NQB + 1;           // tile copies per wave: (2 JT + 2 KT) / 4
  constexpr int JS = (N + 63) / 64;      // 256-byte copies per statistic
  constexpr int NSC = (3 * JS + 3) / 4;  // statistic copies per wave (at most)
  const AttnArgs& a = b.f;
  const int H = a.H;
  float* Xs = reinterpret_cast<float*>(smem_raw + 2 * BUF);  // [KT][K,V][DT*4][64], query group 1

  constexpr int NKW = N / (16 * KT);
  const long G = (long)((a.R + b.rows_per_chunk - 1) / b.rows_per_chunk) * H * NKW;
  const int bid = (int)xcd_block(G);
  if (bid >= G) return;
  const int kw = bid % NKW;
  const int h = (bid / NKW) % H;
  const int ch = bid / (NKW * H);
  const int r0 = ch * b.rows_per_chunk;
  const int r1 = min(a.R, r0 + b.rows_per_chunk);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kt_ = wave % KT, qs = wave / KT;
  const int lk = lane & 15, g = lane >> 4;
  const int klocal = kt_ * 16 + lk;
  const int k = kw * 16 * KT + klocal;
  const long HD = (long)H * D;
  const unsigned lds0 = lds_addr(smem_raw);

  // blocks of this wave: 32-query block ib * QS + qs for ib < FULL, and
  // queries [16 qs, 16 qs + 16) of block NQB - 1 when HALF
  auto blk_q0 = [&](int ib) { return ib < FULL ? (ib * QS + qs) * 32 : (NQB - 1) * 32; };
  float bsl[NB][8], dbias[NB][8];

#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {
    const int qb = blk_q0(ib);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bsl[ib][e] = (float)a.bias[bias_frag_index(h, qb + (e / 4) * 16 + 4 * g + (e % 4), k, N)];
      dbias[ib][e] = 0.f;
    }
  }

  // Tile copy j (1 KB) fills rows 16 j'..16 j'+15 of one tile: lane i writes
  // physical chunk i & 3 of row 16 j' + i / 4, read from the logical chunk
  // the swizzle puts there.  Wave w issues tile copies w + 4 i (Q: j < JT,
  // dO: j < 2 JT, then K, V) and statistic copies w + 4 i (lse, -Dsum, mask).
  unsigned voff[NCP], sdst[NCP];
  long soff[NCP];
  bool sdo[NCP];
#pragma unroll
  for (int i = 0; i < NCP; ++i) {
    const int j = wave + 4 * i;
    const int tile = j < 2 * JT ? j / JT : 2 + (j - 2 * JT) / KT;  // Q, dO, K, V
    const int jr = j < 2 * JT ? j % JT : (j - 2 * JT) % KT;
    const int row = jr * 16 + (lane >> 2);
    const int c = (lane & 3) ^ ((row >> 1) & 3);
    sdo[i] = tile == 1;
    const long ld = tile == 1 ? a.ldo : a.ld;
    voff[i] = (unsigned)((row * ld + c * 8) * 2);
    soff[i] = tile == 0 || tile == 1 ? (long)h * D * 2
                                     : ((long)kw * 16 * KT * a.ld + (tile - 1) * HD + h * D) * 2;
    sdst[i] = (tile < 2 ? tile * TILE : 2 * TILE + (tile - 2) * KVT) + jr * 1024;
  }
  unsigned svoff[NSC], ssdst[NSC];
  int swhich[NSC];
  bool son[NSC], slive[NSC];
#pragma unroll
  for (int i = 0; i < NSC; ++i) {
    const int j = wave + 4 * i;
    son[i] = j < 3 * JS;
    const int which = son[i] ? j / JS : 0, js = son[i] ? j % JS : 0;
    const int q = js * 64 + lane;
    swhich[i] = which;
    slive[i] = q < N;
    svoff[i] = which == 2 ? (unsigned)(q * a.mask_sk * 4) : (unsigned)(q * 4);
    ssdst[i] = SOFF + which * N * 4 + js * 256;
  }
  auto copy_row = [&](int r, int u) __attribute__((always_inline)) {
    const unsigned base = lds0 + u * BUF;
    const char* qrow = reinterpret_cast<const char*>(a.qkvg + (long)r * N * a.ld);
    const char* orow = reinterpret_cast<const char*>(b.dO + (long)r * N * a.ldo);
#pragma unroll
    for (int i = 0; i < NCP; ++i) dma16s(voff[i], (sdo[i] ? orow : qrow) + soff[i], base + sdst[i]);
    const long srow = ((long)r * H + h) * N;
#pragma unroll
    for (int i = 0; i < NSC; ++i) {
      if (son[i]) {
        const float* sb = swhich[i] == 0 ? a.lse + srow
                        : swhich[i] == 1 ? b.nDsum + srow
                                         : a.mask + (long)r * a.mask_sr;
        if (slive[i]) dma4s(svoff[i], sb, base + ssdst[i]);
      }
    }
  };

  // lane-constant swizzled offsets (h16 units): row reads at rows ≡ lk
  // (mod 16), transposed reads at rows 4g + lk/4 (mod 16)
  const int rsw = ((g ^ ((lk >> 1) & 3)) << 3);
  const int trow = 4 * g + (lk >> 2);
  const int tsw0 = (((lk & 3) >> 1) ^ ((trow >> 1) & 3)) * 8 + 4 * (lk & 1);       // columns 0..15
  const int tsw1 = ((2 + ((lk & 3) >> 1)) ^ ((trow >> 1) & 3)) * 8 + 4 * (lk & 1);  // columns 16..31
  auto tr4 = [&](const h16* T, int r0_, int dh) __attribute__((always_inline)) -> h16x4 {
    const h16* p = T + (r0_ + trow) * 32 + (dh ? tsw1 : tsw0);
    return __builtin_bit_cast(h16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
  };
  auto tr8 = [&](const h16* T, int r0_, int dh) __attribute__((always_inline)) -> h16x8 {
    const h16x4 x = tr4(T, r0_, dh), y = tr4(T, r0_ + 16, dh);
    h16x8 v;
    v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
    v[4] = y[0]; v[5] = y[1]; v[6] = y[2]; v[7] = y[3];
    return v;
  };

  const int nst = r1 - r0;
  copy_row(r0, 0);
  wait_vm<0>();  // the bias tile and row r0's copies
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  for (int s = 0; s < nst; ++s) {
    const int r = r0 + s, u = s & 1;
    // this row's copies are in; query group 0's four dK/dV stores of the
    // previous row may still be in flight
    if (qs == 0) wait_vm<4>();
    else wait_vm<0>();
    __syncthreads();
    copy_row(min(r + 1, r1 - 1), u ^ 1);  // the last row reloads itself: same count every row
    const unsigned char* cur = smem_raw + u * BUF;
    const h16* Qs = reinterpret_cast<const h16*>(cur);
    const h16* Os = reinterpret_cast<const h16*>(cur + TILE);
    const h16* Ks = reinterpret_cast<const h16*>(cur + 2 * TILE);
    const h16* Vs = reinterpret_cast<const h16*>(cur + 2 * TILE + KVT);
    const float* Ls = reinterpret_cast<const float*>(cur + SOFF);  // lse
    const float* Ds = Ls + N;                                      // -Dsum
    const float* Ms = Ds + N;                                      // key mask
    HFrag<D> kf, vf;
    kf.v = ld8(Ks + klocal * 32 + rsw);
    vf.v = ld8(Vs + klocal * 32 + rsw);
    const bool mk = Ms[k] != 0.f;
    bool any = false;
#pragma unroll
    for (int i = 0; i < JS; ++i)
      if (i * 64 + lane < N) any |= Ms[i * 64 + lane] != 0.f;
    // the row has an unmasked key; every key of this wave is unmasked
    const bool live = __builtin_amdgcn_ballot_w64(any) != 0;
    const bool allk = __builtin_amdgcn_ballot_w64(!mk) == 0;
    f32x4 accK[DT], accV[DT];
#pragma unroll
    for (int i = 0; i < DT; ++i) { accK[i] = z4; accV[i] = z4; }

    // One unit = this wave's 16 keys against 32 queries (block ib, or the
    // 16-query half qs of the last block).  Its LDS operands are read in one
    // batch, and the next unit's batch is issued right after this unit's
    // S / dP products, so the reads are in flight during the exponentials.
    struct Ops {
      h16x8 q[2], o[2];
      float4 l[2], d[2];
    };
    auto load_ops = [&](int ib, Ops& x) __attribute__((always_inline)) {
      const int qb = blk_q0(ib);
#pragma unroll
      for (int qh = 0; qh < 2; ++qh) {
        x.q[qh] = ld8(Qs + (qb + qh * 16 + lk) * 32 + rsw);
        x.o[qh] = ld8(Os + (qb + qh * 16 + lk) * 32 + rsw);
        x.l[qh] = *reinterpret_cast<const float4*>(Ls + qb + qh * 16 + 4 * g);
        x.d[qh] = *reinterpret_cast<const float4*>(Ds + qb + qh * 16 + 4 * g);
      }
    };
    // MODE 0: every key of the wave unmasked (no selects); 1: a masked key
    // gets exponent -inf; 2: fully masked row (p = 1/N, dS = 0)
    auto row_units = [&](auto mode_c) __attribute__((always_inline)) {
      constexpr int MODE = decltype(mode_c)::value;
      Ops cur, nxt;
      load_ops(0, cur);
#pragma unroll
      for (int ib = 0; ib < NB; ++ib) {
        const bool half = HALF && ib == FULL;
        const int qb = blk_q0(ib);
        f32x4 s4[2], dp[2];
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
          f32x4 cs, cd;
          cs[0] = bsl[ib][qh * 4 + 0] - cur.l[qh].x;
          cs[1] = bsl[ib][qh * 4 + 1] - cur.l[qh].y;
          cs[2] = bsl[ib][qh * 4 + 2] - cur.l[qh].z;
          cs[3] = bsl[ib][qh * 4 + 3] - cur.l[qh].w;
          cd[0] = cur.d[qh].x; cd[1] = cur.d[qh].y; cd[2] = cur.d[qh].z; cd[3] = cur.d[qh].w;
          HFrag<D> qa, da;
          qa.v = cur.q[qh];
          da.v = cur.o[qh];
          if constexpr (MODE != 2) {
            s4[qh] = HFrag<D>::mma(qa, kf, cs);  // S + bias - lse
            dp[qh] = HFrag<D>::mma(da, vf, cd);  // dP - Dsum
          }
        }
        if (ib + 1 < NB) load_ops(ib + 1, nxt);
        h16x8 pf, dsf;
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
          const bool on = !half || qh == qs;  // this wave's half of a split block
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            float p, ds;
            if constexpr (MODE == 0) {
              p = fast_exp2(s4[qh][i]);
              ds = p * dp[qh][i];
            } else if constexpr (MODE == 1) {
              p = fast_exp2(mk ? s4[qh][i] : -INFINITY);
              ds = p * dp[qh][i];
            } else {
              p = 1.f / N;
              ds = 0.f;
            }
            if (!on) {
              p = 0.f;
              ds = 0.f;
            }
            pf[qh * 4 + i] = (h16)p;
            dsf[qh * 4 + i] = (h16)ds;
            if constexpr (MODE != 2) dbias[ib][qh * 4 + i] += ds;
          }
        }
#pragma unroll
        for (int dh = 0; dh < DT; ++dh) {
          accV[dh] = mfma16x16x32(tr8(Os, qb, dh), pf, accV[dh]);
          if constexpr (MODE != 2) accK[dh] = mfma16x16x32(tr8(Qs, qb, dh), dsf, accK[dh]);
        }
        if (ib + 1 < NB) cur = nxt;
      }
    };
    if (live && allk) row_units(std::integral_constant<int, 0>{});
    else if (live) row_units(std::integral_constant<int, 1>{});
    else row_units(std::integral_constant<int, 2>{});

    // row done: query group 1 parks its partials, query group 0 adds them
    // and writes dK, dV of its key tile
    if (qs == 1) {
      float* x = Xs + kt_ * (2 * DT * 4 * 64);
#pragma unroll
      for (int dh = 0; dh < DT; ++dh)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[(dh * 4 + i) * 64 + lane] = accK[dh][i];
          x[(DT * 4 + dh * 4 + i) * 64 + lane] = accV[dh][i];
        }
    }
    __syncthreads();
    if (qs == 0) {
      const float* x = Xs + kt_ * (2 * DT * 4 * 64);
      h16* dk = b.dqkvg + ((long)r * N + k) * a.ld + HD + h * D;
      h16* dvp = dk + HD;
      // lane (lk, g) holds channels [4g, 4g+4) and [16+4g, 16+4g+4) of key k;
      // dK is w.r.t. the unscaled k: sum_q dS * q_scaled / log2(e)
#pragma unroll
      for (int dh = 0; dh < DT; ++dh) {
        h16x4 kv, vv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          kv[i] = (h16)((accK[dh][i] + x[(dh * 4 + i) * 64 + lane]) * (1.f / LOG2E));
          vv[i] = (h16)(accV[dh][i] + x[(DT * 4 + dh * 4 + i) * 64 + lane]);
        }
        *reinterpret_cast<h16x4*>(dk + dh * 16 + 4 * g) = kv;
        *reinterpret_cast<h16x4*>(dvp + dh * 16 + 4 * g) = vv;
      }
    }
  }
  if (b.dbias_part == nullptr) return;
  float* part = b.dbias_part + (((long)ch * H + h) * N) * N;
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {
    const int qb = blk_q0(ib);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (ib == FULL && e / 4 != qs) continue;  // the other group's half
      const int qi = qb + (e / 4) * 16 + 4 * g + (e % 4);
      part[(long)qi * N + k] = dbias[ib][e];
    }
  }
}

// dK/dV/dBias for D = 32 and 256 < N <= 512 with direct global -> LDS
// copies, as attn_bwd_dkv_lds_kernel, reorganised around the copy volume:
// every workgroup re-stages each row's Q and dO for its own keys, so at
// L = 512 the staging moved 2.4 GB from L2 a launch and cost about as much
// as the products (531 us with it, 363 us with it taken out).  Here a
// workgroup owns 64 keys (eight waves: four 16-key tiles x two query
// groups, one workgroup a CU), which halves that volume, and the pair bias
// it keeps in registers for all its rows is binary16 as stored (the bias
// gradient sums stay f32).
//
//  * A stage is one 256-query chunk of a row: the chunk's Q and dO tiles,
//    the workgroup's K and V tiles, the chunk's lse and -Dsum and the row's
//    key mask, copied into one of three LDS buffers two stages ahead of its
//    use.  Tiles are 64-byte h16 rows with the 16-byte chunk c of row t
//    stored at chunk c ^ ((t >> 1) & 3).
//  * Every wave issues the same NCOPY copies every stage (spare statistic
//    slots repeat the wave's own copy: the same bytes to the same place), and
//    only query group 0 stores (four dK/dV stores at a row's end), so the
//    wait that opens a stage retires exactly that stage's copies, leaving the
//    next stage's copies and, in query group 0, the previous row's four
//    stores in flight.
//  * Queries and keys past N are read at clamped, in-bounds addresses (a key
//    tile wholly past N computes nothing and writes nothing); what they
//    stage is never read.
template <int NQB>
__global__ __launch_bounds__(512) void attn_bwd_dkv_lds8_kernel(AttnBwdArgs b) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem_raw[];
  constexpr int D = 32, DT = 2;
  constexpr int N = 32 * NQB;             // == a.N (dispatch)
  static_assert(NQB > 8 && NQB <= 16, "256 < N <= 512");
  constexpr int QS = 2, KT = 4, W = 8;    // query groups x 16-key tiles
  constexpr int CQ = 256, NCH = 2;        // queries a stage, stages a row
  constexpr int UPS = CQ / 32 / QS;       // units a wave a stage (4)
  constexpr int NB = UPS * NCH;           // units a wave a row (8)
  constexpr int TILE = CQ * 64;           // bytes of a [CQ][32] h16 tile
  constexpr int KVT = 16 * KT * 64;       // bytes of the K (or V) tile
  constexpr int JSM = (N + 63) / 64;      // 64-key groups of the mask
  constexpr int SOFF = 2 * TILE + 2 * KVT;
  constexpr int BUF = SOFF + 2 * CQ * 4 + JSM * 64 * 4;  // + lse, -Dsum, mask
  constexpr int NT = 2 * (CQ / 16) + 2 * KT;  // 1 KB tile copies a stage
  static_assert(NT % W == 0, "tile copies: the same count a wave");
  constexpr int NCT = NT / W;                  // a wave's (5)
  constexpr int TS = 2 * (CQ / 64) + JSM;      // 256-byte statistic copies a stage
  static_assert(TS > W && TS <= 2 * W, "two statistic copies a wave");
  constexpr int NCOPY = NCT + 2;
  static_assert(NCOPY + 4 < 16, "vmcnt immediate");
  const AttnArgs& a = b.f;
  const int H = a.H;
  float* Xs = reinterpret_cast<float*>(smem_raw + 3 * BUF);  // [KT][K,V][DT*4][64], query group 1

  constexpr int NKW = (N + 16 * KT - 1) / (16 * KT);
  const long G = (long)((a.R + b.rows_per_chunk - 1) / b.rows_per_chunk) * H * NKW;
  const int bid = (int)xcd_block(G);
  if (bid >= G) return;
  const int kw = bid % NKW;
  const int h = (bid / NKW) % H;
  const int ch = bid / (NKW * H);
  const int r0 = ch * b.rows_per_chunk;
  const int r1 = min(a.R, r0 + b.rows_per_chunk);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int kt_ = wave % KT, qs = wave / KT;
  const int lk = lane & 15, g = lane >> 4;
  const int klocal = kt_ * 16 + lk;
  const bool kon = kw * 16 * KT + kt_ * 16 < N;  // the wave's key tile exists (wave-uniform)
  const int k = min(kw * 16 * KT + klocal, N - 1);
  const bool stores = qs == 0 && kon;  // writes dK, dV at each row's end
  const long HD = (long)H * D;
  const unsigned lds0 = lds_addr(smem_raw);

  // unit ib = UPS c + i of this wave: 32-query block 8 c + qs + QS i (rows
  // ql = 32 (qs + QS i) of chunk c's tiles); the bias column k at its
  // queries (binary16), the bias-gradient sums (f32)
  h16x8 bsh[NB];
  float dbias[NB][8];
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {
    const int blk = min(8 * (ib / UPS) + qs + QS * (ib % UPS), NQB - 1);  // past N: never used
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      bsh[ib][e] = a.bias[bias_frag_index(h, blk * 32 + (e / 4) * 16 + 4 * g + (e % 4), k, N)];
      dbias[ib][e] = 0.f;
    }
  }
  // all in flight together, then resident before the first copy is issued:
  // a first use inside the row loop would wait for every copy in flight
  // (vmcnt retires in order)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) asm volatile("" ::"v"(bsh[ib]));

  // Tile copy j (1 KB): rows 16 jr .. 16 jr + 15 of tile Q (j < 16), dO
  // (j < 32), K, V.  Lane i writes physical chunk i & 3 of row 16 jr + i / 4
  // from the logical chunk the swizzle puts there.  Wave w issues copies
  // w + 8 i.
  // (the per-lane offsets are recomputed at each stage: kept, they would
  // take registers the bias-gradient sums need)
  auto tile_voff = [&](int i, int c, int lane) __attribute__((always_inline)) -> unsigned {
    const int j = wave + W * i;
    const int tile = j < CQ / 8 ? j / (CQ / 16) : 2 + (j - CQ / 8) / KT;  // Q, dO, K, V
    const int jr = j < CQ / 8 ? j % (CQ / 16) : (j - CQ / 8) % KT;
    const int row = jr * 16 + (lane >> 2);
    const int c8 = ((lane & 3) ^ ((row >> 1) & 3)) * 8;
    const int ld = tile == 1 ? a.ldo : a.ld;
    // a query of chunk c, or a key of the workgroup's tile
    const int tok = tile < 2 ? min(c * CQ + row, N - 1) : min(kw * 16 * KT + row, N - 1);
    return (unsigned)((tok * ld + c8) * 2);
  };
  unsigned sdst[NCT];
  long soff[NCT];
  bool sdo[NCT];
#pragma unroll
  for (int i = 0; i < NCT; ++i) {
    const int j = wave + W * i;
    const int tile = j < CQ / 8 ? j / (CQ / 16) : 2 + (j - CQ / 8) / KT;
    const int jr = j < CQ / 8 ? j % (CQ / 16) : (j - CQ / 8) % KT;
    sdo[i] = tile == 1;
    soff[i] = tile < 2 ? (long)h * D * 2 : ((tile - 1) * HD + h * D) * 2;
    sdst[i] = (tile < 2 ? tile * TILE : 2 * TILE + (tile - 2) * KVT) + jr * 1024;
  }
  // Statistic copy j (256 bytes): lse (j < 4), -Dsum (j < 8) of the chunk's
  // queries, then the row's key mask; waves w and w + 8 (a slot past TS
  // repeats the wave's first).
  auto stat_voff = [&](int i, int c, int lane) __attribute__((always_inline)) -> unsigned {
    int j = wave + W * i;
    if (j >= TS) j -= W;
    const int which = j < CQ / 64 ? 0 : j < 2 * (CQ / 64) ? 1 : 2;
    const int js = which < 2 ? j % (CQ / 64) : j - 2 * (CQ / 64);
    const int q = which < 2 ? min(c * CQ + js * 64 + lane, N - 1) : min(js * 64 + lane, N - 1);
    return which == 2 ? (unsigned)(q * a.mask_sk * 4) : (unsigned)(q * 4);
  };
  unsigned ssdst[2];
  int swhich[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    int j = wave + W * i;
    if (j >= TS) j -= W;
    const int which = j < CQ / 64 ? 0 : j < 2 * (CQ / 64) ? 1 : 2;
    const int js = which < 2 ? j % (CQ / 64) : j - 2 * (CQ / 64);
    swhich[i] = which;
    ssdst[i] = SOFF + (which < 2 ? which * CQ * 4 : 2 * CQ * 4) + js * 256;
  }
  // the copies of stage (row r, chunk C) into buffer u
  auto copy_stage = [&](int r, auto c_, int u) __attribute__((always_inline)) {
    constexpr int C = decltype(c_)::value;
    const unsigned base = lds0 + u * BUF;
    int ln = lane;  // opaque: the offsets are recomputed here, not hoisted into registers
    asm volatile("" : "+v"(ln));
    const char* qrow = reinterpret_cast<const char*>(a.qkvg + (long)r * N * a.ld);
    const char* orow = reinterpret_cast<const char*>(b.dO + (long)r * N * a.ldo);
#pragma unroll
    for (int i = 0; i < NCT; ++i) dma16s(tile_voff(i, C, ln), (sdo[i] ? orow : qrow) + soff[i], base + sdst[i]);
    const long srow = ((long)r * H + h) * N;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const float* sb = swhich[i] == 0 ? a.lse + srow
                      : swhich[i] == 1 ? b.nDsum + srow
                                       : a.mask + (long)r * a.mask_sr;
      dma4s(stat_voff(i, C, ln), sb, base + ssdst[i]);
    }
  };

  // lane-constant swizzled offsets (h16 units): row reads at rows = lk
  // (mod 16), transposed reads at rows 4g + lk/4 (mod 16)
  const int rsw = ((g ^ ((lk >> 1) & 3)) << 3);
  const int trow = 4 * g + (lk >> 2);
  const int tsw0 = (((lk & 3) >> 1) ^ ((trow >> 1) & 3)) * 8 + 4 * (lk & 1);       // columns 0..15
  const int tsw1 = ((2 + ((lk & 3) >> 1)) ^ ((trow >> 1) & 3)) * 8 + 4 * (lk & 1);  // columns 16..31
  auto tr8 = [&](const h16* T, int r0_, int dh) __attribute__((always_inline)) -> h16x8 {
    const h16* p = T + (r0_ + trow) * 32 + (dh ? tsw1 : tsw0);
    const h16x4 x = __builtin_bit_cast(h16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
    const h16x4 y =
        __builtin_bit_cast(h16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(p + 16 * 32)));
    h16x8 v;
    v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
    v[4] = y[0]; v[5] = y[1]; v[6] = y[2]; v[7] = y[3];
    return v;
  };

  const int nrow = r1 - r0;
  copy_stage(r0, std::integral_constant<int, 0>{}, 0);
  copy_stage(r0, std::integral_constant<int, 1>{}, 1);
  const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
  f32x4 accK[DT], accV[DT];
  int u = 0;  // buffer of the current stage
  for (int rr = 0; rr < nrow; ++rr) {
    const int r = r0 + rr;
#pragma unroll
    for (int i = 0; i < DT; ++i) { accK[i] = z4; accV[i] = z4; }
    auto stage = [&](auto c_) __attribute__((always_inline)) {
      constexpr int C = decltype(c_)::value;
      // this stage's copies are in; the next stage's (and in a storing
      // wave the previous row's four dK/dV stores) may still be in flight
      if (stores && rr > 0) wait_vm<NCOPY + 4>();
      else wait_vm<NCOPY>();
      __syncthreads();
      // two stages ahead: (row r + 1, chunk C) -- the last row reloads itself
      copy_stage(min(r + 1, r1 - 1), c_, u >= 1 ? u - 1 : 2);
      const unsigned char* cur = smem_raw + u * BUF;
      u = u == 2 ? 0 : u + 1;
      if (!kon) return;
      const h16* Qs = reinterpret_cast<const h16*>(cur);
      const h16* Os = reinterpret_cast<const h16*>(cur + TILE);
      const h16* Ks = reinterpret_cast<const h16*>(cur + 2 * TILE);
      const h16* Vs = reinterpret_cast<const h16*>(cur + 2 * TILE + KVT);
      const float* Ls = reinterpret_cast<const float*>(cur + SOFF);  // lse of the chunk
      const float* Ds = Ls + CQ;                                     // -Dsum of the chunk
      const float* Ms = Ds + CQ;                                     // key mask of the row
      HFrag<D> kf, vf;
      kf.v = ld8(Ks + klocal * 32 + rsw);
      vf.v = ld8(Vs + klocal * 32 + rsw);
      const bool mk = Ms[k] != 0.f;
      bool any = false;
#pragma unroll
      for (int i = 0; i < JSM; ++i)
        if (i * 64 + lane < N) any |= Ms[i * 64 + lane] != 0.f;
      const bool live = __builtin_amdgcn_ballot_w64(any) != 0;
      const bool allk = __builtin_amdgcn_ballot_w64(!mk) == 0;

      struct Ops {
        h16x8 q[2], o[2];
        float4 l[2], d[2];
      };
      auto load_ops = [&](int ql, Ops& x) __attribute__((always_inline)) {
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
          x.q[qh] = ld8(Qs + (ql + qh * 16 + lk) * 32 + rsw);
          x.o[qh] = ld8(Os + (ql + qh * 16 + lk) * 32 + rsw);
          x.l[qh] = *reinterpret_cast<const float4*>(Ls + ql + qh * 16 + 4 * g);
          x.d[qh] = *reinterpret_cast<const float4*>(Ds + ql + qh * 16 + 4 * g);
        }
      };
      // MODE 0: every key of the wave unmasked; 1: a masked key gets
      // exponent -inf; 2: fully masked row (p = 1/N, dS = 0)
      auto units = [&](auto mode_c) __attribute__((always_inline)) {
        constexpr int MODE = decltype(mode_c)::value;
#pragma unroll
        for (int i = 0; i < UPS; ++i) {
          if (8 * C + qs + QS * i >= NQB) continue;  // wave-uniform
          const int ib = UPS * C + i;
          const int ql = (qs + QS * i) * 32;
          // the bias stays binary16 between uses: converted here, not
          // hoisted out of the row loop as 64 f32 registers
          asm volatile("" : "+v"(bsh[ib]));
          Ops cur_;
          load_ops(ql, cur_);
          f32x4 s4[2], dp[2];
#pragma unroll
          for (int qh = 0; qh < 2; ++qh) {
            f32x4 cs, cd;
            cs[0] = (float)bsh[ib][qh * 4 + 0] - cur_.l[qh].x;
            cs[1] = (float)bsh[ib][qh * 4 + 1] - cur_.l[qh].y;
            cs[2] = (float)bsh[ib][qh * 4 + 2] - cur_.l[qh].z;
            cs[3] = (float)bsh[ib][qh * 4 + 3] - cur_.l[qh].w;
            cd[0] = cur_.d[qh].x; cd[1] = cur_.d[qh].y; cd[2] = cur_.d[qh].z; cd[3] = cur_.d[qh].w;
            HFrag<D> qa, da;
            qa.v = cur_.q[qh];
            da.v = cur_.o[qh];
            if constexpr (MODE != 2) {
              s4[qh] = HFrag<D>::mma(qa, kf, cs);  // S + bias - lse
              dp[qh] = HFrag<D>::mma(da, vf, cd);  // dP - Dsum
            }
          }
          h16x8 pf, dsf;
#pragma unroll
          for (int qh = 0; qh < 2; ++qh)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              float p, ds;
              if constexpr (MODE == 0) {
                p = fast_exp2(s4[qh][e]);
                ds = p * dp[qh][e];
              } else if constexpr (MODE == 1) {
                p = fast_exp2(mk ? s4[qh][e] : -INFINITY);
                ds = p * dp[qh][e];
              } else {
                p = 1.f / N;
                ds = 0.f;
              }
              pf[qh * 4 + e] = (h16)p;
              dsf[qh * 4 + e] = (h16)ds;
              if constexpr (MODE != 2) dbias[ib][qh * 4 + e] += ds;
            }
#pragma unroll
          for (int dh = 0; dh < DT; ++dh) {
            accV[dh] = mfma16x16x32(tr8(Os, ql, dh), pf, accV[dh]);
            if constexpr (MODE != 2) accK[dh] = mfma16x16x32(tr8(Qs, ql, dh), dsf, accK[dh]);
          }
        }
      };
      if (live && allk) units(std::integral_constant<int, 0>{});
      else if (live) units(std::integral_constant<int, 1>{});
      else units(std::integral_constant<int, 2>{});
    };
    stage(std::integral_constant<int, 0>{});
    stage(std::integral_constant<int, 1>{});

    // row done: query group 1 parks its partials, query group 0 adds them
    // and writes dK, dV of its key tile
    if (qs == 1 && kon) {
      float* x = Xs + kt_ * (2 * DT * 4 * 64);
#pragma unroll
      for (int dh = 0; dh < DT; ++dh)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          x[(dh * 4 + i) * 64 + lane] = accK[dh][i];
          x[(DT * 4 + dh * 4 + i) * 64 + lane] = accV[dh][i];
        }
    }
    __syncthreads();
    if (stores) {
      const float* x = Xs + kt_ * (2 * DT * 4 * 64);
      h16* dk = b.dqkvg + ((long)r * N + k) * a.ld + HD + h * D;
      h16* dvp = dk + HD;
      // lane (lk, g) holds channels [4g, 4g+4) and [16+4g, 16+4g+4) of key k;
      // dK is w.r.t. the unscaled k: sum_q dS * q_scaled / log2(e)
#pragma unroll
      for (int dh = 0; dh < DT; ++dh) {
        h16x4 kv, vv;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          kv[i] = (h16)((accK[dh][i] + x[(dh * 4 + i) * 64 + lane]) * (1.f / LOG2E));
          vv[i] = (h16)(accV[dh][i] + x[(DT * 4 + dh * 4 + i) * 64 + lane]);
        }
        *reinterpret_cast<h16x4*>(dk + dh * 16 + 4 * g) = kv;
        *reinterpret_cast<h16x4*>(dvp + dh * 16 + 4 * g) = vv;
      }
    }
  }
  wait_vm<0>();  // the last stages' copies land before the workgroup's LDS is released
  if (b.dbias_part == nullptr || !kon) return;
  float* part = b.dbias_part + (((long)ch * H + h) * N) * N;
#pragma unroll
  for (int ib = 0; ib < NB; ++ib) {
    const int blk = 8 * (ib / UPS) + qs + QS * (ib % UPS);
    if (blk >= NQB) continue;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int qi = blk * 32 + (e / 4) * 16 + 4 * g + (e % 4);
      part[(long)qi * N + k] = dbias[ib][e];
    }
  }
}

__global__ void attn_dbias_reduce_kernel(const float* __restrict__ part, int nch,
                                         long n, float* __restrict__ out) {
  const long i = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  // eight partials loaded at a time (in flight together), added in chunk order
  float s = 0.f;
  int c = 0;
  for (; c + 8 <= nch; c += 8) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = part[(long)(c + u) * n + i];
#pragma unroll
    for (int u = 0; u < 8; ++u) s += v[u];
  }
  for (; c < nch; ++c) s += part[(long)c * n + i];
  out[i] = s;
}

// ------------------------------------------------------------------ launchers

int attn_bwd_nchunk(int R, int rows_per_chunk) {
  return (R + rows_per_chunk - 1) / rows_per_chunk;
}

// Rows per workgroup of the row-chunk forward: (chunk, head, 64 queries)
// workgroups at two per CU (register bound), one round of 2 x CUs.
int attn_fwd_rows_per_chunk(int R, int N, int H) {
  const long per_chunk = (long)H * ((N + 63) / 64);
  const long nch = std::max(1L, 2L * device_cus() / per_chunk);
  return (int)std::max(1L, ((long)R + nch - 1) / nch);
}

// Rows per bias-gradient chunk.  A chunk is H * N / (keys a workgroup) workgroups of
// the dK/dV kernel, which is register bound at two workgroups per CU; the
// chunk count is the largest that fits one round of 2 x CUs workgroups, so
// no second, partly empty round follows (N = 224, H = 4 on 256 CUs: 18
// chunks of 13 rows).  Fewer chunks also mean fewer [nchunk][H][N][N]
// partials to write and add.
int attn_rows_per_chunk(int R, int N, int H, int D) {
  // keys a workgroup: 64 in the D = 32 kernel for 256 < N <= 512, 32 to
  // N = 768, 16 beyond
  const int kpw = D == 32 && N > 256 && N <= 512 ? 64 : N > 768 ? 16 : 32;
  const long per_chunk = (long)H * ((N + kpw - 1) / kpw);
  const long per_cu = N > 256 ? 1 : 2;  // eight-wave workgroups beyond 256
  const long slots = per_cu * device_cus();
  long nch = std::max(1L, slots / per_chunk);
  // a round that leaves many CUs idle (N = 768: 2 chunks of 96 workgroups
  // fill 192 of 256 CUs) is worth more chunks: the smallest count, up to four
  // rounds, whose rounds are at least 95% full
  auto fill = [&](long c) {
    const long w = c * per_chunk;
    return (double)w / (double)(slots * ((w + slots - 1) / slots));
  };
  if (fill(nch) < 0.85) {
    for (long c = nch + 1; c * per_chunk <= 4 * slots && c <= R; ++c)
      if (fill(c) >= 0.95) {
        nch = c;
        break;
      }
  }
  nch = std::min<long>(nch, R);
  return (int)std::max(1L, ((long)R + nch - 1) / nch);
}

// Calls f(std::integral_constant<int, nb>) for nb = N/32 in 1..32: every
// kernel is instantiated for its exact number of 32-blocks.
template <class F>
static void with_blocks(int nb, F&& f) {
  switch (nb) {
#define BC2N_NB(v) case v: f(std::integral_constant<int, v>()); break;
    BC2N_NB(1) BC2N_NB(2) BC2N_NB(3) BC2N_NB(4) BC2N_NB(5) BC2N_NB(6) BC2N_NB(7) BC2N_NB(8)
    BC2N_NB(9) BC2N_NB(10) BC2N_NB(11) BC2N_NB(12) BC2N_NB(13) BC2N_NB(14) BC2N_NB(15)
    BC2N_NB(16) BC2N_NB(17) BC2N_NB(18) BC2N_NB(19) BC2N_NB(20) BC2N_NB(21) BC2N_NB(22)
    BC2N_NB(23) BC2N_NB(24) BC2N_NB(25) BC2N_NB(26) BC2N_NB(27) BC2N_NB(28) BC2N_NB(29)
    BC2N_NB(30) BC2N_NB(31) BC2N_NB(32)
#undef BC2N_NB
    default: throw std::runtime_error("attention: N/32 out of range");
  }
}

// Timer names per launch site: [kernel][0 triangle D=32, 1 MSA row, 2 D=16]
static const char* const kTimerNames[5][3] = {
    {"attn_fwd", "msarow.attn_fwd", "tpl.attn_fwd"},
    {"attn_gate_bwd", "msarow.attn_gate_bwd", "tpl.attn_gate_bwd"},
    {"attn_bwd_dq", "msarow.attn_bwd_dq", "tpl.attn_bwd_dq"},
    {"attn_bwd_dkv", "msarow.attn_bwd_dkv", "tpl.attn_bwd_dkv"},
    {"attn_dbias_reduce", "msarow.attn_dbias_reduce", "tpl.attn_dbias_reduce"}};
static const char* timer_name(int kernel, const AttnArgs& a) {
  return kTimerNames[kernel][a.site == 1 ? 1 : (a.D == 16 ? 2 : 0)];
}

// keys per LDS chunk of the forward / dQ kernels, rows per chunk of dK/dV
static int attn_chunk(int N) { return N < 256 ? N : 256; }

static void attn_check(const AttnArgs& a) {
  if (a.D != 32 && a.D != 16) throw std::runtime_error("attention: head width must be 16 or 32");
  if (a.N <= 0 || a.N % 32 != 0) throw std::runtime_error("attention: N must be a positive multiple of 32");
  if (a.N > 1024) throw std::runtime_error("attention: N > 1024 not supported");
  if (a.ld % 8 != 0 || a.ldo % 8 != 0) throw std::runtime_error("attention: row strides must be multiples of 8");
  if (!a.qkvg || !a.mask || !a.lse || !a.o) throw std::runtime_error("attention: missing operand");
}

template <int D>
static void attn_fwd_t(hipStream_t st, const AttnArgs& a) {
  const int nqb = (a.N + 63) / 64;
  KTimed kt(timer_name(0, a), st);
  if (a.N <= 256) {
    if (!a.bias) throw std::runtime_error("attention: the row-chunk forward needs the pair bias");
    const int rpc = attn_fwd_rows_per_chunk(a.R, a.N, a.H);
    const long nch = (a.R + rpc - 1) / rpc;
    const size_t lds = (size_t)(2 * a.N + 2 * 64) * lds_ld<D>() * 2 + (size_t)a.N * 8;
    const dim3 grid(xcd_grid(nch * a.H * nqb));
    with_blocks(a.N / 32, [&](auto nb) {
      if constexpr (decltype(nb)::value <= 8)
        hipLaunchKernelGGL((attn_fwd_rows_kernel<D, decltype(nb)::value>), grid, dim3(256), lds, st,
                           a, rpc);
    });
    return;
  }
  if (!a.bias) throw std::runtime_error("attention: the chunked forward needs the pair bias");
  // one 128-key K/V buffer + the row's key mask (two floats a key); eight
  // waves (128 queries) a workgroup, so each row's K/V is read by N / 128
  // workgroups
  constexpr int QW = 8;
  const size_t lds = (size_t)128 * lds_ld<D>() * 2 * 2 + (size_t)a.N * 8;
  const dim3 grid(xcd_grid((long)a.R * a.H * ((a.N + 16 * QW - 1) / (16 * QW))));
  with_blocks(a.N / 32, [&](auto nb) {
    hipLaunchKernelGGL((attn_fwd_kernel<D, decltype(nb)::value, QW>), grid, dim3(64 * QW), lds, st,
                       a);
  });
}

void attn_fwd(hipStream_t st, const AttnArgs& a) {
  attn_check(a);
  if (!a.og) throw std::runtime_error("attention: missing gated output");
  if (a.D == 32) attn_fwd_t<32>(st, a);
  else attn_fwd_t<16>(st, a);
}

template <int D>
static void attn_bwd_t(hipStream_t st, const AttnBwdArgs& b0) {
  // one chunk of rows (the MSA row attention of one sequence): the dK/dV
  // kernel's partial is the whole bias gradient, written in place
  AttnBwdArgs b = b0;
  const bool one_chunk = attn_bwd_nchunk(b.f.R, b.rows_per_chunk) == 1;
  if (one_chunk && b.dbias && b.f.bias) b.dbias_part = b.dbias;
  const AttnArgs& a = b.f;
  const long tot = (long)a.R * a.N * a.H;
  if (!b.gate_done) {
    KTimed kt(timer_name(1, a), st);
    const long per = 256 / (D / 8);
    hipLaunchKernelGGL((attn_gate_bwd_kernel<D>), dim3((unsigned)((tot + per - 1) / per)),
                       dim3(256), 0, st, b);
  }
  const int nqb = (a.N + 63) / 64;
  if (a.N <= 256) {
    if (!a.bias) throw std::runtime_error("attention: the row-chunk dQ needs the pair bias");
    const int rpc = attn_fwd_rows_per_chunk(a.R, a.N, a.H);
    const long nch = (a.R + rpc - 1) / rpc;
    const size_t lds = (size_t)(2 * a.N + 2 * 64) * lds_ld<D>() * 2 + (size_t)(a.N + 2 * 64) * 4;
    KTimed kt(timer_name(2, a), st);
    const dim3 grid(xcd_grid(nch * a.H * nqb));
    with_blocks(a.N / 32, [&](auto nb) {
      if constexpr (decltype(nb)::value <= 8)
        hipLaunchKernelGGL((attn_bwd_dq_rows_kernel<D, decltype(nb)::value>), grid, dim3(256), lds,
                           st, b, rpc);
    });
  } else {
    if (!a.bias) throw std::runtime_error("attention: the chunked dQ needs the pair bias");
    const size_t lds_q = (size_t)attn_chunk(a.N) * lds_ld<D>() * 2 * 2 + (size_t)a.N * 4;
    KTimed kt(timer_name(2, a), st);
    constexpr int QW = 8;  // 128 queries a workgroup, as the forward
    const dim3 grid(xcd_grid((long)a.R * a.H * ((a.N + 16 * QW - 1) / (16 * QW))));
    with_blocks(a.N / 32, [&](auto nb) {
      hipLaunchKernelGGL((attn_bwd_dq_kernel<D, decltype(nb)::value, QW>), grid, dim3(64 * QW),
                         lds_q, st, b);
    });
  }
  const int nch = attn_bwd_nchunk(a.R, b.rows_per_chunk);
  // waves W, query groups QS and key tiles KT per workgroup, as in the kernel
  const int W = a.N > 256 ? 8 : 4;
  const int QS = a.N > 768 ? 8 : a.N > 256 ? 4 : 2, KT = W / QS;
  const int nkw = a.N / (16 * KT);
  const size_t lds_k = (size_t)attn_chunk(a.N) * lds_ld<D>() * 2 * 2 + (size_t)a.N * 4 * 3 +
                       (size_t)(QS - 1) * KT * 2 * (D / 16) * 4 * 64 * 4 +
                       (size_t)2 * 16 * KT * lds_ld<D>() * 2;
  {
    KTimed kt(timer_name(3, a), st);
    const dim3 grid(xcd_grid((long)nch * a.H * nkw));
    if constexpr (D == 32) {
      if (a.N <= 256 && a.bias) {
        // two row buffers (Q, dO tiles + lse, -Dsum, mask) + 4 waves' partials
        const size_t lds = (size_t)2 * (2 * a.N * 64 + 3 * a.N * 4) + (size_t)4 * 2 * 2 * 4 * 64 * 4;
        with_blocks(a.N / 32, [&](auto nb) {
          if constexpr (decltype(nb)::value <= 8)
            hipLaunchKernelGGL((attn_bwd_dkv_lds_kernel<decltype(nb)::value>), grid, dim3(256), lds,
                               st, b);
        });
        goto dkv_done;
      }
      if (a.N > 256 && a.N <= 512 && a.bias) {
        // three stage buffers (Q, dO chunk tiles, K, V tiles, lse, -Dsum,
        // mask) + query group 1's partials
        const size_t buf = (size_t)2 * 256 * 64 + 2 * 64 * 64 + 2 * 256 * 4 + (size_t)((a.N + 63) / 64) * 64 * 4;
        const size_t lds = 3 * buf + (size_t)4 * 2 * 2 * 4 * 64 * 4;
        const dim3 grid8(xcd_grid((long)nch * a.H * ((a.N + 63) / 64)));  // 64 keys a workgroup
        with_blocks(a.N / 32, [&](auto nb) {
          if constexpr (decltype(nb)::value > 8 && decltype(nb)::value <= 16)
            hipLaunchKernelGGL((attn_bwd_dkv_lds8_kernel<decltype(nb)::value>), grid8, dim3(512), lds,
                               st, b);
        });
        goto dkv_done;
      }
    }
    with_blocks(a.N / 32, [&](auto nb) {
      constexpr int NB = decltype(nb)::value;
      hipLaunchKernelGGL((attn_bwd_dkv_kernel<D, NB, (NB > 8 ? 8 : 4), (NB > 24 ? 8 : NB > 8 ? 4 : 2)>),
                         grid, dim3(64 * W), lds_k, st, b);
    });
  }
dkv_done:
  if (b.dbias && a.bias && !one_chunk && !b.dbias_deferred) {
    if (!b.dbias_part) throw std::runtime_error("attention bwd: missing dbias scratch");
    const long n = (long)a.H * a.N * a.N;
    KTimed kt(timer_name(4, a), st);
    hipLaunchKernelGGL(attn_dbias_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st,
                       b.dbias_part, nch, n, b.dbias);
  }
}

void attn_bwd(hipStream_t st, const AttnBwdArgs& b) {
  attn_check(b.f);
  if ((!b.dog && !b.gate_done) || !b.dO || !b.nDsum || !b.dqkvg)
    throw std::runtime_error("attention bwd: missing operand");
  if (b.f.D == 32) attn_bwd_t<32>(st, b);
  else attn_bwd_t<16>(st, b);
}

}  // namespace bc2n
