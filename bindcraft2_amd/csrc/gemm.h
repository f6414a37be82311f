// LDS-tiled binary16 MFMA GEMM for gfx950 with fused, caller-supplied epilogues.
//
//   C_b[m, n] = sum_k A_b[m, k] * B_b[n, k]        (f32 accumulation)
//
// A and B are each either K-contiguous (row-major [rows][K]) or
// row-contiguous (stored [K][rows]); the tile loader transposes the second
// form on its way into LDS, so the MFMA fragments are always read the same
// way.  A 256-thread workgroup (4 waves, 2x2) owns a BM x BN tile; each wave
// owns (BM/2) x (BN/2) as a grid of 16x16 MFMA tiles fed by
// v_mfma_f32_16x16x32_f16.  K is walked in BK steps with a register prefetch
// of the next step's tile: 32-deep steps (K <= 128) into a second LDS buffer,
// 64-deep steps into the one buffer after a barrier, so that either way the
// operand buffers take at most 40 KB and four workgroups share a CU.
//
// Epilogue: the f32 accumulator tile is staged through LDS (reusing the
// operand buffers, half a tile per pass) and handed to the epilogue as
// vectors of 8, either 8 consecutive columns of one row (`row`, the default)
// or 8 consecutive rows of one column (`col`, when `col_mode(n0)` says so for
// the tile starting at column n0 -- channel-major outputs).  Every global
// store of an epilogue is therefore a 16- or 32-byte vector.
#pragma once
#include "common.h"
#include "runtime.h"
#include <stdexcept>
#include <string>
#include <type_traits>

namespace bc2n {

struct GemmArgs {
  int M = 0, N = 0, K = 0, batch = 1;
  // > 0 (the sliced launch): the accumulators fold into the result every
  // kslice of K, in order, giving the bits of a split-K launch of kslice
  // slices summed by gemm_splitk_epi, on a grid of the tiles alone
  int kslice = 0;
  const h16* A = nullptr;
  long a_sm = 0, a_sk = 0, a_sb = 0;  // element strides; a_sm==1 or a_sk==1
  const h16* B = nullptr;
  long b_sn = 0, b_sk = 0, b_sb = 0;  // element strides; b_sn==1 or b_sk==1
};

// ------------------------------------------------------------ vector helpers
__device__ __forceinline__ void ld_f8(const float* p, float (&v)[8]) {
  const float4 a = reinterpret_cast<const float4*>(p)[0];
  const float4 b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
__device__ __forceinline__ void st_f8(float* p, const float (&v)[8]) {
  reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
}
__device__ __forceinline__ void ld_h8f(const h16* p, float (&v)[8]) {
  const h16x8 a = ld8(p);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = (float)a[e];
}
// Epilogue stores round with saturation (f2h_sat): the backward's tensors
// are scaled cotangents, and a masked row may hold a huge finite value that
// a zero mask removes later.
__device__ __forceinline__ void st_h8f(h16* p, const float (&v)[8]) {
  h16x8 a;
#pragma unroll
  for (int e = 0; e < 8; ++e) a[e] = f2h_sat(v[e]);
  st8(p, a);
}
template <class T>
__device__ __forceinline__ void st_any8(T* p, const float (&v)[8]);
template <>
__device__ __forceinline__ void st_any8<float>(float* p, const float (&v)[8]) { st_f8(p, v); }
template <>
__device__ __forceinline__ void st_any8<h16>(h16* p, const float (&v)[8]) { st_h8f(p, v); }
template <class T>
__device__ __forceinline__ void ld_any8(const T* p, float (&v)[8]);
template <>
__device__ __forceinline__ void ld_any8<float>(const float* p, float (&v)[8]) { ld_f8(p, v); }
template <>
__device__ __forceinline__ void ld_any8<h16>(const h16* p, float (&v)[8]) { ld_h8f(p, v); }

// An epilogue with kTwoPhase = true runs both modes on a column-mode tile:
// first `col` (which may rewrite the staged tile through its pointer), then,
// after a barrier, `row` over the rewritten tile.
template <class E, class = void>
struct epi_two_phase : std::false_type {};
template <class E>
struct epi_two_phase<E, std::void_t<decltype(E::kTwoPhase)>> : std::bool_constant<E::kTwoPhase> {};

// An epilogue with kRowBlock = true takes each staged half tile whole: all
// 256 threads call block<WM>(b, mb, T, ldt, tid) over its WM rows x BN
// columns (rows mb.., row stride ldt in LDS), for row-wise reductions.  It
// needs every column of a row in one tile (N == BN, checked on the host).
template <class E, class = void>
struct epi_row_block : std::false_type {};
template <class E>
struct epi_row_block<E, std::void_t<decltype(E::kRowBlock)>> : std::bool_constant<E::kRowBlock> {};

// A row-block epilogue with kProRowFloats > 0 also has a prologue:
// prologue<BM>(m0, pro, tid) fills pro[BM][kProRowFloats] (LDS) for the
// tile's rows while the first operand tiles load, and block() then takes
// pro + (mb - m0) * kProRowFloats as its last argument.
template <class E, class = void>
struct epi_pro_floats : std::integral_constant<int, 0> {};
template <class E>
struct epi_pro_floats<E, std::void_t<decltype(E::kProRowFloats)>>
    : std::integral_constant<int, E::kProRowFloats> {};

// Base of every epilogue: row mode only.
struct EpiRows {
  static constexpr bool kHasCol = false;
  __device__ __forceinline__ bool col_mode(int) const { return false; }
  __device__ __forceinline__ void col(int, int, int, const float (&)[8], const float*, int) const {}
};

// A-operand loaders.  The default reads h16 A as the strides say; the
// others build the K-contiguous A tile from f32 rows on the fly, so the
// elementwise pass that would have written A to memory disappears.  A loader
// with a side output (kSide) writes it as it loads, which is exact only when
// every A element is loaded once: a single tile column (N <= BN), checked on
// the host.
struct ALoadDirect {
  static constexpr bool kDirect = true;
  static constexpr bool kSide = false;
  __device__ __forceinline__ h16x8 operator()(int, int, int) const { return h16x8{}; }
};

// A[m][k] = h16(s * src[src(m)][k] * tbl[(m % nt) * C + k]); src(m)
// transposes the nt x nt grid when `transpose`; tbl may be null (no dropout);
// s = *mul, the backward's cotangent scale (1 when mul is null).
struct ALoadScaledRows {
  static constexpr bool kDirect = false;
  static constexpr bool kSide = false;
  const float* src;
  const float* tbl;
  int nt, C;
  bool transpose;
  const float* mul = nullptr;
  __device__ __forceinline__ h16x8 operator()(int, int m, int k) const {
    const long s = transpose ? (long)(m % nt) * nt + m / nt : m;
    float v[8];
    ld_f8(src + s * C + k, v);
    const float sm = mul ? *mul : 1.f;
    if (tbl) {
      float t[8];
      ld_f8(tbl + (long)(m % nt) * C + k, t);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] *= t[e] * sm;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] *= sm;
    }
    h16x8 r;
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = f2h_sat(v[e]);
    return r;
  }
};

// x32 operand from a k-major LDS tile T[k][col] (row stride ld h16, ld % 4
// == 0): lane l gets column c0 + l%16 at k = r0 + {4g..4g+3, 16+4g..16+4g+3}
// (g = l/16), by two ds_read_b64_tr_b16 (each the column read of a 4 x 16
// block: within a 16-lane group, lane m addresses the 8 bytes at row
// r0 + 4g + m/4, columns c0 + 4(m%4) .. +3).
typedef short gemm_s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) gemm_s16x4 gemm_lds_s16x4;
__device__ __forceinline__ h16x4 gemm_tr4(const h16* T, int ld, int r0, int c0, int lane) {
  const int g = lane >> 4, m = lane & 15;
  const h16* p = T + (r0 + 4 * g + (m >> 2)) * ld + c0 + 4 * (m & 3);
  return __builtin_bit_cast(h16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((gemm_lds_s16x4*)p));
}
__device__ __forceinline__ h16x8 gemm_tr8(const h16* T, int ld, int r0, int c0, int lane) {
  const h16x4 a = gemm_tr4(T, ld, r0, c0, lane), b = gemm_tr4(T, ld, r0 + 16, c0, lane);
  h16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

template <int BM, int BN, int BK>
struct GemmSmem {
  static constexpr int LDK = BK + 8;
  // 64-deep steps (long K) keep one operand buffer and pay a second barrier
  // per step, so four workgroups still fit a CU; 32-deep steps double-buffer
  static constexpr int NBUF = BK >= 64 ? 1 : 2;
  // A k-major operand tile is kept k-major, [BK][rows + 16]: a row stride of
  // 16 (mod 32) h16 puts the 8 rows of a half-wave's transposed read on
  // distinct banks
  static constexpr int LDMA = BM + 16, LDMB = BN + 16;
  static constexpr int cmax(int a, int b) { return a > b ? a : b; }
  static constexpr int AE = cmax(BM * LDK, BK * LDMA);  // h16 of one A buffer
  static constexpr int BE = cmax(BN * LDK, BK * LDMB);  // h16 of one B buffer
  static constexpr int AB = NBUF * (AE + BE) * 2;  // bytes of the operand buffers
  static constexpr int LDT = BN + 4;
  static constexpr int T = (BM / 2) * LDT * 4;          // bytes of one epilogue pass
  static constexpr int BYTES = AB > T ? AB : T;
};

// An epilogue may ask for a minimum occupancy (kMinWaves waves per SIMD: the
// register budget the compiler then keeps to), e.g. to fit a grid in one round.
template <class E, class = void>
struct epi_min_waves : std::integral_constant<int, 1> {};
template <class E>
struct epi_min_waves<E, std::void_t<decltype(E::kMinWaves)>>
    : std::integral_constant<int, E::kMinWaves> {};

template <int BM, int BN, int BK, bool AK, bool BKC, class Epi, class AL = ALoadDirect,
          bool SLICED = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(epi_min_waves<Epi>::value)))
void gemm_kernel(GemmArgs g, Epi epi, AL al = AL{}) {
  static_assert(!SLICED || BK == 32, "the sliced launch folds at 32-deep steps");
  using SM = GemmSmem<BM, BN, BK>;
  constexpr int WM = BM / 2, WN = BN / 2;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int LDK = SM::LDK;
  constexpr int A_CH = BM * BK / 8 / 256;
  constexpr int B_CH = BN * BK / 8 / 256;
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) unsigned char smem[SM::BYTES];
  h16* As = reinterpret_cast<h16*>(smem);            // [NBUF][AE]
  h16* Bs = As + SM::NBUF * SM::AE;                   // [NBUF][BE]
  // With a k-major operand both fragments take the K-slots {4g..4g+3,
  // 16+4g..16+4g+3} of a 32-step (lane group g): the k-major tile gives them
  // by two transposed reads, a K-contiguous tile by two 8-byte reads.  With
  // both K-contiguous, slots 8g..8g+7 (one 16-byte read).
  constexpr bool TR = !AK || !BKC;
  constexpr int LDMA = SM::LDMA, LDMB = SM::LDMB;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  // logical order (batch, m tile, n tile): the n tiles of one m tile, and
  // the tiles of one batch entry, run on one XCD and share its L2
  const int tiles_n = (g.N + BN - 1) / BN;
  const int tiles = ((g.M + BM - 1) / BM) * tiles_n;
  const long bid = xcd_block((long)tiles * g.batch);
  if (bid >= (long)tiles * g.batch) return;
  const int b = (int)(bid / tiles), t = (int)(bid % tiles);
  const int m0 = (t / tiles_n) * BM;
  const int n0 = (t % tiles_n) * BN;
  const h16* __restrict__ A = g.A + (long)b * g.a_sb;
  const h16* __restrict__ B = g.B + (long)b * g.b_sb;
  const int M = g.M, N = g.N;

  h16x8 ra[A_CH], rb[B_CH];
  const h16x8 zero8 = {};

  auto gload = [&](int k0) {
#pragma unroll
    for (int p = 0; p < A_CH; ++p) {
      const int c = tid + 256 * p;
      if constexpr (AK) {
        const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        const int m = m0 + row;
        if constexpr (AL::kDirect) ra[p] = (m < M) ? ld8(A + (long)m * g.a_sm + k0 + kc) : zero8;
        else ra[p] = (m < M) ? al(b, m, k0 + kc) : zero8;
      } else {
        const int k = c / (BM / 8), mc = (c % (BM / 8)) * 8;
        const int m = m0 + mc;
        ra[p] = (m < M) ? ld8(A + (long)(k0 + k) * g.a_sk + m) : zero8;
      }
    }
#pragma unroll
    for (int p = 0; p < B_CH; ++p) {
      const int c = tid + 256 * p;
      if constexpr (BKC) {
        const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        const int n = n0 + row;
        rb[p] = (n < N) ? ld8(B + (long)n * g.b_sn + k0 + kc) : zero8;
      } else {
        const int k = c / (BN / 8), nc = (c % (BN / 8)) * 8;
        const int n = n0 + nc;
        rb[p] = (n < N) ? ld8(B + (long)(k0 + k) * g.b_sk + n) : zero8;
      }
    }
  };
  auto sstore = [&](int buf) {
    h16* as = As + buf * SM::AE;
    h16* bs = Bs + buf * SM::BE;
#pragma unroll
    for (int p = 0; p < A_CH; ++p) {
      const int c = tid + 256 * p;
      if constexpr (AK) {
        const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        st8(&as[row * LDK + kc], ra[p]);
      } else {
        const int k = c / (BM / 8), mc = (c % (BM / 8)) * 8;
        st8(&as[k * LDMA + mc], ra[p]);
      }
    }
#pragma unroll
    for (int p = 0; p < B_CH; ++p) {
      const int c = tid + 256 * p;
      if constexpr (BKC) {
        const int row = c / (BK / 8), kc = (c % (BK / 8)) * 8;
        st8(&bs[row * LDK + kc], rb[p]);
      } else {
        const int k = c / (BN / 8), nc = (c % (BN / 8)) * 8;
        st8(&bs[k * LDMB + nc], rb[p]);
      }
    }
  };
  // fragments in the transposed-read slot order (TR)
  auto frag_rows = [&](const h16* T, int row, int kk) __attribute__((always_inline)) -> h16x8 {
    const h16* q = T + row * LDK + kk * 32 + 4 * (lane >> 4);
    const h16x4 x = *reinterpret_cast<const h16x4*>(q), y = *reinterpret_cast<const h16x4*>(q + 16);
    h16x8 v;
    v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
    v[4] = y[0]; v[5] = y[1]; v[6] = y[2]; v[7] = y[3];
    return v;
  };
  auto frag_cols = [&](const h16* T, int ld, int c0, int kk) __attribute__((always_inline)) -> h16x8 {
    return gemm_tr8(T, ld, kk * 32, c0, lane);
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = g.K / BK;
  f32x4 total[SLICED ? TM : 1][SLICED ? TN : 1];  // the slices' running sum
  constexpr int PRO = epi_pro_floats<Epi>::value;
  __shared__ float pro[PRO > 0 ? BM * PRO : 1];
  gload(0);
  if constexpr (PRO > 0) epi.template prologue<BM>(m0, pro, tid);
  sstore(0);
  __syncthreads();
  const int fr = lane & 15, fk = (lane >> 4) * 8;
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = SM::NBUF == 2 ? (kt & 1) : 0;
    const h16* as = As + buf * SM::AE;
    const h16* bs = Bs + buf * SM::BE;
    if (kt + 1 < nk) gload((kt + 1) * BK);
#pragma unroll
    for (int kk = 0; kk < BK / 32; ++kk) {
      h16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        if constexpr (!TR) af[i] = ld8(&as[(wm * WM + i * 16 + fr) * LDK + kk * 32 + fk]);
        else if constexpr (AK) af[i] = frag_rows(as, wm * WM + i * 16 + fr, kk);
        else af[i] = frag_cols(as, LDMA, wm * WM + i * 16, kk);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if constexpr (!TR) bfr[j] = ld8(&bs[(wn * WN + j * 16 + fr) * LDK + kk * 32 + fk]);
        else if constexpr (BKC) bfr[j] = frag_rows(bs, wn * WN + j * 16 + fr, kk);
        else bfr[j] = frag_cols(bs, LDMB, wn * WN + j * 16, kk);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = mfma16x16x32(af[i], bfr[j], acc[i][j]);
    }
    if constexpr (SLICED) {
      // a slice ends: its partial joins the running sum (the first one as
      // it is, as gemm_splitk_epi starts from partial 0) and restarts at 0
      const int spk = g.kslice / 32;
      if ((kt + 1) % spk == 0) {
        const bool first = kt + 1 == spk;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            total[i][j] = first ? acc[i][j] : total[i][j] + acc[i][j];
            acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
          }
      }
    }
    if constexpr (SM::NBUF == 2) {
      if (kt + 1 < nk) sstore(buf ^ 1);
    } else if (kt + 1 < nk) {
      __syncthreads();  // every wave is done with the buffer
      sstore(0);
    }
    __syncthreads();
  }

  if constexpr (SLICED) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = total[i][j];
  }

  // ---- epilogue: stage half a tile (the rows of one wave row) per pass
  constexpr int LDT = SM::LDT;
  float* T = reinterpret_cast<float*>(smem);
  const bool colm = epi.col_mode(n0);
#pragma unroll 1
  for (int pass = 0; pass < 2; ++pass) {
    if (pass) __syncthreads();  // previous pass consumed
    if (wm == pass) {
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            T[(i * 16 + (lane >> 4) * 4 + r) * LDT + wn * WN + j * 16 + fr] = acc[i][j][r];
    }
    __syncthreads();
    const int mb = m0 + pass * WM;
    auto rows = [&]() {
      for (int it = tid; it < WM * (BN / 8); it += 256) {
        const int r = it / (BN / 8), c8 = (it % (BN / 8)) * 8;
        const int m = mb + r, n = n0 + c8;
        if (m >= M || n >= N) continue;
        float v[8];
        ld_f8(T + r * LDT + c8, v);
        epi.row(b, m, n, v);
      }
    };
    if constexpr (epi_row_block<Epi>::value) {
      if constexpr (PRO > 0) epi.template block<WM>(b, mb, T, LDT, tid, pro + (mb - m0) * PRO);
      else epi.template block<WM>(b, mb, T, LDT, tid);
    } else if (colm) {
      for (int it = tid; it < BN * (WM / 8); it += 256) {
        const int c = it % BN, rg = it / BN;
        const int m = mb + rg * 8, n = n0 + c;
        if (m >= M || n >= N) continue;
        float* tp = T + (rg * 8) * LDT + c;
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = tp[e * LDT];
        epi.col(b, m, n, v, tp, LDT);
      }
      if constexpr (epi_two_phase<Epi>::value) {
        __syncthreads();  // the column pass has rewritten the tile
        rows();
      }
    } else {
      rows();
    }
  }
}

inline void gemm_check(bool ok, const char* what) {
  if (!ok) throw std::runtime_error(std::string("bc2n gemm: ") + what);
}

// The launch: loader form from the strides, BK from K (shapes checked).
template <int BM, int BN, class Epi, class AL>
void gemm_launch(hipStream_t st, const GemmArgs& g, const Epi& epi, const AL& al) {
  const bool ak = (g.a_sk == 1), bk = (g.b_sk == 1);
  const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  dim3 grid(xcd_grid((long)tiles * g.batch)), block(256);
  // K <= 128 (two 64-deep steps at most): 32-deep steps halve the operand
  // buffers (40 KB), so four workgroups share a CU and hide each other's
  // load latency; longer K keeps 64-deep steps (fewer barriers)
  const bool k64 = (g.K % 64 == 0) && g.K > 128;
  // A grid of a few tiles (the MSA's S x N-row products) runs one chain of
  // K steps per workgroup, each waiting for its loads: 128-deep steps halve
  // the chain (the operand tiles fit one buffer of 68 KB).
  const bool k128 = (g.K % 128 == 0) && g.K >= 256 && (long)tiles * g.batch * 8 <= device_cus();
#define BC2N_GEMM_LAUNCH(BKV, AKV, BKCV) \
  hipLaunchKernelGGL((gemm_kernel<BM, BN, BKV, AKV, BKCV, Epi, AL>), grid, block, 0, st, g, epi, al)
  if (k128) {
    if (ak && bk) BC2N_GEMM_LAUNCH(128, true, true);
    else if (ak) BC2N_GEMM_LAUNCH(128, true, false);
    else if (bk) BC2N_GEMM_LAUNCH(128, false, true);
    else BC2N_GEMM_LAUNCH(128, false, false);
  } else if (k64) {
    if (ak && bk) BC2N_GEMM_LAUNCH(64, true, true);
    else if (ak) BC2N_GEMM_LAUNCH(64, true, false);
    else if (bk) BC2N_GEMM_LAUNCH(64, false, true);
    else BC2N_GEMM_LAUNCH(64, false, false);
  } else {
    if (ak && bk) BC2N_GEMM_LAUNCH(32, true, true);
    else if (ak) BC2N_GEMM_LAUNCH(32, true, false);
    else if (bk) BC2N_GEMM_LAUNCH(32, false, true);
    else BC2N_GEMM_LAUNCH(32, false, false);
  }
#undef BC2N_GEMM_LAUNCH
}

// The sliced launch (g.kslice > 0, a multiple of 32 dividing K): 32-deep
// steps, a grid of the tiles alone.
template <int BM, int BN, class Epi, class AL>
void gemm_launch_sliced(hipStream_t st, const GemmArgs& g, const Epi& epi, const AL& al) {
  const bool ak = (g.a_sk == 1), bk = (g.b_sk == 1);
  const int tiles = ((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  dim3 grid(xcd_grid((long)tiles * g.batch)), block(256);
#define BC2N_GEMM_SLICED(AKV, BKCV) \
  hipLaunchKernelGGL((gemm_kernel<BM, BN, 32, AKV, BKCV, Epi, AL, true>), grid, block, 0, st, g, epi, al)
  if (ak && bk) BC2N_GEMM_SLICED(true, true);
  else if (ak) BC2N_GEMM_SLICED(true, false);
  else if (bk) BC2N_GEMM_SLICED(false, true);
  else BC2N_GEMM_SLICED(false, false);
#undef BC2N_GEMM_SLICED
}

// Split K for a grid of a few tiles and a long K (the MSA track's S x N-row
// products at S = 1: e.g. 224 x 256 over K = 1024 is 4 tiles of 128 x 128,
// each a chain of 8 dependent K steps): the K slices run as the batch
// entries of the same kernel (the batch strides step along K) and write f32
// partial tiles; gemm_splitk_epi adds them in slice order (the result does
// not depend on timing) and applies the epilogue's row() to each 8-column
// vector with the kernel's own lane order (consecutive lanes, consecutive
// column groups of one row).
template <class AL>
struct ALoadSliced {
  static constexpr bool kDirect = false;
  static constexpr bool kSide = false;
  AL al;
  int kslice;
  __device__ __forceinline__ h16x8 operator()(int b, int m, int k) const {
    return al(0, m, k + b * kslice);
  }
};

// f32 partial tile of K slice b: part[b][m][n] (row stride ldc, slice stride sb).
struct EpiPartial : EpiRows {
  float* C;
  long ldc, sb;
  __device__ __forceinline__ void row(int b, int m, int n, const float (&v)[8]) const {
    st_f8(C + (long)b * sb + (long)m * ldc + n, v);
  }
};

// The split-K partials: one arena per work lane (two streams may each run a
// split product at once).
inline Arena& gemm_splitk_scratch() {
  static Arena a[NUM_LANES];
  return a[lane()];
}

template <class Epi>
__global__ __launch_bounds__(256) void gemm_splitk_epi(const float* __restrict__ part, int S,
                                                      int M, int N, Epi epi) {
  const long idx = (long)blockIdx.x * blockDim.x + threadIdx.x;
  const int n8 = N / 8;
  if (idx >= (long)M * n8) return;  // M * n8 is a multiple of 8: whole lane groups
  const int m = (int)(idx / n8), n = (int)(idx % n8) * 8;
  const long MN = (long)M * N;
  float v[8];
  ld_f8(part + (long)m * N + n, v);
  for (int sl = 1; sl < S; ++sl) {
    float w[8];
    ld_f8(part + sl * MN + (long)m * N + n, w);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] += w[e];
  }
  epi.row(0, m, n, v);
}

// Launch with tile BM x BN; picks the loader form from the strides and BK
// from K.  Shapes are validated here, on the host, before any launch.  With a
// loader other than ALoadDirect, A is K-contiguous by construction (g.A is
// not read; a_sk must be 1).
template <int BM, int BN, class Epi, class AL = ALoadDirect>
void gemm(hipStream_t st, const GemmArgs& g, const Epi& epi, const char* name = "gemm",
          const AL& al = AL{}) {
  if constexpr (!AL::kDirect) gemm_check(g.a_sk == 1, "A loader: K-contiguous A");
  if constexpr (AL::kSide) gemm_check(g.N <= BN && g.batch == 1, "A loader side output: one tile column");
  gemm_check(g.M > 0 && g.N > 0 && g.K > 0 && g.batch > 0, "empty shape");
  gemm_check(g.K % 32 == 0, "K must be a multiple of 32");
  gemm_check(g.N % 8 == 0, "N must be a multiple of 8 (vector epilogue)");
  gemm_check(!Epi::kHasCol || g.M % 8 == 0, "M must be a multiple of 8 (column epilogue)");
  gemm_check(!epi_row_block<Epi>::value || (g.N == BN && g.batch == 1),
             "row-block epilogue: one tile column (N == BN)");
  const bool ak = (g.a_sk == 1), bk = (g.b_sk == 1);
  gemm_check(ak || g.a_sm == 1, "A needs a unit stride");
  gemm_check(bk || g.b_sn == 1, "B needs a unit stride");
  auto al16 = [](const void* p) { return ((uintptr_t)p & 15) == 0; };
  gemm_check((!AL::kDirect || al16(g.A)) && al16(g.B), "operands must be 16-byte aligned");
  if (ak) gemm_check(g.a_sm % 8 == 0, "A row stride must be a multiple of 8");
  else gemm_check(g.a_sk % 8 == 0, "A(T) stride must be a multiple of 8");
  if (bk) gemm_check(g.b_sn % 8 == 0, "B row stride must be a multiple of 8");
  else gemm_check(g.b_sk % 8 == 0, "B(T) stride must be a multiple of 8");
  gemm_check(g.batch == 1 || (g.a_sb % 8 == 0 && g.b_sb % 8 == 0), "batch strides");
  const long tiles = (long)((g.M + BM - 1) / BM) * ((g.N + BN - 1) / BN);
  KTimed kt(name, st);
  constexpr bool kSplittable = !epi_row_block<Epi>::value && !Epi::kHasCol && !AL::kSide;
  if constexpr (kSplittable) {
    if (g.batch == 1 && tiles * 2 < device_cus() && g.K >= 256 && g.N % 64 == 0) {
      // slices of at least 64 (a multiple of 32 that divides K), about one
      // workgroup per CU in all
      const int kb = g.K / 32;
      int split = (int)std::min<long>((device_cus() + tiles - 1) / tiles, g.K / 64);
      while (split > 1 && kb % split != 0) --split;
      if (split > 1) {
        const int kslice = g.K / split;
        if (lane() != 0) {
          // the side lane runs beside the pair track, the critical path: the
          // same sums on a grid of the tiles alone (no extra workgroups, no
          // partials through memory, no reduction launch) take less of the
          // chip from it; the bits are those of the split launch
          GemmArgs gk = g;
          gk.kslice = kslice;
          gemm_launch_sliced<BM, BN>(st, gk, epi, al);
          return;
        }
        GemmArgs gs = g;
        gs.K = kslice;
        gs.batch = split;
        gs.a_sb = (g.a_sk == 1) ? kslice : (long)kslice * g.a_sk;
        gs.b_sb = (g.b_sk == 1) ? kslice : (long)kslice * g.b_sk;
        Arena& ar = gemm_splitk_scratch();
        std::lock_guard<std::recursive_mutex> lk(ar.lock());
        const size_t elems = (size_t)split * g.M * g.N;
        ar.reset(st, elems * 4 + 256);
        float* part = ar.take_n<float>(elems);
        EpiPartial pe;
        pe.C = part;
        pe.ldc = g.N;
        pe.sb = (long)g.M * g.N;
        if constexpr (AL::kDirect) gemm_launch<BM, BN>(st, gs, pe, al);
        else gemm_launch<BM, BN>(st, gs, pe, ALoadSliced<AL>{al, kslice});
        const long n = (long)g.M * (g.N / 8);
        hipLaunchKernelGGL((gemm_splitk_epi<Epi>), dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                           st, part, split, g.M, g.N, epi);
        return;
      }
    }
  }
  gemm_launch<BM, BN>(st, g, epi, al);
}

// B operand of an N x 128 product (B(n, k), n < N, k < 128), N a multiple of
// 128, rearranged for kernels that read B fragments straight from memory:
// fragment ((j * 4 + w) * 2 + jj) * 4 + ks holds, at lane 16 g + c, the 8
// values B(j*128 + 32w + 16jj + c, ks*32 + 8g + e), e = 0..7 -- the
// v_mfma_f32_16x16x32_f16 B operand when A is K-contiguous -- so a wave
// loads a fragment as one contiguous 1 KB.
template <class B>
std::vector<h16> b_frags_k128(int N, B b) {
  std::vector<h16> f((size_t)N * 128);
  for (int j = 0; j < N / 128; ++j)
    for (int w = 0; w < 4; ++w)
      for (int jj = 0; jj < 2; ++jj)
        for (int ks = 0; ks < 4; ++ks)
          for (int l = 0; l < 64; ++l)
            for (int e = 0; e < 8; ++e)
              f[((size_t)(((j * 4 + w) * 2 + jj) * 4 + ks) * 64 + l) * 8 + e] =
                  (h16)b(j * 128 + 32 * w + 16 * jj + (l & 15), ks * 32 + 8 * (l >> 4) + e);
  return f;
}
__device__ __forceinline__ h16x8 b_frag_k128(const h16* F, int j, int w, int jj, int ks, int lane) {
  return ld8(F + ((long)(((j * 4 + w) * 2 + jj) * 4 + ks) * 64 + lane) * 8);
}

// ---------------------------------------------------------------- epilogues

// C[b][m][n] = act(acc + bias[n]) (+= existing when ACC), OutT in {float, h16}.
template <class OutT, bool RELU = false, bool ACC = false>
struct EpiStore : EpiRows {
  OutT* C;
  long ldc, sb;
  const float* bias;  // may be null
  int N;
  EpiStore(OutT* c, long l, long s, const float* bi, int n) : C(c), ldc(l), sb(s), bias(bi), N(n) {}
  __device__ __forceinline__ void row(int b, int m, int n, const float (&v)[8]) const {
    OutT* p = C + (long)b * sb + (long)m * ldc + n;
    float x[8];
    if (bias) {
      float bb[8];
      ld_f8(bias + n, bb);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = v[e] + bb[e];
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = v[e];
    }
    if (RELU) {
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = fmaxf(x[e], 0.f);
    }
    if (ACC) {
      float o[8];
      ld_any8<OutT>(p, o);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] += o[e];
    }
    st_any8<OutT>(p, x);
  }
};

// h16 store of acc + bias[n], columns n < qcols additionally scaled by
// qscale (attention projections: q carries D^-1/2 log2 e).
struct EpiScaledCols : EpiRows {
  h16* C;
  long ldc;
  const float* bias;
  float qscale;
  int qcols;
  EpiScaledCols(h16* c, long l, const float* b, float q, int qc)
      : C(c), ldc(l), bias(b), qscale(q), qcols(qc) {}
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    float bb[8], x[8];
    ld_f8(bias + n, bb);
    const float s = n < qcols ? qscale : 1.f;  // qcols is a multiple of 8
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (v[e] + bb[e]) * s;
    st_h8f(C + (long)m * ldc + n, x);
  }
};

// out[src(m)][n] = in[src(m)][n] + tbl[(m % nt)*C + n] * (acc + bias[n]);
// src(m) transposes the nt x nt grid when `transpose` (ending-node frame).
struct EpiResidualRows : EpiRows {
  const float* in;
  float* out;
  const float* bias;
  const float* tbl;  // may be null
  int nt, C;
  bool transpose;
  EpiResidualRows(const float* i, float* o, const float* b, const float* t, int n, int c, bool tr)
      : in(i), out(o), bias(b), tbl(t), nt(n), C(c), transpose(tr) {}
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const long src = transpose ? (long)(m % nt) * nt + m / nt : m;
    float bb[8], x[8], r[8];
    ld_f8(bias + n, bb);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = v[e] + bb[e];
    if (tbl) {
      float tt[8];
      ld_f8(tbl + (long)(m % nt) * C + n, tt);
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] *= tt[e];
    }
    ld_f8(in + src * C + n, r);
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] += x[e];
    st_f8(out + src * C + n, r);
  }
};

// Backward through attention's output gate, fused into the GEMM that makes
// d(og) = acc (og = o * sigmoid(g)):  dO = d(og) s,  dG = d(og) o s (1 - s),
// s = sigmoid(g), and nDsum[r][h][q] = -(sum over head h's D columns of dO * o)
// for token m = r * Ntok + q.  The D/8 row-mode calls of one head come from
// consecutive lanes (8 columns each), which add their partials by DPP.
struct EpiGateBwd : EpiRows {
  const h16* qkvg;  // gate pre-activation at column 3*HD + n of row m
  long ld;
  const h16* o;     // ungated attention output [M][HD]
  h16* dO;          // [M][HD]
  h16* dqkvg;       // dG at column 3*HD + n
  float* nDsum;      // [R][H][Ntok]
  int HD, H, D, Ntok;
  template <int W>
  __device__ __forceinline__ float head_sum(float s) const { return group_sum<W>(s); }
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const h16x8 gv = ld8(qkvg + (long)m * ld + 3 * HD + n);
    const h16x8 ov = ld8(o + (long)m * HD + n);
    h16x8 dov, dgv;
    float s = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float sg = sigmoidf_((float)gv[e]);
      const float oo = (float)ov[e];
      const float d = v[e] * sg;
      dov[e] = f2h_sat(d);
      dgv[e] = f2h_sat(v[e] * oo * sg * (1.f - sg));
      s += d * oo;
    }
    st8(dO + (long)m * HD + n, dov);
    st8(dqkvg + (long)m * ld + 3 * HD + n, dgv);
    s = D == 32 ? head_sum<4>(s) : head_sum<2>(s);
    if (n % D == 0) {
      const int r = m / Ntok, q = m % Ntok;
      nDsum[((long)r * H + n / D) * Ntok + q] = -s;
    }
  }
};

// dH = acc * (H > 0): backward through a ReLU of the kept tensor H (h16
// or binary16).
template <class OutT = h16, class HT = h16>
struct EpiReluMask : EpiRows {
  OutT* C;
  const HT* H;
  long ldc;
  EpiReluMask(OutT* c, const HT* h, long l) : C(c), H(h), ldc(l) {}
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const long o = (long)m * ldc + n;
    float h[8];
    ld_any8<HT>(H + o, h);
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = h[e] > 0.f ? v[e] : 0.f;
    st_any8<OutT>(C + o, x);
  }
};

// C[m][n] = h16(relu(acc + bias[n])) as EpiStore<h16, true> writes it, plus
// bits[m * (ldc / 8) + n / 8] bit e = (C[m][n + e] > 0): the ReLU's mask
// taken from the rounded value, so a backward that reads the bits masks
// exactly as one that reads C.
struct EpiReluBits : EpiRows {
  h16* C;
  uint8_t* bits;
  long ldc;
  const float* bias;
  EpiReluBits(h16* c, uint8_t* b, long l, const float* bi) : C(c), bits(b), ldc(l), bias(bi) {}
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    float bb[8], x[8];
    ld_f8(bias + n, bb);
    unsigned mk = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      x[e] = fmaxf(v[e] + bb[e], 0.f);
      mk |= ((float)f2h_sat(x[e]) > 0.f ? 1u : 0u) << e;
    }
    st_any8<h16>(C + (long)m * ldc + n, x);
    bits[(long)m * (ldc >> 3) + (n >> 3)] = (uint8_t)mk;
  }
};

// dH = acc * mask, the ReLU mask as EpiReluBits writes it (row stride ldc
// elements, ldc / 8 bytes).
template <class OutT = h16>
struct EpiReluMaskBits : EpiRows {
  OutT* C;
  const uint8_t* bits;
  long ldc;
  EpiReluMaskBits(OutT* c, const uint8_t* b, long l) : C(c), bits(b), ldc(l) {}
  __device__ __forceinline__ void row(int, int m, int n, const float (&v)[8]) const {
    const unsigned mk = bits[(long)m * (ldc >> 3) + (n >> 3)];
    float x[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = (mk >> e) & 1u ? v[e] : 0.f;
    st_any8<OutT>(C + (long)m * ldc + n, x);
  }
};

// A[m][k] = relu(src[m][k]) of a kept h16 tensor (row stride C).
struct ALoadRelu16 {
  static constexpr bool kDirect = false;
  static constexpr bool kSide = false;
  const h16* src;
  int C;
  __device__ __forceinline__ h16x8 operator()(int, int m, int k) const {
    h16x8 v = ld8(src + (long)m * C + k);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)v[e] > 0.f ? v[e] : (h16)0.f;
    return v;
  }
};


// LayerNorm backward fused into the GEMM that produces its cotangent dy (the
// d(LN output) of a module's input projections), C = BN = 128 channels, with
// the residual cotangent added:
//   out[src] = dres[src] + rstd * (g - mean(g) - xhat * mean(g * xhat)),
//   g = gs * gamma * (dy + sum_h dbias[h][m] wb[c][h]),  xhat = (x[src] - mean) * rstd,
// src = ln_src_row(m, nt) (the transposed orientation when nt > 0), gs =
// *gmul (the module's inverse cotangent scale; 1 when null).  dres may alias
// out.  16 lanes per row (a DPP row), 8 channels each.  dbias may be given as
// dbias_nch partials [nch][H][M], added here in chunk order (the attention
// backward's deferred reduction; the same sums as its reduction kernel).
template <int H>
struct EpiLnBwd : EpiRows {
  static constexpr bool kRowBlock = true;
  static constexpr int C = 128;
  const float *x, *gamma, *mean, *rstd, *dres, *dbias, *wb, *gmul;
  float* out;
  long M;
  int nt;
  int dbias_nch = 1;
  // the bias term's per-row head sums, made in the GEMM's prologue
  static constexpr int kProRowFloats = H;
  EpiLnBwd(const float* x_, const float* g_, const float* mu_, const float* rs_, const float* dres_,
           float* out_, long M_, int nt_, const float* dbias_ = nullptr, const float* wb_ = nullptr,
           const float* gmul_ = nullptr, int dbias_nch_ = 1)
      : x(x_), gamma(g_), mean(mu_), rstd(rs_), dres(dres_), dbias(dbias_), wb(wb_), gmul(gmul_),
        out(out_), M(M_), nt(nt_), dbias_nch(dbias_nch_) {}
  __device__ __forceinline__ void row(int, int, int, const float (&)[8]) const {}
  // pro[r][h] = dbias of row m0 + r, head h: the partials added in chunk
  // order, eight loads in flight (the sums of the attention backward's
  // reduction kernel); rows past M take row M - 1's
  template <int BM>
  __device__ __forceinline__ void prologue(long m0, float* pro, int tid) const {
    if constexpr (H > 0) {
      static_assert(BM * H % 256 == 0, "whole sums a thread");
      constexpr int PT = BM * H / 256;
      const long cs = (long)H * M;
      float s[PT];
      const float* p[PT];
#pragma unroll
      for (int i = 0; i < PT; ++i) {
        const int e = tid + 256 * i, r = e / H, h = e % H;
        p[i] = dbias + (long)h * M + min(m0 + r, M - 1);
        s[i] = 0.f;
      }
      if (dbias_nch == 1) {
#pragma unroll
        for (int i = 0; i < PT; ++i) s[i] = *p[i];
      } else {
        int c = 0;
        for (; c + 8 <= dbias_nch; c += 8) {
          float v[PT][8];
#pragma unroll
          for (int i = 0; i < PT; ++i)
#pragma unroll
            for (int u = 0; u < 8; ++u) v[i][u] = p[i][(c + u) * cs];
#pragma unroll
          for (int i = 0; i < PT; ++i)
#pragma unroll
            for (int u = 0; u < 8; ++u) s[i] += v[i][u];
        }
        for (; c < dbias_nch; ++c)
#pragma unroll
          for (int i = 0; i < PT; ++i) s[i] += p[i][c * cs];
      }
#pragma unroll
      for (int i = 0; i < PT; ++i) pro[tid + 256 * i] = s[i];
    }
  }
  template <int WM>
  __device__ __forceinline__ void block(int, long mb, const float* T, int ldt, int tid,
                                        const float* pro = nullptr) const {
    const int lr = tid >> 4, c0 = (tid & 15) * 8;
    float gm[8];
    ld_f8(gamma + c0, gm);
    if (gmul) {
      const float gs = *gmul;
#pragma unroll
      for (int e = 0; e < 8; ++e) gm[e] *= gs;
    }
    float w[8][H > 0 ? H : 1];
    if constexpr (H > 0) {
      const float4* p = reinterpret_cast<const float4*>(wb + c0 * H);
#pragma unroll
      for (int i = 0; i < 2 * H; ++i) {
        const float4 q = p[i];
        const float f[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) w[(4 * i + k) / H][(4 * i + k) % H] = f[k];
      }
    }
    // G rows a lane group at a time, every global load of the group issued
    // before its arithmetic: one memory round trip a group, not one a row
    // (the GEMM's 64-row halves take 4 rows a lane group; the transition's
    // 48-row tile keeps one, its register budget allows no more)
    constexpr int G = WM % 64 == 0 ? 4 : 1;
    static_assert(WM % (16 * G) == 0, "rows a pass");
#pragma unroll 1
    for (int r0 = 0; r0 < WM; r0 += 16 * G) {
      float xv[G][8], dr[G][8], db[G][H > 0 ? H : 1], mu[G], rs[G];
      long src[G];
#pragma unroll
      for (int q = 0; q < G; ++q) {
        // rows past M read row M - 1 (in bounds) and store nothing
        const long m = min(mb + r0 + 16 * q + lr, M - 1);
        src[q] = ln_src_row(m, nt);
        ld_f8(x + src[q] * C + c0, xv[q]);
        ld_f8(dres + src[q] * C + c0, dr[q]);
        if constexpr (H > 0) {
#pragma unroll
          for (int h = 0; h < H; ++h) {
            if (pro) {
              db[q][h] = pro[(r0 + 16 * q + lr) * H + h];
            } else if (dbias_nch == 1) {
              db[q][h] = dbias[(long)h * M + m];
            } else {
              float s = 0.f;
              for (int c = 0; c < dbias_nch; ++c) s += dbias[((long)c * H + h) * M + m];
              db[q][h] = s;
            }
          }
        }
        mu[q] = mean[m];
        rs[q] = rstd[m];
      }
#pragma unroll
      for (int q = 0; q < G; ++q) {
        if (mb + r0 + 16 * q + lr >= M) continue;  // the row's 16 lanes leave together
        float g[8];
        ld_f8(T + (r0 + 16 * q + lr) * ldt + c0, g);
        if constexpr (H > 0) {
#pragma unroll
          for (int h = 0; h < H; ++h)
#pragma unroll
            for (int e = 0; e < 8; ++e) g[e] += db[q][h] * w[e][h];
        }
        float sg = 0.f, sgx = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          xv[q][e] = (xv[q][e] - mu[q]) * rs[q];
          g[e] *= gm[e];
          sg += g[e];
          sgx += g[e] * xv[q][e];
        }
        sg = group_sum<16>(sg) * (1.f / C);
        sgx = group_sum<16>(sgx) * (1.f / C);
#pragma unroll
        for (int e = 0; e < 8; ++e) dr[q][e] += rs[q] * (g[e] - sg - xv[q][e] * sgx);
        st_f8(out + src[q] * C + c0, dr[q]);
      }
    }
  }
};

}  // namespace bc2n
