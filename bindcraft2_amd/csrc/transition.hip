// Transition (pair and MSA), forward and backward.
//   LN -> GEMM (C -> F*C) + bias + relu (the hidden's ReLU mask kept, a bit
//      an element; the hidden itself is scratch)
//      -> GEMM (F*C -> C) + bias, fused residual (+ shared dropout table)
// Backward: dh = ((tbl*dout) . W2^T) * (h > 0), the dropout scale applied as
// the GEMM loads A; dxn = dh . W1^T; LN backward accumulated into din.
// The pair transition (C = 128, F = 4) runs each direction as one kernel
// (tf::fused_kernel, the hidden never leaves the CU); the MSA and template
// widths as LN + two GEMMs.
//
// The backward's ReLU mask is h > 0, and every pre-activation that rounding
// moves across zero flips a mask entry against the exact model: with bf16
// operands about 0.1% of them flip, 4-5% of d(hidden) in L2; the binary16
// operands flip 8x fewer.
// Reference: modules.py:252-305 (Transition); native/transition.cuh:313-675.
#include "gemm.h"
#include "modules.h"

namespace bc2n {

namespace {

template <class A>
struct TransSave {
  float *mean, *rstd;
  uint8_t* hbits;  // bit n of row m: relu(xn . W1 + b1)[m][n] > 0
  TransSave(A& a, long rows, int C, int F) {
    mean = a.template take<float>(rows);
    rstd = a.template take<float>(rows);
    hbits = a.template take<uint8_t>((size_t)rows * C * F / 8);
  }
};

// ------------------------------------------------------------ fused MLP
// The pair transition (C = 128, hidden H = 512) as one kernel a direction.
// A workgroup owns BM = 16 RT rows.  Its input tile -- the LayerNorm output
// forward, the scaled cotangent backward -- stays in LDS as binary16, and the
// hidden layer is made and consumed 128 columns at a time: GEMM1 of the
// chunk, bias + ReLU (forward) or the kept mask (backward), the binary16
// chunk written k-major to LDS, GEMM2 accumulating into the workgroup's
// BM x 128 output.  The hidden never leaves the CU.  The 4 waves split the
// 128 columns of both products (32 each) over all BM rows, so every weight
// fragment is read from L2 once per workgroup, prefetched one chunk ahead.
//   forward:  xn = LN(x); h = relu(xn . W1 + b1); out = x + tbl * (h . W2 + b2)
//   backward: g = h16(s * tbl * dout); dh = (g . W2^T) * [h > 0];
//             din = dout + LNbwd(dh . W1^T) / s
// Both products take binary16 operands with f32 accumulation, rounded where
// the unfused GEMMs round (the same elementwise formulas).
namespace tf {
constexpr int C = 128, H = 512, HC = 128, NCH = H / HC;

template <int RT>
struct Geom {
  static constexpr int BM = 16 * RT;
  static constexpr int LDX = C + 8;  // xs[BM][LDX]: a 16-row 16-byte read covers every bank once
  static constexpr int LDH = BM + (BM % 32 == 16 ? 32 : 16);  // hs[HC][LDH], 16 mod 32 (transposed reads)
  static constexpr int LDT = C + 4;  // f32 output staging [BM][LDT], aliasing xs and hs
  static constexpr int XS = BM * LDX * 2, HS = HC * LDH * 2, T = BM * LDT * 4;
  static constexpr int MAIN = XS + HS > T ? XS + HS : T;
  static constexpr int BYTES = MAIN + BM * (H / 8);  // + the mask bits of the tile
};

struct Args {
  long M;
  int nt;
  const float* x;       // forward: act_in; backward: dout
  const float* tbl;     // dropout table [nt][C] or null
  const float* sc;      // backward: {s, 1/s}
  const float *ln_g, *ln_b;
  float *mean, *rstd;   // forward writes, backward reads
  const h16* W1;        // GEMM1's B (n < H, k < C) in fragment order: forward W1^T, backward W2
  const h16* W2;        // GEMM2's B (n < C, k < H) in fragment order: forward W2^T, backward W1
  const float* b1;      // forward only
  uint8_t* bits;        // [M][H / 8]: bit n % 8 of byte n / 8 of row m = h[m][n] > 0
};

// TBL (backward only): the cotangent is scaled by the dropout table a.tbl.
template <int RT, bool BWD, bool TBL, class Epi>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3, 3))) void fused_kernel(Args a, Epi epi) {
  using G = Geom<RT>;
  constexpr int BM = G::BM, LDX = G::LDX, LDH = G::LDH, LDT = G::LDT;
  __shared__ __align__(16) char smem[G::BYTES];
  h16* xs = reinterpret_cast<h16*>(smem);
  h16* hs = reinterpret_cast<h16*>(smem + G::XS);
  float* T = reinterpret_cast<float*>(smem);
  uint32_t* bw = reinterpret_cast<uint32_t*>(smem + G::MAIN);  // [BM][H / 32]
  uint16_t* bh = reinterpret_cast<uint16_t*>(bw);              // [BM][H / 16]
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, g = lane >> 4, l16 = lane & 15;
  const long M = a.M, m0 = (long)blockIdx.x * BM;

  h16x8 b1[4][2];
  h16x8 b2[4][2];
  float bb[2] = {0.f, 0.f};  // forward: b1 of this lane's two hidden columns
  // Workgroups walk the hidden chunks from different starting chunks, so the
  // many workgroups in flight do not all read the same weight lines at once.
  const int rot = blockIdx.x & (NCH - 1);
  // fragment f = ((j * 4 + w) * 2 + jj) * 4 + ks of a product's B operand is
  // 64 lanes x 8 binary16, contiguous: one 1 KB wave load
  auto frag = [&](const h16* F, int j, int jj, int ks) {
    return ld8(F + ((long)(((j * 4 + w) * 2 + jj) * 4 + ks) * 64 + lane) * 8);
  };
  auto load_b1 = [&](int jl) {
    const int j = (jl + rot) & (NCH - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) b1[ks][jj] = frag(a.W1, j, jj, ks);
    if constexpr (!BWD) {
      bb[0] = a.b1[j * HC + 32 * w + l16];
      bb[1] = a.b1[j * HC + 32 * w + 16 + l16];
    }
  };
  auto load_b2 = [&](int jl) {
    const int j = (jl + rot) & (NCH - 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) b2[ks][jj] = frag(a.W2, j, jj, ks);
  };

  // front: the binary16 input tile, 16 lanes a row, 8 channels a lane.  Its
  // loads go out first, so that waiting for them does not wait for the
  // weight fragments behind them (the memory counter retires in order).
  {
    const int lr = lane >> 4, c0 = l16 * 8;
    float v[RT][8];
#pragma unroll
    for (int p = 0; p < RT; ++p) {
      const long m = min(m0 + p * 16 + w * 4 + lr, M - 1);  // rows past M: in bounds, zeroed below
      ld_f8(a.x + m * C + c0, v[p]);
    }
    float gm[8], bt[8];
    float t[TBL ? RT : 1][8];
    if constexpr (TBL) {
#pragma unroll
      for (int p = 0; p < RT; ++p) {
        const long m = min(m0 + p * 16 + w * 4 + lr, M - 1);
        ld_f8(a.tbl + (m % a.nt) * C + c0, t[p]);
      }
    }
    if constexpr (!BWD) {
      ld_f8(a.ln_g + c0, gm);
      ld_f8(a.ln_b + c0, bt);
    }
    // backward: the tile's mask bits, 16 bytes a thread (NP pieces; the
    // threads past NP load a valid piece again and store nothing)
    constexpr int NP = BM * (H / 128), NBP = (NP + 255) / 256;
    uint4 mb[BWD ? NBP : 1];
    if constexpr (BWD) {
#pragma unroll
      for (int q = 0; q < NBP; ++q) {
        const int it = min(tid + 256 * q, NP - 1), r = it / (H / 128), c = it % (H / 128);
        const long m = min(m0 + r, M - 1);
        mb[q] = *reinterpret_cast<const uint4*>(a.bits + m * (H / 8) + c * 16);
      }
    }
    load_b1(0);
    load_b2(0);
    if constexpr (BWD) {
#pragma unroll
      for (int q = 0; q < NBP; ++q) {
        const int it = tid + 256 * q, r = it / (H / 128), c = it % (H / 128);
        if (it < NP)
          *reinterpret_cast<uint4*>(bw + r * (H / 32) + c * 4) =
              m0 + r < M ? mb[q] : make_uint4(0u, 0u, 0u, 0u);
      }
    }
#pragma unroll
    for (int p = 0; p < RT; ++p) {
      const int r = p * 16 + w * 4 + lr;
      const long m = m0 + r;
      h16x8 o;
      if constexpr (BWD) {
        const float sm = a.sc[0];
        if constexpr (TBL) {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[p][e] *= t[p][e] * sm;
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) v[p][e] *= sm;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = f2h_sat(v[p][e]);
      } else {
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += v[p][e];
        const float mu = group_sum<16>(s) / C;
        float d2 = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float d = v[p][e] - mu;
          d2 += d * d;
        }
        const float rs = rsqrtf(group_sum<16>(d2) / C + LN_EPS);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = (h16)((v[p][e] - mu) * rs * gm[e] + bt[e]);
        if (l16 == 0 && m < M) {
          a.mean[m] = mu;
          a.rstd[m] = rs;
        }
      }
      if (m >= M) o = h16x8{};
      st8(xs + r * LDX + c0, o);
    }
  }
  __syncthreads();

  f32x4 ao[RT][2];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj) ao[i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int jc = (j + rot) & (NCH - 1);
    // GEMM1: hidden columns jc*HC + 32w + 16jj + l16 of rows i*16 + 4g + r
    f32x4 ah[RT][2];
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) ah[i][jj] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      h16x8 af[RT];
#pragma unroll
      for (int i = 0; i < RT; ++i) af[i] = ld8(xs + (i * 16 + l16) * LDX + ks * 32 + 8 * g);
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) ah[i][jj] = mfma16x16x32(af[i], b1[ks][jj], ah[i][jj]);
    }
    const float bj[2] = {bb[0], bb[1]};
    // unconditional (the last chunk reloads its own): a load under a branch
    // leaves the in-order memory counter unknown at the join, and every wait
    // after it would become a wait for all loads
    load_b1(min(j + 1, NCH - 1));
    __syncthreads();  // the previous chunk's GEMM2 is done with hs
#pragma unroll
    for (int i = 0; i < RT; ++i) {
      unsigned long long bal[2][4];
      uint32_t wd[4];  // backward: the mask words of rows i*16 + 4g + r, this wave's 32 columns
      if constexpr (BWD) {
#pragma unroll
        for (int r = 0; r < 4; ++r) wd[r] = bw[(i * 16 + 4 * g + r) * (H / 32) + jc * 4 + w];
      }
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        h16x4 hv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float x;
          if constexpr (BWD) {
            x = (wd[r] >> (16 * jj + l16)) & 1u ? ah[i][jj][r] : 0.f;
          } else {
            x = fmaxf(ah[i][jj][r] + bj[jj], 0.f);
          }
          hv[r] = f2h_sat(x);
          if constexpr (!BWD) bal[jj][r] = __ballot((float)hv[r] > 0.f);
        }
        *reinterpret_cast<h16x4*>(hs + (32 * w + 16 * jj + l16) * LDH + i * 16 + 4 * g) = hv;
      }
      if constexpr (!BWD) {
        // lane L < 16 holds row i*16 + L = i*16 + 4g' + r' (g' = L/4, r' = L%4):
        // its 32 columns' bits are bits 16g'.. of the ballots of r', jj = 0, 1
        if (lane < 16) {
          const int gq = lane >> 2, rq = lane & 3;
          unsigned long long b0 = bal[0][0], b1v = bal[1][0];
#pragma unroll
          for (int r = 1; r < 4; ++r)
            if (rq == r) {
              b0 = bal[0][r];
              b1v = bal[1][r];
            }
          const uint32_t lo = (uint32_t)(b0 >> (16 * gq)) & 0xffffu;
          const uint32_t hi = (uint32_t)(b1v >> (16 * gq)) & 0xffffu;
          bw[(i * 16 + lane) * (H / 32) + jc * 4 + w] = lo | (hi << 16);
        }
      }
    }
    __syncthreads();
    // GEMM2: output columns 32w + 16jj + l16, K = this chunk's hidden columns
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      h16x8 af[RT];
#pragma unroll
      for (int i = 0; i < RT; ++i) af[i] = gemm_tr8(hs, LDH, ks * 32, i * 16, lane);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj)
#pragma unroll
        for (int i = 0; i < RT; ++i) ao[i][jj] = mfma16x16x32(af[i], b2[ks][jj], ao[i][jj]);
    }
    load_b2(min(j + 1, NCH - 1));
  }

  __syncthreads();  // every wave is done with xs and hs, which T overlays
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int jj = 0; jj < 2; ++jj)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        T[(i * 16 + 4 * g + r) * LDT + 32 * w + 16 * jj + l16] = ao[i][jj][r];
  if constexpr (!BWD) {
    for (int it = tid; it < BM * (H / 128); it += 256) {
      const int r = it / (H / 128), q = it % (H / 128);
      const long m = m0 + r;
      if (m < M)
        *reinterpret_cast<uint4*>(a.bits + m * (H / 8) + q * 16) =
            *reinterpret_cast<const uint4*>(bw + r * (H / 32) + q * 4);
    }
  }
  __syncthreads();
  if constexpr (epi_row_block<Epi>::value) {
    epi.template block<BM>(0, m0, T, LDT, tid);
  } else {
    for (int it = tid; it < BM * (C / 8); it += 256) {
      const int r = it / (C / 8), c8 = (it % (C / 8)) * 8;
      const long m = m0 + r;
      if (m >= M) continue;
      float v[8];
      ld_f8(T + r * LDT + c8, v);
      epi.row(0, (int)m, c8, v);
    }
  }
}

constexpr int kRT = 3;  // 48-row tiles (64 and 32 measured slower)

// B operands in the kernel's fragment order.  Lane l = 16 g + c of fragment
// (j, w, jj, ks) holds B[n][k0 + s(e)], e = 0..7, n = column j*HC + 32w +
// 16jj + c of the product; GEMM1 (A K-contiguous in LDS) takes the K-slots
// k0 = ks*32, s(e) = 8g + e; GEMM2 (A read transposed) takes k0 = j*HC +
// ks*32, s(e) = 4g + e (e < 4) and 16 + 4g + e - 4.  GEMM2's columns are the
// C outputs, so its n drops the j*HC term and its k carries it.
template <class B>
std::vector<h16> make_frags(bool second, B b) {
  std::vector<h16> f((size_t)H * C);
  for (int j = 0; j < NCH; ++j)
    for (int w = 0; w < 4; ++w)
      for (int jj = 0; jj < 2; ++jj)
        for (int ks = 0; ks < 4; ++ks)
          for (int l = 0; l < 64; ++l)
            for (int e = 0; e < 8; ++e) {
              const int g = l >> 4, c = l & 15;
              const int n = (second ? 0 : j * HC) + 32 * w + 16 * jj + c;
              const int k = second ? j * HC + ks * 32 + (e < 4 ? 4 * g + e : 16 + 4 * g + e - 4)
                                   : ks * 32 + 8 * g + e;
              f[((size_t)(((j * 4 + w) * 2 + jj) * 4 + ks) * 64 + l) * 8 + e] = (h16)b(n, k);
            }
  return f;
}

template <bool BWD, class Epi>
void fused(hipStream_t st, const Args& a, const Epi& epi, const char* name) {
  if (a.M <= 0 || a.M > (1L << 30)) throw std::runtime_error("transition: rows out of range");
  if (a.tbl && a.nt <= 0) throw std::runtime_error("transition: dropout table needs nt > 0");
  KTimed kt(name, st);
  const long nb = (a.M + Geom<kRT>::BM - 1) / Geom<kRT>::BM;
  bool tbl = false;
  if constexpr (BWD) tbl = a.tbl != nullptr;
  if (tbl)
    hipLaunchKernelGGL((fused_kernel<kRT, BWD, BWD, Epi>), dim3((unsigned)nb), dim3(256), 0, st, a,
                       epi);
  else
    hipLaunchKernelGGL((fused_kernel<kRT, BWD, false, Epi>), dim3((unsigned)nb), dim3(256), 0, st,
                       a, epi);
}
}  // namespace tf

}  // namespace

TransW transition_weights(WeightStore& ws, const std::string& P) {
  TransW w;
  const HostTensor& w1 = ws.host(P + "transition1/weights");  // [C, F*C]
  w.C = w1.shape[0];
  w.F = w1.shape[1] / w.C;
  const int C = w.C, H = w.C * w.F;
  w.ln_g = ws.f32(P + "input_layer_norm/scale");
  w.ln_b = ws.f32(P + "input_layer_norm/offset");
  w.b1 = ws.f32(P + "transition1/bias");
  w.b2 = ws.f32(P + "transition2/bias");
  const HostTensor& w2 = ws.host(P + "transition2/weights");  // [F*C, C]
  w.w1 = ws.derived<h16>("trans.w1:" + P, [&] { return to_h16(w1.data); });
  w.w1_t = ws.derived<h16>("trans.w1_t:" + P, [&] { return transpose_h16(w1.data.data(), C, H); });
  w.w2 = ws.derived<h16>("trans.w2:" + P, [&] { return to_h16(w2.data); });
  w.w2_t = ws.derived<h16>("trans.w2_t:" + P, [&] { return transpose_h16(w2.data.data(), H, C); });
  if (C == tf::C && H == tf::H) {
    const float* a1 = w1.data.data();  // [C][H]
    const float* a2 = w2.data.data();  // [H][C]
    w.frag1_f = ws.derived<h16>("trans.frag1_f:" + P, [&] {
      return tf::make_frags(false, [&](int n, int k) { return a1[(size_t)k * H + n]; });
    });
    w.frag2_f = ws.derived<h16>("trans.frag2_f:" + P, [&] {
      return tf::make_frags(true, [&](int n, int k) { return a2[(size_t)k * C + n]; });
    });
    w.frag1_b = ws.derived<h16>("trans.frag1_b:" + P, [&] {
      return tf::make_frags(false, [&](int n, int k) { return a2[(size_t)n * C + k]; });
    });
    w.frag2_b = ws.derived<h16>("trans.frag2_b:" + P, [&] {
      return tf::make_frags(true, [&](int n, int k) { return a1[(size_t)n * H + k]; });
    });
  }
  return w;
}

size_t transition_save_bytes(long rows, int C, int F) {
  Sizer s;
  TransSave<Sizer> plan(s, rows, C, F);
  (void)plan;
  return s.off;
}

void transition_fwd(hipStream_t st, const TransW& w, long rows, int nt, const float* act_in,
                    const float* tbl, float* act_out, void* save) {
  nonnull(act_in, "transition act"); nonnull(act_out, "transition out"); nonnull(save, "transition save");
  const int C = w.C, H = w.C * w.F;
  Carver cv(save);
  TransSave<Carver> sv(cv, rows, C, w.F);
  if (C == tf::C && H == tf::H) {
    tf::Args a{};
    a.M = rows; a.nt = nt; a.x = act_in; a.tbl = tbl;
    a.ln_g = w.ln_g; a.ln_b = w.ln_b; a.mean = sv.mean; a.rstd = sv.rstd;
    a.W1 = w.frag1_f; a.W2 = w.frag2_f; a.b1 = w.b1; a.bits = sv.hbits;
    tf::fused<false>(st, a, EpiResidualRows(act_in, act_out, w.b2, tbl, nt, C, false),
                     "trans.fused_fwd");
    return;
  }
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  Sizer need;
  need.take<h16>((size_t)rows * C);
  need.take<h16>((size_t)rows * H);
  ar.reset(st, need.off);
  h16* xn = ar.take_n<h16>((size_t)rows * C);
  h16* hid = ar.take_n<h16>((size_t)rows * H);
  {
    KTimed kt(BC2N_TN(C, "trans.ln_fwd"), st);
    ln_fwd_f32(st, act_in, rows, C, 0, w.ln_g, w.ln_b, xn, sv.mean, sv.rstd, false, 0, nullptr,
               nullptr);
  }
  GemmArgs g1;
  g1.M = (int)rows; g1.N = H; g1.K = C;
  g1.A = xn; g1.a_sm = C; g1.a_sk = 1;
  g1.B = w.w1_t; g1.b_sn = C; g1.b_sk = 1;
  gemm<128, 128>(st, g1, EpiReluBits(hid, sv.hbits, H, w.b1), BC2N_TN(C, "trans.gemm1"));
  GemmArgs g2;
  g2.M = (int)rows; g2.N = C; g2.K = H;
  g2.A = hid; g2.a_sm = H; g2.a_sk = 1;
  g2.B = w.w2_t; g2.b_sn = H; g2.b_sk = 1;
  gemm<128, 128>(st, g2, EpiResidualRows(act_in, act_out, w.b2, tbl, nt, C, false), BC2N_TN(C, "trans.gemm2"));
}

void transition_bwd(hipStream_t st, const TransW& w, long rows, int nt, const float* act_in,
                    const float* tbl, const void* save, const float* dout, float* din,
                    const float* sc) {
  nonnull(act_in, "transition act"); nonnull(save, "transition save");
  nonnull(dout, "transition dout"); nonnull(din, "transition din");
  const int C = w.C, H = w.C * w.F;
  Carver cv(const_cast<void*>(save));
  TransSave<Carver> sv(cv, rows, C, w.F);
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  sc = module_scale(st, sc, dout, rows * C);
  if (C == tf::C && H == tf::H) {
    tf::Args a{};
    a.M = rows; a.nt = nt; a.x = dout; a.tbl = tbl; a.sc = sc;
    a.ln_g = w.ln_g; a.mean = sv.mean; a.rstd = sv.rstd;
    a.W1 = w.frag1_b; a.W2 = w.frag2_b; a.bits = sv.hbits;
    tf::fused<true>(st, a,
                    EpiLnBwd<0>(act_in, w.ln_g, sv.mean, sv.rstd, dout, din, rows, 0, nullptr,
                                nullptr, sc + 1),
                    "trans.fused_bwd");
    return;
  }
  Sizer need;
  need.take<h16>((size_t)rows * H);
  need.take<float>((size_t)rows * C);
  ar.reset(st, need.off);
  h16* dh = ar.take_n<h16>((size_t)rows * H);
  float* dxn = ar.take_n<float>((size_t)rows * C);
  // dH = ((tbl * dout) . W2^T) * (H > 0), the dropout scale applied as A is loaded
  GemmArgs g1;
  g1.M = (int)rows; g1.N = H; g1.K = C;
  g1.a_sm = C; g1.a_sk = 1;
  g1.B = w.w2; g1.b_sn = C; g1.b_sk = 1;
  gemm<128, 128>(st, g1, EpiReluMaskBits<h16>(dh, sv.hbits, H), BC2N_TN(C, "trans.gemm_dh"),
                 ALoadScaledRows{dout, tbl, nt, C, false, sc});
  GemmArgs g2;
  g2.M = (int)rows; g2.N = C; g2.K = H;
  g2.A = dh; g2.a_sm = H; g2.a_sk = 1;
  g2.B = w.w1; g2.b_sn = H; g2.b_sk = 1;
  if (C == 128) {
    // the input LayerNorm's backward and the residual add in the epilogue
    gemm<128, 128>(st, g2,
                   EpiLnBwd<0>(act_in, w.ln_g, sv.mean, sv.rstd, dout, din, rows, 0, nullptr,
                               nullptr, sc + 1),
                   BC2N_TN(C, "trans.gemm_dx_ln"));
    return;
  }
  gemm<128, 128>(st, g2, EpiStore<float>{dxn, C, 0, nullptr, C}, BC2N_TN(C, "trans.gemm_dx"));
  KTimed kt(BC2N_TN(C, "trans.ln_bwd"), st);
  ln_bwd_f32(st, dxn, act_in, rows, C, 0, w.ln_g, sv.mean, sv.rstd, din, true, 0, nullptr, nullptr,
             dout, sc + 1);
}

}  // namespace bc2n
