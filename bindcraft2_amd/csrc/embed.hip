// Input embedder of the multimer model, forward and backward (the
// reference's EmbedderFwd/EmbedderBwd handlers, native/ffi.cu:682-729 over
// native/embed.cuh, for modules_multimer.py:358-483):
//
//   tf    target_feat padded to 21 columns (the caller pads)
//   msa   [s, n] = mask(n) * (tf[n] . W1d + b1d) + (mf[s, n] . Wmsa + bmsa)
//   pair  [i, j] = tf[i] . Wl + bl + tf[j] . Wr + br + relpos(i, j)
//   relpos(i, j) = Wpos[rel] + same_entity * Wpos[66] + Wpos[67 + chain] + bpos
//
// with mask(n) = 0 where target_feat row n sums to zero (padded residues stay
// zero through the bias), rel = clip(off + 32, 0, 64) inside a chain and 65
// across chains (off = offset[i][j], or residue_index[i] - residue_index[j]
// when no offset is given), chain = clip(sym_id[i] - sym_id[j] + 2, 0, 4)
// inside an entity and 5 across entities.  The position one-hots multiply
// out to row gathers of Wpos [73][128]; nothing [N][N][73] is formed.
//
// Everything is f32: the Linears have K = 21 or 49, so the work is a store
// stream (msa and pair out, forward) or a read stream (dmsa and dpair in,
// backward).  No save-set: the backward is a function of the cotangents,
// target_feat and the weights.  The position term gets no gradient (its
// inputs are indices).
#include "embed.h"

#include <algorithm>

namespace bc2n {

using namespace embed;

namespace {

// ------------------------------------------------------------------ forward

struct RowsArgs {
  const float *tf, *mf;
  const float *w1d, *b1d, *wmsa, *bmsa, *wl, *bl, *wr, *br, *bpos;
  float *msa, *lr;
  int N, S;
  int msa_blocks, msa_rpb;  // workgroups on msa rows, rows per workgroup
  int lr_rpb;               // rows per workgroup of the left/right rows
};

// Workgroups [0, msa_blocks) write msa rows, one thread per channel with its
// 49 + 21 weights in registers; the rest write lr [N][256] = (left + bpos |
// right), the per-residue halves of the pair.  Row operands are uniform
// across the workgroup (scalar loads).
__global__ __launch_bounds__(256) void embed_rows_kernel(RowsArgs a) {
  const int t = threadIdx.x;
  const int b = blockIdx.x;
  if (b < a.msa_blocks) {
    float wm[NMF], w1[NAA];
#pragma unroll
    for (int k = 0; k < NMF; ++k) wm[k] = a.wmsa[k * CM + t];
#pragma unroll
    for (int k = 0; k < NAA; ++k) w1[k] = a.w1d[k * CM + t];
    const float bm = a.bmsa[t], b1 = a.b1d[t];
    const long rows = (long)a.S * a.N;
    const long r0 = (long)b * a.msa_rpb, r1 = std::min(rows, r0 + a.msa_rpb);
    for (long r = r0; r < r1; ++r) {
      const int n = (int)(r % a.N);
      const float* tr = a.tf + (long)n * NAA;
      float fs = 0.f, p1 = 0.f;
#pragma unroll
      for (int k = 0; k < NAA; ++k) {
        const float x = tr[k];
        fs += x;
        p1 = fmaf(x, w1[k], p1);
      }
      p1 = fs == 0.f ? 0.f : p1 + b1;
      const float* mr = a.mf + r * NMF;
      float pm = 0.f;
#pragma unroll
      for (int k = 0; k < NMF; ++k) pm = fmaf(mr[k], wm[k], pm);
      a.msa[r * CM + t] = p1 + (pm + bm);
    }
    return;
  }
  const int side = t >> 7, c = t & (CZ - 1);
  const float* W = side ? a.wr : a.wl;
  float w[NAA];
#pragma unroll
  for (int k = 0; k < NAA; ++k) w[k] = W[k * CZ + c];
  const float bias = side ? a.br[c] : a.bl[c] + a.bpos[c];
  const int n0 = (b - a.msa_blocks) * a.lr_rpb, n1 = std::min(a.N, n0 + a.lr_rpb);
  for (int n = n0; n < n1; ++n) {
    const float* tr = a.tf + (long)n * NAA;
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < NAA; ++k) acc = fmaf(tr[k], w[k], acc);
    a.lr[(long)n * 2 * CZ + t] = acc + bias;
  }
}

__device__ __forceinline__ int clip_bin(int d, int m) {
  return d < -m ? 0 : (d > m ? 2 * m : d + m);
}

struct PairArgs {
  const float *lr, *wpos, *ri, *ai, *ei, *si;
  const int32_t* off;
  float* pair;
  int N, JC;
};

// Workgroup (i, 32 consecutive j); 32 lanes cover the 128 channels of one
// (i, j) as float4, 8 j per pass.
__global__ __launch_bounds__(256) void embed_pair_kernel(PairArgs p) {
  const long bid = blockIdx.x;
  if (bid >= (long)p.N * p.JC) return;
  const int i = (int)(bid / p.JC), jc = (int)(bid % p.JC);
  const int t = threadIdx.x, c4 = t & 31, js = t >> 5;
  const f32x4 li = *reinterpret_cast<const f32x4*>(p.lr + (long)i * 2 * CZ + 4 * c4);
  const float ri = p.ri[i], ai = p.ai[i], ei = p.ei[i], si = p.si[i];
  const f32x4 wsame = *reinterpret_cast<const f32x4*>(p.wpos + REL_BINS * CZ + 4 * c4);
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int j = jc * 32 + js + 8 * m;
    if (j >= p.N) continue;
    const int off = p.off ? p.off[(long)i * p.N + j] : (int)ri - (int)p.ri[j];
    const bool same_chain = ai == p.ai[j];
    const int rel = same_chain ? clip_bin(off, MAX_REL) : 2 * MAX_REL + 1;
    const bool same_entity = ei == p.ei[j];
    const int chain = same_entity ? clip_bin((int)si - (int)p.si[j], MAX_CHAIN) : 2 * MAX_CHAIN + 1;
    const f32x4 rj = *reinterpret_cast<const f32x4*>(p.lr + (long)j * 2 * CZ + CZ + 4 * c4);
    f32x4 v = li + rj;
    v += *reinterpret_cast<const f32x4*>(p.wpos + rel * CZ + 4 * c4);
    if (same_entity) v += wsame;
    v += *reinterpret_cast<const f32x4*>(p.wpos + (REL_BINS + 1 + chain) * CZ + 4 * c4);
    *reinterpret_cast<f32x4*>(p.pair + ((long)i * p.N + j) * CZ + 4 * c4) = v;
  }
}

// ----------------------------------------------------------------- backward

constexpr int TI = 8;   // pair rows per workgroup of the pair backward
constexpr int TJ = 32;  // pair columns per workgroup

struct PairBwdArgs {
  const float* dpair;
  float *dleft_part, *dright_part;  // [JC][N][128], [IT][N][128]
  int N, IT, JC;
};

// One read of dpair gives both reductions: workgroup (TI rows, TJ columns)
// writes the column sums over its rows (dright partial for its row tile) and
// the row sums over its columns (dleft partial for its column tile).
__global__ __launch_bounds__(256) void embed_pair_bwd_kernel(PairBwdArgs a) {
  __shared__ f32x4 red[TI][8][32];
  const long bid = blockIdx.x;
  if (bid >= (long)a.IT * a.JC) return;
  const int it = (int)(bid / a.JC), jc = (int)(bid % a.JC);
  const int t = threadIdx.x, c4 = t & 31, js = t >> 5;
  f32x4 col[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) col[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int il = 0; il < TI; ++il) {
    const int i = it * TI + il;
    f32x4 rs = {0.f, 0.f, 0.f, 0.f};
    if (i < a.N) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const int j = jc * TJ + js + 8 * m;
        if (j < a.N) {
          const f32x4 v = *reinterpret_cast<const f32x4*>(a.dpair + ((long)i * a.N + j) * CZ + 4 * c4);
          col[m] += v;
          rs += v;
        }
      }
    }
    red[il][js][c4] = rs;
  }
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int j = jc * TJ + js + 8 * m;
    if (j < a.N)
      *reinterpret_cast<f32x4*>(a.dright_part + ((long)it * a.N + j) * CZ + 4 * c4) = col[m];
  }
  __syncthreads();
  const int il = t >> 5, i = it * TI + il;
  if (i < a.N) {
    f32x4 s = red[il][0][c4];
#pragma unroll
    for (int q = 1; q < 8; ++q) s += red[il][q][c4];
    *reinterpret_cast<f32x4*>(a.dleft_part + ((long)jc * a.N + i) * CZ + 4 * c4) = s;
  }
}

struct RowsBwdArgs {
  const float *dmsa, *dleft_part, *dright_part, *tf, *wcat;
  float* dtf;
  int N, S, IT, JC;
};

// Workgroup n: g = [mask(n) * sum_s dmsa[s][n] | dleft[n] | dright[n]] (512)
// in LDS, then dtf[n][k] = g . wcat[k] for the 21 k, a wave per k.
__global__ __launch_bounds__(256) void embed_rows_bwd_kernel(RowsBwdArgs a) {
  __shared__ __attribute__((aligned(16))) float g[2 * CM];
  const int n = blockIdx.x, t = threadIdx.x;
  float fs = 0.f;
#pragma unroll
  for (int k = 0; k < NAA; ++k) fs += a.tf[(long)n * NAA + k];
  float dp = 0.f;
  for (int s = 0; s < a.S; ++s) dp += a.dmsa[((long)s * a.N + n) * CM + t];
  g[t] = fs == 0.f ? 0.f : dp;
  float d2 = 0.f;
  if (t < CZ) {
    for (int jc = 0; jc < a.JC; ++jc) d2 += a.dleft_part[((long)jc * a.N + n) * CZ + t];
  } else {
    for (int it = 0; it < a.IT; ++it) d2 += a.dright_part[((long)it * a.N + n) * CZ + t - CZ];
  }
  g[CM + t] = d2;
  __syncthreads();
  const int wave = t >> 6, lane = t & 63;
  const f32x4 g0 = *reinterpret_cast<const f32x4*>(&g[lane * 8]);
  const f32x4 g1 = *reinterpret_cast<const f32x4*>(&g[lane * 8 + 4]);
  for (int k = wave; k < NAA; k += 4) {
    const float* wk = a.wcat + (long)k * 2 * CM + lane * 8;
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(wk);
    const f32x4 w1 = *reinterpret_cast<const f32x4*>(wk + 4);
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) acc = fmaf(g0[q], w0[q], acc);
#pragma unroll
    for (int q = 0; q < 4; ++q) acc = fmaf(g1[q], w1[q], acc);
    acc = group_sum<64>(acc);
    if (lane == 0) a.dtf[(long)n * NAA + k] = acc;
  }
}

constexpr int TR = 16;  // msa rows per tile of the msa_feat backward

struct DmfArgs {
  const float *dmsa, *wmsa;
  float* dmf;
  long rows;
  int tiles;
};

// dmf[r][k] = dmsa[r] . Wmsa[k] over the 256 channels.  Wmsa sits in LDS
// transposed ([c][k]: lane k reads consecutive words); a tile of 16 dmsa rows
// is staged beside it and read by broadcast.  Lane k < 49 of wave w computes
// rows 4w..4w+3 of the tile.  Workgroups stride over the tiles.
__global__ __launch_bounds__(256) void embed_dmf_kernel(DmfArgs a) {
  __shared__ float WT[CM * NMF];
  __shared__ f32x4 X[TR][CM / 4];
  const int t = threadIdx.x;
  for (int e = t; e < NMF * CM; e += 256) WT[(e % CM) * NMF + e / CM] = a.wmsa[e];
  const int k = t & 63, rg = t >> 6;
  for (int tile = blockIdx.x; tile < a.tiles; tile += gridDim.x) {
    __syncthreads();  // WT written; the previous tile's readers are done
#pragma unroll
    for (int q = 0; q < TR * CM / 4 / 256; ++q) {
      const int e = t + 256 * q, r = e / (CM / 4), c4 = e % (CM / 4);
      const long row = (long)tile * TR + r;
      X[r][c4] = row < a.rows ? *reinterpret_cast<const f32x4*>(a.dmsa + row * CM + 4 * c4)
                              : f32x4{0.f, 0.f, 0.f, 0.f};
    }
    __syncthreads();
    if (k < NMF) {
      float acc[4] = {0.f, 0.f, 0.f, 0.f};
      for (int c4 = 0; c4 < CM / 4; ++c4) {
        float w[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) w[q] = WT[(4 * c4 + q) * NMF + k];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const f32x4 x = X[rg * 4 + rr][c4];
#pragma unroll
          for (int q = 0; q < 4; ++q) acc[rr] = fmaf(x[q], w[q], acc[rr]);
        }
      }
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const long row = (long)tile * TR + rg * 4 + rr;
        if (row < a.rows) a.dmf[row * NMF + k] = acc[rr];
      }
    }
  }
}

const float* dev_f32(WeightStore& ws, const std::string& name, std::vector<int> shape) {
  const HostTensor& h = ws.host(name);
  if (h.shape != shape) throw std::runtime_error("embedder: " + name + " has the wrong shape");
  return ws.f32(name);
}

void aligned16(const void* p, const char* what) {
  if ((uintptr_t)p & 15) throw std::runtime_error(std::string("embedder: ") + what + " must be 16-byte aligned");
}

}  // namespace

EmbedW embed_weights(WeightStore& ws) {
  EmbedW w;
  const std::string P = "param/";
  w.w1d = dev_f32(ws, P + "preprocess_1d/weights", {NAA, CM});
  w.b1d = dev_f32(ws, P + "preprocess_1d/bias", {CM});
  w.wmsa = dev_f32(ws, P + "preprocess_msa/weights", {NMF, CM});
  w.bmsa = dev_f32(ws, P + "preprocess_msa/bias", {CM});
  w.wl = dev_f32(ws, P + "left_single/weights", {NAA, CZ});
  w.bl = dev_f32(ws, P + "left_single/bias", {CZ});
  w.wr = dev_f32(ws, P + "right_single/weights", {NAA, CZ});
  w.br = dev_f32(ws, P + "right_single/bias", {CZ});
  // haiku scopes a module made inside a method under the method's name
  const std::string scoped = P + "evoformer/~_relative_encoding/position_activations/";
  const std::string pos = ws.has(scoped + "weights") ? scoped : P + "position_activations/";
  w.wpos = dev_f32(ws, pos + "weights", {REL_TOT, CZ});
  w.bpos = dev_f32(ws, pos + "bias", {CZ});
  w.wcat = ws.derived<float>("embed.wcat", [&] {
    const auto& a = ws.host(P + "preprocess_1d/weights").data;
    const auto& l = ws.host(P + "left_single/weights").data;
    const auto& r = ws.host(P + "right_single/weights").data;
    std::vector<float> o((size_t)NAA * 2 * CM);
    for (int k = 0; k < NAA; ++k) {
      std::copy(a.begin() + (size_t)k * CM, a.begin() + (size_t)(k + 1) * CM, o.begin() + (size_t)k * 2 * CM);
      std::copy(l.begin() + (size_t)k * CZ, l.begin() + (size_t)(k + 1) * CZ,
                o.begin() + (size_t)k * 2 * CM + CM);
      std::copy(r.begin() + (size_t)k * CZ, r.begin() + (size_t)(k + 1) * CZ,
                o.begin() + (size_t)k * 2 * CM + CM + CZ);
    }
    return o;
  });
  return w;
}

void embed_fwd(hipStream_t st, const EmbedW& w, int N, int S, const float* tf, const float* mf,
               const float* residue_index, const float* asym_id, const float* entity_id,
               const float* sym_id, const int32_t* offset, float* msa, float* pair) {
  if (N <= 0 || S <= 0) throw std::runtime_error("embedder: N and S must be positive");
  nonnull(tf, "embedder target_feat"); nonnull(mf, "embedder msa_feat");
  nonnull(residue_index, "embedder residue_index"); nonnull(asym_id, "embedder asym_id");
  nonnull(entity_id, "embedder entity_id"); nonnull(sym_id, "embedder sym_id");
  nonnull(msa, "embedder msa"); nonnull(pair, "embedder pair");
  aligned16(pair, "pair");
  const int cus = device_cus();
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)N * 2 * CZ * 4 + 1024);
  float* lr = ar.take_n<float>((size_t)N * 2 * CZ);
  RowsArgs a;
  a.tf = tf; a.mf = mf;
  a.w1d = w.w1d; a.b1d = w.b1d; a.wmsa = w.wmsa; a.bmsa = w.bmsa;
  a.wl = w.wl; a.bl = w.bl; a.wr = w.wr; a.br = w.br; a.bpos = w.bpos;
  a.msa = msa; a.lr = lr; a.N = N; a.S = S;
  const long rows = (long)S * N;
  a.msa_rpb = (int)std::max(1L, (rows + 4L * cus - 1) / (4L * cus));
  a.msa_blocks = (int)((rows + a.msa_rpb - 1) / a.msa_rpb);
  a.lr_rpb = std::max(1, (N + 63) / 64);
  const int lr_blocks = (N + a.lr_rpb - 1) / a.lr_rpb;
  {
    KTimed kt("embed.rows", st);
    hipLaunchKernelGGL(embed_rows_kernel, dim3(a.msa_blocks + lr_blocks), dim3(256), 0, st, a);
  }
  PairArgs p;
  p.lr = lr; p.wpos = w.wpos; p.ri = residue_index; p.ai = asym_id; p.ei = entity_id; p.si = sym_id;
  p.off = offset; p.pair = pair; p.N = N; p.JC = (N + 31) / 32;
  KTimed kt("embed.pair", st);
  hipLaunchKernelGGL(embed_pair_kernel, dim3((unsigned)((long)N * p.JC)), dim3(256), 0, st, p);
}

void embed_bwd(hipStream_t st, const EmbedW& w, int N, int S, const float* dmsa,
               const float* dpair, const float* tf, float* dtf, float* dmf) {
  if (N <= 0 || S <= 0) throw std::runtime_error("embedder: N and S must be positive");
  nonnull(dmsa, "embedder dmsa"); nonnull(dpair, "embedder dpair"); nonnull(tf, "embedder target_feat");
  nonnull(dtf, "embedder dtf"); nonnull(dmf, "embedder dmf");
  aligned16(dmsa, "dmsa"); aligned16(dpair, "dpair");
  const int cus = device_cus();
  const int IT = (N + TI - 1) / TI, JC = (N + TJ - 1) / TJ;
  Arena& ar = arena();
  std::lock_guard<std::recursive_mutex> lk(ar.lock());
  ar.reset(st, (size_t)(IT + JC) * N * CZ * 4 + 2048);
  float* dleft_part = ar.take_n<float>((size_t)JC * N * CZ);
  float* dright_part = ar.take_n<float>((size_t)IT * N * CZ);
  {
    PairBwdArgs b{dpair, dleft_part, dright_part, N, IT, JC};
    KTimed kt("embed.pair_bwd", st);
    hipLaunchKernelGGL(embed_pair_bwd_kernel, dim3((unsigned)((long)IT * JC)), dim3(256), 0, st, b);
  }
  {
    RowsBwdArgs b{dmsa, dleft_part, dright_part, tf, w.wcat, dtf, N, S, IT, JC};
    KTimed kt("embed.rows_bwd", st);
    hipLaunchKernelGGL(embed_rows_bwd_kernel, dim3(N), dim3(256), 0, st, b);
  }
  DmfArgs d;
  d.dmsa = dmsa; d.wmsa = w.wmsa; d.dmf = dmf; d.rows = (long)S * N;
  d.tiles = (int)((d.rows + TR - 1) / TR);
  KTimed kt("embed.dmf", st);
  hipLaunchKernelGGL(embed_dmf_kernel, dim3(std::min(d.tiles, 2 * cus)), dim3(256), 0, st, d);
}

}  // namespace bc2n
