// Triangle multiplication's k-contraction: one N x N product per channel,
//
//   C_c[m][n] = sum_k A_c[m][k] * B_c[n][k],     m, n, k < N = 32*NB <= 256,
//
// for channel-major operand arrays (plane c at c*P).  Each operand plane is
// either K-contiguous (element (r, k) at r*N + k) or k-major (at k*N + r), so
// one kernel serves the outgoing/incoming forward and both backward products.
//
// A workgroup is NB waves on one channel; wave w owns the 32 columns
// n = 32w .. 32w+31 and keeps their B fragments for the whole K in registers
// (NB k-steps x 2 n-tiles x 8 h16).  The workgroup walks strips of 16 rows of
// A (the strips s = g, g+G, ... of its channel, G workgroups per channel):
// each strip is staged in LDS, double-buffered with a register prefetch of the
// next one, and feeds v_mfma_f32_16x16x32_f16 with B as the first operand, so
// a lane ends with 4 consecutive columns of one output row (a vector store).
//
// K-slot order: both operands present the 32 k of a step to lane group g as
// {4g..4g+3, 16+4g..16+4g+3} -- from a K-contiguous LDS row by two 8-byte
// reads, from a k-major tile by two ds_read_b64_tr_b16 (the column read of a
// 4 x 16 block) -- so any pairing of layouts multiplies matching k.
// Reference: modules.py:1044-1088 (the einsum 'ikc,jkc->ijc' / 'kjc,kic->ijc'
// of _fused_triangle_multiplication).
#include "kernels.h"
#include "runtime.h"

namespace bc2n {

namespace {

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

// T[r0 + 4g + j][c0 + l%16], j = 0..3, of a row-major LDS tile (ld % 4 == 0)
__device__ __forceinline__ h16x4 tr4(const h16* T, int ld, int r0, int c0, int lane) {
  const int g = lane >> 4, m = lane & 15;
  const h16* p = T + (r0 + 4 * g + (m >> 2)) * ld + c0 + 4 * (m & 3);
  return __builtin_bit_cast(h16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)p));
}

__device__ __forceinline__ h16x8 cat8(h16x4 a, h16x4 b) {
  h16x8 r;
  r[0] = a[0]; r[1] = a[1]; r[2] = a[2]; r[3] = a[3];
  r[4] = b[0]; r[5] = b[1]; r[6] = b[2]; r[7] = b[3];
  return r;
}

// Fragment of row `row` (the lane's m or n) for k-step ks from a K-contiguous
// tile T[row][k] (row stride ld) ...
__device__ __forceinline__ h16x8 frag_rows(const h16* T, int ld, int row, int ks, int g) {
  const h16* p = T + row * ld + ks * 32 + 4 * g;
  return cat8(*reinterpret_cast<const h16x4*>(p), *reinterpret_cast<const h16x4*>(p + 16));
}
// ... and from a k-major tile T[k][col] (column c0 + l%16).
__device__ __forceinline__ h16x8 frag_cols(const h16* T, int ld, int c0, int ks, int lane) {
  return cat8(tr4(T, ld, ks * 32, c0, lane), tr4(T, ld, ks * 32 + 16, c0, lane));
}

template <class OutT>
__device__ __forceinline__ void store4(OutT* p, f32x4 v);
template <>
__device__ __forceinline__ void store4<float>(float* p, f32x4 v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store4<h16>(h16* p, f32x4 v) {
  h16x4 o;
  o[0] = f2h_sat(v[0]); o[1] = f2h_sat(v[1]); o[2] = f2h_sat(v[2]); o[3] = f2h_sat(v[3]);
  *reinterpret_cast<h16x4*>(p) = o;
}

constexpr int SR = 16;  // rows of A per strip
constexpr int MAXS = 4;  // A strips a workgroup (held in registers)

template <int NB, bool AK, bool BK, class OutT>
__global__ __launch_bounds__(64 * NB) void contract_kernel(const h16* __restrict__ A,
                                                           const h16* __restrict__ B,
                                                           OutT* __restrict__ C, long P,
                                                           int channels, int groups) {
  constexpr int N = 32 * NB;
  constexpr int NT = 64 * NB;      // threads
  constexpr int NS = N / SR;       // strips per channel
  // LDS: B staging chunk (init only) and the two A strip buffers
  constexpr int LDB = BK ? 32 + 8 : N + 8;   // B chunk: [N][32] (K-contig) or [32][N] (k-major)
  constexpr int BROWS = BK ? N : 32;
  constexpr int LDA = AK ? N + 8 : SR + 8;   // A strip: [16][N] (K-contig) or [N][16] (k-major)
  constexpr int AROWS = AK ? SR : N;
  constexpr int ABUF = AROWS * LDA;
  __shared__ __attribute__((aligned(16))) h16 As[2 * ABUF];
  __shared__ __attribute__((aligned(16))) h16 Bs[2 * BROWS * LDB];  // two staging chunks
  static_assert(SR * N / 8 == NT, "one 16-byte chunk of a strip per thread");

  const long G = (long)channels * groups;
  const long bid = xcd_block(G);  // (channel, group): a channel's groups share its B plane in L2
  if (bid >= G) return;
  const int ch = (int)(bid / groups), grp = (int)(bid % groups);
  const h16* Ap = A + (long)ch * P;
  const h16* Bp = B + (long)ch * P;
  OutT* Cp = C + (long)ch * P;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = lane >> 4, l16 = lane & 15;
  const int n0 = wave * 32;

  // Every global load the workgroup needs is issued before its first wait:
  // the staging chunks of B (32 k each) PD chunks ahead of their turn, and
  // all of its A strips (at most MAXS, held in registers) behind the first PD
  // chunks.  Staged one chunk and one strip at a time, each chunk and strip
  // had cost a full memory round trip (7 + 3.5 of them a workgroup at N =
  // 224, about 14 us a launch).
  constexpr int CH = BROWS * (BK ? 4 : N / 8);  // 16-byte pieces per staging chunk
  constexpr int CPT = (CH + NT - 1) / NT;        // a thread's pieces per chunk
  constexpr int PD = NB < 2 ? NB : 2;            // chunks in flight
  auto load_b = [&](int kc, h16x8 (&v)[CPT]) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = min(tid + NT * i, CH - 1);  // a spare piece re-reads the last one
      if constexpr (BK) {
        const int r = c / 4, q = (c % 4) * 8;
        v[i] = ld8(Bp + (long)r * N + kc * 32 + q);
      } else {
        const int r = c / (N / 8), q = (c % (N / 8)) * 8;
        v[i] = ld8(Bp + (long)(kc * 32 + r) * N + q);
      }
    }
  };
  h16x8 vb[PD][CPT];
#pragma unroll
  for (int p = 0; p < PD; ++p) load_b(p, vb[p]);

  // ---- A strips: s = grp + i * groups, i < nsw (the launcher keeps nsw <= MAXS)
  auto load_strip = [&](int s) -> h16x8 {
    if constexpr (AK) {
      const int r = tid / (N / 8), q = (tid % (N / 8)) * 8;
      return ld8(Ap + (long)(s * SR + r) * N + q);
    } else {
      const int k = tid / 2, q = (tid % 2) * 8;
      return ld8(Ap + (long)k * N + s * SR + q);
    }
  };
  const int nsw = grp < NS ? (NS - grp + groups - 1) / groups : 0;
  h16x8 va[MAXS];
#pragma unroll
  for (int i = 0; i < MAXS; ++i) va[i] = load_strip(min(grp + i * groups, NS - 1));  // spares: in bounds

  // ---- B fragments of this wave's 32 columns, all k, via LDS chunks of 32 k
  h16x8 bf[NB][2];
  // (two LDS chunks: the barrier after a chunk's stores also orders the
  // reads of the chunk before it, whose buffer the next stores reuse)
#pragma unroll
  for (int kc = 0; kc < NB; ++kc) {
    h16x8 (&v)[CPT] = vb[kc % PD];
    h16* bs = Bs + (kc & 1) * BROWS * LDB;
#pragma unroll
    for (int i = 0; i < CPT; ++i) {
      const int c = tid + NT * i;
      if (c < CH) {
        if constexpr (BK) st8(&bs[(c / 4) * LDB + (c % 4) * 8], v[i]);
        else st8(&bs[(c / (N / 8)) * LDB + (c % (N / 8)) * 8], v[i]);
      }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      if constexpr (BK) bf[kc][j] = frag_rows(bs, LDB, n0 + j * 16 + l16, 0, g);
      else bf[kc][j] = frag_cols(bs, LDB, n0 + j * 16, 0, lane);
    }
    if (kc + PD < NB) load_b(kc + PD, v);
  }

  auto stash = [&](int buf, h16x8 v) {
    h16* as = As + buf * ABUF;
    if constexpr (AK) st8(&as[(tid / (N / 8)) * LDA + (tid % (N / 8)) * 8], v);
    else st8(&as[(tid / 2) * LDA + (tid % 2) * 8], v);
  };
  if (nsw == 0) return;  // (uniform) no barrier follows
  stash(0, va[0]);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < MAXS; ++i) {
    if (i >= nsw) break;  // uniform
    const int s = grp + i * groups, buf = i & 1;
    const h16* as = As + buf * ABUF;
    f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < NB; ++ks) {
      h16x8 af;
      if constexpr (AK) af = frag_rows(as, LDA, l16, ks, g);
      else af = frag_cols(as, LDA, 0, ks, lane);
#pragma unroll
      for (int j = 0; j < 2; ++j)
        acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(bf[ks][j], af, acc[j], 0, 0, 0);
    }
    // lane: row m = strip row l16, columns n0 + 16j + 4g .. +3
    const int m = s * SR + l16;
#pragma unroll
    for (int j = 0; j < 2; ++j) store4<OutT>(Cp + (long)m * N + n0 + j * 16 + 4 * g, acc[j]);
    if (i + 1 < nsw) stash(buf ^ 1, va[i + 1 < MAXS ? i + 1 : i]);
    __syncthreads();
  }
}

template <int NB, class OutT>
void launch(hipStream_t st, bool ak, bool bk, const h16* A, const h16* B, OutT* C, long P,
            int channels, int groups) {
  const dim3 grid(xcd_grid((long)channels * groups)), block(64 * NB);
#define BC2N_CT(AKV, BKV) \
  hipLaunchKernelGGL((contract_kernel<NB, AKV, BKV, OutT>), grid, block, 0, st, A, B, C, P, channels, groups)
  if (ak && bk) BC2N_CT(true, true);
  else if (ak) BC2N_CT(true, false);
  else if (bk) BC2N_CT(false, true);
  else BC2N_CT(false, false);
#undef BC2N_CT
}

template <class OutT>
bool contract_t(hipStream_t st, int N, int channels, const h16* A, bool ak, const h16* B,
                bool bk, OutT* C, int groups) {
  const long P = (long)N * N;
  switch (N / 32) {
#define BC2N_NB(v) case v: launch<v, OutT>(st, ak, bk, A, B, C, P, channels, groups); return true;
    BC2N_NB(1) BC2N_NB(2) BC2N_NB(3) BC2N_NB(4) BC2N_NB(5) BC2N_NB(6) BC2N_NB(7) BC2N_NB(8)
#undef BC2N_NB
    default: return false;
  }
}

}  // namespace

bool trimul_contract(hipStream_t st, int N, int channels, const h16* A, bool a_kcontig,
                     const h16* B, bool b_kcontig, float* Cf, h16* Cb) {
  if (N <= 0 || N % 32 != 0 || N > 256) return false;
  if (((uintptr_t)A & 15) || ((uintptr_t)B & 15) || ((uintptr_t)Cf & 15) || ((uintptr_t)Cb & 7))
    throw std::runtime_error("contract: operands must be 16-byte aligned");
  int dev = 0, cus = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev),
            "hipDeviceGetAttribute");
  // about two workgroups per CU, a channel's strips spread over its groups
  const int ns = N / SR;
  const int groups = std::max((ns + MAXS - 1) / MAXS,
                              std::max(1, std::min(ns, (2 * cus + channels - 1) / channels)));
  if (Cf) return contract_t<float>(st, N, channels, A, a_kcontig, B, b_kcontig, Cf, groups);
  return contract_t<h16>(st, N, channels, A, a_kcontig, B, b_kcontig, Cb, groups);
}

}  // namespace bc2n
