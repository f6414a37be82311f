// The C ABI (include/bc2n.h): argument checks, weight lookup, error channel.
#include "../../include/bc2n.h"
#include "evoformer.h"
#include "gemm.h"
#include "gemm_f32.h"
#include "modules.h"
#include "tplembed.h"
#include "embed.h"
#include "heads.h"
#include "designstep.h"
#include "confidence.h"

#include <cstdio>
#include <map>
#include <tuple>

using namespace bc2n;

namespace {

// The library's scratch (arenas, detached and own save-sets, cotangent
// scales) is shared by every call on a GPU, so calls on different streams
// are ordered: each call records an event on its stream after its last
// launch, and a call arriving on another stream first waits for the
// previous call's event.  Calls on one stream pay one event record.  Under
// graph capture nothing is recorded or waited for (a captured graph runs on
// the capturing stream's order only).
struct StreamOrder {
  hipStream_t last = nullptr;
  hipEvent_t ev = nullptr;
  bool recorded = false;
};
std::mutex g_order_mu;
std::map<int, StreamOrder> g_order;
thread_local bool t_call_has_stream = false;
thread_local hipStream_t t_call_stream = nullptr;
thread_local int t_call_device = 0;

bool capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  return hipStreamIsCapturing(st, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

hipStream_t as_stream(void* s) {
  hipStream_t st = reinterpret_cast<hipStream_t>(s);
  if (capturing(st)) return st;
  int dev = 0;
  BC2N_HIP(hipGetDevice(&dev));
  {
    std::lock_guard<std::mutex> lk(g_order_mu);
    StreamOrder& o = g_order[dev];
    if (o.recorded && o.last != st) BC2N_HIP(hipStreamWaitEvent(st, o.ev, 0));
  }
  t_call_has_stream = true;
  t_call_stream = st;
  t_call_device = dev;
  return st;
}

// after a call: mark the end of its work on its stream
void end_call() {
  if (!t_call_has_stream) return;
  t_call_has_stream = false;
  std::lock_guard<std::mutex> lk(g_order_mu);
  StreamOrder& o = g_order[t_call_device];
  if (!o.ev && hipEventCreateWithFlags(&o.ev, hipEventDisableTiming) != hipSuccess) return;
  if (hipEventRecord(o.ev, t_call_stream) == hipSuccess) {
    o.last = t_call_stream;
    o.recorded = true;
  }
}

template <class F>
int guarded(F f) {
  t_call_has_stream = false;
  int rc = 0;
  try {
    f();
  } catch (const std::exception& e) {
    set_error(e.what());
    rc = 1;
  } catch (...) {
    set_error("unknown error");
    rc = 1;
  }
  end_call();
  return rc;
}

std::mutex g_mu;
std::map<std::pair<std::string, std::string>, TriAttnW> g_triattn;

const TriAttnW& triattn_w(const char* dir, const char* prefix) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto key = std::make_pair(std::string(dir), std::string(prefix));
  auto it = g_triattn.find(key);
  if (it != g_triattn.end()) return it->second;
  TriAttnW w = triattn_weights(weights(dir), prefix);
  return g_triattn.emplace(key, w).first->second;
}

std::map<std::pair<std::string, std::string>, TriMulW> g_trimul;

const TriMulW& trimul_w(const char* dir, const char* prefix) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto key = std::make_pair(std::string(dir), std::string(prefix));
  auto it = g_trimul.find(key);
  if (it != g_trimul.end()) return it->second;
  TriMulW w = trimul_weights(weights(dir), prefix);
  return g_trimul.emplace(key, w).first->second;
}

template <class W, class F>
const W& cached(std::map<std::pair<std::string, std::string>, W>& m, const char* dir,
                const char* prefix, F make) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto key = std::make_pair(std::string(dir), std::string(prefix));
  auto it = m.find(key);
  if (it != m.end()) return it->second;
  W w = make(weights(dir), std::string(prefix));
  return m.emplace(key, w).first->second;
}
std::map<std::pair<std::string, std::string>, TransW> g_trans;
std::map<std::pair<std::string, std::string>, OpmW> g_opm;
std::map<std::pair<std::string, std::string>, MsaRowW> g_row;
std::map<std::pair<std::string, std::string>, MsaColW> g_col;
std::map<std::pair<std::string, std::string>, StackW> g_stack;

const StackW& stack_w(const char* dir, int depth, StackKind kind) {
  const char* kn = kind == StackKind::EVO ? ":evo" : kind == StackKind::PAIR_ONLY ? ":pair_only" : ":tpl";
  const std::string tag = std::to_string(depth) + kn;
  return cached(g_stack, dir, tag.c_str(), [&](WeightStore& ws, const std::string&) {
    return stack_weights(ws, depth, kind);
  });
}
StackKind evo_kind(int64_t pair_only) { return pair_only ? StackKind::PAIR_ONLY : StackKind::EVO; }

// Library-owned save-set for detached forwards (save=0) and own_save=1.
struct OwnSave {
  void* p = nullptr;
  size_t n = 0;
  void* get(hipStream_t st, size_t need) {
    if (need > n) {
      if (p) {
        BC2N_HIP(hipStreamSynchronize(st));
        BC2N_HIP(hipFree(p));
        p = nullptr;
      }
      BC2N_HIP(hipMalloc(&p, need));
      n = need;
    }
    return p;
  }
};
OwnSave g_own;
// Scratch of detached forwards (save = 0): one block's worth, reused.
OwnSave g_det;

void need(bool ok, const char* msg) {
  if (!ok) throw std::invalid_argument(msg);
}

}  // namespace

extern "C" {

const char* bc2n_last_error(void) { return last_error(); }
int bc2n_abi_version(void) { return 4; }

size_t bc2n_triattn_save_bytes(int N, int C, int H) { return triattn_save_bytes(N, C, H); }

int bc2n_triattn_fwd(void* stream, const char* weights_dir, const char* prefix, int per_column,
                     int N, const float* pair, const float* pair_mask, const float* drop_tbl,
                     float* pair_out, void* save) {
  return guarded([&] {
    need(weights_dir && prefix, "weights_dir/prefix required");
    need(pair && pair_mask && pair_out && save, "null operand");
    need(pair_out != pair, "triattn: pair_out must not alias pair");
    const TriAttnW& w = triattn_w(weights_dir, prefix);
    triattn_fwd(as_stream(stream), w, per_column != 0, N, pair, pair_mask, drop_tbl, pair_out,
                save);
  });
}

int bc2n_triattn_fwd_noalloc(void* stream, const char* weights_dir, const char* prefix,
                             int per_column, int N, const float* pair, const float* pair_mask,
                             const float* drop_tbl, float* pair_out, void* save) {
  return guarded([&] {
    need(weights_dir && prefix, "weights_dir/prefix required");
    need(pair && pair_mask && pair_out && save, "null operand");
    need(pair_out != pair, "triattn: pair_out must not alias pair");
    const TriAttnW* w = nullptr;
    {
      // only weights already on the device: loading would allocate
      std::lock_guard<std::mutex> lk(g_mu);
      auto it = g_triattn.find(std::make_pair(std::string(weights_dir), std::string(prefix)));
      if (it != g_triattn.end()) w = &it->second;
    }
    need(w != nullptr,
         "triattn_fwd_noalloc: weights not resident; call bc2n_triattn_fwd once with this "
         "weights_dir and prefix first");
    triattn_fwd_noalloc(as_stream(stream), *w, per_column != 0, N, pair, pair_mask, drop_tbl,
                        pair_out, save);
  });
}

int bc2n_triattn_bwd(void* stream, const char* weights_dir, const char* prefix, int per_column,
                     int N, const float* pair, const float* pair_mask, const float* drop_tbl,
                     const void* save, const float* dpair_out, float* dpair_in) {
  return guarded([&] {
    need(weights_dir && prefix, "weights_dir/prefix required");
    need(pair && pair_mask && save && dpair_out && dpair_in, "null operand");
    const TriAttnW& w = triattn_w(weights_dir, prefix);
    triattn_bwd(as_stream(stream), w, per_column != 0, N, pair, pair_mask, drop_tbl, save,
                dpair_out, dpair_in);
  });
}

size_t bc2n_trimul_save_bytes(int N, int C, int I) { return trimul_save_bytes(N, C, I); }

int bc2n_trimul_fwd(void* stream, const char* weights_dir, const char* prefix, int outgoing,
                    int N, const float* pair, const float* pair_mask, const float* drop_tbl,
                    float* pair_out, void* save) {
  return guarded([&] {
    need(weights_dir && prefix, "weights_dir/prefix required");
    need(pair && pair_mask && pair_out && save, "null operand");
    need(pair_out != pair, "trimul: pair_out must not alias pair");
    const TriMulW& w = trimul_w(weights_dir, prefix);
    trimul_fwd(as_stream(stream), w, outgoing != 0, N, pair, pair_mask, drop_tbl, pair_out, save);
  });
}

int bc2n_trimul_bwd(void* stream, const char* weights_dir, const char* prefix, int outgoing,
                    int N, const float* pair, const float* pair_mask, const float* drop_tbl,
                    const void* save, const float* dpair_out, float* dpair_in) {
  return guarded([&] {
    need(weights_dir && prefix, "weights_dir/prefix required");
    need(pair && pair_mask && save && dpair_out && dpair_in, "null operand");
    const TriMulW& w = trimul_w(weights_dir, prefix);
    trimul_bwd(as_stream(stream), w, outgoing != 0, N, pair, pair_mask, drop_tbl, save, dpair_out,
               dpair_in);
  });
}

size_t bc2n_transition_save_bytes(long rows, int C, int factor) {
  return transition_save_bytes(rows, C, factor);
}

int bc2n_transition_fwd(void* stream, const char* weights_dir, const char* prefix, long rows,
                        int N, const float* act, const float* drop_tbl, float* act_out,
                        void* save) {
  return guarded([&] {
    need(weights_dir && prefix && act && act_out && save, "null operand");
    need(act_out != act, "transition: act_out must not alias act");
    need(rows > 0 && N > 0 && rows % N == 0, "transition: rows must be a multiple of N");
    const TransW& w = cached(g_trans, weights_dir, prefix, transition_weights);
    transition_fwd(as_stream(stream), w, rows, N, act, drop_tbl, act_out, save);
  });
}

int bc2n_transition_bwd(void* stream, const char* weights_dir, const char* prefix, long rows,
                        int N, const float* act, const float* drop_tbl, const void* save,
                        const float* dact_out, float* dact_in) {
  return guarded([&] {
    need(weights_dir && prefix && act && save && dact_out && dact_in, "null operand");
    const TransW& w = cached(g_trans, weights_dir, prefix, transition_weights);
    transition_bwd(as_stream(stream), w, rows, N, act, drop_tbl, save, dact_out, dact_in);
  });
}

size_t bc2n_opm_save_bytes(int S, int N, int O, int C) { return opm_save_bytes(S, N, O, C); }

int bc2n_opm_fwd(void* stream, const char* weights_dir, const char* prefix, int S, int N,
                 const float* msa, const float* msa_mask, const float* pair,
                 const float* drop_tbl, float* pair_out, void* save) {
  return guarded([&] {
    need(weights_dir && prefix && msa && msa_mask && pair && pair_out && save, "null operand");
    need(pair_out != pair, "opm: pair_out must not alias pair");
    const OpmW& w = cached(g_opm, weights_dir, prefix, opm_weights);
    opm_fwd(as_stream(stream), w, S, N, msa, msa_mask, pair, drop_tbl, pair_out, save);
  });
}

int bc2n_opm_bwd(void* stream, const char* weights_dir, const char* prefix, int S, int N,
                 const float* msa, const float* msa_mask, const float* drop_tbl, const void* save,
                 const float* dpair, const float* dmsa_out, float* dmsa_in) {
  return guarded([&] {
    need(weights_dir && prefix && msa && msa_mask && save && dpair && dmsa_out && dmsa_in,
         "null operand");
    const OpmW& w = cached(g_opm, weights_dir, prefix, opm_weights);
    opm_bwd(as_stream(stream), w, S, N, msa, msa_mask, drop_tbl, save, dpair, dmsa_out, dmsa_in);
  });
}

size_t bc2n_msarow_save_bytes(int S, int N, int Cm, int H) { return msarow_save_bytes(S, N, Cm, H); }

int bc2n_msarow_fwd(void* stream, const char* weights_dir, const char* prefix, int S, int N,
                    const float* msa, const float* msa_mask, const float* pair,
                    const float* drop_tbl, float* msa_out, void* save) {
  return guarded([&] {
    need(weights_dir && prefix && msa && msa_mask && pair && msa_out && save, "null operand");
    need(msa_out != msa, "msarow: msa_out must not alias msa");
    const MsaRowW& w = cached(g_row, weights_dir, prefix, msarow_weights);
    msarow_fwd(as_stream(stream), w, S, N, msa, msa_mask, pair, drop_tbl, msa_out, save);
  });
}

int bc2n_msarow_bwd(void* stream, const char* weights_dir, const char* prefix, int S, int N,
                    const float* msa, const float* msa_mask, const float* pair,
                    const float* drop_tbl, const void* save, const float* dmsa_out,
                    float* dmsa_in, float* dpair) {
  return guarded([&] {
    need(weights_dir && prefix && msa && msa_mask && pair && save && dmsa_out && dmsa_in && dpair,
         "null operand");
    const MsaRowW& w = cached(g_row, weights_dir, prefix, msarow_weights);
    msarow_bwd(as_stream(stream), w, S, N, msa, msa_mask, pair, drop_tbl, save, dmsa_out, dmsa_in,
               dpair);
  });
}

size_t bc2n_msacol_save_bytes(int S, int N, int Cm, int H) { return msacol_save_bytes(S, N, Cm, H); }

int bc2n_msacol_fwd(void* stream, const char* weights_dir, const char* prefix, int S, int N,
                    const float* msa, const float* msa_mask, const float* drop_tbl,
                    float* msa_out, void* save) {
  return guarded([&] {
    need(weights_dir && prefix && msa && msa_mask && msa_out && save, "null operand");
    need(msa_out != msa, "msacol: msa_out must not alias msa");
    const MsaColW& w = cached(g_col, weights_dir, prefix, msacol_weights);
    msacol_fwd(as_stream(stream), w, S, N, msa, msa_mask, drop_tbl, msa_out, save);
  });
}

std::map<std::pair<std::string, std::string>, MsaGlobW> g_glob;

size_t bc2n_msaglobal_save_bytes(const char* weights_dir, const char* prefix, int S, int N) {
  size_t n = 0;
  if (guarded([&] {
        need(weights_dir && prefix && S > 0 && N > 0, "bad arguments");
        const MsaGlobW& w = cached(g_glob, weights_dir, prefix, msaglobal_weights);
        n = msaglobal_save_bytes(w, S, N);
      }) != 0)
    return 0;
  return n;
}

int bc2n_msaglobal_fwd(void* stream, const char* weights_dir, const char* prefix, int S, int N,
                       const float* msa, const float* msa_mask, const float* drop_tbl,
                       float* msa_out, void* save) {
  return guarded([&] {
    need(weights_dir && prefix && msa && msa_mask && msa_out && save, "null operand");
    need(msa_out != msa, "msaglobal: msa_out must not alias msa");
    const MsaGlobW& w = cached(g_glob, weights_dir, prefix, msaglobal_weights);
    msaglobal_fwd(as_stream(stream), w, S, N, msa, msa_mask, drop_tbl, msa_out, save);
  });
}

int bc2n_msaglobal_bwd(void* stream, const char* weights_dir, const char* prefix, int S, int N,
                       const float* msa, const float* msa_mask, const float* drop_tbl,
                       const void* save, const float* dmsa_out, float* dmsa_in) {
  return guarded([&] {
    need(weights_dir && prefix && msa && msa_mask && save && dmsa_out && dmsa_in, "null operand");
    const MsaGlobW& w = cached(g_glob, weights_dir, prefix, msaglobal_weights);
    msaglobal_bwd(as_stream(stream), w, S, N, msa, msa_mask, drop_tbl, save, dmsa_out, dmsa_in);
  });
}

int bc2n_msacol_bwd(void* stream, const char* weights_dir, const char* prefix, int S, int N,
                    const float* msa, const float* msa_mask, const float* drop_tbl,
                    const void* save, const float* dmsa_out, float* dmsa_in) {
  return guarded([&] {
    need(weights_dir && prefix && msa && msa_mask && save && dmsa_out && dmsa_in, "null operand");
    const MsaColW& w = cached(g_col, weights_dir, prefix, msacol_weights);
    msacol_bwd(as_stream(stream), w, S, N, msa, msa_mask, drop_tbl, save, dmsa_out, dmsa_in);
  });
}

// ------------------------------------------------------------ the stack

size_t bc2n_evoformer_save_bytes(const char* weights_dir, int N, int S, int64_t depth,
                                 int64_t pair_only) {
  size_t n = 0;
  if (guarded([&] {
        need(weights_dir != nullptr, "weights_dir required");
        const StackW& w = stack_w(weights_dir, (int)depth, evo_kind(pair_only));
        n = stack_save_bytes(w, N, S, (int)depth) + 256;
      }) != 0)
    return 0;
  return n;
}

size_t bc2n_evoformer_detached_bytes(const char* weights_dir, int N, int S, int64_t depth,
                                     int64_t pair_only) {
  size_t n = 0;
  if (guarded([&] {
        need(weights_dir != nullptr, "weights_dir required");
        const StackW& w = stack_w(weights_dir, (int)depth, evo_kind(pair_only));
        n = stack_detached_bytes(w, N, S, (int)depth) + 256;
      }) != 0)
    return 0;
  return n;
}

int bc2n_set_save_policy(int policy) { return set_save_policy(policy); }

int bc2n_set_msa_overlap(int on) { return set_msa_overlap(on != 0) ? 1 : 0; }

int bc2n_evoformer_replays(const char* weights_dir, int N, int S, int64_t depth,
                           int64_t pair_only) {
  int r = -1;
  if (guarded([&] {
        need(weights_dir != nullptr, "weights_dir required");
        const StackW& w = stack_w(weights_dir, (int)depth, evo_kind(pair_only));
        r = stack_replays(w, N, S, (int)depth) ? 1 : 0;
      }) != 0)
    return -1;
  return r;
}

static const uint32_t* stack_key(hipStream_t st, const uint32_t* seed, int seed_len,
                                 uint32_t* scratch) {
  if (seed_len == 3) return seed;  // [k0, k1, enabled]: jax.random.key_data
  key_from_bits(st, seed, scratch);  // [bits, enabled]: PRNGKey(bits)
  return scratch;
}

int bc2n_evoformer_fwd(void* stream, const float* pair, const float* msa, const float* pair_mask,
                       const float* msa_mask, const uint32_t* seed, int seed_len, int N, int S,
                       int Cm, int64_t depth, int64_t save, int64_t pair_only, int64_t own_save,
                       int64_t opm_first, int64_t dropout, const char* weights_dir,
                       float* pair_out, float* msa_out, void* psave, void* msave) {
  (void)msave;
  return guarded([&] {
    hipStream_t st = as_stream(stream);
    need(weights_dir && pair && pair_mask && pair_out, "null operand");
    need(opm_first == 1, "evoformer: only outer_product_mean.first=True (AF2-multimer) is built");
    need(seed_len == 2 || seed_len == 3, "evoformer: seed must be u32[2] or u32[3]");
    need(!dropout || seed, "evoformer: dropout needs the seed operand");
    need(pair_only || (msa && msa_mask && msa_out), "evoformer: msa operands required");
    need(pair_out != pair && (pair_only || msa_out != msa), "evoformer: outputs must not alias inputs");
    const StackW& w = stack_w(weights_dir, (int)depth, evo_kind(pair_only));
    if (!pair_only) need(Cm == w.blocks[0].row.a.Cin, "evoformer: msa channel width mismatch");
    // save = 0: a detached forward (no backward follows), one block's scratch
    const bool detached = (save == 0);
    const size_t bytes = (detached ? stack_detached_bytes(w, N, S, (int)depth)
                                   : stack_save_bytes(w, N, S, (int)depth)) + 256;
    void* sv = detached ? g_det.get(st, bytes)
               : (own_save != 0 || psave == nullptr) ? g_own.get(st, bytes) : psave;
    uint32_t* keyslot = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(sv) + bytes - 256);
    const uint32_t* key = dropout ? stack_key(st, seed, seed_len, keyslot) : nullptr;
    const uint32_t* enabled = dropout ? seed + (seed_len - 1) : nullptr;
    stack_fwd(st, w, N, S, (int)depth, pair, msa, pair_mask, msa_mask, key, enabled, dropout != 0,
              pair_out, msa_out, sv, detached);
    if (pair_only && msa && msa_out && msa_out != msa && Cm > 0)
      BC2N_HIP(hipMemcpyAsync(msa_out, msa, (size_t)S * N * Cm * 4, hipMemcpyDeviceToDevice, st));
  });
}

int bc2n_evoformer_bwd(void* stream, const float* ct_pair, const float* ct_msa,
                       const float* pair_mask, const float* msa_mask, const void* psave,
                       const void* msave, const uint32_t* seed, int seed_len, int N, int S,
                       int Cm, int64_t depth, int64_t pair_only, int64_t own_save,
                       int64_t opm_first, int64_t dropout, const char* weights_dir,
                       float* dpair, float* dmsa) {
  (void)msave;
  (void)seed;
  (void)seed_len;
  return guarded([&] {
    hipStream_t st = as_stream(stream);
    need(weights_dir && ct_pair && pair_mask && dpair, "null operand");
    need(opm_first == 1, "evoformer: only outer_product_mean.first=True (AF2-multimer) is built");
    need(pair_only || (ct_msa && msa_mask && dmsa), "evoformer: msa operands required");
    const StackW& w = stack_w(weights_dir, (int)depth, evo_kind(pair_only));
    const size_t bytes = stack_save_bytes(w, N, S, (int)depth) + 256;
    const void* sv = (own_save != 0 || psave == nullptr) ? g_own.get(st, bytes) : psave;
    stack_bwd(st, w, N, S, (int)depth, pair_mask, msa_mask, dropout != 0, sv, ct_pair, ct_msa,
              dpair, dmsa);
    if (pair_only && dmsa && ct_msa && dmsa != ct_msa && Cm > 0)
      BC2N_HIP(hipMemcpyAsync(dmsa, ct_msa, (size_t)S * N * Cm * 4, hipMemcpyDeviceToDevice, st));
  });
}

// ------------------------------------------------------------ preallocation
// Called before the first real call (the reference calls its counterparts at
// trace time, before XLA has allocated): upload the component's weights and
// grow every scratch arena to what its calls at these shapes need, so that
// no call allocates afterwards.  The arenas' needs depend on the shapes, not
// on the depth, so one forward and backward of the first block on zero
// inputs (on the null stream, synchronised) grows them exactly; detached
// forwards' scratch is grown to its size as well.  Prints what it took.

namespace {

struct DevBuf {
  void* p = nullptr;
  explicit DevBuf(size_t n) {
    BC2N_HIP(hipMalloc(&p, n < 256 ? 256 : n));
    BC2N_HIP(hipMemset(p, 0, n < 256 ? 256 : n));
  }
  ~DevBuf() { if (p) (void)hipFree(p); }
  float* f() const { return static_cast<float*>(p); }
};

size_t free_bytes(size_t* total = nullptr) {
  size_t f = 0, t = 0;
  BC2N_HIP(hipMemGetInfo(&f, &t));
  if (total) *total = t;
  return f;
}

void report(const char* what, const std::string& shape, size_t f0) {
  size_t t = 0;
  const size_t f1 = free_bytes(&t);
  fprintf(stderr, "bc2n: prealloc %s %s took %.2f GB (%.2f of %.2f GB free after)\n", what,
          shape.c_str(), (double)((f0 > f1) ? f0 - f1 : 0) / 1e9, (double)f1 / 1e9,
          (double)t / 1e9);
}

void stack_dry_run(const StackW& w, int N, int S) {
  const long M = (long)N * N;
  const int Cz = w.blocks[0].tmo.C, Cm = w.pair_only ? 64 : w.blocks[0].row.a.Cin;
  const size_t sb = stack_save_bytes(w, N, S, 1);
  DevBuf pair(M * Cz * 4), pair_out(M * Cz * 4), dpair(M * Cz * 4), pmask(M * 4);
  DevBuf msa((size_t)S * N * Cm * 4), msa_out((size_t)S * N * Cm * 4),
      dmsa((size_t)S * N * Cm * 4), mmask((size_t)S * N * 4), save(sb);
  hipStream_t st = nullptr;
  stack_fwd(st, w, N, S, 1, pair.f(), w.pair_only ? nullptr : msa.f(),
            pmask.f(), mmask.f(), nullptr, nullptr, false, pair_out.f(),
            w.pair_only ? nullptr : msa_out.f(), save.p);
  stack_bwd(st, w, N, S, 1, pmask.f(), mmask.f(), false, save.p,
            pair_out.f(), w.pair_only ? nullptr : msa_out.f(), dpair.f(),
            w.pair_only ? nullptr : dmsa.f());
  BC2N_HIP(hipDeviceSynchronize());
}

}  // namespace

int bc2n_stack_prealloc(int N, int S, int depth, const char* weights_dir, int pair_only,
                        int opm_first, int dropout) {
  (void)dropout;
  return guarded([&] {
    need(weights_dir != nullptr, "weights_dir required");
    need(opm_first == 1, "evoformer: only outer_product_mean.first=True (AF2-multimer) is built");
    const size_t f0 = free_bytes();
    const StackW& w = stack_w(weights_dir, depth, evo_kind(pair_only));
    stack_dry_run(w, N, S);
    (void)g_det.get(nullptr, stack_detached_bytes(w, N, S, depth) + 256);
    BC2N_HIP(hipDeviceSynchronize());
    report("stack", "N=" + std::to_string(N) + " S=" + std::to_string(S) + " depth=" +
           std::to_string(depth) + " pair_only=" + std::to_string(pair_only), f0);
  });
}

int bc2n_tplstack_prealloc(int N, int depth, const char* weights_dir) {
  return guarded([&] {
    need(weights_dir != nullptr, "weights_dir required");
    const size_t f0 = free_bytes();
    stack_dry_run(stack_w(weights_dir, depth, StackKind::TEMPLATE), N, 1);
    report("tplstack", "N=" + std::to_string(N) + " depth=" + std::to_string(depth), f0);
  });
}

// (the structure-module and template-embedding counterparts follow their
// weight caches below)

int bc2n_save_slots_probe(const char* weights_dir, int depth, int N, int S, int pair_only) {
  int slots = -1;
  if (guarded([&] {
        need(weights_dir != nullptr, "weights_dir required");
        const StackW& w = stack_w(weights_dir, depth, evo_kind(pair_only));
        const size_t bytes = stack_save_bytes(w, N, S, depth) + 256;
        const size_t slot = (size_t)N * N * 128 * 2;  // one bf16 [N,N,128] slot
        slots = (int)((bytes + slot - 1) / slot);
      }) != 0)
    return -1;
  return slots;
}

// ------------------------------------------------------ template pair stack

size_t bc2n_tplstack_save_bytes(const char* weights_dir, int N, int64_t depth) {
  size_t n = 0;
  if (guarded([&] {
        need(weights_dir != nullptr, "weights_dir required");
        const StackW& w = stack_w(weights_dir, (int)depth, StackKind::TEMPLATE);
        n = stack_save_bytes(w, N, 1, (int)depth) + 256;
      }) != 0)
    return 0;
  return n;
}

int bc2n_tplstack_fwd(void* stream, const float* pair, const float* pair_mask,
                      const uint32_t* seed, int seed_len, int N, int64_t depth, int64_t dropout,
                      const char* weights_dir, float* out, void* save) {
  return guarded([&] {
    hipStream_t st = as_stream(stream);
    need(weights_dir && pair && pair_mask && out && save, "null operand");
    need(out != pair, "tplstack: out must not alias pair");
    need(seed_len == 2 || seed_len == 3, "tplstack: seed must be u32[2] or u32[3]");
    need(!dropout || seed, "tplstack: dropout needs the seed operand");
    const StackW& w = stack_w(weights_dir, (int)depth, StackKind::TEMPLATE);
    const size_t bytes = stack_save_bytes(w, N, 1, (int)depth) + 256;
    uint32_t* keyslot = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(save) + bytes - 256);
    const uint32_t* key = dropout ? stack_key(st, seed, seed_len, keyslot) : nullptr;
    const uint32_t* enabled = dropout ? seed + (seed_len - 1) : nullptr;
    stack_fwd(st, w, N, 1, (int)depth, pair, nullptr, pair_mask, nullptr, key, enabled,
              dropout != 0, out, nullptr, save);
  });
}

int bc2n_tplstack_bwd(void* stream, const float* ct, const float* pair_mask, const void* save,
                      const uint32_t* seed, int seed_len, int N, int64_t depth, int64_t dropout,
                      const char* weights_dir, float* dpair) {
  (void)seed;
  (void)seed_len;
  return guarded([&] {
    need(weights_dir && ct && pair_mask && save && dpair, "null operand");
    const StackW& w = stack_w(weights_dir, (int)depth, StackKind::TEMPLATE);
    stack_bwd(as_stream(stream), w, N, 1, (int)depth, pair_mask, nullptr, dropout != 0, save, ct,
              nullptr, dpair, nullptr);
  });
}

// --------------------------------------------------------- template embedding

namespace {
std::map<std::pair<std::string, std::string>, TplEmbedW> g_te;
const TplEmbedW& te_w(const char* dir, int depth) {
  return cached(g_te, dir, std::to_string(depth).c_str(), [&](WeightStore& ws, const std::string&) {
    return tplembed_weights(ws, depth);
  });
}
}  // namespace

int bc2n_tplembed_prealloc(int N, int depth, const char* weights_dir) {
  return guarded([&] {
    need(weights_dir != nullptr, "weights_dir required");
    const size_t f0 = free_bytes();
    const TplEmbedW& w = te_w(weights_dir, depth);
    const long M = (long)N * N;
    DevBuf query(M * 128 * 4), act_const(M * 64 * 4), pmask(M * 4), out(M * 128 * 4),
        dq(M * 128 * 4), save(tplembed_save_bytes(w, N) + 256);
    tplembed_fwd(nullptr, w, N, query.f(), act_const.f(), pmask.f(),
                 nullptr, nullptr, false, out.f(), save.p);
    tplembed_bwd(nullptr, w, N, query.f(), pmask.f(), false, save.p,
                 out.f(), dq.f());
    BC2N_HIP(hipDeviceSynchronize());
    report("tplembed", "N=" + std::to_string(N) + " depth=" + std::to_string(depth), f0);
  });
}

size_t bc2n_tplembed_save_bytes(const char* weights_dir, int N, int64_t depth) {
  size_t n = 0;
  if (guarded([&] {
        need(weights_dir != nullptr, "weights_dir required");
        n = tplembed_save_bytes(te_w(weights_dir, (int)depth), N) + 256;
      }) != 0)
    return 0;
  return n;
}

int bc2n_tplembed_fwd(void* stream, const float* query, const float* act_const,
                      const float* pair_mask, const uint32_t* seed, int seed_len, int N,
                      int64_t depth, int64_t dropout, const char* weights_dir, float* out,
                      void* save) {
  return guarded([&] {
    hipStream_t st = as_stream(stream);
    need(weights_dir && query && act_const && pair_mask && out && save, "null operand");
    need(seed_len == 2 || seed_len == 3, "tplembed: seed must be u32[2] or u32[3]");
    need(!dropout || seed, "tplembed: dropout needs the seed operand");
    const TplEmbedW& w = te_w(weights_dir, (int)depth);
    const size_t bytes = tplembed_save_bytes(w, N) + 256;
    uint32_t* keyslot = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(save) + bytes - 256);
    const uint32_t* key = dropout ? stack_key(st, seed, seed_len, keyslot) : nullptr;
    const uint32_t* enabled = dropout ? seed + (seed_len - 1) : nullptr;
    tplembed_fwd(st, w, N, query, act_const, pair_mask, key, enabled, dropout != 0, out, save);
  });
}

int bc2n_tplembed_bwd(void* stream, const float* ct, const float* query, const float* act_const,
                      const float* pair_mask, const void* save, const uint32_t* seed, int seed_len,
                      int N, int64_t depth, int64_t dropout, const char* weights_dir,
                      float* dquery) {
  (void)act_const;
  (void)seed;
  (void)seed_len;
  return guarded([&] {
    need(weights_dir && ct && query && pair_mask && save && dquery, "null operand");
    const TplEmbedW& w = te_w(weights_dir, (int)depth);
    tplembed_bwd(as_stream(stream), w, N, query, pair_mask, dropout != 0, save, ct, dquery);
  });
}

// ------------------------------------------------------------------ embedder

namespace {
std::map<std::pair<std::string, std::string>, EmbedW> g_emb;
const EmbedW& emb_w(const char* dir) {
  return cached(g_emb, dir, "", [&](WeightStore& ws, const std::string&) { return embed_weights(ws); });
}
}  // namespace

int bc2n_embedder_fwd(void* stream, const float* target_feat, const float* msa_feat,
                      const float* residue_index, const float* asym_id, const float* entity_id,
                      const float* sym_id, const int32_t* offset, int N, int S,
                      const char* weights_dir, float* msa, float* pair) {
  return guarded([&] {
    need(weights_dir != nullptr, "weights_dir required");
    embed_fwd(as_stream(stream), emb_w(weights_dir), N, S, target_feat, msa_feat, residue_index,
              asym_id, entity_id, sym_id, offset, msa, pair);
  });
}

int bc2n_embedder_bwd(void* stream, const float* dmsa, const float* dpair, const float* target_feat,
                      int N, int S, const char* weights_dir, float* dtarget_feat, float* dmsa_feat) {
  return guarded([&] {
    need(weights_dir != nullptr, "weights_dir required");
    embed_bwd(as_stream(stream), emb_w(weights_dir), N, S, dmsa, dpair, target_feat, dtarget_feat,
              dmsa_feat);
  });
}

// ------------------------------------------------ structure module folding

namespace {
std::map<std::string, FoldW> g_fold;
const FoldW& fold_w(const char* dir) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_fold.find(dir);
  if (it != g_fold.end()) return it->second;
  FoldW w = fold_weights(weights(dir));
  return g_fold.emplace(dir, w).first->second;
}
}  // namespace

size_t bc2n_fold_save_bytes(const char* weights_dir, int N, int64_t depth) {
  size_t n = 0;
  if (guarded([&] {
        need(weights_dir != nullptr, "weights_dir required");
        need(N > 0 && N <= 1024 && depth > 0, "fold: bad shape");
        (void)fold_w(weights_dir);
        n = fold_save_bytes(N, (int)depth) + 256;
      }) != 0)
    return 0;
  return n;
}

int bc2n_fold_fwd(void* stream, const float* single, const float* pair, const float* seq_mask,
                  const uint32_t* seed, int seed_len, int N, int64_t depth, int64_t dropout,
                  const char* weights_dir, float* act, float* traj, void* save) {
  return guarded([&] {
    hipStream_t st = as_stream(stream);
    need(weights_dir && single && pair && seq_mask && act && traj && save, "null operand");
    need(N > 0 && N <= 1024 && depth > 0, "fold: bad shape");
    need(seed_len == 2 || seed_len == 3, "fold: seed must be u32[2] or u32[3]");
    need(!dropout || seed, "fold: dropout needs the seed operand");
    const FoldW& w = fold_w(weights_dir);
    const size_t bytes = fold_save_bytes(N, (int)depth) + 256;
    uint32_t* keyslot = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(save) + bytes - 256);
    const uint32_t* key = dropout ? stack_key(st, seed, seed_len, keyslot) : nullptr;
    const uint32_t* enabled = dropout ? seed + (seed_len - 1) : nullptr;
    fold_fwd(st, w, N, (int)depth, single, pair, seq_mask, key, enabled, dropout != 0, act, traj,
             save);
  });
}

int bc2n_fold_bwd(void* stream, const float* d_act, const float* d_traj, const float* single,
                  const float* pair, const float* seq_mask, const void* save, int N,
                  int64_t depth, int64_t dropout, const char* weights_dir, float* dsingle,
                  float* dpair) {
  return guarded([&] {
    need(weights_dir && single && pair && seq_mask && save && dsingle && dpair, "null operand");
    need(N > 0 && N <= 1024 && depth > 0, "fold: bad shape");
    const FoldW& w = fold_w(weights_dir);
    fold_bwd(as_stream(stream), w, N, (int)depth, single, pair, seq_mask, dropout != 0, save,
             d_act, d_traj, dsingle, dpair);
  });
}

// ------------------------------------------------ structure module + heads

namespace {
std::map<std::pair<std::string, std::string>, StructHeadsW> g_sh;
const StructHeadsW& sh_w(const char* dir) {
  return cached(g_sh, dir, "", [&](WeightStore& ws, const std::string&) { return structheads_weights(ws); });
}
}  // namespace

int bc2n_sm_prealloc(int N, int depth, const char* weights_dir) {
  return guarded([&] {
    need(weights_dir != nullptr, "weights_dir required");
    need(N > 0 && N <= 1024 && depth > 0, "structure heads: bad shape");
    const size_t f0 = free_bytes();
    const StructHeadsW& w = sh_w(weights_dir);
    const long M = (long)N * N;
    DevBuf single((size_t)N * 384 * 4), pair(M * 128 * 4), seq_mask((size_t)N * 4),
        aatype((size_t)N * 4), atom14((size_t)N * 14 * 3 * 4), dgram(M * 64 * 4),
        pae(M * 64 * 4), plddt((size_t)N * 50 * 4), expres((size_t)N * 37 * 4),
        dsingle((size_t)N * 384 * 4), dpair(M * 128 * 4),
        save(structheads_save_bytes(N, 1) + 256);
    structheads_fwd(nullptr, w, N, 1, single.f(), pair.f(), seq_mask.f(),
                    aatype.f(), nullptr, nullptr, false, atom14.f(),
                    dgram.f(), pae.f(), plddt.f(), expres.f(),
                    save.p);
    structheads_bwd(nullptr, w, N, 1, single.f(), pair.f(), seq_mask.f(),
                    aatype.f(), false, save.p, atom14.f(), dgram.f(),
                    pae.f(), plddt.f(), expres.f(), dsingle.f(),
                    dpair.f());
    BC2N_HIP(hipDeviceSynchronize());
    report("structure module", "N=" + std::to_string(N) + " depth=" + std::to_string(depth), f0);
  });
}

size_t bc2n_structure_heads_save_bytes(const char* weights_dir, int N, int64_t depth) {
  size_t n = 0;
  if (guarded([&] {
        need(weights_dir != nullptr, "weights_dir required");
        need(N > 0 && N <= 1024 && depth > 0, "structure heads: bad shape");
        (void)sh_w(weights_dir);
        n = structheads_save_bytes(N, (int)depth) + 256;
      }) != 0)
    return 0;
  return n;
}

int bc2n_structure_heads_fwd(void* stream, const float* single, const float* pair,
                             const float* seq_mask, const float* aatype, const uint32_t* seed,
                             int seed_len, int N, int64_t depth, int64_t dropout,
                             const char* weights_dir, float* atom14, float* distogram, float* pae,
                             float* plddt, float* expres, void* save) {
  return guarded([&] {
    hipStream_t st = as_stream(stream);
    need(weights_dir && single && pair && seq_mask && aatype && save, "null operand");
    need(atom14 && distogram && pae && plddt && expres, "null output");
    need(N > 0 && N <= 1024 && depth > 0, "structure heads: bad shape");
    need(seed_len == 2 || seed_len == 3, "structure heads: seed must be u32[2] or u32[3]");
    need(!dropout || seed, "structure heads: dropout needs the seed operand");
    const StructHeadsW& w = sh_w(weights_dir);
    const size_t bytes = structheads_save_bytes(N, (int)depth) + 256;
    uint32_t* keyslot = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(save) + bytes - 256);
    const uint32_t* key = dropout ? stack_key(st, seed, seed_len, keyslot) : nullptr;
    const uint32_t* enabled = dropout ? seed + (seed_len - 1) : nullptr;
    structheads_fwd(st, w, N, (int)depth, single, pair, seq_mask, aatype, key, enabled,
                    dropout != 0, atom14, distogram, pae, plddt, expres, save);
  });
}

int bc2n_structure_heads_bwd(void* stream, const float* single, const float* pair,
                             const float* seq_mask, const float* aatype, const float* d_atom14,
                             const float* d_distogram, const float* d_pae, const float* d_plddt,
                             const float* d_expres, void* save, int N, int64_t depth,
                             int64_t dropout, const char* weights_dir, float* dsingle,
                             float* dpair) {
  return guarded([&] {
    need(weights_dir && single && pair && seq_mask && aatype && save && dsingle && dpair,
         "null operand");
    need(N > 0 && N <= 1024 && depth > 0, "structure heads: bad shape");
    const StructHeadsW& w = sh_w(weights_dir);
    structheads_bwd(as_stream(stream), w, N, (int)depth, single, pair, seq_mask, aatype,
                    dropout != 0, save, d_atom14, d_distogram, d_pae, d_plddt, d_expres, dsingle,
                    dpair);
  });
}

// ------------------------------------------------------- one-call design step

namespace {
std::map<std::string, DesignStepW> g_ds;
// The recycle terms' weights live in the embedder's directory
// (native/design_step.cuh:884, bindcraft/af/native.py:515-527).
RecycleW recycle_w(WeightStore& ews) {
  auto rec = [&](const char* name, size_t n) {
    const std::string k = std::string("param/") + name;
    if (ews.host(k).data.size() != n)
      throw std::runtime_error(std::string("recycle terms: ") + k + " has the wrong size");
    return ews.f32(k);
  };
  RecycleW r;
  r.wpp = rec("prev_pos_linear/weights", 15 * 128);
  r.bpp = rec("prev_pos_linear/bias", 128);
  r.s_msa = rec("prev_msa_first_row_norm/scale", 256);
  r.o_msa = rec("prev_msa_first_row_norm/offset", 256);
  r.s_pair = rec("prev_pair_norm/scale", 128);
  r.o_pair = rec("prev_pair_norm/offset", 128);
  return r;
}

const DesignStepW& ds_w(const char* emb, const char* tpl, const char* extra, const char* main,
                        const char* post, int64_t dt, int64_t de, int64_t dm, int64_t df) {
  need(emb && tpl && extra && main && post, "design step: five weights directories required");
  const std::string key = std::string(emb) + "|" + tpl + "|" + extra + "|" + main + "|" + post +
                          "|" + std::to_string(dt) + "," + std::to_string(de) + "," +
                          std::to_string(dm) + "," + std::to_string(df);
  {
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_ds.find(key);
    if (it != g_ds.end()) return it->second;
  }
  DesignStepW w;
  w.d_tpl = (int)dt; w.d_extra = (int)de; w.d_main = (int)dm; w.d_fold = (int)df;
  w.emb = emb_w(emb);
  WeightStore& ews = weights(emb);
  w.wsa = ews.f32("param/single_activations/weights");
  w.bsa = ews.f32("param/single_activations/bias");
  if (ews.host("param/single_activations/weights").data.size() != 256u * 384u)
    throw std::runtime_error("design step: single_activations must be [256,384]");
  w.rec = recycle_w(ews);
  w.tpl = te_w(tpl, (int)dt);
  w.extra = stack_w(extra, (int)de, StackKind::PAIR_ONLY);
  w.main = stack_w(main, (int)dm, StackKind::EVO);
  w.sh = sh_w(post);
  WeightStore& pws = weights(post);
  // the template's MSA row: Linears in the embedder's directory, chi tables
  // in the structure module's (both optional; the row needs all six)
  auto opt = [](WeightStore& ws, const char* name, size_t n) -> const float* {
    if (!ws.has(name)) return nullptr;
    if (ws.host(name).data.size() != n)
      throw std::runtime_error(std::string("design step: ") + name + " has the wrong size");
    return ws.f32(name);
  };
  w.trow.w1 = opt(ews, "param/template_single_embedding/weights", 34 * 256);
  w.trow.b1 = opt(ews, "param/template_single_embedding/bias", 256);
  w.trow.w2 = opt(ews, "param/template_projection/weights", 256 * 256);
  w.trow.b2 = opt(ews, "param/template_projection/bias", 256);
  w.trow.chi_idx = opt(pws, "const/chi_atom_indices", 21 * 16);
  w.trow.chi_mask = opt(pws, "const/chi_angles_mask", 21 * 4);
  if (pws.has("const/atom37_to_atom14") && pws.has("const/atom37_mask")) {
    if (pws.host("const/atom37_to_atom14").data.size() != 21u * 37u ||
        pws.host("const/atom37_mask").data.size() != 21u * 37u)
      throw std::runtime_error("design step: the atom37 tables must be [21,37]");
    w.a37_14 = pws.f32("const/atom37_to_atom14");
    w.a37_mask = pws.f32("const/atom37_mask");
  }
  std::lock_guard<std::mutex> lk(g_mu);
  return g_ds.emplace(key, w).first->second;
}
}  // namespace

size_t bc2n_design_step_save_bytes(const char* emb_dir, const char* tpl_dir,
                                   const char* extra_dir, const char* main_dir,
                                   const char* post_dir, int N, int S, int64_t d_tpl,
                                   int64_t d_extra, int64_t d_main, int64_t d_fold) {
  size_t n = 0;
  if (guarded([&] {
        const DesignStepW& w =
            ds_w(emb_dir, tpl_dir, extra_dir, main_dir, post_dir, d_tpl, d_extra, d_main, d_fold);
        need(N > 0 && S > 0, "design step: bad shape");
        n = design_step_save_bytes(w, N, S);
      }) != 0)
    return 0;
  return n;
}

int bc2n_design_step_fwd(void* stream, const float* target_feat, const float* msa_feat,
                         const float* residue_index, const float* asym_id,
                         const float* entity_id, const float* sym_id, const int32_t* offset,
                         const float* seq_mask, const float* act_const, const float* aatype,
                         const uint32_t* seeds, int N, int S, int64_t d_tpl, int64_t d_extra,
                         int64_t d_main, int64_t d_fold, int64_t dropout, int64_t recycles,
                         const char* emb_dir, const char* tpl_dir, const char* extra_dir,
                         const char* main_dir, const char* post_dir, float* atom14,
                         float* distogram, float* pae, float* plddt, float* expres, void* save) {
  return guarded([&] {
    need(target_feat && msa_feat && residue_index && asym_id && entity_id && sym_id && seq_mask &&
             aatype && save, "null operand");
    need(atom14 && distogram && pae && plddt && expres, "null output");
    need(!dropout || seeds, "design step: dropout needs the seeds operand");
    const DesignStepW& w =
        ds_w(emb_dir, tpl_dir, extra_dir, main_dir, post_dir, d_tpl, d_extra, d_main, d_fold);
    design_step_fwd(as_stream(stream), w, N, S, target_feat, msa_feat, residue_index, asym_id,
                    entity_id, sym_id, offset, seq_mask, act_const, aatype, seeds, dropout != 0,
                    (int)recycles, atom14, distogram, pae, plddt, expres, save);
  });
}

int bc2n_design_step_bwd(void* stream, const float* target_feat, const float* seq_mask,
                         const float* aatype, int64_t with_template, const float* d_atom14,
                         const float* d_distogram, const float* d_pae, const float* d_plddt,
                         const float* d_expres, void* save, int N, int S, int64_t d_tpl,
                         int64_t d_extra, int64_t d_main, int64_t d_fold, int64_t dropout,
                         const char* emb_dir, const char* tpl_dir, const char* extra_dir,
                         const char* main_dir, const char* post_dir, float* d_target_feat,
                         float* d_msa_feat) {
  return guarded([&] {
    need(target_feat && seq_mask && aatype && save && d_target_feat && d_msa_feat, "null operand");
    const DesignStepW& w =
        ds_w(emb_dir, tpl_dir, extra_dir, main_dir, post_dir, d_tpl, d_extra, d_main, d_fold);
    design_step_bwd(as_stream(stream), w, N, S, target_feat, seq_mask, with_template != 0, aatype,
                    dropout != 0, save, d_atom14, d_distogram, d_pae, d_plddt, d_expres,
                    d_target_feat, d_msa_feat);
  });
}

int bc2n_seqfeat_fwd(void* stream, const float* logits, const uint8_t* flags, const float* aa_bias,
                     float softmax_weight, float one_hot_weight, float temperature,
                     float logit_scale, float omitted_half, const float* scalars, int N,
                     float* feat, float* prof) {
  return guarded([&] {
    need(logits && flags && feat && prof, "null operand");
    need(N > 0, "seqfeat: N must be positive");
    need(scalars || temperature != 0.f, "seqfeat: temperature must be non-zero");
    seqfeat_fwd(as_stream(stream), logits, flags, aa_bias,
                SeqScalars{softmax_weight, one_hot_weight, temperature, logit_scale}, scalars,
                omitted_half, N, feat, prof);
  });
}

int bc2n_seqfeat_bwd(void* stream, const float* logits, const uint8_t* flags, const float* aa_bias,
                     const float* d_feat, const float* d_prof, float softmax_weight,
                     float one_hot_weight, float temperature, float logit_scale,
                     float omitted_half, const float* scalars, int N, float* d_logits) {
  return guarded([&] {
    need(logits && flags && d_feat && d_prof && d_logits, "null operand");
    need(N > 0, "seqfeat: N must be positive");
    need(scalars || temperature != 0.f, "seqfeat: temperature must be non-zero");
    seqfeat_bwd(as_stream(stream), logits, flags, aa_bias,
                SeqScalars{softmax_weight, one_hot_weight, temperature, logit_scale}, scalars,
                omitted_half, N, d_feat, d_prof, d_logits);
  });
}

int bc2n_design_inputs_fwd(void* stream, const float* feat, const float* prof, int N,
                           float* target_feat, float* msa_feat, float* aatype) {
  return guarded([&] {
    need(feat && prof && target_feat && msa_feat && aatype, "null operand");
    need(N > 0, "design inputs: N must be positive");
    design_inputs_fwd(as_stream(stream), feat, prof, N, target_feat, msa_feat, aatype);
  });
}

int bc2n_design_inputs_bwd(void* stream, const float* d_target_feat, const float* d_msa_feat,
                           int N, float* d_feat, float* d_prof) {
  return guarded([&] {
    need(d_target_feat && d_msa_feat && d_feat && d_prof, "null operand");
    need(N > 0, "design inputs: N must be positive");
    design_inputs_bwd(as_stream(stream), d_target_feat, d_msa_feat, N, d_feat, d_prof);
  });
}

size_t bc2n_design_step_seq_save_bytes(const char* emb_dir, const char* tpl_dir,
                                       const char* extra_dir, const char* main_dir,
                                       const char* post_dir, int N, int64_t d_tpl,
                                       int64_t d_extra, int64_t d_main, int64_t d_fold) {
  size_t n = 0;
  if (guarded([&] {
        const DesignStepW& w =
            ds_w(emb_dir, tpl_dir, extra_dir, main_dir, post_dir, d_tpl, d_extra, d_main, d_fold);
        need(N > 0, "design step: bad shape");
        n = design_step_seq_save_bytes(w, N);
      }) != 0)
    return 0;
  return n;
}

int bc2n_design_step_seq_fwd(void* stream, const float* logits, const uint8_t* flags,
                             const float* aa_bias, const float* scalars, float omitted_half,
                             const float* residue_index, const float* asym_id,
                             const float* entity_id, const float* sym_id, const int32_t* offset,
                             const float* seq_mask, const float* act_const,
                             const uint32_t* seeds, int N, const int32_t* n, int64_t d_tpl,
                             int64_t d_extra, int64_t d_main, int64_t d_fold, int64_t dropout,
                             int64_t recycles, int64_t cyclic_mode, float flexibility,
                             const char* emb_dir, const char* tpl_dir,
                             const char* extra_dir, const char* main_dir, const char* post_dir,
                             float* atom14, float* distogram, float* pae, float* plddt,
                             float* expres, const float* tpl_atoms37, const float* tpl_mask37,
                             float* atom37,
                             float* atom37_mask, const int32_t* interface_asym,
                             float* conf_plddt, float* conf_pae, float* ptm, float* iptm,
                             float* iptm_per_residue, float* expres_ca, void* save) {
  return guarded([&] {
    need(logits && flags && scalars && residue_index && asym_id && entity_id && sym_id &&
             seq_mask && save, "null operand");
    need(atom14 && distogram && pae && plddt && expres, "null output");
    need(!dropout || seeds, "design step: dropout needs the seeds operand");
    need(!conf_plddt || (interface_asym && conf_pae && ptm && iptm && iptm_per_residue && expres_ca),
         "design step: the confidence outputs come together, with interface_asym");
    const DesignStepW& w =
        ds_w(emb_dir, tpl_dir, extra_dir, main_dir, post_dir, d_tpl, d_extra, d_main, d_fold);
    design_step_seq_fwd(as_stream(stream), w, N, n, logits, flags, aa_bias, scalars, omitted_half,
                        residue_index, asym_id, entity_id, sym_id, offset, seq_mask, act_const,
                        seeds, dropout != 0, (int)recycles, (int)cyclic_mode, flexibility,
                        atom14, distogram, pae, plddt, expres,
                        AtomsOut{tpl_atoms37, tpl_mask37, atom37, atom37_mask},
                        ConfOut{interface_asym, conf_plddt, conf_pae, ptm, iptm, iptm_per_residue,
                                expres_ca},
                        save);
  });
}

int bc2n_design_step_seq_bwd(void* stream, const float* logits, const uint8_t* flags,
                             const float* aa_bias, const float* scalars, float omitted_half,
                             const float* seq_mask, int64_t with_template,
                             const float* d_atom14, const float* d_distogram, const float* d_pae,
                             const float* d_plddt, const float* d_expres, const float* d_atom37,
                             const int32_t* interface_asym, const float* d_conf_plddt,
                             const float* d_conf_pae, const float* d_ptm, const float* d_iptm,
                             const float* d_iptm_per_residue, const float* d_expres_ca, void* save,
                             int N, const int32_t* n, int64_t d_tpl, int64_t d_extra, int64_t d_main, int64_t d_fold,
                             int64_t dropout, const char* emb_dir, const char* tpl_dir,
                             const char* extra_dir, const char* main_dir, const char* post_dir,
                             float* d_logits) {
  return guarded([&] {
    need(logits && flags && scalars && seq_mask && save && d_logits, "null operand");
    const DesignStepW& w =
        ds_w(emb_dir, tpl_dir, extra_dir, main_dir, post_dir, d_tpl, d_extra, d_main, d_fold);
    design_step_seq_bwd(as_stream(stream), w, N, n, logits, flags, aa_bias, scalars, omitted_half,
                        seq_mask, with_template != 0, dropout != 0, save, d_atom14, d_distogram,
                        d_pae, d_plddt, d_expres, d_atom37,
                        ConfCt{interface_asym, d_conf_plddt, d_conf_pae, d_ptm, d_iptm,
                               d_iptm_per_residue, d_expres_ca},
                        d_logits);
  });
}

size_t bc2n_confidence_save_bytes(int N) { return N > 0 ? confidence_save_bytes(N) : 0; }

int bc2n_confidence_fwd(void* stream, const float* plddt_logits, const float* pae_logits,
                        const float* expres_logits, const float* seq_mask,
                        const int32_t* interface_asym, int N, float* plddt, float* pae,
                        float* ptm, float* iptm, float* iptm_per_residue, float* expres_ca,
                        void* save) {
  return guarded([&] {
    need(plddt_logits && pae_logits && expres_logits && seq_mask && interface_asym && save,
         "null operand");
    need(plddt && pae && ptm && iptm && iptm_per_residue && expres_ca, "null output");
    confidence_fwd(as_stream(stream), plddt_logits, pae_logits, expres_logits, seq_mask,
                   interface_asym, N, plddt, pae, ptm, iptm, iptm_per_residue, expres_ca, save);
  });
}

int bc2n_confidence_bwd(void* stream, const float* plddt_logits, const float* pae_logits,
                        const float* expres_logits, const float* seq_mask,
                        const int32_t* interface_asym, const void* save, const float* d_plddt,
                        const float* d_pae, const float* d_ptm, const float* d_iptm,
                        const float* d_iptm_per_residue, const float* d_expres_ca, int N,
                        float* d_plddt_logits, float* d_pae_logits, float* d_expres_logits) {
  return guarded([&] {
    need(plddt_logits && pae_logits && expres_logits && seq_mask && interface_asym && save,
         "null operand");
    need(d_plddt_logits && d_pae_logits && d_expres_logits, "null output");
    confidence_bwd(as_stream(stream), plddt_logits, pae_logits, expres_logits, seq_mask,
                   interface_asym, N, save, d_plddt, d_pae, d_ptm, d_iptm, d_iptm_per_residue,
                   d_expres_ca, d_plddt_logits, d_pae_logits, d_expres_logits);
  });
}

int bc2n_dropout_table(void* stream, float* tbl, int B, int C, uint32_t k0, uint32_t k1,
                       float rate) {
  return guarded([&] {
    need(tbl && B > 0 && C > 0, "bad table shape");
    need(rate >= 0.f && rate < 1.f, "rate must be in [0,1)");
    const float keep = 1.0f - rate;
    dropout_table(as_stream(stream), tbl, B, C, k0, k1, keep);
  });
}

int bc2n_bernoulli_bits(void* stream, uint8_t* out, long n, uint32_t k0, uint32_t k1,
                        float rate) {
  return guarded([&] {
    need(out && n > 0, "bad output");
    need(rate >= 0.f && rate < 1.f, "rate must be in [0,1)");
    bernoulli_bits(as_stream(stream), out, n, k0, k1, 1.0f - rate);
  });
}

int bc2n_stack_keys(void* stream, const uint32_t* seed, int depth, uint32_t* out) {
  return guarded([&] {
    need(seed && out && depth > 0, "bad arguments");
    stack_keys(as_stream(stream), seed, depth, out);
  });
}

int bc2n_prof_enable(int on) {
  return guarded([&] { kprof_enable(on != 0); });
}

int bc2n_prof_filter(const char* name) {
  return guarded([&] { kprof_filter(name); });
}

int bc2n_prof_read(char* names, int name_len, double* ms, int* counts, int cap) {
  int n = -1;
  if (guarded([&] { n = kprof_read(names, name_len, ms, counts, cap); }) != 0) return -1;
  return n;
}

int bc2n_probe_gemm(void* stream, int M, int N, int K, const uint16_t* A, const uint16_t* B,
                    float* C) {
  return guarded([&] {
    need(A && B && C, "null operand");
    GemmArgs g;
    g.M = M; g.N = N; g.K = K;
    g.A = reinterpret_cast<const h16*>(A); g.a_sm = K; g.a_sk = 1;
    g.B = reinterpret_cast<const h16*>(B); g.b_sn = K; g.b_sk = 1;
    gemm<128, 128>(as_stream(stream), g, EpiStore<float>{C, N, 0, nullptr, N});
  });
}

double bc2n_probe_mfma(void* stream, int form, int blocks, int iters, float* out) {
  double flops = -1.0;
  if (guarded([&] { flops = probe_mfma_rate(as_stream(stream), form, blocks, iters, out); }) != 0)
    return -1.0;
  return flops;
}

int bc2n_probe_gemm_f32(void* stream, int M, int N, int K, int batch, const float* A,
                        long a_sm, long a_sk, long a_sb, const float* B, long b_sk, long b_sn,
                        long b_sb, float* C, long c_sm, long c_sn, long c_sb) {
  return guarded([&] {
    GemmF32 g;
    g.M = M; g.N = N; g.K = K; g.batch = batch;
    g.A = A; g.a_sm = a_sm; g.a_sk = a_sk; g.a_sb = a_sb;
    g.B = B; g.b_sk = b_sk; g.b_sn = b_sn; g.b_sb = b_sb;
    g.C = C; g.c_sm = c_sm; g.c_sn = c_sn; g.c_sb = c_sb;
    gemm_f32(as_stream(stream), g, "probe.gemm_f32");
  });
}

int bc2n_probe_recycle(void* stream, int N, const char* emb_dir, const float* aatype,
                       const float* prev_atom14, const float* prev_pair, const float* prev_msa0,
                       float* pair, float* msa0) {
  return guarded([&] {
    need(emb_dir && pair && msa0, "null operand");
    RecycleW r = recycle_w(weights(emb_dir));
    recycle_terms(as_stream(stream), r, N, aatype, prev_atom14, prev_pair, prev_msa0, pair, msa0);
  });
}

int bc2n_probe_layernorm(void* stream, long M, int C, const float* x, const float* gamma,
                         const float* beta, int fast, uint16_t* y, float* mean, float* rstd) {
  return guarded([&] {
    need(x && gamma && beta && y && mean && rstd, "null operand");
    ln_fwd_f32(as_stream(stream), x, M, C, 0, gamma, beta, reinterpret_cast<h16*>(y), mean,
               rstd, fast != 0, 0, nullptr, nullptr);
  });
}

}  // extern "C"
