// The C ABI (include/bc2n.h): argument checks, weight lookup, error channel.
#include "../../include/bc2n.h"
#include "gemm.h"
#include "modules.h"

#include <map>
#include <tuple>

using namespace bc2n;

namespace {

template <class F>
int guarded(F f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    set_error(e.what());
    return 1;
  } catch (...) {
    set_error("unknown error");
    return 1;
  }
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

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

void need(bool ok, const char* msg) {
  if (!ok) throw std::invalid_argument(msg);
}

}  // namespace

extern "C" {

const char* bc2n_last_error(void) { return last_error(); }
int bc2n_abi_version(void) { return 1; }

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
    g.A = reinterpret_cast<const bf16*>(A); g.a_sm = K; g.a_sk = 1;
    g.B = reinterpret_cast<const bf16*>(B); g.b_sn = K; g.b_sk = 1;
    gemm<128, 128>(as_stream(stream), g, EpiStore<float>{C, N, 0, nullptr, N});
  });
}

int bc2n_probe_layernorm(void* stream, long M, int C, const float* x, const float* gamma,
                         const float* beta, int fast, uint16_t* y, float* mean, float* rstd) {
  return guarded([&] {
    need(x && gamma && beta && y && mean && rstd, "null operand");
    ln_fwd_f32(as_stream(stream), x, M, C, 0, gamma, beta, reinterpret_cast<bf16*>(y), mean,
               rstd, fast != 0, 0, nullptr, nullptr);
  });
}

}  // extern "C"
