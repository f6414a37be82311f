// Host runtime: weights manifests, device weight forms, scratch arena and the
// status-code error channel of the C ABI.
#pragma once
#include "common.h"
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <vector>

namespace bc2n {

struct HipError : std::runtime_error {
  using std::runtime_error::runtime_error;
};

void hip_check(hipError_t e, const char* what);
#define BC2N_HIP(x) ::bc2n::hip_check((x), #x)

// One tensor of a weights manifest: `name file ndim d0 d1 ...` + raw LE f32.
struct HostTensor {
  std::vector<int> shape;
  std::vector<float> data;
  size_t size() const { return data.size(); }
};

// A weights directory as written by the reference's manifest writer
// (bindcraft/af/native.py weights_from_params): manifest.txt plus one .f32
// file per parameter, names param/block{b}/<module path>/<param>.  Device
// forms (f32 copies, transposed h16 GEMM operands) are built on first use
// and kept for the life of the process.
class WeightStore {
 public:
  explicit WeightStore(const std::string& dir);
  bool has(const std::string& name) const { return host_.count(name) != 0; }
  const HostTensor& host(const std::string& name) const;
  // f32 copy on the device.
  const float* f32(const std::string& name);
  // A device buffer built once from host data by `make` under cache key `key`.
  template <class T, class F>
  const T* derived(const std::string& key, F make) {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = dev_.find(key);
    if (it != dev_.end()) return reinterpret_cast<const T*>(it->second);
    std::vector<T> h = make();
    void* d = upload(h.data(), h.size() * sizeof(T));
    dev_[key] = d;
    return reinterpret_cast<const T*>(d);
  }
  const std::string& dir() const { return dir_; }

 private:
  void* upload(const void* src, size_t bytes);
  std::string dir_;
  std::map<std::string, HostTensor> host_;
  std::map<std::string, void*> dev_;
  std::mutex mu_;
};

// Process-wide cache of weight stores keyed by directory.
WeightStore& weights(const std::string& dir);

// Host-side conversions used to build GEMM operands.
std::vector<h16> to_h16(const std::vector<float>& v);
// [rows][cols] f32 -> [cols][rows] h16
std::vector<h16> transpose_h16(const float* src, int rows, int cols);

// Grow-only device scratch arena, carved by bump allocation per call.  One
// arena per work lane (below); callers hold `lock()` for the duration of a
// call.
class Arena {
 public:
  void reset(hipStream_t st, size_t need);
  void* take(size_t bytes);
  template <class T>
  T* take_n(size_t n) { return reinterpret_cast<T*>(take(n * sizeof(T))); }
  std::recursive_mutex& lock() { return mu_; }

 private:
  char* base_ = nullptr;
  size_t cap_ = 0, off_ = 0;
  std::recursive_mutex mu_;
};
// The current work lane's arena.
Arena& arena();

// Work lanes.  The Evoformer stacks issue the MSA side of a block (row and
// column attention and the MSA transition, forward; the transition and
// column attention, backward) on a second stream beside the pair track.  A
// module call takes its scratch from the arena of the lane the issuing thread
// is in (lane 0 = the caller's stream, 1 = the side stream), so work of the
// two lanes never shares scratch; the cotangent-scale partials are per lane
// as well.  The library drives one device per process.
constexpr int NUM_LANES = 2;
int lane();
struct LaneGuard {
  int old;
  explicit LaneGuard(int l);
  ~LaneGuard();
};
// The side stream (created on first use, default priority, non-blocking).
hipStream_t side_stream();
// `to` waits for all work issued to `from` so far (an event recorded on
// `from`; captured into a graph when `from` is being captured).
void stream_wait(hipStream_t to, hipStream_t from);
// Whether the stacks overlap the MSA side with the pair track (on by
// default); returns the previous setting.  Off: everything on one stream.
bool set_msa_overlap(bool on);
bool msa_overlap();
// A grow-only device buffer of at least `bytes` (the stacks' second pair
// cotangent when the two streams alternate them); growing waits for the
// device first.  Grown by the preallocation calls' dry runs.
float* stack_pair_scratch(size_t bytes);

// Compute units of the current device (cached per device).
int device_cus();

// Per-kernel device timing: when enabled, every launch site wrapped in
// KTimed records a HIP event pair on its own stream; kprof_read() syncs the
// events and returns per-name totals.  Off by default (no events recorded).
void kprof_enable(bool on);
bool kprof_on();
// Restrict the timer to launches named `name` (null: every launch): events
// around one kernel's launches only perturb the rest of the step least.
void kprof_filter(const char* name);
bool kprof_wants(const char* name);
void kprof_record(const char* name, hipEvent_t a, hipEvent_t b);
hipEvent_t kprof_event();
// Fills names/ms/counts (up to cap entries), returns the number of entries,
// and clears the records.
int kprof_read(char* names, int name_len, double* ms, int* counts, int cap);

// Timer name of a module launch by its channel width C: the pair track's
// names at C = 128, "tpl."-prefixed ones at C = 64 (the template stack),
// "msa."-prefixed ones otherwise (the MSA transition's C = 256), so a
// per-kernel table never mixes launches of different widths under one name.
#define BC2N_TN(C, name) ((C) == 128 ? name : (C) == 64 ? "tpl." name : "msa." name)

struct KTimed {
  const char* name;
  hipStream_t st;
  hipEvent_t a = nullptr;
  KTimed(const char* n, hipStream_t s) : name(n), st(s) {
    if (kprof_on() && kprof_wants(n)) {
      a = kprof_event();
      hip_check(hipEventRecord(a, st), "hipEventRecord");
    }
  }
  ~KTimed() {
    if (a) {
      hipEvent_t b = kprof_event();
      if (hipEventRecord(b, st) == hipSuccess) kprof_record(name, a, b);
    }
  }
};

// Host-side operand check before any launch: a null device pointer becomes
// an error status, never a kernel reading address 0.
inline void nonnull(const void* p, const char* what) {
  if (p == nullptr) throw std::invalid_argument(std::string("null operand: ") + what);
}

// Thread-local last error message of the C ABI.
void set_error(const std::string& msg);
const char* last_error();

// Sequential carve of a caller-owned buffer (save-sets).
struct Carver {
  char* p;
  size_t off = 0;
  explicit Carver(void* base) : p(reinterpret_cast<char*>(base)) {}
  template <class T>
  T* take(size_t n) {
    T* r = reinterpret_cast<T*>(p + off);
    off += (n * sizeof(T) + 255) & ~size_t(255);
    return r;
  }
};
// The same walk, counting bytes only.
struct Sizer {
  size_t off = 0;
  template <class T>
  T* take(size_t n) {
    off += (n * sizeof(T) + 255) & ~size_t(255);
    return nullptr;
  }
};

}  // namespace bc2n
