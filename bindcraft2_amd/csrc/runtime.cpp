#include "runtime.h"

#include <cstdio>
#include <fstream>
#include <sstream>

namespace bc2n {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess)
    throw HipError(std::string(what) + ": " + hipGetErrorString(e));
}

WeightStore::WeightStore(const std::string& dir) : dir_(dir) {
  std::ifstream mf(dir + "/manifest.txt");
  if (!mf) throw std::runtime_error("weights: cannot open " + dir + "/manifest.txt");
  std::string line;
  while (std::getline(mf, line)) {
    if (line.empty()) continue;
    std::istringstream ss(line);
    std::string name, file;
    int nd = 0;
    ss >> name >> file >> nd;
    if (!ss || nd < 0 || nd > 8) throw std::runtime_error("weights: bad manifest line: " + line);
    HostTensor t;
    size_t n = 1;
    for (int i = 0; i < nd; ++i) {
      int d = 0;
      ss >> d;
      if (!ss || d < 0) throw std::runtime_error("weights: bad dims: " + line);
      t.shape.push_back(d);
      n *= (size_t)d;
    }
    t.data.resize(n);
    std::ifstream bf(dir + "/" + file, std::ios::binary);
    if (!bf) throw std::runtime_error("weights: missing file " + file);
    bf.read(reinterpret_cast<char*>(t.data.data()), (std::streamsize)(n * 4));
    if ((size_t)bf.gcount() != n * 4) throw std::runtime_error("weights: short file " + file);
    host_[name] = std::move(t);
  }
}

const HostTensor& WeightStore::host(const std::string& name) const {
  auto it = host_.find(name);
  if (it == host_.end()) throw std::runtime_error("weights: no parameter " + name + " in " + dir_);
  return it->second;
}

void* WeightStore::upload(const void* src, size_t bytes) {
  void* d = nullptr;
  BC2N_HIP(hipMalloc(&d, bytes < 16 ? 16 : bytes));
  BC2N_HIP(hipMemcpy(d, src, bytes, hipMemcpyHostToDevice));
  return d;
}

const float* WeightStore::f32(const std::string& name) {
  const HostTensor& t = host(name);
  return derived<float>("f32:" + name, [&] { return t.data; });
}

WeightStore& weights(const std::string& dir) {
  static std::mutex mu;
  static std::map<std::string, std::unique_ptr<WeightStore>> stores;
  std::lock_guard<std::mutex> lk(mu);
  auto& p = stores[dir];
  if (!p) p.reset(new WeightStore(dir));
  return *p;
}

std::vector<h16> to_h16(const std::vector<float>& v) {
  std::vector<h16> o(v.size());
  for (size_t i = 0; i < v.size(); ++i) o[i] = (h16)v[i];
  return o;
}

std::vector<h16> transpose_h16(const float* src, int rows, int cols) {
  std::vector<h16> o((size_t)rows * cols);
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < cols; ++c) o[(size_t)c * rows + r] = (h16)src[(size_t)r * cols + c];
  return o;
}

void Arena::reset(hipStream_t st, size_t need) {
  off_ = 0;
  if (need <= cap_) return;
  (void)st;
  if (base_) {
    // queued kernels may still read the old block, on either stream
    BC2N_HIP(hipDeviceSynchronize());
    BC2N_HIP(hipFree(base_));
    base_ = nullptr;
  }
  size_t cap = need + need / 4;
  BC2N_HIP(hipMalloc(reinterpret_cast<void**>(&base_), cap));
  cap_ = cap;
}

void* Arena::take(size_t bytes) {
  const size_t b = (bytes + 255) & ~size_t(255);
  if (off_ + b > cap_) throw std::runtime_error("arena: scratch plan exceeded");
  void* r = base_ + off_;
  off_ += b;
  return r;
}

namespace {
thread_local int t_lane = 0;
}  // namespace

int lane() { return t_lane; }
LaneGuard::LaneGuard(int l) : old(t_lane) {
  if (l < 0 || l >= NUM_LANES) throw std::runtime_error("lane out of range");
  t_lane = l;
}
LaneGuard::~LaneGuard() { t_lane = old; }

Arena& arena() {
  static Arena a[NUM_LANES];
  return a[t_lane];
}

namespace {
struct SideStream {
  std::mutex mu;
  hipStream_t st = nullptr;
  std::vector<hipEvent_t> ring;
  size_t next = 0;
  bool overlap = true;
};
SideStream& side() {
  static SideStream s;
  return s;
}
}  // namespace

hipStream_t side_stream() {
  SideStream& s = side();
  std::lock_guard<std::mutex> lk(s.mu);
  if (!s.st) hip_check(hipStreamCreateWithFlags(&s.st, hipStreamNonBlocking), "hipStreamCreate");
  return s.st;
}

void stream_wait(hipStream_t to, hipStream_t from) {
  SideStream& s = side();
  hipEvent_t e;
  {
    std::lock_guard<std::mutex> lk(s.mu);
    if (s.ring.size() < 16) {
      hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
      s.ring.push_back(e);
    }
    e = s.ring[s.next++ % s.ring.size()];
  }
  hip_check(hipEventRecord(e, from), "hipEventRecord");
  hip_check(hipStreamWaitEvent(to, e, 0), "hipStreamWaitEvent");
}

bool set_msa_overlap(bool on) {
  SideStream& s = side();
  std::lock_guard<std::mutex> lk(s.mu);
  const bool old = s.overlap;
  s.overlap = on;
  return old;
}
float* stack_pair_scratch(size_t bytes) {
  static std::mutex mu;
  static char* base = nullptr;
  static size_t cap = 0;
  std::lock_guard<std::mutex> lk(mu);
  if (bytes > cap) {
    if (base) {
      BC2N_HIP(hipDeviceSynchronize());
      BC2N_HIP(hipFree(base));
      base = nullptr;
      cap = 0;
    }
    BC2N_HIP(hipMalloc(reinterpret_cast<void**>(&base), bytes));
    cap = bytes;
  }
  return reinterpret_cast<float*>(base);
}

bool msa_overlap() {
  SideStream& s = side();
  std::lock_guard<std::mutex> lk(s.mu);
  return s.overlap;
}

int device_cus() {
  static int cus[64] = {};
  int dev = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  if (dev < 0 || dev >= 64) dev = 0;
  if (cus[dev] == 0) {
    int n = 0;
    hip_check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev),
              "hipDeviceGetAttribute");
    cus[dev] = n > 0 ? n : 1;
  }
  return cus[dev];
}

namespace {
struct KProf {
  bool on = false;
  std::string filter;  // empty: every launch
  std::mutex mu;
  std::vector<hipEvent_t> pool;
  size_t next = 0;
  std::vector<std::pair<std::string, std::pair<hipEvent_t, hipEvent_t>>> rec;
};
KProf& kp() {
  static KProf k;
  return k;
}
}  // namespace

void kprof_enable(bool on) { kp().on = on; }
bool kprof_on() { return kp().on; }
void kprof_filter(const char* name) {
  KProf& k = kp();
  std::lock_guard<std::mutex> lk(k.mu);
  k.filter = name ? name : "";
}
bool kprof_wants(const char* name) {
  KProf& k = kp();
  std::lock_guard<std::mutex> lk(k.mu);
  return k.filter.empty() || k.filter == name;
}

hipEvent_t kprof_event() {
  KProf& k = kp();
  std::lock_guard<std::mutex> lk(k.mu);
  if (k.next == k.pool.size()) {
    hipEvent_t e;
    hip_check(hipEventCreate(&e), "hipEventCreate");
    k.pool.push_back(e);
  }
  return k.pool[k.next++];
}

void kprof_record(const char* name, hipEvent_t a, hipEvent_t b) {
  KProf& k = kp();
  std::lock_guard<std::mutex> lk(k.mu);
  k.rec.push_back({name, {a, b}});
}

int kprof_read(char* names, int name_len, double* ms, int* counts, int cap) {
  KProf& k = kp();
  std::lock_guard<std::mutex> lk(k.mu);
  std::map<std::string, std::pair<double, int>> tot;
  std::vector<std::string> order;
  for (auto& r : k.rec) {
    hip_check(hipEventSynchronize(r.second.second), "hipEventSynchronize");
    float t = 0.f;
    hip_check(hipEventElapsedTime(&t, r.second.first, r.second.second), "hipEventElapsedTime");
    if (!tot.count(r.first)) order.push_back(r.first);
    tot[r.first].first += t;
    tot[r.first].second += 1;
  }
  k.rec.clear();
  k.next = 0;
  int n = 0;
  for (auto& nm : order) {
    if (n >= cap) break;
    snprintf(names + (size_t)n * name_len, (size_t)name_len, "%s", nm.c_str());
    ms[n] = tot[nm].first;
    counts[n] = tot[nm].second;
    ++n;
  }
  return n;
}

static thread_local std::string g_err;
void set_error(const std::string& msg) { g_err = msg; }
const char* last_error() { return g_err.c_str(); }

}  // namespace bc2n
