// GpuExecutor / GpuPackedWeights: the Provider contract over device-resident
// tensors, with the packed-weight matmul and the decoder-layer Kernels on
// the libmagnetar_gpu C ABI.
#include "executor.hpp"

#include <algorithm>
#include <cerrno>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

namespace magnetar {

namespace {

constexpr size_t kMaxObservations = 4096;  // bounded log (src/lib.rs:171-172)
// Replaced buffers wait for the stream to drain past them before they are
// freed; past this many bytes the executor drains and frees them at once.
constexpr uint64_t kRetiredBytesCap = 256ull << 20;

bool attribute_bool(const KernelInvocation& inv, const char* name, bool fallback) {
  auto it = inv.attributes.find(name);
  if (it == inv.attributes.end()) return fallback;
  return it->second == "true" || it->second == "1";
}

const std::string* attribute_text(const KernelInvocation& inv, const char* name) {
  auto it = inv.attributes.find(name);
  return it == inv.attributes.end() ? nullptr : &it->second;
}

// An integer attribute: nullopt when absent; `bad` set when present but not
// an integer. Negative values are returned as such (the caller decides).
std::optional<int64_t> attribute_integer(const KernelInvocation& inv, const char* name, bool* bad) {
  const std::string* t = attribute_text(inv, name);
  if (!t) return std::nullopt;
  char* end = nullptr;
  errno = 0;
  const long long v = std::strtoll(t->c_str(), &end, 10);
  if (end == t->c_str() || *end != '\0' || errno == ERANGE) {
    if (bad) *bad = true;
    return std::nullopt;
  }
  return static_cast<int64_t>(v);
}

std::optional<float> attribute_float(const KernelInvocation& inv, const char* name, bool* bad) {
  const std::string* t = attribute_text(inv, name);
  if (!t) return std::nullopt;
  char* end = nullptr;
  const float v = std::strtof(t->c_str(), &end);
  if (end == t->c_str() || *end != '\0') {
    if (bad) *bad = true;
    return std::nullopt;
  }
  return v;
}

std::string shape_text(const std::vector<uint64_t>& s) {
  std::string out = "[";
  for (size_t i = 0; i < s.size(); ++i) out += (i ? ", " : "") + std::to_string(s[i]);
  return out + "]";
}

uint64_t element_count(const std::vector<uint64_t>& shape) {
  uint64_t n = 1;
  for (uint64_t d : shape) n *= d;
  return n;
}

bool rows_cols(const std::vector<uint64_t>& shape, uint64_t& rows, uint64_t& cols) {
  if (shape.size() != 2) return false;
  rows = shape[0];
  cols = shape[1];
  return true;
}

KernelError rank2_error(const char* what, const std::vector<uint64_t>& shape) {
  return KernelError::failed(std::string(what) + " expects a rank-2 tensor, got shape " + shape_text(shape));
}

}  // namespace

// ---- value types -------------------------------------------------------------

bool HostTensor::rows_cols(uint64_t& rows, uint64_t& cols) const {
  if (shape.size() != 2) return false;
  rows = shape[0];
  cols = shape[1];
  return rows * cols == data.size();
}

std::vector<uint64_t> PackedWeight::logical_shape() const {
  return transposed ? std::vector<uint64_t>{stored_cols, stored_rows} : std::vector<uint64_t>{stored_rows, stored_cols};
}

std::vector<uint64_t> GpuPackedWeights::Entry::logical_shape() const {
  return transposed ? std::vector<uint64_t>{cols, rows} : std::vector<uint64_t>{rows, cols};
}

// `baseline_advertisement` for every Kernel this Provider runs, under its
// identity (src/lib.rs:1350-1373, src/native/mod.rs:847-864): f32 in/out,
// contiguous, Host memory class, TimeoutOnly; matmul at rank 2.
std::vector<KernelAdvertisement> gpu_kernel_advertisements() {
  static const char* const kNames[][2] = {
      {"matmul", "GpuMatrix"},       {"matmul-bias", "GpuMatrix"},     {"matmul-residual", "GpuMatrix"},
      {"embedding", "GpuGather"},    {"rmsnorm", "GpuNormalization"}, {"rope", "GpuPosition"},
      {"kv-write", "GpuKvHistory"},  {"attention", "GpuAttention"},   {"silu-mul", "GpuElementwise"},
      {"add", "GpuElementwise"},     {"residual-add", "GpuElementwise"},
  };
  std::vector<KernelAdvertisement> out;
  for (const auto& nf : kNames) {
    KernelAdvertisement a;
    a.provider = kGpuProviderName;
    a.name = nf[0];
    a.version = "1.0.0";
    a.operator_id = std::string("magnetar:") + nf[0] + "@1";
    a.family = nf[1];
    a.conformance_profile = kConformanceProfile;
    a.input_dtypes = {"f32"};
    a.output_dtypes = {"f32"};
    a.layouts = {"Contiguous"};
    a.memory_classes = {"Host"};
    a.devices = {kGpuDeviceId};
    a.cancellation = "TimeoutOnly";
    if (a.name == "matmul") a.rank = 2;
    out.push_back(a);
  }
  return out;
}

bool MemoryLedger::admit(const std::string& id, uint64_t bytes) {
  uint64_t previous = 0;
  auto it = allocations_.find(id);
  if (it != allocations_.end()) previous = it->second;
  if (used_ - previous + bytes > capacity_) return false;
  used_ = used_ - previous + bytes;
  allocations_[id] = bytes;
  return true;
}

void MemoryLedger::release(const std::string& id) {
  auto it = allocations_.find(id);
  if (it == allocations_.end()) return;
  used_ -= it->second;
  allocations_.erase(it);
}

uint64_t MemoryLedger::bytes_of(const std::string& id) const {
  auto it = allocations_.find(id);
  return it == allocations_.end() ? 0 : it->second;
}

// ---- GpuPackedWeights ---------------------------------------------------------

GpuPackedWeights::~GpuPackedWeights() {
  std::lock_guard<std::mutex> lock(mu_);
  for (auto& kv : packed_) mq_weight_release(ctx_, kv.second.handle);
}

std::optional<GpuPackedWeights::Entry> GpuPackedWeights::find(const std::string& id) {
  std::lock_guard<std::mutex> lock(mu_);
  auto it = packed_.find(id);
  if (it == packed_.end()) return std::nullopt;
  return it->second;
}

PackedWeightWrite GpuPackedWeights::store(const std::string& id, const PackedWeight& w, std::string* why,
                                          const std::function<bool(uint64_t)>& admit) {
  uint64_t handle = 0;
  int rc = mq_weight_upload(ctx_, w.format, w.stored_rows, w.stored_cols, w.transposed ? 1 : 0, w.bytes.data(),
                            w.bytes.size(), &handle);
  if (rc != MQ_OK) {
    if (why) *why = mq_last_error(ctx_);
    return PackedWeightWrite::Declined;
  }
  if (admit) {
    uint32_t type = 0;
    uint64_t rows = 0, cols = 0, bytes = 0;
    int tr = 0;
    if (mq_weight_info(ctx_, handle, &type, &rows, &cols, &tr, &bytes) != MQ_OK || !admit(bytes)) {
      mq_weight_release(ctx_, handle);
      if (why) *why = "memory admission denied for the packed weight's " + std::to_string(bytes) + " device bytes";
      return PackedWeightWrite::Declined;
    }
  }
  std::lock_guard<std::mutex> lock(mu_);
  auto it = packed_.find(id);
  if (it != packed_.end()) mq_weight_release(ctx_, it->second.handle);
  packed_[id] = Entry{handle, w.format, w.stored_rows, w.stored_cols, w.transposed};
  return PackedWeightWrite::Stored;
}

bool GpuPackedWeights::forget(const std::string& id) {
  std::lock_guard<std::mutex> lock(mu_);
  auto it = packed_.find(id);
  if (it == packed_.end()) return false;
  mq_weight_release(ctx_, it->second.handle);
  packed_.erase(it);
  return true;
}

std::optional<std::vector<uint64_t>> GpuPackedWeights::shape(const std::string& id) {
  auto e = find(id);
  if (!e) return std::nullopt;
  return e->logical_shape();
}

// `materialize` -> `NativeState::expand` -> `PackedWeight::dequantize`: the
// logical values, counted (src/native/mod.rs:196-204, 455-457).
std::optional<HostTensor> GpuPackedWeights::materialize(const std::string& id) {
  auto e = find(id);
  if (!e) return std::nullopt;
  HostTensor t;
  t.shape = e->logical_shape();
  t.data.resize(e->rows * e->cols);
  if (mq_dequantize(ctx_, e->handle, e->transposed ? 1 : 0, t.data.data()) != MQ_OK) return std::nullopt;
  materialized_++;
  return t;
}

bool GpuPackedWeights::materialize_dev(const Entry& e, float* out) {
  if (mq_dequantize_dev(ctx_, e.handle, e.transposed ? 1 : 0, out, mq_context_stream(ctx_)) != MQ_OK) return false;
  materialized_++;
  return true;
}

// ---- GpuExecutor: construction, observations ------------------------------------

struct GpuExecutor::Output {
  std::string id;
  DeviceTensor tensor;
  bool fresh = false;               // a new buffer (the old one is retired on commit)
  uint64_t previous_admitted = 0;   // the ledger's bytes for id before admission
  bool previously_admitted = false;
};

GpuExecutor::GpuExecutor(int device, bool packed_weights, bool int8_activations, uint64_t memory_capacity)
    : packed_weights_(packed_weights), int8_(int8_activations), memory_(memory_capacity) {
  if (mq_create(device, &ctx_) != MQ_OK) {
    init_error_ = mq_last_error(nullptr);
    ctx_ = nullptr;
    return;
  }
  stream_ = mq_context_stream(ctx_);
  packed_ = std::make_unique<GpuPackedWeights>(ctx_);
  const char* p = std::getenv("MAGNETAR_GPU_PROFILE");
  profile_on_ = p && std::strcmp(p, "1") == 0;
  observe({"ProviderRegistered", "", "", kGpuProviderName});
  observe({"DeviceDetected", "", "", kGpuDeviceId});
}

GpuExecutor::~GpuExecutor() {
  if (profile_on_) {
    // the reference prints its profile when the executor drops
    // (src/native/mod.rs:472-497)
    std::fprintf(stderr, "[gpu profile] packed weights expanded to f32: %llu\n",
                 static_cast<unsigned long long>(materializations()));
    for (const auto& row : profile())
      std::fprintf(stderr, "[gpu profile] %s: %llu calls, %.3f ms total, %.4f ms each\n", row.first.c_str(),
                   static_cast<unsigned long long>(row.second.first), row.second.second * 1e3,
                   row.second.second * 1e3 / static_cast<double>(row.second.first));
  }
  if (!ctx_) return;
  mq_synchronize(ctx_, stream_);
  packed_.reset();
  for (auto& kv : storage_) mq_device_free(ctx_, kv.second.dev);
  for (float* p : retired_) mq_device_free(ctx_, p);
  mq_device_free(ctx_, scratch_);
  mq_destroy(ctx_);
}

void GpuExecutor::observe(KernelObservation o) const {
  std::lock_guard<std::mutex> lock(obs_mu_);
  if (observations_.size() >= kMaxObservations) observations_.erase(observations_.begin());
  observations_.push_back(std::move(o));
}

std::vector<KernelObservation> GpuExecutor::observations() const {
  std::lock_guard<std::mutex> lock(obs_mu_);
  return observations_;
}

uint64_t GpuExecutor::memory_used() const {
  std::lock_guard<std::mutex> lock(mu_);
  return memory_.used();
}

uint64_t GpuExecutor::memory_capacity() const {
  std::lock_guard<std::mutex> lock(mu_);
  return memory_.capacity();
}

std::vector<std::pair<std::string, std::pair<uint64_t, double>>> GpuExecutor::profile() const {
  std::lock_guard<std::mutex> lock(mu_);
  std::vector<std::pair<std::string, std::pair<uint64_t, double>>> rows(profile_.begin(), profile_.end());
  std::sort(rows.begin(), rows.end(), [](const auto& a, const auto& b) { return a.second.second > b.second.second; });
  return rows;
}

KernelError GpuExecutor::device_error(const char* what) const {
  return KernelError::failed(std::string(what) + ": " + mq_last_error(ctx_));
}

// ---- storage helpers ------------------------------------------------------------

void GpuExecutor::retire(float* dev, uint64_t bytes) {
  if (!dev) return;
  retired_.push_back(dev);
  retired_bytes_ += bytes;
}

void GpuExecutor::drain_retired() {
  if (retired_.empty()) return;
  mq_synchronize(ctx_, stream_);
  for (float* p : retired_) mq_device_free(ctx_, p);
  retired_.clear();
  retired_bytes_ = 0;
}

// Scratch of at least `count` floats for a Kernel-internal temporary,
// ordered on the stream: a larger one replaces it once queued work is done.
float* GpuExecutor::scratch(uint64_t count, std::string* why) {
  if (count <= scratch_count_) return scratch_;
  if (scratch_) {
    mq_synchronize(ctx_, stream_);
    mq_device_free(ctx_, scratch_);
    scratch_ = nullptr;
    scratch_count_ = 0;
  }
  void* p = nullptr;
  if (mq_device_alloc(ctx_, count * sizeof(float), &p) != MQ_OK) {
    if (why) *why = mq_last_error(ctx_);
    return nullptr;
  }
  scratch_ = static_cast<float*>(p);
  scratch_count_ = count;
  return scratch_;
}

// Copies a host tensor into `id`'s device buffer (reused when large
// enough; a replaced buffer is retired, since queued Kernels may read it).
bool GpuExecutor::store_host(const std::string& id, const HostTensor& t, std::string* why) {
  const uint64_t count = element_count(t.shape);
  if (count != t.data.size()) {
    if (why) *why = "tensor data length " + std::to_string(t.data.size()) + " does not match shape " +
                    shape_text(t.shape);
    return false;
  }
  const uint64_t bytes = count * sizeof(float);
  auto it = storage_.find(id);
  DeviceTensor d;
  bool reuse = it != storage_.end() && it->second.capacity >= bytes && bytes > 0;
  if (reuse) {
    d = it->second;
  } else if (bytes) {
    void* p = nullptr;
    if (mq_device_alloc(ctx_, bytes, &p) != MQ_OK) {
      if (why) *why = mq_last_error(ctx_);
      return false;
    }
    d.dev = static_cast<float*>(p);
    d.capacity = bytes;
  }
  // the copy is ordered after every Kernel already queued on the stream, so
  // a reused buffer is not overwritten under a reader
  if (bytes && mq_copy_to_device(ctx_, d.dev, t.data.data(), bytes) != MQ_OK) {
    if (why) *why = mq_last_error(ctx_);
    if (!reuse) mq_device_free(ctx_, d.dev);
    return false;
  }
  d.shape = t.shape;
  d.count = count;
  if (it != storage_.end() && !reuse) {
    retire(it->second.dev, it->second.capacity);
  }
  storage_[id] = d;
  if (retired_bytes_ > kRetiredBytesCap) drain_retired();
  return true;
}

Result<const DeviceTensor*> GpuExecutor::input(const KernelInvocation& inv, size_t index) {
  using R = Result<const DeviceTensor*>;
  if (index >= inv.inputs.size()) return R::failure(KernelError::failed("missing input at index " + std::to_string(index)));
  auto it = storage_.find(inv.inputs[index]);
  if (it == storage_.end())
    return R::failure(KernelError::failed("no materialized data for input resource " + inv.inputs[index]));
  return R::success(&it->second);
}

// Admits the output's bytes before anything is dispatched (the reference's
// `execute_invocation_with_memory_manager`, src/lib.rs:2132-2230) and picks
// its buffer: the id's own when large enough and not also an input of the
// invocation (a Kernel never writes a buffer it reads, except kv-write's
// in-place store), else a new one.
Result<GpuExecutor::Output> GpuExecutor::begin_output(const KernelInvocation& inv, const std::vector<uint64_t>& shape) {
  using R = Result<Output>;
  Output o;
  o.id = inv.outputs[0];
  o.tensor.shape = shape;
  o.tensor.count = element_count(shape);
  const uint64_t bytes = o.tensor.count * sizeof(float);
  o.previously_admitted = memory_.holds(o.id);
  o.previous_admitted = memory_.bytes_of(o.id);
  if (!memory_.admit(o.id, bytes)) {
    observe({"KernelMemoryFeasibilityFailed", inv.kernel, inv.id, o.id});
    return R::failure(KernelError::failed("memory admission denied for output " + o.id + ": " +
                                          std::to_string(bytes) + " bytes"));
  }
  const bool aliased = std::find(inv.inputs.begin(), inv.inputs.end(), o.id) != inv.inputs.end();
  auto it = storage_.find(o.id);
  if (it != storage_.end() && !aliased && it->second.capacity >= bytes) {
    o.tensor.dev = it->second.dev;
    o.tensor.capacity = it->second.capacity;
    return R::success(o);
  }
  if (bytes) {
    void* p = nullptr;
    if (mq_device_alloc(ctx_, bytes, &p) != MQ_OK) {
      abort_output(o);
      return R::failure(device_error("output allocation"));
    }
    o.tensor.dev = static_cast<float*>(p);
    o.tensor.capacity = bytes;
  }
  o.fresh = true;
  return R::success(o);
}

void GpuExecutor::commit_output(Output& o) {
  auto it = storage_.find(o.id);
  if (it != storage_.end() && o.fresh && it->second.dev != o.tensor.dev) {
    retire(it->second.dev, it->second.capacity);
  }
  storage_[o.id] = o.tensor;
  if (packed_) packed_->forget(o.id);  // the output replaces a packed weight of that id
  if (retired_bytes_ > kRetiredBytesCap) drain_retired();
}

void GpuExecutor::abort_output(Output& o) {
  if (o.previously_admitted)
    memory_.admit(o.id, o.previous_admitted);
  else
    memory_.release(o.id);
  if (o.fresh && o.tensor.dev) {
    retire(o.tensor.dev, o.tensor.capacity);
    o.tensor.dev = nullptr;
  }
}

// ---- ProviderExecutionApi storage ----------------------------------------------------

// `write_packed_weight_tensor` (src/native/mod.rs:638-653).
PackedWeightWrite GpuExecutor::write_packed_weight_tensor(const std::string& id, const PackedWeight& w,
                                                          std::string* why) {
  if (!packed_weights_ || !packed_) {
    if (why) *why = "packed weights are disabled";
    return PackedWeightWrite::Declined;
  }
  // the device bytes are admitted to the ledger before the upload replaces
  // a weight of the same id
  PackedWeightWrite r = packed_->store(id, w, why, [&](uint64_t bytes) {
    std::lock_guard<std::mutex> lock(mu_);
    return memory_.admit(id, bytes);
  });
  if (r == PackedWeightWrite::Stored) {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = storage_.find(id);
    if (it != storage_.end()) {
      retire(it->second.dev, it->second.capacity);
      storage_.erase(it);
    }
  }
  return r;
}

// `write_tensor`: an f32 write forgets a packed weight of the same id
// (src/native/mod.rs:629-636).
bool GpuExecutor::write_tensor(const std::string& id, const HostTensor& tensor, std::string* why) {
  std::lock_guard<std::mutex> lock(mu_);
  if (!store_host(id, tensor, why)) return false;
  if (packed_ && packed_->forget(id)) memory_.release(id);  // the device bytes it held
  return true;
}

// `write_tensor_admitted` (src/native/mod.rs:664-681, src/lib.rs:1711-1735):
// the packed weight is replaced only once its replacement is admitted.
bool GpuExecutor::write_tensor_admitted(const std::string& id, const HostTensor& tensor, bool* denied,
                                        std::string* why) {
  if (denied) *denied = false;
  std::lock_guard<std::mutex> lock(mu_);
  const bool had = memory_.holds(id);
  const uint64_t previous = memory_.bytes_of(id);
  if (!memory_.admit(id, tensor.data.size() * sizeof(float))) {
    if (denied) *denied = true;
    if (why)
      *why = "memory admission denied for " + id + ": " + std::to_string(tensor.data.size() * sizeof(float)) +
             " bytes, " + std::to_string(memory_.capacity() - memory_.used()) + " available";
    return false;
  }
  if (!store_host(id, tensor, why)) {
    if (had)
      memory_.admit(id, previous);
    else
      memory_.release(id);
    return false;
  }
  if (packed_) packed_->forget(id);
  return true;
}

// `read_tensor`: device values copied out after the queued Kernels, or the
// packed weight's materialization (src/lib.rs:1615-1620).
std::optional<HostTensor> GpuExecutor::read_tensor(const std::string& id) {
  {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = storage_.find(id);
    if (it != storage_.end()) {
      HostTensor t;
      t.shape = it->second.shape;
      t.data.resize(it->second.count);
      if (mq_copy_to_host(ctx_, t.data.data(), it->second.dev, it->second.count * sizeof(float)) != MQ_OK)
        return std::nullopt;
      return t;
    }
  }
  if (!packed_) return std::nullopt;
  std::lock_guard<std::mutex> lock(mu_);
  return packed_->materialize(id);
}

std::optional<std::vector<uint64_t>> GpuExecutor::resident_shape(const std::string& id) {
  {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = storage_.find(id);
    if (it != storage_.end()) return it->second.shape;
  }
  if (!packed_) return std::nullopt;
  return packed_->shape(id);
}

bool GpuExecutor::release_tensor(const std::string& id) {
  const bool packed = packed_ && packed_->forget(id);
  std::lock_guard<std::mutex> lock(mu_);
  if (packed) memory_.release(id);  // the packed weight's device bytes
  auto it = storage_.find(id);
  if (it == storage_.end()) return packed;
  retire(it->second.dev, it->second.capacity);
  storage_.erase(it);
  if (retired_bytes_ > kRetiredBytesCap) drain_retired();
  return true;
}

// `release_admitted_tensor` (src/lib.rs:1699-1711, src/native/mod.rs:662-670).
bool GpuExecutor::release_admitted_tensor(const std::string& id) {
  const bool r = release_tensor(id);
  std::lock_guard<std::mutex> lock(mu_);
  memory_.release(id);
  return r;
}

bool GpuExecutor::is_packed(const std::string& id) { return packed_ && packed_->contains(id); }

bool GpuExecutor::read_tensor_value_is_opaque(const std::string& id) {
  if (is_packed(id)) return true;
  std::lock_guard<std::mutex> lock(mu_);
  return storage_.count(id) > 0;
}

// `write_tensor_value` (src/native/mod.rs:708-721, src/lib.rs:1811-1830):
// writing back an Opaque value stores nothing, so a packed weight stays.
bool GpuExecutor::write_tensor_value(const std::string& id, const HostTensor* host, std::string* why) {
  if (!host) return true;
  return write_tensor(id, *host, why);
}

bool GpuExecutor::write_tensor_value_admitted(const std::string& id, const HostTensor* host, bool* denied,
                                              std::string* why) {
  if (denied) *denied = false;
  if (!host) return true;
  return write_tensor_admitted(id, *host, denied, why);
}

// `copy_tensor_admitted` (src/native/mod.rs:746-766, src/lib.rs:1760-1809):
// the source's values (a packed weight's logical values) under `to`,
// admitted first; the copy replaces whatever `to` held.
bool GpuExecutor::copy_tensor_admitted(const std::string& from, const std::string& to, bool* denied,
                                       std::string* why) {
  if (denied) *denied = false;
  std::optional<GpuPackedWeights::Entry> packed_from = packed_ ? packed_->find(from) : std::nullopt;
  std::lock_guard<std::mutex> lock(mu_);
  auto src = storage_.find(from);
  if (src == storage_.end() && !packed_from) {
    if (denied) *denied = true;
    if (why) *why = "copy_tensor_admitted: source resource '" + from + "' not found";
    return false;
  }
  const std::vector<uint64_t> shape = src != storage_.end() ? src->second.shape : packed_from->logical_shape();
  const uint64_t count = element_count(shape), bytes = count * sizeof(float);
  const bool had = memory_.holds(to);
  const uint64_t previous = memory_.bytes_of(to);
  if (!memory_.admit(to, bytes)) {
    if (denied) *denied = true;
    if (why) *why = "memory admission denied for " + to + ": " + std::to_string(bytes) + " bytes";
    return false;
  }
  DeviceTensor d;
  d.shape = shape;
  d.count = count;
  if (from == to && src != storage_.end()) return true;  // a tensor copied onto itself
  if (bytes) {
    void* p = nullptr;
    if (mq_device_alloc(ctx_, bytes, &p) != MQ_OK) {
      if (had)
        memory_.admit(to, previous);
      else
        memory_.release(to);
      if (why) *why = mq_last_error(ctx_);
      return false;
    }
    d.dev = static_cast<float*>(p);
    d.capacity = bytes;
    const bool ok = src != storage_.end()
                        ? mq_copy_dev(ctx_, d.dev, src->second.dev, bytes, stream_) == MQ_OK
                        : packed_->materialize_dev(*packed_from, d.dev);
    if (!ok) {
      if (why) *why = mq_last_error(ctx_);
      retire(d.dev, bytes);
      if (had)
        memory_.admit(to, previous);
      else
        memory_.release(to);
      return false;
    }
  }
  auto it = storage_.find(to);
  if (it != storage_.end()) {
    retire(it->second.dev, it->second.capacity);
  }
  storage_[to] = d;
  if (packed_) packed_->forget(to);
  if (retired_bytes_ > kRetiredBytesCap) drain_retired();
  return true;
}

// `write_zeroed_kv_store(_with_exact_head)` (src/lib.rs:1633-1690,
// src/native/mod.rs:767-799): the store replaces whatever `id` held.
bool GpuExecutor::write_zeroed_kv_store(const std::string& id, const std::vector<uint64_t>& shape,
                                        KvStorePrecision precision, uint64_t head_dimension, uint64_t exact_rows,
                                        std::string* why) {
  (void)exact_rows;  // only the TurboQuant precisions keep an exact head
  if (shape.size() != 2 || head_dimension == 0 || shape[1] % head_dimension) {
    if (why) *why = "a KV store is [capacity, whole heads]";
    return false;
  }
  if (precision != KvStorePrecision::F32) {
    if (why) *why = "TurboQuant KV stores have no GPU path";
    return false;
  }
  if (packed_ && packed_->forget(id)) {
    std::lock_guard<std::mutex> lock(mu_);
    memory_.release(id);
  }
  std::lock_guard<std::mutex> lock(mu_);
  const uint64_t count = shape[0] * shape[1], bytes = count * sizeof(float);
  DeviceTensor d;
  d.shape = shape;
  d.count = count;
  auto it = storage_.find(id);
  const bool reuse = it != storage_.end() && it->second.capacity >= bytes;
  if (reuse) {
    d.dev = it->second.dev;
    d.capacity = it->second.capacity;
  } else if (bytes) {
    void* p = nullptr;
    if (mq_device_alloc(ctx_, bytes, &p) != MQ_OK) {
      if (why) *why = mq_last_error(ctx_);
      return false;
    }
    d.dev = static_cast<float*>(p);
    d.capacity = bytes;
  }
  if (bytes && mq_fill_dev(ctx_, d.dev, count, 0.0f, stream_) != MQ_OK) {
    if (why) *why = mq_last_error(ctx_);
    if (!reuse) mq_device_free(ctx_, d.dev);
    return false;
  }
  if (it != storage_.end() && !reuse) {
    retire(it->second.dev, it->second.capacity);
  }
  storage_[id] = d;
  return true;
}

// `allocate_workspace` (src/lib.rs:2100-2121): scratch admitted through the
// ledger as a TemporaryWorkspace allocation, released by its id.
std::optional<std::string> GpuExecutor::allocate_workspace(uint64_t bytes) {
  std::lock_guard<std::mutex> lock(mu_);
  const std::string allocation = "workspace:" + std::to_string(workspace_ordinal_++);
  if (!memory_.admit(allocation, bytes)) return std::nullopt;
  return allocation;
}

bool GpuExecutor::release_workspace(const std::string& allocation) {
  std::lock_guard<std::mutex> lock(mu_);
  if (allocation.rfind("workspace:", 0) != 0 || !memory_.holds(allocation)) return false;
  memory_.release(allocation);
  return true;
}

bool GpuExecutor::synchronize() {
  std::lock_guard<std::mutex> lock(mu_);
  if (mq_synchronize(ctx_, stream_) != MQ_OK) return false;
  drain_retired();
  return true;
}

// ---- Kernel arms ----------------------------------------------------------------------

// `NativeState::matmul` (src/native/mod.rs:206-236) with `packed_matmul`
// (110-152) and `packed_axpy` (154-194): shape checks, f32-only
// accumulation, routing, and the bias / residual epilogue (`add` /
// `residual_add`, src/lib.rs:1019-1075, 1128-1133) fused into the kernel's
// output write where the shapes allow.
Result<bool> GpuExecutor::run_matmul(const KernelInvocation& inv, const GpuPackedWeights::Entry& w) {
  using R = Result<bool>;
  auto a_in = input(inv, 0);
  if (!a_in.ok()) return R::failure(a_in.error);
  const DeviceTensor& a = **a_in.value;
  const bool transpose_a = attribute_bool(inv, "transpose_a", false);
  const bool transpose_b = attribute_bool(inv, "transpose_b", false);
  const std::string* acc = attribute_text(inv, "accumulation_dtype");
  if (acc && *acc != "f32" && *acc != "float32" && *acc != "Float32")
    return R::failure({KernelErrorKind::DTypeUnsupported,
                       "the GPU packed matmul only accumulates in f32; requested " + *acc});
  uint64_t m = 0, k = 0;
  if (!rows_cols(a.shape, m, k)) return R::failure(rank2_error("matmul", a.shape));
  uint32_t flags = (int8_ ? MQ_INT8_ACTIVATIONS : 0) | (transpose_b ? MQ_TRANSPOSE_B : 0);
  const float* x = a.dev;
  std::string why;
  if (transpose_a) {
    // The reference expands the weight and runs the dense f32 matmul, the
    // activation read transposed: here the activation is transposed on the
    // host (a rare path) and multiplied with f32 activations.
    std::vector<float> h(a.count), t(a.count);
    if (mq_copy_to_host(ctx_, h.data(), a.dev, a.count * sizeof(float)) != MQ_OK)
      return R::failure(device_error("transpose_a"));
    for (uint64_t r = 0; r < m; ++r)
      for (uint64_t c = 0; c < k; ++c) t[c * m + r] = h[r * k + c];
    std::swap(m, k);
    float* s = scratch(a.count, &why);
    if (!s) return R::failure(KernelError::failed(why));
    if (mq_copy_to_device(ctx_, s, t.data(), a.count * sizeof(float)) != MQ_OK)
      return R::failure(device_error("transpose_a"));
    x = s;
    flags &= ~MQ_INT8_ACTIVATIONS;
  }
  // the reference's orientation rule (src/native/mod.rs:217-227)
  const bool output_major = w.transposed != transpose_b;
  if (!output_major) flags &= ~MQ_INT8_ACTIVATIONS;
  if (output_major && (k != w.cols || k % 32 != 0))
    return R::failure(KernelError::failed("packed matmul: activations have " + std::to_string(k) +
                                          " columns, the weight's stored rows " + std::to_string(w.cols)));
  if (!output_major && k != w.rows)
    return R::failure(KernelError::failed("packed matmul: activations have " + std::to_string(k) +
                                          " columns, the weight " + std::to_string(w.rows) + " stored rows"));
  const uint64_t n = output_major ? w.rows : w.cols;
  const std::vector<uint64_t> product_shape{m, n};

  if (inv.kernel == "matmul") {
    auto out = begin_output(inv, product_shape);
    if (!out.ok()) return R::failure(out.error);
    if (mq_matmul_dev(ctx_, w.handle, x, m, k, flags, out.value->tensor.dev, stream_) != MQ_OK) {
      abort_output(*out.value);
      return R::failure(KernelError::failed(mq_last_error(ctx_)));
    }
    commit_output(*out.value);
    return R::success(true);
  }
  auto e_in = input(inv, 2);
  if (!e_in.ok()) return R::failure(e_in.error);
  const DeviceTensor& e = **e_in.value;
  const std::vector<uint64_t> row1{n}, row2{1, n};
  if (inv.kernel == "matmul-bias") {
    // add(product, bias): bias of the product's shape, or one row broadcast
    const bool same = e.shape == product_shape;
    if (!same && e.shape != row1 && e.shape != row2)
      return R::failure(KernelError::failed("add expects b to match a's shape " + shape_text(product_shape) +
                                            " or broadcast as [" + std::to_string(n) + "]/[1, " +
                                            std::to_string(n) + "], got " + shape_text(e.shape)));
    auto out = begin_output(inv, product_shape);
    if (!out.ok()) return R::failure(out.error);
    if (mq_matmul_add_dev(ctx_, w.handle, x, m, k, flags, e.dev, same ? m : 1, out.value->tensor.dev, stream_) !=
        MQ_OK) {
      abort_output(*out.value);
      return R::failure(KernelError::failed(mq_last_error(ctx_)));
    }
    commit_output(*out.value);
    return R::success(true);
  }
  // matmul-residual: residual_add(residual, product) = add(residual, product):
  // the residual's shape; the product adds element-wise when the shapes
  // match, or as one broadcast row when it is [1, n]
  if (e.shape == product_shape) {
    auto out = begin_output(inv, e.shape);
    if (!out.ok()) return R::failure(out.error);
    if (mq_matmul_add_dev(ctx_, w.handle, x, m, k, flags, e.dev, m, out.value->tensor.dev, stream_) != MQ_OK) {
      abort_output(*out.value);
      return R::failure(KernelError::failed(mq_last_error(ctx_)));
    }
    commit_output(*out.value);
    return R::success(true);
  }
  if (e.shape.empty() || e.shape.back() != n || m != 1 || e.count % n != 0)
    return R::failure(KernelError::failed("add expects b to match a's shape " + shape_text(e.shape) +
                                          " or broadcast as [" + std::to_string(e.shape.empty() ? 0 : e.shape.back()) +
                                          "]/[1, " + std::to_string(e.shape.empty() ? 0 : e.shape.back()) +
                                          "], got " + shape_text(product_shape)));
  auto out = begin_output(inv, e.shape);
  if (!out.ok()) return R::failure(out.error);
  float* prod = scratch(transpose_a ? m * k + n : n, &why);
  if (!prod) {
    abort_output(*out.value);
    return R::failure(KernelError::failed(why));
  }
  if (transpose_a) prod += m * k;  // past the transposed activation
  if (mq_matmul_dev(ctx_, w.handle, x, m, k, flags, prod, stream_) != MQ_OK ||
      mq_add_dev(ctx_, e.dev, e.count, prod, n, out.value->tensor.dev, stream_) != MQ_OK) {
    abort_output(*out.value);
    return R::failure(KernelError::failed(mq_last_error(ctx_)));
  }
  commit_output(*out.value);
  return R::success(true);
}

// `NativeState::embedding` (src/native/mod.rs:389-417) and the `scale`
// attribute (432-449): the token rows of a packed table, ids validated on
// the host with the reference's text and gathered on the GPU.
Result<bool> GpuExecutor::run_embedding(const KernelInvocation& inv, const GpuPackedWeights::Entry& table) {
  using R = Result<bool>;
  auto ids_in = input(inv, 1);
  if (!ids_in.ok()) return R::failure(ids_in.error);
  const DeviceTensor& ids = **ids_in.value;
  float scale = std::nanf("");
  bool bad = false;
  if (auto s = attribute_float(inv, "scale", &bad)) scale = *s;
  if (bad) return R::failure(KernelError::attribute("embedding scale " + *attribute_text(inv, "scale") +
                                                    " is not a number"));
  std::vector<float> host(ids.count);
  if (ids.count && mq_copy_to_host(ctx_, host.data(), ids.dev, ids.count * sizeof(float)) != MQ_OK)
    return R::failure(device_error("embedding ids"));
  const uint64_t dim = table.transposed ? table.rows : table.cols;
  auto out = begin_output(inv, {ids.count, dim});
  if (!out.ok()) return R::failure(out.error);
  if (mq_embedding_dev(ctx_, table.handle, host.data(), ids.count, scale, out.value->tensor.dev, stream_) != MQ_OK) {
    abort_output(*out.value);
    return R::failure(KernelError::failed(mq_last_error(ctx_)));
  }
  commit_output(*out.value);
  return R::success(true);
}

// The `rmsnorm` Kernel (src/lib.rs:2679-2726) in its weighted form over
// `rmsnorm` (src/lib.rs:348-402): the weight one row ([cols] / [1, cols])
// or one per row (the input's shape / [rows, cols]). The head-block and
// weightless forms go through the external operator-semantics crate in the
// reference (`rmsnorm_blocks`), whose arithmetic is not in its tree: they
// have no GPU path and are refused as unsupported attributes.
Result<bool> GpuExecutor::run_rmsnorm(const KernelInvocation& inv) {
  using R = Result<bool>;
  auto x_in = input(inv, 0);
  if (!x_in.ok()) return R::failure(x_in.error);
  const DeviceTensor& x = **x_in.value;
  bool bad = false;
  const float eps = attribute_float(inv, "epsilon", &bad).value_or(1e-6f);
  if (bad) return R::failure(KernelError::attribute("rmsnorm epsilon must be a number"));
  const bool heads = attribute_text(inv, "head_count") || attribute_text(inv, "head_dimension");
  if (const std::string* ws = attribute_text(inv, "with_scale")) {
    const bool with_scale = *ws == "true" || *ws == "1";
    if (with_scale != (inv.inputs.size() > 1))
      return R::failure(KernelError::attribute("rmsnorm with_scale " + std::string(with_scale ? "true" : "false") +
                                               " contradicts its " + std::to_string(inv.inputs.size()) +
                                               " input(s)"));
  }
  if (heads || inv.inputs.size() < 2)
    return R::failure(KernelError::attribute("rmsnorm head blocks and the weightless form have no GPU path"));
  auto w_in = input(inv, 1);
  if (!w_in.ok()) return R::failure(w_in.error);
  const DeviceTensor& w = **w_in.value;
  if (x.shape.empty()) return R::failure(KernelError::failed("RMSNorm expects at least one dimension"));
  const uint64_t cols = x.shape.back();
  if (cols == 0) return R::failure(KernelError::failed("RMSNorm hidden dimension must be non-zero"));
  if (x.count % cols)
    return R::failure(KernelError::failed("RMSNorm data length " + std::to_string(x.count) +
                                          " is not divisible by hidden dimension " + std::to_string(cols)));
  const uint64_t rows = x.count / cols;
  const std::vector<uint64_t> one{cols}, one2{1, cols}, per{rows, cols};
  uint64_t w_rows = 1;
  if (w.shape == one || w.shape == one2) {
    w_rows = 1;
  } else if (w.shape == x.shape || w.shape == per) {
    w_rows = rows;
  } else {
    return R::failure(KernelError::failed("RMSNorm weight shape must be [" + std::to_string(cols) + "], [1, " +
                                          std::to_string(cols) + "], input shape " + shape_text(x.shape) + ", or [" +
                                          std::to_string(rows) + ", " + std::to_string(cols) + "], got " +
                                          shape_text(w.shape)));
  }
  auto out = begin_output(inv, x.shape);
  if (!out.ok()) return R::failure(out.error);
  if (mq_rmsnorm_dev(ctx_, x.dev, rows, cols, w.dev, w_rows, eps, out.value->tensor.dev, stream_) != MQ_OK) {
    abort_output(*out.value);
    return R::failure(KernelError::failed(mq_last_error(ctx_)));
  }
  commit_output(*out.value);
  return R::success(true);
}

// The `rope` Kernel (src/lib.rs:2728-2817): sequential positions from
// position_offset, head_count blocks, interleaved or half_split pairing.
// The frequency-scaling attributes (YaRN, banded) and a partial rotary
// factor have no GPU path and are refused by name.
Result<bool> GpuExecutor::run_rope(const KernelInvocation& inv) {
  using R = Result<bool>;
  auto x_in = input(inv, 0);
  if (!x_in.ok()) return R::failure(x_in.error);
  const DeviceTensor& x = **x_in.value;
  static const char* const kKnown[] = {"base", "scale", "dimension", "position_offset", "position_mode",
                                       "head_count", "rotation_pairing"};
  for (const auto& kv : inv.attributes)
    if (std::none_of(std::begin(kKnown), std::end(kKnown), [&](const char* k) { return kv.first == k; }))
      return R::failure(KernelError::attribute("rope attribute " + kv.first + " has no GPU path"));
  bool bad = false;
  const float base = attribute_float(inv, "base", &bad).value_or(10000.0f);
  const float scale = attribute_float(inv, "scale", &bad).value_or(1.0f);
  if (bad) return R::failure(KernelError::attribute("rope base and scale must be numbers"));
  auto dim = attribute_integer(inv, "dimension", &bad);
  if (bad || !dim || *dim < 0) return R::failure(KernelError::attribute("dimension"));
  if (const std::string* mode = attribute_text(inv, "position_mode"))
    if (*mode != "sequential")
      return R::failure(KernelError::attribute("position_mode '" + *mode + "' is not implemented"));
  uint64_t offset = 0;
  if (attribute_text(inv, "position_offset")) {
    bool b = false;
    auto o = attribute_integer(inv, "position_offset", &b);
    if (b) return R::failure(KernelError::attribute("position_offset must be an integer"));
    if (*o < 0)
      return R::failure(KernelError::attribute("position_offset " + std::to_string(*o) + " must not be negative"));
    offset = static_cast<uint64_t>(*o);
  }
  auto hc = attribute_integer(inv, "head_count", &bad);
  const uint64_t head_count = hc && *hc >= 0 ? static_cast<uint64_t>(*hc) : 1;
  int pairing = MQ_ROPE_INTERLEAVED;
  if (const std::string* p = attribute_text(inv, "rotation_pairing")) {
    if (*p == "half_split")
      pairing = MQ_ROPE_HALF_SPLIT;
    else if (*p != "interleaved")
      return R::failure(KernelError::attribute("rotation_pairing '" + *p + "' is not implemented"));
  }
  uint64_t rows = 0, cols = 0;
  if (!rows_cols(x.shape, rows, cols)) return R::failure(rank2_error("RoPE", x.shape));
  auto out = begin_output(inv, x.shape);
  if (!out.ok()) return R::failure(out.error);
  if (mq_rope_dev(ctx_, x.dev, rows, cols, base, scale, static_cast<uint64_t>(*dim), offset, head_count, pairing,
                  out.value->tensor.dev, stream_) != MQ_OK) {
    abort_output(*out.value);
    return R::failure(KernelError::failed(mq_last_error(ctx_)));
  }
  commit_output(*out.value);
  return R::success(true);
}

// `kv-write` (src/lib.rs:2458-2526 with `kv_write_in_place`, 740-768): the
// rows written over the store's rows row_offset.. in place when the output
// is the store, else into a copy stored under the output.
Result<bool> GpuExecutor::run_kv_write(const KernelInvocation& inv) {
  using R = Result<bool>;
  auto rows_in = input(inv, 1);
  if (!rows_in.ok()) return R::failure(rows_in.error);
  bool bad = false;
  auto off = attribute_integer(inv, "row_offset", &bad);
  if (bad || !off || *off < 0) return R::failure(KernelError::attribute("row_offset"));
  if (inv.inputs.empty()) return R::failure(KernelError::failed("missing input at index 0"));
  auto store_in = input(inv, 0);
  if (!store_in.ok()) return R::failure(store_in.error);
  const DeviceTensor& store = **store_in.value;
  const DeviceTensor& rows = **rows_in.value;
  uint64_t capacity = 0, width = 0, count = 0, row_width = 0;
  if (!rows_cols(store.shape, capacity, width)) return R::failure(rank2_error("kv-write", store.shape));
  if (!rows_cols(rows.shape, count, row_width)) return R::failure(rank2_error("kv-write", rows.shape));
  if (row_width != width)
    return R::failure(KernelError::failed("kv-write rows have width " + std::to_string(row_width) + ", the store " +
                                          std::to_string(width)));
  const uint64_t row_offset = static_cast<uint64_t>(*off);
  if (row_offset + count < row_offset || row_offset + count > capacity)
    return R::failure(KernelError::failed("kv-write of " + std::to_string(count) + " rows at " +
                                          std::to_string(row_offset) + " exceeds the store's " +
                                          std::to_string(capacity) + " rows"));
  const bool in_place = inv.outputs[0] == inv.inputs[0];
  if (in_place) {
    // the store is rewritten in its own buffer: admitted at its size
    // (unchanged when already admitted), no new allocation
    const std::string& id = inv.outputs[0];
    const bool had = memory_.holds(id);
    const uint64_t previous = memory_.bytes_of(id);
    if (!memory_.admit(id, store.count * sizeof(float))) {
      observe({"KernelMemoryFeasibilityFailed", inv.kernel, inv.id, id});
      return R::failure(KernelError::failed("memory admission denied for output " + id));
    }
    if (mq_kv_write_dev(ctx_, store.dev, capacity, width, rows.dev, count, row_offset, stream_) != MQ_OK) {
      if (had)
        memory_.admit(id, previous);
      else
        memory_.release(id);
      return R::failure(KernelError::failed(mq_last_error(ctx_)));
    }
    return R::success(true);
  }
  auto out = begin_output(inv, store.shape);
  if (!out.ok()) return R::failure(out.error);
  if (mq_copy_dev(ctx_, out.value->tensor.dev, store.dev, store.count * sizeof(float), stream_) != MQ_OK ||
      mq_kv_write_dev(ctx_, out.value->tensor.dev, capacity, width, rows.dev, count, row_offset, stream_) != MQ_OK) {
    abort_output(*out.value);
    return R::failure(KernelError::failed(mq_last_error(ctx_)));
  }
  commit_output(*out.value);
  return R::success(true);
}

// The `attention` Kernel (src/lib.rs:2819-2950) over
// `attention_with_value_width` (780-990): causal or bidirectional, grouped
// query heads, key_count leading keys, an optional score scale. Sliding
// windows, latent K/V and value widths other than head_dimension have no
// GPU path and are refused by name.
Result<bool> GpuExecutor::run_attention(const KernelInvocation& inv) {
  using R = Result<bool>;
  auto q_in = input(inv, 0);
  if (!q_in.ok()) return R::failure(q_in.error);
  auto k_in = input(inv, 1);
  if (!k_in.ok()) return R::failure(k_in.error);
  auto v_in = input(inv, 2);
  if (!v_in.ok()) return R::failure(v_in.error);
  const DeviceTensor &q = **q_in.value, &k = **k_in.value, &v = **v_in.value;
  bool bad = false;
  auto heads = attribute_integer(inv, "head_count", &bad);
  if (bad || !heads || *heads < 0) return R::failure(KernelError::attribute("head_count"));
  auto head_dim = attribute_integer(inv, "head_dimension", &bad);
  if (bad || !head_dim || *head_dim < 0) return R::failure(KernelError::attribute("head_dimension"));
  auto kvh = attribute_integer(inv, "kv_head_count", &bad);
  for (const char* name : {"window_size", "latent_kv_width", "value_head_stride"})
    if (attribute_text(inv, name))
      return R::failure(KernelError::attribute(std::string("attention ") + name + " has no GPU path"));
  if (auto vhd = attribute_integer(inv, "value_head_dimension", &bad))
    if (*vhd != *head_dim)
      return R::failure(KernelError::attribute("attention value_head_dimension has no GPU path"));
  const bool causal = attribute_bool(inv, "causal", false);
  if (const std::string* kind = attribute_text(inv, "attention_mask_kind")) {
    bool expected = false;
    if (*kind == "causal")
      expected = true;
    else if (*kind != "bidirectional")
      return R::failure(KernelError::attribute("attention_mask_kind '" + *kind + "' is not implemented"));
    if (expected != causal)
      return R::failure(KernelError::attribute("attention_mask_kind '" + *kind + "' is inconsistent with causal=" +
                                               (causal ? "true" : "false")));
  }
  float score_scale = std::nanf("");
  if (auto s = attribute_float(inv, "scale", &bad)) score_scale = *s;
  if (bad) return R::failure(KernelError::attribute("attention scale must be a number"));
  uint64_t seq = 0, q_width = 0, kv_rows = 0, kv_width = 0;
  if (!rows_cols(q.shape, seq, q_width)) return R::failure(rank2_error("attention", q.shape));
  if (!rows_cols(k.shape, kv_rows, kv_width)) return R::failure(rank2_error("attention", k.shape));
  uint64_t key_count = kv_rows;
  if (auto kc = attribute_integer(inv, "key_count", &bad)) {
    if (*kc < 0) return R::failure(KernelError::attribute("key_count"));
    key_count = static_cast<uint64_t>(*kc);
    if (key_count > kv_rows)
      return R::failure(KernelError::failed("key_count " + std::to_string(key_count) + " exceeds the " +
                                            std::to_string(kv_rows) + " rows of K/V"));
  }
  if (!std::isnan(score_scale) && !std::isfinite(score_scale))
    return R::failure(KernelError::failed("attention scale must be finite"));
  if (k.shape != v.shape)
    return R::failure(KernelError::failed("shape mismatch: " + shape_text(k.shape) + " vs " + shape_text(v.shape)));
  const uint64_t h = static_cast<uint64_t>(*heads), d = static_cast<uint64_t>(*head_dim);
  const uint64_t kv_heads = kvh && *kvh >= 0 ? static_cast<uint64_t>(*kvh) : h;
  if (h == 0 || d == 0 || kv_heads == 0)
    return R::failure(KernelError::failed("head_count, kv_head_count, and head_dimension must all be positive"));
  if (h % kv_heads)
    return R::failure(KernelError::failed("head_count " + std::to_string(h) +
                                          " must be an exact multiple of kv_head_count " + std::to_string(kv_heads)));
  if (seq > key_count)
    return R::failure(KernelError::failed("q sequence length " + std::to_string(seq) +
                                          " cannot exceed k/v sequence length " + std::to_string(key_count)));
  if (h * d != q_width)
    return R::failure(KernelError::failed("head_count * head_dimension must equal q row width " +
                                          std::to_string(q_width) + ", got " + std::to_string(h) + " * " +
                                          std::to_string(d)));
  if (kv_heads * d != kv_width)
    return R::failure(KernelError::failed("kv_head_count * head_dimension must equal k/v row width " +
                                          std::to_string(kv_width) + ", got " + std::to_string(kv_heads) + " * " +
                                          std::to_string(d)));
  auto out = begin_output(inv, {seq, h * d});
  if (!out.ok()) return R::failure(out.error);
  const int rc = mq_attention_dev(ctx_, q.dev, seq, k.dev, v.dev, kv_rows, key_count, h, d, kv_heads, causal ? 1 : 0,
                                  score_scale, out.value->tensor.dev, stream_);
  if (rc != MQ_OK) {
    abort_output(*out.value);
    if (rc == MQ_DECLINED) return R::failure(KernelError::attribute(mq_last_error(ctx_)));
    return R::failure(KernelError::failed(mq_last_error(ctx_)));
  }
  commit_output(*out.value);
  return R::success(true);
}

// The `silu-mul` Kernel (src/lib.rs:2592-2596): mul(silu(gate), up), the
// shapes equal.
Result<bool> GpuExecutor::run_silu_mul(const KernelInvocation& inv) {
  using R = Result<bool>;
  auto g_in = input(inv, 0);
  if (!g_in.ok()) return R::failure(g_in.error);
  auto u_in = input(inv, 1);
  if (!u_in.ok()) return R::failure(u_in.error);
  const DeviceTensor &g = **g_in.value, &u = **u_in.value;
  if (g.shape != u.shape)
    return R::failure(KernelError::failed("shape mismatch: " + shape_text(g.shape) + " vs " + shape_text(u.shape)));
  auto out = begin_output(inv, g.shape);
  if (!out.ok()) return R::failure(out.error);
  if (mq_silu_mul_dev(ctx_, g.dev, u.dev, g.count, out.value->tensor.dev, stream_) != MQ_OK) {
    abort_output(*out.value);
    return R::failure(KernelError::failed(mq_last_error(ctx_)));
  }
  commit_output(*out.value);
  return R::success(true);
}

// `add` / `residual-add` (src/lib.rs:2998-3036 over `add`, 1019-1075, and
// `residual_add`, 1128-1133): b of a's shape, or one row broadcast.
Result<bool> GpuExecutor::run_add(const KernelInvocation& inv, bool residual) {
  using R = Result<bool>;
  (void)residual;  // residual_add(input, residual) = add(input, residual)
  auto a_in = input(inv, 0);
  if (!a_in.ok()) return R::failure(a_in.error);
  auto b_in = input(inv, 1);
  if (!b_in.ok()) return R::failure(b_in.error);
  const DeviceTensor &a = **a_in.value, &b = **b_in.value;
  uint64_t b_n = b.count;
  if (a.shape != b.shape) {
    if (a.shape.empty()) return R::failure(KernelError::failed("add expects at least one dimension"));
    const uint64_t cols = a.shape.back();
    const std::vector<uint64_t> r1{cols}, r2{1, cols};
    if (b.shape != r1 && b.shape != r2)
      return R::failure(KernelError::failed("add expects b to match a's shape " + shape_text(a.shape) +
                                            " or broadcast as [" + std::to_string(cols) + "]/[1, " +
                                            std::to_string(cols) + "], got " + shape_text(b.shape)));
    if (cols == 0 || a.count % cols)
      return R::failure(KernelError::failed("add data length " + std::to_string(a.count) +
                                            " is not divisible by broadcast dimension " + std::to_string(cols)));
    b_n = cols;
  }
  auto out = begin_output(inv, a.shape);
  if (!out.ok()) return R::failure(out.error);
  if (a.count && mq_add_dev(ctx_, a.dev, a.count, b.dev, b_n, out.value->tensor.dev, stream_) != MQ_OK) {
    abort_output(*out.value);
    return R::failure(KernelError::failed(mq_last_error(ctx_)));
  }
  commit_output(*out.value);
  return R::success(true);
}

// ---- dispatch ----------------------------------------------------------------------------

// `execute_invocation` (src/lib.rs:2361-2403) and `run_invocation`
// (2528-3058): observe Started; deadline 0 -> KernelTimeout; kv-write; the
// packed hook before the other Kernels; the output admitted before
// dispatch and stored on the device.
KernelResult GpuExecutor::execute_invocation(const KernelInvocation& inv) {
  KernelResult result;
  result.invocation = inv.id;
  observe({"KernelDispatchStarted", inv.kernel, inv.id, ""});
  if (inv.deadline_millis && *inv.deadline_millis == 0) {
    observe({"KernelTimeout", inv.kernel, inv.id, ""});
    result.error = {KernelErrorKind::Timeout, "the invocation's deadline elapsed before dispatch"};
    return result;
  }
  const auto ads = gpu_kernel_advertisements();
  const bool advertised =
      std::any_of(ads.begin(), ads.end(), [&](const KernelAdvertisement& a) { return a.name == inv.kernel; });
  const auto started = std::chrono::steady_clock::now();
  Result<bool> ran = Result<bool>::failure({});
  if (!advertised) {
    ran = Result<bool>::failure({KernelErrorKind::NotFound, "kernel " + inv.kernel + " is not advertised"});
  } else if (inv.outputs.empty()) {
    ran = Result<bool>::failure(KernelError::failed("missing output at index 0"));
  } else {
    std::lock_guard<std::mutex> lock(mu_);
    const std::string& k = inv.kernel;
    const bool is_matmul = k == "matmul" || k == "matmul-bias" || k == "matmul-residual";
    std::optional<GpuPackedWeights::Entry> packed;
    if (packed_ && is_matmul && inv.inputs.size() > 1) packed = packed_->find(inv.inputs[1]);
    if (packed_ && k == "embedding" && !inv.inputs.empty()) packed = packed_->find(inv.inputs[0]);
    if (k == "kv-write") {
      ran = run_kv_write(inv);
    } else if (is_matmul) {
      // PackedWeights::run -> None for an f32 weight: the Reference CPU
      // executor the reference wraps would run it; this executor has no
      // dense f32 matmul of its own
      ran = packed ? run_matmul(inv, *packed)
                   : Result<bool>::failure({KernelErrorKind::NotFound,
                                            "input 1 of " + k + " is not a packed weight resident on this GPU"});
    } else if (k == "embedding") {
      ran = packed ? run_embedding(inv, *packed)
                   : Result<bool>::failure({KernelErrorKind::NotFound,
                                            "input 0 of embedding is not a packed table resident on this GPU"});
    } else if (k == "rmsnorm") {
      ran = run_rmsnorm(inv);
    } else if (k == "rope") {
      ran = run_rope(inv);
    } else if (k == "attention") {
      ran = run_attention(inv);
    } else if (k == "silu-mul") {
      ran = run_silu_mul(inv);
    } else if (k == "add" || k == "residual-add") {
      ran = run_add(inv, k == "residual-add");
    } else {
      ran = Result<bool>::failure({KernelErrorKind::NotFound, "kernel " + k + " has no GPU arm"});
    }
    if (ran.ok() && profile_on_) {
      mq_synchronize(ctx_, stream_);
      auto& p = profile_[k];
      p.first += 1;
      p.second += std::chrono::duration<double>(std::chrono::steady_clock::now() - started).count();
    }
  }
  if (!ran.ok()) {
    observe({"KernelDispatchFailed", inv.kernel, inv.id, ran.error.reason});
    result.error = ran.error;
    return result;
  }
  observe({"KernelDispatchCompleted", inv.kernel, inv.id, ""});
  result.succeeded = true;
  result.updated_resources.push_back(inv.outputs[0]);
  return result;
}

// `submit_kernel_invocation` (src/lib.rs:2301-2330): the result waits under a
// handle "<provider>:<invocation>:<n>". The Kernel is enqueued on the
// device; its outputs are read back (read_tensor) after it completes.
std::string GpuExecutor::submit_kernel(const KernelInvocation& inv) {
  std::string handle =
      std::string(kGpuProviderName) + ":" + inv.id + ":" + std::to_string(ordinal_.fetch_add(1));
  KernelResult r = execute_invocation(inv);
  std::lock_guard<std::mutex> lock(mu_);
  executions_[handle] = std::move(r);
  return handle;
}

// `complete_kernel_invocation` (src/lib.rs:2337-2356): single consumption.
bool GpuExecutor::complete_kernel(const std::string& handle, KernelResult* out) {
  std::lock_guard<std::mutex> lock(mu_);
  auto it = executions_.find(handle);
  if (it == executions_.end()) return false;
  if (out) *out = std::move(it->second);
  executions_.erase(it);
  return true;
}

}  // namespace magnetar
