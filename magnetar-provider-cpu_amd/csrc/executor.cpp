// GpuExecutor / GpuPackedWeights: the Provider-side contract of the
// packed-weight matmul Kernel over the libmagnetar_gpu C ABI.
#include "executor.hpp"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

namespace magnetar {

namespace {

constexpr size_t kMaxObservations = 4096;  // bounded log (src/lib.rs:171-172)

bool attribute_bool(const KernelInvocation& inv, const char* name, bool fallback) {
  auto it = inv.attributes.find(name);
  if (it == inv.attributes.end()) return fallback;
  return it->second == "true" || it->second == "1";
}

std::string shape_text(const std::vector<uint64_t>& s) {
  std::string out = "[";
  for (size_t i = 0; i < s.size(); ++i) out += (i ? ", " : "") + std::to_string(s[i]);
  return out + "]";
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

// `baseline_advertisement` for matmul and its fused forms under this
// Provider's identity (src/lib.rs:1350-1373, src/native/mod.rs:847-864):
// f32 in/out, contiguous, Host memory class, rank 2, TimeoutOnly.
std::vector<KernelAdvertisement> gpu_kernel_advertisements() {
  std::vector<KernelAdvertisement> out;
  for (const char* name : {"matmul", "matmul-bias", "matmul-residual", "embedding"}) {
    KernelAdvertisement a;
    a.provider = kGpuProviderName;
    a.name = name;
    a.version = "1.0.0";
    a.operator_id = std::string("magnetar:") + name + "@1";
    a.family = std::string(name) == "embedding" ? "GpuGather" : "GpuMatrix";
    a.conformance_profile = kConformanceProfile;
    a.input_dtypes = {"f32"};
    a.output_dtypes = {"f32"};
    a.layouts = {"Contiguous"};
    a.memory_classes = {"Host"};
    a.devices = {kGpuDeviceId};
    a.cancellation = "TimeoutOnly";
    if (std::string(name) == "matmul") a.rank = 2;
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

bool GpuPackedWeights::contains(const std::string& id) { return find(id).has_value(); }

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
  return e->transposed ? std::vector<uint64_t>{e->cols, e->rows} : std::vector<uint64_t>{e->rows, e->cols};
}

// `materialize` -> `NativeState::expand` -> `PackedWeight::dequantize`: the
// logical values, counted (src/native/mod.rs:196-204, 455-457).
std::optional<HostTensor> GpuPackedWeights::materialize(const std::string& id) {
  auto e = find(id);
  if (!e) return std::nullopt;
  HostTensor t;
  t.shape = e->transposed ? std::vector<uint64_t>{e->cols, e->rows} : std::vector<uint64_t>{e->rows, e->cols};
  t.data.resize(e->rows * e->cols);
  if (mq_dequantize(ctx_, e->handle, e->transposed ? 1 : 0, t.data.data()) != MQ_OK) return std::nullopt;
  materialized_++;
  return t;
}

// `PackedWeights::run` (src/native/mod.rs:421-430): matmul and its fused
// forms when input 1 is a packed weight.
std::optional<Result<HostTensor>> GpuPackedWeights::run(const GpuExecutor& executor,
                                                        const KernelInvocation& inv) {
  if (inv.kernel == "embedding") {
    // the table is input 0; an f32 table is the wrapped executor's
    if (inv.inputs.size() < 2) return std::nullopt;
    auto t = find(inv.inputs[0]);
    if (!t) return std::nullopt;
    return embedding(executor, inv, *t);
  }
  if (inv.kernel != "matmul" && inv.kernel != "matmul-bias" && inv.kernel != "matmul-residual") return std::nullopt;
  if (inv.inputs.size() < 2) return std::nullopt;
  auto w = find(inv.inputs[1]);
  if (!w) return std::nullopt;
  return matmul(executor, inv, *w);
}

// `NativeState::matmul` (src/native/mod.rs:206-236) with `packed_matmul`
// (110-152): shape checks, f32-only accumulation, routing, and the bias /
// residual epilogue fused into the kernel's output write.
Result<HostTensor> GpuPackedWeights::matmul(const GpuExecutor& executor, const KernelInvocation& inv,
                                            const Entry& w) {
  using R = Result<HostTensor>;
  auto a_opt = executor.read_tensor(inv.inputs[0]);
  if (!a_opt) return R::failure(KernelError::failed("no materialized data for input resource " + inv.inputs[0]));
  HostTensor a = std::move(*a_opt);
  const bool transpose_a = attribute_bool(inv, "transpose_a", false);
  const bool transpose_b = attribute_bool(inv, "transpose_b", false);
  auto acc = inv.attributes.find("accumulation_dtype");
  if (acc != inv.attributes.end() && acc->second != "f32" && acc->second != "float32" && acc->second != "Float32")
    return R::failure({KernelErrorKind::DTypeUnsupported,
                       "the GPU packed matmul only accumulates in f32; requested " + acc->second});
  uint64_t m = 0, k = 0;
  if (!a.rows_cols(m, k))
    return R::failure(KernelError::failed("matmul expects a rank-2 activation tensor, got shape " + shape_text(a.shape)));
  uint32_t flags = (int8_ ? MQ_INT8_ACTIVATIONS : 0) | (transpose_b ? MQ_TRANSPOSE_B : 0);
  if (transpose_a) {
    // The reference expands the weight and runs the dense f32 matmul: f32
    // activations, the transposed activation read by stride swap.
    HostTensor t;
    t.shape = {k, m};
    t.data.resize(a.data.size());
    for (uint64_t r = 0; r < m; ++r)
      for (uint64_t c = 0; c < k; ++c) t.data[c * m + r] = a.data[r * k + c];
    std::swap(m, k);
    a = std::move(t);
    flags &= ~MQ_INT8_ACTIVATIONS;
  }
  // the reference's orientation rule (src/native/mod.rs:217-227): stored
  // rows are the outputs when transposed != transpose_b, else the inputs
  // (`packed_axpy`, f32 activations)
  const bool output_major = w.transposed != transpose_b;
  if (!output_major) flags &= ~MQ_INT8_ACTIVATIONS;
  if (output_major && (k != w.cols || k % 32 != 0))
    return R::failure(KernelError::failed("packed matmul: activations have " + std::to_string(k) +
                                          " columns, the weight's stored rows " + std::to_string(w.cols)));
  if (!output_major && k != w.rows)
    return R::failure(KernelError::failed("packed matmul: activations have " + std::to_string(k) +
                                          " columns, the weight " + std::to_string(w.rows) + " stored rows"));
  const uint64_t n = output_major ? w.rows : w.cols;
  HostTensor out;
  out.shape = {m, n};
  out.data.resize(m * n);
  const float* addend = nullptr;
  uint64_t addend_rows = 0;
  HostTensor extra;
  if (inv.kernel != "matmul") {
    if (inv.inputs.size() < 3) return R::failure(KernelError::failed("missing input at index 2"));
    auto e = executor.read_tensor(inv.inputs[2]);
    if (!e) return R::failure(KernelError::failed("no materialized data for input resource " + inv.inputs[2]));
    extra = std::move(*e);
    const bool same = extra.shape == out.shape;
    const bool broadcast = inv.kernel == "matmul-bias" &&
                           (extra.shape == std::vector<uint64_t>{n} || extra.shape == std::vector<uint64_t>{1, n});
    if (!same && !broadcast)
      return R::failure(KernelError::failed("add expects b to match a's shape " + shape_text(out.shape) +
                                            " or broadcast as [" + std::to_string(n) + "]/[1, " +
                                            std::to_string(n) + "], got " + shape_text(extra.shape)));
    if (extra.data.size() != (same ? m * n : n)) return R::failure(KernelError::failed("addend data length mismatch"));
    addend = extra.data.data();
    addend_rows = same ? m : 1;
  }
  int rc = addend ? mq_matmul_add(ctx_, w.handle, a.data.data(), m, k, flags, addend, addend_rows, out.data.data())
                  : mq_matmul(ctx_, w.handle, a.data.data(), m, k, flags, out.data.data());
  if (rc != MQ_OK) return R::failure(KernelError::failed(mq_last_error(ctx_)));
  return R::success(std::move(out));
}

// `NativeState::embedding` (src/native/mod.rs:389-417) and the `scale`
// attribute (432-449): the token rows of a packed table, validated and
// gathered on the GPU.
Result<HostTensor> GpuPackedWeights::embedding(const GpuExecutor& executor, const KernelInvocation& inv,
                                               const Entry& table) {
  using R = Result<HostTensor>;
  auto ids = executor.read_tensor(inv.inputs[1]);
  if (!ids) return R::failure(KernelError::failed("no materialized data for input resource " + inv.inputs[1]));
  float scale = std::nanf("");
  auto it = inv.attributes.find("scale");
  if (it != inv.attributes.end()) {
    char* end = nullptr;
    scale = std::strtof(it->second.c_str(), &end);
    if (end == it->second.c_str())
      return R::failure({KernelErrorKind::AttributeUnsupported, "embedding scale " + it->second + " is not a number"});
  }
  const uint64_t dim = table.transposed ? table.rows : table.cols;
  HostTensor out;
  out.shape = {static_cast<uint64_t>(ids->data.size()), dim};
  out.data.resize(ids->data.size() * dim);
  if (mq_embedding(ctx_, table.handle, ids->data.data(), ids->data.size(), scale, out.data.data()) != MQ_OK)
    return R::failure(KernelError::failed(mq_last_error(ctx_)));
  return R::success(std::move(out));
}

// ---- GpuExecutor ----------------------------------------------------------------

GpuExecutor::GpuExecutor(int device, bool packed_weights, bool int8_activations, uint64_t memory_capacity)
    : packed_weights_(packed_weights), memory_(memory_capacity) {
  if (mq_create(device, &ctx_) != MQ_OK) {
    init_error_ = mq_last_error(nullptr);
    ctx_ = nullptr;
    return;
  }
  packed_ = std::make_unique<GpuPackedWeights>(ctx_, int8_activations);
  observe({"ProviderRegistered", "", "", kGpuProviderName});
  observe({"DeviceDetected", "", "", kGpuDeviceId});
}

GpuExecutor::~GpuExecutor() {
  packed_.reset();
  if (ctx_) mq_destroy(ctx_);
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
    storage_.erase(id);
  }
  return r;
}

// `write_tensor`: an f32 write forgets a packed weight of the same id
// (src/native/mod.rs:629-636).
void GpuExecutor::write_tensor(const std::string& id, HostTensor tensor) {
  const bool was_packed = packed_ && packed_->forget(id);
  std::lock_guard<std::mutex> lock(mu_);
  if (was_packed) memory_.release(id);  // the device bytes it held
  storage_[id] = std::move(tensor);
}

// `write_tensor_admitted` (src/native/mod.rs:664-681, src/lib.rs:1711-1735):
// the packed weight is replaced only once its replacement is admitted.
bool GpuExecutor::write_tensor_admitted(const std::string& id, HostTensor tensor) {
  {
    std::lock_guard<std::mutex> lock(mu_);
    if (!memory_.admit(id, tensor.data.size() * sizeof(float))) return false;
    storage_[id] = std::move(tensor);
  }
  if (packed_) packed_->forget(id);
  return true;
}

// `read_tensor` falls back to the packed weight's materialization
// (src/lib.rs:1615-1620).
std::optional<HostTensor> GpuExecutor::read_tensor(const std::string& id) const {
  {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = storage_.find(id);
    if (it != storage_.end()) return it->second;
  }
  if (!packed_) return std::nullopt;
  return packed_->materialize(id);
}

std::optional<std::vector<uint64_t>> GpuExecutor::resident_shape(const std::string& id) const {
  {
    std::lock_guard<std::mutex> lock(mu_);
    auto it = storage_.find(id);
    if (it != storage_.end()) return it->second.shape;
  }
  if (!packed_) return std::nullopt;
  return packed_->shape(id);
}

bool GpuExecutor::release_tensor(const std::string& id) {
  bool packed = packed_ && packed_->forget(id);
  std::lock_guard<std::mutex> lock(mu_);
  memory_.release(id);
  return storage_.erase(id) > 0 || packed;
}

bool GpuExecutor::is_packed(const std::string& id) const { return packed_ && packed_->contains(id); }

bool GpuExecutor::read_tensor_value_is_opaque(const std::string& id) const {
  if (is_packed(id)) return true;
  std::lock_guard<std::mutex> lock(mu_);
  return storage_.count(id) > 0;
}

// `execute_invocation` (src/lib.rs:2361-2403) and `run_invocation`
// (2528-2559): observe Started; deadline 0 -> KernelTimeout; the packed hook
// before anything else; store the output.
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
  std::optional<Result<HostTensor>> ran;
  if (!advertised) {
    ran = Result<HostTensor>::failure({KernelErrorKind::NotFound, "kernel " + inv.kernel + " is not advertised"});
  } else if (inv.outputs.empty()) {
    ran = Result<HostTensor>::failure(KernelError::failed("missing output at index 0"));
  } else if (packed_) {
    ran = packed_->run(*this, inv);
  }
  if (!ran) {
    // PackedWeights::run -> None: not a packed-weight invocation. In the
    // Runtime the wrapped Reference CPU executor runs it; this executor
    // holds no f32 kernel of its own.
    ran = Result<HostTensor>::failure(
        {KernelErrorKind::NotFound, "input 1 of " + inv.kernel + " is not a packed weight resident on this GPU"});
  }
  if (!ran->ok()) {
    observe({"KernelDispatchFailed", inv.kernel, inv.id, ran->error.reason});
    result.error = ran->error;
    return result;
  }
  const std::string& out_id = inv.outputs[0];
  {
    std::lock_guard<std::mutex> lock(mu_);
    if (!memory_.admit(out_id, ran->value->data.size() * sizeof(float))) {
      observe({"KernelMemoryFeasibilityFailed", inv.kernel, inv.id, out_id});
      result.error = KernelError::failed("memory admission denied for output " + out_id);
      return result;
    }
    storage_[out_id] = std::move(*ran->value);
  }
  if (packed_) packed_->forget(out_id);
  observe({"KernelDispatchCompleted", inv.kernel, inv.id, ""});
  result.succeeded = true;
  result.updated_resources.push_back(out_id);
  return result;
}

// `submit_kernel_invocation` (src/lib.rs:2301-2330): synchronous; the
// result waits under a handle "<provider>:<invocation>:<n>".
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
