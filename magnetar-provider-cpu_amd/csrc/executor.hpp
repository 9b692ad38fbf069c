// Host-side GPU executor for the Provider's packed-weight matmul Kernel.
//
// C++ stand-in for the Rust side the reference would compile (no Rust
// toolchain here): it mirrors, name for name, the parts of the Provider
// contract this path touches, and reaches the GPU only through the
// libmagnetar_gpu C ABI (include/magnetar_gpu.h).
//
//   GpuPackedWeights  <- `trait PackedWeights` + `NativeState`
//                        (src/native/mod.rs:62-73, 75-236, 420-462)
//   GpuExecutor       <- `NativeCpuExecutor` wrapping `ReferenceCpuExecutor`
//                        (src/native/mod.rs:465-811; src/lib.rs:1556-1868,
//                        2132-2456, 2528-2559)
//   gpu_kernel_advertisements <- `native_cpu_kernel_advertisements` /
//                        `baseline_advertisement` (src/native/mod.rs:847-864;
//                        src/lib.rs:1350-1373)
#pragma once

#include <atomic>
#include <cstdint>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <optional>
#include <string>
#include <vector>

#include "magnetar_gpu.h"

namespace magnetar {

constexpr const char* kGpuProviderName = "magnetar-provider-gpu-mi355x";
constexpr const char* kGpuDeviceId = "gpu-mi355x:hip:0";
constexpr const char* kConformanceProfile = "reference-cpu-conformance-v1";

// `HostTensor` (external magnetar-core type): row-major f32 with a shape.
struct HostTensor {
  std::vector<uint64_t> shape;
  std::vector<float> data;
  bool rows_cols(uint64_t& rows, uint64_t& cols) const;
};

// `PackedWeight` (external magnetar-provider-api type): checkpoint bytes
// of `stored_rows` rows x `stored_cols` values; transposed = the stored
// rows are the output columns, logical shape [stored_cols, stored_rows].
struct PackedWeight {
  uint32_t format = 0;
  uint64_t stored_rows = 0, stored_cols = 0;
  bool transposed = true;
  std::vector<uint8_t> bytes;
  std::vector<uint64_t> logical_shape() const;
};

enum class PackedWeightWrite { Stored, Declined };

// `KernelError` variants (external magnetar-kernel type).
enum class KernelErrorKind {
  None = 0,
  ExecutionFailed = 1,
  DTypeUnsupported = 2,
  AttributeUnsupported = 3,
  NotFound = 4,
  Timeout = 5,
};

struct KernelError {
  KernelErrorKind kind = KernelErrorKind::None;
  std::string reason;
  static KernelError failed(std::string reason) { return {KernelErrorKind::ExecutionFailed, std::move(reason)}; }
};

template <class T>
struct Result {
  std::optional<T> value;
  KernelError error;
  bool ok() const { return value.has_value(); }
  static Result success(T v) { return Result{std::move(v), {}}; }
  static Result failure(KernelError e) { return Result{std::nullopt, std::move(e)}; }
};

// `KernelInvocation`: resource ids of inputs and outputs, attributes as
// text ("true"/"false" for booleans, a dtype name for accumulation_dtype).
struct KernelInvocation {
  std::string id;
  std::string kernel;
  std::vector<std::string> inputs;
  std::vector<std::string> outputs;
  std::map<std::string, std::string> attributes;
  std::optional<uint64_t> deadline_millis;
};

struct KernelResult {
  std::string invocation;
  bool succeeded = false;
  KernelError error;
  std::vector<std::string> updated_resources;
};

struct KernelAdvertisement {
  std::string provider, name, version, operator_id, family, conformance_profile;
  std::vector<std::string> input_dtypes, output_dtypes, layouts, memory_classes, devices;
  std::string cancellation;
  std::optional<uint32_t> rank;
};

std::vector<KernelAdvertisement> gpu_kernel_advertisements();

// `KernelObservationKind` events this executor records.
struct KernelObservation {
  std::string kind, kernel, invocation, detail;
};

// The `MemoryManager` ledger this path needs: admission against a byte
// capacity, one allocation per admitted resource id.
class MemoryLedger {
 public:
  explicit MemoryLedger(uint64_t capacity) : capacity_(capacity) {}
  bool admit(const std::string& id, uint64_t bytes);  // replaces id's allocation
  void release(const std::string& id);
  uint64_t used() const { return used_; }
  uint64_t capacity() const { return capacity_; }

 private:
  uint64_t capacity_, used_ = 0;
  std::map<std::string, uint64_t> allocations_;
};

class GpuExecutor;

// `trait PackedWeights` on the GPU: packed weights by resource id, resident
// in HBM in the context's tiled layout.
class GpuPackedWeights {
 public:
  GpuPackedWeights(mq_ctx* ctx, bool int8_activations) : ctx_(ctx), int8_(int8_activations) {}
  ~GpuPackedWeights();

  // `PackedWeights::run`: std::nullopt lets the wrapped executor's f32
  // kernel run (the invocation does not read a packed weight).
  std::optional<Result<HostTensor>> run(const GpuExecutor& executor, const KernelInvocation& invocation);
  std::optional<HostTensor> materialize(const std::string& id);
  std::optional<std::vector<uint64_t>> shape(const std::string& id);

  // Uploads the weight; `admit` (may be empty) is asked for its device
  // bytes before the upload replaces a weight of the same id: false
  // releases the upload and declines, leaving any previous weight.
  PackedWeightWrite store(const std::string& id, const PackedWeight& weight, std::string* why,
                          const std::function<bool(uint64_t)>& admit = {});
  bool forget(const std::string& id);
  bool contains(const std::string& id);
  uint64_t materializations() const { return materialized_; }

 private:
  struct Entry {
    uint64_t handle;
    uint32_t format;
    uint64_t rows, cols;
    bool transposed;
  };
  std::optional<Entry> find(const std::string& id);
  Result<HostTensor> matmul(const GpuExecutor& executor, const KernelInvocation& invocation, const Entry& weight);
  Result<HostTensor> embedding(const GpuExecutor& executor, const KernelInvocation& invocation, const Entry& table);

  mq_ctx* ctx_;
  bool int8_;
  std::mutex mu_;
  std::map<std::string, Entry> packed_;
  std::atomic<uint64_t> materialized_{0};
};

class GpuExecutor {
 public:
  GpuExecutor(int device, bool packed_weights, bool int8_activations, uint64_t memory_capacity);
  ~GpuExecutor();
  GpuExecutor(const GpuExecutor&) = delete;
  GpuExecutor& operator=(const GpuExecutor&) = delete;

  bool ready() const { return ctx_ != nullptr; }
  const std::string& init_error() const { return init_error_; }

  PackedWeightWrite write_packed_weight_tensor(const std::string& id, const PackedWeight& weight,
                                               std::string* why = nullptr);
  void write_tensor(const std::string& id, HostTensor tensor);
  // `write_tensor_admitted`: false (MemoryError) when admission is denied;
  // a packed weight under `id` stays resident then.
  bool write_tensor_admitted(const std::string& id, HostTensor tensor);
  std::optional<HostTensor> read_tensor(const std::string& id) const;
  std::optional<std::vector<uint64_t>> resident_shape(const std::string& id) const;
  bool release_tensor(const std::string& id);
  bool is_packed(const std::string& id) const;
  // `read_tensor_value` answers Opaque for every resident id (mod.rs:695-702).
  bool read_tensor_value_is_opaque(const std::string& id) const;

  std::string submit_kernel(const KernelInvocation& invocation);
  // Single consumption: false for an unknown or already-completed handle.
  bool complete_kernel(const std::string& handle, KernelResult* out);
  std::vector<KernelObservation> observations() const;
  const MemoryLedger& memory() const { return memory_; }
  uint64_t materializations() const { return packed_ ? packed_->materializations() : 0; }

 private:
  friend class GpuPackedWeights;
  KernelResult execute_invocation(const KernelInvocation& invocation);
  void observe(KernelObservation o) const;

  mq_ctx* ctx_ = nullptr;
  std::string init_error_;
  bool packed_weights_;
  std::unique_ptr<GpuPackedWeights> packed_;
  mutable std::mutex mu_;
  std::map<std::string, HostTensor> storage_;
  std::map<std::string, KernelResult> executions_;
  MemoryLedger memory_;
  std::atomic<uint64_t> ordinal_{0};
  mutable std::mutex obs_mu_;
  mutable std::vector<KernelObservation> observations_;
};

}  // namespace magnetar
