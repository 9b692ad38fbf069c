// Host-side GPU executor: the Provider contract over device-resident
// tensors and the gfx950 kernels.
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
//                        2132-2456, 2528-3058)
//   gpu_kernel_advertisements <- `native_cpu_kernel_advertisements` /
//                        `baseline_advertisement` (src/native/mod.rs:847-864;
//                        src/lib.rs:1350-1373)
//
// Tensors live in HBM (placement ProviderOwnedOpaque): write_tensor copies
// in, read_tensor copies out, and every Kernel reads and writes device
// buffers on the context's stream. read_tensor_value answers Opaque, as the
// reference's optimized Provider does (src/native/mod.rs:695-702), so a
// Runtime chaining Kernels never moves activations across PCIe.
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
  static KernelError attribute(std::string reason) {
    return {KernelErrorKind::AttributeUnsupported, std::move(reason)};
  }
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
// text ("true"/"false" for booleans, a dtype name for accumulation_dtype,
// decimal text for integers and floats).
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
// capacity, one allocation per admitted resource id (workspaces under
// their own allocation ids).
class MemoryLedger {
 public:
  explicit MemoryLedger(uint64_t capacity) : capacity_(capacity) {}
  bool admit(const std::string& id, uint64_t bytes);  // replaces id's allocation
  void release(const std::string& id);
  bool holds(const std::string& id) const { return allocations_.count(id) != 0; }
  uint64_t bytes_of(const std::string& id) const;
  uint64_t used() const { return used_; }
  uint64_t capacity() const { return capacity_; }

 private:
  uint64_t capacity_, used_ = 0;
  std::map<std::string, uint64_t> allocations_;
};

// A tensor resident in this GPU's HBM: row-major f32 in a buffer of
// `capacity` bytes (at least count * 4), owned by the executor.
struct DeviceTensor {
  std::vector<uint64_t> shape;
  uint64_t count = 0;
  float* dev = nullptr;
  uint64_t capacity = 0;
};

// `KvStorePrecision` (external magnetar-provider-api type): f32 stores run
// on the GPU; the TurboQuant precisions are declined.
enum class KvStorePrecision { F32 = 0, TurboQuant = 1 };

// `trait PackedWeights` on the GPU: packed weights by resource id, resident
// in HBM in the context's tiled layout.
class GpuPackedWeights {
 public:
  struct Entry {
    uint64_t handle;
    uint32_t format;
    uint64_t rows, cols;
    bool transposed;
    std::vector<uint64_t> logical_shape() const;
  };

  explicit GpuPackedWeights(mq_ctx* ctx) : ctx_(ctx) {}
  ~GpuPackedWeights();

  // Uploads the weight; `admit` (may be empty) is asked for its device
  // bytes before the upload replaces a weight of the same id: false
  // releases the upload and declines, leaving any previous weight.
  PackedWeightWrite store(const std::string& id, const PackedWeight& weight, std::string* why,
                          const std::function<bool(uint64_t)>& admit = {});
  bool forget(const std::string& id);
  std::optional<Entry> find(const std::string& id);
  bool contains(const std::string& id) { return find(id).has_value(); }
  std::optional<std::vector<uint64_t>> shape(const std::string& id);
  // `materialize`: the logical f32 values (dequantized on the device),
  // counted (src/native/mod.rs:196-204, 455-457).
  std::optional<HostTensor> materialize(const std::string& id);
  // The logical values into device memory `out` (count = rows * cols), on
  // the context's stream, counted like materialize.
  bool materialize_dev(const Entry& e, float* out);
  uint64_t materializations() const { return materialized_; }

 private:
  mq_ctx* ctx_;
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

  // ---- ProviderExecutionApi storage -----------------------------------------
  PackedWeightWrite write_packed_weight_tensor(const std::string& id, const PackedWeight& weight,
                                               std::string* why = nullptr);
  // `write_tensor`: false only when the device refuses the copy (why set).
  bool write_tensor(const std::string& id, const HostTensor& tensor, std::string* why = nullptr);
  // `write_tensor_admitted`: false with *denied when admission is denied (a
  // packed weight under `id` stays resident then).
  bool write_tensor_admitted(const std::string& id, const HostTensor& tensor, bool* denied, std::string* why);
  std::optional<HostTensor> read_tensor(const std::string& id);
  std::optional<std::vector<uint64_t>> resident_shape(const std::string& id);
  bool release_tensor(const std::string& id);
  // `release_admitted_tensor`: also returns the ledger's allocation.
  bool release_admitted_tensor(const std::string& id);
  bool is_packed(const std::string& id);
  // `read_tensor_value` answers Opaque for every resident id (mod.rs:695-702).
  bool read_tensor_value_is_opaque(const std::string& id);
  // `write_tensor_value` / `_admitted`: an Opaque value (host == nullptr)
  // stores nothing, so a packed weight stays; a Host value replaces.
  bool write_tensor_value(const std::string& id, const HostTensor* host, std::string* why);
  bool write_tensor_value_admitted(const std::string& id, const HostTensor* host, bool* denied, std::string* why);
  // `copy_tensor_admitted`: a device copy of `from` (a tensor, or a packed
  // weight's logical values) under `to`, which it replaces, a packed weight
  // included. false with *denied for an admission failure, else why.
  bool copy_tensor_admitted(const std::string& from, const std::string& to, bool* denied, std::string* why);
  // `write_zeroed_kv_store(_with_exact_head)`: a zeroed f32 [capacity, width]
  // store; false for a shape that is not [capacity, whole heads] or a
  // precision without a GPU path.
  bool write_zeroed_kv_store(const std::string& id, const std::vector<uint64_t>& shape,
                             KvStorePrecision precision, uint64_t head_dimension, uint64_t exact_rows,
                             std::string* why);
  // `allocate_workspace`: admits `bytes` of scratch; the allocation id.
  std::optional<std::string> allocate_workspace(uint64_t bytes);
  bool release_workspace(const std::string& allocation);

  // ---- Kernels ----------------------------------------------------------------
  // `submit_kernel`: validates and enqueues the invocation on the device
  // and stores its KernelResult under the returned handle.
  std::string submit_kernel(const KernelInvocation& invocation);
  // Single consumption: false for an unknown or already-completed handle.
  bool complete_kernel(const std::string& handle, KernelResult* out);
  // Waits for every Kernel queued so far.
  bool synchronize();

  std::vector<KernelObservation> observations() const;
  uint64_t memory_used() const;
  uint64_t memory_capacity() const;
  uint64_t materializations() const { return packed_ ? packed_->materializations() : 0; }

  // Per-Kernel (calls, seconds) when MAGNETAR_GPU_PROFILE=1: each Kernel's
  // submission is timed to its completion on the device.
  std::vector<std::pair<std::string, std::pair<uint64_t, double>>> profile() const;

 private:
  struct Output;
  KernelResult execute_invocation(const KernelInvocation& invocation);
  void observe(KernelObservation o) const;

  // Kernel arms (caller holds mu_).
  Result<bool> run_matmul(const KernelInvocation& inv, const GpuPackedWeights::Entry& w);
  Result<bool> run_embedding(const KernelInvocation& inv, const GpuPackedWeights::Entry& table);
  Result<bool> run_rmsnorm(const KernelInvocation& inv);
  Result<bool> run_rope(const KernelInvocation& inv);
  Result<bool> run_kv_write(const KernelInvocation& inv);
  Result<bool> run_attention(const KernelInvocation& inv);
  Result<bool> run_silu_mul(const KernelInvocation& inv);
  Result<bool> run_add(const KernelInvocation& inv, bool residual);

  // Storage helpers (caller holds mu_).
  Result<const DeviceTensor*> input(const KernelInvocation& inv, size_t index);
  Result<Output> begin_output(const KernelInvocation& inv, const std::vector<uint64_t>& shape);
  void commit_output(Output& out);
  void abort_output(Output& out);
  float* scratch(uint64_t count, std::string* why);
  bool store_host(const std::string& id, const HostTensor& tensor, std::string* why);
  void retire(float* dev, uint64_t bytes);
  void drain_retired();
  KernelError device_error(const char* what) const;

  mq_ctx* ctx_ = nullptr;
  void* stream_ = nullptr;
  std::string init_error_;
  bool packed_weights_;
  bool int8_;
  std::unique_ptr<GpuPackedWeights> packed_;
  mutable std::mutex mu_;
  std::map<std::string, DeviceTensor> storage_;
  std::map<std::string, KernelResult> executions_;
  MemoryLedger memory_;
  // buffers replaced while queued Kernels may still read them: freed once
  // the stream has drained past them
  std::vector<float*> retired_;
  uint64_t retired_bytes_ = 0;
  // scratch for Kernel-internal temporaries (a transposed activation, a
  // broadcast product), grown on demand
  float* scratch_ = nullptr;
  uint64_t scratch_count_ = 0;
  std::atomic<uint64_t> ordinal_{0};
  uint64_t workspace_ordinal_ = 0;
  bool profile_on_ = false;
  std::map<std::string, std::pair<uint64_t, double>> profile_;
  mutable std::mutex obs_mu_;
  mutable std::vector<KernelObservation> observations_;
};

}  // namespace magnetar
