/*
 * magnetar_executor: the Provider side of the GPU path (libmagnetar_executor.so),
 * a C surface over the C++ GpuExecutor, which itself calls only
 * libmagnetar_gpu (magnetar_gpu.h).
 *
 * Resource ids are NUL-terminated strings (TensorResourceId). Tensors are
 * row-major f32 with an explicit shape (HostTensor) on the way in and out;
 * inside the executor they are resident in the GPU's HBM, and every Kernel
 * reads and writes device memory. Every call returns an MG_* status;
 * mg_executor_last_error() holds the reason text. Nothing thrown inside
 * crosses this ABI.
 */
#ifndef MAGNETAR_EXECUTOR_H
#define MAGNETAR_EXECUTOR_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; MG_KERNEL_* carry the KernelError variant of a completed
 * invocation (external magnetar-kernel type). */
#define MG_OK 0
#define MG_KERNEL_EXECUTION_FAILED 1
#define MG_KERNEL_DTYPE_UNSUPPORTED 2
#define MG_KERNEL_ATTRIBUTE_UNSUPPORTED 3
#define MG_KERNEL_NOT_FOUND 4
#define MG_KERNEL_TIMEOUT 5
#define MG_MEMORY_DENIED 6  /* MemoryError: admission denied */
#define MG_UNKNOWN 7        /* unknown resource id or execution handle */
#define MG_ERR_ARGUMENT 8
#define MG_ERR_DEVICE 9     /* the GPU context could not be created, or a device copy failed */
#define MG_ERR_OOM 10       /* host memory for the call could not be allocated */

/* KvStorePrecision: f32 stores run on the GPU; the TurboQuant precisions
 * (any other value) are declined. */
#define MG_KV_F32 0u

typedef struct mg_executor mg_executor;

/* An executor on HIP device `device` (`NativeCpuExecutor::with_settings`,
 * src/native/mod.rs:525-544): packed_weights = 0 declines every packed
 * weight (MAGNETAR_CPU_PACKED_WEIGHTS=0), int8_activations selects the
 * reference's default int8 activations (MAGNETAR_CPU_INT8_ACTIVATIONS),
 * memory_capacity bounds admitted bytes (the MemoryManager ledger).
 * MAGNETAR_GPU_PROFILE=1 in the environment times every Kernel to its
 * completion on the device and prints the totals when the executor is
 * destroyed (MAGNETAR_CPU_PROFILE, src/native/mod.rs:29-31, 472-497).
 * Records ProviderRegistered and DeviceDetected observations
 * (`Provider::initialize`, src/native/mod.rs:928-938). */
int mg_executor_create(int device, int packed_weights, int int8_activations,
                       uint64_t memory_capacity, mg_executor **out);
void mg_executor_destroy(mg_executor *ex);
const char *mg_executor_last_error(mg_executor *ex);

/* `write_packed_weight_tensor` (src/native/mod.rs:638-653): *stored = 1
 * (PackedWeightWrite::Stored) or 0 (Declined: a format without a GPU path,
 * packed weights disabled, or device bytes the memory ledger cannot
 * admit). Untransposed weights and tables are stored: matmuls read them
 * by the reference's orientation rule, embeddings gather their rows. */
int mg_write_packed_weight_tensor(mg_executor *ex, const char *id, uint32_t gguf_type,
                                  uint64_t stored_rows, uint64_t stored_cols,
                                  int transposed, const uint8_t *bytes, size_t len,
                                  int *stored);

/* `write_tensor` (src/native/mod.rs:629-636): copied into device memory;
 * forgets a packed weight of the same id. */
int mg_write_tensor(mg_executor *ex, const char *id, const uint64_t *shape,
                    uint32_t rank, const float *data);

/* `write_tensor_admitted` (src/native/mod.rs:672-694): MG_MEMORY_DENIED
 * leaves storage and any packed weight unchanged. */
int mg_write_tensor_admitted(mg_executor *ex, const char *id, const uint64_t *shape,
                             uint32_t rank, const float *data);

/* `write_tensor_value` / `write_tensor_value_admitted`
 * (src/native/mod.rs:708-745; src/lib.rs:1811-1846): opaque != 0 writes
 * back the Opaque value `read_tensor_value` answers, which stores nothing
 * (a packed weight stays resident); otherwise a Host value of the given
 * shape replaces the id's contents, a packed weight included. */
int mg_write_tensor_value(mg_executor *ex, const char *id, int opaque, const uint64_t *shape,
                          uint32_t rank, const float *data);
int mg_write_tensor_value_admitted(mg_executor *ex, const char *id, int opaque,
                                   const uint64_t *shape, uint32_t rank, const float *data);

/* `copy_tensor_admitted` (src/native/mod.rs:746-766; src/lib.rs:1760-1809):
 * a device copy of `from` (a tensor, or a packed weight's logical values)
 * under `to`, admitted first; it replaces whatever `to` held, a packed
 * weight included. MG_MEMORY_DENIED for a denied admission or a missing
 * source ("source resource '<from>' not found"). */
int mg_copy_tensor_admitted(mg_executor *ex, const char *from, const char *to);

/* `write_zeroed_kv_store(_with_exact_head)` (src/native/mod.rs:767-799;
 * src/lib.rs:1633-1690): a zeroed f32 [capacity, width] store replacing
 * whatever `id` held; *created = 0 for a shape that is not [capacity,
 * whole heads of head_dimension] or a precision other than MG_KV_F32.
 * exact_rows matters only to the TurboQuant precisions. */
int mg_write_zeroed_kv_store(mg_executor *ex, const char *id, const uint64_t *shape,
                             uint32_t rank, uint32_t precision, uint64_t head_dimension,
                             uint64_t exact_rows, int *created);

/* `allocate_workspace` (src/native/mod.rs:800-806; src/lib.rs:2100-2121):
 * admits `bytes` of temporary workspace and writes its allocation id;
 * mg_release_workspace returns it to the ledger. */
int mg_allocate_workspace(mg_executor *ex, uint64_t bytes, char *allocation, size_t capacity);
int mg_release_workspace(mg_executor *ex, const char *allocation);

/* `resident_shape` (src/native/mod.rs:704-706): *rank in = capacity of
 * `shape`, out = the rank. A packed weight reports its logical shape. */
int mg_resident_shape(mg_executor *ex, const char *id, uint64_t *shape, uint32_t *rank);

/* `read_tensor` (src/lib.rs:1615-1620): the f32 values copied back after
 * every queued Kernel; a packed weight is materialized (dequantized,
 * logical layout). `count` = capacity of out. */
int mg_read_tensor(mg_executor *ex, const char *id, float *out, uint64_t count);

/* `is_packed` (src/native/mod.rs:554-557); `read_tensor_value` answers
 * Opaque for every resident id (src/native/mod.rs:695-702). */
int mg_is_packed(mg_executor *ex, const char *id);
int mg_read_tensor_value_is_opaque(mg_executor *ex, const char *id);

/* `release_tensor` (src/native/mod.rs:655-660): *released = 1 if the id
 * held a tensor or a packed weight. `release_admitted_tensor`
 * (src/native/mod.rs:662-670; src/lib.rs:1699-1711) also returns the
 * ledger's allocation for the id. */
int mg_release_tensor(mg_executor *ex, const char *id, int *released);
int mg_release_admitted_tensor(mg_executor *ex, const char *id, int *released);

/* One invocation attribute, as text: booleans "true"/"false", integers and
 * floats in decimal, dtype names ("f32", "f16", ...) and strings as is. */
typedef struct {
  const char *name;
  const char *value;
} mg_attribute;

/* `submit_kernel` (src/native/mod.rs:598-620, src/lib.rs:2301-2330):
 * validates the invocation, admits its output, enqueues its kernels on the
 * device and stores its KernelResult under the returned handle text
 * ("<provider>:<invocation>:<n>"; handle_capacity is checked before
 * anything runs). deadline_millis < 0: none; 0 fails with KernelTimeout
 * before dispatch. Kernels: matmul, matmul-bias, matmul-residual (input 1
 * a packed weight), embedding (input 0 a packed table), rmsnorm, rope,
 * kv-write, attention, silu-mul, add, residual-add (src/lib.rs:2528-3058);
 * attributes without a GPU path fail with KernelAttributeUnsupported. */
int mg_submit_kernel(mg_executor *ex, const char *kernel, const char *invocation_id,
                     const char *const *inputs, uint32_t n_inputs, const char *output,
                     const mg_attribute *attributes, uint32_t n_attributes,
                     int64_t deadline_millis, char *handle, size_t handle_capacity);

/* `complete_kernel` (src/lib.rs:2337-2356): consumes the stored result once;
 * MG_UNKNOWN for a handle never submitted or already completed. On success
 * *kernel_error is MG_OK or the KernelError variant, with its reason. */
int mg_complete_kernel(mg_executor *ex, const char *handle, int *kernel_error,
                       char *reason, size_t reason_capacity);

/* Waits for every Kernel queued so far. */
int mg_synchronize(mg_executor *ex);

/* Observation log (`observations`, src/lib.rs:1848-1868), kind text such as
 * "KernelDispatchStarted", "KernelDispatchCompleted", "KernelDispatchFailed",
 * "KernelTimeout", "KernelMemoryFeasibilityFailed". */
uint64_t mg_observation_count(mg_executor *ex);
int mg_observation(mg_executor *ex, uint64_t index, char *kind, size_t kind_capacity,
                   char *kernel, size_t kernel_capacity);

/* Kernel advertisements (`native_cpu_kernel_advertisements`,
 * src/native/mod.rs:847-864) as JSON text, one per index. */
uint32_t mg_kernel_advertisement_count(void);
const char *mg_kernel_advertisement_json(uint32_t index);

/* Packed weights materialized to f32 so far (the profile counter,
 * src/native/mod.rs:79-81). */
uint64_t mg_materialization_count(mg_executor *ex);

/* Bytes the memory ledger holds: admitted f32 tensors, Kernel outputs
 * (admitted before dispatch, src/lib.rs:2132-2285) and workspaces, plus
 * every packed weight's device footprint, which is admitted before its
 * upload replaces a weight of the same id (an upload the ledger cannot
 * hold is declined). */
uint64_t mg_memory_used(mg_executor *ex);

/* The per-Kernel profile under MAGNETAR_GPU_PROFILE=1 (empty otherwise),
 * most time first: Kernel name, calls, seconds. */
uint32_t mg_profile_count(mg_executor *ex);
int mg_profile_entry(mg_executor *ex, uint32_t index, char *kernel, size_t kernel_capacity,
                     uint64_t *calls, double *seconds);

#ifdef __cplusplus
}
#endif
#endif
