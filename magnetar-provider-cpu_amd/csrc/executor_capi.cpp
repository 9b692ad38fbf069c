// C surface of the GpuExecutor (include/magnetar_executor.h). Every entry
// point is a function-try-block: nothing thrown inside (a host allocation
// sized by the caller, a container insert) crosses the C ABI.
#include <cstring>
#include <mutex>
#include <new>
#include <stdexcept>
#include <string>
#include <thread>
#include <unordered_map>

#include "executor.hpp"
#include "magnetar_executor.h"

struct mg_executor {
  std::unique_ptr<magnetar::GpuExecutor> ex;
  std::mutex err_mu;
  std::unordered_map<std::thread::id, std::string> errors;
};

namespace {

thread_local std::string g_create_error;

int fail(mg_executor* e, int code, const std::string& what) {
  if (e) {
    std::lock_guard<std::mutex> lock(e->err_mu);
    e->errors[std::this_thread::get_id()] = what;
  } else {
    g_create_error = what;
  }
  return code;
}

int fail_quietly(mg_executor* e, int code, const char* what) noexcept {
  try {
    return fail(e, code, what);
  } catch (...) {
    return code;
  }
}

#define MG_CATCH(e)                                                                              \
  catch (const std::bad_alloc&) {                                                                \
    return fail_quietly(e, MG_ERR_OOM, "out of host memory");                                    \
  }                                                                                              \
  catch (const std::length_error&) {                                                             \
    return fail_quietly(e, MG_ERR_OOM, "a host buffer of that size cannot be allocated");        \
  }                                                                                              \
  catch (const std::exception& x_) {                                                             \
    return fail_quietly(e, MG_ERR_ARGUMENT, x_.what());                                          \
  }                                                                                              \
  catch (...) {                                                                                  \
    return fail_quietly(e, MG_ERR_ARGUMENT, "unexpected exception");                             \
  }

int copy_text(const std::string& s, char* out, size_t cap) {
  if (!out || cap == 0) return 0;
  size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
  std::memcpy(out, s.data(), n);
  out[n] = '\0';
  return static_cast<int>(n);
}

// A HostTensor of `rank` dims; false for a malformed shape (rank above 8,
// an element count that overflows, null data for a non-empty tensor).
bool make_tensor(const uint64_t* shape, uint32_t rank, const float* data, magnetar::HostTensor& t) {
  if ((!shape && rank) || rank > 8) return false;
  uint64_t count = 1;
  for (uint32_t i = 0; i < rank; ++i) {
    if (shape[i] && count > UINT64_MAX / sizeof(float) / shape[i]) return false;
    count *= shape[i];
  }
  if (count && !data) return false;
  t.shape.assign(shape, shape + rank);
  t.data.assign(data, data + count);
  return true;
}

std::string advertisement_json(const magnetar::KernelAdvertisement& a) {
  auto list = [](const std::vector<std::string>& v) {
    std::string s = "[";
    for (size_t i = 0; i < v.size(); ++i) s += (i ? ",\"" : "\"") + v[i] + "\"";
    return s + "]";
  };
  std::string s = "{\"provider\":\"" + a.provider + "\",\"name\":\"" + a.name + "\",\"version\":\"" + a.version +
                  "\",\"operator\":\"" + a.operator_id + "\",\"family\":\"" + a.family +
                  "\",\"conformance_profile\":\"" + a.conformance_profile + "\",\"input_dtypes\":" +
                  list(a.input_dtypes) + ",\"output_dtypes\":" + list(a.output_dtypes) +
                  ",\"layouts\":" + list(a.layouts) + ",\"memory_classes\":" + list(a.memory_classes) +
                  ",\"devices\":" + list(a.devices) + ",\"cancellation\":\"" + a.cancellation + "\"";
  s += a.rank ? ",\"rank\":" + std::to_string(*a.rank) : ",\"rank\":null";
  return s + "}";
}

}  // namespace

extern "C" {

int mg_executor_create(int device, int packed_weights, int int8_activations, uint64_t memory_capacity,
                       mg_executor** out) try {
  if (!out) return fail(nullptr, MG_ERR_ARGUMENT, "mg_executor_create: null out pointer");
  *out = nullptr;
  auto e = std::make_unique<mg_executor>();
  e->ex = std::make_unique<magnetar::GpuExecutor>(device, packed_weights != 0, int8_activations != 0,
                                                  memory_capacity);
  if (!e->ex->ready()) return fail(nullptr, MG_ERR_DEVICE, e->ex->init_error());
  *out = e.release();
  return MG_OK;
} MG_CATCH(nullptr)

void mg_executor_destroy(mg_executor* e) { delete e; }

const char* mg_executor_last_error(mg_executor* e) {
  if (!e) return g_create_error.c_str();
  std::lock_guard<std::mutex> lock(e->err_mu);
  try {
    return e->errors[std::this_thread::get_id()].c_str();
  } catch (...) {
    return "out of host memory";
  }
}

int mg_write_packed_weight_tensor(mg_executor* e, const char* id, uint32_t gguf_type, uint64_t stored_rows,
                                  uint64_t stored_cols, int transposed, const uint8_t* bytes, size_t len,
                                  int* stored) try {
  if (!e || !id || !stored || (len && !bytes)) return fail(e, MG_ERR_ARGUMENT, "null argument");
  magnetar::PackedWeight w;
  w.format = gguf_type;
  w.stored_rows = stored_rows;
  w.stored_cols = stored_cols;
  w.transposed = transposed != 0;
  w.bytes.assign(bytes, bytes + len);
  std::string why;
  *stored = e->ex->write_packed_weight_tensor(id, w, &why) == magnetar::PackedWeightWrite::Stored ? 1 : 0;
  if (!*stored) fail(e, MG_OK, why);
  return MG_OK;
} MG_CATCH(e)

int mg_write_tensor(mg_executor* e, const char* id, const uint64_t* shape, uint32_t rank, const float* data) try {
  // the tensor is built (and its host copy allocated) before the executor
  // is looked at: a shape too large to hold fails here as MG_ERR_OOM
  magnetar::HostTensor t;
  if (!make_tensor(shape, rank, data, t)) return fail(e, MG_ERR_ARGUMENT, "bad tensor arguments");
  if (!e || !id) return fail(e, MG_ERR_ARGUMENT, "null argument");
  std::string why;
  if (!e->ex->write_tensor(id, t, &why)) return fail(e, MG_ERR_DEVICE, why);
  return MG_OK;
} MG_CATCH(e)

int mg_write_tensor_admitted(mg_executor* e, const char* id, const uint64_t* shape, uint32_t rank,
                             const float* data) try {
  magnetar::HostTensor t;
  if (!e || !id || !make_tensor(shape, rank, data, t)) return fail(e, MG_ERR_ARGUMENT, "bad tensor arguments");
  bool denied = false;
  std::string why;
  if (!e->ex->write_tensor_admitted(id, t, &denied, &why)) return fail(e, denied ? MG_MEMORY_DENIED : MG_ERR_DEVICE, why);
  return MG_OK;
} MG_CATCH(e)

int mg_write_tensor_value(mg_executor* e, const char* id, int opaque, const uint64_t* shape, uint32_t rank,
                          const float* data) try {
  if (!e || !id) return fail(e, MG_ERR_ARGUMENT, "null argument");
  std::string why;
  if (opaque) return e->ex->write_tensor_value(id, nullptr, &why) ? MG_OK : fail(e, MG_ERR_DEVICE, why);
  magnetar::HostTensor t;
  if (!make_tensor(shape, rank, data, t)) return fail(e, MG_ERR_ARGUMENT, "bad tensor arguments");
  if (!e->ex->write_tensor_value(id, &t, &why)) return fail(e, MG_ERR_DEVICE, why);
  return MG_OK;
} MG_CATCH(e)

int mg_write_tensor_value_admitted(mg_executor* e, const char* id, int opaque, const uint64_t* shape, uint32_t rank,
                                   const float* data) try {
  if (!e || !id) return fail(e, MG_ERR_ARGUMENT, "null argument");
  bool denied = false;
  std::string why;
  if (opaque) return e->ex->write_tensor_value_admitted(id, nullptr, &denied, &why) ? MG_OK : fail(e, MG_ERR_DEVICE, why);
  magnetar::HostTensor t;
  if (!make_tensor(shape, rank, data, t)) return fail(e, MG_ERR_ARGUMENT, "bad tensor arguments");
  if (!e->ex->write_tensor_value_admitted(id, &t, &denied, &why))
    return fail(e, denied ? MG_MEMORY_DENIED : MG_ERR_DEVICE, why);
  return MG_OK;
} MG_CATCH(e)

int mg_copy_tensor_admitted(mg_executor* e, const char* from, const char* to) try {
  if (!e || !from || !to) return fail(e, MG_ERR_ARGUMENT, "null argument");
  bool denied = false;
  std::string why;
  if (!e->ex->copy_tensor_admitted(from, to, &denied, &why)) return fail(e, denied ? MG_MEMORY_DENIED : MG_ERR_DEVICE, why);
  return MG_OK;
} MG_CATCH(e)

int mg_write_zeroed_kv_store(mg_executor* e, const char* id, const uint64_t* shape, uint32_t rank, uint32_t precision,
                             uint64_t head_dimension, uint64_t exact_rows, int* created) try {
  if (!e || !id || !created || (rank && !shape)) return fail(e, MG_ERR_ARGUMENT, "null argument");
  std::vector<uint64_t> s(shape, shape + rank);
  std::string why;
  const auto p = precision == MG_KV_F32 ? magnetar::KvStorePrecision::F32 : magnetar::KvStorePrecision::TurboQuant;
  *created = e->ex->write_zeroed_kv_store(id, s, p, head_dimension, exact_rows, &why) ? 1 : 0;
  if (!*created) fail(e, MG_OK, why);
  return MG_OK;
} MG_CATCH(e)

int mg_allocate_workspace(mg_executor* e, uint64_t bytes, char* allocation, size_t capacity) try {
  if (!e || !allocation) return fail(e, MG_ERR_ARGUMENT, "null argument");
  auto a = e->ex->allocate_workspace(bytes);
  if (!a)
    return fail(e, MG_MEMORY_DENIED, "memory admission denied for a workspace of " + std::to_string(bytes) + " bytes");
  if (a->size() + 1 > capacity) {
    e->ex->release_workspace(*a);
    return fail(e, MG_ERR_ARGUMENT, "allocation id capacity too small");
  }
  copy_text(*a, allocation, capacity);
  return MG_OK;
} MG_CATCH(e)

int mg_release_workspace(mg_executor* e, const char* allocation) try {
  if (!e || !allocation) return fail(e, MG_ERR_ARGUMENT, "null argument");
  if (!e->ex->release_workspace(allocation)) return fail(e, MG_UNKNOWN, "no workspace " + std::string(allocation));
  return MG_OK;
} MG_CATCH(e)

int mg_resident_shape(mg_executor* e, const char* id, uint64_t* shape, uint32_t* rank) try {
  if (!e || !id || !rank) return fail(e, MG_ERR_ARGUMENT, "null argument");
  auto s = e->ex->resident_shape(id);
  if (!s) return fail(e, MG_UNKNOWN, "no resident tensor " + std::string(id));
  if (s->size() > *rank || (!shape && !s->empty())) return fail(e, MG_ERR_ARGUMENT, "shape capacity too small");
  for (size_t i = 0; i < s->size(); ++i) shape[i] = (*s)[i];
  *rank = static_cast<uint32_t>(s->size());
  return MG_OK;
} MG_CATCH(e)

int mg_read_tensor(mg_executor* e, const char* id, float* out, uint64_t count) try {
  if (!e || !id) return fail(e, MG_ERR_ARGUMENT, "null argument");
  auto s = e->ex->resident_shape(id);
  if (!s) return fail(e, MG_UNKNOWN, "no tensor " + std::string(id));
  uint64_t need = 1;
  for (uint64_t d : *s) need *= d;
  if (need > count || (!out && need)) return fail(e, MG_ERR_ARGUMENT, "output too small");
  auto t = e->ex->read_tensor(id);
  if (!t) return fail(e, MG_ERR_DEVICE, "reading " + std::string(id) + " back failed");
  if (t->data.size() > count) return fail(e, MG_ERR_ARGUMENT, "output too small");
  if (!t->data.empty()) std::memcpy(out, t->data.data(), t->data.size() * sizeof(float));
  return MG_OK;
} MG_CATCH(e)

int mg_is_packed(mg_executor* e, const char* id) try {
  return e && id && e->ex->is_packed(id) ? 1 : 0;
} catch (...) {
  return 0;
}

int mg_read_tensor_value_is_opaque(mg_executor* e, const char* id) try {
  return e && id && e->ex->read_tensor_value_is_opaque(id) ? 1 : 0;
} catch (...) {
  return 0;
}

int mg_release_tensor(mg_executor* e, const char* id, int* released) try {
  if (!e || !id) return fail(e, MG_ERR_ARGUMENT, "null argument");
  bool r = e->ex->release_tensor(id);
  if (released) *released = r ? 1 : 0;
  return MG_OK;
} MG_CATCH(e)

int mg_release_admitted_tensor(mg_executor* e, const char* id, int* released) try {
  if (!e || !id) return fail(e, MG_ERR_ARGUMENT, "null argument");
  bool r = e->ex->release_admitted_tensor(id);
  if (released) *released = r ? 1 : 0;
  return MG_OK;
} MG_CATCH(e)

int mg_submit_kernel(mg_executor* e, const char* kernel, const char* invocation_id, const char* const* inputs,
                     uint32_t n_inputs, const char* output, const mg_attribute* attributes, uint32_t n_attributes,
                     int64_t deadline_millis, char* handle, size_t handle_capacity) try {
  if (!e || !kernel || !invocation_id || (n_inputs && !inputs) || (n_attributes && !attributes) || !handle)
    return fail(e, MG_ERR_ARGUMENT, "null argument");
  magnetar::KernelInvocation inv;
  inv.kernel = kernel;
  inv.id = invocation_id;
  for (uint32_t i = 0; i < n_inputs; ++i) {
    if (!inputs[i]) return fail(e, MG_ERR_ARGUMENT, "null input id");
    inv.inputs.emplace_back(inputs[i]);
  }
  if (output) inv.outputs.emplace_back(output);
  for (uint32_t i = 0; i < n_attributes; ++i) {
    if (!attributes[i].name || !attributes[i].value) return fail(e, MG_ERR_ARGUMENT, "null attribute");
    inv.attributes[attributes[i].name] = attributes[i].value;
  }
  if (deadline_millis >= 0) inv.deadline_millis = static_cast<uint64_t>(deadline_millis);
  // the handle must fit before anything runs: a submission is never left
  // without a handle to complete it
  // ("<provider>:<invocation>:<ordinal>", the ordinal at most 20 digits)
  if (std::strlen(magnetar::kGpuProviderName) + inv.id.size() + 2 + 20 + 1 > handle_capacity)
    return fail(e, MG_ERR_ARGUMENT, "handle capacity too small");
  std::string h = e->ex->submit_kernel(inv);
  copy_text(h, handle, handle_capacity);
  return MG_OK;
} MG_CATCH(e)

int mg_complete_kernel(mg_executor* e, const char* handle, int* kernel_error, char* reason,
                       size_t reason_capacity) try {
  if (!e || !handle || !kernel_error) return fail(e, MG_ERR_ARGUMENT, "null argument");
  magnetar::KernelResult r;
  if (!e->ex->complete_kernel(handle, &r))
    return fail(e, MG_UNKNOWN,
                "no Kernel execution is associated with this handle: it was never submitted, or has already been "
                "completed once");
  *kernel_error = r.succeeded ? MG_OK : static_cast<int>(r.error.kind);
  copy_text(r.error.reason, reason, reason_capacity);
  return MG_OK;
} MG_CATCH(e)

int mg_synchronize(mg_executor* e) try {
  if (!e) return fail(e, MG_ERR_ARGUMENT, "null executor");
  if (!e->ex->synchronize()) return fail(e, MG_ERR_DEVICE, "the device reported an error");
  return MG_OK;
} MG_CATCH(e)

uint64_t mg_observation_count(mg_executor* e) try {
  return e ? e->ex->observations().size() : 0;
} catch (...) {
  return 0;
}

int mg_observation(mg_executor* e, uint64_t index, char* kind, size_t kind_capacity, char* kernel,
                   size_t kernel_capacity) try {
  if (!e) return fail(e, MG_ERR_ARGUMENT, "null executor");
  auto obs = e->ex->observations();
  if (index >= obs.size()) return fail(e, MG_UNKNOWN, "observation index out of range");
  copy_text(obs[index].kind, kind, kind_capacity);
  copy_text(obs[index].kernel, kernel, kernel_capacity);
  return MG_OK;
} MG_CATCH(e)

uint32_t mg_kernel_advertisement_count(void) try {
  return static_cast<uint32_t>(magnetar::gpu_kernel_advertisements().size());
} catch (...) {
  return 0;
}

const char* mg_kernel_advertisement_json(uint32_t index) try {
  static std::once_flag once;
  static std::vector<std::string> texts;
  std::call_once(once, [] {
    for (const auto& a : magnetar::gpu_kernel_advertisements()) texts.push_back(advertisement_json(a));
  });
  return index < texts.size() ? texts[index].c_str() : nullptr;
} catch (...) {
  return nullptr;
}

uint64_t mg_materialization_count(mg_executor* e) { return e ? e->ex->materializations() : 0; }

uint64_t mg_memory_used(mg_executor* e) { return e ? e->ex->memory_used() : 0; }

uint32_t mg_profile_count(mg_executor* e) try {
  return e ? static_cast<uint32_t>(e->ex->profile().size()) : 0;
} catch (...) {
  return 0;
}

int mg_profile_entry(mg_executor* e, uint32_t index, char* kernel, size_t kernel_capacity, uint64_t* calls,
                     double* seconds) try {
  if (!e || !calls || !seconds) return fail(e, MG_ERR_ARGUMENT, "null argument");
  auto rows = e->ex->profile();
  if (index >= rows.size()) return fail(e, MG_UNKNOWN, "profile index out of range");
  copy_text(rows[index].first, kernel, kernel_capacity);
  *calls = rows[index].second.first;
  *seconds = rows[index].second.second;
  return MG_OK;
} MG_CATCH(e)

}  // extern "C"
