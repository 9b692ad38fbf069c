// C surface of the GpuExecutor (include/magnetar_executor.h).
#include <cstring>
#include <mutex>
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

int copy_text(const std::string& s, char* out, size_t cap) {
  if (!out || cap == 0) return 0;
  size_t n = s.size() < cap - 1 ? s.size() : cap - 1;
  std::memcpy(out, s.data(), n);
  out[n] = '\0';
  return static_cast<int>(n);
}

bool make_tensor(const uint64_t* shape, uint32_t rank, const float* data, magnetar::HostTensor& t) {
  if ((!shape && rank) || rank > 8) return false;
  uint64_t count = 1;
  t.shape.assign(shape, shape + rank);
  for (uint32_t i = 0; i < rank; ++i) count *= shape[i];
  if (count && !data) return false;
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
                       mg_executor** out) {
  if (!out) return fail(nullptr, MG_ERR_ARGUMENT, "mg_executor_create: null out pointer");
  *out = nullptr;
  auto* e = new mg_executor();
  e->ex = std::make_unique<magnetar::GpuExecutor>(device, packed_weights != 0, int8_activations != 0,
                                                  memory_capacity);
  if (!e->ex->ready()) {
    std::string why = e->ex->init_error();
    delete e;
    return fail(nullptr, MG_ERR_DEVICE, why);
  }
  *out = e;
  return MG_OK;
}

void mg_executor_destroy(mg_executor* e) { delete e; }

const char* mg_executor_last_error(mg_executor* e) {
  if (!e) return g_create_error.c_str();
  std::lock_guard<std::mutex> lock(e->err_mu);
  return e->errors[std::this_thread::get_id()].c_str();
}

int mg_write_packed_weight_tensor(mg_executor* e, const char* id, uint32_t gguf_type, uint64_t stored_rows,
                                  uint64_t stored_cols, int transposed, const uint8_t* bytes, size_t len,
                                  int* stored) {
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
}

int mg_write_tensor(mg_executor* e, const char* id, const uint64_t* shape, uint32_t rank, const float* data) {
  magnetar::HostTensor t;
  if (!e || !id || !make_tensor(shape, rank, data, t)) return fail(e, MG_ERR_ARGUMENT, "bad tensor arguments");
  e->ex->write_tensor(id, std::move(t));
  return MG_OK;
}

int mg_write_tensor_admitted(mg_executor* e, const char* id, const uint64_t* shape, uint32_t rank,
                             const float* data) {
  magnetar::HostTensor t;
  if (!e || !id || !make_tensor(shape, rank, data, t)) return fail(e, MG_ERR_ARGUMENT, "bad tensor arguments");
  uint64_t bytes = t.data.size() * sizeof(float);
  if (!e->ex->write_tensor_admitted(id, std::move(t)))
    return fail(e, MG_MEMORY_DENIED,
                "memory admission denied for " + std::string(id) + ": " + std::to_string(bytes) + " bytes, " +
                    std::to_string(e->ex->memory().capacity() - e->ex->memory().used()) + " available");
  return MG_OK;
}

int mg_resident_shape(mg_executor* e, const char* id, uint64_t* shape, uint32_t* rank) {
  if (!e || !id || !rank) return fail(e, MG_ERR_ARGUMENT, "null argument");
  auto s = e->ex->resident_shape(id);
  if (!s) return fail(e, MG_UNKNOWN, "no resident tensor " + std::string(id));
  if (s->size() > *rank || (!shape && !s->empty())) return fail(e, MG_ERR_ARGUMENT, "shape capacity too small");
  for (size_t i = 0; i < s->size(); ++i) shape[i] = (*s)[i];
  *rank = static_cast<uint32_t>(s->size());
  return MG_OK;
}

int mg_read_tensor(mg_executor* e, const char* id, float* out, uint64_t count) {
  if (!e || !id) return fail(e, MG_ERR_ARGUMENT, "null argument");
  auto t = e->ex->read_tensor(id);
  if (!t) return fail(e, MG_UNKNOWN, "no tensor " + std::string(id));
  if (t->data.size() > count || (!out && !t->data.empty())) return fail(e, MG_ERR_ARGUMENT, "output too small");
  std::memcpy(out, t->data.data(), t->data.size() * sizeof(float));
  return MG_OK;
}

int mg_is_packed(mg_executor* e, const char* id) { return e && id && e->ex->is_packed(id) ? 1 : 0; }

int mg_read_tensor_value_is_opaque(mg_executor* e, const char* id) {
  return e && id && e->ex->read_tensor_value_is_opaque(id) ? 1 : 0;
}

int mg_release_tensor(mg_executor* e, const char* id, int* released) {
  if (!e || !id) return fail(e, MG_ERR_ARGUMENT, "null argument");
  bool r = e->ex->release_tensor(id);
  if (released) *released = r ? 1 : 0;
  return MG_OK;
}

int mg_submit_kernel(mg_executor* e, const char* kernel, const char* invocation_id, const char* const* inputs,
                     uint32_t n_inputs, const char* output, const mg_attribute* attributes, uint32_t n_attributes,
                     int64_t deadline_millis, char* handle, size_t handle_capacity) {
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
  std::string h = e->ex->submit_kernel(inv);
  if (h.size() + 1 > handle_capacity) return fail(e, MG_ERR_ARGUMENT, "handle capacity too small");
  copy_text(h, handle, handle_capacity);
  return MG_OK;
}

int mg_complete_kernel(mg_executor* e, const char* handle, int* kernel_error, char* reason, size_t reason_capacity) {
  if (!e || !handle || !kernel_error) return fail(e, MG_ERR_ARGUMENT, "null argument");
  magnetar::KernelResult r;
  if (!e->ex->complete_kernel(handle, &r))
    return fail(e, MG_UNKNOWN,
                "no Kernel execution is associated with this handle: it was never submitted, or has already been "
                "completed once");
  *kernel_error = r.succeeded ? MG_OK : static_cast<int>(r.error.kind);
  copy_text(r.error.reason, reason, reason_capacity);
  return MG_OK;
}

uint64_t mg_observation_count(mg_executor* e) { return e ? e->ex->observations().size() : 0; }

int mg_observation(mg_executor* e, uint64_t index, char* kind, size_t kind_capacity, char* kernel,
                   size_t kernel_capacity) {
  if (!e) return fail(e, MG_ERR_ARGUMENT, "null executor");
  auto obs = e->ex->observations();
  if (index >= obs.size()) return fail(e, MG_UNKNOWN, "observation index out of range");
  copy_text(obs[index].kind, kind, kind_capacity);
  copy_text(obs[index].kernel, kernel, kernel_capacity);
  return MG_OK;
}

uint32_t mg_kernel_advertisement_count(void) {
  return static_cast<uint32_t>(magnetar::gpu_kernel_advertisements().size());
}

const char* mg_kernel_advertisement_json(uint32_t index) {
  static std::once_flag once;
  static std::vector<std::string> texts;
  std::call_once(once, [] {
    for (const auto& a : magnetar::gpu_kernel_advertisements()) texts.push_back(advertisement_json(a));
  });
  return index < texts.size() ? texts[index].c_str() : nullptr;
}

uint64_t mg_materialization_count(mg_executor* e) { return e ? e->ex->materializations() : 0; }

uint64_t mg_memory_used(mg_executor* e) { return e ? e->ex->memory().used() : 0; }

}  // extern "C"
