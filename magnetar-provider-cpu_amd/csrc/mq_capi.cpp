// C ABI of libmagnetar_gpu.so (declared in include/magnetar_gpu.h): device
// contexts, packed-weight upload into the tiled HBM layout, and the
// matmul / quantize / dequantize entry points. Shapes, buffer sizes and
// launch grids are validated here before any kernel runs.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <new>
#include <stdexcept>
#include <mutex>
#include <set>
#include <vector>
#include <string>
#include <thread>
#include <unordered_map>

#include "magnetar_gpu.h"
#include "mq_device.h"
#include "mq_launch.h"
#include "mq_layer.h"

namespace {

struct Weight {
  uint32_t type = 0;
  uint64_t rows = 0, cols = 0, nb = 0, rows_padded = 0;
  int transposed = 1;
  uint8_t* dev = nullptr;
  uint64_t dev_bytes = 0;
  // the prefill GEMM's f16 range factors (mq::weight_f16_factors of the
  // largest dequantized magnitude)
  float f16_up = 1.0f, f16_down = 1.0f;
};

mq::F16Range range(const Weight& w, const float* row_factors) {
  mq::F16Range r;
  r.row = row_factors;
  r.up = w.f16_up;
  r.down = w.f16_down;
  return r;
}

thread_local std::string g_create_error;

// The no-allocation matmul's temporaries (mq_matmul_noalloc_dev): one
// device array per GPU, resolved once per device by mq_create (with that
// device current) and shared by every call on the GPU. Host code uses only
// the resolved address: the array's name is a host-side stand-in.
constexpr size_t kScratchBytes = 32u << 20;
constexpr size_t kScratchCounterBytes = 64u << 10;  // split-K arrival counters, 16384 row blocks
static __device__ __align__(256) uint8_t scratch[kScratchBytes];
std::mutex g_scratch_mu;
std::map<int, uint8_t*> g_scratch_address;

}  // namespace

struct mq_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::mutex mu;
  std::unordered_map<uint64_t, Weight> weights;
  uint64_t next_handle = 1;
  // Activation workspace: stream-ordered on `ws_stream`; a call on another
  // stream first waits for the work already queued on it.
  void* ws = nullptr;
  size_t ws_bytes = 0;
  hipStream_t ws_stream = nullptr;
  hipEvent_t ws_event = nullptr;
  // Host-pointer staging for mq_matmul.
  void* io = nullptr;
  size_t io_bytes = 0;
  // Split-K arrival counters and partials of the decode GEMV: `sk_counters`
  // u32 counters at the front (zeroed at allocation; every launch leaves
  // them zero), partials after them.
  void* sk = nullptr;
  size_t sk_bytes = 0;
  uint64_t sk_counters = 0;
  int gemv_ksplit_override = 0;
  int gemv_narrow_override = -1;
  int gemv_splits_override = 0;
  int gemv_variant = 0;
  int gemm_variant = 0;
  // This device's scratch array (mq_matmul_noalloc_dev).
  uint8_t* scratch = nullptr;
  // Token ids of the embedding lookup (device copy).
  uint32_t* ids = nullptr;
  size_t ids_cap = 0;
  // Attention split-key partials (stream-ordered like the workspace).
  void* attn = nullptr;
  size_t attn_bytes = 0;
  // RoPE frequency tables by (base bits, dimension), computed on the host
  // with the platform's powf as the reference does.
  std::map<std::pair<uint32_t, uint64_t>, float*> rope_tables;
  std::mutex err_mu;
  std::unordered_map<std::thread::id, std::string> errors;
};

namespace {

int fail(mq_ctx* ctx, int code, const std::string& what) {
  if (ctx) {
    std::lock_guard<std::mutex> lock(ctx->err_mu);
    ctx->errors[std::this_thread::get_id()] = what;
  } else {
    g_create_error = what;
  }
  return code;
}

int hip_fail(mq_ctx* ctx, hipError_t e, const char* where) {
  return fail(ctx, e == hipErrorOutOfMemory ? MQ_ERR_OOM : MQ_ERR_HIP,
              std::string(where) + ": " + hipGetErrorString(e));
}

#define MQ_HIP(ctx, call)                                 \
  do {                                                    \
    hipError_t e_ = (call);                               \
    if (e_ != hipSuccess) return hip_fail(ctx, e_, #call); \
  } while (0)

// Records an error without letting a second exception escape (a failure
// to record the text still returns the code).
int fail_quietly(mq_ctx* ctx, int code, const char* what) noexcept {
  try {
    return fail(ctx, code, what);
  } catch (...) {
    return code;
  }
}

// The handlers of every entry point's function-try-block: nothing thrown
// inside the library (a host allocation sized by the caller, a container
// insert) crosses the C ABI.
#define MQ_CATCH(ctx)                                                                         \
  catch (const std::bad_alloc&) {                                                             \
    return fail_quietly(ctx, MQ_ERR_OOM, "out of host memory");                               \
  }                                                                                           \
  catch (const std::length_error&) {                                                          \
    return fail_quietly(ctx, MQ_ERR_OOM, "a host buffer of that size cannot be allocated");   \
  }                                                                                           \
  catch (const std::exception& e_) {                                                          \
    return fail_quietly(ctx, MQ_ERR_ARGUMENT, e_.what());                                     \
  }                                                                                           \
  catch (...) {                                                                               \
    return fail_quietly(ctx, MQ_ERR_ARGUMENT, "unexpected exception");                        \
  }

bool known_type(uint32_t type) {
  return type == MQ_TYPE_Q4_K || type == MQ_TYPE_IQ4_XS || mq::is_plane_format(static_cast<int>(type)) ||
         mq::is_grid_format(static_cast<int>(type));
}

bool plane_type(uint32_t type) { return mq::is_plane_format(static_cast<int>(type)); }
bool grid_type(uint32_t type) { return mq::is_grid_format(static_cast<int>(type)); }

// Devices whose copy of the IQ2 / IQ3 grid tables has been filled, and
// those whose tables hold only magnitude bytes below 128 (every GGUF grid
// does): the MFMA prefill reads the magnitudes as unsigned bytes, so other
// tables keep the 8-row GEMV prefill.
std::mutex g_grid_mu;
std::set<int> g_grid_devices;
std::set<int> g_grid_gemm_devices;

bool grids_ready(int device) {
  std::lock_guard<std::mutex> lock(g_grid_mu);
  return g_grid_devices.count(device) != 0;
}

bool grid_gemm_ready(int device) {
  std::lock_guard<std::mutex> lock(g_grid_mu);
  return g_grid_gemm_devices.count(device) != 0;
}

class DeviceGuard {
 public:
  explicit DeviceGuard(int device) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != device) (void)hipSetDevice(device);
    device_ = device;
  }
  ~DeviceGuard() {
    if (prev_ >= 0 && prev_ != device_) (void)hipSetDevice(prev_);
  }

 private:
  int prev_ = -1, device_ = 0;
};

// Makes `stream` the workspace's stream, ordering it after work queued on
// the previous one, and grows the workspace to `bytes`. Caller holds ctx->mu.
int order_stream(mq_ctx* ctx, hipStream_t stream) {
  if (ctx->ws_stream != stream) {
    MQ_HIP(ctx, hipEventRecord(ctx->ws_event, ctx->ws_stream));
    MQ_HIP(ctx, hipStreamWaitEvent(stream, ctx->ws_event, 0));
    ctx->ws_stream = stream;
  }
  return MQ_OK;
}

int acquire_workspace(mq_ctx* ctx, hipStream_t stream, size_t bytes) {
  int rc = order_stream(ctx, stream);
  if (rc) return rc;
  if (bytes <= ctx->ws_bytes) return MQ_OK;
  MQ_HIP(ctx, hipStreamSynchronize(stream));
  if (ctx->ws) MQ_HIP(ctx, hipFree(ctx->ws));
  ctx->ws = nullptr;
  ctx->ws_bytes = 0;
  size_t want = bytes < (1u << 20) ? (1u << 20) : bytes;
  MQ_HIP(ctx, hipMalloc(&ctx->ws, want));
  ctx->ws_bytes = want;
  return MQ_OK;
}

// Where one matmul's temporaries live: the context's growable buffers
// (fixed == nullptr), or the fixed scratch array of the no-allocation entry
// point, laid out as [split-K counters | split-K partials | workspace].
struct Scratch {
  uint8_t* fixed = nullptr;
  size_t bytes = 0;
  size_t used = kScratchCounterBytes;  // the next free byte past the counters
};

int scratch_overflow(mq_ctx* ctx, size_t need) {
  return fail(ctx, MQ_ERR_SHAPE, "this matmul needs " + std::to_string(need) +
                                     " bytes of temporaries, above the no-allocation entry point's " +
                                     std::to_string(kScratchBytes - kScratchCounterBytes));
}

// `bytes` of workspace: the context's (grown as needed), or the next free
// part of the fixed scratch. Caller holds ctx->mu.
int workspace(mq_ctx* ctx, hipStream_t stream, size_t bytes, Scratch* sc, void** out) {
  if (sc && sc->fixed) {
    const size_t at = (sc->used + 255) & ~static_cast<size_t>(255);
    if (at + bytes > sc->bytes) return scratch_overflow(ctx, at + bytes - kScratchCounterBytes);
    *out = sc->fixed + at;
    sc->used = at + bytes;
    return MQ_OK;
  }
  int rc = acquire_workspace(ctx, stream, bytes);
  if (rc) return rc;
  *out = ctx->ws;
  return MQ_OK;
}

// The GEMV's split-K buffers for `w` and m rows (ks == 1: none). Caller
// holds ctx->mu and has ordered `stream` (order_stream).
int acquire_splitk(mq_ctx* ctx, hipStream_t stream, const Weight& w, uint64_t m, mq::GemvSplitK& sk,
                   Scratch* sc = nullptr) {
  sk = mq::GemvSplitK{};
  sk.ks = ctx->gemv_ksplit_override > 0 ? ctx->gemv_ksplit_override : mq::gemv_default_ksplit(w.rows, w.nb);
  sk.narrow = ctx->gemv_narrow_override;
  if (plane_type(w.type)) {
    // the plane GEMV has no other form: its LDS staging must fit
    const int need = mq::gemv_planes_min_ksplit(w.nb, m);
    if (need > 16)
      return fail(ctx, MQ_DECLINED, "packed rows of " + std::to_string(w.cols) + " values exceed the decode GEMV");
    if (sk.ks < need) sk.ks = need;
  }
  if (sk.ks > 16) sk.ks = 16;
  if (static_cast<uint64_t>(sk.ks) > w.nb) sk.ks = static_cast<int>(w.nb);
  if (sk.ks <= 1) {
    sk.ks = 1;
    return MQ_OK;
  }
  const uint64_t blocks = (w.rows + 63) / 64;
  const size_t partials = static_cast<size_t>(sk.ks) * m * 2 * blocks * 64 * sizeof(float);
  if (sc && sc->fixed) {
    // the counters start at zero for this call whatever an earlier call
    // left there: cleared by a fill kernel, not a memset (graph-safe)
    if (blocks * sizeof(uint32_t) > kScratchCounterBytes) return scratch_overflow(ctx, blocks * sizeof(uint32_t));
    void* part = nullptr;
    int rc = workspace(ctx, stream, partials, sc, &part);
    if (rc) return rc;
    sk.counters = reinterpret_cast<uint32_t*>(sc->fixed);
    sk.partials = static_cast<float*>(part);
    mq::launch_fill(reinterpret_cast<float*>(sc->fixed), blocks, 0.0f, stream);
    return MQ_OK;
  }
  if (blocks > ctx->sk_counters || ctx->sk_counters * sizeof(uint32_t) + partials > ctx->sk_bytes) {
    // grow: the counter region keeps a fixed capacity between growths, so a
    // smaller weight's partials never land on another weight's counters
    MQ_HIP(ctx, hipStreamSynchronize(stream));
    if (ctx->sk) MQ_HIP(ctx, hipFree(ctx->sk));
    ctx->sk = nullptr;
    ctx->sk_bytes = 0;
    ctx->sk_counters = 0;
    const uint64_t cap = (blocks + 1023) / 1024 * 1024;
    const size_t want = cap * sizeof(uint32_t) + 16ull * 8 * 2 * cap * 64 * sizeof(float);
    MQ_HIP(ctx, hipMalloc(&ctx->sk, want));
    MQ_HIP(ctx, hipMemset(ctx->sk, 0, want));
    MQ_HIP(ctx, hipDeviceSynchronize());  // zeroed before any stream's kernel reads it
    ctx->sk_bytes = want;
    ctx->sk_counters = cap;
  }
  sk.counters = static_cast<uint32_t*>(ctx->sk);
  sk.partials = reinterpret_cast<float*>(static_cast<uint8_t*>(ctx->sk) + ctx->sk_counters * sizeof(uint32_t));
  return MQ_OK;
}

const Weight* find_weight(mq_ctx* ctx, uint64_t handle) {
  auto it = ctx->weights.find(handle);
  return it == ctx->weights.end() ? nullptr : &it->second;
}

// The reference's orientation rule (src/native/mod.rs:217-227): the stored
// rows are the output columns when the weight is stored transposed and not
// read transposed, or stored untransposed (a tied table) and read
// transposed; otherwise they are the input rows (the axpy product).
bool output_major(const Weight& w, uint32_t flags) {
  return (w.transposed != 0) != ((flags & MQ_TRANSPOSE_B) != 0);
}

uint64_t out_cols(const Weight& w, uint32_t flags) { return output_major(w, flags) ? w.rows : w.cols; }

int check_k(mq_ctx* ctx, const Weight& w, uint64_t k, uint32_t flags = 0) {
  if (!output_major(w, flags)) {
    if (k != w.rows)
      return fail(ctx, MQ_ERR_SHAPE,
                  "packed matmul: activations have " + std::to_string(k) + " columns, the weight " +
                      std::to_string(w.rows) + " stored rows");
    return MQ_OK;
  }
  if (k != w.cols || k % 32 != 0)
    return fail(ctx, MQ_ERR_SHAPE,
                "packed matmul: activations have " + std::to_string(k) + " columns, the weight's stored rows " +
                    std::to_string(w.cols));
  return MQ_OK;
}

size_t align256(size_t v) { return (v + 255) & ~static_cast<size_t>(255); }

int gemv_splits(mq_ctx* ctx, const Weight& w, uint64_t m, bool int8) {
  if (ctx->gemv_splits_override > 0) {
    int s = ctx->gemv_splits_override;
    return s > 16 ? 16 : s;
  }
  return mq::gemv_default_splits(w.rows, w.nb, m, int8 ? ctx->gemv_variant : 1);
}

constexpr uint64_t kGemvMaxRows = 8;
// Up to this many activation rows, and for rows shorter than kGemmMinK
// values, the matmul runs as decode-GEMV launches of 8 rows each: exact
// integer dots, where the f16 MFMA GEMM rounds every operand to 11 bits
// (a short row has too few terms for those roundings to average out
// against the 1e-3 * ||row||_inf output tolerance).
constexpr uint64_t kGemvChunkRows = 16;
constexpr uint64_t kGemmMinK = 512;

// The decode GEMV for m <= 8 rows. Caller holds ctx->mu and has validated
// the arguments.
int gemv_locked(mq_ctx* ctx, const Weight& w, const float* x, uint64_t m, uint64_t k, bool int8, float* y,
                hipStream_t stream, const float* addend, uint64_t addend_stride, Scratch* sc = nullptr) {
  mq::GemvSplitK sk;
  int rc = MQ_OK;
  if (sc) sc->used = kScratchCounterBytes;  // each launch sequence reuses the scratch, stream-ordered
  if (grid_type(w.type)) {
    int8_t* values = nullptr;
    float* scales = nullptr;
    if (int8) {
      const size_t vb = align256(m * k), sb = align256(m * k / 32 * 4), hb = align256(m * k / 32 * 8);
      void* ws = nullptr;
      rc = workspace(ctx, stream, vb + sb + hb, sc, &ws);
      if (rc) return rc;
      auto* base = static_cast<uint8_t*>(ws);
      values = reinterpret_cast<int8_t*>(base);
      scales = reinterpret_cast<float*>(base + vb);
      mq::launch_quantize_activations(x, m, k, values, scales, reinterpret_cast<int32_t*>(base + vb + sb), stream);
    }
    mq::launch_gemv_grid(static_cast<int>(w.type), w.dev, w.nb, w.rows, values, scales, x, m, int8 ? 1 : 0, y, addend,
                         addend_stride, stream);
    return MQ_OK;
  }
  if (int8) {
    rc = sc && sc->fixed ? MQ_OK : order_stream(ctx, stream);
    if (!rc) rc = acquire_splitk(ctx, stream, w, m, sk, sc);
    if (rc) return rc;
  }
  if (plane_type(w.type)) {
    if (int8)
      mq::launch_gemv_planes_int8(static_cast<int>(w.type), w.dev, w.rows, w.nb, k, nullptr, nullptr, nullptr, x, m,
                                  y, addend, addend_stride, ctx->gemv_splits_override, sk, stream);
    else
      mq::launch_gemv_planes_f32(static_cast<int>(w.type), w.dev, w.rows, w.nb, k, x, m, y, addend, addend_stride,
                                 ctx->gemv_splits_override, stream);
    return MQ_OK;
  }
  const bool fused = int8 && ctx->gemv_variant == 0 &&
                     mq::launch_gemv_fused(static_cast<int>(w.type), w.dev, w.rows, w.nb, x, m, y, addend,
                                           addend_stride, ctx->gemv_splits_override, sk, stream);
  if (fused) {
    // one launch: quantized into LDS and multiplied
  } else if (int8) {
    const size_t vb = align256(m * k), sb = align256(m * k / 32 * 4), hb = align256(m * k / 32 * 8);
    void* ws = nullptr;
    rc = workspace(ctx, stream, vb + sb + hb, sc, &ws);
    if (rc) return rc;
    auto* base = static_cast<uint8_t*>(ws);
    auto* values = reinterpret_cast<int8_t*>(base);
    auto* scales = reinterpret_cast<float*>(base + vb);
    auto* sums = reinterpret_cast<int32_t*>(base + vb + sb);
    mq::launch_quantize_activations(x, m, k, values, scales, sums, stream);
    mq::launch_gemv_int8(static_cast<int>(w.type), w.dev, w.rows, w.nb, values, scales, sums, m, y, addend,
                         addend_stride, ctx->gemv_splits_override, ctx->gemv_variant, sk, stream);
  } else {
    mq::launch_gemv_f32(static_cast<int>(w.type), w.dev, w.rows, w.nb, x, m, y, addend, addend_stride,
                        gemv_splits(ctx, w, m, false), stream);
  }
  return MQ_OK;
}

// Enqueues y = x . W^T [+ addend] on `stream`. Caller holds ctx->mu.
// addend_rows: 0 (no addend), 1 (one row broadcast) or m.
int matmul_locked(mq_ctx* ctx, const Weight& w, const float* x, uint64_t m, uint64_t k, uint32_t flags, float* y,
                  hipStream_t stream, const float* addend = nullptr, uint64_t addend_rows = 0,
                  Scratch* sc = nullptr) {
  if (flags & ~(MQ_INT8_ACTIVATIONS | MQ_TRANSPOSE_B)) return fail(ctx, MQ_ERR_ARGUMENT, "unknown matmul flag bits");
  int rc = check_k(ctx, w, k, flags);
  if (rc) return rc;
  if (m == 0) return MQ_OK;
  if (!x || !y) return fail(ctx, MQ_ERR_ARGUMENT, "null activation or output pointer");
  if (addend && addend_rows != 1 && addend_rows != m)
    return fail(ctx, MQ_ERR_SHAPE, "addend must hold 1 or " + std::to_string(m) + " rows, not " +
                                       std::to_string(addend_rows));
  const uint64_t n = out_cols(w, flags);
  const uint64_t addend_stride = addend && addend_rows == m && m > 1 ? n : 0;
  if (!addend) addend_rows = 0;
  const bool int8 = (flags & MQ_INT8_ACTIVATIONS) != 0;
  if (!output_major(w, flags)) {
    // input-major (axpy): f32 activations whatever the int8 setting, as
    // the reference's `packed_axpy` (src/native/mod.rs:154-194)
    const int ks = mq::axpy_ksplit(k, n);
    void* ws = nullptr;
    if (sc) sc->used = kScratchCounterBytes;
    rc = workspace(ctx, stream, align256(static_cast<size_t>(ks) * 4 * n * sizeof(float)), sc, &ws);
    if (rc) return rc;
    mq::launch_axpy(static_cast<int>(w.type), w.dev, w.nb, k, n, x, m, y, addend, addend_stride,
                    static_cast<float*>(ws), ks, stream);
  } else if (m <= kGemvChunkRows || k < kGemmMinK || (grid_type(w.type) && !grid_gemm_ready(ctx->device))) {
    for (uint64_t r0 = 0; r0 < m; r0 += kGemvMaxRows) {
      const uint64_t mc = m - r0 < kGemvMaxRows ? m - r0 : kGemvMaxRows;
      const float* ad = addend ? addend + (addend_stride ? r0 * w.rows : 0) : nullptr;
      rc = gemv_locked(ctx, w, x + r0 * k, mc, k, int8, y + r0 * w.rows, stream, ad, addend_stride, sc);
      if (rc) return rc;
    }
  } else {
    // workspace: the f16 activations and their row factors, then
    // (under-filled GEMMs) the split-K partials
    const int ks = mq::gemm_splits(static_cast<int>(w.type), w.rows, m, w.nb, k, ctx->gemm_variant);
    const size_t abytes = align256(m * k * 2) + align256(m * sizeof(float));
    const size_t pbytes = ks > 1 ? align256(static_cast<size_t>(ks) * m * w.rows * sizeof(float)) : 0;
    void* ws = nullptr;
    if (sc) sc->used = kScratchCounterBytes;
    rc = workspace(ctx, stream, abytes + pbytes, sc, &ws);
    if (rc) return rc;
    auto* a16 = static_cast<uint16_t*>(ws);
    auto* factors = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + align256(m * k * 2));
    float* part = ks > 1 ? reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + abytes) : nullptr;
    mq::launch_activations_f16(x, m, k, int8 ? 1 : 0, a16, factors, stream);
    mq::launch_gemm(static_cast<int>(w.type), w.dev, w.rows, w.nb, k, a16, m, y, addend, addend_stride,
                    ctx->gemm_variant, stream, range(w, factors), part);
  }
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
}

// The frequency table base^(-2p / dimension), p < dimension / 2, cached per
// (base, dimension) on the device. Caller holds ctx->mu.
int rope_table(mq_ctx* ctx, float base, uint64_t dimension, const float** out) {
  uint32_t base_bits;
  std::memcpy(&base_bits, &base, sizeof base_bits);
  const auto key = std::make_pair(base_bits, dimension);
  auto it = ctx->rope_tables.find(key);
  if (it == ctx->rope_tables.end()) {
    // the reference's table: base.powf(-2.0 * (pair as f32) / dimension as f32), in f32
    std::vector<float> table(dimension / 2);
    for (uint64_t p = 0; p < dimension / 2; ++p)
      table[p] = std::pow(base, -2.0f * static_cast<float>(p) / static_cast<float>(dimension));
    float* dev = nullptr;
    MQ_HIP(ctx, hipMalloc(&dev, table.size() * sizeof(float)));
    hipError_t e = hipMemcpy(dev, table.data(), table.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(dev);
      return hip_fail(ctx, e, "hipMemcpy(rope table)");
    }
    it = ctx->rope_tables.emplace(key, dev).first;
  }
  *out = it->second;
  return MQ_OK;
}

// Rust's `Display` of an f32 as the reference prints a token id: integral
// values without a fraction, NaN and inf by name.
std::string f32_text(float v) {
  if (std::isnan(v)) return "NaN";
  if (std::isinf(v)) return v > 0 ? "inf" : "-inf";
  if (v == std::floor(v) && std::fabs(v) < 1e15f) return std::to_string(static_cast<long long>(v));
  char buf[64];
  for (int prec = 1; prec <= 9; ++prec) {  // the shortest text that reads back as v
    std::snprintf(buf, sizeof buf, "%.*g", prec, static_cast<double>(v));
    if (std::strtof(buf, nullptr) == v) break;
  }
  return buf;
}

// Validates the ids as the reference does (src/native/mod.rs:399-404) and
// copies them to the device as u32. Caller holds ctx->mu.
int stage_ids(mq_ctx* ctx, const Weight& w, const float* ids, uint64_t count, hipStream_t stream) {
  const uint64_t vocab = w.transposed ? w.cols : w.rows;
  std::vector<uint32_t> host(count);
  for (uint64_t i = 0; i < count; ++i) {
    const float raw = ids[i];
    if (!(raw >= 0.0f) || raw != std::floor(raw) || static_cast<double>(raw) >= static_cast<double>(vocab))
      return fail(ctx, MQ_ERR_SHAPE,
                  "token id " + f32_text(raw) + " is not below the vocabulary size " + std::to_string(vocab));
    host[i] = static_cast<uint32_t>(raw);
  }
  if (count > ctx->ids_cap) {
    MQ_HIP(ctx, hipStreamSynchronize(stream));
    if (ctx->ids) MQ_HIP(ctx, hipFree(ctx->ids));
    ctx->ids = nullptr;
    ctx->ids_cap = 0;
    const size_t cap = count < 4096 ? 4096 : count;
    MQ_HIP(ctx, hipMalloc(&ctx->ids, cap * sizeof(uint32_t)));
    ctx->ids_cap = cap;
  }
  MQ_HIP(ctx, hipMemcpyAsync(ctx->ids, host.data(), count * sizeof(uint32_t), hipMemcpyHostToDevice, stream));
  MQ_HIP(ctx, hipStreamSynchronize(stream));  // `host` is released on return
  return MQ_OK;
}

}  // namespace

extern "C" {

const char* mq_version(void) { return "magnetar_gpu 0.1.0 (gfx950)"; }

int mq_create(int device, mq_ctx** out) try {
  if (!out) return fail(nullptr, MQ_ERR_ARGUMENT, "mq_create: null out pointer");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess) return hip_fail(nullptr, e, "hipGetDeviceCount");
  if (device < 0 || device >= count)
    return fail(nullptr, MQ_ERR_ARGUMENT, "mq_create: no HIP device " + std::to_string(device));
  DeviceGuard guard(device);
  auto* ctx = new (std::nothrow) mq_ctx();
  if (!ctx) return fail(nullptr, MQ_ERR_OOM, "mq_create: out of host memory");
  ctx->device = device;
  if ((e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking)) != hipSuccess ||
      (e = hipEventCreateWithFlags(&ctx->ws_event, hipEventDisableTiming)) != hipSuccess) {
    if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return hip_fail(nullptr, e, "mq_create");
  }
  ctx->ws_stream = ctx->stream;
  {
    // the scratch array's address on this device (the device is current)
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    auto it = g_scratch_address.find(device);
    if (it == g_scratch_address.end()) {
      void* p = nullptr;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) {
        (void)hipEventDestroy(ctx->ws_event);
        (void)hipStreamDestroy(ctx->stream);
        delete ctx;
        return hip_fail(nullptr, e != hipSuccess ? e : hipErrorInvalidSymbol, "hipGetSymbolAddress(scratch)");
      }
      it = g_scratch_address.emplace(device, static_cast<uint8_t*>(p)).first;
    }
    ctx->scratch = it->second;
  }
  if (const char* s = std::getenv("MQ_GEMV_SPLITS")) ctx->gemv_splits_override = std::atoi(s);
  if (const char* s = std::getenv("MQ_GEMV_KSPLIT")) ctx->gemv_ksplit_override = std::atoi(s);
  if (const char* s = std::getenv("MQ_GEMV_NARROW")) ctx->gemv_narrow_override = std::atoi(s);
  if (const char* s = std::getenv("MQ_GEMV_VARIANT")) ctx->gemv_variant = std::atoi(s);
  if (const char* s = std::getenv("MQ_GEMM_VARIANT")) ctx->gemm_variant = std::atoi(s);
  *out = ctx;
  return MQ_OK;
} MQ_CATCH(nullptr)

void mq_destroy(mq_ctx* ctx) {
  if (!ctx) return;
  DeviceGuard guard(ctx->device);
  (void)hipDeviceSynchronize();
  for (auto& kv : ctx->weights) (void)hipFree(kv.second.dev);
  if (ctx->ws) (void)hipFree(ctx->ws);
  if (ctx->io) (void)hipFree(ctx->io);
  if (ctx->sk) (void)hipFree(ctx->sk);
  if (ctx->attn) (void)hipFree(ctx->attn);
  if (ctx->ids) (void)hipFree(ctx->ids);
  for (auto& kv : ctx->rope_tables) (void)hipFree(kv.second);
  (void)hipEventDestroy(ctx->ws_event);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

const char* mq_last_error(mq_ctx* ctx) {
  if (!ctx) return g_create_error.c_str();
  std::lock_guard<std::mutex> lock(ctx->err_mu);
  try {
    return ctx->errors[std::this_thread::get_id()].c_str();
  } catch (...) {
    return "out of host memory";
  }
}

int mq_set_iq_grids(mq_ctx* ctx, const uint64_t* iq2xxs, const uint64_t* iq2xs, const uint64_t* iq2s,
                    const uint32_t* iq3xxs, const uint32_t* iq3s) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_set_iq_grids: null context");
  if (!iq2xxs || !iq2xs || !iq2s || !iq3xxs || !iq3s) return fail(ctx, MQ_ERR_ARGUMENT, "mq_set_iq_grids: null table");
  std::vector<uint8_t> tables(mq::kGridTableBytes);
  std::memcpy(tables.data() + mq::kGridIq2Xxs, iq2xxs, 256 * sizeof(uint64_t));
  std::memcpy(tables.data() + mq::kGridIq2Xs, iq2xs, 512 * sizeof(uint64_t));
  std::memcpy(tables.data() + mq::kGridIq2S, iq2s, 1024 * sizeof(uint64_t));
  std::memcpy(tables.data() + mq::kGridIq3Xxs, iq3xxs, 256 * sizeof(uint32_t));
  std::memcpy(tables.data() + mq::kGridIq3S, iq3s, 512 * sizeof(uint32_t));
  std::lock_guard<std::mutex> lock(ctx->mu);
  DeviceGuard guard(ctx->device);
  // every context's work on the device (any stream) may still read the
  // previous tables: the device copy is shared
  MQ_HIP(ctx, hipDeviceSynchronize());
  MQ_HIP(ctx, mq::grid_tables_upload(tables.data(), ctx->stream));
  bool small = true;
  for (uint8_t b : tables) small = small && b < 128;
  std::lock_guard<std::mutex> glock(g_grid_mu);
  g_grid_devices.insert(ctx->device);
  if (small)
    g_grid_gemm_devices.insert(ctx->device);
  else
    g_grid_gemm_devices.erase(ctx->device);
  return MQ_OK;
} MQ_CATCH(ctx)

// The largest magnitude among a weight's dequantized values (device
// dequantization in chunks of whole 8-row tiles, at most 8 Mi values each)
// and the prefill GEMM's f16 factors from it. Caller holds ctx->mu.
hipError_t set_f16_range(mq_ctx* ctx, Weight& w) {
  const int type = static_cast<int>(w.type);
  uint64_t chunk = (8ull << 20) / w.cols / 8 * 8;
  if (chunk < 8) chunk = 8;
  if (chunk > w.rows) chunk = w.rows;
  float* tmp = nullptr;
  uint32_t* amax = nullptr;
  hipError_t e = hipMalloc(&tmp, chunk * w.cols * sizeof(float));
  if (e != hipSuccess) return e;
  e = hipMalloc(&amax, sizeof(uint32_t));
  if (e != hipSuccess) {
    (void)hipFree(tmp);
    return e;
  }
  e = hipMemsetAsync(amax, 0, sizeof(uint32_t), ctx->stream);
  for (uint64_t r0 = 0; e == hipSuccess && r0 < w.rows; r0 += chunk) {
    const uint64_t rc = chunk < w.rows - r0 ? chunk : w.rows - r0;
    if (grid_type(w.type))
      mq::launch_dequantize_grid(type, w.dev + r0 * w.nb * static_cast<uint64_t>(mq::block_bytes_of(type)), rc, w.nb,
                                 0, tmp, ctx->stream);
    else if (plane_type(w.type))
      mq::launch_dequantize_planes(type, w.dev + r0 / 8 * w.nb * static_cast<uint64_t>(mq::tile_bytes(type)), rc,
                                   w.cols, w.nb, 0, tmp, ctx->stream);
    else
      mq::launch_dequantize(type, w.dev + r0 / 8 * w.nb * static_cast<uint64_t>(mq::tile_bytes(type)), rc, w.nb, 0,
                            tmp, ctx->stream);
    mq::launch_absmax(tmp, rc * w.cols, amax, ctx->stream);
    e = hipGetLastError();
  }
  uint32_t bits = 0;
  if (e == hipSuccess) e = hipMemcpyAsync(&bits, amax, sizeof bits, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(tmp);
  (void)hipFree(amax);
  if (e != hipSuccess) return e;
  float a;
  std::memcpy(&a, &bits, sizeof a);
  mq::weight_f16_factors(a, &w.f16_up, &w.f16_down);
  return hipSuccess;
}

int mq_weight_upload(mq_ctx* ctx, uint32_t gguf_type, uint64_t stored_rows, uint64_t stored_cols, int transposed,
                     const uint8_t* bytes, size_t len, uint64_t* handle) try {
  if (!ctx || !handle) return fail(ctx, MQ_ERR_ARGUMENT, "mq_weight_upload: null argument");
  *handle = 0;
  if (!known_type(gguf_type))
    return fail(ctx, MQ_DECLINED, "packed weight format " + std::to_string(gguf_type) + " has no GPU path");
  if (grid_type(gguf_type) && !grids_ready(ctx->device))
    return fail(ctx, MQ_DECLINED, "packed weight format " + std::to_string(gguf_type) +
                                      " needs the IQ2 / IQ3 grid tables (mq_set_iq_grids) on this device");
  const int type = static_cast<int>(gguf_type);
  const uint64_t be = static_cast<uint64_t>(mq::block_values(type)), bb = static_cast<uint64_t>(mq::block_bytes_of(type));
  if (stored_rows == 0 || stored_cols == 0 || stored_cols % be != 0)
    return fail(ctx, MQ_ERR_SHAPE,
                "packed weight: stored shape [" + std::to_string(stored_rows) + ", " + std::to_string(stored_cols) +
                    "] is not whole " + std::to_string(be) + "-value blocks");
  const uint64_t nb = (stored_cols + 255) / 256;
  if (stored_rows > (1ull << 32) || nb > (1ull << 24) || len != stored_rows * (stored_cols / be) * bb)
    return fail(ctx, MQ_ERR_SHAPE,
                "packed weight: " + std::to_string(len) + " bytes for " + std::to_string(stored_rows) + " x " +
                    std::to_string(stored_cols) + " values");
  if (!bytes) return fail(ctx, MQ_ERR_ARGUMENT, "mq_weight_upload: null bytes");
  std::lock_guard<std::mutex> lock(ctx->mu);
  DeviceGuard guard(ctx->device);
  Weight w;
  w.type = gguf_type;
  w.rows = stored_rows;
  w.cols = stored_cols;
  w.nb = nb;
  w.rows_padded = (stored_rows + 7) / 8 * 8;
  w.transposed = transposed;
  w.dev_bytes = grid_type(gguf_type) ? len : w.rows_padded / 8 * nb * static_cast<uint64_t>(mq::tile_bytes(type));
  if (grid_type(gguf_type)) {
    // the checkpoint's blocks as they are
    hipError_t e = hipMalloc(&w.dev, w.dev_bytes);
    if (e != hipSuccess) return hip_fail(ctx, e, "hipMalloc(weight)");
    e = hipMemcpyAsync(w.dev, bytes, len, hipMemcpyHostToDevice, ctx->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
    if (e == hipSuccess) e = set_f16_range(ctx, w);
    if (e != hipSuccess) {
      (void)hipFree(w.dev);
      return hip_fail(ctx, e, "mq_weight_upload");
    }
    *handle = ctx->next_handle++;
    ctx->weights.emplace(*handle, w);
    return MQ_OK;
  }
  uint8_t* raw = nullptr;
  hipError_t e = hipMalloc(&raw, len);
  if (e != hipSuccess) return hip_fail(ctx, e, "hipMalloc(staging)");
  e = hipMalloc(&w.dev, w.dev_bytes);
  if (e != hipSuccess) {
    (void)hipFree(raw);
    return hip_fail(ctx, e, "hipMalloc(weight)");
  }
  if ((e = hipMemcpyAsync(raw, bytes, len, hipMemcpyHostToDevice, ctx->stream)) == hipSuccess &&
      (e = hipMemsetAsync(w.dev, 0, w.dev_bytes, ctx->stream)) == hipSuccess) {
    if (plane_type(gguf_type))
      mq::launch_repack_planes(type, raw, stored_rows, stored_cols, nb, w.dev, ctx->stream);
    else
      mq::launch_repack(type, raw, stored_rows, nb, w.dev, ctx->stream);
    e = hipGetLastError();
    if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  }
  (void)hipFree(raw);
  if (e == hipSuccess) e = set_f16_range(ctx, w);
  if (e != hipSuccess) {
    (void)hipFree(w.dev);
    return hip_fail(ctx, e, "mq_weight_upload");
  }
  *handle = ctx->next_handle++;
  ctx->weights.emplace(*handle, w);
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_gemv_launch_shape(uint32_t gguf_type, uint64_t stored_rows, uint64_t stored_cols, uint64_t m, int waves,
                         int variant, int ksplit, mq_gemv_shape* out) try {
  if (!out) return fail(nullptr, MQ_ERR_ARGUMENT, "mq_gemv_launch_shape: null out pointer");
  if (gguf_type != MQ_TYPE_Q4_K && gguf_type != MQ_TYPE_IQ4_XS)
    return fail(nullptr, MQ_DECLINED, "mq_gemv_launch_shape: Q4_K and IQ4_XS only");
  if (stored_rows == 0 || stored_cols == 0 || stored_cols % 256 || m < 1 || m > 8 || variant < 0 || variant > 3)
    return fail(nullptr, MQ_ERR_SHAPE, "mq_gemv_launch_shape: no decode GEMV of this shape");
  const uint64_t nb = stored_cols / 256;
  mq::GemvSplitK sk;
  sk.ks = ksplit > 0 ? ksplit : mq::gemv_default_ksplit(stored_rows, nb);
  if (sk.ks > 16) sk.ks = 16;  // the context's bounds (acquire_splitk)
  if (static_cast<uint64_t>(sk.ks) > nb) sk.ks = static_cast<int>(nb);
  const mq::GemvShape g =
      mq::gemv_int8_shape(static_cast<int>(gguf_type), stored_rows, nb, m, waves, variant, sk);
  out->form = static_cast<uint32_t>(g.form);
  out->waves = static_cast<uint32_t>(g.waves);
  out->grid_x = g.grid_x;
  out->grid_y = g.grid_y;
  out->lds_bytes = g.lds;
  return MQ_OK;
} MQ_CATCH(nullptr)

int mq_weight_release(mq_ctx* ctx, uint64_t handle) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_weight_release: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  auto it = ctx->weights.find(handle);
  if (it == ctx->weights.end()) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  DeviceGuard guard(ctx->device);
  // Work already queued may still read the weight.
  MQ_HIP(ctx, hipDeviceSynchronize());
  MQ_HIP(ctx, hipFree(it->second.dev));
  ctx->weights.erase(it);
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_weight_info(mq_ctx* ctx, uint64_t handle, uint32_t* gguf_type, uint64_t* stored_rows, uint64_t* stored_cols,
                   int* transposed, uint64_t* device_bytes) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_weight_info: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  if (gguf_type) *gguf_type = w->type;
  if (stored_rows) *stored_rows = w->rows;
  if (stored_cols) *stored_cols = w->cols;
  if (transposed) *transposed = w->transposed;
  if (device_bytes) *device_bytes = w->dev_bytes;
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_matmul_dev(mq_ctx* ctx, uint64_t handle, const float* x_dev, uint64_t m, uint64_t k, uint32_t flags,
                  float* y_dev, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_dev: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  DeviceGuard guard(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  return matmul_locked(ctx, *w, x_dev, m, k, flags, y_dev, s);
} MQ_CATCH(ctx)

int mq_matmul_noalloc_dev(mq_ctx* ctx, uint64_t handle, const float* x_dev, uint64_t m, uint64_t k, uint32_t flags,
                          float* y_dev, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_noalloc_dev: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  if (!ctx->scratch) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_noalloc_dev: no scratch address on this device");
  DeviceGuard guard(ctx->device);
  Scratch sc;
  sc.fixed = ctx->scratch;
  sc.bytes = kScratchBytes;
  return matmul_locked(ctx, *w, x_dev, m, k, flags, y_dev, static_cast<hipStream_t>(stream), nullptr, 0, &sc);
} MQ_CATCH(ctx)

namespace {

// Host-pointer matmul: stage x (and the addend) in device memory, run on the
// context's stream, copy y back. Caller holds ctx->mu.
int matmul_host_locked(mq_ctx* ctx, const Weight& w, const float* x, uint64_t m, uint64_t k, uint32_t flags,
                       const float* addend, uint64_t addend_rows, float* y) {
  if (flags & ~(MQ_INT8_ACTIVATIONS | MQ_TRANSPOSE_B)) return fail(ctx, MQ_ERR_ARGUMENT, "unknown matmul flag bits");
  int rc = check_k(ctx, w, k, flags);
  if (rc) return rc;
  const uint64_t n = out_cols(w, flags);
  if (m == 0) return MQ_OK;
  if (!x || !y) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul: null host pointer");
  if (addend && addend_rows != 1 && addend_rows != m)
    return fail(ctx, MQ_ERR_SHAPE, "addend must hold 1 or " + std::to_string(m) + " rows, not " +
                                       std::to_string(addend_rows));
  const uint64_t add_count = addend ? addend_rows * n : 0;
  const size_t xb = align256(m * k * sizeof(float)), yb = align256(m * n * sizeof(float));
  const size_t ab = align256(add_count * sizeof(float));
  if (xb + yb + ab > ctx->io_bytes) {
    MQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
    if (ctx->io) MQ_HIP(ctx, hipFree(ctx->io));
    ctx->io = nullptr;
    ctx->io_bytes = 0;
    MQ_HIP(ctx, hipMalloc(&ctx->io, xb + yb + ab));
    ctx->io_bytes = xb + yb + ab;
  }
  auto* base = static_cast<uint8_t*>(ctx->io);
  auto* xd = reinterpret_cast<float*>(base);
  auto* yd = reinterpret_cast<float*>(base + xb);
  auto* ad = addend ? reinterpret_cast<float*>(base + xb + yb) : nullptr;
  MQ_HIP(ctx, hipMemcpyAsync(xd, x, m * k * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
  if (ad) MQ_HIP(ctx, hipMemcpyAsync(ad, addend, add_count * sizeof(float), hipMemcpyHostToDevice, ctx->stream));
  rc = matmul_locked(ctx, w, xd, m, k, flags, yd, ctx->stream, ad, addend_rows);
  if (rc) return rc;
  MQ_HIP(ctx, hipMemcpyAsync(y, yd, m * n * sizeof(float), hipMemcpyDeviceToHost, ctx->stream));
  MQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MQ_OK;
}

}  // namespace

int mq_matmul(mq_ctx* ctx, uint64_t handle, const float* x, uint64_t m, uint64_t k, uint32_t flags, float* y) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  DeviceGuard guard(ctx->device);
  return matmul_host_locked(ctx, *w, x, m, k, flags, nullptr, 0, y);
} MQ_CATCH(ctx)

int mq_matmul_add(mq_ctx* ctx, uint64_t handle, const float* x, uint64_t m, uint64_t k, uint32_t flags,
                  const float* addend, uint64_t addend_rows, float* y) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_add: null context");
  if (!addend) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_add: null addend");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  DeviceGuard guard(ctx->device);
  return matmul_host_locked(ctx, *w, x, m, k, flags, addend, addend_rows, y);
} MQ_CATCH(ctx)

int mq_matmul_add_dev(mq_ctx* ctx, uint64_t handle, const float* x_dev, uint64_t m, uint64_t k, uint32_t flags,
                      const float* addend_dev, uint64_t addend_rows, float* y_dev, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_add_dev: null context");
  if (!addend_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_add_dev: null addend");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  DeviceGuard guard(ctx->device);
  return matmul_locked(ctx, *w, x_dev, m, k, flags, y_dev, static_cast<hipStream_t>(stream), addend_dev, addend_rows);
} MQ_CATCH(ctx)

int mq_quantize_activations_dev(mq_ctx* ctx, const float* x_dev, uint64_t m, uint64_t k, int8_t* values_dev,
                                float* scales_dev, int32_t* sums_dev, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_quantize_activations_dev: null context");
  if (k % 32 != 0) return fail(ctx, MQ_ERR_SHAPE, "activation rows must hold whole 32-value blocks");
  if (m == 0) return MQ_OK;
  if (!x_dev || !values_dev || !scales_dev || !sums_dev)
    return fail(ctx, MQ_ERR_ARGUMENT, "mq_quantize_activations_dev: null pointer");
  DeviceGuard guard(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  mq::launch_quantize_activations(x_dev, m, k, values_dev, scales_dev, sums_dev, s);
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_matmul_prequantized_dev(mq_ctx* ctx, uint64_t handle, const int8_t* values_dev, const float* scales_dev,
                               const int32_t* sums_dev, uint64_t m, uint64_t k, float* y_dev, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_prequantized_dev: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  int rc = check_k(ctx, *w, k, w->transposed ? 0u : MQ_TRANSPOSE_B);  // stored rows are the outputs
  if (rc) return rc;
  if (m > kGemvMaxRows) return fail(ctx, MQ_ERR_SHAPE, "prequantized matmul takes at most 8 activation rows");
  if (m == 0) return MQ_OK;
  if (!values_dev || !scales_dev || !sums_dev || !y_dev)
    return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_prequantized_dev: null pointer");
  DeviceGuard guard(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (grid_type(w->type)) {
    mq::launch_gemv_grid(static_cast<int>(w->type), w->dev, w->nb, w->rows, values_dev, scales_dev, nullptr, m, 1,
                         y_dev, nullptr, 0, s);
    MQ_HIP(ctx, hipGetLastError());
    return MQ_OK;
  }
  mq::GemvSplitK sk;
  rc = order_stream(ctx, s);
  if (!rc) rc = acquire_splitk(ctx, s, *w, m, sk);
  if (rc) return rc;
  if (plane_type(w->type))
    mq::launch_gemv_planes_int8(static_cast<int>(w->type), w->dev, w->rows, w->nb, k, values_dev, scales_dev,
                                sums_dev, nullptr, m, y_dev, nullptr, 0, ctx->gemv_splits_override, sk, s);
  else
    mq::launch_gemv_int8(static_cast<int>(w->type), w->dev, w->rows, w->nb, values_dev, scales_dev, sums_dev, m,
                         y_dev, nullptr, 0, ctx->gemv_splits_override, ctx->gemv_variant, sk, s);
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_prepare_activations_f16_dev(mq_ctx* ctx, const float* x_dev, uint64_t m, uint64_t k, uint32_t flags,
                                   uint16_t* a16_dev, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_prepare_activations_f16_dev: null context");
  if (flags & ~MQ_INT8_ACTIVATIONS) return fail(ctx, MQ_ERR_ARGUMENT, "unknown flag bits");
  if (k % 32 != 0) return fail(ctx, MQ_ERR_SHAPE, "activation rows must hold whole 32-value blocks");
  if (m == 0) return MQ_OK;
  if (!x_dev || !a16_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_prepare_activations_f16_dev: null pointer");
  DeviceGuard guard(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  mq::launch_activations_f16(x_dev, m, k, (flags & MQ_INT8_ACTIVATIONS) ? 1 : 0, a16_dev,
                             reinterpret_cast<float*>(a16_dev + m * k), s);
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_matmul_f16_dev(mq_ctx* ctx, uint64_t handle, const uint16_t* a16_dev, uint64_t m, uint64_t k, float* y_dev,
                      void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_f16_dev: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  int rc = check_k(ctx, *w, k, w->transposed ? 0u : MQ_TRANSPOSE_B);  // stored rows are the outputs
  if (rc) return rc;
  if (m == 0) return MQ_OK;
  if (!a16_dev || !y_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_matmul_f16_dev: null pointer");
  if (grid_type(w->type) && !grid_gemm_ready(ctx->device))
    return fail(ctx, MQ_DECLINED, "the f16 MFMA GEMM of the IQ2 / IQ3 grid formats needs grid magnitudes below 128");
  DeviceGuard guard(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int ks = mq::gemm_splits(static_cast<int>(w->type), w->rows, m, w->nb, w->cols, ctx->gemm_variant);
  float* part = nullptr;
  if (ks > 1) {
    rc = acquire_workspace(ctx, s, align256(static_cast<size_t>(ks) * m * w->rows * sizeof(float)));
    if (rc) return rc;
    part = static_cast<float*>(ctx->ws);
  }
  mq::launch_gemm(static_cast<int>(w->type), w->dev, w->rows, w->nb, w->cols, a16_dev, m, y_dev, nullptr, 0,
                  ctx->gemm_variant, s, range(*w, reinterpret_cast<const float*>(a16_dev + m * k)), part);
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_dequantize_dev(mq_ctx* ctx, uint64_t handle, int logical, float* out_dev, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_dequantize_dev: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  if (!out_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_dequantize_dev: null output");
  DeviceGuard guard(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (grid_type(w->type))
    mq::launch_dequantize_grid(static_cast<int>(w->type), w->dev, w->rows, w->nb, logical, out_dev, s);
  else if (plane_type(w->type))
    mq::launch_dequantize_planes(static_cast<int>(w->type), w->dev, w->rows, w->cols, w->nb, logical, out_dev, s);
  else
    mq::launch_dequantize(static_cast<int>(w->type), w->dev, w->rows, w->nb, logical, out_dev, s);
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_dequantize(mq_ctx* ctx, uint64_t handle, int logical, float* out) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_dequantize: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  if (!out) return fail(ctx, MQ_ERR_ARGUMENT, "mq_dequantize: null output");
  DeviceGuard guard(ctx->device);
  const size_t bytes = w->rows * w->cols * sizeof(float);
  float* dev = nullptr;
  MQ_HIP(ctx, hipMalloc(&dev, bytes));
  if (grid_type(w->type))
    mq::launch_dequantize_grid(static_cast<int>(w->type), w->dev, w->rows, w->nb, logical, dev, ctx->stream);
  else if (plane_type(w->type))
    mq::launch_dequantize_planes(static_cast<int>(w->type), w->dev, w->rows, w->cols, w->nb, logical, dev,
                                 ctx->stream);
  else
    mq::launch_dequantize(static_cast<int>(w->type), w->dev, w->rows, w->nb, logical, dev, ctx->stream);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipMemcpyAsync(out, dev, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  (void)hipFree(dev);
  if (e != hipSuccess) return hip_fail(ctx, e, "mq_dequantize");
  return MQ_OK;
} MQ_CATCH(ctx)


// ---- decode-step fusions ----------------------------------------------------------

int mq_decode_matmul_dev(mq_ctx* ctx, uint64_t handle, const float* x_dev, uint64_t k, const mq_decode_fusion* f,
                         float* y_dev, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_decode_matmul_dev: null context");
  if (!f || !x_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_decode_matmul_dev: null argument");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  const uint32_t orient = w->transposed ? 0u : MQ_TRANSPOSE_B;  // stored rows are the outputs
  int rc = check_k(ctx, *w, k, orient);
  if (rc) return rc;
  if (plane_type(w->type) || grid_type(w->type))
    return fail(ctx, MQ_DECLINED, "decode-step fusions cover Q4_K and IQ4_XS weights");
  // the reference's test (src/lib.rs:388): a NaN epsilon passes and gives NaN
  if (f->norm_weight && f->norm_epsilon <= 0.0f)
    return fail(ctx, MQ_ERR_SHAPE, "RMSNorm epsilon must be positive");
  mq::GemvFusion fu;
  fu.norm_w = f->norm_weight;
  fu.norm_eps = f->norm_epsilon;
  DeviceGuard guard(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (f->epilogue == MQ_EPILOGUE_ROPE_KV) {
    if (f->rope_dim == 0 || f->rope_dim % 2 || f->rope_rows % f->rope_dim || f->rope_rows > w->rows)
      return fail(ctx, MQ_ERR_SHAPE, "rope rows must be whole heads of an even dimension within the output");
    if (!std::isfinite(f->rope_base) || f->rope_base <= 0.0f || !std::isfinite(f->rope_scale) ||
        f->rope_scale <= 0.0f)
      return fail(ctx, MQ_ERR_SHAPE, "RoPE base and scale must be finite and positive");
    if (f->seg_begin[0] != 0 || f->seg_begin[1] < f->seg_begin[0] || f->seg_begin[2] < f->seg_begin[1] ||
        f->seg_begin[2] > w->rows)
      return fail(ctx, MQ_ERR_SHAPE, "output segments must start at 0 and be ordered within the output");
    const uint64_t ends[3] = {f->seg_begin[1], f->seg_begin[2], w->rows};
    for (int i = 0; i < 3; ++i) {
      if (ends[i] > f->seg_begin[i] && !f->seg_out[i])
        return fail(ctx, MQ_ERR_ARGUMENT, "null output for a non-empty segment");
      fu.seg_begin[i] = static_cast<uint32_t>(f->seg_begin[i]);
      fu.seg_out[i] = f->seg_out[i];
    }
    const float* freq = nullptr;
    rc = rope_table(ctx, f->rope_base, f->rope_dim, &freq);
    if (rc) return rc;
    fu.freq = freq;
    fu.position = static_cast<float>(f->rope_offset) * f->rope_scale;
    fu.rope_rows = static_cast<uint32_t>(f->rope_rows);
    fu.rope_dim = static_cast<uint32_t>(f->rope_dim);
  } else if (f->epilogue == MQ_EPILOGUE_SILU_PAIRS) {
    if (w->rows % 64) return fail(ctx, MQ_ERR_SHAPE, "gate/up pairs need a multiple of 64 stored rows");
    if (!y_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_decode_matmul_dev: null output");
  } else if (f->epilogue == MQ_EPILOGUE_NONE) {
    if (!y_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_decode_matmul_dev: null output");
    if (!f->norm_weight) return matmul_locked(ctx, *w, x_dev, 1, k, MQ_INT8_ACTIVATIONS | orient, y_dev, s);
  } else {
    return fail(ctx, MQ_ERR_ARGUMENT, "unknown decode epilogue " + std::to_string(f->epilogue));
  }
  mq::GemvSplitK sk;
  rc = order_stream(ctx, s);
  if (!rc) rc = acquire_splitk(ctx, s, *w, 1, sk);
  if (rc) return rc;
  if (!mq::launch_gemv_decode_fused(static_cast<int>(w->type), w->dev, w->rows, w->nb, x_dev, y_dev,
                                    f->norm_weight != nullptr, static_cast<int>(f->epilogue), fu, sk, s))
    return fail(ctx, MQ_DECLINED, "the row does not fit the fused decode GEMV's LDS staging");
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

// ---- embedding lookup ------------------------------------------------------------

int mq_embedding_dev(mq_ctx* ctx, uint64_t handle, const float* ids, uint64_t count, float scale, float* out_dev,
                     void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_embedding_dev: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  if (count == 0) return MQ_OK;
  if (!ids || !out_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_embedding_dev: null pointer");
  DeviceGuard guard(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = order_stream(ctx, s);
  if (!rc) rc = stage_ids(ctx, *w, ids, count, s);
  if (rc) return rc;
  const uint64_t dim = w->transposed ? w->rows : w->cols;
  mq::launch_embedding(static_cast<int>(w->type), w->dev, w->nb, w->transposed, ctx->ids, count, dim, scale,
                       std::isnan(scale) ? 0 : 1, out_dev, s);
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_embedding(mq_ctx* ctx, uint64_t handle, const float* ids, uint64_t count, float scale, float* out) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_embedding: null context");
  std::lock_guard<std::mutex> lock(ctx->mu);
  const Weight* w = find_weight(ctx, handle);
  if (!w) return fail(ctx, MQ_ERR_ARGUMENT, "unknown weight handle " + std::to_string(handle));
  if (count == 0) return MQ_OK;
  if (!ids || !out) return fail(ctx, MQ_ERR_ARGUMENT, "mq_embedding: null pointer");
  DeviceGuard guard(ctx->device);
  int rc = order_stream(ctx, ctx->stream);
  if (!rc) rc = stage_ids(ctx, *w, ids, count, ctx->stream);
  if (rc) return rc;
  const uint64_t dim = w->transposed ? w->rows : w->cols;
  const size_t bytes = count * dim * sizeof(float);
  rc = acquire_workspace(ctx, ctx->stream, bytes);
  if (rc) return rc;
  auto* dev = static_cast<float*>(ctx->ws);
  mq::launch_embedding(static_cast<int>(w->type), w->dev, w->nb, w->transposed, ctx->ids, count, dim, scale,
                       std::isnan(scale) ? 0 : 1, dev, ctx->stream);
  MQ_HIP(ctx, hipGetLastError());
  MQ_HIP(ctx, hipMemcpyAsync(out, dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
  MQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MQ_OK;
} MQ_CATCH(ctx)

// ---- decoder-layer operators ----------------------------------------------------

int mq_rmsnorm_dev(mq_ctx* ctx, const float* x_dev, uint64_t rows, uint64_t cols, const float* w_dev,
                   uint64_t w_rows, float epsilon, float* out_dev, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_rmsnorm_dev: null context");
  if (cols == 0) return fail(ctx, MQ_ERR_SHAPE, "RMSNorm hidden dimension must be non-zero");
  // the reference's test (src/lib.rs:388): a NaN epsilon passes and gives NaN
  if (epsilon <= 0.0f) return fail(ctx, MQ_ERR_SHAPE, "RMSNorm epsilon must be positive");
  if (w_rows != 1 && w_rows != rows)
    return fail(ctx, MQ_ERR_SHAPE, "RMSNorm weight shape must be [" + std::to_string(cols) + "] or [" +
                                       std::to_string(rows) + ", " + std::to_string(cols) + "]");
  if (rows == 0) return MQ_OK;
  if (!x_dev || !w_dev || !out_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_rmsnorm_dev: null pointer");
  DeviceGuard guard(ctx->device);
  mq::launch_rmsnorm(x_dev, rows, cols, w_dev, w_rows == 1 ? 0 : cols, epsilon, out_dev,
                     static_cast<hipStream_t>(stream));
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_rope_dev(mq_ctx* ctx, const float* x_dev, uint64_t rows, uint64_t cols, float base, float scale,
                uint64_t dimension, uint64_t position_offset, uint64_t head_count, int pairing, float* out_dev,
                void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_rope_dev: null context");
  if (head_count == 0 || cols % head_count)
    return fail(ctx, MQ_ERR_SHAPE, "RoPE head_count " + std::to_string(head_count) +
                                       " must be positive and evenly divide the row width " + std::to_string(cols));
  const uint64_t head_width = cols / head_count;
  if (dimension == 0 || dimension % 2 || dimension > head_width)
    return fail(ctx, MQ_ERR_SHAPE, "RoPE dimension " + std::to_string(dimension) +
                                       " must be positive, even, and at most the head width " +
                                       std::to_string(head_width));
  if (!std::isfinite(base) || base <= 0.0f) return fail(ctx, MQ_ERR_SHAPE, "RoPE base must be finite and positive");
  if (!std::isfinite(scale) || scale <= 0.0f)
    return fail(ctx, MQ_ERR_SHAPE, "RoPE scale must be finite and positive");
  if (pairing != MQ_ROPE_INTERLEAVED && pairing != MQ_ROPE_HALF_SPLIT)
    return fail(ctx, MQ_ERR_ARGUMENT, "unknown RoPE pairing " + std::to_string(pairing));
  if (rows == 0) return MQ_OK;
  if (!x_dev || !out_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_rope_dev: null pointer");
  std::lock_guard<std::mutex> lock(ctx->mu);
  DeviceGuard guard(ctx->device);
  const float* freq = nullptr;
  int rc = rope_table(ctx, base, dimension, &freq);
  if (rc) return rc;
  mq::launch_rope(x_dev, rows, cols, head_count, dimension, scale, position_offset, pairing, freq, out_dev,
                  static_cast<hipStream_t>(stream));
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_kv_write_dev(mq_ctx* ctx, float* store_dev, uint64_t capacity, uint64_t width, const float* rows_dev,
                    uint64_t count, uint64_t row_offset, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_kv_write_dev: null context");
  if (row_offset + count < row_offset || row_offset + count > capacity)
    return fail(ctx, MQ_ERR_SHAPE, "kv-write of " + std::to_string(count) + " rows at " +
                                       std::to_string(row_offset) + " exceeds the store's " +
                                       std::to_string(capacity) + " rows");
  if (count == 0 || width == 0) return MQ_OK;
  if (!store_dev || !rows_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_kv_write_dev: null pointer");
  float* dst = store_dev + row_offset * width;
  if (dst < rows_dev + count * width && rows_dev < dst + count * width)
    return fail(ctx, MQ_ERR_ARGUMENT, "kv-write rows overlap the store rows they replace");
  DeviceGuard guard(ctx->device);
  mq::launch_copy(rows_dev, count * width, dst, static_cast<hipStream_t>(stream));
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_attention_dev(mq_ctx* ctx, const float* q_dev, uint64_t seq, const float* k_dev, const float* v_dev,
                     uint64_t kv_rows, uint64_t key_count, uint64_t heads, uint64_t head_dim, uint64_t kv_heads,
                     int causal, float score_scale, float* out_dev, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_attention_dev: null context");
  if (heads == 0 || head_dim == 0 || kv_heads == 0)
    return fail(ctx, MQ_ERR_SHAPE, "head_count, kv_head_count, and head_dimension must all be positive");
  if (heads % kv_heads)
    return fail(ctx, MQ_ERR_SHAPE, "head_count " + std::to_string(heads) + " must be an exact multiple of kv_head_count " +
                                       std::to_string(kv_heads));
  if (key_count > kv_rows)
    return fail(ctx, MQ_ERR_SHAPE, "key_count " + std::to_string(key_count) + " exceeds the " +
                                       std::to_string(kv_rows) + " rows of K/V");
  if (seq > key_count)
    return fail(ctx, MQ_ERR_SHAPE, "q sequence length " + std::to_string(seq) +
                                       " cannot exceed k/v sequence length " + std::to_string(key_count));
  if (!std::isnan(score_scale) && !std::isfinite(score_scale))
    return fail(ctx, MQ_ERR_SHAPE, "attention scale must be finite");
  const uint64_t group = heads / kv_heads;
  if (head_dim != 128 || (group != 1 && group != 2 && group != 4 && group != 8))
    return fail(ctx, MQ_DECLINED, "attention with head_dim " + std::to_string(head_dim) + " and " +
                                      std::to_string(group) + " query heads per kv head has no GPU path");
  if (seq == 0) return MQ_OK;
  if (!q_dev || !k_dev || !v_dev || !out_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_attention_dev: null pointer");
  const float scale = std::isnan(score_scale) ? 1.0f / std::sqrt(static_cast<float>(head_dim)) : score_scale;
  std::lock_guard<std::mutex> lock(ctx->mu);
  DeviceGuard guard(ctx->device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  int rc = order_stream(ctx, s);
  if (rc) return rc;
  const size_t need = seq * heads * mq::attention_chunks(key_count) * (2 + head_dim) * sizeof(float);
  if (need > ctx->attn_bytes) {
    MQ_HIP(ctx, hipStreamSynchronize(s));
    if (ctx->attn) MQ_HIP(ctx, hipFree(ctx->attn));
    ctx->attn = nullptr;
    ctx->attn_bytes = 0;
    MQ_HIP(ctx, hipMalloc(&ctx->attn, need));
    ctx->attn_bytes = need;
  }
  if (!mq::launch_attention(q_dev, k_dev, v_dev, seq, key_count, heads, head_dim, kv_heads, causal ? 1 : 0, scale,
                            static_cast<float*>(ctx->attn), out_dev, s))
    return fail(ctx, MQ_DECLINED, "attention shape has no GPU path");
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_silu_mul_dev(mq_ctx* ctx, const float* gate_dev, const float* up_dev, uint64_t n, float* out_dev,
                    void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_silu_mul_dev: null context");
  if (n == 0) return MQ_OK;
  if (!gate_dev || !up_dev || !out_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_silu_mul_dev: null pointer");
  DeviceGuard guard(ctx->device);
  mq::launch_silu_mul(gate_dev, up_dev, n, out_dev, static_cast<hipStream_t>(stream));
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_add_dev(mq_ctx* ctx, const float* a_dev, uint64_t n, const float* b_dev, uint64_t b_n, float* out_dev,
               void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_add_dev: null context");
  if (b_n == 0 || n % b_n) return fail(ctx, MQ_ERR_SHAPE, "add: b must match a or be one row of a");
  if (n == 0) return MQ_OK;
  if (!a_dev || !b_dev || !out_dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_add_dev: null pointer");
  DeviceGuard guard(ctx->device);
  mq::launch_add(a_dev, n, b_dev, b_n, out_dev, static_cast<hipStream_t>(stream));
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

// ---- device-resident tensor storage -------------------------------------------

void* mq_context_stream(mq_ctx* ctx) { return ctx ? static_cast<void*>(ctx->stream) : nullptr; }

int mq_device_alloc(mq_ctx* ctx, uint64_t bytes, void** dev) try {
  if (!ctx || !dev) return fail(ctx, MQ_ERR_ARGUMENT, "mq_device_alloc: null argument");
  *dev = nullptr;
  if (bytes == 0) return MQ_OK;
  DeviceGuard guard(ctx->device);
  MQ_HIP(ctx, hipMalloc(dev, bytes));
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_device_free(mq_ctx* ctx, void* dev) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_device_free: null context");
  if (!dev) return MQ_OK;
  DeviceGuard guard(ctx->device);
  MQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
  MQ_HIP(ctx, hipFree(dev));
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_copy_to_device(mq_ctx* ctx, void* dst_dev, const void* src, uint64_t bytes) try {
  if (!ctx || (bytes && (!dst_dev || !src))) return fail(ctx, MQ_ERR_ARGUMENT, "mq_copy_to_device: null argument");
  if (bytes == 0) return MQ_OK;
  DeviceGuard guard(ctx->device);
  MQ_HIP(ctx, hipMemcpyAsync(dst_dev, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  MQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_copy_to_host(mq_ctx* ctx, void* dst, const void* src_dev, uint64_t bytes) try {
  if (!ctx || (bytes && (!dst || !src_dev))) return fail(ctx, MQ_ERR_ARGUMENT, "mq_copy_to_host: null argument");
  if (bytes == 0) return MQ_OK;
  DeviceGuard guard(ctx->device);
  MQ_HIP(ctx, hipMemcpyAsync(dst, src_dev, bytes, hipMemcpyDeviceToHost, ctx->stream));
  MQ_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_copy_dev(mq_ctx* ctx, void* dst_dev, const void* src_dev, uint64_t bytes, void* stream) try {
  if (!ctx || (bytes && (!dst_dev || !src_dev))) return fail(ctx, MQ_ERR_ARGUMENT, "mq_copy_dev: null argument");
  if (bytes == 0 || dst_dev == src_dev) return MQ_OK;
  DeviceGuard guard(ctx->device);
  MQ_HIP(ctx, hipMemcpyAsync(dst_dev, src_dev, bytes, hipMemcpyDeviceToDevice, static_cast<hipStream_t>(stream)));
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_fill_dev(mq_ctx* ctx, float* dst_dev, uint64_t count, float value, void* stream) try {
  if (!ctx || (count && !dst_dev)) return fail(ctx, MQ_ERR_ARGUMENT, "mq_fill_dev: null argument");
  if (count == 0) return MQ_OK;
  DeviceGuard guard(ctx->device);
  mq::launch_fill(dst_dev, count, value, static_cast<hipStream_t>(stream));
  MQ_HIP(ctx, hipGetLastError());
  return MQ_OK;
} MQ_CATCH(ctx)

int mq_synchronize(mq_ctx* ctx, void* stream) try {
  if (!ctx) return fail(ctx, MQ_ERR_ARGUMENT, "mq_synchronize: null context");
  DeviceGuard guard(ctx->device);
  MQ_HIP(ctx, hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  return MQ_OK;
} MQ_CATCH(ctx)

}  // extern "C"
