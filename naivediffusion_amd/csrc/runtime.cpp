// Device, tensors, memory pool, errors and the host int8 quantiser.
//
// Replaces Dml/DmlDevice.cs, Dml/DmlBufferPool.cs, Dml/DeviceTensor.cs and
// Dml/DeviceExceptions.cs of the reference: one HIP stream per device instead
// of one D3D12 queue, hipMalloc blocks recycled by size instead of committed
// resources, and the same two failure kinds (out of memory, device lost).

#include "runtime.h"

#include <string.h>

#include <algorithm>
#include <cmath>
#include <thread>
#include <vector>

namespace ndx {

static thread_local std::string g_last_error;

void set_last_error(const std::string& message) { g_last_error = message; }

[[noreturn]] void fail(ndx_status status, const std::string& message) {
  throw Error{status, message};
}

void hip_check(hipError_t err, const char* what) {
  if (err == hipSuccess) return;
  std::string msg = std::string(what) + ": " + hipGetErrorString(err);
  if (err == hipErrorOutOfMemory) fail(NDX_OOM, msg);
  fail(NDX_DEVICE_LOST, msg);
}

const char* dtype_name(int dt) {
  switch (dt) {
    case NDX_F32: return "Float32";
    case NDX_F16: return "Float16";
    case NDX_BF16: return "BFloat16";
    case NDX_U32: return "UInt32";
    case NDX_I32: return "Int32";
    case NDX_U16: return "UInt16";
    case NDX_I64: return "Int64";
    case NDX_I8: return "Int8";
    default: return "?";
  }
}

size_t pool_round(size_t bytes) {
  if (bytes == 0) bytes = 1;
  if (bytes <= (1u << 20)) return (bytes + 511) & ~size_t(511);
  return (bytes + (2u << 20) - 1) & ~size_t((2u << 20) - 1);
}

void check_shape(const int64_t* shape, int rank) {
  if (rank < 1 || rank > 4) fail(NDX_INVALID_ARG, "rank must be 1 to 4, not " + std::to_string(rank));
  if (!shape) fail(NDX_INVALID_ARG, "shape is null");
  for (int i = 0; i < rank; i++)
    if (shape[i] <= 0) fail(NDX_INVALID_ARG, "extents must be positive");
}

ndx_tensor* new_tensor(ndx_device* dev, int dtype, const int64_t* shape, int rank) {
  check_shape(shape, rank);
  if (dtype_size(dtype) == 0) fail(NDX_INVALID_ARG, "unknown element type " + std::to_string(dtype));
  auto* t = new ndx_tensor();
  t->dev = dev;
  t->dtype = dtype;
  t->rank = rank;
  for (int i = 0; i < rank; i++) t->shape[i] = shape[i];
  t->bytes = size_t(t->numel()) * dtype_size(dtype);
  t->alloc = pool_round(t->bytes);
  try {
    t->ptr = dev->alloc(t->alloc);
  } catch (...) {
    delete t;
    throw;
  }
  return t;
}

void free_tensor(ndx_tensor* t) {
  if (!t) return;
  if (t->dev && t->ptr) t->dev->release(t->ptr, t->alloc);
  delete t;
}

// ---- host quantiser (Tensors/BlockQuantizer.cs:34-101) -----------------------

static inline float widen(const void* data, int dtype, int64_t i) {
  switch (dtype) {
    case NDX_F32: return ((const float*)data)[i];
    case NDX_F16: return (float)((const _Float16*)data)[i];
    case NDX_BF16: {
      uint32_t bits = uint32_t(((const uint16_t*)data)[i]) << 16;
      float f;
      memcpy(&f, &bits, 4);
      return f;
    }
    default: return 0.f;
  }
}

void quantize_host(const void* w, int dtype, int64_t rows, int64_t cols, int block, int s_dtype,
                   int8_t* q, void* scales) {
  const int64_t blocks = cols / block;
  auto work = [&](int64_t r0, int64_t r1) {
    for (int64_t r = r0; r < r1; r++) {
      for (int64_t b = 0; b < blocks; b++) {
        const int64_t start = r * cols + b * block;
        float peak = 0.f;
        for (int i = 0; i < block; i++) peak = std::max(peak, std::fabs(widen(w, dtype, start + i)));
        // The scale is quantised to its storage type first and the values
        // are quantised against the stored scale (BlockQuantizer.cs:61-72).
        float stored;
        if (s_dtype == NDX_F16) {
          _Float16 h = (_Float16)(peak / 127.0f);
          ((_Float16*)scales)[r * blocks + b] = h;
          stored = (float)h;
        } else {
          stored = peak / 127.0f;
          ((float*)scales)[r * blocks + b] = stored;
        }
        int8_t* out = q + start;
        if (stored == 0.f) {
          memset(out, 0, block);
          continue;
        }
        const float inverse = 1.0f / stored;
        for (int i = 0; i < block; i++) {
          float v = rintf(widen(w, dtype, start + i) * inverse);  // round half to even
          v = std::min(127.f, std::max(-127.f, v));
          out[i] = (int8_t)(int)v;
        }
      }
    }
  };
  unsigned threads = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  if (rows * cols < (1 << 20)) threads = 1;
  std::vector<std::thread> pool;
  int64_t per = (rows + threads - 1) / threads;
  for (unsigned t = 0; t < threads; t++) {
    int64_t r0 = t * per, r1 = std::min(rows, r0 + per);
    if (r0 >= r1) break;
    pool.emplace_back(work, r0, r1);
  }
  for (auto& th : pool) th.join();
}

}  // namespace ndx

using namespace ndx;

// ---- device -------------------------------------------------------------------

hipStream_t ndx_device::aux_stream() {
  if (!aux) {
    // Default priority, like the device stream (streams of different
    // priorities are never mixed here).
    hip_check(hipStreamCreateWithFlags(&aux, hipStreamNonBlocking), "hipStreamCreate");
  }
  return aux;
}

void* ndx_device::alloc(size_t bytes) {
  check_usable();
  if (fault == 1) {
    fault = 0;
    fail(NDX_OOM, "out of device memory (injected)");
  }
  auto it = free_blocks.find(bytes);
  if (it != free_blocks.end()) {
    void* p = it->second;
    free_blocks.erase(it);
    pooled_bytes -= bytes;
    live_bytes += bytes;
    refs++;
    return p;
  }
  void* p = nullptr;
  hipError_t err = hipMalloc(&p, bytes);
  if (err == hipErrorOutOfMemory) {
    (void)hipGetLastError();
    trim();
    err = hipMalloc(&p, bytes);
  }
  if (err == hipErrorOutOfMemory) {
    (void)hipGetLastError();
    fail(NDX_OOM, "out of device memory allocating " + std::to_string(bytes) + " bytes");
  }
  hip_check(err, "hipMalloc");
  live_bytes += bytes;
  refs++;
  return p;
}

void ndx_device::release(void* p, size_t bytes) {
  if (!p) return;
  live_bytes -= bytes;
  if (destroyed) {
    (void)hipFree(p);
    if (--refs == 0) delete this;
    return;
  }
  free_blocks.emplace(bytes, p);
  pooled_bytes += bytes;
}

void ndx_device::trim() {
  if (!free_blocks.empty()) (void)hipStreamSynchronize(stream);
  for (auto& kv : free_blocks) {
    (void)hipFree(kv.second);
    refs--;
  }
  free_blocks.clear();
  pooled_bytes = 0;
}

void ndx_device::check_usable() const {
  if (destroyed) fail(NDX_INVALID_STATE, "the device was destroyed");
  if (lost || fault == 2) fail(NDX_DEVICE_LOST, "the device was lost");
}

static void mark_lost_on(ndx_device* dev, const ndx::Error& e) {
  if (dev && e.status == NDX_DEVICE_LOST) dev->lost = true;
}

extern "C" {

NDX_API const char* ndx_last_error(void) { return g_last_error.c_str(); }
#ifndef NDX_SOURCE_HASH
#define NDX_SOURCE_HASH "unknown"
#endif
// The last word is the hash of the sources the library was built from
// (naivediffusion_amd/build.py); the Python loader refuses a mismatch.
NDX_API const char* ndx_version(void) { return "ndx 0.2 (gfx950) src " NDX_SOURCE_HASH; }

NDX_API ndx_status ndx_device_count(int32_t* count) {
  NDX_TRY
  if (!count) fail(NDX_INVALID_ARG, "count is null");
  int n = 0;
  hipError_t err = hipGetDeviceCount(&n);
  if (err != hipSuccess) {
    (void)hipGetLastError();
    n = 0;
  }
  *count = n;
  NDX_CATCH
}

// The temporary memory of ndx_model_run_into_static_async: every GPU the
// library runs on holds its own copy from the library's load until the
// process ends, and every static run on that GPU shares it. In host code the
// name `scratch` is a host-side stand-in, not a device address: the address
// is looked up once per device below (hipGetSymbolAddress, with the device
// current) and only that address, ndx_device::static_scratch, is used.
static __device__ __align__(256) char scratch[ndx::kStaticScratchBytes];

// Looks up this GPU's copy of the static scratch array; a failure is kept
// and reported by the static run, not by the device creation.
static void find_static_scratch(ndx_device* dev) {
  void* p = nullptr;
  const hipError_t err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (err != hipSuccess || !p) {
    (void)hipGetLastError();
    dev->static_scratch_error = std::string("hipGetSymbolAddress: ") + hipGetErrorString(err);
    return;
  }
  dev->static_scratch = p;
}

NDX_API ndx_status ndx_device_create(int32_t adapter, ndx_device** out) {
  NDX_TRY
  if (!out) fail(NDX_INVALID_ARG, "out is null");
  *out = nullptr;
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    (void)hipGetLastError();
    fail(NDX_DEVICE_LOST, "no GPU is visible");
  }
  int id = adapter < 0 ? 0 : adapter;
  if (id >= n) fail(NDX_INVALID_ARG, "adapter " + std::to_string(adapter) + " of " + std::to_string(n));
  hip_check(hipSetDevice(id), "hipSetDevice");
  hipDeviceProp_t prop;
  hip_check(hipGetDeviceProperties(&prop, id), "hipGetDeviceProperties");
  std::string arch = prop.gcnArchName;
  if (arch.rfind("gfx950", 0) != 0)
    fail(NDX_UNSUPPORTED, "this library is built for gfx950, the device is " + arch);
  auto* dev = new ndx_device();
  dev->id = id;
  dev->name = std::string(prop.name) + " (" + arch + ")";
  // Default priority on purpose: every stream of the library shares it.
  hipError_t err = hipStreamCreateWithFlags(&dev->stream, hipStreamNonBlocking);
  if (err != hipSuccess) {
    delete dev;
    hip_check(err, "hipStreamCreate");
  }
  find_static_scratch(dev);
  *out = dev;
  NDX_CATCH
}

NDX_API ndx_status ndx_device_destroy(ndx_device* device) {
  NDX_TRY
  if (!device || device->destroyed) return NDX_OK;
  (void)hipStreamSynchronize(device->stream);
  if (device->aux) (void)hipStreamSynchronize(device->aux);
  device->trim();
  (void)hipStreamDestroy(device->stream);
  device->stream = nullptr;
  if (device->aux) (void)hipStreamDestroy(device->aux);
  device->aux = nullptr;
  device->destroyed = true;
  // Tensors and models still alive keep the object until they go.
  if (device->refs == 0) delete device;
  NDX_CATCH
}

NDX_API ndx_status ndx_device_name(ndx_device* device, char* buffer, int32_t capacity) {
  NDX_TRY
  if (!device || !buffer || capacity <= 0) fail(NDX_INVALID_ARG, "null argument");
  snprintf(buffer, capacity, "%s", device->name.c_str());
  NDX_CATCH
}

NDX_API ndx_status ndx_device_memory(ndx_device* device, uint64_t* used, uint64_t* budget) {
  NDX_TRY
  if (!device || !used || !budget) fail(NDX_INVALID_ARG, "null argument");
  device->check_usable();
  size_t free_b = 0, total = 0;
  hip_check(hipMemGetInfo(&free_b, &total), "hipMemGetInfo");
  *used = total - free_b;
  *budget = total;
  NDX_CATCH
}

NDX_API ndx_status ndx_device_release_pooled(ndx_device* device) {
  NDX_TRY
  if (!device) fail(NDX_INVALID_ARG, "device is null");
  device->trim();
  NDX_CATCH
}

NDX_API ndx_status ndx_device_synchronize(ndx_device* device) {
  if (!device) {
    set_last_error("device is null");
    return NDX_INVALID_ARG;
  }
  try {
    device->check_usable();
    hip_check(hipStreamSynchronize(device->stream), "stream synchronize");
  } catch (const ndx::Error& e) {
    mark_lost_on(device, e);
    set_last_error(e.message);
    return e.status;
  }
  return NDX_OK;
}

NDX_API ndx_status ndx_device_set_fault_injection(ndx_device* device, int32_t kind) {
  NDX_TRY
  if (!device) fail(NDX_INVALID_ARG, "device is null");
  if (kind < 0 || kind > 2) fail(NDX_INVALID_ARG, "fault kind must be 0, 1 or 2");
  device->fault = kind;
  NDX_CATCH
}

// ---- tensors ------------------------------------------------------------------

NDX_API ndx_status ndx_tensor_upload(ndx_device* device, int32_t dtype, const int64_t* shape,
                                     int32_t rank, const void* data, uint64_t bytes,
                                     ndx_tensor** out) {
  NDX_TRY
  if (!device || !out || !data) fail(NDX_INVALID_ARG, "null argument");
  *out = nullptr;
  check_shape(shape, rank);
  int64_t n = 1;
  for (int i = 0; i < rank; i++) n *= shape[i];
  if (dtype_size(dtype) == 0) fail(NDX_INVALID_ARG, "unknown element type");
  if (uint64_t(n) * dtype_size(dtype) != bytes)
    fail(NDX_INVALID_ARG, std::to_string(bytes) + " bytes do not fill a " + dtype_name(dtype) +
                              " tensor of " + std::to_string(n) + " elements");
  ndx_tensor* t = new_tensor(device, dtype, shape, rank);
  try {
    hip_check(hipMemcpyAsync(t->ptr, data, bytes, hipMemcpyHostToDevice, device->stream), "upload");
    hip_check(hipStreamSynchronize(device->stream), "upload");
  } catch (...) {
    free_tensor(t);
    throw;
  }
  *out = t;
  NDX_CATCH
}

NDX_API ndx_status ndx_tensor_empty(ndx_device* device, int32_t dtype, const int64_t* shape,
                                    int32_t rank, ndx_tensor** out) {
  NDX_TRY
  if (!device || !out) fail(NDX_INVALID_ARG, "null argument");
  *out = new_tensor(device, dtype, shape, rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_tensor_download(ndx_tensor* tensor, void* data, uint64_t bytes) {
  NDX_TRY
  if (!tensor || !data) fail(NDX_INVALID_ARG, "null argument");
  tensor->dev->check_usable();
  if (bytes != tensor->bytes)
    fail(NDX_INVALID_ARG, "download of " + std::to_string(bytes) + " bytes from a tensor of " +
                              std::to_string(tensor->bytes));
  hip_check(hipMemcpyAsync(data, tensor->ptr, bytes, hipMemcpyDeviceToHost, tensor->dev->stream),
            "download");
  hip_check(hipStreamSynchronize(tensor->dev->stream), "download");
  NDX_CATCH
}

NDX_API ndx_status ndx_tensor_release(ndx_tensor* tensor) {
  NDX_TRY
  free_tensor(tensor);
  NDX_CATCH
}

NDX_API ndx_status ndx_tensor_info(ndx_tensor* tensor, int32_t* dtype, int64_t* shape,
                                   int32_t* rank) {
  NDX_TRY
  if (!tensor) fail(NDX_INVALID_ARG, "tensor is null");
  if (dtype) *dtype = tensor->dtype;
  if (rank) *rank = tensor->rank;
  if (shape)
    for (int i = 0; i < 4; i++) shape[i] = i < tensor->rank ? tensor->shape[i] : 1;
  NDX_CATCH
}

NDX_API ndx_status ndx_tensor_fill_normal(ndx_tensor* tensor, uint64_t seed, float mean,
                                          float std_dev) {
  NDX_TRY
  if (!tensor) fail(NDX_INVALID_ARG, "tensor is null");
  if (!dtype_is_float(tensor->dtype)) fail(NDX_INVALID_ARG, "fill_normal needs a float tensor");
  tensor->dev->check_usable();
  launch_fill_normal(tensor->ptr, tensor->dtype, tensor->numel(), seed, mean, std_dev,
                     tensor->dev->stream);
  hip_check(hipGetLastError(), "fill_normal launch");
  hip_check(hipStreamSynchronize(tensor->dev->stream), "fill_normal");
  NDX_CATCH
}

// ---- quantiser ----------------------------------------------------------------

NDX_API int32_t ndx_quantize_fits(int64_t elements, int32_t rows, int32_t block) {
  return rows > 0 && block > 0 && elements % rows == 0 && (elements / rows) % block == 0;
}

NDX_API ndx_status ndx_quantize_block_int8(const void* w, int32_t dtype, int64_t rows,
                                           int64_t cols, int32_t block, int32_t scale_dtype,
                                           int8_t* q, void* scales) {
  NDX_TRY
  if (!w || !q || !scales) fail(NDX_INVALID_ARG, "null argument");
  if (dtype != NDX_F32 && dtype != NDX_F16 && dtype != NDX_BF16)
    fail(NDX_INVALID_ARG, "the quantiser reads Float32, Float16 or BFloat16");
  if (scale_dtype != NDX_F16 && scale_dtype != NDX_F32)
    fail(NDX_INVALID_ARG, "scales are Float16 or Float32");
  if (!ndx_quantize_fits(rows * cols, (int32_t)rows, block))
    fail(NDX_INVALID_ARG, std::to_string(rows * cols) + " elements in " + std::to_string(rows) +
                              " rows do not split into blocks of " + std::to_string(block));
  quantize_host(w, dtype, rows, cols, block, scale_dtype, q, scales);
  NDX_CATCH
}

NDX_API ndx_status ndx_quantize_block_int8_device(ndx_tensor* w, int32_t block,
                                                  int32_t scale_dtype, ndx_tensor* q,
                                                  ndx_tensor* scales) {
  NDX_TRY
  if (!w || !q || !scales) fail(NDX_INVALID_ARG, "null argument");
  w->dev->check_usable();
  if (!dtype_is_float(w->dtype)) fail(NDX_INVALID_ARG, "the quantiser reads a float tensor");
  int64_t cols = w->shape[w->rank - 1];
  int64_t rows = w->numel() / cols;
  if (block <= 0 || cols % block) fail(NDX_INVALID_ARG, "the blocks do not tile the columns");
  if (q->dtype != NDX_I8 || q->numel() != w->numel()) fail(NDX_INVALID_ARG, "q must be Int8 like w");
  if (scales->dtype != scale_dtype || scales->numel() != rows * (cols / block))
    fail(NDX_INVALID_ARG, "scales must be [rows, cols/block] of the scale type");
  if (scale_dtype != NDX_F16 && scale_dtype != NDX_F32) fail(NDX_INVALID_ARG, "scales are F16 or F32");
  launch_quantize(w->ptr, w->dtype, rows, cols, block, scale_dtype, (int8_t*)q->ptr, scales->ptr,
                  w->dev->stream);
  hip_check(hipGetLastError(), "quantize launch");
  hip_check(hipStreamSynchronize(w->dev->stream), "quantize");
  NDX_CATCH
}

}  // extern "C"
