// Device, tensor and memory-pool objects behind the opaque C handles.
#pragma once

#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "ndx_internal.h"

namespace ndx {
// Bytes of the static scratch array that ndx_model_run_into_static_async
// uses as a model's temporary memory (one array per GPU, process lifetime).
constexpr size_t kStaticScratchBytes = size_t(64) << 20;
}  // namespace ndx

struct ndx_device {
  int id = 0;
  hipStream_t stream = nullptr;
  hipStream_t aux = nullptr;  // the second lane, made when a two-lane model is compiled
  std::string name;
  bool lost = false;
  bool destroyed = false;  // ndx_device_destroy ran; freed when refs drops to 0
  int64_t refs = 0;        // live tensors and model arenas allocated here
  int fault = 0;           // ndx_device_set_fault_injection kind
  // Device address of the static scratch array on this GPU (looked up when
  // the device is created), or null with the reason in static_scratch_error.
  void* static_scratch = nullptr;
  std::string static_scratch_error;

  // Caching pool: freed blocks are kept by rounded size and handed out
  // again, the way DmlBufferPool recycles committed resources.
  std::multimap<size_t, void*> free_blocks;
  size_t pooled_bytes = 0;
  size_t live_bytes = 0;

  void* alloc(size_t bytes);
  hipStream_t aux_stream();
  // Returns a block to the pool; after destroy it is freed instead, and the
  // device object goes when the last block does.
  void release(void* p, size_t bytes);
  void trim();
  void check_usable() const;
};

struct ndx_tensor {
  ndx_device* dev = nullptr;
  int dtype = NDX_F32;
  int rank = 0;
  int64_t shape[4] = {1, 1, 1, 1};
  void* ptr = nullptr;
  size_t bytes = 0;    // payload bytes (elements * size)
  size_t alloc = 0;    // pool block size
  int64_t numel() const {
    int64_t n = 1;
    for (int i = 0; i < rank; i++) n *= shape[i];
    return n;
  }
};

namespace ndx {

size_t pool_round(size_t bytes);
ndx_tensor* new_tensor(ndx_device* dev, int dtype, const int64_t* shape, int rank);
void free_tensor(ndx_tensor* t);
void check_shape(const int64_t* shape, int rank);

}  // namespace ndx
