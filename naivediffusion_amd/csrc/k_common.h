// Device helpers shared by the kernel files: element access by runtime type,
// rounding, activations and wavefront (64-lane) reductions.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ndx_internal.h"

namespace ndx {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// Bounds-checked buffer loads: an offset at or past the resource's size
// reads zeros (a load straight to LDS writes zeros), so tile edges need no
// branches.
constexpr uint32_t kOutOfRange = 0x80000000u;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* p, uint32_t bytes) {
  // Word 3 = 0x00020000: raw 32-bit dword access, the gfx9-family setting.
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, bytes, 0x00020000);
}
// An LDS address for buffer_load ... lds (wave-uniform; lane l lands at
// byte 16 l of a 16-byte-per-lane load).
typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(uint32_t(h) << 16);
}

// Reads element i of a float tensor stored as dt.
__device__ __forceinline__ float load_f(const void* p, int dt, int64_t i) {
  switch (dt) {
    case NDX_F32: return ((const float*)p)[i];
    case NDX_F16: return (float)((const _Float16*)p)[i];
    case NDX_BF16: return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    case NDX_I32: return (float)((const int32_t*)p)[i];
    case NDX_I8: return (float)((const int8_t*)p)[i];
    default: return 0.f;
  }
}

// Writes v as dt, rounding to nearest even.
__device__ __forceinline__ void store_f(void* p, int dt, int64_t i, float v) {
  switch (dt) {
    case NDX_F32: ((float*)p)[i] = v; break;
    case NDX_F16: ((_Float16*)p)[i] = (_Float16)v; break;
    case NDX_BF16: ((__bf16*)p)[i] = (__bf16)v; break;
    default: break;
  }
}

// v rounded to dt and back: the value a tensor of that type would hold.
__device__ __forceinline__ float round_to(float v, int dt) {
  switch (dt) {
    case NDX_F16: return (float)(_Float16)v;
    case NDX_BF16: return (float)(__bf16)v;
    default: return v;
  }
}

__device__ __forceinline__ float sigmoid_f(float x) { return 1.0f / (1.0f + __expf(-x)); }
__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + __expf(-x)); }
__device__ __forceinline__ float gelu_f(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }
// x * sigmoid(2 * sqrt(2/pi) * (x + 0.044715 x^3)), QwenImageDit.cs:510-515.
__device__ __forceinline__ float gelu_tanh_f(float x) {
  float inner = 1.5957691216057308f * (x + 0.044715f * x * x * x);
  return x / (1.0f + __expf(-inner));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// splitmix64 of (seed, index) -> two uniform doubles -> one normal by
// Box-Muller (the cosine branch). Shared by the device fill and mirrored by
// the host generator naivediffusion_amd/rng.py.
__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

}  // namespace ndx
