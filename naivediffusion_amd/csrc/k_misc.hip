// Bandwidth-bound helpers: the strided elementwise kernel (casts, views made
// packed, activations, scale/bias, binary arithmetic), nearest upsampling,
// patchify, the synthetic normal fill and the device int8 quantiser.

#include "k_common.h"

namespace ndx {

struct Idx4 {
  int64_t size[4];
};

__device__ __forceinline__ int64_t offset_of(const View4& v, int64_t i0, int64_t i1, int64_t i2, int64_t i3) {
  return i0 * v.stride[0] + i1 * v.stride[1] + i2 * v.stride[2] + i3 * v.stride[3];
}

__device__ __forceinline__ float apply_elem(int op, float a, float b, float scale, float bias) {
  switch (op) {
    case ELEM_COPY: return a;
    case ELEM_SIGMOID: return sigmoid_f(a);
    case ELEM_SILU: return silu_f(a);
    case ELEM_GELU: return gelu_f(a);
    case ELEM_TANH: return tanhf(a);
    case ELEM_GELU_TANH: return gelu_tanh_f(a);
    case ELEM_SCALE_BIAS: return a * scale + bias;
    case ELEM_ADD: return a + b;
    case ELEM_SUB: return a - b;
    case ELEM_MUL: return a * b;
    case ELEM_DIV: return a / b;
    case ELEM_MUL_GELU: return a * b;  // b already gelu(y), rounded
    default: return a;
  }
}

// One thread per output element of a 4-D strided view; the innermost axis
// is the fastest so packed tensors read and write coalesced.
__global__ void elementwise_kernel(ElemArgs a, int64_t total) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t step = int64_t(gridDim.x) * blockDim.x;
  const int64_t s3 = a.vo.size[3], s2 = a.vo.size[2], s1 = a.vo.size[1];
  for (; i < total; i += step) {
    int64_t r = i;
    int64_t i3 = r % s3;
    r /= s3;
    int64_t i2 = r % s2;
    r /= s2;
    int64_t i1 = r % s1;
    int64_t i0 = r / s1;
    float x = load_f(a.in0, a.dt0, offset_of(a.v0, i0, i1, i2, i3));
    float y = a.in1 ? load_f(a.in1, a.dt1, offset_of(a.v1, i0, i1, i2, i3)) : 0.f;
    if (a.op == ELEM_MUL_GELU) y = round_to(gelu_f(y), a.dto);
    store_f(a.out, a.dto, offset_of(a.vo, i0, i1, i2, i3), apply_elem(a.op, x, y, a.scale, a.bias));
  }
}

static int grid_for(int64_t total, int threads) {
  int64_t blocks = (total + threads - 1) / threads;
  if (blocks > 65536 * 8) blocks = 65536 * 8;
  if (blocks < 1) blocks = 1;
  return (int)blocks;
}

// Eight consecutive elements of type DT as fp32, and back.
template <int DT>
__device__ __forceinline__ void ld8(const void* p, int64_t i, float (&o)[8]) {
  if constexpr (DT == NDX_F32) {
    const float4 x = *(const float4*)((const float*)p + i), y = *(const float4*)((const float*)p + i + 4);
    o[0] = x.x; o[1] = x.y; o[2] = x.z; o[3] = x.w; o[4] = y.x; o[5] = y.y; o[6] = y.z; o[7] = y.w;
  } else {
    const uint4 u = *(const uint4*)((const uint16_t*)p + i);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      if constexpr (DT == NDX_BF16) {
        o[2 * e] = __uint_as_float(w[e] << 16);
        o[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
      } else {
        o[2 * e] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e] & 0xffff));
        o[2 * e + 1] = (float)__builtin_bit_cast(_Float16, (uint16_t)(w[e] >> 16));
      }
    }
  }
}
template <int DT>
__device__ __forceinline__ void st8(void* p, int64_t i, const float (&v)[8]) {
  if constexpr (DT == NDX_F32) {
    *(float4*)((float*)p + i) = make_float4(v[0], v[1], v[2], v[3]);
    *(float4*)((float*)p + i + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else if constexpr (DT == NDX_BF16) {
    __bf16 h[8];
#pragma unroll
    for (int e = 0; e < 8; e++) h[e] = (__bf16)v[e];
    *(uint4*)((__bf16*)p + i) = *(const uint4*)h;
  } else {
    _Float16 h[8];
#pragma unroll
    for (int e = 0; e < 8; e++) h[e] = (_Float16)v[e];
    *(uint4*)((_Float16*)p + i) = *(const uint4*)h;
  }
}

// The elementwise op over eight consecutive innermost elements per thread,
// every tensor of type DT: the output packed within each index of dimension
// 0 (a packed tensor or a join's channel slice), the first input's innermost
// axis contiguous, the second's contiguous or broadcast (stride 0), every
// row start a multiple of eight elements. Index arithmetic once per eight
// elements in 32 bits, 16-byte loads and stores, no type switch per load:
// the generic kernel's per-element 64-bit divisions and typed loads held it
// near 1.2 TB/s on SDXL's GEGLU and broadcast adds.
template <int DT>
__global__ __launch_bounds__(256) void elementwise_vec_kernel(ElemArgs a, int chunks) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= chunks) return;
  const int s3 = (int)a.vo.size[3] >> 3, s2 = (int)a.vo.size[2], s1 = (int)a.vo.size[1];
  int r = c;
  const int i3 = (r % s3) * 8;
  r /= s3;
  const int i2 = r % s2;
  r /= s2;
  const int i1 = r % s1;
  const int i0 = r / s1;
  float x[8], y[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  ld8<DT>(a.in0, offset_of(a.v0, i0, i1, i2, i3), x);
  if (a.in1) {
    const int64_t o1 = offset_of(a.v1, i0, i1, i2, i3);
    if (a.v1.stride[3] == 0) {
      const float b = load_f(a.in1, DT, o1);
#pragma unroll
      for (int e = 0; e < 8; e++) y[e] = b;
    } else {
      ld8<DT>(a.in1, o1, y);
    }
  }
  if (a.op == ELEM_MUL_GELU) {
#pragma unroll
    for (int e = 0; e < 8; e++) y[e] = round_to(gelu_f(y[e]), DT);
  }
  float z[8];
#pragma unroll
  for (int e = 0; e < 8; e++) z[e] = apply_elem(a.op, x[e], y[e], a.scale, a.bias);
  st8<DT>(a.out, offset_of(a.vo, i0, i1, i2, i3), z);
}

// out = in0 (+ in1) where in0 is a token-major [B, H*W, C] tensor viewed as
// [B, C, H, W] (channel stride 1, pixel stride P) and out and in1 are packed
// NCHW: SDXL's ToImage(tokens) + x. A workgroup moves a 64-channel x 64-pixel
// tile through LDS, reading 16 bytes along the channels of each pixel and
// writing 16 bytes along the pixels of each channel; the generic kernel read
// the transposed operand one strided element per thread.
template <typename T>
__global__ __launch_bounds__(256) void transpose_add_kernel(ElemArgs a, int C, int HW, int64_t P) {
  __shared__ __align__(16) T tile[64][64 + 8];  // [pixel][channel], rows padded by 16 bytes
  const int tid = threadIdx.x;
  const int p0 = blockIdx.x * 64, c0 = blockIdx.y * 64, b = blockIdx.z;
  const T* x = (const T*)a.in0 + b * a.v0.stride[0];
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int id = tid + k * 256;        // 512 chunks: 64 pixels x 8 chunks of 8 channels
    const int px = id >> 3, ch = (id & 7) * 8;
    *(uint4*)&tile[px][ch] = *(const uint4*)(x + int64_t(p0 + px) * P + c0 + ch);
  }
  __syncthreads();
  const int64_t obase = (int64_t(b) * C + c0) * HW + p0;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int id = tid + k * 256;        // 512 chunks: 64 channels x 8 chunks of 8 pixels
    const int c = id >> 3, px = (id & 7) * 8;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; e++) v[e] = (float)tile[px + e][c];
    const int64_t o = obase + int64_t(c) * HW + px;
    if (a.in1) {
      const uint4 u = *(const uint4*)((const T*)a.in1 + o);
      const T* y = (const T*)&u;
#pragma unroll
      for (int e = 0; e < 8; e++) v[e] += (float)y[e];
    }
    T r[8];
#pragma unroll
    for (int e = 0; e < 8; e++) r[e] = (T)v[e];
    *(uint4*)((T*)a.out + o) = *(const uint4*)r;
  }
}

static bool vec_view(const View4& v, bool allow_splat) {
  if (allow_splat && v.stride[3] == 0) return true;  // one scalar load per eight outputs
  if (v.stride[3] != 1) return false;
  for (int d = 0; d < 3; d++)
    if (v.stride[d] % 8) return false;
  return true;
}

void launch_elementwise(const ElemArgs& a, hipStream_t s) {
  int64_t total = a.vo.size[0] * a.vo.size[1] * a.vo.size[2] * a.vo.size[3];
  if (total == 0) return;
  const View4& o = a.vo;
  // Rows of the output packed within each index of dimension 0: a packed
  // tensor, or a join's channel slice of an NCHW one.
  const bool inner_packed_out = o.stride[3] == 1 && o.stride[2] == o.size[3] && o.stride[1] == o.size[2] * o.size[3];
  const bool packed_out = inner_packed_out && o.stride[0] == o.size[1] * o.size[2] * o.size[3];
  const int dt = a.dto;
  const int es = dtype_size(dt);
  const bool typed = (dt == NDX_F16 || dt == NDX_BF16 || dt == NDX_F32) && a.dt0 == dt && (!a.in1 || a.dt1 == dt);
  if (typed && inner_packed_out && o.stride[0] % 8 == 0 && o.size[3] % 8 == 0 && total / 8 < (int64_t(1) << 31) && vec_view(a.v0, false) &&
      (!a.in1 || vec_view(a.v1, true)) && (uintptr_t)a.out % 16 == 0 && (uintptr_t)a.in0 % 16 == 0 &&
      (!a.in1 || a.v1.stride[3] == 0 || (uintptr_t)a.in1 % 16 == 0) && es > 0) {
    const int chunks = (int)(total / 8);
    const dim3 g((unsigned)((chunks + 255) / 256));
    if (dt == NDX_F16) hipLaunchKernelGGL((elementwise_vec_kernel<NDX_F16>), g, dim3(256), 0, s, a, chunks);
    else if (dt == NDX_BF16) hipLaunchKernelGGL((elementwise_vec_kernel<NDX_BF16>), g, dim3(256), 0, s, a, chunks);
    else hipLaunchKernelGGL((elementwise_vec_kernel<NDX_F32>), g, dim3(256), 0, s, a, chunks);
    return;
  }
  // The token-major operand of ToImage(tokens) + x.
  const View4& t = a.v0;
  const int64_t C = o.size[1], HW = o.size[2] * o.size[3];
  const bool tr_ok = packed_out && (dt == NDX_F16 || dt == NDX_BF16) && a.dt0 == dt && t.stride[1] == 1 &&
                     t.stride[3] >= C && t.stride[2] == t.stride[3] * o.size[3] && t.stride[3] % 8 == 0 &&
                     t.stride[0] % 8 == 0 && C % 64 == 0 && HW % 64 == 0 && (uintptr_t)a.in0 % 16 == 0 &&
                     (uintptr_t)a.out % 16 == 0 && o.size[0] <= 65535 && C / 64 <= 65535 &&
                     (a.op == ELEM_COPY || (a.op == ELEM_ADD && a.in1 && a.dt1 == dt && (uintptr_t)a.in1 % 16 == 0 &&
                                            a.v1.stride[3] == 1 && a.v1.stride[2] == o.size[3] &&
                                            a.v1.stride[1] == HW && a.v1.stride[0] == C * HW));
  if (tr_ok && (a.op == ELEM_ADD || !a.in1)) {
    const dim3 g((unsigned)(HW / 64), (unsigned)(C / 64), (unsigned)o.size[0]);
    if (dt == NDX_F16) hipLaunchKernelGGL(transpose_add_kernel<_Float16>, g, dim3(256), 0, s, a, (int)C, (int)HW, t.stride[3]);
    else hipLaunchKernelGGL(transpose_add_kernel<__bf16>, g, dim3(256), 0, s, a, (int)C, (int)HW, t.stride[3]);
    return;
  }
  hipLaunchKernelGGL(elementwise_kernel, dim3(grid_for(total, 256)), dim3(256), 0, s, a, total);
}

__global__ void upsample_kernel(UpsampleArgs a, int64_t total) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t step = int64_t(gridDim.x) * blockDim.x;
  const int64_t Wo = a.W * a.scale, Ho = a.H * a.scale;
  for (; i < total; i += step) {
    int64_t r = i;
    int64_t x = r % Wo;
    r /= Wo;
    int64_t y = r % Ho;
    r /= Ho;
    int64_t c = r % a.C;
    int64_t n = r / a.C;
    float v = load_f(a.x, a.dtype, offset_of(a.vx, n, c, y / a.scale, x / a.scale));
    store_f(a.y, a.dtype, i, v);
  }
}

// The 2x case for 16-bit images whose rows are read four pixels (8 bytes)
// at a time: each thread writes the 2x8 output pixels of four input pixels
// as two 16-byte stores.
__global__ void upsample2_vec_kernel(UpsampleArgs a, int64_t total) {
  const int64_t wq = a.W / 4, Wo = a.W * 2, Ho = a.H * 2;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    int64_t r = i;
    const int64_t xq = r % wq;
    r /= wq;
    const int64_t y = r % a.H;
    r /= a.H;
    const int64_t c = r % a.C, n = r / a.C;
    const uint2 u = *(const uint2*)((const uint16_t*)a.x + offset_of(a.vx, n, c, y, xq * 4));
    const uint4 o = make_uint4((u.x & 0xffffu) | (u.x << 16), (u.x >> 16) | (u.x & 0xffff0000u),
                               (u.y & 0xffffu) | (u.y << 16), (u.y >> 16) | (u.y & 0xffff0000u));
    uint16_t* dst = (uint16_t*)a.y + ((n * a.C + c) * Ho + 2 * y) * Wo + 8 * xq;
    *(uint4*)dst = o;
    *(uint4*)(dst + Wo) = o;
  }
}

void launch_upsample(const UpsampleArgs& a, hipStream_t s) {
  const View4& v = a.vx;
  if (a.scale == 2 && dtype_size(a.dtype) == 2 && a.W % 4 == 0 && v.stride[3] == 1 && v.stride[2] % 4 == 0 &&
      v.stride[1] % 4 == 0 && v.stride[0] % 4 == 0 && (uintptr_t)a.x % 8 == 0 && (uintptr_t)a.y % 16 == 0) {
    const int64_t total = a.N * a.C * a.H * (a.W / 4);
    hipLaunchKernelGGL(upsample2_vec_kernel, dim3(grid_for(total, 256)), dim3(256), 0, s, a, total);
    return;
  }
  int64_t total = a.N * a.C * a.H * a.scale * a.W * a.scale;
  hipLaunchKernelGGL(upsample_kernel, dim3(grid_for(total, 256)), dim3(256), 0, s, a, total);
}

// [N, C, H, W] <-> [N, (H/p)(W/p), C p p] with feature order (c, dy, dx),
// or (dy, dx, c) when channel_last.
__global__ void patch_kernel(PatchArgs a, int64_t total) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t step = int64_t(gridDim.x) * blockDim.x;
  const int p = a.p, hp = a.H / p, wp = a.W / p;
  const int64_t feat = int64_t(a.C) * p * p;
  const int64_t per = int64_t(a.C) * a.H * a.W;
  for (; i < total; i += step) {
    // i indexes the token layout.
    int64_t n = i / per, j = i % per;
    int64_t token = j / feat, f = j % feat;
    int64_t ty = token / wp, tx = token % wp;
    int64_t c, dy, dx;
    if (a.channel_last) {
      dy = f / (int64_t(p) * a.C);
      dx = (f / a.C) % p;
      c = f % a.C;
    } else {
      c = f / (p * p);
      dy = (f / p) % p;
      dx = f % p;
    }
    int64_t img = n * per + (c * a.H + ty * p + dy) * a.W + tx * p + dx;
    if (!a.inverse)
      store_f(a.y, a.y_dtype, i, load_f(a.x, a.x_dtype, img));
    else
      store_f(a.y, a.y_dtype, img, load_f(a.x, a.x_dtype, i));
  }
  (void)hp;
}

void launch_patch(const PatchArgs& a, hipStream_t s) {
  int64_t total = int64_t(a.N) * a.C * a.H * a.W;
  hipLaunchKernelGGL(patch_kernel, dim3(grid_for(total, 256)), dim3(256), 0, s, a, total);
}

__global__ void fill_normal_kernel(void* p, int dt, int64_t n, uint64_t seed, float mean, float sd) {
  int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  int64_t step = int64_t(gridDim.x) * blockDim.x;
  for (; i < n; i += step) {
    uint64_t h1 = splitmix64(seed ^ splitmix64(2ull * uint64_t(i)));
    uint64_t h2 = splitmix64(seed ^ splitmix64(2ull * uint64_t(i) + 1ull));
    double u1 = (double((h1 >> 11) + 1ull)) * (1.0 / 9007199254740992.0);  // (0, 1]
    double u2 = double(h2 >> 11) * (1.0 / 9007199254740992.0);            // [0, 1)
    double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
    float v = (float)(double(mean) + double(sd) * z);
    store_f(p, dt, i, v);
  }
}

void launch_fill_normal(void* ptr, int dtype, int64_t n, uint64_t seed, float mean, float std,
                        hipStream_t s) {
  hipLaunchKernelGGL(fill_normal_kernel, dim3(grid_for(n, 256)), dim3(256), 0, s, ptr, dtype, n, seed, mean, std);
}

// One thread per (row, block): the rule of Tensors/BlockQuantizer.cs:55-72.
__global__ void quantize_kernel(const void* w, int wdt, int64_t rows, int64_t cols, int block, int sdt,
                                int8_t* q, void* scales) {
  int64_t blocks = cols / block;
  int64_t id = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (id >= rows * blocks) return;
  int64_t r = id / blocks, b = id % blocks;
  int64_t start = r * cols + b * block;
  float peak = 0.f;
  for (int i = 0; i < block; i++) peak = fmaxf(peak, fabsf(load_f(w, wdt, start + i)));
  float stored;
  if (sdt == NDX_F16) {
    _Float16 h = (_Float16)(peak / 127.0f);
    ((_Float16*)scales)[id] = h;
    stored = (float)h;
  } else {
    stored = peak / 127.0f;
    ((float*)scales)[id] = stored;
  }
  if (stored == 0.f) {
    for (int i = 0; i < block; i++) q[start + i] = 0;
    return;
  }
  float inverse = 1.0f / stored;
  for (int i = 0; i < block; i++) {
    float v = rintf(load_f(w, wdt, start + i) * inverse);
    v = fminf(127.f, fmaxf(-127.f, v));
    q[start + i] = (int8_t)(int)v;
  }
}

void launch_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols, int block, int s_dtype, int8_t* q,
                     void* scales, hipStream_t s) {
  int64_t n = rows * (cols / block);
  int blocks = (int)((n + 255) / 256);
  hipLaunchKernelGGL(quantize_kernel, dim3(blocks), dim3(256), 0, s, w, w_dtype, rows, cols, block, s_dtype, q, scales);
}

// The sampler step with classifier-free guidance, in the reference's float
// arithmetic: p = u + g * (c - u) (GuidanceStrategy.cs:34-44; p = c with no
// unconditional branch), then x + p * (sigma_next - sigma) (EulerScheduler.
// Step, Schedulers.cs:270-279, with FlowPrediction's derivative, the model
// output itself, Prediction.cs:83-84). Each operation is rounded on its own,
// as the C# loops round them: no fused multiply-add. The scalars (g, sigma,
// sigma_next) are read from device memory, so a step changes no launch.
__global__ void guided_euler_kernel(const float* __restrict__ x, const float* __restrict__ u,
                                    const float* __restrict__ c, const float* __restrict__ scalars,
                                    float* __restrict__ out, int64_t n) {
#pragma clang fp contract(off)
  const float g = scalars[0];
  const float delta = scalars[2] - scalars[1];
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += int64_t(gridDim.x) * blockDim.x) {
    float p = c[i];
    if (u) {
      const float diff = p - u[i];
      const float scaled = g * diff;
      p = u[i] + scaled;
    }
    const float step = p * delta;
    out[i] = x[i] + step;
  }
}

void launch_guided_euler(const float* x, const float* u, const float* c, const float* scalars, float* out, int64_t n,
                         hipStream_t s) {
  if (n == 0) return;
  const int blocks = (int)std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(guided_euler_kernel, dim3(blocks), dim3(256), 0, s, x, u, c, scalars, out, n);
}

// LoRA fold (LoraMerge.Merge, Weights/LoraFile.cs:355-420). A thread owns
// one column of ROWS consecutive rows and keeps them widened to fp32 in
// registers; for each pair covering a row and each rank r in order it adds
// (scale * up[row - first, r]) * down[r, col], the product and the sum each
// rounded on their own as the C# vector multiply-add rounds them, and skips a
// zero factor as the reference does; the row is narrowed once at the end.
// A block reads each down row once for its ROWS rows; the up factors are the
// same for every lane, so they come through the scalar unit.
template <int ROWS>
__global__ __launch_bounds__(256) void lora_fold_kernel(LoraFoldArgs a) {
#pragma clang fp contract(off)
  const int64_t col = int64_t(blockIdx.y) * 256 + threadIdx.x;
  const int64_t r0 = int64_t(blockIdx.x) * ROWS;
  if (col >= a.cols) return;
  const int live = (int)min<int64_t>(ROWS, a.rows - r0);
  float acc[ROWS];
#pragma unroll
  for (int i = 0; i < ROWS; i++) acc[i] = i < live ? load_f(a.w, a.w_dtype, (r0 + i) * a.cols + col) : 0.f;
  for (int k = 0; k < a.patches; k++) {
    const LoraPatchArgs& p = a.p[k];
    if (r0 + live <= p.first || r0 >= p.first + p.count) continue;
    for (int r = 0; r < p.rank; r++) {
      const float d = load_f(p.down, p.down_dtype, int64_t(r) * a.cols + col);
#pragma unroll
      for (int i = 0; i < ROWS; i++) {
        const int64_t row = r0 + i;
        if (i >= live || row < p.first || row >= p.first + p.count) continue;
        const float factor = p.scale * load_f(p.up, p.up_dtype, (row - p.first) * p.rank + r);
        if (factor == 0.f) continue;
        const float term = d * factor;
        acc[i] = term + acc[i];
      }
    }
  }
#pragma unroll
  for (int i = 0; i < ROWS; i++)
    if (i < live) store_f(a.out, a.out_dtype, (r0 + i) * a.cols + col, acc[i]);
}

void launch_lora_fold(const LoraFoldArgs& a, hipStream_t s) {
  if (a.rows == 0 || a.cols == 0) return;
  constexpr int R = 16;
  // Row groups on x (up to 2^31 of them), column groups on y.
  const dim3 grid((unsigned)((a.rows + R - 1) / R), (unsigned)((a.cols + 255) / 256));
  hipLaunchKernelGGL(lora_fold_kernel<R>, grid, dim3(256), 0, s, a);
}

}  // namespace ndx
