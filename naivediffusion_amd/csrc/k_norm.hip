// Wavefront-reduction normalisation kernels: LayerNorm (+affine),
// Transformer.Modulate (LayerNorm * (1 + scale) + shift, cast), RMSNorm,
// the same norms over the channels of an NCHW image written as tokens
// (+SiLU), the per-head RMSNorm + rotate-half RoPE of the attention inputs,
// and GroupNorm (+affine, +SiLU).

#include <algorithm>
#include <cstdlib>
#include <stdexcept>

#include "k_common.h"

namespace ndx {

// Offsets of row `within` (of batch `batch`) into the weight and bias: one
// row for all (ld 0), a row per row, or two rows split at `split`.
__device__ __forceinline__ int64_t param_off(int64_t batch, int64_t within, int64_t bstride, int64_t ld, int64_t split,
                                             int64_t split_off) {
  return batch * bstride + within * ld + (within >= split ? split_off : 0);
}

// One 64-lane wave per row; lane l holds elements l, l + 64, ... so every
// load and store of the wave is one contiguous run. VPT values per lane stay
// in registers between the statistics and the output pass.
template <int VPT>
__global__ __launch_bounds__(256) void row_norm_kernel(RowNormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int64_t batch = row / a.rows_per_batch;
  const int64_t within = row % a.rows_per_batch;
  const int64_t xoff = batch * a.batch_x + within * a.ldx;
  const int D = a.D;
  float v[VPT];
#pragma unroll
  for (int j = 0; j < VPT; j++) {
    int c = j * 64 + lane;
    v[j] = c < D ? load_f(a.x, a.x_dtype, xoff + c) : 0.f;
  }
  float mean = 0.f, rstd;
  if (a.mode == 2) {
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < VPT; j++) ss += v[j] * v[j];
    ss = wave_sum(ss);
    rstd = 1.0f / sqrtf(ss / D + a.eps);
  } else {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < VPT; j++) s += v[j];
    mean = wave_sum(s) / D;
    float ss = 0.f;
#pragma unroll
    for (int j = 0; j < VPT; j++) {
      int c = j * 64 + lane;
      float d = c < D ? v[j] - mean : 0.f;
      ss += d * d;
    }
    ss = wave_sum(ss);
    rstd = 1.0f / sqrtf(ss / D + a.eps);
  }
  const int64_t woff = param_off(batch, row % a.rows_per_batch, a.batch_w, a.ldw, a.split, a.split_w_off),
                boff = param_off(batch, row % a.rows_per_batch, a.batch_b, a.ldb, a.split, a.split_b_off);
  const int64_t yoff = row * a.ldy;
#pragma unroll
  for (int j = 0; j < VPT; j++) {
    int c = j * 64 + lane;
    if (c >= D) break;
    float n = (v[j] - mean) * rstd;
    float y;
    if (a.mode == 1) {
      float sc = load_f(a.weight, a.w_dtype, woff + c);
      float sh = a.bias ? load_f(a.bias, a.b_dtype, boff + c) : 0.f;
      y = n * (1.0f + sc) + sh;
    } else {
      y = n;
      if (a.weight) y *= load_f(a.weight, a.w_dtype, woff + c);
      if (a.bias) y += load_f(a.bias, a.b_dtype, boff + c);
    }
    store_f(a.y, a.y_dtype, yoff + c, y);
  }
}

// Large rows: one 256-thread block per row, statistics by block reduction,
// values re-read from memory for the output pass.
__global__ __launch_bounds__(256) void row_norm_wide_kernel(RowNormArgs a) {
  __shared__ float red[2][4];
  const int64_t row = blockIdx.x;
  const int64_t batch = row / a.rows_per_batch;
  const int64_t within = row % a.rows_per_batch;
  const int64_t xoff = batch * a.batch_x + within * a.ldx;
  const int D = a.D, t = threadIdx.x, lane = t & 63, w = t >> 6;
  float s = 0.f, ss = 0.f;
  for (int c = t; c < D; c += 256) {
    float x = load_f(a.x, a.x_dtype, xoff + c);
    s += x;
    ss += x * x;
  }
  s = wave_sum(s);
  ss = wave_sum(ss);
  if (lane == 0) {
    red[0][w] = s;
    red[1][w] = ss;
  }
  __syncthreads();
  s = red[0][0] + red[0][1] + red[0][2] + red[0][3];
  ss = red[1][0] + red[1][1] + red[1][2] + red[1][3];
  float mean = 0.f, rstd;
  if (a.mode == 2) {
    rstd = 1.0f / sqrtf(ss / D + a.eps);
  } else {
    mean = s / D;
    __syncthreads();
    float q = 0.f;
    for (int c = t; c < D; c += 256) {
      float d = load_f(a.x, a.x_dtype, xoff + c) - mean;
      q += d * d;
    }
    q = wave_sum(q);
    if (lane == 0) red[0][w] = q;
    __syncthreads();
    q = red[0][0] + red[0][1] + red[0][2] + red[0][3];
    rstd = 1.0f / sqrtf(q / D + a.eps);
  }
  const int64_t woff = param_off(batch, row % a.rows_per_batch, a.batch_w, a.ldw, a.split, a.split_w_off),
                boff = param_off(batch, row % a.rows_per_batch, a.batch_b, a.ldb, a.split, a.split_b_off);
  for (int c = t; c < D; c += 256) {
    float n = (load_f(a.x, a.x_dtype, xoff + c) - mean) * rstd;
    float y;
    if (a.mode == 1) {
      y = n * (1.0f + load_f(a.weight, a.w_dtype, woff + c)) + (a.bias ? load_f(a.bias, a.b_dtype, boff + c) : 0.f);
    } else {
      y = n;
      if (a.weight) y *= load_f(a.weight, a.w_dtype, woff + c);
      if (a.bias) y += load_f(a.bias, a.b_dtype, boff + c);
    }
    store_f(a.y, a.y_dtype, row * a.ldy + c, y);
  }
}

// Four consecutive elements of a row as floats (fp32: 16 bytes, bf16 or
// f16: 8 bytes); the caller guarantees the alignment.
__device__ __forceinline__ float4 load4(const void* p, int dt, int64_t i) {
  if (dt == NDX_F32) return *(const float4*)((const float*)p + i);
  const uint2 u = *(const uint2*)((const uint16_t*)p + i);
  if (dt == NDX_BF16)
    return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                       __uint_as_float(u.y & 0xffff0000u));
  const _Float16* h = (const _Float16*)&u;
  return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}

__device__ __forceinline__ void store4(void* p, int dt, int64_t i, float4 v) {
  if (dt == NDX_F32) {
    *(float4*)((float*)p + i) = v;
  } else if (dt == NDX_BF16) {
    __bf16 h[4] = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
    *(uint2*)((__bf16*)p + i) = *(const uint2*)h;
  } else {
    _Float16 h[4] = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
    *(uint2*)((_Float16*)p + i) = *(const uint2*)h;
  }
}

// The same three norms with D = 256 * NC: lane l holds the four-element
// chunks l, l + 64, ... (NC of them), so every access is a 16- or 8-byte
// vector and the wave reads one contiguous kilobyte per instruction. PART:
// D a multiple of 4 up to 256 * NC (SDXL's 640-wide rows), the chunks past
// the row neither read nor written.
template <int NC, bool PART = false>
__global__ __launch_bounds__(256) void row_norm_vec_kernel(RowNormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int64_t batch = row / a.rows_per_batch;
  const int64_t xoff = batch * a.batch_x + (row % a.rows_per_batch) * a.ldx;
  const int D = PART ? a.D : NC * 256;
  float4 v[NC];
#pragma unroll
  for (int j = 0; j < NC; j++) {
    const int c = (j * 64 + lane) * 4;
    v[j] = !PART || c < D ? load4(a.x, a.x_dtype, xoff + c) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float mean = 0.f;
  if (a.mode != 2) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NC; j++) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    mean = wave_sum(s) * (1.0f / D);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NC; j++) {
    if (PART && (j * 64 + lane) * 4 >= D) break;
    const float a0 = v[j].x - mean, a1 = v[j].y - mean, a2 = v[j].z - mean, a3 = v[j].w - mean;
    ss += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
  }
  const float rstd = 1.0f / sqrtf(wave_sum(ss) * (1.0f / D) + a.eps);
  const int64_t woff = param_off(batch, row % a.rows_per_batch, a.batch_w, a.ldw, a.split, a.split_w_off),
                boff = param_off(batch, row % a.rows_per_batch, a.batch_b, a.ldb, a.split, a.split_b_off);
  const int64_t yoff = row * a.ldy;
#pragma unroll
  for (int j = 0; j < NC; j++) {
    const int c = (j * 64 + lane) * 4;
    if (PART && c >= D) break;
    float4 n = make_float4((v[j].x - mean) * rstd, (v[j].y - mean) * rstd, (v[j].z - mean) * rstd,
                           (v[j].w - mean) * rstd);
    if (a.mode == 1) {
      const float4 sc = load4(a.weight, a.w_dtype, woff + c);
      const float4 sh = a.bias ? load4(a.bias, a.b_dtype, boff + c) : make_float4(0.f, 0.f, 0.f, 0.f);
      n = make_float4(n.x * (1.0f + sc.x) + sh.x, n.y * (1.0f + sc.y) + sh.y, n.z * (1.0f + sc.z) + sh.z,
                      n.w * (1.0f + sc.w) + sh.w);
    } else {
      if (a.weight) {
        const float4 w = load4(a.weight, a.w_dtype, woff + c);
        n = make_float4(n.x * w.x, n.y * w.y, n.z * w.z, n.w * w.w);
      }
      if (a.bias) {
        const float4 b = load4(a.bias, a.b_dtype, boff + c);
        n = make_float4(n.x + b.x, n.y + b.y, n.z + b.z, n.w + b.w);
      }
    }
    store4(a.y, a.y_dtype, yoff + c, n);
  }
}

// Compile-time-typed loads and stores for the fast row-norm kernel.
template <int DT>
__device__ __forceinline__ float4 load4_t(const void* p, int64_t i) {
  if constexpr (DT == NDX_F32) {
    return *(const float4*)((const float*)p + i);
  } else {
    const uint2 u = *(const uint2*)((const uint16_t*)p + i);
    if constexpr (DT == NDX_BF16) {
      return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u), __uint_as_float(u.y << 16),
                         __uint_as_float(u.y & 0xffff0000u));
    } else {
      const _Float16* h = (const _Float16*)&u;
      return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
    }
  }
}
template <int DT>
__device__ __forceinline__ void store4_t(void* p, int64_t i, float4 v) {
  if constexpr (DT == NDX_F32) {
    *(float4*)((float*)p + i) = v;
  } else if constexpr (DT == NDX_BF16) {
    __bf16 h[4] = {(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
    *(uint2*)((__bf16*)p + i) = *(const uint2*)h;
  } else {
    _Float16 h[4] = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
    *(uint2*)((_Float16*)p + i) = *(const uint2*)h;
  }
}

// row_norm_vec_kernel for fp32 rows and fp32 affine terms (the residual
// stream's norms: Modulate, LayerNorm, RmsNorm) with the output type fixed at
// compile time: the row, the weight and the bias are all requested before
// the statistics are reduced, and nothing in the loops branches on a type,
// so a wave has its whole row and affine terms in flight at once.
template <int NC, int YT>
__global__ __launch_bounds__(256) void row_norm_f32_kernel(RowNormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const int64_t batch = row / a.rows_per_batch;
  const int64_t xoff = batch * a.batch_x + (row % a.rows_per_batch) * a.ldx;
  constexpr int D = NC * 256;
  const int64_t woff = param_off(batch, row % a.rows_per_batch, a.batch_w, a.ldw, a.split, a.split_w_off),
                boff = param_off(batch, row % a.rows_per_batch, a.batch_b, a.ldb, a.split, a.split_b_off);
  float4 v[NC], w[NC], bb[NC];
#pragma unroll
  for (int j = 0; j < NC; j++) v[j] = load4_t<NDX_F32>(a.x, xoff + (j * 64 + lane) * 4);
  const bool hw = a.weight != nullptr, hb = a.bias != nullptr;
#pragma unroll
  for (int j = 0; j < NC; j++) {
    const int c = (j * 64 + lane) * 4;
    w[j] = hw ? load4_t<NDX_F32>(a.weight, woff + c) : make_float4(0.f, 0.f, 0.f, 0.f);
    bb[j] = hb ? load4_t<NDX_F32>(a.bias, boff + c) : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  float mean = 0.f;
  if (a.mode != 2) {
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < NC; j++) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    mean = wave_sum(s) * (1.0f / D);
  }
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < NC; j++) {
    const float a0 = v[j].x - mean, a1 = v[j].y - mean, a2 = v[j].z - mean, a3 = v[j].w - mean;
    ss += (a0 * a0 + a1 * a1) + (a2 * a2 + a3 * a3);
  }
  const float rstd = 1.0f / sqrtf(wave_sum(ss) * (1.0f / D) + a.eps);
  const int64_t yoff = row * a.ldy;
  // Modulate scales by (1 + scale); the others by the weight when there is one.
  const float w1 = a.mode == 1 ? 1.0f : 0.0f;
#pragma unroll
  for (int j = 0; j < NC; j++) {
    const int c = (j * 64 + lane) * 4;
    float4 n = make_float4((v[j].x - mean) * rstd, (v[j].y - mean) * rstd, (v[j].z - mean) * rstd,
                           (v[j].w - mean) * rstd);
    if (hw) n = make_float4(n.x * (w1 + w[j].x), n.y * (w1 + w[j].y), n.z * (w1 + w[j].z), n.w * (w1 + w[j].w));
    if (hb) n = make_float4(n.x + bb[j].x, n.y + bb[j].y, n.z + bb[j].z, n.w + bb[j].w);
    store4_t<YT>(a.y, yoff + c, n);
  }
}

static bool vec_ok(const void* p, int dt, int64_t ld, int64_t batch) {
  if (!p) return true;
  const int es = dtype_size(dt);
  if (dt != NDX_F32 && dt != NDX_BF16 && dt != NDX_F16) return false;
  const int need = dt == NDX_F32 ? 16 : 8;
  return (uintptr_t)p % need == 0 && (ld * es) % need == 0 && (batch * es) % need == 0;
}

void launch_row_norm(const RowNormArgs& a, hipStream_t s) {
  if (a.rows == 0) return;
  int vpt = (a.D + 63) / 64;
  dim3 grid((unsigned)((a.rows + 3) / 4)), block(256);
  const bool vec = a.D % 256 == 0 && a.D <= 4096 && vec_ok(a.x, a.x_dtype, a.ldx, a.batch_x) &&
                   vec_ok(a.y, a.y_dtype, a.ldy, 0) && vec_ok(a.weight, a.w_dtype, a.ldw, a.batch_w) && vec_ok(a.weight, a.w_dtype, 0, a.split_w_off) &&
                   vec_ok(a.bias, a.b_dtype, a.ldb, a.batch_b) && vec_ok(a.bias, a.b_dtype, 0, a.split_b_off);
  const bool f32_terms = a.x_dtype == NDX_F32 && (!a.weight || a.w_dtype == NDX_F32) &&
                         (!a.bias || a.b_dtype == NDX_F32);
  if (vec && f32_terms && (a.D == 2048 || a.D == 3072 || a.D == 4096)) {
#define NDX_RN(NC)                                                                                        \
  do {                                                                                                    \
    if (a.y_dtype == NDX_BF16) hipLaunchKernelGGL((row_norm_f32_kernel<NC, NDX_BF16>), grid, block, 0, s, a); \
    else if (a.y_dtype == NDX_F16) hipLaunchKernelGGL((row_norm_f32_kernel<NC, NDX_F16>), grid, block, 0, s, a); \
    else hipLaunchKernelGGL((row_norm_f32_kernel<NC, NDX_F32>), grid, block, 0, s, a);                       \
  } while (0)
    if (a.D == 2048) NDX_RN(8);
    else if (a.D == 3072) NDX_RN(12);
    else NDX_RN(16);
#undef NDX_RN
    return;
  }
  if (vec) {
    switch (a.D / 256) {
      case 1: hipLaunchKernelGGL(row_norm_vec_kernel<1>, grid, block, 0, s, a); return;
      case 2: hipLaunchKernelGGL(row_norm_vec_kernel<2>, grid, block, 0, s, a); return;
      case 3: hipLaunchKernelGGL(row_norm_vec_kernel<3>, grid, block, 0, s, a); return;
      case 4: hipLaunchKernelGGL(row_norm_vec_kernel<4>, grid, block, 0, s, a); return;
      case 5: hipLaunchKernelGGL(row_norm_vec_kernel<5>, grid, block, 0, s, a); return;
      case 6: hipLaunchKernelGGL(row_norm_vec_kernel<6>, grid, block, 0, s, a); return;
      case 8: hipLaunchKernelGGL(row_norm_vec_kernel<8>, grid, block, 0, s, a); return;
      case 10: hipLaunchKernelGGL(row_norm_vec_kernel<10>, grid, block, 0, s, a); return;
      case 12: hipLaunchKernelGGL(row_norm_vec_kernel<12>, grid, block, 0, s, a); return;
      case 16: hipLaunchKernelGGL(row_norm_vec_kernel<16>, grid, block, 0, s, a); return;
      default: break;
    }
  }
  const bool part = a.D % 4 == 0 && a.D % 256 != 0 && a.D < 2048 && vec_ok(a.x, a.x_dtype, a.ldx, a.batch_x) &&
                    vec_ok(a.y, a.y_dtype, a.ldy, 0) && vec_ok(a.weight, a.w_dtype, a.ldw, a.batch_w) && vec_ok(a.weight, a.w_dtype, 0, a.split_w_off) &&
                    vec_ok(a.bias, a.b_dtype, a.ldb, a.batch_b) && vec_ok(a.bias, a.b_dtype, 0, a.split_b_off);
  if (part) {
    switch ((a.D + 255) / 256) {
      case 1: hipLaunchKernelGGL((row_norm_vec_kernel<1, true>), grid, block, 0, s, a); return;
      case 2: hipLaunchKernelGGL((row_norm_vec_kernel<2, true>), grid, block, 0, s, a); return;
      case 3: hipLaunchKernelGGL((row_norm_vec_kernel<3, true>), grid, block, 0, s, a); return;
      case 4: hipLaunchKernelGGL((row_norm_vec_kernel<4, true>), grid, block, 0, s, a); return;
      case 5: hipLaunchKernelGGL((row_norm_vec_kernel<5, true>), grid, block, 0, s, a); return;
      case 6: hipLaunchKernelGGL((row_norm_vec_kernel<6, true>), grid, block, 0, s, a); return;
      case 7: hipLaunchKernelGGL((row_norm_vec_kernel<7, true>), grid, block, 0, s, a); return;
      case 8: hipLaunchKernelGGL((row_norm_vec_kernel<8, true>), grid, block, 0, s, a); return;
      default: break;
    }
  }
  if (vpt <= 4) hipLaunchKernelGGL(row_norm_kernel<4>, grid, block, 0, s, a);
  else if (vpt <= 8) hipLaunchKernelGGL(row_norm_kernel<8>, grid, block, 0, s, a);
  else if (vpt <= 16) hipLaunchKernelGGL(row_norm_kernel<16>, grid, block, 0, s, a);
  else if (vpt <= 32) hipLaunchKernelGGL(row_norm_kernel<32>, grid, block, 0, s, a);
  else if (vpt <= 48) hipLaunchKernelGGL(row_norm_kernel<48>, grid, block, 0, s, a);
  else if (vpt <= 64) hipLaunchKernelGGL(row_norm_kernel<64>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(row_norm_wide_kernel, dim3((unsigned)a.rows), block, 0, s, a);
}

// The row norm of the token view of a packed NCHW image, written as packed
// tokens. A workgroup owns 64 pixels of one image; lane l of every wave
// holds pixel l, so each load of a wave is 64 consecutive pixels of one
// channel. Pass 1: wave w sums channels w, w + 4, ... and the four partial
// sums meet in LDS (a LayerNorm re-reads for the squared deviations). Pass 2
// re-reads 64-channel slabs, normalises them into an LDS tile
// [pixel][channel], and writes each pixel's slab as one contiguous run.
__global__ __launch_bounds__(256) void channel_norm_kernel(ChannelNormArgs a) {
  __shared__ float red[2][4][64];
  __shared__ float tile[64][65];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int64_t C = a.C, P = a.P;
  const int64_t n = blockIdx.y, p0 = int64_t(blockIdx.x) * 64, p = p0 + lane;
  const bool live = p < P;
  const int64_t xb = n * C * P + p;
  float s = 0.f, ss = 0.f;
  if (live) {
#pragma unroll 8
    for (int64_t c = w; c < C; c += 4) {
      const float v = load_f(a.x, a.x_dtype, xb + c * P);
      s += v;
      ss += v * v;
    }
  }
  red[0][w][lane] = s;
  red[1][w][lane] = ss;
  __syncthreads();
  s = red[0][0][lane] + red[0][1][lane] + red[0][2][lane] + red[0][3][lane];
  ss = red[1][0][lane] + red[1][1][lane] + red[1][2][lane] + red[1][3][lane];
  float mean = 0.f, rstd;
  if (a.mode == 2) {
    rstd = 1.0f / sqrtf(ss / C + a.eps);
  } else {
    mean = s / C;
    float q = 0.f;
    if (live) {
#pragma unroll 8
      for (int64_t c = w; c < C; c += 4) {
        const float d = load_f(a.x, a.x_dtype, xb + c * P) - mean;
        q += d * d;
      }
    }
    __syncthreads();
    red[0][w][lane] = q;
    __syncthreads();
    q = red[0][0][lane] + red[0][1][lane] + red[0][2][lane] + red[0][3][lane];
    rstd = 1.0f / sqrtf(q / C + a.eps);
  }
  const int64_t yb = (n * P + p0) * C;
  for (int64_t c0 = 0; c0 < C; c0 += 64) {
#pragma unroll 4
    for (int j = w; j < 64; j += 4) {
      const int64_t c = c0 + j;
      float y = 0.f;
      if (live && c < C) {
        y = (load_f(a.x, a.x_dtype, xb + c * P) - mean) * rstd;
        if (a.weight) y *= load_f(a.weight, a.w_dtype, c);
        if (a.bias) y += load_f(a.bias, a.b_dtype, c);
        if (a.silu) y = silu_f(round_to(y, a.y_dtype));
      }
      tile[lane][j] = y;
    }
    __syncthreads();
    const int64_t cols = C - c0 < 64 ? C - c0 : 64;
    for (int i = threadIdx.x; i < 64 * 64; i += 256) {
      const int px = i >> 6, cc = i & 63;
      if (cc < cols && p0 + px < P) store_f(a.y, a.y_dtype, yb + px * C + c0 + cc, tile[px][cc]);
    }
    __syncthreads();
  }
}

// Eight 16-bit values from 16 bytes, as floats.
template <typename T>
__device__ __forceinline__ void unpack8(const uint4 u, float v[8]) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if constexpr (__is_same(T, __bf16)) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    } else {
      const _Float16* h = (const _Float16*)&w[i];
      v[2 * i] = (float)h[0];
      v[2 * i + 1] = (float)h[1];
    }
  }
}

template <typename T>
__device__ __forceinline__ float half_to_f(uint16_t h) {
  if constexpr (__is_same(T, __bf16)) return bf16_bits_to_f32(h);
  else return (float)__builtin_bit_cast(_Float16, h);
}

// channel_norm_kernel for 16-bit images whose channels and pixels are
// multiples of 8, with 16-byte accesses on both sides. A workgroup of
// THREADS owns 64 pixels; thread t holds the eight pixels 8 (t % 8) ..
// 8 (t % 8) + 7 and the channels t / 8 + ROWS r (ROWS = THREADS / 8 rows a
// pass), so eight lanes read one channel's 128 contiguous bytes and a wave
// eight channels per load. With RPT > 0 (RMSNorm, C <= ROWS RPT) a thread
// keeps its RPT channel rows in registers from the statistics to the
// output and the image is read once; with RPT = 0 it is read again (and a
// LayerNorm a third time, for the squared deviations). The statistics meet
// across a pixel group's lanes by shuffles and across the waves in LDS; the
// output pass stages ROWS-channel slabs in LDS [channel][pixel] and writes
// eight channels of a pixel per 16-byte store.
template <typename T, int RPT, int THREADS>
__global__ __launch_bounds__(THREADS) void channel_norm_vec_kernel(ChannelNormArgs a) {
  constexpr int WAVES = THREADS / 64, ROWS = THREADS / 8, PER_PX = ROWS / 8;
  __shared__ float red[2][WAVES][64];
  __shared__ float stat[2][64];
  // RPT > 0: the whole block [channel][pixel]; else one ROWS-channel slab.
  __shared__ __align__(16) uint16_t tile[RPT > 0 ? RPT * ROWS : ROWS][66];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, g = t & 7, row = t >> 3;
  const int64_t C = a.C, P = a.P;
  const int64_t n = blockIdx.y, p0 = int64_t(blockIdx.x) * 64;
  const bool live = p0 + 8 * g < P;  // P is a multiple of 8: a group is whole or past the end
  const T* x = (const T*)a.x + n * C * P + p0 + 8 * g;
  auto load_row = [&](int64_t c) {
    return live && c < C ? *(const uint4*)(x + c * P) : make_uint4(0, 0, 0, 0);
  };

  // Sums of the eight pixels over this wave's lanes that hold them, then
  // into red[which][wave].
  auto reduce_groups = [&](float v[8], int which) {
#pragma unroll
    for (int e = 0; e < 8; e++)
#pragma unroll
      for (int o = 8; o < 64; o <<= 1) v[e] += __shfl_xor(v[e], o, 64);
    if (lane < 8)
#pragma unroll
      for (int e = 0; e < 8; e++) red[which][w][8 * lane + e] = v[e];
  };
  auto total = [&](int which) {
    float v = 0.f;
#pragma unroll
    for (int i = 0; i < WAVES; i++) v += red[which][i][t];
    return v;
  };

  uint4 keep[RPT > 0 ? RPT : 1];
  if constexpr (RPT > 0) {
#pragma unroll
    for (int r = 0; r < RPT; r++) keep[r] = load_row(row + ROWS * r);
  }
  float s[8], ss[8];
#pragma unroll
  for (int e = 0; e < 8; e++) s[e] = ss[e] = 0.f;
  auto accumulate = [&](const uint4 u) {
    float v[8];
    unpack8<T>(u, v);
#pragma unroll
    for (int e = 0; e < 8; e++) {
      s[e] += v[e];
      ss[e] += v[e] * v[e];
    }
  };
  if constexpr (RPT > 0) {
#pragma unroll
    for (int r = 0; r < RPT; r++) accumulate(keep[r]);  // rows past C hold zeros
  } else if (live) {
#pragma unroll 4
    for (int64_t c = row; c < C; c += ROWS) accumulate(*(const uint4*)(x + c * P));
  }
  reduce_groups(s, 0);
  reduce_groups(ss, 1);
  __syncthreads();
  if (t < 64) {
    stat[0][t] = a.mode == 2 ? 0.f : total(0) / C;
    stat[1][t] = 1.0f / sqrtf(total(1) / C + a.eps);
  }
  __syncthreads();
  if constexpr (RPT == 0) {
    if (a.mode != 2) {
      // LayerNorm: the squared deviations from the mean.
      float m[8], q[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        m[e] = stat[0][8 * g + e];
        q[e] = 0.f;
      }
      if (live) {
#pragma unroll 4
        for (int64_t c = row; c < C; c += ROWS) {
          float v[8];
          unpack8<T>(*(const uint4*)(x + c * P), v);
#pragma unroll
          for (int e = 0; e < 8; e++) q[e] += (v[e] - m[e]) * (v[e] - m[e]);
        }
      }
      reduce_groups(q, 0);
      __syncthreads();
      if (t < 64) stat[1][t] = 1.0f / sqrtf(total(0) / C + a.eps);
      __syncthreads();
    }
  }

  // Channels c0 .. c0 + ROWS - 1, thread row `row` holding u.
  T* y = (T*)a.y + (n * P + p0) * C;
  auto slab = [&](int64_t c0, const uint4 u) {
    uint32_t* d = (uint32_t*)&tile[row][8 * g];
    d[0] = u.x;
    d[1] = u.y;
    d[2] = u.z;
    d[3] = u.w;
    __syncthreads();
    const int px = t / PER_PX, cc = (t % PER_PX) * 8;
    const int64_t c = c0 + cc;
    if (c < C && p0 + px < P) {
      const float mean = stat[0][px], rstd = stat[1][px];
      __align__(16) T out[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        float v = (half_to_f<T>(tile[cc + e][px]) - mean) * rstd;
        if (a.weight) v *= load_f(a.weight, a.w_dtype, c + e);
        if (a.bias) v += load_f(a.bias, a.b_dtype, c + e);
        if (a.silu) v = silu_f((float)(T)v);
        out[e] = (T)v;
      }
      *(uint4*)(y + px * C + c) = *(const uint4*)out;
    }
    __syncthreads();
  };
  if constexpr (RPT > 0) {
    // The block's rows into LDS at once, then its 64 pixels x C outputs,
    // one contiguous run of the tokens, written in 16-byte pieces: every
    // cache line whole, one barrier. The weight and bias go to LDS as fp32
    // first (each output piece reads eight of them).
    __shared__ float wb[2][RPT * ROWS];
    for (int c = t; c < C; c += THREADS) {
      wb[0][c] = a.weight ? load_f(a.weight, a.w_dtype, c) : 1.f;
      wb[1][c] = a.bias ? load_f(a.bias, a.b_dtype, c) : 0.f;
    }
#pragma unroll
    for (int r = 0; r < RPT; r++) {
      uint32_t* d = (uint32_t*)&tile[row + ROWS * r][8 * g];
      d[0] = keep[r].x;
      d[1] = keep[r].y;
      d[2] = keep[r].z;
      d[3] = keep[r].w;
    }
    __syncthreads();
    const int64_t pieces = min(int64_t(64), P - p0) * C / 8;
    for (int64_t i = t; i < pieces; i += THREADS) {
      const int px = (int)(i * 8 / C), c = (int)(i * 8 - int64_t(px) * C);
      const float mean = stat[0][px], rstd = stat[1][px];
      __align__(16) T out[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        float v = (half_to_f<T>(tile[c + e][px]) - mean) * rstd * wb[0][c + e] + wb[1][c + e];
        if (a.silu) v = silu_f((float)(T)v);
        out[e] = (T)v;
      }
      *(uint4*)(y + i * 8) = *(const uint4*)out;
    }
  } else {
    for (int64_t c0 = 0; c0 < C; c0 += ROWS) slab(c0, load_row(c0 + row));
  }
}

void launch_channel_norm(const ChannelNormArgs& a, hipStream_t s) {
  if (a.N == 0 || a.P == 0 || a.C == 0) return;
  if (a.N > 65535 || a.mode == 1) throw std::runtime_error("channel_norm: up to 65535 images, LayerNorm or RMSNorm");
  dim3 grid((unsigned)((a.P + 63) / 64), (unsigned)a.N);
  const bool half = (a.x_dtype == NDX_BF16 || a.x_dtype == NDX_F16) && a.y_dtype == a.x_dtype;
  if (half && a.C % 8 == 0 && a.P % 8 == 0 && (uintptr_t)a.x % 16 == 0 && (uintptr_t)a.y % 16 == 0) {
#define NDX_CHANNEL_NORM(RPT, THREADS)                                                                        \
  do {                                                                                                       \
    if (a.x_dtype == NDX_BF16)                                                                               \
      hipLaunchKernelGGL((channel_norm_vec_kernel<__bf16, RPT, THREADS>), grid, dim3(THREADS), 0, s, a);      \
    else                                                                                                     \
      hipLaunchKernelGGL((channel_norm_vec_kernel<_Float16, RPT, THREADS>), grid, dim3(THREADS), 0, s, a);    \
    return;                                                                                                  \
  } while (0)
    // An RMSNorm keeps each thread's rows in registers: up to ten 16-byte
    // rows, the workgroup widened to 512 threads for wider images. Wider
    // still, 1024 threads re-read (ten rows would not fit their registers).
    if (a.mode == 2) {
      if (a.C <= 64) NDX_CHANNEL_NORM(2, 256);
      if (a.C <= 128) NDX_CHANNEL_NORM(4, 256);
      if (a.C <= 192) NDX_CHANNEL_NORM(6, 256);
      if (a.C <= 320) NDX_CHANNEL_NORM(10, 256);
      if (a.C <= 640) NDX_CHANNEL_NORM(10, 512);
    }
    if (a.C > 320) NDX_CHANNEL_NORM(0, 1024);
    NDX_CHANNEL_NORM(0, 256);
#undef NDX_CHANNEL_NORM
  }
  hipLaunchKernelGGL(channel_norm_kernel, grid, dim3(256), 0, s, a);
}

// One wave per (batch, token, head): RMSNorm of the head's d features with
// the weight, rounded to the input's type (the HeadNorm output,
// Graph/Transformer.cs:37-43), then the rotate-half rotation in fp32
// (Graph/Transformer.cs:50-64) and the cast to the output type. Lane l owns
// the pairs (i, i + d/2) for i = l, l + 64, ...
__global__ __launch_bounds__(256) void head_norm_rotate_kernel(HeadNormRotateArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t item = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int64_t total = int64_t(a.B) * a.T * a.H;
  if (item >= total) return;
  const int head = (int)(item % a.H);
  const int64_t bt = item / a.H;
  const int t = (int)(bt % a.T);
  const int64_t b = bt / a.T;
  const int half = a.d / 2;
  const int64_t xo = b * a.batch_x + int64_t(t) * a.ldx + int64_t(head) * a.d;
  const int64_t yo = b * a.batch_y + int64_t(t) * a.ldy + int64_t(head) * a.d;
  float lo[2], hi[2];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    int i = lane + k * 64;
    lo[k] = hi[k] = 0.f;
    if (i < half) {
      lo[k] = load_f(a.x, a.x_dtype, xo + i);
      hi[k] = load_f(a.x, a.x_dtype, xo + i + half);
      ss += lo[k] * lo[k] + hi[k] * hi[k];
    }
  }
  ss = wave_sum(ss);
  const float r = 1.0f / sqrtf(ss / a.d + a.eps);
#pragma unroll
  for (int k = 0; k < 2; k++) {
    int i = lane + k * 64;
    if (i >= half) continue;
    float wl = a.weight ? load_f(a.weight, a.w_dtype, i) : 1.f;
    float wh = a.weight ? load_f(a.weight, a.w_dtype, i + half) : 1.f;
    float l = round_to(lo[k] * r * wl, a.x_dtype);
    float h = round_to(hi[k] * r * wh, a.x_dtype);
    if (a.cos) {
      float c = a.cos[int64_t(t) * half + i], s = a.sin[int64_t(t) * half + i];
      float nl = l * c - h * s;
      float nh = h * c + l * s;
      l = nl;
      h = nh;
    }
    store_f(a.y, a.y_dtype, yo + i, l);
    store_f(a.y, a.y_dtype, yo + i + half, h);
  }
}

// d = 128: 16 lanes per (token, head); lane i of the group owns the four
// pairs (4i .. 4i+3, 64 + 4i .. 64 + 4i + 3), read and written as vectors.
__global__ __launch_bounds__(256) void head_norm_rotate128_kernel(HeadNormRotateArgs a) {
  const int lane = threadIdx.x & 15;
  const int64_t item = int64_t(blockIdx.x) * 16 + (threadIdx.x >> 4);
  const int64_t total = int64_t(a.B) * a.T * a.H;
  if (item >= total) return;
  const int head = (int)(item % a.H);
  const int64_t bt = item / a.H;
  const int t = (int)(bt % a.T);
  const int64_t b = bt / a.T;
  const int64_t xo = b * a.batch_x + int64_t(t) * a.ldx + int64_t(head) * 128;
  const int64_t yo = b * a.batch_y + int64_t(t) * a.ldy + int64_t(head) * 128;
  const int i = lane * 4;
  float4 lo = load4(a.x, a.x_dtype, xo + i), hi = load4(a.x, a.x_dtype, xo + 64 + i);
  float ss = (lo.x * lo.x + lo.y * lo.y) + (lo.z * lo.z + lo.w * lo.w) + (hi.x * hi.x + hi.y * hi.y) +
             (hi.z * hi.z + hi.w * hi.w);
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 16);
  const float r = 1.0f / sqrtf(ss * (1.0f / 128) + a.eps);
  float4 wl = make_float4(1.f, 1.f, 1.f, 1.f), wh = wl;
  if (a.weight) {
    wl = make_float4(load_f(a.weight, a.w_dtype, i), load_f(a.weight, a.w_dtype, i + 1),
                     load_f(a.weight, a.w_dtype, i + 2), load_f(a.weight, a.w_dtype, i + 3));
    wh = make_float4(load_f(a.weight, a.w_dtype, 64 + i), load_f(a.weight, a.w_dtype, 65 + i),
                     load_f(a.weight, a.w_dtype, 66 + i), load_f(a.weight, a.w_dtype, 67 + i));
  }
  const int xd = a.x_dtype;
  float l[4] = {round_to(lo.x * r * wl.x, xd), round_to(lo.y * r * wl.y, xd), round_to(lo.z * r * wl.z, xd),
                round_to(lo.w * r * wl.w, xd)};
  float h[4] = {round_to(hi.x * r * wh.x, xd), round_to(hi.y * r * wh.y, xd), round_to(hi.z * r * wh.z, xd),
                round_to(hi.w * r * wh.w, xd)};
  if (a.cos) {
    const float4 c = *(const float4*)(a.cos + int64_t(t) * 64 + i);
    const float4 sn = *(const float4*)(a.sin + int64_t(t) * 64 + i);
    const float cc[4] = {c.x, c.y, c.z, c.w}, sv[4] = {sn.x, sn.y, sn.z, sn.w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const float nl = l[e] * cc[e] - h[e] * sv[e];
      const float nh = h[e] * cc[e] + l[e] * sv[e];
      l[e] = nl;
      h[e] = nh;
    }
  }
  store4(a.y, a.y_dtype, yo + i, make_float4(l[0], l[1], l[2], l[3]));
  store4(a.y, a.y_dtype, yo + 64 + i, make_float4(h[0], h[1], h[2], h[3]));
}

// Eight consecutive elements, widened to fp32 (16-bit types: one 16-byte load).
template <int DT>
__device__ __forceinline__ void load8_t(const void* p, int64_t i, float (&o)[8]) {
  if constexpr (DT == NDX_F32) {
    const float4 a = *(const float4*)((const float*)p + i), b = *(const float4*)((const float*)p + i + 4);
    o[0] = a.x; o[1] = a.y; o[2] = a.z; o[3] = a.w; o[4] = b.x; o[5] = b.y; o[6] = b.z; o[7] = b.w;
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
__device__ __forceinline__ void store8_t(void* p, int64_t i, const float (&v)[8]) {
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
template <int DT>
__device__ __forceinline__ float round_t(float v) {
  if constexpr (DT == NDX_BF16) return (float)(__bf16)v;
  else if constexpr (DT == NDX_F16) return (float)(_Float16)v;
  else return v;
}

// d = 128 with the element types fixed at compile time (x and y of one type
// T, the weight of type WT, or WT = -1 for none): 8 lanes per (token, head), lane i
// owning the pairs (8i .. 8i+7, 64 + 8i .. 64 + 8i + 7), so every load and
// store is 16 bytes and no load waits on a type switch. Twice the bandwidth
// of the 16-lane form on the MMDiT's q and k.
template <int T, int WT>
__global__ __launch_bounds__(256) void head_norm_rotate128_t_kernel(HeadNormRotateArgs a) {
  const int lane = threadIdx.x & 7;
  const int64_t item = int64_t(blockIdx.x) * 32 + (threadIdx.x >> 3);
  const int64_t total = int64_t(a.B) * a.T * a.H;
  if (item >= total) return;
  const int head = (int)(item % a.H);
  const int64_t bt = item / a.H;
  const int t = (int)(bt % a.T);
  const int64_t b = bt / a.T;
  const int64_t xo = b * a.batch_x + int64_t(t) * a.ldx + int64_t(head) * 128;
  const int64_t yo = b * a.batch_y + int64_t(t) * a.ldy + int64_t(head) * 128;
  const int i = lane * 8;
  float lo[8], hi[8], wl[8], wh[8];
  load8_t<T>(a.x, xo + i, lo);
  load8_t<T>(a.x, xo + 64 + i, hi);
  if constexpr (WT >= 0) {
    load8_t<WT>(a.weight, i, wl);
    load8_t<WT>(a.weight, 64 + i, wh);
  }
  float4 c0 = make_float4(1.f, 1.f, 1.f, 1.f), c1 = c0, s0 = make_float4(0.f, 0.f, 0.f, 0.f), s1 = s0;
  if (a.cos) {
    c0 = *(const float4*)(a.cos + int64_t(t) * 64 + i);
    c1 = *(const float4*)(a.cos + int64_t(t) * 64 + i + 4);
    s0 = *(const float4*)(a.sin + int64_t(t) * 64 + i);
    s1 = *(const float4*)(a.sin + int64_t(t) * 64 + i + 4);
  }
  float ss = 0.f;
#pragma unroll
  for (int e = 0; e < 8; e++) ss += lo[e] * lo[e] + hi[e] * hi[e];
#pragma unroll
  for (int o = 4; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 8);
  const float r = 1.0f / sqrtf(ss * (1.0f / 128) + a.eps);
  const float cc[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
  float yl[8], yh[8];
#pragma unroll
  for (int e = 0; e < 8; e++) {
    const float l = round_t<T>(lo[e] * r * (WT >= 0 ? wl[e] : 1.f));
    const float h = round_t<T>(hi[e] * r * (WT >= 0 ? wh[e] : 1.f));
    yl[e] = l * cc[e] - h * sv[e];
    yh[e] = h * cc[e] + l * sv[e];
  }
  store8_t<T>(a.y, yo + i, yl);
  store8_t<T>(a.y, yo + 64 + i, yh);
}

void launch_head_norm_rotate(const HeadNormRotateArgs& a, hipStream_t s) {
  int64_t total = int64_t(a.B) * a.T * a.H;
  if (total == 0) return;
  const bool typed16 = a.d == 128 && a.x_dtype == a.y_dtype && (a.x_dtype == NDX_BF16 || a.x_dtype == NDX_F16) &&
                       (uintptr_t)a.x % 16 == 0 && (a.ldx * 2) % 16 == 0 && (a.batch_x * 2) % 16 == 0 &&
                       (uintptr_t)a.y % 16 == 0 && (a.ldy * 2) % 16 == 0 && (a.batch_y * 2) % 16 == 0 &&
                       (!a.weight || ((uintptr_t)a.weight % 16 == 0 &&
                                      (a.w_dtype == a.x_dtype || a.w_dtype == NDX_F32))) &&
                       (!a.cos || ((uintptr_t)a.cos % 16 == 0 && (uintptr_t)a.sin % 16 == 0));
  if (typed16) {
    const dim3 g((unsigned)((total + 31) / 32));
#define NDX_HNR(T)                                                                                    \
  do {                                                                                                \
    if (!a.weight) hipLaunchKernelGGL((head_norm_rotate128_t_kernel<T, -1>), g, dim3(256), 0, s, a);   \
    else if (a.w_dtype == NDX_F32) hipLaunchKernelGGL((head_norm_rotate128_t_kernel<T, NDX_F32>), g, dim3(256), 0, s, a); \
    else hipLaunchKernelGGL((head_norm_rotate128_t_kernel<T, T>), g, dim3(256), 0, s, a);            \
  } while (0)
    if (a.x_dtype == NDX_BF16) NDX_HNR(NDX_BF16);
    else NDX_HNR(NDX_F16);
#undef NDX_HNR
    return;
  }
  if (a.d == 128 && vec_ok(a.x, a.x_dtype, a.ldx, a.batch_x) && vec_ok(a.y, a.y_dtype, a.ldy, a.batch_y) &&
      (!a.cos || ((uintptr_t)a.cos % 16 == 0 && (uintptr_t)a.sin % 16 == 0))) {
    hipLaunchKernelGGL(head_norm_rotate128_kernel, dim3((unsigned)((total + 15) / 16)), dim3(256), 0, s, a);
    return;
  }
  hipLaunchKernelGGL(head_norm_rotate_kernel, dim3((unsigned)((total + 3) / 4)), dim3(256), 0, s, a);
}

// GroupNorm over NCHW: one 1024-thread block per (n, group), two passes for
// the statistics (mean, then the centred sum of squares) and one for the
// output with the per-channel affine and the optional SiLU.
// GroupNorm in two launches so every CU has work: `splits` workgroups per
// (n, group) each reduce one contiguous chunk of the group to (count, mean,
// M2) (two passes over the chunk, which stays in cache), then each
// workgroup of the apply pass combines its group's partials (Chan et al.'s
// pairwise update) and normalises one chunk, with the per-channel affine
// and the optional SiLU.
int group_norm_splits(int64_t count) {
  int64_t s = (count + 8191) / 8192;
  return (int)std::max<int64_t>(1, std::min<int64_t>(s, 64));
}

// Chunk `split` of a group's count elements: a multiple of 4 long, so the
// chunks keep the 4-element alignment of the group's start.
__device__ __forceinline__ void gn_chunk(const GroupNormArgs& a, int64_t count, int split, int64_t& lo,
                                         int64_t& hi) {
  const int64_t per = ((count + a.splits - 1) / a.splits + 3) & ~int64_t(3);
  lo = min(count, int64_t(split) * per);
  hi = min(count, lo + per);
}

__device__ __forceinline__ float block_sum_256(float v, float* red) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  v = wave_sum(v);
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void group_norm_stats_kernel(GroupNormArgs a) {
  __shared__ float red[4];
  const int ng = blockIdx.x, split = blockIdx.y;
  const int n = ng / a.groups, g = ng % a.groups;
  const int cpg = a.C / a.groups;
  const int64_t count = int64_t(cpg) * a.HW;
  const int64_t base = (int64_t(n) * a.C + int64_t(g) * cpg) * a.HW;
  int64_t lo, hi;
  gn_chunk(a, count, split, lo, hi);
  // Four elements per thread and step when the chunk and the rows allow
  // 4-element vector access (a uniform choice).
  const bool vec = (uintptr_t)a.x % 16 == 0 && ((base + lo) & 3) == 0 && ((hi - lo) & 3) == 0;
  float s = 0.f;
  if (vec) {
    for (int64_t i = lo + 4 * threadIdx.x; i < hi; i += 1024) {
      const float4 v = load4(a.x, a.dtype, base + i);
      s += (v.x + v.y) + (v.z + v.w);
    }
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256) s += load_f(a.x, a.dtype, base + i);
  }
  const float cnt = float(hi - lo);
  const float mean = cnt > 0 ? block_sum_256(s, red) / cnt : 0.f;
  float q = 0.f;
  if (vec) {
    for (int64_t i = lo + 4 * threadIdx.x; i < hi; i += 1024) {
      const float4 v = load4(a.x, a.dtype, base + i);
      const float d0 = v.x - mean, d1 = v.y - mean, d2 = v.z - mean, d3 = v.w - mean;
      q += (d0 * d0 + d1 * d1) + (d2 * d2 + d3 * d3);
    }
  } else {
    for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
      const float d = load_f(a.x, a.dtype, base + i) - mean;
      q += d * d;
    }
  }
  q = block_sum_256(q, red);
  if (threadIdx.x == 0) {
    float* p = a.partial + (int64_t(ng) * a.splits + split) * 3;
    p[0] = cnt;
    p[1] = mean;
    p[2] = q;
  }
}

__global__ __launch_bounds__(256) void group_norm_apply_kernel(GroupNormArgs a) {
  __shared__ float stat[2];
  const int ng = blockIdx.x, split = blockIdx.y;
  const int n = ng / a.groups, g = ng % a.groups;
  const int cpg = a.C / a.groups;
  const int64_t count = int64_t(cpg) * a.HW;
  const int64_t base = (int64_t(n) * a.C + int64_t(g) * cpg) * a.HW;
  if (threadIdx.x == 0) {
    const float* p = a.partial + int64_t(ng) * a.splits * 3;
    float c = 0.f, mean = 0.f, m2 = 0.f;
    for (int k = 0; k < a.splits; k++) {
      const float cb = p[3 * k], mb = p[3 * k + 1], qb = p[3 * k + 2];
      if (cb == 0.f) continue;
      const float ct = c + cb, d = mb - mean;
      mean += d * (cb / ct);
      m2 += qb + d * d * (c * cb / ct);
      c = ct;
    }
    stat[0] = mean;
    stat[1] = 1.0f / sqrtf(m2 / c + a.eps);
  }
  __syncthreads();
  const float mean = stat[0], rstd = stat[1];
  int64_t lo, hi;
  gn_chunk(a, count, split, lo, hi);
  // Vector path: 4 elements of one channel (HW a multiple of 4).
  const bool vec = (uintptr_t)a.x % 16 == 0 && (uintptr_t)a.y % 16 == 0 && ((base + lo) & 3) == 0 &&
                   ((hi - lo) & 3) == 0 && (a.HW & 3) == 0;
  if (vec) {
    for (int64_t i = lo + 4 * threadIdx.x; i < hi; i += 1024) {
      const int c = g * cpg + (int)(i / a.HW);
      const float w = a.weight ? load_f(a.weight, a.w_dtype, c) * rstd : rstd;
      const float b = (a.bias ? load_f(a.bias, a.w_dtype, c) : 0.f) - mean * w;
      const float4 v = load4(a.x, a.dtype, base + i);
      float y[4] = {v.x * w + b, v.y * w + b, v.z * w + b, v.w * w + b};
      if (a.silu)
        for (int e = 0; e < 4; e++) y[e] = silu_f(y[e]);
      store4(a.y, a.y_dtype, base + i, make_float4(y[0], y[1], y[2], y[3]));
    }
    return;
  }
  for (int64_t i = lo + threadIdx.x; i < hi; i += 256) {
    const int c = g * cpg + (int)(i / a.HW);
    float y = (load_f(a.x, a.dtype, base + i) - mean) * rstd;
    if (a.weight) y *= load_f(a.weight, a.w_dtype, c);
    if (a.bias) y += load_f(a.bias, a.w_dtype, c);
    if (a.silu) y = silu_f(y);
    store_f(a.y, a.y_dtype, base + i, y);
  }
}

// Where group_norm_final_kernel leaves (mean, rstd) per (n, group): after the
// split partials in the same scratch.
__device__ __forceinline__ float* group_norm_final(const GroupNormArgs& a) {
  return a.partial + int64_t(a.N) * a.groups * a.splits * 3;
}

// The statistics of each (n, group) combined from its split partials
// (Chan's pairwise update, as group_norm_apply_kernel does per workgroup),
// once: thread i of the grid takes (n, g) = (i / groups, i % groups).
__global__ __launch_bounds__(64) void group_norm_final_kernel(GroupNormArgs a) {
  const int i = blockIdx.x * 64 + threadIdx.x;
  if (i >= a.N * a.groups) return;
  const float* p = a.partial + int64_t(i) * a.splits * 3;
  float c = 0.f, mean = 0.f, m2 = 0.f;
  for (int k = 0; k < a.splits; k++) {
    const float cb = p[3 * k], mb = p[3 * k + 1], qb = p[3 * k + 2];
    if (cb == 0.f) continue;
    const float ct = c + cb, d = mb - mean;
    mean += d * (cb / ct);
    m2 += qb + d * d * (c * cb / ct);
    c = ct;
  }
  float* f = group_norm_final(a) + int64_t(i) * 2;
  f[0] = mean;
  f[1] = 1.0f / sqrtf(m2 / c + a.eps);
}

// The apply writing NHWC, the layout the implicit-GEMM convolution reads,
// so no NCHW -> NHWC copy follows: a workgroup takes PT pixels of one image
// and every channel. The per-group statistics are combined from the split
// partials as group_norm_apply_kernel does; each channel's PT pixels are read
// by PT / 8 lanes in 16-byte loads, normalised with the same arithmetic
// (x * (weight * rstd) + (bias - mean * weight * rstd), then SiLU), staged
// transposed in LDS, and written as whole NHWC pixel rows in 16-byte stores.
// PT = 64 for up to 512 channels, 32 for up to 1280.
template <typename T, int PT, int CMAX>
__global__ __launch_bounds__(256) void group_norm_apply_nhwc_kernel(GroupNormArgs a) {
  constexpr int LPC = PT / 8, CPP = 256 / LPC;  // lanes per channel, channels per pass
  __shared__ float gstat[128];
  __shared__ __attribute__((aligned(16))) T tile[PT * (CMAX + 8)];
  const int LDC = a.C + 8;
  const int n = blockIdx.y, p0 = blockIdx.x * PT, tid = threadIdx.x;
  const int cpg = a.C / a.groups;
  // (mean, rstd) of each group of image n, finalised once by
  // group_norm_final_kernel after the split partials.
  if (tid < 2 * a.groups) gstat[tid] = group_norm_final(a)[int64_t(n) * a.groups * 2 + tid];
  __syncthreads();
  const int pg = tid % LPC, cl = tid / LPC;
  for (int c0 = 0; c0 < a.C; c0 += CPP) {
    const int c = c0 + cl;
    if (c < a.C) {
      const int g = c / cpg;
      const float mean = gstat[2 * g], rstd = gstat[2 * g + 1];
      const float w = a.weight ? load_f(a.weight, a.w_dtype, c) * rstd : rstd;
      const float b = (a.bias ? load_f(a.bias, a.w_dtype, c) : 0.f) - mean * w;
      const uint4 u = *(const uint4*)((const T*)a.x + (int64_t(n) * a.C + c) * a.HW + p0 + pg * 8);
      const T* xv = (const T*)&u;
#pragma unroll
      for (int e = 0; e < 8; e++) {
        float y = (float)xv[e] * w + b;
        if (a.silu) y = silu_f(y);
        tile[(pg * 8 + e) * LDC + c] = (T)y;
      }
    }
  }
  __syncthreads();
  const int cw = a.C / 8;  // 16-byte chunks in a pixel row
  for (int k = tid; k < PT * cw; k += 256) {
    const int p = k / cw, cc = (k - p * cw) * 8;
    *(uint4*)((T*)a.y + (int64_t(n) * a.HW + p0 + p) * a.C + cc) = *(const uint4*)&tile[p * LDC + cc];
  }
}

// What the NHWC apply can take: 16-bit data, C a multiple of 8 up to 1280,
// whole pixel tiles, at most 64 groups.
static bool group_norm_nhwc_shape(int dtype, int y_dtype, int64_t C, int64_t HW, int groups) {
  return dtype == y_dtype && (dtype == NDX_BF16 || dtype == NDX_F16) && C % 8 == 0 && C <= 1280 &&
         HW % (C <= 512 ? 64 : 32) == 0 && groups <= 64;
}

// Where the graph writes a group norm's output NHWC: up to 512 channels. The
// 32-pixel tiles of wider images cost more than the copy they remove (SDXL's
// 640- and 1280-channel norms: 32.68 against 32.45 ms a step); they are
// taken with NDX_GN_NHWC_WIDE=1 (read at compile time).
bool group_norm_nhwc_ok(int dtype, int y_dtype, int64_t C, int64_t HW, int groups) {
  const char* wide = getenv("NDX_GN_NHWC_WIDE");
  return group_norm_nhwc_shape(dtype, y_dtype, C, HW, groups) && (C <= 512 || (wide && wide[0] == '1'));
}

void launch_group_norm(const GroupNormArgs& a, hipStream_t s) {
  dim3 g(a.N * a.groups, a.splits);
  hipLaunchKernelGGL(group_norm_stats_kernel, g, dim3(256), 0, s, a);
  if (!a.nhwc) {
    hipLaunchKernelGGL(group_norm_apply_kernel, g, dim3(256), 0, s, a);
    return;
  }
  if (!group_norm_nhwc_shape(a.dtype, a.y_dtype, a.C, a.HW, a.groups) || (uintptr_t)a.x % 16 || (uintptr_t)a.y % 16)
    throw std::runtime_error("group norm: an NHWC output needs 16-bit data, C a multiple of 8 up to 1280 and whole "
                             "pixel tiles");
  hipLaunchKernelGGL(group_norm_final_kernel, dim3((a.N * a.groups + 63) / 64), dim3(64), 0, s, a);
  const bool wide = a.C > 512;
  dim3 gn(a.HW / (wide ? 32 : 64), a.N);
  if (a.dtype == NDX_BF16) {
    if (wide) hipLaunchKernelGGL((group_norm_apply_nhwc_kernel<__bf16, 32, 1280>), gn, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((group_norm_apply_nhwc_kernel<__bf16, 64, 512>), gn, dim3(256), 0, s, a);
  } else {
    if (wide) hipLaunchKernelGGL((group_norm_apply_nhwc_kernel<_Float16, 32, 1280>), gn, dim3(256), 0, s, a);
    else hipLaunchKernelGGL((group_norm_apply_nhwc_kernel<_Float16, 64, 512>), gn, dim3(256), 0, s, a);
  }
}

// Softmax over the last axis (DmlOps.ActivationSoftmax with axes {3},
// Dml/DmlOps.cs:175-184) of scale * x, written at x's type: one 256-thread
// workgroup per row. Pass one keeps a running (max, sum of exp) per thread and
// merges them across the workgroup; pass two reads the row again (from L2: a
// row is at most a few hundred KB) and writes exp(scale * x - max) / sum.
// Rows whose length is a multiple of 8 at 16-byte aligned addresses move 8
// elements per load.
template <int DT, bool VEC>
__global__ __launch_bounds__(256) void softmax_rows_kernel(const void* __restrict__ x, void* __restrict__ y,
                                                           int64_t cols, float scale) {
  const int64_t base = int64_t(blockIdx.x) * cols;
  const int tid = threadIdx.x;
  float m = -INFINITY, sum = 0.f;
  auto take = [&](float v) {
    v *= scale;
    if (v > m) {
      sum = sum * __expf(m - v) + 1.f;
      m = v;
    } else {
      sum += __expf(v - m);
    }
  };
  if constexpr (VEC) {
    for (int64_t c = int64_t(tid) * 8; c < cols; c += 256 * 8) {
      float v[8];
      load8_t<DT>(x, base + c, v);
#pragma unroll
      for (int j = 0; j < 8; j++) take(v[j]);
    }
  } else {
    for (int64_t c = tid; c < cols; c += 256) take(load_f(x, DT, base + c));
  }
  // merge (m, sum) over the wave, then over the four waves
  for (int off = 32; off > 0; off >>= 1) {
    const float om = __shfl_xor(m, off);
    const float os = __shfl_xor(sum, off);
    const float nm = fmaxf(m, om);
    sum = (m == -INFINITY ? 0.f : sum * __expf(m - nm)) + (om == -INFINITY ? 0.f : os * __expf(om - nm));
    m = nm;
  }
  __shared__ float red[2][4];
  if ((tid & 63) == 0) {
    red[0][tid >> 6] = m;
    red[1][tid >> 6] = sum;
  }
  __syncthreads();
  float M = red[0][0];
  for (int w = 1; w < 4; w++) M = fmaxf(M, red[0][w]);
  float S = 0.f;
  for (int w = 0; w < 4; w++)
    if (red[0][w] != -INFINITY) S += red[1][w] * __expf(red[0][w] - M);
  const float inv = 1.0f / S;
  if constexpr (VEC) {
    for (int64_t c = int64_t(tid) * 8; c < cols; c += 256 * 8) {
      float v[8];
      load8_t<DT>(x, base + c, v);
#pragma unroll
      for (int j = 0; j < 8; j++) v[j] = __expf(v[j] * scale - M) * inv;
      store8_t<DT>(y, base + c, v);
    }
  } else {
    for (int64_t c = tid; c < cols; c += 256) store_f(y, DT, base + c, __expf(load_f(x, DT, base + c) * scale - M) * inv);
  }
}

void launch_softmax(const void* x, void* y, int dtype, int64_t rows, int64_t cols, float scale, hipStream_t s) {
  if (rows == 0 || cols == 0) return;
  const bool vec = cols % 8 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0;
#define NDX_SM(DT)                                                                                          \
  do {                                                                                                      \
    if (vec) hipLaunchKernelGGL((softmax_rows_kernel<DT, true>), dim3((unsigned)rows), dim3(256), 0, s, x, y, cols, scale); \
    else hipLaunchKernelGGL((softmax_rows_kernel<DT, false>), dim3((unsigned)rows), dim3(256), 0, s, x, y, cols, scale);    \
  } while (0)
  if (dtype == NDX_BF16) NDX_SM(NDX_BF16);
  else if (dtype == NDX_F16) NDX_SM(NDX_F16);
  else NDX_SM(NDX_F32);
#undef NDX_SM
}

}  // namespace ndx
