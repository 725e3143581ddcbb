// Wavefront-reduction normalisation kernels: LayerNorm (+affine),
// Transformer.Modulate (LayerNorm * (1 + scale) + shift, cast), RMSNorm,
// the per-head RMSNorm + rotate-half RoPE of the attention inputs, and
// GroupNorm (+affine, +SiLU).

#include "k_common.h"

namespace ndx {

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
  const int64_t woff = batch * a.batch_w, boff = batch * a.batch_b;
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
  const int64_t woff = batch * a.batch_w, boff = batch * a.batch_b;
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

void launch_row_norm(const RowNormArgs& a, hipStream_t s) {
  if (a.rows == 0) return;
  int vpt = (a.D + 63) / 64;
  dim3 grid((unsigned)((a.rows + 3) / 4)), block(256);
  if (vpt <= 4) hipLaunchKernelGGL(row_norm_kernel<4>, grid, block, 0, s, a);
  else if (vpt <= 8) hipLaunchKernelGGL(row_norm_kernel<8>, grid, block, 0, s, a);
  else if (vpt <= 16) hipLaunchKernelGGL(row_norm_kernel<16>, grid, block, 0, s, a);
  else if (vpt <= 32) hipLaunchKernelGGL(row_norm_kernel<32>, grid, block, 0, s, a);
  else if (vpt <= 48) hipLaunchKernelGGL(row_norm_kernel<48>, grid, block, 0, s, a);
  else if (vpt <= 64) hipLaunchKernelGGL(row_norm_kernel<64>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(row_norm_wide_kernel, dim3((unsigned)a.rows), block, 0, s, a);
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

void launch_head_norm_rotate(const HeadNormRotateArgs& a, hipStream_t s) {
  int64_t total = int64_t(a.B) * a.T * a.H;
  if (total == 0) return;
  hipLaunchKernelGGL(head_norm_rotate_kernel, dim3((unsigned)((total + 3) / 4)), dim3(256), 0, s, a);
}

// GroupNorm over NCHW: one 1024-thread block per (n, group), two passes for
// the statistics (mean, then the centred sum of squares) and one for the
// output with the per-channel affine and the optional SiLU.
__global__ __launch_bounds__(1024) void group_norm_kernel(GroupNormArgs a) {
  __shared__ float red[16];
  const int n = blockIdx.x / a.groups, g = blockIdx.x % a.groups;
  const int cpg = a.C / a.groups;
  const int64_t count = int64_t(cpg) * a.HW;
  const int64_t base = (int64_t(n) * a.C + int64_t(g) * cpg) * a.HW;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  float s = 0.f;
  for (int64_t i = t; i < count; i += 1024) s += load_f(a.x, a.dtype, base + i);
  s = wave_sum(s);
  if (lane == 0) red[w] = s;
  __syncthreads();
  s = 0.f;
  for (int k = 0; k < 16; k++) s += red[k];
  const float mean = s / count;
  __syncthreads();
  float q = 0.f;
  for (int64_t i = t; i < count; i += 1024) {
    float d = load_f(a.x, a.dtype, base + i) - mean;
    q += d * d;
  }
  q = wave_sum(q);
  if (lane == 0) red[w] = q;
  __syncthreads();
  q = 0.f;
  for (int k = 0; k < 16; k++) q += red[k];
  const float rstd = 1.0f / sqrtf(q / count + a.eps);
  for (int64_t i = t; i < count; i += 1024) {
    int c = g * cpg + (int)(i / a.HW);
    float y = (load_f(a.x, a.dtype, base + i) - mean) * rstd;
    if (a.weight) y *= load_f(a.weight, a.w_dtype, c);
    if (a.bias) y += load_f(a.bias, a.w_dtype, c);
    if (a.silu) y = silu_f(y);
    store_f(a.y, a.y_dtype, base + i, y);
  }
}

void launch_group_norm(const GroupNormArgs& a, hipStream_t s) {
  hipLaunchKernelGGL(group_norm_kernel, dim3(a.N * a.groups), dim3(1024), 0, s, a);
}

}  // namespace ndx
