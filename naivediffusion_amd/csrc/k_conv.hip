// 2-D convolution (cross-correlation) over NCHW, the semantics of
// DmlOps.Convolution (Dml/DmlOps.cs:265-299): filters [Cout, Cin, kh, kw],
// start padding `pad` on both spatial axes (the end padding only changes the
// output extent, which the graph computed), bias per output channel, an
// optional residual added to the output. Filters may be int8 with block
// scales along Cin*kh*kw (ModelBuilder.Weight, Graph/ModelBuilder.cs:61-64).
//
// Direct form: one thread per output element, fp32 accumulation. The
// 16-bit convolutions with Cin a multiple of 64 go to the implicit GEMM of
// k_gemm.hip instead; the layout changes it needs are here.

#include <stdexcept>

#include "k_common.h"

namespace ndx {

__global__ void conv2d_direct_kernel(ConvArgs a, int64_t total) {
  const int taps = a.Cin * a.kh * a.kw;
  const int lds = a.qblock ? taps / a.qblock : 0;
  for (int64_t id = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; id < total;
       id += int64_t(gridDim.x) * blockDim.x) {
    int64_t r = id;
    const int ox = (int)(r % a.Wo);
    r /= a.Wo;
    const int oy = (int)(r % a.Ho);
    r /= a.Ho;
    const int co = (int)(r % a.Cout);
    const int64_t n = r / a.Cout;
    float acc = 0.f;
    for (int ci = 0; ci < a.Cin; ci++) {
      const int64_t xb = (n * a.Cin + ci) * int64_t(a.H) * a.W;
      for (int ky = 0; ky < a.kh; ky++) {
        const int iy = oy * a.stride - a.pad + ky;
        if (iy < 0 || iy >= a.H) continue;
        for (int kx = 0; kx < a.kw; kx++) {
          const int ix = ox * a.stride - a.pad + kx;
          if (ix < 0 || ix >= a.W) continue;
          const int tap = (ci * a.kh + ky) * a.kw + kx;
          const int64_t wi = int64_t(co) * taps + tap;
          float w;
          if (a.w_dtype == NDX_I8) {
            float sc = a.s_dtype == NDX_F16 ? (float)((const _Float16*)a.scales)[int64_t(co) * lds + tap / a.qblock]
                                            : ((const float*)a.scales)[int64_t(co) * lds + tap / a.qblock];
            w = float(((const int8_t*)a.w)[wi]) * sc;
          } else {
            w = load_f(a.w, a.w_dtype, wi);
          }
          acc += load_f(a.x, a.x_dtype, xb + int64_t(iy) * a.W + ix) * w;
        }
      }
    }
    if (a.bias) acc += load_f(a.bias, a.bias_dtype, co);
    if (a.resid) acc += load_f(a.resid, a.y_dtype, id);
    store_f(a.y, a.y_dtype, id, acc);
  }
}

// [n, c, hw] -> [n, hw, c] for 16-bit elements, through a 64 x 64 LDS tile:
// reads run along hw, writes along c.
__global__ __launch_bounds__(256) void nchw_to_nhwc_kernel(const uint16_t* x, uint16_t* y, int64_t c, int64_t hw) {
  __shared__ uint16_t tile[64][65];
  const int64_t b = blockIdx.z;
  const int64_t c0 = int64_t(blockIdx.y) * 64, p0 = int64_t(blockIdx.x) * 64;
  const uint16_t* xb = x + b * c * hw;
  uint16_t* yb = y + b * c * hw;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
  for (int r = ty; r < 64; r += 4) {
    const int64_t ch = c0 + r, p = p0 + tx;
    if (ch < c && p < hw) tile[r][tx] = xb[ch * hw + p];
  }
  __syncthreads();
  for (int r = ty; r < 64; r += 4) {
    const int64_t p = p0 + r, ch = c0 + tx;
    if (ch < c && p < hw) yb[p * c + ch] = tile[tx][r];
  }
}

// The same transposition for c and hw multiples of 64 with 16-byte accesses
// on both sides: each thread reads 8 pixels of one channel and writes 8
// channels of one pixel.
__global__ __launch_bounds__(256) void nchw_to_nhwc_vec_kernel(const uint16_t* x, uint16_t* y, int64_t c, int64_t hw) {
  __shared__ __align__(16) uint16_t tile[64][64 + 8];  // [channel][pixel], rows padded by 16 bytes
  const int64_t b = blockIdx.z;
  const int64_t c0 = int64_t(blockIdx.y) * 64, p0 = int64_t(blockIdx.x) * 64;
  const uint16_t* xb = x + b * c * hw;
  uint16_t* yb = y + b * c * hw;
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int id = threadIdx.x + k * 256;  // 512 chunks: 64 channels x 8 chunks of 8 pixels
    const int ch = id >> 3, px = (id & 7) * 8;
    *(uint4*)&tile[ch][px] = *(const uint4*)(xb + (c0 + ch) * hw + p0 + px);
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 2; k++) {
    const int id = threadIdx.x + k * 256;  // 512 chunks: 64 pixels x 8 chunks of 8 channels
    const int px = id >> 3, ch = (id & 7) * 8;
    __align__(16) uint16_t r[8];
#pragma unroll
    for (int e = 0; e < 8; e++) r[e] = tile[ch + e][px];
    *(uint4*)(yb + (p0 + px) * c + c0 + ch) = *(const uint4*)r;
  }
}

void launch_nchw_to_nhwc(const void* x, void* y, int dtype, int64_t n, int64_t c, int64_t hw, hipStream_t s) {
  if (dtype_size(dtype) != 2) throw std::runtime_error("nchw_to_nhwc: 16-bit elements only");
  dim3 g((unsigned)((hw + 63) / 64), (unsigned)((c + 63) / 64), (unsigned)n);
  if (c % 64 == 0 && hw % 64 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0) {
    hipLaunchKernelGGL(nchw_to_nhwc_vec_kernel, g, dim3(256), 0, s, (const uint16_t*)x, (uint16_t*)y, c, hw);
    return;
  }
  hipLaunchKernelGGL(nchw_to_nhwc_kernel, g, dim3(256), 0, s, (const uint16_t*)x, (uint16_t*)y, c, hw);
}

// Filters [cout, cin, taps] -> rows of `row` elements holding [taps,
// cin_pad] (16-bit elements), channels past cin and the row's tail zero.
__global__ void reorder_filter_kernel(const uint16_t* w, uint16_t* y, int64_t cout, int64_t cin, int64_t taps,
                                      int64_t cin_pad, int64_t row) {
  const int64_t total = cout * row;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += int64_t(gridDim.x) * blockDim.x) {
    const int64_t k = i % row, co = i / row;
    const int64_t ci = k % cin_pad, t = k / cin_pad;
    y[i] = ci < cin && t < taps ? w[(co * cin + ci) * taps + t] : uint16_t(0);
  }
}

void launch_reorder_filter(const void* w, void* y, int dtype, int64_t cout, int64_t cin, int64_t taps,
                           hipStream_t s, int64_t cin_pad, int64_t row) {
  if (dtype_size(dtype) != 2) throw std::runtime_error("reorder_filter: 16-bit elements only");
  if (cin_pad < cin) cin_pad = cin;
  if (row < taps * cin_pad) row = taps * cin_pad;
  const int64_t total = cout * row;
  const int blocks = (int)std::min<int64_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(reorder_filter_kernel, dim3(std::max(blocks, 1)), dim3(256), 0, s, (const uint16_t*)w,
                     (uint16_t*)y, cout, cin, taps, cin_pad, row);
}

void launch_conv2d(const ConvArgs& a, hipStream_t s) {
  int64_t total = int64_t(a.N) * a.Cout * a.Ho * a.Wo;
  int blocks = (int)std::min<int64_t>((total + 255) / 256, 65536 * 4);
  hipLaunchKernelGGL(conv2d_direct_kernel, dim3(std::max(blocks, 1)), dim3(256), 0, s, a, total);
}

}  // namespace ndx
