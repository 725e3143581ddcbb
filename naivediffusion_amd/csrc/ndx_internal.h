// Internal declarations shared by the runtime (runtime.cpp, graph.cpp) and
// the kernel files (k_*.hip). Nothing here crosses the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/ndx.h"

namespace ndx {

// ---- element types ---------------------------------------------------------

__host__ __device__ inline int dtype_size(int dt) {
  switch (dt) {
    case NDX_F32: case NDX_U32: case NDX_I32: return 4;
    case NDX_F16: case NDX_BF16: case NDX_U16: return 2;
    case NDX_I64: return 8;
    case NDX_I8: return 1;
    default: return 0;
  }
}
__host__ __device__ inline bool dtype_is_float(int dt) { return dt == NDX_F32 || dt == NDX_F16 || dt == NDX_BF16; }
const char* dtype_name(int dt);

// ---- errors ----------------------------------------------------------------

// Thrown inside the library, turned into an ndx_status at the C boundary.
struct Error {
  ndx_status status;
  std::string message;
};
[[noreturn]] void fail(ndx_status status, const std::string& message);
void set_last_error(const std::string& message);
// Checks a HIP call; out-of-memory becomes NDX_OOM, anything else DEVICE_LOST.
void hip_check(hipError_t err, const char* what);

}  // namespace ndx

// The body of every C entry point: library errors become the returned status
// and ndx_last_error's message.
#define NDX_TRY try {
#define NDX_CATCH                   \
  }                                 \
  catch (const ndx::Error& e) {     \
    ndx::set_last_error(e.message); \
    return e.status;                \
  }                                 \
  catch (const std::exception& e) { \
    ndx::set_last_error(e.what());  \
    return NDX_INVALID_STATE;       \
  }                                 \
  return NDX_OK;

#define NEED(x) \
  if (!(x)) ndx::fail(NDX_INVALID_ARG, #x " is null")

namespace ndx {

// ---- strided 4-D views -----------------------------------------------------

// Every tensor inside the library is a 4-D view: sizes outermost first,
// strides in elements (0 repeats an axis), like DmlTensorDesc.
struct View4 {
  int64_t size[4];
  int64_t stride[4];
};

// ---- kernel launch arguments ------------------------------------------------

enum Epilogue {
  EPI_NONE = NDX_EPI_NONE,
  EPI_GELU_TANH = NDX_EPI_GELU_TANH,
  EPI_GELU = NDX_EPI_GELU,
  EPI_SILU = NDX_EPI_SILU,
  EPI_GATED_RESIDUAL = NDX_EPI_GATED_RESIDUAL,
  EPI_RESIDUAL = NDX_EPI_RESIDUAL,
  EPI_SWIGLU = NDX_EPI_SWIGLU,
  // Compile-time only (no public code): a QKV projection whose q and k
  // thirds go through the per-head RMSNorm and rotary embedding in the
  // epilogue (the fields norm_* and rope_* of GemmArgs).
  EPI_QK_NORM_ROPE = 100,
};

// One linear layer's product: C[b] = epi(A[b] (M x K, rows lda apart) *
// W^T (W is N x K, rows ldw apart) + bias). W may be int8 with per-(row,
// block) scales. gate is a per-batch [N] row; resid is [b][M][N] (ldr).
struct GemmArgs {
  const void* a; int64_t lda; int64_t batch_a; int a_dtype;
  const void* w; int64_t ldw; int64_t batch_w; int w_dtype;
  const void* scales; int64_t lds; int qblock; int s_dtype;  // int8 weights only
  void* c; int64_t ldc; int64_t batch_c; int c_dtype;
  const void* bias; int bias_dtype;
  // The gate of (b, row, col): b * batch_gate + row * ldg + col, plus
  // gate_split_off for rows at or past gate_split (ldg 0: one row for all;
  // the split: two such rows, the reference's join of two row broadcasts).
  const void* gate; int64_t batch_gate; int gate_dtype;
  int64_t ldg, gate_split, gate_split_off;
  const void* resid; int64_t ldr; int64_t batch_r; int r_dtype;
  int M, N, K, batch;
  int epilogue;
  // A per-row term added with the bias (a convolution's per-channel bias,
  // where rows are output channels).
  const void* row_bias; int row_bias_dtype;
  // Implicit-GEMM convolution: with conv_cin > 0 the weight operand's row n
  // is output pixel n, gathered from an NHWC input [batch, H, W, conv_c] (w,
  // batch_w elements per image) at taps (ky, kx) of a kw-wide filter whose
  // K index is (ky * kw + kx) * conv_cin + ci; channels ci at or past conv_c
  // read as zero. With conv_kcont, K runs over the taps with no padding
  // between them, (ky * kw + kx) * conv_c + ci, past conv_kh * kw taps
  // zeros. With conv_up the input is read through a nearest 2x upsample:
  // conv_h x conv_w is the upsampled size, memory holds half.
  int conv_cin, conv_c, conv_h, conv_w, conv_wo, conv_kw, conv_stride, conv_pad, conv_up;
  int conv_kcont, conv_kh;
  // The 16-bit tile to use regardless of the latency model (0: the model;
  // 1..4: 256x256, 128x128, 64x128, 64x64).
  int tile_hint;
  // EPI_QK_NORM_ROPE: columns below qk_cols are q (the first half) and k
  // heads of 128. Each head of a row is RMS-normalised (norm_eps) over the
  // product rounded to c_dtype, scaled by norm_q / norm_k (null: none),
  // rounded, then rotated (rotate-half) in fp32 by rope_cos / rope_sin
  // ([M, 64] fp32 rows, the row's position within its batch; null: no
  // rotation) and stored; columns from qk_cols on get the bias only.
  const void* norm_q; const void* norm_k; int norm_dtype;
  const float* rope_cos; const float* rope_sin;
  int qk_cols; float norm_eps;
};

// DmlOps.Gemm in full generality (any strides, transposes, alpha, beta): a
// plain fp32-accumulating kernel for the small cases the builder emits.
struct GemmGenericArgs {
  const void* a; View4 va; int a_dtype;
  const void* b; View4 vb; int b_dtype;
  const void* c; View4 vc; int c_dtype;  // may be null
  void* out; int out_dtype;
  int64_t M, N, K;  // per (d0, d1) batch
  int64_t batch0, batch1;
  int trans_a, trans_b;
  float alpha, beta;
};

// Attention over packed [B, T, H*d] rows: each of q, k, v, out may come in two
// row segments (the image and the text stream of a joint sequence) so that a
// join feeding the attention costs no copy.
struct AttnSeg {
  const void* ptr[2];
  int64_t rows0;       // rows in the first segment; the rest in the second
  int64_t ld[2];       // row stride (elements) of each segment
  int64_t batch[2];    // batch stride (elements) of each segment
};
struct AttnArgs {
  AttnSeg q, k, v;
  void* out[2]; int64_t out_rows0; int64_t out_ld[2]; int64_t out_batch[2];
  int B, T, S, H, d, dv;
  float scale;
  int dtype;            // F32, BF16 or F16 for q/k/v/out
  int mask_kind;
  const int32_t* mask;  // key length (1 value) or boolean table
  int64_t mask_stride[4];  // [b, h, t, s] element strides of the boolean table
};

struct HeadNormRotateArgs {
  const void* x; int64_t ldx; int64_t batch_x; int x_dtype;
  void* y; int64_t ldy; int64_t batch_y; int y_dtype;
  const void* weight; int w_dtype;      // [d] or null
  const float* cos; const float* sin;   // [T, d/2] or null
  int B, T, H, d;
  float eps;
};

struct RowNormArgs {
  // LayerNorm / Modulate / RmsNorm over the last axis of [rows, D].
  const void* x; int64_t ldx; int64_t batch_x; int x_dtype;
  void* y; int64_t ldy; int y_dtype;
  int64_t rows; int D;
  int64_t rows_per_batch;            // batch index = row / rows_per_batch
  const void* weight; int64_t batch_w; int w_dtype;   // LN weight / (1+scale) / RMS weight
  const void* bias; int64_t batch_b; int b_dtype;     // LN bias / shift
  // Row r (within its batch) reads weight/bias at batch * batch_w + r * ldw
  // (ldw 0: one row for all), plus split_w_off / split_b_off when r >= split
  // (two rows: the reference's join of two row broadcasts).
  int64_t ldw, ldb, split, split_w_off, split_b_off;
  float eps;
  int mode;   // 0 layernorm(+affine), 1 modulate, 2 rmsnorm
};

struct GroupNormArgs {
  const void* x; void* y; int dtype; int y_dtype;
  int N, C, HW, groups;
  const void* weight; const void* bias; int w_dtype;
  float eps;
  int silu;
  // Split statistics: `splits` workgroups per (n, group) each leave (count,
  // mean, M2) in `partial` (N * groups * splits * 3 floats of scratch).
  float* partial; int splits;
  // The output in NHWC ([N, H, W, C] packed), for the implicit-GEMM
  // convolution that reads it (group_norm_nhwc_ok).
  int nhwc;
};
// Whether the group norm can write NHWC for this shape and type.
bool group_norm_nhwc_ok(int dtype, int y_dtype, int64_t C, int64_t HW, int groups);
// The split count the group norm uses for a shape, and its scratch bytes.
int group_norm_splits(int64_t count);

struct ConvArgs {
  // [N, Cin, H, W] packed; NHWC ([N, H, W, Cin] packed) for the implicit GEMM
  const void* x; int x_dtype;
  // [Cout, Cin, kh, kw] packed (or int8 + scales); [Cout, kh, kw, cin_k]
  // for the implicit GEMM
  const void* w; int w_dtype;
  const void* scales; int qblock; int s_dtype;
  const void* bias; int bias_dtype;
  const void* resid;           // [N, Cout, Ho, Wo] packed, same dtype as y
  void* y; int y_dtype;
  int N, Cin, H, W, Cout, kh, kw, stride, pad, Ho, Wo;
  // Implicit GEMM only: the filter's channels per tap (a multiple of 64, the
  // taps each whole K tiles; or Cin itself, a multiple of 8 but not of 64:
  // the filter [Cout, roundup(kh kw Cin, 64)], K running over the taps with
  // no padding between them), and whether x is read through a nearest 2x
  // upsample (H x W the upsampled size; x holds H/2 x W/2 pixels).
  int cin_k, up;
};

// A norm over the channels of packed NCHW [N, C, P] written as packed tokens
// [N, P, C]: the row norm (LayerNorm, mode 0, or RMSNorm, mode 2) of the
// token view of an image without a transposed copy first, the result
// optionally passed through SiLU (rounded to y's type before and after).
struct ChannelNormArgs {
  const void* x; int x_dtype;
  void* y; int y_dtype;
  int64_t N, C, P;
  const void* weight; int w_dtype;  // [C] or null
  const void* bias; int b_dtype;    // [C] or null
  float eps;
  int mode;
  int silu;
};

// Generic strided elementwise: out = f(in0, in1) over a 4-D shape.
enum ElemOp {
  ELEM_COPY = 0,       // cast/identity/pack
  ELEM_SIGMOID, ELEM_SILU, ELEM_GELU, ELEM_TANH, ELEM_GELU_TANH,
  ELEM_SCALE_BIAS,
  ELEM_ADD, ELEM_SUB, ELEM_MUL, ELEM_DIV,
  ELEM_MUL_GELU,       // x * gelu(y), gelu(y) rounded to the output type first (a GEGLU in one pass)
};
struct ElemArgs {
  const void* in0; View4 v0; int dt0;
  const void* in1; View4 v1; int dt1;
  void* out; View4 vo; int dto;
  int op;
  float scale, bias;
};

struct UpsampleArgs {
  const void* x; View4 vx; void* y; int dtype; int scale;
  int64_t N, C, H, W;
};
struct PatchArgs {
  const void* x; void* y; int x_dtype; int y_dtype;
  int N, C, H, W, p;
  int inverse;
  int channel_last;  // feature order (dy, dx, c) instead of (c, dy, dx)
};

// ---- launchers (defined in the k_*.hip files) ---------------------------------

void launch_gemm(const GemmArgs& a, hipStream_t s);
void launch_gemm_generic(const GemmGenericArgs& a, hipStream_t s);
// Attention; `scratch` holds attention_scratch_bytes(...) bytes (the split
// schedule's partials), or is null to run without the split.
void launch_attention(const AttnArgs& a, void* scratch, hipStream_t s);
int64_t attention_scratch_bytes(int B, int T, int S, int H, int d, int dv, int dtype);
void launch_head_norm_rotate(const HeadNormRotateArgs& a, hipStream_t s);
void launch_row_norm(const RowNormArgs& a, hipStream_t s);
void launch_group_norm(const GroupNormArgs& a, hipStream_t s);
// Softmax of scale * x over the last axis of packed [rows, cols] rows, at
// dtype (F32, BF16 or F16) in and out.
void launch_softmax(const void* x, void* y, int dtype, int64_t rows, int64_t cols, float scale, hipStream_t s);
void launch_conv2d(const ConvArgs& a, hipStream_t s);
void launch_channel_norm(const ChannelNormArgs& a, hipStream_t s);
// The implicit-GEMM convolution: filters reordered to [Cout, kh, kw, cin_k]
// (reorder_filter), the input in NHWC (launch_nchw_to_nhwc), 16-bit types.
// conv_gemm_cin is the channel count per tap of the filter the GEMM runs
// with (ConvArgs::cin_k): Cin for a multiple of 8 (a multiple of 64: whole
// K tiles per tap; otherwise K contiguous over the taps), else 0: the
// direct kernel runs instead.
int64_t conv_gemm_cin(int x_dtype, int w_dtype, int64_t cin);
// Elements per row of the reordered filter for cin_k channels per tap.
int64_t conv_filter_row(int64_t cin_k, int64_t taps);
void launch_conv_gemm(const ConvArgs& a, hipStream_t s);
void launch_nchw_to_nhwc(const void* x, void* y, int dtype, int64_t n, int64_t c, int64_t hw, hipStream_t s);
// Filters [cout, cin, taps] -> rows of `row` elements (0: taps * cin_pad)
// holding [taps, cin_pad], channels past cin and the row's tail zero.
void launch_reorder_filter(const void* w, void* y, int dtype, int64_t cout, int64_t cin, int64_t taps,
                           hipStream_t s, int64_t cin_pad = 0, int64_t row = 0);
const char* conv_family(const ConvArgs& a);
// Whether the kernel launch_gemm picks for a (pointers aside) can run
// EPI_QK_NORM_ROPE with qk_cols: a 16-bit direct-to-LDS tile of 64-column
// waves whose width divides qk_cols.
bool gemm_qk_norm_ok(const GemmArgs& a, int qk_cols);
// Whether the fused head norm runs on the product's own (256 x 256) tile
// with one head per wave: the form that costs the product nothing extra.
bool gemm_qk_norm_fast(const GemmArgs& a, int qk_cols);
void launch_elementwise(const ElemArgs& a, hipStream_t s);
void launch_upsample(const UpsampleArgs& a, hipStream_t s);
void launch_patch(const PatchArgs& a, hipStream_t s);
void launch_guided_euler(const float* x, const float* u, const float* c, const float* scalars, float* out, int64_t n,
                         hipStream_t s);
void launch_fill_normal(void* ptr, int dtype, int64_t n, uint64_t seed, float mean, float std,
                        hipStream_t s);
void launch_quantize(const void* w, int w_dtype, int64_t rows, int64_t cols, int block,
                     int s_dtype, int8_t* q, void* scales, hipStream_t s);

// Host quantiser (runtime.cpp), shared by ndx_quantize_block_int8 and the
// graph's ModelBuilder.Weight path.
void quantize_host(const void* w, int dtype, int64_t rows, int64_t cols, int block, int s_dtype,
                   int8_t* q, void* scales);

// A LoRA's low-rank pairs folded into a weight (LoraMerge.Merge): each
// output row is widened to fp32, takes scale * up[row - first, r] * down[r, :]
// for every pair covering it, rank by rank, and is narrowed once.
constexpr int kMaxLoraPatches = NDX_MAX_LORA_PATCHES;
struct LoraPatchArgs {
  const void* down;  // [rank, cols]
  const void* up;    // [count, rank]
  int down_dtype, up_dtype;
  int rank;
  int64_t first, count;
  float scale;
};
struct LoraFoldArgs {
  const void* w; int w_dtype;
  void* out; int out_dtype;
  int64_t rows, cols;
  int patches;
  LoraPatchArgs p[kMaxLoraPatches];
};
void launch_lora_fold(const LoraFoldArgs& a, hipStream_t s);

// Which GEMM kernel a shape goes to, and the algorithmic work, for profiling.
const char* gemm_family(const GemmArgs& a);
// Two independent products with equal N, K, batch and types as one launch
// (the second's row tiles after the first's); false when they cannot share
// a kernel, and then nothing was launched.
bool launch_gemm_pair(const GemmArgs& a, const GemmArgs& b, hipStream_t s);
// Whether one launch of the two products is modelled faster than two.
bool gemm_pair_pays(int64_t M1, int64_t M2, int64_t N, int64_t K, int64_t batch);
const char* gemm_pair_family(const GemmArgs& a, const GemmArgs& b);

}  // namespace ndx
