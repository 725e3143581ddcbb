// The linear layer's GEMM for gfx950: y[M, N] = x[M, K] * W[N, K]^T with
// fused epilogues (bias, GELU-tanh / GELU / SiLU, gated residual).
//
// Both operands are K-contiguous rows (torch's [out, in] weight order, the
// layout Layers.Linear feeds DirectML, Graph/Layers.cs:131-160), so A and B
// tiles load the same way: 16-byte chunks of 8 elements, staged through LDS
// in a double buffer, each 64-element K row of the tile XOR-swizzled by 16-
// byte chunk so the MFMA fragment reads are bank-conflict free.
//
// Kernels:
//  - gemm_mfma_kernel: bf16 or f16 activations on v_mfma_f32_32x32x16_{bf16,f16};
//    weights of the same type or int8 with per-(row, block) scales that are
//    dequantised in registers on the way into LDS.
//  - gemm_f32_kernel: fp32 activations on v_mfma_f32_32x32x2_f32; weights of
//    any float width or int8, widened on the way into LDS.
//  - gemv_kernel: a handful of rows (the adaLN modulation, the time MLP):
//    weight-bandwidth bound, one wave per output feature group.
//  - gemm_generic_kernel: DmlOps.Gemm with arbitrary strides and transposes.

#include <string.h>

#include <algorithm>
#include <cstdlib>
#include <stdexcept>

#include "k_common.h"

namespace ndx {

static constexpr int BK = 64;

template <typename T>
struct MfmaOp;
template <>
struct MfmaOp<__bf16> {
  typedef bf16x8 V;
  static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static constexpr int dtype = NDX_BF16;
};
template <>
struct MfmaOp<_Float16> {
  typedef f16x8 V;
  static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static constexpr int dtype = NDX_F16;
};

// Tile order: workgroup i runs on XCD i % 8, so consecutive ids are
// re-indexed to give each XCD one contiguous run of tiles, and tiles are
// walked in groups of 8 tile-rows so neighbours share A rows and W rows in
// that XCD's L2.
__device__ __forceinline__ bool tile_of(int pid, int grid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int per = grid / 8;
  pid = (pid % 8) * per + pid / 8;
  if (pid >= tiles_m * tiles_n) return false;
  const int G = 8;
  const int width = G * tiles_n;
  const int group = pid / width;
  const int first_m = group * G;
  const int gsz = min(tiles_m - first_m, G);
  tm = first_m + (pid % width) % gsz;
  tn = (pid % width) / gsz;
  return true;
}

__device__ __forceinline__ float scale_at(const void* s, int sdt, int64_t i) {
  return sdt == NDX_F16 ? (float)((const _Float16*)s)[i] : ((const float*)s)[i];
}

// Element offset of the gate of (b, row, col = 0): one row for all rows
// (ldg 0), a row per row, or two rows split at gate_split.
__device__ __forceinline__ int64_t gate_off(const GemmArgs& a, int64_t b, int row) {
  return b * a.batch_gate + int64_t(row) * a.ldg + (row >= a.gate_split ? a.gate_split_off : 0);
}

// The epilogue of one output element (row, col) of batch b.
__device__ __forceinline__ void epilogue_one(const GemmArgs& a, int64_t b, int row, int col, float v, float bias,
                                             float gate) {
  v += bias;
  switch (a.epilogue) {
    case EPI_GELU_TANH: v = gelu_tanh_f(v); break;
    case EPI_GELU: v = gelu_f(v); break;
    case EPI_SILU: v = silu_f(v); break;
    case EPI_GATED_RESIDUAL:
      v = load_f(a.resid, a.r_dtype, b * a.batch_r + int64_t(row) * a.ldr + col) + gate * round_to(v, a.a_dtype);
      break;
    case EPI_RESIDUAL:
      v = load_f(a.resid, a.r_dtype, b * a.batch_r + int64_t(row) * a.ldr + col) + round_to(v, a.a_dtype);
      break;
    default: break;
  }
  store_f(a.c, a.c_dtype, b * a.batch_c + int64_t(row) * a.ldc + col, v);
}

// Four consecutive values p[off .. off + 4) widened to fp32, in one 16-byte
// (fp32) or 8-byte (16-bit) load; the address must allow it.
__device__ __forceinline__ float4 load4_vec(const void* p, int dt, int64_t off) {
  if (dt == NDX_F32) return *(const float4*)((const float*)p + off);
  const uint2 u = dt == NDX_BF16 ? *(const uint2*)((const __bf16*)p + off) : *(const uint2*)((const _Float16*)p + off);
  if (dt == NDX_BF16) {
    const __bf16* h = (const __bf16*)&u;
    return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
  }
  const _Float16* h = (const _Float16*)&u;
  return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
}

__host__ __device__ __forceinline__ bool aligned16(const void* p, int64_t elems_a, int64_t elems_b, int es) {
  return (uintptr_t)p % 16 == 0 && (elems_a * es) % 16 == 0 && (elems_b * es) % 16 == 0;
}

// Up to four per-column values p[off .. off + n) (zeros past n).
__device__ __forceinline__ float4 load_cols(const void* p, int dt, int64_t off, int n, bool vec) {
  if (n >= 4 && vec) return load4_vec(p, dt, off);
  float v[4] = {0.f, 0.f, 0.f, 0.f};
  for (int e = 0; e < n && e < 4; e++) v[e] = load_f(p, dt, off + e);
  return make_float4(v[0], v[1], v[2], v[3]);
}

// Stores four consecutive outputs in one 16-byte (fp32) or 8-byte (16-bit)
// store; the address must allow it.
__device__ __forceinline__ void store4_vec(void* p, int dt, int64_t off, const float (&v)[4]) {
  if (dt == NDX_F32) {
    *(float4*)((float*)p + off) = make_float4(v[0], v[1], v[2], v[3]);
  } else if (dt == NDX_BF16) {
    __bf16 h[4] = {(__bf16)v[0], (__bf16)v[1], (__bf16)v[2], (__bf16)v[3]};
    *(uint2*)((__bf16*)p + off) = *(const uint2*)h;
  } else {
    _Float16 h[4] = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
    *(uint2*)((_Float16*)p + off) = *(const uint2*)h;
  }
}

// The linear epilogues of four consecutive outputs with every input already
// in registers and every address vector-aligned: bias (per column, plus rb
// per row), then the (gated) residual r + g * y with y rounded to the
// product's type, or nothing more.
__device__ __forceinline__ void epilogue_fast(const GemmArgs& a, int64_t b, int row, int col, float4 acc, float4 bias,
                                              float rb, float4 gate, float4 res) {
  if (row >= a.M) return;
  float v[4] = {acc.x + bias.x + rb, acc.y + bias.y + rb, acc.z + bias.z + rb, acc.w + bias.w + rb};
  if (a.epilogue == EPI_GATED_RESIDUAL || a.epilogue == EPI_RESIDUAL) {
    const float g[4] = {gate.x, gate.y, gate.z, gate.w}, r[4] = {res.x, res.y, res.z, res.w};
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = r[e] + g[e] * round_to(v[e], a.a_dtype);
  }
  store4_vec(a.c, a.c_dtype, b * a.batch_c + int64_t(row) * a.ldc + col, v);
}

// Any epilogue of outputs (row, col .. col + n), n <= 4, reading what it
// needs per element: bias and gate come in (per column), the row bias and
// the residual are read here; GELU-tanh, GELU or SiLU, or the (gated)
// residual; vector stores where all four are there and vec allows.
__device__ __forceinline__ void epilogue_any(const GemmArgs& a, int64_t b, int row, int col, int n, float4 acc,
                                             float4 bias, float4 gate, bool vec, bool gate_rows = false) {
  if (row >= a.M || n <= 0) return;
  const float rb = a.row_bias ? load_f(a.row_bias, a.row_bias_dtype, row) : 0.f;
  float v[4] = {acc.x + bias.x + rb, acc.y + bias.y + rb, acc.z + bias.z + rb, acc.w + bias.w + rb};
  const int ep = a.epilogue;
  if (ep == EPI_SWIGLU) {
    // Columns col .. col + 3 (col a multiple of 4) are two (gate, up) pairs
    // of the interleaved projection: outputs col / 2 and col / 2 + 1. The
    // gate, the up projection and the SiLU are each rounded to the product's
    // type, as the reference's separate operators leave them.
    float o[2];
#pragma unroll
    for (int p = 0; p < 2; p++) {
      const float g = round_to(v[2 * p], a.a_dtype), u = round_to(v[2 * p + 1], a.a_dtype);
      o[p] = round_to(silu_f(g), a.a_dtype) * u;
    }
    const int64_t co = b * a.batch_c + int64_t(row) * a.ldc + col / 2;
#pragma unroll
    for (int p = 0; p < 2; p++)
      if (2 * p + 1 < n) store_f(a.c, a.c_dtype, co + p, o[p]);
    return;
  }
  if (gate_rows && ep == EPI_GATED_RESIDUAL) gate = load_cols(a.gate, a.gate_dtype, gate_off(a, b, row) + col, n, false);
  if (ep == EPI_GELU_TANH) {
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = gelu_tanh_f(v[e]);
  } else if (ep == EPI_GELU) {
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = gelu_f(v[e]);
  } else if (ep == EPI_SILU) {
#pragma unroll
    for (int e = 0; e < 4; e++) v[e] = silu_f(v[e]);
  } else if (ep == EPI_GATED_RESIDUAL || ep == EPI_RESIDUAL) {
    const float g[4] = {gate.x, gate.y, gate.z, gate.w};
    const int64_t ro = b * a.batch_r + int64_t(row) * a.ldr + col;
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (e < n) v[e] = load_f(a.resid, a.r_dtype, ro + e) + g[e] * round_to(v[e], a.a_dtype);
  }
  const int64_t co = b * a.batch_c + int64_t(row) * a.ldc + col;
  if (n >= 4 && vec) {
    store4_vec(a.c, a.c_dtype, co, v);
    return;
  }
#pragma unroll
  for (int e = 0; e < 4; e++)
    if (e < n) store_f(a.c, a.c_dtype, co + e, v[e]);
}

// What every slice of a wave's epilogue shares: the lane's columns, the
// bias and gate of those columns, and which epilogue path runs.
struct EpiLane {
  int col, n, c4, rl0;
  float4 bias, gate, gate2;  // gate2: the gate of rows at or past gate_split
  bool fast, out_vec, gate_rows;
};

// Orders a wave's LDS writes before its later LDS reads (and those reads
// before its next writes) without meeting the other waves: a wave's LDS
// instructions execute in issue order, so only the compiler must be kept
// from moving them across this point.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// One 32-row slice (accumulator row block i of the wave) through LDS, so
// the epilogue walks rows of four consecutive outputs and every global
// store is a vector. The stage is the wave's own (the caller's workgroup
// barrier after the K loop freed the tiles it overlaps), so the slices sync
// per wave and the waves' epilogues run apart: one wave's residual loads
// overlap another's stores. On the fast path (a linear epilogue, every column of
// the wave in range, aligned rows) the loop is unrolled so that the slice's
// residual and row-bias loads all go out before its first store, and their
// latency is paid once per slice rather than once per row. Anything else
// (the activations, whose code is long and which read nothing per row;
// ragged or unaligned edges) runs a rolled loop.
template <int TN, int WN>
__device__ __forceinline__ void epilogue_slice(const GemmArgs& a, int64_t bidx, const EpiLane& L,
                                               f32x16 (&acc)[TN], float* stage, int row0) {
  constexpr int CS = WN + 4;
  constexpr int C4 = WN / 4;        // four-column groups in a wave's row
  constexpr int RSTEP = 64 / C4;    // rows one pass of the wave covers
  constexpr int IT = 32 / RSTEP;    // passes per 32-row slice
  static_assert(64 % C4 == 0 && 32 % RSTEP == 0, "wave columns do not tile the slice");
  const int lane = threadIdx.x & 63, lrow = lane & 31, lhalf = lane >> 5;
  const bool residual = a.epilogue == EPI_GATED_RESIDUAL || a.epilogue == EPI_RESIDUAL;
  float4 res[IT];
  float rb[IT];
  if (L.fast) {
#pragma unroll
    for (int t = 0; t < IT; t++) {
      const int row = row0 + L.rl0 + t * RSTEP;
      const bool in = row < a.M;
      res[t] = (residual && in) ? load4_vec(a.resid, a.r_dtype, bidx * a.batch_r + int64_t(row) * a.ldr + L.col)
                                : make_float4(0.f, 0.f, 0.f, 0.f);
      rb[t] = (a.row_bias && in) ? load_f(a.row_bias, a.row_bias_dtype, row) : 0.f;
    }
  }
#pragma unroll
  for (int j = 0; j < TN; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) stage[(8 * (r >> 2) + 4 * lhalf + (r & 3)) * CS + j * 32 + lrow] = acc[j][r];
  wave_lds_sync();
  if (L.fast) {
#pragma unroll
    for (int t = 0; t < IT; t++) {
      const int rl = L.rl0 + t * RSTEP;
      const float4 v = *(const float4*)&stage[rl * CS + L.c4 * 4];
      epilogue_fast(a, bidx, row0 + rl, L.col, v, L.bias, rb[t], row0 + rl >= a.gate_split ? L.gate2 : L.gate,
                    res[t]);
    }
  } else {
#pragma unroll 1
    for (int t = 0; t < IT; t++) {
      const int rl = L.rl0 + t * RSTEP;
      const float4 v = *(const float4*)&stage[rl * CS + L.c4 * 4];
      epilogue_any(a, bidx, row0 + rl, L.col, L.n, v, L.bias, row0 + rl >= a.gate_split ? L.gate2 : L.gate,
                   L.out_vec, L.gate_rows);
    }
  }
  wave_lds_sync();
}

// Slices I .. TM - 1, expanded at compile time so every accumulator index
// is a constant (a runtime index would put the accumulators in scratch).
template <int I, int TM, int TN, int WN>
__device__ __forceinline__ void epilogue_slices(const GemmArgs& a, int64_t bidx, const EpiLane& L,
                                                f32x16 (&acc)[TM][TN], float* stage, int row0) {
  if constexpr (I < TM) {
    epilogue_slice<TN, WN>(a, bidx, L, acc[I], stage, row0 + I * 32);
    epilogue_slices<I + 1, TM, TN, WN>(a, bidx, L, acc, stage, row0);
  }
}

// EPI_QK_NORM_ROPE for one 32-row slice of a wave of 64 columns: half a
// head of 128, the other half in the partner wave (wave ^ 1, same rows).
// Each lane walks eight rows of four columns as epilogue_slice does. The
// product plus bias is rounded to the output type (the projection's
// output), each row's sum of squares over the wave's 64 columns meets the
// partner's in LDS (ssq), the normalised, scaled values are rounded (the
// head norm's output) and staged, and after a barrier each lane reads the
// partner's value of the same rotary frequency: the low half stores
// l cos - h sin, the high half h cos + l sin (Transformer.cs:37-64).
// ssq holds 32 floats per wave.
__device__ __forceinline__ void qk_norm_rope_slice(const GemmArgs& a, int64_t bidx, f32x16 (&acc)[2], float* stage,
                                                   const float* partner_stage, float* ssq, int row0, int col0) {
  constexpr int CS = 64 + 4, C4 = 16, RSTEP = 4, IT = 8;
  const int lane = threadIdx.x & 63, lrow = lane & 31, lhalf = lane >> 5;
  const int wave = threadIdx.x >> 6;
  const int c4 = lane % C4, rl0 = lane / C4;
  const int col = col0 + c4 * 4;
  const int dim = col & 127;  // within the head
  const bool high = dim >= 64;
  // The weight of the wave's third (q or k), picked by arithmetic: a select
  // between two fields of the argument block would copy the block to
  // scratch memory.
  const uintptr_t wq = (uintptr_t)a.norm_q, wk = (uintptr_t)a.norm_k;
  const void* nw = (const void*)(wq + uintptr_t(col0 >= a.qk_cols / 2) * (wk - wq));
  float bias[4], w[4];
#pragma unroll
  for (int e = 0; e < 4; e++) {
    bias[e] = a.bias ? load_f(a.bias, a.bias_dtype, col + e) : 0.f;
    w[e] = nw ? load_f(nw, a.norm_dtype, dim + e) : 1.f;
  }
#pragma unroll
  for (int j = 0; j < 2; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) stage[(8 * (r >> 2) + 4 * lhalf + (r & 3)) * CS + j * 32 + lrow] = acc[j][r];
  __syncthreads();
  // The product rounded to the output type, back into the stage; each row's
  // sum of squares over the wave's 64 columns into ssq.
#pragma unroll
  for (int t = 0; t < IT; t++) {
    const int rl = rl0 + t * RSTEP;
    float4* sp = (float4*)&stage[rl * CS + c4 * 4];
    const float4 s = *sp;
    const float v0 = round_to(s.x + bias[0], a.c_dtype), v1 = round_to(s.y + bias[1], a.c_dtype),
                v2 = round_to(s.z + bias[2], a.c_dtype), v3 = round_to(s.w + bias[3], a.c_dtype);
    *sp = make_float4(v0, v1, v2, v3);
    float ss = v0 * v0 + v1 * v1 + v2 * v2 + v3 * v3;
#pragma unroll
    for (int o = 1; o < C4; o <<= 1) ss += __shfl_xor(ss, o, 64);
    if (c4 == 0) ssq[wave * 32 + rl] = ss;
  }
  __syncthreads();
  // The rotary table rows of this lane's eight rows are requested here, so
  // their latency passes under this pass and its barrier (rows past M read
  // row M - 1).
  const float* __restrict__ cos_t = a.rope_cos;
  const float* __restrict__ sin_t = a.rope_sin;
  float4 cs[IT], sn[IT];
  if (cos_t) {
#pragma unroll
    for (int t = 0; t < IT; t++) {
      const int64_t row = min(row0 + rl0 + t * RSTEP, a.M - 1);
      cs[t] = *(const float4*)(cos_t + row * 64 + (dim & 63));
      sn[t] = *(const float4*)(sin_t + row * 64 + (dim & 63));
    }
  }
  // The head norm's output, rounded, back into the stage.
  const float* pssq = ssq + (wave ^ 1) * 32;
#pragma unroll
  for (int t = 0; t < IT; t++) {
    const int rl = rl0 + t * RSTEP;
    const float r = 1.0f / sqrtf((ssq[wave * 32 + rl] + pssq[rl]) * (1.0f / 128) + a.norm_eps);
    float4* sp = (float4*)&stage[rl * CS + c4 * 4];
    const float4 v = *sp;
    *sp = make_float4(round_to(v.x * r * w[0], a.c_dtype), round_to(v.y * r * w[1], a.c_dtype),
                      round_to(v.z * r * w[2], a.c_dtype), round_to(v.w * r * w[3], a.c_dtype));
  }
  __syncthreads();
  const bool out_vec = aligned16(a.c, a.ldc, a.batch_c, dtype_size(a.c_dtype));
#pragma unroll
  for (int t = 0; t < IT; t++) {
    const int rl = rl0 + t * RSTEP, row = row0 + rl;
    if (row >= a.M) continue;
    const float4 n = *(const float4*)&stage[rl * CS + c4 * 4];
    float y[4] = {n.x, n.y, n.z, n.w};
    if (cos_t) {
      const float4 p = *(const float4*)&partner_stage[rl * CS + c4 * 4];
      const float nn[4] = {n.x, n.y, n.z, n.w}, pp[4] = {p.x, p.y, p.z, p.w};
      const float cc[4] = {cs[t].x, cs[t].y, cs[t].z, cs[t].w}, sv[4] = {sn[t].x, sn[t].y, sn[t].z, sn[t].w};
#pragma unroll
      for (int e = 0; e < 4; e++) y[e] = high ? nn[e] * cc[e] + pp[e] * sv[e] : nn[e] * cc[e] - pp[e] * sv[e];
    }
    const int64_t co = bidx * a.batch_c + int64_t(row) * a.ldc + col;
    if (out_vec) {
      store4_vec(a.c, a.c_dtype, co, y);
    } else {
#pragma unroll
      for (int e = 0; e < 4; e++) store_f(a.c, a.c_dtype, co + e, y[e]);
    }
  }
  __syncthreads();
}

// Slices I .. TM - 1 of EPI_QK_NORM_ROPE, expanded at compile time as
// epilogue_slices is.
template <int I, int TM>
__device__ __forceinline__ void qk_norm_rope_slices(const GemmArgs& a, int64_t bidx, f32x16 (&acc)[TM][2],
                                                    float* stage, const float* partner_stage, float* ssq, int row0,
                                                    int col0) {
  if constexpr (I < TM) {
    qk_norm_rope_slice(a, bidx, acc[I], stage, partner_stage, ssq, row0 + I * 32, col0);
    qk_norm_rope_slices<I + 1, TM>(a, bidx, acc, stage, partner_stage, ssq, row0, col0);
  }
}

// Writes the accumulators of one wave (TM x TN tiles of 32 x 32, the MFMA
// layout: lane l holds column l % 32, rows 8 (r / 4) + 4 (l / 32) + r % 4)
// through the epilogue, one 32-row slice at a time. A lane's four columns
// are the same in every row it visits, so its bias and gate are read once.
// stage must hold 32 x (WN + 4) floats for each wave and be free (the main
// loop is done). QKN: the kernel takes EPI_QK_NORM_ROPE (stage then holds
// 32 more floats per wave after the waves' stages); only its own
// instantiations carry that code.
template <int TM, int TN, int WN, bool QKN = false>
__device__ __forceinline__ void staged_epilogue(const GemmArgs& a, int64_t bidx, f32x16 (&acc)[TM][TN],
                                                float* stage, int row0, int col0) {
  if constexpr (QKN && WN == 64) {
    // The whole workgroup takes this path or none: qk_cols is a multiple of
    // the tile's width (gemm_qk_norm_ok).
    if (a.epilogue == EPI_QK_NORM_ROPE && col0 < a.qk_cols) {
      constexpr int CS = WN + 4;
      const int wave = threadIdx.x >> 6, waves = blockDim.x >> 6;
      float* all = stage - wave * 32 * CS;
      float* ssq = all + waves * 32 * CS;
      qk_norm_rope_slices<0, TM>(a, bidx, acc, stage, all + (wave ^ 1) * 32 * CS, ssq, row0, col0);
      return;
    }
  }
  constexpr int C4 = WN / 4;
  const int lane = threadIdx.x & 63;
  EpiLane L;
  L.c4 = lane % C4;
  L.rl0 = lane / C4;
  L.col = col0 + L.c4 * 4;
  L.n = min(4, a.N - L.col);
  const int ep = a.epilogue;
  const bool residual = ep == EPI_GATED_RESIDUAL || ep == EPI_RESIDUAL;
  const bool act = ep == EPI_GELU_TANH || ep == EPI_GELU || ep == EPI_SILU || ep == EPI_SWIGLU;
  L.out_vec = aligned16(a.c, a.ldc, a.batch_c, dtype_size(a.c_dtype));
  const bool res_vec = residual && aligned16(a.resid, a.ldr, a.batch_r, dtype_size(a.r_dtype));
  // A gate per row is read per row; one or two gate rows once per lane.
  L.gate_rows = ep == EPI_GATED_RESIDUAL && a.ldg != 0;
  // Uniform over the wave: all of its columns in range, aligned rows.
  L.fast = !act && !L.gate_rows && col0 + WN <= a.N && L.out_vec && (!residual || res_vec);
  L.bias = make_float4(0.f, 0.f, 0.f, 0.f);
  L.gate = make_float4(1.f, 1.f, 1.f, 1.f);
  L.gate2 = L.gate;
  if (L.n > 0 && a.bias) L.bias = load_cols(a.bias, a.bias_dtype, L.col, L.n, (uintptr_t)a.bias % 16 == 0);
  if (L.n > 0 && ep == EPI_GATED_RESIDUAL && !L.gate_rows) {
    const int gs = dtype_size(a.gate_dtype);
    L.gate = load_cols(a.gate, a.gate_dtype, bidx * a.batch_gate + L.col, L.n, aligned16(a.gate, a.batch_gate, 0, gs));
    L.gate2 = a.gate_split_off == 0
                  ? L.gate
                  : load_cols(a.gate, a.gate_dtype, bidx * a.batch_gate + a.gate_split_off + L.col, L.n,
                              aligned16(a.gate, a.batch_gate, a.gate_split_off, gs));
  }
  epilogue_slices<0, TM, TN, WN>(a, bidx, L, acc, stage, row0);
}

// ---- The fast epilogue ------------------------------------------------------
//
// The same staging as staged_epilogue, for launches whose every wave column
// is in range, whose output (and residual, of the output's type) rows are
// 16-byte aligned, whose gate is one row and whose epilogue is linear (bias,
// row bias, residual, gated residual) or an activation (epi_fast_ok). The
// output type and the mode are decided once per wave, so each slice is one
// straight run of code: an epilogue with a type or mode test per row left
// taken branches all through it, and refetching that code cost 16-18 us per
// 256 x 256 tile (2 us straight).

// Four consecutive values at byte offset off of a bounds-checked buffer,
// widened to fp32 (zeros past its end).
template <typename OT>
__device__ __forceinline__ float4 buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  if constexpr (sizeof(OT) == 4) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  } else {
    const uint2 u = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0));
    const OT* h = (const OT*)&u;
    return make_float4((float)h[0], (float)h[1], (float)h[2], (float)h[3]);
  }
}
// Stores four consecutive outputs at byte offset off (dropped past the
// buffer's end).
template <typename OT>
__device__ __forceinline__ void buf_store4(__amdgpu_buffer_rsrc_t r, uint32_t off, const float (&v)[4]) {
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
  if constexpr (sizeof(OT) == 4) {
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, make_float4(v[0], v[1], v[2], v[3])), r, off, 0, 0);
  } else {
    OT h[4] = {(OT)v[0], (OT)v[1], (OT)v[2], (OT)v[3]};
    __builtin_amdgcn_raw_buffer_store_b64(*(const u32x2*)h, r, off, 0, 0);
  }
}

enum FastMode { FM_PLAIN, FM_RESID, FM_ACT };

// The row bias of rows row0 + t * step (zeros without one; rows past M
// read row M - 1, whose outputs are dropped).
template <int IT>
__device__ __forceinline__ void load_row_bias(const GemmArgs& a, int row0, int step, float (&rb)[IT]) {
  const int dt = a.row_bias_dtype;
  if (!a.row_bias) {
#pragma unroll
    for (int t = 0; t < IT; t++) rb[t] = 0.f;
  } else if (dt == NDX_F32) {
#pragma unroll
    for (int t = 0; t < IT; t++) rb[t] = ((const float*)a.row_bias)[min(row0 + t * step, a.M - 1)];
  } else if (dt == NDX_F16) {
#pragma unroll
    for (int t = 0; t < IT; t++) rb[t] = (float)((const _Float16*)a.row_bias)[min(row0 + t * step, a.M - 1)];
  } else {
#pragma unroll
    for (int t = 0; t < IT; t++) rb[t] = (float)((const __bf16*)a.row_bias)[min(row0 + t * step, a.M - 1)];
  }
}

// One 32-row slice of the fast epilogue. T is the product's type (the
// residual adds the product rounded to it), OT the output's. The output
// and the residual are buffers ending at row M: a row past M stores
// nothing and reads zeros with no branch, so the stores of a slice go out
// back to back (a per-row branch made the compiler wait for each store
// before the next).
template <int TN, int WN, typename T, typename OT, int MODE>
__device__ __forceinline__ void fast_slice(const GemmArgs& a, int64_t bidx, const EpiLane& L, f32x16 (&acc)[TN],
                                           float* stage, int row0) {
  constexpr int CS = WN + 4, C4 = WN / 4, RSTEP = 64 / C4, IT = 32 / RSTEP;
  // Residual rows in flight at once: all of a slice's on 64-column waves (8),
  // groups of 8 on 128-column ones (16 rows a slice would hold 64 more
  // registers and spill).
  constexpr int PF = IT < 8 ? IT : 8;
  constexpr int ES = (int)sizeof(OT);
  const int lane = threadIdx.x & 63, lrow = lane & 31, lhalf = lane >> 5;
  const __amdgpu_buffer_rsrc_t rc = make_rsrc((const OT*)a.c + bidx * a.batch_c, (uint32_t)(int64_t(a.M) * a.ldc * ES));
  const __amdgpu_buffer_rsrc_t rr = make_rsrc(MODE == FM_RESID ? (const OT*)a.resid + bidx * a.batch_r : nullptr,
                                              MODE == FM_RESID ? (uint32_t)(int64_t(a.M) * a.ldr * ES) : 0u);
  float4 res[MODE == FM_RESID ? PF : 1];
  float rb[IT];
  auto load_res = [&](int h) __attribute__((always_inline)) {
    if constexpr (MODE == FM_RESID) {
#pragma unroll
      for (int t = 0; t < PF; t++) {
        const int row = row0 + L.rl0 + (h + t) * RSTEP;
        res[t] = buf_load4<OT>(rr, uint32_t((row * a.ldr + L.col) * ES));
      }
    }
  };
  load_res(0);
  load_row_bias(a, row0 + L.rl0, RSTEP, rb);
#pragma unroll
  for (int j = 0; j < TN; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) stage[(8 * (r >> 2) + 4 * lhalf + (r & 3)) * CS + j * 32 + lrow] = acc[j][r];
  wave_lds_sync();
  if constexpr (MODE == FM_ACT) {
    // Rolled loops, one per activation (their code is long).
    const int ep = a.epilogue;
    auto act_rows = [&](auto f) __attribute__((always_inline)) {
#pragma unroll 1
      for (int t = 0; t < IT; t++) {
        const int rl = L.rl0 + t * RSTEP, row = row0 + rl;
        const float4 v = *(const float4*)&stage[rl * CS + L.c4 * 4];
        float b = 0.f;
#pragma unroll
        for (int u = 0; u < IT; u++) b = u == t ? rb[u] : b;
        float x[4] = {f(v.x + L.bias.x + b), f(v.y + L.bias.y + b), f(v.z + L.bias.z + b), f(v.w + L.bias.w + b)};
        buf_store4<OT>(rc, uint32_t((row * a.ldc + L.col) * ES), x);
      }
    };
    if (ep == EPI_GELU_TANH) act_rows([](float x) { return gelu_tanh_f(x); });
    else if (ep == EPI_GELU) act_rows([](float x) { return gelu_f(x); });
    else act_rows([](float x) { return silu_f(x); });
  } else {
#pragma unroll
    for (int h = 0; h < IT; h += PF) {
      if (h > 0) load_res(h);
#pragma unroll
      for (int u = 0; u < PF; u++) {
        const int t = h + u;
        const int rl = L.rl0 + t * RSTEP, row = row0 + rl;
        const float4 v = *(const float4*)&stage[rl * CS + L.c4 * 4];
        float x[4] = {v.x + L.bias.x + rb[t], v.y + L.bias.y + rb[t], v.z + L.bias.z + rb[t],
                      v.w + L.bias.w + rb[t]};
        if constexpr (MODE == FM_RESID) {
          const float4 g = row >= a.gate_split ? L.gate2 : L.gate;
          x[0] = res[u].x + g.x * (float)(T)x[0];
          x[1] = res[u].y + g.y * (float)(T)x[1];
          x[2] = res[u].z + g.z * (float)(T)x[2];
          x[3] = res[u].w + g.w * (float)(T)x[3];
        }
        buf_store4<OT>(rc, uint32_t((row * a.ldc + L.col) * ES), x);
      }
    }
  }
  wave_lds_sync();
}

template <int I, int TM, int TN, int WN, typename T, typename OT, int MODE>
__device__ __forceinline__ void fast_slices(const GemmArgs& a, int64_t bidx, const EpiLane& L, f32x16 (&acc)[TM][TN],
                                            float* stage, int row0) {
  if constexpr (I < TM) {
    fast_slice<TN, WN, T, OT, MODE>(a, bidx, L, acc[I], stage, row0 + I * 32);
    fast_slices<I + 1, TM, TN, WN, T, OT, MODE>(a, bidx, L, acc, stage, row0);
  }
}

template <int TM, int TN, int WN, typename T, typename OT>
__device__ __forceinline__ void fast_epilogue_typed(const GemmArgs& a, int64_t bidx, const EpiLane& L,
                                                    f32x16 (&acc)[TM][TN], float* stage, int row0) {
  const int ep = a.epilogue;
  if (ep == EPI_GATED_RESIDUAL || ep == EPI_RESIDUAL)
    fast_slices<0, TM, TN, WN, T, OT, FM_RESID>(a, bidx, L, acc, stage, row0);
  else if (ep == EPI_GELU_TANH || ep == EPI_GELU || ep == EPI_SILU)
    fast_slices<0, TM, TN, WN, T, OT, FM_ACT>(a, bidx, L, acc, stage, row0);
  else
    fast_slices<0, TM, TN, WN, T, OT, FM_PLAIN>(a, bidx, L, acc, stage, row0);
}

// EPI_QK_NORM_ROPE on waves 128 columns wide: each wave's columns are one
// whole head of q or k (or v columns, which take the plain path). Per row:
// the product plus bias rounded to the output type, its sum of squares over
// the head (the lane's four, then lanes ^1, ^2, ^4, ^8: 64 columns, then
// ^16: the other 64, the summation order of two 64-column halves), the
// RMS-normalised values times the weight rounded again (the head norm's
// output), then the rotate-half rotation in fp32 with the partner value
// (dim +- 64) from lane ^ 16 and the row's rotary table entry
// (Transformer.cs:37-64). No LDS beyond the wave's own stage and no
// barrier: the wave runs its epilogue alone, as fast_slice does.
template <int TN, typename OT, bool ROT>
__device__ __forceinline__ void fast_qkn_slice(const GemmArgs& a, int64_t bidx, const EpiLane& L, f32x16 (&acc)[TN],
                                               float* stage, int row0, const float (&w)[4]) {
  constexpr int WN = 128, CS = WN + 4, C4 = WN / 4, RSTEP = 64 / C4, IT = 32 / RSTEP, HALF = 8;
  constexpr int ES = (int)sizeof(OT);
  const int lane = threadIdx.x & 63, lrow = lane & 31, lhalf = lane >> 5;
  const __amdgpu_buffer_rsrc_t rc = make_rsrc((const OT*)a.c + bidx * a.batch_c, (uint32_t)(int64_t(a.M) * a.ldc * ES));
  const int dim = L.col & 127;
  const bool high = dim >= 64;
#pragma unroll
  for (int j = 0; j < TN; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) stage[(8 * (r >> 2) + 4 * lhalf + (r & 3)) * CS + j * 32 + lrow] = acc[j][r];
  wave_lds_sync();
#pragma unroll
  for (int h = 0; h < IT; h += HALF) {
    // The rotary rows of these rows (rows past M read row M - 1).
    float4 cs[HALF], sn[HALF];
    if constexpr (ROT) {
#pragma unroll
      for (int t = 0; t < HALF; t++) {
        const int64_t row = min(row0 + L.rl0 + (h + t) * RSTEP, a.M - 1);
        cs[t] = *(const float4*)(a.rope_cos + row * 64 + (dim & 63));
        sn[t] = *(const float4*)(a.rope_sin + row * 64 + (dim & 63));
      }
    }
#pragma unroll
    for (int t = 0; t < HALF; t++) {
      const int rl = L.rl0 + (h + t) * RSTEP, row = row0 + rl;
      const float4 sv = *(const float4*)&stage[rl * CS + L.c4 * 4];
      const float v[4] = {(float)(OT)(sv.x + L.bias.x), (float)(OT)(sv.y + L.bias.y), (float)(OT)(sv.z + L.bias.z),
                          (float)(OT)(sv.w + L.bias.w)};
      float ss = v[0] * v[0] + v[1] * v[1] + v[2] * v[2] + v[3] * v[3];
#pragma unroll
      for (int o = 1; o < 16; o <<= 1) ss += __shfl_xor(ss, o, 64);
      ss += __shfl_xor(ss, 16, 64);
      const float r = 1.0f / sqrtf(ss * (1.0f / 128) + a.norm_eps);
      float n[4], y[4];
#pragma unroll
      for (int e = 0; e < 4; e++) n[e] = (float)(OT)(v[e] * r * w[e]);
      if constexpr (ROT) {
        const float cc[4] = {cs[t].x, cs[t].y, cs[t].z, cs[t].w}, sx[4] = {sn[t].x, sn[t].y, sn[t].z, sn[t].w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const float pv = __shfl_xor(n[e], 16, 64);
          y[e] = high ? n[e] * cc[e] + pv * sx[e] : n[e] * cc[e] - pv * sx[e];
        }
      } else {
#pragma unroll
        for (int e = 0; e < 4; e++) y[e] = n[e];
      }
      buf_store4<OT>(rc, uint32_t((row * a.ldc + L.col) * ES), y);
    }
  }
  wave_lds_sync();
}

template <int I, int TM, int TN, typename OT, bool ROT>
__device__ __forceinline__ void fast_qkn_slices(const GemmArgs& a, int64_t bidx, const EpiLane& L,
                                                f32x16 (&acc)[TM][TN], float* stage, int row0, const float (&w)[4]) {
  if constexpr (I < TM) {
    fast_qkn_slice<TN, OT, ROT>(a, bidx, L, acc[I], stage, row0 + I * 32, w);
    fast_qkn_slices<I + 1, TM, TN, OT, ROT>(a, bidx, L, acc, stage, row0, w);
  }
}

template <int TM, int TN, typename OT>
__device__ __forceinline__ void fast_qkn(const GemmArgs& a, int64_t bidx, const EpiLane& L, f32x16 (&acc)[TM][TN],
                                         float* stage, int row0, int col0) {
  // The weight of the wave's head (q or k), picked by arithmetic (a select
  // between two argument fields would copy the block to scratch).
  const uintptr_t wq = (uintptr_t)a.norm_q, wk = (uintptr_t)a.norm_k;
  const void* nw = (const void*)(wq + uintptr_t(col0 >= a.qk_cols / 2) * (wk - wq));
  float w[4];
  const int dim = L.col & 127;
#pragma unroll
  for (int e = 0; e < 4; e++) w[e] = nw ? load_f(nw, a.norm_dtype, dim + e) : 1.f;
  if (a.rope_cos) fast_qkn_slices<0, TM, TN, OT, true>(a, bidx, L, acc, stage, row0, w);
  else fast_qkn_slices<0, TM, TN, OT, false>(a, bidx, L, acc, stage, row0, w);
}

template <int TM, int TN, int WN, typename T>
__device__ __forceinline__ void fast_epilogue(const GemmArgs& a, int64_t bidx, f32x16 (&acc)[TM][TN], float* stage,
                                              int row0, int col0) {
  constexpr int C4 = WN / 4;
  const int lane = threadIdx.x & 63;
  EpiLane L;
  L.c4 = lane % C4;
  L.rl0 = lane / C4;
  L.col = col0 + L.c4 * 4;
  L.n = 4;
  L.fast = true;
  L.out_vec = true;
  L.gate_rows = false;
  L.bias = a.bias ? load_cols(a.bias, a.bias_dtype, L.col, 4, (uintptr_t)a.bias % 16 == 0) : make_float4(0.f, 0.f, 0.f, 0.f);
  L.gate = make_float4(1.f, 1.f, 1.f, 1.f);
  L.gate2 = L.gate;
  if (a.epilogue == EPI_GATED_RESIDUAL) {
    const int gs = dtype_size(a.gate_dtype);
    L.gate = load_cols(a.gate, a.gate_dtype, bidx * a.batch_gate + L.col, 4, aligned16(a.gate, a.batch_gate, 0, gs));
    L.gate2 = a.gate_split_off == 0
                  ? L.gate
                  : load_cols(a.gate, a.gate_dtype, bidx * a.batch_gate + a.gate_split_off + L.col, 4,
                              aligned16(a.gate, a.batch_gate, a.gate_split_off, gs));
  }
  if constexpr (WN == 128) {
    // Uniform over the workgroup: qk_cols is a multiple of the tile width.
    if (a.epilogue == EPI_QK_NORM_ROPE && col0 < a.qk_cols) {
      if (a.c_dtype == NDX_F32) fast_qkn<TM, TN, float>(a, bidx, L, acc, stage, row0, col0);
      else if (a.c_dtype == NDX_BF16) fast_qkn<TM, TN, __bf16>(a, bidx, L, acc, stage, row0, col0);
      else fast_qkn<TM, TN, _Float16>(a, bidx, L, acc, stage, row0, col0);
      return;
    }
  }
  if (a.c_dtype == NDX_F32) fast_epilogue_typed<TM, TN, WN, T, float>(a, bidx, L, acc, stage, row0);
  else if (a.c_dtype == NDX_BF16) fast_epilogue_typed<TM, TN, WN, T, __bf16>(a, bidx, L, acc, stage, row0);
  else fast_epilogue_typed<TM, TN, WN, T, _Float16>(a, bidx, L, acc, stage, row0);
}

// Whether a launch may take fast_epilogue with tiles BN wide (QKN: the
// fused head norm on 128-column waves).
static bool epi_fast_ok(const GemmArgs& a, int bn, bool qkn = false) {
  if (a.M == 0) return true;  // the absent second product of a launch
  const int ep = a.epilogue;
  const bool residual = ep == EPI_GATED_RESIDUAL || ep == EPI_RESIDUAL;
  if (!(ep == EPI_NONE || ep == EPI_GELU_TANH || ep == EPI_GELU || ep == EPI_SILU || residual ||
        (qkn && ep == EPI_QK_NORM_ROPE && a.qk_cols % 128 == 0)))
    return false;
  if (a.c_dtype != NDX_F32 && a.c_dtype != NDX_BF16 && a.c_dtype != NDX_F16) return false;
  if (a.N % bn) return false;
  if (residual && a.r_dtype != a.c_dtype) return false;
  // Without pointers (a kernel family named before a run) the shape decides.
  if (!a.c) return true;
  if (!aligned16(a.c, a.ldc, a.batch_c, dtype_size(a.c_dtype))) return false;
  if (residual && (a.r_dtype != a.c_dtype || !aligned16(a.resid, a.ldr, a.batch_r, dtype_size(a.r_dtype)))) return false;
  if (ep == EPI_GATED_RESIDUAL && a.ldg != 0) return false;
  // Output and residual rows are addressed by 32-bit byte offsets from the
  // batch's first row; a row at or past M must lie past the buffer's end.
  const int64_t lim = int64_t(1) << 31, es = dtype_size(a.c_dtype);
  if (int64_t(a.M) * a.ldc * es >= lim || (residual && int64_t(a.M) * a.ldr * es >= lim)) return false;
  if (a.ldc < a.N || (residual && a.ldr < a.N)) return false;
  // Rows up to a tile past M stay below 2^32 bytes (no wrap into range).
  if (a.ldc * es >= (int64_t(1) << 22) || (residual && a.ldr * es >= (int64_t(1) << 22))) return false;
  return true;
}

// Element offset of 16-byte chunk c of row r in a swizzled [rows][64] tile
// (128-byte rows). gfx950's LDS serves a ds_read_b128 sixteen lanes at a
// time across 64 four-byte banks (256 bytes); the fragment reads have those
// lanes on sixteen consecutive rows at one logical chunk, so the physical
// chunk c ^ ((r / 2) % 8) puts them on sixteen distinct 16-byte bank
// groups ((r % 2) * 8 + physical chunk). A plain c ^ (r % 8) would put rows
// r and r + 8 on the same banks: a two-way conflict on every read.
__device__ __forceinline__ int swz_key(int r) { return (r >> 1) & 7; }
__device__ __forceinline__ int swz(int r, int c) { return r * BK + ((c ^ swz_key(r)) << 3); }

__device__ __forceinline__ uint4 load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

template <int BM, int BN, int WM, int WN, typename T, bool W_INT8>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_mfma_kernel(GemmArgs a, int grid) {
  typedef typename MfmaOp<T>::V V;
  constexpr int WAVES_N = BN / WN;
  constexpr int NT = (BM / WM) * (BN / WN) * 64;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_PER = BM * (BK / 8) / NT;
  constexpr int B_CHUNK = W_INT8 ? 16 : 8;  // elements per 16-byte global load
  constexpr int B_PER = BN * (BK / B_CHUNK) / NT;
  static_assert(A_PER * NT == BM * (BK / 8), "A tile does not split over the threads");
  static_assert(B_PER * NT == BN * (BK / B_CHUNK), "B tile does not split over the threads");
  // One LDS block holds the double-buffered A and B tiles during the K
  // loop and the epilogue's staging rows afterwards.
  constexpr int TILE_BYTES = 2 * (BM + BN) * BK * (int)sizeof(T);
  constexpr int STAGE_BYTES = (BM / WM) * (BN / WN) * 32 * (WN + 4) * 4;
  __shared__ __attribute__((aligned(16))) char smem[TILE_BYTES > STAGE_BYTES ? TILE_BYTES : STAGE_BYTES];
  T (*As)[BM * BK] = reinterpret_cast<T (*)[BM * BK]>(smem);
  T (*Bs)[BN * BK] = reinterpret_cast<T (*)[BN * BK]>(smem + 2 * BM * BK * sizeof(T));

  int tm, tn;
  if (!tile_of(blockIdx.x, grid, (a.M + BM - 1) / BM, (a.N + BN - 1) / BN, tm, tn)) return;
  const int64_t bidx = blockIdx.y;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;

  // The A rows of this batch and the whole weight, as bounds-checked
  // buffers (their byte spans are below 2^31, checked on the host).
  const T* A = (const T*)a.a + bidx * a.batch_a;
  const __amdgpu_buffer_rsrc_t ra_rsrc =
      make_rsrc(A, (uint32_t)((int64_t(a.M - 1) * a.lda + a.K) * (int64_t)sizeof(T)));
  const int wes = W_INT8 ? 1 : (int)sizeof(T);
  const __amdgpu_buffer_rsrc_t rw_rsrc = make_rsrc(a.w, (uint32_t)((int64_t(a.N - 1) * a.ldw + a.K) * wes));

  // Per-thread load coordinates are fixed across the K loop; the K offset
  // is added per tile.
  uint32_t a_off[A_PER], w_off[B_PER];
  int a_k[A_PER], w_k[B_PER];
#pragma unroll
  for (int i = 0; i < A_PER; i++) {
    const int id = tid + i * NT, r = id >> 3, c = id & 7;
    a_k[i] = c * 8;
    a_off[i] = (m0 + r < a.M) ? (uint32_t)((int64_t(m0 + r) * a.lda + c * 8) * (int64_t)sizeof(T)) : kOutOfRange;
  }
#pragma unroll
  for (int i = 0; i < B_PER; i++) {
    const int id = tid + i * NT, r = id / (BK / B_CHUNK), c = id % (BK / B_CHUNK);
    w_k[i] = c * B_CHUNK;
    w_off[i] = (n0 + r < a.N) ? (uint32_t)((int64_t(n0 + r) * a.ldw + c * B_CHUNK) * wes) : kOutOfRange;
  }

  uint4 ra[A_PER];
  uint4 rb[B_PER];
  float rs[W_INT8 ? B_PER : 1];

  auto load_tile = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      const bool in = k0 + a_k[i] < a.K;
      ra[i] = load16(ra_rsrc, in ? a_off[i] + uint32_t(k0 * (int)sizeof(T)) : kOutOfRange);
    }
#pragma unroll
    for (int i = 0; i < B_PER; i++) {
      const bool in = k0 + w_k[i] < a.K;
      rb[i] = load16(rw_rsrc, in ? w_off[i] + uint32_t(k0 * wes) : kOutOfRange);
      if (W_INT8) {
        const int id = tid + i * NT, r = id / (BK / 16);
        const int gn = min(n0 + r, a.N - 1);
        rs[W_INT8 ? i : 0] = scale_at(a.scales, a.s_dtype, int64_t(gn) * a.lds + (k0 + w_k[i]) / a.qblock);
      }
    }
  };

  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_PER; i++) {
      int id = tid + i * NT;
      int r = id >> 3, c = id & 7;
      *(uint4*)&As[buf][swz(r, c)] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_PER; i++) {
      int id = tid + i * NT;
      if (W_INT8) {
        int r = id / (BK / 16), c = id % (BK / 16);
        const int8_t* q = (const int8_t*)&rb[i];
        float s = rs[W_INT8 ? i : 0];
        V lo, hi;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          lo[e] = (T)(float(q[e]) * s);
          hi[e] = (T)(float(q[e + 8]) * s);
        }
        *(V*)&Bs[buf][swz(r, 2 * c)] = lo;
        *(V*)&Bs[buf][swz(r, 2 * c + 1)] = hi;
      } else {
        int r = id >> 3, c = id & 7;
        *(uint4*)&Bs[buf][swz(r, c)] = rb[i];
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int KT = (a.K + BK - 1) / BK;
  load_tile(0);
  store_tile(0);
  __syncthreads();

  const int lrow = lane & 31, lhalf = lane >> 5;
  for (int kt = 0; kt < KT; kt++) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_tile(kt + 1);
#pragma unroll
    for (int s = 0; s < BK / 16; s++) {
      V af[TM], bf[TN];
      const int c = 2 * s + lhalf;
#pragma unroll
      for (int i = 0; i < TM; i++) af[i] = *(const V*)&As[cur][swz(wm * WM + i * 32 + lrow, c)];
#pragma unroll
      for (int j = 0; j < TN; j++) bf[j] = *(const V*)&Bs[cur][swz(wn * WN + j * 32 + lrow, c)];
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = MfmaOp<T>::mma(af[i], bf[j], acc[i][j]);
    }
    if (kt + 1 < KT) store_tile(cur ^ 1);
    __syncthreads();
  }

  float* stage = reinterpret_cast<float*>(smem) + wave * 32 * (WN + 4);
  staged_epilogue<TM, TN, WN>(a, bidx, acc, stage, m0 + wm * WM, n0 + wn * WN);
}

// The large-tile GEMM with the tile loads going straight to LDS
// (buffer_load_dwordx4 ... lds): each wave-wide load fills one contiguous
// kilobyte of LDS, eight 128-byte tile rows, lane l landing at l * 16 bytes.
// The XOR swizzle is applied on the source side: lane l fetches the K chunk
// (l % 8) ^ (row % 8) of its row, so the tile lands swizzled and no register
// or LDS-write instruction is spent on staging. Fragments are double
// buffered in registers: the LDS reads of step s + 1 are in flight while
// the MFMAs of step s run.

// a0 and a1 are two products with the same N, K and batch run as one grid
// (a0's row tiles first, then a1's); a1.M = 0 for a single product.
template <int BM, int BN, int WM, int WN, typename T, bool CONV, bool KFULL, bool QKN, bool FAST>
__device__ __forceinline__ void gemm_lds_body(const GemmArgs& a0, const GemmArgs& a1, int grid) {
  typedef typename MfmaOp<T>::V V;
  constexpr int WAVES_N = BN / WN;
  constexpr int NW = (BM / WM) * (BN / WN);
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_LOADS = BM / 8 / NW;  // kilobyte loads per wave per tile
  constexpr int B_LOADS = BN / 8 / NW;
  static_assert(A_LOADS * 8 * NW == BM && B_LOADS * 8 * NW == BN, "tile rows do not split over the waves");
  constexpr int TILE_BYTES = 2 * (BM + BN) * BK * (int)sizeof(T);
  // The epilogue's stage, and for EPI_QK_NORM_ROPE 32 floats per wave after
  // it (the row sums).
  constexpr int STAGE_BYTES = NW * 32 * (WN + 4) * 4 + (QKN ? NW * 32 * 4 : 0);
  __shared__ __attribute__((aligned(1024))) char smem[TILE_BYTES > STAGE_BYTES ? TILE_BYTES : STAGE_BYTES];
  T (*As)[BM * BK] = reinterpret_cast<T (*)[BM * BK]>(smem);
  T (*Bs)[BN * BK] = reinterpret_cast<T (*)[BN * BK]>(smem + 2 * BM * BK * sizeof(T));

  int tm, tn;
  const int tiles_m0 = (a0.M + BM - 1) / BM;
  if (!tile_of(blockIdx.x, grid, tiles_m0 + (a1.M + BM - 1) / BM, (a0.N + BN - 1) / BN, tm, tn)) return;
  const bool second = tm >= tiles_m0;
  const GemmArgs& a = second ? a1 : a0;
  if (second) tm -= tiles_m0;
  const int64_t bidx = blockIdx.y;
  const int m0 = tm * BM, n0 = tn * BN;
  // The wave index is uniform: from an SGPR, every LDS destination of the
  // tile DMA is scalar.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  constexpr int ES = (int)sizeof(T);

  const T* A = (const T*)a.a + bidx * a.batch_a;
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)((int64_t(a.M - 1) * a.lda + a.K) * ES));
  const __amdgpu_buffer_rsrc_t rw =
      CONV ? make_rsrc((const T*)a.w + bidx * a.batch_w,
                       (uint32_t)(int64_t(a.conv_h >> a.conv_up) * (a.conv_w >> a.conv_up) * a.conv_c * ES))
           : make_rsrc(a.w, (uint32_t)((int64_t(a.N - 1) * a.ldw + a.K) * ES));

  // Lane l of a kilobyte load: row (l / 8) of its 8-row group, physical
  // chunk l % 8 holding logical K chunk (l % 8) ^ swz_key(row). Group q
  // covers rows 8 q .. 8 q + 7, so swz_key(row) = 4 (q % 2) + (l / 8) / 2:
  // the chunk depends on the group's parity.
  const int lrow8 = lane >> 3;
  const int kchunk_q[2] = {(lane & 7) ^ (lrow8 >> 1), (lane & 7) ^ (4 | (lrow8 >> 1))};
  uint32_t a_row[A_LOADS], w_row[B_LOADS];
  int pix_y[CONV ? B_LOADS : 1], pix_x[CONV ? B_LOADS : 1];
#pragma unroll
  for (int i = 0; i < A_LOADS; i++) {
    const int r = (wave * A_LOADS + i) * 8 + lrow8;
    a_row[i] = m0 + r < a.M ? (uint32_t)(int64_t(m0 + r) * a.lda * ES) : kOutOfRange;
  }
#pragma unroll
  for (int i = 0; i < B_LOADS; i++) {
    const int r = (wave * B_LOADS + i) * 8 + lrow8;
    if (CONV) {
      // Output pixel n0 + r reads input rows oy * stride - pad + ky; a row
      // past the output puts its taps far outside the image.
      const int n = n0 + r;
      const int oy = n / a.conv_wo, ox = n - oy * a.conv_wo;
      pix_y[i] = n < a.N ? oy * a.conv_stride - a.conv_pad : -(1 << 20);
      pix_x[i] = ox * a.conv_stride - a.conv_pad;
    } else {
      w_row[i] = n0 + r < a.N ? (uint32_t)(int64_t(n0 + r) * a.ldw * ES) : kOutOfRange;
    }
  }

  // A convolution whose K runs over the taps without padding between them:
  // each lane's two 8-channel chunks (q) keep their own tap and channel,
  // set here for tile 0 and advanced by BK as each tile is issued (tiles
  // are issued in order, 0 to KT).
  int cky[2] = {0, 0}, ckx[2] = {0, 0}, cci[2] = {0, 0};
  if constexpr (CONV) {
    if (a.conv_kcont) {
#pragma unroll
      for (int q = 0; q < 2; q++) {
        const int k = kchunk_q[q] * 8, tap = k / a.conv_c;
        cci[q] = k - tap * a.conv_c;
        cky[q] = tap / a.conv_kw;
        ckx[q] = tap - cky[q] * a.conv_kw;
      }
    }
  }

  // With K a multiple of BK (KFULL) no tile reaches past K except the one
  // loaded after the last (never read): no per-load K check. A row past M
  // keeps kOutOfRange plus any K offset, still past the buffer's end.
  auto issue_tile = [&](int kt, int buf) {
    int k[2];
    bool kin[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
      k[q] = kt * BK + kchunk_q[q] * 8;
      kin[q] = k[q] < a.K;
    }
    if constexpr (KFULL) {
#pragma unroll
      for (int i = 0; i < A_LOADS; i++) {
        const int q = (wave * A_LOADS + i) & 1;
        const uint32_t off = a_row[i] + uint32_t(k[q] * ES);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)&As[buf][(wave * A_LOADS + i) * 8 * BK], 16, off, 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < A_LOADS; i++) {
        const int q = (wave * A_LOADS + i) & 1;
        const uint32_t off = (kin[q] && a_row[i] != kOutOfRange) ? a_row[i] + uint32_t(k[q] * ES) : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)&As[buf][(wave * A_LOADS + i) * 8 * BK], 16, off, 0, 0, 0);
      }
    }
    if constexpr (CONV) {
      if (a.conv_kcont) {
        // Each chunk at its own tap: past the last tap (cky == conv_kh) it
        // reads zeros, as it does outside the image.
        const int up = a.conv_up, row_w = a.conv_w >> up;
#pragma unroll
        for (int i = 0; i < B_LOADS; i++) {
          const int q = (wave * B_LOADS + i) & 1;
          const int iy = pix_y[i] + cky[q], ix = pix_x[i] + ckx[q];
          const bool in = cky[q] < a.conv_kh && (unsigned)iy < (unsigned)a.conv_h && (unsigned)ix < (unsigned)a.conv_w;
          const uint32_t off =
              in ? uint32_t((((iy >> up) * row_w + (ix >> up)) * a.conv_c + cci[q]) * ES) : kOutOfRange;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)&Bs[buf][(wave * B_LOADS + i) * 8 * BK], 16, off, 0, 0,
                                                   0);
        }
#pragma unroll
        for (int q = 0; q < 2; q++) {
          cci[q] += BK;
          while (cci[q] >= a.conv_c) {
            cci[q] -= a.conv_c;
            if (++ckx[q] == a.conv_kw) {
              ckx[q] = 0;
              cky[q]++;
            }
          }
        }
        return;
      }
      // A K tile lies within one tap (conv_cin is a multiple of BK): (ky,
      // kx) and the channel offset are uniform over the workgroup. An
      // 8-channel chunk at or past conv_c (a multiple of 8) reads zeros;
      // through the upsample, pixel (iy, ix) is stored at (iy / 2, ix / 2).
      const int k0 = kt * BK;
      const int tap = k0 / a.conv_cin;
      const int ci0 = k0 - tap * a.conv_cin;
      const int ky = tap / a.conv_kw, kx = tap - ky * a.conv_kw;
      const int up = a.conv_up, row_w = a.conv_w >> up;
#pragma unroll
      for (int i = 0; i < B_LOADS; i++) {
        const int q = (wave * B_LOADS + i) & 1;
        const int iy = pix_y[i] + ky, ix = pix_x[i] + kx, ci = ci0 + kchunk_q[q] * 8;
        const bool in =
            kin[q] && ci < a.conv_c && (unsigned)iy < (unsigned)a.conv_h && (unsigned)ix < (unsigned)a.conv_w;
        const uint32_t off = in ? uint32_t((((iy >> up) * row_w + (ix >> up)) * a.conv_c + ci) * ES) : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)&Bs[buf][(wave * B_LOADS + i) * 8 * BK], 16, off, 0, 0, 0);
      }
    } else if constexpr (KFULL) {
#pragma unroll
      for (int i = 0; i < B_LOADS; i++) {
        const int q = (wave * B_LOADS + i) & 1;
        const uint32_t off = w_row[i] + uint32_t(k[q] * ES);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)&Bs[buf][(wave * B_LOADS + i) * 8 * BK], 16, off, 0, 0, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < B_LOADS; i++) {
        const int q = (wave * B_LOADS + i) & 1;
        const uint32_t off = (kin[q] && w_row[i] != kOutOfRange) ? w_row[i] + uint32_t(k[q] * ES) : kOutOfRange;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)&Bs[buf][(wave * B_LOADS + i) * 8 * BK], 16, off, 0, 0, 0);
      }
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int lrow = lane & 31, lhalf = lane >> 5;
  const int KT = (a.K + BK - 1) / BK;
  issue_tile(0, 0);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  V af[2][TM], bf[2][TN];
#pragma unroll
  for (int i = 0; i < TM; i++) af[0][i] = *(const V*)&As[0][swz(wm * WM + i * 32 + lrow, lhalf)];
#pragma unroll
  for (int j = 0; j < TN; j++) bf[0][j] = *(const V*)&Bs[0][swz(wn * WN + j * 32 + lrow, lhalf)];
  constexpr int NF = TM + TN, NM = TM * TN, NS = BK / 16;
  for (int kt = 0; kt < KT; kt++) {
    const int cur = kt & 1;
    // Tile kt + 1 goes into the other buffer, whose last reads (tile kt - 1)
    // every wave finished before the previous iteration's barrier. The tile
    // after the last reads zeros (every offset is past K): the loop body
    // stays one block for the scheduler.
    issue_tile(kt + 1, cur ^ 1);
#pragma unroll
    for (int s = 0; s < NS; s++) {
      const int p = s & 1;
      if (s + 1 < NS) {
        const int c = 2 * (s + 1) + lhalf;
#pragma unroll
        for (int i = 0; i < TM; i++) af[p ^ 1][i] = *(const V*)&As[cur][swz(wm * WM + i * 32 + lrow, c)];
#pragma unroll
        for (int j = 0; j < TN; j++) bf[p ^ 1][j] = *(const V*)&Bs[cur][swz(wn * WN + j * 32 + lrow, c)];
      } else {
        // Before the last step's MFMAs: wait for this wave's part of tile
        // kt + 1, meet the other waves (the whole tile has landed, and
        // every read of tile kt is done), then read the next tile's first
        // fragments under the last step's MFMAs. Waiting this late gives
        // the DMA three of the four steps to land, and the next iteration
        // starts with its fragments in registers.
        __builtin_amdgcn_sched_barrier(0);
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_s_barrier();
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < TM; i++) af[p ^ 1][i] = *(const V*)&As[cur ^ 1][swz(wm * WM + i * 32 + lrow, lhalf)];
#pragma unroll
        for (int j = 0; j < TN; j++) bf[p ^ 1][j] = *(const V*)&Bs[cur ^ 1][swz(wn * WN + j * 32 + lrow, lhalf)];
      }
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = MfmaOp<T>::mma(af[p][i], bf[p][j], acc[i][j]);
      // Schedule: the tile DMA first, then each step's MFMAs with the next
      // fragments' LDS reads threaded between them. With eight or more
      // MFMAs a step, the reads go out in two early groups (after the
      // second and the sixth MFMA), so each has most of the step to land
      // before the next step's first MFMAs need it (qkv 1118 -> 1335
      // TFLOP/s at 5376 x 9216 x 3072).
      if (s == 0) __builtin_amdgcn_sched_group_barrier(0x0010, A_LOADS + B_LOADS, 0);
      if constexpr (NM >= 8) {
        __builtin_amdgcn_sched_group_barrier(0x0008, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x0100, NF / 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x0008, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x0100, NF - NF / 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x0008, NM - 6, 0);
      } else if (NM >= NF) {
#pragma unroll
        for (int f = 0; f < NF; f++) {
          __builtin_amdgcn_sched_group_barrier(0x0008, NM / NF, 0);
          __builtin_amdgcn_sched_group_barrier(0x0100, 1, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x0008, NM - (NM / NF) * NF, 0);
      } else {
        __builtin_amdgcn_sched_group_barrier(0x0100, NF, 0);
        __builtin_amdgcn_sched_group_barrier(0x0008, NM, 0);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  float* stage = reinterpret_cast<float*>(smem) + wave * 32 * (WN + 4);
  if constexpr (FAST) fast_epilogue<TM, TN, WN, T>(a, bidx, acc, stage, m0 + wm * WM, n0 + wn * WN);
  else staged_epilogue<TM, TN, WN, QKN>(a, bidx, acc, stage, m0 + wm * WM, n0 + wn * WN);
}

template <int BM, int BN, int WM, int WN, typename T, bool CONV, bool KFULL, bool QKN = false, bool FAST = false>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_mfma_lds_kernel(GemmArgs a0, GemmArgs a1,
                                                                                    int grid) {
  gemm_lds_body<BM, BN, WM, WN, T, CONV, KFULL, QKN, FAST>(a0, a1, grid);
}

// The 64 x 64 tile capped at 64 registers a lane (eight waves a SIMD), for a
// product on the second stream: beside a 256 x 256 workgroup (two waves a
// SIMD of about 220 registers, 128 KB of LDS) a CU has 64 registers a SIMD
// lane and 32 KB of LDS left, so this tile runs next to it instead of
// waiting for the CU. Whole K tiles and the fast epilogue only.
template <typename T>
__global__ __launch_bounds__(256) __attribute__((amdgpu_num_vgpr(64))) void gemm_slim_kernel(GemmArgs a0, GemmArgs a1, int grid) {
  gemm_lds_body<64, 64, 32, 32, T, false, true, false, true>(a0, a1, grid);
}

// ---- int8 weights, direct to LDS ----------------------------------------------
//
// The weight tile travels as int8 (half the bytes of bf16): DMA'd into an
// LDS staging buffer like the activations, then each thread turns one
// (row, 32-column block) of it — one scale — into bf16 in the swizzled tile
// the MFMA loop reads. q * scale is rounded to the compute type, as
// DmlOps.Dequantize's output is (Graph/ModelBuilder.cs:28-35). Scales are
// per (row, qblock columns): BlockQuantizer's 32 (fp16), or the whole row
// (per output channel, fp32).
//
// The dequantisation is software pipelined: while the MFMAs of tile kt run,
// each thread turns tile kt + 1's int8 into bf16, one 8-column chunk per
// 16-deep MFMA step, so the VALU work hides under the matrix cores instead of
// running between barriers with the MFMAs idle. Tile kt + 1's A and tile
// kt + 2's int8 are DMA'd when iteration kt starts and waited for when it
// ends. The six tiles (A, int8 and bf16, two of each) are distinct restrict
// pointers and the loop is unrolled by two, so no LDS read waits for a DMA
// into another tile; at 256 x 256 they fill the 160 KB of LDS.
template <int BM, int BN, int WM, int WN, typename T, bool SF16, bool FAST>
__device__ __forceinline__ void gemm_w8_body(const GemmArgs& a, int grid, T* __restrict__ A0, T* __restrict__ A1,
                                             int8_t* __restrict__ Q0, int8_t* __restrict__ Q1,
                                             T* __restrict__ B0, T* __restrict__ B1, float* stage_all) {
  typedef typename MfmaOp<T>::V V;
  constexpr int WAVES_N = BN / WN;
  constexpr int NW = (BM / WM) * (BN / WN), NT = NW * 64;
  constexpr int TM = WM / 32, TN = WN / 32;
  constexpr int A_LOADS = BM / 8 / NW;    // kilobyte loads of A per wave per tile (8 rows x 128 B)
  constexpr int W_LOADS = BN / 16 / NW;   // kilobyte loads of W per wave per tile (16 rows x 64 B)
  static_assert(A_LOADS * 8 * NW == BM && W_LOADS * 16 * NW == BN, "tile rows do not split over the waves");

  int tm, tn;
  if (!tile_of(blockIdx.x, grid, (a.M + BM - 1) / BM, (a.N + BN - 1) / BN, tm, tn)) return;
  const int64_t bidx = blockIdx.y;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WAVES_N, wn = wave % WAVES_N;
  constexpr int ES = (int)sizeof(T);

  const T* A = (const T*)a.a + bidx * a.batch_a;
  const __amdgpu_buffer_rsrc_t ra = make_rsrc(A, (uint32_t)((int64_t(a.M - 1) * a.lda + a.K) * ES));
  const __amdgpu_buffer_rsrc_t rw = make_rsrc(a.w, (uint32_t)(int64_t(a.N - 1) * a.ldw + a.K));

  // A: as the 16-bit kernel (8 rows x 8 swizzled 16-byte chunks per load,
  // the chunk depending on the 8-row group's parity).
  const int lrow8 = lane >> 3;
  const int kchunk_q[2] = {(lane & 7) ^ (lrow8 >> 1), (lane & 7) ^ (4 | (lrow8 >> 1))};
  uint32_t a_row[A_LOADS], w_row[W_LOADS];
#pragma unroll
  for (int i = 0; i < A_LOADS; i++) {
    const int r = (wave * A_LOADS + i) * 8 + lrow8;
    a_row[i] = m0 + r < a.M ? (uint32_t)(int64_t(m0 + r) * a.lda * ES) : kOutOfRange;
  }
  // W: 16 rows x 4 chunks of 16 int8 per load, row-major in LDS.
  const int wrow16 = lane >> 2, wchunk = lane & 3;
#pragma unroll
  for (int i = 0; i < W_LOADS; i++) {
    const int r = (wave * W_LOADS + i) * 16 + wrow16;
    w_row[i] = n0 + r < a.N ? (uint32_t)(int64_t(n0 + r) * a.ldw) : kOutOfRange;
  }

  auto issue_a = [&](int kt, T* buf) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < A_LOADS; i++) {
      const int k = kt * BK + kchunk_q[(wave * A_LOADS + i) & 1] * 8;
      const uint32_t off = (k < a.K && a_row[i] != kOutOfRange) ? a_row[i] + uint32_t(k * ES) : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)&buf[(wave * A_LOADS + i) * 8 * BK], 16, off, 0, 0, 0);
    }
  };
  auto issue_q = [&](int kt, int8_t* buf) __attribute__((always_inline)) {
    const int kw = kt * BK + wchunk * 16;
    const bool kwin = kw < a.K;
#pragma unroll
    for (int i = 0; i < W_LOADS; i++) {
      const uint32_t off = (kwin && w_row[i] != kOutOfRange) ? w_row[i] + uint32_t(kw) : kOutOfRange;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (lds_ptr_t)&buf[(wave * W_LOADS + i) * 16 * BK], 16, off, 0, 0, 0);
    }
  };

  // Dequant tasks: (row r, columns [32 h, 32 h + 32)) for task 2 r + h, one
  // scale each (qblock is a multiple of 32). A scale's raw bits (fp16 or
  // fp32 by SF16) are loaded an iteration ahead and converted only when used.
  constexpr int TPT = (2 * BN + NT - 1) / NT;  // tasks per thread
  auto load_scales = [&](int kt, uint32_t (&raw)[TPT]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < TPT; t++) {
      const int task = tid + t * NT, dr = task >> 1, k0 = kt * BK + (task & 1) * 32;
      const int64_t i = int64_t(n0 + dr) * a.lds + k0 / a.qblock;
      const bool in = task < 2 * BN && n0 + dr < a.N && k0 < a.K;
      if (SF16) raw[t] = in ? (uint32_t)((const uint16_t*)a.scales)[i] : 0u;
      else raw[t] = in ? ((const uint32_t*)a.scales)[i] : 0u;
    }
  };
  auto to_float = [&](const uint32_t (&raw)[TPT], float (&sc)[TPT]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < TPT; t++)
      sc[t] = SF16 ? (float)__builtin_bit_cast(_Float16, (uint16_t)raw[t]) : __uint_as_float(raw[t]);
  };
  // The 32 int8 of every task of this thread. (Read before the iteration's
  // DMA is issued: an LDS access after it would wait for the DMA.)
  auto read_q = [&](const int8_t* q, uint4 (&qv)[TPT][2]) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < TPT; t++) {
      const int task = tid + t * NT;
      if (NT * TPT != 2 * BN && task >= 2 * BN) break;
      const int dr = task >> 1, dh = task & 1;
      qv[t][0] = *(const uint4*)&q[dr * BK + dh * 32];
      qv[t][1] = *(const uint4*)&q[dr * BK + dh * 32 + 16];
    }
  };
  // Chunk c (columns 8 c .. 8 c + 7 of the task's 32) of every task of this
  // thread, from the registers read_q filled, into the swizzled bf16 tile.
  auto dequant_chunk = [&](T* b, const float (&sc)[TPT], const uint4 (&qv)[TPT][2], int c) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < TPT; t++) {
      const int task = tid + t * NT;
      if (NT * TPT != 2 * BN && task >= 2 * BN) break;
      const int dr = task >> 1, dh = task & 1;
      const uint4 x = qv[t][c >> 1];
      const uint32_t w[2] = {(c & 1) ? x.z : x.x, (c & 1) ? x.w : x.y};
      T h[8];
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const int v = (int)(int8_t)((w[e / 4] >> (8 * (e & 3))) & 0xff);
        h[e] = (T)((float)v * sc[t]);
      }
      *(uint4*)&b[swz(dr, dh * 4 + c)] = *(const uint4*)h;
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int lrow = lane & 31, lhalf = lane >> 5;
  const int KT = (a.K + BK - 1) / BK;
  uint32_t sc_raw[TPT];
  {
    // A of tile 0, the int8 of tiles 0 and 1 and their scales; tile 0
    // dequantised.
    uint32_t raw0[TPT];
    load_scales(0, raw0);
    issue_a(0, A0);
    issue_q(0, Q0);
    issue_q(1, Q1);
    load_scales(1, sc_raw);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    float sc0[TPT];
    to_float(raw0, sc0);
    uint4 qv[TPT][2];
    read_q(Q0, qv);
#pragma unroll
    for (int c = 0; c < 4; c++) dequant_chunk(B0, sc0, qv, c);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  }

  // Iteration kt: the MFMAs of tile kt (Ac, Bc) with tile kt + 1's int8 (Qd)
  // dequantised into Bn under them; tile kt + 1's A goes to An and tile
  // kt + 2's int8 to Qn.
  constexpr int NF = TM + TN, NM = TM * TN, NS = BK / 16;
  auto iter = [&](int kt, const T* Ac, const T* Bc, T* An, const int8_t* Qd, T* Bn, int8_t* Qn) __attribute__((always_inline)) {
    float sc[TPT];
    to_float(sc_raw, sc);
    uint4 qv[TPT][2];
    read_q(Qd, qv);
    issue_a(kt + 1, An);
    issue_q(kt + 2, Qn);
    load_scales(kt + 2, sc_raw);
    V af[2][TM], bf[2][TN];
#pragma unroll
    for (int i = 0; i < TM; i++) af[0][i] = *(const V*)&Ac[swz(wm * WM + i * 32 + lrow, lhalf)];
#pragma unroll
    for (int j = 0; j < TN; j++) bf[0][j] = *(const V*)&Bc[swz(wn * WN + j * 32 + lrow, lhalf)];
#pragma unroll
    for (int s = 0; s < NS; s++) {
      const int p = s & 1;
      if (s + 1 < NS) {
        const int c = 2 * (s + 1) + lhalf;
#pragma unroll
        for (int i = 0; i < TM; i++) af[p ^ 1][i] = *(const V*)&Ac[swz(wm * WM + i * 32 + lrow, c)];
#pragma unroll
        for (int j = 0; j < TN; j++) bf[p ^ 1][j] = *(const V*)&Bc[swz(wn * WN + j * 32 + lrow, c)];
      }
      dequant_chunk(Bn, sc, qv, s);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = MfmaOp<T>::mma(af[p][i], bf[p][j], acc[i][j]);
    }
    // Tile kt + 1 (A and the bf16 just written) and tile kt + 2's int8 are
    // complete for every wave after this.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };
  for (int kt = 0; kt < KT; kt += 2) {
    iter(kt, A0, B0, A1, Q1, B1, Q0);
    if (kt + 1 < KT) iter(kt + 1, A1, B1, A0, Q0, B0, Q1);
  }

  // Each wave's epilogue stage: in an array of its own (stage_all), or, when
  // the tiles can hold every wave's, inside them (the loop is done with
  // them): as many per tile as fit, A tiles first, then bf16, then int8.
  constexpr int SW = 32 * (WN + 4);
  constexpr int CA = BM * BK * (int)sizeof(T) / (SW * 4), CB = BN * BK * (int)sizeof(T) / (SW * 4);
  constexpr int CQ = BN * BK / (SW * 4);
  float* stage;
  if (stage_all) {
    stage = stage_all + wave * SW;
  } else {
    int w = wave;
    float* const bases[6] = {reinterpret_cast<float*>(A0), reinterpret_cast<float*>(A1), reinterpret_cast<float*>(B0),
                             reinterpret_cast<float*>(B1), reinterpret_cast<float*>(Q0), reinterpret_cast<float*>(Q1)};
    const int caps[6] = {CA, CA, CB, CB, CQ, CQ};
    stage = bases[0];
#pragma unroll
    for (int t = 0; t < 6; t++) {
      if (w >= 0 && w < caps[t]) stage = bases[t] + w * SW;
      w -= caps[t];
    }
  }
  if constexpr (FAST) fast_epilogue<TM, TN, WN, T>(a, bidx, acc, stage, m0 + wm * WM, n0 + wn * WN);
  else staged_epilogue<TM, TN, WN>(a, bidx, acc, stage, m0 + wm * WM, n0 + wn * WN);
}

// Every tile is an LDS array of its own: the compiler orders an LDS access
// after a DMA only against the arrays the DMA may write, and tells distinct
// arrays apart (slices of one array it cannot), so no read or write of one
// tile waits for the DMA into another. At 256 x 256 the six tiles fill the
// 160 KB of LDS; the epilogue stages in the tiles wherever they can hold
// every wave's stage.
template <int BM, int BN, int WM, int WN, typename T, bool SF16, bool FAST>
__global__ __launch_bounds__((BM / WM) * (BN / WN) * 64) void gemm_w8_lds_kernel(GemmArgs a, int grid) {
  constexpr int NW = (BM / WM) * (BN / WN);
  constexpr int TILES = 2 * (BM * BK * (int)sizeof(T) + BN * BK + BN * BK * (int)sizeof(T));
  constexpr int SWB = 32 * (WN + 4) * 4;
  constexpr int CAP = 2 * (BM * BK * (int)sizeof(T) / SWB + BN * BK * (int)sizeof(T) / SWB + BN * BK / SWB);
  static_assert(TILES <= 160 * 1024 && (CAP >= NW || TILES + NW * SWB <= 160 * 1024), "tiles exceed the LDS");
  __shared__ __attribute__((aligned(1024))) T a0[BM * BK];
  __shared__ __attribute__((aligned(1024))) T a1[BM * BK];
  __shared__ __attribute__((aligned(1024))) int8_t q0[BN * BK];
  __shared__ __attribute__((aligned(1024))) int8_t q1[BN * BK];
  __shared__ __attribute__((aligned(1024))) T b0[BN * BK];
  __shared__ __attribute__((aligned(1024))) T b1[BN * BK];
  if constexpr (CAP >= NW) {
    gemm_w8_body<BM, BN, WM, WN, T, SF16, FAST>(a, grid, a0, a1, q0, q1, b0, b1, nullptr);
  } else {
    __shared__ __attribute__((aligned(1024))) float st[NW * SWB / 4];
    gemm_w8_body<BM, BN, WM, WN, T, SF16, FAST>(a, grid, a0, a1, q0, q1, b0, b1, st);
  }
}

// ---- fp32 -------------------------------------------------------------------

static constexpr int BK32 = 32;
__device__ __forceinline__ int swz32(int r, int c) { return r * BK32 + ((c ^ (r & 7)) << 2); }

// Eight consecutive weights starting at element (row n, column k) widened
// to fp32 (any float width, or int8 times its block scale).
__device__ __forceinline__ void load_w8(const GemmArgs& a, const char* W, int n, int k, float* out) {
  switch (a.w_dtype) {
    case NDX_F32: {
      const float4* p = (const float4*)(W + (int64_t(n) * a.ldw + k) * 4);
      float4 x = p[0], y = p[1];
      out[0] = x.x; out[1] = x.y; out[2] = x.z; out[3] = x.w;
      out[4] = y.x; out[5] = y.y; out[6] = y.z; out[7] = y.w;
      break;
    }
    case NDX_BF16: {
      uint4 v = *(const uint4*)(W + (int64_t(n) * a.ldw + k) * 2);
      const uint16_t* h = (const uint16_t*)&v;
      for (int e = 0; e < 8; e++) out[e] = bf16_bits_to_f32(h[e]);
      break;
    }
    case NDX_F16: {
      uint4 v = *(const uint4*)(W + (int64_t(n) * a.ldw + k) * 2);
      const _Float16* h = (const _Float16*)&v;
      for (int e = 0; e < 8; e++) out[e] = (float)h[e];
      break;
    }
    default: {  // int8
      uint2 v = *(const uint2*)(W + int64_t(n) * a.ldw + k);
      const int8_t* q = (const int8_t*)&v;
      float s = scale_at(a.scales, a.s_dtype, int64_t(n) * a.lds + k / a.qblock);
      for (int e = 0; e < 8; e++) out[e] = float(q[e]) * s;
      break;
    }
  }
}

// fp32 activations: 128x128 tiles of four 64x64 waves on the fp32 MFMA.
// Within a 16-wide K step, lane half h feeds k = h*8 + t to MFMA number t,
// the same permutation for both operands, so eight MFMAs cover the step
// from one 16-byte-pair LDS read per operand.
template <bool FAST>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmArgs a, int grid) {
  constexpr int BM = 128, BN = 128, WM = 64, WN = 64, TM = 2, TN = 2;
  constexpr int TILE_BYTES = 2 * (BM + BN) * BK32 * 4;
  constexpr int STAGE_BYTES = 4 * 32 * (WN + 4) * 4;
  __shared__ __attribute__((aligned(16))) char smem[TILE_BYTES > STAGE_BYTES ? TILE_BYTES : STAGE_BYTES];
  float (*As)[BM * BK32] = reinterpret_cast<float (*)[BM * BK32]>(smem);
  float (*Bs)[BN * BK32] = reinterpret_cast<float (*)[BN * BK32]>(smem + 2 * BM * BK32 * 4);
  int tm, tn;
  if (!tile_of(blockIdx.x, grid, (a.M + BM - 1) / BM, (a.N + BN - 1) / BN, tm, tn)) return;
  const int64_t bidx = blockIdx.y;
  const int m0 = tm * BM, n0 = tn * BN;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / 2, wn = wave % 2;
  const float* A = (const float*)a.a + bidx * a.batch_a;
  const char* W = (const char*)a.w;

  float4 ra[4];
  float rb[2][8];
  auto load_tile = [&](int kt) {
    const int k0 = kt * BK32;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int id = tid + i * 256;
      int r = id >> 3, c = id & 7;
      int gm = m0 + r, gk = k0 + c * 4;
      if (gm < a.M && gk < a.K)
        ra[i] = *(const float4*)(A + int64_t(gm) * a.lda + gk);
      else
        ra[i] = make_float4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
      int id = tid + i * 256;
      int r = id >> 2, c = id & 3;
      int gn = n0 + r, gk = k0 + c * 8;
      if (gn < a.N && gk < a.K)
        load_w8(a, W, gn, gk, rb[i]);
      else
        for (int e = 0; e < 8; e++) rb[i][e] = 0.f;
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      int id = tid + i * 256;
      int r = id >> 3, c = id & 7;
      *(float4*)&As[buf][swz32(r, c)] = ra[i];
    }
#pragma unroll
    for (int i = 0; i < 2; i++) {
      int id = tid + i * 256;
      int r = id >> 2, c = id & 3;
      *(float4*)&Bs[buf][swz32(r, 2 * c)] = make_float4(rb[i][0], rb[i][1], rb[i][2], rb[i][3]);
      *(float4*)&Bs[buf][swz32(r, 2 * c + 1)] = make_float4(rb[i][4], rb[i][5], rb[i][6], rb[i][7]);
    }
  };

  f32x16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

  const int KT = (a.K + BK32 - 1) / BK32;
  load_tile(0);
  store_tile(0);
  __syncthreads();
  const int lrow = lane & 31, lhalf = lane >> 5;
  for (int kt = 0; kt < KT; kt++) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_tile(kt + 1);
#pragma unroll
    for (int s = 0; s < BK32 / 16; s++) {
      float af[TM][8], bf[TN][8];
      const int c = 4 * s + 2 * lhalf;  // two 4-float chunks: k = s*16 + h*8 + 0..7
#pragma unroll
      for (int i = 0; i < TM; i++) {
        int r = wm * WM + i * 32 + lrow;
        float4 x = *(const float4*)&As[cur][swz32(r, c)];
        float4 y = *(const float4*)&As[cur][swz32(r, c + 1)];
        af[i][0] = x.x; af[i][1] = x.y; af[i][2] = x.z; af[i][3] = x.w;
        af[i][4] = y.x; af[i][5] = y.y; af[i][6] = y.z; af[i][7] = y.w;
      }
#pragma unroll
      for (int j = 0; j < TN; j++) {
        int r = wn * WN + j * 32 + lrow;
        float4 x = *(const float4*)&Bs[cur][swz32(r, c)];
        float4 y = *(const float4*)&Bs[cur][swz32(r, c + 1)];
        bf[j][0] = x.x; bf[j][1] = x.y; bf[j][2] = x.z; bf[j][3] = x.w;
        bf[j][4] = y.x; bf[j][5] = y.y; bf[j][6] = y.z; bf[j][7] = y.w;
      }
#pragma unroll
      for (int t = 0; t < 8; t++)
#pragma unroll
        for (int i = 0; i < TM; i++)
#pragma unroll
          for (int j = 0; j < TN; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][t], bf[j][t], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < KT) store_tile(cur ^ 1);
    __syncthreads();
  }
  float* stage = reinterpret_cast<float*>(smem) + wave * 32 * (WN + 4);
  if constexpr (FAST) fast_epilogue<TM, TN, WN, float>(a, bidx, acc, stage, m0 + wm * WM, n0 + wn * WN);
  else staged_epilogue<TM, TN, WN>(a, bidx, acc, stage, m0 + wm * WM, n0 + wn * WN);
}

// ---- GEMV ---------------------------------------------------------------------

// M <= 4 rows: the rows go to LDS as fp32, each wave produces 4 output
// features, lanes stride K in runs of 8 so every weight load is 16 bytes.
// Eight weights of row n from column k (k a multiple of 8) widened to fp32,
// the weight type fixed at compile time so the loads of several rows and
// K steps can be in flight together.
template <int WT, bool SF16 = true>
__device__ __forceinline__ void load_w8_t(const GemmArgs& a, const char* W, int n, int k, float (&out)[8]) {
  if constexpr (WT == NDX_F32) {
    const float4* p = (const float4*)(W + (int64_t(n) * a.ldw + k) * 4);
    const float4 x = p[0], y = p[1];
    out[0] = x.x; out[1] = x.y; out[2] = x.z; out[3] = x.w;
    out[4] = y.x; out[5] = y.y; out[6] = y.z; out[7] = y.w;
  } else if constexpr (WT == NDX_BF16) {
    const uint4 v = *(const uint4*)(W + (int64_t(n) * a.ldw + k) * 2);
    const uint16_t* h = (const uint16_t*)&v;
#pragma unroll
    for (int e = 0; e < 8; e++) out[e] = bf16_bits_to_f32(h[e]);
  } else if constexpr (WT == NDX_F16) {
    const uint4 v = *(const uint4*)(W + (int64_t(n) * a.ldw + k) * 2);
    const _Float16* h = (const _Float16*)&v;
#pragma unroll
    for (int e = 0; e < 8; e++) out[e] = (float)h[e];
  } else {  // int8, one scale (fp16 or fp32 by SF16) per qblock columns (a multiple of 8)
    const uint2 v = *(const uint2*)(W + int64_t(n) * a.ldw + k);
    const int8_t* q = (const int8_t*)&v;
    const int64_t si = int64_t(n) * a.lds + k / a.qblock;
    const float sc = SF16 ? (float)((const _Float16*)a.scales)[si] : ((const float*)a.scales)[si];
#pragma unroll
    for (int e = 0; e < 8; e++) out[e] = float(q[e]) * sc;
  }
}

// A handful of rows (MR <= 4) times the weight: x goes to LDS once per
// workgroup (fp32), then each wave takes four output features at once, its
// lanes striding K by 8 columns, so every iteration has four 16-byte weight
// loads per lane in flight (two iterations unrolled: eight); the weight
// bytes are the whole cost.
template <int MR, int WT, bool SF16 = true>
__global__ __launch_bounds__(256) void gemv_kernel(GemmArgs a) {
  extern __shared__ float xs[];  // [MR][K]
  const int64_t bidx = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int K = a.K;
  if (a.a_dtype == NDX_F32 && K % 4 == 0 && a.lda % 4 == 0 && a.batch_a % 4 == 0 && (uintptr_t)a.a % 16 == 0) {
#pragma unroll
    for (int m = 0; m < MR; m++) {
      const float* xr = (const float*)a.a + bidx * a.batch_a + int64_t(min(m, a.M - 1)) * a.lda;
      // Four loads out before the first store.
      for (int k0 = 0; k0 < K; k0 += 4096) {
        float4 v[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int k = k0 + j * 1024 + tid * 4;
          v[j] = k < K ? *(const float4*)(xr + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const int k = k0 + j * 1024 + tid * 4;
          if (k < K) *(float4*)&xs[m * K + k] = m < a.M ? v[j] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
  } else {
    for (int i = tid; i < MR * K; i += 256) {
      const int m = i / K, k = i % K;
      xs[i] = m < a.M ? load_f(a.a, a.a_dtype, bidx * a.batch_a + int64_t(m) * a.lda + k) : 0.f;
    }
  }
  __syncthreads();
  const char* W = (const char*)a.w;
  const int nbase = blockIdx.x * 16 + wave * 4;
  int rows[4];
#pragma unroll
  for (int q = 0; q < 4; q++) rows[q] = min(nbase + q, a.N - 1);  // rows past N load row N-1, unused
  float acc[4][MR];
#pragma unroll
  for (int q = 0; q < 4; q++)
#pragma unroll
    for (int m = 0; m < MR; m++) acc[q][m] = 0.f;
#pragma unroll 2
  for (int k = lane * 8; k < K; k += 512) {
    float w[4][8];
#pragma unroll
    for (int q = 0; q < 4; q++) load_w8_t<WT, SF16>(a, W, rows[q], k, w[q]);
#pragma unroll
    for (int m = 0; m < MR; m++) {
      float xv[8];
      const float4 x0 = *(const float4*)&xs[m * K + k], x1 = *(const float4*)&xs[m * K + k + 4];
      xv[0] = x0.x; xv[1] = x0.y; xv[2] = x0.z; xv[3] = x0.w; xv[4] = x1.x; xv[5] = x1.y; xv[6] = x1.z; xv[7] = x1.w;
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int e = 0; e < 8; e++) acc[q][m] += xv[e] * w[q][e];
    }
  }
#pragma unroll
  for (int q = 0; q < 4; q++) {
    const int n = nbase + q;
#pragma unroll
    for (int m = 0; m < MR; m++) {
      const float v = wave_sum(acc[q][m]);
      if (lane == 0 && m < a.M && n < a.N) {
        const float bias = a.bias ? load_f(a.bias, a.bias_dtype, n) : 0.f;
        const float gate = a.gate ? load_f(a.gate, a.gate_dtype, gate_off(a, bidx, m) + n) : 0.f;
        epilogue_one(a, bidx, m, n, v, bias, gate);
      }
    }
  }
}

// ---- generic (DmlOps.Gemm, any layout) ----------------------------------------

__global__ void gemm_generic_kernel(GemmGenericArgs g) {
  const int64_t total = g.batch0 * g.batch1 * g.M * g.N;
  for (int64_t id = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; id < total;
       id += int64_t(gridDim.x) * blockDim.x) {
    int64_t n = id % g.N, r = id / g.N;
    int64_t m = r % g.M;
    r /= g.M;
    int64_t b1 = r % g.batch1, b0 = r / g.batch1;
    const int64_t ao = b0 * g.va.stride[0] + b1 * g.va.stride[1];
    const int64_t bo = b0 * g.vb.stride[0] + b1 * g.vb.stride[1];
    float acc = 0.f;
    for (int64_t k = 0; k < g.K; k++) {
      int64_t ai = g.trans_a ? k * g.va.stride[2] + m * g.va.stride[3] : m * g.va.stride[2] + k * g.va.stride[3];
      int64_t bi = g.trans_b ? n * g.vb.stride[2] + k * g.vb.stride[3] : k * g.vb.stride[2] + n * g.vb.stride[3];
      acc += load_f(g.a, g.a_dtype, ao + ai) * load_f(g.b, g.b_dtype, bo + bi);
    }
    float v = g.alpha * acc;
    if (g.c) {
      int64_t ci = b0 * g.vc.stride[0] + b1 * g.vc.stride[1] + m * g.vc.stride[2] + n * g.vc.stride[3];
      v += g.beta * load_f(g.c, g.c_dtype, ci);
    }
    store_f(g.out, g.out_dtype, id, v);
  }
}

void launch_gemm_generic(const GemmGenericArgs& g, hipStream_t s) {
  int64_t total = g.batch0 * g.batch1 * g.M * g.N;
  int blocks = (int)std::min<int64_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(gemm_generic_kernel, dim3(std::max(blocks, 1)), dim3(256), 0, s, g);
}

// ---- dispatch -----------------------------------------------------------------

enum GemmKind {
  K_GEMV, K_MFMA_256, K_MFMA_128, K_MFMA_64, K_MFMA_64x64, K_LDS_256, K_LDS_128, K_LDS_64x128, K_LDS_64x64,
  K_LDS_256W8, K_LDS_128W8, K_W8_256W8, K_W8_128, K_W8_64x128, K_W8_64x64, K_F32, K_GENERIC_LINEAR, K_LDS_SLIM
};

// Whether every 16-byte (or 8-byte, int8 GEMV) vector load a kernel makes
// of the weight / the activation rows is aligned.
static bool w_aligned(const GemmArgs& a) {
  const int es = a.w_dtype == NDX_I8 ? 1 : dtype_size(a.w_dtype);
  const int need = a.w_dtype == NDX_I8 ? 8 : 16;
  return (uintptr_t)a.w % need == 0 && (a.ldw * es) % need == 0;
}
static bool a_aligned(const GemmArgs& a) {
  const int es = dtype_size(a.a_dtype);
  return (uintptr_t)a.a % 16 == 0 && (a.lda * es) % 16 == 0 && (a.batch_a * es) % 16 == 0;
}

// The buffer loads address one batch of A and the whole weight with 32-bit
// byte offsets.
static bool spans_fit(const GemmArgs& a) {
  const int64_t lim = int64_t(1) << 31;
  const int64_t a_span = (int64_t(a.M - 1) * a.lda + a.K) * dtype_size(a.a_dtype);
  const int64_t w_span = (int64_t(a.N - 1) * a.ldw + a.K) * (a.w_dtype == NDX_I8 ? 1 : dtype_size(a.w_dtype));
  return a_span < lim && w_span < lim;
}

// The tile for an M x N x K product (batch of them): the one with the least
// modelled time, rounds * (work per tile) / (rate per workgroup), where a
// round is one workgroup on every slot (256 CUs x the workgroups one CU
// holds) and a tile's work is BM * BN * (K + K0), K0 its fixed cost in
// K-equivalents. Rates and K0 are fitted to a sweep of every tile over the
// DiTs' and the UNet's GEMM shapes on MI355X (34 shapes: rows 154 to 13778,
// N 640 to 12288, K 640 to 12288): the pick is the best tile on all but one,
// 0.3% off there. Index 0..3: 256x256 (8 waves), 128x128, 64x128, 64x64.
static int pick_tile(int64_t M, int64_t N, int64_t K, int64_t batch, double* model_time = nullptr) {
  struct Tile { int bm, bn, per_cu; double rate; double k0; };
  static const Tile tiles[4] = {
      {256, 256, 1, 1000.0, 256.0}, {128, 128, 2, 850.0, 128.0}, {64, 128, 3, 700.0, 128.0}, {64, 64, 4, 560.0, 128.0}};
  int best = 0;
  double best_t = 0;
  for (int i = 0; i < 4; i++) {
    const Tile& t = tiles[i];
    const int64_t count = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * batch;
    const int64_t slots = 256 * t.per_cu;
    const int64_t rounds = (count + slots - 1) / slots;
    const double time = double(rounds) * t.bm * t.bn * (double(K) + t.k0) * slots / t.rate;
    if (i == 0 || time < best_t) {
      best = i;
      best_t = time;
    }
  }
  // In microseconds: 2 flops per multiply-add over rates in TFLOP/s.
  if (model_time) *model_time = best_t * 2.0 * 1e-6;
  return best;
}

static GemmKind choose(const GemmArgs& a) {
  const int MR = a.M;
  if (!w_aligned(a)) return K_GENERIC_LINEAR;
  if (MR <= 4 && int64_t(4) * a.K * 4 <= 65536 && a.K % 8 == 0 && a.epilogue != EPI_SWIGLU) return K_GEMV;
  if (!a_aligned(a) || !spans_fit(a)) return K_GENERIC_LINEAR;
  if (a.w_dtype == NDX_I8 && ((uintptr_t)a.w % 16 || a.ldw % 16)) return K_GENERIC_LINEAR;
  if ((a.a_dtype == NDX_BF16 || a.a_dtype == NDX_F16) && a.K % 16 == 0) {
    // NDX_GEMM_TILE pins the tile (for sweeps and the tests that cover every
    // variant): 256, 128, 64x128, 64x64 select the register-staged kernels,
    // the same names with an "lds" suffix the direct-to-LDS ones (16-bit
    // weights only); read per launch.
    const char* pin = getenv("NDX_GEMM_TILE");
    if (pin) {
      if (!strcmp(pin, "256")) return K_MFMA_256;
      if (!strcmp(pin, "128")) return K_MFMA_128;
      if (!strcmp(pin, "64x128")) return K_MFMA_64;
      if (!strcmp(pin, "64x64")) return K_MFMA_64x64;
      if (!strcmp(pin, "256lds") && a.w_dtype != NDX_I8) return K_LDS_256;
      if (!strcmp(pin, "128lds") && a.w_dtype != NDX_I8) return K_LDS_128;
      if (!strcmp(pin, "64x128lds") && a.w_dtype != NDX_I8) return K_LDS_64x128;
      if (!strcmp(pin, "64x64lds") && a.w_dtype != NDX_I8) return K_LDS_64x64;
      if (!strcmp(pin, "256w8lds") && a.w_dtype != NDX_I8) return K_LDS_256W8;
      if (!strcmp(pin, "128w8lds") && a.w_dtype != NDX_I8) return K_LDS_128W8;
      if (!strcmp(pin, "slim") && a.w_dtype != NDX_I8)
        return a.K % BK == 0 && epi_fast_ok(a, 64) ? K_LDS_SLIM : K_LDS_64x64;
      if (a.w_dtype == NDX_I8 && a.qblock % 32 == 0) {
        if (!strcmp(pin, "256w8lds") || !strcmp(pin, "256lds")) return K_W8_256W8;
        if (!strcmp(pin, "128lds")) return K_W8_128;
        if (!strcmp(pin, "64x128lds")) return K_W8_64x128;
        if (!strcmp(pin, "64x64lds")) return K_W8_64x64;
      }
    }
    // Hint 5: the register-capped 64 x 64 tile for the second stream, where
    // its conditions hold (16-bit weights, whole K tiles, the fast epilogue).
    if (a.tile_hint == 5 && a.w_dtype != NDX_I8) {
      if (a.K % BK == 0 && epi_fast_ok(a, 64)) return K_LDS_SLIM;
      return K_LDS_64x64;
    }
    static const GemmKind lds[4] = {K_LDS_256W8, K_LDS_128, K_LDS_64x128, K_LDS_64x64};
    static const GemmKind w8[4] = {K_W8_256W8, K_W8_128, K_W8_64x128, K_W8_64x64};
    static const GemmKind reg[4] = {K_MFMA_256, K_MFMA_128, K_MFMA_64, K_MFMA_64x64};
    const int t = a.tile_hint >= 1 && a.tile_hint <= 4 ? a.tile_hint - 1 : pick_tile(a.M, a.N, a.K, a.batch);
    if (a.w_dtype != NDX_I8) return lds[t];
    // The direct-to-LDS int8 kernel takes one scale per 32 columns.
    return a.qblock % 32 == 0 ? w8[t] : reg[t];
  }
  if (a.a_dtype == NDX_F32 && a.K % 8 == 0) return K_F32;
  return K_GENERIC_LINEAR;
}

const char* gemm_family(const GemmArgs& a) {
  const bool i8 = a.w_dtype == NDX_I8;
  switch (choose(a)) {
    case K_GEMV: return "gemv";
    case K_MFMA_256: return i8 ? "gemm_w8_mfma_256x256" : "gemm_mfma_256x256";
    case K_MFMA_128: return i8 ? "gemm_w8_mfma_128x128" : "gemm_mfma_128x128";
    case K_MFMA_64: return i8 ? "gemm_w8_mfma_64x128" : "gemm_mfma_64x128";
    case K_MFMA_64x64: return i8 ? "gemm_w8_mfma_64x64" : "gemm_mfma_64x64";
    case K_LDS_256: return "gemm_mfma_lds_256x256";
    case K_LDS_128: return "gemm_mfma_lds_128x128";
    case K_LDS_64x128: return "gemm_mfma_lds_64x128";
    case K_LDS_64x64: return "gemm_mfma_lds_64x64";
    case K_LDS_SLIM: return "gemm_mfma_lds_64x64_slim";
    case K_LDS_256W8: return "gemm_mfma_lds_256x256w8";
    case K_LDS_128W8: return "gemm_mfma_lds_128x128w8";
    case K_W8_256W8: return "gemm_w8_lds_256x256w8";
    case K_W8_128: return "gemm_w8_lds_128x128";
    case K_W8_64x128: return "gemm_w8_lds_64x128";
    case K_W8_64x64: return "gemm_w8_lds_64x64";
    case K_F32: return "gemm_f32_mfma_128x128";
    default: return "gemm_linear_generic";
  }
}

// The interleaved SwiGLU in the generic kernel: output j of row m from
// the gate (row 2j of W) and up (row 2j + 1) dot products.
__device__ __forceinline__ float generic_dot(const GemmArgs& a, int64_t b, int m, int n) {
  float acc = 0.f;
  for (int k = 0; k < a.K; k++) {
    float w = a.w_dtype == NDX_I8
                  ? float(((const int8_t*)a.w)[int64_t(n) * a.ldw + k]) *
                        scale_at(a.scales, a.s_dtype, int64_t(n) * a.lds + k / a.qblock)
                  : load_f(a.w, a.w_dtype, int64_t(n) * a.ldw + k);
    acc += load_f(a.a, a.a_dtype, b * a.batch_a + int64_t(m) * a.lda + k) * w;
  }
  return acc + (a.bias ? load_f(a.bias, a.bias_dtype, n) : 0.f);
}

__global__ void linear_generic_kernel(GemmArgs a) {
  if (a.epilogue == EPI_SWIGLU) {
    const int NO = a.N / 2;
    const int64_t total = int64_t(a.batch) * a.M * NO;
    for (int64_t id = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; id < total;
         id += int64_t(gridDim.x) * blockDim.x) {
      const int j = (int)(id % NO);
      const int64_t r = id / NO;
      const int m = (int)(r % a.M);
      const int64_t b = r / a.M;
      const float g = round_to(generic_dot(a, b, m, 2 * j), a.a_dtype);
      const float u = round_to(generic_dot(a, b, m, 2 * j + 1), a.a_dtype);
      store_f(a.c, a.c_dtype, b * a.batch_c + int64_t(m) * a.ldc + j, round_to(silu_f(g), a.a_dtype) * u);
    }
    return;
  }
  const int64_t total = int64_t(a.batch) * a.M * a.N;
  for (int64_t id = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; id < total;
       id += int64_t(gridDim.x) * blockDim.x) {
    int n = (int)(id % a.N);
    int64_t r = id / a.N;
    int m = (int)(r % a.M);
    int64_t b = r / a.M;
    float acc = 0.f;
    for (int k = 0; k < a.K; k++) {
      float w = a.w_dtype == NDX_I8
                    ? float(((const int8_t*)a.w)[int64_t(n) * a.ldw + k]) *
                          scale_at(a.scales, a.s_dtype, int64_t(n) * a.lds + k / a.qblock)
                    : load_f(a.w, a.w_dtype, int64_t(n) * a.ldw + k);
      acc += load_f(a.a, a.a_dtype, b * a.batch_a + int64_t(m) * a.lda + k) * w;
    }
    const float bias = a.bias ? load_f(a.bias, a.bias_dtype, n) : 0.f;
    const float gate = a.gate ? load_f(a.gate, a.gate_dtype, gate_off(a, b, m) + n) : 0.f;
    epilogue_one(a, b, m, n, acc, bias, gate);
  }
}

template <int BM, int BN, int WM, int WN>
static void launch_mfma(const GemmArgs& a, hipStream_t s) {
  int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  int grid = (tiles + 7) / 8 * 8;
  dim3 g(grid, a.batch), b((BM / WM) * (BN / WN) * 64);
  const bool i8 = a.w_dtype == NDX_I8;
  if (a.a_dtype == NDX_BF16) {
    if (i8) hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, WM, WN, __bf16, true>), g, b, 0, s, a, grid);
    else hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, WM, WN, __bf16, false>), g, b, 0, s, a, grid);
  } else {
    if (i8) hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, WM, WN, _Float16, true>), g, b, 0, s, a, grid);
    else hipLaunchKernelGGL((gemm_mfma_kernel<BM, BN, WM, WN, _Float16, false>), g, b, 0, s, a, grid);
  }
}

template <int BM, int BN, int WM, int WN, bool CONV = false>
static void launch_mfma_lds(const GemmArgs& a, hipStream_t s, const GemmArgs* second = nullptr) {
  GemmArgs a1{};
  if (second) a1 = *second;
  int tiles = ((a.M + BM - 1) / BM + (a1.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  int grid = (tiles + 7) / 8 * 8;
  dim3 g(grid, a.batch), b((BM / WM) * (BN / WN) * 64);
  const bool fast = epi_fast_ok(a, BN) && epi_fast_ok(a1, BN);
  // A convolution's K (taps x Cin, Cin a multiple of BK) is always whole.
  if constexpr (CONV) {
    if (a.a_dtype == NDX_BF16) {
      if (fast) hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, __bf16, true, true, false, true>), g, b, 0, s, a, a1, grid);
      else hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, __bf16, true, true>), g, b, 0, s, a, a1, grid);
    } else {
      if (fast) hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, _Float16, true, true, false, true>), g, b, 0, s, a, a1, grid);
      else hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, _Float16, true, true>), g, b, 0, s, a, a1, grid);
    }
  } else {
    const bool kfull = a.K % BK == 0;
    if constexpr (WN == 128 && BM == 256) {
      // The fused head norm on whole heads per wave (the fast epilogue).
      if (a.epilogue == EPI_QK_NORM_ROPE) {
        if (a.a_dtype == NDX_BF16)
          hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, __bf16, false, true, true, true>), g, b, 0, s, a, a1,
                             grid);
        else
          hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, _Float16, false, true, true, true>), g, b, 0, s, a,
                             a1, grid);
        return;
      }
    }
    if constexpr (WN == 64) {
      // The fused head norm (whole K tiles only, one problem per launch).
      if (a.epilogue == EPI_QK_NORM_ROPE) {
        if (a.a_dtype == NDX_BF16)
          hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, __bf16, false, true, true>), g, b, 0, s, a, a1, grid);
        else
          hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, _Float16, false, true, true>), g, b, 0, s, a, a1,
                             grid);
        return;
      }
    }
    if (a.a_dtype == NDX_BF16) {
      if (kfull && fast) hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, __bf16, false, true, false, true>), g, b, 0, s, a, a1, grid);
      else if (kfull) hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, __bf16, false, true>), g, b, 0, s, a, a1, grid);
      else hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, __bf16, false, false>), g, b, 0, s, a, a1, grid);
    } else {
      if (kfull && fast) hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, _Float16, false, true, false, true>), g, b, 0, s, a, a1, grid);
      else if (kfull) hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, _Float16, false, true>), g, b, 0, s, a, a1, grid);
      else hipLaunchKernelGGL((gemm_mfma_lds_kernel<BM, BN, WM, WN, _Float16, false, false>), g, b, 0, s, a, a1, grid);
    }
  }
}

// ---- implicit-GEMM convolution ----------------------------------------------
//
// y[b, co, p] = sum_k F[co, k] * X_b[p, k] with F the filter reordered to
// [Cout, kh, kw, Cin] and X_b the implicit im2col of the NHWC input: the
// output lands in NCHW directly (rows are channels, columns pixels).

int64_t conv_gemm_cin(int x_dtype, int w_dtype, int64_t cin) {
  if (!((x_dtype == NDX_BF16 || x_dtype == NDX_F16) && w_dtype == x_dtype)) return 0;
  return cin % 8 == 0 ? cin : 0;
}

int64_t conv_filter_row(int64_t cin_k, int64_t taps) {
  return cin_k % BK == 0 ? taps * cin_k : (taps * cin_k + BK - 1) / BK * BK;
}

enum ConvKind { CK_256, CK_128, CK_64x128, CK_64x64 };

static ConvKind conv_choose(const GemmArgs& g) {
  // NDX_CONV_TILE=256|128|64x128|64x64 pins the tile (for sweeps and the
  // tests that cover every variant); read per launch.
  if (const char* pin = getenv("NDX_CONV_TILE")) {
    if (!strcmp(pin, "256")) return CK_256;
    if (!strcmp(pin, "128")) return CK_128;
    if (!strcmp(pin, "64x128")) return CK_64x128;
    if (!strcmp(pin, "64x64")) return CK_64x64;
  }
  static const ConvKind kinds[4] = {CK_256, CK_128, CK_64x128, CK_64x64};
  return kinds[pick_tile(g.M, g.N, g.K, g.batch)];
}

static GemmArgs conv_gemm_args(const ConvArgs& c) {
  GemmArgs g{};
  const int taps = c.kh * c.kw;
  const int64_t row = conv_filter_row(c.cin_k, taps);
  g.a = c.w; g.lda = row; g.batch_a = 0; g.a_dtype = c.x_dtype;
  g.w = c.x; g.ldw = 0; g.batch_w = int64_t(c.H >> c.up) * (c.W >> c.up) * c.Cin; g.w_dtype = c.x_dtype;
  g.c = c.y; g.ldc = int64_t(c.Ho) * c.Wo; g.batch_c = int64_t(c.Cout) * c.Ho * c.Wo; g.c_dtype = c.y_dtype;
  g.row_bias = c.bias; g.row_bias_dtype = c.bias_dtype;
  if (c.resid) {
    g.resid = c.resid; g.ldr = g.ldc; g.batch_r = g.batch_c; g.r_dtype = c.y_dtype;
    g.epilogue = EPI_RESIDUAL;
  }
  g.M = c.Cout; g.N = c.Ho * c.Wo; g.K = (int)row; g.batch = c.N;
  g.conv_cin = c.cin_k; g.conv_c = c.Cin; g.conv_h = c.H; g.conv_w = c.W; g.conv_wo = c.Wo; g.conv_kw = c.kw;
  g.conv_stride = c.stride; g.conv_pad = c.pad; g.conv_up = c.up;
  g.conv_kcont = c.cin_k % BK != 0; g.conv_kh = c.kh;
  return g;
}

const char* conv_family(const ConvArgs& c) {
  switch (conv_choose(conv_gemm_args(c))) {
    case CK_256: return "conv_mfma_256x256w8";
    case CK_128: return "conv_mfma_128x128";
    case CK_64x128: return "conv_mfma_64x128";
    default: return "conv_mfma_64x64";
  }
}

void launch_conv_gemm(const ConvArgs& c, hipStream_t s) {
  if (c.cin_k < c.Cin || c.Cin % 8 || (c.cin_k % BK && c.cin_k != c.Cin) || (c.up && (c.H % 2 || c.W % 2)))
    throw std::runtime_error("conv_gemm: a multiple of 8 input channels, per tap either whole K tiles or unpadded");
  const GemmArgs g = conv_gemm_args(c);
  if (g.M == 0 || g.N == 0 || g.batch == 0) return;
  switch (conv_choose(g)) {
    case CK_256: launch_mfma_lds<256, 256, 64, 128, true>(g, s); break;
    case CK_128: launch_mfma_lds<128, 128, 64, 64, true>(g, s); break;
    case CK_64x128: launch_mfma_lds<64, 128, 32, 64, true>(g, s); break;
    default: launch_mfma_lds<64, 64, 32, 32, true>(g, s); break;
  }
}

template <int BM, int BN, int WM, int WN>
static void launch_w8_lds(const GemmArgs& a, hipStream_t s) {
  int tiles = ((a.M + BM - 1) / BM) * ((a.N + BN - 1) / BN);
  int grid = (tiles + 7) / 8 * 8;
  dim3 g(grid, a.batch), b((BM / WM) * (BN / WN) * 64);
  const bool f16s = a.s_dtype == NDX_F16, fast = epi_fast_ok(a, BN);
#define NDX_W8(TT, SF)                                                                                        \
  do {                                                                                                        \
    if (fast) hipLaunchKernelGGL((gemm_w8_lds_kernel<BM, BN, WM, WN, TT, SF, true>), g, b, 0, s, a, grid);  \
    else hipLaunchKernelGGL((gemm_w8_lds_kernel<BM, BN, WM, WN, TT, SF, false>), g, b, 0, s, a, grid);      \
  } while (0)
  if (a.a_dtype == NDX_BF16) {
    if (f16s) NDX_W8(__bf16, true);
    else NDX_W8(__bf16, false);
  } else {
    if (f16s) NDX_W8(_Float16, true);
    else NDX_W8(_Float16, false);
  }
#undef NDX_W8
}

static bool is_lds_kind(GemmKind k) {
  return k == K_LDS_256 || k == K_LDS_128 || k == K_LDS_64x128 || k == K_LDS_64x64 || k == K_LDS_256W8 ||
         k == K_LDS_128W8;
}

bool gemm_pair_pays(int64_t M1, int64_t M2, int64_t N, int64_t K, int64_t batch) {
  // One launch must beat two by the model (a pair can push the tile count
  // past a round of the machine's slots), counting 5 us fixed per launch.
  double t1, t2, t12;
  pick_tile(M1, N, K, batch, &t1);
  pick_tile(M2, N, K, batch, &t2);
  pick_tile(M1 + M2, N, K, batch, &t12);
  return t12 + 5.0 < t1 + t2 + 10.0;
}

bool launch_gemm_pair(const GemmArgs& a, const GemmArgs& b, hipStream_t s) {
  if (a.epilogue == EPI_QK_NORM_ROPE || b.epilogue == EPI_QK_NORM_ROPE) return false;
  if (a.M == 0 || b.M == 0 || a.N != b.N || a.K != b.K || a.batch != b.batch || a.a_dtype != b.a_dtype ||
      a.w_dtype != b.w_dtype || !is_lds_kind(choose(a)) || !is_lds_kind(choose(b)))
    return false;
  GemmArgs both = a;
  both.M = a.M + b.M;
  switch (choose(both)) {
    case K_LDS_256: launch_mfma_lds<256, 256, 128, 128>(a, s, &b); break;
    case K_LDS_128: launch_mfma_lds<128, 128, 64, 64>(a, s, &b); break;
    case K_LDS_64x128: launch_mfma_lds<64, 128, 32, 64>(a, s, &b); break;
    case K_LDS_64x64: launch_mfma_lds<64, 64, 32, 32>(a, s, &b); break;
    case K_LDS_256W8: launch_mfma_lds<256, 256, 64, 128>(a, s, &b); break;
    case K_LDS_128W8: launch_mfma_lds<128, 128, 64, 32>(a, s, &b); break;
    default: return false;
  }
  return true;
}

const char* gemm_pair_family(const GemmArgs& a, const GemmArgs& b) {
  GemmArgs both = a;
  both.M = a.M + b.M;
  return gemm_family(both);
}

// The 256 x 256 tile runs the fused head norm on 8 waves of 64 x 128 (one
// head per wave, fast_qkn) where the fast epilogue's conditions hold.
static bool qkn_wide_ok(const GemmArgs& a, int qk_cols) {
  GemmArgs q = a;
  q.epilogue = EPI_QK_NORM_ROPE;
  q.qk_cols = qk_cols;
  return q.N % 256 == 0 && qk_cols % 128 == 0 && (!a.c || epi_fast_ok(q, 256, true));
}

bool gemm_qk_norm_fast(const GemmArgs& a, int qk_cols) {
  if (qk_cols <= 0 || qk_cols % 128 || a.K % BK ||
      (a.c_dtype != NDX_BF16 && a.c_dtype != NDX_F16 && a.c_dtype != NDX_F32))
    return false;
  return choose(a) == K_LDS_256W8 && qkn_wide_ok(a, qk_cols);
}

bool gemm_qk_norm_ok(const GemmArgs& a, int qk_cols) {
  if (qk_cols <= 0 || qk_cols % 128 || a.K % BK ||
      (a.c_dtype != NDX_BF16 && a.c_dtype != NDX_F16 && a.c_dtype != NDX_F32))
    return false;
  switch (choose(a)) {
    case K_LDS_256W8: return qk_cols % 256 == 0 || qkn_wide_ok(a, qk_cols);
    case K_LDS_128:
    case K_LDS_64x128: return true;
    default: return false;
  }
}

void launch_gemm(const GemmArgs& a, hipStream_t s) {
  if (a.M == 0 || a.N == 0 || a.batch == 0) return;
  if (a.epilogue == EPI_QK_NORM_ROPE && !gemm_qk_norm_ok(a, a.qk_cols))
    throw std::runtime_error("gemm: the fused head norm needs a 64-column-wave tile dividing the q and k columns");
  switch (choose(a)) {
    case K_GEMV: {
      dim3 g((a.N + 15) / 16, a.batch);
      size_t lds = size_t(4) * a.K * sizeof(float);
#define NDX_GEMV(MR, BYTES)                                                                         \
  do {                                                                                              \
    if (a.w_dtype == NDX_BF16) hipLaunchKernelGGL((gemv_kernel<MR, NDX_BF16>), g, dim3(256), BYTES, s, a); \
    else if (a.w_dtype == NDX_F16) hipLaunchKernelGGL((gemv_kernel<MR, NDX_F16>), g, dim3(256), BYTES, s, a); \
    else if (a.w_dtype == NDX_F32) hipLaunchKernelGGL((gemv_kernel<MR, NDX_F32>), g, dim3(256), BYTES, s, a); \
    else if (a.s_dtype == NDX_F16) hipLaunchKernelGGL((gemv_kernel<MR, NDX_I8, true>), g, dim3(256), BYTES, s, a); \
    else hipLaunchKernelGGL((gemv_kernel<MR, NDX_I8, false>), g, dim3(256), BYTES, s, a);        \
  } while (0)
      if (a.M == 1) NDX_GEMV(1, lds / 4);
      else if (a.M == 2) NDX_GEMV(2, lds / 2);
      else NDX_GEMV(4, lds);
#undef NDX_GEMV
      break;
    }
    case K_MFMA_256: launch_mfma<256, 256, 128, 128>(a, s); break;
    case K_MFMA_128: launch_mfma<128, 128, 64, 64>(a, s); break;
    case K_MFMA_64: launch_mfma<64, 128, 32, 64>(a, s); break;
    case K_MFMA_64x64: launch_mfma<64, 64, 32, 32>(a, s); break;
    case K_LDS_256: launch_mfma_lds<256, 256, 128, 128>(a, s); break;
    case K_LDS_128: launch_mfma_lds<128, 128, 64, 64>(a, s); break;
    case K_LDS_64x128: launch_mfma_lds<64, 128, 32, 64>(a, s); break;
    case K_LDS_64x64: launch_mfma_lds<64, 64, 32, 32>(a, s); break;
    case K_LDS_SLIM: {
      const int tiles = ((a.M + 63) / 64) * ((a.N + 63) / 64), grid = (tiles + 7) / 8 * 8;
      const GemmArgs none{};
      if (a.a_dtype == NDX_BF16)
        hipLaunchKernelGGL(gemm_slim_kernel<__bf16>, dim3(grid, a.batch), dim3(256), 0, s, a, none, grid);
      else
        hipLaunchKernelGGL(gemm_slim_kernel<_Float16>, dim3(grid, a.batch), dim3(256), 0, s, a, none, grid);
      break;
    }
    case K_LDS_256W8:
      if (a.epilogue == EPI_QK_NORM_ROPE && qkn_wide_ok(a, a.qk_cols)) launch_mfma_lds<256, 256, 64, 128>(a, s);
      else launch_mfma_lds<256, 256, 128, 64>(a, s);
      break;
    case K_LDS_128W8: launch_mfma_lds<128, 128, 64, 32>(a, s); break;
    case K_W8_256W8: launch_w8_lds<256, 256, 128, 64>(a, s); break;
    case K_W8_128: launch_w8_lds<128, 128, 64, 64>(a, s); break;
    case K_W8_64x128: launch_w8_lds<64, 128, 64, 32>(a, s); break;
    case K_W8_64x64: launch_w8_lds<64, 64, 32, 32>(a, s); break;
    case K_F32: {
      int tiles = ((a.M + 127) / 128) * ((a.N + 127) / 128);
      int grid = (tiles + 7) / 8 * 8;
      if (epi_fast_ok(a, 128)) hipLaunchKernelGGL(gemm_f32_kernel<true>, dim3(grid, a.batch), dim3(256), 0, s, a, grid);
      else hipLaunchKernelGGL(gemm_f32_kernel<false>, dim3(grid, a.batch), dim3(256), 0, s, a, grid);
      break;
    }
    default: {
      int64_t total = int64_t(a.batch) * a.M * a.N;
      int blocks = (int)std::min<int64_t>((total + 255) / 256, 65536);
      hipLaunchKernelGGL(linear_generic_kernel, dim3(blocks), dim3(256), 0, s, a);
    }
  }
}

}  // namespace ndx
