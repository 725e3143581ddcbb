// Fused attention: softmax(Q_h K_h^T * scale + mask) V_h over packed
// [B, T, H*d] rows, the semantics of DmlOps.MultiheadAttention
// (Dml/DmlOps.cs:480-520; a ruled-out score gets -10000 added, :483).
//
// flash_attn_kernel (bf16 / f16, d = 64 or 128): a workgroup of 4 waves takes
// 128 queries of one (batch, head); each wave owns 32 queries. Scores are
// computed transposed, S^T = K Q^T, on v_mfma_f32_32x32x16: lane l then holds
// column l % 32 of S^T, i.e. one query, so the running max, the rescale of
// the output and the row sum are per-lane registers and one exchange with
// lane l ^ 32. The output is accumulated transposed, O^T += V^T P^T, with P^T
// fed straight from the score registers: the key order inside each 16-key
// MFMA step is permuted identically on both operands, so V^T is read from
// LDS in that order and no score ever leaves registers. K and V^T tiles of 64
// keys are double buffered in LDS (V transposed on its way in), swizzled by
// 16- and 8-byte granules.
//
// flash_attn_f32_kernel (fp32, d = 64 or 128): the same scheme on fp32
// MFMA, described at the kernel.
//
// attn_generic_kernel: any float type and head size, fp32 arithmetic with
// expf; the path for odd shapes.

#include <cstdlib>

#include "k_common.h"

namespace ndx {

template <typename T>
struct AMfma;
template <>
struct AMfma<__bf16> {
  typedef bf16x8 V;
  static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct AMfma<_Float16> {
  typedef f16x8 V;
  static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <typename T>
__device__ __forceinline__ const T* seg_row(const AttnSeg& s, int64_t b, int64_t r) {
  if (r < s.rows0) return (const T*)s.ptr[0] + b * s.batch[0] + r * s.ld[0];
  return (const T*)s.ptr[1] + b * s.batch[1] + (r - s.rows0) * s.ld[1];
}

__device__ __forceinline__ void* out_row(const AttnArgs& a, int64_t b, int64_t r, int esize) {
  if (r < a.out_rows0) return (char*)a.out[0] + (b * a.out_batch[0] + r * a.out_ld[0]) * esize;
  return (char*)a.out[1] + (b * a.out_batch[1] + (r - a.out_rows0) * a.out_ld[1]) * esize;
}

// Decodes a workgroup id into (query block, head, batch), keeping each XCD on
// a contiguous run so the query blocks of one head share that XCD's L2.
__device__ __forceinline__ bool attn_tile(int pid, int grid, int qblocks, int H, int B, int& qb, int& h, int& b) {
  const int per = grid / 8;
  pid = (pid % 8) * per + pid / 8;
  if (pid >= qblocks * H * B) return false;
  qb = pid % qblocks;
  int r = pid / qblocks;
  h = r % H;
  b = r / H;
  return true;
}

constexpr float kLog2e = 1.4426950408889634f;

// QT query tiles of 32 per wave: every K and V fragment read from LDS feeds
// QT MFMAs. QT = 1 keeps the register file under 256 (two waves per SIMD);
// QT = 2 halves the LDS traffic per MFMA at one wave per SIMD.
template <typename T, int D, int MASK, int QT>
__global__ __launch_bounds__(256, QT == 1 ? 2 : 1) void flash_attn_kernel(AttnArgs a, int grid) {
  typedef typename AMfma<T>::V V;
  constexpr int BQ = 128 * QT, BKEY = 64;
  constexpr int KCH = D / 8;                      // 16-byte chunks per key row
  constexpr int KMASK = (KCH < 16 ? KCH : 16) - 1;
  constexpr int K_PER = BKEY * KCH / 256;         // K chunks per thread
  constexpr int V_TASKS = (BKEY / 4) * (D / 8);   // (4-key group, 8-d chunk) tasks
  constexpr int DT = D / 32;                      // output tiles along d
  __shared__ __attribute__((aligned(16))) T Ks[2][BKEY * D];
  __shared__ __attribute__((aligned(16))) T Vt[2][D * BKEY];

  int qb, head, b;
  if (!attn_tile(blockIdx.x, grid, (a.T + BQ - 1) / BQ, a.H, a.B, qb, head, b)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lq = lane & 31, lh = lane >> 5;
  const int64_t col0 = int64_t(head) * D;
  int qi[QT];
#pragma unroll
  for (int t = 0; t < QT; t++) qi[t] = qb * BQ + (wave * QT + t) * 32 + lq;

  // Q^T fragments, resident for the whole key loop.
  V qf[QT][D / 16];
#pragma unroll
  for (int t = 0; t < QT; t++) {
    const T* qrow = seg_row<T>(a.q, b, min(qi[t], a.T - 1)) + col0;
#pragma unroll
    for (int s = 0; s < D / 16; s++) qf[t][s] = *(const V*)(qrow + s * 16 + lh * 8);
  }

  uint4 rk[K_PER];
  uint4 rv[4];
  const int vkg = tid / (D / 8), vdc = tid % (D / 8);
  auto load_kv = [&](int kb) {
    const int key0 = kb * BKEY;
#pragma unroll
    for (int i = 0; i < K_PER; i++) {
      const int id = tid + i * 256;
      const int key = id / KCH, c = id % KCH;
      const int gk = min(key0 + key, a.S - 1);  // tail keys are masked below
      rk[i] = *(const uint4*)(seg_row<T>(a.k, b, gk) + col0 + c * 8);
    }
    if (tid < V_TASKS) {
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int gk = key0 + vkg * 4 + e;
        // Tail rows must be zero: a zero probability times a stale value
        // could still be NaN.
        rv[e] = gk < a.S ? *(const uint4*)(seg_row<T>(a.v, b, gk) + col0 + vdc * 8) : make_uint4(0, 0, 0, 0);
      }
    }
  };
  auto store_kv = [&](int buf) {
#pragma unroll
    for (int i = 0; i < K_PER; i++) {
      const int id = tid + i * 256;
      const int key = id / KCH, c = id % KCH;
      *(uint4*)&Ks[buf][key * D + ((c ^ (key & KMASK)) << 3)] = rk[i];
    }
    if (tid < V_TASKS) {
      const uint32_t* w0 = (const uint32_t*)&rv[0];
      const uint32_t* w1 = (const uint32_t*)&rv[1];
      const uint32_t* w2 = (const uint32_t*)&rv[2];
      const uint32_t* w3 = (const uint32_t*)&rv[3];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        // Two d rows per 32-bit word: (d, d+1) of keys 4g..4g+3.
        const uint32_t lo01 = __builtin_amdgcn_perm(w1[e], w0[e], 0x05040100);
        const uint32_t lo23 = __builtin_amdgcn_perm(w3[e], w2[e], 0x05040100);
        const uint32_t hi01 = __builtin_amdgcn_perm(w1[e], w0[e], 0x07060302);
        const uint32_t hi23 = __builtin_amdgcn_perm(w3[e], w2[e], 0x07060302);
        const int d = vdc * 8 + 2 * e;
        *(uint2*)&Vt[buf][d * BKEY + ((vkg ^ (d & 15)) << 2)] = make_uint2(lo01, lo23);
        *(uint2*)&Vt[buf][(d + 1) * BKEY + ((vkg ^ ((d + 1) & 15)) << 2)] = make_uint2(hi01, hi23);
      }
    }
  };

  f32x16 o[QT][DT];
#pragma unroll
  for (int t = 0; t < QT; t++)
#pragma unroll
    for (int j = 0; j < DT; j++)
#pragma unroll
      for (int r = 0; r < 16; r++) o[t][j][r] = 0.f;
  float m_run[QT], l_part[QT];
#pragma unroll
  for (int t = 0; t < QT; t++) {
    m_run[t] = -INFINITY;
    l_part[t] = 0.f;
  }
  const float sl = a.scale * kLog2e;
  const float mask_add = -10000.0f * kLog2e;
  const int key_len = MASK == NDX_MASK_KEY_LENGTH ? a.mask[0] : a.S;

  const int KB = (a.S + BKEY - 1) / BKEY;
  load_kv(0);
  store_kv(0);
  __syncthreads();
  for (int kb = 0; kb < KB; kb++) {
    const int cur = kb & 1;
    if (kb + 1 < KB) load_kv(kb + 1);

    // S^T for 64 keys: two 32-key tiles per query tile.
    f32x16 sacc[QT][2];
#pragma unroll
    for (int t = 0; t < QT; t++)
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) sacc[t][kt][r] = 0.f;
#pragma unroll
    for (int kt = 0; kt < 2; kt++) {
      const int key = kt * 32 + lq;
#pragma unroll
      for (int s = 0; s < D / 16; s++) {
        const int c = 2 * s + lh;
        const V kf = *(const V*)&Ks[cur][key * D + ((c ^ (key & KMASK)) << 3)];
#pragma unroll
        for (int t = 0; t < QT; t++) sacc[t][kt] = AMfma<T>::mma(kf, qf[t][s], sacc[t][kt]);
      }
    }
    // Scale (into log2 units), mask, running max. The key tail is only
    // checked in the last block.
    const bool tail = (kb + 1) * BKEY > a.S;
#pragma unroll
    for (int t = 0; t < QT; t++) {
      const int qm = min(qi[t], a.T - 1);
      float mloc = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float x = sacc[t][kt][r] * sl;
          const int key = kb * BKEY + kt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
          if (MASK == NDX_MASK_KEY_LENGTH) {
            if (key >= key_len) x += mask_add;
          } else if (MASK == NDX_MASK_BOOLEAN) {
            const int64_t mi = b * a.mask_stride[0] + head * a.mask_stride[1] + int64_t(qm) * a.mask_stride[2] +
                               int64_t(min(key, a.S - 1)) * a.mask_stride[3];
            if (a.mask[mi] == 0) x += mask_add;
          }
          if (tail && key >= a.S) x = -INFINITY;
          sacc[t][kt][r] = x;
          mloc = fmaxf(mloc, x);
        }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
      const float m_new = fmaxf(m_run[t], mloc);
      // Rescale the running output only when some lane's max moved: after
      // the first blocks the maxima settle and the multiply is skipped.
      if (__builtin_amdgcn_ballot_w64(m_new > m_run[t])) {
        const float alpha = exp2f(m_run[t] - m_new);
        l_part[t] *= alpha;
#pragma unroll
        for (int j = 0; j < DT; j++)
#pragma unroll
          for (int r = 0; r < 16; r++) o[t][j][r] *= alpha;
      }
      m_run[t] = m_new;
      float psum = 0.f;
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float p = exp2f(sacc[t][kt][r] - m_new);
          sacc[t][kt][r] = p;
          psum += p;
        }
      l_part[t] += psum;
    }

    // O^T += V^T P^T over four 16-key steps.
#pragma unroll
    for (int u = 0; u < 4; u++) {
      V pb[QT];
#pragma unroll
      for (int t = 0; t < QT; t++)
#pragma unroll
        for (int j = 0; j < 8; j++) pb[t][j] = (T)sacc[t][u >> 1][(u & 1) * 8 + j];
#pragma unroll
      for (int dt = 0; dt < DT; dt++) {
        const int d = dt * 32 + lq;
        const int g1 = 4 * u + lh, g2 = 4 * u + 2 + lh;
        const uint2 x1 = *(const uint2*)&Vt[cur][d * BKEY + ((g1 ^ (d & 15)) << 2)];
        const uint2 x2 = *(const uint2*)&Vt[cur][d * BKEY + ((g2 ^ (d & 15)) << 2)];
        const V vf = __builtin_bit_cast(V, make_uint4(x1.x, x1.y, x2.x, x2.y));
#pragma unroll
        for (int t = 0; t < QT; t++) o[t][dt] = AMfma<T>::mma(vf, pb[t], o[t][dt]);
      }
    }
    if (kb + 1 < KB) store_kv(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int t = 0; t < QT; t++) {
    const float l_tot = l_part[t] + __shfl_xor(l_part[t], 32, 64);
    const float inv = 1.0f / l_tot;
    if (qi[t] < a.T) {
      T* orow = (T*)out_row(a, b, qi[t], sizeof(T)) + col0;
#pragma unroll
      for (int dt = 0; dt < DT; dt++)
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const int d = dt * 32 + 8 * g + 4 * lh;
          T v4[4];
#pragma unroll
          for (int e = 0; e < 4; e++) v4[e] = (T)(o[t][dt][g * 4 + e] * inv);
          *(uint2*)(orow + d) = *(const uint2*)v4;
        }
    }
  }
}

// ---- fp32 ---------------------------------------------------------------------
//
// flash_attn_f32_kernel: the same transposed flash form on
// v_mfma_f32_32x32x2_f32 (two K steps per instruction, one per lane half).
// In the score product lane half h covers head features [h d/2, (h+1) d/2),
// so each lane streams one contiguous half-row of K from LDS; in the output
// product step s of a 32-key tile takes, in lane half h, the key of score
// register s (row 8 (s / 4) + 4 h + s % 4 of S^T), so P^T again comes straight
// from the score registers. K and V tiles of 64 keys sit in LDS row-major,
// rows padded by 16 bytes; the next tile is prefetched into registers while
// the current one is consumed.

template <int D, int MASK>
__global__ __launch_bounds__(256) void flash_attn_f32_kernel(AttnArgs a, int grid) {
  constexpr int BQ = 128, BKEY = 64, LD = D + 4, DH = D / 2, DT = D / 32;
  constexpr int F4 = BKEY * D / 4 / 256;  // float4 loads per thread per tile
  __shared__ __attribute__((aligned(16))) float Ks[BKEY * LD];
  __shared__ __attribute__((aligned(16))) float Vs[BKEY * LD];

  int qb, head, b;
  if (!attn_tile(blockIdx.x, grid, (a.T + BQ - 1) / BQ, a.H, a.B, qb, head, b)) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lq = lane & 31, lh = lane >> 5;
  const int64_t col0 = int64_t(head) * D;
  const int qi = qb * BQ + wave * 32 + lq;
  const int qm = min(qi, a.T - 1);

  float qf[DH];
  {
    const float* qrow = seg_row<float>(a.q, b, qm) + col0 + lh * DH;
#pragma unroll
    for (int t = 0; t < DH; t += 4) *(float4*)&qf[t] = *(const float4*)(qrow + t);
  }

  float4 rk[F4], rv[F4];
  auto load_kv = [&](int kb) {
#pragma unroll
    for (int i = 0; i < F4; i++) {
      const int id = tid + i * 256;
      const int key = id / (D / 4), c4 = id % (D / 4);
      const int gk = kb * BKEY + key;
      rk[i] = *(const float4*)(seg_row<float>(a.k, b, min(gk, a.S - 1)) + col0 + c4 * 4);
      // Tail rows of V are zero: a zero probability times a stale value
      // could still be NaN.
      rv[i] = gk < a.S ? *(const float4*)(seg_row<float>(a.v, b, gk) + col0 + c4 * 4) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  auto store_kv = [&]() {
#pragma unroll
    for (int i = 0; i < F4; i++) {
      const int id = tid + i * 256;
      const int key = id / (D / 4), c4 = id % (D / 4);
      *(float4*)&Ks[key * LD + c4 * 4] = rk[i];
      *(float4*)&Vs[key * LD + c4 * 4] = rv[i];
    }
  };

  f32x16 o[DT];
#pragma unroll
  for (int j = 0; j < DT; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[j][r] = 0.f;
  float m_run = -INFINITY, l_part = 0.f;
  const float sl = a.scale * kLog2e;
  const float mask_add = -10000.0f * kLog2e;
  const int key_len = MASK == NDX_MASK_KEY_LENGTH ? a.mask[0] : a.S;

  const int KB = (a.S + BKEY - 1) / BKEY;
  load_kv(0);
  for (int kb = 0; kb < KB; kb++) {
    __syncthreads();  // the previous tile is consumed
    store_kv();
    __syncthreads();
    if (kb + 1 < KB) load_kv(kb + 1);

    f32x16 sacc[2];
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int r = 0; r < 16; r++) sacc[kt][r] = 0.f;
    const float* k0 = &Ks[lq * LD + lh * DH];
    const float* k1 = &Ks[(32 + lq) * LD + lh * DH];
#pragma unroll
    for (int t = 0; t < DH; t += 4) {
      const float4 a0 = *(const float4*)(k0 + t);
      const float4 a1 = *(const float4*)(k1 + t);
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.x, qf[t], sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.x, qf[t], sacc[1], 0, 0, 0);
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.y, qf[t + 1], sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.y, qf[t + 1], sacc[1], 0, 0, 0);
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.z, qf[t + 2], sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.z, qf[t + 2], sacc[1], 0, 0, 0);
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.w, qf[t + 3], sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.w, qf[t + 3], sacc[1], 0, 0, 0);
    }

    const bool tail = (kb + 1) * BKEY > a.S;
    float mloc = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        float x = sacc[kt][r] * sl;
        const int key = kb * BKEY + kt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
        if (MASK == NDX_MASK_KEY_LENGTH) {
          if (key >= key_len) x += mask_add;
        } else if (MASK == NDX_MASK_BOOLEAN) {
          const int64_t mi = b * a.mask_stride[0] + head * a.mask_stride[1] + int64_t(qm) * a.mask_stride[2] +
                             int64_t(min(key, a.S - 1)) * a.mask_stride[3];
          if (a.mask[mi] == 0) x += mask_add;
        }
        if (tail && key >= a.S) x = -INFINITY;
        sacc[kt][r] = x;
        mloc = fmaxf(mloc, x);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32, 64));
    const float m_new = fmaxf(m_run, mloc);
    if (__builtin_amdgcn_ballot_w64(m_new > m_run)) {
      const float alpha = exp2f(m_run - m_new);
      l_part *= alpha;
#pragma unroll
      for (int j = 0; j < DT; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[j][r] *= alpha;
    }
    m_run = m_new;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int r = 0; r < 16; r++) {
        const float p = exp2f(sacc[kt][r] - m_new);
        sacc[kt][r] = p;
        l_part += p;
      }

#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const int key = kt * 32 + 8 * (s >> 2) + 4 * lh + (s & 3);
        const float* vrow = &Vs[key * LD + lq];
#pragma unroll
        for (int dt = 0; dt < DT; dt++)
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x2f32(vrow[dt * 32], sacc[kt][s], o[dt], 0, 0, 0);
      }
  }

  const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = 1.0f / l_tot;
  if (qi < a.T) {
    float* orow = (float*)out_row(a, b, qi, sizeof(float)) + col0;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int d = dt * 32 + 8 * g + 4 * lh;
        *(float4*)(orow + d) = make_float4(o[dt][g * 4] * inv, o[dt][g * 4 + 1] * inv, o[dt][g * 4 + 2] * inv,
                                           o[dt][g * 4 + 3] * inv);
      }
  }
}

// ---- generic ----------------------------------------------------------------

// 16 queries of one (batch, head) per workgroup, 4 per wave; 64-key tiles
// of K and V in LDS; lane j scores key j, lanes split d for the output.
constexpr int GQ = 16, GK = 64, GDMAX = 128;

__device__ __forceinline__ const char* seg_row_bytes(const AttnSeg& s, int64_t b, int64_t r, int esize) {
  if (r < s.rows0) return (const char*)s.ptr[0] + (b * s.batch[0] + r * s.ld[0]) * esize;
  return (const char*)s.ptr[1] + (b * s.batch[1] + (r - s.rows0) * s.ld[1]) * esize;
}

__global__ __launch_bounds__(256) void attn_generic_kernel(AttnArgs a) {
  extern __shared__ float sm[];
  const int D = a.d, DV = a.dv;
  float* Qs = sm;                  // [GQ][D]
  float* Ks = Qs + GQ * D;         // [GK][D + 1]
  float* Vs = Ks + GK * (D + 1);   // [GK][DV]
  float* Ps = Vs + GK * DV;        // [GQ][GK]
  const int esize = dtype_size(a.dtype);
  const int qb = blockIdx.x, head = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < GQ * D; i += 256) {
    int q = qb * GQ + i / D;
    Qs[i] = q < a.T ? load_f(seg_row_bytes(a.q, b, q, esize), a.dtype, int64_t(head) * D + i % D) : 0.f;
  }
  float m_run[4], l_run[4], acc[4][GDMAX / 64];
  for (int q = 0; q < 4; q++) {
    m_run[q] = -INFINITY;
    l_run[q] = 0.f;
    for (int e = 0; e < GDMAX / 64; e++) acc[q][e] = 0.f;
  }
  int key_len = a.mask_kind == NDX_MASK_KEY_LENGTH ? a.mask[0] : a.S;
  for (int k0 = 0; k0 < a.S; k0 += GK) {
    __syncthreads();
    for (int i = tid; i < GK * D; i += 256) {
      int key = k0 + i / D;
      Ks[(i / D) * (D + 1) + i % D] =
          key < a.S ? load_f(seg_row_bytes(a.k, b, key, esize), a.dtype, int64_t(head) * D + i % D) : 0.f;
    }
    for (int i = tid; i < GK * DV; i += 256) {
      int key = k0 + i / DV;
      Vs[i] = key < a.S ? load_f(seg_row_bytes(a.v, b, key, esize), a.dtype, int64_t(head) * DV + i % DV) : 0.f;
    }
    __syncthreads();
    for (int q = 0; q < 4; q++) {
      const int ql = wave * 4 + q, qi = qb * GQ + ql;
      const int key = k0 + lane;
      float x = -INFINITY;
      if (key < a.S) {
        float dot = 0.f;
        for (int d = 0; d < D; d++) dot += Qs[ql * D + d] * Ks[lane * (D + 1) + d];
        x = dot * a.scale;
        if (a.mask_kind == NDX_MASK_KEY_LENGTH && key >= key_len) x += -10000.0f;
        if (a.mask_kind == NDX_MASK_BOOLEAN && qi < a.T) {
          int64_t mi = b * a.mask_stride[0] + head * a.mask_stride[1] + int64_t(qi) * a.mask_stride[2] +
                       int64_t(key) * a.mask_stride[3];
          if (a.mask[mi] == 0) x += -10000.0f;
        }
      }
      const float m_new = fmaxf(m_run[q], wave_max(x));
      const float alpha = expf(m_run[q] - m_new);
      const float p = key < a.S ? expf(x - m_new) : 0.f;
      l_run[q] = l_run[q] * alpha + wave_sum(p);
      m_run[q] = m_new;
      Ps[ql * GK + lane] = p;
      for (int e = 0; e < GDMAX / 64; e++) acc[q][e] *= alpha;
    }
    __syncthreads();
    for (int q = 0; q < 4; q++) {
      const int ql = wave * 4 + q;
      for (int e = 0; e < GDMAX / 64; e++) {
        int d = lane + e * 64;
        if (d >= DV) break;
        float s = 0.f;
        for (int j = 0; j < GK; j++) s += Ps[ql * GK + j] * Vs[j * DV + d];
        acc[q][e] += s;
      }
    }
  }
  for (int q = 0; q < 4; q++) {
    const int qi = qb * GQ + wave * 4 + q;
    if (qi >= a.T) continue;
    char* orow = (char*)out_row(a, b, qi, esize);
    for (int e = 0; e < GDMAX / 64; e++) {
      int d = lane + e * 64;
      if (d >= DV) break;
      store_f(orow, a.dtype, int64_t(head) * DV + d, acc[q][e] / l_run[q]);
    }
  }
}

static bool rows_aligned(const AttnSeg& s, int esize) {
  for (int p = 0; p < 2; p++) {
    if ((uintptr_t)s.ptr[p] % 16) return false;
    if ((s.ld[p] * esize) % 16 || (s.batch[p] * esize) % 16) return false;
  }
  return true;
}

void launch_attention(const AttnArgs& a, hipStream_t s) {
  if (a.T == 0 || a.B == 0) return;
  const bool mfma = (a.dtype == NDX_BF16 || a.dtype == NDX_F16) && a.d == a.dv && (a.d == 128 || a.d == 64) &&
                    rows_aligned(a.q, 2) && rows_aligned(a.k, 2) && rows_aligned(a.v, 2) &&
                    (uintptr_t)a.out[0] % 16 == 0 && (uintptr_t)a.out[1] % 16 == 0;
  if (mfma) {
    // NDX_ATTN_QT=1|2 pins the query tiles per wave (for sweeps).
    const char* pin = getenv("NDX_ATTN_QT");
    int qt = pin ? atoi(pin) : 1;
    if (qt != 2 || a.d != 128) qt = 1;
    const int qblocks = (a.T + 128 * qt - 1) / (128 * qt);
    const int grid = (qblocks * a.H * a.B + 7) / 8 * 8;
    const bool bf = a.dtype == NDX_BF16;
#define NDX_FA(TYPE, DIM, MK, QT) \
  hipLaunchKernelGGL((flash_attn_kernel<TYPE, DIM, MK, QT>), dim3(grid), dim3(256), 0, s, a, grid)
#define NDX_FA_MASKS(TYPE, DIM, QT)                                      \
  do {                                                                   \
    if (a.mask_kind == NDX_MASK_KEY_LENGTH) NDX_FA(TYPE, DIM, 1, QT);    \
    else if (a.mask_kind == NDX_MASK_BOOLEAN) NDX_FA(TYPE, DIM, 2, QT);  \
    else NDX_FA(TYPE, DIM, 0, QT);                                       \
  } while (0)
    if (bf) {
      if (a.d == 128) {
        if (qt == 2) NDX_FA_MASKS(__bf16, 128, 2);
        else NDX_FA_MASKS(__bf16, 128, 1);
      } else {
        NDX_FA_MASKS(__bf16, 64, 1);
      }
    } else {
      if (a.d == 128) {
        if (qt == 2) NDX_FA_MASKS(_Float16, 128, 2);
        else NDX_FA_MASKS(_Float16, 128, 1);
      } else {
        NDX_FA_MASKS(_Float16, 64, 1);
      }
    }
#undef NDX_FA_MASKS
#undef NDX_FA
    return;
  }
  const bool mfma32 = a.dtype == NDX_F32 && a.d == a.dv && (a.d == 128 || a.d == 64) && rows_aligned(a.q, 4) &&
                      rows_aligned(a.k, 4) && rows_aligned(a.v, 4) && (uintptr_t)a.out[0] % 16 == 0 &&
                      (uintptr_t)a.out[1] % 16 == 0 && (a.out_ld[0] * 4) % 16 == 0 && (a.out_ld[1] * 4) % 16 == 0;
  if (mfma32) {
    const int qblocks = (a.T + 127) / 128;
    const int grid = (qblocks * a.H * a.B + 7) / 8 * 8;
#define NDX_FA32(DIM, MK) hipLaunchKernelGGL((flash_attn_f32_kernel<DIM, MK>), dim3(grid), dim3(256), 0, s, a, grid)
#define NDX_FA32_MASKS(DIM)                                                \
  do {                                                                     \
    if (a.mask_kind == NDX_MASK_KEY_LENGTH) NDX_FA32(DIM, 1);              \
    else if (a.mask_kind == NDX_MASK_BOOLEAN) NDX_FA32(DIM, 2);            \
    else NDX_FA32(DIM, 0);                                                 \
  } while (0)
    if (a.d == 128) NDX_FA32_MASKS(128);
    else NDX_FA32_MASKS(64);
#undef NDX_FA32_MASKS
#undef NDX_FA32
    return;
  }
  size_t lds = (size_t(GQ) * a.d + size_t(GK) * (a.d + 1) + size_t(GK) * a.dv + size_t(GQ) * GK) * sizeof(float);
  static bool raised = false;
  if (!raised) {
    hip_check(hipFuncSetAttribute((const void*)attn_generic_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  160 * 1024),
              "attention LDS limit");
    raised = true;
  }
  dim3 grid((a.T + GQ - 1) / GQ, a.H, a.B);
  hipLaunchKernelGGL(attn_generic_kernel, grid, dim3(256), lds, s, a);
}

}  // namespace ndx
