// Fused attention: softmax(Q_h K_h^T * scale + mask) V_h over packed
// [B, T, H*d] rows, the semantics of DmlOps.MultiheadAttention
// (Dml/DmlOps.cs:480-520; a ruled-out score gets -10000 added, :483).
//
// flash_attn_kernel (bf16 / f16, d = 64 or 128): a tile of 4 waves takes
// 128 queries of one (batch, head); each wave owns 32 queries. Scores are
// computed transposed, S^T = K Q^T, on v_mfma_f32_32x32x16: lane l then holds
// column l % 32 of S^T, i.e. one query, so the running max, the rescale of
// the output and the row sum are per-lane registers and one exchange with
// lane l ^ 32. The output is accumulated transposed, O^T += V^T P^T, with P^T
// fed straight from the score registers: the key order inside each 16-key
// MFMA step is permuted identically on both operands, so no score ever
// leaves registers. K and V tiles of 64 keys arrive by DMA into row-major,
// chunk-swizzled LDS, double buffered; the V^T operand comes out of LDS
// through gfx950's transposing ds_read_b64_tr_b16, in the score order.
//
// flash_attn_f32_kernel (fp32, d = 64 or 128): the same scheme on fp32
// MFMA, described at the kernel.
//
// attn_generic_kernel: any float type and head size, fp32 arithmetic with
// expf; the path for odd shapes.

#include <algorithm>
#include <cstdlib>

#include "k_common.h"

namespace ndx {

template <typename T>
struct AMfma;
// mma: the 32x32x16 MFMA. sum8: acc plus the eight elements of a fragment,
// as four two-element dot products with (1, 1) (v_dot2_f32_bf16 / _f16):
// half the VALU instructions of eight adds.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
template <>
struct AMfma<__bf16> {
  typedef bf16x8 V;
  static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float sum8(V v, float acc) {
    const bf16x2_t one = {(__bf16)1.0f, (__bf16)1.0f};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const bf16x2_t pr = {v[2 * j], v[2 * j + 1]};
      acc = __builtin_amdgcn_fdot2_f32_bf16(pr, one, acc, false);
    }
    return acc;
  }
};
template <>
struct AMfma<_Float16> {
  typedef f16x8 V;
  static __device__ __forceinline__ f32x16 mma(V a, V b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
  static __device__ __forceinline__ float sum8(V v, float acc) {
    const f16x2_t one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const f16x2_t pr = {v[2 * j], v[2 * j + 1]};
      acc = __builtin_amdgcn_fdot2(pr, one, acc, false);
    }
    return acc;
  }
};

// Both segments' addresses are formed from fields read by constant index and
// one of them selected: a per-lane choice of which field to read (an index
// into the argument block) makes the compiler copy the block to scratch.
template <typename T>
__device__ __forceinline__ const T* seg_row(const AttnSeg& s, int64_t b, int64_t r) {
  const T* first = (const T*)s.ptr[0] + b * s.batch[0] + r * s.ld[0];
  const T* second = (const T*)s.ptr[1] + b * s.batch[1] + (r - s.rows0) * s.ld[1];
  return r < s.rows0 ? first : second;
}

__device__ __forceinline__ void* out_row(const AttnArgs& a, int64_t b, int64_t r, int esize) {
  char* first = (char*)a.out[0] + (b * a.out_batch[0] + r * a.out_ld[0]) * esize;
  char* second = (char*)a.out[1] + (b * a.out_batch[1] + (r - a.out_rows0) * a.out_ld[1]) * esize;
  return r < a.out_rows0 ? first : second;
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

// LDS layouts of the key and value tiles: 64 rows of D elements each, row
// major as in memory (both arrive by DMA), swizzled by 16-byte chunk for
// gfx950's LDS (64 four-byte banks; a 16-byte read is served sixteen lanes
// at a time, an 8-byte read thirty-two at a time). Chunk c of row `key`
// sits at chunk c ^ x(key).
// Keys are read 16 bytes per lane, sixteen consecutive rows at one chunk:
// x = key % 16 at D = 128; at D = 64 rows are 128 bytes, so rows r and r + 1
// share the bank span and x = (key / 2) % 8.
template <int D>
__device__ __forceinline__ int k_swz(int key) {
  return D == 128 ? (key & 15) : ((key >> 1) & 7);
}
// Values are read by the transposing ds_read_b64_tr_b16: thirty-two lanes
// cover four consecutive rows, 64 bytes (four chunks) of each. x = 4 (key % 4)
// at D = 128 puts each row's four chunks on their own 16 banks; at D = 64
// rows r and r + 1 already sit on different halves and x = 4 ((key / 2) % 2)
// separates r and r + 2.
template <int D>
__device__ __forceinline__ int v_swz(int key) {
  return D == 128 ? ((key & 3) << 2) : (((key >> 1) & 1) << 2);
}

// ds_read_b64_tr_b16: in each group of 16 lanes, lane L supplies the address
// of four 16-bit elements (row L / 4 of a 4 x 16 block, columns 4 (L % 4) ..
// 4 (L % 4) + 3); lane j receives column j of the block, rows 0..3.
typedef short s16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_read_tr16(const char* p) {
  typedef __attribute__((address_space(3))) s16x4* lds_s16x4;
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4)(p)));
}

// One tile: 128 queries (4 waves x 32) of one (batch, head) over key blocks
// [kb0, kb1) of 64 keys. With part == nullptr the tile covers every key and
// writes the normalised output; otherwise it leaves its unnormalised O^T
// registers, running max and partial row sum in `part` (field-major, one
// float per thread per field) for attn_combine_kernel.
//
// K and V blocks are double buffered in four distinct LDS arrays (K0/V0 for
// even blocks, K1/V1 for odd): the DMA of block kb + 1 starts when block kb
// does, and since its destination is a different restrict pointer from
// every array read during block kb, no LDS read has to wait for it.
//
// Softmax: the running max is kept over raw scores, so a probability is one
// fused multiply-add (score * scale * log2 e - max) and one v_exp_f32
// (2^x; results below 2^-126 flush to zero, far below a bf16 probability's
// resolution); the max in use may trail the true one by up to 2^8 (see the
// rescale below). Masks and the key tail change the raw scores in a uniform
// branch (only the masked kernels and the last key block take it): a ruled-
// out key gets -10000 / scale added, i.e. -10000 after scaling, and keys
// past the end get -inf.
template <typename T, int D, int MASK>
__device__ __forceinline__ void attn_tile_body(const AttnArgs& a, int qb, int head, int b, int kb0, int kb1,
                                               float* part, T* __restrict__ K0, T* __restrict__ K1,
                                               T* __restrict__ V0, T* __restrict__ V1) {
  typedef typename AMfma<T>::V V;
  constexpr int BQ = 128, BKEY = 64;
  constexpr int KCH = D / 8;                      // 16-byte chunks per row
  constexpr int DT = D / 32;                      // output tiles along d

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lq = lane & 31, lh = lane >> 5;
  const int64_t col0 = int64_t(head) * D;
  const int qi = qb * BQ + wave * 32 + lq;
  const int qm = min(qi, a.T - 1);

  // Q^T fragments, resident for the whole key loop.
  V qf[D / 16];
  {
    const T* qrow = seg_row<T>(a.q, b, qm) + col0;
#pragma unroll
    for (int s = 0; s < D / 16; s++) qf[s] = *(const V*)(qrow + s * 16 + lh * 8);
  }

  // K and V go global -> LDS by DMA (buffer_load ... lds): a wave-wide load
  // fills one kilobyte, KROWS rows; lane l lands at byte 16 l (row l / (D/8)
  // of the group, physical chunk l % (D/8)) and fetches the logical chunk
  // that the swizzle places there.
  constexpr int KROWS = 512 / D;            // rows per kilobyte load
  constexpr int LOADS = BKEY / KROWS / 4;   // loads per wave per block and tensor
  const int kr = lane / KCH, kpc = lane % KCH;
  int kcol[LOADS], vcol[LOADS];
#pragma unroll
  for (int i = 0; i < LOADS; i++) {
    const int key = (wave * LOADS + i) * KROWS + kr;
    kcol[i] = (int)col0 + ((kpc ^ k_swz<D>(key)) << 3);
    vcol[i] = (int)col0 + ((kpc ^ v_swz<D>(key)) << 3);
  }
  // (Offsets fit in 32 bits when a row stride is below 2^24 elements.)
  const bool small_ld = a.k.ld[0] < (1 << 24) && a.k.ld[1] < (1 << 24) && a.v.ld[0] < (1 << 24) &&
                        a.v.ld[1] < (1 << 24);
  // Block kb of one tensor into `buf`. The base of a block inside one
  // segment is uniform. Ternaries, not s.ptr[sg]: a runtime index into the
  // kernel arguments makes the compiler fetch them from memory every block.
  auto issue = [&](const AttnSeg& sg, T* buf, int kb, const int (&col)[LOADS], bool value) {
    const int key0 = kb * BKEY;
    const bool second = key0 >= sg.rows0;
    if (small_ld && (second || key0 + BKEY <= sg.rows0)) {
      // Rows past the keys (or past the segment) read as zeros: a zero
      // value row keeps 0 * stale from turning into NaN, and a zero key row
      // is masked like every key past the end.
      const int64_t end = second ? a.S : std::min<int64_t>(sg.rows0, a.S);
      const int rows = (int)std::min<int64_t>(BKEY, end - key0);
      const int64_t ld = second ? sg.ld[1] : sg.ld[0];
      const T* base = second ? (const T*)sg.ptr[1] + b * sg.batch[1] + (key0 - sg.rows0) * sg.ld[1]
                             : (const T*)sg.ptr[0] + b * sg.batch[0] + key0 * sg.ld[0];
      const __amdgpu_buffer_rsrc_t rk = make_rsrc(base, uint32_t(rows * ld * 2));
#pragma unroll
      for (int i = 0; i < LOADS; i++) {
        const int key = (wave * LOADS + i) * KROWS + kr;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (lds_ptr_t)&buf[(wave * LOADS + i) * KROWS * D], 16,
                                                 uint32_t((key * ld + col[i]) * 2), 0, 0, 0);
      }
      return;
    }
    // A block across the two segments (or huge strides): chunk by chunk
    // through registers; value rows past the keys are zeroed.
#pragma unroll 1
    for (int i = 0; i < BKEY * KCH / 256; i++) {
      const int id = tid + i * 256;
      const int key = id / KCH, c = id % KCH;
      const int gk = min(key0 + key, a.S - 1);
      uint4 x = *(const uint4*)(seg_row<T>(sg, b, gk) + col0 + c * 8);
      if (value && key0 + key >= a.S) x = make_uint4(0, 0, 0, 0);
      *(uint4*)&buf[key * D + ((c ^ (value ? v_swz<D>(key) : k_swz<D>(key))) << 3)] = x;
    }
  };

  f32x16 o[DT];
#pragma unroll
  for (int j = 0; j < DT; j++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[j][r] = 0.f;
  float m_run = -INFINITY;
  // Row sums of the rounded probabilities (the values the output is weighted
  // with), one partial per 16-key step so the dot-product chains stay short.
  float lp[4] = {0.f, 0.f, 0.f, 0.f};
  const float sl = a.scale * kLog2e;
  const bool pos = sl > 0.f;
  const float mask_raw = -10000.0f / a.scale;
  const int key_len = MASK == NDX_MASK_KEY_LENGTH ? a.mask[0] : a.S;
  const f32x16 zero16 = {};

  // Byte offsets of this lane's fragment reads within one buffer. Keys:
  // step s reads chunk 2 s + lh of row lq (the second 32-key tile is 32 rows
  // on); the swizzle of row kt * 32 + lq does not depend on kt. Values: for
  // the 16-key step u, output tile dt and half h, lane L of 16-lane group g
  // addresses row 16 u + 8 h + kl, kl = 4 (g / 2) + L / 4, at d = 32 dt +
  // 16 (g % 2) + 4 (L % 4): the transposed read then hands lane l the values
  // of d = 32 dt + l % 32 at keys 16 u + 8 h + 4 (l / 32) + 0..3, which are
  // the keys of the score registers that P^T takes its operand from. The
  // swizzle depends on kl only, so u and h are immediates.
  constexpr int NSD = D / 16;
  int kq[NSD], vq[DT];
  {
    const int kx = k_swz<D>(lq);
#pragma unroll
    for (int s2 = 0; s2 < NSD; s2++) kq[s2] = (lq * D + (((2 * s2 + lh) ^ kx) << 3)) * 2;
    const int g = lane >> 4, L = lane & 15;
    const int kl = 4 * (g >> 1) + (L >> 2);
    const int vx = v_swz<D>(kl) >> 2;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
      vq[dt] = kl * D * 2 + ((((dt ^ vx) << 2) | ((g & 1) << 1) | ((L >> 1) & 1)) << 4) + ((L & 1) << 3);
  }

  // Block kb from Kc/Vc, with block kb + 1 on its way into Kn/Vn.
  auto block = [&](int kb, const T* Kc, const T* Vc, T* Kn, T* Vn) {
    if (kb + 1 < kb1) {
      issue(a.k, Kn, kb + 1, kcol, false);
      issue(a.v, Vn, kb + 1, vcol, true);
    }
    // S^T for 64 keys: two 32-key tiles (raw scores), the key fragment of
    // the next step read under the current step's MFMA.
    f32x16 sacc[2];
    {
      const char* kbuf = (const char*)Kc;
      V kf[2];
      kf[0] = *(const V*)(kbuf + kq[0]);
#pragma unroll
      for (int i = 0; i < 2 * NSD; i++) {
        const int kt = i / NSD, s = i % NSD;
        if (i + 1 < 2 * NSD)
          kf[(i + 1) & 1] = *(const V*)(kbuf + kq[(i + 1) % NSD] + ((i + 1) / NSD) * (32 * D * 2));
        sacc[kt] = AMfma<T>::mma(kf[i & 1], qf[s], s == 0 ? zero16 : sacc[kt]);
      }
    }
    if (MASK != NDX_MASK_NONE || (kb + 1) * BKEY > a.S) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          float x = sacc[kt][r];
          const int key = kb * BKEY + kt * 32 + 8 * (r >> 2) + 4 * lh + (r & 3);
          if (MASK == NDX_MASK_KEY_LENGTH) {
            if (key >= key_len) x += mask_raw;
          } else if (MASK == NDX_MASK_BOOLEAN) {
            const int64_t mi = b * a.mask_stride[0] + head * a.mask_stride[1] + int64_t(qm) * a.mask_stride[2] +
                               int64_t(min(key, a.S - 1)) * a.mask_stride[3];
            if (a.mask[mi] == 0) x += mask_raw;
          }
          if (key >= a.S) x = pos ? -INFINITY : INFINITY;
          sacc[kt][r] = x;
        }
    }
    // Running max in scaled units: the largest raw score times a positive
    // scale (the smallest for a negative one).
    float mx = sacc[0][0];
    if (pos) {
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) mx = fmaxf(mx, sacc[kt][r]);
    } else {
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) mx = fminf(mx, sacc[kt][r]);
    }
    const float mloc = mx * sl;
    const float m_blk = fmaxf(m_run, fmaxf(mloc, __shfl_xor(mloc, 32, 64)));
    // The max subtracted in the exponent may lag the true running max by up
    // to 8 (log2 units): probabilities then reach at most 2^8, exact in fp32
    // and bf16, and the output and row sum carry the same factor, so the
    // result is unchanged. The rescale of the output (64 multiplies) runs
    // only when some lane's max grows by more than that, which after the
    // first blocks is rare, instead of whenever any of the wave's 32 queries
    // meets a new maximum.
    if (__builtin_amdgcn_ballot_w64(m_blk > m_run + 8.0f)) {
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_blk);
#pragma unroll
      for (int u = 0; u < 4; u++) lp[u] *= alpha;
#pragma unroll
      for (int j = 0; j < DT; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[j][r] *= alpha;
      m_run = m_blk;
    }
    const float m_new = m_run;
#pragma unroll
    for (int kt = 0; kt < 2; kt++)
#pragma unroll
      for (int r = 0; r < 16; r++) sacc[kt][r] = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[kt][r], sl, -m_new));

    // O^T += V^T P^T over four 16-key steps.
    const char* vbuf = (const char*)Vc;
#pragma unroll
    for (int u = 0; u < 4; u++) {
      V pb;
#pragma unroll
      for (int j = 0; j < 8; j++) pb[j] = (T)sacc[u >> 1][(u & 1) * 8 + j];
      lp[u] = AMfma<T>::sum8(pb, lp[u]);
#pragma unroll
      for (int dt = 0; dt < DT; dt++) {
        const uint2 x0 = lds_read_tr16(vbuf + vq[dt] + (u * 16) * D * 2);
        const uint2 x1 = lds_read_tr16(vbuf + vq[dt] + (u * 16 + 8) * D * 2);
        const V vf = __builtin_bit_cast(V, make_uint4(x0.x, x0.y, x1.x, x1.y));
        o[dt] = AMfma<T>::mma(vf, pb, o[dt]);
      }
    }
    // This wave's DMA of block kb + 1 has landed; after the barrier, every
    // wave's has, and every wave is done reading block kb.
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };

  issue(a.k, K0, kb0, kcol, false);
  issue(a.v, V0, kb0, vcol, true);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int kb = kb0; kb < kb1; kb += 2) {
    block(kb, K0, V0, K1, V1);
    if (kb + 1 < kb1) block(kb + 1, K1, V1, K0, V0);
  }

  const float l_part = (lp[0] + lp[1]) + (lp[2] + lp[3]);
  if (part) {
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int r = 0; r < 16; r++) part[(dt * 16 + r) * 256 + tid] = o[dt][r];
    part[DT * 16 * 256 + tid] = m_run;
    part[(DT * 16 + 1) * 256 + tid] = l_part;
    return;
  }
  const float l_tot = l_part + __shfl_xor(l_part, 32, 64);
  const float inv = 1.0f / l_tot;
  if (qi < a.T) {
    T* orow = (T*)out_row(a, b, qi, sizeof(T)) + col0;
#pragma unroll
    for (int dt = 0; dt < DT; dt++)
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int d = dt * 32 + 8 * g + 4 * lh;
        T v4[4];
#pragma unroll
        for (int e = 0; e < 4; e++) v4[e] = (T)(o[dt][g * 4 + e] * inv);
        *(uint2*)(orow + d) = *(const uint2*)v4;
      }
  }
}

// How tiles are spread over workgroups. Without `split` there is one tile
// per workgroup (decoded XCD-aware by attn_tile). With it the grid is the
// head_tiles whole tiles (a whole number of rounds of the resident
// workgroups), then `ps` pieces of each of the tail_tiles remaining tiles,
// piece k taking key blocks [k KB / ps, (k + 1) KB / ps): the dispatcher
// starts them in order, so the last round is short pieces instead of a few
// whole tiles. A piece leaves its partial in `part`; attn_combine_kernel
// merges the ps partials of each tail tile.
struct AttnSched {
  int grid;
  int split;
  int qblocks, KB;
  int head_tiles, tail_tiles, ps;
  float* part;
};

__device__ __forceinline__ void decode_tile(int t, int qblocks, int H, int& qb, int& head, int& b) {
  qb = t % qblocks;
  const int r = t / qblocks;
  head = r % H;
  b = r / H;
}

template <typename T, int D, int MASK>
__global__ __launch_bounds__(256, 2) void flash_attn_kernel(AttnArgs a, AttnSched sc) {
  constexpr int DT = D / 32;
  __shared__ __attribute__((aligned(1024))) T K0[64 * D];
  __shared__ __attribute__((aligned(1024))) T K1[64 * D];
  __shared__ __attribute__((aligned(1024))) T V0[64 * D];
  __shared__ __attribute__((aligned(1024))) T V1[64 * D];
  int qb, head, b;
  if (!sc.split) {
    if (!attn_tile(blockIdx.x, sc.grid, sc.qblocks, a.H, a.B, qb, head, b)) return;
    attn_tile_body<T, D, MASK>(a, qb, head, b, 0, sc.KB, nullptr, K0, K1, V0, V1);
    return;
  }
  const int w = blockIdx.x;
  if (w < sc.head_tiles) {
    // Consecutive tiles (the query blocks of one head) to one XCD.
    const int t = (w % 8) * (sc.head_tiles / 8) + w / 8;
    decode_tile(t, sc.qblocks, a.H, qb, head, b);
    attn_tile_body<T, D, MASK>(a, qb, head, b, 0, sc.KB, nullptr, K0, K1, V0, V1);
    return;
  }
  const int p = w - sc.head_tiles;
  const int ti = p / sc.ps, k = p % sc.ps;
  decode_tile(sc.head_tiles + ti, sc.qblocks, a.H, qb, head, b);
  attn_tile_body<T, D, MASK>(a, qb, head, b, k * sc.KB / sc.ps, (k + 1) * sc.KB / sc.ps,
                             sc.part + int64_t(p) * ((DT * 16 + 2) * 256), K0, K1, V0, V1);
}

// Merges the ps partials of tail tile blockIdx.x, columns d in [32 y,
// 32 y + 32) with y = blockIdx.y: each piece left O^T, the running max and
// the partial row sum in the same lane layout, so each thread combines its
// own registers; the maxima and sums first (two loads per piece), then the
// 16 outputs of its column group (all loads independent).
template <typename T, int D>
__global__ __launch_bounds__(256) void attn_combine_kernel(AttnArgs a, AttnSched sc) {
  constexpr int F = D / 32 * 16;
  const int ti = blockIdx.x, dt = blockIdx.y, tid = threadIdx.x;
  const float* base = sc.part + int64_t(ti) * sc.ps * ((F + 2) * 256);
  float m = -INFINITY;
  for (int k = 0; k < sc.ps; k++) m = fmaxf(m, base[int64_t(k) * (F + 2) * 256 + F * 256 + tid]);
  float l = 0.f, o[16];
#pragma unroll
  for (int r = 0; r < 16; r++) o[r] = 0.f;
  for (int k = 0; k < sc.ps; k++) {
    const float* part = base + int64_t(k) * (F + 2) * 256;
    const float w = exp2f(part[F * 256 + tid] - m);
    l += part[(F + 1) * 256 + tid] * w;
#pragma unroll
    for (int r = 0; r < 16; r++) o[r] += part[(dt * 16 + r) * 256 + tid] * w;
  }
  int qb, head, b;
  decode_tile(sc.head_tiles + ti, sc.qblocks, a.H, qb, head, b);
  const int lane = tid & 63, wave = tid >> 6, lq = lane & 31, lh = lane >> 5;
  const int qi = qb * 128 + wave * 32 + lq;
  const float inv = 1.0f / (l + __shfl_xor(l, 32, 64));
  if (qi < a.T) {
    T* orow = (T*)out_row(a, b, qi, sizeof(T)) + int64_t(head) * D;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const int d = dt * 32 + 8 * g + 4 * lh;
      T v4[4];
#pragma unroll
      for (int e = 0; e < 4; e++) v4[e] = (T)(o[g * 4 + e] * inv);
      *(uint2*)(orow + d) = *(const uint2*)v4;
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

  // The query half-row as float4 values indexed by constants only (a float
  // array written through float4 pointers would live in scratch memory).
  float4 qf[DH / 4];
  {
    const float* qrow = seg_row<float>(a.q, b, qm) + col0 + lh * DH;
#pragma unroll
    for (int t = 0; t < DH / 4; t++) qf[t] = *(const float4*)(qrow + 4 * t);
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
      const float4 q = qf[t / 4];
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.x, q.x, sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.x, q.x, sacc[1], 0, 0, 0);
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.y, q.y, sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.y, q.y, sacc[1], 0, 0, 0);
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.z, q.z, sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.z, q.z, sacc[1], 0, 0, 0);
      sacc[0] = __builtin_amdgcn_mfma_f32_32x32x2f32(a0.w, q.w, sacc[0], 0, 0, 0);
      sacc[1] = __builtin_amdgcn_mfma_f32_32x32x2f32(a1.w, q.w, sacc[1], 0, 0, 0);
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
    // The lazy rescale of the 16-bit kernel: the max in use may trail the
    // running max by up to 8 (log2 units).
    const float m_blk = fmaxf(m_run, mloc);
    if (__builtin_amdgcn_ballot_w64(m_blk > m_run + 8.0f)) {
      const float alpha = exp2f(m_run - m_blk);
      l_part *= alpha;
#pragma unroll
      for (int j = 0; j < DT; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[j][r] *= alpha;
      m_run = m_blk;
    }
    const float m_new = m_run;
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

static int cu_count() {
  static int n = 0;
  if (n == 0) {
    int dev = 0, c = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) ==
                                                 hipSuccess && c > 0)
      n = c;
    else
      n = 256;
  }
  return n;
}

// The schedule of the 16-bit flash kernel for a shape: split when at least
// one full round of whole tiles leaves a last round at most three quarters
// full (two resident workgroups per CU); the tail tiles are cut into as
// many pieces as fill one round, at most 8 (the pieces' own overhead and
// the merge grow with their count) and at least 2 key blocks each.
static AttnSched attn_schedule(int B, int T, int S, int H) {
  AttnSched sc{};
  sc.qblocks = (T + 127) / 128;
  sc.KB = (S + 63) / 64;
  const int tiles = sc.qblocks * H * B;
  const int slots = cu_count() * 2;
  const int full = tiles / slots, tail = tiles - full * slots;
  const int ps = std::min(std::min((slots + tail - 1) / std::max(tail, 1), 8), sc.KB / 2);
  if (full >= 1 && tail > 0 && tail * 4 <= slots * 3 && ps >= 2 && slots % 8 == 0) {
    sc.split = 1;
    sc.head_tiles = full * slots;
    sc.tail_tiles = tail;
    sc.ps = ps;
    sc.grid = sc.head_tiles + tail * ps;
  } else {
    sc.grid = (tiles + 7) / 8 * 8;
  }
  return sc;
}

static bool attn_mfma16(int dtype, int d, int dv) {
  return (dtype == NDX_BF16 || dtype == NDX_F16) && d == dv && (d == 128 || d == 64);
}

int64_t attention_scratch_bytes(int B, int T, int S, int H, int d, int dv, int dtype) {
  if (T == 0 || B == 0 || !attn_mfma16(dtype, d, dv)) return 0;
  const AttnSched sc = attn_schedule(B, T, S, H);
  if (!sc.split) return 0;
  return int64_t(sc.tail_tiles) * sc.ps * (d / 32 * 16 + 2) * 256 * int64_t(sizeof(float));
}

void launch_attention(const AttnArgs& a, void* scratch, hipStream_t s) {
  if (a.T == 0 || a.B == 0) return;
  const bool mfma = attn_mfma16(a.dtype, a.d, a.dv) && rows_aligned(a.q, 2) && rows_aligned(a.k, 2) &&
                    rows_aligned(a.v, 2) && (uintptr_t)a.out[0] % 16 == 0 && (uintptr_t)a.out[1] % 16 == 0;
  if (mfma) {
    AttnSched sc = attn_schedule(a.B, a.T, a.S, a.H);
    // NDX_ATTN_SPLIT=0 runs one whole tile per workgroup (for sweeps); read per launch.
    const char* pin = getenv("NDX_ATTN_SPLIT");
    if (pin && pin[0] == '0') scratch = nullptr;
    if (sc.split && !scratch) sc = AttnSched{(sc.qblocks * a.H * a.B + 7) / 8 * 8, 0, sc.qblocks, sc.KB, 0, 0, 0, nullptr};
    sc.part = (float*)scratch;
    const bool bf = a.dtype == NDX_BF16;
#define NDX_FA(TYPE, DIM, MK) \
  hipLaunchKernelGGL((flash_attn_kernel<TYPE, DIM, MK>), dim3(sc.grid), dim3(256), 0, s, a, sc)
#define NDX_FA_MASKS(TYPE, DIM)                                      \
  do {                                                               \
    if (a.mask_kind == NDX_MASK_KEY_LENGTH) NDX_FA(TYPE, DIM, 1);    \
    else if (a.mask_kind == NDX_MASK_BOOLEAN) NDX_FA(TYPE, DIM, 2);  \
    else NDX_FA(TYPE, DIM, 0);                                       \
  } while (0)
    if (bf) {
      if (a.d == 128) NDX_FA_MASKS(__bf16, 128);
      else NDX_FA_MASKS(__bf16, 64);
    } else {
      if (a.d == 128) NDX_FA_MASKS(_Float16, 128);
      else NDX_FA_MASKS(_Float16, 64);
    }
#undef NDX_FA_MASKS
#undef NDX_FA
    if (sc.split) {
      if (bf) {
        if (a.d == 128) hipLaunchKernelGGL((attn_combine_kernel<__bf16, 128>), dim3(sc.tail_tiles, 128 / 32), dim3(256), 0, s, a, sc);
        else hipLaunchKernelGGL((attn_combine_kernel<__bf16, 64>), dim3(sc.tail_tiles, 64 / 32), dim3(256), 0, s, a, sc);
      } else {
        if (a.d == 128) hipLaunchKernelGGL((attn_combine_kernel<_Float16, 128>), dim3(sc.tail_tiles, 128 / 32), dim3(256), 0, s, a, sc);
        else hipLaunchKernelGGL((attn_combine_kernel<_Float16, 64>), dim3(sc.tail_tiles, 64 / 32), dim3(256), 0, s, a, sc);
      }
    }
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
