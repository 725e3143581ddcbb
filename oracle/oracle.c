/*
 * The oracle: a CPU restatement, in plain C, of NaiveDiffusion's own CPU
 * layer math and of the DirectML operator semantics its graphs rely on.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product links or calls this
 * file: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * load liboracle.so, and only to check the GPU's results against (or, for
 * the CPU baseline, as the thing timed beside the GPU). Every function cites the reference
 * member it restates (paths relative to src/NaiveDiffusion/ of the
 * reference). The reference is C#/.NET on DirectML and cannot be built or
 * run here, so nothing is compiled from its sources.
 *
 * Arithmetic follows the reference where the reference fixes it: fp32
 * products with the 4 x 8-lane accumulator dot product, norms accumulated
 * in double, max-subtracted fp32 softmax, the A&S 7.1.26 erf. Built with
 * -ffp-contract=off so products and sums round separately as in .NET.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define API __attribute__((visibility("default")))

/* ---- narrow float types (Tensors/HostTensor.cs:110-130, 168-192) ---------- */

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* IEEE binary16 from binary32, round to nearest even (what (Half)x and
 * TensorPrimitives.ConvertToHalf do). Written bit by bit: gcc here has no
 * _Float16, and an independent restatement is the point of an oracle. */
API uint16_t orc_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) /* inf or nan */
        return (uint16_t)(sign | 0x7c00u | (ax > 0x7f800000u ? 0x200u | ((ax >> 13) & 0x3ffu) : 0u));
    int32_t e = (int32_t)(ax >> 23) - 127;
    uint32_t m = ax & 0x7fffffu;
    if (e > 15) return (uint16_t)(sign | 0x7c00u); /* overflow */
    if (e >= -14) {
        /* normal half: 10 mantissa bits, round the 13 dropped bits */
        uint32_t h = ((uint32_t)(e + 15) << 10) | (m >> 13);
        uint32_t rest = m & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++; /* may carry into inf: correct */
        return (uint16_t)(sign | h);
    }
    if (e < -25) return (uint16_t)sign; /* below half the smallest subnormal */
    /* subnormal half: value = m' * 2^-24 */
    uint32_t full = m | 0x800000u;          /* 24-bit significand, value full * 2^(e-23) */
    int shift = -e - 1;                      /* = (-14 - e) + 13 */
    uint32_t h = full >> shift;
    uint32_t rest = full & ((1u << shift) - 1u);
    uint32_t halfway = 1u << (shift - 1);
    if (rest > halfway || (rest == halfway && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

API float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        if (m == 0) return u2f(sign);
        float v = (float)m * (1.0f / 16777216.0f); /* m * 2^-24, exact */
        return sign ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* bfloat16 is the top half of a float32 (HostTensor.cs:178-187); narrowing
 * (used for the synthetic weights) rounds to nearest even. */
API uint16_t orc_f32_to_bf16(float f) {
    uint32_t x = f2u(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}
API float orc_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* ---- CpuMath (Tensors/CpuMath.cs) ----------------------------------------- */

/* CpuMath.Dot, CpuMath.cs:311-335: four 8-lane accumulators, summed lane-wise
 * ((s0 + s1) + s2) + s3, then across lanes, then the scalar tail. */
API float orc_dot(const float* a, const float* b, int n) {
    float s0[8] = {0}, s1[8] = {0}, s2[8] = {0}, s3[8] = {0};
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        for (int j = 0; j < 8; j++) {
            s0[j] += a[i + j] * b[i + j];
            s1[j] += a[i + 8 + j] * b[i + 8 + j];
            s2[j] += a[i + 16 + j] * b[i + 16 + j];
            s3[j] += a[i + 24 + j] * b[i + 24 + j];
        }
    }
    float total = 0.f;
    for (int j = 0; j < 8; j++) total += ((s0[j] + s1[j]) + s2[j]) + s3[j];
    for (; i < n; i++) total += a[i] * b[i];
    return total;
}

/* CpuMath.Linear, CpuMath.cs:34-64: y[m, o] = dot(x[m, :], w[o, :]) + bias[o],
 * one parallel task per output column. */
API void orc_linear(const float* x, int rows, int inner, const float* w, const float* bias, float* y,
                    int outer) {
#pragma omp parallel for schedule(dynamic, 16)
    for (int o = 0; o < outer; o++) {
        const float* col = w + (size_t)o * inner;
        float shift = bias ? bias[o] : 0.f;
        for (int m = 0; m < rows; m++) y[(size_t)m * outer + o] = orc_dot(x + (size_t)m * inner, col, inner) + shift;
    }
}

/* CpuMath.LayerNorm, CpuMath.cs:92-122: two passes in double; weight and
 * bias may be NULL (the affine-free LayerNorm the DiTs modulate). */
API void orc_layer_norm(const float* x, int rows, int width, const float* weight, const float* bias, float* y,
                        float eps) {
#pragma omp parallel for
    for (int m = 0; m < rows; m++) {
        const float* s = x + (size_t)m * width;
        float* t = y + (size_t)m * width;
        double sum = 0;
        for (int i = 0; i < width; i++) sum += s[i];
        double mean = sum / width;
        double sq = 0;
        for (int i = 0; i < width; i++) {
            double c = s[i] - mean;
            sq += c * c;
        }
        double scale = 1.0 / sqrt(sq / width + eps);
        for (int i = 0; i < width; i++) {
            float v = (float)((s[i] - mean) * scale);
            if (weight) v = v * weight[i];
            if (bias) v = v + bias[i];
            t[i] = v;
        }
    }
}

/* CpuMath.RmsNorm, CpuMath.cs:128-146. weight may be NULL. */
API void orc_rms_norm(const float* x, int rows, int width, const float* weight, float* y, float eps) {
#pragma omp parallel for
    for (int m = 0; m < rows; m++) {
        const float* s = x + (size_t)m * width;
        float* t = y + (size_t)m * width;
        double sq = 0;
        for (int i = 0; i < width; i++) sq += (double)s[i] * s[i];
        float scale = (float)(1.0 / sqrt(sq / width + eps));
        for (int i = 0; i < width; i++) t[i] = weight ? s[i] * scale * weight[i] : s[i] * scale;
    }
}

/* CpuMath.Rope, CpuMath.cs:154-173: rotate-half, in place over [rows, heads, dim]. */
API void orc_rope(float* x, int rows, int heads, int dim, const float* cos, const float* sin) {
    int half = dim / 2;
#pragma omp parallel for
    for (int m = 0; m < rows; m++) {
        const float* c = cos + (size_t)m * half;
        const float* s = sin + (size_t)m * half;
        for (int h = 0; h < heads; h++) {
            float* v = x + ((size_t)m * heads + h) * dim;
            for (int i = 0; i < half; i++) {
                float lo = v[i], hi = v[i + half];
                v[i] = lo * c[i] - hi * s[i];
                v[i + half] = hi * c[i] + lo * s[i];
            }
        }
    }
}

/* CpuMath.RopeTables, CpuMath.cs:177-194. */
API void orc_rope_tables(int rows, int dim, double theta, float* cos_out, float* sin_out) {
    int half = dim / 2;
    for (int i = 0; i < half; i++) {
        float freq = 1.0f / powf((float)theta, 2.0f * i / dim);
        for (int m = 0; m < rows; m++) {
            float angle = m * freq;
            cos_out[(size_t)m * half + i] = cosf(angle);
            sin_out[(size_t)m * half + i] = sinf(angle);
        }
    }
}

/* CpuMath.Attention, CpuMath.cs:203-248 (GQA, causal). */
API void orc_attention(const float* q, const float* k, const float* v, int rows, int key_rows, int q_heads,
                       int k_heads, int dim, int causal, float* y) {
    int qw = q_heads * dim, kw = k_heads * dim, group = q_heads / k_heads;
    float scale = 1.0f / sqrtf((float)dim);
#pragma omp parallel for schedule(dynamic, 8)
    for (int work = 0; work < q_heads * rows; work++) {
        int head = work / rows, i = work % rows;
        int qo = head * dim, ko = head / group * dim;
        int visible = causal ? (i + 1 < key_rows ? i + 1 : key_rows) : key_rows;
        float* scores = (float*)malloc(sizeof(float) * (size_t)visible);
        const float* qr = q + (size_t)i * qw + qo;
        float largest = -INFINITY;
        for (int j = 0; j < visible; j++) {
            float s = orc_dot(qr, k + (size_t)j * kw + ko, dim) * scale;
            scores[j] = s;
            if (s > largest) largest = s;
        }
        float total = 0;
        for (int j = 0; j < visible; j++) {
            scores[j] = expf(scores[j] - largest);
            total += scores[j];
        }
        float norm = 1.0f / total;
        float* t = y + (size_t)i * qw + qo;
        memset(t, 0, sizeof(float) * (size_t)dim);
        for (int j = 0; j < visible; j++) {
            float wgt = scores[j] * norm;
            const float* vr = v + (size_t)j * kw + ko;
            for (int d = 0; d < dim; d++) t[d] += wgt * vr[d];
        }
        free(scores);
    }
}

/* DmlOps.MultiheadAttention semantics (Dml/DmlOps.cs:480-520) in the
 * arithmetic of CpuMath.Attention: packed [batch, tokens, heads*dim], scores
 * scaled, -10000 added where the mask rules a key out (:483), fp32
 * max-subtracted softmax. mask_kind 0 none, 1 key length (key_len real
 * leading keys), 2 boolean [batch or 1][heads or 1][rows][keys] table with
 * the given element strides (0 broadcasts). */
API void orc_mha(const float* q, const float* k, const float* v, int batch, int rows, int keys, int heads,
                 int dim, float scale, int mask_kind, int key_len, const int32_t* mask, int64_t mb, int64_t mh,
                 int64_t mt, int64_t ms, float* y) {
    int width = heads * dim;
#pragma omp parallel for schedule(dynamic, 8)
    for (int work = 0; work < batch * heads * rows; work++) {
        int i = work % rows, head = (work / rows) % heads, b = work / rows / heads;
        const float* qr = q + ((size_t)b * rows + i) * width + (size_t)head * dim;
        float* scores = (float*)malloc(sizeof(float) * (size_t)keys);
        float largest = -INFINITY;
        for (int j = 0; j < keys; j++) {
            float s = orc_dot(qr, k + ((size_t)b * keys + j) * width + (size_t)head * dim, dim) * scale;
            if (mask_kind == 1 && j >= key_len) s += -10000.0f;
            if (mask_kind == 2 && mask[b * mb + head * mh + (int64_t)i * mt + (int64_t)j * ms] == 0) s += -10000.0f;
            scores[j] = s;
            if (s > largest) largest = s;
        }
        float total = 0;
        for (int j = 0; j < keys; j++) {
            scores[j] = expf(scores[j] - largest);
            total += scores[j];
        }
        float norm = 1.0f / total;
        float* t = y + ((size_t)b * rows + i) * width + (size_t)head * dim;
        memset(t, 0, sizeof(float) * (size_t)dim);
        for (int j = 0; j < keys; j++) {
            float wgt = scores[j] * norm;
            const float* vr = v + ((size_t)b * keys + j) * width + (size_t)head * dim;
            for (int d = 0; d < dim; d++) t[d] += wgt * vr[d];
        }
        free(scores);
    }
}

/* CpuMath.Silu, CpuMath.cs:260-266. */
API void orc_silu(float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] *= 1.0f / (1.0f + expf(-x[i]));
}

/* Abramowitz and Stegun 7.1.26, CpuMath.cs:299-307. */
static float orc_erf(float x) {
    float sign = (x > 0) - (x < 0);
    x = fabsf(x);
    float t = 1.0f / (1.0f + 0.3275911f * x);
    float series = ((((1.061405429f * t - 1.453152027f) * t + 1.421413741f) * t - 0.284496736f) * t + 0.254829592f) * t;
    return sign * (1.0f - series * expf(-x * x));
}

/* CpuMath.Gelu, CpuMath.cs:289-295: the exact GELU through the A&S erf. */
API void orc_gelu(float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = 0.5f * x[i] * (1.0f + orc_erf(x[i] * 0.70710678f));
}

/* GELU, tanh form, as the graph composes it (QwenImageDit.cs:510-515):
 * x * sigmoid(2 * 0.7978845608 * (x + 0.044715 x^3)). */
API void orc_gelu_tanh(float* x, int64_t n) {
    const float scale = 2.0f * 0.7978845608f;
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        float cubic = v * v * v * 0.044715f + v;
        x[i] = v * (1.0f / (1.0f + expf(-(cubic * scale))));
    }
}

API void orc_sigmoid(float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = 1.0f / (1.0f + expf(-x[i]));
}

API void orc_tanh(float* x, int64_t n) {
    for (int64_t i = 0; i < n; i++) x[i] = tanhf(x[i]);
}

/* ---- Transformer (Graph/Transformer.cs) --------------------------------- */

/* Transformer.Sinusoid, Transformer.cs:20-32. */
API void orc_sinusoid(float time, int width, float* out) {
    int half = width / 2;
    for (int i = 0; i < half; i++) {
        float freq = expf(-logf(10000.0f) * i / half);
        float angle = time * freq;
        out[i] = cosf(angle);
        out[half + i] = sinf(angle);
    }
}

/* Transformer.Modulate, Transformer.cs:72-80: LayerNorm without affine, then
 * * (1 + scale) + shift (shift may be NULL); one scale/shift row for all rows. */
API void orc_modulate(const float* x, int rows, int width, const float* shift, const float* scale, float eps,
                      float* y) {
    orc_layer_norm(x, rows, width, NULL, NULL, y, eps);
#pragma omp parallel for
    for (int m = 0; m < rows; m++)
        for (int i = 0; i < width; i++) {
            float v = y[(size_t)m * width + i] * (scale[i] + 1.0f);
            if (shift) v = v + shift[i];
            y[(size_t)m * width + i] = v;
        }
}

/* ---- Layers (Graph/Layers.cs) and DmlOps semantics ------------------------- */

/* Layers.GroupNorm, Layers.cs:166-185 (MVN over [N, G, C/G, HW] then the
 * per-channel affine), statistics in double as SmokeTest.cs:227-237. */
API void orc_group_norm(const float* x, int n, int c, int hw, int groups, const float* weight, const float* bias,
                        float eps, int silu, float* y) {
    int cpg = c / groups;
#pragma omp parallel for
    for (int ng = 0; ng < n * groups; ng++) {
        int b = ng / groups, g = ng % groups;
        size_t base = ((size_t)b * c + (size_t)g * cpg) * hw;
        size_t count = (size_t)cpg * hw;
        double mean = 0, var = 0;
        for (size_t i = 0; i < count; i++) mean += x[base + i];
        mean /= count;
        for (size_t i = 0; i < count; i++) var += (x[base + i] - mean) * (x[base + i] - mean);
        var /= count;
        for (size_t i = 0; i < count; i++) {
            int ch = g * cpg + (int)(i / hw);
            float v = (float)((x[base + i] - mean) / sqrt(var + eps));
            if (weight) v = v * weight[ch];
            if (bias) v = v + bias[ch];
            if (silu) v = v * (1.0f / (1.0f + expf(-v)));
            y[base + i] = v;
        }
    }
}

/* DmlOps.Convolution, Dml/DmlOps.cs:265-299: NCHW cross-correlation, filters
 * [cout, cin, kh, kw], start padding pad, output extent
 * (H + pad + pad_end - k) / stride + 1 (:276-281), bias per channel. */
API void orc_conv2d(const float* x, int n, int cin, int h, int w, const float* filt, int cout, int kh, int kw,
                    const float* bias, int stride, int pad, int pad_end, float* y) {
    int ho = (h + pad + pad_end - kh) / stride + 1, wo = (w + pad + pad_end - kw) / stride + 1;
#pragma omp parallel for collapse(2)
    for (int b = 0; b < n; b++)
        for (int co = 0; co < cout; co++)
            for (int oy = 0; oy < ho; oy++)
                for (int ox = 0; ox < wo; ox++) {
                    double acc = 0;
                    for (int ci = 0; ci < cin; ci++)
                        for (int ky = 0; ky < kh; ky++) {
                            int iy = oy * stride - pad + ky;
                            if (iy < 0 || iy >= h) continue;
                            for (int kx = 0; kx < kw; kx++) {
                                int ix = ox * stride - pad + kx;
                                if (ix < 0 || ix >= w) continue;
                                acc += (double)x[(((size_t)b * cin + ci) * h + iy) * w + ix] *
                                       filt[(((size_t)co * cin + ci) * kh + ky) * kw + kx];
                            }
                        }
                    if (bias) acc += bias[co];
                    y[(((size_t)b * cout + co) * ho + oy) * wo + ox] = (float)acc;
                }
}

/* DmlOps.Upsample2D nearest, Dml/DmlOps.cs:418-435. */
API void orc_upsample_nearest(const float* x, int n, int c, int h, int w, int scale, float* y) {
    int ho = h * scale, wo = w * scale;
    for (size_t i = 0; i < (size_t)n * c; i++)
        for (int oy = 0; oy < ho; oy++)
            for (int ox = 0; ox < wo; ox++)
                y[(i * ho + oy) * wo + ox] = x[(i * h + oy / scale) * w + ox / scale];
}

/* ---- BlockQuantizer (Tensors/BlockQuantizer.cs:34-101) --------------------- */

/* Quantize, BlockQuantizer.cs:34-80. w is [rows, cols] fp32 (the widened
 * weight); per row, per block of `block` columns: peak = max |w|, the
 * scale is peak / 127 rounded to its storage type (fp16 when fp16_scales,
 * else fp32), and with s the stored scale q = clamp(round_half_even(w *
 * (1 / s)), -127, 127), or an all-zero block where s == 0. Returns -1 when
 * the blocks do not tile the columns (Fits, :24-25). */
API int orc_quantize(const float* w, int rows, int cols, int block, int fp16_scales, int8_t* q, void* scales) {
    if (rows <= 0 || block <= 0 || cols % block != 0) return -1;
    int blocks = cols / block;
#pragma omp parallel for
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < blocks; b++) {
            const float* src = w + (size_t)r * cols + (size_t)b * block;
            int8_t* dst = q + (size_t)r * cols + (size_t)b * block;
            float peak = 0.f;
            for (int i = 0; i < block; i++) {
                float a = fabsf(src[i]);
                if (a > peak) peak = a;
            }
            float stored;
            if (fp16_scales) {
                uint16_t h = orc_f32_to_f16(peak / 127.0f);
                ((uint16_t*)scales)[(size_t)r * blocks + b] = h;
                stored = orc_f16_to_f32(h);
            } else {
                stored = peak / 127.0f;
                ((float*)scales)[(size_t)r * blocks + b] = stored;
            }
            if (stored == 0.f) {
                memset(dst, 0, (size_t)block);
                continue;
            }
            float inverse = 1.0f / stored;
            for (int i = 0; i < block; i++) {
                float v = nearbyintf(src[i] * inverse); /* default rounding mode: half to even */
                if (v > 127.f) v = 127.f;
                if (v < -127.f) v = -127.f;
                dst[i] = (int8_t)v;
            }
        }
    return 0;
}

/* NarrowingLoss.Quantization, Tensors/NarrowingLoss.cs:178-196: the error
 * energy sum (w - dequant)^2 and the signal energy sum w^2, in double. */
API void orc_quantization_loss(const float* w, int rows, int cols, int block, double* error, double* energy) {
    int8_t* q = (int8_t*)malloc((size_t)rows * cols);
    uint16_t* s = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)rows * (cols / block));
    orc_quantize(w, rows, cols, block, 1, q, s);
    double e = 0, g = 0;
    for (size_t i = 0; i < (size_t)rows * cols; i++) {
        size_t r = i / cols, b = (i % cols) / block;
        double d = (double)w[i] - (double)q[i] * orc_f16_to_f32(s[r * (cols / block) + b]);
        e += d * d;
        g += (double)w[i] * w[i];
    }
    *error = e;
    *energy = g;
    free(q);
    free(s);
}

/* ---- Qwen-Image inputs (Models/QwenImage) ----------------------------------- */

static const int kRopeAxes[3] = {16, 56, 56};

static void axis_frequencies(double* freq) {
    int p = 0;
    for (int a = 0; a < 3; a++)
        for (int k = 0; k < kRopeAxes[a] / 2; k++) freq[p++] = 1.0 / pow(10000.0, 2.0 * k / kRopeAxes[a]);
}

static void fill_rope(float* c, float* s, int token, double f0, double f1, double f2, const double* freq) {
    double pos[3] = {f0, f1, f2};
    int p = 0;
    for (int a = 0; a < 3; a++)
        for (int k = 0; k < kRopeAxes[a] / 2; k++, p++) {
            double angle = pos[a] * freq[p];
            c[(size_t)token * 64 + p] = (float)cos(angle);
            s[(size_t)token * 64 + p] = (float)sin(angle);
        }
}

/* QwenImageDit.RopeTables, QwenImageDit.cs:189-240: image cell (i, j) at
 * (textLength, i - ceil(h/2), j - ceil(w/2)), text token p at (p, p, p);
 * [tokens, 64] fp32. */
API void orc_qwen_rope_tables(int rows, int cols, int text_length, int context_rows, float* cos_out,
                              float* sin_out) {
    double freq[64];
    axis_frequencies(freq);
    int row_start = rows - rows / 2, col_start = cols - cols / 2;
    for (int i = 0; i < rows; i++)
        for (int j = 0; j < cols; j++)
            fill_rope(cos_out, sin_out, i * cols + j, text_length, i - row_start, j - col_start, freq);
    for (int p = 0; p < context_rows; p++) fill_rope(cos_out, sin_out, rows * cols + p, p, p, p, freq);
}

/* The MMDiT block's tables: image cells from the same {16, 56, 56} layout
 * with the frame axis at 0, text rows unrotated (cos 1, sin 0). */
API void orc_mmdit_rope_tables(int rows, int cols, int text_rows, float* cos_out, float* sin_out) {
    double freq[64];
    axis_frequencies(freq);
    int row_start = rows - rows / 2, col_start = cols - cols / 2;
    for (int i = 0; i < rows; i++)
        for (int j = 0; j < cols; j++) fill_rope(cos_out, sin_out, i * cols + j, 0, i - row_start, j - col_start, freq);
    for (int p = 0; p < text_rows; p++)
        for (int k = 0; k < 64; k++) {
            cos_out[(size_t)(rows * cols + p) * 64 + k] = 1.0f;
            sin_out[(size_t)(rows * cols + p) * 64 + k] = 0.0f;
        }
}

/* ---- Anima inputs (Models/Anima) ------------------------------------------- */

/* AnimaDit.RopeTables, AnimaDit.cs:149-188: per patch (i, j) of a rows x cols
 * grid (row-major tokens), head_dim / 2 pairs: the first (head_dim - 2s) / 2
 * temporal pairs still (a single frame), then s / 2 pairs turning with the
 * row and s / 2 with the column, s = head_dim / 6 * 2, at frequencies
 * 1 / theta^(2k / s) with theta = 10000 * 4^(s / (s - 2)) (the NTK factor),
 * all in fp32. [tokens, head_dim / 2]. */
API void orc_anima_rope_tables(int rows, int cols, int head_dim, float* cos_out, float* sin_out) {
    int spatial = head_dim / 6 * 2, temporal = head_dim - 2 * spatial, pairs = head_dim / 2;
    double ntk = pow(4.0, spatial / (double)(spatial - 2));
    float theta = (float)(10000.0 * ntk);
    float freq[64];
    for (int k = 0; k < spatial / 2; k++) freq[k] = 1.0f / powf(theta, 2.0f * k / spatial);
    for (int i = 0; i < rows; i++)
        for (int j = 0; j < cols; j++) {
            size_t off = (size_t)(i * cols + j) * pairs;
            for (int d = 0; d < temporal / 2; d++) {
                cos_out[off + d] = 1.0f;
                sin_out[off + d] = 0.0f;
            }
            for (int k = 0; k < spatial / 2; k++) {
                float ra = i * freq[k], ca = j * freq[k];
                cos_out[off + temporal / 2 + k] = cosf(ra);
                sin_out[off + temporal / 2 + k] = sinf(ra);
                cos_out[off + temporal / 2 + spatial / 2 + k] = cosf(ca);
                sin_out[off + temporal / 2 + spatial / 2 + k] = sinf(ca);
            }
        }
}

/* QwenImageConditioning.CausalTable, QwenImageConditioner.cs:69-80: row i
 * reads keys 0..min(i, real - 1). */
API void orc_causal_table(int real, int rows, int32_t* out) {
    for (int i = 0; i < rows; i++)
        for (int j = 0; j < rows; j++) out[(size_t)i * rows + j] = (j <= i && j < real) ? 1 : 0;
}

/* ---- the MMDiT dual-stream block ----------------------------------------- */

/* One stream's weights, all widened to fp32, torch [out, in] order. */
typedef struct {
    const float *w_mod, *b_mod;   /* [6D, T], [6D]  (shift1, scale1, gate1, shift2, scale2, gate2) */
    const float *w_qkv, *b_qkv;   /* [3D, D], [3D]  (q | k | v) */
    const float *norm_q, *norm_k; /* [d], [d] */
    const float *w_o, *b_o;       /* [D, D], [D] */
    const float *w_fc1, *b_fc1;   /* [F, D], [F] */
    const float *w_fc2, *b_fc2;   /* [D, F], [F] */
} orc_stream;

/* The dual-stream joint block composed from the reference's primitives
 * (Layers.Linear, Transformer.Modulate, Transformer.HeadNorm,
 * Transformer.Rotate, Layers.Attend over the joined sequence, GELU-tanh and
 * the gated residuals of QwenImageDit.cs:411-428): for each stream s,
 * (sh1, sc1, g1, sh2, sc2, g2) = Linear(SiLU(temb), W_mod); h = Modulate(x,
 * sh1, sc1); q, k, v = Linear(h); q, k = HeadNorm; then over the image-first
 * joined sequence RoPE and attention (key_len < 0: no mask); then per stream
 * x += g1 * Linear(a, W_o) and x += g2 * Linear(GELU_tanh(Linear(Modulate(x,
 * sh2, sc2), W_fc1)), W_fc2). x_img [n_img, D] and x_txt [n_txt, D] are
 * updated in place. temb is [T]; cos/sin are [n_img + n_txt, d/2]. */
API void orc_mmdit_block(float* x_img, int n_img, float* x_txt, int n_txt, const float* temb, int temb_dim, int D,
                         int heads, int F, const orc_stream* img, const orc_stream* txt, const float* cos_t,
                         const float* sin_t, int key_len, float eps) {
    const int N = n_img + n_txt, d = D / heads;
    float* st = (float*)malloc(sizeof(float) * temb_dim);
    memcpy(st, temb, sizeof(float) * temb_dim);
    orc_silu(st, temb_dim);
    float* mod[2];
    const orc_stream* w[2] = {img, txt};
    float* x[2] = {x_img, x_txt};
    int n[2] = {n_img, n_txt};
    int off[2] = {0, n_img};
    float* q = (float*)malloc(sizeof(float) * (size_t)N * D);
    float* k = (float*)malloc(sizeof(float) * (size_t)N * D);
    float* v = (float*)malloc(sizeof(float) * (size_t)N * D);
    float* a = (float*)malloc(sizeof(float) * (size_t)N * D);
    size_t maxn = (size_t)(n_img > n_txt ? n_img : n_txt);
    float* h = (float*)malloc(sizeof(float) * maxn * D);
    float* qkv = (float*)malloc(sizeof(float) * maxn * 3 * D);
    float* f = (float*)malloc(sizeof(float) * maxn * F);
    float* o = (float*)malloc(sizeof(float) * maxn * D);
    for (int s = 0; s < 2; s++) {
        mod[s] = (float*)malloc(sizeof(float) * 6 * D);
        orc_linear(st, 1, temb_dim, w[s]->w_mod, w[s]->b_mod, mod[s], 6 * D);
        orc_modulate(x[s], n[s], D, mod[s] + 0 * D, mod[s] + 1 * D, eps, h);
        orc_linear(h, n[s], D, w[s]->w_qkv, w[s]->b_qkv, qkv, 3 * D);
        for (int r = 0; r < n[s]; r++) {
            memcpy(q + (size_t)(off[s] + r) * D, qkv + (size_t)r * 3 * D, sizeof(float) * D);
            memcpy(k + (size_t)(off[s] + r) * D, qkv + (size_t)r * 3 * D + D, sizeof(float) * D);
            memcpy(v + (size_t)(off[s] + r) * D, qkv + (size_t)r * 3 * D + 2 * D, sizeof(float) * D);
        }
        orc_rms_norm(q + (size_t)off[s] * D, n[s] * heads, d, w[s]->norm_q, q + (size_t)off[s] * D, eps);
        orc_rms_norm(k + (size_t)off[s] * D, n[s] * heads, d, w[s]->norm_k, k + (size_t)off[s] * D, eps);
    }
    orc_rope(q, N, heads, d, cos_t, sin_t);
    orc_rope(k, N, heads, d, cos_t, sin_t);
    orc_mha(q, k, v, 1, N, N, heads, d, 1.0f / sqrtf((float)d), key_len >= 0 ? 1 : 0, key_len, NULL, 0, 0, 0, 0,
            a);
    for (int s = 0; s < 2; s++) {
        const float* g1 = mod[s] + 2 * D;
        const float* g2 = mod[s] + 5 * D;
        orc_linear(a + (size_t)off[s] * D, n[s], D, w[s]->w_o, w[s]->b_o, o, D);
        for (size_t i = 0; i < (size_t)n[s] * D; i++) x[s][i] += g1[i % D] * o[i];
        orc_modulate(x[s], n[s], D, mod[s] + 3 * D, mod[s] + 4 * D, eps, h);
        orc_linear(h, n[s], D, w[s]->w_fc1, w[s]->b_fc1, f, F);
        orc_gelu_tanh(f, (int64_t)n[s] * F);
        orc_linear(f, n[s], F, w[s]->w_fc2, w[s]->b_fc2, o, D);
        for (size_t i = 0; i < (size_t)n[s] * D; i++) x[s][i] += g2[i % D] * o[i];
        free(mod[s]);
    }
    free(st);
    free(q);
    free(k);
    free(v);
    free(a);
    free(h);
    free(qkv);
    free(f);
    free(o);
}

/* LoraMerge.Merge (Weights/LoraFile.cs:362-420), one pair: rows holds the
 * weight widened to float32 ([n_rows, cols]) and is updated in place. For
 * each covered row (first .. first + count) and each rank r in order, the
 * factor scale * up[row - first, r] is formed in float32, skipped when it is
 * zero, and down[r, :] * factor is added to the row, the product and the sum
 * each rounded (TensorPrimitives.MultiplyAdd, not fused). Several pairs are
 * applied by calling this once per pair in order: every element sees the
 * same sequence of operations as in the reference's row loop. */
API void orc_lora_merge(float* rows, int64_t n_rows, int64_t cols, const float* down, const float* up, int rank,
                        float scale, int64_t first, int64_t count) {
    for (int64_t row = first; row < first + count && row < n_rows; row++) {
        float* acc = rows + (size_t)row * cols;
        for (int r = 0; r < rank; r++) {
            const float factor = scale * up[(size_t)(row - first) * rank + r];
            if (factor == 0.0f) continue;
            const float* d = down + (size_t)r * cols;
            for (int64_t c = 0; c < cols; c++) {
                const float term = d[c] * factor;
                acc[c] = term + acc[c];
            }
        }
    }
}
