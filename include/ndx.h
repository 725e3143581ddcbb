/*
 * ndx.h — C ABI of the MI355X denoiser backend (libndx.so).
 *
 * The library stands where NaiveDiffusion's DirectML layer stands: a device,
 * device tensors, an expression graph of layer operators, a compiled model
 * that is initialised once with owned weights and then dispatched. Every
 * argument is blittable (integers, floats, plain pointers, opaque handles),
 * so a C# [LibraryImport] or a Python ctypes binding needs no marshalling.
 *
 * Each entry point cites the reference member it replaces (paths relative to
 * the reference repository root, src/NaiveDiffusion/...).
 *
 * Conventions
 *  - Every call returns an ndx_status; on failure ndx_last_error() holds a
 *    thread-local UTF-8 sentence saying why.
 *  - Shapes are int64 extents, rank 1..4, outermost first (the graphs use
 *    [batch, 1, tokens, features] and NCHW). Strides are in elements; a
 *    stride of 0 repeats an axis (a broadcast), as DmlTensorDesc allows.
 *  - Element types use the HostDataType ordinals (Tensors/HostTensor.cs:8-18).
 *  - Everything is synchronous unless the name says _async, as the reference
 *    device is (Dml/DmlDevice.cs:9-14): a call that launches GPU work has
 *    finished it on return.
 *  - A device is not thread-safe; use one thread per device.
 */
#ifndef NDX_H
#define NDX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NDX_API __attribute__((visibility("default")))

typedef int32_t ndx_status;
enum {
    NDX_OK = 0,
    NDX_INVALID_ARG = 1,   /* ArgumentException: shape, dtype or argument error */
    NDX_INVALID_STATE = 2, /* InvalidOperationException: wrong call order */
    NDX_OOM = 3,           /* OutOfVideoMemoryException: device stays usable */
    NDX_DEVICE_LOST = 4,   /* DeviceRemovedException: the device is unusable */
    NDX_UNSUPPORTED = 5    /* a combination this backend does not implement */
};

/* Element types: the HostDataType ordinals (Tensors/HostTensor.cs:8-18). */
enum {
    NDX_F32 = 0,
    NDX_F16 = 1,
    NDX_BF16 = 2,
    NDX_U32 = 3,
    NDX_I32 = 4,
    NDX_U16 = 5,
    NDX_I64 = 6,
    NDX_I8 = 7
};

typedef struct ndx_device ndx_device;
typedef struct ndx_tensor ndx_tensor;
typedef struct ndx_graph ndx_graph;
typedef struct ndx_model ndx_model;
typedef struct ndx_safetensors ndx_safetensors;

/* A value (expression) inside one graph; NDX_NONE marks an absent optional
 * operand (the nulls of DmlGraph.Emit, Dml/DmlGraph.cs:38-53). */
typedef int32_t ndx_value;
#define NDX_NONE (-1)

/* ---- errors / version --------------------------------------------------- */
NDX_API const char* ndx_last_error(void);
NDX_API const char* ndx_version(void);

/* ---- device (Dml/DmlDevice.cs) ------------------------------------------- */
/* EnumerateAdapters, Dml/DmlDevice.cs:207-225: how many GPUs are visible. */
NDX_API ndx_status ndx_device_count(int32_t* count);
/* new DmlDevice(useDebugLayer, adapterIndex), Dml/DmlDevice.cs:232. adapter -1 = first. */
NDX_API ndx_status ndx_device_create(int32_t adapter, ndx_device** out);
/* DmlDevice.Dispose, Dml/DmlDevice.cs:965. */
NDX_API ndx_status ndx_device_destroy(ndx_device* device);
/* AdapterName, Dml/DmlDevice.cs:56. Writes a NUL-terminated name. */
NDX_API ndx_status ndx_device_name(ndx_device* device, char* buffer, int32_t capacity);
/* VideoMemory(), Dml/DmlDevice.cs:91-99: bytes in use and the device total. */
NDX_API ndx_status ndx_device_memory(ndx_device* device, uint64_t* used, uint64_t* budget);
/* ReleasePooledBuffers / TrimBuffers, Dml/DmlDevice.cs:722-727. */
NDX_API ndx_status ndx_device_release_pooled(ndx_device* device);
/* Waits for everything queued on the device (ExecuteAndWait's fence,
 * Dml/DmlDevice.cs:940-946). */
NDX_API ndx_status ndx_device_synchronize(ndx_device* device);
/* Test hook with no reference counterpart: force the next failure from the
 * host. kind 0 clears, 1 = the next device allocation reports NDX_OOM,
 * 2 = the device reports itself lost from now on. */
NDX_API ndx_status ndx_device_set_fault_injection(ndx_device* device, int32_t kind);

/* ---- device tensors (Dml/DeviceTensor.cs; DmlDevice.Upload/Download) ----- */
/* DmlDevice.Upload, Dml/DmlDevice.cs:657-689: the host bytes are copied and
 * borrowed for the call only. */
NDX_API ndx_status ndx_tensor_upload(ndx_device* device, int32_t dtype, const int64_t* shape,
                                     int32_t rank, const void* data, uint64_t bytes,
                                     ndx_tensor** out);
/* An uninitialised packed tensor (no reference counterpart: a destination for
 * ndx_model_run_into and the synthetic fills). */
NDX_API ndx_status ndx_tensor_empty(ndx_device* device, int32_t dtype, const int64_t* shape,
                                    int32_t rank, ndx_tensor** out);
/* DmlDevice.Download, Dml/DmlDevice.cs:693-714. bytes must equal the size. */
NDX_API ndx_status ndx_tensor_download(ndx_tensor* tensor, void* data, uint64_t bytes);
/* DeviceTensor.Dispose, Dml/DeviceTensor.cs:44-52: back to the device pool. */
NDX_API ndx_status ndx_tensor_release(ndx_tensor* tensor);
/* DeviceTensor.Shape / DataType, Dml/DeviceTensor.cs:33-39. shape holds 4. */
NDX_API ndx_status ndx_tensor_info(ndx_tensor* tensor, int32_t* dtype, int64_t* shape,
                                   int32_t* rank);
/* Synthetic data with no reference counterpart: fills a float tensor with
 * mean + std * N(0,1) from the library's counter-based generator (splitmix64
 * of seed and element index, Box-Muller in double), rounded to the tensor's
 * type. The host generator in naivediffusion_amd.rng gives the same values. */
NDX_API ndx_status ndx_tensor_fill_normal(ndx_tensor* tensor, uint64_t seed, float mean,
                                          float std_dev);

/* ---- int8 block quantiser (Tensors/BlockQuantizer.cs:34-101) ------------- */
/* Fits, BlockQuantizer.cs:24-25: whether [rows, elements/rows] tiles into blocks. */
NDX_API int32_t ndx_quantize_fits(int64_t elements, int32_t rows, int32_t block);
/* Quantize, BlockQuantizer.cs:34-80, on the host: w is [rows, cols] of
 * F32/F16/BF16; per row and per block of `block` columns the scale is
 * (scale_dtype)(max|w| / 127) and q = clamp(rne(w * (1 / scale)), -127, 127),
 * an all-zero block where the stored scale is 0. scale_dtype F16 with block 32
 * is the reference's format; F32 with block = cols is per-output-channel. */
NDX_API ndx_status ndx_quantize_block_int8(const void* w, int32_t dtype, int64_t rows,
                                           int64_t cols, int32_t block, int32_t scale_dtype,
                                           int8_t* q, void* scales);
/* The same quantiser on the device, bit-identical to the host one: w is a
 * device tensor [rows, cols]; q ([rows, cols] I8) and scales ([rows,
 * cols/block] of scale_dtype) must already exist. */
NDX_API ndx_status ndx_quantize_block_int8_device(ndx_tensor* w, int32_t block,
                                                  int32_t scale_dtype, ndx_tensor* q,
                                                  ndx_tensor* scales);

/* ---- graph construction (Dml/DmlGraph.cs, Graph/ModelBuilder.cs) --------- */
/* new ModelBuilder(device, dataType, int8Weights), Graph/ModelBuilder.cs:20-26.
 * device may be NULL: the graph then only infers shapes and cannot compile. */
NDX_API ndx_status ndx_graph_create(ndx_device* device, int32_t dtype, int32_t int8_weights,
                                    ndx_graph** out);
NDX_API ndx_status ndx_graph_destroy(ndx_graph* graph);
/* No counterpart in the reference (DirectML schedules a graph itself): the
 * stream that operations emitted from now on run on, 0 (the device's, the
 * default) or 1 (a second stream of the same default priority). Independent
 * chains on the two streams run concurrently; the compiled model waits
 * across streams where one reads what the other wrote or reuses its memory,
 * and a run ends with both streams joined on the device stream. */
NDX_API ndx_status ndx_graph_set_stream(ndx_graph* graph, int32_t stream);
/* ModelBuilder.Placeholder, Graph/ModelBuilder.cs:93-98 (DmlGraph.Input,
 * owned false): bound by position at run time. */
NDX_API ndx_status ndx_graph_input(ndx_graph* graph, int32_t dtype, const int64_t* shape,
                                   int32_t rank, ndx_value* out);
/* ModelBuilder.Constant, Graph/ModelBuilder.cs:45-57: host data of host_dtype
 * converted to dtype (F32/F16/BF16 widen or round to nearest even) and owned
 * by the graph on the device from here on; the host buffer is not kept. */
NDX_API ndx_status ndx_graph_constant(ndx_graph* graph, int32_t dtype, const int64_t* shape,
                                      int32_t rank, const void* data, int32_t host_dtype,
                                      ndx_value* out);
/* A constant whose data is already on the device (no reference counterpart:
 * synthetic weights made on the GPU). The graph takes the tensor over; the
 * caller must not release it. */
NDX_API ndx_status ndx_graph_constant_device(ndx_graph* graph, ndx_tensor* tensor,
                                             ndx_value* out);
/* ModelBuilder.Weight, Graph/ModelBuilder.cs:65-88: a weight matrix of
 * `rows` output rows. Under int8_weights, with at least 2^16 elements and
 * whole blocks per row, it is block-quantised (32 columns, fp16 scales) and
 * dequantised inside the consuming GEMM; otherwise it is a constant at the
 * graph's dtype. */
NDX_API ndx_status ndx_graph_weight(ndx_graph* graph, const int64_t* shape, int32_t rank,
                                    const void* data, int32_t host_dtype, int32_t rows,
                                    ndx_value* out);
/* ModelBuilder.Weight for a weight already on the device (bf16/f16/f32);
 * quantised on the device under int8_weights. Takes the tensor over. */
NDX_API ndx_status ndx_graph_weight_device(ndx_graph* graph, ndx_tensor* tensor, int32_t rows,
                                           ndx_value* out);
/* A pre-quantised weight: q [rows, cols] I8 and scales [rows, cols/block]
 * (F16 or F32) on the device, both taken over. */
NDX_API ndx_status ndx_graph_weight_int8(ndx_graph* graph, ndx_tensor* q, ndx_tensor* scales,
                                         int32_t block, ndx_value* out);
/* DmlExpression.Shape / Desc.DataType. shape holds 4. */
NDX_API ndx_status ndx_value_info(ndx_graph* graph, ndx_value value, int32_t* dtype,
                                  int64_t* shape, int32_t* rank);

/* ---- operators (Dml/DmlOps.cs, Graph/Layers.cs, Graph/Transformer.cs) ---- */
/* DmlOps.Reinterpret, Dml/DmlOps.cs:190-200: a view, no kernel. strides may
 * be NULL for packed; 0 repeats an axis. */
NDX_API ndx_status ndx_op_reinterpret(ndx_graph* graph, ndx_value x, const int64_t* shape,
                                      int32_t rank, const int64_t* strides, ndx_value* out);
/* DmlOps.Slice, Dml/DmlOps.cs:348-364 (positive strides). A view. */
NDX_API ndx_status ndx_op_slice(ndx_graph* graph, ndx_value x, const int64_t* offsets,
                                const int64_t* sizes, const int64_t* strides, ndx_value* out);
/* DmlOps.Join, Dml/DmlOps.cs:366-380. */
NDX_API ndx_status ndx_op_join(ndx_graph* graph, const ndx_value* xs, int32_t count,
                               int32_t axis, ndx_value* out);
/* DmlOps.Cast, Dml/DmlOps.cs:85-97 (float widths round to nearest even). */
NDX_API ndx_status ndx_op_cast(ndx_graph* graph, ndx_value x, int32_t dtype, ndx_value* out);

enum {
    NDX_UNARY_IDENTITY = 0, /* DmlOps.ActivationIdentity :165-173 (a packed copy) */
    NDX_UNARY_SIGMOID = 1,  /* :121-129 */
    NDX_UNARY_SILU = 2,     /* ActivationSwish :133-142 */
    NDX_UNARY_GELU = 3,     /* ActivationGelu :145-153, exact erf */
    NDX_UNARY_TANH = 4,     /* :155-163 */
    NDX_UNARY_GELU_TANH = 5 /* x*sigmoid(2*0.7978845608*(x+0.044715x^3)),
                               Models/QwenImage/QwenImageDit.cs:510-515 */
};
NDX_API ndx_status ndx_op_unary(ndx_graph* graph, ndx_value x, int32_t kind, ndx_value* out);
/* DmlOps.Identity, Dml/DmlOps.cs:59-68: x * scale + bias (the scalar operators
 * of DmlExpression.cs:44-51). */
NDX_API ndx_status ndx_op_scale_bias(ndx_graph* graph, ndx_value x, float scale, float bias,
                                     ndx_value* out);
enum { NDX_BINARY_ADD = 0, NDX_BINARY_SUB = 1, NDX_BINARY_MUL = 2, NDX_BINARY_DIV = 3 };
/* DmlOps.Add/Subtract/Multiply/Divide, Dml/DmlOps.cs:41-55: same shape and
 * dtype (broadcast through stride-0 views). */
NDX_API ndx_status ndx_op_binary(ndx_graph* graph, ndx_value a, ndx_value b, int32_t kind,
                                 ndx_value* out);

/* Epilogues fused into the linear layer's GEMM. */
enum {
    NDX_EPI_NONE = 0,
    NDX_EPI_GELU_TANH = 1,      /* QwenImageDit.cs:510-515 on the product */
    NDX_EPI_GELU = 2,           /* exact GELU on the product */
    NDX_EPI_SILU = 3,           /* SiLU on the product */
    NDX_EPI_GATED_RESIDUAL = 4, /* out = aux1 + aux0 * Cast(product, aux1.dtype):
                                   the gated residual of QwenImageDit.cs:421,425 and
                                   Models/Anima/AnimaDit.cs:344,349,355; aux0 is a
                                   [.., 1, N] gate broadcast over rows or a
                                   [.., M, N] gate per row (a join of two row
                                   broadcasts, QwenImageDit.cs:307-315, is read
                                   in place), aux1 the residual [.., M, N]; out
                                   takes aux1's dtype */
    NDX_EPI_RESIDUAL = 5,       /* out = aux1 + Cast(product, aux1.dtype) */
    NDX_EPI_SWIGLU = 6          /* SwiGLU, Models/QwenImage/QwenImageDit.cs:390-406:
                                   W's rows interleave the gate and up projections
                                   (row 2j gate j, row 2j+1 up j); out[j] =
                                   SiLU(gate_j) * up_j with gate, up and the SiLU
                                   rounded to x's dtype as the reference's separate
                                   operators are; out has N/2 columns */
};
/* Layers.Linear, Graph/Layers.cs:131-160 (DmlOps.Gemm with transB,
 * Dml/DmlOps.cs:231-262): y = x[.., M, K] * W[N, K]^T (+ bias[N]) then the
 * epilogue. W is a value from an ndx_graph_weight call or a constant; bias may be NONE.
 * The product is computed at x's dtype (F32, BF16 or F16) with fp32
 * accumulation; a narrower weight is widened inside the kernel. */
NDX_API ndx_status ndx_op_linear(ndx_graph* graph, ndx_value x, ndx_value w, ndx_value bias,
                                 int32_t epilogue, ndx_value aux0, ndx_value aux1,
                                 ndx_value* out);
/* DmlOps.Gemm, Dml/DmlOps.cs:231-262: alpha * op(a) * op(b) + beta * c over
 * the two leading (batch) axes; c may be NONE. */
NDX_API ndx_status ndx_op_gemm(ndx_graph* graph, ndx_value a, ndx_value b, ndx_value c,
                               int32_t trans_a, int32_t trans_b, float alpha, float beta,
                               ndx_value* out);

enum { NDX_MASK_NONE = 0, NDX_MASK_KEY_LENGTH = 1, NDX_MASK_BOOLEAN = 2 };
/* Layers.Attend, Graph/Layers.cs:260-279 -> DmlOps.MultiheadAttention,
 * Dml/DmlOps.cs:480-520: softmax(Q_h K_h^T * scale + mask) V_h per head over
 * packed [B, 1, T, H*d] tensors. A masked score has -10000 added (:483). The
 * key-length mask is an I32 [1,1,1,1] count of real leading keys; the boolean
 * mask an I32 [B or 1, H or 1, T, S] table (1 = may read). */
NDX_API ndx_status ndx_op_attention(ndx_graph* graph, ndx_value q, ndx_value k, ndx_value v,
                                    int32_t heads, float scale, int32_t mask_kind,
                                    ndx_value mask, ndx_value* out);
/* Transformer.HeadNorm then Transformer.Rotate, Graph/Transformer.cs:37-64:
 * per-head RMSNorm of x [B, 1, T, H*d] (weight [d] or NONE), rounded to x's
 * dtype, then (if cos is given) the rotate-half RoPE in fp32 with [1, T, 1,
 * d/2] tables, cast to out_dtype. */
NDX_API ndx_status ndx_op_head_norm_rotate(ndx_graph* graph, ndx_value x, ndx_value weight,
                                           float eps, ndx_value cos, ndx_value sin,
                                           int32_t heads, int32_t out_dtype, ndx_value* out);
/* DmlOps.ActivationSoftmax over the last axis (Dml/DmlOps.cs:175-184) of
 * scale * x, at x's type; scale folds the alpha of the Gemm that made x
 * (AutoencoderKl.AttentionBlock, Vae/AutoencoderKl.cs:57-60). */
NDX_API ndx_status ndx_op_softmax(ndx_graph* graph, ndx_value x, float scale, ndx_value* out);
/* Layers.LayerNorm(x, eps) and the affine form, Graph/Layers.cs:189-197,
 * 225-226 (MVN1 over the last axis, Dml/DmlOps.cs:305-319). */
NDX_API ndx_status ndx_op_layer_norm(ndx_graph* graph, ndx_value x, ndx_value weight,
                                     ndx_value bias, float eps, ndx_value* out);
/* Transformer.Modulate, Graph/Transformer.cs:72-80:
 * Cast(LayerNorm(x) * (1 + scale) + shift, out_dtype); shift may be NONE;
 * scale and shift are [.., 1, D] rows broadcast over tokens, or [.., T, D]
 * per token (a join of two row broadcasts, the image and text rows of
 * QwenImageDit.cs:307-315, is read in place without being materialised). */
NDX_API ndx_status ndx_op_modulate(ndx_graph* graph, ndx_value x, ndx_value shift,
                                   ndx_value scale, float eps, int32_t out_dtype,
                                   ndx_value* out);
/* Layers.RmsNorm, Graph/Layers.cs:209-221 (MVN2 without the mean): over the
 * last axis, weight [D] or NONE. */
NDX_API ndx_status ndx_op_rms_norm(ndx_graph* graph, ndx_value x, ndx_value weight, float eps,
                                   ndx_value* out);
/* Layers.GroupNorm, Graph/Layers.cs:166-185, over NCHW with a per-channel
 * affine, optionally followed by SiLU (ResnetBlock, Models/Sdxl/UNetModel.cs:230-254). */
NDX_API ndx_status ndx_op_group_norm(ndx_graph* graph, ndx_value x, ndx_value weight,
                                     ndx_value bias, int32_t groups, float eps, int32_t silu,
                                     ndx_value* out);
/* Layers.Conv2d, Graph/Layers.cs:115-127 -> DmlOps.Convolution,
 * Dml/DmlOps.cs:265-299: NCHW cross-correlation, filters [Cout, Cin, kh, kw]
 * (a value from ndx_graph_weight*), bias [Cout] or NONE. residual (NONE or
 * [N, Cout, Ho, Wo]) is added to the output. */
NDX_API ndx_status ndx_op_conv2d(ndx_graph* graph, ndx_value x, ndx_value w, ndx_value bias,
                                 int32_t stride, int32_t pad_start, int32_t pad_end,
                                 ndx_value residual, ndx_value* out);
/* Layers.UpsampleNearest, Graph/Layers.cs:234-235 (DmlOps.Upsample2D). */
NDX_API ndx_status ndx_op_upsample_nearest(ndx_graph* graph, ndx_value x, int32_t scale,
                                           ndx_value* out);
/* The patch layouts of the DiTs' embed and unembed, on the device:
 * [B, C, H, W] -> [B, 1, (H/p)(W/p), C*p*p] and back. Feature order
 * NDX_PATCH_CHANNEL_FIRST is (c, dy, dx): AnimaDit.Patchify (Models/Anima/
 * AnimaDit.cs:193-219) and the MMDiT's 2x2 embed; NDX_PATCH_CHANNEL_LAST is
 * (dy, dx, c): AnimaDit.Unpatchify (:223-247). */
#define NDX_PATCH_CHANNEL_FIRST 0
#define NDX_PATCH_CHANNEL_LAST 1
NDX_API ndx_status ndx_op_patchify(ndx_graph* graph, ndx_value x, int32_t patch, int32_t order,
                                   ndx_value* out);
NDX_API ndx_status ndx_op_unpatchify(ndx_graph* graph, ndx_value x, int32_t patch,
                                     int32_t channels, int32_t height, int32_t width,
                                     int32_t order, ndx_value* out);

/* The sampler's step on the device, so the latent never leaves it (the
 * reference downloads it every step, Pipeline/GenerationPipeline.cs:578-616):
 * classifier-free guidance p = uncond + g * (cond - uncond)
 * (Pipeline/GuidanceStrategy.cs:34-44; p = cond when uncond is NONE), then
 * the Euler step x + p * (sigma_next - sigma) (Sampling/Schedulers.cs:270-279)
 * with the flow prediction's derivative, the model output itself
 * (Sampling/Prediction.cs:83-84). x, uncond, cond: F32 of one shape;
 * scalars: F32 [>= 3] holding (g, sigma, sigma_next), read on the device so a
 * new step binds new values without a new graph. Each float operation is
 * rounded on its own, as the reference's loops are: bit-exact with them. */
NDX_API ndx_status ndx_op_guided_euler_step(ndx_graph* graph, ndx_value x, ndx_value uncond, ndx_value cond,
                                            ndx_value scalars, ndx_value* out);

/* ---- compile / run (Dml/DmlCompiledModel.cs, ModelBuilder.Compile/Run) --- */
/* DmlGraph.Compile + DmlCompiledModel.Initialize, Dml/DmlGraph.cs:58-163,
 * Dml/DmlCompiledModel.cs:66-75: schedule, plan the intermediates into one
 * arena, keep the owned weights. An input or constant cannot be an output
 * (Dml/DmlGraph.cs:108-112). The graph may be destroyed afterwards. */
NDX_API ndx_status ndx_graph_compile(ndx_graph* graph, const ndx_value* outputs, int32_t count,
                                     ndx_model** out);
/* PersistentSize / TemporarySize, Dml/DmlCompiledModel.cs:58-61. */
NDX_API ndx_status ndx_model_sizes(ndx_model* model, uint64_t* persistent, uint64_t* temporary);
NDX_API ndx_status ndx_model_counts(ndx_model* model, int32_t* inputs, int32_t* outputs,
                                    int32_t* kernels);
/* ModelBuilder.RunOnDevice / DmlCompiledModel.DispatchOnDevice,
 * Graph/ModelBuilder.cs:158-175, Dml/DmlCompiledModel.cs:96-142: inputs bound
 * to the placeholders in order; the outputs are new tensors the caller owns. */
NDX_API ndx_status ndx_model_run(ndx_model* model, ndx_tensor* const* inputs, int32_t n_inputs,
                                 ndx_tensor** outputs, int32_t n_outputs);
/* The same into caller-owned output tensors of the right shape, queued on the
 * device's stream without waiting (ndx_device_synchronize waits). */
NDX_API ndx_status ndx_model_run_into_async(ndx_model* model, ndx_tensor* const* inputs,
                                            int32_t n_inputs, ndx_tensor* const* outputs,
                                            int32_t n_outputs);
/* No counterpart in the reference: ndx_model_run_into_async for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc). The model's temporary memory (every
 * intermediate and the kernels' scratch: attention key-split partials,
 * GroupNorm split statistics) lives in a static array the library holds on
 * each GPU until the process ends, 64 MiB (NDX_STATIC_SCRATCH_BYTES), instead
 * of the model's own arena; the call allocates nothing and records no timing
 * events. A model whose temporary size (ndx_model_sizes) exceeds the array
 * is refused with NDX_INVALID_ARG. Every static run on a GPU shares that
 * GPU's array: runs queued on one device handle are ordered by its stream,
 * but runs that overlap on one GPU (two device handles, or other streams)
 * race. */
#define NDX_STATIC_SCRATCH_BYTES (64ull << 20)
NDX_API ndx_status ndx_model_run_into_static_async(ndx_model* model, ndx_tensor* const* inputs,
                                                   int32_t n_inputs, ndx_tensor* const* outputs,
                                                   int32_t n_outputs);
/* GraphChain.Run (Graph/GraphChain.cs:218-282) dispatches one link after
 * another, each ended by a fence wait (Dml/DmlDevice.cs:908-957). With
 * replay enabled, ndx_model_run_into_async records the whole run (both
 * streams) as one HIP graph on its first call and replays it with a single
 * graph launch on later calls that bind the same input and output tensors
 * (other tensors record it again). Profiled runs are never replayed. Off by
 * default; disabling frees the recorded graph. */
NDX_API ndx_status ndx_model_set_graph_replay(ndx_model* model, int32_t enabled);
/* Kernel timing with no reference counterpart: while enabled, every kernel a
 * run launches is bracketed by HIP events on the device stream. */
NDX_API ndx_status ndx_model_set_profiling(ndx_model* model, int32_t enabled);
/* No counterpart in the reference either: with a family name (as the
 * profile entries name them), profiling brackets only that family's kernels
 * and waits for nothing until the entries are read, so a timed run carries
 * a few events instead of two per kernel and a wait per run. NULL or ""
 * returns to bracketing every kernel. */
NDX_API ndx_status ndx_model_set_profile_filter(ndx_model* model, const char* family);
/* Per kernel family since profiling was enabled: the family name, launches,
 * summed milliseconds and summed algorithmic flops and bytes. index runs
 * 0..families-1; returns NDX_INVALID_ARG past the end. */
NDX_API ndx_status ndx_model_profile_entry(ndx_model* model, int32_t index, char* name,
                                           int32_t capacity, int64_t* launches, double* ms,
                                           double* flops, double* bytes);
/* DmlCompiledModel.Dispose, Dml/DmlCompiledModel.cs:233. */
NDX_API ndx_status ndx_model_release(ndx_model* model);

/* ---- checkpoint files and LoRA folding ------------------------------------
 *
 * SafetensorsFile (Weights/SafetensorsFile.cs:22-259): the file is mapped
 * read-only and its header parsed and checked once, at open; every offset is
 * checked against the file before anything reads there. A refused file is
 * unmapped before open returns. Strings and mapped bytes handed out stay
 * valid until ndx_safetensors_close. */

/* The constructor (:35-66) and ReadHeader (:70-149). NDX_INVALID_ARG with the
 * reference's reasons: too short, a header that does not fit the file, JSON
 * that does not parse, JSON that is not a tensor table, an entry pointing
 * outside the file. */
NDX_API ndx_status ndx_safetensors_open(const char* path, ndx_safetensors** out);
/* Dispose (:198-214). NULL is allowed. */
NDX_API ndx_status ndx_safetensors_close(ndx_safetensors* file);
/* How many tensor entries and string-valued __metadata__ notes the header has. */
NDX_API ndx_status ndx_safetensors_count(ndx_safetensors* file, int32_t* entries, int32_t* metadata);
/* Keys and TryGetInfo (:151-169): entry index's name, dtype as written (which
 * may be one ndx_safetensors_read refuses), shape (up to 8 axes), rank and
 * byte length. Any output may be NULL. */
NDX_API ndx_status ndx_safetensors_entry(ndx_safetensors* file, int32_t index, const char** name,
                                         const char** dtype, int64_t* shape, int32_t* rank, uint64_t* bytes);
/* Metadata (:151-155): note index's key and value. */
NDX_API ndx_status ndx_safetensors_metadata(ndx_safetensors* file, int32_t index, const char** key,
                                            const char** value);
/* Read's window (:172-180): the mapped bytes of a tensor, no copy. */
NDX_API ndx_status ndx_safetensors_data(ndx_safetensors* file, const char* name, const void** data,
                                        uint64_t* bytes);
/* Read (:172-180) straight into device memory, narrowed on the way as
 * LazyWeights narrows (Weights/LazyWeights.cs:39-48, HostTensor.ConvertTo):
 * the bytes go from the mapping through pinned staging buffers to the device
 * and a float tensor is converted there to dtype (a float type; -1 keeps the
 * stored type), rounding to nearest even. A dtype IsSupportedDataType
 * (:229-240) refuses is NDX_UNSUPPORTED ("safetensors dtype X is not
 * supported"). More than 4 axes are folded into the first. Returns when the
 * tensor is on the device. */
NDX_API ndx_status ndx_safetensors_read(ndx_safetensors* file, const char* name, ndx_device* device,
                                        int32_t dtype, ndx_tensor** out);

/* One LoRA pair to fold: down is [rank, the weight's row length] (trailing
 * axes of a convolution flattened), up is [rows covered, rank], added from
 * row first_row on with factor scale (weight * alpha / rank,
 * Weights/LoraFile.cs:492). */
typedef struct ndx_lora_patch {
    const ndx_tensor* down;
    const ndx_tensor* up;
    float scale;
    int32_t first_row;
} ndx_lora_patch;
#define NDX_MAX_LORA_PATCHES 16
/* LoraMerge.Merge (Weights/LoraFile.cs:355-420) on the device: a new tensor
 * of the weight's shape, each row widened to float32, given
 * (scale * up[row, r]) * down[r, :] for every pair covering it (in order) and
 * every rank r in order, each product and sum rounded on its own, zero
 * factors skipped, then narrowed once to dtype (-1: the reference's width,
 * Float32 for a Float32 weight, else Float16). Up to NDX_MAX_LORA_PATCHES
 * pairs; the pairs' matrices may be any float type. */
NDX_API ndx_status ndx_lora_fold(const ndx_tensor* weight, const ndx_lora_patch* patches, int32_t count,
                                 int32_t dtype, ndx_tensor** out);

#ifdef __cplusplus
}
#endif

#endif /* NDX_H */
