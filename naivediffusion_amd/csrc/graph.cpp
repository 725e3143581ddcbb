// The expression graph, its compiler and its executor.
//
// Replaces Dml/DmlGraph.cs, Dml/DmlOps.cs (shape rules and argument checks),
// Dml/DmlCompiledModel.cs and the graph half of Graph/ModelBuilder.cs. A graph
// is a list of values (inputs, owned constants, node outputs and views onto
// any of them) and nodes in creation order, which is a valid schedule.
// Compiling drops what the outputs do not need, feeds a join straight into
// the attention that reads it (segments instead of a copy), packs views a
// kernel cannot read, and plans every intermediate into one arena by
// lifetime. Running binds the inputs, resolves pointers and launches one
// kernel per node on the device's stream.

#include <string.h>

#include <algorithm>
#include <functional>
#include <array>
#include <map>
#include <memory>
#include <sstream>

#include "runtime.h"

using namespace ndx;

namespace {

enum ValueKind { VK_INPUT, VK_CONST, VK_NODE, VK_VIEW };

struct ConstStore {
  std::vector<ndx_tensor*> tensors;
  // Convolution filters reordered to [Cout, kh, kw, Cin] for the implicit
  // GEMM, by original tensor; made once, at the first compile that needs it.
  std::map<const ndx_tensor*, ndx_tensor*> nhwc_filters;
  ~ConstStore() {
    for (auto* t : tensors) free_tensor(t);
  }
};

struct GValue {
  int dtype = NDX_F32;
  int rank = 4;
  View4 v{};            // 4-D sizes and strides (left-padded with 1)
  int64_t offset = 0;   // elements from the start of the base buffer
  int base = -1;        // the buffer-owning value
  int kind = VK_NODE;
  int producer = -1;
  int input_index = -1;
  ndx_tensor* data = nullptr;     // constants
  ndx_tensor* scales = nullptr;   // int8 weights
  int qblock = 0;
  bool quant = false;
  int64_t buffer_elems = 0;       // owners: elements in the buffer
};

enum OpKind {
  OP_ELEM, OP_JOIN, OP_LINEAR, OP_GEMM, OP_ATTN, OP_HNR, OP_ROWNORM, OP_GROUPNORM, OP_CONV,
  OP_UPSAMPLE, OP_PATCH, OP_SAMPLE, OP_SOFTMAX,
  OP_NHWC,  // compile-time only: an NCHW value copied to NHWC for the implicit-GEMM convolution
};

struct GNode {
  int op = OP_ELEM;
  std::vector<int> in;
  int out = -1;
  int i0 = 0, i1 = 0, i2 = 0, i3 = 0, i4 = 0, i5 = 0;
  float f0 = 0.f, f1 = 0.f;
  // attention segments (compile-time rewrite): per q/k/v up to two values
  int seg[3][2] = {{-1, -1}, {-1, -1}, {-1, -1}};
  // Two-row operands (compile-time rewrite of a join of two row broadcasts):
  // per operand slot, the first row from rows_split on is rows_off elements
  // past the one the operand's view starts at (0: not split).
  int64_t rows_split[5] = {0, 0, 0, 0, 0}, rows_off[5] = {0, 0, 0, 0, 0};
  // scratch in the arena, live only while this node runs
  int64_t scratch_bytes = 0, scratch_off = -1;
  // An implicit-GEMM convolution: the reordered filter's channels per tap
  // (a multiple of 64, zeros past the input's own), and whether the input is
  // read through a nearest 2x upsample (a fused UpsampleNearest).
  int64_t conv_cin_k = 0;
  int conv_up = 0;
  // A linear's tile fixed at compile time (1..4 as GemmArgs::tile_hint; 0:
  // the second stream's choice or the latency model's).
  int tile_hint = 0;
  // the stream (0 the device's, 1 the second) the node runs on
  int lane = 0;
  // profiling
  std::string family;
  double flops = 0, bytes = 0;
};

int64_t numel4(const View4& v) { return v.size[0] * v.size[1] * v.size[2] * v.size[3]; }

// The tile of a linear on the second stream. The latency model picks small
// tiles for a product of few rows (many short workgroups finish soonest on
// an idle GPU); beside the first stream's large products, though, what
// counts is how many CU-cycles the product takes from them, and 128x128
// tiles do the same work in about two thirds of the CU time of 64x64 ones
// (the MMDiT text stream: 2% less step time on MI355X; 256x256 tiles hold
// CUs so long that the other stream's rounds stall).
// NDX_SECOND_STREAM_TILE=1..5 (256x256, 128x128, 64x128, 64x64, the register-capped 64x64) pins it,
// read at compile time, for sweeps.
int second_stream_tile(const GNode& n, int64_t rows) {
  if (n.lane != 1 || rows < 128) return 0;
  if (const char* pin = getenv("NDX_SECOND_STREAM_TILE"); pin && pin[0] >= '1' && pin[0] <= '5' && !pin[1])
    return pin[0] - '0';
  return 2;
}

View4 packed4(const int64_t* size) {
  View4 v;
  for (int i = 0; i < 4; i++) v.size[i] = size[i];
  v.stride[3] = 1;
  for (int i = 2; i >= 0; i--) v.stride[i] = v.stride[i + 1] * v.size[i + 1];
  return v;
}

bool is_packed(const View4& v) {
  int64_t s = 1;
  for (int i = 3; i >= 0; i--) {
    if (v.size[i] != 1 && v.stride[i] != s) return false;
    s *= v.size[i];
  }
  return true;
}

std::string shape_str(const View4& v, int dtype) {
  std::ostringstream o;
  o << dtype_name(dtype) << " [" << v.size[0] << ", " << v.size[1] << ", " << v.size[2] << ", "
    << v.size[3] << "]";
  return o.str();
}

// Rows of a [b0, b1, R, C] view: C contiguous, rows ld apart, the (b0, b1)
// batch one uniform stride. Returns false when a kernel needs it packed.
bool rows_layout(const View4& v, int64_t& ld, int64_t& batch_stride) {
  if (v.size[3] > 1 && v.stride[3] != 1) return false;
  ld = v.size[2] > 1 ? v.stride[2] : v.size[3];
  if (ld < v.size[3] && v.size[2] > 1) return false;
  if (v.size[0] > 1 && v.size[1] > 1) {
    if (v.stride[0] != v.size[1] * v.stride[1]) return false;
    batch_stride = v.stride[1];
  } else if (v.size[0] > 1) {
    batch_stride = v.stride[0];
  } else if (v.size[1] > 1) {
    batch_stride = v.stride[1];
  } else {
    batch_stride = 0;
  }
  return true;
}

}  // namespace

struct ndx_graph {
  ndx_device* dev = nullptr;
  int dtype = NDX_F32;
  bool int8_weights = false;
  std::vector<GValue> values;
  std::vector<GNode> nodes;
  int n_inputs = 0;
  std::shared_ptr<ConstStore> consts = std::make_shared<ConstStore>();

  GValue& val(int id) {
    if (id < 0 || id >= (int)values.size()) fail(NDX_INVALID_ARG, "value " + std::to_string(id) + " is not in this graph");
    return values[id];
  }
  GValue* opt(int id) { return id == NDX_NONE ? nullptr : &val(id); }

  int add_value(GValue v) {
    values.push_back(v);
    return (int)values.size() - 1;
  }
  // A fresh packed value produced by a node.
  int node_output(int dtype, const int64_t* size4, int rank) {
    GValue v;
    v.dtype = dtype;
    v.rank = rank;
    v.v = packed4(size4);
    v.kind = VK_NODE;
    v.buffer_elems = numel4(v.v);
    int id = add_value(v);
    values[id].base = id;
    return id;
  }
  int lane = 0;  // ndx_graph_set_stream: the lane new nodes go to
  int emit(GNode n, int dtype, const int64_t* size4, int rank) {
    n.lane = lane;
    n.out = node_output(dtype, size4, rank);
    values[n.out].producer = (int)nodes.size();
    nodes.push_back(n);
    return n.out;
  }
};

struct ProfEntry {
  int64_t launches = 0;
  double ms = 0, flops = 0, bytes = 0;
};

struct ndx_model {
  ndx_device* dev = nullptr;
  std::vector<GValue> values;
  std::vector<GNode> nodes;
  std::vector<int> inputs;   // value ids by placeholder order
  std::vector<int> outputs;  // value ids
  std::vector<int64_t> arena_off;
  std::vector<int> out_slot;  // value id -> output index or -1
  void* arena = nullptr;
  size_t arena_alloc = 0, arena_bytes = 0;
  uint64_t persistent = 0;
  std::shared_ptr<ConstStore> consts;
  int kernels = 0;
  bool profiling = false;
  std::vector<hipEvent_t> events;
  // Filtered profiling (ndx_model_set_profile_filter): only nodes of one
  // kernel family are bracketed, from a pool of events that grows across
  // runs; nothing waits until the entries are read.
  std::string prof_filter;
  std::vector<std::string> node_family;  // per node, made when profiling starts
  std::vector<hipEvent_t> fevents;
  std::vector<int> prof_pending;  // node of each bracketed launch, in record order
  // Two lanes: per node, the latest node of each lane it must wait for (-1
  // none), the event a node records for others (-1 none), and the events.
  bool two_lanes = false;
  std::vector<std::array<int, 2>> waits;
  std::vector<int> signal;
  std::vector<hipEvent_t> lane_events;  // [signals..., start join, end join]
  std::map<std::string, ProfEntry> prof;
  // Graph replay (ndx_model_set_graph_replay): the run's launches captured
  // once as a HIP graph, for the pointers in graph_key (inputs, outputs,
  // arena); replayed while a run binds the same ones.
  bool replay = false;
  hipGraphExec_t graph_exec = nullptr;
  std::vector<void*> graph_key;
};

namespace {

void to4(const int64_t* shape, int rank, int64_t* out4) {
  check_shape(shape, rank);
  for (int i = 0; i < 4; i++) out4[i] = 1;
  for (int i = 0; i < rank; i++) out4[4 - rank + i] = shape[i];
}

void require_float(const GValue& v, const char* what) {
  if (!dtype_is_float(v.dtype)) fail(NDX_INVALID_ARG, std::string(what) + " must be a float tensor");
}

bool same_shape(const View4& a, const View4& b) {
  for (int i = 0; i < 4; i++)
    if (a.size[i] != b.size[i]) return false;
  return true;
}

// ---- elementwise shape + dtype helpers -------------------------------------

int make_elem(ndx_graph* g, int op, int a, int b, int out_dtype, float scale = 1.f, float bias = 0.f) {
  GValue& va = g->val(a);
  require_float(va, "an elementwise operand");
  if (b != NDX_NONE) {
    GValue& vb = g->val(b);
    if (!same_shape(va.v, vb.v))
      fail(NDX_INVALID_ARG, "elementwise operands differ in shape: " + shape_str(va.v, va.dtype) + " vs " + shape_str(vb.v, vb.dtype));
    if (va.dtype != vb.dtype)
      fail(NDX_INVALID_ARG, "elementwise operands differ in precision: " + shape_str(va.v, va.dtype) + " vs " + shape_str(vb.v, vb.dtype));
  }
  GNode n;
  n.op = OP_ELEM;
  n.in = {a, b};
  n.i0 = op;
  n.f0 = scale;
  n.f1 = bias;
  int rank = va.rank;
  int64_t size[4];
  for (int i = 0; i < 4; i++) size[i] = va.v.size[i];
  return g->emit(n, out_dtype, size, rank);
}

}  // namespace

extern "C" {

NDX_API ndx_status ndx_graph_create(ndx_device* device, int32_t dtype, int32_t int8_weights,
                                    ndx_graph** out) {
  NDX_TRY
  NEED(out);
  if (dtype != NDX_F32 && dtype != NDX_F16 && dtype != NDX_BF16)
    fail(NDX_INVALID_ARG, "a graph computes at Float32, Float16 or BFloat16");
  auto* g = new ndx_graph();
  g->dev = device;
  g->dtype = dtype;
  g->int8_weights = int8_weights != 0;
  *out = g;
  NDX_CATCH
}

NDX_API ndx_status ndx_graph_destroy(ndx_graph* graph) {
  NDX_TRY
  delete graph;
  NDX_CATCH
}

NDX_API ndx_status ndx_graph_set_stream(ndx_graph* g, int32_t stream) {
  NDX_TRY
  NEED(g);
  if (stream != 0 && stream != 1) fail(NDX_INVALID_ARG, "the stream is 0 or 1");
  g->lane = stream;
  NDX_CATCH
}

NDX_API ndx_status ndx_graph_input(ndx_graph* g, int32_t dtype, const int64_t* shape, int32_t rank,
                                   ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  if (dtype_size(dtype) == 0) fail(NDX_INVALID_ARG, "unknown element type");
  GValue v;
  int64_t s4[4];
  to4(shape, rank, s4);
  v.dtype = dtype;
  v.rank = rank;
  v.v = packed4(s4);
  v.kind = VK_INPUT;
  v.input_index = g->n_inputs++;
  v.buffer_elems = numel4(v.v);
  int id = g->add_value(v);
  g->values[id].base = id;
  *out = id;
  NDX_CATCH
}

static int add_const_value(ndx_graph* g, ndx_tensor* t, int dtype, const int64_t* s4, int rank) {
  GValue v;
  v.dtype = dtype;
  v.rank = rank;
  v.v = packed4(s4);
  v.kind = VK_CONST;
  v.data = t;
  v.buffer_elems = numel4(v.v);
  if (t) g->consts->tensors.push_back(t);
  int id = g->add_value(v);
  g->values[id].base = id;
  return id;
}

// Converts host floats of host_dtype to dtype on the host (round to nearest
// even), then uploads. Returns a new device tensor.
static ndx_tensor* upload_converted(ndx_device* dev, const void* data, int host_dtype, int dtype,
                                    const int64_t* s4) {
  int64_t n = s4[0] * s4[1] * s4[2] * s4[3];
  std::vector<char> buf;
  const void* src = data;
  if (host_dtype != dtype) {
    if (!dtype_is_float(host_dtype) || !dtype_is_float(dtype))
      fail(NDX_INVALID_ARG, std::string("cannot convert ") + dtype_name(host_dtype) + " to " + dtype_name(dtype));
    buf.resize(size_t(n) * dtype_size(dtype));
    for (int64_t i = 0; i < n; i++) {
      float f;
      switch (host_dtype) {
        case NDX_F32: f = ((const float*)data)[i]; break;
        case NDX_F16: f = (float)((const _Float16*)data)[i]; break;
        default: {
          uint32_t bits = uint32_t(((const uint16_t*)data)[i]) << 16;
          memcpy(&f, &bits, 4);
        }
      }
      switch (dtype) {
        case NDX_F32: ((float*)buf.data())[i] = f; break;
        case NDX_F16: ((_Float16*)buf.data())[i] = (_Float16)f; break;
        default: ((__bf16*)buf.data())[i] = (__bf16)f; break;
      }
    }
    src = buf.data();
  }
  int64_t shape[4] = {s4[0], s4[1], s4[2], s4[3]};
  ndx_tensor* t = new_tensor(dev, dtype, shape, 4);
  try {
    hip_check(hipMemcpyAsync(t->ptr, src, t->bytes, hipMemcpyHostToDevice, dev->stream), "constant upload");
    hip_check(hipStreamSynchronize(dev->stream), "constant upload");
  } catch (...) {
    free_tensor(t);
    throw;
  }
  return t;
}

NDX_API ndx_status ndx_graph_constant(ndx_graph* g, int32_t dtype, const int64_t* shape,
                                      int32_t rank, const void* data, int32_t host_dtype,
                                      ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  if (dtype_size(dtype) == 0 || dtype_size(host_dtype) == 0) fail(NDX_INVALID_ARG, "unknown element type");
  int64_t s4[4];
  to4(shape, rank, s4);
  ndx_tensor* t = nullptr;
  if (g->dev) {
    NEED(data);
    t = upload_converted(g->dev, data, host_dtype, dtype, s4);
  }
  *out = add_const_value(g, t, dtype, s4, rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_graph_constant_device(ndx_graph* g, ndx_tensor* t, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(t);
  NEED(out);
  if (t->dev != g->dev) fail(NDX_INVALID_ARG, "the tensor belongs to another device");
  int64_t s4[4];
  to4(t->shape, t->rank, s4);
  *out = add_const_value(g, t, t->dtype, s4, t->rank);
  NDX_CATCH
}

static int add_quant_value(ndx_graph* g, ndx_tensor* q, ndx_tensor* scales, int block,
                           const int64_t* s4, int rank) {
  GValue v;
  v.dtype = g->dtype;  // the weight reads as the graph's precision (ModelBuilder.cs:82-87)
  v.rank = rank;
  v.v = packed4(s4);
  v.kind = VK_CONST;
  v.data = q;
  v.scales = scales;
  v.qblock = block;
  v.quant = true;
  v.buffer_elems = numel4(v.v);
  if (q) g->consts->tensors.push_back(q);
  if (scales) g->consts->tensors.push_back(scales);
  int id = g->add_value(v);
  g->values[id].base = id;
  return id;
}

static bool quantizable(ndx_graph* g, int64_t elements, int64_t rows) {
  return g->int8_weights && elements >= (1 << 16) && ndx_quantize_fits(elements, (int32_t)rows, 32);
}

NDX_API ndx_status ndx_graph_weight(ndx_graph* g, const int64_t* shape, int32_t rank,
                                    const void* data, int32_t host_dtype, int32_t rows,
                                    ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  int64_t s4[4];
  to4(shape, rank, s4);
  int64_t n = numel4(packed4(s4));
  if (!dtype_is_float(host_dtype)) fail(NDX_INVALID_ARG, "weights are Float32, Float16 or BFloat16");
  if (rows <= 0) fail(NDX_INVALID_ARG, "rows must be positive");
  if (!quantizable(g, n, rows)) {
    ndx_tensor* t = nullptr;
    if (g->dev) {
      NEED(data);
      t = upload_converted(g->dev, data, host_dtype, g->dtype, s4);
    }
    *out = add_const_value(g, t, g->dtype, s4, rank);
    return NDX_OK;
  }
  int64_t cols = n / rows;
  ndx_tensor *q = nullptr, *sc = nullptr;
  if (g->dev) {
    NEED(data);
    std::vector<int8_t> hq(n);
    std::vector<uint16_t> hs(size_t(rows) * (cols / 32));
    quantize_host(data, host_dtype, rows, cols, 32, NDX_F16, hq.data(), hs.data());
    int64_t qs[2] = {rows, cols}, ss[2] = {rows, cols / 32};
    q = new_tensor(g->dev, NDX_I8, qs, 2);
    try {
      sc = new_tensor(g->dev, NDX_F16, ss, 2);
    } catch (...) {
      free_tensor(q);
      throw;
    }
    hip_check(hipMemcpyAsync(q->ptr, hq.data(), q->bytes, hipMemcpyHostToDevice, g->dev->stream), "weight upload");
    hip_check(hipMemcpyAsync(sc->ptr, hs.data(), sc->bytes, hipMemcpyHostToDevice, g->dev->stream), "weight upload");
    hip_check(hipStreamSynchronize(g->dev->stream), "weight upload");
  }
  *out = add_quant_value(g, q, sc, 32, s4, rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_graph_weight_device(ndx_graph* g, ndx_tensor* t, int32_t rows, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(t);
  NEED(out);
  if (t->dev != g->dev) fail(NDX_INVALID_ARG, "the tensor belongs to another device");
  if (!dtype_is_float(t->dtype)) fail(NDX_INVALID_ARG, "weights are Float32, Float16 or BFloat16");
  int64_t s4[4];
  to4(t->shape, t->rank, s4);
  int64_t n = t->numel();
  if (!quantizable(g, n, rows)) {
    if (t->dtype != g->dtype) {
      // Widen or narrow once, on the device, into the graph's precision.
      ndx_tensor* c = new_tensor(g->dev, g->dtype, t->shape, t->rank);
      ElemArgs e{};
      e.in0 = t->ptr;
      e.v0 = packed4(s4);
      e.dt0 = t->dtype;
      e.out = c->ptr;
      e.vo = packed4(s4);
      e.dto = g->dtype;
      e.op = ELEM_COPY;
      launch_elementwise(e, g->dev->stream);
      hip_check(hipStreamSynchronize(g->dev->stream), "weight conversion");
      free_tensor(t);
      t = c;
    }
    *out = add_const_value(g, t, g->dtype, s4, t->rank);
    return NDX_OK;
  }
  int64_t cols = n / rows;
  const int t_rank = t->rank;
  int64_t qs[2] = {rows, cols}, ss[2] = {rows, cols / 32};
  ndx_tensor* q = new_tensor(g->dev, NDX_I8, qs, 2);
  ndx_tensor* sc = nullptr;
  try {
    sc = new_tensor(g->dev, NDX_F16, ss, 2);
  } catch (...) {
    free_tensor(q);
    throw;
  }
  launch_quantize(t->ptr, t->dtype, rows, cols, 32, NDX_F16, (int8_t*)q->ptr, sc->ptr, g->dev->stream);
  hip_check(hipGetLastError(), "quantize launch");
  hip_check(hipStreamSynchronize(g->dev->stream), "quantize");
  free_tensor(t);
  *out = add_quant_value(g, q, sc, 32, s4, t_rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_graph_weight_int8(ndx_graph* g, ndx_tensor* q, ndx_tensor* scales, int32_t block,
                                         ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(q);
  NEED(scales);
  NEED(out);
  if (q->dtype != NDX_I8 || q->rank != 2) fail(NDX_INVALID_ARG, "q must be an Int8 [rows, cols] tensor");
  int64_t rows = q->shape[0], cols = q->shape[1];
  if (block <= 0 || cols % block) fail(NDX_INVALID_ARG, "the blocks do not tile the columns");
  if ((scales->dtype != NDX_F16 && scales->dtype != NDX_F32) || scales->numel() != rows * (cols / block))
    fail(NDX_INVALID_ARG, "scales must be [rows, cols/block] of Float16 or Float32");
  int64_t s4[4] = {1, 1, rows, cols};
  *out = add_quant_value(g, q, scales, block, s4, 2);
  NDX_CATCH
}

NDX_API ndx_status ndx_value_info(ndx_graph* g, ndx_value value, int32_t* dtype, int64_t* shape,
                                  int32_t* rank) {
  NDX_TRY
  NEED(g);
  GValue& v = g->val(value);
  if (dtype) *dtype = v.dtype;
  if (rank) *rank = v.rank;
  if (shape)
    for (int i = 0; i < 4; i++) shape[i] = i < v.rank ? v.v.size[4 - v.rank + i] : 1;
  NDX_CATCH
}

// ---- views -------------------------------------------------------------------

NDX_API ndx_status ndx_op_reinterpret(ndx_graph* g, ndx_value x, const int64_t* shape, int32_t rank,
                                      const int64_t* strides, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue src = g->val(x);
  int64_t s4[4];
  to4(shape, rank, s4);
  GValue v = src;
  v.kind = VK_VIEW;
  v.rank = rank;
  if (strides) {
    for (int i = 0; i < 4; i++) {
      v.v.size[i] = s4[i];
      v.v.stride[i] = i < 4 - rank ? 0 : strides[i - (4 - rank)];
      if (v.v.stride[i] < 0) fail(NDX_INVALID_ARG, "strides must not be negative");
    }
  } else {
    v.v = packed4(s4);
  }
  // Every element the view reaches must lie in the buffer.
  int64_t last = v.offset;
  for (int i = 0; i < 4; i++) last += (v.v.size[i] - 1) * v.v.stride[i];
  const GValue& owner = g->values[src.base];
  if (last >= owner.buffer_elems)
    fail(NDX_INVALID_ARG, "the view " + shape_str(v.v, v.dtype) + " reaches past its tensor " +
                              shape_str(owner.v, owner.dtype));
  if (src.quant && !same_shape(v.v, src.v) && numel4(v.v) != numel4(src.v))
    fail(NDX_UNSUPPORTED, "an int8 weight can only be viewed at its own size");
  *out = g->add_value(v);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_slice(ndx_graph* g, ndx_value x, const int64_t* offsets, const int64_t* sizes,
                                const int64_t* strides, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  NEED(offsets);
  NEED(sizes);
  GValue src = g->val(x);
  if (src.quant) fail(NDX_UNSUPPORTED, "an int8 weight cannot be sliced");
  int r = src.rank;
  GValue v = src;
  v.kind = VK_VIEW;
  for (int d = 0; d < r; d++) {
    int i = 4 - r + d;
    int64_t st = strides ? strides[d] : 1;
    if (st <= 0) fail(NDX_INVALID_ARG, "slice strides must be positive");
    if (offsets[d] < 0 || sizes[d] <= 0 || offsets[d] + sizes[d] > src.v.size[i])
      fail(NDX_INVALID_ARG, "the slice window leaves " + shape_str(src.v, src.dtype));
    v.offset += offsets[d] * src.v.stride[i];
    v.v.size[i] = (sizes[d] + st - 1) / st;
    v.v.stride[i] = src.v.stride[i] * st;
  }
  *out = g->add_value(v);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_join(ndx_graph* g, const ndx_value* xs, int32_t count, int32_t axis, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(xs);
  NEED(out);
  if (count < 1) fail(NDX_INVALID_ARG, "join needs at least one input");
  GValue first = g->val(xs[0]);
  if (axis < 0 || axis >= first.rank) fail(NDX_INVALID_ARG, "join axis out of range");
  int ax = 4 - first.rank + axis;
  int64_t size[4];
  for (int i = 0; i < 4; i++) size[i] = first.v.size[i];
  GNode n;
  n.op = OP_JOIN;
  n.i0 = ax;
  n.in.push_back(xs[0]);
  for (int k = 1; k < count; k++) {
    GValue& v = g->val(xs[k]);
    if (v.dtype != first.dtype || v.rank != first.rank) fail(NDX_INVALID_ARG, "joined tensors differ in type or rank");
    for (int i = 0; i < 4; i++)
      if (i != ax && v.v.size[i] != first.v.size[i]) fail(NDX_INVALID_ARG, "joined tensors differ off the axis");
    size[ax] += v.v.size[ax];
    n.in.push_back(xs[k]);
  }
  for (int k = 0; k < count; k++)
    if (g->val(xs[k]).quant) fail(NDX_UNSUPPORTED, "an int8 weight cannot be joined");
  *out = g->emit(n, first.dtype, size, first.rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_cast(ndx_graph* g, ndx_value x, int32_t dtype, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  if (!dtype_is_float(dtype)) fail(NDX_UNSUPPORTED, "casts are between float widths");
  if (g->val(x).quant) fail(NDX_UNSUPPORTED, "an int8 weight is read by a linear or a convolution only");
  *out = make_elem(g, ELEM_COPY, x, NDX_NONE, dtype);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_unary(ndx_graph* g, ndx_value x, int32_t kind, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  static const int map[] = {ELEM_COPY, ELEM_SIGMOID, ELEM_SILU, ELEM_GELU, ELEM_TANH, ELEM_GELU_TANH};
  if (kind < 0 || kind > 5) fail(NDX_INVALID_ARG, "unknown unary kind");
  if (g->val(x).quant) fail(NDX_UNSUPPORTED, "an int8 weight is read by a linear or a convolution only");
  *out = make_elem(g, map[kind], x, NDX_NONE, g->val(x).dtype);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_scale_bias(ndx_graph* g, ndx_value x, float scale, float bias, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  *out = make_elem(g, ELEM_SCALE_BIAS, x, NDX_NONE, g->val(x).dtype, scale, bias);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_binary(ndx_graph* g, ndx_value a, ndx_value b, int32_t kind, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  if (kind < 0 || kind > 3) fail(NDX_INVALID_ARG, "unknown binary kind");
  if (b == NDX_NONE) fail(NDX_INVALID_ARG, "binary needs two operands");
  *out = make_elem(g, ELEM_ADD + kind, a, b, g->val(a).dtype);
  NDX_CATCH
}

// ---- layers ------------------------------------------------------------------

NDX_API ndx_status ndx_op_linear(ndx_graph* g, ndx_value x, ndx_value w, ndx_value bias, int32_t epilogue,
                                 ndx_value aux0, ndx_value aux1, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& vx = g->val(x);
  GValue& vw = g->val(w);
  require_float(vx, "the linear input");
  if (vx.dtype != NDX_F32 && vx.dtype != NDX_BF16 && vx.dtype != NDX_F16)
    fail(NDX_INVALID_ARG, "the linear input must be a float tensor");
  int64_t K = vx.v.size[3], M = vx.v.size[2];
  // W is [N, K]: the last two axes; any leading axes must be 1 or a stride-0
  // broadcast over the batch (Layers.cs:142-148).
  int64_t N = vw.v.size[2];
  if (vw.v.size[3] != K)
    fail(NDX_INVALID_ARG, "gemm inner extents differ: " + shape_str(vx.v, vx.dtype) + " vs " + shape_str(vw.v, vw.dtype));
  for (int i = 0; i < 2; i++)
    if (vw.v.size[i] != 1 && vw.v.stride[i] != 0)
      fail(NDX_INVALID_ARG, "a linear weight has no batch axes of its own");
  if (!vw.quant && !dtype_is_float(vw.dtype))
    fail(NDX_UNSUPPORTED, std::string("a linear weight of ") + dtype_name(vw.dtype) + " without block scales");
  int wdt = vw.quant ? NDX_I8 : vw.dtype;
  bool ok = (vx.dtype == NDX_BF16 && (wdt == NDX_BF16 || wdt == NDX_I8)) ||
            (vx.dtype == NDX_F16 && (wdt == NDX_F16 || wdt == NDX_I8)) ||
            (vx.dtype == NDX_F32 && (wdt == NDX_F32 || wdt == NDX_BF16 || wdt == NDX_F16 || wdt == NDX_I8));
  if (!ok)
    fail(NDX_UNSUPPORTED, std::string("a ") + dtype_name(vx.dtype) + " product with " + dtype_name(wdt) + " weights");
  if (bias != NDX_NONE) {
    GValue& vb = g->val(bias);
    require_float(vb, "the bias");
    if (numel4(vb.v) != N) fail(NDX_INVALID_ARG, "the bias must have one value per output feature");
  }
  if (epilogue < 0 || epilogue > NDX_EPI_SWIGLU) fail(NDX_INVALID_ARG, "unknown epilogue");
  if (epilogue == NDX_EPI_SWIGLU && N % 2) fail(NDX_INVALID_ARG, "a SwiGLU needs interleaved gate and up rows (an even count)");
  int out_dtype = vx.dtype;
  if (epilogue == NDX_EPI_GATED_RESIDUAL || epilogue == NDX_EPI_RESIDUAL) {
    if (aux1 == NDX_NONE) fail(NDX_INVALID_ARG, "a residual epilogue needs the residual");
    GValue& r = g->val(aux1);
    require_float(r, "the residual");
    if (r.v.size[0] != vx.v.size[0] || r.v.size[1] != vx.v.size[1] || r.v.size[2] != M || r.v.size[3] != N)
      fail(NDX_INVALID_ARG, "the residual " + shape_str(r.v, r.dtype) + " is not the product's shape");
    out_dtype = r.dtype;
    if (epilogue == NDX_EPI_GATED_RESIDUAL) {
      if (aux0 == NDX_NONE) fail(NDX_INVALID_ARG, "a gated residual needs the gate");
      GValue& gt = g->val(aux0);
      require_float(gt, "the gate");
      if (gt.v.size[3] != N || (gt.v.size[2] != 1 && gt.v.size[2] != M))
        fail(NDX_INVALID_ARG, "the gate must be a [.., 1, N] row or [.., M, N]");
      if ((gt.v.size[0] != 1 && gt.v.size[0] != vx.v.size[0]) || (gt.v.size[1] != 1 && gt.v.size[1] != vx.v.size[1]))
        fail(NDX_INVALID_ARG, "the gate's batch does not match the input's");
    }
  }
  GNode n;
  n.op = OP_LINEAR;
  n.in = {x, w, bias, aux0, aux1};
  n.i0 = epilogue;
  int64_t size[4] = {vx.v.size[0], vx.v.size[1], M, epilogue == NDX_EPI_SWIGLU ? N / 2 : N};
  *out = g->emit(n, out_dtype, size, vx.rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_gemm(ndx_graph* g, ndx_value a, ndx_value b, ndx_value c, int32_t trans_a,
                               int32_t trans_b, float alpha, float beta, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& va = g->val(a);
  GValue& vb = g->val(b);
  require_float(va, "gemm operand a");
  require_float(vb, "gemm operand b");
  if (vb.quant) fail(NDX_UNSUPPORTED, "an int8 weight goes through the linear layer");
  int64_t rows = trans_a ? va.v.size[3] : va.v.size[2];
  int64_t inner = trans_a ? va.v.size[2] : va.v.size[3];
  int64_t innerB = trans_b ? vb.v.size[3] : vb.v.size[2];
  int64_t cols = trans_b ? vb.v.size[2] : vb.v.size[3];
  if (inner != innerB)
    fail(NDX_INVALID_ARG, "gemm inner extents differ: " + shape_str(va.v, va.dtype) + " vs " + shape_str(vb.v, vb.dtype));
  if (va.v.size[0] != vb.v.size[0] || va.v.size[1] != vb.v.size[1])
    fail(NDX_INVALID_ARG, "gemm operands differ in their batch axes");
  int64_t size[4] = {va.v.size[0], va.v.size[1], rows, cols};
  if (c != NDX_NONE) {
    GValue& vc = g->val(c);
    View4 want = packed4(size);
    if (!same_shape(vc.v, want)) fail(NDX_INVALID_ARG, "gemm operand c is not the output's shape");
  }
  GNode n;
  n.op = OP_GEMM;
  n.in = {a, b, c};
  n.i0 = trans_a != 0;
  n.i1 = trans_b != 0;
  n.f0 = alpha;
  n.f1 = beta;
  *out = g->emit(n, va.dtype, size, va.rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_attention(ndx_graph* g, ndx_value q, ndx_value k, ndx_value v, int32_t heads,
                                    float scale, int32_t mask_kind, ndx_value mask, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& vq = g->val(q);
  GValue& vk = g->val(k);
  GValue& vv = g->val(v);
  if (vq.dtype != vk.dtype || vq.dtype != vv.dtype) fail(NDX_INVALID_ARG, "query, key and value differ in precision");
  require_float(vq, "the query");
  if (heads <= 0) fail(NDX_INVALID_ARG, "heads must be positive");
  // [B, 1, T, H*d] packed layout (the batch may sit on either leading axis,
  // Dml/DmlOps.cs:557-569).
  auto batch_of = [](const GValue& x) { return x.v.size[0] * x.v.size[1]; };
  int64_t B = batch_of(vq);
  if (batch_of(vk) != B || batch_of(vv) != B) fail(NDX_INVALID_ARG, "query, key and value differ in batch");
  if (vq.v.size[3] % heads || vk.v.size[3] % heads || vv.v.size[3] % heads)
    fail(NDX_INVALID_ARG, "the widths do not split into the heads");
  if (vq.v.size[3] != vk.v.size[3]) fail(NDX_INVALID_ARG, "query and key widths differ");
  if (vk.v.size[2] != vv.v.size[2]) fail(NDX_INVALID_ARG, "key and value lengths differ");
  int64_t d = vq.v.size[3] / heads, dv = vv.v.size[3] / heads;
  if (d != dv || d > 128)
    fail(NDX_UNSUPPORTED, "attention head size " + std::to_string(d));
  if ((mask == NDX_NONE) != (mask_kind == NDX_MASK_NONE))
    fail(NDX_INVALID_ARG, "a mask and its type come together");
  if (mask != NDX_NONE) {
    GValue& m = g->val(mask);
    if (m.dtype != NDX_I32) fail(NDX_INVALID_ARG, "masks are Int32");
    if (mask_kind == NDX_MASK_KEY_LENGTH) {
      if (numel4(m.v) != 1) fail(NDX_INVALID_ARG, "a key-length mask is [1, 1, 1, 1]");
    } else if (mask_kind == NDX_MASK_BOOLEAN) {
      if (m.v.size[2] != vq.v.size[2] || m.v.size[3] != vk.v.size[2] ||
          (m.v.size[1] != heads && m.v.size[1] != 1) || (m.v.size[0] != B && m.v.size[0] != 1))
        fail(NDX_INVALID_ARG, "a boolean mask is [batch, heads, tokens, keys]");
    } else {
      fail(NDX_INVALID_ARG, "unknown mask type");
    }
  }
  GNode n;
  n.op = OP_ATTN;
  n.in = {q, k, v, mask};
  n.i0 = heads;
  n.i1 = mask_kind;
  n.f0 = scale;
  int64_t size[4] = {vq.v.size[0], vq.v.size[1], vq.v.size[2], vv.v.size[3]};
  *out = g->emit(n, vq.dtype, size, vq.rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_head_norm_rotate(ndx_graph* g, ndx_value x, ndx_value weight, float eps,
                                           ndx_value cos, ndx_value sin, int32_t heads, int32_t out_dtype,
                                           ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& vx = g->val(x);
  require_float(vx, "the head norm input");
  if (heads <= 0 || vx.v.size[3] % heads) fail(NDX_INVALID_ARG, "the width does not split into the heads");
  int64_t d = vx.v.size[3] / heads;
  if (d % 2 || d > 256) fail(NDX_UNSUPPORTED, "head size " + std::to_string(d));
  if (weight != NDX_NONE && numel4(g->val(weight).v) != d) fail(NDX_INVALID_ARG, "the head norm weight is [d]");
  if ((cos == NDX_NONE) != (sin == NDX_NONE)) fail(NDX_INVALID_ARG, "cos and sin come together");
  if (cos != NDX_NONE) {
    for (int t : {cos, sin}) {
      GValue& c = g->val(t);
      if (c.dtype != NDX_F32) fail(NDX_INVALID_ARG, "rotary tables are Float32");
      if (numel4(c.v) != vx.v.size[2] * (d / 2)) fail(NDX_INVALID_ARG, "rotary tables are [1, tokens, 1, d/2]");
    }
  }
  if (!dtype_is_float(out_dtype)) fail(NDX_INVALID_ARG, "the output must be a float type");
  GNode n;
  n.op = OP_HNR;
  n.in = {x, weight, cos, sin};
  n.i0 = heads;
  n.f0 = eps;
  int64_t size[4] = {vx.v.size[0], vx.v.size[1], vx.v.size[2], vx.v.size[3]};
  *out = g->emit(n, out_dtype, size, vx.rank);
  NDX_CATCH
}

static int row_norm(ndx_graph* g, int mode, int x, int w, int b, float eps, int out_dtype) {
  GValue& vx = g->val(x);
  require_float(vx, "the normalised tensor");
  int64_t D = vx.v.size[3];
  for (int id : {w, b}) {
    if (id == NDX_NONE) continue;
    GValue& p = g->val(id);
    require_float(p, "a norm parameter");
    if (p.v.size[3] != D) fail(NDX_INVALID_ARG, "a norm parameter must span the normalised axis");
    if (p.v.size[2] != 1 && p.v.size[2] != vx.v.size[2])
      fail(NDX_INVALID_ARG, "a norm parameter is one row (per batch) or one per row");
  }
  GNode n;
  n.op = OP_ROWNORM;
  n.in = {x, w, b};
  n.i0 = mode;
  n.f0 = eps;
  int64_t size[4] = {vx.v.size[0], vx.v.size[1], vx.v.size[2], D};
  return g->emit(n, out_dtype, size, vx.rank);
}

NDX_API ndx_status ndx_op_layer_norm(ndx_graph* g, ndx_value x, ndx_value weight, ndx_value bias, float eps,
                                     ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  *out = row_norm(g, 0, x, weight, bias, eps, g->val(x).dtype);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_modulate(ndx_graph* g, ndx_value x, ndx_value shift, ndx_value scale, float eps,
                                   int32_t out_dtype, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  if (scale == NDX_NONE) fail(NDX_INVALID_ARG, "modulate needs a scale");
  if (!dtype_is_float(out_dtype)) fail(NDX_INVALID_ARG, "the output must be a float type");
  *out = row_norm(g, 1, x, scale, shift, eps, out_dtype);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_rms_norm(ndx_graph* g, ndx_value x, ndx_value weight, float eps, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  *out = row_norm(g, 2, x, weight, NDX_NONE, eps, g->val(x).dtype);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_group_norm(ndx_graph* g, ndx_value x, ndx_value weight, ndx_value bias, int32_t groups,
                                     float eps, int32_t silu, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& vx = g->val(x);
  require_float(vx, "the group norm input");
  int64_t C = vx.v.size[1];
  if (groups <= 0 || C % groups) fail(NDX_INVALID_ARG, std::to_string(C) + " channels do not divide into " + std::to_string(groups) + " groups");
  for (int id : {weight, bias})
    if (id != NDX_NONE && numel4(g->val(id).v) != C) fail(NDX_INVALID_ARG, "the group norm affine is per channel");
  if (weight != NDX_NONE && bias != NDX_NONE && g->val(weight).dtype != g->val(bias).dtype)
    fail(NDX_INVALID_ARG, "the group norm scale and bias differ in precision");
  GNode n;
  n.op = OP_GROUPNORM;
  n.in = {x, weight, bias};
  n.i0 = groups;
  n.i1 = silu != 0;
  n.f0 = eps;
  int64_t size[4] = {vx.v.size[0], vx.v.size[1], vx.v.size[2], vx.v.size[3]};
  *out = g->emit(n, vx.dtype, size, vx.rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_conv2d(ndx_graph* g, ndx_value x, ndx_value w, ndx_value bias, int32_t stride,
                                 int32_t pad_start, int32_t pad_end, ndx_value residual, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& vx = g->val(x);
  GValue& vw = g->val(w);
  require_float(vx, "the convolution input");
  if (stride <= 0 || pad_start < 0 || pad_end < 0) fail(NDX_INVALID_ARG, "bad stride or padding");
  // [Cout, Cin, kh, kw]; an int8 filter keeps that logical shape and is
  // stored as [Cout, Cin*kh*kw] rows.
  int64_t Cout = vw.v.size[0], Cin = vw.v.size[1], kh = vw.v.size[2], kw = vw.v.size[3];
  if (Cin != vx.v.size[1]) fail(NDX_INVALID_ARG, "the filter's input channels differ from the input's");
  int wdt = vw.quant ? NDX_I8 : vw.dtype;
  if (!((wdt == vx.dtype) || wdt == NDX_I8 || (vx.dtype == NDX_F32 && dtype_is_float(wdt))))
    fail(NDX_UNSUPPORTED, "filter and input precisions");
  int64_t Ho = (vx.v.size[2] + pad_start + pad_end - kh) / stride + 1;
  int64_t Wo = (vx.v.size[3] + pad_start + pad_end - kw) / stride + 1;
  if (Ho <= 0 || Wo <= 0) fail(NDX_INVALID_ARG, "the convolution output is empty");
  if (bias != NDX_NONE && numel4(g->val(bias).v) != Cout) fail(NDX_INVALID_ARG, "the bias is per output channel");
  int64_t size[4] = {vx.v.size[0], Cout, Ho, Wo};
  if (residual != NDX_NONE) {
    GValue& r = g->val(residual);
    if (!same_shape(r.v, packed4(size)) || r.dtype != vx.dtype) fail(NDX_INVALID_ARG, "the residual is not the output's shape");
  }
  GNode n;
  n.op = OP_CONV;
  n.in = {x, w, bias, residual};
  n.i0 = stride;
  n.i1 = pad_start;
  n.i2 = pad_end;
  n.i3 = (int)kh;
  n.i4 = (int)kw;
  *out = g->emit(n, vx.dtype, size, 4);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_upsample_nearest(ndx_graph* g, ndx_value x, int32_t scale, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& vx = g->val(x);
  require_float(vx, "the upsampled tensor");
  if (scale < 1) fail(NDX_INVALID_ARG, "scale must be at least 1");
  GNode n;
  n.op = OP_UPSAMPLE;
  n.in = {x};
  n.i0 = scale;
  int64_t size[4] = {vx.v.size[0], vx.v.size[1], vx.v.size[2] * scale, vx.v.size[3] * scale};
  *out = g->emit(n, vx.dtype, size, 4);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_patchify(ndx_graph* g, ndx_value x, int32_t patch, int32_t order, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& vx = g->val(x);
  require_float(vx, "the latent");
  int64_t C = vx.v.size[1], H = vx.v.size[2], W = vx.v.size[3];
  if (patch < 1 || H % patch || W % patch) fail(NDX_INVALID_ARG, "the latent does not divide into patches");
  if (order != NDX_PATCH_CHANNEL_FIRST && order != NDX_PATCH_CHANNEL_LAST) fail(NDX_INVALID_ARG, "bad patch order");
  GNode n;
  n.op = OP_PATCH;
  n.in = {x};
  n.i0 = patch;
  n.i1 = 0;
  n.i5 = order;
  n.i2 = (int)C;
  n.i3 = (int)H;
  n.i4 = (int)W;
  int64_t size[4] = {vx.v.size[0], 1, (H / patch) * (W / patch), C * patch * patch};
  *out = g->emit(n, vx.dtype, size, 4);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_guided_euler_step(ndx_graph* g, ndx_value x, ndx_value uncond, ndx_value cond,
                                           ndx_value scalars, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& vx = g->val(x);
  GValue& vc = g->val(cond);
  GValue& vs = g->val(scalars);
  if (vx.dtype != NDX_F32 || vc.dtype != NDX_F32 || vs.dtype != NDX_F32)
    fail(NDX_INVALID_ARG, "the sample, the predictions and the scalars are Float32");
  if (numel4(vs.v) < 3) fail(NDX_INVALID_ARG, "the scalars are (guidance, sigma, sigma_next)");
  if (!same_shape(vx.v, vc.v)) fail(NDX_INVALID_ARG, "the prediction " + shape_str(vc.v, vc.dtype) + " is not the sample's shape");
  if (uncond != NDX_NONE) {
    GValue& vu = g->val(uncond);
    if (vu.dtype != NDX_F32 || !same_shape(vx.v, vu.v))
      fail(NDX_INVALID_ARG, "the unconditional prediction is not the sample's Float32 shape");
  }
  GNode n;
  n.op = OP_SAMPLE;
  n.in = {x, uncond, cond, scalars};
  *out = g->emit(n, NDX_F32, vx.v.size, vx.rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_softmax(ndx_graph* g, ndx_value x, float scale, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& vx = g->val(x);
  if (vx.dtype != NDX_F32 && vx.dtype != NDX_BF16 && vx.dtype != NDX_F16)
    fail(NDX_INVALID_ARG, "a softmax reads Float32, Float16 or BFloat16");
  GNode n;
  n.op = OP_SOFTMAX;
  n.in = {x};
  n.f0 = scale;
  *out = g->emit(n, vx.dtype, vx.v.size, vx.rank);
  NDX_CATCH
}

NDX_API ndx_status ndx_op_unpatchify(ndx_graph* g, ndx_value x, int32_t patch, int32_t channels, int32_t height,
                                     int32_t width, int32_t order, ndx_value* out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  GValue& vx = g->val(x);
  require_float(vx, "the tokens");
  if (patch < 1 || height % patch || width % patch) fail(NDX_INVALID_ARG, "the image does not divide into patches");
  if (vx.v.size[1] != 1 || vx.v.size[2] != int64_t(height / patch) * (width / patch) ||
      vx.v.size[3] != int64_t(channels) * patch * patch)
    fail(NDX_INVALID_ARG, "the tokens do not fill the latent");
  if (order != NDX_PATCH_CHANNEL_FIRST && order != NDX_PATCH_CHANNEL_LAST) fail(NDX_INVALID_ARG, "bad patch order");
  GNode n;
  n.op = OP_PATCH;
  n.in = {x};
  n.i0 = patch;
  n.i1 = 1;
  n.i5 = order;
  n.i2 = channels;
  n.i3 = height;
  n.i4 = width;
  int64_t size[4] = {vx.v.size[0], channels, height, width};
  *out = g->emit(n, vx.dtype, size, 4);
  NDX_CATCH
}

}  // extern "C"

// ---- compile -------------------------------------------------------------------

namespace {

struct Compiler {
  ndx_graph* g;
  std::vector<GValue> values;
  std::vector<GNode> nodes;
  int lane = 0;  // of the node being scheduled: the nodes inserted for it share it

  int new_owner(int dtype, const View4& shape_from, int rank) {
    GValue v;
    v.dtype = dtype;
    v.rank = rank;
    int64_t s[4] = {shape_from.size[0], shape_from.size[1], shape_from.size[2], shape_from.size[3]};
    v.v = packed4(s);
    v.kind = VK_NODE;
    v.buffer_elems = numel4(v.v);
    values.push_back(v);
    int id = (int)values.size() - 1;
    values[id].base = id;
    return id;
  }

  // The filter value `wid` (a packed constant [Cout, Cin, kh, kw]) reordered
  // on the device to rows of [kh, kw, cin_pad] (conv_filter_row elements,
  // the channels past Cin and the row's tail zero), as a new constant value.
  int reordered_filter(int wid, int64_t cin_pad) {
    const GValue& w = values[wid];
    ndx_tensor* src = w.data;
    ndx_tensor* r;
    const int64_t taps = w.v.size[2] * w.v.size[3], row = conv_filter_row(cin_pad, taps);
    // [Cout, row] as 4-D: [Cout, cin_pad, kh, kw] when the taps are whole K
    // tiles, [Cout, row, 1, 1] when K runs over the taps unpadded.
    const int64_t shape[4] = {w.v.size[0], row == taps * cin_pad ? cin_pad : row,
                              row == taps * cin_pad ? w.v.size[2] : 1, row == taps * cin_pad ? w.v.size[3] : 1};
    auto it = g->consts->nhwc_filters.find(src);
    if (it != g->consts->nhwc_filters.end()) {
      r = it->second;
    } else {
      r = new_tensor(g->dev, w.dtype, shape, 4);
      g->consts->tensors.push_back(r);
      g->consts->nhwc_filters[src] = r;
      launch_reorder_filter(src->ptr, r->ptr, w.dtype, w.v.size[0], w.v.size[1], taps, g->dev->stream, cin_pad, row);
      hip_check(hipGetLastError(), "filter reorder launch");
      hip_check(hipStreamSynchronize(g->dev->stream), "filter reorder");
    }
    GValue v = w;
    v.data = r;
    v.v = packed4(shape);
    values.push_back(v);
    int id = (int)values.size() - 1;
    values[id].base = id;
    return id;
  }

  // A packed copy of a view, scheduled just before `before` (appended to
  // `sched`); returns the copy's value id.
  int pack(int id, std::vector<GNode>& sched) {
    GValue src = values[id];
    int out = new_owner(src.dtype, src.v, src.rank);
    // The token view [N, 1, P, C] of a packed [N, C, P] buffer (ToTokens of
    // an NCHW image): the tiled NCHW -> NHWC transposition.
    const View4& v = src.v;
    if (dtype_size(src.dtype) == 2 && src.offset == 0 && v.size[1] == 1 && v.stride[2] == 1 &&
        v.stride[3] == v.size[2] && (v.size[0] == 1 || v.stride[0] == v.size[2] * v.size[3]) && v.size[3] > 1) {
      GNode t;
      t.op = OP_NHWC;
      t.in = {id};
      t.i1 = 1;
      t.out = out;
      t.lane = lane;
      sched.push_back(t);
      return out;
    }
    GNode n;
    n.op = OP_ELEM;
    n.in = {id, NDX_NONE};
    n.i0 = ELEM_COPY;
    n.f0 = 1.f;
    n.out = out;
    n.lane = lane;
    sched.push_back(n);
    return out;
  }
};

void prof_info(GNode& n, const std::vector<GValue>& V) {
  auto bytes_of = [&](int id) -> double {
    if (id < 0) return 0;
    const GValue& v = V[id];
    if (v.quant) return double(numel4(v.v)) + (v.scales ? double(v.scales->bytes) : 0.0);
    return double(numel4(v.v)) * dtype_size(v.dtype);
  };
  double out_b = bytes_of(n.out);
  switch (n.op) {
    case OP_LINEAR: {
      const GValue& x = V[n.in[0]];
      const GValue& w = V[n.in[1]];
      double M = double(x.v.size[2]) * x.v.size[0] * x.v.size[1], K = x.v.size[3], N = w.v.size[2];
      n.flops = 2 * M * N * K;
      n.bytes = bytes_of(n.in[0]) + bytes_of(n.in[1]) + out_b + bytes_of(n.in[4]);
      break;
    }
    case OP_GEMM: {
      const GValue& o = V[n.out];
      const GValue& a = V[n.in[0]];
      double K = n.i0 ? a.v.size[2] : a.v.size[3];
      n.flops = 2.0 * numel4(o.v) * K;
      n.bytes = bytes_of(n.in[0]) + bytes_of(n.in[1]) + out_b;
      n.family = "gemm_generic";
      break;
    }
    case OP_ATTN: {
      const GValue& q = V[n.in[0]];
      const GValue& k = V[n.in[1]];
      double B = double(q.v.size[0]) * q.v.size[1], T = q.v.size[2], S = k.v.size[2], D = q.v.size[3];
      n.flops = 4.0 * B * T * S * D;
      n.bytes = bytes_of(n.in[0]) + bytes_of(n.in[1]) + bytes_of(n.in[2]) + out_b;
      n.family = std::string("attention_") + dtype_name(q.dtype);
      break;
    }
    case OP_CONV: {
      const GValue& o = V[n.out];
      const GValue& x = V[n.in[0]];
      n.flops = 2.0 * numel4(o.v) * x.v.size[1] * n.i3 * n.i4;
      n.bytes = bytes_of(n.in[0]) + bytes_of(n.in[1]) + out_b + bytes_of(n.in[2]) + bytes_of(n.in[3]);
      n.family = std::string("conv2d_") + dtype_name(x.dtype);
      if (n.i5) {
        ConvArgs a{};
        a.N = (int)x.v.size[0];
        a.Cin = (int)x.v.size[1];
        a.H = (int)x.v.size[2] << n.conv_up;
        a.W = (int)x.v.size[3] << n.conv_up;
        a.Cout = (int)o.v.size[1];
        a.kh = n.i3;
        a.kw = n.i4;
        a.Ho = (int)o.v.size[2];
        a.Wo = (int)o.v.size[3];
        a.cin_k = (int)n.conv_cin_k;
        a.up = n.conv_up;
        n.family = conv_family(a);
      }
      break;
    }
    case OP_NHWC:
      n.bytes = 2 * out_b;
      n.family = "nchw_to_nhwc";
      break;
    default: {
      double b = out_b;
      for (int id : n.in) b += bytes_of(id);
      n.bytes = b;
      static const char* names[] = {"elementwise", "join", "linear", "gemm", "attention", "head_norm_rotate",
                                    "row_norm", "group_norm", "conv2d", "upsample", "patchify", "guided_euler",
                                    "softmax"};
      static_assert(sizeof(names) / sizeof(names[0]) == OP_SOFTMAX + 1, "a kernel family name per operator");
      n.family = names[n.op];
      if (n.op == OP_ROWNORM)
        n.family = n.i1 ? (n.i0 == 0 ? "channel_layer_norm" : "channel_rms_norm")
                        : (n.i0 == 0 ? "layer_norm" : n.i0 == 1 ? "modulate" : "rms_norm");
    }
  }
}

}  // namespace

// The cross-lane waits of a two-lane model: a node waits for the latest
// node of the other lane that produced a value it reads, and, where the
// arena hands it bytes that a dead value occupied, for every node of the
// other lane that touched that value. A paired linear's second half runs
// inside the first's launch and counts as it.
static void plan_lanes(ndx_model* m, const std::vector<int>& last) {
  const int nn = (int)m->nodes.size(), nv = (int)m->values.size();
  m->two_lanes = false;
  for (const auto& n : m->nodes)
    if (n.lane) m->two_lanes = true;
  if (!m->two_lanes) return;
  auto exec = [&](int j) { return (m->nodes[j].op == OP_LINEAR && m->nodes[j].i5 == 2) ? j - 1 : j; };
  std::vector<int> prod(nv, -1);
  for (int i = 0; i < nn; i++) prod[m->nodes[i].out] = exec(i);
  m->waits.assign(nn, {-1, -1});
  auto dep = [&](int i, int j) {
    if (j < 0) return;
    i = exec(i);
    j = exec(j);
    const int lj = m->nodes[j].lane;
    if (m->nodes[i].lane == lj || j >= i) return;
    m->waits[i][lj] = std::max(m->waits[i][lj], j);
  };
  std::vector<std::vector<int>> users(nv);
  for (int i = 0; i < nn; i++) {
    const GNode& n = m->nodes[i];
    auto use = [&](int id) {
      if (id < 0) return;
      const int b = m->values[id].base;
      dep(i, prod[b]);
      users[b].push_back(exec(i));
    };
    for (int id : n.in) use(id);
    if (n.op == OP_ATTN)
      for (int j = 0; j < 3; j++) {
        use(n.seg[j][0]);
        use(n.seg[j][1]);
      }
    users[n.out].push_back(exec(i));
  }
  struct Alloc {
    int64_t off, size;
    int first, last, base;
  };
  std::vector<Alloc> al;
  for (int id = 0; id < nv; id++) {
    if (m->arena_off[id] < 0 || m->values[id].base != id || prod[id] < 0) continue;
    const int64_t bytes = (int64_t(m->values[id].buffer_elems) * dtype_size(m->values[id].dtype) + 255) & ~int64_t(255);
    al.push_back({m->arena_off[id], bytes, prod[id], exec(std::max(last[id], prod[id])), id});
  }
  for (int i = 0; i < nn; i++)
    if (m->nodes[i].scratch_bytes > 0)
      al.push_back({m->nodes[i].scratch_off, (m->nodes[i].scratch_bytes + 255) & ~int64_t(255), exec(i), exec(i), -1 - i});
  for (const Alloc& a : al)
    for (const Alloc& b : al) {
      if (b.last >= a.first || a.off >= b.off + b.size || b.off >= a.off + a.size) continue;
      if (b.base >= 0) {
        for (int u : users[b.base]) dep(a.first, u);
      } else {
        dep(a.first, -1 - b.base);
      }
    }
  m->signal.assign(nn, -1);
  int ne = 0;
  for (int i = 0; i < nn; i++)
    for (int t = 0; t < 2; t++)
      if (m->waits[i][t] >= 0 && m->signal[m->waits[i][t]] < 0) m->signal[m->waits[i][t]] = ne++;
  m->lane_events.resize(ne + 2);
  // The second stream exists before the first run, so no run creates it.
  (void)m->dev->aux_stream();
  // Both lanes are on this device: a device-scope release makes a lane's
  // writes visible to the other (all XCDs), without the system-scope cache
  // writeback a default event does.
  for (auto& e : m->lane_events)
    hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming | hipEventReleaseToDevice), "hipEventCreate");
}

extern "C" NDX_API ndx_status ndx_graph_compile(ndx_graph* g, const ndx_value* outputs, int32_t count,
                                                ndx_model** out) {
  NDX_TRY
  NEED(g);
  NEED(out);
  NEED(outputs);
  *out = nullptr;
  if (!g->dev) fail(NDX_INVALID_STATE, "a graph without a device only infers shapes and cannot compile");
  g->dev->check_usable();
  if (count < 1) fail(NDX_INVALID_ARG, "a model needs an output");
  Compiler c{g, g->values, {}};
  std::vector<GNode> sched;
  std::vector<int> outs;
  std::vector<GNode> src = g->nodes;

  for (int i = 0; i < count; i++) {
    GValue& v = g->val(outputs[i]);
    const GValue& owner = g->values[v.base];
    if (owner.kind == VK_INPUT || owner.kind == VK_CONST)
      fail(NDX_INVALID_ARG, "a graph input cannot be an output");
    outs.push_back(outputs[i]);
  }

  // Consumer counts by base value, over all nodes.
  std::vector<int> uses(c.values.size(), 0);
  for (auto& n : src)
    for (int id : n.in)
      if (id >= 0) uses[c.values[id].base]++;

  // Rewrite: a join along the token axis of two pieces feeding an attention
  // becomes two row segments of that attention's operand.
  for (auto& n : src) {
    if (n.op != OP_ATTN) continue;
    for (int j = 0; j < 3; j++) {
      int id = n.in[j];
      const GValue& v = c.values[id];
      n.seg[j][0] = id;
      if (v.kind != VK_NODE || v.offset != 0 || !is_packed(v.v)) continue;
      const GNode& p = src[v.producer];
      if (p.op != OP_JOIN || p.in.size() != 2 || p.i0 != 2) continue;
      int64_t ld, bs;
      bool ok = true;
      for (int k = 0; k < 2; k++) {
        const GValue& s = c.values[p.in[k]];
        if (c.values[s.base].quant || !rows_layout(s.v, ld, bs)) ok = false;
      }
      if (!ok) continue;
      n.seg[j][0] = p.in[0];
      n.seg[j][1] = p.in[1];
    }
  }

  // Rewrite: a join along the tokens of two broadcasts of single rows of
  // one value, read as a Modulate's scale or shift or a gated residual's
  // gate (the image and text rows of Models/QwenImage/QwenImageDit.cs:
  // 307-315), is never materialised: the operand becomes the first
  // broadcast, and the node reads the second row from the split on.
  auto two_rows = [&](int id, int64_t& split, int64_t& off) -> int {
    const GValue& v = c.values[id];
    if (v.kind != VK_NODE || v.base != id || v.producer < 0 || v.v.size[2] <= 1) return -1;
    const GNode& p = src[v.producer];
    if (p.op != OP_JOIN || p.in.size() != 2 || p.i0 != 2) return -1;
    const GValue& a = c.values[p.in[0]];
    const GValue& b = c.values[p.in[1]];
    if (a.base != b.base || a.dtype != b.dtype || c.values[a.base].quant) return -1;
    for (const GValue* e : {&a, &b})
      if ((e->v.size[2] > 1 && e->v.stride[2] != 0) || (e->v.size[3] > 1 && e->v.stride[3] != 1) ||
          e->v.size[0] != v.v.size[0] ||
          e->v.size[1] != v.v.size[1])
        return -1;
    if (a.v.stride[0] != b.v.stride[0] || a.v.stride[1] != b.v.stride[1]) return -1;
    split = a.v.size[2];
    off = b.offset - a.offset;
    return p.in[0];
  };
  for (auto& n : src) {
    if (n.op == OP_LINEAR && n.i0 == EPI_GATED_RESIDUAL && n.in[3] >= 0) {
      int64_t split, off;
      const int first = two_rows(n.in[3], split, off);
      if (first >= 0) {
        n.in[3] = first;
        n.rows_split[3] = split;
        n.rows_off[3] = off;
      }
    } else if (n.op == OP_ROWNORM) {
      int64_t split[3] = {0, 0, 0}, off[3] = {0, 0, 0};
      int first[3] = {-1, -1, -1};
      for (int j = 1; j < 3; j++)
        if (n.in[j] >= 0) first[j] = two_rows(n.in[j], split[j], off[j]);
      // The kernel takes one split for the weight and the bias.
      if (first[1] >= 0 && first[2] >= 0 && split[1] != split[2]) first[2] = -1;
      for (int j = 1; j < 3; j++)
        if (first[j] >= 0) {
          n.in[j] = first[j];
          n.rows_split[j] = split[j];
          n.rows_off[j] = off[j];
        }
    }
  }

  // Rewrite: x * Gelu(y), the GELU's output read by this product only (the
  // GEGLU of SDXL's feed-forward, Models/Sdxl/UNetLayers.cs), becomes one
  // elementwise pass; the GELU node is then unreachable and never runs.
  for (auto& n : src) {
    if (n.op != OP_ELEM || n.i0 != ELEM_MUL || n.in.size() < 2 || n.in[1] < 0) continue;
    const int gid = n.in[1];
    const GValue& gv = c.values[gid];
    if (gv.kind != VK_NODE || gv.base != gid || gv.producer < 0 || uses[gid] != 1) continue;
    if (std::find(outs.begin(), outs.end(), gid) != outs.end()) continue;
    const GNode& p = src[gv.producer];
    if (p.op != OP_ELEM || p.i0 != ELEM_GELU || p.in.empty() || p.in[0] < 0 ||
        (p.in.size() > 1 && p.in[1] >= 0) || gv.dtype != c.values[n.out].dtype ||
        c.values[p.in[0]].dtype != gv.dtype || p.lane != n.lane)
      continue;
    n.i0 = ELEM_MUL_GELU;
    n.in[1] = p.in[0];
  }

  // The K channels per tap an implicit-GEMM convolution of `n` runs with
  // over input value xid (read through a 2x upsample when up), or 0 when
  // the direct kernel runs: 16-bit filters held as constants, and 32-bit
  // offsets into the input image and the filter.
  auto conv_gemm_k = [&](const GNode& n, int xid) -> int64_t {
    const GValue& x = c.values[xid];
    const GValue& w = c.values[n.in[1]];
    if (w.quant || w.kind != VK_CONST || w.base != n.in[1] || w.offset != 0 || !w.data) return 0;
    const int64_t cin = conv_gemm_cin(x.dtype, w.dtype, x.v.size[1]);
    const int64_t lim = int64_t(1) << 31;
    if (!cin || x.v.size[1] * x.v.size[2] * x.v.size[3] * 2 >= lim ||
        w.v.size[0] * conv_filter_row(cin, w.v.size[2] * w.v.size[3]) * 2 >= lim)
      return 0;
    return cin;
  };

  // Rewrite: a nearest 2x upsample read only by an implicit-GEMM
  // convolution (UpsampleNearest then a 3x3 convolution: the decoders'
  // upsamplers) is never materialised; the convolution reads each
  // upsampled pixel from its source.
  for (auto& n : src) {
    if (n.op != OP_CONV) continue;
    const int uid = n.in[0];
    const GValue& uv = c.values[uid];
    if (uv.kind != VK_NODE || uv.base != uid || uv.producer < 0 || uses[uid] != 1) continue;
    if (std::find(outs.begin(), outs.end(), uid) != outs.end()) continue;
    const GNode& p = src[uv.producer];
    if (p.op != OP_UPSAMPLE || p.i0 != 2 || p.lane != n.lane || !conv_gemm_k(n, p.in[0])) continue;
    n.in[0] = p.in[0];
    n.conv_up = 1;
  }

  // Rewrite: the LayerNorm or RMSNorm of an image's token view [N, 1, P, C]
  // (a packed [N, C, P] seen as tokens; the Wan VAE's channel norms,
  // Vae/WanVae.cs:103-113) reads the image as it lies and writes the tokens
  // (i1 = 1), with no transposed copy first; a SiLU that alone reads such a
  // norm's output joins it (i2 = 1).
  auto one_row = [&](int id) {
    if (id < 0) return true;
    const View4& v = c.values[id].v;
    return !c.values[c.values[id].base].quant && v.size[0] == 1 && v.size[1] == 1 && v.size[2] == 1 &&
           (v.size[3] == 1 || v.stride[3] == 1);
  };
  for (auto& n : src) {
    if (n.op != OP_ROWNORM || n.i0 == 1 || n.rows_split[1] || n.rows_split[2]) continue;
    const GValue& x = c.values[n.in[0]];
    const View4& v = x.v;
    if (c.values[x.base].quant || x.offset != 0 || v.size[1] != 1 || v.size[2] < 2 || v.size[3] < 2 ||
        v.stride[2] != 1 || v.stride[3] != v.size[2] || (v.size[0] > 1 && v.stride[0] != v.size[2] * v.size[3]))
      continue;
    if (!one_row(n.in[1]) || !one_row(n.in[2])) continue;
    n.i1 = 1;
  }
  for (auto& n : src) {
    if (n.op != OP_ELEM || n.i0 != ELEM_SILU || n.in.empty() || n.in[0] < 0 || (n.in.size() > 1 && n.in[1] >= 0))
      continue;
    const int nid = n.in[0];
    const GValue& nv = c.values[nid];
    if (nv.kind != VK_NODE || nv.base != nid || nv.producer < 0 || uses[nid] != 1) continue;
    if (std::find(outs.begin(), outs.end(), nid) != outs.end()) continue;
    const GNode& p = src[nv.producer];
    if (p.op != OP_ROWNORM || !p.i1 || p.i2 || p.lane != n.lane || nv.dtype != c.values[n.out].dtype) continue;
    GNode fused = p;
    fused.out = n.out;
    fused.i2 = 1;
    n = fused;
  }

  // By default only where the product runs on the 256x256 tile with one head
  // per wave (gemm_qk_norm_fast): there the fused epilogue is a straight run
  // of shuffles and the two head-norm passes go away. On the narrower tiles
  // each head spans two waves that meet in LDS four times a slice, which
  // costs the product more than the passes it removes; NDX_FUSE_QK_NORM=1
  // (read at compile time) fuses there too, NDX_FUSE_QK_NORM=0 nowhere.
  const char* fuse_qk_env = getenv("NDX_FUSE_QK_NORM");
  const bool fuse_any = fuse_qk_env && fuse_qk_env[0] == '1';
  const bool fuse_qk = !(fuse_qk_env && fuse_qk_env[0] == '0');
  // Rewrite: the head norm + rotation of the q and k thirds of a QKV
  // projection (Rotate(HeadNorm(Linear(x))), QwenImageDit.cs:342-347;
  // Transformer.cs:37-64) runs in the projection's epilogue
  // (EPI_QK_NORM_ROPE): the two head-norm nodes' outputs become views of
  // the projection's q and k columns and the nodes never run. It applies
  // when the projection's output is read only by those two and through
  // views of its v third, the heads are 128 wide, and the tile the product
  // runs on can hold a head pair in its epilogue.
  for (size_t li = 0; li < src.size() && fuse_qk; li++) {
    GNode& L = src[li];
    if (L.op != OP_LINEAR || L.i0 != EPI_NONE || L.in.size() != 5 || L.in[3] >= 0 || L.in[4] >= 0) continue;
    const int lo = L.out;
    const GValue& ov = c.values[lo];
    const GValue& wv = c.values[L.in[1]];
    const int64_t N = wv.v.size[2], rows = ov.v.size[2];
    if (ov.kind != VK_NODE || ov.base != lo || N % 3 || (N / 3) % 128 || !is_packed(ov.v) || ov.v.size[3] != N) continue;
    if (std::find(outs.begin(), outs.end(), lo) != outs.end()) continue;
    const int64_t D = N / 3;
    int hnr[2] = {-1, -1};
    bool ok = true;
    // A view of lo within the v third: whole rows of N, columns [2D, 3D).
    auto in_v = [&](int id) {
      const GValue& v = c.values[id];
      const int64_t c0 = v.offset % N;
      return v.v.stride[3] == 1 && (v.v.size[2] <= 1 || v.v.stride[2] == N) && c0 >= 2 * D &&
             c0 + v.v.size[3] <= N;
    };
    for (size_t ni = 0; ni < src.size() && ok; ni++) {
      const GNode& u = src[ni];
      std::vector<int> reads(u.in.begin(), u.in.end());
      if (u.op == OP_ATTN)
        for (int j = 0; j < 3; j++) reads.insert(reads.end(), {u.seg[j][0], u.seg[j][1]});
      for (size_t k = 0; k < reads.size(); k++) {
        const int id = reads[k];
        if (id < 0 || c.values[id].base != lo || (int)ni == (int)li) continue;
        if (u.op == OP_HNR && k == 0) {
          const GValue& x = c.values[id];
          const int which = x.offset == 0 ? 0 : x.offset == D ? 1 : -1;
          if (which < 0 || hnr[which] >= 0 || x.v.size[3] != D || x.v.stride[3] != 1 || x.v.size[2] != rows ||
              x.v.stride[2] != N)
            ok = false;
          else
            hnr[which] = (int)ni;
        } else if (!in_v(id)) {
          ok = false;
        }
      }
    }
    for (int o : outs)
      if (c.values[o].base == lo && !in_v(o)) ok = false;
    if (!ok || hnr[0] < 0 || hnr[1] < 0) continue;
    const GNode& hq = src[hnr[0]];
    const GNode& hk = src[hnr[1]];
    auto same_dtype = [&](int a, int b) {
      return (a < 0 && b < 0) || (a >= 0 && b >= 0 && c.values[a].dtype == c.values[b].dtype);
    };
    if (hq.f0 != hk.f0 || hq.i0 != hk.i0 || D / hq.i0 != 128 || hq.in[2] != hk.in[2] || hq.in[3] != hk.in[3] ||
        !same_dtype(hq.in[1], hk.in[1]) || hq.lane != L.lane || hk.lane != L.lane ||
        c.values[hq.out].dtype != ov.dtype || c.values[hk.out].dtype != ov.dtype)
      continue;
    bool tables = true;
    for (int t : {hq.in[2], hq.in[3]})
      if (t >= 0 && (c.values[t].v.size[3] != 64 || !is_packed(c.values[t].v) || numel4(c.values[t].v) != rows * 64))
        tables = false;
    for (int wq : {hq.in[1], hk.in[1]})
      if (wq >= 0 && (!is_packed(c.values[wq].v) || numel4(c.values[wq].v) != 128 || c.values[wq].quant)) tables = false;
    if (!tables) continue;
    GemmArgs p{};
    const GValue& xv = c.values[L.in[0]];
    p.a_dtype = xv.dtype;
    p.w_dtype = wv.quant ? NDX_I8 : wv.dtype;
    p.c_dtype = ov.dtype;
    p.M = (int)rows;
    p.N = (int)N;
    p.K = (int)xv.v.size[3];
    p.batch = (int)(xv.v.size[0] * xv.v.size[1]);
    p.tile_hint = second_stream_tile(L, p.M);
    if (!fuse_any && !gemm_qk_norm_fast(p, (int)(2 * D))) continue;
    if (!gemm_qk_norm_ok(p, (int)(2 * D))) {
      // Where the chosen tile's waves do not hold half a head, the 64x128
      // or the 128x128 tile: the fusion then does not depend on which
      // stream the projection runs on.
      for (int hint : {3, 2}) {
        p.tile_hint = hint;
        if (gemm_qk_norm_ok(p, (int)(2 * D))) break;
        p.tile_hint = 0;
      }
      if (!p.tile_hint) continue;
      L.tile_hint = p.tile_hint;
    }
    // Views taken of the head norms' outputs (the query chunks of
    // Models/QwenImage/QwenImageDit.cs:353-373) name those outputs as their
    // base: they are re-expressed over the projection's buffer, a stride of
    // 1, D or rows * D (column, row, batch of the packed [.., rows, D]
    // output) becoming 1, N or rows * N. Any other view keeps the head norms
    // apart.
    auto rebase = [&](int hid, int64_t col0, bool apply) {
      for (int id = 0; id < (int)c.values.size(); id++) {
        GValue& v = c.values[id];
        if (id == hid || v.base != hid) continue;
        View4 nv = v.v;
        for (int i = 0; i < 4; i++) {
          const int64_t st = v.v.stride[i];
          if (v.v.size[i] <= 1) continue;
          if (st == 1) nv.stride[i] = 1;
          else if (st == D) nv.stride[i] = N;
          else if (st == rows * D) nv.stride[i] = rows * N;
          else return false;
        }
        if (apply) {
          const int64_t o = v.offset, b = o / (rows * D), r = o % (rows * D) / D, col = o % D;
          v.v = nv;
          v.offset = col0 + b * rows * N + r * N + col;
          v.base = lo;
        }
      }
      return true;
    };
    if (!rebase(hq.out, 0, false) || !rebase(hk.out, D, false)) continue;
    rebase(hq.out, 0, true);
    rebase(hk.out, D, true);
    L.i0 = EPI_QK_NORM_ROPE;
    L.f0 = hq.f0;
    L.in.resize(9, -1);
    L.in[5] = hq.in[1];
    L.in[6] = hk.in[1];
    L.in[7] = hq.in[2];
    L.in[8] = hq.in[3];
    for (int h : hnr) {
      const GValue x = c.values[src[h].in[0]];
      GValue& hv = c.values[src[h].out];
      hv.kind = VK_VIEW;
      hv.base = lo;
      hv.offset = x.offset;
      hv.v = x.v;
      hv.producer = -1;
    }
  }

  // Reachability from the outputs (through views to their owners).
  std::vector<char> need_node(src.size(), 0);
  std::function<void(int)> mark_value = [&](int id) {
    if (id < 0) return;
    const GValue& owner = c.values[c.values[id].base];
    if (owner.kind == VK_NODE && owner.producer >= 0 && !need_node[owner.producer]) {
      need_node[owner.producer] = 1;
      const GNode& n = src[owner.producer];
      if (n.op == OP_ATTN) {
        for (int j = 0; j < 3; j++) {
          mark_value(n.seg[j][0]);
          mark_value(n.seg[j][1]);
        }
        mark_value(n.in[3]);
      } else {
        for (int in : n.in) mark_value(in);
      }
    }
  };
  for (int o : outs) mark_value(o);

  // Whether value `owner` (and every view of it) is read by node `reader`
  // alone among the scheduled nodes, and is no output.
  const char* fuse_gn_env = getenv("NDX_FUSE_GN_NHWC");
  const bool fuse_gn_nhwc = !(fuse_gn_env && fuse_gn_env[0] == '0');
  auto sole_reader = [&](int owner, size_t reader) {
    for (int o : outs)
      if (c.values[o].base == owner) return false;
    for (size_t k = 0; k < src.size(); k++) {
      if (!need_node[k] || k == reader) continue;
      const GNode& u = src[k];
      std::vector<int> reads(u.in.begin(), u.in.end());
      if (u.op == OP_ATTN)
        for (int j = 0; j < 3; j++) reads.insert(reads.end(), {u.seg[j][0], u.seg[j][1]});
      for (int id : reads)
        if (id >= 0 && c.values[id].base == owner) return false;
    }
    return true;
  };

  // Schedule in creation order, packing what a kernel cannot read as is.
  for (size_t i = 0; i < src.size(); i++) {
    if (!need_node[i]) continue;
    GNode n = src[i];
    c.lane = n.lane;
    auto rows_ok = [&](int id) {
      int64_t ld, bs;
      return id < 0 || rows_layout(c.values[id].v, ld, bs);
    };
    auto ensure_rows = [&](int& id) {
      if (id >= 0 && !c.values[c.values[id].base].quant && !rows_ok(id)) id = c.pack(id, sched);
    };
    auto ensure_packed = [&](int& id) {
      if (id >= 0 && !(is_packed(c.values[id].v))) id = c.pack(id, sched);
    };
    switch (n.op) {
      case OP_LINEAR:
        ensure_rows(n.in[0]);
        ensure_packed(n.in[2]);
        ensure_rows(n.in[4]);
        if (n.in[3] >= 0) {
          const GValue& gt = c.values[n.in[3]];
          if (gt.v.size[3] > 1 && gt.v.stride[3] != 1) n.in[3] = c.pack(n.in[3], sched);
          else if (gt.v.size[2] > 1 && !n.rows_split[3]) ensure_rows(n.in[3]);
        }
        {
          const GValue& w = c.values[n.in[1]];
          if (!w.quant && w.v.size[3] > 1 && w.v.stride[3] != 1) n.in[1] = c.pack(n.in[1], sched);
        }
        break;
      case OP_ATTN: {
        for (int j = 0; j < 3; j++) {
          if (n.seg[j][1] >= 0) continue;
          ensure_rows(n.seg[j][0]);
        }
        const View4& qv = c.values[n.in[0]].v;
        const View4& kv = c.values[n.in[1]].v;
        const View4& vv = c.values[n.in[2]].v;
        n.scratch_bytes = attention_scratch_bytes((int)(qv.size[0] * qv.size[1]), (int)qv.size[2], (int)kv.size[2], n.i0,
                                                  (int)(qv.size[3] / n.i0), (int)(vv.size[3] / n.i0),
                                                  c.values[n.in[0]].dtype);
        break;
      }
      case OP_HNR:
        ensure_rows(n.in[0]);
        ensure_packed(n.in[1]);
        ensure_packed(n.in[2]);
        ensure_packed(n.in[3]);
        break;
      case OP_ROWNORM:
        if (n.i1) break;  // a channel norm: the image and one-row parameters as they are
        ensure_rows(n.in[0]);
        for (int j = 1; j < 3; j++) {
          if (n.in[j] < 0) continue;
          const GValue& pv = c.values[n.in[j]];
          if (pv.v.size[3] > 1 && pv.v.stride[3] != 1) n.in[j] = c.pack(n.in[j], sched);
          else if (pv.v.size[2] > 1 && !n.rows_split[j]) ensure_rows(n.in[j]);
        }
        break;
      case OP_GROUPNORM: {
        for (auto& id : n.in)
          if (id >= 0 && !c.values[c.values[id].base].quant) ensure_packed(id);
        const View4& xv = c.values[n.in[0]].v;
        const int64_t count = xv.size[1] / n.i0 * xv.size[2] * xv.size[3];
        // The split partials, then (mean, rstd) per (n, group) for the NHWC apply.
        n.scratch_bytes = int64_t(xv.size[0]) * n.i0 * (group_norm_splits(count) * 3 + 2) * sizeof(float);
        break;
      }
      case OP_PATCH:
      case OP_SAMPLE:
      case OP_SOFTMAX:
        for (auto& id : n.in)
          if (id >= 0 && !c.values[c.values[id].base].quant) ensure_packed(id);
        break;
      case OP_CONV: {
        for (size_t j = 1; j < n.in.size(); j++)
          if (n.in[j] >= 0 && !c.values[c.values[n.in[j]].base].quant) ensure_packed(n.in[j]);
        const int64_t cin_k = conv_gemm_k(n, n.in[0]);
        if (!cin_k) {
          if (n.conv_up) fail(NDX_UNSUPPORTED, "a fused upsample needs the implicit-GEMM convolution");
          ensure_packed(n.in[0]);
          break;
        }
        // The implicit GEMM reads its input in NHWC: an image whose view
        // already lies that way (a norm's token rows seen as an image) in
        // place, any other copied to NHWC just before. The filter is
        // reordered once.
        const GValue& x = c.values[n.in[0]];
        const View4& v = x.v;
        bool nhwc = x.offset % 8 == 0 && v.stride[1] == 1 && v.stride[3] == v.size[1] &&
                          v.stride[2] == v.size[3] * v.size[1] &&
                          (v.size[0] == 1 || v.stride[0] == v.size[1] * v.size[2] * v.size[3]);
        // A group norm read by this convolution alone writes NHWC itself
        // (NDX_FUSE_GN_NHWC=0, read at compile time, keeps the copy).
        if (!nhwc && fuse_gn_nhwc && x.kind == VK_NODE && x.base == n.in[0] && x.offset == 0 && is_packed(v) &&
            x.producer >= 0 && src[x.producer].op == OP_GROUPNORM && sole_reader(n.in[0], i)) {
          const GValue& gx = c.values[src[x.producer].in[0]];
          if (group_norm_nhwc_ok(gx.dtype, x.dtype, v.size[1], v.size[2] * v.size[3], src[x.producer].i0) &&
              gx.offset % 8 == 0 && is_packed(gx.v)) {
            for (auto it = sched.rbegin(); it != sched.rend(); ++it)
              if (it->op == OP_GROUPNORM && it->out == n.in[0]) {
                it->i2 = 1;
                View4& nv = c.values[n.in[0]].v;
                nv.stride[1] = 1;
                nv.stride[3] = nv.size[1];
                nv.stride[2] = nv.size[3] * nv.size[1];
                nv.stride[0] = nv.size[2] * nv.size[3] * nv.size[1];
                nhwc = true;
                break;
              }
          }
        }
        if (!nhwc) {
          ensure_packed(n.in[0]);
          GNode t;
          t.op = OP_NHWC;
          t.lane = n.lane;
          t.in = {n.in[0]};
          t.out = c.new_owner(c.values[n.in[0]].dtype, c.values[n.in[0]].v, 4);
          sched.push_back(t);
          n.in[0] = t.out;
        }
        n.conv_cin_k = cin_k;
        n.in[1] = c.reordered_filter(n.in[1], cin_k);
        n.i5 = 1;
        break;
      }
      default:
        break;
    }
    sched.push_back(n);
  }

  c.lane = 0;
  // Outputs must be packed owners: copy a view out.
  for (auto& o : outs) {
    const GValue& v = c.values[o];
    if (v.kind == VK_NODE && v.base == o && v.offset == 0) continue;
    o = c.pack(o, sched);
  }

  // Pair adjacent independent linears of equal N and K (the image and text
  // streams' projections): they run as one launch, the second's row tiles
  // after the first's (i5 = 1 on the first, 2 on the second).
  for (size_t i = 0; i + 1 < sched.size(); i++) {
    GNode& x = sched[i];
    GNode& y = sched[i + 1];
    if (x.op != OP_LINEAR || y.op != OP_LINEAR || x.i5 || y.i5 || x.lane != y.lane) continue;
    if (x.i0 == EPI_QK_NORM_ROPE || y.i0 == EPI_QK_NORM_ROPE) continue;
    const GValue& wx = c.values[x.in[1]];
    const GValue& wy = c.values[y.in[1]];
    const GValue& ax = c.values[x.in[0]];
    const GValue& ay = c.values[y.in[0]];
    if (wx.quant || wy.quant || ax.dtype != ay.dtype || wx.dtype != wy.dtype) continue;
    if (ax.dtype != NDX_BF16 && ax.dtype != NDX_F16) continue;
    if (wx.v.size[2] != wy.v.size[2] || ax.v.size[3] != ay.v.size[3]) continue;
    if (ax.v.size[0] * ax.v.size[1] != ay.v.size[0] * ay.v.size[1]) continue;
    if (ax.v.size[2] <= 4 || ay.v.size[2] <= 4) continue;  // GEMVs stay single
    if (!gemm_pair_pays(ax.v.size[2], ay.v.size[2], wx.v.size[2], ax.v.size[3], ax.v.size[0] * ax.v.size[1]))
      continue;
    bool dependent = false;
    for (int id : y.in)
      if (id >= 0 && c.values[id].base == c.values[x.out].base) dependent = true;
    if (dependent) continue;
    x.i5 = 1;
    y.i5 = 2;
    i++;
  }

  auto* m = new ndx_model();
  try {
    m->dev = g->dev;
    m->consts = g->consts;
    m->values = c.values;
    m->nodes = sched;
    m->outputs = outs;
    m->inputs.assign(g->n_inputs, -1);
    for (size_t i = 0; i < m->values.size(); i++)
      if (m->values[i].kind == VK_INPUT) m->inputs[m->values[i].input_index] = (int)i;
    m->out_slot.assign(m->values.size(), -1);
    for (size_t k = 0; k < outs.size(); k++) {
      if (m->out_slot[outs[k]] >= 0) fail(NDX_INVALID_ARG, "the same value is an output twice");
      m->out_slot[outs[k]] = (int)k;
    }
    for (auto& n : m->nodes) prof_info(n, m->values);
    // NDX_DUMP_SCHEDULE=1: the schedule on stderr, one node a line (kernel
    // family, lane, output shape, each input's shape and strides).
    if (const char* dump = getenv("NDX_DUMP_SCHEDULE"); dump && dump[0] == '1') {
      auto shape = [&](int id) {
        if (id < 0) return std::string("-");
        const GValue& v = m->values[id];
        char b[160];
        snprintf(b, sizeof b, "%s[%lld,%lld,%lld,%lld]/[%lld,%lld,%lld,%lld]", dtype_name(v.dtype),
                 (long long)v.v.size[0], (long long)v.v.size[1], (long long)v.v.size[2], (long long)v.v.size[3],
                 (long long)v.v.stride[0], (long long)v.v.stride[1], (long long)v.v.stride[2],
                 (long long)v.v.stride[3]);
        return std::string(b);
      };
      for (size_t i = 0; i < m->nodes.size(); i++) {
        const GNode& n = m->nodes[i];
        std::string line = std::to_string(i) + " " + n.family + " lane" + std::to_string(n.lane) + " -> " +
                           shape(n.out) + " <-";
        for (int id : n.in) line += " " + shape(id);
        fprintf(stderr, "[ndx schedule] %s\n", line.c_str());
      }
    }
    for (size_t i = 0; i + 1 < m->nodes.size(); i++)
      if (m->nodes[i].op == OP_LINEAR && m->nodes[i].i5 == 1) {
        m->nodes[i].flops += m->nodes[i + 1].flops;
        m->nodes[i].bytes += m->nodes[i + 1].bytes;
      }
    for (const auto* t : g->consts->tensors) m->persistent += t->bytes;

    // Lifetimes and the arena.
    const int nv = (int)m->values.size();
    std::vector<int> def(nv, -1), last(nv, -1);
    for (int i = 0; i < (int)m->nodes.size(); i++) {
      const GNode& n = m->nodes[i];
      def[n.out] = i;
      auto use = [&](int id) {
        if (id >= 0) last[m->values[id].base] = std::max(last[m->values[id].base], i);
      };
      for (int id : n.in) use(id);
      if (n.op == OP_ATTN)
        for (int j = 0; j < 3; j++) {
          use(n.seg[j][0]);
          use(n.seg[j][1]);
        }
    }
    m->arena_off.assign(nv, -1);
    struct Live {
      int64_t off, size;
      int last;
    };
    // Each lane gets a region of its own: a value never takes bytes that a
    // value of the other lane held, so freeing memory never makes one
    // stream wait for the other (only data does). Lane 1's region follows
    // lane 0's.
    std::vector<Live> live[2];
    int64_t top[2] = {0, 0};
    std::vector<int8_t> region(nv, 0);
    std::vector<int8_t> scratch_region(m->nodes.size(), 0);
    // First fit of [size] bytes among the region's live ranges; returns the offset.
    auto place = [&](int r, int64_t bytes, int until) {
      int64_t size = (bytes + 255) & ~int64_t(255);
      auto& lv = live[r];
      std::sort(lv.begin(), lv.end(), [](const Live& a, const Live& b) { return a.off < b.off; });
      int64_t off = 0;
      for (const Live& l : lv) {
        if (off + size <= l.off) break;
        off = std::max(off, l.off + l.size);
      }
      lv.push_back({off, size, until});
      top[r] = std::max(top[r], off + size);
      return off;
    };
    for (int i = 0; i < (int)m->nodes.size(); i++) {
      GNode& node = m->nodes[i];
      for (auto& lv : live)
        lv.erase(std::remove_if(lv.begin(), lv.end(), [&](const Live& l) { return l.last < i; }), lv.end());
      // The second of a paired linear is written by the first's launch: its
      // output is placed (and live) from there.
      if (node.op == OP_LINEAR && node.i5 == 2) continue;
      const int r = node.lane & 1;
      for (int k = 0; k < (node.op == OP_LINEAR && node.i5 == 1 ? 2 : 1); k++) {
        const int id = m->nodes[i + k].out;
        if (m->out_slot[id] < 0) {
          m->arena_off[id] =
              place(r, int64_t(m->values[id].buffer_elems) * dtype_size(m->values[id].dtype), std::max(last[id], i + k));
          region[id] = (int8_t)r;
        }
      }
      if (node.scratch_bytes > 0) {
        node.scratch_off = place(r, node.scratch_bytes, i);
        scratch_region[i] = (int8_t)r;
      }
    }
    const int64_t base1 = (top[0] + 255) & ~int64_t(255);
    for (int id = 0; id < nv; id++)
      if (m->arena_off[id] >= 0 && region[id] == 1) m->arena_off[id] += base1;
    for (size_t i = 0; i < m->nodes.size(); i++)
      if (m->nodes[i].scratch_bytes > 0 && scratch_region[i] == 1) m->nodes[i].scratch_off += base1;
    // The arena (the reference's temporary resource) is allocated by the
    // first run that uses it, as DmlDevice sizes its temporary buffer at
    // dispatch; a model run only through ndx_model_run_into_static_async
    // never allocates one.
    m->arena_bytes = (size_t)(top[1] > 0 ? base1 + top[1] : top[0]);
    plan_lanes(m, last);
    for (auto& n : m->nodes) m->kernels += (n.op == OP_JOIN) ? (int)n.in.size() : 1;
  } catch (...) {
    delete m;
    throw;
  }
  *out = m;
  NDX_CATCH
}

// ---- run -------------------------------------------------------------------

namespace {

struct Runner {
  ndx_model* m;
  ndx_tensor* const* in;
  std::vector<void*> out_ptr;
  char* arena = nullptr;  // the temporary memory of this run

  char* base_ptr(int base) {
    const GValue& b = m->values[base];
    switch (b.kind) {
      case VK_INPUT: return (char*)in[b.input_index]->ptr;
      case VK_CONST: return (char*)b.data->ptr;
      default:
        if (m->out_slot[base] >= 0) return (char*)out_ptr[m->out_slot[base]];
        // Only an owner the planner placed has bytes: anything else is a
        // compiler error, refused here rather than read from the device.
        if (b.base != base || m->arena_off[base] < 0) fail(NDX_INVALID_STATE, "a value with no storage was read");
        return arena + m->arena_off[base];
    }
  }
  void* ptr(int id) {
    if (id < 0) return nullptr;
    const GValue& v = m->values[id];
    if (v.quant) return base_ptr(v.base);
    return base_ptr(v.base) + v.offset * dtype_size(v.dtype);
  }
  const GValue& val(int id) { return m->values[id]; }

  // The GEMM of a linear node (x [B,1,M,K] rows, W [N,K], epilogue inputs).
  GemmArgs linear_args(const GNode& n) {
    const GValue& x = val(n.in[0]);
    const GValue& w = val(n.in[1]);
    const GValue& o = val(n.out);
    GemmArgs a{};
    int64_t ld, bs;
    rows_layout(x.v, ld, bs);
    a.a = ptr(n.in[0]);
    a.lda = ld;
    a.batch_a = bs;
    a.a_dtype = x.dtype;
    a.M = (int)x.v.size[2];
    a.K = (int)x.v.size[3];
    a.batch = (int)(x.v.size[0] * x.v.size[1]);
    a.N = (int)w.v.size[2];
    if (w.quant) {
      a.w = w.data->ptr;
      a.ldw = w.v.size[3];
      a.w_dtype = NDX_I8;
      a.scales = w.scales->ptr;
      a.qblock = w.qblock;
      a.lds = w.v.size[3] / w.qblock;
      a.s_dtype = w.scales->dtype;
    } else {
      a.w = ptr(n.in[1]);
      a.ldw = w.v.size[2] > 1 ? w.v.stride[2] : w.v.size[3];
      a.w_dtype = w.dtype;
    }
    a.batch_w = 0;
    a.tile_hint = n.tile_hint ? n.tile_hint : second_stream_tile(n, a.M);
    a.c = ptr(n.out);
    // A SwiGLU writes one column per interleaved (gate, up) pair: N / 2.
    a.ldc = n.i0 == EPI_SWIGLU ? a.N / 2 : a.N;
    a.batch_c = int64_t(a.M) * a.ldc;
    a.c_dtype = o.dtype;
    // Every row the product writes must lie in its output's buffer.
    if (o.offset + int64_t(a.batch) * a.batch_c > m->values[o.base].buffer_elems)
      fail(NDX_INVALID_STATE, "a linear's output rows overrun its buffer");
    if (n.in[2] >= 0) {
      a.bias = ptr(n.in[2]);
      a.bias_dtype = val(n.in[2]).dtype;
    }
    a.epilogue = n.i0;
    if (n.in[3] >= 0) {
      const GValue& gt = val(n.in[3]);
      a.gate = ptr(n.in[3]);
      a.gate_dtype = gt.dtype;
      a.batch_gate = (gt.v.size[0] > 1) ? gt.v.stride[0] : (gt.v.size[1] > 1 ? gt.v.stride[1] : 0);
      a.ldg = gt.v.size[2] > 1 ? gt.v.stride[2] : 0;
      a.gate_split = n.rows_split[3];
      a.gate_split_off = n.rows_off[3];
    }
    if (n.in[4] >= 0) {
      const GValue& r = val(n.in[4]);
      rows_layout(r.v, ld, bs);
      a.resid = ptr(n.in[4]);
      a.ldr = ld;
      a.batch_r = bs;
      a.r_dtype = r.dtype;
    }
    if (n.i0 == EPI_QK_NORM_ROPE) {
      a.qk_cols = 2 * (a.N / 3);
      a.norm_eps = n.f0;
      if (n.in[5] >= 0) {
        a.norm_q = ptr(n.in[5]);
        a.norm_k = ptr(n.in[6]);
        a.norm_dtype = val(n.in[5]).dtype;
      }
      if (n.in[7] >= 0) {
        a.rope_cos = (const float*)ptr(n.in[7]);
        a.rope_sin = (const float*)ptr(n.in[8]);
      }
    }
    return a;
  }

  void elem(int op, int a, int b, int o, float scale, float bias, hipStream_t s, const View4* out_view = nullptr,
            void* out_p = nullptr) {
    ElemArgs e{};
    e.in0 = ptr(a);
    e.v0 = val(a).v;
    e.dt0 = val(a).dtype;
    if (b >= 0) {
      e.in1 = ptr(b);
      e.v1 = val(b).v;
      e.dt1 = val(b).dtype;
    }
    e.out = out_p ? out_p : ptr(o);
    e.vo = out_view ? *out_view : val(o).v;
    e.dto = val(o).dtype;
    e.op = op;
    e.scale = scale;
    e.bias = bias;
    launch_elementwise(e, s);
  }

  void launch(const GNode& n, hipStream_t s) {
    switch (n.op) {
      case OP_ELEM:
        elem(n.i0, n.in[0], n.in.size() > 1 ? n.in[1] : -1, n.out, n.f0, n.f1, s);
        break;
      case OP_JOIN: {
        const GValue& o = val(n.out);
        int64_t at = 0;
        for (int id : n.in) {
          View4 sub = o.v;
          sub.size[n.i0] = val(id).v.size[n.i0];
          char* p = (char*)ptr(n.out) + at * o.v.stride[n.i0] * dtype_size(o.dtype);
          elem(ELEM_COPY, id, -1, n.out, 1.f, 0.f, s, &sub, p);
          at += sub.size[n.i0];
        }
        break;
      }
      case OP_LINEAR: {
        if (n.i5 == 2) break;  // launched with the node before it
        const GemmArgs a = linear_args(n);
        if (n.i5 == 1) {
          const GemmArgs b = linear_args(*(&n + 1));
          if (!launch_gemm_pair(a, b, s)) {
            launch_gemm(a, s);
            launch_gemm(b, s);
          }
        } else {
          launch_gemm(a, s);
        }
        break;
      }
      case OP_GEMM: {
        GemmGenericArgs a{};
        const GValue& va = val(n.in[0]);
        const GValue& vb = val(n.in[1]);
        const GValue& o = val(n.out);
        a.a = ptr(n.in[0]);
        a.va = va.v;
        a.a_dtype = va.dtype;
        a.b = ptr(n.in[1]);
        a.vb = vb.v;
        a.b_dtype = vb.dtype;
        if (n.in[2] >= 0) {
          a.c = ptr(n.in[2]);
          a.vc = val(n.in[2]).v;
          a.c_dtype = val(n.in[2]).dtype;
        }
        a.out = ptr(n.out);
        a.out_dtype = o.dtype;
        a.M = o.v.size[2];
        a.N = o.v.size[3];
        a.K = n.i0 ? va.v.size[2] : va.v.size[3];
        a.batch0 = o.v.size[0];
        a.batch1 = o.v.size[1];
        a.trans_a = n.i0;
        a.trans_b = n.i1;
        a.alpha = n.f0;
        a.beta = n.f1;
        launch_gemm_generic(a, s);
        break;
      }
      case OP_ATTN: {
        AttnArgs a{};
        const GValue& q = val(n.in[0]);
        const GValue& k = val(n.in[1]);
        const GValue& v = val(n.in[2]);
        const GValue& o = val(n.out);
        AttnSeg* segs[3] = {&a.q, &a.k, &a.v};
        const GValue* vals[3] = {&q, &k, &v};
        for (int j = 0; j < 3; j++) {
          AttnSeg& sg = *segs[j];
          for (int p = 0; p < 2; p++) {
            int id = n.seg[j][p];
            if (id < 0) {
              sg.ptr[p] = nullptr;
              continue;
            }
            int64_t ld, bs;
            rows_layout(val(id).v, ld, bs);
            sg.ptr[p] = ptr(id);
            sg.ld[p] = ld;
            sg.batch[p] = bs;
          }
          sg.rows0 = n.seg[j][1] >= 0 ? val(n.seg[j][0]).v.size[2] : vals[j]->v.size[2];
          if (n.seg[j][1] < 0) {
            sg.ptr[1] = sg.ptr[0];
            sg.ld[1] = sg.ld[0];
            sg.batch[1] = sg.batch[0];
          }
        }
        a.out[0] = a.out[1] = ptr(n.out);
        a.out_rows0 = o.v.size[2];
        a.out_ld[0] = a.out_ld[1] = o.v.size[3];
        a.out_batch[0] = a.out_batch[1] = o.v.size[2] * o.v.size[3];
        a.B = (int)(q.v.size[0] * q.v.size[1]);
        a.T = (int)q.v.size[2];
        a.S = (int)k.v.size[2];
        a.H = n.i0;
        a.d = (int)(q.v.size[3] / n.i0);
        a.dv = (int)(v.v.size[3] / n.i0);
        a.scale = n.f0;
        a.dtype = q.dtype;
        a.mask_kind = n.i1;
        if (n.in[3] >= 0) {
          const GValue& mk = val(n.in[3]);
          a.mask = (const int32_t*)ptr(n.in[3]);
          // [b, h, t, s] strides; a size-1 axis broadcasts.
          for (int i = 0; i < 4; i++) a.mask_stride[i] = mk.v.size[i] == 1 ? 0 : mk.v.stride[i];
        }
        launch_attention(a, n.scratch_bytes > 0 ? arena + n.scratch_off : nullptr, s);
        break;
      }
      case OP_HNR: {
        HeadNormRotateArgs a{};
        const GValue& x = val(n.in[0]);
        const GValue& o = val(n.out);
        int64_t ld, bs;
        rows_layout(x.v, ld, bs);
        a.x = ptr(n.in[0]);
        a.ldx = ld;
        a.batch_x = bs;
        a.x_dtype = x.dtype;
        a.y = ptr(n.out);
        a.ldy = o.v.size[3];
        a.batch_y = o.v.size[2] * o.v.size[3];
        a.y_dtype = o.dtype;
        if (n.in[1] >= 0) {
          a.weight = ptr(n.in[1]);
          a.w_dtype = val(n.in[1]).dtype;
        }
        a.cos = (const float*)ptr(n.in[2]);
        a.sin = (const float*)ptr(n.in[3]);
        a.B = (int)(x.v.size[0] * x.v.size[1]);
        a.T = (int)x.v.size[2];
        a.H = n.i0;
        a.d = (int)(x.v.size[3] / n.i0);
        a.eps = n.f0;
        launch_head_norm_rotate(a, s);
        break;
      }
      case OP_ROWNORM: {
        if (n.i1) {
          ChannelNormArgs a{};
          const GValue& x = val(n.in[0]);
          a.x = ptr(n.in[0]);
          a.x_dtype = x.dtype;
          a.y = ptr(n.out);
          a.y_dtype = val(n.out).dtype;
          a.N = x.v.size[0];
          a.P = x.v.size[2];
          a.C = x.v.size[3];
          if (n.in[1] >= 0) {
            a.weight = ptr(n.in[1]);
            a.w_dtype = val(n.in[1]).dtype;
          }
          if (n.in[2] >= 0) {
            a.bias = ptr(n.in[2]);
            a.b_dtype = val(n.in[2]).dtype;
          }
          a.eps = n.f0;
          a.mode = n.i0;
          a.silu = n.i2;
          launch_channel_norm(a, s);
          break;
        }
        RowNormArgs a{};
        const GValue& x = val(n.in[0]);
        const GValue& o = val(n.out);
        int64_t ld, bs;
        rows_layout(x.v, ld, bs);
        a.x = ptr(n.in[0]);
        a.ldx = ld;
        a.x_dtype = x.dtype;
        a.y = ptr(n.out);
        a.ldy = o.v.size[3];
        a.y_dtype = o.dtype;
        a.D = (int)x.v.size[3];
        a.rows = x.v.size[0] * x.v.size[1] * x.v.size[2];
        a.rows_per_batch = x.v.size[2];
        // A row's source offset: (row / rows_per_batch) * bs + (row % rows_per_batch) * ld.
        a.mode = n.i0;
        a.eps = n.f0;
        auto param = [&](int id, const void*& p, int64_t& batch, int64_t& ld, int& dt) {
          if (id < 0) return;
          const GValue& pv = val(id);
          p = ptr(id);
          dt = pv.dtype;
          // Per-batch rows (modulation) when the parameter has a batch > 1,
          // a row per token when it has tokens.
          batch = pv.v.size[0] > 1 ? pv.v.stride[0] : (pv.v.size[1] > 1 ? pv.v.stride[1] : 0);
          ld = pv.v.size[2] > 1 ? pv.v.stride[2] : 0;
        };
        param(n.in[1], a.weight, a.batch_w, a.ldw, a.w_dtype);
        param(n.in[2], a.bias, a.batch_b, a.ldb, a.b_dtype);
        a.split = std::max(n.rows_split[1], n.rows_split[2]);
        a.split_w_off = n.rows_off[1];
        a.split_b_off = n.rows_off[2];
        a.batch_x = bs;
        launch_row_norm(a, s);
        break;
      }
      case OP_GROUPNORM: {
        GroupNormArgs a{};
        const GValue& x = val(n.in[0]);
        a.x = ptr(n.in[0]);
        a.y = ptr(n.out);
        a.dtype = x.dtype;
        a.y_dtype = val(n.out).dtype;
        a.N = (int)x.v.size[0];
        a.C = (int)x.v.size[1];
        a.HW = (int)(x.v.size[2] * x.v.size[3]);
        a.groups = n.i0;
        a.eps = n.f0;
        a.silu = n.i1;
        if (n.in[1] >= 0) {
          a.weight = ptr(n.in[1]);
          a.w_dtype = val(n.in[1]).dtype;
        }
        if (n.in[2] >= 0) {
          a.bias = ptr(n.in[2]);
          a.w_dtype = val(n.in[2]).dtype;
        }
        a.partial = (float*)(arena + n.scratch_off);
        a.splits = group_norm_splits(int64_t(a.C / a.groups) * a.HW);
        a.nhwc = n.i2;
        launch_group_norm(a, s);
        break;
      }
      case OP_CONV: {
        ConvArgs a{};
        const GValue& x = val(n.in[0]);
        const GValue& w = val(n.in[1]);
        const GValue& o = val(n.out);
        a.x = ptr(n.in[0]);
        a.x_dtype = x.dtype;
        if (w.quant) {
          a.w = w.data->ptr;
          a.w_dtype = NDX_I8;
          a.scales = w.scales->ptr;
          a.qblock = w.qblock;
          a.s_dtype = w.scales->dtype;
        } else {
          a.w = ptr(n.in[1]);
          a.w_dtype = w.dtype;
        }
        if (n.in[2] >= 0) {
          a.bias = ptr(n.in[2]);
          a.bias_dtype = val(n.in[2]).dtype;
        }
        a.resid = ptr(n.in[3]);
        a.y = ptr(n.out);
        a.y_dtype = o.dtype;
        a.N = (int)x.v.size[0];
        a.Cin = (int)x.v.size[1];
        a.H = (int)x.v.size[2] << n.conv_up;
        a.W = (int)x.v.size[3] << n.conv_up;
        a.Cout = (int)o.v.size[1];
        a.kh = n.i3;
        a.kw = n.i4;
        a.stride = n.i0;
        a.pad = n.i1;
        a.Ho = (int)o.v.size[2];
        a.Wo = (int)o.v.size[3];
        a.cin_k = (int)n.conv_cin_k;
        a.up = n.conv_up;
        if (n.i5) launch_conv_gemm(a, s);
        else launch_conv2d(a, s);
        break;
      }
      case OP_NHWC: {
        // A packed NCHW value, or (i1) the token view [N, 1, P, C] of one.
        const GValue& x = val(n.in[0]);
        const int64_t c = n.i1 ? x.v.size[3] : x.v.size[1];
        const int64_t hw = n.i1 ? x.v.size[2] : x.v.size[2] * x.v.size[3];
        launch_nchw_to_nhwc(ptr(n.in[0]), ptr(n.out), x.dtype, x.v.size[0], c, hw, s);
        break;
      }
      case OP_UPSAMPLE: {
        UpsampleArgs a{};
        const GValue& x = val(n.in[0]);
        a.x = ptr(n.in[0]);
        a.vx = x.v;
        a.y = ptr(n.out);
        a.dtype = x.dtype;
        a.scale = n.i0;
        a.N = x.v.size[0];
        a.C = x.v.size[1];
        a.H = x.v.size[2];
        a.W = x.v.size[3];
        launch_upsample(a, s);
        break;
      }
      case OP_SOFTMAX: {
        const View4& o = val(n.out).v;
        launch_softmax(ptr(n.in[0]), ptr(n.out), val(n.out).dtype, o.size[0] * o.size[1] * o.size[2], o.size[3], n.f0,
                       s);
        break;
      }
      case OP_SAMPLE:
        launch_guided_euler((const float*)ptr(n.in[0]), (const float*)ptr(n.in[1]), (const float*)ptr(n.in[2]),
                            (const float*)ptr(n.in[3]), (float*)ptr(n.out), numel4(val(n.out).v), s);
        break;
      case OP_PATCH: {
        PatchArgs a{};
        a.x = ptr(n.in[0]);
        a.y = ptr(n.out);
        a.x_dtype = val(n.in[0]).dtype;
        a.y_dtype = val(n.out).dtype;
        a.p = n.i0;
        a.inverse = n.i1;
        a.channel_last = n.i5;
        a.N = (int)val(n.out).v.size[0];
        a.C = n.i2;
        a.H = n.i3;
        a.W = n.i4;
        launch_patch(a, s);
        break;
      }
    }
  }
};

void check_inputs(ndx_model* m, ndx_tensor* const* inputs, int32_t n_inputs) {
  if (n_inputs != (int)m->inputs.size())
    fail(NDX_INVALID_ARG, "expected " + std::to_string(m->inputs.size()) + " inputs, got " + std::to_string(n_inputs));
  for (int i = 0; i < n_inputs; i++) {
    if (!inputs[i]) fail(NDX_INVALID_ARG, "input " + std::to_string(i) + " is null");
    int id = m->inputs[i];
    if (id < 0) continue;
    const GValue& v = m->values[id];
    ndx_tensor* t = inputs[i];
    if (t->dev != m->dev) fail(NDX_INVALID_ARG, "input " + std::to_string(i) + " is on another device");
    if (t->dtype != v.dtype) fail(NDX_INVALID_ARG, "input " + std::to_string(i) + " is " + dtype_name(t->dtype) + ", the graph declared " + dtype_name(v.dtype));
    if (t->numel() != numel4(v.v))
      fail(NDX_INVALID_ARG, "input " + std::to_string(i) + " has " + std::to_string(t->numel()) + " elements, the graph declared " + shape_str(v.v, v.dtype));
  }
}

// The model's own arena, allocated by its first run.
char* model_arena(ndx_model* m) {
  if (!m->arena && m->arena_bytes > 0) {
    m->arena_alloc = pool_round(m->arena_bytes);
    m->arena = m->dev->alloc(m->arena_alloc);
  }
  return (char*)m->arena;
}

// Checks the caller's output tensors and records their pointers.
void bind_outputs(ndx_model* m, Runner& r, ndx_tensor* const* outputs, int32_t n_outputs) {
  if (!outputs) fail(NDX_INVALID_ARG, "outputs is null");
  if (n_outputs != (int)m->outputs.size()) fail(NDX_INVALID_ARG, "wrong number of outputs");
  for (int k = 0; k < n_outputs; k++) {
    const GValue& v = m->values[m->outputs[k]];
    ndx_tensor* t = outputs[k];
    if (!t || t->dtype != v.dtype || t->numel() != numel4(v.v) || t->dev != m->dev)
      fail(NDX_INVALID_ARG, "output " + std::to_string(k) + " is not " + shape_str(v.v, v.dtype));
    r.out_ptr.push_back(t->ptr);
  }
}

// Queues every node. With profile false no timing events are recorded (and
// none created), whatever the model's profiling setting.
void run_nodes(ndx_model* m, Runner& r, bool profile = true) {
  hipStream_t s = m->dev->stream;
  hipStream_t st[2] = {s, m->two_lanes ? m->dev->aux_stream() : s};
  const int ne = (int)m->lane_events.size();
  if (m->two_lanes) {
    // The second lane starts after what the device stream holds (inputs,
    // the previous run) and the device stream ends after the second lane.
    hip_check(hipEventRecord(m->lane_events[ne - 2], s), "hipEventRecord");
    hip_check(hipStreamWaitEvent(st[1], m->lane_events[ne - 2], 0), "hipStreamWaitEvent");
  }
  const bool filtered = profile && m->profiling && !m->prof_filter.empty();
  const bool full = profile && m->profiling && !filtered;
  size_t need = m->nodes.size() * 2;
  while (full && m->events.size() < need) {
    hipEvent_t e;
    // Timing only: no cache writeback when recorded (it would slow what follows).
    hip_check(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreate");
    m->events.push_back(e);
  }
  for (size_t i = 0; i < m->nodes.size(); i++) {
    const GNode& n = m->nodes[i];
    hipStream_t ns = st[n.lane & 1];
    if (m->two_lanes)
      for (int t = 0; t < 2; t++)
        if (m->waits[i][t] >= 0)
          hip_check(hipStreamWaitEvent(ns, m->lane_events[m->signal[m->waits[i][t]]], 0), "hipStreamWaitEvent");
    const bool bracket = filtered && !(n.op == OP_LINEAR && n.i5 == 2) && m->node_family[i] == m->prof_filter;
    const size_t fe = 2 * m->prof_pending.size();
    if (bracket) {
      while (m->fevents.size() < fe + 2) {
        hipEvent_t e;
        // Timing only: no cache writeback when recorded (it would slow what follows).
    hip_check(hipEventCreateWithFlags(&e, hipEventDisableSystemFence), "hipEventCreate");
        m->fevents.push_back(e);
      }
      hip_check(hipEventRecord(m->fevents[fe], ns), "hipEventRecord");
    }
    if (full) hip_check(hipEventRecord(m->events[2 * i], ns), "hipEventRecord");
    r.launch(n, ns);
    if (full) hip_check(hipEventRecord(m->events[2 * i + 1], ns), "hipEventRecord");
    if (bracket) {
      hip_check(hipEventRecord(m->fevents[fe + 1], ns), "hipEventRecord");
      m->prof_pending.push_back((int)i);
    }
    if (m->two_lanes && m->signal[i] >= 0)
      hip_check(hipEventRecord(m->lane_events[m->signal[i]], ns), "hipEventRecord");
  }
  if (m->two_lanes) {
    hip_check(hipEventRecord(m->lane_events[ne - 1], st[1]), "hipEventRecord");
    hip_check(hipStreamWaitEvent(s, m->lane_events[ne - 1], 0), "hipStreamWaitEvent");
  }
  if (!full) {
    hip_check(hipGetLastError(), "kernel launch");
    return;
  }
  hip_check(hipGetLastError(), "kernel launch");
  hip_check(hipStreamSynchronize(s), "profiled run");
  for (size_t i = 0; i < m->nodes.size(); i++) {
    const GNode& n = m->nodes[i];
    if (n.op == OP_LINEAR && n.i5 == 2) continue;  // timed with the node before it
    float ms = 0;
    hip_check(hipEventElapsedTime(&ms, m->events[2 * i], m->events[2 * i + 1]), "hipEventElapsedTime");
    ProfEntry& e = m->prof[m->node_family[i]];
    e.launches++;
    e.ms += ms;
    e.flops += n.flops;
    e.bytes += n.bytes;
  }
}

// The kernel family of each node, as profiles name them (a pair of linears
// launched together under the first node).
void compute_families(ndx_model* m) {
  m->node_family.assign(m->nodes.size(), std::string());
  auto probe = [&](const GNode& k) {
    GemmArgs p{};
    const GValue& x = m->values[k.in[0]];
    const GValue& w = m->values[k.in[1]];
    p.a_dtype = x.dtype;
    p.w_dtype = w.quant ? NDX_I8 : w.dtype;
    p.M = (int)(x.v.size[2]);
    p.N = (int)w.v.size[2];
    p.K = (int)x.v.size[3];
    p.batch = (int)(x.v.size[0] * x.v.size[1]);
    p.tile_hint = k.tile_hint ? k.tile_hint : second_stream_tile(k, p.M);
    p.c_dtype = m->values[k.out].dtype;
    p.epilogue = k.i0;
    if (k.in.size() > 4 && k.in[4] >= 0) p.r_dtype = m->values[k.in[4]].dtype;
    return p;
  };
  // NDX_PROFILE_LANES=1 names the second stream's kernels apart ("@lane1"),
  // to see what each stream spends; read when profiling is switched on.
  const char* by_lane = getenv("NDX_PROFILE_LANES");
  const bool lanes = by_lane && by_lane[0] == '1';
  for (size_t i = 0; i < m->nodes.size(); i++) {
    const GNode& n = m->nodes[i];
    std::string fam = n.family;
    if (n.op == OP_LINEAR && n.i5 != 2)
      fam = n.i5 == 1 ? gemm_pair_family(probe(n), probe(m->nodes[i + 1])) : gemm_family(probe(n));
    if (lanes && n.lane == 1) fam += "@lane1";
    m->node_family[i] = fam;
  }
}

// Waits for the filtered brackets recorded so far and adds them up.
void harvest_filtered(ndx_model* m) {
  if (m->prof_pending.empty()) return;
  hip_check(hipStreamSynchronize(m->dev->stream), "profiled runs");
  for (size_t k = 0; k < m->prof_pending.size(); k++) {
    const int i = m->prof_pending[k];
    float ms = 0;
    hip_check(hipEventElapsedTime(&ms, m->fevents[2 * k], m->fevents[2 * k + 1]), "hipEventElapsedTime");
    const GNode& n = m->nodes[i];
    ProfEntry& e = m->prof[m->node_family[i]];
    e.launches++;
    e.ms += ms;
    e.flops += n.flops + (n.op == OP_LINEAR && n.i5 == 1 ? m->nodes[i + 1].flops : 0.0);
    e.bytes += n.bytes + (n.op == OP_LINEAR && n.i5 == 1 ? m->nodes[i + 1].bytes : 0.0);
  }
  m->prof_pending.clear();
}

// Launches the run as one HIP graph: captured from run_nodes when the
// bound pointers differ from the captured graph's (the first run, or other
// tensors), then replayed with one hipGraphLaunch on the device stream. The
// second lane joins the capture through the run's own fork and join events.
void run_replay(ndx_model* m, Runner& r, int n_inputs) {
  std::vector<void*> key;
  for (int i = 0; i < n_inputs; i++) key.push_back(r.in[i]->ptr);
  key.insert(key.end(), r.out_ptr.begin(), r.out_ptr.end());
  key.push_back(r.arena);
  hipStream_t s = m->dev->stream;
  if (!m->graph_exec || key != m->graph_key) {
    if (m->graph_exec) {
      hip_check(hipStreamSynchronize(s), "graph replay");
      (void)hipGraphExecDestroy(m->graph_exec);
      m->graph_exec = nullptr;
    }
    hip_check(hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed), "hipStreamBeginCapture");
    hipGraph_t graph = nullptr;
    try {
      run_nodes(m, r, false);
    } catch (...) {
      (void)hipStreamEndCapture(s, &graph);
      if (graph) (void)hipGraphDestroy(graph);
      (void)hipGetLastError();
      throw;
    }
    hip_check(hipStreamEndCapture(s, &graph), "hipStreamEndCapture");
    const hipError_t err = hipGraphInstantiate(&m->graph_exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (err != hipSuccess) m->graph_exec = nullptr;
    hip_check(err, "hipGraphInstantiate");
    m->graph_key = key;
  }
  hip_check(hipGraphLaunch(m->graph_exec, s), "hipGraphLaunch");
}

}  // namespace

extern "C" {

NDX_API ndx_status ndx_model_sizes(ndx_model* m, uint64_t* persistent, uint64_t* temporary) {
  NDX_TRY
  NEED(m);
  if (persistent) *persistent = m->persistent;
  if (temporary) *temporary = m->arena_bytes;
  NDX_CATCH
}

NDX_API ndx_status ndx_model_counts(ndx_model* m, int32_t* inputs, int32_t* outputs, int32_t* kernels) {
  NDX_TRY
  NEED(m);
  if (inputs) *inputs = (int32_t)m->inputs.size();
  if (outputs) *outputs = (int32_t)m->outputs.size();
  if (kernels) *kernels = m->kernels;
  NDX_CATCH
}

NDX_API ndx_status ndx_model_run(ndx_model* m, ndx_tensor* const* inputs, int32_t n_inputs, ndx_tensor** outputs,
                                 int32_t n_outputs) {
  if (!m) {
    set_last_error("model is null");
    return NDX_INVALID_ARG;
  }
  std::vector<ndx_tensor*> made;
  try {
    m->dev->check_usable();
    if (n_inputs > 0 && !inputs) fail(NDX_INVALID_ARG, "inputs is null");
    if (!outputs) fail(NDX_INVALID_ARG, "outputs is null");
    check_inputs(m, inputs, n_inputs);
    if (n_outputs != (int)m->outputs.size())
      fail(NDX_INVALID_ARG, "the model has " + std::to_string(m->outputs.size()) + " outputs, not " + std::to_string(n_outputs));
    Runner r{m, inputs, {}};
    r.arena = model_arena(m);
    for (int id : m->outputs) {
      const GValue& v = m->values[id];
      int64_t shape[4];
      for (int i = 0; i < v.rank; i++) shape[i] = v.v.size[4 - v.rank + i];
      ndx_tensor* t = new_tensor(m->dev, v.dtype, shape, v.rank);
      made.push_back(t);
      r.out_ptr.push_back(t->ptr);
    }
    run_nodes(m, r);
    hip_check(hipStreamSynchronize(m->dev->stream), "model run");
    for (int i = 0; i < n_outputs; i++) outputs[i] = made[i];
  } catch (const ndx::Error& e) {
    for (auto* t : made) free_tensor(t);
    if (e.status == NDX_DEVICE_LOST) m->dev->lost = true;
    set_last_error(e.message);
    return e.status;
  }
  return NDX_OK;
}

NDX_API ndx_status ndx_model_run_into_async(ndx_model* m, ndx_tensor* const* inputs, int32_t n_inputs,
                                            ndx_tensor* const* outputs, int32_t n_outputs) {
  if (!m) {
    set_last_error("model is null");
    return NDX_INVALID_ARG;
  }
  try {
    m->dev->check_usable();
    if (n_inputs > 0 && !inputs) fail(NDX_INVALID_ARG, "inputs is null");
    if (!outputs) fail(NDX_INVALID_ARG, "outputs is null");
    check_inputs(m, inputs, n_inputs);
    Runner r{m, inputs, {}};
    bind_outputs(m, r, outputs, n_outputs);
    r.arena = model_arena(m);
    if (m->replay && !m->profiling)
      run_replay(m, r, n_inputs);
    else
      run_nodes(m, r);
  } catch (const ndx::Error& e) {
    if (e.status == NDX_DEVICE_LOST) m->dev->lost = true;
    set_last_error(e.message);
    return e.status;
  }
  return NDX_OK;
}

NDX_API ndx_status ndx_model_run_into_static_async(ndx_model* m, ndx_tensor* const* inputs, int32_t n_inputs,
                                                   ndx_tensor* const* outputs, int32_t n_outputs) {
  if (!m) {
    set_last_error("model is null");
    return NDX_INVALID_ARG;
  }
  try {
    m->dev->check_usable();
    if (n_inputs > 0 && !inputs) fail(NDX_INVALID_ARG, "inputs is null");
    check_inputs(m, inputs, n_inputs);
    Runner r{m, inputs, {}};
    bind_outputs(m, r, outputs, n_outputs);
    if (m->arena_bytes > kStaticScratchBytes)
      fail(NDX_INVALID_ARG, "the model needs " + std::to_string(m->arena_bytes) +
                                " bytes of temporary memory; the static scratch holds " +
                                std::to_string(kStaticScratchBytes));
    if (!m->dev->static_scratch)
      fail(NDX_UNSUPPORTED, "the static scratch is not available on this device (" +
                                m->dev->static_scratch_error + ")");
    // Every intermediate and every kernel's scratch (attention key-split
    // partials, GroupNorm split statistics) is written before it is read
    // within one run, so nothing left by an earlier run needs clearing.
    r.arena = (char*)m->dev->static_scratch;
    run_nodes(m, r, false);
  } catch (const ndx::Error& e) {
    if (e.status == NDX_DEVICE_LOST) m->dev->lost = true;
    set_last_error(e.message);
    return e.status;
  }
  return NDX_OK;
}

NDX_API ndx_status ndx_model_set_graph_replay(ndx_model* m, int32_t enabled) {
  NDX_TRY
  NEED(m);
  m->replay = enabled != 0;
  if (!m->replay && m->graph_exec) {
    hip_check(hipStreamSynchronize(m->dev->stream), "graph replay");
    (void)hipGraphExecDestroy(m->graph_exec);
    m->graph_exec = nullptr;
    m->graph_key.clear();
  }
  NDX_CATCH
}

NDX_API ndx_status ndx_model_set_profiling(ndx_model* m, int32_t enabled) {
  NDX_TRY
  NEED(m);
  harvest_filtered(m);
  m->profiling = enabled != 0;
  if (m->profiling) {
    m->prof.clear();
    if (m->node_family.size() != m->nodes.size()) compute_families(m);
  }
  NDX_CATCH
}

NDX_API ndx_status ndx_model_set_profile_filter(ndx_model* m, const char* family) {
  NDX_TRY
  NEED(m);
  harvest_filtered(m);
  m->prof_filter = family ? family : "";
  NDX_CATCH
}

NDX_API ndx_status ndx_model_profile_entry(ndx_model* m, int32_t index, char* name, int32_t capacity,
                                           int64_t* launches, double* ms, double* flops, double* bytes) {
  NDX_TRY
  NEED(m);
  harvest_filtered(m);
  if (index < 0 || index >= (int)m->prof.size()) fail(NDX_INVALID_ARG, "no such profile entry");
  auto it = m->prof.begin();
  std::advance(it, index);
  if (name && capacity > 0) snprintf(name, capacity, "%s", it->first.c_str());
  if (launches) *launches = it->second.launches;
  if (ms) *ms = it->second.ms;
  if (flops) *flops = it->second.flops;
  if (bytes) *bytes = it->second.bytes;
  NDX_CATCH
}

NDX_API ndx_status ndx_model_release(ndx_model* m) {
  NDX_TRY
  if (!m) return NDX_OK;
  if (m->arena) {
    (void)hipStreamSynchronize(m->dev->stream);
    m->dev->release(m->arena, m->arena_alloc);
  }
  if (m->two_lanes && m->dev->aux) (void)hipStreamSynchronize(m->dev->aux);
  if (m->graph_exec) (void)hipGraphExecDestroy(m->graph_exec);
  for (auto e : m->events) (void)hipEventDestroy(e);
  for (auto e : m->fevents) (void)hipEventDestroy(e);
  for (auto e : m->lane_events) (void)hipEventDestroy(e);
  delete m;
  NDX_CATCH
}

}  // extern "C"
