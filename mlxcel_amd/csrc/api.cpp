// api.cpp — the C ABI declared in include/mlxq.h.
//
// Validation restates the reference op layer so callers see the same accept /
// reject decisions and the same messages (overlays/rocm/mlx/ops.cpp):
//   validate_quantized_input / extract_quantized_matmul_dims   ops.cpp:111-179
//   quantization_params_from_mode / validate_mode_with_type    ops.cpp:4846-4925
//   quantized_matmul                                            ops.cpp:4955-5008
//   quantize / affine_quantize / fp_quantize checks             ops.cpp:5277-5290, 5340-5358, 5454-5492
//   dequantize / affine_dequantize / fp_dequantize checks       ops.cpp:5494-5530, 5596-5640, 5753-5805
//   gather_qmm / indices_or_default                             ops.cpp:5841-5948, 79-109
//   string_to_quantization_mode                                 overlays/rocm/mlx/primitives.cpp:3617-3635
// The eval side (what the reference's QuantizedMatmul/GatherQMM::eval_gpu do,
// overlays/rocm/mlx/backend/rocm/quantized/qmm.hip:3550, 6590) is replaced by
// the dispatch at the bottom of this file.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdlib>
#include <cstdarg>
#include <cstring>
#include <map>
#include <mutex>
#include <sstream>
#include <string>
#include <vector>

#include "../../include/mlxq.h"
#include "common.hpp"
#include "kernels.hpp"

namespace {

using Shape = std::vector<int64_t>;

thread_local std::string g_last_error;

struct Error {
  mlxq_status code;
  std::string msg;
};

[[noreturn]] void fail(mlxq_status code, const std::string& msg) { throw Error{code, msg}; }
[[noreturn]] void invalid(const std::ostringstream& os) { fail(MLXQ_EINVAL, os.str()); }
[[noreturn]] void unsupported(const std::string& msg) { fail(MLXQ_EUNSUPPORTED, "[mlxq] " + msg); }

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(MLXQ_EHIP, std::string("[mlxq] ") + what + ": " + hipGetErrorString(e));
}

template <typename F>
mlxq_status guarded(F&& f) {
  try {
    f();
    g_last_error.clear();
    return MLXQ_OK;
  } catch (const Error& e) {
    g_last_error = e.msg;
    return e.code;
  } catch (const std::exception& e) {
    g_last_error = std::string("[mlxq] internal error: ") + e.what();
    return MLXQ_EHIP;
  }
}

// ---- dtype facts (mlx::core::Dtype order) ----------------------------------

const char* dtype_name(int d) {
  static const char* names[] = {"bool",  "uint8",   "uint16",  "uint32",  "uint64",
                                "int8",  "int16",   "int32",   "int64",   "float16",
                                "float32", "float64", "bfloat16", "complex64"};
  return (d >= 0 && d <= 13) ? names[d] : "unknown";
}
bool is_floating(int d) { return d == MLXQ_FLOAT16 || d == MLXQ_FLOAT32 || d == MLXQ_FLOAT64 || d == MLXQ_BFLOAT16; }
bool is_integral(int d) { return d >= MLXQ_BOOL + 1 && d <= MLXQ_INT64; }
int dtype_size(int d) {
  static const int sz[] = {1, 1, 2, 4, 8, 1, 2, 4, 8, 2, 4, 8, 2, 8};
  return (d >= 0 && d <= 13) ? sz[d] : 0;
}

// Upstream MLX promote_types for the floating types this op layer meets
// (jax-style lattice: f16+bf16 -> f32, anything with f32/f64 -> the wider).
int promote(int a, int b) {
  if (a == b) return a;
  if (!is_floating(a) && !is_floating(b)) return a < b ? b : a;  // stays integral
  if (a == MLXQ_FLOAT64 || b == MLXQ_FLOAT64) return MLXQ_FLOAT64;
  if (is_floating(a) && !is_floating(b)) return a;
  if (is_floating(b) && !is_floating(a)) return b;
  return MLXQ_FLOAT32;  // f16/bf16/f32 mixes
}

// ---- array views -------------------------------------------------------------

struct View {
  const mlxq_array* a = nullptr;
  int64_t dim(int i) const { return a->shape[i < 0 ? i + a->ndim : i]; }
  int ndim() const { return a->ndim; }
  Shape shape() const { return Shape(a->shape, a->shape + a->ndim); }
  int dtype() const { return a->dtype; }
  int64_t size() const {
    int64_t s = 1;
    for (int i = 0; i < a->ndim; i++) s *= a->shape[i];
    return s;
  }
  bool row_contiguous() const {
    int64_t st = 1;
    for (int i = a->ndim - 1; i >= 0; i--) {
      if (a->shape[i] != 1 && a->strides[i] != st) return false;
      st *= a->shape[i];
    }
    return true;
  }
};

std::string fmt_shape(const Shape& s) {
  std::ostringstream os;
  os << "(";
  for (size_t i = 0; i < s.size(); i++) os << s[i] << (i + 1 == s.size() ? "" : ",");
  os << ")";
  return os.str();
}

void check_array(const mlxq_array* a, const char* name) {
  if (!a) fail(MLXQ_EINVAL, std::string("[mlxq] ") + name + " must not be NULL");
  if (a->ndim < 0 || a->ndim > MLXQ_MAX_DIMS)
    fail(MLXQ_EINVAL, std::string("[mlxq] ") + name + " has an invalid ndim");
  for (int i = 0; i < a->ndim; i++)
    if (a->shape[i] < 0) fail(MLXQ_EINVAL, std::string("[mlxq] ") + name + " has a negative dimension");
}

Shape broadcast_shapes(const Shape& s1, const Shape& s2) {
  const size_t nd = std::max(s1.size(), s2.size());
  Shape out(nd);
  for (size_t i = 0; i < nd; i++) {
    const int64_t a = i < nd - s1.size() ? 1 : s1[i - (nd - s1.size())];
    const int64_t b = i < nd - s2.size() ? 1 : s2[i - (nd - s2.size())];
    if (a == b || b == 1) out[i] = a;
    else if (a == 1) out[i] = b;
    else {
      std::ostringstream os;
      os << "[broadcast_shapes] Shapes " << fmt_shape(s1) << " and " << fmt_shape(s2) << " cannot be broadcast.";
      invalid(os);
    }
  }
  return out;
}

// ---- mode / params (ops.cpp:4846-4925, primitives.cpp:3617-3635) ----------

enum Mode { AFFINE = 0, MXFP4_M = 1, MXFP8_M = 2, NVFP4_M = 3 };

Mode parse_mode(const char* mode, const char* tag) {
  const std::string m = mode ? mode : "affine";
  if (m == "affine") return AFFINE;
  if (m == "mxfp4") return MXFP4_M;
  if (m == "mxfp8") return MXFP8_M;
  if (m == "nvfp4") return NVFP4_M;
  std::ostringstream os;
  if (tag && *tag) os << "[" << tag << "]";
  os << " Invalid quantization mode '" << m << "'.";
  invalid(os);
}

void params_from_mode(Mode mode, int32_t& gs, int32_t& bits) {
  int dgs = 64, dbits = 4;
  if (mode == NVFP4_M) dgs = 16;
  if (mode == MXFP4_M) dgs = 32;
  if (mode == MXFP8_M) { dgs = 32; dbits = 8; }
  if (gs <= 0) gs = dgs;
  if (bits <= 0) bits = dbits;
}

// returns the output dtype
int validate_mode_with_type(const char* tag, const mlxq_array* scales, const mlxq_array* biases,
                            int out_type, Mode mode, const char* mode_str) {
  if (out_type >= 0 && !is_floating(out_type)) {
    std::ostringstream os;
    os << "[" << tag << "] Only real floating types are supported but output dtype == " << dtype_name(out_type)
       << ".";
    invalid(os);
  }
  if (mode == AFFINE) {
    if (!biases) {
      std::ostringstream os;
      os << "[" << tag << "] Biases must be provided for affine quantization.";
      invalid(os);
    }
    const int dt = promote(scales->dtype, biases->dtype);
    if (!is_floating(dt)) {
      std::ostringstream os;
      os << "[" << tag << "] Only real floating types are supported but scales.dtype() == "
         << dtype_name(scales->dtype) << " and biases.dtype() == " << dtype_name(biases->dtype) << ".";
      invalid(os);
    }
    return out_type >= 0 ? out_type : dt;
  } else if (scales->dtype != MLXQ_UINT8) {
    std::ostringstream os;
    os << "[" << tag << "] Scale type must be uint8 but received type " << dtype_name(scales->dtype) << ".";
    invalid(os);
  }
  if (biases) {
    std::ostringstream os;
    os << "[" << tag << "] Biases must be null for quantization mode '" << (mode_str ? mode_str : "") << "'.";
    invalid(os);
  }
  return out_type >= 0 ? out_type : (int)MLXQ_BFLOAT16;
}

void validate_quantized_input(const char* tag, View w, View scales, int gs, int bits, const mlxq_array* biases) {
  if (w.dtype() != MLXQ_UINT32) {
    std::ostringstream os;
    os << "[" << tag << "] The weight matrix should be uint32 but received " << dtype_name(w.dtype());
    invalid(os);
  }
  if (biases && View{biases}.shape() != scales.shape()) {
    std::ostringstream os;
    os << "[" << tag << "] Scales and biases should have the same shape. Received scales with shape "
       << fmt_shape(scales.shape()) << " and biases with " << fmt_shape(View{biases}.shape());
    invalid(os);
  }
  if (w.ndim() < 2 || scales.ndim() < 1) {
    std::ostringstream os;
    os << "[" << tag << "] The weight matrix must have at least 2 dimensions but received shape "
       << fmt_shape(w.shape()) << ".";
    invalid(os);
  }
  bool batch_eq = scales.ndim() >= w.ndim() - 2;
  for (int i = 0; batch_eq && i < w.ndim() - 2; i++) batch_eq = w.dim(i) == scales.dim(i);
  if (!batch_eq) {
    std::ostringstream os;
    os << "[" << tag << "] Weight and scales should have the same batch shape. Received weight with shape "
       << fmt_shape(w.shape()) << ", scales with " << fmt_shape(scales.shape()) << ".";
    invalid(os);
  }
  if (w.dim(-1) * 32 / bits != scales.dim(-1) * gs) {
    std::ostringstream os;
    os << "[" << tag << "] The shapes of the weight and scales are incompatible based on bits and group_size. "
       << "w.shape() == " << fmt_shape(w.shape()) << " and scales.shape() == " << fmt_shape(scales.shape())
       << " with group_size=" << gs << " and bits=" << bits;
    invalid(os);
  }
}

// returns {w_inner, w_outer}
std::pair<int64_t, int64_t> extract_dims(const char* tag, View x, View w, View scales, const mlxq_array* biases,
                                         bool transpose, int gs, int bits) {
  validate_quantized_input(tag, w, scales, gs, bits, biases);
  if (x.ndim() < 1) {
    std::ostringstream os;
    os << "[" << tag << "] The input must have at least 1 dimension.";
    invalid(os);
  }
  const int64_t x_inner = x.dim(-1);
  const int64_t w_inner = transpose ? w.dim(-1) * 32 / bits : w.dim(-2);
  const int64_t w_outer = transpose ? w.dim(-2) : w.dim(-1) * 32 / bits;
  if (w_inner != x_inner) {
    std::ostringstream os;
    os << "[" << tag << "] Last dimension of first input with shape (..., " << x_inner
       << ") does not match the expanded quantized matrix (" << w_inner << ", " << w_outer
       << ") computed from shape " << fmt_shape(w.shape()) << " with group_size=" << gs << ", bits=" << bits
       << " and transpose=" << (transpose ? "true" : "false");
    invalid(os);
  }
  return {w_inner, w_outer};
}

// ---- quantized_matmul validation (ops.cpp:4955-5008) ------------------------

struct QmmSpec {
  Mode mode;
  int gs, bits;
  int64_t K, N;
  int out_dtype;
  Shape out_shape;
  bool transpose = true;
  bool fast = true;  // the specialised kernels take the call (else qmm_gen.hip)
  bool small_w = true;  // each weight matrix and its scales below 2 GiB (buffer-resource kernels)
};

// The specialised kernels address each operand (or one weight matrix of it)
// through a buffer resource with 32-bit byte offsets, and lanes without work
// read at offset 2^31 (common.hpp kDeadOfs), so every such operand stays
// below 2 GiB.  Larger ones take other routes: 2-D-weight calls run as row
// chunks below the limit, gathers as chunks of index entries, and weight
// matrices of 2 GiB or more the general kernel (64-bit indexing).
constexpr int64_t kBufMax = (int64_t)1 << 31;

// Index entries per gather launch (a grid dimension holds at most 65535); a
// multiple of 8, so every chunk's output starts 16-byte aligned.
constexpr int64_t kGatherChunk = 65528;

// Elements of one dequantize / quantize call: the conversion kernels index in
// 64 bits and take >= 8 elements per thread, and a launch covers < 2^32 threads.
constexpr int64_t kElemMax = (int64_t)1 << 34;

QmmSpec spec_quantized_matmul(const mlxq_array* xa, const mlxq_array* wa, const mlxq_array* sa,
                              const mlxq_array* ba, bool transpose, int32_t gs, int32_t bits,
                              const char* mode_str) {
  check_array(xa, "x");
  check_array(wa, "w");
  check_array(sa, "scales");
  if (ba) check_array(ba, "biases");
  const char* tag = "quantized_matmul";
  QmmSpec sp;
  sp.transpose = transpose;
  sp.mode = parse_mode(mode_str, tag);
  int dtype = validate_mode_with_type(tag, sa, ba, -1, sp.mode, mode_str);
  params_from_mode(sp.mode, gs, bits);
  sp.gs = gs;
  sp.bits = bits;
  View x{xa}, w{wa}, s{sa};
  auto [wi, wo] = extract_dims(tag, x, w, s, ba, transpose, gs, bits);
  sp.K = wi;
  sp.N = wo;
  dtype = sp.mode == AFFINE ? promote(x.dtype(), dtype) : x.dtype();
  if (!is_floating(dtype)) {
    std::ostringstream os;
    os << "[quantized_matmul] Only real floating types are supported but x.dtype() == " << dtype_name(x.dtype())
       << ".";
    invalid(os);
  }
  sp.out_dtype = dtype;
  Shape xs = x.shape();
  if (x.ndim() > 2 && w.ndim() > 2) {
    const Shape wsh = w.shape();
    Shape xb(xs.begin(), xs.end() - 2), wb(wsh.begin(), wsh.end() - 2);
    Shape bb = broadcast_shapes(xb, wb);
    bb.push_back(xs[xs.size() - 2]);
    bb.push_back(xs.back());
    xs = bb;
  }
  xs.back() = wo;
  sp.out_shape = xs;
  return sp;
}

// ---- gather_qmm validation (ops.cpp:5841-5948) -------------------------------

struct GatherSpec {
  QmmSpec q;
  Shape idx_shape;  // broadcast index shape
};

void check_indices(const mlxq_array* idx, View base) {
  if (base.ndim() < 2) {
    std::ostringstream os;
    os << "[gather_qmm] Input must have at least two dimensions but got input with shape "
       << fmt_shape(base.shape()) << ".";
    invalid(os);
  }
  if (idx && !is_integral(idx->dtype)) {
    std::ostringstream os;
    os << "[gather_qmm] Got indices with invalid dtype. Indices must be integral.";
    invalid(os);
  }
}

Shape default_index_shape(View base) { return Shape(base.a->shape, base.a->shape + base.ndim() - 2); }

GatherSpec spec_gather(const mlxq_array* xa, const mlxq_array* wa, const mlxq_array* sa, const mlxq_array* ba,
                       const mlxq_array* lhs, const mlxq_array* rhs, bool transpose, int32_t gs, int32_t bits,
                       const char* mode_str, const mlxq_array* global_scale) {
  check_array(xa, "x");
  check_array(wa, "w");
  check_array(sa, "scales");
  if (ba) check_array(ba, "biases");
  if (lhs) check_array(lhs, "lhs_indices");
  if (rhs) check_array(rhs, "rhs_indices");
  const char* tag = "gather_qmm";
  GatherSpec g;
  QmmSpec& sp = g.q;
  sp.transpose = transpose;
  sp.mode = parse_mode(mode_str, tag);
  int out_type = validate_mode_with_type(tag, sa, ba, -1, sp.mode, mode_str);
  params_from_mode(sp.mode, gs, bits);
  sp.gs = gs;
  sp.bits = bits;
  View x{xa}, w{wa}, s{sa};
  auto [wi, wo] = extract_dims(tag, x, w, s, ba, transpose, gs, bits);
  sp.K = wi;
  sp.N = wo;
  if (global_scale && sp.mode != NVFP4_M) {
    std::ostringstream os;
    os << "[gather_qmm] Global scale is only supported for 'nvfp4' quantization mode.";
    invalid(os);
  }
  out_type = sp.mode == AFFINE ? promote(x.dtype(), out_type) : x.dtype();
  if (!is_floating(out_type)) {
    std::ostringstream os;
    os << "[gather_qmm] Only real floating types are supported but x.dtype() == " << dtype_name(x.dtype()) << ".";
    invalid(os);
  }
  sp.out_dtype = out_type;
  check_indices(lhs, x);
  check_indices(rhs, w);
  Shape ls = lhs ? View{lhs}.shape() : default_index_shape(x);
  Shape rs = rhs ? View{rhs}.shape() : default_index_shape(w);
  g.idx_shape = broadcast_shapes(ls, rs);
  sp.out_shape = g.idx_shape;
  sp.out_shape.push_back(x.dim(-2));
  sp.out_shape.push_back(wo);
  return g;
}

void write_shape(const Shape& s, int dtype, int32_t* ndim, int64_t* shape, int32_t* out_dtype) {
  if ((int)s.size() > MLXQ_MAX_DIMS) fail(MLXQ_EUNSUPPORTED, "[mlxq] result has too many dimensions");
  if (ndim) *ndim = (int32_t)s.size();
  if (shape)
    for (size_t i = 0; i < s.size(); i++) shape[i] = s[i];
  if (out_dtype) *out_dtype = dtype;
}

void check_out(const mlxq_array* out, const Shape& shape, int dtype, const char* tag) {
  check_array(out, "out");
  if (View{out}.shape() != shape || out->dtype != dtype) {
    std::ostringstream os;
    os << "[" << tag << "] out must have shape " << fmt_shape(shape) << " and dtype " << dtype_name(dtype)
       << " but has shape " << fmt_shape(View{out}.shape()) << " and dtype " << dtype_name(out->dtype) << ".";
    invalid(os);
  }
}

void require_contiguous(const mlxq_array* a, const char* name) {
  if (a && !View{a}.row_contiguous())
    unsupported(std::string(name) + " must be row-contiguous (make a contiguous copy first)");
  if (a && a->data && (reinterpret_cast<uintptr_t>(a->data) & 15u) != 0 && View{a}.size() > 0)
    unsupported(std::string(name) + " must be 16-byte aligned");
}

// ---- per-device facts and per-stream workspace -------------------------------

struct DevInfo {
  int cus = 256;
};

std::mutex g_mu;
std::map<int, DevInfo> g_dev;

// Per-(device, stream) scratch.  A buffer is never freed while the library
// may still use it: when a call needs more, a larger buffer replaces it and
// the old one moves to `retired`, which only mlxq_clear_cache() frees (a HIP
// graph captured earlier, or a launch another thread has not issued yet, may
// still hold the old pointer).  No call synchronizes a stream, and none
// allocates while its stream is being captured.
struct Workspace {
  void* data = nullptr;
  size_t bytes = 0;
  std::vector<void*> retired;
  size_t retired_bytes = 0;
};
// key: (device, stream, slot); slot 0 holds kernel scratch, slot 1 the
// row-contiguous copies of strided operands, slot 2 the flat index lists of
// gathers run in chunks
std::map<std::tuple<int, hipStream_t, int>, Workspace> g_ws;

int current_device() {
  int dev = 0;
  hip_check(hipGetDevice(&dev), "hipGetDevice");
  return dev;
}

DevInfo device_info(int dev) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_dev.find(dev);
  if (it != g_dev.end()) return it->second;
  DevInfo d;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && cus > 0) d.cus = cus;
  g_dev[dev] = d;
  return d;
}

bool stream_capturing(hipStream_t stream) {
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  hip_check(hipStreamIsCapturing(stream, &st), "hipStreamIsCapturing");
  return st != hipStreamCaptureStatusNone;
}

// Grows the stream's workspace to at least `bytes` (a power of two from
// 1 MiB); the caller must not be capturing `stream`.
void* grow_workspace(Workspace& w, size_t bytes) {
  size_t sz = 1 << 20;
  while (sz < bytes) sz <<= 1;
  void* p = nullptr;
  if (hipMalloc(&p, sz) != hipSuccess) {
    (void)hipGetLastError();
    fail(MLXQ_ENOMEM, "[mlxq] workspace allocation of " + std::to_string(sz) + " bytes failed");
  }
  if (w.data) {
    w.retired.push_back(w.data);
    w.retired_bytes += w.bytes;
  }
  w.data = p;
  w.bytes = sz;
  return p;
}

// Scratch source of one call: the per-stream workspace, or a fixed buffer
// (the no-allocation entry point's device array) of at most `max` bytes.
struct ScratchSrc {
  void* fixed = nullptr;
  size_t max = 0;
};

void* workspace(int dev, hipStream_t stream, size_t bytes, const ScratchSrc& src = ScratchSrc{}, int slot = 0) {
  if (src.fixed) {
    if (bytes > src.max)
      fail(MLXQ_ENOMEM, "[mlxq] this call needs " + std::to_string(bytes) +
                            " bytes of scratch; the no-allocation entry point has " + std::to_string(src.max));
    return src.fixed;
  }
  std::lock_guard<std::mutex> lk(g_mu);
  Workspace& w = g_ws[{dev, stream, slot}];
  if (w.bytes >= bytes) return w.data;
  if (stream_capturing(stream))
    fail(MLXQ_ENOMEM, "[mlxq] this call needs " + std::to_string(bytes) + " bytes of workspace on a stream that is "
                      "being captured (which holds " + std::to_string(w.bytes) +
                      "); run it once before the capture or reserve with mlxq_workspace_reserve");
  return grow_workspace(w, bytes);
}

// Stream-K counters of a stream (slot 3): mlxq::kSplitCounters words,
// zeroed on the stream when allocated; every launch that uses them leaves
// them zero.
void alloc_counters(Workspace& w, hipStream_t stream) {
  grow_workspace(w, (size_t)mlxq::kSplitCounters * sizeof(uint32_t));
  hip_check(hipMemsetAsync(w.data, 0, w.bytes, stream), "hipMemsetAsync (stream-K counters)");
}

// The prefill plan of a dense call: stream-K only where its partials and
// counters can be had without allocating under a capture, and not for the
// no-allocation entry point (its fixed scratch is small); otherwise the plan
// without it.
mlxq::QmmPlan prefill_plan(int fmt, int gs, int64_t rows, int64_t N, int64_t K, int dev, hipStream_t stream,
                           const ScratchSrc& ss, int tile_req, int ksplit_req, int mix, int streamk,
                           uint32_t** cnt) {
  *cnt = nullptr;
  const int cus = device_info(dev).cus;
  mlxq::QmmPlan qp = mlxq::qmm_plan(fmt, gs, rows, N, K, cus, tile_req, ksplit_req, mix, ss.fixed ? 0 : streamk);
  if (qp.sk_len <= 0) return qp;
  std::lock_guard<std::mutex> lk(g_mu);
  const bool capturing = stream_capturing(stream);
  Workspace& w = g_ws[{dev, stream, 0}];
  Workspace& c = g_ws[{dev, stream, 3}];
  const bool ok = qp.sk_wgs <= mlxq::kSplitCounters &&
                  (!capturing || (w.bytes >= (size_t)mlxq::qmm_sk_bytes(qp) && c.data));
  if (!ok) return mlxq::qmm_plan(fmt, gs, rows, N, K, cus, tile_req, ksplit_req, mix, 0);
  if (!c.data) alloc_counters(c, stream);
  *cnt = static_cast<uint32_t*>(c.data);
  return qp;
}

// Rows from which a dense quantized_matmul runs the prefill GEMM (qmm.hip):
// at 9-16 rows its 128 x 128 tiles already beat the skinny kernels on
// MI355X (MLXQ_QMM_MIN_ROWS overrides, for tests and measurements).
constexpr int kQmmMinRows = 9;

// Environment switches for A/B measurement and tests, latched at the first
// call (mlxq_reload_options re-reads them).
struct Knobs {
  int qmv_nw = 0, qmv_tk = 0, qmv_r = 0, b4_rg = 0, b4_cpw = 0;
  int qmm_min_rows = kQmmMinRows, qmm_tile = -1, qmm_ksplit = 0;
  int qmv_mid = 1, qmv_multi = 1;
  int qmv_mr = 1;  // whole-row mid-size kernel where it applies (0: off)
  int mr_ring = 0;  // its weight ring depth in windows (0: planner)
  int gen_ks = 0;  // K splits of the general kernel (0: planner)
  int gen_qmv = 1;  // 0: 1-2-row general calls stay on the tile kernel
  int gather_sorted = 1, gather_group = -1, gather_runs = 2, gather_direct = 1;
  int red_vec = 0;  // outputs per thread of the mid-size kernel's split-K reduction (0: default)
  int qmm_mix = 1;  // prefill: two-launch plan for a part-full last round of tiles (0: off)
  int mid_win = 0;  // mid-size kernel: windows per workgroup (4 or 8; 0: planner)
  int gather_scale_table = 1;  // grouped sorted gather: scales staged in LDS where they fit (0: per block)
  int gather_tiles = 0;  // grouped sorted gather: 2 or 3 weight tiles per wave (0: planner)
  int qmv_kq = 1;  // K split over a workgroup's waves for matrices of one round of 16/32-row blocks (0: off)
  int kq_t = 0;    // its 16-row tiles per workgroup (1-4; 0: planner)
  int qmm_streamk = 1;  // prefill: stream-K plan for a part-full last round of 256 x 256 tiles (0: off)
  int sk_fallback = 0;  // stream-K: every cut tile's head computes its tail itself (tests)
  std::string qmv_kernel;  // "", "rs", "b4", "mid", "mr", "kq", "fr", "mfma"
};

int env_int(const char* name, int dflt) {
  const char* v = std::getenv(name);
  if (!v || !*v) return dflt;
  return std::atoi(v);
}

const Knobs* read_knobs() {
  Knobs* k = new Knobs;
  k->qmv_nw = env_int("MLXQ_QMV_NW", 0);
  k->qmv_tk = env_int("MLXQ_QMV_TK", 0);
  k->qmv_r = env_int("MLXQ_QMV_R", 0);
  k->b4_rg = env_int("MLXQ_QMV_B4_RG", 0);
  k->b4_cpw = env_int("MLXQ_QMV_B4_CPW", 0);
  k->qmm_min_rows = env_int("MLXQ_QMM_MIN_ROWS", kQmmMinRows);
  k->qmm_tile = env_int("MLXQ_QMM_TILE", -1);
  k->qmm_ksplit = env_int("MLXQ_QMM_KSPLIT", 0);
  k->qmv_mid = env_int("MLXQ_QMV_MID", 1);
  k->qmv_multi = env_int("MLXQ_QMV_MULTI", 1);
  k->qmv_mr = env_int("MLXQ_QMV_MR", 1);
  k->mr_ring = env_int("MLXQ_MR_RING", 0);
  k->gen_ks = env_int("MLXQ_GEN_KS", 0);
  k->gen_qmv = env_int("MLXQ_GEN_QMV", 1);
  k->gather_sorted = env_int("MLXQ_GATHER_SORTED", 1);
  k->gather_group = env_int("MLXQ_GATHER_GROUP", -1);
  k->gather_runs = env_int("MLXQ_GATHER_RUNS", 2);
  k->gather_direct = env_int("MLXQ_GATHER_DIRECT", 1);
  k->red_vec = env_int("MLXQ_REDUCE_VEC", 0);
  k->qmm_mix = env_int("MLXQ_QMM_MIX", 1);
  k->mid_win = env_int("MLXQ_QMV_MID_WIN", 0);
  k->gather_scale_table = env_int("MLXQ_GATHER_SCALE_TABLE", 1);
  k->gather_tiles = env_int("MLXQ_GATHER_TILES", 0);
  k->qmv_kq = env_int("MLXQ_QMV_KQ", 1);
  k->kq_t = env_int("MLXQ_QMV_KQ_T", 0);
  k->qmm_streamk = env_int("MLXQ_QMM_STREAMK", 1);
  k->sk_fallback = env_int("MLXQ_QMM_SK_FALLBACK", 0);
  const char* v = std::getenv("MLXQ_QMV_KERNEL");
  k->qmv_kernel = v ? v : "";
  return k;
}

// Replaced snapshots are kept (a concurrent call may still read one).
std::atomic<const Knobs*> g_knobs{nullptr};

const Knobs& knobs() {
  const Knobs* k = g_knobs.load(std::memory_order_acquire);
  if (k) return *k;
  const Knobs* fresh = read_knobs();
  if (!g_knobs.compare_exchange_strong(k, fresh, std::memory_order_acq_rel)) {
    delete fresh;
    return *k;
  }
  return *fresh;
}

// Default (waves per workgroup, loads in flight) by shape.
void qmv_shape_choice(int64_t N, int64_t K, int& nw, int& p) {
  (void)N;
  (void)K;
  // A/B overrides (waves per workgroup, K-steps per wave); 0 keeps the defaults
  nw = knobs().qmv_nw;
  p = knobs().qmv_tk;
}

// Broadcast strides of an index array (or of the default arange over `dshape`)
// against the broadcast shape `b`.
void bstrides_for(const mlxq_array* idx, const Shape& dshape, const Shape& b, int64_t* out) {
  const int bnd = (int)b.size();
  Shape sh;
  std::vector<int64_t> st;
  if (idx) {
    sh = View{idx}.shape();
    st.assign(idx->strides, idx->strides + idx->ndim);
  } else {
    sh = dshape;
    st.assign(sh.size(), 0);
    int64_t acc = 1;
    for (int i = (int)sh.size() - 1; i >= 0; i--) {
      st[i] = acc;
      acc *= sh[i];
    }
  }
  const int off = bnd - (int)sh.size();
  for (int d = 0; d < bnd; d++) {
    const int sd = d - off;
    out[d] = (sd < 0 || sh[sd] == 1) ? 0 : st[sd];
  }
}

// An index array the decode kernels can read in place (no index_prep
// launch): contiguous 32- or 64-bit integers already in the broadcast shape;
// or, with no array, the default arange over `dflt` when it equals the
// leading broadcast dims followed by ones, so entry b maps to b / div (x rows
// repeated over trailing index dims, as for MoE top-k routing).
struct DirectIdx {
  bool ok = false;
  const uint32_t* p = nullptr;
  int stride = 1;
  int div = 1;
};

DirectIdx direct_index(const mlxq_array* idx, const Shape& dflt, const Shape& b) {
  DirectIdx d;
  if (idx) {
    if (View{idx}.shape() != b) return d;
    const int dt = idx->dtype;
    if (dt != MLXQ_INT32 && dt != MLXQ_UINT32 && dt != MLXQ_INT64 && dt != MLXQ_UINT64) return d;
    int64_t acc = 1;
    for (int i = idx->ndim - 1; i >= 0; i--) {
      if (idx->shape[i] != 1 && idx->strides[i] != acc) return d;
      acc *= idx->shape[i];
    }
    d.ok = true;
    d.p = static_cast<const uint32_t*>(idx->data);
    d.stride = (dt == MLXQ_INT64 || dt == MLXQ_UINT64) ? 2 : 1;
    return d;
  }
  if (dflt.size() != b.size()) return d;
  size_t k = b.size();
  while (k > 0 && dflt[k - 1] == 1 && b[k - 1] != 1) k--;
  for (size_t i = 0; i < k; i++)
    if (dflt[i] != b[i]) return d;
  int64_t div = 1;
  for (size_t i = k; i < b.size(); i++) div *= b[i];
  if (div > (1 << 30)) return d;
  d.ok = true;
  d.div = (int)div;
  return d;
}

int fmt_of(Mode m, int bits) {
  if (m == MXFP4_M) return mlxq::MXFP4;
  return bits == 8 ? mlxq::AFF8 : mlxq::AFF4;
}

int gen_type(int dt) {
  if (dt == MLXQ_BFLOAT16) return mlxq::GEN_BF16;
  if (dt == MLXQ_FLOAT16) return mlxq::GEN_F16;
  if (dt == MLXQ_FLOAT32) return mlxq::GEN_F32;
  return -1;
}

// Whether the specialised kernels take a validated call: transpose=true,
// bfloat16 activations, scales, biases and result, affine 4- or 8-bit codes
// in groups of 32/64/128 or mxfp4, K a multiple of 32.  (Operands are made
// row-contiguous before the kernels run.)
bool fast_route(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* scales, const mlxq_array* biases) {
  if (!sp.transpose || sp.out_dtype != MLXQ_BFLOAT16 || x->dtype != MLXQ_BFLOAT16 || sp.K % 32 != 0) return false;
  if (sp.mode == AFFINE)
    return (sp.bits == 4 || sp.bits == 8) && (sp.gs == 32 || sp.gs == 64 || sp.gs == 128) &&
           scales->dtype == MLXQ_BFLOAT16 && (!biases || biases->dtype == MLXQ_BFLOAT16);
  return sp.mode == MXFP4_M && sp.gs == 32 && sp.bits == 4;
}

// What the general kernel (qmm_gen.hip) covers; anything else is refused
// with MLXQ_EUNSUPPORTED (the caller falls back).
void require_gen_support(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* scales, const mlxq_array* biases,
                         const char* tag) {
  if (sp.mode == NVFP4_M || sp.mode == MXFP8_M)
    unsupported(std::string(tag) + ": mode '" + (sp.mode == NVFP4_M ? "nvfp4" : "mxfp8") + "' is not implemented");
  if (sp.mode == MXFP4_M && (sp.gs != 32 || sp.bits != 4))
    unsupported(std::string(tag) + ": mxfp4 needs group_size 32 and bits 4");
  if (sp.mode == AFFINE && (sp.bits < 1 || sp.bits > 8 || sp.bits == 7))
    unsupported(std::string(tag) + ": affine bits " + std::to_string(sp.bits) + " is not implemented");
  if (sp.mode == AFFINE && sp.gs != 32 && sp.gs != 64 && sp.gs != 128)
    unsupported(std::string(tag) + ": group_size must be 32, 64 or 128");
  if (gen_type(sp.out_dtype) < 0)
    unsupported(std::string(tag) + ": result dtype " + dtype_name(sp.out_dtype) +
                " is not implemented (bfloat16, float16 and float32 are)");
  if (gen_type(x->dtype) < 0) unsupported(std::string(tag) + ": x dtype " + dtype_name(x->dtype) + " is not implemented");
  if (sp.mode == AFFINE && (gen_type(scales->dtype) < 0 || (biases && gen_type(biases->dtype) < 0)))
    unsupported(std::string(tag) + ": scales/biases dtype is not implemented");
  if (sp.K > (int64_t)1 << 30 || sp.N > (int64_t)1 << 30) unsupported(std::string(tag) + ": dimension too large");
}

// Route of a validated call: sets sp.fast, or refuses what no kernel covers.
void choose_route(QmmSpec& sp, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                  const mlxq_array* biases, const char* tag) {
  View wv{w}, sv{scales};
  const int s_esz = std::max(dtype_size(scales->dtype), biases ? dtype_size(biases->dtype) : 0);
  sp.small_w = wv.dim(-2) * wv.dim(-1) * 4 < kBufMax && sv.dim(-2) * sv.dim(-1) * s_esz < kBufMax;
  sp.fast = fast_route(sp, x, scales, biases) && sp.small_w && sp.K <= ((int64_t)1 << 30) &&
            sp.N <= ((int64_t)1 << 30);
  if (!sp.fast) require_gen_support(sp, x, scales, biases, tag);
}

void require_dtype(const mlxq_array* a, int dt, const char* name, const char* tag) {
  if (a && a->dtype != dt)
    unsupported(std::string(tag) + ": " + name + " must be " + dtype_name(dt) + " (got " + dtype_name(a->dtype) +
                ")");
}

// Skinny-kernel choice for segments of `rows` rows (measured on MI355X at the
// Llama-3-8B MLP and gpt-oss shapes): the row-streaming kernel (qmv_rs.hip)
// for 1-2 rows, the MFMA kernel (qmv.hip) for more, or when a shape is not
// covered.  MLXQ_QMV_KERNEL=fr|rs|mfma forces one (fr: the full-row kernel,
// qmv_fr.hip, 1-2 rows; rs: up to 4 rows; falling back the same way) and
// MLXQ_QMV_R sets rows per wave (fr) or per workgroup (rs): A/B switches for
// tests and measurements.
enum class Skinny { FR, RS, B4, MFMA };

// The mid-size decode kernel takes 5-16 rows (affine), where it beats the
// block-MFMA, skinny-MFMA and prefill kernels (MI355X, Llama-3-8B MLP shapes:
// 4-bit gate M=8 13.4 us vs 17.7, down M=8 16.5 us vs 33.6, gate M=16 22 us
// vs 40).
constexpr int kMidMinRows = 5;

// Row counts the default route gives the K-split-over-waves kernel over a
// matrix too small for the whole-row one: 5-8 rows at any K; 9-16 rows and,
// with 4-bit codes, 3-4 rows over at most 12 staged ranges (rows up to 12288
// long with 4-bit codes, 6144 with 8-bit).  MI355X, g64, against the split-K
// kernel: 16 rows Qwen3-8B down K = 12288 4-bit 15.3 us vs 17.0, 8-bit
// 20.5 vs 19.9, Llama-3-8B down K = 14336 4-bit 19.3 vs 17.8; 3-4 rows over
// Llama-3-8B down row streaming stays faster (4-bit 4 rows 12.9 vs 13.5,
// 8-bit 18.2 vs 21.7).
bool kq_default_rows(int fmt, int64_t rows, int64_t K) {
  const bool few_ranges = K * (fmt == mlxq::AFF8 ? 8 : 4) <= 12288 * 4;
  if (rows >= kMidMinRows && rows <= 8) return true;
  if (rows > 8 && rows <= 16) return few_ranges;
  return rows >= 3 && rows < kMidMinRows && fmt == mlxq::AFF4 && few_ranges;
}

// Defaults measured at the Llama-3-8B MLP shapes (gate K=4096, down
// K=14336): row-streaming up to 4 rows; block-MFMA for 5-8 rows of 8-bit
// and mxfp4 codes, and of 4-bit codes with K <= 8192; the MFMA kernel
// otherwise.  (Above 8 rows a dense quantized_matmul goes to the prefill
// GEMM instead, see kQmmMinRows.)
Skinny skinny_choice(int rows, int fmt = mlxq::AFF4, int64_t K = 0) {
  const std::string& k = knobs().qmv_kernel;
  if (k == "mfma") return Skinny::MFMA;
  if (k == "rs") return rows <= 4 ? Skinny::RS : Skinny::MFMA;
  if (k == "fr") return rows <= 2 ? Skinny::FR : Skinny::MFMA;
  if (k == "b4") return rows <= 16 ? Skinny::B4 : Skinny::MFMA;
  // 3-4 rows over short affine rows (less than one 16-piece chunk per
  // wave): the block-MFMA kernel with 32 weight rows per workgroup is faster
  // (MI355X, 4-bit 2880 x 2880, 3 rows: 6.6 us vs 7.7); at K = 4096 row
  // streaming is (1024 x 4096: 4.3 vs 6.9; 4096 x 4096: 6.7 vs 7.9)
  if (rows >= 3 && rows <= 4 && fmt != mlxq::MXFP4 && K * (fmt == mlxq::AFF8 ? 8 : 4) < 16384) return Skinny::B4;
  if (rows <= 4) return Skinny::RS;
  if (rows <= 8 && (fmt != mlxq::AFF4 || K <= 8192)) return Skinny::B4;
  return Skinny::MFMA;
}

// Dense (2-D weight) calls of `rows` activation rows that the mid-size decode
// kernel takes (affine only): MLXQ_QMV_KERNEL=mid forces it (up to 16 rows),
// another MLXQ_QMV_KERNEL value or MLXQ_QMV_MID=0 keeps it off.
bool use_mid(int rows, int fmt, int64_t K) {
  if (fmt == mlxq::MXFP4 || rows > 16) return false;
  const std::string& k = knobs().qmv_kernel;
  if (k == "mid" || k == "mr" || k == "kq") return true;
  if (!k.empty()) return false;
  if (knobs().qmv_mid == 0) return false;
  (void)K;
  return rows >= kMidMinRows;
}

// Launches the full-row or row-streaming kernel when chosen and covered;
// false: the caller runs the MFMA kernel.
bool try_fr_rs(const QmmSpec& sp, const mlxq::QmvArgs& a, int nseg, int rows, hipStream_t stream) {
  const int fmt = fmt_of(sp.mode, sp.bits);
  Skinny c = skinny_choice(rows, fmt, sp.K);
  const int r_req = knobs().qmv_r;
  if (c == Skinny::FR) {
    const mlxq::QmvFrPlan p = mlxq::qmv_fr_plan(fmt, sp.gs, sp.N, sp.K, rows, r_req);
    if (p.ok) {
      if (nseg > 65535) unsupported("too many segments for one launch");
      hip_check(mlxq::qmv_fr_launch(fmt, sp.gs, a, nseg, p, stream), "qmv launch");
      return true;
    }
    c = Skinny::RS;
  }
  if (c == Skinny::B4) {
    const mlxq::QmvB4Plan p = mlxq::qmv_b4_plan(fmt, sp.gs, sp.N, sp.K, rows, knobs().b4_rg,
                                                knobs().b4_cpw);
    if (p.ok) {
      if (nseg > 65535) unsupported("too many segments for one launch");
      hip_check(mlxq::qmv_b4_launch(fmt, sp.gs, a, nseg, p, stream), "qmv launch");
      return true;
    }
    c = rows <= 4 ? Skinny::RS : Skinny::MFMA;
  }
  if (c == Skinny::RS) {
    const mlxq::QmvRsPlan p = mlxq::qmv_rs_plan(fmt, sp.gs, sp.N, sp.K, rows, r_req);
    if (p.ok) {
      if (nseg > 65535) unsupported("too many segments for one launch");
      hip_check(mlxq::qmv_rs_launch(fmt, sp.gs, a, nseg, p, stream), "qmv launch");
      return true;
    }
  }
  return false;
}

// Launch the skinny kernel over `nseg` segments of at most `max_rows` rows.
void run_qmv(const QmmSpec& sp, mlxq::QmvArgs a, int nseg, int max_rows, hipStream_t stream,
             const ScratchSrc& ss) {
  if (max_rows <= 16 && try_fr_rs(sp, a, nseg, max_rows, stream)) return;
  const int fmt = fmt_of(sp.mode, sp.bits);
  const int dev = current_device();
  const DevInfo di = device_info(dev);
  int nw, pf;
  qmv_shape_choice(sp.N, sp.K, nw, pf);
  a.rows_lds = max_rows;
  mlxq::QmvPlan p = mlxq::qmv_plan(fmt, sp.gs, sp.N, sp.K, max_rows, nseg, di.cus, nw, pf);
  if (p.lds > mlxq::kQmvLdsMax) unsupported("activation tile does not fit in LDS");
  a.ks = p.ks;
  a.kst_per_wg = p.kst_per_wg;
  if (p.ks > 1) {
    const size_t ws_bytes = (size_t)p.ks * a.out_rows * sp.N * sizeof(float);
    a.ws = reinterpret_cast<float*>(workspace(dev, stream, ws_bytes, ss));
  }
  if (nseg > 65535) unsupported("too many segments for one launch");
  hip_check(mlxq::qmv_launch(fmt, sp.gs, a, nseg, p, stream), "qmv launch");
}

// Argument checks of one quantized_matmul call (the reference's validation,
// then what the kernels here cover); returns the call's spec.
QmmSpec check_quantized_matmul(const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                               const mlxq_array* biases, bool transpose, int32_t group_size, int32_t bits,
                               const char* mode, const mlxq_array* out, const char* tag) {
  QmmSpec sp = spec_quantized_matmul(x, w, scales, biases, transpose, group_size, bits, mode);
  check_out(out, sp.out_shape, sp.out_dtype, tag);
  choose_route(sp, x, w, scales, biases, tag);
  return sp;
}

// ---- row-contiguous staging of strided operands --------------------------

bool needs_staging(const mlxq_array* a) {
  if (!a || View{a}.size() == 0) return false;
  return !View{a}.row_contiguous() || (reinterpret_cast<uintptr_t>(a->data) & 15u) != 0;
}

mlxq_array contiguous_like(const mlxq_array* a, void* data) {
  mlxq_array c = *a;
  c.data = data;
  int64_t st = 1;
  for (int i = a->ndim - 1; i >= 0; i--) {
    c.strides[i] = st;
    st *= a->shape[i];
  }
  return c;
}

void copy_view(const mlxq_array* src, const mlxq_array* dst, hipStream_t stream) {
  mlxq::CopyArgs c{};
  c.src = src->data;
  c.dst = dst->data;
  c.ndim = src->ndim;
  c.esz = dtype_size(src->dtype);
  c.n = View{src}.size();
  for (int i = 0; i < src->ndim; i++) {
    c.shape[i] = src->shape[i];
    c.src_strides[i] = src->strides[i];
    c.dst_strides[i] = dst->strides[i];
  }
  hip_check(mlxq::launch_strided_copy(c, stream), "strided copy launch");
}

// The operands of one call as the kernels need them: row-contiguous and
// 16-byte aligned.  Others are first copied into the stream's staging
// workspace (as the reference copies them, rocm/quantized/qmm.hip:3557-3564);
// a strided `out` is computed into the staging buffer and copied back by
// finish().  With allow = false (the no-allocation entry point) such
// operands are refused instead.
struct Staged {
  const mlxq_array* in[4] = {nullptr, nullptr, nullptr, nullptr};  // x, w, scales, biases
  mlxq_array* out = nullptr;
  mlxq_array copies[5];
  mlxq_array* user_out = nullptr;
  hipStream_t stream = nullptr;
  void finish() {
    if (user_out) copy_view(out, user_out, stream);
  }
};

Staged stage_operands(const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                      const mlxq_array* biases, mlxq_array* out, hipStream_t stream, bool allow, const char* tag) {
  Staged st;
  st.stream = stream;
  const mlxq_array* ops[4] = {x, w, scales, biases};
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  bool need[5];
  size_t bytes = 0;
  for (int i = 0; i < 4; i++) {
    st.in[i] = ops[i];
    need[i] = needs_staging(ops[i]);
    if (need[i]) bytes += al((size_t)View{ops[i]}.size() * dtype_size(ops[i]->dtype));
  }
  st.out = out;
  need[4] = needs_staging(out);
  if (need[4]) bytes += al((size_t)View{out}.size() * dtype_size(out->dtype));
  if (bytes == 0) return st;
  if (!allow) unsupported(std::string(tag) + ": operands must be row-contiguous and 16-byte aligned");
  char* base = static_cast<char*>(workspace(current_device(), stream, bytes, ScratchSrc{}, 1));
  size_t off = 0;
  for (int i = 0; i < 4; i++) {
    if (!need[i]) continue;
    st.copies[i] = contiguous_like(ops[i], base + off);
    off += al((size_t)View{ops[i]}.size() * dtype_size(ops[i]->dtype));
    copy_view(ops[i], &st.copies[i], stream);
    st.in[i] = &st.copies[i];
  }
  if (need[4]) {
    st.copies[4] = contiguous_like(out, base + off);
    st.out = &st.copies[4];
    st.user_out = out;
  }
  return st;
}

// The general kernel (qmm_gen.hip) over nseg segments of M rows: segment s
// multiplies x batch lhs[s] by weight matrix rhs[s] (flat index lists built
// by index_prep from `ip`), or, with no `ip`, x batch 0 by matrix 0.
void run_gen(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
             const mlxq_array* biases, mlxq_array* out, int64_t M, int64_t nseg, int64_t X, int64_t E,
             mlxq::IdxPrepArgs* ip, hipStream_t stream, const ScratchSrc& ss) {
  if (nseg == 0 || M == 0 || sp.N == 0) return;
  if (sp.K == 0) unsupported("quantized_matmul: K == 0");
  const int dev = current_device();
  // 1-2 rows with transpose=true and affine codes: the decode kernel (one
  // wave per 4 weight rows, no K split); otherwise the tile kernel
  const bool dec = knobs().gen_qmv != 0 && knobs().gen_ks <= 0 &&
                   sp.mode == AFFINE && biases != nullptr && mlxq::qmv_gen_fits(mlxq::GEN_AFFINE, sp.transpose, M, sp.N, sp.K, nseg, sp.bits);
  // the same for transpose=false: column pieces over K ranges
  const mlxq::GenTPlan tp = knobs().gen_qmv != 0 && knobs().gen_ks <= 0 && sp.mode == AFFINE && biases != nullptr &&
                                    !sp.transpose
                                ? mlxq::qmv_gen_t_plan(M, sp.N, sp.K, nseg, sp.bits, mlxq::GEN_AFFINE, device_info(dev).cus)
                                : mlxq::GenTPlan{};
  const bool dect = tp.ok;
  const mlxq::GenPlan p = dec || dect ? mlxq::GenPlan{}
                                      : mlxq::gen_plan(M, sp.N, sp.K, nseg, device_info(dev).cus, knobs().gen_ks);
  if (!dec && !dect && !p.ok) unsupported("quantized matmul: too many row tiles or segments for one launch");
  const int tc = gen_type(sp.out_dtype);
  const int64_t out_elems = nseg * M * sp.N;
  auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
  const size_t idx_bytes = ip ? al((size_t)nseg * 2 * sizeof(uint32_t)) : 0;
  const int parts = dect ? tp.ks : dec ? 1 : p.ks;
  const size_t part_bytes = parts > 1 ? (size_t)parts * out_elems * sizeof(float) : 0;
  char* base = idx_bytes + part_bytes ? static_cast<char*>(workspace(dev, stream, idx_bytes + part_bytes, ss))
                                      : nullptr;
  mlxq::GenArgs a{};
  if (ip) {
    uint32_t* flat = reinterpret_cast<uint32_t*>(base);
    ip->out[0] = flat;
    ip->out[1] = flat + nseg;
    hip_check(mlxq::launch_index_prep(*ip, stream), "index_prep launch");
    a.lhs = flat;
    a.rhs = flat + nseg;
  }
  a.x = x->data;
  a.w = static_cast<const uint32_t*>(w->data);
  a.scales = scales->data;
  a.biases = biases ? biases->data : nullptr;
  a.out = out->data;
  a.ws = part_bytes ? reinterpret_cast<float*>(base + idx_bytes) : nullptr;
  a.x_dtype = gen_type(x->dtype);
  a.s_dtype = sp.mode == AFFINE ? gen_type(scales->dtype) : mlxq::GEN_BF16;
  a.b_dtype = sp.mode == AFFINE && biases ? gen_type(biases->dtype) : a.s_dtype;
  a.mode = sp.mode == MXFP4_M ? mlxq::GEN_MXFP4 : mlxq::GEN_AFFINE;
  a.bits = sp.bits;
  int shift = 0;
  while ((1 << shift) < sp.gs) shift++;
  a.gs_shift = shift;
  a.M = (int)M;
  a.N = (int)sp.N;
  a.K = (int)sp.K;
  a.X = (int)std::max<int64_t>(X, 1);
  a.E = (int)std::max<int64_t>(E, 1);
  a.x_vec = sp.K % 8 == 0;
  View wv{w}, sv{scales};
  a.w_expert_stride = wv.dim(-2) * wv.dim(-1);
  a.s_expert_stride = sv.dim(-2) * sv.dim(-1);
  a.out_elems = out_elems;
  if (dec) {
    hip_check(mlxq::qmv_gen_launch(a, tc, nseg, stream), "qmv_gen launch");
    return;
  }
  if (dect) {
    hip_check(mlxq::qmv_gen_t_launch(a, tp, tc, nseg, stream), "qmv_gen_t launch");
    if (tp.ks > 1) hip_check(mlxq::launch_gen_reduce(a.ws, out->data, out_elems, tp.ks, tc, stream), "reduce launch");
    return;
  }
  hip_check(mlxq::qmm_gen_launch(a, p, tc, sp.transpose, nseg, stream), "qmm_gen launch");
  if (p.ks > 1) hip_check(mlxq::launch_gen_reduce(a.ws, out->data, out_elems, p.ks, tc, stream), "reduce launch");
}

// Batched weights on the general kernel: the default indices of gather_qmm
// over the broadcast batch shape (x batches and weight matrices broadcast
// against it), any rows per batch.
void run_gen_batched(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                     const mlxq_array* biases, mlxq_array* out, hipStream_t stream, const ScratchSrc& ss) {
  View wv{w}, xv{x};
  if (xv.ndim() <= 2) unsupported("quantized_matmul: batched w needs batched x");
  const Shape ob(sp.out_shape.begin(), sp.out_shape.end() - 2);
  if ((int)ob.size() > MLXQ_MAX_DIMS) unsupported("quantized_matmul: batch rank too large");
  mlxq::IdxPrepArgs ip{};
  ip.bnd = (int)ob.size();
  int64_t B = 1;
  for (int d = 0; d < ip.bnd; d++) {
    ip.bshape[d] = ob[d];
    B *= ob[d];
  }
  ip.B = B;
  const Shape dx = default_index_shape(xv), dw = default_index_shape(wv);
  bstrides_for(nullptr, dx, ob, ip.bstrides[0]);
  bstrides_for(nullptr, dw, ob, ip.bstrides[1]);
  ip.dtype[0] = ip.dtype[1] = MLXQ_UINT32;
  int64_t X = 1, E = 1;
  for (auto d : dx) X *= d;
  for (auto d : dw) E *= d;
  ip.clamp[0] = std::max<int64_t>(X, 1);
  ip.clamp[1] = std::max<int64_t>(E, 1);
  run_gen(sp, x, w, scales, biases, out, xv.dim(-2), B, X, E, &ip, stream, ss);
}

// Rows [r0, r0 + rc) of a row-contiguous operand with `cols` elements per
// row, as a 2-D view.
mlxq_array rows_view(const mlxq_array* a, int64_t r0, int64_t rc, int64_t cols) {
  mlxq_array v{};
  v.data = static_cast<char*>(a->data) + r0 * cols * dtype_size(a->dtype);
  v.dtype = a->dtype;
  v.ndim = 2;
  v.shape[0] = rc;
  v.shape[1] = cols;
  v.strides[0] = cols;
  v.strides[1] = 1;
  return v;
}

// float16 decode (1-4 rows, 2-D weights): the row-streaming kernel's float16
// instantiation, when x, scales, biases and result are all float16 (affine
// 4/8-bit) or x and result are (mxfp4).  False: not covered.
bool try_rs_f16(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                const mlxq_array* biases, mlxq_array* out, int64_t rows, hipStream_t stream) {
  if (!sp.transpose || rows < 1 || rows > 4 || sp.K % 32 != 0 || sp.out_dtype != MLXQ_FLOAT16 ||
      x->dtype != MLXQ_FLOAT16 || knobs().qmv_kernel == "mr" || knobs().qmv_kernel == "mid")
    return false;
  if (sp.mode == AFFINE) {
    if ((sp.bits != 4 && sp.bits != 8) || (sp.gs != 32 && sp.gs != 64 && sp.gs != 128)) return false;
    if (scales->dtype != MLXQ_FLOAT16 || !biases || biases->dtype != MLXQ_FLOAT16) return false;
  } else if (sp.mode != MXFP4_M || sp.gs != 32 || sp.bits != 4) {
    return false;
  }
  const int fmt = fmt_of(sp.mode, sp.bits);
  const mlxq::QmvRsPlan p = mlxq::qmv_rs_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, knobs().qmv_r);
  if (!p.ok) return false;
  mlxq::QmvArgs a{};
  a.x = static_cast<const uint16_t*>(x->data);
  a.w = static_cast<const uint32_t*>(w->data);
  a.scales = scales->data;
  a.biases = biases ? static_cast<const uint16_t*>(biases->data) : nullptr;
  a.out = static_cast<uint16_t*>(out->data);
  a.N = (int)sp.N;
  a.K = (int)sp.K;
  a.E = 1;
  a.X = 1;
  a.rps = (int)rows;
  a.total_rows = (int)rows;
  a.out_rows = (int)rows;
  a.xt = 1;
  hip_check(mlxq::qmv_rs_launch(fmt, sp.gs, a, 1, p, stream), "qmv launch");
  return true;
}

// float16 x / scales / biases / result, affine 4/8-bit codes (the mid-size
// decode kernels' float16 instantiations)
bool f16_affine(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* scales, const mlxq_array* biases) {
  return sp.transpose && sp.mode == AFFINE && (sp.bits == 4 || sp.bits == 8) && x->dtype == MLXQ_FLOAT16 &&
         sp.out_dtype == MLXQ_FLOAT16 && scales->dtype == MLXQ_FLOAT16 && biases && biases->dtype == MLXQ_FLOAT16;
}

// float16, 5-16 rows (3-4 for 4-bit codes; any row count when
// MLXQ_QMV_KERNEL=mr) against a matrix with ~one 64-row block per CU: the
// whole-row mid-size kernel (gate/up M=8 10.8 us vs 55 on the general kernel).
bool try_mr_f16(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                const mlxq_array* biases, mlxq_array* out, int64_t rows, hipStream_t stream) {
  const bool forced = knobs().qmv_kernel == "mr";
  if (!f16_affine(sp, x, scales, biases) || rows < 1 || rows > 16) return false;
  const int64_t min_rows = sp.bits == 4 ? 3 : kMidMinRows;
  if (!forced && (rows < min_rows || knobs().qmv_mr == 0 || !knobs().qmv_kernel.empty())) return false;
  const int fmt = fmt_of(sp.mode, sp.bits);
  const int cus = device_info(current_device()).cus;
  const mlxq::QmvMrPlan rp = mlxq::qmv_mr_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, forced, knobs().mr_ring);
  if (!rp.ok) return false;
  // past one round of the CUs, 4-bit codes take the split-K kernel where it
  // applies, and at 9-16 rows the K-split-over-waves kernel where its tiles
  // fit one round three to a workgroup, as bfloat16 calls do
  if (!forced && fmt == mlxq::AFF4 && rp.row_blocks > cus && use_mid((int)rows, fmt, sp.K) &&
      mlxq::qmv_mid_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, knobs().mid_win).ok)
    return false;
  if (!forced && fmt == mlxq::AFF4 && rows > 8 && knobs().qmv_kq != 0 && kq_default_rows(fmt, rows, sp.K)) {
    const mlxq::QmvMrPlan kp = mlxq::qmv_kq_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, knobs().kq_t);
    if (kp.ok && kp.t <= 3) return false;
  }
  mlxq::QmvMrArgs m{};
  m.x = static_cast<const uint16_t*>(x->data);
  m.w = static_cast<const uint32_t*>(w->data);
  m.scales = static_cast<const uint16_t*>(scales->data);
  m.biases = static_cast<const uint16_t*>(biases->data);
  m.out = static_cast<uint16_t*>(out->data);
  m.M = (int)rows;
  m.N = (int)sp.N;
  m.K = (int)sp.K;
  int shift = 0;
  while ((1 << shift) < sp.gs) shift++;
  m.gs_shift = shift;
  m.xt = 1;
  hip_check(mlxq::qmv_mr_launch(fmt, m, rp, stream), "qmv_mr launch");
  return true;
}

// float16 over matrices with too few rows for the whole-row kernel: the
// K-split-over-waves kernel at the bfloat16 route's row counts
// (kq_default_rows; any row count when MLXQ_QMV_KERNEL=kq).
bool try_kq_f16(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                const mlxq_array* biases, mlxq_array* out, int64_t rows, hipStream_t stream) {
  const bool forced = knobs().qmv_kernel == "kq";
  if (!f16_affine(sp, x, scales, biases) || rows < 1 || rows > 16) return false;
  const int fmt = fmt_of(sp.mode, sp.bits);
  const int cus = device_info(current_device()).cus;
  if (!forced) {
    if (knobs().qmv_kq == 0 || !knobs().qmv_kernel.empty()) return false;
    if (!kq_default_rows(fmt, rows, sp.K)) return false;
    if (rows < kMidMinRows && mlxq::qmv_mr_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, false, 0).ok) return false;
  }
  const mlxq::QmvMrPlan kp = mlxq::qmv_kq_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, knobs().kq_t);
  if (!kp.ok) return false;
  mlxq::QmvMrArgs m{};
  m.x = static_cast<const uint16_t*>(x->data);
  m.w = static_cast<const uint32_t*>(w->data);
  m.scales = static_cast<const uint16_t*>(scales->data);
  m.biases = static_cast<const uint16_t*>(biases->data);
  m.out = static_cast<uint16_t*>(out->data);
  m.M = (int)rows;
  m.N = (int)sp.N;
  m.K = (int)sp.K;
  int shift = 0;
  while ((1 << shift) < sp.gs) shift++;
  m.gs_shift = shift;
  m.xt = 1;
  hip_check(mlxq::qmv_mr_launch(fmt, m, kp, stream), "qmv_kq launch");
  return true;
}

// float16, 5-16 rows (any row count when MLXQ_QMV_KERNEL=mid), other
// matrices: the split-K mid-size kernel (down M=8: vs 84 us on the general
// kernel).
bool try_mid_f16(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                 const mlxq_array* biases, mlxq_array* out, int64_t rows, hipStream_t stream, const ScratchSrc& ss) {
  const bool forced = knobs().qmv_kernel == "mid";
  if (!f16_affine(sp, x, scales, biases) || rows < 1 || rows > 16) return false;
  if (!forced && (rows < kMidMinRows || knobs().qmv_mid == 0 || !knobs().qmv_kernel.empty())) return false;
  const int fmt = fmt_of(sp.mode, sp.bits);
  const mlxq::QmvMidPlan mp =
      mlxq::qmv_mid_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, device_info(current_device()).cus, knobs().mid_win);
  if (!mp.ok) return false;
  const int dev = current_device();
  mlxq::QmvMidArgs m{};
  m.x = static_cast<const uint16_t*>(x->data);
  m.w = static_cast<const uint32_t*>(w->data);
  m.scales = static_cast<const uint16_t*>(scales->data);
  m.biases = static_cast<const uint16_t*>(biases->data);
  m.out = static_cast<uint16_t*>(out->data);
  m.M = (int)rows;
  m.N = (int)sp.N;
  m.K = (int)sp.K;
  int shift = 0;
  while ((1 << shift) < sp.gs) shift++;
  m.gs_shift = shift;
  m.ks = mp.ks;
  m.xt = 1;
  m.red_vec = knobs().red_vec;
  if (mp.ks > 1)
    m.ws = reinterpret_cast<float*>(workspace(dev, stream, (size_t)mp.ks * rows * sp.N * sizeof(float), ss));
  hip_check(mlxq::qmv_mid_launch(fmt, m, mp, stream), "qmv_mid launch");
  return true;
}

// float16 prefill (rows >= MLXQ_QMM_MIN_ROWS once the mid-size kernels have
// declined): the 32x32-MFMA tile kernel's float16 instantiation; a requested
// tile of the 16x16-MFMA kernel (bfloat16 only) falls back to the planner's.
bool try_qmm_f16(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                 const mlxq_array* biases, mlxq_array* out, int64_t rows, hipStream_t stream, const ScratchSrc& ss) {
  if (!f16_affine(sp, x, scales, biases) || rows < knobs().qmm_min_rows) return false;
  const int fmt = fmt_of(sp.mode, sp.bits);
  const int dev = current_device();
  const int tile_req = knobs().qmm_tile >= 4 ? knobs().qmm_tile : -1;
  uint32_t* cnt = nullptr;
  const mlxq::QmmPlan qp = prefill_plan(fmt, sp.gs, rows, sp.N, sp.K, dev, stream, ss, tile_req, knobs().qmm_ksplit,
                                        knobs().qmm_mix, knobs().qmm_streamk, &cnt);
  if (!qp.ok || qp.tile < 4) return false;
  mlxq::QmmArgs q{};
  q.x = static_cast<const uint16_t*>(x->data);
  q.w = static_cast<const uint32_t*>(w->data);
  q.scales = scales->data;
  q.biases = static_cast<const uint16_t*>(biases->data);
  q.out = static_cast<uint16_t*>(out->data);
  q.M = (int)rows;
  q.x_rows = (int)rows;
  q.N = (int)sp.N;
  q.K = (int)sp.K;
  int shift = 0;
  while ((1 << shift) < sp.gs) shift++;
  q.gs_shift = shift;
  q.ksplit = qp.ksplit;
  q.ksteps_per_split = qp.ksteps_per_split;
  q.xt = 1;
  if (qp.ksplit > 1)
    q.ws = reinterpret_cast<float*>(workspace(dev, stream, (size_t)qp.ksplit * rows * sp.N * sizeof(float), ss));
  if (qp.sk_len > 0) {
    q.ws = reinterpret_cast<float*>(workspace(dev, stream, (size_t)mlxq::qmm_sk_bytes(qp), ss));
    q.cnt = cnt;
    q.sk_fallback = knobs().sk_fallback;
  }
  hip_check(mlxq::qmm_launch(fmt, q, qp, stream), "qmm launch");
  return true;
}

// Route of a dense (2-D weight) bfloat16 call of `rows` activation rows on
// the mid-size decode kernels, or DR_OTHER (row streaming, block MFMA,
// prefill GEMM):
// - 3-4 rows of 4-bit codes against a tall matrix: the whole-row kernel also
//   beats the block-MFMA kernel (gate/up M=4: 10.4 us vs 12.6; 8-bit keeps
//   the row-streaming kernel: 15.3 us vs 16.3);
// - 5-16 rows: matrices with ~one 64-row workgroup per CU take the whole-row
//   kernel, one launch (qmv_mr.hip), faster than the split-K kernel at every
//   row count (MI355X, Llama-3-8B gate/up, graph-timed: 4-bit M=8 10.5 us vs
//   12.4, M=16 15.3 vs 15.6-16.7; 8-bit M=8 16.7 vs 20.8, M=16 17.4 vs 21.8);
//   other matrices the split-K kernel (activations staged once per 128
//   weight rows, fp32 partials of the K ranges added by a second launch,
//   qmv_mid.hip).
enum DenseKind { DR_OTHER, DR_MR, DR_MID };
struct DenseRoute {
  DenseKind kind = DR_OTHER;
  mlxq::QmvMrPlan mr;
  mlxq::QmvMidPlan mid;
};

// single: a call of its own (false for the projections of a fused launch,
// whose kernels must agree).
DenseRoute dense_route(const QmmSpec& sp, int64_t rows, int cus, bool single = true) {
  DenseRoute r;
  const int fmt = fmt_of(sp.mode, sp.bits);
  if (rows < 1 || rows > 16) return r;
  const std::string& forced = knobs().qmv_kernel;
  const mlxq::QmvMrPlan mr0 = mlxq::qmv_mr_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, false, 0);
  const bool mr_fits = mr0.ok;
  // Single calls of 4-bit codes (MI355X, g64, K=4096, graph-timed):
  // - 3-4 rows past one round of the CUs: the split-K kernel (151936 rows:
  //   78.3 us vs 84.3 whole-row at 3 rows, 79.4 vs 85.4 at 4);
  // - 9-16 rows over a matrix whose 16-row tiles fit one round three to a
  //   workgroup: the K-split-over-waves kernel (12288 rows: 12 rows 12.6 us
  //   vs 14.2 whole-row, 16 rows 12.9 vs 14.5; 14336 rows need four tiles
  //   per workgroup and stay whole-row, 14.9 vs 14.5).
  if (single && forced.empty() && fmt == mlxq::AFF4 && knobs().qmv_mr != 0) {
    if (rows >= 3 && rows < kMidMinRows && mr_fits && mr0.row_blocks > cus && knobs().qmv_mid != 0) {
      r.mid = mlxq::qmv_mid_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, knobs().mid_win);
      if (r.mid.ok) {
        r.kind = DR_MID;
        return r;
      }
    }
    if (rows > 8 && mr_fits && knobs().qmv_kq != 0 && kq_default_rows(fmt, rows, sp.K)) {
      const mlxq::QmvMrPlan kp = mlxq::qmv_kq_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, knobs().kq_t);
      if (kp.ok && kp.t <= 3) {
        r.mr = kp;
        r.kind = DR_MR;
        return r;
      }
    }
  }
  const bool mr_small = rows >= 3 && rows < kMidMinRows && fmt == mlxq::AFF4 && knobs().qmv_mr != 0 &&
                        forced.empty() && mr_fits;
  // 3-4 rows over matrices with too few rows for the whole-row kernel: the
  // K-split-over-waves kernel below where kq_default_rows allows (MI355X,
  // Qwen3-8B, 4-bit g64, 3-4 rows: o 5.9 us vs 7.8 on the block-MFMA kernel,
  // q/k/v in one launch 7.8 vs 23.2 as three, down K = 12288 11.3 vs 11.8 on
  // row streaming; row streaming stays faster at 2 rows, o 4.7 vs 5.9)
  const bool kq_small = rows >= 3 && rows < kMidMinRows && forced.empty() && knobs().qmv_kq != 0 && !mr_fits &&
                        kq_default_rows(fmt, rows, sp.K);
  if (!mr_small && !kq_small && !use_mid((int)rows, fmt, sp.K)) return r;
  if (!kq_small && (forced == "mr" || (knobs().qmv_mr != 0 && forced.empty()))) {
    r.mr = mlxq::qmv_mr_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, forced == "mr", knobs().mr_ring);
    // The whole-row kernel holds one 64-row block per CU at a time: past one
    // round of the CUs the split-K mid-size kernel is faster for 4-bit codes
    // where it applies (MI355X, 4-bit g64 K=4096: 151936 rows, 2374 blocks,
    // 16 rows 133 -> 124 us, 8 rows 88.7 -> 85.6; 12288 rows, 192 blocks,
    // stays whole-row); 8-bit codes stay whole-row at any size (151936
    // rows: 5 rows 131 us vs 175 on the split-K kernel, 16 rows 155 vs 194;
    // 24576 rows 29.4 vs 33.0)
    if (r.mr.ok && !(forced.empty() && fmt == mlxq::AFF4 && r.mr.row_blocks > cus &&
                     use_mid((int)rows, fmt, sp.K) &&
                     mlxq::qmv_mid_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, knobs().mid_win).ok)) {
      r.kind = DR_MR;
      return r;
    }
  }
  // Matrices that fit one round of the CUs in workgroups of 16-64 rows
  // (q / k / v / o / down at 7-8B shapes): every workgroup walks the whole
  // of K with the K windows split over its waves, so no second launch adds
  // K ranges; the row counts of kq_default_rows.
  if (forced == "kq" || kq_small ||
      (forced.empty() && knobs().qmv_kq != 0 && rows >= kMidMinRows && kq_default_rows(fmt, rows, sp.K))) {
    r.mr = mlxq::qmv_kq_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, knobs().kq_t);
    if (r.mr.ok) {
      r.kind = DR_MR;
      return r;
    }
  }
  if (kq_small) return r;  // not planned: the 1-4-row kernels
  r.mid = mlxq::qmv_mid_plan(fmt, sp.gs, sp.N, sp.K, (int)rows, cus, knobs().mid_win);
  if (r.mid.ok) r.kind = DR_MID;
  return r;
}

int gs_shift_of(int gs) {
  int shift = 0;
  while ((1 << shift) < gs) shift++;
  return shift;
}

mlxq::QmvMrArgs mr_args(const QmmSpec& sp, const uint16_t* x, int64_t rows, const uint32_t* w, const void* scales,
                        const uint16_t* biases, uint16_t* out) {
  mlxq::QmvMrArgs m{};
  m.x = x;
  m.w = w;
  m.scales = static_cast<const uint16_t*>(scales);
  m.biases = biases;
  m.out = out;
  m.M = (int)rows;
  m.N = (int)sp.N;
  m.K = (int)sp.K;
  m.gs_shift = gs_shift_of(sp.gs);
  return m;
}

mlxq::QmvMidArgs mid_args(const QmmSpec& sp, const uint16_t* x, int64_t rows, const uint32_t* w,
                          const void* scales, const uint16_t* biases, uint16_t* out, int ks) {
  mlxq::QmvMidArgs m{};
  m.x = x;
  m.w = w;
  m.scales = static_cast<const uint16_t*>(scales);
  m.biases = biases;
  m.out = out;
  m.M = (int)rows;
  m.N = (int)sp.N;
  m.K = (int)sp.K;
  m.gs_shift = gs_shift_of(sp.gs);
  m.ks = ks;
  m.red_vec = knobs().red_vec;
  return m;
}

// Several projections of one activation block (quantized_matmul_multi) on
// the whole-row or split-K mid-size kernel as one launch (the split-K
// partials of all matrices summed by one reduction launch).  False: the
// projections take different kernels or plans (the caller runs them one by
// one).
bool try_multi_mid(const std::vector<QmmSpec>& sp, int n, const mlxq_array* x, const mlxq_array* const* w,
                   const mlxq_array* const* scales, const mlxq_array* const* biases, mlxq_array* const* out,
                   int64_t rows, hipStream_t stream) {
  const int dev = current_device();
  const int cus = device_info(dev).cus;
  const int fmt = fmt_of(sp[0].mode, sp[0].bits);
  if (sp[0].mode != AFFINE) return false;
  std::vector<DenseRoute> r;
  for (int i = 0; i < n; i++) {
    if (sp[i].N == 0 || sp[i].K != sp[0].K || sp[i].gs != sp[0].gs) return false;
    r.push_back(dense_route(sp[i], rows, cus, false));
    if (r[i].kind == DR_OTHER || r[i].kind != r[0].kind) return false;
    if (r[i].kind == DR_MR) {
      const mlxq::QmvMrPlan &a = r[i].mr, &b = r[0].mr;
      if (a.s != b.s || a.na != b.na || a.xr != b.xr || a.rk != b.rk || a.ring != b.ring || a.lds != b.lds ||
          (a.t > 0) != (b.t > 0))
        return false;
    } else {
      const mlxq::QmvMidPlan &a = r[i].mid, &b = r[0].mid;
      if (a.s != b.s || a.na != b.na || a.kr != b.kr || a.ks != b.ks || a.sw != b.sw || a.lds != b.lds) return false;
    }
  }
  // The whole-row kernel runs one 64-row block per CU at a time: where the
  // projections' blocks together need more than one round of the CUs
  // (gate + up, 2 x 12288 rows: 384 blocks), the split-K mid-size kernel
  // takes the launch instead for 4-bit codes, if it covers every projection
  // alike (MI355X, Qwen3-8B gate + up, 4-bit g64: 16 rows 27.8 -> 24.6 us,
  // 8 rows 19.2 -> 18.3; 8-bit codes stay whole-row, 16 rows 31.7 us vs
  // 34.8).  Each output then has the mid-size kernel's bits (those of
  // single calls with MLXQ_QMV_MR=0), within tolerance of the single calls'.
  // K split over the waves: one tile count for all projections, the
  // fewest whose blocks together fit one round of the CUs (else the
  // projections run one by one).
  if (r[0].kind == DR_MR && r[0].mr.t > 0) {
    const int t_req = knobs().kq_t;
    bool planned = false;
    for (int t = 1; t <= 4; t++) {
      if (planned || (mlxq::kq_tiles_ok(t_req) && t != t_req)) continue;
      int64_t blocks = 0;
      bool ok = true;
      std::vector<DenseRoute> m(r);
      for (int i = 0; i < n && ok; i++) {
        m[i].mr = mlxq::qmv_kq_plan(fmt, sp[i].gs, sp[i].N, sp[i].K, (int)rows, cus, t, 0);
        ok = m[i].mr.ok && m[i].mr.lds == m[0].mr.lds;
        blocks += m[i].mr.row_blocks;
      }
      if (ok && (blocks <= cus || mlxq::kq_tiles_ok(t_req))) {
        r = m;
        planned = true;
      }
    }
    if (!planned) return false;
  }
  if (r[0].kind == DR_MR && r[0].mr.t == 0 && knobs().qmv_kernel.empty() && fmt == mlxq::AFF4 &&
      use_mid((int)rows, fmt, sp[0].K)) {
    int64_t mr_blocks = 0;
    for (int i = 0; i < n; i++) mr_blocks += r[i].mr.row_blocks;
    if (mr_blocks > cus) {
      std::vector<DenseRoute> m(r);
      bool ok = true;
      for (int i = 0; i < n && ok; i++) {
        m[i].kind = DR_MID;
        m[i].mid = mlxq::qmv_mid_plan(fmt, sp[i].gs, sp[i].N, sp[i].K, (int)rows, cus, knobs().mid_win);
        const mlxq::QmvMidPlan &a = m[i].mid, &b0 = m[0].mid;
        ok = a.ok && a.s == b0.s && a.na == b0.na && a.kr == b0.kr && a.ks == b0.ks && a.sw == b0.sw &&
             a.lds == b0.lds;
      }
      if (ok) r = m;
    }
  }
  mlxq::QmvMatTable t{};
  t.n = n;
  int64_t blocks = 0, ntot = 0;
  for (int i = 0; i < n; i++) {
    blocks += r[i].kind == DR_MR ? r[i].mr.row_blocks : r[i].mid.row_blocks;
    t.blk_end[i] = (int)blocks;
    t.N[i] = (int)sp[i].N;
    t.noff[i] = (int)ntot;
    ntot += sp[i].N;
    t.w[i] = static_cast<const uint32_t*>(w[i]->data);
    t.scales[i] = static_cast<const uint16_t*>(scales[i]->data);
    t.biases[i] = static_cast<const uint16_t*>(biases[i]->data);
    t.out[i] = static_cast<uint16_t*>(out[i]->data);
  }
  for (int i = n; i < mlxq::kQmvMultiMax; i++) {  // unused entries repeat the last one
    t.blk_end[i] = t.blk_end[n - 1];
    t.N[i] = t.N[n - 1];
    t.noff[i] = t.noff[n - 1];
    t.w[i] = t.w[n - 1];
    t.scales[i] = t.scales[n - 1];
    t.biases[i] = t.biases[n - 1];
    t.out[i] = t.out[n - 1];
  }
  if (blocks > 65535 || ntot >= ((int64_t)1 << 30)) return false;
  t.ntot = (int)ntot;
  const uint16_t* xd = static_cast<const uint16_t*>(x->data);
  if (r[0].kind == DR_MR) {
    mlxq::QmvMrArgs m = mr_args(sp[0], xd, rows, t.w[0], t.scales[0], t.biases[0], t.out[0]);
    m.mt = t;
    mlxq::QmvMrPlan p = r[0].mr;
    p.row_blocks = (int)blocks;
    hip_check(mlxq::qmv_mr_launch(fmt, m, p, stream), "qmv_mr launch");
    return true;
  }
  mlxq::QmvMidPlan p = r[0].mid;
  p.row_blocks = (int)blocks;
  mlxq::QmvMidArgs m = mid_args(sp[0], xd, rows, t.w[0], t.scales[0], t.biases[0], t.out[0], p.ks);
  m.mt = t;
  if (p.ks > 1) {
    const size_t part = (size_t)p.ks * rows * ntot * sizeof(float);
    if ((int64_t)part >= kBufMax) return false;
    m.ws = reinterpret_cast<float*>(workspace(dev, stream, part));
  }
  hip_check(mlxq::qmv_mid_launch(fmt, m, p, stream), "qmv_mid launch");
  return true;
}

// Enqueues one checked quantized_matmul call.
void run_quantized_matmul(const QmmSpec& sp, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                          const mlxq_array* biases, mlxq_array* out, hipStream_t stream,
                          const ScratchSrc& ss = ScratchSrc{}) {
  const int64_t rows_total = View{out}.size() / std::max<int64_t>(sp.N, 1);
  if (rows_total == 0 || sp.N == 0) return;
  if (sp.K == 0) unsupported("quantized_matmul: K == 0");
  if (View{w}.ndim() == 2) {
    // Rows of x and out are independent: activations or results of 2 GiB
    // and more run as row chunks below the limit, each on the same kernels
    // (operands are row-contiguous here, after staging).
    const int64_t per_row = std::max(sp.K * dtype_size(x->dtype), sp.N * dtype_size(out->dtype));
    if (per_row >= kBufMax) unsupported("quantized_matmul: one row of x or of the result reaches 2 GiB");
    if (rows_total * per_row >= kBufMax) {
      // equal chunks (a small last one would plan differently, e.g. split K),
      // multiples of 256 rows where possible, so chunk starts stay 16-byte aligned
      const int64_t max_rows = (kBufMax - 1) / per_row;
      const int64_t n = (rows_total + max_rows - 1) / max_rows;
      int64_t chunk = (rows_total + n - 1) / n;
      if (((chunk + 255) & ~(int64_t)255) <= max_rows) chunk = (chunk + 255) & ~(int64_t)255;
      else if (max_rows >= 256) chunk = max_rows & ~(int64_t)255;
      else chunk = max_rows;
      for (int64_t r0 = 0; r0 < rows_total; r0 += chunk) {
        const int64_t rc = std::min(chunk, rows_total - r0);
        mlxq_array xc = rows_view(x, r0, rc, sp.K), oc = rows_view(out, r0, rc, sp.N);
        run_quantized_matmul(sp, &xc, w, scales, biases, &oc, stream, ss);
      }
      return;
    }
  }
  if (!sp.fast) {
    View wv{w};
    const bool dense = wv.ndim() == 2 && sp.small_w;  // the float16 routes use buffer resources too
    if (dense && try_mr_f16(sp, x, w, scales, biases, out, rows_total, stream)) return;
    if (dense && try_kq_f16(sp, x, w, scales, biases, out, rows_total, stream)) return;
    if (dense && try_rs_f16(sp, x, w, scales, biases, out, rows_total, stream)) return;
    if (dense && try_mid_f16(sp, x, w, scales, biases, out, rows_total, stream, ss)) return;
    if (dense && try_qmm_f16(sp, x, w, scales, biases, out, rows_total, stream, ss)) return;
    if (wv.ndim() == 2) {
      // every leading dim of x folds into rows
      run_gen(sp, x, w, scales, biases, out, rows_total, 1, 1, 1, nullptr, stream, ss);
      return;
    }
    run_gen_batched(sp, x, w, scales, biases, out, stream, ss);
    return;
  }

  mlxq::QmvArgs a{};
  a.x = static_cast<const uint16_t*>(x->data);
  a.w = static_cast<const uint32_t*>(w->data);
  a.scales = scales->data;
  a.biases = biases ? static_cast<const uint16_t*>(biases->data) : nullptr;
  a.out = static_cast<uint16_t*>(out->data);
  a.N = (int)sp.N;
  a.K = (int)sp.K;
  a.out_rows = (int)rows_total;
  const int fmt = fmt_of(sp.mode, sp.bits);
  const int cap = mlxq::qmv_max_rows(fmt, sp.gs);
  View wv{w}, xv{x};
  if (wv.ndim() == 2) {
    const DenseRoute dr = dense_route(sp, rows_total, device_info(current_device()).cus);
    if (dr.kind == DR_MR) {
      mlxq::QmvMrArgs m = mr_args(sp, a.x, rows_total, a.w, a.scales, a.biases, a.out);
      hip_check(mlxq::qmv_mr_launch(fmt, m, dr.mr, stream), "qmv_mr launch");
      return;
    }
    if (dr.kind == DR_MID) {
      mlxq::QmvMidArgs m = mid_args(sp, a.x, rows_total, a.w, a.scales, a.biases, a.out, dr.mid.ks);
      if (dr.mid.ks > 1)
        m.ws = reinterpret_cast<float*>(
            workspace(current_device(), stream, (size_t)dr.mid.ks * rows_total * sp.N * sizeof(float), ss));
      hip_check(mlxq::qmv_mid_launch(fmt, m, dr.mid, stream), "qmv_mid launch");
      return;
    }
  }
  if (wv.ndim() == 2 && rows_total >= knobs().qmm_min_rows) {
    // prefill: one GEMM over all rows (every leading dim of x folds into rows)
    const int dev = current_device();
    // MLXQ_QMM_TILE / MLXQ_QMM_KSPLIT: A/B overrides of the tile shape and K split
    uint32_t* cnt = nullptr;
    const mlxq::QmmPlan qp = prefill_plan(fmt, sp.gs, rows_total, sp.N, sp.K, dev, stream, ss, knobs().qmm_tile,
                                          knobs().qmm_ksplit, knobs().qmm_mix, knobs().qmm_streamk, &cnt);
    if (qp.ok) {
      mlxq::QmmArgs q{};
      q.x = a.x;
      q.w = a.w;
      q.scales = a.scales;
      q.biases = a.biases;
      q.out = a.out;
      q.M = (int)rows_total;
      q.x_rows = (int)rows_total;
      q.N = (int)sp.N;
      q.K = (int)sp.K;
      int shift = 0;
      while ((1 << shift) < sp.gs) shift++;
      q.gs_shift = shift;
      q.ksplit = qp.ksplit;
      q.ksteps_per_split = qp.ksteps_per_split;
      if (qp.ksplit > 1)
        q.ws = reinterpret_cast<float*>(
            workspace(dev, stream, (size_t)qp.ksplit * rows_total * sp.N * sizeof(float), ss));
      if (qp.sk_len > 0) {
        q.ws = reinterpret_cast<float*>(workspace(dev, stream, (size_t)mlxq::qmm_sk_bytes(qp), ss));
        q.cnt = cnt;
        q.sk_fallback = knobs().sk_fallback;
      }
      hip_check(mlxq::qmm_launch(fmt, q, qp, stream), "qmm launch");
      return;
    }
  }
  if (wv.ndim() == 2) {
    // every leading dim of x folds into rows (qmm.hip:3606-3620 does the same fold)
    a.E = 1;
    a.X = 1;
    a.w_expert_stride = 0;
    a.s_expert_stride = 0;
    int rps = (int)std::min<int64_t>(rows_total, cap);
    {
      int nw, pf;
      qmv_shape_choice(sp.N, sp.K, nw, pf);
      const DevInfo di = device_info(current_device());
      while (rps > 1 && mlxq::qmv_plan(fmt, sp.gs, sp.N, sp.K, rps, 1, di.cus, nw, pf).lds > mlxq::kQmvLdsMax)
        rps = (rps + 1) / 2;
    }
    a.rps = rps;
    a.total_rows = (int)rows_total;
    a.X = (int)((rows_total + rps - 1) / rps);
    const int nseg = a.X;
    run_qmv(sp, a, nseg, rps, stream, ss);
  } else {
    // batched weights: each batch element is a segment of x.shape[-2] rows
    const Shape wsh = wv.shape(), xsh = xv.shape();
    Shape wb(wsh.begin(), wsh.end() - 2);
    Shape ob(sp.out_shape.begin(), sp.out_shape.end() - 2);
    Shape xb = xv.ndim() > 2 ? Shape(xsh.begin(), xsh.end() - 2) : Shape{};
    // Batches that broadcast, or more rows per batch than the decode kernels
    // stage (the reference takes any M: qmm.hip:3606-3620, 2362-2766), run
    // on the general kernel over the default gather indices.
    if (xv.ndim() <= 2 || wb != ob || xb != ob || xv.dim(-2) > cap) {
      run_gen_batched(sp, x, w, scales, biases, out, stream, ss);
      return;
    }
    const int64_t M = xv.dim(-2);
    int64_t nb = 1;
    for (auto d : wb) nb *= d;
    // so do batches whose rows' activation tile does not fit the skinny
    // kernel's LDS (e.g. 64 rows of 4-bit g128 codes)
    if (M > 16) {
      int nw, pf;
      qmv_shape_choice(sp.N, sp.K, nw, pf);
      const mlxq::QmvPlan qp = mlxq::qmv_plan(fmt, sp.gs, sp.N, sp.K, (int)M, (int)nb,
                                              device_info(current_device()).cus, nw, pf);
      if (qp.lds > mlxq::kQmvLdsMax) {
        run_gen_batched(sp, x, w, scales, biases, out, stream, ss);
        return;
      }
    }
    a.E = (int)nb;
    a.X = (int)nb;
    a.w_expert_stride = wv.dim(-2) * wv.dim(-1);
    a.s_expert_stride = View{scales}.dim(-2) * View{scales}.dim(-1);
    a.rps = (int)M;
    a.total_rows = (int)rows_total;
    run_qmv(sp, a, (int)nb, (int)M, stream, ss);
  }
}

const char* mode_name(Mode m) {
  return m == AFFINE ? "affine" : (m == MXFP4_M ? "mxfp4" : (m == MXFP8_M ? "mxfp8" : "nvfp4"));
}

// A row-contiguous operand as [batch, rows, cols] (its leading dims folded).
mlxq_array as3(const mlxq_array* a, int64_t batch) {
  mlxq_array v = *a;
  View av{a};
  v.ndim = 3;
  v.shape[0] = batch;
  v.shape[1] = av.dim(-2);
  v.shape[2] = av.dim(-1);
  v.strides[2] = 1;
  v.strides[1] = v.shape[2];
  v.strides[0] = v.shape[1] * v.shape[2];
  return v;
}

// A contiguous 1-D uint32 array of n entries.
mlxq_array u32_view(uint32_t* p, int64_t n) {
  mlxq_array v{};
  v.data = p;
  v.dtype = MLXQ_UINT32;
  v.ndim = 1;
  v.shape[0] = n;
  v.strides[0] = 1;
  return v;
}

void gather_run(GatherSpec& g, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                const mlxq_array* biases, const mlxq_array* lhs_indices, const mlxq_array* rhs_indices,
                bool sorted_indices, mlxq_array* out, hipStream_t stream);

// A gather with more index entries than one launch covers (the reference's
// dispatch has no cap, qmm.hip:6590; nor its CPU gather, quantized.cpp:764-813):
// the flat uint32 indices of every entry (clamped by index_prep) go to the
// stream's workspace slot 2, then the entries run in chunks of kGatherChunk,
// each a gather with contiguous index arrays over the same x and w.  A chunk
// of a sorted rhs is sorted, and where the default lhs maps entry b to x batch
// b the chunk keeps the default over the matching slice of x, so the sorted
// routes stay open.  The chunks' own scratch lives in slots 0 and 1.
void gather_chunked(const GatherSpec& g, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                    const mlxq_array* biases, const mlxq_array* lhs_indices, bool sorted_indices,
                    mlxq_array* out, hipStream_t stream, mlxq::IdxPrepArgs ip, int64_t B, int64_t X, int64_t E) {
  const QmmSpec& sp = g.q;
  View xv{x};
  const int64_t M = xv.dim(-2);
  if (B >= ((int64_t)1 << 30)) unsupported("gather_qmm: more than 2^30 index entries");
  uint32_t* flat = static_cast<uint32_t*>(
      workspace(current_device(), stream, (size_t)B * 2 * sizeof(uint32_t), ScratchSrc{}, 2));
  ip.out[0] = flat;
  ip.out[1] = flat + B;
  hip_check(mlxq::launch_index_prep(ip, stream), "index_prep launch");
  const bool lhs_default = !lhs_indices && default_index_shape(xv) == g.idx_shape;
  const mlxq_array x3 = as3(x, X), w3 = as3(w, E), s3 = as3(scales, E);
  const mlxq_array b3 = biases ? as3(biases, E) : mlxq_array{};
  const int64_t xrow = M * sp.K * dtype_size(x->dtype), orow = M * sp.N * dtype_size(out->dtype);
  for (int64_t c0 = 0; c0 < B; c0 += kGatherChunk) {
    const int64_t cb = std::min(kGatherChunk, B - c0);
    mlxq_array li = u32_view(flat + c0, cb), ri = u32_view(flat + B + c0, cb);
    mlxq_array xc = x3;
    if (lhs_default) {
      xc.data = static_cast<char*>(x->data) + c0 * xrow;
      xc.shape[0] = cb;
    }
    mlxq_array oc = as3(out, cb);
    oc.shape[1] = M;
    oc.shape[2] = sp.N;
    oc.strides[2] = 1;
    oc.strides[1] = sp.N;
    oc.strides[0] = M * sp.N;
    oc.data = static_cast<char*>(out->data) + c0 * orow;
    const mlxq_array* lc = lhs_default ? nullptr : &li;
    GatherSpec gc = spec_gather(&xc, &w3, &s3, biases ? &b3 : nullptr, lc, &ri, sp.transpose, sp.gs, sp.bits,
                                mode_name(sp.mode), nullptr);
    choose_route(gc.q, &xc, &w3, &s3, biases ? &b3 : nullptr, "gather_qmm");
    gather_run(gc, &xc, &w3, &s3, biases ? &b3 : nullptr, lc, &ri, sorted_indices, &oc, stream);
  }
}

// One gather_qmm call on staged (row-contiguous, 16-byte aligned) operands.
void gather_run(GatherSpec& g, const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                const mlxq_array* biases, const mlxq_array* lhs_indices, const mlxq_array* rhs_indices,
                bool sorted_indices, mlxq_array* out, hipStream_t stream) {
  QmmSpec& sp = g.q;
  View xv{x}, wv{w}, sv{scales};
  const int64_t M = xv.dim(-2);
  int64_t B = 1;
  for (auto d : g.idx_shape) B *= d;
  if (B == 0 || M == 0 || sp.N == 0) return;
  if ((int)g.idx_shape.size() > MLXQ_MAX_DIMS) unsupported("gather_qmm: index rank too large");
  const int64_t X = xv.size() / std::max<int64_t>(M * sp.K, 1);
  const int64_t E = wv.size() / std::max<int64_t>(wv.dim(-2) * wv.dim(-1), 1);

  // flat uint32 lhs/rhs over the broadcast index shape, in the workspace tail
  mlxq::IdxPrepArgs ip{};
  ip.bnd = (int)g.idx_shape.size();
  for (int d = 0; d < ip.bnd; d++) ip.bshape[d] = g.idx_shape[d];
  ip.B = B;
  const mlxq_array* idx[2] = {lhs_indices, rhs_indices};
  const Shape dsh[2] = {default_index_shape(xv), default_index_shape(wv)};
  for (int s = 0; s < 2; s++) {
    ip.data[s] = idx[s] ? idx[s]->data : nullptr;
    ip.dtype[s] = idx[s] ? idx[s]->dtype : MLXQ_UINT32;
    bstrides_for(idx[s], dsh[s], g.idx_shape, ip.bstrides[s]);
  }
  ip.clamp[0] = std::max<int64_t>(X, 1);
  ip.clamp[1] = std::max<int64_t>(E, 1);
  if (B > kGatherChunk) {
    gather_chunked(g, x, w, scales, biases, lhs_indices, sorted_indices, out, stream, ip, B, X, E);
    return;
  }

  if (!sp.fast) {
    run_gen(sp, x, w, scales, biases, out, M, B, X, E, &ip, stream, ScratchSrc{});
    return;
  }
  const int fmt = fmt_of(sp.mode, sp.bits);
  const int cap = mlxq::qmv_max_rows(fmt, sp.gs);
  if (M > cap) {
    // more rows per gathered matrix than the decode kernels stage: the
    // general kernel tiles any row count
    run_gen(sp, x, w, scales, biases, out, M, B, X, E, &ip, stream, ScratchSrc{});
    return;
  }

  const int dev = current_device();
  const DevInfo di = device_info(dev);

  // Expert-sorted mxfp4 gathers with one row per entry and >= 4 rows per
  // expert on average (mlxcel's sorted MoE path, gpt_oss.rs:317-345): one
  // kernel streams each expert's weights once per 64 of its rows, finding
  // the rows by binary search in the sorted indices (qmm_group.hip); fewer
  // rows per expert run as segments of up to 4 entries (below).  Like the reference's sorted route, it
  // relies on sorted_indices being true.  MLXQ_GATHER_SORTED=0 turns it off.
  if (sorted_indices && M == 1 && fmt == mlxq::MXFP4 && B >= 32 && B >= 4 * E &&
      knobs().gather_sorted != 0) {
    const DirectIdx dl = direct_index(lhs_indices, dsh[0], g.idx_shape);
    const DirectIdx dr = direct_index(rhs_indices, dsh[1], g.idx_shape);
    mlxq::QmmGroupPlan gp =
        mlxq::qmm_group_plan(fmt, sp.N, sp.K, E, B, device_info(current_device()).cus, knobs().gather_tiles);
    if (knobs().gather_scale_table == 0) gp.scale_table = false;
    if (gp.ok && dr.ok && dr.p && dl.ok && !dl.p && dl.div == 1) {
      mlxq::QmmGroupArgs q{};
      q.x = static_cast<const uint16_t*>(x->data);
      q.w = static_cast<const uint32_t*>(w->data);
      q.scales = static_cast<const uint8_t*>(scales->data);
      q.out = static_cast<uint16_t*>(out->data);
      q.rhs = dr.p;
      q.rhs_stride = dr.stride;
      q.N = (int)sp.N;
      q.K = (int)sp.K;
      q.E = (int)E;
      q.B = (int)B;
      hip_check(mlxq::qmm_group_launch(q, gp, stream), "gather group launch");
      return;
    }
  }

  // Many rows per expert (MoE prefill, large batches): group rows by expert
  // on the device, then one GEMM tile reads each expert's weights once per
  // tile of rows (qmm.hip), instead of once per index entry.  Auto when the
  // entries average >= 8 rows per touched expert; MLXQ_GATHER_GROUP=0|1
  // forces the choice (A/B switch for tests).
  const int grp_env = knobs().gather_group;
  const int64_t rows = B * M;
  const bool want_group = grp_env == 1 || (grp_env != 0 && rows >= 8 * std::min<int64_t>(E, B));
  if (E <= mlxq::kGroupMaxExperts && want_group) {
    const int64_t per_expert = rows / std::max<int64_t>(1, std::min<int64_t>(E, B));
    const mlxq::QmmPlan qp =
        mlxq::qmm_plan_grouped(fmt, sp.gs, sp.N, sp.K, per_expert <= 64 ? 3 : (per_expert <= 128 ? 2 : 0));
    const bool use_qmm = qp.ok && X * M * sp.K * 2 < ((int64_t)1 << 31);
    // K not a multiple of 64: the MFMA skinny kernel over the same grouping,
    // in segments of fewer rows where the activation tile would not fit in
    // LDS (e.g. 64 rows of 4-bit g128 codes)
    int cap_rows = use_qmm ? qp.rows_per_tile : (int)std::min<int64_t>(cap, rows);
    auto segs = [&](int cr) { return rows / cr + std::min<int64_t>(E, B) + 1; };
    int nw = 0, pf = 0;
    if (!use_qmm) {
      qmv_shape_choice(sp.N, sp.K, nw, pf);
      while (cap_rows > 1 && mlxq::qmv_plan(fmt, sp.gs, sp.N, sp.K, cap_rows,
                                            (int)std::min<int64_t>(segs(cap_rows), 65535), di.cus, nw, pf)
                                     .lds > mlxq::kQmvLdsMax)
        cap_rows = (cap_rows + 1) / 2;
    }
    const int64_t maxseg = segs(cap_rows);
    if (maxseg > 65535) unsupported("gather_qmm: too many expert segments for one launch");
    mlxq::QmvPlan p;
    if (!use_qmm) {
      p = mlxq::qmv_plan(fmt, sp.gs, sp.N, sp.K, cap_rows, (int)maxseg, di.cus, nw, pf);
      if (p.lds > mlxq::kQmvLdsMax) unsupported("gather_qmm: activation tile does not fit in LDS");
    }
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const size_t o_x = al((size_t)B * 2 * sizeof(uint32_t));
    const size_t o_o = o_x + al((size_t)rows * sizeof(uint32_t));
    const size_t o_seg = o_o + al((size_t)rows * sizeof(uint32_t));
    const size_t o_n = o_seg + al((size_t)maxseg * 3 * sizeof(uint32_t));
    const size_t o_part = o_n + 256;
    const size_t part = (!use_qmm && p.ks > 1) ? (size_t)p.ks * rows * sp.N * sizeof(float) : 0;
    char* base = static_cast<char*>(workspace(dev, stream, o_part + part));
    uint32_t* flat = reinterpret_cast<uint32_t*>(base);
    ip.out[0] = flat;
    ip.out[1] = flat + B;
    hip_check(mlxq::launch_index_prep(ip, stream), "index_prep launch");
    mlxq::GroupArgs ga{};
    ga.lhs = flat;
    ga.rhs = flat + B;
    ga.B = (int)B;
    ga.M = (int)M;
    ga.E = (int)E;
    ga.cap = cap_rows;
    ga.xrows = reinterpret_cast<uint32_t*>(base + o_x);
    ga.orows = reinterpret_cast<uint32_t*>(base + o_o);
    ga.seg = reinterpret_cast<uint32_t*>(base + o_seg);
    ga.nseg = reinterpret_cast<uint32_t*>(base + o_n);
    hip_check(mlxq::launch_group_by_expert(ga, stream), "group launch");
    if (use_qmm) {
      mlxq::QmmArgs q{};
      q.x = static_cast<const uint16_t*>(x->data);
      q.w = static_cast<const uint32_t*>(w->data);
      q.scales = scales->data;
      q.biases = biases ? static_cast<const uint16_t*>(biases->data) : nullptr;
      q.out = static_cast<uint16_t*>(out->data);
      q.M = (int)rows;
      q.x_rows = (int)(X * M);
      q.N = (int)sp.N;
      q.K = (int)sp.K;
      int shift = 0;
      while ((1 << shift) < sp.gs) shift++;
      q.gs_shift = shift;
      q.ksplit = 1;
      q.ksteps_per_split = qp.ksteps_per_split;
      q.seg = ga.seg;
      q.nseg_dev = ga.nseg;
      q.xrows = ga.xrows;
      q.orows = ga.orows;
      q.w_expert_stride = wv.dim(-2) * wv.dim(-1);
      q.s_expert_stride = sv.dim(-2) * sv.dim(-1);
      mlxq::QmmPlan gp = qp;
      gp.tiles_m = (int)maxseg;
      hip_check(mlxq::qmm_launch(fmt, q, gp, stream), "gather qmm launch");
      return;
    }
    mlxq::QmvArgs a{};
    a.x = static_cast<const uint16_t*>(x->data);
    a.w = static_cast<const uint32_t*>(w->data);
    a.scales = scales->data;
    a.biases = biases ? static_cast<const uint16_t*>(biases->data) : nullptr;
    a.out = static_cast<uint16_t*>(out->data);
    a.N = (int)sp.N;
    a.K = (int)sp.K;
    a.E = (int)E;
    a.X = (int)X;
    a.w_expert_stride = wv.dim(-2) * wv.dim(-1);
    a.s_expert_stride = sv.dim(-2) * sv.dim(-1);
    a.rps = cap_rows;
    a.total_rows = (int)rows;
    a.out_rows = (int)rows;
    a.rows_lds = cap_rows;
    a.ks = p.ks;
    a.kst_per_wg = p.kst_per_wg;
    if (p.ks > 1) a.ws = reinterpret_cast<float*>(base + o_part);
    a.seg = ga.seg;
    a.nseg_dev = ga.nseg;
    a.xrows = ga.xrows;
    a.orows = ga.orows;
    hip_check(mlxq::qmv_launch(fmt, sp.gs, a, (int)maxseg, p, stream), "gather qmv launch");
    return;
  }

  // Sorted gathers with one row per entry (the expert-sorted MoE decode of
  // mlxcel's callers): on the block-MFMA kernel, one workgroup row per
  // expert finds the expert's entries by binary search and streams its
  // weights once per 4 of them (MLXQ_GATHER_RUNS=2, the default; it relies
  // on the order, as the reference's sorted route does).  Otherwise
  // (MLXQ_GATHER_RUNS=1, or the row-streaming kernel) runs of equal
  // consecutive experts, split at multiples of 4, correct for any order;
  // MLXQ_GATHER_RUNS=0: one segment per entry.
  const int r_req = knobs().qmv_r;
  {
    const DirectIdx dl = direct_index(lhs_indices, dsh[0], g.idx_shape);
    const DirectIdx dr = direct_index(rhs_indices, dsh[1], g.idx_shape);
    if (sorted_indices && M == 1 && B >= 8 && dr.ok && dr.p && dl.ok && !dl.p && dl.div == 1 &&
        knobs().gather_runs != 0) {
      // 4 entries at a time on the block-MFMA kernel (gpt-oss MoE shapes,
      // T=16: runs of 4 were 9% faster than one segment per entry, runs of
      // 8 or 16 slower; the row-streaming kernel with the expert search was
      // 13% slower than the block-MFMA one), else on the row-streaming kernel
      const mlxq::QmvB4Plan bp = mlxq::qmv_b4_plan(fmt, sp.gs, sp.N, sp.K, 4, 0, 0);
      const mlxq::QmvRsPlan rp = bp.ok ? mlxq::QmvRsPlan{} : mlxq::qmv_rs_plan(fmt, sp.gs, sp.N, sp.K, 4, r_req);
      if (bp.ok || rp.ok) {
        mlxq::QmvArgs a{};
        a.x = static_cast<const uint16_t*>(x->data);
        a.w = static_cast<const uint32_t*>(w->data);
        a.scales = scales->data;
        a.biases = biases ? static_cast<const uint16_t*>(biases->data) : nullptr;
        a.out = static_cast<uint16_t*>(out->data);
        a.rhs = dr.p;
        a.rhs_stride = dr.stride;
        a.lhs_stride = 1;
        a.lhs_div = 1;
        a.N = (int)sp.N;
        a.K = (int)sp.K;
        a.E = (int)E;
        a.X = (int)X;
        a.w_expert_stride = wv.dim(-2) * wv.dim(-1);
        a.s_expert_stride = sv.dim(-2) * sv.dim(-1);
        a.rps = 1;
        a.total_rows = (int)B;
        a.out_rows = (int)B;
        a.rows_lds = 1;
        a.runs = 4;
        if (bp.ok && knobs().gather_runs >= 2 && E <= B) {
          // one workgroup row per expert, its entries found by binary search
          // (with more experts than entries most rows would only search
          // and exit: runs then)
          a.runs = -1;
          hip_check(mlxq::qmv_b4_launch(fmt, sp.gs, a, (int)E, bp, stream), "gather qmv launch");
        } else if (bp.ok) {
          hip_check(mlxq::qmv_b4_launch(fmt, sp.gs, a, (int)B, bp, stream), "gather qmv launch");
        } else {
          hip_check(mlxq::qmv_rs_launch(fmt, sp.gs, a, (int)B, rp, stream), "gather qmv launch");
        }
        return;
      }
    }
  }

  const Skinny kind = skinny_choice((int)M, fmt, sp.K);
  const mlxq::QmvFrPlan fp =
      kind == Skinny::FR ? mlxq::qmv_fr_plan(fmt, sp.gs, sp.N, sp.K, (int)M, r_req) : mlxq::QmvFrPlan{};
  const mlxq::QmvB4Plan bp =
      kind == Skinny::B4 ? mlxq::qmv_b4_plan(fmt, sp.gs, sp.N, sp.K, (int)M, knobs().b4_rg,
                                             knobs().b4_cpw)
                         : mlxq::QmvB4Plan{};
  const mlxq::QmvRsPlan rp =
      (kind == Skinny::RS || (kind == Skinny::FR && !fp.ok) || (kind == Skinny::B4 && !bp.ok && M <= 4))
          ? mlxq::qmv_rs_plan(fmt, sp.gs, sp.N, sp.K, (int)M, r_req)
          : mlxq::QmvRsPlan{};
  const bool use_rs = fp.ok || rp.ok || bp.ok;
  int nw, pf;
  qmv_shape_choice(sp.N, sp.K, nw, pf);
  mlxq::QmvPlan p;
  if (!use_rs) {
    p = mlxq::qmv_plan(fmt, sp.gs, sp.N, sp.K, (int)M, (int)B, di.cus, nw, pf);
    if (p.lds > mlxq::kQmvLdsMax) {
      // more rows per entry than the skinny kernel's LDS holds at this
      // group size: the general kernel tiles any row count
      run_gen(sp, x, w, scales, biases, out, M, B, X, E, &ip, stream, ScratchSrc{});
      return;
    }
  }
  // indices the kernels can read in place skip the index_prep launch
  const DirectIdx dl = direct_index(lhs_indices, dsh[0], g.idx_shape);
  const DirectIdx dr = direct_index(rhs_indices, dsh[1], g.idx_shape);
  const bool direct = dl.ok && dr.ok && dr.div == 1 && knobs().gather_direct != 0;
  const size_t idx_bytes = direct ? 0 : ((size_t)B * 2 * sizeof(uint32_t) + 255) & ~(size_t)255;
  const size_t part_bytes = p.ks > 1 ? (size_t)p.ks * B * M * sp.N * sizeof(float) : 0;
  char* wsb = nullptr;
  if (idx_bytes + part_bytes > 0) wsb = static_cast<char*>(workspace(dev, stream, idx_bytes + part_bytes));
  const uint32_t* lhs_p = dl.p;
  const uint32_t* rhs_p = dr.p;
  int lhs_stride = dl.stride, rhs_stride = dr.stride, lhs_div = dl.div;
  if (!direct) {
    uint32_t* flat = reinterpret_cast<uint32_t*>(wsb);
    ip.out[0] = flat;
    ip.out[1] = flat + B;
    hip_check(mlxq::launch_index_prep(ip, stream), "index_prep launch");
    lhs_p = flat;
    rhs_p = flat + B;
    lhs_stride = rhs_stride = lhs_div = 1;
  }

  mlxq::QmvArgs a{};
  a.x = static_cast<const uint16_t*>(x->data);
  a.w = static_cast<const uint32_t*>(w->data);
  a.scales = scales->data;
  a.biases = biases ? static_cast<const uint16_t*>(biases->data) : nullptr;
  a.out = static_cast<uint16_t*>(out->data);
  a.lhs = lhs_p;
  a.rhs = rhs_p;
  a.lhs_stride = lhs_stride;
  a.rhs_stride = rhs_stride;
  a.lhs_div = lhs_div;
  a.N = (int)sp.N;
  a.K = (int)sp.K;
  a.E = (int)E;
  a.X = (int)X;
  a.w_expert_stride = wv.dim(-2) * wv.dim(-1);
  a.s_expert_stride = sv.dim(-2) * sv.dim(-1);
  a.rps = (int)M;
  a.total_rows = (int)(B * M);
  a.out_rows = (int)(B * M);
  a.rows_lds = (int)M;
  if (fp.ok) {
    hip_check(mlxq::qmv_fr_launch(fmt, sp.gs, a, (int)B, fp, stream), "gather qmv launch");
    return;
  }
  if (bp.ok) {
    hip_check(mlxq::qmv_b4_launch(fmt, sp.gs, a, (int)B, bp, stream), "gather qmv launch");
    return;
  }
  if (rp.ok) {
    hip_check(mlxq::qmv_rs_launch(fmt, sp.gs, a, (int)B, rp, stream), "gather qmv launch");
    return;
  }
  a.ks = p.ks;
  a.kst_per_wg = p.kst_per_wg;
  if (p.ks > 1) a.ws = reinterpret_cast<float*>(wsb + idx_bytes);
  hip_check(mlxq::qmv_launch(fmt, sp.gs, a, (int)B, p, stream), "gather qmv launch");
}

}  // namespace

// ===========================================================================
extern "C" {

const char* mlxq_last_error(void) { return g_last_error.c_str(); }

const char* mlxq_version(void) { return "mlxq 0.1.0 gfx950"; }

mlxq_status mlxq_quantized_matmul_shape(const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                                        const mlxq_array* biases, bool transpose, int32_t group_size,
                                        int32_t bits, const char* mode, int32_t* out_ndim, int64_t* out_shape,
                                        int32_t* out_dtype) {
  return guarded([&] {
    QmmSpec sp = spec_quantized_matmul(x, w, scales, biases, transpose, group_size, bits, mode);
    write_shape(sp.out_shape, sp.out_dtype, out_ndim, out_shape, out_dtype);
  });
}

mlxq_status mlxq_quantized_matmul(const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                                  const mlxq_array* biases, bool transpose, int32_t group_size, int32_t bits,
                                  const char* mode, mlxq_array* out, void* stream_) {
  return guarded([&] {
    const QmmSpec sp =
        check_quantized_matmul(x, w, scales, biases, transpose, group_size, bits, mode, out, "quantized_matmul");
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    Staged st = stage_operands(x, w, scales, biases, out, stream, true, "quantized_matmul");
    run_quantized_matmul(sp, st.in[0], st.in[1], st.in[2], st.in[3], st.out, stream);
    st.finish();
  });
}

mlxq_status mlxq_quantized_matmul_noalloc(const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                                          const mlxq_array* biases, bool transpose, int32_t group_size,
                                          int32_t bits, const char* mode, mlxq_array* out, void* stream_) {
  return guarded([&] {
    const QmmSpec sp = check_quantized_matmul(x, w, scales, biases, transpose, group_size, bits, mode, out,
                                              "quantized_matmul_noalloc");
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    // no staging buffer here: strided or misaligned operands are refused
    stage_operands(x, w, scales, biases, out, stream, false, "quantized_matmul_noalloc");
    ScratchSrc ss;
    hip_check(mlxq::static_scratch(current_device(), &ss.fixed), "hipGetSymbolAddress(scratch)");
    ss.max = mlxq::static_scratch_bytes();
    run_quantized_matmul(sp, x, w, scales, biases, out, stream, ss);
  });
}

void mlxq_reload_options(void) {
  // the previous snapshot stays allocated: a concurrent call may still read it
  g_knobs.store(read_knobs(), std::memory_order_release);
}

mlxq_status mlxq_workspace_reserve(size_t bytes, void* stream_) {
  return guarded([&] {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    const int dev = current_device();
    // the no-allocation entry point's scratch address, resolved here too so a
    // caller that reserves before a capture never resolves it under capture
    void* fixed = nullptr;
    hip_check(mlxq::static_scratch(dev, &fixed), "hipGetSymbolAddress(scratch)");
    std::lock_guard<std::mutex> lk(g_mu);
    // kernel scratch (slot 0) and the staging copies of strided operands (slot 1)
    for (int slot = 0; slot < 2; slot++) {
      Workspace& w = g_ws[{dev, stream, slot}];
      if (w.bytes >= bytes) continue;
      if (stream_capturing(stream)) unsupported("mlxq_workspace_reserve: the stream is being captured");
      grow_workspace(w, bytes);
    }
    // and the stream-K counters (slot 3), so a capture after the reserve can
    // take the stream-K prefill plan where the reserve covers its partials
    Workspace& c = g_ws[{dev, stream, 3}];
    if (!c.data && !stream_capturing(stream)) alloc_counters(c, stream);
  });
}

size_t mlxq_get_cache_memory(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  size_t total = 0;
  for (auto& kv : g_ws) total += kv.second.bytes + kv.second.retired_bytes;
  return total;
}

mlxq_status mlxq_clear_cache(void) {
  return guarded([&] {
    std::lock_guard<std::mutex> lk(g_mu);
    int cur = 0;
    hip_check(hipGetDevice(&cur), "hipGetDevice");
    std::map<int, bool> synced;
    for (auto& kv : g_ws) {
      const int dev = std::get<0>(kv.first);
      if (!synced[dev]) {
        hip_check(hipSetDevice(dev), "hipSetDevice");
        hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
        synced[dev] = true;
      }
      hip_check(hipSetDevice(dev), "hipSetDevice");
      for (void* p : kv.second.retired) hip_check(hipFree(p), "hipFree");
      if (kv.second.data) hip_check(hipFree(kv.second.data), "hipFree");
    }
    g_ws.clear();
    hip_check(hipSetDevice(cur), "hipSetDevice");
  });
}

mlxq_status mlxq_quantized_linear(const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                                  const mlxq_array* biases, const mlxq_array* linear_bias, int32_t group_size,
                                  int32_t bits, const char* mode, mlxq_array* out, void* stream_) {
  return guarded([&] {
    const char* tag = "quantized_linear";
    const QmmSpec sp = check_quantized_matmul(x, w, scales, biases, true, group_size, bits, mode, out, tag);
    int64_t bias_n = 0;
    if (linear_bias) {
      check_array(linear_bias, "linear_bias");
      View lb{linear_bias}, ov{out};
      // MLX's add broadcasts the bias against the (..., N) product; the two
      // layouts a linear layer uses are covered: (N) / (1, ..., N), and the
      // product's own shape
      Shape osh = ov.shape();
      Shape lsh = lb.shape();
      while (!lsh.empty() && lsh.front() == 1 && (int)lsh.size() > 1) lsh.erase(lsh.begin());
      if (lsh == Shape{sp.N}) bias_n = sp.N;
      else if (lb.shape() == osh) bias_n = ov.size();
      else
        unsupported(std::string(tag) + ": linear_bias must have shape (N) or the output's shape (got " +
                    fmt_shape(lb.shape()) + ")");
      if (linear_bias->dtype != out->dtype)
        unsupported(std::string(tag) + ": linear_bias must have the output's dtype (" + dtype_name(out->dtype) +
                    "; the reference's add would promote)");
      require_contiguous(linear_bias, "linear_bias");
    }
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    Staged st = stage_operands(x, w, scales, biases, out, stream, true, tag);
    run_quantized_matmul(sp, st.in[0], st.in[1], st.in[2], st.in[3], st.out, stream);
    if (bias_n > 0 && View{out}.size() > 0)
      hip_check(mlxq::launch_bias_add(st.out->data, linear_bias->data, View{out}.size(), bias_n,
                                      gen_type(out->dtype), stream),
                "bias add launch");
    st.finish();
  });
}

int32_t mlxq_quantized_matmul_matches_dense_gemm(const mlxq_array* x, const mlxq_array* w,
                                                 const mlxq_array* scales, const mlxq_array* biases,
                                                 int32_t group_size, int32_t bits) {
  (void)x;
  (void)w;
  (void)scales;
  (void)biases;
  (void)group_size;
  (void)bits;
  // Every route here dequantizes inside the matmul kernel (no dequantize +
  // dense GEMM route), so no call returns the bytes of dequantize + matmul.
  return 0;
}

mlxq_status mlxq_quantized_matmul_multi(const mlxq_array* x, int32_t n, const mlxq_array* const* w,
                                        const mlxq_array* const* scales, const mlxq_array* const* biases,
                                        int32_t group_size, int32_t bits, const char* mode, mlxq_array* const* out,
                                        void* stream_) {
  return guarded([&] {
    const char* tag = "quantized_matmul_multi";
    if (n < 1 || n > mlxq::kQmvMultiMax) {
      std::ostringstream os;
      os << "[" << tag << "] n must be between 1 and " << mlxq::kQmvMultiMax << " but is " << n << ".";
      invalid(os);
    }
    if (!w || !scales || !out) fail(MLXQ_EINVAL, std::string("[") + tag + "] w, scales and out must not be NULL");
    std::vector<QmmSpec> sp;
    for (int i = 0; i < n; i++) {
      const mlxq_array* b = biases ? biases[i] : nullptr;
      sp.push_back(check_quantized_matmul(x, w[i], scales[i], b, true, group_size, bits, mode, out[i], tag));
      if (View{w[i]}.ndim() != 2) unsupported(std::string(tag) + ": 2-D weights only");
    }
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    // One launch of the row-streaming kernel over every projection when each
    // call alone would run it with the same plan (decode rows, no kernel
    // override): the results are then those of the separate calls, bit for
    // bit.  Otherwise the calls run one after another.
    const int fmt = fmt_of(sp[0].mode, sp[0].bits);
    const int64_t rows = View{out[0]}.size() / std::max<int64_t>(sp[0].N, 1);
    bool plain = true;  // every projection on the specialised kernels, no operand to stage
    for (int i = 0; i < n; i++)
      plain = plain && sp[i].fast && !needs_staging(x) && !needs_staging(w[i]) && !needs_staging(scales[i]) &&
              !needs_staging(biases ? biases[i] : nullptr) && !needs_staging(out[i]);
    bool fused = plain && n > 1 && sp[0].K > 0 && rows >= 1 && rows < knobs().qmm_min_rows &&
                 rows <= mlxq::qmv_max_rows(fmt, sp[0].gs) && !use_mid((int)rows, fmt, sp[0].K) &&
                 skinny_choice((int)rows, fmt, sp[0].K) == Skinny::RS && knobs().qmv_multi != 0;
    mlxq::QmvRsPlan plan{};
    mlxq::QmvMulti mp{};
    mp.n = n;
    for (int i = 0; i < n && fused; i++) {
      // a projection that alone would take a mid-size kernel is not fused here
      if (sp[i].N == 0 || dense_route(sp[i], rows, device_info(current_device()).cus, false).kind != DR_OTHER)
        fused = false;
      const mlxq::QmvRsPlan p =
          mlxq::qmv_rs_plan(fmt, sp[i].gs, sp[i].N, sp[i].K, (int)rows, knobs().qmv_r);
      if (!p.ok || (i > 0 && (p.mr != plan.mr || p.r != plan.r || p.cpw != plan.cpw || p.nw != plan.nw ||
                              p.lds != plan.lds)))
        fused = false;
      if (i == 0) plan = p;
      mp.tile_end[i] = (i ? mp.tile_end[i - 1] : 0) + p.tiles;
      mp.N[i] = (int)sp[i].N;
      mp.w[i] = static_cast<const uint32_t*>(w[i]->data);
      mp.scales[i] = scales[i]->data;
      mp.biases[i] = biases && biases[i] ? static_cast<const uint16_t*>(biases[i]->data) : nullptr;
      mp.out[i] = static_cast<uint16_t*>(out[i]->data);
    }
    if (!fused) {
      // 3-16 rows on the mid-size kernels: one launch when every projection
      // alone takes the same kernel with the same plan (only the row blocks
      // differ), so each output is the separate call's, bit for bit
      if (plain && n > 1 && knobs().qmv_multi != 0 && sp[0].K > 0 && rows >= 1 &&
          try_multi_mid(sp, n, x, w, scales, biases, out, rows, stream))
        return;
      for (int i = 0; i < n; i++) {
        Staged st = stage_operands(x, w[i], scales[i], biases ? biases[i] : nullptr, out[i], stream, true, tag);
        run_quantized_matmul(sp[i], st.in[0], st.in[1], st.in[2], st.in[3], st.out, stream);
        st.finish();
      }
      return;
    }
    mlxq::QmvArgs a{};
    a.x = static_cast<const uint16_t*>(x->data);
    a.w = mp.w[0];
    a.scales = mp.scales[0];
    a.biases = mp.biases[0];
    a.out = mp.out[0];
    a.N = mp.N[0];
    a.K = (int)sp[0].K;
    a.out_rows = (int)rows;
    a.E = 1;
    a.X = 1;
    a.rps = (int)rows;
    a.total_rows = (int)rows;
    hip_check(mlxq::qmv_rs_launch(fmt, sp[0].gs, a, 1, plan, stream, &mp), "qmv launch");
  });
}

mlxq_status mlxq_gather_qmm_shape(const mlxq_array* x, const mlxq_array* w, const mlxq_array* scales,
                                  const mlxq_array* biases, const mlxq_array* lhs_indices,
                                  const mlxq_array* rhs_indices, bool transpose, int32_t group_size, int32_t bits,
                                  const char* mode, int32_t* out_ndim, int64_t* out_shape, int32_t* out_dtype) {
  if (!lhs_indices && !rhs_indices)
    return mlxq_quantized_matmul_shape(x, w, scales, biases, transpose, group_size, bits, mode, out_ndim,
                                       out_shape, out_dtype);
  return guarded([&] {
    GatherSpec g = spec_gather(x, w, scales, biases, lhs_indices, rhs_indices, transpose, group_size, bits, mode,
                               nullptr);
    write_shape(g.q.out_shape, g.q.out_dtype, out_ndim, out_shape, out_dtype);
  });
}

mlxq_status mlxq_gather_qmm(const mlxq_array* x_, const mlxq_array* w_, const mlxq_array* scales_,
                            const mlxq_array* biases_, const mlxq_array* lhs_indices, const mlxq_array* rhs_indices,
                            bool transpose, int32_t group_size, int32_t bits, bool sorted_indices, const char* mode,
                            const mlxq_array* global_scale, mlxq_array* out_, void* stream_) {
  // sorted_indices selects the routes that rely on rhs being non-decreasing
  // (after the uint32 cast); with a false promise their rows are unspecified
  if (!lhs_indices && !rhs_indices) {
    if (global_scale) {
      g_last_error = "[gather_qmm] Global scale is not supported without indices.";
      return MLXQ_EINVAL;
    }
    return mlxq_quantized_matmul(x_, w_, scales_, biases_, transpose, group_size, bits, mode, out_, stream_);
  }
  return guarded([&] {
    const char* tag = "gather_qmm";
    GatherSpec g = spec_gather(x_, w_, scales_, biases_, lhs_indices, rhs_indices, transpose, group_size, bits,
                               mode, global_scale);
    QmmSpec& sp = g.q;
    check_out(out_, sp.out_shape, sp.out_dtype, tag);
    choose_route(sp, x_, w_, scales_, biases_, tag);
    if (global_scale) unsupported("gather_qmm: global_scale (nvfp4) is not implemented");
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    Staged st = stage_operands(x_, w_, scales_, biases_, out_, stream, true, tag);
    const mlxq_array* x = st.in[0];
    const mlxq_array* w = st.in[1];
    const mlxq_array* scales = st.in[2];
    const mlxq_array* biases = st.in[3];
    mlxq_array* out = st.out;
    gather_run(g, x, w, scales, biases, lhs_indices, rhs_indices, sorted_indices, out, stream);
    st.finish();
  });
}

mlxq_status mlxq_dequantize(const mlxq_array* w, const mlxq_array* scales, const mlxq_array* biases,
                            int32_t group_size, int32_t bits, const char* mode_str, int32_t dtype,
                            mlxq_array* out, void* stream_) {
  return guarded([&] {
    check_array(w, "w");
    check_array(scales, "scales");
    if (biases) check_array(biases, "biases");
    const char* tag = "dequantize";
    Mode mode = parse_mode(mode_str, tag);
    const int out_type = validate_mode_with_type(tag, scales, biases, dtype, mode, mode_str);
    params_from_mode(mode, group_size, bits);
    if (bits <= 0) {
      std::ostringstream os;
      os << "[dequantize] Invalid value for bits: " << bits;
      invalid(os);
    }
    if (group_size <= 0) {
      std::ostringstream os;
      os << "[dequantize] Invalid value for group_size: " << group_size;
      invalid(os);
    }
    View wv{w}, sv{scales};
    if (w->dtype != MLXQ_UINT32) fail(MLXQ_EINVAL, "[dequantize] The matrix should be given as a uint32");
    if (wv.ndim() < 2) {
      std::ostringstream os;
      os << "[dequantize] The matrix to be dequantized must have at least 2 dimension but it has only " << wv.ndim()
         << ".";
      invalid(os);
    }
    if (mode == AFFINE) {
      View bv{biases};
      if (wv.ndim() != sv.ndim() || wv.ndim() != bv.ndim())
        fail(MLXQ_EINVAL, "[dequantize] Shape of scales and biases does not match the matrix");
      Shape a = wv.shape(), b = sv.shape(), c = bv.shape();
      a.back() = b.back() = c.back() = -1;
      if (a != b || a != c) fail(MLXQ_EINVAL, "[dequantize] Shape of scales and biases does not match the matrix");
      // Stricter than ops.cpp:5512-5515, which lets the biases' last dim differ
      // from the scales' and then reads past the biases: rejected here.
      if (bv.shape() != sv.shape())
        fail(MLXQ_EINVAL, "[dequantize] Shape of scales and biases does not match the matrix");
      if (wv.dim(-1) * 32 / bits != sv.dim(-1) * group_size) {
        std::ostringstream os;
        os << "[dequantize] Shape of scales and biases does not match the matrix given the quantization parameters. "
           << "Provided matrix of shape " << fmt_shape(wv.shape()) << " and scales/biases of shape "
           << fmt_shape(sv.shape()) << " with group_size=" << group_size << " and bits=" << bits << ".";
        invalid(os);
      }
    } else {
      const int egs = mode == NVFP4_M ? 16 : 32, ebits = mode == MXFP8_M ? 8 : 4;
      const char* mname = mode == NVFP4_M ? "nvfp4" : (mode == MXFP8_M ? "mxfp8" : "mxfp4");
      if (group_size != egs) {
        std::ostringstream os;
        os << "[dequantize] " << mname << " quantization requires group size " << egs << " but got " << group_size
           << ".";
        invalid(os);
      }
      if (bits != ebits) {
        std::ostringstream os;
        os << "[dequantize] " << mname << " quantization requires bits to be " << ebits << " but got " << bits << ".";
        invalid(os);
      }
      if (wv.ndim() != sv.ndim()) fail(MLXQ_EINVAL, "[dequantize] Shape of scales does not match the matrix");
      Shape a = wv.shape(), b = sv.shape();
      a.back() = b.back() = -1;
      if (a != b) fail(MLXQ_EINVAL, "[dequantize] Shape of scales does not match the matrix");
      if (wv.dim(-1) * 32 / bits != sv.dim(-1) * group_size) {
        std::ostringstream os;
        os << "[dequantize] Shape of scales does not match the matrix given the quantization parameters. "
           << "Provided matrix of shape " << fmt_shape(wv.shape()) << " and scales of shape " << fmt_shape(sv.shape())
           << ".";
        invalid(os);
      }
    }
    Shape oshape = wv.shape();
    oshape.back() = wv.dim(-1) * 32 / bits;
    check_out(out, oshape, out_type, tag);
    // bfloat16 results of bfloat16 affine 2/4/6/8-bit and of the fp modes run
    // the dedicated kernels; the general one takes float16/float32 scales or
    // results, affine 3/5-bit codes and mxfp4 to float16/float32
    const bool bf16_all = out_type == MLXQ_BFLOAT16 &&
                          (mode != AFFINE || (scales->dtype == MLXQ_BFLOAT16 && biases->dtype == MLXQ_BFLOAT16));
    const bool dedicated = bf16_all && (mode != AFFINE || bits == 2 || bits == 4 || bits == 6 || bits == 8);
    if (!dedicated) {
      if (mode == AFFINE && (bits < 1 || bits > 8 || bits == 7))
        unsupported("dequantize: affine bits " + std::to_string(bits) + " is not implemented");
      if (mode == MXFP8_M || mode == NVFP4_M) unsupported("dequantize: only bfloat16 output is implemented for this mode");
      if (gen_type(out_type) < 0) unsupported("dequantize: output dtype " + std::string(dtype_name(out_type)) +
                                              " is not implemented");
      if (mode == AFFINE && (gen_type(scales->dtype) < 0 || biases->dtype != scales->dtype))
        unsupported("dequantize: scales and biases of one float type (bfloat16, float16 or float32) are implemented");
      if (mode == AFFINE && group_size != 32 && group_size != 64 && group_size != 128)
        unsupported("dequantize: group_size must be 32, 64 or 128");
    }
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    Staged st = stage_operands(nullptr, w, scales, biases, out, stream, true, tag);
    w = st.in[1];
    scales = st.in[2];
    biases = st.in[3];
    out = st.out;
    const int64_t K = oshape.back();
    const int64_t rows = View{out}.size() / std::max<int64_t>(K, 1);
    if (rows == 0 || K == 0) return;
    if (K % group_size) unsupported("dequantize: K must be a multiple of group_size");
    // 64-bit element indices; one launch grid covers at most 2^32 threads of >= 8 elements
    if (rows * K >= kElemMax) unsupported("dequantize: 2^34 elements or more");
    if (!dedicated) {
      hip_check(mlxq::launch_gen_dequantize(mode == MXFP4_M ? mlxq::GEN_MXFP4 : mlxq::GEN_AFFINE,
                                            static_cast<const uint32_t*>(w->data), scales->data,
                                            biases ? biases->data : nullptr, out->data, rows, K, group_size, bits,
                                            mode == AFFINE ? gen_type(scales->dtype) : 0, gen_type(out_type), stream),
                "dequantize launch");
      st.finish();
      return;
    }
    if (mode == AFFINE) {
      hip_check(mlxq::launch_affine_dequantize(static_cast<const uint32_t*>(w->data),
                                               static_cast<const uint16_t*>(scales->data),
                                               static_cast<const uint16_t*>(biases->data),
                                               static_cast<uint16_t*>(out->data), rows, K, group_size, bits, stream),
                "dequantize launch");
    } else if (mode == MXFP4_M) {
      hip_check(mlxq::launch_mxfp4_dequantize(static_cast<const uint32_t*>(w->data),
                                              static_cast<const uint8_t*>(scales->data),
                                              static_cast<uint16_t*>(out->data), rows, K, stream),
                "dequantize launch");
    } else {
      hip_check(mlxq::launch_fp_dequantize(mode == MXFP8_M ? mlxq::FP_MXFP8 : mlxq::FP_NVFP4,
                                           static_cast<const uint32_t*>(w->data),
                                           static_cast<const uint8_t*>(scales->data),
                                           static_cast<uint16_t*>(out->data), rows, K, stream),
                "dequantize launch");
    }
    st.finish();
  });
}

mlxq_status mlxq_quantize(const mlxq_array* w, int32_t group_size, int32_t bits, const char* mode_str,
                          mlxq_array* wq_out, mlxq_array* scales_out, mlxq_array* biases_out, void* stream_) {
  return guarded([&] {
    check_array(w, "w");
    const char* tag = "quantize";
    Mode mode = parse_mode(mode_str, tag);
    params_from_mode(mode, group_size, bits);
    View wv{w};
    if (!is_floating(w->dtype)) {
      std::ostringstream os;
      os << "[quantize] Only real floating types can be quantized but w has type " << dtype_name(w->dtype) << ".";
      invalid(os);
    }
    if (wv.ndim() < 2) {
      std::ostringstream os;
      os << "[quantize] The matrix to be quantized must have at least 2 dimension but it has only " << wv.ndim()
         << ".";
      invalid(os);
    }
    if (wv.dim(-1) % group_size != 0) {
      std::ostringstream os;
      os << "[quantize] The last dimension of the matrix needs to be divisible by the quantization group size "
         << group_size << ". However the provided  matrix has shape " << fmt_shape(wv.shape());
      invalid(os);
    }
    if (mode == AFFINE) {
      if (group_size != 32 && group_size != 64 && group_size != 128) {
        std::ostringstream os;
        os << "[quantize] The requested group size " << group_size
           << " is not supported. The supported group sizes are 32, 64, and 128.";
        invalid(os);
      }
      if (bits < 1 || bits > 8 || bits == 7) {
        std::ostringstream os;
        os << "[quantize] The requested number of bits " << bits
           << " is not supported. The supported bits are 1, 2, 3, 4, 5, 6 and 8.";
        invalid(os);
      }
    } else {
      const int egs = mode == NVFP4_M ? 16 : 32, ebits = mode == MXFP8_M ? 8 : 4;
      const char* mname = mode == NVFP4_M ? "nvfp4" : (mode == MXFP8_M ? "mxfp8" : "mxfp4");
      if (group_size != egs) {
        std::ostringstream os;
        os << "[quantize] " << mname << " quantization requires group size " << egs << " but got " << group_size
           << ".";
        invalid(os);
      }
      if (bits != ebits) {
        std::ostringstream os;
        os << "[quantize] " << mname << " quantization requires bits to be " << ebits << " but got " << bits << ".";
        invalid(os);
      }
    }
    Shape qs = wv.shape(), ss = wv.shape();
    qs.back() = wv.dim(-1) * bits / 32;
    ss.back() = wv.dim(-1) / group_size;
    check_out(wq_out, qs, MLXQ_UINT32, tag);
    check_out(scales_out, ss, mode == AFFINE ? w->dtype : (int)MLXQ_UINT8, tag);
    if (mode == AFFINE) check_out(biases_out, ss, w->dtype, tag);
    if (mode == AFFINE && gen_type(w->dtype) < 0)
      unsupported(std::string("quantize: ") + dtype_name(w->dtype) +
                  " weights are not implemented (bfloat16, float16 and float32 are)");
    if (mode != AFFINE && w->dtype != MLXQ_BFLOAT16)
      unsupported("quantize: only bfloat16 weights are implemented for this mode");
    require_contiguous(w, "w");
    const int64_t K = wv.dim(-1);
    const int64_t rows = wv.size() / std::max<int64_t>(K, 1);
    if (rows == 0 || K == 0) return;
    if (rows * K >= kElemMax) unsupported("quantize: 2^34 elements or more");
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
    if (mode == AFFINE) {
      hip_check(mlxq::launch_affine_quantize(w->data, gen_type(w->dtype), static_cast<uint32_t*>(wq_out->data),
                                             scales_out->data, biases_out->data, rows, K, group_size, bits,
                                             stream),
                "quantize launch");
    } else if (mode == MXFP4_M) {
      hip_check(mlxq::launch_mxfp4_quantize(static_cast<const uint16_t*>(w->data),
                                            static_cast<uint32_t*>(wq_out->data),
                                            static_cast<uint8_t*>(scales_out->data), rows, K, stream),
                "quantize launch");
    } else {
      hip_check(mlxq::launch_fp_quantize(mode == MXFP8_M ? mlxq::FP_MXFP8 : mlxq::FP_NVFP4,
                                         static_cast<const uint16_t*>(w->data), static_cast<uint32_t*>(wq_out->data),
                                         static_cast<uint8_t*>(scales_out->data), rows, K, stream),
                "quantize launch");
    }
  });
}

}  // extern "C"

// ---- fused single-token decode MoE -------------------------------------------
//
// fused_moe_expert_kernel / fused_moe_geglu_kernel (mlx_cxx_bridge.h:2061-2084,
// lib.rs:2336-2380; host side mlx_cxx_kernels.cpp:3817-4112).  The reference
// casts its inputs to the activation dtype and reads them unchecked; here the
// shapes are checked (EINVAL) and configurations the kernels do not cover are
// refused (EUNSUPPORTED), which the caller answers with its gather_qmm
// fallback, as it answers the reference's "no kernel port" refusal.

namespace {

void fused_moe(const char* tag, const mlxq_array* x, const mlxq_array* indices, const mlxq_array* gate_w,
               const mlxq_array* gate_s, const mlxq_array* gate_b, const mlxq_array* up_w, const mlxq_array* up_s,
               const mlxq_array* up_b, const mlxq_array* down_w, const mlxq_array* down_s, const mlxq_array* down_b,
               const mlxq_array* scores, int32_t din, int32_t dff, int32_t k, int32_t gu_bits, int32_t d_bits,
               int32_t group_size, int act, mlxq_array* out, void* stream_) {
  const mlxq_array* all[] = {x, indices, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s, down_b, scores, out};
  const char* names[] = {"x",      "indices", "gate_w", "gate_s", "gate_b", "up_w", "up_s",
                         "up_b",   "down_w",  "down_s", "down_b", "scores", "out"};
  for (int i = 0; i < 13; i++) check_array(all[i], names[i]);
  auto bad = [&](const std::string& what) {
    std::ostringstream os;
    os << "[" << tag << "] " << what;
    invalid(os);
  };
  if (din <= 0 || dff <= 0 || k <= 0) bad("din, dff and k must be positive");
  if (k > 65535) unsupported(std::string(tag) + ": at most 65535 experts per token");
  if (gu_bits != 4 && gu_bits != 8)
    unsupported(std::string(tag) + ": gate/up bits must be 4 or 8 (got " + std::to_string(gu_bits) + ")");
  if (d_bits != 4 && d_bits != 6 && d_bits != 8)
    unsupported(std::string(tag) + ": down bits must be 4, 6 or 8 (got " + std::to_string(d_bits) + ")");
  if (group_size != 32 && group_size != 64 && group_size != 128)
    unsupported(std::string(tag) + ": group_size must be 32, 64 or 128 (got " + std::to_string(group_size) + ")");
  // (with group_size >= 32 this also gives whole uint32 columns at 6 bits)
  if (din % group_size || dff % group_size) bad("din and dff must be multiples of group_size");

  View xv{x}, iv{indices}, sv{scores}, ov{out};
  if (xv.size() != din) bad("x must have din elements");
  if (iv.size() != k) bad("indices must have k elements");
  if (sv.size() != k) bad("scores must have k elements");
  if (ov.ndim() != 1 || ov.dim(0) != din) bad("out must have shape (din)");
  if (!is_integral(indices->dtype) || (dtype_size(indices->dtype) != 4 && dtype_size(indices->dtype) != 8))
    unsupported(std::string(tag) + ": indices must be 32- or 64-bit integers");
  if (x->dtype != MLXQ_BFLOAT16 || out->dtype != MLXQ_BFLOAT16)
    unsupported(std::string(tag) + ": only bfloat16 activations are implemented");
  if (scores->dtype != MLXQ_FLOAT32 && scores->dtype != MLXQ_BFLOAT16 && scores->dtype != MLXQ_FLOAT16)
    unsupported(std::string(tag) + ": scores must be float32, bfloat16 or float16");

  View gw{gate_w};
  if (gw.ndim() != 3) bad("gate_w must have shape (E, dff, din * bits / 32)");
  const int64_t E = gw.dim(0);
  if (E <= 0) bad("the expert count must be positive");
  auto want = [&](const mlxq_array* a, const char* name, Shape shape, int dtype) {
    if (View{a}.shape() != shape) bad(std::string(name) + " must have shape " + fmt_shape(shape));
    if (a->dtype != dtype) bad(std::string(name) + " must be " + dtype_name(dtype));
    require_contiguous(a, name);
  };
  want(gate_w, "gate_w", {E, dff, (int64_t)din * gu_bits / 32}, MLXQ_UINT32);
  want(up_w, "up_w", {E, dff, (int64_t)din * gu_bits / 32}, MLXQ_UINT32);
  want(down_w, "down_w", {E, din, (int64_t)dff * d_bits / 32}, MLXQ_UINT32);
  for (auto p : {std::make_pair(gate_s, "gate_s"), std::make_pair(gate_b, "gate_b"), std::make_pair(up_s, "up_s"),
                 std::make_pair(up_b, "up_b")})
    want(p.first, p.second, {E, dff, din / group_size}, MLXQ_BFLOAT16);
  for (auto p : {std::make_pair(down_s, "down_s"), std::make_pair(down_b, "down_b")})
    want(p.first, p.second, {E, din, dff / group_size}, MLXQ_BFLOAT16);
  require_contiguous(x, "x");
  require_contiguous(indices, "indices");
  require_contiguous(scores, "scores");
  require_contiguous(out, "out");
  // 32-bit buffer offsets: one expert's gate matrix, its scales and the
  // activation staging stay below 2 GiB
  if ((int64_t)dff * din * gu_bits / 8 >= ((int64_t)1 << 31) || (int64_t)k * dff * 4 >= ((int64_t)1 << 31) ||
      (int64_t)dff * (din / group_size) * 2 >= ((int64_t)1 << 31) || (int64_t)din * 2 >= ((int64_t)1 << 31))
    unsupported(std::string(tag) + ": operands above 2 GiB per expert");

  const int dev = current_device();
  hipStream_t stream = reinterpret_cast<hipStream_t>(stream_);
  mlxq::MoeArgs a{};
  a.x = static_cast<const uint16_t*>(x->data);
  a.idx = static_cast<const uint32_t*>(indices->data);
  a.idx_stride = dtype_size(indices->dtype) / 4;
  a.scores = scores->data;
  a.score_dt = scores->dtype == MLXQ_FLOAT32 ? 0 : (scores->dtype == MLXQ_BFLOAT16 ? 1 : 2);
  a.gate_w = static_cast<const uint32_t*>(gate_w->data);
  a.gate_s = static_cast<const uint16_t*>(gate_s->data);
  a.gate_b = static_cast<const uint16_t*>(gate_b->data);
  a.up_w = static_cast<const uint32_t*>(up_w->data);
  a.up_s = static_cast<const uint16_t*>(up_s->data);
  a.up_b = static_cast<const uint16_t*>(up_b->data);
  a.down_w = static_cast<const uint32_t*>(down_w->data);
  a.down_s = static_cast<const uint16_t*>(down_s->data);
  a.down_b = static_cast<const uint16_t*>(down_b->data);
  a.out = static_cast<uint16_t*>(out->data);
  a.din = din;
  a.dff = dff;
  a.k = k;
  a.E = (int)std::min<int64_t>(E, INT32_MAX);
  a.gs_shift = group_size == 32 ? 5 : (group_size == 64 ? 6 : 7);
  a.act = reinterpret_cast<float*>(workspace(dev, stream, (size_t)k * dff * sizeof(float)));
  hip_check(mlxq::moe_launch(a, gu_bits, d_bits, act, stream), "fused MoE launch");
}

}  // namespace

extern "C" {

mlxq_status mlxq_fused_moe_expert(const mlxq_array* x, const mlxq_array* indices, const mlxq_array* gate_w,
                                  const mlxq_array* gate_s, const mlxq_array* gate_b, const mlxq_array* up_w,
                                  const mlxq_array* up_s, const mlxq_array* up_b, const mlxq_array* down_w,
                                  const mlxq_array* down_s, const mlxq_array* down_b, const mlxq_array* scores,
                                  int32_t din, int32_t dff, int32_t k, int32_t gu_bits, int32_t d_bits,
                                  int32_t group_size, mlxq_array* out, void* stream) {
  return guarded([&] {
    fused_moe("fused_moe_expert_kernel", x, indices, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s,
              down_b, scores, din, dff, k, gu_bits, d_bits, group_size, mlxq::MOE_SWIGLU, out, stream);
  });
}

mlxq_status mlxq_fused_moe_geglu(const mlxq_array* x, const mlxq_array* indices, const mlxq_array* gate_w,
                                 const mlxq_array* gate_s, const mlxq_array* gate_b, const mlxq_array* up_w,
                                 const mlxq_array* up_s, const mlxq_array* up_b, const mlxq_array* down_w,
                                 const mlxq_array* down_s, const mlxq_array* down_b, const mlxq_array* scores,
                                 int32_t din, int32_t dff, int32_t k, int32_t gu_bits, int32_t d_bits,
                                 int32_t group_size, mlxq_array* out, void* stream) {
  return guarded([&] {
    fused_moe("fused_moe_geglu_kernel", x, indices, gate_w, gate_s, gate_b, up_w, up_s, up_b, down_w, down_s,
              down_b, scores, din, dff, k, gu_bits, d_bits, group_size, mlxq::MOE_GEGLU, out, stream);
  });
}

}  // extern "C"
